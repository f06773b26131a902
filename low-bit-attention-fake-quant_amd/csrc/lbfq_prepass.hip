// Memory-bound prepass kernels for the fake-quant attention path (gfx950).
//
// One generic row-tile kernel covers every per-token transform of the
// reference's preprocess + quant stage:
//   gather (k-means order)  ->  subtract a mean (K mean / Q group mean / V
//   block mean)  ->  round to the work dtype  ->  optional random-sign FWHT
//   ->  quantise (FP8 block / channel / MX-QK / MX-V, or amax-only)
// and writes the smoothed work tensor, the FP8 codes (NHD, head-major BHSD,
// or transposed BHDS for the attention kernel's V operand) and the scales.
// Column means use a fixed sequential fp64 order (colsum / finalize kernels)
// so the CPU oracle reproduces them bit for bit.
//
// Reference semantics: quant_triton.py:26-416, preprocess.py:10-193,
// hadamard.py:25-117, kmeans.py:84-89 / 127-135.
#include <stdarg.h>

#include "lbfq_common.h"
#include "../../include/lbfq.h"

using namespace lbfq;

static thread_local char g_err[512];

extern "C" const char* lbfq_last_error(void) { return g_err; }

void lbfq_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

namespace {

constexpr int kThreads = 256;

struct RowTileArgs {
  const void* x;
  int x_dtype;
  int64_t B, S, H, D;
  int R;
  const int32_t* gather;
  int sub_mode;
  const float* sub;
  int sub_block;
  void* smoothed;
  int hadamard;
  const int8_t* signs;
  float had_scale;
  int quant_mode;
  uint8_t* codes;
  int codes_layout;
  int64_t codes_spitch;
  float* scale;
  int64_t sc_b, sc_s, sc_h, sc_d;
  uint32_t* amax_table;
  int mx_block;
  int smoothed_stage;
  int scale_e8m0;
};

__device__ __forceinline__ void load8(const void* x, int dt, int64_t idx, float v[8]) {
  if (dt == kF32) {
    const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(x) + idx);
    float4 a = p[0], b = p[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    uint4 r = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(x) + idx);
    uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint16_t lo = static_cast<uint16_t>(w[i] & 0xffffu), hi = static_cast<uint16_t>(w[i] >> 16);
      if (dt == kBF16) { v[2 * i] = bf16_bits_to_f32(lo); v[2 * i + 1] = bf16_bits_to_f32(hi); }
      else { v[2 * i] = f16_bits_to_f32(lo); v[2 * i + 1] = f16_bits_to_f32(hi); }
    }
  }
}

__device__ __forceinline__ void store8(void* y, int dt, int64_t idx, const float v[8]) {
  if (dt == kF32) {
    float4* p = reinterpret_cast<float4*>(reinterpret_cast<float*>(y) + idx);
    p[0] = make_float4(v[0], v[1], v[2], v[3]);
    p[1] = make_float4(v[4], v[5], v[6], v[7]);
  } else {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint16_t lo = dt == kBF16 ? f32_to_bf16_bits(v[2 * i]) : f32_to_f16_bits(v[2 * i]);
      uint16_t hi = dt == kBF16 ? f32_to_bf16_bits(v[2 * i + 1]) : f32_to_f16_bits(v[2 * i + 1]);
      w[i] = static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
    }
    *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(y) + idx) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// Produce the 8 transformed values of (row s_out, cols d0..d0+7) of head
// (b, h).  Lanes of one row are lanes [g*lpr, g*lpr+lpr) of the wave; the
// FWHT needs all of them active, so invalid rows still run it on zeros.
__device__ __forceinline__ void transform8(const RowTileArgs& a, int64_t b, int64_t h, int64_t s_out,
                                           bool valid, int d0, int lpr, float v[8], bool store_smoothed) {
  if (valid) {
    int64_t src = s_out;
    if (a.gather) src = a.gather[(b * a.H + h) * a.S + s_out];
    load8(a.x, a.x_dtype, ((b * a.S + src) * a.H + h) * a.D + d0, v);
    if (a.sub_mode != LBFQ_SUB_NONE) {
      const float* m;
      if (a.sub_mode == LBFQ_SUB_COLVEC) m = a.sub + (b * a.H + h) * a.D + d0;
      else m = a.sub + ((b * (a.S / a.sub_block) + s_out / a.sub_block) * a.H + h) * a.D + d0;
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = round_to_dtype(v[i] - m[i], a.x_dtype);
    }
    if (store_smoothed && a.smoothed && a.smoothed_stage == 0)
      store8(a.smoothed, a.x_dtype, ((b * a.S + s_out) * a.H + h) * a.D + d0, v);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = 0.0f;
  }
  if (a.hadamard) {
    if (a.signs) {
      const int8_t* sg = a.signs + h * a.D + d0;
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = sg[i] < 0 ? -v[i] : v[i];
    }
    // In-lane stages: stride 1, 2, 4.
#pragma unroll
    for (int st = 1; st < 8; st <<= 1) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if ((i & st) == 0) {
          float l = v[i], r = v[i + st];
          v[i] = l + r;
          v[i + st] = l - r;
        }
      }
    }
    // Cross-lane stages: stride 8, 16, ... within the row's lpr lanes.
    int lane = threadIdx.x & 63;
    for (int m = 1; m < lpr; m <<= 1) {
      bool upper = (lane & m) != 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float o = __shfl_xor(v[i], m, 64);
        v[i] = upper ? (o - v[i]) : (v[i] + o);
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = round_to_dtype(v[i] * a.had_scale, a.x_dtype);
    if (valid && store_smoothed && a.smoothed && a.smoothed_stage == 1)
      store8(a.smoothed, a.x_dtype, ((b * a.S + s_out) * a.H + h) * a.D + d0, v);
  }
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

__global__ void __launch_bounds__(kThreads) rowtile_kernel(RowTileArgs a) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int lpr = static_cast<int>(a.D / 8);       // lanes per row
  const int rpw = 64 / lpr;                        // rows per wave per pass
  const int rpp = rpw * (kThreads / 64);           // rows per pass
  const int d0 = (lane % lpr) * 8;
  const int row_in_wave = lane / lpr;

  const int64_t ntile = (a.S + a.R - 1) / a.R;
  int64_t bid = blockIdx.x;
  const int64_t h = bid % a.H; bid /= a.H;
  const int64_t tile = bid % ntile;
  const int64_t b = bid / ntile;
  const int64_t s0 = tile * a.R;

  __shared__ float red[kThreads / 64][128];
  __shared__ float sc_sh[128];
  extern __shared__ uint8_t tcodes[];  // BHDS staging: R * D bytes

  const int qm = a.quant_mode;
  const bool two_pass = (qm == LBFQ_Q_FP8_BLOCK || qm == LBFQ_Q_MX_V || qm == LBFQ_Q_CHANNEL_AMAX);
  float v[8];

  // ---- pass 1: reductions for tile-wide scales -----------------------------
  float tmax = 0.0f;
  float cmax[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) cmax[i] = 0.0f;
  if (two_pass) {
    for (int r0 = 0; r0 < a.R; r0 += rpp) {
      int r = r0 + wave * rpw + row_in_wave;
      int64_t s = s0 + r;
      bool valid = r < a.R && s < a.S;
      transform8(a, b, h, s, valid, d0, lpr, v, qm == LBFQ_Q_CHANNEL_AMAX);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float av = valid ? fabsf(v[i]) : 0.0f;
        tmax = fmaxf(tmax, av);
        cmax[i] = fmaxf(cmax[i], av);
      }
    }
    if (qm == LBFQ_Q_FP8_BLOCK) {
      tmax = wave_max(tmax);
      if (lane == 0) red[wave][0] = tmax;
      __syncthreads();
      if (threadIdx.x == 0) {
        float m = red[0][0];
        for (int w = 1; w < kThreads / 64; ++w) m = fmaxf(m, red[w][0]);
        m = fmaxf(m, kAmaxFloor);
        float sc = m / kFp8Max;
        sc_sh[0] = sc;
        a.scale[b * a.sc_b + tile * a.sc_s + h * a.sc_h] = sc;
      }
      __syncthreads();
    } else {
      // per-column max over rows: lanes with equal (lane % lpr) share columns
#pragma unroll
      for (int i = 0; i < 8; ++i)
        for (int m = lpr; m < 64; m <<= 1) cmax[i] = fmaxf(cmax[i], __shfl_xor(cmax[i], m, 64));
      if (row_in_wave == 0) {
#pragma unroll
        for (int i = 0; i < 8; ++i) red[wave][d0 + i] = cmax[i];
      }
      __syncthreads();
      if (threadIdx.x < a.D) {
        float m = red[0][threadIdx.x];
        for (int w = 1; w < kThreads / 64; ++w) m = fmaxf(m, red[w][threadIdx.x]);
        if (qm == LBFQ_Q_CHANNEL_AMAX) {
          atomicMax(a.amax_table + (b * a.H + h) * a.D + threadIdx.x, __float_as_uint(m));
        } else {
          m = fmaxf(m, kAmaxFloor);
          float sc = mx_scale_from_amax(m);
          sc_sh[threadIdx.x] = sc;
          int64_t si = b * a.sc_b + tile * a.sc_s + h * a.sc_h + threadIdx.x * a.sc_d;
          if (a.scale_e8m0) reinterpret_cast<uint8_t*>(a.scale)[si] = static_cast<uint8_t>(__float_as_uint(sc) >> 23);
          else a.scale[si] = sc;
        }
      }
      __syncthreads();
    }
    if (qm == LBFQ_Q_CHANNEL_AMAX) return;
  }

  // ---- pass 2 (or the only pass): transform, quantise, write -------------
  if (qm == LBFQ_Q_CHANNEL && tile == 0 && threadIdx.x < a.D && a.scale) {
    float m = __uint_as_float(a.amax_table[(b * a.H + h) * a.D + threadIdx.x]);
    a.scale[b * a.sc_b + h * a.sc_h + threadIdx.x * a.sc_d] = m / kFp8Max;
  }
  for (int r0 = 0; r0 < a.R; r0 += rpp) {
    int r = r0 + wave * rpw + row_in_wave;
    int64_t s = s0 + r;
    bool valid = r < a.R && s < a.S;
    transform8(a, b, h, s, valid, d0, lpr, v, true);
    if (qm == LBFQ_Q_NONE) continue;
    float sc8[8];
    if (qm == LBFQ_Q_FP8_BLOCK) {
#pragma unroll
      for (int i = 0; i < 8; ++i) sc8[i] = sc_sh[0];
    } else if (qm == LBFQ_Q_MX_V) {
#pragma unroll
      for (int i = 0; i < 8; ++i) sc8[i] = sc_sh[d0 + i];
    } else if (qm == LBFQ_Q_CHANNEL) {
      const uint32_t* t = a.amax_table + (b * a.H + h) * a.D + d0;
#pragma unroll
      for (int i = 0; i < 8; ++i) sc8[i] = __uint_as_float(t[i]) / kFp8Max;
    } else {  // LBFQ_Q_MX_QK: mx_block/8 lanes share a scale
      float m = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(v[i]));
      const int ml = a.mx_block / 8;
      for (int o = 1; o < ml; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
      m = fmaxf(m, kAmaxFloor);
      float sc = mx_scale_from_amax(m);
#pragma unroll
      for (int i = 0; i < 8; ++i) sc8[i] = sc;
      if (valid && (lane & (ml - 1)) == 0) {
        int64_t si = b * a.sc_b + s * a.sc_s + h * a.sc_h + (d0 / a.mx_block) * a.sc_d;
        if (a.scale_e8m0) reinterpret_cast<uint8_t*>(a.scale)[si] = static_cast<uint8_t>(__float_as_uint(sc) >> 23);
        else a.scale[si] = sc;
      }
    }
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) lo |= static_cast<uint32_t>(quant_e4m3(v[i], sc8[i])) << (8 * i);
#pragma unroll
    for (int i = 0; i < 4; ++i) hi |= static_cast<uint32_t>(quant_e4m3(v[4 + i], sc8[4 + i])) << (8 * i);
    if (!valid) continue;
    if (a.codes_layout == LBFQ_LAYOUT_NHD) {
      *reinterpret_cast<uint2*>(a.codes + ((b * a.S + s) * a.H + h) * a.D + d0) = make_uint2(lo, hi);
    } else if (a.codes_layout == LBFQ_LAYOUT_BHSD) {
      *reinterpret_cast<uint2*>(a.codes + ((b * a.H + h) * a.codes_spitch + s) * a.D + d0) = make_uint2(lo, hi);
    } else {
      *reinterpret_cast<uint2*>(tcodes + r * a.D + d0) = make_uint2(lo, hi);
    }
  }
  if (qm != LBFQ_Q_NONE && a.codes_layout == LBFQ_LAYOUT_BHDS) {
    __syncthreads();
    // Write the tile transposed: row d of the output holds R consecutive keys.
    int64_t nvalid = a.S - s0 < a.R ? a.S - s0 : a.R;
    for (int e = threadIdx.x; e < a.D * a.R; e += kThreads) {
      int d = e / a.R, r = e % a.R;
      if (r < nvalid) a.codes[((b * a.H + h) * a.D + d) * a.codes_spitch + s0 + r] = tcodes[r * a.D + d];
    }
  }
}

// Sequential fp64 column sums of `chunk` rows (optionally gathered).
// mode 0: write fp64 partial sums (B, nchunk, H, D);
// mode 1: write fp32 means fp32(sum / rows_in_chunk) (B, nchunk, H, D).
__global__ void colsum_kernel(const void* x, int dt, int64_t B, int64_t S, int64_t H, int64_t D,
                              int chunk, const int32_t* gather, int mode, double* part, float* mean) {
  const int64_t nchunk = (S + chunk - 1) / chunk;
  int64_t bid = blockIdx.x;
  const int64_t h = bid % H; bid /= H;
  const int64_t c = bid % nchunk;
  const int64_t b = bid / nchunk;
  const int d = threadIdx.x;
  if (d >= D) return;
  const int64_t s0 = c * chunk;
  const int64_t s1 = s0 + chunk < S ? s0 + chunk : S;
  double acc = 0.0;
  for (int64_t s = s0; s < s1; ++s) {
    int64_t src = gather ? gather[(b * H + h) * S + s] : s;
    acc += static_cast<double>(load_as_f32(x, ((b * S + src) * H + h) * D + d, dt));
  }
  int64_t o = ((b * nchunk + c) * H + h) * D + d;
  if (mode == 0) part[o] = acc;
  else mean[o] = static_cast<float>(acc / static_cast<double>(s1 - s0));
}

// Sum the chunk partials in chunk order; mean = fp32(total / S).
__global__ void colsum_finalize_kernel(const double* part, int64_t B, int64_t nchunk, int64_t H, int64_t D,
                                       int64_t S, float* mean) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= B * H * D) return;
  int64_t d = i % D, h = (i / D) % H, b = i / (D * H);
  double t = 0.0;
  for (int64_t c = 0; c < nchunk; ++c) t += part[((b * nchunk + c) * H + h) * D + d];
  mean[(b * H + h) * D + d] = static_cast<float>(t / static_cast<double>(S));
}

__global__ void fill_u32_kernel(uint32_t* p, int64_t n, uint32_t v) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// codes (B,S,H,D) NHD -> out dtype, value = dtype(decode(code) * scale).
__global__ void dequant_kernel(const uint8_t* codes, const float* scale, int64_t B, int64_t S, int64_t H,
                               int64_t D, int mode, int block, void* out, int out_dt) {
  int64_t i = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 8;
  int64_t n = B * S * H * D;
  if (i >= n) return;
  int64_t d0 = i % D, h = (i / D) % H, s = (i / (D * H)) % S, b = i / (D * H * S);
  uint2 c = *reinterpret_cast<const uint2*>(codes + i);
  float v[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    uint32_t w = k < 4 ? c.x : c.y;
    uint8_t cb = static_cast<uint8_t>((w >> (8 * (k & 3))) & 0xffu);
    int64_t d = d0 + k;
    float sc;
    if (mode == LBFQ_DQ_BLOCK) sc = scale[(b * (S / block) + s / block) * H + h];
    else if (mode == LBFQ_DQ_CHANNEL) sc = scale[(b * H + h) * D + d];
    else if (mode == LBFQ_DQ_MX_QK) sc = scale[((b * S + s) * H + h) * (D / block) + d / block];
    else sc = scale[((b * (S / block) + s / block) * H + h) * D + d];
    v[k] = e4m3_decode(cb) * sc;
  }
  store8(out, out_dt, i, v);
}

}  // namespace

extern "C" int lbfq_rowtile(const lbfq_rowtile_params* p, lbfq_stream_t stream) {
  LBFQ_CHECK_ARG(p && p->x, "lbfq_rowtile: null input");
  LBFQ_CHECK_ARG(p->D == 64 || p->D == 128, "lbfq_rowtile: D must be 64 or 128; got %lld", (long long)p->D);
  LBFQ_CHECK_ARG(p->x_dtype >= 0 && p->x_dtype <= 2, "lbfq_rowtile: bad dtype %d", p->x_dtype);
  LBFQ_CHECK_ARG(p->R > 0 && p->R <= 1024, "lbfq_rowtile: bad tile rows %d", p->R);
  LBFQ_CHECK_ARG(p->B > 0 && p->S > 0 && p->H > 0, "lbfq_rowtile: empty shape");
  LBFQ_CHECK_ARG(p->sub_mode != LBFQ_SUB_BLOCKVEC || (p->sub_block > 0 && p->S % p->sub_block == 0),
                 "lbfq_rowtile: sub_block must divide S");
  LBFQ_CHECK_ARG(p->sub_mode == LBFQ_SUB_NONE || p->sub, "lbfq_rowtile: missing subtract table");
  const int qm = p->quant_mode;
  LBFQ_CHECK_ARG(qm >= LBFQ_Q_NONE && qm <= LBFQ_Q_CHANNEL_AMAX, "lbfq_rowtile: bad quant mode %d", qm);
  LBFQ_CHECK_ARG(qm == LBFQ_Q_NONE || qm == LBFQ_Q_CHANNEL_AMAX || p->codes, "lbfq_rowtile: missing codes");
  LBFQ_CHECK_ARG(qm == LBFQ_Q_NONE || qm == LBFQ_Q_CHANNEL_AMAX || qm == LBFQ_Q_CHANNEL || p->scale,
                 "lbfq_rowtile: missing scale output");
  LBFQ_CHECK_ARG((qm != LBFQ_Q_CHANNEL && qm != LBFQ_Q_CHANNEL_AMAX) || p->amax_table,
                 "lbfq_rowtile: channel modes need the amax table");
  LBFQ_CHECK_ARG(qm != LBFQ_Q_FP8_BLOCK || p->S % p->R == 0, "lbfq_rowtile: S=%lld must be divisible by block %d",
                 (long long)p->S, p->R);
  LBFQ_CHECK_ARG(qm != LBFQ_Q_MX_V || p->S % p->R == 0, "lbfq_rowtile: S must be divisible by the MX-V block");
  LBFQ_CHECK_ARG(qm != LBFQ_Q_MX_QK || (p->mx_block >= 8 && p->mx_block <= p->D && (p->mx_block & (p->mx_block - 1)) == 0),
                 "lbfq_rowtile: MX block along D must be a power of two in [8, D]; got %d", p->mx_block);
  LBFQ_CHECK_ARG(p->codes_layout != LBFQ_LAYOUT_BHDS || p->R * p->D <= 65536, "lbfq_rowtile: tile too large");
  LBFQ_CHECK_ARG(p->codes_layout == LBFQ_LAYOUT_NHD || p->codes_spitch >= p->S, "lbfq_rowtile: bad codes pitch");
  RowTileArgs a;
  a.x = p->x; a.x_dtype = p->x_dtype; a.B = p->B; a.S = p->S; a.H = p->H; a.D = p->D; a.R = p->R;
  a.gather = p->gather; a.sub_mode = p->sub_mode; a.sub = p->sub; a.sub_block = p->sub_block;
  a.smoothed = p->smoothed; a.hadamard = p->hadamard; a.signs = p->signs; a.had_scale = p->had_scale;
  a.quant_mode = qm; a.codes = p->codes; a.codes_layout = p->codes_layout; a.codes_spitch = p->codes_spitch;
  a.scale = p->scale; a.sc_b = p->sc_b; a.sc_s = p->sc_s; a.sc_h = p->sc_h; a.sc_d = p->sc_d;
  a.amax_table = p->amax_table;
  a.mx_block = p->mx_block;
  a.smoothed_stage = p->smoothed_stage;
  a.scale_e8m0 = p->scale_e8m0;
  int64_t ntile = (p->S + p->R - 1) / p->R;
  int64_t nblocks = p->B * p->H * ntile;
  LBFQ_CHECK_ARG(nblocks < (1ll << 31), "lbfq_rowtile: grid too large");
  size_t shmem = p->codes_layout == LBFQ_LAYOUT_BHDS ? static_cast<size_t>(p->R * p->D) : 0;
  hipLaunchKernelGGL(rowtile_kernel, dim3(static_cast<unsigned>(nblocks)), dim3(kThreads), shmem,
                     static_cast<hipStream_t>(stream), a);
  LBFQ_LAUNCH_CHECK("lbfq_rowtile");
  return 0;
}

extern "C" int lbfq_colsum(const void* x, int dtype, int64_t B, int64_t S, int64_t H, int64_t D, int chunk,
                           const int32_t* gather, int mode, double* partial, float* mean, lbfq_stream_t stream) {
  LBFQ_CHECK_ARG(x && (D == 64 || D == 128) && chunk > 0 && B > 0 && S > 0 && H > 0, "lbfq_colsum: bad args");
  LBFQ_CHECK_ARG(mode == 0 ? partial != nullptr : mean != nullptr, "lbfq_colsum: missing output");
  int64_t nchunk = (S + chunk - 1) / chunk;
  int64_t nblocks = B * nchunk * H;
  hipLaunchKernelGGL(colsum_kernel, dim3(static_cast<unsigned>(nblocks)), dim3(static_cast<unsigned>(D)), 0,
                     static_cast<hipStream_t>(stream), x, dtype, B, S, H, D, chunk, gather, mode, partial, mean);
  LBFQ_LAUNCH_CHECK("lbfq_colsum");
  return 0;
}

extern "C" int lbfq_colsum_finalize(const double* partial, int64_t B, int64_t nchunk, int64_t H, int64_t D,
                                    int64_t S, float* mean, lbfq_stream_t stream) {
  LBFQ_CHECK_ARG(partial && mean && nchunk > 0 && S > 0, "lbfq_colsum_finalize: bad args");
  int64_t n = B * H * D;
  hipLaunchKernelGGL(colsum_finalize_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), partial, B, nchunk, H, D, S, mean);
  LBFQ_LAUNCH_CHECK("lbfq_colsum_finalize");
  return 0;
}

extern "C" int lbfq_fill_u32(uint32_t* p, int64_t n, uint32_t value, lbfq_stream_t stream) {
  LBFQ_CHECK_ARG(p && n > 0, "lbfq_fill_u32: bad args");
  hipLaunchKernelGGL(fill_u32_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), p, n, value);
  LBFQ_LAUNCH_CHECK("lbfq_fill_u32");
  return 0;
}

extern "C" int lbfq_dequant(const uint8_t* codes, const float* scale, int64_t B, int64_t S, int64_t H, int64_t D,
                            int mode, int block, void* out, int out_dtype, lbfq_stream_t stream) {
  LBFQ_CHECK_ARG(codes && scale && out && (D == 64 || D == 128), "lbfq_dequant: bad args");
  LBFQ_CHECK_ARG(mode >= LBFQ_DQ_BLOCK && mode <= LBFQ_DQ_MX_V, "lbfq_dequant: bad mode");
  LBFQ_CHECK_ARG(mode == LBFQ_DQ_CHANNEL || block > 0, "lbfq_dequant: bad block");
  int64_t n8 = B * S * H * D / 8;
  hipLaunchKernelGGL(dequant_kernel, dim3(static_cast<unsigned>((n8 + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), codes, scale, B, S, H, D, mode, block, out, out_dtype);
  LBFQ_LAUNCH_CHECK("lbfq_dequant");
  return 0;
}
