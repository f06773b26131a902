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
  uint32_t ntile;  // ceil(S / R)
  uint32_t nsub;   // S / sub_block (BLOCKVEC)
};

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

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

// Load 8 consecutive elements of dtype DT as fp32 (exact widening).
template <int DT>
__device__ __forceinline__ void load8t(const void* x, int64_t idx, float v[8]) {
  if constexpr (DT == kF32) {
    const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(x) + idx);
    const float4 a = p[0], b = p[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    const uint4 r = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(x) + idx);
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint16_t lo = static_cast<uint16_t>(w[i] & 0xffffu), hi = static_cast<uint16_t>(w[i] >> 16);
      if constexpr (DT == kBF16) { v[2 * i] = bf16_bits_to_f32(lo); v[2 * i + 1] = bf16_bits_to_f32(hi); }
      else { v[2 * i] = f16_bits_to_f32(lo); v[2 * i + 1] = f16_bits_to_f32(hi); }
    }
  }
}

template <int DT>
__device__ __forceinline__ void load8p(const uint8_t* p, float v[8]) {
  if constexpr (DT == kF32) {
    const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    const uint4 r = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint16_t lo = static_cast<uint16_t>(w[i] & 0xffffu), hi = static_cast<uint16_t>(w[i] >> 16);
      if constexpr (DT == kBF16) { v[2 * i] = bf16_bits_to_f32(lo); v[2 * i + 1] = bf16_bits_to_f32(hi); }
      else { v[2 * i] = f16_bits_to_f32(lo); v[2 * i + 1] = f16_bits_to_f32(hi); }
    }
  }
}

template <int DT>
__device__ __forceinline__ float round_dt(float v) {
  if constexpr (DT == kBF16) return bf16_bits_to_f32(f32_to_bf16_bits(v));
  else if constexpr (DT == kF16) return f16_bits_to_f32(f32_to_f16_bits(v));
  else return v;
}


// ---- one workgroup per R-row tile ------------------------------------------
// A workgroup of four waves owns one (b, h, R-row tile).  A pass covers
// rpw = 64 / (D/8) rows: lane l holds columns d0 = 8 (l % (D/8)) .. d0+7 of
// row rl = l / (D/8) of the pass.  Wave w takes passes w, w + 4, w + 8, ..., so
// at every step the four waves read 4 rpw adjacent rows.  Tile reductions
// (block amax, per-column amax) are wave reductions followed by one LDS
// exchange.  A tile of up to 4 kKeep passes whose scale depends on the whole
// tile stays in registers (fp32), so it is read from memory once; a longer one
// is read twice.  Transposed (BHDS) codes go through an LDS stage of
// kStageRows rows that all 256 threads write out as dwords of four
// consecutive keys.  Consecutive workgroups take adjacent heads of one row
// tile (adjacent D-element pieces of the same NHD rows).  SUB (a mean is
// subtracted) and HAD (FWHT) are compile-time so that the common cases carry
// no per-element work for the others; the kernel is VALU-issue-bound.
constexpr int kTileWaves = 4;
constexpr int kKeep = 4;        // resident passes per wave
constexpr int kLB = 4;          // passes per wave in flight when streaming
constexpr int kStageRows = 64;  // rows per BHDS staging chunk

template <int DT, int QM, bool SUB, bool HAD>
__global__ void __launch_bounds__(kTileWaves * 64) rowtile_kernel(RowTileArgs a) {
  constexpr bool TILE_RED = QM == LBFQ_Q_FP8_BLOCK || QM == LBFQ_Q_MX_V || QM == LBFQ_Q_CHANNEL_AMAX;
  constexpr bool RESIDENT_MODE = QM == LBFQ_Q_FP8_BLOCK || QM == LBFQ_Q_MX_V;
  constexpr int ES = DT == kF32 ? 4 : 2;  // input element bytes
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // wave-uniform (scalar): the per-wave pass counts below stay scalar, so pass
  // guards are branches, not exec masks that serialise the loads
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lpr = static_cast<int>(a.D / 8);  // lanes per row
  const int rpw = 64 / lpr;                   // rows per wave pass
  const int d0 = (lane % lpr) * 8;
  const int rl = lane / lpr;

  // 32-bit index arithmetic: the grid (B * H * ntile workgroups, exactly) is
  // below 2^31
  const uint32_t ntile = a.ntile;
  const uint32_t H32 = static_cast<uint32_t>(a.H);
  uint32_t t = blockIdx.x;
  const int64_t h = t % H32;
  t /= H32;
  const int64_t tile = t % ntile;
  const int64_t b = t / ntile;
  const int64_t bh = b * a.H + h;
  const int64_t s0 = tile * a.R;
  const int np = a.R / rpw;                                     // passes of the tile (R is a multiple of rpw)
  const int npw_max = (np + kTileWaves - 1) / kTileWaves;       // passes of wave 0 (the most)
  const int npw = np > wv ? (np - wv + kTileWaves - 1) / kTileWaves : 0;  // passes of this wave
  const int nvalid = a.S - s0 < a.R ? static_cast<int>(a.S - s0) : a.R;  // rows of the tile below S
  // every pass of every wave holds valid rows (no zeroing needed)
  const bool tile_full = nvalid == a.R && np % kTileWaves == 0;
  const int tcp = static_cast<int>(a.D) + 4;
  const bool bhds = a.codes_layout == LBFQ_LAYOUT_BHDS;
  const int ipc = kStageRows / rpw / kTileWaves;                // passes per wave and staging chunk

  // Per-tile bases; a row offset within one (b, h) is a 32 x 32 -> 64-bit
  // product (S, H * D and the code pitch are below 2^31, checked on the host).
  const uint32_t hd = static_cast<uint32_t>(a.H * a.D);
  const uint8_t* xlane = static_cast<const uint8_t*>(a.x) + ((b * a.S * a.H + h) * a.D + d0) * ES;
  const uint32_t x_row_bytes = hd * ES;
  const int32_t* gath = a.gather ? a.gather + bh * a.S : nullptr;
  // the subtracted mean row: one per tile for COLVEC and for a BLOCKVEC group
  // that holds the whole tile (sub_block a multiple of R), else one per pass
  bool sub_fixed = true;
  const float* sub_lane = nullptr;
  float mfix[8];
  if constexpr (SUB) {
    sub_fixed = a.sub_mode == LBFQ_SUB_COLVEC || a.sub_block % a.R == 0;
    sub_lane = a.sub_mode == LBFQ_SUB_COLVEC ? a.sub + bh * a.D + d0 : a.sub + (b * a.nsub * a.H + h) * a.D + d0;
    if (sub_fixed) {
      const float* m = sub_lane + (a.sub_mode == LBFQ_SUB_BLOCKVEC
                                       ? static_cast<uint64_t>(static_cast<uint32_t>(s0) / static_cast<uint32_t>(a.sub_block)) * hd
                                       : 0);
      const float4 m0 = reinterpret_cast<const float4*>(m)[0], m1 = reinterpret_cast<const float4*>(m)[1];
      mfix[0] = m0.x; mfix[1] = m0.y; mfix[2] = m0.z; mfix[3] = m0.w;
      mfix[4] = m1.x; mfix[5] = m1.y; mfix[6] = m1.z; mfix[7] = m1.w;
    }
  }
  const bool sm0 = a.smoothed && a.smoothed_stage == 0, sm1 = a.smoothed && a.smoothed_stage == 1;
  __shared__ float red[kTileWaves][128];  // cross-wave reductions (D <= 128)
  extern __shared__ uint8_t stage[];      // BHDS staging: kStageRows rows of tcp bytes

  // ---- load + transform -----------------------------------------------------
  // source row of pass p (a row >= nvalid reads the tile's first row, unused)
  auto pass_src = [&](int p) -> uint32_t {
    const int r = p * rpw + rl;
    uint32_t src = static_cast<uint32_t>(s0 + (r < nvalid ? r : 0));
    if (gath) src = static_cast<uint32_t>(gath[src]);
    return src;
  };
  auto load_pass = [&](uint32_t src, float (&x)[8]) {
    load8p<DT>(xlane + static_cast<uint64_t>(src) * x_row_bytes, x);
  };
  // subtract, zero rows past the tile, optional smoothed copy, optional FWHT
  auto transform = [&](int p, float (&x)[8], bool store_smoothed) {
    const int r = p * rpw + rl;
    const bool okp = r < nvalid;
    const int64_t s_out = s0 + (okp ? r : 0);
    if constexpr (SUB) {
      float mm[8];
      if (sub_fixed) {
#pragma unroll
        for (int k = 0; k < 8; ++k) mm[k] = mfix[k];
      } else {
        const float* m = sub_lane + static_cast<uint64_t>(static_cast<uint32_t>(s_out) /
                                                          static_cast<uint32_t>(a.sub_block)) * hd;
        const float4 m0 = reinterpret_cast<const float4*>(m)[0], m1 = reinterpret_cast<const float4*>(m)[1];
        mm[0] = m0.x; mm[1] = m0.y; mm[2] = m0.z; mm[3] = m0.w;
        mm[4] = m1.x; mm[5] = m1.y; mm[6] = m1.z; mm[7] = m1.w;
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) x[k] = round_dt<DT>(as_f32(x[k] - mm[k]));
    }
    if (!tile_full) {
#pragma unroll
      for (int k = 0; k < 8; ++k) x[k] = okp ? x[k] : 0.0f;
    }
    if (store_smoothed && sm0 && okp) store8(a.smoothed, DT, ((b * a.S + s_out) * a.H + h) * a.D + d0, x);
    if constexpr (HAD) {
      if (a.signs) {
        const int8_t* sg = a.signs + h * a.D + d0;
#pragma unroll
        for (int k = 0; k < 8; ++k) x[k] = sg[k] < 0 ? -x[k] : x[k];
      }
#pragma unroll
      for (int st = 1; st < 8; st <<= 1) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          if ((k & st) == 0) {
            const float l = x[k], rr = x[k + st];
            x[k] = l + rr;
            x[k + st] = l - rr;
          }
        }
      }
      // cross-lane stages: stride 8, 16, ... within the row's lpr lanes
      for (int m = 1; m < lpr; m <<= 1) {
        const bool upper = (lane & m) != 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const float o = __shfl_xor(x[k], m, 64);
          x[k] = upper ? (o - x[k]) : (x[k] + o);
        }
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) x[k] = round_dt<DT>(as_f32(x[k] * a.had_scale));
      if (store_smoothed && sm1 && okp) store8(a.smoothed, DT, ((b * a.S + s_out) * a.H + h) * a.D + d0, x);
    }
  };
  // this wave's passes i0 .. i0 + kLB - 1 (pass p = wv + 4 i): every load in
  // flight before the first transform
  float v[kLB][8];
  auto load_group = [&](int i0, bool store_smoothed) {
    uint32_t src[kLB];
#pragma unroll
    for (int i = 0; i < kLB; ++i) src[i] = pass_src(wv + kTileWaves * (i0 + i));
#pragma unroll
    for (int i = 0; i < kLB; ++i) load_pass(src[i], v[i]);
#pragma unroll
    for (int i = 0; i < kLB; ++i) transform(wv + kTileWaves * (i0 + i), v[i], store_smoothed);
  };

  // ---- quantise one pass and write its codes -------------------------------
  float sc8[8], rc8[8];  // per-column scale and reciprocal (block: all equal)
  // NHD / BHSD codes of row s at crow + s * cstride
  const bool nhd = a.codes_layout == LBFQ_LAYOUT_NHD;
  uint8_t* const crow = nhd ? a.codes + (b * a.S * a.H + h) * a.D + d0 : a.codes + bh * a.codes_spitch * a.D + d0;
  const uint32_t cstride = nhd ? hd : static_cast<uint32_t>(a.D);
  uint8_t* const codes_bhds = a.codes + bh * a.D * a.codes_spitch + s0;  // + d * pitch + r
  // rows [r0, r0 + nrows) of the tile are staged: all threads write them
  // transposed, each packing 4 consecutive keys of one d into a dword
  auto flush_stage = [&](int r0, int nrows) {
    const int nv = nvalid - r0 < nrows ? nvalid - r0 : nrows;
    const uint32_t pitch = static_cast<uint32_t>(a.codes_spitch);
    if (nv == kStageRows) {  // a full chunk: 16 dwords per code row
      constexpr int rq = kStageRows / 4;
      for (int e = tid; e < a.D * rq; e += kTileWaves * 64) {
        const int d = e / rq, r = (e % rq) * 4;
        uint32_t w = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) w |= static_cast<uint32_t>(stage[(r + k) * tcp + d]) << (8 * k);
        *reinterpret_cast<uint32_t*>(codes_bhds + static_cast<uint64_t>(static_cast<uint32_t>(d)) * pitch + r0 + r) = w;
      }
      return;
    }
    const int rq = nrows / 4;
    for (int e = tid; e < a.D * rq; e += kTileWaves * 64) {
      const int d = e / rq, r = (e - d * rq) * 4;
      uint8_t* dst = codes_bhds + static_cast<uint64_t>(static_cast<uint32_t>(d)) * pitch + r0 + r;
      if (r + 4 <= nv) {
        uint32_t w = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) w |= static_cast<uint32_t>(stage[(r + k) * tcp + d]) << (8 * k);
        *reinterpret_cast<uint32_t*>(dst) = w;
      } else {
        for (int k = 0; r + k < nv; ++k) dst[k] = stage[(r + k) * tcp + d];
      }
    }
  };
  auto quant_pass = [&](int p, const float (&x)[8]) {
    const int r = p * rpw + rl;
    const bool valid = r < nvalid;
    const uint32_t s = static_cast<uint32_t>(s0 + r);
    float q[8];
    if constexpr (QM == LBFQ_Q_FP8_BLOCK || QM == LBFQ_Q_CHANNEL) {
#pragma unroll
      for (int k = 0; k < 8; ++k) q[k] = clamp448(div_by(x[k], sc8[k], rc8[k]));
    } else if constexpr (QM == LBFQ_Q_MX_V) {
#pragma unroll
      for (int k = 0; k < 8; ++k) q[k] = clamp448(x[k] * rc8[k]);  // rc8 = 2^-e exactly
    } else {  // LBFQ_Q_MX_QK: mx_block/8 lanes of the row share a power-of-two scale
      float m = 0.0f;
#pragma unroll
      for (int k = 0; k < 8; ++k) m = fmaxf(m, fabsf(x[k]));
      const int ml = a.mx_block / 8;
      for (int o = 1; o < ml; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
      m = fmaxf(m, kAmaxFloor);
      const float sc = mx_scale_from_amax(m);
      const float inv = 1.0f / sc;  // exact: 2^-e
#pragma unroll
      for (int k = 0; k < 8; ++k) q[k] = clamp448(x[k] * inv);
      if (valid && (lane & (ml - 1)) == 0) {
        const int64_t si = b * a.sc_b + static_cast<int64_t>(s) * a.sc_s + h * a.sc_h + (d0 / a.mx_block) * a.sc_d;
        if (a.scale_e8m0) reinterpret_cast<uint8_t*>(a.scale)[si] = static_cast<uint8_t>(__float_as_uint(sc) >> 23);
        else a.scale[si] = sc;
      }
    }
    const uint32_t lo = cvt4_e4m3(q), hi = cvt4_e4m3(q + 4);
    if (bhds) {
      uint32_t* st = reinterpret_cast<uint32_t*>(stage + (r % kStageRows) * tcp + d0);
      st[0] = lo;
      st[1] = hi;
    } else if (valid) {
      *reinterpret_cast<uint2*>(crow + static_cast<uint64_t>(s) * cstride) = make_uint2(lo, hi);
    }
  };
  // after this wave's pass i (every wave reaches the same i): BHDS writes out
  // a complete staging chunk, or the last one
  auto after_pass = [&](int i) {
    if (bhds && ((i + 1) % ipc == 0 || i + 1 == npw_max)) {
      const int c = i / ipc;
      __syncthreads();
      flush_stage(c * kStageRows, np * rpw - c * kStageRows < kStageRows ? np * rpw - c * kStageRows : kStageRows);
      __syncthreads();
    }
  };

  // ---- scales that do not depend on the tile --------------------------------
  if constexpr (QM == LBFQ_Q_CHANNEL) {
    const uint32_t* tb = a.amax_table + bh * a.D + d0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      sc8[k] = __uint_as_float(tb[k]) / kFp8Max;
      rc8[k] = 1.0f / sc8[k];
    }
    if (tile == 0 && wv == 0 && rl == 0 && a.scale) {
#pragma unroll
      for (int k = 0; k < 8; ++k) a.scale[b * a.sc_b + h * a.sc_h + (d0 + k) * a.sc_d] = sc8[k];
    }
  }

  if constexpr (TILE_RED) {
    // ---- reductions over the tile (resident: keep the values) ---------------
    const bool resident = RESIDENT_MODE && npw_max <= kKeep;
    float keep[kKeep][8];
    float tmax = 0.0f, cmax[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) cmax[k] = 0.0f;
    auto reduce_pass = [&](const float (&x)[8]) {
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float av = fabsf(x[k]);  // zero for rows past the tile
        if constexpr (QM == LBFQ_Q_FP8_BLOCK) tmax = fmaxf(tmax, av);
        else cmax[k] = fmaxf(cmax[k], av);
      }
    };
    if (resident) {
      // compile-time pass slots, so the kept values stay in registers; every
      // slot is loaded (a slot past this wave's passes reads a safe row and is
      // not used), so all loads are in flight together
      uint32_t src[kKeep];
#pragma unroll
      for (int i = 0; i < kKeep; ++i) src[i] = pass_src(wv + kTileWaves * i);
#pragma unroll
      for (int i = 0; i < kKeep; ++i) load_pass(src[i], keep[i]);
#pragma unroll
      for (int i = 0; i < kKeep; ++i) {
        if (i < npw) {
          transform(wv + kTileWaves * i, keep[i], true);
          reduce_pass(keep[i]);
        }
      }
    } else {
      for (int i0 = 0; i0 < npw; i0 += kLB) {
        load_group(i0, QM == LBFQ_Q_CHANNEL_AMAX);
#pragma unroll
        for (int i = 0; i < kLB; ++i)
          if (i0 + i < npw) reduce_pass(v[i]);
      }
    }
    if constexpr (QM == LBFQ_Q_FP8_BLOCK) {
      const float wm = wave_max(tmax);
      if (lane == 0) red[wv][0] = wm;
      __syncthreads();
      const float m = fmaxf(fmaxf(fmaxf(red[0][0], red[1][0]), fmaxf(red[2][0], red[3][0])), kAmaxFloor);
      const float sc = m / kFp8Max, rc = 1.0f / sc;
#pragma unroll
      for (int k = 0; k < 8; ++k) { sc8[k] = sc; rc8[k] = rc; }
      if (tid == 0) a.scale[b * a.sc_b + tile * a.sc_s + h * a.sc_h] = sc;
    } else {
      // per-column max over the tile: lanes with equal d0 hold the same
      // columns, then the four waves' maxima
#pragma unroll
      for (int k = 0; k < 8; ++k)
        for (int m = lpr; m < 64; m <<= 1) cmax[k] = fmaxf(cmax[k], __shfl_xor(cmax[k], m, 64));
      if (rl == 0) {
#pragma unroll
        for (int k = 0; k < 8; ++k) red[wv][d0 + k] = cmax[k];
      }
      __syncthreads();
#pragma unroll
      for (int k = 0; k < 8; ++k)
        cmax[k] = fmaxf(fmaxf(red[0][d0 + k], red[1][d0 + k]), fmaxf(red[2][d0 + k], red[3][d0 + k]));
      if constexpr (QM == LBFQ_Q_CHANNEL_AMAX) {
        if (wv == 0 && rl == 0) {
#pragma unroll
          for (int k = 0; k < 8; ++k) atomicMax(a.amax_table + bh * a.D + d0 + k, __float_as_uint(cmax[k]));
        }
        return;
      } else {  // MX_V
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const float sc = mx_scale_from_amax(fmaxf(cmax[k], kAmaxFloor));
          sc8[k] = sc;
          rc8[k] = 1.0f / sc;  // exact: 2^-e
          if (wv == 0 && rl == 0) {
            const int64_t si = b * a.sc_b + tile * a.sc_s + h * a.sc_h + (d0 + k) * a.sc_d;
            if (a.scale_e8m0) reinterpret_cast<uint8_t*>(a.scale)[si] = static_cast<uint8_t>(__float_as_uint(sc) >> 23);
            else a.scale[si] = sc;
          }
        }
      }
    }
    if (resident) {
#pragma unroll
      for (int i = 0; i < kKeep; ++i) {
        if (i < npw_max) {
          if (i < npw) quant_pass(wv + kTileWaves * i, keep[i]);
          after_pass(i);
        }
      }
      return;
    }
  }

  // ---- streaming passes (single-pass modes, or a second read of a large tile)
  for (int i0 = 0; i0 < npw_max; i0 += kLB) {
    load_group(i0, true);
    if constexpr (QM == LBFQ_Q_NONE) continue;
#pragma unroll
    for (int i = 0; i < kLB; ++i) {
      if (i0 + i < npw_max) {
        if (i0 + i < npw) quant_pass(wv + kTileWaves * (i0 + i), v[i]);
        after_pass(i0 + i);
      }
    }
  }
}

// Sequential fp64 column sums of `chunk` rows (optionally gathered).
// mode 0: write fp64 partial sums (B, nchunk, H, D);
// mode 1: write fp32 means fp32(sum / rows_in_chunk) (B, nchunk, H, D).
// One thread sums 8 adjacent columns of one (b, chunk, h) over the chunk's
// rows in order; adjacent threads take adjacent 16-byte pieces of a row
// (columns, then heads), so a wave reads contiguous memory.  Loads of 8 rows
// are in flight before they are added, in row order.
template <int DT>
__global__ void __launch_bounds__(256) colsum_kernel(const void* x, int64_t B, int64_t S, int64_t H, int64_t D,
                                                     int chunk, const int32_t* gather, int mode, double* part,
                                                     float* mean) {
  const int64_t ndg = D / 8;
  const int64_t nchunk = (S + chunk - 1) / chunk;
  int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= B * nchunk * H * ndg) return;
  const int64_t dg = t % ndg; t /= ndg;
  const int64_t h = t % H; t /= H;
  const int64_t c = t % nchunk;
  const int64_t b = t / nchunk;
  const int64_t s0 = c * chunk;
  const int64_t s1 = s0 + chunk < S ? s0 + chunk : S;
  const int64_t d0 = dg * 8;
  double acc[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) acc[k] = 0.0;
  constexpr int kRows = 8;
  for (int64_t sb = s0; sb < s1; sb += kRows) {
    float v[kRows][8];
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
      int64_t s = sb + i < s1 ? sb + i : s0;  // a safe row past the chunk end (not added)
      if (gather) s = gather[(b * H + h) * S + s];
      load8t<DT>(x, ((b * S + s) * H + h) * D + d0, v[i]);
    }
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
      if (sb + i < s1) {
#pragma unroll
        for (int k = 0; k < 8; ++k) acc[k] += static_cast<double>(v[i][k]);
      }
    }
  }
  const int64_t o = ((b * nchunk + c) * H + h) * D + d0;
  if (mode == 0) {
#pragma unroll
    for (int k = 0; k < 8; ++k) part[o + k] = acc[k];
  } else {
    const double n = static_cast<double>(s1 - s0);
#pragma unroll
    for (int k = 0; k < 8; ++k) mean[o + k] = static_cast<float>(acc[k] / n);
  }
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

namespace {

template <int DT, int QM>
void launch_rowtile_qm(bool sub, bool had, dim3 grid, dim3 block, size_t shmem, hipStream_t st, const RowTileArgs& a) {
  if constexpr (QM == LBFQ_Q_NONE || QM == LBFQ_Q_FP8_BLOCK || QM == LBFQ_Q_MX_QK) {
    if (had) {
      if (sub) hipLaunchKernelGGL((rowtile_kernel<DT, QM, true, true>), grid, block, shmem, st, a);
      else hipLaunchKernelGGL((rowtile_kernel<DT, QM, false, true>), grid, block, shmem, st, a);
      return;
    }
  }
  if (sub) hipLaunchKernelGGL((rowtile_kernel<DT, QM, true, false>), grid, block, shmem, st, a);
  else hipLaunchKernelGGL((rowtile_kernel<DT, QM, false, false>), grid, block, shmem, st, a);
}

template <int DT>
void launch_rowtile(int qm, bool sub, bool had, dim3 grid, dim3 block, size_t shmem, hipStream_t st,
                    const RowTileArgs& a) {
  switch (qm) {
    case LBFQ_Q_NONE: launch_rowtile_qm<DT, LBFQ_Q_NONE>(sub, had, grid, block, shmem, st, a); break;
    case LBFQ_Q_FP8_BLOCK: launch_rowtile_qm<DT, LBFQ_Q_FP8_BLOCK>(sub, had, grid, block, shmem, st, a); break;
    case LBFQ_Q_CHANNEL: launch_rowtile_qm<DT, LBFQ_Q_CHANNEL>(sub, had, grid, block, shmem, st, a); break;
    case LBFQ_Q_MX_QK: launch_rowtile_qm<DT, LBFQ_Q_MX_QK>(sub, had, grid, block, shmem, st, a); break;
    case LBFQ_Q_MX_V: launch_rowtile_qm<DT, LBFQ_Q_MX_V>(sub, had, grid, block, shmem, st, a); break;
    default: launch_rowtile_qm<DT, LBFQ_Q_CHANNEL_AMAX>(sub, had, grid, block, shmem, st, a); break;
  }
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
  LBFQ_CHECK_ARG(!p->hadamard || qm == LBFQ_Q_NONE || qm == LBFQ_Q_FP8_BLOCK || qm == LBFQ_Q_MX_QK,
                 "lbfq_rowtile: the Hadamard rotation goes with quant modes NONE, FP8_BLOCK and MX_QK");
  LBFQ_CHECK_ARG(qm == LBFQ_Q_NONE || qm == LBFQ_Q_CHANNEL_AMAX || qm == LBFQ_Q_CHANNEL || p->scale,
                 "lbfq_rowtile: missing scale output");
  LBFQ_CHECK_ARG((qm != LBFQ_Q_CHANNEL && qm != LBFQ_Q_CHANNEL_AMAX) || p->amax_table,
                 "lbfq_rowtile: channel modes need the amax table");
  LBFQ_CHECK_ARG(qm != LBFQ_Q_FP8_BLOCK || p->S % p->R == 0, "lbfq_rowtile: S=%lld must be divisible by block %d",
                 (long long)p->S, p->R);
  LBFQ_CHECK_ARG(qm != LBFQ_Q_MX_V || p->S % p->R == 0, "lbfq_rowtile: S must be divisible by the MX-V block");
  LBFQ_CHECK_ARG(qm != LBFQ_Q_MX_QK || (p->mx_block >= 8 && p->mx_block <= p->D && (p->mx_block & (p->mx_block - 1)) == 0),
                 "lbfq_rowtile: MX block along D must be a power of two in [8, D]; got %d", p->mx_block);

  LBFQ_CHECK_ARG(p->S < (1ll << 31) && p->H * p->D < (1ll << 28) && p->codes_spitch < (1ll << 31),
                 "lbfq_rowtile: S, H * D or the code pitch too large");
  LBFQ_CHECK_ARG(p->codes_layout != LBFQ_LAYOUT_BHDS || p->codes_spitch % 4 == 0,
                 "lbfq_rowtile: transposed codes pitch must be a multiple of 4");
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
  const int64_t ntiles = p->B * p->H * ntile;
  a.ntile = static_cast<uint32_t>(ntile);
  a.nsub = p->sub_mode == LBFQ_SUB_BLOCKVEC ? static_cast<uint32_t>(p->S / p->sub_block) : 0u;
  const int64_t nblocks = ntiles;  // one workgroup per tile
  LBFQ_CHECK_ARG(nblocks < (1ll << 31), "lbfq_rowtile: grid too large");
  LBFQ_CHECK_ARG(p->R % (512 / p->D) == 0, "lbfq_rowtile: R must be a multiple of %lld", (long long)(512 / p->D));
  size_t shmem = p->codes_layout == LBFQ_LAYOUT_BHDS ? static_cast<size_t>(kStageRows * (p->D + 4)) : 0;
  const dim3 grid(static_cast<unsigned>(nblocks)), block(kTileWaves * 64);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const bool sub = p->sub_mode != LBFQ_SUB_NONE, had = p->hadamard != 0;
  if (p->x_dtype == kBF16) launch_rowtile<kBF16>(qm, sub, had, grid, block, shmem, st, a);
  else if (p->x_dtype == kF16) launch_rowtile<kF16>(qm, sub, had, grid, block, shmem, st, a);
  else launch_rowtile<kF32>(qm, sub, had, grid, block, shmem, st, a);
  LBFQ_LAUNCH_CHECK("lbfq_rowtile");
  return 0;
}

extern "C" int lbfq_colsum(const void* x, int dtype, int64_t B, int64_t S, int64_t H, int64_t D, int chunk,
                           const int32_t* gather, int mode, double* partial, float* mean, lbfq_stream_t stream) {
  LBFQ_CHECK_ARG(x && (D == 64 || D == 128) && chunk > 0 && B > 0 && S > 0 && H > 0, "lbfq_colsum: bad args");
  LBFQ_CHECK_ARG(mode == 0 ? partial != nullptr : mean != nullptr, "lbfq_colsum: missing output");
  LBFQ_CHECK_ARG(dtype >= 0 && dtype <= 2, "lbfq_colsum: bad dtype %d", dtype);
  const int64_t nchunk = (S + chunk - 1) / chunk;
  const int64_t nthreads = B * nchunk * H * (D / 8);
  const dim3 grid(static_cast<unsigned>((nthreads + 255) / 256)), block(256);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == kBF16)
    hipLaunchKernelGGL(colsum_kernel<kBF16>, grid, block, 0, st, x, B, S, H, D, chunk, gather, mode, partial, mean);
  else if (dtype == kF16)
    hipLaunchKernelGGL(colsum_kernel<kF16>, grid, block, 0, st, x, B, S, H, D, chunk, gather, mode, partial, mean);
  else
    hipLaunchKernelGGL(colsum_kernel<kF32>, grid, block, 0, st, x, B, S, H, D, chunk, gather, mode, partial, mean);
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
