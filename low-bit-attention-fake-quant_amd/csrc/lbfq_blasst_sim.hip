// BLASST tile-skip simulator kernels (gfx950).
//
// The reference simulator (blasst_skip.py:389-654) measures FP8 fake quant +
// whole-tile BLASST skipping on 128-query x 128-key tiles with per-head static
// FP8 scales.  Its semantics, restated here:
//
//   per-head quant    scale_h = max(amax_h / 448, FLT_MIN); deq = e4m3(x / scale) * scale
//                     (blasst_skip.py:278-297)
//   scores            s = (q . k) * sm_scale in fp32 over operands already rounded
//                     to the matmul dtype (blasst_skip.py:477-480, 499-500)
//   block statistics  bmax_j = max over the 128 keys of block j; running max
//                     rm_j = max(rm_{j-1}, bmax_j); final max M = rm_last
//   rungs             exact: p = exp(s - M)                          (:484-491)
//                     online: w = exp(s - rm_j) * exp(rm_j - M)      (:502-519)
//                     static P: pq = e4m3(exp(s - rm_j) * 256) / 256, numerator
//                     pq * exp(rm_j - M), denominator the unquantised w (:526-570)
//                     PV operands rounded to the matmul dtype, fp32 sums
//   tile predicate    tile_margin_j = max over the tile's 128 rows of (bmax_j - rm_j);
//                     keep_j = tile_margin_j >= log(threshold); a tile keeping no
//                     block keeps the first block of largest max-over-rows bmax
//                     (blasst_skip.py:375-386, 584-619)
//
// Work decomposition: one wave per 64 / LPR query rows of one head, LPR =
// D / 64 lanes per row, each holding 64 dimensions of the row's q and output
// in registers; the lanes of a row read the same key rows at a time, four
// keys' dot products as four independent chains.  The online and static-P
// rungs form each key block's scores once, in the block-max pass, and keep
// them in LDS (32 KB per wave at D = 64, 16 KB at D = 128) for the
// accumulation pass.  Tile statistics are combined across the waves of a
// 128-row tile by ordered-integer atomicMax.
#include <algorithm>

#include "lbfq_common.h"
#include "../../include/lbfq.h"

using namespace lbfq;

namespace {

constexpr int kTileQ = 128;  // query tile / key block (QUERY_TILE, KEY_BLOCK)
constexpr float kDenomFloor = 1e-30f;

__device__ __forceinline__ uint32_t ordered_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float from_ordered_bits(uint32_t u) {
  return __uint_as_float((u & 0x80000000u) ? (u & 0x7fffffffu) : ~u);
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}
__device__ __forceinline__ float round_bf16(float v) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }

// ---- per-head static FP8 fake quant --------------------------------------------
template <int DT>
__global__ void __launch_bounds__(256) head_amax_kernel(const void* x, int64_t S, int64_t H, int64_t D,
                                                        uint32_t* amax_bits) {
  const int64_t h = blockIdx.y;
  float m = 0.0f;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; e < S * D;
       e += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t s = e / D, d = e - s * D;
    m = fmaxf(m, fabsf(load_as_f32(x, (s * H + h) * D + d, DT)));
  }
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) atomicMax(amax_bits + h, __float_as_uint(m));  // m >= 0
}

template <int DT>
__global__ void __launch_bounds__(256) head_quant_kernel(const void* x, int64_t n, int64_t H, int64_t D,
                                                         const uint32_t* amax_bits, float* deq, float* deq_mm,
                                                         int mm_bf16, float* scale_out,
                                                         unsigned long long* counts, double* sqerr) {
  unsigned long long sat = 0, uf = 0;
  double sq = 0.0;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t h = (i / D) % H;
    const float sc = fmaxf(__uint_as_float(amax_bits[h]) / kFp8Max, 1.17549435e-38f);
    const float xf = load_as_f32(x, i, DT);
    const float scaled = xf / sc;
    const float q = e4m3_decode(e4m3_encode(scaled));
    const float dq = q * sc;
    if (deq) deq[i] = dq;
    if (deq_mm) deq_mm[i] = mm_bf16 ? round_bf16(dq) : dq;
    sat += fabsf(scaled) > kFp8Max ? 1ull : 0ull;
    uf += (q == 0.0f && scaled != 0.0f) ? 1ull : 0ull;
    const double e = static_cast<double>(dq) - static_cast<double>(xf);
    sq += e * e;
  }
  if (blockIdx.x == 0 && threadIdx.x < H && scale_out)
    scale_out[threadIdx.x] = fmaxf(__uint_as_float(amax_bits[threadIdx.x]) / kFp8Max, 1.17549435e-38f);
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    sat += __shfl_xor(sat, m, 64);
    uf += __shfl_xor(uf, m, 64);
    sq += __shfl_xor(sq, m, 64);
  }
  if ((threadIdx.x & 63) == 0) {
    atomicAdd(counts + 0, sat);
    atomicAdd(counts + 1, uf);
    atomicAdd(sqerr, sq);
  }
}

// ---- scores of one row against key rows ---------------------------------------
// A row's D dimensions are split over LPR = D / 64 lanes (lane l holds
// row l % (64 / LPR), dimensions [l / (64 / LPR) * 64, + 64)), so a lane keeps
// 64 q and 64 output values and D = 128 runs more than one wave per SIMD.
// Each lane's partial dot product is a chain in dimension order; the LPR
// partials are then added (partner lanes l and l ^ 32 form the same sum).
template <int D>
struct Split {
  static constexpr int LPR = D / 64;     // lanes per row
  static constexpr int DL = D / LPR;     // dimensions per lane
  static constexpr int RPW = 64 / LPR;   // rows per wave
};

template <int DL, int LPR>
__device__ __forceinline__ float row_sum(float acc) {
  // lanes l, l ^ (64 / LPR), ... hold the partials of one row; every one of
  // them forms the same sum (pairwise, commutative at each step)
#pragma unroll
  for (int m = 64 / LPR; m < 64; m <<= 1) acc += __shfl_xor(acc, m, 64);
  return acc;
}

template <int DL, int LPR>
__device__ __forceinline__ float dot_part(const float (&q)[DL], const float* krow, float sm_scale) {
  float acc = 0.0f;
#pragma unroll
  for (int d = 0; d < DL; d += 4) {
    const float4 k4 = *reinterpret_cast<const float4*>(krow + d);
    acc = fmaf(q[d], k4.x, acc);
    acc = fmaf(q[d + 1], k4.y, acc);
    acc = fmaf(q[d + 2], k4.z, acc);
    acc = fmaf(q[d + 3], k4.w, acc);
  }
  return row_sum<DL, LPR>(acc) * sm_scale;
}

// dot_part for four consecutive keys (rows `stride` floats apart): four
// independent chains, each in the order of dot_part.
template <int DL, int LPR>
__device__ __forceinline__ void dot_part4(const float (&q)[DL], const float* krow, int64_t stride, float sm_scale,
                                          float (&s)[4]) {
  float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int d = 0; d < DL; d += 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 k4 = *reinterpret_cast<const float4*>(krow + i * stride + d);
      a[i] = fmaf(q[d], k4.x, a[i]);
      a[i] = fmaf(q[d + 1], k4.y, a[i]);
      a[i] = fmaf(q[d + 2], k4.z, a[i]);
      a[i] = fmaf(q[d + 3], k4.w, a[i]);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s[i] = row_sum<DL, LPR>(a[i]) * sm_scale;
  }
}

// Pass 1: per row the final max; per (tile, key block) the max over the tile's
// rows of bmax_j - rm_j and of bmax_j.  A workgroup is one 128-row query tile
// (128 / (64 / LPR) waves); 32-key slices of K are staged in LDS, double
// buffered, and every wave reads its key rows from there (the two lane
// halves of a D = 128 wave read two addresses: broadcast reads).
constexpr int kScanKeys = 32;  // keys per staged slice

template <int D>
__global__ void __launch_bounds__(256) scan_kernel(const float* q, const float* k, int64_t S, int64_t H,
                                                   float sm_scale, float* final_max, uint32_t* tile_margin,
                                                   uint32_t* tile_bmax) {
  using SP = Split<D>;
  constexpr int DL = SP::DL, NWV = kTileQ / SP::RPW, NT = 64 * NWV;
  constexpr int F4 = kScanKeys * D / 4 / NT;  // float4 per thread per slice
  __shared__ __align__(16) float ks[2][kScanKeys * D];
  const int64_t h = blockIdx.y;
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int r = lane % SP::RPW, part = lane / SP::RPW;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kTileQ + wave * SP::RPW + r;
  const int64_t nb = S / kTileQ, mt = blockIdx.x;
  float qr[DL];
#pragma unroll
  for (int d = 0; d < DL; d += 4) {
    const float4 v = *reinterpret_cast<const float4*>(q + (row * H + h) * D + part * DL + d);
    qr[d] = v.x; qr[d + 1] = v.y; qr[d + 2] = v.z; qr[d + 3] = v.w;
  }
  // slice n covers keys [32 n, 32 n + 32); thread chunk i is float4 (tid + NT i)
  // of the slice, key (tid + NT i) / (D / 4)
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  f32x4 kreg[F4];
  const int64_t nslice = S / kScanKeys;
#pragma unroll
  for (int i = 0; i < F4; ++i) {
    const int c = threadIdx.x + NT * i, kk = c / (D / 4), c4 = c % (D / 4);
    kreg[i] = *reinterpret_cast<const f32x4*>(k + (static_cast<int64_t>(kk) * H + h) * D + 4 * c4);
  }
#pragma unroll
  for (int i = 0; i < F4; ++i) *reinterpret_cast<f32x4*>(&ks[0][4 * (threadIdx.x + NT * i)]) = kreg[i];
  __syncthreads();
  float rm = -INFINITY, bmax = -INFINITY;
  for (int64_t n = 0; n < nslice; ++n) {
    {  // slice n + 1 (slice n again after the last), in flight during slice n
      const int64_t key0 = (n + 1 < nslice ? n + 1 : n) * kScanKeys;
#pragma unroll
      for (int i = 0; i < F4; ++i) {
        const int c = threadIdx.x + NT * i, kk = c / (D / 4), c4 = c % (D / 4);
        kreg[i] = *reinterpret_cast<const f32x4*>(k + ((key0 + kk) * H + h) * D + 4 * c4);
      }
    }
    const float* kb = &ks[n & 1][part * DL];
    for (int kk = 0; kk < kScanKeys; kk += 4) {
      float s4[4];
      dot_part4<DL, SP::LPR>(qr, kb + kk * D, D, sm_scale, s4);
#pragma unroll
      for (int i = 0; i < 4; ++i) bmax = fmaxf(bmax, s4[i]);
    }
    if ((n + 1) % (kTileQ / kScanKeys) == 0) {  // the end of key block j
      const int64_t j = n / (kTileQ / kScanKeys);
      rm = fmaxf(rm, bmax);
      const float tm = wave_max(bmax - rm), tb = wave_max(bmax);
      if (lane == 0) {
        const int64_t o = (h * (S / kTileQ) + mt) * nb + j;
        atomicMax(tile_margin + o, ordered_bits(tm));
        atomicMax(tile_bmax + o, ordered_bits(tb));
      }
      bmax = -INFINITY;
    }
    // into the buffer every wave finished reading a slice ago (unread after the last)
#pragma unroll
    for (int i = 0; i < F4; ++i) *reinterpret_cast<f32x4*>(&ks[(n + 1) & 1][4 * (threadIdx.x + NT * i)]) = kreg[i];
    __syncthreads();
  }
  if (part == 0) final_max[h * S + row] = rm;
}

// Tile keep masks for T thresholds, with the empty-tile safeguard.
__global__ void __launch_bounds__(256) keep_kernel(const uint32_t* tile_margin, const uint32_t* tile_bmax,
                                                   int64_t HM, int64_t nb, const float* log_thr, int T,
                                                   uint8_t* keep, unsigned long long* counts) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= HM * T) return;
  const int t = static_cast<int>(i / HM);
  const int64_t hm = i - static_cast<int64_t>(t) * HM;
  const float lt = log_thr[t];
  uint8_t* kp = keep + i * nb;
  const uint32_t* mp = tile_margin + hm * nb;
  const uint32_t* bp = tile_bmax + hm * nb;
  int64_t kept = 0, best = 0;
  float bestv = -INFINITY;
  for (int64_t j = 0; j < nb; ++j) {
    const bool kj = from_ordered_bits(mp[j]) >= lt;
    kp[j] = kj ? 1 : 0;
    kept += kj ? 1 : 0;
    const float bv = from_ordered_bits(bp[j]);
    if (bv > bestv) { bestv = bv; best = j; }
  }
  unsigned long long forced = 0;
  if (kept == 0) {
    kp[best] = 1;
    kept = 1;
    forced = 1;
  }
  atomicAdd(counts + 2 * t, static_cast<unsigned long long>(nb - kept));
  if (forced) atomicAdd(counts + 2 * t + 1, forced);
}

// Pass 2: one rung (exact / online / static P with a tile keep mask).
template <int D, int MODE>
__global__ void __launch_bounds__(64) attend_kernel(const float* q, const float* k, const float* v, int64_t S,
                                                    int64_t H, float sm_scale, int round_p, const float* final_max,
                                                    const uint8_t* keep, float* out, float* dropped,
                                                    unsigned long long* p_counts, double* p_sqerr) {
  using SP = Split<D>;
  constexpr int DL = SP::DL, RPW = SP::RPW;
  // the block's scores of the wave's rows (column r), formed in the block-max
  // pass and read back by the lanes of the same row in the accumulation pass
  __shared__ float sc[MODE != 0 ? kTileQ * RPW : 1];
  const int64_t h = blockIdx.y;
  const int r = threadIdx.x % RPW, part = threadIdx.x / RPW;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * RPW + r;
  const int64_t nb = S / kTileQ, mt = row / kTileQ;
  const int64_t dofs = part * DL;  // this lane's dimensions of q, v and the output row
  float qr[DL], acc[DL];
#pragma unroll
  for (int d = 0; d < DL; d += 4) {
    const float4 x = *reinterpret_cast<const float4*>(q + (row * H + h) * D + dofs + d);
    qr[d] = x.x; qr[d + 1] = x.y; qr[d + 2] = x.z; qr[d + 3] = x.w;
    acc[d] = acc[d + 1] = acc[d + 2] = acc[d + 3] = 0.0f;
  }
  const float fm = final_max[h * S + row];
  const uint8_t* kr = keep ? keep + (h * (S / kTileQ) + mt) * nb : nullptr;
  float den = 0.0f, tot_l = 0.0f, drop_l = 0.0f, rm = -INFINITY;
  unsigned long long uf = 0, cnt = 0;
  double sq = 0.0;
  for (int64_t j = 0; j < nb; ++j) {
    const bool kj = kr ? kr[j] != 0 : true;
    float rescale = 1.0f;
    if (MODE != 0) {
      float bmax = -INFINITY;
      for (int kk = 0; kk < kTileQ; kk += 4) {
        const int64_t key = j * kTileQ + kk;
        float s4[4];
        dot_part4<DL, SP::LPR>(qr, k + (key * H + h) * D + dofs, H * D, sm_scale, s4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          sc[(kk + i) * RPW + r] = s4[i];  // the LPR lanes of a row store the same value
          bmax = fmaxf(bmax, s4[i]);
        }
      }
      rm = fmaxf(rm, bmax);
      rescale = expf(rm - fm);
    }
    // a skipped block adds nothing; its unquantised mass is still needed for
    // the dropped-mass diagnostic and the P statistics cover all blocks
    if (!kj && !dropped && !p_counts) continue;
    float lb = 0.0f;
    for (int kk = 0; kk < kTileQ; ++kk) {
      const int64_t key = j * kTileQ + kk;
      const float s =
          MODE != 0 ? sc[kk * RPW + r] : dot_part<DL, SP::LPR>(qr, k + (key * H + h) * D + dofs, sm_scale);
      float pw;
      if (MODE == 0) {
        const float p = expf(s - fm);
        den += p;
        pw = p;
      } else {
        const float on = expf(s - rm);
        const float w = on * rescale;
        if (MODE == 1) {
          den += w;
          pw = w;
        } else {
          lb += w;
          const float scaled = on * 256.0f;
          const float pq = e4m3_decode(e4m3_encode(scaled)) * (1.0f / 256.0f);
          if (p_counts && part == 0) {  // once per row
            uf += (pq == 0.0f && scaled != 0.0f) ? 1ull : 0ull;
            cnt += 1;
            const double e = static_cast<double>(pq) - static_cast<double>(on);
            sq += e * e;
          }
          pw = pq * rescale;
        }
      }
      if (!kj) continue;
      if (round_p) pw = round_bf16(pw);
      const float* vrow = v + (key * H + h) * D + dofs;
#pragma unroll
      for (int d = 0; d < DL; d += 4) {
        const float4 v4 = *reinterpret_cast<const float4*>(vrow + d);
        acc[d] = fmaf(pw, v4.x, acc[d]);
        acc[d + 1] = fmaf(pw, v4.y, acc[d + 1]);
        acc[d + 2] = fmaf(pw, v4.z, acc[d + 2]);
        acc[d + 3] = fmaf(pw, v4.w, acc[d + 3]);
      }
    }
    if (MODE == 2) {
      if (kj) den += lb;
      tot_l += lb;
      if (!kj) drop_l += lb;
    }
  }
  const float dn = MODE == 2 ? fmaxf(den, kDenomFloor) : den;
  float* orow = out + (row * H + h) * D + dofs;
#pragma unroll
  for (int d = 0; d < DL; d += 4) {
    float4 o;
    o.x = acc[d] / dn; o.y = acc[d + 1] / dn; o.z = acc[d + 2] / dn; o.w = acc[d + 3] / dn;
    *reinterpret_cast<float4*>(orow + d) = o;
  }
  if (MODE == 2 && dropped && part == 0) dropped[h * S + row] = drop_l / fmaxf(tot_l, kDenomFloor);
  if (MODE == 2 && p_counts) {
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
      uf += __shfl_xor(uf, m, 64);
      cnt += __shfl_xor(cnt, m, 64);
      sq += __shfl_xor(sq, m, 64);
    }
    if (threadIdx.x == 0) {
      atomicAdd(p_counts + 0, uf);
      atomicAdd(p_counts + 1, cnt);
      atomicAdd(p_sqerr, sq);
    }
  }
}

__global__ void fill_kernel(uint32_t* p, int64_t n, uint32_t v) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) p[i] = v;
}

}  // namespace

extern "C" int lbfq_head_fp8_quant(const void* x, int dtype, int64_t S, int64_t H, int64_t D, float* deq,
                                   float* deq_mm, int mm_bf16, float* scale, uint32_t* amax_ws,
                                   int64_t* counts, double* sqerr, lbfq_stream_t stream) {
  LBFQ_CHECK_ARG(x && amax_ws && counts && sqerr, "head_fp8_quant: null pointer");
  LBFQ_CHECK_ARG(dtype == kF32 || dtype == kF16 || dtype == kBF16, "head_fp8_quant: unsupported dtype %d", dtype);
  LBFQ_CHECK_ARG(S > 0 && H > 0 && D > 0 && H <= 256, "head_fp8_quant: bad shape");
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(fill_kernel, dim3(static_cast<unsigned>((H + 255) / 256)), dim3(256), 0, st, amax_ws, H, 0u);
  const unsigned gx = static_cast<unsigned>(std::min<int64_t>((S * D + 255) / 256, 1024));
  const int64_t n = S * H * D;
  const unsigned gq = static_cast<unsigned>(std::min<int64_t>((n + 255) / 256, 8192));
  auto* cnt = reinterpret_cast<unsigned long long*>(counts);
#define LBFQ_HQ(DT)                                                                                            \
  do {                                                                                                         \
    hipLaunchKernelGGL(head_amax_kernel<DT>, dim3(gx, static_cast<unsigned>(H)), dim3(256), 0, st, x, S, H, D, \
                       amax_ws);                                                                               \
    hipLaunchKernelGGL(head_quant_kernel<DT>, dim3(gq), dim3(256), 0, st, x, n, H, D, amax_ws, deq, deq_mm,    \
                       mm_bf16, scale, cnt, sqerr);                                                            \
  } while (0)
  if (dtype == kF32) LBFQ_HQ(kF32);
  else if (dtype == kF16) LBFQ_HQ(kF16);
  else LBFQ_HQ(kBF16);
#undef LBFQ_HQ
  LBFQ_LAUNCH_CHECK("head_fp8_quant");
  return 0;
}

extern "C" int lbfq_blasst_scan(const float* q, const float* k, int64_t S, int64_t H, int64_t D, float sm_scale,
                                float* final_max, uint32_t* tile_margin, uint32_t* tile_bmax,
                                lbfq_stream_t stream) {
  LBFQ_CHECK_ARG(q && k && final_max && tile_margin && tile_bmax, "blasst_scan: null pointer");
  LBFQ_CHECK_ARG(D == 64 || D == 128, "blasst_scan: D must be 64 or 128");
  LBFQ_CHECK_ARG(S > 0 && S % kTileQ == 0, "blasst_scan: S must be a positive multiple of %d", kTileQ);
  LBFQ_CHECK_ARG(H > 0 && H < 65536, "blasst_scan: bad H");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t nt = H * (S / kTileQ) * (S / kTileQ);
  const uint32_t neg_inf = 0x007fffffu;  // ordered bits of -inf
  hipLaunchKernelGGL(fill_kernel, dim3(static_cast<unsigned>((nt + 255) / 256)), dim3(256), 0, st, tile_margin, nt,
                     neg_inf);
  hipLaunchKernelGGL(fill_kernel, dim3(static_cast<unsigned>((nt + 255) / 256)), dim3(256), 0, st, tile_bmax, nt,
                     neg_inf);
  if (D == 128)
    hipLaunchKernelGGL(scan_kernel<128>, dim3(static_cast<unsigned>(S / kTileQ), static_cast<unsigned>(H)),
                       dim3(64 * kTileQ / Split<128>::RPW), 0, st, q, k, S, H, sm_scale, final_max, tile_margin,
                       tile_bmax);
  else
    hipLaunchKernelGGL(scan_kernel<64>, dim3(static_cast<unsigned>(S / kTileQ), static_cast<unsigned>(H)),
                       dim3(64 * kTileQ / Split<64>::RPW), 0, st, q, k, S, H, sm_scale, final_max, tile_margin,
                       tile_bmax);
  LBFQ_LAUNCH_CHECK("blasst_scan");
  return 0;
}

extern "C" int lbfq_blasst_keep(const uint32_t* tile_margin, const uint32_t* tile_bmax, int64_t H, int64_t S,
                                const float* log_thresholds, int T, uint8_t* keep, int64_t* counts,
                                lbfq_stream_t stream) {
  LBFQ_CHECK_ARG(tile_margin && tile_bmax && log_thresholds && keep && counts, "blasst_keep: null pointer");
  LBFQ_CHECK_ARG(T > 0 && S > 0 && S % kTileQ == 0 && H > 0, "blasst_keep: bad shape");
  const int64_t hm = H * (S / kTileQ), nb = S / kTileQ;
  const int64_t n = hm * T;
  hipLaunchKernelGGL(keep_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), tile_margin, tile_bmax, hm, nb, log_thresholds, T, keep,
                     reinterpret_cast<unsigned long long*>(counts));
  LBFQ_LAUNCH_CHECK("blasst_keep");
  return 0;
}

extern "C" int lbfq_blasst_attend(const lbfq_blasst_attend_params* p, lbfq_stream_t stream) {
  LBFQ_CHECK_ARG(p && p->q && p->k && p->v && p->final_max && p->out, "blasst_attend: null pointer");
  LBFQ_CHECK_ARG(p->D == 64 || p->D == 128, "blasst_attend: D must be 64 or 128");
  LBFQ_CHECK_ARG(p->S > 0 && p->S % kTileQ == 0, "blasst_attend: S must be a positive multiple of %d", kTileQ);
  LBFQ_CHECK_ARG(p->mode >= 0 && p->mode <= 2, "blasst_attend: mode must be 0, 1 or 2");
  LBFQ_CHECK_ARG(p->mode == 2 || (!p->keep && !p->dropped && !p->p_counts),
                 "blasst_attend: keep masks, dropped mass and P statistics need mode 2");
  LBFQ_CHECK_ARG(!p->p_counts || p->p_sqerr, "blasst_attend: p_counts needs p_sqerr");
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto* pc = reinterpret_cast<unsigned long long*>(p->p_counts);
#define LBFQ_ATT(DD, MM)                                                                                          \
  hipLaunchKernelGGL((attend_kernel<DD, MM>), dim3(static_cast<unsigned>(p->S / Split<DD>::RPW),                 \
                     static_cast<unsigned>(p->H)), dim3(64), 0, st, p->q, p->k, p->v, p->S, p->H, p->sm_scale, \
                     p->round_p_bf16, p->final_max, p->keep, p->out, p->dropped, pc, p->p_sqerr)
  if (p->D == 128) {
    if (p->mode == 0) LBFQ_ATT(128, 0);
    else if (p->mode == 1) LBFQ_ATT(128, 1);
    else LBFQ_ATT(128, 2);
  } else {
    if (p->mode == 0) LBFQ_ATT(64, 0);
    else if (p->mode == 1) LBFQ_ATT(64, 1);
    else LBFQ_ATT(64, 2);
  }
#undef LBFQ_ATT
  LBFQ_LAUNCH_CHECK("blasst_attend");
  return 0;
}
