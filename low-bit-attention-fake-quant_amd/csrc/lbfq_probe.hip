// Diagnostic kernels beside the attention path (gfx950).
//
// * p_requant_rows: materialised FP8 P of small score matrices, with row sums
//   and log-sum-exp (the reference probe p_requant.py:12-73).
// * rowmax_count: row-max update / rescale counters of the K loop under the
//   FA4-style online rule or the qm_k estimate with up/down thresholds (the
//   reference diagnostic bench/count_rowmax_updates_triton.py:27-171), over
//   the FP8 codes and qm correction table the attention kernel consumes.
// * hbm_stream: read-only / write-only / copy streams of 16-byte words, the
//   measured HBM ceiling the prepass is held against (no reference
//   counterpart).
// * issue_probe: cycles per wave-instruction of the instruction classes the
//   attention step is made of, and of the step's inherent per-tile mix, at a
//   given number of waves per SIMD (no reference counterpart: it measures the
//   floor the attention kernel is held against).
#include "lbfq_common.h"
#include "../../include/lbfq.h"

using namespace lbfq;

namespace {

constexpr int kRowThreads = 256;

__device__ __forceinline__ float block_reduce_max(float v, float* red) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  const int wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < kRowThreads / 64; ++w) r = fmaxf(r, red[w]);
  return r;
}

__device__ __forceinline__ float block_reduce_sum(float v, float* red) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v += __shfl_xor(v, m, 64);
  const int wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < kRowThreads / 64; ++w) r += red[w];
  return r;
}

// One workgroup per row (b, m): row max, then p = 2^((x - max) * c + offset)
// stored as E4M3 (round to nearest even, saturating at 448), its fp32 sum and
// lse = max * sm_scale + ln(sum) - offset * ln 2.
template <int DT>
__global__ void __launch_bounds__(kRowThreads) p_requant_rows_kernel(
    const void* scores, int64_t M, int64_t N, int64_t ssb, int64_t ssm, int64_t ssn, uint8_t* p, int64_t psb,
    int64_t psm, int64_t psn, float* row_sum, float* lse, float c, float sm_scale, float offset, float off_ln2) {
  __shared__ float red[kRowThreads / 64];
  const int64_t row = blockIdx.x;
  const int64_t b = row / M, m = row - b * M;
  const int64_t sbase = b * ssb + m * ssm, pbase = b * psb + m * psm;
  float mx = -INFINITY;
  for (int64_t n = threadIdx.x; n < N; n += kRowThreads) mx = fmaxf(mx, load_as_f32(scores, sbase + n * ssn, DT));
  mx = block_reduce_max(mx, red);
  float sum = 0.0f;
  for (int64_t n = threadIdx.x; n < N; n += kRowThreads) {
    const float z = fmaf(load_as_f32(scores, sbase + n * ssn, DT) - mx, c, offset);
    const float pv = exp2f(z);
    p[pbase + n * psn] = e4m3_encode(pv);
    sum += pv;
  }
  sum = block_reduce_sum(sum, red);
  if (threadIdx.x == 0) {
    row_sum[row] = sum;
    lse[row] = fmaf(mx, sm_scale, logf(sum)) - off_ln2;
  }
}

// ---- row-max update counters --------------------------------------------------
typedef int v8i_t __attribute__((ext_vector_type(8)));
typedef float v16f_t __attribute__((ext_vector_type(16)));

struct CountArgs {
  int S, P, H, G, lg_qgroup, lg_qkblk, nqkblk;
  float sml2;           // sm_scale * log2(e)
  float up, down;       // thresholds, log2 units
  float floor_shift;    // 80 * log2(e): the reference's m - 80 bound in log2 units
  float mass_floor;
  int down_always;
  const uint8_t* q_codes;
  const uint8_t* k_codes;
  const float* q_scale;
  const float* k_scale;
  const float* bias;    // (B,H,G,P) log2 units or null
  const float* rowmax;  // (B,H,G) log2 units (estimate mode)
  unsigned long long* counters;
};

__device__ __forceinline__ v8i_t load_operand(const uint8_t* row, int hh, int g) {
  const uint4 x = *reinterpret_cast<const uint4*>(row + 64 * hh + 16 * g);
  const uint4 y = *reinterpret_cast<const uint4*>(row + 64 * hh + 32 + 16 * g);
  v8i_t r;
  r[0] = x.x; r[1] = x.y; r[2] = x.z; r[3] = x.w;
  r[4] = y.x; r[5] = y.y; r[6] = y.z; r[7] = y.w;
  return r;
}

// One wave = 32 query rows of one (b, h); lane l holds row l % 32 and, for the
// 64-key tile, the keys 32 t + 8 (r / 4) + 4 (l / 32) + r % 4 (t in {0, 1},
// r in 0..15) of S^T = K Q^T on the FP8 matrix cores.  Scores in log2 units:
// u = (q . k) * sq * sk * sm_scale * log2(e) + bias.  Per tile and row the
// update rule of the reference diagnostic is applied (thresholds in log2
// units), the tile's p = 2^(u - m) summed into l, and per-row counts kept;
// lanes of the first half add them into the six 64-bit counters.  A
// workgroup is four waves (128 rows) sharing each K tile through LDS.
template <int D, bool EST>
__global__ void __launch_bounds__(256) rowmax_count_kernel(const CountArgs a) {
  constexpr int NH = D / 64;
  // K tiles (64 keys) staged in LDS and shared by the four waves, double
  // buffered; rows padded by 16 bytes so that the 32 rows one operand read
  // touches fall on distinct banks
  constexpr int KP = D + 16, CPR = D / 16, CPT = 64 * CPR / 256;
  __shared__ __align__(16) uint8_t kl[2][64 * KP];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int li = lane & 31, g = lane >> 5;
  const int bh = blockIdx.y;
  const int q0 = blockIdx.x * 128 + wave * 32;
  // every wave stages tiles and meets the barriers; a wave past the rows
  // (q0 >= S) reads row S - 1 and counts nothing
  const int qi = q0 + li;
  const bool qvalid = qi < a.S;
  const int qr = qvalid ? qi : a.S - 1;
  const uint8_t* qrow = a.q_codes + (static_cast<size_t>(bh) * a.P + qr) * D;
  v8i_t qop[NH];
#pragma unroll
  for (int hh = 0; hh < NH; ++hh) qop[hh] = load_operand(qrow, hh, g);
  const float qC = a.sml2 * a.q_scale[bh * a.nqkblk + (qr >> a.lg_qkblk)];
  int grp = qr >> a.lg_qgroup;  // qm group of this lane's row
  if (grp >= a.G) grp = a.G - 1;
  const float* brow = a.bias ? a.bias + (static_cast<size_t>(bh) * a.G + grp) * a.P : nullptr;
  const uint8_t* kbase = a.k_codes + static_cast<size_t>(bh) * a.P * D;

  float m = EST ? a.rowmax[bh * a.G + grp] : -INFINITY;
  float l = 0.0f, max_seen = -INFINITY;
  int updates = 0, rescales = 0, upward = 0, downward = 0;
  const int nt = (a.S + 63) / 64;  // tile rows stay below the pitch (a multiple of 128 >= S)
  // thread chunk i: row (tid + 256 i) / CPR, 16-byte column (tid + 256 i) % CPR
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  u32x4 kreg[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = threadIdx.x + 256 * i;
    kreg[i] = *reinterpret_cast<const u32x4*>(kbase + static_cast<size_t>(c / CPR) * D + 16 * (c % CPR));
  }
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = threadIdx.x + 256 * i;
    *reinterpret_cast<u32x4*>(&kl[0][(c / CPR) * KP + 16 * (c % CPR)]) = kreg[i];
  }
  __syncthreads();
  for (int it = 0; it < nt; ++it) {
    const int key0 = it * 64;
    {  // the next tile (the last one again after the last), in flight during this one
      const int knext = it + 1 < nt ? key0 + 64 : key0;
#pragma unroll
      for (int i = 0; i < CPT; ++i) {
        const int c = threadIdx.x + 256 * i;
        kreg[i] = *reinterpret_cast<const u32x4*>(kbase + static_cast<size_t>(knext + c / CPR) * D + 16 * (c % CPR));
      }
    }
    float u[2][16];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      v16f_t c;
#pragma unroll
      for (int r = 0; r < 16; ++r) c[r] = 0.0f;
      const uint8_t* krow = &kl[it & 1][(32 * t + li) * KP];
#pragma unroll
      for (int hh = 0; hh < NH; ++hh)
        c = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(load_operand(krow, hh, g), qop[hh], c, 0, 0, 0, 0, 0, 0);
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int kk = key0 + 32 * t + 8 * r4 + 4 * g;  // first of 4 consecutive keys
        int kb = kk >> a.lg_qkblk;
        kb = kb < a.nqkblk ? kb : a.nqkblk - 1;
        const float C = qC * a.k_scale[bh * a.nqkblk + kb];
        float4 bb = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (brow) bb = *reinterpret_cast<const float4*>(brow + kk);
        const float bv[4] = {bb.x, bb.y, bb.z, bb.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float s = fmaf(c[4 * r4 + j], C, bv[j]);
          u[t][4 * r4 + j] = (kk + j < a.S) ? s : -INFINITY;
        }
      }
    }
    float bmax = -INFINITY;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) bmax = fmaxf(bmax, u[t][r]);
    bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));

    bool adjust, rescale;
    float m_new, alpha;
    if constexpr (EST) {
      const float seen = fmaxf(max_seen, bmax);
      const bool under = (bmax - m) > a.up;
      bool over = (m - seen) > a.down;
      if (!a.down_always) over = over && (l < a.mass_floor);
      adjust = under || over;
      const float down_bounded = fmaxf(seen + a.down, m - a.floor_shift);
      const float down_m = (l == 0.0f) ? seen : down_bounded;
      m_new = adjust ? (under ? bmax : down_m) : m;
      alpha = adjust ? ((l == 0.0f) ? 0.0f : exp2f(m - m_new)) : 1.0f;
      max_seen = seen;
      rescale = adjust && (l != 0.0f);
      upward += (adjust && under) ? 1 : 0;
      downward += (adjust && !under) ? 1 : 0;
    } else {
      const bool first = m == -INFINITY;
      adjust = first || (bmax - m) > a.up;
      m_new = adjust ? bmax : m;
      alpha = first ? 0.0f : exp2f(m - m_new);
      rescale = adjust && !first;
      upward += adjust ? 1 : 0;
    }
    float ps = 0.0f;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) ps += exp2f(u[t][r] - m_new);
    ps += __shfl_xor(ps, 32, 64);
    l = l * alpha + ps;
    m = m_new;
    updates += adjust ? 1 : 0;
    rescales += rescale ? 1 : 0;
    // into the buffer every wave finished reading a tile ago (unread after the last tile)
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = threadIdx.x + 256 * i;
      *reinterpret_cast<u32x4*>(&kl[(it + 1) & 1][(c / CPR) * KP + 16 * (c % CPR)]) = kreg[i];
    }
    __syncthreads();
  }
  // rows of this wave: lanes 0..31 (the second half holds the same rows)
  const bool counted = qvalid && g == 0;
  unsigned long long v[6] = {counted ? (unsigned long long)updates : 0ull,
                             counted ? (unsigned long long)rescales : 0ull,
                             counted ? (unsigned long long)upward : 0ull,
                             counted ? (unsigned long long)downward : 0ull,
                             (counted && updates > 0) ? 1ull : 0ull,
                             counted ? (unsigned long long)updates : 0ull};
#pragma unroll
  for (int msk = 1; msk < 64; msk <<= 1) {
#pragma unroll
    for (int i = 0; i < 5; ++i) v[i] += __shfl_xor(v[i], msk, 64);
    const unsigned long long o = __shfl_xor(v[5], msk, 64);
    v[5] = o > v[5] ? o : v[5];
  }
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < 5; ++i) atomicAdd(a.counters + i, v[i]);
    atomicMax(a.counters + 5, v[5]);
  }
}

// HBM streaming probe: 256 threads, each moving kUnroll 16-byte words per
// chunk of 256 * kUnroll words (a wave touches 1 KiB contiguous per load);
// chunks are dealt out grid-stride.  MODE 0 reads and folds the words into
// one value per thread, stored only when it equals a constant (so the loads
// are live but nothing is written); MODE 1 writes; MODE 2 copies.
constexpr int kStreamThreads = 256;
constexpr int kStreamUnroll = 4;

template <int MODE>
__global__ void __launch_bounds__(kStreamThreads) hbm_stream_kernel(const uint4* __restrict__ src,
                                                                    uint4* __restrict__ dst, int64_t n16,
                                                                    uint32_t* sink) {
  constexpr int64_t kChunk = kStreamThreads * kStreamUnroll;
  const int64_t nchunk = (n16 + kChunk - 1) / kChunk;
  uint32_t acc = 0;
  for (int64_t c = blockIdx.x; c < nchunk; c += gridDim.x) {
    const int64_t base = c * kChunk + threadIdx.x;
    uint4 v[kStreamUnroll];
    if (base + kStreamThreads * (kStreamUnroll - 1) < n16) {
      if constexpr (MODE != 1) {
#pragma unroll
        for (int u = 0; u < kStreamUnroll; ++u) v[u] = src[base + kStreamThreads * u];
      }
#pragma unroll
      for (int u = 0; u < kStreamUnroll; ++u) {
        const int64_t i = base + kStreamThreads * u;
        if constexpr (MODE == 0) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
        if constexpr (MODE == 1) dst[i] = make_uint4(static_cast<uint32_t>(i), 0u, 0u, 0u);
        if constexpr (MODE == 2) dst[i] = v[u];
      }
    } else {
#pragma unroll
      for (int u = 0; u < kStreamUnroll; ++u) {
        const int64_t i = base + kStreamThreads * u;
        if (i < n16) {
          if constexpr (MODE == 0) {
            const uint4 w = src[i];
            acc ^= w.x ^ w.y ^ w.z ^ w.w;
          }
          if constexpr (MODE == 1) dst[i] = make_uint4(static_cast<uint32_t>(i), 0u, 0u, 0u);
          if constexpr (MODE == 2) dst[i] = src[i];
        }
      }
    }
  }
  if constexpr (MODE == 0) {
    if (acc == 0x9e3779b9u) sink[threadIdx.x] = acc;
  }
}

// Issue-cost probe.  One workgroup of 4 * W waves runs on one CU, so each of
// its four SIMDs holds W waves; every wave runs `iters` iterations of a loop
// body of independent instructions (16 chains of one class, or the tile mix
// below) between two s_memtime reads and records (start, end, SIMD id).  The
// host takes, per SIMD, (latest end - earliest start) / (waves x iterations x
// instructions per iteration): the SIMD's cost per wave-instruction.  The
// VALU chains never touch the MFMA accumulators, so no operand of an
// in-flight MFMA is read.
typedef int v8i_t __attribute__((ext_vector_type(8)));
typedef float v16f_t __attribute__((ext_vector_type(16)));

#define LBFQ_P_MUL(i) asm volatile("v_mul_f32 %0, %0, %1" : "+v"(x[(i) & 31]) : "v"(c));
#define LBFQ_P_ADD(i) asm volatile("v_add_f32 %0, %0, %1" : "+v"(x[(i) & 31]) : "v"(c));
#define LBFQ_P_FMA(i) asm volatile("v_fma_f32 %0, %0, %1, %1" : "+v"(x[(i) & 31]) : "v"(c));
#define LBFQ_P_MAX3(i) asm volatile("v_max3_f32 %0, %0, %1, %0" : "+v"(x[(i) & 31]) : "v"(c));
#define LBFQ_P_MAX(i) asm volatile("v_max_f32 %0, %0, %1" : "+v"(x[(i) & 31]) : "v"(c));
#define LBFQ_P_EXP(i) asm volatile("v_exp_f32 %0, %0" : "+v"(x[(i) & 31]));
#define LBFQ_P_CVT(i) asm volatile("v_cvt_pk_fp8_f32 %0, %0, %1" : "+v"(x[(i) & 31]) : "v"(c));
#define LBFQ_P_PERM(i) asm volatile("v_permlane32_swap_b32 %0, %1" : "+v"(x[(i) & 31]), "+v"(x[((i) + 1) & 31]));

// OP: 0 mul, 1 add, 2 fma, 3 max3, 4 exp, 5 cvt_pk_fp8, 6 permlane32_swap (16
// per iteration); 7 FP8 MFMA 32x32x64 (8 per iteration, four accumulator
// chains); 8 the attention step's inherent per-tile mix: 8 MFMAs, 32 fma,
// 16 max3 + 3 max, 34 exp, 16 cvt, 32 add, 64 mul, 1 permlane (the work of
// one wave on a 32-query x 64-key tile, dynamic P); 9 its VALU part alone.
template <int OP>
__global__ void __launch_bounds__(512) issue_probe_kernel(float* sink, int iters, long long* rec) {
  float x[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) x[i] = threadIdx.x * 0.001f + i;
  const float c = 1.0000001f;
  v8i_t a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) { a[i] = 0x38383838 + static_cast<int>(threadIdx.x); b[i] = 0x38383838; }
  v16f_t acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;
  unsigned hw;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
  __syncthreads();
  const long long t0 = clock64();
  for (int it = 0; it < iters; ++it) {
    if constexpr (OP <= 6) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if constexpr (OP == 0) LBFQ_P_MUL(i)
        if constexpr (OP == 1) LBFQ_P_ADD(i)
        if constexpr (OP == 2) LBFQ_P_FMA(i)
        if constexpr (OP == 3) LBFQ_P_MAX3(i)
        if constexpr (OP == 4) LBFQ_P_EXP(i)
        if constexpr (OP == 5) LBFQ_P_CVT(i)
        if constexpr (OP == 6) LBFQ_P_PERM(2 * i)
      }
    } else {
#pragma unroll
      for (int g = 0; g < 8; ++g) {
        if constexpr (OP == 7 || OP == 8)
          acc[g & 3] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, acc[g & 3], 0, 0, 0, 127, 0, 127);
        if constexpr (OP == 8 || OP == 9) {
          const int o = 4 * g;
          LBFQ_P_FMA(o) LBFQ_P_FMA(o + 1) LBFQ_P_FMA(o + 2) LBFQ_P_FMA(o + 3)
          LBFQ_P_MAX3(o) LBFQ_P_MAX3(o + 1)
          LBFQ_P_EXP(o) LBFQ_P_EXP(o + 1) LBFQ_P_EXP(o + 2) LBFQ_P_EXP(o + 3)
          LBFQ_P_CVT(o) LBFQ_P_CVT(o + 1)
          LBFQ_P_ADD(o) LBFQ_P_ADD(o + 1) LBFQ_P_ADD(o + 2) LBFQ_P_ADD(o + 3)
          LBFQ_P_MUL(o) LBFQ_P_MUL(o + 1) LBFQ_P_MUL(o + 2) LBFQ_P_MUL(o + 3)
          LBFQ_P_MUL(o + 4) LBFQ_P_MUL(o + 5) LBFQ_P_MUL(o + 6) LBFQ_P_MUL(o + 7)
        }
      }
      if constexpr (OP == 8 || OP == 9) {
        LBFQ_P_EXP(1) LBFQ_P_EXP(2) LBFQ_P_MAX(3) LBFQ_P_MAX(4) LBFQ_P_MAX(5) LBFQ_P_PERM(6)
      }
    }
  }
  const long long t1 = clock64();
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 32; ++i) s += x[i];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) s += acc[j][r];
  sink[threadIdx.x] = s;
  if ((threadIdx.x & 63) == 0) {
    const int w = threadIdx.x >> 6;
    rec[3 * w] = t0;
    rec[3 * w + 1] = t1;
    rec[3 * w + 2] = (hw >> 4) & 3;  // HW_ID.SIMD_ID
  }
}

#undef LBFQ_P_MUL
#undef LBFQ_P_ADD
#undef LBFQ_P_FMA
#undef LBFQ_P_MAX3
#undef LBFQ_P_MAX
#undef LBFQ_P_EXP
#undef LBFQ_P_CVT
#undef LBFQ_P_PERM

}  // namespace

extern "C" int lbfq_issue_probe(int op, int waves_per_simd, int iters, long long* rec, float* sink,
                                lbfq_stream_t stream) {
  LBFQ_CHECK_ARG(op >= 0 && op <= 9, "lbfq_issue_probe: op must be in [0, 9]");
  LBFQ_CHECK_ARG(waves_per_simd == 1 || waves_per_simd == 2, "lbfq_issue_probe: 1 or 2 waves per SIMD");
  LBFQ_CHECK_ARG(iters > 0 && rec && sink, "lbfq_issue_probe: bad args");
  const dim3 g(1), blk(static_cast<unsigned>(256 * waves_per_simd));
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (op) {
    case 0: hipLaunchKernelGGL(issue_probe_kernel<0>, g, blk, 0, st, sink, iters, rec); break;
    case 1: hipLaunchKernelGGL(issue_probe_kernel<1>, g, blk, 0, st, sink, iters, rec); break;
    case 2: hipLaunchKernelGGL(issue_probe_kernel<2>, g, blk, 0, st, sink, iters, rec); break;
    case 3: hipLaunchKernelGGL(issue_probe_kernel<3>, g, blk, 0, st, sink, iters, rec); break;
    case 4: hipLaunchKernelGGL(issue_probe_kernel<4>, g, blk, 0, st, sink, iters, rec); break;
    case 5: hipLaunchKernelGGL(issue_probe_kernel<5>, g, blk, 0, st, sink, iters, rec); break;
    case 6: hipLaunchKernelGGL(issue_probe_kernel<6>, g, blk, 0, st, sink, iters, rec); break;
    case 7: hipLaunchKernelGGL(issue_probe_kernel<7>, g, blk, 0, st, sink, iters, rec); break;
    case 8: hipLaunchKernelGGL(issue_probe_kernel<8>, g, blk, 0, st, sink, iters, rec); break;
    default: hipLaunchKernelGGL(issue_probe_kernel<9>, g, blk, 0, st, sink, iters, rec); break;
  }
  LBFQ_LAUNCH_CHECK("lbfq_issue_probe");
  return 0;
}

extern "C" int lbfq_hbm_stream(int mode, const void* src, void* dst, int64_t bytes, int grid, uint32_t* sink,
                               lbfq_stream_t stream) {
  LBFQ_CHECK_ARG(mode >= 0 && mode <= 2, "lbfq_hbm_stream: mode must be 0 (read), 1 (write) or 2 (copy)");
  LBFQ_CHECK_ARG(bytes > 0 && bytes % 16 == 0, "lbfq_hbm_stream: bytes must be a positive multiple of 16");
  LBFQ_CHECK_ARG(grid > 0, "lbfq_hbm_stream: grid must be > 0");
  LBFQ_CHECK_ARG(mode == 1 || (src && reinterpret_cast<uintptr_t>(src) % 16 == 0),
                 "lbfq_hbm_stream: src must be 16-byte aligned");
  LBFQ_CHECK_ARG(mode == 0 || (dst && reinterpret_cast<uintptr_t>(dst) % 16 == 0),
                 "lbfq_hbm_stream: dst must be 16-byte aligned");
  LBFQ_CHECK_ARG(mode != 0 || sink, "lbfq_hbm_stream: mode 0 needs a sink of 256 words");
  const int64_t n16 = bytes / 16;
  const dim3 g(static_cast<unsigned>(grid)), blk(kStreamThreads);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint4* s4 = static_cast<const uint4*>(src);
  uint4* d4 = static_cast<uint4*>(dst);
  if (mode == 0) hipLaunchKernelGGL(hbm_stream_kernel<0>, g, blk, 0, st, s4, d4, n16, sink);
  else if (mode == 1) hipLaunchKernelGGL(hbm_stream_kernel<1>, g, blk, 0, st, s4, d4, n16, sink);
  else hipLaunchKernelGGL(hbm_stream_kernel<2>, g, blk, 0, st, s4, d4, n16, sink);
  LBFQ_LAUNCH_CHECK("lbfq_hbm_stream");
  return 0;
}

extern "C" int lbfq_p_requant_rows(const void* scores, int dtype, int64_t B, int64_t M, int64_t N, int64_t ssb,
                                   int64_t ssm, int64_t ssn, uint8_t* p, int64_t psb, int64_t psm, int64_t psn,
                                   float* row_sum, float* lse, double sm_scale, int p_max_offset,
                                   lbfq_stream_t stream) {
  LBFQ_CHECK_ARG(scores && p && row_sum && lse, "p_requant_rows: null pointer");
  LBFQ_CHECK_ARG(dtype == kF32 || dtype == kF16 || dtype == kBF16, "p_requant_rows: unsupported dtype %d", dtype);
  LBFQ_CHECK_ARG(B > 0 && M > 0 && N > 0, "p_requant_rows: empty shape (%lld, %lld, %lld)", (long long)B,
                 (long long)M, (long long)N);
  LBFQ_CHECK_ARG(B * M < (int64_t(1) << 31), "p_requant_rows: too many rows");
  // the reference folds SM_SCALE * LOG2E in double and rounds the constant once
  const double log2e = 1.4426950408889634;
  const float c = static_cast<float>(sm_scale * log2e);
  const float sm = static_cast<float>(sm_scale);
  const float off_ln2 = static_cast<float>(p_max_offset * 0.6931471805599453);
  const dim3 grid(static_cast<unsigned>(B * M)), block(kRowThreads);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const float off = static_cast<float>(p_max_offset);
#define LBFQ_PRR(DT)                                                                                              \
  hipLaunchKernelGGL(p_requant_rows_kernel<DT>, grid, block, 0, st, scores, M, N, ssb, ssm, ssn, p, psb, psm, psn, \
                     row_sum, lse, c, sm, off, off_ln2)
  if (dtype == kF32) LBFQ_PRR(kF32);
  else if (dtype == kF16) LBFQ_PRR(kF16);
  else LBFQ_PRR(kBF16);
#undef LBFQ_PRR
  LBFQ_LAUNCH_CHECK("p_requant_rows");
  return 0;
}

extern "C" int lbfq_rowmax_count(const lbfq_rowmax_count_params* p, lbfq_stream_t stream) {
  LBFQ_CHECK_ARG(p && p->q_codes && p->k_codes && p->q_scale && p->k_scale && p->counters,
                 "rowmax_count: null pointer");
  LBFQ_CHECK_ARG(p->D == 64 || p->D == 128, "rowmax_count: D must be 64 or 128, got %lld", (long long)p->D);
  LBFQ_CHECK_ARG(p->B > 0 && p->H > 0 && p->S > 0, "rowmax_count: empty shape");
  LBFQ_CHECK_ARG(p->s_pitch % 128 == 0 && p->s_pitch >= p->S, "rowmax_count: s_pitch must be a multiple of 128 >= S");
  LBFQ_CHECK_ARG(p->B * p->H * p->s_pitch * p->D < (int64_t(1) << 31) * 64, "rowmax_count: operands too large");
  LBFQ_CHECK_ARG(p->qk_block > 0 && (p->qk_block & (p->qk_block - 1)) == 0 && p->qk_block >= 4,
                 "rowmax_count: qk_block must be a power of two >= 4, got %d", p->qk_block);
  const bool est = p->use_estimate != 0;
  LBFQ_CHECK_ARG(!est || p->rowmax_est, "rowmax_count: the estimate mode needs rowmax_est");
  LBFQ_CHECK_ARG(!(p->bias || p->rowmax_est) ||
                     (p->q_group > 0 && (p->q_group & (p->q_group - 1)) == 0 && p->S % p->q_group == 0),
                 "rowmax_count: q_group must be a power of two dividing S");
  CountArgs a{};
  a.S = static_cast<int>(p->S);
  a.P = static_cast<int>(p->s_pitch);
  a.H = static_cast<int>(p->H);
  const int qg = p->q_group > 0 ? p->q_group : static_cast<int>(p->s_pitch);
  a.G = static_cast<int>((p->S + qg - 1) / qg);
  a.lg_qgroup = __builtin_ctz(static_cast<unsigned>(qg));
  a.lg_qkblk = __builtin_ctz(static_cast<unsigned>(p->qk_block));
  a.nqkblk = static_cast<int>((p->S + p->qk_block - 1) / p->qk_block);
  const double log2e = 1.4426950408889634;
  a.sml2 = static_cast<float>(static_cast<double>(p->sm_scale) * log2e);
  a.up = p->up_threshold_log2;
  a.down = p->down_threshold_log2;
  a.floor_shift = static_cast<float>(80.0 * log2e);
  a.mass_floor = p->mass_floor;
  a.down_always = p->down_always;
  a.q_codes = p->q_codes;
  a.k_codes = p->k_codes;
  a.q_scale = p->q_scale;
  a.k_scale = p->k_scale;
  a.bias = p->bias;
  a.rowmax = p->rowmax_est;
  a.counters = reinterpret_cast<unsigned long long*>(p->counters);
  const dim3 grid(static_cast<unsigned>((p->S + 127) / 128), static_cast<unsigned>(p->B * p->H)), block(256);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (p->D == 128) {
    if (est) hipLaunchKernelGGL((rowmax_count_kernel<128, true>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((rowmax_count_kernel<128, false>), grid, block, 0, st, a);
  } else {
    if (est) hipLaunchKernelGGL((rowmax_count_kernel<64, true>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((rowmax_count_kernel<64, false>), grid, block, 0, st, a);
  }
  LBFQ_LAUNCH_CHECK("rowmax_count");
  return 0;
}
