// FP8-MFMA P-requant attention for gfx950 (CDNA4).
//
// Reference semantics: the K-loop of _fake_quant_attn_fwd_kernel
// (attention_triton.py:109-407) and the guards of fake_quant_attention_triton
// (attention_triton.py:463-624).  The reference dequantises Q/K/V to bf16 and
// runs bf16 dots; this kernel multiplies the FP8 codes on the matrix cores
// (v_mfma[_scale]_f32_32x32x64_f8f6f4) and applies the scales outside.
//
// Work decomposition: one workgroup = 4 waves = 128 queries of one (b, h);
// each wave owns 32 queries.  K and V^T tiles of 64 keys are staged in LDS
// (double buffered) and shared by the 4 waves.  Scores are computed
// transposed, S^T = K Q^T, so every lane owns exactly one query: lane l holds
// query l % 32 and, in lane group g = l / 32, the 32 keys 32t + 16g + r
// (t in {0,1}, r in 0..15) of the tile.  K rows are permuted in LDS so that
// the MFMA accumulator layout yields that key order; the same 32 keys then
// form the lane's B operand of the PV product O^T = V^T P^T without any
// data movement.  Row statistics are in-lane reductions plus one exchange
// with lane l ^ 32.
//
// Operand K-index layout of v_mfma[_scale]_f32_32x32x64_f8f6f4 (measured):
// lane l supplies row/column l % 32; lane group g = l / 32 holds the 32
// K-elements 16g + [0,16) (bytes 0..15) and 32 + 16g + [0,16) (bytes
// 16..31); the E8M0 scale of K-block b (k in [32b, 32b+32)) comes from lane
// (l % 32) + 32b.  MX scale blocks along D therefore align with 64-wide
// contraction halves loaded as two 16-byte pieces, and in PV the tile's key
// index equals the hardware K index.
//
// Per-query FP32 factors of the accumulator (online-softmax alpha, dynamic P
// scale, fp8_block V scale) are folded into one rescale of O^T per tile,
// skipped when the whole wave has factor 1 (the common qm_k case).
#include "lbfq_common.h"
#include "../../include/lbfq.h"

using namespace lbfq;

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kWaves = 4;
constexpr int kThreadsA = kWaves * 64;
constexpr int kQB = kWaves * 32;  // queries per workgroup
constexpr int kTN = 64;           // keys per tile (== reference block_n)
constexpr int kVR = kTN + 16;     // LDS row pitch of V^T (bytes)

enum { FILL_ZERO = 0, FILL_MAX, FILL_MEAN, FILL_LOGN, FILL_SAMPLE8, FILL_THR, FILL_UTA };

__device__ __forceinline__ int e8m0_of(float pow2) {
  return static_cast<int>((__float_as_uint(pow2) >> 23) & 0xffu);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

template <bool SCALED>
__device__ __forceinline__ v16f mfma32(const v8i& a, const v8i& b, const v16f& c, int sa, int sb) {
  if constexpr (SCALED) return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, sa, 0, sb);
  else return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

__device__ __forceinline__ v8i lds_read32(const uint8_t* p0, const uint8_t* p1) {
  uint4 x = *reinterpret_cast<const uint4*>(p0);
  uint4 y = *reinterpret_cast<const uint4*>(p1);
  v8i r;
  r[0] = x.x; r[1] = x.y; r[2] = x.z; r[3] = x.w;
  r[4] = y.x; r[5] = y.y; r[6] = y.z; r[7] = y.w;
  return r;
}

// LDS row of key k (0..31) inside a 32-key MFMA block: the inverse of
// pi(i) = 16*((i>>2)&1) + 4*(i>>3) + (i&3).
__device__ __forceinline__ int kperm_inv(int k) { return 8 * ((k >> 2) & 3) + 4 * (k >> 4) + (k & 3); }

// UTA bins of BS <= 16 keys: each bin lies inside one lane's 16-key chunk.
template <int BS>
__device__ __forceinline__ void uta_small(const float (&u)[32], float m_new, float off, float fa, int g,
                                          int64_t key0, int64_t S, float (&fillv)[32]) {
  const float mnat = m_new / kLog2e;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
#pragma unroll
    for (int b0 = 0; b0 < 16; b0 += BS) {
      float bs = 0.0f, bm = -INFINITY, bc = 0.0f;
#pragma unroll
      for (int r = b0; r < b0 + BS; ++r) {
        float x = u[16 * t + r];
        if (x != -INFINITY) { bs += x / kLog2e; bm = fmaxf(bm, x); bc += 1.0f; }
      }
      float sbc = fmaxf(bc, 1.0f);
      float bmean = bs / sbc;
      float bound = sbc * fast_exp2(bm - m_new + off);
      float mass = fminf(fa * sbc * fast_exp2((bmean - mnat) * kLog2e + off), bound);
      float val = mass / sbc;
#pragma unroll
      for (int r = b0; r < b0 + BS; ++r) fillv[16 * t + r] = (key0 + 32 * t + 16 * g + r) < S ? val : 0.0f;
    }
  }
}

// UTA bins of 32 (one MFMA key block, split over lanes l and l^32) or 64 keys.
template <int BS>
__device__ __forceinline__ void uta_large(const float (&u)[32], float m_new, float off, float fa, int g,
                                          int64_t key0, int64_t S, float (&fillv)[32]) {
  const float mnat = m_new / kLog2e;
  float bs[2] = {0.0f, 0.0f}, bm[2] = {-INFINITY, -INFINITY}, bc[2] = {0.0f, 0.0f};
#pragma unroll
  for (int t = 0; t < 2; ++t) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float x = u[16 * t + r];
      if (x != -INFINITY) { bs[t] += x / kLog2e; bm[t] = fmaxf(bm[t], x); bc[t] += 1.0f; }
    }
    bs[t] += __shfl_xor(bs[t], 32, 64);
    bm[t] = fmaxf(bm[t], __shfl_xor(bm[t], 32, 64));
    bc[t] += __shfl_xor(bc[t], 32, 64);
  }
  if (BS == 64) {
    bs[0] += bs[1]; bm[0] = fmaxf(bm[0], bm[1]); bc[0] += bc[1];
    bs[1] = bs[0]; bm[1] = bm[0]; bc[1] = bc[0];
  }
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    float sbc = fmaxf(bc[t], 1.0f);
    float bmean = bs[t] / sbc;
    float bound = sbc * fast_exp2(bm[t] - m_new + off);
    float mass = fminf(fa * sbc * fast_exp2((bmean - mnat) * kLog2e + off), bound);
    float val = mass / sbc;
#pragma unroll
    for (int r = 0; r < 16; ++r) fillv[16 * t + r] = (key0 + 32 * t + 16 * g + r) < S ? val : 0.0f;
  }
}

// Fill values of a BLASST-skipped row (attention_triton.py:231-324), in the
// kernel's lane layout.  u: scores in log2 units (-inf where masked).
template <int P_MODE>
__device__ __forceinline__ void blasst_fill_values(const lbfq_attn_params& a, const float (&u)[32], float c0,
                                                   float m_new, float bmax, float off, int g, int64_t key0,
                                                   float (&fillv)[32]) {
  const int64_t S = a.S;
  const int fk = a.blasst_fill;
#pragma unroll
  for (int j = 0; j < 32; ++j) fillv[j] = 0.0f;
  if (fk == FILL_ZERO) return;
  const float fa = a.blasst_fill_alpha;
  if (fk == FILL_UTA) {
    const int bsz = kTN / a.blasst_uta_bins;
    switch (bsz) {
      case 1: uta_small<1>(u, m_new, off, fa, g, key0, S, fillv); break;
      case 2: uta_small<2>(u, m_new, off, fa, g, key0, S, fillv); break;
      case 4: uta_small<4>(u, m_new, off, fa, g, key0, S, fillv); break;
      case 8: uta_small<8>(u, m_new, off, fa, g, key0, S, fillv); break;
      case 16: uta_small<16>(u, m_new, off, fa, g, key0, S, fillv); break;
      case 32: uta_large<32>(u, m_new, off, fa, g, key0, S, fillv); break;
      default: uta_large<64>(u, m_new, off, fa, g, key0, S, fillv); break;
    }
    return;
  }
  const int64_t nv64 = S - key0 < kTN ? S - key0 : kTN;
  const float n = static_cast<float>(nv64);
  // statistics in natural units (s = u / log2e), as the reference
  float ssum = 0.0f;
#pragma unroll
  for (int j = 0; j < 32; ++j) ssum += (u[j] == -INFINITY ? 0.0f : u[j] / kLog2e);
  ssum += __shfl_xor(ssum, 32, 64);
  const float mean = ssum / n;
  const float mnat = m_new / kLog2e;
  const float max_bound = n * fast_exp2(bmax - m_new + off);
  float fp = 0.0f;
  if (fk == FILL_MAX) {
    fp = max_bound * fa / n;
  } else if (fk == FILL_MEAN) {
    fp = fminf(fa * n * fast_exp2((mean - mnat) * kLog2e + off), max_bound) / n;
  } else if (fk == FILL_LOGN) {
    float vs = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      float c = u[j] == -INFINITY ? 0.0f : (u[j] / kLog2e - mean);
      vs += c * c;
    }
    vs += __shfl_xor(vs, 32, 64);
    float var = vs / n;
    fp = fminf(n * fast_exp2((mean + 0.5f * var - mnat) * kLog2e + off), max_bound) / n;
  } else if (fk == FILL_SAMPLE8) {
    // sampled keys rel % 8 == 0 are r in {0, 8} of both 32-key blocks
    float sp = 0.0f;
#pragma unroll
    for (int t = 0; t < 2; ++t) sp += fast_exp2(u[16 * t] + c0) + fast_exp2(u[16 * t + 8] + c0);
    sp += __shfl_xor(sp, 32, 64);
    float cnt = 0.0f;
    for (int kk = 0; kk < kTN; kk += 8) cnt += (key0 + kk < S) ? 1.0f : 0.0f;
    cnt = fmaxf(cnt, 1.0f);
    fp = fminf(fa * n * sp / cnt, max_bound) / n;
  } else {  // FILL_THR
    float offs = P_MODE == 0 ? exp2f(static_cast<float>(a.p_max_offset)) : 1.0f;
    fp = fa * n * a.blasst_lambda * offs / n;
  }
#pragma unroll
  for (int j = 0; j < 32; ++j) fillv[j] = (key0 + 32 * (j >> 4) + 16 * g + (j & 15)) < S ? fp : 0.0f;
}

template <int D, bool QK_MX, int P_MODE, bool BLASST, bool VALPHA>
__global__ void __launch_bounds__(kThreadsA, 1) attn_fwd_kernel(lbfq_attn_params a) {
  constexpr int NH = D / 64;   // 64-wide contraction halves of D
  constexpr int NDB = D / 32;  // 32-row blocks of O^T
  constexpr int KR = D + 16;   // LDS row pitch of K (bytes)
  constexpr int KR_PITCH = KR;
  constexpr int KCH = kTN * D / 16;  // 16-byte chunks per K tile (== per V tile)
  constexpr int CPT = KCH / kThreadsA;
  constexpr bool PV_SCALED_P = (P_MODE == 1);

  __shared__ __attribute__((aligned(16))) uint8_t k_lds[2][kTN * KR];
  __shared__ __attribute__((aligned(16))) uint8_t v_lds[2][D * kVR];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int li = lane & 31, g = lane >> 5;

  const int64_t S = a.S, H = a.H, P = a.s_pitch;
  const int64_t nqb = (S + kQB - 1) / kQB;
  const int64_t nblk = a.B * H * nqb;
  int64_t w = blockIdx.x;
  if ((nblk & 7) == 0) w = (w & 7) * (nblk >> 3) + (w >> 3);  // XCD-contiguous work ranges
  const int64_t bh = w / nqb, qb = w % nqb;
  const int64_t b = bh / H, h = bh % H;
  const int64_t q0 = qb * kQB + wave * 32;
  const int64_t qi = q0 + li;
  const bool qvalid = qi < S;
  const bool v_mx = a.v_kind == 2;

  // ---- Q operand (B of S^T = K Q^T) and Q scales --------------------------
  v8i qop[NH];
  {
    const uint8_t* qrow = a.q_codes + (bh * P + qi) * D;
#pragma unroll
    for (int hh = 0; hh < NH; ++hh) {
      // operand K-index layout: lane group g holds k = 16g+[0,16) and 32+16g+[0,16)
      uint4 x = *reinterpret_cast<const uint4*>(qrow + 64 * hh + 16 * g);
      uint4 y = *reinterpret_cast<const uint4*>(qrow + 64 * hh + 32 + 16 * g);
      qop[hh][0] = x.x; qop[hh][1] = x.y; qop[hh][2] = x.z; qop[hh][3] = x.w;
      qop[hh][4] = y.x; qop[hh][5] = y.y; qop[hh][6] = y.z; qop[hh][7] = y.w;
    }
  }
  float sq = 1.0f;
  int qe[NH];
#pragma unroll
  for (int hh = 0; hh < NH; ++hh) qe[hh] = 127;
  if constexpr (!QK_MX) {
    if (qvalid) sq = a.q_scale[b * a.qsc_b + (qi / a.qk_block) * a.qsc_s + h * a.qsc_h];
  } else {
    if (qvalid) {
#pragma unroll
      for (int hh = 0; hh < NH; ++hh)
        qe[hh] = e8m0_of(a.q_scale[b * a.qsc_b + qi * a.qsc_s + h * a.qsc_h + (2 * hh + g) * a.qsc_d]);
    }
  }
  const float sml2 = a.sm_scale * kLog2e;

  // ---- per-wave qm group: correction row and row-max estimate -------------
  const int64_t G = a.q_group > 0 ? (S / a.q_group) : 1;
  int64_t grp = a.q_group > 0 ? (q0 / a.q_group) : 0;
  if (grp >= G) grp = G - 1;  // waves made only of padding rows
  const float* bias_row = a.qk_bias ? a.qk_bias + (bh * G + grp) * P : nullptr;
  const bool has_est = a.rowmax_est != nullptr;
  constexpr bool use_blasst = BLASST;
  float m2 = -INFINITY;  // running row max, log2 units
  if (has_est) m2 = a.rowmax_est[bh * G + grp] * kLog2e;
  const float est2 = m2;
  const bool dyn_est = has_est && !use_blasst && a.rowmax_dynamic && P_MODE == 2;
  const bool fixed_est = has_est && !use_blasst && !dyn_est;
  const float off = P_MODE == 0 ? static_cast<float>(a.p_max_offset) : 0.0f;
  const float log2_lam = use_blasst ? __logf(a.blasst_lambda) * kLog2e : 0.0f;

  float l = 0.0f;          // partial row sum of pre-quant p over this lane's keys
  float max_seen = -INFINITY;
  float sigma = 1.0f;      // acc holds O^T / sigma
  float skipped = 0.0f, total = 0.0f;
  v16f acc[NDB];
  v16f cacc[VALPHA ? NDB : 1];
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[db][r] = 0.0f;
  }
#pragma unroll
  for (int db = 0; db < (VALPHA ? NDB : 1); ++db) {
#pragma unroll
    for (int r = 0; r < 16; ++r) cacc[db][r] = 0.0f;
  }

  // ---- tile staging ---------------------------------------------------------
  const uint8_t* kbase = a.k_codes + bh * P * D;
  const uint8_t* vbase = a.v_codes_t + bh * D * P;
  uint4 kr0, kr1, vr0, vr1;
#define LBFQ_LD(KR, VR, C, IT)                                                             \
  {                                                                                         \
    int e = tid + (C) * kThreadsA;                                                          \
    int n = e / (D / 16), ch = e % (D / 16);                                                \
    KR = *reinterpret_cast<const uint4*>(kbase + ((IT) * kTN + n) * D + ch * 16);           \
    int d = e / (kTN / 16), cv = e % (kTN / 16);                                            \
    VR = *reinterpret_cast<const uint4*>(vbase + d * P + (IT) * kTN + cv * 16);             \
  }
#define LBFQ_ST(KR, VR, C, BUF)                                                            \
  {                                                                                         \
    int e = tid + (C) * kThreadsA;                                                          \
    int n = e / (D / 16), ch = e % (D / 16);                                                \
    int t = n >> 5, k = n & 31;                                                             \
    *reinterpret_cast<uint4*>(&k_lds[BUF][(32 * t + kperm_inv(k)) * KR_PITCH + ch * 16]) = KR; \
    int d = e / (kTN / 16), cv = e % (kTN / 16);                                            \
    *reinterpret_cast<uint4*>(&v_lds[BUF][d * kVR + cv * 16]) = VR;                         \
  }
#define LBFQ_LOAD_TILE(IT)                       \
  LBFQ_LD(kr0, vr0, 0, IT)                       \
  if constexpr (CPT > 1) LBFQ_LD(kr1, vr1, 1, IT)
#define LBFQ_STORE_TILE(BUF)                     \
  LBFQ_ST(kr0, vr0, 0, BUF)                      \
  if constexpr (CPT > 1) LBFQ_ST(kr1, vr1, 1, BUF)

  const int64_t nt = (S + kTN - 1) / kTN;
  LBFQ_LOAD_TILE(0)
  LBFQ_STORE_TILE(0)
  __syncthreads();

  for (int64_t it = 0; it < nt; ++it) {
    const int cur = static_cast<int>(it & 1);
    if (it + 1 < nt) { LBFQ_LOAD_TILE(it + 1) }
    const int64_t key0 = it * kTN;

    // ---- S^T = K Q^T ---------------------------------------------------------
    v16f s[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[t][r] = 0.0f;
#pragma unroll
      for (int hh = 0; hh < NH; ++hh) {
        const uint8_t* rowp = &k_lds[cur][(32 * t + li) * KR + 64 * hh + 16 * g];
        v8i ka = lds_read32(rowp, rowp + 32);
        if constexpr (QK_MX) {
          int64_t key = key0 + 32 * t + 16 * ((li >> 2) & 1) + 4 * (li >> 3) + (li & 3);
          int ke = key < S ? e8m0_of(a.k_scale[b * a.ksc_b + key * a.ksc_s + h * a.ksc_h + (2 * hh + g) * a.ksc_d])
                           : 127;
          s[t] = mfma32<true>(ka, qop[hh], s[t], ke, qe[hh]);
        } else {
          s[t] = mfma32<false>(ka, qop[hh], s[t], 0, 0);
        }
      }
    }

    // ---- scores in log2 units: u = dot * C + bias * log2e, masked --------------
    float u[32];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      float C = sml2;
      if constexpr (!QK_MX) {
        int64_t kb = key0 + 32 * t + 16 * g;
        float sk = kb < S ? a.k_scale[b * a.ksc_b + (kb / a.qk_block) * a.ksc_s + h * a.ksc_h] : 1.0f;
        C = sq * sk * sml2;
      }
      float bias[16];
      if (bias_row) {
        const float4* bp = reinterpret_cast<const float4*>(bias_row + key0 + 32 * t + 16 * g);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float4 x = bp[q];
          bias[4 * q] = x.x; bias[4 * q + 1] = x.y; bias[4 * q + 2] = x.z; bias[4 * q + 3] = x.w;
        }
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float v = s[t][r] * C;
        if (bias_row) v = fmaf(bias[r], kLog2e, v);
        u[16 * t + r] = v;
      }
    }
    if (key0 + kTN > S) {
#pragma unroll
      for (int j = 0; j < 32; ++j) {
        int64_t key = key0 + 32 * (j >> 4) + 16 * g + (j & 15);
        if (key >= S) u[j] = -INFINITY;
      }
    }
    float bmax = -INFINITY;
#pragma unroll
    for (int j = 0; j < 32; ++j) bmax = fmaxf(bmax, u[j]);
    bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));

    // ---- row max / rescale factor --------------------------------------------
    float m_new, alpha;
    bool skip = false;
    if (use_blasst) {
      float mij = fmaxf(m2, bmax);
      skip = qvalid && (bmax - mij) < log2_lam;
      alpha = skip ? 1.0f : fast_exp2(m2 - mij);
      m_new = skip ? m2 : mij;
      if (g == 0) { skipped += skip ? 1.0f : 0.0f; total += qvalid ? 1.0f : 0.0f; }
    } else if (dyn_est) {
      float lfull = l + __shfl_xor(l, 32, 64);
      float ms = fmaxf(max_seen, bmax);
      bool under = (bmax - m2) > 16.0f;
      bool over = (m2 - ms) > 32.0f;
      float down_b = fmaxf(ms + 32.0f, m2 - 80.0f * kLog2e);
      float down = lfull == 0.0f ? ms : down_b;
      float adj = under ? bmax : down;
      bool adjust = under || over;
      m_new = adjust ? adj : m2;
      float au = lfull == 0.0f ? 0.0f : fast_exp2(m2 - m_new);
      alpha = adjust ? au : 1.0f;
      max_seen = ms;
    } else if (fixed_est) {
      m_new = est2;
      alpha = 1.0f;
    } else {
      m_new = fmaxf(m2, bmax);
      alpha = fast_exp2(m2 - m_new);
    }

    // ---- P = exp2(u - m + off), BLASST fill -----------------------------------
    const float c0 = off - m_new;
    float p[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) p[j] = fast_exp2(u[j] + c0);
    if constexpr (BLASST) {
      if (__any(skip)) {
        float fillv[32];
        blasst_fill_values<P_MODE>(a, u, c0, m_new, bmax, off, g, key0, fillv);
        if (skip) {
#pragma unroll
          for (int j = 0; j < 32; ++j) p[j] = fillv[j];
        }
      }
    }

    float psum = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; ++j) psum += p[j];
    l = l * alpha + psum;

    // ---- P quantisation ---------------------------------------------------------
    float pscale = 1.0f;    // P_deq = code * pscale
    int pe = 127;           // E8M0 of pscale (mx mode)
    float qmul = 1.0f;
    if constexpr (P_MODE == 1) {
      float pa = 0.0f;
#pragma unroll
      for (int j = 0; j < 32; ++j) pa = fmaxf(pa, p[j]);
      pa = fmaxf(pa, __shfl_xor(pa, 32, 64));
      pa = fmaxf(pa, kAmaxFloor);
      int e = ceil_log2_exact(pa / kFp8Max);
      e = e < -127 ? -127 : (e > 127 ? 127 : e);
      pe = e + 127;
      qmul = ldexpf(1.0f, -e);
      pscale = ldexpf(1.0f, e);
    } else if constexpr (P_MODE == 2) {
      float pa = 0.0f;
#pragma unroll
      for (int j = 0; j < 32; ++j) pa = fmaxf(pa, p[j]);
      pa = fmaxf(pa, __shfl_xor(pa, 32, 64));
      pa = fmaxf(pa, 1e-12f);
      pscale = pa / kFp8Max;
      qmul = kFp8Max / pa;
    }
    v8i pop;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      float x0 = fminf(p[4 * q] * qmul, kFp8Max), x1 = fminf(p[4 * q + 1] * qmul, kFp8Max);
      float x2 = fminf(p[4 * q + 2] * qmul, kFp8Max), x3 = fminf(p[4 * q + 3] * qmul, kFp8Max);
      int wd = __builtin_amdgcn_cvt_pk_fp8_f32(x0, x1, 0, false);
      wd = __builtin_amdgcn_cvt_pk_fp8_f32(x2, x3, wd, true);
      pop[q] = wd;
    }

    // ---- accumulator rescale (alpha, dynamic P scale, fp8_block V scale) ------
    float sig_new = (P_MODE == 2) ? pscale : 1.0f;
    if (a.v_kind == 1) {
      float svb = a.v_scale[(b * (S / a.v_block) + key0 / a.v_block) * H + h];
      sig_new *= svb;
    }
    float f = alpha * (sigma / sig_new);
    sigma = sig_new;
    if (__any(f != 1.0f)) {
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[db][r] *= f;
      }
    }

    // ---- O^T += V^T P^T ---------------------------------------------------------
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const uint8_t* vp = &v_lds[cur][(32 * db + li) * kVR + 16 * g];
      v8i va = lds_read32(vp, vp + 32);
      if (v_mx || PV_SCALED_P) {
        int ve = 127;
        if (v_mx) ve = e8m0_of(a.v_scale[((b * (S / a.v_block) + key0 / a.v_block) * H + h) * D + 32 * db + li]);
        acc[db] = mfma32<true>(va, pop, acc[db], ve, pe);
      } else {
        acc[db] = mfma32<false>(va, pop, acc[db], 0, 0);
      }
    }

    // ---- V-smoothing accumulator: c = c * alpha + rowsum(P_deq) (x) alpha_v ----
    if constexpr (VALPHA) {
      float cs = 0.0f;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        int wd = pop[q];
#pragma unroll
        for (int k = 0; k < 4; ++k) cs += e4m3_decode(static_cast<uint8_t>((wd >> (8 * k)) & 0xff));
      }
      cs += __shfl_xor(cs, 32, 64);
      float rs = cs * pscale;
      const float* av = a.v_alpha + ((b * (S / a.v_smooth_block) + key0 / a.v_smooth_block) * H + h) * D;
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          int d = 32 * db + 8 * (r >> 2) + 4 * g + (r & 3);
          cacc[db][r] = fmaf(rs, av[d], cacc[db][r] * alpha);
        }
      }
    }
    m2 = m_new;

    if (it + 1 < nt) { LBFQ_STORE_TILE(1 - cur) }
    __syncthreads();
  }

#undef LBFQ_LOAD_TILE
#undef LBFQ_STORE_TILE
#undef LBFQ_LD
#undef LBFQ_ST
  // ---- epilogue -------------------------------------------------------------------
  const float lfull = l + __shfl_xor(l, 32, 64);
  if (a.blasst_stats && g == 0) {
    // per block_m rows: all lanes of the wave add into their row block
    int64_t rb = qi / a.block_m;
    if (qvalid) {
      atomicAdd(a.blasst_stats + (rb * (a.B * H) + bh) * 2 + 0, skipped);
      atomicAdd(a.blasst_stats + (rb * (a.B * H) + bh) * 2 + 1, total);
    }
  }
  if (!qvalid) return;
  const float inv_l = 1.0f / lfull;
  const int64_t orow = a.out_row_map ? a.out_row_map[bh * S + qi] : qi;
  const int64_t obase = ((b * S + orow) * H + h) * D;
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      float o[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        int d = 32 * db + 8 * r4 + 4 * g + k;
        float main = acc[db][4 * r4 + k] * sigma;
        if (a.v_kind == 0) main *= a.v_scale[(b * H + h) * D + d];
        if constexpr (VALPHA) main += cacc[db][4 * r4 + k];
        // the reference writes a bf16 BHSD tensor, then casts to the output dtype
        o[k] = bf16_bits_to_f32(f32_to_bf16_bits(main * inv_l));
      }
      int d0 = 32 * db + 8 * r4 + 4 * g;
      if (a.out_dtype == kF32) {
        *reinterpret_cast<float4*>(reinterpret_cast<float*>(a.out) + obase + d0) = make_float4(o[0], o[1], o[2], o[3]);
      } else {
        uint32_t w0, w1;
        if (a.out_dtype == kBF16) {
          w0 = f32_to_bf16_bits(o[0]) | (static_cast<uint32_t>(f32_to_bf16_bits(o[1])) << 16);
          w1 = f32_to_bf16_bits(o[2]) | (static_cast<uint32_t>(f32_to_bf16_bits(o[3])) << 16);
        } else {
          w0 = f32_to_f16_bits(o[0]) | (static_cast<uint32_t>(f32_to_f16_bits(o[1])) << 16);
          w1 = f32_to_f16_bits(o[2]) | (static_cast<uint32_t>(f32_to_f16_bits(o[3])) << 16);
        }
        *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(a.out) + obase + d0) = make_uint2(w0, w1);
      }
    }
  }
}

// ---- self tests of the builtins ------------------------------------------------
__global__ void selftest_cvt_kernel(const float* x, int64_t n, uint8_t* out) {
  int64_t i = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
  if (i + 3 >= n + 3 || i >= n) return;
  float x0 = x[i], x1 = i + 1 < n ? x[i + 1] : 0.f, x2 = i + 2 < n ? x[i + 2] : 0.f, x3 = i + 3 < n ? x[i + 3] : 0.f;
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(x0, x1, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(x2, x3, w, true);
  for (int k = 0; k < 4 && i + k < n; ++k) out[i + k] = static_cast<uint8_t>((w >> (8 * k)) & 0xff);
}

__global__ void selftest_mfma_kernel(const uint8_t* A, const uint8_t* Bm, const uint8_t* as, const uint8_t* bs,
                                     float* C) {
  int lane = threadIdx.x, li = lane & 31, g = lane >> 5;
  v8i av, bv;
  for (int q = 0; q < 8; ++q) {
    int wa = 0, wb = 0;
    for (int k = 0; k < 4; ++k) {
      int slot = 4 * q + k;
      int kk = slot < 16 ? 16 * g + slot : 32 + 16 * g + (slot - 16);
      wa |= static_cast<int>(A[li * 64 + kk]) << (8 * k);
      wb |= static_cast<int>(Bm[kk * 32 + li]) << (8 * k);
    }
    av[q] = wa; bv[q] = wb;
  }
  v16f c;
  for (int r = 0; r < 16; ++r) c[r] = 0.0f;
  if (as) c = mfma32<true>(av, bv, c, as[li * 2 + g], bs[li * 2 + g]);
  else c = mfma32<false>(av, bv, c, 0, 0);
  for (int r = 0; r < 16; ++r) C[(8 * (r >> 2) + 4 * g + (r & 3)) * 32 + li] = c[r];
}

template <int D, bool QK_MX, int P_MODE, bool BL, bool VA>
int launch(const lbfq_attn_params* p, hipStream_t st) {
  int64_t nqb = (p->S + kQB - 1) / kQB;
  int64_t nblk = p->B * p->H * nqb;
  hipLaunchKernelGGL((attn_fwd_kernel<D, QK_MX, P_MODE, BL, VA>), dim3(static_cast<unsigned>(nblk)), dim3(kThreadsA), 0,
                     st, *p);
  LBFQ_LAUNCH_CHECK("lbfq_attention_fwd");
  return 0;
}

template <int D, bool BL, bool VA>
int dispatch_p(const lbfq_attn_params* p, hipStream_t st) {
  if (p->qk_mx) {
    if (p->p_mode == 0) return launch<D, true, 0, BL, VA>(p, st);
    if (p->p_mode == 1) return launch<D, true, 1, BL, VA>(p, st);
    return launch<D, true, 2, BL, VA>(p, st);
  }
  if (p->p_mode == 0) return launch<D, false, 0, BL, VA>(p, st);
  if (p->p_mode == 1) return launch<D, false, 1, BL, VA>(p, st);
  return launch<D, false, 2, BL, VA>(p, st);
}

template <int D>
int dispatch_d(const lbfq_attn_params* p, hipStream_t st) {
  const bool bl = p->blasst_lambda > 0.0f, va = p->v_alpha != nullptr;
  if (bl) return va ? dispatch_p<D, true, true>(p, st) : dispatch_p<D, true, false>(p, st);
  return va ? dispatch_p<D, false, true>(p, st) : dispatch_p<D, false, false>(p, st);
}

}  // namespace

extern "C" int lbfq_attention_fwd(const lbfq_attn_params* p, lbfq_stream_t stream) {
  LBFQ_CHECK_ARG(p, "lbfq_attention_fwd: null params");
  LBFQ_CHECK_ARG(p->D == 64 || p->D == 128, "lbfq_attention_fwd: D must be 64 or 128; got %lld", (long long)p->D);
  LBFQ_CHECK_ARG(p->B > 0 && p->H > 0 && p->S > 0, "lbfq_attention_fwd: empty shape");
  LBFQ_CHECK_ARG(p->s_pitch >= p->S && p->s_pitch % kQB == 0,
                 "lbfq_attention_fwd: s_pitch must be >= S and a multiple of %d", kQB);
  LBFQ_CHECK_ARG(p->q_codes && p->k_codes && p->v_codes_t && p->out && p->q_scale && p->k_scale,
                 "lbfq_attention_fwd: missing tensor");
  LBFQ_CHECK_ARG(p->qk_mx || (p->qk_block >= 16 && p->qk_block % 16 == 0),
                 "lbfq_attention_fwd: fp8_block size must be a multiple of 16; got %d", p->qk_block);
  LBFQ_CHECK_ARG(p->v_kind >= 0 && p->v_kind <= 2 && p->v_scale, "lbfq_attention_fwd: bad V kind");
  LBFQ_CHECK_ARG(p->v_kind == 0 || (p->v_block >= kTN && p->v_block % kTN == 0 && p->S % p->v_block == 0),
                 "lbfq_attention_fwd: V block (%d) must be a multiple of %d dividing S", p->v_block, kTN);
  LBFQ_CHECK_ARG(p->p_mode >= 0 && p->p_mode <= 2, "lbfq_attention_fwd: bad P mode");
  LBFQ_CHECK_ARG(!p->qk_bias || (p->q_group >= 32 && p->q_group % 32 == 0 && p->s_pitch % p->q_group == 0),
                 "lbfq_attention_fwd: q_group must be a multiple of 32 dividing s_pitch");
  LBFQ_CHECK_ARG(!p->rowmax_est || (p->q_group >= 32 && p->q_group % 32 == 0 && p->S % p->q_group == 0),
                 "lbfq_attention_fwd: rowmax_est needs q_group dividing S");
  LBFQ_CHECK_ARG(!p->v_alpha || (p->v_smooth_block >= kTN && p->v_smooth_block % kTN == 0 &&
                                  p->S % p->v_smooth_block == 0),
                 "lbfq_attention_fwd: v_smooth_block must be a multiple of %d dividing S", kTN);
  LBFQ_CHECK_ARG(!p->blasst_stats || (p->block_m > 0 && p->block_m % 32 == 0),
                 "lbfq_attention_fwd: block_m must be a multiple of 32");
  LBFQ_CHECK_ARG(p->blasst_lambda <= 0.0f || p->blasst_lambda < 1.0f, "lbfq_attention_fwd: lambda must be < 1");
  LBFQ_CHECK_ARG(p->blasst_fill != FILL_UTA || (p->blasst_uta_bins > 0 && kTN % p->blasst_uta_bins == 0),
                 "lbfq_attention_fwd: UTA bins must divide %d", kTN);
  LBFQ_CHECK_ARG(p->out_dtype >= 0 && p->out_dtype <= 2, "lbfq_attention_fwd: bad out dtype");
  hipStream_t st = static_cast<hipStream_t>(stream);
  return p->D == 128 ? dispatch_d<128>(p, st) : dispatch_d<64>(p, st);
}

extern "C" int lbfq_selftest_cvt_fp8(const float* x, int64_t n, uint8_t* out, lbfq_stream_t stream) {
  LBFQ_CHECK_ARG(x && out && n > 0, "lbfq_selftest_cvt_fp8: bad args");
  int64_t nt = (n + 3) / 4;
  hipLaunchKernelGGL(selftest_cvt_kernel, dim3(static_cast<unsigned>((nt + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, n, out);
  LBFQ_LAUNCH_CHECK("lbfq_selftest_cvt_fp8");
  return 0;
}

extern "C" int lbfq_selftest_mfma(const uint8_t* a, const uint8_t* b, const uint8_t* a_scale, const uint8_t* b_scale,
                                  float* c, lbfq_stream_t stream) {
  LBFQ_CHECK_ARG(a && b && c && ((a_scale == nullptr) == (b_scale == nullptr)), "lbfq_selftest_mfma: bad args");
  hipLaunchKernelGGL(selftest_mfma_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), a, b, a_scale,
                     b_scale, c);
  LBFQ_LAUNCH_CHECK("lbfq_selftest_mfma");
  return 0;
}
