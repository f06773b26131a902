// FP8-MFMA P-requant attention for gfx950 (CDNA4): templated kernel body.
//
// Reference semantics: the K-loop of _fake_quant_attn_fwd_kernel
// (attention_triton.py:109-407).  The reference dequantises Q/K/V to bf16 and
// runs bf16 dots; this kernel multiplies the FP8 codes on the matrix cores
// (v_mfma[_scale]_f32_32x32x64_f8f6f4) and applies the scales outside, or
// through the E8M0 block scales of the MFMA for the MX formats.
//
// Work decomposition: one workgroup = 4 waves = 128 queries of one (b, h);
// each wave owns 32 queries.  K and V^T tiles of 64 keys (== the reference
// block_n) are staged in LDS, double buffered, together with the per-tile
// metadata (qm correction row, K/V scales, V block means), and shared by the
// 4 waves.  Scores are computed transposed, S^T = K Q^T, so every lane owns
// exactly one query: lane l holds query l % 32 and, in lane group
// g = l / 32, the 32 keys 32t + 16g + r (t in {0,1}, r in 0..15) of the tile.
// K rows are permuted in LDS so that the MFMA accumulator layout yields that
// key order; the same 32 keys are then the lane's B operand of the PV
// product O^T = V^T P^T without any data movement.  Row statistics are
// in-lane reductions plus one exchange with lane l ^ 32.
//
// Operand K-index layout of v_mfma[_scale]_f32_32x32x64_f8f6f4 (measured):
// lane l supplies row/column l % 32; lane group g = l / 32 holds the 32
// K-elements 16g + [0,16) (bytes 0..15) and 32 + 16g + [0,16) (bytes
// 16..31); the E8M0 scale of K-block b (k in [32b, 32b+32)) comes from lane
// (l % 32) + 32b.  MX scale blocks along D therefore align with 64-wide
// contraction halves loaded as two 16-byte pieces, and in PV the tile's key
// index equals the hardware K index.
//
// P is produced directly in its quantised units: p_q = exp2(u - T) with u the
// score in log2 units and T chosen per row and tile so that p_q = p / s_P
// (elementwise: T = m - p_max_offset; mx: T = m + E; dynamic:
// T = max(rowmax, m + log2 1e-12) - log2 448).  The row sum uses
// s_P * sum(p_q) (= sum of the pre-quant p, as the reference).
//
// Per-query fp32 factors of the accumulator (online-softmax alpha, dynamic P
// scale, fp8_block V scale) are folded into one rescale of O^T per tile,
// skipped when the whole wave has factor 1.
#pragma once

#include "lbfq_common.h"
#include "../../include/lbfq.h"

namespace lbfq_attn {

using namespace lbfq;

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLog2Fp8Max = 8.807354922057604f;     // log2(448)
constexpr float kLog2DynFloor = -39.86313713864835f;  // log2(1e-12)
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kQB = kWaves * 32;  // queries per workgroup
constexpr int kTN = 64;           // keys per tile (== reference block_n)

enum { RB_ONLINE = 0, RB_ONLINE_BIAS = 1, RB_EST_BIAS = 2 };
enum { FILL_ZERO = 0, FILL_MAX, FILL_MEAN, FILL_LOGN, FILL_SAMPLE8, FILL_THR, FILL_UTA };

// Kernel-side arguments (32-bit sizes, log2 block sizes), built on the host.
struct KArgs {
  int B, H, S, P, nqb;
  int G, lg_qgroup;
  int lg_qkblk, nqkblk;
  int v_kind, lg_vblk, nvblk;
  int lg_vsb, nvsb;
  int p_max_offset, block_m, rowmax_dynamic;
  float sml2;
  float log2_lam, lam, fill_alpha;
  int fill_kind, uta_bins;
  const uint8_t* q_codes;
  const uint8_t* k_codes;
  const uint8_t* v_codes_t;
  const void* q_scale;
  const void* k_scale;
  const void* v_scale;
  const float* bias;
  const float* rowmax;
  const float* v_alpha;
  float* stats;
  void* out;
  int out_dtype;
  const int32_t* out_row_map;
};

// Per-tile metadata staged in LDS next to the K / V^T codes.  The K side is
// consumed by the softmax of the tile, the V side by its PV product.
struct KMeta {
  float bias[kWaves][kTN];  // qm correction (log2 units) of each wave's group
  float ksc[4];             // fp8_block K scale of each 16-key group
};

template <int D>
struct VMeta {
  uint32_t ve[D / 4];       // E8M0 byte of each V column (4 per word); 127 unless V is MX
  float vsc;                // fp8_block V scale of the tile
  float valpha[D];          // V block mean of the tile
};

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

// Asynchronous global -> LDS copies (gfx950 global_load_lds): every active
// lane copies 16 (or 4) bytes from its own global address to
// lds_base + lane * 16 (or 4); lds_base is wave-uniform and goes through M0.
// Issued as inline asm so that the compiler does not order every later LDS
// read behind them: the kernel makes them visible itself, with an explicit
// vmcnt(0) wait before the barrier that publishes a tile (lds_publish).  The
// kernel never indexes registers dynamically, so the compiler holds nothing
// in M0 across these statements.
__device__ __forceinline__ void g2l16(const void* gsrc, const void* lds_base) {
  const uint32_t la = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds_base)));
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gsrc), "s"(la) : "memory", "m0");
}
__device__ __forceinline__ void g2l4(const void* gsrc, const void* lds_base) {
  const uint32_t la = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds_base)));
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(gsrc), "s"(la) : "memory", "m0");
}
// Wait for this wave's global -> LDS copies, then the workgroup barrier.
__device__ __forceinline__ void lds_publish() {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
}

// XOR swizzles of the 16-byte chunks of a K row (D bytes) and of a V^T row
// (64 bytes): the 16 rows read together by one half-wave land in distinct
// bank groups, without padding.
template <int D>
__device__ __forceinline__ int swz_k(int r) { return D == 128 ? ((r >> 1) & 7) : ((r >> 2) & 3); }
__device__ __forceinline__ int swz_v(int r) { return (r >> 2) & 3; }

// Key held by accumulator row i of a 32-key MFMA block:
// pi(i) = 16*((i>>2)&1) + 4*(i>>3) + (i&3); kperm_inv is its inverse.
__device__ __forceinline__ int kperm(int i) { return 16 * ((i >> 2) & 1) + 4 * (i >> 3) + (i & 3); }
__device__ __forceinline__ int kperm_inv(int k) { return 8 * ((k >> 2) & 3) + 4 * (k >> 4) + (k & 3); }

__device__ __forceinline__ float xor32_max(float v) { return fmaxf(v, __shfl_xor(v, 32, 64)); }
__device__ __forceinline__ float xor32_add(float v) { return v + __shfl_xor(v, 32, 64); }

// ---- BLASST fill values (attention_triton.py:231-324) in the lane layout -----
// u: scores in log2 units (-inf where masked); p units include the elementwise
// p_max_offset ("off") as in the reference.
template <int BS>
__device__ __forceinline__ void uta_small(const float (&u)[32], float m_new, float off, float fa, int g,
                                          int key0, int S, float (&fillv)[32]) {
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

template <int BS>
__device__ __forceinline__ void uta_large(const float (&u)[32], float m_new, float off, float fa, int g,
                                          int key0, int S, float (&fillv)[32]) {
  const float mnat = m_new / kLog2e;
  float bs[2] = {0.0f, 0.0f}, bm[2] = {-INFINITY, -INFINITY}, bc[2] = {0.0f, 0.0f};
#pragma unroll
  for (int t = 0; t < 2; ++t) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float x = u[16 * t + r];
      if (x != -INFINITY) { bs[t] += x / kLog2e; bm[t] = fmaxf(bm[t], x); bc[t] += 1.0f; }
    }
    bs[t] = xor32_add(bs[t]);
    bm[t] = xor32_max(bm[t]);
    bc[t] = xor32_add(bc[t]);
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

template <int P_MODE>
__device__ __forceinline__ void blasst_fill_values(const KArgs& a, const float (&u)[32], float m_new, float bmax,
                                                   float off, int g, int key0, float (&fillv)[32]) {
  const int S = a.S;
  const int fk = a.fill_kind;
#pragma unroll
  for (int j = 0; j < 32; ++j) fillv[j] = 0.0f;
  if (fk == FILL_ZERO) return;
  const float fa = a.fill_alpha;
  if (fk == FILL_UTA) {
    switch (kTN / a.uta_bins) {
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
  const float n = static_cast<float>(S - key0 < kTN ? S - key0 : kTN);
  float ssum = 0.0f;
#pragma unroll
  for (int j = 0; j < 32; ++j) ssum += (u[j] == -INFINITY ? 0.0f : u[j] / kLog2e);
  ssum = xor32_add(ssum);
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
    vs = xor32_add(vs);
    float var = vs / n;
    fp = fminf(n * fast_exp2((mean + 0.5f * var - mnat) * kLog2e + off), max_bound) / n;
  } else if (fk == FILL_SAMPLE8) {
    // sampled keys rel % 8 == 0 are r in {0, 8} of both 32-key blocks
    const float c0 = off - m_new;
    float sp = 0.0f;
#pragma unroll
    for (int t = 0; t < 2; ++t) sp += fast_exp2(u[16 * t] + c0) + fast_exp2(u[16 * t + 8] + c0);
    sp = xor32_add(sp);
    float cnt = 0.0f;
    for (int kk = 0; kk < kTN; kk += 8) cnt += (key0 + kk < S) ? 1.0f : 0.0f;
    cnt = fmaxf(cnt, 1.0f);
    fp = fminf(fa * n * sp / cnt, max_bound) / n;
  } else {  // FILL_THR
    float offs = P_MODE == 0 ? exp2f(static_cast<float>(a.p_max_offset)) : 1.0f;
    fp = fa * n * a.lam * offs / n;
  }
#pragma unroll
  for (int j = 0; j < 32; ++j) fillv[j] = (key0 + 32 * (j >> 4) + 16 * g + (j & 15)) < S ? fp : 0.0f;
}

template <int D, bool QK_MX, int P_MODE, int RB, bool BLASST, bool VALPHA>
__global__ void __launch_bounds__(kThreads, (BLASST || VALPHA) ? 1 : 2) attn_fwd_kernel(const KArgs a) {
  constexpr int NH = D / 64;          // 64-wide contraction halves of D
  constexpr int NDB = D / 32;         // 32-row blocks of O^T
  constexpr int CPT = kTN * D / 16 / kThreads;  // 16-byte chunks per thread per K (and V) tile
  constexpr bool HAS_BIAS = RB != RB_ONLINE;
  constexpr bool HAS_EST = RB == RB_EST_BIAS;

  __shared__ __attribute__((aligned(16))) uint8_t k_lds[2][kTN * D];   // swizzled K rows (key order kperm)
  __shared__ __attribute__((aligned(16))) uint8_t v_lds[2][D * kTN];   // swizzled V^T rows
  __shared__ __attribute__((aligned(16))) uint32_t ke_lds[2][kTN];  // MX: E8M0 bytes of the key's D/32 chunks
  __shared__ __attribute__((aligned(16))) KMeta kmeta[2];
  __shared__ __attribute__((aligned(16))) VMeta<D> vmeta[2];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int li = lane & 31, g = lane >> 5;
  const int S = a.S, P = a.P;

  // XCD-aware work order: consecutive work items of one head land on one XCD
  const int nblk = a.B * a.H * a.nqb;
  int w = blockIdx.x;
  if ((nblk & 7) == 0) w = (w & 7) * (nblk >> 3) + (w >> 3);
  const int bh = w / a.nqb, qb = w - bh * a.nqb;
  const int h = bh % a.H, b = bh / a.H;
  const int q0 = qb * kQB + wave * 32;
  const int qi = q0 + li;
  const bool qvalid = qi < S;

  const uint8_t* kbase = a.k_codes + static_cast<size_t>(bh) * P * D;
  const uint8_t* vbase = a.v_codes_t + static_cast<size_t>(bh) * D * P;

  // ---- Q operand (B of S^T = K Q^T) and Q scales ----------------------------
  v8i qop[NH];
  int qe[NH];
  {
    const uint8_t* qrow = a.q_codes + (static_cast<size_t>(bh) * P + qi) * D;
#pragma unroll
    for (int hh = 0; hh < NH; ++hh) {
      uint4 x = *reinterpret_cast<const uint4*>(qrow + 64 * hh + 16 * g);
      uint4 y = *reinterpret_cast<const uint4*>(qrow + 64 * hh + 32 + 16 * g);
      qop[hh][0] = x.x; qop[hh][1] = x.y; qop[hh][2] = x.z; qop[hh][3] = x.w;
      qop[hh][4] = y.x; qop[hh][5] = y.y; qop[hh][6] = y.z; qop[hh][7] = y.w;
      qe[hh] = 127;
    }
  }
  float qC = a.sml2;  // fp8_block: sq * sm_scale * log2(e)
  if constexpr (!QK_MX) {
    if (qvalid) qC *= reinterpret_cast<const float*>(a.q_scale)[bh * a.nqkblk + (qi >> a.lg_qkblk)];
  } else {
    const uint8_t* qs = reinterpret_cast<const uint8_t*>(a.q_scale) + (static_cast<size_t>(bh) * P + qi) * (D / 32);
#pragma unroll
    for (int hh = 0; hh < NH; ++hh) qe[hh] = qvalid ? qs[2 * hh + g] : 127;
  }

  // ---- qm group of this wave; row-max state ------------------------------------
  int grp = 0;
  if constexpr (HAS_BIAS) {
    grp = q0 >> a.lg_qgroup;
    if (grp >= a.G) grp = a.G - 1;  // waves made only of padding rows
  }
  float m2 = -INFINITY;  // running row max, log2 units
  if constexpr (HAS_EST) m2 = a.rowmax[bh * a.G + grp];
  const float est2 = m2;
  const bool dyn_est = HAS_EST && !BLASST && P_MODE == 2 && a.rowmax_dynamic;
  const float off = P_MODE == 0 ? static_cast<float>(a.p_max_offset) : 0.0f;

  float l = 0.0f;  // partial row sum of the pre-quant p over this lane's keys
  float max_seen = -INFINITY;
  float sigma = 1.0f;  // acc holds O^T / sigma
  float skipped = 0.0f, total = 0.0f;
  v16f acc[NDB];
  v16f cacc[VALPHA ? NDB : 1];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[db][r] = 0.0f;
#pragma unroll
  for (int db = 0; db < (VALPHA ? NDB : 1); ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) cacc[db][r] = 0.0f;

  // ---- tile loader ------------------------------------------------------------
  // K codes (and MX K scales) are staged two tiles ahead -- the scores of tile
  // t+1 are computed while the softmax of tile t runs -- V codes and the other
  // metadata one tile ahead.  All copies go global -> LDS directly (no
  // registers); each thread owns CPT 16-byte chunks of the K and V^T tiles.
  // LDS chunk slot s of the K tile is (row s / (D/16), physical chunk s % (D/16));
  // row r holds key 32*(r/32) + kperm(r%32), so that the MFMA accumulator rows
  // come out in the lane's key order.  V^T rows are the D columns of V.
  int kofs[CPT], vofs[CPT];
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int sl = c * kThreads + tid;
    const int r = sl / (D / 16), ch = (sl % (D / 16)) ^ swz_k<D>(sl / (D / 16));
    kofs[c] = (32 * (r >> 5) + kperm(r & 31)) * D + ch * 16;
    const int d = sl / (kTN / 16), cv = (sl % (kTN / 16)) ^ swz_v(sl / (kTN / 16));
    vofs[c] = d * P + cv * 16;
  }
  int bias_grp = 0;
  if constexpr (HAS_BIAS) {
    bias_grp = (qb * kQB + wave * 32) >> a.lg_qgroup;
    if (bias_grp >= a.G) bias_grp = a.G - 1;
  }
  const float* bias_src = HAS_BIAS ? a.bias + (static_cast<size_t>(bh) * a.G + bias_grp) * P : nullptr;
  const int nt = (S + kTN - 1) / kTN;
  // V^T E8M0 column scales are constant 127 (= 1) unless V is MX
  if (a.v_kind != 2 && tid < D / 4) {
    vmeta[0].ve[tid] = 0x7f7f7f7fu;
    vmeta[1].ve[tid] = 0x7f7f7f7fu;
  }

  auto load_k = [&](int it, int buf) {
    const uint8_t* src = kbase + (it * kTN) * D;
#pragma unroll
    for (int c = 0; c < CPT; ++c) g2l16(src + kofs[c], &k_lds[buf][(c * kThreads + wave * 64) * 16]);
    if constexpr (QK_MX) {
      // E8M0 bytes of the 64 keys (D/32 per key), one dword per lane
      const uint8_t* kp = reinterpret_cast<const uint8_t*>(a.k_scale) + (static_cast<size_t>(bh) * P + it * kTN) * (D / 32);
      if (wave == 0 && lane < kTN * (D / 32) / 4) g2l4(kp + 4 * lane, &ke_lds[buf][0]);
    }
  };
  auto load_v = [&](int it, int buf) {
    const int key0 = it * kTN;
#pragma unroll
    for (int c = 0; c < CPT; ++c) g2l16(vbase + key0 + vofs[c], &v_lds[buf][(c * kThreads + wave * 64) * 16]);
    if constexpr (HAS_BIAS) g2l4(bias_src + key0 + lane, &kmeta[buf].bias[wave][0]);
    if constexpr (!QK_MX) {
      if (wave == 1 && lane < 4) {
        int kb = (key0 + 16 * lane) >> a.lg_qkblk;
        kb = kb < a.nqkblk ? kb : a.nqkblk - 1;
        g2l4(reinterpret_cast<const float*>(a.k_scale) + bh * a.nqkblk + kb, &kmeta[buf].ksc[0]);
      }
    }
    const int vblk = bh * a.nvblk + (key0 >> a.lg_vblk);
    if (a.v_kind == 1) {
      if (wave == 2 && lane == 0) g2l4(reinterpret_cast<const float*>(a.v_scale) + vblk, &vmeta[buf].vsc);
    } else if (a.v_kind == 2) {
      if (wave == 2 && lane < D / 4)
        g2l4(reinterpret_cast<const uint32_t*>(a.v_scale) + vblk * (D / 4) + lane, &vmeta[buf].ve[0]);
    }
    if constexpr (VALPHA) {
      const float* va = a.v_alpha + (static_cast<size_t>(bh) * a.nvsb + (key0 >> a.lg_vsb)) * D;
      if (wave == 3) {
#pragma unroll
        for (int c = 0; c < D / 64; ++c) g2l4(va + 64 * c + lane, &vmeta[buf].valpha[64 * c]);
      }
    }
  };
  // S^T = K Q^T of the K tile in buffer kb
  auto scores = [&](int kb, v16f (&s)[2]) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[t][r] = 0.0f;
#pragma unroll
      for (int hh = 0; hh < NH; ++hh) {
        const int r = 32 * t + li;
        const uint8_t* rp = &k_lds[kb][r * D];
        v8i ka = lds_read32(rp + 16 * ((4 * hh + g) ^ swz_k<D>(r)), rp + 16 * ((4 * hh + 2 + g) ^ swz_k<D>(r)));
        if constexpr (QK_MX) {
          int ke;
          if constexpr (D == 128) ke = (ke_lds[kb][32 * t + kperm(li)] >> (8 * (2 * hh + g))) & 0xff;
          else ke = reinterpret_cast<const uint8_t*>(&ke_lds[kb][0])[2 * (32 * t + kperm(li)) + g];
          s[t] = mfma32<true>(ka, qop[hh], s[t], ke, qe[hh]);
        } else {
          s[t] = mfma32<false>(ka, qop[hh], s[t], 0, 0);
        }
      }
    }
  };

  // prologue: tile 0 complete, K codes of tile 1
  load_k(0, 0);
  load_v(0, 0);
  load_k(nt > 1 ? 1 : 0, 1);
  lds_publish();
  v16f s_a[2], s_b[2];
  scores(0, s_a);
  __syncthreads();  // every wave has read K tile 0 before it is overwritten

  // one K/V tile: softmax of s_cur (tile it) while the scores of tile it+1
  // are computed into s_nxt
  auto step = [&](const int it, v16f (&s_cur)[2], v16f (&s_nxt)[2]) __attribute__((always_inline)) {
    const int cur = it & 1;
    const int key0 = it * kTN;
    // global -> LDS prefetch: K of tile it+2 into the buffer of tile it (read
    // before the last barrier), V and metadata of tile it+1 (clamped: the last
    // iterations reload the last tile into buffers nobody reads any more)
    load_k(it + 2 < nt ? it + 2 : nt - 1, cur);
    load_v(it + 1 < nt ? it + 1 : nt - 1, 1 - cur);
    // scores of the next tile run on the matrix cores during this softmax
    if (it + 1 < nt) scores(1 - cur, s_nxt);
    const KMeta& km = kmeta[cur];

    // ---- scores in log2 units: u = dot * C (+ qm correction), masked ------------
    float u[32];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      float C = qC;
      if constexpr (!QK_MX) C *= km.ksc[2 * t + g];
      if constexpr (HAS_BIAS) {
        const float4* bp = reinterpret_cast<const float4*>(&km.bias[wave][32 * t + 16 * g]);
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          float4 bb = bp[q4];
          u[16 * t + 4 * q4 + 0] = fmaf(s_cur[t][4 * q4 + 0], C, bb.x);
          u[16 * t + 4 * q4 + 1] = fmaf(s_cur[t][4 * q4 + 1], C, bb.y);
          u[16 * t + 4 * q4 + 2] = fmaf(s_cur[t][4 * q4 + 2], C, bb.z);
          u[16 * t + 4 * q4 + 3] = fmaf(s_cur[t][4 * q4 + 3], C, bb.w);
        }
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) u[16 * t + r] = s_cur[t][r] * C;
      }
    }
    if (key0 + kTN > S) {
#pragma unroll
      for (int j = 0; j < 32; ++j)
        if (key0 + 32 * (j >> 4) + 16 * g + (j & 15) >= S) u[j] = -INFINITY;
    }
    float bmax = u[0];
#pragma unroll
    for (int j = 1; j < 32; ++j) bmax = fmaxf(bmax, u[j]);
    bmax = xor32_max(bmax);

    // ---- row max, P in quantised units, row sum ----------------------------------
    float alpha, m_new;
    float pq[32];
    float s_lp;          // P_deq = code * s_lp
    int pe = 127;        // E8M0 of the MX P scale
    float sig_p = 1.0f;  // fp32 P scale carried by the accumulator (dynamic)
    float psum = 0.0f;   // this lane's sum of the pre-quant p
    if constexpr (!BLASST) {
      float T;
      if constexpr (HAS_EST && P_MODE == 2) {
        if (dyn_est) {
          const bool lzero = (l == 0.0f) && (__shfl_xor(l, 32, 64) == 0.0f);
          const float ms = fmaxf(max_seen, bmax);
          const bool under = (bmax - m2) > 16.0f;
          const bool over = (m2 - ms) > 32.0f;
          const float down = lzero ? ms : fmaxf(ms + 32.0f, m2 - 80.0f * kLog2e);
          const bool adjust = under || over;
          m_new = adjust ? (under ? bmax : down) : m2;
          alpha = adjust ? (lzero ? 0.0f : fast_exp2(m2 - m_new)) : 1.0f;
          max_seen = ms;
        } else {
          m_new = est2;
          alpha = 1.0f;
        }
      } else if constexpr (HAS_EST) {
        m_new = est2;
        alpha = 1.0f;
      } else {
        m_new = fmaxf(m2, bmax);
        alpha = fast_exp2(m2 - m_new);
      }
      if constexpr (P_MODE == 0) {
        T = m_new - off;
        s_lp = 1.0f;
      } else if constexpr (P_MODE == 1) {
        const float ra = fmaxf(fast_exp2(bmax - m_new), kAmaxFloor);
        int e = ceil_log2_exact(ra / kFp8Max);
        e = e < -127 ? -127 : (e > 127 ? 127 : e);
        T = m_new + static_cast<float>(e);
        s_lp = __uint_as_float(static_cast<uint32_t>(e + 127) << 23);
        pe = e + 127;
      } else {
        const float ra = fast_exp2(bmax - m_new);
        const bool floored = !(ra > 1e-12f);
        s_lp = (floored ? 1e-12f : ra) * (1.0f / kFp8Max);
        T = (floored ? m_new + kLog2DynFloor : bmax) - kLog2Fp8Max;
        sig_p = s_lp;
      }
#pragma unroll
      for (int j = 0; j < 32; ++j) {
        pq[j] = fast_exp2(u[j] - T);
        psum += pq[j];
      }
      if constexpr (P_MODE == 0) {
        if (HAS_EST || a.p_max_offset > 8) {  // p may exceed 448: satfinite cast
#pragma unroll
          for (int j = 0; j < 32; ++j) pq[j] = fminf(pq[j], kFp8Max);
        }
      }
      psum *= s_lp;  // sum of the pre-quant p
    } else {
      // BLASST: explicit p (fills replace skipped rows), then the P scale of the
      // resulting row, exactly in the reference order.
      const float mij = fmaxf(m2, bmax);
      const bool skip = qvalid && (bmax - mij) < a.log2_lam;
      alpha = skip ? 1.0f : fast_exp2(m2 - mij);
      m_new = skip ? m2 : mij;
      if (g == 0) { skipped += skip ? 1.0f : 0.0f; total += qvalid ? 1.0f : 0.0f; }
      const float c0 = off - m_new;
#pragma unroll
      for (int j = 0; j < 32; ++j) pq[j] = fast_exp2(u[j] + c0);
      if (__any(skip)) {
        float fillv[32];
        blasst_fill_values<P_MODE>(a, u, m_new, bmax, off, g, key0, fillv);
        if (skip) {
#pragma unroll
          for (int j = 0; j < 32; ++j) pq[j] = fillv[j];
        }
      }
#pragma unroll
      for (int j = 0; j < 32; ++j) psum += pq[j];
      s_lp = 1.0f;
      float qmul = 1.0f;
      if constexpr (P_MODE == 1) {
        float pa = 0.0f;
#pragma unroll
        for (int j = 0; j < 32; ++j) pa = fmaxf(pa, pq[j]);
        pa = fmaxf(xor32_max(pa), kAmaxFloor);
        int e = ceil_log2_exact(pa / kFp8Max);
        e = e < -127 ? -127 : (e > 127 ? 127 : e);
        pe = e + 127;
        qmul = __uint_as_float(static_cast<uint32_t>(127 - e) << 23);
        s_lp = __uint_as_float(static_cast<uint32_t>(e + 127) << 23);
      } else if constexpr (P_MODE == 2) {
        float pa = 0.0f;
#pragma unroll
        for (int j = 0; j < 32; ++j) pa = fmaxf(pa, pq[j]);
        pa = fmaxf(xor32_max(pa), 1e-12f);
        s_lp = pa / kFp8Max;
        sig_p = s_lp;
        qmul = kFp8Max / pa;
      }
#pragma unroll
      for (int j = 0; j < 32; ++j) pq[j] = fminf(pq[j] * qmul, kFp8Max);
    }
    l = l * alpha + psum;

    v8i pop;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      int wd = __builtin_amdgcn_cvt_pk_fp8_f32(pq[4 * q], pq[4 * q + 1], 0, false);
      wd = __builtin_amdgcn_cvt_pk_fp8_f32(pq[4 * q + 2], pq[4 * q + 3], wd, true);
      pop[q] = wd;
    }

    // ---- accumulator rescale (alpha, dynamic P scale, fp8_block V scale) ---------
    const VMeta<D>& vm = vmeta[cur];
    float sig_new = sig_p;
    if (a.v_kind == 1) sig_new *= vm.vsc;
    const float f = alpha * sigma * __builtin_amdgcn_rcpf(sig_new);
    sigma = sig_new;
    if (P_MODE == 2 || __any(f != 1.0f)) {
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[db][r] *= f;
    }

    // ---- O^T += V^T P^T (E8M0 scales: MX V columns, MX P; 127 = 1 otherwise) -------
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const int r = 32 * db + li;
      const uint8_t* vp = &v_lds[cur][r * kTN];
      v8i va = lds_read32(vp + 16 * (g ^ swz_v(r)), vp + 16 * ((2 + g) ^ swz_v(r)));
      const int ve = static_cast<int>((vm.ve[(32 * db + li) >> 2] >> (8 * (li & 3))) & 0xff);
      acc[db] = mfma32<true>(va, pop, acc[db], ve, pe);
    }

    // ---- V-smoothing accumulator: c = c * alpha + rowsum(P_deq) (x) alpha_v -------
    if constexpr (VALPHA) {
      float cs = 0.0f;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int wd = pop[q];
        cs += __builtin_amdgcn_cvt_f32_fp8(wd, 0) + __builtin_amdgcn_cvt_f32_fp8(wd, 1) +
              __builtin_amdgcn_cvt_f32_fp8(wd, 2) + __builtin_amdgcn_cvt_f32_fp8(wd, 3);
      }
      const float rs = xor32_add(cs) * s_lp;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int d = 32 * db + 8 * (r >> 2) + 4 * g + (r & 3);
          cacc[db][r] = fmaf(rs, vm.valpha[d], cacc[db][r] * alpha);
        }
    }
    m2 = m_new;

    lds_publish();
  };
  for (int it = 0; it < nt; ++it) {
    step(it, s_a, s_b);
#pragma unroll
    for (int t = 0; t < 2; ++t) s_a[t] = s_b[t];
  }

  // ---- epilogue ---------------------------------------------------------------------
  const float lfull = xor32_add(l);
  if constexpr (BLASST) {
    if (a.stats && g == 0 && qvalid) {
      const int rb = qi / a.block_m;
      atomicAdd(a.stats + (static_cast<size_t>(rb) * (a.B * a.H) + bh) * 2 + 0, skipped);
      atomicAdd(a.stats + (static_cast<size_t>(rb) * (a.B * a.H) + bh) * 2 + 1, total);
    }
  }
  if (!qvalid) return;
  const float inv_l = 1.0f / lfull;
  const int orow = a.out_row_map ? a.out_row_map[static_cast<size_t>(bh) * S + qi] : qi;
  const size_t obase = ((static_cast<size_t>(b) * S + orow) * a.H + h) * D;
  const float* vch = a.v_kind == 0 ? reinterpret_cast<const float*>(a.v_scale) + static_cast<size_t>(bh) * D : nullptr;
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const int d0 = 32 * db + 8 * r4 + 4 * g;
      float o[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        float mainv = acc[db][4 * r4 + k] * sigma;
        if (vch) mainv *= vch[d0 + k];
        if constexpr (VALPHA) mainv += cacc[db][4 * r4 + k];
        // the reference writes a bf16 BHSD tensor, then casts to the output dtype
        o[k] = bf16_bits_to_f32(f32_to_bf16_bits(mainv * inv_l));
      }
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

// Launch one instantiation (defined in the per-P-mode translation units).
int launch_p0(const KArgs& a, int D, bool qk_mx, int rb, bool blasst, bool valpha, hipStream_t st);
int launch_p1(const KArgs& a, int D, bool qk_mx, int rb, bool blasst, bool valpha, hipStream_t st);
int launch_p2(const KArgs& a, int D, bool qk_mx, int rb, bool blasst, bool valpha, hipStream_t st);

template <int P_MODE>
int launch_p(const KArgs& a, int D, bool qk_mx, int rb, bool blasst, bool valpha, hipStream_t st) {
  const int nblk = a.B * a.H * a.nqb;
  dim3 grid(static_cast<unsigned>(nblk)), block(kThreads);
#define LBFQ_L(DD, MX, RBV, BL, VA) \
  hipLaunchKernelGGL((attn_fwd_kernel<DD, MX, P_MODE, RBV, BL, VA>), grid, block, 0, st, a)
#define LBFQ_VA(DD, MX, RBV, BL) \
  if (valpha) LBFQ_L(DD, MX, RBV, BL, true); else LBFQ_L(DD, MX, RBV, BL, false)
#define LBFQ_BL(DD, MX, RBV) \
  if (blasst) { LBFQ_VA(DD, MX, RBV, true); } else { LBFQ_VA(DD, MX, RBV, false); }
#define LBFQ_RB(DD, MX)                    \
  if (rb == RB_ONLINE) { LBFQ_BL(DD, MX, RB_ONLINE) }            \
  else if (rb == RB_ONLINE_BIAS) { LBFQ_BL(DD, MX, RB_ONLINE_BIAS) } \
  else { LBFQ_BL(DD, MX, RB_EST_BIAS) }
#define LBFQ_MX(DD) \
  if (qk_mx) { LBFQ_RB(DD, true) } else { LBFQ_RB(DD, false) }
  if (D == 128) { LBFQ_MX(128) } else { LBFQ_MX(64) }
#undef LBFQ_MX
#undef LBFQ_RB
#undef LBFQ_BL
#undef LBFQ_VA
#undef LBFQ_L
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    lbfq_set_error("lbfq_attention_fwd: launch failed: %s", hipGetErrorString(e));
    return -2;
  }
  return 0;
}

}  // namespace lbfq_attn
