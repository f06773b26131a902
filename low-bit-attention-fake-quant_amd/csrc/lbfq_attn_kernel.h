// FP8-MFMA P-requant attention for gfx950 (CDNA4): templated kernel body.
//
// Reference semantics: the K-loop of _fake_quant_attn_fwd_kernel
// (attention_triton.py:109-407).  The reference dequantises Q/K/V to bf16 and
// runs bf16 dots; this kernel multiplies the FP8 codes on the matrix cores
// (v_mfma[_scale]_f32_32x32x64_f8f6f4) and applies the scales outside, or
// through the E8M0 block scales of the MFMA for the MX formats.
//
// Work decomposition: one workgroup = NW waves = 32 NW queries of one (b, h)
// (NW = 4, or 8 for the dense fp8_block D = 128 kernels); each wave owns 32
// queries.  K and V^T tiles of 64 keys (== the reference block_n) are copied
// global -> LDS directly (four-slot K and V^T rings, staged three and two
// tiles ahead) together with the per-tile metadata (qm correction row, K/V
// scales, V block means), and shared by the workgroup's waves.  Scores are computed transposed, S^T = K Q^T, so every lane owns
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
//
// Schedule of one tile step (per wave): the softmax of tile t runs in four
// chunks of 8 keys per lane; each chunk carries one or two MFMAs that do not
// depend on it -- the PV of tile t-1 (P codes kept in registers) and the QK of
// tile t+1 (written into score registers the earlier chunks have consumed).
// On gfx950 independent VALU work of either wave of a SIMD issues while a
// 32x32x64 MFMA runs (each MFMA takes ~15-20 cycles of VALU issue), and the
// softmax of a tile needs more VALU cycles than its MFMAs need matrix cycles
// (exp, the FP8 conversion and permlane take 8 cycles per wave instruction,
// fma / max 4, add / mul / mov 2-4), so a tile costs about its VALU cycles;
// the interleave keeps the wave from idling on its own LDS reads and MFMA
// results.  Empty asm fences (pin / use) and sched_barrier keep each chunk's
// work together, and all LDS reads of a step are issued before the first
// instruction that waits on any of them.
#pragma once

#include <cstddef>
#include <type_traits>

#include "lbfq_common.h"
#include "../../include/lbfq.h"

namespace lbfq_attn {

using namespace lbfq;

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLog2Fp8Max = 8.807354922057604f;     // log2(448)
constexpr float kLog2DynFloor = -39.86313713864835f;  // log2(1e-12)
// Waves per workgroup: 4 (128 queries), or 8 (256 queries, one workgroup per
// CU) for the kernels launch_p picks them for; the 4-wave figures below are
// what the host requires of every call (s_pitch a multiple of kQB).
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
  float* row_skips;
  int* wave_tiles;
  const float* vcol;  // (B*H, P/64, D) V tile column sums, or null
  const float* rowmax_init;  // (B*H, S) initial row max, log2 units (kernel row order), or null
  void* out;
  int out_dtype;
  const int32_t* out_row_map;
};

// Per-tile metadata staged in LDS next to the K / V^T codes.  The K side is
// consumed by the softmax of the tile, the V side by its PV product.
template <int NW>
struct KMeta {
  float bias[NW][kTN];      // qm correction (log2 units) of each wave's group
  uint32_t ke[kTN];         // MX: E8M0 bytes of the keys' D/32 chunks
  float ksc[kTN];           // fp8_block: scale of the 16-key group of each key
};

template <int D, bool COLSUM>
struct VMeta {
  uint32_t ve[kTN];         // E8M0 byte of each V column (4 per word, D/4 words); 127 unless V is MX
  float valpha[D];          // V block mean of the tile
  float vsc[kTN];           // fp8_block V scale of the tile (all entries equal)
  float vcol[COLSUM ? D : 1];  // sum over the tile's keys of each V column (codes, MX-scaled)
};

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Max of raw scores (v_max3_f32 / v_max_f32).  These must stay visible to the
// compiler: the scores are MFMA results, and on gfx950 a VALU instruction may
// read the destination of a 16-pass XDL MFMA only 20 wait states after it
// issues.  The compiler inserts those wait states for its own instructions but
// never inspects the operands that inline asm reads, so a max written as asm
// can read a partly written accumulator (a wrong row max, then inf / NaN
// rows, depending on timing).  With this compiler fmaxf needs no
// canonicalisation of MFMA results, lane exchanges or loop-carried values.
__device__ __forceinline__ float hmax3(float a, float b, float c) { return fmaxf(fmaxf(a, b), c); }
__device__ __forceinline__ float hmax(float a, float b) { return fmaxf(a, b); }

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
// Addressing: wave-uniform 64-bit global base (SGPRs) + per-lane 32-bit byte
// offset, LDS base as a wave-uniform byte address.
// On GFX9-family parts (gfx950 included) an LDS DMA that reads M0 right after
// an SALU write of M0 needs one wait state; the compiler's hazard recognizer
// cannot see inside inline asm, so each copy carries its own s_nop 0 (else the
// copy may use the previous M0 and land in the previous copy's LDS slot).
// build_lib.py rejects any object in which an M0 write directly precedes an
// LDS DMA.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p)));
}
__device__ __forceinline__ void g2l16(const void* gbase, uint32_t vofs, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(vofs), "s"(gbase),
               "s"(lds_base)
               : "memory", "m0");
}
__device__ __forceinline__ void g2l4(const void* gbase, uint32_t vofs, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(vofs), "s"(gbase),
               "s"(lds_base)
               : "memory", "m0");
}
// Scheduling fences for register values (no instruction is emitted): pin(x)
// makes x look redefined here, so work that reads it cannot start earlier;
// use(x) makes x look read here, so the work that produces it cannot sink
// below.  Between sched_barrier(0) fences they hold a chunk of independent
// VALU and MFMA work together, so one wave issues both side by side.
// (The host pass type-checks device code too and has no "v" registers.)
template <typename T>
__device__ __forceinline__ void pin(T& x) {
#if defined(__HIP_DEVICE_COMPILE__)
  asm volatile("" : "+v"(x));
#endif
}
template <typename T>
__device__ __forceinline__ void use(const T& x) {
#if defined(__HIP_DEVICE_COMPILE__)
  asm volatile("" ::"v"(x));
#endif
}

// Wait until at most N of this wave's global -> LDS copies are in flight (the
// ones issued during the current tile), then the workgroup barrier: every
// copy issued one tile earlier has landed for every wave.
template <int N>
__device__ __forceinline__ void lds_publish() {
  static_assert(N >= 0 && N < 16, "vmcnt immediate");
  __builtin_amdgcn_s_waitcnt(0x0F70 | N);  // vmcnt(N), expcnt / lgkmcnt unconstrained
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

// Combine lane l with lane l ^ 32: v_permlane32_swap exchanges the upper half
// of its first operand with the lower half of its second, so (r0, r1) hold
// (v[l], v[l^32]) in one order or the other, and max / sum of the pair is the
// same in both halves of the wave.
__device__ __forceinline__ float xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return hmax(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_add(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// ---- BLASST fill values (attention_triton.py:229-324) in the lane layout -----
// A skipped row keeps no exact p; its valid keys get a fill, in p units (which
// include the elementwise p_max_offset "off", as in the reference).  Scores u
// are in log2 units (-inf where masked), so the reference's natural-log
// statistics become: (mean_nat - m_nat) * log2e = mean(u) - m and
// var_nat * log2e = var(u) * ln2.  Sums run over the lane's 32 keys, then over
// the lane pair (l, l ^ 32) that holds the rest of the 64-key row.  All of it
// is select-based (no divergent branches); divides by counts go through a
// reciprocal, so fills agree with the reference to float rounding.  Each
// function writes fp[j] (0 on masked keys) and returns the row's largest fill.
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ float valid_or(float u, float other) { return u != -INFINITY ? u : other; }

// UTA bins of BS keys (attention_triton.py:292-323): per bin, from its count,
// mean and max, fill = min(fa * cnt * 2^(mean-m+off), cnt * 2^(max-m+off)) / cnt.
// BS <= 16: a bin is a run of BS consecutive keys of the lane; 32: one 16-key
// run of each lane of the pair; 64: both runs of both.
template <int BS>
__device__ __forceinline__ float uta_fill(const float (&u)[32], float m_new, float off, float fa, float (&fp)[32]) {
  constexpr int RUN = BS <= 16 ? BS : 16;  // lane-local keys per run
  constexpr int NR = 32 / RUN;            // runs of the lane
  float s[NR], mx[NR], c[NR];
#pragma unroll
  for (int b = 0; b < NR; ++b) {
    s[b] = 0.0f; mx[b] = -INFINITY; c[b] = 0.0f;
#pragma unroll
    for (int r = 0; r < RUN; ++r) {
      const float x = u[RUN * b + r];
      s[b] += valid_or(x, 0.0f);
      mx[b] = hmax(mx[b], x);
      c[b] += x != -INFINITY ? 1.0f : 0.0f;
    }
    if constexpr (BS >= 32) {
      s[b] = xor32_add(s[b]);
      mx[b] = xor32_max(mx[b]);
      c[b] = xor32_add(c[b]);
    }
  }
  if constexpr (BS == 64) {
    s[0] += s[1]; mx[0] = hmax(mx[0], mx[1]); c[0] += c[1];
    s[1] = s[0]; mx[1] = mx[0]; c[1] = c[0];
  }
  float fmx = 0.0f;
#pragma unroll
  for (int b = 0; b < NR; ++b) {
    const float sc = fmaxf(c[b], 1.0f), rc = __builtin_amdgcn_rcpf(sc);
    const float f = fminf(fa * sc * fast_exp2(s[b] * rc - m_new + off), sc * fast_exp2(mx[b] - m_new + off)) * rc;
    fmx = fmaxf(fmx, f);
#pragma unroll
    for (int r = 0; r < RUN; ++r) fp[RUN * b + r] = u[RUN * b + r] != -INFINITY ? f : 0.0f;
  }
  return xor32_max(fmx);
}

// Fills with one value per row and tile (zero, max, mean, logn, sample8, thr):
// the value f of the row's valid keys (the keys of a full tile are all valid),
// computed from the scores in place (u = score * C), as blasst_fill does.
template <int P_MODE, bool MASKED>
__device__ __forceinline__ float blasst_row_fill(const KArgs& a, const v16f (&sc)[2], const float (&Ct)[2],
                                                 float m_new, float bmax, float off, int key0) {
  const int fk = a.fill_kind;
  const float fa = a.fill_alpha;
  // valid keys of the row (uniform): a full tile's 64 (1/64 is exact), fewer only in the masked last tile
  const int nv = MASKED ? (a.S - key0 < kTN ? a.S - key0 : kTN) : kTN;
  const float n = static_cast<float>(nv), rn = MASKED ? 1.0f / n : 1.0f / kTN;
  const float max_bound = n * fast_exp2(bmax - m_new + off);
  float f = 0.0f;  // FILL_ZERO
  if (fk == FILL_MAX) {
    f = max_bound * fa * rn;
  } else if (fk == FILL_MEAN || fk == FILL_LOGN) {
    // the scores of a full tile are all finite: each 16-key group's sum is
    // taken in accumulator units (pairwise) and scaled by its C once
    float s;
    if constexpr (MASKED) {
      s = 0.0f;
#pragma unroll
      for (int j = 0; j < 32; ++j) s += valid_or(sc[j >> 4][j & 15] * Ct[j >> 4], 0.0f);
    } else {
      float h[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        float p8[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) p8[r] = sc[t][r] + sc[t][r + 8];
#pragma unroll
        for (int r = 0; r < 4; ++r) p8[r] += p8[r + 4];
        h[t] = (p8[0] + p8[2]) + (p8[1] + p8[3]);
      }
      s = fmaf(h[0], Ct[0], h[1] * Ct[1]);
    }
    const float mean = xor32_add(s) * rn;  // log2 units
    if (fk == FILL_MEAN) {
      f = fminf(fa * n * fast_exp2(mean - m_new + off), max_bound) * rn;
    } else {
      float vs = 0.0f;
#pragma unroll
      for (int j = 0; j < 32; ++j) {
        float c = fmaf(sc[j >> 4][j & 15], Ct[j >> 4], -mean);
        if constexpr (MASKED) c = valid_or(c, 0.0f);
        vs = fmaf(c, c, vs);
      }
      const float var2 = xor32_add(vs) * rn;  // log2 units squared
      f = fminf(n * fast_exp2(mean + 0.5f * var2 * kLn2 - m_new + off), max_bound) * rn;
    }
  } else if (fk == FILL_SAMPLE8) {
    const float c0 = off - m_new;
    const float sp = xor32_add(fast_exp2(sc[0][0] * Ct[0] + c0) + fast_exp2(sc[0][8] * Ct[0] + c0) +
                               fast_exp2(sc[1][0] * Ct[1] + c0) + fast_exp2(sc[1][8] * Ct[1] + c0));
    const float cnt = static_cast<float>((nv + 7) / 8);
    f = fminf(fa * n * sp / cnt, max_bound) * rn;
  } else if (fk == FILL_THR) {
    const float offs = P_MODE == 0 ? exp2f(static_cast<float>(a.p_max_offset)) : 1.0f;
    f = fa * n * a.lam * offs * rn;
  }
  return f;
}

// UTA fill with at most 16 bins (runs of >= 4 keys, at most 8 per lane):
// uta_runs computes the fill of each of the lane's runs (the arithmetic of
// uta_fill, with the scores read in place) and returns the row's largest;
// uta_pack turns them into the lane's E4M3 fill codes, 4 keys per word in the
// order of the P codes, and their sum in the order of the exact row sum.
// In a full tile every bin holds its BS keys (a power of two), so a run's
// scores are summed in accumulator units and scaled by its C once, the counts
// cancel exactly (fa * cnt * x / cnt == fa * x), and a run's four-key words
// share one code.
template <int BS, bool MASKED>
__device__ __forceinline__ float uta_runs(const v16f (&sc)[2], const float (&Ct)[2], float m_new, float off,
                                          float fa, float (&fr)[8]) {
  constexpr int RUN = BS <= 16 ? BS : 16;
  constexpr int NR = 32 / RUN;
  static_assert(NR <= 8 && RUN >= 4, "uta_runs: 4 to 16 keys per run");
  float fmx = 0.0f;
  if constexpr (!MASKED) {
    float s[NR], mx[NR];
#pragma unroll
    for (int b = 0; b < NR; ++b) {
      const int t = (RUN * b) >> 4, r0 = (RUN * b) & 15;
      float p[RUN / 2];
#pragma unroll
      for (int r = 0; r < RUN / 2; ++r) p[r] = sc[t][r0 + r] + sc[t][r0 + r + RUN / 2];
#pragma unroll
      for (int w = RUN / 4; w >= 1; w /= 2)
#pragma unroll
        for (int r = 0; r < w; ++r) p[r] += p[r + w];
      float m = hmax(sc[t][r0], sc[t][r0 + 1]);
#pragma unroll
      for (int r = 2; r + 1 < RUN; r += 2) m = hmax3(m, sc[t][r0 + r], sc[t][r0 + r + 1]);
      s[b] = p[0] * Ct[t];
      mx[b] = m * Ct[t];  // C > 0
      if constexpr (BS >= 32) {
        s[b] = xor32_add(s[b]);
        mx[b] = xor32_max(mx[b]);
      }
    }
    if constexpr (BS == 64) {
      s[0] += s[1]; mx[0] = hmax(mx[0], mx[1]);
      s[1] = s[0]; mx[1] = mx[0];
    }
    constexpr float inv = 1.0f / BS;
#pragma unroll
    for (int b = 0; b < NR; ++b) {
      const float f = fminf(fa * fast_exp2(s[b] * inv - m_new + off), fast_exp2(mx[b] - m_new + off));
      fmx = fmaxf(fmx, f);
      fr[b] = f;
    }
  } else {
    float s[NR], mx[NR], c[NR];
#pragma unroll
    for (int b = 0; b < NR; ++b) {
      s[b] = 0.0f; mx[b] = -INFINITY; c[b] = 0.0f;
#pragma unroll
      for (int r = 0; r < RUN; ++r) {
        const int j = RUN * b + r;
        const float x = sc[j >> 4][j & 15] * Ct[j >> 4];
        s[b] += valid_or(x, 0.0f);
        mx[b] = hmax(mx[b], x);
        c[b] += x != -INFINITY ? 1.0f : 0.0f;
      }
      if constexpr (BS >= 32) {
        s[b] = xor32_add(s[b]);
        mx[b] = xor32_max(mx[b]);
        c[b] = xor32_add(c[b]);
      }
    }
    if constexpr (BS == 64) {
      s[0] += s[1]; mx[0] = hmax(mx[0], mx[1]); c[0] += c[1];
      s[1] = s[0]; mx[1] = mx[0]; c[1] = c[0];
    }
#pragma unroll
    for (int b = 0; b < NR; ++b) {
      const float sc_b = fmaxf(c[b], 1.0f), rc = __builtin_amdgcn_rcpf(sc_b);
      const float f = fminf(fa * sc_b * fast_exp2(s[b] * rc - m_new + off), sc_b * fast_exp2(mx[b] - m_new + off)) * rc;
      fmx = fmaxf(fmx, f);
      fr[b] = f;
    }
  }
  return xor32_max(fmx);
}

template <int BS, int P_MODE, bool MASKED>
__device__ __forceinline__ void uta_pack(const v16f (&sc)[2], const float (&fr)[8], float qmul_f, uint32_t (&fpk)[8],
                                         float& fsum) {
  constexpr int RUN = BS <= 16 ? BS : 16;
  constexpr int NR = 32 / RUN;
  if constexpr (!MASKED) {
    float v[NR];
    uint32_t wd[NR];
#pragma unroll
    for (int b = 0; b < NR; ++b) {
      v[b] = P_MODE == 0 ? fminf(fr[b], kFp8Max) : fr[b] * qmul_f;
      const int w2 = __builtin_amdgcn_cvt_pk_fp8_f32(v[b], v[b], __float_as_int(v[b]), false);
      wd[b] = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(v[b], v[b], w2, true));
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) fpk[q] = wd[(4 * q) / RUN];
    float t = v[0];
#pragma unroll
    for (int b = 1; b < NR; ++b) t += v[b];
    fsum = t * static_cast<float>(RUN);
  } else {
    float s4[4];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = 4 * q + i;
        const float f = sc[j >> 4][j & 15] != -INFINITY ? fr[j / RUN] : 0.0f;
        v[i] = P_MODE == 0 ? fminf(f, kFp8Max) : f * qmul_f;
        s4[i] = q == 0 ? v[i] : s4[i] + v[i];
      }
      int wd = __builtin_amdgcn_cvt_pk_fp8_f32(v[0], v[1], __float_as_int(v[0]), false);
      fpk[q] = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(v[2], v[3], wd, true));
    }
    fsum = (s4[0] + s4[1]) + (s4[2] + s4[3]);
  }
}

template <int P_MODE>
__device__ __forceinline__ float blasst_fill(const KArgs& a, const float (&u)[32], float m_new, float bmax, float off,
                                             int key0, float (&fp)[32]) {
  const int fk = a.fill_kind;
  const float fa = a.fill_alpha;
  if (fk == FILL_UTA) {
    switch (kTN / a.uta_bins) {
      case 1: return uta_fill<1>(u, m_new, off, fa, fp);
      case 2: return uta_fill<2>(u, m_new, off, fa, fp);
      case 4: return uta_fill<4>(u, m_new, off, fa, fp);
      case 8: return uta_fill<8>(u, m_new, off, fa, fp);
      case 16: return uta_fill<16>(u, m_new, off, fa, fp);
      case 32: return uta_fill<32>(u, m_new, off, fa, fp);
      default: return uta_fill<64>(u, m_new, off, fa, fp);
    }
  }
  const int nv = a.S - key0 < kTN ? a.S - key0 : kTN;  // valid keys of the row (uniform)
  const float n = static_cast<float>(nv), rn = 1.0f / n;
  const float max_bound = n * fast_exp2(bmax - m_new + off);
  float f = 0.0f;  // FILL_ZERO
  if (fk == FILL_MAX) {
    f = max_bound * fa * rn;
  } else if (fk == FILL_MEAN || fk == FILL_LOGN) {
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; ++j) s += valid_or(u[j], 0.0f);
    const float mean = xor32_add(s) * rn;  // log2 units
    if (fk == FILL_MEAN) {
      f = fminf(fa * n * fast_exp2(mean - m_new + off), max_bound) * rn;
    } else {
      float vs = 0.0f;
#pragma unroll
      for (int j = 0; j < 32; ++j) {
        const float c = valid_or(u[j] - mean, 0.0f);
        vs = fmaf(c, c, vs);
      }
      const float var2 = xor32_add(vs) * rn;  // log2 units squared
      f = fminf(n * fast_exp2(mean + 0.5f * var2 * kLn2 - m_new + off), max_bound) * rn;
    }
  } else if (fk == FILL_SAMPLE8) {
    // sampled keys: rel % 8 == 0, i.e. r in {0, 8} of both 16-key runs of the lane
    const float c0 = off - m_new;
    const float sp = xor32_add(fast_exp2(u[0] + c0) + fast_exp2(u[8] + c0) + fast_exp2(u[16] + c0) +
                               fast_exp2(u[24] + c0));
    const float cnt = static_cast<float>((nv + 7) / 8);
    f = fminf(fa * n * sp / cnt, max_bound) * rn;
  } else if (fk == FILL_THR) {
    const float offs = P_MODE == 0 ? exp2f(static_cast<float>(a.p_max_offset)) : 1.0f;
    f = fa * n * a.lam * offs * rn;
  }
#pragma unroll
  for (int j = 0; j < 32; ++j) fp[j] = u[j] != -INFINITY ? f : 0.0f;
  return f;
}


// ---- BLASST fills over a 128-key block (block_n = 128) ----------------------
// The lane holds 64 keys of the row in four 16-key groups: group k = 2 tt + t
// (tile tt of the block, 32-key half t), keys key0 + 64 tt + 32 t + 16 g + r.
// Same formulas as the 64-key fills; sample8 takes the keys with
// rel % 16 == 0 (r == 0; BLOCK_N / 8 = 16, attention_triton.py:270-276).
template <int P_MODE, bool MASKED>
__device__ __forceinline__ float blasst_row_fill128(const KArgs& a, const v16f (&s4)[4], const float (&C4)[4],
                                                    float m_new, float bmax, float off, int key0) {
  const int fk = a.fill_kind;
  const float fa = a.fill_alpha;
  const int nv = MASKED ? (a.S - key0 < 128 ? a.S - key0 : 128) : 128;
  const float n = static_cast<float>(nv), rn = MASKED ? 1.0f / n : 1.0f / 128.0f;
  const float max_bound = n * fast_exp2(bmax - m_new + off);
  float f = 0.0f;  // FILL_ZERO
  if (fk == FILL_MAX) {
    f = max_bound * fa * rn;
  } else if (fk == FILL_MEAN || fk == FILL_LOGN) {
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if constexpr (MASKED) {
#pragma unroll
        for (int r = 0; r < 16; ++r) s += valid_or(s4[k][r] * C4[k], 0.0f);
      } else {
        float p8[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) p8[r] = s4[k][r] + s4[k][r + 8];
#pragma unroll
        for (int r = 0; r < 4; ++r) p8[r] += p8[r + 4];
        s = fmaf((p8[0] + p8[2]) + (p8[1] + p8[3]), C4[k], s);
      }
    }
    const float mean = xor32_add(s) * rn;  // log2 units
    if (fk == FILL_MEAN) {
      f = fminf(fa * n * fast_exp2(mean - m_new + off), max_bound) * rn;
    } else {
      float vs = 0.0f;
#pragma unroll
      for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float c = fmaf(s4[k][r], C4[k], -mean);
          if constexpr (MASKED) c = valid_or(c, 0.0f);
          vs = fmaf(c, c, vs);
        }
      const float var2 = xor32_add(vs) * rn;  // log2 units squared
      f = fminf(n * fast_exp2(mean + 0.5f * var2 * kLn2 - m_new + off), max_bound) * rn;
    }
  } else if (fk == FILL_SAMPLE8) {
    const float c0 = off - m_new;
    float sp = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) sp += fast_exp2(s4[k][0] * C4[k] + c0);
    sp = xor32_add(sp);
    const float cnt = static_cast<float>((nv + 15) / 16);
    f = fminf(fa * n * sp / cnt, max_bound) * rn;
  } else if (fk == FILL_THR) {
    const float offs = P_MODE == 0 ? exp2f(static_cast<float>(a.p_max_offset)) : 1.0f;
    f = fa * n * a.lam * offs * rn;
  }
  return f;
}

// UTA over a 128-key block, bins of BS = 128 / bins keys: the fill of each
// run of min(BS, 16) lane keys (runs of a bin that spans groups or both lanes
// of the row share the bin's statistics) into fr[0 .. 64 / RUN); returns the
// row's largest fill.
template <int BS, bool MASKED>
__device__ __forceinline__ float uta128_runs(const v16f (&s4)[4], const float (&C4)[4], float m_new, float off,
                                             float fa, float (&fr)[64]) {
  constexpr int RUN = BS < 16 ? BS : 16;
  constexpr int NR = 64 / RUN;
  float s[NR], mx[NR], c[NR];
#pragma unroll
  for (int j = 0; j < NR; ++j) {
    const int k = (RUN * j) >> 4, r0 = (RUN * j) & 15;
    s[j] = 0.0f; mx[j] = -INFINITY; c[j] = 0.0f;
#pragma unroll
    for (int r = 0; r < RUN; ++r) {
      const float x = s4[k][r0 + r] * C4[k];
      s[j] += MASKED ? valid_or(x, 0.0f) : x;
      mx[j] = hmax(mx[j], x);
      c[j] += (!MASKED || x != -INFINITY) ? 1.0f : 0.0f;
    }
  }
  if constexpr (BS >= 64) {  // a bin spans the groups of a tile (64) or of the block (128)
    constexpr int G = BS / 32;  // lane groups per bin
#pragma unroll
    for (int j = 0; j < NR; j += G) {
#pragma unroll
      for (int i = 1; i < G; ++i) { s[j] += s[j + i]; mx[j] = hmax(mx[j], mx[j + i]); c[j] += c[j + i]; }
#pragma unroll
      for (int i = 1; i < G; ++i) { s[j + i] = s[j]; mx[j + i] = mx[j]; c[j + i] = c[j]; }
    }
  }
  if constexpr (BS >= 32) {  // and both lanes of the row
#pragma unroll
    for (int j = 0; j < NR; ++j) { s[j] = xor32_add(s[j]); mx[j] = xor32_max(mx[j]); c[j] = xor32_add(c[j]); }
  }
  float fmx = 0.0f;
#pragma unroll
  for (int j = 0; j < NR; ++j) {
    const float sc_b = fmaxf(c[j], 1.0f), rc = __builtin_amdgcn_rcpf(sc_b);
    const float f = fminf(fa * sc_b * fast_exp2(s[j] * rc - m_new + off), sc_b * fast_exp2(mx[j] - m_new + off)) * rc;
    fmx = fmaxf(fmx, f);
    fr[j] = f;
  }
  return xor32_max(fmx);
}

// The lane's UTA fill codes of both tiles (fpk[8 tt + q]: keys 4q..4q+3 of
// tile tt, in the order of the P codes) and the sum of its pre-quant fills.
template <int BS, int P_MODE>
__device__ __forceinline__ void uta128_pack(const v16f (&s4)[4], const float (&fr)[64], float qmul_f,
                                            uint32_t (&fpk)[16], float& fsum) {
  constexpr int RUN = BS < 16 ? BS : 16;
  float sum = 0.0f;
#pragma unroll
  for (int w = 0; w < 16; ++w) {
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int jl = 4 * w + i;  // lane key 32 tt + 16 t + r
      const float f = s4[jl >> 4][jl & 15] != -INFINITY ? fr[jl / RUN] : 0.0f;
      sum += P_MODE == 0 ? f : f * qmul_f;
      v[i] = P_MODE == 0 ? fminf(f, kFp8Max) : f * qmul_f;
    }
    const int wd = __builtin_amdgcn_cvt_pk_fp8_f32(v[0], v[1], __float_as_int(v[0]), false);
    fpk[w] = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(v[2], v[3], wd, true));
  }
  fsum = sum;
}

// BL: BLASST off (0); with a fill of one value per row and tile (1); with the
// UTA fill of at most 16 bins (2: packed fill codes per lane); with the UTA
// fill of 32 or 64 bins (3: one fill code per key in 32 registers, one wave
// per SIMD).  BLASST together with V smoothing also runs one wave per SIMD.
// BN: the reference's block_n, the keys that share one row-max update, one
// P scale and one BLASST decision: 64 (one MFMA tile per step) or 128 (two).
constexpr int attn_waves_per_simd(int d, int p_mode, int rb, int bl, bool valpha, int bn) {
  if (bl == 3 || (bl != 0 && valpha)) return 1;
  if (bn == 128 && bl == 2) return 1;
  // block_n = 128 with a per-row fill fits 256 VGPRs, except the online-row-max
  // variants with a scaled P at D = 128
  if (bn == 128 && bl == 1 && d == 128 && p_mode != 0 && rb == 0) return 1;
  return 2;
}
// V-smoothing correction acc[db][d, q] += valpha[d] * w (w: the lane's query)
// as an outer product on the fp32 matrix cores: v_mfma_f32_32x32x2_f32 with
// A[d][0] = valpha[32 db + d], B[0][q] = w and the K = 1 half (lanes 32-63)
// zero.  Its output layout is the accumulator's, so it replaces 64 VALU FMAs
// per lane (the kernel is VALU-issue-bound, the matrix cores are not).
template <int NDB>
__device__ __forceinline__ void valpha_outer(v16f (&acc)[NDB], const float* valpha, float w, int li, int g) {
  const float bw = g == 0 ? w : 0.0f;
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    const float av = g == 0 ? valpha[32 * db + li] : 0.0f;
    acc[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bw, acc[db], 0, 0, 0);
  }
}

template <int D, bool QK_MX, int P_MODE, int RB, int BL, bool VALPHA, int BN, int NW>
__global__ void __launch_bounds__(NW * 64, attn_waves_per_simd(D, P_MODE, RB, BL, VALPHA, BN)) attn_fwd_kernel(const KArgs a) {
  constexpr int kWaves = NW, kThreads = NW * 64, kQB = NW * 32;  // this kernel's workgroup
  using KMeta = lbfq_attn::KMeta<NW>;
  static_assert(BN == 64 || BN == 128, "block_n is 64 or 128");
  constexpr bool BLASST = BL != 0;
  // BLASST with one fill value per row and tile, without V smoothing: a tile
  // that every row of the wave skips adds fill * (column sums of V) to the
  // accumulator instead of running its four PV MFMAs
  constexpr bool ELIDE = BL == 1 && !VALPHA && BN == 64;
  using VM = VMeta<D, ELIDE>;
  constexpr int NH = D / 64;          // 64-wide contraction halves of D
  constexpr int NDB = D / 32;         // 32-row blocks of O^T
  constexpr int CPT = kTN * D / 16 / kThreads;  // 16-byte chunks per thread per K (and V) tile
  constexpr bool HAS_BIAS = RB != RB_ONLINE;
  constexpr bool HAS_EST = RB == RB_EST_BIAS;

  // rings: K tile i lives in slot i % 4, V^T tile i in slot i % 4 (76 KB at
  // D = 128 with four waves, so two workgroups share a CU; 82 KB with eight).  The main loop runs four tile steps
  // per iteration, so every slot index is a compile-time constant there and
  // the LDS addresses are immediate offsets.
  // One ordered block: the small per-tile tables first, so that every access
  // to them is a base register plus a 16-bit immediate offset (ds_read /
  // ds_write offsets stop at 64 KB), then the rings.
  struct __attribute__((aligned(16))) Smem {
    float binit[HAS_BIAS ? kWaves : 1][2][kTN];  // bias / C per query half
    KMeta kmeta[4];
    VM vmeta[4];
    uint8_t k_lds[4][kTN * D];  // swizzled K rows (key order kperm)
    uint8_t v_lds[4][D * kTN];  // swizzled V^T rows
  };
  __shared__ Smem smem;
  auto& binit = smem.binit;
  auto& kmeta = smem.kmeta;
  auto& vmeta = smem.vmeta;
  auto& k_lds = smem.k_lds;
  auto& v_lds = smem.v_lds;

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
  // rowmax_init (attention_triton.py:127-130): the online max starts at the given value
  if constexpr (!HAS_EST) {
    if (a.rowmax_init && qvalid) m2 = a.rowmax_init[static_cast<size_t>(bh) * S + qi];
  }
  const float est2 = m2;
  const bool dyn_est = HAS_EST && !BLASST && P_MODE == 2 && a.rowmax_dynamic;
  const float off = P_MODE == 0 ? static_cast<float>(a.p_max_offset) : 0.0f;

  float l = 0.0f;  // partial row sum of the pre-quant p over this lane's keys
  float max_seen = -INFINITY;
  float sigma = 1.0f;  // acc holds O^T / sigma
  float skipped = 0.0f;  // BLASST: tiles this row skipped
  int wt_all = 0, wt_any = 0;  // BLASST: tiles every / some row of the wave skipped (wave-uniform)
  v16f acc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[db][r] = 0.0f;
  // The accumulator must never be a known constant at a PV MFMA: with a
  // constant-zero input (e.g. in a peeled first iteration) the compiler does
  // not tie the MFMA's destination to it and may give the destination the
  // register of the V scale operand, which the MFMA still reads.
#pragma unroll
  for (int db = 0; db < NDB; ++db) pin(acc[db]);
  // V smoothing (attention_triton.py c = c * alpha + rowsum(P_deq) (x) alpha_v)
  // is folded into acc: the correction of a tile, rowsum(P_deq) / sigma (x)
  // alpha_v, is added in the same units as the tile's PV product, so the
  // accumulator rescale applies to both.  rowsum(codes) comes from one FP8
  // MFMA of the codes against a constant A = 1.0 (exact in fp32).
  v8i ones;
#pragma unroll
  for (int q = 0; q < 8; ++q) ones[q] = 0x38383838;  // E4M3 1.0
  float vw_prev = 0.0f;  // s_P / sigma of tile it-1 (weight of its correction)

  // ---- tile loader ------------------------------------------------------------
  // K codes, the qm bias rows and the MX K scales are staged three tiles ahead
  // (the scores of tile t are computed during tile t-1), V codes, the MX V
  // column scales and the V block means two tiles ahead, so every copy has a
  // whole tile of compute to land.  All copies go global -> LDS directly;
  // every wave issues the same copies with all 64 lanes (the small tables are
  // copied by every wave, redundantly), so the loop has no lane masks and the
  // publish wait is a compile-time vmcnt.
  uint32_t kofs[CPT], vofs[CPT];
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int sl = c * kThreads + tid;
    const int r = sl / (D / 16), ch = (sl % (D / 16)) ^ swz_k<D>(sl / (D / 16));
    kofs[c] = (32 * (r >> 5) + kperm(r & 31)) * D + ch * 16;
    const int d = sl / (kTN / 16), cv = (sl % (kTN / 16)) ^ swz_v(sl / (kTN / 16));
    vofs[c] = d * P + cv * 16;
  }
  const int nt = (S + kTN - 1) / kTN;
  // wave-uniform pieces of the copy addresses (SGPRs)
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  int bias_grp = 0;
  if constexpr (HAS_BIAS) {
    bias_grp = (qb * kQB + wv * 32) >> a.lg_qgroup;
    if (bias_grp >= a.G) bias_grp = a.G - 1;
  }
  const float* bias_src = HAS_BIAS ? a.bias + (static_cast<size_t>(bh) * a.G + bias_grp) * P : nullptr;
  const uint32_t k_lds0 = lds_addr(&k_lds[0][0]), v_lds0 = lds_addr(&v_lds[0][0]);
  const uint32_t km0 = lds_addr(&kmeta[0]), vm0 = lds_addr(&vmeta[0]);
  constexpr uint32_t kKBuf = kTN * D, kVBuf = D * kTN;
  constexpr uint32_t kKMeta = sizeof(KMeta), kVMeta = sizeof(VM);
  const bool v_mx = a.v_kind == 2, v_blk = a.v_kind == 1;
  constexpr int kCopies = 2 * CPT + (HAS_BIAS ? 1 : 0) + 2 + (VALPHA ? D / 64 : 0) + (ELIDE ? D / 64 : 0);
  // per-lane byte offsets of the small tables (lanes past a table's end repeat it)
  const uint32_t ke_lofs = 4 * (lane & (kTN * (D / 32) / 4 - 1));
  const uint32_t ve_lofs = 4 * (lane & (D / 4 - 1));
  // V^T column scales are constant 127 (= 1) unless V is MX (then copied per tile)
  if (!v_mx && tid < 4 * (D / 4)) vmeta[tid / (D / 4)].ve[tid % (D / 4)] = 0x7f7f7f7fu;

  const float* ksc_base = QK_MX ? nullptr : reinterpret_cast<const float*>(a.k_scale) + bh * a.nqkblk;
  auto load_k = [&](int it, int buf) {
    const int key0 = it * kTN;
#pragma unroll
    for (int c = 0; c < CPT; ++c) g2l16(kbase + key0 * D, kofs[c], k_lds0 + buf * kKBuf + (c * kThreads + wv * 64) * 16);
    const uint32_t kmb = km0 + buf * kKMeta;
    if constexpr (HAS_BIAS) g2l4(bias_src + key0, 4 * lane, kmb + wv * kTN * 4);
    if constexpr (QK_MX) {
      g2l4(reinterpret_cast<const uint8_t*>(a.k_scale) + (static_cast<size_t>(bh) * P + key0) * (D / 32), ke_lofs,
           kmb + offsetof(KMeta, ke));
    } else {
      // lane l fetches the scale of key l's 16-key group (clamped at the last block)
      int kb = (key0 + 16 * (lane >> 4)) >> a.lg_qkblk;
      kb = kb < a.nqkblk ? kb : a.nqkblk - 1;
      g2l4(ksc_base, 4 * kb, kmb + offsetof(KMeta, ksc));
    }
  };
  auto load_v = [&](int it, int buf) {
    const int key0 = it * kTN;
#pragma unroll
    for (int c = 0; c < CPT; ++c) g2l16(vbase + key0, vofs[c], v_lds0 + buf * kVBuf + (c * kThreads + wv * 64) * 16);
    const uint32_t vmb = vm0 + buf * kVMeta;
    // one V-side scale copy per tile whatever V carries (no branch): the MX
    // column scales into ve, the fp8_block scale into vsc, or for per-channel
    // scales (applied in the epilogue) an unused copy of the first one into vsc
    const int vblk = bh * a.nvblk + (key0 >> a.lg_vblk);
    const void* vsrc = v_mx ? static_cast<const void*>(reinterpret_cast<const uint32_t*>(a.v_scale) + vblk * (D / 4))
                            : static_cast<const void*>(reinterpret_cast<const float*>(a.v_scale) + (v_blk ? vblk : 0));
    g2l4(vsrc, v_mx ? ve_lofs : 0u, vmb + (v_mx ? offsetof(VM, ve) : offsetof(VM, vsc)));
    if constexpr (VALPHA) {
      const float* va = a.v_alpha + (static_cast<size_t>(bh) * a.nvsb + (key0 >> a.lg_vsb)) * D;
#pragma unroll
      for (int c = 0; c < D / 64; ++c) g2l4(va + 64 * c, 4 * lane, vmb + offsetof(VM, valpha) + 256 * c);
    }
    if constexpr (ELIDE) {
      // the tile's V column sums (without a table, an unused copy of the
      // first D * 4 bytes of the head's V^T codes, so the copy count stays fixed)
      const float* cs = a.vcol ? a.vcol + (static_cast<size_t>(bh) * (P / kTN) + it) * D
                               : reinterpret_cast<const float*>(vbase);
#pragma unroll
      for (int c = 0; c < D / 64; ++c) g2l4(cs + 64 * c, 4 * lane, vmb + offsetof(VM, vcol) + 256 * c);
    }
  };

  // qm correction folded into the scores: the MFMA accumulator of a key starts
  // at bias / C (C = the score scale of the lane's query and the key's group),
  // so acc * C = dot * C + bias.  Each wave rescales its bias row of the tile
  // into two rows of its own LDS area, one per 16-query half of the wave (the
  // halves can straddle an fp8_block Q scale of 16 rows); lane k handles key k.
  float qCh0 = qC, qCh1 = qC;
  if constexpr (HAS_BIAS && !QK_MX) {
    qCh0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(qC), 0));
    qCh1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(qC), 16));
  }
  const float inv_qC0 = 1.0f / qCh0, inv_qC1 = 1.0f / qCh1;
  // Ct_next: the score scale C of the lane's query for the two 16-key groups
  // (t = 0, 1) of the lane in the next tile, read with the K-side metadata
  float Ct_next[2] = {qC, qC};
  // bias_fetch reads the K-side metadata of the tile in slot sl (and sets
  // Ct_next); bias_store turns it into the wave's two binit rows.  Split so the
  // LDS reads issue first in a step and the rows are written once they land.
  struct BiasIn {
    float b, ks;  // bias of key `lane` (log2 units), fp8_block scale of its group
  };
  auto bias_fetch = [&](int sl) -> BiasIn {
    BiasIn x{0.0f, 1.0f};
    if constexpr (!QK_MX) {
#pragma unroll
      for (int t = 0; t < 2; ++t) Ct_next[t] = qC * kmeta[sl].ksc[16 * (2 * t + g)];
    }
    if constexpr (HAS_BIAS) {
      x.b = kmeta[sl].bias[wave][lane];
      if constexpr (!QK_MX) x.ks = kmeta[sl].ksc[lane];
    }
    return x;
  };
  auto bias_store = [&](const BiasIn& x) {
    if constexpr (HAS_BIAS) {
      float r = 1.0f;
      if constexpr (!QK_MX) r = __builtin_amdgcn_rcpf(x.ks);
      binit[wave][0][lane] = x.b * (inv_qC0 * r);
      binit[wave][1][lane] = x.b * (inv_qC1 * r);
    }
  };
  // S^T = K Q^T (+ bias / C) of the K tile in slot kb
  // per-lane byte offsets of the MFMA operand reads within a K / V^T slot:
  // the XOR swizzle of row 32 * t + li (K) or 32 * db + li (V^T) depends on li
  // only, so the block index becomes an immediate offset of the LDS read.
  uint32_t krd[NH][2], vrd[2];
#pragma unroll
  for (int hh = 0; hh < NH; ++hh)
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) krd[hh][h2] = li * D + 16 * ((4 * hh + 2 * h2 + g) ^ swz_k<D>(li));
#pragma unroll
  for (int h2 = 0; h2 < 2; ++h2) vrd[h2] = li * kTN + 16 * ((2 * h2 + g) ^ swz_v(li));

  // ---- S^T = K Q^T (+ bias / C) on the matrix cores ------------------------------
  constexpr int NQK = 2 * NH;  // QK MFMAs per tile: i = NH * t + hh (32-key block t, 64-wide half hh of D)
  // accumulator init of score block t: bias / C of the lane's query half (zero without bias)
  auto qk_init = [&](v16f& s, int t) {
    if constexpr (HAS_BIAS) {
      const float4* bp = reinterpret_cast<const float4*>(&binit[wave][li >> 4][32 * t + 16 * g]);
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const float4 bb = bp[q4];
        s[4 * q4 + 0] = bb.x; s[4 * q4 + 1] = bb.y; s[4 * q4 + 2] = bb.z; s[4 * q4 + 3] = bb.w;
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = 0.0f;
    }
  };
  // K operand of QK MFMA i of the tile in K slot kb
  auto qk_read = [&](int kb, int i) -> v8i {
    const uint8_t* rp = &k_lds[kb][32 * (i / NH) * D];
    return lds_read32(rp + krd[i % NH][0], rp + krd[i % NH][1]);
  };
  // E8M0 of the K rows of QK MFMA i (MX K; unused otherwise)
  auto qk_scale = [&](int kb, int i) -> int {
    if constexpr (QK_MX) {
      const int t = i / NH, hh = i % NH;
      if constexpr (D == 128) return (kmeta[kb].ke[32 * t + kperm(li)] >> (8 * (2 * hh + g))) & 0xff;
      else return reinterpret_cast<const uint8_t*>(&kmeta[kb].ke[0])[2 * (32 * t + kperm(li)) + g];
    } else {
      return 127;
    }
  };
  auto qk_mfma = [&](int i, const v8i& ka, const v16f& c_in, int ke) -> v16f {
    const int hh = i % NH;
    if constexpr (QK_MX) return mfma32<true>(ka, qop[hh], c_in, ke, qe[hh]);
    else return mfma32<false>(ka, qop[hh], c_in, 0, 0);
  };
  // ---- O^T += V^T P^T (E8M0 scales: MX V columns, MX P; 127 = 1 otherwise) ----------
  auto pv_read = [&](int vs, int db) -> v8i {
    const uint8_t* vp = &v_lds[vs][32 * db * kTN];
    return lds_read32(vp + vrd[0], vp + vrd[1]);
  };
  // E8M0 of V^T row 32 db + li (127 unless V is MX)
  auto pv_scale = [&](int vs, int db) -> int { return reinterpret_cast<const uint8_t*>(&vmeta[vs].ve[0])[32 * db + li]; };
  auto pv_mfma = [&](int db, const v8i& va, const v8i& pcodes, int pe_, int ve) {
    acc[db] = mfma32<true>(va, pcodes, acc[db], ve, pe_);
  };

  int ndec = nt;  // row-max / BLASST decisions per row
  if constexpr (BN == 64) {
  // prologue: tiles 0 and 1 complete, K codes of tile 2.  V slot 3 stands for
  // tile -1: zero codes with unit scales, so the PV that the first step issues
  // for the previous tile adds exactly zero.
  load_k(0, 0);
  load_v(0, 0);
  load_k(nt > 1 ? 1 : nt - 1, 1);
  load_v(nt > 1 ? 1 : nt - 1, 1);
  load_k(nt > 2 ? 2 : nt - 1, 2);
  {
    uint4* z = reinterpret_cast<uint4*>(&v_lds[3][0]);
    for (int i = tid; i < D * kTN / 16; i += kThreads) z[i] = make_uint4(0u, 0u, 0u, 0u);
    if (tid < kTN) vmeta[3].ve[tid] = 0x7f7f7f7fu;
    if (VALPHA && tid < D) vmeta[3].valpha[tid] = 0.0f;
  }
  lds_publish<0>();
  v16f sc[2];
  bias_store(bias_fetch(0));
  qk_init(sc[0], 0);
  qk_init(sc[1], 1);
  // E8M0 operands of v_mfma_scale must not share registers with the MFMA's
  // destination.  When the accumulator input is the constant 0 (scores without
  // bias) the compiler does not tie the destination to it and may hand it the
  // register of a scale that dies at the MFMA.  The MX-QK scales are therefore
  // kept live until the next step reads them (ke_live), so no MFMA of a step can
  // be given their registers wherever it is scheduled.  (The PV MFMAs
  // accumulate in place and are not affected.)
  int ke_live[NQK];
#pragma unroll
  for (int i = 0; i < NQK; ++i) ke_live[i] = qk_scale(0, i);
#pragma unroll
  for (int i = 0; i < NQK; ++i) sc[i / NH] = qk_mfma(i, qk_read(0, i), sc[i / NH], ke_live[i]);
  __syncthreads();  // every wave has read K tile 0 and its bias rows before they are overwritten

  // One K/V tile per step.  Step it turns the scores of tile it (in sc) into P
  // codes in four chunks of 8 keys per lane.  The matrix work rides along, one
  // or two MFMAs per chunk, independent of the chunk's VALU work: the PV of
  // tile it-1 (its codes kept in registers, its V^T in a four-slot ring) and
  // the QK MFMAs of tile it+1, written into the score block that chunks 0-1
  // have already consumed (block 0) or after chunk 3 (block 1).  The
  // accumulator rescale for tile it closes the step, so the PV of tile it in
  // the next step accumulates into it directly.
  v8i pop_prev;       // P codes of tile it-1 (zero codes before the first tile)
  int pe_prev = 127;  // their E8M0 scale (MX P)
  float fcq[BL == 3 ? 32 : 1];  // UTA fill, 32/64 bins: fill codes of the lane's keys (current where the row skips)
#pragma unroll
  for (int j = 0; j < (BL == 3 ? 32 : 1); ++j) fcq[j] = 0.0f;
  uint32_t fpk[BL == 2 ? 8 : 1];  // UTA fill, <= 16 bins: packed fill codes (current where the row skips)
  float fsum = 0.0f;              // and their sum in code units
#pragma unroll
  for (int q = 0; q < (BL == 2 ? 8 : 1); ++q) fpk[q] = 0u;
#pragma unroll
  for (int q = 0; q < 8; ++q) pop_prev[q] = 0;
  // MASKED: the tile holds keys >= S (only the last tile, when S % 64 != 0);
  // the body is instantiated with and without the masking so the common tiles
  // carry no merge of masked and unmasked scores
  // ph = it % 4, passed as a literal in the unrolled main loop
  auto step = [&](const int it, auto masked_tag, const int ph) __attribute__((always_inline)) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    const int nxt = (ph + 1) & 3;          // K slot of tile it+1
    const int vprev = (ph + 3) & 3, vcur = ph;
    const int key0 = it * kTN;
    // global -> LDS prefetch: K of tile it+3 into the slot of tile it-1 (read
    // two steps ago), V^T and metadata of tile it+2 into the slot of tile it-2
    // (clamped: the last iterations reload the last tile into slots nobody
    // reads any more)
    load_k(it + 3 < nt ? it + 3 : nt - 1, (ph + 3) & 3);
    load_v(it + 2 < nt ? it + 2 : nt - 1, (ph + 2) & 3);

    // ---- scores: sv = dot + bias / C; the log2-unit score is u = sv * C ----------
    const float Ct[2] = {Ct_next[0], Ct_next[1]};
    // LDS reads first, in the order they are consumed, so each wait covers
    // only what it needs: metadata of tile it+1 (bias rows, Ct_next), the E8M0
    // scales of this step's MFMAs, the V block scale, the first operands
    const BiasIn bn = bias_fetch(nxt);
    if constexpr (QK_MX) {
      __builtin_amdgcn_sched_barrier(0);  // the previous step's MFMAs stay above
#pragma unroll
      for (int i = 0; i < NQK; ++i) use(ke_live[i]);  // the previous step's scales end here
    }
    int ve_p[NDB], ke_n[NQK];
#pragma unroll
    for (int db = 0; db < NDB; ++db) ve_p[db] = pv_scale(vprev, db);
#pragma unroll
    for (int i = 0; i < NQK; ++i) ke_n[i] = qk_scale(nxt, i);
    const float vsc = vmeta[vcur].vsc[0];
    // ELIDE: the PV MFMAs of tile it-1 are skipped (wave-uniform branch) when
    // all of its P codes in the wave are zero -- an elided tile (below) leaves
    // zero codes; the product would add exact zeros
    bool pv_zero = false;
    if constexpr (ELIDE) {
      const int nz = (pop_prev[0] | pop_prev[1] | pop_prev[2] | pop_prev[3]) |
                     (pop_prev[4] | pop_prev[5] | pop_prev[6] | pop_prev[7]);
      pv_zero = __all(nz == 0);
    }
    v8i va[2], ka[2];
    va[0] = pv_read(vprev, 0);
    ka[0] = qk_read(nxt, 0);
    // sv(j) is the accumulator register of key j (16 * t + r), used in place
#define sv(j) sc[(j) >> 4][(j) & 15]
    if constexpr (MASKED) {
#pragma unroll
      for (int j = 0; j < 32; ++j)
        if (key0 + 32 * (j >> 4) + 16 * g + (j & 15) >= S) sv(j) = -INFINITY;
    }
    float bmax;
    {
      float m2v[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        // 16 values, 8 instructions, depth 3
        const float a0 = hmax3(sc[t][0], sc[t][1], sc[t][2]);
        const float a1 = hmax3(sc[t][3], sc[t][4], sc[t][5]);
        const float a2 = hmax3(sc[t][6], sc[t][7], sc[t][8]);
        const float a3 = hmax3(sc[t][9], sc[t][10], sc[t][11]);
        const float a4 = hmax3(sc[t][12], sc[t][13], sc[t][14]);
        const float b0 = hmax3(a0, a1, sc[t][15]);
        m2v[t] = hmax3(b0, a2, hmax(a3, a4)) * Ct[t];   // C > 0
      }
      bmax = xor32_max(hmax(m2v[0], m2v[1]));
    }

    // ---- row max, P in quantised units, row sum ----------------------------------
    float alpha, m_new;
    int pe = 127;        // E8M0 of the MX P scale
    float sig_p = 1.0f;  // fp32 P scale carried by the accumulator (dynamic)
    v8i pop;             // P codes of tile it
    bool skip = false;   // BLASST: the row keeps no exact p in this tile
    if constexpr (BLASST) {
      // attention_triton.py:164-175 (BLASST takes precedence over the estimate)
      const float mij = hmax(m2, bmax);
      skip = qvalid && (bmax - mij) < a.log2_lam;
      alpha = skip ? 1.0f : fast_exp2(m2 - mij);
      m_new = skip ? m2 : mij;
      skipped += skip ? 1.0f : 0.0f;  // branch-free; the g == 0 lanes' counts are written
    } else if constexpr (HAS_EST && P_MODE == 2) {
      // branch-free: without dyn_est, m2 stays at the estimate (adjust is false).
      // l == 0 (no mass accumulated, attention_triton.py:200-207) holds exactly
      // before the first tile: every branch below leaves the tile's largest P at
      // code 448 (ra = 2^(bmax - m_new) >= 2^-32 since `over` fires beyond 32),
      // so l > 0 afterwards -- unless all of a row's scores sit ~197 log2 units
      // under its m, where the reference's fp32 exp2 underflows to 0 as well.
      const bool lzero = it == 0;
      const float ms = hmax(max_seen, bmax);
      const bool under = (bmax - m2) > 16.0f;
      const bool over = (m2 - ms) > 32.0f;
      const float down = lzero ? ms : fmaxf(ms + 32.0f, m2 - 80.0f * kLog2e);
      const bool adjust = dyn_est && (under || over);
      m_new = adjust ? (under ? bmax : down) : m2;
      alpha = adjust ? (lzero ? 0.0f : fast_exp2(m2 - m_new)) : 1.0f;
      max_seen = dyn_est ? ms : max_seen;
    } else if constexpr (HAS_EST) {
      m_new = est2;
      alpha = 1.0f;
    } else {
      m_new = hmax(m2, bmax);
      alpha = fast_exp2(m2 - m_new);
    }
    // BLASST fills of the skipped rows, in p units, and the largest fill of the row
    float fp[BL == 3 ? 32 : 1];
    float fr[8];  // BL 2: fill of each run of the lane
    float fmax = 0.0f;
    bool any_skip = false;
    if constexpr (BLASST) {
      any_skip = __any(skip);
      if (any_skip) {
        if constexpr (BL == 2) {
          switch (kTN / a.uta_bins) {
            case 4: fmax = uta_runs<4, MASKED>(sc, Ct, m_new, off, a.fill_alpha, fr); break;
            case 8: fmax = uta_runs<8, MASKED>(sc, Ct, m_new, off, a.fill_alpha, fr); break;
            case 16: fmax = uta_runs<16, MASKED>(sc, Ct, m_new, off, a.fill_alpha, fr); break;
            case 32: fmax = uta_runs<32, MASKED>(sc, Ct, m_new, off, a.fill_alpha, fr); break;
            default: fmax = uta_runs<64, MASKED>(sc, Ct, m_new, off, a.fill_alpha, fr); break;
          }
        } else if constexpr (BL == 3) {
          float u[32];
#pragma unroll
          for (int j = 0; j < 32; ++j) u[j] = sv(j) * Ct[j >> 4];
          fmax = blasst_fill<P_MODE>(a, u, m_new, bmax, off, key0, fp);
        } else {
          fmax = blasst_row_fill<P_MODE, MASKED>(a, sc, Ct, m_new, bmax, off, key0);
        }
      }
    }
    // P scale of the row (attention_triton.py:330-370): exact rows from the tile
    // max, skipped rows from their largest fill; T puts exact p in code units
    float T, s_lp, qmul_f = 1.0f;  // qmul_f: fill (p units) -> code units
    if constexpr (P_MODE == 0) {
      T = m_new - off;
      s_lp = 1.0f;
    } else if constexpr (P_MODE == 1) {
      const float ra = fmaxf(skip ? fmax : fast_exp2(bmax - m_new), kAmaxFloor);
      int e = ceil_log2_div448(ra);  // == ceil_log2_exact(ra / 448)
      e = e < -127 ? -127 : (e > 127 ? 127 : e);
      T = m_new + static_cast<float>(e);
      s_lp = __uint_as_float(static_cast<uint32_t>(e + 127) << 23);
      qmul_f = __uint_as_float(static_cast<uint32_t>(127 - e) << 23);
      pe = e + 127;
    } else {
      const float ra = skip ? fmax : fast_exp2(bmax - m_new);
      const bool floored = !(ra > 1e-12f);
      const float rf = floored ? 1e-12f : ra;
      s_lp = rf * (1.0f / kFp8Max);
      T = (floored ? m_new + kLog2DynFloor : bmax) - kLog2Fp8Max;
      sig_p = s_lp;
      if constexpr (BLASST) qmul_f = kFp8Max * __builtin_amdgcn_rcpf(rf);
    }
    float fq = 0.0f;  // row fill (BL 1) in code units
    int fqw = 0;      // BL 1, full tiles: four E4M3 codes of fq (the codes of a skipped row)
    if constexpr (BL == 2) {
      if (any_skip) {
        switch (kTN / a.uta_bins) {
          case 4: uta_pack<4, P_MODE, MASKED>(sc, fr, qmul_f, fpk, fsum); break;
          case 8: uta_pack<8, P_MODE, MASKED>(sc, fr, qmul_f, fpk, fsum); break;
          case 16: uta_pack<16, P_MODE, MASKED>(sc, fr, qmul_f, fpk, fsum); break;
          case 32: uta_pack<32, P_MODE, MASKED>(sc, fr, qmul_f, fpk, fsum); break;
          default: uta_pack<64, P_MODE, MASKED>(sc, fr, qmul_f, fpk, fsum); break;
        }
      }
    } else if constexpr (BL == 3) {
      if (any_skip) {
#pragma unroll
        for (int j = 0; j < 32; ++j) fcq[j] = P_MODE == 0 ? fminf(fp[j], kFp8Max) : fp[j] * qmul_f;
      }
    } else if constexpr (BL == 1) {
      fq = P_MODE == 0 ? fminf(fmax, kFp8Max) : fmax * qmul_f;
      if constexpr (!MASKED) {
        fqw = __builtin_amdgcn_cvt_pk_fp8_f32(fq, fq, __float_as_int(fq), false);
        fqw = __builtin_amdgcn_cvt_pk_fp8_f32(fq, fq, fqw, true);
      }
    }
    (void)fq;
    (void)qmul_f;
    (void)fp;
    // p may exceed 448 only against an estimated or offset row max: satfinite cast
    const bool clamp = P_MODE == 0 && (HAS_EST || a.p_max_offset > 8);
    float ps4[4];
    // BLASST: every row of the wave skips this (full) tile (wave-uniform)
    const bool skip_all = (BL == 1 || BL == 2) && !MASKED && __all(skip);
    if constexpr (BLASST) {
      wt_all += __all(skip) ? 1 : 0;
      wt_any += any_skip ? 1 : 0;
    }
    v16f bi1;
    v16f rsm;  // V smoothing: rowsum of the codes of tile it-1
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      __builtin_amdgcn_sched_barrier(0);
      const float Tc = T;
      // matrix work of chunk c: PV block c of tile it-1, QK MFMAs of block 0 of
      // tile it+1 (its scores were consumed by chunks 0-1)
      if (c < NDB) {
        v8i vac = va[c & 1];
        pin(vac);
        if (c + 1 < NDB) va[(c + 1) & 1] = pv_read(vprev, c + 1);
        if (!pv_zero) pv_mfma(c, vac, pop_prev, pe_prev, ve_p[c]);
      }
      if (VALPHA && c == 1) {  // row sums of the codes of tile it-1 (every register holds the lane's)
        const v16f zero = {};
        rsm = mfma32<false>(ones, pop_prev, zero, 0, 0);
      }
      if (c >= 2 && c - 2 < NH) {
        v8i kac = ka[(c - 2) & 1];
        pin(kac);
        sc[0] = qk_mfma(c - 2, kac, sc[0], ke_n[c - 2]);
        if (c < NQK) ka[c & 1] = qk_read(nxt, c);
      }
      if (c == 0 && NQK > 1) ka[1] = qk_read(nxt, 1);
      if (c == 0) bias_store(bn);  // bias rows of tile it+1 -> this wave's binit rows
      if (c == 2) qk_init(bi1, 1);  // accumulator init of score block 1 (bias of tile it+1)
      // VALU work of chunk c: keys 8c .. 8c+7 of the lane (none when every row
      // of the wave skips the tile: its codes are the fill codes)
      if (!skip_all) {
      float pq[8];
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        const int j = 8 * c + jj;
        pq[jj] = fast_exp2(fmaf(sv(j), Ct[j >> 4], -Tc));
        // fill codes of a skipped row (zero on the keys past S of the last tile)
        if constexpr (BL == 3) pq[jj] = skip ? fcq[j] : pq[jj];
        if constexpr (BL == 1 && MASKED) pq[jj] = skip ? (sv(j) == -INFINITY ? 0.0f : fq) : pq[jj];
        ps4[j & 3] = j < 4 ? pq[jj] : ps4[j & 3] + pq[jj];
      }
      if constexpr (P_MODE == 0) {
        if (clamp) {
#pragma unroll
          for (int jj = 0; jj < 8; ++jj) pq[jj] = fminf(pq[jj], kFp8Max);
        }
      }
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        // both 16-bit halves are written: the "old" operand only names a register
        // (pq[4 h2], dead after this instruction), so no zeroing is needed
        int wd = __builtin_amdgcn_cvt_pk_fp8_f32(pq[4 * h2], pq[4 * h2 + 1], __float_as_int(pq[4 * h2]), false);
        pop[2 * c + h2] = __builtin_amdgcn_cvt_pk_fp8_f32(pq[4 * h2 + 2], pq[4 * h2 + 3], wd, true);
        if constexpr (BL == 2) pop[2 * c + h2] = skip ? static_cast<int>(fpk[2 * c + h2]) : pop[2 * c + h2];
        if constexpr (BL == 1 && !MASKED) pop[2 * c + h2] = skip ? fqw : pop[2 * c + h2];
      }
      }
      // score block 0 is consumed: it receives the bias of tile it+1
      if (c == 1) qk_init(sc[0], 0);
      use(pop[2 * c]);
      use(pop[2 * c + 1]);
#pragma unroll
      for (int k = 0; k < 4; ++k) use(ps4[k]);
      if (c < NDB) use(acc[c]);
      if (c >= 2 && c - 2 < NH) use(sc[0]);
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (BL == 1 || BL == 2) {
      if (skip_all) {  // the fill codes (the row sums of skipped rows are set below)
        // (zero codes when the tile is elided: its PV product is added below,
        // and the PV MFMAs of the next step add nothing for it)
#pragma unroll
        for (int q = 0; q < 8; ++q) pop[q] = BL == 1 ? (ELIDE && a.vcol ? 0 : fqw) : static_cast<int>(fpk[q]);
#pragma unroll
        for (int k = 0; k < 4; ++k) ps4[k] = 0.0f;
      }
    }
    // score block 1 is consumed: QK MFMAs of tile it+1 from the bias init
    sc[1] = qk_mfma(NH, ka[NH & 1], bi1, ke_n[NH]);
#pragma unroll
    for (int i = NH + 1; i < NQK; ++i) sc[1] = qk_mfma(i, ka[i & 1], sc[1], ke_n[i]);
    float psum = (ps4[0] + ps4[1]) + (ps4[2] + ps4[3]);
    if constexpr (BL == 2) psum = skip ? fsum : psum;  // the fill codes' sum
    if constexpr (BL == 1) {
      // a skipped row sums its pre-quant fill over the valid keys
      // (attention_triton.py:324-326); each lane of the pair holds 32 keys of
      // the row (32 t + 16 g + r), so it adds the fill once per valid key of its own
      float nvl = 32.0f;
      if constexpr (MASKED) {
        int c = 0;
#pragma unroll
        for (int t = 0; t < 2; ++t) c += min(max(S - key0 - 32 * t - 16 * g, 0), 16);
        nvl = static_cast<float>(c);
      }
      psum = skip ? (P_MODE == 0 ? fmax : fmax * qmul_f) * nvl : psum;
    }
    psum *= s_lp;  // sum of the pre-quant p
    l = l * alpha + psum;
#undef sv

    // ---- V smoothing: correction of tile it-1, in the units of its PV product
    // (added in this step), before this step's rescale ----------------------------
    if constexpr (VALPHA) valpha_outer<NDB>(acc, vmeta[vprev].valpha, rsm[0] * vw_prev, li, g);

    // ---- accumulator rescale for tile it (alpha, dynamic P scale, fp8_block V
    // scale): the PV of tile it, issued in the next step, accumulates on top ------
    float sig_new = sig_p;
    sig_new *= v_blk ? vsc : 1.0f;
    // ELIDE: every row of the wave skipped this full tile, so each row's P is
    // one fill code on all 64 keys and the tile's PV product is that code times
    // the column sums of V.  It is added here in fp32, in the units of the
    // current sigma (alpha is 1 for a skipped row, so nothing is rescaled),
    // and the tile's P codes are left at zero, so the next step skips the
    // tile's PV MFMAs (pv_zero; a flag carried from this step instead takes
    // the kernel past 256 VGPRs).
    const bool elide = ELIDE && !MASKED && skip_all && a.vcol != nullptr;
    // an elided tile keeps sigma (f = 1: no rescale)
    const float sig_keep = elide ? sigma : sig_new;
    const float rsig = __builtin_amdgcn_rcpf(sig_keep);
    if (elide && a.fill_kind != FILL_ZERO)
      valpha_outer<NDB>(acc, vmeta[vcur].vcol, __builtin_amdgcn_cvt_f32_fp8(fqw, 0) * s_lp * (v_blk ? vsc : 1.0f) * rsig,
                        li, g);
    const float f = elide ? 1.0f : alpha * sigma * rsig;
    sigma = sig_keep;
    if constexpr (VALPHA) vw_prev = s_lp * rsig;  // rowsum(P_deq) / sigma per code unit
    if ((P_MODE == 2 && !ELIDE) || __any(f != 1.0f)) {
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[db][r] *= f;
    }
    pop_prev = pop;
    pe_prev = pe;
    m2 = m_new;
    if constexpr (QK_MX) {
#pragma unroll
      for (int i = 0; i < NQK; ++i) ke_live[i] = ke_n[i];
    }

    lds_publish<kCopies>();
  };
  const int nfull = (S % kTN) ? nt - 1 : nt;
  {
    // four steps per iteration: ring slots are constants, and the loop-carried
    // scores, P codes and scale registers rotate through the unrolled steps
    // instead of being copied at the back edge.  Kernels that carry more
    // state through a step -- V smoothing, the packed UTA fill codes, the
    // per-row fills with MX Q/K -- need more than the 256 VGPRs of two waves
    // per SIMD when unrolled four times and spill inside the loop, so they run
    // two steps per iteration (ring slots then come from it % 4; the packed
    // UTA fills spill even at two and run one).
    constexpr bool UNROLL = !VALPHA && (BL == 0 || BL == 3 || (BL == 1 && !QK_MX));
    int it0 = 0;
    if constexpr (UNROLL) {
      for (; it0 + 3 < nfull; it0 += 4) {
        step(it0, std::false_type{}, 0);
        step(it0 + 1, std::false_type{}, 1);
        step(it0 + 2, std::false_type{}, 2);
        step(it0 + 3, std::false_type{}, 3);
      }
    }
    if constexpr (!UNROLL && BL != 2) {
      for (; it0 + 1 < nfull; it0 += 2) {
        step(it0, std::false_type{}, it0 & 3);
        step(it0 + 1, std::false_type{}, (it0 + 1) & 3);
      }
    }
    for (; it0 < nfull; ++it0) step(it0, std::false_type{}, it0 & 3);
  }
  if (nfull < nt) step(nt - 1, std::true_type{}, (nt - 1) & 3);
  if constexpr (QK_MX) {
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NQK; ++i) use(ke_live[i]);  // the last step's scales
  }
  // PV of the last tile; no copy is left in flight when the workgroup ends
  {
    const int vl = (nt - 1) & 3;
#pragma unroll
    for (int db = 0; db < NDB; ++db) pv_mfma(db, pv_read(vl, db), pop_prev, pe_prev, pv_scale(vl, db));
    if constexpr (VALPHA) {  // correction of the last tile
      const v16f zero = {};
      const v16f rl = mfma32<false>(ones, pop_prev, zero, 0, 0);
      valpha_outer<NDB>(acc, vmeta[vl].valpha, rl[0] * vw_prev, li, g);
    }
  }
  } else {
    // ---- block_n = 128 (attention_triton.py:109-407 with BLOCK_N = 128) -------------
    // One step per 128-key block b: the scores of its two 64-key tiles (ring
    // slots 2b % 4 and (2b + 1) % 4), one row-max update, BLASST decision, fill
    // and P scale over the 128 keys, the P codes of both tiles, then the
    // accumulator rescale and the PV of both tiles.  The K/V tiles of block
    // b + 1 are copied into the other two slots during the step, which ends
    // with all copies landed and a barrier.
    const int nb = (S + 127) / 128;
    ndec = nb;
    auto load_block = [&](int bb) {
      const int t0 = 2 * bb, t1 = 2 * bb + 1;
      const int c0 = t0 < nt ? t0 : nt - 1, c1 = t1 < nt ? t1 : nt - 1;
      load_k(c0, t0 & 3);
      load_k(c1, t1 & 3);
      load_v(c0, t0 & 3);
      load_v(c1, t1 & 3);
    };
    load_block(0);
    lds_publish<0>();
    auto step128 = [&](const int bb, auto masked_tag) __attribute__((always_inline)) {
      constexpr bool MASKED = decltype(masked_tag)::value;
      const int key0 = bb * 128;
      const int slA = (2 * bb) & 3, slB = (2 * bb + 1) & 3;
      if (bb + 1 < nb) load_block(bb + 1);
      // scores of both tiles: s4[2 tt + t] for tile tt, C4 its score scales
      v16f s4[4];
      float C4[4];
      auto qk_tile = [&](int sl, int o) __attribute__((always_inline)) {
        const BiasIn x = bias_fetch(sl);
        C4[o] = Ct_next[0];
        C4[o + 1] = Ct_next[1];
        bias_store(x);
        qk_init(s4[o], 0);
        qk_init(s4[o + 1], 1);
        pin(s4[o]);  // never a known constant at the MFMA (see acc)
        pin(s4[o + 1]);
#pragma unroll
        for (int i = 0; i < NQK; ++i) s4[o + i / NH] = qk_mfma(i, qk_read(sl, i), s4[o + i / NH], qk_scale(sl, i));
      };
      qk_tile(slA, 0);
      qk_tile(slB, 2);
      if constexpr (MASKED) {
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (key0 + 64 * (k >> 1) + 32 * (k & 1) + 16 * g + r >= S) s4[k][r] = -INFINITY;
      }
      float bmax;
      {
        float mk[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          float m = hmax3(s4[k][0], s4[k][1], s4[k][2]);
#pragma unroll
          for (int r = 3; r < 15; r += 2) m = hmax3(m, s4[k][r], s4[k][r + 1]);
          mk[k] = hmax(m, s4[k][15]) * C4[k];  // C > 0
        }
        bmax = xor32_max(hmax(hmax(mk[0], mk[1]), hmax(mk[2], mk[3])));
      }
      // row max, BLASST decision (as the 64-key step, over 128 keys)
      float alpha, m_new;
      int pe = 127;
      float sig_p = 1.0f;
      bool skip = false;
      if constexpr (BLASST) {
        const float mij = hmax(m2, bmax);
        skip = qvalid && (bmax - mij) < a.log2_lam;
        alpha = skip ? 1.0f : fast_exp2(m2 - mij);
        m_new = skip ? m2 : mij;
        skipped += skip ? 1.0f : 0.0f;
      } else if constexpr (HAS_EST && P_MODE == 2) {
        const bool lzero = bb == 0;
        const float ms = hmax(max_seen, bmax);
        const bool under = (bmax - m2) > 16.0f;
        const bool over = (m2 - ms) > 32.0f;
        const float down = lzero ? ms : fmaxf(ms + 32.0f, m2 - 80.0f * kLog2e);
        const bool adjust = dyn_est && (under || over);
        m_new = adjust ? (under ? bmax : down) : m2;
        alpha = adjust ? (lzero ? 0.0f : fast_exp2(m2 - m_new)) : 1.0f;
        max_seen = dyn_est ? ms : max_seen;
      } else if constexpr (HAS_EST) {
        m_new = est2;
        alpha = 1.0f;
      } else {
        m_new = hmax(m2, bmax);
        alpha = fast_exp2(m2 - m_new);
      }
      float fmax = 0.0f;
      bool any_skip = false;
      float fr[BL == 2 ? 64 : 1];
      if constexpr (BLASST) {
        any_skip = __any(skip);
        if (any_skip) {
          if constexpr (BL == 1) {
            fmax = blasst_row_fill128<P_MODE, MASKED>(a, s4, C4, m_new, bmax, off, key0);
          } else {
            switch (128 / a.uta_bins) {
              case 1: fmax = uta128_runs<1, MASKED>(s4, C4, m_new, off, a.fill_alpha, fr); break;
              case 2: fmax = uta128_runs<2, MASKED>(s4, C4, m_new, off, a.fill_alpha, fr); break;
              case 4: fmax = uta128_runs<4, MASKED>(s4, C4, m_new, off, a.fill_alpha, fr); break;
              case 8: fmax = uta128_runs<8, MASKED>(s4, C4, m_new, off, a.fill_alpha, fr); break;
              case 16: fmax = uta128_runs<16, MASKED>(s4, C4, m_new, off, a.fill_alpha, fr); break;
              case 32: fmax = uta128_runs<32, MASKED>(s4, C4, m_new, off, a.fill_alpha, fr); break;
              case 64: fmax = uta128_runs<64, MASKED>(s4, C4, m_new, off, a.fill_alpha, fr); break;
              default: fmax = uta128_runs<128, MASKED>(s4, C4, m_new, off, a.fill_alpha, fr); break;
            }
          }
        }
      }
      // P scale of the row over the block (attention_triton.py:330-370)
      float T, s_lp, qmul_f = 1.0f;
      if constexpr (P_MODE == 0) {
        T = m_new - off;
        s_lp = 1.0f;
      } else if constexpr (P_MODE == 1) {
        const float ra = fmaxf(skip ? fmax : fast_exp2(bmax - m_new), kAmaxFloor);
        int e = ceil_log2_div448(ra);
        e = e < -127 ? -127 : (e > 127 ? 127 : e);
        T = m_new + static_cast<float>(e);
        s_lp = __uint_as_float(static_cast<uint32_t>(e + 127) << 23);
        qmul_f = __uint_as_float(static_cast<uint32_t>(127 - e) << 23);
        pe = e + 127;
      } else {
        const float ra = skip ? fmax : fast_exp2(bmax - m_new);
        const bool floored = !(ra > 1e-12f);
        const float rf = floored ? 1e-12f : ra;
        s_lp = rf * (1.0f / kFp8Max);
        T = (floored ? m_new + kLog2DynFloor : bmax) - kLog2Fp8Max;
        sig_p = s_lp;
        if constexpr (BLASST) qmul_f = kFp8Max * __builtin_amdgcn_rcpf(rf);
      }
      float fq = 0.0f;
      int fqw = 0;
      uint32_t fpk[BL == 2 ? 16 : 1];
      float fsum = 0.0f;
      if constexpr (BL == 1) {
        fq = P_MODE == 0 ? fminf(fmax, kFp8Max) : fmax * qmul_f;
        fqw = __builtin_amdgcn_cvt_pk_fp8_f32(fq, fq, __float_as_int(fq), false);
        fqw = __builtin_amdgcn_cvt_pk_fp8_f32(fq, fq, fqw, true);
      } else if constexpr (BL == 2) {
#pragma unroll
        for (int w = 0; w < 16; ++w) fpk[w] = 0u;
        if (any_skip) {
          switch (128 / a.uta_bins) {
            case 1: uta128_pack<1, P_MODE>(s4, fr, qmul_f, fpk, fsum); break;
            case 2: uta128_pack<2, P_MODE>(s4, fr, qmul_f, fpk, fsum); break;
            case 4: uta128_pack<4, P_MODE>(s4, fr, qmul_f, fpk, fsum); break;
            case 8: uta128_pack<8, P_MODE>(s4, fr, qmul_f, fpk, fsum); break;
            case 16: uta128_pack<16, P_MODE>(s4, fr, qmul_f, fpk, fsum); break;
            case 32: uta128_pack<32, P_MODE>(s4, fr, qmul_f, fpk, fsum); break;
            case 64: uta128_pack<64, P_MODE>(s4, fr, qmul_f, fpk, fsum); break;
            default: uta128_pack<128, P_MODE>(s4, fr, qmul_f, fpk, fsum); break;
          }
        }
      }
      (void)fq;
      (void)fqw;
      if constexpr (BLASST) {
        wt_all += __all(skip) ? 1 : 0;
        wt_any += any_skip ? 1 : 0;
      }
      // P codes of both tiles (keys 32 t + 16 g + r of tile tt in word 8 tt + 2 (2 t + r / 8) ...)
      const bool clamp = P_MODE == 0 && (HAS_EST || a.p_max_offset > 8);
      v8i popt[2];
      float ps4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          float pq[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int jl = 32 * tt + 4 * q + i, k = jl >> 4, r = jl & 15;
            pq[i] = fast_exp2(fmaf(s4[k][r], C4[k], -T));
            if constexpr (BL == 1) pq[i] = skip ? (s4[k][r] == -INFINITY ? 0.0f : fq) : pq[i];
            ps4[i] += pq[i];
            if constexpr (P_MODE == 0) pq[i] = clamp ? fminf(pq[i], kFp8Max) : pq[i];
          }
          const int wd = __builtin_amdgcn_cvt_pk_fp8_f32(pq[0], pq[1], __float_as_int(pq[0]), false);
          int word = __builtin_amdgcn_cvt_pk_fp8_f32(pq[2], pq[3], wd, true);
          if constexpr (BL == 2) word = skip ? static_cast<int>(fpk[8 * tt + q]) : word;
          popt[tt][q] = word;
        }
      float psum = (ps4[0] + ps4[1]) + (ps4[2] + ps4[3]);
      if constexpr (BL == 1) {
        // a skipped row sums its pre-quant fill once per valid key of the lane
        float nvl = 64.0f;
        if constexpr (MASKED) {
          int c = 0;
#pragma unroll
          for (int k = 0; k < 4; ++k) c += min(max(S - key0 - 64 * (k >> 1) - 32 * (k & 1) - 16 * g, 0), 16);
          nvl = static_cast<float>(c);
        }
        psum = skip ? (P_MODE == 0 ? fmax : fmax * qmul_f) * nvl : psum;
      }
      if constexpr (BL == 2) psum = skip ? fsum : psum;
      psum *= s_lp;
      l = l * alpha + psum;
      // accumulator rescale (alpha, dynamic P scale, fp8_block V scale), then
      // the PV of both tiles in the new units
      const float vsc = vmeta[slA].vsc[0];
      float sig_new = sig_p;
      sig_new *= v_blk ? vsc : 1.0f;
      const float rsig = __builtin_amdgcn_rcpf(sig_new);
      const float f = alpha * sigma * rsig;
      sigma = sig_new;
      if (P_MODE == 2 || __any(f != 1.0f)) {
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[db][r] *= f;
      }
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        pv_mfma(db, pv_read(slA, db), popt[0], pe, pv_scale(slA, db));
        pv_mfma(db, pv_read(slB, db), popt[1], pe, pv_scale(slB, db));
      }
      if constexpr (VALPHA) {  // rowsum(P_deq) / sigma (x) alpha_v of the block (v_smooth_block >= 128)
        const v16f zero = {};
        v16f rs = mfma32<false>(ones, popt[0], zero, 0, 0);
        rs = mfma32<false>(ones, popt[1], rs, 0, 0);
        // (VALU FMAs here: the outer-product MFMAs take this step past 256 VGPRs)
        const float w = rs[0] * s_lp * rsig;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int d = 32 * db + 8 * (r >> 2) + 4 * g + (r & 3);
            acc[db][r] = fmaf(w, vmeta[slA].valpha[d], acc[db][r]);
          }
      }
      m2 = m_new;
      lds_publish<0>();
    };
    const int nbfull = (S % 128) ? nb - 1 : nb;
    for (int bb = 0; bb < nbfull; ++bb) step128(bb, std::false_type{});
    if (nbfull < nb) step128(nb - 1, std::true_type{});
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)

  // ---- epilogue ---------------------------------------------------------------------
  const float lfull = xor32_add(l);
  if constexpr (BLASST) {
    if (a.stats && g == 0 && qvalid) {
      const int rb = qi / a.block_m;
      atomicAdd(a.stats + (static_cast<size_t>(rb) * (a.B * a.H) + bh) * 2 + 0, skipped);
      atomicAdd(a.stats + (static_cast<size_t>(rb) * (a.B * a.H) + bh) * 2 + 1, static_cast<float>(ndec));  // decisions
    }
  }
  if constexpr (BLASST) {
    if (a.wave_tiles && lane == 0) {
      int* wt = a.wave_tiles + (static_cast<size_t>(bh) * a.nqb * kWaves + qb * kWaves + wave) * 2;
      wt[0] = wt_all;
      wt[1] = wt_any;
    }
  }
  if (!qvalid) return;
  const float inv_l = 1.0f / lfull;
  const int orow = a.out_row_map ? a.out_row_map[static_cast<size_t>(bh) * S + qi] : qi;
  if constexpr (BLASST) {
    if (a.row_skips && g == 0) a.row_skips[static_cast<size_t>(bh) * S + orow] = skipped;
  }
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

// Launch one instantiation (defined in the per-P-mode, per-block_n
// translation units).  bl: 0 no BLASST; BLASST with a per-row fill (1), the
// UTA fill of <= 16 bins (2) or of 32 / 64 bins (3); with block_n = 128 every
// UTA fill is bl 2.
int launch_p0(const KArgs& a, int D, bool qk_mx, int rb, int bl, bool valpha, hipStream_t st);
int launch_p1(const KArgs& a, int D, bool qk_mx, int rb, int bl, bool valpha, hipStream_t st);
int launch_p2(const KArgs& a, int D, bool qk_mx, int rb, int bl, bool valpha, hipStream_t st);
int launch_b128_p0(const KArgs& a, int D, bool qk_mx, int rb, int bl, bool valpha, hipStream_t st);
int launch_b128_p1(const KArgs& a, int D, bool qk_mx, int rb, int bl, bool valpha, hipStream_t st);
int launch_b128_p2(const KArgs& a, int D, bool qk_mx, int rb, int bl, bool valpha, hipStream_t st);

template <int P_MODE, int BN>
int launch_p(const KArgs& a, int D, bool qk_mx, int rb, int bl, bool valpha, hipStream_t st) {
  // Eight-wave workgroups (256 queries sharing each staged K / V^T tile) for
  // the dense D = 128 kernels with fp8_block Q/K, no V smoothing and
  // elementwise or dynamic P, where they measured faster than four; they
  // need s_pitch to be a multiple of 256, so that ceil(S / 256) workgroups
  // read no Q row past the pitch.  BLASST keeps four waves (its per-wave
  // statistics are laid out for 128-query workgroups).
  if constexpr (BN == 64 && P_MODE != 1) {
    if (D == 128 && !qk_mx && bl == 0 && !valpha && a.P % 256 == 0) {
      KArgs a8 = a;
      a8.nqb = (a.S + 255) / 256;
      dim3 grid8(static_cast<unsigned>(a.B * a.H * a8.nqb)), block8(8 * 64);
#define LBFQ_L8(RBV) hipLaunchKernelGGL((attn_fwd_kernel<128, false, P_MODE, RBV, 0, false, BN, 8>), grid8, block8, 0, st, a8)
      if (rb == RB_ONLINE) LBFQ_L8(RB_ONLINE);
      else if (rb == RB_ONLINE_BIAS) LBFQ_L8(RB_ONLINE_BIAS);
      else LBFQ_L8(RB_EST_BIAS);
#undef LBFQ_L8
      hipError_t e = hipGetLastError();
      if (e != hipSuccess) {
        lbfq_set_error("lbfq_attention_fwd: launch failed: %s", hipGetErrorString(e));
        return -2;
      }
      return 0;
    }
  }
  const int nblk = a.B * a.H * a.nqb;
  dim3 grid(static_cast<unsigned>(nblk)), block(kThreads);
#define LBFQ_L(DD, MX, RBV, BL, VA) \
  hipLaunchKernelGGL((attn_fwd_kernel<DD, MX, P_MODE, RBV, BL, VA, BN, kWaves>), grid, block, 0, st, a)
#define LBFQ_VA(DD, MX, RBV, BL) \
  if (valpha) LBFQ_L(DD, MX, RBV, BL, true); else LBFQ_L(DD, MX, RBV, BL, false)
#define LBFQ_BL(DD, MX, RBV)                                                                     \
  if constexpr (BN == 64) {                                                                      \
    if (bl == 3) { LBFQ_VA(DD, MX, RBV, 3); } else if (bl == 2) { LBFQ_VA(DD, MX, RBV, 2); }     \
    else if (bl == 1) { LBFQ_VA(DD, MX, RBV, 1); } else { LBFQ_VA(DD, MX, RBV, 0); }             \
  } else {                                                                                       \
    if (bl >= 2) { LBFQ_VA(DD, MX, RBV, 2); } else if (bl == 1) { LBFQ_VA(DD, MX, RBV, 1); }     \
    else { LBFQ_VA(DD, MX, RBV, 0); }                                                           \
  }
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
