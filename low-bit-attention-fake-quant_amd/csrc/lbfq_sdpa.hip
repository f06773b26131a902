// Path A of fake_quant_attention (p_requant=False, attention.py:245-321 of the
// reference) on gfx950: attention over the dequantised Q/K/V, probabilities
// not quantised.
//
// lbfq_sdpa_dequant turns the E4M3 codes of the prepass into the SDPA dtype
// exactly as the reference's dequantisers do (dtype(code * scale),
// quant_triton.py:81-109/180-198/275-298/373-396), adding the V block means
// in that dtype (attention.py:281-286).  lbfq_sdpa_fwd is a flash-style
// attention over those tensors on the 32x32x16 bf16 / fp16 MFMA with fp32
// accumulation:
//
//   no Q smoothing (qk_bias == NULL): SDPA with P in fp32 (attention.py:289-294,
//     "P stays in FP32"): one online-softmax pass; P enters the PV product as
//     two SDPA-dtype terms, its rounding and the (exact) rounding residual
//     rounded once more, i.e. with ~16 of fp32's 24 significant bits;
//   Q smoothing: s = dtype(q_deq . k_deq) * sm_scale + qm[g] . K_s * sm_scale,
//     P = dtype(softmax(s)), O = P V (attention.py:296-319).  Two passes over
//     the keys: the first forms each row's max and sum, the second rounds the
//     normalised P to the SDPA dtype -- the value the reference rounds --
//     before the PV product.  The correction comes in log2 units from lbfq_qmk.
//
// Work decomposition: one wave = 32 queries of one (b, h), NW waves per
// workgroup, 64-key tiles: NW = 8 (256 queries, one workgroup per CU, two
// waves per SIMD) when that makes at least 256 workgroups, else 4 (128
// queries, two workgroups per CU).  The workgroup's threads load each K and
// V^T tile from global memory one tile ahead and stage it in a double-buffered
// LDS area that all its waves read (one barrier per tile).  Scores are
// computed transposed, S^T = K Q^T: lane (i, g) = (lane % 32, lane / 32)
// holds query i and, in the MFMA accumulator layout, keys 8 (r / 4) + 4 g +
// r % 4 (r = 0..15) of each 32-key block.  The PV product O^T = V^T P^T
// consumes P in that layout: its k-step j of a block contracts the keys of
// registers r = 8 j .. 8 j + 7, i.e. 16 j + 4 g + {0..3} and 16 j + 8 + 4 g +
// {0..3} for lane group g; the staged V^T rows hold those eight keys next to
// each other, so a lane reads its V^T operand as one 16-byte piece.
#include <cmath>

#include "lbfq_common.h"
#include "../../include/lbfq.h"

using namespace lbfq;

namespace {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;

// C (32x32) += A (32x16) B (16x32): lane (i, g) supplies A[i][8g..8g+7] and
// B[8g..8g+7][i] as 8 packed 16-bit values.
template <int DT>
__device__ __forceinline__ v16f mfma16(const uint4& a, const uint4& b, const v16f& c) {
  if constexpr (DT == kBF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                    0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                   0, 0, 0);
}

template <int DT>
__device__ __forceinline__ uint32_t to_bits(float x) {
  if constexpr (DT == kBF16) return f32_to_bf16_bits(x);
  else return f32_to_f16_bits(x);
}
template <int DT>
__device__ __forceinline__ float from_bits(uint32_t x) {
  if constexpr (DT == kBF16) return bf16_bits_to_f32(static_cast<uint16_t>(x));
  else return f16_bits_to_f32(static_cast<uint16_t>(x));
}
template <int DT>
__device__ __forceinline__ float round_dt(float x) { return from_bits<DT>(to_bits<DT>(x)); }

// 2^(e - 127) for an E8M0 byte (e = 0 is the subnormal 2^-127)
__device__ __forceinline__ float e8m0_to_f32(uint32_t e) {
  return __uint_as_float(e ? (e << 23) : 0x00400000u);
}

// The four E4M3 codes of a word as fp32 (exact).
__device__ __forceinline__ void decode4(uint32_t w, float* x) {
  x[0] = __builtin_amdgcn_cvt_f32_fp8(static_cast<int>(w), 0);
  x[1] = __builtin_amdgcn_cvt_f32_fp8(static_cast<int>(w), 1);
  x[2] = __builtin_amdgcn_cvt_f32_fp8(static_cast<int>(w), 2);
  x[3] = __builtin_amdgcn_cvt_f32_fp8(static_cast<int>(w), 3);
}

// dtype(code * scale) as the reference's dequantisers round it: the fp32
// product, then RNE (as_f32 keeps the compiler from rounding the exact
// product to fp16 in one step).
template <int DT>
__device__ __forceinline__ uint32_t dequant_bits(float x, float sc) {
  return to_bits<DT>(as_f32(x * sc));
}

__device__ __forceinline__ float xor32_max(float v) { return fmaxf(v, __shfl_xor(v, 32, 64)); }
__device__ __forceinline__ float xor32_add(float v) { return v + __shfl_xor(v, 32, 64); }

struct SdpaArgs {
  int H, S, P;
  float sml2;  // sm_scale * log2(e)
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v_t;
  const float* bias;  // (B,H,G,P) log2 units, or null
  int G, q_group;
  void* out;
  int out_dtype;
  const int32_t* out_row_map;
};

// LDS staging of one 64-key tile, shared by the workgroup's waves and
// double-buffered: the K rows (D bf16 each, pitch KP bytes) and the V^T rows
// (64 keys each, pitch VP bytes).  The pitches are 16 bytes past a multiple of
// 128 so that the eight rows one ds_read_b128 phase touches fall on distinct
// banks.  Within each 16-key group the V^T keys are stored in the order
// 0-3, 8-11, 4-7, 12-15: lane group g's eight k-elements of a PV k-step are
// then one contiguous 16-byte read.
template <int D>
struct Stage {
  static constexpr int KP = 2 * D + 16;
  static constexpr int VP = 2 * 64 + 16;
  static constexpr int KBYTES = 64 * KP;
  static constexpr int BUF = KBYTES + D * VP;
};
// The copies of a tile per thread of an NW-wave workgroup.
template <int D, int NW>
struct Copy {
  static constexpr int T = 64 * NW;           // threads per workgroup
  static constexpr int KCH = 64 * D / 8 / T;  // 16-byte K chunks per thread
  static constexpr int VCH = D * 8 / T;       // 16-byte V^T chunks per thread
};

// global -> registers: the thread's K and V^T chunks of the tile at key0
template <int D, int NW, bool WITH_V>
__device__ __forceinline__ void stage_load(const uint16_t* kbase, const uint16_t* vbase, int P, int key0, int tid,
                                           u32x4 (&kr)[Copy<D, NW>::KCH], u32x4 (&vr)[Copy<D, NW>::VCH]) {
  using C = Copy<D, NW>;
  constexpr int CPR = D / 8;  // K chunks per row
#pragma unroll
  for (int i = 0; i < C::KCH; ++i) {
    const int c = tid + C::T * i, row = c / CPR, col = c % CPR;
    kr[i] = *reinterpret_cast<const u32x4*>(kbase + static_cast<size_t>(key0 + row) * D + 8 * col);
  }
  if constexpr (WITH_V) {
#pragma unroll
    for (int i = 0; i < C::VCH; ++i) {
      const int c = tid + C::T * i, row = c >> 3, kc = c & 7;
      vr[i] = *reinterpret_cast<const u32x4*>(vbase + static_cast<size_t>(row) * P + key0 + 8 * kc);
    }
  }
}

// registers -> LDS buffer (the key permutation of V^T applied here)
template <int D, int NW, bool WITH_V>
__device__ __forceinline__ void stage_store(uint8_t* buf, int tid, const u32x4 (&kr)[Copy<D, NW>::KCH],
                                            const u32x4 (&vr)[Copy<D, NW>::VCH]) {
  using C = Copy<D, NW>;
  constexpr int CPR = D / 8;
#pragma unroll
  for (int i = 0; i < C::KCH; ++i) {
    const int c = tid + C::T * i, row = c / CPR, col = c % CPR;
    *reinterpret_cast<u32x4*>(buf + row * Stage<D>::KP + 16 * col) = kr[i];
  }
  if constexpr (WITH_V) {
#pragma unroll
    for (int i = 0; i < C::VCH; ++i) {
      const int c = tid + C::T * i, row = c >> 3, kc = c & 7;
      // keys 16 G + 8 h + [0,4) -> positions 16 G + 4 h + [0,4); + [4,8) -> 16 G + 8 + 4 h + [0,4)
      uint8_t* rp = buf + Stage<D>::KBYTES + row * Stage<D>::VP + 2 * (16 * (kc >> 1) + 4 * (kc & 1));
      *reinterpret_cast<u32x2*>(rp) = vr[i].xy;
      *reinterpret_cast<u32x2*>(rp + 16) = vr[i].zw;
    }
  }
}

// S^T of the staged tile for the lane's query: two 32-key blocks
template <int D, int DT>
__device__ __forceinline__ void scores(const uint8_t* buf, int li, int g, const uint4 (&qop)[D / 16], v16f (&s)[2]) {
  constexpr int NKS = D / 16;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    const uint8_t* krow = buf + (32 * kb + li) * Stage<D>::KP + 16 * g;
    uint4 kop[NKS];
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) kop[ks] = *reinterpret_cast<const uint4*>(krow + 32 * ks);
#pragma unroll
    for (int r = 0; r < 16; ++r) s[kb][r] = 0.0f;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) s[kb] = mfma16<DT>(kop[ks], qop[ks], s[kb]);
  }
}

// log2-unit scores of the lane's 32 keys (register r of block kb is key
// key0 + 32 kb + 8 (r / 4) + 4 g + r % 4); in the tile that holds key S - 1,
// keys >= S are set to -inf
template <bool BIAS, int DT>
__device__ __forceinline__ void to_log2(const v16f (&s)[2], int key0, int g, int S, float sml2, const float* brow,
                                        float (&u)[32]) {
  if constexpr (BIAS) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const float4 bv = *reinterpret_cast<const float4*>(brow + key0 + 32 * kb + 8 * q4 + 4 * g);
        const float bb[4] = {bv.x, bv.y, bv.z, bv.w};
#pragma unroll
        for (int e = 0; e < 4; ++e)  // the main term rounded to DT first
          u[16 * kb + 4 * q4 + e] = fmaf(round_dt<DT>(s[kb][4 * q4 + e]), sml2, bb[e]);
      }
      // the second block's correction loads stay behind the first block's use
      // (all eight in flight at once took the kernel past 256 VGPRs)
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) u[16 * kb + r] = s[kb][r] * sml2;
  }
  if (key0 + 64 > S) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (key0 + 32 * kb + 8 * (r >> 2) + 4 * g + (r & 3) >= S) u[16 * kb + r] = -INFINITY;
  }
}

// Two fp32 values rounded (RNE) to the SDPA dtype and packed into one word,
// low half the first: one packed conversion.
template <int DT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  const f32x2 v = {a, b};
  if constexpr (DT == kBF16) return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
  else return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
}
// The two halves of a packed word as fp32 (exact).
template <int DT>
__device__ __forceinline__ float lo_of(uint32_t w) { return from_bits<DT>(w & 0xffffu); }
template <int DT>
__device__ __forceinline__ float hi_of(uint32_t w) {
  if constexpr (DT == kBF16) return __uint_as_float(w & 0xffff0000u);
  else return from_bits<DT>(w >> 16);
}

// The lane's 32 P values (score layout) as packed SDPA-dtype pairs:
// w[kb][j][k] holds registers 16 kb + 8 j + 2 k and + 1.
template <int DT>
__device__ __forceinline__ void pack(const float (&p)[32], uint32_t (&w)[2][2][4]) {
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int r = 16 * kb + 8 * j + 2 * k;
        w[kb][j][k] = pack2<DT>(p[r], p[r + 1]);
      }
}

// P as its SDPA-dtype rounding (whi) plus the rounding's exact residual,
// rounded once more (wlo): p = hi + lo to ~16 significant bits.
template <int DT>
__device__ __forceinline__ void pack_split(const float (&p)[32], uint32_t (&whi)[2][2][4], uint32_t (&wlo)[2][2][4]) {
  pack<DT>(p, whi);
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int r = 16 * kb + 8 * j + 2 * k;
        const uint32_t h = whi[kb][j][k];
        wlo[kb][j][k] = pack2<DT>(p[r] - lo_of<DT>(h), p[r + 1] - hi_of<DT>(h));  // exact differences
      }
}

// O^T (D x 32 queries) += V^T (D x 64 keys) P^T for the staged tile
template <int D, int DT>
__device__ __forceinline__ void pv(const uint8_t* buf, int li, int g, const uint32_t (&w)[2][2][4],
                                   v16f (&acc)[D / 32]) {
  const uint8_t* vb = buf + Stage<D>::KBYTES + li * Stage<D>::VP + 16 * g;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint4 pb = make_uint4(w[kb][j][0], w[kb][j][1], w[kb][j][2], w[kb][j][3]);
#pragma unroll
      for (int db = 0; db < D / 32; ++db) {
        const uint4 va = *reinterpret_cast<const uint4*>(vb + 32 * db * Stage<D>::VP + 32 * (2 * kb + j));
        acc[db] = mfma16<DT>(va, pb, acc[db]);
      }
    }
  }
}

template <int D, bool BIAS, int DT, int NW>
__global__ void __launch_bounds__(NW * 64, 2) sdpa_fwd_kernel(const SdpaArgs a) {
  constexpr int NKS = D / 16, NDB = D / 32;
  using St = Stage<D>;
  __shared__ __align__(16) uint8_t lds[2 * St::BUF];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int li = lane & 31, g = lane >> 5;
  constexpr int QB = 32 * NW;  // queries per workgroup
  const int nqb = (a.P + QB - 1) / QB;
  const int bh = blockIdx.x / nqb, qb = blockIdx.x - bh * nqb;
  const int S = a.S, P = a.P;
  // every wave takes part in the staging and the barriers; a wave whose rows
  // are all padding (rows [S, P) of q are zero; rows past the pitch read the
  // last one) computes and stores nothing
  const int qi = qb * QB + wave * 32 + li;

  uint4 qop[NKS];
  {
    const uint16_t* qrow = a.q + (static_cast<size_t>(bh) * P + (qi < P ? qi : P - 1)) * D + 8 * g;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) qop[ks] = *reinterpret_cast<const uint4*>(qrow + 16 * ks);
  }
  const float* brow = nullptr;
  if constexpr (BIAS) {
    int grp = (qi < S ? qi : S - 1) / a.q_group;
    grp = grp < a.G ? grp : a.G - 1;
    brow = a.bias + (static_cast<size_t>(bh) * a.G + grp) * P;
  }
  const uint16_t* kbase = a.k + static_cast<size_t>(bh) * P * D;
  const uint16_t* vbase = a.v_t + static_cast<size_t>(bh) * D * P;
  const int nt = (S + 63) / 64;
  u32x4 kr[Copy<D, NW>::KCH], vr[Copy<D, NW>::VCH];

  v16f acc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[db][r] = 0.0f;

  float inv_l = 1.0f;
  if constexpr (BIAS) {
    // pass 1: the row's max and sum (each lane over its own keys, merged at the end)
    float m = -INFINITY, l = 0.0f;
    stage_load<D, NW, false>(kbase, vbase, P, 0, tid, kr, vr);
    stage_store<D, NW, false>(lds, tid, kr, vr);
    __syncthreads();
    for (int t = 0; t < nt; ++t) {
      const uint8_t* buf = lds + (t & 1) * St::BUF;
      v16f s[2];
      scores<D, DT>(buf, li, g, qop, s);
      stage_load<D, NW, false>(kbase, vbase, P, 64 * (t + 1 < nt ? t + 1 : t), tid, kr, vr);
      float u[32];
      to_log2<true, DT>(s, 64 * t, g, S, a.sml2, brow, u);
      float tmax = u[0];
#pragma unroll
      for (int j = 1; j < 32; ++j) tmax = fmaxf(tmax, u[j]);
      const float m_new = fmaxf(m, tmax);
      const float ms = m_new == -INFINITY ? 0.0f : m_new;  // a lane whose keys so far are all masked
      float sum = 0.0f;
#pragma unroll
      for (int j = 0; j < 32; ++j) sum += __builtin_amdgcn_exp2f(u[j] - ms);
      l = l * __builtin_amdgcn_exp2f(m - ms) + sum;
      m = m_new;
      stage_store<D, NW, false>(lds + ((t + 1) & 1) * St::BUF, tid, kr, vr);  // idle after the last tile
      __syncthreads();
    }
    const float mo = __shfl_xor(m, 32, 64), lo = __shfl_xor(l, 32, 64);
    const float mrow = fmaxf(m, mo);  // finite: key 0 is valid
    const float inv = 1.0f / (l * __builtin_amdgcn_exp2f(m - mrow) + lo * __builtin_amdgcn_exp2f(mo - mrow));
    // pass 2: P = dtype(exp2(u - max) / sum), O = P V
    stage_load<D, NW, true>(kbase, vbase, P, 0, tid, kr, vr);
    stage_store<D, NW, true>(lds, tid, kr, vr);
    __syncthreads();
    for (int t = 0; t < nt; ++t) {
      const uint8_t* buf = lds + (t & 1) * St::BUF;
      v16f s[2];
      scores<D, DT>(buf, li, g, qop, s);
      stage_load<D, NW, true>(kbase, vbase, P, 64 * (t + 1 < nt ? t + 1 : t), tid, kr, vr);
      float u[32];
      to_log2<true, DT>(s, 64 * t, g, S, a.sml2, brow, u);
#pragma unroll
      for (int j = 0; j < 32; ++j) u[j] = __builtin_amdgcn_exp2f(u[j] - mrow) * inv;
      uint32_t w[2][2][4];
      pack<DT>(u, w);
      pv<D, DT>(buf, li, g, w, acc);
      stage_store<D, NW, true>(lds + ((t + 1) & 1) * St::BUF, tid, kr, vr);  // idle after the last tile
      __syncthreads();
    }
  } else {
    // online softmax; P as its SDPA-dtype rounding plus the rounded residual
    float m = -INFINITY, l = 0.0f;
    stage_load<D, NW, true>(kbase, vbase, P, 0, tid, kr, vr);
    stage_store<D, NW, true>(lds, tid, kr, vr);
    __syncthreads();
    for (int t = 0; t < nt; ++t) {
      const uint8_t* buf = lds + (t & 1) * St::BUF;
      v16f s[2];
      scores<D, DT>(buf, li, g, qop, s);
      stage_load<D, NW, true>(kbase, vbase, P, 64 * (t + 1 < nt ? t + 1 : t), tid, kr, vr);
      float u[32];
      to_log2<false, DT>(s, 64 * t, g, S, a.sml2, nullptr, u);
      float tmax = u[0];
#pragma unroll
      for (int j = 1; j < 32; ++j) tmax = fmaxf(tmax, u[j]);
      const float m_new = fmaxf(m, xor32_max(tmax));  // finite: key 64 t is valid
      const float alpha = __builtin_amdgcn_exp2f(m - m_new);  // 0 on the first tile
      m = m_new;
      float sum = 0.0f;
#pragma unroll
      for (int j = 0; j < 32; ++j) {
        u[j] = __builtin_amdgcn_exp2f(u[j] - m_new);
        sum += u[j];
      }
      l = l * alpha + sum;
      if (__any(alpha != 1.0f)) {
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[db][r] *= alpha;
      }
      uint32_t whi[2][2][4], wlo[2][2][4];
      pack_split<DT>(u, whi, wlo);
      pv<D, DT>(buf, li, g, whi, acc);
      pv<D, DT>(buf, li, g, wlo, acc);
      stage_store<D, NW, true>(lds + ((t + 1) & 1) * St::BUF, tid, kr, vr);  // idle after the last tile
      __syncthreads();
    }
    inv_l = 1.0f / xor32_add(l);
  }

  // epilogue: O rounded to the SDPA dtype (the reference's output), then to the caller's dtype
  if (qi >= S) return;
  const int b = bh / a.H, h = bh - b * a.H;
  const int orow = a.out_row_map ? a.out_row_map[static_cast<size_t>(bh) * S + qi] : qi;
  const size_t obase = ((static_cast<size_t>(b) * S + orow) * a.H + h) * D;
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const int d0 = 32 * db + 8 * r4 + 4 * g;
      float o[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) o[k] = round_dt<DT>(acc[db][4 * r4 + k] * inv_l);
      if (a.out_dtype == kF32) {
        *reinterpret_cast<float4*>(reinterpret_cast<float*>(a.out) + obase + d0) = make_float4(o[0], o[1], o[2], o[3]);
      } else {
        uint32_t wv[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const uint32_t lo16 = a.out_dtype == kBF16 ? f32_to_bf16_bits(o[2 * k]) : f32_to_f16_bits(o[2 * k]);
          const uint32_t hi16 = a.out_dtype == kBF16 ? f32_to_bf16_bits(o[2 * k + 1]) : f32_to_f16_bits(o[2 * k + 1]);
          wv[k] = lo16 | (hi16 << 16);
        }
        *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(a.out) + obase + d0) = make_uint2(wv[0], wv[1]);
      }
    }
  }
}

// ---- dequantisation into the SDPA dtype -----------------------------------------

// Q or K codes (BH, P, D) -> (BH, P, D): rows < S dtype(code * scale), rows >= S zero.
// 8 elements per thread.  qk_mx 0: scale (BH, S / blk) fp32 per blk rows;
// 1: scale (BH, P, D / blk) E8M0 per blk columns.
template <int DT>
__global__ void qk_dequant_kernel(const uint8_t* codes, int qk_mx, const void* scale, int blk, int64_t BH, int S,
                                  int P, int D, uint16_t* out) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int per_row = D / 8;
  if (t >= BH * P * per_row) return;
  const int c8 = static_cast<int>(t % per_row);
  const int64_t rowi = t / per_row;  // bh * P + r
  const int r = static_cast<int>(rowi % P);
  const int64_t bh = rowi / P;
  uint4 o = make_uint4(0, 0, 0, 0);
  if (r < S) {
    float sc;
    if (qk_mx) sc = e8m0_to_f32(reinterpret_cast<const uint8_t*>(scale)[rowi * (D / blk) + (8 * c8) / blk]);
    else sc = reinterpret_cast<const float*>(scale)[bh * (S / blk) + r / blk];
    const uint2 c = reinterpret_cast<const uint2*>(codes)[t];
    float x[8];
    decode4(c.x, x);
    decode4(c.y, x + 4);
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) w[k] = dequant_bits<DT>(x[2 * k], sc) | (dequant_bits<DT>(x[2 * k + 1], sc) << 16);
    o = make_uint4(w[0], w[1], w[2], w[3]);
  }
  reinterpret_cast<uint4*>(out)[t] = o;
}

// V^T codes (BH, D, P) -> (BH, D, P): keys < S dtype(dtype(code * scale) + dtype(alpha)),
// keys >= S zero.  8 keys per thread.  v_kind 0: scale (BH, D) fp32; 1: (BH, S / vb)
// fp32; 2: (BH, S / vb, D) E8M0.  alpha: (BH, S / vsb, D) fp32 or null.
template <int DT>
__global__ void v_dequant_t_kernel(const uint8_t* codes_t, int v_kind, const void* scale, int vb, const float* alpha,
                                   int vsb, int64_t BH, int S, int P, int D, uint16_t* out) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int per_row = P / 8;
  if (t >= BH * D * per_row) return;
  const int k0 = 8 * static_cast<int>(t % per_row);
  const int64_t rowi = t / per_row;  // bh * D + d
  const int d = static_cast<int>(rowi % D);
  const int64_t bh = rowi / D;
  uint4 o = make_uint4(0, 0, 0, 0);
  if (k0 < S) {
    const uint2 c = reinterpret_cast<const uint2*>(codes_t)[t];
    const int nvb = v_kind ? S / vb : 1, nvsb = alpha ? S / vsb : 1;
    // the blocks of keys k0 .. k0 + 7, advanced as the keys cross a boundary
    int sb = v_kind ? k0 / vb : 0, sb_next = v_kind ? (sb + 1) * vb : 0;
    int ab = alpha ? k0 / vsb : 0, ab_next = alpha ? (ab + 1) * vsb : 0;
    float x8[8];
    decode4(c.x, x8);
    decode4(c.y, x8 + 4);
    uint32_t hv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int k = k0 + e;
      if (v_kind && k >= sb_next) { ++sb; sb_next += vb; }
      if (alpha && k >= ab_next) { ++ab; ab_next += vsb; }
      hv[e] = 0u;
      if (k < S) {
        float sc;
        if (v_kind == 0) sc = reinterpret_cast<const float*>(scale)[rowi];
        else if (v_kind == 1) sc = reinterpret_cast<const float*>(scale)[bh * nvb + sb];
        else sc = e8m0_to_f32(reinterpret_cast<const uint8_t*>(scale)[(bh * nvb + sb) * D + d]);
        uint32_t bits = dequant_bits<DT>(x8[e], sc);
        if (alpha) {
          bits = to_bits<DT>(as_f32(from_bits<DT>(bits) + round_dt<DT>(alpha[(bh * nvsb + ab) * D + d])));
        }
        hv[e] = bits;
      }
    }
    o = make_uint4(hv[0] | (hv[1] << 16), hv[2] | (hv[3] << 16), hv[4] | (hv[5] << 16), hv[6] | (hv[7] << 16));
  }
  reinterpret_cast<uint4*>(out)[t] = o;
}

}  // namespace

extern "C" int lbfq_sdpa_dequant(const lbfq_sdpa_dequant_params* p, lbfq_stream_t stream) {
  LBFQ_CHECK_ARG(p, "lbfq_sdpa_dequant: null params");
  LBFQ_CHECK_ARG(p->D == 64 || p->D == 128, "lbfq_sdpa_dequant: D must be 64 or 128");
  LBFQ_CHECK_ARG(p->B > 0 && p->H > 0 && p->S > 0 && p->s_pitch >= p->S && p->s_pitch % 128 == 0,
                 "lbfq_sdpa_dequant: s_pitch must be >= S and a multiple of 128");
  LBFQ_CHECK_ARG(p->s_pitch < (int64_t{1} << 30) && p->B * p->H * p->s_pitch * p->D / 8 < (int64_t{1} << 39),
                 "lbfq_sdpa_dequant: problem too large");
  LBFQ_CHECK_ARG(p->q_codes && p->k_codes && p->v_codes_t && p->q_scale && p->k_scale && p->v_scale,
                 "lbfq_sdpa_dequant: missing codes or scales");
  LBFQ_CHECK_ARG(p->q_out && p->k_out && p->v_t_out, "lbfq_sdpa_dequant: missing output");
  LBFQ_CHECK_ARG(p->sdpa_dtype == kBF16 || p->sdpa_dtype == kF16, "lbfq_sdpa_dequant: the SDPA dtype is bf16 or fp16");
  LBFQ_CHECK_ARG(p->qk_mx ? (p->qk_block >= 8 && p->qk_block <= p->D && (p->qk_block & (p->qk_block - 1)) == 0)
                          : (p->qk_block > 0 && p->S % p->qk_block == 0),
                 "lbfq_sdpa_dequant: bad Q/K block %d", p->qk_block);
  LBFQ_CHECK_ARG(p->v_kind >= 0 && p->v_kind <= 2, "lbfq_sdpa_dequant: bad v_kind %d", p->v_kind);
  LBFQ_CHECK_ARG(p->v_kind == 0 || (p->v_block > 0 && p->S % p->v_block == 0), "lbfq_sdpa_dequant: bad V block %d",
                 p->v_block);
  LBFQ_CHECK_ARG(!p->v_alpha || (p->v_smooth_block > 0 && p->S % p->v_smooth_block == 0),
                 "lbfq_sdpa_dequant: bad V smoothing block %d", p->v_smooth_block);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t BH = p->B * p->H;
  const int S = static_cast<int>(p->S), P = static_cast<int>(p->s_pitch), D = static_cast<int>(p->D);
  const dim3 gqk(static_cast<unsigned>((BH * P * (D / 8) + 255) / 256)), gv(static_cast<unsigned>((BH * D * (P / 8) + 255) / 256));
  const dim3 block(256);
  const bool bf = p->sdpa_dtype == kBF16;
  const void* codes[2] = {p->q_codes, p->k_codes};
  const void* scales[2] = {p->q_scale, p->k_scale};
  void* outs[2] = {p->q_out, p->k_out};
  for (int i = 0; i < 2; ++i) {
    const uint8_t* c = static_cast<const uint8_t*>(codes[i]);
    uint16_t* o = static_cast<uint16_t*>(outs[i]);
    if (bf)
      hipLaunchKernelGGL(qk_dequant_kernel<kBF16>, gqk, block, 0, st, c, p->qk_mx, scales[i], p->qk_block, BH, S, P, D, o);
    else
      hipLaunchKernelGGL(qk_dequant_kernel<kF16>, gqk, block, 0, st, c, p->qk_mx, scales[i], p->qk_block, BH, S, P, D, o);
  }
  uint16_t* vo = static_cast<uint16_t*>(p->v_t_out);
  if (bf)
    hipLaunchKernelGGL(v_dequant_t_kernel<kBF16>, gv, block, 0, st, p->v_codes_t, p->v_kind, p->v_scale, p->v_block,
                       p->v_alpha, p->v_smooth_block, BH, S, P, D, vo);
  else
    hipLaunchKernelGGL(v_dequant_t_kernel<kF16>, gv, block, 0, st, p->v_codes_t, p->v_kind, p->v_scale, p->v_block,
                       p->v_alpha, p->v_smooth_block, BH, S, P, D, vo);
  LBFQ_LAUNCH_CHECK("lbfq_sdpa_dequant");
  return 0;
}

extern "C" int lbfq_sdpa_fwd(const lbfq_sdpa_params* p, lbfq_stream_t stream) {
  LBFQ_CHECK_ARG(p, "lbfq_sdpa_fwd: null params");
  LBFQ_CHECK_ARG(p->D == 64 || p->D == 128, "lbfq_sdpa_fwd: D must be 64 or 128");
  LBFQ_CHECK_ARG(p->B > 0 && p->H > 0 && p->S > 0 && p->s_pitch >= p->S && p->s_pitch % 128 == 0,
                 "lbfq_sdpa_fwd: s_pitch must be >= S and a multiple of 128");
  LBFQ_CHECK_ARG(p->s_pitch < (int64_t{1} << 30) && p->B * p->H * (p->s_pitch / 128) < (int64_t{1} << 31),
                 "lbfq_sdpa_fwd: problem too large");
  LBFQ_CHECK_ARG(p->q && p->k && p->v_t && p->out, "lbfq_sdpa_fwd: missing tensor");
  LBFQ_CHECK_ARG(p->sdpa_dtype == kBF16 || p->sdpa_dtype == kF16, "lbfq_sdpa_fwd: the SDPA dtype is bf16 or fp16");
  LBFQ_CHECK_ARG(p->out_dtype >= kF32 && p->out_dtype <= kBF16, "lbfq_sdpa_fwd: bad output dtype %d", p->out_dtype);
  LBFQ_CHECK_ARG(!p->qk_bias || (p->groups > 0 && p->q_group > 0), "lbfq_sdpa_fwd: bad qm groups");
  SdpaArgs a{};
  a.H = static_cast<int>(p->H);
  a.S = static_cast<int>(p->S);
  a.P = static_cast<int>(p->s_pitch);
  a.sml2 = p->sm_scale * kLog2e;
  a.q = static_cast<const uint16_t*>(p->q);
  a.k = static_cast<const uint16_t*>(p->k);
  a.v_t = static_cast<const uint16_t*>(p->v_t);
  a.bias = p->qk_bias;
  a.G = p->qk_bias ? static_cast<int>(p->groups) : 1;
  a.q_group = p->qk_bias ? p->q_group : 1;
  a.out = p->out;
  a.out_dtype = p->out_dtype;
  a.out_row_map = p->out_row_map;
  // eight-wave workgroups (256 queries, one per CU) where there are enough of
  // them to fill the chip; four-wave ones (two per CU) for small problems
  const int64_t nwg8 = p->B * p->H * ((p->s_pitch + 255) / 256);
  const bool w8 = nwg8 >= 256;
  const dim3 grid(static_cast<unsigned>(w8 ? nwg8 : p->B * p->H * (p->s_pitch / 128))), block(w8 ? 512 : 256);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool bias = p->qk_bias != nullptr, bf = p->sdpa_dtype == kBF16;
#define LBFQ_SD(DD, BI, DT)                                                             \
  do {                                                                                  \
    if (w8) hipLaunchKernelGGL((sdpa_fwd_kernel<DD, BI, DT, 8>), grid, block, 0, st, a); \
    else hipLaunchKernelGGL((sdpa_fwd_kernel<DD, BI, DT, 4>), grid, block, 0, st, a);    \
  } while (0)
#define LBFQ_SD_DT(DD, BI) \
  if (bf) LBFQ_SD(DD, BI, kBF16); else LBFQ_SD(DD, BI, kF16)
#define LBFQ_SD_BI(DD) \
  if (bias) { LBFQ_SD_DT(DD, true); } else { LBFQ_SD_DT(DD, false); }
  if (p->D == 128) { LBFQ_SD_BI(128) } else { LBFQ_SD_BI(64) }
#undef LBFQ_SD_BI
#undef LBFQ_SD_DT
#undef LBFQ_SD
  LBFQ_LAUNCH_CHECK("lbfq_sdpa_fwd");
  return 0;
}
