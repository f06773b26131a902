// qm . K_smooth products for Q smoothing (gfx950), on the fp32 matrix cores.
//
//   bias[b,h,g,n] = (qm[b,g,h,:] . K_s[b,n,h,:]) * scale         (fp32)
//   rowmax[b,h,g] = max_n bias[b,h,g,n]
// The attention path uses scale = sm_scale * log2(e) (scores in log2 units).
//
// bias is the per-key correction the reference adds to every score inside the
// attention K-loop (attention_triton.py:156-160); rowmax is the qm_k row-max
// estimate (attention.py:366-395), shared by the q_group rows of a group.
//
// K_s is formed on the fly from K: K_s = round_to_dtype(K[gather[n]] - mean),
// the same rounding the quantiser applies (so the smoothed K never goes to
// HBM); with mean == NULL the input is already the smoothed K.
//
// Work decomposition: one workgroup = 4 waves = 128 keys of one (b, h); each
// wave holds the smoothed rows of its 32 keys as the B operand of
// v_mfma_f32_32x32x2_f32 (lane (i, half) supplies key i and the 64 (or 32)
// contiguous dimensions d in [half*D/2, (half+1)*D/2): MFMA step s contracts
// d = half*D/2 + s in both operands), loops over chunks of 32 groups (A = qm
// rows, read from L2), and writes the 32x32 output block: for a fixed
// accumulator register the 32 lanes of a half hold 32 consecutive keys of one
// group, so the stores are coalesced.  The 4 waves combine their per-group
// maxima in LDS; one ordered-integer atomicMax per group and workgroup.
#include "lbfq_common.h"
#include "../../include/lbfq.h"

using namespace lbfq;

namespace {

typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kKeysPerWave = 32;
constexpr int kWaves = 4;
constexpr int kKeysPerBlock = kKeysPerWave * kWaves;

__device__ __forceinline__ uint32_t ordered_bits(float f) {
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float from_ordered_bits(uint32_t u) {
  return __uint_as_float((u & 0x80000000u) ? (u & 0x7fffffffu) : ~u);
}

// max over the 32 lanes of each half-wave (xor 1, 2, 4, 8, 16)
__device__ __forceinline__ float half_max(float v) {
#pragma unroll
  for (int m = 1; m < 32; m <<= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

template <int D>
__global__ void __launch_bounds__(256) qmk_kernel(const float* qm, const void* ks, int dt, const int32_t* gather,
                                                  const float* mean, int64_t B, int64_t S, int64_t H, int64_t G,
                                                  float scale, float* bias, int64_t s_pitch,
                                                  uint32_t* rowmax_bits) {
  constexpr int HALF = D / 2;  // contraction steps per MFMA chain
  __shared__ float wmax[kWaves][32];
  const int64_t nkb = (S + kKeysPerBlock - 1) / kKeysPerBlock;
  const int64_t bh = blockIdx.x / nkb;
  const int64_t b = bh / H, h = bh % H;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int li = lane & 31, hf = lane >> 5;
  const int64_t n0 = (blockIdx.x % nkb) * kKeysPerBlock + wave * kKeysPerWave;
  const int64_t n = n0 + li;
  const bool nvalid = n < S;

  // B operand: smoothed key row n, dimensions [hf*HALF, hf*HALF + HALF)
  float kb[HALF];
  {
    const int64_t src = nvalid ? (gather ? gather[bh * S + n] : n) : 0;
    const int64_t base = ((b * S + src) * H + h) * D + hf * HALF;
#pragma unroll
    for (int s = 0; s < HALF; s += 8) {
      float v[8];
      if (dt == kF32) {
        const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(ks) + base + s);
        float4 x = p[0], y = p[1];
        v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w; v[4] = y.x; v[5] = y.y; v[6] = y.z; v[7] = y.w;
      } else {
        uint4 r = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(ks) + base + s);
        uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint16_t lo = static_cast<uint16_t>(w[i] & 0xffffu), hi = static_cast<uint16_t>(w[i] >> 16);
          v[2 * i] = dt == kBF16 ? bf16_bits_to_f32(lo) : f16_bits_to_f32(lo);
          v[2 * i + 1] = dt == kBF16 ? bf16_bits_to_f32(hi) : f16_bits_to_f32(hi);
        }
      }
      if (mean) {
        const float* m = mean + (b * H + h) * D + hf * HALF + s;
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = round_to_dtype(v[i] - m[i], dt);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) kb[s + i] = nvalid ? v[i] : 0.0f;
    }
  }

  for (int64_t g0 = 0; g0 < G; g0 += 32) {
    // A operand: qm row g0 + li (zero past G), same dimension half
    const int64_t gr = g0 + li;
    const bool gvalid = gr < G;
    const float* qa = qm + ((b * G + (gvalid ? gr : 0)) * H + h) * D + hf * HALF;
    v16f acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int s = 0; s < HALF; s += 4) {
      const float4 a4 = *reinterpret_cast<const float4*>(qa + s);
      const float av[4] = {a4.x, a4.y, a4.z, a4.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(gvalid ? av[i] : 0.0f, kb[s + i], acc, 0, 0, 0);
    }
    // accumulator register r of lane (li, hf): group g0 + 8*(r/4) + 4*hf + r%4, key n0 + li
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t g = g0 + 8 * (r >> 2) + 4 * hf + (r & 3);
      const float v = acc[r] * scale;
      if (bias && nvalid && g < G) bias[(bh * G + g) * s_pitch + n] = v;
      acc[r] = nvalid ? v : -INFINITY;
    }
    if (rowmax_bits) {
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = half_max(acc[r]);
      if (li == 0) {
#pragma unroll
        for (int r = 0; r < 16; ++r) wmax[wave][8 * (r >> 2) + 4 * hf + (r & 3)] = acc[r];
      }
      __syncthreads();
      if (tid < 32 && g0 + tid < G) {
        const float m = fmaxf(fmaxf(wmax[0][tid], wmax[1][tid]), fmaxf(wmax[2][tid], wmax[3][tid]));
        atomicMax(rowmax_bits + bh * G + g0 + tid, ordered_bits(m));
      }
      __syncthreads();
    }
  }
}

// bf16 inputs: K_s = bf16(K - mean) is exact in bf16, so qm . K_s runs on the
// bf16 matrix cores (v_mfma_f32_32x32x16_bf16) with qm split into three bf16
// pieces hi + mid + lo (= qm to 24 bits): every product is exact in fp32 and
// the sum is accumulated in fp32, as the fp32 path does, at several times its
// rate.  A workgroup covers 256 keys (four waves of two 32-key blocks); per
// chunk of 32 groups its threads split qm once into LDS, and every wave reads
// its A operands there.  A = 32 qm rows, B = 32 smoothed key rows; lane
// (i, half) supplies dimensions 16 ks + 8 half + [0, 8) of its row in both.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// two fp32 -> packed bf16 pair (one v_cvt_pk_bf16_f32, round to nearest even)
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  const f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

constexpr int kBfKeyBlocks = 2;  // 32-key blocks per wave

// Max over the 32 lanes of each half-wave of 16 values per lane, as a
// reduce-scatter (16 exchanges instead of 80): afterwards lane i of a half
// returns the max over the half of value index
//   8 * bit4(i) + 4 * bit3(i) + 2 * bit2(i) + bit1(i)
// (lanes i and i ^ 1 return the same one).  x is clobbered.
template <int N>  // one step: N values, exchange with lane ^ N, keep N / 2 values
__device__ __forceinline__ void half_max_step(float (&x)[16], int li) {
  const bool up = (li & N) != 0;
#pragma unroll
  for (int k = 0; k < N / 2; ++k) {
    const float keep = up ? x[k + N / 2] : x[k];
    const float give = up ? x[k] : x[k + N / 2];
    x[k] = fmaxf(keep, __shfl_xor(give, N, 64));
  }
}
__device__ __forceinline__ float half_max16(float (&x)[16], int li) {
  half_max_step<16>(x, li);
  half_max_step<8>(x, li);
  half_max_step<4>(x, li);
  half_max_step<2>(x, li);
  return fmaxf(x[0], __shfl_xor(x[0], 1, 64));
}

// qm rows split into three bf16 pieces hi + mid + lo (qm to 24 bits), once per
// (b, h, group): out[((b*H + h)*3 + piece)*G + g][dp] holds the bf16 pair of
// dimensions 2 dp, 2 dp + 1 (low half = even dimension).  With rowmax_bits,
// the same launch sets the row-max accumulators (B*H*G, ordered bits) to -inf.
template <int D>
__global__ void __launch_bounds__(256) qm_split_kernel(const float* qm, int64_t B, int64_t H, int64_t G,
                                                       uint32_t* out, uint32_t* rowmax_bits) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;  // over B*H*G*(D/2)
  if (i >= B * H * G * (D / 2)) return;
  const int dp = static_cast<int>(i % (D / 2));
  const int64_t r = i / (D / 2);
  if (rowmax_bits && dp == 0) rowmax_bits[r] = ordered_bits(-INFINITY);  // r = (b*H + h)*G + g
  const int64_t g = r % G, bh = r / G;
  const int64_t b = bh / H, h = bh % H;
  const float2 x = *reinterpret_cast<const float2*>(qm + ((b * G + g) * H + h) * D + 2 * dp);
  const uint32_t ph = pack_bf16(x.x, x.y);
  const float r0 = x.x - bf16_lo(ph), r1 = x.y - bf16_hi(ph);  // exact
  const uint32_t pm = pack_bf16(r0, r1);
  const uint32_t pl = pack_bf16(r0 - bf16_lo(pm), r1 - bf16_hi(pm));  // exact residual, rounded
  uint32_t* o = out + (bh * 3 * G + g) * (D / 2) + dp;
  o[0] = ph;
  o[G * (D / 2)] = pm;
  o[2 * G * (D / 2)] = pl;
}

// One chunk of split qm rows (32 groups x 3 pieces, D/2 words each) moved as
// 16-byte pieces: thread tid handles pieces tid, tid + 256, ...; rows past G
// are clamped to G - 1 (loads stay in bounds; those rows are never stored).
template <int D>
__device__ __forceinline__ void qm_chunk_load(u32x4 (&qv)[3 * 32 * (D / 8) / 256], const uint32_t* qh, int g0, int G,
                                              int tid) {
  constexpr int C4 = D / 8;
#pragma unroll
  for (int i = 0; i < 3 * 32 * C4 / 256; ++i) {
    const int e = i * 256 + tid;
    const int piece = e / (32 * C4), row = (e / C4) % 32, c4 = e % C4;
    const int g = min(g0 + row, G - 1);
    qv[i] = *reinterpret_cast<const u32x4*>(qh + (piece * G + g) * (D / 2) + 4 * c4);
  }
}
template <int D>
__device__ __forceinline__ void qm_chunk_stage(const u32x4 (&qv)[3 * 32 * (D / 8) / 256], uint32_t* buf, int tid) {
  constexpr int C4 = D / 8;
#pragma unroll
  for (int i = 0; i < 3 * 32 * C4 / 256; ++i) {
    const int e = i * 256 + tid;
    const int piece = e / (32 * C4), row = (e / C4) % 32, c4 = e % C4;
    *reinterpret_cast<u32x4*>(buf + (piece * 32 + row) * (D / 2 + 4) + 4 * c4) = qv[i];
  }
}

// K fp8_block quantiser fused into the qm . K_s kernel (the smoothed rows are
// already in registers): blocks of kblk in {16, 32, 64} keys, each inside one
// wave's 64 keys; amax over the block's smoothed values, sc = max(amax,
// floor) / 448, codes e4m3(clamp(K_s / sc)) with the correctly rounded
// quotient -- the arithmetic of the row-tile quantiser (lbfq_rowtile,
// quant mode fp8_block), so the codes and scales are the same bits.  Codes go
// to (B,H,kpitch,D) row n, scales to (B,H,S/kblk).
template <int D>
__device__ __forceinline__ void kquant_wave(const u32x4 (&kb)[kBfKeyBlocks][D / 16], const bool (&nvalid)[kBfKeyBlocks],
                                            int64_t bh, int64_t nw0, int li, int hf, int64_t S, uint8_t* kcodes,
                                            float* kscale, int64_t kpitch, int kblk) {
  constexpr int NKS = D / 16;
  float am[kBfKeyBlocks];
#pragma unroll
  for (int kbi = 0; kbi < kBfKeyBlocks; ++kbi) {
    float m = 0.0f;  // rows past S hold zeros
#pragma unroll
    for (int st = 0; st < NKS; ++st)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        m = fmaxf(m, fmaxf(fabsf(bf16_lo(kb[kbi][st][i])), fabsf(bf16_hi(kb[kbi][st][i]))));
    // lanes (li, hf) and (li, hf ^ 1) hold the two halves of key li's row
    m = fmaxf(m, __shfl_xor(m, 32, 64));
    // keys of one block: xor over the low log2(kblk) bits of li (kblk <= 32)
#pragma unroll
    for (int o = 1; o < 32; o <<= 1)
      if (o < kblk) m = fmaxf(m, __shfl_xor(m, o, 64));
    am[kbi] = m;
  }
  if (kblk == 64) am[0] = am[1] = fmaxf(am[0], am[1]);
#pragma unroll
  for (int kbi = 0; kbi < kBfKeyBlocks; ++kbi) {
    const float sc = fmaxf(am[kbi], kAmaxFloor) / kFp8Max, rc = 1.0f / sc;
    const int64_t n = nw0 + 32 * kbi + li;
    if (nvalid[kbi]) {
      uint8_t* row = kcodes + (bh * kpitch + n) * D;
#pragma unroll
      for (int st = 0; st < NKS; ++st) {
        float q[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          q[2 * i] = clamp448(div_by(bf16_lo(kb[kbi][st][i]), sc, rc));
          q[2 * i + 1] = clamp448(div_by(bf16_hi(kb[kbi][st][i]), sc, rc));
        }
        *reinterpret_cast<uint2*>(row + 16 * st + 8 * hf) = make_uint2(cvt4_e4m3(q), cvt4_e4m3(q + 4));
      }
    }
    // one lane per block writes its scale: the block's first key
    if (hf == 0 && (li & (kblk - 1)) == 0 && n < S && (kblk < 64 || kbi == 0))
      kscale[bh * (S / kblk) + n / kblk] = sc;
  }
}

template <int D>
__global__ void __launch_bounds__(256) qmk_bf16_kernel(const uint32_t* qsplit, const uint16_t* ks,
                                                       const int32_t* gather, const float* mean, int64_t B, int64_t S,
                                                       int64_t H, int64_t G, float scale, float* bias,
                                                       int64_t s_pitch, uint32_t* rowmax_bits, uint8_t* kcodes,
                                                       float* kscale, int64_t kpitch, int kblk) {
  constexpr int NKS = D / 16;  // MFMA k-steps
  constexpr int KPW = 32 * kBfKeyBlocks;
  __shared__ float wmax[2][kWaves][32];
  // split qm chunks, double-buffered: [buffer][piece][group][dim pair], rows
  // padded by 16 bytes so the 32 rows read together by a half-wave fall in
  // different banks
  __shared__ __attribute__((aligned(16))) uint32_t qs[2][3][32][D / 2 + 4];
  const int64_t nkb = (S + KPW * kWaves - 1) / (KPW * kWaves);
  const int64_t bh = blockIdx.x / nkb;
  const int64_t b = bh / H, h = bh % H;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int li = lane & 31, hf = lane >> 5;
  const int64_t nw0 = (blockIdx.x % nkb) * (KPW * kWaves) + wave * KPW;
  float* tb = bias ? bias + bh * G * s_pitch : nullptr;  // this head's table

  // B operands: smoothed rows of the wave's keys, bf16 packed, per k-step
  u32x4 kb[kBfKeyBlocks][NKS];
  bool nvalid[kBfKeyBlocks];
#pragma unroll
  for (int kbi = 0; kbi < kBfKeyBlocks; ++kbi) nvalid[kbi] = nw0 + 32 * kbi + li < S;
  // Smoothed rows -> B operands.  The rows are read coalesced (16 lanes per
  // 256-byte row, 4 rows per instruction) into a per-wave LDS staging area
  // (the qm chunk buffers, not yet in use), one 32-key block at a time, and
  // read back in the MFMA layout: lane (li, hf) takes dimensions
  // 16 st + 8 hf + [0, 8) of key li.  16-byte chunk c of row r sits at chunk
  // slot c ^ (r & 15), so both the row writes and the column reads spread
  // over the LDS banks.
  {
    uint8_t* stg = reinterpret_cast<uint8_t*>(&qs[0][0][0][0]) + wave * (32 * D * 2);
    constexpr int CPR = D / 8;          // 16-byte chunks per row
    constexpr int RPI = 64 / CPR;       // rows per load instruction
    const int cl = lane % CPR, rl = lane / CPR;
#pragma unroll
    for (int kbi = 0; kbi < kBfKeyBlocks; ++kbi) {
      uint4 raw[32 / RPI];
#pragma unroll
      for (int j = 0; j < 32 / RPI; ++j) {
        const int r = rl + RPI * j;
        const int64_t n = nw0 + 32 * kbi + r;
        const int64_t src = n < S ? (gather ? gather[bh * S + n] : n) : 0;
        raw[j] = *reinterpret_cast<const uint4*>(ks + ((b * S + src) * H + h) * D + 8 * cl);
      }
#pragma unroll
      for (int j = 0; j < 32 / RPI; ++j) {
        const int r = rl + RPI * j;
        *reinterpret_cast<uint4*>(stg + r * (D * 2) + 16 * (cl ^ (r & (CPR - 1)))) = raw[j];
      }
#pragma unroll
      for (int st = 0; st < NKS; ++st) {
        const int d0 = 16 * st + 8 * hf;
        const int c = 2 * st + hf;
        const uint4 r = *reinterpret_cast<const uint4*>(stg + li * (D * 2) + 16 * (c ^ (li & (CPR - 1))));
        const uint32_t w[4] = {r.x, r.y, r.z, r.w};
        float x[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          x[2 * i] = bf16_bits_to_f32(static_cast<uint16_t>(w[i] & 0xffffu));
          x[2 * i + 1] = bf16_bits_to_f32(static_cast<uint16_t>(w[i] >> 16));
        }
        if (mean) {
          const float4 m0 = *reinterpret_cast<const float4*>(mean + bh * D + d0);
          const float4 m1 = *reinterpret_cast<const float4*>(mean + bh * D + d0 + 4);
          const float mm[8] = {m0.x, m0.y, m0.z, m0.w, m1.x, m1.y, m1.z, m1.w};
#pragma unroll
          for (int i = 0; i < 8; ++i) x[i] -= mm[i];  // rounded to bf16 by the packing
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) kb[kbi][st][i] = nvalid[kbi] ? pack_bf16(x[2 * i], x[2 * i + 1]) : 0u;
      }
    }
  }
  if (kcodes) kquant_wave<D>(kb, nvalid, bh, nw0, li, hf, S, kcodes, kscale, kpitch, kblk);

  // Split qm chunks (32 groups x 3 pieces) of this head, moved as 16-byte
  // pieces: loaded into registers one chunk ahead and written into the other
  // LDS buffer right after the chunk's MFMAs, before the chunk's table stores
  // are issued.  Stores and loads share one completion counter, so the wait
  // for those loads covers only stores of the previous chunk, which have had a
  // whole chunk of MFMAs to drain.
  constexpr int C4 = D / 8;                          // 16-byte pieces per split row
  constexpr int NCP = 3 * 32 * C4 / 256;             // pieces per thread per chunk
  static_assert(NCP * 256 == 3 * 32 * C4, "chunk copy must tile the workgroup");
  const int Gi = static_cast<int>(G);
  u32x4 qv[NCP];
  const uint32_t* qh = qsplit + bh * 3 * G * (D / 2);
  const int nch = (Gi + 31) / 32;
  const bool keys_full = nw0 + KPW <= S;  // wave-uniform
  const uint32_t sp = static_cast<uint32_t>(s_pitch);
  qm_chunk_load<D>(qv, qh, 0, Gi, tid);
  __syncthreads();  // every wave has read its K rows out of the staging area
  qm_chunk_stage<D>(qv, &qs[0][0][0][0], tid);
  __syncthreads();
  qm_chunk_load<D>(qv, qh, 32, Gi, tid);  // rows are clamped to G - 1, so these loads are always in bounds
  for (int c = 0; c < nch; ++c) {
    const int g0 = 32 * c, buf = c & 1;
    v16f acc[kBfKeyBlocks];
#pragma unroll
    for (int kbi = 0; kbi < kBfKeyBlocks; ++kbi)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[kbi][r] = 0.0f;
#pragma unroll
    for (int st = 0; st < NKS; ++st) {
      const int dp = (16 * st + 8 * hf) / 2;
      const bf16x8 al = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(&qs[buf][2][li][dp]));
      const bf16x8 am = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(&qs[buf][1][li][dp]));
      const bf16x8 ah = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(&qs[buf][0][li][dp]));
#pragma unroll
      for (int kbi = 0; kbi < kBfKeyBlocks; ++kbi) {
        const bf16x8 bb = __builtin_bit_cast(bf16x8, kb[kbi][st]);
        acc[kbi] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, bb, acc[kbi], 0, 0, 0);
        acc[kbi] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(am, bb, acc[kbi], 0, 0, 0);
        acc[kbi] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bb, acc[kbi], 0, 0, 0);
      }
    }
    qm_chunk_stage<D>(qv, &qs[buf ^ 1][0][0][0], tid);  // read by the next chunk (if any), after this chunk's barrier
    // accumulator register r of lane (li, hf): group g0 + 8*(r/4) + 4*hf + r%4, key (block) + li;
    // table offsets (32-bit, within this head's table): row g0 + 4 hf + c_r,
    // c_r = 8 (r / 4) + r % 4, column key
    float gmax[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) gmax[r] = -INFINITY;
    if (keys_full && g0 + 32 <= Gi) {
#pragma unroll
      for (int kbi = 0; kbi < kBfKeyBlocks; ++kbi) {
        const uint32_t o0 = static_cast<uint32_t>(g0 + 4 * hf) * sp + static_cast<uint32_t>(nw0 + 32 * kbi + li);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float v = acc[kbi][r] * scale;
          if (tb) {
            const uint32_t o = o0 + static_cast<uint32_t>(8 * (r >> 2) + (r & 3)) * sp;
            *reinterpret_cast<float*>(reinterpret_cast<char*>(tb) + (o << 2)) = v;  // 32-bit byte offset
          }
          gmax[r] = fmaxf(gmax[r], v);
        }
      }
    } else {
#pragma unroll
      for (int kbi = 0; kbi < kBfKeyBlocks; ++kbi) {
        const uint32_t o0 = static_cast<uint32_t>(g0 + 4 * hf) * sp + static_cast<uint32_t>(nw0 + 32 * kbi + li);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float v = acc[kbi][r] * scale;
          const int g = g0 + 8 * (r >> 2) + 4 * hf + (r & 3);
          if (tb && nvalid[kbi] && g < Gi) {
            const uint32_t o = o0 + static_cast<uint32_t>(8 * (r >> 2) + (r & 3)) * sp;
            *reinterpret_cast<float*>(reinterpret_cast<char*>(tb) + (o << 2)) = v;
          }
          gmax[r] = fmaxf(gmax[r], nvalid[kbi] ? v : -INFINITY);
        }
      }
    }
    if (rowmax_bits) {
      const float m = half_max16(gmax, li);  // max of register ridx over the half's keys
      const int ridx = ((li >> 4) & 1) * 8 + ((li >> 3) & 1) * 4 + ((li >> 2) & 1) * 2 + ((li >> 1) & 1);
      if ((li & 1) == 0) wmax[buf][wave][8 * (ridx >> 2) + 4 * hf + (ridx & 3)] = m;
    }
    // the next chunk's qm and this chunk's maxima are visible; every wave has
    // read qs[buf] (rewritten in the chunk after next)
    __syncthreads();
    qm_chunk_load<D>(qv, qh, g0 + 64, Gi, tid);
    if (rowmax_bits && tid < 32 && g0 + tid < Gi) {
      const float m = fmaxf(fmaxf(wmax[buf][0][tid], wmax[buf][1][tid]), fmaxf(wmax[buf][2][tid], wmax[buf][3][tid]));
      atomicMax(rowmax_bits + bh * G + g0 + tid, ordered_bits(m));
    }
  }
}

__global__ void fill_ordered_kernel(uint32_t* p, int64_t n) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = ordered_bits(-INFINITY);
}

__global__ void decode_ordered_kernel(uint32_t* p, int64_t n) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) reinterpret_cast<float*>(p)[i] = from_ordered_bits(p[i]);
}

}  // namespace

namespace {

int qmk_launch(const float* qm, const void* ks, int ks_dtype, const int32_t* gather, const float* ks_mean, int64_t B,
               int64_t S, int64_t H, int64_t D, int64_t G, float scale, float* bias, int64_t s_pitch, float* rowmax,
               uint32_t* qm_split, uint8_t* k_codes, int64_t k_pitch, float* k_scale, int64_t k_block,
               lbfq_stream_t stream) {
  LBFQ_CHECK_ARG(qm && ks && (bias || rowmax), "lbfq_qmk: null pointer");
  LBFQ_CHECK_ARG(D == 64 || D == 128, "lbfq_qmk: D must be 64 or 128");
  LBFQ_CHECK_ARG(ks_dtype >= 0 && ks_dtype <= 2, "lbfq_qmk: bad dtype %d", ks_dtype);
  LBFQ_CHECK_ARG(B > 0 && H > 0 && G > 0 && S > 0 && (!bias || s_pitch >= S), "lbfq_qmk: bad sizes");
  hipStream_t st = static_cast<hipStream_t>(stream);
  uint32_t* rb = reinterpret_cast<uint32_t*>(rowmax);
  const int64_t nr = B * H * G;
  // bf16 K: the bf16 matrix-core kernel (its table offsets within one head are 32-bit)
  if (ks_dtype == kBF16 && (!bias || G * s_pitch * 4 < (int64_t{1} << 32))) {
    LBFQ_CHECK_ARG(qm_split, "lbfq_qmk: bf16 K needs the qm_split workspace (B*H*3*G*D/2 words)");
    const int64_t kpb = 32 * kBfKeyBlocks * kWaves;
    const int64_t nb = B * H * ((S + kpb - 1) / kpb);
    LBFQ_CHECK_ARG(nb < (int64_t{1} << 31), "lbfq_qmk: grid too large");
    const uint16_t* k16 = static_cast<const uint16_t*>(ks);
    const int64_t ns = B * H * G * (D / 2);
    const dim3 gs(static_cast<unsigned>((ns + 255) / 256));
    if (D == 128) {
      hipLaunchKernelGGL(qm_split_kernel<128>, gs, dim3(256), 0, st, qm, B, H, G, qm_split, rb);
      hipLaunchKernelGGL(qmk_bf16_kernel<128>, dim3(static_cast<unsigned>(nb)), dim3(256), 0, st, qm_split, k16,
                         gather, ks_mean, B, S, H, G, scale, bias, s_pitch, rb, k_codes, k_scale, k_pitch,
                         static_cast<int>(k_block));
    } else {
      hipLaunchKernelGGL(qm_split_kernel<64>, gs, dim3(256), 0, st, qm, B, H, G, qm_split, rb);
      hipLaunchKernelGGL(qmk_bf16_kernel<64>, dim3(static_cast<unsigned>(nb)), dim3(256), 0, st, qm_split, k16,
                         gather, ks_mean, B, S, H, G, scale, bias, s_pitch, rb, k_codes, k_scale, k_pitch,
                         static_cast<int>(k_block));
    }
    LBFQ_LAUNCH_CHECK("lbfq_qmk");
    if (rb) {
      hipLaunchKernelGGL(decode_ordered_kernel, dim3(static_cast<unsigned>((nr + 255) / 256)), dim3(256), 0, st, rb, nr);
      LBFQ_LAUNCH_CHECK("lbfq_qmk decode");
    }
    return 0;
  }
  LBFQ_CHECK_ARG(!k_codes, "lbfq_qmk_kquant: the fused K quantiser needs bf16 K and a table under 4 GiB per head");
  if (rb) {
    hipLaunchKernelGGL(fill_ordered_kernel, dim3(static_cast<unsigned>((nr + 255) / 256)), dim3(256), 0, st, rb, nr);
    LBFQ_LAUNCH_CHECK("lbfq_qmk fill");
  }
  const int64_t nblk = B * H * ((S + kKeysPerBlock - 1) / kKeysPerBlock);
  LBFQ_CHECK_ARG(nblk < (int64_t{1} << 31), "lbfq_qmk: grid too large");
  if (D == 128)
    hipLaunchKernelGGL(qmk_kernel<128>, dim3(static_cast<unsigned>(nblk)), dim3(256), 0, st, qm, ks, ks_dtype, gather,
                       ks_mean, B, S, H, G, scale, bias, s_pitch, rb);
  else
    hipLaunchKernelGGL(qmk_kernel<64>, dim3(static_cast<unsigned>(nblk)), dim3(256), 0, st, qm, ks, ks_dtype, gather,
                       ks_mean, B, S, H, G, scale, bias, s_pitch, rb);
  LBFQ_LAUNCH_CHECK("lbfq_qmk");
  if (rb) {
    hipLaunchKernelGGL(decode_ordered_kernel, dim3(static_cast<unsigned>((nr + 255) / 256)), dim3(256), 0, st, rb, nr);
    LBFQ_LAUNCH_CHECK("lbfq_qmk decode");
  }
  return 0;
}

}  // namespace

extern "C" int lbfq_qmk(const float* qm, const void* ks, int ks_dtype, const int32_t* gather, const float* ks_mean,
                        int64_t B, int64_t S, int64_t H, int64_t D, int64_t G, float scale, float* bias,
                        int64_t s_pitch, float* rowmax, uint32_t* qm_split, lbfq_stream_t stream) {
  return qmk_launch(qm, ks, ks_dtype, gather, ks_mean, B, S, H, D, G, scale, bias, s_pitch, rowmax, qm_split,
                    nullptr, 0, nullptr, 0, stream);
}

extern "C" int lbfq_qmk_kquant(const float* qm, const void* ks, int ks_dtype, const int32_t* gather,
                               const float* ks_mean, int64_t B, int64_t S, int64_t H, int64_t D, int64_t G,
                               float scale, float* bias, int64_t s_pitch, float* rowmax, uint32_t* qm_split,
                               uint8_t* k_codes, int64_t k_pitch, float* k_scale, int64_t k_block,
                               lbfq_stream_t stream) {
  LBFQ_CHECK_ARG(k_codes && k_scale, "lbfq_qmk_kquant: null K code / scale pointer");
  LBFQ_CHECK_ARG(k_block == 16 || k_block == 32 || k_block == 64, "lbfq_qmk_kquant: K block must be 16, 32 or 64");
  LBFQ_CHECK_ARG(S > 0 && S % k_block == 0 && k_pitch >= S, "lbfq_qmk_kquant: S must be a multiple of the K block");
  LBFQ_CHECK_ARG(ks_dtype == kBF16 && (!bias || G * s_pitch * 4 < (int64_t{1} << 32)),
                 "lbfq_qmk_kquant: the fused K quantiser needs bf16 K and a table under 4 GiB per head");
  return qmk_launch(qm, ks, ks_dtype, gather, ks_mean, B, S, H, D, G, scale, bias, s_pitch, rowmax, qm_split,
                    k_codes, k_pitch, k_scale, k_block, stream);
}
