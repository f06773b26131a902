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

__global__ void fill_ordered_kernel(uint32_t* p, int64_t n) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = ordered_bits(-INFINITY);
}

__global__ void decode_ordered_kernel(uint32_t* p, int64_t n) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) reinterpret_cast<float*>(p)[i] = from_ordered_bits(p[i]);
}

}  // namespace

extern "C" int lbfq_qmk(const float* qm, const void* ks, int ks_dtype, const int32_t* gather, const float* ks_mean,
                        int64_t B, int64_t S, int64_t H, int64_t D, int64_t G, float scale, float* bias,
                        int64_t s_pitch, float* rowmax, lbfq_stream_t stream) {
  LBFQ_CHECK_ARG(qm && ks && (bias || rowmax), "lbfq_qmk: null pointer");
  LBFQ_CHECK_ARG(D == 64 || D == 128, "lbfq_qmk: D must be 64 or 128");
  LBFQ_CHECK_ARG(ks_dtype >= 0 && ks_dtype <= 2, "lbfq_qmk: bad dtype %d", ks_dtype);
  LBFQ_CHECK_ARG(B > 0 && H > 0 && G > 0 && S > 0 && (!bias || s_pitch >= S), "lbfq_qmk: bad sizes");
  hipStream_t st = static_cast<hipStream_t>(stream);
  uint32_t* rb = reinterpret_cast<uint32_t*>(rowmax);
  const int64_t nr = B * H * G;
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
