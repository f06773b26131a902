// qm . K_smooth products for Q smoothing (gfx950).
//
//   bias[b,h,g,n] = (qm[b,g,h,:] . K_s[b,n,h,:]) * scale         (fp32)
//   rowmax[b,h,g] = max_n bias[b,h,g,n]
// The attention path uses scale = sm_scale * log2(e) (scores in log2 units).
//
// bias is the per-key correction the reference adds to every score inside the
// attention K-loop (attention_triton.py:156-160); rowmax is the qm_k row-max
// estimate (attention.py:366-395), shared by the q_group rows of a group.
// K_s may be read through a gather (K co-permuted by the V k-means order).
#include "lbfq_common.h"
#include "../../include/lbfq.h"

using namespace lbfq;

namespace {

constexpr int kKeys = 64;      // keys per workgroup
constexpr int kGChunk = 64;    // groups staged in LDS at a time

__device__ __forceinline__ uint32_t ordered_bits(float f) {
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float from_ordered_bits(uint32_t u) {
  return __uint_as_float((u & 0x80000000u) ? (u & 0x7fffffffu) : ~u);
}

template <int D>
__global__ void __launch_bounds__(256) qmk_kernel(const float* qm, const void* ks, int dt, const int32_t* gather,
                                                  int64_t B, int64_t S, int64_t H, int64_t G, float scale,
                                                  float* bias, int64_t s_pitch, uint32_t* rowmax_bits) {
  __shared__ float q_lds[kGChunk * D];
  __shared__ float k_lds[kKeys * (D + 1)];
  const int64_t nkb = (S + kKeys - 1) / kKeys;
  const int64_t bh = blockIdx.x / nkb;
  const int64_t n0 = (blockIdx.x % nkb) * kKeys;
  const int64_t b = bh / H, h = bh % H;
  const int tid = threadIdx.x;
  // stage the 64 keys (fp32) of this block
  for (int e = tid; e < kKeys * D; e += 256) {
    int j = e / D, d = e % D;
    int64_t n = n0 + j;
    float v = 0.0f;
    if (n < S) {
      int64_t src = gather ? gather[bh * S + n] : n;
      v = load_as_f32(ks, ((b * S + src) * H + h) * D + d, dt);
    }
    k_lds[j * (D + 1) + d] = v;
  }
  const int j = tid & 63;        // key of this thread
  const int gsub = tid >> 6;     // 4 group lanes
  const int64_t n = n0 + j;
  for (int64_t g0 = 0; g0 < G; g0 += kGChunk) {
    __syncthreads();
    const int64_t gc = G - g0 < kGChunk ? G - g0 : kGChunk;
    for (int e = tid; e < gc * D; e += 256) {
      int gg = e / D, d = e % D;
      q_lds[gg * D + d] = qm[((b * G + g0 + gg) * H + h) * D + d];
    }
    __syncthreads();
    for (int gg = gsub; gg < gc; gg += 4) {
      float acc = 0.0f;
#pragma unroll 16
      for (int d = 0; d < D; ++d) acc = fmaf(q_lds[gg * D + d], k_lds[j * (D + 1) + d], acc);
      float v = acc * scale;
      if (n < S) {
        if (bias) bias[(bh * G + g0 + gg) * s_pitch + n] = v;
      }
      // block max over the 64 keys of this group
      float m = n < S ? v : -INFINITY;
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
      if (rowmax_bits && j == 0) atomicMax(rowmax_bits + bh * G + g0 + gg, ordered_bits(m));
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

extern "C" int lbfq_qmk(const float* qm, const void* ks, int ks_dtype, const int32_t* gather, int64_t B, int64_t S,
                        int64_t H, int64_t D, int64_t G, float scale, float* bias, int64_t s_pitch, float* rowmax,
                        lbfq_stream_t stream) {
  LBFQ_CHECK_ARG(qm && ks && (bias || rowmax), "lbfq_qmk: null pointer");
  LBFQ_CHECK_ARG(D == 64 || D == 128, "lbfq_qmk: D must be 64 or 128");
  LBFQ_CHECK_ARG(G > 0 && S > 0 && (!bias || s_pitch >= S), "lbfq_qmk: bad sizes");
  hipStream_t st = static_cast<hipStream_t>(stream);
  uint32_t* rb = reinterpret_cast<uint32_t*>(rowmax);
  const int64_t nr = B * H * G;
  if (rb) {
    hipLaunchKernelGGL(fill_ordered_kernel, dim3(static_cast<unsigned>((nr + 255) / 256)), dim3(256), 0, st, rb, nr);
    LBFQ_LAUNCH_CHECK("lbfq_qmk fill");
  }
  const int64_t nblk = B * H * ((S + kKeys - 1) / kKeys);
  if (D == 128)
    hipLaunchKernelGGL(qmk_kernel<128>, dim3(static_cast<unsigned>(nblk)), dim3(256), 0, st, qm, ks, ks_dtype, gather,
                       B, S, H, G, scale, bias, s_pitch, rb);
  else
    hipLaunchKernelGGL(qmk_kernel<64>, dim3(static_cast<unsigned>(nblk)), dim3(256), 0, st, qm, ks, ks_dtype, gather,
                       B, S, H, G, scale, bias, s_pitch, rb);
  LBFQ_LAUNCH_CHECK("lbfq_qmk");
  if (rb) {
    hipLaunchKernelGGL(decode_ordered_kernel, dim3(static_cast<unsigned>((nr + 255) / 256)), dim3(256), 0, st, rb, nr);
    LBFQ_LAUNCH_CHECK("lbfq_qmk decode");
  }
  return 0;
}
