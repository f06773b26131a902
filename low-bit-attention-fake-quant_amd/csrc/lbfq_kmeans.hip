// Token k-means reorder for the Q / V reorder (gfx950).
//
// Replaces flash-kmeans batch_kmeans_Euclid (called at kmeans.py:78-81 of the
// reference) and the stable argsort / inverse scatter (kmeans.py:84-87).
// Deterministic Lloyd specification shared with the CPU oracle:
//   init   : centroid j = token j*stride + mix(seed, bh, j) % stride,
//            stride = S / K, mix = splitmix64 finaliser;
//   assign : cn_j = sum_d fmaf(c, c), dot_j = sum_d fmaf(x, c) sequential in d,
//            score_j = fmaf(-2, dot_j, cn_j), first minimum wins;
//   update : fp64 sums per 1024-token chunk in token order, chunks added in
//            order, c = (float)(sum / count), empty clusters keep c;
//   labels : those of the last assign of `iters` rounds.
// The order is a stable counting sort of the labels (argsort stable=True).
#include "lbfq_common.h"
#include "../../include/lbfq.h"

using namespace lbfq;

namespace {

constexpr int kChunk = 1024;
constexpr int kMaxD = 128;
constexpr int kMaxKAssign = 64;   // centroids held in LDS by the assign kernel
constexpr int kSortThreads = 1024;
constexpr int kMaxKSort = kMaxKAssign;

__device__ __forceinline__ uint64_t kmix(uint64_t seed, uint64_t bh, uint64_t K, uint64_t j) {
  uint64_t z = seed + 0x9E3779B97F4A7C15ull * (bh * K + j + 1ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__global__ void km_init_kernel(const void* x, int dt, int64_t S, int64_t H, int64_t D, int K, uint64_t seed,
                               float* cent) {
  const int64_t bh = blockIdx.x / K;
  const int j = blockIdx.x % K;
  const int64_t b = bh / H, h = bh % H;
  const int64_t stride = S / K;
  const int64_t idx = j * stride + static_cast<int64_t>(kmix(seed, bh, K, j) % static_cast<uint64_t>(stride));
  const int d = threadIdx.x;
  if (d < D) cent[(bh * K + j) * D + d] = load_as_f32(x, ((b * S + idx) * H + h) * D + d, dt);
}

// One thread per token; centroids of the slice in LDS.
template <int D>
__global__ void __launch_bounds__(256) km_assign_kernel(const void* x, int dt, int64_t S, int64_t H, int K,
                                                        const float* cent, int32_t* labels) {
  __shared__ float c_lds[kMaxKAssign * D];
  __shared__ float cn_lds[kMaxKAssign];
  const int64_t nblk_s = (S + 255) / 256;
  const int64_t bh = blockIdx.x / nblk_s;
  const int64_t t = (blockIdx.x % nblk_s) * 256 + threadIdx.x;
  const int64_t b = bh / H, h = bh % H;
  for (int i = threadIdx.x; i < K * D; i += 256) c_lds[i] = cent[bh * K * D + i];
  __syncthreads();
  if (threadIdx.x < K) {
    float acc = 0.0f;
    for (int d = 0; d < D; ++d) acc = fmaf(c_lds[threadIdx.x * D + d], c_lds[threadIdx.x * D + d], acc);
    cn_lds[threadIdx.x] = acc;
  }
  __syncthreads();
  if (t >= S) return;
  float xv[D];
  const int64_t base = ((b * S + t) * H + h) * D;
#pragma unroll
  for (int d = 0; d < D; ++d) xv[d] = load_as_f32(x, base + d, dt);
  float best = INFINITY;
  int bj = 0;
  for (int j = 0; j < K; ++j) {
    const float* c = c_lds + j * D;
    float dot = 0.0f;
#pragma unroll
    for (int d = 0; d < D; ++d) dot = fmaf(xv[d], c[d], dot);
    float sc = fmaf(-2.0f, dot, cn_lds[j]);
    if (sc < best) { best = sc; bj = j; }
  }
  labels[bh * S + t] = bj;
}

// fp64 per-cluster sums of one 1024-token chunk; one thread per column, 64
// columns per workgroup.
__global__ void km_update_partial_kernel(const void* x, int dt, int64_t S, int64_t H, int64_t D, int K,
                                         const int32_t* labels, double* partial, int32_t* counts) {
  __shared__ double sums[kMaxKAssign * 64];
  __shared__ int cnt[kMaxKAssign];
  const int64_t nchunk = (S + kChunk - 1) / kChunk;
  const int ncg = static_cast<int>(D / 64);
  int64_t bid = blockIdx.x;
  const int cg = static_cast<int>(bid % ncg); bid /= ncg;
  const int64_t bh = bid / nchunk, c = bid % nchunk;
  const int64_t b = bh / H, h = bh % H;
  const int dl = threadIdx.x;
  const int d = cg * 64 + dl;
  for (int i = dl; i < K * 64; i += 64) sums[i] = 0.0;
  for (int i = dl; i < K; i += 64) cnt[i] = 0;
  __syncthreads();
  const int64_t t0 = c * kChunk, t1 = t0 + kChunk < S ? t0 + kChunk : S;
  for (int64_t t = t0; t < t1; ++t) {
    int lab = labels[bh * S + t];
    sums[lab * 64 + dl] += static_cast<double>(load_as_f32(x, ((b * S + t) * H + h) * D + d, dt));
    if (dl == 0) cnt[lab] += 1;
  }
  __syncthreads();
  for (int j = 0; j < K; ++j) partial[((bh * nchunk + c) * K + j) * D + d] = sums[j * 64 + dl];
  if (cg == 0)
    for (int i = dl; i < K; i += 64) counts[(bh * nchunk + c) * K + i] = cnt[i];
}

__global__ void km_finalize_kernel(const double* partial, const int32_t* counts, int64_t nchunk, int K, int64_t D,
                                   float* cent) {
  const int64_t bh = blockIdx.x / K;
  const int j = blockIdx.x % K;
  const int d = threadIdx.x;
  if (d >= D) return;
  double tot = 0.0;
  int64_t cnt = 0;
  for (int64_t c = 0; c < nchunk; ++c) {
    tot += partial[((bh * nchunk + c) * K + j) * D + d];
    cnt += counts[(bh * nchunk + c) * K + j];
  }
  if (cnt > 0) cent[(bh * K + j) * D + d] = static_cast<float>(tot / static_cast<double>(cnt));
}

// Stable counting sort of one slice's labels: order[pos] = t, inverse[t] = pos.
__global__ void __launch_bounds__(kSortThreads) km_sort_kernel(const int32_t* labels, int64_t S, int K,
                                                               int32_t* order, int32_t* inverse) {
  __shared__ int start[kMaxKSort];
  __shared__ int running[kMaxKSort];
  __shared__ int wcnt[kSortThreads / 64][kMaxKSort];
  const int64_t bh = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  constexpr int NW = kSortThreads / 64;
  for (int i = tid; i < K; i += kSortThreads) { start[i] = 0; running[i] = 0; }
  for (int i = tid; i < NW * K; i += kSortThreads) wcnt[i / K][i % K] = 0;
  __syncthreads();
  const int32_t* lab = labels + bh * S;
  for (int64_t t = tid; t < S; t += kSortThreads) atomicAdd(&start[lab[t]], 1);
  __syncthreads();
  if (tid == 0) {
    int acc = 0;
    for (int j = 0; j < K; ++j) { int c = start[j]; start[j] = acc; acc += c; }
  }
  __syncthreads();
  int nbits = 1;
  while ((1 << nbits) < K) ++nbits;
  const uint64_t lt_mask = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  for (int64_t r0 = 0; r0 < S; r0 += kSortThreads) {
    const int64_t t = r0 + tid;
    const bool valid = t < S;
    const int L = valid ? lab[t] : -1;
    uint64_t match = __ballot(valid);
    for (int bit = 0; bit < nbits; ++bit) {
      uint64_t bal = __ballot(valid && ((L >> bit) & 1));
      match &= (valid && ((L >> bit) & 1)) ? bal : ~bal;
    }
    const int rank = __popcll(match & lt_mask);
    const bool leader = valid && ((match >> lane) == 1ull);
    if (leader) wcnt[wave][L] = __popcll(match);
    __syncthreads();
    if (valid) {
      int pos = start[L] + running[L] + rank;
      for (int w = 0; w < wave; ++w) pos += wcnt[w][L];
      order[bh * S + pos] = static_cast<int32_t>(t);
      inverse[bh * S + t] = pos;
    }
    __syncthreads();
    for (int j = tid; j < K; j += kSortThreads) {
      int s = 0;
      for (int w = 0; w < NW; ++w) { s += wcnt[w][j]; wcnt[w][j] = 0; }
      running[j] += s;
    }
    __syncthreads();
  }
}

struct KmWs {
  float* cent;
  double* partial;
  int32_t* counts;
};

KmWs carve(void* ws, int64_t BH, int64_t S, int64_t D, int K) {
  const int64_t nchunk = (S + kChunk - 1) / kChunk;
  uint8_t* p = static_cast<uint8_t*>(ws);
  KmWs w;
  w.partial = reinterpret_cast<double*>(p);
  p += sizeof(double) * BH * nchunk * K * D;
  w.cent = reinterpret_cast<float*>(p);
  p += sizeof(float) * BH * K * D;
  w.counts = reinterpret_cast<int32_t*>(p);
  return w;
}

}  // namespace

extern "C" int64_t lbfq_kmeans_workspace_bytes(int64_t B, int64_t S, int64_t H, int64_t D, int K) {
  const int64_t nchunk = (S + kChunk - 1) / kChunk;
  const int64_t BH = B * H;
  return sizeof(double) * BH * nchunk * K * D + sizeof(float) * BH * K * D + sizeof(int32_t) * BH * nchunk * K;
}

extern "C" int lbfq_kmeans(const void* x, int dtype, int64_t B, int64_t S, int64_t H, int64_t D, int K, int iters,
                           uint64_t seed, void* workspace, int32_t* labels, int32_t* order, int32_t* inverse,
                           lbfq_stream_t stream) {
  LBFQ_CHECK_ARG(x && workspace && labels && order && inverse, "lbfq_kmeans: null pointer");
  LBFQ_CHECK_ARG(D == 64 || D == 128, "lbfq_kmeans: D must be 64 or 128; got %lld", (long long)D);
  LBFQ_CHECK_ARG(K >= 1 && K <= S, "n_clusters must be in [1, S]; got %d for S=%lld", K, (long long)S);
  LBFQ_CHECK_ARG(K <= kMaxKAssign, "lbfq_kmeans: at most %d clusters are supported; got %d", kMaxKAssign, K);
  LBFQ_CHECK_ARG(B * H < (1ll << 31) / 1024, "lbfq_kmeans: too many slices");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t BH = B * H;
  const int64_t nchunk = (S + kChunk - 1) / kChunk;
  KmWs w = carve(workspace, BH, S, D, K);
  hipLaunchKernelGGL(km_init_kernel, dim3(static_cast<unsigned>(BH * K)), dim3(static_cast<unsigned>(D)), 0, st, x,
                     dtype, S, H, D, K, seed, w.cent);
  LBFQ_LAUNCH_CHECK("km_init");
  const int64_t nblk_s = (S + 255) / 256;
  const int rounds = iters > 0 ? iters : 1;
  for (int it = 0; it < rounds; ++it) {
    if (D == 128)
      hipLaunchKernelGGL(km_assign_kernel<128>, dim3(static_cast<unsigned>(BH * nblk_s)), dim3(256), 0, st, x, dtype,
                         S, H, K, w.cent, labels);
    else
      hipLaunchKernelGGL(km_assign_kernel<64>, dim3(static_cast<unsigned>(BH * nblk_s)), dim3(256), 0, st, x, dtype,
                         S, H, K, w.cent, labels);
    LBFQ_LAUNCH_CHECK("km_assign");
    if (it + 1 == rounds) break;  // the last update does not change the labels
    hipLaunchKernelGGL(km_update_partial_kernel, dim3(static_cast<unsigned>(BH * nchunk * (D / 64))), dim3(64), 0,
                       st, x, dtype, S, H, D, K, labels, w.partial, w.counts);
    LBFQ_LAUNCH_CHECK("km_update_partial");
    hipLaunchKernelGGL(km_finalize_kernel, dim3(static_cast<unsigned>(BH * K)), dim3(static_cast<unsigned>(D)), 0, st,
                       w.partial, w.counts, nchunk, K, D, w.cent);
    LBFQ_LAUNCH_CHECK("km_finalize");
  }
  hipLaunchKernelGGL(km_sort_kernel, dim3(static_cast<unsigned>(BH)), dim3(kSortThreads), 0, st, labels, S, K, order,
                     inverse);
  LBFQ_LAUNCH_CHECK("km_sort");
  return 0;
}
