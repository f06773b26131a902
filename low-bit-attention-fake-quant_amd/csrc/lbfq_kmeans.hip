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
// A slice whose assignment leaves every label as it was has converged: its
// later rounds would recompute the same centroids and labels exactly, so its
// workgroups skip them (a per-slice flag on the device, no host round trip).
// The order is a stable counting sort of the labels (argsort stable=True).
#include <mutex>
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

// n consecutive elements of dtype DT as fp32 (n a multiple of 8, 16-byte aligned)
template <int DT, int N>
__device__ __forceinline__ void load_row(const void* x, int64_t idx, float (&v)[N]) {
  if constexpr (DT == kF32) {
    const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(x) + idx);
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
      const float4 f = p[i];
      v[4 * i] = f.x; v[4 * i + 1] = f.y; v[4 * i + 2] = f.z; v[4 * i + 3] = f.w;
    }
  } else {
    const uint4* p = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(x) + idx);
#pragma unroll
    for (int i = 0; i < N / 8; ++i) {
      const uint4 r = p[i];
      const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint16_t lo = static_cast<uint16_t>(w[k] & 0xffffu), hi = static_cast<uint16_t>(w[k] >> 16);
        if constexpr (DT == kBF16) { v[8 * i + 2 * k] = bf16_bits_to_f32(lo); v[8 * i + 2 * k + 1] = bf16_bits_to_f32(hi); }
        else { v[8 * i + 2 * k] = f16_bits_to_f32(lo); v[8 * i + 2 * k + 1] = f16_bits_to_f32(hi); }
      }
    }
  }
}

// One thread per token: its row in registers (16-byte loads), the slice's
// centroids in LDS read as float4 broadcasts; each distance is the sequential
// fmaf chain over d of the specification.
// prev_changed: the flags of the previous round (NULL in the first round);
// changed: this round's flags, set to 1 for a slice in which some label
// changed.  They are zero on entry from the second round on; in the first
// round every label counts as changed, so every slice's flag is written.
template <int D, int DT>
__global__ void __launch_bounds__(256) km_assign_kernel(const void* x, int64_t S, int64_t H, int K, const float* cent,
                                                        int32_t* labels, const int32_t* prev_changed,
                                                        int32_t* changed) {
  __shared__ float4 c_lds[kMaxKAssign * D / 4];
  __shared__ float cn_lds[kMaxKAssign];
  const int64_t nblk_s = (S + 255) / 256;
  const int64_t bh = blockIdx.x / nblk_s;
  if (prev_changed && prev_changed[bh] == 0) return;  // converged slice (uniform per workgroup)
  const int64_t t = (blockIdx.x % nblk_s) * 256 + threadIdx.x;
  const int64_t b = bh / H, h = bh % H;
  const float4* cg = reinterpret_cast<const float4*>(cent + bh * K * D);
  for (int i = threadIdx.x; i < K * D / 4; i += 256) c_lds[i] = cg[i];
  __syncthreads();
  if (threadIdx.x < K) {
    const float* c = reinterpret_cast<const float*>(c_lds) + threadIdx.x * D;
    float acc = 0.0f;
    for (int d = 0; d < D; ++d) acc = fmaf(c[d], c[d], acc);
    cn_lds[threadIdx.x] = acc;
  }
  __syncthreads();
  if (t >= S) return;
  float xv[D];
  load_row<DT>(x, ((b * S + t) * H + h) * D, xv);
  float best = INFINITY;
  int bj = 0;
  // two centroids at a time: independent dot-product chains (each still
  // sequential in d), compared in centroid order, so the first minimum wins
  constexpr int KJ = 2;
  int j = 0;
  for (; j + KJ <= K; j += KJ) {
    float dot[KJ];
#pragma unroll
    for (int u = 0; u < KJ; ++u) dot[u] = 0.0f;
#pragma unroll
    for (int d4 = 0; d4 < D / 4; ++d4) {
#pragma unroll
      for (int u = 0; u < KJ; ++u) {
        const float4 cv = c_lds[(j + u) * (D / 4) + d4];
        dot[u] = fmaf(xv[4 * d4], cv.x, dot[u]);
        dot[u] = fmaf(xv[4 * d4 + 1], cv.y, dot[u]);
        dot[u] = fmaf(xv[4 * d4 + 2], cv.z, dot[u]);
        dot[u] = fmaf(xv[4 * d4 + 3], cv.w, dot[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < KJ; ++u) {
      const float sc = fmaf(-2.0f, dot[u], cn_lds[j + u]);
      if (sc < best) { best = sc; bj = j + u; }
    }
  }
  for (; j < K; ++j) {
    const float4* c = c_lds + j * (D / 4);
    float dot = 0.0f;
#pragma unroll
    for (int d4 = 0; d4 < D / 4; ++d4) {
      const float4 cv = c[d4];
      dot = fmaf(xv[4 * d4], cv.x, dot);
      dot = fmaf(xv[4 * d4 + 1], cv.y, dot);
      dot = fmaf(xv[4 * d4 + 2], cv.z, dot);
      dot = fmaf(xv[4 * d4 + 3], cv.w, dot);
    }
    const float sc = fmaf(-2.0f, dot, cn_lds[j]);
    if (sc < best) { best = sc; bj = j; }
  }
  const int32_t old = prev_changed ? labels[bh * S + t] : -1;
  labels[bh * S + t] = bj;
  if (__any(old != bj) && (threadIdx.x & 63) == 0) changed[bh] = 1;
}

// fp64 per-cluster column sums of one kChunk-token chunk.  The chunk's tokens
// are first sorted by label in LDS, stably (ballot ranks within a wave, waves
// and rounds in token order), so a cluster's tokens keep their order.  Then
// thread (g, d) -- column d, cluster group g -- adds the runs of clusters
// j = g, g + NG, ... in that order: the token-order fp64 sums of the
// specification, over chains NG times shorter, with 8 loads in flight.
constexpr int kUpdThreads = 512;

template <int D, int DT>
__global__ void __launch_bounds__(kUpdThreads) km_update_partial_kernel(const void* x, int64_t S, int64_t H, int K,
                                                                        const int32_t* labels, double* partial,
                                                                        int32_t* counts, const int32_t* changed) {
  constexpr int NG = kUpdThreads / D;  // cluster groups
  constexpr int NW = kUpdThreads / 64;
  __shared__ int lab_s[kChunk];
  __shared__ int ord_s[kChunk];
  __shared__ int start_s[kMaxKAssign + 1];
  __shared__ int running[kMaxKAssign];
  __shared__ int wcnt[NW][kMaxKAssign];
  const int64_t nchunk = (S + kChunk - 1) / kChunk;
  const int64_t bh = blockIdx.x / nchunk, c = blockIdx.x % nchunk;
  if (changed[bh] == 0) return;  // converged slice (uniform per workgroup)
  const int64_t b = bh / H, h = bh % H;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t t0 = c * kChunk;
  const int n = static_cast<int>(t0 + kChunk < S ? kChunk : S - t0);
  for (int i = tid; i < K; i += kUpdThreads) { start_s[i + 1] = 0; running[i] = 0; }
  for (int i = tid; i < NW * K; i += kUpdThreads) wcnt[i / K][i % K] = 0;
  for (int i = tid; i < n; i += kUpdThreads) lab_s[i] = labels[bh * S + t0 + i];
  __syncthreads();
  for (int i = tid; i < n; i += kUpdThreads) atomicAdd(&start_s[lab_s[i] + 1], 1);
  __syncthreads();
  if (tid == 0) {
    start_s[0] = 0;
    for (int j = 0; j < K; ++j) start_s[j + 1] += start_s[j];
  }
  __syncthreads();
  int nbits = 1;
  while ((1 << nbits) < K) ++nbits;
  const uint64_t lt_mask = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  for (int r0 = 0; r0 < n; r0 += kUpdThreads) {
    const int r = r0 + tid;
    const bool valid = r < n;
    const int L = valid ? lab_s[r] : -1;
    uint64_t match = __ballot(valid);
    for (int bit = 0; bit < nbits; ++bit) {
      const uint64_t bal = __ballot(valid && ((L >> bit) & 1));
      match &= (valid && ((L >> bit) & 1)) ? bal : ~bal;
    }
    const int rank = __popcll(match & lt_mask);
    if (valid && (match >> lane) == 1ull) wcnt[wave][L] = __popcll(match);  // the highest lane of its label
    __syncthreads();
    if (valid) {
      int pos = start_s[L] + running[L] + rank;
      for (int w = 0; w < wave; ++w) pos += wcnt[w][L];
      ord_s[pos] = r;
    }
    __syncthreads();
    for (int j = tid; j < K; j += kUpdThreads) {
      int sum = 0;
      for (int w = 0; w < NW; ++w) { sum += wcnt[w][j]; wcnt[w][j] = 0; }
      running[j] += sum;
    }
    __syncthreads();
  }
  if (tid < K) counts[(bh * nchunk + c) * K + tid] = start_s[tid + 1] - start_s[tid];
  // column sums over the sorted runs of this thread's clusters
  const int g = tid / D, dcol = tid % D;
  double* out = partial + (bh * nchunk + c) * K * D + dcol;
  const int64_t xrow0 = (b * S + t0) * H + h;
  for (int j = g; j < K; j += NG) {
    const int p1 = start_s[j + 1];
    double acc = 0.0;
    constexpr int kPf = 8;
    for (int p0 = start_s[j]; p0 < p1; p0 += kPf) {
      float v[kPf];
#pragma unroll
      for (int i = 0; i < kPf; ++i) {
        const int pos = p0 + i < p1 ? p0 + i : p1 - 1;
        v[i] = load_as_f32(x, (xrow0 + static_cast<int64_t>(ord_s[pos]) * H) * D + dcol, DT);
      }
#pragma unroll
      for (int i = 0; i < kPf; ++i)
        if (p0 + i < p1) acc += static_cast<double>(v[i]);
    }
    out[j * D] = acc;
  }
}

// changed: this round's flags; clear_next: the next round's, cleared here
// (the previous round's assignment, their last reader, has finished).
__global__ void km_finalize_kernel(const double* partial, const int32_t* counts, int64_t nchunk, int K, int64_t D,
                                   float* cent, const int32_t* changed, int32_t* clear_next) {
  const int64_t bh = blockIdx.x / K;
  const int j = blockIdx.x % K;
  const int d = threadIdx.x;
  if (j == 0 && d == 0) clear_next[bh] = 0;
  if (d >= D || changed[bh] == 0) return;
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
  int32_t* changed;  // [2][BH]: the convergence flags of two consecutive rounds
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
  p += sizeof(int32_t) * BH * nchunk * K;
  w.changed = reinterpret_cast<int32_t*>(p);
  return w;
}

}  // namespace

extern "C" int64_t lbfq_kmeans_workspace_bytes(int64_t B, int64_t S, int64_t H, int64_t D, int K) {
  const int64_t nchunk = (S + kChunk - 1) / kChunk;
  const int64_t BH = B * H;
  return sizeof(double) * BH * nchunk * K * D + sizeof(float) * BH * K * D + sizeof(int32_t) * BH * nchunk * K +
         sizeof(int32_t) * 2 * BH;
}

extern "C" int lbfq_kmeans(const void* x, int dtype, int64_t B, int64_t S, int64_t H, int64_t D, int K, int iters,
                           uint64_t seed, void* workspace, int32_t* labels, int32_t* order, int32_t* inverse,
                           lbfq_stream_t stream) {
  LBFQ_CHECK_ARG(x && workspace && labels && order && inverse, "lbfq_kmeans: null pointer");
  LBFQ_CHECK_ARG(D == 64 || D == 128, "lbfq_kmeans: D must be 64 or 128; got %lld", (long long)D);
  LBFQ_CHECK_ARG(dtype >= 0 && dtype <= 2, "lbfq_kmeans: bad dtype %d", dtype);
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
    const dim3 ga(static_cast<unsigned>(BH * nblk_s)), gu(static_cast<unsigned>(BH * nchunk));
    // round it writes flag slot it % 2, read by its update and finalize and by
    // round it + 1's assignment; finalize clears slot (it + 1) % 2 first
    int32_t* cur = w.changed + (it & 1) * BH;
    const int32_t* prev = it == 0 ? nullptr : w.changed + ((it - 1) & 1) * BH;
#define LBFQ_KM(DD, DT)                                                                                     \
  hipLaunchKernelGGL((km_assign_kernel<DD, DT>), ga, dim3(256), 0, st, x, S, H, K, w.cent, labels, prev, cur); \
  if (it + 1 < rounds)                                                                                      \
    hipLaunchKernelGGL((km_update_partial_kernel<DD, DT>), gu, dim3(kUpdThreads), 0, st, x, S, H, K, labels,  \
                       w.partial, w.counts, cur);
    if (D == 128) {
      if (dtype == kBF16) { LBFQ_KM(128, kBF16) } else if (dtype == kF16) { LBFQ_KM(128, kF16) } else { LBFQ_KM(128, kF32) }
    } else {
      if (dtype == kBF16) { LBFQ_KM(64, kBF16) } else if (dtype == kF16) { LBFQ_KM(64, kF16) } else { LBFQ_KM(64, kF32) }
    }
#undef LBFQ_KM
    LBFQ_LAUNCH_CHECK("km_assign / km_update_partial");
    if (it + 1 == rounds) break;  // the last update does not change the labels
    hipLaunchKernelGGL(km_finalize_kernel, dim3(static_cast<unsigned>(BH * K)), dim3(static_cast<unsigned>(D)), 0, st,
                       w.partial, w.counts, nchunk, K, D, w.cent, cur, w.changed + ((it + 1) & 1) * BH);
    LBFQ_LAUNCH_CHECK("km_finalize");
  }
  hipLaunchKernelGGL(km_sort_kernel, dim3(static_cast<unsigned>(BH)), dim3(kSortThreads), 0, st, labels, S, K, order,
                     inverse);
  LBFQ_LAUNCH_CHECK("km_sort");
  return 0;
}

// ---- allocation-free variant -------------------------------------------------
// For callers that cannot allocate device memory (code under HIP graph capture,
// serving loops, harnesses that forbid hipMalloc): the workspace is a
// file-scope device array, one copy per GPU, held until the process ends.
// Its device address is looked up once per device (hipGetSymbolAddress, with
// that device current) and kept; host code never uses the array's name as an
// address.  Calls that overlap on one GPU share the array and race.  The
// kernels write every workspace word they read, so nothing is cleared.
constexpr int64_t kKmScratchBytes = int64_t{64} << 20;  // 64 MiB: the 14B Q k-means (40 x 32768, K=32) needs 43 MB
static __device__ __align__(256) uint8_t scratch[kKmScratchBytes];
namespace {
constexpr int kMaxDevices = 64;
void* g_km_scratch[kMaxDevices] = {};
std::mutex g_km_scratch_mu;

int km_scratch_ptr(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  LBFQ_CHECK_ARG(e == hipSuccess, "lbfq_kmeans_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
  LBFQ_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "lbfq_kmeans_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_km_scratch_mu);
  if (!g_km_scratch[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      lbfq_set_error("lbfq_kmeans_noalloc: hipGetSymbolAddress failed: %s", hipGetErrorString(e));
      return -2;
    }
    g_km_scratch[dev] = p;
  }
  *out = g_km_scratch[dev];
  return 0;
}
}  // namespace

extern "C" int64_t lbfq_kmeans_noalloc_max_workspace_bytes(void) { return kKmScratchBytes; }

extern "C" int lbfq_kmeans_noalloc(const void* x, int dtype, int64_t B, int64_t S, int64_t H, int64_t D, int K,
                                   int iters, uint64_t seed, int32_t* labels, int32_t* order, int32_t* inverse,
                                   lbfq_stream_t stream) {
  LBFQ_CHECK_ARG(B > 0 && S > 0 && H > 0 && D > 0 && K > 0, "lbfq_kmeans_noalloc: empty shape");
  const int64_t need = lbfq_kmeans_workspace_bytes(B, S, H, D, K);
  LBFQ_CHECK_ARG(need <= kKmScratchBytes,
                 "lbfq_kmeans_noalloc: the problem needs %lld bytes of workspace, above the %lld-byte built-in "
                 "scratch; use lbfq_kmeans with a caller workspace",
                 (long long)need, (long long)kKmScratchBytes);
  void* ws = nullptr;
  const int rc = km_scratch_ptr(&ws);
  if (rc) return rc;
  return lbfq_kmeans(x, dtype, B, S, H, D, K, iters, seed, ws, labels, order, inverse, stream);
}
