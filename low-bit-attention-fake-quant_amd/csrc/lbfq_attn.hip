// C ABI of the FP8-MFMA P-requant attention (gfx950) and self tests of the
// builtins it relies on.  The guards mirror what fake_quant_attention_triton
// (attention_triton.py:463-624) lets reach its kernel; the kernel body is in
// lbfq_attn_kernel.h and is instantiated per P mode in lbfq_attn_p{0,1,2}.hip.
#include <cmath>

#include "lbfq_attn_kernel.h"

using namespace lbfq;
using namespace lbfq_attn;

namespace {

bool is_pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }

int ilog2(int64_t x) {
  int r = 0;
  while ((int64_t{1} << r) < x) ++r;
  return r;
}

__global__ void selftest_cvt_kernel(const float* x, int64_t n, uint8_t* out) {
  int64_t i = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
  if (i >= n) return;
  float x0 = x[i], x1 = i + 1 < n ? x[i + 1] : 0.f, x2 = i + 2 < n ? x[i + 2] : 0.f, x3 = i + 3 < n ? x[i + 3] : 0.f;
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(x0, x1, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(x2, x3, w, true);
  for (int k = 0; k < 4 && i + k < n; ++k) out[i + k] = static_cast<uint8_t>((w >> (8 * k)) & 0xff);
}

// One 32x32x64 MFMA: lane (i, g) supplies row/column i and K-elements
// 16g + [0,16), 32 + 16g + [0,16); the scale of K-block b comes from lane i + 32b.
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
  const int sa = as ? as[li * 2 + g] : 127, sb = as ? bs[li * 2 + g] : 127;
  if (as) c = mfma32<true>(av, bv, c, sa, sb);
  else c = mfma32<false>(av, bv, c, 0, 0);
  for (int r = 0; r < 16; ++r) C[(8 * (r >> 2) + 4 * g + (r & 3)) * 32 + li] = c[r];
  // the scale registers stay live past the MFMA (after the stores that need its
  // result), so they cannot be given to its destination
  use(sa);
  use(sb);
}

// Argument checks shared by the attention and its score probe; fills the
// kernel arguments.  Returns 0 or -1 (error message set).
int make_kargs(const lbfq_attn_params* p, KArgs& a, const char* who) {
  LBFQ_CHECK_ARG(p, "%s: null params", who);
  LBFQ_CHECK_ARG(p->D == 64 || p->D == 128, "%s: D must be 64 or 128; got %lld", who, (long long)p->D);
  LBFQ_CHECK_ARG(p->B > 0 && p->H > 0 && p->S > 0, "%s: empty shape", who);
  LBFQ_CHECK_ARG(p->s_pitch >= p->S && p->s_pitch % kQB == 0, "%s: s_pitch must be >= S and a multiple of %d", who,
                 kQB);
  LBFQ_CHECK_ARG(p->s_pitch < (int64_t{1} << 30) && p->B * p->H * (p->s_pitch / kQB) < (int64_t{1} << 31),
                 "%s: problem too large", who);
  LBFQ_CHECK_ARG(p->q_codes && p->k_codes && p->q_scale && p->k_scale, "%s: missing tensor", who);
  LBFQ_CHECK_ARG(p->qk_mx || (p->qk_block >= 16 && is_pow2(p->qk_block)),
                 "%s: fp8_block size must be a power of two >= 16; got %d", who, p->qk_block);
  LBFQ_CHECK_ARG(!p->rowmax_est || p->qk_bias, "%s: rowmax_est needs the qm correction table", who);
  LBFQ_CHECK_ARG(!(p->rowmax_est && p->rowmax_init), "%s: rowmax_init and rowmax_est are mutually exclusive", who);
  LBFQ_CHECK_ARG(p->block_n == 0 || p->block_n == 64 || p->block_n == 128, "%s: block_n must be 64 or 128; got %d",
                 who, p->block_n);
  LBFQ_CHECK_ARG(!p->qk_bias || (p->q_group >= 32 && is_pow2(p->q_group) && p->S % p->q_group == 0),
                 "%s: q_group must be a power of two >= 32 dividing S", who);
  const bool blasst = p->blasst_lambda > 0.0f;
  a = KArgs{};
  a.B = static_cast<int>(p->B);
  a.H = static_cast<int>(p->H);
  a.S = static_cast<int>(p->S);
  a.P = static_cast<int>(p->s_pitch);
  a.nqb = static_cast<int>((p->S + kQB - 1) / kQB);
  a.G = p->qk_bias ? static_cast<int>(p->S / p->q_group) : 1;
  a.lg_qgroup = p->qk_bias ? ilog2(p->q_group) : 0;
  a.lg_qkblk = p->qk_mx ? 0 : ilog2(p->qk_block);
  a.nqkblk = p->qk_mx ? 1 : static_cast<int>((p->S + p->qk_block - 1) / p->qk_block);
  a.v_kind = p->v_kind;
  a.lg_vblk = p->v_kind ? ilog2(p->v_block) : 0;
  a.nvblk = p->v_kind ? static_cast<int>(p->S / p->v_block) : 1;
  a.lg_vsb = p->v_alpha ? ilog2(p->v_smooth_block) : 0;
  a.nvsb = p->v_alpha ? static_cast<int>(p->S / p->v_smooth_block) : 1;
  a.p_max_offset = p->p_max_offset;
  a.block_m = p->block_m > 0 ? p->block_m : 64;
  a.rowmax_dynamic = p->rowmax_dynamic;
  a.sml2 = p->sm_scale * kLog2e;
  a.lam = blasst ? p->blasst_lambda : 0.0f;
  a.log2_lam = blasst ? static_cast<float>(std::log2(static_cast<double>(p->blasst_lambda))) : 0.0f;
  a.fill_alpha = p->blasst_fill_alpha;
  a.fill_kind = p->blasst_fill;
  a.uta_bins = p->blasst_uta_bins > 0 ? p->blasst_uta_bins : 1;
  a.q_codes = p->q_codes;
  a.k_codes = p->k_codes;
  a.v_codes_t = p->v_codes_t;
  a.q_scale = p->q_scale;
  a.k_scale = p->k_scale;
  a.v_scale = p->v_scale;
  a.bias = p->qk_bias;
  a.rowmax = p->rowmax_est;
  a.v_alpha = p->v_alpha;
  a.stats = p->blasst_stats;
  a.row_skips = p->blasst_row_skips;
  a.wave_tiles = p->blasst_wave_tiles;
  a.vcol = p->v_tile_colsum;
  a.rowmax_init = p->rowmax_init;
  a.out = p->out;
  a.out_dtype = p->out_dtype;
  a.out_row_map = p->out_row_map;
  return 0;
}

// Scores of the attention K-loop, in log2 units, u = acc * C, for a list of
// query rows: the same operand bytes in the same MFMA K slots (slot k of the
// 64-wide half hh holds d = 64 hh + k), the same accumulator start
// bias * (1/qC * rcp(k scale)), the halves accumulated in the same order and
// the same score scale C = qC * k scale, so the values are the ones the
// attention kernel forms (its keys sit in other accumulator rows, which does
// not change any element's sum).  One wave = 32 rows x 32 keys.
template <int D, bool QK_MX, bool HAS_BIAS>
__global__ void __launch_bounds__(64) attn_scores_kernel(const KArgs a, const int32_t* rows, int nrows, float* u) {
  constexpr int NH = D / 64;
  const int lane = threadIdx.x, li = lane & 31, g = lane >> 5;
  const int bh = blockIdx.z;
  const int ri = blockIdx.y * 32 + li;
  const int qi = rows[ri < nrows ? ri : nrows - 1];
  const int kb0 = blockIdx.x * 32;
  const int S = a.S, P = a.P;
  v8i qop[NH], kop[NH];
  int qe[NH], ke[NH];
  const int key_a = kb0 + li < S ? kb0 + li : S - 1;  // A row li (keys past S are never stored)
  const uint8_t* qrow = a.q_codes + (static_cast<size_t>(bh) * P + qi) * D;
  const uint8_t* krow = a.k_codes + (static_cast<size_t>(bh) * P + key_a) * D;
#pragma unroll
  for (int hh = 0; hh < NH; ++hh) {
    qop[hh] = lds_read32(qrow + 64 * hh + 16 * g, qrow + 64 * hh + 32 + 16 * g);
    kop[hh] = lds_read32(krow + 64 * hh + 16 * g, krow + 64 * hh + 32 + 16 * g);
    qe[hh] = 127;
    ke[hh] = 127;
    if constexpr (QK_MX) {
      qe[hh] = reinterpret_cast<const uint8_t*>(a.q_scale)[(static_cast<size_t>(bh) * P + qi) * (D / 32) + 2 * hh + g];
      ke[hh] = reinterpret_cast<const uint8_t*>(a.k_scale)[(static_cast<size_t>(bh) * P + key_a) * (D / 32) + 2 * hh + g];
    }
  }
  float qC = a.sml2;
  if constexpr (!QK_MX) qC *= reinterpret_cast<const float*>(a.q_scale)[bh * a.nqkblk + (qi >> a.lg_qkblk)];
  const float inv_qC = 1.0f / qC;
  int grp = 0;
  if constexpr (HAS_BIAS) {
    grp = qi >> a.lg_qgroup;
    if (grp >= a.G) grp = a.G - 1;
  }
  auto kscale = [&](int key) -> float {
    int kb = key >> a.lg_qkblk;
    kb = kb < a.nqkblk ? kb : a.nqkblk - 1;
    return reinterpret_cast<const float*>(a.k_scale)[bh * a.nqkblk + kb];
  };
  v16f acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    acc[r] = 0.0f;
    if constexpr (HAS_BIAS) {
      const int kr = kb0 + 8 * (r >> 2) + 4 * g + (r & 3);
      const int kc = kr < S ? kr : S - 1;
      float rr = 1.0f;
      if constexpr (!QK_MX) rr = __builtin_amdgcn_rcpf(kscale(kc));
      acc[r] = a.bias[(static_cast<size_t>(bh) * a.G + grp) * P + kc] * (inv_qC * rr);
    }
  }
#pragma unroll
  for (int hh = 0; hh < NH; ++hh) acc = mfma32<QK_MX>(kop[hh], qop[hh], acc, ke[hh], qe[hh]);
  if (ri >= nrows) return;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int kr = kb0 + 8 * (r >> 2) + 4 * g + (r & 3);
    if (kr >= S) continue;
    const float Ct = QK_MX ? qC : qC * kscale(kr);
    u[(static_cast<size_t>(bh) * nrows + ri) * S + kr] = acc[r] * Ct;
  }
#pragma unroll
  for (int hh = 0; hh < NH; ++hh) {
    use(qe[hh]);
    use(ke[hh]);
  }
}

// Column sums of the V^T codes over each 64-key tile: colsum[bh][t][d] =
// sum over keys k < S of tile t of decode(code[d][k]), times the E8M0 scale
// of the (key block, d) pair for MX V (every tile lies inside one V block).
// One thread per d reads the row's 64 contiguous bytes.
__global__ void __launch_bounds__(128) v_colsum_kernel(const uint8_t* __restrict__ vt, int S, int P, int D,
                                                       int v_mx, const uint8_t* __restrict__ ve, int lg_vblk,
                                                       int nvblk, float* __restrict__ out) {
  const int d = threadIdx.x, t = blockIdx.x, bh = blockIdx.y;
  if (d >= D) return;
  const int key0 = t * kTN;
  const uint8_t* row = vt + (static_cast<size_t>(bh) * D + d) * P + key0;
  const int nv = S - key0 < kTN ? S - key0 : kTN;
  float part[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int c = 0; c < kTN / 16; ++c) {
    const uint4 x = *reinterpret_cast<const uint4*>(row + 16 * c);
    const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int k = 16 * c + 4 * q + b;
        const float v = __builtin_amdgcn_cvt_f32_fp8(static_cast<int>(w[q] >> (8 * b)), 0);
        part[b] += k < nv ? v : 0.0f;
      }
  }
  float sum = (part[0] + part[1]) + (part[2] + part[3]);
  if (v_mx) sum = ldexpf(sum, static_cast<int>(ve[(static_cast<size_t>(bh) * nvblk + (key0 >> lg_vblk)) * D + d]) - 127);
  out[(static_cast<size_t>(bh) * (P / kTN) + t) * D + d] = sum;
}

}  // namespace

extern "C" int lbfq_v_tile_colsum(const uint8_t* v_codes_t, int64_t BH, int64_t S, int64_t s_pitch, int64_t D,
                                  int v_kind, const void* v_scale, int v_block, float* colsum,
                                  lbfq_stream_t stream) {
  LBFQ_CHECK_ARG(v_codes_t && colsum && BH > 0 && S > 0, "lbfq_v_tile_colsum: bad arguments");
  LBFQ_CHECK_ARG(D == 64 || D == 128, "lbfq_v_tile_colsum: D must be 64 or 128");
  LBFQ_CHECK_ARG(s_pitch >= S && s_pitch % kTN == 0 && s_pitch < (int64_t{1} << 30),
                 "lbfq_v_tile_colsum: s_pitch must be >= S and a multiple of %d", kTN);
  LBFQ_CHECK_ARG(BH <= 65535, "lbfq_v_tile_colsum: too many heads");
  LBFQ_CHECK_ARG(v_kind != 2 || (v_scale && v_block >= kTN && is_pow2(v_block) && S % v_block == 0),
                 "lbfq_v_tile_colsum: MX V needs its scales and a block (power of two >= %d) dividing S", kTN);
  const int mx = v_kind == 2;
  dim3 grid(static_cast<unsigned>((S + kTN - 1) / kTN), static_cast<unsigned>(BH));
  hipLaunchKernelGGL(v_colsum_kernel, grid, dim3(128), 0, static_cast<hipStream_t>(stream), v_codes_t,
                     static_cast<int>(S), static_cast<int>(s_pitch), static_cast<int>(D), mx,
                     reinterpret_cast<const uint8_t*>(v_scale), mx ? ilog2(v_block) : 0,
                     mx ? static_cast<int>(S / v_block) : 1, colsum);
  LBFQ_LAUNCH_CHECK("lbfq_v_tile_colsum");
  return 0;
}

extern "C" int lbfq_attention_fwd(const lbfq_attn_params* p, lbfq_stream_t stream) {
  KArgs a;
  if (make_kargs(p, a, "lbfq_attention_fwd")) return -1;
  LBFQ_CHECK_ARG(p->v_codes_t && p->out, "lbfq_attention_fwd: missing tensor");
  LBFQ_CHECK_ARG(p->v_kind >= 0 && p->v_kind <= 2 && p->v_scale, "lbfq_attention_fwd: bad V kind");
  const int bn = p->block_n == 128 ? 128 : kTN;
  LBFQ_CHECK_ARG(p->v_kind == 0 || (p->v_block >= kTN && is_pow2(p->v_block) && p->S % p->v_block == 0),
                 "lbfq_attention_fwd: V block (%d) must be a power of two >= %d dividing S", p->v_block, kTN);
  LBFQ_CHECK_ARG(p->v_kind != 1 || p->v_block % bn == 0,
                 "lbfq_attention_fwd: v_block_size (%d) must be a multiple of block_n (%d)", p->v_block, bn);
  LBFQ_CHECK_ARG(p->p_mode >= 0 && p->p_mode <= 2, "lbfq_attention_fwd: bad P mode");
  LBFQ_CHECK_ARG(!p->v_alpha || (p->v_smooth_block >= bn && is_pow2(p->v_smooth_block) &&
                                  p->S % p->v_smooth_block == 0),
                 "lbfq_attention_fwd: v_smooth_block must be a power of two >= block_n (%d) dividing S", bn);
  LBFQ_CHECK_ARG(!p->blasst_stats || p->block_m > 0, "lbfq_attention_fwd: block_m must be positive");
  LBFQ_CHECK_ARG(p->blasst_lambda < 1.0f, "lbfq_attention_fwd: lambda must be < 1");
  LBFQ_CHECK_ARG(p->blasst_lambda <= 0.0f || p->blasst_fill != FILL_UTA ||
                     (p->blasst_uta_bins > 0 && bn % p->blasst_uta_bins == 0),
                 "lbfq_attention_fwd: UTA bins must divide block_n (%d)", bn);
  LBFQ_CHECK_ARG(p->blasst_fill >= FILL_ZERO && p->blasst_fill <= FILL_UTA, "lbfq_attention_fwd: bad fill kind");
  LBFQ_CHECK_ARG(p->out_dtype >= 0 && p->out_dtype <= 2, "lbfq_attention_fwd: bad out dtype");

  const bool blasst = p->blasst_lambda > 0.0f;
  const int rb = p->rowmax_est ? RB_EST_BIAS : (p->qk_bias ? RB_ONLINE_BIAS : RB_ONLINE);
  const bool valpha = p->v_alpha != nullptr;
  const bool mx = p->qk_mx != 0;
  const int D = static_cast<int>(p->D);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int bl = !blasst ? 0 : p->blasst_fill != FILL_UTA ? 1 : (p->blasst_uta_bins <= 16 ? 2 : 3);
  if (bn == 128) {
    if (p->p_mode == 0) return launch_b128_p0(a, D, mx, rb, bl, valpha, st);
    if (p->p_mode == 1) return launch_b128_p1(a, D, mx, rb, bl, valpha, st);
    return launch_b128_p2(a, D, mx, rb, bl, valpha, st);
  }
  if (p->p_mode == 0) return launch_p0(a, D, mx, rb, bl, valpha, st);
  if (p->p_mode == 1) return launch_p1(a, D, mx, rb, bl, valpha, st);
  return launch_p2(a, D, mx, rb, bl, valpha, st);
}

extern "C" int lbfq_attention_scores(const lbfq_attn_params* p, const int32_t* rows, int64_t n_rows, float* u,
                                     lbfq_stream_t stream) {
  KArgs a;
  if (make_kargs(p, a, "lbfq_attention_scores")) return -1;
  LBFQ_CHECK_ARG(rows && u && n_rows > 0 && n_rows < (int64_t{1} << 24), "lbfq_attention_scores: bad row list");
  dim3 grid(static_cast<unsigned>((p->S + 31) / 32), static_cast<unsigned>((n_rows + 31) / 32),
            static_cast<unsigned>(p->B * p->H));
  LBFQ_CHECK_ARG(grid.z <= 65535 && grid.y <= 65535, "lbfq_attention_scores: grid too large");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int nr = static_cast<int>(n_rows);
  const bool bias = p->qk_bias != nullptr;
#define LBFQ_SC(DD, MX, BI) hipLaunchKernelGGL((attn_scores_kernel<DD, MX, BI>), grid, dim3(64), 0, st, a, rows, nr, u)
#define LBFQ_SC_B(DD, MX) \
  if (bias) { LBFQ_SC(DD, MX, true); } else { LBFQ_SC(DD, MX, false); }
#define LBFQ_SC_M(DD) \
  if (p->qk_mx) { LBFQ_SC_B(DD, true) } else { LBFQ_SC_B(DD, false) }
  if (p->D == 128) { LBFQ_SC_M(128) } else { LBFQ_SC_M(64) }
#undef LBFQ_SC_M
#undef LBFQ_SC_B
#undef LBFQ_SC
  LBFQ_LAUNCH_CHECK("lbfq_attention_scores");
  return 0;
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
