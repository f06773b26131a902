/*
 * liblbfq_hip.so -- C ABI of the MI355X (gfx950) fake-quant attention path.
 *
 * Every entry point takes raw device pointers, int64 sizes and a HIP stream
 * (hipStream_t passed as void*), launches asynchronously on that stream and
 * returns 0 on success, -1 for an invalid argument and -2 for a launch
 * failure; lbfq_last_error() returns the message of the last failure on the
 * calling thread.  The library never allocates or frees device memory and
 * never synchronises: the caller owns every input, output and workspace
 * (the reference wrappers likewise allocate with torch.empty before each
 * Triton launch, e.g. quant_triton.py:68-69, attention_triton.py:616-626).
 *
 * Tensor conventions: "NHD" is (B, S, H, D) contiguous, the reference's
 * layout; "BHSD" is (B, H, S_pitch, D) and "BHDS" is (B, H, D, S_pitch), the
 * head-major layouts the attention kernel streams.  dtype codes: 0 fp32,
 * 1 fp16, 2 bf16.  FP8 is OCP E4M3FN stored as uint8.
 *
 * Citations are the reference interfaces each entry replaces (paths relative
 * to the reference checkout src/low_bit_fake_quant/).
 */
#ifndef LBFQ_H
#define LBFQ_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* lbfq_stream_t;

/* ---- enums ---------------------------------------------------------------- */
enum { LBFQ_F32 = 0, LBFQ_F16 = 1, LBFQ_BF16 = 2 };
enum { LBFQ_SUB_NONE = 0, LBFQ_SUB_COLVEC = 1, LBFQ_SUB_BLOCKVEC = 2 };
enum {
  LBFQ_Q_NONE = 0,          /* transform (+gather/smooth/Hadamard) only          */
  LBFQ_Q_FP8_BLOCK = 1,     /* one FP32 scale per R-row tile of one head        */
  LBFQ_Q_CHANNEL = 2,       /* scale per (b,h,d) = amax_table / 448             */
  LBFQ_Q_MX_QK = 3,         /* power-of-two scale per (row, 32 columns)         */
  LBFQ_Q_MX_V = 4,          /* power-of-two scale per (R-row tile, column)      */
  LBFQ_Q_CHANNEL_AMAX = 5   /* atomic max of |x| per (b,h,d) into amax_table    */
};
enum { LBFQ_LAYOUT_NHD = 0, LBFQ_LAYOUT_BHSD = 1, LBFQ_LAYOUT_BHDS = 2 };
enum { LBFQ_DQ_BLOCK = 0, LBFQ_DQ_CHANNEL = 1, LBFQ_DQ_MX_QK = 2, LBFQ_DQ_MX_V = 3 };

const char* lbfq_last_error(void);

/* ---- prepass: row-tile transform + quantisation ---------------------------
 * Replaces the quantisers quant_triton.py:61-77 (fp8_block_quant), :163-176
 * (fp8_per_channel_quant, with LBFQ_Q_CHANNEL_AMAX then LBFQ_Q_CHANNEL),
 * :255-271 (mxfp8_qk_quant), :354-369 (mxfp8_v_quant); the smoothing
 * writers preprocess.py:38-57, :135-166, :169-193 (subtract a mean, write
 * the work tensor); the Hadamard rotation hadamard.py:77-117; and the
 * reorder gathers kmeans.py:88-89 / :127-135 (gather != NULL).
 * Per element: x[gather[s]] - sub -> round to x_dtype -> (signs, FWHT,
 * *had_scale, round) -> quantise.  One tile = R rows of one (b, h).  The
 * Hadamard rotation goes with quant modes NONE, FP8_BLOCK and MX_QK only
 * (it rotates Q/K); S and the code pitch must be below 2^31. */
typedef struct {
  const void* x; int x_dtype;              /* input, NHD                        */
  int64_t B, S, H, D;                      /* D in {64, 128}                    */
  int R;                                   /* tile rows (quant block along S)   */
  const int32_t* gather;                   /* (B*H, S) source rows or NULL      */
  int sub_mode; const float* sub;          /* COLVEC (B,H,D) / BLOCKVEC (B,S/G,H,D) */
  int sub_block;                           /* G for BLOCKVEC                    */
  void* smoothed;                          /* optional NHD output in x_dtype    */
  int hadamard; const int8_t* signs;       /* signs (H, D) +-1 or NULL          */
  float had_scale;                         /* fp32(1/sqrt(D))                   */
  int quant_mode;                          /* LBFQ_Q_*                          */
  uint8_t* codes; int codes_layout;        /* LBFQ_LAYOUT_*                     */
  int64_t codes_spitch;                    /* S extent of BHSD/BHDS buffers     */
  float* scale;                            /* scale output (see strides)        */
  int64_t sc_b, sc_s, sc_h, sc_d;          /* element strides of scale          */
  uint32_t* amax_table;                    /* (B,H,D) fp32 bits, channel modes  */
  int mx_block;                            /* MX-QK columns per scale (8..D)    */
  int smoothed_stage;                      /* 0: after subtract, 1: after FWHT  */
  int scale_e8m0;                          /* MX modes: write E8M0 bytes, not fp32 */
} lbfq_rowtile_params;

int lbfq_rowtile(const lbfq_rowtile_params* p, lbfq_stream_t stream);

/* Sequential fp64 column sums over `chunk`-row chunks (optionally gathered):
 * mode 0 -> partial (B, nchunk, H, D) fp64; mode 1 -> mean fp32 per chunk.
 * Replaces the reductions of preprocess.py:10-36 (smooth_k, mode 0 +
 * lbfq_colsum_finalize), :60-91 (group_mean_q, mode 1, chunk = block_q) and
 * :94-132 (smooth_v_per_block, mode 1, chunk = block_s). */
int lbfq_colsum(const void* x, int dtype, int64_t B, int64_t S, int64_t H, int64_t D, int chunk,
                const int32_t* gather, int mode, double* partial, float* mean, lbfq_stream_t stream);
int lbfq_colsum_finalize(const double* partial, int64_t B, int64_t nchunk, int64_t H, int64_t D,
                         int64_t S, float* mean, lbfq_stream_t stream);

/* Fill n uint32 words (initialises the channel amax table to bits(1e-4f)). */
int lbfq_fill_u32(uint32_t* p, int64_t n, uint32_t value, lbfq_stream_t stream);

/* FP8 dequantisation of NHD codes to out_dtype: quant_triton.py:111-131
 * (BLOCK), :200-218 (CHANNEL), :300-319 (MX_QK, block = block_d),
 * :398-416 (MX_V, block = block_s). */
int lbfq_dequant(const uint8_t* codes, const float* scale, int64_t B, int64_t S, int64_t H, int64_t D,
                 int mode, int block, void* out, int out_dtype, lbfq_stream_t stream);

/* ---- k-means token reorder (replaces flash-kmeans batch_kmeans_Euclid as
 * called at kmeans.py:78-81 and the argsort/scatter at kmeans.py:84-87) ----
 * x: NHD tensor; per (b, h) slice cluster S tokens of dimension D into K
 * clusters with `iters` Lloyd rounds (deterministic init from `seed`).
 * Workspace: centroids (B*H, K, D) fp32, partial (B*H, ceil(S/1024), K, D)
 * fp64, counts (B*H, ceil(S/1024), K) int32.  Outputs labels / order /
 * inverse as (B*H, S) int32. */
int64_t lbfq_kmeans_workspace_bytes(int64_t B, int64_t S, int64_t H, int64_t D, int K);
int lbfq_kmeans(const void* x, int dtype, int64_t B, int64_t S, int64_t H, int64_t D, int K, int iters,
                uint64_t seed, void* workspace, int32_t* labels, int32_t* order, int32_t* inverse,
                lbfq_stream_t stream);

/* Allocation-free lbfq_kmeans (no counterpart in the reference): for callers
 * that cannot allocate device memory -- code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc.  Same kernels and results
 * as lbfq_kmeans; the workspace is a built-in device array of
 * lbfq_kmeans_noalloc_max_workspace_bytes() (64 MiB) per GPU, held until the
 * process ends.  Returns -1 when lbfq_kmeans_workspace_bytes() exceeds it.
 * Calls that overlap on one GPU share that array and race. */
int64_t lbfq_kmeans_noalloc_max_workspace_bytes(void);
int lbfq_kmeans_noalloc(const void* x, int dtype, int64_t B, int64_t S, int64_t H, int64_t D, int K, int iters,
                        uint64_t seed, int32_t* labels, int32_t* order, int32_t* inverse, lbfq_stream_t stream);

/* ---- qm_k row-max estimate + qm correction table --------------------------
 * Replaces attention.py:366-395 (_estimate_rowmax_from_qm_k) and precomputes
 * the kernel's qm correction attention_triton.py:156-160:
 *   bias[b,h,g,n]   = (qm[b,g,h,:] . K_s[b,n,h,:]) * scale       (fp32)
 *   rowmax[b,h,g]   = max_n bias[b,h,g,n]
 * (the attention path passes scale = sm_scale * log2(e): scores in log2 units)
 * K_s = round_to_dtype(ks[gather[n]] - ks_mean) when ks_mean (B,H,D) fp32 is
 * given (ks is then the raw NHD K), else ks itself (already smoothed); gather
 * (the V-kmeans order) may be NULL.  bias is (B,H,G,s_pitch) (NULL to skip),
 * rowmax (B,H,G) (NULL to skip).  qm_split: caller workspace of B*H*3*G*(D/2)
 * 32-bit words (qm split into bf16 hi/mid/lo), required for bf16 K. */
int lbfq_qmk(const float* qm, const void* ks, int ks_dtype, const int32_t* gather, const float* ks_mean, int64_t B,
             int64_t S, int64_t H, int64_t D, int64_t G, float scale, float* bias, int64_t s_pitch, float* rowmax,
             uint32_t* qm_split, lbfq_stream_t stream);

/* lbfq_qmk fused with the K fp8_block quantiser (quant_triton.py:27-78,
 * applied to K_s in attention.py:533), for bf16 K: the same table and
 * row maxima, plus K_s's codes (B,H,k_pitch,D) E4M3 (rows >= S untouched) and
 * block scales (B,H,S/k_block) fp32, bit-identical to lbfq_rowtile's fp8_block
 * mode on the same K_s.  One pass over K instead of two.  k_block in
 * {16, 32, 64}, S a multiple of it. */
int lbfq_qmk_kquant(const float* qm, const void* ks, int ks_dtype, const int32_t* gather, const float* ks_mean,
                    int64_t B, int64_t S, int64_t H, int64_t D, int64_t G, float scale, float* bias, int64_t s_pitch,
                    float* rowmax, uint32_t* qm_split, uint8_t* k_codes, int64_t k_pitch, float* k_scale,
                    int64_t k_block, lbfq_stream_t stream);

/* ---- FP8-MFMA P-requant attention ------------------------------------------
 * Replaces fake_quant_attention_triton (attention_triton.py:410-671) and its
 * kernel _fake_quant_attn_fwd_kernel (attention_triton.py:48-407), taking
 * FP8 codes + scales instead of pre-dequantised bf16 tensors. */
typedef struct {
  int64_t B, H, S, D;             /* S queries == S keys; D in {64, 128}          */
  int64_t s_pitch;                /* rows of the code buffers, multiple of 128;    */
                                  /* rows [S, s_pitch) of the Q/K codes and columns*/
                                  /* [S, s_pitch) of V^T must hold finite codes    */
                                  /* (the package writes zeros): the masked keys of*/
                                  /* the last tile are read and multiplied by P = 0*/
  const uint8_t* q_codes;         /* (B,H,s_pitch,D)                               */
  const uint8_t* k_codes;         /* (B,H,s_pitch,D)                               */
  const uint8_t* v_codes_t;       /* (B,H,D,s_pitch)                               */
  int qk_mx;                      /* 0: fp8_block scales, 1: MX E8M0 per 32 along D */
  const void* q_scale;            /* fp8_block: (B,H,S/qk_block) fp32;             */
  const void* k_scale;            /* mx: (B,H,s_pitch,D/32) E8M0 bytes             */
  int qk_block;                   /* fp8_block rows per scale: power of two >= 16  */
  int v_kind;                     /* 0 channel, 1 fp8_block, 2 mx                  */
  const void* v_scale;            /* channel (B,H,D) fp32; block (B,H,S/vb) fp32;  */
                                  /* mx (B,H,S/vb,D) E8M0 bytes                    */
  int v_block;                    /* rows per V scale: power of two, >= 64         */
  int p_mode;                     /* 0 elementwise, 1 mx, 2 dynamic               */
  float sm_scale;
  int p_max_offset;
  int block_m;                    /* BLASST stats rows per block (> 0)             */
  const float* qk_bias;           /* (B,H,G,s_pitch) qm.K_s*sm_scale*log2(e), or NULL */
  int q_group;                    /* rows per qm group: power of two >= 32         */
  const float* rowmax_est;        /* (B,H,G) estimate in log2 units, or NULL       */
  int rowmax_dynamic;             /* 1: qm_k thresholds (dynamic P), 0: fixed m    */
  const float* v_alpha;           /* (B,H,S/vsb,D) fp32 or NULL                    */
  int v_smooth_block;             /* power of two, >= 64                           */
  float blasst_lambda;            /* <= 0 disables BLASST                          */
  int blasst_fill;                /* 0 zero,1 max,2 mean,3 logn,4 sample8,5 thr,6 uta */
  float blasst_fill_alpha;
  int blasst_uta_bins;
  float* blasst_stats;            /* (ceil(S/block_m), B*H, 2) fp32, zeroed, or NULL */
  void* out; int out_dtype;       /* NHD (B,S,H,D)                                 */
  const int32_t* out_row_map;     /* (B*H, S): output row of reordered query, or NULL */
  float* blasst_row_skips;        /* (B*H, S) fp32 in output-row order: K blocks each */
                                  /* row skipped (the per-row decisions behind the  */
                                  /* stats, attention_triton.py:165-175), or NULL   */
  int32_t* blasst_wave_tiles;     /* (B*H, ceil(S/128)*4, 2) int32, or NULL: per    */
                                  /* wave of 32 reordered query rows, the block_n-  */
                                  /* key decision blocks (64-key tiles at block_n   */
                                  /* 64, 128-key blocks at 128) every row of it     */
                                  /* skipped and those some row of it skipped       */
  const float* v_tile_colsum;     /* (B*H, s_pitch/64, D) from lbfq_v_tile_colsum, */
                                  /* or NULL.  With a per-row BLASST fill (not uta) */
                                  /* and no V smoothing, a full tile that all 32    */
                                  /* rows of a wave skip is applied as fill x these */
                                  /* sums instead of its PV MFMAs                   */
  int block_n;                    /* keys per row-max update, P scale and BLASST   */
                                  /* decision (the reference's block_n): 64 or 128 */
                                  /* (0 = 64)                                      */
  const float* rowmax_init;       /* (B,H,S) fp32 initial row max in log2 units     */
                                  /* (rowmax_init_bhs * log2(e)), rows in kernel    */
                                  /* order, or NULL; not with rowmax_est            */
} lbfq_attn_params;

int lbfq_attention_fwd(const lbfq_attn_params* p, lbfq_stream_t stream);

/* Column sums of the V^T codes (B*H, D, s_pitch) over each 64-key tile, for
 * lbfq_attn_params.v_tile_colsum: colsum (B*H, s_pitch/64, D) fp32 =
 * sum over the tile's keys k < S of decode(code[d][k]), times 2^(e - 127)
 * with e the E8M0 scale of (block of k, d) for MX V (v_kind 2; v_scale as in
 * lbfq_attn_params).  No counterpart in the reference: it supports the skip
 * of PV work that BLASST decides (attention_triton.py:165-175) -- when every
 * key of a row carries the same fill p, that row's PV product is p times
 * these sums. */
int lbfq_v_tile_colsum(const uint8_t* v_codes_t, int64_t BH, int64_t S, int64_t s_pitch, int64_t D, int v_kind,
                       const void* v_scale, int v_block, float* colsum, lbfq_stream_t stream);

/* Scores of lbfq_attention_fwd's K-loop in log2 units, u = (Q K^T * sm_scale +
 * the qm correction) * log2(e), formed exactly as the kernel forms them (same
 * FP8 MFMA operand layout, accumulation order and scale products), for the
 * query rows `rows` (n_rows indices into the kernel's row order, the same for
 * every (b, h)): u is (B*H, n_rows, S) fp32.  Uses the Q/K fields of p only.
 * A diagnostic: it replaces the score part of attention_triton.py:150-162 so
 * that the reference's softmax / P quantisation can be replayed on the
 * kernel's own scores. */
int lbfq_attention_scores(const lbfq_attn_params* p, const int32_t* rows, int64_t n_rows, float* u,
                          lbfq_stream_t stream);

/* ---- path A: dequantised SDPA, P not quantised -------------------------------
 * Replaces the dequantisation of _fake_quant_attention_sdpa (attention.py:
 * 276-286: _dequant_qk / _dequant_v into the SDPA dtype, quant_triton.py:
 * 81-109, 180-198, 275-298, 373-396, then the V block means added in that
 * dtype).  Codes and scales in the layouts of lbfq_attn_params (the prepass
 * writes them); outputs in the SDPA dtype: q_out, k_out (B,H,s_pitch,D) and
 * v_t_out (B,H,D,s_pitch), rows / keys [S, s_pitch) zero. */
typedef struct {
  int64_t B, H, S, D;             /* D in {64, 128}                                */
  int64_t s_pitch;                /* multiple of 128, >= S                         */
  const uint8_t* q_codes;         /* (B,H,s_pitch,D)                               */
  const uint8_t* k_codes;         /* (B,H,s_pitch,D)                               */
  const uint8_t* v_codes_t;       /* (B,H,D,s_pitch)                               */
  int qk_mx;                      /* 0: fp8_block, 1: MX E8M0 along D              */
  const void* q_scale;            /* fp8_block (B,H,S/qk_block) fp32;              */
  const void* k_scale;            /* mx (B,H,s_pitch,D/qk_block) E8M0 bytes        */
  int qk_block;                   /* fp8_block rows (dividing S) / MX columns      */
  int v_kind;                     /* 0 channel, 1 fp8_block, 2 mx                  */
  const void* v_scale;            /* channel (B,H,D) fp32; block (B,H,S/vb) fp32;  */
                                  /* mx (B,H,S/vb,D) E8M0 bytes                    */
  int v_block;                    /* rows per V scale, dividing S                  */
  const float* v_alpha;           /* (B,H,S/v_smooth_block,D) fp32 V block means,  */
                                  /* or NULL                                       */
  int v_smooth_block;
  int sdpa_dtype;                 /* 1 fp16, 2 bf16                                */
  void* q_out; void* k_out; void* v_t_out;
} lbfq_sdpa_dequant_params;

int lbfq_sdpa_dequant(const lbfq_sdpa_dequant_params* p, lbfq_stream_t stream);

/* Replaces the attention of _fake_quant_attention_sdpa (attention.py:288-319):
 * without qk_bias, F.scaled_dot_product_attention over the dequantised
 * tensors with P in fp32 (:289-294); with qk_bias, the chunked Q-smoothing
 * branch (:296-319): scores = dtype(q.k) * sm_scale + qm.K_s * sm_scale,
 * P = dtype(softmax), O = P V.  Output NHD (B,S,H,D), rounded to the SDPA
 * dtype and stored in out_dtype. */
typedef struct {
  int64_t B, H, S, D, s_pitch;
  const void* q;                  /* (B,H,s_pitch,D) sdpa dtype, rows >= S zero    */
  const void* k;                  /* (B,H,s_pitch,D)                               */
  const void* v_t;                /* (B,H,D,s_pitch), keys >= S zero               */
  int sdpa_dtype;                 /* 1 fp16, 2 bf16                                */
  float sm_scale;
  const float* qk_bias;           /* (B,H,groups,s_pitch) qm.K_s*sm_scale*log2(e)  */
                                  /* (lbfq_qmk), or NULL                           */
  int64_t groups;                 /* qm groups                                     */
  int q_group;                    /* rows per qm group (> 0)                       */
  void* out; int out_dtype;       /* NHD (B,S,H,D)                                 */
  const int32_t* out_row_map;     /* (B*H, S): output row of reordered query, or NULL */
} lbfq_sdpa_params;

int lbfq_sdpa_fwd(const lbfq_sdpa_params* p, lbfq_stream_t stream);

/* ---- diagnostics -------------------------------------------------------------
 * Replaces p_requant.py:44-73 (p_requant_rows, kernel :12-41).  scores is
 * (B, M, N) of dtype `dtype` with element strides ss*; p (E4M3 bytes) has
 * element strides ps*; row_sum and lse are (B, M) fp32, contiguous.  Per row:
 * p = e4m3(2^((x - max) * sm_scale * log2e + p_max_offset)) (saturating),
 * row_sum = sum p, lse = max * sm_scale + ln(row_sum) - p_max_offset * ln 2.
 * sm_scale is double: sm_scale * log2e is folded in double and rounded once,
 * as the reference folds its constexpr product. */
int lbfq_p_requant_rows(const void* scores, int dtype, int64_t B, int64_t M, int64_t N, int64_t ssb, int64_t ssm,
                        int64_t ssn, uint8_t* p, int64_t psb, int64_t psm, int64_t psn, float* row_sum, float* lse,
                        double sm_scale, int p_max_offset, lbfq_stream_t stream);

/* Replaces the diagnostic kernel bench/count_rowmax_updates_triton.py:27-171
 * (_count_kernel) over the operands of lbfq_attention_fwd: FP8 codes BHSD
 * with fp8_block scales, the qm correction table and row-max estimate in log2
 * units.  Adds into counters[6] (int64, caller-zeroed): updates, rescales,
 * upward updates, downward updates, rows with an update, max updates of one
 * row (atomic max).  use_estimate = 0: FA4-style online rule (update when
 * tile max - m > up); 1: qm_k estimate with up/down thresholds, mass floor
 * and down_always as in the reference.  Key tiles are 64 keys. */
typedef struct {
  int64_t B, H, S, D, s_pitch;
  const uint8_t* q_codes; const uint8_t* k_codes;   /* (B,H,s_pitch,D) E4M3     */
  const float* q_scale; const float* k_scale;       /* (B,H,ceil(S/qk_block))   */
  int qk_block;                                     /* fp8_block rows per scale */
  const float* bias;                                /* (B,H,G,s_pitch) or NULL  */
  const float* rowmax_est;                          /* (B,H,G) or NULL          */
  int q_group;                                      /* rows per qm group        */
  float sm_scale;
  float up_threshold_log2, down_threshold_log2, mass_floor;
  int down_always, use_estimate;
  int64_t* counters;
} lbfq_rowmax_count_params;

int lbfq_rowmax_count(const lbfq_rowmax_count_params* p, lbfq_stream_t stream);

/* ---- BLASST tile-skip simulator (blasst_skip.py:389-654) ---------------------
 * Per-head static FP8 fake quant (fake_quant_per_head, blasst_skip.py:278-297):
 * x (S, H, D) of dtype `dtype`; deq (S,H,D) fp32 = e4m3(x / scale) * scale or
 * NULL; deq_mm the same rounded to bf16 (mm_bf16 = 1) or not, or NULL;
 * scale (H) fp32 or NULL; amax_ws (H) workspace; counts[2] += saturated,
 * underflowed-to-zero elements; sqerr[0] += sum (deq - x)^2 (fp64). */
int lbfq_head_fp8_quant(const void* x, int dtype, int64_t S, int64_t H, int64_t D, float* deq, float* deq_mm,
                        int mm_bf16, float* scale, uint32_t* amax_ws, int64_t* counts, double* sqerr,
                        lbfq_stream_t stream);

/* Score scan over (S, H, D) fp32 operands, 128-key blocks: final_max (H, S) =
 * the row max; tile_margin / tile_bmax (H, S/128, S/128) = ordered-integer
 * bits of max over a 128-row tile of (block max - running max) and of block
 * max (blasst_skip.py:375-386, 497-506, 584-590).  S % 128 == 0, D in {64,128}. */
int lbfq_blasst_scan(const float* q, const float* k, int64_t S, int64_t H, int64_t D, float sm_scale,
                     float* final_max, uint32_t* tile_margin, uint32_t* tile_bmax, lbfq_stream_t stream);

/* Tile keep masks for T thresholds (log_thresholds: device fp32, -inf for 0):
 * keep (T, H, S/128, S/128) bytes; a tile keeping no block keeps the first
 * block of largest tile_bmax; counts[2t] += skipped blocks, counts[2t+1] +=
 * forced tiles (blasst_skip.py:597-612). */
int lbfq_blasst_keep(const uint32_t* tile_margin, const uint32_t* tile_bmax, int64_t H, int64_t S,
                     const float* log_thresholds, int T, uint8_t* keep, int64_t* counts, lbfq_stream_t stream);

/* One rung of the simulator (blasst_skip.py:482-619).  mode 0: exact softmax
 * against final_max; 1: online weights exp(s - rm) * exp(rm - M); 2: static P
 * e4m3(exp(s - rm) * 256) / 256 * exp(rm - M) over kept blocks, unquantised
 * denominator (keep == NULL keeps all).  P weights are rounded to bf16 before
 * PV when round_p_bf16.  mode 2 only: dropped (H, S) = fraction of the row's
 * unquantised mass in dropped blocks; p_counts[2] += underflowed-to-zero P,
 * P count; p_sqerr[0] += sum (pq - p)^2. */
typedef struct {
  int64_t S, H, D;
  const float* q; const float* k; const float* v;   /* (S, H, D) fp32 operands   */
  float sm_scale;
  int mode;
  int round_p_bf16;
  const float* final_max;                           /* (H, S) from the scan      */
  const uint8_t* keep;                              /* (H, S/128, S/128) or NULL */
  float* out;                                       /* (S, H, D) fp32            */
  float* dropped;                                   /* (H, S) or NULL            */
  int64_t* p_counts;                                /* [2] or NULL               */
  double* p_sqerr;                                  /* [1] or NULL               */
} lbfq_blasst_attend_params;

int lbfq_blasst_attend(const lbfq_blasst_attend_params* p, lbfq_stream_t stream);

/* ---- measurement probe ----------------------------------------------------- */
/* HBM streaming probe (no counterpart in the reference: it measures the
 * ceiling the prepass is held against).  mode 0 reads `bytes` from src
 * (global_load_dwordx4; sink: 256 uint32 that receive nothing in practice),
 * 1 writes them to dst, 2 copies src to dst; `grid` workgroups of 256
 * threads walk 16 KiB chunks grid-stride.  bytes % 16 == 0, 16-byte aligned
 * pointers. */
int lbfq_hbm_stream(int mode, const void* src, void* dst, int64_t bytes, int grid, uint32_t* sink,
                    lbfq_stream_t stream);
/* Issue-cost probe (no counterpart in the reference: it measures the floor
 * the attention kernel is held against).  One workgroup of 4 * waves_per_simd
 * waves (1 or 2 per SIMD of one CU) runs `iters` iterations of independent
 * instructions of class `op` -- 0 v_mul_f32, 1 v_add_f32, 2 v_fma_f32,
 * 3 v_max3_f32, 4 v_exp_f32, 5 v_cvt_pk_fp8_f32, 6 v_permlane32_swap (16 per
 * iteration), 7 FP8 MFMA 32x32x64 (8 per iteration), 8 the attention step's
 * inherent per-tile mix (8 MFMAs + 198 VALU), 9 that mix's VALU part.
 * rec: 3 int64 per wave (s_memtime at start, at end, SIMD id); sink: one
 * float per thread. */
int lbfq_issue_probe(int op, int waves_per_simd, int iters, long long* rec, float* sink, lbfq_stream_t stream);

/* ---- building-block self tests (GPU unit tests of compiler builtins) ------ */
/* E4M3 conversion of n fp32 values (n even) by the hardware converter. */
int lbfq_selftest_cvt_fp8(const float* x, int64_t n, uint8_t* out, lbfq_stream_t stream);
/* One 32x32x64 FP8 MFMA per wave: A (32x64), B (64x32) E4M3 row-major,
 * optional E8M0 scales per (row, 32-col block) of A and per (col, 32-row
 * block) of B; C (32x32) fp32 row-major. */
int lbfq_selftest_mfma(const uint8_t* a, const uint8_t* b, const uint8_t* a_scale, const uint8_t* b_scale,
                       float* c, lbfq_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* LBFQ_H */
