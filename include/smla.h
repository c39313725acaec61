/* smla — MI355X (gfx950) sparse multi-head latent attention for DeepSeek-V4-Flash.
 *
 * C ABI of libsmla.so.  Every entry point takes device pointers, element counts and a HIP
 * stream (as void*, NULL = the default stream), enqueues its kernels on that stream and returns
 * without synchronising.  The caller owns every buffer (inputs, outputs, workspace); the library
 * never allocates or frees caller memory.  Tensors are dense and row-major in the shapes given.
 *
 * Return value: SMLA_OK (0); a negative SMLA_E_* code for an argument error, detected on the
 * host before anything is launched; or a positive hipError_t from the launch.
 *
 * Reference counterparts (the reference is plain Python; these replace its functions):
 *   smla_sparse_attn          ref_torch/sparse_attn.py:23-34   sparse_attn(q, kv, attn_sink, topk_idxs, scale)
 *                             v4mlx/sparse_attn.py:26-39       (MLX twin)
 *   smla_sparse_attn_ex       ref_torch/sparse_attn.py:23-34   (the same, with an explicit split plan / phases)
 *   smla_prefill_attn         oracle/decode_engine.py:107-117  per-position prompt attention (row sets on device)
 *   smla_decode_attn          oracle/decode_engine.py:110-117  decode index build + attention (indexer-ranked cidx)
 *   smla_window_topk_idxs     ref_torch/sparse_attn.py:9-20    get_window_topk_idxs(window_size, bsz, seqlen, start_pos)
 *   smla_decode_window_idxs   oracle/decode_engine.py:110-111  widx = range(max(0, p-127), p+1)
 *   smla_indexer_score        (none: the reference attends every visible compressed row,
 *                              oracle/decode_engine.py:112-114; the indexer is the build's)
 *   smla_indexer_score_fp4    (none, as above; keys in the form v4mlx/compressor.py:57-59 gives them)
 *   smla_topk                 oracle/decode_engine.py:112-114  cidx selection (take-all when nvis <= k)
 *   smla_select_decode        oracle/decode_engine.py:110-114  widx + cidx in one launch
 *   smla_index_decode         oracle/decode_engine.py:110-114  indexer scores + widx + cidx (fused)
 *   smla_block_mean_pool      (none: block mean of the 32K decode workload)
 *   smla_gated_pool           ref_torch/compressor.py:41-49    pooling + RMSNorm + RoPE of compressor_prefill
 *   smla_ring_step            oracle/decode_engine.py:96-105   decode compressor ring step and cache append
 *   smla_quant_fp8_pow2       v4mlx/compressor.py:11-20        act_quant_sim (stored form: codes + pow2 scales)
 *   smla_row_epilogue         oracle/decode_engine.py:78-83    q/kv row norms, RoPE, fp8 sim, window-cache write
 *   smla_ring_step_kv         oracle/decode_engine.py:81-84,96-105  kv window append + ring step in one launch
 *   smla_row_epilogue_ids     oracle/decode_engine.py:78-80,110-114  per-head q epilogue + decode ids in one launch
 *   smla_decode_ids           oracle/decode_engine.py:110-114  decode id list (window + visible compressed rows)
 *   smla_rotate_fp4           v4mlx/qat.py:8-31                hadamard_rotate, fp4_act_quant (and stored form)
 *                             v4mlx/compressor.py:57-59        the indexer compressor's key transform
 *   smla_rope                 ref_torch/norm_rope.py:53-62     apply_rotary_emb(x, freqs_cis, inverse) in place
 *                             v4mlx/norm_rope.py:46-62         (MLX twin, cos/sin tables)
 *   smla_linear               v4mlx/mla.py:16-18               linear(x, W) (and the grouped form of mla.py:49-53)
 *   smla_o_proj               oracle/decode_engine.py:118-119  inverse RoPE of o's rope dims + o_grouped
 *                             v4mlx/mla.py:42-56               o_grouped(o, wo_a, wo_b)
 */
#ifndef SMLA_H
#define SMLA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SMLA_API_VERSION 2

/* element types */
enum {
  SMLA_F32 = 0,
  SMLA_BF16 = 1,
  SMLA_FP8_E4M3 = 2, /* OCP e4m3fn (max 448), one byte per element */
  SMLA_F16 = 3,
  SMLA_I32 = 4
};

/* status codes */
enum {
  SMLA_OK = 0,
  SMLA_E_NULL = -1,        /* a required pointer is NULL */
  SMLA_E_SHAPE = -2,       /* a size is non-positive or inconsistent */
  SMLA_E_DTYPE = -3,       /* unsupported element type for this argument */
  SMLA_E_UNSUPPORTED = -4, /* valid but unimplemented combination */
  SMLA_E_WORKSPACE = -5,   /* workspace missing or too small */
  SMLA_E_RANGE = -6        /* a scalar argument is out of its valid range */
};

/* Human-readable text for a status code (static storage). */
const char* smla_strerror(int status);

/* SMLA_API_VERSION of the loaded library. */
int smla_api_version(void);

/* ---------------------------------------------------------------------------------------------
 * Sparse attention over gathered latent rows (absorbed MLA).
 * Replaces ref_torch/sparse_attn.py:23-34 (sparse_attn) and v4mlx/sparse_attn.py:26-39.
 *
 *   q          [B, S, H, D]          q_dtype: F32 or BF16
 *   kv0        [B, n0, D]            kv rows; kv_dtype: F32, BF16 or FP8_E4M3
 *   kv1        [B, n1, D] or NULL    second row source; the index space is the virtual
 *                                    concatenation [kv0; kv1] (the engine's [window; compressed]
 *                                    buffer, oracle/decode_engine.py:108-109) without copying
 *   kv0_scale, kv1_scale             FP8 only: [B, n, D/64] fp32 scale per 64-element tile
 *                                    (row value = decode(code) * scale); NULL otherwise
 *   attn_sink  [H] fp32 or NULL      NULL = -inf (no sink)
 *   topk_idxs  [B, S, T] int32       row ids in [0, n0+n1); negative = masked.  Ids outside the
 *                                    range are treated as masked (the reference raises instead).
 *   out        [B, S, H, DV]         out_dtype: F32 or BF16; value = first DV columns of the rows
 *   scale      softmax scale applied to q.kv
 *
 * out[b,s,h,:] = sum_t p_t kv[idx_t, :DV] / (sum_t p_t + exp(sink_h - m)),
 *   p_t = exp(scale q.kv[idx_t] - m), m = max over valid t.  No valid index -> NaN.
 * Duplicate ids count once per occurrence.
 *
 * Kernels: q BF16 with BF16 or FP8 rows, H % 16 == 0, D 576 or 512, DV 512 and a plan of at
 * most 1024 splits (index lists up to 8192 rows per split) run the split-K MFMA kernel plus the
 * merge, in launches of at most 65528 query rows (whole sequences while one fits, else pieces of
 * one); every other call (F32 / F16 operands, other H / D / DV, more splits) runs the vector-ALU
 * kernel, one workgroup per (query row, head) -- with fewer of those than compute units, per run
 * of the list (up to 64 runs and a merge) -- with the same results to the tolerance of its dtype
 * (both kernels are tested against the oracle for F32, BF16 and FP8 rows).
 *
 * workspace: smla_sparse_attn_workspace() bytes (split-K partial states), may be 0.
 */
int smla_sparse_attn(const void* q, int q_dtype,
                     const void* kv0, int64_t n0, const void* kv1, int64_t n1, int kv_dtype,
                     const float* kv0_scale, const float* kv1_scale,
                     const float* attn_sink, const int32_t* topk_idxs, int64_t T,
                     int64_t B, int64_t S, int64_t H, int64_t D, int64_t DV, float scale,
                     void* out, int out_dtype, void* workspace, size_t workspace_bytes,
                     void* stream);

/* Workspace bytes smla_sparse_attn needs for these sizes (its default split plan), enough for
 * either output type. */
size_t smla_sparse_attn_workspace(int64_t B, int64_t S, int64_t H, int64_t D, int64_t DV,
                                  int64_t T, int q_dtype, int kv_dtype);

/* The split plan of the attention path for these sizes, a pure function of the arguments and the
 * device's compute-unit count.  rows_per_split: index-list rows per split requested (a multiple of
 * 32), or 0 for the default plan (enough splits to give every compute unit a workgroup, at least
 * two 32-row tiles each).  Writes the number of splits (0 when the vector-ALU kernel runs: F32 /
 * F16 operands or shapes the MFMA kernel does not take; its own list runs are not reported) and
 * the rows per split, either pointer may be NULL; returns the workspace bytes that plan needs for
 * out_dtype (0: none; for the vector-ALU kernel, its runs' states). */
size_t smla_sparse_attn_plan(int64_t B, int64_t S, int64_t H, int64_t D, int64_t DV, int64_t T,
                             int q_dtype, int kv_dtype, int out_dtype, int64_t rows_per_split,
                             int64_t* nsplit, int64_t* rows_per_split_out);

/* Phases of smla_sparse_attn_ex: the split kernel (partial states into the workspace, or the
 * output itself when the plan has one split) and the merge of the partial states into out. */
enum { SMLA_ATTN_SPLIT = 1, SMLA_ATTN_MERGE = 2 };

/* smla_sparse_attn with an explicit split plan (rows_per_split as in smla_sparse_attn_plan, 0 =
 * the default) and a choice of its launches (phases: SMLA_ATTN_SPLIT, SMLA_ATTN_MERGE or both).
 * Both phases with rows_per_split 0 is smla_sparse_attn.  A merge alone reads the partial states
 * a split launch with the same arguments left in the workspace; a split alone writes out only
 * when the plan has one split.  The workspace holds smla_sparse_attn_plan(...) bytes.
 * Replaces ref_torch/sparse_attn.py:23-34, like smla_sparse_attn. */
int smla_sparse_attn_ex(const void* q, int q_dtype,
                        const void* kv0, int64_t n0, const void* kv1, int64_t n1, int kv_dtype,
                        const float* kv0_scale, const float* kv1_scale,
                        const float* attn_sink, const int32_t* topk_idxs, int64_t T,
                        int64_t B, int64_t S, int64_t H, int64_t D, int64_t DV, float scale,
                        void* out, int out_dtype, int64_t rows_per_split, int phases,
                        void* workspace, size_t workspace_bytes, void* stream);

/* smla_sparse_attn without a workspace argument: the same plan, kernels and output, with the split
 * partial states in a buffer of SMLA_NOALLOC_SCRATCH_BYTES that the library holds on each device
 * (from the first call on that device until the process ends).  No counterpart in the reference:
 * it is for callers that cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Allocates nothing; returns SMLA_E_WORKSPACE, before any
 * launch, when the plan's partial states exceed the buffer (smla_sparse_attn_workspace gives the
 * size).  Every call on a device shares that device's buffer: calls that overlap on one device
 * (concurrent streams, threads) race and must be serialised by the caller.  The partial states
 * are fully written before they are read, so nothing needs clearing between calls. */
#define SMLA_NOALLOC_SCRATCH_BYTES (32u << 20)
int smla_sparse_attn_noalloc(const void* q, int q_dtype,
                             const void* kv0, int64_t n0, const void* kv1, int64_t n1, int kv_dtype,
                             const float* kv0_scale, const float* kv1_scale,
                             const float* attn_sink, const int32_t* topk_idxs, int64_t T,
                             int64_t B, int64_t S, int64_t H, int64_t D, int64_t DV, float scale,
                             void* out, int out_dtype, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Prompt (prefill) attention with the row sets computed on the device.  Replaces the per-position
 * loop of oracle/decode_engine.py:107-117 with decode_pos = None: query s of sequence b sits at
 * position p = q_pos0 + s and attends
 *   raw rows max(0, p-window+1) .. p            (ids 0 .. n_raw-1, list entries 0 .. window-1)
 *   compressed rows 0 .. min((p+1)/ratio, n_comp)-1 (ratio > 0; list entries window ..)
 * exactly the sparse_attn call of the reference for that position (same result as
 * smla_sparse_attn over those index lists, bit for bit).  No index tensor and no workspace.
 *   q [B,S,H,D] BF16, kv_raw [B,n_raw,D] BF16, kv_comp [B,n_comp,D] BF16 or NULL (ratio 0),
 *   D 576 or 512, DV 512, H % 16 == 0, q_pos0 + S <= n_raw,
 *   out [B,S,H,DV] BF16 or F32.  Workgroups take the queries longest list first, in launches of
 *   at most 65528 queries (whole sequences while one fits, else pieces of one). */
int smla_prefill_attn(const void* q, int q_dtype, const void* kv_raw, int64_t n_raw,
                      const void* kv_comp, int64_t n_comp, int kv_dtype, const float* attn_sink,
                      int64_t q_pos0, int64_t window, int64_t ratio, int64_t B, int64_t S,
                      int64_t H, int64_t D, int64_t DV, float scale, void* out, int out_dtype,
                      void* stream);

/* ---------------------------------------------------------------------------------------------
 * Decode attention over the engine's index build in one call.  Replaces
 * oracle/decode_engine.py:110-117 (widx + cidx, then sparse_attn over [window; compressed]) with
 * the compressed part ranked by indexer scores: query row r (of R = B*S) attends
 *   the raw rows of positions pos[r]-window+1 .. pos[r] (those >= 0), position pp at row
 *   pp mod n_raw (ids 0 .. n_raw-1; kv_raw is a ring of n_raw >= window rows, e.g. the 128-row
 *   window of oracle/v4_fast.py:93-96, or a cache with a row per position)
 *   the min(k, nvis[r]) best of scores[r, 0 .. nvis[r]-1] (score descending, index ascending,
 *   -0 == +0), compressed row c as id n_raw + c
 * i.e. the list smla_select_decode(scores, R, N, nvis, k, pos, window, ids, window+k, n_raw)
 * writes, followed by smla_sparse_attn(q, kv_raw, n_raw, kv_comp, n_comp, ..., ids, window+k).
 * The output equals that pair's bit for bit.  With bf16 rows, the short-split plan and
 * N <= 18432, the attention workgroups run the selection themselves (no list in memory, one
 * launch fewer); otherwise the list is built in the workspace first.
 *   q [B,S,H,D] BF16, kv_raw [B,n_raw,D], kv_comp [B,n_comp,D] BF16 (or F32 / F16: list path),
 *   scores [R,N] F32, nvis [R] int32 or NULL (all N), pos [R] int32, out [B,S,H,DV] BF16 or F32.
 * workspace: smla_decode_attn_workspace(B, S, H, D, DV, window, k, q_dtype, kv_dtype, out_dtype)
 * bytes.  Requires N <= 65536 and window <= n_raw (else SMLA_E_SHAPE). */
size_t smla_decode_attn_workspace(int64_t B, int64_t S, int64_t H, int64_t D, int64_t DV, int64_t window,
                                  int64_t k, int q_dtype, int kv_dtype, int out_dtype);
int smla_decode_attn(const void* q, int q_dtype, const void* kv_raw, int64_t n_raw, const void* kv_comp,
                     int64_t n_comp, int kv_dtype, const float* attn_sink, const float* scores, int64_t N,
                     const int32_t* nvis, const int32_t* pos, int64_t window, int64_t k, int64_t B,
                     int64_t S, int64_t H, int64_t D, int64_t DV, float scale, void* out, int out_dtype,
                     void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Window index matrix.  Replaces ref_torch/sparse_attn.py:9-20 (get_window_topk_idxs).
 * out: [bsz, w] int32 when start_pos > 0 (ring or partial window), [bsz, seqlen, min(seqlen, w)]
 * when start_pos == 0 (prefill causal band, -1 above the diagonal).
 */
int smla_window_topk_idxs(int64_t window_size, int64_t bsz, int64_t seqlen, int64_t start_pos,
                          int32_t* out, void* stream);

/* Engine decode window: for each row r, out[r*out_stride + j] = pos[r]-window+1+j (j < window),
 * or -1 where that is negative.  Replaces the widx list of oracle/decode_engine.py:110-111 with
 * ids into an un-ringed raw cache.  pos: [R] int32 on the device. */
int smla_decode_window_idxs(const int32_t* pos, int64_t R, int64_t window, int32_t* out,
                            int64_t out_stride, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Indexer score (no reference counterpart; the build's definition, fixed fp32 order):
 *   dot_h = fma chain over d of q[b,s,h,d]*k[b,n,d];  r_h = max(dot_h, +0)
 *   acc   = fma chain over h of w[b,s,h]*r_h;          score = acc * kscale[b,n]
 *   score = -inf for n >= nvis[b,s].
 *   q [B,S,Hi,Di] F32|BF16;  keys [B,N,Di] F32|BF16|FP8_E4M3;  kscale [B,N] fp32 or NULL (= 1);
 *   weights [B,S,Hi] fp32;  nvis [B,S] int32 or NULL (= N);  scores [B,S,N] fp32.
 */
int smla_indexer_score(const void* q, int q_dtype, const void* keys, int k_dtype,
                       const float* kscale, const float* weights, const int32_t* nvis,
                       int64_t B, int64_t S, int64_t Hi, int64_t Di, int64_t N,
                       float* scores, void* stream);

/* The same score over keys in the indexer compressor's stored fp4 form (v4mlx/compressor.py:57-59
 * applies v4mlx/qat.py:23-31 to every indexer key; smla_rotate_fp4 writes this form):
 *   codes         [B,N,Di/2] uint8, element 2i of a row in the low nibble of byte i, bit 3 the sign
 *                 (e2m1: magnitudes 0, 0.5, 1, 1.5, 2, 3, 4, 6);
 *   block_scales  [B,N,Di/32] uint8 ue8m0: k[b,n,d] = e2m1(code) * 2^(block_scales[b,n,d/32] - 127)
 *                 (byte 0 = 2^-127, byte 255 = NaN), exact in fp32.
 * Every score equals smla_indexer_score's on the decoded fp32 keys, bit for bit.  Di is 32, 64 or
 * 128; q and codes 16-byte aligned, block_scales 2-byte aligned.  Other arguments as above. */
int smla_indexer_score_fp4(const void* q, int q_dtype, const uint8_t* codes,
                           const uint8_t* block_scales, const float* kscale, const float* weights,
                           const int32_t* nvis, int64_t B, int64_t S, int64_t Hi, int64_t Di,
                           int64_t N, float* scores, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Top-k selection over rows of scores [R, N]: rank the first nvis[r] entries (NULL = N) by
 * (score desc, index asc), -0 == +0; keep min(k, nvis); write them in ascending index order as
 * out[r*out_stride + j] = id + id_offset, then -1 up to k.  Bit-exact.  Replaces the compressed
 * index selection of oracle/decode_engine.py:112-114 (identical when nvis <= k).
 * Scores must not be NaN.  workspace: none.
 */
int smla_topk(const float* scores, int64_t R, int64_t N, const int32_t* nvis, int64_t k,
              int32_t* out, int64_t out_stride, int32_t id_offset, void* stream);

/* The whole decode index build of oracle/decode_engine.py:110-114 in one launch: for row r,
 * out[r*out_stride + j] = the raw row of position pp = pos[r]-window+1+j (or -1 where pp < 0) for
 * j < window, then the smla_topk selection of scores row r (ids + id_offset, -1 padded) at columns
 * window..window+k-1.  The raw row of position pp is pp mod id_offset when id_offset > 0 (the
 * raw source is a ring of id_offset rows, the ring order of ref_torch/sparse_attn.py:11-13; a cache
 * with a row per position is the identity), else pp.  pos: [R] int32 on the device;
 * out_stride >= window + k; window <= id_offset when id_offset > 0 (else SMLA_E_SHAPE). */
int smla_select_decode(const float* scores, int64_t R, int64_t N, const int32_t* nvis, int64_t k,
                       const int32_t* pos, int64_t window, int32_t* out, int64_t out_stride,
                       int32_t id_offset, void* stream);

/* Indexer score and decode index build in one call: smla_indexer_score into the workspace
 * followed by smla_select_decode (or smla_topk when window == 0; pos may then be NULL), for
 * R = B*S query rows, with the same output bit for bit.  Replaces the compressed index selection
 * of oracle/decode_engine.py:110-114 with an indexer-ranked one.
 * workspace: smla_index_decode_workspace(B, S, N) bytes (the B*S*N fp32 scores).  Requires
 * ceil(N / 1024) <= 64.  flags: 0 or SMLA_INDEX_EXACT (accepted, no effect: the scores are always
 * the fixed-order ones).
 */
enum { SMLA_INDEX_EXACT = 1 };
int smla_index_decode(const void* q, int q_dtype, const void* keys, int k_dtype, const float* kscale,
                      const float* weights, const int32_t* nvis, int64_t B, int64_t S, int64_t Hi,
                      int64_t Di, int64_t N, int64_t k, const int32_t* pos, int64_t window,
                      int32_t* out, int64_t out_stride, int32_t id_offset, int flags, void* workspace,
                      size_t workspace_bytes, void* stream);
size_t smla_index_decode_workspace(int64_t B, int64_t S, int64_t N);

/* ---------------------------------------------------------------------------------------------
 * Compressor.
 *
 * smla_block_mean_pool: out[b,g,:] = (x[b,rg] + x[b,rg+1] + ... + x[b,rg+r-1]) * (1/r), fp32
 * sum in row order, g < N/r.  x [B,N,D] F32|BF16, out [B,N/r,D] F32|BF16.
 */
int smla_block_mean_pool(const void* x, int x_dtype, int64_t B, int64_t N, int64_t D,
                         int64_t ratio, void* out, int out_dtype, void* stream);

/* Quantisation applied to a compressed row after its RoPE (the `sim` argument of smla_gated_pool
 * and smla_ring_step):
 *   SMLA_SIM_NONE        none (ref_torch/compressor.py:21-50);
 *   SMLA_SIM_FP8         the d-rd non-rope channels fp8 round-tripped with pow2 block-64 scales
 *                        (v4mlx/compressor.py:60-62, apply_sim=True);
 *   SMLA_SIM_ROTATE_FP4  all d channels Hadamard-rotated, then fp4 round-tripped with pow2
 *                        block-32 scales (v4mlx/compressor.py:57-59, rotate=True: the indexer
 *                        compressor). */
enum { SMLA_SIM_NONE = 0, SMLA_SIM_FP8 = 1, SMLA_SIM_ROTATE_FP4 = 2 };

/* smla_gated_pool: the pooling half of ref_torch/compressor.py:21-50 (compressor_prefill), from
 * the projections kv = x@wkv^T and score = x@wgate^T:
 *   kv, score [B,N,2d] fp32 (N a multiple of ratio);  ape [ratio,2d];  norm_w [d];
 *   cos, sin [>= N, rd/2] fp32 rotation tables indexed by token position (row g uses position
 *   g*ratio);  out [B, N/ratio, d] fp32, quantised as `sim` says (SMLA_SIM_*).
 *   d is 128, 256 or 512; (d - rd) % 64 == 0; ratio <= 8; kv, score and ape 8-byte aligned
 *   (SMLA_E_UNSUPPORTED otherwise).
 */
int smla_gated_pool(const float* kv, const float* score, const float* ape, const float* norm_w,
                    const float* cos_t, const float* sin_t, int64_t B, int64_t N, int64_t d,
                    int64_t ratio, int64_t rd, float eps, int sim, float* out, void* stream);

/* smla_ring_step: one decode token of the compressor ring (oracle/decode_engine.py:96-105) for
 * B sequences at positions pos[b]:
 *   ring_kv, ring_sc [B, 2*ratio, 2d] fp32 (updated);  kv_p, score_p: B rows of 2d fp32
 *   projections, ld_p elements apart (0: 2d);
 *   when (pos+1) % ratio == 0 the ring emits a row (softmax pool, RMSNorm(norm_w), RoPE with
 *   cos/sin [n_pos, rd/2] at position pos+1-ratio, then the `sim` quantisation, SMLA_SIM_*)
 *   written to comp_cache[b, (pos+1)/ratio - 1, :] ([B, comp_cap, d] fp32), then
 *   shifts.  Rows that would land at or past comp_cap are not written.  A sequence whose pos is
 *   negative or whose RoPE position is not below n_pos is left untouched. */
int smla_ring_step(float* ring_kv, float* ring_sc, const float* kv_p, const float* score_p,
                   const int32_t* pos, const float* ape, const float* norm_w,
                   const float* cos_t, const float* sin_t, int64_t n_pos, int64_t B, int64_t d,
                   int64_t ratio, int64_t rd, float eps, int sim, float* comp_cache,
                   int64_t comp_cap, int64_t ld_p, void* stream);

/* smla_row_epilogue: the per-row work of oracle/decode_engine.py:78-83 on rows the caller has
 * projected.  x [rows, d] fp32 (128 <= d <= 1024, d % 64 == 0) -> RMSNorm with norm_w [d]
 * (ref_torch/norm_rope.py:10-16; norm_w NULL gives the weightless per-head norm of v4mlx/mla.py:
 * 26-28), RoPE of the last rd channels (ref_torch/norm_rope.py:53-62, interleaved pairs, cos/sin
 * [n_pos, rd/2]) at position pos[r / rows_per_pos], then `sim` (SMLA_SIM_NONE or SMLA_SIM_FP8: the
 * d-rd other channels fp8 round-tripped, v4mlx/compressor.py:11-20).  Row r goes to row r of out
 * [rows, d] (SMLA_F32 / SMLA_BF16), or, with cache_rows > 0, to row pos mod cache_rows of sequence
 * r / rows_per_pos of a cache [.., cache_rows, d] (the window append, decode_engine.py:84; a cache
 * shorter than the positions is the ring of oracle/v4_fast.py:93-96, winr[p % 128]).  eps: the
 * RMSNorm eps.  ldx: elements between consecutive input rows (0: d).  A row whose position is
 * negative or lies outside [0, n_pos) (when rd > 0) is not written. */
int smla_row_epilogue(const float* x, int64_t rows, int64_t d, int64_t ldx, int64_t rows_per_pos, const int32_t* pos,
                      const float* norm_w, const float* cos_t, const float* sin_t, int64_t n_pos,
                      int64_t rd, float eps, int sim, void* out, int out_dtype, int64_t cache_rows,
                      void* stream);

/* smla_ring_step_kv: smla_ring_step and smla_row_epilogue for the same B sequences at positions
 * pos[b], in one launch: the decode step's kv row (oracle/decode_engine.py:81-84) and its
 * compressor ring (:96-105) both follow the input projection and read nothing else.  The ring
 * arguments are smla_ring_step's.  kv_x [B, d] fp32 (the ring's d) rows ld_kv elements apart
 * (0: d) are normed with kv_norm, their last kv_rd channels rotated with kv_cos/kv_sin
 * [kv_n_pos, kv_rd/2], quantised as kv_sim says (SMLA_SIM_NONE / SMLA_SIM_FP8), and written to row
 * pos[b] mod kv_cache_rows of kv_cache [B, kv_cache_rows, d] (kv_cache_rows > 0) in kv_cache_dtype (SMLA_F32 /
 * SMLA_BF16).  Arguments are checked as the two entry points check them; the results are theirs
 * bit for bit. */
/* smla_row_epilogue_ids: smla_row_epilogue (rows of d = 512; its arguments first) and
 * smla_decode_ids (its arguments after cache_rows, with its own position array ids_pos and
 * row width comp_d) in one launch: the decode step's per-head q norm and RoPE
 * (oracle/decode_engine.py:78-80) and its id list (:110-114) share no data.  Arguments are
 * checked as the two entry points check them (d other than 512: SMLA_E_UNSUPPORTED); the results
 * are theirs bit for bit. */
int smla_row_epilogue_ids(const float* x, int64_t rows, int64_t d, int64_t ldx, int64_t rows_per_pos,
                          const int32_t* pos, const float* norm_w, const float* cos_t, const float* sin_t,
                          int64_t n_pos, int64_t rd, float eps, int sim, void* out, int out_dtype,
                          int64_t cache_rows, const int32_t* ids_pos, int64_t B, int64_t window,
                          int64_t ratio, int64_t n_raw, int64_t ncomp, int32_t* ids, int64_t T,
                          const float* comp32, uint16_t* comp_out, int64_t comp_d, void* stream);

int smla_ring_step_kv(float* ring_kv, float* ring_sc, const float* kv_p, const float* score_p,
                      const int32_t* pos, const float* ape, const float* norm_w, const float* cos_t,
                      const float* sin_t, int64_t n_pos, int64_t B, int64_t d, int64_t ratio, int64_t rd,
                      float eps, int sim, float* comp_cache, int64_t comp_cap, int64_t ld_p,
                      const float* kv_x, int64_t ld_kv, const float* kv_norm, const float* kv_cos,
                      const float* kv_sin, int64_t kv_n_pos, int64_t kv_rd, float kv_eps, int kv_sim,
                      void* kv_cache, int kv_cache_dtype, int64_t kv_cache_rows, void* stream);

/* smla_decode_ids: the decode id list of oracle/decode_engine.py:110-114 for B sequences at
 * positions pos [B]: ids [B, T] int32 (T >= window), columns 0..window-1 = the raw rows of
 * positions max(0, p-window+1)..p (position pp at row pp mod n_raw: a ring of n_raw >= window
 * rows, or a cache with a row per position) then -1, columns window.. = n_raw + j for the (p+1)/ratio visible
 * compressed rows j < ncomp (ratio 0: none), then -1 (window <= n_raw, else SMLA_E_SHAPE).
 * With comp32 / comp_out (both or neither;
 * [B, ncomp, d] fp32 / bf16), a row the ring emitted at this step ((p+1) % ratio == 0) is copied
 * to comp_out as bf16. */
int smla_decode_ids(const int32_t* pos, int64_t B, int64_t window, int64_t ratio, int64_t n_raw, int64_t ncomp,
                    int32_t* ids, int64_t T, const float* comp32, uint16_t* comp_out, int64_t d, void* stream);

/* smla_quant_fp8_pow2: per 64-element block, s = 2^ceil(log2(max(|x|,1e-4)/448)),
 * code = e4m3(clip(x/s, +-448)) (round to nearest even).  x [rows, D] F32|BF16 (D % 64 == 0),
 * codes [rows, D] uint8, scales [rows, D/64] fp32.  The stored form of act_quant_sim,
 * v4mlx/compressor.py:11-20. */
int smla_quant_fp8_pow2(const void* x, int x_dtype, int64_t rows, int64_t D, uint8_t* codes,
                        float* scales, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Indexer-key transform.  Replaces v4mlx/qat.py:8-31 (hadamard_rotate, fp4_act_quant) as the
 * indexer compressor applies them (v4mlx/compressor.py:57-59).
 *
 *   x       [rows, n] F32 or BF16, n a power of two in 32..1024, 16-byte aligned
 *   flags   SMLA_QAT_ROTATE: y = H_n x * float32(n^-0.5), the butterfly with stages
 *           h = 1, 2, ..., n/2 in float32 (pairs (y[i], y[i+h]) -> (sum, difference));
 *           SMLA_QAT_FP4: per block of 32, s = 2^ceil(log2(max(amax, 6*2^-126) / 6)),
 *           q = e2m1(clip(y / s, +-6)) (round to nearest even, grid 0..6);
 *           both: rotation first (the indexer key path)
 *   out     [rows, n] fp32 or NULL: the result (with FP4, the round trip q * s)
 *   codes   [rows, n/2] uint8 or NULL: packed e2m1 codes, element 2i in the low nibble of byte
 *           i, bit 3 the sign (needs SMLA_QAT_FP4);
 *   scales  [rows, n/32] uint8 ue8m0 (log2(s) + 127), given exactly when codes is.
 * At least one of out / codes.  Bit-exact with the reference's float32 arithmetic; the scale
 * exponent is the exact ceiling of log2 of the float32 quotient amax / 6. */
enum { SMLA_QAT_ROTATE = 1, SMLA_QAT_FP4 = 2 };
int smla_rotate_fp4(const void* x, int x_dtype, int64_t rows, int64_t n, int flags, float* out,
                    uint8_t* codes, uint8_t* scales, void* stream);

/* ---------------------------------------------------------------------------------------------
 * RoPE and the projections around the attention core.
 *
 * smla_rope: in place on x [T, heads, head_dim] (F32 or BF16, 8-byte aligned): the last rd dims
 * of every head, as interleaved pairs (x0, x1), become (x0 c - x1 s, x0 s + x1 c) with
 * c = cos_t[pos[t], j], s = sin_t[pos[t], j] (negated when `inverse`), every product and sum
 * rounded in float32, then the result rounded to x's type.  cos_t, sin_t [n_pos, rd/2] fp32;
 * pos [T] int32 in [0, n_pos).  Replaces ref_torch/norm_rope.py:53-62 and v4mlx/norm_rope.py:46-62. */
int smla_rope(void* x, int x_dtype, int64_t T, int64_t heads, int64_t head_dim, int64_t rd,
              const int32_t* pos, const float* cos_t, const float* sin_t, int64_t n_pos, int inverse,
              void* stream);

/* smla_linear: y[t, g*N + n] = sum_k x[t, g*K + k] * w[g*N + n, k] for G groups of N rows (G = 1
 * is v4mlx/mla.py:16-18, y = x @ W^T; G > 1 is the grouped product of v4mlx/mla.py:49-53).
 *   x [T, G*K], w [G*N, K]: both BF16 or both F32; y [T, G*N] BF16 or F32; float32 accumulation.
 *   16-byte aligned pointers; K % 8 == 0 (BF16) or K % 4 == 0 (F32); any T >= 1.
 *   Decode shapes (BF16, T <= 32, N % 16 == 0, K % 512 == 0) stream w from HBM once (the bound);
 *   other shapes run a tiled MFMA GEMM (128 x 128 tiles, bf16 or fp32 MFMA by operand type). */
int smla_linear(const void* x, int x_dtype, const void* w, int w_dtype, int64_t T, int64_t G,
                int64_t N, int64_t K, void* y, int y_dtype, void* stream);

/* smla_o_proj: the attention output path of oracle/decode_engine.py:118-119 for T tokens:
 *   o [T, heads, head_dim] BF16; when pos != NULL the last rd dims of every head are rotated back
 *   (inverse RoPE at pos[t], cos_t/sin_t [n_pos, rd/2] fp32) on the fly, rounded to bf16;
 *   mid [T, G*R] BF16 (caller workspace) = grouped projection with wo_a [G*R, heads*head_dim/G];
 *   y [T, dim] BF16 or F32 = mid @ wo_b^T with wo_b [dim, G*R].  w_dtype: BF16.
 *   Same limits as smla_linear (BF16 operands); with RoPE head_dim % 64 == 0, rd % 64 == 0 and
 *   each group's slice a whole number of heads, and rd == 64 outside the decode shapes.
 *   Replaces v4mlx/mla.py:42-56 (o_grouped) after the inverse rotary call. */
int smla_o_proj(const void* o, int o_dtype, const int32_t* pos, const float* cos_t,
                const float* sin_t, int64_t n_pos, int64_t T, int64_t heads, int64_t head_dim,
                int64_t rd, int64_t G, int64_t R, const void* wo_a, const void* wo_b, int w_dtype,
                int64_t dim, void* mid, void* y, int y_dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SMLA_H */
