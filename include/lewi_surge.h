/* C ABI of the MI355X (gfx950) MoE-layer hot path of Lewi Surge.
 *
 * Every entry point is stateless and stream-ordered: it enqueues HIP kernels on `stream` and returns
 * without a host synchronisation.  All pointers are caller-owned device buffers; the library never
 * allocates device memory.  Scratch space is passed in as `workspace` of at least the size the matching
 * `*_workspace_bytes` function reports.  Return value: 0 on success, a negative LSURGE_ERR_* code
 * otherwise; `lsurge_last_error()` then holds a message (thread-local).
 *
 * Reference interfaces replaced (paths in prostos2162-maker/lewi-surge):
 *   modal/moe_permute.py   gather_rows / gather_reduce / gather_dot / sort_indices / dispatch /
 *                          combine / permute_rows (the Pallas-TPU kernels and XLA refs)
 *   modal/padded_gmm.py    padded_ragged_dot (the jax.lax.ragged_dot replacement)
 *   MaxText RoutedMoE      router top-k, SwiGLU experts and shared expert (third-party, not vendored)
 * Each function below cites the reference line it stands in for.  The reference binds its kernels with
 * `pl.pallas_call` inside jit (modal/moe_permute.py:150-158, 203-211); the binding a JAX user adds for
 * these is an XLA FFI custom call per entry point.
 */
#ifndef LEWI_SURGE_H_
#define LEWI_SURGE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* lsurge_stream_t; /* == hipStream_t */

/* element types of row arrays (modal/moe_permute.py:53-54 accepts 32- and 16-bit floats) */
enum { LSURGE_F32 = 0, LSURGE_BF16 = 1, LSURGE_F16 = 2 };

enum {
  LSURGE_OK = 0,
  LSURGE_ERR_INVALID = -1,     /* bad shape / null pointer / out-of-range argument */
  LSURGE_ERR_DTYPE = -2,       /* unsupported element type */
  LSURGE_ERR_LAUNCH = -3,      /* HIP launch failure */
  LSURGE_ERR_WORKSPACE = -4    /* workspace too small */
};

#define LSURGE_ABI_VERSION 3
#define LSURGE_BLOCK_ROWS 128 /* rows per padded expert block */

int lsurge_abi_version(void);
const char* lsurge_last_error(void);

/* Run the independent chains of lsurge_moe_fwd / lsurge_moe_bwd (shared expert, weight gradients, router
 * backward) on helper streams of the current device that fork from and join back into the caller's stream
 * (on = 1), or everything on the caller's stream (on = 0, the default).  Either way a call is stream-ordered
 * on its stream and never synchronises the host.  Process-wide setting.  No reference counterpart: the
 * reference's XLA program is scheduled by XLA. */
int lsurge_set_concurrency(int on);
int lsurge_get_concurrency(void);

/* Kernel family of the bf16 / f16 grouped GEMMs (the layer's row GEMMs and ragged_dot): LSURGE_GEMM_CLASSIC
 * (128 x 256 tiles over 128-row blocks, and the 8-wave ping-pong kernel over 256-row tiles) or LSURGE_GEMM_G256 (the
 * default: persistent 256 x 256 x 64 tiles, one workgroup per CU).  Both compute every output element with the same
 * sequence of MFMA steps, so the results are bitwise identical; the switch exists for same-process A/B timing and for
 * the tests that check that identity.  Process-wide setting.  No reference counterpart (XLA picks the reference's
 * GEMM kernels). */
#define LSURGE_GEMM_CLASSIC 0
#define LSURGE_GEMM_G256 1
int lsurge_set_gemm_variant(int variant);
int lsurge_get_gemm_variant(void);

/* ------------------------------------------------------------------------------------------------
 * Row movement (memory-bound).
 * ------------------------------------------------------------------------------------------------ */

/* out[i] = x[idx[i]], or dtype(f32(x[idx[i]]) * scale[i]) when scale != NULL.
 * x: [n, d] of `dtype`; idx: [m] int32 in [0, n); scale: [m] f32 or NULL; out: [m, d] of `dtype`.
 * Replaces moe_permute.gather_rows (modal/moe_permute.py:116-158). */
int lsurge_gather_rows(const void* x, int64_t n, int64_t d, int dtype, const int32_t* idx, int64_t m,
                       const float* scale, void* out, lsurge_stream_t stream);

/* out[t] = sum_{j<k} w[t,j] * y[pos[t,j]] accumulated in f32, j ascending; w == NULL means w = 1.
 * y: [m, d] of y_dtype; pos: [n, k] int32 in [0, m); out: [n, d] of out_dtype.
 * Replaces moe_permute.gather_reduce (modal/moe_permute.py:161-225, dot=False). */
int lsurge_gather_reduce(const void* y, int64_t m, int64_t d, int y_dtype, const int32_t* pos, int64_t n,
                         int64_t k, const float* w, void* out, int out_dtype, lsurge_stream_t stream);

/* out[t,j] = <g[t], y[pos[t,j]]> in f32.  y: [m, d]; pos: [n, k]; g: [n, d]; out: [n, k] f32.
 * Replaces moe_permute.gather_dot (modal/moe_permute.py:228-234, _reduce_like dot=True). */
int lsurge_gather_dot(const void* y, int64_t m, int64_t d, int y_dtype, const int32_t* pos, int64_t n,
                      int64_t k, const void* g, int g_dtype, float* out, lsurge_stream_t stream);

/* Fused combine backward in one pass over g:  dy[order[p]] ... i.e. for every token t and j<k:
 *   dy[pos[t,j]] = y_dtype(w[t,j] * f32(g[t]))      (moe_permute.py:306-307)
 *   dw[t,j]      = <f32(g[t]), f32(y[pos[t,j]])>    (moe_permute.py:308)
 * y, dy: [n*k, d] of y_dtype; g: [n, d] of g_dtype (rounded to y_dtype first, as g.astype(y.dtype));
 * pos: [n*k] int32 (a permutation); w: [n, k] f32; dw: [n, k] f32.
 * Replaces the two-kernel moe_permute._combine_bwd (modal/moe_permute.py:303-309). */
int lsurge_combine_bwd(const void* y, int y_dtype, const int32_t* pos, const float* w, int64_t n, int64_t k,
                       int64_t d, const void* g, int g_dtype, void* dy, float* dw, lsurge_stream_t stream);

/* inv[idx[i]] = i for a permutation idx of [0, m).  Replaces jnp.argsort(idx) in
 * moe_permute._permute_rows_bwd (modal/moe_permute.py:325-326).  For an idx that is not a permutation: entries
 * outside [0, m) are skipped, entries of inv that no idx hits are m (so a gather through inv gives zero rows
 * there), and of duplicated entries one unspecified i is kept.  No write ever leaves inv. */
int lsurge_invert_permutation(const int32_t* idx, int64_t m, int32_t* inv, lsurge_stream_t stream);

/* ------------------------------------------------------------------------------------------------
 * Routing indices (integer, bit-exact).
 * ------------------------------------------------------------------------------------------------ */

/* Stable sort of the m flat slot experts: order[p] = slot at sorted position p, pos = order^-1;
 * group_sizes (optional, [num_experts]) = bincount.  flat values must lie in [0, num_experts).
 * Replaces moe_permute.sort_indices (modal/moe_permute.py:240-264). */
size_t lsurge_sort_indices_workspace_bytes(int64_t m, int64_t num_experts);
int lsurge_sort_indices(const int32_t* flat, int64_t m, int64_t num_experts, int32_t* order, int32_t* pos,
                        int32_t* group_sizes, void* workspace, size_t workspace_bytes, lsurge_stream_t stream);

/* Router: logits = x @ w_r (+ bias) in f32, summed sequentially over d; sel = top-k with ties broken
 * toward the lower expert index; weights = softmax over the k selected logits.
 * x: [t, d] bf16; w_r: [d, e] bf16; bias: [e] f32 or NULL; logits: [t, e] f32 (may be NULL);
 * sel: [t, k] int32; weights: [t, k] f32.  1 <= k <= e <= 256.
 * Replaces MaxText RoutedMoE gate + top-k (third-party; configs/stage1.yml:34-37). */
int lsurge_router_topk(const void* x, const void* w_r, const float* bias, int64_t t, int64_t d, int64_t e,
                       int64_t k, float* logits, int32_t* sel, float* weights, lsurge_stream_t stream);

/* Padded block layout of the flat slots (m = t*k): stable expert sort (as lsurge_sort_indices) plus
 *   offsets[e]   = exclusive scan of group_sizes,
 *   block_off[e] = exclusive scan of ceil(group_sizes/128),
 *   slot[i]      = 128*block_off[flat[i]] + (pos[i] - offsets[flat[i]])  (padded row of slot i),
 *   row_src[r]   = flat slot stored at padded row r, -1 for padding rows,
 *   blk_expert / blk_rows [max_blocks] = expert and valid rows of block b (-1 / 0 past the end),
 *   num_blocks[0] = sum_e ceil(group_sizes[e]/128).
 * max_blocks must be lsurge_max_blocks(m, e); row_src has 128*max_blocks entries.
 * Replaces sort_indices (modal/moe_permute.py:240-264) + padded_gmm's row<->slot maps
 * (modal/padded_gmm.py:51-64), dropless. */
int64_t lsurge_max_blocks(int64_t m, int64_t num_experts);
size_t lsurge_layout_workspace_bytes(int64_t m, int64_t num_experts);
int lsurge_build_layout(const int32_t* flat, int64_t m, int64_t num_experts, int32_t* group_sizes,
                        int32_t* offsets, int32_t* block_off, int32_t* order, int32_t* pos, int32_t* slot,
                        int32_t* row_src, int32_t* blk_expert, int32_t* blk_rows, int32_t* num_blocks,
                        void* workspace, size_t workspace_bytes, lsurge_stream_t stream);

/* ------------------------------------------------------------------------------------------------
 * Grouped GEMM (bf16 MFMA, f32 accumulation).
 * ------------------------------------------------------------------------------------------------ */

/* Dropless ragged_dot: out[r] = lhs[r] @ rhs[e(r)] for r < sum(group_sizes), 0 for the rows after.
 * lhs: [m, kdim] rows sorted by group and rhs: [e, kdim, n], both of in_dtype (LSURGE_BF16, LSURGE_F16 or
 * LSURGE_F32); group_sizes: [e] int32 (device); out: [m, n] of out_dtype (in_dtype, or LSURGE_F32 for
 * preferred_element_type=float32; f32 operands: LSURGE_F32 or LSURGE_BF16); f32 accumulation.  kdim % 8 == 0,
 * n % 8 == 0.  Workspace: lsurge_ragged_dot_workspace_bytes(m, e) for 16-bit operands,
 * lsurge_ragged_dot_f32_workspace_bytes(m, kdim, n, e) for f32 ones.
 * f32 operands run on the bf16 matrix cores: each value is split into three bf16 terms (24 significant bits) and the
 * six term products of order <= 2 are summed in f32, a GEMM six times as deep (about 2^-24 relative error per
 * product, the einsum's f32 result at precision=HIGHEST); lhs and rhs 16-byte aligned.
 * Replaces padded_gmm.padded_ragged_dot (modal/padded_gmm.py:45-69) / jax.lax.ragged_dot. */
size_t lsurge_ragged_dot_workspace_bytes(int64_t m, int64_t e);
size_t lsurge_ragged_dot_f32_workspace_bytes(int64_t m, int64_t kdim, int64_t n, int64_t e);
int lsurge_ragged_dot(const void* lhs, const void* rhs, const int32_t* group_sizes, int64_t m, int64_t kdim,
                      int64_t n, int64_t e, int in_dtype, void* out, int out_dtype, void* workspace,
                      size_t workspace_bytes, lsurge_stream_t stream);

/* lsurge_ragged_dot that allocates nothing and takes no workspace: its block table lives in a static device array
 * of the library (221 KB per GPU, held until the process ends), so m <= lsurge_ragged_dot_noalloc_max_rows() (2^21)
 * and e <= lsurge_ragged_dot_noalloc_max_groups() (1024); larger calls return LSURGE_ERR_INVALID.  16-bit operands
 * only (f32 ones return LSURGE_ERR_DTYPE: their split terms need a workspace).  Same results as lsurge_ragged_dot.  Calls that overlap on one GPU share the array and race: serialise them (one stream).
 * No counterpart in the reference: for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). */
size_t lsurge_ragged_dot_noalloc_max_rows(void);
size_t lsurge_ragged_dot_noalloc_max_groups(void);
int lsurge_ragged_dot_noalloc(const void* lhs, const void* rhs, const int32_t* group_sizes, int64_t m, int64_t kdim,
                              int64_t n, int64_t e, int in_dtype, void* out, int out_dtype, lsurge_stream_t stream);

/* Backward of lsurge_ragged_dot for upstream g [m, n] of in_dtype: dlhs [m, kdim] in_dtype (rows past the groups
 * = 0) and drhs [e, kdim, n] f32.  Replaces the VJP of padded_gmm.padded_ragged_dot
 * (modal/padded_gmm.py:35-39 + XLA autodiff of the einsum at 67-68).
 * Workspace: lsurge_ragged_dot_bwd_workspace_bytes(m, kdim, n, e) lets drhs cut hot groups into row chunks
 * (e <= 256); the forward's lsurge_ragged_dot_workspace_bytes(m, e) is also accepted (one slice per group).
 * f32 operands (split into bf16 terms as in the forward; 6 m < 2^31) need
 * lsurge_ragged_dot_bwd_f32_workspace_bytes(m, kdim, n, e). */
size_t lsurge_ragged_dot_bwd_workspace_bytes(int64_t m, int64_t kdim, int64_t n, int64_t e);
size_t lsurge_ragged_dot_bwd_f32_workspace_bytes(int64_t m, int64_t kdim, int64_t n, int64_t e);
int lsurge_ragged_dot_bwd(const void* lhs, const void* rhs, const int32_t* group_sizes, const void* g,
                          int64_t m, int64_t kdim, int64_t n, int64_t e, int in_dtype, void* dlhs, float* drhs,
                          void* workspace, size_t workspace_bytes, lsurge_stream_t stream);

/* ------------------------------------------------------------------------------------------------
 * Whole MoE layer: router -> layout -> dispatch -> gate/up GEMM (+SiLU*mul) -> down GEMM -> combine
 * (+ shared expert), and its gather-only backward.
 * Weights follow MaxText's layout: w_gate/w_up = wi_0/wi_1 [e, d, f], w_down = wo [e, f, d]
 * (modal/stage2.py:338-345); shared expert ws_gate/ws_up [d, fs], ws_down [fs, d]; router w_r [d, e].
 * ------------------------------------------------------------------------------------------------ */
typedef struct {
  int64_t t;  /* tokens */
  int64_t d;  /* d_model */
  int64_t e;  /* routed experts */
  int64_t k;  /* experts per token */
  int64_t f;  /* routed expert FFN dim */
  int64_t fs; /* shared expert FFN dim, 0 = no shared expert */
} lsurge_moe_shape;

typedef struct {
  const void* x;       /* [t, d] bf16 */
  const void* w_r;     /* [d, e] bf16 */
  const float* bias;   /* [e] f32 router logit bias or NULL */
  const void* w_gate;  /* [e, d, f] bf16 */
  const void* w_up;    /* [e, d, f] bf16 */
  const void* w_down;  /* [e, f, d] bf16 */
  const void* ws_gate; /* [d, fs] bf16 or NULL */
  const void* ws_up;   /* [d, fs] bf16 or NULL */
  const void* ws_down; /* [fs, d] bf16 or NULL */
} lsurge_moe_params;

typedef struct {
  void* dx;        /* [t, d] bf16 */
  float* dw_r;     /* [d, e] f32 */
  float* dw_gate;  /* [e, d, f] f32 */
  float* dw_up;    /* [e, d, f] f32 */
  float* dw_down;  /* [e, f, d] f32 */
  float* dws_gate; /* [d, fs] f32 or NULL */
  float* dws_up;   /* [d, fs] f32 or NULL */
  float* dws_down; /* [fs, d] f32 or NULL */
  float* dweights; /* [t, k] f32 gradient of the routing weights (may be NULL) */
} lsurge_moe_grads;

/* Bytes of the `saved` buffer the forward fills and the backward reads (activations, layout, the weight gradients'
 * chunk table and W_r^T).  The FP8 forward also keeps its E4M3 x and h there and needs lsurge_moe_saved_bytes_fp8
 * (the bf16 layout is a prefix of it). */
size_t lsurge_moe_saved_bytes(const lsurge_moe_shape* s);
size_t lsurge_moe_saved_bytes_fp8(const lsurge_moe_shape* s);
/* Scratch bytes for forward and backward (not kept between calls). */
size_t lsurge_moe_fwd_workspace_bytes(const lsurge_moe_shape* s);
size_t lsurge_moe_bwd_workspace_bytes(const lsurge_moe_shape* s);

/* out: [t, d] bf16 = sum_j w[t,j] * expert_{sel[t,j]}(x[t]) + shared(x[t]) (f32 sum, one rounding). */
int lsurge_moe_fwd(const lsurge_moe_shape* s, const lsurge_moe_params* p, void* out, void* saved,
                   size_t saved_bytes, void* workspace, size_t workspace_bytes, lsurge_stream_t stream);
/* dy: [t, d] bf16 upstream gradient.  `saved` must come from lsurge_moe_fwd with the same s and p. */
int lsurge_moe_bwd(const lsurge_moe_shape* s, const lsurge_moe_params* p, const void* dy, const void* saved,
                   const lsurge_moe_grads* g, void* workspace, size_t workspace_bytes, lsurge_stream_t stream);

/* Views into `saved` (device pointers), for tests and the Python surface. */
typedef struct {
  float* logits;       /* [t, e] */
  int32_t* sel;        /* [t, k] */
  float* weights;      /* [t, k] */
  int32_t* group_sizes, *offsets, *block_off; /* [e] */
  int32_t* order, *pos, *slot;                /* [t*k] */
  int32_t* row_src;    /* [128*max_blocks] */
  int32_t* blk_expert, *blk_rows;             /* [max_blocks] */
  int32_t* num_blocks; /* [1] */
  void* h_gate;        /* [128*max_blocks, f] bf16 x.W_gate */
  void* h_up;          /* [128*max_blocks, f] bf16 x.W_up */
  void* h;             /* [128*max_blocks, f] bf16 silu(gate)*up */
  void* y_pad;         /* [128*max_blocks, d] bf16 expert outputs */
} lsurge_moe_saved_views;
int lsurge_moe_saved_layout(const lsurge_moe_shape* s, void* saved, lsurge_moe_saved_views* v);

/* ------------------------------------------------------------------------------------------------
 * FP8 variant of the expert GEMMs (OCP FP8 operands, f32 accumulation, v_mfma_f32_32x32x64_f8f6f4).
 * Current scaling: every tensor, or every group of one (an expert's weight matrix), is quantised with its
 * own scale taken just before the cast (1 when amax = 0); values are rounded to nearest even and saturated at
 * +-fmax; scale_inv = 1 / scale multiplies the GEMM's accumulator back.  Activations and weights are E4M3
 * (fmax 448) with scale = 448 / amax; gradients are E5M2 (fmax 57344) with scale = the largest power of two not
 * above 57344 / amax (Transformer Engine's force_pow_2_scales variant, so that a one-ulp change of a gradient's
 * amax moves the quantisation grid only at a binade; TE is not importable here, so parity with its recipe is
 * not checked).  This is the hybrid recipe of Transformer Engine's FP8
 * current scaling that the reference trains with through MaxText's `quantization=te_fp8_currentscaling`
 * (modal/te_run.py:95-99; TE and MaxText are third-party, and the reference's own MoE path has no FP8 entry
 * point, so these functions replace none of its interfaces).
 * ------------------------------------------------------------------------------------------------ */
#define LSURGE_FP8_E4M3 0
#define LSURGE_FP8_E5M2 1

/* x: `groups` consecutive [rows, cols] bf16 matrices -> q: the same shape in E4M3 bytes, or [cols, rows]
 * per group with transpose = 1 (rows, cols multiples of 16; untransposed: rows * cols a multiple of 16);
 * scale_inv: [groups] f32.  x and q 16-byte aligned. */
size_t lsurge_fp8_quantize_workspace_bytes(int64_t groups, int64_t rows, int64_t cols);
int lsurge_fp8_quantize(const void* x, int64_t groups, int64_t rows, int64_t cols, int transpose, void* q,
                        float* scale_inv, void* workspace, size_t workspace_bytes, lsurge_stream_t stream);

/* One [rows, cols] bf16 tensor (cols % 16 == 0) -> format (LSURGE_FP8_E4M3 / _E5M2) with one scale, written
 * row-wise to q [rows, cols] and / or transposed to qt [cols, ldqt] (ldqt >= rows rounded up to 64, a multiple
 * of 16; columns past rows hold zeros up to the next multiple of 16) -- the cast + transpose a training step
 * makes of an activation or gradient whose two GEMMs need it K-contiguous in both directions.  Either q or qt
 * may be null; all pointers 16-byte aligned; scale_inv [1] f32.  The scale follows the format's rule above:
 * 448 / amax for E4M3, the largest power of two not above 57344 / amax for E5M2. */
size_t lsurge_fp8_cast_workspace_bytes(void);
int lsurge_fp8_cast_transpose(const void* x, int64_t rows, int64_t cols, int format, void* q, void* qt,
                              int64_t ldqt, float* scale_inv, void* workspace, size_t workspace_bytes,
                              lsurge_stream_t stream);

/* lsurge_ragged_dot on FP8 operands: out[r] = (lhs_q[r] . rhs_q[e(r)]^T) * lhs_scale_inv[0] *
 * rhs_scale_inv[e(r)] for r < sum(group_sizes), 0 after.  lhs_q: [m, kdim] E4M3; rhs_q: [e, n, kdim] E4M3
 * (K contiguous, as lsurge_fp8_quantize with transpose = 1 makes it from [e, kdim, n]); scale_inv f32
 * device arrays [1] and [e]; out [m, n] bf16 or f32.  kdim % 16 == 0, n % 8 == 0.  Workspace:
 * lsurge_ragged_dot_workspace_bytes(m, e). */
int lsurge_ragged_dot_fp8(const void* lhs_q, const float* lhs_scale_inv, const void* rhs_q,
                          const float* rhs_scale_inv, const int32_t* group_sizes, int64_t m, int64_t kdim,
                          int64_t n, int64_t e, void* out, int out_dtype, void* workspace, size_t workspace_bytes,
                          lsurge_stream_t stream);

/* The layer's weights in E4M3, one buffer: gate, up [e, f, d], down [e, d, f] (K contiguous for the
 * forward), shared gate, up [fs, d], down [d, fs], the same codes again in the weights' own layout (K
 * contiguous for the backward's dgrads), then the f32 scale_inv of gate, up, down per expert and of the
 * three shared matrices.  Filled by lsurge_moe_fp8_quantize_weights from the bf16 weights of p (one scale
 * per expert and matrix); a caller whose weights do not change (serving) fills it once, a training step
 * after every weight update. */
size_t lsurge_moe_fp8_weights_bytes(const lsurge_moe_shape* s);
size_t lsurge_moe_fp8_quantize_weights_workspace_bytes(const lsurge_moe_shape* s);
int lsurge_moe_fp8_quantize_weights(const lsurge_moe_shape* s, const lsurge_moe_params* p, void* wq,
                                    size_t wq_bytes, void* workspace, size_t workspace_bytes,
                                    lsurge_stream_t stream);
/* lsurge_moe_fwd with every expert GEMM in FP8: x is quantised per tensor, h = silu(g) * u (bf16, kept in
 * `saved`) per tensor (routed and shared separately) before the down projections.  Router, layout and
 * combine are those of lsurge_moe_fwd.  `saved` (lsurge_moe_saved_bytes_fp8 bytes) starts with the bf16
 * layout, so lsurge_moe_bwd (bf16) runs on it too. */
size_t lsurge_moe_fwd_fp8_workspace_bytes(const lsurge_moe_shape* s);
int lsurge_moe_fwd_fp8(const lsurge_moe_shape* s, const lsurge_moe_params* p, const void* wq, size_t wq_bytes,
                       void* out, void* saved, size_t saved_bytes, void* workspace, size_t workspace_bytes,
                       lsurge_stream_t stream);
/* lsurge_moe_bwd with every expert GEMM in FP8, after lsurge_moe_fwd_fp8 on the same `saved` and weight
 * buffer (it reads the scales the forward saved).  Gradients are cast to E5M2 per tensor: the routed dY rows
 * and [dG | dU] over all routed rows, the shared expert's dY and [dG | dU] on their own.  dgrads: E5M2 x the
 * weights' E4M3 codes (each weight at its own scale); wgrads: the forward's E4M3 codes of h and x (same
 * scales) x the E5M2 gradients.  Combine, dispatch and router backward are those of lsurge_moe_bwd; the
 * gradients come out in the same buffers and dtypes.  p needs x and w_r (the bf16 expert weights are not
 * read). */
size_t lsurge_moe_bwd_fp8_workspace_bytes(const lsurge_moe_shape* s);
int lsurge_moe_bwd_fp8(const lsurge_moe_shape* s, const lsurge_moe_params* p, const void* wq, size_t wq_bytes,
                       const void* dy, const void* saved, const lsurge_moe_grads* g, void* workspace,
                       size_t workspace_bytes, lsurge_stream_t stream);

/* ------------------------------------------------------------------------------------------------
 * Causal depthwise Conv1D of the Gated DeltaNet block (memory-bound).
 * ------------------------------------------------------------------------------------------------ */

/* y[b,t,c] = sum_{j<k} w[j,c] * x[b, t-(k-1)+j, c] (zero before t = 0), f32 accumulation, one rounding.
 * x, y: [b, t, c] bf16; w: [k, c] bf16 (the kernel [k, 1, c] of nnx.Conv).  c % 8 == 0, 1 <= k <= 8.
 * Replaces fast_conv._fast_call (modal/fast_conv.py:14-31), the stand-in for
 * nnx.Conv(padding="CAUSAL", feature_group_count=c). */
int lsurge_causal_conv1d(const void* x, const void* w, int64_t b, int64_t t, int64_t c, int64_t k, void* y,
                         lsurge_stream_t stream);
/* Backward of lsurge_causal_conv1d for upstream dy [b, t, c] bf16:
 *   dx[b,t,c] = sum_j w[j,c] * dy[b, t+(k-1)-j, c] (bf16),  dw[j,c] = sum_{b,t} dy[b,t,c] * x[b, t-(k-1)+j, c]
 * (f32, summed in a fixed order).  Replaces the XLA autodiff of fast_conv._fast_call (modal/fast_conv.py:27-30). */
size_t lsurge_causal_conv1d_bwd_workspace_bytes(int64_t b, int64_t t, int64_t c, int64_t k);
int lsurge_causal_conv1d_bwd(const void* x, const void* w, const void* dy, int64_t b, int64_t t, int64_t c, int64_t k,
                             void* dx, float* dw, void* workspace, size_t workspace_bytes, lsurge_stream_t stream);

/* ------------------------------------------------------------------------------------------------
 * Chunked gated delta rule of the Gated DeltaNet block (forward).
 * ------------------------------------------------------------------------------------------------ */

/* Per sequence and head, state S [dk, dv]: S_t = exp(g_t) (I - beta_t k_t k_t^T) S_{t-1} + beta_t k_t v_t^T,
 * o_t = S_t^T q_t / sqrt(dk), computed in 64-token chunks (WY form) with the reference's bf16 rounding points
 * (q * scale, k beta, v beta, and the chunk-local u and w) and f32 arithmetic otherwise.
 * q, k: [b, t, h, dk] bf16; v: [b, t, h, dv] bf16; g: [b, t, h] f32 (log decay); beta: [b, t, h] bf16;
 * h0: [b, h, dk, dv] f32 initial state or NULL; o: [b, t, h, dv] bf16; h_out: [b, h, dk, dv] f32 or NULL.
 * dk = dv = 128.  Replaces fast_chunk_gated_delta_rule (modal/gdn_fast.py:37-113) without qk-norm or context
 * parallelism. */
size_t lsurge_gdn_chunked_workspace_bytes(int64_t b, int64_t t, int64_t h, int64_t dk, int64_t dv);
int lsurge_gdn_chunked_fwd(const void* q, const void* k, const void* v, const float* g, const void* beta, int64_t b,
                           int64_t t, int64_t h, int64_t dk, int64_t dv, const float* h0, void* o, float* h_out,
                           void* workspace, size_t workspace_bytes, lsurge_stream_t stream);

/* Backward of lsurge_gdn_chunked_fwd for upstream do [b, t, h, dv] bf16 and dh_final [b, h, dk, dv] f32 (the final
 * state's gradient, or NULL for 0): dq, dk, dv [b, t, h, 128] bf16, dg, dbeta [b, t, h] f32 and dh0 [b, h, dk, dv] f32
 * (NULL: not written).  h0 is the forward's initial state (NULL = 0).  The forward is recomputed from the inputs.
 * The gradients are those XLA's autodiff gives for the reference's chunked form (the bf16 rounding points taken with
 * derivative 1, as for a dtype cast), computed in f32.  Replaces the training backward of fast_chunk_gated_delta_rule
 * (modal/gdn_fast.py:37-113; installed for training at lightning/train_stage1.py:67-69). */
size_t lsurge_gdn_chunked_bwd_workspace_bytes(int64_t b, int64_t t, int64_t h, int64_t dk, int64_t dv);
int lsurge_gdn_chunked_bwd(const void* q, const void* k, const void* v, const float* g, const void* beta, int64_t b,
                           int64_t t, int64_t h, int64_t dk, int64_t dv, const float* h0, const void* dout,
                           const float* dh_final, void* dq, void* dk_out, void* dv_out, float* dg, float* dbeta,
                           float* dh0, void* workspace, size_t workspace_bytes, lsurge_stream_t stream);

/* The same forward and backward split at the residuals, as jax.vjp splits fast_chunk_gated_delta_rule when XLA's
 * autodiff trains through it (modal/gdn_fast.py:37-113; lightning/train_stage1.py:67-69).  The training forward also
 * keeps the chunk products and the state entering every chunk in `saved` (lsurge_gdn_chunked_saved_bytes: about
 * 2.25 KiB per token and head at dk = dv = 128), and the backward starts from them instead of recomputing the forward,
 * with its own scratch `workspace` (lsurge_gdn_chunked_bwd_saved_workspace_bytes).  o, h_out and every gradient are
 * bitwise those of lsurge_gdn_chunked_fwd / lsurge_gdn_chunked_bwd.  The backward only reads `saved`.  Arguments
 * otherwise as above (the backward needs neither g nor h0). */
size_t lsurge_gdn_chunked_saved_bytes(int64_t b, int64_t t, int64_t h, int64_t dk, int64_t dv);
int lsurge_gdn_chunked_fwd_save(const void* q, const void* k, const void* v, const float* g, const void* beta,
                                int64_t b, int64_t t, int64_t h, int64_t dk, int64_t dv, const float* h0, void* o,
                                float* h_out, void* saved, size_t saved_bytes, lsurge_stream_t stream);
size_t lsurge_gdn_chunked_bwd_saved_workspace_bytes(int64_t b, int64_t t, int64_t h, int64_t dk, int64_t dv);
int lsurge_gdn_chunked_bwd_saved(const void* q, const void* k, const void* v, const void* beta, int64_t b, int64_t t,
                                 int64_t h, int64_t dk, int64_t dv, const void* dout, const float* dh_final, void* dq,
                                 void* dk_out, void* dv_out, float* dg, float* dbeta, float* dh0, const void* saved,
                                 size_t saved_bytes, void* workspace, size_t workspace_bytes, lsurge_stream_t stream);

/* Row-wise l2 normalisation of the GDN block's query and key heads, the use_qk_norm_in_gdn branch of
 * fast_chunk_gated_delta_rule (modal/gdn_fast.py:43-46, MaxText's l2norm(x, dim=-1, eps=1e-6)):
 * y = x * rsqrt(sum(x^2) + eps) per row of dim elements, x and y bf16 [rows, dim], f32 arithmetic; rnorm [rows] f32
 * receives rsqrt(sum(x^2) + eps) for the backward (NULL: not written).  rows < 2^31, dim a multiple of 8 in
 * [8, 512], x and y 16-byte aligned. */
int lsurge_l2norm_rows(const void* x, int64_t rows, int64_t dim, float eps, void* y, float* rnorm,
                       lsurge_stream_t stream);
/* Its backward: dx = r dy - r^3 x (x . dy) per row (r = rnorm of the forward), x, dy and dx bf16 [rows, dim]. */
int lsurge_l2norm_rows_bwd(const void* x, const void* dy, const float* rnorm, int64_t rows, int64_t dim, void* dx,
                           lsurge_stream_t stream);

/* ------------------------------------------------------------------------------------------------
 * Test hooks (no reference counterpart): failure injection for the error paths.
 * ------------------------------------------------------------------------------------------------ */
/* Arm a host-side failure: the nth launch (counting from 1) of the kernel with profiler id kernel_id
 * (lsurge_prof_kernel_name) returns LSURGE_ERR_LAUNCH without launching; nth = 0 disarms.  Process-wide. */
int lsurge_test_fail_launch(int kernel_id, int nth);
/* 1 when every helper stream of the current device has finished its work (hipStreamQuery), 0 when one is
 * still busy, -1 when no helper stream exists yet. */
int lsurge_test_helpers_idle(void);

/* ------------------------------------------------------------------------------------------------
 * Live per-kernel timing with HIP events on the launch stream (used by the benchmark).
 * ------------------------------------------------------------------------------------------------ */
int lsurge_prof_enable(int on);            /* on=1: create events, start recording; 0: stop */
int lsurge_prof_collect(void);             /* after a device sync: fold recorded pairs into totals */
int lsurge_prof_kernel_count(void);
const char* lsurge_prof_kernel_name(int id);
int lsurge_prof_read(int id, double* total_ms, int64_t* launches);
void lsurge_prof_reset(void);

/* Calibration (no reference counterpart; used by the benchmark): the matrix cores' sustained bf16 rate.  1024
 * workgroups of 4 waves each issue iters x 64 v_mfma_f32_32x32x16_bf16 (32768 flops each) on register-resident
 * operands -- pseudo-random bf16 values, or zeros with zero_operands = 1 -- and write one float per lane to out
 * (lsurge_mfma_rate_probe_out_floats() floats).  Time it with events on the stream: iters x 2^33 flops divided by the
 * time is the rate the chip sustains on such data (its power limit holds random operands below the
 * datasheet peak).  iters in [1, 2^20]. */
size_t lsurge_mfma_rate_probe_out_floats(void);
int lsurge_mfma_rate_probe(int zero_operands, int iters, float* out, lsurge_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* LEWI_SURGE_H_ */
