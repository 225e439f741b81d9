// Internal launchers shared by the translation units of the library (not part of the C ABI): the layer
// (moe_layer.hip) composes them; layout.hip, permute.hip and gemm.hip define them.
#pragma once
#include "common.h"

namespace lsurge {

// ---- router (router.hip): lsurge_router_topk with an optional event recorded right after the logits kernel
// after_logits (optional): a hipEvent recorded on the stream right after the logits kernel of the split path (after
// the fused kernel on the fused path), so a caller can start independent work beside the selection
int router_topk_impl(const void* x, const void* w_r, const float* bias, int64_t t, int64_t d, int64_t e, int64_t k,
                     float* logits, int32_t* sel, float* weights, hipStream_t s, hipEvent_t after_logits,
                     int32_t* hist = nullptr);
// Shapes the workgroup-fused router takes (logits, top-k, softmax and the per-64-token expert histograms in one
// kernel): e in {32, 64, 128}, k <= 8, d a multiple of 64.  router_topk_impl uses it when given hist
// ([ceil(t / 64)][e] int32, the layout's chunk counts for chunks of 64 tokens).
bool router_fused_ok(int64_t d, int64_t e, int64_t k);

// ---- routing layout (layout.hip)
// Device-side outputs of a weight-gradient chunk table (the entries of wgrad_chunk_table_ints; see WgradChunks) and
// the plan values it is written with: R rows per chunk, the bounds, and the extra expert's rows (x_rows < 0: none)
// from row x_row0.  c_expert == nullptr: no table.
struct ChunkTableOut {
  int32_t *c_expert = nullptr, *c_row0 = nullptr, *c_rows = nullptr, *c_part = nullptr, *e_pbase = nullptr,
          *e_nparts = nullptr, *split_list = nullptr, *num_chunks = nullptr, *num_split = nullptr;
  int R = 0, max_chunks = 0, max_parts = 0, x_rows = -1, x_row0 = 0;
};
// Optional 256-row tile table of the layer's grouped GEMMs, written by the layout's scan kernel: expert e gets
// ceil(gs[e] / 256) tiles, each two consecutive 128-row blocks of its own (the last may hold one block); TS tiles of
// a shared expert carried as expert E follow (rows P + 256 j of its T rows; row_src of those rows = t k); entries up
// to TB + TS past them are empty.  num_tiles[0] = routed tiles, num_tiles[1] = all.
struct LayoutTiles {
  int32_t* t_expert = nullptr;
  int32_t* t_rows = nullptr;
  int32_t* t_row0 = nullptr;
  int32_t* num_tiles = nullptr;
  int TB = 0, TS = 0;
  int64_t P = 0, T = 0;
  int k = 1;
  // optional: the weight gradients' chunk table over the padded layout (expert e's rows from 128 block_off[e]),
  // written by the layout too, so the backward launches no kernel for it; needs E + 1 <= 1024
  ChunkTableOut chunks;
};
// Optional per-chunk expert histograms made by the caller (the fused router): hist [nchunk][E] for chunks of
// waves x 64 consecutive slots (overwritten with the per-expert chunk bases); the layout then skips its own.
struct LayoutChunks {
  int32_t* hist = nullptr;
  int waves = 0;
};
int build_layout_impl(const int32_t* flat, int64_t M, int64_t E, int32_t* gs, int32_t* offsets, int32_t* block_off,
                      int32_t* order, int32_t* pos, int32_t* slot, int32_t* row_src, int32_t* blk_expert,
                      int32_t* blk_rows, int32_t* num_blocks, void* ws, size_t ws_bytes, hipStream_t s,
                      const LayoutTiles& tiles = LayoutTiles(), const LayoutChunks& pre = LayoutChunks());

// ---- row movement (permute.hip)
int launch_dispatch_pad(const void* x, int64_t d, int k, const int32_t* row_src, const int32_t* num_blocks,
                        int64_t max_rows, void* xp, hipStream_t s);
int launch_combine_pad(const void* yp, int64_t d, int k, const int32_t* slot, const float* w, int64_t n,
                       const void* add, void* out, int out_dtype, hipStream_t s);
// dlog (optional, needs sel and dl): also the dense bf16 d(logits) [n, E] of the router's weight gradient.
// FP8 backward (dyq set): the dY rows as E5M2 codes with scale[0] (launch_dy_scale) in dyq [rows, d]; the rows of
// real blocks (nblocks[0] of 128) are written, dyp is scratch.
struct CombineFp8 {
  void* dyq = nullptr;
  const float* scale = nullptr;
  const int32_t* nblocks = nullptr;
};
int launch_combine_bwd_pad(const void* yp, int64_t rows, const int32_t* slot, const float* w, int64_t n, int k,
                           int64_t d, const void* g, void* dyp, float* dw, float* dl, hipStream_t s,
                           void* gcopy = nullptr, const int32_t* sel = nullptr, void* dlog = nullptr, int E = 0,
                           const CombineFp8& f8 = CombineFp8(), float* wpad = nullptr);
// The E5M2 scale (power of two) of the dY rows w[t, j] g[t] (bf16-rounded) from g [n, d] and w [n, k] alone: amax
// partials (dy_rows_amax_parts() floats at partial), then scale[0] and sinv[0] = 1 / scale; also clears
// zero[0 .. nzero).
int dy_rows_amax_parts();
int launch_dy_scale(const void* g, const float* w, int64_t n, int64_t d, int k, float* partial, float* scale,
                    float* sinv, hipStream_t s, uint32_t* zero = nullptr, int nzero = 0);
int launch_dispatch_bwd_pad(const void* dxp, int64_t d, int k, const int32_t* slot, int64_t n, const float* dl,
                            const int32_t* sel, const void* w_rT, const void* add, void* dx, hipStream_t s);
int launch_transpose_bf16(const void* a, int R, int C, void* at, hipStream_t s);
int launch_scatter_dlogits(const float* dl, const int32_t* sel, int64_t T, int E, int k, void* dlog, hipStream_t s);

// ---- grouped GEMMs (gemm.hip).  et: element type of the 16-bit operands (LSURGE_BF16, or LSURGE_F16 for the plain-store
// row GEMMs and the weight gradients of the ragged_dot entry points).
// Row tiles: the padded 128-row expert blocks (blk_expert set) or a dense matrix of dense_rows rows.
struct GemmBlocks {
  const int32_t* blk_expert;
  const int32_t* blk_rows;
  const int32_t* blk_row0;   // first row of block b (nullptr: tile_rows b)
  const int32_t* num_blocks;
  int max_blocks;
  int64_t dense_rows;        // used when blk_expert == nullptr
  int tile_rows = 128;       // rows per tile: 128 (4-wave kernel) or 256 (8-wave ping-pong kernel; a table of
                             // 256-row tiles, or dense rows)
};
// Optional row gather of the A operand: row r of the rows operand (a tile row of gemm_rows, a reduction row of an
// expert in gemm_wgrad) reads A[rows[r] / div], indexed by padded row (negative index: zero row).
struct RowGather {
  const int32_t* rows = nullptr;
  int div = 1;
  int64_t nrows = 0;  // rows of the gathered-from matrix
  // gemm_wgrad_chunked only: gather B instead of A, each row times scale[r] (padded row; the extra expert's rows: 1)
  // rounded to bf16 -- the persistent kernel only
  bool on_b = false;
  const float* scale = nullptr;
};
// One extra expert id whose weights live in matrices of their own (the layer's shared expert, carried along the
// routed experts as expert E): its tiles read B / B2 here instead of the routed weight stack.
struct ExtraExpert {
  int expert = -1;
  const void* B = nullptr;
  const void* B2 = nullptr;
};
int gemm_rows_kn(int kid, const GemmBlocks& g, const void* A, int64_t lda, const void* B, int64_t ldb,
                 int64_t b_estride, int64_t K, int64_t N, void* C, int64_t ldc, hipStream_t s, bool out_f32 = false,
                 const ExtraExpert& xe = ExtraExpert(), int et = LSURGE_BF16);
int gemm_rows_swiglu_fwd(int kid, const GemmBlocks& g, const void* A, int64_t lda, const void* Bg, const void* Bu,
                         int64_t ldb, int64_t b_estride, int64_t K, int64_t N, void* H, void* Gs, void* Us,
                         int64_t ldh, hipStream_t s, const RowGather& gather = RowGather(),
                         const ExtraExpert& xe = ExtraExpert());
int gemm_rows_nk(int kid, const GemmBlocks& g, const void* A, int64_t lda, const void* B, const void* B2,
                 int64_t k_split, int64_t ldb, int64_t b_estride, int64_t K, int64_t N, void* C, int64_t ldc,
                 bool swiglu_bwd, const void* Gs, const void* Us, int64_t ldg, hipStream_t s, bool out_f32 = false,
                 const ExtraExpert& xe = ExtraExpert(), int et = LSURGE_BF16, const RowGather& gather = RowGather(),
                 const float* row_scale = nullptr);
// FP8 row GEMM, both operands K-contiguous (B_e stored [N, K], E4M3; A E4M3, or E5M2 with a_e5m2); byte pitches;
// epilogue F8_STORE, F8_SWIGLU_FWD or F8_SWIGLU_BWD; k_split: B2 for k >= k_split (multiple of 64); see gemm.hip
enum F8Epi { F8_STORE = 0, F8_SWIGLU_FWD = 1, F8_SWIGLU_BWD = 2 };
int gemm_rows_f8(int kid, const GemmBlocks& g, const void* A, int64_t lda, const float* a_sinv, const void* B,
                 const void* B2, int64_t ldb, int64_t b_estride, const float* b_sinv, const float* b2_sinv, int64_t K,
                 int64_t N, void* C, int64_t ldc, bool out_f32, int epi, void* Gs, void* Us, uint32_t* amax,
                 hipStream_t s, const RowGather& gather = RowGather(), int64_t k_split = 0, bool a_e5m2 = false);
size_t wgrad_workspace_bytes(int E, int64_t I, int64_t N, int S);
int gemm_wgrad(int kid, int E, const int32_t* e_row0, int row0_mult, const int32_t* e_rows, int64_t dense_rows,
               int64_t max_rows, const void* A, int64_t lda, const void* B, int64_t ldb, int64_t I, int64_t N,
               float* C, float* C2, int64_t n_split, int64_t ldc, int64_t c_estride, int S, void* ws, size_t ws_bytes,
               hipStream_t s, const RowGather& gather = RowGather(), int et = LSURGE_BF16);

// Chunked routed weight gradient: every expert's rows cut into chunks of at most R rows (see WgradArgs), so a
// hot expert spreads over many workgroups; split experts are reduced from f32 partial slots in chunk order.
struct WgradChunkPlan {
  int R = 0;           // rows per chunk
  int max_chunks = 0;  // bound on the chunk count
  int max_parts = 0;   // bound on the partial slots
};
struct WgradChunks {
  const int32_t *c_expert, *c_row0, *c_rows, *c_part, *num_chunks, *e_pbase, *e_nparts, *split_list, *num_split;
  int max_chunks, max_parts;
};
WgradChunkPlan wgrad_chunk_plan(int64_t M, int64_t E);
// A dense weight gradient C[I, N] = A^T B over M rows as the chunk table's only (extra) expert: ceil(256 / tiles of
// 256 x 256) chunks of equal rows (at most 16, at least 1024 rows each), so the chunks' tiles fill the GPU once.
WgradChunkPlan wgrad_chunk_plan_dense(int64_t M, int64_t I, int64_t N);
size_t wgrad_chunk_table_ints(const WgradChunkPlan& p, int64_t E);
// builds the table (in `table`, wgrad_chunk_table_ints entries) from device group sizes and block offsets
// Expert e's rows start at row0_mult block_off[e] (128 for the padded layout, 1 for a ragged one).  Extra expert
// of the chunk table (id E, after the routed ones): x_rows rows from row x_row0 (x_rows < 0: none); its gradient
// goes to C / C2 of an ExtraOut.  E = 0 with an extra expert is a dense weight gradient (gs, block_off unused).
int build_wgrad_chunks(const int32_t* gs, const int32_t* block_off, int E, const WgradChunkPlan& p, int32_t* table,
                       WgradChunks* ch, hipStream_t s, int64_t x_rows = -1, int64_t x_row0 = 0,
                       int row0_mult = LSURGE_BLOCK_ROWS);
// The table's entries inside `table` for a plan and an extra expert, and the view the GEMMs read, without a launch
// (for a table another kernel writes, such as the layout's)
ChunkTableOut chunk_table_out(int32_t* table, int E, const WgradChunkPlan& p, int64_t x_rows = -1,
                              int64_t x_row0 = 0);
WgradChunks chunk_table_view(const ChunkTableOut& o);
struct ExtraOut {
  int expert = -1;
  float* C = nullptr;
  float* C2 = nullptr;
};
size_t wgrad_chunked_workspace_bytes(const WgradChunkPlan& p, int64_t I, int64_t N);
int gemm_wgrad_chunked(int kid, const WgradChunks& ch, int E, int64_t max_rows, const void* A, int64_t lda,
                       const void* B, int64_t ldb, int64_t I, int64_t N, float* C, float* C2, int64_t n_split,
                       int64_t ldc, int64_t c_estride, void* part, size_t part_bytes, hipStream_t s,
                       const RowGather& gather = RowGather(), const ExtraOut& xo = ExtraOut(), int et = LSURGE_BF16);

// FP8 weight gradients (E4M3 activations x E5M2 gradients) from the row-major FP8 tensors: A [rows, lda] and B
// [rows, ldb] bytes (A optionally gathered through row_src, as gemm_wgrad_chunked), C = A^T B a_sinv[0] b_sinv[0].
// Chunked: the routed experts over a chunk table; dense: one matrix over `rows` rows split S ways (f32 partials in ws,
// wgrad_workspace_bytes(1, I, N, S)).  I, N, lda, ldb multiples of 16.
int gemm_wgrad_f8_chunked(int kid, const WgradChunks& ch, int E, int64_t max_rows, const void* A, int64_t lda,
                          const float* a_sinv, const void* B, int64_t ldb, const float* b_sinv, int64_t I, int64_t N,
                          float* C, float* C2, int64_t n_split, int64_t ldc, int64_t c_estride, void* part,
                          size_t part_bytes, hipStream_t s, const RowGather& gather = RowGather());
int gemm_wgrad_f8_dense(int kid, int64_t rows, const void* A, int64_t lda, const float* a_sinv, const void* B,
                        int64_t ldb, const float* b_sinv, int64_t I, int64_t N, float* C, float* C2, int64_t n_split,
                        int64_t ldc, int S, void* ws, size_t ws_bytes, hipStream_t s);

// ---- FP8 quantisation (fp8.hip), current scaling to OCP E4M3 (and E5M2 for gradients)
size_t fp8_partial_bytes(int64_t groups);  // amax partials of fp8_quantize_impl
// groups of [rows, cols] bf16 -> q (transpose: [cols, rows] per group), sinv[g] = 1 / scale; zero[0 .. nzero) is
// cleared by the cast kernel (untransposed only), for slots a later kernel fills by atomic max.  q_nt (transposed
// casts only): the same codes untransposed as well.  scale_out (untransposed only): the scale of each group.
int fp8_quantize_impl(const void* x, int64_t groups, int64_t rows, int64_t cols, bool transpose, void* q, float* sinv,
                      float* partial, hipStream_t s, uint32_t* zero = nullptr, int nzero = 0, void* q_nt = nullptr,
                      float* scale_out = nullptr);
// cast of n bf16 values with the amax in *amax_bits (float bits); nrows (optional): only the first
// nrows[0] * row_elems values; scale_out (optional) receives the scale
int fp8_cast_with_amax(const void* x, int64_t n, const uint32_t* amax_bits, void* q, float* sinv,
                       const int32_t* nrows, int64_t row_elems, hipStream_t s, float* scale_out = nullptr);
// Row-layout casts of the backward.  Rows r < min(rows, nrows[0] nmul) (nrows optional: a block count and its rows
// per block, or a row count and 1) with row_src[r] >= 0 (row_src optional) are data, read from x row r, or from x row row_src[r] / kdiv when gathered; the others are zeros.
// fp8_amax_rows writes one amax partial per workgroup into partial (fp8_rows_partial_bytes) and returns their count
// (negative: an error code); its first workgroup also clears zero[0 .. nzero).
size_t fp8_rows_partial_bytes();
// amax partials of n bf16 values (n % 8 == 0, fp8_partial_bytes(1)); returns their count (negative: an error code)
int fp8_amax(const void* x, int64_t n, float* partial, hipStream_t s);
// E5M2 cast (power-of-two scale) of n bf16 values with the amax of nparts partials (or nparts = 1 and an amax slot;
// nparts < 0: amax[0] is the scale itself, and sinv may be null); nrows (optional): only the first
// nrows[0] * row_elems values
int fp8_cast_e5m2(const void* x, int64_t n, const float* amax, int nparts, void* q, float* sinv, const int32_t* nrows,
                  int64_t row_elems, hipStream_t s, uint32_t* zero = nullptr, int nzero = 0);
int fp8_amax_rows(const void* x, int64_t rows, int64_t cols, const int32_t* nrows, int nmul, const int32_t* row_src,
                  int kdiv, bool gather, float* partial, hipStream_t s, uint32_t* zero = nullptr, int nzero = 0);
// cast to E4M3 or E5M2 (e5m2) into a row-wise copy qr [rows, cols] and / or a transposed copy qt [cols, ldq]; the
// scale comes from nparts > 0 amax partials at src, from an amax slot (nparts == 0: float bits), or is src[0]
// (nparts < 0).  sinv[0] receives 1 / scale and scale_out[0] (optional) the scale.
int fp8_cast_rows(const void* x, int64_t rows, int64_t cols, const int32_t* nrows, int nmul, const int32_t* row_src,
                  int kdiv, bool gather, const float* src, int nparts, bool e5m2, void* qr, void* qt, int64_t ldq,
                  float* sinv, float* scale_out, hipStream_t s);

}  // namespace lsurge
