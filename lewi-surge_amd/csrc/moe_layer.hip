// Whole MoE layer, forward and gather-only backward, as one stream-ordered sequence of the hot-path kernels.
//
// Forward:  router top-k -> routing layout -> gate/up grouped GEMM over 128-row expert blocks whose rows are
//           gathered from x (the dispatch, fused into the GEMM's operand load) with the SiLU*mul epilogue -> down
//           grouped GEMM -> weighted combine (+ shared expert).
// Shared expert.  Its forward runs as dense (E = 1) GEMMs on a helper stream, where it overlaps the router and the
// layout (it depends on x only).  When its FFN width equals the routed one (fs == f) its rows (every token once)
// sit right after the routed block bound in the padded row space, and in the backward it rides along the routed
// experts as expert E: every grouped GEMM covers routed and shared rows in one launch (tiles of expert E read the
// shared weights) and its weight gradients join the routed chunk table.  Otherwise its backward is dense GEMMs
// of its own on a helper stream.
// Backward: fused combine backward (dY rows, d(routing weights), d(router logits)) -> down dgrad with the
//           SwiGLU backward epilogue -> down wgrad -> gate/up dgrad -> gate/up wgrad -> shared expert ->
//           router wgrad -> dispatch backward (gather-reduce, plus the router and shared-expert dx terms).
// No scatter-add anywhere: every row written by a kernel has exactly one writer.
//
// The reference composes these from MaxText RoutedMoE (third-party) with the patches of modal/moe_permute.py
// (dispatch/combine, 270-312) and modal/padded_gmm.py (ragged_dot, 45-69); the call order mirrors
// moe_permute.moe_block (modal/moe_permute.py:348-353) with a SwiGLU expert_fn.
#include <cstring>

#include "launchers.h"

namespace {

constexpr int BLK = LSURGE_BLOCK_ROWS;

// Bump allocator over a caller buffer, 256-byte aligned pieces.
struct Carve {
  char* base;
  size_t off = 0;
  explicit Carve(void* b) : base((char*)b) {}
  template <class T> T* take(size_t count) {
    off = (off + 255) & ~(size_t)255;
    T* p = base ? (T*)(base + off) : nullptr;
    off += sizeof(T) * count;
    return p;
  }
};

struct Dims {
  int64_t T, d, E, k, f, fs, M, MB, P;
  bool merged;      // shared expert carried as expert E of the grouped GEMMs (fs == f)
  int64_t SB;       // its blocks (ceil(T / 128)), after the routed block bound MB
  int64_t PT;       // padded rows including them
  int64_t TB, TS;   // 256-row tiles: bound on the routed ones, the shared expert's (merged only)
};

Dims dims_of(const lsurge_moe_shape* s) {
  Dims q;
  q.T = s->t; q.d = s->d; q.E = s->e; q.k = s->k; q.f = s->f; q.fs = s->fs;
  q.M = q.T * q.k;
  q.MB = lsurge_max_blocks(q.M, q.E);
  q.P = q.MB * BLK;
  q.merged = q.fs > 0 && q.fs == q.f;
  q.SB = q.merged ? (q.T + BLK - 1) / BLK : 0;
  q.PT = (q.MB + q.SB) * BLK;
  // expert e has ceil(gs[e] / 256) tiles, and sum_e ceil(gs[e] / 256) <= ceil(M / 256) + E
  q.TB = (q.M + 2 * BLK - 1) / (2 * BLK) + q.E;
  q.TS = q.merged ? (q.T + 2 * BLK - 1) / (2 * BLK) : 0;
  return q;
}

struct Saved {
  float* logits;
  int32_t *sel;
  float* weights;
  int32_t *gs, *offsets, *block_off, *order, *pos, *slot, *row_src, *blk_expert, *blk_rows, *num_blocks;
  // 256-row tile table of the grouped GEMMs: routed tiles (two consecutive blocks of one expert), then those of a
  // merged shared expert; num_tiles[0] counts the routed ones, num_tiles[1] all
  int32_t *t_expert, *t_rows, *t_row0, *num_tiles;
  bf16_t *g, *u, *h, *y_pad;
  bf16_t *sg, *su, *sh, *sy;  // shared expert run on its own: gate, up, h, output
  bf16_t* w_rT;               // W_r^T [E, d]: the dispatch backward's router dx term, made by the forward off the
                              // critical stream
  int32_t* chunk_tab;         // the bf16 backward's chunk table of the routed weight gradients (routed_chunk_plan),
                              // written by the layout of either forward
  // FP8 forward: x [T, d], routed h [P, f] (padded rows) and shared h [T, fs] in E4M3, and their scale_inv, the
  // operands the FP8 backward's weight gradients read again.  Carved after the bf16 layout and only for the FP8
  // path (null otherwise), so a bf16 buffer is a prefix of an FP8 one.
  uint8_t *xq, *hq, *shq;
  float* f8_sinv;
};

// chunk table of the routed weight gradients (a merged shared expert as the extra expert E) and its partial slots
lsurge::WgradChunkPlan routed_chunk_plan(const Dims& q) {
  return q.merged ? lsurge::wgrad_chunk_plan(q.M + q.T, q.E + 1) : lsurge::wgrad_chunk_plan(q.M, q.E);
}

size_t carve_saved(const Dims& q, void* base, Saved* sv, bool fp8) {
  Carve c(base);
  sv->logits = c.take<float>(q.T * q.E);
  sv->sel = c.take<int32_t>(q.M);
  sv->weights = c.take<float>(q.M);
  sv->gs = c.take<int32_t>(q.E);
  sv->offsets = c.take<int32_t>(q.E);
  sv->block_off = c.take<int32_t>(q.E);
  sv->order = c.take<int32_t>(q.M);
  sv->pos = c.take<int32_t>(q.M);
  sv->slot = c.take<int32_t>(q.M);
  sv->row_src = c.take<int32_t>(q.PT);
  sv->blk_expert = c.take<int32_t>(q.MB);
  sv->blk_rows = c.take<int32_t>(q.MB);
  sv->num_blocks = c.take<int32_t>(4);
  sv->t_expert = c.take<int32_t>(q.TB + q.TS);
  sv->t_rows = c.take<int32_t>(q.TB + q.TS);
  sv->t_row0 = c.take<int32_t>(q.TB + q.TS);
  sv->num_tiles = c.take<int32_t>(4);
  sv->g = c.take<bf16_t>(q.PT * q.f);
  sv->u = c.take<bf16_t>(q.PT * q.f);
  sv->h = c.take<bf16_t>(q.PT * q.f);
  sv->y_pad = c.take<bf16_t>(q.PT * q.d);
  const int64_t own = (q.fs && !q.merged) ? q.T : 0;  // rows of the separately run shared expert
  sv->sg = c.take<bf16_t>(own * q.fs);
  sv->su = c.take<bf16_t>(own * q.fs);
  sv->sh = c.take<bf16_t>(own * q.fs);
  sv->sy = c.take<bf16_t>(own * q.d);
  sv->w_rT = c.take<bf16_t>(q.E * q.d);
  sv->chunk_tab = c.take<int32_t>(lsurge::wgrad_chunk_table_ints(routed_chunk_plan(q), q.E));
  if (fp8) {
    sv->xq = c.take<uint8_t>(q.T * q.d);
    sv->hq = c.take<uint8_t>(q.P * q.f);
    sv->shq = c.take<uint8_t>(q.T * q.fs);
    sv->f8_sinv = c.take<float>(4);
  } else {
    sv->xq = sv->hq = sv->shq = nullptr;
    sv->f8_sinv = nullptr;
  }
  return c.off + 256;
}

// split count for a dense (one-expert) weight gradient: enough workgroups to fill 256 CUs
int dense_splits(int64_t rows, int64_t I, int64_t N) {
  const int64_t tiles = ((I + 127) / 128) * ((N + 127) / 128);
  int64_t S = (512 + tiles - 1) / tiles;
  S = std::min<int64_t>(S, 16);
  S = std::min<int64_t>(S, std::max<int64_t>(1, rows / 256));
  return (int)std::max<int64_t>(1, S);
}

struct BwdWs {
  bf16_t *dy_pad, *dgu, *dx_pad, *sdgu, *sdx, *dlog;
  float* dl;
  float* dweights;
  float* wpad;        // routing weight of each padded row (the down GEMMs scale by it instead of reading dY_pad)
  void* part;         // chunk partials of a shared expert's own dense weight gradients
  size_t part_bytes;
  int32_t* dense_tab;  // their chunk table (the shared expert as the only, extra expert of a dense table)
  void* part_r;       // split-K partials of the router weight gradient (another stream)
  size_t part_r_bytes;
  lsurge::WgradChunkPlan cplan;  // chunk table of the routed weight gradients and the partials of split experts
  int32_t* chunk_tab;            // the FP8 backward's chunk table (bf16: the forward's, in the saved buffer)
  void* part_dn;      // down-projection weight gradient (helper stream)
  size_t part_dn_bytes;
  void* part_gu;      // gate/up weight gradient (caller's stream)
  size_t part_gu_bytes;
};

size_t carve_bwd(const Dims& q, void* base, BwdWs* w) {
  Carve c(base);
  w->dy_pad = c.take<bf16_t>(q.PT * q.d);
  w->dgu = c.take<bf16_t>(q.PT * 2 * q.f);
  w->dx_pad = c.take<bf16_t>(q.PT * q.d);
  const int64_t own = (q.fs && !q.merged) ? q.T : 0;
  w->sdgu = c.take<bf16_t>(own * 2 * q.fs);
  w->sdx = c.take<bf16_t>(own * q.d);
  w->dlog = c.take<bf16_t>(q.T * q.E);
  w->dl = c.take<float>(q.M);
  w->dweights = c.take<float>(q.M);
  w->wpad = c.take<float>(q.PT);
  size_t part = 0, tab = 0;
  if (q.fs && !q.merged) {
    const lsurge::WgradChunkPlan pg = lsurge::wgrad_chunk_plan_dense(q.T, q.d, 2 * q.fs);
    const lsurge::WgradChunkPlan pd = lsurge::wgrad_chunk_plan_dense(q.T, q.fs, q.d);
    part = std::max(lsurge::wgrad_chunked_workspace_bytes(pg, q.d, 2 * q.fs),
                    lsurge::wgrad_chunked_workspace_bytes(pd, q.fs, q.d));
    tab = std::max(lsurge::wgrad_chunk_table_ints(pg, 0), lsurge::wgrad_chunk_table_ints(pd, 0));
  }
  w->part_bytes = part;
  w->part = c.take<char>(part);
  w->dense_tab = c.take<int32_t>(tab);
  w->part_r_bytes = lsurge::wgrad_workspace_bytes(1, q.d, q.E, dense_splits(q.T, q.d, q.E));
  w->part_r = c.take<char>(w->part_r_bytes);
  w->cplan = routed_chunk_plan(q);
  w->chunk_tab = c.take<int32_t>(lsurge::wgrad_chunk_table_ints(w->cplan, q.E));
  w->part_dn_bytes = lsurge::wgrad_chunked_workspace_bytes(w->cplan, q.f, q.d);
  w->part_dn = c.take<char>(w->part_dn_bytes);
  w->part_gu_bytes = lsurge::wgrad_chunked_workspace_bytes(w->cplan, q.d, 2 * q.f);
  w->part_gu = c.take<char>(w->part_gu_bytes);
  return c.off + 256;
}

// The fused router's per-64-token expert histograms (the layout's chunk counts), at the start of the forward
// workspace; 0 when the shape takes the split router.
size_t router_hist_bytes(const lsurge_moe_shape* s) {
  if (!lsurge::router_fused_ok(s->d, s->e, s->k)) return 0;
  return ((size_t)((s->t + 63) / 64) * (size_t)s->e * sizeof(int32_t) + 255) / 256 * 256;
}

// FP8 weights (one caller buffer): E4M3 gate, up [E, f, d], down [E, d, f], shared gate, up [fs, d], down [d, fs]
// (all K-contiguous for the forward), the same codes in the weights' own layout for the backward's dgrads (gate, up
// [E, d, f], down [E, f, d], shared gate, up [d, fs], down [fs, d]: K-contiguous there), then the scale_inv of gate,
// up, down [E] each and of the three shared matrices (one scale per matrix, both copies).
struct Fp8W {
  uint8_t *q_gate, *q_up, *q_down, *qs_gate, *qs_up, *qs_down;
  uint8_t *qb_gate, *qb_up, *qb_down, *qbs_gate, *qbs_up, *qbs_down;
  float *s_gate, *s_up, *s_down, *s_shared;
};
size_t carve_fp8w(const Dims& q, void* base, Fp8W* w) {
  Carve c(base);
  w->q_gate = c.take<uint8_t>(q.E * q.f * q.d);
  w->q_up = c.take<uint8_t>(q.E * q.f * q.d);
  w->q_down = c.take<uint8_t>(q.E * q.d * q.f);
  w->qs_gate = c.take<uint8_t>(q.fs * q.d);
  w->qs_up = c.take<uint8_t>(q.fs * q.d);
  w->qs_down = c.take<uint8_t>(q.d * q.fs);
  w->qb_gate = c.take<uint8_t>(q.E * q.d * q.f);
  w->qb_up = c.take<uint8_t>(q.E * q.d * q.f);
  w->qb_down = c.take<uint8_t>(q.E * q.f * q.d);
  w->qbs_gate = c.take<uint8_t>(q.d * q.fs);
  w->qbs_up = c.take<uint8_t>(q.d * q.fs);
  w->qbs_down = c.take<uint8_t>(q.fs * q.d);
  w->s_gate = c.take<float>(q.E);
  w->s_up = c.take<float>(q.E);
  w->s_down = c.take<float>(q.E);
  w->s_shared = c.take<float>(3);
  return c.off + 256;
}

// FP8 forward scratch: x's amax partials and the atomic-max slots of the routed and shared h (the E4M3 tensors and
// their scale_inv go to the saved buffer)
struct Fp8Ws {
  float* partial;
  uint32_t* slots;
};
size_t carve_fp8ws(const Dims&, void* base, Fp8Ws* w) {
  Carve c(base);
  w->partial = c.take<float>(lsurge::fp8_partial_bytes(1) / sizeof(float));
  w->slots = c.take<uint32_t>(2);
  return c.off;
}

// FP8 backward scratch (after the bf16 backward's BwdWs in the same workspace): the E5M2 gradients, row-major --
// routed dY and [dG | dU] over the padded rows, the shared expert's dY and [dG | dU] over its T rows -- the shared
// expert's [dG | dU] and dx in bf16, amax partials per stream, the atomic-max slots of the two [dG | dU] and the
// scale_inv of the four E5M2 tensors (0 dY, 1 dGU, 2 shared dY, 3 shared dGU).
struct Fp8Bws {
  uint8_t *dyq, *dguq, *sdyq, *sdguq;
  bf16_t *sdgu, *sdx;
  float *part_main, *part_side;
  uint32_t* slots;
  float* sinv;
  float* dy_scale;  // the scale of the routed dY rows
  void* part_s;  // split-K partials of the shared weight gradients
  size_t part_s_bytes;
};
size_t carve_fp8bws(const Dims& q, void* base, Fp8Bws* w) {
  Carve c(base);
  const int64_t T = q.fs ? q.T : 0;
  w->dyq = c.take<uint8_t>(q.P * q.d);
  w->dguq = c.take<uint8_t>(q.P * 2 * q.f);
  w->sdyq = c.take<uint8_t>(T * q.d);
  w->sdguq = c.take<uint8_t>(T * 2 * q.fs);
  w->sdgu = c.take<bf16_t>(T * 2 * q.fs);
  w->sdx = c.take<bf16_t>(T * q.d);
  w->part_main = c.take<float>(lsurge::dy_rows_amax_parts());
  w->part_side = c.take<float>(lsurge::fp8_partial_bytes(1) / sizeof(float));
  w->slots = c.take<uint32_t>(2);
  w->sinv = c.take<float>(4);
  w->dy_scale = c.take<float>(1);
  size_t part = 0;
  if (q.fs) {
    part = std::max(part, lsurge::wgrad_workspace_bytes(1, q.d, 2 * q.fs, dense_splits(q.T, q.d, 2 * q.fs)));
    part = std::max(part, lsurge::wgrad_workspace_bytes(1, q.fs, q.d, dense_splits(q.T, q.fs, q.d)));
  }
  w->part_s_bytes = part;
  w->part_s = c.take<char>(part);
  return c.off + 256;
}

int check_shape(const lsurge_moe_shape* s) {
  LSURGE_REQUIRE(s, "moe: null shape");
  LSURGE_REQUIRE(s->t >= 1 && s->d >= 8 && s->e >= 1 && s->e <= 256 && s->k >= 1 && s->k <= s->e && s->k <= 16 &&
                     s->f >= 64 && s->fs >= 0,
                 "moe: bad shape t=%lld d=%lld e=%lld k=%lld f=%lld fs=%lld", (long long)s->t, (long long)s->d,
                 (long long)s->e, (long long)s->k, (long long)s->f, (long long)s->fs);
  LSURGE_REQUIRE(s->e % 8 == 0, "moe: e=%lld must be a multiple of 8", (long long)s->e);
  LSURGE_REQUIRE(s->d % 64 == 0 && s->f % 64 == 0 && s->fs % 64 == 0,
                 "moe: d, f and fs must be multiples of 64 (d=%lld f=%lld fs=%lld)", (long long)s->d, (long long)s->f,
                 (long long)s->fs);
  LSURGE_REQUIRE(s->t * s->k < (1ll << 31) && (lsurge_max_blocks(s->t * s->k, s->e) + s->t / BLK + 1) * BLK < (1ll << 31),
                 "moe: too many routed rows");
  return LSURGE_OK;
}

}  // namespace

extern "C" {

size_t lsurge_moe_saved_bytes(const lsurge_moe_shape* s) {
  if (check_shape(s)) return 0;
  Saved sv;
  return carve_saved(dims_of(s), nullptr, &sv, false);
}

size_t lsurge_moe_saved_bytes_fp8(const lsurge_moe_shape* s) {
  if (check_shape(s)) return 0;
  Saved sv;
  return carve_saved(dims_of(s), nullptr, &sv, true);
}

size_t lsurge_moe_fwd_workspace_bytes(const lsurge_moe_shape* s) {
  if (check_shape(s)) return 0;
  return router_hist_bytes(s) + lsurge_layout_workspace_bytes(s->t * s->k, s->e) + 256;
}

size_t lsurge_moe_fwd_fp8_workspace_bytes(const lsurge_moe_shape* s) {
  if (check_shape(s)) return 0;
  Fp8Ws w;
  const size_t f8 = (carve_fp8ws(dims_of(s), nullptr, &w) + 255) / 256 * 256;
  return router_hist_bytes(s) + f8 + lsurge_layout_workspace_bytes(s->t * s->k, s->e) + 256;
}

size_t lsurge_moe_fp8_weights_bytes(const lsurge_moe_shape* s) {
  if (check_shape(s)) return 0;
  Fp8W w;
  return carve_fp8w(dims_of(s), nullptr, &w);
}

size_t lsurge_moe_fp8_quantize_weights_workspace_bytes(const lsurge_moe_shape* s) {
  if (check_shape(s)) return 0;
  return lsurge::fp8_partial_bytes(s->e) + lsurge::fp8_partial_bytes(1);
}

}  // extern "C"
namespace {
// Holds a device's helper streams for the duration of one layer call.  A call that returns early (an error after
// the fork) leaves work on the helpers that the caller's stream has not joined yet: the destructor then makes the
// caller's stream wait for every helper before the lock is released, so the call stays stream-ordered on every
// path.  joined() marks the normal path, whose own joins already ordered everything.
struct ForkGuard {
  lsurge::ForkSet f;
  hipStream_t main = nullptr;
  bool held = false, done = false;
  int acquire(hipStream_t m) {
    main = m;
    const int rc = lsurge::fork_acquire(&f, m);
    held = rc == LSURGE_OK;
    return rc;
  }
  int joined(int rc = LSURGE_OK) {
    done = rc == LSURGE_OK;
    return rc;
  }
  ~ForkGuard() {
    if (!held) return;
    if (!done) lsurge::fork_join_all(&f, main);
    lsurge::fork_release(&f);
  }
};
}  // namespace
extern "C" {

// one scale per expert and matrix; each weight is transposed into the K-contiguous operand of the forward's FP8 GEMM
// and also kept in its own layout, the K-contiguous operand of the backward's dgrad (same codes).  The small
// shared-expert matrices (latency-bound launches) go on a helper stream beside the routed ones.
int lsurge_moe_fp8_quantize_weights(const lsurge_moe_shape* s, const lsurge_moe_params* p, void* wq, size_t wq_bytes,
                                    void* workspace, size_t workspace_bytes, lsurge_stream_t stream) {
  if (int rc = check_shape(s)) return rc;
  LSURGE_REQUIRE(p && p->w_gate && p->w_up && p->w_down && wq && workspace, "moe_fp8_quantize_weights: null pointer");
  LSURGE_REQUIRE(!s->fs || (p->ws_gate && p->ws_up && p->ws_down), "moe_fp8_quantize_weights: shared expert weights missing");
  const Dims q = dims_of(s);
  Fp8W w;
  LSURGE_REQUIRE(wq_bytes >= carve_fp8w(q, nullptr, &w), "moe_fp8_quantize_weights: weight buffer %zu < %zu bytes",
                 wq_bytes, carve_fp8w(q, nullptr, &w));
  LSURGE_REQUIRE(workspace_bytes >= lsurge_moe_fp8_quantize_weights_workspace_bytes(s),
                 "moe_fp8_quantize_weights: workspace too small");
  carve_fp8w(q, wq, &w);
  hipStream_t st = (hipStream_t)stream;
  float* part = (float*)workspace;
  float* part_s = part + lsurge::fp8_partial_bytes(q.E) / sizeof(float);
  ForkGuard fg;
  if (int rc = fg.acquire(st)) return rc;
  hipStream_t s0 = fg.f.side[0];
  if (q.fs) {
    if (int rc = lsurge::stream_after(s0, st, fg.f.ev[0])) return rc;
    if (int rc = lsurge::fp8_quantize_impl(p->ws_gate, 1, q.d, q.fs, true, w.qs_gate, w.s_shared, part_s, s0, nullptr,
                                           0, w.qbs_gate))
      return rc;
    if (int rc = lsurge::fp8_quantize_impl(p->ws_up, 1, q.d, q.fs, true, w.qs_up, w.s_shared + 1, part_s, s0, nullptr,
                                           0, w.qbs_up))
      return rc;
    if (int rc = lsurge::fp8_quantize_impl(p->ws_down, 1, q.fs, q.d, true, w.qs_down, w.s_shared + 2, part_s, s0,
                                           nullptr, 0, w.qbs_down))
      return rc;
  }
  if (int rc = lsurge::fp8_quantize_impl(p->w_gate, q.E, q.d, q.f, true, w.q_gate, w.s_gate, part, st, nullptr, 0,
                                         w.qb_gate))
    return rc;
  if (int rc = lsurge::fp8_quantize_impl(p->w_up, q.E, q.d, q.f, true, w.q_up, w.s_up, part, st, nullptr, 0, w.qb_up))
    return rc;
  if (int rc = lsurge::fp8_quantize_impl(p->w_down, q.E, q.f, q.d, true, w.q_down, w.s_down, part, st, nullptr, 0,
                                         w.qb_down))
    return rc;
  return fg.joined(q.fs ? lsurge::stream_after(st, s0, fg.f.ev[1]) : LSURGE_OK);
}

size_t lsurge_moe_bwd_workspace_bytes(const lsurge_moe_shape* s) {
  if (check_shape(s)) return 0;
  BwdWs w;
  return carve_bwd(dims_of(s), nullptr, &w);
}

int lsurge_moe_saved_layout(const lsurge_moe_shape* s, void* saved, lsurge_moe_saved_views* v) {
  if (int rc = check_shape(s)) return rc;
  LSURGE_REQUIRE(saved && v, "moe_saved_layout: null pointer");
  Saved sv;
  carve_saved(dims_of(s), saved, &sv, false);
  v->logits = sv.logits; v->sel = sv.sel; v->weights = sv.weights; v->group_sizes = sv.gs; v->offsets = sv.offsets;
  v->block_off = sv.block_off; v->order = sv.order; v->pos = sv.pos; v->slot = sv.slot; v->row_src = sv.row_src;
  v->blk_expert = sv.blk_expert; v->blk_rows = sv.blk_rows; v->num_blocks = sv.num_blocks;
  v->h_gate = sv.g; v->h_up = sv.u; v->h = sv.h; v->y_pad = sv.y_pad;
  return LSURGE_OK;
}


// Forward.  Stream plan:
//   main: router logits -> selection -> layout (-> tile table of the backward) -> gate/up GEMM -> down GEMM ->
//         [join] -> combine
//   s0:   shared expert (depends on x only): bf16 from the start, on the classic kernels beside the router; FP8
//         after the router's kernel
// The dispatch into padded expert blocks is fused into the gate/up GEMM: its A tiles are gathered straight from
// the token rows x through row_src (padded row -> flat slot t*k + j), so the padded copy of x is never
// materialised (the backward's gate/up weight gradient gathers the same way).
// FP8 (w8 set): x is quantised first (its cast kernel also clears the h amax slots); the expert GEMMs run on E4M3
// operands (routed: 128-row blocks, 4-wave kernel; dense shared: ping-pong kernel), the gate/up epilogues take the
// amax of h, and h is cast before each down projection.
static int moe_fwd_impl(const lsurge_moe_shape* s, const lsurge_moe_params* p, const Fp8W* w8, void* out, void* saved,
                        size_t saved_bytes, void* workspace, size_t workspace_bytes, lsurge_stream_t stream) {
  if (int rc = check_shape(s)) return rc;
  LSURGE_REQUIRE(p && p->x && p->w_r && p->w_gate && p->w_up && p->w_down && out && saved, "moe_fwd: null pointer");
  LSURGE_REQUIRE(!s->fs || (p->ws_gate && p->ws_up && p->ws_down), "moe_fwd: shared expert weights missing");
  const Dims q = dims_of(s);
  Saved sv;
  const size_t need = carve_saved(q, nullptr, &sv, w8 != nullptr);
  LSURGE_REQUIRE(saved_bytes >= need, "moe_fwd: saved buffer %zu < %zu bytes%s", saved_bytes, need,
                 w8 ? " (lsurge_moe_saved_bytes_fp8)" : "");
  carve_saved(q, saved, &sv, w8 != nullptr);
  hipStream_t st = (hipStream_t)stream;
  ForkGuard fg;
  if (int rc = fg.acquire(st)) return rc;
  // A shared expert of its own width (fs != f) runs on the caller's stream: its dense GEMMs are as large as the
  // routed ones and, beside them on a helper stream, each waits for the other's persistent workgroups to drain (C5:
  // 19.2 against 18.3 ms per step with everything on one stream)
  hipStream_t s0 = (q.fs && !q.merged) ? st : fg.f.side[0];

  // main: router logits -> (s0 forks here) -> top-k selection; where the fused router takes the shape, one kernel
  // (logits, top-k, softmax and the layout's per-64-token histograms), after which s0 forks
  // (serial mode: the helpers are the caller's stream and have no events)
  const size_t hist_bytes = router_hist_bytes(s);
  Fp8Ws f8{};
  const size_t f8_bytes = w8 ? (carve_fp8ws(q, nullptr, &f8) + 255) / 256 * 256 : 0;
  LSURGE_REQUIRE(workspace && workspace_bytes >= hist_bytes + f8_bytes, "moe_fwd: workspace %zu bytes too small",
                 workspace_bytes);
  int32_t* rhist = hist_bytes ? (int32_t*)workspace : nullptr;
  // bf16: the shared expert's dense GEMMs fork at the start of the call and run on the classic kernels, whose
  // workgroups (72 KiB of LDS, 4 waves) share a CU with the fused router's (66 KiB, 8 waves): MFMA-bound beside
  // VALU-bound.  The persistent kernels take a CU's whole LDS, so beside them the router would wait for whole GEMMs.
  // C2: 1.547 -> 1.537 ms per step, forward 0.537 -> 0.528 ms (same-box A/B against forking after the router with
  // the persistent kernels).
  const bool early = !w8 && q.fs && s0 != st;
  // a merged shared expert forked early: its down projection rides along the routed down GEMM as expert E (its
  // tiles follow the routed ones in the tile table), so the helper's classic-kernel GEMMs end with the layout
  const bool ride = early && q.merged && lsurge::gemm_variant() == LSURGE_GEMM_G256;
  if (early)
    if (int rc = lsurge::stream_after(s0, st, fg.f.ev[3])) return rc;
  // W_r^T for the backward's router dx term (saved): on the helper stream when it forks here (off the critical path),
  // else first on the caller's stream
  if (!w8)
    if (int rc = lsurge::launch_transpose_bf16(p->w_r, (int)q.d, (int)q.E, sv.w_rT, early ? s0 : st)) return rc;
  // FP8: x's quantisation (memory-bound) runs on s0 beside the router (VALU-bound); the caller's stream waits for
  // it (event ev[2]) only before the routed gate/up GEMM
  if (w8) {
    carve_fp8ws(q, (char*)workspace + hist_bytes, &f8);
    if (int rc = lsurge::stream_after(s0, st, fg.f.ev[3])) return rc;
    if (int rc = lsurge::launch_transpose_bf16(p->w_r, (int)q.d, (int)q.E, sv.w_rT, s0)) return rc;
    if (int rc = lsurge::fp8_quantize_impl(p->x, 1, q.T, q.d, false, sv.xq, sv.f8_sinv, f8.partial, s0, f8.slots, 2))
      return rc;
    if (s0 != st && hipEventRecord(fg.f.ev[2], s0) != hipSuccess)
      return lsurge::set_error(LSURGE_ERR_LAUNCH, "moe_fwd: hipEventRecord failed");
  }
  if (int rc = lsurge::router_topk_impl(p->x, p->w_r, p->bias, q.T, q.d, q.E, q.k, sv.logits, sv.sel, sv.weights, st,
                                        s0 != st && !early ? fg.f.ev[0] : nullptr, rhist))
    return rc;
  // s0: the shared expert's forward, dense GEMMs over all T tokens.  It depends on x only: in bf16 it runs beside the
  // router (above); FP8 starts it after the router's kernel, beside the selection and the layout, whose small grids
  // leave most of the GPU idle.  A merged shared expert writes its g, u, h and output rows where the backward's tile
  // table expects expert E (padded rows 128 MB + t).
  bf16_t *sg = sv.sg, *su = sv.su, *sh = sv.sh, *sy = sv.sy;
  if (q.merged) {
    sg = sv.g + q.P * q.f;
    su = sv.u + q.P * q.f;
    sh = sv.h + q.P * q.f;
    sy = sv.y_pad + q.P * q.d;
  }
  if (s0 != st && !early && hipStreamWaitEvent(s0, fg.f.ev[0], 0) != hipSuccess)
    return lsurge::set_error(LSURGE_ERR_LAUNCH, "moe_fwd: hipStreamWaitEvent failed");
  if (q.fs && w8) {
    const lsurge::GemmBlocks dense{nullptr, nullptr, nullptr, nullptr, 0, q.T, 256};
    if (int rc = lsurge::gemm_rows_f8(KID_SHARED_GU_FWD, dense, sv.xq, q.d, sv.f8_sinv, w8->qs_gate, w8->qs_up, q.d, 0,
                                      w8->s_shared, w8->s_shared + 1, q.d, q.fs, sh, q.fs, false, lsurge::F8_SWIGLU_FWD,
                                      sg, su, f8.slots + 1, s0))
      return rc;
    if (int rc = lsurge::fp8_cast_with_amax(sh, q.T * q.fs, f8.slots + 1, sv.shq, sv.f8_sinv + 2, nullptr, 0, s0))
      return rc;
    if (int rc = lsurge::gemm_rows_f8(KID_SHARED_DOWN_FWD, dense, sv.shq, q.fs, sv.f8_sinv + 2, w8->qs_down, nullptr, q.fs,
                                      0, w8->s_shared + 2, nullptr, q.fs, q.d, sy, q.d, false, lsurge::F8_STORE,
                                      nullptr, nullptr, nullptr, s0))
      return rc;
  } else if (q.fs) {
    const lsurge::GemmBlocks dense{nullptr, nullptr, nullptr, nullptr, 0, q.T, early ? 128 : 256};
    if (int rc = lsurge::gemm_rows_swiglu_fwd(KID_SHARED_GU_FWD, dense, p->x, q.d, p->ws_gate, p->ws_up, q.fs, 0, q.d,
                                              q.fs, sh, sg, su, q.fs, s0))
      return rc;
    if (!ride)
      if (int rc = lsurge::gemm_rows_kn(KID_SHARED_DOWN_FWD, dense, sh, q.fs, p->ws_down, q.d, 0, q.fs, q.d, sy, q.d,
                                        s0))
        return rc;
  }
  // the layout also writes the backward's 256-row tile table: routed tiles, then the merged shared expert's (and
  // its row_src)
  lsurge::LayoutTiles tiles;
  tiles.t_expert = sv.t_expert;
  tiles.t_rows = sv.t_rows;
  tiles.t_row0 = sv.t_row0;
  tiles.num_tiles = sv.num_tiles;
  tiles.TB = (int)q.TB;
  tiles.TS = (int)q.TS;
  tiles.P = q.P;
  tiles.T = q.T;
  tiles.k = (int)q.k;
  // the layout also writes the bf16 backward's chunk table of the routed weight gradients (that backward also runs
  // after the FP8 forward, on its saved buffer)
  tiles.chunks = lsurge::chunk_table_out(sv.chunk_tab, (int)q.E, routed_chunk_plan(q), q.merged ? q.T : -1, q.P);
  lsurge::LayoutChunks chunks;  // the fused router's histograms: chunks of 64 tokens = k waves of 64 slots
  chunks.hist = rhist;
  chunks.waves = (int)q.k;
  if (int rc = lsurge::build_layout_impl(sv.sel, q.M, q.E, sv.gs, sv.offsets, sv.block_off, sv.order, sv.pos, sv.slot,
                                         sv.row_src, sv.blk_expert, sv.blk_rows, sv.num_blocks,
                                         (char*)workspace + hist_bytes + f8_bytes,
                                         workspace_bytes - hist_bytes - f8_bytes, st, tiles, chunks))
    return rc;
  // the routed forward GEMMs: the 256-row tiles (routed ones) on the persistent kernel, or, with the classic kernels,
  // 128-row blocks on the 4-wave kernel (the ping-pong kernel measured no faster there)
  const lsurge::GemmBlocks blocks = lsurge::gemm_variant() == LSURGE_GEMM_G256
                                        ? lsurge::GemmBlocks{sv.t_expert, sv.t_rows, sv.t_row0, sv.num_tiles, (int)q.TB, 0, 256}
                                        : lsurge::GemmBlocks{sv.blk_expert, sv.blk_rows, nullptr, sv.num_blocks, (int)q.MB, 0};
  lsurge::RowGather gather;
  gather.rows = sv.row_src;
  gather.div = (int)q.k;
  gather.nrows = q.T;
  if (w8) {
    // 128-row blocks on the 4-wave kernel (single-buffered FP8 loop, two workgroups per CU): 0.191 / 0.105 ms for
    // gate/up / down at C2 against 0.200 / 0.110 on the ping-pong kernel's 256-row tiles; h is cast over the rows of
    // real blocks
    const lsurge::GemmBlocks blocks8{sv.blk_expert, sv.blk_rows, nullptr, sv.num_blocks, (int)q.MB, 0, 128};
    if (s0 != st && hipStreamWaitEvent(st, fg.f.ev[2], 0) != hipSuccess)
      return lsurge::set_error(LSURGE_ERR_LAUNCH, "moe_fwd: hipStreamWaitEvent failed");
    if (int rc = lsurge::gemm_rows_f8(KID_GEMM_GU_FWD, blocks8, sv.xq, q.d, sv.f8_sinv, w8->q_gate, w8->q_up, q.d,
                                      q.f * q.d, w8->s_gate, w8->s_up, q.d, q.f, sv.h, q.f, false,
                                      lsurge::F8_SWIGLU_FWD, sv.g, sv.u, f8.slots, st, gather))
      return rc;
    if (int rc = lsurge::fp8_cast_with_amax(sv.h, q.P * q.f, f8.slots, sv.hq, sv.f8_sinv + 1, sv.num_blocks, BLK * q.f,
                                            st))
      return rc;
    if (int rc = lsurge::gemm_rows_f8(KID_GEMM_DOWN_FWD, blocks8, sv.hq, q.f, sv.f8_sinv + 1, w8->q_down, nullptr, q.f,
                                      q.d * q.f, w8->s_down, nullptr, q.f, q.d, sv.y_pad, q.d, false, lsurge::F8_STORE,
                                      nullptr, nullptr, nullptr, st))
      return rc;
    if (int rc = fg.joined(lsurge::stream_after(st, s0, fg.f.ev[1]))) return rc;
    return lsurge::launch_combine_pad(sv.y_pad, q.d, (int)q.k, sv.slot, sv.weights, q.T, q.fs ? sy : nullptr, out,
                                      LSURGE_BF16, st);
  }
  if (int rc = lsurge::gemm_rows_swiglu_fwd(KID_GEMM_GU_FWD, blocks, p->x, q.d, p->w_gate, p->w_up, q.f, q.d * q.f,
                                            q.d, q.f, sv.h, sv.g, sv.u, q.f, st, gather))
    return rc;
  lsurge::GemmBlocks dblocks = blocks;
  lsurge::ExtraExpert xdn;
  if (ride) {  // the shared expert's h rows come from the helper: join before the down GEMM
    if (int rc = fg.joined(lsurge::stream_after(st, s0, fg.f.ev[1]))) return rc;
    dblocks = lsurge::GemmBlocks{sv.t_expert, sv.t_rows, sv.t_row0, sv.num_tiles + 1, (int)(q.TB + q.TS), 0, 256};
    xdn.expert = (int)q.E;
    xdn.B = p->ws_down;
  }
  if (int rc = lsurge::gemm_rows_kn(KID_GEMM_DOWN_FWD, dblocks, sv.h, q.f, p->w_down, q.d, q.f * q.d, q.f, q.d,
                                    sv.y_pad, q.d, st, false, xdn))
    return rc;
  if (!ride)
    if (int rc = fg.joined(lsurge::stream_after(st, s0, fg.f.ev[1]))) return rc;
  return lsurge::launch_combine_pad(sv.y_pad, q.d, (int)q.k, sv.slot, sv.weights, q.T, q.fs ? sy : nullptr, out,
                                    LSURGE_BF16, st);
}

int lsurge_moe_fwd(const lsurge_moe_shape* s, const lsurge_moe_params* p, void* out, void* saved, size_t saved_bytes,
                   void* workspace, size_t workspace_bytes, lsurge_stream_t stream) {
  return moe_fwd_impl(s, p, nullptr, out, saved, saved_bytes, workspace, workspace_bytes, stream);
}

int lsurge_moe_fwd_fp8(const lsurge_moe_shape* s, const lsurge_moe_params* p, const void* wq, size_t wq_bytes, void* out,
                       void* saved, size_t saved_bytes, void* workspace, size_t workspace_bytes,
                       lsurge_stream_t stream) {
  if (int rc = check_shape(s)) return rc;
  LSURGE_REQUIRE(wq, "moe_fwd_fp8: null weight buffer");
  const Dims q = dims_of(s);
  Fp8W w;
  LSURGE_REQUIRE(wq_bytes >= carve_fp8w(q, nullptr, &w), "moe_fwd_fp8: weight buffer %zu < %zu bytes", wq_bytes,
                 carve_fp8w(q, nullptr, &w));
  carve_fp8w(q, (void*)wq, &w);
  return moe_fwd_impl(s, p, &w, out, saved, saved_bytes, workspace, workspace_bytes, stream);
}

// Backward.  Stream plan (caller's stream = critical path):
//   main:  [fs != f: the shared expert's own backward: down dgrad, down wgrad, gate/up dgrad, gate/up wgrad] ->
//          combine bwd -> [fork] -> down dgrad (+SwiGLU bwd) -> gate/up dgrad ->
//          dispatch bwd -> gate/up wgrad -> [join]
//   s0:    after the fork, with a merged shared expert: router wgrad
//   s1:    after the fork: down wgrad (then the router wgrad when the shared expert is not merged)
// The helper chains overlap the dgrads of the main chain; nothing on the main chain reads their outputs, so the join
// closes the call.  The dispatch backward reads dX_pad right after the GEMM that wrote it, while it is still in cache.
// Every event record or wait on a stream idles it for several microseconds between the kernels around it, so the
// critical stream gets one record (the fork, shared by both helpers) and one wait (the join: s1 waits for s0 first).
int lsurge_moe_bwd(const lsurge_moe_shape* s, const lsurge_moe_params* p, const void* dy, const void* saved,
                   const lsurge_moe_grads* g, void* workspace, size_t workspace_bytes, lsurge_stream_t stream) {
  if (int rc = check_shape(s)) return rc;
  LSURGE_REQUIRE(p && p->x && p->w_r && p->w_gate && p->w_up && p->w_down && dy && saved && g, "moe_bwd: null pointer");
  LSURGE_REQUIRE(g->dx && g->dw_r && g->dw_gate && g->dw_up && g->dw_down, "moe_bwd: null gradient pointer");
  LSURGE_REQUIRE(!s->fs || (p->ws_gate && p->ws_up && p->ws_down && g->dws_gate && g->dws_up && g->dws_down),
                 "moe_bwd: shared expert pointers missing");
  const Dims q = dims_of(s);
  Saved sv;
  carve_saved(q, (void*)saved, &sv, false);
  BwdWs w;
  const size_t need = carve_bwd(q, nullptr, &w);
  LSURGE_REQUIRE(workspace && workspace_bytes >= need, "moe_bwd: workspace %zu < %zu bytes", workspace_bytes, need);
  carve_bwd(q, workspace, &w);
  hipStream_t st = (hipStream_t)stream;
  float* dweights = g->dweights ? g->dweights : w.dweights;
  // the dgrads run 256-row tiles on the ping-pong kernel (routed tiles, then a merged shared expert's)
  lsurge::GemmBlocks blocks{sv.t_expert, sv.t_rows, sv.t_row0, sv.num_tiles, (int)q.TB, 0, 256};
  lsurge::ExtraExpert xgu, xdn;  // the shared expert carried as expert E: its weights and gradients
  lsurge::ExtraOut ogu, odn;
  if (q.merged) {
    blocks = lsurge::GemmBlocks{sv.t_expert, sv.t_rows, sv.t_row0, sv.num_tiles + 1, (int)(q.TB + q.TS), 0, 256};
    xgu.expert = xdn.expert = ogu.expert = odn.expert = (int)q.E;
    xgu.B = p->ws_gate;
    xgu.B2 = p->ws_up;
    xdn.B = p->ws_down;
    ogu.C = g->dws_gate;
    ogu.C2 = g->dws_up;
    odn.C = g->dws_down;
  }
  ForkGuard fg;
  if (int rc = fg.acquire(st)) return rc;
  // a shared expert of its own width runs its backward on the caller's stream (as in the forward)
  hipStream_t s0 = (q.fs && !q.merged) ? st : fg.f.side[0], s1 = fg.f.side[1];
  hipEvent_t* ev = fg.f.ev;

  // s0: backward of a shared expert of its own width, from the start of the call (after everything the caller
  // enqueued before it)
  if (q.fs && !q.merged) {
    if (int rc = lsurge::stream_after(s0, st, ev[0])) return rc;
    const lsurge::GemmBlocks dense{nullptr, nullptr, nullptr, nullptr, 0, q.T, 256};
    if (int rc = lsurge::gemm_rows_nk(KID_SHARED_DOWN_DGRAD, dense, dy, q.d, p->ws_down, nullptr, 0, q.d, 0, q.d, q.fs,
                                      w.sdgu, 2 * q.fs, true, sv.sg, sv.su, q.fs, s0))
      return rc;
    // the dense weight gradients as chunk tables of one (extra) expert: equal row chunks whose tiles fill the GPU
    // once, reduced from f32 partials in chunk order (the persistent kernel, or the classic one, on the same table)
    lsurge::WgradChunks dch;
    lsurge::ExtraOut dxo;
    dxo.expert = 0;
    dxo.C = g->dws_down;
    if (int rc = lsurge::build_wgrad_chunks(nullptr, nullptr, 0, lsurge::wgrad_chunk_plan_dense(q.T, q.fs, q.d),
                                           w.dense_tab, &dch, s0, q.T, 0, 1))
      return rc;
    if (int rc = lsurge::gemm_wgrad_chunked(KID_SHARED_DOWN_WGRAD, dch, 0, q.T, sv.sh, q.fs, dy, q.d, q.fs, q.d,
                                            nullptr, nullptr, 0, q.d, 0, w.part, w.part_bytes, s0,
                                            lsurge::RowGather(), dxo))
      return rc;
    if (int rc = lsurge::gemm_rows_nk(KID_SHARED_GU_DGRAD, dense, w.sdgu, 2 * q.fs, p->ws_gate, p->ws_up, q.fs, q.fs, 0,
                                      2 * q.fs, q.d, w.sdx, q.d, false, nullptr, nullptr, 0, s0))
      return rc;
    dxo.C = g->dws_gate;
    dxo.C2 = g->dws_up;
    if (int rc = lsurge::build_wgrad_chunks(nullptr, nullptr, 0, lsurge::wgrad_chunk_plan_dense(q.T, q.d, 2 * q.fs),
                                           w.dense_tab, &dch, s0, q.T, 0, 1))
      return rc;
    if (int rc = lsurge::gemm_wgrad_chunked(KID_SHARED_GU_WGRAD, dch, 0, q.T, p->x, q.d, w.sdgu, 2 * q.fs, q.d,
                                            2 * q.fs, nullptr, nullptr, q.fs, q.fs, 0, w.part, w.part_bytes, s0,
                                            lsurge::RowGather(), dxo))
      return rc;
  }
  // the chunk table of the routed weight gradients and W_r^T (the router's dx term) were made by the forward
  const lsurge::WgradChunks chunks =
      lsurge::chunk_table_view(lsurge::chunk_table_out(sv.chunk_tab, (int)q.E, w.cplan, q.merged ? q.T : -1, q.P));
  // main: combine backward: d(weights), d(router logits at sel) and their dense bf16 rows for the router's weight
  // gradient, and the padded dY rows bf16(w dY) of the down projection's GEMMs (a merged shared expert's rows get dY
  // itself).
  // Where the down weight gradient runs on the persistent kernel anyway (at least 16 tiles of 256 x 256 per chunk:
  // f d >= 16 * 65536, as at C5) the dY rows are not written out: the combine backward writes the routing weight of
  // every padded row (wpad) instead, the down dgrad gathers dY rows and scales dH = dY W_down^T by wpad in its
  // epilogue, and the weight gradient gathers and scales them as it stages them, to the bits of bf16(w dY).  C5:
  // 18.20 -> 18.00 ms per step (the combine backward 0.91 -> 0.48 ms, the two down GEMMs +0.31 ms).  With fewer tiles
  // per chunk the scaled gather costs the weight gradient more than the rows save (C2: 1.640 against 1.641 ms).
  // The classic kernels' weight gradient copies its operands straight to LDS, so it reads the written rows; its dgrad
  // takes the gathered path too, so both kernel families give the same bits.
  const bool dy_gather = ((q.f + 255) / 256) * ((q.d + 255) / 256) >= 16;
  const bool dy_rows = !dy_gather || lsurge::gemm_variant() != LSURGE_GEMM_G256;
  if (int rc = lsurge::launch_combine_bwd_pad(sv.y_pad, q.P, sv.slot, sv.weights, q.T, (int)q.k, q.d, dy,
                                              dy_rows ? w.dy_pad : nullptr, dweights, w.dl, st,
                                              dy_rows && q.merged ? w.dy_pad + q.P * q.d : nullptr, sv.sel, w.dlog,
                                              (int)q.E, lsurge::CombineFp8(), dy_gather ? w.wpad : nullptr))
    return rc;
  lsurge::RowGather dyg;  // dY rows through row_src (padded row -> flat slot t k + j, the shared rows -> t k)
  dyg.rows = sv.row_src;
  dyg.div = (int)q.k;
  dyg.nrows = q.T;
  // fork: the helpers start after the combine backward (and everything the caller enqueued before the call); one
  // record on the critical stream serves both
  if (s1 != st) {
    if (hipEventRecord(ev[2], st) != hipSuccess || hipStreamWaitEvent(s1, ev[2], 0) != hipSuccess ||
        (q.merged && hipStreamWaitEvent(s0, ev[2], 0) != hipSuccess))
      return lsurge::set_error(LSURGE_ERR_LAUNCH, "moe_bwd: fork events failed");
  }
  // s1: down wgrad dW_down[e] = h_e^T dY_e (without written dY rows: gathered and scaled by wpad)
  {
    lsurge::RowGather bg = dyg;
    bg.on_b = true;
    bg.scale = w.wpad;
    if (int rc = lsurge::gemm_wgrad_chunked(KID_GEMM_DOWN_WGRAD, chunks, (int)q.E, q.T, sv.h, q.f,
                                            dy_rows ? (const void*)w.dy_pad : dy, q.d, q.f, q.d, g->dw_down, nullptr, 0,
                                            q.d, q.f * q.d, w.part_dn, w.part_dn_bytes, s1,
                                            dy_rows ? lsurge::RowGather() : bg, odn))
      return rc;
  }
  // router backward dW_r = x^T dlogits (bf16 MFMA over the dense [T, E] dlogits): on s0 beside the down wgrad when
  // s0 is free (merged shared expert), else after the down wgrad on s1
  hipStream_t sr = q.merged ? s0 : s1;
  {
    const int S = dense_splits(q.T, q.d, q.E);
    if (int rc = lsurge::gemm_wgrad(KID_ROUTER_WGRAD, 1, nullptr, 1, nullptr, q.T, q.T, p->x, q.d, w.dlog, q.E, q.d,
                                    q.E, g->dw_r, nullptr, 0, q.E, 0, S, w.part_r, w.part_r_bytes, sr))
      return rc;
  }
  // main: down dgrad + SwiGLU backward: dH = dY_pad W_down^T, or w (dY W_down^T) from gathered dY rows -> [dG | dU]
  if (int rc = lsurge::gemm_rows_nk(KID_GEMM_DOWN_DGRAD, blocks, dy_gather ? dy : (const void*)w.dy_pad, q.d, p->w_down,
                                    nullptr, 0, q.d, q.f * q.d, q.d, q.f, w.dgu, 2 * q.f, true, sv.g, sv.u, q.f, st,
                                    false, xdn, LSURGE_BF16, dy_gather ? dyg : lsurge::RowGather(),
                                    dy_gather ? w.wpad : nullptr))
    return rc;
  // main: gate/up dgrad: dX_pad = dG W_gate^T + dU W_up^T
  if (int rc = lsurge::gemm_rows_nk(KID_GEMM_GU_DGRAD, blocks, w.dgu, 2 * q.f, p->w_gate, p->w_up, q.f, q.f, q.d * q.f,
                                    2 * q.f, q.d, w.dx_pad, q.d, false, nullptr, nullptr, 0, st, false, xgu))
    return rc;
  // main: dx = gather-reduce of dX_pad + router dx term + shared-expert dx, one rounding (all made on this stream)
  const bf16_t* shared_dx = q.merged ? w.dx_pad + q.P * q.d : (q.fs ? w.sdx : nullptr);
  if (int rc = lsurge::launch_dispatch_bwd_pad(w.dx_pad, q.d, (int)q.k, sv.slot, q.T, w.dl, sv.sel, sv.w_rT, shared_dx,
                                              g->dx, st))
    return rc;
  // main: gate/up wgrad: [dW_gate | dW_up][e] = x_e^T [dG | dU]_e
  {
    lsurge::RowGather gather;  // x_e rows gathered from x through row_src, as in the forward
    gather.rows = sv.row_src;
    gather.div = (int)q.k;
    gather.nrows = q.T;
    if (int rc = lsurge::gemm_wgrad_chunked(KID_GEMM_GU_WGRAD, chunks, (int)q.E, q.T, p->x, q.d, w.dgu, 2 * q.f, q.d,
                                            2 * q.f, g->dw_gate, g->dw_up, q.f, q.f, q.d * q.f, w.part_gu,
                                            w.part_gu_bytes, st, gather, ogu))
      return rc;
  }
  // join all helpers (s1 after s0, the critical stream after s1) at the end: nothing on the critical stream reads
  // their outputs, and the wait lands next to the caller's following stream operation (the next forward's fork
  // record), whose idle gap it then shares
  if (int rc = lsurge::stream_after(s1, s0, ev[4])) return rc;
  return fg.joined(lsurge::stream_after(st, s1, ev[5]));
}

size_t lsurge_moe_bwd_fp8_workspace_bytes(const lsurge_moe_shape* s) {
  if (check_shape(s)) return 0;
  const Dims q = dims_of(s);
  BwdWs w;
  Fp8Bws f;
  return (carve_bwd(q, nullptr, &w) + 255) / 256 * 256 + carve_fp8bws(q, nullptr, &f);
}

// FP8 backward (Transformer Engine's current-scaling training recipe, hybrid formats): gradients are cast to E5M2
// with power-of-two scales of their own (dY rows, [dG | dU], per tensor, just before use), the dgrads multiply them
// with the weights' E4M3 codes of the forward (their untransposed copies, same scales), and the wgrads multiply the
// forward's E4M3 x and h (kept in `saved`) with them.  Every FP8 operand is row-major: the weight gradients stage
// both operands N-major and read K-contiguous fragments with the 8-bit LDS transpose read, so nothing is cast twice
// or transposed.  The dY rows come out of the combine backward as E5M2 directly (their amax from dy and the routing
// weights beforehand).  Combine, dispatch and router backward are those of the bf16 backward; the shared expert runs
// its FP8 backward as dense GEMMs of its own.
// Stream plan (caller's stream = critical path):
//   main: dY scale -> combine bwd (E5M2 dY rows) -> [record] -> down dgrad (+SwiGLU bwd, amax of [dG | dU]) ->
//         [dG | dU] cast -> gate/up dgrad -> [join] -> dispatch bwd -> gate/up wgrad
//   s1:   from the start: the chunk table; after the record: down wgrad
//   s0:   from the start: the shared expert's backward; after the record: router wgrad
int lsurge_moe_bwd_fp8(const lsurge_moe_shape* s, const lsurge_moe_params* p, const void* wq, size_t wq_bytes,
                       const void* dy, const void* saved, const lsurge_moe_grads* g, void* workspace,
                       size_t workspace_bytes, lsurge_stream_t stream) {
  if (int rc = check_shape(s)) return rc;
  LSURGE_REQUIRE(p && p->x && p->w_r && wq && dy && saved && g, "moe_bwd_fp8: null pointer");
  LSURGE_REQUIRE(g->dx && g->dw_r && g->dw_gate && g->dw_up && g->dw_down, "moe_bwd_fp8: null gradient pointer");
  LSURGE_REQUIRE(!s->fs || (g->dws_gate && g->dws_up && g->dws_down), "moe_bwd_fp8: shared expert gradients missing");
  const Dims q = dims_of(s);
  Fp8W w8;
  LSURGE_REQUIRE(wq_bytes >= carve_fp8w(q, nullptr, &w8), "moe_bwd_fp8: weight buffer %zu < %zu bytes", wq_bytes,
                 carve_fp8w(q, nullptr, &w8));
  carve_fp8w(q, (void*)wq, &w8);
  Saved sv;
  carve_saved(q, (void*)saved, &sv, true);
  BwdWs w;
  Fp8Bws f8;
  const size_t wb = (carve_bwd(q, nullptr, &w) + 255) / 256 * 256;
  const size_t need = wb + carve_fp8bws(q, nullptr, &f8);
  LSURGE_REQUIRE(workspace && workspace_bytes >= need, "moe_bwd_fp8: workspace %zu < %zu bytes", workspace_bytes, need);
  carve_bwd(q, workspace, &w);
  carve_fp8bws(q, (char*)workspace + wb, &f8);
  hipStream_t st = (hipStream_t)stream;
  float* dweights = g->dweights ? g->dweights : w.dweights;
  const int64_t d = q.d, f = q.f, fs = q.fs, P = q.P, T = q.T;
  // the routed dgrads run the forward's 128-row blocks on the 4-wave kernel
  const lsurge::GemmBlocks blocks8{sv.blk_expert, sv.blk_rows, nullptr, sv.num_blocks, (int)q.MB, 0, 128};
  ForkGuard fg;
  if (int rc = fg.acquire(st)) return rc;
  hipStream_t s0 = fg.f.side[0], s1 = fg.f.side[1];
  hipEvent_t* ev = fg.f.ev;
  if (int rc = lsurge::stream_after(s1, st, ev[0])) return rc;
  if (s0 != st && hipStreamWaitEvent(s0, ev[0], 0) != hipSuccess)
    return lsurge::set_error(LSURGE_ERR_LAUNCH, "moe_bwd_fp8: hipStreamWaitEvent failed");

  // s1: the chunk table (W_r^T was made by the forward)
  lsurge::WgradChunks chunks;
  if (int rc = lsurge::build_wgrad_chunks(sv.gs, sv.block_off, (int)q.E, w.cplan, w.chunk_tab, &chunks, s1)) return rc;

  // s0: the shared expert's backward over its T rows (its own dY cast; g, u where the forward left them)
  if (fs) {
    const bf16_t* sg = q.merged ? sv.g + P * f : sv.sg;
    const bf16_t* su = q.merged ? sv.u + P * f : sv.su;
    const lsurge::GemmBlocks dense{nullptr, nullptr, nullptr, nullptr, 0, T, 256};
    const int nb = lsurge::fp8_amax(dy, T * d, f8.part_side, s0);
    if (nb < 0) return nb;
    if (int rc = lsurge::fp8_cast_e5m2(dy, T * d, f8.part_side, nb, f8.sdyq, f8.sinv + 2, nullptr, 0, s0, f8.slots + 1, 1))
      return rc;
    if (int rc = lsurge::gemm_rows_f8(KID_SHARED_DOWN_DGRAD, dense, f8.sdyq, d, f8.sinv + 2, w8.qbs_down, nullptr, d, 0,
                                      w8.s_shared + 2, nullptr, d, fs, f8.sdgu, 2 * fs, false, lsurge::F8_SWIGLU_BWD,
                                      (void*)sg, (void*)su, f8.slots + 1, s0, lsurge::RowGather(), 0, true))
      return rc;
    if (int rc = lsurge::fp8_cast_e5m2(f8.sdgu, T * 2 * fs, (const float*)(f8.slots + 1), 1, f8.sdguq, f8.sinv + 3,
                                       nullptr, 0, s0))
      return rc;
    if (int rc = lsurge::gemm_rows_f8(KID_SHARED_GU_DGRAD, dense, f8.sdguq, 2 * fs, f8.sinv + 3, w8.qbs_gate, w8.qbs_up,
                                      fs, 0, w8.s_shared, w8.s_shared + 1, 2 * fs, d, f8.sdx, d, false,
                                      lsurge::F8_STORE, nullptr, nullptr, nullptr, s0, lsurge::RowGather(), fs, true))
      return rc;
    if (int rc = lsurge::gemm_wgrad_f8_dense(KID_SHARED_DOWN_WGRAD, T, sv.shq, fs, sv.f8_sinv + 2, f8.sdyq, d,
                                             f8.sinv + 2, fs, d, g->dws_down, nullptr, 0, d, dense_splits(T, fs, d),
                                             f8.part_s, f8.part_s_bytes, s0))
      return rc;
    if (int rc = lsurge::gemm_wgrad_f8_dense(KID_SHARED_GU_WGRAD, T, sv.xq, d, sv.f8_sinv, f8.sdguq, 2 * fs,
                                             f8.sinv + 3, d, 2 * fs, g->dws_gate, g->dws_up, fs, fs,
                                             dense_splits(T, d, 2 * fs), f8.part_s, f8.part_s_bytes, s0))
      return rc;
  }

  // main: the scale of the dY rows (from dy and the routing weights; also clears the [dG | dU] amax slot), then the
  // combine backward writing them as E5M2 (plus d(weights), d(logits) and their dense rows)
  {
    if (int rc = lsurge::launch_dy_scale(dy, sv.weights, T, d, (int)q.k, f8.part_main, f8.dy_scale, f8.sinv, st,
                                         f8.slots, 1))
      return rc;
    lsurge::CombineFp8 c8;
    c8.dyq = f8.dyq;
    c8.scale = f8.dy_scale;
    c8.nblocks = sv.num_blocks;
    if (int rc = lsurge::launch_combine_bwd_pad(sv.y_pad, P, sv.slot, sv.weights, T, (int)q.k, d, dy, w.dy_pad,
                                                dweights, w.dl, st, nullptr, sv.sel, w.dlog, (int)q.E, c8))
      return rc;
  }
  if (s1 != st) {
    if (hipEventRecord(ev[2], st) != hipSuccess || hipStreamWaitEvent(s1, ev[2], 0) != hipSuccess ||
        hipStreamWaitEvent(s0, ev[2], 0) != hipSuccess)
      return lsurge::set_error(LSURGE_ERR_LAUNCH, "moe_bwd_fp8: fork events failed");
  }
  // s1: down wgrad dW_down[e] = h_e^T dY_e;  s0: router wgrad dW_r = x^T dlogits (bf16)
  if (int rc = lsurge::gemm_wgrad_f8_chunked(KID_GEMM_DOWN_WGRAD, chunks, (int)q.E, T, sv.hq, f, sv.f8_sinv + 1,
                                             f8.dyq, d, f8.sinv, f, d, g->dw_down, nullptr, 0, d, f * d, w.part_dn,
                                             w.part_dn_bytes, s1))
    return rc;
  {
    const int S = dense_splits(T, d, q.E);
    if (int rc = lsurge::gemm_wgrad(KID_ROUTER_WGRAD, 1, nullptr, 1, nullptr, T, T, p->x, d, w.dlog, q.E, d, q.E,
                                    g->dw_r, nullptr, 0, q.E, 0, S, w.part_r, w.part_r_bytes, s0))
      return rc;
  }
  // main: down dgrad + SwiGLU backward, dH = dY W_down^T -> [dG | dU] (bf16) and its amax
  if (int rc = lsurge::gemm_rows_f8(KID_GEMM_DOWN_DGRAD, blocks8, f8.dyq, d, f8.sinv, w8.qb_down, nullptr, d, f * d,
                                    w8.s_down, nullptr, d, f, w.dgu, 2 * f, false, lsurge::F8_SWIGLU_BWD, sv.g, sv.u,
                                    f8.slots, st, lsurge::RowGather(), 0, true))
    return rc;
  if (int rc = lsurge::fp8_cast_e5m2(w.dgu, P * 2 * f, (const float*)f8.slots, 1, f8.dguq, f8.sinv + 1, sv.num_blocks,
                                     BLK * 2 * f, st))
    return rc;
  // main: gate/up dgrad dX_pad = dG W_gate^T + dU W_up^T (each weight at its own scale)
  if (int rc = lsurge::gemm_rows_f8(KID_GEMM_GU_DGRAD, blocks8, f8.dguq, 2 * f, f8.sinv + 1, w8.qb_gate, w8.qb_up, f,
                                    d * f, w8.s_gate, w8.s_up, 2 * f, d, w.dx_pad, d, false, lsurge::F8_STORE, nullptr,
                                    nullptr, nullptr, st, lsurge::RowGather(), f, true))
    return rc;
  // join (s1 after s0, the caller's stream after s1), then the dispatch backward and the gate/up wgrad over the
  // E4M3 x rows gathered through row_src
  if (int rc = lsurge::stream_after(s1, s0, ev[4])) return rc;
  if (int rc = fg.joined(lsurge::stream_after(st, s1, ev[5]))) return rc;
  if (int rc = lsurge::launch_dispatch_bwd_pad(w.dx_pad, d, (int)q.k, sv.slot, T, w.dl, sv.sel, sv.w_rT,
                                              fs ? f8.sdx : nullptr, g->dx, st))
    return rc;
  lsurge::RowGather gather;
  gather.rows = sv.row_src;
  gather.div = (int)q.k;
  gather.nrows = T;
  return lsurge::gemm_wgrad_f8_chunked(KID_GEMM_GU_WGRAD, chunks, (int)q.E, T, sv.xq, d, sv.f8_sinv, f8.dguq, 2 * f,
                                       f8.sinv + 1, d, 2 * f, g->dw_gate, g->dw_up, f, f, d * f, w.part_gu,
                                       w.part_gu_bytes, st, gather);
}

}  // extern "C"
