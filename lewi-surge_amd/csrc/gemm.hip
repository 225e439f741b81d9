// Launchers and C ABI of the grouped GEMMs of the MoE layer (the kernels are in gemm_kernels.h): shape checks,
// grid sizes, the split-K reduction of dense weight gradients, and the ragged_dot entry points that replace
// modal/padded_gmm.py:45-69 (padded_ragged_dot and its gather-only VJP).
#include "gemm_kernels.h"
#include "launchers.h"

namespace {
using namespace lsgemm;

// The tile shape of every grouped GEMM: 128 rows (one padded expert block) x 256 columns, 4 waves of 64 x 128,
// K in 32-deep stages through a 3-stage LDS ring (72 KiB), two workgroups per CU so that one's barrier and
// epilogue overlap the other's MFMAs.
using Cfg = GemmCfg<128, 256, 32, 2, 2, 3, 2>;
constexpr int BM = Cfg::BM, BN = Cfg::BN, BK = Cfg::BK, GT = Cfg::GT;

// sum of the S split partials in split order -> C (and C2 for n >= n_split)
__global__ void splitk_reduce_kernel(const float* __restrict__ part, int S, int E, int64_t I, int64_t N,
                                     float* __restrict__ C, float* __restrict__ C2, int64_t n_split, int64_t ldc,
                                     int64_t c_estride) {
  const int64_t total = (int64_t)E * I * N;
  for (int64_t x = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; x < total; x += (int64_t)gridDim.x * blockDim.x) {
    float v = 0.f;
    for (int s = 0; s < S; ++s) v += part[(int64_t)s * total + x];
    const int64_t e = x / (I * N), rem = x % (I * N);
    const int64_t row = rem / N, col = rem % N;
    if (C2 && col >= n_split) C2[e * c_estride + row * ldc + (col - n_split)] = v;
    else C[e * c_estride + row * ldc + col] = v;
  }
}

// block table of an unpadded ragged layout (rows of group e start at sum_{e'<e} gs[e']).  Group sizes are
// clamped so that no group reaches past row m: negative sizes count as 0 and a sum above m is cut at m, so a
// bad group_sizes array can never send the GEMMs outside lhs/out.
__global__ void ragged_blocks_kernel(const int32_t* __restrict__ gs, int E, int64_t m, int max_blocks,
                                     int32_t* __restrict__ blk_row0, int32_t* __restrict__ blk_rows,
                                     int32_t* __restrict__ blk_expert, int32_t* __restrict__ num_blocks,
                                     int32_t* __restrict__ total_rows, int32_t* __restrict__ e_row0,
                                     int32_t* __restrict__ e_rows) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  int b = 0, run = 0;
  for (int e = 0; e < E; ++e) {
    const int g = (int)min((int64_t)max(gs[e], 0), m - run);
    e_rows[e] = g;
    e_row0[e] = run;
    for (int j = 0; j * BM < g; ++j, ++b) {
      if (b < max_blocks) {
        blk_row0[b] = run + j * BM;
        blk_rows[b] = min(BM, g - j * BM);
        blk_expert[b] = e;
      }
    }
    run += g;
  }
  num_blocks[0] = min(b, max_blocks);
  total_rows[0] = run;
  for (int i = b; i < max_blocks; ++i) {
    blk_rows[i] = 0;
    blk_expert[i] = -1;
  }
}

// zero the rows [from[0], m) of an [m, n] matrix with esize-byte elements (rows past the groups)
__global__ void zero_rows_from_kernel(void* __restrict__ out, int64_t m, int64_t n, int esize,
                                      const int32_t* __restrict__ from) {
  const int64_t r0 = from[0];
  const int64_t total = (m - r0) * n;
  for (int64_t x = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; x < total; x += (int64_t)gridDim.x * blockDim.x) {
    if (esize == 4) ((float*)out)[r0 * n + x] = 0.f;
    else ((bf16_t*)out)[r0 * n + x] = 0;
  }
}

inline unsigned pad8(int64_t g) { return (unsigned)((g + 7) / 8 * 8); }

}  // namespace

// ------------------------------------------------------------------------------ internal launchers
namespace lsurge {


static int check_gemm_shape(int64_t K, int64_t N, const char* what) {
  LSURGE_REQUIRE(K > 0 && N > 0 && K % 8 == 0 && N % 8 == 0, "%s: K=%lld N=%lld must be positive multiples of 8", what,
                 (long long)K, (long long)N);
  return LSURGE_OK;
}

// every buffer descriptor must cover fewer than 2^31 bytes (the out-of-range offset is 2^31)
static int check_desc(int64_t bytes, const char* what) {
  LSURGE_REQUIRE(bytes >= 0 && bytes < (1ll << 31), "%s: operand span of %lld bytes exceeds 2 GiB", what,
                 (long long)bytes);
  return LSURGE_OK;
}

static int max_blocks_of(const GemmBlocks& g) {
  return g.blk_expert ? g.max_blocks : (int)((g.dense_rows + BM - 1) / BM);
}

// C[rows, N] = A[rows, K] @ B_e where B_e is [K, N] (n-major) -- forward projections
int gemm_rows_kn(int kid, const GemmBlocks& g, const void* A, int64_t lda, const void* B, int64_t ldb,
                 int64_t b_estride, int64_t K, int64_t N, void* C, int64_t ldc, hipStream_t s, bool out_f32) {
  if (int rc = check_gemm_shape(K, N, "gemm_rows_kn")) return rc;
  if (int rc = check_desc(std::max<int64_t>(BM * lda, K * ldb) * 2, "gemm_rows_kn")) return rc;
  RowsArgs a{};
  a.A = (const bf16_t*)A; a.lda = lda; a.B = (const bf16_t*)B; a.ldb = ldb; a.b_estride = b_estride;
  a.K = K; a.N = N; a.ldc = ldc;
  if (out_f32) a.Cf = (float*)C;
  else a.C = (bf16_t*)C;
  a.t_expert = g.blk_expert; a.t_rows = g.blk_rows; a.t_row0 = g.blk_row0; a.num_tiles = g.num_blocks;
  a.dense_rows = g.dense_rows; a.max_tiles = max_blocks_of(g);
  a.n_tiles = (int)((N + BN - 1) / BN);
  if (a.max_tiles == 0) return LSURGE_OK;
  LSURGE_LAUNCH(kid, s, hipLaunchKernelGGL((gemm_rows_kernel<Cfg, B_KN, EPI_STORE>),
                                           dim3(pad8((int64_t)a.n_tiles * a.max_tiles)), dim3(GT), 0, s, a));
  return LSURGE_OK;
}

// h = silu(A @ Bg) * (A @ Bu); also stores g, u.  Bg, Bu: [K, N] per expert.  With a gather (gather.rows set),
// tile row r reads A[gather.rows[row0 + r] / gather.div] of an A with gather.nrows rows (negative: zero row).
int gemm_rows_swiglu_fwd(int kid, const GemmBlocks& g, const void* A, int64_t lda, const void* Bg, const void* Bu,
                         int64_t ldb, int64_t b_estride, int64_t K, int64_t N, void* H, void* Gs, void* Us,
                         int64_t ldh, hipStream_t s, const RowGather& gather) {
  if (int rc = check_gemm_shape(K, N, "gemm_rows_swiglu_fwd")) return rc;
  if (int rc = check_desc(std::max<int64_t>(BM * lda, K * ldb) * 2, "gemm_rows_swiglu_fwd")) return rc;
  if (gather.rows) {
    LSURGE_REQUIRE(gather.div >= 1 && gather.nrows >= 1, "gemm_rows_swiglu_fwd: bad row gather");
    if (int rc = check_desc(gather.nrows * lda * 2, "gemm_rows_swiglu_fwd gather")) return rc;
  }
  RowsArgs a{};
  a.a_rows = gather.rows; a.a_nrows = gather.nrows; a.a_div = gather.div;
  a.A = (const bf16_t*)A; a.lda = lda; a.B = (const bf16_t*)Bg; a.B2 = (const bf16_t*)Bu; a.ldb = ldb;
  a.b_estride = b_estride; a.K = K; a.N = N; a.C = (bf16_t*)H; a.ldc = ldh; a.G = (bf16_t*)Gs; a.U = (bf16_t*)Us;
  a.ldg = ldh;
  a.t_expert = g.blk_expert; a.t_rows = g.blk_rows; a.t_row0 = g.blk_row0; a.num_tiles = g.num_blocks;
  a.dense_rows = g.dense_rows; a.max_tiles = max_blocks_of(g);
  a.n_tiles = (int)((N + BN / 2 - 1) / (BN / 2));
  if (a.max_tiles == 0) return LSURGE_OK;
  LSURGE_LAUNCH(kid, s, hipLaunchKernelGGL((gemm_rows_kernel<Cfg, B_KN, EPI_SWIGLU_FWD>),
                                           dim3(pad8((int64_t)a.n_tiles * a.max_tiles)), dim3(GT), 0, s, a));
  return LSURGE_OK;
}

// C[rows, N] = A[rows, K] @ B_e^T where B_e is stored [N, K] (k-major); with B2 and k_split the K range
// [k_split, K) reads B2 (gate/up dgrad: A = [dG | dU], B = W_gate, B2 = W_up, k_split = f).
// swiglu_bwd: C = [dG | dU] from dH = A @ B^T and the saved G, U (ldg pitch).
int gemm_rows_nk(int kid, const GemmBlocks& g, const void* A, int64_t lda, const void* B, const void* B2,
                 int64_t k_split, int64_t ldb, int64_t b_estride, int64_t K, int64_t N, void* C, int64_t ldc,
                 bool swiglu_bwd, const void* Gs, const void* Us, int64_t ldg, hipStream_t s, bool out_f32) {
  if (int rc = check_gemm_shape(K, N, "gemm_rows_nk")) return rc;
  if (int rc = check_desc(std::max<int64_t>(BM * lda, N * ldb) * 2, "gemm_rows_nk")) return rc;
  LSURGE_REQUIRE(!B2 || (k_split > 0 && k_split % BK == 0), "gemm_rows_nk: k_split must be a multiple of %d", BK);
  RowsArgs a{};
  a.A = (const bf16_t*)A; a.lda = lda; a.B = (const bf16_t*)B; a.B2 = (const bf16_t*)B2; a.k_split = B2 ? k_split : 0;
  a.ldb = ldb; a.b_estride = b_estride; a.K = K; a.N = N; a.ldc = ldc;
  if (out_f32 && !swiglu_bwd) a.Cf = (float*)C;
  else a.C = (bf16_t*)C;
  a.G = (bf16_t*)Gs; a.U = (bf16_t*)Us; a.ldg = ldg;
  a.t_expert = g.blk_expert; a.t_rows = g.blk_rows; a.t_row0 = g.blk_row0; a.num_tiles = g.num_blocks;
  a.dense_rows = g.dense_rows; a.max_tiles = max_blocks_of(g);
  a.n_tiles = (int)((N + BN - 1) / BN);
  if (a.max_tiles == 0) return LSURGE_OK;
  const dim3 grid(pad8((int64_t)a.n_tiles * a.max_tiles));
  if (swiglu_bwd)
    LSURGE_LAUNCH(kid, s, hipLaunchKernelGGL((gemm_rows_kernel<Cfg, B_NK, EPI_SWIGLU_BWD>), grid, dim3(GT), 0, s, a));
  else
    LSURGE_LAUNCH(kid, s, hipLaunchKernelGGL((gemm_rows_kernel<Cfg, B_NK, EPI_STORE>), grid, dim3(GT), 0, s, a));
  return LSURGE_OK;
}

size_t wgrad_workspace_bytes(int E, int64_t I, int64_t N, int S) {
  return S > 1 ? sizeof(float) * (size_t)S * E * I * N : 0;
}

// C_e[I, N] = A_e^T @ B_e over the rows of expert e; columns >= n_split go to C2 (if given).  max_rows bounds
// the rows of any one expert (the dense row count, or the token count for routed rows).
int gemm_wgrad(int kid, int E, const int32_t* e_row0, int row0_mult, const int32_t* e_rows, int64_t dense_rows,
               int64_t max_rows, const void* A, int64_t lda, const void* B, int64_t ldb, int64_t I, int64_t N, float* C,
               float* C2, int64_t n_split, int64_t ldc, int64_t c_estride, int S, void* ws, size_t ws_bytes,
               hipStream_t s, const RowGather& gather) {
  if (int rc = check_gemm_shape(I, N, "gemm_wgrad")) return rc;
  if (int rc = check_desc(max_rows * std::max(lda, ldb) * 2, "gemm_wgrad")) return rc;
  LSURGE_REQUIRE(S >= 1 && E >= 1, "gemm_wgrad: bad S/E");
  if (gather.rows) {
    LSURGE_REQUIRE(gather.div >= 1 && gather.nrows >= 1 && e_rows, "gemm_wgrad: bad row gather");
    if (int rc = check_desc(gather.nrows * lda * 2, "gemm_wgrad gather")) return rc;
  }
  WgradArgs a{};
  a.a_rows = gather.rows; a.a_nrows = gather.nrows; a.a_div = gather.div;
  a.A = (const bf16_t*)A; a.lda = lda; a.B = (const bf16_t*)B; a.ldb = ldb; a.I = I; a.N = N; a.C = C; a.C2 = C2;
  a.n_split = n_split; a.ldc = ldc; a.c_estride = c_estride; a.e_row0 = e_row0; a.e_rows = e_rows;
  a.row0_mult = row0_mult;
  a.dense_rows = dense_rows; a.E = E; a.S = S;
  a.i_tiles = (int)((I + BM - 1) / BM);
  a.n_tiles = (int)((N + BN - 1) / BN);
  if (S > 1) {
    const size_t need = wgrad_workspace_bytes(E, I, N, S);
    LSURGE_REQUIRE(ws && ws_bytes >= need, "gemm_wgrad: workspace %zu < %zu", ws_bytes, need);
    a.part = (float*)ws;
  }
  const int64_t tiles = (int64_t)E * S * a.i_tiles * a.n_tiles;
  LSURGE_LAUNCH(kid, s, hipLaunchKernelGGL(gemm_wgrad_kernel<Cfg>, dim3(pad8(tiles)), dim3(GT), 0, s, a));
  if (S > 1) {
    const int64_t total = (int64_t)E * I * N;
    const unsigned grid = (unsigned)std::min<int64_t>((total + 255) / 256, 8192);
    LSURGE_LAUNCH(KID_SPLITK_REDUCE, s,
                  hipLaunchKernelGGL(splitk_reduce_kernel, dim3(grid), dim3(256), 0, s, (const float*)ws, S, E, I, N, C,
                                     C2, n_split, ldc, c_estride));
  }
  return LSURGE_OK;
}

}  // namespace lsurge

// ------------------------------------------------------------------------------ C ABI: ragged_dot
// workspace: blk_row0, blk_rows, blk_expert [max_blocks] | num_blocks, total_rows | e_row0 [e]
extern "C" {

size_t lsurge_ragged_dot_workspace_bytes(int64_t m, int64_t e) {
  const int64_t mb = lsurge_max_blocks(m, e);
  return sizeof(int32_t) * (size_t)(3 * mb + 4 + 2 * e);
}

static int ragged_setup(const int32_t* gs, int64_t m, int64_t e, void* ws, size_t ws_bytes, hipStream_t s,
                        lsurge::GemmBlocks* g, int32_t** total_rows, int32_t** e_row0, int32_t** e_rows) {
  const size_t need = lsurge_ragged_dot_workspace_bytes(m, e);
  LSURGE_REQUIRE(ws && ws_bytes >= need, "ragged_dot: workspace %zu < %zu bytes", ws_bytes, need);
  const int64_t mb = lsurge_max_blocks(m, e);
  int32_t* p = (int32_t*)ws;
  int32_t* blk_row0 = p;
  int32_t* blk_rows = p + mb;
  int32_t* blk_expert = p + 2 * mb;
  int32_t* nb = p + 3 * mb;
  *total_rows = nb + 1;
  *e_row0 = nb + 4;
  *e_rows = nb + 4 + e;
  LSURGE_LAUNCH(KID_MISC, s,
                hipLaunchKernelGGL(ragged_blocks_kernel, dim3(1), dim3(64), 0, s, gs, (int)e, m, (int)mb, blk_row0,
                                   blk_rows, blk_expert, nb, *total_rows, *e_row0, *e_rows));
  g->blk_expert = blk_expert;
  g->blk_rows = blk_rows;
  g->blk_row0 = blk_row0;
  g->num_blocks = nb;
  g->max_blocks = (int)mb;
  g->dense_rows = 0;
  return LSURGE_OK;
}

int lsurge_ragged_dot(const void* lhs, const void* rhs, const int32_t* group_sizes, int64_t m, int64_t kdim, int64_t n,
                      int64_t e, void* out, int out_dtype, void* workspace, size_t workspace_bytes,
                      lsurge_stream_t stream) {
  LSURGE_REQUIRE(m >= 0 && e >= 1 && m < (1ll << 31), "ragged_dot: bad m/e");
  LSURGE_REQUIRE(out_dtype == LSURGE_BF16 || out_dtype == LSURGE_F32, "ragged_dot: out_dtype must be bf16 or f32");
  if (m == 0) return LSURGE_OK;
  LSURGE_REQUIRE(lhs && rhs && group_sizes && out, "ragged_dot: null pointer");
  hipStream_t s = (hipStream_t)stream;
  lsurge::GemmBlocks g;
  int32_t *total, *e_row0, *e_rows;
  if (int rc = ragged_setup(group_sizes, m, e, workspace, workspace_bytes, s, &g, &total, &e_row0, &e_rows)) return rc;
  const bool f32 = out_dtype == LSURGE_F32;
  if (int rc = lsurge::gemm_rows_kn(KID_MISC, g, lhs, kdim, rhs, n, kdim * n, kdim, n, out, n, s, f32)) return rc;
  LSURGE_LAUNCH(KID_MISC, s,
                hipLaunchKernelGGL(zero_rows_from_kernel, dim3(1024), dim3(256), 0, s, out, m, n, f32 ? 4 : 2, total));
  return LSURGE_OK;
}

int lsurge_ragged_dot_bwd(const void* lhs, const void* rhs, const int32_t* group_sizes, const void* g, int64_t m,
                          int64_t kdim, int64_t n, int64_t e, void* dlhs, float* drhs, void* workspace,
                          size_t workspace_bytes, lsurge_stream_t stream) {
  LSURGE_REQUIRE(m >= 0 && e >= 1 && m < (1ll << 31), "ragged_dot_bwd: bad m/e");
  LSURGE_REQUIRE(lhs && rhs && group_sizes && g && dlhs && drhs, "ragged_dot_bwd: null pointer");
  hipStream_t s = (hipStream_t)stream;
  lsurge::GemmBlocks gb;
  int32_t *total, *e_row0, *e_rows;
  if (int rc = ragged_setup(group_sizes, m, e, workspace, workspace_bytes, s, &gb, &total, &e_row0, &e_rows)) return rc;
  // dlhs[r] = g[r] @ rhs[e]^T : rhs[e] is [K, N] = k-major storage of the [N -> K] operand
  if (m > 0) {
    if (int rc = lsurge::gemm_rows_nk(KID_MISC, gb, g, n, rhs, nullptr, 0, n, kdim * n, n, kdim, dlhs, kdim, false,
                                      nullptr, nullptr, 0, s, false))
      return rc;
    LSURGE_LAUNCH(KID_MISC, s,
                  hipLaunchKernelGGL(zero_rows_from_kernel, dim3(1024), dim3(256), 0, s, dlhs, m, kdim, 2, total));
  }
  // drhs[e] = lhs_e^T @ g_e
  return lsurge::gemm_wgrad(KID_MISC, (int)e, e_row0, 1, e_rows, 0, m, lhs, kdim, g, n, kdim, n, drhs, nullptr, 0, n,
                            kdim * n, 1, nullptr, 0, s, lsurge::RowGather());
}

}  // extern "C"
