// Launchers and C ABI of the grouped GEMMs of the MoE layer (the kernels are in gemm_kernels.h): shape checks,
// grid sizes, the split-K reduction of dense weight gradients, and the ragged_dot entry points that replace
// modal/padded_gmm.py:45-69 (padded_ragged_dot and its gather-only VJP).
#include <mutex>

#include "chunk_table.h"
#include "gemm256.h"
#include "gemm_kernels.h"
#include "launchers.h"

namespace {
using namespace lsgemm;

// The tile shape of every grouped GEMM: 128 rows (one padded expert block) x 256 columns, 4 waves of 64 x 128,
// K in 32-deep stages through a 3-stage LDS ring (72 KiB), two workgroups per CU so that one's barrier and
// epilogue overlap the other's MFMAs.
using Cfg = GemmCfg<128, 256, 32, 2, 2, 3, 2>;
constexpr int BM = Cfg::BM, BN = Cfg::BN, BK = Cfg::BK, GT = Cfg::GT;
// Row GEMMs over 256-row tiles (GemmBlocks::tile_rows = 256; the layer's dgrads and its dense shared-expert
// forward): 256 x 256 tiles, 8 waves of 128 x 64 in two ping-pong groups, a 3-stage ring of 32-deep stages
// (96 KiB), one workgroup per CU.  Same MFMA sequence per output element, so the results are bitwise those of Cfg.
using CfgPP = GemmCfg<256, 256, 32, 2, 4, 3, 1, 1>;

// sum of the S split partials in split order -> C (and C2 for n >= n_split).  V = 4: four consecutive columns per
// thread with 16-byte loads and stores (N, n_split, ldc, c_estride multiples of 4, C and C2 16-byte aligned), and
// the S loads of an element group issued before the adds; the same additions in the same order either way.
template <int V>
__global__ void splitk_reduce_kernel(const float* __restrict__ part, int S, int E, int64_t I, int64_t N,
                                     float* __restrict__ C, float* __restrict__ C2, int64_t n_split, int64_t ldc,
                                     int64_t c_estride) {
  typedef float fv __attribute__((ext_vector_type(V)));
  const int64_t total = (int64_t)E * I * N;
  for (int64_t x = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * V; x < total;
       x += (int64_t)gridDim.x * blockDim.x * V) {
    fv v = *reinterpret_cast<const fv*>(part + x);
    int s = 1;
    for (; s + 4 <= S; s += 4) {
      const fv a0 = *reinterpret_cast<const fv*>(part + (int64_t)s * total + x);
      const fv a1 = *reinterpret_cast<const fv*>(part + (int64_t)(s + 1) * total + x);
      const fv a2 = *reinterpret_cast<const fv*>(part + (int64_t)(s + 2) * total + x);
      const fv a3 = *reinterpret_cast<const fv*>(part + (int64_t)(s + 3) * total + x);
      v += a0;
      v += a1;
      v += a2;
      v += a3;
    }
    for (; s < S; ++s) v += *reinterpret_cast<const fv*>(part + (int64_t)s * total + x);
    const int64_t e = x / (I * N), rem = x % (I * N);
    const int64_t row = rem / N, col = rem % N;
    float* dst = (C2 && col >= n_split) ? C2 + e * c_estride + row * ldc + (col - n_split)
                                        : C + e * c_estride + row * ldc + col;
    *reinterpret_cast<fv*>(dst) = v;
  }
}

static int launch_splitk_reduce(const float* part, int S, int E, int64_t I, int64_t N, float* C, float* C2,
                                int64_t n_split, int64_t ldc, int64_t c_estride, hipStream_t s) {
  const int64_t total = (int64_t)E * I * N;
  const bool v4 = N % 4 == 0 && n_split % 4 == 0 && ldc % 4 == 0 && c_estride % 4 == 0 &&
                  ((uintptr_t)C | (uintptr_t)C2 | (uintptr_t)part) % 16 == 0;
  const int64_t items = v4 ? total / 4 : total;
  const unsigned grid = (unsigned)std::min<int64_t>((items + 255) / 256, 8192);
  if (v4)
    LSURGE_LAUNCH(KID_SPLITK_REDUCE, s,
                  hipLaunchKernelGGL(splitk_reduce_kernel<4>, dim3(grid), dim3(256), 0, s, part, S, E, I, N, C, C2,
                                     n_split, ldc, c_estride));
  else
    LSURGE_LAUNCH(KID_SPLITK_REDUCE, s,
                  hipLaunchKernelGGL(splitk_reduce_kernel<1>, dim3(grid), dim3(256), 0, s, part, S, E, I, N, C, C2,
                                     n_split, ldc, c_estride));
  return LSURGE_OK;
}

// Block table of an unpadded ragged layout (rows of group e start at sum_{e'<e} gs[e']), in two launches.  Group
// sizes are clamped so that no group reaches past row m: negative sizes count as 0 and a sum above m is cut at m,
// so a bad group_sizes array can never send the GEMMs outside lhs/out.
// ragged_groups_kernel (one workgroup): clamped group starts and sizes and the exclusive scan of their tr-row
// block counts (tr = 128, or 256 for the ping-pong kernel's tiles), 1024 groups per pass with a running carry; then
// (fill != 0) the block table itself, see fill_block.  Past kRaggedOneLaunchBlocks table entries the table is filled
// by ragged_blocks_fill_kernel's grid instead, so that no thread walks more than 32 entries of it.
constexpr int kRaggedOneLaunchBlocks = 32768;

// block b belongs to the group e with e_boff[e] <= b < e_boff[e + 1] (binary search; empty groups have
// e_boff[e] == e_boff[e + 1]), and entries past the count nb are empty
__device__ __forceinline__ void fill_block(int b, int nb, int E, int tr, const int32_t* __restrict__ e_row0,
                                           const int32_t* __restrict__ e_rows, const int32_t* __restrict__ e_boff,
                                           int32_t* __restrict__ blk_row0, int32_t* __restrict__ blk_rows,
                                           int32_t* __restrict__ blk_expert) {
  if (b >= nb) {
    blk_row0[b] = 0;
    blk_rows[b] = 0;
    blk_expert[b] = -1;
    return;
  }
  int lo = 0, hi = E - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (e_boff[mid] <= b) lo = mid;
    else hi = mid - 1;
  }
  const int j = b - e_boff[lo];
  blk_row0[b] = e_row0[lo] + j * tr;
  blk_rows[b] = min(tr, e_rows[lo] - j * tr);
  blk_expert[b] = lo;
}

__global__ __launch_bounds__(256) void ragged_blocks_fill_kernel(int E, int tr, int max_blocks,
                                                                 const int32_t* __restrict__ e_row0,
                                                                 const int32_t* __restrict__ e_rows,
                                                                 const int32_t* __restrict__ e_boff,
                                                                 const int32_t* __restrict__ num_blocks,
                                                                 int32_t* __restrict__ blk_row0,
                                                                 int32_t* __restrict__ blk_rows,
                                                                 int32_t* __restrict__ blk_expert) {
  const int nb = num_blocks[0];
  for (int b = blockIdx.x * 256 + threadIdx.x; b < max_blocks; b += gridDim.x * 256)
    fill_block(b, nb, E, tr, e_row0, e_rows, e_boff, blk_row0, blk_rows, blk_expert);
}

__global__ __launch_bounds__(1024) void ragged_groups_kernel(const int32_t* __restrict__ gs, int E, int64_t m, int tr,
                                                            int fill, int max_blocks, int32_t* __restrict__ e_row0,
                                                            int32_t* __restrict__ e_rows, int32_t* __restrict__ e_boff,
                                                            int32_t* __restrict__ num_blocks,
                                                            int32_t* __restrict__ total_rows,
                                                            int32_t* __restrict__ blk_row0,
                                                            int32_t* __restrict__ blk_rows,
                                                            int32_t* __restrict__ blk_expert) {
  __shared__ int64_t wsum[16];
  __shared__ int wblk[16];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  int64_t carry_rows = 0;
  int carry_blk = 0;
  for (int base = 0; base < E; base += 1024) {
    const int e = base + tid;
    const int64_t g = e < E ? (int64_t)max(gs[e], 0) : 0;
    int64_t x = g;  // inclusive prefix of the raw sizes within the wave
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int64_t y = __shfl_up(x, o, 64);
      if (lane >= o) x += y;
    }
    if (lane == 63) wsum[w] = x;
    __syncthreads();
    int64_t wb = 0, tot = 0;
    for (int i = 0; i < 16; ++i) {
      if (i < w) wb += wsum[i];
      tot += wsum[i];
    }
    const int64_t incl = carry_rows + wb + x;
    const int64_t row0 = min(incl - g, m), rows = min(incl, m) - row0;
    const int nb = (int)((rows + tr - 1) / tr);
    int xb = nb;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(xb, o, 64);
      if (lane >= o) xb += y;
    }
    __syncthreads();  // everyone has read wsum
    if (lane == 63) wblk[w] = xb;
    __syncthreads();
    int bb = 0, btot = 0;
    for (int i = 0; i < 16; ++i) {
      if (i < w) bb += wblk[i];
      btot += wblk[i];
    }
    if (e < E) {
      e_row0[e] = (int32_t)row0;
      e_rows[e] = (int32_t)rows;
      e_boff[e] = carry_blk + bb + xb - nb;
    }
    carry_rows += tot;
    carry_blk += btot;
    __syncthreads();  // everyone has read wblk before the next pass overwrites it
  }
  if (tid == 0) {
    e_boff[E] = carry_blk;
    num_blocks[0] = min(carry_blk, max_blocks);
    total_rows[0] = (int32_t)min(carry_rows, m);
  }
  if (!fill) return;
  __syncthreads();  // the workgroup's e_row0, e_rows and e_boff writes are visible to all its threads
  const int nb = min(carry_blk, max_blocks);
  for (int b = tid; b < max_blocks; b += 1024)
    fill_block(b, nb, E, tr, e_row0, e_rows, e_boff, blk_row0, blk_rows, blk_expert);
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

// f32 operands on the bf16 matrix cores.  An f32 value x is the sum of three bf16 terms x0 = bf16(x),
// x1 = bf16(x - x0), x2 = bf16(x - x0 - x1) (round to nearest even; each difference is exact in f32): 24 significant
// bits.  The product x y is the sum of the six term products of order <= 2 (x0 y0, x1 y0, x2 y0, x0 y1, x1 y1,
// x0 y2); the three left out and the remainder of each split are below 2^-24 |x y|, and every term product is exact
// in the MFMA's f32 accumulation.  Laid side by side along a GEMM's reduction dimension, the six products are one
// bf16 GEMM of six times the depth.  Term j of a split row is term ((pattern >> 2j) & 3) of the f32 row; the two
// patterns below pair up as (t_j, s_j) = (0,0) (1,0) (2,0) (0,1) (1,1) (0,2).
constexpr uint32_t kSplitT = 0u | 1u << 2 | 2u << 4 | 0u << 6 | 1u << 8 | 0u << 10;  // terms 0 1 2 0 1 0
constexpr uint32_t kSplitS = 0u | 0u << 2 | 0u << 4 | 1u << 6 | 1u << 8 | 2u << 10;  // terms 0 0 0 1 1 2

// x [rows, cols] f32 -> out [rows, 6 cols] bf16: out[r, j cols + c] = term ((PAT >> 2j) & 3) of x[r, c].  cols % 4 == 0
// and x 16-byte aligned; one float4 per lane and step, six 8-byte stores (HBM-bound: 4 bytes in, 12 out per value).
template <uint32_t PAT>
__global__ __launch_bounds__(256) void split3_bf16_kernel(const float* __restrict__ x, int64_t rows, int64_t cols,
                                                          bf16_t* __restrict__ out) {
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  const int64_t c4n = cols / 4;
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    const float4* __restrict__ xr = reinterpret_cast<const float4*>(x + r * cols);
    bf16_t* __restrict__ orow = out + r * 6 * cols;
    for (int64_t c4 = (int64_t)blockIdx.x * 256 + threadIdx.x; c4 < c4n; c4 += (int64_t)gridDim.x * 256) {
      const float4 v = xr[c4];
      float rem[4] = {v.x, v.y, v.z, v.w};
      u32x2 t[3];
#pragma unroll
      for (int q = 0; q < 3; ++q) {
        t[q] = u32x2{pack_bf16x2(rem[0], rem[1]), pack_bf16x2(rem[2], rem[3])};
        rem[0] -= __uint_as_float(t[q][0] << 16);
        rem[1] -= __uint_as_float(t[q][0] & 0xffff0000u);
        rem[2] -= __uint_as_float(t[q][1] << 16);
        rem[3] -= __uint_as_float(t[q][1] & 0xffff0000u);
      }
#pragma unroll
      for (int j = 0; j < 6; ++j)
        *reinterpret_cast<u32x2*>(orow + j * cols + 4 * c4) = t[(PAT >> (2 * j)) & 3];
    }
  }
}

// group sizes times f (the row counts of the split weight gradient)
__global__ void scale_counts_kernel(const int32_t* __restrict__ gs, int e, int f, int32_t* __restrict__ out) {
  for (int i = threadIdx.x; i < e; i += blockDim.x) out[i] = gs[i] * f;
}

inline unsigned pad8(int64_t g) { return (unsigned)((g + 7) / 8 * 8); }

// Chunk table of the routed weight gradients (one workgroup of 512 threads, thread e = expert e).  Expert e owns
// rows [row0_mult block_off[e], row0_mult block_off[e] + gs[e]) (row0_mult = 128 for the padded layout, 1 for a
// ragged one); they are cut into ceil(gs[e] / R) chunks of R rows.
// An optional extra expert (id E: the shared expert) owns x_rows rows from padded row x_row0.  An empty expert
// keeps one empty chunk, which writes its zero gradient.  An expert with more than one chunk gets consecutive
// partial slots (summed in chunk order by wgrad_chunk_reduce_kernel) and an entry in split_list (ascending e).
// The bounds max_chunks >= E' + ceil(M' / R) and max_parts >= 2 M' / R (E', M': experts and rows including the
// extra one) hold for any group sizes that sum to at most M; if the slots would not fit anyway (corrupt sizes),
// every expert is left as one unsplit chunk.
constexpr int WC_THREADS = 512;
__device__ __forceinline__ int block_excl_scan(int v, int* sh) {  // WC_THREADS threads; returns the exclusive prefix
  constexpr int NWV = WC_THREADS / 64;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) sh[w] = x;
  __syncthreads();
  int base = 0, total = 0;
  for (int i = 0; i < NWV; ++i) {
    if (i < w) base += sh[i];
    total += sh[i];
  }
  __syncthreads();
  if (tid == 0) sh[NWV] = total;
  __syncthreads();
  return base + x - v;
}

__global__ __launch_bounds__(WC_THREADS) void wgrad_chunks_kernel(const int32_t* __restrict__ gs,
                                                                   const int32_t* __restrict__ block_off,
                                                                   int row0_mult, int E, lsurge::ChunkTableOut o) {
  __shared__ int sh[WC_THREADS / 64 + 1];
  constexpr int TOT = WC_THREADS / 64;
  lsurge::write_chunk_table(
      o, E, [&](int e) { return gs[e]; }, [&](int e) { return block_off[e] * row0_mult; },
      [&](int v, int* total) {
        const int base = block_excl_scan(v, sh);
        *total = sh[TOT];
        return base;
      });
}

// dW of each split expert = its chunk partials summed in chunk order (f32, deterministic), -> C (and C2 for
// columns >= n_split).  Grid-stride over (split expert, 4-element group).
__global__ void wgrad_chunk_reduce_kernel(const float* __restrict__ part, const int32_t* __restrict__ split_list,
                                          const int32_t* __restrict__ num_split, const int32_t* __restrict__ e_pbase,
                                          const int32_t* __restrict__ e_nparts, int64_t I, int64_t N,
                                          float* __restrict__ C, float* __restrict__ C2, int64_t n_split, int64_t ldc,
                                          int64_t c_estride, int x_expert, float* __restrict__ Cx,
                                          float* __restrict__ C2x) {
  const int64_t IN = I * N, q4 = IN / 4;
  const int64_t total = (int64_t)num_split[0] * q4;
  for (int64_t x = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; x < total; x += (int64_t)gridDim.x * blockDim.x) {
    const int e = split_list[x / q4];
    const int64_t o = (x % q4) * 4;
    const float* p0 = part + (int64_t)e_pbase[e] * IN + o;
    f32x4 v = *reinterpret_cast<const f32x4*>(p0);
    const int np = e_nparts[e];
    int q = 1;
    for (; q + 4 <= np; q += 4) {  // four partials in flight, added in order
      const f32x4 a0 = *reinterpret_cast<const f32x4*>(p0 + (int64_t)q * IN);
      const f32x4 a1 = *reinterpret_cast<const f32x4*>(p0 + (int64_t)(q + 1) * IN);
      const f32x4 a2 = *reinterpret_cast<const f32x4*>(p0 + (int64_t)(q + 2) * IN);
      const f32x4 a3 = *reinterpret_cast<const f32x4*>(p0 + (int64_t)(q + 3) * IN);
      v += a0;
      v += a1;
      v += a2;
      v += a3;
    }
    for (; q < np; ++q) v += *reinterpret_cast<const f32x4*>(p0 + (int64_t)q * IN);
    const int64_t row = o / N, col = o % N;
    float* dst;
    if (e == x_expert) dst = (C2x && col >= n_split) ? C2x + row * ldc + (col - n_split) : Cx + row * ldc + col;
    else dst = (C2 && col >= n_split) ? C2 + e * c_estride + row * ldc + (col - n_split) : C + e * c_estride + row * ldc + col;
    *reinterpret_cast<f32x4*>(dst) = v;
  }
}

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
  return g.blk_expert ? g.max_blocks : (int)((g.dense_rows + g.tile_rows - 1) / g.tile_rows);
}

// launch g256::rows_kernel (the persistent 256 x 256 kernel) over 256-row tiles or dense rows: one workgroup per CU
template <int BMODE, int EPI>
static int launch_rows256(int kid, const GemmBlocks& g, RowsArgs& a, hipStream_t s, int et) {
  constexpr int nout = EPI == EPI_SWIGLU_FWD ? g256::BN / 2 : g256::BN;
  a.max_tiles = max_blocks_of(g);
  a.n_tiles = (int)((a.N + nout - 1) / nout);
  if (a.max_tiles == 0) return LSURGE_OK;
  const dim3 grid(g256::NWG), block(256);
  const bool f16 = et == LSURGE_F16, f32out = a.Cf != nullptr;
  // the epilogue's buffer descriptors span one tile's rows of each output
  if (int rc = check_desc((int64_t)g256::BM * a.ldc * (f32out ? 4 : 2), "grouped GEMM output")) return rc;
  if (int rc = check_desc((int64_t)g256::BM * a.ldg * 2, "grouped GEMM g / u")) return rc;
  if constexpr (EPI == EPI_SWIGLU_FWD) {
    if (a.a_rows) LSURGE_LAUNCH(kid, s, hipLaunchKernelGGL((g256::rows_kernel<BMODE, EPI, true>), grid, block, 0, s, a));
    else LSURGE_LAUNCH(kid, s, hipLaunchKernelGGL((g256::rows_kernel<BMODE, EPI, false>), grid, block, 0, s, a));
  } else if constexpr (EPI == EPI_SWIGLU_BWD) {
    if (a.a_rows) LSURGE_LAUNCH(kid, s, hipLaunchKernelGGL((g256::rows_kernel<BMODE, EPI, true>), grid, block, 0, s, a));
    else LSURGE_LAUNCH(kid, s, hipLaunchKernelGGL((g256::rows_kernel<BMODE, EPI, false>), grid, block, 0, s, a));
  } else {
    LSURGE_REQUIRE(!a.a_rows, "grouped GEMM: no row gather with the plain store");
    if (f16 && f32out)
      LSURGE_LAUNCH(kid, s, hipLaunchKernelGGL((g256::rows_kernel<BMODE, EPI, false, LSURGE_F16, true>), grid, block, 0, s, a));
    else if (f16)
      LSURGE_LAUNCH(kid, s, hipLaunchKernelGGL((g256::rows_kernel<BMODE, EPI, false, LSURGE_F16, false>), grid, block, 0, s, a));
    else if (f32out)
      LSURGE_LAUNCH(kid, s, hipLaunchKernelGGL((g256::rows_kernel<BMODE, EPI, false, LSURGE_BF16, true>), grid, block, 0, s, a));
    else
      LSURGE_LAUNCH(kid, s, hipLaunchKernelGGL((g256::rows_kernel<BMODE, EPI, false, LSURGE_BF16, false>), grid, block, 0, s, a));
  }
  return LSURGE_OK;
}

// launch gemm_rows_kernel with the tile config that matches the row tiles of g (column tiles: BN output columns, or
// BN / 2 for the SwiGLU forward); 256-row tiles of bf16 / f16 operands go to the persistent kernel when it is selected
template <int BMODE, int EPI, int F8 = 0>
static int launch_rows(int kid, const GemmBlocks& g, RowsArgs& a, hipStream_t s, int et = LSURGE_BF16) {
  if constexpr (!F8) {
    if (gemm_variant() == LSURGE_GEMM_G256 && g.tile_rows == 256 && !a.amax && a.k_split % g256::BK == 0)
      return launch_rows256<BMODE, EPI>(kid, g, a, s, et);
  }
  LSURGE_REQUIRE(g.tile_rows == 128 || g.tile_rows == 256, "grouped GEMM: tile_rows=%d must be 128 or 256", g.tile_rows);
  a.max_tiles = max_blocks_of(g);
  a.n_tiles = (int)((a.N + (EPI == EPI_SWIGLU_FWD ? BN / 2 : BN) - 1) / (EPI == EPI_SWIGLU_FWD ? BN / 2 : BN));
  if (a.max_tiles == 0) return LSURGE_OK;
  const dim3 grid(pad8((int64_t)a.n_tiles * a.max_tiles));
  // FP8: 256-row tiles on the ping-pong kernel, 128-row tiles on the 4-wave kernel with the single-buffered K loop
  if constexpr (EPI == EPI_STORE && !F8) {
    if (et == LSURGE_F16) {  // f16 operands (the ragged_dot entry points): 4-wave kernel
      LSURGE_REQUIRE(g.tile_rows == 128, "grouped GEMM: f16 operands take 128-row tiles");
      LSURGE_LAUNCH(kid, s, hipLaunchKernelGGL((gemm_rows_kernel<Cfg, BMODE, EPI, false, LSURGE_F16>), grid,
                                               dim3(Cfg::GT), 0, s, a));
      return LSURGE_OK;
    }
  }
  LSURGE_REQUIRE(et == LSURGE_BF16 || (EPI == EPI_STORE && !F8), "grouped GEMM: f16 operands need the plain epilogue");
  if constexpr (F8) {
    if (g.tile_rows == 256)
      LSURGE_LAUNCH(kid, s, hipLaunchKernelGGL((gemm_rows_kernel<CfgPP, BMODE, EPI, F8>), grid, dim3(CfgPP::GT), 0, s, a));
    else
      LSURGE_LAUNCH(kid, s, hipLaunchKernelGGL((gemm_rows_kernel<Cfg, BMODE, EPI, F8>), grid, dim3(Cfg::GT), 0, s, a));
  } else if (g.tile_rows == 256)
    LSURGE_LAUNCH(kid, s, hipLaunchKernelGGL((gemm_rows_kernel<CfgPP, BMODE, EPI>), grid, dim3(CfgPP::GT), 0, s, a));
  else
    LSURGE_LAUNCH(kid, s, hipLaunchKernelGGL((gemm_rows_kernel<Cfg, BMODE, EPI>), grid, dim3(Cfg::GT), 0, s, a));
  return LSURGE_OK;
}

// C[rows, N] = A[rows, K] @ B_e where B_e is [K, N] (n-major) -- forward projections
int gemm_rows_kn(int kid, const GemmBlocks& g, const void* A, int64_t lda, const void* B, int64_t ldb,
                 int64_t b_estride, int64_t K, int64_t N, void* C, int64_t ldc, hipStream_t s, bool out_f32,
                 const ExtraExpert& xe, int et) {
  if (int rc = check_gemm_shape(K, N, "gemm_rows_kn")) return rc;
  if (int rc = check_desc(std::max<int64_t>(g.tile_rows * lda, K * ldb) * 2, "gemm_rows_kn")) return rc;
  RowsArgs a{};
  a.A = (const bf16_t*)A; a.lda = lda; a.B = (const bf16_t*)B; a.ldb = ldb; a.b_estride = b_estride;
  a.K = K; a.N = N; a.ldc = ldc;
  if (out_f32) a.Cf = (float*)C;
  else a.C = (bf16_t*)C;
  a.t_expert = g.blk_expert; a.t_rows = g.blk_rows; a.t_row0 = g.blk_row0; a.num_tiles = g.num_blocks;
  a.dense_rows = g.dense_rows;
  a.x_expert = xe.expert; a.Bx = (const bf16_t*)xe.B; a.B2x = (const bf16_t*)xe.B2;
  LSURGE_REQUIRE(xe.expert < 0 || (xe.B && (xe.B2 || !a.B2)), "grouped GEMM: extra expert weights missing");
  return launch_rows<B_KN, EPI_STORE>(kid, g, a, s, et);
}

// h = silu(A @ Bg) * (A @ Bu); also stores g, u.  Bg, Bu: [K, N] per expert.  With a gather (gather.rows set),
// tile row r reads A[gather.rows[row0 + r] / gather.div] of an A with gather.nrows rows (negative: zero row).
int gemm_rows_swiglu_fwd(int kid, const GemmBlocks& g, const void* A, int64_t lda, const void* Bg, const void* Bu,
                         int64_t ldb, int64_t b_estride, int64_t K, int64_t N, void* H, void* Gs, void* Us,
                         int64_t ldh, hipStream_t s, const RowGather& gather, const ExtraExpert& xe) {
  if (int rc = check_gemm_shape(K, N, "gemm_rows_swiglu_fwd")) return rc;
  if (int rc = check_desc(std::max<int64_t>(g.tile_rows * lda, K * ldb) * 2, "gemm_rows_swiglu_fwd")) return rc;
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
  a.dense_rows = g.dense_rows;
  a.x_expert = xe.expert; a.Bx = (const bf16_t*)xe.B; a.B2x = (const bf16_t*)xe.B2;
  LSURGE_REQUIRE(xe.expert < 0 || (xe.B && (xe.B2 || !a.B2)), "grouped GEMM: extra expert weights missing");
  return launch_rows<B_KN, EPI_SWIGLU_FWD>(kid, g, a, s);
}

// C[rows, N] = A[rows, K] @ B_e^T where B_e is stored [N, K] (k-major); with B2 and k_split the K range
// [k_split, K) reads B2 (gate/up dgrad: A = [dG | dU], B = W_gate, B2 = W_up, k_split = f).
// swiglu_bwd: C = [dG | dU] from dH = A @ B^T and the saved G, U (ldg pitch); with row_scale, dH row r is first
// multiplied by row_scale[r] (padded row; tiles of xe.expert: 1).  A row gather (gather.rows set) as in
// gemm_rows_swiglu_fwd.
int gemm_rows_nk(int kid, const GemmBlocks& g, const void* A, int64_t lda, const void* B, const void* B2,
                 int64_t k_split, int64_t ldb, int64_t b_estride, int64_t K, int64_t N, void* C, int64_t ldc,
                 bool swiglu_bwd, const void* Gs, const void* Us, int64_t ldg, hipStream_t s, bool out_f32,
                 const ExtraExpert& xe, int et, const RowGather& gather, const float* row_scale) {
  if (int rc = check_gemm_shape(K, N, "gemm_rows_nk")) return rc;
  if (int rc = check_desc(std::max<int64_t>(g.tile_rows * lda, N * ldb) * 2, "gemm_rows_nk")) return rc;
  LSURGE_REQUIRE(!B2 || (k_split > 0 && k_split % BK == 0), "gemm_rows_nk: k_split must be a multiple of %d", BK);
  LSURGE_REQUIRE(!row_scale || swiglu_bwd, "gemm_rows_nk: row_scale is for the SwiGLU backward");
  LSURGE_REQUIRE(!gather.rows || et == LSURGE_BF16, "gemm_rows_nk: the row gather takes bf16 operands");
  if (gather.rows) {
    LSURGE_REQUIRE(gather.div >= 1 && gather.nrows >= 1, "gemm_rows_nk: bad row gather");
    if (int rc = check_desc(gather.nrows * lda * 2, "gemm_rows_nk gather")) return rc;
  }
  RowsArgs a{};
  a.a_rows = gather.rows; a.a_nrows = gather.nrows; a.a_div = gather.div;
  a.row_scale = row_scale;
  a.A = (const bf16_t*)A; a.lda = lda; a.B = (const bf16_t*)B; a.B2 = (const bf16_t*)B2; a.k_split = B2 ? k_split : 0;
  a.ldb = ldb; a.b_estride = b_estride; a.K = K; a.N = N; a.ldc = ldc;
  if (out_f32 && !swiglu_bwd) a.Cf = (float*)C;
  else a.C = (bf16_t*)C;
  a.G = (bf16_t*)Gs; a.U = (bf16_t*)Us; a.ldg = ldg;
  a.t_expert = g.blk_expert; a.t_rows = g.blk_rows; a.t_row0 = g.blk_row0; a.num_tiles = g.num_blocks;
  a.dense_rows = g.dense_rows;
  a.x_expert = xe.expert; a.Bx = (const bf16_t*)xe.B; a.B2x = (const bf16_t*)xe.B2;
  LSURGE_REQUIRE(xe.expert < 0 || (xe.B && (xe.B2 || !a.B2)), "grouped GEMM: extra expert weights missing");
  return swiglu_bwd ? launch_rows<B_NK, EPI_SWIGLU_BWD>(kid, g, a, s, et) : launch_rows<B_NK, EPI_STORE>(kid, g, a, s, et);
}

// FP8 row GEMM: C[rows, N] = (A[rows, K] @ B_e^T) * a_sinv[0] * b_sinv[e], B_e = [N, K] in E4M3 and A in E4M3 (or
// E5M2 with a_e5m2: a gradient), both K contiguous, pitches lda / ldb and expert stride in bytes.
//   F8_SWIGLU_FWD: B2 holds the up rows (scaled by b2_sinv[e]), C = h = silu(g) * u, Gs / Us (optional) receive g and
//                  u, and amax (optional) the max |h| as bf16-rounded float bits (atomic max: the caller zeroes it).
//   F8_SWIGLU_BWD: the product is dH; C = [dG | dU] (pitch ldc >= 2N) from the saved Gs, Us (pitch N), and amax
//                  (optional) receives max(|dG|, |dU|) as for the forward.
//   F8_STORE:      C (bf16) or Cf (f32) is the product; with k_split, K columns [k_split, K) read B2 (at k - k_split)
//                  with its own per-expert scale b2_sinv (the gate/up dgrad over [dG | dU]).
int gemm_rows_f8(int kid, const GemmBlocks& g, const void* A, int64_t lda, const float* a_sinv, const void* B,
                 const void* B2, int64_t ldb, int64_t b_estride, const float* b_sinv, const float* b2_sinv, int64_t K,
                 int64_t N, void* C, int64_t ldc, bool out_f32, int epi, void* Gs, void* Us, uint32_t* amax,
                 hipStream_t s, const RowGather& gather, int64_t k_split, bool a_e5m2) {
  const bool swiglu = epi == F8_SWIGLU_FWD, sbwd = epi == F8_SWIGLU_BWD;
  LSURGE_REQUIRE(epi == F8_STORE || swiglu || sbwd, "gemm_rows_f8: bad epilogue %d", epi);
  const int64_t kb = k_split ? k_split : K;  // K extent of one B matrix
  LSURGE_REQUIRE(K > 0 && N > 0 && K % 16 == 0 && N % 8 == 0 && lda % 16 == 0 && ldb % 16 == 0 && lda >= K && ldb >= kb,
                 "gemm_rows_f8: K=%lld (multiple of 16), N=%lld (multiple of 8), lda=%lld, ldb=%lld (multiples of 16, >= K)",
                 (long long)K, (long long)N, (long long)lda, (long long)ldb);
  LSURGE_REQUIRE(A && B && C && a_sinv && b_sinv && (!swiglu || (B2 && b2_sinv)) && (!sbwd || (Gs && Us)),
                 "gemm_rows_f8: null pointer");
  LSURGE_REQUIRE(!k_split || (epi == F8_STORE && B2 && b2_sinv && k_split % 64 == 0 && 2 * k_split == K),
                 "gemm_rows_f8: k_split=%lld must be K / 2 and a multiple of 64, with B2 and its scales",
                 (long long)k_split);
  LSURGE_REQUIRE(!a_e5m2 || !swiglu, "gemm_rows_f8: the SwiGLU forward takes E4M3 activations");
  LSURGE_REQUIRE(((uintptr_t)A | (uintptr_t)B | (uintptr_t)B2 | (uintptr_t)(b_estride)) % 16 == 0,
                 "gemm_rows_f8: operands and the expert stride must be 16-byte aligned");
  LSURGE_REQUIRE(!(swiglu || sbwd) || !out_f32, "gemm_rows_f8: the SwiGLU epilogues write bf16");
  LSURGE_REQUIRE(!sbwd || ldc >= 2 * N, "gemm_rows_f8: the SwiGLU backward writes [dG | dU] rows of 2N");
  if (int rc = check_desc(std::max<int64_t>(g.tile_rows * lda, N * ldb), "gemm_rows_f8")) return rc;
  if (gather.rows) {
    LSURGE_REQUIRE(gather.div >= 1 && gather.nrows >= 1, "gemm_rows_f8: bad row gather");
    if (int rc = check_desc(gather.nrows * lda, "gemm_rows_f8 gather")) return rc;
  }
  RowsArgs a{};
  a.a_rows = gather.rows; a.a_nrows = gather.nrows; a.a_div = gather.div;
  a.A = (const bf16_t*)A; a.lda = lda; a.B = (const bf16_t*)B; a.B2 = (const bf16_t*)B2; a.ldb = ldb;
  a.b_estride = b_estride; a.K = K; a.N = N; a.ldc = ldc;
  if (out_f32) a.Cf = (float*)C;
  else a.C = (bf16_t*)C;
  a.G = (bf16_t*)Gs; a.U = (bf16_t*)Us; a.ldg = sbwd ? N : ldc;
  a.k_split = k_split;
  a.t_expert = g.blk_expert; a.t_rows = g.blk_rows; a.t_row0 = g.blk_row0; a.num_tiles = g.num_blocks;
  a.dense_rows = g.dense_rows;
  a.a_sinv = a_sinv; a.b_sinv = b_sinv; a.b2_sinv = b2_sinv; a.amax = amax;
  if (swiglu) return launch_rows<B_NK, EPI_SWIGLU_FWD, 1>(kid, g, a, s);
  if (sbwd) return a_e5m2 ? launch_rows<B_NK, EPI_SWIGLU_BWD, 2>(kid, g, a, s) : launch_rows<B_NK, EPI_SWIGLU_BWD, 1>(kid, g, a, s);
  return a_e5m2 ? launch_rows<B_NK, EPI_STORE, 2>(kid, g, a, s) : launch_rows<B_NK, EPI_STORE, 1>(kid, g, a, s);
}

size_t wgrad_workspace_bytes(int E, int64_t I, int64_t N, int S) {
  return S > 1 ? sizeof(float) * (size_t)S * E * I * N : 0;
}

// C_e[I, N] = A_e^T @ B_e over the rows of expert e; columns >= n_split go to C2 (if given).  max_rows bounds
// the rows of any one expert (the dense row count, or the token count for routed rows).
int gemm_wgrad(int kid, int E, const int32_t* e_row0, int row0_mult, const int32_t* e_rows, int64_t dense_rows,
               int64_t max_rows, const void* A, int64_t lda, const void* B, int64_t ldb, int64_t I, int64_t N, float* C,
               float* C2, int64_t n_split, int64_t ldc, int64_t c_estride, int S, void* ws, size_t ws_bytes,
               hipStream_t s, const RowGather& gather, int et) {
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
  if (et == LSURGE_F16)
    LSURGE_LAUNCH(kid, s, hipLaunchKernelGGL((gemm_wgrad_kernel<Cfg, LSURGE_F16>), dim3(pad8(tiles)), dim3(GT), 0, s, a));
  else
    LSURGE_LAUNCH(kid, s, hipLaunchKernelGGL(gemm_wgrad_kernel<Cfg>, dim3(pad8(tiles)), dim3(GT), 0, s, a));
  if (S > 1) return launch_splitk_reduce((const float*)ws, S, E, I, N, C, C2, n_split, ldc, c_estride, s);
  return LSURGE_OK;
}

WgradChunkPlan wgrad_chunk_plan(int64_t M, int64_t E) {
  WgradChunkPlan p;
  // R: at least 2048 rows and 1.5 x the mean expert load, so balanced routings keep one chunk per routed expert,
  // while a hot expert (or the shared expert's rows) is cut into chunks near the routed ones' size, which keeps the
  // XCDs' shares of the launch even.  (A floor of M / 32 rows made C2's shared-expert chunks 3584 rows against
  // 1536-row routed ones; without it the C2 / C3 weight gradients run 1-7% faster.)  At most 2 M / R partial slots.
  const int64_t mean15 = ((3 * M + 2 * E - 1) / (2 * E) + BM - 1) / BM * BM;  // 1.5 x the mean load, in blocks
  p.R = (int)std::max<int64_t>(2048, mean15);
  p.max_chunks = (int)(E + (M + p.R - 1) / p.R);
  p.max_parts = (int)std::max<int64_t>(1, (2 * M + p.R - 1) / p.R);
  return p;
}

WgradChunkPlan wgrad_chunk_plan_dense(int64_t M, int64_t I, int64_t N) {
  WgradChunkPlan p;
  const int64_t tiles = ((I + g256::BM - 1) / g256::BM) * ((N + g256::BN - 1) / g256::BN);
  const int64_t n = std::max<int64_t>(1, std::min<int64_t>({(g256::NWG + tiles - 1) / tiles, 16, M / 1024}));
  p.R = (int)std::max<int64_t>(BM, ((M + n - 1) / n + BM - 1) / BM * BM);
  p.max_chunks = (int)std::max<int64_t>(1, (M + p.R - 1) / p.R);
  p.max_parts = p.max_chunks;
  return p;
}

size_t wgrad_chunk_table_ints(const WgradChunkPlan& p, int64_t E) {
  return 4 * (size_t)p.max_chunks + 2 * (size_t)(E + 1) + (size_t)p.max_parts + 2;
}

ChunkTableOut chunk_table_out(int32_t* table, int E, const WgradChunkPlan& p, int64_t x_rows, int64_t x_row0) {
  ChunkTableOut o;
  int32_t* t = table;
  o.c_expert = t; t += p.max_chunks;
  o.c_row0 = t; t += p.max_chunks;
  o.c_rows = t; t += p.max_chunks;
  o.c_part = t; t += p.max_chunks;
  o.e_pbase = t; t += E + 1;
  o.e_nparts = t; t += E + 1;
  o.split_list = t; t += p.max_parts;
  o.num_chunks = t;
  o.num_split = t + 1;
  o.R = p.R;
  o.max_chunks = p.max_chunks;
  o.max_parts = p.max_parts;
  o.x_rows = (int)x_rows;
  o.x_row0 = (int)x_row0;
  return o;
}

WgradChunks chunk_table_view(const ChunkTableOut& o) {
  WgradChunks ch;
  ch.c_expert = o.c_expert;
  ch.c_row0 = o.c_row0;
  ch.c_rows = o.c_rows;
  ch.c_part = o.c_part;
  ch.num_chunks = o.num_chunks;
  ch.e_pbase = o.e_pbase;
  ch.e_nparts = o.e_nparts;
  ch.split_list = o.split_list;
  ch.num_split = o.num_split;
  ch.max_chunks = o.max_chunks;
  ch.max_parts = o.max_parts;
  return ch;
}

int build_wgrad_chunks(const int32_t* gs, const int32_t* block_off, int E, const WgradChunkPlan& p, int32_t* table,
                       WgradChunks* ch, hipStream_t s, int64_t x_rows, int64_t x_row0, int row0_mult) {
  LSURGE_REQUIRE((E >= 1 && E <= 256) || (E == 0 && x_rows >= 0), "wgrad chunks: E=%d must be in [1, 256] (0 with "
                 "an extra expert)", E);
  LSURGE_REQUIRE(E == 0 || (gs && block_off), "wgrad chunks: null group sizes");
  LSURGE_REQUIRE(x_rows < (1ll << 31) && x_row0 >= 0 && x_row0 < (1ll << 31), "wgrad chunks: extra expert rows");
  const ChunkTableOut o = chunk_table_out(table, E, p, x_rows, x_row0);
  *ch = chunk_table_view(o);
  LSURGE_LAUNCH(KID_MISC, s,
                hipLaunchKernelGGL(wgrad_chunks_kernel, dim3(1), dim3(WC_THREADS), 0, s, gs, block_off, row0_mult, E, o));
  return LSURGE_OK;
}

size_t wgrad_chunked_workspace_bytes(const WgradChunkPlan& p, int64_t I, int64_t N) {
  return sizeof(float) * (size_t)p.max_parts * I * N;
}

// C_e[I, N] = A_e^T @ B_e over the chunks of a chunk table (see WgradArgs); split experts are summed from their
// partials afterwards.  max_rows bounds the rows of any one chunk (the token count for routed rows: a chunk never
// spans more rows than its expert, and a token picks an expert at most once).
int gemm_wgrad_chunked(int kid, const WgradChunks& ch, int E, int64_t max_rows, const void* A, int64_t lda,
                       const void* B, int64_t ldb, int64_t I, int64_t N, float* C, float* C2, int64_t n_split,
                       int64_t ldc, int64_t c_estride, void* part, size_t part_bytes, hipStream_t s,
                       const RowGather& gather, const ExtraOut& xo, int et) {
  if (int rc = check_gemm_shape(I, N, "gemm_wgrad_chunked")) return rc;
  LSURGE_REQUIRE(xo.expert < 0 || (xo.C && (xo.C2 || !C2)), "gemm_wgrad_chunked: extra expert outputs missing");
  if (int rc = check_desc(max_rows * std::max(lda, ldb) * 2, "gemm_wgrad_chunked")) return rc;
  LSURGE_REQUIRE((E >= 1 || (E == 0 && xo.expert == 0)) && ch.max_chunks >= 1, "gemm_wgrad_chunked: bad E / chunk table");
  LSURGE_REQUIRE(part && part_bytes >= sizeof(float) * (size_t)ch.max_parts * I * N,
                 "gemm_wgrad_chunked: partial workspace %zu < %zu bytes", part_bytes,
                 sizeof(float) * (size_t)ch.max_parts * I * N);
  LSURGE_REQUIRE(!C2 || n_split % 4 == 0, "gemm_wgrad_chunked: n_split must be a multiple of 4");
  if (gather.rows) {
    LSURGE_REQUIRE(gather.div >= 1 && gather.nrows >= 1, "gemm_wgrad_chunked: bad row gather");
    if (int rc = check_desc(gather.nrows * (gather.on_b ? ldb : lda) * 2, "gemm_wgrad_chunked gather")) return rc;
  }
  LSURGE_REQUIRE(!gather.on_b || (gather.rows && gather.scale && et == LSURGE_BF16 && gemm_variant() == LSURGE_GEMM_G256),
                 "gemm_wgrad_chunked: the scaled B gather needs bf16 operands, row indices, weights and the persistent "
                 "kernels");
  WgradArgs a{};
  a.a_rows = gather.rows; a.a_nrows = gather.on_b ? 0 : gather.nrows; a.a_div = gather.div;
  a.gather_b = gather.on_b; a.b_nrows = gather.on_b ? gather.nrows : 0; a.b_scale = gather.scale;
  a.A = (const bf16_t*)A; a.lda = lda; a.B = (const bf16_t*)B; a.ldb = ldb; a.I = I; a.N = N; a.C = C; a.C2 = C2;
  a.n_split = n_split; a.ldc = ldc; a.c_estride = c_estride;
  a.E = E; a.S = 1; a.part = (float*)part;
  a.c_expert = ch.c_expert; a.c_row0 = ch.c_row0; a.c_rows = ch.c_rows; a.c_part = ch.c_part;
  a.num_chunks = ch.num_chunks; a.max_chunks = ch.max_chunks;
  a.x_expert = xo.expert; a.Cx = xo.C; a.C2x = xo.C2;
  // The persistent 256 x 256 kernel when a chunk has at least 16 tiles (the gate/up weight gradient: 16 per chunk at
  // d = 1024, 2f = 1024).  With fewer (the down weight gradient: 8 per chunk at f = 512, d = 1024) the persistent
  // grid gets about two tiles per workgroup and the last round leaves most CUs idle; the 4-wave 128 x 256 kernel,
  // whose non-persistent grid the dispatcher balances, measured faster there (176 against 203 us at C2).  Both give
  // the same bits.
  const bool g256_tiles = (int64_t)((I + g256::BM - 1) / g256::BM) * ((N + g256::BN - 1) / g256::BN) >= 16;
  if (gemm_variant() == LSURGE_GEMM_G256 && (g256_tiles || gather.on_b)) {
    // persistent 256 x 256 tiles, one workgroup per CU; the epilogue's descriptors span one tile's rows of an output
    if (int rc = check_desc((int64_t)g256::BM * std::max(N, ldc) * 4, "gemm_wgrad_chunked output")) return rc;
    a.i_tiles = (int)((I + g256::BM - 1) / g256::BM);
    a.n_tiles = (int)((N + g256::BN - 1) / g256::BN);
    const dim3 grid(g256::NWG), block(256);
    if (et == LSURGE_F16) {
      LSURGE_REQUIRE(!a.a_rows, "gemm_wgrad_chunked: no row gather with f16 operands");
      LSURGE_LAUNCH(kid, s, hipLaunchKernelGGL((g256::wgrad_kernel<false, LSURGE_F16>), grid, block, 0, s, a));
    } else if (a.gather_b) {
      LSURGE_LAUNCH(kid, s, hipLaunchKernelGGL((g256::wgrad_kernel<true, LSURGE_BF16, true>), grid, block, 0, s, a));
    } else if (a.a_rows) {
      LSURGE_LAUNCH(kid, s, hipLaunchKernelGGL((g256::wgrad_kernel<true>), grid, block, 0, s, a));
    } else {
      LSURGE_LAUNCH(kid, s, hipLaunchKernelGGL((g256::wgrad_kernel<false>), grid, block, 0, s, a));
    }
  } else {
    a.i_tiles = (int)((I + BM - 1) / BM);
    a.n_tiles = (int)((N + BN - 1) / BN);
    const int64_t tiles = (int64_t)pad8(ch.max_chunks) * a.i_tiles * a.n_tiles;  // see the chunk tile order
    if (et == LSURGE_F16)
      LSURGE_LAUNCH(kid, s, hipLaunchKernelGGL((gemm_wgrad_kernel<Cfg, LSURGE_F16>), dim3((unsigned)tiles), dim3(GT), 0, s, a));
    else
      LSURGE_LAUNCH(kid, s, hipLaunchKernelGGL(gemm_wgrad_kernel<Cfg>, dim3((unsigned)tiles), dim3(GT), 0, s, a));
  }
  // grid-stride over the split experts' elements: two experts' worth of threads per pass
  const unsigned grid = (unsigned)std::min<int64_t>(2 * ((I * N / 4 + 255) / 256), 2048);
  LSURGE_LAUNCH(KID_SPLITK_REDUCE, s,
                hipLaunchKernelGGL(wgrad_chunk_reduce_kernel, dim3(grid), dim3(256), 0, s, (const float*)part,
                                   ch.split_list, ch.num_split, ch.e_pbase, ch.e_nparts, I, N, C, C2, n_split, ldc,
                                   c_estride, xo.expert, xo.C, xo.C2));
  return LSURGE_OK;
}

static int check_wgrad_f8(const void* A, int64_t lda, const float* a_sinv, const void* B, int64_t ldb,
                          const float* b_sinv, int64_t I, int64_t N, float* C, int64_t max_rows, const char* what) {
  LSURGE_REQUIRE(A && B && a_sinv && b_sinv && C, "%s: null pointer", what);
  LSURGE_REQUIRE(I > 0 && N > 0 && I % 16 == 0 && N % 16 == 0 && lda % 16 == 0 && ldb % 16 == 0 && lda >= I &&
                     ldb >= N,
                 "%s: I=%lld N=%lld (multiples of 16), lda=%lld ldb=%lld (multiples of 16, >= I / N)", what,
                 (long long)I, (long long)N, (long long)lda, (long long)ldb);
  LSURGE_REQUIRE(((uintptr_t)A | (uintptr_t)B) % 16 == 0, "%s: operands must be 16-byte aligned", what);
  return check_desc(max_rows * std::max(lda, ldb), what);
}

int gemm_wgrad_f8_chunked(int kid, const WgradChunks& ch, int E, int64_t max_rows, const void* A, int64_t lda,
                          const float* a_sinv, const void* B, int64_t ldb, const float* b_sinv, int64_t I, int64_t N,
                          float* C, float* C2, int64_t n_split, int64_t ldc, int64_t c_estride, void* part,
                          size_t part_bytes, hipStream_t s, const RowGather& gather) {
  if (int rc = check_wgrad_f8(A, lda, a_sinv, B, ldb, b_sinv, I, N, C, max_rows, "gemm_wgrad_f8_chunked")) return rc;
  LSURGE_REQUIRE(E >= 1 && ch.max_chunks >= 1, "gemm_wgrad_f8_chunked: bad E / chunk table");
  LSURGE_REQUIRE(part && part_bytes >= sizeof(float) * (size_t)ch.max_parts * I * N,
                 "gemm_wgrad_f8_chunked: partial workspace %zu < %zu bytes", part_bytes,
                 sizeof(float) * (size_t)ch.max_parts * I * N);
  LSURGE_REQUIRE(!C2 || n_split % 4 == 0, "gemm_wgrad_f8_chunked: n_split must be a multiple of 4");
  if (gather.rows) {
    LSURGE_REQUIRE(gather.div >= 1 && gather.nrows >= 1, "gemm_wgrad_f8_chunked: bad row gather");
    if (int rc = check_desc(gather.nrows * lda, "gemm_wgrad_f8_chunked gather")) return rc;
  }
  WgradArgs a{};
  a.a_rows = gather.rows; a.a_nrows = gather.nrows; a.a_div = gather.div;
  a.A = (const bf16_t*)A; a.lda = lda; a.B = (const bf16_t*)B; a.ldb = ldb; a.I = I; a.N = N; a.C = C; a.C2 = C2;
  a.n_split = n_split; a.ldc = ldc; a.c_estride = c_estride;
  a.E = E; a.S = 1; a.part = (float*)part;
  a.c_expert = ch.c_expert; a.c_row0 = ch.c_row0; a.c_rows = ch.c_rows; a.c_part = ch.c_part;
  a.num_chunks = ch.num_chunks; a.max_chunks = ch.max_chunks;
  a.a_sinv = a_sinv; a.b_sinv = b_sinv;
  a.i_tiles = (int)((I + BM - 1) / BM);
  a.n_tiles = (int)((N + BN - 1) / BN);
  const int64_t tiles = (int64_t)pad8(ch.max_chunks) * a.i_tiles * a.n_tiles;
  LSURGE_LAUNCH(kid, s, hipLaunchKernelGGL((gemm_wgrad_f8_kernel<Cfg, 0, 1>), dim3((unsigned)tiles), dim3(GT), 0, s, a));
  const unsigned grid = (unsigned)std::min<int64_t>(2 * ((I * N / 4 + 255) / 256), 2048);
  LSURGE_LAUNCH(KID_SPLITK_REDUCE, s,
                hipLaunchKernelGGL(wgrad_chunk_reduce_kernel, dim3(grid), dim3(256), 0, s, (const float*)part,
                                   ch.split_list, ch.num_split, ch.e_pbase, ch.e_nparts, I, N, C, C2, n_split, ldc,
                                   c_estride, -1, (float*)nullptr, (float*)nullptr));
  return LSURGE_OK;
}

int gemm_wgrad_f8_dense(int kid, int64_t rows, const void* A, int64_t lda, const float* a_sinv, const void* B,
                        int64_t ldb, const float* b_sinv, int64_t I, int64_t N, float* C, float* C2, int64_t n_split,
                        int64_t ldc, int S, void* ws, size_t ws_bytes, hipStream_t s) {
  if (int rc = check_wgrad_f8(A, lda, a_sinv, B, ldb, b_sinv, I, N, C, rows, "gemm_wgrad_f8_dense")) return rc;
  LSURGE_REQUIRE(rows >= 1 && S >= 1, "gemm_wgrad_f8_dense: rows=%lld, S=%d", (long long)rows, S);
  WgradArgs a{};
  a.A = (const bf16_t*)A; a.lda = lda; a.B = (const bf16_t*)B; a.ldb = ldb; a.I = I; a.N = N; a.C = C; a.C2 = C2;
  a.n_split = n_split; a.ldc = ldc; a.c_estride = 0; a.dense_rows = rows; a.E = 1; a.S = S;
  a.a_sinv = a_sinv; a.b_sinv = b_sinv;
  a.i_tiles = (int)((I + BM - 1) / BM);
  a.n_tiles = (int)((N + BN - 1) / BN);
  if (S > 1) {
    const size_t need = wgrad_workspace_bytes(1, I, N, S);
    LSURGE_REQUIRE(ws && ws_bytes >= need, "gemm_wgrad_f8_dense: workspace %zu < %zu", ws_bytes, need);
    a.part = (float*)ws;
  }
  const int64_t tiles = (int64_t)S * a.i_tiles * a.n_tiles;
  LSURGE_LAUNCH(kid, s, hipLaunchKernelGGL((gemm_wgrad_f8_kernel<Cfg, 0, 1>), dim3(pad8(tiles)), dim3(GT), 0, s, a));
  if (S > 1) return launch_splitk_reduce((const float*)ws, S, 1, I, N, C, C2, n_split, ldc, 0, s);
  return LSURGE_OK;
}

}  // namespace lsurge

// ------------------------------------------------------------------------------ C ABI: ragged_dot
// workspace: blk_row0, blk_rows, blk_expert [max_blocks] | num_blocks, total_rows | e_row0 [e]
extern "C" {

// workspace: blk_row0, blk_rows, blk_expert [max_blocks] | num_blocks, total_rows, 2 spare | e_row0, e_rows [e] |
// e_boff [e + 1]; the backward's chunked weight gradient adds its chunk table and partial slots after that
static size_t ragged_table_ints(int64_t m, int64_t e) { return (size_t)(3 * lsurge_max_blocks(m, e) + 4 + 3 * e + 1); }

size_t lsurge_ragged_dot_workspace_bytes(int64_t m, int64_t e) { return sizeof(int32_t) * ragged_table_ints(m, e); }

// the chunked weight gradient of the backward takes the table's rows as chunks of at most R (hot groups split)
static bool ragged_chunked(int64_t e) { return e >= 1 && e <= 256; }

size_t lsurge_ragged_dot_bwd_workspace_bytes(int64_t m, int64_t kdim, int64_t n, int64_t e) {
  size_t b = lsurge_ragged_dot_workspace_bytes(m, e);
  if (m > 0 && ragged_chunked(e)) {
    const lsurge::WgradChunkPlan p = lsurge::wgrad_chunk_plan(m, e);
    b = (b + 255) / 256 * 256 + sizeof(int32_t) * lsurge::wgrad_chunk_table_ints(p, e);
    b = (b + 255) / 256 * 256 + lsurge::wgrad_chunked_workspace_bytes(p, kdim, n);
  }
  return b;
}

// tile table of a ragged layout: tr = 128 (4-wave kernel) or 256 (ping-pong kernel); the bound
// lsurge_max_blocks(m, e) on 128-row blocks covers both
static int ragged_setup(const int32_t* gs, int64_t m, int64_t e, void* ws, size_t ws_bytes, hipStream_t s,
                        lsurge::GemmBlocks* g, int32_t** total_rows, int32_t** e_row0, int32_t** e_rows, int tr = 128) {
  const size_t need = lsurge_ragged_dot_workspace_bytes(m, e);
  LSURGE_REQUIRE(ws && ws_bytes >= need, "ragged_dot: workspace %zu < %zu bytes", ws_bytes, need);
  LSURGE_REQUIRE(e < (1 << 30), "ragged_dot: e too large");
  const int64_t mb = lsurge_max_blocks(m, e);
  int32_t* p = (int32_t*)ws;
  int32_t* blk_row0 = p;
  int32_t* blk_rows = p + mb;
  int32_t* blk_expert = p + 2 * mb;
  int32_t* nb = p + 3 * mb;
  *total_rows = nb + 1;
  *e_row0 = nb + 4;
  *e_rows = nb + 4 + e;
  int32_t* e_boff = nb + 4 + 2 * e;
  const bool one = mb <= kRaggedOneLaunchBlocks;
  LSURGE_LAUNCH(KID_MISC, s,
                hipLaunchKernelGGL(ragged_groups_kernel, dim3(1), dim3(1024), 0, s, gs, (int)e, m, tr, (int)one,
                                   (int)mb, *e_row0, *e_rows, e_boff, nb, *total_rows, blk_row0, blk_rows, blk_expert));
  if (!one)
    LSURGE_LAUNCH(KID_MISC, s,
                  hipLaunchKernelGGL(ragged_blocks_fill_kernel, dim3((unsigned)std::min<int64_t>((mb + 255) / 256, 4096)),
                                     dim3(256), 0, s, (int)e, tr, (int)mb, *e_row0, *e_rows, e_boff, nb, blk_row0,
                                     blk_rows, blk_expert));
  g->blk_expert = blk_expert;
  g->blk_rows = blk_rows;
  g->blk_row0 = blk_row0;
  g->num_blocks = nb;
  g->max_blocks = (int)mb;
  g->dense_rows = 0;
  g->tile_rows = tr;
  return LSURGE_OK;
}

// row tiles of the bf16 / f16 ragged_dot GEMMs: 256 rows for the persistent kernel, else 128
static int ragged_tile_rows() { return lsurge::gemm_variant() == LSURGE_GEMM_G256 ? 256 : 128; }

// ---- f32 operands: three bf16 terms per value, six term products along a reduction six times as deep (the pairing
// is described at split3_bf16_kernel).
//   forward  out = A' B'      A' [m, 6k] = lhs terms t, B'_e [6k, n] = rhs terms s stacked along k
//   dlhs     dl = G' R''^T    G' [m, 6n] = g terms s,   R''_e [k, 6n] = rhs terms t side by side along n
//   drhs     dr_e = A'_e^T G'_e over 6 gs_e rows: A' and G' read as [6m, k] and [6m, n], whose row 6i + j holds term
//            t_j of lhs row i and term s_j of g row i, so group e owns rows [6 start_e, 6 (start_e + gs_e))
static size_t al256(size_t b) { return (b + 255) / 256 * 256; }
static size_t split_bytes(int64_t rows, int64_t cols) { return al256(12 * (size_t)std::max<int64_t>(0, rows) * cols); }

size_t lsurge_ragged_dot_f32_workspace_bytes(int64_t m, int64_t kdim, int64_t n, int64_t e) {
  return al256(lsurge_ragged_dot_workspace_bytes(m, e)) + split_bytes(m, kdim) + split_bytes(e * kdim, n);
}

// the f32 backward's chunked weight gradient (e <= 256) runs over 6 m rows
static bool f32_bwd_chunked(int64_t m, int64_t e) { return m > 0 && ragged_chunked(e); }

size_t lsurge_ragged_dot_bwd_f32_workspace_bytes(int64_t m, int64_t kdim, int64_t n, int64_t e) {
  size_t b = al256(lsurge_ragged_dot_workspace_bytes(m, e)) + al256(lsurge_ragged_dot_workspace_bytes(6 * m, e)) +
             al256(sizeof(int32_t) * (size_t)std::max<int64_t>(e, 0)) + split_bytes(m, kdim) + split_bytes(m, n) +
             split_bytes(e * kdim, n);
  if (f32_bwd_chunked(m, e)) {
    const lsurge::WgradChunkPlan p = lsurge::wgrad_chunk_plan(6 * m, e);
    b += al256(sizeof(int32_t) * lsurge::wgrad_chunk_table_ints(p, e)) + lsurge::wgrad_chunked_workspace_bytes(p, kdim, n);
  }
  return b;
}

// x [rows, cols] f32 -> [rows, 6 cols] bf16 terms in the order of pattern kSplitT (t) or kSplitS (s)
static int split3(const float* x, int64_t rows, int64_t cols, bool t_terms, bf16_t* out, hipStream_t s) {
  LSURGE_REQUIRE(cols % 4 == 0 && (uintptr_t)x % 16 == 0 && (uintptr_t)out % 16 == 0,
                 "ragged_dot f32: operands must be 16-byte aligned with rows of a multiple of 4 values");
  if (rows == 0) return LSURGE_OK;
  const int64_t c4 = cols / 4;
  const unsigned gx = (unsigned)std::min<int64_t>((c4 + 255) / 256, 1024);
  const unsigned gy = (unsigned)std::min<int64_t>(rows, std::max<int64_t>(1, 8192 / gx));
  if (t_terms)
    LSURGE_LAUNCH(KID_MISC, s, hipLaunchKernelGGL(split3_bf16_kernel<kSplitT>, dim3(gx, gy), dim3(256), 0, s, x, rows,
                                                  cols, out));
  else
    LSURGE_LAUNCH(KID_MISC, s, hipLaunchKernelGGL(split3_bf16_kernel<kSplitS>, dim3(gx, gy), dim3(256), 0, s, x, rows,
                                                  cols, out));
  return LSURGE_OK;
}

static int ragged_dot_f32(const float* lhs, const float* rhs, const int32_t* gs, int64_t m, int64_t kdim, int64_t n,
                          int64_t e, void* out, int out_dtype, void* ws, size_t ws_bytes, hipStream_t s) {
  if (out_dtype != LSURGE_F32 && out_dtype != LSURGE_BF16)
    return lsurge::set_error(LSURGE_ERR_DTYPE, "ragged_dot: out_dtype of f32 operands must be f32 or bf16");
  if (int rc = lsurge::check_gemm_shape(kdim, n, "ragged_dot f32")) return rc;
  const size_t need = lsurge_ragged_dot_f32_workspace_bytes(m, kdim, n, e);
  LSURGE_REQUIRE(ws && ws_bytes >= need, "ragged_dot f32: workspace %zu < %zu bytes", ws_bytes, need);
  char* base = (char*)ws;
  size_t off = al256(lsurge_ragged_dot_workspace_bytes(m, e));
  bf16_t* a2 = (bf16_t*)(base + off);
  off += split_bytes(m, kdim);
  bf16_t* b2 = (bf16_t*)(base + off);
  lsurge::GemmBlocks g;
  int32_t *total, *e_row0, *e_rows;
  if (int rc = ragged_setup(gs, m, e, ws, ws_bytes, s, &g, &total, &e_row0, &e_rows, ragged_tile_rows())) return rc;
  if (int rc = split3(lhs, m, kdim, true, a2, s)) return rc;
  if (int rc = split3(rhs, e, kdim * n, false, b2, s)) return rc;
  const bool f32 = out_dtype == LSURGE_F32;
  if (int rc = lsurge::gemm_rows_kn(KID_MISC, g, a2, 6 * kdim, b2, n, 6 * kdim * n, 6 * kdim, n, out, n, s, f32,
                                    lsurge::ExtraExpert(), LSURGE_BF16))
    return rc;
  LSURGE_LAUNCH(KID_MISC, s,
                hipLaunchKernelGGL(zero_rows_from_kernel, dim3(1024), dim3(256), 0, s, out, m, n, f32 ? 4 : 2, total));
  return LSURGE_OK;
}

static int ragged_dot_bwd_f32(const float* lhs, const float* rhs, const int32_t* gs, const float* g, int64_t m,
                              int64_t kdim, int64_t n, int64_t e, float* dlhs, float* drhs, void* ws, size_t ws_bytes,
                              hipStream_t s) {
  if (int rc = lsurge::check_gemm_shape(kdim, n, "ragged_dot_bwd f32")) return rc;
  LSURGE_REQUIRE(6 * m < (1ll << 31), "ragged_dot_bwd f32: m=%lld too large (6 m rows)", (long long)m);
  const size_t need = lsurge_ragged_dot_bwd_f32_workspace_bytes(m, kdim, n, e);
  LSURGE_REQUIRE(ws && ws_bytes >= need, "ragged_dot_bwd f32: workspace %zu < %zu bytes", ws_bytes, need);
  char* base = (char*)ws;
  const size_t t1 = al256(lsurge_ragged_dot_workspace_bytes(m, e));
  const size_t t6 = al256(lsurge_ragged_dot_workspace_bytes(6 * m, e));
  int32_t* gs6 = (int32_t*)(base + t1 + t6);
  size_t off = t1 + t6 + al256(sizeof(int32_t) * e);
  bf16_t* a2 = (bf16_t*)(base + off);
  off += split_bytes(m, kdim);
  bf16_t* g2 = (bf16_t*)(base + off);
  off += split_bytes(m, n);
  bf16_t* r2 = (bf16_t*)(base + off);
  off += split_bytes(e * kdim, n);
  lsurge::GemmBlocks gb, gb6;
  int32_t *total, *e_row0, *e_rows, *total6, *e_row0_6, *e_rows_6;
  if (int rc = ragged_setup(gs, m, e, base, t1, s, &gb, &total, &e_row0, &e_rows, ragged_tile_rows())) return rc;
  LSURGE_LAUNCH(KID_MISC, s, hipLaunchKernelGGL(scale_counts_kernel, dim3(1), dim3(256), 0, s, gs, (int)e, 6, gs6));
  if (int rc = ragged_setup(gs6, 6 * m, e, base + t1, t6, s, &gb6, &total6, &e_row0_6, &e_rows_6)) return rc;
  if (int rc = split3(lhs, m, kdim, true, a2, s)) return rc;
  if (int rc = split3(g, m, n, false, g2, s)) return rc;
  if (int rc = split3(rhs, e * kdim, n, true, r2, s)) return rc;
  if (m > 0) {
    if (int rc = lsurge::gemm_rows_nk(KID_MISC, gb, g2, 6 * n, r2, nullptr, 0, 6 * n, 6 * kdim * n, 6 * n, kdim, dlhs,
                                      kdim, false, nullptr, nullptr, 0, s, true, lsurge::ExtraExpert(), LSURGE_BF16))
      return rc;
    LSURGE_LAUNCH(KID_MISC, s,
                  hipLaunchKernelGGL(zero_rows_from_kernel, dim3(1024), dim3(256), 0, s, dlhs, m, kdim, 4, total));
  }
  if (f32_bwd_chunked(m, e)) {
    const lsurge::WgradChunkPlan p = lsurge::wgrad_chunk_plan(6 * m, e);
    int32_t* table = (int32_t*)(base + off);
    off += al256(sizeof(int32_t) * lsurge::wgrad_chunk_table_ints(p, e));
    lsurge::WgradChunks ch;
    if (int rc = lsurge::build_wgrad_chunks(e_rows_6, e_row0_6, (int)e, p, table, &ch, s, -1, 0, 1)) return rc;
    return lsurge::gemm_wgrad_chunked(KID_MISC, ch, (int)e, 6 * m, a2, kdim, g2, n, kdim, n, drhs, nullptr, 0, n,
                                      kdim * n, base + off, lsurge::wgrad_chunked_workspace_bytes(p, kdim, n), s,
                                      lsurge::RowGather(), lsurge::ExtraOut(), LSURGE_BF16);
  }
  return lsurge::gemm_wgrad(KID_MISC, (int)e, e_row0_6, 1, e_rows_6, 0, 6 * m, a2, kdim, g2, n, kdim, n, drhs, nullptr,
                            0, n, kdim * n, 1, nullptr, 0, s, lsurge::RowGather(), LSURGE_BF16);
}

int lsurge_ragged_dot(const void* lhs, const void* rhs, const int32_t* group_sizes, int64_t m, int64_t kdim, int64_t n,
                      int64_t e, int in_dtype, void* out, int out_dtype, void* workspace, size_t workspace_bytes,
                      lsurge_stream_t stream) {
  LSURGE_REQUIRE(m >= 0 && e >= 1 && m < (1ll << 31), "ragged_dot: bad m/e");
  if (in_dtype == LSURGE_F32) {
    if (m == 0) return LSURGE_OK;
    LSURGE_REQUIRE(lhs && rhs && group_sizes && out, "ragged_dot: null pointer");
    return ragged_dot_f32((const float*)lhs, (const float*)rhs, group_sizes, m, kdim, n, e, out, out_dtype, workspace,
                          workspace_bytes, (hipStream_t)stream);
  }
  if (in_dtype != LSURGE_BF16 && in_dtype != LSURGE_F16)
    return lsurge::set_error(LSURGE_ERR_DTYPE, "ragged_dot: operands must be f32, bf16 or f16 (got dtype %d)", in_dtype);
  if (out_dtype != in_dtype && out_dtype != LSURGE_F32)
    return lsurge::set_error(LSURGE_ERR_DTYPE, "ragged_dot: out_dtype must be the operand dtype or f32");
  if (m == 0) return LSURGE_OK;
  LSURGE_REQUIRE(lhs && rhs && group_sizes && out, "ragged_dot: null pointer");
  hipStream_t s = (hipStream_t)stream;
  lsurge::GemmBlocks g;
  int32_t *total, *e_row0, *e_rows;
  if (int rc = ragged_setup(group_sizes, m, e, workspace, workspace_bytes, s, &g, &total, &e_row0, &e_rows,
                            ragged_tile_rows()))
    return rc;
  const bool f32 = out_dtype == LSURGE_F32;
  if (int rc = lsurge::gemm_rows_kn(KID_MISC, g, lhs, kdim, rhs, n, kdim * n, kdim, n, out, n, s, f32,
                                    lsurge::ExtraExpert(), in_dtype))
    return rc;
  LSURGE_LAUNCH(KID_MISC, s,
                hipLaunchKernelGGL(zero_rows_from_kernel, dim3(1024), dim3(256), 0, s, out, m, n, f32 ? 4 : 2, total));
  return LSURGE_OK;
}

}  // extern "C"

// ------------------------------------------------------------------------ sustained matrix-core rate (calibration)
// Each wave keeps 8 operand fragments and 16 accumulator blocks (256 registers) resident and issues 64
// v_mfma_f32_32x32x16_bf16 per iteration, the fragments rotating after every 16 so that consecutive MFMAs see other
// data.  Nothing touches memory inside the loop, so the rate is what the matrix cores sustain on such operands; the
// chip's power limit holds it below the datasheet peak for random values.  Operands: pseudo-random bf16 (random sign
// and 7-bit mantissa, exponents 2^-4 .. 2^3, a lowbias32 hash of the element index) or zeros.  out: one f32 per lane
// (the accumulators' sum, so the MFMAs are live).
namespace {
constexpr int kMfmaRateWG = 1024;
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void mfma_rate_kernel(int zero, int iters, float* __restrict__ out) {
  const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
  bf16x8 f[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    u32x4 w;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t h = gid * 32u + (uint32_t)(4 * i + q);
      h ^= h >> 16; h *= 0x7feb352du; h ^= h >> 15; h *= 0x846ca68bu; h ^= h >> 16;
      const uint32_t lo = (h & 0x807fu) | ((123u + ((h >> 7) & 7u)) << 7);
      const uint32_t hi = ((h >> 16) & 0x807fu) | ((123u + ((h >> 23) & 7u)) << 7);
      w[q] = zero ? 0u : (lo | (hi << 16));
    }
    f[i] = lsgemm::as_bf16x8(w);
  }
  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = lsgemm::mfma32(f[4 + j], f[i], acc[i][j]);
      const bf16x8 t = f[0];
#pragma unroll
      for (int i = 0; i < 7; ++i) f[i] = f[i + 1];
      f[7] = t;
    }
  }
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) sum += acc[i][j][e];
  out[gid] = sum;
}
}  // namespace

extern "C" {

size_t lsurge_mfma_rate_probe_out_floats(void) { return (size_t)kMfmaRateWG * 256; }

int lsurge_mfma_rate_probe(int zero_operands, int iters, float* out, lsurge_stream_t stream) {
  LSURGE_REQUIRE(out && iters >= 1 && iters <= (1 << 20), "mfma_rate_probe: null output or iters=%d not in [1, 2^20]",
                 iters);
  hipStream_t s = (hipStream_t)stream;
  LSURGE_LAUNCH(KID_MISC, s,
                hipLaunchKernelGGL(mfma_rate_kernel, dim3(kMfmaRateWG), dim3(256), 0, s, zero_operands ? 1 : 0, iters,
                                   out));
  return LSURGE_OK;
}

}  // extern "C"

// ------------------------------------------------------------------------------ C ABI: ragged_dot without allocation
// The block table of lsurge_ragged_dot_noalloc lives in this file-scope device array instead of a caller workspace.
// Each GPU holds its own copy until the process ends; in host code `scratch` only names the symbol, so kernels get
// the per-device address that hipGetSymbolAddress returns (looked up once per device, with that device current).
// Every entry the table's kernels read is written earlier in the same call, so nothing needs clearing between calls;
// calls that overlap on one GPU (different streams) share the array and race.
namespace {
constexpr int64_t kNoallocMaxRows = 1ll << 21;  // m <= 2^21 rows
constexpr int64_t kNoallocMaxGroups = 1024;     // e <= 1024 groups
constexpr size_t kScratchInts = 3 * (size_t)((kNoallocMaxRows + LSURGE_BLOCK_ROWS - 1) / LSURGE_BLOCK_ROWS +
                                             kNoallocMaxGroups) + 4 + 3 * (size_t)kNoallocMaxGroups + 1;  // 221 KB
__device__ __align__(256) int32_t scratch[kScratchInts];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
int32_t* g_scratch_ptr[kMaxScratchDevices] = {};

// the current device's address of `scratch` (looked up on its first call), or nullptr with the error set
int32_t* scratch_on_current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices) {
    lsurge::set_error(LSURGE_ERR_LAUNCH, "ragged_dot_noalloc: no usable current device");
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int32_t* p = nullptr;
    const hipError_t e = hipGetSymbolAddress((void**)&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      lsurge::set_error(LSURGE_ERR_LAUNCH, "ragged_dot_noalloc: hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}
}  // namespace

extern "C" {

size_t lsurge_ragged_dot_noalloc_max_rows(void) { return (size_t)kNoallocMaxRows; }
size_t lsurge_ragged_dot_noalloc_max_groups(void) { return (size_t)kNoallocMaxGroups; }

int lsurge_ragged_dot_noalloc(const void* lhs, const void* rhs, const int32_t* group_sizes, int64_t m, int64_t kdim,
                              int64_t n, int64_t e, int in_dtype, void* out, int out_dtype, lsurge_stream_t stream) {
  LSURGE_REQUIRE(m >= 0 && m <= kNoallocMaxRows && e >= 1 && e <= kNoallocMaxGroups,
                 "ragged_dot_noalloc: m=%lld e=%lld outside the static scratch (m <= %lld, e <= %lld)", (long long)m,
                 (long long)e, (long long)kNoallocMaxRows, (long long)kNoallocMaxGroups);
  const size_t need = lsurge_ragged_dot_workspace_bytes(m, e);
  LSURGE_REQUIRE(need <= sizeof(int32_t) * kScratchInts, "ragged_dot_noalloc: table of %zu bytes exceeds the scratch",
                 need);
  if (in_dtype == LSURGE_F32)
    return lsurge::set_error(LSURGE_ERR_DTYPE, "ragged_dot_noalloc: f32 operands need the split-term workspace of "
                             "lsurge_ragged_dot");
  if (m == 0) return LSURGE_OK;
  int32_t* ws = scratch_on_current_device();
  if (!ws) return LSURGE_ERR_LAUNCH;
  return lsurge_ragged_dot(lhs, rhs, group_sizes, m, kdim, n, e, in_dtype, out, out_dtype, ws,
                           sizeof(int32_t) * kScratchInts, stream);
}

int lsurge_ragged_dot_fp8(const void* lhs_q, const float* lhs_scale_inv, const void* rhs_q, const float* rhs_scale_inv,
                          const int32_t* group_sizes, int64_t m, int64_t kdim, int64_t n, int64_t e, void* out,
                          int out_dtype, void* workspace, size_t workspace_bytes, lsurge_stream_t stream) {
  LSURGE_REQUIRE(m >= 0 && e >= 1 && m < (1ll << 31), "ragged_dot_fp8: bad m/e");
  LSURGE_REQUIRE(out_dtype == LSURGE_BF16 || out_dtype == LSURGE_F32, "ragged_dot_fp8: out_dtype must be bf16 or f32");
  if (m == 0) return LSURGE_OK;
  LSURGE_REQUIRE(lhs_q && lhs_scale_inv && rhs_q && rhs_scale_inv && group_sizes && out, "ragged_dot_fp8: null pointer");
  hipStream_t s = (hipStream_t)stream;
  lsurge::GemmBlocks g;
  int32_t *total, *e_row0, *e_rows;
  if (int rc = ragged_setup(group_sizes, m, e, workspace, workspace_bytes, s, &g, &total, &e_row0, &e_rows)) return rc;
  const bool f32 = out_dtype == LSURGE_F32;
  if (int rc = lsurge::gemm_rows_f8(KID_MISC, g, lhs_q, kdim, lhs_scale_inv, rhs_q, nullptr, kdim, n * kdim,
                                    rhs_scale_inv, nullptr, kdim, n, out, n, f32, lsurge::F8_STORE, nullptr, nullptr, nullptr, s))
    return rc;
  LSURGE_LAUNCH(KID_MISC, s,
                hipLaunchKernelGGL(zero_rows_from_kernel, dim3(1024), dim3(256), 0, s, out, m, n, f32 ? 4 : 2, total));
  return LSURGE_OK;
}

int lsurge_ragged_dot_bwd(const void* lhs, const void* rhs, const int32_t* group_sizes, const void* g, int64_t m,
                          int64_t kdim, int64_t n, int64_t e, int in_dtype, void* dlhs, float* drhs, void* workspace,
                          size_t workspace_bytes, lsurge_stream_t stream) {
  LSURGE_REQUIRE(m >= 0 && e >= 1 && m < (1ll << 31), "ragged_dot_bwd: bad m/e");
  if (in_dtype != LSURGE_F32 && in_dtype != LSURGE_BF16 && in_dtype != LSURGE_F16)
    return lsurge::set_error(LSURGE_ERR_DTYPE, "ragged_dot_bwd: operands must be f32, bf16 or f16 (got dtype %d)",
                             in_dtype);
  LSURGE_REQUIRE(lhs && rhs && group_sizes && g && dlhs && drhs, "ragged_dot_bwd: null pointer");
  hipStream_t s = (hipStream_t)stream;
  if (in_dtype == LSURGE_F32)
    return ragged_dot_bwd_f32((const float*)lhs, (const float*)rhs, group_sizes, (const float*)g, m, kdim, n, e,
                              (float*)dlhs, drhs, workspace, workspace_bytes, s);
  lsurge::GemmBlocks gb;
  int32_t *total, *e_row0, *e_rows;
  if (int rc = ragged_setup(group_sizes, m, e, workspace, workspace_bytes, s, &gb, &total, &e_row0, &e_rows,
                            ragged_tile_rows()))
    return rc;
  // dlhs[r] = g[r] @ rhs[e]^T : rhs[e] is [K, N] = k-major storage of the [N -> K] operand
  if (m > 0) {
    if (int rc = lsurge::gemm_rows_nk(KID_MISC, gb, g, n, rhs, nullptr, 0, n, kdim * n, n, kdim, dlhs, kdim, false,
                                      nullptr, nullptr, 0, s, false, lsurge::ExtraExpert(), in_dtype))
      return rc;
    LSURGE_LAUNCH(KID_MISC, s,
                  hipLaunchKernelGGL(zero_rows_from_kernel, dim3(1024), dim3(256), 0, s, dlhs, m, kdim, 2, total));
  }
  // drhs[e] = lhs_e^T @ g_e.  With room for the chunk table and partials (lsurge_ragged_dot_bwd_workspace_bytes), a
  // hot group's rows are cut into chunks that spread over the GPU; with only the forward's workspace, one slice
  // per group.
  if (m > 0 && ragged_chunked(e) && workspace_bytes >= lsurge_ragged_dot_bwd_workspace_bytes(m, kdim, n, e)) {
    const lsurge::WgradChunkPlan p = lsurge::wgrad_chunk_plan(m, e);
    char* base = (char*)workspace;
    size_t off = (lsurge_ragged_dot_workspace_bytes(m, e) + 255) / 256 * 256;
    int32_t* table = (int32_t*)(base + off);
    off = (off + sizeof(int32_t) * lsurge::wgrad_chunk_table_ints(p, e) + 255) / 256 * 256;
    lsurge::WgradChunks ch;
    if (int rc = lsurge::build_wgrad_chunks(e_rows, e_row0, (int)e, p, table, &ch, s, -1, 0, 1)) return rc;
    return lsurge::gemm_wgrad_chunked(KID_MISC, ch, (int)e, m, lhs, kdim, g, n, kdim, n, drhs, nullptr, 0, n, kdim * n,
                                      base + off, lsurge::wgrad_chunked_workspace_bytes(p, kdim, n), s,
                                      lsurge::RowGather(), lsurge::ExtraOut(), in_dtype);
  }
  return lsurge::gemm_wgrad(KID_MISC, (int)e, e_row0, 1, e_rows, 0, m, lhs, kdim, g, n, kdim, n, drhs, nullptr, 0, n,
                            kdim * n, 1, nullptr, 0, s, lsurge::RowGather(), in_dtype);
}

}  // extern "C"
