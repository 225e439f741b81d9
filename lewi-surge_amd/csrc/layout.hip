// Routing layout: stable counting sort of the flat (token, choice) slots by expert, without atomics on
// global memory, plus the padded 128-row block table.
//
// Replaces moe_permute.sort_indices (modal/moe_permute.py:240-264: one-hot chunk cumsum -> offsets ->
// pos = offsets[e] + rank) and padded_gmm's row<->slot maps (modal/padded_gmm.py:51-64).
//
// Three kernels:
//   hist  one workgroup per chunk of LT_CHUNK slots; per-wave LDS histograms -> hist[chunk][E]
//   scan  one workgroup: per expert, exclusive scan over chunks (chunk_base), group sizes, expert
//         offsets, block offsets, block table and padding markers in row_src (and, for the layer, the
//         256-row tile table of its grouped GEMMs)
//   rank  one workgroup per chunk again (or per chunk of the fused router's histograms, which replace the hist
//         kernel in the layer); each wave walks its slots 64 at a time in ascending slot order:
//         lanes with the same expert are found with 8 ballots over the expert-id bits, the rank inside
//         the wave is popcount(peers below me), and a per-wave LDS counter advances by popcount(peers).
// In the layer, when the fused router's histograms are small, one kernel does it all (layout_fused_kernel): each
// rank workgroup sums the histograms itself, so the scan's launch between the router and the ranks goes away.
#include "chunk_table.h"
#include "launchers.h"

namespace {

constexpr int LT_THREADS = 256;
constexpr int LT_WAVES = LT_THREADS / 64;
constexpr int LT_PER_WAVE = 512;                       // slots per wave per chunk
constexpr int LT_CHUNK = LT_WAVES * LT_PER_WAVE;       // 2048 slots per workgroup
constexpr int LT_EMAX = 1024;
constexpr int BLK = LSURGE_BLOCK_ROWS;

__global__ __launch_bounds__(LT_THREADS) void layout_hist_kernel(const int32_t* __restrict__ flat, int64_t M,
                                                                 int E, int32_t* __restrict__ hist) {
  extern __shared__ int32_t h[];  // [LT_WAVES][E]
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  for (int i = tid; i < LT_WAVES * E; i += LT_THREADS) h[i] = 0;
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * LT_CHUNK + (int64_t)wv * LT_PER_WAVE;
  for (int r = 0; r < LT_PER_WAVE; r += 64) {
    const int64_t i = base + r + lane;
    if (i < M) {
      const int e = flat[i];
      if (e >= 0 && e < E) atomicAdd(&h[wv * E + e], 1);  // LDS counter: order-independent result
    }
  }
  __syncthreads();
  for (int e = tid; e < E; e += LT_THREADS) {
    int c = 0;
    for (int w = 0; w < LT_WAVES; ++w) c += h[w * E + e];
    hist[(int64_t)blockIdx.x * E + e] = c;
  }
}

// Exclusive scan of one int per thread over the workgroup (blockDim.x <= 1024): returns the prefix and the total,
// through the 16-entry LDS scratch ws (reusable after the trailing barrier).
__device__ __forceinline__ int block_scan_excl(int v, int* ws, int* total) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, nw = (int)blockDim.x >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) ws[w] = x;
  __syncthreads();
  int base = 0, tot = 0;
  for (int i = 0; i < nw; ++i) {
    const int t = ws[i];
    if (i < w) base += t;
    tot += t;
  }
  __syncthreads();
  *total = tot;
  return base + x - v;
}

// The scan's tables from the expert-level results in LDS (gs_s [E], boff_s and tb_s [E + 1]: block and 256-row tile
// bases, totals last): the block table, the padding markers of row_src, the tile table and the shared expert's
// row_src, each over its entries i0, i0 + stride, ... (one workgroup's threads, or those of every workgroup).
__device__ __forceinline__ void write_layout_tables(int E, const int32_t* gs_s, const int32_t* boff_s,
                                                    const int32_t* tb_s, int32_t* __restrict__ row_src,
                                                    int32_t* __restrict__ blk_expert, int32_t* __restrict__ blk_rows,
                                                    int32_t* __restrict__ num_blocks, int max_blocks,
                                                    const lsurge::LayoutTiles& tiles, int i0, int stride) {
  const int nbt = boff_s[E], ntt = tb_s[E];
  if (i0 == 0 && num_blocks) num_blocks[0] = nbt;
  if (blk_expert) {
    // block table: expert e with boff[e] <= b < boff[e + 1] (skips empty experts)
    for (int b = i0; b < max_blocks; b += stride) {
      if (b >= nbt) {
        blk_expert[b] = -1;
        blk_rows[b] = 0;
        continue;
      }
      int lo = 0, hi = E - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (boff_s[mid] <= b) lo = mid;
        else hi = mid - 1;
      }
      blk_expert[b] = lo;
      blk_rows[b] = min(BLK, gs_s[lo] - (b - boff_s[lo]) * BLK);
    }
    // padding rows of each expert's last block: row_src = -1
    for (int i = i0; i < E * BLK; i += stride) {
      const int e = i / BLK, r = i % BLK;
      const int ge = gs_s[e], pad = (ge + BLK - 1) / BLK * BLK - ge;
      if (r < pad) row_src[(int64_t)BLK * boff_s[e] + ge + r] = -1;
    }
  }
  if (tiles.t_expert) {
    // routed tiles (two consecutive blocks of one expert; the last may hold a single block), then the shared expert's
    // (expert E, rows P + 256 j), then empty entries up to the bound TB + TS
    const int total = min(ntt, tiles.TB);  // never clipped for layout-made sizes (they sum to M)
    for (int t = i0; t < tiles.TB + tiles.TS; t += stride) {
      int ex = -1, r0 = 0, rows = 0;
      if (t < total) {
        int lo = 0, hi = E - 1;
        while (lo < hi) {
          const int mid = (lo + hi + 1) >> 1;
          if (tb_s[mid] <= t) lo = mid;
          else hi = mid - 1;
        }
        const int j = t - tb_s[lo];
        ex = lo;
        r0 = BLK * boff_s[lo] + 2 * BLK * j;
        rows = min(2 * BLK, gs_s[lo] - 2 * BLK * j);
      } else if (t < total + tiles.TS) {
        const int j = t - total;
        ex = E;
        r0 = (int)(tiles.P + 2 * BLK * (int64_t)j);
        rows = (int)min((int64_t)2 * BLK, tiles.T - 2 * BLK * (int64_t)j);
      }
      tiles.t_expert[t] = ex;
      tiles.t_row0[t] = r0;
      tiles.t_rows[t] = rows;
    }
    if (tiles.TS > 0)
      for (int64_t r = i0; r < tiles.T; r += stride) row_src[tiles.P + r] = (int32_t)(r * tiles.k);
    if (i0 == 0) {
      tiles.num_tiles[0] = total;
      tiles.num_tiles[1] = total + tiles.TS;
    }
  }
}

// One workgroup of 1024 threads (at least E).  hist [nchunk][E] is overwritten with the exclusive per-expert
// chunk base.
// Thread (e, j) owns expert e's chunks [j cpt, (j + 1) cpt), kept in registers between the two passes (up to
// LS_REG chunks; more are read again).  The expert-level scans are block-wide shuffle scans, and the padding
// markers of row_src are spread over all threads.  With tiles.t_expert set it also writes the 256-row tile table of
// the layer's grouped GEMMs (see LayoutTiles), and with tiles.chunks.c_expert the weight gradients' chunk table.
constexpr int LS_REG = 16, LS_BATCH = 32;
__global__ __launch_bounds__(1024) void layout_scan_kernel(int32_t* __restrict__ hist, int nchunk, int E,
                                                           int32_t* __restrict__ group_sizes,
                                                           int32_t* __restrict__ offsets,
                                                           int32_t* __restrict__ block_off,
                                                           int32_t* __restrict__ row_src,
                                                           int32_t* __restrict__ blk_expert,
                                                           int32_t* __restrict__ blk_rows,
                                                           int32_t* __restrict__ num_blocks, int max_blocks,
                                                           lsurge::LayoutTiles tiles) {
  __shared__ int32_t gs_s[LT_EMAX], boff_s[LT_EMAX + 1], tb_s[LT_EMAX + 1], part_s[1024], ws[16];
  const int tid = threadIdx.x;
  int tpe = 1;
  while (tpe * 2 * E <= (int)blockDim.x && tpe < 64) tpe *= 2;
  const int e_t = tid % E, j_t = tid / E;
  const bool scan_lane = j_t < tpe;
  const int cpt = (nchunk + tpe - 1) / tpe;
  const int c0 = j_t * cpt, c1 = min(nchunk, c0 + cpt);
  const bool in_regs = cpt <= LS_REG;
  int v[LS_REG];
  if (scan_lane) {
    int sum = 0;
    if (in_regs) {
#pragma unroll
      for (int u = 0; u < LS_REG; ++u) v[u] = c0 + u < c1 ? hist[(int64_t)(c0 + u) * E + e_t] : 0;
#pragma unroll
      for (int u = 0; u < LS_REG; ++u) sum += v[u];
    } else {  // LS_BATCH loads in flight per step: the scan is one round trip per batch, not per 8 chunks
      for (int c = c0; c < c1; c += LS_BATCH) {
        int wb[LS_BATCH];
#pragma unroll
        for (int u = 0; u < LS_BATCH; ++u) wb[u] = c + u < c1 ? hist[(int64_t)(c + u) * E + e_t] : 0;
#pragma unroll
        for (int u = 0; u < LS_BATCH; ++u) sum += wb[u];
      }
    }
    part_s[j_t * E + e_t] = sum;
  }
  __syncthreads();
  for (int e = tid; e < E; e += blockDim.x) {
    int run = 0;
    for (int j = 0; j < tpe; ++j) {
      const int x = part_s[j * E + e];
      part_s[j * E + e] = run;
      run += x;
    }
    gs_s[e] = run;
  }
  __syncthreads();
  if (scan_lane) {
    int run = part_s[j_t * E + e_t];
    if (in_regs) {
#pragma unroll
      for (int u = 0; u < LS_REG; ++u) {
        if (c0 + u < c1) hist[(int64_t)(c0 + u) * E + e_t] = run;
        run += v[u];
      }
    } else {
      for (int c = c0; c < c1; c += LS_BATCH) {
        int wb[LS_BATCH];
#pragma unroll
        for (int u = 0; u < LS_BATCH; ++u) wb[u] = c + u < c1 ? hist[(int64_t)(c + u) * E + e_t] : 0;
#pragma unroll
        for (int u = 0; u < LS_BATCH; ++u) {
          if (c + u < c1) hist[(int64_t)(c + u) * E + e_t] = run;
          run += wb[u];
        }
      }
    }
  }
  // expert offsets and block offsets (E <= 1024 = one expert per thread), and the 256-row tile bases
  const int g = tid < E ? gs_s[tid] : 0;
  int tot;
  const int off = block_scan_excl(g, ws, &tot);
  const int nb = (g + BLK - 1) / BLK;
  int nbt;
  const int boff = block_scan_excl(nb, ws, &nbt);
  const int nt = (g + 2 * BLK - 1) / (2 * BLK);
  int ntt = 0;
  const int tbase = tiles.t_expert ? block_scan_excl(nt, ws, &ntt) : 0;
  if (tid < E) {
    boff_s[tid] = boff;
    tb_s[tid] = tbase;
    if (group_sizes) group_sizes[tid] = g;
    if (offsets) offsets[tid] = off;
    if (block_off) block_off[tid] = boff;
  }
  if (tid == 0) {
    boff_s[E] = nbt;
    tb_s[E] = ntt;
  }
  __syncthreads();
  write_layout_tables(E, gs_s, boff_s, tb_s, row_src, blk_expert, blk_rows, num_blocks, max_blocks, tiles, tid,
                      (int)blockDim.x);
  if (tiles.chunks.c_expert)
    lsurge::write_chunk_table(
        tiles.chunks, E, [&](int e) { return gs_s[e]; }, [&](int e) { return BLK * boff_s[e]; },
        [&](int v, int* total) { return block_scan_excl(v, ws, total); });
}

__device__ __forceinline__ uint64_t peers_of(int key, int nbits) {
  uint64_t m = ~0ull;
  for (int b = 0; b < nbits; ++b) {
    const uint64_t bal = __ballot((key >> b) & 1);
    m &= ((key >> b) & 1) ? bal : ~bal;
  }
  return m;
}

// Ranks of one chunk's slots: chunk blockIdx.x of (blockDim.x / 64) * per_wave slots, each wave walking its own
// per_wave slots 64 at a time in ascending order.  cnt [waves][E] in LDS must be zero (and the zeroing made visible
// with a barrier); base(e) is the rank in expert e of the chunk's first slot, off(e) and boff(e) the expert's offset
// and block offset.
template <class Base, class Off, class Boff>
__device__ __forceinline__ void rank_chunk(const int32_t* __restrict__ flat, int64_t M, int E, int32_t* cnt, Base base,
                                           Off off, Boff boff, int nbits, int per_wave, int32_t* __restrict__ order,
                                           int32_t* __restrict__ pos, int32_t* __restrict__ slot,
                                           int32_t* __restrict__ row_src) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, nw = (int)blockDim.x >> 6;
  const int64_t cbase = (int64_t)blockIdx.x * nw * per_wave;
  // per-wave histograms of this chunk
  for (int r = 0; r < per_wave; r += 64) {
    const int64_t i = cbase + (int64_t)wv * per_wave + r + lane;
    if (i < M) {
      const int e = flat[i];
      if (e >= 0 && e < E) atomicAdd(&cnt[wv * E + e], 1);
    }
  }
  __syncthreads();
  // exclusive scan over waves, seeded with the chunk base (rank of the first slot of this chunk in e)
  for (int e = tid; e < E; e += blockDim.x) {
    int run = base(e);
    for (int w = 0; w < nw; ++w) {
      const int v = cnt[w * E + e];
      cnt[w * E + e] = run;
      run += v;
    }
  }
  __syncthreads();
  int32_t* my = cnt + wv * E;
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int r = 0; r < per_wave; r += 64) {
    const int64_t i = cbase + (int64_t)wv * per_wave + r + lane;
    const int fe = i < M ? flat[i] : -1;
    const bool valid = fe >= 0 && fe < E;  // ids outside [0, E) are skipped (documented as invalid input)
    const int e = valid ? fe : -1;
    // invalid lanes use key with all bits set above E's range; they never match a valid expert
    const int key = valid ? e : ((1 << nbits) - 1);
    uint64_t peers = peers_of(key, nbits) & __ballot(valid);
    if (!valid) peers = 0;
    const int rank_in = __popcll(peers & below);
    int rank = 0;
    if (valid) rank = my[e] + rank_in;
    // the highest peer lane advances the counter after everyone has read it
    __builtin_amdgcn_wave_barrier();
    if (valid && (peers >> lane) == 1ull) my[e] = rank + 1;
    __builtin_amdgcn_wave_barrier();
    if (valid) {
      const int p = off(e) + rank;
      if (pos) pos[i] = p;
      if (order) order[p] = (int32_t)i;
      if (slot) {
        const int sl = BLK * boff(e) + rank;
        slot[i] = sl;
        if (row_src) row_src[sl] = (int32_t)i;
      }
    }
  }
}

// One workgroup per chunk of (blockDim.x / 64) * per_wave slots (LT_CHUNK for the layout's own histograms, 64 k
// when the fused router made them: one 64-slot pass per wave).
__global__ __launch_bounds__(1024) void layout_rank_kernel(
    const int32_t* __restrict__ flat, int64_t M, int E, const int32_t* __restrict__ chunk_base,
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ block_off, int nbits, int per_wave,
    int32_t* __restrict__ order, int32_t* __restrict__ pos, int32_t* __restrict__ slot,
    int32_t* __restrict__ row_src) {
  extern __shared__ int32_t sh[];  // cnt[waves][E] (per-wave running rank base inside the expert)
  const int nw = (int)blockDim.x >> 6;
  for (int i = threadIdx.x; i < nw * E; i += blockDim.x) sh[i] = 0;
  __syncthreads();
  rank_chunk(
      flat, M, E, sh, [&](int e) { return chunk_base[(int64_t)blockIdx.x * E + e]; },
      [&](int e) { return offsets[e]; }, [&](int e) { return block_off[e]; }, nbits, per_wave, order, pos, slot,
      row_src);
}

// The whole layout in one launch, for the layer when the fused router made the chunk histograms and they are small
// (nchunk E <= LF_HIST_MAX): every workgroup sums the histograms itself (the chunks before its own give its
// per-expert rank bases, all of them the expert totals), so no scan kernel runs between the router and the ranks.
// The scan's tables are spread over all workgroups, and the last one writes the weight gradients' chunk table.
// Needs E + 1 <= blockDim.x: a thread per expert in the expert-level scans, and one more for the chunk table's
// extra expert.  Each workgroup reads nchunk E ints of histograms (64 KB at T = 16384 tokens, 64 experts), from L2.
constexpr int LF_HIST_MAX = 32768, LF_LOADS = 16;
__global__ __launch_bounds__(1024) void layout_fused_kernel(
    const int32_t* __restrict__ flat, int64_t M, int E, const int32_t* __restrict__ hist, int nchunk, int nbits,
    int per_wave, int32_t* __restrict__ order, int32_t* __restrict__ pos, int32_t* __restrict__ slot,
    int32_t* __restrict__ row_src, int32_t* __restrict__ group_sizes, int32_t* __restrict__ offsets,
    int32_t* __restrict__ block_off, int32_t* __restrict__ blk_expert, int32_t* __restrict__ blk_rows,
    int32_t* __restrict__ num_blocks, int max_blocks, lsurge::LayoutTiles tiles) {
  extern __shared__ int32_t sh[];
  const int tid = threadIdx.x, nt = (int)blockDim.x, nw = nt >> 6, me = (int)blockIdx.x;
  const int tpe = nt / E;               // threads per expert in the histogram sums
  int32_t* cnt = sh;                    // [nw][E]
  int32_t* part = cnt + nw * E;         // [2][tpe][E]: partial sums below this chunk, and over all chunks
  int32_t* below_s = part + 2 * tpe * E;
  int32_t* gs_s = below_s + E;
  int32_t* off_s = gs_s + E;
  int32_t* boff_s = off_s + E;          // [E + 1]
  int32_t* tb_s = boff_s + E + 1;       // [E + 1]
  int32_t* ws = tb_s + E + 1;           // [16]
  for (int i = tid; i < nw * E; i += nt) cnt[i] = 0;
  const int e_t = tid % E, j_t = tid / E;
  if (j_t < tpe) {
    int below = 0, all = 0;
    for (int c0 = j_t; c0 < nchunk; c0 += LF_LOADS * tpe) {
      int v[LF_LOADS];
#pragma unroll
      for (int u = 0; u < LF_LOADS; ++u) {
        const int c = c0 + u * tpe;
        v[u] = c < nchunk ? hist[(int64_t)c * E + e_t] : 0;
      }
#pragma unroll
      for (int u = 0; u < LF_LOADS; ++u) {
        all += v[u];
        below += c0 + u * tpe < me ? v[u] : 0;
      }
    }
    part[j_t * E + e_t] = below;
    part[(tpe + j_t) * E + e_t] = all;
  }
  __syncthreads();
  if (tid < E) {
    int below = 0, all = 0;
    for (int j = 0; j < tpe; ++j) {
      below += part[j * E + tid];
      all += part[(tpe + j) * E + tid];
    }
    below_s[tid] = below;
    gs_s[tid] = all;
  }
  __syncthreads();
  // expert offsets, block offsets and tile bases: the same scans as the scan kernel's
  const int g = tid < E ? gs_s[tid] : 0;
  int tot, nbt, ntt = 0;
  const int off = block_scan_excl(g, ws, &tot);
  const int boff = block_scan_excl((g + BLK - 1) / BLK, ws, &nbt);
  const int tbase = tiles.t_expert ? block_scan_excl((g + 2 * BLK - 1) / (2 * BLK), ws, &ntt) : 0;
  if (tid < E) {
    off_s[tid] = off;
    boff_s[tid] = boff;
    tb_s[tid] = tbase;
    if (me == 0) {
      if (group_sizes) group_sizes[tid] = g;
      if (offsets) offsets[tid] = off;
      if (block_off) block_off[tid] = boff;
    }
  }
  if (tid == 0) {
    boff_s[E] = nbt;
    tb_s[E] = ntt;
  }
  __syncthreads();
  rank_chunk(
      flat, M, E, cnt, [&](int e) { return below_s[e]; }, [&](int e) { return off_s[e]; },
      [&](int e) { return boff_s[e]; }, nbits, per_wave, order, pos, slot, row_src);
  write_layout_tables(E, gs_s, boff_s, tb_s, row_src, blk_expert, blk_rows, num_blocks, max_blocks, tiles,
                      me * nt + tid, (int)gridDim.x * nt);
  if (tiles.chunks.c_expert && me == (int)gridDim.x - 1)
    lsurge::write_chunk_table(
        tiles.chunks, E, [&](int e) { return gs_s[e]; }, [&](int e) { return BLK * boff_s[e]; },
        [&](int v, int* total) { return block_scan_excl(v, ws, total); });
}

// inv[v] = m for every v (the entries that no index hits keep it; a gather through inv gives zero rows there)
__global__ void fill_i32_kernel(int32_t* __restrict__ p, int64_t m, int32_t v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < m) p[i] = v;
}
// inv[idx[i]] = i; entries of idx outside [0, m) are skipped, so no index can write outside inv
__global__ void invert_perm_kernel(const int32_t* __restrict__ idx, int64_t m, int32_t* __restrict__ inv) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < m) {
    const int32_t v = idx[i];
    if ((uint32_t)v < (uint32_t)m) inv[v] = (int32_t)i;
  }
}

int layout_common(const int32_t* flat, int64_t M, int64_t E, int32_t* gs, int32_t* offsets, int32_t* block_off,
                  int32_t* order, int32_t* pos, int32_t* slot, int32_t* row_src, int32_t* blk_expert,
                  int32_t* blk_rows, int32_t* num_blocks, int64_t max_blocks, void* ws, size_t ws_bytes,
                  hipStream_t s, const lsurge::LayoutTiles& tiles = lsurge::LayoutTiles(),
                  const lsurge::LayoutChunks& pre = lsurge::LayoutChunks()) {
  // chunks: LT_CHUNK slots with histograms made here, or the caller's (pre.hist, pre.waves x 64 slots each)
  const int waves = pre.hist ? pre.waves : LT_WAVES, per_wave = pre.hist ? 64 : LT_PER_WAVE;
  const int64_t chunk = (int64_t)waves * per_wave;
  const int64_t nchunk = (M + chunk - 1) / chunk;
  // workspace: hist [nchunk][E] (unless given) | offsets [E] | block_off [E] | num_blocks (when caller gives none)
  const size_t need = sizeof(int32_t) * (size_t)((pre.hist ? 0 : nchunk * E) + 2 * E + 4);
  LSURGE_REQUIRE(ws && ws_bytes >= need, "layout: workspace %zu < %zu bytes", ws_bytes, need);
  int32_t* hist = pre.hist ? pre.hist : (int32_t*)ws;
  int32_t* off_ws = (int32_t*)ws + (pre.hist ? 0 : nchunk * E);
  int32_t* boff_ws = off_ws + E;
  int32_t* nb_ws = boff_ws + E;
  if (!offsets) offsets = off_ws;
  if (!block_off) block_off = boff_ws;
  if (!num_blocks) num_blocks = nb_ws;
  int nbits = 1;
  while ((1ll << nbits) <= E) ++nbits;  // keys 0..E-1 valid, (1<<nbits)-1 >= E reserved for idle lanes
  // the scan needs a thread per expert: 1024 threads whatever E, which took the C5 scan from 84 to 59 us (against 512
  // threads for E <= 512); the 512-thread choice had been meant to let the scan share a CU with a running 8-wave GEMM
  // tile (the layer's shared expert runs beside the layout), and the measured gain of the wider scan was larger
  const unsigned scan_threads = 1024;
  if (M == 0) {
    LSURGE_LAUNCH(KID_LAYOUT_SCAN, s,
                  hipLaunchKernelGGL(layout_scan_kernel, dim3(1), dim3(scan_threads), 0, s, hist, 0, (int)E, gs, offsets,
                                     block_off, row_src, blk_expert, blk_rows, num_blocks, (int)max_blocks, tiles));
    return LSURGE_OK;
  }
  // the fused router's histograms, when small: the whole layout in one launch (layout_fused_kernel)
  if (pre.hist && 64 * waves >= E + 1 && nchunk * E <= LF_HIST_MAX) {
    const int nt = 64 * waves, tpe = nt / (int)E;
    const size_t lds = sizeof(int32_t) * ((size_t)waves * E + 2 * (size_t)tpe * E + 5 * (size_t)E + 2 + 16);
    LSURGE_LAUNCH(KID_LAYOUT_RANK, s,
                  hipLaunchKernelGGL(layout_fused_kernel, dim3((unsigned)nchunk), dim3(nt), lds, s, flat, M, (int)E,
                                     hist, (int)nchunk, nbits, per_wave, order, pos, slot, row_src, gs, offsets,
                                     block_off, blk_expert, blk_rows, num_blocks, (int)max_blocks, tiles));
    return LSURGE_OK;
  }
  if (!pre.hist)
    LSURGE_LAUNCH(KID_LAYOUT_HIST, s,
                  hipLaunchKernelGGL(layout_hist_kernel, dim3((unsigned)nchunk), dim3(LT_THREADS),
                                     sizeof(int32_t) * LT_WAVES * (size_t)E, s, flat, M, (int)E, hist));
  LSURGE_LAUNCH(KID_LAYOUT_SCAN, s,
                hipLaunchKernelGGL(layout_scan_kernel, dim3(1), dim3(scan_threads), 0, s, hist, (int)nchunk, (int)E, gs,
                                   offsets, block_off, row_src, blk_expert, blk_rows, num_blocks,
                                   (int)max_blocks, tiles));
  LSURGE_LAUNCH(KID_LAYOUT_RANK, s,
                hipLaunchKernelGGL(layout_rank_kernel, dim3((unsigned)nchunk), dim3(64 * waves),
                                   sizeof(int32_t) * waves * (size_t)E, s, flat, M, (int)E, hist, offsets, block_off,
                                   nbits, per_wave, order, pos, slot, row_src));
  return LSURGE_OK;
}

}  // namespace

namespace lsurge {
int build_layout_impl(const int32_t* flat, int64_t M, int64_t E, int32_t* gs, int32_t* offsets, int32_t* block_off,
                      int32_t* order, int32_t* pos, int32_t* slot, int32_t* row_src, int32_t* blk_expert,
                      int32_t* blk_rows, int32_t* num_blocks, void* ws, size_t ws_bytes, hipStream_t s,
                      const LayoutTiles& tiles, const LayoutChunks& pre) {
  LSURGE_REQUIRE(!tiles.t_expert || (tiles.t_rows && tiles.t_row0 && tiles.num_tiles && row_src && E <= 1024),
                 "layout: incomplete tile table outputs");
  LSURGE_REQUIRE(!pre.hist || (pre.waves >= 1 && pre.waves <= 16), "layout: chunk waves=%d not in [1, 16]", pre.waves);
  LSURGE_REQUIRE(!tiles.chunks.c_expert || (tiles.t_expert && E + 1 <= 1024 && tiles.chunks.R >= 1),
                 "layout: chunk table needs the tile table, E + 1 <= 1024 and R >= 1");
  return layout_common(flat, M, E, gs, offsets, block_off, order, pos, slot, row_src, blk_expert, blk_rows,
                       num_blocks, lsurge_max_blocks(M, E), ws, ws_bytes, s, tiles, pre);
}
}  // namespace lsurge

extern "C" {

int64_t lsurge_max_blocks(int64_t m, int64_t num_experts) { return (m + BLK - 1) / BLK + num_experts; }

size_t lsurge_layout_workspace_bytes(int64_t m, int64_t num_experts) {
  const int64_t nchunk = (m + LT_CHUNK - 1) / LT_CHUNK;
  return sizeof(int32_t) * (size_t)(nchunk * num_experts + 2 * num_experts + 4);
}

size_t lsurge_sort_indices_workspace_bytes(int64_t m, int64_t num_experts) {
  return lsurge_layout_workspace_bytes(m, num_experts);
}

int lsurge_sort_indices(const int32_t* flat, int64_t m, int64_t num_experts, int32_t* order, int32_t* pos,
                        int32_t* group_sizes, void* workspace, size_t workspace_bytes, lsurge_stream_t stream) {
  LSURGE_REQUIRE(m >= 0 && m < (1ll << 31), "sort_indices: bad m=%lld", (long long)m);
  LSURGE_REQUIRE(num_experts >= 1 && num_experts <= LT_EMAX, "sort_indices: num_experts=%lld not in [1, %d]",
                 (long long)num_experts, LT_EMAX);
  LSURGE_REQUIRE(m == 0 || (flat && order && pos), "sort_indices: null pointer");
  return layout_common(flat, m, num_experts, group_sizes, nullptr, nullptr, order, pos, nullptr, nullptr, nullptr,
                       nullptr, nullptr, 0, workspace, workspace_bytes, (hipStream_t)stream);
}

int lsurge_build_layout(const int32_t* flat, int64_t m, int64_t num_experts, int32_t* group_sizes, int32_t* offsets,
                        int32_t* block_off, int32_t* order, int32_t* pos, int32_t* slot, int32_t* row_src,
                        int32_t* blk_expert, int32_t* blk_rows, int32_t* num_blocks, void* workspace,
                        size_t workspace_bytes, lsurge_stream_t stream) {
  LSURGE_REQUIRE(m >= 0 && m < (1ll << 31), "build_layout: bad m=%lld", (long long)m);
  LSURGE_REQUIRE(num_experts >= 1 && num_experts <= LT_EMAX, "build_layout: num_experts=%lld not in [1, %d]",
                 (long long)num_experts, LT_EMAX);
  LSURGE_REQUIRE(m == 0 || (flat && order && pos && slot && row_src), "build_layout: null pointer");
  LSURGE_REQUIRE(blk_expert && blk_rows && num_blocks, "build_layout: null block table");
  return lsurge::build_layout_impl(flat, m, num_experts, group_sizes, offsets, block_off, order, pos, slot, row_src,
                                   blk_expert, blk_rows, num_blocks, workspace, workspace_bytes,
                                   (hipStream_t)stream);
}

int lsurge_invert_permutation(const int32_t* idx, int64_t m, int32_t* inv, lsurge_stream_t stream) {
  LSURGE_REQUIRE(m >= 0 && m < (1ll << 31), "invert_permutation: bad m");
  if (m == 0) return LSURGE_OK;
  LSURGE_REQUIRE(idx && inv, "invert_permutation: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)((m + 255) / 256));
  LSURGE_LAUNCH(KID_MISC, s, hipLaunchKernelGGL(fill_i32_kernel, grid, dim3(256), 0, s, inv, m, (int32_t)m));
  LSURGE_LAUNCH(KID_MISC, s, hipLaunchKernelGGL(invert_perm_kernel, grid, dim3(256), 0, s, idx, m, inv));
  return LSURGE_OK;
}

}  // extern "C"
