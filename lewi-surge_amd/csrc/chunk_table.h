// The weight gradients' chunk table, written by one workgroup from per-expert group sizes.  Shared by the chunk
// table's own kernel (gemm.hip) and the layout kernels that write it as they lay out the routing (layout.hip), so
// both give the same table.
#pragma once
#include "launchers.h"

namespace lsurge {

// Every thread of the workgroup calls it (it holds block-wide scans).  Thread 0 stands for the extra expert (id E,
// when o.x_rows >= 0) and the next E threads for the routed experts, so blockDim.x must be at least E + 1 (E without
// an extra expert).  gsz(e) and row0(e) give routed expert e's rows and first row; scan(v, &total) is an exclusive
// block-wide scan of v that also gives the total.
// Each expert gets ceil(rows / R) chunks (one for an empty expert).  An expert of several chunks also gets that many
// f32 partial slots, unless the slots would exceed o.max_parts: then every expert keeps a single chunk.  The extra
// expert (the largest: every token) takes the first chunks, so its long tiles start first.
template <class Gs, class Row0, class Scan>
__device__ __forceinline__ void write_chunk_table(const ChunkTableOut& o, int E, Gs gsz, Row0 row0, Scan scan) {
  const int tid = threadIdx.x;
  const bool has_x = o.x_rows >= 0;
  const bool extra = has_x && tid == 0;
  const int e = has_x ? (tid == 0 ? E : tid - 1) : tid;
  const bool routed = !extra && e < E;
  const int g = routed ? max(gsz(e), 0) : (extra ? o.x_rows : 0);
  const int r0 = routed ? row0(e) : o.x_row0;
  int n = (routed || extra) ? max(1, (g + o.R - 1) / o.R) : 0;
  int nparts;
  const int pbase = scan(n > 1 ? n : 0, &nparts);
  if (nparts > o.max_parts && n > 1) n = 1;
  int nchunks;
  const int cbase = scan(n, &nchunks);
  int nsplit;
  const int sidx = scan(n > 1 ? 1 : 0, &nsplit);
  if (tid == 0) {
    o.num_chunks[0] = min(nchunks, o.max_chunks);
    o.num_split[0] = nsplit;
  }
  if (!routed && !extra) return;
  o.e_pbase[e] = pbase;
  o.e_nparts[e] = n > 1 ? n : 0;
  if (n > 1) o.split_list[sidx] = e;
  for (int j = 0; j < n; ++j) {
    const int c = cbase + j;
    if (c >= o.max_chunks) break;
    o.c_expert[c] = e;
    o.c_row0[c] = r0 + j * o.R;
    o.c_rows[c] = n > 1 ? min(o.R, g - j * o.R) : g;
    o.c_part[c] = n > 1 ? pbase + j : -1;
  }
}

}  // namespace lsurge
