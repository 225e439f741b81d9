// Grouped GEMMs of the MoE layer on CDNA4 matrix cores: bf16 inputs, f32 accumulation,
// v_mfma_f32_32x32x16_bf16, 128 x 256 workgroup tiles (4 waves, 64 x 128 each), K staged through LDS in
// BK-wide double-buffered chunks fed from two register sets (global loads run two chunks ahead); two
// workgroups share a CU.
//
// Replaces the padded batched einsum of modal/padded_gmm.py:66-69 (cuBLAS on the reference's GPU path) and
// its autodiff.  Two kernel families:
//
//  gemm_rows   row-blocked: C[block rows, n-tile] = A[block rows, :] @ B[expert(block)], one 128-row expert
//              block per workgroup row.  Blocks past the device-side block count exit at once, so padding
//              tiles cost nothing; rows past a block's valid count are loaded as zeros.
//              B either K-major ([N, K], read with ds_read_b128) or N-major ([K, N], read with the gfx950
//              LDS transpose read ds_read_b64_tr_b16).  Epilogues: plain store (bf16 or f32), SwiGLU forward
//              (gate and up columns side by side in one accumulator set -> h = silu(g) * u, plus g and u
//              for the backward), SwiGLU backward (dH -> dG, dU from the saved g, u).
//  gemm_wgrad  per-expert weight gradient: C_e = A_e^T @ B_e with the reduction over the expert's rows
//              (ragged K); both operands N-major in LDS, transpose-read.  Optional split of the rows into
//              S slices with f32 partials summed afterwards in a fixed order (deterministic, no atomics).
// The MFMA operands are passed weight-first, so each lane's accumulators hold four consecutive output
// columns of one row and every epilogue store is an 8-byte (bf16) or 16-byte (f32) vector.
#include "common.h"

namespace {

// Workgroup tile: BM rows (one 128-row expert block) x BN columns, 4 waves in a 2 x 2 grid of 64 x 128 wave
// tiles; K is staged through LDS BK at a time (54-57 KB of LDS, so two workgroups fit in a CU's 160 KB).  Per wave and 16-wide k step: 2 activation fragments + 4 weight
// fragments (6 x 1 KiB of LDS reads) feed 8 MFMAs, which keeps LDS traffic at 3/4 of what 64 x 64 wave tiles
// need.  Global loads run two K stages ahead through two register sets.
constexpr int BM = 128, BN = 256, BK = 32;
constexpr int GT = 256;            // threads per workgroup
constexpr int OCC = 2;             // workgroups per CU: one's prologue/epilogue overlaps the other's MFMAs
constexpr int NPB = BN + 32;       // N-major B tile pitch: 576 B, rows k..k+3 fall on distinct 64 B bank groups
constexpr int NPA = BM + 32;       // N-major A tile pitch (wgrad): 320 B, same property

enum { B_NK = 0, B_KN = 1 };                        // B operand storage
enum { EPI_STORE = 0, EPI_SWIGLU_FWD = 1, EPI_SWIGLU_BWD = 2 };

struct RowsArgs {
  const bf16_t* A;  // rows with K contiguous
  int64_t lda;
  const bf16_t* B;   // expert 0 of the first B matrix
  const bf16_t* B2;  // second B (SwiGLU up weights / dgrad up weights), same strides
  int64_t ldb;       // row pitch of B as stored
  int64_t b_estride; // elements between experts
  int64_t K, N;      // reduction dim, output columns (EPI_SWIGLU_FWD: N = f, a tile covers BN/2 outputs)
  int64_t k_split;   // B_NK with B2: k < k_split from B, else B2 at k - k_split (0 = unused)
  bf16_t* C;         // output [rows, ldc]
  float* Cf;         // EPI_STORE: f32 output instead of C when set
  int64_t ldc;
  bf16_t* G;         // SwiGLU saved gate pre-activation [rows, ldg] (fwd: written, bwd: read)
  bf16_t* U;         // SwiGLU saved up projection
  int64_t ldg;
  const int32_t* blk_expert;  // nullptr: dense (expert 0, rows = min(128, dense_rows - 128 b))
  const int32_t* blk_rows;
  const int32_t* blk_row0;    // first row of block b (nullptr: 128 b)
  const int32_t* num_blocks;
  int64_t dense_rows;
  int n_tiles;
  int max_blocks;
};

struct WgradArgs {
  const bf16_t* A;   // [rows, lda], the reduction runs over rows; C's rows are A's columns
  int64_t lda;
  const bf16_t* B;   // [rows, ldb]
  int64_t ldb;
  int64_t I, N;      // output [I, N] per expert
  float* C;          // expert e at C + e * c_estride, row pitch ldc
  float* C2;         // columns n >= n_split go to C2 at column n - n_split (nullptr: unused)
  int64_t n_split;
  int64_t ldc, c_estride;
  float* part;       // split partials [S][E][I][N] when S > 1
  const int32_t* e_row0;  // first row of expert e, in units of row0_mult rows (nullptr: dense)
  const int32_t* e_rows;  // rows of expert e
  int row0_mult;
  int64_t dense_rows;
  int E, S, i_tiles, n_tiles;
};

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// D[32 x 32] += P[32 x 16] Q[16 x 32]; lane l supplies row l%32 of P and column l%32 of Q, k = 8(l/32)..+7.
// The layer calls it with P = the weight fragment and Q = the activation fragment, so the accumulator holds
// C^T: lane l owns activation row l%32 and output columns 8(r/4) + 4(l/32) + r%4 -- four consecutive columns
// per register quad, which the epilogues store as one 8- or 16-byte vector.
__device__ __forceinline__ f32x16 mfma32(bf16x8 p, bf16x8 q, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(p, q, c, 0, 0, 0);
}

// K-major tiles hold BK = 32 k per row (4 chunks of 16 B, 64 B rows, no padding).  Chunk c of row r sits at
// slot c ^ ((r >> 2) & 3): a 16-lane group storing 4 whole rows covers 256 contiguous bytes, and a 16-lane
// group reading one chunk of 16 consecutive rows hits 16 distinct 16-byte slots of a 256-byte bank window, so
// neither direction has bank conflicts.
__device__ __forceinline__ int km_off(int row, int chunk) { return row * BK + ((chunk ^ ((row >> 2) & 3)) << 3); }

// K-major fragment: 8 consecutive k (chunk kc) of one row -> one 16-byte LDS read
__device__ __forceinline__ bf16x8 frag_k(const bf16_t* tile, int row, int kc) {
  return as_bf16x8(*reinterpret_cast<const u32x4*>(tile + km_off(row, kc)));
}

// N-major fragment for the 32x32x16 operand layout: lane l needs rows (k) 8(l/32)+0..7 of column l%32.
// ds_read_b64_tr_b16 in a 16-lane group g: lane i receives D[4j + i/4][i%4], j = 0..3, where D[s] are the four
// 16-bit values at source lane s's address.  With source lane s pointing at (k = kb + s/4, n = nb + 4(s%4)),
// lane i receives column nb + i, rows kb..kb+3.  Two reads give the 8 k values.
__device__ __forceinline__ bf16x8 frag_n(const bf16_t* tile, int pitch, int kbase, int nbase, int lane) {
  const int g = lane >> 4, s = lane & 15;
  const int n = nbase + 16 * (g & 1) + 4 * (s & 3);
  const int k0 = kbase + 8 * (g >> 1) + (s >> 2);
  const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_PTR(s16x4, tile + k0 * pitch + n));
  const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_PTR(s16x4, tile + (k0 + 4) * pitch + n));
  typedef short s16x8 __attribute__((ext_vector_type(8)));
  const s16x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(bf16x8, v);
}

__device__ __forceinline__ void st16(bf16_t* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

// Operand tiles are fetched with raw buffer loads: one descriptor per operand covers exactly the bytes the tile
// may read (a block's valid rows, an expert's weight matrix), and a lane whose element lies outside the tile
// (rows past the block, K or N tails) passes an offset past the end, for which the buffer unit returns zeros.
// That keeps the load path free of branches and the zero padding exact.
constexpr uint32_t OOB = 0x80000000u;  // every descriptor covers < 2^31 bytes (checked on the host)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 bload16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, 0, 0);
}

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void st_bf16x4(bf16_t* p, float a, float b, float c, float d) {
  *reinterpret_cast<u32x2*>(p) = u32x2{pack_bf16x2(a, b), pack_bf16x2(c, d)};
}
__device__ __forceinline__ void ld_bf16x4(const bf16_t* p, float* o) {
  const u32x2 v = *reinterpret_cast<const u32x2*>(p);
  o[0] = __uint_as_float(v[0] << 16);
  o[1] = __uint_as_float(v[0] & 0xffff0000u);
  o[2] = __uint_as_float(v[1] << 16);
  o[3] = __uint_as_float(v[1] & 0xffff0000u);
}

// 1 / (1 + e^-g) with the hardware reciprocal (about 1 ulp): plenty for bf16 outputs, and it keeps the
// epilogue short
__device__ __forceinline__ float sigmoid_f(float g) { return __builtin_amdgcn_rcpf(1.f + __expf(-g)); }
__device__ __forceinline__ float silu_f(float g) { return g * sigmoid_f(g); }

// XCD-aware tile order: workgroups are dispatched round-robin over the 8 XCDs, so consecutive logical
// tiles (same expert block, neighbouring N tiles and experts) are sent to the same XCD's L2.
__device__ __forceinline__ int64_t xcd_logical(int64_t id, int64_t total) {
  const int64_t per = total / 8;
  return (id % 8) * per + id / 8;
}

constexpr int KC = BK / 8;          // 16-byte chunks per K-major tile row
static_assert(KC == 4, "km_off swizzles 4 chunks per row");
constexpr int SA = BM * BK / 8 / GT;  // 16-byte loads per thread: activation tile (or wgrad A tile)
constexpr int SB = BN * BK / 8 / GT;  // weight tile (or wgrad B tile)
struct Stage {
  u32x4 a[SA];
  u32x4 b[SB];
};

// N-major B tile (BK k-rows x BN columns): 16-byte chunk i of thread tid -> (k row, first column).  Loads
// i < SB/2 cover columns [0, BN/2) and the rest [BN/2, BN), so in the SwiGLU forward (gate columns, then up
// columns) every load instruction reads from one weight matrix and its descriptor stays wave-uniform.
__device__ __forceinline__ int2 kn_chunk(int tid, int i) {
  constexpr int HALF_CHUNKS = BN / 2 / 8;                     // 16 chunks per half row
  const int v = tid + GT * (i % (SB / 2));                    // 0 .. BK * 16 - 1
  return int2{v / HALF_CHUNKS, (i < SB / 2 ? 0 : BN / 2) + (v % HALF_CHUNKS) * 8};
}

// =====================================================================================================
template <int BMODE, int EPI>
__global__ __launch_bounds__(GT, OCC) void gemm_rows_kernel(RowsArgs a) {
  __shared__ __attribute__((aligned(16))) bf16_t As[2][BM * BK];
  __shared__ __attribute__((aligned(16))) bf16_t Bs[2][BMODE == B_NK ? BN * BK : BK * NPB];

  const int64_t total = (int64_t)gridDim.x;
  const int64_t logical = xcd_logical(blockIdx.x, total);
  const int nt = (int)(logical % a.n_tiles);
  const int b = (int)(logical / a.n_tiles);
  if (b >= a.max_blocks) return;
  int expert, rows;
  int64_t row0;
  if (a.blk_expert) {
    if (b >= a.num_blocks[0]) return;
    expert = a.blk_expert[b];
    rows = a.blk_rows[b];
    row0 = a.blk_row0 ? (int64_t)a.blk_row0[b] : (int64_t)b * BM;
  } else {
    expert = 0;
    row0 = (int64_t)b * BM;
    rows = (int)min((int64_t)BM, a.dense_rows - row0);
    if (rows <= 0) return;
  }
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  // column origin of this tile: weight columns for B, output columns for C (SwiGLU: gate and up halves)
  const int64_t n0 = (int64_t)nt * (EPI == EPI_SWIGLU_FWD ? BN / 2 : BN);
  const bf16_t* Bbase = a.B + (int64_t)expert * a.b_estride;
  const bf16_t* B2base = a.B2 ? a.B2 + (int64_t)expert * a.b_estride : nullptr;
  const int64_t K = a.K, N = a.N;
  const int nk = (int)((K + BK - 1) / BK);

  // descriptors: this block's rows of A; the expert's B (and B2) matrix
  const __amdgpu_buffer_rsrc_t rsA = make_rsrc(a.A + row0 * a.lda, (int64_t)rows * a.lda * 2);
  const int64_t b_bytes = (BMODE == B_NK ? N : K) * a.ldb * 2;
  const __amdgpu_buffer_rsrc_t rsB = make_rsrc(Bbase, b_bytes);
  const __amdgpu_buffer_rsrc_t rsB2 = make_rsrc(B2base ? B2base : Bbase, b_bytes);

  auto load = [&](Stage& st, int kt) {
    const int k0 = kt * BK;
#pragma unroll
    for (int i = 0; i < SA; ++i) {
      const int v = tid + GT * i;
      const int r = v / KC, kc = (v % KC) * 8;
      const bool ok = r < rows && k0 + kc < K;
      st.a[i] = bload16(rsA, ok ? (uint32_t)((r * a.lda + k0 + kc) * 2) : OOB);
    }
    if (BMODE == B_NK) {
      const bool second = a.k_split && k0 >= a.k_split;
      const int kk0 = second ? k0 - (int)a.k_split : k0;
#pragma unroll
      for (int i = 0; i < SB; ++i) {
        const int v = tid + GT * i;
        const int n = v / KC, kc = (v % KC) * 8;
        const int64_t gn = n0 + n;
        const bool ok = gn < N && k0 + kc < K;
        const uint32_t off = ok ? (uint32_t)((gn * a.ldb + kk0 + kc) * 2) : OOB;
        st.b[i] = second ? bload16(rsB2, off) : bload16(rsB, off);
      }
    } else {
#pragma unroll
      for (int i = 0; i < SB; ++i) {
        const int2 kn = kn_chunk(tid, i);
        const int64_t gk = k0 + kn.x;
        if (EPI == EPI_SWIGLU_FWD) {  // tile columns [0, 128) gate, [128, 256) up, same output columns
          const int64_t gn = n0 + (kn.y & (BN / 2 - 1));
          const uint32_t off = (gk < K && gn < N) ? (uint32_t)((gk * a.ldb + gn) * 2) : OOB;
          st.b[i] = i < SB / 2 ? bload16(rsB, off) : bload16(rsB2, off);  // uniform choice of descriptor
        } else {
          const int64_t gn = n0 + kn.y;
          st.b[i] = bload16(rsB, (gk < K && gn < N) ? (uint32_t)((gk * a.ldb + gn) * 2) : OOB);
        }
      }
    }
  };
  auto store = [&](const Stage& st, int buf) {
#pragma unroll
    for (int i = 0; i < SA; ++i) {
      const int v = tid + GT * i;
      st16(&As[buf][km_off(v / KC, v % KC)], st.a[i]);
    }
#pragma unroll
    for (int i = 0; i < SB; ++i) {
      const int v = tid + GT * i;
      if (BMODE == B_NK) {
        st16(&Bs[buf][km_off(v / KC, v % KC)], st.b[i]);
      } else {
        const int2 kn = kn_chunk(tid, i);
        st16(&Bs[buf][kn.x * NPB + kn.y], st.b[i]);
      }
    }
  };
  // tile column of this wave's weight fragment j
  auto bcol = [&](int j) {
    if (EPI == EPI_SWIGLU_FWD) return (j < 2 ? 0 : BN / 2) + wn * 64 + 32 * (j & 1);
    return wn * 128 + 32 * j;
  };

  f32x16 acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};

  auto compute = [&](int buf) {
    __builtin_amdgcn_iglp_opt(0);  // interleave the fragment reads with the MFMAs
    const bf16_t* at = As[buf];
    const bf16_t* bt = Bs[buf];
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      bf16x8 xf[2], wf[4];
#pragma unroll
      for (int i = 0; i < 2; ++i) xf[i] = frag_k(at, wm * 64 + 32 * i + (lane & 31), kk / 8 + (lane >> 5));
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (BMODE == B_NK) wf[j] = frag_k(bt, bcol(j) + (lane & 31), kk / 8 + (lane >> 5));
        else wf[j] = frag_n(bt, NPB, kk, bcol(j), lane);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma32(wf[j], xf[i], acc[i][j]);
    }
  };

  // Software pipeline: LDS buffers 0/1, register sets ra/rb; the loads of stage kt+2 are issued while stage kt
  // is multiplied, so global latency has two compute phases to hide behind.  One barrier per stage.  The loop
  // body is branch-free: stages past the end load as zeros (out-of-range offsets), so the wait counts are the
  // same on every trip and an odd stage count just multiplies one zero stage.
  Stage ra, rb;
  load(ra, 0);
  load(rb, 1);
  store(ra, 0);
  load(ra, 2);
  __syncthreads();
  for (int kt = 0; kt < nk; kt += 2) {
    store(rb, 1);
    load(rb, kt + 3);
    compute(0);
    __syncthreads();
    store(ra, 0);
    load(ra, kt + 4);
    compute(1);
    __syncthreads();
  }

  // ---- epilogue.  acc[i][j][4q + t]: activation row wm*64 + 32 i + lane%32, tile column bcol(j) + 8 q +
  // 4 (lane/32) + t.
  const int lm = lane & 31, lh = lane >> 5;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int mloc = wm * 64 + 32 * i + lm;
    if (mloc >= rows) continue;
    const int64_t gr = row0 + mloc;
    if (EPI == EPI_SWIGLU_FWD) {
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int64_t col = n0 + wn * 64 + 32 * j + 8 * q + 4 * lh;
          if (col >= N) continue;
          float h[4], g[4], u[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            g[t] = acc[i][j][4 * q + t];
            u[t] = acc[i][j + 2][4 * q + t];
            h[t] = silu_f(g[t]) * u[t];
          }
          st_bf16x4(a.C + gr * a.ldc + col, h[0], h[1], h[2], h[3]);
          if (a.G) st_bf16x4(a.G + gr * a.ldg + col, g[0], g[1], g[2], g[3]);
          if (a.U) st_bf16x4(a.U + gr * a.ldg + col, u[0], u[1], u[2], u[3]);
        }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int64_t col = n0 + wn * 128 + 32 * j + 8 * q + 4 * lh;
          if (col >= N) continue;
          const float v[4] = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
          if (EPI == EPI_STORE) {
            if (a.Cf) {
              *reinterpret_cast<f32x4*>(a.Cf + gr * a.ldc + col) = f32x4{v[0], v[1], v[2], v[3]};
            } else {
              st_bf16x4(a.C + gr * a.ldc + col, v[0], v[1], v[2], v[3]);
            }
          }
        }
    }
  }
  if (EPI == EPI_SWIGLU_BWD) {
    // v = dH; C row = [dG (N cols) | dU (N cols)].  The saved g, u of one 32-row half are fetched in one batch
    // (32 loads in flight per lane) before any output is written, so their latency is paid twice per tile
    // rather than once per 4-column group.
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int mloc = wm * 64 + 32 * i + lm;
      if (mloc >= rows) continue;
      const int64_t gr = row0 + mloc;
      u32x2 gq[4][4], uq[4][4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int64_t col = n0 + wn * 128 + 32 * j + 8 * q + 4 * lh;
          const int64_t c = col < N ? col : 0;
          gq[j][q] = *reinterpret_cast<const u32x2*>(a.G + gr * a.ldg + c);
          uq[j][q] = *reinterpret_cast<const u32x2*>(a.U + gr * a.ldg + c);
        }
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int64_t col = n0 + wn * 128 + 32 * j + 8 * q + 4 * lh;
          if (col >= N) continue;
          float dg[4], du[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const uint32_t gw = gq[j][q][t >> 1], uw = uq[j][q][t >> 1];
            const float g = __uint_as_float((t & 1) ? (gw & 0xffff0000u) : (gw << 16));
            const float u = __uint_as_float((t & 1) ? (uw & 0xffff0000u) : (uw << 16));
            const float v = acc[i][j][4 * q + t];
            const float sg = sigmoid_f(g);
            dg[t] = v * u * sg * (1.f + g * (1.f - sg));
            du[t] = v * g * sg;
          }
          st_bf16x4(a.C + gr * a.ldc + col, dg[0], dg[1], dg[2], dg[3]);
          st_bf16x4(a.C + gr * a.ldc + N + col, du[0], du[1], du[2], du[3]);
        }
    }
  }
}

// =====================================================================================================
// Weight gradient C_e[I, N] = A_e^T B_e, reduced over the rows of expert e: both operands are row-major
// [rows, .] (the reduction dim is the slow one), so both are staged N-major and read with the transpose read.
__global__ __launch_bounds__(GT, OCC) void gemm_wgrad_kernel(WgradArgs a) {
  __shared__ __attribute__((aligned(16))) bf16_t As[2][BK * NPA];
  __shared__ __attribute__((aligned(16))) bf16_t Bs[2][BK * NPB];
  const int64_t total = (int64_t)gridDim.x;
  int64_t logical = xcd_logical(blockIdx.x, total);
  const int64_t tiles_per_e = (int64_t)a.S * a.i_tiles * a.n_tiles;
  const int e = (int)(logical / tiles_per_e);
  if (e >= a.E) return;
  int64_t rem = logical % tiles_per_e;
  const int s = (int)(rem / ((int64_t)a.i_tiles * a.n_tiles));
  rem %= (int64_t)a.i_tiles * a.n_tiles;
  const int it = (int)(rem / a.n_tiles), nt = (int)(rem % a.n_tiles);
  int64_t r0, nrows;
  if (a.e_rows) {
    r0 = (int64_t)a.e_row0[e] * a.row0_mult;
    nrows = a.e_rows[e];
  } else {
    r0 = 0;
    nrows = a.dense_rows;
  }
  // rows of split s
  const int64_t chunk = ((nrows + a.S - 1) / a.S + BK - 1) / BK * BK;
  const int64_t rs = (int64_t)s * chunk;
  const int64_t re = min(nrows, rs + chunk);
  const int64_t i0 = (int64_t)it * BM, n0 = (int64_t)nt * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t I = a.I, N = a.N;

  f32x16 acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};

  const int nk = re > rs ? (int)((re - rs + BK - 1) / BK) : 0;
  // descriptors over rows [rs, re) of this expert (empty when the split has no rows)
  const int64_t span = re > rs ? re - rs : 0;
  const __amdgpu_buffer_rsrc_t rsA = make_rsrc(a.A + (r0 + rs) * a.lda, span * a.lda * 2);
  const __amdgpu_buffer_rsrc_t rsB = make_rsrc(a.B + (r0 + rs) * a.ldb, span * a.ldb * 2);
  auto load = [&](Stage& st, int kt) {
    const int rbase = kt * BK;
#pragma unroll
    for (int q = 0; q < SA; ++q) {
      const int v = tid + GT * q;
      const int rr = rbase + (v >> 4), ic = (v & 15) * 8;
      const bool ok = rr < span && i0 + ic < I;
      st.a[q] = bload16(rsA, ok ? (uint32_t)((rr * a.lda + i0 + ic) * 2) : OOB);
    }
#pragma unroll
    for (int q = 0; q < SB; ++q) {
      const int v = tid + GT * q;
      const int rr = rbase + (v >> 5), nc = (v & 31) * 8;
      const bool ok = rr < span && n0 + nc < N;
      st.b[q] = bload16(rsB, ok ? (uint32_t)((rr * a.ldb + n0 + nc) * 2) : OOB);
    }
  };
  auto store = [&](const Stage& st, int buf) {
#pragma unroll
    for (int q = 0; q < SA; ++q) {
      const int v = tid + GT * q;
      st16(&As[buf][(v >> 4) * NPA + (v & 15) * 8], st.a[q]);
    }
#pragma unroll
    for (int q = 0; q < SB; ++q) {
      const int v = tid + GT * q;
      st16(&Bs[buf][(v >> 5) * NPB + (v & 31) * 8], st.b[q]);
    }
  };
  auto compute = [&](int buf) {
    __builtin_amdgcn_iglp_opt(0);
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      bf16x8 af[2], bfr[4];
#pragma unroll
      for (int i = 0; i < 2; ++i) af[i] = frag_n(As[buf], NPA, kk, wm * 64 + 32 * i, lane);
#pragma unroll
      for (int j = 0; j < 4; ++j) bfr[j] = frag_n(Bs[buf], NPB, kk, wn * 128 + 32 * j, lane);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma32(bfr[j], af[i], acc[i][j]);
    }
  };
  // same branch-free pipeline as gemm_rows_kernel (rows past the split load as zeros)
  Stage ra, rb;
  load(ra, 0);
  load(rb, 1);
  store(ra, 0);
  load(ra, 2);
  __syncthreads();
  for (int kt = 0; kt < nk; kt += 2) {
    store(rb, 1);
    load(rb, kt + 3);
    compute(0);
    __syncthreads();
    store(ra, 0);
    load(ra, kt + 4);
    compute(1);
    __syncthreads();
  }
  // epilogue (f32): acc[i][j][4q + t] = C[i0 + wm*64 + 32 i + lane%32][n0 + wn*128 + 32 j + 8 q + 4 (lane/32) + t]
  const int lm = lane & 31, lh = lane >> 5;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int64_t row = i0 + wm * 64 + 32 * i + lm;
    if (row >= I) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t col = n0 + wn * 128 + 32 * j + 8 * q + 4 * lh;
        if (col >= N) continue;
        const f32x4 v = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
        float* dst;
        if (a.S > 1) dst = a.part + (((int64_t)s * a.E + e) * I + row) * N + col;
        else if (a.C2 && col >= a.n_split) dst = a.C2 + (int64_t)e * a.c_estride + row * a.ldc + (col - a.n_split);
        else dst = a.C + (int64_t)e * a.c_estride + row * a.ldc + col;
        *reinterpret_cast<f32x4*>(dst) = v;
      }
  }
}

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

struct GemmBlocks {
  const int32_t* blk_expert;
  const int32_t* blk_rows;
  const int32_t* blk_row0;
  const int32_t* num_blocks;
  int max_blocks;
  int64_t dense_rows;  // used when blk_expert == nullptr
};

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
  a.blk_expert = g.blk_expert; a.blk_rows = g.blk_rows; a.blk_row0 = g.blk_row0; a.num_blocks = g.num_blocks;
  a.dense_rows = g.dense_rows; a.max_blocks = max_blocks_of(g);
  a.n_tiles = (int)((N + BN - 1) / BN);
  if (a.max_blocks == 0) return LSURGE_OK;
  LSURGE_LAUNCH(kid, s, hipLaunchKernelGGL((gemm_rows_kernel<B_KN, EPI_STORE>),
                                           dim3(pad8((int64_t)a.n_tiles * a.max_blocks)), dim3(GT), 0, s, a));
  return LSURGE_OK;
}

// h = silu(A @ Bg) * (A @ Bu); also stores g, u.  Bg, Bu: [K, N] per expert.
int gemm_rows_swiglu_fwd(int kid, const GemmBlocks& g, const void* A, int64_t lda, const void* Bg, const void* Bu,
                         int64_t ldb, int64_t b_estride, int64_t K, int64_t N, void* H, void* Gs, void* Us,
                         int64_t ldh, hipStream_t s) {
  if (int rc = check_gemm_shape(K, N, "gemm_rows_swiglu_fwd")) return rc;
  if (int rc = check_desc(std::max<int64_t>(BM * lda, K * ldb) * 2, "gemm_rows_swiglu_fwd")) return rc;
  RowsArgs a{};
  a.A = (const bf16_t*)A; a.lda = lda; a.B = (const bf16_t*)Bg; a.B2 = (const bf16_t*)Bu; a.ldb = ldb;
  a.b_estride = b_estride; a.K = K; a.N = N; a.C = (bf16_t*)H; a.ldc = ldh; a.G = (bf16_t*)Gs; a.U = (bf16_t*)Us;
  a.ldg = ldh;
  a.blk_expert = g.blk_expert; a.blk_rows = g.blk_rows; a.blk_row0 = g.blk_row0; a.num_blocks = g.num_blocks;
  a.dense_rows = g.dense_rows; a.max_blocks = max_blocks_of(g);
  a.n_tiles = (int)((N + BN / 2 - 1) / (BN / 2));
  if (a.max_blocks == 0) return LSURGE_OK;
  LSURGE_LAUNCH(kid, s, hipLaunchKernelGGL((gemm_rows_kernel<B_KN, EPI_SWIGLU_FWD>),
                                           dim3(pad8((int64_t)a.n_tiles * a.max_blocks)), dim3(GT), 0, s, a));
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
  a.blk_expert = g.blk_expert; a.blk_rows = g.blk_rows; a.blk_row0 = g.blk_row0; a.num_blocks = g.num_blocks;
  a.dense_rows = g.dense_rows; a.max_blocks = max_blocks_of(g);
  a.n_tiles = (int)((N + BN - 1) / BN);
  if (a.max_blocks == 0) return LSURGE_OK;
  const dim3 grid(pad8((int64_t)a.n_tiles * a.max_blocks));
  if (swiglu_bwd)
    LSURGE_LAUNCH(kid, s, hipLaunchKernelGGL((gemm_rows_kernel<B_NK, EPI_SWIGLU_BWD>), grid, dim3(GT), 0, s, a));
  else
    LSURGE_LAUNCH(kid, s, hipLaunchKernelGGL((gemm_rows_kernel<B_NK, EPI_STORE>), grid, dim3(GT), 0, s, a));
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
               hipStream_t s) {
  if (int rc = check_gemm_shape(I, N, "gemm_wgrad")) return rc;
  if (int rc = check_desc(max_rows * std::max(lda, ldb) * 2, "gemm_wgrad")) return rc;
  LSURGE_REQUIRE(S >= 1 && E >= 1, "gemm_wgrad: bad S/E");
  WgradArgs a{};
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
  LSURGE_LAUNCH(kid, s, hipLaunchKernelGGL(gemm_wgrad_kernel, dim3(pad8(tiles)), dim3(GT), 0, s, a));
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
                            kdim * n, 1, nullptr, 0, s);
}

}  // extern "C"
