// Grouped GEMMs of the MoE layer on CDNA4 matrix cores: bf16 inputs, f32 accumulation,
// v_mfma_f32_32x32x16_bf16, 128 x 256 workgroup tiles (4 waves, 64 x 128 each), K in 32-wide stages that the
// buffer unit copies straight into a 3-deep LDS ring (buffer_load_dwordx4 ... lds), two workgroups per CU.
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
// columns of one row.  Epilogues park the accumulators in the idle LDS ring and read them back
// row-contiguous, so every global epilogue access is a 16-byte vector and 16 lanes cover a whole row.
#include "common.h"

namespace {

// Workgroup tile: BM rows (one 128-row expert block) x BN columns, 4 waves in a 2 x 2 grid of 64 x 128 wave
// tiles.  Per wave and 16-wide k step: 2 activation fragments + 4 weight fragments (6 x 1 KiB of LDS reads)
// feed 8 MFMAs.  K runs in BK = 32 stages; a stage is 8 KiB of activations + 16 KiB of weights, the ring holds
// 3 stages (72 KiB), so two workgroups share a CU's 160 KiB and one's prologue/epilogue overlaps the other's
// MFMAs.
constexpr int BM = 128, BN = 256, BK = 32;
constexpr int GT = 256;            // threads per workgroup
constexpr int OCC = 2;             // workgroups per CU

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

// ---------------------------------------------------------------------------------------------- LDS tiles
// K-major tile: rows of BK = 32 k (4 chunks of 16 B, 64 B rows, no padding).  Chunk c of row r sits at slot
// c ^ ((r >> 2) & 3): the 16 lanes that fill 4 whole rows cover 256 contiguous bytes, and the 16 lanes that
// read one chunk of 16 consecutive rows hit 16 distinct 16-byte slots of a 256-byte bank window, so neither
// direction has bank conflicts.  One 1 KiB copy instruction fills 16 rows.
__device__ __forceinline__ int km_off(int row, int chunk) { return row * BK + ((chunk ^ ((row >> 2) & 3)) << 3); }

// N-major sub-tile: BK k-rows x 128 columns (16 chunks of 16 B, 256 B rows).  Chunk c of row k sits at slot
// c ^ ((k & 3) << 2), which moves the 64-byte column group of 4 consecutive rows to 4 different 64-byte bank
// groups: a transpose read (4 rows x 64 B per 32 lanes) is conflict-free.  One copy instruction fills 4 rows.
constexpr int NS = 128;  // columns per N-major sub-tile
__device__ __forceinline__ int nm_off(int k, int n) { return k * NS + ((((n >> 3) ^ ((k & 3) << 2))) << 3) + (n & 7); }

// K-major fragment: 8 consecutive k (chunk kc) of one row -> one 16-byte LDS read
__device__ __forceinline__ bf16x8 frag_k(const bf16_t* tile, int row, int kc) {
  return as_bf16x8(*reinterpret_cast<const u32x4*>(tile + km_off(row, kc)));
}

// N-major fragment for the 32x32x16 operand layout: lane l needs rows (k) 8(l/32)+0..7 of column l%32.
// ds_read_b64_tr_b16 in a 16-lane group g: lane i receives D[4j + i/4][i%4], j = 0..3, where D[s] are the four
// 16-bit values at source lane s's address.  With source lane s pointing at (k = kb + s/4, n = nb + 4(s%4)),
// lane i receives column nb + i, rows kb..kb+3.  Two reads give the 8 k values.
__device__ __forceinline__ bf16x8 frag_n(const bf16_t* sub, int kbase, int nbase, int lane) {
  const int g = lane >> 4, s = lane & 15;
  const int n = nbase + 16 * (g & 1) + 4 * (s & 3);
  const int k0 = kbase + 8 * (g >> 1) + (s >> 2);
  const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_PTR(s16x4, sub + nm_off(k0, n)));
  const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_PTR(s16x4, sub + nm_off(k0 + 4, n)));
  typedef short s16x8 __attribute__((ext_vector_type(8)));
  const s16x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(bf16x8, v);
}

// ---------------------------------------------------------------------------------------------- global -> LDS
// Operand tiles are copied by the buffer unit straight into LDS (buffer_load_dwordx4 ... lds): lane p of a copy
// instruction writes its 16 bytes at (M0 + 16 p), so the LDS layouts above are produced by choosing which global
// chunk each lane fetches.  One descriptor per operand covers exactly the bytes the tile may read (a block's
// valid rows, an expert's weight matrix), and a lane whose element lies outside (rows past the block, K or N
// tails) passes an offset past the end, for which the buffer unit writes zeros.  No VGPR staging, no LDS store
// instructions.
//
// The copy is issued from inline asm so that the compiler does not see an LDS write: it would otherwise guard
// LDS reads with waits for every copy in flight (it cannot tell the ring slots apart through the transpose
// reads), draining the prefetch ring.  Completion is tracked by hand instead: stage_barrier<N> waits until at
// most N copies of this wave are outstanding before the workgroup barrier.
constexpr uint32_t OOB = 0x80000000u;  // every descriptor covers < 2^31 bytes (checked on the host)
__device__ __forceinline__ u32x4 make_rsrc(const void* base, int64_t bytes) {
  const uint64_t b = (uint64_t)base;
  // base (48 bits), stride 0, num_records = bytes, dword3 = 32-bit data format, no swizzle
  return u32x4{(uint32_t)b, (uint32_t)(b >> 32) & 0xffffu, (uint32_t)bytes, 0x00020000u};
}
__device__ __forceinline__ void copy16(u32x4 rsrc, uint32_t byte_off, bf16_t* lds_1k) {
  // descriptor and LDS base are wave-uniform; readfirstlane pins them to scalar registers for the asm
  const u32x4 r = {(uint32_t)__builtin_amdgcn_readfirstlane(rsrc[0]), (uint32_t)__builtin_amdgcn_readfirstlane(rsrc[1]),
                   (uint32_t)__builtin_amdgcn_readfirstlane(rsrc[2]), (uint32_t)__builtin_amdgcn_readfirstlane(rsrc[3])};
  const uint32_t m0 = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(size_t)LDS_PTR(void, lds_1k));
  asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(byte_off), "s"(r), "s"(m0)
               : "memory");
}

// Per wave and stage: A tile 8 KiB = 2 copies, B tile 16 KiB = 4 copies.
constexpr int CP_STAGE = 6;
static_assert(BM * BK * 2 / 1024 == 2 * 4 && BN * BK * 2 / 1024 == 4 * 4, "copy counts assume 4 waves");

// Wait until at most N copies of this wave are in flight and its LDS reads are done, then barrier: after it
// every wave's copies of the stage in question have landed and nobody still reads the buffer about to be
// refilled.  The barrier is an asm statement with a memory clobber so the compiler keeps LDS accesses on
// their side of it without adding a wait for all copies (which would drain the prefetch ring).
template <int N>
__device__ __forceinline__ void stage_barrier() {
  static_assert(N < 64, "vmcnt field");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (0 << 8) | ((N >> 4) << 14));  // vmcnt(N) lgkmcnt(0)
  asm volatile("s_barrier" ::: "memory");
}

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void st_bf16x4(bf16_t* p, float a, float b, float c, float d) {
  *reinterpret_cast<u32x2*>(p) = u32x2{pack_bf16x2(a, b), pack_bf16x2(c, d)};
}
__device__ __forceinline__ void st_bf16x8(bf16_t* p, const float* v) {
  *reinterpret_cast<u32x4*>(p) =
      u32x4{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7])};
}

// Epilogue staging: a wave parks 32 rows x 128 f32 columns in LDS with a row pitch of SP floats.  The 4-float
// pad shifts consecutive rows by 4 banks, so the 16-byte accumulator writes (one column group of 32 rows)
// spread over all banks.  4 waves x 32 x SP x 4 B = 66 KiB fits in the 72 KiB ring.
constexpr int SP = 132;
static_assert(4 * 32 * SP * 4 <= 3 * (BM + BN) * BK * 2, "epilogue staging must fit in the LDS ring");

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

// Run the K loop: stage kt lives in ring slot kt % 3.  Each step waits for its own stage, barriers, refills the
// slot read one step earlier with stage kt + 2, and multiplies.  Stages past the end copy zeros (out-of-range
// offsets), so every step has the same shape.  issue(slot, kt) enqueues the copies, compute(slot) the MFMAs.
template <class Issue, class Compute>
__device__ __forceinline__ void k_loop(int nk, Issue&& issue, Compute&& compute) {
  issue(0, 0);
  issue(1, 1);
  for (int kt = 0;; kt += 3) {
    stage_barrier<CP_STAGE>();
    issue(2, kt + 2);
    compute(0);
    if (kt + 1 >= nk) break;
    stage_barrier<CP_STAGE>();
    issue(0, kt + 3);
    compute(1);
    if (kt + 2 >= nk) break;
    stage_barrier<CP_STAGE>();
    issue(1, kt + 4);
    compute(2);
    if (kt + 3 >= nk) break;
  }
  __builtin_amdgcn_s_waitcnt(0);  // the copies of the zero stages past the end land before the epilogue
}

// =====================================================================================================
template <int BMODE, int EPI>
__global__ __launch_bounds__(GT, OCC) void gemm_rows_kernel(RowsArgs a) {
  // LDS ring: 3 stages of A (K-major 128 x 32) and B (K-major 256 x 32, or two N-major 32 x 128 sub-tiles).
  // After the K loop the same memory stages the epilogue.
  __shared__ __attribute__((aligned(1024))) bf16_t smem[3 * (BM + BN) * BK];
  bf16_t* const A0 = smem;
  bf16_t* const A1 = smem + BM * BK;
  bf16_t* const A2 = smem + 2 * BM * BK;
  bf16_t* const B0 = smem + 3 * BM * BK;
  bf16_t* const B1 = B0 + BN * BK;
  bf16_t* const B2 = B1 + BN * BK;

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
  // the wave index is uniform: keeping it in a scalar register keeps the copy destinations (M0) and the choice
  // of weight descriptor scalar as well
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  // column origin of this tile: weight columns for B, output columns for C (SwiGLU: gate and up halves)
  const int64_t n0 = (int64_t)nt * (EPI == EPI_SWIGLU_FWD ? BN / 2 : BN);
  const bf16_t* Bbase = a.B + (int64_t)expert * a.b_estride;
  const bf16_t* B2base = a.B2 ? a.B2 + (int64_t)expert * a.b_estride : Bbase;
  const int64_t K = a.K, N = a.N;
  const int nk = (int)((K + BK - 1) / BK);

  // descriptors: this block's rows of A; the expert's B (and B2) matrix
  const u32x4 rsA = make_rsrc(a.A + row0 * a.lda, (int64_t)rows * a.lda * 2);
  const int64_t b_bytes = (BMODE == B_NK ? N : K) * a.ldb * 2;
  const u32x4 rsB = make_rsrc(Bbase, b_bytes);
  const u32x4 rsB2 = make_rsrc(B2base, b_bytes);

  // ---- per-lane copy geometry (fixed over k): which global row / column chunk this lane fetches
  // A: copies q = 2 wave + c (c = 0, 1), 16 rows each; lane -> row 16 q + lane / 4, slot lane % 4
  int a_row[2], a_kc[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int r = 16 * (2 * wave + c) + (lane >> 2);
    a_row[c] = r;
    a_kc[c] = (lane & 3) ^ ((r >> 2) & 3);
  }
  // B K-major: copies q = 4 wave + c, 16 rows (n) each.  B N-major: sub-tile wave / 2, copies (wave & 1) * 4 + c
  // of 4 k-rows each; lane -> k row 4 q' + lane / 16, slot lane % 16.
  int b_r[4], b_c[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    if (BMODE == B_NK) {
      const int n = 16 * (4 * wave + c) + (lane >> 2);
      b_r[c] = n;
      b_c[c] = (lane & 3) ^ ((n >> 2) & 3);
    } else {
      const int k = 4 * ((wave & 1) * 4 + c) + (lane >> 4);
      b_r[c] = k;
      b_c[c] = (lane & 15) ^ ((k & 3) << 2);
    }
  }
  const bool b_sub1 = (wave >> 1) != 0;  // N-major: this wave fills sub-tile 1 (columns 128..255)

  auto issue = [&](int slot, int kt) {
    bf16_t* At = slot == 0 ? A0 : slot == 1 ? A1 : A2;
    bf16_t* Bt = slot == 0 ? B0 : slot == 1 ? B1 : B2;
    const int k0 = kt * BK;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int r = a_row[c], kk = k0 + 8 * a_kc[c];
      const bool ok = r < rows && kk < K;
      copy16(rsA, ok ? (uint32_t)((r * a.lda + kk) * 2) : OOB, At + 512 * (2 * wave + c));
    }
    if (BMODE == B_NK) {
      const bool second = a.k_split && k0 >= a.k_split;  // k range of B2 (gate/up dgrad)
      const int kb = second ? k0 - (int)a.k_split : k0;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int64_t gn = n0 + b_r[c];
        const int kk = kb + 8 * b_c[c];
        const uint32_t off = (gn < N && k0 + 8 * b_c[c] < K) ? (uint32_t)((gn * a.ldb + kk) * 2) : OOB;
        if (second) copy16(rsB2, off, Bt + 512 * (4 * wave + c));
        else copy16(rsB, off, Bt + 512 * (4 * wave + c));
      }
    } else {
      bf16_t* sub = Bt + (b_sub1 ? BK * NS : 0);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int64_t gk = k0 + b_r[c];
        int64_t gn;
        if (EPI == EPI_SWIGLU_FWD) gn = n0 + 8 * b_c[c];                      // sub-tile 0 gate, 1 up
        else gn = n0 + (b_sub1 ? NS : 0) + 8 * b_c[c];
        const uint32_t off = (gk < K && gn < N) ? (uint32_t)((gk * a.ldb + gn) * 2) : OOB;
        bf16_t* dst = sub + 512 * ((wave & 1) * 4 + c);
        if (EPI == EPI_SWIGLU_FWD && b_sub1) copy16(rsB2, off, dst);
        else copy16(rsB, off, dst);
      }
    }
  };

  f32x16 acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};

  // tile column of this wave's weight fragment j (SwiGLU: j < 2 gate, j >= 2 up, same output columns)
  auto bcol = [&](int j) {
    if (EPI == EPI_SWIGLU_FWD) return (j < 2 ? 0 : BN / 2) + wn * 64 + 32 * (j & 1);
    return wn * 128 + 32 * j;
  };
  auto compute = [&](int slot) {
    __builtin_amdgcn_iglp_opt(0);  // interleave the fragment reads with the MFMAs
    const bf16_t* at = slot == 0 ? A0 : slot == 1 ? A1 : A2;
    const bf16_t* bt = slot == 0 ? B0 : slot == 1 ? B1 : B2;
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      bf16x8 xf[2], wf[4];
#pragma unroll
      for (int i = 0; i < 2; ++i) xf[i] = frag_k(at, wm * 64 + 32 * i + (lane & 31), kk / 8 + (lane >> 5));
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int col = bcol(j);
        if (BMODE == B_NK) wf[j] = frag_k(bt, col + (lane & 31), kk / 8 + (lane >> 5));
        else wf[j] = frag_n(bt + (col >= NS ? BK * NS : 0), kk, col & (NS - 1), lane);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma32(wf[j], xf[i], acc[i][j]);
    }
  };

  k_loop(nk, issue, compute);

  // ---- epilogue, staged through LDS.  acc[i][j][4q + t] holds activation row wm*64 + 32 i + lane%32 and
  // wave column 32 j + 8 q + 4 (lane/32) + t (SwiGLU: j < 2 gate, j >= 2 up).  Written straight out, one
  // store instruction would cover 16 bytes of 32 different rows.  Instead each wave parks one 32-row half
  // of its accumulators in the (now idle) ring as f32 rows, then reads them back row-contiguous: 16 lanes x
  // 16 bytes cover a row's 128 columns, so every global load and store spans whole 128-byte lines.
  __syncthreads();  // all waves are done with the ring
  float* const stg = reinterpret_cast<float*>(smem) + wave * (32 * SP);
  const int lm = lane & 31, lh = lane >> 5;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int mbase = wm * 64 + 32 * i;  // first tile row of this half
    // SwiGLU backward: fetch the saved g, u of this half before parking the accumulators, so the loads'
    // latency overlaps the LDS round trip.  Lane -> row 4 it + lane/16, 8 columns at 8 (lane % 16).
    u32x4 gq[8], uq[8];
    if (EPI == EPI_SWIGLU_BWD) {
#pragma unroll
      for (int it = 0; it < 8; ++it) {
        const int r = 4 * it + (lane >> 4);
        const int64_t col = n0 + wn * 128 + 8 * (lane & 15);
        const bool ok = mbase + r < rows && col < N;
        const int64_t off = ok ? (row0 + mbase + r) * a.ldg + col : row0 * a.ldg;
        gq[it] = *reinterpret_cast<const u32x4*>(a.G + off);
        uq[it] = *reinterpret_cast<const u32x4*>(a.U + off);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<f32x4*>(stg + lm * SP + 32 * j + 8 * q + 4 * lh) =
            f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
    if (EPI == EPI_SWIGLU_FWD) {
      // 64 gate + 64 up columns per row: lane -> row 8 it + lane/8, 8 output columns at 8 (lane % 8)
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const int r = 8 * it + (lane >> 3), c = 8 * (lane & 7);
        const int64_t col = n0 + wn * 64 + c;
        if (mbase + r >= rows || col >= N) continue;
        const float* src = stg + r * SP + c;
        const f32x4 g0 = *reinterpret_cast<const f32x4*>(src), g1 = *reinterpret_cast<const f32x4*>(src + 4);
        const f32x4 u0 = *reinterpret_cast<const f32x4*>(src + 64), u1 = *reinterpret_cast<const f32x4*>(src + 68);
        const float g[8] = {g0[0], g0[1], g0[2], g0[3], g1[0], g1[1], g1[2], g1[3]};
        const float u[8] = {u0[0], u0[1], u0[2], u0[3], u1[0], u1[1], u1[2], u1[3]};
        float h[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) h[t] = silu_f(g[t]) * u[t];
        const int64_t gr = row0 + mbase + r;
        st_bf16x8(a.C + gr * a.ldc + col, h);
        if (a.G) st_bf16x8(a.G + gr * a.ldg + col, g);
        if (a.U) st_bf16x8(a.U + gr * a.ldg + col, u);
      }
    } else {
#pragma unroll
      for (int it = 0; it < 8; ++it) {
        const int r = 4 * it + (lane >> 4), c = 8 * (lane & 15);
        const int64_t col = n0 + wn * 128 + c;
        if (mbase + r >= rows || col >= N) continue;
        const float* src = stg + r * SP + c;
        const f32x4 v0 = *reinterpret_cast<const f32x4*>(src), v1 = *reinterpret_cast<const f32x4*>(src + 4);
        const int64_t gr = row0 + mbase + r;
        if (EPI == EPI_STORE) {
          if (a.Cf) {
            *reinterpret_cast<f32x4*>(a.Cf + gr * a.ldc + col) = v0;
            *reinterpret_cast<f32x4*>(a.Cf + gr * a.ldc + col + 4) = v1;
          } else {
            const float v[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
            st_bf16x8(a.C + gr * a.ldc + col, v);
          }
        } else {  // EPI_SWIGLU_BWD: v = dH; C row = [dG (N cols) | dU (N cols)]
          const float v[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
          float dg[8], du[8];
#pragma unroll
          for (int t = 0; t < 8; ++t) {
            const uint32_t gw = gq[it][t >> 1], uw = uq[it][t >> 1];
            const float g = __uint_as_float((t & 1) ? (gw & 0xffff0000u) : (gw << 16));
            const float u = __uint_as_float((t & 1) ? (uw & 0xffff0000u) : (uw << 16));
            const float sg = sigmoid_f(g);
            dg[t] = v[t] * u * sg * (1.f + g * (1.f - sg));
            du[t] = v[t] * g * sg;
          }
          st_bf16x8(a.C + gr * a.ldc + col, dg);
          st_bf16x8(a.C + gr * a.ldc + N + col, du);
        }
      }
    }
  }
}

// =====================================================================================================
// Weight gradient C_e[I, N] = A_e^T B_e, reduced over the rows of expert e: both operands are row-major
// [rows, .] (the reduction dim is the slow one), so both are staged N-major and read with the transpose read.
__global__ __launch_bounds__(GT, OCC) void gemm_wgrad_kernel(WgradArgs a) {
  // ring: A 32 rows x 128 columns (one N-major sub-tile), B 32 rows x 256 columns (two sub-tiles); after the
  // K loop the same memory stages the epilogue
  __shared__ __attribute__((aligned(1024))) bf16_t smem[3 * (NS + BN) * BK];
  bf16_t* const A0 = smem;
  bf16_t* const A1 = smem + BK * NS;
  bf16_t* const A2 = smem + 2 * BK * NS;
  bf16_t* const B0 = smem + 3 * BK * NS;
  bf16_t* const B1 = B0 + BK * BN;
  bf16_t* const B2 = B1 + BK * BN;
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
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
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
  const u32x4 rsA = make_rsrc(a.A + (r0 + rs) * a.lda, span * a.lda * 2);
  const u32x4 rsB = make_rsrc(a.B + (r0 + rs) * a.ldb, span * a.ldb * 2);
  // copies: A sub-tile 8 copies of 4 rows (wave w: 2 w, 2 w + 1); B 16 copies (wave w: sub-tile w / 2,
  // copies (w & 1) * 4 + c)
  int a_k[2], a_c[2], b_k[4], b_c[4];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    a_k[c] = 4 * (2 * wave + c) + (lane >> 4);
    a_c[c] = (lane & 15) ^ ((a_k[c] & 3) << 2);
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    b_k[c] = 4 * ((wave & 1) * 4 + c) + (lane >> 4);
    b_c[c] = (lane & 15) ^ ((b_k[c] & 3) << 2);
  }
  const int b_sub = wave >> 1;
  auto issue = [&](int slot, int kt) {
    bf16_t* At = slot == 0 ? A0 : slot == 1 ? A1 : A2;
    bf16_t* Bt = slot == 0 ? B0 : slot == 1 ? B1 : B2;
    const int rb = kt * BK;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int rr = rb + a_k[c];
      const int64_t ic = i0 + 8 * a_c[c];
      copy16(rsA, (rr < span && ic < I) ? (uint32_t)((rr * a.lda + ic) * 2) : OOB, At + 512 * (2 * wave + c));
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int rr = rb + b_k[c];
      const int64_t nc = n0 + NS * b_sub + 8 * b_c[c];
      copy16(rsB, (rr < span && nc < N) ? (uint32_t)((rr * a.ldb + nc) * 2) : OOB,
             Bt + BK * NS * b_sub + 512 * ((wave & 1) * 4 + c));
    }
  };
  auto compute = [&](int slot) {
    __builtin_amdgcn_iglp_opt(0);
    const bf16_t* at = slot == 0 ? A0 : slot == 1 ? A1 : A2;
    const bf16_t* bt = slot == 0 ? B0 : slot == 1 ? B1 : B2;
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      bf16x8 af[2], bfr[4];
#pragma unroll
      for (int i = 0; i < 2; ++i) af[i] = frag_n(at, kk, wm * 64 + 32 * i, lane);
#pragma unroll
      for (int j = 0; j < 4; ++j) bfr[j] = frag_n(bt + BK * NS * wn, kk, 32 * j, lane);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma32(bfr[j], af[i], acc[i][j]);
    }
  };
  k_loop(nk, issue, compute);

  // epilogue (f32), staged through LDS as in gemm_rows_kernel: acc[i][j][4q + t] is C row
  // i0 + wm*64 + 32 i + lane%32, column n0 + wn*128 + 32 j + 8 q + 4 (lane/32) + t.  Read back with 16 lanes
  // per row, each store instruction covers 4 rows x 512 contiguous bytes.
  __syncthreads();  // all waves are done with the ring
  float* const stg = reinterpret_cast<float*>(smem) + wave * (32 * SP);
  const int lm = lane & 31, lh = lane >> 5;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<f32x4*>(stg + lm * SP + 32 * j + 8 * q + 4 * lh) =
            f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
#pragma unroll
    for (int r8 = 0; r8 < 8; ++r8) {
      const int r = 4 * r8 + (lane >> 4), c = 8 * (lane & 15);
      const int64_t row = i0 + wm * 64 + 32 * i + r;
      if (row >= I) continue;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int64_t col = n0 + wn * 128 + c + 4 * h;
        if (col >= N) continue;
        const f32x4 v = *reinterpret_cast<const f32x4*>(stg + r * SP + c + 4 * h);
        float* dst;
        if (a.S > 1) dst = a.part + (((int64_t)s * a.E + e) * I + row) * N + col;
        else if (a.C2 && col >= a.n_split) dst = a.C2 + (int64_t)e * a.c_estride + row * a.ldc + (col - a.n_split);
        else dst = a.C + (int64_t)e * a.c_estride + row * a.ldc + col;
        *reinterpret_cast<f32x4*>(dst) = v;
      }
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
