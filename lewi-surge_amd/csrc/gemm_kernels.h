// Grouped-GEMM kernels of the MoE layer on CDNA4 matrix cores: bf16 inputs, f32 accumulation,
// v_mfma_f32_32x32x16_bf16.  The tile shape is a template parameter (GemmCfg): BM x BN workgroup tiles split
// over WM x WN waves, K in BK-wide stages that the buffer unit copies straight into an ST-deep LDS ring
// (buffer_load_dwordx4 ... lds).  gemm.hip instantiates the shapes the layer uses.
//
// Replaces the padded batched einsum of modal/padded_gmm.py:66-69 (cuBLAS on the reference's GPU path) and
// its autodiff.  Two kernel families:
//
//  gemm_rows   row-tiled: C[tile rows, n-tile] = A[tile rows, :] @ B[expert(tile)].  A row tile is up to BM
//              consecutive rows of one expert, looked up in a device tile table (128-row padded blocks, or
//              256-row pairs of an expert's consecutive blocks).  Tiles past the device-side tile count exit at
//              once, so padding tiles cost nothing; rows past a tile's valid count are loaded as zeros.
//              B either K-major ([N, K], read with ds_read_b128) or N-major ([K, N], read with the gfx950
//              LDS transpose read ds_read_b64_tr_b16).  Epilogues: plain store (bf16 or f32), SwiGLU forward
//              (gate and up columns side by side in one accumulator set -> h = silu(g) * u, plus g and u
//              for the backward), SwiGLU backward (dH -> dG, dU from the saved g, u).
//  gemm_wgrad  per-expert weight gradient: C_e = A_e^T @ B_e with the reduction over the expert's rows
//              (ragged K); both operands N-major in LDS, transpose-read.  Optional split of the rows into
//              S slices with f32 partials summed afterwards in a fixed order (deterministic, no atomics).
// The MFMA operands are passed weight-first, so each lane's accumulators hold four consecutive output
// columns of one row.  Epilogues park the accumulators in the idle LDS ring and read them back
// row-contiguous, so every global epilogue access is a 16-byte vector and a few lanes cover a whole row.
//
// Every output element is the same ascending sequence of 16-deep MFMA steps whatever the tile shape, so all
// shapes give bitwise identical results.
//
// FP8 variant of gemm_rows (template flag F8): B in OCP E4M3, A in E4M3 (F8 = 1) or E5M2 (F8 = 2, a gradient), both
// K-contiguous, v_mfma_f32_32x32x64_f8f6f4.  The operands move through the same copy and LDS machinery counted in
// 2-byte units, so a 32-unit stage holds 64 values of k, one MFMA step; the epilogue multiplies the accumulators by
// the dequantisation factors (per-tensor for A, per expert for B and B2) before the usual epilogues.  With a k split
// (B up to k_split, B2 after it: the gate/up dgrad) the two weights keep scales of their own: at the first B2 stage
// the accumulators are multiplied by b_sinv / b2_sinv, and the epilogue by a_sinv b2_sinv.
// gemm_wgrad_f8_kernel is the FP8 weight gradient: it stages the row-major FP8 tensors N-major like the bf16 weight
// gradient and reads K-contiguous fragments with the 8-bit LDS transpose read.
#pragma once
#include <type_traits>

#include "common.h"

namespace lsgemm {

enum { B_NK = 0, B_KN = 1 };                        // B operand storage
enum { EPI_STORE = 0, EPI_SWIGLU_FWD = 1, EPI_SWIGLU_BWD = 2 };

constexpr int NS = 128;  // columns per N-major LDS sub-tile (256-byte rows)

// Tile shape: BM x BN per workgroup, WM x WN waves (wave tile TM x TN = FM x FN fragments of 32 x 32), K in
// BK-deep stages, an ST-stage LDS ring, OCC workgroups per CU.  PP selects the ping-pong K loop (k_loop_pp): eight
// waves in two groups of four, one wave of each group per SIMD, taking turns between the matrix pipe and the
// memory pipes.
template <int BM_, int BN_, int BK_, int WM_, int WN_, int ST_, int OCC_, int PP_ = 0>
struct GemmCfg {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_, ST = ST_, OCC = OCC_, PP = PP_;
  static constexpr int NW = WM * WN, GT = 64 * NW;
  static constexpr int TM = BM / WM, TN = BN / WN, FM = TM / 32, FN = TN / 32;
  static constexpr int A_EL = BM * BK, B_EL = BN * BK;                   // bf16 elements per stage
  static constexpr int CPA = A_EL * 2 / 1024 / NW, CPB = B_EL * 2 / 1024 / NW, CP = CPA + CPB;  // copies per wave
  static constexpr int RING_EL = ST * (A_EL + B_EL);
  static constexpr int SP = TN + 4;                  // epilogue staging pitch (f32)
  static constexpr int STG_EL = NW * 32 * SP * 2;    // epilogue staging, in bf16 element units
  static constexpr int SMEM_EL = RING_EL > STG_EL ? RING_EL : STG_EL;
  static_assert(BK == 32 || BK == 64, "BK");
  static_assert(TM % 32 == 0 && TN % 64 == 0 && BN % NS == 0 && BM % NS == 0, "tile");
  static_assert(CPA * NW * 1024 == A_EL * 2 && CPB * NW * 1024 == B_EL * 2, "copies must split evenly over waves");
  static_assert((ST - 1) * CP < 64 && ST >= 2, "vmcnt field");
  static_assert(SMEM_EL * 2 <= 160 * 1024 / OCC, "LDS");
  static_assert(!PP || (NW == 8 && WM == 2 && OCC == 1 && ST >= 3), "ping-pong: 8 waves, groups = wave rows");
};

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
  const int32_t* t_expert;   // tile table (nullptr: dense, expert 0, rows = min(BM, dense_rows - BM t))
  const int32_t* t_rows;     // valid rows of tile t
  const int32_t* t_row0;     // first row of tile t (nullptr: BM t)
  const int32_t* num_tiles;  // device-side tile count
  const int32_t* a_rows;     // row gather: A row r of the tile is A[a_rows[row0 + r] / a_div] (< 0: zero row),
  int64_t a_nrows;           // A spans a_nrows rows; nullptr: the tile's rows are A[row0 .. row0 + rows)
  int a_div;
  int64_t dense_rows;
  int n_tiles;               // column tiles
  int max_tiles;             // row tiles the grid covers
  int x_expert = -1;         // tiles of this expert id read Bx / B2x instead of B / B2 (-1: none); the layer's
  const bf16_t* Bx = nullptr;   // shared expert rides along the routed ones as expert E
  const bf16_t* B2x = nullptr;
  // FP8 (F8 kernels only; A, B and B2 point at FP8 bytes and K, lda, ldb, b_estride count them): dequantisation
  // factors of A (one value) and of B / B2 (one per expert)
  const float* a_sinv = nullptr;
  const float* b_sinv = nullptr;
  const float* b2_sinv = nullptr;
  // SwiGLU forward: atomic max of |h|; FP8 SwiGLU backward: of |dG| and |dU|; as bf16-rounded float bits (nullptr:
  // none)
  uint32_t* amax = nullptr;
  // SwiGLU backward (bf16): dH row r of a tile is multiplied by row_scale[row0 + r] (indexed by padded row) before
  // the SwiGLU backward, except in tiles of x_expert (scale 1); nullptr: no scaling.  The layer's routing weights,
  // applied to dY @ W_down^T instead of to the dY rows.
  const float* row_scale = nullptr;
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
  const int32_t* a_rows;  // row gather of A: reduction row r (an index into the expert's row range) reads
  int64_t a_nrows;        // A[a_rows[r] / a_div] of an A with a_nrows rows; nullptr: A's rows are contiguous
  int a_div;
  // Chunk table (replaces e_row0 / e_rows / S when set): chunk c reduces rows [c_row0[c], c_row0[c] + c_rows[c])
  // of expert c_expert[c] and writes C (c_part[c] < 0: the expert's only chunk) or the f32 partial slot
  // part + c_part[c] * I * N, summed afterwards in chunk order.  Chunks of at most a few thousand rows keep
  // one hot expert from serialising the whole launch behind its few tiles.
  const int32_t* c_expert;
  const int32_t* c_row0;
  const int32_t* c_rows;
  const int32_t* c_part;
  const int32_t* num_chunks;  // device-side chunk count
  int max_chunks;             // chunks the grid covers
  int x_expert = -1;          // this expert id writes Cx / C2x (row pitch ldc) instead of C / C2 (-1: none)
  float* Cx = nullptr;
  float* C2x = nullptr;
  // Row gather of B instead of A (persistent kernel only): reduction row r reads B[a_rows[r] / a_div] of a B with
  // b_nrows rows, times b_scale[r] (indexed by padded row like a_rows; chunks of x_expert: times 1), rounded to bf16
  // as the staged operand -- the layer's dY rows scaled by their routing weight, as the combine backward would have
  // written them.
  bool gather_b = false;
  int64_t b_nrows = 0;
  const float* b_scale = nullptr;
  // FP8 (gemm_wgrad_f8_kernel): A = [I, lda] and B = [N, ldb] bytes, K-contiguous over the rows; dequantisation
  // factors of each (one value)
  const float* a_sinv = nullptr;
  const float* b_sinv = nullptr;
};

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// D[32 x 32] += P[32 x 16] Q[16 x 32]; lane l supplies row l%32 of P and column l%32 of Q, k = 8(l/32)..+7.
// The kernels call it with P = the weight fragment and Q = the activation fragment, so the accumulator holds
// C^T: lane l owns activation row l%32 and output columns 8(r/4) + 4(l/32) + r%4 -- four consecutive columns
// per register quad.
// ET = LSURGE_F16: the same fragments hold IEEE half bit patterns (v_mfma_f32_32x32x16_f16, same operand layout).
template <int ET = LSURGE_BF16>
__device__ __forceinline__ f32x16 mfma32(bf16x8 p, bf16x8 q, f32x16 c) {
  if constexpr (ET == LSURGE_F16) {
    typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, p), __builtin_bit_cast(f16x8, q), c, 0, 0,
                                                  0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(p, q, c, 0, 0, 0);
  }
}

// D[32 x 32] += P[32 x 64] Q[64 x 32] with FP8 operands of formats FP, FQ (0 = E4M3, 1 = E5M2); with zero scale
// operands the compiler emits the unscaled v_mfma_f32_32x32x64_f8f6f4.  Lane l supplies row l%32 of P and column
// l%32 of Q as 32 bytes; P and Q take their bytes from the same k positions, and D sums over all 64, so which k a
// byte slot stands for never matters.  Same output layout as mfma32.
template <int FP = 0, int FQ = 0>
__device__ __forceinline__ f32x16 mfma32_f8(i32x8 p, i32x8 q, f32x16 c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(p, q, c, FP, FQ, 0, 0, 0, 0);
}

// ---------------------------------------------------------------------------------------------- LDS tiles
// K-major tile: rows of BK k (BK/8 chunks of 16 B; 64 B rows for BK = 32, 128 B rows for BK = 64), no padding.
// Chunk c of row r sits at slot c ^ swz(r).  A fragment read takes one chunk of 32 consecutive rows; the 16
// lanes of each read phase then hit 16 distinct 16-byte slots of a 256-byte bank window:
//   BK = 32: granule 4 (r & 3) + (c ^ ((r >> 2) & 3))      BK = 64: granule 8 (r & 1) + (c ^ ((r >> 1) & 7))
// and a copy instruction writes 1 KiB contiguously, so neither direction has bank conflicts.
template <int BK>
__device__ __forceinline__ int km_swz(int row) { return BK == 32 ? (row >> 2) & 3 : (row >> 1) & 7; }
template <int BK>
__device__ __forceinline__ int km_off(int row, int chunk) { return row * BK + ((chunk ^ km_swz<BK>(row)) << 3); }

// FP8 fragment of a 32-unit (64-byte) K-major row: lane half h takes chunks h and h + 2, 32 of the stage's 64 k
__device__ __forceinline__ i32x8 frag_k8(const bf16_t* tile, int row, int h) {
  const u32x4 lo = *reinterpret_cast<const u32x4*>(tile + km_off<32>(row, h));
  const u32x4 hi = *reinterpret_cast<const u32x4*>(tile + km_off<32>(row, h + 2));
  return i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
}

// N-major sub-tile: BK k-rows x 128 columns (16 chunks of 16 B, 256 B rows).  Chunk c of row k sits at slot
// c ^ ((k & 3) << 2), which moves the 64-byte column group of 4 consecutive rows to 4 different 64-byte bank
// groups: a transpose read (4 rows x 64 B per 32 lanes) is conflict-free.  One copy instruction fills 4 rows.
__device__ __forceinline__ int nm_off(int k, int n) { return k * NS + ((((n >> 3) ^ ((k & 3) << 2))) << 3) + (n & 7); }

// K-major fragment: 8 consecutive k (chunk kc) of one row -> one 16-byte LDS read
template <int BK>
__device__ __forceinline__ bf16x8 frag_k(const bf16_t* tile, int row, int kc) {
  return as_bf16x8(*reinterpret_cast<const u32x4*>(tile + km_off<BK>(row, kc)));
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
// chunk each lane fetches.  One descriptor per operand covers exactly the bytes the tile may read (a tile's
// valid rows, an expert's weight matrix), and a lane whose element lies outside (rows past the tile, K or N
// tails) passes an offset past the end, for which the buffer unit writes zeros.  No VGPR staging, no LDS store
// instructions.
//
// The copy is issued from inline asm so that the compiler does not see an LDS write: it would otherwise guard
// LDS reads with waits for every copy in flight (it cannot tell the ring slots apart through the transpose
// reads), draining the prefetch ring.  Completion is tracked by hand instead: stage_barrier<N> waits until at
// most N copies of this wave are outstanding before the workgroup barrier.
constexpr uint32_t OOB = 0x80000000u;  // every descriptor covers < 2^31 bytes (checked on the host)
constexpr int KBIG = 1 << 30;          // per-lane k of a chunk outside the operand: never below K
__device__ __forceinline__ u32x4 make_rsrc(const void* base, int64_t bytes) {
  const uint64_t b = (uint64_t)base;
  // base (48 bits), stride 0, num_records = bytes, dword3 = 32-bit data format, no swizzle; all wave-uniform,
  // readfirstlane keeps the descriptor in scalar registers for the copies
  return u32x4{(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b),
               (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32) & 0xffffu),
               (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)bytes), 0x00020000u};
}
// One 1 KiB copy: lane p's 16 bytes at byte_off of the buffer land at LDS byte address m0 + 16 p.  m0 is the
// wave-uniform LDS address of the destination (the LDS base of the kernel's array plus a constant offset).
__device__ __forceinline__ void copy16(u32x4 rsrc, uint32_t byte_off, uint32_t m0) {
  // m0 is uniform by construction; readfirstlane states it for the compiler (free when already scalar)
  const uint32_t m0s = (uint32_t)__builtin_amdgcn_readfirstlane(m0);
  asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(byte_off), "s"(rsrc), "s"(m0s)
               : "memory");
}
// n / d for 0 <= n < 2^31 and 1 <= d <= 256 as one 64-bit multiply: with m = ceil(2^40 / d),
// n m / 2^40 = n / d + n (m - 2^40 / d) / 2^40, and the error term stays below 1 / d for n < 2^40 / d.
__device__ __forceinline__ uint64_t div_magic(int d) { return ((1ull << 40) + (uint64_t)d - 1) / (uint64_t)d; }
__device__ __forceinline__ int div_by(int n, uint64_t magic) { return (int)(((uint64_t)(uint32_t)n * magic) >> 40); }

// LDS byte address of the kernel's shared array, as a scalar
__device__ __forceinline__ uint32_t lds_addr(const bf16_t* p) {
  return (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(size_t)LDS_PTR(const void, p));
}

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

// Software-pipelined K loop over an ST-deep ring; stage kt lives in slot kt % ST and a stage is KS = BK / 16
// MFMA steps.  The fragments of step n + 1 are read from LDS (into the other half of a double buffer) before the
// MFMAs of step n are issued, so the matrix pipe never waits for an LDS read.  The stage switch happens inside
// the last step of a stage: wait until the next stage has landed (at most ST - 2 younger stages in flight),
// barrier -- after which every wave has also finished reading the current slot -- refill the current slot with
// stage kt + ST, read the next stage's first fragments, then issue the last step's MFMAs.  Stages past the end
// copy zeros (out-of-range offsets), so every step has the same shape and the wait counts stay exact.
//   issue(slot, kt)     enqueue the copies of stage kt into ring slot `slot`
//   load(slot, s, F)    read the fragments of step s of the stage in `slot` into F
//   mma(F)              the MFMAs of one step
// One pass of the outer loop covers R = ST stages (2 ST when ST KS is odd), so that the fragment buffer a step
// uses is fixed at compile time.
template <int ST, int CP, int KS, class Frags, class Issue, class Load, class Mma>
__device__ __forceinline__ void k_loop(int nk, Issue&& issue, Load&& load, Mma&& mma) {
  constexpr int R = (ST * KS) % 2 ? 2 * ST : ST;
#pragma unroll
  for (int s = 0; s < ST; ++s) issue(s, s);
  stage_barrier<(ST - 1) * CP>();
  Frags f0, f1;
  load(0, 0, f0);
  for (int kt0 = 0;; kt0 += R) {
    bool done = false;
#pragma unroll
    for (int j = 0; j < R; ++j) {
      if (!done) {
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const int step = j * KS + s;
          Frags& cur = (step & 1) ? f1 : f0;
          Frags& nxt = (step & 1) ? f0 : f1;
          if (s + 1 < KS) {
            load(j % ST, s + 1, nxt);
          } else {
            stage_barrier<(ST - 2) * CP>();
            issue(j % ST, kt0 + j + ST);
            load((j + 1) % ST, 0, nxt);
          }
          // keep the reads of the next step ahead of this step's MFMAs (the scheduler would otherwise sink
          // each read to just before its first use and the MFMAs would wait on LDS latency again)
          __builtin_amdgcn_sched_barrier(0);
          mma(cur);
          __builtin_amdgcn_sched_barrier(0);  // and this step's MFMAs ahead of the next stage barrier
        }
        done = kt0 + j + 1 >= nk;
      }
    }
    if (done) break;
  }
  __builtin_amdgcn_s_waitcnt(0);  // the copies of the zero stages past the end land before the epilogue
}

// vmcnt(N) alone (expcnt and lgkmcnt at their maxima: no wait on them)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N < 64, "vmcnt field");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(0xC07F); }  // lgkmcnt(0) alone
__device__ __forceinline__ void wg_barrier() { asm volatile("s_barrier" ::: "memory"); }

// Ping-pong K loop.  The eight waves form two groups of four (group = wave / 4; waves w and w + 4 share SIMD w % 4)
// that alternate between a memory phase -- read all fragments of stage i from LDS, enqueue the copies of stage
// i + ST - 1 -- and a compute phase -- the MFMAs of stage i from registers -- with a workgroup barrier between
// phases.  Group 1 runs one phase behind group 0, so on every SIMD one wave feeds the matrix pipe while the other
// issues its LDS reads and copies.  Barrier b starts phase b; group 0 does memory(i) in phase 2i and compute(i) in
// 2i + 1, group 1 memory(i) in 2i + 1 and compute(i) in 2i + 2.
//  - Data ready: every wave waits until at most ST - 2 younger stages of its own copies are in flight before the
//    barrier that starts phase 2i + 2 (group 0 after compute(i), group 1 after memory(i)), so stage i + 1 has
//    landed everywhere before group 0 reads it in phase 2i + 2 (and group 1 in 2i + 3).
//  - Slot reuse: stage i + ST - 1 overwrites the slot of stage i - 1, whose last reader is group 1's memory phase
//    2i - 1; group 1 drains its LDS reads before the barrier that ends it, and group 0 enqueues the copies in
//    phase 2i, group 1 in 2i + 1.
// Both groups pass 2 nk + 2 barriers (group 1 one extra at the start, group 0 one at the end).  Stages past the
// end copy zeros (out-of-range offsets), so the wait counts stay exact.
template <int ST, int CP, int KS, class Frags, class Issue, class Load, class Mma>
__device__ __forceinline__ void k_loop_pp(int nk, int grp, Issue&& issue, Load&& load, Mma&& mma) {
  static_assert(ST >= 3, "ping-pong ring depth");
#pragma unroll
  for (int s = 0; s < ST - 1; ++s) issue(s, s);
  wait_vmcnt<(ST - 2) * CP>();
  wg_barrier();
  if (grp == 1) wg_barrier();
  Frags f[KS];
  int slot = 0;
  for (int i = 0; i < nk; ++i) {
    // memory phase
#pragma unroll
    for (int s = 0; s < KS; ++s) load(slot, s, f[s]);
    const int refill = slot == 0 ? ST - 1 : slot - 1;
    issue(refill, i + ST - 1);
    if (grp == 1) {
      wait_vmcnt<(ST - 2) * CP>();
      wait_lgkmcnt0();
    }
    __builtin_amdgcn_sched_barrier(0);
    wg_barrier();
    // compute phase
#pragma unroll
    for (int s = 0; s < KS; ++s) mma(f[s]);
    __builtin_amdgcn_sched_barrier(0);
    if (grp == 0) wait_vmcnt<(ST - 2) * CP>();
    wg_barrier();
    slot = slot == ST - 1 ? 0 : slot + 1;
  }
  if (grp == 0) wg_barrier();
  __builtin_amdgcn_s_waitcnt(0);  // the copies of the zero stages past the end land before the epilogue
}

// Single-buffered K loop for one MFMA step per stage: wait until stage kt has landed (at most ST - 2 younger stages
// in flight) and barrier -- after which every wave is also done with the slot of stage kt - 1 --, refill that slot
// with stage kt + ST - 1, then read stage kt's fragments and issue its MFMAs.  No fragment double buffer: the
// registers it saves keep two workgroups on a CU, and the other workgroup's waves cover this one's LDS reads.
template <int ST, int CP, class Frags, class Issue, class Load, class Mma>
__device__ __forceinline__ void k_loop_sb(int nk, Issue&& issue, Load&& load, Mma&& mma) {
#pragma unroll
  for (int s = 0; s < ST - 1; ++s) issue(s, s);
  int slot = 0;
  for (int kt = 0; kt < nk; ++kt) {
    stage_barrier<(ST - 2) * CP>();
    issue(slot == 0 ? ST - 1 : slot - 1, kt + ST - 1);
    Frags f;
    load(slot, 0, f);
    mma(f);
    slot = slot == ST - 1 ? 0 : slot + 1;
  }
  __builtin_amdgcn_s_waitcnt(0);  // the copies of the zero stages past the end land before the epilogue
}

// KS: MFMA steps per stage (BK / 16 for bf16, 1 for an FP8 stage of 64 values).  SB: the single-buffered loop
// (4-wave FP8).
template <class Cfg, class Frags, int KS = Cfg::BK / 16, bool SB = false, class Issue, class Load, class Mma>
__device__ __forceinline__ void run_k_loop(int nk, int wave, Issue&& issue, Load&& load, Mma&& mma) {
  if constexpr (Cfg::PP) k_loop_pp<Cfg::ST, Cfg::CP, KS, Frags>(nk, wave >> 2, issue, load, mma);
  else if constexpr (SB) k_loop_sb<Cfg::ST, Cfg::CP, Frags>(nk, issue, load, mma);
  else k_loop<Cfg::ST, Cfg::CP, KS, Frags>(nk, issue, load, mma);
}

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void st_bf16x8(bf16_t* p, const float* v) {
  *reinterpret_cast<u32x4*>(p) =
      u32x4{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7])};
}
// 8 f32 -> 8 16-bit values of element type ET (round to nearest even), one 16-byte store
template <int ET>
__device__ __forceinline__ void st_x8(bf16_t* p, const float* v) {
  if constexpr (ET == LSURGE_F16) {
    uint32_t u[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) u[i] = (uint32_t)f32_to_f16(v[2 * i]) | ((uint32_t)f32_to_f16(v[2 * i + 1]) << 16);
    *reinterpret_cast<u32x4*>(p) = u32x4{u[0], u[1], u[2], u[3]};
  } else {
    st_bf16x8(p, v);
  }
}

// 1 / (1 + e^-g) with the hardware reciprocal (about 1 ulp): plenty for bf16 outputs, and it keeps the
// epilogue short
__device__ __forceinline__ float sigmoid_f(float g) { return __builtin_amdgcn_rcpf(1.f + __expf(-g)); }
__device__ __forceinline__ float silu_f(float g) { return g * sigmoid_f(g); }

// XCD-aware tile order: workgroups are dispatched round-robin over the 8 XCDs, so consecutive logical
// tiles (same expert tile, neighbouring N tiles and experts) are sent to the same XCD's L2.
__device__ __forceinline__ int64_t xcd_logical(int64_t id, int64_t total) {
  const int64_t per = total / 8;
  return (id % 8) * per + id / 8;
}

// Tile of a chunk-table launch (grid = 8 x ceil(max_chunks / 8) x tpc tiles per chunk, nch chunks real): chunk c runs
// on XCD c % 8 with its tiles consecutive there, so the chunks that exist are spread evenly over the XCDs, and a hot
// expert's chunks too.  With fewer chunks than XCDs that would leave XCDs idle (one chunk: 1/8 of the chip), so there
// every XCD takes an equal contiguous share of all nch * tpc tiles instead.  -1: no tile for this workgroup.
__device__ __forceinline__ int64_t chunk_logical(int64_t tpc, int nch) {
  const int64_t l = blockIdx.x / 8, x = blockIdx.x % 8;
  if (nch >= 8) return (8 * (l / tpc) + x) * tpc + l % tpc;
  const int64_t all = (int64_t)nch * tpc, b = x * all / 8;
  return l < (x + 1) * all / 8 - b ? b + l : -1;
}

// Park fragment row i of the accumulators (32 rows x TN f32 columns) in this wave's staging area.
// acc[i][j][4q + t] is row lane%32, wave column 32 j + 8 q + 4 (lane/32) + t.
template <class Cfg>
__device__ __forceinline__ void park(float* stg, const f32x16 (&acc)[Cfg::FM][Cfg::FN], int i, int lane) {
  const int lm = lane & 31, lh = lane >> 5;
#pragma unroll
  for (int j = 0; j < Cfg::FN; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      *reinterpret_cast<f32x4*>(stg + lm * Cfg::SP + 32 * j + 8 * q + 4 * lh) =
          f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
}

template <int FM, int FN, class FT = bf16x8>
struct FragSet {
  FT x[FM], w[FN];
};

// =====================================================================================================
template <class Cfg, int BMODE, int EPI, int F8 = 0, int ET = LSURGE_BF16>
__global__ __launch_bounds__(Cfg::GT) __attribute__((amdgpu_waves_per_eu(Cfg::NW * Cfg::OCC / 4)))
void gemm_rows_kernel(RowsArgs a) {
  static_assert(!F8 || (BMODE == B_NK && Cfg::BK == 32), "FP8: both operands K-contiguous, 64-value stages");
  static_assert(ET == LSURGE_BF16 || (EPI == EPI_STORE && !F8), "f16 operands: plain store epilogue only");
  static_assert(EPI != EPI_SWIGLU_FWD || (Cfg::BN / NS) % 2 == 0,
                "SwiGLU forward: the gate and up halves need whole N-major sub-tiles each (BN a multiple of 256)");
  constexpr int UE = F8 ? 2 : 1;  // operand elements per 2-byte copy unit
  constexpr int BM = Cfg::BM, BN = Cfg::BN, BK = Cfg::BK, ST = Cfg::ST;
  constexpr int TM = Cfg::TM, TN = Cfg::TN, FM = Cfg::FM, FN = Cfg::FN, SP = Cfg::SP;
  constexpr int CPA = Cfg::CPA, CPB = Cfg::CPB;
  constexpr int RPC = 1024 / (2 * BK), CPR = BK / 8;  // K-major copy: rows per copy, chunks per row
  constexpr int NSUB = BN / NS;                      // N-major B: sub-tiles
  constexpr int CPS = BK / 4;                        // N-major: copies per sub-tile
  // LDS ring: ST stages of A (K-major BM x BK) and B (K-major BN x BK, or NSUB N-major BK x 128 sub-tiles).
  // After the K loop the same memory stages the epilogue.
  __shared__ __attribute__((aligned(1024))) bf16_t smem[Cfg::SMEM_EL];
  constexpr uint32_t A_SLOT = Cfg::A_EL * 2, B_SLOT = Cfg::B_EL * 2, B_RING = ST * A_SLOT;  // bytes

  // XCD-aware tile order over the tiles that exist: with a tile table the grid covers the bound max_tiles, but only
  // num_tiles row tiles are real, so the per-XCD ranges are cut from the device-side count (an XCD whose range
  // would start past the real tiles would otherwise sit idle while the others take its share).
  int64_t logical;
  if (a.t_expert) {
    const int64_t real = (int64_t)min(a.num_tiles[0], a.max_tiles) * a.n_tiles;
    const int64_t per = (real + 7) / 8, l = blockIdx.x / 8;
    if (l >= per) return;
    logical = (blockIdx.x % 8) * per + l;
    if (logical >= real) return;
  } else {
    logical = xcd_logical(blockIdx.x, (int64_t)gridDim.x);
  }
  const int nt = (int)(logical % a.n_tiles);
  const int b = (int)(logical / a.n_tiles);
  if (b >= a.max_tiles) return;
  int expert, rows;
  int64_t row0;
  if (a.t_expert) {
    expert = a.t_expert[b];
    rows = a.t_rows[b];
    row0 = a.t_row0 ? (int64_t)a.t_row0[b] : (int64_t)b * BM;
  } else {
    expert = 0;
    row0 = (int64_t)b * BM;
    rows = (int)min((int64_t)BM, a.dense_rows - row0);
    if (rows <= 0) return;
  }
  // the wave index is uniform: keeping it in a scalar register keeps the copy destinations (M0) and the choice
  // of weight descriptor scalar as well
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;
  // column origin of this tile: weight columns for B, output columns for C (SwiGLU: gate and up halves)
  const int64_t n0 = (int64_t)nt * (EPI == EPI_SWIGLU_FWD ? BN / 2 : BN);
  const bool xe = expert == a.x_expert;
  // K, pitches and expert stride in 2-byte units (FP8: pairs of values)
  const int64_t lda64 = a.lda / UE, ldb64 = a.ldb / UE, bes = a.b_estride / UE;
  const bf16_t* Bbase = xe ? a.Bx : a.B + (int64_t)expert * bes;
  const bf16_t* B2base = xe ? (a.B2x ? a.B2x : Bbase) : (a.B2 ? a.B2 + (int64_t)expert * bes : Bbase);
  const int K = (int)(a.K / UE), N = (int)a.N, lda = (int)lda64, ldb = (int)ldb64, ksplit = (int)(a.k_split / UE);
  const int nk = (K + BK - 1) / BK;
  const uint32_t lds0 = lds_addr(smem);

  // descriptors: this tile's rows of A; the expert's B (and B2) matrix
  const u32x4 rsA = a.a_rows ? make_rsrc(a.A, a.a_nrows * lda64 * 2) : make_rsrc(a.A + row0 * lda64, (int64_t)rows * lda64 * 2);
  const int64_t b_bytes = (int64_t)(BMODE == B_NK ? N : K) * ldb64 * 2;
  const u32x4 rsB = make_rsrc(Bbase, b_bytes);
  const u32x4 rsB2 = make_rsrc(B2base, b_bytes);

  // ---- per-lane copy geometry, fixed over k: byte offset of this lane's chunk at k = 0 and the k of the chunk
  // within a stage (KBIG when its row or column is outside the operand, so the k test alone rejects it).
  // K-major: copy q covers rows RPC q .. RPC q + RPC - 1; lane -> row RPC q + lane / CPR, slot lane % CPR.
  uint32_t a_off[CPA];
  int a_k[CPA];
#pragma unroll
  for (int c = 0; c < CPA; ++c) {
    const int r = RPC * (CPA * wave + c) + lane / CPR;
    const int kc = (lane % CPR) ^ km_swz<BK>(r);
    if (a.a_rows) {  // gathered rows: the source row of tile row r (padding rows and rows past the tile: zeros)
      const int flat = r < rows ? a.a_rows[row0 + r] : -1;
      const int src = flat >= 0 ? div_by(flat, div_magic(a.a_div)) : -1;
      a_off[c] = (uint32_t)(max(src, 0) * lda + 8 * kc) * 2u;
      a_k[c] = src >= 0 ? 8 * kc : KBIG;
    } else {
      a_off[c] = (uint32_t)(r * lda + 8 * kc) * 2u;
      a_k[c] = r < rows ? 8 * kc : KBIG;
    }
  }
  // B K-major: as A over n (SwiGLU forward: tile columns [0, BN/2) gate rows, [BN/2, BN) up rows, same output
  // columns).  B N-major: copy q fills k rows 4 (q % CPS) + lane / 16 of sub-tile q / CPS, slot lane % 16
  // (SwiGLU forward: sub-tiles [0, NSUB/2) gate, [NSUB/2, NSUB) up).
  uint32_t b_off[CPB];
  int b_k[CPB];
#pragma unroll
  for (int c = 0; c < CPB; ++c) {
    const int q = CPB * wave + c;
    if (BMODE == B_NK) {
      const int n = RPC * q + lane / CPR;
      const int kc = (lane % CPR) ^ km_swz<BK>(n);
      const int64_t gn = n0 + (EPI == EPI_SWIGLU_FWD ? n % (BN / 2) : n);
      b_off[c] = (uint32_t)(gn * ldb + 8 * kc) * 2u;
      b_k[c] = gn < N ? 8 * kc : KBIG;
    } else {
      const int sub = q / CPS;
      const int k = 4 * (q % CPS) + (lane >> 4);
      const int ch = (lane & 15) ^ ((k & 3) << 2);
      const int64_t gn = EPI == EPI_SWIGLU_FWD ? n0 + NS * (sub % (NSUB / 2)) + 8 * ch : n0 + NS * sub + 8 * ch;
      b_off[c] = (uint32_t)(k * ldb + gn) * 2u;
      b_k[c] = gn < N ? k : KBIG;
    }
  }

  auto issue = [&](int slot, int kt) {
    const int k0 = kt * BK;
    const uint32_t at = lds0 + slot * A_SLOT, bt = lds0 + B_RING + slot * B_SLOT;
#pragma unroll
    for (int c = 0; c < CPA; ++c)
      copy16(rsA, k0 + a_k[c] < K ? a_off[c] + 2u * k0 : OOB, at + 1024 * (CPA * wave + c));
    if (BMODE == B_NK) {
      const bool second = ksplit && k0 >= ksplit;  // k range of B2 (gate/up dgrad); uniform
      const int kb = second ? k0 - ksplit : k0;
#pragma unroll
      for (int c = 0; c < CPB; ++c) {
        // SwiGLU forward: the copy's rows are all gate or all up (RPC divides BN / 2); wave-uniform
        const u32x4 rs = EPI == EPI_SWIGLU_FWD ? (RPC * (CPB * wave + c) >= BN / 2 ? rsB2 : rsB) : (second ? rsB2 : rsB);
        copy16(rs, k0 + b_k[c] < K ? b_off[c] + 2u * kb : OOB, bt + 1024 * (CPB * wave + c));
      }
    } else {
      const uint32_t kstep = 2u * (uint32_t)k0 * (uint32_t)ldb;
#pragma unroll
      for (int c = 0; c < CPB; ++c) {
        const int q = CPB * wave + c, sub = q / CPS;  // wave-uniform
        const u32x4 rs = (EPI == EPI_SWIGLU_FWD && sub >= NSUB / 2) ? rsB2 : rsB;
        copy16(rs, k0 + b_k[c] < K ? b_off[c] + kstep : OOB,
               bt + sub * (BK * NS * 2) + 1024 * (q % CPS));
      }
    }
  };

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x16{};

  // tile column of this wave's weight fragment j (SwiGLU: the first FN/2 gate, the rest up, same outputs)
  auto bcol = [&](int j) {
    if (EPI == EPI_SWIGLU_FWD)
      return (j < FN / 2 ? 0 : BN / 2) + wn * (TN / 2) + 32 * (j < FN / 2 ? j : j - FN / 2);
    return wn * TN + 32 * j;
  };
  typedef FragSet<FM, FN, typename std::conditional<F8 != 0, i32x8, bf16x8>::type> F;
  constexpr int KS = F8 ? 1 : BK / 16;
  auto load = [&](int slot, int s, F& f) {
    const bf16_t* at = smem + slot * Cfg::A_EL;
    const bf16_t* bt = smem + ST * Cfg::A_EL + slot * Cfg::B_EL;
    if constexpr (F8) {
#pragma unroll
      for (int i = 0; i < FM; ++i) f.x[i] = frag_k8(at, wm * TM + 32 * i + (lane & 31), lane >> 5);
#pragma unroll
      for (int j = 0; j < FN; ++j) f.w[j] = frag_k8(bt, bcol(j) + (lane & 31), lane >> 5);
    } else {
      const int kk = 16 * s;
#pragma unroll
      for (int i = 0; i < FM; ++i) f.x[i] = frag_k<BK>(at, wm * TM + 32 * i + (lane & 31), kk / 8 + (lane >> 5));
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int col = bcol(j);
        if (BMODE == B_NK) f.w[j] = frag_k<BK>(bt, col + (lane & 31), kk / 8 + (lane >> 5));
        else f.w[j] = frag_n(bt + (col / NS) * (BK * NS), kk, col % NS, lane);
      }
    }
  };
  // FP8 k split: stage index where B2 starts (-1: none) and the factor that carries the B part over to B2's scale
  [[maybe_unused]] int kstage = 0;
  [[maybe_unused]] const int ks_stage = (F8 && ksplit) ? ksplit / BK : -1;
  [[maybe_unused]] float ks_ratio = 1.f;
  if constexpr (F8 != 0 && EPI != EPI_SWIGLU_FWD)
    if (ksplit) ks_ratio = a.b_sinv[expert] / a.b2_sinv[expert];
  auto mma = [&](const F& f) {
    if constexpr (F8 != 0 && EPI != EPI_SWIGLU_FWD) {
      if (kstage++ == ks_stage) {  // wave-uniform; once per tile
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j) acc[i][j] *= ks_ratio;
      }
    }
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        if constexpr (F8 != 0) acc[i][j] = mfma32_f8<0, F8 == 2 ? 1 : 0>(f.w[j], f.x[i], acc[i][j]);
        else acc[i][j] = mfma32<ET>(f.w[j], f.x[i], acc[i][j]);
      }
  };
  // a wave whose rows or output columns all lie outside the tile (a one-block tile of a 256-row table, the N tail)
  // runs the loop for its copies and barriers only, without fragment reads or MFMAs; its accumulators stay zero and
  // are never stored.  One branch per wave, so the live loop is the plain one.
  if (wm * TM < rows && n0 + wn * (EPI == EPI_SWIGLU_FWD ? TN / 2 : TN) < N)
    run_k_loop<Cfg, F, KS, F8 != 0>(nk, wave, issue, load, mma);
  else
    run_k_loop<Cfg, F, KS, F8 != 0>(nk, wave, issue, [](int, int, F&) {}, [](const F&) {});
  if constexpr (F8 != 0) {  // dequantise: gate (or plain) columns by a_sinv * b_sinv[e], up columns by a_sinv * b2_sinv[e]
    // (k split: everything by a_sinv * b2_sinv[e], the B part having been carried over at the switch)
    const float sa = a.a_sinv[0];
    const float s1 = sa * ((EPI != EPI_SWIGLU_FWD && ksplit) ? a.b2_sinv[expert] : a.b_sinv[expert]);
    const float s2 = a.b2_sinv ? sa * a.b2_sinv[expert] : s1;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] *= (EPI == EPI_SWIGLU_FWD && j >= FN / 2) ? s2 : s1;
  }

  // ---- epilogue, staged through LDS.  Written straight out, one store instruction would cover 16 bytes of 32
  // different rows.  Instead each wave parks one 32-row slice of its accumulators in the (now idle) ring as f32
  // rows, then reads them back row-contiguous: TN / 8 lanes x 8 columns cover a row, so every global load and
  // store spans whole lines.
  __syncthreads();  // all waves are done with the ring
  float* const stg = reinterpret_cast<float*>(smem) + wave * (32 * SP);
  constexpr int LPR = TN / 8, RPP = 64 / LPR, PASSES = 32 / RPP;          // store mapping
  constexpr int LPR2 = TN / 16, RPP2 = 64 / LPR2, PASSES2 = 32 / RPP2;    // SwiGLU forward: TN / 2 outputs
  [[maybe_unused]] float hmax = 0.f;  // with a.amax: max |h| (|dG|, |dU| in the FP8 backward) over this lane's outputs
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int mbase = wm * TM + 32 * i;  // first tile row of this slice
    // SwiGLU backward: fetch the saved g, u of this slice before parking the accumulators, so the loads'
    // latency overlaps the LDS round trip.
    u32x4 gq[PASSES], uq[PASSES];
    float wsc[PASSES];  // routing weights of the rows (row_scale; 1 without, and in tiles of the extra expert)
    if (EPI == EPI_SWIGLU_BWD) {
      const bool scl = !F8 && a.row_scale && expert != a.x_expert;
#pragma unroll
      for (int it = 0; it < PASSES; ++it) {
        const int r = RPP * it + lane / LPR;
        const int64_t col = n0 + wn * TN + 8 * (lane % LPR);
        const bool ok = mbase + r < rows && col < N;
        const int64_t off = ok ? (row0 + mbase + r) * a.ldg + col : row0 * a.ldg;
        gq[it] = *reinterpret_cast<const u32x4*>(a.G + off);
        uq[it] = *reinterpret_cast<const u32x4*>(a.U + off);
        wsc[it] = scl && mbase + r < rows ? a.row_scale[row0 + mbase + r] : 1.f;
      }
    }
    if (i > 0) __builtin_amdgcn_wave_barrier();
    park<Cfg>(stg, acc, i, lane);
    if (EPI == EPI_SWIGLU_FWD) {
#pragma unroll
      for (int it = 0; it < PASSES2; ++it) {
        const int r = RPP2 * it + lane / LPR2, c = 8 * (lane % LPR2);
        const int64_t col = n0 + wn * (TN / 2) + c;
        if (mbase + r >= rows || col >= N) continue;
        const float* src = stg + r * SP + c;
        const f32x4 g0 = *reinterpret_cast<const f32x4*>(src), g1 = *reinterpret_cast<const f32x4*>(src + 4);
        const f32x4 u0 = *reinterpret_cast<const f32x4*>(src + TN / 2);
        const f32x4 u1 = *reinterpret_cast<const f32x4*>(src + TN / 2 + 4);
        const float g[8] = {g0[0], g0[1], g0[2], g0[3], g1[0], g1[1], g1[2], g1[3]};
        const float u[8] = {u0[0], u0[1], u0[2], u0[3], u1[0], u1[1], u1[2], u1[3]};
        float h[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          h[t] = silu_f(g[t]) * u[t];
          hmax = fmaxf(hmax, fabsf(h[t]));
        }
        const int64_t gr = row0 + mbase + r;
        st_bf16x8(a.C + gr * a.ldc + col, h);
        if (a.G) st_bf16x8(a.G + gr * a.ldg + col, g);
        if (a.U) st_bf16x8(a.U + gr * a.ldg + col, u);
      }
    } else {
#pragma unroll
      for (int it = 0; it < PASSES; ++it) {
        const int r = RPP * it + lane / LPR, c = 8 * (lane % LPR);
        const int64_t col = n0 + wn * TN + c;
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
            st_x8<ET>(a.C + gr * a.ldc + col, v);
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
            const float dh = v[t] * wsc[it];
            dg[t] = dh * u * sg * (1.f + g * (1.f - sg));
            du[t] = dh * g * sg;
            if constexpr (F8 != 0) hmax = fmaxf(hmax, fmaxf(fabsf(dg[t]), fabsf(du[t])));
          }
          st_bf16x8(a.C + gr * a.ldc + col, dg);
          st_bf16x8(a.C + gr * a.ldc + N + col, du);
        }
      }
    }
  }
  if ((EPI == EPI_SWIGLU_FWD || (F8 != 0 && EPI == EPI_SWIGLU_BWD)) && a.amax) {
    // max |bf16(h)| = bf16(max |h|) (rounding is monotonic); non-negative floats order like their bit patterns,
    // so an unsigned max over the bits is the float max, whatever order the waves arrive in
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) hmax = fmaxf(hmax, __shfl_xor(hmax, o, 64));
    if (lane == 0) atomicMax(a.amax, (uint32_t)f32_to_bf16(hmax) << 16);
  }
}

// Weight-gradient epilogue (f32), staged through LDS as in gemm_rows_kernel: acc[i][j][4q + t] is C row
// i0 + wm*TM + 32 i + lane%32, column n0 + wn*TN + 32 j + 8 q + 4 (lane/32) + t.  Read back with TN/8 lanes per row,
// each lane storing 8 contiguous f32, to the chunk's partial slot, the split partials, or the gradient itself.
template <class Cfg>
__device__ __forceinline__ void wgrad_epilogue(const WgradArgs& a, const f32x16 (&acc)[Cfg::FM][Cfg::FN],
                                               bf16_t* smem, int wave, int lane, int64_t i0, int64_t n0,
                                               float* part_out, int S, int s, int e) {
  constexpr int TM = Cfg::TM, TN = Cfg::TN, FM = Cfg::FM, SP = Cfg::SP;
  const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;
  const int64_t I = a.I, N = a.N;
  __syncthreads();  // all waves are done with the ring
  float* const stg = reinterpret_cast<float*>(smem) + wave * (32 * SP);
  constexpr int LPR = TN / 8, RPP = 64 / LPR, PASSES = 32 / RPP;
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    if (i > 0) __builtin_amdgcn_wave_barrier();
    park<Cfg>(stg, acc, i, lane);
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const int r = RPP * p + lane / LPR, c = 8 * (lane % LPR);
      const int64_t row = i0 + wm * TM + 32 * i + r;
      if (row >= I) continue;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int64_t col = n0 + wn * TN + c + 4 * h;
        if (col >= N) continue;
        const f32x4 v = *reinterpret_cast<const f32x4*>(stg + r * SP + c + 4 * h);
        float* dst;
        if (part_out) dst = part_out + row * N + col;
        else if (S > 1) dst = a.part + (((int64_t)s * a.E + e) * I + row) * N + col;
        else if (e == a.x_expert) dst = (a.C2x && col >= a.n_split) ? a.C2x + row * a.ldc + (col - a.n_split)
                                                                    : a.Cx + row * a.ldc + col;
        else if (a.C2 && col >= a.n_split) dst = a.C2 + (int64_t)e * a.c_estride + row * a.ldc + (col - a.n_split);
        else dst = a.C + (int64_t)e * a.c_estride + row * a.ldc + col;
        *reinterpret_cast<f32x4*>(dst) = v;
      }
    }
  }
}

// =====================================================================================================
// Weight gradient C_e[I, N] = A_e^T B_e, reduced over the rows of expert e: both operands are row-major
// [rows, .] (the reduction dim is the slow one), so both are staged N-major and read with the transpose read.
template <class Cfg, int ET = LSURGE_BF16>
__global__ __launch_bounds__(Cfg::GT) __attribute__((amdgpu_waves_per_eu(Cfg::NW * Cfg::OCC / 4)))
void gemm_wgrad_kernel(WgradArgs a) {
  constexpr int BM = Cfg::BM, BN = Cfg::BN, BK = Cfg::BK, ST = Cfg::ST;
  constexpr int TM = Cfg::TM, TN = Cfg::TN, FM = Cfg::FM, FN = Cfg::FN;
  constexpr int CPA = Cfg::CPA, CPB = Cfg::CPB, CPS = BK / 4;
  // ring: A BM/128 N-major sub-tiles (BK rows x 128 columns), B BN/128 sub-tiles; after the K loop the same
  // memory stages the epilogue
  __shared__ __attribute__((aligned(1024))) bf16_t smem[Cfg::SMEM_EL];
  constexpr uint32_t A_SLOT = Cfg::A_EL * 2, B_SLOT = Cfg::B_EL * 2, B_RING = ST * A_SLOT;  // bytes
  const int64_t total = (int64_t)gridDim.x;
  const int64_t tiles_per_e = (int64_t)(a.c_expert ? 1 : a.S) * a.i_tiles * a.n_tiles;
  // Tile order.  Expert slices: XCD-aware contiguous ranges (xcd_logical).  Chunk table: chunk_logical.
  int64_t logical;
  if (a.c_expert) {
    logical = chunk_logical(tiles_per_e, min(a.num_chunks[0], a.max_chunks));
    if (logical < 0) return;
  } else {
    logical = xcd_logical(blockIdx.x, total);
  }
  const int g = (int)(logical / tiles_per_e);  // expert, or chunk with a chunk table
  int64_t rem = logical % tiles_per_e;
  const int s = (int)(rem / ((int64_t)a.i_tiles * a.n_tiles));
  rem %= (int64_t)a.i_tiles * a.n_tiles;
  const int it = (int)(rem / a.n_tiles), nt = (int)(rem % a.n_tiles);
  int e, S = a.S;
  int64_t r0, nrows;
  float* part_out = nullptr;  // chunk partial slot ([I][N] f32), when the chunk writes one
  if (a.c_expert) {
    if (g >= a.max_chunks || g >= a.num_chunks[0]) return;
    e = a.c_expert[g];
    r0 = a.c_row0[g];
    nrows = a.c_rows[g];
    S = 1;
    const int ps = a.c_part[g];
    if (ps >= 0) part_out = a.part + (int64_t)ps * a.I * a.N;
  } else {
    e = g;
    if (e >= a.E) return;
    if (a.e_rows) {
      r0 = (int64_t)a.e_row0[e] * a.row0_mult;
      nrows = a.e_rows[e];
    } else {
      r0 = 0;
      nrows = a.dense_rows;
    }
  }
  // rows of split s
  const int64_t chunk = ((nrows + S - 1) / S + BK - 1) / BK * BK;
  const int64_t rs = (int64_t)s * chunk;
  const int64_t re = min(nrows, rs + chunk);
  const int64_t i0 = (int64_t)it * BM, n0 = (int64_t)nt * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;
  const int64_t I = a.I, N = a.N;
  const int lda = (int)a.lda, ldb = (int)a.ldb;
  const uint32_t lds0 = lds_addr(smem);

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x16{};

  const int nk = re > rs ? (int)((re - rs + BK - 1) / BK) : 0;
  // descriptors over rows [rs, re) of this expert (empty when the split has no rows); a gathered A spans the
  // whole source matrix and its row indices come through an LDS window (below)
  const int span = re > rs ? (int)(re - rs) : 0;
  const bool gath = a.a_rows != nullptr;
  const u32x4 rsA = gath ? make_rsrc(a.A, a.a_nrows * a.lda * 2) : make_rsrc(a.A + (r0 + rs) * a.lda, (int64_t)span * a.lda * 2);
  const u32x4 rsB = make_rsrc(a.B + (r0 + rs) * a.ldb, (int64_t)span * a.ldb * 2);
  // Gathered A: the row indices of the span pass through a double-buffered LDS window of 2 x 256 entries.  Wave 0
  // copies window m (rows [256 m, 256 m + 256)) into buffer m % 2 when the first stage of window m - 1 is
  // issued, i.e. SPW stages before its first use and after every wave is done with the buffer's previous
  // window; the stage waits and barriers of the K loop then cover its completion like any other copy.
  constexpr int SPW = 256 / BK;  // stages per window
  __shared__ __attribute__((aligned(1024))) int32_t idxwin[512];
  const uint32_t win0 = lds_addr(reinterpret_cast<const bf16_t*>(idxwin));
  const u32x4 rsI = make_rsrc(gath ? a.a_rows + r0 + rs : nullptr, gath ? (int64_t)span * 4 : 0);
  const uint64_t magic = div_magic(gath ? a.a_div : 1);
  int nidx[Cfg::CPA];  // gathered A: row indices of the next stage to issue (this lane's rows)
  if (gath) {
    if (wave == 0) {
      copy16(rsI, 16u * lane, win0);
      copy16(rsI, 1024u + 16u * lane, win0 + 1024);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  // copy q of an operand fills k rows 4 (q % CPS) + lane / 16 of sub-tile q / CPS, slot lane % 16: byte offset of
  // this lane's chunk at row 0 of the span and its row in a stage (KBIG when its column is outside the operand)
  uint32_t a_off[CPA], b_off[CPB];
  int a_k[CPA], b_k[CPB];
#pragma unroll
  for (int c = 0; c < CPA; ++c) {
    const int q = CPA * wave + c, sub = q / CPS;
    const int k = 4 * (q % CPS) + (lane >> 4);
    const int64_t ic = i0 + NS * sub + 8 * ((lane & 15) ^ ((k & 3) << 2));
    a_off[c] = gath ? (uint32_t)ic * 2u : (uint32_t)(k * lda + ic) * 2u;  // gathered: the row part comes later
    a_k[c] = ic < I ? k : KBIG;
  }
#pragma unroll
  for (int c = 0; c < CPB; ++c) {
    const int q = CPB * wave + c, sub = q / CPS;
    const int k = 4 * (q % CPS) + (lane >> 4);
    const int64_t nc = n0 + NS * sub + 8 * ((lane & 15) ^ ((k & 3) << 2));
    b_off[c] = (uint32_t)(k * ldb + nc) * 2u;
    b_k[c] = nc < N ? k : KBIG;
  }
#pragma unroll
  for (int c = 0; c < CPA; ++c) nidx[c] = gath ? idxwin[a_k[c] & 511] : 0;  // stage 0
  auto issue = [&](int slot, int kt) {
    const int rb = kt * BK;
    const uint32_t at = lds0 + slot * A_SLOT, bt = lds0 + B_RING + slot * B_SLOT;
    const uint32_t astep = 2u * (uint32_t)rb * (uint32_t)lda, bstep = 2u * (uint32_t)rb * (uint32_t)ldb;
    if (gath) {
      // the window holding stage kt's rows is resident; refill the other buffer with the window after it
      if (kt % SPW == 0 && kt >= SPW && wave == 0) {
        const int m = kt / SPW + 1;
        copy16(rsI, 1024u * m + 16u * lane, win0 + 1024u * (m & 1));
      }
#pragma unroll
      for (int c = 0; c < CPA; ++c) {
        const int q = CPA * wave + c;
        const int rr = rb + a_k[c];
        const int idx = nidx[c];  // read one stage earlier
        const bool ok = rr < span && idx >= 0;
        copy16(rsA, ok ? (uint32_t)div_by(idx, magic) * (2u * (uint32_t)lda) + a_off[c] : OOB,
               at + (q / CPS) * (BK * NS * 2) + 1024 * (q % CPS));
      }
      // indices of the next stage: its window is resident (copied at least SPW - 1 stages ago, and this step's
      // barrier has passed), so the LDS reads overlap this stage instead of stalling the next copy issue
#pragma unroll
      for (int c = 0; c < CPA; ++c) nidx[c] = idxwin[(rb + BK + a_k[c]) & 511];
    } else {
#pragma unroll
      for (int c = 0; c < CPA; ++c) {
        const int q = CPA * wave + c;
        copy16(rsA, rb + a_k[c] < span ? a_off[c] + astep : OOB,
               at + (q / CPS) * (BK * NS * 2) + 1024 * (q % CPS));
      }
    }
#pragma unroll
    for (int c = 0; c < CPB; ++c) {
      const int q = CPB * wave + c;
      copy16(rsB, rb + b_k[c] < span ? b_off[c] + bstep : OOB,
             bt + (q / CPS) * (BK * NS * 2) + 1024 * (q % CPS));
    }
  };
  typedef FragSet<FM, FN> F;
  auto load = [&](int slot, int st, F& f) {
    const bf16_t* at = smem + slot * Cfg::A_EL;
    const bf16_t* bt = smem + ST * Cfg::A_EL + slot * Cfg::B_EL;
    const int kk = 16 * st;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int col = wm * TM + 32 * i;
      f.x[i] = frag_n(at + (col / NS) * (BK * NS), kk, col % NS, lane);
    }
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int col = wn * TN + 32 * j;
      f.w[j] = frag_n(bt + (col / NS) * (BK * NS), kk, col % NS, lane);
    }
  };
  auto mma = [&](const F& f) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = mfma32<ET>(f.w[j], f.x[i], acc[i][j]);
  };
  if (nk > 0) {  // waves outside the tile: copies and barriers only, as in gemm_rows_kernel
    if (i0 + wm * TM < I && n0 + wn * TN < N) run_k_loop<Cfg, F>(nk, wave, issue, load, mma);
    else run_k_loop<Cfg, F>(nk, wave, issue, [](int, int, F&) {}, [](const F&) {});
  }

  wgrad_epilogue<Cfg>(a, acc, smem, wave, lane, i0, n0, part_out, S, s, e);
}

// =====================================================================================================
// FP8 weight gradient C_e[I, N] = (A_e^T B_e) a_sinv b_sinv over the rows of expert e, from the row-major FP8
// tensors themselves (activations A in format FA: E4M3 x or h; gradients B in FB: E5M2 dY or [dG | dU]; one byte per
// value, pitches in bytes).  As in gemm_wgrad_kernel both operands are staged N-major -- a stage is SK = 64 rows of
// the reduction by 128-column sub-tiles -- and the MFMA fragments come out of LDS already K-contiguous through the
// gfx950 8-bit transpose read, so no transposed copy of any operand is ever written.  Chunk table, row gather of A
// (the token rows of x through row_src), split partials and output routing are those of gemm_wgrad_kernel.
//
// LDS sub-tile: 64 rows x 128 bytes; 16-byte chunk c of row k sits at slot c ^ (2 ((k >> 1) & 3)).  A copy fills 8
// rows (lane p: row p / 8, slot p % 8).  A fragment read (below) takes, per 32-lane half of the wave, 8 rows x 2
// adjacent chunks; the 4 even rows' chunks land on distinct slots of banks 0-31 and the odd rows' on 32-63, so the
// 256 bytes of each pass hit all 64 banks once.
constexpr int SK8 = 64;  // reduction rows per FP8 stage (one 32x32x64 MFMA step)
__device__ __forceinline__ int nm8_off(int k, int n) {
  return k * NS + ((((n >> 4) ^ (((k >> 1) & 3) << 1))) << 4) + (n & 15);
}
// ds_read_b64_tr_b8 in a 16-lane group: source lane s points at 8 bytes (row kb + s / 2, columns nb + 8 (s % 2) ..
// + 7 of an N-major tile); lane i receives column nb + i, rows kb .. kb + 7, row j in byte j.  Fragment for the
// 32x32x64 operand layout: lane l (column nbase + l % 32, half h = l / 32) gets rows 32 h .. 32 h + 31 of its column,
// byte b = row 32 h + b, in four reads.
typedef int i32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ i32x8 frag_n8(const uint8_t* sub, int nbase, int lane) {
  const int g = lane >> 4, s = lane & 15, h = lane >> 5;
  const int n = nbase + 16 * (g & 1) + 8 * (s & 1);
  i32x8 f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int k = 32 * h + 8 * q + (s >> 1);
    const i32x2 v = __builtin_amdgcn_ds_read_tr8_b64_v2i32(LDS_PTR(i32x2, sub + nm8_off(k, n)));
    f[2 * q] = v[0];
    f[2 * q + 1] = v[1];
  }
  return f;
}

template <class Cfg, int FA, int FB>
__global__ __launch_bounds__(Cfg::GT) __attribute__((amdgpu_waves_per_eu(Cfg::NW * Cfg::OCC / 4)))
void gemm_wgrad_f8_kernel(WgradArgs a) {
  static_assert(Cfg::BK == 32 && !Cfg::PP, "FP8 weight gradient: 64-row stages, 4-wave single-buffered loop");
  constexpr int BM = Cfg::BM, BN = Cfg::BN, ST = Cfg::ST;
  constexpr int TM = Cfg::TM, TN = Cfg::TN, FM = Cfg::FM, FN = Cfg::FN;
  constexpr int CPA = Cfg::CPA, CPB = Cfg::CPB;
  constexpr int SUB = SK8 * NS;      // bytes per sub-tile (8 KiB)
  constexpr int CPS = SUB / 1024;    // copies per sub-tile
  static_assert(CPA * Cfg::NW * 1024 == (BM / NS) * SUB && CPB * Cfg::NW * 1024 == (BN / NS) * SUB, "stage bytes");
  __shared__ __attribute__((aligned(1024))) bf16_t smem[Cfg::SMEM_EL];
  constexpr uint32_t A_SLOT = Cfg::A_EL * 2, B_SLOT = Cfg::B_EL * 2, B_RING = ST * A_SLOT;  // bytes
  const int64_t tiles_per_e = (int64_t)(a.c_expert ? 1 : a.S) * a.i_tiles * a.n_tiles;
  int64_t logical;
  if (a.c_expert) {
    logical = chunk_logical(tiles_per_e, min(a.num_chunks[0], a.max_chunks));
    if (logical < 0) return;
  } else {
    logical = xcd_logical(blockIdx.x, (int64_t)gridDim.x);
  }
  const int g = (int)(logical / tiles_per_e);
  int64_t rem = logical % tiles_per_e;
  const int s = (int)(rem / ((int64_t)a.i_tiles * a.n_tiles));
  rem %= (int64_t)a.i_tiles * a.n_tiles;
  const int it = (int)(rem / a.n_tiles), nt = (int)(rem % a.n_tiles);
  int e, S = a.S;
  int64_t r0, nrows;
  float* part_out = nullptr;
  if (a.c_expert) {
    if (g >= a.max_chunks || g >= a.num_chunks[0]) return;
    e = a.c_expert[g];
    r0 = a.c_row0[g];
    nrows = a.c_rows[g];
    S = 1;
    const int ps = a.c_part[g];
    if (ps >= 0) part_out = a.part + (int64_t)ps * a.I * a.N;
  } else {
    e = g;
    if (e >= a.E) return;
    r0 = 0;
    nrows = a.dense_rows;
  }
  const int64_t chunk = ((nrows + S - 1) / S + SK8 - 1) / SK8 * SK8;
  const int64_t rs = (int64_t)s * chunk, re = min(nrows, rs + chunk);
  const int span = re > rs ? (int)(re - rs) : 0;
  const int nk = (span + SK8 - 1) / SK8;
  const int64_t i0 = (int64_t)it * BM, n0 = (int64_t)nt * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;
  const uint32_t lds0 = lds_addr(smem);
  const uint8_t* A8 = reinterpret_cast<const uint8_t*>(a.A);
  const uint8_t* B8 = reinterpret_cast<const uint8_t*>(a.B);
  const bool gath = a.a_rows != nullptr;
  const u32x4 rsA = gath ? make_rsrc(A8, a.a_nrows * a.lda) : make_rsrc(A8 + (r0 + rs) * a.lda, (int64_t)span * a.lda);
  const u32x4 rsB = make_rsrc(B8 + (r0 + rs) * a.ldb, (int64_t)span * a.ldb);
  // gathered A: the row indices pass through a double-buffered LDS window of 2 x 256 entries, as in
  // gemm_wgrad_kernel (SPW stages per window)
  constexpr int SPW = 256 / SK8;
  __shared__ __attribute__((aligned(1024))) int32_t idxwin[512];
  const uint32_t win0 = lds_addr(reinterpret_cast<const bf16_t*>(idxwin));
  const u32x4 rsI = make_rsrc(gath ? a.a_rows + r0 + rs : nullptr, gath ? (int64_t)span * 4 : 0);
  const uint64_t magic = div_magic(gath ? a.a_div : 1);
  int nidx[CPA];
  if (gath) {
    if (wave == 0) {
      copy16(rsI, 16u * lane, win0);
      copy16(rsI, 1024u + 16u * lane, win0 + 1024);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  // copy q of an operand fills rows 8 (q % CPS) + lane / 8 of sub-tile q / CPS, slot lane % 8: byte offset of this
  // lane's chunk at row 0 of the span and its row in a stage (KBIG when its columns are outside the operand)
  uint32_t a_off[CPA], b_off[CPB];
  int a_k[CPA], b_k[CPB];
#pragma unroll
  for (int c = 0; c < CPA; ++c) {
    const int q = CPA * wave + c, sub = q / CPS;
    const int k = 8 * (q % CPS) + (lane >> 3);
    const int64_t ic = i0 + NS * sub + 16 * ((lane & 7) ^ (((k >> 1) & 3) << 1));
    a_off[c] = gath ? (uint32_t)ic : (uint32_t)(k * a.lda + ic);  // gathered: the row part comes later
    a_k[c] = ic < a.I ? k : KBIG;
  }
#pragma unroll
  for (int c = 0; c < CPB; ++c) {
    const int q = CPB * wave + c, sub = q / CPS;
    const int k = 8 * (q % CPS) + (lane >> 3);
    const int64_t nc = n0 + NS * sub + 16 * ((lane & 7) ^ (((k >> 1) & 3) << 1));
    b_off[c] = (uint32_t)(k * a.ldb + nc);
    b_k[c] = nc < a.N ? k : KBIG;
  }
#pragma unroll
  for (int c = 0; c < CPA; ++c) nidx[c] = gath ? idxwin[a_k[c] & 511] : 0;  // stage 0
  const uint32_t lda = (uint32_t)a.lda, ldb = (uint32_t)a.ldb;
  auto issue = [&](int slot, int kt) {
    const int rb = kt * SK8;
    const uint32_t at = lds0 + slot * A_SLOT, bt = lds0 + B_RING + slot * B_SLOT;
    if (gath) {
      if (kt % SPW == 0 && kt >= SPW && wave == 0) {
        const int m = kt / SPW + 1;
        copy16(rsI, 1024u * m + 16u * lane, win0 + 1024u * (m & 1));
      }
#pragma unroll
      for (int c = 0; c < CPA; ++c) {
        const int q = CPA * wave + c;
        const int idx = nidx[c];
        const bool ok = rb + a_k[c] < span && idx >= 0;
        copy16(rsA, ok ? (uint32_t)div_by(idx, magic) * lda + a_off[c] : OOB, at + (q / CPS) * SUB + 1024 * (q % CPS));
      }
#pragma unroll
      for (int c = 0; c < CPA; ++c) nidx[c] = idxwin[(rb + SK8 + a_k[c]) & 511];
    } else {
#pragma unroll
      for (int c = 0; c < CPA; ++c) {
        const int q = CPA * wave + c;
        copy16(rsA, rb + a_k[c] < span ? a_off[c] + (uint32_t)rb * lda : OOB,
               at + (q / CPS) * SUB + 1024 * (q % CPS));
      }
    }
#pragma unroll
    for (int c = 0; c < CPB; ++c) {
      const int q = CPB * wave + c;
      copy16(rsB, rb + b_k[c] < span ? b_off[c] + (uint32_t)rb * ldb : OOB, bt + (q / CPS) * SUB + 1024 * (q % CPS));
    }
  };
  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x16{};
  typedef FragSet<FM, FN, i32x8> F;
  auto load = [&](int slot, int, F& f) {
    const uint8_t* at = reinterpret_cast<const uint8_t*>(smem) + slot * A_SLOT;
    const uint8_t* bt = reinterpret_cast<const uint8_t*>(smem) + B_RING + slot * B_SLOT;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int col = wm * TM + 32 * i;
      f.x[i] = frag_n8(at + (col / NS) * SUB, col % NS, lane);
    }
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int col = wn * TN + 32 * j;
      f.w[j] = frag_n8(bt + (col / NS) * SUB, col % NS, lane);
    }
  };
  auto mma = [&](const F& f) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[i][j] = mfma32_f8<FB, FA>(f.w[j], f.x[i], acc[i][j]);
  };
  if (nk > 0) {  // waves outside the tile: copies and barriers only
    if (i0 + wm * TM < a.I && n0 + wn * TN < a.N) run_k_loop<Cfg, F, 1, true>(nk, wave, issue, load, mma);
    else run_k_loop<Cfg, F, 1, true>(nk, wave, issue, [](int, int, F&) {}, [](const F&) {});
  }
  const float sab = a.a_sinv[0] * a.b_sinv[0];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] *= sab;
  wgrad_epilogue<Cfg>(a, acc, smem, wave, lane, i0, n0, part_out, S, s, e);
}

}  // namespace lsgemm
