// Persistent 256 x 256 grouped GEMM of the MoE layer on CDNA4 matrix cores (bf16 or f16 inputs, f32 accumulation,
// v_mfma_f32_32x32x16_bf16 / _f16).  One workgroup of 4 waves per CU; wave (wm, wn) owns a 128 x 128 block of the
// 256 x 256 output tile: 256 accumulator registers, the whole AccVGPR file of a wave that is alone on its SIMD.
//
// Replaces the padded batched einsum of modal/padded_gmm.py:66-69 (and its autodiff) for the layer's row GEMMs, like
// gemm_rows_kernel in gemm_kernels.h, whose operand layouts, tile tables and epilogues it keeps.  What differs is how
// a tile's K loop is fed:
//  - Global -> VGPR -> LDS.  K moves in 64-deep stages.  Every lane holds one stage of its copies in registers
//    (16 x 16 bytes) and writes it to the other half of an LDS double buffer (2 x 64 KiB) while the MFMAs run on the
//    current half; the registers are then refilled with the stage after.  One workgroup barrier per stage.  The
//    VGPR path moves about twice the bytes per clock of buffer_load ... lds on this chip, which is what the 4-wave
//    128 x 256 x 32 kernel's copy stream was limited by.
//  - Explicit issue order.  A stage is four 16-deep MFMA steps of 16 MFMAs each.  During a step the wave issues the
//    next step's 8 fragment reads, then a third of the stage's register -> LDS writes and global loads, each pinned
//    between two MFMAs with sched_group_barrier, so the matrix pipe never waits on a burst of memory instructions.
//    The last step starts with the stage barrier and reads the next stage's first fragments.
//  - Persistent tiles.  The grid is one workgroup per CU (256); workgroup l of XCD x walks the tiles
//    xbeg + l, xbeg + l + nper, ... of that XCD's contiguous share of the tiles (so neighbouring tiles of one expert
//    share an XCD's L2).  The load stream runs across tile boundaries: the next tile's first stages are loaded while
//    the current tile's last stages compute; its first two stages are in LDS and its third in registers before the
//    epilogue's stores are issued.
//  - Epilogue through a wave-private 8 KiB LDS area beside the ring (32 rows of the wave's block at a time), so every
//    global store (and the SwiGLU backward's loads of g and u) covers whole 128- or 256-byte row segments; the copy
//    ring is untouched, and the next tile's loads stay in flight.
//
// Every output element is the same ascending sequence of 16-deep MFMA steps as in gemm_rows_kernel, so the results
// are bitwise those of the other tile shapes.  Stages past K load zeros.
#pragma once
#include "gemm_kernels.h"

namespace lsgemm {
namespace g256 {

constexpr int BM = 256, BN = 256, BK = 64;
constexpr int OP_BYTES = 256 * BK * 2;        // one operand of one stage: 32 KiB
constexpr int STAGE_BYTES = 2 * OP_BYTES;     // A then B
constexpr int RING_BYTES = 2 * STAGE_BYTES;   // double buffer, 128 KiB
constexpr int STG_BYTES = 8192;               // per-wave epilogue staging
constexpr int SMEM_BYTES = RING_BYTES + 4 * STG_BYTES;  // 160 KiB: the whole LDS of a CU
constexpr int NWG = 256;                      // persistent grid: one workgroup per CU (a multiple of 8 XCDs)

typedef __amdgpu_buffer_rsrc_t rsrc_t;
// raw buffer over [p, p + bytes): loads past the end return zeros (every span is below 2^31 bytes, host-checked)
__device__ __forceinline__ rsrc_t rsrc(const void* p, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 ld16(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}
__device__ __forceinline__ float ldf(rsrc_t r, uint32_t off) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}

enum { SG_MFMA = 0x8, SG_VMEM_R = 0x20, SG_DS_R = 0x100, SG_DS_W = 0x200 };

// Row tile of the 256-row table, or of a dense matrix.  The table is read after the kernel's own stores, so the
// compiler cannot tell the values are uniform; readfirstlane keeps them (and the descriptors made from them) in
// scalar registers, where a divergent descriptor would wrap every buffer load in a waterfall loop.
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
// Entry i (uniform) of a tile or chunk table through the scalar unit.  The tables are written by earlier launches
// and only read here, so a constant-address-space load is valid; it lands in a scalar register and is counted by
// lgkmcnt.  A vector load would be counted by the in-order vector memory count instead, and the wait for it would
// drain every copy load issued before it.
typedef const __attribute__((address_space(4))) int32_t cint32_t;
__device__ __forceinline__ int ctab(const int32_t* p, int i) { return ((cint32_t*)p)[i]; }
struct Tile {
  int expert, rows;
  int64_t row0;
};
__device__ __forceinline__ Tile row_tile(const RowsArgs& a, int b) {
  Tile t;
  if (a.t_expert) {
    t.expert = ctab(a.t_expert, b);
    t.rows = ctab(a.t_rows, b);
    t.row0 = a.t_row0 ? (int64_t)ctab(a.t_row0, b) : (int64_t)b * BM;
  } else {
    t.expert = 0;
    t.row0 = (int64_t)b * BM;
    t.rows = (int)min((int64_t)BM, a.dense_rows - t.row0);
  }
  return t;
}

// One stage on LDS half `cur` (four 16-deep MFMA steps over fragment buffers f0 / f1).  Step s reads step s + 1's
// fragments (step 3: after the barrier that publishes the next stage, its step 0 from the other half) and, in steps
// 0..2, moves copies [16 s / 3, 16 (s + 1) / 3) of stage lk from registers to the other half, each followed by the
// load of the same chunk of the stage after.  The issue order is pinned: the NR fragment reads first, then the
// write / load pairs, spread evenly over the step's 16 MFMAs.
// COPY = false: no copies in this stage (the fragment reads and MFMAs only).
//   fread(F&, buf, step)   swrite(c, buf)   gload(c, lk)   mma(const F&)
template <int NR, bool COPY = true, class F, class Fread, class Swrite, class Gload, class Mma>
__device__ __forceinline__ void run_stage(F& f0, F& f1, int cur, int lk, Fread&& fread, Swrite&& swrite, Gload&& gload,
                                          Mma&& mma) {
  const int nxt = cur ^ 1;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    F& fc = (s & 1) ? f1 : f0;
    F& fn = (s & 1) ? f0 : f1;
    if (s == 3) {
      // every wave's copies of the next stage have landed, and nobody reads this half's predecessor any more
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      fread(fn, nxt, 0);
    } else {
      fread(fn, cur, s + 1);
    }
    const int lo = COPY && s < 3 ? 16 * s / 3 : 0, hi = COPY && s < 3 ? 16 * (s + 1) / 3 : 0;
#pragma unroll
    for (int c = lo; c < hi; ++c) {
      swrite(c, nxt);
      gload(c, lk);
    }
    mma(fc);
    const int nops = NR + 2 * (hi - lo);
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
      const int o0 = m * nops / 16, o1 = (m + 1) * nops / 16;
#pragma unroll
      for (int o = o0; o < o1; ++o) {
        if (o < NR) __builtin_amdgcn_sched_group_barrier(SG_DS_R, 1, 0);
        else if ((o - NR) % 2 == 0) __builtin_amdgcn_sched_group_barrier(SG_DS_W, 1, 0);
        else __builtin_amdgcn_sched_group_barrier(SG_VMEM_R, 1, 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Row GEMM C[tile rows, n tile] = A[tile rows, :] @ B[expert(tile)] over the row tiles of a.t_expert / t_rows /
// t_row0 (num_tiles[0] real ones) or of a dense matrix, n tiles of BN columns (SwiGLU forward: BN / 2 outputs, the
// gate and up columns side by side).  Operands, epilogues and arguments as gemm_rows_kernel (RowsArgs); amax is not
// supported here.  GATHER: A rows through a.a_rows; OUTF32: the plain store writes a.Cf.
template <int BMODE, int EPI, bool GATHER, int ET = LSURGE_BF16, bool OUTF32 = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void rows_kernel(RowsArgs a) {
  static_assert(ET == LSURGE_BF16 || EPI == EPI_STORE, "f16 operands: plain store epilogue only");
  __shared__ __attribute__((aligned(1024))) char smem[SMEM_BYTES];
  constexpr int NOUT = EPI == EPI_SWIGLU_FWD ? BN / 2 : BN;  // output columns of an n tile

  // ---- this workgroup's tiles: XCD x = blockIdx % 8 takes tiles [x T / 8, (x + 1) T / 8) of the T that exist
  const int ntr = a.t_expert ? min(ctab(a.num_tiles, 0), a.max_tiles) : (int)((a.dense_rows + BM - 1) / BM);
  const int total = ntr * a.n_tiles;
  const int xcd = blockIdx.x % 8, nper = gridDim.x / 8;
  const int xbeg = (int)((int64_t)xcd * total / 8), xend = (int)((int64_t)(xcd + 1) * total / 8);
  int t_cur = xbeg + blockIdx.x / 8;
  if (t_cur >= xend) return;

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int fr = lane & 31, fh = lane >> 5;
  const int K = (int)a.K, N = (int)a.N, ksplit = (int)a.k_split;
  const int nk = ((K + 2 * BK - 1) / (2 * BK)) * 2;  // stages per tile, even (trailing zero stage for odd counts)
  const uint32_t lda2 = (uint32_t)a.lda * 2u, ldb2 = (uint32_t)a.ldb * 2u;

  // ---- copy geometry.  K-major operand (A, and B_NK): copy i of a lane takes row 32 i + tid / 8, 16-byte chunk
  // tid % 8 of the stage's 64 k; LDS row r of 128 B holds chunk c at slot c ^ ((r >> 1) & 7).
  const int kr = tid >> 3, kc = tid & 7;
  const uint32_t km_w = (uint32_t)(kr * 128 + ((kc ^ ((kr >> 1) & 7)) << 4));
  // N-major B (B_KN): copy i takes k row 16 (i % 4) + tid / 16 of sub-tile i / 4 (128 columns; SwiGLU: 0 gate, 1 up),
  // chunk tid % 16; LDS: sub-tiles of 64 k rows x 256 B, chunk c of row k at slot c ^ ((k & 3) << 2) (nm_off).
  const int nr = tid >> 4, nc = tid & 15;
  const uint32_t nm_w = (uint32_t)(nr * 256 + ((nc ^ ((nr & 3) << 2)) << 4));

  // ---- load cursor: stage lk of tile lt; its descriptors and per-lane offsets
  int lt = t_cur, lk = 0;
  rsrc_t la, lb, lb2;
  const int a_kc = 8 * kc;  // k of this lane's K-major chunk within a stage
  // K-major copies (contiguous A rows, B_NK): row 32 i + kr of the operand at a byte offset of km_base + 32 i ld
  const uint32_t ka_base = (uint32_t)kr * lda2 + 16u * kc, kb_base = (uint32_t)kr * ldb2 + 16u * kc;
  // B_KN copies: k row 16 (i % 4) + nr, column n0 + 8 nc (+ 128 for sub-tile 1 of the plain store); whether the
  // column exists, per sub-tile
  const uint32_t nb_base = (uint32_t)nr * ldb2 + 16u * nc;
  bool ncol_ok[2] = {true, true};
  // gathered A: byte offsets of this lane's 8 source rows in the cursor's tile, and the raw row indices of the tile
  // after it (read one tile ahead, so their latency hides behind a whole tile) with that tile's row count.  Nothing
  // reads a loaded index before set_ld uses it: a select on it here would wait for it at once, and with the in-order
  // vector memory count that wait drains every copy load in flight.
  uint32_t a_off[8];
  const uint64_t magic = div_magic(GATHER ? a.a_div : 1);
  int pf_rows = 0;
  int pf_idx[8];
  auto fetch_idx = [&](int t) {
    const Tile rt = row_tile(a, t / a.n_tiles);
#pragma unroll
    for (int i = 0; i < 8; ++i) pf_idx[i] = a.a_rows[rt.row0 + min(32 * i + kr, rt.rows - 1)];
    pf_rows = rt.rows;
  };
  auto set_ld = [&]() {
    const int b = lt / a.n_tiles, nt = lt % a.n_tiles;
    const Tile rt = row_tile(a, b);
    const bool xe = rt.expert == a.x_expert;
    const bf16_t* Bb = xe ? a.Bx : a.B + (int64_t)rt.expert * a.b_estride;
    const bf16_t* B2b = xe ? (a.B2x ? a.B2x : Bb) : (a.B2 ? a.B2 + (int64_t)rt.expert * a.b_estride : Bb);
    if (GATHER) {
      la = rsrc(a.A, a.a_nrows * (int64_t)a.lda * 2);  // pf_idx: tile lt's indices
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int src = 32 * i + kr < pf_rows && pf_idx[i] >= 0 ? div_by(pf_idx[i], magic) : -1;  // rows past the tile: -1
        a_off[i] = src >= 0 ? (uint32_t)src * lda2 + 16u * kc : OOB;
      }
      if (lt + nper < xend) fetch_idx(lt + nper);
    } else {
      la = rsrc(a.A + rt.row0 * a.lda, (int64_t)rt.rows * a.lda * 2);  // rows past the tile: zeros
    }
    if (BMODE == B_NK) {
      const int64_t n0 = (int64_t)nt * BN;
      const int64_t nb = max((int64_t)0, (int64_t)N - n0);  // columns of this tile that exist
      lb = rsrc(Bb + n0 * a.ldb, nb * a.ldb * 2);
      lb2 = rsrc(B2b + n0 * a.ldb, nb * a.ldb * 2);
    } else {
      const int64_t n0 = (int64_t)nt * NOUT;
      lb = rsrc(Bb + n0, ((int64_t)K * a.ldb - n0) * 2);  // rows past K: zeros
      lb2 = rsrc(B2b + n0, ((int64_t)K * a.ldb - n0) * 2);
#pragma unroll
      for (int h = 0; h < 2; ++h) ncol_ok[h] = n0 + (EPI == EPI_SWIGLU_FWD ? 0 : NOUT / 2 * h) + 8 * nc < N;
    }
  };
  if (GATHER) fetch_idx(lt);  // the first tile's indices; set_ld then reads each next tile's one tile ahead
  set_ld();

  u32x4 R[16];  // one stage of this lane's copies: A chunks 0..7, B chunks 8..15
  // copy c of stage lk of the cursor's tile (nothing past the last tile: zeros)
  auto gload = [&](int c, int lk) {
    const bool live = lt < xend;
    const int k0 = lk * BK;
    if (c < 8) {
      const bool ok = live && k0 + a_kc < K;
      const uint32_t off = GATHER ? a_off[c] : ka_base + (uint32_t)(32 * c) * lda2;
      R[c] = ld16(la, ok ? off + 2u * (uint32_t)k0 : OOB);
    } else {
      const int i = c - 8;
      if (BMODE == B_NK) {
        const bool second = ksplit && k0 >= ksplit;  // uniform
        const int kb = second ? k0 - ksplit : k0;
        const bool ok = live && k0 + a_kc < K;
        R[c] = ld16(second ? lb2 : lb, ok ? kb_base + (uint32_t)(32 * i) * ldb2 + 2u * (uint32_t)kb : OOB);
      } else {
        const bool up = EPI == EPI_SWIGLU_FWD && i >= 4;
        const uint32_t off = nb_base + (uint32_t)(16 * (i & 3) + k0) * ldb2 + (EPI == EPI_SWIGLU_FWD ? 0u : 256u * (i >> 2));
        R[c] = ld16(up ? lb2 : lb, live && ncol_ok[i >> 2] ? off : OOB);
      }
    }
  };
  auto swrite = [&](int c, int buf) {
    char* p = smem + buf * STAGE_BYTES;
    if (c < 8) p += 4096 * c + km_w;
    else if (BMODE == B_NK) p += OP_BYTES + 4096 * (c - 8) + km_w;
    else p += OP_BYTES + ((c - 8) >> 2) * (BK * 256) + 16 * 256 * ((c - 8) & 3) + nm_w;
    *reinterpret_cast<u32x4*>(p) = R[c];
  };

  // ---- fragments: A rows wm 128 + 32 i + lane % 32, chunk 2 s + lane / 32 (same swizzle for every i)
  uint32_t rofs[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) rofs[s] = (uint32_t)(fr * 128 + (((2 * s + fh) ^ ((fr >> 1) & 7)) << 4));
  // B column of fragment j within the tile (SwiGLU forward: j < 2 gate, j >= 2 up, same output columns)
  auto bcol = [&](int j) {
    if (EPI == EPI_SWIGLU_FWD) return (j >> 1) * 128 + wn * 64 + 32 * (j & 1);
    return wn * 128 + 32 * j;
  };
  typedef FragSet<4, 4> F;
  auto fread = [&](F& f, int buf, int s) {
    const char* st = smem + buf * STAGE_BYTES;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      f.x[i] = as_bf16x8(*reinterpret_cast<const u32x4*>(st + rofs[s] + wm * 128 * 128 + 4096 * i));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (BMODE == B_NK) {
        f.w[j] = as_bf16x8(*reinterpret_cast<const u32x4*>(st + OP_BYTES + rofs[s] + wn * 128 * 128 + 4096 * j));
      } else {
        const int col = bcol(j);
        f.w[j] = frag_n(reinterpret_cast<const bf16_t*>(st + OP_BYTES) + (col >> 7) * (BK * 128), 16 * s, col & 127,
                        lane);
      }
    }
  };
  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};
  auto mma = [&](const F& f) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = mfma32<ET>(f.w[j], f.x[i], acc[i][j]);
  };

  // the cursor's next stage (past the last of a tile: the next tile's first)
  auto adv = [&]() {
    if (++lk == nk) {
      lk = 0;
      lt += nper;
      if (lt < xend) set_ld();
    }
  };

  // The SwiGLU forward (three outputs per tile) moves the next tile's stage 1 into LDS before its epilogue (EARLY,
  // see the tile loop); the other epilogues keep stage 1 in registers, which leaves them more registers.
  constexpr bool EARLY = EPI == EPI_SWIGLU_FWD;

  // ---- prologue: stage 0 -> LDS half 0, stage 1 -> registers (EARLY: -> half 1, and stage 2 -> registers)
#pragma unroll
  for (int c = 0; c < 16; ++c) gload(c, lk);
  adv();
#pragma unroll
  for (int c = 0; c < 16; ++c) swrite(c, 0);
#pragma unroll
  for (int c = 0; c < 16; ++c) gload(c, lk);
  adv();
  if constexpr (EARLY) {
#pragma unroll
    for (int c = 0; c < 16; ++c) swrite(c, 1);
#pragma unroll
    for (int c = 0; c < 16; ++c) gload(c, lk);
    adv();
  }
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  F f0, f1;
  fread(f0, 0, 0);

  // ---- epilogue of tile t_cur from the accumulators, through this wave's staging area; clears the accumulators.
  // No divergent control flow: every lane takes part in every LDS pass (passes split the wave's block by columns),
  // and the global accesses are raw buffer accesses over the tile's rows, so rows past the tile fall outside the
  // descriptor and a column past N takes the out-of-range offset -- the hardware drops such stores and returns zeros
  // for such loads.  (An exec-masked staging pass was miscompiled: reads of a later pass were sunk into the masked
  // write block of another.)
  char* const stg = smem + RING_BYTES + wave * STG_BYTES;
  auto st16 = [&](rsrc_t r, uint32_t off, u32x4 v) { __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, 0); };
  auto epilogue = [&]() {
    // the lane index, opaque to the compiler here: the per-lane row offsets below are then formed inside each
    // epilogue, instead of being hoisted out of the tile loop and held (or spilled) across every K loop
    int el = lane;
    asm volatile("" : "+v"(el));
    const int efr = el & 31, efh = el >> 5;
    const int b = t_cur / a.n_tiles, nt = t_cur % a.n_tiles;
    const Tile rt = row_tile(a, b);
    const int64_t n0 = (int64_t)nt * NOUT;
    // the tile's rows of each output (pitches in elements; an absent output gets an empty descriptor)
    const int osz = (EPI == EPI_STORE && OUTF32) ? 4 : 2;
    const rsrc_t rC = rsrc(reinterpret_cast<const char*>(OUTF32 ? (const void*)a.Cf : (const void*)a.C) + rt.row0 * a.ldc * osz,
                           (int64_t)rt.rows * a.ldc * osz);
    const rsrc_t rG = rsrc(a.G ? a.G + rt.row0 * a.ldg : nullptr, a.G ? (int64_t)rt.rows * a.ldg * 2 : 0);
    const rsrc_t rU = rsrc(a.U ? a.U + rt.row0 * a.ldg : nullptr, a.U ? (int64_t)rt.rows * a.ldg * 2 : 0);
    // SwiGLU backward: the routing weight of each row (tiles of the extra expert: 1)
    const bool scl = EPI == EPI_SWIGLU_BWD && a.row_scale && rt.expert != a.x_expert;
    const rsrc_t rW = rsrc(scl ? a.row_scale + rt.row0 : nullptr, scl ? (int64_t)rt.rows * 4 : 0);
    const uint32_t ldc_b = (uint32_t)a.ldc * osz, ldg_b = (uint32_t)a.ldg * 2;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int rbase = wm * 128 + 32 * i;  // first tile row of this slice
      if (EPI == EPI_SWIGLU_FWD) {
        // 32 rows x 64 outputs in two passes of 32 columns: the f32 gate fragment j (chunks 0-7 of a 256-byte staging
        // row) and up fragment j + 2 (chunks 8-15, same columns); read back 8 columns per lane -> h = silu(g) u, g, u
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int ch = 2 * q + efh;
            *reinterpret_cast<f32x4*>(stg + efr * 256 + ((ch ^ (efr & 15)) << 4)) =
                f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
            *reinterpret_cast<f32x4*>(stg + efr * 256 + (((8 + ch) ^ (efr & 15)) << 4)) =
                f32x4{acc[i][j + 2][4 * q], acc[i][j + 2][4 * q + 1], acc[i][j + 2][4 * q + 2], acc[i][j + 2][4 * q + 3]};
          }
#pragma unroll
          for (int it = 0; it < 2; ++it) {
            const int r = 16 * it + (el >> 2), c8 = el & 3;
            float g[8], u[8], h[8];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
              const f32x4 gv = *reinterpret_cast<const f32x4*>(stg + r * 256 + (((2 * c8 + e) ^ (r & 15)) << 4));
              const f32x4 uv = *reinterpret_cast<const f32x4*>(stg + r * 256 + (((8 + 2 * c8 + e) ^ (r & 15)) << 4));
#pragma unroll
              for (int t = 0; t < 4; ++t) {
                g[4 * e + t] = gv[t];
                u[4 * e + t] = uv[t];
              }
            }
#pragma unroll
            for (int t = 0; t < 8; ++t) h[t] = silu_f(g[t]) * u[t];
            const int64_t col = n0 + wn * 64 + 32 * j + 8 * c8;
            const bool cok = col < N;
            const uint32_t oc = cok ? (uint32_t)(rbase + r) * ldc_b + (uint32_t)col * 2u : OOB;
            const uint32_t og = cok ? (uint32_t)(rbase + r) * ldg_b + (uint32_t)col * 2u : OOB;
            st16(rC, oc, u32x4{pack_bf16x2(h[0], h[1]), pack_bf16x2(h[2], h[3]), pack_bf16x2(h[4], h[5]),
                               pack_bf16x2(h[6], h[7])});
            st16(rG, og, u32x4{pack_bf16x2(g[0], g[1]), pack_bf16x2(g[2], g[3]), pack_bf16x2(g[4], g[5]),
                               pack_bf16x2(g[6], g[7])});
            st16(rU, og, u32x4{pack_bf16x2(u[0], u[1]), pack_bf16x2(u[2], u[3]), pack_bf16x2(u[4], u[5]),
                               pack_bf16x2(u[6], u[7])});
          }
        }
      } else if (EPI == EPI_SWIGLU_BWD) {
        // dH of 32 rows x 64 columns per pass (fragments 2 jp, 2 jp + 1, f32), read back 8 columns per lane beside
        // the saved g and u -> [dG | dU]; dH rows scaled by their routing weight first (row_scale)
        float ws[4];
#pragma unroll
        for (int it = 0; it < 4; ++it) ws[it] = scl ? ldf(rW, (uint32_t)(rbase + 8 * it + (el >> 3)) * 4u) : 1.f;
#pragma unroll
        for (int jp = 0; jp < 2; ++jp) {
          u32x4 gq[4], uq[4];  // fetched first, so their latency overlaps the LDS round trip
          uint32_t oo[4];
#pragma unroll
          for (int it = 0; it < 4; ++it) {
            const int r = 8 * it + (el >> 3);
            const int64_t col = n0 + wn * 128 + 64 * jp + 8 * (el & 7);
            const uint32_t og = col < N ? (uint32_t)(rbase + r) * ldg_b + (uint32_t)col * 2u : OOB;
            oo[it] = col < N ? (uint32_t)(rbase + r) * ldc_b + (uint32_t)col * 2u : OOB;
            gq[it] = ld16(rG, og);
            uq[it] = ld16(rU, og);
          }
#pragma unroll
          for (int jj = 0; jj < 2; ++jj)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int ch = 8 * jj + 2 * q + efh;
              *reinterpret_cast<f32x4*>(stg + efr * 256 + ((ch ^ (efr & 15)) << 4)) =
                  f32x4{acc[i][2 * jp + jj][4 * q], acc[i][2 * jp + jj][4 * q + 1], acc[i][2 * jp + jj][4 * q + 2],
                        acc[i][2 * jp + jj][4 * q + 3]};
            }
#pragma unroll
          for (int it = 0; it < 4; ++it) {
            const int r = 8 * it + (el >> 3), c8 = el & 7;
            float v[8], dg[8], du[8];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
              const f32x4 x = *reinterpret_cast<const f32x4*>(stg + r * 256 + (((2 * c8 + e) ^ (r & 15)) << 4));
#pragma unroll
              for (int t = 0; t < 4; ++t) v[4 * e + t] = x[t];
            }
#pragma unroll
            for (int t = 0; t < 8; ++t) {
              const uint32_t gw = gq[it][t >> 1], uw = uq[it][t >> 1];
              const float g = __uint_as_float((t & 1) ? (gw & 0xffff0000u) : (gw << 16));
              const float u = __uint_as_float((t & 1) ? (uw & 0xffff0000u) : (uw << 16));
              const float sg = sigmoid_f(g);
              const float dh = v[t] * ws[it];
              dg[t] = dh * u * sg * (1.f + g * (1.f - sg));
              du[t] = dh * g * sg;
            }
            st16(rC, oo[it], u32x4{pack_bf16x2(dg[0], dg[1]), pack_bf16x2(dg[2], dg[3]), pack_bf16x2(dg[4], dg[5]),
                                   pack_bf16x2(dg[6], dg[7])});
            st16(rC, oo[it] == OOB ? OOB : oo[it] + (uint32_t)N * 2u,
                 u32x4{pack_bf16x2(du[0], du[1]), pack_bf16x2(du[2], du[3]), pack_bf16x2(du[4], du[5]),
                       pack_bf16x2(du[6], du[7])});
          }
        }
      } else if (EPI == EPI_STORE && !OUTF32) {
        // 32 rows x 128 columns of 16-bit outputs; read back 8 columns per lane, 16 lanes per 256-byte row
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            uint32_t w0, w1;
            if constexpr (ET == LSURGE_F16) {
              typedef _Float16 h2 __attribute__((ext_vector_type(2)));
              w0 = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){acc[i][j][4 * q], acc[i][j][4 * q + 1]}, h2));
              w1 = __builtin_bit_cast(uint32_t,
                                      __builtin_convertvector((f32x2_t){acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]}, h2));
            } else {
              w0 = pack_bf16x2(acc[i][j][4 * q], acc[i][j][4 * q + 1]);
              w1 = pack_bf16x2(acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
            }
            *reinterpret_cast<u32x2*>(stg + efr * 256 + (((4 * j + q) ^ (efr & 15)) << 4) + 8 * efh) = u32x2{w0, w1};
          }
#pragma unroll
        for (int it = 0; it < 8; ++it) {
          const int r = 4 * it + (el >> 4), c = el & 15;
          const u32x4 v = *reinterpret_cast<const u32x4*>(stg + r * 256 + ((c ^ (r & 15)) << 4));
          const int64_t col = n0 + wn * 128 + 8 * c;
          st16(rC, col < N ? (uint32_t)(rbase + r) * ldc_b + (uint32_t)col * 2u : OOB, v);
        }
      } else {
        // plain f32 store: 32 rows x 64 columns per pass (fragments 2 jp, 2 jp + 1), 16 lanes per 256-byte row
#pragma unroll
        for (int jp = 0; jp < 2; ++jp) {
#pragma unroll
          for (int jj = 0; jj < 2; ++jj)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int ch = 8 * jj + 2 * q + efh;  // 16-byte chunk of 4 f32 columns
              *reinterpret_cast<f32x4*>(stg + efr * 256 + ((ch ^ (efr & 15)) << 4)) =
                  f32x4{acc[i][2 * jp + jj][4 * q], acc[i][2 * jp + jj][4 * q + 1], acc[i][2 * jp + jj][4 * q + 2],
                        acc[i][2 * jp + jj][4 * q + 3]};
            }
#pragma unroll
          for (int it = 0; it < 8; ++it) {
            const int r = 4 * it + (el >> 4), c = el & 15;
            const u32x4 v = *reinterpret_cast<const u32x4*>(stg + r * 256 + ((c ^ (r & 15)) << 4));
            const int64_t col = n0 + wn * 128 + 64 * jp + 4 * c;
            st16(rC, col < N ? (uint32_t)(rbase + r) * ldc_b + (uint32_t)col * 4u : OOB, v);
          }
        }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};
    }
  };

  // Stage k writes stage k + 1 from the registers to LDS and loads stage k + 2 (past the tile's end: the next tile's
  // stages 0 and 1).
  // EARLY: a tile starts with stage 0 in LDS half 0, stage 1 in half 1 and stage 2 in registers, and its stage 0
  // copies nothing.  Between the last stage and the epilogue the next tile's stage 1 goes to LDS (the half the last
  // stage has just released) and its stage 2 is loaded, so every load the next tile's first two stages wait for was
  // issued before the epilogue's stores.  The tile's output write (all workgroups finish their tiles at about the
  // same time, so it is an HBM-bound burst) then drains while the next tile computes, instead of holding its LDS
  // writes, which wait for the vector memory count in issue order.  Measured on the gate/up forward (three outputs
  // per tile): 5% faster; on the plain-store and SwiGLU-backward epilogues no gain, and the plain store then spills.
  constexpr int NR = BMODE == B_NK ? 8 : 12;  // LDS reads per MFMA step (transpose reads take two per fragment)
  while (true) {
    if constexpr (EARLY) {
      run_stage<NR, false>(f0, f1, 0, lk, fread, swrite, gload, mma);
      run_stage<NR>(f0, f1, 1, lk, fread, swrite, gload, mma);
      adv();
      for (int kt = 2; kt < nk; kt += 2) {
        run_stage<NR>(f0, f1, 0, lk, fread, swrite, gload, mma);
        adv();
        run_stage<NR>(f0, f1, 1, lk, fread, swrite, gload, mma);
        adv();
      }
#pragma unroll
      for (int c = 0; c < 16; ++c) {
        swrite(c, 1);
        gload(c, lk);
      }
      adv();
    } else {
      for (int kt = 0; kt < nk; kt += 2) {
        run_stage<NR>(f0, f1, 0, lk, fread, swrite, gload, mma);
        adv();
        run_stage<NR>(f0, f1, 1, lk, fread, swrite, gload, mma);
        adv();
      }
    }
    epilogue();
    t_cur += nper;
    if (t_cur >= xend) break;
  }
  __builtin_amdgcn_s_waitcnt(0);  // the zero loads past the last tile land before the wave ends
}

// Weight gradient C_e[I, N] = A_e^T B_e over the chunk table of gemm_wgrad_kernel (a.c_expert / c_row0 / c_rows /
// c_part, num_chunks[0] real chunks): chunk c reduces rows [c_row0, c_row0 + c_rows) of expert c_expert and writes its
// partial slot (c_part >= 0, summed afterwards in chunk order) or the gradient itself (C / C2 split at n_split, Cx / C2x
// for the extra expert).  Tiles are 256 I-rows x 256 N-columns of one chunk (16 per chunk at the gate/up shape).
// Both operands are row-major [rows, ld] with the reduction over the rows, so both are staged N-major (64 reduction
// rows x 2 sub-tiles of 128 columns, the layout of the row GEMM's B_KN operand) and read with the transpose read.
// GATHER: reduction row r of A is A[a_rows[r] / a_div] (the layer's x rows through row_src).  An index cursor runs one
// stage ahead of the copies: each stage's row indices are read before the previous stage's data loads are issued,
// so the wait for them never waits for data.
// ONB (with GATHER): the gather applies to B instead, and each gathered B row is multiplied by b_scale[r] (chunks of
// x_expert: 1) and rounded to bf16 as it is staged into LDS (the layer's dY rows times their routing weight, the
// operand the combine backward would otherwise write out); the weights ride along the row indices.
template <bool GATHER, int ET = LSURGE_BF16, bool ONB = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void wgrad_kernel(WgradArgs a) {
  __shared__ __attribute__((aligned(1024))) char smem[SMEM_BYTES];
  const int nch = min(ctab(a.num_chunks, 0), a.max_chunks);
  const int tpc = a.i_tiles * a.n_tiles;
  // Tile order: chunk c runs on XCD c % 8 (the table puts the hot and shared experts' chunks first, so they spread over
  // the XCDs), its tiles on consecutive workgroups of that XCD, which share its rows in L2.  With fewer chunks than
  // XCDs that would leave XCDs idle (one chunk: 1/8 of the chip), so there every XCD takes an equal contiguous share
  // of all nch * tpc tiles instead.  Persistent grid (one workgroup per CU): workgroup l of an XCD takes the XCD's
  // tiles l, l + 32, ... and, of a last partial round, tile 31 - l, so that round lands on the workgroups that did
  // not start with a heavy chunk.  Otherwise one tile per workgroup, dealt the same way over the grid.
  const int xcd = blockIdx.x % 8, wl = blockIdx.x / 8;
  const bool flat = nch < 8;
  const int xbase = flat ? xcd * nch * tpc / 8 : 0;
  const int xchunks = nch > xcd ? (nch - xcd + 7) / 8 : 0;  // chunks xcd, xcd + 8, ...
  const int xlen = flat ? (xcd + 1) * nch * tpc / 8 - xbase : xchunks * tpc;
  const int npx = gridDim.x / 8;  // workgroups per XCD
  const bool pers = gridDim.x == NWG;
  const int full = pers ? xlen / npx : 0, part_n = pers ? xlen % npx : 0;
  const int ntiles_wg = pers ? full + ((npx - 1 - wl) < part_n ? 1 : 0) : (wl < xlen ? 1 : 0);
  // k-th tile of this workgroup as (chunk, tile in chunk) packed into c * tpc + r
  auto tile_of = [&](int k) {
    const int idx = !pers ? wl : (k < full ? npx * k + wl : npx * full + (npx - 1 - wl));
    return flat ? xbase + idx : (xcd + 8 * (idx / tpc)) * tpc + idx % tpc;
  };
  if (ntiles_wg == 0) return;
  int k_cur = 0, t_cur = tile_of(0);
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int I = (int)a.I, N = (int)a.N;
  const uint32_t lda2 = (uint32_t)a.lda * 2u, ldb2 = (uint32_t)a.ldb * 2u;
  // copy geometry (both operands N-major): copy i takes reduction row 16 (i % 4) + nr of sub-tile i / 4, chunk nc
  const int nr = tid >> 4, nc = tid & 15;
  const uint32_t nm_w = (uint32_t)(nr * 256 + ((nc ^ ((nr & 3) << 2)) << 4));
  auto stages_of = [](int rows) { return max(2, (rows + 2 * BK - 1) / (2 * BK) * 2); };  // even, at least one pair

  // ---- copy cursor: the workgroup's tile number lk_t (tile lt); its chunk's rows, descriptors and column offsets
  int lk_t = 0, lt = t_cur;
  rsrc_t la, lb;
  uint32_t acol[2], bcol[2];  // byte offsets of this lane's A / B column in each sub-tile (OOB: past I / N)
  auto set_ld = [&]() {
    const int c = lt / tpc, rem = lt % tpc, it = rem / a.n_tiles, nt = rem % a.n_tiles;
    const int64_t row0 = ctab(a.c_row0, c);
    const int rows = ctab(a.c_rows, c);
    if (GATHER && !ONB) la = rsrc(a.A, a.a_nrows * (int64_t)a.lda * 2);
    else la = rsrc(a.A + row0 * a.lda, (int64_t)rows * a.lda * 2);  // rows past the chunk: zeros
    if (ONB) lb = rsrc(a.B, a.b_nrows * (int64_t)a.ldb * 2);
    else lb = rsrc(a.B + row0 * a.ldb, (int64_t)rows * a.ldb * 2);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t ca = (int64_t)it * BM + 128 * h + 8 * nc, cb = (int64_t)nt * BN + 128 * h + 8 * nc;
      acol[h] = ca < I ? (uint32_t)ca * 2u : OOB;
      bcol[h] = cb < N ? (uint32_t)cb * 2u : OOB;
    }
  };
  set_ld();

  // ---- gathered A: index cursor (tile xt, stage xk), one stage ahead of the copies; raw indices in flight (pend)
  // and the source-row byte offsets of the stage being copied (g_off)
  const uint64_t magic = div_magic(GATHER ? a.a_div : 1);
  int xk_t = 0, xt = t_cur, xk = 0, x_rows = 0, x_nk = 2;
  int64_t x_row0 = 0;
  bool x_one = false;  // ONB: the cursor's chunk belongs to x_expert (weights 1)
  // Raw indices in flight, and which of them are rows of the chunk (bit q; known at issue).  Nothing reads a loaded
  // index before x_take, a stage later: a select on it at issue would wait for it there, and with the in-order
  // vector memory count that wait drains every copy load in flight.
  int pend[4];
  uint32_t pend_ok = 0;
  bool pend_one = false;  // ONB: x_one of the pending rows
  // ONB: weights of the pending rows, of the copy stage, and of the B chunks in the staging registers (chunks i and
  // i + 4 share row i: the later one's load, the row's last in a stage, moves the weight along)
  float pend_w[4], w_cur[4], w_dat[4];
  uint32_t g_off[4];
  auto x_set = [&]() {  // unconditional stores (past the last tile: chunk 0's entries, no rows)
    const bool live = xk_t < ntiles_wg;
    const int c = live ? xt / tpc : 0;
    const int rows = ctab(a.c_rows, c);
    x_row0 = ctab(a.c_row0, c);
    x_rows = live ? rows : 0;
    x_nk = stages_of(rows);
    if (ONB) x_one = ctab(a.c_expert, c) == a.x_expert;
  };
  auto x_issue = [&]() {  // read the indices at the index cursor into pend, then advance the cursor
    pend_ok = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int r = xk * BK + 16 * q + nr;
      const bool ok = r < x_rows;
      pend[q] = a.a_rows[x_row0 + (ok ? r : 0)];
      pend_ok |= ok ? 1u << q : 0u;
      if (ONB) pend_w[q] = a.b_scale[x_row0 + (ok ? r : 0)];
    }
    if (ONB) pend_one = x_one;
    if (++xk == x_nk) {
      xk = 0;
      if (++xk_t < ntiles_wg) xt = tile_of(xk_t);
      x_set();
    }
  };
  auto x_take = [&]() {  // the pending indices become the copy cursor's stage
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      g_off[q] = ((pend_ok >> q) & 1u) && pend[q] >= 0 ? (uint32_t)div_by(pend[q], magic) * (ONB ? ldb2 : lda2) : OOB;
      if (ONB) w_cur[q] = pend_one ? 1.f : pend_w[q];
    }
  };
  if (GATHER) x_set();

  u32x4 R[16];
  // Copy c of stage lk.  Branch-free: the out-of-range tests are per-lane selects (a row offset or a column past the
  // operand is OOB; every in-range offset is below 2^31).  Past the last tile the cursor keeps that tile's descriptors
  // and re-reads its first stages, which nothing consumes.
  auto gload = [&](int c, int lk) {
    const int i = c & 7, h = i >> 2, q = i & 3;
    const uint32_t krow = (uint32_t)(lk * BK + 16 * q + nr);
    if (c < 8) {
      const uint32_t ro = GATHER && !ONB ? g_off[q] : krow * lda2;
      R[c] = ld16(la, ((acol[h] | ro) & OOB) ? OOB : ro + acol[h]);
    } else {
      const uint32_t ro = ONB ? g_off[q] : krow * ldb2;
      R[c] = ld16(lb, ((bcol[h] | ro) & OOB) ? OOB : ro + bcol[h]);
      if (ONB && h == 1) w_dat[q] = w_cur[q];
    }
  };
  auto swrite = [&](int c, int buf) {
    const int i = c & 7;
    char* p = smem + buf * STAGE_BYTES + (c < 8 ? 0 : OP_BYTES) + (i >> 2) * (BK * 256) + 16 * 256 * (i & 3) + nm_w;
    u32x4 v = R[c];
    if (ONB && c >= 8) {  // bf16(w * b), the rounding of the materialised operand
      const float w = w_dat[i & 3];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        v[e] = pack_bf16x2(__uint_as_float(v[e] << 16) * w, __uint_as_float(v[e] & 0xffff0000u) * w);
    }
    *reinterpret_cast<u32x4*>(p) = v;
  };
  typedef FragSet<4, 4> F;
  auto fread = [&](F& f, int buf, int s) {
    const bf16_t* st = reinterpret_cast<const bf16_t*>(smem + buf * STAGE_BYTES);
#pragma unroll
    for (int i = 0; i < 4; ++i) f.x[i] = frag_n(st + wm * (BK * 128), 16 * s, 32 * i, lane);
#pragma unroll
    for (int j = 0; j < 4; ++j) f.w[j] = frag_n(st + OP_BYTES / 2 + wn * (BK * 128), 16 * s, 32 * j, lane);
  };
  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};
  auto mma = [&](const F& f) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = mfma32<ET>(f.w[j], f.x[i], acc[i][j]);
  };

  // ---- prologue: stage 0 -> LDS half 0, stage 1 -> registers; the index cursor then points at stage 2.  Stage 2's
  // indices are read before stage 1's copies, as in the loop, so that at the loop head they are 16 loads deep on
  // either path (the wait there is then for them alone, not for the copies behind them).
  if (GATHER) {
    x_issue();
    x_take();
  }
#pragma unroll
  for (int c = 0; c < 16; ++c) gload(c, 0);
#pragma unroll
  for (int c = 0; c < 16; ++c) swrite(c, 0);
  if (GATHER) {
    x_issue();
    x_take();
    x_issue();
  }
#pragma unroll
  for (int c = 0; c < 16; ++c) gload(c, 1);
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  F f0, f1;
  fread(f0, 0, 0);

  // ---- epilogue of tile t_cur (f32): the chunk's partial slot, or the gradient split at n_split -- two uniform
  // destinations, lanes whose columns belong to the other one pass the out-of-range offset
  char* const stg = smem + RING_BYTES + wave * STG_BYTES;
  auto epilogue = [&]() {
    // the lane index, opaque to the compiler here (as in the row kernel's epilogue): the per-lane offsets below are
    // formed inside each epilogue instead of being held across the K loop, which the gathered-B variant's extra
    // registers would otherwise spill
    int el = lane;
    if (ONB) asm volatile("" : "+v"(el));
    const int efr = el & 31, efh = el >> 5;
    const int c = t_cur / tpc, rem = t_cur % tpc, it = rem / a.n_tiles, nt = rem % a.n_tiles;
    const int expert = ctab(a.c_expert, c), part = ctab(a.c_part, c);
    const int64_t i0 = (int64_t)it * BM, n0 = (int64_t)nt * BN;
    const int64_t irows = min((int64_t)BM, (int64_t)I - i0);
    const float* d1;
    const float* d2 = nullptr;
    int64_t pitch, split;
    if (part >= 0) {
      d1 = a.part + (int64_t)part * I * N;
      pitch = N;
      split = N;
    } else {
      const bool xe = expert == a.x_expert;
      d1 = xe ? a.Cx : a.C + (int64_t)expert * a.c_estride;
      d2 = xe ? a.C2x : (a.C2 ? a.C2 + (int64_t)expert * a.c_estride : nullptr);
      pitch = a.ldc;
      split = d2 ? a.n_split : N;
    }
    const rsrc_t r1 = rsrc(d1 + i0 * pitch, irows * pitch * 4);
    const rsrc_t r2 = rsrc(d2 ? d2 + i0 * pitch : nullptr, d2 ? irows * pitch * 4 : 0);
    const uint32_t pb = (uint32_t)pitch * 4u;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int rbase = wm * 128 + 32 * i;
#pragma unroll
      for (int jp = 0; jp < 2; ++jp) {
#pragma unroll
        for (int jj = 0; jj < 2; ++jj)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int ch4 = 8 * jj + 2 * q + efh;
            *reinterpret_cast<f32x4*>(stg + efr * 256 + ((ch4 ^ (efr & 15)) << 4)) =
                f32x4{acc[i][2 * jp + jj][4 * q], acc[i][2 * jp + jj][4 * q + 1], acc[i][2 * jp + jj][4 * q + 2],
                      acc[i][2 * jp + jj][4 * q + 3]};
          }
        // the pass's 64 columns: all before the split (one store to the first destination), all after it (one to
        // the second), or across it (both, each lane's column on one side)
        const int64_t seg = n0 + wn * 128 + 64 * jp;
        const int side = seg + 64 <= split ? 0 : seg >= split ? 1 : 2;
#pragma unroll
        for (int it2 = 0; it2 < 8; ++it2) {
          const int r = 4 * it2 + (el >> 4), cc = el & 15;
          const u32x4 v = *reinterpret_cast<const u32x4*>(stg + r * 256 + ((cc ^ (r & 15)) << 4));
          const int64_t col = seg + 4 * cc;
          const uint32_t rb = (uint32_t)(rbase + r) * pb;
          const uint32_t o1 = col < split ? rb + (uint32_t)col * 4u : OOB;
          const uint32_t o2 = col >= split && col < N ? rb + (uint32_t)(col - split) * 4u : OOB;
          if (side != 1) __builtin_amdgcn_raw_buffer_store_b128(v, r1, o1, 0, 0);
          if (side != 0) __builtin_amdgcn_raw_buffer_store_b128(v, r2, o2, 0, 0);
        }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};
    }
  };

  // stage kt loads stage kt + 2; the last pair loads the next tile's first two stages
  while (true) {
    const int nk = stages_of(ctab(a.c_rows, t_cur / tpc));
    for (int kt = 0; kt < nk; kt += 2) {
      if (kt + 2 == nk) {
        if (++lk_t < ntiles_wg) {
          lt = tile_of(lk_t);
          set_ld();
        }
      }
      const int lk = kt + 2 == nk ? 0 : kt + 2;
      if (GATHER) {
        x_take();
        x_issue();
      }
      run_stage<16>(f0, f1, 0, lk, fread, swrite, gload, mma);
      if (GATHER) {
        x_take();
        x_issue();
      }
      run_stage<16>(f0, f1, 1, lk + 1, fread, swrite, gload, mma);
    }
    epilogue();
    if (++k_cur >= ntiles_wg) break;
    t_cur = tile_of(k_cur);
  }
  __builtin_amdgcn_s_waitcnt(0);
}

}  // namespace g256
}  // namespace lsgemm
