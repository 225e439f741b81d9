// Chunked gated delta rule of the Gated DeltaNet block, forward and backward (head dims 128, chunks of 64 tokens),
// and the row l2 normalisation of its qk-norm branch.
//
// Replaces fast_chunk_gated_delta_rule (modal/gdn_fast.py:37-113; compute dtype bf16, no context parallelism) and its
// XLA autodiff.  Per sequence b and head h, with state S [Dk, Dv]:
//   S_t = exp(g_t) (I - beta_t k_t k_t^T) S_{t-1} + beta_t k_t v_t^T,   o_t = S_t^T q_t / sqrt(Dk)
// computed in the reference's chunked WY form.  Forward, two kernels:
//   gdn_chunk_kernel  one workgroup per (chunk, head, sequence), all chunks at once: the decayed strictly-lower
//                     S = (k beta) k^T, A = (I + S)^-1 by blocked forward substitution, u = A (v beta),
//                     w = A (k beta e^gcum) (both rounded to bf16, as the reference's compute dtype:
//                     gdn_fast.py:88-90), and the decayed intra-chunk attention q k^T (the scan body's attn_i,
//                     gdn_fast.py:103-105, which does not depend on the state); optionally S and A for the backward.
//   gdn_scan_kernel   one workgroup per (32 value columns, head, sequence), the chunks in order: the value columns
//                     of the state evolve independently, so the state's 128 x 32 slice stays in the accumulators of
//                     four waves and the scan runs on 4x as many workgroups as there are heads.  Per chunk
//                     (gdn_fast.py:99-109):
//                       v_new = u - w S,  o = (q e^gcum) S + attn v_new,  S = e^gcum_last S + (k e^(gcum_last-gcum))^T v_new
//                     optionally storing the state entering every chunk for the backward.
// Backward, three more: gdn_bscan_kernel (reverse scan of the state gradient), gdn_bgrad_kernel (per chunk, the
// products with the stored state and its gradient) and gdn_bchunk_kernel (the chunk-local backward through A, S and
// the attention).  The training forward keeps the chunk products and the per-chunk states for them
// (lsurge_gdn_chunked_fwd_save); lsurge_gdn_chunked_bwd recomputes them instead.
// Every product runs on the bf16 matrix cores with each f32 operand split into two bf16 terms (16 significant bits,
// products exact, f32 sums), as the reference runs them at HIGHEST precision.  Padding tokens past T are zeros with
// g = 0, as the reference pads (gdn_fast.py:61-65).
#include <cstring>

#include "launchers.h"

namespace {

constexpr int GC = 64;   // chunk
constexpr int GD = 128;  // head dim (keys and values)
constexpr int GP = GD + 8;  // LDS row pitch of a bf16 [GC][GD] tile (272 bytes: rows start 16 bytes apart in banks)
constexpr int GTH = 512;  // 8 waves: one workgroup fills a CU (its LDS tiles leave no room for a second)
constexpr int SB = 32;   // value columns per scan workgroup

__device__ __forceinline__ void unpack8g(u32x4 v, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(v[i] << 16);
    f[2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u);
  }
}

// bf16 matrix-core helpers.  D[32 x 32] += P[32 x 16] Q[16 x 32] (v_mfma_f32_32x32x16_bf16): lane l
// supplies row l % 32 of P and column l % 32 of Q at k = 8 (l / 32) .. + 7, and holds D[8 (r / 4) + 4 (l / 32) + r % 4]
// [l % 32] in acc[r].  An f32 operand goes in as two bf16 terms, hi = bf16(x) and lo = bf16(x - hi): 16 significant
// bits, the products exact and summed in f32.
__device__ __forceinline__ f32x16 mma_bf16(bf16x8 p, bf16x8 q, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(p, q, c, 0, 0, 0);
}
// 8 consecutive bf16 at (row, k) of a row-major LDS array of pitch PITCH elements (16-byte aligned rows)
template <int PITCH>
__device__ __forceinline__ bf16x8 frag_row(const bf16_t* base, int row, int k) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(base + row * PITCH + k));
}
// the same fragment with P[m][k] = A[k][m] read from a row-major A (rows k, pitch PITCH) by two transpose reads
// (ds_read_b64_tr_b16: in a 16-lane group, source lane s points at 4 values of row kb + s / 4, columns nb + 4 (s % 4);
// lane i receives column nb + i, rows kb .. kb + 3)
template <int PITCH>
__device__ __forceinline__ bf16x8 frag_col(const bf16_t* base, int mbase, int kbase, int lane) {
  const int g = lane >> 4, s = lane & 15;
  const int m = mbase + 16 * (g & 1) + 4 * (s & 3);
  const int k0 = kbase + 8 * (g >> 1) + (s >> 2);
  const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_PTR(s16x4, base + k0 * PITCH + m));
  const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_PTR(s16x4, base + (k0 + 4) * PITCH + m));
  typedef short s16x8 __attribute__((ext_vector_type(8)));
  const s16x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(bf16x8, v);
}
__device__ __forceinline__ uint32_t bf16_hi_lo(float x, uint32_t* lo) {
  const bf16_t h = f32_to_bf16(x);
  *lo = f32_to_bf16(x - bf16_to_f32(h));
  return h;
}
// four f32 -> hi and lo bf16 quads, 8-byte stores at two row-major places
__device__ __forceinline__ void store_hi_lo4(bf16_t* hi, bf16_t* lo, const float* x) {
  uint32_t l[4], h[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) h[i] = bf16_hi_lo(x[i], &l[i]);
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  *reinterpret_cast<u32x2*>(hi) = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
  *reinterpret_cast<u32x2*>(lo) = u32x2{l[0] | (l[1] << 16), l[2] | (l[3] << 16)};
}

// eight f32 -> bf16 fragment, and its hi / lo split
__device__ __forceinline__ bf16x8 pack8(const float* f) {
  return __builtin_bit_cast(bf16x8, u32x4{pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                                          pack_bf16x2(f[6], f[7])});
}
__device__ __forceinline__ void split8(const float* f, bf16x8& hi, bf16x8& lo) {
  float r[8];
  hi = pack8(f);
  const u32x4 hw = __builtin_bit_cast(u32x4, hi);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    r[2 * i] = f[2 * i] - __uint_as_float(hw[i] << 16);
    r[2 * i + 1] = f[2 * i + 1] - __uint_as_float(hw[i] & 0xffff0000u);
  }
  lo = pack8(r);
}

// Workgroup -> (value-column slice, head, sequence) of a scan grid (GD / SB, H, B).  The hardware deals workgroups to
// the 8 XCDs round-robin by linear id; renumbering id -> (id % 8) (count / 8) + id / 8 puts the GD / SB slices of one
// (sequence, head), which read the same q, k, w and attention tiles at the same time, on one XCD, whose L2 then
// fetches those tiles once instead of once per slice.
__device__ __forceinline__ void scan_ids(int& cb, int& h, int& b) {
  const int nx = gridDim.x, total = nx * gridDim.y * gridDim.z;
  int id = blockIdx.x + nx * (blockIdx.y + gridDim.y * blockIdx.z);
  if (total % 8 == 0) id = (id % 8) * (total / 8) + id / 8;
  cb = SB * (id % nx);
  const int bh = id / nx;
  h = bh % gridDim.y;
  b = bh / gridDim.y;
}

// MFMA fragments of an f32 [GC][GC + 1] LDS matrix M as hi / lo bf16 pairs: of row r (M[r][k .. k + 7]) or of column
// c (M[k .. k + 7][c])
__device__ __forceinline__ void frag_rowf(const float (*M)[GC + 1], int r, int k, bf16x8& hi, bf16x8& lo) {
  float f[8];
#pragma unroll
  for (int x = 0; x < 8; ++x) f[x] = M[r][k + x];
  split8(f, hi, lo);
}
__device__ __forceinline__ void frag_colf(const float (*M)[GC + 1], int c, int k, bf16x8& hi, bf16x8& lo) {
  float f[8];
#pragma unroll
  for (int x = 0; x < 8; ++x) f[x] = M[k + x][c];
  split8(f, hi, lo);
}

// grid (N, H, B).  Outputs per (b, h, n): u, w [GC][GD] bf16, attn [GC][GC] f32 (zero above the diagonal), gcum [GC].
// A = (I + S)^-1 by blocked forward substitution, as the reference's default (gdn_fast.py:21-27, inv="solve").  The
// reference's other mode, the Neumann product (I - S)(I + S^2)..(I + S^32), is exact in exact arithmetic but loses
// all accuracy in f32 once keys correlate (|S| up to 0.7 makes the partial products grow like binomials).
__global__ __launch_bounds__(GTH) void gdn_chunk_kernel(const bf16_t* __restrict__ q, const bf16_t* __restrict__ k,
                                                        const bf16_t* __restrict__ v, const float* __restrict__ g,
                                                        const bf16_t* __restrict__ beta, int T, int H, float qscale,
                                                        bf16_t* __restrict__ u_out, bf16_t* __restrict__ w_out,
                                                        float* __restrict__ attn_out, float* __restrict__ gcum_out,
                                                        float* __restrict__ s_out = nullptr,
                                                        float* __restrict__ a_out = nullptr) {
  // k (then k beta) and q (then v beta once the attention is done); in the S product k beta is formed from k where it
  // is used.  68,864 bytes of LDS: two workgroups per CU.
  __shared__ __attribute__((aligned(16))) bf16_t ks[GC][GP], qs[GC][GP];
  __shared__ float Sm[GC][GC + 1], Am[GC][GC + 1];  // S (its upper triangle: scratch of the inverse); A
  __shared__ float gc[GC], eg[GC], bt[GC];
  const int n = blockIdx.x, h = blockIdx.y, b = blockIdx.z, N = gridDim.x;
  const int tid = threadIdx.x, t0 = n * GC;
  const int wave = tid >> 6, lane = tid & 63, lc = lane & 31, lh = lane >> 5;
  const int64_t row0 = (int64_t)b * T;
  const int64_t chunk_id = ((int64_t)b * H + h) * N + n;
  constexpr int TI = GC * (GD / 8) / GTH;
  u32x4 vr[TI];  // v, loaded with k and q, used after the attention
  {  // every load first (rows past T read row T - 1 and are zeroed when used), then the LDS stores
    u32x4 kr[TI], qr[TI];
#pragma unroll
    for (int x = 0; x < TI; ++x) {
      const int e = tid + GTH * x, i = e / (GD / 8), c = 8 * (e % (GD / 8));
      const int64_t off = ((row0 + min(t0 + i, T - 1)) * H + h) * GD + c;
      kr[x] = *reinterpret_cast<const u32x4*>(k + off);
      qr[x] = *reinterpret_cast<const u32x4*>(q + off);
      vr[x] = *reinterpret_cast<const u32x4*>(v + off);
    }
    float gl = 0.f;
    bf16_t br = 0;
    if (tid < GC) {
      const int64_t tr = row0 + min(t0 + tid, T - 1);
      gl = g[tr * H + h];
      br = beta[tr * H + h];
    }
#pragma unroll
    for (int x = 0; x < TI; ++x) {
      const int e = tid + GTH * x, i = e / (GD / 8), c = 8 * (e % (GD / 8));
      const bool in = t0 + i < T;
      float f[8];
      unpack8g(qr[x], f);  // q * scale in the compute dtype (gdn_fast.py:56-57)
      *reinterpret_cast<u32x4*>(&ks[i][c]) = in ? kr[x] : u32x4{0u, 0u, 0u, 0u};
      *reinterpret_cast<u32x4*>(&qs[i][c]) =
          in ? u32x4{pack_bf16x2(f[0] * qscale, f[1] * qscale), pack_bf16x2(f[2] * qscale, f[3] * qscale),
                     pack_bf16x2(f[4] * qscale, f[5] * qscale), pack_bf16x2(f[6] * qscale, f[7] * qscale)}
             : u32x4{0u, 0u, 0u, 0u};
    }
    if (tid < GC) {
      const bool in = t0 + tid < T;
      gc[tid] = in ? gl : 0.f;
      bt[tid] = in ? bf16_to_f32(br) : 0.f;
    }
  }
  __syncthreads();
  if (tid < GC) {  // inclusive cumulative sum of g over the chunk (wave 0)
    float x = gc[tid];
#pragma unroll
    for (int o = 1; o < GC; o <<= 1) {
      const float y = __shfl_up(x, o, 64);
      if (tid >= o) x += y;
    }
    gc[tid] = x;
    eg[tid] = __expf(x);
    gcum_out[chunk_id * GC + tid] = x;
  }
  __syncthreads();
  // S = (k beta) k^T (strictly lower) and attn = (q scale) k^T (lower incl. diagonal), decayed: one 32 x 32 tile per
  // wave (waves 0-3 S, 4-7 attn), K = 128 on the bf16 matrix cores (both operands bf16: the products are exact).
  // The wave index goes through readfirstlane so that both branches are scalar and straight-line.
  {
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const int ti = 32 * ((wv & 3) >> 1), tj = 32 * (wv & 1), j = tj + lc;
    f32x16 acc = {};
    if (wv < 4) {
      const float bi = bt[ti + lc];  // beta of this lane's row
#pragma unroll
      for (int k0 = 0; k0 < GD; k0 += 16) {
        const int kk = k0 + 8 * lh;
        float f[8];  // k beta in the compute dtype (gdn_fast.py:78)
        unpack8g(*reinterpret_cast<const u32x4*>(&ks[ti + lc][kk]), f);
#pragma unroll
        for (int x = 0; x < 8; ++x) f[x] *= bi;
        acc = mma_bf16(pack8(f), frag_row<GP>(&ks[0][0], j, kk), acc);
      }
    } else {
#pragma unroll
      for (int k0 = 0; k0 < GD; k0 += 16) {
        const int kk = k0 + 8 * lh;
        acc = mma_bf16(frag_row<GP>(&qs[0][0], ti + lc, kk), frag_row<GP>(&ks[0][0], j, kk), acc);
      }
    }
    // decay e^(gcum_i - gcum_j) for j <= i, zero above (selected, so an overflow above the diagonal never propagates)
    const float gj = gc[j];
    float dec[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = ti + 8 * (r / 4) + 4 * lh + r % 4;
      const float e = __expf(gc[i] - gj);
      dec[r] = (wv < 4 ? j < i : j <= i) ? acc[r] * e : 0.f;
    }
    if (wv < 4) {
#pragma unroll
      for (int r = 0; r < 16; ++r) Sm[ti + 8 * (r / 4) + 4 * lh + r % 4][j] = dec[r];
      if (s_out)  // the backward reads the decayed S of every chunk
#pragma unroll
        for (int r = 0; r < 16; ++r) s_out[chunk_id * GC * GC + (ti + 8 * (r / 4) + 4 * lh + r % 4) * GC + j] = dec[r];
    } else {
      float* att = attn_out + chunk_id * GC * GC;
#pragma unroll
      for (int r = 0; r < 16; ++r) att[(ti + 8 * (r / 4) + 4 * lh + r % 4) * GC + j] = dec[r];
    }
  }
  __syncthreads();
  // every read of q and of raw k is done: v beta replaces q and k beta replaces k, in the compute dtype
  // (gdn_fast.py:78, 87), formed once here for the u and w products below
#pragma unroll
  for (int x = 0; x < TI; ++x) {
    const int e = tid + GTH * x, i = e / (GD / 8), c = 8 * (e % (GD / 8));
    float f[8], kf[8];
    unpack8g(t0 + i < T ? vr[x] : u32x4{0u, 0u, 0u, 0u}, f);
    unpack8g(*reinterpret_cast<const u32x4*>(&ks[i][c]), kf);
    const float bi = bt[i];
    *reinterpret_cast<u32x4*>(&qs[i][c]) =
        u32x4{pack_bf16x2(f[0] * bi, f[1] * bi), pack_bf16x2(f[2] * bi, f[3] * bi), pack_bf16x2(f[4] * bi, f[5] * bi),
              pack_bf16x2(f[6] * bi, f[7] * bi)};
    *reinterpret_cast<u32x4*>(&ks[i][c]) =
        u32x4{pack_bf16x2(kf[0] * bi, kf[1] * bi), pack_bf16x2(kf[2] * bi, kf[3] * bi),
              pack_bf16x2(kf[4] * bi, kf[5] * bi), pack_bf16x2(kf[6] * bi, kf[7] * bi)};
  }
  // A = (I + S)^-1 (L = I + S unit lower triangular), in three steps with a workgroup barrier after each:
  //  1. wave 0: the four diagonal 16 x 16 blocks B_b = L_bb^-1 by forward substitution: lane (b = l / 16,
  //     c = l % 16) keeps column c of B_b in registers, row i = -sum_{j < i} S_bb[i][j] B_b[j][c] (column entries
  //     above c are zero); the other waves zero the blocks above the diagonal;
  //  2. waves 0-1: the 32 x 32 inverses A_pp = [[B_2p, 0], [-B_2p+1 (S_2p+1,2p B_2p), B_2p+1]], wave-local (the
  //     partial product goes through the unused upper block of S);
  //  3. wave 0: A_10 = -A_11 (S_10 A_00), 32 x 32 tiles on the matrix cores with operands split hi / lo.
  // Three barriers where the row-by-row substitution takes 64.
  if (wave == 0) {  // S is in LDS since the barrier above
    const int o = 16 * (lane >> 4), c = lane & 15;
    float col[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float sacc = 0.f;
#pragma unroll
      for (int j = 0; j < i; ++j) sacc = fmaf(Sm[o + i][o + j], col[j], sacc);
      col[i] = c < i ? -sacc : (c == i ? 1.f : 0.f);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) Am[o + i][o + c] = col[i];
  } else {
    for (int e = tid - 64; e < 2 * 256 + 32 * 32; e += GTH - 64) {  // above the diagonal: two 16 blocks, one 32
      const int r = e < 256 ? e / 16 : e < 512 ? 32 + (e - 256) / 16 : (e - 512) / 32;
      const int c = e < 256 ? 16 + e % 16 : e < 512 ? 48 + e % 16 : 32 + (e - 512) % 32;
      Am[r][c] = 0.f;
    }
  }
  __syncthreads();
  if (wave < 2) {
    const int p = wave, ob = 32 * p, od = ob + 16;  // block 2p at ob, block 2p + 1 at od
    const int r = lane >> 2, cq = 4 * (lane & 3);
    float t4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      const float sv = Sm[od + r][ob + m];
#pragma unroll
      for (int x = 0; x < 4; ++x) t4[x] = fmaf(sv, Am[ob + m][ob + cq + x], t4[x]);
    }
#pragma unroll
    for (int x = 0; x < 4; ++x) Sm[16 * p + r][32 + cq + x] = t4[x];  // S above the diagonal is no longer needed
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's partial product is in LDS
    float x4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      const float av = Am[od + r][od + m];
#pragma unroll
      for (int x = 0; x < 4; ++x) x4[x] = fmaf(av, Sm[16 * p + m][32 + cq + x], x4[x]);
    }
#pragma unroll
    for (int x = 0; x < 4; ++x) Am[od + r][ob + cq + x] = -x4[x];
  }
  __syncthreads();
  if (wave == 0) {
    f32x16 y = {};
#pragma unroll
    for (int k0 = 0; k0 < 32; k0 += 16) {  // Y = S_10 A_00 (K = 32)
      const int kk = k0 + 8 * lh;
      bf16x8 ph_, pl_, qh_, ql_;
      frag_rowf(Sm, 32 + lc, kk, ph_, pl_);
      frag_colf(Am, lc, kk, qh_, ql_);
      y = mma_bf16(ph_, qh_, y);
      y = mma_bf16(ph_, ql_, y);
      y = mma_bf16(pl_, qh_, y);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) Sm[8 * (r / 4) + 4 * lh + r % 4][32 + lc] = y[r];  // into S's upper block
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    f32x16 z = {};
#pragma unroll
    for (int k0 = 0; k0 < 32; k0 += 16) {  // A_10 = -A_11 Y (K = 32)
      const int kk = k0 + 8 * lh;
      bf16x8 ph_, pl_, qh_, ql_;
      frag_rowf(Am, 32 + lc, 32 + kk, ph_, pl_);
      frag_colf(Sm, 32 + lc, kk, qh_, ql_);
      z = mma_bf16(ph_, qh_, z);
      z = mma_bf16(ph_, ql_, z);
      z = mma_bf16(pl_, qh_, z);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) Am[32 + 8 * (r / 4) + 4 * lh + r % 4][lc] = -z[r];
  }
  __syncthreads();
  // u = A vb, w = (A e^gcum) kb (= A (kb e^gcum)): one 32 x 32 tile of each per wave (token rows 32 (wave / 4),
  // columns 32 (wave % 4)), K = 64 on the bf16 matrix cores with A as hi / lo pairs; rounded to bf16
  // (gdn_fast.py:88-90)
  {
    const int ti = 32 * (wave >> 2), cd = 32 * (wave & 3);
    f32x16 ua = {}, wa = {};
#pragma unroll
    for (int k0 = 0; k0 < GC; k0 += 16) {
      const int kk = k0 + 8 * lh;
      float a8[8], e8[8];
#pragma unroll
      for (int x = 0; x < 8; ++x) {
        a8[x] = Am[ti + lc][kk + x];
        e8[x] = a8[x] * eg[kk + x];
      }
      bf16x8 ah, al, eh, el;
      split8(a8, ah, al);
      split8(e8, eh, el);
      const bf16x8 qv = frag_col<GP>(&qs[0][0], cd, k0, lane);  // v beta
      const bf16x8 qk = frag_col<GP>(&ks[0][0], cd, k0, lane);  // k beta
      ua = mma_bf16(ah, qv, ua);
      ua = mma_bf16(al, qv, ua);
      wa = mma_bf16(eh, qk, wa);
      wa = mma_bf16(el, qk, wa);
    }
    if (a_out)  // the backward reads A = (I + S)^-1 of every chunk
      for (int e = tid; e < GC * GC; e += GTH) a_out[chunk_id * GC * GC + e] = Am[e / GC][e % GC];
    bf16_t* ub = u_out + chunk_id * GC * GD;
    bf16_t* wb = w_out + chunk_id * GC * GD;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = ti + 8 * (r / 4) + 4 * lh + r % 4;
      ub[i * GD + cd + lc] = f32_to_bf16(ua[r]);
      wb[i * GD + cd + lc] = f32_to_bf16(wa[r]);
    }
  }
}

// Scan over the chunks of one (32 value columns, head, sequence), on the matrix cores.  Eight waves:
//   waves 4-7 hold the state slice S [128 x 32] in their accumulators (rows 32 (wave - 4) .., one 32 x 32 tile each),
//   waves 0-1 form w S (rows 32 wave ..) and v_new = u - w S, waves 2-3 form (q e^gcum) S and o = that + attn v_new.
// Per chunk, three phases between barriers:
//   A  every thread stages its prefetched share of q (scaled), k, w, attn (hi / lo) and u in LDS;
//   B  waves 0-3: w S or q S (K = 128); v_new to LDS as hi / lo, and e^(gcum_last - gcum) v_new for the update;
//   C  waves 2-3: o = (q S) e^gcum + attn v_new; waves 4-7: S = e^gcum_last S + k^T (e^(gcum_last - gcum) v_new),
//      then the new state to LDS (hi / lo, transposed) for the next chunk's phase B.
// The next chunk's tiles load into registers while a wave is otherwise idle: waves 4-7 during phase B, waves 2-3
// after their phase-B products, waves 0-1 during phase C.  LDS fragments of the next 16-deep step are read before
// the MFMAs of the current one, and the hi and lo products of a phase accumulate in two independent chains.
constexpr int KP = GC + 8;  // pitch of the [.][GC] bf16 tiles (144 bytes)
constexpr int UP = SB + 8;  // pitch of the u tile [GC][SB] (80 bytes)
__global__ __launch_bounds__(GTH) void gdn_scan_kernel(const bf16_t* __restrict__ q, const bf16_t* __restrict__ k,
                                                       const bf16_t* __restrict__ u_in, const bf16_t* __restrict__ w_in,
                                                       const float* __restrict__ attn_in,
                                                       const float* __restrict__ gcum_in, int T, int H, int N,
                                                       float qscale, const float* __restrict__ h0,
                                                       bf16_t* __restrict__ o, float* __restrict__ h_out,
                                                       float* __restrict__ h_chunks = nullptr) {
  __shared__ __attribute__((aligned(16))) bf16_t qs[GC][GP], ws[GC][GP], ks[GC][GP];  // [t][d]
  __shared__ __attribute__((aligned(16))) bf16_t ah[GC][KP], al[GC][KP];             // attn hi / lo [t][j]
  __shared__ __attribute__((aligned(16))) bf16_t shh[SB][GP], shl[SB][GP];           // state hi / lo [c][d]
  __shared__ __attribute__((aligned(16))) bf16_t vh[SB][KP], vl[SB][KP];             // v_new hi / lo [c][t]
  __shared__ __attribute__((aligned(16))) bf16_t vkh[SB][KP], vkl[SB][KP];           // e^(gl - g) v_new [c][t]
  __shared__ __attribute__((aligned(16))) bf16_t us[GC][UP];                          // u [t][c]
  __shared__ float gc[GC], ek[GC];  // gcum, exp(gcum_last - gcum)
  int cb, h, b;
  scan_ids(cb, h, b);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lc = lane & 31, lh = lane >> 5;  // this lane's column of a 32 x 32 tile, and its row quad offset (x 4)
  const int64_t row0 = (int64_t)b * T;
  const int64_t bh = (int64_t)b * H + h;
  // tile rows of this lane's accumulators: row(r) = rb + 8 (r / 4) + 4 lh + r % 4 (tokens for waves 0-3, state rows
  // for waves 4-7)
  const int rb = wave < 4 ? 32 * (wave & 1) : 32 * (wave - 4);
  f32x16 acc = {};  // waves 4-7: the state tile; waves 0-3: this chunk's product
  // waves 4-7: the state entering the next chunk to LDS (hi / lo, transposed)
  auto put_state = [&]() {
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int d = rb + 8 * q4 + 4 * lh;
      const float sv[4] = {acc[4 * q4], acc[4 * q4 + 1], acc[4 * q4 + 2], acc[4 * q4 + 3]};
      store_hi_lo4(&shh[lc][d], &shl[lc][d], sv);
    }
  };
  if (wave >= 4) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int d = rb + 8 * (r / 4) + 4 * lh + r % 4;
      acc[r] = h0 ? h0[(bh * GD + d) * GD + cb + lc] : 0.f;
    }
    put_state();
  }
  // This thread's share of the next chunk's tiles: two 16-byte pieces of each of q, k and w (piece e = tid + GTH p:
  // row e / 16, columns 8 (e % 16)), eight attn values, (threads < GC) one gcum value and (waves 4-7) 8 u values
  // (row (tid - 256) / 4, columns 8 ((tid - 256) % 4)).
  constexpr int PP = GC * (GD / 8) / GTH;  // pieces per thread and tile
  static_assert(PP * GTH == GC * (GD / 8) && GC * GC == 8 * GTH && GC * SB / 8 == GTH / 2, "scan tile split");
  u32x4 pq[PP], pk[PP], pw[PP], pu = {0u, 0u, 0u, 0u};
  f32x4 pa[2];
  float pg = 0.f;
  auto fetch = [&](int n) {
    const int t0 = n * GC;
    const int64_t chunk_id = bh * N + n;
#pragma unroll
    for (int p = 0; p < PP; ++p) {
      const int e = tid + GTH * p, i = e / (GD / 8), c = 8 * (e % (GD / 8));
      const bool in = t0 + i < T;
      const int64_t off = ((row0 + t0 + i) * H + h) * GD + c;
      pq[p] = in ? *reinterpret_cast<const u32x4*>(q + off) : u32x4{0u, 0u, 0u, 0u};
      pk[p] = in ? *reinterpret_cast<const u32x4*>(k + off) : u32x4{0u, 0u, 0u, 0u};
      pw[p] = *reinterpret_cast<const u32x4*>(w_in + chunk_id * GC * GD + i * GD + c);
    }
    const float* asrc = attn_in + chunk_id * GC * GC;
    pa[0] = *reinterpret_cast<const f32x4*>(asrc + 4 * tid);
    pa[1] = *reinterpret_cast<const f32x4*>(asrc + 4 * (tid + GTH));
    if (tid < GC) pg = gcum_in[chunk_id * GC + tid];
    if (wave >= 4) {
      const int e = tid - GTH / 2;
      pu = *reinterpret_cast<const u32x4*>(u_in + chunk_id * GC * GD + (e / (SB / 8)) * GD + cb + 8 * (e % (SB / 8)));
    }
  };
  fetch(0);
  for (int n = 0; n < N; ++n) {
    const int t0 = n * GC;
    __syncthreads();  // the previous chunk is done with every LDS tile
#pragma unroll
    for (int p = 0; p < PP; ++p) {
      const int e = tid + GTH * p, i = e / (GD / 8), c = 8 * (e % (GD / 8));
      float f[8];
      unpack8g(pq[p], f);  // q * scale in the compute dtype (gdn_fast.py:56-57)
      *reinterpret_cast<u32x4*>(&qs[i][c]) =
          u32x4{pack_bf16x2(f[0] * qscale, f[1] * qscale), pack_bf16x2(f[2] * qscale, f[3] * qscale),
                pack_bf16x2(f[4] * qscale, f[5] * qscale), pack_bf16x2(f[6] * qscale, f[7] * qscale)};
      *reinterpret_cast<u32x4*>(&ks[i][c]) = pk[p];
      *reinterpret_cast<u32x4*>(&ws[i][c]) = pw[p];
    }
#pragma unroll
    for (int hlf = 0; hlf < 2; ++hlf) {
      const int e = 4 * (tid + GTH * hlf);
      const float av[4] = {pa[hlf][0], pa[hlf][1], pa[hlf][2], pa[hlf][3]};
      store_hi_lo4(&ah[e / GC][e % GC], &al[e / GC][e % GC], av);
    }
    if (tid < GC) {  // wave 0: gcum and exp(gcum_last - gcum)
      gc[tid] = pg;
      ek[tid] = __expf(__shfl(pg, GC - 1, 64) - pg);
    }
    if (wave >= 4) {
      const int e = tid - GTH / 2;
      *reinterpret_cast<u32x4*>(&us[e / (SB / 8)][8 * (e % (SB / 8))]) = pu;
      if (h_chunks)  // the state entering chunk n, for the backward (issued here, after this phase's load wait)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          h_chunks[((bh * N + n) * GD + rb + 8 * (r / 4) + 4 * lh + r % 4) * GD + cb + lc] = acc[r];
    }
    __syncthreads();
    const bool more = n + 1 < N;
    if (wave >= 4 && more) fetch(n + 1);
    if (wave < 4) {  // w S (waves 0-1) or (q scale) S (waves 2-3), K = 128
      const bf16_t* P = wave < 2 ? &ws[0][0] : &qs[0][0];
      acc = f32x16{};
      f32x16 acc2 = {};
      bf16x8 pf[2], fh[2], fl[2];
      auto frags = [&](int s, int k0) {
        const int kk = k0 + 8 * lh;
        pf[s] = frag_row<GP>(P, rb + lc, kk);
        fh[s] = frag_row<GP>(&shh[0][0], lc, kk);
        fl[s] = frag_row<GP>(&shl[0][0], lc, kk);
      };
      frags(0, 0);
#pragma unroll
      for (int j = 0; j < GD / 16; ++j) {
        if (j + 1 < GD / 16) frags((j + 1) & 1, 16 * (j + 1));
        __builtin_amdgcn_sched_barrier(0);
        acc = mma_bf16(pf[j & 1], fh[j & 1], acc);
        acc2 = mma_bf16(pf[j & 1], fl[j & 1], acc2);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] += acc2[r];
      if (wave < 2) {  // v_new = u - w S, to LDS as hi / lo and, scaled by exp(gcum_last - gcum), for the update
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const int t = rb + 8 * q4 + 4 * lh;
          float vv[4], vk[4];
#pragma unroll
          for (int x = 0; x < 4; ++x) {
            vv[x] = bf16_to_f32(us[t + x][lc]) - acc[4 * q4 + x];
            vk[x] = vv[x] * ek[t + x];
          }
          store_hi_lo4(&vh[lc][t], &vl[lc][t], vv);
          store_hi_lo4(&vkh[lc][t], &vkl[lc][t], vk);
        }
      } else {  // inter = (q S) e^gcum
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] *= __expf(gc[rb + 8 * (r / 4) + 4 * lh + r % 4]);
        if (more) fetch(n + 1);
      }
    }
    __syncthreads();  // v_new is in LDS
    if (wave < 2) {
      if (more) fetch(n + 1);
    } else if (wave < 4) {  // o = inter + attn v_new (attn is zero above the diagonal), K = 64
      bf16x8 ph[2], pl[2], qh[2], ql[2];
      auto frags = [&](int s, int k0) {
        const int kk = k0 + 8 * lh;
        ph[s] = frag_row<KP>(&ah[0][0], rb + lc, kk);
        pl[s] = frag_row<KP>(&al[0][0], rb + lc, kk);
        qh[s] = frag_row<KP>(&vh[0][0], lc, kk);
        ql[s] = frag_row<KP>(&vl[0][0], lc, kk);
      };
      frags(0, 0);
      f32x16 acc2 = {};
#pragma unroll
      for (int j = 0; j < GC / 16; ++j) {
        if (j + 1 < GC / 16) frags((j + 1) & 1, 16 * (j + 1));
        __builtin_amdgcn_sched_barrier(0);
        acc = mma_bf16(ph[j & 1], qh[j & 1], acc);
        acc2 = mma_bf16(ph[j & 1], ql[j & 1], acc2);
        acc2 = mma_bf16(pl[j & 1], qh[j & 1], acc2);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] += acc2[r];
      if (o)  // the backward's recompute needs the states only
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int t = rb + 8 * (r / 4) + 4 * lh + r % 4;
          if (t0 + t < T) o[((row0 + t0 + t) * H + h) * GD + cb + lc] = f32_to_bf16(acc[r]);
        }
    } else {  // S = e^gcum_last S + k^T (e^(gcum_last - gcum) v_new), K = 64
      const float el = __expf(gc[GC - 1]);
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] *= el;
      bf16x8 pf[2], fh[2], fl[2];
      auto frags = [&](int s, int k0) {
        const int kk = k0 + 8 * lh;
        pf[s] = frag_col<GP>(&ks[0][0], rb, k0, lane);
        fh[s] = frag_row<KP>(&vkh[0][0], lc, kk);
        fl[s] = frag_row<KP>(&vkl[0][0], lc, kk);
      };
      frags(0, 0);
      f32x16 acc2 = {};
#pragma unroll
      for (int j = 0; j < GC / 16; ++j) {
        if (j + 1 < GC / 16) frags((j + 1) & 1, 16 * (j + 1));
        __builtin_amdgcn_sched_barrier(0);
        acc = mma_bf16(pf[j & 1], fh[j & 1], acc);
        acc2 = mma_bf16(pf[j & 1], fl[j & 1], acc2);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] += acc2[r];
      if (more) put_state();  // phase B of this chunk, the last reader of shh / shl, is past the barrier
    }
  }
  if (h_out && wave >= 4)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int d = rb + 8 * (r / 4) + 4 * lh + r % 4;
      h_out[(bh * GD + d) * GD + cb + lc] = acc[r];
    }
}


// =====================================================================================================================
// Backward.  XLA differentiates the reference's chunked form when the model trains through it (gdn_fast.py:37-113,
// installed for training at lightning/train_stage1.py:67-69); these kernels compute the same gradients in reverse
// order.  With the upstream gradient do of o and dH_T of the final state, per chunk (rows i, j of the chunk; the bf16
// rounding points of the forward are taken with derivative 1, as autodiff takes a dtype cast):
//   reverse scan   dH_n = the gradient of the state leaving chunk n (dH_T for the last chunk), and
//                  dv_new = attn^T do + kd dH_n,  dH_{n-1} = e^gl dH_n + qg^T do - w^T dv_new
//                  with kd = k e^(gl - gcum), qg = q e^gcum, gl = gcum of the last row;
//   chunk grads    (all chunks at once, from the forward's saved states h_n and the reverse scan's dH_n)
//                  v_new = u - w h_n, dqg = do h_n^T, dkd = v_new dH_n^T, dP = do v_new^T (lower), du = dv_new,
//                  dw = -dv_new h_n^T, dgl = e^gl <dH_n, h_n>;
//   chunk-local    dA = du vb^T + dw kbg^T, dS = -(A^T dA A^T) (strictly lower), dvb = A^T du, dkbg = A^T dw and from
//                  there dq, dk, dv, dbeta and dg (the gradient of gcum, then a suffix sum over the chunk).

// grid (GD / SB, H, B): the reverse scan for SB value columns of the state gradient.
__global__ __launch_bounds__(GTH) void gdn_bscan_kernel(const bf16_t* __restrict__ q, const bf16_t* __restrict__ k,
                                                        const bf16_t* __restrict__ w_in, const float* __restrict__ attn_in,
                                                        const float* __restrict__ gcum_in, const bf16_t* __restrict__ dout,
                                                        int T, int H, int N, float qscale,
                                                        const float* __restrict__ dh_final,
                                                        float* __restrict__ dh_chunks, float* __restrict__ dh0) {
  // On the bf16 matrix cores, as the forward scan: waves 4-7 hold the state gradient dH [128 x 32] in their
  // accumulators; waves 0-1 form dv_new for token rows 32 wave .. (attn^T do + e^(gl - g) k dH); waves 4-7 then update
  // dH <- e^gl dH + q^T (e^g do) - w^T dv_new.  f32 operands enter as hi / lo bf16 pairs.
  __shared__ __attribute__((aligned(16))) bf16_t qs[GC][GP], ks[GC][GP], ws[GC][GP];  // [t][d]
  __shared__ __attribute__((aligned(16))) bf16_t ah[GC][KP], al[GC][KP];             // attn hi / lo [j][t]
  __shared__ __attribute__((aligned(16))) bf16_t dhh[SB][GP], dhl[SB][GP];           // dH hi / lo [c][d]
  __shared__ __attribute__((aligned(16))) bf16_t doT[SB][KP];                        // do [c][t]
  __shared__ __attribute__((aligned(16))) bf16_t deh[SB][KP], del_[SB][KP];          // e^g do hi / lo [c][t]
  __shared__ __attribute__((aligned(16))) bf16_t dvh[SB][KP], dvl[SB][KP];           // -dv_new hi / lo [c][t]
  __shared__ float gc[GC], ek[GC];
  int cb, h, b;
  scan_ids(cb, h, b);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lc = lane & 31, lh = lane >> 5;
  const int64_t row0 = (int64_t)b * T;
  const int64_t bh = (int64_t)b * H + h;
  const int rb = wave < 4 ? 32 * (wave & 1) : 32 * (wave - 4);
  f32x16 acc = {};
  if (wave >= 4)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int d = rb + 8 * (r / 4) + 4 * lh + r % 4;
      acc[r] = dh_final ? dh_final[(bh * GD + d) * GD + cb + lc] : 0.f;
    }
  // next chunk's tiles in registers: q, k, w pieces as the forward scan, attn, and (threads < 256) one 8-column piece
  // of do (row e / 4, columns 8 (e % 4) of this block) with its row's gcum; (threads < GC) gcum of row tid
  constexpr int PP = GC * (GD / 8) / GTH;
  u32x4 pq[PP], pk[PP], pw[PP], pd = {0u, 0u, 0u, 0u};
  f32x4 pa[2];
  float pg = 0.f, pgd = 0.f;
  auto fetch = [&](int n) {
    const int t0 = n * GC;
    const int64_t chunk_id = bh * N + n;
#pragma unroll
    for (int p = 0; p < PP; ++p) {
      const int e = tid + GTH * p, i = e / (GD / 8), c = 8 * (e % (GD / 8));
      const bool in = t0 + i < T;
      const int64_t off = ((row0 + t0 + i) * H + h) * GD + c;
      pq[p] = in ? *reinterpret_cast<const u32x4*>(q + off) : u32x4{0u, 0u, 0u, 0u};
      pk[p] = in ? *reinterpret_cast<const u32x4*>(k + off) : u32x4{0u, 0u, 0u, 0u};
      pw[p] = *reinterpret_cast<const u32x4*>(w_in + chunk_id * GC * GD + i * GD + c);
    }
    const float* asrc = attn_in + chunk_id * GC * GC;
    pa[0] = *reinterpret_cast<const f32x4*>(asrc + 4 * tid);
    pa[1] = *reinterpret_cast<const f32x4*>(asrc + 4 * (tid + GTH));
    if (tid < GC) pg = gcum_in[chunk_id * GC + tid];
    if (tid < GC * SB / 8) {
      const int i = tid / (SB / 8), c = 8 * (tid % (SB / 8));
      pd = t0 + i < T ? *reinterpret_cast<const u32x4*>(dout + ((row0 + t0 + i) * H + h) * GD + cb + c)
                      : u32x4{0u, 0u, 0u, 0u};
      pgd = gcum_in[chunk_id * GC + i];
    }
  };
  fetch(N - 1);
  for (int n = N - 1; n >= 0; --n) {
    const int64_t chunk_id = bh * N + n;
    __syncthreads();  // the previous chunk is done with every LDS tile
#pragma unroll
    for (int p = 0; p < PP; ++p) {
      const int e = tid + GTH * p, i = e / (GD / 8), c = 8 * (e % (GD / 8));
      float f[8];
      unpack8g(pq[p], f);
      *reinterpret_cast<u32x4*>(&qs[i][c]) =
          u32x4{pack_bf16x2(f[0] * qscale, f[1] * qscale), pack_bf16x2(f[2] * qscale, f[3] * qscale),
                pack_bf16x2(f[4] * qscale, f[5] * qscale), pack_bf16x2(f[6] * qscale, f[7] * qscale)};
      *reinterpret_cast<u32x4*>(&ks[i][c]) = pk[p];
      *reinterpret_cast<u32x4*>(&ws[i][c]) = pw[p];
    }
#pragma unroll
    for (int hlf = 0; hlf < 2; ++hlf) {
      const int e = 4 * (tid + GTH * hlf);
      const float av[4] = {pa[hlf][0], pa[hlf][1], pa[hlf][2], pa[hlf][3]};
      store_hi_lo4(&ah[e / GC][e % GC], &al[e / GC][e % GC], av);
    }
    if (tid < GC) {
      gc[tid] = pg;
      ek[tid] = __expf(__shfl(pg, GC - 1, 64) - pg);
    }
    if (tid < GC * SB / 8) {  // do and e^g do, transposed to [column][row]
      const int i = tid / (SB / 8), c = 8 * (tid % (SB / 8));
      float f[8];
      unpack8g(pd, f);
      const float eg = __expf(pgd);
#pragma unroll
      for (int x = 0; x < 8; ++x) {
        doT[c + x][i] = f32_to_bf16(f[x]);
        uint32_t lo;
        deh[c + x][i] = (bf16_t)bf16_hi_lo(f[x] * eg, &lo);
        del_[c + x][i] = (bf16_t)lo;
      }
    }
    if (wave >= 4) {  // the gradient of the state leaving this chunk: hi / lo for the products, and to the chunk grads
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int d = rb + 8 * q4 + 4 * lh;
        const float sv[4] = {acc[4 * q4], acc[4 * q4 + 1], acc[4 * q4 + 2], acc[4 * q4 + 3]};
        store_hi_lo4(&dhh[lc][d], &dhl[lc][d], sv);
#pragma unroll
        for (int x = 0; x < 4; ++x) dh_chunks[(chunk_id * GD + d + x) * GD + cb + lc] = sv[x];
      }
    }
    __syncthreads();
    if (n > 0) fetch(n - 1);
    if (wave < 2) {  // dv_new = attn^T do + e^(gl - g) (k dH) for token rows rb ..
      f32x16 a1 = {}, a2 = {};
#pragma unroll
      for (int k0 = 0; k0 < GC; k0 += 16) {
        const int kk = k0 + 8 * lh;
        const bf16x8 qf = frag_row<KP>(&doT[0][0], lc, kk);
        a1 = mma_bf16(frag_col<KP>(&ah[0][0], rb, k0, lane), qf, a1);
        a1 = mma_bf16(frag_col<KP>(&al[0][0], rb, k0, lane), qf, a1);
      }
#pragma unroll
      for (int k0 = 0; k0 < GD; k0 += 16) {
        const int kk = k0 + 8 * lh;
        const bf16x8 pf = frag_row<GP>(&ks[0][0], rb + lc, kk);
        a2 = mma_bf16(pf, frag_row<GP>(&dhh[0][0], lc, kk), a2);
        a2 = mma_bf16(pf, frag_row<GP>(&dhl[0][0], lc, kk), a2);
      }
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int t = rb + 8 * q4 + 4 * lh;
        float nv[4];
#pragma unroll
        for (int x = 0; x < 4; ++x) nv[x] = -fmaf(ek[t + x], a2[4 * q4 + x], a1[4 * q4 + x]);
        store_hi_lo4(&dvh[lc][t], &dvl[lc][t], nv);
      }
    }
    __syncthreads();  // -dv_new is in LDS
    if (wave >= 4) {  // dH <- e^gl dH + q^T (e^g do) - w^T dv_new, K = 64
      const float el = __expf(gc[GC - 1]);
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] *= el;
      f32x16 acc2 = {};  // a second, independent MFMA chain
#pragma unroll
      for (int k0 = 0; k0 < GC; k0 += 16) {
        const int kk = k0 + 8 * lh;
        const bf16x8 pq_ = frag_col<GP>(&qs[0][0], rb, k0, lane);
        acc = mma_bf16(pq_, frag_row<KP>(&deh[0][0], lc, kk), acc);
        acc2 = mma_bf16(pq_, frag_row<KP>(&del_[0][0], lc, kk), acc2);
        const bf16x8 pw_ = frag_col<GP>(&ws[0][0], rb, k0, lane);
        acc = mma_bf16(pw_, frag_row<KP>(&dvh[0][0], lc, kk), acc);
        acc2 = mma_bf16(pw_, frag_row<KP>(&dvl[0][0], lc, kk), acc2);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] += acc2[r];
    }
  }
  if (dh0 && wave >= 4)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int d = rb + 8 * (r / 4) + 4 * lh + r % 4;
      dh0[(bh * GD + d) * GD + cb + lc] = acc[r];
    }
}

// grid (N, H, B): per chunk, the products with the saved state h_n and the scan's dH_n, streamed over the value
// columns in blocks of SB: v_new, dv_new (= du, written in bf16, the compute dtype of u), dqg, dkd, dw (bf16, the
// compute dtype of w), dP (lower incl. diagonal) and dgl.
__global__ __launch_bounds__(GTH) void gdn_bgrad_kernel(const bf16_t* __restrict__ k,
                                                        const bf16_t* __restrict__ u_in, const bf16_t* __restrict__ w_in,
                                                        const float* __restrict__ attn_in,
                                                        const float* __restrict__ gcum_in, const bf16_t* __restrict__ dout,
                                                        const float* __restrict__ h_chunks,
                                                        const float* __restrict__ dh_chunks, int T, int H,
                                                        float* __restrict__ dqg_out, float* __restrict__ dkd_out,
                                                        bf16_t* __restrict__ du_out, bf16_t* __restrict__ dw_out,
                                                        float* __restrict__ dp_out, float* __restrict__ dgl_out) {
  // On the bf16 matrix cores (f32 operands as hi / lo bf16 pairs).  Per value-column block (4 of 32): waves 0-1 form
  // v_new = u - w h for token rows 32 wave .., waves 2-3 dv_new = e^(gl - g) (k dH) + attn^T do; then every wave adds
  // the block's share (K = 32 columns) of one 32 x 32 tile each of dqg += do h^T, dkd += v_new dH^T, dw -= dv_new h^T
  // (wave w: token rows 32 (w / 4), state rows 32 (w % 4)) and waves 0-3 of dP += do v_new^T.
  constexpr int BP = SB + 8;  // pitch of the [.][SB] bf16 block tiles (80 bytes)
  __shared__ __attribute__((aligned(16))) bf16_t ks[GC][GP], ws[GC][GP];           // [t][d]
  __shared__ __attribute__((aligned(16))) bf16_t ah[GC][KP], al[GC][KP];           // attn hi / lo [j][t]
  __shared__ __attribute__((aligned(16))) bf16_t hh[GD][BP], hl[GD][BP];           // h block hi / lo [d][c]
  __shared__ __attribute__((aligned(16))) bf16_t dhh[GD][BP], dhl[GD][BP];         // dH block hi / lo [d][c]
  __shared__ __attribute__((aligned(16))) bf16_t dos[GC][BP];                      // do block [t][c]
  __shared__ __attribute__((aligned(16))) bf16_t vh[GC][BP], vl[GC][BP];           // v_new hi / lo [t][c]
  __shared__ __attribute__((aligned(16))) bf16_t dvh[GC][BP], dvl[GC][BP];         // dv_new hi / lo [t][c]
  __shared__ float gc[GC], ek[GC], red[GTH / 64];
  const int n = blockIdx.x, h = blockIdx.y, b = blockIdx.z, N = gridDim.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, t0 = n * GC;
  const int lc = lane & 31, lh = lane >> 5;
  const int64_t row0 = (int64_t)b * T;
  const int64_t chunk_id = ((int64_t)b * H + h) * N + n;
  // The setup's loads all issue before any is used (rows past T read row T - 1 and are zeroed here); the h, dH and
  // do pieces of block cb + SB load into registers while block cb computes.
  constexpr int TI = GC * (GD / 8) / GTH, HI = GD * SB / 4 / GTH;
  static_assert(TI == 2 && GC * GC / 4 / GTH == TI && HI == 2 && GC * SB / 8 <= GTH, "bgrad thread mapping");
  const float* hsrc = h_chunks + chunk_id * GD * GD;
  const float* dsrc = dh_chunks + chunk_id * GD * GD;
  f32x4 hv[HI], dv[HI];
  u32x4 dov = {0u, 0u, 0u, 0u};
  auto fetch_block = [&](int cb) {
#pragma unroll
    for (int x = 0; x < HI; ++x) {
      const int e = tid + GTH * x, d = e / (SB / 4), c = 4 * (e % (SB / 4));
      hv[x] = *reinterpret_cast<const f32x4*>(hsrc + d * GD + cb + c);
      dv[x] = *reinterpret_cast<const f32x4*>(dsrc + d * GD + cb + c);
    }
    if (tid < GC * SB / 8) {
      const int i = tid / (SB / 8), c = 8 * (tid % (SB / 8));
      dov = *reinterpret_cast<const u32x4*>(dout + ((row0 + min(t0 + i, T - 1)) * H + h) * GD + cb + c);
    }
  };
  {
    u32x4 kr[TI], wr[TI];
    f32x4 ar[TI];
#pragma unroll
    for (int x = 0; x < TI; ++x) {
      const int e = tid + GTH * x, i = e / (GD / 8), c = 8 * (e % (GD / 8));
      kr[x] = *reinterpret_cast<const u32x4*>(k + ((row0 + min(t0 + i, T - 1)) * H + h) * GD + c);
      wr[x] = *reinterpret_cast<const u32x4*>(w_in + chunk_id * GC * GD + i * GD + c);
      ar[x] = *reinterpret_cast<const f32x4*>(attn_in + chunk_id * GC * GC + 4 * e);
    }
    const float gcl = tid < GC ? gcum_in[chunk_id * GC + tid] : 0.f;
    const float gll = gcum_in[chunk_id * GC + GC - 1];
    fetch_block(0);
#pragma unroll
    for (int x = 0; x < TI; ++x) {
      const int e = tid + GTH * x, i = e / (GD / 8), c = 8 * (e % (GD / 8));
      *reinterpret_cast<u32x4*>(&ks[i][c]) = t0 + i < T ? kr[x] : u32x4{0u, 0u, 0u, 0u};
      *reinterpret_cast<u32x4*>(&ws[i][c]) = wr[x];
      const float av[4] = {ar[x][0], ar[x][1], ar[x][2], ar[x][3]};
      store_hi_lo4(&ah[(4 * e) / GC][(4 * e) % GC], &al[(4 * e) / GC][(4 * e) % GC], av);
    }
    if (tid < GC) {
      gc[tid] = gcl;
      ek[tid] = __expf(gll - gcl);
    }
  }
  const int tr = 32 * (wave / 4), dr = 32 * (wave % 4);  // this wave's tile of the [GC][GD] accumulators
  const int rb = 32 * (wave & 1);                        // token rows of the block products (waves 0-3)
  f32x16 aq = {}, ak = {}, aw = {}, ap = {};
  float gl_part = 0.f;
  for (int cb = 0; cb < GD; cb += SB) {
    __syncthreads();  // the previous block's tiles are consumed (and the setup above is done)
#pragma unroll
    for (int x = 0; x < HI; ++x) {  // h and dH blocks: hi / lo, and <dH, h>
      const int e = tid + GTH * x, d = e / (SB / 4), c = 4 * (e % (SB / 4));
      const float h4[4] = {hv[x][0], hv[x][1], hv[x][2], hv[x][3]}, d4[4] = {dv[x][0], dv[x][1], dv[x][2], dv[x][3]};
      store_hi_lo4(&hh[d][c], &hl[d][c], h4);
      store_hi_lo4(&dhh[d][c], &dhl[d][c], d4);
#pragma unroll
      for (int y = 0; y < 4; ++y) gl_part = fmaf(h4[y], d4[y], gl_part);
    }
    if (tid < GC * SB / 8) {  // do block
      const int i = tid / (SB / 8), c = 8 * (tid % (SB / 8));
      *reinterpret_cast<u32x4*>(&dos[i][c]) = t0 + i < T ? dov : u32x4{0u, 0u, 0u, 0u};
    }
    if (cb + SB < GD) fetch_block(cb + SB);
    __syncthreads();
    if (wave < 4) {
      f32x16 acc = {};
      if (wave < 2) {  // w h (K = 128)
#pragma unroll
        for (int k0 = 0; k0 < GD; k0 += 16) {
          const bf16x8 pf = frag_row<GP>(&ws[0][0], rb + lc, k0 + 8 * lh);
          acc = mma_bf16(pf, frag_col<BP>(&hh[0][0], 0, k0, lane), acc);
          acc = mma_bf16(pf, frag_col<BP>(&hl[0][0], 0, k0, lane), acc);
        }
        const bf16_t* ub = u_in + chunk_id * GC * GD + cb + lc;
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const int t = rb + 8 * q4 + 4 * lh;
          float vv[4];
#pragma unroll
          for (int x = 0; x < 4; ++x) vv[x] = bf16_to_f32(ub[(t + x) * GD]) - acc[4 * q4 + x];
          // rows t .. t + 3 of column lc: four scattered 2-byte stores each
#pragma unroll
          for (int x = 0; x < 4; ++x) {
            uint32_t lo;
            vh[t + x][lc] = (bf16_t)bf16_hi_lo(vv[x], &lo);
            vl[t + x][lc] = (bf16_t)lo;
          }
        }
      } else {  // dv_new = e^(gl - g) (k dH) + attn^T do (K = 128, then 64)
#pragma unroll
        for (int k0 = 0; k0 < GD; k0 += 16) {
          const bf16x8 pf = frag_row<GP>(&ks[0][0], rb + lc, k0 + 8 * lh);
          acc = mma_bf16(pf, frag_col<BP>(&dhh[0][0], 0, k0, lane), acc);
          acc = mma_bf16(pf, frag_col<BP>(&dhl[0][0], 0, k0, lane), acc);
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] *= ek[rb + 8 * (r / 4) + 4 * lh + r % 4];
#pragma unroll
        for (int k0 = 0; k0 < GC; k0 += 16) {
          const bf16x8 qf = frag_col<BP>(&dos[0][0], 0, k0, lane);
          acc = mma_bf16(frag_col<KP>(&ah[0][0], rb, k0, lane), qf, acc);
          acc = mma_bf16(frag_col<KP>(&al[0][0], rb, k0, lane), qf, acc);
        }
        bf16_t* dub = du_out + chunk_id * GC * GD + cb + lc;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int t = rb + 8 * (r / 4) + 4 * lh + r % 4;
          uint32_t lo;
          const bf16_t hi = (bf16_t)bf16_hi_lo(acc[r], &lo);
          dvh[t][lc] = hi;
          dvl[t][lc] = (bf16_t)lo;
          dub[t * GD] = f32_to_bf16(acc[r]);
        }
      }
    }
    __syncthreads();  // v_new and dv_new of the block are in LDS
    // this block's K = 32 share of the tile products
#pragma unroll
    for (int k0 = 0; k0 < SB; k0 += 16) {
      const int kk = k0 + 8 * lh;
      const bf16x8 dof = frag_row<BP>(&dos[0][0], tr + lc, kk);
      const bf16x8 qhh = frag_row<BP>(&hh[0][0], dr + lc, kk), qhl = frag_row<BP>(&hl[0][0], dr + lc, kk);
      aq = mma_bf16(dof, qhh, aq);
      aq = mma_bf16(dof, qhl, aq);
      const bf16x8 pvh = frag_row<BP>(&vh[0][0], tr + lc, kk), pvl = frag_row<BP>(&vl[0][0], tr + lc, kk);
      const bf16x8 qdh = frag_row<BP>(&dhh[0][0], dr + lc, kk);
      ak = mma_bf16(pvh, qdh, ak);
      ak = mma_bf16(pvh, frag_row<BP>(&dhl[0][0], dr + lc, kk), ak);
      ak = mma_bf16(pvl, qdh, ak);
      const bf16x8 pdh = frag_row<BP>(&dvh[0][0], tr + lc, kk), pdl = frag_row<BP>(&dvl[0][0], tr + lc, kk);
      aw = mma_bf16(pdh, qhh, aw);
      aw = mma_bf16(pdh, qhl, aw);
      aw = mma_bf16(pdl, qhh, aw);
      if (wave < 4) {  // dP tile: token rows 32 (wave / 2), columns 32 (wave % 2)
        const int pr = 32 * (wave / 2), pc = 32 * (wave % 2);
        const bf16x8 pdo = frag_row<BP>(&dos[0][0], pr + lc, kk);
        ap = mma_bf16(pdo, frag_row<BP>(&vh[0][0], pc + lc, kk), ap);
        ap = mma_bf16(pdo, frag_row<BP>(&vl[0][0], pc + lc, kk), ap);
      }
    }
  }
  // the tiles: lane holds rows tr + 8 (r / 4) + 4 lh + r % 4, column dr + lc
  const int64_t ob = chunk_id * GC * GD;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int i = tr + 8 * (r / 4) + 4 * lh + r % 4;
    dqg_out[ob + i * GD + dr + lc] = aq[r];
    dkd_out[ob + i * GD + dr + lc] = ak[r];
    dw_out[ob + i * GD + dr + lc] = f32_to_bf16(-aw[r]);
  }
  if (wave < 4) {
    const int pr = 32 * (wave / 2), pc = 32 * (wave % 2);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = pr + 8 * (r / 4) + 4 * lh + r % 4, j = pc + lc;
      dp_out[chunk_id * GC * GC + i * GC + j] = j <= i ? ap[r] : 0.f;
    }
  }
  // dgl = e^gl <dH, h>: wave sums, then the 8 waves in order
  float v = gl_part;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  if ((tid & 63) == 0) red[tid >> 6] = v;
  __syncthreads();
  if (tid == 0) {
    float t = 0.f;
    for (int i = 0; i < GTH / 64; ++i) t += red[i];
    dgl_out[chunk_id] = __expf(gc[GC - 1]) * t;
  }
}

// grid (N, H, B): the chunk-local backward of one chunk and the assembly of its input gradients, on the bf16 matrix
// cores (f32 operands as hi / lo bf16 pairs).  The [GC][GD] products (dq, dk, dvb, dkbg, dkb terms) take one 32 x 32
// tile per wave (token rows 32 (wave / 4), columns 32 (wave % 4)); the [GC][GC] ones (dA, X, dS) one tile per wave
// 0-3 (rows 32 (wave / 2), columns 32 (wave % 2)).  Every global load of a phase is issued before its first use, and
// the row and column sums for dgcum come from registers (lane shuffles, then per-wave partials in a fixed order).
__global__ __launch_bounds__(GTH) void gdn_bchunk_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
    const bf16_t* __restrict__ beta, const float* __restrict__ attn_in, const float* __restrict__ gcum_in,
    const float* __restrict__ s_in, const float* __restrict__ a_in, const float* __restrict__ dqg_in,
    const float* __restrict__ dkd_in, const bf16_t* __restrict__ du_in, const bf16_t* __restrict__ dw_in,
    const float* __restrict__ dp_in, const float* __restrict__ dgl_in, int T, int H, float qscale,
    bf16_t* __restrict__ dq, bf16_t* __restrict__ dk, bf16_t* __restrict__ dv, float* __restrict__ dg,
    float* __restrict__ dbeta) {
  // T1 k, T2 q * scale, T3 k beta, T4 v beta, T5 du, T6 dw (bf16 tiles); M1 / M2 scratch [GC][GC], M3 A
  __shared__ __attribute__((aligned(16))) bf16_t T1[GC][GP], T2[GC][GP], T3[GC][GP], T4[GC][GP], T5[GC][GP], T6[GC][GP];
  __shared__ float M1[GC][GC + 1], M2[GC][GC + 1], M3[GC][GC + 1];
  __shared__ float gc[GC], eg[GC], bt[GC];
  __shared__ float rs1[GC], cs1[GTH / 64][GC];     // dP . P: row sums; column sums of each wave's rows
  __shared__ float rs2[2][GC], cs2[2][GC];         // dS . S: row sums of the two column tiles, column sums of the two row tiles
  __shared__ float rowp[2][GD / 32][GC];           // dgcum and dbeta terms: row sums of the four [GC][GD] column tiles
  __shared__ float glw[GTH / 64];
  constexpr int TI = GC * (GD / 8) / GTH;          // u32x4 of a bf16 [GC][GD] tile per thread
  static_assert(TI == 2 && GC * GC / 4 / GTH == TI && GD == 128 && GTH == 512, "thread mapping of the prologue");
  const int n = blockIdx.x, h = blockIdx.y, b = blockIdx.z, N = gridDim.x;
  const int tid = threadIdx.x, t0 = n * GC;
  const int lane = tid & 63, wave = tid >> 6, lc = lane & 31, lh = lane >> 5;
  const int64_t row0 = (int64_t)b * T;
  const int64_t chunk_id = ((int64_t)b * H + h) * N + n;
  const int64_t mo = chunk_id * GC * GC, to = chunk_id * GC * GD;
  const int ti = 32 * (wave >> 2), cd = 32 * (wave & 3);        // [GC][GD] tile of this wave
  const int pi = 32 * ((wave & 3) >> 1), pj = 32 * (wave & 1);  // [GC][GC] tile (waves 0-3)
  // prologue loads: rows tid / 16 + 32 x, bf16 columns 8 (tid % 16), f32 columns 4 (tid % 16)
  const int cq = 8 * (tid & 15), cm = 4 * (tid & 15);
  // Rows past T (the last chunk's tail) read row T - 1 and are zeroed where the values are used, so every load is
  // unconditional and none waits for another.
  u32x4 kr[TI], qr[TI], vr[TI], ur[TI], wr[TI];
  f32x4 dpr[TI], pr[TI], ar[TI];
  bf16_t bir[TI];
#pragma unroll
  for (int x = 0; x < TI; ++x) {
    const int i = (tid >> 4) + 32 * x;
    const int64_t tr = row0 + min(t0 + i, T - 1);
    const int64_t go = (tr * H + h) * GD + cq;
    kr[x] = *reinterpret_cast<const u32x4*>(k + go);
    qr[x] = *reinterpret_cast<const u32x4*>(q + go);
    vr[x] = *reinterpret_cast<const u32x4*>(v + go);
    bir[x] = beta[tr * H + h];
    ur[x] = *reinterpret_cast<const u32x4*>(du_in + to + i * GD + cq);
    wr[x] = *reinterpret_cast<const u32x4*>(dw_in + to + i * GD + cq);
    dpr[x] = *reinterpret_cast<const f32x4*>(dp_in + mo + i * GC + cm);
    pr[x] = *reinterpret_cast<const f32x4*>(attn_in + mo + i * GC + cm);
    ar[x] = *reinterpret_cast<const f32x4*>(a_in + mo + i * GC + cm);
  }
  float gcl = 0.f;
  bf16_t btr = 0;
  if (tid < GC) {
    gcl = gcum_in[chunk_id * GC + tid];
    btr = beta[(row0 + min(t0 + tid, T - 1)) * H + h];
  }
  float sv[16];  // S in the [GC][GC] tile layout (waves 0-3), for dS . S
  if (wave < 4)
#pragma unroll
    for (int r = 0; r < 16; ++r) sv[r] = s_in[mo + (pi + 8 * (r / 4) + 4 * lh + r % 4) * GC + pj + lc];
  if (tid < GC) {
    gc[tid] = gcl;
    eg[tid] = __expf(gcl);
    bt[tid] = t0 + tid < T ? bf16_to_f32(btr) : 0.f;
  }
  // k, q * scale (gdn_fast.py:56-57), k beta and v beta in the compute dtype (gdn_fast.py:78, 87), du, dw, A
#pragma unroll
  for (int x = 0; x < TI; ++x) {
    const int i = (tid >> 4) + 32 * x;
    if (t0 + i >= T) kr[x] = qr[x] = vr[x] = u32x4{0u, 0u, 0u, 0u};
    float kf[8], qf[8], vf[8];
    unpack8g(kr[x], kf);
    unpack8g(qr[x], qf);
    unpack8g(vr[x], vf);
    const float bi = t0 + i < T ? bf16_to_f32(bir[x]) : 0.f;
#pragma unroll
    for (int y = 0; y < 8; ++y) {
      qf[y] *= qscale;
      vf[y] *= bi;
      kf[y] *= bi;
    }
    *reinterpret_cast<u32x4*>(&T1[i][cq]) = kr[x];
    *reinterpret_cast<u32x4*>(&T2[i][cq]) = __builtin_bit_cast(u32x4, pack8(qf));
    *reinterpret_cast<u32x4*>(&T3[i][cq]) = __builtin_bit_cast(u32x4, pack8(kf));
    *reinterpret_cast<u32x4*>(&T4[i][cq]) = __builtin_bit_cast(u32x4, pack8(vf));
    *reinterpret_cast<u32x4*>(&T5[i][cq]) = ur[x];
    *reinterpret_cast<u32x4*>(&T6[i][cq]) = wr[x];
#pragma unroll
    for (int y = 0; y < 4; ++y) M3[i][cm + y] = ar[x][y];
  }
  // dP . P: its row sums less its column sums go to dgcum
  {
    float cs[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int x = 0; x < TI; ++x) {
      float r = 0.f;
#pragma unroll
      for (int y = 0; y < 4; ++y) {
        const float m = dpr[x][y] * pr[x][y];
        r += m;
        cs[y] += m;
      }
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) r += __shfl_xor(r, o, 64);
      if ((tid & 15) == 0) rs1[(tid >> 4) + 32 * x] = r;
    }
#pragma unroll
    for (int y = 0; y < 4; ++y) {
      cs[y] += __shfl_xor(cs[y], 16, 64);
      cs[y] += __shfl_xor(cs[y], 32, 64);
    }
    if (lane < 16)
#pragma unroll
      for (int y = 0; y < 4; ++y) cs1[wave][cm + y] = cs[y];
  }
  __syncthreads();
  // dP_r = dP . Gi (Gi = e^(gcum_i - gcum_j), lower incl. diagonal)
#pragma unroll
  for (int x = 0; x < TI; ++x) {
    const int i = (tid >> 4) + 32 * x;
    const float gi = gc[i];
#pragma unroll
    for (int y = 0; y < 4; ++y) {
      const int j = cm + y;
      const float e = __expf(gi - gc[j]);
      M2[i][j] = j <= i ? dpr[x][y] * e : 0.f;
    }
  }
  // dA = du vb^T + dw kbg^T (kbg = kb e^gcum), K = 128
  f32x16 da1 = {}, da2 = {};
  if (wave < 4) {
#pragma unroll
    for (int k0 = 0; k0 < GD; k0 += 16) {
      const int kk = k0 + 8 * lh;
      da1 = mma_bf16(frag_row<GP>(&T5[0][0], pi + lc, kk), frag_row<GP>(&T4[0][0], pj + lc, kk), da1);
      da2 = mma_bf16(frag_row<GP>(&T6[0][0], pi + lc, kk), frag_row<GP>(&T3[0][0], pj + lc, kk), da2);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) M1[pi + 8 * (r / 4) + 4 * lh + r % 4][pj + lc] = fmaf(eg[pj + lc], da2[r], da1[r]);
  }
  __syncthreads();
  const float gl = gc[GC - 1];
  // dq = dP_r k (+ dqg e^gcum in the epilogue); dk = dP_r^T q (+ dkd e^(gl - gcum) and the chunk-local terms), K = 64
  f32x16 aq = {}, ak = {};
#pragma unroll
  for (int k0 = 0; k0 < GC; k0 += 16) {
    const int kk = k0 + 8 * lh;
    bf16x8 ph, pl;
    frag_rowf(M2, ti + lc, kk, ph, pl);
    const bf16x8 qk = frag_col<GP>(&T1[0][0], cd, k0, lane);
    aq = mma_bf16(ph, qk, aq);
    aq = mma_bf16(pl, qk, aq);
    frag_colf(M2, ti + lc, kk, ph, pl);
    const bf16x8 qq = frag_col<GP>(&T2[0][0], cd, k0, lane);
    ak = mma_bf16(ph, qq, ak);
    ak = mma_bf16(pl, qq, ak);
  }
  // X = A^T dA, K = 64
  f32x16 xa = {};
  if (wave < 4)
#pragma unroll
    for (int k0 = 0; k0 < GC; k0 += 16) {
      const int kk = k0 + 8 * lh;
      bf16x8 ph, pl, qh, ql;
      frag_colf(M3, pi + lc, kk, ph, pl);
      frag_colf(M1, pj + lc, kk, qh, ql);
      xa = mma_bf16(ph, qh, xa);
      xa = mma_bf16(ph, ql, xa);
      xa = mma_bf16(pl, qh, xa);
    }
  __syncthreads();  // dP_r (M2) and dA (M1) are read
  if (wave < 4)
#pragma unroll
    for (int r = 0; r < 16; ++r) M2[pi + 8 * (r / 4) + 4 * lh + r % 4][pj + lc] = xa[r];
  __syncthreads();
  // dS = -(X A^T), strictly lower, K = 64; dS0 = dS . Gs -> M1; row and column sums of dS . S for dgcum
  if (wave < 4) {
    xa = f32x16{};
#pragma unroll
    for (int k0 = 0; k0 < GC; k0 += 16) {
      const int kk = k0 + 8 * lh;
      bf16x8 ph, pl, qh, ql;
      frag_rowf(M2, pi + lc, kk, ph, pl);
      frag_rowf(M3, pj + lc, kk, qh, ql);
      xa = mma_bf16(ph, qh, xa);
      xa = mma_bf16(ph, ql, xa);
      xa = mma_bf16(pl, qh, xa);
    }
    const int j = pj + lc;
    const float gj = gc[j];
    float cs = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = pi + 8 * (r / 4) + 4 * lh + r % 4;
      const float ds = j < i ? -xa[r] : 0.f;
      const float e = __expf(gc[i] - gj);
      M1[i][j] = j < i ? ds * e : 0.f;
      float t = ds * sv[r];
      cs += t;
#pragma unroll
      for (int o = 1; o < 32; o <<= 1) t += __shfl_xor(t, o, 64);
      if (lc == 0) rs2[wave & 1][i] = t;
    }
    cs += __shfl_xor(cs, 32, 64);
    if (lh == 0) cs2[wave >> 1][j] = cs;
  }
  // epilogue loads, in flight during the products below
  float gqv[16], gkv[16];
  bf16_t v1v[16];  // raw, converted (and zeroed past T) where used
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int i = ti + 8 * (r / 4) + 4 * lh + r % 4, c = cd + lc;
    gqv[r] = dqg_in[to + i * GD + c];
    gkv[r] = dkd_in[to + i * GD + c];
    v1v[r] = v[((row0 + min(t0 + i, T - 1)) * H + h) * GD + c];
  }
  __syncthreads();
  // dvb = A^T du, dkbg = A^T dw; dkb = dkbg e^gcum + dS0 k; dk += dS0^T kb, K = 64
  f32x16 avb = {}, akg = {}, akb = {};
#pragma unroll
  for (int k0 = 0; k0 < GC; k0 += 16) {
    const int kk = k0 + 8 * lh;
    bf16x8 ph, pl;
    frag_colf(M3, ti + lc, kk, ph, pl);  // A^T
    const bf16x8 qu = frag_col<GP>(&T5[0][0], cd, k0, lane), qw = frag_col<GP>(&T6[0][0], cd, k0, lane);
    avb = mma_bf16(ph, qu, avb);
    avb = mma_bf16(pl, qu, avb);
    akg = mma_bf16(ph, qw, akg);
    akg = mma_bf16(pl, qw, akg);
    frag_rowf(M1, ti + lc, kk, ph, pl);  // dS0
    const bf16x8 qk = frag_col<GP>(&T1[0][0], cd, k0, lane);
    akb = mma_bf16(ph, qk, akb);
    akb = mma_bf16(pl, qk, akb);
    frag_colf(M1, ti + lc, kk, ph, pl);  // dS0^T
    const bf16x8 qb = frag_col<GP>(&T3[0][0], cd, k0, lane);
    ak = mma_bf16(ph, qb, ak);
    ak = mma_bf16(pl, qb, ak);
  }
  float dgr[16], dbr[16], dgl_rows = 0.f;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int i = ti + 8 * (r / 4) + 4 * lh + r % 4, c = cd + lc;
    const float gq = gqv[r], gk = gkv[r];
    const float k1 = bf16_to_f32(T1[i][c]), kb1 = bf16_to_f32(T3[i][c]);
    const float e = eg[i], ed = __expf(gl - gc[i]), bi = bt[i];
    aq[r] = fmaf(gq, e, aq[r]);
    ak[r] = fmaf(gk, ed, ak[r]);
    const float s2 = gk * k1 * ed;              // <dkd, kd>: - to row i, + to gl
    dgl_rows += s2;
    const float dkb = fmaf(akg[r], e, akb[r]);  // dkbg e^gcum + dS0 k
    dgr[r] = fmaf(akg[r], kb1 * e, fmaf(gq, bf16_to_f32(T2[i][c]) * e, -s2));  // <dkbg, kbg> + <dqg, qg> - s2
    dbr[r] = fmaf(avb[r], t0 + i < T ? bf16_to_f32(v1v[r]) : 0.f, dkb * k1);
    if (t0 + i < T) {
      const int64_t off = ((row0 + t0 + i) * H + h) * GD + c;
      dq[off] = f32_to_bf16(aq[r] * qscale);
      dk[off] = f32_to_bf16(fmaf(dkb, bi, ak[r]));
      dv[off] = f32_to_bf16(avb[r] * bi);
    }
  }
  // per-row sums: over the 32 columns of this lane group (xor butterfly), then the four column tiles in order
#pragma unroll
  for (int r = 0; r < 16; ++r) {
#pragma unroll
    for (int o = 1; o < 32; o <<= 1) {
      dgr[r] += __shfl_xor(dgr[r], o, 64);
      dbr[r] += __shfl_xor(dbr[r], o, 64);
    }
  }
  if (lc == 0)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = ti + 8 * (r / 4) + 4 * lh + r % 4;
      rowp[0][wave & 3][i] = dgr[r];
      rowp[1][wave & 3][i] = dbr[r];
    }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) dgl_rows += __shfl_xor(dgl_rows, o, 64);
  if (lane == 0) glw[wave] = dgl_rows;
  __syncthreads();
  if (tid < GC) {  // dgcum of row tid, then dg = its suffix sum over the chunk (gcum = cumsum(g)), one wave
    float x = rs1[tid] + (rs2[0][tid] + rs2[1][tid]) - (cs2[0][tid] + cs2[1][tid]);
    float c1 = 0.f, dbrow = 0.f;
#pragma unroll
    for (int w = 0; w < GTH / 64; ++w) c1 += cs1[w][tid];
    x -= c1;
#pragma unroll
    for (int w = 0; w < GD / 32; ++w) {
      x += rowp[0][w][tid];
      dbrow += rowp[1][w][tid];
    }
    if (tid == GC - 1) {
      float t = dgl_in[chunk_id];
      for (int w = 0; w < GTH / 64; ++w) t += glw[w];
      x += t;
    }
#pragma unroll
    for (int o = 1; o < GC; o <<= 1) {
      const float y = __shfl_down(x, o, 64);
      if (tid + o < GC) x += y;
    }
    const int t = t0 + tid;
    if (t < T) {
      dg[(row0 + t) * H + h] = x;
      dbeta[(row0 + t) * H + h] = dbrow;
    }
  }
}

// Row-wise l2 normalisation of the GDN block's query and key heads (use_qk_norm_in_gdn, gdn_fast.py:43-46, MaxText's
// l2norm): y = x rsqrt(sum x^2 + eps), bf16 in and out, f32 arithmetic.  LPR = dim / 8 lanes per row (rounded up to
// a power of two), each holding 8 consecutive elements; the row sum is a butterfly over those lanes.  rnorm keeps
// rsqrt(sum x^2 + eps) per row for the backward: dx = r dy - r^3 x (x . dy).
template <int LPR>
__global__ __launch_bounds__(256) void l2norm_rows_kernel(const bf16_t* __restrict__ x, int64_t rows, int dim,
                                                          float eps, bf16_t* __restrict__ y, float* __restrict__ rnorm) {
  const int64_t row = (int64_t)blockIdx.x * (256 / LPR) + threadIdx.x / LPR;
  const int part = threadIdx.x % LPR, c = 8 * part;
  const bool ok = row < rows && c < dim;
  float f[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (ok) unpack8g(*reinterpret_cast<const u32x4*>(x + row * dim + c), f);
  float sq = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) sq = fmaf(f[i], f[i], sq);
#pragma unroll
  for (int o = 1; o < LPR; o <<= 1) sq += __shfl_xor(sq, o, 64);
  const float r = 1.f / sqrtf(sq + eps);
  if (ok) {
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] *= r;
    *reinterpret_cast<u32x4*>(y + row * dim + c) = __builtin_bit_cast(u32x4, pack8(f));
    if (part == 0 && rnorm) rnorm[row] = r;
  }
}
template <int LPR>
__global__ __launch_bounds__(256) void l2norm_rows_bwd_kernel(const bf16_t* __restrict__ x, const bf16_t* __restrict__ dy,
                                                              const float* __restrict__ rnorm, int64_t rows, int dim,
                                                              bf16_t* __restrict__ dx) {
  const int64_t row = (int64_t)blockIdx.x * (256 / LPR) + threadIdx.x / LPR;
  const int part = threadIdx.x % LPR, c = 8 * part;
  const bool ok = row < rows && c < dim;
  float xf[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, gf[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float r = 0.f;
  if (ok) {
    unpack8g(*reinterpret_cast<const u32x4*>(x + row * dim + c), xf);
    unpack8g(*reinterpret_cast<const u32x4*>(dy + row * dim + c), gf);
    r = rnorm[row];
  }
  float dot = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) dot = fmaf(xf[i], gf[i], dot);
#pragma unroll
  for (int o = 1; o < LPR; o <<= 1) dot += __shfl_xor(dot, o, 64);
  if (ok) {
    const float r3d = r * r * r * dot;
#pragma unroll
    for (int i = 0; i < 8; ++i) xf[i] = fmaf(r, gf[i], -r3d * xf[i]);
    *reinterpret_cast<u32x4*>(dx + row * dim + c) = __builtin_bit_cast(u32x4, pack8(xf));
  }
}

int64_t gdn_chunks(int64_t t) { return (t + GC - 1) / GC; }

// f32 -> bf16 -> f32 on the host, round to nearest even (finite inputs)
float round_bf16_host(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  u = (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
  memcpy(&f, &u, 4);
  return f;
}

}  // namespace

extern "C" {

size_t lsurge_gdn_chunked_workspace_bytes(int64_t b, int64_t t, int64_t h, int64_t dk, int64_t dv) {
  if (b < 1 || t < 1 || h < 1 || dk != GD || dv != GD) return 0;
  const size_t chunks = (size_t)(b * h * gdn_chunks(t));
  return chunks * ((size_t)2 * GC * GD * sizeof(bf16_t) + (size_t)GC * GC * sizeof(float) + GC * sizeof(float)) + 1024;
}

int lsurge_gdn_chunked_fwd(const void* q, const void* k, const void* v, const float* g, const void* beta, int64_t b,
                           int64_t t, int64_t h, int64_t dk, int64_t dv, const float* h0, void* o, float* h_out,
                           void* workspace, size_t workspace_bytes, lsurge_stream_t stream) {
  LSURGE_REQUIRE(q && k && v && g && beta && o && workspace, "gdn_chunked_fwd: null pointer");
  LSURGE_REQUIRE(dk == GD && dv == GD, "gdn_chunked_fwd: head dims dk=%lld dv=%lld must be %d", (long long)dk,
                 (long long)dv, GD);
  LSURGE_REQUIRE(b >= 1 && b < 65536 && h >= 1 && h < 65536 && t >= 1 && b * t * h < (1ll << 31) / GD &&
                     gdn_chunks(t) < (1ll << 31),
                 "gdn_chunked_fwd: bad shape b=%lld t=%lld h=%lld", (long long)b, (long long)t, (long long)h);
  LSURGE_REQUIRE(((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)o | (uintptr_t)workspace) % 16 == 0,
                 "gdn_chunked_fwd: q, k, v, o and workspace must be 16-byte aligned");
  const size_t need = lsurge_gdn_chunked_workspace_bytes(b, t, h, dk, dv);
  LSURGE_REQUIRE(workspace_bytes >= need, "gdn_chunked_fwd: workspace %zu < %zu bytes", workspace_bytes, need);
  hipStream_t s = (hipStream_t)stream;
  const int64_t N = gdn_chunks(t), chunks = b * h * N;
  char* p = (char*)workspace;
  bf16_t* u = (bf16_t*)p;
  bf16_t* w = u + chunks * GC * GD;
  float* attn = (float*)(w + chunks * GC * GD);
  float* gcum = attn + chunks * GC * GC;
  const float qscale = round_bf16_host(1.f / sqrtf((float)GD));  // the scale in the compute dtype (gdn_fast.py:56)
  LSURGE_LAUNCH(KID_GDN_CHUNK, s,
                hipLaunchKernelGGL(gdn_chunk_kernel, dim3((unsigned)N, (unsigned)h, (unsigned)b), dim3(GTH), 0, s,
                                   (const bf16_t*)q, (const bf16_t*)k, (const bf16_t*)v, g, (const bf16_t*)beta, (int)t,
                                   (int)h, qscale, u, w, attn, gcum));
  LSURGE_LAUNCH(KID_GDN_SCAN, s,
                hipLaunchKernelGGL(gdn_scan_kernel, dim3(GD / SB, (unsigned)h, (unsigned)b), dim3(GTH), 0, s,
                                   (const bf16_t*)q, (const bf16_t*)k, (const bf16_t*)u, (const bf16_t*)w,
                                   (const float*)attn, (const float*)gcum, (int)t, (int)h, (int)N, qscale, h0,
                                   (bf16_t*)o, h_out));
  return LSURGE_OK;
}

// workspace of the backward: the forward's residuals -- its chunk products (u, w, attn, gcum) plus S, A and the state
// entering each chunk -- then the backward's scratch: the reverse scan's state gradients and the chunk gradients (dqg,
// dkd f32; du, dw bf16; dP, dgl).  The two parts can live in separate buffers (lsurge_gdn_chunked_fwd_save keeps the
// first between the passes).
struct GdnBwdWs {
  bf16_t *u, *w, *du, *dw;
  float *attn, *gcum, *S, *A, *hs, *dhs, *dqg, *dkd, *dP, *dgl;
};
struct Carver {
  char* base;
  size_t off = 0;
  char* take(size_t bytes) {
    char* r = base ? base + off : nullptr;
    off += (bytes + 255) / 256 * 256;
    return r;
  }
};
static size_t gdn_carve_saved(int64_t chunks, void* base, GdnBwdWs* p) {
  Carver c{(char*)base};
  const size_t tile16 = (size_t)chunks * GC * GD * sizeof(bf16_t), mat = (size_t)chunks * GC * GC * sizeof(float);
  p->u = (bf16_t*)c.take(tile16);
  p->w = (bf16_t*)c.take(tile16);
  p->attn = (float*)c.take(mat);
  p->gcum = (float*)c.take((size_t)chunks * GC * sizeof(float));
  p->S = (float*)c.take(mat);
  p->A = (float*)c.take(mat);
  p->hs = (float*)c.take((size_t)chunks * GD * GD * sizeof(float));
  return c.off;
}
static size_t gdn_carve_scratch(int64_t chunks, void* base, GdnBwdWs* p) {
  Carver c{(char*)base};
  const size_t tile16 = (size_t)chunks * GC * GD * sizeof(bf16_t), tile32 = (size_t)chunks * GC * GD * sizeof(float);
  p->du = (bf16_t*)c.take(tile16);
  p->dw = (bf16_t*)c.take(tile16);
  p->dhs = (float*)c.take((size_t)chunks * GD * GD * sizeof(float));
  p->dqg = (float*)c.take(tile32);
  p->dkd = (float*)c.take(tile32);
  p->dP = (float*)c.take((size_t)chunks * GC * GC * sizeof(float));
  p->dgl = (float*)c.take((size_t)chunks * sizeof(float));
  return c.off;
}
// both parts in one buffer (the recomputing backward)
static size_t gdn_bwd_carve(int64_t chunks, void* base, GdnBwdWs* p) {
  const size_t a = gdn_carve_saved(chunks, base, p);
  return a + gdn_carve_scratch(chunks, base ? (char*)base + a : nullptr, p);
}

size_t lsurge_gdn_chunked_bwd_workspace_bytes(int64_t b, int64_t t, int64_t h, int64_t dk, int64_t dv) {
  if (b < 1 || t < 1 || h < 1 || dk != GD || dv != GD) return 0;
  GdnBwdWs p;
  return gdn_bwd_carve(b * h * gdn_chunks(t), nullptr, &p);
}
size_t lsurge_gdn_chunked_saved_bytes(int64_t b, int64_t t, int64_t h, int64_t dk, int64_t dv) {
  if (b < 1 || t < 1 || h < 1 || dk != GD || dv != GD) return 0;
  GdnBwdWs p;
  return gdn_carve_saved(b * h * gdn_chunks(t), nullptr, &p);
}
size_t lsurge_gdn_chunked_bwd_saved_workspace_bytes(int64_t b, int64_t t, int64_t h, int64_t dk, int64_t dv) {
  if (b < 1 || t < 1 || h < 1 || dk != GD || dv != GD) return 0;
  GdnBwdWs p;
  return gdn_carve_scratch(b * h * gdn_chunks(t), nullptr, &p);
}

// The backward's launches after the forward's chunk products and states are in the workspace: the reverse scan of
// the state gradient, then the chunk gradients and the chunk-local backward.
static int gdn_bwd_from_ws(const void* q, const void* k, const void* v, const void* beta, int64_t b, int64_t t,
                           int64_t h, const void* dout, const float* dh_final, void* dq, void* dk_out, void* dv_out,
                           float* dg, float* dbeta, float* dh0, const GdnBwdWs& p, hipStream_t s) {
  const int64_t N = gdn_chunks(t);
  const float qscale = round_bf16_host(1.f / sqrtf((float)GD));
  const dim3 chunk_grid((unsigned)N, (unsigned)h, (unsigned)b), scan_grid(GD / SB, (unsigned)h, (unsigned)b);
  LSURGE_LAUNCH(KID_GDN_BSCAN, s,
                hipLaunchKernelGGL(gdn_bscan_kernel, scan_grid, dim3(GTH), 0, s, (const bf16_t*)q, (const bf16_t*)k,
                                   (const bf16_t*)p.w, (const float*)p.attn, (const float*)p.gcum, (const bf16_t*)dout,
                                   (int)t, (int)h, (int)N, qscale, dh_final, p.dhs, dh0));
  LSURGE_LAUNCH(KID_GDN_BGRAD, s,
                hipLaunchKernelGGL(gdn_bgrad_kernel, chunk_grid, dim3(GTH), 0, s, (const bf16_t*)k,
                                   (const bf16_t*)p.u, (const bf16_t*)p.w, (const float*)p.attn, (const float*)p.gcum,
                                   (const bf16_t*)dout, (const float*)p.hs, (const float*)p.dhs, (int)t, (int)h, p.dqg,
                                   p.dkd, p.du, p.dw, p.dP, p.dgl));
  LSURGE_LAUNCH(KID_GDN_BCHUNK, s,
                hipLaunchKernelGGL(gdn_bchunk_kernel, chunk_grid, dim3(GTH), 0, s, (const bf16_t*)q, (const bf16_t*)k,
                                   (const bf16_t*)v, (const bf16_t*)beta, (const float*)p.attn, (const float*)p.gcum,
                                   (const float*)p.S, (const float*)p.A, (const float*)p.dqg, (const float*)p.dkd,
                                   (const bf16_t*)p.du, (const bf16_t*)p.dw, (const float*)p.dP, (const float*)p.dgl,
                                   (int)t, (int)h, qscale, (bf16_t*)dq, (bf16_t*)dk_out, (bf16_t*)dv_out, dg, dbeta));
  return LSURGE_OK;
}

// The forward's chunk products (with S and A) and, with o, its output as well, into the backward's workspace; the
// scan stores the state entering every chunk.
static int gdn_fwd_to_ws(const void* q, const void* k, const void* v, const float* g, const void* beta, int64_t b,
                         int64_t t, int64_t h, const float* h0, void* o, float* h_out, const GdnBwdWs& p, hipStream_t s) {
  const int64_t N = gdn_chunks(t);
  const float qscale = round_bf16_host(1.f / sqrtf((float)GD));
  const dim3 chunk_grid((unsigned)N, (unsigned)h, (unsigned)b), scan_grid(GD / SB, (unsigned)h, (unsigned)b);
  LSURGE_LAUNCH(KID_GDN_CHUNK, s,
                hipLaunchKernelGGL(gdn_chunk_kernel, chunk_grid, dim3(GTH), 0, s, (const bf16_t*)q, (const bf16_t*)k,
                                   (const bf16_t*)v, g, (const bf16_t*)beta, (int)t, (int)h, qscale, p.u, p.w, p.attn,
                                   p.gcum, p.S, p.A));
  LSURGE_LAUNCH(KID_GDN_SCAN, s,
                hipLaunchKernelGGL(gdn_scan_kernel, scan_grid, dim3(GTH), 0, s, (const bf16_t*)q, (const bf16_t*)k,
                                   (const bf16_t*)p.u, (const bf16_t*)p.w, (const float*)p.attn, (const float*)p.gcum,
                                   (int)t, (int)h, (int)N, qscale, h0, (bf16_t*)o, h_out, p.hs));
  return LSURGE_OK;
}

#define GDN_BWD_SHAPE_CHECKS(NAME)                                                                                     \
  LSURGE_REQUIRE(dk == GD && dv == GD, NAME ": head dims dk=%lld dv=%lld must be %d", (long long)dk, (long long)dv,   \
                 GD);                                                                                                  \
  LSURGE_REQUIRE(b >= 1 && b < 65536 && h >= 1 && h < 65536 && t >= 1 && b * t * h < (1ll << 31) / GD &&              \
                     b * h * gdn_chunks(t) < (1ll << 31) / (GD * GD),                                                  \
                 NAME ": bad shape b=%lld t=%lld h=%lld", (long long)b, (long long)t, (long long)h)

int lsurge_gdn_chunked_bwd(const void* q, const void* k, const void* v, const float* g, const void* beta, int64_t b,
                           int64_t t, int64_t h, int64_t dk, int64_t dv, const float* h0, const void* dout,
                           const float* dh_final, void* dq, void* dk_out, void* dv_out, float* dg, float* dbeta,
                           float* dh0, void* workspace, size_t workspace_bytes, lsurge_stream_t stream) {
  LSURGE_REQUIRE(q && k && v && g && beta && dout && dq && dk_out && dv_out && dg && dbeta && workspace,
                 "gdn_chunked_bwd: null pointer");
  GDN_BWD_SHAPE_CHECKS("gdn_chunked_bwd");
  LSURGE_REQUIRE(((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)dout | (uintptr_t)dq | (uintptr_t)dk_out |
                  (uintptr_t)dv_out | (uintptr_t)workspace) % 16 == 0,
                 "gdn_chunked_bwd: q, k, v, do, dq, dk, dv and workspace must be 16-byte aligned");
  const size_t need = lsurge_gdn_chunked_bwd_workspace_bytes(b, t, h, dk, dv);
  LSURGE_REQUIRE(workspace_bytes >= need, "gdn_chunked_bwd: workspace %zu < %zu bytes", workspace_bytes, need);
  hipStream_t s = (hipStream_t)stream;
  GdnBwdWs p;
  gdn_bwd_carve(b * h * gdn_chunks(t), workspace, &p);
  // forward recompute: chunk products (with S and A) and the state entering every chunk (no output)
  const int rc = gdn_fwd_to_ws(q, k, v, g, beta, b, t, h, h0, nullptr, nullptr, p, s);
  if (rc != LSURGE_OK) return rc;
  return gdn_bwd_from_ws(q, k, v, beta, b, t, h, dout, dh_final, dq, dk_out, dv_out, dg, dbeta, dh0, p, s);
}

int lsurge_gdn_chunked_fwd_save(const void* q, const void* k, const void* v, const float* g, const void* beta, int64_t b,
                                int64_t t, int64_t h, int64_t dk, int64_t dv, const float* h0, void* o, float* h_out,
                                void* saved, size_t saved_bytes, lsurge_stream_t stream) {
  LSURGE_REQUIRE(q && k && v && g && beta && o && saved, "gdn_chunked_fwd_save: null pointer");
  GDN_BWD_SHAPE_CHECKS("gdn_chunked_fwd_save");
  LSURGE_REQUIRE(((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)o | (uintptr_t)saved) % 16 == 0,
                 "gdn_chunked_fwd_save: q, k, v, o and saved must be 16-byte aligned");
  const size_t need = lsurge_gdn_chunked_saved_bytes(b, t, h, dk, dv);
  LSURGE_REQUIRE(saved_bytes >= need, "gdn_chunked_fwd_save: saved buffer %zu < %zu bytes", saved_bytes, need);
  GdnBwdWs p;
  gdn_carve_saved(b * h * gdn_chunks(t), saved, &p);
  return gdn_fwd_to_ws(q, k, v, g, beta, b, t, h, h0, o, h_out, p, (hipStream_t)stream);
}

int lsurge_gdn_chunked_bwd_saved(const void* q, const void* k, const void* v, const void* beta, int64_t b, int64_t t,
                                 int64_t h, int64_t dk, int64_t dv, const void* dout, const float* dh_final, void* dq,
                                 void* dk_out, void* dv_out, float* dg, float* dbeta, float* dh0, const void* saved,
                                 size_t saved_bytes, void* workspace, size_t workspace_bytes, lsurge_stream_t stream) {
  LSURGE_REQUIRE(q && k && v && beta && dout && dq && dk_out && dv_out && dg && dbeta && saved && workspace,
                 "gdn_chunked_bwd_saved: null pointer");
  GDN_BWD_SHAPE_CHECKS("gdn_chunked_bwd_saved");
  LSURGE_REQUIRE(((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)dout | (uintptr_t)dq | (uintptr_t)dk_out |
                  (uintptr_t)dv_out | (uintptr_t)saved | (uintptr_t)workspace) % 16 == 0,
                 "gdn_chunked_bwd_saved: q, k, v, do, dq, dk, dv, saved and workspace must be 16-byte aligned");
  const size_t need = lsurge_gdn_chunked_saved_bytes(b, t, h, dk, dv);
  LSURGE_REQUIRE(saved_bytes >= need, "gdn_chunked_bwd_saved: saved buffer %zu < %zu bytes", saved_bytes, need);
  const size_t need_ws = lsurge_gdn_chunked_bwd_saved_workspace_bytes(b, t, h, dk, dv);
  LSURGE_REQUIRE(workspace_bytes >= need_ws, "gdn_chunked_bwd_saved: workspace %zu < %zu bytes", workspace_bytes,
                 need_ws);
  GdnBwdWs p;
  const int64_t chunks = b * h * gdn_chunks(t);
  gdn_carve_saved(chunks, const_cast<void*>(saved), &p);  // read only here
  gdn_carve_scratch(chunks, workspace, &p);
  return gdn_bwd_from_ws(q, k, v, beta, b, t, h, dout, dh_final, dq, dk_out, dv_out, dg, dbeta, dh0, p,
                         (hipStream_t)stream);
}
#undef GDN_BWD_SHAPE_CHECKS

int lsurge_l2norm_rows(const void* x, int64_t rows, int64_t dim, float eps, void* y, float* rnorm,
                       lsurge_stream_t stream) {
  LSURGE_REQUIRE(x && y, "l2norm_rows: null pointer");
  LSURGE_REQUIRE(rows >= 0 && rows < (1ll << 31) && dim >= 8 && dim <= 512 && dim % 8 == 0 && eps >= 0.f,
                 "l2norm_rows: rows=%lld dim=%lld eps=%g (rows < 2^31, dim a multiple of 8 in [8, 512], eps >= 0)", (long long)rows,
                 (long long)dim, (double)eps);
  LSURGE_REQUIRE(((uintptr_t)x | (uintptr_t)y) % 16 == 0, "l2norm_rows: x and y must be 16-byte aligned");
  if (rows == 0) return LSURGE_OK;
  hipStream_t s = (hipStream_t)stream;
  const int lpr = dim <= 64 ? 8 : dim <= 128 ? 16 : dim <= 256 ? 32 : 64;
  const dim3 grid((unsigned)((rows + 256 / lpr - 1) / (256 / lpr)));
#define L2_CASE(LPR)                                                                                             \
  LSURGE_LAUNCH(KID_MISC, s,                                                                                     \
                hipLaunchKernelGGL(l2norm_rows_kernel<LPR>, grid, dim3(256), 0, s, (const bf16_t*)x, rows, (int)dim, \
                                   eps, (bf16_t*)y, rnorm))
  if (lpr == 8) L2_CASE(8);
  else if (lpr == 16) L2_CASE(16);
  else if (lpr == 32) L2_CASE(32);
  else L2_CASE(64);
#undef L2_CASE
  return LSURGE_OK;
}

int lsurge_l2norm_rows_bwd(const void* x, const void* dy, const float* rnorm, int64_t rows, int64_t dim, void* dx,
                           lsurge_stream_t stream) {
  LSURGE_REQUIRE(x && dy && rnorm && dx, "l2norm_rows_bwd: null pointer");
  LSURGE_REQUIRE(rows >= 0 && rows < (1ll << 31) && dim >= 8 && dim <= 512 && dim % 8 == 0,
                 "l2norm_rows_bwd: rows=%lld dim=%lld (rows < 2^31, dim a multiple of 8 in [8, 512])", (long long)rows,
                 (long long)dim);
  LSURGE_REQUIRE(((uintptr_t)x | (uintptr_t)dy | (uintptr_t)dx) % 16 == 0,
                 "l2norm_rows_bwd: x, dy and dx must be 16-byte aligned");
  if (rows == 0) return LSURGE_OK;
  hipStream_t s = (hipStream_t)stream;
  const int lpr = dim <= 64 ? 8 : dim <= 128 ? 16 : dim <= 256 ? 32 : 64;
  const dim3 grid((unsigned)((rows + 256 / lpr - 1) / (256 / lpr)));
#define L2B_CASE(LPR)                                                                                               \
  LSURGE_LAUNCH(KID_MISC, s,                                                                                        \
                hipLaunchKernelGGL(l2norm_rows_bwd_kernel<LPR>, grid, dim3(256), 0, s, (const bf16_t*)x,           \
                                   (const bf16_t*)dy, rnorm, rows, (int)dim, (bf16_t*)dx))
  if (lpr == 8) L2B_CASE(8);
  else if (lpr == 16) L2B_CASE(16);
  else if (lpr == 32) L2B_CASE(32);
  else L2B_CASE(64);
#undef L2B_CASE
  return LSURGE_OK;
}

}  // extern "C"
