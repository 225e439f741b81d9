// Chunked gated delta rule of the Gated DeltaNet block, forward (head dims 128, chunks of 64 tokens).
//
// Replaces fast_chunk_gated_delta_rule (modal/gdn_fast.py:37-113; compute dtype bf16, no qk-norm, no context
// parallelism).  Per sequence b and head h, with state S [Dk, Dv]:
//   S_t = exp(g_t) (I - beta_t k_t k_t^T) S_{t-1} + beta_t k_t v_t^T,   o_t = S_t^T q_t / sqrt(Dk)
// computed in the reference's chunked WY form.  Two kernels:
//   gdn_chunk_kernel  one workgroup per (chunk, head, sequence), all chunks at once: the decayed strictly-lower
//                     S = (k beta) k^T, A = (I + S)^-1 by forward substitution, u = A (v beta), w = A (k beta e^gcum)
//                     (both rounded to bf16, as the reference's compute dtype: gdn_fast.py:88-90), and the decayed
//                     intra-chunk attention q k^T (the scan body's attn_i, gdn_fast.py:103-105, which does not
//                     depend on the state).
//   gdn_scan_kernel   one workgroup per (32 value columns, head, sequence), the chunks in order: the value columns
//                     of the state evolve independently, so the state's 128 x 32 slice stays in LDS and the scan
//                     runs on 4x as many workgroups as there are heads.  Per chunk (gdn_fast.py:99-109):
//                       v_new = u - w S,  o = (q e^gcum) S + attn v_new,  S = e^gcum_last S + (k e^(gcum_last-gcum))^T v_new
// Arithmetic is f32 on the VALU (the reference runs these products at HIGHEST precision); padding tokens past T are
// zeros with g = 0, as the reference pads (gdn_fast.py:61-65).
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

// rows [t0, t0 + 64) of head h of a [B, T, H, GD] bf16 tensor (row0 = b T) into an LDS tile (zeros past T), each
// element optionally scaled and rounded back to bf16 (scale != 1)
__device__ __forceinline__ void load_tile(bf16_t (*dst)[GP], const bf16_t* src, int64_t row0, int T, int t0, int H,
                                          int h, float scale) {
  for (int e = threadIdx.x; e < GC * (GD / 8); e += GTH) {
    const int i = e / (GD / 8), c = 8 * (e % (GD / 8));
    u32x4 v = {0u, 0u, 0u, 0u};
    if (t0 + i < T) v = *reinterpret_cast<const u32x4*>(src + ((row0 + t0 + i) * H + h) * GD + c);
    if (scale != 1.f) {
      float f[8];
      unpack8g(v, f);
      v = u32x4{pack_bf16x2(f[0] * scale, f[1] * scale), pack_bf16x2(f[2] * scale, f[3] * scale),
                pack_bf16x2(f[4] * scale, f[5] * scale), pack_bf16x2(f[6] * scale, f[7] * scale)};
    }
    *reinterpret_cast<u32x4*>(&dst[i][c]) = v;
  }
}

// grid (N, H, B).  Outputs per (b, h, n): u, w [GC][GD] bf16, attn [GC][GC] f32 (zero above the diagonal), gcum [GC].
__global__ __launch_bounds__(GTH) void gdn_chunk_kernel(const bf16_t* __restrict__ q, const bf16_t* __restrict__ k,
                                                        const bf16_t* __restrict__ v, const float* __restrict__ g,
                                                        const bf16_t* __restrict__ beta, int T, int H, float qscale,
                                                        bf16_t* __restrict__ u_out, bf16_t* __restrict__ w_out,
                                                        float* __restrict__ attn_out, float* __restrict__ gcum_out) {
  // k (then k beta) and q (then v beta once the attention is done); in the S product k beta is formed from k where it
  // is used.  72,128 bytes (70.4 KiB) of LDS: two workgroups per CU.
  __shared__ __attribute__((aligned(16))) bf16_t ks[GC][GP], qs[GC][GP];
  __shared__ float Sm[GC][GC + 1], Am[GC][GC + 1];
  __shared__ float Tb[GC / 16 - 1][16][17];  // the blocked inverse's partial products of one level
  __shared__ float gc[GC], eg[GC], bt[GC];
  const int n = blockIdx.x, h = blockIdx.y, b = blockIdx.z, N = gridDim.x;
  const int tid = threadIdx.x, t0 = n * GC;
  const int64_t row0 = (int64_t)b * T;
  const int64_t chunk_id = ((int64_t)b * H + h) * N + n;
  if (tid < GC) {
    const int t = t0 + tid;
    gc[tid] = t < T ? g[(row0 + t) * H + h] : 0.f;
    bt[tid] = t < T ? bf16_to_f32(beta[(row0 + t) * H + h]) : 0.f;
  }
  load_tile(ks, k, row0, T, t0, H, h, 1.f);
  load_tile(qs, q, row0, T, t0, H, h, qscale);  // q * scale in the compute dtype (gdn_fast.py:56-57)
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
  // S (strictly lower) and attn (lower incl. diagonal), 2 x 4 entries per thread, dot products over GD
  {
    const int i0 = 2 * (tid / 16), j0 = 4 * (tid % 16);
    float sd[2][4] = {}, ad[2][4] = {};
    const float b0 = bt[i0], b1 = bt[i0 + 1];
    for (int d = 0; d < GD; d += 8) {
      float kb8[2][8], q8[2][8], k8[4][8];
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        unpack8g(*reinterpret_cast<const u32x4*>(&ks[i0 + r][d]), kb8[r]);
        unpack8g(*reinterpret_cast<const u32x4*>(&qs[i0 + r][d]), q8[r]);
      }
#pragma unroll
      for (int x = 0; x < 8; ++x) {  // k beta in the compute dtype (gdn_fast.py:78)
        kb8[0][x] = bf16_to_f32(f32_to_bf16(kb8[0][x] * b0));
        kb8[1][x] = bf16_to_f32(f32_to_bf16(kb8[1][x] * b1));
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) unpack8g(*reinterpret_cast<const u32x4*>(&ks[j0 + r][d]), k8[r]);
#pragma unroll
      for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
          for (int x = 0; x < 8; ++x) {
            sd[r][s] = fmaf(kb8[r][x], k8[s][x], sd[r][s]);
            ad[r][s] = fmaf(q8[r][x], k8[s][x], ad[r][s]);
          }
    }
    float* att = attn_out + chunk_id * GC * GC;
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int i = i0 + r, j = j0 + s;
        const float dec = j <= i ? __expf(gc[i] - gc[j]) : 0.f;
        Sm[i][j] = j < i ? sd[r][s] * dec : 0.f;
        att[i * GC + j] = ad[r][s] * dec;
      }
  }
  __syncthreads();
  // every read of q and of raw k is done: v beta replaces q and k beta replaces k, in the compute dtype
  // (gdn_fast.py:78, 87), formed once here for the u and w products below
  for (int e = tid; e < GC * (GD / 8); e += GTH) {
    const int i = e / (GD / 8), c = 8 * (e % (GD / 8));
    u32x4 raw = {0u, 0u, 0u, 0u};
    if (t0 + i < T) raw = *reinterpret_cast<const u32x4*>(v + ((row0 + t0 + i) * H + h) * GD + c);
    float f[8], kf[8];
    unpack8g(raw, f);
    unpack8g(*reinterpret_cast<const u32x4*>(&ks[i][c]), kf);
    const float bi = bt[i];
    *reinterpret_cast<u32x4*>(&qs[i][c]) =
        u32x4{pack_bf16x2(f[0] * bi, f[1] * bi), pack_bf16x2(f[2] * bi, f[3] * bi), pack_bf16x2(f[4] * bi, f[5] * bi),
              pack_bf16x2(f[6] * bi, f[7] * bi)};
    *reinterpret_cast<u32x4*>(&ks[i][c]) =
        u32x4{pack_bf16x2(kf[0] * bi, kf[1] * bi), pack_bf16x2(kf[2] * bi, kf[3] * bi),
              pack_bf16x2(kf[4] * bi, kf[5] * bi), pack_bf16x2(kf[6] * bi, kf[7] * bi)};
  }
  // A = (I + S)^-1 in 16 x 16 blocks (L = I + S is unit lower triangular; its off-diagonal blocks are those of S):
  //  1. the four diagonal blocks A_II = L_II^-1 at once, row by row: A[i][c] = -sum_{c <= j < i} S[i][j] A[j][c]
  //     (c < i), A[i][i] = 1, 0 above; eight threads per column split the sum (combined by an xor butterfly);
  //  2. block row I = 1 .. 3: A_IJ = -A_II sum_{K=J}^{I-1} S_IK A_KJ for every J < I (from L A = I), blocks above the
  //     diagonal 0.  22 workgroup barriers where the plain row-by-row substitution takes 64.
  {
    for (int e = tid; e < GC * GC; e += GTH) {
      const int r = e / GC, c = e % GC;
      if (r / 16 != c / 16) Am[r][c] = 0.f;  // off-diagonal blocks: filled below (lower) or zero (upper)
    }
    const int blk = tid / 128, c = (tid % 128) / 8, part = tid % 8, o = 16 * blk;
    for (int i = 0; i < 16; ++i) {
      float s = 0.f;
      for (int j = c + part; j < i; j += 8) s = fmaf(Sm[o + i][o + j], Am[o + j][o + c], s);
      s += __shfl_xor(s, 1, 64);
      s += __shfl_xor(s, 2, 64);
      s += __shfl_xor(s, 4, 64);
      if (part == 0) Am[o + i][o + c] = c < i ? -s : (c == i ? 1.f : 0.f);
      __syncthreads();
    }
    for (int I = 1; I < GC / 16; ++I) {
      for (int e = tid; e < I * 256; e += GTH) {  // T_J = sum_{K=J}^{I-1} S_IK A_KJ
        const int J = e / 256, r = (e % 256) / 16, cc = e % 16;
        float t = 0.f;
        for (int m = 16 * J; m < 16 * I; ++m) t = fmaf(Sm[16 * I + r][m], Am[m][16 * J + cc], t);
        Tb[J][r][cc] = t;
      }
      __syncthreads();
      for (int e = tid; e < I * 256; e += GTH) {  // A_IJ = -A_II T_J
        const int J = e / 256, r = (e % 256) / 16, cc = e % 16;
        float t = 0.f;
#pragma unroll
        for (int m = 0; m < 16; ++m) t = fmaf(Am[16 * I + r][16 * I + m], Tb[J][m][cc], t);
        Am[16 * I + r][16 * J + cc] = -t;
      }
      __syncthreads();
    }
  }
  // u = A vb, w = A (kb e^gcum): 2 rows x 8 columns of each per thread, rounded to bf16 (gdn_fast.py:88-90)
  {
    const int i0 = 2 * (tid / 16), c0 = 8 * (tid % 16);
    float ua[2][8] = {}, wa[2][8] = {};
    for (int j = 0; j < GC; ++j) {
      float vb8[8], kb8[8];
      unpack8g(*reinterpret_cast<const u32x4*>(&qs[j][c0]), vb8);  // v beta
      unpack8g(*reinterpret_cast<const u32x4*>(&ks[j][c0]), kb8);  // k beta
      const float e = eg[j];
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const float a = Am[i0 + r][j];
#pragma unroll
        for (int x = 0; x < 8; ++x) {
          ua[r][x] = fmaf(a, vb8[x], ua[r][x]);
          wa[r][x] = fmaf(a, kb8[x] * e, wa[r][x]);
        }
      }
    }
    bf16_t* ub = u_out + chunk_id * GC * GD;
    bf16_t* wb = w_out + chunk_id * GC * GD;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      *reinterpret_cast<u32x4*>(ub + (i0 + r) * GD + c0) =
          u32x4{pack_bf16x2(ua[r][0], ua[r][1]), pack_bf16x2(ua[r][2], ua[r][3]), pack_bf16x2(ua[r][4], ua[r][5]),
                pack_bf16x2(ua[r][6], ua[r][7])};
      *reinterpret_cast<u32x4*>(wb + (i0 + r) * GD + c0) =
          u32x4{pack_bf16x2(wa[r][0], wa[r][1]), pack_bf16x2(wa[r][2], wa[r][3]), pack_bf16x2(wa[r][4], wa[r][5]),
                pack_bf16x2(wa[r][6], wa[r][7])};
    }
  }
}

// grid (GD / SB, H, B): the scan over the chunks of one sequence and head for SB value columns.
__global__ __launch_bounds__(GTH) void gdn_scan_kernel(const bf16_t* __restrict__ q, const bf16_t* __restrict__ k,
                                                       const bf16_t* __restrict__ u_in, const bf16_t* __restrict__ w_in,
                                                       const float* __restrict__ attn_in,
                                                       const float* __restrict__ gcum_in, int T, int H, int N,
                                                       float qscale, const float* __restrict__ h0,
                                                       bf16_t* __restrict__ o, float* __restrict__ h_out) {
  __shared__ __attribute__((aligned(16))) bf16_t qs[GC][GP], ks[GC][GP], ws[GC][GP];
  // state slice and v_new with 16-byte aligned rows (pitch SB + 4): a thread reads 4 or 8 consecutive columns at once,
  // and the 8 column groups of a row that a wave reads at one d are distinct 16-byte slots
  constexpr int SP = SB + 4;
  __shared__ __attribute__((aligned(16))) float hs[GD][SP], vn[GC][SP];
  __shared__ float at[GC][GC + 1];
  __shared__ float gc[GC], ek[GC];  // gcum, exp(gcum_last - gcum)
  const int cb = blockIdx.x * SB, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  const int64_t row0 = (int64_t)b * T;
  const int64_t bh = (int64_t)b * H + h;
  for (int e = tid; e < GD * SB; e += GTH) {
    const int d = e / SB, c = e % SB;
    hs[d][c] = h0 ? h0[(bh * GD + d) * GD + cb + c] : 0.f;
  }
  // outputs of this thread: row ri, columns ci .. ci + 3 of the [GC][SB] chunk products; state entries row hd (of
  // GD), columns hc .. hc + 7
  const int ri = tid / 8, ci = 4 * (tid % 8);
  const int hd = tid / 4, hc = 8 * (tid % 4);
  // The next chunk's tiles are fetched into registers while the current one computes: this thread's two 16-byte
  // pieces of each of q, k and w (piece e = tid + GTH p: row e / 16, columns 8 (e % 16)), its eight attn values and
  // (threads < GC) one gcum value.
  constexpr int PP = GC * (GD / 8) / GTH;  // pieces per thread and tile
  static_assert(PP * GTH == GC * (GD / 8) && GC * GC == 8 * GTH, "scan tile split");
  u32x4 pq[PP], pk[PP], pw[PP];
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
  };
  fetch(0);
  for (int n = 0; n < N; ++n) {
    const int t0 = n * GC;
    const int64_t chunk_id = bh * N + n;
    __syncthreads();  // the previous chunk is done with the tiles
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
    for (int hlf = 0; hlf < 2; ++hlf)
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        const int e = 4 * (tid + GTH * hlf) + x;
        at[e / GC][e % GC] = pa[hlf][x];
      }
    if (tid < GC) gc[tid] = pg;
    __syncthreads();
    if (tid < GC) ek[tid] = __expf(gc[GC - 1] - gc[tid]);  // read after the barrier that follows v_new
    if (n + 1 < N) fetch(n + 1);
    // v_new = u - w S and inter = (q e^gcum) S for this thread's 1 x 4 outputs
    float vacc[1][4] = {}, iacc[1][4] = {};
    for (int d = 0; d < GD; d += 8) {
      float w8[1][8], q8[1][8];
      unpack8g(*reinterpret_cast<const u32x4*>(&ws[ri][d]), w8[0]);
      unpack8g(*reinterpret_cast<const u32x4*>(&qs[ri][d]), q8[0]);
#pragma unroll
      for (int x = 0; x < 8; ++x) {
        const f32x4 hv = *reinterpret_cast<const f32x4*>(&hs[d + x][ci]);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          vacc[0][s] = fmaf(w8[0][x], hv[s], vacc[0][s]);
          iacc[0][s] = fmaf(q8[0][x], hv[s], iacc[0][s]);
        }
      }
    }
    const bf16_t* ub = u_in + chunk_id * GC * GD;
#pragma unroll
    for (int s = 0; s < 4; ++s) vn[ri][ci + s] = bf16_to_f32(ub[ri * GD + cb + ci + s]) - vacc[0][s];
    __syncthreads();
    // o = inter e^gcum + attn v_new (attn is zero above the diagonal)
    {
      const int r = 0, i = ri;
      float acc[4];
      const float e = __expf(gc[i]);
#pragma unroll
      for (int s = 0; s < 4; ++s) acc[s] = iacc[r][s] * e;
      for (int j = 0; j <= i; ++j) {
        const float a = at[i][j];
        const f32x4 vv = *reinterpret_cast<const f32x4*>(&vn[j][ci]);
#pragma unroll
        for (int s = 0; s < 4; ++s) acc[s] = fmaf(a, vv[s], acc[s]);
      }
      if (t0 + i < T) {
        bf16_t* op = o + ((row0 + t0 + i) * H + h) * GD + cb + ci;
        *reinterpret_cast<uint2*>(op) = uint2{pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3])};
      }
    }
    // S = e^gcum_last S + (k e^(gcum_last - gcum))^T v_new; every read of the old state happened before the barrier
    // above
    const float gl = gc[GC - 1], el = __expf(gl);
    float hn[8];
#pragma unroll
    for (int x = 0; x < 8; ++x) hn[x] = hs[hd][hc + x] * el;
    for (int i = 0; i < GC; ++i) {
      const float k0 = bf16_to_f32(ks[i][hd]) * ek[i];
      const f32x4 v0 = *reinterpret_cast<const f32x4*>(&vn[i][hc]), v1 = *reinterpret_cast<const f32x4*>(&vn[i][hc + 4]);
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        hn[x] = fmaf(k0, v0[x], hn[x]);
        hn[x + 4] = fmaf(k0, v1[x], hn[x + 4]);
      }
    }
    __syncthreads();  // every thread has read the old state (o used only vn and at)
#pragma unroll
    for (int x = 0; x < 8; ++x) hs[hd][hc + x] = hn[x];
  }
  __syncthreads();
  if (h_out)
    for (int e = tid; e < GD * SB; e += GTH) {
      const int d = e / SB, c = e % SB;
      h_out[(bh * GD + d) * GD + cb + c] = hs[d][c];
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
  LSURGE_LAUNCH(KID_MISC, s,
                hipLaunchKernelGGL(gdn_chunk_kernel, dim3((unsigned)N, (unsigned)h, (unsigned)b), dim3(GTH), 0, s,
                                   (const bf16_t*)q, (const bf16_t*)k, (const bf16_t*)v, g, (const bf16_t*)beta, (int)t,
                                   (int)h, qscale, u, w, attn, gcum));
  LSURGE_LAUNCH(KID_MISC, s,
                hipLaunchKernelGGL(gdn_scan_kernel, dim3(GD / SB, (unsigned)h, (unsigned)b), dim3(GTH), 0, s,
                                   (const bf16_t*)q, (const bf16_t*)k, (const bf16_t*)u, (const bf16_t*)w,
                                   (const float*)attn, (const float*)gcum, (int)t, (int)h, (int)N, qscale, h0,
                                   (bf16_t*)o, h_out));
  return LSURGE_OK;
}

}  // extern "C"
