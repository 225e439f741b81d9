// Causal depthwise Conv1D of the Gated DeltaNet block, forward and backward (memory-bound).
//
// Replaces fast_conv._fast_call (modal/fast_conv.py:14-31), itself the stand-in for flax nnx.Conv(padding="CAUSAL",
// feature_group_count=C) on [B, T, C] inputs with a [K, 1, C] kernel:
//   y[b, t, c] = sum_{j<K} w[j, c] x[b, t-(K-1)+j, c]   (zero before t = 0; j ascending, as fast_conv.py:27-30)
// Backward (what XLA derives from it for the reference):
//   dx[b, t, c] = sum_{j<K} w[j, c] dy[b, t+(K-1)-j, c]   (zero past T)
//   dw[j, c]    = sum_{b, t} dy[b, t, c] x[b, t-(K-1)+j, c]
// Layout: x, y, dy, dx [B, T, C] bf16 (C contiguous); w [K, C] bf16; dw [K, C] f32.  One thread owns 8 channels
// (16 bytes) over CT_STEPS consecutive steps of one sequence.  Its taps and a sliding window of the K - 1 neighbouring
// rows stay in registers, so every row is read once (plus K - 1 halo rows per segment) and written once, and a wave
// covers 512 contiguous channels of a row.  Products accumulate in f32 with one rounding to bf16.  dw: each thread
// keeps an f32 partial over its steps, a workgroup folds its four segments' partials into one slot, and a second
// kernel sums the slots in order (deterministic, no atomics).
#include "launchers.h"

namespace {

constexpr int CT = 256;       // threads per workgroup
constexpr int CT_STEPS = 64;  // steps per thread
constexpr int CONV_KMAX = 8;

__device__ __forceinline__ void unpack8(u32x4 v, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(v[i] << 16);
    f[2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u);
  }
}
__device__ __forceinline__ u32x4 pack8(const float* f) {
  return u32x4{pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]), pack_bf16x2(f[6], f[7])};
}
__device__ __forceinline__ u32x4 ld_row(const bf16_t* base, int64_t t, int T, int64_t C) {
  return (t >= 0 && t < T) ? *reinterpret_cast<const u32x4*>(base + t * C) : u32x4{0u, 0u, 0u, 0u};
}

// grid (ceil(C / 8 / CT), segments, B)
template <int K>
__global__ __launch_bounds__(CT) void causal_conv_fwd_kernel(const bf16_t* __restrict__ x, const bf16_t* __restrict__ w,
                                                             int T, int C, bf16_t* __restrict__ y) {
  const int cg = blockIdx.x * CT + threadIdx.x;
  if (cg >= C / 8) return;
  const int t0 = blockIdx.y * CT_STEPS;
  const int64_t boff = (int64_t)blockIdx.z * T * C + 8 * cg;
  const bf16_t* xb = x + boff;
  bf16_t* yb = y + boff;
  float wk[K][8];
#pragma unroll
  for (int j = 0; j < K; ++j) unpack8(*reinterpret_cast<const u32x4*>(w + (int64_t)j * C + 8 * cg), wk[j]);
  float win[K][8];  // win[j] = x[t - (K-1) + j]; win[K-1] is the current row
#pragma unroll
  for (int j = 0; j < K - 1; ++j) unpack8(ld_row(xb, t0 - (K - 1) + j, T, C), win[j]);
  const int t1 = min(T, t0 + CT_STEPS);
  constexpr int U = 8;  // rows loaded ahead
  for (int tb = t0; tb < t1; tb += U) {
    u32x4 raw[U];
#pragma unroll
    for (int u = 0; u < U; ++u) raw[u] = ld_row(xb, tb + u, t1, C);  // rows past the segment (and T): zeros, unused
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (tb + u >= t1) break;
      unpack8(raw[u], win[K - 1]);
      float o[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float acc = wk[0][i] * win[0][i];
#pragma unroll
        for (int j = 1; j < K; ++j) acc = fmaf(wk[j][i], win[j][i], acc);
        o[i] = acc;
      }
      *reinterpret_cast<u32x4*>(yb + (int64_t)(tb + u) * C) = pack8(o);
#pragma unroll
      for (int j = 0; j < K - 1; ++j)
#pragma unroll
        for (int i = 0; i < 8; ++i) win[j][i] = win[j + 1][i];
    }
  }
}

// dx and the partials of dw.  A workgroup's BW waves take BW consecutive segments of the same 64 channel groups
// (grid (ceil(C / 8 / 64), ceil(segments / BW), B)); their dw partials are summed in wave order through LDS, and one
// slot per workgroup is written: part [B * ceil(segments / BW)][K][C] f32.
constexpr int BW = CT / 64;
template <int K>
__global__ __launch_bounds__(CT) void causal_conv_bwd_kernel(const bf16_t* __restrict__ x, const bf16_t* __restrict__ w,
                                                             const bf16_t* __restrict__ dy, int T, int C,
                                                             bf16_t* __restrict__ dx, float* __restrict__ part) {
  __shared__ f32x4 red[BW][64][2];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int cg = blockIdx.x * 64 + lane;
  const int seg = blockIdx.y * BW + wave;
  const int t0 = seg * CT_STEPS;
  // lanes past the channels and waves past the sequence still reach the barriers of the dw sum below
  const bool live = cg < C / 8 && t0 < T;
  const int cgc = min(cg, C / 8 - 1);
  const int64_t boff = (int64_t)blockIdx.z * T * C + 8 * cgc;
  const bf16_t* xb = x + boff;
  const bf16_t* gb = dy + boff;
  bf16_t* db = dx + boff;
  float wk[K][8];
#pragma unroll
  for (int j = 0; j < K; ++j) unpack8(*reinterpret_cast<const u32x4*>(w + (int64_t)j * C + 8 * cgc), wk[j]);
  float xw[K][8];  // xw[j] = x[t - (K-1) + j]
  float gw[K][8];  // gw[i] = dy[t + i]
#pragma unroll
  for (int j = 0; j < K - 1; ++j) unpack8(ld_row(xb, t0 - (K - 1) + j, T, C), xw[j]);
#pragma unroll
  for (int i = 1; i < K; ++i) unpack8(ld_row(gb, t0 + i - 1, T, C), gw[i]);
  float dwk[K][8];
#pragma unroll
  for (int j = 0; j < K; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) dwk[j][i] = 0.f;
  const int t1 = live ? min(T, t0 + CT_STEPS) : t0;
  constexpr int U = 4;
  for (int tb = t0; tb < t1; tb += U) {
    u32x4 rx[U], rg[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      rx[u] = ld_row(xb, tb + u, t1, C);
      rg[u] = ld_row(gb, tb + u + K - 1, T, C);  // lookahead row (zero past T)
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (tb + u >= t1) break;
      // slide: gw[i] <- gw[i + 1], gw[K-1] = dy[t + K - 1]; xw[K-1] = x[t]
#pragma unroll
      for (int i = 0; i < K - 1; ++i)
#pragma unroll
        for (int c = 0; c < 8; ++c) gw[i][c] = gw[i + 1][c];
      unpack8(rg[u], gw[K - 1]);
      unpack8(rx[u], xw[K - 1]);
      float o[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        float acc = wk[0][c] * gw[K - 1][c];
#pragma unroll
        for (int j = 1; j < K; ++j) acc = fmaf(wk[j][c], gw[K - 1 - j][c], acc);
        o[c] = acc;
      }
      *reinterpret_cast<u32x4*>(db + (int64_t)(tb + u) * C) = pack8(o);
      // dw[j] += dy[t] x[t - (K-1) + j]  (dy[t] = gw[0])
#pragma unroll
      for (int j = 0; j < K; ++j)
#pragma unroll
        for (int c = 0; c < 8; ++c) dwk[j][c] = fmaf(gw[0][c], xw[j][c], dwk[j][c]);
#pragma unroll
      for (int j = 0; j < K - 1; ++j)
#pragma unroll
        for (int c = 0; c < 8; ++c) xw[j][c] = xw[j + 1][c];
    }
  }
  // dw of the workgroup's segments, summed in wave (time) order, one tap at a time through LDS
  float* pb = part + ((int64_t)blockIdx.z * gridDim.y + blockIdx.y) * K * C + 8 * cgc;
#pragma unroll
  for (int j = 0; j < K; ++j) {
    red[wave][lane][0] = f32x4{dwk[j][0], dwk[j][1], dwk[j][2], dwk[j][3]};
    red[wave][lane][1] = f32x4{dwk[j][4], dwk[j][5], dwk[j][6], dwk[j][7]};
    __syncthreads();
    if (wave == 0 && cg < C / 8) {
      f32x4 a = red[0][lane][0], b = red[0][lane][1];
#pragma unroll
      for (int v = 1; v < BW; ++v) {
        a += red[v][lane][0];
        b += red[v][lane][1];
      }
      *reinterpret_cast<f32x4*>(pb + (int64_t)j * C) = a;
      *reinterpret_cast<f32x4*>(pb + (int64_t)j * C + 4) = b;
    }
    __syncthreads();
  }
}

// dw[e] = sum over the nparts slots in slot order (sequence-major, then segment group), 8 loads in flight
__global__ void causal_conv_dw_reduce_kernel(const float* __restrict__ part, int nparts, int64_t KC, float* __restrict__ dw) {
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < KC; e += (int64_t)gridDim.x * blockDim.x) {
    float s = 0.f;
    int p = 0;
    for (; p + 8 <= nparts; p += 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = part[(int64_t)(p + u) * KC + e];
#pragma unroll
      for (int u = 0; u < 8; ++u) s += v[u];
    }
    for (; p < nparts; ++p) s += part[(int64_t)p * KC + e];
    dw[e] = s;
  }
}

int check_conv(const void* x, const void* w, int64_t b, int64_t t, int64_t c, int64_t k) {
  LSURGE_REQUIRE(x && w, "causal_conv1d: null pointer");
  LSURGE_REQUIRE(b >= 1 && b < 65536 && t >= 1 && t < (1ll << 31) && c >= 8 && c % 8 == 0 && c < (1ll << 31) &&
                     k >= 1 && k <= CONV_KMAX && b * t * c < (1ll << 62),
                 "causal_conv1d: b=%lld t=%lld c=%lld k=%lld (c a multiple of 8, 1 <= k <= %d)", (long long)b,
                 (long long)t, (long long)c, (long long)k, CONV_KMAX);
  LSURGE_REQUIRE((t + CT_STEPS - 1) / CT_STEPS < 65536, "causal_conv1d: t=%lld too long", (long long)t);
  return LSURGE_OK;
}

#define CONV_K_CASES(M) M(1) M(2) M(3) M(4) M(5) M(6) M(7) M(8)

}  // namespace

extern "C" {

int lsurge_causal_conv1d(const void* x, const void* w, int64_t b, int64_t t, int64_t c, int64_t k, void* y,
                         lsurge_stream_t stream) {
  if (int rc = check_conv(x, w, b, t, c, k)) return rc;
  LSURGE_REQUIRE(y, "causal_conv1d: null output");
  LSURGE_REQUIRE(((uintptr_t)x | (uintptr_t)w | (uintptr_t)y) % 16 == 0, "causal_conv1d: buffers must be 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)((c / 8 + CT - 1) / CT), (unsigned)((t + CT_STEPS - 1) / CT_STEPS), (unsigned)b);
  switch (k) {
#define CONV_FWD(KK)                                                                                             \
  case KK:                                                                                                       \
    LSURGE_LAUNCH(KID_MISC, s, hipLaunchKernelGGL(causal_conv_fwd_kernel<KK>, grid, dim3(CT), 0, s,              \
                                                  (const bf16_t*)x, (const bf16_t*)w, (int)t, (int)c, (bf16_t*)y)); \
    break;
    CONV_K_CASES(CONV_FWD)
#undef CONV_FWD
  }
  return LSURGE_OK;
}

static int64_t conv_seg_groups(int64_t t) { return ((t + CT_STEPS - 1) / CT_STEPS + BW - 1) / BW; }

size_t lsurge_causal_conv1d_bwd_workspace_bytes(int64_t b, int64_t t, int64_t c, int64_t k) {
  if (b < 1 || t < 1 || c < 1 || k < 1) return 0;
  return sizeof(float) * (size_t)(b * conv_seg_groups(t)) * (size_t)(k * c);
}

int lsurge_causal_conv1d_bwd(const void* x, const void* w, const void* dy, int64_t b, int64_t t, int64_t c, int64_t k,
                             void* dx, float* dw, void* workspace, size_t workspace_bytes, lsurge_stream_t stream) {
  if (int rc = check_conv(x, w, b, t, c, k)) return rc;
  LSURGE_REQUIRE(dy && dx && dw && workspace, "causal_conv1d_bwd: null pointer");
  LSURGE_REQUIRE(((uintptr_t)x | (uintptr_t)w | (uintptr_t)dy | (uintptr_t)dx | (uintptr_t)dw | (uintptr_t)workspace) %
                         16 == 0,
                 "causal_conv1d_bwd: buffers must be 16-byte aligned");
  const size_t need = lsurge_causal_conv1d_bwd_workspace_bytes(b, t, c, k);
  LSURGE_REQUIRE(workspace_bytes >= need, "causal_conv1d_bwd: workspace %zu < %zu bytes", workspace_bytes, need);
  hipStream_t s = (hipStream_t)stream;
  const int groups = (int)conv_seg_groups(t);
  const dim3 grid((unsigned)((c / 8 + 63) / 64), (unsigned)groups, (unsigned)b);
  float* part = (float*)workspace;
  switch (k) {
#define CONV_BWD(KK)                                                                                              \
  case KK:                                                                                                        \
    LSURGE_LAUNCH(KID_MISC, s, hipLaunchKernelGGL(causal_conv_bwd_kernel<KK>, grid, dim3(CT), 0, s,               \
                                                  (const bf16_t*)x, (const bf16_t*)w, (const bf16_t*)dy, (int)t,   \
                                                  (int)c, (bf16_t*)dx, part));                                     \
    break;
    CONV_K_CASES(CONV_BWD)
#undef CONV_BWD
  }
  const int64_t KC = k * c;
  const unsigned rgrid = (unsigned)std::min<int64_t>((KC + 255) / 256, 1024);
  LSURGE_LAUNCH(KID_MISC, s, hipLaunchKernelGGL(causal_conv_dw_reduce_kernel, dim3(rgrid), dim3(256), 0, s,
                                                (const float*)part, (int)(b * groups), KC, dw));
  return LSURGE_OK;
}

}  // extern "C"
