// Router: f32 logits (sequential sum over d), top-k with lower-index tie-break, softmax over the selection.
//
// Stands in for MaxText RoutedMoE's gate + top-k (third-party; configured by configs/stage1.yml:34-37 of the
// reference).  Logit order contract: logits[t,e] = (((x[t,0]w[0,e]) + x[t,1]w[1,e]) + ...) in f32, then
// + bias[e].  bf16 x bf16 products are exact in f32, so this is reproducible bit for bit on the CPU.
#include "common.h"

namespace {

constexpr int RT_TOK = 32;      // tokens per workgroup
constexpr int RT_DC = 64;       // d chunk staged in LDS
constexpr int RT_THREADS = 256;
constexpr int RT_EMAX = 256;

// LDS: x chunk transposed [RT_DC][RT_TOK] f32 (8 KB) + w chunk [RT_DC][EP] f32 (<= 64 KB).
// After the d loop the w region is reused for the [RT_TOK][EP] logits.
template <int EP>  // experts padded to a multiple of 32
__global__ __launch_bounds__(RT_THREADS) void router_topk_kernel(const bf16_t* __restrict__ x,
                                                                 const bf16_t* __restrict__ w,
                                                                 const float* __restrict__ bias, int T, int d,
                                                                 int E, int k, float* __restrict__ logits,
                                                                 int32_t* __restrict__ sel,
                                                                 float* __restrict__ weights) {
  constexpr int EJ = EP / 32;  // experts per thread
  __shared__ float xs[RT_DC][RT_TOK];
  __shared__ float ws[RT_DC * EP > RT_TOK * EP ? RT_DC * EP : RT_TOK * EP];
  const int tid = threadIdx.x;
  const int t0 = blockIdx.x * RT_TOK;
  const int q = tid & 7;    // token quad: tokens 4q..4q+3
  const int s = tid >> 3;   // expert slice: experts s + 32 j
  float acc[4][EJ];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int j = 0; j < EJ; ++j) acc[a][j] = 0.f;

  for (int d0 = 0; d0 < d; d0 += RT_DC) {
    const int dc = min(RT_DC, d - d0);
    // stage x[t0 .. t0+32, d0 .. d0+dc) transposed, as f32 (zeros past T / d)
    for (int i = tid; i < RT_TOK * RT_DC; i += RT_THREADS) {
      const int tt = i / RT_DC, dd = i % RT_DC;
      const int t = t0 + tt;
      xs[dd][tt] = (t < T && dd < dc) ? bf16_to_f32(x[(int64_t)t * d + d0 + dd]) : 0.f;
    }
    // stage w[d0 .. d0+dc, 0 .. E) as f32, experts padded with zeros
    for (int i = tid; i < RT_DC * EP; i += RT_THREADS) {
      const int dd = i / EP, e = i % EP;
      ws[i] = (dd < dc && e < E) ? bf16_to_f32(w[(int64_t)(d0 + dd) * E + e]) : 0.f;
    }
    __syncthreads();
    for (int dd = 0; dd < dc; ++dd) {
      const f32x4 xv = *reinterpret_cast<const f32x4*>(&xs[dd][4 * q]);
#pragma unroll
      for (int j = 0; j < EJ; ++j) {
        const float wv = ws[dd * EP + s + 32 * j];
        // exact products; one f32 rounding per add, ascending d
        acc[0][j] = acc[0][j] + xv[0] * wv;
        acc[1][j] = acc[1][j] + xv[1] * wv;
        acc[2][j] = acc[2][j] + xv[2] * wv;
        acc[3][j] = acc[3][j] + xv[3] * wv;
      }
    }
    __syncthreads();
  }
  // logits -> LDS [RT_TOK][EP] and global
  float* ls = ws;
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const int tt = 4 * q + a;
    const int t = t0 + tt;
#pragma unroll
    for (int j = 0; j < EJ; ++j) {
      const int e = s + 32 * j;
      float v = acc[a][j];
      if (e < E && bias) v = v + bias[e];
      ls[tt * EP + e] = (e < E) ? v : -INFINITY;
      if (t < T && e < E && logits) logits[(int64_t)t * E + e] = v;
    }
  }
  __syncthreads();
  // top-k: one wave per token, 8 tokens per wave
  const int lane = tid & 63, wv = tid >> 6;
  for (int tt = wv; tt < RT_TOK; tt += RT_THREADS / 64) {
    const int t = t0 + tt;
    if (t >= T) break;
    constexpr int EC = (EP + 63) / 64;
    float v[EC];
    bool taken[EC];
#pragma unroll
    for (int c = 0; c < EC; ++c) {
      const int e = lane + 64 * c;
      v[c] = (e < E) ? ls[tt * EP + e] : -INFINITY;
      taken[c] = !(e < E);
    }
    float top0 = 0.f, denom = 0.f;
    float selv[8];
    int seli[8];
    for (int j = 0; j < k; ++j) {
      // lane-local best (lowest index wins ties: c ascending, strict >)
      float bv = -INFINITY;
      int bi = 0x7fffffff;
#pragma unroll
      for (int c = 0; c < EC; ++c) {
        const int e = lane + 64 * c;
        if (!taken[c] && (bi == 0x7fffffff || v[c] > bv)) {
          bv = v[c];
          bi = e;
        }
      }
      // wave argmax: larger value, then lower index
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        if (oi != 0x7fffffff && (bi == 0x7fffffff || ov > bv || (ov == bv && oi < bi))) {
          bv = ov;
          bi = oi;
        }
      }
#pragma unroll
      for (int c = 0; c < EC; ++c)
        if (lane + 64 * c == bi) taken[c] = true;
      if (j < 8) {
        selv[j] = bv;
        seli[j] = bi;
      }
      if (j == 0) top0 = bv;
      const float z = __expf(bv - top0);
      denom += z;
      if (lane == 0) {
        sel[(int64_t)t * k + j] = bi;
        weights[(int64_t)t * k + j] = z;  // normalised below
      }
    }
    if (lane == 0) {
      const float inv = 1.f / denom;
      for (int j = 0; j < k; ++j) weights[(int64_t)t * k + j] *= inv;
    }
    (void)selv;
    (void)seli;
  }
}

}  // namespace

extern "C" int lsurge_router_topk(const void* x, const void* w_r, const float* bias, int64_t t, int64_t d,
                                  int64_t e, int64_t k, float* logits, int32_t* sel, float* weights,
                                  lsurge_stream_t stream) {
  LSURGE_REQUIRE(x && w_r && sel && weights, "router_topk: null pointer");
  LSURGE_REQUIRE(t >= 0 && d > 0 && e >= 1 && e <= RT_EMAX && k >= 1 && k <= e, "router_topk: bad shape t=%lld d=%lld e=%lld k=%lld",
                 (long long)t, (long long)d, (long long)e, (long long)k);
  LSURGE_REQUIRE(t < (1ll << 31) && t * d < (1ll << 40), "router_topk: too large");
  if (t == 0) return LSURGE_OK;
  dim3 grid((unsigned)((t + RT_TOK - 1) / RT_TOK)), block(RT_THREADS);
  hipStream_t s = (hipStream_t)stream;
  const bf16_t* xb = (const bf16_t*)x;
  const bf16_t* wb = (const bf16_t*)w_r;
#define RT_CASE(EP)                                                                                       \
  LSURGE_LAUNCH(KID_ROUTER, s,                                                                            \
                hipLaunchKernelGGL(router_topk_kernel<EP>, grid, block, 0, s, xb, wb, bias, (int)t, (int)d, \
                                   (int)e, (int)k, logits, sel, weights))
  if (e <= 32) RT_CASE(32);
  else if (e <= 64) RT_CASE(64);
  else if (e <= 128) RT_CASE(128);
  else RT_CASE(256);
#undef RT_CASE
  return LSURGE_OK;
}
