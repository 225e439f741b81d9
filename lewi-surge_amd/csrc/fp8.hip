// FP8 (OCP E4M3) quantisation with current scaling, for the FP8 variant of the grouped GEMMs.
//
// Current scaling (Transformer Engine's Float8CurrentScaling recipe, which the reference tries through MaxText's
// `quantization=te_fp8_currentscaling`, modal/te_run.py:99; both are third-party): each tensor (or each group: an
// expert's weight matrix) gets its own scale from its own amax, computed just before the cast:
//   amax = max |x|,  scale = 448 / amax (1 when amax is 0, the largest float when the quotient overflows),
//   q = e4m3(x * scale) rounded to nearest even and saturated at +-448,  scale_inv = 1 / scale.
// Two passes: per-block amax partials, then the cast, whose blocks each reduce their group's partials (a few
// hundred floats) before converting; max is order-independent, so the result is deterministic.  The cast can
// also take its amax from one slot filled by an earlier kernel (the SwiGLU epilogue's atomic max of h).
// The transposed cast writes [C, R] per group, so that a weight stored [K, N] becomes the K-contiguous [N, K]
// operand of the FP8 GEMM.
#include <cfloat>

#include "launchers.h"

namespace {

constexpr int QT = 256;       // threads per workgroup
constexpr int MAX_PARTS = 1024; // amax partials per group
constexpr int AU = 4;           // independent 16-byte loads per thread and step of the amax kernel

__device__ __forceinline__ float block_max(float v, float* sh) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  const int w = threadIdx.x >> 6;
  __syncthreads();  // sh may still be read by a previous call
  if ((threadIdx.x & 63) == 0) sh[w] = v;
  __syncthreads();
  float m = sh[0];
  for (int i = 1; i < (int)(blockDim.x >> 6); ++i) m = fmaxf(m, sh[i]);
  return m;
}

// scale of a group from its amax partials (every thread gets it)
__device__ __forceinline__ float group_scale(const float* partial, int nparts, float* sh) {
  float m = 0.f;
  for (int i = threadIdx.x; i < nparts; i += blockDim.x) m = fmaxf(m, partial[i]);
  const float amax = block_max(m, sh);
  if (!(amax > 0.f)) return 1.f;
  const float s = __fdiv_rn(448.f, amax);
  return s <= FLT_MAX ? s : FLT_MAX;
}

// four floats (already scaled) -> four E4M3 bytes, element 0 in the low byte
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d) {
  a = fminf(fmaxf(a, -448.f), 448.f);
  b = fminf(fmaxf(b, -448.f), 448.f);
  c = fminf(fmaxf(c, -448.f), 448.f);
  d = fminf(fmaxf(d, -448.f), 448.f);
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (uint32_t)w;
}

__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// amax partials: grid (nb, G); block b of group g reads the 8-element chunks b AU QT + u QT + tid (u < AU), then
// + nb AU QT, ... of the group's n elements (n % 8 == 0), AU loads in flight per thread, and writes
// partial[g nb + b]
__global__ __launch_bounds__(QT) void fp8_amax_kernel(const bf16_t* __restrict__ x, int64_t n, int64_t gstride, int nb,
                                                      float* __restrict__ partial) {
  __shared__ float sh[QT / 64];
  const bf16_t* xg = x + (int64_t)blockIdx.y * gstride;
  const int64_t nc = n / 8;
  float m = 0.f;
  for (int64_t c = (int64_t)blockIdx.x * AU * QT + threadIdx.x; c < nc; c += (int64_t)nb * AU * QT) {
    u32x4 v[AU];
#pragma unroll
    for (int u = 0; u < AU; ++u)
      v[u] = c + u * QT < nc ? *reinterpret_cast<const u32x4*>(xg + 8 * (c + u * QT)) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int u = 0; u < AU; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) m = fmaxf(m, fmaxf(fabsf(bf_lo(v[u][i])), fabsf(bf_hi(v[u][i]))));
  }
  m = block_max(m, sh);
  if (threadIdx.x == 0) partial[(int64_t)blockIdx.y * nb + blockIdx.x] = m;
}

// cast of group blockIdx.y: 16 elements per thread and step, grid-stride over the group's n elements (n % 16 == 0;
// with nrows set, only the first nrows[0] * row_elems).  Block (0, g) writes sinv[g]; block (0, 0) zeroes
// zero[0 .. nzero) (slots a later kernel fills by atomic max).
__global__ __launch_bounds__(QT) void fp8_cast_kernel(const bf16_t* __restrict__ x, int64_t n, int64_t gstride,
                                                      const float* __restrict__ partial, int nparts,
                                                      uint8_t* __restrict__ q, float* __restrict__ sinv,
                                                      const int32_t* __restrict__ nrows, int64_t row_elems,
                                                      uint32_t* __restrict__ zero, int nzero) {
  __shared__ float sh[QT / 64];
  const int g = blockIdx.y;
  const float scale = group_scale(partial + (int64_t)g * nparts, nparts, sh);
  if (blockIdx.x == 0 && threadIdx.x == 0) sinv[g] = __fdiv_rn(1.f, scale);
  if (blockIdx.x == 0 && g == 0 && (int)threadIdx.x < nzero) zero[threadIdx.x] = 0u;
  const int64_t ne = nrows ? min(n, (int64_t)max(nrows[0], 0) * row_elems) : n;
  const bf16_t* xg = x + (int64_t)g * gstride;
  uint8_t* qg = q + (int64_t)g * n;
  for (int64_t c = (int64_t)blockIdx.x * QT + threadIdx.x; c < ne / 16; c += (int64_t)gridDim.x * QT) {
    const u32x4 v0 = *reinterpret_cast<const u32x4*>(xg + 16 * c);
    const u32x4 v1 = *reinterpret_cast<const u32x4*>(xg + 16 * c + 8);
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      o[i] = e4m3x4(bf_lo(v0[2 * i]) * scale, bf_hi(v0[2 * i]) * scale, bf_lo(v0[2 * i + 1]) * scale,
                    bf_hi(v0[2 * i + 1]) * scale);
      o[i + 2] = e4m3x4(bf_lo(v1[2 * i]) * scale, bf_hi(v1[2 * i]) * scale, bf_lo(v1[2 * i + 1]) * scale,
                        bf_hi(v1[2 * i + 1]) * scale);
    }
    *reinterpret_cast<u32x4*>(qg + 16 * c) = o;
  }
}

// transposed cast: group g of x is [R, C] bf16 -> q group g [C, R] e4m3 (R, C multiples of 16); one 64 x 64 tile per
// workgroup (grid (tiles, G), edge tiles partial), staged through LDS as scaled floats (pitch 65: both directions
// conflict-free)
__global__ __launch_bounds__(QT) void fp8_cast_t_kernel(const bf16_t* __restrict__ x, int R, int C,
                                                        const float* __restrict__ partial, int nparts,
                                                        uint8_t* __restrict__ q, float* __restrict__ sinv) {
  __shared__ float sh[QT / 64];
  __shared__ float t[64][65];
  const int g = blockIdx.y;
  const float scale = group_scale(partial + (int64_t)g * nparts, nparts, sh);
  if (blockIdx.x == 0 && threadIdx.x == 0) sinv[g] = __fdiv_rn(1.f, scale);
  const int ct = (C + 63) / 64;
  const int r0 = (blockIdx.x / ct) * 64, c0 = (blockIdx.x % ct) * 64;
  const int tid = threadIdx.x, rr = tid >> 2, cq = 16 * (tid & 3);
  u32x4 v0 = {0u, 0u, 0u, 0u}, v1 = {0u, 0u, 0u, 0u};
  if (r0 + rr < R && c0 + cq < C) {  // 16-element chunks: C % 16 == 0
    const bf16_t* src = x + (int64_t)g * R * C + (int64_t)(r0 + rr) * C + c0 + cq;
    v0 = *reinterpret_cast<const u32x4*>(src);
    v1 = *reinterpret_cast<const u32x4*>(src + 8);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    t[cq + 2 * i][rr] = bf_lo(v0[i]) * scale;
    t[cq + 2 * i + 1][rr] = bf_hi(v0[i]) * scale;
    t[cq + 8 + 2 * i][rr] = bf_lo(v1[i]) * scale;
    t[cq + 8 + 2 * i + 1][rr] = bf_hi(v1[i]) * scale;
  }
  __syncthreads();
  if (c0 + rr >= C || r0 + cq >= R) return;  // R % 16 == 0
  const float* row = &t[rr][cq];  // output row c0 + rr, elements r0 + cq .. + 15
  u32x4 o;
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = e4m3x4(row[4 * i], row[4 * i + 1], row[4 * i + 2], row[4 * i + 3]);
  *reinterpret_cast<u32x4*>(q + (int64_t)g * R * C + (int64_t)(c0 + rr) * R + r0 + cq) = o;
}

// blocks per group: about two steps of AU chunks per thread
int amax_parts(int64_t n) {
  return (int)std::min<int64_t>(MAX_PARTS, std::max<int64_t>(1, (n / 8 + 2 * AU * QT - 1) / (2 * AU * QT)));
}

}  // namespace

namespace lsurge {

size_t fp8_partial_bytes(int64_t groups) { return sizeof(float) * (size_t)groups * MAX_PARTS; }

int fp8_quantize_impl(const void* x, int64_t groups, int64_t rows, int64_t cols, bool transpose, void* q, float* sinv,
                      float* partial, hipStream_t s, uint32_t* zero, int nzero) {
  LSURGE_REQUIRE(groups >= 1 && groups < 65536 && rows >= 1 && cols >= 1 && rows < (1 << 30) && cols < (1 << 30) &&
                     rows * cols < (1ll << 40),
                 "fp8_quantize: bad shape groups=%lld rows=%lld cols=%lld", (long long)groups, (long long)rows,
                 (long long)cols);
  LSURGE_REQUIRE(transpose ? (rows % 16 == 0 && cols % 16 == 0) : (rows * cols) % 16 == 0,
                 "fp8_quantize: rows and cols must be multiples of 16 (transposed), rows x cols of 16 (untransposed)");
  LSURGE_REQUIRE(((uintptr_t)x | (uintptr_t)q) % 16 == 0, "fp8_quantize: x and q must be 16-byte aligned");
  LSURGE_REQUIRE(nzero >= 0 && nzero <= QT, "fp8_quantize: too many slots to zero");
  const int64_t n = rows * cols;
  const int nb = amax_parts(n);
  LSURGE_LAUNCH(KID_FP8_QUANT, s,
                hipLaunchKernelGGL(fp8_amax_kernel, dim3(nb, (unsigned)groups), dim3(QT), 0, s, (const bf16_t*)x, n, n,
                                   nb, partial));
  if (transpose) {
    const unsigned tiles = (unsigned)(((rows + 63) / 64) * ((cols + 63) / 64));
    LSURGE_REQUIRE(nzero == 0, "fp8_quantize: transposed cast zeroes no slots");
    LSURGE_LAUNCH(KID_FP8_QUANT, s,
                  hipLaunchKernelGGL(fp8_cast_t_kernel, dim3(tiles, (unsigned)groups), dim3(QT), 0, s, (const bf16_t*)x,
                                     (int)rows, (int)cols, (const float*)partial, nb, (uint8_t*)q, sinv));
  } else {
    const unsigned grid = (unsigned)std::min<int64_t>((n / 16 + QT - 1) / QT, 2048);
    LSURGE_LAUNCH(KID_FP8_QUANT, s,
                  hipLaunchKernelGGL(fp8_cast_kernel, dim3(grid, (unsigned)groups), dim3(QT), 0, s, (const bf16_t*)x, n, n,
                                     (const float*)partial, nb, (uint8_t*)q, sinv, (const int32_t*)nullptr, (int64_t)0,
                                     zero, nzero));
  }
  return LSURGE_OK;
}

int fp8_cast_with_amax(const void* x, int64_t n, const uint32_t* amax_bits, void* q, float* sinv,
                       const int32_t* nrows, int64_t row_elems, hipStream_t s) {
  LSURGE_REQUIRE(n >= 16 && n % 16 == 0, "fp8_cast: n=%lld must be a positive multiple of 16", (long long)n);
  LSURGE_REQUIRE(((uintptr_t)x | (uintptr_t)q) % 16 == 0, "fp8_cast: x and q must be 16-byte aligned");
  const unsigned grid = (unsigned)std::min<int64_t>((n / 16 + QT - 1) / QT, 2048);
  LSURGE_LAUNCH(KID_FP8_QUANT, s,
                hipLaunchKernelGGL(fp8_cast_kernel, dim3(grid, 1), dim3(QT), 0, s, (const bf16_t*)x, n, n,
                                   (const float*)amax_bits, 1, (uint8_t*)q, sinv, nrows, row_elems, (uint32_t*)nullptr, 0));
  return LSURGE_OK;
}

}  // namespace lsurge

extern "C" {

size_t lsurge_fp8_quantize_workspace_bytes(int64_t groups, int64_t rows, int64_t cols) {
  (void)rows;
  (void)cols;
  return groups >= 1 ? lsurge::fp8_partial_bytes(groups) : 0;
}

int lsurge_fp8_quantize(const void* x, int64_t groups, int64_t rows, int64_t cols, int transpose, void* q,
                        float* scale_inv, void* workspace, size_t workspace_bytes, lsurge_stream_t stream) {
  LSURGE_REQUIRE(x && q && scale_inv && workspace, "fp8_quantize: null pointer");
  const size_t need = lsurge_fp8_quantize_workspace_bytes(groups, rows, cols);
  LSURGE_REQUIRE(workspace_bytes >= need, "fp8_quantize: workspace %zu < %zu bytes", workspace_bytes, need);
  return lsurge::fp8_quantize_impl(x, groups, rows, cols, transpose != 0, q, scale_inv, (float*)workspace,
                                   (hipStream_t)stream, nullptr, 0);
}

}  // extern "C"
