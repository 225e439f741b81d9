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

// scale of a group from its amax partials (every thread gets it); E5: the power-of-two E5M2 scale of gradients
template <bool E5 = false>
__device__ __forceinline__ float group_scale(const float* partial, int nparts, float* sh) {
  if (nparts < 0) return partial[0];  // the scale itself
  float m = 0.f;
  for (int i = threadIdx.x; i < nparts; i += blockDim.x) m = fmaxf(m, partial[i]);
  const float amax = block_max(m, sh);
  if constexpr (E5) return e5m2_scale(amax);
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

// four scaled floats -> E4M3, or E5M2 (gradients: common.h) with E5
template <bool E5>
__device__ __forceinline__ uint32_t f8x4(float a, float b, float c, float d) {
  if constexpr (E5) return e5m2x4(a, b, c, d);
  else return e4m3x4(a, b, c, d);
}

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
// with nrows set, only the first nrows[0] * row_elems).  Block (0, g) writes sinv[g] (and scale_out[g] when set:
// the backward casts the same tensor again with it); block (0, 0) zeroes zero[0 .. nzero) (slots a later kernel
// fills by atomic max).  E5: E5M2 codes with the power-of-two scale (gradients).
template <bool E5 = false>
__global__ __launch_bounds__(QT) void fp8_cast_kernel(const bf16_t* __restrict__ x, int64_t n, int64_t gstride,
                                                      const float* __restrict__ partial, int nparts,
                                                      uint8_t* __restrict__ q, float* __restrict__ sinv,
                                                      const int32_t* __restrict__ nrows, int64_t row_elems,
                                                      uint32_t* __restrict__ zero, int nzero,
                                                      float* __restrict__ scale_out) {
  __shared__ float sh[QT / 64];
  const int g = blockIdx.y;
  const float scale = group_scale<E5>(partial + (int64_t)g * max(nparts, 0), nparts, sh);
  if (blockIdx.x == 0 && threadIdx.x == 0 && sinv) {
    sinv[g] = __fdiv_rn(1.f, scale);
    if (scale_out) scale_out[g] = scale;
  }
  if (blockIdx.x == 0 && g == 0 && (int)threadIdx.x < nzero) zero[threadIdx.x] = 0u;
  const int64_t ne = nrows ? min(n, (int64_t)max(nrows[0], 0) * row_elems) : n;
  const bf16_t* xg = x + (int64_t)g * gstride;
  uint8_t* qg = q + (int64_t)g * n;
  // two 16-element chunks per thread and step (four 16-byte loads in flight)
  const int64_t nc = ne / 16, stride = (int64_t)gridDim.x * QT;
  for (int64_t c = (int64_t)blockIdx.x * QT + threadIdx.x; c < nc; c += 2 * stride) {
    const bool two = c + stride < nc;
    u32x4 v[4];
    v[0] = *reinterpret_cast<const u32x4*>(xg + 16 * c);
    v[1] = *reinterpret_cast<const u32x4*>(xg + 16 * c + 8);
    if (two) {
      v[2] = *reinterpret_cast<const u32x4*>(xg + 16 * (c + stride));
      v[3] = *reinterpret_cast<const u32x4*>(xg + 16 * (c + stride) + 8);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (h == 1 && !two) break;
      const u32x4 v0 = v[2 * h], v1 = v[2 * h + 1];
      u32x4 o;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        o[i] = f8x4<E5>(bf_lo(v0[2 * i]) * scale, bf_hi(v0[2 * i]) * scale, bf_lo(v0[2 * i + 1]) * scale,
                        bf_hi(v0[2 * i + 1]) * scale);
        o[i + 2] = f8x4<E5>(bf_lo(v1[2 * i]) * scale, bf_hi(v1[2 * i]) * scale, bf_lo(v1[2 * i + 1]) * scale,
                            bf_hi(v1[2 * i + 1]) * scale);
      }
      *reinterpret_cast<u32x4*>(qg + 16 * (c + h * stride)) = o;
    }
  }
}

// transposed cast: group g of x is [R, C] bf16 -> q group g [C, R] e4m3 (R, C multiples of 16); one 64 x 64 tile per
// workgroup (grid (tiles, G), edge tiles partial), staged through LDS as scaled floats (pitch 65: both directions
// conflict-free).  With q_nt set the same codes also go out untransposed, [R, C] per group (a weight's forward
// operand and its backward operand from one read, with one scale).
__global__ __launch_bounds__(QT) void fp8_cast_t_kernel(const bf16_t* __restrict__ x, int R, int C,
                                                        const float* __restrict__ partial, int nparts,
                                                        uint8_t* __restrict__ q, float* __restrict__ sinv,
                                                        uint8_t* __restrict__ q_nt) {
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
    if (q_nt) {
      u32x4 o;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        o[i] = e4m3x4(bf_lo(v0[2 * i]) * scale, bf_hi(v0[2 * i]) * scale, bf_lo(v0[2 * i + 1]) * scale,
                      bf_hi(v0[2 * i + 1]) * scale);
        o[i + 2] = e4m3x4(bf_lo(v1[2 * i]) * scale, bf_hi(v1[2 * i]) * scale, bf_lo(v1[2 * i + 1]) * scale,
                          bf_hi(v1[2 * i + 1]) * scale);
      }
      *reinterpret_cast<u32x4*>(q_nt + (int64_t)g * R * C + (int64_t)(r0 + rr) * C + c0 + cq) = o;
    }
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

// ---------------------------------------------------------------------------------------------------- backward casts
// The FP8 backward quantises tensors of the padded row layout (dY, [dG | dU], h) and the rows of x gathered into it.
// Padding rows hold no data there, so these kernels read row r only when r < nrows[0] nmul (the real blocks) and
// row_src[r] >= 0 (zeros otherwise), and they take the format as a template argument: E4M3 for activations (largest 448), E5M2 for
// gradients (largest 57344), the hybrid format of Transformer Engine's FP8 training.

// amax partials of the valid rows of a [rows, cols] bf16 matrix (cols % 8 == 0): row r is read from x row
// row_src[r] / kdiv when gathered, else row r itself; grid-strided 8-element chunks, one partial per block.  Block 0
// also zeroes zero[0 .. nzero) (slots a later kernel fills by atomic max).
__global__ __launch_bounds__(QT) void fp8_amax_rows_kernel(const bf16_t* __restrict__ x, int64_t cols,
                                                           const int32_t* __restrict__ nrows, int nmul, int64_t rows,
                                                           const int32_t* __restrict__ row_src, int kdiv, bool gather,
                                                           float* __restrict__ partial, uint32_t* __restrict__ zero,
                                                           int nzero) {
  __shared__ float sh[QT / 64];
  if (blockIdx.x == 0 && (int)threadIdx.x < nzero) zero[threadIdx.x] = 0u;
  const int64_t nr = nrows ? min(rows, (int64_t)max(nrows[0], 0) * nmul) : rows;
  const int64_t cpr = cols / 8, nc = nr * cpr;
  float m = 0.f;
  for (int64_t c = (int64_t)blockIdx.x * QT + threadIdx.x; c < nc; c += (int64_t)gridDim.x * QT) {
    const int64_t r = c / cpr;
    const int src = row_src ? row_src[r] : (int)r;
    if (src < 0) continue;
    const int64_t xr = gather ? src / kdiv : r;
    const u32x4 v = *reinterpret_cast<const u32x4*>(x + xr * cols + 8 * (c % cpr));
#pragma unroll
    for (int i = 0; i < 4; ++i) m = fmaxf(m, fmaxf(fabsf(bf_lo(v[i])), fabsf(bf_hi(v[i]))));
  }
  m = block_max(m, sh);
  if (threadIdx.x == 0) partial[blockIdx.x] = m;
}

// The scale of a cast, from nparts > 0 amax partials, from one amax slot (nparts == 0: float bits written by an
// atomic max), or given (nparts < 0: src[0] is the scale an earlier cast of the same tensor used, so that a second
// copy of it holds the same codes).  E5M2 (gradient) scales are rounded down to a power of two (Transformer
// Engine's power-of-two option of current scaling): a gradient's amax is one element produced by a GEMM, and a
// one-ulp change of it would otherwise move the whole tensor's quantisation grid; a power-of-two scale only moves
// when the amax crosses a binade, and it dequantises exactly.
template <bool E5>
__device__ __forceinline__ float cast_scale(const float* src, int nparts, float* sh) {
  if (nparts < 0) return src[0];
  float amax;
  if (nparts > 0) {
    float m = 0.f;
    for (int i = threadIdx.x; i < nparts; i += blockDim.x) m = fmaxf(m, src[i]);
    amax = block_max(m, sh);
  } else {
    amax = src[0];
  }
  if constexpr (E5) return e5m2_scale(amax);
  if (!(amax > 0.f)) return 1.f;
  const float s = __fdiv_rn(448.f, amax);
  return s <= FLT_MAX ? s : FLT_MAX;
}

// Cast of the valid rows of a [rows, cols] bf16 matrix (row r read from x row row_src[r] / kdiv when gathered) into
// a row-wise copy qr [rows, cols] (optional) and a transposed copy qt [cols, ldq] (optional, element (c, r)).  Rows
// past nrows[0] nmul or with row_src < 0 become zeros, up to the 64-row tile bound of the valid rows.  One 64 x 64 tile per
// workgroup over the host-side bound of rows; the transpose is staged through LDS as scaled floats (pitch 65).
// cols % 16 == 0; ldq >= rows rounded up to 64.  Block 0 writes sinv[0] (and scale_out[0] when set).
template <bool E5>
__global__ __launch_bounds__(QT) void fp8_cast_rows_kernel(const bf16_t* __restrict__ x, int64_t rows, int64_t cols,
                                                           const int32_t* __restrict__ nrows, int nmul,
                                                           const int32_t* __restrict__ row_src, int kdiv, bool gather,
                                                           const float* __restrict__ src, int nparts,
                                                           uint8_t* __restrict__ qr, uint8_t* __restrict__ qt,
                                                           int64_t ldq, float* __restrict__ sinv,
                                                           float* __restrict__ scale_out) {
  __shared__ float sh[QT / 64];
  __shared__ float t[64][65];
  const float scale = cast_scale<E5>(src, nparts, sh);
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    sinv[0] = __fdiv_rn(1.f, scale);
    if (scale_out) scale_out[0] = scale;
  }
  const int64_t nr = nrows ? min(rows, (int64_t)max(nrows[0], 0) * nmul) : rows;
  const int64_t ct = (cols + 63) / 64;
  const int64_t r0 = (int64_t)(blockIdx.x / ct) * 64, c0 = (int64_t)(blockIdx.x % ct) * 64;
  if (r0 >= (nr + 63) / 64 * 64) return;  // tiles past the valid rows' tile bound are never read
  const int tid = threadIdx.x, rr = tid >> 2, cq = 16 * (tid & 3);
  u32x4 v0 = {0u, 0u, 0u, 0u}, v1 = {0u, 0u, 0u, 0u};
  const int64_t r = r0 + rr;
  const bool cin = c0 + cq < cols;
  if (r < nr && cin) {
    const int sr = row_src ? row_src[r] : (int)r;
    if (sr >= 0) {
      const bf16_t* p = x + (gather ? (int64_t)(sr / kdiv) : r) * cols + c0 + cq;
      v0 = *reinterpret_cast<const u32x4*>(p);
      v1 = *reinterpret_cast<const u32x4*>(p + 8);
    }
  }
  if (qr && r < rows && cin) {
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      o[i] = f8x4<E5>(bf_lo(v0[2 * i]) * scale, bf_hi(v0[2 * i]) * scale, bf_lo(v0[2 * i + 1]) * scale,
                      bf_hi(v0[2 * i + 1]) * scale);
      o[i + 2] = f8x4<E5>(bf_lo(v1[2 * i]) * scale, bf_hi(v1[2 * i]) * scale, bf_lo(v1[2 * i + 1]) * scale,
                          bf_hi(v1[2 * i + 1]) * scale);
    }
    *reinterpret_cast<u32x4*>(qr + r * cols + c0 + cq) = o;
  }
  if (!qt) return;  // uniform
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    t[cq + 2 * i][rr] = bf_lo(v0[i]) * scale;
    t[cq + 2 * i + 1][rr] = bf_hi(v0[i]) * scale;
    t[cq + 8 + 2 * i][rr] = bf_lo(v1[i]) * scale;
    t[cq + 8 + 2 * i + 1][rr] = bf_hi(v1[i]) * scale;
  }
  __syncthreads();
  if (c0 + rr >= cols) return;
  const float* row = &t[rr][cq];  // output row c0 + rr, elements r0 + cq .. + 15 (zeros past nrows)
  u32x4 o;
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = f8x4<E5>(row[4 * i], row[4 * i + 1], row[4 * i + 2], row[4 * i + 3]);
  *reinterpret_cast<u32x4*>(qt + (c0 + rr) * ldq + r0 + cq) = o;
}

// blocks per group: about two steps of AU chunks per thread
int amax_parts(int64_t n) {
  return (int)std::min<int64_t>(MAX_PARTS, std::max<int64_t>(1, (n / 8 + 2 * AU * QT - 1) / (2 * AU * QT)));
}

}  // namespace

namespace lsurge {

size_t fp8_partial_bytes(int64_t groups) { return sizeof(float) * (size_t)groups * MAX_PARTS; }

int fp8_quantize_impl(const void* x, int64_t groups, int64_t rows, int64_t cols, bool transpose, void* q, float* sinv,
                      float* partial, hipStream_t s, uint32_t* zero, int nzero, void* q_nt, float* scale_out) {
  LSURGE_REQUIRE(groups >= 1 && groups < 65536 && rows >= 1 && cols >= 1 && rows < (1 << 30) && cols < (1 << 30) &&
                     rows * cols < (1ll << 40),
                 "fp8_quantize: bad shape groups=%lld rows=%lld cols=%lld", (long long)groups, (long long)rows,
                 (long long)cols);
  LSURGE_REQUIRE(transpose ? (rows % 16 == 0 && cols % 16 == 0) : (rows * cols) % 16 == 0,
                 "fp8_quantize: rows and cols must be multiples of 16 (transposed), rows x cols of 16 (untransposed)");
  LSURGE_REQUIRE(((uintptr_t)x | (uintptr_t)q | (uintptr_t)q_nt) % 16 == 0, "fp8_quantize: x and q must be 16-byte aligned");
  LSURGE_REQUIRE(nzero >= 0 && nzero <= QT, "fp8_quantize: too many slots to zero");
  LSURGE_REQUIRE(!q_nt || transpose, "fp8_quantize: the untransposed second copy comes with the transposed cast");
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
                                     (int)rows, (int)cols, (const float*)partial, nb, (uint8_t*)q, sinv,
                                     (uint8_t*)q_nt));
  } else {
    const unsigned grid = (unsigned)std::min<int64_t>((n / 16 + QT - 1) / QT, 2048);
    LSURGE_LAUNCH(KID_FP8_QUANT, s,
                  hipLaunchKernelGGL(fp8_cast_kernel<false>, dim3(grid, (unsigned)groups), dim3(QT), 0, s, (const bf16_t*)x, n, n,
                                     (const float*)partial, nb, (uint8_t*)q, sinv, (const int32_t*)nullptr, (int64_t)0,
                                     zero, nzero, scale_out));
  }
  return LSURGE_OK;
}

int fp8_cast_with_amax(const void* x, int64_t n, const uint32_t* amax_bits, void* q, float* sinv,
                       const int32_t* nrows, int64_t row_elems, hipStream_t s, float* scale_out) {
  LSURGE_REQUIRE(n >= 16 && n % 16 == 0, "fp8_cast: n=%lld must be a positive multiple of 16", (long long)n);
  LSURGE_REQUIRE(((uintptr_t)x | (uintptr_t)q) % 16 == 0, "fp8_cast: x and q must be 16-byte aligned");
  const unsigned grid = (unsigned)std::min<int64_t>((n / 16 + QT - 1) / QT, 2048);
  LSURGE_LAUNCH(KID_FP8_QUANT, s,
                hipLaunchKernelGGL(fp8_cast_kernel<false>, dim3(grid, 1), dim3(QT), 0, s, (const bf16_t*)x, n, n,
                                   (const float*)amax_bits, 1, (uint8_t*)q, sinv, nrows, row_elems, (uint32_t*)nullptr, 0,
                                   scale_out));
  return LSURGE_OK;
}

int fp8_amax_rows(const void* x, int64_t rows, int64_t cols, const int32_t* nrows, int nmul, const int32_t* row_src,
                  int kdiv, bool gather, float* partial, hipStream_t s, uint32_t* zero, int nzero) {
  LSURGE_REQUIRE(rows >= 1 && cols >= 8 && cols % 8 == 0 && kdiv >= 1 && nmul >= 1 && nzero >= 0 && nzero <= QT,
                 "fp8_amax_rows: bad shape rows=%lld cols=%lld", (long long)rows, (long long)cols);
  LSURGE_REQUIRE((uintptr_t)x % 16 == 0, "fp8_amax_rows: x must be 16-byte aligned");
  const int nb = (int)std::min<int64_t>(MAX_PARTS, std::max<int64_t>(1, (rows * cols / 8 + 2 * QT - 1) / (2 * QT)));
  LSURGE_LAUNCH(KID_FP8_QUANT, s,
                hipLaunchKernelGGL(fp8_amax_rows_kernel, dim3(nb), dim3(QT), 0, s, (const bf16_t*)x, cols, nrows, nmul,
                                   rows, row_src, kdiv, gather, partial, zero, nzero));
  return nb;
}

int fp8_cast_rows(const void* x, int64_t rows, int64_t cols, const int32_t* nrows, int nmul, const int32_t* row_src,
                  int kdiv, bool gather, const float* src, int nparts, bool e5m2, void* qr, void* qt, int64_t ldq,
                  float* sinv, float* scale_out, hipStream_t s) {
  LSURGE_REQUIRE(rows >= 1 && cols >= 16 && cols % 16 == 0 && kdiv >= 1 && nmul >= 1 && (qr || qt) && src && sinv &&
                     (!qt || (ldq >= (rows + 63) / 64 * 64 && ldq % 16 == 0)),
                 "fp8_cast_rows: bad shape rows=%lld cols=%lld ldq=%lld", (long long)rows, (long long)cols,
                 (long long)ldq);
  LSURGE_REQUIRE(((uintptr_t)x | (uintptr_t)qr | (uintptr_t)qt) % 16 == 0, "fp8_cast_rows: 16-byte alignment");
  LSURGE_REQUIRE(rows < (1ll << 31) && cols < (1ll << 31) && (rows + 63) / 64 * ((cols + 63) / 64) < (1ll << 31),
                 "fp8_cast_rows: too many tiles");
  const unsigned tiles = (unsigned)(((rows + 63) / 64) * ((cols + 63) / 64));
  if (e5m2)
    LSURGE_LAUNCH(KID_FP8_QUANT, s, hipLaunchKernelGGL(fp8_cast_rows_kernel<true>, dim3(tiles), dim3(QT), 0, s,
                                                       (const bf16_t*)x, rows, cols, nrows, nmul, row_src, kdiv, gather, src,
                                                       nparts, (uint8_t*)qr, (uint8_t*)qt, ldq, sinv, scale_out));
  else
    LSURGE_LAUNCH(KID_FP8_QUANT, s, hipLaunchKernelGGL(fp8_cast_rows_kernel<false>, dim3(tiles), dim3(QT), 0, s,
                                                       (const bf16_t*)x, rows, cols, nrows, nmul, row_src, kdiv, gather, src,
                                                       nparts, (uint8_t*)qr, (uint8_t*)qt, ldq, sinv, scale_out));
  return LSURGE_OK;
}

size_t fp8_rows_partial_bytes() { return sizeof(float) * MAX_PARTS; }

int fp8_amax(const void* x, int64_t n, float* partial, hipStream_t s) {
  LSURGE_REQUIRE(n >= 8 && n % 8 == 0 && (uintptr_t)x % 16 == 0, "fp8_amax: n=%lld", (long long)n);
  const int nb = amax_parts(n);
  LSURGE_LAUNCH(KID_FP8_QUANT, s,
                hipLaunchKernelGGL(fp8_amax_kernel, dim3(nb, 1), dim3(QT), 0, s, (const bf16_t*)x, n, n, nb, partial));
  return nb;
}

int fp8_cast_e5m2(const void* x, int64_t n, const float* amax, int nparts, void* q, float* sinv, const int32_t* nrows,
                  int64_t row_elems, hipStream_t s, uint32_t* zero, int nzero) {
  LSURGE_REQUIRE(n >= 16 && n % 16 == 0 && nparts != 0 && nzero >= 0 && nzero <= QT,
                 "fp8_cast_e5m2: n=%lld must be a positive multiple of 16", (long long)n);
  LSURGE_REQUIRE(((uintptr_t)x | (uintptr_t)q) % 16 == 0, "fp8_cast_e5m2: x and q must be 16-byte aligned");
  const unsigned grid = (unsigned)std::min<int64_t>((n / 16 + QT - 1) / QT, 4096);
  LSURGE_LAUNCH(KID_FP8_QUANT, s,
                hipLaunchKernelGGL(fp8_cast_kernel<true>, dim3(grid, 1), dim3(QT), 0, s, (const bf16_t*)x, n, n, amax,
                                   nparts, (uint8_t*)q, sinv, nrows, row_elems, zero, nzero, (float*)nullptr));
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

size_t lsurge_fp8_cast_workspace_bytes(void) { return lsurge::fp8_rows_partial_bytes(); }

int lsurge_fp8_cast_transpose(const void* x, int64_t rows, int64_t cols, int format, void* q, void* qt, int64_t ldqt,
                              float* scale_inv, void* workspace, size_t workspace_bytes, lsurge_stream_t stream) {
  LSURGE_REQUIRE(x && scale_inv && workspace && (q || qt), "fp8_cast_transpose: null pointer");
  LSURGE_REQUIRE(format == LSURGE_FP8_E4M3 || format == LSURGE_FP8_E5M2, "fp8_cast_transpose: format %d", format);
  LSURGE_REQUIRE(workspace_bytes >= lsurge::fp8_rows_partial_bytes(), "fp8_cast_transpose: workspace %zu < %zu bytes",
                 workspace_bytes, lsurge::fp8_rows_partial_bytes());
  LSURGE_REQUIRE(rows >= 1 && cols >= 16 && cols % 16 == 0, "fp8_cast_transpose: rows=%lld, cols=%lld (multiple of 16)",
                 (long long)rows, (long long)cols);
  hipStream_t s = (hipStream_t)stream;
  float* part = (float*)workspace;
  const int nb = lsurge::fp8_amax_rows(x, rows, cols, nullptr, 1, nullptr, 1, false, part, s);
  if (nb < 0) return nb;
  return lsurge::fp8_cast_rows(x, rows, cols, nullptr, 1, nullptr, 1, false, part, nb, format == LSURGE_FP8_E5M2, q,
                               qt, ldqt, scale_inv, nullptr, s);
}

}  // extern "C"
