// Memory-bound row movement: gather_rows, gather_reduce, gather_dot, fused combine backward, and the
// padded-layout dispatch / combine / dispatch-backward used by the fused layer.
//
// Replaces the Pallas-TPU row-DMA kernels of modal/moe_permute.py:116-234 (gather_rows, _reduce_like).
// On CDNA a row is moved by one wave with 16-byte vector accesses (coalesced 1 KiB per instruction); there
// is no need for the TPU's bf16 u32 packing (moe_permute.py:68-84).  All reductions run in f32 with the
// choice index j ascending, the order of moe_permute.py:189-200.
#include "launchers.h"

namespace {

constexpr int PM_THREADS = 256;
constexpr int PM_WAVES = PM_THREADS / 64;

// 8 consecutive elements <-> 8 floats
template <int DT> struct V8;
// (Raw / ldraw / cvt: the load and the conversion apart, so that a batch of loads is in flight before any is used)
template <> struct V8<LSURGE_BF16> {
  typedef u32x4 Raw;
  static __device__ __forceinline__ Raw ldraw(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
  static __device__ __forceinline__ void cvt(const Raw& u, float* v) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(u[i] << 16);
      v[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
    }
  }
  static __device__ __forceinline__ void ld(const void* p, float* v) { cvt(ldraw(p), v); }
  static __device__ __forceinline__ void st(void* p, const float* v) {
    u32x4 u;
#pragma unroll
    for (int i = 0; i < 4; ++i) u[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
    *reinterpret_cast<u32x4*>(p) = u;
  }
};
template <> struct V8<LSURGE_F16> {
  typedef u32x4 Raw;
  static __device__ __forceinline__ Raw ldraw(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
  static __device__ __forceinline__ void cvt(const Raw& u, float* v) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = f16_to_f32((uint16_t)(u[i] & 0xffffu));
      v[2 * i + 1] = f16_to_f32((uint16_t)(u[i] >> 16));
    }
  }
  static __device__ __forceinline__ void ld(const void* p, float* v) { cvt(ldraw(p), v); }
  static __device__ __forceinline__ void st(void* p, const float* v) {
    u32x4 u;
#pragma unroll
    for (int i = 0; i < 4; ++i) u[i] = (uint32_t)f32_to_f16(v[2 * i]) | ((uint32_t)f32_to_f16(v[2 * i + 1]) << 16);
    *reinterpret_cast<u32x4*>(p) = u;
  }
};
template <> struct V8<LSURGE_F32> {
  struct Raw {
    f32x4 a, b;
  };
  static __device__ __forceinline__ Raw ldraw(const void* p) {
    return Raw{reinterpret_cast<const f32x4*>(p)[0], reinterpret_cast<const f32x4*>(p)[1]};
  }
  static __device__ __forceinline__ void cvt(const Raw& r, float* v) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = r.a[i];
      v[4 + i] = r.b[i];
    }
  }
  static __device__ __forceinline__ void ld(const void* p, float* v) { cvt(ldraw(p), v); }
  static __device__ __forceinline__ void st(void* p, const float* v) {
    f32x4 a, b;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[i] = v[i];
      b[i] = v[4 + i];
    }
    reinterpret_cast<f32x4*>(p)[0] = a;
    reinterpret_cast<f32x4*>(p)[1] = b;
  }
};

template <int DT> constexpr int esize() { return DT == LSURGE_F32 ? 4 : 2; }

// value after a round trip through element type DT
template <int DT> __device__ __forceinline__ float round_to(float v) {
  if (DT == LSURGE_BF16) return bf16_to_f32(f32_to_bf16(v));
  if (DT == LSURGE_F16) return f16_to_f32(f32_to_f16(v));
  return v;
}

// ------------------------------------------------------------------------------ gather_rows
// out[i] = x[idx[i]] (byte copy), or round(f32(x[idx[i]]) * scale[i]).  An index outside [0, n) gives a zero
// row (padded_gmm's zero-row sentinel, modal/padded_gmm.py:26-28).
template <int DT, bool VEC>
__global__ __launch_bounds__(PM_THREADS) void gather_rows_kernel(const void* __restrict__ x, int64_t n, int64_t d,
                                                                 const int32_t* __restrict__ idx, int64_t m,
                                                                 const float* __restrict__ scale,
                                                                 void* __restrict__ out) {
  constexpr int ES = esize<DT>();
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * PM_WAVES + (threadIdx.x >> 6);
  const int64_t nwaves = (int64_t)gridDim.x * PM_WAVES;
  for (int64_t i = wave; i < m; i += nwaves) {
    const int64_t src = idx[i];
    const char* xr = (const char*)x + src * d * ES;
    char* orow = (char*)out + i * d * ES;
    if (src < 0 || src >= n) {
      if (VEC) {
        for (int64_t c = lane * 8; c < d; c += 64 * 8)
          for (int h = 0; h < ES * 8 / 16; ++h) reinterpret_cast<u32x4*>(orow + c * ES)[h] = u32x4{0, 0, 0, 0};
      } else {
        typedef typename Elem<DT>::T T;
        for (int64_t c = lane; c < d; c += 64) ((T*)orow)[c] = (T)0;
      }
      continue;
    }
    if (VEC) {
      if (!scale) {
        for (int64_t c = lane * 8; c < d; c += 64 * 8)
          for (int h = 0; h < ES * 8 / 16; ++h)
            reinterpret_cast<u32x4*>(orow + c * ES)[h] = reinterpret_cast<const u32x4*>(xr + c * ES)[h];
      } else {
        const float sc = scale[i];
        for (int64_t c = lane * 8; c < d; c += 64 * 8) {
          float v[8];
          V8<DT>::ld(xr + c * ES, v);
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] *= sc;
          V8<DT>::st(orow + c * ES, v);
        }
      }
    } else {
      typedef typename Elem<DT>::T T;
      const T* xs = (const T*)xr;
      T* os = (T*)orow;
      if (!scale) {
        for (int64_t c = lane; c < d; c += 64) os[c] = xs[c];
      } else {
        const float sc = scale[i];
        for (int64_t c = lane; c < d; c += 64) Elem<DT>::st(os, c, Elem<DT>::ld(xs, c) * sc);
      }
    }
  }
}

// ------------------------------------------------------------------------------ gather_reduce / dot
constexpr int GK = 8;   // choices whose row loads are issued together
// 512-column chunks of a row per pass: GK x GCH row loads in flight per lane.  Measured at the reference microbench's
// shapes: two chunks make gather_reduce 2% faster and gather_dot 3% slower than one.
constexpr int GCH_REDUCE = 2, GCH_DOT = 1;
template <int DT, int OT, bool VEC>
__global__ __launch_bounds__(PM_THREADS) void gather_reduce_kernel(const void* __restrict__ y, int64_t m, int64_t d,
                                                                   const int32_t* __restrict__ pos, int64_t n, int k,
                                                                   const float* __restrict__ w,
                                                                   void* __restrict__ out) {
  constexpr int ES = esize<DT>(), OS = esize<OT>();
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * PM_WAVES + (threadIdx.x >> 6);
  const int64_t nwaves = (int64_t)gridDim.x * PM_WAVES;
  for (int64_t t = wave; t < n; t += nwaves) {
    if (VEC) {
      for (int64_t c0 = lane * 8; c0 < d; c0 += GCH_REDUCE * 64 * 8) {
        float acc[GCH_REDUCE][8];
#pragma unroll
        for (int h = 0; h < GCH_REDUCE; ++h)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;
        for (int j0 = 0; j0 < k; j0 += GK) {
          // a batch of GK choices over GCH_REDUCE column chunks: positions first, then every row load, then the sums in
          // ascending j, so no row load waits for another.  An out-of-range position contributes nothing (its
          // load reads row 0).
          int64_t src[GK];
          bool ok[GK];
          float wj[GK];
#pragma unroll
          for (int q = 0; q < GK; ++q) {
            const int j = j0 + q;
            const int64_t r = j < k ? pos[t * k + j] : -1;
            ok[q] = r >= 0 && r < m;
            src[q] = ok[q] ? r : 0;
            wj[q] = (w && j < k) ? w[t * k + j] : 1.f;
          }
          typename V8<DT>::Raw raw[GCH_REDUCE][GK];
#pragma unroll
          for (int h = 0; h < GCH_REDUCE; ++h)
#pragma unroll
            for (int q = 0; q < GK; ++q)
              if (m > 0 && j0 + q < k && c0 + 512 * h < d)
                raw[h][q] = V8<DT>::ldraw((const char*)y + (src[q] * d + c0 + 512 * h) * ES);
#pragma unroll
          for (int h = 0; h < GCH_REDUCE; ++h) {
            if (c0 + 512 * h >= d) break;
#pragma unroll
            for (int q = 0; q < GK; ++q) {
              if (!ok[q]) continue;
              float v[8];
              V8<DT>::cvt(raw[h][q], v);
#pragma unroll
              for (int e = 0; e < 8; ++e) acc[h][e] = w ? acc[h][e] + wj[q] * v[e] : acc[h][e] + v[e];
            }
          }
        }
#pragma unroll
        for (int h = 0; h < GCH_REDUCE; ++h)
          if (c0 + 512 * h < d) V8<OT>::st((char*)out + (t * d + c0 + 512 * h) * OS, acc[h]);
      }
    } else {
      typedef typename Elem<DT>::T T;
      typedef typename Elem<OT>::T O;
      for (int64_t c = lane; c < d; c += 64) {
        float acc = 0.f;
        for (int j = 0; j < k; ++j) {
          const int64_t r = pos[t * k + j];
          if (r < 0 || r >= m) continue;
          const float v = Elem<DT>::ld((const T*)y, r * d + c);
          acc = w ? acc + w[t * k + j] * v : acc + v;
        }
        Elem<OT>::st((O*)out, t * d + c, acc);
      }
    }
  }
}

template <int DT, int GT, bool VEC>
__global__ __launch_bounds__(PM_THREADS) void gather_dot_kernel(const void* __restrict__ y, int64_t m, int64_t d,
                                                                const int32_t* __restrict__ pos, int64_t n, int k,
                                                                const void* __restrict__ g,
                                                                float* __restrict__ out) {
  constexpr int ES = esize<DT>(), GS = esize<GT>();
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * PM_WAVES + (threadIdx.x >> 6);
  const int64_t nwaves = (int64_t)gridDim.x * PM_WAVES;
  for (int64_t t = wave; t < n; t += nwaves) {
    for (int j0 = 0; j0 < k; j0 += GK) {
      // a batch of GK choices, as in gather_reduce: positions first, then the row loads of every choice per column
      // chunk; an out-of-range position gives the dot product 0
      int64_t src[GK];
      bool ok[GK];
#pragma unroll
      for (int q = 0; q < GK; ++q) {
        const int64_t r = j0 + q < k ? pos[t * k + j0 + q] : -1;
        ok[q] = r >= 0 && r < m;
        src[q] = ok[q] ? r : 0;
      }
      float acc[GK];
#pragma unroll
      for (int q = 0; q < GK; ++q) acc[q] = 0.f;
      if (VEC) {
        for (int64_t c0 = lane * 8; c0 < d; c0 += GCH_DOT * 64 * 8) {
          typename V8<GT>::Raw graw[GCH_DOT];
          typename V8<DT>::Raw raw[GCH_DOT][GK];
#pragma unroll
          for (int h = 0; h < GCH_DOT; ++h) {
            const int64_t c = c0 + 512 * h;
            if (c >= d) continue;
            graw[h] = V8<GT>::ldraw((const char*)g + (t * d + c) * GS);
#pragma unroll
            for (int q = 0; q < GK; ++q)
              if (m > 0 && j0 + q < k) raw[h][q] = V8<DT>::ldraw((const char*)y + (src[q] * d + c) * ES);
          }
#pragma unroll
          for (int h = 0; h < GCH_DOT; ++h) {
            if (c0 + 512 * h >= d) break;
            float gv[8];
            V8<GT>::cvt(graw[h], gv);
#pragma unroll
            for (int q = 0; q < GK; ++q) {
              if (!ok[q]) continue;
              float v[8];
              V8<DT>::cvt(raw[h][q], v);
#pragma unroll
              for (int e = 0; e < 8; ++e) acc[q] += v[e] * gv[e];
            }
          }
        }
      } else {
        typedef typename Elem<DT>::T T;
        typedef typename Elem<GT>::T G;
#pragma unroll
        for (int q = 0; q < GK; ++q)
          if (ok[q])
            for (int64_t c = lane; c < d; c += 64)
              acc[q] += Elem<DT>::ld((const T*)y, src[q] * d + c) * Elem<GT>::ld((const G*)g, t * d + c);
      }
#pragma unroll
      for (int q = 0; q < GK; ++q) {
        if (j0 + q >= k) break;
        const float sum = wave_sum(acc[q]);
        if (lane == 0) out[t * k + j0 + q] = sum;
      }
    }
  }
}

// ------------------------------------------------------------------------------ fused combine backward
// One wave per token: g[t] is read once; for every j the expert row y[pos] is read, dy[pos] written (dy optional)
// and the dot <g, y[pos]> reduced.  Optionally also the router backward dl[t,j] = w_j (dw_j - sum_i w_i dw_i).
template <int DT, int GT, bool VEC>
__global__ __launch_bounds__(PM_THREADS) void combine_bwd_kernel(const void* __restrict__ y, int64_t m,
                                                                 const int32_t* __restrict__ pos,
                                                                 const float* __restrict__ w, int64_t n, int k,
                                                                 int64_t d, const void* __restrict__ g,
                                                                 void* __restrict__ dy, float* __restrict__ dw,
                                                                 float* __restrict__ dl) {
  constexpr int ES = esize<DT>(), GS = esize<GT>();
  typedef typename Elem<DT>::T T;
  typedef typename Elem<GT>::T G;
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * PM_WAVES + (threadIdx.x >> 6);
  const int64_t nwaves = (int64_t)gridDim.x * PM_WAVES;
  for (int64_t t = wave; t < n; t += nwaves) {
    float dwv[16];
    for (int j0 = 0; j0 < k; j0 += GK) {
      // a batch of GK choices, as in gather_dot: positions and weights first, then g and the expert rows of every
      // choice per column chunk.  An out-of-range position writes nothing and gives dw = 0.
      int64_t src[GK];
      bool ok[GK];
      float wj[GK], acc[GK];
#pragma unroll
      for (int q = 0; q < GK; ++q) {
        const int j = j0 + q;
        const int64_t r = j < k ? pos[t * k + j] : -1;
        ok[q] = r >= 0 && r < m;
        src[q] = ok[q] ? r : 0;
        wj[q] = j < k ? w[t * k + j] : 0.f;
        acc[q] = 0.f;
      }
      if (VEC) {
        for (int64_t c = lane * 8; c < d; c += 64 * 8) {
          const typename V8<GT>::Raw graw = V8<GT>::ldraw((const char*)g + (t * d + c) * GS);
          typename V8<DT>::Raw raw[GK];
#pragma unroll
          for (int q = 0; q < GK; ++q)
            if (m > 0 && j0 + q < k) raw[q] = V8<DT>::ldraw((const char*)y + (src[q] * d + c) * ES);
          float gv[8];
          V8<GT>::cvt(graw, gv);
          if (GT != DT)
#pragma unroll
            for (int e = 0; e < 8; ++e) gv[e] = round_to<DT>(gv[e]);  // g.astype(y.dtype) first (moe_permute.py:307)
#pragma unroll
          for (int q = 0; q < GK; ++q) {
            if (!ok[q]) continue;
            float v[8], o[8];
            V8<DT>::cvt(raw[q], v);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              acc[q] += v[e] * gv[e];
              o[e] = wj[q] * gv[e];
            }
            if (dy) V8<DT>::st((char*)dy + (src[q] * d + c) * ES, o);
          }
        }
      } else {
#pragma unroll
        for (int q = 0; q < GK; ++q) {
          if (!ok[q]) continue;
          for (int64_t c = lane; c < d; c += 64) {
            float gv = Elem<GT>::ld((const G*)g, t * d + c);
            if (GT != DT) gv = round_to<DT>(gv);
            acc[q] += Elem<DT>::ld((const T*)y, src[q] * d + c) * gv;
            if (dy) Elem<DT>::st((T*)dy, src[q] * d + c, wj[q] * gv);
          }
        }
      }
#pragma unroll
      for (int q = 0; q < GK; ++q) {
        const int j = j0 + q;
        if (j >= k) break;
        const float sum = wave_sum(acc[q]);
        if (j < 16) dwv[j] = sum;
        if (lane == 0 && dw) dw[t * k + j] = sum;
      }
    }
    if (dl && lane == 0) {  // choices past the 16 kept in registers come back from dw (written by this lane)
      float s = 0.f;
      for (int j = 0; j < k; ++j) s += w[t * k + j] * (j < 16 ? dwv[j] : dw[t * k + j]);
      for (int j = 0; j < k; ++j) dl[t * k + j] = w[t * k + j] * ((j < 16 ? dwv[j] : dw[t * k + j]) - s);
    }
  }
}

// ------------------------------------------------------------------------------ padded-layout layer kernels
// One wave per token (or padded row).  A row of d elements is NC chunks of 8 per lane (d == 512 NC) and the
// loop over the k choices is unrolled KK times when NC and KK are compile-time constants (d = 1024 / 2048,
// k = 6 / 8 at the BASELINE configs), so every row load of a token is in flight at once; NC = 0 or KK = 0
// select the run-time loops for other shapes.  The wave's token index is made scalar so the routing
// indices come through the scalar cache.
__device__ __forceinline__ int64_t wave_id() {
  return (int64_t)blockIdx.x * PM_WAVES + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
}

// dispatch: x_pad[r] = x[row_src[r] / k] for valid padded rows of the used blocks (padding rows untouched;
// the GEMMs mask them by blk_rows).
template <int NC>
__global__ __launch_bounds__(PM_THREADS) void dispatch_pad_kernel(const bf16_t* __restrict__ x, int64_t d, int k,
                                                                  const int32_t* __restrict__ row_src,
                                                                  const int32_t* __restrict__ num_blocks,
                                                                  int64_t max_rows, bf16_t* __restrict__ xp) {
  const int lane = threadIdx.x & 63;
  const int64_t nwaves = (int64_t)gridDim.x * PM_WAVES;
  const int64_t rows = min((int64_t)num_blocks[0] * LSURGE_BLOCK_ROWS, max_rows);
  for (int64_t r = wave_id(); r < rows; r += nwaves) {
    const int32_t src = row_src[r];
    if (src < 0) continue;
    const bf16_t* xr = x + (int64_t)(src / k) * d;
    bf16_t* o = xp + r * d;
    if (NC) {
      u32x4 v[NC > 0 ? NC : 1];
#pragma unroll
      for (int c = 0; c < NC; ++c) v[c] = *reinterpret_cast<const u32x4*>(xr + (c * 64 + lane) * 8);
#pragma unroll
      for (int c = 0; c < NC; ++c) *reinterpret_cast<u32x4*>(o + (c * 64 + lane) * 8) = v[c];
    } else {
      for (int64_t c = lane * 8; c < d; c += 64 * 8)
        *reinterpret_cast<u32x4*>(o + c) = *reinterpret_cast<const u32x4*>(xr + c);
    }
  }
}

// combine: out[t] = sum_j w[t,j] * y_pad[slot[t,j]] (+ add[t]), f32 accumulate, j ascending, one rounding.
template <int NC, int KK, int OT>
__global__ __launch_bounds__(PM_THREADS) void combine_pad_kernel(const bf16_t* __restrict__ yp, int64_t d, int k,
                                                                 const int32_t* __restrict__ slot,
                                                                 const float* __restrict__ w, int64_t n,
                                                                 const bf16_t* __restrict__ add,
                                                                 void* __restrict__ out) {
  constexpr int OS = esize<OT>();
  const int lane = threadIdx.x & 63;
  const int64_t nwaves = (int64_t)gridDim.x * PM_WAVES;
  const int kk = KK ? KK : k;
  for (int64_t t = wave_id(); t < n; t += nwaves) {
    if (NC) {
      float acc[NC > 0 ? NC : 1][8] = {};
#pragma unroll
      for (int j = 0; j < (KK ? KK : 1); ++j) {
        if (!KK) break;
        const int64_t r = slot[t * kk + j];
        const float wj = w[t * kk + j];
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          float v[8];
          V8<LSURGE_BF16>::ld(yp + r * d + (c * 64 + lane) * 8, v);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[c][e] += wj * v[e];
        }
      }
      if (!KK) {
        for (int j = 0; j < kk; ++j) {
          const int64_t r = slot[t * kk + j];
          const float wj = w[t * kk + j];
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            float v[8];
            V8<LSURGE_BF16>::ld(yp + r * d + (c * 64 + lane) * 8, v);
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[c][e] += wj * v[e];
          }
        }
      }
      if (add) {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          float v[8];
          V8<LSURGE_BF16>::ld(add + t * d + (c * 64 + lane) * 8, v);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[c][e] += v[e];
        }
      }
#pragma unroll
      for (int c = 0; c < NC; ++c) V8<OT>::st((char*)out + (t * d + (c * 64 + lane) * 8) * OS, acc[c]);
    } else {
      for (int64_t c = lane * 8; c < d; c += 64 * 8) {
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int j = 0; j < kk; ++j) {
          const int64_t r = slot[t * kk + j];
          const float wj = w[t * kk + j];
          float v[8];
          V8<LSURGE_BF16>::ld(yp + r * d + c, v);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[e] += wj * v[e];
        }
        if (add) {
          float v[8];
          V8<LSURGE_BF16>::ld(add + t * d + c, v);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[e] += v[e];
        }
        V8<OT>::st((char*)out + (t * d + c) * OS, acc);
      }
    }
  }
}

// amax of the FP8 backward's dY rows bf16(w[t,j] dy[t]) without forming them: f32 products and bf16 rounding are
// monotonic, so max over (t, j, c) of |bf16(w[t,j] dy[t,c])| = max over t of bf16(max_j |w[t,j]| max_c |dy[t,c]|).  One
// wave per token (grid-strided), one partial per workgroup.  d % 8 == 0.
__global__ __launch_bounds__(PM_THREADS) void dy_rows_amax_kernel(const bf16_t* __restrict__ dy,
                                                                  const float* __restrict__ w, int64_t n, int64_t d,
                                                                  int k, float* __restrict__ partial) {
  __shared__ float sh[PM_WAVES];
  const int lane = threadIdx.x & 63;
  const int64_t nwaves = (int64_t)gridDim.x * PM_WAVES;
  float m = 0.f;
  for (int64_t t = wave_id(); t < n; t += nwaves) {
    float a = 0.f;
    for (int64_t c = 8 * lane; c < d; c += 512) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(dy + t * d + c);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        a = fmaxf(a, fmaxf(fabsf(__uint_as_float(v[i] << 16)), fabsf(__uint_as_float(v[i] & 0xffff0000u))));
    }
    a = wave_max(a);
    float wm = 0.f;
    for (int j = 0; j < k; ++j) wm = fmaxf(wm, fabsf(w[t * k + j]));
    m = fmaxf(m, bf16_to_f32(f32_to_bf16(wm * a)));
  }
  if (lane == 0) sh[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    float b = sh[0];
    for (int i = 1; i < PM_WAVES; ++i) b = fmaxf(b, sh[i]);
    partial[blockIdx.x] = b;
  }
}

// The power-of-two E5M2 scale of the dY rows from the partials (one workgroup): scale[0], and sinv[0] = 1 / scale;
// also clears zero[0 .. nzero) (slots a later kernel fills by atomic max)
__global__ __launch_bounds__(PM_THREADS) void dy_scale_kernel(const float* __restrict__ partial, int nparts,
                                                              float* __restrict__ scale, float* __restrict__ sinv,
                                                              uint32_t* __restrict__ zero, int nzero) {
  __shared__ float sh[PM_WAVES];
  if ((int)threadIdx.x < nzero) zero[threadIdx.x] = 0u;
  float m = 0.f;
  for (int i = threadIdx.x; i < nparts; i += PM_THREADS) m = fmaxf(m, partial[i]);
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < PM_WAVES; ++i) m = fmaxf(m, sh[i]);
    m = fmaxf(m, sh[0]);
    const float sc = e5m2_scale(m);
    scale[0] = sc;
    sinv[0] = __fdiv_rn(1.f, sc);
  }
}

// wpad[slot[i]] = w[i] for the n k flat slots (positions outside [0, rows) skipped): the routing weight of each
// padded row, for the generic-shape path of launch_combine_bwd_pad.
__global__ void scatter_weights_kernel(const int32_t* __restrict__ slot, const float* __restrict__ w, int64_t m,
                                       int64_t rows, float* __restrict__ wpad) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < m; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = slot[i];
    if (r >= 0 && r < rows) wpad[r] = w[i];
  }
}

// Fused combine backward of the layer (bf16 rows): per token, g is read once; for every choice j the expert
// row y_pad[slot] is read once, dy_pad[slot] = bf16(w_j g) written once and <g, y> reduced; then the router
// term dl[t,j] = w_j (dw_j - sum_i w_i dw_i).  moe_permute.py:303-309 does this in two passes over g and y.
// gcopy (optional): g row t is also copied to gcopy[t] (the shared expert's rows of the padded dY, when the shared
// expert rides along the routed experts).  dlog (optional, with sel): the dense bf16 row [E] of d(logits), dl[t,j] at
// column sel[t,j] and 0 elsewhere -- the operand of the router's weight gradient.
// FP8 backward (dyq set): the dY rows go out as E5M2 codes of bf16(w_j g) times scale[0] (dy_scale_kernel; dyp is
// not written).  dyp may be null (no dY rows: the persistent GEMMs gather g and apply w_j themselves); wpad (optional)
// receives w_j at padded row slot[t, j], the weight those GEMMs apply.
template <int NC, int KK>
__global__ __launch_bounds__(PM_THREADS) void combine_bwd_pad_kernel(const bf16_t* __restrict__ yp,
                                                                     const int32_t* __restrict__ slot,
                                                                     const float* __restrict__ w, int64_t n,
                                                                     int64_t d, const bf16_t* __restrict__ g,
                                                                     bf16_t* __restrict__ dyp, float* __restrict__ dw,
                                                                     float* __restrict__ dl,
                                                                     bf16_t* __restrict__ gcopy,
                                                                     const int32_t* __restrict__ sel,
                                                                     bf16_t* __restrict__ dlog, int E,
                                                                     uint8_t* __restrict__ dyq,
                                                                     const float* __restrict__ dy_scale,
                                                                     float* __restrict__ wpad) {
  static_assert(NC > 0 && KK > 0, "fixed-shape kernel");
  const int lane = threadIdx.x & 63;
  const int64_t nwaves = (int64_t)gridDim.x * PM_WAVES;
  const float scale = dyq ? dy_scale[0] : 1.f;
  for (int64_t t = wave_id(); t < n; t += nwaves) {
    float gv[NC][8];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int64_t o = t * d + (c * 64 + lane) * 8;
      if (gcopy) *reinterpret_cast<u32x4*>(gcopy + o) = *reinterpret_cast<const u32x4*>(g + o);
      V8<LSURGE_BF16>::ld(g + o, gv[c]);
    }
    float dot[KK];
#pragma unroll
    for (int j = 0; j < KK; ++j) {
      const int64_t r = slot[t * KK + j];
      const float wj = w[t * KK + j];
      float acc = 0.f;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        float v[8], o[8];
        V8<LSURGE_BF16>::ld(yp + r * d + (c * 64 + lane) * 8, v);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          acc += v[e] * gv[c][e];
          o[e] = wj * gv[c][e];
        }
        if (dyq) {
#pragma unroll
          for (int e = 0; e < 8; ++e) o[e] = bf16_to_f32(f32_to_bf16(o[e])) * scale;
          typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
          *reinterpret_cast<u32x2*>(dyq + r * d + (c * 64 + lane) * 8) =
              u32x2{e5m2x4(o[0], o[1], o[2], o[3]), e5m2x4(o[4], o[5], o[6], o[7])};
        } else if (dyp) {
          V8<LSURGE_BF16>::st(dyp + r * d + (c * 64 + lane) * 8, o);
        }
      }
      if (wpad && lane == 0) wpad[r] = wj;
      dot[j] = acc;
    }
#pragma unroll
    for (int j = 0; j < KK; ++j) dot[j] = wave_sum(dot[j]);
    // every lane holds the reduced dots; the router terms are computed wave-wide (the same operations in the same
    // order on every lane)
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < KK; ++j) s += w[t * KK + j] * dot[j];
    float dlj[KK];
#pragma unroll
    for (int j = 0; j < KK; ++j) dlj[j] = w[t * KK + j] * (dot[j] - s);
    if (lane == 0) {
#pragma unroll
      for (int j = 0; j < KK; ++j) {
        if (dw) dw[t * KK + j] = dot[j];
        if (dl) dl[t * KK + j] = dlj[j];
      }
    }
    if (dlog) {
      for (int e = lane; e < E; e += 64) {
        float v = 0.f;
#pragma unroll
        for (int j = 0; j < KK; ++j)
          if (sel[t * KK + j] == e) v = dlj[j];
        dlog[t * E + e] = f32_to_bf16(v);
      }
    }
  }
}

// dispatch backward + router dx + shared-expert dx, one rounding:
//   dx[t] = sum_j dxp[slot[t,j]] + sum_j dl[t,j] * w_rT[sel[t,j]] + add[t]
template <int NC, int KK>
__global__ __launch_bounds__(PM_THREADS) void dispatch_bwd_pad_kernel(
    const bf16_t* __restrict__ dxp, int64_t d, int k, const int32_t* __restrict__ slot, int64_t n,
    const float* __restrict__ dl, const int32_t* __restrict__ sel, const bf16_t* __restrict__ w_rT,
    const bf16_t* __restrict__ add, bf16_t* __restrict__ dx) {
  const int lane = threadIdx.x & 63;
  const int64_t nwaves = (int64_t)gridDim.x * PM_WAVES;
  for (int64_t t = wave_id(); t < n; t += nwaves) {
    if (NC && KK) {
      float acc[NC > 0 ? NC : 1][8] = {};
#pragma unroll
      for (int j = 0; j < KK; ++j) {
        const int64_t r = slot[t * KK + j];
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          float v[8];
          V8<LSURGE_BF16>::ld(dxp + r * d + (c * 64 + lane) * 8, v);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[c][e] += v[e];
        }
      }
      if (dl) {
#pragma unroll
        for (int j = 0; j < KK; ++j) {
          const float lj = dl[t * KK + j];
          const int64_t e_ = sel[t * KK + j];
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            float v[8];
            V8<LSURGE_BF16>::ld(w_rT + e_ * d + (c * 64 + lane) * 8, v);
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[c][e] += lj * v[e];
          }
        }
      }
      if (add) {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          float v[8];
          V8<LSURGE_BF16>::ld(add + t * d + (c * 64 + lane) * 8, v);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[c][e] += v[e];
        }
      }
#pragma unroll
      for (int c = 0; c < NC; ++c) V8<LSURGE_BF16>::st(dx + t * d + (c * 64 + lane) * 8, acc[c]);
    } else {
      for (int64_t c = lane * 8; c < d; c += 64 * 8) {
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int j = 0; j < k; ++j) {
          float v[8];
          V8<LSURGE_BF16>::ld(dxp + (int64_t)slot[t * k + j] * d + c, v);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[e] += v[e];
        }
        if (dl) {
          for (int j = 0; j < k; ++j) {
            const float lj = dl[t * k + j];
            float v[8];
            V8<LSURGE_BF16>::ld(w_rT + (int64_t)sel[t * k + j] * d + c, v);
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[e] += lj * v[e];
          }
        }
        if (add) {
          float v[8];
          V8<LSURGE_BF16>::ld(add + t * d + c, v);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[e] += v[e];
        }
        V8<LSURGE_BF16>::st(dx + t * d + c, acc);
      }
    }
  }
}

// Transpose a small [R, C] bf16 matrix into [C, R] (router weight for the dx term).
__global__ void transpose_bf16_kernel(const bf16_t* __restrict__ a, int R, int C, bf16_t* __restrict__ at) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < (int64_t)R * C) {
    const int r = (int)(i / C), c = (int)(i % C);
    at[(int64_t)c * R + r] = a[i];
  }
}

// dense dlogits [T, E] bf16 from the k selected gradients (zeros elsewhere)
__global__ void scatter_dlogits_kernel(const float* __restrict__ dl, const int32_t* __restrict__ sel, int64_t T,
                                       int E, int k, bf16_t* __restrict__ dlog) {
  const int64_t t = (int64_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (t >= T) return;
  for (int e = lane; e < E; e += 64) {
    float v = 0.f;
    for (int j = 0; j < k; ++j)
      if (sel[t * k + j] == e) v = dl[t * k + j];
    dlog[t * E + e] = f32_to_bf16(v);
  }
}

inline unsigned grid_for_rows(int64_t rows) {
  const int64_t g = (rows + PM_WAVES - 1) / PM_WAVES;
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>(g, 256 * 16));
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

// ------------------------------------------------------------------------------ internal launchers
namespace lsurge {

// Fixed chunk counts for the row kernels: NC = d / 512 for d in {512, 1024, 2048, 4096}, else 0 (run-time loop).
static int row_chunks(int64_t d) {
  return (d == 512 || d == 1024 || d == 2048 || d == 4096) ? (int)(d / 512) : 0;
}
#define LS_NC_SWITCH(nc, NCV, ...)                          \
  switch (nc) {                                             \
    case 1: { constexpr int NCV = 1; __VA_ARGS__; } break;  \
    case 2: { constexpr int NCV = 2; __VA_ARGS__; } break;  \
    case 4: { constexpr int NCV = 4; __VA_ARGS__; } break;  \
    case 8: { constexpr int NCV = 8; __VA_ARGS__; } break;  \
    default: { constexpr int NCV = 0; __VA_ARGS__; } break; \
  }
#define LS_KK_SWITCH(k, KKV, ...)                           \
  switch (k) {                                              \
    case 6: { constexpr int KKV = 6; __VA_ARGS__; } break;  \
    case 8: { constexpr int KKV = 8; __VA_ARGS__; } break;  \
    default: { constexpr int KKV = 0; __VA_ARGS__; } break; \
  }

int launch_dispatch_pad(const void* x, int64_t d, int k, const int32_t* row_src, const int32_t* num_blocks,
                        int64_t max_rows, void* xp, hipStream_t s) {
  LS_NC_SWITCH(row_chunks(d), NC,
               LSURGE_LAUNCH(KID_DISPATCH, s,
                             hipLaunchKernelGGL(dispatch_pad_kernel<NC>, dim3(grid_for_rows(max_rows)),
                                                dim3(PM_THREADS), 0, s, (const bf16_t*)x, d, k, row_src, num_blocks,
                                                max_rows, (bf16_t*)xp)));
  return LSURGE_OK;
}

int launch_combine_pad(const void* yp, int64_t d, int k, const int32_t* slot, const float* w, int64_t n,
                       const void* add, void* out, int out_dtype, hipStream_t s) {
  const dim3 grid(grid_for_rows(n));
  LS_NC_SWITCH(row_chunks(d), NC, LS_KK_SWITCH(k, KK, {
    if (out_dtype == LSURGE_BF16)
      LSURGE_LAUNCH(KID_COMBINE_FWD, s,
                    hipLaunchKernelGGL((combine_pad_kernel<NC, KK, LSURGE_BF16>), grid, dim3(PM_THREADS), 0, s,
                                       (const bf16_t*)yp, d, k, slot, w, n, (const bf16_t*)add, out));
    else
      LSURGE_LAUNCH(KID_COMBINE_FWD, s,
                    hipLaunchKernelGGL((combine_pad_kernel<NC, KK, LSURGE_F32>), grid, dim3(PM_THREADS), 0, s,
                                       (const bf16_t*)yp, d, k, slot, w, n, (const bf16_t*)add, out));
  }));
  return LSURGE_OK;
}

int dy_rows_amax_parts() { return 1024; }

int launch_dy_scale(const void* g, const float* w, int64_t n, int64_t d, int k, float* partial, float* scale,
                    float* sinv, hipStream_t s, uint32_t* zero, int nzero) {
  LSURGE_REQUIRE(n >= 1 && d >= 8 && d % 8 == 0 && k >= 1 && aligned16(g) && nzero >= 0 && nzero <= PM_THREADS,
                 "dy_scale: bad shape");
  const int nb = (int)std::min<int64_t>(dy_rows_amax_parts(), (n + PM_WAVES - 1) / PM_WAVES);
  LSURGE_LAUNCH(KID_FP8_QUANT, s,
                hipLaunchKernelGGL(dy_rows_amax_kernel, dim3(nb), dim3(PM_THREADS), 0, s, (const bf16_t*)g, w, n, d, k,
                                   partial));
  LSURGE_LAUNCH(KID_FP8_QUANT, s,
                hipLaunchKernelGGL(dy_scale_kernel, dim3(1), dim3(PM_THREADS), 0, s, (const float*)partial, nb, scale,
                                   sinv, zero, nzero));
  return LSURGE_OK;
}

int launch_combine_bwd_pad(const void* yp, int64_t rows, const int32_t* slot, const float* w, int64_t n, int k,
                           int64_t d, const void* g, void* dyp, float* dw, float* dl, hipStream_t s, void* gcopy,
                           const int32_t* sel, void* dlog, int E, const CombineFp8& f8, float* wpad) {
  const dim3 grid(grid_for_rows(n));
  const int nc = row_chunks(d);
  LSURGE_REQUIRE(!dlog || (sel && dl && E >= 1), "combine_bwd: dense d(logits) needs sel, dl and E");
  LSURGE_REQUIRE(!dl || dw, "combine_bwd: the router backward needs dw");
  LSURGE_REQUIRE(!f8.dyq || (f8.scale && f8.nblocks && !gcopy), "combine_bwd: the FP8 dY rows need their scale and "
                 "the block count");
  LSURGE_REQUIRE(dyp || (!f8.dyq && !gcopy), "combine_bwd: the FP8 rows and the shared copy need the dY rows");
  if (nc && (k == 6 || k == 8)) {
    LS_NC_SWITCH(nc, NC, LS_KK_SWITCH(k, KK, {
      if (NC && KK)
        LSURGE_LAUNCH(KID_COMBINE_BWD, s,
                      hipLaunchKernelGGL((combine_bwd_pad_kernel<NC ? NC : 1, KK ? KK : 1>), grid, dim3(PM_THREADS), 0,
                                         s, (const bf16_t*)yp, slot, w, n, d, (const bf16_t*)g, (bf16_t*)dyp, dw, dl,
                                         (bf16_t*)gcopy, sel, (bf16_t*)dlog, E, (uint8_t*)f8.dyq, f8.scale, wpad));
    }));
    return LSURGE_OK;
  }
  if (wpad)
    LSURGE_LAUNCH(KID_COMBINE_BWD, s,
                  hipLaunchKernelGGL(scatter_weights_kernel, dim3((unsigned)std::min<int64_t>((n * k + 255) / 256, 4096)),
                                     dim3(256), 0, s, slot, w, n * k, rows, wpad));
  if (gcopy)  // generic shapes: a plain copy of g into the shared expert's rows
    if (hipMemcpyAsync(gcopy, g, (size_t)n * d * 2, hipMemcpyDeviceToDevice, s) != hipSuccess)
      return lsurge::set_error(LSURGE_ERR_LAUNCH, "combine_bwd: copy of dY into the shared rows failed");
  LSURGE_LAUNCH(KID_COMBINE_BWD, s,
                hipLaunchKernelGGL((combine_bwd_kernel<LSURGE_BF16, LSURGE_BF16, true>), grid, dim3(PM_THREADS), 0, s,
                                   yp, rows, slot, w, n, k, d, g, dyp, dw, dl));
  if (dlog)
    if (int rc = launch_scatter_dlogits(dl, sel, n, E, k, dlog, s)) return rc;
  // generic shapes, FP8: the bf16 rows are cast afterwards with the same scale (the rows of real blocks; padding rows
  // are never read)
  if (f8.dyq)
    return fp8_cast_e5m2(dyp, rows * d, f8.scale, -1, f8.dyq, nullptr, f8.nblocks, (int64_t)LSURGE_BLOCK_ROWS * d, s);
  return LSURGE_OK;
}

int launch_dispatch_bwd_pad(const void* dxp, int64_t d, int k, const int32_t* slot, int64_t n, const float* dl,
                            const int32_t* sel, const void* w_rT, const void* add, void* dx, hipStream_t s) {
  LS_NC_SWITCH(row_chunks(d), NC, LS_KK_SWITCH(k, KK,
               LSURGE_LAUNCH(KID_DISPATCH_BWD, s,
                             hipLaunchKernelGGL((dispatch_bwd_pad_kernel<NC, KK>), dim3(grid_for_rows(n)),
                                                dim3(PM_THREADS), 0, s, (const bf16_t*)dxp, d, k, slot, n, dl, sel,
                                                (const bf16_t*)w_rT, (const bf16_t*)add, (bf16_t*)dx))));
  return LSURGE_OK;
}

int launch_transpose_bf16(const void* a, int R, int C, void* at, hipStream_t s) {
  const int64_t n = (int64_t)R * C;
  LSURGE_LAUNCH(KID_MISC, s,
                hipLaunchKernelGGL(transpose_bf16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                                   (const bf16_t*)a, R, C, (bf16_t*)at));
  return LSURGE_OK;
}

int launch_scatter_dlogits(const float* dl, const int32_t* sel, int64_t T, int E, int k, void* dlog, hipStream_t s) {
  LSURGE_LAUNCH(KID_MISC, s,
                hipLaunchKernelGGL(scatter_dlogits_kernel, dim3((unsigned)((T + 3) / 4)), dim3(256), 0, s, dl, sel, T,
                                   E, k, (bf16_t*)dlog));
  return LSURGE_OK;
}

}  // namespace lsurge

// ------------------------------------------------------------------------------ C ABI
#define DT_SWITCH(dt, DT, ...)                                                \
  switch (dt) {                                                               \
    case LSURGE_F32: { constexpr int DT = LSURGE_F32; __VA_ARGS__; } break;   \
    case LSURGE_BF16: { constexpr int DT = LSURGE_BF16; __VA_ARGS__; } break; \
    case LSURGE_F16: { constexpr int DT = LSURGE_F16; __VA_ARGS__; } break;   \
    default: return lsurge::set_error(LSURGE_ERR_DTYPE, "unsupported dtype %d", (int)(dt)); \
  }

extern "C" {

int lsurge_gather_rows(const void* x, int64_t n, int64_t d, int dtype, const int32_t* idx, int64_t m,
                       const float* scale, void* out, lsurge_stream_t stream) {
  LSURGE_REQUIRE(n >= 0 && d >= 0 && m >= 0, "gather_rows: negative shape");
  if (m == 0 || d == 0) return LSURGE_OK;
  LSURGE_REQUIRE(x && idx && out && n > 0, "gather_rows: null pointer or empty source");
  hipStream_t s = (hipStream_t)stream;
  const bool vec = (d % 8 == 0) && aligned16(x) && aligned16(out);
  DT_SWITCH(dtype, DT, {
    if (vec)
      LSURGE_LAUNCH(KID_MISC, s, hipLaunchKernelGGL((gather_rows_kernel<DT, true>), dim3(grid_for_rows(m)),
                                                    dim3(PM_THREADS), 0, s, x, n, d, idx, m, scale, out));
    else
      LSURGE_LAUNCH(KID_MISC, s, hipLaunchKernelGGL((gather_rows_kernel<DT, false>), dim3(grid_for_rows(m)),
                                                    dim3(PM_THREADS), 0, s, x, n, d, idx, m, scale, out));
  });
  return LSURGE_OK;
}

int lsurge_gather_reduce(const void* y, int64_t m, int64_t d, int y_dtype, const int32_t* pos, int64_t n, int64_t k,
                         const float* w, void* out, int out_dtype, lsurge_stream_t stream) {
  LSURGE_REQUIRE(m >= 0 && d >= 0 && n >= 0 && k >= 0, "gather_reduce: negative shape");
  if (n == 0 || d == 0) return LSURGE_OK;
  LSURGE_REQUIRE(out && (k == 0 || (y && pos)), "gather_reduce: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const bool vec = (d % 8 == 0) && aligned16(y) && aligned16(out);
  DT_SWITCH(y_dtype, DT, DT_SWITCH(out_dtype, OT, {
    if (vec)
      LSURGE_LAUNCH(KID_MISC, s, hipLaunchKernelGGL((gather_reduce_kernel<DT, OT, true>), dim3(grid_for_rows(n)),
                                                    dim3(PM_THREADS), 0, s, y, m, d, pos, n, (int)k, w, out));
    else
      LSURGE_LAUNCH(KID_MISC, s, hipLaunchKernelGGL((gather_reduce_kernel<DT, OT, false>), dim3(grid_for_rows(n)),
                                                    dim3(PM_THREADS), 0, s, y, m, d, pos, n, (int)k, w, out));
  }));
  return LSURGE_OK;
}

int lsurge_gather_dot(const void* y, int64_t m, int64_t d, int y_dtype, const int32_t* pos, int64_t n, int64_t k,
                      const void* g, int g_dtype, float* out, lsurge_stream_t stream) {
  LSURGE_REQUIRE(m >= 0 && d >= 0 && n >= 0 && k >= 0, "gather_dot: negative shape");
  if (n == 0 || k == 0) return LSURGE_OK;
  LSURGE_REQUIRE(y && pos && g && out, "gather_dot: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const bool vec = (d % 8 == 0) && aligned16(y) && aligned16(g);
  DT_SWITCH(y_dtype, DT, DT_SWITCH(g_dtype, GT, {
    if (vec)
      LSURGE_LAUNCH(KID_MISC, s, hipLaunchKernelGGL((gather_dot_kernel<DT, GT, true>), dim3(grid_for_rows(n)),
                                                    dim3(PM_THREADS), 0, s, y, m, d, pos, n, (int)k, g, out));
    else
      LSURGE_LAUNCH(KID_MISC, s, hipLaunchKernelGGL((gather_dot_kernel<DT, GT, false>), dim3(grid_for_rows(n)),
                                                    dim3(PM_THREADS), 0, s, y, m, d, pos, n, (int)k, g, out));
  }));
  return LSURGE_OK;
}

int lsurge_combine_bwd(const void* y, int y_dtype, const int32_t* pos, const float* w, int64_t n, int64_t k, int64_t d,
                       const void* g, int g_dtype, void* dy, float* dw, lsurge_stream_t stream) {
  LSURGE_REQUIRE(n >= 0 && k >= 0 && d >= 0, "combine_bwd: negative shape");
  if (n == 0 || k == 0) return LSURGE_OK;
  LSURGE_REQUIRE(y && pos && w && g && dy && dw, "combine_bwd: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const bool vec = (d % 8 == 0) && aligned16(y) && aligned16(g) && aligned16(dy);
  DT_SWITCH(y_dtype, DT, DT_SWITCH(g_dtype, GT, {
    if (vec)
      LSURGE_LAUNCH(KID_COMBINE_BWD, s,
                    hipLaunchKernelGGL((combine_bwd_kernel<DT, GT, true>), dim3(grid_for_rows(n)), dim3(PM_THREADS), 0,
                                       s, y, n * k, pos, w, n, (int)k, d, g, dy, dw, (float*)nullptr));
    else
      LSURGE_LAUNCH(KID_COMBINE_BWD, s,
                    hipLaunchKernelGGL((combine_bwd_kernel<DT, GT, false>), dim3(grid_for_rows(n)), dim3(PM_THREADS),
                                       0, s, y, n * k, pos, w, n, (int)k, d, g, dy, dw, (float*)nullptr));
  }));
  return LSURGE_OK;
}

}  // extern "C"
