// Shared device/host helpers for the MI355X (gfx950) MoE hot-path kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/lewi_surge.h"

typedef uint16_t bf16_t;  // bf16 storage (bit pattern)
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));

#define LDS_PTR(T, p) ((__attribute__((address_space(3))) T*)(p))

// ------------------------------------------------------------------------------------ scalar conversions

__device__ __forceinline__ float bf16_to_f32(bf16_t b) { return __uint_as_float(((uint32_t)b) << 16); }

// f32 -> bf16, round to nearest even (gfx950 v_cvt_pk_bf16_f32; NaN stays a quiet NaN)
__device__ __forceinline__ bf16_t f32_to_bf16(float f) { return __builtin_bit_cast(bf16_t, (__bf16)f); }

// two f32 -> packed bf16 pair (lo in bits 0..15), one v_cvt_pk_bf16_f32
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f32_to_f16(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// element load/store by runtime dtype tag (LSURGE_F32 / LSURGE_BF16 / LSURGE_F16)
template <int DT> struct Elem;
template <> struct Elem<LSURGE_F32> {
  typedef float T;
  static __device__ __forceinline__ float ld(const T* p, int64_t i) { return p[i]; }
  static __device__ __forceinline__ void st(T* p, int64_t i, float v) { p[i] = v; }
};
template <> struct Elem<LSURGE_BF16> {
  typedef uint16_t T;
  static __device__ __forceinline__ float ld(const T* p, int64_t i) { return bf16_to_f32(p[i]); }
  static __device__ __forceinline__ void st(T* p, int64_t i, float v) { p[i] = f32_to_bf16(v); }
};
template <> struct Elem<LSURGE_F16> {
  typedef uint16_t T;
  static __device__ __forceinline__ float ld(const T* p, int64_t i) { return f16_to_f32(p[i]); }
  static __device__ __forceinline__ void st(T* p, int64_t i, float v) { p[i] = f32_to_f16(v); }
};

// ------------------------------------------------------------------------------------ FP8 gradients (E5M2)
// Gradients of the FP8 backward are OCP E5M2 with a power-of-two current scale: scale = the largest power of two
// not above 57344 / amax (1 when amax is 0).  A gradient's amax is one element of a GEMM's output, and a one-ulp
// change of it would otherwise move the whole tensor's quantisation grid; a power-of-two scale moves only when the
// amax crosses a binade, and it dequantises exactly.
__device__ __forceinline__ float e5m2_scale(float amax) {
  if (!(amax > 0.f)) return 1.f;
  float s = __fdiv_rn(57344.f, amax);
  if (!(s <= 3.4028234663852886e38f)) s = 3.4028234663852886e38f;
  int e;
  (void)frexpf(s, &e);  // s = m 2^e, m in [0.5, 1)
  return ldexpf(1.f, e - 1);
}
// four floats (already scaled) -> four E5M2 bytes (nearest even, saturated at +-57344), element 0 in the low byte
__device__ __forceinline__ uint32_t e5m2x4(float a, float b, float c, float d) {
  a = fminf(fmaxf(a, -57344.f), 57344.f);
  b = fminf(fmaxf(b, -57344.f), 57344.f);
  c = fminf(fmaxf(c, -57344.f), 57344.f);
  d = fminf(fmaxf(d, -57344.f), 57344.f);
  int w = __builtin_amdgcn_cvt_pk_bf8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_bf8_f32(c, d, w, true);
  return (uint32_t)w;
}

// ------------------------------------------------------------------------------------ wave helpers

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// ------------------------------------------------------------------------------------ host-side status

namespace lsurge {
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);

// helper streams of the current device (see abi.cpp); fork_acquire locks the device's set until fork_release.
// With concurrency off (the default) every helper is the caller's stream and nothing is locked.
constexpr int kForkStreams = 3, kForkEvents = 12;
struct ForkSet {
  hipStream_t side[kForkStreams];
  hipEvent_t ev[kForkEvents];
  int dev;
};
int fork_acquire(ForkSet* f, hipStream_t main);
// the grouped-GEMM kernel family (lsurge_set_gemm_variant)
int gemm_variant();
void fork_release(ForkSet* f);
// make `main` wait for everything enqueued so far on every helper of f (the error path of a forked call)
void fork_join_all(ForkSet* f, hipStream_t main);
// test hook: true when this launch of kernel id `kid` is the one lsurge_test_fail_launch armed (it then fails
// without launching)
bool test_fail_hit(int kid);
// enqueue on `waiter` a wait for everything enqueued so far on `producer`
int stream_after(hipStream_t waiter, hipStream_t producer, hipEvent_t ev);
hipError_t prof_mark_begin(int kernel_id, hipStream_t s);
hipError_t prof_mark_end(int kernel_id, hipStream_t s);
}  // namespace lsurge

#define LSURGE_REQUIRE(cond, ...)                                         \
  do {                                                                    \
    if (!(cond)) return lsurge::set_error(LSURGE_ERR_INVALID, __VA_ARGS__); \
  } while (0)

// Kernel ids for the live profiler (lsurge_prof_*); names in abi.cpp.
enum {
  KID_ROUTER = 0,
  KID_LAYOUT_HIST,
  KID_LAYOUT_SCAN,
  KID_LAYOUT_RANK,
  KID_DISPATCH,
  KID_GEMM_GU_FWD,
  KID_GEMM_DOWN_FWD,
  KID_COMBINE_FWD,
  KID_COMBINE_BWD,
  KID_GEMM_DOWN_DGRAD,
  KID_GEMM_DOWN_WGRAD,
  KID_GEMM_GU_DGRAD,
  KID_GEMM_GU_WGRAD,
  KID_DISPATCH_BWD,
  KID_ROUTER_WGRAD,
  KID_SHARED_GU_FWD,
  KID_SHARED_DOWN_FWD,
  KID_SHARED_DOWN_DGRAD,
  KID_SHARED_DOWN_WGRAD,
  KID_SHARED_GU_DGRAD,
  KID_SHARED_GU_WGRAD,
  KID_SPLITK_REDUCE,
  KID_MISC,
  KID_ROUTER_SELECT,
  KID_FP8_QUANT,
  KID_GDN_CHUNK,
  KID_GDN_SCAN,
  KID_GDN_BSCAN,
  KID_GDN_BGRAD,
  KID_GDN_BCHUNK,
  KID_COUNT
};

// RAII-free launch bracket used by the layer entry points.
#define LSURGE_LAUNCH(kid, stream, ...)             \
  do {                                              \
    if (lsurge::test_fail_hit(kid))                 \
      return lsurge::set_error(LSURGE_ERR_LAUNCH, "%s: launch failure injected by lsurge_test_fail_launch", #kid); \
    (void)lsurge::prof_mark_begin((kid), (stream)); \
    __VA_ARGS__;                                    \
    (void)lsurge::prof_mark_end((kid), (stream));   \
    int _rc = lsurge::check_launch(#kid);           \
    if (_rc) return _rc;                            \
  } while (0)
