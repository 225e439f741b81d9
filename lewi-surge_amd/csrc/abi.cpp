// Status reporting and the live event profiler of the C ABI.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <atomic>
#include <mutex>
#include <vector>

#include "common.h"

namespace lsurge {

static thread_local char g_err[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(LSURGE_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  return LSURGE_OK;
}

// ------------------------------------------------------------------------------ live profiler
// Brackets selected kernels with a pair of HIP events recorded on the launch stream.  Only kernels whose
// bit is set in the mask are bracketed, so the timed layer carries one event pair per step at most.

namespace {
struct Pair {
  int kid;
  hipEvent_t a, b;
};
std::mutex g_mu;
bool g_on = false;
uint64_t g_mask = 0;
std::vector<Pair> g_pool;
size_t g_used = 0;
int g_open[KID_COUNT];
double g_total_ms[KID_COUNT];
int64_t g_count[KID_COUNT];
const char* g_names[KID_COUNT] = {
    "router_topk",      "layout_hist",       "layout_scan",       "layout_rank",      "dispatch",
    "gemm_gu_fwd",      "gemm_down_fwd",     "combine_fwd",       "combine_bwd",      "gemm_down_dgrad",
    "gemm_down_wgrad",  "gemm_gu_dgrad",     "gemm_gu_wgrad",     "dispatch_bwd",     "router_wgrad",
    "shared_gu_fwd",    "shared_down_fwd",   "shared_down_dgrad", "shared_down_wgrad", "shared_gu_dgrad",
    "shared_gu_wgrad",  "splitk_reduce",     "misc",             "router_select",
    "fp8_quantize",     "gdn_chunk",         "gdn_scan",          "gdn_bscan",        "gdn_bgrad",
    "gdn_bchunk"};
static_assert(KID_COUNT <= 31, "lsurge_prof_enable takes the kernel ids as bits of an int");
constexpr size_t kPool = 8192;
}  // namespace

hipError_t prof_mark_begin(int kid, hipStream_t s) {
  if (!g_on || !((g_mask >> kid) & 1)) return hipSuccess;
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_used >= g_pool.size()) return hipSuccess;  // pool exhausted: skip (collect() reports counts)
  g_pool[g_used].kid = kid;
  g_open[kid] = (int)g_used;
  return hipEventRecord(g_pool[g_used++].a, s);
}

hipError_t prof_mark_end(int kid, hipStream_t s) {
  if (!g_on || !((g_mask >> kid) & 1)) return hipSuccess;
  std::lock_guard<std::mutex> lk(g_mu);
  int i = g_open[kid];
  if (i < 0) return hipSuccess;
  g_open[kid] = -1;
  return hipEventRecord(g_pool[i].b, s);
}

// ------------------------------------------------------------------------------ helper streams
// The layer entry points run independent kernel chains (shared expert, weight gradients, router backward) on
// helper streams that fork from and join back into the caller's stream through events, so each call stays
// stream-ordered with respect to that stream and never synchronises the host.  One set per device, created
// on first use (default priority); calls that overlap on one device serialise their enqueueing on its mutex.
namespace {
struct DeviceFork {
  std::mutex mu;
  bool ready = false;
  hipStream_t side[kForkStreams];
  hipEvent_t ev[kForkEvents];
};
constexpr int kMaxDevices = 64;
DeviceFork g_fork[kMaxDevices];
}  // namespace

static std::atomic<int> g_concurrency{0};
static std::atomic<int> g_gemm_variant{LSURGE_GEMM_G256};

int gemm_variant() { return g_gemm_variant.load(std::memory_order_relaxed); }

int fork_acquire(ForkSet* f, hipStream_t main) {
  if (!g_concurrency.load(std::memory_order_relaxed)) {  // serial: every chain on the caller's stream
    for (int i = 0; i < kForkStreams; ++i) f->side[i] = main;
    f->dev = -1;
    return LSURGE_OK;
  }
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(LSURGE_ERR_LAUNCH, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return set_error(LSURGE_ERR_INVALID, "device %d out of range", dev);
  DeviceFork& d = g_fork[dev];
  d.mu.lock();
  if (!d.ready) {
    for (int i = 0; i < kForkStreams; ++i) {
      e = hipStreamCreateWithFlags(&d.side[i], hipStreamNonBlocking);
      if (e != hipSuccess) {
        d.mu.unlock();
        return set_error(LSURGE_ERR_LAUNCH, "hipStreamCreateWithFlags: %s", hipGetErrorString(e));
      }
    }
    for (int i = 0; i < kForkEvents; ++i) {
      e = hipEventCreateWithFlags(&d.ev[i], hipEventDisableTiming);
      if (e != hipSuccess) {
        d.mu.unlock();
        return set_error(LSURGE_ERR_LAUNCH, "hipEventCreateWithFlags: %s", hipGetErrorString(e));
      }
    }
    d.ready = true;
  }
  for (int i = 0; i < kForkStreams; ++i) f->side[i] = d.side[i];
  for (int i = 0; i < kForkEvents; ++i) f->ev[i] = d.ev[i];
  f->dev = dev;
  return LSURGE_OK;
}

void fork_release(ForkSet* f) {
  if (f->dev >= 0) g_fork[f->dev].mu.unlock();
}

// the last kForkStreams events of a set are reserved for this join (the layer's own joins use the first ones)
void fork_join_all(ForkSet* f, hipStream_t main) {
  for (int i = 0; i < kForkStreams; ++i) {
    if (f->side[i] == main) continue;
    hipEvent_t ev = f->ev[kForkEvents - kForkStreams + i];
    if (hipEventRecord(ev, f->side[i]) == hipSuccess) (void)hipStreamWaitEvent(main, ev, 0);
  }
}

// ------------------------------------------------------------------------------ test hooks
static std::atomic<int> g_fail_kid{-1};
static std::atomic<int> g_fail_left{0};

bool test_fail_hit(int kid) {
  if (g_fail_kid.load(std::memory_order_relaxed) != kid) return false;
  if (g_fail_left.fetch_sub(1) != 1) return false;
  g_fail_kid.store(-1);
  return true;
}

int stream_after(hipStream_t waiter, hipStream_t producer, hipEvent_t ev) {
  if (waiter == producer) return LSURGE_OK;
  hipError_t e = hipEventRecord(ev, producer);
  if (e == hipSuccess) e = hipStreamWaitEvent(waiter, ev, 0);
  if (e != hipSuccess) return set_error(LSURGE_ERR_LAUNCH, "stream join: %s", hipGetErrorString(e));
  return LSURGE_OK;
}

}  // namespace lsurge

using namespace lsurge;

extern "C" {

int lsurge_abi_version(void) { return LSURGE_ABI_VERSION; }

int lsurge_set_concurrency(int on) {
  g_concurrency.store(on ? 1 : 0);
  return LSURGE_OK;
}
int lsurge_get_concurrency(void) { return g_concurrency.load(); }
int lsurge_set_gemm_variant(int variant) {
  if (variant != LSURGE_GEMM_CLASSIC && variant != LSURGE_GEMM_G256)
    return set_error(LSURGE_ERR_INVALID, "gemm variant %d: expected LSURGE_GEMM_CLASSIC (0) or LSURGE_GEMM_G256 (1)",
                     variant);
  g_gemm_variant.store(variant);
  return LSURGE_OK;
}
int lsurge_get_gemm_variant(void) { return g_gemm_variant.load(); }
const char* lsurge_last_error(void) { return g_err; }

int lsurge_test_fail_launch(int kernel_id, int nth) {
  if (kernel_id < -1 || kernel_id >= KID_COUNT || nth < 0) return set_error(LSURGE_ERR_INVALID, "bad test hook arguments");
  g_fail_left.store(nth);
  g_fail_kid.store(nth > 0 ? kernel_id : -1);
  return LSURGE_OK;
}

int lsurge_test_helpers_idle(void) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return -1;
  DeviceFork& d = g_fork[dev];
  std::lock_guard<std::mutex> lk(d.mu);
  if (!d.ready) return -1;
  for (int i = 0; i < kForkStreams; ++i)
    if (hipStreamQuery(d.side[i]) != hipSuccess) return 0;
  return 1;
}

int lsurge_prof_kernel_count(void) { return KID_COUNT; }
const char* lsurge_prof_kernel_name(int id) { return (id >= 0 && id < KID_COUNT) ? g_names[id] : ""; }

void lsurge_prof_reset(void) {
  std::lock_guard<std::mutex> lk(g_mu);
  for (int i = 0; i < KID_COUNT; ++i) {
    g_total_ms[i] = 0;
    g_count[i] = 0;
    g_open[i] = -1;
  }
  g_used = 0;
}

// on: 0 = off, otherwise a bit mask of kernel ids to bracket (all ones = every kernel).
int lsurge_prof_enable(int on) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (on && g_pool.empty()) {
    g_pool.resize(kPool);
    for (auto& p : g_pool) {
      if (hipEventCreate(&p.a) != hipSuccess || hipEventCreate(&p.b) != hipSuccess)
        return set_error(LSURGE_ERR_LAUNCH, "hipEventCreate failed");
    }
  }
  g_on = on != 0;
  g_mask = (on == -1) ? ~0ull : (uint64_t)(uint32_t)on;
  for (int i = 0; i < KID_COUNT; ++i) g_open[i] = -1;
  return LSURGE_OK;
}

int lsurge_prof_collect(void) {
  std::lock_guard<std::mutex> lk(g_mu);
  for (size_t i = 0; i < g_used; ++i) {
    float ms = 0;
    hipError_t e = hipEventElapsedTime(&ms, g_pool[i].a, g_pool[i].b);
    if (e != hipSuccess) return set_error(LSURGE_ERR_LAUNCH, "hipEventElapsedTime: %s", hipGetErrorString(e));
    g_total_ms[g_pool[i].kid] += ms;
    g_count[g_pool[i].kid] += 1;
  }
  g_used = 0;
  return LSURGE_OK;
}

int lsurge_prof_read(int id, double* total_ms, int64_t* launches) {
  if (id < 0 || id >= KID_COUNT) return set_error(LSURGE_ERR_INVALID, "bad kernel id %d", id);
  *total_ms = g_total_ms[id];
  *launches = g_count[id];
  return LSURGE_OK;
}

}  // extern "C"
