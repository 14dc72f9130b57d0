// Library runtime: error reporting, the scratch arena, fills and kernel timers.
#include <stdarg.h>
#include <stdio.h>

#include <map>
#include <mutex>
#include <string>
#include <tuple>
#include <vector>

#include "common.hpp"
#include "kernels.hpp"

static thread_local char g_err[1024] = "";

void wgbm_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

const char* wgbm_last_error_impl() { return g_err; }

namespace wgbm {

// ---------------------------------------------------------------------------
// scratch arena: one grow-only buffer per (device, stream, slot).  Work on one
// stream is ordered, so reusing a slot across calls on the same stream is
// safe; calls on different streams get different buffers.
// ---------------------------------------------------------------------------
struct ScratchBuf {
  void* p = nullptr;
  size_t n = 0;
};
static std::mutex g_scratch_mu;
static std::map<std::tuple<int, void*, int>, ScratchBuf> g_scratch;

void* scratch_get(hipStream_t st, size_t bytes, int slot) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  ScratchBuf& b = g_scratch[std::make_tuple(dev, (void*)st, slot)];
  if (bytes == 0) bytes = 1;
  if (b.n < bytes) {
    if (b.p) {
      // the old buffer may still be in use by queued work on this stream
      if (hipStreamSynchronize(st) != hipSuccess) return nullptr;
      (void)hipFree(b.p);
      b.p = nullptr;
      b.n = 0;
    }
    size_t want = bytes + bytes / 4;
    if (hipMalloc(&b.p, want) != hipSuccess) {
      b.p = nullptr;
      return nullptr;
    }
    b.n = want;
  }
  return b.p;
}

void scratch_release_all() {
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  for (auto& kv : g_scratch)
    if (kv.second.p) (void)hipFree(kv.second.p);
  g_scratch.clear();
}

// ---------------------------------------------------------------------------
// fills (kernels rather than hipMemsetAsync so that the sequences stay valid
// under stream capture)
// ---------------------------------------------------------------------------
__global__ void fill_u32_kernel(uint32_t* p, int64_t n, uint32_t v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}
__global__ void fill_u64_kernel(unsigned long long* p, int64_t n, unsigned long long v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}
int fill_u32(uint32_t* p, int64_t n, uint32_t v, hipStream_t st) {
  if (n <= 0) return 0;
  hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, p, n, v);
  WGBM_LAUNCH_CHECK();
  return 0;
}
int fill_u64(void* p, int64_t n, unsigned long long v, hipStream_t st) {
  if (n <= 0) return 0;
  hipLaunchKernelGGL(fill_u64_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                     (unsigned long long*)p, n, v);
  WGBM_LAUNCH_CHECK();
  return 0;
}

// ---------------------------------------------------------------------------
// kernel timers, wgbm_timer_enable(mode): mode 1 records a HIP event on the
// kernel's stream right before and right after the launch of a timed kernel
// (hipEventRecord markers: the interval is the kernel's execution plus the
// dispatch of its packet); mode 2 attaches the pair to the kernel's own
// dispatch (hipExtLaunchKernel start / stop events).  wgbm_timer_read sums
// the intervals per tag.
// ---------------------------------------------------------------------------
struct TimerRec {
  std::string tag;
  hipEvent_t a, b;
};
static std::mutex g_timer_mu;
static int g_timer_mode = 0;
static std::vector<TimerRec> g_timer_pending;
static std::map<std::string, std::pair<double, long>> g_timer_acc;

bool timer_enabled() { return g_timer_mode != 0; }
int timer_mode() { return g_timer_mode; }

void* timer_begin(const char* tag) {
  if (!g_timer_mode || !tag) return nullptr;
  TimerRec* r = new TimerRec{tag, nullptr, nullptr};
  if (hipEventCreate(&r->a) != hipSuccess) {
    delete r;
    return nullptr;
  }
  if (hipEventCreate(&r->b) != hipSuccess) {
    (void)hipEventDestroy(r->a);
    delete r;
    return nullptr;
  }
  return r;
}

hipEvent_t timer_start_event(void* h) { return h ? ((TimerRec*)h)->a : nullptr; }
hipEvent_t timer_stop_event(void* h) { return h ? ((TimerRec*)h)->b : nullptr; }

void timer_end(void* h) {
  if (!h) return;
  TimerRec* r = (TimerRec*)h;
  std::lock_guard<std::mutex> lk(g_timer_mu);
  g_timer_pending.push_back(*r);
  delete r;
}

void timer_enable(int mode) {
  std::lock_guard<std::mutex> lk(g_timer_mu);
  g_timer_mode = mode == 1 || mode == 2 ? mode : 0;
}

int timer_read(const char* tag, double* total_ms, long* count) {
  std::lock_guard<std::mutex> lk(g_timer_mu);
  for (auto& r : g_timer_pending) {
    float ms = 0.0f;
    WGBM_CHECK(hipEventSynchronize(r.b));
    WGBM_CHECK(hipEventElapsedTime(&ms, r.a, r.b));
    auto& acc = g_timer_acc[r.tag];
    acc.first += ms;
    acc.second += 1;
    (void)hipEventDestroy(r.a);
    (void)hipEventDestroy(r.b);
  }
  g_timer_pending.clear();
  auto it = g_timer_acc.find(tag);
  *total_ms = it == g_timer_acc.end() ? 0.0 : it->second.first;
  *count = it == g_timer_acc.end() ? 0 : it->second.second;
  return 0;
}

void timer_reset() {
  std::lock_guard<std::mutex> lk(g_timer_mu);
  for (auto& r : g_timer_pending) {
    (void)hipEventSynchronize(r.b);
    (void)hipEventDestroy(r.a);
    (void)hipEventDestroy(r.b);
  }
  g_timer_pending.clear();
  g_timer_acc.clear();
}

}  // namespace wgbm
