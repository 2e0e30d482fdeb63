// Runtime of libtorchjs_hip.so: device init, the library stream, the
// stream-ordered caching allocator, copies, errors and launch timing.
//
// Replaces the WebGPU runtime of torch.js: initWebGPU/getDevice
// (src/backend/webgpu/device.ts:27-97), GPUBufferPool and the upload /
// readback helpers (src/backend/webgpu/buffer.ts:21-206), syncDevice
// (src/backend/webgpu/dispatch.ts:115-118) and the memory counters behind
// torch.webgpu.memory_stats (src/webgpu.ts:11-51).

#include "common.h"

#include <rocprofiler-sdk-roctx/roctx.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <map>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

namespace tjh {

// ---------------------------------------------------------------- errors

static thread_local char g_err[1024] = {0};

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_err[0] = 0; }

int hip_fail(hipError_t e, const char* what) {
  return set_error(TJH_ERR_HIP, "%s failed: %s (%d)", what,
                   hipGetErrorString(e), (int)e);
}

// ---------------------------------------------------------------- device

static std::mutex g_init_mu;
static bool g_init = false;
static int g_ordinal = -1;
static int g_cus = 0;
static hipStream_t g_stream = nullptr;

hipStream_t stream() { return g_stream; }

bool initialized() { return g_init; }
int device_ordinal() { return g_ordinal; }
int num_cus() { return g_cus; }

int require_init() {
  if (!g_init)
    return set_error(TJH_ERR_NOT_INITIALIZED,
                     "hip backend not initialized. Call torch.init() first.");
  return TJH_OK;
}

int check_launch(const char* kernel) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, kernel);
  return TJH_OK;
}

// ---------------------------------------------------------------- allocator
//
// One stream => a block freed by the host can be reused by the next
// launch without waiting: the next user is ordered after every earlier
// user on the stream.  Blocks are cached by rounded size; a cached block
// is reused when it is at most 1/8 larger than the request.

namespace {

constexpr size_t kSmall = size_t(1) << 20;      // 1 MiB
constexpr size_t kSmallRound = 512;
constexpr size_t kLargeRound = size_t(2) << 20; // 2 MiB

size_t round_size(size_t bytes) {
  if (bytes == 0) bytes = 1;
  if (bytes <= kSmall) return (bytes + kSmallRound - 1) / kSmallRound * kSmallRound;
  return (bytes + kLargeRound - 1) / kLargeRound * kLargeRound;
}

struct Allocator {
  std::mutex mu;
  std::multimap<size_t, void*> free_blocks;   // size -> ptr
  std::unordered_map<void*, size_t> live;     // ptr -> size
  tjh_mem_stats st{};
  // HIP graphs: a block allocated or freed while a graph is being captured
  // belongs to that graph (its kernels may touch it on every replay), so
  // when free it goes back to the graph's own pool, never to other work,
  // until the graph is destroyed.
  int capturing = 0;                                        // graph id, 0 = none
  std::unordered_map<void*, int> owner;                     // ptr -> graph id
  std::unordered_map<int, std::multimap<size_t, void*>> gpool;  // graph -> free blocks

  void release_cached_locked() {
    for (auto& kv : free_blocks) {
      (void)hipFree(kv.second);
    }
    free_blocks.clear();
    st.pooled_bytes = 0;
  }
};

Allocator& alloc() {
  static Allocator* a = new Allocator();  // never destroyed: outlives atexit
  return *a;
}

}  // namespace

static int do_malloc(size_t bytes, void** out) {
  Allocator& A = alloc();
  size_t sz = round_size(bytes);
  std::lock_guard<std::mutex> lk(A.mu);
  if (A.capturing) {
    // the captured graph's own free blocks first
    auto& pool = A.gpool[A.capturing];
    auto gi = pool.lower_bound(sz);
    if (gi != pool.end() && gi->first <= sz + sz / 8) {
      void* p = gi->second;
      size_t bsz = gi->first;
      pool.erase(gi);
      A.live[p] = bsz;
      A.st.active_bytes += bsz;
      if (A.st.active_bytes > A.st.peak_bytes) A.st.peak_bytes = A.st.active_bytes;
      A.st.allocations++;
      *out = p;
      return TJH_OK;
    }
  }
  auto it = A.free_blocks.lower_bound(sz);
  if (it != A.free_blocks.end() && it->first <= sz + sz / 8) {
    void* p = it->second;
    size_t bsz = it->first;
    A.free_blocks.erase(it);
    A.st.pooled_bytes -= bsz;
    A.live[p] = bsz;
    if (A.capturing) A.owner[p] = A.capturing;
    A.st.active_bytes += bsz;
    if (A.st.active_bytes > A.st.peak_bytes) A.st.peak_bytes = A.st.active_bytes;
    A.st.allocations++;
    *out = p;
    return TJH_OK;
  }
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, sz);
  if (e != hipSuccess && A.capturing) {
    (void)hipGetLastError();
    return set_error(TJH_ERR_OOM, "out of device memory allocating %zu bytes while capturing a graph",
                     sz);
  }
  if (e != hipSuccess) {
    (void)hipGetLastError();
    // Out of memory: wait for the stream, drop the cache, try once more.
    (void)hipStreamSynchronize(g_stream);
    A.release_cached_locked();
    e = hipMalloc(&p, sz);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      return set_error(TJH_ERR_OOM,
                       "out of device memory allocating %zu bytes "
                       "(active %llu bytes)",
                       sz, (unsigned long long)A.st.active_bytes);
    }
  }
  A.live[p] = sz;
  if (A.capturing) A.owner[p] = A.capturing;
  A.st.active_bytes += sz;
  if (A.st.active_bytes > A.st.peak_bytes) A.st.peak_bytes = A.st.active_bytes;
  A.st.allocations++;
  A.st.device_mallocs++;
  *out = p;
  return TJH_OK;
}

static int do_free(void* p) {
  if (!p) return TJH_OK;
  Allocator& A = alloc();
  std::lock_guard<std::mutex> lk(A.mu);
  auto it = A.live.find(p);
  if (it == A.live.end())
    return set_error(TJH_ERR_INVALID, "tjh_free: %p was not allocated by tjh_malloc", p);
  size_t sz = it->second;
  A.live.erase(it);
  A.st.active_bytes -= sz;
  int g = A.capturing;  // freed during a capture: the graph may still read it
  auto oi = A.owner.find(p);
  if (oi != A.owner.end()) g = oi->second;
  if (g) {
    A.owner[p] = g;
    A.gpool[g].emplace(sz, p);
    return TJH_OK;
  }
  A.free_blocks.emplace(sz, p);
  A.st.pooled_bytes += sz;
  return TJH_OK;
}

// ---------------------------------------------------------------- graphs

namespace {

struct Graphs {
  std::mutex mu;
  int next = 1;
  std::unordered_map<int, hipGraphExec_t> exec;
};

Graphs& graphs() {
  static Graphs* g = new Graphs();
  return *g;
}

}  // namespace

bool capturing() {
  Allocator& A = alloc();
  std::lock_guard<std::mutex> lk(A.mu);
  return A.capturing != 0;
}

void* scratch_alloc(size_t bytes) {
  void* p = nullptr;
  if (do_malloc(bytes, &p) != TJH_OK) return nullptr;
  return p;
}

void scratch_free(void* p) { (void)do_free(p); }

// ---------------------------------------------------------------- timing

namespace {

struct Family {
  std::string name;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> pending;
  int64_t launches = 0;
  double ms = 0.0;
};

struct Prof {
  std::mutex mu;
  bool on = false;
  std::string only;  // time only this family ("" = every family)
  std::vector<Family> fams;
  std::unordered_map<std::string, int> index;
  std::vector<hipEvent_t> spare;
  std::vector<hipEvent_t> timers;  // start events of wall timers
  std::unordered_map<int, hipEvent_t> timer_ends;  // end events recorded by tjh_timer_end
};

Prof& prof() {
  static Prof* p = new Prof();
  return *p;
}

hipEvent_t take_event(Prof& P) {
  if (!P.spare.empty()) {
    hipEvent_t e = P.spare.back();
    P.spare.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

// Drains finished events of every family into their totals.
void drain(Prof& P) {
  for (auto& f : P.fams) {
    for (auto& pr : f.pending) {
      float ms = 0.f;
      if (hipEventElapsedTime(&ms, pr.first, pr.second) == hipSuccess) f.ms += ms;
      P.spare.push_back(pr.first);
      P.spare.push_back(pr.second);
    }
    f.pending.clear();
  }
}

}  // namespace

static thread_local int g_open_slot = -1;  // family of the open KernelScope (-1: untimed)

KernelScope::KernelScope(const char* family) : slot(-1), prev(g_open_slot) {
  Prof& P = prof();
  if (!P.on) {
    g_open_slot = -1;
    return;
  }
  std::lock_guard<std::mutex> lk(P.mu);
  if (!P.only.empty() && P.only != family) {
    g_open_slot = -1;
    return;
  }
  auto it = P.index.find(family);
  if (it == P.index.end()) {
    P.fams.push_back(Family{family, {}, 0, 0.0});
    it = P.index.emplace(family, (int)P.fams.size() - 1).first;
  }
  slot = it->second;
  P.fams[slot].launches++;
  g_open_slot = slot;
}

KernelScope::~KernelScope() { g_open_slot = prev; }

bool launch_events(hipEvent_t* start, hipEvent_t* stop) {
  if (g_open_slot < 0 || capturing()) return false;
  Prof& P = prof();
  std::lock_guard<std::mutex> lk(P.mu);
  if (!P.on || g_open_slot >= (int)P.fams.size()) return false;
  hipEvent_t s = take_event(P);
  if (!s) return false;
  hipEvent_t e = take_event(P);
  if (!e) {
    P.spare.push_back(s);
    return false;
  }
  Family& f = P.fams[g_open_slot];
  f.pending.emplace_back(s, e);
  // keep the number of outstanding events bounded
  if (f.pending.size() > 4096) {
    f.pending.pop_back();
    (void)hipStreamSynchronize(g_stream);
    drain(P);
    f.pending.emplace_back(s, e);
  }
  *start = s;
  *stop = e;
  return true;
}

// ---------------------------------------------------------------- readbacks
//
// tjh_d2h_start enqueues a device-to-host copy into pinned staging on the
// library stream at call time (so it sees every earlier call and no later
// one), records an event and hands out a ticket; tjh_d2h_finish, on any
// thread, waits for that event and copies the staging out.  Staging
// blocks are cached (hipHostMalloc is slow) and never returned to HIP.

namespace {

struct Readback {
  void* staging;
  size_t cap;
  size_t bytes;
  hipEvent_t ev;
};

struct Readbacks {
  std::mutex mu;
  std::multimap<size_t, void*> pinned;  // capacity -> staging block
  std::unordered_map<uint64_t, Readback> live;
  std::vector<hipEvent_t> events;
  uint64_t next = 1;
};

Readbacks& readbacks() {
  static Readbacks* r = new Readbacks();
  return *r;
}

}  // namespace

}  // namespace tjh

using namespace tjh;

// ====================================================================== C ABI

extern "C" {

const char* tjh_last_error(void) { return tjh::g_err; }

const char* tjh_version(void) { return "torchjs_hip 0.1.0 (gfx950)"; }

int tjh_device_count(int* out) {
  TJH_ARG(out, "tjh_device_count: out is NULL");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    n = 0;
  }
  *out = n;
  return TJH_OK;
}

int tjh_init(int ordinal) {
  std::lock_guard<std::mutex> lk(g_init_mu);
  if (g_init) {
    if (ordinal != g_ordinal)
      return set_error(TJH_ERR_INVALID,
                       "tjh_init: already initialised on device %d, asked for %d",
                       g_ordinal, ordinal);
    return TJH_OK;
  }
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0) {
    (void)hipGetLastError();
    return set_error(TJH_ERR_HIP, "tjh_init: no HIP device available (%s)",
                     e == hipSuccess ? "0 devices" : hipGetErrorString(e));
  }
  if (ordinal < 0 || ordinal >= n)
    return set_error(TJH_ERR_INVALID, "tjh_init: ordinal %d out of range [0,%d)", ordinal, n);
  TJH_HIP(hipSetDevice(ordinal));
  hipDeviceProp_t prop;
  TJH_HIP(hipGetDeviceProperties(&prop, ordinal));
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return set_error(TJH_ERR_UNSUPPORTED,
                     "tjh_init: device %d is %s; this library is built for gfx950 only",
                     ordinal, prop.gcnArchName);
  // the static scratch of the allocation-free entry points, addressed per
  // device with this device current
  {
    int rc = noalloc_setup(ordinal);
    if (rc != TJH_OK) return rc;
  }
  // default priority stream, non-blocking w.r.t. the legacy null stream
  TJH_HIP(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking));
  g_cus = prop.multiProcessorCount;
  g_ordinal = ordinal;
  g_init = true;
  clear_error();
  return TJH_OK;
}

int tjh_is_initialized(void) { return g_init ? 1 : 0; }

int tjh_get_device_info(tjh_device_info* out) {
  TJH_REQUIRE_INIT();
  TJH_ARG(out, "tjh_get_device_info: out is NULL");
  hipDeviceProp_t prop;
  TJH_HIP(hipGetDeviceProperties(&prop, g_ordinal));
  memset(out, 0, sizeof(*out));
  snprintf(out->name, sizeof(out->name), "%s", prop.name);
  snprintf(out->arch, sizeof(out->arch), "%s", prop.gcnArchName);
  out->compute_units = prop.multiProcessorCount;
  out->warp_size = prop.warpSize;
  out->total_mem = (int64_t)prop.totalGlobalMem;
  out->max_alloc = (int64_t)prop.totalGlobalMem;
  out->lds_per_block = (int32_t)prop.sharedMemPerBlock;
  out->clock_khz = prop.clockRate;
  out->l2_bytes = prop.l2CacheSize;
  out->ordinal = g_ordinal;
  return TJH_OK;
}

int tjh_synchronize(void) {
  TJH_REQUIRE_INIT();
  if (capturing())
    return set_error(TJH_ERR_UNSUPPORTED, "%s: not allowed while a graph is being captured", __func__);
  TJH_HIP(hipStreamSynchronize(g_stream));
  return TJH_OK;
}

int tjh_malloc(size_t bytes, void** out) {
  TJH_REQUIRE_INIT();
  TJH_ARG(out, "tjh_malloc: out is NULL");
  return do_malloc(bytes, out);
}

int tjh_free(void* ptr) {
  TJH_REQUIRE_INIT();
  return do_free(ptr);
}

int tjh_memory_stats(tjh_mem_stats* out) {
  TJH_ARG(out, "tjh_memory_stats: out is NULL");
  Allocator& A = alloc();
  std::lock_guard<std::mutex> lk(A.mu);
  *out = A.st;
  return TJH_OK;
}

int tjh_empty_cache(void) {
  TJH_REQUIRE_INIT();
  if (capturing())
    return set_error(TJH_ERR_UNSUPPORTED, "%s: not allowed while a graph is being captured", __func__);
  TJH_HIP(hipStreamSynchronize(g_stream));
  Allocator& A = alloc();
  std::lock_guard<std::mutex> lk(A.mu);
  A.release_cached_locked();
  return TJH_OK;
}

int tjh_reset_peak(void) {
  Allocator& A = alloc();
  std::lock_guard<std::mutex> lk(A.mu);
  A.st.peak_bytes = A.st.active_bytes;
  return TJH_OK;
}

int tjh_h2d(void* dst, const void* src, size_t bytes) {
  TJH_REQUIRE_INIT();
  if (capturing())
    return set_error(TJH_ERR_UNSUPPORTED, "%s: not allowed while a graph is being captured", __func__);
  if (bytes == 0) return TJH_OK;
  TJH_ARG(dst && src, "tjh_h2d: NULL pointer");
  // The source is pageable host memory owned by the caller: wait for the
  // copy so the caller may reuse it as soon as we return.
  TJH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_stream));
  TJH_HIP(hipStreamSynchronize(g_stream));
  return TJH_OK;
}

int tjh_d2h(void* dst, const void* src, size_t bytes) {
  TJH_REQUIRE_INIT();
  if (capturing())
    return set_error(TJH_ERR_UNSUPPORTED, "%s: not allowed while a graph is being captured", __func__);
  if (bytes == 0) return TJH_OK;
  TJH_ARG(dst && src, "tjh_d2h: NULL pointer");
  TJH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_stream));
  TJH_HIP(hipStreamSynchronize(g_stream));
  return TJH_OK;
}

int tjh_d2h_start(const void* src, size_t bytes, uint64_t* ticket) {
  TJH_REQUIRE_INIT();
  if (capturing())
    return set_error(TJH_ERR_UNSUPPORTED, "%s: not allowed while a graph is being captured", __func__);
  TJH_ARG(ticket, "tjh_d2h_start: ticket is NULL");
  TJH_ARG(src || bytes == 0, "tjh_d2h_start: NULL source");
  Readbacks& R = readbacks();
  std::lock_guard<std::mutex> lk(R.mu);
  Readback rb{nullptr, 0, bytes, nullptr};
  if (bytes) {
    auto it = R.pinned.lower_bound(bytes);
    if (it != R.pinned.end() && it->first <= 2 * bytes + (size_t(64) << 10)) {
      rb.cap = it->first;
      rb.staging = it->second;
      R.pinned.erase(it);
    } else {
      rb.cap = (bytes + 4095) / 4096 * 4096;
      TJH_HIP(hipHostMalloc(&rb.staging, rb.cap, hipHostMallocDefault));
    }
    hipError_t e = hipMemcpyAsync(rb.staging, src, bytes, hipMemcpyDeviceToHost, g_stream);
    if (e != hipSuccess) {
      R.pinned.emplace(rb.cap, rb.staging);
      return hip_fail(e, "tjh_d2h_start: hipMemcpyAsync");
    }
  }
  if (!R.events.empty()) {
    rb.ev = R.events.back();
    R.events.pop_back();
  } else {
    hipError_t e = hipEventCreateWithFlags(&rb.ev, hipEventDisableTiming);
    if (e != hipSuccess) {
      if (rb.staging) R.pinned.emplace(rb.cap, rb.staging);
      TJH_HIP(hipStreamSynchronize(g_stream));  // the copy may still be reading staging
      return hip_fail(e, "tjh_d2h_start: hipEventCreate");
    }
  }
  TJH_HIP(hipEventRecord(rb.ev, g_stream));
  uint64_t t = R.next++;
  R.live.emplace(t, rb);
  *ticket = t;
  return TJH_OK;
}

int tjh_d2h_finish(uint64_t ticket, void* dst) {
  if (capturing())
    return set_error(TJH_ERR_UNSUPPORTED, "%s: not allowed while a graph is being captured", __func__);
  Readback rb;
  {
    Readbacks& R = readbacks();
    std::lock_guard<std::mutex> lk(R.mu);
    auto it = R.live.find(ticket);
    TJH_ARG(it != R.live.end(), "tjh_d2h_finish: unknown ticket %llu",
            (unsigned long long)ticket);
    rb = it->second;
    R.live.erase(it);
  }
  // wait outside the lock: other threads may start readbacks meanwhile
  hipError_t e = hipEventSynchronize(rb.ev);
  if (e == hipSuccess && rb.bytes) {
    if (dst) memcpy(dst, rb.staging, rb.bytes);
  }
  {
    Readbacks& R = readbacks();
    std::lock_guard<std::mutex> lk(R.mu);
    if (rb.staging) R.pinned.emplace(rb.cap, rb.staging);
    R.events.push_back(rb.ev);
  }
  if (e != hipSuccess) return hip_fail(e, "tjh_d2h_finish: hipEventSynchronize");
  TJH_ARG(dst || rb.bytes == 0, "tjh_d2h_finish: NULL destination (the ticket is released)");
  return TJH_OK;
}

int tjh_d2d(void* dst, const void* src, size_t bytes) {
  TJH_REQUIRE_INIT();
  if (bytes == 0) return TJH_OK;
  TJH_ARG(dst && src, "tjh_d2d: NULL pointer");
  KernelScope ks("copy_d2d");
  TJH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, g_stream));
  return TJH_OK;
}

int tjh_kprof_enable(int on) {
  Prof& P = prof();
  std::lock_guard<std::mutex> lk(P.mu);
  P.on = on != 0;
  return TJH_OK;
}

int tjh_kprof_filter(const char* family) {
  Prof& P = prof();
  std::lock_guard<std::mutex> lk(P.mu);
  P.only = family ? family : "";
  return TJH_OK;
}

int tjh_kprof_reset(void) {
  TJH_REQUIRE_INIT();
  TJH_HIP(hipStreamSynchronize(g_stream));
  Prof& P = prof();
  std::lock_guard<std::mutex> lk(P.mu);
  drain(P);
  for (auto& f : P.fams) {
    f.launches = 0;
    f.ms = 0.0;
  }
  return TJH_OK;
}

int tjh_kprof_query(const char* family, int64_t* launches, double* total_ms) {
  if (capturing())
    return set_error(TJH_ERR_UNSUPPORTED, "%s: not allowed while a graph is being captured", __func__);
  TJH_REQUIRE_INIT();
  TJH_ARG(family && launches && total_ms, "tjh_kprof_query: NULL argument");
  TJH_HIP(hipStreamSynchronize(g_stream));
  Prof& P = prof();
  std::lock_guard<std::mutex> lk(P.mu);
  drain(P);
  int64_t n = 0;
  double ms = 0.0;
  size_t fl = strlen(family);
  for (auto& f : P.fams) {
    if (f.name.compare(0, fl, family) == 0) {
      n += f.launches;
      ms += f.ms;
    }
  }
  *launches = n;
  *total_ms = ms;
  return TJH_OK;
}

int tjh_kprof_names(char* buf, size_t buflen) {
  TJH_ARG(buf && buflen > 0, "tjh_kprof_names: empty buffer");
  Prof& P = prof();
  std::lock_guard<std::mutex> lk(P.mu);
  std::string s;
  for (auto& f : P.fams) {
    s += f.name;
    s += '\n';
  }
  snprintf(buf, buflen, "%s", s.c_str());
  return TJH_OK;
}

int tjh_timer_start(int* id) {
  if (capturing())
    return set_error(TJH_ERR_UNSUPPORTED, "%s: not allowed while a graph is being captured", __func__);
  TJH_REQUIRE_INIT();
  TJH_ARG(id, "tjh_timer_start: id is NULL");
  Prof& P = prof();
  std::lock_guard<std::mutex> lk(P.mu);
  hipEvent_t e = take_event(P);
  if (!e) return set_error(TJH_ERR_HIP, "tjh_timer_start: hipEventCreate failed");
  TJH_HIP(hipEventRecord(e, g_stream));
  int slot = -1;
  for (int i = 0; i < (int)P.timers.size(); ++i)
    if (!P.timers[i]) { slot = i; break; }
  if (slot < 0) {
    P.timers.push_back(e);
    slot = (int)P.timers.size() - 1;
  } else {
    P.timers[slot] = e;
  }
  *id = slot;
  return TJH_OK;
}

int tjh_timer_end(int id) {
  if (capturing())
    return set_error(TJH_ERR_UNSUPPORTED, "%s: not allowed while a graph is being captured", __func__);
  TJH_REQUIRE_INIT();
  Prof& P = prof();
  std::lock_guard<std::mutex> lk(P.mu);
  TJH_ARG(id >= 0 && id < (int)P.timers.size() && P.timers[id],
          "tjh_timer_end: unknown timer %d", id);
  TJH_ARG(P.timer_ends.find(id) == P.timer_ends.end(), "tjh_timer_end: timer %d already ended",
          id);
  hipEvent_t e = take_event(P);
  if (!e) return set_error(TJH_ERR_HIP, "tjh_timer_end: hipEventCreate failed");
  TJH_HIP(hipEventRecord(e, g_stream));
  P.timer_ends[id] = e;
  return TJH_OK;
}

int tjh_timer_read(int id, double* ms) {
  if (capturing())
    return set_error(TJH_ERR_UNSUPPORTED, "%s: not allowed while a graph is being captured", __func__);
  TJH_REQUIRE_INIT();
  TJH_ARG(ms, "tjh_timer_read: ms is NULL");
  hipEvent_t s0, e;
  {
    Prof& P = prof();
    std::lock_guard<std::mutex> lk(P.mu);
    auto it = P.timer_ends.find(id);
    TJH_ARG(id >= 0 && id < (int)P.timers.size() && P.timers[id] && it != P.timer_ends.end(),
            "tjh_timer_read: timer %d was not ended", id);
    s0 = P.timers[id];
    e = it->second;
  }
  TJH_HIP(hipEventSynchronize(e));
  float t = 0.f;
  TJH_HIP(hipEventElapsedTime(&t, s0, e));
  *ms = t;
  Prof& P = prof();
  std::lock_guard<std::mutex> lk(P.mu);
  P.timer_ends.erase(id);
  P.spare.push_back(s0);
  P.spare.push_back(e);
  P.timers[id] = nullptr;
  return TJH_OK;
}

int tjh_range_push(const char* name) {
  TJH_ARG(name, "tjh_range_push: name is NULL");
  roctxRangePushA(name);
  return TJH_OK;
}

int tjh_range_pop(void) {
  roctxRangePop();
  return TJH_OK;
}

int tjh_mark(const char* name) {
  TJH_ARG(name, "tjh_mark: name is NULL");
  roctxMarkA(name);
  return TJH_OK;
}

int tjh_timer_stop(int id, double* ms) {
  if (capturing())
    return set_error(TJH_ERR_UNSUPPORTED, "%s: not allowed while a graph is being captured", __func__);
  TJH_REQUIRE_INIT();
  TJH_ARG(ms, "tjh_timer_stop: ms is NULL");
  Prof& P = prof();
  std::lock_guard<std::mutex> lk(P.mu);
  TJH_ARG(id >= 0 && id < (int)P.timers.size() && P.timers[id],
          "tjh_timer_stop: unknown timer %d", id);
  hipEvent_t e = take_event(P);
  if (!e) return set_error(TJH_ERR_HIP, "tjh_timer_stop: hipEventCreate failed");
  TJH_HIP(hipEventRecord(e, g_stream));
  TJH_HIP(hipEventSynchronize(e));
  float t = 0.f;
  TJH_HIP(hipEventElapsedTime(&t, P.timers[id], e));
  *ms = t;
  P.spare.push_back(P.timers[id]);
  P.spare.push_back(e);
  P.timers[id] = nullptr;
  return TJH_OK;
}


// ---------------------------------------------------------------- graphs

int tjh_graph_begin(int* graph) {
  TJH_REQUIRE_INIT();
  TJH_ARG(graph, "tjh_graph_begin: graph is NULL");
  Allocator& A = alloc();
  {
    std::lock_guard<std::mutex> lk(A.mu);
    if (A.capturing) return set_error(TJH_ERR_INVALID, "tjh_graph_begin: a capture is already open");
  }
  int id;
  {
    Graphs& G = graphs();
    std::lock_guard<std::mutex> lk(G.mu);
    id = G.next++;
  }
  // relaxed: allocations (hipMalloc) stay legal while the stream captures
  TJH_HIP(hipStreamBeginCapture(g_stream, hipStreamCaptureModeRelaxed));
  {
    std::lock_guard<std::mutex> lk(A.mu);
    A.capturing = id;
  }
  *graph = id;
  return TJH_OK;
}

namespace {
// Returns graph g's free blocks to the general cache and forgets which
// live blocks it owned (they go to the cache when freed).
void release_graph_blocks(int g) {
  Allocator& A = alloc();
  std::lock_guard<std::mutex> lk(A.mu);
  auto pi = A.gpool.find(g);
  if (pi != A.gpool.end()) {
    for (auto& kv : pi->second) {
      A.free_blocks.emplace(kv.first, kv.second);
      A.st.pooled_bytes += kv.first;
      A.owner.erase(kv.second);
    }
    A.gpool.erase(pi);
  }
  for (auto it = A.owner.begin(); it != A.owner.end();) {
    if (it->second == g) it = A.owner.erase(it);
    else ++it;
  }
}
}  // namespace

int tjh_graph_end(int graph) {
  TJH_REQUIRE_INIT();
  Allocator& A = alloc();
  {
    std::lock_guard<std::mutex> lk(A.mu);
    if (A.capturing != graph || graph == 0)
      return set_error(TJH_ERR_INVALID, "tjh_graph_end: graph %d is not being captured", graph);
  }
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(g_stream, &g);
  {
    std::lock_guard<std::mutex> lk(A.mu);
    A.capturing = 0;
  }
  hipGraphExec_t ex = nullptr;
  if (e == hipSuccess) e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
  if (g) (void)hipGraphDestroy(g);
  if (e != hipSuccess) {
    (void)hipStreamSynchronize(g_stream);
    release_graph_blocks(graph);
    return hip_fail(e, "tjh_graph_end");
  }
  Graphs& G = graphs();
  std::lock_guard<std::mutex> lk(G.mu);
  G.exec[graph] = ex;
  return TJH_OK;
}

int tjh_graph_replay(int graph) {
  TJH_REQUIRE_INIT();
  if (capturing())
    return set_error(TJH_ERR_UNSUPPORTED, "tjh_graph_replay: not allowed while a graph is being captured");
  hipGraphExec_t ex = nullptr;
  {
    Graphs& G = graphs();
    std::lock_guard<std::mutex> lk(G.mu);
    auto it = G.exec.find(graph);
    if (it == G.exec.end()) return set_error(TJH_ERR_INVALID, "tjh_graph_replay: no graph %d", graph);
    ex = it->second;
  }
  TJH_HIP(hipGraphLaunch(ex, g_stream));
  return TJH_OK;
}

int tjh_graph_destroy(int graph) {
  TJH_REQUIRE_INIT();
  hipGraphExec_t ex = nullptr;
  {
    Graphs& G = graphs();
    std::lock_guard<std::mutex> lk(G.mu);
    auto it = G.exec.find(graph);
    if (it == G.exec.end()) return set_error(TJH_ERR_INVALID, "tjh_graph_destroy: no graph %d", graph);
    ex = it->second;
    G.exec.erase(it);
  }
  // a replay may still be running: its blocks are released once it is done
  TJH_HIP(hipStreamSynchronize(g_stream));
  TJH_HIP(hipGraphExecDestroy(ex));
  release_graph_blocks(graph);
  return TJH_OK;
}

}  // extern "C"
