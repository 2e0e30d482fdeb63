// Shared internals of libtorchjs_hip.so: error reporting, the library
// stream, launch checking, per-family launch timing and scratch memory.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/torchjs_hip.h"

namespace tjh {

// Sets the thread-local error message and returns `code`.
int set_error(int code, const char* fmt, ...);
void clear_error();

// The library stream (valid after tjh_init).
hipStream_t stream();
bool initialized();
int device_ordinal();
int num_cus();
// Takes the device address of the allocation-free entry points' static
// scratch (norm.hip) for the current device; tjh_init calls it once.
int noalloc_setup(int ordinal);

// Whether the library stream is being captured into a HIP graph (then
// host copies, synchronisation and timing events are refused).
bool capturing();

// Returns TJH_ERR_NOT_INITIALIZED (with message) unless tjh_init succeeded.
int require_init();

// Maps a HIP error to TJH_ERR_HIP with the call site in the message.
int hip_fail(hipError_t e, const char* what);

// Per-family launch timing.  A `KernelScope` names the family of the
// kernels launched while it is open and counts one call of that family;
// when timing is enabled (tjh_kprof_enable) each kernel launched through
// tjh_launch inside it carries a start / stop event pair on its own
// dispatch (hipExtLaunchKernel), so the family's time is the sum of its
// kernels' execution times, with no marker packets between launches.
struct KernelScope {
  int slot;
  int prev;  // the enclosing scope's slot, restored on close
  explicit KernelScope(const char* family);
  ~KernelScope();
};

// Two timing events for the next kernel of the open scope, or false when
// that kernel is not timed.
bool launch_events(hipEvent_t* start, hipEvent_t* stop);

// Launches a kernel on `s` (the library stream), timed by its dispatch
// timestamps when the open KernelScope is being timed.
template <typename... Args, typename F = void (*)(Args...)>
inline void tjh_launch(F kernel, const dim3& grid, const dim3& block, uint32_t shmem,
                       hipStream_t s, Args... args) {
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (launch_events(&e0, &e1))
    hipExtLaunchKernelGGL(kernel, grid, block, shmem, s, e0, e1, 0, args...);
  else
    hipLaunchKernelGGL(kernel, grid, block, shmem, s, args...);
}

// Checks hipGetLastError after a launch; returns TJH_OK or TJH_ERR_HIP.
int check_launch(const char* kernel);

// Stream-ordered scratch from the caching allocator.  Released with
// scratch_free once the kernels using it have been enqueued.
void* scratch_alloc(size_t bytes);
void scratch_free(void* p);

// RAII holder for scratch memory.
struct Scratch {
  void* p = nullptr;
  explicit Scratch(size_t bytes) { if (bytes) p = scratch_alloc(bytes); }
  ~Scratch() { if (p) scratch_free(p); }
  template <typename T> T* as() const { return static_cast<T*>(p); }
  bool ok() const { return p != nullptr; }
  // hands the block to the caller, who scratch_free()s it later
  void* release() {
    void* q = p;
    p = nullptr;
    return q;
  }
};

// The MFMA GEMM behind tjh_gemm / tjh_gemm_act, timed under `family` (so
// products issued inside attention are reported apart from tjh_gemm's).
// act: 0 none, 1 GELU (aux <- pre-activation), 2 times GELU'(aux).
int gemm(const char* family, int transA, int transB, int64_t M, int64_t N, int64_t K,
         float alpha, const float* A, int64_t lda, int64_t strideA, const float* B, int64_t ldb,
         int64_t strideB, float beta, float* C, int64_t ldc, int64_t strideC, int64_t batch,
         const float* bias, int bias_mode, float* aux = nullptr, int64_t ldaux = 0, int act = 0,
         const float* ce_rows = nullptr);

// Flash attention for head dims D <= 128, D % 4 == 0 (flash.hip).
// `flash_supported` checks the head dim and that every tensor has 16-byte
// aligned, D-contiguous rows.
bool flash_supported(int64_t D, const void* const* ptrs, const int64_t* const* strides, int n);
int flash_forward(const float* q, const float* k, const float* v, float* o, float* lse, int64_t B,
                  int64_t H, int64_t Tq, int64_t Tk, int64_t D, const int64_t* qs,
                  const int64_t* ks, const int64_t* vs, const int64_t* os, float scale,
                  int causal);
int flash_backward(const float* q, const float* k, const float* v, const float* o,
                   const float* dout, const float* lse, float* dq, float* dk, float* dv,
                   int64_t B, int64_t H, int64_t Tq, int64_t Tk, int64_t D,
                   const int64_t* const* strides, float scale, int causal);

// 16-byte alignment of a device pointer (128-bit access paths).
inline bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Streaming (non-temporal) 128-bit global loads and stores, for data that
// is dead after the access (optimizer state, logits read by the loss
// backward): on MI355X they lift a 1 GiB copy from 5.7 to 6.2 TB/s, but a
// tensor written this way and read by the next kernel is no longer in the
// caches, so outputs consumed downstream use ordinary stores.
typedef float nt_floatx4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld_nt(const float* p) {
  const nt_floatx4 v = __builtin_nontemporal_load(reinterpret_cast<const nt_floatx4*>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st_nt(float* p, const float4& v) {
  __builtin_nontemporal_store(nt_floatx4{v.x, v.y, v.z, v.w}, reinterpret_cast<nt_floatx4*>(p));
}

// Grid size helper: ceil(n / d).
__host__ __device__ inline int64_t cdiv(int64_t n, int64_t d) { return (n + d - 1) / d; }

}  // namespace tjh

#define TJH_REQUIRE_INIT()                   \
  do {                                       \
    int _rc = ::tjh::require_init();         \
    if (_rc != TJH_OK) return _rc;           \
  } while (0)

#define TJH_HIP(call)                                  \
  do {                                                 \
    hipError_t _e = (call);                            \
    if (_e != hipSuccess) return ::tjh::hip_fail(_e, #call); \
  } while (0)

#define TJH_ARG(cond, ...)                                          \
  do {                                                              \
    if (!(cond)) return ::tjh::set_error(TJH_ERR_INVALID, __VA_ARGS__); \
  } while (0)
