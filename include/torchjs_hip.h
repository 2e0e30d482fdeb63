/*
 * torchjs_hip.h — C ABI of libtorchjs_hip.so, the MI355X (gfx950) compute
 * backend behind torch.js's `'hip'` device.
 *
 * torch.js has no backend interface of its own: every op builds WebGPU
 * objects inline and submits them (src/backend/index.ts:6 re-exports
 * src/backend/webgpu/index.ts:6-25).  This header is the boundary that
 * replaces that runtime (device init, buffer pool, uploads/readbacks,
 * pipeline dispatch, queue sync) and the WGSL kernels of the autograd hot
 * path.  Each declaration names the reference interface it replaces.
 *
 * Conventions
 *  - Every function returns an int status (TJH_OK == 0).  On failure a
 *    thread-local message is available from tjh_last_error().
 *  - All device work is enqueued on ONE library-owned HIP stream, so the
 *    order of calls is the order of execution, like WebGPU's single queue
 *    (src/backend/webgpu/dispatch.ts:115-118).  Kernel entry points are
 *    asynchronous; tjh_d2h and tjh_synchronize block.
 *  - Device pointers are plain `void*`/`float*` obtained from tjh_malloc.
 *    Floating-point data is IEEE fp32; index data is int32 (torch.js
 *    stores integer tensors as Int32Array, src/dtype.ts:7-15).
 *  - Shapes and strides are int64 arrays counted in ELEMENTS, ndim <= 8.
 */
#ifndef TORCHJS_HIP_H
#define TORCHJS_HIP_H

/* runtime-compiled kernels (hipRTC) include this header for its op codes;
 * hipRTC defines the fixed-width integer types itself */
#ifndef __HIPCC_RTC__
#include <stddef.h>
#include <stdint.h>
#else
typedef __hip_internal::uint8_t uint8_t;
typedef __hip_internal::int32_t int32_t;
typedef __hip_internal::uint32_t uint32_t;
typedef __hip_internal::int64_t int64_t;
typedef __hip_internal::uint64_t uint64_t;
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define TJH_MAX_DIMS 8

/* status codes */
#define TJH_OK 0
#define TJH_ERR_INVALID 1         /* bad argument (shape, pointer, op code) */
#define TJH_ERR_NOT_INITIALIZED 2 /* tjh_init not called                   */
#define TJH_ERR_OOM 3             /* device allocation failed              */
#define TJH_ERR_HIP 4             /* HIP runtime error                     */
#define TJH_ERR_UNSUPPORTED 5     /* valid request the library cannot do   */

/* ------------------------------------------------------------------ */
/* Lifecycle — replaces initWebGPU / getDevice / getCapabilities /      */
/* syncDevice (src/backend/webgpu/device.ts:27-97,                      */
/* src/backend/webgpu/capabilities.ts:42-101,                           */
/* src/backend/webgpu/dispatch.ts:115-118).                             */
/* ------------------------------------------------------------------ */

typedef struct {
  char name[256];         /* marketing name                                */
  char arch[64];          /* gcnArchName, e.g. "gfx950:sramecc+:xnack-"    */
  int32_t compute_units;
  int32_t warp_size;      /* 64 on CDNA                                    */
  int64_t total_mem;      /* bytes of HBM                                  */
  int64_t max_alloc;      /* largest single allocation accepted            */
  int32_t lds_per_block;  /* bytes                                         */
  int32_t clock_khz;
  int32_t l2_bytes;
  int32_t ordinal;
} tjh_device_info;

/* Message of the last failing call on this thread ("" when none). */
const char* tjh_last_error(void);
/* Library version string. */
const char* tjh_version(void);
/* Idempotent device init (like initWebGPU, device.ts:27-86): selects the
 * device, creates the library stream.  A second call with another ordinal
 * fails with TJH_ERR_INVALID. */
int tjh_init(int ordinal);
/* 1 if tjh_init succeeded, else 0 (the "WebGPU not initialized" check,
 * device.ts:92-97). */
int tjh_is_initialized(void);
/* Number of visible HIP devices (0 when none; never initialises one). */
int tjh_device_count(int* out);
/* Capability query (getCapabilities, capabilities.ts:42-101). */
int tjh_get_device_info(tjh_device_info* out);
/* Block until every enqueued call has finished (syncDevice). */
int tjh_synchronize(void);

/* ------------------------------------------------------------------ */
/* Memory — replaces GPUBufferPool / createStorageBuffer /              */
/* createBufferWithData / readBuffer / copyBufferToBuffer and           */
/* torch.webgpu.memory_stats (src/backend/webgpu/buffer.ts:10-206,      */
/* src/webgpu.ts:11-51).                                                */
/* ------------------------------------------------------------------ */

typedef struct {
  uint64_t active_bytes;  /* bytes handed out and not yet freed          */
  uint64_t pooled_bytes;  /* bytes cached for reuse                       */
  uint64_t peak_bytes;    /* max active_bytes since the last reset        */
  uint64_t allocations;   /* tjh_malloc calls served                      */
  uint64_t device_mallocs;/* hipMalloc calls made (cache misses): the
                             reference's allocationCount /
                             total_allocations, which count the buffers its
                             pool creates (buffer.ts:50-57)               */
} tjh_mem_stats;

/* Stream-ordered caching allocator on HBM.  Blocks are 256-byte aligned.
 * A block released by tjh_free may be handed out again at once: every
 * later use is on the same stream, so it runs after the work that used
 * the block before (GPUBufferPool.acquire/release, buffer.ts:21-114).
 * bytes == 0 returns a valid unique pointer. */
int tjh_malloc(size_t bytes, void** out);
int tjh_free(void* ptr);
int tjh_memory_stats(tjh_mem_stats* out);
/* Synchronises and returns every cached block to HIP (bufferPool.clear). */
int tjh_empty_cache(void);
int tjh_reset_peak(void);

/* Copies.  tjh_h2d and tjh_d2d are stream-ordered; tjh_d2h waits for the
 * stream and returns with `dst` filled (readBuffer, buffer.ts:150-206). */
int tjh_h2d(void* dst, const void* src, size_t bytes);
int tjh_d2h(void* dst, const void* src, size_t bytes);
int tjh_d2d(void* dst, const void* src, size_t bytes);
/* Asynchronous readback, the mapAsync path of readBuffer
 * (src/backend/webgpu/buffer.ts:150-206, Tensor.toArray, Tensor.ts:253-257):
 * tjh_d2h_start enqueues the copy of `bytes` from `src` into pinned staging
 * owned by the library, in stream order at the time of the call (it sees
 * every earlier call; later calls, including frees and kernels writing
 * `src`, cannot change what it reads), and returns a ticket.
 * tjh_d2h_finish waits for that copy, writes the bytes to `dst` and
 * releases the ticket; it may run on another thread (a Node-API worker)
 * while the caller keeps launching work. */
int tjh_d2h_start(const void* src, size_t bytes, uint64_t* ticket);
int tjh_d2h_finish(uint64_t ticket, void* dst);

/* ------------------------------------------------------------------ */
/* Timing — device-side counterpart of the profiler's record_function   */
/* (src/profiler/index.ts:145-166) and benchmark Timer                  */
/* (src/utils/benchmark/timer.ts:45-108).  When enabled, each launch of */
/* a kernel family is bracketed by HIP events on the library stream.    */
/* ------------------------------------------------------------------ */

int tjh_kprof_enable(int on);
/* Restricts timing to the family named exactly `family` (NULL or "" =
 * every family), so a timed region brackets only the launches it reports
 * and the others run without events between them. */
int tjh_kprof_filter(const char* family);
int tjh_kprof_reset(void);
/* Synchronises, then reports launches and summed event time for every
 * kernel family whose name starts with `family` ("" = all). */
int tjh_kprof_query(const char* family, int64_t* launches, double* total_ms);
/* Names of families seen so far, '\n'-separated, into buf (truncated). */
int tjh_kprof_names(char* buf, size_t buflen);
/* Wall timer on the stream: returns an id; tjh_timer_stop gives ms. */
int tjh_timer_start(int* id);
int tjh_timer_stop(int id, double* ms);
/* The same timer closed without waiting (tjh_timer_end records the end on
 * the stream) and read later (tjh_timer_read waits for that end and
 * releases the id): the device time of a record_function block. */
int tjh_timer_end(int id);
int tjh_timer_read(int id, double* ms);
/* Named ranges and marks on the ROCm tracer's marker timeline (roctx),
 * the device-side counterpart of record_function
 * (src/profiler/index.ts:145-166): `rocprofv3 --marker-trace` shows each
 * range around the kernels launched while it is open.  Cheap no-ops when
 * no tracer is attached. */
int tjh_range_push(const char* name);
int tjh_range_pop(void);
int tjh_mark(const char* name);

/* ------------------------------------------------------------------ */
/* Fill / RNG / copies — fill.wgsl, random.wgsl:9-46 (with the LCG seed */
/* step of src/ops/creation.ts:921 applied by the host), expand.wgsl,   */
/* transpose(_nd).wgsl, slice(_backward).wgsl, Tensor.cat               */
/* (Tensor.ts:152-235, 1537-2130).                                      */
/* ------------------------------------------------------------------ */

int tjh_fill_f32(float* out, int64_t n, float value);
int tjh_fill_i32(int32_t* out, int64_t n, int32_t value);
/* normal == 0: U[0,1) = xorshift32(seed ^ (i*1664525+1013904223)) / 2^32;
 * normal != 0: Box-Muller of two successive xorshift32 states. */
int tjh_random(float* out, int64_t n, uint32_t seed, int normal);
/* dst[idx] = src[idx] for every index of `shape`, both sides strided
 * (permute, contiguous, expand, slice, slice-backward, cat). */
int tjh_copy_strided(int ndim, const int64_t* shape,
                     const float* src, const int64_t* src_strides,
                     float* dst, const int64_t* dst_strides);
/* int32 variant (index tensors). */
int tjh_copy_strided_i32(int ndim, const int64_t* shape,
                         const int32_t* src, const int64_t* src_strides,
                         int32_t* dst, const int64_t* dst_strides);
/* float <-> int32 conversions (Tensor.to(dtype)); f2i truncates toward 0 */
int tjh_cast_f32_i32(const float* src, int32_t* dst, int64_t n);
int tjh_cast_i32_f32(const int32_t* src, float* dst, int64_t n);
/* Element types of tjh_cast: float32, int32, uint8 and bool (one byte per
 * element, 0 / 1) — the dtypes torch.js keeps (src/dtype.ts:7-15). */
enum { TJH_DTYPE_F32 = 0, TJH_DTYPE_I32, TJH_DTYPE_U8, TJH_DTYPE_BOOL, TJH_DTYPE_COUNT };
/* Tensor.to(dtype) / .bool() / .float() / .int() between any two of them:
 * to bool is `!= 0`; float to an integer type truncates toward zero; to
 * uint8 keeps the low 8 bits of that integer. */
int tjh_cast(int src_dtype, int dst_dtype, const void* src, void* dst,
             int64_t n);
/* uint8 / bool fills and strided copies (masks, Tensor.bool()). */
int tjh_fill_u8(uint8_t* out, int64_t n, uint8_t value);
int tjh_copy_strided_u8(int ndim, const int64_t* shape,
                        const uint8_t* src, const int64_t* src_strides,
                        uint8_t* dst, const int64_t* dst_strides);
/* Tensor.triu / tril (triu.wgsl, tril.wgsl) of `batch` contiguous
 * [rows, cols] matrices: element (r, c) is kept when c - r >= diagonal
 * (upper != 0) or c - r <= diagonal, else 0.  Also the backward (the
 * same mask applied to the gradient). */
int tjh_triangle(const float* x, float* out, int64_t batch, int64_t rows,
                 int64_t cols, int64_t diagonal, int upper);

/* ------------------------------------------------------------------ */
/* Elementwise — elementwise.wgsl:5-31, broadcast.wgsl:28-175,          */
/* scalar.wgsl:10-67, unary.wgsl:5-252, masked_fill.wgsl, and the       */
/* backward formulas the reference lacks (Tensor.ts:3409-3656).         */
/* ------------------------------------------------------------------ */

/* unary op codes */
enum {
  TJH_UNARY_NEG = 0, TJH_UNARY_EXP, TJH_UNARY_LOG, TJH_UNARY_SQRT,
  TJH_UNARY_RSQRT, TJH_UNARY_TANH, TJH_UNARY_SIGMOID, TJH_UNARY_RELU,
  TJH_UNARY_GELU, TJH_UNARY_SQUARE, TJH_UNARY_RECIPROCAL, TJH_UNARY_ERF,
  TJH_UNARY_ABS, TJH_UNARY_SIN, TJH_UNARY_COS, TJH_UNARY_SILU,
  TJH_UNARY_LEAKY_RELU, TJH_UNARY_ELU, TJH_UNARY_SOFTPLUS, TJH_UNARY_SIGN,
  TJH_UNARY_COUNT
};
/* binary op codes (tensor op tensor); pow = a^b */
enum {
  TJH_BINARY_ADD = 0, TJH_BINARY_SUB, TJH_BINARY_MUL, TJH_BINARY_DIV,
  TJH_BINARY_POW, TJH_BINARY_MAXIMUM, TJH_BINARY_MINIMUM,
  TJH_BINARY_COUNT
};
/* scalar op codes: out = x op s (reverse != 0: out = s op x) */
enum {
  TJH_SCALAR_ADD = 0, TJH_SCALAR_SUB, TJH_SCALAR_MUL, TJH_SCALAR_DIV,
  TJH_SCALAR_POW, TJH_SCALAR_MAXIMUM, TJH_SCALAR_MINIMUM,
  TJH_SCALAR_COUNT
};

/* out[i] = op(x[i]); alpha is the slope/alpha of leaky_relu/elu. */
int tjh_unary(int op, const float* x, float* out, int64_t n, float alpha);
/* out[i] = g[i] * op'(x[i]) using the saved input x and/or output y
 * (y may be NULL for ops whose derivative needs only x). */
int tjh_unary_backward(int op, const float* g, const float* x,
                       const float* y, float* out, int64_t n, float alpha);
/* out (contiguous, `shape`) = a op b with broadcast strides (0 = broadcast
 * dim).  Handles any ndim <= 8; contiguous and row-broadcast layouts take
 * vectorised paths. */
int tjh_binary(int op, int ndim, const int64_t* shape,
               const float* a, const int64_t* a_strides,
               const float* b, const int64_t* b_strides, float* out);
/* Ternary backward helpers over a contiguous, common shape:
 *  TJH_TERNARY_DIV_B:  out = -g * a / (b*b)
 *  TJH_TERNARY_POW_A:  out =  g * b * a^(b-1)
 *  TJH_TERNARY_POW_B:  out =  g * a^b * ln(a)
 *  TJH_TERNARY_MUL3 :  out =  g * a * b
 * Each operand is strided over `shape` like tjh_binary. */
enum { TJH_TERNARY_DIV_B = 0, TJH_TERNARY_POW_A, TJH_TERNARY_POW_B,
       TJH_TERNARY_MUL3, TJH_TERNARY_COUNT };
int tjh_ternary(int op, int ndim, const int64_t* shape,
                const float* g, const int64_t* g_strides,
                const float* a, const int64_t* a_strides,
                const float* b, const int64_t* b_strides, float* out);
int tjh_scalar(int op, const float* x, float s, int reverse, float* out,
               int64_t n);
/* pow_scalar backward: out = g * s * x^(s-1) (scalar.wgsl:53-66 for the
 * forward's integer-exponent rule). */
int tjh_pow_scalar_backward(const float* g, const float* x, float s,
                            float* out, int64_t n);
/* out = alpha*x + y, contiguous (accumulateGrad, Tensor.ts:3670-3677). */
int tjh_axpy(float alpha, const float* x, const float* y, float* out,
             int64_t n);
/* out = mask[idx] != 0 ? value : x[idx]; mask is uint8, strided (may
 * broadcast).  Backward is the same call with x = g and value = 0
 * (masked_fill.wgsl, Tensor.ts:804-832). */
int tjh_masked_fill(int ndim, const int64_t* shape,
                    const float* x, const int64_t* x_strides,
                    const uint8_t* mask, const int64_t* mask_strides,
                    float value, float* out);
/* comparisons producing float 0/1 (compare.wgsl): op 0 eq,1 ne,2 lt,3 le,
 * 4 gt, 5 ge; b strided over shape like tjh_binary. */
int tjh_compare(int op, int ndim, const int64_t* shape,
                const float* a, const int64_t* a_strides,
                const float* b, const int64_t* b_strides, float* out);

/* ------------------------------------------------------------------ */
/* Reductions — reduce_sum.wgsl (+max/min/prod), reduce_dim.wgsl,       */
/* reduce_broadcast_grad.wgsl, argmax (Tensor.ts:2359-2577, 3794-3906). */
/* ------------------------------------------------------------------ */

enum { TJH_REDUCE_SUM = 0, TJH_REDUCE_MEAN, TJH_REDUCE_MAX, TJH_REDUCE_MIN,
       TJH_REDUCE_PROD, TJH_REDUCE_COUNT };
/* x viewed as contiguous [outer, r, inner]; out[outer, inner] = reduce
 * over r.  Deterministic (fixed split and combine order).  outer=inner=1
 * is the full reduction; outer=1 is the broadcast-grad column sum. */
int tjh_reduce(int op, const float* x, int64_t outer, int64_t r,
               int64_t inner, float* out);
/* first index of the max (min when is_min) along r; ties keep the first
 * index (Tensor.ts:2568). */
int tjh_argmax(const float* x, int64_t outer, int64_t r, int64_t inner,
               int is_min, int32_t* out);

/* ------------------------------------------------------------------ */
/* HIP graphs — no counterpart in the reference (WebGPU has no command   */
/* replay): for callers whose steps are bound by host-side launch cost   */
/* (small MLPs, elementwise chains), the work a step enqueues on the     */
/* library stream is captured once and replayed with one launch.        */
/* ------------------------------------------------------------------ */

/* Starts capturing the library stream into a new graph (id in *graph).
 * While capturing, every entry point enqueues instead of running; host
 * copies, synchronisation, timers and nonzero are refused
 * (TJH_ERR_UNSUPPORTED).  Memory allocated or freed during the capture
 * belongs to the graph: it is never handed to other work until
 * tjh_graph_destroy, so replays may rewrite it. */
int tjh_graph_begin(int* graph);
/* Ends the capture and instantiates the graph. */
int tjh_graph_end(int graph);
/* Enqueues one replay on the library stream (same pointers, same
 * arguments as captured). */
int tjh_graph_replay(int graph);
/* Waits for the stream, destroys the graph and releases its memory. */
int tjh_graph_destroy(int graph);

/* ------------------------------------------------------------------ */
/* Fused elementwise expressions — one launch for a chain of the unary / */
/* binary / scalar / ternary ops above, which the reference runs as one */
/* submit each (Tensor.ts _unaryOp / _binaryOp / _broadcastBinaryOp /   */
/* _scalarOp, 3409-3656, 3742-3792), and for the broadcast-gradient     */
/* column sum of such a chain (Tensor.ts:3560-3591).                    */
/* ------------------------------------------------------------------ */

#define TJH_EXPR_MAX_INS 48
#define TJH_EXPR_MAX_LEAVES 8
#define TJH_EXPR_MAX_REGS 16
#define TJH_EXPR_NONE 255 /* absent optional register operand */

/* instruction kinds: dst <- ...
 *  LOAD       leaf[a]
 *  CONST      f
 *  UNARY      unary op `code` of r[a] (alpha f)
 *  UNARY_BWD  tjh_unary_backward's value for op `code`: g = r[a], x = r[b],
 *             y = r[c] (b / c may be TJH_EXPR_NONE when the op does not
 *             read them), alpha f
 *  BINARY     binary op `code` of r[a], r[b]
 *  TERNARY    ternary op `code` of g = r[a], a = r[b], b = r[c]
 *  SCALAR     scalar op `code`: r[a] (op) f;  SCALAR_REV: f (op) r[a]
 *  AXPY       f * r[a] + r[b]                                            */
enum { TJH_EXPR_LOAD = 0, TJH_EXPR_CONST, TJH_EXPR_UNARY, TJH_EXPR_UNARY_BWD,
       TJH_EXPR_BINARY, TJH_EXPR_TERNARY, TJH_EXPR_SCALAR, TJH_EXPR_SCALAR_REV,
       TJH_EXPR_AXPY, TJH_EXPR_OPS };
/* how leaf k is indexed at output element e: CONTIG e, ROW e % period,
 * COL e / period, SCALAR 0 */
enum { TJH_LEAF_CONTIG = 0, TJH_LEAF_ROW, TJH_LEAF_COL, TJH_LEAF_SCALAR };

typedef struct {
  uint8_t op, code, dst, a, b, c, pad0, pad1;
  float f;
} tjh_expr_ins;

/* A program: n_ins instructions in order over TJH_EXPR_MAX_REGS
 * registers (each source defined by an earlier instruction); the value of
 * output element e is r[result] after the last one.  Every instruction
 * computes exactly what the single-op entry points compute.  result2, when
 * not 0, names a second value r[result2 - 1] that tjh_expr_colsum2 also
 * writes out (two values of one chain, computed from the same loads);
 * result3, when not 0, a third value r[result3 - 1] that tjh_expr_colsum3
 * also sums over the same rows. */
typedef struct {
  int32_t n_ins, n_leaves, result, result2, result3, pad;
  tjh_expr_ins ins[TJH_EXPR_MAX_INS];
  const float* leaf[TJH_EXPR_MAX_LEAVES];
  int64_t period[TJH_EXPR_MAX_LEAVES];
  int32_t kind[TJH_EXPR_MAX_LEAVES];
} tjh_expr;

/* out[e] = value(e), e in [0, n). */
int tjh_expr_eval(const tjh_expr* prog, int64_t n, float* out);
/* Value viewed as contiguous [outer, r, inner]: out[outer, inner] = sum
 * over r, bit-identical to tjh_reduce(TJH_REDUCE_SUM) of the materialised
 * value (16-byte aligned, inner % 4 == 0) and of the same determinism;
 * `values` (may be NULL) also receives the value.  Needs outer <= 64,
 * r >= 64, inner >= 2 (else TJH_ERR_UNSUPPORTED). */
int tjh_expr_colsum(const tjh_expr* prog, int64_t outer, int64_t r, int64_t inner,
                    float* out, float* values);
/* tjh_expr_colsum that also writes the program's second value
 * (prog->result2 != 0) to `values2` (may be NULL), in the same pass: the
 * gradients of two inputs of one elementwise chain (y's and x's of
 * GELU(x + b) * y, the latter with the bias gradient's column sum) from
 * one read of the chain's inputs. */
int tjh_expr_colsum2(const tjh_expr* prog, int64_t outer, int64_t r, int64_t inner,
                     float* out, float* values, float* values2);
/* tjh_expr_colsum2 that also sums the program's third value
 * (prog->result3 != 0) over the same rows into out3 [outer, inner], with
 * the same partition and order (bit-identical to summing that value
 * alone): a forward column sum left pending until the backward pass reads
 * the same inputs (the loss of GELU(x + b) * y summed over rows, from the
 * pass that forms x's and y's gradients).  Needs 2 * outer <= 64. */
int tjh_expr_colsum3(const tjh_expr* prog, int64_t outer, int64_t r, int64_t inner,
                     float* out, float* values, float* values2, float* out3);
/* Validates `prog` and compiles the kernel tjh_expr_eval (colsum == 0) or
 * tjh_expr_colsum (colsum != 0) would run for n elements, without a
 * device (kernels are compiled at run time, once per program shape). */
int tjh_expr_compile(const tjh_expr* prog, int64_t n, int colsum);

/* ------------------------------------------------------------------ */
/* Softmax / losses — log_softmax.wgsl, log_softmax_backward.wgsl,      */
/* nll_loss(_backward).wgsl; F.softmax/F.log_softmax/F.cross_entropy/   */
/* F.nll_loss (src/nn/functional.ts:79-234, src/nn/losses.ts:18-145).   */
/* ------------------------------------------------------------------ */

/* y = softmax(x) or log_softmax(x) over the last dim of [rows, cols],
 * row strides ldx/ldy (>= cols). */
int tjh_softmax_forward(const float* x, int64_t ldx, float* y, int64_t ldy,
                        int64_t rows, int64_t cols, int log);
/* dx from y and dy: softmax: y*(dy - sum(dy*y)); log: dy - exp(y)*sum(dy). */
int tjh_softmax_backward(const float* dy, const float* y, float* dx,
                         int64_t rows, int64_t cols, int log);
/* Reductions of the losses (apply_reduction, losses.ts:18-32):
 *   0 none      per-row losses
 *   1 mean      sum / (number of valid rows, or the sum of their targets'
 *               class weights when `weight` is given: PyTorch's weighted mean)
 *   2 sum
 *   3 batchmean sum / rows
 * A row is valid when its target is not ignore_index and lies in [0, cols).
 *
 * Fused cross entropy over logits [rows, cols] (row stride ld) with int32
 * targets (F.cross_entropy, losses.ts:129-168): lse[r] = logsumexp(x[r]);
 * for a valid row with target t, eps = label_smoothing and w the optional
 * class weights [cols] (w = 1 when NULL),
 *   loss_rows[r] = (1-eps) w_t (lse - x[r,t]) + (eps/cols) sum_c w_c (lse - x[r,c])
 * (0 for invalid rows); `out` (1 float) receives the reduction. */
int tjh_cross_entropy_forward(const float* logits, int64_t ld,
                              const int32_t* targets, int64_t rows,
                              int64_t cols, int32_t ignore_index,
                              const float* weight, float label_smoothing,
                              float* lse, float* loss_rows, int reduction,
                              float* out);
/* dlogits[r,c] = s_r [((1-eps) w_t + (eps/cols) W) p_c - (1-eps) w_t [c == t]
 *                     - (eps/cols) w_c ],
 * p = exp(x - lse), W = sum_c w_c, s_r = grad_out[r] (none) or grad_out[0]
 * divided as the reduction divides (mean, batchmean) or not (sum); invalid
 * rows get 0.  Without weights and smoothing this is (softmax - onehot) * s_r.
 * dlogits row stride ldd; accumulate != 0 adds into dlogits. */
int tjh_cross_entropy_backward(const float* logits, int64_t ld,
                               const int32_t* targets, const float* weight,
                               float label_smoothing, const float* lse,
                               const float* grad_out, int64_t rows,
                               int64_t cols, int32_t ignore_index,
                               int reduction, float* dlogits, int64_t ldd,
                               int accumulate);
/* row_scale[r] = s_r for a valid row, 0 otherwise: the factor of row r
 * in tjh_cross_entropy_backward's gradient without weights and smoothing,
 * (softmax - onehot) * s_r.  For tjh_gemm_ce, which forms that gradient
 * while loading it instead of reading a stored dlogits. */
int tjh_cross_entropy_row_scale(const int32_t* targets,
                                const float* grad_out, int64_t rows,
                                int64_t cols, int32_t ignore_index,
                                int reduction, float* row_scale);
/* The forward of F.cross_entropy without class weights or smoothing
 * (losses.ts:129-168: lse, loss_rows, the scalar loss in `out` for
 * reduction 1 mean, 2 sum, 3 batchmean) together with the logits' gradient
 * of that loss for a unit upstream gradient — what loss.backward() seeds
 * (Tensor.ts:3686-3740) — written to dlogits [rows, ldd].  Equal bit for bit
 * to tjh_cross_entropy_forward followed by tjh_cross_entropy_backward with
 * grad_out = 1; rows of 2049 to 51200 classes, 16-byte aligned with ld and
 * ldd multiples of 4, are read once (the row kept in registers between the
 * two), others take those two calls. */
int tjh_cross_entropy_forward_grad(const float* logits, int64_t ld,
                                   const int32_t* targets, int64_t rows,
                                   int64_t cols, int32_t ignore_index,
                                   float* lse, float* loss_rows, int reduction,
                                   float* out, float* dlogits, int64_t ldd);
/* nll over log-probs [rows, cols] (F.nll_loss, losses.ts:63-94):
 * loss_rows[r] = -w_t logp[r, t] for valid rows, else 0. */
int tjh_nll_loss_forward(const float* logp, int64_t ld,
                         const int32_t* targets, int64_t rows, int64_t cols,
                         int32_t ignore_index, const float* weight,
                         float* loss_rows, int reduction, float* out);
/* dlogp = 0 except dlogp[r, t] = -w_t s_r (same scale rule as above). */
int tjh_nll_loss_backward(const int32_t* targets, const float* weight,
                          const float* grad_out, int64_t rows, int64_t cols,
                          int32_t ignore_index, int reduction, float* dlogp);

/* ------------------------------------------------------------------ */
/* LayerNorm — layernorm.wgsl:14-42, nn.LayerNorm                       */
/* (src/nn/layernorm.ts:25-119); backward is new (reference has none). */
/* ------------------------------------------------------------------ */

/* y = (x-mean)*rstd*gamma + beta over the last dim; rstd = 1/sqrt(biased
 * var + eps).  gamma/beta may be NULL (no affine).  mean/rstd [rows]
 * are saved for the backward. */
int tjh_layer_norm_forward(const float* x, const float* gamma,
                           const float* beta, float* y, float* mean,
                           float* rstd, int64_t rows, int64_t cols,
                           float eps);
/* dx (may be NULL), dgamma, dbeta (may be NULL).  accumulate != 0 adds
 * dgamma/dbeta into existing values. */
int tjh_layer_norm_backward(const float* dy, const float* x,
                            const float* gamma, const float* mean,
                            const float* rstd, float* dx, float* dgamma,
                            float* dbeta, int64_t rows, int64_t cols,
                            int accumulate);
/* tjh_layer_norm_backward with dx = res + the LayerNorm input gradient, in
 * one pass (res [rows, cols] or NULL; with res, dx is required and may not
 * overlap it).  The pre-LN residual stream x -> x + f(LayerNorm(x)) of
 * torch.js's transformer blocks gives x two gradient contributions that
 * its autograd sums with a separate add (accumulateGrad,
 * Tensor.ts:3670-3677); this entry folds that add into the LayerNorm
 * backward, equal bit for bit to tjh_layer_norm_backward followed by the
 * add.  flags: bit 0 (1) accumulates dgamma/dbeta as `accumulate` does;
 * TJH_LN_DEFER lets the library postpone the dgamma/dbeta finishing pass
 * to the next tjh_flush_deferred, which finishes every postponed
 * LayerNorm in one launch (dx is final on return; dgamma/dbeta are not
 * until the flush).  An autograd pass over a model with many LayerNorms
 * (25 in GPT-2 124M) defers them all and flushes once at its end. */
enum { TJH_LN_DEFER = 2 };
int tjh_layer_norm_backward_res(const float* dy, const float* x,
                                const float* gamma, const float* mean,
                                const float* rstd, const float* res,
                                float* dx, float* dgamma, float* dbeta,
                                int64_t rows, int64_t cols, int flags);
/* Runs the finishing passes postponed by TJH_LN_DEFER (none: no launch). */
int tjh_flush_deferred(void);
/* tjh_layer_norm_backward_res (flags = accumulate & 1, no deferral) that
 * allocates nothing.  No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving or training loops, harnesses that forbid hipMalloc).  The
 * dgamma / dbeta partial rows live in a static 6 MiB device array of the
 * library (2 x 256 rows of up to 3072 floats, enough for any row count on
 * a 256-CU MI355X) instead of the caching allocator; the kernels and the
 * results are those of tjh_layer_norm_backward_res, bit for bit.  Takes
 * cols a multiple of 4 up to 3072 with 16-byte aligned operands (else
 * TJH_ERR_UNSUPPORTED) and rejects a request whose partials would exceed
 * the array (TJH_ERR_INVALID).  Every call on a GPU shares that GPU's
 * array: calls run in order on the library stream, but a captured graph
 * replayed concurrently with another call on the same GPU races on it. */
int tjh_layer_norm_backward_noalloc(const float* dy, const float* x,
                                    const float* gamma, const float* mean,
                                    const float* rstd, const float* res,
                                    float* dx, float* dgamma, float* dbeta,
                                    int64_t rows, int64_t cols,
                                    int accumulate);

/* ------------------------------------------------------------------ */
/* Embedding / indexing — embedding.wgsl:13-27, index_select.wgsl,      */
/* Tensor.gather/argmax/nonzero, F.one_hot (src/nn/embedding.ts:25-101, */
/* Tensor.ts:1242-1345, 2651-2705, src/nn/functional.ts:764-796).       */
/* ------------------------------------------------------------------ */

/* out[i,:] = weight[clamp(ids[i], 0, num-1), :] (embedding.wgsl:24). */
int tjh_embedding_forward(const float* weight, int64_t num, int64_t dim,
                          const int32_t* ids, int64_t n, float* out);
/* dweight[v,:] (+)= sum over i with clamp(ids[i]) == v of dout[i,:], summed
 * in increasing i (deterministic). accumulate == 0 zero-fills dweight. */
int tjh_embedding_backward(const float* dout, const int32_t* ids,
                           int64_t n, int64_t dim, float* dweight,
                           int64_t num, int accumulate);
/* A token embedding plus a position embedding over [batch, T] ids, as a
 * transformer's input is built from two Embedding lookups and an add
 * (src/nn/embedding.ts:25-101 twice, then Tensor.add, Tensor.ts:3409-3466):
 * out[b,t,:] = weight[clamp(ids[b,t])] + pos_weight[pos0 + t], with
 * pos0 + T <= num_pos.  The sum is the same float add as the two lookups
 * followed by the add. */
int tjh_embedding_pos_forward(const float* weight, int64_t num, int64_t dim,
                              const int32_t* ids, int64_t batch, int64_t T,
                              const float* pos_weight, int64_t num_pos,
                              int64_t pos0, float* out);
/* Both tables' gradients of tjh_embedding_pos_forward in one launch: dweight
 * as tjh_embedding_backward over the batch * T ids, and dpos[pos0 + t,:]
 * (+)= dout[0,t,:] + dout[1,t,:] + ... in batch order (the embedding
 * backward's rule for ids pos0 + t repeated per batch item; rows outside
 * [pos0, pos0 + T) are zeroed unless acc_pos).  Either table may be NULL
 * (no gradient wanted). */
int tjh_embedding_pos_backward(const float* dout, const int32_t* ids,
                               int64_t batch, int64_t T, int64_t dim,
                               float* dweight, int64_t num, int accumulate,
                               float* dpos, int64_t num_pos, int64_t pos0,
                               int acc_pos);
/* x viewed [outer, src_len, inner]; out [outer, n_idx, inner] =
 * x[:, idx[j], :] (index_select.wgsl:20-55).  Valid indices are
 * 0 <= idx[j] < src_len, PyTorch's contract for index_select: the host
 * layer raises for any other value (the WGSL casts a negative i32 to u32
 * and reads out of bounds).  The kernel itself never reads outside x: an
 * out-of-range index yields a zero row here and contributes nothing in
 * tjh_index_add. */
int tjh_index_select(const float* x, int64_t outer, int64_t src_len,
                     int64_t inner, const int32_t* idx, int64_t n_idx,
                     float* out);
/* backward of index_select: dx[:, idx[j], :] += dout[:, j, :] (dx must be
 * zeroed by the caller); deterministic (sums in increasing j). */
int tjh_index_add(float* dx, int64_t outer, int64_t src_len, int64_t inner,
                  const int32_t* idx, int64_t n_idx, const float* dout);
/* gather along `dim` of a contiguous [outer, src_len, inner] source by an
 * index of shape [outer, idx_len, inner] (Tensor.ts:2651-2705); negative
 * indices wrap (Tensor.ts:2686-2687). */
int tjh_gather(const float* x, int64_t outer, int64_t src_len,
               int64_t inner, const int32_t* idx, int64_t idx_len,
               float* out);
/* scatter_add: dx[o, idx[o,j,i], i] += src[o,j,i] (deterministic). */
int tjh_scatter_add(float* dx, int64_t outer, int64_t dst_len,
                    int64_t inner, const int32_t* idx, int64_t idx_len,
                    const float* src);
/* one_hot: out[i, c] = (round(x[i]) == c) for 0 <= round(x[i]) < classes,
 * else the row stays zero (src/nn/functional.ts:786-791).  x is float
 * (torch.js passes values as f32). */
int tjh_one_hot(const float* x, int64_t n, int64_t classes, float* out);
int tjh_one_hot_i32(const int32_t* x, int64_t n, int64_t classes,
                    float* out);
/* nonzero in row-major order (Tensor.ts:1323-1345): *count receives nnz
 * (blocking), out [nnz, ndim] int32 must hold max_out rows. */
int tjh_nonzero(const float* x, int ndim, const int64_t* shape,
                int32_t* out, int64_t max_out, int64_t* count);

/* Tensor.multinomial (src/tensor/Tensor.ts:271-359) on the device: out
 * [rows, num_samples] int32 category indices drawn from each row of probs
 * [rows, cols] (contiguous).  Row weights are max(0, x) (negatives and
 * -inf weigh 0), normalised by their sum; a row summing to <= 0 samples
 * uniformly.  With replacement, a draw u picks the first index whose
 * running sum of the normalised weights exceeds u; without it, each draw
 * renormalises over the indices not yet taken (num_samples <= cols,
 * cols <= 2^18), and once the positive-weight categories are used up each
 * draw takes the last untaken index.  Draw s of row r uses the uniform of
 * element r * num_samples + s of tjh_random with the same seed, so callers
 * can replay every draw.  A row holding NaN or +inf is an error
 * (TJH_ERR_INVALID, as PyTorch raises; the reference's result is undefined
 * there): its draws are written as -1.  The call reads a status word per
 * row back, so it synchronises the stream and is refused during capture. */
int tjh_multinomial(const float* probs, int64_t rows, int64_t cols,
                    int64_t num_samples, int replacement, uint32_t seed,
                    int32_t* out);

/* ------------------------------------------------------------------ */
/* Dense contractions — matmul.wgsl:17-50 / Tensor.matmul, bmm, Linear  */
/* (Tensor.ts:2132-2331, src/nn/linear.ts:43-66): fp32 MFMA GEMM.       */
/* ------------------------------------------------------------------ */

/* C[b] = alpha * op(A[b]) . op(B[b]) + beta * C[b] (+ bias), row-major;
 * op(X) = X^T when trans != 0.  A is [M,K] (or [K,M] when transA), B is
 * [K,N] (or [N,K] when transB); lda/ldb/ldc are row strides; strides
 * between batch items may be 0 (broadcast).  bias_mode: 0 none, 1 bias[N]
 * added to every row, 2 bias[M] added to every column, 3 bias[M] is an
 * OUTPUT: bias[m] = sum_k op(A)[m][k] (batch 1; the bias gradient of a
 * Linear layer computed with its weight gradient, which replaces the
 * separate column sum of dY).  beta == 0 never reads C. */
int tjh_gemm(int transA, int transB, int64_t M, int64_t N, int64_t K,
             float alpha, const float* A, int64_t lda, int64_t strideA,
             const float* B, int64_t ldb, int64_t strideB, float beta,
             float* C, int64_t ldc, int64_t strideC, int64_t batch,
             const float* bias, int bias_mode);
/* tjh_gemm (batch 1) with the elementwise op that follows a Linear layer in
 * torch.js's transformer fused into the epilogue: the GELU of the
 * Linear -> GELU -> Linear MLP (src/nn/activation.ts GELU between
 * src/nn/linear.ts layers), which otherwise runs as separate elementwise
 * passes over the [tokens, 4*d] activation (unary.wgsl:246-252 and its
 * backward), and the residual add x + Linear(...) of the pre-LN block
 * (elementwise.wgsl add).  With v the final value of C[m][n] (alpha, beta
 * and bias applied):
 *   act 1: aux[m*ldaux + n] = v, C = GELU(v)       (forward: keeps the
 *          pre-activation for the backward)
 *   act 2: C = v * GELU'(aux[m*ldaux + n])          (backward through GELU)
 *   act 3: C = aux[m*ldaux + n] + v                 (residual add; aux is
 *          only read and may not overlap C)
 * act 0 is tjh_gemm.  GELU, GELU' and the add are the library's
 * elementwise ones, so the results equal the unfused sequence bit for bit. */
int tjh_gemm_act(int transA, int transB, int64_t M, int64_t N, int64_t K,
                 float alpha, const float* A, int64_t lda, const float* B,
                 int64_t ldb, float beta, float* C, int64_t ldc,
                 const float* bias, int bias_mode, float* aux, int64_t ldaux,
                 int act);
/* The products of torch.js's LM head backward (Linear.backward of
 * src/nn/linear.ts:43-66 fed by cross_entropy's gradient, losses.ts:129-168)
 * without the stored cross-entropy gradient: C[M,N] = op(D) B[K,N] (row
 * stride ldb, not transposed), where D[r][c] = (exp(logits[r][c] - lse[r])
 * - [c == targets[r]]) * row_scale[r] is tjh_cross_entropy_backward's
 * dlogits (no weights, no smoothing) formed while the A tiles are loaded.
 * transA 0: D is [M rows, K classes] (dx = dlogits W); transA 1: op(D) =
 * D^T with D [K rows, M classes] (dW = dlogits^T x).  Logits row stride
 * ld; row_scale from tjh_cross_entropy_row_scale.  Equal bit for bit to
 * tjh_cross_entropy_backward followed by tjh_gemm. */
int tjh_gemm_ce(int transA, int64_t M, int64_t N, int64_t K,
                const float* logits, int64_t ld, const float* lse,
                const int32_t* targets, const float* row_scale,
                const float* B, int64_t ldb, float* C, int64_t ldc);

/* ------------------------------------------------------------------ */
/* Attention — F.scaled_dot_product_attention                           */
/* (src/nn/functional.ts:866-890), MultiheadAttention                   */
/* (src/nn/attention.ts:112-271).  Flash-style: O(T) extra memory.      */
/* ------------------------------------------------------------------ */

/* q [B,H,Tq,D], k/v [B,H,Tk,D] given by strides (elements) for the B, H
 * and T axes; D is contiguous.  o written with its own strides.  lse
 * [B,H,Tq] (contiguous) saved for the backward.  causal masks key j >
 * query i (top-left aligned, as torch's is_causal).  Head dims D <= 128
 * with D % 4 == 0 and 16-byte aligned rows run the flash kernels (O(T)
 * extra memory); any other D runs GEMM-composed attention over [H,Tq,Tk]
 * scores of one batch item at a time. */
int tjh_sdpa_forward(const float* q, const float* k, const float* v,
                     float* o, float* lse, int64_t B, int64_t H, int64_t Tq,
                     int64_t Tk, int64_t D, const int64_t* q_strides,
                     const int64_t* k_strides, const int64_t* v_strides,
                     const int64_t* o_strides, float scale, int causal);
/* dq/dk/dv written (not accumulated).  Every tensor has its own strides
 * for the B, H, T axes (D contiguous): strides[0..4] = q, k, v, o, do_;
 * strides[5..7] = dq, dk, dv; each entry points at 3 int64. */
int tjh_sdpa_backward(const float* q, const float* k, const float* v,
                      const float* o, const float* do_, const float* lse,
                      float* dq, float* dk, float* dv, int64_t B, int64_t H,
                      int64_t Tq, int64_t Tk, int64_t D,
                      const int64_t* const* strides, float scale, int causal);

/* ------------------------------------------------------------------ */
/* Convolution — conv.wgsl:25-60, conv_backward.wgsl:24-119, F.conv2d   */
/* (src/nn/functional.ts:438-660): NCHW, implicit GEMM on MFMA.         */
/* ------------------------------------------------------------------ */

typedef struct {
  int64_t n, c, h, w;        /* input                                    */
  int64_t oc, kh, kw;        /* weight [oc, c/groups, kh, kw]            */
  int64_t stride_h, stride_w, pad_h, pad_w, dil_h, dil_w, groups;
  int64_t oh, ow;            /* output spatial size (filled by caller)   */
} tjh_conv2d_desc;

int tjh_conv2d_forward(const tjh_conv2d_desc* d, const float* x,
                       const float* w, const float* bias, float* y);
/* tjh_conv2d_forward with the activation that follows the convolution in
 * torch.js's CNNs (conv2d then relu, src/nn/conv.ts + F.relu's
 * unary.wgsl) applied as the output is written: act 0 none, 1 ReLU (the
 * library's own, so the result equals tjh_conv2d_forward then tjh_unary
 * RELU bit for bit; ReLU's gradient can be taken from this output). */
int tjh_conv2d_forward_act(const tjh_conv2d_desc* d, const float* x,
                           const float* w, const float* bias, float* y,
                           int act);
/* dx = conv_transpose(dy, w) (written, not accumulated). */
int tjh_conv2d_backward_input(const tjh_conv2d_desc* d, const float* dy,
                              const float* w, float* dx);
/* dw (+)= correlation of x and dy; accumulate != 0 adds. */
int tjh_conv2d_backward_weight(const tjh_conv2d_desc* d, const float* dy,
                               const float* x, float* dw, int accumulate);
/* The same, plus the bias gradient db[oc] (+)= sum over images and output
 * pixels of dy (the bias grad of F.conv2d, functional.ts:438-660) when db
 * is not NULL, taken from the dy tiles the weight-gradient product stages
 * (no second pass over dy).  With db NULL it is tjh_conv2d_backward_weight. */
int tjh_conv2d_backward_weight_bias(const tjh_conv2d_desc* d, const float* dy,
                                    const float* x, float* dw, float* db,
                                    int accumulate);

/* ------------------------------------------------------------------ */
/* Optimizers — Adam.step / AdamW.step (src/optim/adam.ts:46-133,       */
/* src/optim/adamw.ts:46-154) as ONE fused multi-tensor launch.         */
/* ------------------------------------------------------------------ */

/* For each tensor t (host arrays of n_tensors device pointers):
 *   Adam  (decoupled == 0): g' = g + f32(wd)*p           (adam.ts:62-63)
 *   AdamW (decoupled != 0): g' = g
 *   m = f32(b1)*m + f32(1-b1)*g'                         (adam.ts:82)
 *   v = f32(b2)*v + f32(1-b2)*(g'*g')                    (adam.ts:85)
 *   denom = sqrt(v / f32(bc2)) + f32(eps), bc_i = 1 - b_i^step[t]
 *                                                         (adam.ts:96)
 *   AdamW: p = p*(1 - lr*wd)                             (adamw.ts:129)
 *   p = p - (lr/bc1) * m / denom                         (adam.ts:114)
 * m, v and denom are rounded to fp32 after every operation (the reference
 * computes them as separate fp32 tensor ops); the parameter update is
 * evaluated in double and rounded once, as the reference's JS loop does
 * (adam.ts:104-120, adamw.ts:114-133).  The hyper-parameters are doubles
 * (JS numbers). */
int tjh_adam_step(int n_tensors, float* const* params,
                  const float* const* grads, float* const* exp_avg,
                  float* const* exp_avg_sq, const int64_t* numels,
                  const int64_t* steps, double lr, double beta1,
                  double beta2, double eps, double weight_decay,
                  int decoupled);
/* The same step with each tensor's step count in device memory
 * (steps[i] -> int64 counter): the call advances every counter by one and
 * takes the bias corrections of the new count from a table the host fills
 * with the same pow as tjh_adam_step (bit-identical results), so the step
 * can be captured in a graph and replayed.  The table for (lr, beta1,
 * beta2) is made on the first call, which must not be inside a capture. */
int tjh_adam_step_dev(int n_tensors, float* const* params,
                      const float* const* grads, float* const* exp_avg,
                      float* const* exp_avg_sq, const int64_t* numels,
                      int64_t* const* steps, double lr, double beta1,
                      double beta2, double eps, double weight_decay,
                      int decoupled);

#ifdef __cplusplus
}
#endif
#endif /* TORCHJS_HIP_H */
