// Fused elementwise expressions.
//
// torch.js runs every elementwise op as its own submit that reads its
// inputs from and writes its output to memory (Tensor.ts _unaryOp,
// _binaryOp, _broadcastBinaryOp, _scalarOp: 3409-3656, 3742-3792), and
// its broadcast-gradient column sum is one more pass
// (Tensor.ts:3560-3591).  The host layer here defers chains of those ops
// and hands the chain to one of two entry points as a small program
// (tjh_expr, include/torchjs_hip.h):
//   * tjh_expr_eval writes the chain's value;
//   * tjh_expr_colsum sums the value over the middle axis of an
//     [outer, r, inner] view (a bias gradient, `sum(0)`), optionally
//     writing the value in the same pass.
// So a chain costs one read of its leaves (and one write of what is kept)
// instead of a write and a read of every intermediate.
//
// Each distinct program shape (instructions, op codes, leaf kinds, vector
// width, entry point) becomes one kernel, generated as HIP source in
// static single assignment form over the device prelude expr_jit.h,
// compiled for the device with hipRTC on first use and cached for the
// life of the process (about a quarter of a second per shape).  Leaf
// pointers, periods and scalar constants are kernel arguments, so new
// data never recompiles.  An interpreter was measured against this: a
// uniform program over a register file indexed at run time puts the file
// in scratch memory (LLVM folds a switch over registers back into an
// indexed array), or costs a select chain per operand.
//
// Every instruction is the ABI's scalar op (ew_ops.h) behind a
// contraction barrier, so a fused value is bit-identical to the op-by-op
// one.  A lane evaluates W = 4 adjacent elements (128-bit leaf loads and
// stores) when every leaf allows it, else 1.  The column sum keeps the row
// partition and the compensated per-column order of the unfused column
// sum (colsum_plan, k_colsum, colsum_final), so its result is
// bit-identical to summing the materialised value.

#include "colsum.h"
#include "common.h"
#include "expr_jit.h"

#include <dlfcn.h>
#include <hip/hiprtc.h>

#include <mutex>
#include <string>
#include <unordered_map>

namespace tjh {
namespace {

constexpr int kBlock = jit::kBlock;
constexpr int NL = TJH_EXPR_MAX_LEAVES;
constexpr int NR = TJH_EXPR_MAX_REGS;

// Checks the program and returns W (4 when every leaf and `extra` allow
// 128-bit access at multiples of 4 elements, else 1), or 0 on error.
int check_prog(const tjh_expr* P, int64_t n, const float* const* extra, int nextra) {
  if (!P) return set_error(TJH_ERR_INVALID, "tjh_expr: NULL program"), 0;
  if (P->n_ins < 1 || P->n_ins > TJH_EXPR_MAX_INS)
    return set_error(TJH_ERR_INVALID, "tjh_expr: %d instructions", P->n_ins), 0;
  if (P->n_leaves < 0 || P->n_leaves > NL)
    return set_error(TJH_ERR_INVALID, "tjh_expr: %d leaves", P->n_leaves), 0;
  if (P->result < 0 || P->result >= NR)
    return set_error(TJH_ERR_INVALID, "tjh_expr: result register %d", P->result), 0;
  if (P->result2 < 0 || P->result2 > NR)
    return set_error(TJH_ERR_INVALID, "tjh_expr: second result %d", P->result2), 0;
  if (P->result3 < 0 || P->result3 > NR)
    return set_error(TJH_ERR_INVALID, "tjh_expr: third result %d", P->result3), 0;
  bool vec = n % 4 == 0;
  for (int k = 0; k < P->n_leaves; ++k) {
    const int kind = P->kind[k];
    if (!P->leaf[k] || kind < TJH_LEAF_CONTIG || kind > TJH_LEAF_SCALAR)
      return set_error(TJH_ERR_INVALID, "tjh_expr: bad leaf %d", k), 0;
    if ((kind == TJH_LEAF_ROW || kind == TJH_LEAF_COL) && P->period[k] < 1)
      return set_error(TJH_ERR_INVALID, "tjh_expr: leaf %d period %lld", k,
                       (long long)P->period[k]), 0;
    if (kind == TJH_LEAF_CONTIG || kind == TJH_LEAF_ROW) vec = vec && aligned16(P->leaf[k]);
    if (kind == TJH_LEAF_ROW || kind == TJH_LEAF_COL) vec = vec && P->period[k] % 4 == 0;
  }
  unsigned defined = 0;  // registers written so far
  auto def = [&](int reg) { return reg < NR && ((defined >> reg) & 1u); };
  for (int i = 0; i < P->n_ins; ++i) {
    const tjh_expr_ins& in = P->ins[i];
    const bool reg_a = in.op != TJH_EXPR_LOAD && in.op != TJH_EXPR_CONST;
    bool ok = in.op < TJH_EXPR_OPS && in.dst < NR;
    if (in.op == TJH_EXPR_LOAD) ok = ok && in.a < P->n_leaves;
    if (reg_a) ok = ok && def(in.a);
    if (in.op == TJH_EXPR_BINARY || in.op == TJH_EXPR_AXPY) ok = ok && def(in.b);
    if (in.op == TJH_EXPR_TERNARY) ok = ok && def(in.b) && def(in.c);
    if (in.op == TJH_EXPR_UNARY_BWD)
      ok = ok && (in.b == TJH_EXPR_NONE || def(in.b)) && (in.c == TJH_EXPR_NONE || def(in.c));
    switch (in.op) {
      case TJH_EXPR_UNARY: ok = ok && in.code < TJH_UNARY_COUNT; break;
      case TJH_EXPR_UNARY_BWD: ok = ok && in.code < TJH_UNARY_COUNT; break;
      case TJH_EXPR_BINARY: ok = ok && in.code < TJH_BINARY_COUNT; break;
      case TJH_EXPR_TERNARY: ok = ok && in.code < TJH_TERNARY_COUNT; break;
      case TJH_EXPR_SCALAR:
      case TJH_EXPR_SCALAR_REV: ok = ok && in.code < TJH_SCALAR_COUNT; break;
      default: break;
    }
    if (!ok) return set_error(TJH_ERR_INVALID, "tjh_expr: bad instruction %d", i), 0;
    defined |= 1u << in.dst;
  }
  if (!def(P->result)) return set_error(TJH_ERR_INVALID, "tjh_expr: result never written"), 0;
  if (P->result2 && !def(P->result2 - 1))
    return set_error(TJH_ERR_INVALID, "tjh_expr: second result never written"), 0;
  if (P->result3 && !def(P->result3 - 1))
    return set_error(TJH_ERR_INVALID, "tjh_expr: third result never written"), 0;
  for (int i = 0; i < nextra; ++i) vec = vec && (!extra[i] || aligned16(extra[i]));
  return vec ? 4 : 1;
}

int grid_for(int64_t items) {
  int64_t g = cdiv(items, kBlock);
  const int64_t cap = (int64_t)(num_cus() > 0 ? num_cus() : 256) * 32;
  if (g > cap) g = cap;
  return (int)(g < 1 ? 1 : g);
}

// ------------------------------------------------------------ codegen

enum Mode { kEval = 0, kColsum = 1, kColsum3 = 2 };

// HIP source of the kernel for program P at width W.
std::string generate(const tjh_expr* P, int W, Mode mode) {
  std::string s;
  char buf[256];
  s += "#include \"expr_jit.h\"\nusing namespace tjh::jit;\nnamespace {\nstruct F {\n";
  if (mode == kColsum3)
    snprintf(buf, sizeof buf,
             "  __device__ __forceinline__ V<%d> operator()(const Args& a, long long e, V<%d>* c3) "
             "const {\n", W, W);
  else
    snprintf(buf, sizeof buf,
             "  __device__ __forceinline__ V<%d> operator()(const Args& a, long long e) const {\n",
             W);
  s += buf;
  for (int k = 0; k < P->n_leaves; ++k) {
    snprintf(buf, sizeof buf, "    const V<%d> l%d = leaf<%d, %d>(a, %d, e);\n", W, k, W, P->kind[k], k);
    s += buf;
  }
  std::string reg[NR];
  for (int i = 0; i < P->n_ins; ++i) {
    const tjh_expr_ins& in = P->ins[i];
    auto R = [&](int r) { return r < NR ? reg[r] : std::string(); };
    auto opt = [&](int r) {
      return r < NR ? reg[r] : "splat<" + std::to_string(W) + ">(0.f)";
    };
    std::string rhs;
    const std::string w = std::to_string(W), code = std::to_string(in.code),
                      f = "a.f[" + std::to_string(i) + "]";
    switch (in.op) {
      case TJH_EXPR_LOAD: rhs = "l" + std::to_string(in.a); break;
      case TJH_EXPR_CONST: rhs = "splat<" + w + ">(" + f + ")"; break;
      case TJH_EXPR_UNARY: rhs = "vunary<" + w + ", " + code + ">(" + R(in.a) + ", " + f + ")"; break;
      case TJH_EXPR_UNARY_BWD:
        rhs = "vunary_bwd<" + w + ", " + code + ">(" + R(in.a) + ", " + opt(in.b) + ", " +
              opt(in.c) + ", " + f + ")";
        break;
      case TJH_EXPR_BINARY:
        rhs = "vbinary<" + w + ", " + code + ">(" + R(in.a) + ", " + R(in.b) + ")";
        break;
      case TJH_EXPR_TERNARY:
        rhs = "vternary<" + w + ", " + code + ">(" + R(in.a) + ", " + R(in.b) + ", " + R(in.c) + ")";
        break;
      case TJH_EXPR_SCALAR:
      case TJH_EXPR_SCALAR_REV:
        rhs = "vscalar<" + w + ", " + code + ", " + (in.op == TJH_EXPR_SCALAR_REV ? "true" : "false") +
              ">(" + R(in.a) + ", " + f + ")";
        break;
      default: rhs = "vaxpy<" + w + ">(" + f + ", " + R(in.a) + ", " + R(in.b) + ")"; break;
    }
    const std::string t = "t" + std::to_string(i);
    s += "    const V<" + w + "> " + t + " = " + rhs + ";\n";
    reg[in.dst] = t;
  }
  if (P->result2)
    s += "    if (a.values2) store<" + std::to_string(W) + ">(a.values2 + e, " + reg[P->result2 - 1] +
         ");\n";
  if (mode == kColsum3) s += "    *c3 = " + reg[P->result3 - 1] + ";\n";
  s += "    return " + reg[P->result] + ";\n  }\n};\n}  // namespace\n";
  snprintf(buf, sizeof buf,
           "extern \"C\" __global__ __launch_bounds__(%d) void tjh_expr_kernel(Args a) {\n"
           "  %s<%d>(F(), a);\n}\n",
           kBlock, mode == kEval ? "eval_body" : (mode == kColsum ? "colsum_body" : "colsum3_body"),
           W);
  s += buf;
  return s;
}

// Directory holding this library (csrc/ and ../include/ are beside it).
std::string library_dir() {
  Dl_info info;
  if (dladdr(reinterpret_cast<void*>(&library_dir), &info) == 0 || !info.dli_fname) return ".";
  std::string p = info.dli_fname;
  const size_t slash = p.rfind('/');
  return slash == std::string::npos ? std::string(".") : p.substr(0, slash);
}

struct Compiled {
  hipModule_t mod;
  hipFunction_t fn;
};

std::mutex g_jit_mu;
std::unordered_map<std::string, Compiled>& jit_cache() {
  static std::unordered_map<std::string, Compiled> c;
  return c;
}

// Code object of `src` for gfx950 (hipRTC only: no device needed).
int compile_code(const std::string& src, std::string* code_out) {
  const std::string dir = library_dir();
  const std::string inc1 = "-I" + dir + "/csrc", inc2 = "-I" + dir + "/../include";
  const char* opts[] = {"--offload-arch=gfx950", "-O3", "-std=c++17", inc1.c_str(), inc2.c_str(),
                        // packed fp32 ops stay disabled, as for every other kernel
                        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};
  hiprtcProgram prog;
  if (hiprtcCreateProgram(&prog, src.c_str(), "tjh_expr.hip", 0, nullptr, nullptr) != HIPRTC_SUCCESS)
    return set_error(TJH_ERR_HIP, "tjh_expr: hiprtcCreateProgram failed");
  const hiprtcResult rc = hiprtcCompileProgram(prog, (int)(sizeof(opts) / sizeof(opts[0])), opts);
  if (rc != HIPRTC_SUCCESS) {
    size_t n = 0;
    hiprtcGetProgramLogSize(prog, &n);
    std::string log(n, '\0');
    if (n) hiprtcGetProgramLog(prog, &log[0]);
    hiprtcDestroyProgram(&prog);
    return set_error(TJH_ERR_HIP, "tjh_expr: compile failed (%s): %.600s", hiprtcGetErrorString(rc),
                     log.c_str());
  }
  size_t size = 0;
  hiprtcGetCodeSize(prog, &size);
  code_out->assign(size, '\0');
  hiprtcGetCode(prog, &(*code_out)[0]);
  hiprtcDestroyProgram(&prog);
  return TJH_OK;
}

// Compact key of everything the generated source depends on: device,
// width, entry point, instructions (not their constants) and leaf kinds.
std::string signature(const tjh_expr* P, int W, Mode mode) {
  std::string k;
  k.reserve(16 + 6 * P->n_ins + P->n_leaves);
  k.push_back((char)device_ordinal());
  k.push_back((char)W);
  k.push_back((char)mode);
  k.push_back((char)P->n_ins);
  k.push_back((char)P->n_leaves);
  k.push_back((char)P->result);
  k.push_back((char)P->result2);
  k.push_back((char)P->result3);
  for (int i = 0; i < P->n_ins; ++i) {
    const tjh_expr_ins& in = P->ins[i];
    const char b[6] = {(char)in.op, (char)in.code, (char)in.dst, (char)in.a, (char)in.b, (char)in.c};
    k.append(b, 6);
  }
  for (int j = 0; j < P->n_leaves; ++j) k.push_back((char)P->kind[j]);
  return k;
}

// The kernel of program P on the current device, compiled on first use.
int get_kernel(const tjh_expr* P, int W, Mode mode, hipFunction_t* fn) {
  const std::string key = signature(P, W, mode);
  std::lock_guard<std::mutex> lock(g_jit_mu);
  auto it = jit_cache().find(key);
  if (it != jit_cache().end()) {
    *fn = it->second.fn;
    return TJH_OK;
  }
  const std::string src = generate(P, W, mode);
  std::string code;
  const int rc = compile_code(src, &code);
  if (rc != TJH_OK) return rc;
  Compiled c;
  hipError_t e = hipModuleLoadData(&c.mod, code.data());
  if (e != hipSuccess) return hip_fail(e, "tjh_expr: hipModuleLoadData");
  e = hipModuleGetFunction(&c.fn, c.mod, "tjh_expr_kernel");
  if (e != hipSuccess) return hip_fail(e, "tjh_expr: hipModuleGetFunction");
  jit_cache()[key] = c;
  *fn = c.fn;
  return TJH_OK;
}

jit::Args make_args(const tjh_expr* P) {
  jit::Args a{};
  for (int k = 0; k < P->n_leaves; ++k) {
    a.leaf[k] = P->leaf[k];
    a.period[k] = P->period[k];
  }
  for (int i = 0; i < P->n_ins; ++i) a.f[i] = P->ins[i].f;
  return a;
}

int launch(hipFunction_t fn, dim3 grid, jit::Args& a, const char* what) {
  void* params[] = {&a};
  hipEvent_t e0 = nullptr, e1 = nullptr;
  const bool timed = launch_events(&e0, &e1);
  const hipError_t err = hipExtModuleLaunchKernel(
      fn, grid.x * kBlock, grid.y, grid.z, kBlock, 1, 1, 0, stream(), params, nullptr,
      timed ? e0 : nullptr, timed ? e1 : nullptr, 0);
  if (err != hipSuccess) return set_error(TJH_ERR_HIP, "%s: %s", what, hipGetErrorString(err));
  return check_launch(what);
}

}  // namespace
}  // namespace tjh

using namespace tjh;

extern "C" {

int tjh_expr_eval(const tjh_expr* prog, int64_t n, float* out) {
  TJH_REQUIRE_INIT();
  TJH_ARG(n >= 0, "tjh_expr_eval: negative size");
  const float* ex[1] = {out};
  const int W = check_prog(prog, n, ex, 1);
  if (W == 0) return TJH_ERR_INVALID;
  if (n == 0) return TJH_OK;
  TJH_ARG(out != nullptr, "tjh_expr_eval: NULL output");
  hipFunction_t fn;
  int rc = get_kernel(prog, W, kEval, &fn);
  if (rc != TJH_OK) return rc;
  KernelScope ks("expr");
  jit::Args a = make_args(prog);
  a.out = out;
  a.n = n;
  return launch(fn, dim3(grid_for(cdiv(n / W, 4))), a, "expr_eval");
}

int tjh_expr_compile(const tjh_expr* prog, int64_t n, int colsum) {
  TJH_ARG(n >= 0, "tjh_expr_compile: negative size");
  const int W = check_prog(prog, n, nullptr, 0);
  if (W == 0) return TJH_ERR_INVALID;
  std::string code;
  const Mode m = !colsum ? kEval : (prog->result3 ? kColsum3 : kColsum);
  return compile_code(generate(prog, W, m), &code);
}

int tjh_expr_colsum(const tjh_expr* prog, int64_t outer, int64_t r, int64_t inner, float* out,
                    float* values) {
  return tjh_expr_colsum2(prog, outer, r, inner, out, values, nullptr);
}

int tjh_expr_colsum2(const tjh_expr* prog, int64_t outer, int64_t r, int64_t inner, float* out,
                     float* values, float* values2) {
  return tjh_expr_colsum3(prog, outer, r, inner, out, values, values2, nullptr);
}

int tjh_expr_colsum3(const tjh_expr* prog, int64_t outer, int64_t r, int64_t inner, float* out,
                     float* values, float* values2, float* out3) {
  TJH_REQUIRE_INIT();
  TJH_ARG(outer >= 0 && r >= 0 && inner >= 0, "tjh_expr_colsum: negative size");
  if (outer > kFinalMax || r < 64 || inner < 2)
    return set_error(TJH_ERR_UNSUPPORTED,
                     "tjh_expr_colsum: outer %lld <= %d, r %lld >= 64 and inner %lld >= 2 needed",
                     (long long)outer, kFinalMax, (long long)r, (long long)inner);
  const bool third = prog && prog->result3 && out3;
  if (third && 2 * outer > kFinalMax)
    return set_error(TJH_ERR_UNSUPPORTED, "tjh_expr_colsum3: 2 * outer %lld > %d",
                     (long long)(2 * outer), kFinalMax);
  const float* ex[2] = {values, values2};
  int W = check_prog(prog, outer * r * inner, ex, 2);
  if (W == 0) return TJH_ERR_INVALID;
  if (outer == 0) return TJH_OK;
  TJH_ARG(out != nullptr, "tjh_expr_colsum: NULL output");
  if (inner % 4) W = 1;
  hipFunction_t fn;
  int rc = get_kernel(prog, W, third ? kColsum3 : kColsum, &fn);
  if (rc != TJH_OK) return rc;
  KernelScope ks(third ? "expr_colsum3" : "expr_colsum");
  // the partition of the unfused sum of the materialised (aligned) value
  int64_t nb = 0, rchunk = 0;
  colsum_plan(outer, r, inner, inner % 4 == 0, &nb, &rchunk);
  const int64_t per = outer * nb * inner;  // partial rows of one column sum
  Scratch part((size_t)(third ? 2 * per : per) * sizeof(float));
  if (!part.ok()) return set_error(TJH_ERR_OOM, "tjh_expr_colsum: no scratch memory");
  jit::Args a = make_args(prog);
  a.out = part.as<float>();
  a.out3 = third ? part.as<float>() + per : nullptr;
  a.values = values;
  a.values2 = prog->result2 ? values2 : nullptr;
  a.r = r;
  a.inner = inner;
  a.rchunk = rchunk;
  const int64_t col_groups = cdiv(cdiv(inner, W), kBlock);
  rc = launch(fn, dim3((unsigned)nb, (unsigned)col_groups, (unsigned)outer), a, "expr_colsum");
  if (rc != TJH_OK) return rc;
  float* parts[kFinalMax];
  float* outs[kFinalMax];
  for (int64_t i = 0; i < outer; ++i) {
    parts[i] = part.as<float>() + i * nb * inner;
    outs[i] = out + i * inner;
    if (third) {  // the third value's sums finish in the same launch
      parts[outer + i] = a.out3 + i * nb * inner;
      outs[outer + i] = out3 + i * inner;
    }
  }
  return colsum_final(parts, outs, (int)(third ? 2 * outer : outer), nb, inner, 0, 1.0f);
}

}  // extern "C"
