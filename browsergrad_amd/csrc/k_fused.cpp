// Fused elementwise (+ optional last-axis reduction) for gfx950, generated
// per program at run time with hipRTC.
//
// The reference generates one WGSL compute shader per fused op list and
// caches the pipeline by an FNV-1a hash of the list
// (packages/browsergrad-kernels/src/kernels/fused_elementwise.ts:56-69,
// 93-179).  This is the MI355X counterpart: the op list (plus the input
// dtypes, their broadcast pattern, the output dtype and the reduction) is
// turned into a straight-line HIP kernel, compiled once for gfx950 with
// hipRTC, and cached in-process and on disk by a 64-bit FNV-1a hash of the
// generated source.  Straight-line code keeps every value in VGPRs; an
// interpreter with runtime-indexed registers would spill them to scratch.
//
// Generated kernel shapes
//   map:    grid-stride loop; each lane handles VEC (4 when aligned)
//           consecutive elements of one row with 16-byte loads; every
//           streaming input is loaded before the op chain runs.
//   reduce: TPR lanes (64: one wavefront per row, 256: one workgroup per
//           row) walk a row, reduce the chain's value in registers, then
//           across lanes (DPP shuffles) and LDS; one store per row.  The C2
//           "relu(a*b+c)*exp(-a*a) -> row sum" graph is one such launch.
// Numerics: every op runs in f32 and is rounded per op (-ffp-contract=off,
// so a*b+c never becomes an FMA), matching NumPy's per-ufunc rounding; f16 /
// bf16 rounding ops are explicit round-to-nearest-even conversions.
#include <hip/hip_ext.h>
#include <hip/hiprtc.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <mutex>
#include <sstream>
#include <sys/stat.h>
#include <unistd.h>
#include <unordered_map>

#include "core.h"

namespace {

constexpr int kMaxDims = 4;
enum : int32_t { IN_CONTIG = 0, IN_SCALAR = 1, IN_STRIDED = 2 };

// Runtime arguments of every generated kernel (layout shared with the
// generated source's `Args`).
struct FusedArgs {
  const void* in[BG_FUSED_MAX_INPUTS];
  int64_t stride[BG_FUSED_MAX_INPUTS][kMaxDims];
  uint32_t dims[kMaxDims];
  int64_t rows;
  int64_t cols;
  float imm[BG_FUSED_MAX_IMMS];
  void* out;
  // Split reductions: each row is cut into `nch` chunks of `cw` columns whose
  // partial results go to `part[row * nch + chunk]`.
  int64_t cw;
  int64_t nch;
  float* part;
  // Division by runtime constants (Granlund-Montgomery round-up method):
  // divisor, multiplier, shift of the vectors per row (map kernels) and of
  // each leading dim (strided inputs).
  uint32_t vc_d, vc_m, vc_s;
  uint32_t dim_d[kMaxDims], dim_m[kMaxDims], dim_s[kMaxDims];
};

const char* kPrelude = R"(
typedef long long i64;
typedef unsigned int u32;
typedef unsigned short u16;
struct Args {
  const void* in[8];
  i64 stride[8][4];
  u32 dims[4];
  i64 rows;
  i64 cols;
  float imm[16];
  void* out;
  i64 cw;
  i64 nch;
  float* part;
  u32 vc_d, vc_m, vc_s;
  u32 dim_d[4], dim_m[4], dim_s[4];
};
typedef float f4v_ __attribute__((ext_vector_type(4)));
typedef u32 u2v_ __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float bg_h2f(u16 v) { return (float)__builtin_bit_cast(_Float16, v); }
__device__ __forceinline__ u16 bg_f2h(float f) { return __builtin_bit_cast(u16, (_Float16)f); }
__device__ __forceinline__ float bg_b2f(u16 v) { return __builtin_bit_cast(float, ((u32)v) << 16); }
__device__ __forceinline__ u16 bg_f2b(float f) { return __builtin_bit_cast(u16, (__bf16)f); }
__device__ __forceinline__ float bg_rh(float x) { return (float)(_Float16)x; }
__device__ __forceinline__ float bg_rb(float x) { return (float)(__bf16)x; }
__device__ __forceinline__ float bg_max(float a, float b) { return (a != a || b != b) ? a + b : fmaxf(a, b); }
__device__ __forceinline__ u32 bg_fdiv(u32 n, u32 d, u32 m, u32 s) {
  if (d == 1u) return n;
  const u32 t = (u32)(((unsigned long long)n * m) >> 32);
  return (t + ((n - t) >> 1)) >> (s - 1u);
}
__device__ __forceinline__ float bg_min(float a, float b) { return (a != a || b != b) ? a + b : fminf(a, b); }
)";

std::string fmt_f(float v) {
  // Exact hex literal for a float immediate.
  char buf[64];
  std::snprintf(buf, sizeof(buf), "%a", double(v));
  return std::string("((float)") + buf + ")";
}

uint64_t fnv1a64(const std::string& s) {
  uint64_t h = 1469598103934665603ull;
  for (unsigned char c : s) {
    h ^= c;
    h *= 1099511628211ull;
  }
  return h;
}

int arity(int code) {
  switch (code) {
    case BG_OP_NEG: case BG_OP_EXP: case BG_OP_LOG: case BG_OP_ROUND_F16:
    case BG_OP_ROUND_BF16: case BG_OP_TANH: case BG_OP_SQRT: case BG_OP_RECIP:
    case BG_OP_ABS: case BG_OP_COPY:
      return 1;
    case BG_OP_WHERE: return 3;
    case BG_OP_IMM: return 0;
    default: return 2;
  }
}

struct Plan {
  int n_in = 0;
  int kind[BG_FUSED_MAX_INPUTS] = {};
  int dtype[BG_FUSED_MAX_INPUTS] = {};
  int nlead = 0;
  int vec = 1;
  int reduce = BG_RED_NONE;
  int tpr = 64;
  int split = 0;
  int one_pass = 0;  // every row fits one vector per lane of its TPR lanes
  int out_dtype = BG_F32;
  std::vector<bg_fused_op> ops;
};

// Source of one element load of input i at element offset expression `off`.
std::string load1_expr(int dtype, int i, const std::string& off) {
  std::ostringstream os;
  switch (dtype) {
    case BG_F32: os << "((const float*)A.in[" << i << "])[" << off << "]"; break;
    case BG_F16: os << "bg_h2f(((const u16*)A.in[" << i << "])[" << off << "])"; break;
    case BG_BF16: os << "bg_b2f(((const u16*)A.in[" << i << "])[" << off << "])"; break;
    default: os << "(((const unsigned char*)A.in[" << i << "])[" << off << "] ? 1.f : 0.f)"; break;
  }
  return os.str();
}

// Emits `float x<i>[V]` holding V consecutive elements starting at `off`.
void emit_vec_load(std::ostringstream& os, int dtype, int i, const std::string& off, int V) {
  if (V == 4) {
    switch (dtype) {
      // 16-byte (8-byte) aligned vector loads (the launcher picks V = 4
      // only for aligned bases and strides); LD_ is the nontemporal load in
      // reductions, whose operands stream through once with nothing
      // written back (measured: 6.3 -> 6.7 TB/s read on the C2 shape), and a
      // plain load in map kernels (the hint slowed f32 -> f16 casts by 20%).
      case BG_F32:
        os << "    f4v_ t" << i << " = LD_((const f4v_*)((const float*)A.in[" << i << "] + (" << off
           << ")));\n    float x" << i << "[4] = {t" << i << ".x, t" << i << ".y, t" << i << ".z, t" << i
           << ".w};\n";
        return;
      case BG_F16:
      case BG_BF16: {
        const char* cv = dtype == BG_F16 ? "bg_h2f" : "bg_b2f";
        os << "    u2v_ t" << i << " = LD_((const u2v_*)((const u16*)A.in[" << i << "] + (" << off << ")));\n"
           << "    float x" << i << "[4] = {" << cv << "((u16)t" << i << ".x), " << cv << "((u16)(t" << i
           << ".x >> 16)), " << cv << "((u16)t" << i << ".y), " << cv << "((u16)(t" << i << ".y >> 16))};\n";
        return;
      }
      default:
        os << "    u32 t" << i << " = *(const u32*)((const unsigned char*)A.in[" << i << "] + (" << off
           << "));\n    float x" << i << "[4] = {(t" << i << " & 0xffu) ? 1.f : 0.f, (t" << i
           << " & 0xff00u) ? 1.f : 0.f, (t" << i << " & 0xff0000u) ? 1.f : 0.f, (t" << i
           << " & 0xff000000u) ? 1.f : 0.f};\n";
        return;
    }
  }
  os << "    float x" << i << "[1] = {" << load1_expr(dtype, i, off) << "};\n";
}

std::string operand(int ref, int n_in) {
  if (ref < 0) {
    const int i = -ref - 1;
    (void)n_in;
    return "x" + std::to_string(i) + "[j]";
  }
  return "s" + std::to_string(ref) + "[j]";
}

std::string op_expr(const bg_fused_op& op, int n_in) {
  const std::string a = op.code == BG_OP_IMM ? "" : operand(op.a, n_in);
  const int na = arity(op.code);
  const std::string b = na >= 2 ? operand(op.b, n_in) : "";
  const std::string c = na >= 3 ? operand(op.c, n_in) : "";
  switch (op.code) {
    case BG_OP_ADD: return a + " + " + b;
    case BG_OP_MUL: return a + " * " + b;
    case BG_OP_DIV: return a + " / " + b;
    case BG_OP_SUB: return a + " - " + b;
    case BG_OP_NEG: return "-" + a;
    case BG_OP_EXP: return "expf(" + a + ")";
    case BG_OP_LOG: return "logf(" + a + ")";
    case BG_OP_MAX: return "bg_max(" + a + ", " + b + ")";
    case BG_OP_MIN: return "bg_min(" + a + ", " + b + ")";
    case BG_OP_CMP_EQ: return "(" + a + " == " + b + ") ? 1.f : 0.f";
    case BG_OP_CMP_NE: return "(" + a + " != " + b + ") ? 1.f : 0.f";
    case BG_OP_CMP_LT: return "(" + a + " < " + b + ") ? 1.f : 0.f";
    case BG_OP_CMP_LE: return "(" + a + " <= " + b + ") ? 1.f : 0.f";
    case BG_OP_CMP_GT: return "(" + a + " > " + b + ") ? 1.f : 0.f";
    case BG_OP_CMP_GE: return "(" + a + " >= " + b + ") ? 1.f : 0.f";
    case BG_OP_WHERE: return "(" + a + " != 0.f) ? " + b + " : " + c;
    case BG_OP_IMM: return "A.imm[" + std::to_string(op.a) + "]";
    case BG_OP_ROUND_F16: return "bg_rh(" + a + ")";
    case BG_OP_ROUND_BF16: return "bg_rb(" + a + ")";
    case BG_OP_TANH: return "tanhf(" + a + ")";
    case BG_OP_SQRT: return "sqrtf(" + a + ")";
    case BG_OP_RECIP: return "1.0f / " + a;
    case BG_OP_ABS: return "fabsf(" + a + ")";
    case BG_OP_COPY: return a;
    default: return "0.f";
  }
}

// Body shared by both kernel shapes: loads at (row, col, lin), op chain,
// result in s<last>[V].
void emit_body(std::ostringstream& os, const Plan& p, int V) {
  bool any_strided = false;
  for (int i = 0; i < p.n_in; ++i) any_strided |= p.kind[i] == IN_STRIDED;
  if (any_strided) {
    // The outermost leading index is what remains (row < rows), the others
    // come from multiply-high divisions.
    os << "    u32 idx[4] = {0u, 0u, 0u, 0u};\n    { u32 rr = (u32)row;\n";
    for (int d = p.nlead - 1; d >= 1; --d)
      os << "      { const u32 q = bg_fdiv(rr, A.dim_d[" << d << "], A.dim_m[" << d << "], A.dim_s[" << d
         << "]); idx[" << d << "] = rr - q * A.dim_d[" << d << "]; rr = q; }\n";
    if (p.nlead >= 1) os << "      idx[0] = rr;\n";
    os << "    }\n";
  }
  // Which inputs are used at all.
  std::vector<bool> used(p.n_in, false);
  for (const auto& op : p.ops) {
    const int na = arity(op.code);
    const int r[3] = {op.a, op.b, op.c};
    for (int k = 0; k < na; ++k)
      if (r[k] < 0) used[-r[k] - 1] = true;
  }
  for (int i = 0; i < p.n_in; ++i) {
    if (!used[i]) continue;
    if (p.kind[i] == IN_CONTIG) {
      emit_vec_load(os, p.dtype[i], i, "lin", V);
    } else if (p.kind[i] == IN_SCALAR) {
      os << "    float x" << i << "[" << V << "];\n#pragma unroll\n    for (int j = 0; j < " << V
         << "; ++j) x" << i << "[j] = xs" << i << ";\n";
    } else {
      os << "    i64 o" << i << " = col * A.stride[" << i << "][" << p.nlead << "]";
      for (int d = 0; d < p.nlead; ++d) os << " + (i64)idx[" << d << "] * A.stride[" << i << "][" << d << "]";
      os << ";\n";
      // Vector load only when the innermost stride is 1 (decided at run time).
      os << "    float x" << i << "[" << V << "];\n";
      os << "    { const i64 is = A.stride[" << i << "][" << p.nlead << "];\n";
      if (V == 4) {
        os << "      if (is == 1) {\n";
        std::ostringstream tmp;
        emit_vec_load(tmp, p.dtype[i], i, "o" + std::to_string(i), 4);
        std::string t = tmp.str();
        // Rename the temporary array to avoid clashing with x<i>.
        const std::string from = "float x" + std::to_string(i) + "[4]";
        const std::string to = "float y" + std::to_string(i) + "[4]";
        t.replace(t.find(from), from.size(), to);
        os << t;
        os << "        for (int j = 0; j < 4; ++j) x" << i << "[j] = y" << i << "[j];\n";
        os << "      } else {\n";
        os << "#pragma unroll\n        for (int j = 0; j < 4; ++j) x" << i << "[j] = "
           << load1_expr(p.dtype[i], i, "o" + std::to_string(i) + " + j * is") << ";\n";
        os << "      }\n";
      } else {
        os << "      x" << i << "[0] = " << load1_expr(p.dtype[i], i, "o" + std::to_string(i)) << ";\n";
      }
      os << "    }\n";
    }
  }
  for (size_t k = 0; k < p.ops.size(); ++k) {
    os << "    float s" << k << "[" << V << "];\n#pragma unroll\n    for (int j = 0; j < " << V
       << "; ++j) s" << k << "[j] = " << op_expr(p.ops[k], p.n_in) << ";\n";
  }
}

std::string store_expr(int dtype, const std::string& ptr_off, const std::string& val) {
  std::ostringstream os;
  switch (dtype) {
    case BG_F32: os << "((float*)A.out)[" << ptr_off << "] = " << val << ";"; break;
    case BG_F16: os << "((u16*)A.out)[" << ptr_off << "] = bg_f2h(" << val << ");"; break;
    case BG_BF16: os << "((u16*)A.out)[" << ptr_off << "] = bg_f2b(" << val << ");"; break;
    default: os << "((unsigned char*)A.out)[" << ptr_off << "] = (" << val << ") != 0.f ? 1 : 0;"; break;
  }
  return os.str();
}

std::string generate(const Plan& p) {
  std::ostringstream os;
  os << kPrelude;
  const int V = p.vec;
  const int last = int(p.ops.size()) - 1;
  os << (p.reduce == BG_RED_NONE ? "#define LD_(p) (*(p))\n" : "#define LD_(p) __builtin_nontemporal_load(p)\n");
  os << "extern \"C\" __global__ void __launch_bounds__(256) bg_fused(Args A) {\n";
  // Scalars hoisted out of the loop.
  for (int i = 0; i < p.n_in; ++i)
    if (p.kind[i] == IN_SCALAR) os << "  const float xs" << i << " = " << load1_expr(p.dtype[i], i, "0") << ";\n";
  if (p.reduce == BG_RED_NONE) {
    os << "  const i64 vcols = A.cols / " << V << ";\n"
       << "  const i64 nvec = A.rows * vcols;\n"
       << "  for (i64 g = (i64)blockIdx.x * 256 + threadIdx.x; g < nvec; g += (i64)gridDim.x * 256) {\n"
       << "    const i64 lin = g * " << V << ";\n"
       // Fewer than 2^31 elements (the launcher's limit): 32-bit indices.
       << "    const u32 g32 = (u32)g;\n"
       << "    const u32 row32 = bg_fdiv(g32, A.vc_d, A.vc_m, A.vc_s);\n"
       << "    const i64 row = row32;\n"
       << "    const i64 col = (i64)(g32 - row32 * A.vc_d) * " << V << ";\n";
    emit_body(os, p, V);
    if (V == 4 && p.out_dtype == BG_F32) {
      os << "    f4v_ r = {s" << last << "[0], s" << last << "[1], s" << last << "[2], s" << last << "[3]};\n"
         << "    *(f4v_*)((float*)A.out + lin) = r;\n";
    } else if (V == 4 && (p.out_dtype == BG_F16 || p.out_dtype == BG_BF16)) {
      const char* cv = p.out_dtype == BG_F16 ? "bg_f2h" : "bg_f2b";
      os << "    u2v_ r = {(u32)" << cv << "(s" << last << "[0]) | ((u32)" << cv << "(s" << last
         << "[1]) << 16), (u32)" << cv << "(s" << last << "[2]) | ((u32)" << cv << "(s" << last
         << "[3]) << 16)};\n    *(u2v_*)((u16*)A.out + lin) = r;\n";
    } else {
      os << "#pragma unroll\n    for (int j = 0; j < " << V << "; ++j) { "
         << store_expr(p.out_dtype, "lin + j", "s" + std::to_string(last) + "[j]") << " }\n";
    }
    os << "  }\n}\n";
    return os.str();
  }
  // Reduction over the innermost axis.
  const char* comb = p.reduce == BG_RED_MAX ? "bg_max" : p.reduce == BG_RED_MIN ? "bg_min" : nullptr;
  const char* ident = p.reduce == BG_RED_MAX ? "(-__builtin_inff())"
                      : p.reduce == BG_RED_MIN ? "__builtin_inff()" : "0.f";
  auto combine = [&](const std::string& a, const std::string& b) {
    return comb ? std::string(comb) + "(" + a + ", " + b + ")" : "(" + a + " + " + b + ")";
  };
  // TPR lanes per row (a power of two dividing 64, or 256 = the whole
  // workgroup); split plans give each workgroup one chunk of a row and write
  // the raw partial, which a second kernel combines per row in chunk order.
  const int TPR = p.split ? 256 : p.tpr;
  const int RPB = 256 / TPR;
  os << "  __shared__ float part[4];\n"
     << "  const int lane = threadIdx.x % " << TPR << ";\n"
     << "  const int sub = threadIdx.x / " << TPR << ";\n";
  if (p.one_pass && TPR <= 64) {
    // Narrow rows (one vector per lane covers the row): each workgroup pass
    // takes NU row blocks, all loads issued before the first butterfly.
    const int NU = V == 1 ? 8 : 4;
    os << "  for (i64 row0 = (i64)blockIdx.x * " << RPB * NU << "; row0 < A.rows; row0 += (i64)gridDim.x * "
       << RPB * NU << ") {\n"
       << "    float accu[" << NU << "];\n"
       << "#pragma unroll\n"
       << "    for (int q = 0; q < " << NU << "; ++q) {\n"
       << "    const i64 row = row0 + q * " << RPB << " + sub;\n"
       << "    const i64 col = (i64)lane * " << V << ";\n"
       << "    float acc = " << ident << ";\n"
       << "    if (row < A.rows && col < A.cols) {\n"
       << "    const i64 lin = row * A.cols + col;\n";
    emit_body(os, p, V);
    os << "#pragma unroll\n    for (int j = 0; j < " << V << "; ++j) acc = "
       << combine("acc", "s" + std::to_string(last) + "[j]") << ";\n";
    os << "    }\n    accu[q] = acc;\n    }\n";
    os << "#pragma unroll\n    for (int q = 0; q < " << NU << "; ++q) {\n"
       << "    float acc = accu[q];\n";
    if (TPR > 1)
      os << "#pragma unroll\n    for (int s = " << TPR / 2 << "; s >= 1; s >>= 1) acc = "
         << combine("acc", "__shfl_xor(acc, s, 64)") << ";\n";
    os << "    const i64 row = row0 + q * " << RPB << " + sub;\n"
       << "    if (row < A.rows && lane == 0) {\n";
    if (p.reduce == BG_RED_MEAN) os << "      acc = acc / (float)A.cols;\n";
    os << "      " << store_expr(p.out_dtype, "row", "acc") << "\n    }\n    }\n  }\n}\n";
    return os.str();
  }
  if (p.split) {
    os << "  const i64 units = A.rows * A.nch;\n"
       << "  for (i64 u = blockIdx.x; u < units; u += gridDim.x) {\n"
       << "    const i64 row = u / A.nch;\n"
       << "    const i64 c0 = (u - row * A.nch) * A.cw;\n"
       << "    const i64 c1 = c0 + A.cw < A.cols ? c0 + A.cw : A.cols;\n"
       << "    const bool live = true;\n"
       << "    float acc = " << ident << ";\n"
       << "    {\n"
       << "#pragma unroll 4\n"
       << "    for (i64 col = c0 + (i64)lane * " << V << "; col < c1; col += " << TPR * V << ") {\n"
       << "    const i64 lin = row * A.cols + col;\n";
  } else {
    os << "  for (i64 row0 = (i64)blockIdx.x * " << RPB << "; row0 < A.rows; row0 += (i64)gridDim.x * " << RPB
       << ") {\n"
       << "    const i64 row = row0 + sub;\n"
       << "    const bool live = row < A.rows;\n"
       << "    float acc = " << ident << ";\n"
       << "    if (live) {\n"
       << "#pragma unroll 4\n"
       << "    for (i64 col = (i64)lane * " << V << "; col < A.cols; col += " << TPR * V << ") {\n"
       << "    const i64 lin = row * A.cols + col;\n";
  }
  emit_body(os, p, V);
  os << "#pragma unroll\n    for (int j = 0; j < " << V << "; ++j) acc = "
     << combine("acc", "s" + std::to_string(last) + "[j]") << ";\n";
  os << "    }\n    }\n";
  if (TPR > 1)
    os << "#pragma unroll\n    for (int s = " << (TPR < 64 ? TPR : 64) / 2 << "; s >= 1; s >>= 1) acc = "
       << combine("acc", "__shfl_xor(acc, s, 64)") << ";\n";
  if (TPR == 256) {
    os << "    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;\n"
       << "    __syncthreads();\n"
       << "    acc = " << combine(combine("part[0]", "part[1]"), combine("part[2]", "part[3]")) << ";\n"
       << "    __syncthreads();\n";
  }
  if (p.split) {
    os << "    if (threadIdx.x == 0) A.part[u] = acc;\n  }\n}\n";
    return os.str();
  }
  os << "    if (live && lane == 0) {\n";
  if (p.reduce == BG_RED_MEAN) os << "      acc = acc / (float)A.cols;\n";
  os << "      " << store_expr(p.out_dtype, "row", "acc") << "\n    }\n  }\n}\n";
  return os.str();
}

// ---- compile + cache ------------------------------------------------------------

struct KernelCache {
  std::mutex mu;
  std::unordered_map<uint64_t, hipFunction_t> fns;  // keyed by hash(device, source)
  // Front cache keyed by the compact plan signature, so a repeated launch
  // skips source generation, hashing and the device-property query.
  std::unordered_map<std::string, hipFunction_t> by_plan;
};

KernelCache& cache() {
  static KernelCache c;
  return c;
}

std::string cache_dir() {
  const char* e = std::getenv("BG_KERNEL_CACHE");
  if (e && *e) return e;
  const char* home = std::getenv("HOME");
  return std::string(home && *home ? home : "/tmp") + "/.cache/bghip";
}

bool read_file(const std::string& path, std::vector<char>& out) {
  std::ifstream f(path, std::ios::binary);
  if (!f) return false;
  out.assign(std::istreambuf_iterator<char>(f), std::istreambuf_iterator<char>());
  return !out.empty();
}

void write_file_atomic(const std::string& dir, const std::string& name, const std::vector<char>& data) {
  std::string cur;
  for (size_t i = 1; i <= dir.size(); ++i) {
    if (i == dir.size() || dir[i] == '/') {
      cur = dir.substr(0, i);
      mkdir(cur.c_str(), 0755);
    }
  }
  const std::string tmp = dir + "/" + name + ".tmp" + std::to_string(getpid());
  {
    std::ofstream f(tmp, std::ios::binary);
    if (!f) return;
    f.write(data.data(), std::streamsize(data.size()));
  }
  std::rename(tmp.c_str(), (dir + "/" + name).c_str());
}

std::vector<char> compile_source(const std::string& src, const std::string& arch) {
  hiprtcProgram prog;
  if (hiprtcCreateProgram(&prog, src.c_str(), "bg_fused.hip", 0, nullptr, nullptr) != HIPRTC_SUCCESS)
    bg::fail(BG_E_HIP, "fused_elementwise: hiprtcCreateProgram failed");
  const std::string archopt = "--offload-arch=" + arch;
  const char* opts[] = {archopt.c_str(), "-O3", "-ffp-contract=off", "-std=c++17",
                        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};
  hiprtcResult r = hiprtcCompileProgram(prog, int(sizeof(opts) / sizeof(opts[0])), opts);
  if (r != HIPRTC_SUCCESS) {
    size_t n = 0;
    hiprtcGetProgramLogSize(prog, &n);
    std::string log(n + 1, '\0');
    hiprtcGetProgramLog(prog, &log[0]);
    hiprtcDestroyProgram(&prog);
    bg::fail(BG_E_HIP, "fused_elementwise: hipRTC compile failed: " + log);
  }
  size_t n = 0;
  hiprtcGetCodeSize(prog, &n);
  std::vector<char> code(n);
  hiprtcGetCode(prog, code.data());
  hiprtcDestroyProgram(&prog);
  return code;
}

std::string device_arch(int device) {
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) return "gfx950";
  std::string a = prop.gcnArchName;
  const size_t colon = a.find(':');
  if (colon != std::string::npos) a = a.substr(0, colon);
  return a.empty() ? "gfx950" : a;
}

hipFunction_t get_kernel(int device, const std::string& src) {
  const std::string arch = device_arch(device);
  const uint64_t key = fnv1a64(arch + "\n" + src) ^ uint64_t(device);
  KernelCache& c = cache();
  {
    std::lock_guard<std::mutex> g(c.mu);
    auto it = c.fns.find(key);
    if (it != c.fns.end()) return it->second;
  }
  char name[40];
  std::snprintf(name, sizeof(name), "%016llx.%s.co", static_cast<unsigned long long>(key), arch.c_str());
  const std::string dir = cache_dir();
  std::vector<char> code;
  if (!read_file(dir + "/" + name, code)) {
    code = compile_source(src, arch);
    write_file_atomic(dir, name, code);
  }
  hipModule_t mod;
  bg::hip_check(hipModuleLoadData(&mod, code.data()), "fused_elementwise module load");
  hipFunction_t fn;
  bg::hip_check(hipModuleGetFunction(&fn, mod, "bg_fused"), "fused_elementwise function");
  std::lock_guard<std::mutex> g(c.mu);
  c.fns[key] = fn;
  return fn;
}

}  // namespace

namespace bg {

void launch_fused(bg_ctx* ctx, const bg_fused_desc& d, Record& out) {
  FusedArgs A;
  std::memset(&A, 0, sizeof(A));
  Plan plan;
  const int n_in = d.n_inputs;
  plan.n_in = n_in;
  auto shape = to_shape(d.shape, d.rank);
  const int64_t total = numel(shape);

  std::vector<std::vector<int64_t>> strides(n_in);
  for (int i = 0; i < n_in; ++i) {
    Record& r = get(ctx, d.inputs[i], "fused_elementwise[in]");
    if (r.dtype != BG_F32 && r.dtype != BG_F16 && r.dtype != BG_BF16 && r.dtype != BG_BOOL &&
        r.dtype != BG_U8)
      fail(BG_E_DTYPE, std::string("fused_elementwise: input dtype ") + dtype_name(r.dtype) +
                           " not supported");
    A.in[i] = r.ptr();
    plan.dtype[i] = r.dtype;
    std::vector<int64_t> st(shape.size());
    if (d.in_strides) {
      for (size_t k = 0; k < shape.size(); ++k) st[k] = d.in_strides[i * d.rank + k];
    } else {
      if (r.numel() != total)
        fail(BG_E_SHAPE, "fused_elementwise: input " + std::to_string(i) +
                             " does not match the iteration shape");
      int64_t s = 1;
      for (int k = int(shape.size()) - 1; k >= 0; --k) {
        st[k] = s;
        s *= shape[k];
      }
    }
    if (total > 0) {
      int64_t hi = 0;
      for (size_t k = 0; k < shape.size(); ++k) {
        if (st[k] < 0) fail(BG_E_INVALID, "fused_elementwise: negative stride");
        hi += (shape[k] - 1) * st[k];
      }
      if (hi >= r.numel())
        fail(BG_E_SHAPE, "fused_elementwise: input " + std::to_string(i) +
                             " view reaches outside its tensor");
    }
    strides[i] = std::move(st);
  }

  // rows x cols with cols the innermost dim; leading dims collapsed.
  std::vector<int64_t> lead(shape.begin(), shape.end());
  int64_t cols = 1;
  std::vector<int64_t> inner(n_in, 0);
  if (!lead.empty()) {
    cols = lead.back();
    lead.pop_back();
    for (int i = 0; i < n_in; ++i) inner[i] = strides[i].back();
  }
  std::vector<std::vector<int64_t>> lst(n_in);
  {
    std::vector<int64_t> l2;
    for (int i = 0; i < n_in; ++i) lst[i].clear();
    for (size_t k = 0; k < lead.size(); ++k) {
      if (lead[k] == 1) continue;
      l2.push_back(lead[k]);
      for (int i = 0; i < n_in; ++i) lst[i].push_back(strides[i][k]);
    }
    lead = l2;
  }
  for (size_t k = 0; k + 1 < lead.size();) {
    bool ok = true;
    for (int i = 0; i < n_in; ++i)
      if (lst[i][k] != lst[i][k + 1] * lead[k + 1]) ok = false;
    if (ok) {
      lead[k] *= lead[k + 1];
      lead.erase(lead.begin() + long(k) + 1);
      for (int i = 0; i < n_in; ++i) {
        lst[i][k] = lst[i][k + 1];
        lst[i].erase(lst[i].begin() + long(k) + 1);
      }
    } else {
      ++k;
    }
  }
  if (lead.size() > 3)
    fail(BG_E_UNSUPPORTED, "fused_elementwise: more than 3 non-mergeable leading dims");
  if (total >= (int64_t(1) << 31))
    fail(BG_E_UNSUPPORTED, "fused_elementwise: more than 2^31 elements");
  int64_t rows = 1;
  for (int64_t v : lead) rows *= v;
  plan.nlead = int(lead.size());
  for (size_t k = 0; k < lead.size(); ++k) A.dims[k] = uint32_t(lead[k]);
  A.rows = rows;
  A.cols = cols;
  for (int i = 0; i < n_in; ++i) {
    bool scalar = (cols == 1 || inner[i] == 0);
    for (int64_t s : lst[i])
      if (s != 0) scalar = false;
    bool contig = (inner[i] == 1 || cols == 1);
    int64_t expect = cols;
    for (int k = int(lead.size()) - 1; k >= 0; --k) {
      if (lst[i][k] != expect) contig = false;
      expect *= lead[k];
    }
    if (contig) {
      plan.kind[i] = IN_CONTIG;
    } else if (scalar) {
      plan.kind[i] = IN_SCALAR;
    } else {
      plan.kind[i] = IN_STRIDED;
      for (size_t k = 0; k < lead.size(); ++k) A.stride[i][k] = lst[i][k];
      A.stride[i][lead.size()] = cols == 1 ? 0 : inner[i];
    }
  }

  // A large operand read transposed (innermost stride neither 0 nor 1)
  // would gather each lane's vector from distant rows; it is first copied
  // to row-major order (the tiled-transpose copy) and read contiguously.
  {
    int64_t need = 0;
    std::vector<int> tr;
    for (int i = 0; i < n_in; ++i) {
      if (plan.kind[i] != IN_STRIDED || cols == 1) continue;
      const int64_t is = A.stride[i][lead.size()];
      if (is == 0 || is == 1 || total < (int64_t(1) << 20)) continue;
      tr.push_back(i);
      need += (total * dtype_size(plan.dtype[i]) + 255) / 256 * 256;
    }
    if (!tr.empty()) {
      char* buf = static_cast<char*>(scratch(ctx, size_t(need), 2));
      for (int i : tr) {
        std::vector<int64_t> shp(lead.begin(), lead.end()), st;
        shp.push_back(cols);
        for (size_t k = 0; k < lead.size(); ++k) st.push_back(A.stride[i][k]);
        st.push_back(A.stride[i][lead.size()]);
        const int64_t es = dtype_size(plan.dtype[i]);
        launch_copy_strided(ctx, A.in[i], es, buf, shp, st);
        A.in[i] = buf;
        plan.kind[i] = IN_CONTIG;
        for (size_t k = 0; k <= lead.size(); ++k) A.stride[i][k] = 0;
        buf += (total * es + 255) / 256 * 256;
      }
    }
  }

  // Validate the op list (SSA refs, arities, immediates).
  if (d.n_imms > BG_FUSED_MAX_IMMS) fail(BG_E_INVALID, "fused_elementwise: too many immediates");
  for (int i = 0; i < d.n_imms; ++i) A.imm[i] = float(d.imms[i]);
  for (int s = 0; s < d.n_ops; ++s) {
    const bg_fused_op& op = d.ops[s];
    if (op.code < 0 || op.code >= BG_OP_COUNT_)
      fail(BG_E_UNSUPPORTED, "fused_elementwise: unsupported opcode " + std::to_string(op.code));
    if (op.code == BG_OP_IMM) {
      if (op.a < 0 || op.a >= d.n_imms)
        fail(BG_E_INVALID, "fused_elementwise: immediate index out of range");
    } else {
      const int refs[3] = {op.a, op.b, op.c};
      for (int k = 0; k < arity(op.code); ++k) {
        const int ref = refs[k];
        if (ref < 0 && -ref - 1 >= n_in)
          fail(BG_E_INVALID, "fused_elementwise: step " + std::to_string(s) + " references input " +
                                 std::to_string(-ref - 1) + " of " + std::to_string(n_in));
        if (ref >= s)
          fail(BG_E_INVALID, "fused_elementwise: step " + std::to_string(s) +
                                 " references step " + std::to_string(ref) + " (not earlier)");
      }
    }
    bg_fused_op clean = op;
    if (arity(op.code) < 3) clean.c = 0;
    if (arity(op.code) < 2) clean.b = 0;
    plan.ops.push_back(clean);
  }
  plan.out_dtype = d.out_dtype;
  plan.reduce = d.reduce_op;
  A.out = out.ptr();
  if (total == 0) return;

  // Vector width 4 when every streaming input (and the output of a map) can
  // be read with aligned 4-element vectors along the innermost dim.
  bool v4 = cols % 4 == 0;
  for (int i = 0; i < n_in && v4; ++i) {
    if (plan.kind[i] == IN_SCALAR) continue;
    const int64_t es = dtype_size(plan.dtype[i]);
    if (reinterpret_cast<uintptr_t>(A.in[i]) % uintptr_t(4 * es) != 0) v4 = false;
    if (plan.kind[i] == IN_STRIDED)
      for (int k = 0; k < plan.nlead; ++k)
        if (A.stride[i][k] % 4 != 0) v4 = false;
  }
  if (d.reduce_op == BG_RED_NONE &&
      reinterpret_cast<uintptr_t>(A.out) % uintptr_t(4 * dtype_size(d.out_dtype)) != 0)
    v4 = false;
  plan.vec = v4 ? 4 : 1;
  // Multiply-high division constants (Granlund and Montgomery, PLDI 1994,
  // round-up method): l = ceil(log2 d), m = floor(2^32 (2^l - d) / d) + 1.
  auto magic = [](int64_t dv, uint32_t& d, uint32_t& m, uint32_t& sh) {
    d = uint32_t(dv);
    uint32_t l = 0;
    while ((uint64_t(1) << l) < d) ++l;
    m = uint32_t(((uint64_t(1) << 32) * ((uint64_t(1) << l) - d)) / d + 1);
    sh = l;
  };
  magic(cols / plan.vec, A.vc_d, A.vc_m, A.vc_s);
  for (size_t k = 0; k < lead.size(); ++k) magic(lead[k], A.dim_d[k], A.dim_m[k], A.dim_s[k]);
  // Lanes per row for reductions: the whole workgroup for wide rows, else
  // the fewest power-of-two lanes (at most a wavefront) that cover the row
  // in one vector each, so narrow rows do not leave most lanes idle.
  if (cols >= 2048) {
    plan.tpr = 256;
  } else {
    int t = 1;
    while (t < 64 && int64_t(t) * plan.vec < cols) t *= 2;
    plan.tpr = t;
    plan.one_pass = int64_t(t) * plan.vec >= cols;
  }
  // Few wide rows: cut each row into chunks of whole 256-lane vector steps
  // (at least 8 per chunk) until about 1024 workgroups stream the input;
  // a second kernel combines each row's chunk partials in order.
  if (d.reduce_op != BG_RED_NONE && plan.tpr == 256 && rows < 512) {
    const int64_t step = 256 * int64_t(plan.vec);
    const int64_t min_cw = 8 * step;
    int64_t nch = std::min<int64_t>((1024 + rows - 1) / rows, (cols + min_cw - 1) / min_cw);
    if (nch > 1) {
      int64_t cw = (cols + nch - 1) / nch;
      cw = (cw + step - 1) / step * step;
      plan.split = 1;
      A.cw = cw;
      A.nch = (cols + cw - 1) / cw;
    }
  }

  int64_t in_bytes = 0;
  for (int i = 0; i < n_in; ++i)
    if (plan.kind[i] != IN_SCALAR) in_bytes += dtype_size(plan.dtype[i]);

  // Compact binary signature of everything generate() depends on.
  std::string sig;
  {
    int32_t head[10] = {ctx->device, plan.n_in, plan.nlead, plan.vec, plan.reduce, plan.tpr,
                        plan.split, plan.one_pass, plan.out_dtype, int32_t(plan.ops.size())};
    sig.append(reinterpret_cast<const char*>(head), sizeof(head));
    for (int i = 0; i < plan.n_in; ++i) {
      int32_t io[2] = {plan.kind[i], plan.dtype[i]};
      sig.append(reinterpret_cast<const char*>(io), sizeof(io));
    }
    sig.append(reinterpret_cast<const char*>(plan.ops.data()), plan.ops.size() * sizeof(bg_fused_op));
  }
  hipFunction_t fn = nullptr;
  {
    KernelCache& c = cache();
    std::lock_guard<std::mutex> g(c.mu);
    auto it = c.by_plan.find(sig);
    if (it != c.by_plan.end()) fn = it->second;
  }
  if (!fn) {
    fn = get_kernel(ctx->device, generate(plan));
    KernelCache& c = cache();
    std::lock_guard<std::mutex> g(c.mu);
    c.by_plan[sig] = fn;
  }
  size_t argsz = sizeof(A);
  void* cfg[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, &A, HIP_LAUNCH_PARAM_BUFFER_SIZE, &argsz,
                 HIP_LAUNCH_PARAM_END};
  unsigned grid;
  int64_t obytes;
  if (d.reduce_op == BG_RED_NONE) {
    const int64_t items = total / plan.vec;
    grid = unsigned(std::max<int64_t>(1, std::min<int64_t>((items + 255) / 256, 256 * 16)));
    obytes = total * dtype_size(d.out_dtype);
  } else if (plan.split) {
    A.part = static_cast<float*>(scratch(ctx, size_t(rows * A.nch) * 4, 0));
    grid = unsigned(rows * A.nch);
    obytes = rows * dtype_size(d.out_dtype);
  } else {
    // Rows per workgroup pass: 256 / tpr, times the row blocks a narrow-row
    // kernel takes per pass (8 with scalar loads, 4 with vectors).
    const int64_t rpb = (256 / plan.tpr) * (plan.one_pass ? (plan.vec == 1 ? 8 : 4) : 1);
    grid = unsigned(std::max<int64_t>(1, std::min<int64_t>((rows + rpb - 1) / rpb, int64_t(1) << 20)));
    obytes = rows * dtype_size(d.out_dtype);
  }
  Profile prof(ctx, d.reduce_op == BG_RED_NONE ? "fused_elementwise" : "fused_reduce",
               total * in_bytes + obytes, total * int64_t(plan.ops.size()));
  hipEvent_t ev_start = nullptr, ev_stop = nullptr;
  next_dispatch_events(ctx, &ev_start, &ev_stop);
  // Global size in work-items (grid blocks x 256 lanes).
  hip_check(hipExtModuleLaunchKernel(fn, grid * 256u, 1, 1, 256, 1, 1, 0, ctx->stream, nullptr, cfg,
                                     ev_start, plan.split ? nullptr : ev_stop, 0),
            "fused_elementwise launch");
  if (plan.split) {
    launch_reduce_partials(ctx, A.part, rows, A.nch, d.reduce_op, cols, A.out, d.out_dtype);
    if (ev_stop) hip_check(hipEventRecord(ev_stop, ctx->stream), "hipEventRecord");
  }
}

}  // namespace bg

// Codegen self-test: generates and compiles (hipRTC, no device needed) a set
// of representative programs covering every opcode, dtype, input kind,
// vector width and reduction shape.  Returns the number of failures; the
// first error is copied into `err`.
extern "C" int bg_fused_codegen_selftest(char* err, size_t cap) {
  int failures = 0;
  auto attempt = [&](const Plan& p) {
    try {
      (void)compile_source(generate(p), "gfx950");
    } catch (const bg::Error& e) {
      if (failures == 0 && err && cap) std::snprintf(err, cap, "%s", e.what());
      ++failures;
    }
  };
  const int dtypes[] = {BG_F32, BG_F16, BG_BF16, BG_BOOL};
  for (int vec : {1, 4}) {
    for (int red : {int(BG_RED_NONE), int(BG_RED_SUM), int(BG_RED_MAX), int(BG_RED_MEAN)}) {
      for (int od : {int(BG_F32), int(BG_F16), int(BG_BF16), int(BG_BOOL)}) {
        if (red != BG_RED_NONE && od == BG_BOOL) continue;
        Plan p;
        p.n_in = 4;
        p.vec = vec;
        p.reduce = red;
        p.tpr = red == BG_RED_SUM ? 256 : od == BG_F16 ? 1 : od == BG_BF16 ? 8 : 64;
        p.split = red == BG_RED_MEAN;
        p.one_pass = red == BG_RED_MAX;
        p.out_dtype = od;
        p.nlead = 2;
        for (int i = 0; i < 4; ++i) {
          p.dtype[i] = dtypes[(i + vec + od) % 4];
          p.kind[i] = i % 3;  // contig, scalar, strided
        }
        p.kind[3] = IN_STRIDED;
        int s = 0;
        auto push = [&](int code, int a, int b, int c) { p.ops.push_back({code, a, b, c}); return s++; };
        int t0 = push(BG_OP_MUL, -1, -2, 0);
        int t1 = push(BG_OP_ADD, t0, -3, 0);
        int t2 = push(BG_OP_IMM, 0, 0, 0);
        int t3 = push(BG_OP_CMP_GT, t1, t2, 0);
        int t4 = push(BG_OP_WHERE, t3, t1, t2);
        int t5 = push(BG_OP_NEG, -4, 0, 0);
        int t6 = push(BG_OP_EXP, t5, 0, 0);
        int t7 = push(BG_OP_LOG, t6, 0, 0);
        int t8 = push(BG_OP_DIV, t7, t4, 0);
        int t9 = push(BG_OP_MAX, t8, t0, 0);
        int t10 = push(BG_OP_MIN, t9, t1, 0);
        int t11 = push(BG_OP_ROUND_F16, t10, 0, 0);
        int t12 = push(BG_OP_ROUND_BF16, t11, 0, 0);
        int t13 = push(BG_OP_TANH, t12, 0, 0);
        int t14 = push(BG_OP_SQRT, t13, 0, 0);
        int t15 = push(BG_OP_RECIP, t14, 0, 0);
        int t16 = push(BG_OP_ABS, t15, 0, 0);
        int t17 = push(BG_OP_SUB, t16, t2, 0);
        int t18 = push(BG_OP_CMP_EQ, t17, t16, 0);
        int t19 = push(BG_OP_CMP_NE, t18, t17, 0);
        int t20 = push(BG_OP_CMP_LT, t19, t18, 0);
        int t21 = push(BG_OP_CMP_LE, t20, t19, 0);
        int t22 = push(BG_OP_CMP_GE, t21, t20, 0);
        push(BG_OP_COPY, t22, 0, 0);
        attempt(p);
      }
    }
  }
  return failures;
}
