// Internal declarations shared by the libbghip translation units.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <tuple>
#include <unordered_map>
#include <vector>

#include "../../include/bghip.h"

namespace bg {

// Thrown inside the library, converted to a status + message at the C ABI.
struct Error : std::runtime_error {
  int code;
  Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

[[noreturn]] void fail(int code, const std::string& msg);
void hip_check(hipError_t e, const char* what);

int64_t dtype_size(int dtype);
const char* dtype_name(int dtype);

// A device allocation.  Several handles may share one (reshape views).
struct Alloc {
  void* ptr = nullptr;
  size_t bytes = 0;   // requested bytes
  size_t cap = 0;     // bytes of the pooled block
  int refs = 0;
};

struct Record {
  Alloc* alloc = nullptr;
  int64_t offset = 0;  // byte offset of this view inside alloc
  int64_t nbytes = 0;
  std::vector<int64_t> shape;
  int dtype = BG_F32;
  char* ptr() const { return static_cast<char*>(alloc->ptr) + offset; }
  int64_t numel() const {
    int64_t n = 1;
    for (int64_t d : shape) n *= d;
    return n;
  }
};

struct Profile;

struct PendingProfile {
  hipEvent_t start;
  hipEvent_t stop;
  bg_pass_profile info;
};

}  // namespace bg

struct bg_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  bool profiling = false;
  std::string err;
  uint64_t next_id = 1;
  std::unordered_map<uint64_t, bg::Record> handles;

  // Accounting, per allocation (realizer.ts:908-943 counts per buffer).
  int64_t current_owned = 0;
  int64_t peak_owned = 0;
  int64_t total_allocated = 0;
  int64_t total_released = 0;

  // Block cache: pooled-size -> free device blocks.
  std::multimap<size_t, void*> free_blocks;
  int64_t cached_bytes = 0;
  int64_t pool_hits = 0;
  int64_t pool_misses = 0;

  // Profiling.
  std::vector<bg::PendingProfile> pending;
  std::vector<bg_pass_profile> done;
  std::vector<hipEvent_t> event_pool;
  bg::Profile* active_profile = nullptr;

  // Scratch buffers reused across launches (workspace for pre-passes):
  // slot 0 = re-laid-out GEMM operand, slot 1 = f32 GEMM result awaiting an
  // elementwise epilogue pass.
  // GEMM scratch slots: 0 B re-layout / B cast, 1 f32 pre-GELU product,
  // 2 A cast, 3 split-K partials.
  void* scratch[4] = {nullptr, nullptr, nullptr, nullptr};
  size_t scratch_bytes[4] = {0, 0, 0, 0};

  // Device address of this device's fixed no-allocation scratch (NULL when
  // it could not be resolved; bg_matmul_noalloc then refuses).
  char* noalloc_scratch = nullptr;
  size_t noalloc_scratch_bytes = 0;
  std::string noalloc_error;

  // Launch log (bg_set_launch_log): one record per dispatch while on.
  bool log_launches = false;
  std::vector<bg_launch_record> launch_log;
};

namespace bg {

// Handle table / allocation helpers (core.cpp).
Record& get(bg_ctx* ctx, bg_handle h, const char* op);
bg_handle mint(bg_ctx* ctx, size_t nbytes, const std::vector<int64_t>& shape,
               int dtype);
bg_handle mint_view(bg_ctx* ctx, const Record& src, int64_t offset,
                    int64_t nbytes, const std::vector<int64_t>& shape,
                    int dtype);
void* scratch(bg_ctx* ctx, size_t bytes, int slot = 0);
std::vector<int64_t> to_shape(const int64_t* shape, int rank);
int64_t numel(const std::vector<int64_t>& shape);

// RAII profiling scope around the dispatches of one bridge operation.  The
// first kernel dispatched inside the scope carries the scope's start/stop
// events in its own dispatch packet (hipExtLaunchKernel), so the measured
// time is the kernel's execution time; when a scope dispatches more than one
// kernel, the stop event is re-recorded on the stream when the scope closes.
struct Profile {
  bg_ctx* ctx;
  bool on;
  int launches = 0;
  Profile* prev = nullptr;
  PendingProfile p;
  Profile(bg_ctx* c, const char* label, int64_t bytes, int64_t flops);
  ~Profile();
};

// Events the next dispatch on ctx->stream should carry (both NULL when no
// profiling scope is open or the scope already dispatched a kernel).
void next_dispatch_events(bg_ctx* ctx, hipEvent_t* start, hipEvent_t* stop);

// Appends one bg_launch_record for a launch of `kernel` (core.cpp).
void log_launch(bg_ctx* ctx, const void* kernel, dim3 grid, dim3 block, size_t shmem);

// Launch `kernel` on the context stream with the profiling scope's events.
template <typename... KArgs, typename... Args>
void dispatch(bg_ctx* ctx, void (*kernel)(KArgs...), dim3 grid, dim3 block, size_t shmem,
              Args... args) {
  static_assert(sizeof...(KArgs) == sizeof...(Args), "kernel argument count");
  std::tuple<KArgs...> vals(static_cast<KArgs>(args)...);
  void* ptrs[sizeof...(KArgs)];
  std::apply([&ptrs](auto&... v) {
    size_t i = 0;
    ((ptrs[i++] = static_cast<void*>(&v)), ...);
  }, vals);
  hipEvent_t start = nullptr, stop = nullptr;
  next_dispatch_events(ctx, &start, &stop);
  if (ctx->log_launches) log_launch(ctx, reinterpret_cast<const void*>(kernel), grid, block, shmem);
  hip_check(hipExtLaunchKernel(reinterpret_cast<const void*>(kernel), grid, block, ptrs, shmem,
                               ctx->stream, start, stop, 0),
            "kernel launch");
}

// Kernel launchers (one per translation unit).
void launch_fused(bg_ctx* ctx, const bg_fused_desc& d, Record& out);
void launch_gelu_rows(bg_ctx* ctx, const float* src, int64_t ld_src, int64_t stride_src, void* dst,
                      int64_t ld_dst, int64_t stride_dst, int dst_dtype, int64_t batch, int64_t rows,
                      int64_t cols, const float* residual = nullptr);
void launch_cast(bg_ctx* ctx, const void* src, int src_dtype, void* dst,
                 int dst_dtype, int64_t n);
void launch_cast_transpose(bg_ctx* ctx, const void* src, int src_dtype,
                           void* dst, int dst_dtype, int64_t rows,
                           int64_t cols, int64_t batch);
void launch_copy_strided(bg_ctx* ctx, const void* src, int64_t elem_size,
                         void* dst, const std::vector<int64_t>& shape,
                         const std::vector<int64_t>& strides);
void launch_layer_norm(bg_ctx* ctx, const void* x, int x_dtype,
                       const float* w, const float* b, void* y, int y_dtype,
                       int64_t rows, int64_t cols, float eps);
// A convolution in the "conv picture": x [n][c][in...] -> y [n][o][out...],
// weight [o][c/groups][k...]; spatial arrays are (D, H, W), unit-padded for
// 1-D and 2-D problems.
struct ConvProblem {
  int64_t n, c, o, groups;
  int64_t in[3], out[3], k[3], stride[3], pad[3], dil[3];
};
// Where a forward convolution's outputs go when they are one phase of a
// larger tensor: output (oh, ow) lands at (oh * sh + ph, ow * sw + pw) of an
// H x W plane (used by the strided input gradient's phase convolutions).
struct ConvOutMap {
  int sh, sw, ph, pw, H, W;
};
// mode 0: y = conv(a = x, b = w) (+ bias[o]); 1: dx = a = dy against b = w
// (+ bias[c]); 2: dw from a = dy, b = x.
// b_kmajor: mode 0 only, b already laid out [G][K][Opg] (the ring kernel's
// operand order).  omap: mode 0 only, 2-D, the outputs' phase placement.
void launch_conv(bg_ctx* ctx, const ConvProblem& p, int mode, const float* a, const float* b, const float* bias,
                 float* out, bool b_kmajor = false, const ConvOutMap* omap = nullptr);
void launch_conv_bias_grad(bg_ctx* ctx, const float* dy, float* out, int64_t n, int64_t o, int64_t spatial);
void launch_ln_backward_input(bg_ctx* ctx, const float* dy, const float* x, const float* w, float* dx,
                              int64_t rows, int64_t cols, float eps);
// Column sums over rows of dy * x_hat (weight) or dy (bias, x unused).
void launch_ln_backward_cols(bg_ctx* ctx, const float* dy, const float* x, float* out, int64_t rows, int64_t cols,
                             float eps, bool weight);
// Internal optimizer kinds: ADAMW_UPDATE_M, _V and _PARAM (or the ADAM_
// chain) as one pass over (param, grad, m, v), the plan executor's fusion of
// those chains.  `a` is the PARAM step's arguments; m_beta1 / v_beta2 (and,
// for Adam, the decays m_wd / v_wd) come from the M and V steps.
constexpr int kOptAdamwFused = 7;
constexpr int kOptAdamFused = 8;
void launch_optimizer_fused(bg_ctx* ctx, int kind, const bg_optim_args& a, double m_beta1, double v_beta2,
                            double m_wd, double v_wd, const float* const (&in)[4], float* out, int64_t n);
// in[] holds the kind's inputs in bg_optimizer_update order (unused slots NULL).
void launch_optimizer(bg_ctx* ctx, int kind, const bg_optim_args& a, const float* const (&in)[4], float* out,
                      int64_t n);
void launch_softmax_last(bg_ctx* ctx, const void* x, int x_dtype, void* y, int y_dtype,
                         int64_t rows, int64_t cols);
// Second pass of a split row reduction: out[r] = the BG_RED_* `op` over
// part[r * nch + 0 .. nch), combined in a fixed order (MEAN divides by cols).
void launch_reduce_partials(bg_ctx* ctx, const float* part, int64_t rows, int64_t nch, int op,
                            int64_t cols, void* out, int out_dtype);
// x[B][R][C] (f32, f16 or bf16, contiguous) reduced with BG_RED_* `op` over
// R into out[B][C] of dtype od (f32, f16 or bf16).
void launch_reduce_lead(bg_ctx* ctx, const void* x, int xd, int64_t B, int64_t R, int64_t C, int op, void* out,
                        int od);
// Extras of bg_matmul_ex2: operand storage dtypes converted in a pre-pass
// and an f32 residual added after the epilogue.
struct GemmExtra {
  const float* residual = nullptr;  // contiguous [batch][M][N] f32, or NULL
  int a_dtype = -1;                 // storage dtype of a (-1: d.in_dtype)
  int b_dtype = -1;                 // storage dtype of b (-1: d.in_dtype)
};
void launch_matmul(bg_ctx* ctx, const bg_matmul_desc& d, const Record& a,
                   const Record& b, const Record* bias, Record& out, const GemmExtra* ex = nullptr);
// Device scratch for one GEMM call's pre- and post-passes: the context's
// growable slots (fixed == NULL), or a fixed region of cap bytes handed out
// front to back (the no-allocation entry point).
struct GemmWorkspace {
  bg_ctx* ctx;
  char* fixed = nullptr;
  size_t cap = 0;
  size_t used = 0;
  void* get(size_t bytes, int slot);
};
// The GEMM on raw device pointers (a, b: operand storage, d.offset_a /
// d.offset_b applied inside; bias f32 [N] or NULL; c: the output with d.ldc /
// d.stride_c already resolved).
void run_matmul(bg_ctx* ctx, const bg_matmul_desc& d, const char* a, const char* b, const float* bias, void* c,
                GemmWorkspace& ws, const GemmExtra* ex = nullptr);
// Resolves this device's no-allocation scratch address (noalloc.hip); called
// by bg_ctx_create with the context's device current.
void noalloc_setup(bg_ctx* ctx);
void launch_attention(bg_ctx* ctx, const bg_attention_desc& d,
                      const Record& q, const Record& k, const Record& v,
                      Record& out);
// f32 attention on MFMA (k_attn32.hip), head dim 1..64: q/k/v/o point at the
// operands' first elements; mask is NULL or f32 with the given strides.
// Launch shape of the f32 GEMM (k_gemm.hip), shared with the launch-plan query.
struct Gemm32Shape {
  int tiles_m = 0, tiles_n = 0;
  bool aligned = false;
  bool wide = false;  // gemm32_wide_k_kernel: 32 x 32 blocks, K split over 16 wavefronts
};
Gemm32Shape gemm32_shape(const bg_matmul_desc& d, bool ptrs_aligned);
void plan_matmul(const bg_matmul_desc& d, bg_launch_plan& out);
void plan_attention(const bg_attention_desc& d, bg_launch_plan& out);
bool fa32_supported(const bg_attention_desc& d);
void launch_fa32(bg_ctx* ctx, const bg_attention_desc& d, const float* q, const float* k, const float* v,
                 const float* mask, int64_t m_sb, int64_t m_sh, int64_t m_ss, void* o);
void launch_attention_generic(bg_ctx* ctx, const bg_attention_desc& d, const void* q,
                              const void* k, const void* v, const float* mask, int64_t mask_sb,
                              int64_t mask_sh, void* o, bool two_pass);
void launch_attention_masked_f32(bg_ctx* ctx, const float* q, const float* k,
                                 const float* v, const float* mask,
                                 int64_t mask_b, int64_t mask_h, float* o,
                                 int64_t b, int64_t h, int64_t sq, int64_t sk,
                                 int64_t d, float scale);

// Plan executor (plan.cpp).
// requests_json: the semantic permutation side table (NULL for the legacy
// route); resident: the root must be an allocation of its own.
bg_handle run_plan(bg_ctx* ctx, const char* json, const char* requests_json, const int64_t* ids,
                   const bg_handle* handles, int n, int dtype, bool resident);
// Parse, validate and fuse a plan without running it (bg_plan_inspect).
std::string inspect_plan(const char* json, const char* requests_json);

}  // namespace bg

// Body of every C entry point: bg::Error -> its status and message in
// ctx->err; any other exception -> BG_E_INVALID.
#define BG_API_BEGIN \
  if (!ctx) return BG_E_INVALID; \
  try {
#define BG_API_END                          \
  }                                         \
  catch (const bg::Error& e) {              \
    ctx->err = e.what();                    \
    return e.code;                          \
  }                                         \
  catch (const std::exception& e) {         \
    ctx->err = std::string("HIP bridge: ") + e.what(); \
    return BG_E_INVALID;                    \
  }                                         \
  return BG_OK;

