// The GEMM for callers that cannot allocate device memory (code under HIP
// graph capture, serving loops that forbid hipMalloc): bg_matmul_noalloc runs
// the same kernels as bg_matmul_ex on caller-owned device pointers, and takes
// the scratch those kernels need (split-K partial sums, the re-laid-out B
// operand of x @ w, the f32 product awaiting a GELU pass) from one fixed,
// file-scope device array instead of the context's growable slots.
//
// The array holds kNoAllocScratchBytes per GPU for the life of the process.
// Its device address is resolved once per context (hence per device) when
// the context is created, with that device current, and kept in the
// context; host code never uses the array's name as an address.  Every call
// on one GPU shares the array and nothing in it needs to start at zero (each
// kernel writes the scratch it later reads), so calls that overlap on one
// GPU (two contexts' streams, or two host threads) race on it; calls on one
// context are ordered by its stream.
#include "core.h"

#include <string>

static constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;  // 16 MiB

// At file scope: host code below names it as ::scratch (inside namespace bg
// the bare name would find the host function bg::scratch).
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace bg {

void noalloc_setup(bg_ctx* ctx) {
  void* ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(::scratch));
  if (e != hipSuccess || ptr == nullptr) {
    (void)hipGetLastError();
    ctx->noalloc_scratch = nullptr;
    ctx->noalloc_scratch_bytes = 0;
    ctx->noalloc_error = e != hipSuccess ? hipGetErrorString(e) : "NULL address";
    return;
  }
  ctx->noalloc_scratch = static_cast<char*>(ptr);
  ctx->noalloc_scratch_bytes = kNoAllocScratchBytes;
}

}  // namespace bg

using namespace bg;

extern "C" {

int bg_matmul_noalloc(bg_ctx* ctx, const bg_matmul_desc* desc, const void* a, const void* b, const float* bias,
                      void* c) {
  BG_API_BEGIN
  if (!desc) fail(BG_E_INVALID, "matmul_noalloc: desc is NULL");
  if (!a || !b || !c) fail(BG_E_INVALID, "matmul_noalloc: a, b and c must be device pointers");
  const bg_matmul_desc& d = *desc;
  if (d.a || d.b || d.bias)
    fail(BG_E_INVALID, "matmul_noalloc: operands are passed as pointers; desc.a, desc.b and desc.bias must be 0");
  if (d.m <= 0 || d.n <= 0 || d.k <= 0 || d.batch <= 0)
    fail(BG_E_INVALID, "matmul: batch, m, k, n must be positive integers");
  if (d.in_dtype != BG_F32 && d.in_dtype != BG_F16 && d.in_dtype != BG_BF16)
    fail(BG_E_DTYPE, std::string("matmul: dtype ") + dtype_name(d.in_dtype) + " not supported");
  if (d.out_dtype != BG_F32 && d.out_dtype != BG_F16 && d.out_dtype != BG_BF16)
    fail(BG_E_DTYPE, "matmul: output dtype not supported");
  if (d.stride_a < 0 || d.stride_b < 0 || d.stride_c < 0 || d.offset_a < 0 || d.offset_b < 0 || d.lda < 0 ||
      d.ldb < 0 || d.ldc < 0)
    fail(BG_E_INVALID, "matmul: negative stride/offset");
  if (d.lda < d.k) fail(BG_E_SHAPE, "matmul: lda < k");
  if (d.trans_b ? d.ldb < d.k : d.ldb < d.n) fail(BG_E_SHAPE, d.trans_b ? "matmul: ldb < k" : "matmul: ldb < n");
  bg_matmul_desc dd = d;
  if (dd.ldc == 0) dd.ldc = d.n;
  if (dd.stride_c == 0) dd.stride_c = d.m * dd.ldc;
  if (dd.ldc < d.n) fail(BG_E_SHAPE, "matmul: ldc < n");
  if (d.batch > 1 && dd.stride_c < (d.m - 1) * dd.ldc + d.n)
    fail(BG_E_SHAPE, "matmul: stride_c makes the output matrices of the batch overlap");
  if (!ctx->noalloc_scratch)
    fail(BG_E_HIP, "matmul_noalloc: the device's fixed scratch address could not be resolved (" +
                       ctx->noalloc_error + ")");
  GemmWorkspace ws{ctx};
  ws.fixed = ctx->noalloc_scratch;
  ws.cap = ctx->noalloc_scratch_bytes;
  // Profiling events come from a pool that may create new ones: no
  // profiling inside this call.
  const bool profiling = ctx->profiling;
  ctx->profiling = false;
  try {
    run_matmul(ctx, dd, static_cast<const char*>(a), static_cast<const char*>(b), bias, c, ws);
  } catch (...) {
    ctx->profiling = profiling;
    throw;
  }
  ctx->profiling = profiling;
  BG_API_END
}

}  // extern "C"
