// libbghip core: context, handle table, block cache, profiling and the C ABI
// entry points of the bridge (include/bghip.h).
//
// Handle semantics follow createWebGpuRealizerBridge
// (packages/browsergrad-kernels/src/realizer.ts:902-1005): ids minted from 1,
// unknown handles raise an op-qualified error, release is idempotent, and the
// owned-bytes counters are kept per device allocation.
#include "core.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <sstream>

namespace bg {

void fail(int code, const std::string& msg) { throw Error(code, msg); }

void hip_check(hipError_t e, const char* what) {
  if (e == hipSuccess) return;
  const char* s = hipGetErrorString(e);
  if (e == hipErrorOutOfMemory)
    fail(BG_E_OOM, std::string("HIP bridge: ") + what + ": out of device memory");
  fail(BG_E_HIP, std::string("HIP bridge: ") + what + ": " + (s ? s : "hip error"));
}

int64_t dtype_size(int dtype) {
  switch (dtype) {
    case BG_F32: return 4;
    case BG_F16: return 2;
    case BG_BF16: return 2;
    case BG_BOOL: return 1;
    case BG_I32: return 4;
    case BG_I64: return 8;
    case BG_U8: return 1;
    case BG_F64: return 8;
    default: return -1;
  }
}

const char* dtype_name(int dtype) {
  switch (dtype) {
    case BG_F32: return "float32";
    case BG_F16: return "float16";
    case BG_BF16: return "bfloat16";
    case BG_BOOL: return "bool";
    case BG_I32: return "int32";
    case BG_I64: return "int64";
    case BG_U8: return "uint8";
    case BG_F64: return "float64";
    default: return "unknown";
  }
}

std::vector<int64_t> to_shape(const int64_t* shape, int rank) {
  if (rank < 0 || rank > BG_MAX_RANK)
    fail(BG_E_INVALID, "HIP bridge: rank " + std::to_string(rank) + " outside [0, 8]");
  if (rank > 0 && shape == nullptr) fail(BG_E_INVALID, "HIP bridge: shape is NULL");
  std::vector<int64_t> s(shape, shape + rank);
  for (int64_t d : s)
    if (d < 0) fail(BG_E_SHAPE, "HIP bridge: negative dimension in shape");
  return s;
}

int64_t numel(const std::vector<int64_t>& shape) {
  int64_t n = 1;
  for (int64_t d : shape) n *= d;
  return n;
}

// Pool block size: small blocks round to 512 B, large ones to 2 MiB so that
// repeated requests of one tensor size reuse the same block.
static size_t pooled_size(size_t bytes) {
  if (bytes == 0) bytes = 1;
  if (bytes <= (1u << 20)) return (bytes + 511) & ~size_t(511);
  const size_t g = size_t(2) << 20;
  return (bytes + g - 1) / g * g;
}

static const int64_t kMaxCachedBytes = int64_t(32) << 30;

static void* pool_alloc(bg_ctx* ctx, size_t cap) {
  auto it = ctx->free_blocks.find(cap);
  if (it != ctx->free_blocks.end()) {
    void* p = it->second;
    ctx->free_blocks.erase(it);
    ctx->cached_bytes -= int64_t(cap);
    ctx->pool_hits++;
    return p;
  }
  ctx->pool_misses++;
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, cap);
  if (e == hipErrorOutOfMemory) {
    // Drop the cache and retry once.
    (void)hipGetLastError();
    hip_check(hipStreamSynchronize(ctx->stream), "synchronize before cache flush");
    for (auto& kv : ctx->free_blocks) (void)hipFree(kv.second);
    ctx->free_blocks.clear();
    ctx->cached_bytes = 0;
    e = hipMalloc(&p, cap);
  }
  hip_check(e, "hipMalloc");
  return p;
}

static void pool_free(bg_ctx* ctx, void* p, size_t cap) {
  if (ctx->cached_bytes + int64_t(cap) > kMaxCachedBytes) {
    // Blocks may still be read by queued kernels: synchronise before freeing.
    hip_check(hipStreamSynchronize(ctx->stream), "synchronize before free");
    hip_check(hipFree(p), "hipFree");
    return;
  }
  // Stream order guarantees later users of the block run after earlier ones.
  ctx->free_blocks.emplace(cap, p);
  ctx->cached_bytes += int64_t(cap);
}

Record& get(bg_ctx* ctx, bg_handle h, const char* op) {
  auto it = ctx->handles.find(h);
  if (it == ctx->handles.end()) {
    std::ostringstream os;
    os << "HIP bridge: " << op << " called with unknown handle " << h
       << ". It may have been released already.";
    fail(BG_E_HANDLE, os.str());
  }
  return it->second;
}

bg_handle mint(bg_ctx* ctx, size_t nbytes, const std::vector<int64_t>& shape,
               int dtype) {
  size_t cap = pooled_size(nbytes);
  Alloc* a = new Alloc();
  a->ptr = pool_alloc(ctx, cap);
  a->bytes = nbytes;
  a->cap = cap;
  a->refs = 1;
  ctx->current_owned += int64_t(nbytes);
  ctx->total_allocated += int64_t(nbytes);
  ctx->peak_owned = std::max(ctx->peak_owned, ctx->current_owned);
  Record r;
  r.alloc = a;
  r.offset = 0;
  r.nbytes = int64_t(nbytes);
  r.shape = shape;
  r.dtype = dtype;
  bg_handle id = ctx->next_id++;
  ctx->handles.emplace(id, std::move(r));
  return id;
}

bg_handle mint_view(bg_ctx* ctx, const Record& src, int64_t offset,
                    int64_t nbytes, const std::vector<int64_t>& shape,
                    int dtype) {
  if (offset < 0 || offset + nbytes > int64_t(src.alloc->bytes))
    fail(BG_E_SHAPE, "HIP bridge: view exceeds its allocation");
  Record r;
  r.alloc = src.alloc;
  r.alloc->refs++;
  r.offset = offset;
  r.nbytes = nbytes;
  r.shape = shape;
  r.dtype = dtype;
  bg_handle id = ctx->next_id++;
  ctx->handles.emplace(id, std::move(r));
  return id;
}

static void drop(bg_ctx* ctx, Record& r) {
  Alloc* a = r.alloc;
  if (--a->refs == 0) {
    ctx->current_owned = std::max<int64_t>(0, ctx->current_owned - int64_t(a->bytes));
    ctx->total_released += int64_t(a->bytes);
    pool_free(ctx, a->ptr, a->cap);
    delete a;
  }
  r.alloc = nullptr;
}

void log_launch(bg_ctx* ctx, const void* kernel, dim3 grid, dim3 block, size_t shmem) {
  bg_launch_record r{};
  const char* name = hipKernelNameRefByPtr(kernel, ctx->stream);
  std::snprintf(r.kernel, sizeof(r.kernel), "%s", name ? name : "?");
  r.grid[0] = grid.x;
  r.grid[1] = grid.y;
  r.grid[2] = grid.z;
  r.block[0] = int32_t(block.x);
  r.block[1] = int32_t(block.y);
  r.block[2] = int32_t(block.z);
  r.dynamic_lds = int64_t(shmem);
  hipFuncAttributes fa{};
  if (hipFuncGetAttributes(&fa, kernel) == hipSuccess) {
    r.static_lds = int64_t(fa.sharedSizeBytes);
    r.vgprs = int32_t(fa.numRegs);
    r.scratch = int32_t(fa.localSizeBytes);
    r.max_threads = int32_t(fa.maxThreadsPerBlock);
  } else {
    (void)hipGetLastError();
  }
  ctx->launch_log.push_back(r);
}

void* scratch(bg_ctx* ctx, size_t bytes, int slot) {
  if (bytes <= ctx->scratch_bytes[slot]) return ctx->scratch[slot];
  if (ctx->scratch[slot]) {
    hip_check(hipStreamSynchronize(ctx->stream), "synchronize before scratch grow");
    hip_check(hipFree(ctx->scratch[slot]), "hipFree(scratch)");
    ctx->scratch[slot] = nullptr;
    ctx->scratch_bytes[slot] = 0;
  }
  size_t cap = pooled_size(bytes);
  hip_check(hipMalloc(&ctx->scratch[slot], cap), "hipMalloc(scratch)");
  ctx->scratch_bytes[slot] = cap;
  return ctx->scratch[slot];
}

static hipEvent_t take_event(bg_ctx* ctx) {
  if (!ctx->event_pool.empty()) {
    hipEvent_t e = ctx->event_pool.back();
    ctx->event_pool.pop_back();
    return e;
  }
  hipEvent_t e;
  hip_check(hipEventCreate(&e), "hipEventCreate");
  return e;
}

Profile::Profile(bg_ctx* c, const char* label, int64_t bytes, int64_t flops)
    : ctx(c), on(c->profiling) {
  if (!on) return;
  std::memset(&p.info, 0, sizeof(p.info));
  std::snprintf(p.info.label, sizeof(p.info.label), "%s", label);
  p.info.bytes = bytes;
  p.info.flops = flops;
  p.start = take_event(ctx);
  p.stop = take_event(ctx);
  prev = ctx->active_profile;
  ctx->active_profile = this;
}

Profile::~Profile() {
  if (!on) return;
  ctx->active_profile = prev;
  if (launches == 0) {
    // Nothing was dispatched (e.g. an empty tensor): no timing to report.
    ctx->event_pool.push_back(p.start);
    ctx->event_pool.push_back(p.stop);
    return;
  }
  if (launches > 1 && hipEventRecord(p.stop, ctx->stream) != hipSuccess) return;
  ctx->pending.push_back(p);
}

void next_dispatch_events(bg_ctx* ctx, hipEvent_t* start, hipEvent_t* stop) {
  *start = nullptr;
  *stop = nullptr;
  Profile* pr = ctx->active_profile;
  if (!pr || !pr->on) return;
  if (pr->launches++ == 0) {
    *start = pr->p.start;
    *stop = pr->p.stop;
  }
}

static void resolve_profiles(bg_ctx* ctx) {
  for (auto& p : ctx->pending) {
    hip_check(hipEventSynchronize(p.stop), "hipEventSynchronize");
    float ms = 0.f;
    hip_check(hipEventElapsedTime(&ms, p.start, p.stop), "hipEventElapsedTime");
    p.info.gpu_ms = ms;
    ctx->done.push_back(p.info);
    ctx->event_pool.push_back(p.start);
    ctx->event_pool.push_back(p.stop);
  }
  ctx->pending.clear();
}

}  // namespace bg

using namespace bg;

// Context-free entries: the refusal message goes to err.
template <class F>
static int no_ctx_call(char* err, size_t err_cap, F&& f) {
  std::string text;
  int rc = BG_OK;
  try {
    f();
  } catch (const bg::Error& e) {
    rc = e.code;
    text = e.what();
  } catch (const std::exception& e) {
    rc = BG_E_INVALID;
    text = e.what();
  }
  if (err && err_cap > 0) {
    const size_t n = std::min(err_cap - 1, text.size());
    std::memcpy(err, text.data(), n);
    err[n] = 0;
  }
  return rc;
}

extern "C" {

const char* bg_version(void) { return "bghip 0.1 gfx950"; }

int bg_dtype_from_name(const char* name) {
  if (!name) return -1;
  std::string s(name);
  if (s == "float32" || s == "f32") return BG_F32;
  if (s == "float16" || s == "f16") return BG_F16;
  if (s == "bfloat16" || s == "bf16") return BG_BF16;
  if (s == "bool") return BG_BOOL;
  if (s == "int32") return BG_I32;
  if (s == "int64") return BG_I64;
  if (s == "uint8") return BG_U8;
  if (s == "float64") return BG_F64;
  return -1;
}

int64_t bg_dtype_size(int dtype) { return dtype_size(dtype); }

int bg_ctx_create(int device, int profiling, bg_ctx** out) {
  if (!out) return BG_E_INVALID;
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return BG_E_HIP;
  if (device < 0 || device >= n) return BG_E_INVALID;
  if (hipSetDevice(device) != hipSuccess) return BG_E_HIP;
  bg_ctx* ctx = new bg_ctx();
  ctx->device = device;
  ctx->profiling = profiling != 0;
  // Default-priority, non-blocking stream.
  if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) {
    delete ctx;
    return BG_E_HIP;
  }
  noalloc_setup(ctx);
  *out = ctx;
  return BG_OK;
}

int bg_ctx_destroy(bg_ctx* ctx) {
  if (!ctx) return BG_OK;
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  for (auto& kv : ctx->handles) {
    Alloc* a = kv.second.alloc;
    if (a && --a->refs == 0) {
      (void)hipFree(a->ptr);
      delete a;
    }
  }
  ctx->handles.clear();
  for (auto& kv : ctx->free_blocks) (void)hipFree(kv.second);
  for (auto& p : ctx->pending) {
    (void)hipEventDestroy(p.start);
    (void)hipEventDestroy(p.stop);
  }
  for (auto e : ctx->event_pool) (void)hipEventDestroy(e);
  for (void* sp : ctx->scratch)
    if (sp) (void)hipFree(sp);
  (void)hipStreamDestroy(ctx->stream);
  delete ctx;
  return BG_OK;
}

const char* bg_last_error(const bg_ctx* ctx) {
  if (!ctx) return "HIP bridge: null context";
  return ctx->err.c_str();
}

int bg_synchronize(bg_ctx* ctx) {
  BG_API_BEGIN
  hip_check(hipStreamSynchronize(ctx->stream), "synchronize");
  BG_API_END
}

int bg_upload(bg_ctx* ctx, const void* data, size_t nbytes,
              const int64_t* shape, int rank, int dtype, bg_handle* out) {
  BG_API_BEGIN
  if (!out) fail(BG_E_INVALID, "HIP bridge: upload: out is NULL");
  int64_t es = dtype_size(dtype);
  if (es < 0) fail(BG_E_DTYPE, "HIP bridge: upload: unknown dtype");
  auto s = to_shape(shape, rank);
  int64_t n = numel(s);
  if (int64_t(nbytes) != n * es) {
    std::ostringstream os;
    os << "HIP bridge: upload: " << nbytes << " bytes do not match shape of "
       << n << " " << dtype_name(dtype) << " elements";
    fail(BG_E_SHAPE, os.str());
  }
  if (nbytes > 0 && !data) fail(BG_E_INVALID, "HIP bridge: upload: data is NULL");
  bg_handle h = mint(ctx, nbytes, s, dtype);
  Record& r = ctx->handles[h];
  if (nbytes > 0) {
    hip_check(hipMemcpyAsync(r.ptr(), data, nbytes, hipMemcpyHostToDevice, ctx->stream),
              "upload");
    // The host buffer may be reused by the caller as soon as we return.
    hip_check(hipStreamSynchronize(ctx->stream), "upload");
  }
  *out = h;
  BG_API_END
}

int bg_materialize(bg_ctx* ctx, bg_handle h, void* dst, size_t nbytes) {
  BG_API_BEGIN
  Record& r = get(ctx, h, "materialize");
  if (int64_t(nbytes) != r.nbytes) {
    std::ostringstream os;
    os << "HIP bridge: materialize: destination holds " << nbytes
       << " bytes, handle " << h << " holds " << r.nbytes;
    fail(BG_E_SHAPE, os.str());
  }
  if (nbytes > 0) {
    hip_check(hipMemcpyAsync(dst, r.ptr(), nbytes, hipMemcpyDeviceToHost, ctx->stream),
              "materialize");
  }
  hip_check(hipStreamSynchronize(ctx->stream), "materialize");
  BG_API_END
}

int bg_release(bg_ctx* ctx, bg_handle h) {
  BG_API_BEGIN
  auto it = ctx->handles.find(h);
  if (it == ctx->handles.end()) return BG_OK;  // idempotent
  drop(ctx, it->second);
  ctx->handles.erase(it);
  BG_API_END
}

int bg_handle_info(bg_ctx* ctx, bg_handle h, int64_t* shape_out, int* rank,
                   int* dtype, int64_t* nbytes) {
  BG_API_BEGIN
  Record& r = get(ctx, h, "handle_info");
  // Callers size shape_out for BG_MAX_RANK entries; every entry point that
  // sets a record's shape keeps it within that, and this guard keeps a
  // violation from ever writing past the caller's array.
  if (r.shape.size() > BG_MAX_RANK)
    fail(BG_E_SHAPE, "handle_info: handle has rank " + std::to_string(r.shape.size()) + ", above " +
                         std::to_string(BG_MAX_RANK));
  if (shape_out)
    for (size_t i = 0; i < r.shape.size(); ++i) shape_out[i] = r.shape[i];
  if (rank) *rank = int(r.shape.size());
  if (dtype) *dtype = r.dtype;
  if (nbytes) *nbytes = r.nbytes;
  BG_API_END
}

int bg_alive_handles(bg_ctx* ctx, int64_t* out) {
  BG_API_BEGIN
  if (out) *out = int64_t(ctx->handles.size());
  BG_API_END
}

int bg_resource_snapshot(bg_ctx* ctx, bg_snapshot* out) {
  BG_API_BEGIN
  if (!out) fail(BG_E_INVALID, "HIP bridge: resource_snapshot: out is NULL");
  std::memset(out, 0, sizeof(*out));
  out->current_owned_bytes = ctx->current_owned;
  out->peak_owned_bytes = ctx->peak_owned;
  out->total_allocated_bytes = ctx->total_allocated;
  out->total_released_bytes = ctx->total_released;
  out->alive_handle_count = int64_t(ctx->handles.size());
  out->pending_profile_count = int64_t(ctx->pending.size());
  out->pass_profile_count = int64_t(ctx->done.size());
  out->pool_cached_bytes = ctx->cached_bytes;
  out->pool_hits = ctx->pool_hits;
  out->pool_misses = ctx->pool_misses;
  out->timing_mode = (ctx->profiling && (!ctx->done.empty() || !ctx->pending.empty())) ? 1 : 0;
  out->timestamp_query_available = 1;
  BG_API_END
}

int bg_flush_profiles(bg_ctx* ctx, bg_pass_profile* out, int cap, int* n_out) {
  BG_API_BEGIN
  hip_check(hipStreamSynchronize(ctx->stream), "flush_profiles");
  resolve_profiles(ctx);
  int n = 0;
  if (out && cap > 0) {
    n = std::min<int>(cap, int(ctx->done.size()));
    std::memcpy(out, ctx->done.data(), sizeof(bg_pass_profile) * size_t(n));
  }
  if (n_out) *n_out = int(ctx->done.size());
  BG_API_END
}

int bg_set_profiling(bg_ctx* ctx, int on) {
  BG_API_BEGIN
  ctx->profiling = on != 0;
  BG_API_END
}

int bg_device_ptr(bg_ctx* ctx, bg_handle h, void** ptr) {
  BG_API_BEGIN
  Record& r = get(ctx, h, "device_ptr");
  if (ptr) *ptr = r.ptr();
  BG_API_END
}

int bg_stream(bg_ctx* ctx, void** stream) {
  BG_API_BEGIN
  if (stream) *stream = reinterpret_cast<void*>(ctx->stream);
  BG_API_END
}

// ---- compute entry points ------------------------------------------------

int bg_fused_elementwise(bg_ctx* ctx, const bg_handle* inputs, int n_inputs,
                         const bg_fused_op* ops, int n_ops,
                         const int64_t* shape, int rank, int dtype,
                         bg_handle* out) {
  BG_API_BEGIN
  // Reference refusal ranges (fused_elementwise.ts:97-110) and opcode set
  // (fused_elementwise.ts:83-90).
  if (n_inputs < 1 || n_inputs > BG_FUSED_MAX_INPUTS)
    fail(BG_E_INVALID, "fused_elementwise: numInputs=" + std::to_string(n_inputs) +
                           " outside supported range [1, 8]");
  if (n_ops < 1 || n_ops > BG_FUSED_MAX_OPS)
    fail(BG_E_INVALID, "fused_elementwise: ops.length=" + std::to_string(n_ops) +
                           " outside supported range [1, 32]");
  for (int i = 0; i < n_ops; ++i)
    if (ops[i].code < BG_OP_ADD || ops[i].code > BG_OP_LOG)
      fail(BG_E_UNSUPPORTED, "fused_elementwise: unsupported opcode " +
                                 std::to_string(ops[i].code));
  bg_fused_desc d{};
  d.n_inputs = n_inputs;
  d.inputs = inputs;
  d.in_strides = nullptr;
  d.n_ops = n_ops;
  d.ops = ops;
  d.rank = rank;
  d.shape = shape;
  d.out_dtype = dtype;
  d.reduce_op = BG_RED_NONE;
  // The reference kernel reads in[i] for i < N with N = numel(shape): every
  // input must hold exactly numel elements (fused_elementwise.ts:23-38).
  auto s = to_shape(shape, rank);
  int64_t n = numel(s);
  for (int i = 0; i < n_inputs; ++i) {
    Record& r = get(ctx, inputs[i], "fused_elementwise[in]");
    if (r.numel() != n)
      fail(BG_E_SHAPE, "fused_elementwise: input " + std::to_string(i) + " has " +
                           std::to_string(r.numel()) + " elements, expected " +
                           std::to_string(n));
  }
  int64_t es = dtype_size(dtype);
  if (dtype != BG_F32 && dtype != BG_F16 && dtype != BG_BF16)
    fail(BG_E_DTYPE, std::string("fused_elementwise: dtype ") + dtype_name(dtype) +
                         " not supported");
  bg_handle h = mint(ctx, size_t(n * es), s, dtype);
  launch_fused(ctx, d, ctx->handles[h]);
  *out = h;
  BG_API_END
}

int bg_fused_ex(bg_ctx* ctx, const bg_fused_desc* desc, bg_handle* out) {
  BG_API_BEGIN
  if (!desc || !out) fail(BG_E_INVALID, "fused_ex: NULL argument");
  const bg_fused_desc& d = *desc;
  if (d.n_inputs < 0 || d.n_inputs > BG_FUSED_MAX_INPUTS)
    fail(BG_E_INVALID, "fused_ex: numInputs=" + std::to_string(d.n_inputs) +
                           " outside supported range [0, 8]");
  if (d.n_ops < 1 || d.n_ops > BG_FUSED_MAX_OPS)
    fail(BG_E_INVALID, "fused_ex: ops.length=" + std::to_string(d.n_ops) +
                           " outside supported range [1, 32]");
  if (d.n_imms < 0 || d.n_imms > BG_FUSED_MAX_IMMS)
    fail(BG_E_INVALID, "fused_ex: too many immediates");
  auto s = to_shape(d.shape, d.rank);
  std::vector<int64_t> os = s;
  if (d.reduce_op != BG_RED_NONE) {
    if (s.empty()) fail(BG_E_SHAPE, "fused_ex: reduction needs rank >= 1");
    if (d.reduce_keepdims) os.back() = 1;
    else os.pop_back();
  }
  int64_t es = dtype_size(d.out_dtype);
  if (d.out_dtype != BG_F32 && d.out_dtype != BG_F16 && d.out_dtype != BG_BF16 &&
      d.out_dtype != BG_BOOL)
    fail(BG_E_DTYPE, std::string("fused_ex: output dtype ") + dtype_name(d.out_dtype) +
                         " not supported");
  bg_handle h = mint(ctx, size_t(numel(os) * es), os, d.out_dtype);
  try {
    launch_fused(ctx, d, ctx->handles[h]);
  } catch (...) {
    bg_release(ctx, h);
    throw;
  }
  *out = h;
  BG_API_END
}

int bg_cast(bg_ctx* ctx, bg_handle h, int src_dtype, int dst_dtype,
            const int64_t* shape, int rank, bg_handle* out) {
  BG_API_BEGIN
  Record& r = get(ctx, h, "cast");
  auto s = to_shape(shape, rank);
  int64_t n = numel(s);
  if (r.dtype != src_dtype)
    fail(BG_E_DTYPE, std::string("cast: handle holds ") + dtype_name(r.dtype) +
                         ", srcDtype is " + dtype_name(src_dtype));
  if (n != r.numel()) fail(BG_E_SHAPE, "cast: shape does not match the handle");
  auto ok = [](int t) { return t == BG_F32 || t == BG_F16 || t == BG_BF16; };
  if (!ok(src_dtype) || !ok(dst_dtype))
    fail(BG_E_DTYPE, std::string("cast ") + dtype_name(src_dtype) + "->" +
                         dtype_name(dst_dtype) + " not supported");
  bg_handle o = mint(ctx, size_t(n * dtype_size(dst_dtype)), s, dst_dtype);
  Record& ro = ctx->handles[o];
  Record& rs = ctx->handles[h];
  {
    Profile prof(ctx, "cast", n * (dtype_size(src_dtype) + dtype_size(dst_dtype)), 0);
    if (src_dtype == dst_dtype) {
      if (n > 0)
        hip_check(hipMemcpyAsync(ro.ptr(), rs.ptr(), size_t(rs.nbytes),
                                 hipMemcpyDeviceToDevice, ctx->stream),
                  "cast copy");
    } else {
      launch_cast(ctx, rs.ptr(), src_dtype, ro.ptr(), dst_dtype, n);
    }
  }
  *out = o;
  BG_API_END
}

int bg_copy_strided(bg_ctx* ctx, bg_handle src, int64_t offset,
                    const int64_t* shape, const int64_t* strides, int rank,
                    bg_handle* out) {
  BG_API_BEGIN
  Record& r = get(ctx, src, "copy_strided");
  auto s = to_shape(shape, rank);
  std::vector<int64_t> st(strides, strides + rank);
  int64_t n = numel(s);
  // Bounds: the largest reachable element must lie inside the source.
  if (n > 0) {
    int64_t lo = offset, hi = offset;
    for (int i = 0; i < rank; ++i) {
      int64_t span = (s[i] - 1) * st[i];
      if (span > 0) hi += span; else lo += span;
    }
    if (lo < 0 || hi >= r.numel())
      fail(BG_E_SHAPE, "copy_strided: view reaches outside the source tensor");
  }
  int64_t es = dtype_size(r.dtype);
  bg_handle o = mint(ctx, size_t(n * es), s, r.dtype);
  Record& ro = ctx->handles[o];
  Record& rs = ctx->handles[src];
  if (n > 0) {
    Profile prof(ctx, "copy_strided", 2 * n * es, 0);
    launch_copy_strided(ctx, rs.ptr() + offset * es, es, ro.ptr(), s, st);
  }
  *out = o;
  BG_API_END
}

int bg_reshape(bg_ctx* ctx, bg_handle h, const int64_t* shape, int rank,
               bg_handle* out) {
  BG_API_BEGIN
  Record& r = get(ctx, h, "reshape");
  auto s = to_shape(shape, rank);
  if (numel(s) != r.numel())
    fail(BG_E_SHAPE, "reshape: element count changes");
  Record copy = r;
  *out = mint_view(ctx, copy, r.offset, r.nbytes, s, r.dtype);
  BG_API_END
}

int bg_layer_norm(bg_ctx* ctx, bg_handle x, bg_handle weight, bg_handle bias,
                  int64_t rows, int64_t cols, float eps, int out_dtype,
                  bg_handle* out) {
  BG_API_BEGIN
  Record& rx = get(ctx, x, "layer_norm[x]");
  Record& rw = get(ctx, weight, "layer_norm[weight]");
  Record& rb = get(ctx, bias, "layer_norm[bias]");
  if (rows < 0 || cols <= 0 || rows * cols != rx.numel())
    fail(BG_E_SHAPE, "layer_norm: rows*cols does not match x");
  if (rw.numel() != cols || rb.numel() != cols || rw.dtype != BG_F32 || rb.dtype != BG_F32)
    fail(BG_E_SHAPE, "layer_norm: weight/bias must be float32 [cols]");
  if (rx.dtype != BG_F32 && rx.dtype != BG_F16 && rx.dtype != BG_BF16)
    fail(BG_E_DTYPE, "layer_norm: x dtype not supported");
  if (out_dtype != BG_F32 && out_dtype != BG_F16 && out_dtype != BG_BF16)
    fail(BG_E_DTYPE, "layer_norm: out dtype not supported");
  bg_handle o = mint(ctx, size_t(rows * cols * dtype_size(out_dtype)), rx.shape, out_dtype);
  Record& ro = ctx->handles[o];
  Record& rx2 = ctx->handles[x];
  Record& rw2 = ctx->handles[weight];
  Record& rb2 = ctx->handles[bias];
  {
    Profile prof(ctx, "layer_norm",
                 rows * cols * (dtype_size(rx2.dtype) + dtype_size(out_dtype)), 0);
    launch_layer_norm(ctx, rx2.ptr(), rx2.dtype, reinterpret_cast<float*>(rw2.ptr()),
                      reinterpret_cast<float*>(rb2.ptr()), ro.ptr(), out_dtype, rows,
                      cols, eps);
  }
  *out = o;
  BG_API_END
}

// Shared checks of the LayerNorm backward entry points: an f32 handle of
// exactly `want` elements.
static Record& ln_bwd_operand(bg_ctx* ctx, bg_handle h, int64_t want, const char* what) {
  Record& r = get(ctx, h, what);
  if (r.dtype != BG_F32) fail(BG_E_DTYPE, std::string(what) + " must be float32");
  if (r.numel() != want) fail(BG_E_SHAPE, std::string(what) + " does not hold rows*cols (or cols) elements");
  return r;
}

static void ln_bwd_dims(int64_t rows, int64_t cols, float eps, const char* op) {
  if (rows <= 0 || cols <= 0) fail(BG_E_INVALID, std::string(op) + ": rows and cols must be positive");
  if (!(eps > 0.f) || !std::isfinite(eps)) fail(BG_E_INVALID, std::string(op) + ": eps must be finite and > 0");
}

int bg_layer_norm_backward_input(bg_ctx* ctx, bg_handle dy, bg_handle x, bg_handle weight, int64_t rows,
                                 int64_t cols, float eps, bg_handle* out) {
  BG_API_BEGIN
  ln_bwd_dims(rows, cols, eps, "layer_norm_backward_input");
  ln_bwd_operand(ctx, dy, rows * cols, "layer_norm_backward_input[dy]");
  const std::vector<int64_t> shape = ln_bwd_operand(ctx, x, rows * cols, "layer_norm_backward_input[x]").shape;
  ln_bwd_operand(ctx, weight, cols, "layer_norm_backward_input[weight]");
  bg_handle o = mint(ctx, size_t(rows * cols * 4), shape, BG_F32);
  const float* pdy = reinterpret_cast<const float*>(ctx->handles[dy].ptr());
  const float* px = reinterpret_cast<const float*>(ctx->handles[x].ptr());
  const float* pw = reinterpret_cast<const float*>(ctx->handles[weight].ptr());
  float* po = reinterpret_cast<float*>(ctx->handles[o].ptr());
  {
    Profile prof(ctx, "layer_norm_backward_input", rows * cols * 12 + cols * 4, 0);
    launch_ln_backward_input(ctx, pdy, px, pw, po, rows, cols, eps);
  }
  *out = o;
  BG_API_END
}

int bg_layer_norm_backward_weight(bg_ctx* ctx, bg_handle dy, bg_handle x, int64_t rows, int64_t cols, float eps,
                                  bg_handle* out) {
  BG_API_BEGIN
  ln_bwd_dims(rows, cols, eps, "layer_norm_backward_weight");
  ln_bwd_operand(ctx, dy, rows * cols, "layer_norm_backward_weight[dy]");
  ln_bwd_operand(ctx, x, rows * cols, "layer_norm_backward_weight[x]");
  bg_handle o = mint(ctx, size_t(cols * 4), {cols}, BG_F32);
  const float* pdy = reinterpret_cast<const float*>(ctx->handles[dy].ptr());
  const float* px = reinterpret_cast<const float*>(ctx->handles[x].ptr());
  float* po = reinterpret_cast<float*>(ctx->handles[o].ptr());
  {
    Profile prof(ctx, "layer_norm_backward_weight", rows * cols * 8 + cols * 4, 0);
    launch_ln_backward_cols(ctx, pdy, px, po, rows, cols, eps, true);
  }
  *out = o;
  BG_API_END
}

int bg_layer_norm_backward_bias(bg_ctx* ctx, bg_handle dy, int64_t rows, int64_t cols, bg_handle* out) {
  BG_API_BEGIN
  ln_bwd_dims(rows, cols, 1.f, "layer_norm_backward_bias");
  ln_bwd_operand(ctx, dy, rows * cols, "layer_norm_backward_bias[dy]");
  bg_handle o = mint(ctx, size_t(cols * 4), {cols}, BG_F32);
  const float* pdy = reinterpret_cast<const float*>(ctx->handles[dy].ptr());
  float* po = reinterpret_cast<float*>(ctx->handles[o].ptr());
  {
    Profile prof(ctx, "layer_norm_backward_bias", rows * cols * 4 + cols * 4, 0);
    launch_ln_backward_cols(ctx, pdy, nullptr, po, rows, cols, 0.f, false);
  }
  *out = o;
  BG_API_END
}

int bg_optimizer_update(bg_ctx* ctx, int kind, const bg_handle* inputs, int n_inputs, const bg_optim_args* args,
                        int64_t n, bg_handle* out) {
  BG_API_BEGIN
  static const int arity[] = {2, 2, 2, 4, 3, 3, 3};
  static const char* names[] = {"sgd_update",    "adamw_update_m", "adamw_update_v", "adamw_update_param",
                                "adam_update_m", "adam_update_v",  "adam_update_param"};
  if (kind < BG_OPT_SGD || kind > BG_OPT_ADAM_PARAM) fail(BG_E_INVALID, "optimizer_update: unknown kind");
  const std::string op = names[kind];
  if (!args || !out) fail(BG_E_INVALID, op + ": args and out must be non-NULL");
  if (n_inputs != arity[kind] || !inputs)
    fail(BG_E_INVALID, op + ": expects " + std::to_string(arity[kind]) + " inputs");
  if (n < 0) fail(BG_E_INVALID, op + ": n must be >= 0");
  const bg_optim_args& a = *args;
  for (double v : {a.lr, a.beta1, a.beta2, a.eps, a.weight_decay})
    if (!std::isfinite(v)) fail(BG_E_INVALID, op + ": arguments must be finite");
  if (a.lr < 0) fail(BG_E_INVALID, op + ": lr must be >= 0");
  if (kind != BG_OPT_SGD && a.step < 1) fail(BG_E_INVALID, op + ": step must be >= 1");
  std::vector<int64_t> shape;
  for (int i = 0; i < n_inputs; ++i) {
    Record& r = get(ctx, inputs[i], op.c_str());
    if (r.dtype != BG_F32) fail(BG_E_DTYPE, op + ": inputs must be float32");
    if (r.numel() != n) fail(BG_E_SHAPE, op + ": input " + std::to_string(i) + " does not hold n elements");
    if (i == 0) shape = r.shape;
  }
  bg_handle o = mint(ctx, size_t(n * 4), shape, BG_F32);
  const float* in[4] = {nullptr, nullptr, nullptr, nullptr};
  for (int i = 0; i < n_inputs; ++i) in[i] = reinterpret_cast<const float*>(ctx->handles[inputs[i]].ptr());
  float* po = reinterpret_cast<float*>(ctx->handles[o].ptr());
  {
    Profile prof(ctx, names[kind], n * 4 * (n_inputs + 1), 0);
    launch_optimizer(ctx, kind, a, in, po, n);
  }
  *out = o;
  BG_API_END
}

int bg_reduce_last(bg_ctx* ctx, bg_handle x, int64_t rows, int64_t cols, int op,
                   int keepdims, bg_handle* out) {
  BG_API_BEGIN
  Record& rx = get(ctx, x, "reduce[x]");
  if (rows < 0 || cols <= 0 || rows * cols != rx.numel())
    fail(BG_E_SHAPE, "reduce: rows*cols mismatch");
  if (op < BG_RED_SUM || op > BG_RED_MIN) fail(BG_E_INVALID, "reduce: unknown op");
  // A one-op program (COPY) with the reduction epilogue of the fused kernel.
  bg_fused_op cp{BG_OP_COPY, -1, 0, 0};
  int64_t shp[2] = {rows, cols};
  bg_fused_desc d{};
  d.n_inputs = 1;
  d.inputs = &x;
  d.n_ops = 1;
  d.ops = &cp;
  d.rank = 2;
  d.shape = shp;
  d.out_dtype = rx.dtype == BG_BOOL || rx.dtype == BG_U8 ? BG_F32 : rx.dtype;
  d.reduce_op = op;
  d.reduce_keepdims = keepdims;
  int rc = bg_fused_ex(ctx, &d, out);
  if (rc != BG_OK) return rc;
  // Report the caller's shape: leading dims of x plus the reduced axis.
  std::vector<int64_t> os(rx.shape);
  if (!os.empty()) {
    if (keepdims) os.back() = 1; else os.pop_back();
  }
  if (numel(os) == rows) ctx->handles[*out].shape = os;
  BG_API_END
}

int bg_matmul(bg_ctx* ctx, bg_handle a, bg_handle b, int64_t m, int64_t k,
              int64_t n, int dtype, bg_handle* out) {
  BG_API_BEGIN
  if (m <= 0 || k <= 0 || n <= 0)
    fail(BG_E_INVALID, "matmul: m, k, n must be positive integers");
  Record& ra = get(ctx, a, "matmul[A]");
  Record& rb = get(ctx, b, "matmul[B]");
  if (ra.numel() != m * k || rb.numel() != k * n)
    fail(BG_E_SHAPE, "matmul: handle sizes do not match m, k, n");
  if (ra.dtype != dtype || rb.dtype != dtype)
    fail(BG_E_DTYPE, std::string("matmul: operands must be ") + dtype_name(dtype));
  bg_matmul_desc d{};
  d.a = a;
  d.b = b;
  d.batch = 1;
  d.m = m;
  d.n = n;
  d.k = k;
  d.lda = k;
  d.ldb = n;
  d.ldc = n;
  d.trans_b = 0;
  d.in_dtype = dtype;
  d.out_dtype = dtype;
  d.round_f16 = 0;
  d.act = BG_ACT_NONE;
  return bg_matmul_ex(ctx, &d, out);
  BG_API_END
}

// bg_matmul_ex and bg_matmul_ex2: ext NULL = no extras.
static void matmul_entry(bg_ctx* ctx, const bg_matmul_desc* desc, const bg_matmul_ext* ext, bg_handle* out) {
  if (!desc || !out) fail(BG_E_INVALID, "matmul_ex: NULL argument");
  const bg_matmul_desc& d = *desc;
  GemmExtra ex;
  if (ext) {
    for (int32_t r : ext->reserved)
      if (r != 0) fail(BG_E_INVALID, "matmul_ex2: reserved fields must be 0");
    ex.a_dtype = ext->a_dtype;
    ex.b_dtype = ext->b_dtype;
  }
  const int a_dt = ex.a_dtype >= 0 ? ex.a_dtype : d.in_dtype;
  const int b_dt = ex.b_dtype >= 0 ? ex.b_dtype : d.in_dtype;
  for (int dt : {a_dt, b_dt})
    if (dt != BG_F32 && dt != BG_F16 && dt != BG_BF16)
      fail(BG_E_DTYPE, std::string("matmul_ex2: operand storage dtype ") + dtype_name(dt) + " not supported");
  if (d.m <= 0 || d.n <= 0 || d.k <= 0 || d.batch <= 0)
    fail(BG_E_INVALID, "matmul: batch, m, k, n must be positive integers");
  Record& ra = get(ctx, d.a, "matmul[A]");
  Record& rb = get(ctx, d.b, "matmul[B]");
  const Record* rbias = nullptr;
  if (d.bias) {
    rbias = &get(ctx, d.bias, "matmul[bias]");
    if (rbias->dtype != BG_F32 || rbias->numel() != d.n)
      fail(BG_E_SHAPE, "matmul: bias must be float32 [N]");
  }
  if (ra.dtype != a_dt || rb.dtype != b_dt) {
    if (!ext) fail(BG_E_DTYPE, std::string("matmul: operands must be ") + dtype_name(d.in_dtype));
    fail(BG_E_DTYPE, std::string("matmul_ex2: operands must be stored as ") + dtype_name(a_dt) + " and " +
                         dtype_name(b_dt));
  }
  if (a_dt != d.in_dtype && (d.in_dtype == BG_F32 || d.lda != d.k ||
                             (d.batch > 1 && d.stride_a != 0 && d.stride_a != d.m * d.k)))
    fail(BG_E_UNSUPPORTED, "matmul_ex2: a cast operand must be a dense [batch][m][k] block for a 16-bit GEMM");
  if (b_dt != d.in_dtype && (d.in_dtype == BG_F32 || d.ldb != (d.trans_b ? d.k : d.n) ||
                             (d.batch > 1 && d.stride_b != 0 && d.stride_b != d.k * d.n)))
    fail(BG_E_UNSUPPORTED, "matmul_ex2: a cast operand must be a dense [batch] x matrix for a 16-bit GEMM");
  if (d.in_dtype != BG_F32 && d.in_dtype != BG_F16 && d.in_dtype != BG_BF16)
    fail(BG_E_DTYPE, std::string("matmul: dtype ") + dtype_name(d.in_dtype) +
                         " not supported");
  if (d.out_dtype != BG_F32 && d.out_dtype != BG_F16 && d.out_dtype != BG_BF16)
    fail(BG_E_DTYPE, "matmul: output dtype not supported");
  if (d.stride_a < 0 || d.stride_b < 0 || d.stride_c < 0 || d.offset_a < 0 || d.offset_b < 0 ||
      d.lda < 0 || d.ldb < 0 || d.ldc < 0)
    fail(BG_E_INVALID, "matmul: negative stride/offset");
  // Bounds of the strided operands.
  auto need = [](int64_t off, int64_t batch, int64_t sb, int64_t rows, int64_t ld,
                 int64_t cols) {
    return off + (batch - 1) * sb + (rows - 1) * ld + cols;
  };
  if (d.lda < d.k) fail(BG_E_SHAPE, "matmul: lda < k");
  if (need(d.offset_a, d.batch, d.stride_a, d.m, d.lda, d.k) > ra.numel())
    fail(BG_E_SHAPE, "matmul: A view exceeds its handle");
  if (d.trans_b) {
    if (d.ldb < d.k) fail(BG_E_SHAPE, "matmul: ldb < k");
    if (need(d.offset_b, d.batch, d.stride_b, d.n, d.ldb, d.k) > rb.numel())
      fail(BG_E_SHAPE, "matmul: B view exceeds its handle");
  } else {
    if (d.ldb < d.n) fail(BG_E_SHAPE, "matmul: ldb < n");
    if (need(d.offset_b, d.batch, d.stride_b, d.k, d.ldb, d.n) > rb.numel())
      fail(BG_E_SHAPE, "matmul: B view exceeds its handle");
  }
  bg_matmul_desc dd = d;
  if (dd.ldc == 0) dd.ldc = d.n;
  if (dd.stride_c == 0) dd.stride_c = d.m * dd.ldc;
  if (dd.ldc < d.n) fail(BG_E_SHAPE, "matmul: ldc < n");
  if (d.batch > 1 && dd.stride_c < (d.m - 1) * dd.ldc + d.n)
    fail(BG_E_SHAPE, "matmul: stride_c makes the output matrices of the batch overlap");
  if (ext && ext->residual) {
    const Record& rr = get(ctx, ext->residual, "matmul[residual]");
    if (rr.dtype != BG_F32 || rr.numel() != d.batch * d.m * d.n)
      fail(BG_E_SHAPE, "matmul_ex2: residual must be float32 holding batch * m * n elements");
    if (dd.ldc != d.n || (d.batch > 1 && dd.stride_c != d.m * d.n))
      fail(BG_E_UNSUPPORTED, "matmul_ex2: a residual needs a dense output (ldc = n, stride_c = m * n)");
  }
  std::vector<int64_t> os;
  if (d.batch > 1) os.push_back(d.batch);
  os.push_back(d.m);
  os.push_back(d.n);
  int64_t out_elems = (d.batch - 1) * dd.stride_c + (d.m - 1) * dd.ldc + d.n;
  bg_handle o = mint(ctx, size_t(out_elems * dtype_size(d.out_dtype)), os, d.out_dtype);
  Record& ro = ctx->handles[o];
  Record& ra2 = ctx->handles[d.a];
  Record& rb2 = ctx->handles[d.b];
  const Record* rbias2 = d.bias ? &ctx->handles[d.bias] : nullptr;
  if (ext && ext->residual) ex.residual = reinterpret_cast<const float*>(ctx->handles[ext->residual].ptr());
  try {
    launch_matmul(ctx, dd, ra2, rb2, rbias2, ro, &ex);
  } catch (...) {
    bg_release(ctx, o);
    throw;
  }
  *out = o;
}

int bg_matmul_ex(bg_ctx* ctx, const bg_matmul_desc* desc, bg_handle* out) {
  BG_API_BEGIN
  matmul_entry(ctx, desc, nullptr, out);
  BG_API_END
}

int bg_matmul_ex2(bg_ctx* ctx, const bg_matmul_desc* desc, const bg_matmul_ext* ext, bg_handle* out) {
  BG_API_BEGIN
  if (!ext) fail(BG_E_INVALID, "matmul_ex2: NULL ext");
  matmul_entry(ctx, desc, ext, out);
  BG_API_END
}

// True when rows of `row` contiguous elements placed at sum_i idx_i *
// strides[i] (idx_i < extents[i]) never overlap: taken in increasing stride
// order, every stride must clear the span of the dimensions inside it.
// Dimensions of extent 1 take no part.
static bool disjoint_rows(std::vector<int64_t> extents, std::vector<int64_t> strides, int64_t row) {
  std::vector<size_t> order;
  for (size_t i = 0; i < extents.size(); ++i)
    if (extents[i] > 1) order.push_back(i);
  std::sort(order.begin(), order.end(), [&](size_t a, size_t b) { return strides[a] < strides[b]; });
  int64_t span = row;
  for (size_t i : order) {
    if (strides[i] < span) return false;
    span = strides[i] * (extents[i] - 1) + span;
  }
  return true;
}

int bg_attention_ex(bg_ctx* ctx, const bg_attention_desc* desc, bg_handle* out) {
  BG_API_BEGIN
  if (!desc || !out) fail(BG_E_INVALID, "attention_ex: NULL argument");
  bg_attention_desc d = *desc;
  if (d.batch <= 0 || d.heads <= 0 || d.sq <= 0 || d.sk <= 0 || d.d <= 0)
    fail(BG_E_INVALID, "flash_attention: b, h, sq, sk, d must be positive integers");
  Record& rq = get(ctx, d.q, "flash_attention[Q]");
  Record& rk = get(ctx, d.k, "flash_attention[K]");
  Record& rv = get(ctx, d.v, "flash_attention[V]");
  if (rq.dtype != d.in_dtype || rk.dtype != d.in_dtype || rv.dtype != d.in_dtype)
    fail(BG_E_DTYPE, "flash_attention: Q/K/V dtype differs from in_dtype");
  // Default strides: contiguous [B,H,S,D].
  auto fix = [&](int64_t& sb, int64_t& sh, int64_t& ss, int64_t s) {
    if (sb == 0 && sh == 0 && ss == 0) {
      ss = d.d;
      sh = s * d.d;
      sb = d.heads * s * d.d;
    }
  };
  fix(d.q_sb, d.q_sh, d.q_ss, d.sq);
  fix(d.k_sb, d.k_sh, d.k_ss, d.sk);
  fix(d.v_sb, d.v_sh, d.v_ss, d.sk);
  fix(d.o_sb, d.o_sh, d.o_ss, d.sq);
  for (int64_t x : {d.q_off, d.k_off, d.v_off, d.q_sb, d.q_sh, d.q_ss, d.k_sb, d.k_sh, d.k_ss, d.v_sb,
                    d.v_sh, d.v_ss, d.o_sb, d.o_sh, d.o_ss})
    if (x < 0) fail(BG_E_INVALID, "flash_attention: negative offset or stride");
  if (!disjoint_rows({d.batch, d.heads, d.sq}, {d.o_sb, d.o_sh, d.o_ss}, d.d))
    fail(BG_E_SHAPE, "flash_attention: output strides make output rows overlap");
  auto reach = [&](int64_t off, int64_t sb, int64_t sh, int64_t ss, int64_t s) {
    return off + (d.batch - 1) * sb + (d.heads - 1) * sh + (s - 1) * ss + d.d;
  };
  if (reach(d.q_off, d.q_sb, d.q_sh, d.q_ss, d.sq) > rq.numel() ||
      reach(d.k_off, d.k_sb, d.k_sh, d.k_ss, d.sk) > rk.numel() ||
      reach(d.v_off, d.v_sb, d.v_sh, d.v_ss, d.sk) > rv.numel())
    fail(BG_E_SHAPE, "flash_attention: Q/K/V views exceed their handles");
  int64_t out_elems = reach(0, d.o_sb, d.o_sh, d.o_ss, d.sq);
  std::vector<int64_t> os = {d.batch, d.heads, d.sq, d.d};
  bg_handle o = mint(ctx, size_t(out_elems * dtype_size(d.out_dtype)), os, d.out_dtype);
  Record& ro = ctx->handles[o];
  try {
    launch_attention(ctx, d, ctx->handles[d.q], ctx->handles[d.k], ctx->handles[d.v], ro);
  } catch (...) {
    bg_release(ctx, o);
    throw;
  }
  *out = o;
  BG_API_END
}

int bg_matmul_launch_plan(const bg_matmul_desc* desc, bg_launch_plan* out, char* err, size_t err_cap) {
  return no_ctx_call(err, err_cap, [&] {
    if (!desc || !out) fail(BG_E_INVALID, "matmul_launch_plan: NULL argument");
    plan_matmul(*desc, *out);
  });
}

int bg_attention_launch_plan(const bg_attention_desc* desc, bg_launch_plan* out, char* err, size_t err_cap) {
  return no_ctx_call(err, err_cap, [&] {
    if (!desc || !out) fail(BG_E_INVALID, "attention_launch_plan: NULL argument");
    plan_attention(*desc, *out);
  });
}

int bg_flash_attention(bg_ctx* ctx, bg_handle q, bg_handle k, bg_handle v,
                       bg_handle mask, int64_t b, int64_t h, int64_t sq,
                       int64_t sk, int64_t d, float scale, int dtype,
                       bg_handle* out) {
  BG_API_BEGIN
  if (b <= 0 || h <= 0 || sq <= 0 || sk <= 0 || d <= 0)
    fail(BG_E_INVALID, "flash_attention: b, h, sq, sk, d must be positive integers");
  Record& rq = get(ctx, q, "flash_attention[Q]");
  Record& rk = get(ctx, k, "flash_attention[K]");
  Record& rv = get(ctx, v, "flash_attention[V]");
  if (rq.numel() != b * h * sq * d || rk.numel() != b * h * sk * d ||
      rv.numel() != b * h * sk * d)
    fail(BG_E_SHAPE, "flash_attention: Q/K/V sizes do not match [b,h,s,d]");
  if (rq.dtype != dtype || rk.dtype != dtype || rv.dtype != dtype)
    fail(BG_E_DTYPE, std::string("flash_attention: operands must be ") + dtype_name(dtype));
  if (mask == 0) {
    bg_attention_desc a{};
    a.q = q;
    a.k = k;
    a.v = v;
    a.batch = b;
    a.heads = h;
    a.sq = sq;
    a.sk = sk;
    a.d = d;
    a.scale = scale;
    a.causal = 0;
    a.in_dtype = dtype;
    a.out_dtype = dtype;
    a.round_scores = 0;
    return bg_attention_ex(ctx, &a, out);
  }
  // Additive mask path (flash_attention.ts:45-131): f32 only, mask shaped
  // [1|b, 1|h, sq, sk].
  if (dtype != BG_F32)
    fail(BG_E_DTYPE, "flash_attention: an additive mask requires float32");
  Record& rm = get(ctx, mask, "flash_attention[mask]");
  if (rm.dtype != BG_F32) fail(BG_E_DTYPE, "flash_attention: mask must be float32");
  // Broadcast comes from the mask's recorded shape: [1|b, 1|h, sq, sk] or
  // [sq, sk].  Any other shape must hold the full b*h*sq*sk elements, the
  // layout the reference bridge reads (mask_B = B, mask_H = H).
  const int64_t per = sq * sk;
  const std::vector<int64_t>& ms = rm.shape;
  int64_t mb = 0, mh = 0;
  if (ms.size() == 4 && ms[2] == sq && ms[3] == sk && (ms[0] == 1 || ms[0] == b) &&
      (ms[1] == 1 || ms[1] == h)) {
    mh = ms[1] == 1 ? 0 : per;
    mb = ms[0] == 1 ? 0 : ms[1] * per;
  } else if (ms.size() == 2 && ms[0] == sq && ms[1] == sk) {
    mb = mh = 0;
  } else if (rm.numel() == b * h * per) {
    mb = h * per;
    mh = per;
  } else {
    fail(BG_E_SHAPE, "flash_attention: mask must be [1|b,1|h,sq,sk] or [sq,sk]");
  }
  std::vector<int64_t> os = {b, h, sq, d};
  bg_handle o = mint(ctx, size_t(b * h * sq * d * 4), os, BG_F32);
  Record& ro = ctx->handles[o];
  {
    Profile prof(ctx, "flash_attention_masked", 4 * (2 * b * h * sq * d + 2 * b * h * sk * d),
                 4 * b * h * sq * sk * d);
    launch_attention_masked_f32(
        ctx, reinterpret_cast<float*>(ctx->handles[q].ptr()),
        reinterpret_cast<float*>(ctx->handles[k].ptr()),
        reinterpret_cast<float*>(ctx->handles[v].ptr()),
        reinterpret_cast<float*>(ctx->handles[mask].ptr()), mb, mh,
        reinterpret_cast<float*>(ro.ptr()), b, h, sq, sk, d, scale);
  }
  *out = o;
  BG_API_END
}

static int run_plan_abi(bg_ctx* ctx, const char* plan_json, const char* requests_json,
                        const int64_t* input_ids, const bg_handle* input_handles, int n_inputs,
                        int dtype, void* dst, size_t dst_nbytes, bg_handle* root_out) {
  BG_API_BEGIN
  if (!plan_json) fail(BG_E_INVALID, "run_tensor_plan: plan is NULL");
  if (n_inputs < 0 || (n_inputs > 0 && (!input_ids || !input_handles)))
    fail(BG_E_INVALID, "run_tensor_plan: bad input arrays");
  if (!dst && !root_out) fail(BG_E_INVALID, "run_tensor_plan: neither dst nor root_out given");
  bg_handle root = run_plan(ctx, plan_json, requests_json, input_ids, input_handles, n_inputs, dtype,
                            dst == nullptr);
  if (dst) {
    int rc = bg_materialize(ctx, root, dst, dst_nbytes);
    if (rc != BG_OK) {
      std::string m = ctx->err;
      bg_release(ctx, root);
      fail(rc, m);
    }
    bg_release(ctx, root);
    if (root_out) *root_out = 0;
  } else {
    *root_out = root;
  }
  BG_API_END
}

int bg_run_tensor_plan(bg_ctx* ctx, const char* plan_json,
                       const int64_t* input_ids, const bg_handle* input_handles,
                       int n_inputs, int dtype, void* dst, size_t dst_nbytes,
                       bg_handle* root_out) {
  return run_plan_abi(ctx, plan_json, nullptr, input_ids, input_handles, n_inputs, dtype, dst, dst_nbytes,
                      root_out);
}

int bg_run_tensor_plan_semantic(bg_ctx* ctx, const char* plan_json, const char* requests_json,
                                const int64_t* input_ids, const bg_handle* input_handles, int n_inputs,
                                int dtype, void* dst, size_t dst_nbytes, bg_handle* root_out) {
  if (!requests_json) {
    if (ctx) ctx->err = "run_tensor_plan_semantic: requests are NULL";
    return BG_E_INVALID;
  }
  return run_plan_abi(ctx, plan_json, requests_json, input_ids, input_handles, n_inputs, dtype, dst,
                      dst_nbytes, root_out);
}

int bg_set_launch_log(bg_ctx* ctx, int on) {
  BG_API_BEGIN
  ctx->log_launches = on != 0;
  BG_API_END
}

int bg_take_launch_log(bg_ctx* ctx, bg_launch_record* out, int cap, int* n_out) {
  BG_API_BEGIN
  if (!n_out) fail(BG_E_INVALID, "take_launch_log: NULL count");
  auto& log = ctx->launch_log;
  if (!out) {
    *n_out = int(log.size());
  } else {
    const size_t n = std::min(log.size(), size_t(cap < 0 ? 0 : cap));
    std::copy(log.begin(), log.begin() + n, out);
    log.erase(log.begin(), log.begin() + n);
    *n_out = int(n);
  }
  BG_API_END
}

int bg_plan_inspect(const char* plan_json, const char* requests_json, char* out, size_t out_cap,
                    size_t* needed) {
  std::string text;
  int rc = BG_OK;
  try {
    if (!plan_json) fail(BG_E_INVALID, "plan_inspect: plan is NULL");
    text = inspect_plan(plan_json, requests_json);
  } catch (const Error& e) {
    rc = e.code;
    text = e.what();
  } catch (const std::exception& e) {
    rc = BG_E_INVALID;
    text = e.what();
  }
  if (needed) *needed = text.size() + 1;
  if (out && out_cap > 0) {
    const size_t n = std::min(out_cap - 1, text.size());
    std::memcpy(out, text.data(), n);
    out[n] = 0;
  }
  return rc;
}

int bg_softmax_last(bg_ctx* ctx, bg_handle x, int64_t rows, int64_t cols, int out_dtype, bg_handle* out) {
  BG_API_BEGIN
  if (!out) fail(BG_E_INVALID, "softmax: NULL output");
  Record& rx = get(ctx, x, "softmax[x]");
  if (rows < 0 || cols <= 0 || rows * cols != rx.numel()) fail(BG_E_SHAPE, "softmax: rows*cols does not match x");
  if (rx.dtype != BG_F32 && rx.dtype != BG_F16 && rx.dtype != BG_BF16)
    fail(BG_E_DTYPE, "softmax: x dtype not supported");
  if (out_dtype != BG_F32 && out_dtype != BG_F16 && out_dtype != BG_BF16)
    fail(BG_E_DTYPE, "softmax: out dtype not supported");
  bg_handle o = mint(ctx, size_t(rows * cols * dtype_size(out_dtype)), rx.shape, out_dtype);
  Record& ro = ctx->handles[o];
  Record& rx2 = ctx->handles[x];
  try {
    Profile prof(ctx, "softmax", rows * cols * (dtype_size(rx2.dtype) + dtype_size(out_dtype)), 0);
    launch_softmax_last(ctx, rx2.ptr(), rx2.dtype, ro.ptr(), out_dtype, rows, cols);
  } catch (...) {
    bg_release(ctx, o);
    throw;
  }
  *out = o;
  BG_API_END
}

}  // extern "C"
