// N-API binding of libbghip: the native half of createHipRealizerBridge
// (index.js), the Node twin of the reference's createWebGpuRealizerBridge
// (packages/browsergrad-kernels/src/realizer.ts:902-1005).
//
// Every export is a thin wrapper over one C-ABI entry point of
// include/bghip.h; the context is a napi External owned by the JS bridge
// object.  Failures become a JS Error named "KernelError" whose message is
// bg_last_error(ctx), like the reference's op-qualified KernelError
// (types.ts:87-92).  materializeAsync and runTensorPlanAsync return Promises
// settled off the event loop: the blocking read-back runs on a libuv worker
// (napi_async_work), as the reference resolves them after mapAsync
// (realizer.ts:79-91, runner.ts:537-581).  A context is used by one thread
// at a time: every binding holds the context's mutex while it calls the
// library, so a call made while a worker is busy waits for it.
#include <node_api.h>

#include <cstdint>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "bghip.h"

namespace {

struct Ctx {
  bg_ctx* ctx = nullptr;
  std::mutex mu;  // one thread in the library per context
};

void finalize_ctx(napi_env, void* data, void*) {
  auto* c = static_cast<Ctx*>(data);
  if (c->ctx) bg_ctx_destroy(c->ctx);
  delete c;
}

napi_value throw_kernel_error(napi_env env, const std::string& msg) {
  napi_value m, err, name;
  napi_create_string_utf8(env, msg.c_str(), msg.size(), &m);
  napi_create_error(env, nullptr, m, &err);
  napi_create_string_utf8(env, "KernelError", NAPI_AUTO_LENGTH, &name);
  napi_set_named_property(env, err, "name", name);
  napi_throw(env, err);
  return nullptr;
}

// Throws (and returns false) when rc is not BG_OK.
bool check(napi_env env, bg_ctx* ctx, int rc) {
  if (rc == BG_OK) return true;
  throw_kernel_error(env, ctx ? bg_last_error(ctx) : "HIP bridge: null context");
  return false;
}

struct Args {
  napi_env env;
  std::vector<napi_value> v;
  bool ok = true;
  Ctx* holder = nullptr;
  std::unique_lock<std::mutex> lock;  // held for the rest of the call once ctx() is read
  Args(napi_env e, napi_callback_info info, size_t n) : env(e), v(n) {
    size_t argc = n;
    napi_get_cb_info(e, info, &argc, v.data(), nullptr, nullptr);
    if (argc < n) {
      throw_kernel_error(e, "HIP bridge: expected " + std::to_string(n) + " arguments");
      ok = false;
    }
  }
  bg_ctx* ctx(size_t i = 0) {
    void* p = nullptr;
    if (napi_get_value_external(env, v[i], &p) != napi_ok || !p) {
      throw_kernel_error(env, "HIP bridge: bad context");
      ok = false;
      return nullptr;
    }
    holder = static_cast<Ctx*>(p);
    lock = std::unique_lock<std::mutex>(holder->mu);
    return holder->ctx;
  }
  double num(size_t i) {
    double d = 0;
    if (napi_get_value_double(env, v[i], &d) != napi_ok) {
      throw_kernel_error(env, "HIP bridge: argument " + std::to_string(i) + " must be a number");
      ok = false;
    }
    return d;
  }
  int64_t i64(size_t i) { return static_cast<int64_t>(num(i)); }
  bg_handle handle(size_t i) { return static_cast<bg_handle>(num(i)); }
  bool is_nullish(size_t i) {
    napi_valuetype t;
    napi_typeof(env, v[i], &t);
    return t == napi_null || t == napi_undefined;
  }
  std::string str(size_t i) {
    size_t n = 0;
    if (napi_get_value_string_utf8(env, v[i], nullptr, 0, &n) != napi_ok) {
      throw_kernel_error(env, "HIP bridge: argument " + std::to_string(i) + " must be a string");
      ok = false;
      return {};
    }
    std::string s(n, '\0');
    napi_get_value_string_utf8(env, v[i], &s[0], n + 1, &n);
    return s;
  }
  std::vector<double> nums(size_t i) {
    std::vector<double> out;
    bool is_arr = false;
    napi_is_array(env, v[i], &is_arr);
    if (!is_arr) {
      throw_kernel_error(env, "HIP bridge: argument " + std::to_string(i) + " must be an array");
      ok = false;
      return out;
    }
    uint32_t n = 0;
    napi_get_array_length(env, v[i], &n);
    for (uint32_t k = 0; k < n; ++k) {
      napi_value e;
      double d = 0;
      napi_get_element(env, v[i], k, &e);
      if (napi_get_value_double(env, e, &d) != napi_ok) {
        throw_kernel_error(env, "HIP bridge: array elements must be numbers");
        ok = false;
        return {};
      }
      out.push_back(d);
    }
    return out;
  }
  std::vector<int64_t> shape(size_t i) {
    std::vector<int64_t> s;
    for (double d : nums(i)) s.push_back(static_cast<int64_t>(d));
    return s;
  }
  int dtype(size_t i) {
    std::string s = str(i);
    int d = bg_dtype_from_name(s.c_str());
    if (ok && d < 0) {
      throw_kernel_error(env, "HIP bridge: unknown dtype " + s);
      ok = false;
    }
    return d;
  }
};

napi_value number(napi_env env, double d) {
  napi_value r;
  napi_create_double(env, d, &r);
  return r;
}

napi_value bytes(napi_env env, const void* src, size_t n) {
  void* data = nullptr;
  napi_value ab, u8;
  napi_create_arraybuffer(env, n, &data, &ab);
  if (n) std::memcpy(data, src, n);
  napi_create_typedarray(env, napi_uint8_array, n, ab, 0, &u8);
  return u8;
}

// ---- lifecycle ------------------------------------------------------------

napi_value CtxCreate(napi_env env, napi_callback_info info) {  // (device, profiling)
  Args a(env, info, 2);
  if (!a.ok) return nullptr;
  int device = static_cast<int>(a.num(0));
  bool prof = false;
  napi_get_value_bool(env, a.v[1], &prof);
  auto* c = new Ctx;
  int rc = bg_ctx_create(device, prof ? 1 : 0, &c->ctx);
  if (rc != BG_OK) {
    delete c;
    return throw_kernel_error(env, "HIP bridge: cannot open HIP device " + std::to_string(device) +
                                       " (status " + std::to_string(rc) + "); the HIP realizer has no CPU fallback");
  }
  napi_value ext;
  napi_create_external(env, c, finalize_ctx, nullptr, &ext);
  return ext;
}

napi_value CtxDestroy(napi_env env, napi_callback_info info) {
  Args a(env, info, 1);
  if (!a.ok) return nullptr;
  void* p = nullptr;
  napi_get_value_external(env, a.v[0], &p);
  auto* c = static_cast<Ctx*>(p);
  if (c) {
    std::lock_guard<std::mutex> lk(c->mu);  // waits for a read-back in flight
    if (c->ctx) {
      bg_ctx_destroy(c->ctx);
      c->ctx = nullptr;
    }
  }
  return nullptr;
}

// ---- data movement (realizer.ts:1007-1041) ---------------------------------

napi_value Upload(napi_env env, napi_callback_info info) {  // (ctx, Uint8Array, shape, dtype)
  Args a(env, info, 4);
  bg_ctx* ctx = a.ctx();
  if (!a.ok) return nullptr;
  bool is_ta = false;
  napi_is_typedarray(env, a.v[1], &is_ta);
  if (!is_ta) return throw_kernel_error(env, "WebGPU bridge: upload data must be a Uint8Array");
  napi_typedarray_type t;
  size_t len = 0, off = 0;
  void* data = nullptr;
  napi_value ab;
  napi_get_typedarray_info(env, a.v[1], &t, &len, &data, &ab, &off);
  size_t esz = t == napi_float32_array || t == napi_int32_array || t == napi_uint32_array ? 4
               : t == napi_float64_array ? 8 : t == napi_int16_array || t == napi_uint16_array ? 2 : 1;
  auto shape = a.shape(2);
  int dt = a.dtype(3);
  if (!a.ok) return nullptr;
  bg_handle h = 0;
  if (!check(env, ctx, bg_upload(ctx, data, len * esz, shape.data(), int(shape.size()), dt, &h))) return nullptr;
  return number(env, double(h));
}

napi_value Materialize(napi_env env, napi_callback_info info) {  // (ctx, h) -> Uint8Array
  Args a(env, info, 2);
  bg_ctx* ctx = a.ctx();
  bg_handle h = a.handle(1);
  if (!a.ok) return nullptr;
  int64_t shp[16];
  int rank = 0, dt = 0;
  int64_t nb = 0;
  if (!check(env, ctx, bg_handle_info(ctx, h, shp, &rank, &dt, &nb))) return nullptr;
  std::vector<uint8_t> buf(static_cast<size_t>(nb));
  if (!check(env, ctx, bg_materialize(ctx, h, buf.data(), buf.size()))) return nullptr;
  return bytes(env, buf.data(), buf.size());
}

napi_value Release(napi_env env, napi_callback_info info) {
  Args a(env, info, 2);
  bg_ctx* ctx = a.ctx();
  bg_handle h = a.handle(1);
  if (!a.ok) return nullptr;
  check(env, ctx, bg_release(ctx, h));
  return nullptr;
}

napi_value HandleInfo(napi_env env, napi_callback_info info) {
  Args a(env, info, 2);
  bg_ctx* ctx = a.ctx();
  bg_handle h = a.handle(1);
  if (!a.ok) return nullptr;
  int64_t shp[16];
  int rank = 0, dt = 0;
  int64_t nb = 0;
  if (!check(env, ctx, bg_handle_info(ctx, h, shp, &rank, &dt, &nb))) return nullptr;
  napi_value o, arr, s;
  napi_create_object(env, &o);
  napi_create_array_with_length(env, size_t(rank), &arr);
  for (int i = 0; i < rank; ++i) napi_set_element(env, arr, uint32_t(i), number(env, double(shp[i])));
  napi_set_named_property(env, o, "shape", arr);
  napi_create_int32(env, dt, &s);
  napi_set_named_property(env, o, "dtypeCode", s);
  napi_set_named_property(env, o, "byteLength", number(env, double(nb)));
  return o;
}

// ---- compute (realizer.ts:1043-1151) ---------------------------------------

napi_value Matmul(napi_env env, napi_callback_info info) {  // (ctx, a, b, m, k, n, dtype)
  Args a(env, info, 7);
  bg_ctx* ctx = a.ctx();
  bg_handle x = a.handle(1), y = a.handle(2);
  int64_t m = a.i64(3), k = a.i64(4), n = a.i64(5);
  int dt = a.dtype(6);
  if (!a.ok) return nullptr;
  bg_handle out = 0;
  if (!check(env, ctx, bg_matmul(ctx, x, y, m, k, n, dt, &out))) return nullptr;
  return number(env, double(out));
}

// (ctx, inputs[], opsFlat[] = [code, a, b, ...], shape[], dtype)
napi_value FusedElementwise(napi_env env, napi_callback_info info) {
  Args a(env, info, 5);
  bg_ctx* ctx = a.ctx();
  auto ins_d = a.nums(1);
  auto ops_d = a.nums(2);
  auto shape = a.shape(3);
  int dt = a.dtype(4);
  if (!a.ok) return nullptr;
  std::vector<bg_handle> ins(ins_d.begin(), ins_d.end());
  std::vector<bg_fused_op> ops;
  for (size_t i = 0; i + 2 < ops_d.size(); i += 3)
    ops.push_back({int32_t(ops_d[i]), int32_t(ops_d[i + 1]), int32_t(ops_d[i + 2]), 0});
  bg_handle out = 0;
  if (!check(env, ctx, bg_fused_elementwise(ctx, ins.data(), int(ins.size()), ops.data(), int(ops.size()),
                                            shape.data(), int(shape.size()), dt, &out)))
    return nullptr;
  return number(env, double(out));
}

napi_value Cast(napi_env env, napi_callback_info info) {  // (ctx, h, src, dst, shape)
  Args a(env, info, 5);
  bg_ctx* ctx = a.ctx();
  bg_handle h = a.handle(1);
  int sd = a.dtype(2), dd = a.dtype(3);
  auto shape = a.shape(4);
  if (!a.ok) return nullptr;
  bg_handle out = 0;
  if (!check(env, ctx, bg_cast(ctx, h, sd, dd, shape.data(), int(shape.size()), &out))) return nullptr;
  return number(env, double(out));
}

// (ctx, op, transposed, a, b|null, bias|null, n, cIn, cOut, groups, in[], out[],
//  k[], stride[], pad[], dilation[], outputPad[]) -> bg_conv_ex
napi_value Conv(napi_env env, napi_callback_info info) {
  Args a(env, info, 17);
  bg_ctx* ctx = a.ctx();
  bg_conv_desc d{};
  d.op = int32_t(a.i64(1));
  d.transposed = int32_t(a.i64(2));
  d.a = a.handle(3);
  d.b = a.is_nullish(4) ? 0 : a.handle(4);
  d.bias = a.is_nullish(5) ? 0 : a.handle(5);
  d.n = a.i64(6);
  d.c_in = a.i64(7);
  d.c_out = a.i64(8);
  d.groups = a.i64(9);
  int64_t* arrays[7] = {d.in, d.out, d.k, d.stride, d.pad, d.dilation, d.output_pad};
  for (int j = 0; j < 7 && a.ok; ++j) {
    const std::vector<double> v = a.nums(size_t(10 + j));
    if (!a.ok) break;
    if (j == 0) d.spatial = int32_t(v.size());
    if (v.size() != size_t(d.spatial) || v.size() < 1 || v.size() > 3) {
      throw_kernel_error(env, "HIP bridge: conv spatial arrays must hold 1 to 3 equal-length entries");
      return nullptr;
    }
    for (size_t i = 0; i < v.size(); ++i) arrays[j][i] = int64_t(v[i]);
  }
  if (!a.ok) return nullptr;
  bg_handle out = 0;
  if (!check(env, ctx, bg_conv_ex(ctx, &d, &out))) return nullptr;
  return number(env, double(out));
}

// (ctx, q, k, v, mask|null, b, h, sq, sk, d, scale, dtype)
napi_value FlashAttention(napi_env env, napi_callback_info info) {
  Args a(env, info, 12);
  bg_ctx* ctx = a.ctx();
  bg_handle q = a.handle(1), k = a.handle(2), v = a.handle(3);
  bg_handle mask = a.is_nullish(4) ? 0 : a.handle(4);
  int64_t b = a.i64(5), h = a.i64(6), sq = a.i64(7), sk = a.i64(8), d = a.i64(9);
  double scale = a.num(10);
  int dt = a.dtype(11);
  if (!a.ok) return nullptr;
  bg_handle out = 0;
  if (!check(env, ctx, bg_flash_attention(ctx, q, k, v, mask, b, h, sq, sk, d, float(scale), dt, &out)))
    return nullptr;
  return number(env, double(out));
}

// (ctx, planJson, requestsJson|null, ids[], handles[], dtype, resident, rootBytes)
napi_value RunTensorPlan(napi_env env, napi_callback_info info) {
  Args a(env, info, 8);
  bg_ctx* ctx = a.ctx();
  std::string plan = a.str(1);
  bool semantic = !a.is_nullish(2);
  std::string req = semantic ? a.str(2) : std::string();
  auto ids_d = a.nums(3);
  auto hs_d = a.nums(4);
  int dt = a.dtype(5);
  bool resident = false;
  napi_get_value_bool(env, a.v[6], &resident);
  int64_t nbytes = resident ? 0 : a.i64(7);
  if (!a.ok) return nullptr;
  std::vector<int64_t> ids(ids_d.begin(), ids_d.end());
  std::vector<bg_handle> hs(hs_d.begin(), hs_d.end());
  std::vector<uint8_t> buf(resident ? 0 : size_t(nbytes));
  bg_handle root = 0;
  void* dst = resident ? nullptr : static_cast<void*>(buf.data());
  int rc = semantic ? bg_run_tensor_plan_semantic(ctx, plan.c_str(), req.c_str(), ids.data(), hs.data(),
                                                  int(ids.size()), dt, dst, buf.size(), &root)
                    : bg_run_tensor_plan(ctx, plan.c_str(), ids.data(), hs.data(), int(ids.size()), dt, dst,
                                         buf.size(), &root);
  if (!check(env, ctx, rc)) return nullptr;
  if (resident) return number(env, double(root));
  return bytes(env, buf.data(), buf.size());
}

// ---- Promise-returning read-backs (napi_async_work) ---------------------------

// One queued blocking call: `run` executes on a libuv worker with the
// context's mutex held; the Promise resolves with `out` bytes (or the root
// handle) or rejects with the library's message.
struct Work {
  Ctx* holder = nullptr;
  napi_ref keep = nullptr;  // keeps the context External alive while queued
  napi_deferred deferred = nullptr;
  napi_async_work work = nullptr;
  int rc = BG_OK;
  std::string err;
  std::vector<uint8_t> out;
  bool resident = false;
  bg_handle root = 0;
  // materialize
  bg_handle h = 0;
  // tensor plan
  std::string plan, req;
  bool semantic = false;
  std::vector<int64_t> ids;
  std::vector<bg_handle> hs;
  int dtype = 0;
};

void work_execute(napi_env, void* data) {
  auto* w = static_cast<Work*>(data);
  std::lock_guard<std::mutex> lk(w->holder->mu);
  bg_ctx* ctx = w->holder->ctx;
  if (!ctx) {  // closed while the call was queued
    w->rc = BG_E_INVALID;
    w->err = "HIP bridge: context closed";
    return;
  }
  if (!w->plan.empty()) {
    void* dst = w->resident ? nullptr : static_cast<void*>(w->out.data());
    w->rc = w->semantic ? bg_run_tensor_plan_semantic(ctx, w->plan.c_str(), w->req.c_str(), w->ids.data(),
                                                      w->hs.data(), int(w->ids.size()), w->dtype, dst,
                                                      w->out.size(), &w->root)
                        : bg_run_tensor_plan(ctx, w->plan.c_str(), w->ids.data(), w->hs.data(),
                                             int(w->ids.size()), w->dtype, dst, w->out.size(), &w->root);
  } else {
    w->rc = bg_materialize(ctx, w->h, w->out.data(), w->out.size());
  }
  if (w->rc != BG_OK) w->err = bg_last_error(ctx);
}

void work_complete(napi_env env, napi_status, void* data) {
  auto* w = static_cast<Work*>(data);
  if (w->rc == BG_OK) {
    napi_value v = w->resident ? number(env, double(w->root)) : bytes(env, w->out.data(), w->out.size());
    napi_resolve_deferred(env, w->deferred, v);
  } else {
    napi_value m, e, name;
    napi_create_string_utf8(env, w->err.c_str(), w->err.size(), &m);
    napi_create_error(env, nullptr, m, &e);
    napi_create_string_utf8(env, "KernelError", NAPI_AUTO_LENGTH, &name);
    napi_set_named_property(env, e, "name", name);
    napi_reject_deferred(env, w->deferred, e);
  }
  napi_delete_reference(env, w->keep);
  napi_delete_async_work(env, w->work);
  delete w;
}

napi_value queue(napi_env env, napi_value ctx_value, Work* w, const char* name) {
  napi_value promise, res_name;
  napi_create_promise(env, &w->deferred, &promise);
  napi_create_reference(env, ctx_value, 1, &w->keep);
  napi_create_string_utf8(env, name, NAPI_AUTO_LENGTH, &res_name);
  napi_create_async_work(env, nullptr, res_name, work_execute, work_complete, w, &w->work);
  napi_queue_async_work(env, w->work);
  return promise;
}

napi_value MaterializeAsync(napi_env env, napi_callback_info info) {  // (ctx, h) -> Promise<Uint8Array>
  Args a(env, info, 2);
  bg_ctx* ctx = a.ctx();
  bg_handle h = a.handle(1);
  if (!a.ok) return nullptr;
  int64_t shp[BG_MAX_RANK];
  int rank = 0, dt = 0;
  int64_t nb = 0;
  if (!check(env, ctx, bg_handle_info(ctx, h, shp, &rank, &dt, &nb))) return nullptr;
  auto* w = new Work();
  w->holder = a.holder;
  w->h = h;
  w->out.resize(static_cast<size_t>(nb));
  a.lock.unlock();  // the worker takes the mutex itself
  return queue(env, a.v[0], w, "bghip.materialize");
}

// (ctx, planJson, requestsJson|null, ids[], handles[], dtype, resident, rootBytes) -> Promise
napi_value RunTensorPlanAsync(napi_env env, napi_callback_info info) {
  Args a(env, info, 8);
  a.ctx();
  auto* w = new Work();
  w->plan = a.str(1);
  w->semantic = !a.is_nullish(2);
  if (w->semantic) w->req = a.str(2);
  auto ids_d = a.nums(3);
  auto hs_d = a.nums(4);
  w->dtype = a.dtype(5);
  napi_get_value_bool(env, a.v[6], &w->resident);
  const int64_t nbytes = w->resident ? 0 : a.i64(7);
  if (!a.ok || w->plan.empty() || nbytes < 0) {
    if (a.ok) throw_kernel_error(env, "HIP bridge: runTensorPlanAsync: bad plan or root size");
    delete w;
    return nullptr;
  }
  w->holder = a.holder;
  w->ids.assign(ids_d.begin(), ids_d.end());
  w->hs.assign(hs_d.begin(), hs_d.end());
  w->out.resize(size_t(nbytes));
  a.lock.unlock();
  return queue(env, a.v[0], w, "bghip.run_tensor_plan");
}

// ---- diagnostics (realizer.ts:275-298) ---------------------------------------

napi_value AliveHandles(napi_env env, napi_callback_info info) {
  Args a(env, info, 1);
  bg_ctx* ctx = a.ctx();
  if (!a.ok) return nullptr;
  int64_t n = 0;
  if (!check(env, ctx, bg_alive_handles(ctx, &n))) return nullptr;
  return number(env, double(n));
}

napi_value ResourceSnapshot(napi_env env, napi_callback_info info) {
  Args a(env, info, 1);
  bg_ctx* ctx = a.ctx();
  if (!a.ok) return nullptr;
  bg_snapshot s{};
  if (!check(env, ctx, bg_resource_snapshot(ctx, &s))) return nullptr;
  napi_value o, tm, tq;
  napi_create_object(env, &o);
  napi_create_string_utf8(env, s.timing_mode == 1 ? "hip-event" : "unavailable", NAPI_AUTO_LENGTH, &tm);
  napi_set_named_property(env, o, "timingMode", tm);
  napi_get_boolean(env, s.timestamp_query_available != 0, &tq);
  napi_set_named_property(env, o, "timestampQueryAvailable", tq);
  napi_set_named_property(env, o, "currentOwnedGpuBytes", number(env, double(s.current_owned_bytes)));
  napi_set_named_property(env, o, "peakOwnedGpuBytes", number(env, double(s.peak_owned_bytes)));
  napi_set_named_property(env, o, "totalAllocatedGpuBytes", number(env, double(s.total_allocated_bytes)));
  napi_set_named_property(env, o, "totalReleasedGpuBytes", number(env, double(s.total_released_bytes)));
  napi_set_named_property(env, o, "aliveHandleCount", number(env, double(s.alive_handle_count)));
  napi_set_named_property(env, o, "pendingProfileCount", number(env, double(s.pending_profile_count)));
  napi_set_named_property(env, o, "passProfileCount", number(env, double(s.pass_profile_count)));
  return o;
}

napi_value FlushProfiles(napi_env env, napi_callback_info info) {
  Args a(env, info, 1);
  bg_ctx* ctx = a.ctx();
  if (!a.ok) return nullptr;
  int n = 0;
  if (!check(env, ctx, bg_flush_profiles(ctx, nullptr, 0, &n))) return nullptr;
  std::vector<bg_pass_profile> ps(size_t(n > 0 ? n : 1));
  int got = 0;
  if (!check(env, ctx, bg_flush_profiles(ctx, ps.data(), n, &got))) return nullptr;
  napi_value arr;
  napi_create_array_with_length(env, size_t(got), &arr);
  for (int i = 0; i < got && i < n; ++i) {
    napi_value o, label;
    napi_create_object(env, &o);
    napi_create_string_utf8(env, ps[i].label, NAPI_AUTO_LENGTH, &label);
    napi_set_named_property(env, o, "label", label);
    napi_set_named_property(env, o, "gpuMs", number(env, ps[i].gpu_ms));
    napi_set_named_property(env, o, "bytes", number(env, double(ps[i].bytes)));
    napi_set_named_property(env, o, "flops", number(env, double(ps[i].flops)));
    napi_set_element(env, arr, uint32_t(i), o);
  }
  return arr;
}

napi_value Version(napi_env env, napi_callback_info) {
  napi_value s;
  napi_create_string_utf8(env, bg_version(), NAPI_AUTO_LENGTH, &s);
  return s;
}

napi_value Init(napi_env env, napi_value exports) {
  struct {
    const char* name;
    napi_callback fn;
  } fns[] = {
      {"ctxCreate", CtxCreate},       {"ctxDestroy", CtxDestroy},
      {"upload", Upload},             {"materialize", Materialize},
      {"release", Release},           {"handleInfo", HandleInfo},
      {"matmul", Matmul},             {"fusedElementwise", FusedElementwise},
      {"cast", Cast},                 {"flashAttention", FlashAttention},
      {"conv", Conv},
      {"runTensorPlan", RunTensorPlan}, {"aliveHandles", AliveHandles},
      {"materializeAsync", MaterializeAsync}, {"runTensorPlanAsync", RunTensorPlanAsync},
      {"resourceSnapshot", ResourceSnapshot}, {"flushProfiles", FlushProfiles},
      {"version", Version},
  };
  for (auto& f : fns) {
    napi_value v;
    napi_create_function(env, f.name, NAPI_AUTO_LENGTH, f.fn, nullptr, &v);
    napi_set_named_property(env, exports, f.name, v);
  }
  return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, Init)
