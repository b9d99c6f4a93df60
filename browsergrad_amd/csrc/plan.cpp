// Tensor-plan executor: the run_tensor_plan* route of the bridge.
//
// Reference: packages/browsergrad-kernels/src/tensor_plan.ts
//   normalizeTensorGpuPlan  :135-181   (snake_case or camelCase fields)
//   executeTensorGpuPlan    :301-373   (value table, early release)
//   releaseDeadOwnedBuffers :375-409
//   executeStep             :424-707   (per-op lowering)
//   validatePlan            :3173-3195
//   expectAxes / expectReduceSpec / expectFusedOps / expectFusedSoftmaxAxis
//                           :3965-4038
// and the semantic permutation side table of tensor_plan_semantics.ts:
//   parseRequestEnvelope / parseDensePermutationRequest :381-467,
//   verifyPlanProjection / compareShape :313-379.
//
// Every step becomes one (or, for REDUCE over non-trailing axes, two) calls
// of this library's own entry points on the context stream, so a plan runs
// back to back on the GPU with no host round trip until the root is
// materialised.  Values are handles; LOAD / RESHAPE / f32->f32 CAST are
// zero-copy views sharing the producer's allocation (reference-counted), so
// releasing a value at its last use frees memory exactly when the last view
// of it dies -- the reference's buffer-identity liveness rule.
//
// Beyond the reference's op set (which refuses CONST, CMP, WHERE, batched
// MATMUL, broadcasting elementwise inputs and non-f32 values) the executor
// also lowers:
//   CONST            -> fused program {IMM}
//   CMP / WHERE      -> fused programs with numpy broadcasting (bool results)
//   ADD/MUL/DIV with broadcastable (not only equal-numel) inputs
//   MATMUL rank > 2  -> batched GEMM (bg_matmul_ex), numpy batch broadcasting
//   CAST between f32 / f16 / bf16 / bool
// LAYER_NORM_BACKWARD_{INPUT,WEIGHT,BIAS}, SGD_UPDATE, ADAMW_UPDATE_{M,V,PARAM}
// and ADAM_UPDATE_{M,V,PARAM} lower onto bg_layer_norm_backward_* and
// bg_optimizer_update; CONV1D*, CONV2D*, CONV3D* and CONV_TRANSPOSE2D* onto
// bg_conv_ex (all f32 only, as in the reference).
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <initializer_list>
#include <set>
#include <string>
#include <unordered_map>
#include <vector>

#include "core.h"
#include "plan.h"

namespace bg {
namespace {

// ---- a small JSON reader ---------------------------------------------------

class JsonReader {
 public:
  explicit JsonReader(const char* s, const char* what) : p_(s), what_(what) {}
  JVal parse() {
    JVal v = value(0);
    ws();
    if (*p_) err("trailing characters");
    return v;
  }

 private:
  const char* p_;
  const char* what_;

  [[noreturn]] void err(const char* m) { fail(BG_E_INVALID, std::string(what_) + " must be valid JSON: " + m); }
  void ws() {
    while (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r') ++p_;
  }
  bool lit(const char* w) {
    size_t n = std::strlen(w);
    if (std::strncmp(p_, w, n) == 0) {
      p_ += n;
      return true;
    }
    return false;
  }
  JVal value(int depth) {
    if (depth > 64) err("nesting too deep");
    ws();
    JVal v;
    if (*p_ == '{') {
      ++p_;
      v.kind = JVal::Obj;
      ws();
      if (*p_ == '}') {
        ++p_;
        return v;
      }
      for (;;) {
        ws();
        if (*p_ != '"') err("object key expected");
        std::string k = string();
        ws();
        if (*p_ != ':') err("':' expected");
        ++p_;
        v.obj.emplace_back(std::move(k), value(depth + 1));
        ws();
        if (*p_ == ',') {
          ++p_;
          continue;
        }
        if (*p_ == '}') {
          ++p_;
          return v;
        }
        err("',' or '}' expected");
      }
    }
    if (*p_ == '[') {
      ++p_;
      v.kind = JVal::Arr;
      ws();
      if (*p_ == ']') {
        ++p_;
        return v;
      }
      for (;;) {
        v.arr.push_back(value(depth + 1));
        ws();
        if (*p_ == ',') {
          ++p_;
          continue;
        }
        if (*p_ == ']') {
          ++p_;
          return v;
        }
        err("',' or ']' expected");
      }
    }
    if (*p_ == '"') {
      v.kind = JVal::Str;
      v.str = string();
      return v;
    }
    if (lit("true")) {
      v.kind = JVal::Bool;
      v.b = true;
      return v;
    }
    if (lit("false")) {
      v.kind = JVal::Bool;
      return v;
    }
    if (lit("null")) return v;
    // Python's json.dumps writes these for non-finite floats.
    if (lit("NaN")) {
      v.kind = JVal::Num;
      v.num = NAN;
      return v;
    }
    if (lit("Infinity")) {
      v.kind = JVal::Num;
      v.num = INFINITY;
      return v;
    }
    if (lit("-Infinity")) {
      v.kind = JVal::Num;
      v.num = -INFINITY;
      return v;
    }
    const char* start = p_;
    if (*p_ == '-') ++p_;
    if (!(*p_ >= '0' && *p_ <= '9')) err("value expected");
    bool integral = true;
    while ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' || *p_ == 'E' || *p_ == '+' || *p_ == '-') {
      if (*p_ == '.' || *p_ == 'e' || *p_ == 'E') integral = false;
      ++p_;
    }
    v.kind = JVal::Num;
    v.num = std::strtod(std::string(start, p_).c_str(), nullptr);
    v.is_int = integral;
    return v;
  }
  std::string string() {
    ++p_;  // opening quote
    std::string out;
    while (*p_ && *p_ != '"') {
      if (*p_ == '\\') {
        ++p_;
        switch (*p_) {
          case '"': out += '"'; break;
          case '\\': out += '\\'; break;
          case '/': out += '/'; break;
          case 'b': out += '\b'; break;
          case 'f': out += '\f'; break;
          case 'n': out += '\n'; break;
          case 'r': out += '\r'; break;
          case 't': out += '\t'; break;
          case 'u': {
            unsigned cp = 0;
            for (int i = 1; i <= 4; ++i) {
              char c = p_[i];
              cp <<= 4;
              if (c >= '0' && c <= '9') cp |= unsigned(c - '0');
              else if (c >= 'a' && c <= 'f') cp |= unsigned(c - 'a' + 10);
              else if (c >= 'A' && c <= 'F') cp |= unsigned(c - 'A' + 10);
              else err("bad \\u escape");
            }
            p_ += 4;
            if (cp < 0x80) out += char(cp);
            else if (cp < 0x800) {
              out += char(0xC0 | (cp >> 6));
              out += char(0x80 | (cp & 0x3F));
            } else {
              out += char(0xE0 | (cp >> 12));
              out += char(0x80 | ((cp >> 6) & 0x3F));
              out += char(0x80 | (cp & 0x3F));
            }
            break;
          }
          default: err("bad escape");
        }
        ++p_;
      } else {
        out += *p_++;
      }
    }
    if (*p_ != '"') err("unterminated string");
    ++p_;
    return out;
  }
};

[[noreturn]] void plan_fail(const std::string& m, int code = BG_E_INVALID) { fail(code, "tensor plan " + m); }

// Integers travel as JSON numbers (doubles): only those a double holds
// exactly (|x| <= 2^53) are accepted, so the conversion is always defined.
int64_t expect_int(const JVal* v, const std::string& name) {
  if (!v || v->kind != JVal::Num || !std::isfinite(v->num) || v->num != std::floor(v->num) ||
      std::fabs(v->num) > 9007199254740992.0)
    fail(BG_E_INVALID, name + " must be an integer (|x| <= 2^53)");
  return int64_t(v->num);
}

const JVal& expect_arr(const JVal* v, const std::string& name) {
  if (!v || v->kind != JVal::Arr) fail(BG_E_INVALID, name + " must be an array");
  return *v;
}

std::vector<int64_t> int_list(const JVal* v, const std::string& name) {
  const JVal& a = expect_arr(v, name);
  std::vector<int64_t> out;
  for (size_t i = 0; i < a.arr.size(); ++i) out.push_back(expect_int(&a.arr[i], name + "[" + std::to_string(i) + "]"));
  return out;
}

// Value dtypes this executor handles.  The reference accepts "float32" only
// (expectFloat32, tensor_plan.ts:4040-4043); the others are extensions.
int plan_dtype(const std::string& s, const std::string& where) {
  if (s == "float32") return BG_F32;
  if (s == "float16") return BG_F16;
  if (s == "bfloat16") return BG_BF16;
  if (s == "bool") return BG_BOOL;
  fail(BG_E_DTYPE, where + " must be \"float32\" (or float16 / bfloat16 / bool), got \"" + s + "\"");
}

Plan normalize(const JVal& root) {
  if (root.kind != JVal::Obj) plan_fail("must be an object");
  Plan p;
  const JVal& steps = expect_arr(root.get("steps"), "tensor plan.steps");
  for (size_t i = 0; i < steps.arr.size(); ++i) {
    const JVal& s = steps.arr[i];
    const std::string at = "steps[" + std::to_string(i) + "]";
    if (s.kind != JVal::Obj) fail(BG_E_INVALID, "tensor plan." + at + " must be an object");
    Step st;
    st.step = expect_int(s.get("step"), at + ".step");
    st.value_id = expect_int(s.get2("value_id", "valueId"), at + ".valueId");
    const JVal* op = s.get("op");
    if (!op || op->kind != JVal::Str) fail(BG_E_INVALID, at + ".op must be a string");
    st.op = op->str;
    if (st.op.find('+') != std::string::npos)
      fail(BG_E_INVALID, at + ".op \"" + st.op + "\" is not a plan opcode");
    st.inputs = int_list(s.get2("input_ids", "inputIds"), at + ".inputIds");
    st.shape = int_list(s.get("shape"), at + ".shape");
    if (st.shape.size() > BG_MAX_RANK)
      fail(BG_E_INVALID, at + ".shape has rank " + std::to_string(st.shape.size()) + ", above " +
                             std::to_string(BG_MAX_RANK));
    for (int64_t d : st.shape)
      if (d < 0) fail(BG_E_INVALID, at + ".shape has a negative extent");
    const JVal* dt = s.get("dtype");
    if (!dt || dt->kind != JVal::Str) fail(BG_E_INVALID, at + ".dtype must be a string");
    st.dtype = dt->str;
    // float64 appears only on constants (NumPy scalars before AMP's CAST);
    // they are held as float32, which is what the CAST that reads them yields.
    if (!(st.op == "CONST" && st.dtype == "float64")) plan_dtype(st.dtype, at + ".dtype");
    st.arg = s.get("arg");
    p.steps.push_back(std::move(st));
  }
  // buffers[] carries liveness metadata the executor recomputes from steps;
  // it is still validated for shape like the reference does.
  expect_arr(root.get("buffers"), "tensor plan.buffers");
  p.root_id = expect_int(root.get2("root_id", "rootId"), "tensor plan.rootId");
  const JVal* mb = root.get2("materialization_boundary", "materializationBoundary");
  if (!mb || mb->kind != JVal::Str || mb->str != "root")
    fail(BG_E_INVALID, "tensor plan.materializationBoundary must be \"root\"");
  p.peak_live_bytes = expect_int(root.get2("peak_live_bytes", "peakLiveBytes"), "tensor plan.peakLiveBytes");
  const JVal* hc = root.get2("has_custom_ops", "hasCustomOps");
  if (!hc || hc->kind != JVal::Bool || hc->b) fail(BG_E_INVALID, "tensor plan.hasCustomOps must be false");
  // validatePlan (tensor_plan.ts:3173-3195)
  std::set<int64_t> seen;
  for (const Step& st : p.steps) {
    if (seen.count(st.value_id)) plan_fail("value " + std::to_string(st.value_id) + " produced twice");
    for (int64_t in : st.inputs)
      if (!seen.count(in))
        plan_fail("step " + std::to_string(st.step) + " reads " + std::to_string(in) + " before production");
    seen.insert(st.value_id);
  }
  if (!seen.count(p.root_id)) plan_fail("root " + std::to_string(p.root_id) + " missing from steps");
  return p;
}

// ---- semantic permutation requests (tensor_plan_semantics.ts:381-467) ------

struct PermRequest {
  int64_t value_id;
  std::vector<int64_t> input_shape;
  std::vector<int64_t> axes;
};

[[noreturn]] void sem_fail(const std::string& path, const std::string& m) {
  fail(BG_E_INVALID, "tensor plan semantic requests " + path + ": " + m);
}

void expect_closed(const JVal& v, std::vector<std::string> keys, const std::string& path) {
  if (v.kind != JVal::Obj) sem_fail(path, "expected an object");
  std::vector<std::string> actual;
  for (const auto& kv : v.obj) actual.push_back(kv.first);
  std::sort(actual.begin(), actual.end());
  std::sort(keys.begin(), keys.end());
  if (actual != keys) {
    std::string all;
    for (size_t i = 0; i < keys.size(); ++i) all += (i ? ", " : "") + keys[i];
    sem_fail(path, "expected closed fields " + all);
  }
}

int64_t safe_int(const JVal* v, const std::string& path) {
  if (!v || v->kind != JVal::Num || !v->is_int || std::fabs(v->num) > 9007199254740991.0)
    sem_fail(path, "expected a safe integer");
  return int64_t(v->num);
}

// A WireI64 is canonical base-10 ASCII in a JSON string.
int64_t wire_i64(const JVal& v, const std::string& path) {
  const std::string& s = v.str;
  bool ok = v.kind == JVal::Str && !s.empty();
  if (ok) {
    size_t i = s[0] == '-' ? 1 : 0;
    ok = i < s.size() && !(s[i] == '0' && s.size() > i + 1) && !(s == "-0");
    for (size_t j = i; ok && j < s.size(); ++j) ok = s[j] >= '0' && s[j] <= '9';
    ok = ok && s.size() <= 20;
  }
  if (!ok)
    fail(BG_E_INVALID, "tensor plan semantic requests " + path +
                           ": WireI64 must be canonical ASCII base-10 without +, whitespace, leading zeroes, or -0");
  const long double x = std::strtold(s.c_str(), nullptr);
  if (x <= 0 || x > 9007199254740991.0L)
    sem_fail(path, "extent must be positive and exactly representable by the frozen plan");
  return int64_t(x);
}

std::vector<PermRequest> parse_requests(const char* text) {
  if (std::strlen(text) > 512 * 1024) sem_fail("$", "JSON request envelope exceeds 524288 code units");
  JVal env = JsonReader(text, "tensor plan semantic requests").parse();
  expect_closed(env, {"schema", "version", "requests"}, "$");
  const JVal* schema = env.get("schema");
  if (schema->kind != JVal::Str || schema->str != "browsergrad.jit.tensor-plan-semantic-requests")
    sem_fail("$.schema", "expected browsergrad.jit.tensor-plan-semantic-requests");
  const JVal* ver = env.get("version");
  expect_closed(*ver, {"major", "minor"}, "$.version");
  if (ver->get("major")->kind != JVal::Num || ver->get("major")->num != 1 ||
      ver->get("minor")->kind != JVal::Num || ver->get("minor")->num != 0)
    sem_fail("$.version", "only semantic request version 1.0 is supported");
  const JVal* reqs = env.get("requests");
  if (reqs->kind != JVal::Arr) sem_fail("$.requests", "requests must be an array");
  if (reqs->arr.size() > 4096) sem_fail("$.requests", "request count exceeds 4096");
  std::vector<PermRequest> out;
  for (size_t i = 0; i < reqs->arr.size(); ++i) {
    const std::string path = "$.requests[" + std::to_string(i) + "]";
    const JVal& r = reqs->arr[i];
    expect_closed(r, {"kind", "valueId", "inputShape", "axes", "dtype"}, path);
    if (r.get("kind")->kind != JVal::Str || r.get("kind")->str != "dense-permutation-view-copy")
      sem_fail(path + ".kind", "expected dense-permutation-view-copy");
    PermRequest q;
    q.value_id = safe_int(r.get("valueId"), path + ".valueId");
    if (q.value_id < 0) sem_fail(path + ".valueId", "valueId must be non-negative");
    if (r.get("dtype")->kind != JVal::Str || r.get("dtype")->str != "f32")
      sem_fail(path + ".dtype", "initial semantic permutation request requires f32");
    const JVal* is = r.get("inputShape");
    if (is->kind != JVal::Arr) sem_fail(path + ".inputShape", "inputShape must be an array");
    if (is->arr.size() != 2 && is->arr.size() != 3)
      sem_fail(path + ".inputShape", "initial semantic permutation request requires rank 2 or 3");
    for (size_t a = 0; a < is->arr.size(); ++a)
      q.input_shape.push_back(wire_i64(is->arr[a], path + ".inputShape[" + std::to_string(a) + "]"));
    const JVal* ax = r.get("axes");
    if (ax->kind != JVal::Arr || ax->arr.size() != q.input_shape.size())
      sem_fail(path + ".axes", "axes must contain exactly one entry per input rank");
    std::set<int64_t> seen;
    for (size_t a = 0; a < ax->arr.size(); ++a) {
      int64_t v = safe_int(&ax->arr[a], path + ".axes[" + std::to_string(a) + "]");
      if (v < 0 || v >= int64_t(q.input_shape.size()) || seen.count(v))
        sem_fail(path + ".axes", "axes must be an exact non-negative permutation");
      seen.insert(v);
      q.axes.push_back(v);
    }
    out.push_back(std::move(q));
  }
  return out;
}

// The request side table must match the plan's PERMUTE steps one to one, in
// order, with the legacy axes erased from the plan (verifyPlanProjection).
std::unordered_map<int64_t, std::vector<int64_t>> bind_requests(const Plan& p, const std::vector<PermRequest>& reqs) {
  std::vector<const Step*> perms;
  std::unordered_map<int64_t, const Step*> by_id;
  for (const Step& s : p.steps) {
    by_id[s.value_id] = &s;
    if (s.op == "PERMUTE") perms.push_back(&s);
  }
  if (reqs.size() != perms.size())
    sem_fail("$.requests", "expected exactly " + std::to_string(perms.size()) +
                               " request(s) for plan PERMUTE steps, got " + std::to_string(reqs.size()));
  std::unordered_map<int64_t, std::vector<int64_t>> axes;
  for (size_t i = 0; i < reqs.size(); ++i) {
    const std::string path = "$.requests[" + std::to_string(i) + "]";
    const PermRequest& q = reqs[i];
    const Step& st = *perms[i];
    if (q.value_id != st.value_id)
      sem_fail(path + ".valueId", "request order/valueId must match plan PERMUTE value " + std::to_string(st.value_id));
    if (st.inputs.size() != 1) sem_fail(path + ".valueId", "plan PERMUTE must have exactly one input");
    auto src = by_id.find(st.inputs[0]);
    if (src == by_id.end()) sem_fail(path + ".valueId", "plan PERMUTE source is missing");
    if (src->second->dtype != "float32" || st.dtype != "float32")
      sem_fail(path + ".dtype", "plan projection must remain float32");
    if (st.arg && st.arg->kind != JVal::Null)
      sem_fail(path + ".valueId", "semantic-route PERMUTE must erase legacy arg meaning from the scheduling plan");
    auto cmp = [&](const std::vector<int64_t>& sem, const std::vector<int64_t>& plan, const std::string& where) {
      if (sem.size() != plan.size()) sem_fail(where, "semantic request and plan projection ranks differ");
      for (size_t a = 0; a < sem.size(); ++a) {
        if (plan[a] <= 0) sem_fail(where, "plan extent " + std::to_string(a) + " must be a positive safe integer");
        if (sem[a] != plan[a])
          sem_fail(where, "semantic request and plan projection differ at axis " + std::to_string(a));
      }
    };
    cmp(q.input_shape, src->second->shape, path + ".inputShape");
    std::vector<int64_t> expect_out;
    for (int64_t a : q.axes) expect_out.push_back(q.input_shape[size_t(a)]);
    cmp(expect_out, st.shape, path + ".axes");
    axes[st.value_id] = q.axes;
  }
  return axes;
}

// ---- argument rules of the LayerNorm and optimizer steps ----------------------

// expectShape (tensor_plan.ts:3215-3226).
void expect_shape(const std::vector<int64_t>& actual, const std::vector<int64_t>& expected,
                  const std::string& name) {
  auto str = [](const std::vector<int64_t>& v) {
    std::string r = "[";
    for (size_t i = 0; i < v.size(); ++i) r += (i ? "," : "") + std::to_string(v[i]);
    return r + "]";
  };
  if (actual.size() != expected.size())
    fail(BG_E_SHAPE, name + " expected rank " + std::to_string(expected.size()) + ", got " + str(actual));
  for (size_t i = 0; i < expected.size(); ++i)
    if (actual[i] != expected[i])
      fail(BG_E_SHAPE, name + " shape mismatch at dim " + std::to_string(i) + ": expected " +
                           std::to_string(expected[i]) + ", got " + std::to_string(actual[i]));
}

// The first of `keys` present and not null, else nullptr (JavaScript's `??`
// chain over snake_case then camelCase spellings).
const JVal* first_of(const JVal& arg, std::initializer_list<const char*> keys) {
  for (const char* k : keys)
    if (const JVal* v = arg.get(k); v && v->kind != JVal::Null) return v;
  return nullptr;
}

// expectFiniteNumber with a default for an absent field (tensor_plan.ts:3948-3953).
double finite_or(const JVal* v, double dflt, bool required, const std::string& name) {
  if (!v) {
    if (required) fail(BG_E_INVALID, name + " must be a finite number");
    return dflt;
  }
  if (v->kind != JVal::Num || !std::isfinite(v->num)) fail(BG_E_INVALID, name + " must be a finite number");
  return v->num;
}

const JVal& arg_object(const JVal* arg, const std::string& op) {
  if (!arg || arg->kind != JVal::Obj) plan_fail(op + ".arg must be an object");
  return *arg;
}

struct LnArg {
  std::vector<int64_t> normalized_shape;
  int64_t rows = 0, cols = 0;
  float eps = 1e-5f;
};

// expectLayerNormArg (tensor_plan.ts:3829-3852).
LnArg ln_arg(const Step& s) {
  const JVal& arg = arg_object(s.arg, s.op);
  LnArg a;
  const JVal* ns = first_of(arg, {"normalized_shape", "normalizedShape"});
  if (!ns || ns->kind != JVal::Arr) fail(BG_E_INVALID, s.op + ".normalized_shape must be an array");
  for (size_t i = 0; i < ns->arr.size(); ++i)
    a.normalized_shape.push_back(expect_int(&ns->arr[i], s.op + ".normalized_shape[" + std::to_string(i) + "]"));
  a.rows = expect_int(arg.get("rows"), s.op + ".rows");
  a.cols = expect_int(arg.get("cols"), s.op + ".cols");
  const double eps = finite_or(first_of(arg, {"eps"}), 1e-5, false, s.op + ".eps");
  if (a.normalized_shape.empty()) plan_fail(s.op + ".normalized_shape must be non-empty");
  if (a.rows <= 0 || a.cols <= 0) plan_fail(s.op + ".rows and cols must be positive");
  if (numel(a.normalized_shape) != a.cols) plan_fail(s.op + ".cols must equal normalized_shape numel");
  if (eps <= 0) plan_fail(s.op + ".eps must be > 0");
  a.eps = float(eps);
  return a;
}

int optim_kind(const std::string& op) {
  static const char* names[7] = {"SGD_UPDATE",    "ADAMW_UPDATE_M", "ADAMW_UPDATE_V", "ADAMW_UPDATE_PARAM",
                                 "ADAM_UPDATE_M", "ADAM_UPDATE_V",  "ADAM_UPDATE_PARAM"};
  for (int k = 0; k < 7; ++k)
    if (op == names[k]) return k;
  return -1;
}

// expectSgdUpdateArg / expectAdamwUpdateArg / expectAdamUpdateArg
// (tensor_plan.ts:3776-3827): SGD needs lr; AdamW needs beta1, beta2 and
// step (lr 0.001, eps 1e-8 by default); Adam defaults every field (lr 0.001,
// betas 0.9 / 0.999, eps 1e-8, step 1); weight_decay defaults to 0.
bg_optim_args optim_arg(const Step& s, int kind) {
  const JVal& arg = arg_object(s.arg, s.op);
  const std::string& op = s.op;
  bg_optim_args a{};
  const double wd = finite_or(first_of(arg, {"weight_decay", "weightDecay"}), 0.0, false, op + ".weight_decay");
  if (kind == BG_OPT_SGD) {
    a.lr = finite_or(first_of(arg, {"lr"}), 0, true, "SGD_UPDATE.lr");
    a.weight_decay = wd;
    if (a.lr < 0) plan_fail("SGD_UPDATE.lr must be >= 0");
    a.beta1 = a.beta2 = a.eps = 0;
    a.step = 1;
    return a;
  }
  const bool adamw = kind <= BG_OPT_ADAMW_PARAM;
  a.lr = finite_or(first_of(arg, {"lr"}), 0.001, false, op + ".lr");
  a.beta1 = finite_or(first_of(arg, {"beta1"}), 0.9, adamw, op + ".beta1");
  a.beta2 = finite_or(first_of(arg, {"beta2"}), 0.999, adamw, op + ".beta2");
  a.eps = finite_or(first_of(arg, {"eps"}), 1e-8, false, op + ".eps");
  a.weight_decay = wd;
  const JVal* st = first_of(arg, {"step"});
  if (!st && !adamw) {
    a.step = 1;
  } else {
    a.step = expect_int(st, op + ".step");
  }
  if (a.lr < 0) plan_fail(op + ".lr must be >= 0");
  if (a.step <= 0) plan_fail(op + ".step must be >= 1");
  return a;
}

// ---- convolution steps (tensor_plan.ts:554-641, 2321-2830, 3228-3775) --------

struct ConvStep {
  int spatial = 0;
  bool transposed = false;
  int op = 0;  // BG_CONV_*
};

// CONV1D*, CONV2D*, CONV3D*, CONV_TRANSPOSE2D* -> (rank, transposed, op);
// spatial 0 for any other op.
ConvStep conv_step(const std::string& op) {
  ConvStep c;
  std::string base = op;
  static const std::pair<const char*, int> suffixes[] = {
      {"_BACKWARD_INPUT", BG_CONV_BACKWARD_INPUT},
      {"_BACKWARD_WEIGHT", BG_CONV_BACKWARD_WEIGHT},
      {"_BACKWARD_BIAS", BG_CONV_BACKWARD_BIAS}};
  for (const auto& sf : suffixes) {
    const std::string suf = sf.first;
    if (base.size() > suf.size() && base.compare(base.size() - suf.size(), suf.size(), suf) == 0) {
      base = base.substr(0, base.size() - suf.size());
      c.op = sf.second;
      break;
    }
  }
  if (base == "CONV1D") c.spatial = 1;
  else if (base == "CONV2D") c.spatial = 2;
  else if (base == "CONV3D") c.spatial = 3;
  else if (base == "CONV_TRANSPOSE2D") {
    c.spatial = 2;
    c.transposed = true;
  }
  return c;
}

struct ConvArg {
  std::unordered_map<std::string, int64_t> v;
  int64_t operator[](const char* k) const { return v.at(k); }
};

// expectConv1dArg / expectConv2dArg / expectConvTranspose2dArg /
// expectConv3dArg followed by the matching validate*Shape: every field an
// integer (in the interface's order), sizes positive, padding non-negative,
// the channel rule of the family.
ConvArg conv_arg(const Step& s, const ConvStep& c) {
  const JVal& arg = arg_object(s.arg, s.op);
  const std::string& op = s.op;
  static const std::vector<std::string> k1 = {"n", "c_in", "l_in", "c_out", "k", "stride", "padding", "dilation",
                                              "groups", "l_out"};
  static const std::vector<std::string> k2 = {"n", "c_in", "h", "w", "c_out", "kh", "kw", "stride_h", "stride_w",
                                              "pad_h", "pad_w", "dilation_h", "dilation_w", "groups", "out_h",
                                              "out_w"};
  static const std::vector<std::string> kt = {"n", "c_in", "h", "w", "c_out", "c_out_per_group", "kh", "kw",
                                              "stride_h", "stride_w", "pad_h", "pad_w", "output_pad_h",
                                              "output_pad_w", "dilation_h", "dilation_w", "groups", "out_h",
                                              "out_w"};
  static const std::vector<std::string> k3 = {"n", "c_in", "d", "h", "w", "c_out", "kd", "kh", "kw", "stride_d",
                                              "stride_h", "stride_w", "pad_d", "pad_h", "pad_w", "dilation_d",
                                              "dilation_h", "dilation_w", "groups", "out_d", "out_h", "out_w"};
  const std::vector<std::string>& keys = c.transposed ? kt : c.spatial == 1 ? k1 : c.spatial == 2 ? k2 : k3;
  ConvArg a;
  for (const std::string& k : keys) a.v[k] = expect_int(arg.get(k.c_str()), op + "." + k);
  // validate*Shape: positive sizes under their camelCase names.
  static const std::vector<std::pair<const char*, const char*>> p1 = {
      {"n", "n"}, {"c_in", "cIn"}, {"l_in", "lIn"}, {"c_out", "cOut"}, {"k", "k"}, {"stride", "stride"},
      {"dilation", "dilation"}, {"groups", "groups"}, {"l_out", "lOut"}};
  static const std::vector<std::pair<const char*, const char*>> p2 = {
      {"n", "n"}, {"c_in", "cIn"}, {"h", "h"}, {"w", "w"}, {"c_out", "cOut"}, {"kh", "kh"}, {"kw", "kw"},
      {"stride_h", "strideH"}, {"stride_w", "strideW"}, {"dilation_h", "dilationH"},
      {"dilation_w", "dilationW"}, {"groups", "groups"}, {"out_h", "outH"}, {"out_w", "outW"}};
  static const std::vector<std::pair<const char*, const char*>> pt = {
      {"n", "n"}, {"c_in", "cIn"}, {"h", "h"}, {"w", "w"}, {"c_out", "cOut"},
      {"c_out_per_group", "cOutPerGroup"}, {"kh", "kh"}, {"kw", "kw"}, {"stride_h", "strideH"},
      {"stride_w", "strideW"}, {"dilation_h", "dilationH"}, {"dilation_w", "dilationW"}, {"groups", "groups"},
      {"out_h", "outH"}, {"out_w", "outW"}};
  static const std::vector<std::pair<const char*, const char*>> p3 = {
      {"n", "n"}, {"c_in", "cIn"}, {"d", "d"}, {"h", "h"}, {"w", "w"}, {"c_out", "cOut"}, {"kd", "kd"},
      {"kh", "kh"}, {"kw", "kw"}, {"stride_d", "strideD"}, {"stride_h", "strideH"}, {"stride_w", "strideW"},
      {"dilation_d", "dilationD"}, {"dilation_h", "dilationH"}, {"dilation_w", "dilationW"},
      {"groups", "groups"}, {"out_d", "outD"}, {"out_h", "outH"}, {"out_w", "outW"}};
  const auto& pos = c.transposed ? pt : c.spatial == 1 ? p1 : c.spatial == 2 ? p2 : p3;
  for (const auto& kv : pos)
    if (a[kv.first] <= 0) plan_fail(op + "." + kv.second + " must be a positive integer");
  if (c.spatial == 1) {
    if (a["padding"] < 0) plan_fail(op + ".padding must be a non-negative integer");
  } else {
    for (const char* k : {"pad_d", "pad_h", "pad_w"})
      if (a.v.count(k) && a[k] < 0) plan_fail(op + " padding must be non-negative integers");
  }
  if (c.transposed) {
    if (a["output_pad_h"] < 0 || a["output_pad_w"] < 0)
      plan_fail(op + " output_padding must be non-negative integers");
    if (a["c_in"] % a["groups"] != 0 || a["c_out"] != a["c_out_per_group"] * a["groups"])
      plan_fail(op + " channels must match groups");
    if (a["output_pad_h"] >= a["stride_h"] || a["output_pad_w"] >= a["stride_w"])
      plan_fail(op + " output_padding must be smaller than stride");
  } else if (a["c_in"] % a["groups"] != 0 || a["c_out"] % a["groups"] != 0) {
    plan_fail(op + " channels must be divisible by groups");
  }
  return a;
}

// ---- plan-level fusion --------------------------------------------------------

const char* const kAdamwFused = "ADAMW_UPDATE_M+V+PARAM";
const char* const kAdamFused = "ADAM_UPDATE_M+V+PARAM";

// An ADAMW_UPDATE_PARAM step whose m and v inputs come from ADAMW_UPDATE_M and
// ADAMW_UPDATE_V steps over the same gradient, read by nothing else and not
// the root, becomes one step over (param, grad, m, v): one pass reading 16 B
// and writing 4 B per parameter instead of three passes moving 44 B, with the
// same float32 operations in the same order.
void fuse_adamw(Plan& plan) {
  std::unordered_map<int64_t, int> uses;
  std::unordered_map<int64_t, size_t> producer;
  for (size_t i = 0; i < plan.steps.size(); ++i) {
    for (int64_t in : plan.steps[i].inputs) uses[in]++;
    producer[plan.steps[i].value_id] = i;
  }
  std::vector<bool> drop(plan.steps.size(), false);
  for (Step& p : plan.steps) {
    if (p.op == "ADAM_UPDATE_PARAM" && p.inputs.size() == 3) {
      // Adam: M and V read (param, grad, moment); PARAM reads (param, m', v').
      const int64_t param = p.inputs[0], m_id = p.inputs[1], v_id = p.inputs[2];
      if (m_id == plan.root_id || v_id == plan.root_id || uses[m_id] != 1 || uses[v_id] != 1) continue;
      auto pm = producer.find(m_id), pv = producer.find(v_id);
      if (pm == producer.end() || pv == producer.end()) continue;
      const Step& sm = plan.steps[pm->second];
      const Step& sv = plan.steps[pv->second];
      if (sm.op != "ADAM_UPDATE_M" || sv.op != "ADAM_UPDATE_V" || sm.inputs.size() != 3 ||
          sv.inputs.size() != 3 || sm.inputs[0] != param || sv.inputs[0] != param ||
          sm.inputs[1] != sv.inputs[1])
        continue;
      p.arg_m = sm.arg;
      p.arg_v = sv.arg;
      p.inputs = {param, sm.inputs[1], sm.inputs[2], sv.inputs[2]};
      p.op = kAdamFused;
      drop[pm->second] = drop[pv->second] = true;
      continue;
    }
    if (p.op != "ADAMW_UPDATE_PARAM" || p.inputs.size() != 4) continue;
    const int64_t grad = p.inputs[1], m_id = p.inputs[2], v_id = p.inputs[3];
    if (m_id == plan.root_id || v_id == plan.root_id || uses[m_id] != 1 || uses[v_id] != 1) continue;
    auto pm = producer.find(m_id), pv = producer.find(v_id);
    if (pm == producer.end() || pv == producer.end()) continue;
    const Step& sm = plan.steps[pm->second];
    const Step& sv = plan.steps[pv->second];
    if (sm.op != "ADAMW_UPDATE_M" || sv.op != "ADAMW_UPDATE_V" || sm.inputs.size() != 2 ||
        sv.inputs.size() != 2 || sm.inputs[1] != grad || sv.inputs[1] != grad)
      continue;
    p.arg_m = sm.arg;
    p.arg_v = sv.arg;
    p.inputs = {p.inputs[0], grad, sm.inputs[0], sv.inputs[0]};
    p.op = kAdamwFused;
    drop[pm->second] = drop[pv->second] = true;
  }
  std::vector<Step> kept;
  for (size_t i = 0; i < plan.steps.size(); ++i)
    if (!drop[i]) kept.push_back(std::move(plan.steps[i]));
  plan.steps = std::move(kept);
}

// ---- execution -------------------------------------------------------------

struct Runner {
  bg_ctx* ctx;
  std::unordered_map<int64_t, bg_handle> vals;   // value_id -> handle
  std::set<bg_handle> owned;                     // handles this run minted
  std::set<bg_handle> inputs;                    // caller's handles (borrowed)
  const std::unordered_map<int64_t, std::vector<int64_t>>* sem_axes = nullptr;

  void call(int rc) {
    if (rc != BG_OK) fail(rc, ctx->err);
  }
  bg_handle own(bg_handle h) {
    owned.insert(h);
    return h;
  }
  bg_handle need(const Step& s, size_t i) {
    if (i >= s.inputs.size()) plan_fail(s.op + " missing input");
    auto it = vals.find(s.inputs[i]);
    if (it == vals.end()) plan_fail(s.op + " input " + std::to_string(s.inputs[i]) + " not resident");
    return it->second;
  }
  const Record& rec(bg_handle h) { return ctx->handles.at(h); }

  bg_handle view(bg_handle src, const std::vector<int64_t>& shape) {
    bg_handle out = 0;
    call(bg_reshape(ctx, src, shape.data(), int(shape.size()), &out));
    return own(out);
  }

  // numpy broadcasting strides of `in` against output shape `out`.
  static std::vector<int64_t> bstrides(const std::vector<int64_t>& in, const std::vector<int64_t>& out,
                                       const std::string& op) {
    if (in.size() > out.size()) plan_fail(op + " input rank exceeds output rank");
    std::vector<int64_t> st(out.size(), 0);
    int64_t stride = 1;
    for (size_t k = 0; k < in.size(); ++k) {
      size_t ii = in.size() - 1 - k, oo = out.size() - 1 - k;
      if (in[ii] == out[oo]) st[oo] = in[ii] == 1 ? 0 : stride;
      else if (in[ii] == 1) st[oo] = 0;
      else plan_fail(op + " incompatible broadcast dim " + std::to_string(ii));
      stride *= in[ii];
    }
    return st;
  }

  bg_handle fused(const Step& s, std::vector<bg_handle> ins, const std::vector<bg_fused_op>& ops,
                  const std::vector<double>& imms, int out_dtype, int reduce_op = BG_RED_NONE,
                  bool keepdims = false) {
    std::vector<int64_t> strides;
    bool all_equal = true;
    for (bg_handle h : ins)
      if (rec(h).numel() != numel(s.shape)) all_equal = false;
    if (!all_equal)
      for (bg_handle h : ins) {
        auto st = bstrides(rec(h).shape, s.shape, s.op);
        strides.insert(strides.end(), st.begin(), st.end());
      }
    bg_fused_desc d{};
    d.n_inputs = int(ins.size());
    d.inputs = ins.data();
    d.in_strides = all_equal ? nullptr : strides.data();
    d.n_ops = int(ops.size());
    d.ops = ops.data();
    d.n_imms = int(imms.size());
    d.imms = imms.data();
    std::vector<int64_t> shape = s.shape.empty() ? std::vector<int64_t>{1} : s.shape;
    d.rank = int(shape.size());
    d.shape = shape.data();
    d.out_dtype = out_dtype;
    d.reduce_op = reduce_op;
    d.reduce_keepdims = keepdims ? 1 : 0;
    bg_handle out = 0;
    call(bg_fused_ex(ctx, &d, &out));
    if (s.shape.empty()) ctx->handles[out].shape.clear();
    return own(out);
  }

  static int opcode(const std::string& name, const std::string& where) {
    static const std::unordered_map<std::string, int> m = {
        {"ADD", BG_OP_ADD}, {"MUL", BG_OP_MUL}, {"DIV", BG_OP_DIV}, {"NEG", BG_OP_NEG},
        {"EXP", BG_OP_EXP}, {"LOG", BG_OP_LOG},
        // extensions
        {"MAX", BG_OP_MAX}, {"MIN", BG_OP_MIN}, {"SUB", BG_OP_SUB}, {"TANH", BG_OP_TANH},
        {"SQRT", BG_OP_SQRT}, {"ABS", BG_OP_ABS}, {"WHERE", BG_OP_WHERE},
        {"CMP_EQ", BG_OP_CMP_EQ}, {"CMP_NE", BG_OP_CMP_NE}, {"CMP_LT", BG_OP_CMP_LT},
        {"CMP_LE", BG_OP_CMP_LE}, {"CMP_GT", BG_OP_CMP_GT}, {"CMP_GE", BG_OP_CMP_GE}};
    auto it = m.find(name);
    if (it == m.end()) plan_fail(where + " unsupported fused opcode \"" + name + "\"");
    return it->second;
  }

  static int cmp_code(const std::string& c) {
    if (c == "eq") return BG_OP_CMP_EQ;
    if (c == "ne") return BG_OP_CMP_NE;
    if (c == "lt") return BG_OP_CMP_LT;
    if (c == "le") return BG_OP_CMP_LE;
    if (c == "gt") return BG_OP_CMP_GT;
    if (c == "ge") return BG_OP_CMP_GE;
    plan_fail("CMP unknown comparison \"" + c + "\"");
  }

  static std::vector<int64_t> axes_arg(const Step& s, size_t rank) {
    if (!s.arg || s.arg->kind != JVal::Obj) plan_fail(s.op + ".arg must be an object");
    const JVal& a = expect_arr(s.arg->get("axes"), "tensor plan " + s.op + ".arg.axes");
    if (a.arr.size() != rank) plan_fail(s.op + " axes length must equal rank");
    std::vector<int64_t> out;
    std::set<int64_t> seen;
    for (size_t i = 0; i < a.arr.size(); ++i) {
      int64_t n = expect_int(&a.arr[i], "tensor plan " + s.op + ".arg.axes[" + std::to_string(i) + "]");
      if (n < 0 || n >= int64_t(rank))
        plan_fail(s.op + " axis " + std::to_string(n) + " out of range for rank " + std::to_string(rank));
      if (seen.count(n)) plan_fail(s.op + " duplicate axis " + std::to_string(n));
      seen.insert(n);
      out.push_back(n);
    }
    return out;
  }

  bg_handle permute(bg_handle src, const std::vector<int64_t>& axes) {
    const Record& r = rec(src);
    std::vector<int64_t> cstr(r.shape.size(), 1);
    for (int i = int(r.shape.size()) - 2; i >= 0; --i) cstr[i] = cstr[i + 1] * r.shape[i + 1];
    std::vector<int64_t> shape, strides;
    for (int64_t a : axes) {
      shape.push_back(r.shape[size_t(a)]);
      strides.push_back(cstr[size_t(a)]);
    }
    bg_handle out = 0;
    call(bg_copy_strided(ctx, src, 0, shape.data(), strides.data(), int(shape.size()), &out));
    return own(out);
  }

  bg_handle exec(const Step& s) {
    const std::string& op = s.op;
    const int dt = s.op == "CONST" && s.dtype == "float64" ? BG_F32
                                                           : plan_dtype(s.dtype, "steps[" + std::to_string(s.step) + "].dtype");
    if (op == "+PROGRAM") {
      std::vector<bg_handle> ins;
      for (size_t i = 0; i < s.inputs.size(); ++i) ins.push_back(need(s, i));
      Step it = s;  // iteration shape for the broadcast strides
      it.shape = s.iter;
      bg_handle out = fused(it, ins, s.prog, s.imms, dt, s.reduce_op, s.keepdims);
      ctx->handles[out].shape = s.shape;
      return out;
    }
    if (op == "+LINEAR") {
      bg_matmul_desc d = s.mm;
      bg_matmul_ext e = s.mm_ext;
      d.a = need(s, 0);
      d.b = need(s, 1);
      size_t nxt = 2;
      if (s.has_bias) d.bias = need(s, nxt++);
      if (s.has_residual) e.residual = need(s, nxt++);
      // An operand already held in the GEMM's dtype needs no cast (a plan
      // may declare a view's dtype as built rather than as carried).
      if (rec(d.a).dtype == d.in_dtype) e.a_dtype = -1;
      if (rec(d.b).dtype == d.in_dtype) e.b_dtype = -1;
      d.stride_a = d.m * d.lda;
      d.stride_b = (d.trans_b ? d.n : d.k) * d.ldb;
      d.stride_c = d.m * d.ldc;
      bg_handle out = 0;
      call(bg_matmul_ex2(ctx, &d, &e, &out));
      ctx->handles[out].shape = s.shape;
      return own(out);
    }
    if (op == "+ATTENTION") {
      bg_attention_desc d = s.att;
      d.q = need(s, 0);
      d.k = need(s, 1);
      d.v = need(s, 2);
      d.q_ss = d.d;
      d.q_sh = d.sq * d.d;
      d.q_sb = d.heads * d.sq * d.d;
      d.k_ss = d.v_ss = d.d;
      d.k_sh = d.v_sh = d.sk * d.d;
      d.k_sb = d.v_sb = d.heads * d.sk * d.d;
      bg_handle out = 0;
      call(bg_attention_ex(ctx, &d, &out));
      ctx->handles[out].shape = s.shape;
      return own(out);
    }
    if (op == "SLICE") {
      // arg.slices: one [start, stop, step] per axis, step >= 1 (extension).
      bg_handle src = need(s, 0);
      const Record& r = rec(src);
      const JVal& sl = expect_arr(s.arg && s.arg->kind == JVal::Obj ? s.arg->get("slices") : nullptr,
                                  "tensor plan SLICE.arg.slices");
      if (sl.arr.size() != r.shape.size()) plan_fail("SLICE needs one [start, stop, step] per axis");
      std::vector<int64_t> cstr(r.shape.size(), 1);
      for (int i = int(r.shape.size()) - 2; i >= 0; --i) cstr[size_t(i)] = cstr[size_t(i) + 1] * r.shape[size_t(i) + 1];
      int64_t offset = 0;
      std::vector<int64_t> shape, strides;
      for (size_t i = 0; i < sl.arr.size(); ++i) {
        const std::vector<int64_t> t = int_list(&sl.arr[i], "tensor plan SLICE.arg.slices[" + std::to_string(i) + "]");
        if (t.size() != 3 || t[2] < 1 || t[0] < 0 || t[1] < t[0] || t[1] > r.shape[i])
          plan_fail("SLICE axis " + std::to_string(i) + " needs 0 <= start <= stop <= extent and step >= 1");
        offset += t[0] * cstr[i];
        shape.push_back((t[1] - t[0] + t[2] - 1) / t[2]);
        strides.push_back(t[2] * cstr[i]);
      }
      if (shape != s.shape) plan_fail("SLICE output shape differs from the plan");
      bg_handle out = 0;
      call(bg_copy_strided(ctx, src, offset, shape.data(), strides.data(), int(shape.size()), &out));
      return own(out);
    }
    if (op == "CAUSAL_MASK") {
      // The top-left-aligned causal mask of SDPA (extension): bool
      // [.., rows, cols], true where the key index exceeds the query index
      // (numpy.triu(ones, k=1)).  Built on the host when no fused attention
      // absorbed it.
      if (s.shape.size() < 2 || dt != BG_BOOL) plan_fail("CAUSAL_MASK must be a bool matrix");
      const int64_t rows = s.shape[s.shape.size() - 2], cols = s.shape.back();
      const int64_t lead = numel(s.shape) / std::max<int64_t>(rows * cols, 1);
      std::vector<uint8_t> host(size_t(numel(s.shape)));
      for (int64_t b = 0; b < lead; ++b)
        for (int64_t i = 0; i < rows; ++i)
          for (int64_t j = 0; j < cols; ++j) host[size_t((b * rows + i) * cols + j)] = j > i ? 1 : 0;
      bg_handle out = 0;
      call(bg_upload(ctx, host.data(), host.size(), s.shape.data(), int(s.shape.size()), BG_BOOL, &out));
      return own(out);
    }
    if (op == "BUFFER") {
      auto it = vals.find(s.value_id);  // pre-bound by the caller
      if (it == vals.end()) plan_fail("missing BUFFER input " + std::to_string(s.value_id));
      const Record& r = rec(it->second);
      if (r.numel() != numel(s.shape))
        fail(BG_E_SHAPE, "BUFFER " + std::to_string(s.value_id) + " data length " + std::to_string(r.numel()) +
                             " does not match shape (" + std::to_string(numel(s.shape)) + ")");
      if (r.dtype != dt) fail(BG_E_DTYPE, "BUFFER " + std::to_string(s.value_id) + " dtype differs from the plan");
      return it->second;
    }
    if (op == "LOAD" || op == "RESHAPE") {
      bg_handle src = need(s, 0);
      if (rec(src).numel() != numel(s.shape)) plan_fail(op + " cannot change numel");
      return view(src, s.shape);
    }
    if (op == "CAST") {
      bg_handle src = need(s, 0);
      const Record& r = rec(src);
      if (r.dtype == dt) return view(src, s.shape);
      bg_handle out = 0;
      call(bg_cast(ctx, src, r.dtype, dt, s.shape.data(), int(s.shape.size()), &out));
      return own(out);
    }
    if (op == "CONST") {
      if (!s.arg || s.arg->kind != JVal::Obj) plan_fail("CONST.arg must be an object");
      const JVal* v = s.arg->get("value");
      if (!v || (v->kind != JVal::Num && v->kind != JVal::Bool)) plan_fail("CONST.arg.value must be a number");
      double x = v->kind == JVal::Bool ? (v->b ? 1.0 : 0.0) : v->num;
      return fused(s, {}, {{BG_OP_IMM, 0, 0, 0}}, {x}, dt);
    }
    if (op == "ADD" || op == "MUL" || op == "DIV") {
      if (s.inputs.size() != 2) plan_fail(op + " expected 2 inputs");
      return fused(s, {need(s, 0), need(s, 1)}, {{opcode(op, op), -1, -2, 0}}, {}, dt);
    }
    if (op == "NEG" || op == "EXP" || op == "LOG") {
      if (s.inputs.size() != 1) plan_fail(op + " expected 1 inputs");
      return fused(s, {need(s, 0)}, {{opcode(op, op), -1, -1, 0}}, {}, dt);
    }
    if (op == "CMP") {
      if (s.inputs.size() != 2) plan_fail("CMP expected 2 inputs");
      if (!s.arg || s.arg->kind != JVal::Obj || !s.arg->get("op") || s.arg->get("op")->kind != JVal::Str)
        plan_fail("CMP.arg.op must be a string");
      return fused(s, {need(s, 0), need(s, 1)}, {{cmp_code(s.arg->get("op")->str), -1, -2, 0}}, {}, BG_BOOL);
    }
    if (op == "WHERE") {
      if (s.inputs.size() != 3) plan_fail("WHERE expected 3 inputs");
      return fused(s, {need(s, 0), need(s, 1), need(s, 2)}, {{BG_OP_WHERE, -1, -2, -3}}, {}, dt);
    }
    if (op == "FUSED_ELEMENTWISE") {
      if (!s.arg || s.arg->kind != JVal::Obj) plan_fail("FUSED_ELEMENTWISE.arg must be an object");
      const JVal& ops = expect_arr(s.arg->get("ops"), "tensor plan FUSED_ELEMENTWISE.arg.ops");
      std::vector<bg_fused_op> prog;
      for (size_t i = 0; i < ops.arr.size(); ++i) {
        const std::string at = "FUSED_ELEMENTWISE.arg.ops[" + std::to_string(i) + "]";
        const JVal& it = ops.arr[i];
        if (it.kind != JVal::Arr || it.arr.size() < 2 || it.arr.size() > 4)
          plan_fail(at + " must be [opcode, lhs, rhs?]");
        if (it.arr[0].kind != JVal::Str) plan_fail(at + "[0] must be a string");
        int code = opcode(it.arr[0].str, at);
        auto ref32 = [&](const JVal* v, const std::string& name) {
          const int64_t r = expect_int(v, name);
          if (r < -1024 || r > 1024) plan_fail(at + " reference out of range");
          return int32_t(r);
        };
        int32_t a = ref32(&it.arr[1], "tensor plan " + at + "[1]");
        int32_t b = a, c = 0;
        if (it.arr.size() >= 3 && it.arr[2].kind != JVal::Null) b = ref32(&it.arr[2], "tensor plan " + at + "[2]");
        if (it.arr.size() == 4 && it.arr[3].kind != JVal::Null) c = ref32(&it.arr[3], "tensor plan " + at + "[3]");
        prog.push_back({code, a, b, c});
      }
      std::vector<bg_handle> ins;
      for (size_t i = 0; i < s.inputs.size(); ++i) ins.push_back(need(s, i));
      return fused(s, ins, prog, {}, dt);
    }
    if (op == "MATMUL") return matmul(s, dt);
    if (op == "PERMUTE") {
      bg_handle src = need(s, 0);
      std::vector<int64_t> axes;
      if (sem_axes) {
        auto it = sem_axes->find(s.value_id);
        if (it == sem_axes->end())
          plan_fail("PERMUTE value " + std::to_string(s.value_id) + " is missing its prepared semantic request");
        axes = it->second;
      } else {
        axes = axes_arg(s, rec(src).shape.size());
      }
      bg_handle out = permute(src, axes);
      if (rec(out).shape != s.shape) plan_fail("PERMUTE output shape differs from the plan");
      return out;
    }
    if (op == "BROADCAST_TO") {
      bg_handle src = need(s, 0);
      auto st = bstrides(rec(src).shape, s.shape, op);
      bg_handle out = 0;
      call(bg_copy_strided(ctx, src, 0, s.shape.data(), st.data(), int(s.shape.size()), &out));
      return own(out);
    }
    if (op == "REDUCE") return reduce(s);
    if (op == "FUSED_SOFTMAX") {
      bg_handle src = need(s, 0);
      const Record& r = rec(src);
      const int64_t rank = int64_t(r.shape.size());
      int64_t axis = rank - 1;
      if (s.arg && s.arg->kind == JVal::Obj && s.arg->get("axis") && s.arg->get("axis")->kind != JVal::Null)
        axis = expect_int(s.arg->get("axis"), "tensor plan FUSED_SOFTMAX.arg.axis");
      if (axis < 0) axis += rank;
      if (rank == 0) plan_fail("FUSED_SOFTMAX scalar input is unsupported");
      if (axis != rank - 1) plan_fail("FUSED_SOFTMAX currently supports last-axis softmax only");
      const int64_t cols = r.shape.back();
      bg_handle out = 0;
      call(bg_softmax_last(ctx, src, cols == 0 ? 0 : r.numel() / cols, cols, dt, &out));
      return own(out);
    }
    if (op == "LAYER_NORM") {
      const LnArg a = ln_arg(s);
      expect_shape(rec(need(s, 0)).shape, s.shape, op + ".input");
      expect_shape(rec(need(s, 1)).shape, a.normalized_shape, op + ".weight");
      expect_shape(rec(need(s, 2)).shape, a.normalized_shape, op + ".bias");
      bg_handle out = 0;
      call(bg_layer_norm(ctx, need(s, 0), need(s, 1), need(s, 2), a.rows, a.cols, a.eps, dt, &out));
      ctx->handles[out].shape = s.shape;
      return own(out);
    }
    if (op == "LAYER_NORM_BACKWARD_INPUT" || op == "LAYER_NORM_BACKWARD_WEIGHT" ||
        op == "LAYER_NORM_BACKWARD_BIAS") {
      // tensor_plan.ts:648-662 (lowering), :2855-2929 (shape rules)
      const LnArg a = ln_arg(s);
      if (dt != BG_F32) fail(BG_E_DTYPE, "tensor plan " + op + " supports float32 only");
      bg_handle out = 0;
      if (op == "LAYER_NORM_BACKWARD_INPUT") {
        expect_shape(rec(need(s, 0)).shape, s.shape, op + ".dy");
        expect_shape(rec(need(s, 1)).shape, s.shape, op + ".input");
        expect_shape(rec(need(s, 2)).shape, a.normalized_shape, op + ".weight");
        call(bg_layer_norm_backward_input(ctx, need(s, 0), need(s, 1), need(s, 2), a.rows, a.cols, a.eps, &out));
      } else if (op == "LAYER_NORM_BACKWARD_WEIGHT") {
        expect_shape(rec(need(s, 0)).shape, rec(need(s, 1)).shape, op + ".dy");
        expect_shape(s.shape, a.normalized_shape, op + ".output");
        call(bg_layer_norm_backward_weight(ctx, need(s, 0), need(s, 1), a.rows, a.cols, a.eps, &out));
      } else {
        expect_shape(s.shape, a.normalized_shape, op + ".output");
        call(bg_layer_norm_backward_bias(ctx, need(s, 0), a.rows, a.cols, &out));
      }
      ctx->handles[out].shape = s.shape;
      return own(out);
    }
    if (const ConvStep cs = conv_step(op); cs.spatial) {
      const ConvArg a = conv_arg(s, cs);
      if (dt != BG_F32) fail(BG_E_DTYPE, "tensor plan " + op + " supports float32 only");
      const int r = cs.spatial;
      static const char* ax3[3] = {"d", "h", "w"};
      bg_conv_desc d{};
      d.op = cs.op;
      d.transposed = cs.transposed ? 1 : 0;
      d.spatial = r;
      d.n = a["n"];
      d.c_in = a["c_in"];
      d.c_out = a["c_out"];
      d.groups = a["groups"];
      for (int i = 0; i < r; ++i) {
        const std::string x = ax3[3 - r + i];
        if (r == 1) {
          d.in[0] = a["l_in"];
          d.out[0] = a["l_out"];
          d.k[0] = a["k"];
          d.stride[0] = a["stride"];
          d.pad[0] = a["padding"];
          d.dilation[0] = a["dilation"];
        } else {
          d.in[i] = a.v.at(x);
          d.out[i] = a.v.at("out_" + x);
          d.k[i] = a.v.at("k" + x);
          d.stride[i] = a.v.at("stride_" + x);
          d.pad[i] = a.v.at("pad_" + x);
          d.dilation[i] = a.v.at("dilation_" + x);
          if (cs.transposed) d.output_pad[i] = a.v.at("output_pad_" + x);
        }
      }
      std::vector<int64_t> xs{d.n, d.c_in}, ys{d.n, d.c_out}, ws;
      ws = cs.transposed ? std::vector<int64_t>{d.c_in, a["c_out_per_group"]}
                         : std::vector<int64_t>{d.c_out, d.c_in / d.groups};
      for (int i = 0; i < r; ++i) {
        xs.push_back(d.in[i]);
        ys.push_back(d.out[i]);
        ws.push_back(d.k[i]);
      }
      if (cs.op == BG_CONV_FORWARD) {
        d.a = need(s, 0);
        d.b = need(s, 1);
        expect_shape(rec(d.a).shape, xs, op + ".input");
        expect_shape(rec(d.b).shape, ws, op + ".weight");
        expect_shape(s.shape, ys, op + ".output");
        if (s.inputs.size() > 2) {
          d.bias = need(s, 2);
          expect_shape(rec(d.bias).shape, {d.c_out}, op + ".bias");
        }
      } else if (cs.op == BG_CONV_BACKWARD_INPUT) {
        d.a = need(s, 0);
        d.b = need(s, 1);
        expect_shape(rec(d.a).shape, ys, op + ".dy");
        expect_shape(rec(d.b).shape, ws, op + ".weight");
        expect_shape(s.shape, xs, op + ".output");
      } else if (cs.op == BG_CONV_BACKWARD_WEIGHT) {
        d.a = need(s, 0);
        d.b = need(s, 1);
        expect_shape(rec(d.a).shape, ys, op + ".dy");
        expect_shape(rec(d.b).shape, xs, op + ".input");
        expect_shape(s.shape, ws, op + ".output");
      } else {
        d.a = need(s, 0);
        expect_shape(rec(d.a).shape, ys, op + ".dy");
        expect_shape(s.shape, {d.c_out}, op + ".output");
      }
      bg_handle out = 0;
      call(bg_conv_ex(ctx, &d, &out));
      ctx->handles[out].shape = s.shape;
      return own(out);
    }
    if (op == kAdamwFused || op == kAdamFused) {
      // The absorbed steps' argument and shape rules, in their order.
      const bool adamw = op == kAdamwFused;
      const std::string fam = adamw ? "ADAMW_UPDATE_" : "ADAM_UPDATE_";
      Step sm = s, sv = s, sp = s;
      sm.op = fam + "M";
      sm.arg = s.arg_m;
      sv.op = fam + "V";
      sv.arg = s.arg_v;
      sp.op = fam + "PARAM";
      const bg_optim_args am = optim_arg(sm, adamw ? BG_OPT_ADAMW_M : BG_OPT_ADAM_M);
      const bg_optim_args av = optim_arg(sv, adamw ? BG_OPT_ADAMW_V : BG_OPT_ADAM_V);
      const bg_optim_args ap = optim_arg(sp, adamw ? BG_OPT_ADAMW_PARAM : BG_OPT_ADAM_PARAM);
      if (dt != BG_F32) fail(BG_E_DTYPE, "tensor plan " + sp.op + " supports float32 only");
      const std::string r0 = sp.op + ".param", r1 = sm.op + ".grad", r2 = sm.op + ".m", r3 = sv.op + ".v";
      const char* roles[4] = {r0.c_str(), r1.c_str(), r2.c_str(), r3.c_str()};
      const float* in[4];
      for (int i = 0; i < 4; ++i) {
        const Record& r = rec(need(s, size_t(i)));
        expect_shape(r.shape, s.shape, roles[i]);
        if (r.dtype != BG_F32) fail(BG_E_DTYPE, std::string("tensor plan ") + roles[i] + " must be float32");
        in[i] = reinterpret_cast<const float*>(r.ptr());
      }
      const int64_t n = numel(s.shape);
      bg_handle out = mint(ctx, size_t(n) * 4, s.shape, BG_F32);
      float* po = reinterpret_cast<float*>(ctx->handles[out].ptr());
      {
        Profile prof(ctx, adamw ? "adamw_update_fused" : "adam_update_fused", n * 20, 0);
        launch_optimizer_fused(ctx, adamw ? kOptAdamwFused : kOptAdamFused, ap, am.beta1, av.beta2,
                               am.weight_decay, av.weight_decay, in, po, n);
      }
      return own(out);
    }
    if (const int kind = optim_kind(op); kind >= 0) {
      // tensor_plan.ts:663-702 (lowering), :2926-3113 (shape rules),
      // :3776-3827 (arguments)
      static const char* roles[7][4] = {{"param", "grad"},          {"m", "grad"},
                                        {"v", "grad"},              {"param", "grad", "m", "v"},
                                        {"param", "grad", "m"},     {"param", "grad", "v"},
                                        {"param", "m", "v"}};
      static const int arity[7] = {2, 2, 2, 4, 3, 3, 3};
      const bg_optim_args a = optim_arg(s, kind);
      if (dt != BG_F32) fail(BG_E_DTYPE, "tensor plan " + op + " supports float32 only");
      bg_handle in[4] = {0, 0, 0, 0};
      for (int i = 0; i < arity[kind]; ++i) {
        in[i] = need(s, size_t(i));
        expect_shape(rec(in[i]).shape, s.shape, op + "." + roles[kind][i]);
      }
      bg_handle out = 0;
      call(bg_optimizer_update(ctx, kind, in, arity[kind], &a, numel(s.shape), &out));
      ctx->handles[out].shape = s.shape;
      return own(out);
    }
    fail(BG_E_UNSUPPORTED, "tensor plan op " + op + " is not available in this build");
  }

  bg_handle matmul(const Step& s, int dt) {
    bg_handle a = need(s, 0), b = need(s, 1);
    const Record &ra = rec(a), &rb = rec(b);
    if (ra.shape.size() < 2 || rb.shape.size() < 2 || s.shape.size() < 2)
      plan_fail("MATMUL supports operands of rank >= 2");
    const int64_t m = ra.shape[ra.shape.size() - 2], k = ra.shape.back();
    const int64_t k2 = rb.shape[rb.shape.size() - 2], n = rb.shape.back();
    if (k != k2 || s.shape[s.shape.size() - 2] != m || s.shape.back() != n)
      plan_fail("MATMUL shape mismatch");
    if (ra.dtype != rb.dtype) fail(BG_E_DTYPE, "tensor plan MATMUL operands differ in dtype");
    const int64_t bo = numel(s.shape) / (m * n);
    const int64_t ba = ra.numel() / (m * k), bb = rb.numel() / (k * n);
    if ((ba != bo && ba != 1) || (bb != bo && bb != 1))
      plan_fail("MATMUL batch dims must match or broadcast from a single matrix");
    bg_matmul_desc d{};
    d.a = a;
    d.b = b;
    d.batch = bo;
    d.m = m;
    d.n = n;
    d.k = k;
    d.lda = k;
    d.ldb = n;
    d.ldc = n;
    d.stride_a = ba == 1 ? 0 : m * k;
    d.stride_b = bb == 1 ? 0 : k * n;
    d.stride_c = m * n;
    d.in_dtype = ra.dtype;
    d.out_dtype = dt;
    bg_handle out = 0;
    call(bg_matmul_ex(ctx, &d, &out));
    ctx->handles[out].shape = s.shape;
    return own(out);
  }

  bg_handle reduce(const Step& s) {
    bg_handle src = need(s, 0);
    const Record& r = rec(src);
    const int64_t rank = int64_t(r.shape.size());
    if (!s.arg || s.arg->kind != JVal::Obj) plan_fail("REDUCE.arg must be an object");
    const JVal* opv = s.arg->get("op");
    if (!opv || opv->kind != JVal::Str) fail(BG_E_INVALID, "tensor plan REDUCE.arg.op must be a string");
    int rop;
    if (opv->str == "sum") rop = BG_RED_SUM;
    else if (opv->str == "mean") rop = BG_RED_MEAN;
    else if (opv->str == "max") rop = BG_RED_MAX;  // extension
    else if (opv->str == "min") rop = BG_RED_MIN;  // extension
    else plan_fail("REDUCE supports sum/mean in v0 (got " + opv->str + ")");
    std::vector<int64_t> axes;
    const JVal* ax = s.arg->get("axis");
    auto norm = [&](int64_t a) {
      int64_t n = a < 0 ? a + rank : a;
      if (n < 0 || n >= rank)
        plan_fail("REDUCE axis " + std::to_string(a) + " out of range for rank " + std::to_string(rank));
      return n;
    };
    if (!ax || ax->kind == JVal::Null) {
      for (int64_t i = 0; i < rank; ++i) axes.push_back(i);
    } else if (ax->kind == JVal::Arr) {
      for (size_t i = 0; i < ax->arr.size(); ++i)
        axes.push_back(norm(expect_int(&ax->arr[i], "tensor plan REDUCE.arg.axis[" + std::to_string(i) + "]")));
    } else {
      axes.push_back(norm(expect_int(ax, "tensor plan REDUCE.arg.axis")));
    }
    std::set<int64_t> red(axes.begin(), axes.end());
    if (red.size() != axes.size()) plan_fail("REDUCE duplicate axis");
    int64_t cols = 1;
    for (int64_t a : red) cols *= r.shape[size_t(a)];
    const int64_t rows = cols == 0 ? 0 : r.numel() / std::max<int64_t>(cols, 1);
    // Move the reduced axes innermost (one strided copy) unless they already
    // are the trailing axes.
    bool trailing = true;
    for (int64_t i = 0; i < int64_t(red.size()); ++i)
      if (!red.count(rank - 1 - i)) trailing = false;
    // Reduced axes that are not all trailing, without a transposing copy:
    //  - one contiguous block of axes [a0, a1) (a leading prefix is the bias
    //    gradient's sum over the batch): x read in place as
    //    [B = dims before a0][R = the block][C = dims from a1];
    //  - a leading prefix plus a trailing suffix (batch and spatial axes of
    //    [N, C, L]): the suffix by the fused row reduction into f32, then
    //    the prefix in place.
    if (!trailing && cols > 0 && rows > 0 && (r.dtype == BG_F32 || r.dtype == BG_F16 || r.dtype == BG_BF16)) {
      if (numel(s.shape) != rows) plan_fail("REDUCE output shape differs from the plan");
      const int dt = r.dtype;
      if (dt != plan_dtype(s.dtype, "REDUCE dtype")) fail(BG_E_DTYPE, "tensor plan REDUCE dtype differs");
      const std::vector<int64_t> ax(red.begin(), red.end());  // ascending
      const std::vector<int64_t> shp = r.shape;
      auto prod = [&](int64_t lo, int64_t hi) {
        int64_t v = 1;
        for (int64_t i = lo; i < hi; ++i) v *= shp[size_t(i)];
        return v;
      };
      const int64_t es = dtype_size(dt);
      const int64_t na = int64_t(ax.size());
      if (ax.back() - ax.front() + 1 == na) {
        const int64_t a0 = ax.front(), a1 = ax.back() + 1;
        bg_handle out = own(mint(ctx, size_t(rows * es), s.shape, dt));
        Profile prof(ctx, "reduce_lead", (rows * cols + rows) * es, rows * cols);
        launch_reduce_lead(ctx, rec(src).ptr(), dt, prod(0, a0), cols, prod(a1, rank), rop, ctx->handles[out].ptr(),
                           dt);
        return out;
      }
      int64_t np = 0;
      while (np < na && ax[size_t(np)] == np) ++np;
      const int64_t s0 = ax[size_t(np)];
      const bool suffix = np > 0 && ax.back() == rank - 1 && ax.back() - s0 + 1 == na - np;
      if (suffix) {
        const int64_t P = prod(0, np), M = prod(np, s0), L = prod(s0, rank);
        bg_fused_op cp{BG_OP_COPY, -1, 0, 0};
        int64_t rs[2] = {P * M, L};
        bg_fused_desc d{};
        d.n_inputs = 1;
        d.inputs = &src;
        d.n_ops = 1;
        d.ops = &cp;
        d.rank = 2;
        d.shape = rs;
        d.out_dtype = BG_F32;
        d.reduce_op = rop;
        bg_handle y = 0;
        call(bg_fused_ex(ctx, &d, &y));
        own(y);
        bg_handle out = own(mint(ctx, size_t(rows * es), s.shape, dt));
        {
          Profile prof(ctx, "reduce_lead", P * M * 4 + rows * es, P * M);
          launch_reduce_lead(ctx, rec(y).ptr(), BG_F32, 1, P, M, rop, ctx->handles[out].ptr(), dt);
        }
        bg_release(ctx, y);
        owned.erase(y);
        return out;
      }
    }
    bg_handle x = src;
    if (!trailing) {
      std::vector<int64_t> perm;
      for (int64_t i = 0; i < rank; ++i)
        if (!red.count(i)) perm.push_back(i);
      for (int64_t a : red) perm.push_back(a);
      x = permute(src, perm);
    }
    if (cols == 0 || rows == 0) plan_fail("REDUCE over an empty axis is unsupported");
    bg_handle out = 0;
    call(bg_reduce_last(ctx, x, rows, cols, rop, 0, &out));
    if (x != src) {
      bg_release(ctx, x);
      owned.erase(x);
    }
    if (numel(s.shape) != rows) plan_fail("REDUCE output shape differs from the plan");
    ctx->handles[out].shape = s.shape;
    if (rec(out).dtype != plan_dtype(s.dtype, "REDUCE dtype")) fail(BG_E_DTYPE, "tensor plan REDUCE dtype differs");
    return own(out);
  }

  void release_all() {
    for (bg_handle h : owned) bg_release(ctx, h);
    owned.clear();
  }
};

}  // namespace

// Parses, validates and fuses a plan without a device (bg_plan_inspect):
// one JSON object per step the executor would run, in order.
std::string inspect_plan(const char* json, const char* requests_json) {
  JVal doc = JsonReader(json, "tensor plan").parse();
  Plan plan = normalize(doc);
  std::unordered_map<int64_t, std::vector<int64_t>> sem;
  if (requests_json) sem = bind_requests(plan, parse_requests(requests_json));
  fuse_adamw(plan);
  fuse_plan(plan, requests_json ? &sem : nullptr);
  std::string out = "{\"steps\":[";
  for (size_t i = 0; i < plan.steps.size(); ++i) {
    const Step& s = plan.steps[i];
    if (i) out += ",";
    out += "{\"value_id\":" + std::to_string(s.value_id) + ",\"op\":\"";
    for (char c : s.op) {
      if (c == '"' || c == '\\') out += '\\';
      out += (unsigned char)c < 0x20 ? '?' : c;
    }
    out += "\",\"inputs\":[";
    for (size_t j = 0; j < s.inputs.size(); ++j) out += (j ? "," : "") + std::to_string(s.inputs[j]);
    out += "]";
    if (s.op == "+PROGRAM") {
      out += ",\"n_ops\":" + std::to_string(s.prog.size()) + ",\"reduce\":" + std::to_string(s.reduce_op);
      out += ",\"imms\":[";
      for (size_t j = 0; j < s.imms.size(); ++j) {
        char b[40];
        std::snprintf(b, sizeof b, "%.17g", s.imms[j]);
        out += (j ? "," : "") + std::string(b);
      }
      out += "]";
    } else if (s.op == "+LINEAR") {
      out += ",\"trans_b\":" + std::to_string(s.mm.trans_b) + ",\"round\":" + std::to_string(s.mm.round_f16) +
             ",\"act\":" + std::to_string(s.mm.act) + ",\"bias\":" + std::to_string(int(s.has_bias)) +
             ",\"residual\":" + std::to_string(int(s.has_residual)) + ",\"a_dtype\":" +
             std::to_string(s.mm_ext.a_dtype) + ",\"b_dtype\":" + std::to_string(s.mm_ext.b_dtype);
    } else if (s.op == "+ATTENTION") {
      out += ",\"causal\":" + std::to_string(s.att.causal) + ",\"scale\":" + std::to_string(s.att.scale);
    }
    out += "}";
  }
  out += "],\"root_id\":" + std::to_string(plan.root_id) + "}";
  return out;
}

bg_handle run_plan(bg_ctx* ctx, const char* json, const char* requests_json, const int64_t* ids,
                   const bg_handle* handles, int n, int dtype, bool resident) {
  if (dtype != BG_F32 && dtype != BG_F16 && dtype != BG_BF16 && dtype != BG_BOOL)
    fail(BG_E_DTYPE, "run_tensor_plan: dtype not supported");
  JVal doc = JsonReader(json, "tensor plan").parse();
  Plan plan = normalize(doc);
  std::unordered_map<int64_t, std::vector<int64_t>> sem;
  if (requests_json) sem = bind_requests(plan, parse_requests(requests_json));
  fuse_adamw(plan);
  fuse_plan(plan, requests_json ? &sem : nullptr);

  Runner R{ctx};
  if (requests_json) R.sem_axes = &sem;
  for (int i = 0; i < n; ++i) {
    if (R.vals.count(ids[i])) plan_fail("input " + std::to_string(ids[i]) + " provided twice");
    get(ctx, handles[i], "tensor_plan[input]");
    R.vals[ids[i]] = handles[i];
    R.inputs.insert(handles[i]);
  }
  // Last step that reads each value (liveness, tensor_plan.ts:375-409).
  std::unordered_map<int64_t, size_t> last_use;
  for (size_t i = 0; i < plan.steps.size(); ++i)
    for (int64_t in : plan.steps[i].inputs) last_use[in] = i;

  try {
    for (size_t i = 0; i < plan.steps.size(); ++i) {
      const Step& s = plan.steps[i];
      bg_handle h = R.exec(s);
      R.vals[s.value_id] = h;
      // Values whose last reader was this step (never the root).
      for (int64_t in : s.inputs) {
        if (in == plan.root_id || last_use[in] != i) continue;
        bg_handle hin = R.vals[in];
        if (R.owned.count(hin)) {
          bg_release(ctx, hin);
          R.owned.erase(hin);
        }
      }
      // A value nobody reads (dead code) is released right away.
      if (s.value_id != plan.root_id && !last_use.count(s.value_id) && R.owned.count(h)) {
        bg_release(ctx, h);
        R.owned.erase(h);
      }
    }
  } catch (...) {
    R.release_all();
    throw;
  }
  bg_handle root = R.vals.at(plan.root_id);
  if (resident) {
    // The root must be an allocation of its own (runTensorGpuPlanResident).
    const Alloc* ra = ctx->handles.at(root).alloc;
    bool aliases = !R.owned.count(root);
    for (bg_handle in : R.inputs)
      if (ctx->handles.count(in) && ctx->handles.at(in).alloc == ra) aliases = true;
    if (aliases) {
      R.release_all();
      plan_fail("root " + std::to_string(plan.root_id) +
                " aliases an input buffer; resident output requires an owned root");
    }
  }
  R.owned.erase(root);
  R.release_all();
  if (!R.inputs.count(root)) return root;
  // Root is a caller's input (materialising plan): hand back a view so the
  // caller may release it like any other root.
  bg_handle v = 0;
  const Record& rr = ctx->handles.at(root);
  if (bg_reshape(ctx, root, rr.shape.data(), int(rr.shape.size()), &v) != BG_OK) fail(BG_E_HIP, ctx->err);
  return v;
}

}  // namespace bg
