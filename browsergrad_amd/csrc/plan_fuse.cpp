// Plan-level fusion for the tensor-plan executor (plan.cpp).
//
// The reference executes a tensor plan one WGSL dispatch per step
// (executeStep, packages/browsergrad-kernels/src/tensor_plan.ts:424-707) and
// names fusing whole SDPA-shaped graphs as the runtime's direction
// (packages/browsergrad-kernels/README.md:53-70).  Here the plan is
// rewritten before it runs, so that each of these step groups becomes one
// launch of this library's kernels:
//
//   SDPA        MATMUL(Q, PERMUTE(K)) [-> CAST f32] -> MUL(scale) ->
//               [WHERE(CAUSAL_MASK, -inf, .)] -> FUSED_SOFTMAX [-> CAST] ->
//               MATMUL(., V)                      -> "+ATTENTION"
//   LINEAR      MATMUL(A | CAST(A), B | PERMUTE(W) | CAST(PERMUTE(W))) ->
//               [CAST f32] -> [ADD bias[N]] -> [relu] -> [ADD residual]
//                                                 -> "+LINEAR" (GEMM epilogue)
//   PROGRAM     a DAG of elementwise steps of one shape (ADD MUL DIV NEG EXP
//               LOG CMP WHERE CONST CAST FUSED_ELEMENTWISE) with an optional
//               trailing REDUCE over the last axis -> "+PROGRAM" (one
//               bg_fused_ex, values in registers)
//
// Every rewrite keeps the float32 operations and their order: a fused
// program rounds each 16-bit step's value through that type (ROUND_F16 /
// ROUND_BF16) exactly where the step would have stored it, the GEMM epilogue
// applies round -> bias -> relu -> residual in the graph's order, and
// attention computes the same softmax(scale * Q K^T) P V (with S kept in
// f32, as the walker's default, unless BG_ATTN_EXACT_ROUNDING is set).
// A value is absorbed into a group only when every step that reads it is in
// the group and it is not the plan's root; anything else stays a step of
// its own.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <map>
#include <set>
#include <string>
#include <unordered_map>
#include <vector>

#include "plan.h"

namespace bg {
namespace {

bool is_narrow(const std::string& dt) { return dt == "float16" || dt == "bfloat16"; }

int wire_dtype(const std::string& s) {
  if (s == "float32" || s == "float64") return BG_F32;  // float64 only for constants (stored as f32)
  if (s == "float16") return BG_F16;
  if (s == "bfloat16") return BG_BF16;
  if (s == "bool") return BG_BOOL;
  return -1;
}

int64_t prod(const std::vector<int64_t>& v, size_t from = 0, size_t to = size_t(-1)) {
  int64_t p = 1;
  for (size_t i = from; i < std::min(to, v.size()); ++i) p *= v[i];
  return p;
}

// Producers, readers and the root of a plan, rebuilt by each pass.
struct Graph {
  Plan& plan;
  std::unordered_map<int64_t, size_t> producer;   // value id -> step index
  std::unordered_map<int64_t, std::set<size_t>> readers;
  std::vector<bool> drop;

  explicit Graph(Plan& p) : plan(p), drop(p.steps.size(), false) {
    for (size_t i = 0; i < p.steps.size(); ++i) {
      producer[p.steps[i].value_id] = i;
      for (int64_t in : p.steps[i].inputs) readers[in].insert(i);
    }
  }
  const Step* prod_of(int64_t v) const {
    auto it = producer.find(v);
    if (it == producer.end() || drop[it->second]) return nullptr;
    return &plan.steps[it->second];
  }
  Step* prod_of(int64_t v) {
    auto it = producer.find(v);
    if (it == producer.end() || drop[it->second]) return nullptr;
    return &plan.steps[it->second];
  }
  size_t index_of(int64_t v) const { return producer.at(v); }
  // Read by exactly one step and not the root.
  bool single(int64_t v) const {
    if (v == plan.root_id) return false;
    auto it = readers.find(v);
    return it != readers.end() && it->second.size() == 1;
  }
  // The one step reading v (nullptr unless single(v)).
  Step* sole_reader(int64_t v) {
    if (!single(v)) return nullptr;
    const size_t r = *readers[v].begin();
    return drop[r] ? nullptr : &plan.steps[r];
  }
  void remove(int64_t v) { drop[index_of(v)] = true; }
  void commit() {
    std::vector<Step> kept;
    for (size_t i = 0; i < plan.steps.size(); ++i)
      if (!drop[i]) kept.push_back(std::move(plan.steps[i]));
    plan.steps = std::move(kept);
  }
};

// An integral JSON number a double holds exactly (|x| <= 2^53).
bool as_int(const JVal& v, int64_t& out) {
  if (v.kind != JVal::Num || !std::isfinite(v.num) || v.num != std::floor(v.num) ||
      std::fabs(v.num) > 9007199254740992.0)
    return false;
  out = int64_t(v.num);
  return true;
}

const JVal* arg_field(const Step& s, const char* key) {
  return s.arg && s.arg->kind == JVal::Obj ? s.arg->get(key) : nullptr;
}

bool const_value(const Step* s, double& v) {
  if (!s || s->op != "CONST") return false;
  const JVal* x = arg_field(*s, "value");
  if (!x || x->kind != JVal::Num) {
    // -inf / nan travel as strings or null in some encoders; accept "-inf".
    if (x && x->kind == JVal::Str && (x->str == "-inf" || x->str == "-Infinity")) {
      v = -INFINITY;
      return true;
    }
    return false;
  }
  v = x->num;
  return true;
}

// PERMUTE axes bound from the semantic side table for this run (NULL on the
// legacy route, where a PERMUTE carries its axes in arg).
thread_local const std::unordered_map<int64_t, std::vector<int64_t>>* g_sem_axes = nullptr;

bool axes_are(const Step& s, std::initializer_list<int64_t> want) {
  if (g_sem_axes) {
    auto it = g_sem_axes->find(s.value_id);
    if (it != g_sem_axes->end()) return it->second == std::vector<int64_t>(want);
  }
  const JVal* a = arg_field(s, "axes");
  if (!a || a->kind != JVal::Arr || a->arr.size() != want.size()) return false;
  size_t i = 0;
  for (int64_t w : want) {
    const JVal& e = a->arr[i++];
    int64_t x;
    if (!as_int(e, x) || x != w) return false;
  }
  return true;
}

bool numeric_cast(const Step& s, const Graph& g) {
  if (s.op != "CAST" || s.inputs.size() != 1) return false;
  const int to = wire_dtype(s.dtype);
  if (to != BG_F32 && to != BG_F16 && to != BG_BF16) return false;
  const Step* src = g.prod_of(s.inputs[0]);
  if (!src) return false;
  const int from = wire_dtype(src->dtype);
  return from == BG_F32 || from == BG_F16 || from == BG_BF16;
}

// ---- SDPA ----------------------------------------------------------------

bool exact_score_rounding() {
  const char* e = std::getenv("BG_ATTN_EXACT_ROUNDING");
  if (!e) return false;
  const std::string v(e);
  return v == "1" || v == "true" || v == "yes" || v == "on";
}

void fuse_sdpa(Plan& plan) {
  Graph g(plan);
  for (size_t oi = 0; oi < plan.steps.size(); ++oi) {
    Step& o = plan.steps[oi];
    if (g.drop[oi] || o.op != "MATMUL" || o.inputs.size() != 2 || o.shape.size() != 4) continue;
    std::vector<int64_t> absorbed;
    int64_t p_id = o.inputs[0];
    const int64_t v_id = o.inputs[1];
    if (is_narrow(o.dtype)) {
      const Step* c = g.prod_of(p_id);
      if (!c || c->op != "CAST" || c->dtype != o.dtype || !g.single(p_id)) continue;
      absorbed.push_back(p_id);
      p_id = c->inputs[0];
    }
    const Step* sm = g.prod_of(p_id);
    if (!sm || sm->op != "FUSED_SOFTMAX" || sm->dtype != "float32" || !g.single(p_id)) continue;
    const JVal* ax = arg_field(*sm, "axis");
    if (ax && ax->kind == JVal::Num && !(ax->num == -1 || ax->num == double(sm->shape.size()) - 1)) continue;
    absorbed.push_back(p_id);
    int64_t x_id = sm->inputs[0];
    bool causal = false;
    const Step* wh = g.prod_of(x_id);
    if (wh && wh->op == "WHERE" && wh->inputs.size() == 3 && g.single(x_id)) {
      const Step* mask = g.prod_of(wh->inputs[0]);
      double fv = 0;
      if (!mask || mask->op != "CAUSAL_MASK" || !const_value(g.prod_of(wh->inputs[1]), fv) || fv != -INFINITY)
        continue;
      const size_t r = mask->shape.size();
      if (r < 2 || mask->shape[r - 2] != o.shape[2]) continue;
      causal = true;
      absorbed.push_back(x_id);
      x_id = wh->inputs[2];
    }
    const Step* mul = g.prod_of(x_id);
    if (!mul || mul->op != "MUL" || mul->inputs.size() != 2 || !g.single(x_id)) continue;
    double scale = 0;
    int64_t s_id = 0;
    if (const_value(g.prod_of(mul->inputs[1]), scale)) s_id = mul->inputs[0];
    else if (const_value(g.prod_of(mul->inputs[0]), scale)) s_id = mul->inputs[1];
    else continue;
    if (!(scale > 0) || !std::isfinite(scale)) continue;
    absorbed.push_back(x_id);
    const Step* s32 = g.prod_of(s_id);
    if (s32 && s32->op == "CAST" && s32->dtype == "float32" && g.single(s_id)) {
      const Step* s16 = g.prod_of(s32->inputs[0]);
      if (!s16 || !is_narrow(s16->dtype)) continue;
      absorbed.push_back(s_id);
      s_id = s32->inputs[0];
    }
    const Step* qk = g.prod_of(s_id);
    if (!qk || qk->op != "MATMUL" || qk->inputs.size() != 2 || !g.single(s_id)) continue;
    absorbed.push_back(s_id);
    const int64_t q_id = qk->inputs[0];
    int64_t kt_id = qk->inputs[1];
    Step* kt = g.prod_of(kt_id);
    if (!kt || !g.single(kt_id)) continue;
    int64_t k_id = 0;
    // K's shape and dtype as the attention reads it.  A CAST(PERMUTE(K)) is
    // only recorded here; it is re-pointed at K once every check has passed,
    // so a plan the checks turn away is left exactly as it was.
    std::vector<int64_t> ks;
    std::string k_dtype;
    int64_t perm_id = -1, perm_src = -1;
    if (kt->op == "PERMUTE" && axes_are(*kt, {0, 1, 3, 2})) {
      absorbed.push_back(kt_id);
      k_id = kt->inputs[0];
      const Step* k = g.prod_of(k_id);
      if (!k) continue;
      ks = k->shape;
      k_dtype = k->dtype;
    } else if (kt->op == "CAST" && is_narrow(kt->dtype)) {
      // CAST(PERMUTE(K)) -> the cast applies to K itself (a cast commutes
      // with a permutation); the attention reads K unpermuted.
      const Step* perm = g.prod_of(kt->inputs[0]);
      if (!perm || perm->op != "PERMUTE" || !axes_are(*perm, {0, 1, 3, 2}) || !g.single(kt->inputs[0])) continue;
      const Step* src = g.prod_of(perm->inputs[0]);
      if (!src) continue;
      perm_id = kt->inputs[0];
      perm_src = perm->inputs[0];
      k_id = kt_id;
      ks = src->shape;
      k_dtype = kt->dtype;
    } else {
      continue;
    }
    const Step* q = g.prod_of(q_id);
    const Step* v = g.prod_of(v_id);
    if (!q || !v || q->shape.size() != 4 || ks.size() != 4 || v->shape.size() != 4) continue;
    if (q->dtype != k_dtype || k_dtype != v->dtype || !is_narrow(q->dtype)) continue;
    const auto &qs = q->shape, &vs = v->shape;
    if (qs[0] != ks[0] || qs[1] != ks[1] || ks != vs || qs[3] != ks[3] || o.shape[2] != qs[2] ||
        o.shape[3] != vs[3])
      continue;
    for (int64_t a : absorbed) g.remove(a);
    if (perm_id >= 0) {
      // Re-point the cast at the unpermuted source: it now produces K.
      kt->inputs = {perm_src};
      kt->shape = ks;
      g.remove(perm_id);
    }
    bg_attention_desc& d = o.att;
    d = bg_attention_desc{};
    d.batch = qs[0];
    d.heads = qs[1];
    d.sq = qs[2];
    d.sk = ks[2];
    d.d = qs[3];
    d.scale = float(scale);
    d.causal = causal ? 1 : 0;
    d.in_dtype = wire_dtype(q->dtype);
    d.out_dtype = wire_dtype(o.dtype);
    d.round_scores = exact_score_rounding() ? 1 : 0;
    o.op = "+ATTENTION";
    o.inputs = {q_id, k_id, v_id};
  }
  g.commit();
}

// ---- LINEAR ----------------------------------------------------------------

// A fused-elementwise step whose program is ADD(mm, bias) (then, optionally,
// ADD(that, residual)) in either operand order.  Returns false otherwise.
bool linear_epilogue_program(const Step& f, int64_t mm_id, int64_t& bias_id, int64_t& res_id) {
  const JVal* ops = arg_field(f, "ops");
  if (!ops || ops->kind != JVal::Arr || ops->arr.empty() || ops->arr.size() > 2) return false;
  auto op_at = [&](size_t i, std::string& code, int64_t& a, int64_t& b) {
    const JVal& o = ops->arr[i];
    if (o.kind != JVal::Arr || o.arr.size() < 3 || o.arr[0].kind != JVal::Str) return false;
    code = o.arr[0].str;
    return as_int(o.arr[1], a) && as_int(o.arr[2], b);
  };
  auto input_of = [&](int64_t ref) -> int64_t {  // ref < 0 -> input value id
    const size_t i = size_t(-ref - 1);
    return ref < 0 && i < f.inputs.size() ? f.inputs[i] : -1;
  };
  std::string c0;
  int64_t a0, b0;
  if (!op_at(0, c0, a0, b0) || c0 != "ADD" || a0 >= 0 || b0 >= 0) return false;
  const int64_t x0 = input_of(a0), y0 = input_of(b0);
  if (x0 == mm_id && y0 != mm_id) bias_id = y0;
  else if (y0 == mm_id && x0 != mm_id) bias_id = x0;
  else return false;
  res_id = -1;
  if (ops->arr.size() == 2) {
    std::string c1;
    int64_t a1, b1;
    if (!op_at(1, c1, a1, b1) || c1 != "ADD") return false;
    if (a1 == 0 && b1 < 0) res_id = input_of(b1);
    else if (b1 == 0 && a1 < 0) res_id = input_of(a1);
    else return false;
    if (res_id == mm_id || res_id == bias_id) return false;
  }
  for (int64_t in : f.inputs)
    if (in != mm_id && in != bias_id && in != res_id) return false;
  return true;
}

void fuse_linear(Plan& plan) {
  Graph g(plan);
  for (size_t mi = 0; mi < plan.steps.size(); ++mi) {
    if (g.drop[mi]) continue;
    Step& mm = plan.steps[mi];
    if (mm.op != "MATMUL" || mm.inputs.size() != 2 || mm.shape.size() < 2) continue;
    const Step* A = g.prod_of(mm.inputs[0]);
    const Step* B = g.prod_of(mm.inputs[1]);
    if (!A || !B || A->shape.size() < 2 || B->shape.size() != 2) continue;
    std::vector<int64_t> absorbed;
    int64_t a_src = mm.inputs[0], b_src = mm.inputs[1];
    int a_dt = -1, b_dt = -1;
    bool trans_b = false;
    const bool narrow = is_narrow(mm.dtype);
    // B side: [CAST narrow] of [PERMUTE (1, 0)] of W.
    if (narrow && B->op == "CAST" && B->dtype == mm.dtype && g.single(mm.inputs[1])) {
      const Step* in = g.prod_of(B->inputs[0]);
      if (in && in->dtype == "float32") {
        absorbed.push_back(mm.inputs[1]);
        b_dt = BG_F32;
        b_src = B->inputs[0];
        if (in->op == "PERMUTE" && axes_are(*in, {1, 0}) && g.single(B->inputs[0])) {
          absorbed.push_back(B->inputs[0]);
          b_src = in->inputs[0];
          trans_b = true;
        }
      }
    } else if (B->op == "PERMUTE" && axes_are(*B, {1, 0}) && g.single(mm.inputs[1])) {
      absorbed.push_back(mm.inputs[1]);
      b_src = B->inputs[0];
      trans_b = true;
    }
    // A side: CAST narrow of an f32 value.
    if (narrow && A->op == "CAST" && A->dtype == mm.dtype && g.single(mm.inputs[0])) {
      const Step* in = g.prod_of(A->inputs[0]);
      if (in && in->dtype == "float32") {
        absorbed.push_back(mm.inputs[0]);
        a_dt = BG_F32;
        a_src = A->inputs[0];
      }
    }
    const Step* Bs = g.prod_of(b_src);
    if (!Bs || Bs->shape.size() != 2) continue;
    const int64_t K = A->shape.back();
    const int64_t M = prod(A->shape, 0, A->shape.size() - 1);
    const int64_t N = trans_b ? Bs->shape[0] : Bs->shape[1];
    if ((trans_b ? Bs->shape[1] : Bs->shape[0]) != K || mm.shape.back() != N || prod(mm.shape) != M * N) continue;
    // Epilogue chain from the product.
    int64_t cur = mm.value_id;
    std::string out_dtype = mm.dtype;
    bool round_out = false, has_bias = false, has_res = false;
    int act = BG_ACT_NONE;
    int64_t bias_id = -1, res_id = -1;
    std::vector<int64_t> epi;  // epilogue steps absorbed (the last one survives)
    auto value_ok_bias = [&](int64_t v) {
      const Step* b = g.prod_of(v);
      return b && b->dtype == "float32" && prod(b->shape) == N && !b->shape.empty() && b->shape.back() == N;
    };
    auto value_ok_res = [&](int64_t v, const std::vector<int64_t>& shape) {
      const Step* r = g.prod_of(v);
      return r && r->dtype == "float32" && r->shape == shape;
    };
    if (narrow) {
      Step* c = g.sole_reader(cur);
      if (c && c->op == "CAST" && c->dtype == "float32") {
        round_out = true;
        out_dtype = "float32";
        epi.push_back(cur);
        cur = c->value_id;
      }
    }
    if (Step* c = g.sole_reader(cur)) {
      if (c->op == "ADD" && c->inputs.size() == 2 && c->dtype == "float32") {
        const int64_t other = c->inputs[0] == cur ? c->inputs[1] : c->inputs[0];
        if (other != cur && value_ok_bias(other)) {
          has_bias = true;
          bias_id = other;
          epi.push_back(cur);
          cur = c->value_id;
        }
      } else if (c->op == "FUSED_ELEMENTWISE" && c->dtype == "float32") {
        int64_t bid = -1, rid = -1;
        if (linear_epilogue_program(*c, cur, bid, rid) && value_ok_bias(bid) &&
            (rid < 0 || value_ok_res(rid, c->shape))) {
          has_bias = true;
          bias_id = bid;
          if (rid >= 0) {
            has_res = true;
            res_id = rid;
          }
          epi.push_back(cur);
          cur = c->value_id;
        }
      }
    }
    if (has_bias && !has_res && out_dtype == "float32") {
      // relu: CMP(gt, y, CONST 0) and WHERE(cmp, y, CONST 0) are y's only readers.
      auto rd = g.readers.find(cur);
      if (cur != plan.root_id && rd != g.readers.end() && rd->second.size() == 2) {
        Step* cmp = nullptr;
        Step* wh = nullptr;
        for (size_t r : rd->second) {
          if (g.drop[r]) continue;
          Step& st = plan.steps[r];
          if (st.op == "CMP") cmp = &st;
          else if (st.op == "WHERE") wh = &st;
        }
        double z0 = 1, z1 = 1;
        const JVal* cop = cmp ? arg_field(*cmp, "op") : nullptr;
        if (cmp && wh && cop && cop->kind == JVal::Str && cop->str == "gt" && cmp->inputs.size() == 2 &&
            cmp->inputs[0] == cur && const_value(g.prod_of(cmp->inputs[1]), z0) && z0 == 0.0 &&
            g.single(cmp->value_id) && wh->inputs.size() == 3 && wh->inputs[0] == cmp->value_id &&
            wh->inputs[1] == cur && const_value(g.prod_of(wh->inputs[2]), z1) && z1 == 0.0 &&
            wh->dtype == "float32") {
          act = BG_ACT_RELU;
          epi.push_back(cur);
          epi.push_back(cmp->value_id);
          cur = wh->value_id;
        }
      }
    }
    if (has_bias && !has_res) {
      if (Step* c = g.sole_reader(cur)) {
        if (c->op == "ADD" && c->inputs.size() == 2 && c->dtype == "float32") {
          const int64_t other = c->inputs[0] == cur ? c->inputs[1] : c->inputs[0];
          const Step* cs = g.prod_of(cur);
          if (other != cur && cs && value_ok_res(other, cs->shape) && c->shape == cs->shape) {
            has_res = true;
            res_id = other;
            epi.push_back(cur);
            cur = c->value_id;
          }
        }
      }
    }
    if (absorbed.empty() && !has_bias && !round_out) continue;  // nothing gained over the plain MATMUL
    Step& out = *g.prod_of(cur);
    bg_matmul_desc d{};
    d.batch = 1;
    d.m = M;
    d.n = N;
    d.k = K;
    d.lda = K;
    d.ldb = trans_b ? K : N;
    d.ldc = N;
    d.trans_b = trans_b ? 1 : 0;
    d.in_dtype = wire_dtype(mm.dtype);
    d.out_dtype = wire_dtype(out_dtype);
    d.round_f16 = round_out ? 1 : 0;
    d.act = act;
    bg_matmul_ext e{};
    e.a_dtype = a_dt;
    e.b_dtype = b_dt;
    std::vector<int64_t> ins = {a_src, b_src};
    if (has_bias) ins.push_back(bias_id);
    if (has_res) ins.push_back(res_id);
    for (int64_t a : absorbed) g.remove(a);
    for (int64_t a : epi) g.remove(a);
    if (&out != &mm) g.remove(mm.value_id);
    out.mm = d;
    out.mm_ext = e;
    out.has_bias = has_bias;
    out.has_residual = has_res;
    out.op = "+LINEAR";
    out.inputs = ins;
  }
  g.commit();
}

// ---- elementwise programs ------------------------------------------------------

bool mappable(const Step& s, const Graph& g) {
  static const std::set<std::string> ops = {"ADD", "MUL", "DIV", "NEG", "EXP", "LOG",
                                            "CMP", "WHERE", "CONST", "FUSED_ELEMENTWISE"};
  if (ops.count(s.op)) return wire_dtype(s.dtype) >= 0;
  return numeric_cast(s, g);
}

int fused_code(const std::string& name) {
  static const std::unordered_map<std::string, int> m = {
      {"ADD", BG_OP_ADD}, {"MUL", BG_OP_MUL}, {"DIV", BG_OP_DIV}, {"NEG", BG_OP_NEG}, {"EXP", BG_OP_EXP},
      {"LOG", BG_OP_LOG}, {"MAX", BG_OP_MAX}, {"MIN", BG_OP_MIN}, {"SUB", BG_OP_SUB}, {"TANH", BG_OP_TANH},
      {"SQRT", BG_OP_SQRT}, {"ABS", BG_OP_ABS}, {"WHERE", BG_OP_WHERE},
      {"CMP_EQ", BG_OP_CMP_EQ}, {"CMP_NE", BG_OP_CMP_NE}, {"CMP_LT", BG_OP_CMP_LT},
      {"CMP_LE", BG_OP_CMP_LE}, {"CMP_GT", BG_OP_CMP_GT}, {"CMP_GE", BG_OP_CMP_GE}};
  auto it = m.find(name);
  return it == m.end() ? -1 : it->second;
}

int cmp_code_of(const Step& s) {
  const JVal* c = arg_field(s, "op");
  if (!c || c->kind != JVal::Str) return -1;
  const std::string& o = c->str;
  if (o == "eq") return BG_OP_CMP_EQ;
  if (o == "ne") return BG_OP_CMP_NE;
  if (o == "lt") return BG_OP_CMP_LT;
  if (o == "le") return BG_OP_CMP_LE;
  if (o == "gt") return BG_OP_CMP_GT;
  if (o == "ge") return BG_OP_CMP_GE;
  return -1;
}

// Value of a constant expression (a CONST, or casts of one between float
// types), rounded as each cast rounds; false for anything else.
bool const_expr(const Graph& g, int64_t v, double& out, int depth = 0) {
  const Step* s = g.prod_of(v);
  if (!s || depth > 8) return false;
  if (s->op == "CONST") {
    if (const_value(s, out)) {
      if (s->dtype == "float32") out = double(float(out));
      else if (s->dtype == "float16") out = double(float(_Float16(float(out))));
      else if (s->dtype == "bfloat16") out = double(float(__bf16(float(out))));
      return true;
    }
    return false;
  }
  if (s->op != "CAST" || s->inputs.size() != 1) return false;
  double x;
  if (!const_expr(g, s->inputs[0], x, depth + 1)) return false;
  if (s->dtype == "float32") out = double(float(x));
  else if (s->dtype == "float16") out = double(float(_Float16(float(x))));
  else if (s->dtype == "bfloat16") out = double(float(__bf16(float(x))));
  else return false;
  return true;
}

// Builds the program of a group (members in plan order).  Returns false when
// a member cannot be expressed or the program exceeds the kernel's limits.
// A scalar constant expression read from outside the group is inlined as an
// immediate (its steps then have no reader left and are dropped).
bool build_program(const Graph& g, const std::vector<size_t>& members, std::vector<int64_t>& ext,
                   std::vector<bg_fused_op>& prog, std::vector<double>& imms) {
  std::unordered_map<int64_t, int32_t> ref;  // value id -> program ref
  auto emit = [&](int code, int32_t a, int32_t b, int32_t c) {
    prog.push_back({code, a, b, c});
    return int32_t(prog.size()) - 1;
  };
  auto in_ref = [&](int64_t v) -> int32_t {
    auto it = ref.find(v);
    if (it != ref.end()) return it->second;
    double cv;
    const Step* p = g.prod_of(v);
    if (p && prod(p->shape) == 1 && const_expr(g, v, cv)) {
      imms.push_back(cv);
      const int32_t r = emit(BG_OP_IMM, int32_t(imms.size()) - 1, 0, 0);
      ref[v] = r;
      return r;
    }
    for (size_t i = 0; i < ext.size(); ++i)
      if (ext[i] == v) return -int32_t(i) - 1;
    ext.push_back(v);
    return -int32_t(ext.size());
  };
  for (size_t mi : members) {
    const Step& s = g.plan.steps[mi];
    int32_t r = -1;
    const int dt = wire_dtype(s.dtype);
    if (s.op == "CONST") {
      double v = 0;
      if (!const_value(&s, v)) {
        const JVal* x = arg_field(s, "value");
        if (!x || x->kind != JVal::Bool) return false;
        v = x->b ? 1.0 : 0.0;
      }
      imms.push_back(v);
      r = emit(BG_OP_IMM, int32_t(imms.size()) - 1, 0, 0);
    } else if (s.op == "CAST") {
      r = emit(BG_OP_COPY, in_ref(s.inputs[0]), 0, 0);
    } else if (s.op == "NEG" || s.op == "EXP" || s.op == "LOG") {
      if (s.inputs.size() != 1) return false;
      r = emit(fused_code(s.op), in_ref(s.inputs[0]), 0, 0);
    } else if (s.op == "ADD" || s.op == "MUL" || s.op == "DIV") {
      if (s.inputs.size() != 2) return false;
      const int32_t a = in_ref(s.inputs[0]), b = in_ref(s.inputs[1]);
      r = emit(fused_code(s.op), a, b, 0);
    } else if (s.op == "CMP") {
      const int code = cmp_code_of(s);
      if (code < 0 || s.inputs.size() != 2) return false;
      const int32_t a = in_ref(s.inputs[0]), b = in_ref(s.inputs[1]);
      r = emit(code, a, b, 0);
    } else if (s.op == "WHERE") {
      if (s.inputs.size() != 3) return false;
      const int32_t a = in_ref(s.inputs[0]), b = in_ref(s.inputs[1]), c = in_ref(s.inputs[2]);
      r = emit(BG_OP_WHERE, a, b, c);
    } else if (s.op == "FUSED_ELEMENTWISE") {
      const JVal* ops = arg_field(s, "ops");
      if (!ops || ops->kind != JVal::Arr || ops->arr.empty()) return false;
      std::vector<int32_t> in_refs;
      for (int64_t v : s.inputs) in_refs.push_back(in_ref(v));  // may emit immediates
      const int32_t base = int32_t(prog.size());  // the step's own ops start here
      for (const JVal& o : ops->arr) {
        if (o.kind != JVal::Arr || o.arr.size() < 2 || o.arr[0].kind != JVal::Str) return false;
        const int code = fused_code(o.arr[0].str);
        if (code < 0) return false;
        int32_t x[3] = {0, 0, 0};
        for (size_t j = 1; j < o.arr.size() && j < 4; ++j) {
          if (o.arr[j].kind == JVal::Null) {
            x[j - 1] = x[0];
            continue;
          }
          int64_t rr;
          if (!as_int(o.arr[j], rr)) return false;
          if (rr < 0) {
            if (size_t(-rr - 1) >= in_refs.size()) return false;
            x[j - 1] = in_refs[size_t(-rr - 1)];
          } else {
            if (base + rr >= int32_t(prog.size())) return false;
            x[j - 1] = base + int32_t(rr);
          }
        }
        if (o.arr.size() == 2) x[1] = x[0];
        emit(code, x[0], x[1], x[2]);
      }
      r = int32_t(prog.size()) - 1;
    } else {
      return false;
    }
    // A 16-bit step stores its value rounded; the register copy must match.
    if (dt == BG_F16) r = emit(BG_OP_ROUND_F16, r, 0, 0);
    else if (dt == BG_BF16) r = emit(BG_OP_ROUND_BF16, r, 0, 0);
    ref[s.value_id] = r;
  }
  return ext.size() <= BG_FUSED_MAX_INPUTS && prog.size() <= BG_FUSED_MAX_OPS && imms.size() <= BG_FUSED_MAX_IMMS;
}

bool trailing_reduce(const Step& r, int& rop) {
  if (r.op != "REDUCE" || r.inputs.size() != 1) return false;
  const JVal* op = arg_field(r, "op");
  if (!op || op->kind != JVal::Str) return false;
  if (op->str == "sum") rop = BG_RED_SUM;
  else if (op->str == "mean") rop = BG_RED_MEAN;
  else if (op->str == "max") rop = BG_RED_MAX;
  else if (op->str == "min") rop = BG_RED_MIN;
  else return false;
  return true;
}

void fuse_elementwise(Plan& plan) {
  Graph g(plan);
  std::vector<bool> taken(plan.steps.size(), false);
  for (size_t ii = plan.steps.size(); ii-- > 0;) {
    if (g.drop[ii] || taken[ii]) continue;
    Step& top_step = plan.steps[ii];
    size_t top = ii;
    int rop = BG_RED_NONE;
    bool keepdims = false;
    if (trailing_reduce(top_step, rop)) {
      const int64_t in = top_step.inputs[0];
      const Step* src = g.prod_of(in);
      if (!src || !mappable(*src, g) || !g.single(in) || taken[g.index_of(in)] || src->shape.empty()) continue;
      // Only the last axis (or, for rank 1, the whole vector).
      const JVal* ax = arg_field(top_step, "axis");
      const int64_t rank = int64_t(src->shape.size());
      bool last = false;
      int64_t a0;
      if (ax && as_int(*ax, a0)) last = a0 == rank - 1 || a0 == -1;
      else if (ax && ax->kind == JVal::Arr && ax->arr.size() == 1 && as_int(ax->arr[0], a0))
        last = a0 == rank - 1 || a0 == -1;
      else if ((!ax || ax->kind == JVal::Null) && rank == 1) last = true;
      if (!last) continue;
      const JVal* kd = arg_field(top_step, "keepdims");
      keepdims = kd && kd->kind == JVal::Bool && kd->b;
      top = g.index_of(in);
    } else if (!mappable(top_step, g)) {
      continue;
    }
    const std::vector<int64_t> iter = plan.steps[top].shape;
    std::set<size_t> group = {top};
    for (bool grew = true; grew;) {
      grew = false;
      for (size_t m : std::vector<size_t>(group.begin(), group.end())) {
        for (int64_t v : plan.steps[m].inputs) {
          const Step* p = g.prod_of(v);
          if (!p) continue;
          const size_t pi = g.index_of(v);
          if (group.count(pi) || taken[pi] || v == plan.root_id || !mappable(*p, g)) continue;
          if (p->op != "CONST" && p->shape != iter) continue;
          bool inside = true;
          for (size_t r : g.readers[v])
            if (!group.count(r)) inside = false;
          if (!inside) continue;
          group.insert(pi);
          grew = true;
        }
      }
    }
    if (group.size() == 1 && rop == BG_RED_NONE) continue;  // a single step is one launch already
    std::vector<size_t> members(group.begin(), group.end());  // plan order (indices ascend)
    std::vector<int64_t> ext;
    std::vector<bg_fused_op> prog;
    std::vector<double> imms;
    if (!build_program(g, members, ext, prog, imms)) continue;
    const size_t out_i = rop == BG_RED_NONE ? top : ii;
    Step& out = plan.steps[out_i];
    for (size_t m : members) {
      taken[m] = true;
      if (m != out_i) g.drop[m] = true;
    }
    taken[out_i] = true;
    out.op = "+PROGRAM";
    out.inputs = ext;
    out.prog = prog;
    out.imms = imms;
    out.iter = iter;
    out.reduce_op = rop;
    out.keepdims = keepdims;
  }
  g.commit();
}

// Steps whose value no step reads and that are not the root (constants a
// fused group no longer needs): every plan op is free of side effects.
void drop_dead(Plan& plan) {
  for (bool again = true; again;) {
    again = false;
    std::set<int64_t> read;
    for (const Step& s : plan.steps)
      for (int64_t in : s.inputs) read.insert(in);
    std::vector<Step> kept;
    for (Step& s : plan.steps) {
      if (s.value_id != plan.root_id && !read.count(s.value_id) && s.op != "BUFFER") {
        again = true;
        continue;
      }
      kept.push_back(std::move(s));
    }
    plan.steps = std::move(kept);
  }
}

}  // namespace

void fuse_plan(Plan& plan, const std::unordered_map<int64_t, std::vector<int64_t>>* sem_axes) {
  // BG_DISABLE_FUSION (the front end's fusion switch) also runs plans step by step.
  if (const char* e = std::getenv("BG_DISABLE_FUSION")) {
    const std::string v(e);
    if (v == "1" || v == "true" || v == "yes" || v == "on") return;
  }
  // BG_PLAN_FUSION=<comma list of sdpa, linear, program> runs only the
  // named passes (for comparisons and diagnosis); unset runs all three.
  const char* sel = std::getenv("BG_PLAN_FUSION");
  auto on = [&](const char* pass) { return !sel || std::string(sel).find(pass) != std::string::npos; };
  // The matchers read inputs by position: a plan with a step of the wrong
  // arity is left unfused (the executor refuses that step when it runs it).
  static const std::unordered_map<std::string, size_t> arity = {
      {"CAST", 1}, {"PERMUTE", 1}, {"FUSED_SOFTMAX", 1}, {"NEG", 1}, {"EXP", 1}, {"LOG", 1}, {"REDUCE", 1},
      {"LOAD", 1}, {"RESHAPE", 1}, {"SLICE", 1}, {"ADD", 2}, {"MUL", 2}, {"DIV", 2}, {"CMP", 2},
      {"MATMUL", 2}, {"WHERE", 3}, {"CONST", 0}, {"CAUSAL_MASK", 0}, {"BUFFER", 0}};
  for (const Step& s : plan.steps) {
    auto it = arity.find(s.op);
    if (it != arity.end() && s.inputs.size() != it->second) return;
  }
  g_sem_axes = sem_axes;
  if (on("sdpa")) fuse_sdpa(plan);
  if (on("linear")) fuse_linear(plan);
  if (on("program")) fuse_elementwise(plan);
  drop_dead(plan);
  g_sem_axes = nullptr;
}

}  // namespace bg
