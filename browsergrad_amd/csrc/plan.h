// Tensor-plan model shared by the executor (plan.cpp) and the plan-level
// fuser (plan_fuse.cpp).
#pragma once

#include <cstdint>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "core.h"

namespace bg {

// A parsed JSON value (the executor's own small reader builds these).
struct JVal {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  bool b = false;
  double num = 0;
  bool is_int = false;  // written without fraction / exponent
  std::string str;
  std::vector<JVal> arr;
  std::vector<std::pair<std::string, JVal>> obj;

  const JVal* get(const char* key) const {
    if (kind != Obj) return nullptr;
    for (const auto& kv : obj)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
  // snake_case or camelCase (tensor_plan.ts:139-180 accepts both)
  const JVal* get2(const char* snake, const char* camel) const {
    const JVal* v = get(camel);
    return v && v->kind != Null ? v : get(snake);
  }
};


// ---- plan model (tensor_plan.ts:63-97) -------------------------------------

struct Step {
  int64_t step = 0;
  int64_t value_id = 0;
  std::string op;
  std::vector<int64_t> inputs;
  std::vector<int64_t> shape;
  std::string dtype;
  const JVal* arg = nullptr;  // may be null / JSON null
  // Fused AdamW step (fuse_adamw): the absorbed M and V steps' args.
  const JVal* arg_m = nullptr;
  const JVal* arg_v = nullptr;
  // Set by fuse_plan on the steps it creates:
  //   "+PROGRAM"    one bg_fused_ex over `inputs`: prog / imms over the
  //                 iteration shape `iter`, then reduce_op over its last
  //                 axis (BG_RED_NONE: none);
  //   "+LINEAR"     one bg_matmul_ex2: inputs {a, b[, bias][, residual]}
  //                 with mm (handles filled at execution) and mm_ext;
  //   "+ATTENTION"  one bg_attention_ex over inputs {q, k, v} with att.
  std::vector<bg_fused_op> prog;
  std::vector<double> imms;
  std::vector<int64_t> iter;
  int reduce_op = BG_RED_NONE;
  bool keepdims = false;
  bg_matmul_desc mm{};
  bg_matmul_ext mm_ext{};
  bool has_bias = false, has_residual = false;
  bg_attention_desc att{};
};

struct Plan {
  std::vector<Step> steps;
  int64_t root_id = 0;
  int64_t peak_live_bytes = 0;
};


// Plan-level fusion (plan_fuse.cpp): rewrites groups of steps into single
// steps whose op names start with '+', which a wire plan cannot name.
// sem_axes: PERMUTE axes bound from a semantic side table (NULL: legacy
// route, axes in each PERMUTE's arg).
void fuse_plan(Plan& plan, const std::unordered_map<int64_t, std::vector<int64_t>>* sem_axes);

}  // namespace bg
