// Tensor-plan executor (placeholder until the JSON plan route lands).
#include "core.h"

namespace bg {

bg_handle run_plan(bg_ctx* ctx, const char* json, const int64_t* ids,
                   const bg_handle* handles, int n, int dtype) {
  (void)ctx; (void)json; (void)ids; (void)handles; (void)n; (void)dtype;
  fail(BG_E_UNSUPPORTED, "run_tensor_plan: not available in this build");
}

}  // namespace bg
