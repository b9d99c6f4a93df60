// Backward and optimizer kernels of the tensor-plan route for gfx950 (f32):
//   * LayerNorm backward: input (tensor_plan.ts:2209-2255), weight
//     (:2257-2295) and bias (:2297-2321) gradients; oracle
//     _realize.py:1008-1072.
//   * SGD / Adam / AdamW updates (tensor_plan.ts:2000-2168; oracle
//     _realize.py:1637-1721).
// All are HBM-bound.  Arithmetic follows the oracle's NumPy order with every
// operation rounded to f32 (no contraction in this build); the scalar
// constants arrive already rounded the way NumPy rounds a Python float that
// meets a float32 array (see bg_optimizer_update).
//
// The reference's WGSL recomputes each row's mean and variance once per
// column for the weight gradient (O(rows * cols^2)); here the row statistics
// are computed once (a wavefront per row), the column sums run as coalesced
// per-column partial sums over row chunks, and a last pass adds the partials
// in a fixed order, so results do not depend on scheduling.
#include <algorithm>
#include <cmath>

#include "common.cuh"
#include "core.h"

namespace {

using namespace bgk;

// ---- LayerNorm backward --------------------------------------------------------

// dx for one row per wavefront, the row held in registers (cols <= 64 * PER):
//   mean, centered, var, inv_std as in the forward pass, x_hat = centered * inv,
//   g = dy * w, sum_g, sum_gx = sum(g * x_hat),
//   dx = (inv / n) * (n * g - sum_g - x_hat * sum_gx).
template <int PER>
__global__ void __launch_bounds__(256) ln_bwd_input_kernel(const float* __restrict__ dy, const float* __restrict__ x,
                                                           const float* __restrict__ w, float* __restrict__ dx,
                                                           int64_t rows, int64_t cols, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // no block-level barriers below
  const int64_t base = row * cols;
  const float n = float(cols);
  float v[PER];
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int64_t c = int64_t(j) * 64 + lane;
    v[j] = c < cols ? x[base + c] : 0.f;
    s += v[j];
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
  const float mean = s / n;
  float q = 0.f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int64_t c = int64_t(j) * 64 + lane;
    const float cv = v[j] - mean;
    v[j] = cv;
    if (c < cols) q += cv * cv;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) q += __shfl_xor(q, o, 64);
  const float inv = 1.0f / sqrtf(q / n + eps);
  float g[PER];
  float sg = 0.f, sgx = 0.f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int64_t c = int64_t(j) * 64 + lane;
    v[j] = v[j] * inv;  // x_hat
    g[j] = c < cols ? dy[base + c] * w[c] : 0.f;
    sg += g[j];
    sgx += g[j] * v[j];
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    sg += __shfl_xor(sg, o, 64);
    sgx += __shfl_xor(sgx, o, 64);
  }
  const float k = inv / n;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int64_t c = int64_t(j) * 64 + lane;
    if (c < cols) {
      const float t = n * g[j] - sg;
      dx[base + c] = k * (t - v[j] * sgx);
    }
  }
}

// Same for rows wider than the register-resident variants: three passes over
// global memory per row.
__global__ void __launch_bounds__(256) ln_bwd_input_wide_kernel(const float* __restrict__ dy,
                                                                const float* __restrict__ x,
                                                                const float* __restrict__ w, float* __restrict__ dx,
                                                                int64_t rows, int64_t cols, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t base = row * cols;
  const float n = float(cols);
  float s = 0.f;
  for (int64_t c = lane; c < cols; c += 64) s += x[base + c];
  for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
  const float mean = s / n;
  float q = 0.f;
  for (int64_t c = lane; c < cols; c += 64) {
    const float cv = x[base + c] - mean;
    q += cv * cv;
  }
  for (int o = 32; o >= 1; o >>= 1) q += __shfl_xor(q, o, 64);
  const float inv = 1.0f / sqrtf(q / n + eps);
  float sg = 0.f, sgx = 0.f;
  for (int64_t c = lane; c < cols; c += 64) {
    const float xh = (x[base + c] - mean) * inv;
    const float gv = dy[base + c] * w[c];
    sg += gv;
    sgx += gv * xh;
  }
  for (int o = 32; o >= 1; o >>= 1) {
    sg += __shfl_xor(sg, o, 64);
    sgx += __shfl_xor(sgx, o, 64);
  }
  const float k = inv / n;
  for (int64_t c = lane; c < cols; c += 64) {
    const float xh = (x[base + c] - mean) * inv;
    const float t = n * (dy[base + c] * w[c]) - sg;
    dx[base + c] = k * (t - xh * sgx);
  }
}

// Row statistics for the weight gradient: stats[2 r] = mean, stats[2 r + 1]
// = inv_std, one wavefront per row.
__global__ void __launch_bounds__(256) ln_row_stats_kernel(const float* __restrict__ x, float* __restrict__ stats,
                                                           int64_t rows, int64_t cols, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t base = row * cols;
  const float n = float(cols);
  float s = 0.f;
  for (int64_t c = lane; c < cols; c += 64) s += x[base + c];
  for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
  const float mean = s / n;
  float q = 0.f;
  for (int64_t c = lane; c < cols; c += 64) {
    const float cv = x[base + c] - mean;
    q += cv * cv;
  }
  for (int o = 32; o >= 1; o >>= 1) q += __shfl_xor(q, o, 64);
  if (lane == 0) {
    stats[2 * row] = mean;
    stats[2 * row + 1] = 1.0f / sqrtf(q / n + eps);
  }
}

// Column partial sums over one chunk of rows: part[chunk][c] = sum over the
// chunk's rows r of dy[r][c] * x_hat[r][c] (WEIGHT) or dy[r][c] (BIAS).  A
// thread owns one column, so every row's loads are coalesced across lanes.
template <bool WEIGHT>
__global__ void __launch_bounds__(256) ln_col_partial_kernel(const float* __restrict__ dy,
                                                             const float* __restrict__ x,
                                                             const float* __restrict__ stats,
                                                             float* __restrict__ part, int64_t rows, int64_t cols,
                                                             int64_t rows_per_chunk) {
  const int64_t c = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (c >= cols) return;
  const int64_t r0 = int64_t(blockIdx.y) * rows_per_chunk;
  const int64_t r1 = min(rows, r0 + rows_per_chunk);
  float acc = 0.f;
  for (int64_t r = r0; r < r1; ++r) {
    const float d = dy[r * cols + c];
    if constexpr (WEIGHT) {
      const float xh = (x[r * cols + c] - stats[2 * r]) * stats[2 * r + 1];
      acc += d * xh;
    } else {
      acc += d;
    }
  }
  part[int64_t(blockIdx.y) * cols + c] = acc;
}

// out[c] = sum over chunks (in order) of part[chunk][c].
__global__ void __launch_bounds__(256) ln_col_final_kernel(const float* __restrict__ part, float* __restrict__ out,
                                                           int64_t chunks, int64_t cols) {
  const int64_t c = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (c >= cols) return;
  float acc = 0.f;
  for (int64_t k = 0; k < chunks; ++k) acc += part[k * cols + c];
  out[c] = acc;
}

// ---- optimizer updates -------------------------------------------------------------

struct OptimConsts {
  float lr;      // f32(lr)
  float b1;      // f32(beta1)
  float omb1;    // f32(1 - beta1), the difference taken in double
  float b2;      // f32(beta2)
  float omb2;    // f32(1 - beta2)
  float eps;     // f32(eps)
  float wd;      // f32(weight_decay)
  float lr_wd;   // f32(lr * weight_decay), the product taken in double
  float c1;      // f32(1 - beta1^step), in double
  float c2;      // f32(1 - beta2^step), in double
  int has_wd;    // weight_decay != 0 (the oracle skips the term otherwise)
};

// One element of each update, in the oracle's operation order.
template <int KIND>
__device__ __forceinline__ float optim_elem(const OptimConsts& k, const float* const (&in)[4], int64_t i) {
  if constexpr (KIND == BG_OPT_SGD) {  // in: param, grad
    const float p = in[0][i];
    float u = in[1][i];
    if (k.has_wd) u = u + k.wd * p;
    return p - k.lr * u;
  } else if constexpr (KIND == BG_OPT_ADAMW_M) {  // in: m, grad
    return k.b1 * in[0][i] + k.omb1 * in[1][i];
  } else if constexpr (KIND == BG_OPT_ADAMW_V) {  // in: v, grad
    const float gv = in[1][i];
    return k.b2 * in[0][i] + k.omb2 * (gv * gv);
  } else if constexpr (KIND == BG_OPT_ADAMW_PARAM) {  // in: param, grad, m_new, v_new
    const float p = in[0][i];
    const float mh = in[2][i] / k.c1;
    const float vh = in[3][i] / k.c2;
    const float u = mh / (sqrtf(vh) + k.eps);
    return (p - k.lr * u) - k.lr_wd * p;
  } else if constexpr (KIND == BG_OPT_ADAM_M) {  // in: param, grad, m
    float gv = in[1][i];
    if (k.has_wd) gv = gv + k.wd * in[0][i];
    return k.b1 * in[2][i] + k.omb1 * gv;
  } else if constexpr (KIND == BG_OPT_ADAM_V) {  // in: param, grad, v
    float gv = in[1][i];
    if (k.has_wd) gv = gv + k.wd * in[0][i];
    return k.b2 * in[2][i] + k.omb2 * (gv * gv);
  } else {  // BG_OPT_ADAM_PARAM, in: param, m_new, v_new
    const float mh = in[1][i] / k.c1;
    const float vh = in[2][i] / k.c2;
    return in[0][i] - k.lr * (mh / (sqrtf(vh) + k.eps));
  }
}

// Grid-stride over n elements; each thread handles 4 consecutive elements per
// iteration (16-byte accesses when every buffer is 16-byte aligned, which
// the caller checks through VEC).
template <int KIND, bool VEC>
__global__ void __launch_bounds__(256) optim_kernel(OptimConsts k, const float* a, const float* b, const float* c,
                                                    const float* d, float* __restrict__ out, int64_t n) {
  const float* const in[4] = {a, b, c, d};
  const int64_t stride = int64_t(gridDim.x) * blockDim.x * 4;
  for (int64_t i = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) * 4; i < n; i += stride) {
    if (VEC && i + 3 < n) {
      float r[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) r[j] = optim_elem<KIND>(k, in, i + j);
      *reinterpret_cast<float4*>(out + i) = make_float4(r[0], r[1], r[2], r[3]);
    } else {
      for (int64_t j = i; j < min(n, i + 4); ++j) out[j] = optim_elem<KIND>(k, in, j);
    }
  }
}

template <int KIND>
void launch_optim_kind(bg_ctx* ctx, const OptimConsts& k, const float* const (&in)[4], float* out, int64_t n,
                       bool vec) {
  const int64_t blocks = std::min<int64_t>((n + 1023) / 1024, 8192);
  const dim3 grid(unsigned(std::max<int64_t>(blocks, 1)));
  if (vec)
    bg::dispatch(ctx, optim_kernel<KIND, true>, grid, dim3(256), 0, k, in[0], in[1], in[2], in[3], out, n);
  else
    bg::dispatch(ctx, optim_kernel<KIND, false>, grid, dim3(256), 0, k, in[0], in[1], in[2], in[3], out, n);
}

}  // namespace

namespace bg {

void launch_ln_backward_input(bg_ctx* ctx, const float* dy, const float* x, const float* w, float* dx,
                              int64_t rows, int64_t cols, float eps) {
  if (rows == 0) return;
  const dim3 grid(unsigned((rows + 3) / 4));
  if (cols <= 256)
    bg::dispatch(ctx, ln_bwd_input_kernel<4>, grid, dim3(256), 0, dy, x, w, dx, rows, cols, eps);
  else if (cols <= 1024)
    bg::dispatch(ctx, ln_bwd_input_kernel<16>, grid, dim3(256), 0, dy, x, w, dx, rows, cols, eps);
  else
    bg::dispatch(ctx, ln_bwd_input_wide_kernel, grid, dim3(256), 0, dy, x, w, dx, rows, cols, eps);
  hip_check(hipGetLastError(), "layer_norm_backward_input launch");
}

void launch_ln_backward_cols(bg_ctx* ctx, const float* dy, const float* x, float* out, int64_t rows, int64_t cols,
                             float eps, bool weight) {
  // Enough row chunks for ~4 workgroups per CU; each thread sums at least
  // 16 rows of its column.
  const int64_t col_blocks = (cols + 255) / 256;
  int64_t chunks = std::max<int64_t>(1, std::min<int64_t>((rows + 15) / 16, 1024 / std::max<int64_t>(col_blocks, 1)));
  const int64_t rpc = (rows + chunks - 1) / chunks;
  chunks = (rows + rpc - 1) / rpc;
  float* stats = nullptr;
  size_t ws = size_t(chunks * cols) * sizeof(float);
  if (weight) ws += size_t(rows) * 2 * sizeof(float);
  float* part = static_cast<float*>(bg::scratch(ctx, ws, 0));
  if (weight) {
    stats = part + chunks * cols;
    bg::dispatch(ctx, ln_row_stats_kernel, dim3(unsigned((rows + 3) / 4)), dim3(256), 0, x, stats, rows, cols, eps);
    bg::dispatch(ctx, ln_col_partial_kernel<true>, dim3(unsigned(col_blocks), unsigned(chunks)), dim3(256), 0, dy,
                 x, stats, part, rows, cols, rpc);
  } else {
    bg::dispatch(ctx, ln_col_partial_kernel<false>, dim3(unsigned(col_blocks), unsigned(chunks)), dim3(256), 0, dy,
                 x, stats, part, rows, cols, rpc);
  }
  bg::dispatch(ctx, ln_col_final_kernel, dim3(unsigned(col_blocks)), dim3(256), 0, part, out, chunks, cols);
  hip_check(hipGetLastError(), "layer_norm_backward column launch");
}

void launch_optimizer(bg_ctx* ctx, int kind, const bg_optim_args& a, const float* const (&in)[4], float* out,
                      int64_t n) {
  if (n == 0) return;
  OptimConsts k{};
  k.lr = float(a.lr);
  k.b1 = float(a.beta1);
  k.omb1 = float(1.0 - a.beta1);
  k.b2 = float(a.beta2);
  k.omb2 = float(1.0 - a.beta2);
  k.eps = float(a.eps);
  k.wd = float(a.weight_decay);
  k.lr_wd = float(a.lr * a.weight_decay);
  k.c1 = float(1.0 - std::pow(a.beta1, double(a.step)));
  k.c2 = float(1.0 - std::pow(a.beta2, double(a.step)));
  k.has_wd = a.weight_decay != 0.0;
  bool vec = reinterpret_cast<uintptr_t>(out) % 16 == 0;
  for (const float* p : in) vec = vec && (p == nullptr || reinterpret_cast<uintptr_t>(p) % 16 == 0);
  switch (kind) {
    case BG_OPT_SGD: launch_optim_kind<BG_OPT_SGD>(ctx, k, in, out, n, vec); break;
    case BG_OPT_ADAMW_M: launch_optim_kind<BG_OPT_ADAMW_M>(ctx, k, in, out, n, vec); break;
    case BG_OPT_ADAMW_V: launch_optim_kind<BG_OPT_ADAMW_V>(ctx, k, in, out, n, vec); break;
    case BG_OPT_ADAMW_PARAM: launch_optim_kind<BG_OPT_ADAMW_PARAM>(ctx, k, in, out, n, vec); break;
    case BG_OPT_ADAM_M: launch_optim_kind<BG_OPT_ADAM_M>(ctx, k, in, out, n, vec); break;
    case BG_OPT_ADAM_V: launch_optim_kind<BG_OPT_ADAM_V>(ctx, k, in, out, n, vec); break;
    default: launch_optim_kind<BG_OPT_ADAM_PARAM>(ctx, k, in, out, n, vec); break;
  }
  hip_check(hipGetLastError(), "optimizer_update launch");
}

}  // namespace bg
