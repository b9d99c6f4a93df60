// Backward and optimizer kernels of the tensor-plan route for gfx950 (f32):
//   * LayerNorm backward: input (tensor_plan.ts:2209-2255), weight
//     (:2257-2295) and bias (:2297-2321) gradients; oracle
//     _realize.py:1008-1072.
//   * SGD / Adam / AdamW updates (tensor_plan.ts:2000-2168; oracle
//     _realize.py:1637-1721).
// All are HBM-bound.  Arithmetic follows the oracle's NumPy order with every
// operation rounded to f32 (no contraction in this build); the scalar
// constants arrive already rounded the way NumPy rounds a Python float that
// meets a float32 array (launch_optimizer).
//
// The reference's WGSL for the weight gradient runs one thread per column
// and recomputes every row's mean and variance in each of them
// (O(rows * cols^2) loads).  Here, for rows of up to 1024 columns, a block
// reads 16 whole rows once (a wavefront per row, statistics by shuffles),
// accumulates each column's sum in registers and writes one partial row;
// wider rows take a statistics pass and one thread per column over chunks of
// 16 rows.  A last kernel adds the partial rows with 16 lanes per column and
// a fixed-order combine, so results do not depend on scheduling.
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

// dX for aligned rows of 1025 to NT * 4 * NV columns: one NT-thread
// workgroup per row, thread t holding float4 groups j * NT + t of x and of
// g = dy * w in registers; each row statistic (sum x, centred sum of squares,
// sum g, sum g * x_hat) is summed per wavefront (shuffles), then over the
// wavefronts through LDS in wavefront order.  One read of dy and x, one
// write of dx (the wavefront-per-row kernel below reads the row three times).
template <int NT, int NV>
__global__ void __launch_bounds__(NT) ln_bwd_input_row_kernel(const float4* __restrict__ dy,
                                                              const float4* __restrict__ x,
                                                              const float4* __restrict__ w,
                                                              float4* __restrict__ dx, int64_t cols, float eps) {
  constexpr int NWV = NT / 64;
  __shared__ float red[3][NWV];
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int64_t groups = cols >> 2;
  const int64_t base = int64_t(blockIdx.x) * groups;
  const float n = float(cols);
  auto block_sum = [&](float v, int slot) {
    v = wave_sum(v);
    if (lane == 0) red[slot][wv] = v;
    __syncthreads();
    float r = 0.f;
#pragma unroll
    for (int i = 0; i < NWV; ++i) r += red[slot][i];
    return r;
  };
  float4 v[NV], g[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int64_t c = int64_t(j) * NT + t;
    v[j] = c < groups ? x[base + c] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
  const float mean = block_sum(s, 0) / n;
  float q = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int64_t c = int64_t(j) * NT + t;
    v[j] = make_float4(v[j].x - mean, v[j].y - mean, v[j].z - mean, v[j].w - mean);
    if (c < groups) q += (v[j].x * v[j].x + v[j].y * v[j].y) + (v[j].z * v[j].z + v[j].w * v[j].w);
  }
  const float inv = 1.0f / sqrtf(block_sum(q, 1) / n + eps);
  float sg = 0.f, sgx = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int64_t c = int64_t(j) * NT + t;
    v[j] = make_float4(v[j].x * inv, v[j].y * inv, v[j].z * inv, v[j].w * inv);  // x_hat
    if (c < groups) {
      const float4 d = dy[base + c], ww = w[c];
      g[j] = make_float4(d.x * ww.x, d.y * ww.y, d.z * ww.z, d.w * ww.w);
    } else {
      g[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    sg += (g[j].x + g[j].y) + (g[j].z + g[j].w);
    sgx += (g[j].x * v[j].x + g[j].y * v[j].y) + (g[j].z * v[j].z + g[j].w * v[j].w);
  }
  // Two statistics in one pass through LDS.
  sg = wave_sum(sg);
  sgx = wave_sum(sgx);
  if (lane == 0) {
    red[2][wv] = sg;
    red[0][wv] = sgx;  // slot 0's mean was read by every thread before the second barrier
  }
  __syncthreads();
  float tsg = 0.f, tsgx = 0.f;
#pragma unroll
  for (int i = 0; i < NWV; ++i) {
    tsg += red[2][i];
    tsgx += red[0][i];
  }
  const float k = inv / n;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int64_t c = int64_t(j) * NT + t;
    if (c < groups)
      dx[base + c] = make_float4(k * ((n * g[j].x - tsg) - v[j].x * tsgx), k * ((n * g[j].y - tsg) - v[j].y * tsgx),
                                 k * ((n * g[j].z - tsg) - v[j].z * tsgx), k * ((n * g[j].w - tsg) - v[j].w * tsgx));
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

// The same statistics for aligned rows of up to NT * 4 * NV columns: one
// NT-thread workgroup per row, the row read once into registers, wavefront
// sums combined through LDS in wavefront order.
template <int NT, int NV>
__global__ void __launch_bounds__(NT) ln_row_stats_row_kernel(const float4* __restrict__ x,
                                                              float* __restrict__ stats, int64_t cols, float eps) {
  constexpr int NWV = NT / 64;
  __shared__ float red[2][NWV];
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int64_t groups = cols >> 2;
  const int64_t base = int64_t(blockIdx.x) * groups;
  const float n = float(cols);
  float4 v[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int64_t c = int64_t(j) * NT + t;
    v[j] = c < groups ? x[base + c] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
  s = wave_sum(s);
  if (lane == 0) red[0][wv] = s;
  __syncthreads();
  float ts = 0.f;
#pragma unroll
  for (int i = 0; i < NWV; ++i) ts += red[0][i];
  const float mean = ts / n;
  float q = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int64_t c = int64_t(j) * NT + t;
    const float4 a = make_float4(v[j].x - mean, v[j].y - mean, v[j].z - mean, v[j].w - mean);
    if (c < groups) q += (a.x * a.x + a.y * a.y) + (a.z * a.z + a.w * a.w);
  }
  q = wave_sum(q);
  if (lane == 0) red[1][wv] = q;
  __syncthreads();
  if (t == 0) {
    float tq = 0.f;
#pragma unroll
    for (int i = 0; i < NWV; ++i) tq += red[1][i];
    stats[2 * blockIdx.x] = mean;
    stats[2 * blockIdx.x + 1] = 1.0f / sqrtf(tq / n + eps);
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

// Column sums for rows held in registers (cols <= 64 * PER): a block owns
// 4 * RPW consecutive rows and wavefront w takes RPW of them, w, w+4, ...,
// issuing the loads of all its rows before any arithmetic (rows past the end
// are clamped to the last row and not accumulated).  For the weight
// gradient each wavefront computes its rows' mean and inv_std with shuffles
// (no separate statistics pass, x read once) and accumulates dy * x_hat per
// column in registers.  The four wavefronts' sums are added in a fixed order
// through LDS into part[block][c].
template <int PER, int RPW, bool WEIGHT>
__global__ void __launch_bounds__(256) ln_col_rows_kernel(const float* __restrict__ dy, const float* __restrict__ x,
                                                          float* __restrict__ part, int64_t rows, int64_t cols,
                                                          float eps) {
  __shared__ float sm[4][64 * PER];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const float n = float(cols);
  const int64_t r0 = int64_t(blockIdx.x) * (4 * RPW) + w;
  float d[RPW][PER];
  float v[WEIGHT ? RPW : 1][PER];
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int64_t base = min(r0 + 4 * i, rows - 1) * cols;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int64_t c = int64_t(j) * 64 + lane;
      d[i][j] = c < cols ? dy[base + c] : 0.f;
      if constexpr (WEIGHT) v[i][j] = c < cols ? x[base + c] : 0.f;
    }
  }
  float acc[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) acc[j] = 0.f;
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    if (r0 + 4 * i >= rows) break;  // wave-uniform
    if constexpr (WEIGHT) {
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < PER; ++j) s += v[i][j];
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
      const float mean = s / n;
      float q = 0.f;
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        const int64_t c = int64_t(j) * 64 + lane;
        v[i][j] = v[i][j] - mean;
        if (c < cols) q += v[i][j] * v[i][j];
      }
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) q += __shfl_xor(q, o, 64);
      const float inv = 1.0f / sqrtf(q / n + eps);
#pragma unroll
      for (int j = 0; j < PER; ++j) acc[j] += d[i][j] * (v[i][j] * inv);
    } else {
#pragma unroll
      for (int j = 0; j < PER; ++j) acc[j] += d[i][j];
    }
  }
#pragma unroll
  for (int j = 0; j < PER; ++j) sm[w][j * 64 + lane] = acc[j];
  __syncthreads();
  for (int64_t c = threadIdx.x; c < cols; c += 256)
    part[int64_t(blockIdx.x) * cols + c] = ((sm[0][c] + sm[1][c]) + sm[2][c]) + sm[3][c];
}

// out[c] = sum over k < chunks of part[k][c]: 16 columns per 1024-thread
// block, 64 lanes per column each summing every 64th partial row (their
// loads all in flight, 64 bytes of one partial row per 16 lanes), then one
// lane per column adds the 64 sums in lane order (deterministic).
__global__ void __launch_bounds__(1024) ln_col_final_kernel(const float* __restrict__ part, float* __restrict__ out,
                                                            int64_t chunks, int64_t cols) {
  __shared__ float sm[64][17];
  const int cl = threadIdx.x & 15;
  const int kl = threadIdx.x >> 4;
  const int64_t c = int64_t(blockIdx.x) * 16 + cl;
  float acc = 0.f;
  if (c < cols) {
    int64_t k = kl;
    for (; k + 3 * 64 < chunks; k += 4 * 64) {
      float t[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) t[u] = part[(k + 64 * u) * cols + c];
#pragma unroll
      for (int u = 0; u < 4; ++u) acc += t[u];
    }
    for (; k < chunks; k += 64) acc += part[k * cols + c];
  }
  sm[kl][cl] = acc;
  __syncthreads();
  if (kl == 0 && c < cols) {
    float t = 0.f;
#pragma unroll 8
    for (int i = 0; i < 64; ++i) t += sm[i][cl];
    out[c] = t;
  }
}

typedef float lnf4 __attribute__((ext_vector_type(4)));

// float4 form of ln_col_rows_kernel for 4-aligned rows of at most 256 * PER4
// columns: lane l of a wavefront owns column groups j * 64 + l (j < PER4, 4
// columns each); a block of NW wavefronts owns NW * RPW consecutive rows,
// wavefront w the rows w, w + NW, ...  Every load is unconditional (row and
// group indices clamped, out-of-range values zeroed after the load), so a
// wavefront issues all of them before its first row reduction.  The NW
// wavefront sums are added in wavefront order through LDS into part[block].
template <int PER4, int RPW, int NW, bool WEIGHT>
__global__ void __launch_bounds__(NW * 64) ln_col4_kernel(const lnf4* __restrict__ dy, const lnf4* __restrict__ x,
                                                        lnf4* __restrict__ part, int64_t rows, int64_t groups,
                                                        float eps) {
  __shared__ lnf4 sm[NW][64 * PER4];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const float n = float(groups * 4);
  const int64_t r0 = int64_t(blockIdx.x) * (NW * RPW) + w;
  lnf4 d[RPW][PER4];
  lnf4 v[WEIGHT ? RPW : 1][PER4];
  bool gin[PER4];
  int64_t gc[PER4];
#pragma unroll
  for (int j = 0; j < PER4; ++j) {
    gin[j] = int64_t(j) * 64 + lane < groups;
    gc[j] = min(int64_t(j) * 64 + lane, groups - 1);
  }
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int64_t base = min(r0 + NW * i, rows - 1) * groups;
#pragma unroll
    for (int j = 0; j < PER4; ++j) {
      d[i][j] = dy[base + gc[j]];
      if constexpr (WEIGHT) v[i][j] = x[base + gc[j]];
    }
  }
#pragma unroll
  for (int i = 0; i < RPW; ++i)
#pragma unroll
    for (int j = 0; j < PER4; ++j) {
      if (!gin[j]) d[i][j] = lnf4{0.f, 0.f, 0.f, 0.f};
      if constexpr (WEIGHT)
        if (!gin[j]) v[i][j] = lnf4{0.f, 0.f, 0.f, 0.f};
    }
  lnf4 acc[PER4];
#pragma unroll
  for (int j = 0; j < PER4; ++j) acc[j] = lnf4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    // Rows past the end repeat the last row (clamped above) and are dropped
    // by selects, not by a branch: a branch would let the compiler sink
    // their loads behind the previous row's reductions.
    const bool rin = r0 + NW * i < rows;
    if constexpr (WEIGHT) {
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < PER4; ++j) s += (v[i][j].x + v[i][j].y) + (v[i][j].z + v[i][j].w);
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
      const float mean = s / n;
      float q = 0.f;
#pragma unroll
      for (int j = 0; j < PER4; ++j) {
        lnf4 t = v[i][j] - mean;
        if (!gin[j]) t = lnf4{0.f, 0.f, 0.f, 0.f};
        v[i][j] = t;
        q += (t.x * t.x + t.y * t.y) + (t.z * t.z + t.w * t.w);
      }
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) q += __shfl_xor(q, o, 64);
      const float inv = 1.0f / sqrtf(q / n + eps);
#pragma unroll
      for (int j = 0; j < PER4; ++j) {
        const lnf4 t = acc[j] + d[i][j] * (v[i][j] * inv);
        acc[j] = rin ? t : acc[j];
      }
    } else {
#pragma unroll
      for (int j = 0; j < PER4; ++j) {
        const lnf4 t = acc[j] + d[i][j];
        acc[j] = rin ? t : acc[j];
      }
    }
  }
#pragma unroll
  for (int j = 0; j < PER4; ++j) sm[w][j * 64 + lane] = acc[j];
  __syncthreads();
  for (int64_t g = threadIdx.x; g < groups; g += NW * 64) {
    lnf4 t = sm[0][g];
#pragma unroll
    for (int u = 1; u < NW; ++u) t += sm[u][g];
    part[int64_t(blockIdx.x) * groups + g] = t;
  }
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
  // Fused steps only: the M and V steps' own betas (and Adam's decays).
  float mb1, momb1, vb2, vomb2;
  float mwd, vwd;
};

constexpr int optim_arity(int kind) {
  return kind == BG_OPT_ADAMW_PARAM || kind == bg::kOptAdamwFused || kind == bg::kOptAdamFused
             ? 4
             : (kind >= BG_OPT_ADAM_M ? 3 : 2);
}

// One element of each update, in the oracle's operation order; v holds the
// element of each input in bg_optimizer_update order.
template <int KIND>
__device__ __forceinline__ float optim_val(const OptimConsts& k, const float (&v)[4]) {
  if constexpr (KIND == BG_OPT_SGD) {  // param, grad
    float u = v[1];
    if (k.has_wd) u = u + k.wd * v[0];
    return v[0] - k.lr * u;
  } else if constexpr (KIND == BG_OPT_ADAMW_M) {  // m, grad
    return k.b1 * v[0] + k.omb1 * v[1];
  } else if constexpr (KIND == BG_OPT_ADAMW_V) {  // v, grad
    return k.b2 * v[0] + k.omb2 * (v[1] * v[1]);
  } else if constexpr (KIND == BG_OPT_ADAMW_PARAM) {  // param, grad, m_new, v_new
    const float mh = v[2] / k.c1;
    const float vh = v[3] / k.c2;
    const float u = mh / (sqrtf(vh) + k.eps);
    return (v[0] - k.lr * u) - k.lr_wd * v[0];
  } else if constexpr (KIND == BG_OPT_ADAM_M) {  // param, grad, m
    float g = v[1];
    if (k.has_wd) g = g + k.wd * v[0];
    return k.b1 * v[2] + k.omb1 * g;
  } else if constexpr (KIND == BG_OPT_ADAM_V) {  // param, grad, v
    float g = v[1];
    if (k.has_wd) g = g + k.wd * v[0];
    return k.b2 * v[2] + k.omb2 * (g * g);
  } else if constexpr (KIND == BG_OPT_ADAM_PARAM) {  // param, m_new, v_new
    const float mh = v[1] / k.c1;
    const float vh = v[2] / k.c2;
    return v[0] - k.lr * (mh / (sqrtf(vh) + k.eps));
  } else if constexpr (KIND == bg::kOptAdamFused) {  // param, grad, m, v -> ADAM_UPDATE_M, _V, _PARAM
    const float gm = k.mwd != 0.f ? v[1] + k.mwd * v[0] : v[1];
    const float gv = k.vwd != 0.f ? v[1] + k.vwd * v[0] : v[1];
    const float m_new = k.mb1 * v[2] + k.momb1 * gm;
    const float v_new = k.vb2 * v[3] + k.vomb2 * (gv * gv);
    const float mh = m_new / k.c1;
    const float vh = v_new / k.c2;
    return v[0] - k.lr * (mh / (sqrtf(vh) + k.eps));
  } else {  // kOptAdamwFused: param, grad, m, v -> the ADAMW_UPDATE_M, _V and _PARAM chain
    const float m_new = k.mb1 * v[2] + k.momb1 * v[1];
    const float v_new = k.vb2 * v[3] + k.vomb2 * (v[1] * v[1]);
    const float mh = m_new / k.c1;
    const float vh = v_new / k.c2;
    const float u = mh / (sqrtf(vh) + k.eps);
    return (v[0] - k.lr * u) - k.lr_wd * v[0];
  }
}

template <int KIND>
__device__ __forceinline__ float4 optim_vec(const OptimConsts& k, const float4 (&x)[4]) {
  constexpr int NIN = optim_arity(KIND);
  float r[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float v[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < NIN; ++q) v[q] = e == 0 ? x[q].x : e == 1 ? x[q].y : e == 2 ? x[q].z : x[q].w;
    r[e] = optim_val<KIND>(k, v);
  }
  return make_float4(r[0], r[1], r[2], r[3]);
}

// Grid-stride update of n elements.  VEC (every buffer 16-byte aligned):
// each thread takes two float4 groups per iteration, issuing all their loads
// before any arithmetic; the n % 4 tail goes one element per thread.
template <int KIND, bool VEC>
__global__ void __launch_bounds__(256) optim_kernel(OptimConsts k, const float* __restrict__ a,
                                                    const float* __restrict__ b, const float* __restrict__ c,
                                                    const float* __restrict__ d, float* __restrict__ out,
                                                    int64_t n) {
  constexpr int NIN = optim_arity(KIND);
  const float* in[4] = {a, b, c, d};
  const int64_t tid = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t T = int64_t(gridDim.x) * blockDim.x;
  int64_t done = 0;
  if constexpr (VEC) {
    const int64_t nv = n >> 2;
    for (int64_t v0 = tid; v0 < nv; v0 += 2 * T) {
      const int64_t v1 = v0 + T;
      const bool two = v1 < nv;
      float4 x0[4], x1[4];
#pragma unroll
      for (int q = 0; q < NIN; ++q) {
        x0[q] = reinterpret_cast<const float4*>(in[q])[v0];
        if (two) x1[q] = reinterpret_cast<const float4*>(in[q])[v1];
      }
      reinterpret_cast<float4*>(out)[v0] = optim_vec<KIND>(k, x0);
      if (two) reinterpret_cast<float4*>(out)[v1] = optim_vec<KIND>(k, x1);
    }
    done = nv << 2;
  }
  for (int64_t i = done + tid; i < n; i += T) {
    float v[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < NIN; ++q) v[q] = in[q][i];
    out[i] = optim_val<KIND>(k, v);
  }
}

template <int KIND>
void launch_optim_kind(bg_ctx* ctx, const OptimConsts& k, const float* const (&in)[4], float* out, int64_t n,
                       bool vec) {
  const int64_t blocks = std::min<int64_t>((n + 2047) / 2048, 8192);
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
  const auto al16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  const dim3 grid(unsigned((rows + 3) / 4));
  if (cols <= 256)
    bg::dispatch(ctx, ln_bwd_input_kernel<4>, grid, dim3(256), 0, dy, x, w, dx, rows, cols, eps);
  else if (cols <= 512)
    bg::dispatch(ctx, ln_bwd_input_kernel<8>, grid, dim3(256), 0, dy, x, w, dx, rows, cols, eps);
  else if (cols <= 768)
    bg::dispatch(ctx, ln_bwd_input_kernel<12>, grid, dim3(256), 0, dy, x, w, dx, rows, cols, eps);
  else if (cols <= 1024)
    bg::dispatch(ctx, ln_bwd_input_kernel<16>, grid, dim3(256), 0, dy, x, w, dx, rows, cols, eps);
  else if (cols % 4 == 0 && cols <= 1024 * 4 * 8 && rows <= 0x7fffffff && al16(dy) && al16(x) && al16(w) &&
           al16(dx)) {
    // A workgroup per row: 256 threads up to 8192 columns, else 1024.
    const dim3 rgrid(static_cast<unsigned>(rows));
    const float4 *dy4 = reinterpret_cast<const float4*>(dy), *x4 = reinterpret_cast<const float4*>(x),
                 *w4 = reinterpret_cast<const float4*>(w);
    float4* dx4 = reinterpret_cast<float4*>(dx);
    if (cols <= 256 * 4 * 2)
      bg::dispatch(ctx, ln_bwd_input_row_kernel<256, 2>, rgrid, dim3(256), 0, dy4, x4, w4, dx4, cols, eps);
    else if (cols <= 256 * 4 * 4)
      bg::dispatch(ctx, ln_bwd_input_row_kernel<256, 4>, rgrid, dim3(256), 0, dy4, x4, w4, dx4, cols, eps);
    else if (cols <= 256 * 4 * 8)
      bg::dispatch(ctx, ln_bwd_input_row_kernel<256, 8>, rgrid, dim3(256), 0, dy4, x4, w4, dx4, cols, eps);
    else if (cols <= 1024 * 4 * 4)
      bg::dispatch(ctx, ln_bwd_input_row_kernel<1024, 4>, rgrid, dim3(1024), 0, dy4, x4, w4, dx4, cols, eps);
    else
      bg::dispatch(ctx, ln_bwd_input_row_kernel<1024, 8>, rgrid, dim3(1024), 0, dy4, x4, w4, dx4, cols, eps);
  } else {
    bg::dispatch(ctx, ln_bwd_input_wide_kernel, grid, dim3(256), 0, dy, x, w, dx, rows, cols, eps);
  }
  hip_check(hipGetLastError(), "layer_norm_backward_input launch");
}

template <int PER>
void launch_ln_col_rows(bg_ctx* ctx, const float* dy, const float* x, float* part, int64_t rows, int64_t cols,
                        int64_t blocks, float eps, bool weight) {
  if (weight)
    bg::dispatch(ctx, ln_col_rows_kernel<PER, 4, true>, dim3(unsigned(blocks)), dim3(256), 0, dy, x, part, rows,
                 cols, eps);
  else
    bg::dispatch(ctx, ln_col_rows_kernel<PER, 4, false>, dim3(unsigned(blocks)), dim3(256), 0, dy, x, part, rows,
                 cols, eps);
}

template <int PER4>
void launch_ln_col4(bg_ctx* ctx, const lnf4* dy, const lnf4* x, lnf4* part, int64_t rows, int64_t groups,
                    int64_t blocks, float eps, bool weight) {
  constexpr int RPW = 2, NW = 8;
  if (weight)
    bg::dispatch(ctx, ln_col4_kernel<PER4, RPW, NW, true>, dim3(unsigned(blocks)), dim3(NW * 64), 0, dy, x, part,
                 rows, groups, eps);
  else
    bg::dispatch(ctx, ln_col4_kernel<PER4, RPW, NW, false>, dim3(unsigned(blocks)), dim3(NW * 64), 0, dy, x, part,
                 rows, groups, eps);
}

void launch_ln_backward_cols(bg_ctx* ctx, const float* dy, const float* x, float* out, int64_t rows, int64_t cols,
                             float eps, bool weight) {
  float* part;
  int64_t chunks;
  const bool al4 = cols % 4 == 0 && (reinterpret_cast<uintptr_t>(dy) & 15) == 0 &&
                   (!weight || (reinterpret_cast<uintptr_t>(x) & 15) == 0);
  if (al4 && cols <= 1024) {
    // 16-byte loads, 16 rows per block (2 per wavefront, 8 wavefronts).
    const int64_t rpb = 16;
    chunks = (rows + rpb - 1) / rpb;
    part = static_cast<float*>(bg::scratch(ctx, size_t(chunks * cols) * sizeof(float), 0));
    const lnf4* dy4 = reinterpret_cast<const lnf4*>(dy);
    const lnf4* x4 = reinterpret_cast<const lnf4*>(weight ? x : dy);
    lnf4* p4 = reinterpret_cast<lnf4*>(part);
    const int64_t g = cols / 4;
    if (cols <= 256)
      launch_ln_col4<1>(ctx, dy4, x4, p4, rows, g, chunks, eps, weight);
    else if (cols <= 512)
      launch_ln_col4<2>(ctx, dy4, x4, p4, rows, g, chunks, eps, weight);
    else if (cols <= 768)
      launch_ln_col4<3>(ctx, dy4, x4, p4, rows, g, chunks, eps, weight);
    else
      launch_ln_col4<4>(ctx, dy4, x4, p4, rows, g, chunks, eps, weight);
  } else if (cols <= 1024) {
    // Rows held in registers, 16 rows per block (4 per wavefront).
    const int64_t rpb = 16;  // 4 * RPW
    chunks = (rows + rpb - 1) / rpb;
    part = static_cast<float*>(bg::scratch(ctx, size_t(chunks * cols) * sizeof(float), 0));
    if (cols <= 256)
      launch_ln_col_rows<4>(ctx, dy, x, part, rows, cols, chunks, eps, weight);
    else if (cols <= 512)
      launch_ln_col_rows<8>(ctx, dy, x, part, rows, cols, chunks, eps, weight);
    else if (cols <= 768)
      launch_ln_col_rows<12>(ctx, dy, x, part, rows, cols, chunks, eps, weight);
    else
      launch_ln_col_rows<16>(ctx, dy, x, part, rows, cols, chunks, eps, weight);
  } else {
    // Wide rows: row statistics first, then one thread per column over
    // chunks of 16 rows, for ~2 blocks of 256 columns per chunk and CU.
    const int64_t col_blocks = (cols + 255) / 256;
    const int64_t rpc = std::max<int64_t>(16, (rows + 65534) / 65535);  // grid y <= 65535
    chunks = (rows + rpc - 1) / rpc;
    size_t ws = size_t(chunks * cols) * sizeof(float);
    if (weight) ws += size_t(rows) * 2 * sizeof(float);
    part = static_cast<float*>(bg::scratch(ctx, ws, 0));
    float* stats = weight ? part + chunks * cols : nullptr;
    const bool row_stats = weight && cols % 4 == 0 && cols <= 1024 * 4 * 8 && rows <= 0x7fffffff &&
                           (reinterpret_cast<uintptr_t>(x) & 15) == 0;
    if (row_stats) {
      // A workgroup per row, the row read once.
      const dim3 rgrid(static_cast<unsigned>(rows));
      const float4* x4 = reinterpret_cast<const float4*>(x);
      if (cols <= 256 * 4 * 2)
        bg::dispatch(ctx, ln_row_stats_row_kernel<256, 2>, rgrid, dim3(256), 0, x4, stats, cols, eps);
      else if (cols <= 256 * 4 * 4)
        bg::dispatch(ctx, ln_row_stats_row_kernel<256, 4>, rgrid, dim3(256), 0, x4, stats, cols, eps);
      else if (cols <= 256 * 4 * 8)
        bg::dispatch(ctx, ln_row_stats_row_kernel<256, 8>, rgrid, dim3(256), 0, x4, stats, cols, eps);
      else if (cols <= 1024 * 4 * 4)
        bg::dispatch(ctx, ln_row_stats_row_kernel<1024, 4>, rgrid, dim3(1024), 0, x4, stats, cols, eps);
      else
        bg::dispatch(ctx, ln_row_stats_row_kernel<1024, 8>, rgrid, dim3(1024), 0, x4, stats, cols, eps);
    } else if (weight) {
      bg::dispatch(ctx, ln_row_stats_kernel, dim3(unsigned((rows + 3) / 4)), dim3(256), 0, x, stats, rows, cols,
                   eps);
    }
    if (weight)
      bg::dispatch(ctx, ln_col_partial_kernel<true>, dim3(unsigned(col_blocks), unsigned(chunks)), dim3(256), 0, dy,
                   x, stats, part, rows, cols, rpc);
    else
      bg::dispatch(ctx, ln_col_partial_kernel<false>, dim3(unsigned(col_blocks), unsigned(chunks)), dim3(256), 0,
                   dy, x, stats, part, rows, cols, rpc);
  }
  bg::dispatch(ctx, ln_col_final_kernel, dim3(unsigned((cols + 15) / 16)), dim3(1024), 0, part, out, chunks, cols);
  hip_check(hipGetLastError(), "layer_norm_backward column launch");
}

static OptimConsts optim_consts(const bg_optim_args& a);

void launch_optimizer_fused(bg_ctx* ctx, int kind, const bg_optim_args& a, double m_beta1, double v_beta2,
                            double m_wd, double v_wd, const float* const (&in)[4], float* out, int64_t n) {
  if (n == 0) return;
  OptimConsts k = optim_consts(a);
  k.mb1 = float(m_beta1);
  k.momb1 = float(1.0 - m_beta1);
  k.vb2 = float(v_beta2);
  k.vomb2 = float(1.0 - v_beta2);
  // Adam folds each moment step's weight decay into that step's gradient
  // (f32(wd) is nonzero exactly when wd is, for the finite wd accepted).
  k.mwd = kind == kOptAdamFused ? float(m_wd) : 0.f;
  k.vwd = kind == kOptAdamFused ? float(v_wd) : 0.f;
  bool vec = reinterpret_cast<uintptr_t>(out) % 16 == 0;
  for (const float* p : in) vec = vec && reinterpret_cast<uintptr_t>(p) % 16 == 0;
  if (kind == kOptAdamFused) launch_optim_kind<kOptAdamFused>(ctx, k, in, out, n, vec);
  else launch_optim_kind<kOptAdamwFused>(ctx, k, in, out, n, vec);
  hip_check(hipGetLastError(), "optimizer_update launch");
}

static OptimConsts optim_consts(const bg_optim_args& a) {
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
  return k;
}

void launch_optimizer(bg_ctx* ctx, int kind, const bg_optim_args& a, const float* const (&in)[4], float* out,
                      int64_t n) {
  if (n == 0) return;
  OptimConsts k = optim_consts(a);
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
