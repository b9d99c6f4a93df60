// Data-movement and normalisation kernels for gfx950:
//   * cast between f32 / f16 / bf16 with round-to-nearest-even narrowing
//     (the reference bridge only copies f32->f32, realizer.ts:1087-1120; the
//     oracle is NumPy astype, _realize.py:210-212);
//   * cast + batched 2-D transpose through LDS (GEMM operand re-layout);
//   * strided gather copy (PERMUTE / SLICE / BROADCAST materialisation,
//     tensor_plan.ts:824-997);
//   * LayerNorm, one wavefront per row with the row held in registers
//     (tensor_plan.ts:2170-2208; oracle _realize.py:1008-1034);
//   * a generic attention kernel (one wavefront per query row) used for f32,
//     for additive masks (flash_attention.ts:45-131) and for head sizes the
//     MFMA kernel does not cover.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <type_traits>

#include "common.cuh"
#include "core.h"

namespace {

using namespace bgk;

// ---- cast -------------------------------------------------------------------

__global__ void __launch_bounds__(256) cast_kernel(const void* __restrict__ src, int sd,
                                                   void* __restrict__ dst, int dd, int64_t n) {
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  int64_t i = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
  for (; i + 3 < n; i += stride * 4) {
    float v[4];
    if (sd == 0) {
      float4 t = *reinterpret_cast<const float4*>(static_cast<const float*>(src) + i);
      v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
    } else {
      uint2 t = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(src) + i);
      uint16_t h[4] = {uint16_t(t.x), uint16_t(t.x >> 16), uint16_t(t.y), uint16_t(t.y >> 16)};
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = sd == 1 ? f16_bits_to_f32(h[j]) : bf16_bits_to_f32(h[j]);
    }
    if (dd == 0) {
      *reinterpret_cast<float4*>(static_cast<float*>(dst) + i) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
      uint16_t h[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) h[j] = dd == 1 ? f32_to_f16_bits(v[j]) : f32_to_bf16_bits(v[j]);
      uint2 t;
      t.x = uint32_t(h[0]) | (uint32_t(h[1]) << 16);
      t.y = uint32_t(h[2]) | (uint32_t(h[3]) << 16);
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(dst) + i) = t;
    }
  }
  // Tail (at most 3 elements, handled by the thread that reached it).
  if (i < n) {
    for (; i < n; ++i) store_from_f32(dst, dd, i, load_as_f32(src, sd, i));
  }
}

__global__ void __launch_bounds__(256) cast_scalar_kernel(const void* __restrict__ src, int sd,
                                                          void* __restrict__ dst, int dd, int64_t n) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += int64_t(gridDim.x) * blockDim.x)
    store_from_f32(dst, dd, i, load_as_f32(src, sd, i));
}

// dst[b][c][r] = src[b][r][c] converted; 64x64 tiles through LDS.
__global__ void __launch_bounds__(256) cast_transpose_kernel(const void* __restrict__ src, int sd,
                                                             void* __restrict__ dst, int dd,
                                                             int64_t rows, int64_t cols) {
  __shared__ float tile[64][65];
  const int64_t b = blockIdx.z;
  const int64_t r0 = int64_t(blockIdx.y) * 64, c0 = int64_t(blockIdx.x) * 64;
  const int tx = threadIdx.x % 64, ty = threadIdx.x / 64;
  const int64_t base = b * rows * cols;
  for (int y = ty; y < 64; y += 4) {
    const int64_t r = r0 + y, c = c0 + tx;
    tile[y][tx] = (r < rows && c < cols) ? load_as_f32(src, sd, base + r * cols + c) : 0.f;
  }
  __syncthreads();
  for (int y = ty; y < 64; y += 4) {
    const int64_t c = c0 + y, r = r0 + tx;
    if (r < rows && c < cols) store_from_f32(dst, dd, base + c * rows + r, tile[tx][y]);
  }
}

// Compile-time-dtype forms of the two casts for aligned data (the branchy
// kernels above stay for the unaligned remainder of cases).
template <int D>
__device__ __forceinline__ float cvt_in(uint32_t w, int half) {
  const uint16_t h = uint16_t(half ? w >> 16 : w);
  return D == 1 ? f16_bits_to_f32(h) : bf16_bits_to_f32(h);
}
template <int D>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  const uint16_t x = D == 1 ? f32_to_f16_bits(a) : f32_to_bf16_bits(a);
  const uint16_t y = D == 1 ? f32_to_f16_bits(b) : f32_to_bf16_bits(b);
  return uint32_t(x) | (uint32_t(y) << 16);
}
// 8 consecutive elements as f32 (a 32-byte f32 or 16-byte 16-bit load).
template <int SD>
__device__ __forceinline__ void load8(const void* src, int64_t i, float (&v)[8]) {
  if constexpr (SD == 0) {
    const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(src) + i);
    const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(src) + i + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    const uint4 a = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(src) + i);
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = cvt_in<SD>(w[j >> 1], j & 1);
  }
}
template <int DD>
__device__ __forceinline__ void store8(void* dst, int64_t i, const float (&v)[8]) {
  if constexpr (DD == 0) {
    float* d = static_cast<float*>(dst) + i;
    *reinterpret_cast<float4*>(d) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4*>(d + 4) = make_float4(v[4], v[5], v[6], v[7]);
  } else {
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(dst) + i) =
        make_uint4(pack2<DD>(v[0], v[1]), pack2<DD>(v[2], v[3]), pack2<DD>(v[4], v[5]), pack2<DD>(v[6], v[7]));
  }
}

// n % 8 == 0, both pointers 16-byte aligned: 8 elements per lane per step.
template <int SD, int DD>
__global__ void __launch_bounds__(256) cast8_kernel(const void* __restrict__ src, void* __restrict__ dst,
                                                    int64_t n8) {
  const int64_t stride = int64_t(gridDim.x) * 256;
  for (int64_t g = int64_t(blockIdx.x) * 256 + threadIdx.x; g < n8; g += stride) {
    float v[8];
    load8<SD>(src, g * 8, v);
    store8<DD>(dst, g * 8, v);
  }
}

// dst[b][c][r] = src[b][r][c] converted, rows % 8 == cols % 8 == 0, both
// pointers 16-byte aligned.  64 x 64 tiles: each lane loads 8 consecutive
// columns of one row (two passes of 32 rows), the tile sits in LDS as f32
// with a one-word row pad, and each lane stores 8 consecutive dst elements
// (8 source rows of one column).
template <int SD, int DD>
__global__ void __launch_bounds__(256) cast_transpose8_kernel(const void* __restrict__ src, void* __restrict__ dst,
                                                              int64_t rows, int64_t cols) {
  __shared__ float tile[64][65];
  const int64_t base = int64_t(blockIdx.z) * rows * cols;
  const int64_t r0 = int64_t(blockIdx.y) * 64, c0 = int64_t(blockIdx.x) * 64;
  const int t = threadIdx.x;
  const int lc = (t & 7) * 8, lr = t >> 3;  // 8 lanes per 64-wide row, 32 rows per pass
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int rr = lr + 32 * p;
    float v[8];
    if (r0 + rr < rows && c0 + lc < cols) {
      load8<SD>(src, base + (r0 + rr) * cols + c0 + lc, v);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = 0.f;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) tile[rr][lc + j] = v[j];
  }
  __syncthreads();
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int cc = lr + 32 * p;  // dst row = source column c0 + cc
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = tile[lc + j][cc];
    if (c0 + cc < cols && r0 + lc < rows) store8<DD>(dst, base + (c0 + cc) * rows + r0 + lc, v);
  }
}

// ---- strided copy -------------------------------------------------------------

struct CopyArgs {
  int64_t shape[BG_MAX_RANK];
  int64_t stride[BG_MAX_RANK];
  int rank;
  int64_t n;
};

template <typename T>
__global__ void __launch_bounds__(256) copy_strided_kernel(const T* __restrict__ src,
                                                           T* __restrict__ dst, CopyArgs A) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < A.n;
       i += int64_t(gridDim.x) * blockDim.x) {
    int64_t rem = i, off = 0;
    for (int d = A.rank - 1; d >= 0; --d) {
      const int64_t idx = rem % A.shape[d];
      rem /= A.shape[d];
      off += idx * A.stride[d];
    }
    dst[i] = src[off];
  }
}

// Unsigned 32-bit division by a runtime constant as a multiply-high and a
// shift (the round-up method of Granlund and Montgomery, "Division by
// invariant integers using multiplication", PLDI 1994): for d >= 1,
// l = ceil(log2 d), m = floor(2^32 (2^l - d) / d) + 1, and
// n / d = (mulhi(n, m) + ((n - mulhi(n, m)) >> 1)) >> (l - 1) for l >= 1,
// n itself for d = 1; exact for every 32-bit n.
struct FastDiv {
  uint32_t d, m, s;
};

static FastDiv make_fastdiv(uint32_t d) {
  FastDiv f{d, 0u, 0u};
  uint32_t l = 0;
  while ((uint64_t(1) << l) < d) ++l;
  f.m = uint32_t(((uint64_t(1) << 32) * ((uint64_t(1) << l) - d)) / d + 1);
  f.s = l;
  return f;
}

__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) {
  if (f.d == 1) return n;
  const uint32_t t = __umulhi(n, f.m);
  return (t + ((n - t) >> 1)) >> (f.s - 1);
}

// Row copy: dst[row][v] = src[off(row) + v] in 16-byte pieces, rows of
// `rv` pieces; off(row) from up to 3 outer dims (byte strides).
struct RowCopyArgs {
  FastDiv rv;          // pieces per row
  FastDiv dim[3];      // outer dims, innermost first
  int64_t bstride[3];  // their source strides in bytes
  int nd;
  uint32_t total;      // pieces in all
};

__global__ void __launch_bounds__(256) copy_rows16_kernel(const char* __restrict__ src, uint4* __restrict__ dst,
                                                          RowCopyArgs A) {
  for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < A.total; i += gridDim.x * 256u) {
    uint32_t row = fdiv(i, A.rv);
    const uint32_t v = i - row * A.rv.d;
    int64_t off = int64_t(v) * 16;
#pragma unroll
    for (int d = 0; d < 3; ++d) {
      if (d < A.nd) {
        const uint32_t q = fdiv(row, A.dim[d]);
        off += int64_t(row - q * A.dim[d].d) * A.bstride[d];
        row = q;
      }
    }
    dst[i] = *reinterpret_cast<const uint4*>(src + off);
  }
}

// Batched transpose through LDS: dst is [batch...][K][I] in the collapsed
// order with I innermost, the source has I at stride si and K at stride 1.
// A 64 x 64 tile is read along K (coalesced), written along I.
struct TransposeArgs {
  int64_t I, K, si, dk;  // dk: destination stride of K (elements)
  int64_t tiles_i, tiles_k;
  FastDiv bdim[2];       // batch dims, innermost first
  int64_t bsrc[2], bdst[2];
  int nb;
  int kfast;             // consecutive workgroups step along K (else along I)
};

template <typename T>
__global__ void __launch_bounds__(256) copy_transpose_kernel(const T* __restrict__ src, T* __restrict__ dst,
                                                             TransposeArgs A) {
  __shared__ T tile[64][65];
  const int64_t per_b = A.tiles_i * A.tiles_k;
  uint32_t b = static_cast<uint32_t>(blockIdx.x / per_b);
  const int64_t t = blockIdx.x - int64_t(b) * per_b;
  const int64_t i0 = (A.kfast ? t / A.tiles_k : t % A.tiles_i) * 64;
  const int64_t k0 = (A.kfast ? t % A.tiles_k : t / A.tiles_i) * 64;
  int64_t so = 0, dof = 0;
#pragma unroll
  for (int d = 0; d < 2; ++d) {
    if (d < A.nb) {
      const uint32_t q = fdiv(b, A.bdim[d]);
      const int64_t idx = b - q * A.bdim[d].d;
      so += idx * A.bsrc[d];
      dof += idx * A.bdst[d];
      b = q;
    }
  }
  const int lane = threadIdx.x & 63, row = threadIdx.x >> 6;
  // Read: lane along K (source stride 1), rows along I.
#pragma unroll 4
  for (int r = row; r < 64; r += 4) {
    const int64_t i = i0 + r, k = k0 + lane;
    if (i < A.I && k < A.K) tile[r][lane] = src[so + i * A.si + k];
  }
  __syncthreads();
  // Write: lane along I (destination stride 1), rows along K.
#pragma unroll 4
  for (int r = row; r < 64; r += 4) {
    const int64_t i = i0 + lane, k = k0 + r;
    if (i < A.I && k < A.K) dst[dof + k * A.dk + i] = tile[lane][r];
  }
}

// ---- Softmax over the last axis (FUSED_SOFTMAX) -------------------------------
// The reference kernel's order (kernels/softmax.ts:22-69): m = max(x);
// e = exp(x - m); y = e * (1 / sum(e)).  One wavefront per row, the row held
// in registers (PER values per lane); rows wider than 64*PER stream three
// times through memory.

template <int PER>
__global__ void __launch_bounds__(256) softmax_rows_kernel(const void* __restrict__ x, int xd,
                                                           void* __restrict__ y, int yd, int64_t rows,
                                                           int64_t cols) {
  const int lane = threadIdx.x & 63;
  const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // no block-level barriers below
  const int64_t base = row * cols;
  float v[PER];
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int64_t c = int64_t(j) * 64 + lane;
    v[j] = c < cols ? load_as_f32(x, xd, base + c) : -INFINITY;
    m = fmaxf(m, v[j]);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int64_t c = int64_t(j) * 64 + lane;
    const float e = c < cols ? expf(v[j] - m) : 0.f;
    v[j] = e;
    s += e;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
  const float inv = 1.0f / s;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int64_t c = int64_t(j) * 64 + lane;
    if (c < cols) store_from_f32(y, yd, base + c, v[j] * inv);
  }
}

__global__ void __launch_bounds__(256) softmax_rows_wide_kernel(const void* __restrict__ x, int xd,
                                                                void* __restrict__ y, int yd, int64_t rows,
                                                                int64_t cols) {
  const int lane = threadIdx.x & 63;
  const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t base = row * cols;
  float m = -INFINITY;
  for (int64_t c = lane; c < cols; c += 64) m = fmaxf(m, load_as_f32(x, xd, base + c));
  for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  float s = 0.f;
  for (int64_t c = lane; c < cols; c += 64) s += expf(load_as_f32(x, xd, base + c) - m);
  for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
  const float inv = 1.0f / s;
  for (int64_t c = lane; c < cols; c += 64)
    store_from_f32(y, yd, base + c, expf(load_as_f32(x, xd, base + c) - m) * inv);
}

// ---- LayerNorm -----------------------------------------------------------------
// Same arithmetic as the oracle: mean = sum/cols; centered = x - mean;
// var = sum(centered^2)/cols; inv = 1/sqrt(var + eps); y = centered*inv*w + b,
// every step rounded to f32 (no contraction in this file).

template <int PER>
__global__ void __launch_bounds__(256) layer_norm_kernel(const void* __restrict__ x, int xd,
                                                         const float* __restrict__ w,
                                                         const float* __restrict__ bias,
                                                         void* __restrict__ y, int yd,
                                                         int64_t rows, int64_t cols, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // no block-level barriers below
  const int64_t base = row * cols;
  float v[PER];
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int64_t c = int64_t(j) * 64 + lane;
    v[j] = c < cols ? load_as_f32(x, xd, base + c) : 0.f;
    s += v[j];
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
  const float mean = s / float(cols);
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
  const float var = q / float(cols);
  const float inv = 1.0f / sqrtf(var + eps);
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int64_t c = int64_t(j) * 64 + lane;
    if (c < cols) {
      const float xh = v[j] * inv;
      const float t = xh * w[c];
      store_from_f32(y, yd, base + c, t + bias[c]);
    }
  }
}

// Vectorised LayerNorm for rows whose width is a multiple of 4: a wavefront
// per row, the row in registers as NV groups of 4 consecutive columns per
// lane (16-byte f32 or 8-byte 16-bit loads and stores), input and output
// dtypes fixed at compile time.  Same operation order as layer_norm_kernel:
// mean, centred values, mean of squares, 1/sqrt(var + eps), x_hat * w + b.
template <int D>
__device__ __forceinline__ float4 ln_load4(const void* __restrict__ p, int64_t g) {
  if constexpr (D == BG_F32) {
    return reinterpret_cast<const float4*>(p)[g];
  } else {
    const uint2 u = reinterpret_cast<const uint2*>(p)[g];
    if constexpr (D == BG_F16) {
      return make_float4(f16_bits_to_f32(uint16_t(u.x)), f16_bits_to_f32(uint16_t(u.x >> 16)),
                         f16_bits_to_f32(uint16_t(u.y)), f16_bits_to_f32(uint16_t(u.y >> 16)));
    } else {
      return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u),
                         __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xffff0000u));
    }
  }
}

template <int D>
__device__ __forceinline__ void ln_store4(void* __restrict__ p, int64_t g, float4 v) {
  if constexpr (D == BG_F32) {
    reinterpret_cast<float4*>(p)[g] = v;
  } else if constexpr (D == BG_F16) {
    reinterpret_cast<uint2*>(p)[g] =
        make_uint2(uint32_t(f32_to_f16_bits(v.x)) | (uint32_t(f32_to_f16_bits(v.y)) << 16),
                   uint32_t(f32_to_f16_bits(v.z)) | (uint32_t(f32_to_f16_bits(v.w)) << 16));
  } else {
    reinterpret_cast<uint2*>(p)[g] =
        make_uint2(uint32_t(f32_to_bf16_bits(v.x)) | (uint32_t(f32_to_bf16_bits(v.y)) << 16),
                   uint32_t(f32_to_bf16_bits(v.z)) | (uint32_t(f32_to_bf16_bits(v.w)) << 16));
  }
}

template <int XD, int YD, int NV, int RW>
__global__ void __launch_bounds__(256) layer_norm_vec_kernel(const void* __restrict__ x,
                                                             const float* __restrict__ w,
                                                             const float* __restrict__ bias,
                                                             void* __restrict__ y, int64_t rows,
                                                             int64_t cols, float eps) {
  // RW rows per wavefront, their loads issued together; w and b are read
  // once per wavefront, before the row statistics need them.
  const int lane = threadIdx.x & 63;
  const int64_t row0 = (int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6)) * RW;
  if (row0 >= rows) return;  // no block-level barriers below
  const int64_t groups = cols >> 2;  // groups of 4 columns
  float4 v[RW][NV], wv[NV], bv[NV];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int64_t g = int64_t(j) * 64 + lane;
      v[r][j] = g < groups && row0 + r < rows ? ln_load4<XD>(x, (row0 + r) * groups + g)
                                             : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int64_t g = int64_t(j) * 64 + lane;
    wv[j] = g < groups ? reinterpret_cast<const float4*>(w)[g] : make_float4(0.f, 0.f, 0.f, 0.f);
    bv[j] = g < groups ? reinterpret_cast<const float4*>(bias)[g] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  float inv[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j) s += (v[r][j].x + v[r][j].y) + (v[r][j].z + v[r][j].w);
    const float mean = wave_sum(s) / float(cols);
    float q = 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int64_t g = int64_t(j) * 64 + lane;
      v[r][j] = make_float4(v[r][j].x - mean, v[r][j].y - mean, v[r][j].z - mean, v[r][j].w - mean);
      if (g < groups)
        q += (v[r][j].x * v[r][j].x + v[r][j].y * v[r][j].y) + (v[r][j].z * v[r][j].z + v[r][j].w * v[r][j].w);
    }
    const float var = wave_sum(q) / float(cols);
    inv[r] = 1.0f / sqrtf(var + eps);
  }
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    if (row0 + r >= rows) break;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int64_t g = int64_t(j) * 64 + lane;
      if (g < groups) {
        const float4 a = v[r][j];
        ln_store4<YD>(y, (row0 + r) * groups + g,
                      make_float4(a.x * inv[r] * wv[j].x + bv[j].x, a.y * inv[r] * wv[j].y + bv[j].y,
                                  a.z * inv[r] * wv[j].z + bv[j].z, a.w * inv[r] * wv[j].w + bv[j].w));
      }
    }
  }
}

// Rows of 2048 to 256 * 4 * NV columns (multiples of 4): one 256-thread
// workgroup per row, thread t holding the float4 groups j * 256 + t
// (j < NV) in registers; the row's sum and centred sum of squares are taken
// per wavefront (shuffles) and then over the four wavefronts through LDS in
// wavefront order.  One read of x and one write of y.
template <int XD, int YD, int NV>
__global__ void __launch_bounds__(256) layer_norm_row_kernel(const void* __restrict__ x,
                                                             const float* __restrict__ w,
                                                             const float* __restrict__ bias,
                                                             void* __restrict__ y, int64_t cols, float eps) {
  __shared__ float red[2][4];
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int64_t row = blockIdx.x;
  const int64_t groups = cols >> 2;
  float4 v[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int64_t g = int64_t(j) * 256 + t;
    v[j] = g < groups ? ln_load4<XD>(x, row * groups + g) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
  s = wave_sum(s);
  if (lane == 0) red[0][wv] = s;
  __syncthreads();
  const float mean = ((red[0][0] + red[0][1]) + (red[0][2] + red[0][3])) / float(cols);
  float q = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int64_t g = int64_t(j) * 256 + t;
    v[j] = make_float4(v[j].x - mean, v[j].y - mean, v[j].z - mean, v[j].w - mean);
    if (g < groups)
      q += (v[j].x * v[j].x + v[j].y * v[j].y) + (v[j].z * v[j].z + v[j].w * v[j].w);
  }
  q = wave_sum(q);
  if (lane == 0) red[1][wv] = q;
  __syncthreads();
  const float var = ((red[1][0] + red[1][1]) + (red[1][2] + red[1][3])) / float(cols);
  const float inv = 1.0f / sqrtf(var + eps);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int64_t g = int64_t(j) * 256 + t;
    if (g < groups) {
      const float4 a = v[j];
      const float4 wv4 = reinterpret_cast<const float4*>(w)[g];
      const float4 bv4 = reinterpret_cast<const float4*>(bias)[g];
      ln_store4<YD>(y, row * groups + g,
                    make_float4(a.x * inv * wv4.x + bv4.x, a.y * inv * wv4.y + bv4.y, a.z * inv * wv4.z + bv4.z,
                                a.w * inv * wv4.w + bv4.w));
    }
  }
}

// Softmax over aligned rows of up to NT * 4 * NV columns: one NT-thread
// workgroup per row, the row in registers (one read, one write); the max
// and the sum of exponentials are reduced per wavefront and then over the
// wavefronts through LDS in wavefront order.  Same arithmetic per element
// as softmax_rows_kernel: e = exp(x - max), y = e * (1 / sum).
template <int XD, int YD, int NT, int NV>
__global__ void __launch_bounds__(NT) softmax_row_kernel(const void* __restrict__ x, void* __restrict__ y,
                                                         int64_t cols) {
  constexpr int NWV = NT / 64;
  __shared__ float red[2][NWV];
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int64_t groups = cols >> 2;
  const int64_t base = int64_t(blockIdx.x) * groups;
  float4 v[NV];
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int64_t g = int64_t(j) * NT + t;
    v[j] = g < groups ? ln_load4<XD>(x, base + g) : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
    m = fmaxf(m, fmaxf(fmaxf(v[j].x, v[j].y), fmaxf(v[j].z, v[j].w)));
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  if (lane == 0) red[0][wv] = m;
  __syncthreads();
  m = red[0][0];
#pragma unroll
  for (int i = 1; i < NWV; ++i) m = fmaxf(m, red[0][i]);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int64_t g = int64_t(j) * NT + t;
    if (g < groups) {
      v[j] = make_float4(expf(v[j].x - m), expf(v[j].y - m), expf(v[j].z - m), expf(v[j].w - m));
      s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
    }
  }
  s = wave_sum(s);
  if (lane == 0) red[1][wv] = s;
  __syncthreads();
  float ts = 0.f;
#pragma unroll
  for (int i = 0; i < NWV; ++i) ts += red[1][i];
  const float inv = 1.0f / ts;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int64_t g = int64_t(j) * NT + t;
    if (g < groups)
      ln_store4<YD>(y, base + g, make_float4(v[j].x * inv, v[j].y * inv, v[j].z * inv, v[j].w * inv));
  }
}

// Softmax over rows of up to 1024 * PER columns of any alignment: one
// 1024-thread workgroup per row, thread t holding columns j * 1024 + t in
// registers (one read, one write).
template <int PER>
__global__ void __launch_bounds__(1024) softmax_row_scalar_kernel(const void* __restrict__ x, int xd,
                                                                  void* __restrict__ y, int yd, int64_t cols) {
  __shared__ float red[2][16];
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int64_t base = int64_t(blockIdx.x) * cols;
  float v[PER];
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int64_t c = int64_t(j) * 1024 + t;
    v[j] = c < cols ? load_as_f32(x, xd, base + c) : -INFINITY;
    m = fmaxf(m, v[j]);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  if (lane == 0) red[0][wv] = m;
  __syncthreads();
  m = red[0][0];
#pragma unroll
  for (int i = 1; i < 16; ++i) m = fmaxf(m, red[0][i]);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int64_t c = int64_t(j) * 1024 + t;
    v[j] = c < cols ? expf(v[j] - m) : 0.f;
    s += v[j];
  }
  s = wave_sum(s);
  if (lane == 0) red[1][wv] = s;
  __syncthreads();
  float ts = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) ts += red[1][i];
  const float inv = 1.0f / ts;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int64_t c = int64_t(j) * 1024 + t;
    if (c < cols) store_from_f32(y, yd, base + c, v[j] * inv);
  }
}

// Softmax over any row: one 1024-thread workgroup per row, three passes over
// the row (max, sum of exponentials, write), each coalesced across the
// workgroup (the wavefront-per-row kernel walks a long row with 64 lanes).
__global__ void __launch_bounds__(1024) softmax_block_wide_kernel(const void* __restrict__ x, int xd,
                                                                  void* __restrict__ y, int yd, int64_t cols) {
  __shared__ float red[2][16];
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int64_t base = int64_t(blockIdx.x) * cols;
  float m = -INFINITY;
  for (int64_t c = t; c < cols; c += 1024) m = fmaxf(m, load_as_f32(x, xd, base + c));
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  if (lane == 0) red[0][wv] = m;
  __syncthreads();
  m = red[0][0];
#pragma unroll
  for (int i = 1; i < 16; ++i) m = fmaxf(m, red[0][i]);
  float s = 0.f;
  for (int64_t c = t; c < cols; c += 1024) s += expf(load_as_f32(x, xd, base + c) - m);
  s = wave_sum(s);
  if (lane == 0) red[1][wv] = s;
  __syncthreads();
  float ts = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) ts += red[1][i];
  const float inv = 1.0f / ts;
  for (int64_t c = t; c < cols; c += 1024) store_from_f32(y, yd, base + c, expf(load_as_f32(x, xd, base + c) - m) * inv);
}

// Fallback for very wide rows: three passes over global memory.
__global__ void __launch_bounds__(256) layer_norm_wide_kernel(const void* __restrict__ x, int xd,
                                                              const float* __restrict__ w,
                                                              const float* __restrict__ bias,
                                                              void* __restrict__ y, int yd,
                                                              int64_t rows, int64_t cols, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t base = row * cols;
  float s = 0.f;
  for (int64_t c = lane; c < cols; c += 64) s += load_as_f32(x, xd, base + c);
  for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
  const float mean = s / float(cols);
  float q = 0.f;
  for (int64_t c = lane; c < cols; c += 64) {
    const float cv = load_as_f32(x, xd, base + c) - mean;
    q += cv * cv;
  }
  for (int o = 32; o >= 1; o >>= 1) q += __shfl_xor(q, o, 64);
  const float inv = 1.0f / sqrtf(q / float(cols) + eps);
  for (int64_t c = lane; c < cols; c += 64) {
    const float xh = (load_as_f32(x, xd, base + c) - mean) * inv;
    const float t = xh * w[c];
    store_from_f32(y, yd, base + c, t + bias[c]);
  }
}

// ---- generic attention ----------------------------------------------------------
// One wavefront per query row.  Lanes own keys in chunks of 64 for the score
// pass and own output dims (d = lane + 64*t) for the P@V pass.  Supports:
//   * one-pass online softmax (f32, the legacy kernel's m0 = -1e20 sentinel
//     and 1/l guard, flash_attention.ts:99-129);
//   * exact two-pass softmax with P rounded to the 16-bit input dtype before
//     P@V and scores rounded before scaling (the AMP SDPA graph,
//     _functional.py:1505-1533 realized by _realize.py handlers);
//   * additive f32 mask [1|B,1|H,Sq,Sk] and a causal flag (j > i masked,
//     np.triu(..., k=1) in the reference SDPA).

struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  const float* mask;
  void* o;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  int64_t mask_sb, mask_sh;
  int64_t B, H, Sq, Sk, D;
  float scale;
  int causal;
  int in_dtype;
  int out_dtype;
  int round_scores;
  int two_pass;
};

constexpr int kGenMaxD = 256;

__global__ void __launch_bounds__(256) attention_generic_kernel(AttnArgs A) {
  __shared__ float qs[4][kGenMaxD];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int64_t row = int64_t(blockIdx.x) * 4 + w;
  const int64_t total = A.B * A.H * A.Sq;
  const bool active = row < total;
  const int64_t rr = active ? row : 0;
  const int64_t i = rr % A.Sq;
  const int64_t bh = rr / A.Sq;
  const int64_t h = bh % A.H, b = bh / A.H;
  const char* qp = static_cast<const char*>(A.q);
  const int es = A.in_dtype == 0 ? 4 : 2;
  const int64_t qbase = b * A.q_sb + h * A.q_sh + i * A.q_ss;
  for (int64_t d = lane; d < A.D; d += 64) qs[w][d] = load_as_f32(qp, A.in_dtype, qbase + d);
  __syncthreads();
  (void)es;
  const int64_t kbase = b * A.k_sb + h * A.k_sh;
  const int64_t vbase = b * A.v_sb + h * A.v_sh;
  const float* mrow = A.mask ? A.mask + b * A.mask_sb + h * A.mask_sh + i * A.Sk : nullptr;
  const int64_t kend = A.causal ? std::min<int64_t>(A.Sk, i + 1) : A.Sk;

  auto score = [&](int64_t j) -> float {
    if (j >= kend) return -INFINITY;
    float s = 0.f;
    const int64_t kb = kbase + j * A.k_ss;
    for (int64_t d = 0; d < A.D; ++d) s += qs[w][d] * load_as_f32(A.k, A.in_dtype, kb + d);
    if (A.round_scores) s = round_through(s, A.in_dtype);
    s = s * A.scale;
    if (mrow) s = s + mrow[j];
    return s;
  };

  constexpr int kT = kGenMaxD / 64;
  float acc[kT];
#pragma unroll
  for (int t = 0; t < kT; ++t) acc[t] = 0.f;
  float m = -1.0e20f, l = 0.f;

  if (!A.two_pass) {
    for (int64_t j0 = 0; j0 < A.Sk; j0 += 64) {
      const int64_t j = j0 + lane;
      const float s = (active && j < A.Sk) ? score(j) : -INFINITY;
      float cmax = s;
      for (int o = 32; o >= 1; o >>= 1) cmax = fmaxf(cmax, __shfl_xor(cmax, o, 64));
      const float mn = fmaxf(m, cmax);
      const float alpha = expf(m - mn);
      const float p = expf(s - mn);
      float ps = p;
      for (int o = 32; o >= 1; o >>= 1) ps += __shfl_xor(ps, o, 64);
      l = alpha * l + ps;
      m = mn;
#pragma unroll
      for (int t = 0; t < kT; ++t) acc[t] *= alpha;
      const int64_t jn = std::min<int64_t>(64, A.Sk - j0);
      for (int jj = 0; jj < jn; ++jj) {
        const float pj = __shfl(p, jj, 64);
        const int64_t vb = vbase + (j0 + jj) * A.v_ss;
#pragma unroll
        for (int t = 0; t < kT; ++t) {
          const int64_t d = int64_t(t) * 64 + lane;
          if (d < A.D) acc[t] += pj * load_as_f32(A.v, A.in_dtype, vb + d);
        }
      }
    }
    const float inv = l > 0.f ? 1.0f / l : 0.f;
#pragma unroll
    for (int t = 0; t < kT; ++t) acc[t] *= inv;
  } else {
    // Pass 1: row max and sum of exp(s - max) (softmax in f32).
    float mx = -INFINITY;
    for (int64_t j0 = 0; j0 < A.Sk; j0 += 64) {
      const int64_t j = j0 + lane;
      const float s = (active && j < A.Sk) ? score(j) : -INFINITY;
      mx = fmaxf(mx, s);
    }
    for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    float sum = 0.f;
    for (int64_t j0 = 0; j0 < A.Sk; j0 += 64) {
      const int64_t j = j0 + lane;
      const float s = (active && j < A.Sk) ? score(j) : -INFINITY;
      sum += (j < A.Sk) ? expf(s - mx) : 0.f;
    }
    for (int o = 32; o >= 1; o >>= 1) sum += __shfl_xor(sum, o, 64);
    // Pass 2: P = exp(s - max) / sum rounded to the input dtype, then P@V.
    for (int64_t j0 = 0; j0 < A.Sk; j0 += 64) {
      const int64_t j = j0 + lane;
      const float s = (active && j < A.Sk) ? score(j) : -INFINITY;
      float p = (j < A.Sk) ? expf(s - mx) / sum : 0.f;
      p = round_through(p, A.in_dtype);
      const int64_t jn = std::min<int64_t>(64, A.Sk - j0);
      for (int jj = 0; jj < jn; ++jj) {
        const float pj = __shfl(p, jj, 64);
        const int64_t vb = vbase + (j0 + jj) * A.v_ss;
#pragma unroll
        for (int t = 0; t < kT; ++t) {
          const int64_t d = int64_t(t) * 64 + lane;
          if (d < A.D) acc[t] += pj * load_as_f32(A.v, A.in_dtype, vb + d);
        }
      }
    }
  }
  if (!active) return;
  const int64_t obase = b * A.o_sb + h * A.o_sh + i * A.o_ss;
#pragma unroll
  for (int t = 0; t < kT; ++t) {
    const int64_t d = int64_t(t) * 64 + lane;
    if (d < A.D) store_from_f32(A.o, A.out_dtype, obase + d, acc[t]);
  }
}

int grid1(int64_t n, int per) {
  return int(std::max<int64_t>(1, std::min<int64_t>((n + per - 1) / per, 256 * 64)));
}

// tanh-GELU over the rows of an f32 matrix (the GEMM's activation stage):
// dst[b][r][c] = gelu(src[b][r][c]) stored in dst_dtype.  One block per row
// chunk; four consecutive columns per lane when the rows allow it.
// residual: NULL or contiguous f32 [batch][rows][cols], added after GELU.
__global__ void __launch_bounds__(256) gelu_rows_kernel(const float* __restrict__ src, int64_t ld_src,
                                                        int64_t stride_src, void* __restrict__ dst,
                                                        int64_t ld_dst, int64_t stride_dst, int dd,
                                                        int64_t rows, int64_t cols, int64_t total_rows,
                                                        const float* __restrict__ residual) {
  for (int64_t rr = blockIdx.x; rr < total_rows; rr += gridDim.x) {
    const int64_t b = rr / rows, r = rr - b * rows;
    const float* s = src + b * stride_src + r * ld_src;
    const int64_t o = b * stride_dst + r * ld_dst;
    const float* res = residual ? residual + rr * cols : nullptr;
    for (int64_t c = threadIdx.x; c < cols; c += 256) {
      float g = gelu_tanh(s[c]);
      if (res) g = g + res[c];
      store_from_f32(dst, dd, o + c, g);
    }
  }
}

// Combines the per-chunk partials of a split row reduction: a workgroup per
// row, thread t folding chunks t, t + 256, ... in order, then a butterfly
// per wavefront and the 4 wavefronts in a fixed order; MAX and MIN
// propagate NaN like the single-pass kernel.
__device__ __forceinline__ float red_combine(int op, float a, float b) {
  if (op == BG_RED_MAX) return (a != a || b != b) ? a + b : fmaxf(a, b);
  if (op == BG_RED_MIN) return (a != a || b != b) ? a + b : fminf(a, b);
  return a + b;
}

__global__ void __launch_bounds__(256) reduce_partials_kernel(const float* __restrict__ part, int64_t nch,
                                                              int op, float cols, void* out, int out_dtype) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const float* p = part + row * nch;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float acc = op == BG_RED_MAX ? -__builtin_inff() : op == BG_RED_MIN ? __builtin_inff() : 0.f;
#pragma unroll 4
  for (int64_t k = threadIdx.x; k < nch; k += 256) acc = red_combine(op, acc, p[k]);
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) acc = red_combine(op, acc, __shfl_xor(acc, s, 64));
  if (lane == 0) red[wave] = acc;
  __syncthreads();
  if (threadIdx.x != 0) return;
  acc = red_combine(op, red_combine(op, red[0], red[1]), red_combine(op, red[2], red[3]));
  store_from_f32(out, out_dtype, row, op == BG_RED_MEAN ? acc / cols : acc);
}

// Reduction of x[B][R][C] over R (B = 1: the per-column sums of a bias
// gradient; B > 1: a block of middle axes), reading x once in place.  Workgroup = 4 wavefronts; a
// wavefront's lanes are LC column lanes (V adjacent columns each, so a row
// segment of LC * V columns is read contiguously) x 64 / LC row lanes.
// Workgroup u covers batch b = u / (ngroups * nchunk) and, within it, a
// column group and the rows of one chunk; inside it row r goes to row lane
// (r - r0) % (4 * 64 / LC).  Row lanes combine by a butterfly, wavefronts
// in order 0..3 through LDS.  With one chunk the result is final, otherwise
// it is the chunk's partial, stored at part[(chunk * B + b) * C + col].
template <int XD, int V>
__device__ __forceinline__ void load_v(const void* x, int64_t i, float (&v)[V]) {
  if constexpr (XD == 0) {
    if constexpr (V == 4) {
      const float4 t = *reinterpret_cast<const float4*>(static_cast<const float*>(x) + i);
      v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
    } else {
      v[0] = static_cast<const float*>(x)[i];
    }
  } else {
    const uint16_t* p = static_cast<const uint16_t*>(x) + i;
    if constexpr (V == 4) {
      const uint2 t = *reinterpret_cast<const uint2*>(p);
      const uint16_t h[4] = {uint16_t(t.x), uint16_t(t.x >> 16), uint16_t(t.y), uint16_t(t.y >> 16)};
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = XD == 1 ? f16_bits_to_f32(h[j]) : bf16_bits_to_f32(h[j]);
    } else {
      v[0] = XD == 1 ? f16_bits_to_f32(p[0]) : bf16_bits_to_f32(p[0]);
    }
  }
}

template <int XD, int V, int LC>
__global__ void __launch_bounds__(256) reduce_lead_kernel(const void* __restrict__ x, int64_t R, int64_t C,
                                                          int64_t CR, int64_t ngroups, int64_t nchunk,
                                                          int64_t B, int op, float* part, int final_out,
                                                          void* out, int od) {
  constexpr int RL = 64 / LC;
  __shared__ float red[4][64 * V];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int cl = lane % LC, rl = lane / LC;
  // Column groups rotate with the chunk, so the workgroups that share an
  // XCD (every eighth in dispatch order) do not all read the same few
  // column groups when ngroups divides by 8.
  const int64_t per_b = ngroups * nchunk;
  const int64_t b = blockIdx.x / per_b;
  const int64_t u = blockIdx.x - b * per_b;
  const int64_t chunk = u / ngroups;
  const int64_t group = (u % ngroups + chunk) % ngroups;
  x = static_cast<const char*>(x) + b * R * C * (XD == 0 ? 4 : 2);
  const int64_t col = (group * LC + cl) * V;
  const int64_t r0 = chunk * CR;
  const int64_t r1 = r0 + CR < R ? r0 + CR : R;
  const float ident = op == BG_RED_MAX ? -__builtin_inff() : op == BG_RED_MIN ? __builtin_inff() : 0.f;
  float acc[V];
#pragma unroll
  for (int j = 0; j < V; ++j) acc[j] = ident;
  if (col < C) {
#pragma unroll 4
    for (int64_t r = r0 + wave * RL + rl; r < r1; r += 4 * RL) {
      float v[V];
      load_v<XD, V>(x, r * C + col, v);
#pragma unroll
      for (int j = 0; j < V; ++j) acc[j] = red_combine(op, acc[j], v[j]);
    }
  }
#pragma unroll
  for (int s = LC; s < 64; s <<= 1)
#pragma unroll
    for (int j = 0; j < V; ++j) acc[j] = red_combine(op, acc[j], __shfl_xor(acc[j], s, 64));
  if (rl == 0)
#pragma unroll
    for (int j = 0; j < V; ++j) red[wave][cl * V + j] = acc[j];
  __syncthreads();
  if (wave != 0 || rl != 0 || col >= C) return;
#pragma unroll
  for (int j = 0; j < V; ++j) {
    float a = red[0][cl * V + j];
    a = red_combine(op, a, red[1][cl * V + j]);
    a = red_combine(op, a, red[2][cl * V + j]);
    a = red_combine(op, a, red[3][cl * V + j]);
    if (final_out)
      store_from_f32(out, od, b * C + col + j, op == BG_RED_MEAN ? a / static_cast<float>(R) : a);
    else
      part[(chunk * B + b) * C + col + j] = a;
  }
}

// Second pass: out[c] = the chunks' partials part[k][c], k = 0..nchunk-1.
// A workgroup covers 16 columns with 64 chunk lanes each: lane k folds
// chunks k, k + 64, ... in order; the 4 chunk lanes of a wavefront combine
// by a butterfly, then the 16 wavefronts in order through LDS.
__global__ void __launch_bounds__(1024) reduce_lead_final_kernel(const float* __restrict__ part, int64_t nchunk,
                                                                 int64_t C, int op, float R, void* out, int od) {
  __shared__ float red[16][16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int cx = lane & 15, k0 = wave * 4 + (lane >> 4);
  const int64_t c = int64_t(blockIdx.x) * 16 + cx;
  float acc = op == BG_RED_MAX ? -__builtin_inff() : op == BG_RED_MIN ? __builtin_inff() : 0.f;
  if (c < C) {
#pragma unroll 8
    for (int64_t k = k0; k < nchunk; k += 64) acc = red_combine(op, acc, part[k * C + c]);
  }
  acc = red_combine(op, acc, __shfl_xor(acc, 16, 64));
  acc = red_combine(op, acc, __shfl_xor(acc, 32, 64));
  if (lane < 16) red[wave][cx] = acc;
  __syncthreads();
  if (wave != 0 || lane >= 16 || c >= C) return;
  float a = red[0][cx];
#pragma unroll
  for (int w = 1; w < 16; ++w) a = red_combine(op, a, red[w][cx]);
  store_from_f32(out, od, c, op == BG_RED_MEAN ? a / R : a);
}

// Second pass for few chunks (at most 32): a thread per column folds its
// chunks in order.
__global__ void __launch_bounds__(256) reduce_lead_final_few_kernel(const float* __restrict__ part, int64_t nchunk,
                                                                    int64_t C, int op, float R, void* out, int od) {
  const int64_t c = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (c >= C) return;
  float a = part[c];
#pragma unroll 8
  for (int64_t k = 1; k < nchunk; ++k) a = red_combine(op, a, part[k * C + c]);
  store_from_f32(out, od, c, op == BG_RED_MEAN ? a / R : a);
}

}  // namespace

namespace bg {

// Instantiates f<SD, DD> for the runtime (sd, dd) pair of {f32, f16, bf16}.
template <typename F>
static void with_dtypes(int sd, int dd, F&& f) {
  auto inner = [&](auto s_tag) {
    constexpr int S = decltype(s_tag)::value;
    if (dd == 0) f(std::integral_constant<int, S>{}, std::integral_constant<int, 0>{});
    else if (dd == 1) f(std::integral_constant<int, S>{}, std::integral_constant<int, 1>{});
    else f(std::integral_constant<int, S>{}, std::integral_constant<int, 2>{});
  };
  if (sd == 0) inner(std::integral_constant<int, 0>{});
  else if (sd == 1) inner(std::integral_constant<int, 1>{});
  else inner(std::integral_constant<int, 2>{});
}

static bool cast_dtype(int d) { return d == 0 || d == 1 || d == 2; }

void launch_cast(bg_ctx* ctx, const void* src, int sd, void* dst, int dd, int64_t n) {
  if (n <= 0) return;
  const bool aligned = reinterpret_cast<uintptr_t>(src) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(dst) % 16 == 0;
  if (aligned && n % 8 == 0 && cast_dtype(sd) && cast_dtype(dd)) {
    const int64_t n8 = n / 8;
    const dim3 grid(unsigned(std::min<int64_t>((n8 + 255) / 256, 256 * 32)));
    with_dtypes(sd, dd, [&](auto S, auto D) {
      bg::dispatch(ctx, cast8_kernel<decltype(S)::value, decltype(D)::value>, grid, dim3(256), 0, src, dst, n8);
    });
  } else if (aligned) {
    bg::dispatch(ctx, cast_kernel, dim3(grid1(n / 4 + 1, 256)), dim3(256), 0,
                       src, sd, dst, dd, n);
  } else {
    bg::dispatch(ctx, cast_scalar_kernel, dim3(grid1(n, 256)), dim3(256), 0, src,
                       sd, dst, dd, n);
  }
  hip_check(hipGetLastError(), "cast launch");
}

void launch_cast_transpose(bg_ctx* ctx, const void* src, int sd, void* dst, int dd,
                           int64_t rows, int64_t cols, int64_t batch) {
  if (rows <= 0 || cols <= 0 || batch <= 0) return;
  if (batch > 65535) fail(BG_E_UNSUPPORTED, "cast_transpose: batch > 65535");
  dim3 grid(unsigned((cols + 63) / 64), unsigned((rows + 63) / 64), unsigned(batch));
  const bool vec = reinterpret_cast<uintptr_t>(src) % 16 == 0 && reinterpret_cast<uintptr_t>(dst) % 16 == 0 &&
                   rows % 8 == 0 && cols % 8 == 0 && cast_dtype(sd) && cast_dtype(dd);
  if (vec) {
    with_dtypes(sd, dd, [&](auto S, auto D) {
      bg::dispatch(ctx, cast_transpose8_kernel<decltype(S)::value, decltype(D)::value>, grid, dim3(256), 0, src,
                   dst, rows, cols);
    });
  } else {
    bg::dispatch(ctx, cast_transpose_kernel, grid, dim3(256), 0, src, sd, dst, dd,
                       rows, cols);
  }
  hip_check(hipGetLastError(), "cast_transpose launch");
}

void launch_copy_strided(bg_ctx* ctx, const void* src, int64_t es, void* dst,
                         const std::vector<int64_t>& shape, const std::vector<int64_t>& strides) {
  int64_t n = 1;
  for (int64_t v : shape) n *= v;
  if (n == 0) return;
  // Collapse: drop unit dims, merge a dim into the next one when the pair is
  // contiguous in the source.
  std::vector<int64_t> sh, st;
  for (size_t i = 0; i < shape.size(); ++i) {
    if (shape[i] == 1) continue;
    if (!sh.empty() && st.back() == strides[i] * shape[i]) {
      sh.back() *= shape[i];
      st.back() = strides[i];
    } else {
      sh.push_back(shape[i]);
      st.push_back(strides[i]);
    }
  }
  if (sh.empty()) {
    sh.push_back(1);
    st.push_back(1);
  }
  const int r = int(sh.size());
  bool nonneg = true;
  for (int64_t v : st) nonneg &= v >= 0;
  const bool fast = std::getenv("BG_COPY_GENERIC") == nullptr && nonneg && n * es < (int64_t(1) << 32);
  const uintptr_t sa = reinterpret_cast<uintptr_t>(src), da = reinterpret_cast<uintptr_t>(dst);
  // Rows contiguous in the source, in 16-byte pieces.
  if (fast && st.back() == 1 && r <= 4 && (sh.back() * es) % 16 == 0 && sa % 16 == 0 && da % 16 == 0) {
    bool ok = true;
    for (int d = 0; d < r - 1; ++d) ok &= (st[d] * es) % 16 == 0;
    if (ok) {
      RowCopyArgs A{};
      A.rv = make_fastdiv(uint32_t(sh.back() * es / 16));
      A.nd = r - 1;
      for (int d = 0; d < r - 1; ++d) {
        A.dim[d] = make_fastdiv(uint32_t(sh[r - 2 - d]));
        A.bstride[d] = st[r - 2 - d] * es;
      }
      A.total = uint32_t(n * es / 16);
      const unsigned g = unsigned(std::min<int64_t>((A.total + 255) / 256, 256 * 32));
      bg::dispatch(ctx, copy_rows16_kernel, dim3(g), dim3(256), 0, static_cast<const char*>(src),
                   static_cast<uint4*>(dst), A);
      return;
    }
  }
  // A transpose: the innermost destination dim is strided in the source and
  // another dim is the source's contiguous one; at most two more dims.
  if (fast && st.back() != 1 && r >= 2 && r <= 4) {
    int k = -1;
    for (int d = 0; d < r - 1; ++d)
      if (st[d] == 1) k = d;
    if (k >= 0) {
      TransposeArgs A{};
      A.I = sh[r - 1];
      A.K = sh[k];
      A.si = st[r - 1];
      std::vector<int64_t> dstr(r);
      int64_t acc = 1;
      for (int d = r - 1; d >= 0; --d) {
        dstr[d] = acc;
        acc *= sh[d];
      }
      A.dk = dstr[k];
      A.tiles_i = (A.I + 63) / 64;
      A.tiles_k = (A.K + 63) / 64;
      // Step the longer tile axis fastest (measured: [65536, 768] and
      // [8192, 4096] transposes 7-15% faster along K, [1000, 3000] 14%
      // faster along I).
      A.kfast = A.tiles_i >= A.tiles_k;
      int64_t batch = 1;
      for (int d = r - 2; d >= 0; --d) {
        if (d == k) continue;
        A.bdim[A.nb] = make_fastdiv(uint32_t(sh[d]));
        A.bsrc[A.nb] = st[d];
        A.bdst[A.nb] = dstr[d];
        ++A.nb;
        batch *= sh[d];
      }
      const int64_t blocks = batch * A.tiles_i * A.tiles_k;
      if (blocks < (int64_t(1) << 31)) {
        const dim3 g(static_cast<unsigned>(blocks));
        switch (es) {
          case 1: bg::dispatch(ctx, copy_transpose_kernel<uint8_t>, g, dim3(256), 0,
                               static_cast<const uint8_t*>(src), static_cast<uint8_t*>(dst), A); return;
          case 2: bg::dispatch(ctx, copy_transpose_kernel<uint16_t>, g, dim3(256), 0,
                               static_cast<const uint16_t*>(src), static_cast<uint16_t*>(dst), A); return;
          case 4: bg::dispatch(ctx, copy_transpose_kernel<uint32_t>, g, dim3(256), 0,
                               static_cast<const uint32_t*>(src), static_cast<uint32_t*>(dst), A); return;
          case 8: bg::dispatch(ctx, copy_transpose_kernel<uint64_t>, g, dim3(256), 0,
                               static_cast<const uint64_t*>(src), static_cast<uint64_t*>(dst), A); return;
          default: break;
        }
      }
    }
  }
  CopyArgs A{};
  A.rank = r;
  A.n = n;
  for (int i = 0; i < r; ++i) {
    A.shape[i] = sh[i];
    A.stride[i] = st[i];
  }
  const int g = grid1(A.n, 256);
  switch (es) {
    case 1: bg::dispatch(ctx, copy_strided_kernel<uint8_t>, dim3(g), dim3(256), 0,
                               static_cast<const uint8_t*>(src), static_cast<uint8_t*>(dst), A); break;
    case 2: bg::dispatch(ctx, copy_strided_kernel<uint16_t>, dim3(g), dim3(256), 0,
                               static_cast<const uint16_t*>(src), static_cast<uint16_t*>(dst), A); break;
    case 4: bg::dispatch(ctx, copy_strided_kernel<uint32_t>, dim3(g), dim3(256), 0,
                               static_cast<const uint32_t*>(src), static_cast<uint32_t*>(dst), A); break;
    case 8: bg::dispatch(ctx, copy_strided_kernel<uint64_t>, dim3(g), dim3(256), 0,
                               static_cast<const uint64_t*>(src), static_cast<uint64_t*>(dst), A); break;
    default: fail(BG_E_DTYPE, "copy_strided: unsupported element size");
  }
  hip_check(hipGetLastError(), "copy_strided launch");
}

void launch_gelu_rows(bg_ctx* ctx, const float* src, int64_t ld_src, int64_t stride_src, void* dst,
                      int64_t ld_dst, int64_t stride_dst, int dst_dtype, int64_t batch, int64_t rows,
                      int64_t cols, const float* residual) {
  const int64_t total = batch * rows;
  if (total == 0 || cols == 0) return;
  const unsigned grid = unsigned(std::min<int64_t>(total, 65536));
  bg::dispatch(ctx, gelu_rows_kernel, dim3(grid), dim3(256), 0, src, ld_src, stride_src, dst, ld_dst,
               stride_dst, dst_dtype, rows, cols, total, residual);
}

template <int NT, int NV>
static bool launch_softmax_row(bg_ctx* ctx, const void* x, int xd, void* y, int yd, int64_t rows, int64_t cols) {
  const dim3 grid(static_cast<unsigned>(rows));
#define BG_SMR(XD_, YD_) bg::dispatch(ctx, softmax_row_kernel<XD_, YD_, NT, NV>, grid, dim3(NT), 0, x, y, cols)
#define BG_SMR_Y(XD_)                         \
  switch (yd) {                               \
    case BG_F32: BG_SMR(XD_, BG_F32); break;  \
    case BG_F16: BG_SMR(XD_, BG_F16); break;  \
    case BG_BF16: BG_SMR(XD_, BG_BF16); break; \
    default: return false;                    \
  }
  switch (xd) {
    case BG_F32: BG_SMR_Y(BG_F32); break;
    case BG_F16: BG_SMR_Y(BG_F16); break;
    case BG_BF16: BG_SMR_Y(BG_BF16); break;
    default: return false;
  }
#undef BG_SMR_Y
#undef BG_SMR
  return true;
}

// x[B][R][C] reduced over R into out[B][C] of dtype od; see
// reduce_lead_kernel.
void launch_reduce_lead(bg_ctx* ctx, const void* x, int xd, int64_t B, int64_t R, int64_t C, int op, void* out,
                        int od) {
  if (B <= 0 || R <= 0 || C <= 0) fail(BG_E_SHAPE, "reduce: empty reduction");
  if (xd != BG_F32 && xd != BG_F16 && xd != BG_BF16) fail(BG_E_DTYPE, "reduce: dtype not supported");
  if (od != BG_F32 && od != BG_F16 && od != BG_BF16) fail(BG_E_DTYPE, "reduce: output dtype not supported");
  const int es = xd == BG_F32 ? 4 : 2;
  const bool v4 = C % 4 == 0 && reinterpret_cast<uintptr_t>(x) % uintptr_t(4 * es) == 0;
  const int V = v4 ? 4 : 1;
  const int64_t need = (C + V - 1) / V;  // column lanes the row needs
  const int LC = need <= 4 ? 4 : need <= 16 ? 16 : 64;
  const int64_t ngroups = (C + int64_t(LC) * V - 1) / (int64_t(LC) * V);
  const int64_t rstep = 4 * (64 / LC);  // rows one workgroup pass reads
  // Chunks of whole workgroup passes (at least 8) until about 1024
  // workgroups stream x.
  int64_t nchunk = std::max<int64_t>(1, std::min<int64_t>((1024 + B * ngroups - 1) / (B * ngroups),
                                                        (R + 8 * rstep - 1) / (8 * rstep)));
  int64_t CR = (R + nchunk - 1) / nchunk;
  CR = (CR + rstep - 1) / rstep * rstep;
  nchunk = (R + CR - 1) / CR;
  const int64_t units = B * ngroups * nchunk;
  if (units > int64_t(0x7fffffff)) fail(BG_E_UNSUPPORTED, "reduce: too many column groups");
  float* part = nchunk > 1 ? static_cast<float*>(scratch(ctx, size_t(nchunk * B * C) * 4, 0)) : nullptr;
  const int fin = nchunk == 1 ? 1 : 0;
  auto go = [&](auto xdc, auto vc, auto lcc) {
    bg::dispatch(ctx, reduce_lead_kernel<decltype(xdc)::value, decltype(vc)::value, decltype(lcc)::value>,
                 dim3(static_cast<unsigned>(units)), dim3(256), 0, x, R, C, CR, ngroups, nchunk, B, op, part, fin,
                 out, od);
  };
  auto by_lc = [&](auto xdc, auto vc) {
    if (LC == 4) go(xdc, vc, std::integral_constant<int, 4>{});
    else if (LC == 16) go(xdc, vc, std::integral_constant<int, 16>{});
    else go(xdc, vc, std::integral_constant<int, 64>{});
  };
  auto by_v = [&](auto xdc) {
    if (V == 4) by_lc(xdc, std::integral_constant<int, 4>{});
    else by_lc(xdc, std::integral_constant<int, 1>{});
  };
  if (xd == BG_F32) by_v(std::integral_constant<int, 0>{});
  else if (xd == BG_F16) by_v(std::integral_constant<int, 1>{});
  else by_v(std::integral_constant<int, 2>{});
  if (nchunk > 32)
    bg::dispatch(ctx, reduce_lead_final_kernel, dim3(static_cast<unsigned>((B * C + 15) / 16)), dim3(1024), 0,
                 static_cast<const float*>(part), nchunk, B * C, op, static_cast<float>(R), out, od);
  else if (nchunk > 1)
    bg::dispatch(ctx, reduce_lead_final_few_kernel, dim3(static_cast<unsigned>((B * C + 255) / 256)), dim3(256), 0,
                 static_cast<const float*>(part), nchunk, B * C, op, static_cast<float>(R), out, od);
}

void launch_reduce_partials(bg_ctx* ctx, const float* part, int64_t rows, int64_t nch, int op,
                            int64_t cols, void* out, int out_dtype) {
  if (rows <= 0) return;
  if (out_dtype != BG_F32 && out_dtype != BG_F16 && out_dtype != BG_BF16)
    fail(BG_E_DTYPE, "reduce: output dtype must be float32, float16 or bfloat16");
  bg::dispatch(ctx, reduce_partials_kernel, dim3(static_cast<unsigned>(rows)), dim3(256), 0, part, nch, op,
               static_cast<float>(cols), out, out_dtype);
}

void launch_softmax_last(bg_ctx* ctx, const void* x, int xd, void* y, int yd, int64_t rows, int64_t cols) {
  if (rows == 0) return;
  const dim3 grid(unsigned((rows + 3) / 4));
  const auto al = [](const void* p, size_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; };
  const int64_t xs = dtype_size(xd), ys = dtype_size(yd);
  // Rows narrower than 512 keep the wavefront-per-row kernels below (768
  // columns: 18.1 -> 13.5 us, 2048: 21.0 -> 11.4 us with a workgroup per row).
  if (cols >= 512 && cols % 4 == 0 && cols <= 1024 * 4 * 8 && rows <= 0x7fffffff && al(x, 4 * xs) &&
      al(y, 4 * ys)) {
    const int64_t nv = (cols / 4 + 255) / 256;
    bool ok;
    if (nv <= 1) ok = launch_softmax_row<256, 1>(ctx, x, xd, y, yd, rows, cols);
    else if (nv <= 2) ok = launch_softmax_row<256, 2>(ctx, x, xd, y, yd, rows, cols);
    else if (nv <= 4) ok = launch_softmax_row<256, 4>(ctx, x, xd, y, yd, rows, cols);
    else if (nv <= 8) ok = launch_softmax_row<256, 8>(ctx, x, xd, y, yd, rows, cols);
    else if (nv <= 16) ok = launch_softmax_row<1024, 4>(ctx, x, xd, y, yd, rows, cols);
    else ok = launch_softmax_row<1024, 8>(ctx, x, xd, y, yd, rows, cols);
    if (ok) return;
  }
  if (cols > 2048 && rows <= 0x7fffffff) {
    const dim3 rgrid(static_cast<unsigned>(rows));
    if (cols <= 1024 * 16)
      bg::dispatch(ctx, softmax_row_scalar_kernel<16>, rgrid, dim3(1024), 0, x, xd, y, yd, cols);
    else if (cols <= 1024 * 64)
      bg::dispatch(ctx, softmax_row_scalar_kernel<64>, rgrid, dim3(1024), 0, x, xd, y, yd, cols);
    else
      bg::dispatch(ctx, softmax_block_wide_kernel, rgrid, dim3(1024), 0, x, xd, y, yd, cols);
    return;
  }
  if (cols <= 256) {
    bg::dispatch(ctx, softmax_rows_kernel<4>, grid, dim3(256), 0, x, xd, y, yd, rows, cols);
  } else if (cols <= 1024) {
    bg::dispatch(ctx, softmax_rows_kernel<16>, grid, dim3(256), 0, x, xd, y, yd, rows, cols);
  } else if (cols <= 2048) {
    bg::dispatch(ctx, softmax_rows_kernel<32>, grid, dim3(256), 0, x, xd, y, yd, rows, cols);
  } else {
    bg::dispatch(ctx, softmax_rows_wide_kernel, grid, dim3(256), 0, x, xd, y, yd, rows, cols);
  }
}

template <int NV>
static bool launch_layer_norm_vec(bg_ctx* ctx, const void* x, int xd, const float* w, const float* b, void* y,
                                  int yd, int64_t rows, int64_t cols, float eps) {
  // Two rows per wavefront up to 1024 columns (4 waves, 8 rows a block).
  constexpr int RW = NV <= 4 ? 2 : 1;
  const dim3 grid(unsigned((rows + 4 * RW - 1) / (4 * RW)));
#define BG_LNV(XD_, YD_) \
  bg::dispatch(ctx, layer_norm_vec_kernel<XD_, YD_, NV, RW>, grid, dim3(256), 0, x, w, b, y, rows, cols, eps)
#define BG_LNV_Y(XD_)                         \
  switch (yd) {                               \
    case BG_F32: BG_LNV(XD_, BG_F32); break;  \
    case BG_F16: BG_LNV(XD_, BG_F16); break;  \
    case BG_BF16: BG_LNV(XD_, BG_BF16); break; \
    default: return false;                    \
  }
  switch (xd) {
    case BG_F32: BG_LNV_Y(BG_F32); break;
    case BG_F16: BG_LNV_Y(BG_F16); break;
    case BG_BF16: BG_LNV_Y(BG_BF16); break;
    default: return false;
  }
#undef BG_LNV_Y
#undef BG_LNV
  return true;
}

template <int NV>
static bool launch_layer_norm_row(bg_ctx* ctx, const void* x, int xd, const float* w, const float* b, void* y,
                                  int yd, int64_t rows, int64_t cols, float eps) {
  if (rows > 0x7fffffff) return false;
  const dim3 grid(static_cast<unsigned>(rows));
#define BG_LNR(XD_, YD_) bg::dispatch(ctx, layer_norm_row_kernel<XD_, YD_, NV>, grid, dim3(256), 0, x, w, b, y, cols, eps)
#define BG_LNR_Y(XD_)                         \
  switch (yd) {                               \
    case BG_F32: BG_LNR(XD_, BG_F32); break;  \
    case BG_F16: BG_LNR(XD_, BG_F16); break;  \
    case BG_BF16: BG_LNR(XD_, BG_BF16); break; \
    default: return false;                    \
  }
  switch (xd) {
    case BG_F32: BG_LNR_Y(BG_F32); break;
    case BG_F16: BG_LNR_Y(BG_F16); break;
    case BG_BF16: BG_LNR_Y(BG_BF16); break;
    default: return false;
  }
#undef BG_LNR_Y
#undef BG_LNR
  return true;
}

void launch_layer_norm(bg_ctx* ctx, const void* x, int xd, const float* w, const float* b,
                       void* y, int yd, int64_t rows, int64_t cols, float eps) {
  if (rows == 0) return;
  const dim3 grid(unsigned((rows + 3) / 4));
  // Vector path: 4-column groups aligned for the row's loads and stores.
  const auto al = [](const void* p, size_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; };
  const int64_t xs = dtype_size(xd), ys = dtype_size(yd);
  if (cols % 4 == 0 && cols <= 4 * 64 * 8 && al(x, 4 * xs) && al(y, 4 * ys) && al(w, 16) && al(b, 16)) {
    const int64_t nv = (cols / 4 + 63) / 64;
    bool ok = false;
    if (nv <= 1) ok = launch_layer_norm_vec<1>(ctx, x, xd, w, b, y, yd, rows, cols, eps);
    else if (nv <= 2) ok = launch_layer_norm_vec<2>(ctx, x, xd, w, b, y, yd, rows, cols, eps);
    else if (nv <= 3) ok = launch_layer_norm_vec<3>(ctx, x, xd, w, b, y, yd, rows, cols, eps);
    else if (nv <= 4) ok = launch_layer_norm_vec<4>(ctx, x, xd, w, b, y, yd, rows, cols, eps);
    else ok = launch_layer_norm_vec<8>(ctx, x, xd, w, b, y, yd, rows, cols, eps);
    if (ok) {
      hip_check(hipGetLastError(), "layer_norm launch");
      return;
    }
  }
  // Wider aligned rows: a workgroup per row (the wavefront-per-row kernel
  // below reads them three times).
  if (cols % 4 == 0 && cols > 4 * 64 * 8 && cols <= 256 * 4 * 32 && al(x, 4 * xs) && al(y, 4 * ys) &&
      al(w, 16) && al(b, 16)) {
    const int64_t nv = (cols / 4 + 255) / 256;
    bool ok = false;
    if (nv <= 4) ok = launch_layer_norm_row<4>(ctx, x, xd, w, b, y, yd, rows, cols, eps);
    else if (nv <= 8) ok = launch_layer_norm_row<8>(ctx, x, xd, w, b, y, yd, rows, cols, eps);
    else if (nv <= 16) ok = launch_layer_norm_row<16>(ctx, x, xd, w, b, y, yd, rows, cols, eps);
    else ok = launch_layer_norm_row<32>(ctx, x, xd, w, b, y, yd, rows, cols, eps);
    if (ok) {
      hip_check(hipGetLastError(), "layer_norm launch");
      return;
    }
  }
  if (cols <= 256) {
    bg::dispatch(ctx, layer_norm_kernel<4>, grid, dim3(256), 0, x, xd, w, b, y, yd,
                       rows, cols, eps);
  } else if (cols <= 1024) {
    bg::dispatch(ctx, layer_norm_kernel<16>, grid, dim3(256), 0, x, xd, w, b, y, yd,
                       rows, cols, eps);
  } else if (cols <= 2048) {
    bg::dispatch(ctx, layer_norm_kernel<32>, grid, dim3(256), 0, x, xd, w, b, y, yd,
                       rows, cols, eps);
  } else {
    bg::dispatch(ctx, layer_norm_wide_kernel, grid, dim3(256), 0, x, xd, w, b, y,
                       yd, rows, cols, eps);
  }
  hip_check(hipGetLastError(), "layer_norm launch");
}

void launch_attention_generic(bg_ctx* ctx, const bg_attention_desc& d, const void* q,
                              const void* k, const void* v, const float* mask, int64_t mask_sb,
                              int64_t mask_sh, void* o, bool two_pass) {
  if (d.d > kGenMaxD) fail(BG_E_UNSUPPORTED, "flash_attention: head dim > 256");
  AttnArgs A{};
  A.q = q; A.k = k; A.v = v; A.mask = mask; A.o = o;
  A.q_sb = d.q_sb; A.q_sh = d.q_sh; A.q_ss = d.q_ss;
  A.k_sb = d.k_sb; A.k_sh = d.k_sh; A.k_ss = d.k_ss;
  A.v_sb = d.v_sb; A.v_sh = d.v_sh; A.v_ss = d.v_ss;
  A.o_sb = d.o_sb; A.o_sh = d.o_sh; A.o_ss = d.o_ss;
  A.mask_sb = mask_sb; A.mask_sh = mask_sh;
  A.B = d.batch; A.H = d.heads; A.Sq = d.sq; A.Sk = d.sk; A.D = d.d;
  A.scale = d.scale;
  A.causal = d.causal;
  A.in_dtype = d.in_dtype;
  A.out_dtype = d.out_dtype;
  A.round_scores = d.round_scores;
  A.two_pass = two_pass ? 1 : 0;
  const int64_t rows = d.batch * d.heads * d.sq;
  bg::dispatch(ctx, attention_generic_kernel, dim3(unsigned((rows + 3) / 4)), dim3(256), 0, A);
  hip_check(hipGetLastError(), "attention launch");
}

void launch_attention_masked_f32(bg_ctx* ctx, const float* q, const float* k, const float* v,
                                 const float* mask, int64_t mask_b, int64_t mask_h, float* o,
                                 int64_t b, int64_t h, int64_t sq, int64_t sk, int64_t dd,
                                 float scale) {
  bg_attention_desc d{};
  d.batch = b; d.heads = h; d.sq = sq; d.sk = sk; d.d = dd;
  d.q_ss = dd; d.q_sh = sq * dd; d.q_sb = h * sq * dd;
  d.k_ss = dd; d.k_sh = sk * dd; d.k_sb = h * sk * dd;
  d.v_ss = dd; d.v_sh = sk * dd; d.v_sb = h * sk * dd;
  d.o_ss = dd; d.o_sh = sq * dd; d.o_sb = h * sq * dd;
  d.scale = scale;
  d.in_dtype = BG_F32;
  d.out_dtype = BG_F32;
  if (fa32_supported(d)) {
    launch_fa32(ctx, d, q, k, v, mask, mask_b, mask_h, sk, o);
    return;
  }
  launch_attention_generic(ctx, d, q, k, v, mask, mask_b, mask_h, o, false);
}

}  // namespace bg
