// GEMM for gfx950 on MFMA matrix cores, f32 accumulation.
//
// Replaces the reference's 16x16 scalar tiled WGSL GEMM
// (packages/browsergrad-kernels/src/kernels/matmul_tiled.ts:51-139) behind
// bridge.matmul (realizer.ts:1043-1060) and the autocast MATMUL semantics of
// the CPU oracle (_realize.py:395-412: f16 inputs, f32 accumulate, result
// rounded to f16).
//
// 16-bit path (f16 / bf16 inputs):
//   * NT layout: A [M][K] and B^T [N][K], both K-contiguous, so every MFMA
//     operand is one 16-byte LDS read.  x @ W.T (nn.Linear) is NT natively;
//     x @ w (B = [K][N]) is re-laid out once by a cast/transpose pre-pass.
//   * v_mfma_f32_32x32x16_{f16,bf16}; block tile BM x BN x 64, four
//     wavefronts in a 2x2 grid, each owning (BM/2) x (BN/2) of C in
//     accumulator registers.
//   * Global -> registers -> LDS, double buffered, one barrier per K step;
//     LDS rows are 128 B (64 halfs) with the 16-byte chunk index XOR-swizzled
//     by (row >> 1) & 7 so fragment reads and tile writes are conflict-free.
//   * Tile order is XCD-aware: hardware dispatches workgroup i to XCD i % 8,
//     so consecutive tiles of one XCD are remapped to a compact GROUP_M x N
//     patch that shares A and B panels in that XCD's L2.
//   * Epilogue fused: [round acc to f16/bf16] -> [+ bias[n]] -> [relu /
//     tanh-GELU] -> store f32/f16/bf16 (the reference AMP graph
//     CAST -> MATMUL(f16 out) -> ADD(bias, f32) realized in one pass).
// f32 path: v_mfma_f32_32x32x2_f32 with k-major LDS tiles; NN and NT.
#include <algorithm>

#include "common.cuh"
#include "core.h"

namespace {

using namespace bgk;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf168 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));

struct GemmArgs {
  const void* A;
  const void* B;
  const float* bias;
  void* C;
  int64_t M, N, K;
  int64_t lda, ldb, ldc;
  int64_t sa, sb, sc;  // batch strides (elements)
  int tiles_m, tiles_n;
  int round_dtype;  // 0 none, 1 f16, 2 bf16
  int act;
  int out_dtype;
};

// XCD-aware tile index -> (tile_m, tile_n).
__device__ __forceinline__ void tile_coords(int pid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  if (total % 8 == 0) {
    const int per = total / 8;
    pid = (pid % 8) * per + pid / 8;
  }
  constexpr int G = 4;
  const int group = pid / (G * tiles_n);
  const int first_m = group * G;
  const int gsz = min(G, tiles_m - first_m);
  const int in_group = pid % (G * tiles_n);
  tm = first_m + in_group % gsz;
  tn = in_group / gsz;
}

__device__ __forceinline__ void epilogue_store(const GemmArgs& P, void* C, int64_t row,
                                               int64_t col, float v) {
  if (row >= P.M || col >= P.N) return;
  if (P.round_dtype) v = round_through(v, P.round_dtype);
  if (P.bias) v = v + P.bias[col];
  if (P.act == 1) v = v > 0.f ? v : 0.f;
  else if (P.act == 2) v = gelu_tanh_ref(v);
  store_from_f32(C, P.out_dtype, row * P.ldc + col, v);
}

// ---- 16-bit MFMA kernel ---------------------------------------------------------

constexpr int BK16 = 64;

template <int R, bool ALIGNED>
__device__ __forceinline__ void load_tile16(const uint16_t* __restrict__ base, int64_t ld,
                                            int64_t row0, int64_t rows, int64_t k0, int64_t K,
                                            uint4 (&regs)[R / 32]) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < R / 32; ++i) {
    const int v = i * 256 + tid;
    const int r = v >> 3, c = v & 7;
    const int64_t gr = row0 + r, gk = k0 + c * 8;
    if constexpr (ALIGNED) {
      if (gr < rows && gk < K) regs[i] = *reinterpret_cast<const uint4*>(base + gr * ld + gk);
      else regs[i] = make_uint4(0, 0, 0, 0);
    } else {
      uint16_t e[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) e[j] = (gr < rows && gk + j < K) ? base[gr * ld + gk + j] : 0;
      regs[i] = make_uint4(uint32_t(e[0]) | (uint32_t(e[1]) << 16), uint32_t(e[2]) | (uint32_t(e[3]) << 16),
                           uint32_t(e[4]) | (uint32_t(e[5]) << 16), uint32_t(e[6]) | (uint32_t(e[7]) << 16));
    }
  }
}

template <int R>
__device__ __forceinline__ void store_tile16(uint4* __restrict__ lds, const uint4 (&regs)[R / 32]) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < R / 32; ++i) {
    const int v = i * 256 + tid;
    const int r = v >> 3, c = v & 7;
    lds[r * 8 + (c ^ ((r >> 1) & 7))] = regs[i];
  }
}

template <int BM, int BN, bool BF16, bool ALIGNED>
__global__ void __launch_bounds__(256, 1) gemm16_nt_kernel(GemmArgs P) {
  constexpr int WTM = BM / 2, WTN = BN / 2;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  __shared__ uint4 As[2][BM * 8];
  __shared__ uint4 Bs[2][BN * 8];

  int tm_, tn_;
  tile_coords(blockIdx.x, P.tiles_m, P.tiles_n, tm_, tn_);
  const int64_t m0 = int64_t(tm_) * BM, n0 = int64_t(tn_) * BN;
  const int64_t batch = blockIdx.z;
  const uint16_t* A = static_cast<const uint16_t*>(P.A) + batch * P.sa;
  const uint16_t* B = static_cast<const uint16_t*>(P.B) + batch * P.sb;
  char* C = static_cast<char*>(P.C) + batch * P.sc * (P.out_dtype == 0 ? 4 : 2);

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  float16v acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  uint4 ra[BM / 32], rb[BN / 32];
  const int nk = int((P.K + BK16 - 1) / BK16);
  load_tile16<BM, ALIGNED>(A, P.lda, m0, P.M, 0, P.K, ra);
  load_tile16<BN, ALIGNED>(B, P.ldb, n0, P.N, 0, P.K, rb);
  store_tile16<BM>(As[0], ra);
  store_tile16<BN>(Bs[0], rb);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) {
      load_tile16<BM, ALIGNED>(A, P.lda, m0, P.M, int64_t(kt + 1) * BK16, P.K, ra);
      load_tile16<BN, ALIGNED>(B, P.ldb, n0, P.N, int64_t(kt + 1) * BK16, P.K, rb);
    }
    const uint4* as = As[cur];
    const uint4* bs = Bs[cur];
#pragma unroll
    for (int kk = 0; kk < BK16 / 16; ++kk) {
      const int c = kk * 2 + (lane >> 5);
      uint4 af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = wm * WTM + i * 32 + (lane & 31);
        af[i] = as[r * 8 + (c ^ ((r >> 1) & 7))];
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int r = wn * WTN + j * 32 + (lane & 31);
        bf[j] = bs[r * 8 + (c ^ ((r >> 1) & 7))];
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          if constexpr (BF16) {
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                __builtin_bit_cast(bf168, af[i]), __builtin_bit_cast(bf168, bf[j]), acc[i][j], 0, 0, 0);
          } else {
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                __builtin_bit_cast(half8, af[i]), __builtin_bit_cast(half8, bf[j]), acc[i][j], 0, 0, 0);
          }
        }
    }
    if (kt + 1 < nk) {
      store_tile16<BM>(As[cur ^ 1], ra);
      store_tile16<BN>(Bs[cur ^ 1], rb);
    }
    __syncthreads();
  }

  // C layout of a 32x32 MFMA tile: lane l, register e holds
  // row 8*(e/4) + 4*(l/32) + e%4, column l%32.
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t row = m0 + wm * WTM + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        const int64_t col = n0 + wn * WTN + j * 32 + (lane & 31);
        epilogue_store(P, C, row, col, acc[i][j][e]);
      }
}

// ---- f32 MFMA kernel ----------------------------------------------------------------

constexpr int BK32 = 16;

template <int BM, int BN, bool TRANS_B, bool ALIGNED>
__global__ void __launch_bounds__(256, 1) gemm32_kernel(GemmArgs P) {
  constexpr int WTM = BM / 2, WTN = BN / 2;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  constexpr int LA = BM + 32, LB = BN + 32;  // k-major rows, padded (row % 64 == 32 banks)
  __shared__ float As[2][BK32][LA];
  __shared__ float Bs[2][BK32][LB];

  int tm_, tn_;
  tile_coords(blockIdx.x, P.tiles_m, P.tiles_n, tm_, tn_);
  const int64_t m0 = int64_t(tm_) * BM, n0 = int64_t(tn_) * BN;
  const int64_t batch = blockIdx.z;
  const float* A = static_cast<const float*>(P.A) + batch * P.sa;
  const float* B = static_cast<const float*>(P.B) + batch * P.sb;
  char* C = static_cast<char*>(P.C) + batch * P.sc * (P.out_dtype == 0 ? 4 : 2);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  float16v acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // Row-major [rows][K] operand tile (A, or B^T when TRANS_B): R x 16 floats.
  constexpr int NA = BM * BK32 / 4 / 256;
  constexpr int NB = BN * BK32 / 4 / 256;
  float4 ra[NA], rb[NB];
  auto load_rowk = [&](const float* base, int64_t ld, int64_t row0, int64_t rows, int64_t k0,
                       float4* regs, int n) {
    for (int i = 0; i < n; ++i) {
      const int v = i * 256 + tid;
      const int r = v >> 2, c = (v & 3) * 4;
      const int64_t gr = row0 + r, gk = k0 + c;
      if (ALIGNED) {
        regs[i] = (gr < rows && gk < P.K) ? *reinterpret_cast<const float4*>(base + gr * ld + gk)
                                          : make_float4(0.f, 0.f, 0.f, 0.f);
      } else {
        float e[4];
        for (int j = 0; j < 4; ++j) e[j] = (gr < rows && gk + j < P.K) ? base[gr * ld + gk + j] : 0.f;
        regs[i] = make_float4(e[0], e[1], e[2], e[3]);
      }
    }
  };
  // B in [K][N] layout: BK x BN tile loaded along N.
  auto load_kn = [&](int64_t k0, float4* regs) {
    for (int i = 0; i < NB; ++i) {
      const int v = i * 256 + tid;
      const int kr = v / (BN / 4), c = (v % (BN / 4)) * 4;
      const int64_t gk = k0 + kr, gn = n0 + c;
      if (ALIGNED) {
        regs[i] = (gk < P.K && gn < P.N) ? *reinterpret_cast<const float4*>(B + gk * P.ldb + gn)
                                         : make_float4(0.f, 0.f, 0.f, 0.f);
      } else {
        float e[4];
        for (int j = 0; j < 4; ++j) e[j] = (gk < P.K && gn + j < P.N) ? B[gk * P.ldb + gn + j] : 0.f;
        regs[i] = make_float4(e[0], e[1], e[2], e[3]);
      }
    }
  };
  auto fetch = [&](int64_t k0) {
    load_rowk(A, P.lda, m0, P.M, k0, ra, NA);
    if constexpr (TRANS_B) load_rowk(B, P.ldb, n0, P.N, k0, rb, NB);
    else load_kn(k0, rb);
  };
  auto commit = [&](int buf) {
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int v = i * 256 + tid;
      const int r = v >> 2, c = (v & 3) * 4;
      As[buf][c + 0][r] = ra[i].x;
      As[buf][c + 1][r] = ra[i].y;
      As[buf][c + 2][r] = ra[i].z;
      As[buf][c + 3][r] = ra[i].w;
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int v = i * 256 + tid;
      if constexpr (TRANS_B) {
        const int r = v >> 2, c = (v & 3) * 4;
        Bs[buf][c + 0][r] = rb[i].x;
        Bs[buf][c + 1][r] = rb[i].y;
        Bs[buf][c + 2][r] = rb[i].z;
        Bs[buf][c + 3][r] = rb[i].w;
      } else {
        const int kr = v / (BN / 4), c = (v % (BN / 4)) * 4;
        *reinterpret_cast<float4*>(&Bs[buf][kr][c]) = rb[i];
      }
    }
  };

  const int nk = int((P.K + BK32 - 1) / BK32);
  fetch(0);
  commit(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) fetch(int64_t(kt + 1) * BK32);
#pragma unroll
    for (int s = 0; s < BK32 / 2; ++s) {
      const int k = 2 * s + (lane >> 5);
      float af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) af[i] = As[cur][k][wm * WTM + i * 32 + (lane & 31)];
#pragma unroll
      for (int j = 0; j < TN; ++j) bf[j] = Bs[cur][k][wn * WTN + j * 32 + (lane & 31)];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) commit(cur ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t row = m0 + wm * WTM + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        const int64_t col = n0 + wn * WTN + j * 32 + (lane & 31);
        epilogue_store(P, C, row, col, acc[i][j][e]);
      }
}

template <int BM, int BN, bool BF16>
void launch16(bg_ctx* ctx, const GemmArgs& P, int64_t batch, bool aligned) {
  dim3 grid(unsigned(P.tiles_m * P.tiles_n), 1, unsigned(batch));
  if (aligned)
    hipLaunchKernelGGL((gemm16_nt_kernel<BM, BN, BF16, true>), grid, dim3(256), 0, ctx->stream, P);
  else
    hipLaunchKernelGGL((gemm16_nt_kernel<BM, BN, BF16, false>), grid, dim3(256), 0, ctx->stream, P);
}

template <int BM, int BN>
void launch32(bg_ctx* ctx, const GemmArgs& P, int64_t batch, bool trans_b, bool aligned) {
  dim3 grid(unsigned(P.tiles_m * P.tiles_n), 1, unsigned(batch));
  if (trans_b) {
    if (aligned) hipLaunchKernelGGL((gemm32_kernel<BM, BN, true, true>), grid, dim3(256), 0, ctx->stream, P);
    else hipLaunchKernelGGL((gemm32_kernel<BM, BN, true, false>), grid, dim3(256), 0, ctx->stream, P);
  } else {
    if (aligned) hipLaunchKernelGGL((gemm32_kernel<BM, BN, false, true>), grid, dim3(256), 0, ctx->stream, P);
    else hipLaunchKernelGGL((gemm32_kernel<BM, BN, false, false>), grid, dim3(256), 0, ctx->stream, P);
  }
}

bool aligned_to(const void* p, size_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; }

}  // namespace

namespace bg {

void launch_matmul(bg_ctx* ctx, const bg_matmul_desc& d, const Record& a, const Record& b,
                   const Record* bias, Record& out) {
  if (d.batch > 65535) fail(BG_E_UNSUPPORTED, "matmul: batch > 65535");
  const int64_t es = dtype_size(d.in_dtype);
  GemmArgs P{};
  P.A = a.ptr() + d.offset_a * es;
  P.B = b.ptr() + d.offset_b * es;
  P.bias = bias ? reinterpret_cast<const float*>(bias->ptr()) : nullptr;
  P.C = out.ptr();
  P.M = d.m;
  P.N = d.n;
  P.K = d.k;
  P.lda = d.lda;
  P.ldb = d.ldb;
  P.ldc = d.ldc;
  P.sa = d.stride_a;
  P.sb = d.stride_b;
  P.sc = d.stride_c;
  P.round_dtype = d.round_f16 ? (d.in_dtype == BG_BF16 ? 2 : 1) : 0;
  P.act = d.act;
  P.out_dtype = d.out_dtype;
  const int64_t flops = 2 * d.batch * d.m * d.n * d.k;
  const int64_t bytes = d.batch * (d.m * d.k + d.n * d.k) * es +
                        d.batch * d.m * d.n * dtype_size(d.out_dtype);

  if (d.in_dtype == BG_F32) {
    const bool big = (d.m >= 2048 && d.n >= 2048);
    const int BM = 128, BN = 128;
    (void)big;
    P.tiles_m = int((d.m + BM - 1) / BM);
    P.tiles_n = int((d.n + BN - 1) / BN);
    const bool aligned = aligned_to(P.A, 16) && aligned_to(P.B, 16) && d.lda % 4 == 0 &&
                         d.ldb % 4 == 0 && d.k % 4 == 0 && (d.trans_b || d.n % 4 == 0) &&
                         d.stride_a % 4 == 0 && d.stride_b % 4 == 0;
    Profile prof(ctx, "gemm_f32", bytes, flops);
    launch32<128, 128>(ctx, P, d.batch, d.trans_b != 0, aligned);
    hip_check(hipGetLastError(), "gemm_f32 launch");
    return;
  }

  // 16-bit: bring B to [N][K] when it arrives as [K][N].
  if (!d.trans_b) {
    const int64_t nb = d.stride_b == 0 ? 1 : d.batch;
    const size_t need = size_t(nb * d.n * d.k * es);
    void* tb = scratch(ctx, need);
    {
      Profile prof(ctx, "gemm_b_transpose", 2 * nb * d.n * d.k * es, 0);
      if (d.ldb == d.n && (nb == 1 || d.stride_b == d.k * d.n)) {
        launch_cast_transpose(ctx, P.B, d.in_dtype, tb, d.in_dtype, d.k, d.n, nb);
      } else {
        // General strided B: gather into [nb][N][K] with a strided copy.
        std::vector<int64_t> shape = {nb, d.n, d.k};
        std::vector<int64_t> st = {d.stride_b, 1, d.ldb};
        launch_copy_strided(ctx, P.B, es, tb, shape, st);
      }
    }
    P.B = tb;
    P.ldb = d.k;
    P.sb = d.stride_b == 0 ? 0 : d.n * d.k;
  }
  const bool aligned = aligned_to(P.A, 16) && aligned_to(P.B, 16) && d.k % 8 == 0 &&
                       P.lda % 8 == 0 && P.ldb % 8 == 0 && P.sa % 8 == 0 && P.sb % 8 == 0;
  const bool bf = d.in_dtype == BG_BF16;
  // Large problems: 256x256 tiles (one tile per CU at 4096^2); otherwise 128x128.
  const int64_t t256 = ((d.m + 255) / 256) * ((d.n + 255) / 256) * d.batch;
  Profile prof(ctx, bf ? "gemm_bf16" : "gemm_f16", bytes, flops);
  if (t256 >= 192) {
    P.tiles_m = int((d.m + 255) / 256);
    P.tiles_n = int((d.n + 255) / 256);
    if (bf) launch16<256, 256, true>(ctx, P, d.batch, aligned);
    else launch16<256, 256, false>(ctx, P, d.batch, aligned);
  } else {
    P.tiles_m = int((d.m + 127) / 128);
    P.tiles_n = int((d.n + 127) / 128);
    if (bf) launch16<128, 128, true>(ctx, P, d.batch, aligned);
    else launch16<128, 128, false>(ctx, P, d.batch, aligned);
  }
  hip_check(hipGetLastError(), "gemm16 launch");
}

}  // namespace bg
