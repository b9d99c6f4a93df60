// GEMM for gfx950 on MFMA matrix cores, f32 accumulation.
//
// Replaces the reference's 16x16 scalar tiled WGSL GEMM
// (packages/browsergrad-kernels/src/kernels/matmul_tiled.ts:51-139) behind
// bridge.matmul (realizer.ts:1043-1060) and realizes the autocast MATMUL of
// the CPU oracle (_realize.py:395-412: f16 inputs, f32 accumulate, result
// rounded to f16) together with the bias ADD that follows it.
//
// 16-bit path (f16 / bf16 inputs), gemm16_kernel:
//   * NT layout: A [M][K] and B^T [N][K], both K-contiguous, so every MFMA
//     operand fragment is one 16-byte LDS read.  x @ W.T (nn.Linear) is NT
//     natively; x @ w (B = [K][N]) is re-laid out once by a transpose pass.
//   * v_mfma_f32_32x32x16_{f16,bf16}; block tile BM x BN x 64; four
//     wavefronts in a 2x2 grid, each owning (BM/2) x (BN/2) of C in
//     accumulator registers (256 x 256 tile: 4 x 4 MFMA tiles per wave).
//   * Global -> registers -> LDS, double buffered, one barrier per K step.
//     LDS rows are 128 B (64 halves); the 16-byte chunk index is XOR-swizzled
//     by the row so fragment reads and tile writes spread over all banks.
//   * Loads are branch-free: FULL tiles load unconditionally; edge tiles
//     clamp the address into the matrix and select zero outside it.
//   * Tile order is XCD-aware: workgroup i runs on XCD i % 8, so the tiles
//     one XCD receives are remapped to a compact patch of C that shares A
//     and B panels in that XCD's L2.
//   * Epilogue: the accumulators are staged through LDS (the operand buffers
//     are free by then) and written back as row vectors, applying
//     [round acc to f16/bf16] -> [+ bias[n] in f32] -> [relu / tanh-GELU]
//     -> store f32/f16/bf16 (the reference AMP graph CAST -> MATMUL(f16 out)
//     -> ADD(bias, f32) in one pass).  Staging keeps every accumulator index
//     static, so the accumulators never leave registers.
// f32 path, gemm32_kernel: v_mfma_f32_32x32x2_f32 with k-major LDS tiles
// (NN and NT), the same staged epilogue.
#include <algorithm>
#include <cstdio>

#include <cstdlib>
#include <string>
#include <type_traits>

#include "common.cuh"
#include "core.h"

namespace {

using namespace bgk;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf168 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));
// Native 16-byte vector (HIP's uint4 is a union-based struct, which keeps
// arrays of it from being promoted to registers).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

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
  int act;          // BG_ACT_*
  int out_dtype;    // BG_F32 / BG_F16 / BG_BF16
  int vec_store;    // C rows can take 4-element vector stores (ldc % 4, alignment)
  const float* R;   // residual f32 [batch][M][N] added last (NULL: none)
  int64_t ldr, sr;  // its row and batch strides (elements)
};

// XCD-aware tile index -> (tile_m, tile_n).  Workgroups are dispatched
// round-robin over the 8 XCDs; the tiles of one XCD are made consecutive and
// then walked in groups of G tile-rows so neighbours share A and B panels.
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

__device__ __forceinline__ float epilogue_value(const GemmArgs& P, float v, float bias) {
  if (P.round_dtype) v = round_through(v, P.round_dtype);
  if (P.bias) v = v + bias;
  if (P.act == BG_ACT_RELU) v = v > 0.f ? v : 0.f;
  else if (P.act == BG_ACT_GELU_TANH) v = gelu_tanh(v);
  return v;
}

template <int OUT>
__device__ __forceinline__ void store_elem(char* p, float v) {
  if constexpr (OUT == BG_F32) *reinterpret_cast<float*>(p) = v;
  else if constexpr (OUT == BG_F16) *reinterpret_cast<uint16_t*>(p) = f32_to_f16_bits(v);
  else *reinterpret_cast<uint16_t*>(p) = f32_to_bf16_bits(v);
}

// Epilogue in registers, stored straight to C, one 32x32 accumulator tile
// (16 values per lane) at a time: [round to the 16-bit type] -> [+ bias[n]]
// -> [relu] -> store, each stage behind one uniform branch per tile.
// Scheduling fences between tiles keep the live set to one tile, so the
// accumulators never spill.  tanh-GELU (one exponential and one reciprocal
// per element) runs here for wavefront tiles of up to kGeluEpilogueTiles
// accumulator tiles; wider ones leave it to a separate f32 pass over C
// (run_matmul).
// 32x32 MFMA accumulator layout: lane l, register e holds row
// 8*(e/4) + 4*(l/32) + e%4, column l%32, so each store instruction writes 32
// consecutive columns of two rows.  Addresses are a uniform per-row base plus
// one 32-bit per-lane offset; nothing in the loop waits on memory.
// Largest per-wavefront accumulator tile count (TM * TN) whose epilogue
// evaluates GELU in registers.
constexpr int kGeluEpilogueTiles = 8;

template <int TM, int TN, bool FULL, int OUT>
__device__ __forceinline__ void epilogue_tiles(const GemmArgs& P, char* C, float16v (&acc)[TM][TN],
                                               int64_t row0, int64_t col0, const float (&bz)[TN]) {
  constexpr int ES = OUT == BG_F32 ? 4 : 2;
  const int lane = threadIdx.x & 63;
  const int half = lane >> 5;
  const int64_t cl = col0 + (lane & 31);
  char* corner = C + (row0 * P.ldc + col0) * ES;
  const uint32_t lane_off = uint32_t((4 * half * P.ldc + (lane & 31)) * ES);
  const int64_t row_bytes = P.ldc * ES;
  // Residual (f32, added after the activation): 16 values per tile, same
  // element layout as the accumulator tile.
  float rnext[16];
  const float* rbase = P.R ? P.R + int64_t(blockIdx.z) * P.sr + (row0 + 4 * half) * P.ldr + cl : nullptr;
  auto load_residual = [&](int ti, int tj) {
    const bool ok_c = FULL || cl + tj * 32 < P.N;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int rr = ti * 32 + 8 * (e >> 2) + (e & 3);
      rnext[e] = (FULL || (ok_c && row0 + rr + 4 * half < P.M)) ? rbase[rr * P.ldr + tj * 32] : 0.f;
    }
  };
  if (P.R) load_residual(0, 0);
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      float v[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) v[e] = acc[i][j][e];
      if (P.round_dtype == 1) {
#pragma unroll
        for (int e = 0; e < 16; ++e) v[e] = round_through(v[e], 1);
      } else if (P.round_dtype == 2) {
#pragma unroll
        for (int e = 0; e < 16; ++e) v[e] = round_through(v[e], 2);
      }
      if (P.bias) {
#pragma unroll
        for (int e = 0; e < 16; ++e) v[e] = v[e] + bz[j];
      }
      if (P.act == BG_ACT_RELU) {
#pragma unroll
        for (int e = 0; e < 16; ++e) v[e] = v[e] > 0.f ? v[e] : 0.f;
      } else if constexpr (TM * TN <= kGeluEpilogueTiles) {
        // tanh-GELU on 16 values at a time (the tile fence below keeps the
        // compiler from interleaving tiles); wider wavefront tiles leave no
        // registers for it and take the separate f32 pass instead.
        if (P.act == BG_ACT_GELU_TANH) {
#pragma unroll
          for (int e = 0; e < 16; ++e) v[e] = gelu_tanh(v[e]);
        }
      }
      const bool col_ok = FULL || cl + j * 32 < P.N;
      if (P.R) {
        // The residual of this tile was loaded one tile ahead (before the
        // previous tile's stores), so its wait does not queue behind them.
        float cur[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) cur[e] = rnext[e];
        if (i * TN + j + 1 < TM * TN) load_residual((i * TN + j + 1) / TN, (i * TN + j + 1) % TN);
#pragma unroll
        for (int e = 0; e < 16; ++e) v[e] = v[e] + cur[e];
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int rr = i * 32 + 8 * (e >> 2) + (e & 3);
        if (FULL || (col_ok && row0 + rr + 4 * half < P.M))
          store_elem<OUT>(corner + rr * row_bytes + lane_off + j * 32 * ES, v[e]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
}

template <int TM, int TN, bool FULL>
__device__ __forceinline__ void direct_epilogue(const GemmArgs& P, char* C, float16v (&acc)[TM][TN],
                                                int64_t row0, int64_t col0) {
  const int lane = threadIdx.x & 63;
  const int64_t cl = col0 + (lane & 31);
  float bz[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j)
    bz[j] = (P.bias && (FULL || cl + j * 32 < P.N)) ? P.bias[cl + j * 32] : 0.f;
  if (P.out_dtype == BG_F32) epilogue_tiles<TM, TN, FULL, BG_F32>(P, C, acc, row0, col0, bz);
  else if (P.out_dtype == BG_F16) epilogue_tiles<TM, TN, FULL, BG_F16>(P, C, acc, row0, col0, bz);
  else epilogue_tiles<TM, TN, FULL, BG_BF16>(P, C, acc, row0, col0, bz);
}

// ---- 16-bit MFMA kernel ---------------------------------------------------------

constexpr int BK16 = 64;

// Physical 16-byte chunk of logical chunk c in LDS row r.
template <int SWZ>
__device__ __forceinline__ int swz(int r, int c) {
  if constexpr (SWZ == 0) return c ^ (r & 7);
  else return c ^ ((r >> 1) & 7);
}

// One thread's share of a R x 64 tile (R/32 chunks of 8 halves).  Rows are
// r = i*32 + tid/8, chunk tid%8.  VEC: 16-byte loads (K % 8 == 0 and aligned
// rows); otherwise element loads.  Out-of-matrix rows / columns read a
// clamped in-bounds address and are replaced by zero.
template <int R, bool FULL, bool VEC>
__device__ __forceinline__ void load_tile16(const uint16_t* __restrict__ base, int64_t ld, int64_t row0,
                                            int64_t rows, int64_t k0, int64_t K, u32x4 (&regs)[R / 32]) {
  const int tid = threadIdx.x;
  const int c = tid & 7;
#pragma unroll
  for (int i = 0; i < R / 32; ++i) {
    const int64_t gr = row0 + i * 32 + (tid >> 3);
    const int64_t gk = k0 + c * 8;
    if constexpr (FULL) {
      regs[i] = *reinterpret_cast<const u32x4*>(base + gr * ld + gk);
    } else if constexpr (VEC) {
      const bool ok = gr < rows && gk < K;
      const int64_t r = gr < rows ? gr : rows - 1;
      const int64_t k = gk < K ? gk : K - 8;
      const u32x4 v = *reinterpret_cast<const u32x4*>(base + r * ld + k);
      regs[i] = ok ? v : u32x4{0u, 0u, 0u, 0u};
    } else {
      const int64_t r = gr < rows ? gr : rows - 1;
      uint16_t e[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int64_t k = gk + j < K ? gk + j : K - 1;
        const uint16_t x = base[r * ld + k];
        e[j] = (gr < rows && gk + j < K) ? x : uint16_t(0);
      }
      regs[i] = u32x4{uint32_t(e[0]) | (uint32_t(e[1]) << 16), uint32_t(e[2]) | (uint32_t(e[3]) << 16),
                           uint32_t(e[4]) | (uint32_t(e[5]) << 16), uint32_t(e[6]) | (uint32_t(e[7]) << 16)};
    }
  }
}

template <int R, int SWZ>
__device__ __forceinline__ void store_tile16(u32x4* __restrict__ lds, const u32x4 (&regs)[R / 32]) {
  const int tid = threadIdx.x;
  const int c = tid & 7;
#pragma unroll
  for (int i = 0; i < R / 32; ++i) {
    const int r = i * 32 + (tid >> 3);
    lds[r * 8 + swz<SWZ>(r, c)] = regs[i];
  }
}

template <int BM, int BN, bool BF16, bool FULL, bool VEC, int SWZ>
__global__ void __launch_bounds__(256) gemm16_kernel(GemmArgs P) {
  constexpr int WTM = BM / 2, WTN = BN / 2;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  constexpr int STAGE_BUF = (BM + BN) * 8;  // u32x4 per pipeline stage
  __shared__ u32x4 smem[2 * STAGE_BUF];

  int tm_, tn_;
  tile_coords(blockIdx.x, P.tiles_m, P.tiles_n, tm_, tn_);
  const int64_t m0 = int64_t(tm_) * BM, n0 = int64_t(tn_) * BN;
  const int64_t batch = blockIdx.z;
  const uint16_t* A = static_cast<const uint16_t*>(P.A) + batch * P.sa;
  const uint16_t* B = static_cast<const uint16_t*>(P.B) + batch * P.sb;
  char* C = static_cast<char*>(P.C) + batch * P.sc * (P.out_dtype == BG_F32 ? 4 : 2);

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

  u32x4 ra[BM / 32], rb[BN / 32];
  const int nk = int((P.K + BK16 - 1) / BK16);
  load_tile16<BM, FULL, VEC>(A, P.lda, m0, P.M, 0, P.K, ra);
  load_tile16<BN, FULL, VEC>(B, P.ldb, n0, P.N, 0, P.K, rb);
  store_tile16<BM, SWZ>(smem, ra);
  store_tile16<BN, SWZ>(smem + BM * 8, rb);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const u32x4* as = smem + (kt & 1) * STAGE_BUF;
    const u32x4* bs = as + BM * 8;
    if (kt + 1 < nk) {
      load_tile16<BM, FULL, VEC>(A, P.lda, m0, P.M, int64_t(kt + 1) * BK16, P.K, ra);
      load_tile16<BN, FULL, VEC>(B, P.ldb, n0, P.N, int64_t(kt + 1) * BK16, P.K, rb);
    }
#pragma unroll
    for (int kk = 0; kk < BK16 / 16; ++kk) {
      const int c = kk * 2 + (lane >> 5);
      u32x4 af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = wm * WTM + i * 32 + (lane & 31);
        af[i] = as[r * 8 + swz<SWZ>(r, c)];
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int r = wn * WTN + j * 32 + (lane & 31);
        bf[j] = bs[r * 8 + swz<SWZ>(r, c)];
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
      u32x4* nxt = smem + ((kt + 1) & 1) * STAGE_BUF;
      store_tile16<BM, SWZ>(nxt, ra);
      store_tile16<BN, SWZ>(nxt + BM * 8, rb);
    }
    __syncthreads();
  }

  direct_epilogue<TM, TN, FULL>(P, C, acc, m0 + wm * WTM, n0 + wn * WTN);
}

// ---- 16-bit MFMA kernel, direct-to-LDS multi-stage pipeline -------------------------
//
// Same 2x2-wavefront tiling as gemm16_kernel, built for latency hiding:
//   * Operand tiles stream from HBM straight into LDS with
//     buffer_load_dwordx4 ... lds (no VGPR round trip, no ds_write).  Each
//     wavefront instruction fills 1 KB of LDS, lane L writing 16-byte unit
//     L, so the lane fetches whichever (row, k-chunk) the swizzled layout
//     puts in that unit.
//   * Lanes outside the matrix (rows >= M/N or k >= K) get an offset past
//     the buffer's num_records and the hardware returns zeros: edge tiles and
//     the pipeline's run-out stages need no branches.
//   * S stages of BK-deep tiles form a ring in LDS; loads run S-1 stages
//     ahead of the MFMAs.  Each step waits only for the loads of the next
//     stage (partial vmcnt), so S-2 stages stay in flight across the barrier.
//   * The loop is rotated: the last 16-wide k sub-step's MFMAs are issued
//     after the barrier, behind the next stage's first fragment reads and
//     loads, so neither LDS latency nor the barrier idles the matrix cores.
//     Operand fragments are double buffered in registers across sub-steps.
//   * LDS layout: the tile is viewed as 128-byte lines (RPL = 128 / (2*BK)
//     rows per line); a line's eight 16-byte units are XOR-permuted by the
//     line index so that the 16 lanes ds_read_b128 serves per cycle hit 16
//     distinct 4-bank groups (measured: zero SQ_LDS_BANK_CONFLICT for BK=64;
//     BK=32's earlier line & 7 permutation measured 2-way conflicts).

typedef __attribute__((address_space(3))) void* lds_ptr_t;

constexpr uint32_t kOob = 0x80000000u;  // >= num_records: load returns 0

template <int BK>
struct LdsLayout {
  static constexpr int CPR = BK / 8;    // 16-byte chunks per row
  static constexpr int RPL = 8 / CPR;   // rows per 128-byte line
  // ds_read_b128 serves 16 lanes per cycle across 64 banks (16 groups of
  // four): the 16 rows a group reads must land in 16 distinct groups, i.e.
  // unit % 16 must be a permutation.  128-byte rows: unit % 16 =
  // 8 (r & 1) + (c ^ ((r >> 1) & 7)).  64-byte rows (two per line): the two
  // rows of a line differ in bit 2 of the slot, so lines of one parity need
  // distinct low two bits: (line >> 1) & 3.
  __device__ static __forceinline__ int perm(int line) {
    return RPL == 1 ? ((line >> 1) & 7) : ((line >> 1) & 3);
  }
  // 16-byte unit holding (row r, chunk c).
  __device__ static __forceinline__ int unit(int r, int c) {
    const int line = r / RPL;
    return line * 8 + ((((r % RPL) * CPR) + c) ^ perm(line));
  }
};

// s_waitcnt that waits for vmcnt <= n only (expcnt / lgkmcnt left open).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Same, and also lgkmcnt == 0 (this wavefront's LDS reads have completed).
template <int N>
__device__ __forceinline__ void wait_vmcnt_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
}

// Per-lane operand offsets of one R x BK tile, fixed for the whole K loop:
// instruction i of wavefront w fills 1 KB block blk = i*4 + w; lane L writes
// unit blk*64 + L and fetches the (row, chunk) the layout keeps there.  Rows
// outside the matrix get kOob (the load returns zeros).  The k offset of a
// stage is added through the scalar soffset, so issuing a stage costs one
// instruction per 1 KB block.
template <int R, int BK, int NW = 4>
struct TileLoads {
  static constexpr int INSTR = R * BK * 2 / 1024;  // wavefront instructions per tile
  static_assert(INSTR % NW == 0, "tile must split evenly over the wavefronts");
  uint32_t voff[INSTR / NW];
  uint32_t chunk_k[INSTR / NW];  // k offset of the lane's chunk (elements), for K tails

  __device__ __forceinline__ void init(int w, int64_t ld, int64_t row0, int64_t rows) {
    using L = LdsLayout<BK>;
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < INSTR / NW; ++i) {
      const int u = (i * NW + w) * 64 + lane;
      const int line = u >> 3;
      const int sl = (u & 7) ^ L::perm(line);
      const int r = line * L::RPL + sl / L::CPR;
      const int c = sl % L::CPR;
      const int64_t gr = row0 + r;
      chunk_k[i] = uint32_t(c * 8);
      voff[i] = gr < rows ? uint32_t((gr * ld + c * 8) * 2) : kOob;
    }
  }

  // KTAIL: lanes whose chunk lies at or past K load zeros.
  template <bool KTAIL>
  __device__ __forceinline__ void issue(__amdgpu_buffer_rsrc_t rsrc, char* lds_tile, int w, int64_t k0,
                                        int64_t K) const {
#pragma unroll
    for (int i = 0; i < INSTR / NW; ++i) {
      uint32_t off = voff[i];
      if constexpr (KTAIL) off = (k0 + chunk_k[i] < K) ? off : kOob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_ptr_t)(lds_tile + (i * NW + w) * 1024), 16, off,
                                               uint32_t(k0 * 2), 0, 0);
    }
  }
};

// Scheduling pattern for one sub-step region: MFMA q is followed by one
// fragment read (q < NDS) and LPM operand loads (while loads remain).
template <int Q, int NMF, int NDS, int NVM, int LPM>
__device__ __forceinline__ void sched_pattern() {
  if constexpr (Q < NMF) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    if constexpr (Q < NDS) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    if constexpr (Q * LPM < NVM)
      __builtin_amdgcn_sched_group_barrier(0x020, (NVM - Q * LPM) < LPM ? (NVM - Q * LPM) : LPM, 0);
    sched_pattern<Q + 1, NMF, NDS, NVM, LPM>();
  }
}

// WGM x WGN wavefronts per workgroup, each owning a (BM / WGM) x (BN / WGN)
// block of C: 2 x 2 (one wavefront per SIMD) or 2 x 4 (two per SIMD, half
// the accumulators each, so one wavefront's fragment-read waits overlap the
// other's MFMAs).
template <int BM, int BN, int BK, int S, bool BF16, bool FULL, bool KTAIL, int WGM = 2, int WGN = 2>
__global__ void __launch_bounds__(64 * WGM * WGN) gemm16_lds_kernel(GemmArgs P, uint32_t a_bytes, uint32_t b_bytes) {
  using L = LdsLayout<BK>;
  constexpr int NW = WGM * WGN;
  constexpr int WTM = BM / WGM, WTN = BN / WGN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  constexpr int KK = BK / 16;                          // 16-wide sub-steps per stage
  constexpr int STAGE_BYTES = (BM + BN) * BK * 2;
  constexpr int NLD = (BM + BN) * BK * 2 / 1024 / NW;  // loads per wavefront per stage
  static_assert(KK % 2 == 0, "fragment double buffering needs an even sub-step count");
  static_assert(NLD * (S - 1) < 64, "vmcnt range");
  __shared__ u32x4 smem[S * STAGE_BYTES / 16];

  int tm_, tn_;
  tile_coords(blockIdx.x, P.tiles_m, P.tiles_n, tm_, tn_);
  const int64_t m0 = int64_t(tm_) * BM, n0 = int64_t(tn_) * BN;
  const int64_t batch = blockIdx.z;
  const uint16_t* A = static_cast<const uint16_t*>(P.A) + batch * P.sa;
  const uint16_t* B = static_cast<const uint16_t*>(P.B) + batch * P.sb;
  char* C = static_cast<char*>(P.C) + batch * P.sc * (P.out_dtype == BG_F32 ? 4 : 2);
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void*)A, (short)0, int(a_bytes), 0x00020000);
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc((void*)B, (short)0, int(b_bytes), 0x00020000);
  // Zero-length descriptors: every load of a run-out stage returns zeros.
  const __amdgpu_buffer_rsrc_t ra0 = __builtin_amdgcn_make_buffer_rsrc((void*)A, (short)0, 0, 0x00020000);
  const __amdgpu_buffer_rsrc_t rb0 = __builtin_amdgcn_make_buffer_rsrc((void*)B, (short)0, 0, 0x00020000);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WGN, wn = wave % WGN;
  TileLoads<BM, BK, NW> la;
  TileLoads<BN, BK, NW> lb;
  la.init(wave, P.lda, m0, P.M);
  lb.init(wave, P.ldb, n0, P.N);

  float16v acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  char* sbytes = reinterpret_cast<char*>(smem);
  const int nk = int((P.K + BK - 1) / BK);
  auto issue_stage = [&](int t) {
    char* st = sbytes + (t % S) * STAGE_BYTES;
    const bool real = t < nk;
    const int64_t k0 = real ? int64_t(t) * BK : 0;
    la.template issue<KTAIL>(real ? ra : ra0, st, wave, k0, P.K);
    lb.template issue<KTAIL>(real ? rb : rb0, st + BM * BK * 2, wave, k0, P.K);
  };
  // Fragment reads of sub-step kk of stage t: A rows / B^T rows, 8 halves.
  auto read_frags = [&](int t, int kk, u32x4 (&fa)[TM], u32x4 (&fb)[TN]) {
    const u32x4* as = smem + (t % S) * (STAGE_BYTES / 16);
    const u32x4* bs = as + BM * BK * 2 / 16;
    const int c = kk * 2 + (lane >> 5);
#pragma unroll
    for (int i = 0; i < TM; ++i) fa[i] = as[L::unit(wm * WTM + i * 32 + (lane & 31), c)];
#pragma unroll
    for (int j = 0; j < TN; ++j) fb[j] = bs[L::unit(wn * WTN + j * 32 + (lane & 31), c)];
  };
  auto mfmas = [&](const u32x4 (&fa)[TM], const u32x4 (&fb)[TN]) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        if constexpr (BF16)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf168, fa[i]),
                                                              __builtin_bit_cast(bf168, fb[j]), acc[i][j], 0, 0, 0);
        else
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, fa[i]),
                                                             __builtin_bit_cast(half8, fb[j]), acc[i][j], 0, 0, 0);
      }
  };
  // One fragment read after each of the first TM+TN MFMAs of a sub-step.
  auto interleave = [&]() {
#pragma unroll
    for (int q = 0; q < TM + TN; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, TM * TN - (TM + TN), 0);
  };

#pragma unroll
  for (int t = 0; t < S; ++t) issue_stage(t);
  wait_vmcnt<NLD * (S - 1)>();
  __syncthreads();

  u32x4 fa[2][TM], fb[2][TN];
  read_frags(0, 0, fa[0], fb[0]);
  __builtin_amdgcn_sched_barrier(0);
  for (int t = 0; t < nk; ++t) {
#pragma unroll
    for (int kk = 0; kk < KK - 1; ++kk) {
      read_frags(t, kk + 1, fa[(kk + 1) & 1], fb[(kk + 1) & 1]);
      mfmas(fa[kk & 1], fb[kk & 1]);
      interleave();
      __builtin_amdgcn_sched_barrier(0);
    }
    // End of stage t: its last fragments are in registers.  Wait for stage
    // t+1's loads, let every wavefront finish reading slot t % S, refill it
    // with stage t+S, then run the last sub-step behind the next reads.
    wait_vmcnt_lgkm0<NLD * (S - 2)>();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    issue_stage(t + S);
    read_frags(t + 1, 0, fa[0], fb[0]);
    mfmas(fa[(KK - 1) & 1], fb[(KK - 1) & 1]);
    // MFMA, fragment read and stage load interleaved.
    sched_pattern<0, TM * TN, TM + TN, NLD, (NLD + TM * TN - 1) / (TM * TN)>();
    __builtin_amdgcn_sched_barrier(0);
  }

  direct_epilogue<TM, TN, FULL>(P, C, acc, m0 + wm * WTM, n0 + wn * WTN);
}

// ---- f32 MFMA kernel ----------------------------------------------------------------

constexpr int BK32 = 16;

template <int BM, int BN, bool TRANS_B, bool ALIGNED>
__global__ void __launch_bounds__(256) gemm32_kernel(GemmArgs P) {
  constexpr int WTM = BM / 2, WTN = BN / 2;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  constexpr int LA = BM + 32, LB = BN + 32;  // k-major rows, padded
  constexpr int A_FLOATS = BK32 * LA, B_FLOATS = BK32 * LB;
  constexpr int STAGE_FLOATS = A_FLOATS + B_FLOATS;
  __shared__ float smem[2 * STAGE_FLOATS];

  int tm_, tn_;
  tile_coords(blockIdx.x, P.tiles_m, P.tiles_n, tm_, tn_);
  const int64_t m0 = int64_t(tm_) * BM, n0 = int64_t(tn_) * BN;
  const int64_t batch = blockIdx.z;
  const float* A = static_cast<const float*>(P.A) + batch * P.sa;
  const float* B = static_cast<const float*>(P.B) + batch * P.sb;
  char* C = static_cast<char*>(P.C) + batch * P.sc * (P.out_dtype == BG_F32 ? 4 : 2);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t kbeg = 0, kend = P.K;

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
#pragma unroll
    for (int i = 0; i < n; ++i) {
      const int v = i * 256 + tid;
      const int r = v >> 2, c = (v & 3) * 4;
      const int64_t gr = row0 + r, gk = k0 + c;
      const int64_t rr = gr < rows ? gr : rows - 1;
      if (ALIGNED) {
        const int64_t kc = gk < P.K ? gk : P.K - 4;
        const float4 x = *reinterpret_cast<const float4*>(base + rr * ld + kc);
        regs[i] = (gr < rows && gk < kend) ? x : make_float4(0.f, 0.f, 0.f, 0.f);
      } else {
        float e[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int64_t kc = gk + j < P.K ? gk + j : P.K - 1;
          const float x = base[rr * ld + kc];
          e[j] = (gr < rows && gk + j < kend) ? x : 0.f;
        }
        regs[i] = make_float4(e[0], e[1], e[2], e[3]);
      }
    }
  };
  // B in [K][N] layout: BK x BN tile loaded along N.
  auto load_kn = [&](int64_t k0, float4* regs) {
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int v = i * 256 + tid;
      const int kr = v / (BN / 4), c = (v % (BN / 4)) * 4;
      const int64_t gk = k0 + kr, gn = n0 + c;
      const int64_t kc = gk < P.K ? gk : P.K - 1;
      if (ALIGNED) {
        const int64_t nc = gn < P.N ? gn : P.N - 4;
        const float4 x = *reinterpret_cast<const float4*>(B + kc * P.ldb + nc);
        regs[i] = (gk < kend && gn < P.N) ? x : make_float4(0.f, 0.f, 0.f, 0.f);
      } else {
        float e[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int64_t nc = gn + j < P.N ? gn + j : P.N - 1;
          const float x = B[kc * P.ldb + nc];
          e[j] = (gk < kend && gn + j < P.N) ? x : 0.f;
        }
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
    float* As = smem + buf * STAGE_FLOATS;
    float* Bs = As + A_FLOATS;
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int v = i * 256 + tid;
      const int r = v >> 2, c = (v & 3) * 4;
      As[(c + 0) * LA + r] = ra[i].x;
      As[(c + 1) * LA + r] = ra[i].y;
      As[(c + 2) * LA + r] = ra[i].z;
      As[(c + 3) * LA + r] = ra[i].w;
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int v = i * 256 + tid;
      if constexpr (TRANS_B) {
        const int r = v >> 2, c = (v & 3) * 4;
        Bs[(c + 0) * LB + r] = rb[i].x;
        Bs[(c + 1) * LB + r] = rb[i].y;
        Bs[(c + 2) * LB + r] = rb[i].z;
        Bs[(c + 3) * LB + r] = rb[i].w;
      } else {
        const int kr = v / (BN / 4), c = (v % (BN / 4)) * 4;
        *reinterpret_cast<float4*>(&Bs[kr * LB + c]) = rb[i];
      }
    }
  };

  const int nk = int((kend - kbeg + BK32 - 1) / BK32);
  fetch(kbeg);
  commit(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const float* As = smem + (kt & 1) * STAGE_FLOATS;
    const float* Bs = As + A_FLOATS;
    if (kt + 1 < nk) fetch(kbeg + int64_t(kt + 1) * BK32);
#pragma unroll
    for (int s = 0; s < BK32 / 2; ++s) {
      const int k = 2 * s + (lane >> 5);
      float af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) af[i] = As[k * LA + wm * WTM + i * 32 + (lane & 31)];
#pragma unroll
      for (int j = 0; j < TN; ++j) bf[j] = Bs[k * LB + wn * WTN + j * 32 + (lane & 31)];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) commit((kt + 1) & 1);
    __syncthreads();
  }

  direct_epilogue<TM, TN, false>(P, C, acc, m0 + wm * WTM, n0 + wn * WTN);
}

// ---- f32 GEMM for small outputs with a long K (C1's 64 x 784 x 128) ---------------
//
// One workgroup per 32 x 32 block of C; its 16 wavefronts split K into
// 8-wide chunks (wavefront w takes a contiguous run of them), each
// accumulating a full 32 x 32 partial with v_mfma_f32_32x32x2_f32, then the
// 16 partials are summed through LDS in wavefront order (fixed, so results
// do not depend on timing) and the epilogue is applied and stored in the
// same launch.  MFMA t of chunk c takes k = 8c + 4 (lane / 32) + t on both
// operands, so a lane's A and B values for four MFMAs are one 16-byte load
// each (ALIGNED: rows 16-byte aligned, K % 4 == 0, B as [N][K]); otherwise
// per-element loads.  Operands come straight from global memory (L2): each
// element is read by one lane of one wavefront.
constexpr int kWideWaves = 16;

template <bool TRANS_B, bool ALIGNED>
__device__ __forceinline__ void wide_k_load(const GemmArgs& P, const float* A, const float* B, int64_t m,
                                            int64_t n, int64_t k0, float (&a)[4], float (&b)[4]) {
  if constexpr (ALIGNED && TRANS_B) {
    const bool kin = k0 < P.K;
    typedef float f4 __attribute__((ext_vector_type(4)));
    const f4 z = {0.f, 0.f, 0.f, 0.f};
    const f4 av = (kin && m < P.M) ? *reinterpret_cast<const f4*>(A + m * P.lda + k0) : z;
    const f4 bv = (kin && n < P.N) ? *reinterpret_cast<const f4*>(B + n * P.ldb + k0) : z;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      a[t] = av[t];
      b[t] = bv[t];
    }
  } else {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int64_t k = k0 + t;
      const bool kin = k < P.K;
      a[t] = (kin && m < P.M) ? A[m * P.lda + k] : 0.f;
      b[t] = (kin && n < P.N) ? (TRANS_B ? B[n * P.ldb + k] : B[k * P.ldb + n]) : 0.f;
    }
  }
}

template <int OUT, bool TRANS_B, bool ALIGNED>
__global__ void __launch_bounds__(kWideWaves * 64) gemm32_wide_k_kernel(GemmArgs P) {
  __shared__ float red[kWideWaves][1024];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int hi = lane >> 5, l32 = lane & 31;
  const int tiles_n = (int)((P.N + 31) / 32);
  const int64_t m0 = int64_t(blockIdx.x / tiles_n) * 32, n0 = int64_t(blockIdx.x % tiles_n) * 32;
  const float* A = static_cast<const float*>(P.A);
  const float* B = static_cast<const float*>(P.B);
  const int64_t nchunks = (P.K + 7) / 8;
  const int64_t per = (nchunks + kWideWaves - 1) / kWideWaves;
  const int64_t cb = w * per, ce = min(nchunks, cb + per);
  float16v acc;
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.f;
  const int64_t m = m0 + l32, n = n0 + l32;
  int64_t c = cb;
  for (; c + 2 <= ce; c += 2) {  // two chunks' loads in flight before their MFMAs
    float a0[4], b0[4], a1[4], b1[4];
    wide_k_load<TRANS_B, ALIGNED>(P, A, B, m, n, 8 * c + 4 * hi, a0, b0);
    wide_k_load<TRANS_B, ALIGNED>(P, A, B, m, n, 8 * (c + 1) + 4 * hi, a1, b1);
#pragma unroll
    for (int t = 0; t < 4; ++t) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[t], b0[t], acc, 0, 0, 0);
#pragma unroll
    for (int t = 0; t < 4; ++t) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[t], b1[t], acc, 0, 0, 0);
  }
  if (c < ce) {
    float a0[4], b0[4];
    wide_k_load<TRANS_B, ALIGNED>(P, A, B, m, n, 8 * c + 4 * hi, a0, b0);
#pragma unroll
    for (int t = 0; t < 4; ++t) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[t], b0[t], acc, 0, 0, 0);
  }
  // acc[e] = partial C[m0 + 8 (e / 4) + 4 hi + e % 4][n0 + lane % 32].
#pragma unroll
  for (int e = 0; e < 16; ++e) red[w][e * 64 + lane] = acc[e];
  __syncthreads();
  const int t = threadIdx.x, e = t >> 6, l = t & 63;
  float s = red[0][t];
#pragma unroll
  for (int ww = 1; ww < kWideWaves; ++ww) s += red[ww][t];
  const int64_t mm = m0 + 8 * (e >> 2) + 4 * (l >> 5) + (e & 3), nn = n0 + (l & 31);
  if (mm >= P.M || nn >= P.N) return;
  float v = epilogue_value(P, s, P.bias ? P.bias[nn] : 0.f);
  if (P.R) v = v + P.R[mm * P.ldr + nn];
  store_elem<OUT>(static_cast<char*>(P.C) + (mm * P.ldc + nn) * (OUT == BG_F32 ? 4 : 2), v);
}

template <int BM, int BN, bool BF16, int SWZ>
void launch16(bg_ctx* ctx, const GemmArgs& P, int64_t batch, bool full, bool vec) {
  dim3 grid(unsigned(P.tiles_m * P.tiles_n), 1, unsigned(batch));
  if (full)
    bg::dispatch(ctx, gemm16_kernel<BM, BN, BF16, true, true, SWZ>, grid, dim3(256), 0, P);
  else if (vec)
    bg::dispatch(ctx, gemm16_kernel<BM, BN, BF16, false, true, SWZ>, grid, dim3(256), 0, P);
  else
    bg::dispatch(ctx, gemm16_kernel<BM, BN, BF16, false, false, SWZ>, grid, dim3(256), 0, P);
}

template <int BM, int BN, int BK, int S, bool BF16, int WGM = 2, int WGN = 2>
void launch16_lds(bg_ctx* ctx, const GemmArgs& P, int64_t batch, uint32_t a_bytes, uint32_t b_bytes) {
  dim3 grid(unsigned(P.tiles_m * P.tiles_n), 1, unsigned(batch));
  const dim3 block(64 * WGM * WGN);
  const bool full = P.M % BM == 0 && P.N % BN == 0;
  const bool ktail = P.K % BK != 0;
  if (full && !ktail)
    bg::dispatch(ctx, gemm16_lds_kernel<BM, BN, BK, S, BF16, true, false, WGM, WGN>, grid, block, 0, P, a_bytes,
                 b_bytes);
  else if (!ktail)
    bg::dispatch(ctx, gemm16_lds_kernel<BM, BN, BK, S, BF16, false, false, WGM, WGN>, grid, block, 0, P, a_bytes,
                 b_bytes);
  else
    bg::dispatch(ctx, gemm16_lds_kernel<BM, BN, BK, S, BF16, false, true, WGM, WGN>, grid, block, 0, P, a_bytes,
                 b_bytes);
}

template <int BM, int BN>
void launch32(bg_ctx* ctx, const GemmArgs& P, int64_t batch, bool trans_b, bool aligned) {
  dim3 grid(unsigned(P.tiles_m * P.tiles_n), 1, unsigned(batch));
  if (trans_b) {
    if (aligned) bg::dispatch(ctx, gemm32_kernel<BM, BN, true, true>, grid, dim3(256), 0, P);
    else bg::dispatch(ctx, gemm32_kernel<BM, BN, true, false>, grid, dim3(256), 0, P);
  } else {
    if (aligned) bg::dispatch(ctx, gemm32_kernel<BM, BN, false, true>, grid, dim3(256), 0, P);
    else bg::dispatch(ctx, gemm32_kernel<BM, BN, false, false>, grid, dim3(256), 0, P);
  }
}

bool aligned_to(const void* p, size_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; }

// Tile shapes / pipeline depths of the direct-to-LDS kernel.  LDS per
// workgroup = S * (BM + BN) * BK * 2 bytes (<= 160 KB); loads run S-1 stages
// ahead, so short stages (small tiles or BK = 32) need more of them to cover
// HBM latency.
enum class LdsCfg { T256x256x64s2, T256x256x32s4, T256x128x64s3, T128x256x64s3, T128x128x64s4, T128x128x32s4,
                    T128x128x64s2, T256x256x64s2w8, T256x256x32s4w8, T256x128x64s3w8, T128x192x64s3w8,
                    T128x192x64s2w8 };

template <int BM_, int BN_, int BK_, int S_, int WGM_ = 2, int WGN_ = 2>
struct CfgTag {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, S = S_, WGM = WGM_, WGN = WGN_;
};

LdsCfg choose_lds_cfg(int64_t m, int64_t n, int64_t k, int64_t batch, int act) {
  // Diagnostic override for tuning sweeps: BG_GEMM_TILE=BMxBNxBKsS.
  if (const char* e = std::getenv("BG_GEMM_TILE")) {
    const std::string v(e);
    if (v == "256x256x64s2") return LdsCfg::T256x256x64s2;
    if (v == "256x256x32s4") return LdsCfg::T256x256x32s4;
    if (v == "256x128x64s3") return LdsCfg::T256x128x64s3;
    if (v == "128x256x64s3") return LdsCfg::T128x256x64s3;
    if (v == "128x128x64s4") return LdsCfg::T128x128x64s4;
    if (v == "128x128x32s4") return LdsCfg::T128x128x32s4;
    if (v == "128x128x64s2") return LdsCfg::T128x128x64s2;
    if (v == "256x256x64s2w8") return LdsCfg::T256x256x64s2w8;
    if (v == "256x256x32s4w8") return LdsCfg::T256x256x32s4w8;
    if (v == "256x128x64s3w8") return LdsCfg::T256x128x64s3w8;
    if (v == "128x192x64s3w8") return LdsCfg::T128x192x64s3w8;
    if (v == "128x192x64s2w8") return LdsCfg::T128x192x64s2w8;
  }
  // Measured on MI355X (kernel time, configurations interleaved round-robin
  // so that all share one thermal state; f16 out, + bias):
  //   4096^3:          256x256x64/2 stages, 8 wavefronts  116.1 us
  //                    (256x256x32/4 w8 120.8; 256x128x64/3 w8 131.2;
  //                    128x128x64/2 137.5; f32 out: 120.6 vs 124.7)
  //   8192x2304x768:   128x128x64/2                        42.4 us
  //                    (256x128 w8 44.2; 256x256 w8 45.9)
  //   8192x768x768:    256x128x64/3, 8 wavefronts         16.2 us (128x128: 17.4)
  //   8192x768x3072:   256x128x64/3, 8 wavefronts         43.7 us (128x128: 46.1)
  //   8192x3072x768 + GELU: 128x128x64/2                  57.3 us
  //                    (256x128 w8 58.7; 256x256 w8 61.2)
  // 128x192 tiles, 8 wavefronts as a 4 x 2 grid of 32x96 blocks (kernel
  // trace medians, round-robin launches, f16 out + bias; residual for N=768):
  //   8192x2304x768:         two stages (two per CU)  34.9 us (128x128: 42.8)
  //   8192x3072x768 + GELU:  two stages               51.7 us (128x128: 57.6)
  //   8192x768x3072 + res:   three stages (one per CU) 45.6 us (256x128 w8: 51.5)
  //   8192x768x768 + res:    three stages             19.1 us (256x128 w8: 20.6)
  // GPT-2's widths (768, 2304, 3072) are multiples of 192.
  // 1+ waves of 256x256 tiles with a deep K take them with two wavefronts
  // per SIMD; outputs whose width is a multiple of 192 take 128x192 (two
  // stages when there are two tiles per CU slot pair, else three); else
  // 1.25+ waves of 256x256 tiles (shallow K); narrow outputs (N <= 1024)
  // take 256x128; the rest 128x128, two workgroups per CU.  With tanh-GELU
  // in the epilogue 256x256 tiles lose: their 1.5 waves expose the epilogue.
  const int64_t t256 = ((m + 255) / 256) * ((n + 255) / 256) * batch;
  if (t256 >= 256 && k >= 2048 && act != BG_ACT_GELU_TANH) return LdsCfg::T256x256x64s2w8;
  const int64_t t192 = ((m + 127) / 128) * (n / 192) * batch;
  if (n % 192 == 0 && t192 >= 256) return t192 >= 512 ? LdsCfg::T128x192x64s2w8 : LdsCfg::T128x192x64s3w8;
  if (t256 >= 320 && act != BG_ACT_GELU_TANH) return LdsCfg::T256x256x64s2w8;
  const int64_t t256x128 = ((m + 255) / 256) * ((n + 127) / 128) * batch;
  if (n <= 1024 && t256x128 >= 128) return LdsCfg::T256x128x64s3w8;
  return LdsCfg::T128x128x64s2;
}

// ---- Skinny GEMMs (M <= 64): K split over workgroups ----------------------
// A 128-row tile would leave most of its rows and most CUs idle when M is
// small; the problem is a stream over B.  Workgroup u (16 wavefronts) takes
// 128 columns of C and the K range of split u % nsplit: wavefront w covers
// columns 32 (w % 4) .. +31 and every fourth step of the range, starting at
// step w / 4.  A step is 16 bytes of k per lane: lane l holds row (A) or
// column (B) l % 32 and the k-unit l / 32 of the step, so a 16-bit step is
// one v_mfma_f32_32x32x16 (k = 8 (l / 32) .. +7) and an f32 step (8 deep)
// four v_mfma_f32_32x32x2f32, MFMA t taking k = 4 (l / 32) + t on both
// operands.  Operands come straight from global memory (A is a few KB and
// stays in cache; B streams once): 16-byte loads, or for f32 B stored
// [K][N] (TB false) four 4-byte loads that are coalesced along N.  The
// four K-interleaved wavefronts of a column block are summed through LDS
// in order 0, 1, 2, 3.  With one split the epilogue runs here; otherwise f32
// partials go to part[split][M][N] and gemm_skinny_finish_kernel sums them
// in split order and runs the epilogue.
template <int DT, int MT, bool TB>
__global__ void __launch_bounds__(1024) gemm_skinny_kernel(GemmArgs P, int64_t ks, int nsplit, float* part) {
  constexpr int ES = DT == BG_F32 ? 4 : 2;
  constexpr int KSTEP = 32 / ES;  // k per step
  constexpr int KU = 16 / ES;     // k per lane per step
  __shared__ float red[3][4][MT][16][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nsub = wave & 3, ksub = wave >> 2;
  const int split = int(blockIdx.x % unsigned(nsplit));
  const int64_t n0 = int64_t(blockIdx.x / unsigned(nsplit)) * 128 + nsub * 32;
  const int64_t mb = int64_t(blockIdx.y) * 32 * MT;  // first row of this row block
  const int64_t n = n0 + (lane & 31);
  const bool n_ok = n < P.N;
  const int64_t kb0 = int64_t(split) * ks;
  const int64_t kb1 = kb0 + ks < P.K ? kb0 + ks : P.K;
  const int kl = KU * (lane >> 5);
  const char* A = static_cast<const char*>(P.A);
  const char* B = static_cast<const char*>(P.B);
  float16v acc[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[i][e] = 0.f;
  // Operand vectors: f32 as float 4-vectors (the wide-K kernel's form),
  // 16-bit as raw 16-byte words.
  typedef float f4 __attribute__((ext_vector_type(4)));
  using V = typename std::conditional<DT == BG_F32, f4, u32x4>::type;
  struct Frag {
    V b;
    V a[MT];
  };
  auto load_step = [&](int64_t kb, Frag& f) {
    const int64_t k = kb + kl;
    const bool k_ok = k < kb1;
    f.b = V{};
    if (n_ok && k_ok) {
      if constexpr (DT == BG_F32 && !TB) {
        const float* bp = reinterpret_cast<const float*>(B) + k * P.ldb + n;
        f.b = f4{bp[0], bp[P.ldb], bp[2 * P.ldb], bp[3 * P.ldb]};
      } else {
        f.b = *reinterpret_cast<const V*>(B + (n * P.ldb + k) * ES);
      }
    }
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const int64_t m = mb + i * 32 + (lane & 31);
      f.a[i] = (m < P.M && k_ok) ? *reinterpret_cast<const V*>(A + (m * P.lda + k) * ES) : V{};
    }
  };
  auto mma_step = [&](const Frag& f) {
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      if constexpr (DT == BG_F32) {
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[i] = __builtin_amdgcn_mfma_f32_32x32x2f32(f.a[i][t], f.b[t], acc[i], 0, 0, 0);
      } else if constexpr (DT == BG_BF16) {
        acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf168, f.a[i]),
                                                         __builtin_bit_cast(bf168, f.b), acc[i], 0, 0, 0);
      } else {
        acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, f.a[i]),
                                                        __builtin_bit_cast(half8, f.b), acc[i], 0, 0, 0);
      }
    }
  };
  // This wavefront's steps: kb0 + KSTEP (ksub + 4 j) < kb1.  f32 issues the
  // loads of D steps before their MFMAs (4 with one row block, 2 with two,
  // which stays within 128 VGPRs); 16-bit steps go one at a time (batching
  // them measured slower: 32 x 4096 x 4096 f16 11.4 -> 13.1 us).
  constexpr int D = DT == BG_F32 ? (MT == 1 ? 4 : 2) : 1;
  const int64_t first = kb0 + ksub * KSTEP;
  const int nst = first < kb1 ? int((kb1 - first + 4 * KSTEP - 1) / (4 * KSTEP)) : 0;
  int st = 0;
  for (; st + D <= nst; st += D) {
    Frag f[D];
#pragma unroll
    for (int q = 0; q < D; ++q) load_step(first + int64_t(st + q) * 4 * KSTEP, f[q]);
#pragma unroll
    for (int q = 0; q < D; ++q) mma_step(f[q]);
  }
  for (; st < nst; ++st) {
    Frag f;
    load_step(first + int64_t(st) * 4 * KSTEP, f);
    mma_step(f);
  }
  if (ksub > 0) {
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) red[ksub - 1][nsub][i][e][lane] = acc[i][e];
  }
  __syncthreads();
  if (ksub > 0 || !n_ok) return;
#pragma unroll
  for (int q = 0; q < 3; ++q)
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][e] += red[q][nsub][i][e][lane];
  const float bz = P.bias ? P.bias[n] : 0.f;
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int64_t m = mb + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
      if (m >= P.M) continue;
      if (nsplit > 1) {
        part[(int64_t(split) * P.M + m) * P.N + n] = acc[i][e];
      } else {
        float v = epilogue_value(P, acc[i][e], bz);
        if (P.R) v += P.R[m * P.ldr + n];
        store_from_f32(P.C, P.out_dtype, m * P.ldc + n, v);
      }
    }
}

__global__ void __launch_bounds__(256) gemm_skinny_finish_kernel(GemmArgs P, int nsplit, const float* part) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= P.M * P.N) return;
  const int64_t m = i / P.N, n = i - m * P.N;
  float v = part[i];
#pragma unroll 8
  for (int s = 1; s < nsplit; ++s) v += part[int64_t(s) * P.M * P.N + i];
  v = epilogue_value(P, v, P.bias ? P.bias[n] : 0.f);
  if (P.R) v += P.R[m * P.ldr + n];
  store_from_f32(P.C, P.out_dtype, m * P.ldc + n, v);
}

}  // namespace

namespace bg {

// Launch shape of the f32 GEMM, shared by run_gemm and the launch-plan
// query.  ptrs_aligned: A and B (offsets applied) start on 16 bytes.
// Few output tiles and a long K (C1's 64 x 784 x 128): one 128 x 128
// workgroup would walk K alone, one global-memory latency per 16-wide k
// step, so such GEMMs take the wide-K kernel instead (32 x 32 blocks, K
// split over the wavefronts of a workgroup and summed through LDS, one
// launch).
Gemm32Shape gemm32_shape(const bg_matmul_desc& d, bool ptrs_aligned) {
  Gemm32Shape g;
  g.tiles_m = int((d.m + 127) / 128);
  g.tiles_n = int((d.n + 127) / 128);
  g.aligned = ptrs_aligned && d.lda % 4 == 0 && d.ldb % 4 == 0 && d.k % 4 == 0 && (d.trans_b || d.n % 4 == 0) &&
              d.stride_a % 4 == 0 && d.stride_b % 4 == 0;
  const int64_t nk = (d.k + BK32 - 1) / BK32;
  const int64_t tiles = int64_t(g.tiles_m) * g.tiles_n;
  if (d.batch == 1 && tiles <= 16 && nk >= 8) {
    // One launch: 32 x 32 blocks of C, K split over 16 wavefronts inside
    // each workgroup (gemm32_wide_k_kernel).
    g.wide = true;
    g.tiles_m = int((d.m + 31) / 32);
    g.tiles_n = int((d.n + 31) / 32);
    g.aligned = g.aligned && d.trans_b;
  }
  return g;
}

// GEMM launch with C described by (c, ldc, stride_c, out_dtype, act).
// True when run_gemm would pick a kernel whose epilogue applies GELU (the
// direct-to-LDS kernel with 128-wide wavefront tiles).
static bool gelu_in_epilogue(const bg_matmul_desc& d, const char* a, const char* b) {
  if (d.in_dtype == BG_F32 || !d.trans_b) return false;
  const int64_t es = dtype_size(d.in_dtype);
  const void* A = a + d.offset_a * es;
  const void* B = b + d.offset_b * es;
  const bool vec = aligned_to(A, 16) && aligned_to(B, 16) && d.k % 8 == 0 && d.lda % 8 == 0 &&
                   d.ldb % 8 == 0 && d.stride_a % 8 == 0 && d.stride_b % 8 == 0;
  const int64_t a_span = ((d.m - 1) * d.lda + d.k) * es;
  const int64_t b_span = ((d.n - 1) * d.ldb + d.k) * es;
  if (!vec || a_span >= (int64_t(1) << 31) || b_span >= (int64_t(1) << 31)) return false;
  const LdsCfg c = choose_lds_cfg(d.m, d.n, d.k, d.batch, d.act);
  return c != LdsCfg::T256x256x64s2 && c != LdsCfg::T256x256x32s4;
}

// a / b point at the operands' storage (d.offset_a / d.offset_b are applied
// here); bias is f32 [N] or NULL.
// Skinny GEMMs: at most 512 rows for f32 (blocks of 64) or 64 for 16-bit,
// a K of 512+, fewer 128-column tiles than CUs and one batch (the tiled
// kernels would leave most of the chip idle).
// K slices of at least 256 (and multiples of 64: four wavefronts interleave
// the steps) until about 256 workgroups stream B; a workspace with less
// than `room` bytes free for the partials takes one slice.
struct SkinnyPlan {
  bool on = false;
  int64_t ntiles = 0, rblocks = 1, nsplit = 1, ks = 0;
};

static SkinnyPlan skinny_plan(const bg_matmul_desc& d, int dt, size_t room) {
  SkinnyPlan sp;
  sp.ntiles = (d.n + 127) / 128;
  // Row limit: 512 for f32 (64-row blocks; the tiled f32 kernel has at
  // most 128 workgroups there: 256 x 4096 x 4096 150 against 479 us), 64
  // for 16-bit (two blocks measured slower than the tiled kernel: 50
  // against 40 us at 128 x 4096 x 4096).
  if (d.batch != 1 || d.m > (dt == BG_F32 ? 512 : 64) || d.k < 512 || sp.ntiles >= 256 ||
      std::getenv("BG_GEMM_SKINNY") != nullptr)
    return sp;
  sp.on = true;
  sp.rblocks = (d.m + 63) / 64;
  int64_t nsplit = std::max<int64_t>(1, std::min<int64_t>(256 / (sp.ntiles * sp.rblocks), d.k / 256));
  int64_t ks = (d.k + nsplit - 1) / nsplit;
  ks = (ks + 63) / 64 * 64;
  nsplit = (d.k + ks - 1) / ks;
  if (nsplit > 1 && size_t(nsplit * d.m * d.n) * 4 + 256 > room) {
    nsplit = 1;
    ks = (d.k + 63) / 64 * 64;
  }
  sp.nsplit = nsplit;
  sp.ks = ks;
  return sp;
}

// Operands must allow 16-byte loads along K (the caller checks); tb: B is
// [N][K].  Returns false when the problem is not skinny.
static bool launch_skinny(bg_ctx* ctx, const bg_matmul_desc& d, GemmArgs& P, GemmWorkspace& ws, int dt, bool tb) {
  const SkinnyPlan sp = skinny_plan(d, dt, ws.fixed ? ws.cap - std::min(ws.cap, ws.used) : SIZE_MAX);
  if (!sp.on) return false;
  const int64_t nsplit = sp.nsplit, ks = sp.ks;
  float* part = nsplit > 1 ? static_cast<float*>(ws.get(size_t(nsplit * d.m * d.n) * 4, 3)) : nullptr;
  // Row blocks of 64 (32 when M <= 32) along grid y.
  const dim3 grid(static_cast<unsigned>(sp.ntiles * nsplit), static_cast<unsigned>(sp.rblocks));
  const int ns = int(nsplit);
  auto go = [&](auto dtc, auto mtc, auto tbc) {
    bg::dispatch(ctx, gemm_skinny_kernel<decltype(dtc)::value, decltype(mtc)::value, decltype(tbc)::value>, grid,
                 dim3(1024), 0, P, ks, ns, part);
  };
  auto by_tb = [&](auto dtc, auto mtc) {
    if (tb) go(dtc, mtc, std::true_type{});
    else if constexpr (decltype(dtc)::value == BG_F32) go(dtc, mtc, std::false_type{});
    else fail(BG_E_UNSUPPORTED, "skinny GEMM: 16-bit B must be [N][K]");
  };
  auto by_mt = [&](auto dtc) {
    if (d.m <= 32) by_tb(dtc, std::integral_constant<int, 1>{});
    else by_tb(dtc, std::integral_constant<int, 2>{});
  };
  if (dt == BG_F32) by_mt(std::integral_constant<int, BG_F32>{});
  else if (dt == BG_F16) by_mt(std::integral_constant<int, BG_F16>{});
  else by_mt(std::integral_constant<int, BG_BF16>{});
  if (nsplit > 1)
    bg::dispatch(ctx, gemm_skinny_finish_kernel, dim3(static_cast<unsigned>((d.m * d.n + 255) / 256)), dim3(256), 0,
                 P, ns, static_cast<const float*>(part));
  return true;
}

static void run_gemm(bg_ctx* ctx, const bg_matmul_desc& d, const char* a, const char* b, const float* bias,
                     void* c, int64_t ldc, int64_t stride_c, int out_dtype, int act, GemmWorkspace& ws,
                     const float* residual = nullptr) {
  const int64_t es = dtype_size(d.in_dtype);
  GemmArgs P{};
  P.R = residual;
  P.ldr = d.n;
  P.sr = d.m * d.n;
  P.A = a + d.offset_a * es;
  P.B = b + d.offset_b * es;
  P.bias = bias;
  P.C = c;
  P.M = d.m;
  P.N = d.n;
  P.K = d.k;
  P.lda = d.lda;
  P.ldb = d.ldb;
  P.ldc = ldc;
  P.sa = d.stride_a;
  P.sb = d.stride_b;
  P.sc = stride_c;
  P.round_dtype = d.round_f16 ? (d.in_dtype == BG_BF16 ? 2 : 1) : 0;
  P.act = act;
  P.out_dtype = out_dtype;
  P.vec_store = (ldc % 4 == 0 && stride_c % 4 == 0 && aligned_to(P.C, 16) &&
                 (!P.bias || aligned_to(P.bias, 16)))
                    ? 1
                    : 0;
  const int64_t flops = 2 * d.batch * d.m * d.n * d.k;
  const int64_t bytes = d.batch * (d.m * d.k + d.n * d.k) * es +
                        d.batch * d.m * d.n * dtype_size(out_dtype);

  if (d.in_dtype == BG_F32) {
    const Gemm32Shape g = gemm32_shape(d, aligned_to(P.A, 16) && aligned_to(P.B, 16));
    P.tiles_m = g.tiles_m;
    P.tiles_n = g.tiles_n;
    const bool aligned = g.aligned;
    Profile prof(ctx, "gemm_f32", bytes, flops);
    if (g.wide) {
      const dim3 grid(unsigned(g.tiles_m * g.tiles_n));
      const dim3 block(kWideWaves * 64);
      auto go = [&](auto kern) { bg::dispatch(ctx, kern, grid, block, 0, P); };
      const bool tb = d.trans_b != 0;
#define BG_WIDE(O_)                                                                              \
  (tb ? (aligned ? go(gemm32_wide_k_kernel<O_, true, true>) : go(gemm32_wide_k_kernel<O_, true, false>)) \
      : go(gemm32_wide_k_kernel<O_, false, false>))
      if (out_dtype == BG_F32) BG_WIDE(BG_F32);
      else if (out_dtype == BG_F16) BG_WIDE(BG_F16);
      else BG_WIDE(BG_BF16);
#undef BG_WIDE
      return;
    }
    if (aligned && d.k % 4 == 0 && P.lda % 4 == 0 && P.ldb % 4 == 0) {
      if (launch_skinny(ctx, d, P, ws, BG_F32, d.trans_b != 0)) return;
    }
    launch32<128, 128>(ctx, P, d.batch, d.trans_b != 0, aligned);
    return;
  }

  // 16-bit: bring B to [N][K] when it arrives as [K][N].
  if (!d.trans_b) {
    const int64_t nb = d.stride_b == 0 ? 1 : d.batch;
    const size_t need = size_t(nb * d.n * d.k * es);
    void* tb = ws.get(need, 0);
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
  const bool vec = aligned_to(P.A, 16) && aligned_to(P.B, 16) && d.k % 8 == 0 && P.lda % 8 == 0 &&
                   P.ldb % 8 == 0 && P.sa % 8 == 0 && P.sb % 8 == 0;
  const bool bf = d.in_dtype == BG_BF16;
  Profile prof(ctx, bf ? "gemm_bf16" : "gemm_f16", bytes, flops);
  if (vec && launch_skinny(ctx, d, P, ws, d.in_dtype, true)) return;
  // Direct-to-LDS path: operand byte ranges addressable with 32-bit offsets.
  const int64_t a_span = ((d.m - 1) * P.lda + d.k) * es;
  const int64_t b_span = ((d.n - 1) * P.ldb + d.k) * es;
  const bool lds_ok = vec && a_span < (int64_t(1) << 31) && b_span < (int64_t(1) << 31);
  if (lds_ok) {
    const uint32_t ab = uint32_t(a_span), bb = uint32_t(b_span);
    const LdsCfg cfg = choose_lds_cfg(d.m, d.n, d.k, d.batch, act);
    auto go = [&](auto tag) {
      using T = decltype(tag);
      P.tiles_m = int((d.m + T::BM - 1) / T::BM);
      P.tiles_n = int((d.n + T::BN - 1) / T::BN);
      if (bf) launch16_lds<T::BM, T::BN, T::BK, T::S, true, T::WGM, T::WGN>(ctx, P, d.batch, ab, bb);
      else launch16_lds<T::BM, T::BN, T::BK, T::S, false, T::WGM, T::WGN>(ctx, P, d.batch, ab, bb);
    };
    switch (cfg) {
      case LdsCfg::T256x256x64s2: go(CfgTag<256, 256, 64, 2>{}); break;
      case LdsCfg::T256x256x32s4: go(CfgTag<256, 256, 32, 4>{}); break;
      case LdsCfg::T256x128x64s3: go(CfgTag<256, 128, 64, 3>{}); break;
      case LdsCfg::T128x256x64s3: go(CfgTag<128, 256, 64, 3>{}); break;
      case LdsCfg::T128x128x64s4: go(CfgTag<128, 128, 64, 4>{}); break;
      case LdsCfg::T128x128x32s4: go(CfgTag<128, 128, 32, 4>{}); break;
      case LdsCfg::T256x256x64s2w8: go(CfgTag<256, 256, 64, 2, 2, 4>{}); break;
      case LdsCfg::T256x256x32s4w8: go(CfgTag<256, 256, 32, 4, 2, 4>{}); break;
      case LdsCfg::T256x128x64s3w8: go(CfgTag<256, 128, 64, 3, 4, 2>{}); break;
      case LdsCfg::T128x192x64s3w8: go(CfgTag<128, 192, 64, 3, 4, 2>{}); break;
      case LdsCfg::T128x192x64s2w8: go(CfgTag<128, 192, 64, 2, 4, 2>{}); break;
      default: go(CfgTag<128, 128, 64, 2>{}); break;
    }
    return;
  }
  // Large problems: 256x256 tiles (one tile per CU at 4096^2); otherwise 128x128.
  const int64_t t256 = ((d.m + 255) / 256) * ((d.n + 255) / 256) * d.batch;
  const bool big = t256 >= 192;
  const int BMN = big ? 256 : 128;
  P.tiles_m = int((d.m + BMN - 1) / BMN);
  P.tiles_n = int((d.n + BMN - 1) / BMN);
  const bool full = vec && d.m % BMN == 0 && d.n % BMN == 0 && d.k % BK16 == 0 && P.vec_store;
  if (big) {
    if (bf) launch16<256, 256, true, 0>(ctx, P, d.batch, full, vec);
    else launch16<256, 256, false, 0>(ctx, P, d.batch, full, vec);
  } else {
    if (bf) launch16<128, 128, true, 0>(ctx, P, d.batch, full, vec);
    else launch16<128, 128, false, 0>(ctx, P, d.batch, full, vec);
  }
}

void* GemmWorkspace::get(size_t bytes, int slot) {
  if (!fixed) return scratch(ctx, bytes, slot);
  const size_t off = (used + 255) & ~size_t(255);
  if (off > cap || bytes > cap - off) {
    fail(BG_E_UNSUPPORTED, "matmul_noalloc: this problem needs " + std::to_string(off + bytes) +
                               " bytes of scratch, above the fixed " + std::to_string(cap) +
                               "-byte no-allocation scratch");
  }
  used = off + bytes;
  return fixed + off;
}

// Every workspace request of a call comes before its first kernel launch, so
// a refused request leaves nothing queued.
void run_matmul(bg_ctx* ctx, const bg_matmul_desc& d0, const char* a, const char* b, const float* bias, void* c,
                GemmWorkspace& ws, const GemmExtra* ex) {
  if (d0.batch > 65535) fail(BG_E_UNSUPPORTED, "matmul: batch > 65535");
  bg_matmul_desc d = d0;
  const float* residual = ex ? ex->residual : nullptr;
  const int es = int(dtype_size(d.in_dtype));
  // Operands stored in another dtype are converted (round to nearest even)
  // into scratch first; a [K][N] B is converted and laid out as [N][K] in
  // the same pass.  The caller has checked that such operands are dense.
  const int a_dt = ex && ex->a_dtype >= 0 ? ex->a_dtype : d.in_dtype;
  const int b_dt = ex && ex->b_dtype >= 0 ? ex->b_dtype : d.in_dtype;
  void* ta = nullptr;
  void* tb = nullptr;
  const int64_t na = (d.stride_a == 0 ? 1 : d.batch) * d.m * d.k;
  const int64_t nbm = d.stride_b == 0 ? 1 : d.batch;
  if (a_dt != d.in_dtype) ta = ws.get(size_t(na * es), 2);
  if (b_dt != d.in_dtype) tb = ws.get(size_t(nbm * d.n * d.k * es), 0);
  if (ta) {
    Profile prof(ctx, "gemm_a_cast", na * (dtype_size(a_dt) + es), 0);
    launch_cast(ctx, a + d.offset_a * dtype_size(a_dt), a_dt, ta, d.in_dtype, na);
    a = static_cast<const char*>(ta);
    d.offset_a = 0;
  }
  if (tb) {
    const char* src = b + d.offset_b * dtype_size(b_dt);
    Profile prof(ctx, "gemm_b_cast", nbm * d.n * d.k * (dtype_size(b_dt) + es), 0);
    if (d.trans_b) {
      launch_cast(ctx, src, b_dt, tb, d.in_dtype, nbm * d.n * d.k);
    } else {
      launch_cast_transpose(ctx, src, b_dt, tb, d.in_dtype, d.k, d.n, nbm);
      d.trans_b = 1;
    }
    b = static_cast<const char*>(tb);
    d.offset_b = 0;
    d.ldb = d.k;
    d.stride_b = d.stride_b == 0 ? 0 : d.n * d.k;
  }
  if (d.act != BG_ACT_GELU_TANH || gelu_in_epilogue(d, a, b)) {
    run_gemm(ctx, d, a, b, bias, c, d.ldc, d.stride_c, d.out_dtype, d.act, ws, residual);
    return;
  }
  // GELU follows the (rounded, biased) product in f32, as the reference
  // graph evaluates it: the GEMM leaves f32 in C (or in scratch when C is
  // 16-bit), then one elementwise pass applies GELU (and the residual) and
  // stores C's dtype.
  float* f = reinterpret_cast<float*>(c);
  int64_t ldf = d.ldc, sf = d.stride_c;
  if (d.out_dtype != BG_F32) {
    f = static_cast<float*>(ws.get(size_t(d.batch * d.m * d.n * 4), 1));
    ldf = d.n;
    sf = d.m * d.n;
  }
  run_gemm(ctx, d, a, b, bias, f, ldf, sf, BG_F32, BG_ACT_NONE, ws);
  Profile prof(ctx, "gemm_gelu", d.batch * d.m * d.n * (4 + dtype_size(d.out_dtype)), 0);
  launch_gelu_rows(ctx, f, ldf, sf, c, d.ldc, d.stride_c, d.out_dtype, d.batch, d.m, d.n, residual);
}

void launch_matmul(bg_ctx* ctx, const bg_matmul_desc& d, const Record& a, const Record& b,
                   const Record* bias, Record& out, const GemmExtra* ex) {
  GemmWorkspace ws{ctx};
  run_matmul(ctx, d, a.ptr(), b.ptr(), bias ? reinterpret_cast<const float*>(bias->ptr()) : nullptr, out.ptr(),
             ws, ex);
}

// The launches bg_matmul_ex makes for an f32 GEMM whose operands start at
// their offsets inside this library's (256-byte aligned) allocations.
void plan_matmul(const bg_matmul_desc& d0, bg_launch_plan& out) {
  bg_matmul_desc d = d0;
  if (d.in_dtype != BG_F32) fail(BG_E_UNSUPPORTED, "matmul launch plan: float32 GEMMs only");
  if (d.act == BG_ACT_GELU_TANH) fail(BG_E_UNSUPPORTED, "matmul launch plan: GELU epilogues are not covered");
  if (d.m <= 0 || d.n <= 0 || d.k <= 0 || d.batch <= 0)
    fail(BG_E_INVALID, "matmul: batch, m, k, n must be positive integers");
  if (d.lda == 0) d.lda = d.k;
  if (d.ldb == 0) d.ldb = d.trans_b ? d.k : d.n;
  if (d.ldc == 0) d.ldc = d.n;
  if (d.batch > 65535) fail(BG_E_UNSUPPORTED, "matmul: batch > 65535");
  const bool ptrs = (d.offset_a * 4) % 16 == 0 && (d.offset_b * 4) % 16 == 0;
  const Gemm32Shape g = gemm32_shape(d, ptrs);
  out = bg_launch_plan{};
  out.k_slices = 1;
  out.n_launches = 1;
  bg_launch_plan_entry& e = out.launch[0];
  if (g.wide) {
    out.tile_m = 32;
    out.tile_n = 32;
    out.tile_k = 8;
    out.k_slices = kWideWaves;
    out.lds_bytes = kWideWaves * 1024 * 4;
    std::snprintf(e.family, sizeof e.family, "%s", "gemm32_wide_k_kernel");
    e.n_targs = 3;
    e.targs[0] = d.out_dtype;
    e.targs[1] = d.trans_b ? 1 : 0;
    e.targs[2] = g.aligned ? 1 : 0;
    e.grid[0] = int64_t(g.tiles_m) * g.tiles_n; e.grid[1] = 1; e.grid[2] = 1;
    e.block[0] = kWideWaves * 64; e.block[1] = 1; e.block[2] = 1;
    return;
  }
  const SkinnyPlan sp = g.aligned ? skinny_plan(d, BG_F32, SIZE_MAX) : SkinnyPlan{};
  if (sp.on) {
    const int mt = d.m <= 32 ? 1 : 2;
    out.tile_m = 32 * mt;
    out.tile_n = 128;
    out.tile_k = 8;
    out.k_slices = int32_t(sp.nsplit);
    out.lds_bytes = int64_t(3) * 4 * mt * 16 * 64 * 4;
    out.workspace_bytes = sp.nsplit > 1 ? sp.nsplit * d.m * d.n * 4 : 0;
    std::snprintf(e.family, sizeof e.family, "%s", "gemm_skinny_kernel");
    e.n_targs = 3;
    e.targs[0] = BG_F32;
    e.targs[1] = mt;
    e.targs[2] = d.trans_b ? 1 : 0;
    e.grid[0] = sp.ntiles * sp.nsplit; e.grid[1] = sp.rblocks; e.grid[2] = 1;
    e.block[0] = 1024; e.block[1] = 1; e.block[2] = 1;
    if (sp.nsplit > 1) {
      out.n_launches = 2;
      bg_launch_plan_entry& f = out.launch[1];
      std::snprintf(f.family, sizeof f.family, "%s", "gemm_skinny_finish_kernel");
      f.n_targs = 0;
      f.grid[0] = (d.m * d.n + 255) / 256; f.grid[1] = 1; f.grid[2] = 1;
      f.block[0] = 256; f.block[1] = 1; f.block[2] = 1;
    }
    return;
  }
  out.tile_m = 128;
  out.tile_n = 128;
  out.tile_k = BK32;
  out.lds_bytes = 2 * BK32 * (128 + 32 + 128 + 32) * 4;
  std::snprintf(e.family, sizeof e.family, "%s", "gemm32_kernel");
  e.n_targs = 4;
  e.targs[0] = 128;
  e.targs[1] = 128;
  e.targs[2] = d.trans_b ? 1 : 0;
  e.targs[3] = g.aligned ? 1 : 0;
  e.block[0] = 256; e.block[1] = 1; e.block[2] = 1;
  e.grid[0] = int64_t(g.tiles_m) * g.tiles_n; e.grid[1] = 1; e.grid[2] = d.batch;
}

}  // namespace bg
