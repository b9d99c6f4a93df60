// Float32 attention forward on the matrix cores (gfx950), head dim <= 64.
//
// Replaces the reference's row-wise online-softmax WGSL kernel
// (packages/browsergrad-kernels/src/kernels/flash_attention.ts:45-211: one
// invocation per query row, every K/V row read from storage, f32 throughout,
// optional additive mask [1|B, 1|H, Sq, Sk], MAX_D = 64) behind
// bridge.flash_attention (realizer.ts:1122-1151), the typed
// ATTENTION_FORWARD and the semantic attention, and keeps its numerics:
// scores s = (q . k) * scale (+ mask), online softmax with the running
// maximum starting at the -1e20 sentinel, output O / l with the l > 0 guard.
//
// Design (one 256-thread workgroup = 4 wavefronts x 32 queries of one
// (batch, head); K and V stream through LDS in 64-key tiles):
//   * S^T = K Q^T with v_mfma_f32_32x32x2_f32.  MFMA j of the d loop takes
//     d = 8 (j / 4) + 4 (lane / 32) + j % 4 on both operands, so a lane's
//     K operand for four MFMAs is one 16-byte LDS read and its Q operand sits
//     in registers for the whole loop (Q pre-multiplied by scale * log2 e,
//     which puts the softmax in the exp2 domain).
//   * The accumulator layout gives a lane 16 keys of one query (rows
//     8 (e / 4) + 4 (lane / 32) + e % 4, column lane % 32).  Those registers
//     are, unchanged, the B operands of O^T += V^T P^T: MFMA j of the key loop
//     takes key 8 (j / 4) + 4 (lane / 32) + j % 4 on both operands, so P never
//     leaves the registers; the V^T operand is one 4-byte LDS read per lane.
//   * The row maximum is exact for every 32-key half (f32 has no overflow
//     concern that would allow a lazy one): 16 maxima and one exchange with
//     lane ^ 32; the rescale of O and l costs 33 multiplies against 64 MFMAs
//     of 64 cycles per half.
//   * K rows (256 bytes) store 16-byte chunk c at c ^ (row % 16): the 16
//     lanes a ds_read_b128 serves together read 16 different rows at one
//     chunk, which then covers all 64 banks.  V rows store chunk c at
//     c ^ 8 (row / 4 % 2): the two half-wavefronts of a V read take rows four
//     apart at the same 32 columns, which then land on disjoint banks.
//   * Tiles are staged through registers with one tile of prefetch: the
//     global loads of tile t + 1 are issued before tile t's MFMAs and
//     written to the other LDS buffer after them (one barrier per tile).
//     A tile is 128 MFMAs of 64 cycles per wavefront, which covers HBM
//     latency many times over.
//   * Causal (top-left aligned, key j visible to query i iff j <= i): tiles
//     after the workgroup's last query are not loaded, a wavefront skips
//     halves wholly after its 32 queries, and only halves that cross the
//     diagonal or the key length are masked.  Heavy query blocks go first.
// Bound: fp32 MFMA (157.3 TFLOP/s dense); 4 * B * H * D * (visible pairs)
// FLOP per launch.
#include <algorithm>
#include <cmath>
#include <cstdio>

#include "common.cuh"
#include "core.h"

namespace {

typedef float float16v __attribute__((ext_vector_type(16)));
typedef float float4v __attribute__((ext_vector_type(4)));

constexpr int kQW = 32;        // queries per wavefront
constexpr int kNW = 4;         // wavefronts per workgroup
constexpr int kBQ = kQW * kNW;  // queries per workgroup
constexpr int kBK = 64;        // keys per tile
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kMSentinel = -1.0e20f;  // flash_attention.ts:101 (m_i = -1.0e20)

struct Fa32Args {
  const float* q;
  const float* k;
  const float* v;
  const float* mask;  // NULL: no additive mask
  void* o;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  int64_t m_sb, m_sh, m_ss;  // mask strides (batch, head, query row); keys contiguous
  int H, Sq, Sk, D;
  int n_qblocks;
  float sl2;      // scale * log2(e)
  int causal;
  int out_dtype;  // 0 f32, 1 f16, 2 bf16
};

__device__ __forceinline__ float16v mfma32(float a, float b, float16v c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Value of lane ^ 32 (the other half-wavefront holds the same query).
__device__ __forceinline__ float xor32(float x) {
  const int v = __builtin_bit_cast(int, x);
  const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return __builtin_bit_cast(float, (threadIdx.x & 32) ? r[0] : r[1]);
}

__device__ __forceinline__ int k_slot(int row, int c) { return row * 64 + ((c ^ (row & 15)) << 2); }
__device__ __forceinline__ int v_slot(int row, int c) { return row * 64 + ((c ^ ((row & 4) << 1)) << 2); }

// Four floats of row `row` starting at column 4c of a [rows][D] operand
// (zeros past D or past the row count).  VEC: one 16-byte load (rows
// 16-byte aligned, D % 4 == 0).
template <bool VEC>
__device__ __forceinline__ float4v load4(const float* base, int64_t ss, int row, int nrows, int c, int D) {
  float4v r = {0.f, 0.f, 0.f, 0.f};
  if (row >= nrows || 4 * c >= D) return r;
  const float* p = base + int64_t(row) * ss + 4 * c;
  if constexpr (VEC) {
    return *reinterpret_cast<const float4v*>(p);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = 4 * c + i < D ? p[i] : 0.f;
    return r;
  }
}

// DP: head dim rounded up to 16, 32 or 64 (the MFMA d loop covers DP / 2
// values per half-wavefront; columns past D are zero in LDS and registers).
template <int DP, bool VEC>
__global__ void __launch_bounds__(kNW * 64, 2) fa32_fwd_kernel(Fa32Args P) {
  constexpr int NG = DP / 8;             // 16-byte K reads per lane per half (4 MFMAs each)
  constexpr int NDB = DP > 32 ? 2 : 1;   // 32-row blocks of O^T
  constexpr int CH = DP / 4;             // 16-byte chunks per row that hold data
  // Two buffers of a K tile and a V tile, 64 rows x 256 bytes each.
  __shared__ float4v smem[2 * 2 * kBK * 16];
  float* lds = reinterpret_cast<float*>(smem);

  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int hi = lane >> 5;
  const int l32 = lane & 31;
  const int bh = blockIdx.x;
  const int qblk = P.n_qblocks - 1 - int(blockIdx.y);  // heavy (late) blocks first
  const int b = bh / P.H, h = bh % P.H;
  const int q0 = qblk * kBQ;
  const int q0w = q0 + w * kQW;
  const int qi = q0w + l32;

  const float* Qp = P.q + b * P.q_sb + h * P.q_sh;
  const float* Kp = P.k + b * P.k_sb + h * P.k_sh;
  const float* Vp = P.v + b * P.v_sb + h * P.v_sh;
  const float* Mp = P.mask ? P.mask + b * P.m_sb + h * P.m_sh : nullptr;

  const int nt_all = (P.Sk + kBK - 1) / kBK;
  const int nt = P.causal ? min(nt_all, (q0 + kBQ + kBK - 1) / kBK) : nt_all;

  // Q operand: qf[g][i] = Q[qi][8 g + 4 hi + i] * scale * log2(e).
  float qf[NG][4];
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    const float4v x = load4<VEC>(Qp, P.q_ss, qi, P.Sq, 2 * g + hi, P.D);
#pragma unroll
    for (int i = 0; i < 4; ++i) qf[g][i] = x[i] * P.sl2;
  }

  // Tile staging: thread t moves 16-byte units t, t + 256, ... of the K and
  // V tiles (unit u = row u / 16, chunk u % 16; chunks past DP / 4 stay 0).
  constexpr int UNITS = kBK * 16 / (kNW * 64);  // 4
  float4v kst[UNITS], vst[UNITS];
  auto fetch = [&](int t) {
#pragma unroll
    for (int s = 0; s < UNITS; ++s) {
      const int u = threadIdx.x + s * kNW * 64;
      const int row = u >> 4, c = u & 15;
      const int key = t * kBK + row;
      kst[s] = c < CH ? load4<VEC>(Kp, P.k_ss, key, P.Sk, c, P.D) : float4v{0.f, 0.f, 0.f, 0.f};
      vst[s] = c < CH ? load4<VEC>(Vp, P.v_ss, key, P.Sk, c, P.D) : float4v{0.f, 0.f, 0.f, 0.f};
    }
  };
  auto stash = [&](int buf) {
    float* kt = lds + buf * (2 * kBK * 64);
    float* vt = kt + kBK * 64;
#pragma unroll
    for (int s = 0; s < UNITS; ++s) {
      const int u = threadIdx.x + s * kNW * 64;
      const int row = u >> 4, c = u & 15;
      *reinterpret_cast<float4v*>(kt + k_slot(row, c)) = kst[s];
      *reinterpret_cast<float4v*>(vt + v_slot(row, c)) = vst[s];
    }
  };

  float16v acc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[db][e] = 0.f;
  float m_run = kMSentinel, l_run = 0.f;
  const float mask_l2 = kLog2e;

  if (nt > 0) {
    fetch(0);
    stash(0);
  }
  __syncthreads();
  for (int t = 0; t < nt; ++t) {
    if (t + 1 < nt) fetch(t + 1);
    const float* kt = lds + (t & 1) * (2 * kBK * 64);
    const float* vt = kt + kBK * 64;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int j0 = t * kBK + hh * 32;
      // A half wholly after the wavefront's last query adds nothing (causal).
      if (P.causal && j0 > q0w + kQW - 1) continue;
      if (j0 >= P.Sk) continue;
      float16v s;
#pragma unroll
      for (int e = 0; e < 16; ++e) s[e] = 0.f;
      const int krow = hh * 32 + l32;
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        const float4v kf = *reinterpret_cast<const float4v*>(kt + k_slot(krow, 2 * g + hi));
#pragma unroll
        for (int i = 0; i < 4; ++i) s = mfma32(kf[i], qf[g][i], s);
      }
      // s[e]: key j0 + 8 (e / 4) + 4 hi + e % 4, query qi (log2 domain).
      const bool edge = (P.causal && j0 + 31 > q0w) || j0 + 32 > P.Sk;
      if (Mp) {
        const float* mrow = Mp + int64_t(min(qi, P.Sq - 1)) * P.m_ss;
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const int kj = j0 + 8 * a + 4 * hi + c;
            s[4 * a + c] = kj < P.Sk ? __builtin_fmaf(mrow[kj], mask_l2, s[4 * a + c]) : s[4 * a + c];
          }
      }
      if (edge) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int kj = j0 + 8 * (e >> 2) + 4 * hi + (e & 3);
          if (kj >= P.Sk || (P.causal && kj > qi)) s[e] = -INFINITY;
        }
      }
      float mt = s[0];
#pragma unroll
      for (int e = 1; e < 16; ++e) mt = fmaxf(mt, s[e]);
      mt = fmaxf(mt, xor32(mt));
      const float m_new = fmaxf(m_run, mt);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[db][e] *= alpha;
      float l0 = 0.f, l1 = 0.f;
#pragma unroll
      for (int e = 0; e < 16; e += 2) {
        s[e] = __builtin_amdgcn_exp2f(s[e] - m_new);
        s[e + 1] = __builtin_amdgcn_exp2f(s[e + 1] - m_new);
        l0 += s[e];
        l1 += s[e + 1];
      }
      l_run += l0 + l1;
      // O^T[32 db + lane % 32][q] += sum_j V[key(j)][32 db + lane % 32] P[q][key(j)].
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int vrow = hh * 32 + 8 * (j >> 2) + 4 * hi + (j & 3);
          const int col = 32 * db + l32;
          const float vf = vt[v_slot(vrow, col >> 2) + (col & 3)];
          acc[db] = mfma32(vf, s[j], acc[db]);
        }
    }
    if (t + 1 < nt) stash((t + 1) & 1);
    __syncthreads();
  }

  // O = acc / l (l > 0 guard, flash_attention.ts:125).  acc[db][e] holds
  // O^T[d = 32 db + 8 (e / 4) + 4 hi + e % 4][qi].
  const float lt = l_run + xor32(l_run);
  const float inv = lt > 0.f ? 1.0f / lt : 0.f;
  if (qi >= P.Sq) return;
  const int64_t obase = int64_t(b) * P.o_sb + int64_t(h) * P.o_sh + int64_t(qi) * P.o_ss;
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int d = 32 * db + 8 * (e >> 2) + 4 * hi + (e & 3);
      if (d < P.D) bgk::store_from_f32(P.o, P.out_dtype, obase + d, acc[db][e] * inv);
    }
}

}  // namespace

namespace bg {

// 16-byte loads of Q, K and V rows: D % 4 == 0, strides in whole 16-byte
// units, and the operands' first elements 16-byte aligned (ptrs_aligned).
static bool fa32_vec(const bg_attention_desc& d, bool ptrs_aligned) {
  return ptrs_aligned && d.d % 4 == 0 && d.q_ss % 4 == 0 && d.k_ss % 4 == 0 && d.v_ss % 4 == 0 &&
         d.q_sb % 4 == 0 && d.q_sh % 4 == 0 && d.k_sb % 4 == 0 && d.k_sh % 4 == 0 && d.v_sb % 4 == 0 &&
         d.v_sh % 4 == 0;
}

// True when the f32 MFMA kernel takes this attention (head dim <= 64).
bool fa32_supported(const bg_attention_desc& d) {
  return d.in_dtype == BG_F32 && d.d >= 1 && d.d <= 64 && d.batch * d.heads <= 0x7fffffff &&
         d.sq <= int64_t(65535) * kBQ && d.sk <= (int64_t(1) << 30) && d.sq <= (int64_t(1) << 30);
}

// q, k, v, o point at the first element of each operand (offsets applied);
// mask (f32, keys contiguous) is NULL or addressed by m_sb / m_sh / m_ss.
void launch_fa32(bg_ctx* ctx, const bg_attention_desc& d, const float* q, const float* k, const float* v,
                 const float* mask, int64_t m_sb, int64_t m_sh, int64_t m_ss, void* o) {
  if (!fa32_supported(d)) fail(BG_E_UNSUPPORTED, "flash_attention: f32 MFMA kernel takes head dim 1..64");
  Fa32Args A{};
  A.q = q;
  A.k = k;
  A.v = v;
  A.mask = mask;
  A.o = o;
  A.q_sb = d.q_sb; A.q_sh = d.q_sh; A.q_ss = d.q_ss;
  A.k_sb = d.k_sb; A.k_sh = d.k_sh; A.k_ss = d.k_ss;
  A.v_sb = d.v_sb; A.v_sh = d.v_sh; A.v_ss = d.v_ss;
  A.o_sb = d.o_sb; A.o_sh = d.o_sh; A.o_ss = d.o_ss;
  A.m_sb = m_sb; A.m_sh = m_sh; A.m_ss = m_ss;
  A.H = int(d.heads);
  A.Sq = int(d.sq);
  A.Sk = int(d.sk);
  A.D = int(d.d);
  A.n_qblocks = int((d.sq + kBQ - 1) / kBQ);
  A.sl2 = d.scale * kLog2e;
  A.causal = d.causal ? 1 : 0;
  A.out_dtype = d.out_dtype;
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  const bool vec = fa32_vec(d, al16(q) && al16(k) && al16(v));
  const dim3 grid(unsigned(d.batch * d.heads), unsigned(A.n_qblocks), 1);
  auto go = [&](auto kern) { dispatch(ctx, kern, grid, dim3(kNW * 64), 0, A); };
  if (d.d <= 16) vec ? go(fa32_fwd_kernel<16, true>) : go(fa32_fwd_kernel<16, false>);
  else if (d.d <= 32) vec ? go(fa32_fwd_kernel<32, true>) : go(fa32_fwd_kernel<32, false>);
  else vec ? go(fa32_fwd_kernel<64, true>) : go(fa32_fwd_kernel<64, false>);
  hip_check(hipGetLastError(), "f32 attention launch");
}

// The launch bg_attention_ex makes for an f32 attention whose operands
// start at their offsets inside this library's (256-byte aligned)
// allocations; zero strides mean contiguous [B, H, S, D] as there.
void plan_attention(const bg_attention_desc& d0, bg_launch_plan& out) {
  bg_attention_desc d = d0;
  if (d.batch <= 0 || d.heads <= 0 || d.sq <= 0 || d.sk <= 0 || d.d <= 0)
    fail(BG_E_INVALID, "flash_attention: b, h, sq, sk, d must be positive integers");
  auto fix = [&](int64_t& sb, int64_t& sh, int64_t& ss, int64_t s) {
    if (sb == 0 && sh == 0 && ss == 0) {
      ss = d.d;
      sh = s * d.d;
      sb = d.heads * s * d.d;
    }
  };
  fix(d.q_sb, d.q_sh, d.q_ss, d.sq);
  fix(d.k_sb, d.k_sh, d.k_ss, d.sk);
  fix(d.v_sb, d.v_sh, d.v_ss, d.sk);
  if (!fa32_supported(d))
    fail(BG_E_UNSUPPORTED, "attention launch plan: float32 attention with head dim 1..64 only");
  const bool ptrs = (d.q_off % 4) == 0 && (d.k_off % 4) == 0 && (d.v_off % 4) == 0;
  const int dp = d.d <= 16 ? 16 : d.d <= 32 ? 32 : 64;
  out = bg_launch_plan{};
  out.tile_m = kBQ;
  out.tile_n = kBK;
  out.tile_k = dp;
  out.k_slices = 1;
  out.lds_bytes = 2 * 2 * kBK * 16 * 16;
  out.n_launches = 1;
  bg_launch_plan_entry& e = out.launch[0];
  std::snprintf(e.family, sizeof e.family, "%s", "fa32_fwd_kernel");
  e.n_targs = 2;
  e.targs[0] = dp;
  e.targs[1] = fa32_vec(d, ptrs) ? 1 : 0;
  e.grid[0] = d.batch * d.heads;
  e.grid[1] = (d.sq + kBQ - 1) / kBQ;
  e.grid[2] = 1;
  e.block[0] = kNW * 64; e.block[1] = 1; e.block[2] = 1;
}

}  // namespace bg
