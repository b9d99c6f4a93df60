// Causal / non-causal attention forward on MFMA for gfx950 (head dim 64).
//
// Replaces the reference's row-wise online-softmax WGSL kernel
// (packages/browsergrad-kernels/src/kernels/flash_attention.ts:45-211, one
// thread per query row, no LDS) behind bridge.flash_attention
// (realizer.ts:1122-1151), and realizes the AMP SDPA graph of
// _functional.py:1505-1533 (scores = f16(q@k^T) * scale, causal
// masked_fill(-inf), f32 softmax, P rounded to f16, f16(P@v)) in one pass.
//
// Design (one 256-thread workgroup = 4 wavefronts = 128 queries of one
// (batch, head); K/V streamed in 64-key tiles):
//   * S^T = K Q^T with v_mfma_f32_32x32x16_{f16,bf16}: the accumulator
//     layout puts ONE query per lane column, so the running max / sum of the
//     online softmax are per-lane scalars and a row reduction is 16 local
//     ops plus one cross-half exchange (lane ^ 32).
//   * The S^T accumulators are converted to 16-bit in place and used as the
//     B operand of O^T = V^T P^T: the key order inside each 16-wide MFMA K
//     step is permuted identically on both operands, so P never leaves the
//     registers.
//   * K tiles are staged in LDS as [key][d] (128-byte rows, XOR-swizzled
//     16-byte chunks); V tiles as V^T [d][key] built from 4x4 register
//     transposes, 8-byte chunks XOR-swizzled by (d >> 1) & 15 so the
//     V^T fragment reads are bank-conflict free.  Both are double-buffered
//     with register prefetch (one barrier per tile).
//   * Causal: key tiles beyond the last query of the block are skipped,
//     a wavefront skips tiles entirely above its diagonal, and only the
//     diagonal tiles evaluate the mask.  Work-heavy query blocks (late in
//     the sequence) are dispatched first.
//   * exp via v_exp_f32 in the log2 domain (scale * log2(e) folded into one
//     multiply).
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "common.cuh"
#include "core.h"

namespace {

using namespace bgk;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf168 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));

struct FaArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  void* o;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  int H, Sq, Sk;
  int n_qblocks;
  float sl2;  // scale * log2(e)
  int out_dtype;
};

constexpr int kBQ = 128;
constexpr int kBK = 64;

template <bool BF16>
__device__ __forceinline__ float16v mfma16(uint4 a, uint4 b, float16v c) {
  if constexpr (BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf168, a),
                                                   __builtin_bit_cast(bf168, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, a),
                                                  __builtin_bit_cast(half8, b), c, 0, 0, 0);
}

template <bool BF16>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  if constexpr (BF16) {
    return uint32_t(f32_to_bf16_bits(a)) | (uint32_t(f32_to_bf16_bits(b)) << 16);
  } else {
    return uint32_t(f32_to_f16_bits(a)) | (uint32_t(f32_to_f16_bits(b)) << 16);
  }
}

template <bool BF16>
__device__ __forceinline__ float round16(float x) {
  if constexpr (BF16) return bf16_bits_to_f32(f32_to_bf16_bits(x));
  else return __half2float(__float2half_rn(x));
}

template <bool BF16, bool CAUSAL, bool ROUND_S>
__global__ void __launch_bounds__(256) fa_fwd_d64_kernel(FaArgs P) {
  __shared__ uint4 Ks[2][kBK * 8];   // [key][8 x 16B chunks], swizzled
  __shared__ uint2 Vs[2][64 * 16];   // V^T [d][16 x 8B chunks of 4 keys], swizzled

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int hi = lane >> 5;       // lane half
  const int lq = lane & 31;       // query column within the wave
  const int bh = blockIdx.x;
  const int qb = P.n_qblocks - 1 - int(blockIdx.y);  // heavy blocks first
  const int b = bh / P.H, h = bh % P.H;
  const int q0 = qb * kBQ;
  const int qw = q0 + w * 32;
  const int qi = qw + lq;  // this lane's query

  const uint16_t* Qp = P.q + b * P.q_sb + h * P.q_sh;
  const uint16_t* Kp = P.k + b * P.k_sb + h * P.k_sh;
  const uint16_t* Vp = P.v + b * P.v_sb + h * P.v_sh;

  // Q fragments (B operand of S^T = K Q^T): q row qi, d = 16*dc + 8*hi .. +8.
  uint4 qf[4];
#pragma unroll
  for (int dc = 0; dc < 4; ++dc)
    qf[dc] = qi < P.Sq ? *reinterpret_cast<const uint4*>(Qp + int64_t(qi) * P.q_ss + dc * 16 + hi * 8)
                       : make_uint4(0, 0, 0, 0);

  const int kv_end = CAUSAL ? min(P.Sk, q0 + kBQ) : P.Sk;
  const int ntiles = (kv_end + kBK - 1) / kBK;

  // Staging registers.
  uint4 kr[2];
  uint2 vr[4];
  auto fetch = [&](int j0) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int vv = i * 256 + tid;
      const int key = vv >> 3, c = vv & 7;
      const int kj = j0 + key;
      kr[i] = kj < P.Sk ? *reinterpret_cast<const uint4*>(Kp + int64_t(kj) * P.k_ss + c * 8)
                        : make_uint4(0, 0, 0, 0);
    }
    const int kq = tid >> 4, dq = tid & 15;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int kj = j0 + kq * 4 + r;
      vr[r] = kj < P.Sk ? *reinterpret_cast<const uint2*>(Vp + int64_t(kj) * P.v_ss + dq * 4)
                        : make_uint2(0, 0);
    }
  };
  auto commit = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int vv = i * 256 + tid;
      const int key = vv >> 3, c = vv & 7;
      Ks[buf][key * 8 + (c ^ ((key >> 1) & 7))] = kr[i];
    }
    // 4 keys x 4 d block -> four rows of V^T (d), 4 keys each.
    const int kq = tid >> 4, dq = tid & 15;
    uint2 t[4];
    t[0].x = (vr[0].x & 0xffffu) | (vr[1].x << 16);
    t[0].y = (vr[2].x & 0xffffu) | (vr[3].x << 16);
    t[1].x = (vr[0].x >> 16) | (vr[1].x & 0xffff0000u);
    t[1].y = (vr[2].x >> 16) | (vr[3].x & 0xffff0000u);
    t[2].x = (vr[0].y & 0xffffu) | (vr[1].y << 16);
    t[2].y = (vr[2].y & 0xffffu) | (vr[3].y << 16);
    t[3].x = (vr[0].y >> 16) | (vr[1].y & 0xffff0000u);
    t[3].y = (vr[2].y >> 16) | (vr[3].y & 0xffff0000u);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int d = dq * 4 + e;
      Vs[buf][d * 16 + (kq ^ ((d >> 1) & 15))] = t[e];
    }
  };

  float16v acc_o[2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc_o[i][e] = 0.f;
  float m_run = -1.0e30f;
  float l_run = 0.f;

  if (ntiles > 0) {
    fetch(0);
    commit(0);
  }
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    const int j0 = t * kBK;
    if (t + 1 < ntiles) fetch(j0 + kBK);

    // Wave-uniform tile classification.
    const bool skip = CAUSAL && (j0 > qw + 31);
    const bool need_mask = (CAUSAL && (j0 + kBK - 1 > qw)) || (j0 + kBK > P.Sk);
    if (!skip) {
      const uint4* ks = Ks[buf];
      const uint2* vs = Vs[buf];
      float16v s[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int e = 0; e < 16; ++e) s[kb][e] = 0.f;
#pragma unroll
        for (int dc = 0; dc < 4; ++dc) {
          const int key = kb * 32 + lq;
          const int c = dc * 2 + hi;
          const uint4 kf = ks[key * 8 + (c ^ ((key >> 1) & 7))];
          s[kb] = mfma16<BF16>(kf, qf[dc], s[kb]);
        }
      }
      // Scores -> log2 domain, mask, tile max.
      float mt = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          float x = s[kb][e];
          if constexpr (ROUND_S) x = round16<BF16>(x);
          x = x * P.sl2;
          if (need_mask) {
            const int kj = j0 + kb * 32 + 8 * (e >> 2) + 4 * hi + (e & 3);
            if (kj >= P.Sk || (CAUSAL && kj > qi)) x = -INFINITY;
          }
          s[kb][e] = x;
          mt = fmaxf(mt, x);
        }
      mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
      const float m_new = fmaxf(m_run, mt);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc_o[i][e] *= alpha;
      // P (16-bit) as the B operand: fragment (kb, mm) = s[kb][8mm .. 8mm+7].
      uint4 pf[2][2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int mm = 0; mm < 2; ++mm) {
          float p[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            p[j] = __builtin_amdgcn_exp2f(s[kb][mm * 8 + j] - m_new);
            l_run += p[j];
          }
          pf[kb][mm] = make_uint4(pack2<BF16>(p[0], p[1]), pack2<BF16>(p[2], p[3]),
                                  pack2<BF16>(p[4], p[5]), pack2<BF16>(p[6], p[7]));
        }
      // O^T += V^T P^T.  V^T fragment for (dblk, kb, mm): row d, keys
      // 32kb + 16mm + {4hi..4hi+3, 8+4hi..8+4hi+3} -> chunks 8kb+4mm+hi (+2).
#pragma unroll
      for (int dblk = 0; dblk < 2; ++dblk) {
        const int d = dblk * 32 + lq;
        const int sw = (d >> 1) & 15;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int mm = 0; mm < 2; ++mm) {
            const int c0 = 8 * kb + 4 * mm + hi;
            const uint2 v0 = vs[d * 16 + (c0 ^ sw)];
            const uint2 v1 = vs[d * 16 + ((c0 + 2) ^ sw)];
            acc_o[dblk] = mfma16<BF16>(make_uint4(v0.x, v0.y, v1.x, v1.y), pf[kb][mm], acc_o[dblk]);
          }
      }
    }
    if (t + 1 < ntiles) commit(buf ^ 1);
    __syncthreads();
  }

  // Normalise and store O[q][d]: lane holds d = 32*dblk + 8*g + 4*hi + {0..3}.
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  if (qi < P.Sq) {
    char* Ob = static_cast<char*>(P.o);
    const int64_t obase = int64_t(b) * P.o_sb + int64_t(h) * P.o_sh + int64_t(qi) * P.o_ss;
#pragma unroll
    for (int dblk = 0; dblk < 2; ++dblk)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = dblk * 32 + 8 * g + 4 * hi;
        const float x0 = acc_o[dblk][4 * g + 0] * inv, x1 = acc_o[dblk][4 * g + 1] * inv;
        const float x2 = acc_o[dblk][4 * g + 2] * inv, x3 = acc_o[dblk][4 * g + 3] * inv;
        if (P.out_dtype == 0) {
          *reinterpret_cast<float4*>(Ob + (obase + d0) * 4) = make_float4(x0, x1, x2, x3);
        } else if (P.out_dtype == 1) {
          *reinterpret_cast<uint2*>(Ob + (obase + d0) * 2) =
              make_uint2(pack2<false>(x0, x1), pack2<false>(x2, x3));
        } else {
          *reinterpret_cast<uint2*>(Ob + (obase + d0) * 2) =
              make_uint2(pack2<true>(x0, x1), pack2<true>(x2, x3));
        }
      }
  }
}

template <bool BF16, bool CAUSAL, bool ROUND_S>
void launch_fa(bg_ctx* ctx, const FaArgs& A, int bh, int nqb) {
  dim3 grid(unsigned(bh), unsigned(nqb), 1);
  bg::dispatch(ctx, fa_fwd_d64_kernel<BF16, CAUSAL, ROUND_S>, grid, dim3(256), 0, A);
}

bool al(const void* p, size_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; }


// ---- v2: 8 wavefronts x 32 queries, DMA K/V ring, software-pipelined S --------------
//
// One workgroup = 8 wavefronts x 32 queries = 256 queries of one (batch,
// head), two wavefronts per SIMD (launch bounds 512 x 1 keep each at <= 256
// registers).  Keys are processed in 64-key tiles held in a kFa2S-stage LDS
// ring filled by buffer_load_dwordx4 ... lds (each wavefront moves one 1 KB
// slice of K and one of V per tile).  Per tile t a wavefront
//   1. issues the S^T MFMAs of tile t+1 (K fragments by ds_read_b128, rows
//      swizzled by (r >> 1) & 7; Q^T fragments stay in VGPRs),
//   2. runs the online softmax of tile t on the VALU while those MFMAs run:
//      scores rounded to f16 in pairs (v_cvt_pk_f16_f32), max with
//      v_pk_max_f16, exponent argument by v_fma_mix_f32 from the packed
//      scores, v_exp_f32, P packed to 16 bits, row sums by v_dot2 on the
//      packed P (the normaliser sums exactly the P the MFMA uses),
//   3. accumulates O^T += V^T P^T (V^T fragments by ds_read_b64_tr_b16 from
//      V's natural [key][d] layout; P straight from registers, the key order
//      inside each 16-wide k step permuted identically on both operands).
// The reference max moves only when a lane's max grows by more than 2^8
// (log2 domain): P <= 256 is exact in f16/bf16 and the final 1/l normalises
// it, so the O rescale runs a handful of times per row instead of per tile.
typedef __attribute__((address_space(3))) void* fa_lds_ptr_t;
typedef short fa_v4s __attribute__((ext_vector_type(4)));
typedef _Float16 fa_h2 __attribute__((ext_vector_type(2)));
typedef float fa_f2 __attribute__((ext_vector_type(2)));
typedef uint32_t fa_u4 __attribute__((ext_vector_type(4)));

constexpr int kFa2QW = 32;              // queries per wavefront
constexpr int kFa2NW = 8;               // wavefronts per workgroup
constexpr int kFa2BQ = kFa2NW * kFa2QW; // queries per workgroup
constexpr int kFa2BK = 64;              // keys per tile
constexpr int kFa2S = 4;                // LDS ring stages (the main loop is unrolled by this)
constexpr int kFa2D = kFa2S - 2;        // tiles issued ahead of the one whose K is read
constexpr int kFa2Tile = kFa2BK * 128;  // bytes of one K or V tile
constexpr int kFa2NLD = 2;              // DMA instructions per wavefront per tile (K + V)
constexpr float kFa2Slack = 8.f;        // log2 headroom before the reference max moves
constexpr uint32_t kFa2Oob = 0x80000000u;

struct Fa2Args {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  void* o;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  int H, Sq, Sk, n_qblocks;
  float sl2;  // scale * log2(e), > 0
  int out_dtype;
  int D;      // head dim: 64 (fa2 / fa6 / fa7), or 8..56 in steps of 8 (fa7: columns past D read as zero)
};

__device__ __forceinline__ int fa2_k_unit(int r, int c) { return r * 8 + (c ^ ((r >> 1) & 7)); }
__device__ __forceinline__ int fa2_v_unit(int r, int c) { return r * 8 + (c ^ ((r & 3) << 1)); }

// Value of the lane 32 apart (lanes l and l ^ 32 hold the same query).
// v_permlane32_swap exchanges the upper half of its first operand with the
// lower half of its second: lanes 0-31 find the partner in the second
// result, lanes 32-63 in the first.
__device__ __forceinline__ float fa2_xor32(float x) {
  const int v = __builtin_bit_cast(int, x);
  const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return __builtin_bit_cast(float, (threadIdx.x & 32) ? r[0] : r[1]);
}

template <int N>
__device__ __forceinline__ void fa2_wait_vm_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
}

template <bool BF16>
__device__ __forceinline__ float16v fa2_mfma(fa_u4 a, fa_u4 b, float16v c) {
  if constexpr (BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf168, a), __builtin_bit_cast(bf168, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c,
                                                  0, 0, 0);
}

// Two floats -> packed 16-bit pair (round to nearest even).
template <bool BF16>
__device__ __forceinline__ uint32_t fa2_pack(float a, float b) {
  if constexpr (BF16) {
    return uint32_t(__builtin_bit_cast(uint16_t, static_cast<__bf16>(a))) |
           (uint32_t(__builtin_bit_cast(uint16_t, static_cast<__bf16>(b))) << 16);
  } else {
    const fa_h2 h = __builtin_convertvector((fa_f2){a, b}, fa_h2);
    return __builtin_bit_cast(uint32_t, h);
  }
}

template <bool BF16>
__device__ __forceinline__ float fa2_lo(uint32_t p) {
  if constexpr (BF16) return __uint_as_float(p << 16);
  else return static_cast<float>(__builtin_bit_cast(fa_h2, p)[0]);
}
template <bool BF16>
__device__ __forceinline__ float fa2_hi(uint32_t p) {
  if constexpr (BF16) return __uint_as_float(p & 0xffff0000u);
  else return static_cast<float>(__builtin_bit_cast(fa_h2, p)[1]);
}

// S^T tile (64 keys x 32 queries) of the K tile at kt: s[kb] holds keys
// 32kb + 8*(e/4) + 4*(lane/32) + e%4 for query lane%32.
template <bool BF16>
__device__ __forceinline__ void fa2_scores(const char* kt, const fa_u4 (&qf)[4], float16v (&s)[2]) {
  const int lane = threadIdx.x & 63, hi = lane >> 5;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    const int r = kb * 32 + (lane & 31);
    fa_u4 kf[4];
#pragma unroll
    for (int dc = 0; dc < 4; ++dc) kf[dc] = *reinterpret_cast<const fa_u4*>(kt + fa2_k_unit(r, dc * 2 + hi) * 16);
    s[kb] = fa2_mfma<BF16>(kf[0], qf[0], float16v{});
#pragma unroll
    for (int dc = 1; dc < 4; ++dc) s[kb] = fa2_mfma<BF16>(kf[dc], qf[dc], s[kb]);
  }
}

// Online-softmax update of tile j0 for this lane's query qi; P (16-bit,
// packed as MFMA B fragments) into pf[kb][mm].
template <bool BF16, bool CAUSAL, bool ROUND_S>
__device__ __forceinline__ void fa2_softmax(float16v (&s)[2], int j0, int qi, int Sk, bool need_mask, float sl2,
                                            float& m_run, float& l_run, float16v (&acc)[2], fa_u4 (&pf)[2][2]) {
  const int hi = (threadIdx.x >> 5) & 1;
  if (need_mask) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int kj = j0 + kb * 32 + 8 * (e >> 2) + 4 * hi + (e & 3);
        if (kj >= Sk || (CAUSAL && kj > qi)) s[kb][e] = -INFINITY;
      }
  }
  uint32_t sp[2][8];  // rounded scores, packed pairs (ROUND_S)
  float mt;
  if constexpr (ROUND_S) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 8; ++e) sp[kb][e] = fa2_pack<BF16>(s[kb][2 * e], s[kb][2 * e + 1]);
    if constexpr (!BF16) {
      // IEEE maximum (NaN-propagating, like NumPy's max) pairs into
      // v_pk_maximum3_f16: 8 instructions for the 16 packed pairs.
      fa_h2 m2 = __builtin_bit_cast(fa_h2, sp[0][0]);
#pragma unroll
      for (int i = 1; i < 16; ++i) m2 = __builtin_elementwise_maximum(m2, __builtin_bit_cast(fa_h2, sp[i >> 3][i & 7]));
      mt = fmaxf(static_cast<float>(m2[0]), static_cast<float>(m2[1]));
    } else {
      mt = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 8; ++e) mt = fmaxf(mt, fmaxf(fa2_lo<true>(sp[kb][e]), fa2_hi<true>(sp[kb][e])));
    }
  } else {
    mt = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int e = 0; e < 16; ++e) mt = fmaxf(mt, s[kb][e]);
  }
  mt = fmaxf(mt, fa2_xor32(mt));
  const float mc = mt * sl2;
  // Wavefront-uniform: move the reference max only when some lane's max
  // exceeds it by more than kFa2Slack (always on the first tile: m_run = -inf).
  if (__any(mc > m_run + kFa2Slack)) {
    const float m_new = fmaxf(m_run, mc);
    const float alpha = m_new == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);
    m_run = m_new;
    l_run *= alpha;
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[db][e] *= alpha;
  }
  const float m_use = m_run == -INFINITY ? 0.f : m_run;
  const fa_h2 ones = {(_Float16)1.f, (_Float16)1.f};
  float l_acc = 0.f;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int mm = 0; mm < 2; ++mm) {
      uint32_t pk[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int e = mm * 8 + 2 * j;
        float x0, x1;
        if constexpr (ROUND_S) {
          x0 = __builtin_fmaf(fa2_lo<BF16>(sp[kb][e / 2]), sl2, -m_use);
          x1 = __builtin_fmaf(fa2_hi<BF16>(sp[kb][e / 2]), sl2, -m_use);
        } else {
          x0 = __builtin_fmaf(s[kb][e], sl2, -m_use);
          x1 = __builtin_fmaf(s[kb][e + 1], sl2, -m_use);
        }
        pk[j] = fa2_pack<BF16>(__builtin_amdgcn_exp2f(x0), __builtin_amdgcn_exp2f(x1));
        if constexpr (BF16) l_acc += fa2_lo<true>(pk[j]) + fa2_hi<true>(pk[j]);
        else l_acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(fa_h2, pk[j]), ones, l_acc, false);
      }
      pf[kb][mm] = fa_u4{pk[0], pk[1], pk[2], pk[3]};
    }
  l_run += l_acc;
}

// O^T += V^T P^T over the V tile at vt.  V^T fragments by transpose reads:
// for lane l (group g = l/16, s = l%16) rows 32kb + 16mm + 8r + 4*(l/32) +
// s/4, d = 32db + 16*(g%2) + 4*(s%4).
template <bool BF16>
__device__ __forceinline__ void fa2_pv(const char* vt, const fa_u4 (&pf)[2][2], float16v (&acc)[2]) {
  const int lane = threadIdx.x & 63, hi = lane >> 5;
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int mm = 0; mm < 2; ++mm) {
        fa_v4s part[2];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const int row = kb * 32 + mm * 16 + r * 8 + 4 * hi + ((lane & 15) >> 2);
          const int d = db * 32 + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
          const char* addr = vt + fa2_v_unit(row, d >> 3) * 16 + (d & 4) * 2;
          part[r] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) fa_v4s*)(reinterpret_cast<uintptr_t>(addr)));
        }
        // One bit-cast of the concatenated vector. (Rebuilding the halves
        // element by element through _Float16 casts was miscompiled by
        // this clang into a single element broadcast.)
        const fa_u4 vf =
            __builtin_bit_cast(fa_u4, __builtin_shufflevector(part[0], part[1], 0, 1, 2, 3, 4, 5, 6, 7));
        acc[db] = fa2_mfma<BF16>(vf, pf[kb][mm], acc[db]);
      }
}

template <bool BF16, bool CAUSAL, bool ROUND_S>
__global__ void __launch_bounds__(kFa2NW * 64, 1) fa2_fwd_kernel(Fa2Args P, uint32_t k_bytes, uint32_t v_bytes) {
  __shared__ fa_u4 smem[kFa2S * 2 * kFa2Tile / 16];
  char* sb = reinterpret_cast<char*>(smem);

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hi = lane >> 5;
  const int bh = blockIdx.x;
  const int qblk = P.n_qblocks - 1 - int(blockIdx.y);  // heavy query blocks first
  const int b = bh / P.H, h = bh % P.H;
  const int q0 = qblk * kFa2BQ;
  const int q0w = q0 + w * kFa2QW;
  const int qi = q0w + (lane & 31);

  const uint16_t* Qp = P.q + b * P.q_sb + h * P.q_sh;
  const uint16_t* Kp = P.k + b * P.k_sb + h * P.k_sh;
  const uint16_t* Vp = P.v + b * P.v_sb + h * P.v_sh;
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc((void*)Kp, (short)0, int(k_bytes), 0x00020000);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc((void*)Vp, (short)0, int(v_bytes), 0x00020000);
  const __amdgpu_buffer_rsrc_t r0 = __builtin_amdgcn_make_buffer_rsrc((void*)Kp, (short)0, 0, 0x00020000);

  const int nt_all = (P.Sk + kFa2BK - 1) / kFa2BK;
  const int nt = CAUSAL ? min(nt_all, (q0 + kFa2BQ + kFa2BK - 1) / kFa2BK) : nt_all;
  // Tiles this wavefront computes (causal: up to its own diagonal).
  const int ntw = CAUSAL ? min(nt, (q0w + kFa2QW + kFa2BK - 1) / kFa2BK) : nt;

  // DMA: wavefront w fills the 1 KB slice w (rows 8w .. 8w+7) of each K and
  // V tile; lane L writes 16-byte unit 64w + L = (row r, physical chunk pc),
  // which holds logical chunk pc ^ swizzle(r).
  const int u = w * 64 + lane;
  const int krow = u >> 3, pc = u & 7;
  const uint32_t koff = uint32_t((int64_t(krow) * P.k_ss + ((pc ^ ((krow >> 1) & 7)) * 8)) * 2);
  const uint32_t voff = uint32_t((int64_t(krow) * P.v_ss + ((pc ^ ((krow & 3) << 1)) * 8)) * 2);
  auto issue_tile = [&](int t, int stage) {
    char* st = sb + stage * 2 * kFa2Tile;
    const bool real = t < nt;
    const bool ok = real && t * kFa2BK + krow < P.Sk;
    const uint32_t kso = real ? uint32_t(int64_t(t) * kFa2BK * P.k_ss * 2) : 0u;
    const uint32_t vso = real ? uint32_t(int64_t(t) * kFa2BK * P.v_ss * 2) : 0u;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(real ? rk : r0, (fa_lds_ptr_t)(st + w * 1024), 16,
                                             ok ? koff : kFa2Oob, kso, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(real ? rv : r0, (fa_lds_ptr_t)(st + kFa2Tile + w * 1024), 16,
                                             ok ? voff : kFa2Oob, vso, 0, 0);
  };

  // Q^T fragments (B operand of S^T = K Q^T): query qi, d = 16*dc + 8*hi .. +8.
  fa_u4 qf[4];
#pragma unroll
  for (int dc = 0; dc < 4; ++dc)
    qf[dc] = qi < P.Sq ? *reinterpret_cast<const fa_u4*>(Qp + int64_t(qi) * P.q_ss + dc * 16 + hi * 8)
                       : fa_u4{0u, 0u, 0u, 0u};
  // Tiles 0 .. kFa2D in flight; wait for tile 0 (and Q) only.
#pragma unroll
  for (int t = 0; t <= kFa2D; ++t) issue_tile(t, t);
  fa2_wait_vm_lgkm0<kFa2NLD * kFa2D>();
  __builtin_amdgcn_s_barrier();

  float16v acc[2];
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[db][e] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  const float sl2 = P.sl2;

  float16v s_a[2], s_b[2];
  if (ntw > 0) fa2_scores<BF16>(sb, qf, s_a);

  // Tile t: K(t+1) and V(t) must be resident.  Outstanding DMA at the top:
  // tiles t+1 .. t+kFa2D; wait until t+1 has landed, then (after the
  // barrier every wavefront is done with tile t-1's stage) refill that stage
  // with tile t+1+kFa2D.  The ring stage of t is the compile-time STG, so
  // every LDS address is a loop-invariant lane offset plus an immediate.
  auto step = [&](auto stg, int t, float16v(&s_cur)[2], float16v(&s_nxt)[2]) {
    constexpr int STG = decltype(stg)::value;
    fa2_wait_vm_lgkm0<kFa2NLD * (kFa2D - 1)>();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    issue_tile(t + 1 + kFa2D, (STG + 1 + kFa2D) % kFa2S);
    if (t >= ntw) return;
    const char* kt_next = sb + ((STG + 1) % kFa2S) * 2 * kFa2Tile;
    const char* vt = sb + STG * 2 * kFa2Tile + kFa2Tile;
    if (t + 1 < ntw) fa2_scores<BF16>(kt_next, qf, s_nxt);
    const int j0 = t * kFa2BK;
    const bool need_mask = (CAUSAL && j0 + kFa2BK - 1 > q0w) || (j0 + kFa2BK > P.Sk);
    fa_u4 pf[2][2];
    fa2_softmax<BF16, CAUSAL, ROUND_S>(s_cur, j0, qi, P.Sk, need_mask, sl2, m_run, l_run, acc, pf);
    fa2_pv<BF16>(vt, pf, acc);
  };
  using C0 = std::integral_constant<int, 0>;
  using C1 = std::integral_constant<int, 1>;
  using C2 = std::integral_constant<int, 2>;
  using C3 = std::integral_constant<int, 3>;
  static_assert(kFa2S == 4, "main loop unrolled by the ring size");
  int t = 0;
  for (; t + 3 < nt; t += 4) {
    step(C0{}, t, s_a, s_b);
    step(C1{}, t + 1, s_b, s_a);
    step(C2{}, t + 2, s_a, s_b);
    step(C3{}, t + 3, s_b, s_a);
  }
  if (t < nt) step(C0{}, t, s_a, s_b);
  if (t + 1 < nt) step(C1{}, t + 1, s_b, s_a);
  if (t + 2 < nt) step(C2{}, t + 2, s_a, s_b);
  fa2_wait_vm_lgkm0<0>();  // no DMA into this workgroup's LDS outlives it

  // O = acc / l.  O^T layout: lane = query column, register e holds d row
  // 8*(e/4) + 4*hi + e%4 (+ 32*db): four consecutive d per (e/4) group.
  const float lt = l_run + fa2_xor32(l_run);
  const float inv = lt > 0.f ? 1.0f / lt : 0.f;
  if (qi >= P.Sq) return;
  char* Ob = static_cast<char*>(P.o);
  const int64_t obase = int64_t(b) * P.o_sb + int64_t(h) * P.o_sh + int64_t(qi) * P.o_ss;
  if (P.out_dtype == 0) {
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = db * 32 + 8 * g + 4 * hi;
        *reinterpret_cast<float4*>(Ob + (obase + d0) * 4) =
            make_float4(acc[db][4 * g] * inv, acc[db][4 * g + 1] * inv, acc[db][4 * g + 2] * inv,
                        acc[db][4 * g + 3] * inv);
      }
  } else if (P.out_dtype == 1) {
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = db * 32 + 8 * g + 4 * hi;
        *reinterpret_cast<uint2*>(Ob + (obase + d0) * 2) =
            make_uint2(fa2_pack<false>(acc[db][4 * g] * inv, acc[db][4 * g + 1] * inv),
                       fa2_pack<false>(acc[db][4 * g + 2] * inv, acc[db][4 * g + 3] * inv));
      }
  } else {
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = db * 32 + 8 * g + 4 * hi;
        *reinterpret_cast<uint2*>(Ob + (obase + d0) * 2) =
            make_uint2(fa2_pack<true>(acc[db][4 * g] * inv, acc[db][4 * g + 1] * inv),
                       fa2_pack<true>(acc[db][4 * g + 2] * inv, acc[db][4 * g + 3] * inv));
      }
  }
}

// ---- v6: 32-key halves, softmax folded into the MFMA, two workgroups per CU --
//
// One workgroup = 8 wavefronts x 32 queries of one (batch, head); K and V
// tiles of 64 keys stream through a 4-slot LDS ring (buffer_load ... lds,
// each wavefront copies a 1 KB slice of K and of V per tile; tile j lives in
// slot j % 4, step t refills the slot of tile t-1 with tile t+3 after the
// step's barrier).  Each wavefront works through a tile in two 32-key halves:
//   x  = K Q'^T + (-m)       4 MFMAs (32x32x16), Q' = Q * scale * log2(e)
//   P  = exp2(x)             packed to 16 bits, row sum in f32 by adds
//   O^T += V^T P^T           4 MFMAs, V^T fragments by ds_read_b64_tr_b16
// Q' is rounded to the input dtype once per wavefront, and the S chain starts
// from an accumulator block holding -m (the wavefront's reference max per
// query), so the fast path has no per-score FMA and no per-tile max.  The
// reference max only has to keep P finite in 16 bits: it is set exactly on
// the first half a wavefront sees and moved again only when some P of a half
// may overflow (its f32 row sum reaches 2^15); that slow path takes the
// exact max, rescales O and l and recomputes P.  At 124 registers two
// workgroups share a CU, four wavefronts per SIMD, which hides MFMA, LDS and
// transcendental latency across wavefronts.
// Numerics: S is not rounded to 16 bits before scaling (the reference's AMP
// matmul rounds it); Q' carries one 16-bit rounding instead.  Both are below
// the input precision; the parity tests bound the result at the 16-bit tolerance.
constexpr int kFa6Ring = 4;

__device__ __forceinline__ float fa6_muse(float m_run) { return m_run == -INFINITY ? 0.f : m_run; }

// Per-lane LDS byte offsets of the K and V fragment reads within a tile.
// K: row r = 32 kb + lane % 32, chunk 2 dc + lane / 32, swizzled by
// (r >> 1) & 7 (the same for both kb), so kb only adds 4096.  V (transpose
// reads): row = 32 kb + 16 mm + 8 r + rl with rl = 4 (lane / 32) +
// (lane % 16) / 4 and row % 4 = (lane / 4) % 4, so kb, mm and r only add
// multiples of 1024; d = 32 db + 16 ((lane / 16) % 2) + 4 (lane % 4).
struct Fa6Offs {
  uint32_t k[4];
  uint32_t v[2];
  __device__ __forceinline__ Fa6Offs() {
    const int lane = threadIdx.x & 63, hi = lane >> 5, l32 = lane & 31;
#pragma unroll
    for (int dc = 0; dc < 4; ++dc) k[dc] = uint32_t(fa2_k_unit(l32, dc * 2 + hi) * 16);
    const int rl = 4 * hi + ((lane & 15) >> 2);
#pragma unroll
    for (int db = 0; db < 2; ++db) {
      const int d = db * 32 + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
      v[db] = uint32_t(fa2_v_unit(rl, d >> 3) * 16 + (d & 4) * 2);
    }
  }
};

template <bool BF16>
__device__ __forceinline__ void fa6_pv_half(const char* vt, const Fa6Offs& o, const fa_u4 (&pf)[2], float16v (&acc)[2],
                                            int h) {
#pragma unroll
  for (int mm = 0; mm < 2; ++mm)
#pragma unroll
    for (int db = 0; db < 2; ++db) {
      fa_v4s part[2];
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const char* addr = vt + o.v[db] + (h * 32 + mm * 16 + r * 8) * 128;
        part[r] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) fa_v4s*)(reinterpret_cast<uintptr_t>(addr)));
      }
      const fa_u4 vf = __builtin_bit_cast(fa_u4, __builtin_shufflevector(part[0], part[1], 0, 1, 2, 3, 4, 5, 6, 7));
      acc[db] = fa2_mfma<BF16>(vf, pf[mm], acc[db]);
    }
}

template <bool BF16>
__device__ __forceinline__ uint32_t fa6_scale2(uint32_t w, float sl2) {
  return fa2_pack<BF16>(fa2_lo<BF16>(w) * sl2, fa2_hi<BF16>(w) * sl2);
}

template <bool BF16>
__device__ __forceinline__ float16v fa6_scores_half(const char* kt, const Fa6Offs& o, const fa_u4 (&qf)[4],
                                                    const float16v& mneg, int h) {
  fa_u4 kf[4];
#pragma unroll
  for (int dc = 0; dc < 4; ++dc) kf[dc] = *reinterpret_cast<const fa_u4*>(kt + o.k[dc] + h * 4096);
  float16v s = fa2_mfma<BF16>(kf[0], qf[0], mneg);
#pragma unroll
  for (int dc = 1; dc < 4; ++dc) s = fa2_mfma<BF16>(kf[dc], qf[dc], s);
  return s;
}

// P = exp2(x + delta) packed as two B fragments; returns the row sum of the
// packed values.
template <bool BF16, bool ADD>
// The row sum is taken over the f32 values before the 16-bit rounding, with
// plain adds in two chains: v_dot2 on the packed P does not issue beside
// MFMAs (measured on MI355X: two dot2 per MFMA stretch the MFMA issue
// interval from 14.8 to 24.9 ns, while adds, converts and two v_exp_f32 per
// MFMA fit inside it).
__device__ __forceinline__ float fa6_exp(const float16v& x, float delta, fa_u4 (&pf)[2]) {
  float l0 = 0.f, l1 = 0.f;
#pragma unroll
  for (int mm = 0; mm < 2; ++mm) {
    uint32_t pk[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = mm * 8 + 2 * j;
      const float x0 = ADD ? x[e] + delta : x[e];
      const float x1 = ADD ? x[e + 1] + delta : x[e + 1];
      const float e0 = __builtin_amdgcn_exp2f(x0), e1 = __builtin_amdgcn_exp2f(x1);
      l0 += e0;
      l1 += e1;
      pk[j] = fa2_pack<BF16>(e0, e1);
    }
    pf[mm] = fa_u4{pk[0], pk[1], pk[2], pk[3]};
  }
  return l0 + l1;
}

template <bool BF16, bool CAUSAL>
__global__ void __launch_bounds__(kFa2NW * 64, 2) fa6_fwd_kernel(Fa2Args P, uint32_t k_bytes, uint32_t v_bytes) {
  __shared__ fa_u4 smem[2 * kFa6Ring * kFa2Tile / 16];
  char* sb = reinterpret_cast<char*>(smem);
  char* kring = sb;
  char* vring = sb + kFa6Ring * kFa2Tile;

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hi = lane >> 5;
  const int bh = blockIdx.x;
  const int qblk = P.n_qblocks - 1 - int(blockIdx.y);  // heavy query blocks first
  const int b = bh / P.H, h = bh % P.H;
  const int q0 = qblk * kFa2BQ;
  const int q0w = q0 + w * kFa2QW;
  const int qi = q0w + (lane & 31);

  const uint16_t* Qp = P.q + b * P.q_sb + h * P.q_sh;
  const uint16_t* Kp = P.k + b * P.k_sb + h * P.k_sh;
  const uint16_t* Vp = P.v + b * P.v_sb + h * P.v_sh;
  const bgk::sgpr4_t rk = bgk::buffer_rsrc(Kp, k_bytes);
  const bgk::sgpr4_t rv = bgk::buffer_rsrc(Vp, v_bytes);

  const int nt_all = (P.Sk + kFa2BK - 1) / kFa2BK;
  const int nt = CAUSAL ? min(nt_all, (q0 + kFa2BQ + kFa2BK - 1) / kFa2BK) : nt_all;
  const int ntw = CAUSAL ? min(nt, (q0w + kFa2QW + kFa2BK - 1) / kFa2BK) : nt;

  const int u = w * 64 + lane;
  const int krow = u >> 3, pc = u & 7;
  const uint32_t koff = uint32_t((int64_t(krow) * P.k_ss + ((pc ^ ((krow >> 1) & 7)) * 8)) * 2);
  const uint32_t voff = uint32_t((int64_t(krow) * P.v_ss + ((pc ^ ((krow & 3) << 1)) * 8)) * 2);
  const uint32_t kstep = uint32_t(int64_t(kFa2BK) * P.k_ss * 2);
  const uint32_t vstep = uint32_t(int64_t(kFa2BK) * P.v_ss * 2);
  const uint32_t kl = bgk::lds_addr(kring) + uint32_t(w) * 1024u;
  const uint32_t vl = bgk::lds_addr(vring) + uint32_t(w) * 1024u;
  auto issue = [&](int j) {
    const bool real = j >= 0 && j < nt;
    const bool ok = real && j * kFa2BK + krow < P.Sk;
    const uint32_t sl = uint32_t(j & 3) * kFa2Tile;
    bgk::dma16_to_lds(kl + sl, ok ? koff : kFa2Oob, rk, real ? uint32_t(j) * kstep : 0u);
    bgk::dma16_to_lds(vl + sl, ok ? voff : kFa2Oob, rv, real ? uint32_t(j) * vstep : 0u);
  };

  const float sl2 = P.sl2;
  fa_u4 qf[4];
#pragma unroll
  for (int dc = 0; dc < 4; ++dc)
    qf[dc] = qi < P.Sq ? *reinterpret_cast<const fa_u4*>(Qp + int64_t(qi) * P.q_ss + dc * 16 + hi * 8)
                       : fa_u4{0u, 0u, 0u, 0u};
  issue(0);
  issue(1);
  issue(2);
  fa2_wait_vm_lgkm0<0>();  // also retires the Q loads in the compiler's bookkeeping
  __builtin_amdgcn_s_barrier();
#pragma unroll
  for (int dc = 0; dc < 4; ++dc)
#pragma unroll
    for (int i = 0; i < 4; ++i) qf[dc][i] = fa6_scale2<BF16>(qf[dc][i], sl2);

  float16v acc[2];
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[db][e] = 0.f;
  float16v mneg;  // -m_use in every row of this lane's query column
#pragma unroll
  for (int e = 0; e < 16; ++e) mneg[e] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  const Fa6Offs offs;

  for (int t = 0; t < nt; ++t) {
    if (t > 0) {
      fa2_wait_vm_lgkm0<4>();
      __builtin_amdgcn_s_barrier();
    }
    issue(t + 3);
    if (t < ntw) {
      const char* kt = kring + (t & 3) * kFa2Tile;
      const char* vt = vring + (t & 3) * kFa2Tile;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int j0 = t * kFa2BK + hh * 32;
        float16v x = fa6_scores_half<BF16>(kt, offs, qf, mneg, hh);
        if ((CAUSAL && j0 + 31 > q0w) || (j0 + 32 > P.Sk)) {
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int kj = j0 + 8 * (e >> 2) + 4 * hi + (e & 3);
            if (kj >= P.Sk || (CAUSAL && kj > qi)) x[e] = -INFINITY;
          }
        }
        fa_u4 pf[2];
        float l_acc = fa6_exp<BF16, false>(x, 0.f, pf);
        // The f32 sum bounds every P of the half, so a sum below 2^15 means
        // no P reached the f16 limit; otherwise (or on the first half)
        // take the exact maximum and recompute P.
        if (__any(!(l_acc < 32768.f) || m_run == -INFINITY)) {  // wave-uniform
          // Exact max of this half (x = scores - m_use), moved reference.
          float mt = -INFINITY;
#pragma unroll
          for (int e = 0; e < 16; ++e) mt = fmaxf(mt, x[e]);
          mt = fmaxf(mt, fa2_xor32(mt));
          const float m_use = fa6_muse(m_run);
          const float m_tile = mt + m_use;
          const float m_new = fmaxf(m_run, m_tile);
          const float alpha = m_run == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);
          m_run = m_new;
          const float m_use_new = fa6_muse(m_run);
          l_acc = fa6_exp<BF16, true>(x, m_use - m_use_new, pf);
          l_run *= alpha;
#pragma unroll
          for (int db = 0; db < 2; ++db)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[db][e] *= alpha;
#pragma unroll
          for (int e = 0; e < 16; ++e) mneg[e] = -m_use_new;
        }
        l_run += l_acc;
        fa6_pv_half<BF16>(vt, offs, pf, acc, hh);
      }
    }
  }
  fa2_wait_vm_lgkm0<0>();

  const float lt = l_run + fa2_xor32(l_run);
  const float inv = lt > 0.f ? 1.0f / lt : 0.f;
  if (qi >= P.Sq) return;
  char* Ob = static_cast<char*>(P.o);
  const int64_t obase = int64_t(b) * P.o_sb + int64_t(h) * P.o_sh + int64_t(qi) * P.o_ss;
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const int d0 = db * 32 + 8 * gq + 4 * hi;
      if (d0 >= P.D) continue;
      const float y0 = acc[db][4 * gq] * inv, y1 = acc[db][4 * gq + 1] * inv;
      const float y2 = acc[db][4 * gq + 2] * inv, y3 = acc[db][4 * gq + 3] * inv;
      if (P.out_dtype == 0)
        *reinterpret_cast<float4*>(Ob + (obase + d0) * 4) = make_float4(y0, y1, y2, y3);
      else if (P.out_dtype == 1)
        *reinterpret_cast<uint2*>(Ob + (obase + d0) * 2) =
            make_uint2(fa2_pack<false>(y0, y1), fa2_pack<false>(y2, y3));
      else
        *reinterpret_cast<uint2*>(Ob + (obase + d0) * 2) =
            make_uint2(fa2_pack<true>(y0, y1), fa2_pack<true>(y2, y3));
    }
}

// ---- v7: v6 without the per-half overflow branch ----------------------------
//
// v6's lazy reference max needs a wave-uniform test after every half (does
// some P of this half reach the 16-bit limit?).  The test waits for the
// whole exp2 chain and splits the scheduling region, which measured 35-43%
// of the loop on MI355X.  v7 fixes the reference max per query once, from
// the exact maximum of that query's first 32 keys, and runs every half
// branch-free.  A later key may still exceed it by 16 or more (in log2
// units), rounding some P to infinity in 16 bits; the infinity then reaches
// O (inf * v, or inf * 0 = NaN) or l, so it is caught once at the end: a
// wavefront whose l or O is not finite recomputes its 32 queries with an
// exact running max (fa7_exact), reading K and V straight from global
// memory.  Only inputs with a key that dominates the first 32 by 2^16 take
// that path.
// The loop is split in two: tiles where no wavefront of the workgroup needs
// a causal or length mask, then the remaining (diagonal) tiles with the
// mask test.  Ring, copies and barriers are v6's.

// ROUND_S form of fa6_exp: x holds raw scores S = Q K^T (f32 accumulate);
// each is rounded to the input dtype (the reference's AMP matmul output),
// then scaled into the log2 domain against the reference max:
// P = exp2(16-bit(S) * scale * log2 e - m).  Returns the f32 row sum.
template <bool BF16>
__device__ __forceinline__ float fa7_exp_round(const float16v& x, float sl2, float negm, fa_u4 (&pf)[2]) {
  float l0 = 0.f, l1 = 0.f;
#pragma unroll
  for (int mm = 0; mm < 2; ++mm) {
    uint32_t pk[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = mm * 8 + 2 * j;
      const uint32_t sr = fa2_pack<BF16>(x[e], x[e + 1]);
      const float e0 = __builtin_amdgcn_exp2f(__builtin_fmaf(fa2_lo<BF16>(sr), sl2, negm));
      const float e1 = __builtin_amdgcn_exp2f(__builtin_fmaf(fa2_hi<BF16>(sr), sl2, negm));
      l0 += e0;
      l1 += e1;
      pk[j] = fa2_pack<BF16>(e0, e1);
    }
    pf[mm] = fa_u4{pk[0], pk[1], pk[2], pk[3]};
  }
  return l0 + l1;
}

// O = acc / l for this lane's query; O^T layout: register e of acc[db] holds
// d = 32 db + 8 (e / 4) + 4 hi + e % 4.
__device__ __forceinline__ void fa7_store(const Fa2Args& P, int b, int h, int qi, const float16v (&acc)[2],
                                          float l_run) {
  const int hi = (threadIdx.x >> 5) & 1;
  const float lt = l_run + fa2_xor32(l_run);
  const float inv = lt > 0.f ? 1.0f / lt : 0.f;
  if (qi >= P.Sq) return;
  char* Ob = static_cast<char*>(P.o);
  const int64_t obase = int64_t(b) * P.o_sb + int64_t(h) * P.o_sh + int64_t(qi) * P.o_ss;
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const int d0 = db * 32 + 8 * gq + 4 * hi;
      if (d0 >= P.D) continue;
      const float y0 = acc[db][4 * gq] * inv, y1 = acc[db][4 * gq + 1] * inv;
      const float y2 = acc[db][4 * gq + 2] * inv, y3 = acc[db][4 * gq + 3] * inv;
      if (P.out_dtype == 0)
        *reinterpret_cast<float4*>(Ob + (obase + d0) * 4) = make_float4(y0, y1, y2, y3);
      else if (P.out_dtype == 1)
        *reinterpret_cast<uint2*>(Ob + (obase + d0) * 2) =
            make_uint2(fa2_pack<false>(y0, y1), fa2_pack<false>(y2, y3));
      else
        *reinterpret_cast<uint2*>(Ob + (obase + d0) * 2) =
            make_uint2(fa2_pack<true>(y0, y1), fa2_pack<true>(y2, y3));
    }
}

// Exact pass for one wavefront (the 32 queries from q0w), small in
// registers so that inlining it costs the fast loop nothing: one query at a
// time, one key per lane for the scores (s = sum_d Q'_d K_d with the fast
// path's Q' = 16-bit(Q * scale * log2 e)), the exact running maximum over
// 64-key chunks, and one output dimension per lane for P V (P rounded to
// the input dtype, as the fast path's MFMA operand is).
__device__ __forceinline__ float fa7_wave_max(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, 64));
  return x;
}

template <bool BF16>
__device__ __forceinline__ float fa7_round(float x) {
  if constexpr (BF16) return static_cast<float>(static_cast<__bf16>(x));
  else return static_cast<float>(static_cast<_Float16>(x));
}

template <bool BF16, bool CAUSAL, bool ROUND_S>
__device__ __forceinline__ void fa7_exact(const Fa2Args& P, int b, int h, int q0w) {
  const int lane = threadIdx.x & 63;
  const uint16_t* Qp = P.q + b * P.q_sb + h * P.q_sh;
  const uint16_t* Kp = P.k + b * P.k_sb + h * P.k_sh;
  const uint16_t* Vp = P.v + b * P.v_sb + h * P.v_sh;
  char* Ob = static_cast<char*>(P.o);
  for (int iq = 0; iq < kFa2QW; ++iq) {
    const int qi = q0w + iq;
    if (qi >= P.Sq) break;
    const uint16_t* qrow = Qp + int64_t(qi) * P.q_ss;
    const int nkeys = CAUSAL ? min(P.Sk, qi + 1) : P.Sk;
    float m_run = -INFINITY, l_run = 0.f, o = 0.f;
    for (int j0 = 0; j0 < nkeys; j0 += 64) {
      const int j = j0 + lane;
      float sc = -INFINITY;
      if (j < nkeys) {
        const uint16_t* krow = Kp + int64_t(j) * P.k_ss;
        float acc = 0.f;
        for (int d = 0; d < P.D; d += 2) {
          const uint32_t qw = *reinterpret_cast<const uint32_t*>(qrow + d);
          const uint32_t kw = *reinterpret_cast<const uint32_t*>(krow + d);
          if constexpr (ROUND_S) {
            acc += fa2_lo<BF16>(qw) * fa2_lo<BF16>(kw);
            acc += fa2_hi<BF16>(qw) * fa2_hi<BF16>(kw);
          } else {
            acc += fa7_round<BF16>(fa2_lo<BF16>(qw) * P.sl2) * fa2_lo<BF16>(kw);
            acc += fa7_round<BF16>(fa2_hi<BF16>(qw) * P.sl2) * fa2_hi<BF16>(kw);
          }
        }
        // ROUND_S: the score rounds to the input dtype before scaling.
        sc = ROUND_S ? fa7_round<BF16>(acc) * P.sl2 : acc;
      }
      const float m_new = fmaxf(m_run, fa7_wave_max(sc));
      const float alpha = m_run == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);
      const float pe = j < nkeys ? __builtin_amdgcn_exp2f(sc - m_new) : 0.f;
      l_run = l_run * alpha + bgk::wave_sum(pe);
      o *= alpha;
      m_run = m_new;
      const float p16 = fa7_round<BF16>(pe);
      const int jn = min(64, nkeys - j0);
      for (int jj = 0; jj < jn; ++jj) {
        const float pj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, p16), jj));
        const uint16_t vv = lane < P.D ? Vp[int64_t(j0 + jj) * P.v_ss + lane] : uint16_t(0);
        o += pj * (BF16 ? bgk::bf16_bits_to_f32(vv) : bgk::f16_bits_to_f32(vv));
      }
    }
    const float y = l_run > 0.f ? o / l_run : 0.f;
    if (lane < P.D) {
      const int64_t oi = int64_t(b) * P.o_sb + int64_t(h) * P.o_sh + int64_t(qi) * P.o_ss + lane;
      if (P.out_dtype == 0) reinterpret_cast<float*>(Ob)[oi] = y;
      else if (P.out_dtype == 1) reinterpret_cast<uint16_t*>(Ob)[oi] = bgk::f32_to_f16_bits(y);
      else reinterpret_cast<uint16_t*>(Ob)[oi] = bgk::f32_to_bf16_bits(y);
    }
  }
}

// Workgroup -> (head, query block).  Heavy query blocks (causal: more key
// tiles) come first in a global order whose position g maps to head g % bh
// and block n_qblocks - 1 - g / bh.  Workgroups are dispatched round-robin
// over the 8 XCDs, so XCD x takes positions x, x + 8, ... (a head's blocks
// stay on one XCD when bh % 8 == 0); within an XCD the first rounds of 32
// (one workgroup per CU) alternate direction, so a CU that starts with one
// of the heaviest blocks of a round gets one of the lightest of the next:
// with C5's 96 heads x 8 blocks (2..16 tiles, three per CU) the per-CU
// tile sums go from 20-34 to 24-30 (modelled; 25.0 -> 24.0 us measured).
// Reversing only whole rounds keeps the map a bijection.  Only the
// 128-query shape uses it: its grids fit the resident slots at once, while
// the 256-query shape's larger grids refill slots as blocks finish (there
// the reordering measured 85.0 -> 87.2 us on C4).
__device__ __forceinline__ void fa7_block_of(int64_t lid, int bh, int nqb, bool snake, int& head, int& qblk) {
  if (!snake) {  // plain heavy-first order, head fastest
    head = int(lid % bh);
    qblk = nqb - 1 - int(lid / bh);
    return;
  }
  const int64_t total = int64_t(bh) * nqb;
  constexpr int kXcd = 8, kCusPerXcd = 32;
  const bool split = total % kXcd == 0;
  const int64_t xcd = split ? lid % kXcd : 0;
  const int64_t j = split ? lid / kXcd : lid;
  const int64_t per = split ? total / kXcd : total;
  const int64_t round = j / kCusPerXcd, pos = j % kCusPerXcd;
  const bool flip = (round & 1) && (round + 1) * kCusPerXcd <= per;
  const int64_t jj = round * kCusPerXcd + (flip ? kCusPerXcd - 1 - pos : pos);
  const int64_t g = split ? jj * kXcd + xcd : jj;
  head = int(g % bh);
  qblk = nqb - 1 - int(g / bh);
}

// NW wavefronts x 32 queries per workgroup, a RING-slot LDS ring of 64-key
// K and V tiles.  <8, 4>: two workgroups per CU, four wavefronts per SIMD
// (the long-sequence shape).  <4, 3>: 128-query workgroups, three per CU
// (48 KB of LDS each), for grids too small to fill the CUs evenly with
// 256-query blocks (a causal S = 1024 head has 4 such blocks of 4, 8, 12 and
// 16 tiles; 8 blocks of 128 queries fill three workgroup slots per CU).
//
// ROUND_S follows the reference's AMP rounding of the scores
// (_realize.py:395-412: the f16 matmul's output is stored in f16, then
// scaled in f32): Q is used as stored, the S accumulators start from zero,
// and each score is rounded to the input dtype before it is scaled and
// shifted by the reference max (one FMA per score; the default form folds
// the scale into Q and the shift into the MFMA's accumulator seed instead).
template <bool BF16, bool CAUSAL, int NW, int RING, bool ROUND_S>
__global__ void __launch_bounds__(NW * 64, NW == 8 ? 4 : 3)  // the LDS-bound occupancy
fa7_fwd_kernel(Fa2Args P, uint32_t k_bytes, uint32_t v_bytes) {
  static_assert((NW == 8 && RING == 4) || (NW == 4 && RING == 3), "instantiated shapes");
  constexpr int BQ = NW * kFa2QW;       // queries per workgroup
  constexpr int PARTS = 8 / NW;         // 1 KB slices of each tile per wavefront
  constexpr int DMA = 2 * PARTS;        // copies per wavefront per tile (K and V)
  __shared__ fa_u4 smem[2 * RING * kFa2Tile / 16];
  char* sb = reinterpret_cast<char*>(smem);
  char* kring = sb;
  char* vring = sb + RING * kFa2Tile;

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hi = lane >> 5;
  int bh, qblk;
  fa7_block_of(int64_t(blockIdx.y) * gridDim.x + blockIdx.x, int(gridDim.x), P.n_qblocks, NW == 4, bh, qblk);
  const int b = bh / P.H, h = bh % P.H;
  const int q0 = qblk * BQ;
  const int q0w = q0 + w * kFa2QW;
  const int qi = q0w + (lane & 31);

  const uint16_t* Qp = P.q + b * P.q_sb + h * P.q_sh;
  const uint16_t* Kp = P.k + b * P.k_sb + h * P.k_sh;
  const uint16_t* Vp = P.v + b * P.v_sb + h * P.v_sh;
  const bgk::sgpr4_t rk = bgk::buffer_rsrc(Kp, k_bytes);
  const bgk::sgpr4_t rv = bgk::buffer_rsrc(Vp, v_bytes);

  const int nt_all = (P.Sk + kFa2BK - 1) / kFa2BK;
  const int nt = CAUSAL ? min(nt_all, (q0 + BQ + kFa2BK - 1) / kFa2BK) : nt_all;
  const int ntw = CAUSAL ? min(nt, (q0w + kFa2QW + kFa2BK - 1) / kFa2BK) : nt;
  // Tiles with no masked key for any query of the workgroup.
  const int t_clean = min(nt, CAUSAL ? min(P.Sk / kFa2BK, (q0 + 1) / kFa2BK) : P.Sk / kFa2BK);

  // Wavefront w copies the 1 KB slices w, w + NW, ... (rows 8 s .. 8 s + 7)
  // of each K and V tile; lane L writes 16-byte unit 64 s + L = (row, chunk).
  uint32_t koff[PARTS], voff[PARTS];
  int krow[PARTS];
#pragma unroll
  for (int p = 0; p < PARTS; ++p) {
    const int u = (w + p * NW) * 64 + lane;
    const int pc = u & 7;
    krow[p] = u >> 3;
    // 16-byte chunks past the head dim read zeros (an offset past the buffer).
    const int kc = pc ^ ((krow[p] >> 1) & 7), vc = pc ^ ((krow[p] & 3) << 1);
    koff[p] = kc * 8 < P.D ? uint32_t((int64_t(krow[p]) * P.k_ss + kc * 8) * 2) : kFa2Oob;
    voff[p] = vc * 8 < P.D ? uint32_t((int64_t(krow[p]) * P.v_ss + vc * 8) * 2) : kFa2Oob;
  }
  const uint32_t kstep = uint32_t(int64_t(kFa2BK) * P.k_ss * 2);
  const uint32_t vstep = uint32_t(int64_t(kFa2BK) * P.v_ss * 2);
  const uint32_t kl = bgk::lds_addr(kring) + uint32_t(w) * 1024u;
  const uint32_t vl = bgk::lds_addr(vring) + uint32_t(w) * 1024u;
  auto issue = [&](int j) {
    const bool real = j >= 0 && j < nt;
    const uint32_t sl = uint32_t(j % RING) * kFa2Tile;
#pragma unroll
    for (int p = 0; p < PARTS; ++p) {
      const bool ok = real && j * kFa2BK + krow[p] < P.Sk;
      const uint32_t at = sl + uint32_t(p * NW) * 1024u;
      bgk::dma16_to_lds(kl + at, ok ? koff[p] : kFa2Oob, rk, real ? uint32_t(j) * kstep : 0u);
      bgk::dma16_to_lds(vl + at, ok ? voff[p] : kFa2Oob, rv, real ? uint32_t(j) * vstep : 0u);
    }
  };

  const float sl2 = P.sl2;
  fa_u4 qf[4];
#pragma unroll
  for (int dc = 0; dc < 4; ++dc)
    qf[dc] = qi < P.Sq && dc * 16 + hi * 8 < P.D
                 ? *reinterpret_cast<const fa_u4*>(Qp + int64_t(qi) * P.q_ss + dc * 16 + hi * 8)
                 : fa_u4{0u, 0u, 0u, 0u};
  // PAIRS (the 4-slot ring): tiles are awaited and refilled two at a time,
  // one barrier per two tiles: at an even step t the wavefronts wait for
  // tiles t and t+1, pass the barrier and copy tiles t+2 and t+3 into the
  // slots of t-2 and t-1, so each copy has two tiles of compute to land.
  constexpr bool PAIRS = RING == 4;
  if constexpr (PAIRS) {
    issue(0);
    issue(1);
  } else {
#pragma unroll
    for (int j = 0; j < RING - 1; ++j) issue(j);
  }
  fa2_wait_vm_lgkm0<0>();  // also retires the Q loads in the compiler's bookkeeping
  __builtin_amdgcn_s_barrier();
  if constexpr (PAIRS) {
    issue(2);
    issue(3);
  }
  if constexpr (!ROUND_S) {
#pragma unroll
    for (int dc = 0; dc < 4; ++dc)
#pragma unroll
      for (int i = 0; i < 4; ++i) qf[dc][i] = fa6_scale2<BF16>(qf[dc][i], sl2);
  }

  const Fa6Offs offs;
  float16v zero;
#pragma unroll
  for (int e = 0; e < 16; ++e) zero[e] = 0.f;
  // Reference max: exact maximum over this query's keys 0..31 (key 0 is
  // always visible), the same for the wavefront's two lanes of a query.
  // Default form: -m seeds the S accumulators (mneg).  ROUND_S: the scores
  // start from zero and negm is added by the per-score FMA.
  float16v mneg;
  float negm;
  {
    float16v x = fa6_scores_half<BF16>(kring, offs, qf, zero, 0);
    float mt = -INFINITY;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int kj = 8 * (e >> 2) + 4 * hi + (e & 3);
      const float xe = ROUND_S ? fa7_round<BF16>(x[e]) * sl2 : x[e];
      if (!(kj >= P.Sk || (CAUSAL && kj > qi))) mt = fmaxf(mt, xe);
    }
    mt = fmaxf(mt, fa2_xor32(mt));
    const float m_use = mt == -INFINITY ? 0.f : mt;
    negm = -m_use;
#pragma unroll
    for (int e = 0; e < 16; ++e) mneg[e] = ROUND_S ? 0.f : -m_use;
  }

  float16v acc[2];
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[db][e] = 0.f;
  float l_run = 0.f;

  int t = 0;
  for (; t < t_clean; ++t) {
    if constexpr (PAIRS) {
      if (t > 0 && (t & 1) == 0) {
        fa2_wait_vm_lgkm0<0>();  // tiles t, t+1 landed
        __builtin_amdgcn_s_barrier();
        issue(t + 2);  // into the slots of tiles t-2, t-1, which every wavefront has left
        issue(t + 3);
      }
    } else {
      if (t > 0) {
        fa2_wait_vm_lgkm0<(RING - 2) * DMA>();  // tile t landed; t+1 .. t+RING-2 may be in flight
        __builtin_amdgcn_s_barrier();
      }
      issue(t + RING - 1);  // into the slot of tile t-1, which every wavefront has left
    }
    const char* kt = kring + (t % RING) * kFa2Tile;
    const char* vt = vring + (t % RING) * kFa2Tile;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const float16v x = fa6_scores_half<BF16>(kt, offs, qf, mneg, hh);
      fa_u4 pf[2];
      if constexpr (ROUND_S) l_run += fa7_exp_round<BF16>(x, sl2, negm, pf);
      else l_run += fa6_exp<BF16, false>(x, 0.f, pf);
      fa6_pv_half<BF16>(vt, offs, pf, acc, hh);
    }
  }
  for (; t < nt; ++t) {
    if constexpr (PAIRS) {
      if (t > 0 && (t & 1) == 0) {
        fa2_wait_vm_lgkm0<0>();
        __builtin_amdgcn_s_barrier();
        issue(t + 2);
        issue(t + 3);
      }
    } else {
      if (t > 0) {
        fa2_wait_vm_lgkm0<(RING - 2) * DMA>();
        __builtin_amdgcn_s_barrier();
      }
      issue(t + RING - 1);
    }
    const char* kt = kring + (t % RING) * kFa2Tile;
    const char* vt = vring + (t % RING) * kFa2Tile;
    if (t < ntw) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        // j0 and q0w are multiples of 32: a half with j0 > q0w lies after
        // every query of the wavefront and adds nothing; j0 == q0w is the
        // diagonal half, j0 < q0w a fully visible one.
        const int j0 = t * kFa2BK + hh * 32;
        if (CAUSAL && j0 > q0w) break;
        float16v x = fa6_scores_half<BF16>(kt, offs, qf, mneg, hh);
        if ((CAUSAL && j0 + 31 > q0w) || (j0 + 32 > P.Sk)) {
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int kj = j0 + 8 * (e >> 2) + 4 * hi + (e & 3);
            if (kj >= P.Sk || (CAUSAL && kj > qi)) x[e] = -INFINITY;
          }
        }
        fa_u4 pf[2];
        if constexpr (ROUND_S) l_run += fa7_exp_round<BF16>(x, sl2, negm, pf);
        else l_run += fa6_exp<BF16, false>(x, 0.f, pf);
        fa6_pv_half<BF16>(vt, offs, pf, acc, hh);
      }
    }
  }
  fa2_wait_vm_lgkm0<0>();

  // A P that rounded to infinity shows as a non-finite l or O.
  bool bad = !(fabsf(l_run) <= 3.0e38f);
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int e = 0; e < 16; ++e) bad |= !(fabsf(acc[db][e]) <= 3.0e38f);
  if (__any(bad)) {
    fa7_exact<BF16, CAUSAL, ROUND_S>(P, b, h, q0w);
    return;
  }
  fa7_store(P, b, h, qi, acc, l_run);
}

// ---- v8: fa7's ring and schedule on 16x16x32 MFMAs ------------------------------
//
// The same workgroup shapes, LDS ring, copies, barriers, reference-max rule
// and exact recompute pass as fa7, with every product on
// v_mfma_f32_16x16x32_{f16,bf16} instead of 32x32x16 (the 16x16 form
// sustains more of the matrix core's nominal rate on random data than the
// 32x32 form in this library's register-only measurements).  Per 32-key half
// and wavefront (32 queries): S^T is 2 key blocks x 2 query blocks of 16x16,
// two MFMAs each over d; O^T += V^T P^T is 4 d blocks x 2 query blocks, one
// MFMA each over the half's 32 keys.
//   * S^T accumulator layout: lane l holds rows (keys) 4 (l / 16) + i of its
//     16-key block for query l % 16 of its query block.  So a lane's 8 P
//     values of one query block (keys 4g + i and 16 + 4g + i, g = l / 16)
//     are, packed, the B operand of the PV MFMA when its k-slot 8g + j means
//     key 4g + j (j < 4) or 16 + 4g + j - 4; the V^T operand takes the same
//     keys, read by two ds_read_b64_tr_b16 per d block (rows 4g .. 4g + 3 and
//     16 + 4g .. 16 + 4g + 3 of the half).  P never leaves the registers.
//   * K operand: one ds_read_b128 per (key block, d half): row 16 kb + l % 16,
//     16-byte chunk 4 dc + l / 16.  K keeps fa7's layout (chunk c of row r at
//     c ^ ((r >> 1) & 7)): the 16 rows one read cycle serves land on 16
//     distinct 4-bank groups.
//   * V rows store 32-byte block b at b ^ ((r >> 1) & 3) (chunk c at
//     c ^ (((r >> 1) & 3) << 1)): a transpose read cycle serves two 16-lane
//     groups, 8 rows at one 32-byte column block, and rows of one parity then
//     take four distinct blocks (conflict-free).
//   * The reference max is per query: the max over its first 32 keys, which
//     four lanes (l % 16 equal) hold between them; the row sum l is kept per
//     lane and query block and summed over those four lanes at the end.
typedef float fa_f4 __attribute__((ext_vector_type(4)));

template <bool BF16>
__device__ __forceinline__ fa_f4 fa8_mfma(fa_u4 a, fa_u4 b, fa_f4 c) {
  if constexpr (BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf168, a), __builtin_bit_cast(bf168, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c,
                                                  0, 0, 0);
}

// Value of the lanes 16 and 32 apart combined by max / sum: the four lanes
// with one l % 16 hold one query between them.
__device__ __forceinline__ float fa8_max4(float x) {
  x = fmaxf(x, __shfl_xor(x, 16, 64));
  return fmaxf(x, __shfl_xor(x, 32, 64));
}
__device__ __forceinline__ float fa8_sum4(float x) {
  x = x + __shfl_xor(x, 16, 64);
  return x + __shfl_xor(x, 32, 64);
}

// Per-lane LDS byte offsets of the fragment reads within a tile (the key
// block, the half and the transpose read's second row set only add
// multiples of 2048 bytes, since rows 16 apart share both swizzles).
struct Fa8Offs {
  uint32_t k[2];  // d half dc: row l % 16, chunk 4 dc + l / 16
  uint32_t v[4];  // d block db: row 4 (l / 16) + (l % 16) / 4, d = 16 db + 4 (l % 4)
  __device__ __forceinline__ Fa8Offs() {
    const int lane = threadIdx.x & 63, g = lane >> 4, w = lane & 15;
#pragma unroll
    for (int dc = 0; dc < 2; ++dc) k[dc] = uint32_t(fa2_k_unit(w, 4 * dc + g) * 16);
    const int r = 4 * g + (w >> 2);
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const int c = 2 * db + ((w & 3) >> 1);
      const int pc = c ^ (((r >> 1) & 3) << 1);
      v[db] = uint32_t(r * 128 + pc * 16 + 8 * (w & 1));
    }
  }
};

template <bool BF16>
__device__ __forceinline__ void fa8_scores_half(const char* kt, const Fa8Offs& o, const fa_u4 (&qf)[2][2],
                                                const fa_f4 (&seed)[2], int h, fa_f4 (&s)[2][2]) {
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    fa_u4 kf[2];
#pragma unroll
    for (int dc = 0; dc < 2; ++dc)
      kf[dc] = *reinterpret_cast<const fa_u4*>(kt + o.k[dc] + h * 4096 + kb * 2048);
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      s[kb][qb] = fa8_mfma<BF16>(kf[0], qf[qb][0], seed[qb]);
      s[kb][qb] = fa8_mfma<BF16>(kf[1], qf[qb][1], s[kb][qb]);
    }
  }
}

template <bool BF16>
__device__ __forceinline__ void fa8_pv_half(const char* vt, const Fa8Offs& o, const fa_u4 (&pf)[2], fa_f4 (&acc)[4][2],
                                            int h) {
#pragma unroll
  for (int db = 0; db < 4; ++db) {
    fa_v4s part[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const char* addr = vt + o.v[db] + h * 4096 + r * 2048;
      part[r] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) fa_v4s*)(reinterpret_cast<uintptr_t>(addr)));
    }
    const fa_u4 vf = __builtin_bit_cast(fa_u4, __builtin_shufflevector(part[0], part[1], 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) acc[db][qb] = fa8_mfma<BF16>(vf, pf[qb], acc[db][qb]);
  }
}

// P of one query block: exp2 of the 8 scores (key blocks 0 and 1), packed
// as the PV B operand; returns their f32 sum.  ROUND_S: the scores are raw
// S, rounded to the input dtype, then scaled and shifted (negm).
template <bool BF16, bool ROUND_S>
__device__ __forceinline__ float fa8_exp(const fa_f4& x0, const fa_f4& x1, float sl2, float negm, fa_u4& pf) {
  float e[8];
#pragma unroll
  for (int i = 0; i < 4; i += 2) {
    if constexpr (ROUND_S) {
      const uint32_t a = fa2_pack<BF16>(x0[i], x0[i + 1]), b = fa2_pack<BF16>(x1[i], x1[i + 1]);
      e[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(fa2_lo<BF16>(a), sl2, negm));
      e[i + 1] = __builtin_amdgcn_exp2f(__builtin_fmaf(fa2_hi<BF16>(a), sl2, negm));
      e[4 + i] = __builtin_amdgcn_exp2f(__builtin_fmaf(fa2_lo<BF16>(b), sl2, negm));
      e[5 + i] = __builtin_amdgcn_exp2f(__builtin_fmaf(fa2_hi<BF16>(b), sl2, negm));
    } else {
      e[i] = __builtin_amdgcn_exp2f(x0[i]);
      e[i + 1] = __builtin_amdgcn_exp2f(x0[i + 1]);
      e[4 + i] = __builtin_amdgcn_exp2f(x1[i]);
      e[5 + i] = __builtin_amdgcn_exp2f(x1[i + 1]);
    }
  }
  pf = fa_u4{fa2_pack<BF16>(e[0], e[1]), fa2_pack<BF16>(e[2], e[3]), fa2_pack<BF16>(e[4], e[5]),
             fa2_pack<BF16>(e[6], e[7])};
  return ((e[0] + e[1]) + (e[2] + e[3])) + ((e[4] + e[5]) + (e[6] + e[7]));
}

// O = acc / l; acc[db][qb] lane l holds O^T[d = 16 db + 4 (l / 16) + i][q = 16 qb + l % 16].
__device__ __forceinline__ void fa8_store(const Fa2Args& P, int b, int h, int q0w, const fa_f4 (&acc)[4][2],
                                          const float (&l_run)[2]) {
  const int lane = threadIdx.x & 63, g = lane >> 4;
  char* Ob = static_cast<char*>(P.o);
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const float lt = fa8_sum4(l_run[qb]);
    const float inv = lt > 0.f ? 1.0f / lt : 0.f;
    const int qi = q0w + 16 * qb + (lane & 15);
    if (qi >= P.Sq) continue;
    const int64_t obase = int64_t(b) * P.o_sb + int64_t(h) * P.o_sh + int64_t(qi) * P.o_ss;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const int d0 = 16 * db + 4 * g;
      if (d0 >= P.D) continue;
      const float y0 = acc[db][qb][0] * inv, y1 = acc[db][qb][1] * inv;
      const float y2 = acc[db][qb][2] * inv, y3 = acc[db][qb][3] * inv;
      if (P.out_dtype == 0)
        *reinterpret_cast<float4*>(Ob + (obase + d0) * 4) = make_float4(y0, y1, y2, y3);
      else if (P.out_dtype == 1)
        *reinterpret_cast<uint2*>(Ob + (obase + d0) * 2) =
            make_uint2(fa2_pack<false>(y0, y1), fa2_pack<false>(y2, y3));
      else
        *reinterpret_cast<uint2*>(Ob + (obase + d0) * 2) =
            make_uint2(fa2_pack<true>(y0, y1), fa2_pack<true>(y2, y3));
    }
  }
}

template <bool BF16, bool CAUSAL, int NW, int RING, bool ROUND_S>
__global__ void __launch_bounds__(NW * 64, NW == 8 ? 4 : 3)  // the LDS-bound occupancy
fa8_fwd_kernel(Fa2Args P, uint32_t k_bytes, uint32_t v_bytes) {
  static_assert(NW == 8 && RING == 4, "v8 is built for the 256-query shape only");
  constexpr int BQ = NW * kFa2QW;
  constexpr int PARTS = 8 / NW;
  constexpr int DMA = 2 * PARTS;
  __shared__ fa_u4 smem[2 * RING * kFa2Tile / 16];
  char* sb = reinterpret_cast<char*>(smem);
  char* kring = sb;
  char* vring = sb + RING * kFa2Tile;

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4;
  int bh, qblk;
  fa7_block_of(int64_t(blockIdx.y) * gridDim.x + blockIdx.x, int(gridDim.x), P.n_qblocks, NW == 4, bh, qblk);
  const int b = bh / P.H, h = bh % P.H;
  const int q0 = qblk * BQ;
  const int q0w = q0 + w * kFa2QW;

  const uint16_t* Qp = P.q + b * P.q_sb + h * P.q_sh;
  const uint16_t* Kp = P.k + b * P.k_sb + h * P.k_sh;
  const uint16_t* Vp = P.v + b * P.v_sb + h * P.v_sh;
  const bgk::sgpr4_t rk = bgk::buffer_rsrc(Kp, k_bytes);
  const bgk::sgpr4_t rv = bgk::buffer_rsrc(Vp, v_bytes);

  const int nt_all = (P.Sk + kFa2BK - 1) / kFa2BK;
  const int nt = CAUSAL ? min(nt_all, (q0 + BQ + kFa2BK - 1) / kFa2BK) : nt_all;
  const int ntw = CAUSAL ? min(nt, (q0w + kFa2QW + kFa2BK - 1) / kFa2BK) : nt;
  const int t_clean = min(nt, CAUSAL ? min(P.Sk / kFa2BK, (q0 + 1) / kFa2BK) : P.Sk / kFa2BK);

  // Copies as fa7's, with V's 32-byte-block swizzle.
  uint32_t koff[PARTS], voff[PARTS];
  int krow[PARTS];
#pragma unroll
  for (int p = 0; p < PARTS; ++p) {
    const int u = (w + p * NW) * 64 + lane;
    const int pc = u & 7;
    krow[p] = u >> 3;
    const int kc = pc ^ ((krow[p] >> 1) & 7), vc = pc ^ (((krow[p] >> 1) & 3) << 1);
    koff[p] = kc * 8 < P.D ? uint32_t((int64_t(krow[p]) * P.k_ss + kc * 8) * 2) : kFa2Oob;
    voff[p] = vc * 8 < P.D ? uint32_t((int64_t(krow[p]) * P.v_ss + vc * 8) * 2) : kFa2Oob;
  }
  const uint32_t kstep = uint32_t(int64_t(kFa2BK) * P.k_ss * 2);
  const uint32_t vstep = uint32_t(int64_t(kFa2BK) * P.v_ss * 2);
  const uint32_t kl = bgk::lds_addr(kring) + uint32_t(w) * 1024u;
  const uint32_t vl = bgk::lds_addr(vring) + uint32_t(w) * 1024u;
  auto issue = [&](int j) {
    const bool real = j >= 0 && j < nt;
    const uint32_t sl = uint32_t(j % RING) * kFa2Tile;
#pragma unroll
    for (int p = 0; p < PARTS; ++p) {
      const bool ok = real && j * kFa2BK + krow[p] < P.Sk;
      const uint32_t at = sl + uint32_t(p * NW) * 1024u;
      bgk::dma16_to_lds(kl + at, ok ? koff[p] : kFa2Oob, rk, real ? uint32_t(j) * kstep : 0u);
      bgk::dma16_to_lds(vl + at, ok ? voff[p] : kFa2Oob, rv, real ? uint32_t(j) * vstep : 0u);
    }
  };

  const float sl2 = P.sl2;
  // Q operand: qf[qb][dc] = Q[q0w + 16 qb + l % 16][32 dc + 8 (l / 16) .. + 7].
  fa_u4 qf[2][2];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int dc = 0; dc < 2; ++dc) {
      const int qi = q0w + 16 * qb + (lane & 15);
      const int d0 = 32 * dc + 8 * g;
      qf[qb][dc] = qi < P.Sq && d0 < P.D ? *reinterpret_cast<const fa_u4*>(Qp + int64_t(qi) * P.q_ss + d0)
                                         : fa_u4{0u, 0u, 0u, 0u};
    }
  constexpr bool PAIRS = RING == 4;
  if constexpr (PAIRS) {
    issue(0);
    issue(1);
  } else {
#pragma unroll
    for (int j = 0; j < RING - 1; ++j) issue(j);
  }
  fa2_wait_vm_lgkm0<0>();
  __builtin_amdgcn_s_barrier();
  if constexpr (PAIRS) {
    issue(2);
    issue(3);
  }
  if constexpr (!ROUND_S) {
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int dc = 0; dc < 2; ++dc)
#pragma unroll
        for (int i = 0; i < 4; ++i) qf[qb][dc][i] = fa6_scale2<BF16>(qf[qb][dc][i], sl2);
  }

  const Fa8Offs offs;
  // Reference max per query block: the exact maximum over keys 0..31 (key 0
  // is always visible), combined over the four lanes of the query.
  fa_f4 seed[2];
  float negm[2];
  {
    fa_f4 zero[2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) zero[qb] = fa_f4{0.f, 0.f, 0.f, 0.f};
    fa_f4 x[2][2];
    fa8_scores_half<BF16>(kring, offs, qf, zero, 0, x);
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      const int qi = q0w + 16 * qb + (lane & 15);
      float mt = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int kj = 16 * kb + 4 * g + i;
          const float xe = ROUND_S ? fa7_round<BF16>(x[kb][qb][i]) * sl2 : x[kb][qb][i];
          if (!(kj >= P.Sk || (CAUSAL && kj > qi))) mt = fmaxf(mt, xe);
        }
      mt = fa8_max4(mt);
      const float m_use = mt == -INFINITY ? 0.f : mt;
      negm[qb] = -m_use;
      const float sv = ROUND_S ? 0.f : -m_use;
      seed[qb] = fa_f4{sv, sv, sv, sv};
    }
  }

  fa_f4 acc[4][2];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) acc[db][qb] = fa_f4{0.f, 0.f, 0.f, 0.f};
  float l_run[2] = {0.f, 0.f};

  int t = 0;
  for (; t < t_clean; ++t) {
    if constexpr (PAIRS) {
      if (t > 0 && (t & 1) == 0) {
        fa2_wait_vm_lgkm0<0>();
        __builtin_amdgcn_s_barrier();
        issue(t + 2);
        issue(t + 3);
      }
    } else {
      if (t > 0) {
        fa2_wait_vm_lgkm0<(RING - 2) * DMA>();
        __builtin_amdgcn_s_barrier();
      }
      issue(t + RING - 1);
    }
    const char* kt = kring + (t % RING) * kFa2Tile;
    const char* vt = vring + (t % RING) * kFa2Tile;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      fa_f4 x[2][2];
      fa8_scores_half<BF16>(kt, offs, qf, seed, hh, x);
      fa_u4 pf[2];
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) l_run[qb] += fa8_exp<BF16, ROUND_S>(x[0][qb], x[1][qb], sl2, negm[qb], pf[qb]);
      fa8_pv_half<BF16>(vt, offs, pf, acc, hh);
    }
  }
  for (; t < nt; ++t) {
    if constexpr (PAIRS) {
      if (t > 0 && (t & 1) == 0) {
        fa2_wait_vm_lgkm0<0>();
        __builtin_amdgcn_s_barrier();
        issue(t + 2);
        issue(t + 3);
      }
    } else {
      if (t > 0) {
        fa2_wait_vm_lgkm0<(RING - 2) * DMA>();
        __builtin_amdgcn_s_barrier();
      }
      issue(t + RING - 1);
    }
    const char* kt = kring + (t % RING) * kFa2Tile;
    const char* vt = vring + (t % RING) * kFa2Tile;
    if (t < ntw) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int j0 = t * kFa2BK + hh * 32;
        if (CAUSAL && j0 > q0w) break;
        fa_f4 x[2][2];
        fa8_scores_half<BF16>(kt, offs, qf, seed, hh, x);
        if ((CAUSAL && j0 + 31 > q0w) || (j0 + 32 > P.Sk)) {
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int qb = 0; qb < 2; ++qb)
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                const int kj = j0 + 16 * kb + 4 * g + i;
                const int qi = q0w + 16 * qb + (lane & 15);
                if (kj >= P.Sk || (CAUSAL && kj > qi)) x[kb][qb][i] = -INFINITY;
              }
        }
        fa_u4 pf[2];
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
          l_run[qb] += fa8_exp<BF16, ROUND_S>(x[0][qb], x[1][qb], sl2, negm[qb], pf[qb]);
        fa8_pv_half<BF16>(vt, offs, pf, acc, hh);
      }
    }
  }
  fa2_wait_vm_lgkm0<0>();

  bool bad = !(fabsf(l_run[0]) <= 3.0e38f) || !(fabsf(l_run[1]) <= 3.0e38f);
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int i = 0; i < 4; ++i) bad |= !(fabsf(acc[db][qb][i]) <= 3.0e38f);
  if (__any(bad)) {
    fa7_exact<BF16, CAUSAL, ROUND_S>(P, b, h, q0w);
    return;
  }
  fa8_store(P, b, h, q0w, acc, l_run);
}

// The 256-query shape runs v8 (measured against v7 on one box, C4: 87.3 /
// 88.1 us against 90.8 / 90.5; with the score rounding 96.1 / 96.2 against
// 99.6 / 99.0); the 128-query shape runs v7, which was faster there (C5
// attention 26.0 / 26.2 us against 27.4 / 27.8 for v8's 128-query form,
// which is therefore not built).  BG_ATTN_KERNEL=7 runs v7 for both.
template <bool BF16, bool CAUSAL, bool ROUND_S>
void launch_fa8(bg_ctx* ctx, const Fa2Args& A0, int bh, uint32_t kb, uint32_t vb) {
  Fa2Args A = A0;
  const int64_t big = int64_t(bh) * ((A.Sq + 255) / 256);
  const char* force = std::getenv("BG_FA7_BLOCK");
  const bool want256 = force && std::strcmp(force, "256") == 0;
  const bool want128 = force && std::strcmp(force, "128") == 0;
  if (want256 || (!want128 && big >= 768) || (A.Sq + 127) / 128 > 65535) {
    A.n_qblocks = (A.Sq + 255) / 256;
    bg::dispatch(ctx, fa8_fwd_kernel<BF16, CAUSAL, 8, 4, ROUND_S>, dim3(unsigned(bh), unsigned(A.n_qblocks), 1),
                 dim3(8 * 64), 0, A, kb, vb);
  } else {
    A.n_qblocks = (A.Sq + 127) / 128;
    bg::dispatch(ctx, fa7_fwd_kernel<BF16, CAUSAL, 4, 3, ROUND_S>, dim3(unsigned(bh), unsigned(A.n_qblocks), 1),
                 dim3(4 * 64), 0, A, kb, vb);
  }
}

// 256-query workgroups when they give at least three per CU's two slots
// (C4: 128 heads x 8 blocks); 128-query workgroups otherwise (C5: 96 heads
// x 4 blocks of 256 would leave a 2:1 imbalance between CUs).
template <bool BF16, bool CAUSAL, bool ROUND_S>
void launch_fa7(bg_ctx* ctx, const Fa2Args& A0, int bh, uint32_t kb, uint32_t vb) {
  Fa2Args A = A0;
  const int64_t big = int64_t(bh) * ((A.Sq + 255) / 256);
  // Diagnostic override for tests and sweeps: BG_FA7_BLOCK=256 or 128.
  const char* force = std::getenv("BG_FA7_BLOCK");
  const bool want256 = force && std::strcmp(force, "256") == 0;
  const bool want128 = force && std::strcmp(force, "128") == 0;
  if (want256 || (!want128 && big >= 768) || (A.Sq + 127) / 128 > 65535) {
    A.n_qblocks = (A.Sq + 255) / 256;
    bg::dispatch(ctx, fa7_fwd_kernel<BF16, CAUSAL, 8, 4, ROUND_S>, dim3(unsigned(bh), unsigned(A.n_qblocks), 1),
                 dim3(8 * 64), 0, A, kb, vb);
  } else {
    A.n_qblocks = (A.Sq + 127) / 128;
    bg::dispatch(ctx, fa7_fwd_kernel<BF16, CAUSAL, 4, 3, ROUND_S>, dim3(unsigned(bh), unsigned(A.n_qblocks), 1),
                 dim3(4 * 64), 0, A, kb, vb);
  }
}

template <bool BF16, bool CAUSAL>
void launch_fa6(bg_ctx* ctx, const Fa2Args& A, int bh, int nqb, uint32_t kb, uint32_t vb) {
  bg::dispatch(ctx, fa6_fwd_kernel<BF16, CAUSAL>, dim3(unsigned(bh), unsigned(nqb), 1),
               dim3(kFa2NW * 64), 0, A, kb, vb);
}

// BG_ATTN_KERNEL=2 / 6 / 7 selects the v2 / v6 / v7 kernel for every call,
// for comparisons (default: v8 for 256-query workgroups, v7 for 128).
// Independently of it, v6 runs only where its numerics hold: S is not
// rounded (round_scores == 0; v2 rounds S exactly), and Q' = Q * scale *
// log2(e) cannot overflow f16 (scale * log2(e) <= 1, so |Q'| <= |Q|).
int attn_version() {
  static const int v = [] {
    const char* e = std::getenv("BG_ATTN_KERNEL");
    if (e && e[0] == '2') return 2;
    if (e && e[0] == '6') return 6;
    if (e && e[0] == '7') return 7;
    return 8;  // v8 for 256-query workgroups, v7 for 128-query ones
  }();
  return v;
}

template <bool BF16, bool CAUSAL, bool ROUND_S>
void launch_fa2(bg_ctx* ctx, const Fa2Args& A, int bh, int nqb, uint32_t kb, uint32_t vb) {
  dim3 grid(unsigned(bh), unsigned(nqb), 1);
  bg::dispatch(ctx, fa2_fwd_kernel<BF16, CAUSAL, ROUND_S>, grid, dim3(kFa2NW * 64), 0, A, kb, vb);
}

}  // namespace

namespace bg {

void launch_attention(bg_ctx* ctx, const bg_attention_desc& d, const Record& q, const Record& k,
                      const Record& v, Record& out) {
  const int64_t es = dtype_size(d.in_dtype);
  const char* qp = q.ptr() + d.q_off * es;
  const char* kp = k.ptr() + d.k_off * es;
  const char* vp = v.ptr() + d.v_off * es;
  const int64_t sq = d.sq, sk = d.sk;
  const int64_t keys = d.causal ? 0 : d.batch * d.heads * sq * sk;
  int64_t pairs = keys;
  if (d.causal) {
    // Valid (q, k) pairs of the top-left-aligned causal mask (k <= q).
    for (int64_t i = 0; i < sq; ++i) pairs += std::min<int64_t>(i + 1, sk);
    pairs *= d.batch * d.heads;
  }
  const int64_t flops = 4 * pairs * d.d;
  const int64_t bytes = d.batch * d.heads * (sq * d.d + 2 * sk * d.d) * es +
                        d.batch * d.heads * sq * d.d * dtype_size(d.out_dtype);
  // Head dims below 64 (multiples of 8) run the fast kernel with the
  // missing 16-byte chunks read as zeros; the other kernels take 64 only.
  const bool d64 = d.d == 64;
  const bool mfma_ok = (d.in_dtype == BG_F16 || d.in_dtype == BG_BF16) && d.d % 8 == 0 && d.d <= 64 &&
                       d.q_ss % 8 == 0 && d.k_ss % 8 == 0 && d.v_ss % 4 == 0 && d.o_ss % 4 == 0 &&
                       d.q_sb % 8 == 0 && d.q_sh % 8 == 0 && d.k_sb % 8 == 0 && d.k_sh % 8 == 0 &&
                       d.v_sb % 4 == 0 && d.v_sh % 4 == 0 && d.o_sb % 4 == 0 && d.o_sh % 4 == 0 &&
                       al(qp, 16) && al(kp, 16) && al(vp, 8) && al(out.ptr(), 16) &&
                       d.batch * d.heads <= 0x7fffffff && sq <= (1 << 30) && sk <= (1 << 30);
  if (d.in_dtype == BG_F32 && fa32_supported(d)) {
    Profile prof(ctx, "attention_f32", bytes, flops);
    launch_fa32(ctx, d, reinterpret_cast<const float*>(qp), reinterpret_cast<const float*>(kp),
                reinterpret_cast<const float*>(vp), nullptr, 0, 0, 0, out.ptr());
    return;
  }
  const bool r = d.round_scores != 0;
  const float sl2 = d.scale * 1.4426950408889634f;
  const bool fa7_takes = r || d.in_dtype == BG_BF16 || sl2 <= 1.0f;  // Q * scale * log2 e stays in f16 range
  if (!mfma_ok || (!d64 && (attn_version() < 7 || !fa7_takes))) {
    Profile prof(ctx, "attention_generic", bytes, flops);
    launch_attention_generic(ctx, d, qp, kp, vp, nullptr, 0, 0, out.ptr(),
                             d.in_dtype != BG_F32);
    return;
  }
  // v2 kernel: K/V rows 16-byte aligned for the DMA, byte spans within a
  // 32-bit buffer offset, positive scale (the row max is taken before scaling).
  const int64_t k_span = ((d.batch - 1) * d.k_sb + (d.heads - 1) * d.k_sh + (sk - 1) * d.k_ss + d.d) * es;
  const int64_t v_span = ((d.batch - 1) * d.v_sb + (d.heads - 1) * d.v_sh + (sk - 1) * d.v_ss + d.d) * es;
  const int64_t k_head = ((sk - 1) * d.k_ss + d.d) * es, v_head = ((sk - 1) * d.v_ss + d.d) * es;
  const bool v2_ok = d.k_ss % 8 == 0 && d.v_ss % 8 == 0 && d.k_sb % 8 == 0 && d.k_sh % 8 == 0 &&
                     d.v_sb % 8 == 0 && d.v_sh % 8 == 0 && al(vp, 16) && d.scale > 0.f &&
                     k_span > 0 && v_span > 0 && k_head < (int64_t(1) << 31) &&
                     v_head < (int64_t(1) << 31) && (sq + kFa2BQ - 1) / kFa2BQ <= 65535;
  if (!d64 && !v2_ok) {
    Profile prof(ctx, "attention_generic", bytes, flops);
    launch_attention_generic(ctx, d, qp, kp, vp, nullptr, 0, 0, out.ptr(), true);
    return;
  }
  if (v2_ok) {
    Fa2Args A{};
    A.q = reinterpret_cast<const uint16_t*>(qp);
    A.k = reinterpret_cast<const uint16_t*>(kp);
    A.v = reinterpret_cast<const uint16_t*>(vp);
    A.o = out.ptr();
    A.q_sb = d.q_sb; A.q_sh = d.q_sh; A.q_ss = d.q_ss;
    A.k_sb = d.k_sb; A.k_sh = d.k_sh; A.k_ss = d.k_ss;
    A.v_sb = d.v_sb; A.v_sh = d.v_sh; A.v_ss = d.v_ss;
    A.o_sb = d.o_sb; A.o_sh = d.o_sh; A.o_ss = d.o_ss;
    A.H = int(d.heads);
    A.Sq = int(sq);
    A.Sk = int(sk);
    A.n_qblocks = int((sq + kFa2BQ - 1) / kFa2BQ);
    A.sl2 = sl2;
    A.out_dtype = d.out_dtype;
    A.D = int(d.d);
    const int bh = int(d.batch * d.heads);
    const bool bf = d.in_dtype == BG_BF16;
    const bool c = d.causal != 0;
    const uint32_t kb = uint32_t(k_head), vb = uint32_t(v_head);
    Profile prof(ctx, bf ? "attention_bf16" : "attention_f16", bytes, flops);
    const int ver = attn_version();
    // fa7 with the scale folded into Q needs |Q * scale * log2 e| <= |Q| for
    // f16 (no overflow); its ROUND_S form scales each rounded score instead.
    const bool fast = ver != 2 && fa7_takes;
#define BG_FA2(B_, C_, R_)                                                                     \
  (fast ? (ver == 6 && !R_ ? launch_fa6<B_, C_>(ctx, A, bh, A.n_qblocks, kb, vb)               \
           : ver == 7       ? launch_fa7<B_, C_, R_>(ctx, A, bh, kb, vb)                     \
                            : launch_fa8<B_, C_, R_>(ctx, A, bh, kb, vb))                    \
        : launch_fa2<B_, C_, R_>(ctx, A, bh, A.n_qblocks, kb, vb))
    if (bf) {
      if (c) { if (r) BG_FA2(true, true, true); else BG_FA2(true, true, false); }
      else { if (r) BG_FA2(true, false, true); else BG_FA2(true, false, false); }
    } else {
      if (c) { if (r) BG_FA2(false, true, true); else BG_FA2(false, true, false); }
      else { if (r) BG_FA2(false, false, true); else BG_FA2(false, false, false); }
    }
#undef BG_FA2
    return;
  }
  FaArgs A{};
  A.q = reinterpret_cast<const uint16_t*>(qp);
  A.k = reinterpret_cast<const uint16_t*>(kp);
  A.v = reinterpret_cast<const uint16_t*>(vp);
  A.o = out.ptr();
  A.q_sb = d.q_sb; A.q_sh = d.q_sh; A.q_ss = d.q_ss;
  A.k_sb = d.k_sb; A.k_sh = d.k_sh; A.k_ss = d.k_ss;
  A.v_sb = d.v_sb; A.v_sh = d.v_sh; A.v_ss = d.v_ss;
  A.o_sb = d.o_sb; A.o_sh = d.o_sh; A.o_ss = d.o_ss;
  A.H = int(d.heads);
  A.Sq = int(sq);
  A.Sk = int(sk);
  A.n_qblocks = int((sq + kBQ - 1) / kBQ);
  A.sl2 = d.scale * 1.4426950408889634f;
  A.out_dtype = d.out_dtype;
  if (A.n_qblocks > 65535) fail(BG_E_UNSUPPORTED, "flash_attention: sequence too long");
  const int bh = int(d.batch * d.heads);
  const bool bf = d.in_dtype == BG_BF16;
  const bool c = d.causal != 0;
  Profile prof(ctx, bf ? "attention_bf16" : "attention_f16", bytes, flops);
#define BG_FA(B_, C_, R_) launch_fa<B_, C_, R_>(ctx, A, bh, A.n_qblocks)
  if (bf) {
    if (c) { if (r) BG_FA(true, true, true); else BG_FA(true, true, false); }
    else { if (r) BG_FA(true, false, true); else BG_FA(true, false, false); }
  } else {
    if (c) { if (r) BG_FA(false, true, true); else BG_FA(false, true, false); }
    else { if (r) BG_FA(false, false, true); else BG_FA(false, false, false); }
  }
#undef BG_FA
  hip_check(hipGetLastError(), "attention launch");
}

}  // namespace bg
