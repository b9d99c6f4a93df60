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
  const bool mfma_ok = (d.in_dtype == BG_F16 || d.in_dtype == BG_BF16) && d.d == 64 &&
                       d.q_ss % 8 == 0 && d.k_ss % 8 == 0 && d.v_ss % 4 == 0 && d.o_ss % 4 == 0 &&
                       d.q_sb % 8 == 0 && d.q_sh % 8 == 0 && d.k_sb % 8 == 0 && d.k_sh % 8 == 0 &&
                       d.v_sb % 4 == 0 && d.v_sh % 4 == 0 && d.o_sb % 4 == 0 && d.o_sh % 4 == 0 &&
                       al(qp, 16) && al(kp, 16) && al(vp, 8) && al(out.ptr(), 16) &&
                       d.batch * d.heads <= 0x7fffffff && sq <= (1 << 30) && sk <= (1 << 30);
  if (!mfma_ok) {
    Profile prof(ctx, "attention_generic", bytes, flops);
    launch_attention_generic(ctx, d, qp, kp, vp, nullptr, 0, 0, out.ptr(),
                             d.in_dtype != BG_F32);
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
  const bool r = d.round_scores != 0;
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
