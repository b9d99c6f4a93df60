// Convolutions for gfx950 (f32): conv1d / conv2d / conv3d and the transposed
// conv2d, forward and backward (realizer.ts:325-720, 1153-1521;
// tensor_plan.ts:554-641, WGSL :1117-1999; CPU handlers _realize.py:413-1005).
//
// Every op is one of three implicit GEMMs over a 3-D description (1-D and
// 2-D convolutions have unit leading spatial dims), in the "conv picture"
// x [N][C][D][H][W] -> y [N][O][oD][oH][oW], weight [O][C/G][KD][KH][KW]:
//   FWD    y[n, g, o, p]  = sum_{c, kv} x[n, g, c, p*s + kv*dil - pad] * w[g, o, c, kv]
//          GEMM rows m = (n, p), columns o, reduction k = (c, kv)
//   DGRAD  dx[n, g, c, q] = sum_{o, kv} dy[n, g, o, (q + pad - kv*dil) / s] * w[g, o, c, kv]
//          (terms whose division is inexact or out of range vanish)
//          rows m = (n, q), columns c, reduction k = (o, kv)
//   WGRAD  dw[g, o, c, kv] = sum_{n, p} dy[n, g, o, p] * x[n, g, c, p*s + kv*dil - pad]
//          rows o, columns (c, kv), reduction k = (n, p), split along k
// The transposed convolution is DGRAD forward, FWD for its input gradient and
// WGRAD with x and dy exchanged for its weight gradient (the host maps it).
// Operands are gathered straight from the NCDHW tensors into LDS (no im2col
// buffer in HBM); out-of-range taps load 0, exactly as the reference's
// bounds-checked loops skip them.  The product runs on v_mfma_f32_32x32x2f32
// (full f32) in 64- or 128-wide workgroup tiles of four wavefronts.
#include <algorithm>
#include <cstdlib>
#include <type_traits>
#include <vector>

#include "common.cuh"
#include "core.h"

namespace {

using namespace bgk;

typedef float float16v __attribute__((ext_vector_type(16)));

// n / d for 0 <= n < 2^31: (n * m) >> (31 + s) with s = ceil(log2 d) and
// m = ceil(2^(31+s) / d) < 2^32; the product's error n*(m - 2^(31+s)/d) /
// 2^(31+s) stays below 1/d, so the floor is exact.
struct FDiv {
  uint32_t m;
  uint32_t s;
};

__device__ __forceinline__ uint32_t fdiv(uint32_t n, FDiv f) {
  return uint32_t((uint64_t(n) * f.m) >> (31 + f.s));
}

FDiv make_fdiv(uint32_t d) {
  uint32_t s = 0;
  while ((uint64_t(1) << s) < d) ++s;
  const uint64_t p = uint64_t(1) << (31 + s);
  return FDiv{uint32_t((p + d - 1) / d), s};
}

enum { MODE_FWD = 0, MODE_DGRAD = 1, MODE_WGRAD = 2 };

struct ConvK {
  const float* a;  // FWD: x; DGRAD: dy; WGRAD: dy
  const float* b;  // FWD: w; DGRAD: w; WGRAD: x
  const float* bias;
  float* out;      // y / dx / dw, or the WGRAD split-K workspace
  int C, O, Cpg, Opg;
  int D, H, W, oD, oH, oW;
  int S, oS;
  int KD, KH, KW, KV;
  int sd, sh, sw, pd, ph, pw, dd, dh, dw;
  int M, NC, K;  // per-group GEMM: rows, columns, reduction
  int tiles_m, ksplit, k_chunk;
  int b_kmajor;         // FWD ring kernel: b is w laid out [G][K][Opg]
  int om, om_sh, om_sw, om_ph, om_pw, om_H, om_W;  // FWD: outputs are one phase of an om_H x om_W plane
  int64_t part_stride;  // WGRAD: floats per split slice (G * Opg * NC)
  FDiv f_oS, f_oHW, f_oW, f_S, f_HW, f_W, f_KV, f_KHW, f_KW, f_sd, f_sh, f_sw;
};

constexpr int CBK = 16;  // k-step of every tile; WGRAD slices are multiples of it

// Epilogue shared by the conv GEMM kernels: bias, then the store of each
// wavefront's (BM/2) x (BN/2) block (WGRAD: into its split slice).
template <int MODE, int BM, int BN>
__device__ __forceinline__ void conv_epilogue(const ConvK& P, float16v (&acc)[BM / 64][BN / 64], int m0, int n0,
                                              int wm, int wn, int g, int split, int m_end) {
  constexpr int TM = BM / 64, TN = BN / 64;
  const int lane = threadIdx.x & 63;
  // Lane l holds rows 8*(e/4) + (e%4) + 4*(l/32) and column l%32 of each
  // 32 x 32 tile: groups of four consecutive rows, stored as one float4 when
  // they are contiguous and aligned in the output (spatial size % 4 == 0 and
  // the first row a multiple of 4).  Rows from m_end on are not stored.
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int col = n0 + wn * (BN / 2) + j * 32 + (lane & 31);
    if (col >= P.NC) continue;
    float bz = 0.f;
    if constexpr (MODE == MODE_FWD) {
      if (P.bias) bz = P.bias[int64_t(g) * P.Opg + col];
    } else if constexpr (MODE == MODE_DGRAD) {
      if (P.bias) bz = P.bias[int64_t(g) * P.Cpg + col];
    }
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int row = m0 + wm * (BM / 2) + i * 32 + 8 * q + 4 * (lane >> 5);
        if (row >= m_end) continue;
        if constexpr (MODE == MODE_WGRAD) {
          float* dst = P.out + int64_t(split) * P.part_stride + (int64_t(g) * P.Opg + row) * P.NC + col;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (row + e < m_end) dst[int64_t(e) * P.NC] = acc[i][j][4 * q + e];
        } else {
          const int spatial = MODE == MODE_FWD ? P.oS : P.S;
          const int chans = MODE == MODE_FWD ? P.O : P.C;
          const int cpg = MODE == MODE_FWD ? P.Opg : P.Cpg;
          if constexpr (MODE == MODE_FWD) {
            if (P.om) {
              // One phase of a larger 2-D output: output (oh, ow) goes to
              // (oh * om_sh + om_ph, ow * om_sw + om_pw).
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const int re = row + e;
                if (re >= m_end) break;
                const uint32_t ne = fdiv(uint32_t(re), P.f_oS);
                const uint32_t se = uint32_t(re) - ne * uint32_t(P.oS);
                const uint32_t oh = fdiv(se, P.f_oW), ow = se - oh * uint32_t(P.oW);
                P.out[(int64_t(ne) * chans + int64_t(g) * cpg + col) * (int64_t(P.om_H) * P.om_W) +
                      int64_t(oh * P.om_sh + P.om_ph) * P.om_W + ow * P.om_sw + P.om_pw] = acc[i][j][4 * q + e] + bz;
              }
              continue;
            }
          }
          const uint32_t n = fdiv(uint32_t(row), MODE == MODE_FWD ? P.f_oS : P.f_S);
          const uint32_t sp = uint32_t(row) - n * uint32_t(spatial);
          float* dst = P.out + (int64_t(n) * chans + int64_t(g) * cpg + col) * spatial + sp;
          const float4 v = make_float4(acc[i][j][4 * q] + bz, acc[i][j][4 * q + 1] + bz,
                                       acc[i][j][4 * q + 2] + bz, acc[i][j][4 * q + 3] + bz);
          if ((spatial & 3) == 0 && (row & 3) == 0 && row + 3 < m_end) {
            *reinterpret_cast<float4*>(dst) = v;
          } else {
            // Rows may cross into the next image: place each one on its own.
            const float vals[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int re = row + e;
              if (re >= m_end) break;
              const uint32_t ne = fdiv(uint32_t(re), MODE == MODE_FWD ? P.f_oS : P.f_S);
              const uint32_t se = uint32_t(re) - ne * uint32_t(spatial);
              P.out[(int64_t(ne) * chans + int64_t(g) * cpg + col) * spatial + se] = vals[e];
            }
          }
        }
      }
  }
}

// Workgroup tile BM x BN (64 or 128 each), four wavefronts in a 2 x 2 grid,
// each holding (BM/2) x (BN/2) as TM x TN MFMA 32 x 32 accumulators.
// Operand tiles are staged k-major in LDS (rows padded by one float).
//
// Two load mappings: "row-mapped" (FWD / DGRAD A) gives thread t the fixed
// row t % BM and the k offsets t / BM + (256 / BM) * i, which are uniform
// over a wavefront, so the k decomposition runs on the scalar unit;
// "k-mapped" (the other operands) gives the fixed k offset t % BK and the
// rows t / BK + (256 / BK) * i.
template <int MODE, int BM, int BN>
__global__ void __launch_bounds__(256) conv_gemm_kernel(ConvK P) {
  constexpr int LDA = BM + 1, LDB = BN + 1;
  constexpr int TM = BM / 64, TN = BN / 64;
  constexpr int NA = BM * CBK / 256, NB = BN * CBK / 256;
  constexpr int RSTEP = 256 / BM;   // row-mapped k stride
  constexpr int KROWS = 256 / CBK;  // k-mapped row stride
  __shared__ float As[2][CBK * LDA];
  __shared__ float Bs[2][CBK * LDB];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int tm = int(blockIdx.x) % P.tiles_m, tn = int(blockIdx.x) / P.tiles_m;
  const int g = MODE == MODE_WGRAD ? int(blockIdx.y) / P.ksplit : int(blockIdx.y);
  const int split = MODE == MODE_WGRAD ? int(blockIdx.y) % P.ksplit : 0;
  const int m0 = tm * BM, n0 = tn * BN;
  const int kbeg = split * P.k_chunk;
  const int kend = min(P.K, kbeg + P.k_chunk);
  const int HW = P.H * P.W, oHW = P.oH * P.oW, KHW = P.KH * P.KW;

  const int r_row = tid % BM;                                   // row-mapped row
  const int k_row0 = __builtin_amdgcn_readfirstlane(tid / BM);  // row-mapped first k offset
  const int kk_k = tid % CBK;                                   // k-mapped k offset
  const int r_k = tid / CBK;                                    // k-mapped first row

  // FWD / DGRAD A: this thread's output (FWD) or input (DGRAD) position.
  int64_t a_base = 0;
  int a_p0 = 0, a_p1 = 0, a_p2 = 0;
  bool a_row_ok = false;
  // WGRAD B: (c, kd, kh, kw) of this thread's NB columns.
  int64_t wb_chan[NB];
  int wb_d[NB], wb_h[NB], wb_w[NB];
  bool wb_ok[NB];
  if constexpr (MODE == MODE_FWD || MODE == MODE_DGRAD) {
    const int m = m0 + r_row;
    a_row_ok = m < P.M;
    const uint32_t mm = a_row_ok ? uint32_t(m) : 0u;
    if constexpr (MODE == MODE_FWD) {
      const uint32_t n = fdiv(mm, P.f_oS), sp = mm - n * uint32_t(P.oS);
      const uint32_t od = fdiv(sp, P.f_oHW), r = sp - od * uint32_t(oHW);
      const uint32_t oh = fdiv(r, P.f_oW), ow = r - oh * uint32_t(P.oW);
      a_base = (int64_t(n) * P.C + int64_t(g) * P.Cpg) * P.S;
      a_p0 = int(od) * P.sd - P.pd;
      a_p1 = int(oh) * P.sh - P.ph;
      a_p2 = int(ow) * P.sw - P.pw;
    } else {
      const uint32_t n = fdiv(mm, P.f_S), sp = mm - n * uint32_t(P.S);
      const uint32_t id = fdiv(sp, P.f_HW), r = sp - id * uint32_t(HW);
      const uint32_t ih = fdiv(r, P.f_W), iw = r - ih * uint32_t(P.W);
      a_base = (int64_t(n) * P.O + int64_t(g) * P.Opg) * P.oS;
      a_p0 = int(id) + P.pd;
      a_p1 = int(ih) + P.ph;
      a_p2 = int(iw) + P.pw;
    }
  }
  if constexpr (MODE == MODE_WGRAD) {
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int j = n0 + r_k + KROWS * i;
      wb_ok[i] = j < P.NC;
      const uint32_t jj = wb_ok[i] ? uint32_t(j) : 0u;
      const uint32_t c = fdiv(jj, P.f_KV), kv = jj - c * uint32_t(P.KV);
      const uint32_t kd = fdiv(kv, P.f_KHW), r = kv - kd * uint32_t(KHW);
      const uint32_t kh = fdiv(r, P.f_KW), kw = r - kh * uint32_t(P.KW);
      wb_chan[i] = (int64_t(g) * P.Cpg + c) * P.S;
      wb_d[i] = int(kd) * P.dd - P.pd;
      wb_h[i] = int(kh) * P.dh - P.ph;
      wb_w[i] = int(kw) * P.dw - P.pw;
    }
  }

  float ra[NA], rb[NB];
  auto fetch = [&](int k0) {
    if constexpr (MODE == MODE_FWD) {
#pragma unroll
      for (int i = 0; i < NA; ++i) {  // A: x at (m, k = (c, kv)); k uniform over the wavefront
        // Branch-free: every lane loads (out-of-range taps from the group's
        // first element, always in bounds) and zeroes what lies outside.
        const int k = k0 + k_row0 + RSTEP * i;
        const bool k_ok = k < kend;
        const uint32_t kc = k_ok ? uint32_t(k) : 0u;
        const uint32_t c = fdiv(kc, P.f_KV), kv = kc - c * uint32_t(P.KV);
        const uint32_t kd = fdiv(kv, P.f_KHW), r = kv - kd * uint32_t(KHW);
        const uint32_t kh = fdiv(r, P.f_KW), kw = r - kh * uint32_t(P.KW);
        const int id = a_p0 + int(kd) * P.dd, ih = a_p1 + int(kh) * P.dh, iw = a_p2 + int(kw) * P.dw;
        const bool ok = k_ok && a_row_ok && unsigned(id) < unsigned(P.D) && unsigned(ih) < unsigned(P.H) &&
                        unsigned(iw) < unsigned(P.W);
        const int64_t off = ok ? int64_t(c) * P.S + (int64_t(id) * P.H + ih) * P.W + iw : 0;
        const float t = P.a[a_base + off];
        ra[i] = ok ? t : 0.f;
      }
      const int k = k0 + kk_k;
#pragma unroll
      for (int i = 0; i < NB; ++i) {  // B: w[g*Opg + o][k], contiguous along k
        const int o = n0 + r_k + KROWS * i;
        const bool ok = o < P.NC && k < kend;
        const float t = P.b[ok ? (int64_t(g) * P.Opg + o) * P.K + k : 0];
        rb[i] = ok ? t : 0.f;
      }
    } else if constexpr (MODE == MODE_DGRAD) {
#pragma unroll
      for (int i = 0; i < NA; ++i) {  // A: dy at (m, k = (o, kv)); k uniform over the wavefront
        const int k = k0 + k_row0 + RSTEP * i;  // branch-free as in FWD
        const bool k_ok = k < kend;
        const uint32_t kc = k_ok ? uint32_t(k) : 0u;
        const uint32_t o = fdiv(kc, P.f_KV), kv = kc - o * uint32_t(P.KV);
        const uint32_t kd = fdiv(kv, P.f_KHW), r = kv - kd * uint32_t(KHW);
        const uint32_t kh = fdiv(r, P.f_KW), kw = r - kh * uint32_t(P.KW);
        const int td = a_p0 - int(kd) * P.dd, th = a_p1 - int(kh) * P.dh, tw = a_p2 - int(kw) * P.dw;
        const bool nonneg = td >= 0 && th >= 0 && tw >= 0;
        const uint32_t ud = nonneg ? uint32_t(td) : 0u, uh = nonneg ? uint32_t(th) : 0u,
                       uw = nonneg ? uint32_t(tw) : 0u;
        const uint32_t od = fdiv(ud, P.f_sd), oh = fdiv(uh, P.f_sh), ow = fdiv(uw, P.f_sw);
        const bool ok = k_ok && a_row_ok && nonneg && od * uint32_t(P.sd) == ud && oh * uint32_t(P.sh) == uh &&
                        ow * uint32_t(P.sw) == uw && od < uint32_t(P.oD) && oh < uint32_t(P.oH) &&
                        ow < uint32_t(P.oW);
        const int64_t off = ok ? int64_t(o) * P.oS + (int64_t(od) * P.oH + oh) * P.oW + ow : 0;
        const float t = P.a[a_base + off];
        ra[i] = ok ? t : 0.f;
      }
      const int k = k0 + kk_k;
      const bool k_ok = k < kend;
      const uint32_t kc = k_ok ? uint32_t(k) : 0u;
      const uint32_t o = fdiv(kc, P.f_KV), kv = kc - o * uint32_t(P.KV);
#pragma unroll
      for (int i = 0; i < NB; ++i) {  // B: w[g*Opg + o][c][kv]
        const int c = n0 + r_k + KROWS * i;
        const bool ok = c < P.NC && k_ok;
        const float t = P.b[ok ? ((int64_t(g) * P.Opg + o) * P.Cpg + c) * P.KV + kv : 0];
        rb[i] = ok ? t : 0.f;
      }
    } else {
      const int k = k0 + kk_k;
      const bool k_ok = k < kend;
      const uint32_t kc = k_ok ? uint32_t(k) : 0u;
      const uint32_t n = fdiv(kc, P.f_oS), sp = kc - n * uint32_t(P.oS);
#pragma unroll
      for (int i = 0; i < NA; ++i) {  // A: dy[n][g*Opg + o][sp]
        const int o = m0 + r_k + KROWS * i;
        const bool ok = o < P.M && k_ok;
        const float t = P.a[ok ? (int64_t(n) * P.O + int64_t(g) * P.Opg + o) * P.oS + sp : 0];
        ra[i] = ok ? t : 0.f;
      }
      const uint32_t od = fdiv(sp, P.f_oHW), r = sp - od * uint32_t(oHW);
      const uint32_t oh = fdiv(r, P.f_oW), ow = r - oh * uint32_t(P.oW);
      const int64_t xn = int64_t(n) * P.C * P.S;
#pragma unroll
      for (int i = 0; i < NB; ++i) {  // B: x at (k = (n, p), j = (c, kv))
        const int id = int(od) * P.sd + wb_d[i], ih = int(oh) * P.sh + wb_h[i], iw = int(ow) * P.sw + wb_w[i];
        const bool ok = wb_ok[i] && k_ok && unsigned(id) < unsigned(P.D) && unsigned(ih) < unsigned(P.H) &&
                        unsigned(iw) < unsigned(P.W);
        const float t = P.b[ok ? xn + wb_chan[i] + (int64_t(id) * P.H + ih) * P.W + iw : 0];
        rb[i] = ok ? t : 0.f;
      }
    }
  };
  auto commit = [&](int buf) {
    if constexpr (MODE == MODE_WGRAD) {
#pragma unroll
      for (int i = 0; i < NA; ++i) As[buf][kk_k * LDA + r_k + KROWS * i] = ra[i];
    } else {
#pragma unroll
      for (int i = 0; i < NA; ++i) As[buf][(k_row0 + RSTEP * i) * LDA + r_row] = ra[i];
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) Bs[buf][kk_k * LDB + r_k + KROWS * i] = rb[i];
  };

  float16v acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
  const int nk = kend > kbeg ? (kend - kbeg + CBK - 1) / CBK : 0;
  if (nk > 0) {
    fetch(kbeg);
    commit(0);
  }
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) fetch(kbeg + (kt + 1) * CBK);
#pragma unroll
    for (int s = 0; s < CBK / 2; ++s) {
      const int k = 2 * s + (lane >> 5);
      float af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) af[i] = As[buf][k * LDA + wm * (BM / 2) + i * 32 + (lane & 31)];
#pragma unroll
      for (int j = 0; j < TN; ++j) bf[j] = Bs[buf][k * LDB + wn * (BN / 2) + j * 32 + (lane & 31)];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) commit(buf ^ 1);
    __syncthreads();
  }

  conv_epilogue<MODE, BM, BN>(P, acc, m0, n0, wm, wn, g, split, P.M);
}

// Forward convolution with the operands gathered straight into an S-stage
// LDS ring by buffer_load_dword ... lds (one wavefront instruction fills one
// 64-float row of a k-major tile: lane L writes element L, fetching whatever
// x or w value that row position needs).  Taps outside the input, rows past
// M, columns past NC and k past the reduction get an offset beyond the
// buffer's num_records and read 0, so the gathers need no branches and no
// register round trip; copies run S-1 k-steps ahead of the MFMAs and each
// step waits only for its own stage.  Same tile, MFMA and epilogue as
// conv_gemm_kernel<MODE_FWD>; requires x and w below 2 GiB (32-bit offsets).
constexpr uint32_t kConvOob = 0x80000000u;

// buffer_load_dword ... lds: lane L copies the 4 bytes at voffset + soffset
// of the buffer to LDS byte lds_base + 4 L.  Inline assembly for the reason
// given at bgk::dma16_to_lds: with the builtin the compiler makes every later
// LDS read wait for all outstanding copies, which empties the ring.  The
// leading s_nop keeps five wait states between a VALU write of an SGPR
// operand and this VMEM read of it.
__device__ __forceinline__ void conv_dma4_to_lds(uint32_t lds_base, uint32_t voffset, bgk::sgpr4_t rsrc,
                                                 uint32_t soffset) {
  asm volatile(
      "s_nop 4\n\t"
      "buffer_load_dword %1, %2, %3 offen lds"
      :
      : "{m0}"(lds_base), "v"(voffset), "s"(rsrc), "s"(soffset)
      : "memory");
}

template <int N>
__device__ __forceinline__ void conv_wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// B16: the weight arrives k-major with Opg % 4 == 0, and its tile is copied
// with 16-byte copies, one 1 KB instruction per 1024 / (4 BN) k rows of an
// unpadded tile (4x fewer copy instructions for it than one 64-float row
// per instruction).
template <int BM, int BN, int S, bool B16>
__global__ void __launch_bounds__(256) conv_fwd_ring_kernel(ConvK P, uint32_t a_bytes, uint32_t b_bytes) {
  constexpr int LDA = BM + 1, LDB = B16 ? BN : BN + 1;
  constexpr int TM = BM / 64, TN = BN / 64;
  constexpr int QA = BM / 64, QB = BN / 64;  // 64-float rows per k row
  constexpr int IA = CBK * QA / 4;           // instructions per wavefront per stage
  constexpr int IB = B16 ? CBK * BN / 256 / 4 : CBK * QB / 4;
  constexpr int NLD = IA + IB;
  static_assert(NLD * (S - 1) < 64, "vmcnt range");
  static_assert(!B16 || IB >= 1, "one 1 KB copy per wavefront at least");
  __shared__ __attribute__((aligned(16))) float As[S][CBK * LDA];
  __shared__ __attribute__((aligned(16))) float Bs[S][CBK * LDB];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int tm = int(blockIdx.x) % P.tiles_m, tn = int(blockIdx.x) / P.tiles_m;
  const int g = int(blockIdx.y);
  const int m0 = tm * BM, n0 = tn * BN;
  const int K = P.K;
  const int KHW = P.KH * P.KW;

  // Instruction i of wavefront w covers tile row block (i*4 + w) % Q at k
  // offset (i*4 + w) / Q; for Q = 1 or 2 the block is fixed per wavefront.
  const int qa = QA == 1 ? 0 : (wave & 1);
  const int qb = QB == 1 ? 0 : (wave & 1);
  // A: this lane's output position m -> x base and input origin.
  const int m = m0 + qa * 64 + lane;
  const bool row_ok = m < P.M;
  const uint32_t mm = row_ok ? uint32_t(m) : 0u;
  const uint32_t n = fdiv(mm, P.f_oS), sp = mm - n * uint32_t(P.oS);
  const uint32_t od = fdiv(sp, P.f_oHW), rr = sp - od * uint32_t(P.oH * P.oW);
  const uint32_t oh = fdiv(rr, P.f_oW), ow = rr - oh * uint32_t(P.oW);
  const int64_t a_base = (int64_t(n) * P.C + int64_t(g) * P.Cpg) * P.S;
  const int p0 = int(od) * P.sd - P.pd, p1 = int(oh) * P.sh - P.ph, p2 = int(ow) * P.sw - P.pw;
  // B: this lane's output channel o -> w row.
  const int o = n0 + qb * 64 + lane;
  // w [G][Opg][K] makes one copy instruction (64 channels at one k) touch 64
  // rows 4K bytes apart; the k-major copy [G][K][Opg] makes it 256
  // contiguous bytes.
  const uint32_t b_lane = o >= P.NC ? kConvOob
                          : P.b_kmajor ? uint32_t((int64_t(g) * K * P.Opg + o) * 4)
                                       : uint32_t((int64_t(g) * P.Opg + o) * K * 4);
  const uint32_t b_kstride = P.b_kmajor ? uint32_t(P.Opg) * 4u : 4u;
  // B16: copy i of this wavefront fills tile floats f = (4 i + w) * 256 + 4 l
  // .. + 3: k row f / BN, channels n0 + f % BN .. + 3 (all valid or all past
  // NC, since NC % 4 == 0).
  uint32_t b16_off[B16 ? IB : 1];
  int b16_row[B16 ? IB : 1];
  if constexpr (B16) {
#pragma unroll
    for (int i = 0; i < IB; ++i) {
      const int f = (i * 4 + wave) * 256 + lane * 4;
      b16_row[i] = f / BN;
      const int oc = n0 + f % BN;
      b16_off[i] = oc < P.NC ? uint32_t(((int64_t(g) * K + b16_row[i]) * P.Opg + oc) * 4) : kConvOob;
    }
  }

  const bgk::sgpr4_t ra = bgk::buffer_rsrc(P.a, a_bytes);
  const bgk::sgpr4_t rb = bgk::buffer_rsrc(P.b, b_bytes);
  const int nk = (K + CBK - 1) / CBK;

  auto issue_stage = [&](int t) {
    const int slot = t % S;
    const int k0 = t * CBK;
#pragma unroll
    for (int i = 0; i < IA; ++i) {
      const int kl = (i * 4 + wave) / QA;
      const int k = k0 + kl;  // uniform
      const bool k_ok = k < K;
      const uint32_t kc = k_ok ? uint32_t(k) : 0u;
      const uint32_t c = fdiv(kc, P.f_KV), kv = kc - c * uint32_t(P.KV);
      const uint32_t kd = fdiv(kv, P.f_KHW), r = kv - kd * uint32_t(KHW);
      const uint32_t kh = fdiv(r, P.f_KW), kw = r - kh * uint32_t(P.KW);
      const int id = p0 + int(kd) * P.dd, ih = p1 + int(kh) * P.dh, iw = p2 + int(kw) * P.dw;
      const bool ok = k_ok && row_ok && unsigned(id) < unsigned(P.D) && unsigned(ih) < unsigned(P.H) &&
                      unsigned(iw) < unsigned(P.W);
      const uint32_t off =
          ok ? uint32_t((a_base + int64_t(c) * P.S + (int64_t(id) * P.H + ih) * P.W + iw) * 4) : kConvOob;
      conv_dma4_to_lds(bgk::lds_addr(&As[slot][kl * LDA + qa * 64]), off, ra, 0u);
    }
    if constexpr (B16) {
#pragma unroll
      for (int i = 0; i < IB; ++i) {
        const uint32_t off = k0 + b16_row[i] < K ? b16_off[i] : kConvOob;
        bgk::dma16_to_lds(bgk::lds_addr(&Bs[slot][(i * 4 + wave) * 256]), off, rb,
                          k0 < K ? uint32_t(k0) * b_kstride : 0u);
      }
    } else {
#pragma unroll
      for (int i = 0; i < IB; ++i) {
        const int kl = (i * 4 + wave) / QB;
        const int k = k0 + kl;  // uniform
        const uint32_t off = k < K ? b_lane : kConvOob;
        conv_dma4_to_lds(bgk::lds_addr(&Bs[slot][kl * LDB + qb * 64]), off, rb,
                         k < K ? uint32_t(k) * b_kstride : 0u);
      }
    }
  };

  float16v acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // Stages past the reduction load only zeros (every offset out of range),
  // so each step issues the same number of copies and the partial waits
  // below always name the right stage.
#pragma unroll
  for (int t = 0; t < S - 1; ++t) issue_stage(t);
  for (int kt = 0; kt < nk; ++kt) {
    // Stage kt has landed (later stages may still be in flight), every
    // wavefront has finished reading the slot refilled next.
    conv_wait_vmcnt<NLD * (S - 2)>();
    __syncthreads();
    issue_stage(kt + S - 1);
    const int buf = kt % S;
#pragma unroll
    for (int s = 0; s < CBK / 2; ++s) {
      const int k = 2 * s + (lane >> 5);
      float af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) af[i] = As[buf][k * LDA + wm * (BM / 2) + i * 32 + (lane & 31)];
#pragma unroll
      for (int j = 0; j < TN; ++j) bf[j] = Bs[buf][k * LDB + wn * (BN / 2) + j * 32 + (lane & 31)];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
  }
  conv_wait_vmcnt<0>();  // the run-out copies still write LDS; let them land before exit

  conv_epilogue<MODE_FWD, BM, BN>(P, acc, m0, n0, wm, wn, g, 0, P.M);
}

// ---- 3x3 stride-1 forward with input patches (2-D) --------------------------------
//
// The ring kernel copies, for every k = (c, tap), the 64 input values its 64
// output rows need: nine shifted, unaligned gathers per channel.  Here a
// BM-row tile is TR whole output rows of one image (TR = BM / oW), and each
// stage copies, for CB input channels, the (TR + 2) x (W + 2 pad) input
// patch those rows read (pad columns and rows outside the image read 0), a
// few row-contiguous copies per channel instead of nine gathers.  The A
// operand of k = (c, kh, kw) for tile row s = r oW + cc is patch[c][(r + kh)
// (oW + 2) + cc + kw] (stride 1, so oW + 2 = W + 2 pad).  The weight tile
// (k-major, 9 CB k rows x BN channels) streams in with 16-byte copies.  Each
// stage is the 9 CB k of CB channels (CB even, so every stage starts on an
// even k), taken in the ring kernel's k order and MFMA pairs, so the sums
// are bit-identical to it.
//
// WM wavefronts along M (BM = 32 WM tile rows) and WN along N (BN = 32 WN
// columns), each with one 32 x 32 accumulator; PC dword copies per
// wavefront per stage hold the CB patches.  Weight copies past
// the tile's rows land in a scratch area of LDS nobody reads, so that every
// wavefront issues the same number of copies per stage (the vmcnt waits
// count them).
template <int S, int CB, int WM, int WN, int PC>
__global__ void __launch_bounds__(64 * WM * WN) conv_fwd_halo_kernel(ConvK P, uint32_t a_bytes, uint32_t b_bytes,
                                                                     int TR) {
  constexpr int NW = WM * WN, BN = 32 * WN, KS = 9 * CB;
  static_assert(CB % 2 == 0, "stages must start on even k");
  constexpr int PATCH = PC * NW * 64;               // floats per stage slot
  constexpr int BCOPIES = (KS * BN + 255) / 256;    // 1 KB copies that hold the weight tile
  constexpr int BC = (BCOPIES + NW - 1) / NW;       // per wavefront
  constexpr int NLD = PC + BC;
  static_assert(NLD * (S - 1) < 64, "vmcnt range");
  __shared__ __attribute__((aligned(16))) float Ps[S][PATCH];
  __shared__ __attribute__((aligned(16))) float Bs[S][BCOPIES * 256];
  __shared__ __attribute__((aligned(16))) float Bsink[NW * BC > BCOPIES ? 256 : 4];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
  const int wm = wave % WM, wn = wave / WM;
  const int tiles_n = (P.NC + BN - 1) / BN;
  const int tn = int(blockIdx.x) % tiles_n, tm = int(blockIdx.x) / tiles_n;
  const int g = int(blockIdx.y);
  const int n0 = tn * BN;
  const int K = P.K;
  // Tile tm: image n, output rows oh0 .. oh0 + TR - 1.
  const int tiles_per_image = (P.oH + TR - 1) / TR;
  const int n = tm / tiles_per_image;
  const int oh0 = (tm - n * tiles_per_image) * TR;
  const int m0 = n * P.oS + oh0 * P.oW;
  const int m_end = min(m0 + TR * P.oW, (n + 1) * P.oS);
  const int PW = P.oW + 2, PSZ = (TR + 2) * PW;  // patch row width, floats per channel

  // A operand: this lane's tile row s = wm * 32 + lane % 32 -> patch offset.
  const int s_row = wm * 32 + (lane & 31);
  const int r = s_row / P.oW, cc = s_row - r * P.oW;
  const int a_base = s_row < TR * P.oW ? r * PW + cc : 0;  // rows past the tile read row 0 (never stored)
  // Per MFMA pair p of a stage, this lane-half's k = 2 p + lane / 32 ->
  // (channel, kh, kw) -> patch offset.
  int a_off[KS / 2];
#pragma unroll
  for (int p = 0; p < KS / 2; ++p) {
    const int k = 2 * p + (lane >> 5);
    const int cl = k / 9, t = k % 9;
    a_off[p] = a_base + cl * PSZ + (t / 3) * PW + (t % 3);
  }
  // Patch copies: copy i of wave w fills patch floats f = (NW i + w) * 64 + l.
  const int64_t x_img = (int64_t(n) * P.C + int64_t(g) * P.Cpg) * P.S;
  int pc_c[PC], pc_src[PC];
  bool pc_ok[PC];
#pragma unroll
  for (int i = 0; i < PC; ++i) {
    const int f = (i * NW + wave) * 64 + lane;
    const int cl = f / PSZ, rem = f - cl * PSZ;
    const int pr = rem / PW, pcol = rem - pr * PW;
    const int ih = oh0 - P.ph + pr, iw = pcol - P.pw;
    pc_c[i] = cl;
    pc_src[i] = ih * P.W + iw;
    pc_ok[i] = cl < CB && unsigned(ih) < unsigned(P.H) && unsigned(iw) < unsigned(P.W);
  }
  // Weight copies (k-major [G][K][Opg], Opg % 4 == 0): copy c = NW i + w
  // fills tile floats f = 256 c + 4 l: k row f / BN, channels n0 + f % BN
  // .. + 3.
  uint32_t b_off[BC];
  int b_row[BC];
  uint32_t b_lds[BC];
#pragma unroll
  for (int i = 0; i < BC; ++i) {
    const int c = i * NW + wave;
    const int f = c * 256 + lane * 4;
    b_row[i] = f / BN;
    const int oc = n0 + f % BN;
    b_off[i] = c < BCOPIES && oc < P.NC && b_row[i] < KS ? uint32_t(((int64_t(g) * K + b_row[i]) * P.Opg + oc) * 4)
                                                          : kConvOob;
    if (c >= BCOPIES) b_row[i] = K;  // never in range
    b_lds[i] = c < BCOPIES ? uint32_t(c * 256 * 4) : 0u;
  }

  const bgk::sgpr4_t ra = bgk::buffer_rsrc(P.a, a_bytes);
  const bgk::sgpr4_t rb = bgk::buffer_rsrc(P.b, b_bytes);
  const int nk = (P.Cpg + CB - 1) / CB;

  auto issue_stage = [&](int t) {
    const int slot = t % S;
    const int c0 = t * CB;
#pragma unroll
    for (int i = 0; i < PC; ++i) {
      const bool ok = pc_ok[i] && c0 + pc_c[i] < P.Cpg;
      const uint32_t off = ok ? uint32_t((x_img + int64_t(c0 + pc_c[i]) * P.S + pc_src[i]) * 4) : kConvOob;
      conv_dma4_to_lds(bgk::lds_addr(&Ps[slot][(i * NW + wave) * 64]), off, ra, 0u);
    }
    const int k0 = c0 * 9;
#pragma unroll
    for (int i = 0; i < BC; ++i) {
      const uint32_t off = k0 + b_row[i] < K ? b_off[i] : kConvOob;
      const uint32_t dst = i * NW + wave < BCOPIES ? bgk::lds_addr(&Bs[slot][0]) + b_lds[i] : bgk::lds_addr(&Bsink[0]);
      bgk::dma16_to_lds(dst, off, rb, k0 < K ? uint32_t(k0) * uint32_t(P.Opg) * 4u : 0u);
    }
  };

  float16v acc[1][1];
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[0][0][e] = 0.f;

#pragma unroll
  for (int t = 0; t < S - 1; ++t) issue_stage(t);
  for (int kt = 0; kt < nk; ++kt) {
    conv_wait_vmcnt<NLD * (S - 2)>();
    __syncthreads();
    issue_stage(kt + S - 1);
    const int buf = kt % S;
#pragma unroll
    for (int p = 0; p < KS / 2; ++p) {
      const float af = Ps[buf][a_off[p]];
      const float bf = Bs[buf][(2 * p + (lane >> 5)) * BN + wn * 32 + (lane & 31)];
      acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(af, bf, acc[0][0], 0, 0, 0);
    }
  }
  conv_wait_vmcnt<0>();  // the run-out copies still write LDS; let them land before exit

  // Wavefront (wm, wn) holds rows m0 + 32 wm .. + 31 and columns n0 + 32 wn
  // .. + 31: wavefront (0, 0) of a 64 x 64 epilogue placed there.
  conv_epilogue<MODE_FWD, 64, 64>(P, acc, m0 + wm * 32, n0 + wn * 32, 0, 0, g, 0, m_end);
}

// dw[i] = sum over split slices (in order) of part[s][i].
__global__ void __launch_bounds__(256) conv_split_reduce_kernel(const float* __restrict__ part,
                                                                float* __restrict__ out, int64_t total,
                                                                int splits) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total) return;
  float acc = 0.f;
  int s = 0;
  for (; s + 8 <= splits; s += 8) {
    float t[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) t[u] = part[int64_t(s + u) * total + i];
#pragma unroll
    for (int u = 0; u < 8; ++u) acc += t[u];
  }
  for (; s < splits; ++s) acc += part[int64_t(s) * total + i];
  out[i] = acc;
}

// part[r] = sum of dy row r (r = n * O + o, `spatial` floats): one
// wavefront per row, four independent loads in flight per lane.
__global__ void __launch_bounds__(256) conv_row_sum_kernel(const float* __restrict__ dy, float* __restrict__ part,
                                                           int64_t rows, int64_t spatial) {
  const int lane = threadIdx.x & 63;
  const int64_t r = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const float* row = dy + r * spatial;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  int64_t p = lane;
  for (; p + 192 < spatial; p += 256) {
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[u] += row[p + 64 * u];
  }
  for (; p < spatial; p += 64) acc[0] += row[p];
  float s = (acc[0] + acc[1]) + (acc[2] + acc[3]);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
  if (lane == 0) part[r] = s;
}

// The same sum for rows of spatial4 float4s (row length a multiple of 4, the
// tensor 16-byte aligned): each lane has up to four float4 loads in flight
// before it adds any of them.
__global__ void __launch_bounds__(256) conv_row_sum4_kernel(const float4* __restrict__ dy, float* __restrict__ part,
                                                            int64_t rows, int64_t spatial4) {
  const int lane = threadIdx.x & 63;
  const int64_t r = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const float4* row = dy + r * spatial4;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int64_t base = 0; base < spatial4; base += 256) {
    float4 t[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t q = base + lane + 64 * u;
      t[u] = q < spatial4 ? row[q] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[u] += (t[u].x + t[u].y) + (t[u].z + t[u].w);
  }
  float s = (acc[0] + acc[1]) + (acc[2] + acc[3]);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
  if (lane == 0) part[r] = s;
}

// db[o] = sum over n (in order) of part[n * O + o]; eight loads are issued
// before they are added.
__global__ void __launch_bounds__(256) conv_bias_final_kernel(const float* __restrict__ part, float* __restrict__ db,
                                                              int64_t n, int64_t o_count) {
  const int64_t o = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (o >= o_count) return;
  float acc = 0.f;
  int64_t b = 0;
  for (; b + 8 <= n; b += 8) {
    float t[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) t[u] = part[(b + u) * o_count + o];
#pragma unroll
    for (int u = 0; u < 8; ++u) acc += t[u];
  }
  for (; b < n; ++b) acc += part[b * o_count + o];
  db[o] = acc;
}

// db[o] = sum over (n, p) of dy[n][o][p] in one launch, one workgroup per
// channel: thread t adds the float4 groups t, t + 1024, ... of the channel's
// n x spatial4 groups in order, then the 1024 sums are added pairwise in a
// fixed tree through LDS (the result does not depend on scheduling).
__global__ void __launch_bounds__(1024) conv_bias_grad1_kernel(const float4* __restrict__ dy, float* __restrict__ db,
                                                               int64_t n, int64_t o_count, int64_t spatial4) {
  __shared__ float red[1024];
  const int64_t o = blockIdx.x;
  const int64_t total = n * spatial4;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  int64_t i = threadIdx.x;
  for (; i + 3 * 1024 < total; i += 4 * 1024) {
    float4 t[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t ii = i + u * 1024;
      const int64_t nn = ii / spatial4, q = ii - nn * spatial4;
      t[u] = dy[(nn * o_count + o) * spatial4 + q];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[u] += (t[u].x + t[u].y) + (t[u].z + t[u].w);
  }
  for (; i < total; i += 1024) {
    const int64_t nn = i / spatial4, q = i - nn * spatial4;
    const float4 t = dy[(nn * o_count + o) * spatial4 + q];
    acc[0] += (t.x + t.y) + (t.z + t.w);
  }
  red[threadIdx.x] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  __syncthreads();
#pragma unroll
  for (int w = 512; w >= 1; w >>= 1) {
    if (int(threadIdx.x) < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) db[o] = red[0];
}

// wt[g][k][o] = w[g][o][k] through a 32 x 32 LDS tile (both sides coalesced).
__global__ void __launch_bounds__(256) conv_w_kmajor_kernel(const float* __restrict__ w, float* __restrict__ wt,
                                                            int Opg, int K) {
  __shared__ float t[32][33];
  const int64_t g = blockIdx.z;
  const int k0 = int(blockIdx.x) * 32, o0 = int(blockIdx.y) * 32;
  const int tx = int(threadIdx.x) & 31, ty = int(threadIdx.x) >> 5;
  const float* src = w + g * Opg * int64_t(K);
  float* dst = wt + g * int64_t(K) * Opg;
  for (int r = ty; r < 32; r += 8) {
    const int o = o0 + r, k = k0 + tx;
    if (o < Opg && k < K) t[r][tx] = src[int64_t(o) * K + k];
  }
  __syncthreads();
  for (int r = ty; r < 32; r += 8) {
    const int k = k0 + r, o = o0 + tx;
    if (o < Opg && k < K) dst[int64_t(k) * Opg + o] = t[tx][r];
  }
}

// w2[(g*Cpg + c)*Opg*KV + o*KV + kv] = w[((g*Opg + o)*Cpg + c)*KV + KV-1-kv]:
// the weight of the forward convolution equal to a stride-1 input gradient
// (channel roles exchanged, every spatial tap reversed).
__global__ void __launch_bounds__(256) conv_flip_weight_kernel(const float* __restrict__ w, float* __restrict__ w2,
                                                               int64_t G, int64_t Opg, int64_t Cpg, int64_t KV) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t total = G * Opg * Cpg * KV;
  if (i >= total) return;
  const int64_t kv = i % KV;
  const int64_t o = (i / KV) % Opg;
  const int64_t gc = i / (KV * Opg);  // g * Cpg + c
  const int64_t g = gc / Cpg, c = gc % Cpg;
  w2[i] = w[((g * Opg + o) * Cpg + c) * KV + (KV - 1 - kv)];
}

// The same flipped weight written k-major for the LDS-ring forward kernel:
// w2t[g][k][c] with k = o * KV + kv (the flipped problem's reduction index)
// and c its output channel.
__global__ void __launch_bounds__(256) conv_flip_kmajor_kernel(const float* __restrict__ w, float* __restrict__ w2t,
                                                               int64_t G, int64_t Opg, int64_t Cpg, int64_t KV) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t K2 = Opg * KV;
  const int64_t total = G * K2 * Cpg;
  if (i >= total) return;
  const int64_t c = i % Cpg;
  const int64_t k = (i / Cpg) % K2;
  const int64_t g = i / (Cpg * K2);
  const int64_t o = k / KV, kv = k % KV;
  w2t[i] = w[((g * Opg + o) * Cpg + c) * KV + (KV - 1 - kv)];
}

// Weight of one phase convolution of a strided input gradient, k-major for
// the ring kernel: wt[(g*K' + o*KVp + th*KWp + tw)*Cpg + c] =
// w[((g*Opg + o)*Cpg + c)*KH*KW + kh[th]*KW + kw[tw]] (K' = Opg*KVp; the
// phase's taps in the order the phase convolution reads them).
struct PhaseTaps {
  int khp, kwp;
  int kh[16], kw[16];
};

__global__ void __launch_bounds__(256) conv_phase_weight_kernel(const float* __restrict__ w, float* __restrict__ wt,
                                                                int64_t G, int64_t Opg, int64_t Cpg, int KH, int KW,
                                                                PhaseTaps t) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t kvp = int64_t(t.khp) * t.kwp;
  const int64_t total = G * Opg * kvp * Cpg;
  if (i >= total) return;
  const int64_t c = i % Cpg;
  const int64_t k = (i / Cpg) % (Opg * kvp);
  const int64_t g = i / (Cpg * Opg * kvp);
  const int64_t o = k / kvp, tv = k % kvp;
  const int th = int(tv / t.kwp), tw = int(tv % t.kwp);
  wt[i] = w[((g * Opg + o) * Cpg + c) * (int64_t(KH) * KW) + t.kh[th] * KW + t.kw[tw]];
}

// A phase of dx that no tap reaches: dx[n][c][y*sh + ph][x*sw + pw] =
// bias[c] (or 0), for y < Hph, x < Wph.
__global__ void __launch_bounds__(256) conv_phase_fill_kernel(float* __restrict__ dx, const float* __restrict__ bias,
                                                              int64_t NC, int64_t C, int H, int W, int sh, int sw,
                                                              int ph, int pw, int Hph, int Wph) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t per = int64_t(Hph) * Wph;
  if (i >= NC * per) return;
  const int64_t nc = i / per;
  const int r = int(i % per);
  const int y = r / Wph, x = r % Wph;
  dx[nc * (int64_t(H) * W) + int64_t(y * sh + ph) * W + x * sw + pw] = bias ? bias[nc % C] : 0.f;
}

// Whether the forward of problem p runs the LDS-ring kernel (x and w within
// 32-bit byte offsets; BG_CONV_RING=0 selects the register-staged kernel).
bool conv_fwd_ring(const bg::ConvProblem& p) {
  const int64_t S = p.in[0] * p.in[1] * p.in[2];
  const int64_t K = (p.c / p.groups) * p.k[0] * p.k[1] * p.k[2];
  const int64_t a_bytes = p.n * p.c * S * 4, b_bytes = p.o * K * 4;
  const char* ring_env = std::getenv("BG_CONV_RING");
  return a_bytes < (int64_t(1) << 31) && b_bytes < (int64_t(1) << 31) && !(ring_env && ring_env[0] == '0');
}

}  // namespace

namespace bg {

// Strided 2-D input gradient as stride_h x stride_w phase convolutions.
// dx[y][x] with y = sh*i + ry, x = sw*j + rx takes only the taps kh with
// kh = ry + pad_h (mod sh) (and likewise kw), at dy[i + (ry + pad_h - kh)/sh]
// [j + (rx + pad_w - kw)/sw]: for each phase (ry, rx) a dense stride-1
// forward convolution of dy by that phase's taps (channel roles
// exchanged), written to the phase's positions of dx.  The implicit GEMM of
// the DGRAD kernel visits every (tap, position) pair and finds a term in
// only 1 / (sh sw) of them.  False when the problem does not fit this form
// (3-D, dilation, operands past the ring kernel's 32-bit offsets);
// BG_CONV_DGRAD_PHASES=0 keeps the DGRAD kernel.
static bool launch_dgrad_phases(bg_ctx* ctx, const ConvProblem& p, const float* dy, const float* w,
                                const float* bias, float* dx) {
  const char* env = std::getenv("BG_CONV_DGRAD_PHASES");
  if (env && env[0] == '0') return false;
  if (p.in[0] != 1 || p.out[0] != 1 || p.k[0] != 1 || p.stride[0] != 1 || p.dil[1] != 1 || p.dil[2] != 1) return false;
  const int64_t G = p.groups, Opg = p.o / G, Cpg = p.c / G;
  const int sh = int(p.stride[1]), sw = int(p.stride[2]);
  const int KH = int(p.k[1]), KW = int(p.k[2]);
  const int H = int(p.in[1]), W = int(p.in[2]);
  if (KH > 16 || KW > 16 || G > 65535 || p.n <= 0 || H <= 0 || W <= 0) return false;
  struct Phase {
    int ry, rx, hph, wph, padh, padw;
    PhaseTaps t;
  };
  std::vector<Phase> phases;
  int64_t max_w = 0;
  for (int ry = 0; ry < sh && ry < H; ++ry) {
    for (int rx = 0; rx < sw && rx < W; ++rx) {
      Phase f{};
      f.ry = ry;
      f.rx = rx;
      f.hph = (H - ry + sh - 1) / sh;
      f.wph = (W - rx + sw - 1) / sw;
      // Taps in descending kh: ascending dy row offset (ry + pad - kh) / sh.
      for (int kh = KH - 1; kh >= 0; --kh)
        if (((ry + int(p.pad[1]) - kh) % sh + sh) % sh == 0) f.t.kh[f.t.khp++] = kh;
      for (int kw = KW - 1; kw >= 0; --kw)
        if (((rx + int(p.pad[2]) - kw) % sw + sw) % sw == 0) f.t.kw[f.t.kwp++] = kw;
      if (f.t.khp > 0 && f.t.kwp > 0) {
        // Leading padding of the phase convolution; negative when the
        // phase's first tap reads past dy's first row / column (the ring
        // kernel's index arithmetic is signed, its bounds checks unsigned).
        f.padh = (f.t.kh[0] - ry - int(p.pad[1])) / sh;
        f.padw = (f.t.kw[0] - rx - int(p.pad[2])) / sw;
        max_w = std::max<int64_t>(max_w, G * Opg * f.t.khp * f.t.kwp * Cpg);
        ConvProblem q{};
        q.n = p.n;
        q.c = p.o;
        q.o = p.c;
        q.groups = G;
        q.in[0] = 1; q.in[1] = p.out[1]; q.in[2] = p.out[2];
        q.k[0] = 1; q.k[1] = f.t.khp; q.k[2] = f.t.kwp;
        if (!conv_fwd_ring(q)) return false;
      }
      phases.push_back(f);
    }
  }
  float* wt = max_w > 0 ? static_cast<float*>(scratch(ctx, size_t(max_w) * 4, 1)) : nullptr;
  for (const Phase& f : phases) {
    if (f.t.khp == 0 || f.t.kwp == 0) {
      const int64_t total = p.n * p.c * int64_t(f.hph) * f.wph;
      if (total > 0)
        dispatch(ctx, conv_phase_fill_kernel, dim3(unsigned((total + 255) / 256)), dim3(256), 0, dx, bias,
                 p.n * p.c, p.c, H, W, sh, sw, f.ry, f.rx, f.hph, f.wph);
      continue;
    }
    const int64_t total = G * Opg * f.t.khp * f.t.kwp * Cpg;
    dispatch(ctx, conv_phase_weight_kernel, dim3(unsigned((total + 255) / 256)), dim3(256), 0, w, wt, G, Opg, Cpg,
             KH, KW, f.t);
    ConvProblem q{};
    q.n = p.n;
    q.c = p.o;
    q.o = p.c;
    q.groups = G;
    q.in[0] = 1; q.in[1] = p.out[1]; q.in[2] = p.out[2];
    q.out[0] = 1; q.out[1] = f.hph; q.out[2] = f.wph;
    q.k[0] = 1; q.k[1] = f.t.khp; q.k[2] = f.t.kwp;
    q.stride[0] = q.stride[1] = q.stride[2] = 1;
    q.pad[0] = 0; q.pad[1] = f.padh; q.pad[2] = f.padw;
    q.dil[0] = q.dil[1] = q.dil[2] = 1;
    const ConvOutMap m{sh, sw, f.ry, f.rx, H, W};
    launch_conv(ctx, q, 0, dy, wt, bias, dx, true, &m);
  }
  hip_check(hipGetLastError(), "conv launch");
  return true;
}

void launch_conv(bg_ctx* ctx, const ConvProblem& p, int mode, const float* a, const float* b, const float* bias,
                 float* out, bool b_kmajor, const ConvOutMap* omap) {
  if (mode == 1 && (p.stride[1] > 1 || p.stride[2] > 1) && launch_dgrad_phases(ctx, p, a, b, bias, out)) return;
  if (mode == 1 && p.stride[0] == 1 && p.stride[1] == 1 && p.stride[2] == 1) {
    // dx[q] = sum dy[q + pad - kv*dil] w[kv] is, with kv' = K-1-kv, the
    // forward convolution of dy by the tap-reversed, channel-exchanged
    // weight with padding dil*(K-1) - pad (when that is not negative).
    ConvProblem f = p;
    bool ok = true;
    for (int i = 0; i < 3; ++i) {
      f.pad[i] = p.dil[i] * (p.k[i] - 1) - p.pad[i];
      ok = ok && f.pad[i] >= 0;
      f.in[i] = p.out[i];
      f.out[i] = p.in[i];
    }
    if (ok) {
      f.c = p.o;
      f.o = p.c;
      const int64_t G = p.groups, Opg = p.o / G, Cpg = p.c / G, KV = p.k[0] * p.k[1] * p.k[2];
      const int64_t total = G * Opg * Cpg * KV;
      float* w2 = static_cast<float*>(scratch(ctx, size_t(total) * 4, 1));
      // The ring kernel takes the flipped weight k-major, written in the
      // same pass; the register-staged kernel takes it as [G][Opg'][K'].
      const bool km = conv_fwd_ring(f) && G <= 65535;
      if (total > 0)
        dispatch(ctx, km ? conv_flip_kmajor_kernel : conv_flip_weight_kernel, dim3(unsigned((total + 255) / 256)),
                 dim3(256), 0, b, w2, G, Opg, Cpg, KV);
      launch_conv(ctx, f, 0, a, w2, bias, out, km);
      return;
    }
  }
  ConvK k{};
  k.a = a;
  k.b = b;
  k.bias = bias;
  if (omap) {
    if (mode != 0 || p.in[0] != 1 || p.out[0] != 1) fail(BG_E_UNSUPPORTED, "conv: an output map needs a 2-D forward");
    k.om = 1;
    k.om_sh = omap->sh;
    k.om_sw = omap->sw;
    k.om_ph = omap->ph;
    k.om_pw = omap->pw;
    k.om_H = omap->H;
    k.om_W = omap->W;
  }
  k.C = int(p.c);
  k.O = int(p.o);
  k.Cpg = int(p.c / p.groups);
  k.Opg = int(p.o / p.groups);
  k.D = int(p.in[0]);
  k.H = int(p.in[1]);
  k.W = int(p.in[2]);
  k.oD = int(p.out[0]);
  k.oH = int(p.out[1]);
  k.oW = int(p.out[2]);
  k.S = k.D * k.H * k.W;
  k.oS = k.oD * k.oH * k.oW;
  k.KD = int(p.k[0]);
  k.KH = int(p.k[1]);
  k.KW = int(p.k[2]);
  k.KV = k.KD * k.KH * k.KW;
  k.sd = int(p.stride[0]);
  k.sh = int(p.stride[1]);
  k.sw = int(p.stride[2]);
  k.pd = int(p.pad[0]);
  k.ph = int(p.pad[1]);
  k.pw = int(p.pad[2]);
  k.dd = int(p.dil[0]);
  k.dh = int(p.dil[1]);
  k.dw = int(p.dil[2]);
  const int64_t G = p.groups;
  if (mode == 0) {
    k.M = int(p.n * k.oS);
    k.NC = k.Opg;
    k.K = k.Cpg * k.KV;
  } else if (mode == 1) {
    k.M = int(p.n * k.S);
    k.NC = k.Cpg;
    k.K = k.Opg * k.KV;
  } else {
    k.M = k.Opg;
    k.NC = k.Cpg * k.KV;
    k.K = int(p.n * k.oS);
  }
  k.f_oS = make_fdiv(uint32_t(k.oS));
  k.f_oHW = make_fdiv(uint32_t(k.oH * k.oW));
  k.f_oW = make_fdiv(uint32_t(k.oW));
  k.f_S = make_fdiv(uint32_t(k.S));
  k.f_HW = make_fdiv(uint32_t(k.H * k.W));
  k.f_W = make_fdiv(uint32_t(k.W));
  k.f_KV = make_fdiv(uint32_t(k.KV));
  k.f_KHW = make_fdiv(uint32_t(k.KH * k.KW));
  k.f_KW = make_fdiv(uint32_t(k.KW));
  k.f_sd = make_fdiv(uint32_t(k.sd));
  k.f_sh = make_fdiv(uint32_t(k.sh));
  k.f_sw = make_fdiv(uint32_t(k.sw));
  // 128-wide tiles where the GEMM is large enough along that side and they
  // still give 512 workgroups; otherwise 64-wide ones (more workgroups in
  // flight: these kernels are bound by latency, not by the matrix core).
  int bm = k.M >= 128 ? 128 : 64;
  int bn = k.NC >= 128 ? 128 : 64;
  if (mode != 2 && ((k.M + bm - 1) / bm) * int64_t((k.NC + bn - 1) / bn) * G < 512) bm = bn = 64;
  k.tiles_m = int((k.M + bm - 1) / bm);
  const int64_t tiles_n = (k.NC + bn - 1) / bn;
  const int64_t tiles = int64_t(k.tiles_m) * tiles_n;
  if (mode == 2) {
    // Split the (n, p) reduction into at most 128 slices, whose partial sums
    // a second kernel adds in order, each over at least 8 k-steps, so that
    // about 768 workgroups run (three per CU).  A CU's time follows the
    // slices it holds times the slice length: on the ResNet 3x3 layers the
    // former rule (1024 workgroups, at most 64 slices) and a 512-workgroup
    // one each lose 5-20% somewhere (e.g. 32 x 128 x 28 x 28: 145 / 124 /
    // 119 us; 128 x 512 x 7 x 7: 406 / 491 / 400 us).
    const int64_t steps = (int64_t(k.K) + CBK - 1) / CBK;
    int64_t splits = std::max<int64_t>(1, std::min<int64_t>(768 / std::max<int64_t>(tiles * G, 1), steps / 8));
    splits = std::min<int64_t>(splits, 128);
    splits = std::min<int64_t>(splits, 65535 / G);
    const int64_t chunk_steps = (steps + splits - 1) / std::max<int64_t>(splits, 1);
    k.k_chunk = int(std::max<int64_t>(chunk_steps, 1) * CBK);
    k.ksplit = int(std::max<int64_t>(1, (int64_t(k.K) + k.k_chunk - 1) / k.k_chunk));
    k.part_stride = G * k.Opg * int64_t(k.NC);
    k.out = k.ksplit > 1 ? static_cast<float*>(scratch(ctx, size_t(k.ksplit * k.part_stride) * 4, 0)) : out;
  } else {
    k.ksplit = 1;
    k.k_chunk = k.K;
    k.part_stride = 0;
    k.out = out;
  }
  if (k.M == 0 || k.NC == 0) return;
  const dim3 grid(unsigned(tiles), unsigned(G * k.ksplit));
  // Forward: the LDS-ring kernel when x and w fit 32-bit byte offsets
  // (BG_CONV_RING=0 selects the register-staged kernel, for comparisons).
  const int64_t a_bytes = p.n * int64_t(k.C) * k.S * 4, b_bytes = int64_t(k.O) * k.K * 4;
  const bool ring = mode == 0 && conv_fwd_ring(p);
  if (b_kmajor && !ring) fail(BG_E_UNSUPPORTED, "conv: a k-major weight reached the register-staged kernel");
  if (ring) {
    // The weight copied k-major first (0.6 MB for a 128 x 128 3x3 layer;
    // the copy's grid takes the groups along z), unless it arrives so.
    if (b_kmajor) {
      k.b_kmajor = 1;
    } else if (G <= 65535) {
      float* wt = static_cast<float*>(scratch(ctx, size_t(b_bytes), 2));
      dispatch(ctx, conv_w_kmajor_kernel, dim3(unsigned((k.K + 31) / 32), unsigned((k.Opg + 31) / 32), unsigned(G)),
               dim3(256), 0, k.b, wt, k.Opg, k.K);
      k.b = wt;
      k.b_kmajor = 1;
    }
    const bool b16 = k.b_kmajor && k.Opg % 4 == 0;
    // 3x3, stride 1, dilation 1, 2-D: tiles of whole output rows fed from
    // input patches, 128 x 64 (eight wavefronts) where two channels' patches
    // fit 512 floats, the grid still has a workgroup per CU and the tiles
    // use as many of their rows as 64-row ones would, else 64 x 64 (a 7 x 7
    // image fills 49 of 128 rows but 49 of 64: 211 against 158 us on a
    // 32 x 512 x 7 x 7 layer).  BG_CONV_HALO=0 keeps the ring kernel; =64 or
    // =128 asks for that tile height where it fits, for comparisons.
    const char* halo_env = std::getenv("BG_CONV_HALO");
    const int halo_ask = halo_env ? std::atoi(halo_env) : -1;
    // Output rows per tile, 0 if two channels' patches do not fit the tile's
    // copies: 512 floats, or 1024 for 128-row tiles with two copies per
    // wavefront (output rows of 84 to 128).
    auto halo_rows = [&](int bm) {
      const int tr = k.oW > 0 ? bm / k.oW : 0;
      return tr > 0 && 2 * (tr + 2) * (k.oW + 2) <= (bm == 128 ? 1024 : 512) ? tr : 0;
    };
    if (b16 && k.D == 1 && k.oD == 1 && k.KD == 1 && k.KH == 3 && k.KW == 3 && k.sh == 1 && k.sw == 1 &&
        k.dh == 1 && k.dw == 1 && halo_ask != 0) {
      const int64_t tiles_n64 = (k.NC + 63) / 64;
      const int tr128 = halo_rows(128), tr64 = halo_rows(64);
      int bm = 0;
      if (halo_ask == 128 || halo_ask == 64) {
        bm = halo_rows(halo_ask) ? halo_ask : 0;
      } else if (tr128 && (!tr64 || (p.n * ((k.oH + tr128 - 1) / tr128) * tiles_n64 * G >= 256 &&
                                      int64_t((k.oH + tr64 - 1) / tr64) * 64 >=
                                          int64_t((k.oH + tr128 - 1) / tr128) * 128))) {
        // (rows of an image's 64-row tiles >= rows of its 128-row tiles: no
        // more of the larger tiles is left empty; rows past 64 have only
        // the larger tiles)
        bm = 128;
      } else if (tr64) {
        bm = 64;
      }
      if (bm) {
        const int tr = bm == 128 ? tr128 : tr64;
        k.tiles_m = int(p.n * ((k.oH + tr - 1) / tr));
        const dim3 hgrid(unsigned(int64_t(k.tiles_m) * tiles_n64), unsigned(G));
        if (bm == 128 && 2 * (tr + 2) * (k.oW + 2) > 512)
          dispatch(ctx, conv_fwd_halo_kernel<4, 2, 4, 2, 2>, hgrid, dim3(512), 0, k, uint32_t(a_bytes),
                   uint32_t(b_bytes), tr);
        else if (bm == 128)
          dispatch(ctx, conv_fwd_halo_kernel<4, 2, 4, 2, 1>, hgrid, dim3(512), 0, k, uint32_t(a_bytes),
                   uint32_t(b_bytes), tr);
        else
          dispatch(ctx, conv_fwd_halo_kernel<4, 2, 2, 2, 2>, hgrid, dim3(256), 0, k, uint32_t(a_bytes),
                   uint32_t(b_bytes), tr);
        hip_check(hipGetLastError(), "conv launch");
        return;
      }
    }
    auto go_ring = [&](auto kern) { dispatch(ctx, kern, grid, dim3(256), 0, k, uint32_t(a_bytes), uint32_t(b_bytes)); };
#define BG_RING(BM_, BN_)                                      \
  (b16 ? go_ring(conv_fwd_ring_kernel<BM_, BN_, 4, true>)      \
       : go_ring(conv_fwd_ring_kernel<BM_, BN_, 4, false>))
    if (bm == 128 && bn == 128) BG_RING(128, 128);
    else if (bm == 128) BG_RING(128, 64);
    else if (bn == 128) BG_RING(64, 128);
    else BG_RING(64, 64);
#undef BG_RING
    hip_check(hipGetLastError(), "conv launch");
    return;
  }
  auto go = [&](auto kern) { dispatch(ctx, kern, grid, dim3(256), 0, k); };
  auto pick = [&](auto mode_tag) {
    constexpr int MD = decltype(mode_tag)::value;
    if (bm == 128 && bn == 128) go(conv_gemm_kernel<MD, 128, 128>);
    else if (bm == 128) go(conv_gemm_kernel<MD, 128, 64>);
    else if (bn == 128) go(conv_gemm_kernel<MD, 64, 128>);
    else go(conv_gemm_kernel<MD, 64, 64>);
  };
  if (mode == 0) pick(std::integral_constant<int, MODE_FWD>{});
  else if (mode == 1) pick(std::integral_constant<int, MODE_DGRAD>{});
  else pick(std::integral_constant<int, MODE_WGRAD>{});
  if (mode == 2 && k.ksplit > 1) {
    const int64_t total = k.part_stride;
    dispatch(ctx, conv_split_reduce_kernel, dim3(unsigned((total + 255) / 256)), dim3(256), 0, k.out, out, total,
             k.ksplit);
  }
  hip_check(hipGetLastError(), "conv launch");
}

void launch_conv_bias_grad(bg_ctx* ctx, const float* dy, float* out, int64_t n, int64_t o, int64_t spatial) {
  if (o == 0) return;
  const int64_t rows = n * o;
  if (spatial % 4 == 0 && (reinterpret_cast<uintptr_t>(dy) & 15) == 0 && n * (spatial / 4) <= (int64_t(1) << 16) &&
      o <= 65535) {
    // Up to 1 MB per channel: one workgroup per channel, one launch.
    dispatch(ctx, conv_bias_grad1_kernel, dim3(unsigned(o)), dim3(1024), 0, reinterpret_cast<const float4*>(dy), out,
             n, o, spatial / 4);
    hip_check(hipGetLastError(), "conv bias-gradient launch");
    return;
  }
  float* part = static_cast<float*>(scratch(ctx, size_t(rows) * 4, 0));
  if (spatial % 4 == 0 && (reinterpret_cast<uintptr_t>(dy) & 15) == 0)
    dispatch(ctx, conv_row_sum4_kernel, dim3(unsigned((rows + 3) / 4)), dim3(256), 0,
             reinterpret_cast<const float4*>(dy), part, rows, spatial / 4);
  else
    dispatch(ctx, conv_row_sum_kernel, dim3(unsigned((rows + 3) / 4)), dim3(256), 0, dy, part, rows, spatial);
  dispatch(ctx, conv_bias_final_kernel, dim3(unsigned((o + 255) / 256)), dim3(256), 0, part, out, n, o);
  hip_check(hipGetLastError(), "conv bias-gradient launch");
}

}  // namespace bg
