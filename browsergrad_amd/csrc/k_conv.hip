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
// (full f32) in 64 x 64 workgroup tiles, four wavefronts of 32 x 32.
#include <algorithm>

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
  int64_t part_stride;  // WGRAD: floats per split slice (G * Opg * NC)
  FDiv f_oS, f_oHW, f_oW, f_S, f_HW, f_W, f_KV, f_KHW, f_KW, f_sd, f_sh, f_sw;
};

constexpr int CBM = 64, CBN = 64, CBK = 16, CLD = CBM + 1;

template <int MODE>
__global__ void __launch_bounds__(256) conv_gemm_kernel(ConvK P) {
  __shared__ float As[2][CBK * CLD];
  __shared__ float Bs[2][CBK * CLD];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int tm = int(blockIdx.x) % P.tiles_m, tn = int(blockIdx.x) / P.tiles_m;
  const int g = MODE == MODE_WGRAD ? int(blockIdx.y) / P.ksplit : int(blockIdx.y);
  const int split = MODE == MODE_WGRAD ? int(blockIdx.y) % P.ksplit : 0;
  const int m0 = tm * CBM, n0 = tn * CBN;
  const int kbeg = split * P.k_chunk;
  const int kend = min(P.K, kbeg + P.k_chunk);
  const int HW = P.H * P.W, oHW = P.oH * P.oW, KHW = P.KH * P.KW;

  // Per-thread fixed coordinates.  "Row-mapped" operands give lane l row
  // m0 + l and the k offsets wave + 4 i; "k-mapped" ones give every thread
  // the k offset tid & 15 and the rows (tid >> 4) + 16 i.
  const int kk_k = tid & 15;
  const int r_k = tid >> 4;
  // FWD / DGRAD A (row-mapped): output (FWD) or input (DGRAD) position.
  int64_t a_base = 0;
  int a_p0 = 0, a_p1 = 0, a_p2 = 0;
  bool a_row_ok = false;
  // WGRAD B rows (k-mapped): (c, kd, kh, kw) of the four columns j.
  int64_t wb_chan[4] = {0, 0, 0, 0};
  int wb_d[4] = {0, 0, 0, 0}, wb_h[4] = {0, 0, 0, 0}, wb_w[4] = {0, 0, 0, 0};
  bool wb_ok[4] = {false, false, false, false};
  if constexpr (MODE == MODE_FWD || MODE == MODE_DGRAD) {
    const int m = m0 + lane;
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
    for (int i = 0; i < 4; ++i) {
      const int j = n0 + r_k + 16 * i;
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

  float ra[4], rb[4];
  auto fetch = [&](int k0) {
    if constexpr (MODE == MODE_FWD) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {  // A: x gathered at (m, k)
        const int k = k0 + wave + 4 * i;
        float v = 0.f;
        if (a_row_ok && k < kend) {
          const uint32_t c = fdiv(uint32_t(k), P.f_KV), kv = uint32_t(k) - c * uint32_t(P.KV);
          const uint32_t kd = fdiv(kv, P.f_KHW), r = kv - kd * uint32_t(KHW);
          const uint32_t kh = fdiv(r, P.f_KW), kw = r - kh * uint32_t(P.KW);
          const int id = a_p0 + int(kd) * P.dd, ih = a_p1 + int(kh) * P.dh, iw = a_p2 + int(kw) * P.dw;
          if (unsigned(id) < unsigned(P.D) && unsigned(ih) < unsigned(P.H) && unsigned(iw) < unsigned(P.W))
            v = P.a[a_base + int64_t(c) * P.S + (int64_t(id) * P.H + ih) * P.W + iw];
        }
        ra[i] = v;
      }
      const int k = k0 + kk_k;
#pragma unroll
      for (int i = 0; i < 4; ++i) {  // B: w[g*Opg + o][k], contiguous along k
        const int o = n0 + r_k + 16 * i;
        rb[i] = (o < P.NC && k < kend) ? P.b[(int64_t(g) * P.Opg + o) * P.K + k] : 0.f;
      }
    } else if constexpr (MODE == MODE_DGRAD) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {  // A: dy gathered at (m, k = (o, kv))
        const int k = k0 + wave + 4 * i;
        float v = 0.f;
        if (a_row_ok && k < kend) {
          const uint32_t o = fdiv(uint32_t(k), P.f_KV), kv = uint32_t(k) - o * uint32_t(P.KV);
          const uint32_t kd = fdiv(kv, P.f_KHW), r = kv - kd * uint32_t(KHW);
          const uint32_t kh = fdiv(r, P.f_KW), kw = r - kh * uint32_t(P.KW);
          const int td = a_p0 - int(kd) * P.dd, th = a_p1 - int(kh) * P.dh, tw = a_p2 - int(kw) * P.dw;
          if (td >= 0 && th >= 0 && tw >= 0) {
            const uint32_t od = fdiv(uint32_t(td), P.f_sd), oh = fdiv(uint32_t(th), P.f_sh),
                           ow = fdiv(uint32_t(tw), P.f_sw);
            if (od * uint32_t(P.sd) == uint32_t(td) && oh * uint32_t(P.sh) == uint32_t(th) &&
                ow * uint32_t(P.sw) == uint32_t(tw) && od < uint32_t(P.oD) && oh < uint32_t(P.oH) &&
                ow < uint32_t(P.oW))
              v = P.a[a_base + int64_t(o) * P.oS + (int64_t(od) * P.oH + oh) * P.oW + ow];
          }
        }
        ra[i] = v;
      }
      const int k = k0 + kk_k;
      const bool k_ok = k < kend;
      const uint32_t kc = k_ok ? uint32_t(k) : 0u;
      const uint32_t o = fdiv(kc, P.f_KV), kv = kc - o * uint32_t(P.KV);
#pragma unroll
      for (int i = 0; i < 4; ++i) {  // B: w[g*Opg + o][c][kv]
        const int c = n0 + r_k + 16 * i;
        rb[i] = (c < P.NC && k_ok) ? P.b[((int64_t(g) * P.Opg + o) * P.Cpg + c) * P.KV + kv] : 0.f;
      }
    } else {
      const int k = k0 + kk_k;
      const bool k_ok = k < kend;
      const uint32_t kc = k_ok ? uint32_t(k) : 0u;
      const uint32_t n = fdiv(kc, P.f_oS), sp = kc - n * uint32_t(P.oS);
#pragma unroll
      for (int i = 0; i < 4; ++i) {  // A: dy[n][g*Opg + o][sp]
        const int o = m0 + r_k + 16 * i;
        ra[i] = (o < P.M && k_ok) ? P.a[(int64_t(n) * P.O + int64_t(g) * P.Opg + o) * P.oS + sp] : 0.f;
      }
      const uint32_t od = fdiv(sp, P.f_oHW), r = sp - od * uint32_t(oHW);
      const uint32_t oh = fdiv(r, P.f_oW), ow = r - oh * uint32_t(P.oW);
      const int64_t xn = int64_t(n) * P.C * P.S;
#pragma unroll
      for (int i = 0; i < 4; ++i) {  // B: x gathered at (k = (n, p), j = (c, kv))
        const int id = int(od) * P.sd + wb_d[i], ih = int(oh) * P.sh + wb_h[i], iw = int(ow) * P.sw + wb_w[i];
        const bool ok = wb_ok[i] && k_ok && unsigned(id) < unsigned(P.D) && unsigned(ih) < unsigned(P.H) &&
                        unsigned(iw) < unsigned(P.W);
        rb[i] = ok ? P.b[xn + wb_chan[i] + (int64_t(id) * P.H + ih) * P.W + iw] : 0.f;
      }
    }
  };
  auto commit = [&](int buf) {
    if constexpr (MODE == MODE_WGRAD) {
#pragma unroll
      for (int i = 0; i < 4; ++i) As[buf][kk_k * CLD + r_k + 16 * i] = ra[i];
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) As[buf][(wave + 4 * i) * CLD + lane] = ra[i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) Bs[buf][kk_k * CLD + r_k + 16 * i] = rb[i];
  };

  float16v acc;
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.f;
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
      const float af = As[buf][k * CLD + wm * 32 + (lane & 31)];
      const float bf = Bs[buf][k * CLD + wn * 32 + (lane & 31)];
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(af, bf, acc, 0, 0, 0);
    }
    if (kt + 1 < nk) commit(buf ^ 1);
    __syncthreads();
  }

  // Lane l holds rows 8*(e/4) + (e%4) + 4*(l/32) and column l%32 of its
  // wavefront's 32 x 32 tile.
  const int col = n0 + wn * 32 + (lane & 31);
  if (col >= P.NC) return;
  float bz = 0.f;
  if constexpr (MODE == MODE_FWD) {
    if (P.bias) bz = P.bias[int64_t(g) * P.Opg + col];
  } else if constexpr (MODE == MODE_DGRAD) {
    if (P.bias) bz = P.bias[int64_t(g) * P.Cpg + col];
  }
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int row = m0 + wm * 32 + 8 * (e >> 2) + (e & 3) + 4 * (lane >> 5);
    if (row >= P.M) continue;
    if constexpr (MODE == MODE_FWD) {
      const uint32_t n = fdiv(uint32_t(row), P.f_oS), sp = uint32_t(row) - n * uint32_t(P.oS);
      P.out[(int64_t(n) * P.O + int64_t(g) * P.Opg + col) * P.oS + sp] = acc[e] + bz;
    } else if constexpr (MODE == MODE_DGRAD) {
      const uint32_t n = fdiv(uint32_t(row), P.f_S), sp = uint32_t(row) - n * uint32_t(P.S);
      P.out[(int64_t(n) * P.C + int64_t(g) * P.Cpg + col) * P.S + sp] = acc[e] + bz;
    } else {
      P.out[int64_t(split) * P.part_stride + (int64_t(g) * P.Opg + row) * P.NC + col] = acc[e];
    }
  }
}

// dw[i] = sum over split slices (in order) of part[s][i].
__global__ void __launch_bounds__(256) conv_split_reduce_kernel(const float* __restrict__ part,
                                                                float* __restrict__ out, int64_t total,
                                                                int splits) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total) return;
  float acc = 0.f;
  for (int s = 0; s < splits; ++s) acc += part[int64_t(s) * total + i];
  out[i] = acc;
}

// db[o] = sum over n and the spatial positions of dy[n][o][.]: one
// workgroup per channel, a fixed-order LDS tree at the end.
__global__ void __launch_bounds__(256) conv_bias_grad_kernel(const float* __restrict__ dy, float* __restrict__ db,
                                                             int64_t n, int64_t o_count, int64_t spatial) {
  __shared__ float sm[256];
  const int64_t o = blockIdx.x;
  float acc = 0.f;
  for (int64_t b = 0; b < n; ++b) {
    const float* row = dy + (b * o_count + o) * spatial;
    for (int64_t p = threadIdx.x; p < spatial; p += 256) acc += row[p];
  }
  sm[threadIdx.x] = acc;
  __syncthreads();
  for (int w = 128; w >= 1; w >>= 1) {
    if (int(threadIdx.x) < w) sm[threadIdx.x] += sm[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) db[o] = sm[0];
}

}  // namespace

namespace bg {

void launch_conv(bg_ctx* ctx, const ConvProblem& p, int mode, const float* a, const float* b, const float* bias,
                 float* out) {
  ConvK k{};
  k.a = a;
  k.b = b;
  k.bias = bias;
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
  k.tiles_m = int((k.M + CBM - 1) / CBM);
  const int64_t tiles_n = (k.NC + CBN - 1) / CBN;
  const int64_t tiles = int64_t(k.tiles_m) * tiles_n;
  if (mode == 2) {
    // Split the (n, p) reduction so that about 2048 workgroups run, each
    // over at least 8 k-steps; slices are summed in order afterwards.
    const int64_t steps = (int64_t(k.K) + CBK - 1) / CBK;
    int64_t splits = std::max<int64_t>(1, std::min<int64_t>(2048 / std::max<int64_t>(tiles * G, 1), steps / 8));
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
  if (mode == 0)
    dispatch(ctx, conv_gemm_kernel<MODE_FWD>, grid, dim3(256), 0, k);
  else if (mode == 1)
    dispatch(ctx, conv_gemm_kernel<MODE_DGRAD>, grid, dim3(256), 0, k);
  else
    dispatch(ctx, conv_gemm_kernel<MODE_WGRAD>, grid, dim3(256), 0, k);
  if (mode == 2 && k.ksplit > 1) {
    const int64_t total = k.part_stride;
    dispatch(ctx, conv_split_reduce_kernel, dim3(unsigned((total + 255) / 256)), dim3(256), 0, k.out, out, total,
             k.ksplit);
  }
  hip_check(hipGetLastError(), "conv launch");
}

void launch_conv_bias_grad(bg_ctx* ctx, const float* dy, float* out, int64_t n, int64_t o, int64_t spatial) {
  if (o == 0) return;
  dispatch(ctx, conv_bias_grad_kernel, dim3(unsigned(o)), dim3(256), 0, dy, out, n, o, spatial);
  hip_check(hipGetLastError(), "conv bias-gradient launch");
}

}  // namespace bg
