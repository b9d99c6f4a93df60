// Device helpers shared by the kernel translation units.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>

namespace bgk {

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t v) {
  return __uint_as_float(uint32_t(v) << 16);
}

// Round-to-nearest-even f32 -> bf16 bits (gfx950 v_cvt_pk_bf16_f32; NaN
// stays a quiet NaN).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// Round-to-nearest-even f32 -> f16 bits (v_cvt_f16_f32).
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t v) {
  return static_cast<float>(__builtin_bit_cast(_Float16, v));
}

// x + (x of another lane chosen by the DPP control word CTRL).  Every
// control used below names a lane inside the same row of 16, so all lanes
// read a valid source.
template <int CTRL>
__device__ __forceinline__ float dpp_add(float x) {
  return x + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

// Sum over the 64 lanes of a wavefront, the same value in every lane: inside
// each row of 16 lanes, quad_perm swaps of neighbours (0xB1) and pairs (0x4E)
// and row rotations by 4 (0x124) and 8 (0x128); then the four row sums as
// read from lanes 0, 16, 32, 48.  Costs no LDS traffic, unlike ds_bpermute
// shuffles.
__device__ __forceinline__ float wave_sum(float x) {
  x = dpp_add<0xB1>(x);
  x = dpp_add<0x4E>(x);
  x = dpp_add<0x124>(x);
  x = dpp_add<0x128>(x);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 48));
  return (r0 + r1) + (r2 + r3);
}

// dtype codes follow include/bghip.h (0 f32, 1 f16, 2 bf16).
__device__ __forceinline__ float load_as_f32(const void* p, int dtype, int64_t i) {
  if (dtype == 0) return static_cast<const float*>(p)[i];
  const uint16_t v = static_cast<const uint16_t*>(p)[i];
  return dtype == 1 ? f16_bits_to_f32(v) : bf16_bits_to_f32(v);
}

__device__ __forceinline__ void store_from_f32(void* p, int dtype, int64_t i, float x) {
  if (dtype == 0) {
    static_cast<float*>(p)[i] = x;
  } else {
    static_cast<uint16_t*>(p)[i] = dtype == 1 ? f32_to_f16_bits(x) : f32_to_bf16_bits(x);
  }
}

// Round an f32 value through the 16-bit dtype (1 f16, 2 bf16) and back.
__device__ __forceinline__ float round_through(float x, int dtype) {
  if (dtype == 1) return static_cast<float>(static_cast<_Float16>(x));
  if (dtype == 2) return static_cast<float>(static_cast<__bf16>(x));
  return x;
}

// The reference's tanh-approximate GELU (_functional.py:123-134, tanh from
// _functional.py:115-120): 0.5*x * (1 + tanh u), u = c*(x + ((0.044715*x)*x)*x),
// tanh u = (e^u - e^-u)/(e^u + e^-u), every op in f32.  Evaluated as the
// equal x * sigmoid(2u) = x / (1 + 2^(-s)), s = 2 log2(e) u = x (k0 + k1 x^2):
// one FMA, two multiplies, one v_exp_f32, one add, one v_rcp_f32 and a
// multiply, within a few ulp of the reference form, with no cancellation
// (2^(-s) -> 0 gives x, -> inf gives a signed 0, as the reference does).
// The reference is NaN exactly where one of its f32 exponentials overflows,
// |u| >= 88.72283935546875 (the least f32 whose exp rounds past FLT_MAX),
// and for NaN or infinite x.  Its f32 u(x) is odd and non-decreasing, so
// that set is |x| >= 0x1.9ff1b8p+3 (12.998256683..., found by walking every
// f32 through the reference's op order; the edge test in the GPU suite
// checks the f32 values on both sides) or x NaN.
__device__ __forceinline__ float gelu_tanh(float x) {
  const float k0 = 2.302208198144325f;   // 2 log2(e) sqrt(2/pi)
  const float k1 = 0.1029432395800235f;  // k0 * 0.044715
  const float neg_s = x * __builtin_fmaf(x * x, -k1, -k0);
  const float g = x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(neg_s));
  return fabsf(x) < 0x1.9ff1b8p+3f ? g : __builtin_nanf("");
}

// Raw buffer descriptor in four SGPRs: 48-bit base, stride 0, size in bytes
// (offsets at or beyond it read zeros), gfx950 raw-buffer format word.
typedef uint32_t sgpr4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ sgpr4_t buffer_rsrc(const void* base, uint32_t nbytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  return sgpr4_t{uint32_t(a), uint32_t(a >> 32) & 0xffffu, nbytes, 0x00020000u};
}

// LDS byte address of a pointer into __shared__ memory.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const char*)(p)));
}

// buffer_load_dwordx4 ... lds: lane L copies the 16 bytes at voffset +
// soffset of the buffer to LDS byte lds_base + 16 L (lds_base wave-uniform).
// Issued as inline assembly on purpose: the compiler cannot tell which LDS
// bytes such a copy writes, so for the builtin form it makes every later LDS
// read wait for all outstanding copies (vmcnt(0)), which serialises a
// multi-stage prefetch ring.  Callers order LDS reads after the copies they
// need with s_waitcnt vmcnt(N) and a workgroup barrier themselves.
// M0 holds the LDS base (set by the compiler for the asm operand).  The
// compiler does not look inside the asm for hazards, so the asm opens with
// five wait states: a VMEM instruction must not read an SGPR (descriptor,
// soffset) fewer than five wait states after a VALU wrote it (for example a
// v_readlane restoring a spilled SGPR), and M0 needs one after its write.
__device__ __forceinline__ void dma16_to_lds(uint32_t lds_base, uint32_t voffset, sgpr4_t rsrc,
                                             uint32_t soffset) {
  asm volatile(
      "s_nop 4\n\t"
      "buffer_load_dwordx4 %1, %2, %3 offen lds"
      :
      : "{m0}"(lds_base), "v"(voffset), "s"(rsrc), "s"(soffset)
      : "memory");
}

}  // namespace bgk
