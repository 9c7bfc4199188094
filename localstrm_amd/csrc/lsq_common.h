// Shared device helpers for the gfx950 weight-only quantized linear kernels.
//
// Numeric contract (reference: src/kernels/quantization.py:104-141):
//   dequant:  W[n,k] = round_T( float(q) * round_T(scale) )   -- one product, no FMA
//   linear:   y[m,n] = round_T( sum_k x[m,k] * W[n,k]  (fp32)  + round_T(bias[n]) )
// round_T is IEEE round-to-nearest-even into the activation type T; on gfx950 the
// fp32->bf16 conversion is the hardware v_cvt_pk_bf16_f32 (RNE, NaN-preserving) and
// fp32->fp16 is v_cvt_f16_f32 under the default RNE mode.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "../../include/localstrm_amd.h"

namespace lsq {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// ---------------------------------------------------------------- scalar conversions

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  __hip_bfloat16 h = __float2bfloat16(f);
  return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ float f16_to_f32(uint16_t b) {
  return __half2float(__builtin_bit_cast(__half, b));
}

__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  return __builtin_bit_cast(uint16_t, __float2half(f));
}

// Activation/output dtype traits. `storage` is the element type in memory.
template <int DT> struct Act;

template <> struct Act<LSQ_F32> {
  using storage = float;
  static __device__ __forceinline__ float load(const storage* p) { return *p; }
  static __device__ __forceinline__ float to_f32(storage v) { return v; }
  static __device__ __forceinline__ storage from_f32(float v) { return v; }
  static __device__ __forceinline__ float round(float v) { return v; }
};

template <> struct Act<LSQ_F16> {
  using storage = uint16_t;
  static __device__ __forceinline__ float to_f32(storage v) { return f16_to_f32(v); }
  static __device__ __forceinline__ storage from_f32(float v) { return f32_to_f16(v); }
  static __device__ __forceinline__ float round(float v) { return f16_to_f32(f32_to_f16(v)); }
};

template <> struct Act<LSQ_BF16> {
  using storage = uint16_t;
  static __device__ __forceinline__ float to_f32(storage v) { return bf16_to_f32(v); }
  static __device__ __forceinline__ storage from_f32(float v) { return f32_to_bf16(v); }
  static __device__ __forceinline__ float round(float v) { return bf16_to_f32(f32_to_bf16(v)); }
};

// Read element i of a scale / bias array stored with dtype code `dt`, as fp32.
__device__ __forceinline__ float load_as_f32(const void* p, int dt, int64_t i) {
  if (dt == LSQ_F32) return static_cast<const float*>(p)[i];
  const uint16_t v = static_cast<const uint16_t*>(p)[i];
  return dt == LSQ_BF16 ? bf16_to_f32(v) : f16_to_f32(v);
}

// Product q * s with a single rounding to fp32 (never contracted into an FMA).
__device__ __forceinline__ float mul_rn(float a, float b) { return __fmul_rn(a, b); }

// fp32 product and sum that the compiler may not fuse with a neighbouring add or
// multiply (the reference evaluates them as separate elementwise kernels, each rounding
// once).
__device__ __forceinline__ float mul_nc(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ __forceinline__ float add_nc(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}

// The reference dequant closed form for one element, returned as the fp32 value of the
// T-typed result: round_T( float(q) * s_T ), s_T already rounded to T.
template <int DT>
__device__ __forceinline__ float dequant_elem(int q, float s_T) {
  return Act<DT>::round(mul_rn(static_cast<float>(q), s_T));
}

// The value of x as computed, kept from being folded into a following conversion: gfx950
// can multiply (or FMA) and round straight to fp16 / bf16 in one instruction (v_fma_mix),
// which rounds once where the separate fp32 operation and conversion round twice. Code
// that must round like an fp32 result converted to T passes the fp32 value through here.
// (Not volatile: a volatile asm would also pin the surrounding memory operations in
// place, serializing loads around every use.)
__device__ __forceinline__ float opaque(float x) {
  __asm__("" : "+v"(x));
  return x;
}

// ---------------------------------------------------------------- W8A8 activations
// Per-token scale from the row's max|x| (as fp32): clamp(round_T(max * fp32(1/127)),
// min = round_T(1e-8)), the GPU evaluation of quantization.py:412-413 (torch multiplies
// by the fp32 reciprocal when dividing a tensor by a Python scalar). NaN stays NaN.
template <int DT>
__device__ __forceinline__ float a8_scale(float mx) {
  constexpr float kInv127 = 1.0f / 127.0f;
  const float s = Act<DT>::round(opaque(mul_nc(mx, kInv127)));  // fp32 product, then T
  const float smin = Act<DT>::round(1e-8f);
  return s < smin ? smin : s;
}

// clamp(rint(v / s), -128, 127) with IEEE division (quantization.py:414); NaN (0 / 0 when
// a fp16 scale is 0) becomes 0.
__device__ __forceinline__ int quant_i8(float v, float s) {
  float q = __builtin_rintf(__fdiv_rn(v, s));
  if (q != q) return 0;
  q = q < -128.f ? -128.f : (q > 127.f ? 127.f : q);
  return static_cast<int>(q);
}

// quant_i8(v, s) with a product instead of the division: t = v * rcp(s) is within 2^-14
// of v / s (|v / s| < 192 by construction of s, fp16 subnormal scales included; v_rcp_f32
// is accurate to 1 ulp), so when t is more than 2^-10 from every half-integer, rint of
// the IEEE quotient v / s equals rint(t). Otherwise (a near-tie, s = 0, or a non-finite
// value, where t - rint(t) is NaN) the exact division decides. `r` is rcp(s), once per row.
__device__ __forceinline__ int quant_i8_fast(float v, float s, float r) {
  const float t = mul_nc(v, r);
  const float q = __builtin_rintf(t);
  if (!(__builtin_fabsf(t - q) < 0.5f - 0x1p-10f)) return quant_i8(v, s);
  return static_cast<int>(q < -128.f ? -128.f : (q > 127.f ? 127.f : q));
}

// ---------------------------------------------------------------- wavefront helpers

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Non-temporal 16-byte global load: weights are streamed exactly once per call.
__device__ __forceinline__ u32x4 load_nt_u32x4(const void* p) {
  return __builtin_nontemporal_load(static_cast<const u32x4*>(p));
}

__device__ __forceinline__ u32x4 load_u32x4(const void* p) {
  return *static_cast<const u32x4*>(p);
}

// ---------------------------------------------------------------- buffer loads
// The fast kernels read global memory through buffer descriptors bounding a region the
// workgroup owns; a load at an offset past the bound returns zero without touching
// memory, so out-of-range rows and pipeline loads past the end need no clamping or
// branches.
using rsrc_t = __amdgpu_buffer_rsrc_t;
constexpr int kRsrcWord3 = 0x00020000;  // gfx9-family descriptor word 3: raw 32-bit dwords
constexpr uint32_t kOOB = 0x80000000u;  // past every descriptor's range
constexpr int kNT = 2;                  // cache policy: non-temporal (weights, read once)

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, kRsrcWord3);
}

template <int AUX>
__device__ __forceinline__ u32x4 bload16(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, AUX);
}

__device__ __forceinline__ uint32_t bload4(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}

// Buffer loads into LDS (buffer_load_dwordx4 ... lds: 16 bytes per lane, lane l's bytes
// at the wave's LDS address + 16 l) that the compiler does not see. Through the builtin,
// every LDS read after such a load waits for it to land (the compiler cannot tell which
// LDS bytes it writes), so a DMA issued several pipeline steps ahead is drained at the
// next step. Written as assembly the load is invisible to that analysis; the caller
// waits for it itself (s_waitcnt vmcnt with an exact count) before the barrier that
// publishes the data, and keeps it out of the LDS it reads meanwhile. The compiler's
// own vmcnt waits stay correct: loads it does not know of only make them wait longer.
using rsrc4_t = int __attribute__((ext_vector_type(4)));

__device__ __forceinline__ rsrc4_t make_rsrc4(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  return rsrc4_t{static_cast<int>(static_cast<uint32_t>(a)), static_cast<int>((a >> 32) & 0xFFFFu),
                 static_cast<int>(bytes), kRsrcWord3};
}

// M0 holds the LDS address. The compiler reserves M0 and warns about the clobber; the
// kernels using this helper have no other M0 use (they issue no builtin LDS DMA, GWS or
// LDS-parameter instruction), so nothing live is lost.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16_async(rsrc4_t r, void* lds, uint32_t voff, uint32_t soff) {
  const uint32_t m0 = static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) void*)lds));
  asm volatile(
      "s_mov_b32 m0, %3\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %0, %1, %2 offen lds"
      :
      : "v"(voff), "s"(r), "s"(soff), "s"(m0)
      : "memory", "m0");
}
#pragma clang diagnostic pop

// Workgroup barrier that orders LDS only: the compiler's __syncthreads() also waits for
// every outstanding global load, which would drain the weight pipeline.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// fp32 value of element `half` (0 or 1) of a dword of 16-bit floats, or of an fp32 dword.
__device__ __forceinline__ float dword_elem(uint32_t w, int half, int dt) {
  if (dt == LSQ_F32) return __uint_as_float(w);
  const uint32_t h = half ? (w >> 16) : (w & 0xFFFFu);
  return dt == LSQ_BF16 ? __uint_as_float(h << 16) : f16_to_f32(static_cast<uint16_t>(h));
}

}  // namespace lsq
