// Building blocks shared by the decode-shaped kernels (v_mfma_f32_16x16x32 on gfx950):
// the MFMA wrapper per activation type, the in-register weight unpack / conversion into
// B operands, and the activation column order that matches them.
#pragma once

#include "lsq_common.h"
#include "lsq_internal.h"
#include "lsq_decode.h"

namespace lsq {
namespace {

__host__ __device__ constexpr int64_t align16(int64_t v) { return (v + 15) & ~int64_t(15); }

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

template <int DT> struct Mma;

template <> struct Mma<LSQ_BF16> {
  static constexpr uint32_t kMagic = 0x43004300u;  // bf16 pair (128, 128)
  static constexpr uint32_t kOne2 = 0x3F803F80u;   // bf16 pair (1, 1)
  static constexpr float kOff4 = 136.f;            // 128 + the nibble bias 8
  static __device__ __forceinline__ f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                    __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
  }
  static __device__ __forceinline__ float lo(uint32_t v) { return __uint_as_float(v << 16); }
  static __device__ __forceinline__ float hi(uint32_t v) { return __uint_as_float(v & 0xFFFF0000u); }
};

template <> struct Mma<LSQ_F16> {
  static constexpr uint32_t kMagic = 0x64006400u;  // fp16 pair (1024, 1024)
  static constexpr uint32_t kOne2 = 0x3C003C00u;   // fp16 pair (1, 1)
  static constexpr float kOff4 = 1032.f;           // 1024 + the nibble bias 8
  static __device__ __forceinline__ f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                   __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  // Round-toward-zero is exact here: the inputs are integers with |v| <= 128.
  static __device__ __forceinline__ uint32_t pack2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a, b));
  }
  static __device__ __forceinline__ float lo(uint32_t v) { return f16_to_f32(v & 0xFFFFu); }
  static __device__ __forceinline__ float hi(uint32_t v) { return f16_to_f32(v >> 16); }
};

// 8 nibbles of one dword -> B operand of one MFMA: pair j = (nibble j, nibble j + 4),
// each as the exact value 128 + u (bf16) / 1024 + u (fp16). `mask` = 0x000F000F and
// `magic` = Mma<DT>::kMagic are passed in registers (see the main loop).
__device__ __forceinline__ u32x4 unpack_w4(uint32_t w, uint32_t mask, uint32_t magic) {
  u32x4 b;
  b[0] = (w & mask) | magic;
  b[1] = ((w >> 4) & mask) | magic;
  b[2] = ((w >> 8) & mask) | magic;
  b[3] = ((w >> 12) & mask) | magic;
  return b;
}

// 8 signed bytes (two dwords, column order) -> B operand, exact.
template <int DT>
__device__ __forceinline__ u32x4 convert_w8(uint32_t w0, uint32_t w1) {
  u32x4 b;
  b[0] = Mma<DT>::pack2(static_cast<float>(static_cast<int8_t>(w0)),
                        static_cast<float>(static_cast<int8_t>(w0 >> 8)));
  b[1] = Mma<DT>::pack2(static_cast<float>(static_cast<int8_t>(w0 >> 16)),
                        static_cast<float>(static_cast<int8_t>(w0 >> 24)));
  b[2] = Mma<DT>::pack2(static_cast<float>(static_cast<int8_t>(w1)),
                        static_cast<float>(static_cast<int8_t>(w1 >> 8)));
  b[3] = Mma<DT>::pack2(static_cast<float>(static_cast<int8_t>(w1 >> 16)),
                        static_cast<float>(static_cast<int8_t>(w1 >> 24)));
  return b;
}

// 8 activations (x0..x7) reordered to (x0,x4,x1,x5,x2,x6,x3,x7), the order unpack_w4
// yields for a canonical dword, where nibble p is column p.
__device__ __forceinline__ u32x4 permute_canon(u32x4 a) {
  u32x4 r;
  r[0] = __builtin_amdgcn_perm(a[2], a[0], 0x05040100u);
  r[1] = __builtin_amdgcn_perm(a[2], a[0], 0x07060302u);
  r[2] = __builtin_amdgcn_perm(a[3], a[1], 0x05040100u);
  r[3] = __builtin_amdgcn_perm(a[3], a[1], 0x07060302u);
  return r;
}

// Column (within a 128-column k tile) of the first of the 8 activations lane-quad q
// feeds to MFMA d. INT4 and tiled INT8: lane quad q owns columns [32q, 32q + 32), MFMA d
// takes columns 32q + 8d .. +7. Canonical INT8: the two 16-byte loads cover columns
// [16q, 16q + 16) and [64 + 16q, 64 + 16q + 16).
template <int KIND>
__device__ __forceinline__ int a_col(int q, int d) {
  return KIND == kW8 ? (d >> 1) * 64 + q * 16 + (d & 1) * 8 : q * 32 + d * 8;
}

}  // namespace
}  // namespace lsq
