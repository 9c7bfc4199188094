// Weight-only quantized linear layer: y = x W^T + b with INT8 / INT4 W (gfx950).
//
// GPU form of QuantizedLinear.forward (src/kernels/quantization.py:129-141), which in the
// reference materializes W = dequantize(x.dtype) and then calls F.linear. Here the
// weights are never materialized in HBM:
//
//  * decode kernel (M <= 64, fp16/bf16, K % 128 == 0): one workgroup owns RT tiles of
//    16 output rows; its waves split the K dimension in 128-column tiles. Each lane
//    streams 16 bytes of weights per tile (a whole 1 KB tile per wavefront load for the
//    tiled INT4 layout), unpacks them in registers and feeds v_mfma_f32_16x16x32_{bf16,f16}
//    with the activations as the A operand (M padded to 16). Partial sums of the waves are
//    reduced through LDS. Scales are applied in fp32 registers after the MFMA (per
//    128-column group) instead of to every weight.
//  * generic kernel (any dtype / shape / group): exact dequant per element, fp32 FMA,
//    wavefront reduction. Used for fp32 activations and shapes the fast kernels do not
//    cover.
//  * prefill GEMM (M > 64): lsq_gemm.hip.
//
// INT4 unpack trick: a nibble u in [0, 15] OR-ed into the mantissa of bf16 128.0
// (0x4300) gives the exact bf16 value 128 + u (fp16: 0x6400 -> 1024 + u). The constant
// offset (128 + 8, resp. 1024 + 8) is removed by seeding each 128-column accumulation
// with one extra MFMA against a B operand filled with -(offset), which yields
// -(offset) * sum_k x[m,k] in exactly the accumulator layout.

#include "lsq_common.h"
#include "lsq_internal.h"
#include "lsq_gemm.h"
#include "lsq_decode.h"

#include <cstdlib>
#include <cstring>

namespace lsq {

// ============================================================ generic kernel

constexpr int kGenMB = 8;  // activation rows per wavefront

template <int DT, bool W4>
__global__ void __launch_bounds__(256) linear_generic_kernel(
    const typename Act<DT>::storage* __restrict__ x, int64_t ldx, const void* __restrict__ w,
    const void* __restrict__ scale, int scale_dt, int64_t group, const void* __restrict__ bias,
    int bias_dt, typename Act<DT>::storage* __restrict__ y, int64_t ldy, int64_t M, int64_t N,
    int64_t K) {
  const int lane = threadIdx.x & 63;
  const int64_t n = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t m0 = blockIdx.y * (int64_t)kGenMB;
  if (n >= N) return;
  const int64_t ng = (K + group - 1) / group;
  float acc[kGenMB];
#pragma unroll
  for (int i = 0; i < kGenMB; ++i) acc[i] = 0.f;
  for (int64_t k = lane; k < K; k += 64) {
    int q;
    float s;
    if (W4) {
      const uint8_t byte = static_cast<const uint8_t*>(w)[n * ((K + 1) / 2) + (k >> 1)];
      q = static_cast<int>((k & 1) ? (byte >> 4) : (byte & 0xF)) - 8;
      s = load_as_f32(scale, scale_dt, n * ng + k / group);
    } else {
      q = static_cast<const int8_t*>(w)[n * K + k];
      s = load_as_f32(scale, scale_dt, n);
    }
    const float wv = dequant_elem<DT>(q, Act<DT>::round(s));
#pragma unroll
    for (int i = 0; i < kGenMB; ++i) {
      if (m0 + i < M) acc[i] = fmaf(Act<DT>::to_f32(x[(m0 + i) * ldx + k]), wv, acc[i]);
    }
  }
  const float b = bias ? Act<DT>::round(load_as_f32(bias, bias_dt, n)) : 0.f;
#pragma unroll
  for (int i = 0; i < kGenMB; ++i) {
    const float v = wave_sum(acc[i]);
    if (lane == 0 && m0 + i < M) y[(m0 + i) * ldy + n] = Act<DT>::from_f32(v + b);
  }
}

// ============================================================ decode kernel

template <int DT> struct Mfma;

template <> struct Mfma<LSQ_BF16> {
  static constexpr uint32_t kMagic = 0x43004300u;  // bf16 pair (128, 128)
  static constexpr uint32_t kNegOff = 0xC308C308u; // bf16 pair (-136, -136)
  static __device__ __forceinline__ f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                    __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack2(float a, float b) {
    return static_cast<uint32_t>(f32_to_bf16(a)) | (static_cast<uint32_t>(f32_to_bf16(b)) << 16);
  }
};

template <> struct Mfma<LSQ_F16> {
  static constexpr uint32_t kMagic = 0x64006400u;  // fp16 pair (1024, 1024)
  static constexpr uint32_t kNegOff = 0xE408E408u; // fp16 pair (-1032, -1032)
  static __device__ __forceinline__ f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                   __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a, b));
  }
};

// 8 nibbles -> B operand of one 16x16x32 MFMA. Pair j is (nibble j, nibble j + 4).
template <int DT>
__device__ __forceinline__ u32x4 unpack_nibbles(uint32_t w) {
  u32x4 b;
  b[0] = (w & 0x000F000Fu) | Mfma<DT>::kMagic;
  b[1] = ((w >> 4) & 0x000F000Fu) | Mfma<DT>::kMagic;
  b[2] = ((w >> 8) & 0x000F000Fu) | Mfma<DT>::kMagic;
  b[3] = ((w >> 12) & 0x000F000Fu) | Mfma<DT>::kMagic;
  return b;
}

// 8 signed bytes (two dwords, natural column order) -> B operand, exact in bf16/fp16.
template <int DT>
__device__ __forceinline__ u32x4 convert_bytes(uint32_t w0, uint32_t w1) {
  u32x4 b;
  b[0] = Mfma<DT>::pack2(static_cast<float>(static_cast<int8_t>(w0)),
                         static_cast<float>(static_cast<int8_t>(w0 >> 8)));
  b[1] = Mfma<DT>::pack2(static_cast<float>(static_cast<int8_t>(w0 >> 16)),
                         static_cast<float>(static_cast<int8_t>(w0 >> 24)));
  b[2] = Mfma<DT>::pack2(static_cast<float>(static_cast<int8_t>(w1)),
                         static_cast<float>(static_cast<int8_t>(w1 >> 8)));
  b[3] = Mfma<DT>::pack2(static_cast<float>(static_cast<int8_t>(w1 >> 16)),
                         static_cast<float>(static_cast<int8_t>(w1 >> 24)));
  return b;
}

// Activation pairs (x_j, x_{j+4}) to match unpack_nibbles() on the canonical layout,
// where nibble p of a dword is column p.
__device__ __forceinline__ u32x4 permute_canon(u32x4 a) {
  u32x4 r;
  r[0] = __builtin_amdgcn_perm(a[2], a[0], 0x05040100u);
  r[1] = __builtin_amdgcn_perm(a[2], a[0], 0x07060302u);
  r[2] = __builtin_amdgcn_perm(a[3], a[1], 0x05040100u);
  r[3] = __builtin_amdgcn_perm(a[3], a[1], 0x07060302u);
  return r;
}

template <int DT, int KIND, int MT, int RT, int WAVES, int UNR, bool GROUPED>
__global__ void __launch_bounds__(64 * WAVES) linear_decode_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const uint8_t* __restrict__ w,
    const void* __restrict__ scale, int scale_dt, int64_t group, int64_t ngroups,
    const void* __restrict__ bias, int bias_dt, uint16_t* __restrict__ y, int64_t ldy, int M,
    int N, int K) {
  constexpr bool kW4 = KIND != kW8;
  constexpr int kBDw = kW4 ? 1 : 2;  // u32x4 weight loads per lane per (row tile, k tile)
  __shared__ float red[WAVES * RT * MT * 4 * 64];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane & 15;
  const int q = lane >> 4;
  const int nkt = K / kTileK;
  const int nrt = (N + kTileN - 1) / kTileN;
  const int rt0 = blockIdx.x * RT;

  f32x4 acc[RT][MT];
  f32x4 xoff[MT];  // per-channel INT4: running -(offset) * sum(x)
#pragma unroll
  for (int i = 0; i < RT; ++i)
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < MT; ++j) xoff[j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Weight row pointers for this lane (row index clamped for the canonical layouts; the
  // tiled layout is padded to whole row tiles).
  const uint8_t* wrow[RT];
#pragma unroll
  for (int i = 0; i < RT; ++i) {
    const int rt = min(rt0 + i, nrt - 1);
    if (KIND == kW4Tiled) {
      wrow[i] = w + (static_cast<int64_t>(rt) * nkt) * kTileBytes + lane * 16;
    } else {
      const int n = min(rt * kTileN + r, N - 1);
      wrow[i] = KIND == kW4Canon ? w + static_cast<int64_t>(n) * (K / 2) + q * 16
                                 : w + static_cast<int64_t>(n) * K + q * 32;
    }
  }
  const u32x4 negoff = u32x4{Mfma<DT>::kNegOff, Mfma<DT>::kNegOff, Mfma<DT>::kNegOff,
                             Mfma<DT>::kNegOff};

  for (int kt0 = wave; kt0 < nkt; kt0 += WAVES * UNR) {
    u32x4 braw[UNR][RT][kBDw];
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int kt = kt0 + u * WAVES;
      if (kt < nkt) {
#pragma unroll
        for (int i = 0; i < RT; ++i) {
          if (KIND == kW4Tiled) {
            braw[u][i][0] = load_nt_u32x4(wrow[i] + static_cast<int64_t>(kt) * kTileBytes);
          } else if (KIND == kW4Canon) {
            braw[u][i][0] = load_nt_u32x4(wrow[i] + kt * (kTileK / 2));
          } else {
            braw[u][i][0] = load_nt_u32x4(wrow[i] + kt * kTileK);
            braw[u][i][1] = load_nt_u32x4(wrow[i] + kt * kTileK + 16);
          }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int kt = kt0 + u * WAVES;
      if (kt >= nkt) break;
      // A operand: x[m, kt*128 + 32 q + 8 d + (0..7)], m = 16 mt + r.
      u32x4 a[MT][4];
#pragma unroll
      for (int j = 0; j < MT; ++j) {
        const int m = j * 16 + r;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          if (m < M) {
            a[j][d] = load_u32x4(x + static_cast<int64_t>(m) * ldx + kt * kTileK + q * 32 + d * 8);
            if (KIND == kW4Canon) a[j][d] = permute_canon(a[j][d]);
          } else {
            a[j][d] = u32x4{0u, 0u, 0u, 0u};
          }
        }
      }
      // -(offset) * sum_k x over this k tile, in accumulator layout (INT4 only).
      f32x4 xo[MT];
      if (kW4) {
#pragma unroll
        for (int j = 0; j < MT; ++j) {
          xo[j] = GROUPED ? f32x4{0.f, 0.f, 0.f, 0.f} : xoff[j];
#pragma unroll
          for (int d = 0; d < 4; ++d) xo[j] = Mfma<DT>::mma(a[j][d], negoff, xo[j]);
          if (!GROUPED) xoff[j] = xo[j];
        }
      }
#pragma unroll
      for (int i = 0; i < RT; ++i) {
        u32x4 b[4];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          b[d] = kW4 ? unpack_nibbles<DT>(braw[u][i][0][d])
                     : convert_bytes<DT>(braw[u][i][d >> 1][2 * (d & 1)],
                                         braw[u][i][d >> 1][2 * (d & 1) + 1]);
        }
        if (GROUPED) {
          const int n = min((rt0 + i) * kTileN + r, N - 1);
          const int g = static_cast<int>((static_cast<int64_t>(kt) * kTileK) / group);
          const float s = Act<DT>::round(load_as_f32(scale, scale_dt,
                                                     static_cast<int64_t>(n) * ngroups + g));
#pragma unroll
          for (int j = 0; j < MT; ++j) {
            f32x4 dacc = xo[j];
#pragma unroll
            for (int d = 0; d < 4; ++d) dacc = Mfma<DT>::mma(a[j][d], b[d], dacc);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[i][j][e] = fmaf(s, dacc[e], acc[i][j][e]);
          }
        } else {
#pragma unroll
          for (int j = 0; j < MT; ++j)
#pragma unroll
            for (int d = 0; d < 4; ++d) acc[i][j] = Mfma<DT>::mma(a[j][d], b[d], acc[i][j]);
        }
      }
    }
  }

  // Cross-wave reduction. Per-channel sums still carry the offset term; add it here.
#pragma unroll
  for (int i = 0; i < RT; ++i)
#pragma unroll
    for (int j = 0; j < MT; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float v = acc[i][j][e];
        if (kW4 && !GROUPED) v += xoff[j][e];
        red[(((wave * RT + i) * MT + j) * 4 + e) * 64 + lane] = v;
      }
  __syncthreads();

  constexpr int kOutN = RT * kTileN;
  constexpr int kOut = kOutN * MT * 16;
  for (int o = threadIdx.x; o < kOut; o += 64 * WAVES) {
    const int nl = o % kOutN, ml = o / kOutN;
    const int i = nl / kTileN, rr = nl % kTileN;
    const int j = ml / 16, mm = ml % 16;
    const int src_lane = rr + 16 * (mm >> 2), e = mm & 3;
    float v = 0.f;
#pragma unroll
    for (int wv = 0; wv < WAVES; ++wv) v += red[(((wv * RT + i) * MT + j) * 4 + e) * 64 + src_lane];
    const int m = j * 16 + mm;
    const int n = (rt0 + i) * kTileN + rr;
    if (m < M && n < N) {
      if (!GROUPED) v *= Act<DT>::round(load_as_f32(scale, scale_dt, static_cast<int64_t>(n) * ngroups));
      if (bias) v += Act<DT>::round(load_as_f32(bias, bias_dt, n));
      y[static_cast<int64_t>(m) * ldy + n] = Act<DT>::from_f32(v);
    }
  }
}

// ------------------------------------------------------------ decode launch table

struct DecodeCfg {
  int mt, rt, waves, unr;
};

static DecodeCfg pick_decode_cfg(int kind, int64_t M) {
  (void)kind;
  return DecodeCfg{static_cast<int>((M + 15) / 16), 1, 4, 0};
}

template <int DT, int KIND, int MT, int RT, int WAVES, int UNR>
static int launch_decode_cfg(const void* x, int64_t ldx, const uint8_t* w, const void* scale,
                             int scale_dt, int64_t group, int64_t ngroups, bool grouped,
                             const void* bias, int bias_dt, void* y, int64_t ldy, int64_t M,
                             int64_t N, int64_t K, hipStream_t s) {
  const int nrt = static_cast<int>((N + kTileN - 1) / kTileN);
  const dim3 grid((nrt + RT - 1) / RT);
  const dim3 block(64 * WAVES);
  if (grouped) {
    linear_decode_kernel<DT, KIND, MT, RT, WAVES, UNR, true><<<grid, block, 0, s>>>(
        static_cast<const uint16_t*>(x), ldx, w, scale, scale_dt, group, ngroups, bias, bias_dt,
        static_cast<uint16_t*>(y), ldy, static_cast<int>(M), static_cast<int>(N),
        static_cast<int>(K));
  } else {
    linear_decode_kernel<DT, KIND, MT, RT, WAVES, UNR, false><<<grid, block, 0, s>>>(
        static_cast<const uint16_t*>(x), ldx, w, scale, scale_dt, group, ngroups, bias, bias_dt,
        static_cast<uint16_t*>(y), ldy, static_cast<int>(M), static_cast<int>(N),
        static_cast<int>(K));
  }
  return static_cast<int>(hipGetLastError());
}

template <int DT, int KIND>
static int launch_decode(const void* x, int64_t ldx, const uint8_t* w, const void* scale,
                         int scale_dt, int64_t group, int64_t ngroups, bool grouped,
                         const void* bias, int bias_dt, void* y, int64_t ldy, int64_t M, int64_t N,
                         int64_t K, hipStream_t s) {
  const DecodeCfg c = pick_decode_cfg(KIND, M);
#define LSQ_DECODE_CASE(MT_, UNR_)                                                              \
  if (c.mt == MT_)                                                                            \
    return launch_decode_cfg<DT, KIND, MT_, 1, 4, UNR_>(x, ldx, w, scale, scale_dt, group,    \
                                                        ngroups, grouped, bias, bias_dt, y,   \
                                                        ldy, M, N, K, s);
  LSQ_DECODE_CASE(1, 8)
  LSQ_DECODE_CASE(2, 4)
  LSQ_DECODE_CASE(3, 2)
  LSQ_DECODE_CASE(4, 2)
#undef LSQ_DECODE_CASE
  return LSQ_E_SHAPE;
}

// ------------------------------------------------------------ generic launch

template <int DT>
static int launch_generic(bool w4, const void* x, int64_t ldx, const void* w, const void* scale,
                          int scale_dt, int64_t group, const void* bias, int bias_dt, void* y,
                          int64_t ldy, int64_t M, int64_t N, int64_t K, hipStream_t s) {
  using S = typename Act<DT>::storage;
  const dim3 grid(static_cast<unsigned>((N + 3) / 4), static_cast<unsigned>((M + kGenMB - 1) / kGenMB));
  if (grid.y > 65535u) return LSQ_E_SHAPE;
  if (w4)
    linear_generic_kernel<DT, true><<<grid, 256, 0, s>>>(static_cast<const S*>(x), ldx, w, scale,
                                                         scale_dt, group, bias, bias_dt,
                                                         static_cast<S*>(y), ldy, M, N, K);
  else
    linear_generic_kernel<DT, false><<<grid, 256, 0, s>>>(static_cast<const S*>(x), ldx, w, scale,
                                                          scale_dt, group, bias, bias_dt,
                                                          static_cast<S*>(y), ldy, M, N, K);
  return static_cast<int>(hipGetLastError());
}

static int check_common(const void* x, int64_t ldx, const void* w, const void* scale, void* y,
                        int64_t ldy, int dtype, int bias_dt, const void* bias, int64_t M,
                        int64_t N, int64_t K) {
  // An empty x or y (M, N or K zero) may come with a NULL data pointer, as torch gives
  // for zero-element tensors; such a pointer is never dereferenced.
  if (!w || !scale) return LSQ_E_NULL;
  if ((!x && M > 0 && K > 0) || (!y && M > 0 && N > 0)) return LSQ_E_NULL;
  if (M < 0 || N < 0 || K < 0 || ldx < K || ldy < N) return LSQ_E_SHAPE;
  if (N > INT32_MAX / 2 || K > INT32_MAX / 2 || M > INT32_MAX / 2) return LSQ_E_SHAPE;
  if (dtype != LSQ_F32 && dtype != LSQ_F16 && dtype != LSQ_BF16) return LSQ_E_DTYPE;
  if (bias && bias_dt != LSQ_F32 && bias_dt != LSQ_F16 && bias_dt != LSQ_BF16) return LSQ_E_DTYPE;
  return LSQ_OK;
}

// The fast kernels read x with 16-byte loads at column offsets that are multiples of 8.
static bool x_aligned16(const void* x, int64_t ldx) {
  return (reinterpret_cast<uintptr_t>(x) & 15) == 0 && (ldx % 8) == 0;
}

template <int DT>
static int dispatch(bool w4, const void* x, int64_t ldx, const uint8_t* w, const uint8_t* tiled,
                    const void* scale, int scale_dt, int64_t group, const void* bias, int bias_dt,
                    void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, hipStream_t s) {
  const int64_t ng = (K + group - 1) / group;
  const bool grouped = w4 && group < K;
  if constexpr (DT != LSQ_F32) {
    const bool mfma_ok = K % kTileK == 0 && x_aligned16(x, ldx) &&
                         (reinterpret_cast<uintptr_t>(w) & 15) == 0 &&
                         (!grouped || group % kTileK == 0);
    if (mfma_ok && M <= 16) {
      LinearArgs a{x, ldx, tiled ? tiled : w, scale, scale_dt, bias, bias_dt, y, ldy,
                   M, N, K, group, ng};
      const int kind = w4 ? (tiled ? kW4Tiled : kW4Canon) : (tiled ? kW8Tiled : kW8);
      const int rc = launch_decode<DT>(kind, a, s);
      if (rc != LSQ_E_LAYOUT) return rc;
    }
    if (mfma_ok && M <= 64) {
      if (!w4)
        return launch_decode<DT, kW8>(x, ldx, w, scale, scale_dt, group, ng, false, bias, bias_dt,
                                      y, ldy, M, N, K, s);
      if (tiled)
        return launch_decode<DT, kW4Tiled>(x, ldx, tiled, scale, scale_dt, group, ng, grouped,
                                           bias, bias_dt, y, ldy, M, N, K, s);
      return launch_decode<DT, kW4Canon>(x, ldx, w, scale, scale_dt, group, ng, grouped, bias,
                                         bias_dt, y, ldy, M, N, K, s);
    }
    if (mfma_ok) {
      const int rc = launch_gemm<DT>(w4, x, ldx, w, scale, scale_dt, group, ng, bias, bias_dt, y,
                                     ldy, M, N, K, s);
      if (rc != LSQ_E_LAYOUT) return rc;
    }
  }
  return launch_generic<DT>(w4, x, ldx, w, scale, scale_dt, group, bias, bias_dt, y, ldy, M, N, K,
                            s);
}

}  // namespace lsq

using namespace lsq;

extern "C" int lsq_version(void) { return 100; }

extern "C" const char* lsq_status_string(int status) {
  switch (status) {
    case LSQ_OK: return "success";
    case LSQ_E_NULL: return "lsq: a required pointer is NULL";
    case LSQ_E_SHAPE: return "lsq: M, N or K out of range, or leading dimension smaller than the row";
    case LSQ_E_DTYPE: return "lsq: unsupported dtype code";
    case LSQ_E_GROUP: return "lsq: group_size must be >= 1";
    case LSQ_E_LAYOUT: return "lsq: the tiled weight layouts need K % 128 == 0";
    case LSQ_E_ALIGN: return "lsq: pointer or leading dimension not aligned as required";
    default: break;
  }
  if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
  return "lsq: unknown status";
}

extern "C" int lsq_w8_linear(const void* x, int64_t ldx, const int8_t* weight_q,
                             const int8_t* tiled, const void* scale, int scale_dtype,
                             const void* bias, int bias_dtype, void* y, int64_t ldy, int dtype,
                             int64_t M, int64_t N, int64_t K, void* stream) {
  const int rc = check_common(x, ldx, weight_q, scale, y, ldy, dtype, bias_dtype, bias, M, N, K);
  if (rc != LSQ_OK) return rc;
  if (scale_dtype != LSQ_F32 && scale_dtype != LSQ_F16 && scale_dtype != LSQ_BF16) return LSQ_E_DTYPE;
  if (tiled && (reinterpret_cast<uintptr_t>(tiled) & 15)) return LSQ_E_ALIGN;
  if (tiled && K % kTileK != 0) return LSQ_E_LAYOUT;
  if (M == 0 || N == 0) return LSQ_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint8_t* w = reinterpret_cast<const uint8_t*>(weight_q);
  const uint8_t* t = reinterpret_cast<const uint8_t*>(tiled);
  const int64_t group = K > 0 ? K : 1;
  switch (dtype) {
    case LSQ_F32: return dispatch<LSQ_F32>(false, x, ldx, w, t, scale, scale_dtype, group, bias, bias_dtype, y, ldy, M, N, K, s);
    case LSQ_F16: return dispatch<LSQ_F16>(false, x, ldx, w, t, scale, scale_dtype, group, bias, bias_dtype, y, ldy, M, N, K, s);
    default: return dispatch<LSQ_BF16>(false, x, ldx, w, t, scale, scale_dtype, group, bias, bias_dtype, y, ldy, M, N, K, s);
  }
}

extern "C" int lsq_w4_linear(const void* x, int64_t ldx, const uint8_t* weight_packed,
                             const uint8_t* tiled, const void* scale, int scale_dtype,
                             int64_t group_size, const void* bias, int bias_dtype, void* y,
                             int64_t ldy, int dtype, int64_t M, int64_t N, int64_t K, void* stream) {
  const int rc = check_common(x, ldx, weight_packed, scale, y, ldy, dtype, bias_dtype, bias, M, N, K);
  if (rc != LSQ_OK) return rc;
  if (group_size < 1) return LSQ_E_GROUP;
  if (scale_dtype != LSQ_F32 && scale_dtype != LSQ_F16 && scale_dtype != LSQ_BF16) return LSQ_E_DTYPE;
  if (tiled && (reinterpret_cast<uintptr_t>(tiled) & 15)) return LSQ_E_ALIGN;
  if (tiled && K % kTileK != 0) return LSQ_E_LAYOUT;
  if (M == 0 || N == 0) return LSQ_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t group = K > 0 ? (group_size < K ? group_size : K) : 1;
  switch (dtype) {
    case LSQ_F32: return dispatch<LSQ_F32>(true, x, ldx, weight_packed, tiled, scale, scale_dtype, group, bias, bias_dtype, y, ldy, M, N, K, s);
    case LSQ_F16: return dispatch<LSQ_F16>(true, x, ldx, weight_packed, tiled, scale, scale_dtype, group, bias, bias_dtype, y, ldy, M, N, K, s);
    default: return dispatch<LSQ_BF16>(true, x, ldx, weight_packed, tiled, scale, scale_dtype, group, bias, bias_dtype, y, ldy, M, N, K, s);
  }
}
