// Prefill-shaped weight-only GEMM, M > 16 tokens (gfx950).
//
// GPU form of QuantizedLinear.forward (src/kernels/quantization.py:129-141) for prefill:
// y[M, N] = x[M, K] @ dequant(W)^T + bias, where the reference materializes the whole
// dequantized weight in HBM and calls F.linear. Here each workgroup dequantizes the
// weight tiles it needs straight into LDS and feeds bf16 / fp16 MFMA from there; the
// dequantized weight never exists in HBM.
//
// Tiling. A workgroup computes a 256 x 256 tile of y with 4 waves in a 2 x 2 layout; each
// wave owns 128 x 128 outputs as 4 x 4 blocks of v_mfma_f32_32x32x16_{bf16,f16} (fp32
// accumulators, 256 registers, in AGPRs). K advances 64 columns per step:
//   * the activation tile x[256, 64] is copied to LDS (row stride 72 elements = 144 B, so
//     the MFMA operand reads ds_read_b128 of 32 consecutive rows hit disjoint banks);
//   * the weight tile W[256, 64] is loaded packed (INT4: 8 KB, INT8: 16 KB), unpacked in
//     registers and written to LDS as T: group-wise INT4 as round_T(q * round_T(s)), the
//     reference's dequantized weight exactly; per-channel INT4 / INT8 as the exact integer
//     q, with the row scale applied to the fp32 accumulator in the epilogue;
//   * LDS is double-buffered: the global loads of step k+1 are issued before the MFMAs of
//     step k and written to the other buffer after them, one barrier per step.
// All global reads go through buffer descriptors bounding the workgroup's rows, so
// partial tiles at the M / N edges read zeros without branches.

#include "lsq_common.h"
#include "lsq_internal.h"
#include "lsq_gemm.h"

#include <atomic>

namespace lsq {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr int BM = 256, BN = 256, BK = 64, NT = 256;
constexpr int LDP = BK + 8;  // LDS row stride of both tiles, elements
constexpr int kTileElems = BM * LDP;
constexpr int kLdsBytes = 2 * 2 * kTileElems * 2;  // {x, w} x 2 buffers x bf16

template <int DT> struct Mma32;

template <> struct Mma32<LSQ_BF16> {
  static __device__ __forceinline__ f32x16 mma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                    __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  // two fp32 -> packed pair, round to nearest even
  static __device__ __forceinline__ uint32_t pack2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
  }
};

template <> struct Mma32<LSQ_F16> {
  static __device__ __forceinline__ f32x16 mma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                   __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, f16x2));
  }
};

// Byte b of a dword as an unsigned value, as fp32 (v_cvt_f32_ubyte{0..3}).
__device__ __forceinline__ float ub(uint32_t w, int b) {
  return static_cast<float>((w >> (8 * b)) & 0xFFu);
}

// 8 nibbles of one dword -> 8 values of T for 8 consecutive columns, in column order:
// value = round_T((u - 8) * s) computed as fma(u, s, -8 s), exact before the rounding
// (q has 4 significant bits, s 8 or 11). TILED: nibble p holds column tiled_nibble_k(p);
// canonical: nibble p holds column p.
template <int DT, bool TILED>
__device__ __forceinline__ u32x4 dequant8_w4(uint32_t w, float s, float ms8) {
  const uint32_t lo = w & 0x0F0F0F0Fu;         // nibbles 0, 2, 4, 6
  const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;  // nibbles 1, 3, 5, 7
  float c[8];
  if (TILED) {  // lo bytes -> columns 0, 4, 1, 5; hi bytes -> columns 2, 6, 3, 7
    c[0] = ub(lo, 0); c[4] = ub(lo, 1); c[1] = ub(lo, 2); c[5] = ub(lo, 3);
    c[2] = ub(hi, 0); c[6] = ub(hi, 1); c[3] = ub(hi, 2); c[7] = ub(hi, 3);
  } else {      // byte b holds columns 2b (low nibble) and 2b + 1 (high nibble)
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      c[2 * b] = ub(lo, b);
      c[2 * b + 1] = ub(hi, b);
    }
  }
  u32x4 r;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    r[j] = Mma32<DT>::pack2(fmaf(c[2 * j], s, ms8), fmaf(c[2 * j + 1], s, ms8));
  return r;
}

// 8 signed bytes (two dwords, column order) -> 8 exact values of T.
template <int DT>
__device__ __forceinline__ u32x4 convert8_w8(uint32_t w0, uint32_t w1) {
  u32x4 r;
  r[0] = Mma32<DT>::pack2(static_cast<float>(static_cast<int8_t>(w0)),
                          static_cast<float>(static_cast<int8_t>(w0 >> 8)));
  r[1] = Mma32<DT>::pack2(static_cast<float>(static_cast<int8_t>(w0 >> 16)),
                          static_cast<float>(static_cast<int8_t>(w0 >> 24)));
  r[2] = Mma32<DT>::pack2(static_cast<float>(static_cast<int8_t>(w1)),
                          static_cast<float>(static_cast<int8_t>(w1 >> 8)));
  r[3] = Mma32<DT>::pack2(static_cast<float>(static_cast<int8_t>(w1 >> 16)),
                          static_cast<float>(static_cast<int8_t>(w1 >> 24)));
  return r;
}

// Per-thread share of one weight tile W[256 rows, 64 columns] of a step:
//   kW4Tiled : 2 rows x 32 columns (two 16-byte lane chunks of a 1 KB tile)
//   kW4Canon : 1 row  x 64 columns (32 bytes of a row)
//   kW8Tiled : 2 rows x 32 columns (four 16-byte lane chunks of a 2 KB tile)
//   kW8      : 1 row  x 64 columns (64 bytes of a row)
template <int KIND> struct WPlan;
template <> struct WPlan<kW4Tiled> { static constexpr int kLoads = 2, kRows = 2; };
template <> struct WPlan<kW4Canon> { static constexpr int kLoads = 2, kRows = 1; };
template <> struct WPlan<kW8Tiled> { static constexpr int kLoads = 4, kRows = 2; };
template <> struct WPlan<kW8> { static constexpr int kLoads = 4, kRows = 1; };

template <int DT, int KIND, bool GROUPED>
__global__ void __launch_bounds__(NT) gemm_kernel(LinearArgs p) {
  constexpr bool W4 = KIND == kW4Tiled || KIND == kW4Canon;
  constexpr bool TILED = KIND == kW4Tiled || KIND == kW8Tiled;
  constexpr int WL = WPlan<KIND>::kLoads;
  constexpr int WR = WPlan<KIND>::kRows;
  extern __shared__ __align__(16) unsigned char smem[];
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem);  // [2][BM][LDP]
  uint16_t* ws = xs + 2 * kTileElems;                 // [2][BN][LDP]
  using S = typename Act<DT>::storage;

  const int M = static_cast<int>(p.M), N = static_cast<int>(p.N), K = static_cast<int>(p.K);
  const int nsteps = K / BK;
  const int nkt = K / kTileK;
  const int ng = static_cast<int>(p.ngroups);
  const int group = static_cast<int>(p.group);
  const int mtiles = (M + BM - 1) / BM;
  const int mt = blockIdx.x % mtiles;  // M fastest: consecutive workgroups share W tiles
  const int nt = blockIdx.x / mtiles;
  const int m0 = mt * BM, n0 = nt * BN;
  const int rows_m = min(BM, M - m0);
  const int rows_n = min(BN, N - n0);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wid & 1, wn = wid >> 1;

  // ---- descriptors
  const rsrc_t rx = make_rsrc(static_cast<const uint16_t*>(p.x) + static_cast<int64_t>(m0) * p.ldx,
                              static_cast<uint32_t>(((rows_m - 1) * p.ldx + K) * 2));
  const uint8_t* wbase;
  uint32_t wbytes;
  if (TILED) {
    const int rt0 = n0 / kTileN;
    const int nrt = (N + kTileN - 1) / kTileN;
    const int tb = W4 ? kTileBytes : kTileBytes8;
    wbase = p.w + static_cast<int64_t>(rt0) * nkt * tb;
    wbytes = static_cast<uint32_t>(min(BN / kTileN, nrt - rt0) * nkt * tb);
  } else {
    const int rb = W4 ? K / 2 : K;
    wbase = p.w + static_cast<int64_t>(n0) * rb;
    wbytes = static_cast<uint32_t>(rows_n * rb);
  }
  const rsrc_t rw = make_rsrc(wbase, wbytes);
  const int es_s = p.scale_dt == LSQ_F32 ? 4 : 2;
  const int ngs = GROUPED ? ng : 1;
  // (see lsq_decode.hip: the dword of the last 16-bit element may reach 2 bytes past the
  // array; an aligned dword never crosses a page)
  const rsrc_t rs = make_rsrc(static_cast<const uint8_t*>(p.scale) + static_cast<int64_t>(n0) * ngs * es_s,
                              static_cast<uint32_t>((rows_n * ngs * es_s + 3) & ~3));

  // ---- per-thread load plan
  // activations: chunk c = tid + NT u (u < 8) of the 256 x 64 tile, 8 chunks per row
  uint32_t xoff[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int c = tid + NT * u;
    xoff[u] = static_cast<uint32_t>(((c >> 3) * p.ldx + (c & 7) * 8) * 2);
  }
  // weights: row(s) and first column of this thread's share, and its byte offsets
  int wrow0, wcol0;  // tile-local
  uint32_t woff[WL];
  if (TILED) {
    const int rtl = tid >> 4, e0 = 2 * (tid & 15);
    wrow0 = rtl * kTileN + (e0 & 15);
    wcol0 = 32 * (e0 >> 4);
    // step-independent part; the step adds (k tile) * tile bytes + half * lanes
    const int tb = W4 ? kTileBytes : kTileBytes8;
#pragma unroll
    for (int l = 0; l < WL; ++l) {
      const int e = W4 ? l : (l & 1), j = W4 ? 0 : (l >> 1);
      woff[l] = static_cast<uint32_t>(rtl * nkt * tb + j * (kTileBytes8 / 2) + (e0 + e) * 16);
    }
  } else {
    wrow0 = tid;
    wcol0 = 0;
    const int rb = W4 ? K / 2 : K;
#pragma unroll
    for (int l = 0; l < WL; ++l) woff[l] = static_cast<uint32_t>(tid * rb + l * 16);
  }

  u32x4 xr[8];
  u32x4 wr[WL];
  uint32_t sr[WR];
  auto prefetch = [&](int st) {
    const uint32_t kx = static_cast<uint32_t>(st * BK * 2);
#pragma unroll
    for (int u = 0; u < 8; ++u) xr[u] = bload16<0>(rx, xoff[u] + kx);
    uint32_t kw;
    if (TILED) {
      const int tb = W4 ? kTileBytes : kTileBytes8;
      kw = static_cast<uint32_t>((st >> 1) * tb + (st & 1) * 32 * 16);  // k tile, half
    } else {
      kw = static_cast<uint32_t>(st * (W4 ? BK / 2 : BK));
    }
#pragma unroll
    for (int l = 0; l < WL; ++l) wr[l] = bload16<kNT>(rw, woff[l] + kw);
    if (GROUPED) {
      const int g = (st * BK) / group;
#pragma unroll
      for (int r = 0; r < WR; ++r) {
        const uint32_t eb = static_cast<uint32_t>(((wrow0 + r) * ng + g) * es_s);
        sr[r] = bload4(rs, eb & ~3u) >> (es_s == 2 ? 8 * (eb & 2) : 0);
      }
    }
  };

  auto store = [&](int buf) {
    uint16_t* xb = xs + buf * kTileElems;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int c = tid + NT * u;
      *reinterpret_cast<u32x4*>(xb + (c >> 3) * LDP + (c & 7) * 8) = xr[u];
    }
    uint16_t* wbp = ws + buf * kTileElems;
    if (W4) {
#pragma unroll
      for (int r = 0; r < WR; ++r) {
        float s = 1.f;
        if (GROUPED) s = Act<DT>::round(dword_elem(sr[r], 0, p.scale_dt));
        const float ms8 = -8.f * s;
        // this row's dwords: tiled: lane chunk r (4 dwords, 32 columns); canonical: 8
        // dwords (64 columns) over the two loads
        constexpr int DW = TILED ? 4 : 8;
#pragma unroll
        for (int d = 0; d < DW; ++d) {
          const uint32_t w = TILED ? wr[r][d] : wr[d >> 2][d & 3];
          *reinterpret_cast<u32x4*>(wbp + (wrow0 + r) * LDP + wcol0 + 8 * d) =
              dequant8_w4<DT, TILED>(w, s, ms8);
        }
      }
    } else {
#pragma unroll
      for (int r = 0; r < WR; ++r) {
        // tiled: chunk (j, e=r) holds 16 columns wcol0 + 16 j; canonical: 64 columns
        constexpr int C16 = TILED ? 2 : 4;  // 16-column chunks of this row
#pragma unroll
        for (int c16 = 0; c16 < C16; ++c16) {
          const u32x4 v = TILED ? wr[2 * c16 + r] : wr[c16];
          uint16_t* dst = wbp + (wrow0 + r) * LDP + wcol0 + 16 * c16;
          *reinterpret_cast<u32x4*>(dst) = convert8_w8<DT>(v[0], v[1]);
          *reinterpret_cast<u32x4*>(dst + 8) = convert8_w8<DT>(v[2], v[3]);
        }
      }
    }
  };

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int arow = wm * 128 + (lane & 31);
  const int brow = wn * 128 + (lane & 31);
  const int kcol = 8 * (lane >> 5);

  prefetch(0);
  store(0);
  lds_barrier();
  for (int st = 0; st < nsteps; ++st) {
    const int buf = st & 1;
    if (st + 1 < nsteps) prefetch(st + 1);
    const uint16_t* xb = xs + buf * kTileElems;
    const uint16_t* wbp = ws + buf * kTileElems;
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      u32x4 a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        a[i] = *reinterpret_cast<const u32x4*>(xb + (arow + 32 * i) * LDP + kk * 16 + kcol);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        b[j] = *reinterpret_cast<const u32x4*>(wbp + (brow + 32 * j) * LDP + kk * 16 + kcol);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = Mma32<DT>::mma(a[i], b[j], acc[i][j]);
    }
    if (st + 1 < nsteps) store(buf ^ 1);
    lds_barrier();
  }

  // ---- epilogue: per-channel scale, bias, one rounding to T
  S* y = static_cast<S*>(p.y);
  const int es_b = p.bias_dt == LSQ_F32 ? 4 : 2;
  const rsrc_t rb = make_rsrc(p.bias ? static_cast<const uint8_t*>(p.bias) + static_cast<int64_t>(n0) * es_b
                                     : static_cast<const uint8_t*>(p.scale),
                              p.bias ? static_cast<uint32_t>((rows_n * es_b + 3) & ~3) : 0u);
  float scn[4], bsn[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int nl = wn * 128 + 32 * j + (lane & 31);  // tile-local column
    if (GROUPED) {
      scn[j] = 1.f;
    } else {
      const uint32_t eb = static_cast<uint32_t>(nl * es_s);
      scn[j] = Act<DT>::round(dword_elem(bload4(rs, eb & ~3u), (eb >> 1) & 1, p.scale_dt));
    }
    const uint32_t ebb = static_cast<uint32_t>(nl * es_b);
    bsn[j] = p.bias ? Act<DT>::round(dword_elem(bload4(rb, ebb & ~3u), (ebb >> 1) & 1, p.bias_dt)) : 0.f;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + wn * 128 + 32 * j + (lane & 31);
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = m0 + wm * 128 + 32 * i + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        if (m < M && n < N)
          y[static_cast<int64_t>(m) * p.ldy + n] = Act<DT>::from_f32(fmaf(acc[i][j][v], scn[j], bsn[j]));
      }
    }
}

template <int DT, int KIND, bool GROUPED>
int launch_kind(const LinearArgs& a, hipStream_t s) {
  auto kern = gemm_kernel<DT, KIND, GROUPED>;
  static std::atomic<int> attr_set{0};
  if (!attr_set.load(std::memory_order_acquire)) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
    if (e != hipSuccess) return static_cast<int>(e);
    attr_set.store(1, std::memory_order_release);
  }
  const int64_t tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  kern<<<dim3(static_cast<unsigned>(tiles)), dim3(NT), kLdsBytes, s>>>(a);
  return static_cast<int>(hipGetLastError());
}

}  // namespace

template <int DT>
int launch_gemm(int kind, const LinearArgs& a, hipStream_t s) {
  if (a.M < 1 || a.K % kTileK != 0 || a.K < kTileK) return LSQ_E_LAYOUT;
  const bool grouped = (kind == kW4Tiled || kind == kW4Canon) && a.group < a.K;
  if (grouped && a.group % BK != 0) return LSQ_E_LAYOUT;
  auto aligned4 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 3) == 0; };
  if (!aligned4(a.scale) || (a.bias && !aligned4(a.bias))) return LSQ_E_LAYOUT;
  // 32-bit descriptor ranges
  if ((static_cast<int64_t>(BM - 1) * a.ldx + a.K) * 2 >= (int64_t(1) << 31)) return LSQ_E_LAYOUT;
  if (static_cast<int64_t>(BN) * a.K >= (int64_t(1) << 31)) return LSQ_E_LAYOUT;
  if (a.M * a.ldx >= (int64_t(1) << 40)) return LSQ_E_LAYOUT;
  switch (kind) {
    case kW8: return launch_kind<DT, kW8, false>(a, s);
    case kW8Tiled: return launch_kind<DT, kW8Tiled, false>(a, s);
    case kW4Tiled:
      return grouped ? launch_kind<DT, kW4Tiled, true>(a, s) : launch_kind<DT, kW4Tiled, false>(a, s);
    case kW4Canon:
      return grouped ? launch_kind<DT, kW4Canon, true>(a, s) : launch_kind<DT, kW4Canon, false>(a, s);
    default: return LSQ_E_LAYOUT;
  }
}

template int launch_gemm<LSQ_BF16>(int, const LinearArgs&, hipStream_t);
template int launch_gemm<LSQ_F16>(int, const LinearArgs&, hipStream_t);

}  // namespace lsq
