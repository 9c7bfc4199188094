// Prefill-shaped weight-only GEMM, M > 16 tokens (gfx950).
//
// GPU form of QuantizedLinear.forward (src/kernels/quantization.py:129-141) for prefill:
// y[M, N] = x[M, K] @ dequant(W)^T + bias, where the reference materializes the whole
// dequantized weight in HBM and calls F.linear. Here each workgroup dequantizes the
// weight tiles it needs on chip (into MFMA operand registers, or into LDS) and feeds
// bf16 / fp16 MFMA from there; the dequantized weight never exists in HBM.
//
// Two kernels. gemm_rw_kernel (register weights; the default, in tiles of 256 x 256,
// 128 x 128, 64 x 128 or 64 x 64 chosen by how many workgroups each gives: rw_shape) is
// described at its definition below. gemm_kernel (LDS weights, LSQ_GEMM=lds) follows.
//
// Tiling. A workgroup computes a 256 x 256 tile of y with 8 waves in a 2 x 4 layout (two
// waves per SIMD, so one issues MFMAs while the other waits); each wave owns 128 x 64
// outputs as 4 x 2 blocks of v_mfma_f32_32x32x16_{bf16,f16} (fp32 accumulators, 128
// registers). K advances 64 columns per step:
//   * the activation tile x[256, 64] goes from HBM / L2 straight into LDS with
//     buffer_load ... lds (no registers, no VALU), one step ahead;
//   * the weight tile W[256, 64] is loaded packed (INT4: 8 KB, INT8: 16 KB) two steps
//     ahead, unpacked in registers and written to LDS as T: group-wise INT4 as
//     round_T(q * round_T(s)), the reference's dequantized weight exactly; per-channel
//     INT4 / INT8 as the exact integer q, with the row scale applied to the fp32
//     accumulator in the epilogue;
//   * both LDS tiles store row r's 16-byte column chunk c at position c ^ ((r >> 1) & 7):
//     the LDS serves a 16-byte-per-lane access 16 lanes at a time across 64 banks, and
//     with this swizzle 16 consecutive rows at one column chunk hit 16 disjoint 4-bank
//     groups (MFMA operand reads, weight stores);
//   * LDS is double-buffered, one barrier per step; MFMA operands are double-buffered in
//     registers across the four 16-column sub-steps.
// All global reads go through buffer descriptors bounding the workgroup's rows, so
// partial tiles at the M / N edges read zeros without branches.

#include "lsq_common.h"
#include "lsq_internal.h"
#include "lsq_gemm.h"

#include <algorithm>
#include <atomic>
#include <cstdlib>

namespace lsq {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// 16 bytes per lane from `r` (per-lane offset `voff`, scalar offset `soff`) into LDS at
// `lds` + 16 * lane (a device function of its own: with the builtin in a kernel body,
// clang emitted no host launch stub for some instantiations).
__device__ __forceinline__ void dma16_lds(rsrc_t r, unsigned char* lds, uint32_t voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
}

constexpr int BM = 256, BN = 256, BK = 64, NT = 512;
constexpr int WTM = 128, WTN = 64;  // wave tile: 2 x 4 waves
constexpr int FM = WTM / 32, FN = WTN / 32;  // 32x32 MFMA blocks per wave
constexpr int kLdsBytes = 2 * 2 * BM * BK * 2;  // {x, w} x 2 buffers x 16-bit

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

// 8 nibbles of one dword -> 8 values of T for 8 consecutive columns, in column order:
// value = round_T((u - 8) * s). The AND-OR (w >> 4p) & 0x000F000F | 0x64006400 turns
// nibbles p and p + 4 into the fp16 pair (1024 + u_p, 1024 + u_{p+4}); v_fma_mix_f32 then
// computes (1024 + u) * s - 1032 * s in fp32, which is exact ((1024 + u) has 11
// significant bits, s at most 11, 1032 = 2^10 + 2^3), and one v_cvt_pk rounds to T.
// TILED: nibble p holds column tiled_nibble_k(p), so pair p is columns (2p, 2p + 1);
// canonical: nibble p holds column p, so pair p is columns (p, p + 4). `mask` and
// `magic` are the two constants, kept in VGPRs (VOP3 takes no literal).
template <int DT, bool TILED>
__device__ __forceinline__ u32x4 dequant8_w4(uint32_t w, float s, float c, uint32_t mask, uint32_t magic) {
  float v[8];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const uint32_t pair = ((w >> (4 * p)) & mask) | magic;
    const float lo = __builtin_fmaf(static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(pair))), s, c);
    const float hi = __builtin_fmaf(static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(pair >> 16))), s, c);
    if (TILED) {
      v[2 * p] = lo;
      v[2 * p + 1] = hi;
    } else {
      v[p] = lo;
      v[p + 4] = hi;
    }
  }
  u32x4 r;
#pragma unroll
  for (int j = 0; j < 4; ++j) r[j] = Mma32<DT>::pack2(v[2 * j], v[2 * j + 1]);
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

// Per-thread share of one weight tile W[256 rows, 64 columns] of a step: thread t takes
// row t & 255, columns 32 (t >> 8) .. +32 (so 16 consecutive lanes store 16 consecutive
// rows), as 16-byte loads: INT4 one (a lane chunk of the tiled layout / 16 bytes of the
// canonical row), INT8 two (two 1 KB halves of the tiled layout / 32 bytes of the row).
template <int KIND> struct WPlan;
template <> struct WPlan<kW4Tiled> { static constexpr int kLoads = 1, kRows = 1; };
template <> struct WPlan<kW4Canon> { static constexpr int kLoads = 1, kRows = 1; };
template <> struct WPlan<kW8Tiled> { static constexpr int kLoads = 2, kRows = 1; };
template <> struct WPlan<kW8> { static constexpr int kLoads = 2, kRows = 1; };

template <int DT, int KIND, bool GROUPED>
__global__ void __launch_bounds__(NT) gemm_kernel(LinearArgs p) {
  constexpr bool W4 = KIND == kW4Tiled || KIND == kW4Canon;
  constexpr bool TILED = KIND == kW4Tiled || KIND == kW8Tiled;
  constexpr int WL = WPlan<KIND>::kLoads;
  constexpr int WR = WPlan<KIND>::kRows;
  extern __shared__ __align__(16) unsigned char smem[];
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
  const int wm = wid & 1, wn = wid >> 1;  // wave tile rows wm * 128, columns wn * 64
  uint32_t nib_mask, nib_magic;
  asm volatile("v_mov_b32 %0, 0x000f000f" : "=v"(nib_mask));
  asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(nib_magic));

  // K rotation. Workgroups are dealt to the 8 XCDs round-robin and the ~32 resident on
  // one XCD share activation rows; walking K in lockstep, every step's activation tile
  // would be a fresh HBM miss all of them wait on. Each workgroup instead starts at a
  // different step (spread over K by its slot on the XCD) and wraps around, so after the
  // first two steps the tiles it needs are already in the XCD's L2. The order of the
  // fp32 sums over K is fixed per workgroup, so results do not depend on timing.
  const int rot = (((blockIdx.x >> 3) & 31) * nsteps) >> 5;
  auto gstep = [&](int st) { const int g = st + rot; return g >= nsteps ? g - nsteps : g; };

  // LDS: x tiles at [0, 2 * kTile), w tiles after; each tile is 256 rows of 8 chunks of
  // 16 bytes, chunk c of row r stored at position c ^ ((r >> 1) & 7).
  constexpr int kTile = BM * BK * 2;
  auto xs_at = [&](int buf) { return smem + buf * kTile; };
  auto ws_at = [&](int buf) { return smem + (2 + buf) * kTile; };

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
  // (the dword of the last 16-bit element may reach 2 bytes past the array; an aligned
  // dword never crosses a page)
  const rsrc_t rs = make_rsrc(static_cast<const uint8_t*>(p.scale) + static_cast<int64_t>(n0) * ngs * es_s,
                              static_cast<uint32_t>((rows_n * ngs * es_s + 3) & ~3));

  // ---- activations: DMA straight into LDS. One wave instruction fills 8 rows (1 KB):
  // lane l writes LDS row rb + (l >> 3), position l & 7, which must hold column chunk
  // (l & 7) ^ (((rb + (l >> 3)) >> 1) & 7); rb is a multiple of 8, so that swizzle term
  // is ((rb >> 1) & 4) | (l >> 4). The row goes into the per-lane offset, which the
  // descriptor's range check covers (the scalar offset is not checked), so rows past M
  // read zeros; the scalar offset carries only the column of the step.
  constexpr int kXB = BM / 8 / (NT / 64);  // 4 row blocks of 8 per wave
  uint32_t x_lane_off[kXB];
#pragma unroll
  for (int b = 0; b < kXB; ++b) {
    const int rb = (wid * kXB + b) * 8;  // (rb >> 1) & 4 == (b & 1) * 4
    x_lane_off[b] = static_cast<uint32_t>(
        ((rb + (lane >> 3)) * p.ldx + 8 * ((lane & 7) ^ (((b & 1) << 2) | (lane >> 4)))) * 2);
  }
  auto issue_x = [&](int st, int buf) {
    unsigned char* dst = xs_at(buf);
#pragma unroll
    for (int b = 0; b < kXB; ++b) {
      const int rb = (wid * kXB + b) * 8;
      dma16_lds(rx, dst + rb * BK * 2, x_lane_off[b], static_cast<int>(gstep(st) * BK * 2));
    }
  };

  // ---- weights: packed tile share of this thread, prefetched two steps ahead
  const int wrow0 = tid & (BN - 1);  // tile-local row
  const int wc = tid >> 8;           // which 32 of the step's 64 columns
  uint32_t woff[WL];
  if (TILED) {
    // lane chunk (row & 15) + 16 wc of the half-tile; INT8 adds the 1 KB half j
    const int tb = W4 ? kTileBytes : kTileBytes8;
#pragma unroll
    for (int l = 0; l < WL; ++l)
      woff[l] = static_cast<uint32_t>((wrow0 >> 4) * nkt * tb + l * (kTileBytes8 / 2) +
                                      ((wrow0 & 15) + 16 * wc) * 16);
  } else {
    const int rb = W4 ? K / 2 : K;
#pragma unroll
    for (int l = 0; l < WL; ++l)
      woff[l] = static_cast<uint32_t>(wrow0 * rb + (W4 ? 16 : 32) * wc + l * 16);
  }
  struct WRegs {
    u32x4 w[WL];
    uint32_t s[WR];
  };
  auto issue_w = [&](int st, WRegs& r) {
    const bool real = st < nsteps;
    const int gs = gstep(min(st, nsteps - 1));
    uint32_t kw;
    if (TILED) {
      const int tb = W4 ? kTileBytes : kTileBytes8;
      kw = static_cast<uint32_t>((gs >> 1) * tb + (gs & 1) * 32 * 16);  // k tile, half
    } else {
      kw = static_cast<uint32_t>(gs * (W4 ? BK / 2 : BK));
    }
#pragma unroll
    for (int l = 0; l < WL; ++l) r.w[l] = bload16<kNT>(rw, real ? woff[l] + kw : kOOB);
    if (GROUPED) {
      const int g = (gs * BK) / group;
#pragma unroll
      for (int rr = 0; rr < WR; ++rr)
        r.s[rr] = bload4(rs, static_cast<uint32_t>(((wrow0 + rr) * ng + g) * es_s) & ~3u);
    }
  };
  // The thread's share of a weight tile is 4 units of 8 columns (INT4: one dword, INT8: a
  // pair of dwords). put_w_unit(r, sf, buf, u) dequantizes unit u into LDS; the main loop
  // spreads the 4 units over the MFMA sub-steps so the VALU work overlaps the MFMAs.
  // Group scales of this thread's rows for step st, round_T, as fp32 (1 per-channel).
  auto w_scales = [&](const WRegs& r, int st, float (&sf)[WR]) {
#pragma unroll
    for (int rr = 0; rr < WR; ++rr) sf[rr] = 1.f;
    if (GROUPED) {
      const int g = (gstep(min(st, nsteps - 1)) * BK) / group;
#pragma unroll
      for (int rr = 0; rr < WR; ++rr) {
        const uint32_t eb = static_cast<uint32_t>(((wrow0 + rr) * ng + g) * es_s);
        sf[rr] = Act<DT>::round(dword_elem(r.s[rr], (eb >> 1) & 1, p.scale_dt));
      }
    }
  };
  // unit u = columns 32 wc + 8u .. +7 of the thread's row (u = 0..3)
  auto put_w_unit = [&](const WRegs& r, const float (&sf)[WR], int buf, int u) {
    const int row = wrow0;
    unsigned char* addr = ws_at(buf) + row * (BK * 2) + (((4 * wc + u) ^ ((row >> 1) & 7)) << 4);
    if (W4) {
      *reinterpret_cast<u32x4*>(addr) = dequant8_w4<DT, TILED>(r.w[0][u], sf[0], -1032.f * sf[0], nib_mask, nib_magic);
    } else {
      // 16 columns per load (tiled: the 1 KB half u >> 1; canonical: bytes 16 (u >> 1))
      const u32x4 v = r.w[u >> 1];
      *reinterpret_cast<u32x4*>(addr) = (u & 1) ? convert8_w8<DT>(v[2], v[3]) : convert8_w8<DT>(v[0], v[1]);
    }
  };
  auto put_w = [&](const WRegs& r, int st, int buf) {
    float sf[WR];
    w_scales(r, st, sf);
#pragma unroll
    for (int u = 0; u < 4; ++u) put_w_unit(r, sf, buf, u);
  };

  // ---- MFMA operands: lane l reads row (l & 31) of each 32-row block, 8 columns at
  // 16 kk + 8 (l >> 5); with the swizzle that is position (2 kk + (l >> 5)) ^ (((l & 31) >> 1) & 7).
  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
  const int frow = lane & 31;
  auto frag_off = [&](int kk) {
    return frow * (BK * 2) + (((2 * kk + (lane >> 5)) ^ ((frow >> 1) & 7)) << 4);
  };
  // One step of MFMAs on LDS buffer `buf`; after each 16-column sub-step, side(kk) does
  // a quarter of the next weight tile's dequantization.
  auto compute = [&](int buf, auto&& side) {
    const unsigned char* xb = xs_at(buf) + wm * WTM * (BK * 2);
    const unsigned char* wbp = ws_at(buf) + wn * WTN * (BK * 2);
    u32x4 a[2][FM], b[2][FN];
    auto load = [&](int kk, u32x4 (&aa)[FM], u32x4 (&bb)[FN]) {
      const int off = frag_off(kk);
#pragma unroll
      for (int i = 0; i < FM; ++i)
        aa[i] = *reinterpret_cast<const u32x4*>(xb + 32 * i * (BK * 2) + off);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bb[j] = *reinterpret_cast<const u32x4*>(wbp + 32 * j * (BK * 2) + off);
    };
    load(0, a[0], b[0]);
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      if (kk + 1 < BK / 16) load(kk + 1, a[(kk + 1) & 1], b[(kk + 1) & 1]);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = Mma32<DT>::mma(a[kk & 1][i], b[kk & 1][j], acc[i][j]);
      side(kk);
    }
  };

  // ---- pipeline: x one step ahead (LDS DMA), w two steps ahead (registers). The step
  // count K / 64 is even (K % 128 == 0), so the loop runs whole pairs of steps and every
  // load is unconditional: past the last step the w loads are out of range and the x DMA
  // lands in a buffer nobody reads again. Before each barrier only the x DMA must have
  // landed: the w loads issued after it (for three steps ahead) stay in flight.
  constexpr int kWLoads = WL + (GROUPED ? WR : 0);
  constexpr int kWaitX = (kWLoads & 15) | (7 << 4) | ((kWLoads >> 4) << 14);  // vmcnt(kWLoads), lgkmcnt(0)
  WRegs wr0, wr1;
  issue_x(0, 0);
  issue_w(0, wr0);
  issue_w(1, wr1);
  put_w(wr0, 0, 0);
  issue_w(2, wr0);
  __builtin_amdgcn_s_waitcnt(kWaitX);
  lds_barrier();
  auto step = [&](int st, WRegs& next) {  // next holds step st + 1; refilled with st + 3
    const int buf = st & 1;
    issue_x(st + 1, buf ^ 1);
    float sf[WR];
    w_scales(next, st + 1, sf);
    compute(buf, [&](int kk) {
      put_w_unit(next, sf, buf ^ 1, kk);
    });
    issue_w(st + 3, next);
    __builtin_amdgcn_s_waitcnt(kWaitX);
    lds_barrier();
  };
  for (int st = 0; st < nsteps; st += 2) {
    step(st, wr1);
    step(st + 1, wr0);
  }

  // ---- epilogue: per-channel scale, bias, one rounding to T
  S* y = static_cast<S*>(p.y);
  const int es_b = p.bias_dt == LSQ_F32 ? 4 : 2;
  const rsrc_t rb = make_rsrc(p.bias ? static_cast<const uint8_t*>(p.bias) + static_cast<int64_t>(n0) * es_b
                                     : static_cast<const uint8_t*>(p.scale),
                              p.bias ? static_cast<uint32_t>((rows_n * es_b + 3) & ~3) : 0u);
  float scn[FN], bsn[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int nl = wn * WTN + 32 * j + (lane & 31);  // tile-local column
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
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int n = n0 + wn * WTN + 32 * j + (lane & 31);
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = m0 + wm * WTM + 32 * i + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        if (m < M && n < N)
          y[static_cast<int64_t>(m) * p.ldy + n] = Act<DT>::from_f32(fmaf(acc[i][j][v], scn[j], bsn[j]));
      }
    }
}

// ---------------------------------------------------------------------------------------
// Register-weight variant, two shapes. 128 x 128 tiles: 4 waves, two workgroups per CU
// (one wave of each per SIMD), each with its own barrier, so one workgroup's barrier and
// LDS latency bubbles are filled by the other's MFMAs. 256 x 256 tiles: 8 waves (two per
// SIMD), one workgroup per CU. Either way wave w owns weight rows (output columns)
// [32 w, 32 w + 32) for all the tile's activation rows (RFM x 1 blocks of 32 x 32). Only
// the activations go through LDS (two stages, DMA one step ahead); each wave loads its
// own weight rows straight into registers in MFMA operand order (three steps in flight)
// and dequantizes them right before use, so weight tiles never touch LDS.
// K order inside a step: lane l at 16-column sub-step kk multiplies columns
// 32 (l >> 5) + 8 kk .. +7 (the same permutation on both operands), which makes each
// lane's weights one contiguous 32-column chunk per step.
// three activation stages: 96 KB for 256-row tiles, 48 KB for 128-row tiles
__host__ __device__ constexpr int rw_lds_bytes(int rbm) { return 3 * rbm * BK * 2; }

// RFN_ 32-column blocks per wave, RFM_ 32-row blocks, RNT_ threads, MINB workgroups per CU.
// SPLIT: workgroup b takes K slice b % p.ksplit of tile b / p.ksplit and writes its fp32
// sums (per-channel scale applied, no bias) to p.part [ksplit][M][N] for the merge kernel.
template <int DT, int KIND, bool GROUPED, int RFN_, int RFM_, int RNT_, int MINB, bool SPLIT>
__global__ void __launch_bounds__(RNT_, MINB) gemm_rw_kernel(LinearArgs p) {
  constexpr int RFN = RFN_, RFM = RFM_, RNT = RNT_;
  constexpr int RBM = 32 * RFM;
  constexpr int RBN = (RNT / 64) * 32 * RFN;
  constexpr bool W4 = KIND == kW4Tiled || KIND == kW4Canon;
  constexpr bool TILED = KIND == kW4Tiled || KIND == kW8Tiled;
  constexpr int WLB = W4 ? 1 : 2;  // 16-byte loads per lane per 32-row block per step
  extern __shared__ __align__(16) unsigned char smem[];
  using S = typename Act<DT>::storage;

  const int M = static_cast<int>(p.M), N = static_cast<int>(p.N), K = static_cast<int>(p.K);
  // K slice: steps [st0, st0 + nsteps) of the layer's 64-column steps (all of them unsplit)
  const int NS = SPLIT ? p.ksplit : 1;
  const int tile = SPLIT ? static_cast<int>(blockIdx.x) / NS : static_cast<int>(blockIdx.x);
  const int sl = SPLIT ? static_cast<int>(blockIdx.x) - tile * NS : 0;
  const int st0 = sl * (K / BK) / NS;
  const int nsteps = (sl + 1) * (K / BK) / NS - st0;
  const int nkt = K / kTileK;
  const int ng = static_cast<int>(p.ngroups);
  const int group = static_cast<int>(p.group);
  const int mtiles = (M + RBM - 1) / RBM;
  // Tile of this workgroup. Workgroups are dealt to the 8 XCDs round-robin (XCD b % 8),
  // each XCD with its own L2. 128-row tiles: M fastest, so consecutive workgroups share
  // W tiles. 256-row tiles: the tiles are ordered in groups of 4 M tiles (M fastest
  // inside a group, then N, then the next group) and XCD x takes the x-th eighth of that
  // order, so the ~32 workgroups resident on an XCD form a 4 x 8 block of tiles and, all
  // walking K in step, share each activation tile 8 ways and each weight tile 4 ways in
  // that XCD's L2 (when the grid does not divide so, M fastest as for 128-row tiles).
  int mt = tile % mtiles;
  int nt = tile / mtiles;
  const int ntiles = (N + RBN - 1) / RBN;
  const bool blocked = !SPLIT && RFM == 8 && mtiles % 4 == 0 && (mtiles * ntiles) % 8 == 0;
  if (blocked) {
    const int L = (tile & 7) * (mtiles * ntiles / 8) + (tile >> 3);
    const int r = L % (4 * ntiles);
    mt = 4 * (L / (4 * ntiles)) + (r & 3);
    nt = r >> 2;
  }
  const int m0 = mt * RBM, n0 = nt * RBN;
  const int rows_m = min(RBM, M - m0);
  const int rows_n = min(RBN, N - n0);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5;  // which 32-column half of the step this lane multiplies
  uint32_t nib_mask, nib_magic;
  asm volatile("v_mov_b32 %0, 0x000f000f" : "=v"(nib_mask));
  asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(nib_magic));

  // K rotation per workgroup (see gemm_kernel): spreads first-touch misses over K; none
  // for the blocked 256-row tiles, whose workgroups share tiles by walking K in step
  // (14336 x 4096 M=8192: 891 -> 792 us without it).
  const int rot = blocked ? 0 : (((blockIdx.x >> 3) & 31) * nsteps) >> 5;
  auto gstep = [&](int st) { const int g = st + rot; return st0 + (g >= nsteps ? g - nsteps : g); };
  // scale group of K step gs (group % 64 == 0): a shift for power-of-two groups, else a
  // division (uniform; the scalar unit is shared by the CU's waves)
  const int spg = group / BK;
  const int spg_sh = __builtin_ctz(static_cast<uint32_t>(spg));
  const bool spg_pow2 = (spg & (spg - 1)) == 0;
  auto group_of = [&](int gs) { return spg_pow2 ? gs >> spg_sh : gs / spg; };

  // ---- descriptors
  const rsrc_t rx = make_rsrc(static_cast<const uint16_t*>(p.x) + static_cast<int64_t>(m0) * p.ldx,
                              static_cast<uint32_t>(((rows_m - 1) * p.ldx + K) * 2));
  const int tb = W4 ? kTileBytes : kTileBytes8;
  const uint8_t* wbase;
  uint32_t wbytes;
  if (TILED) {
    const int rt0 = n0 / kTileN;
    const int nrt = (N + kTileN - 1) / kTileN;
    wbase = p.w + static_cast<int64_t>(rt0) * nkt * tb;
    wbytes = static_cast<uint32_t>(min(RBN / kTileN, nrt - rt0) * nkt * tb);
  } else {
    const int rb = W4 ? K / 2 : K;
    wbase = p.w + static_cast<int64_t>(n0) * rb;
    wbytes = static_cast<uint32_t>(rows_n * rb);
  }
  const rsrc_t rw = make_rsrc(wbase, wbytes);
  const int es_s = p.scale_dt == LSQ_F32 ? 4 : 2;
  const int ngs = GROUPED ? ng : 1;
  const rsrc_t rs = make_rsrc(static_cast<const uint8_t*>(p.scale) + static_cast<int64_t>(n0) * ngs * es_s,
                              static_cast<uint32_t>((rows_n * ngs * es_s + 3) & ~3));

  // ---- activations: three LDS stages of RBM rows x 64 columns, chunk c of row r at
  // position c ^ ((r >> 1) & 7); DMA as in gemm_kernel (4 x 1 KB per wave per step).
  constexpr int kStage = RBM * BK * 2;
  constexpr int kXB = RBM / 8 / (RNT / 64);  // 4 row blocks of 8 per wave
  uint32_t x_lane_off[kXB];  // row in the range-checked per-lane offset, as in gemm_kernel
#pragma unroll
  for (int b = 0; b < kXB; ++b) {
    const int rb = (wid * kXB + b) * 8;  // (rb >> 1) & 4 == (b & 1) * 4
    x_lane_off[b] = static_cast<uint32_t>(
        ((rb + (lane >> 3)) * p.ldx + 8 * ((lane & 7) ^ (((b & 1) << 2) | (lane >> 4)))) * 2);
  }
  auto issue_x = [&](int st, int buf) {
    unsigned char* dst = smem + buf * kStage;
#pragma unroll
    for (int b = 0; b < kXB; ++b) {
      const int rb = (wid * kXB + b) * 8;
      dma16_lds(rx, dst + rb * BK * 2, x_lane_off[b], static_cast<int>(gstep(st) * BK * 2));
    }
  };

  // ---- weights: lane's row of block j is tile-local row lr[j]; per step it reads the
  // 32-column chunk h of the step (INT8: two 16-byte loads).
  uint32_t woff[RFN];
  int lr[RFN];
#pragma unroll
  for (int j = 0; j < RFN; ++j) {
    lr[j] = 32 * RFN * wid + 32 * j + (lane & 31);
    woff[j] = TILED ? static_cast<uint32_t>((lr[j] >> 4) * nkt * tb + ((lr[j] & 15) + 16 * h) * 16)
                    : static_cast<uint32_t>(lr[j] * (W4 ? K / 2 : K) + (W4 ? 16 : 32) * h);
  }
  struct WSet {
    u32x4 w[RFN][WLB];
    uint32_t s[RFN];
  };
  auto issue_w = [&](int st, WSet& r) {
    const bool real = st < nsteps;
    const int gs = gstep(min(st, nsteps - 1));
    const uint32_t kw = TILED ? static_cast<uint32_t>((gs >> 1) * tb + (gs & 1) * 512)
                              : static_cast<uint32_t>(gs * (W4 ? BK / 2 : BK));
#pragma unroll
    for (int j = 0; j < RFN; ++j)
#pragma unroll
      for (int l = 0; l < WLB; ++l)
        r.w[j][l] = bload16<kNT>(rw, real ? woff[j] + kw + l * (TILED ? kTileBytes8 / 2 : 16) : kOOB);
    if (GROUPED) {
      const int g = group_of(gs);
#pragma unroll
      for (int j = 0; j < RFN; ++j)
        r.s[j] = bload4(rs, static_cast<uint32_t>((lr[j] * ng + g) * es_s) & ~3u);
    }
  };

  // ---- MFMA fragments
  f32x16 acc[RFM][RFN];
#pragma unroll
  for (int i = 0; i < RFM; ++i)
#pragma unroll
    for (int j = 0; j < RFN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
  const int frow = lane & 31;
  auto frag_off = [&](int kk) { return frow * (BK * 2) + (((4 * h + kk) ^ ((frow >> 1) & 7)) << 4); };

  // A fragments, double-buffered by sub-step; a[0] holds sub-step 0 of the next step when
  // a step starts. The step's barrier sits before its last sub-step's MFMAs: right after
  // it the next step's first fragments are read from the other LDS stage while those
  // MFMAs run, so the MFMA pipe does not drain at the barrier.
  u32x4 a[2][RFM];
  auto load_a = [&](int buf, int kk, u32x4 (&aa)[RFM]) {
    const unsigned char* xb = smem + buf * kStage;
    const int off = frag_off(kk);
#pragma unroll
    for (int i = 0; i < RFM; ++i) aa[i] = *reinterpret_cast<const u32x4*>(xb + 32 * i * (BK * 2) + off);
  };
  auto step = [&](int st, const WSet& cur, WSet& nxt2) {
    // three stages, the DMA two steps ahead (the stage it fills was last read before the
    // previous step's barrier)
    const int buf = st % 3;
    issue_x(st + 2, (st + 2) % 3);
    issue_w(st + 2, nxt2);
    float sf[RFN], cf[RFN];
#pragma unroll
    for (int j = 0; j < RFN; ++j) {
      sf[j] = 1.f;
      if (GROUPED) {
        const int g = group_of(gstep(min(st, nsteps - 1)));
        const uint32_t eb = static_cast<uint32_t>((lr[j] * ng + g) * es_s);
        sf[j] = Act<DT>::round(dword_elem(cur.s[j], (eb >> 1) & 1, p.scale_dt));
      }
      cf[j] = -1032.f * sf[j];
    }
    // B operands one sub-step ahead: the dequantization of sub-step kk + 1 is independent
    // of the MFMAs of sub-step kk, so the two interleave.
    u32x4 b[2][RFN];
    auto dequant = [&](int kk, u32x4 (&bb)[RFN]) {
#pragma unroll
      for (int j = 0; j < RFN; ++j)
        bb[j] = W4 ? dequant8_w4<DT, TILED>(cur.w[j][0][kk], sf[j], cf[j], nib_mask, nib_magic)
                   : convert8_w8<DT>(cur.w[j][kk >> 1][2 * (kk & 1)], cur.w[j][kk >> 1][2 * (kk & 1) + 1]);
    };
    dequant(0, b[0]);
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      if (kk + 1 < BK / 16) {
        load_a(buf, kk + 1, a[(kk + 1) & 1]);
        dequant(kk + 1, b[(kk + 1) & 1]);
      } else {
        // The next step's activation DMA must have landed (the loads issued after it stay
        // in flight: its step's weight loads, and the DMA and weights issued in this step;
        // in step 0 the count also waits for step 0's weights, issued after step 1's DMA in
        // the prologue, which is merely conservative); the barrier also orders every wave's
        // reads of this stage before a later DMA into it.
        constexpr int kW = RFN * WLB + (GROUPED ? RFN : 0);
        constexpr int kAfter = 2 * kW + kXB;
        __builtin_amdgcn_s_waitcnt((kAfter & 15) | (7 << 4) | ((kAfter >> 4) << 14));
        lds_barrier();
        load_a((st + 1) % 3, 0, a[0]);
      }
#pragma unroll
      for (int i = 0; i < RFM; ++i)
#pragma unroll
        for (int j = 0; j < RFN; ++j) acc[i][j] = Mma32<DT>::mma(a[kk & 1][i], b[kk & 1][j], acc[i][j]);
      if constexpr (W4 && RFM * RFN == 8) {
        // Issue order for the INT4 256 x 32 wave tile, twice per sub-step: four of the
        // next fragment reads, then four MFMAs with three VALU ops (dequantization) after
        // each. Measured 3 % faster than the compiler's own order (14336 x 4096, INT4
        // g128: M=2048 226 -> 219 us, M=8192 909 -> 883 us); the INT8 instances spill
        // registers under it and keep the compiler's order.
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
          __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // DS reads
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // VALU
          }
        }
      }
    }
  };

  WSet r0, r1, r2;
  issue_x(0, 0);
  issue_x(1, 1);
  issue_w(0, r0);
  issue_w(1, r1);
  {
    constexpr int kAfter = 2 * (RFN * WLB + (GROUPED ? RFN : 0));
    __builtin_amdgcn_s_waitcnt((kAfter & 15) | (7 << 4) | ((kAfter >> 4) << 14));
  }
  lds_barrier();
  load_a(0, 0, a[0]);
  int st = 0;
  for (; st + 3 <= nsteps; st += 3) {
    step(st, r0, r2);
    step(st + 1, r1, r0);
    step(st + 2, r2, r1);
  }
  if (st < nsteps) step(st, r0, r2);
  if (st + 1 < nsteps) step(st + 1, r1, r0);

  // ---- epilogue: per-channel scale, bias, one rounding to T
  S* y = static_cast<S*>(p.y);
  const int es_b = p.bias_dt == LSQ_F32 ? 4 : 2;
  const rsrc_t rb = make_rsrc(p.bias ? static_cast<const uint8_t*>(p.bias) + static_cast<int64_t>(n0) * es_b
                                     : static_cast<const uint8_t*>(p.scale),
                              p.bias ? static_cast<uint32_t>((rows_n * es_b + 3) & ~3) : 0u);
  float scn[RFN], bsn[RFN];
#pragma unroll
  for (int j = 0; j < RFN; ++j) {
    if (GROUPED) {
      scn[j] = 1.f;
    } else {
      const uint32_t eb = static_cast<uint32_t>(lr[j] * es_s);
      scn[j] = Act<DT>::round(dword_elem(bload4(rs, eb & ~3u), (eb >> 1) & 1, p.scale_dt));
    }
    const uint32_t ebb = static_cast<uint32_t>(lr[j] * es_b);
    bsn[j] = p.bias ? Act<DT>::round(dword_elem(bload4(rb, ebb & ~3u), (ebb >> 1) & 1, p.bias_dt)) : 0.f;
  }
#pragma unroll
  for (int i = 0; i < RFM; ++i)
#pragma unroll
    for (int j = 0; j < RFN; ++j) {
      const int n = n0 + lr[j];
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = m0 + 32 * i + 8 * (v >> 2) + 4 * h + (v & 3);
        if (m < M && n < N) {
          if constexpr (SPLIT)  // this slice's scaled sum; the bias and the rounding come in the merge
            p.part[(static_cast<int64_t>(sl) * M + m) * N + n] = acc[i][j][v] * scn[j];
          else
            y[static_cast<int64_t>(m) * p.ldy + n] = Act<DT>::from_f32(fmaf(acc[i][j][v], scn[j], bsn[j]));
        }
      }
    }
}

template <int DT, int KIND, bool GROUPED, int RFN, int RFM, int RNT, int MINB, bool SPLIT>
int launch_rw_shape(const LinearArgs& a, hipStream_t s) {
  constexpr int rbm = 32 * RFM, rbn = (RNT / 64) * 32 * RFN;
  const int64_t tiles = ((a.M + rbm - 1) / rbm) * ((a.N + rbn - 1) / rbn) * (SPLIT ? a.ksplit : 1);
  auto kern = gemm_rw_kernel<DT, KIND, GROUPED, RFN, RFM, RNT, MINB, SPLIT>;
  if (rw_lds_bytes(rbm) > 64 * 1024) {
    static std::atomic<int> attr_set{0};
    if (!attr_set.load(std::memory_order_acquire)) {
      const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, rw_lds_bytes(rbm));
      if (e != hipSuccess) return static_cast<int>(e);
      attr_set.store(1, std::memory_order_release);
    }
  }
  kern<<<dim3(static_cast<unsigned>(tiles)), dim3(RNT), rw_lds_bytes(rbm), s>>>(a);
  return static_cast<int>(hipGetLastError());
}

// Register-weight shapes (activation rows x weight rows per workgroup): 0 = 128 x 128
// (4 waves of 128 x 32, two workgroups per CU), 1 = 256 x 256 (8 waves of 256 x 32, one
// workgroup per CU), 2 = 64 x 128 (4 waves of 64 x 32), 3 = 64 x 64 (2 waves of 64 x 32).
template <int DT, int KIND, bool GROUPED, bool SPLIT>
int launch_rw(const LinearArgs& a, int shape, hipStream_t s) {
  if (shape == 1) return launch_rw_shape<DT, KIND, GROUPED, 1, 8, 512, 1, SPLIT>(a, s);
  if (shape == 2) return launch_rw_shape<DT, KIND, GROUPED, 1, 2, 256, 4, SPLIT>(a, s);
  if (shape == 3) return launch_rw_shape<DT, KIND, GROUPED, 1, 2, 128, 4, SPLIT>(a, s);
  return launch_rw_shape<DT, KIND, GROUPED, 1, 4, 256, 2, SPLIT>(a, s);
}

// Split-K plan for the register-weight kernel: when the chosen tile gives fewer than 128
// workgroups, or fewer than 384 on a long K (128+ steps of 64 columns), K is cut into S
// slices of at least 8 steps so that about 512 workgroups run (256 x 256 tiles, one
// workgroup per CU: on a long K with fewer than 256 tiles, as many slices as fit one
// round of 256 workgroups), each slice's fp32 sums
// going to the caller's workspace [S][M][N] and the ordered merge (launch_split_merge)
// adding them, the bias and the rounding. Measured (us, unsplit -> split): 896 x 4864
// INT4 M=65 36.0 -> 11.0, M=256 36.5 -> 17.2, INT8 M=256 34.1 -> 16.1; 3584 x 18944 INT4
// M=128 130 -> 56, M=256 130 -> 91, INT8 M=128 117 -> 46; kept unsplit where it measured
// slower: 14336 x 4096 M=128 (224 tiles of 64 steps) 38.3 vs 40.3, 896 x 4864 M=2048
// 44.7 vs 47.1. LSQ_GEMM_SPLITK=0 turns it off, =n forces n slices (sweeps).
struct GemmSplit {
  int64_t S, bytes;
};

GemmSplit gemm_split_plan(int64_t M, int64_t N, int64_t K, int shape) {
  GemmSplit sp{1, 0};
  if (shape < 0 || K % BK != 0) return sp;
  const int64_t bm = shape == 1 ? 256 : (shape == 0 ? 128 : 64);
  const int64_t bn = shape == 1 ? 256 : (shape == 3 ? 64 : 128);
  const int64_t tiles = ((M + bm - 1) / bm) * ((N + bn - 1) / bn);
  const int64_t steps = K / BK;
  const char* e = std::getenv("LSQ_GEMM_SPLITK");
  if (e && e[0] == '0') return sp;
  const int64_t forced = e ? std::atoi(e) : 0;
  int64_t S = 1;
  if (shape == 1) {  // one workgroup per CU: as many slices as keep the grid to one round
    if (tiles < 256 && steps >= 128) S = 256 / tiles;
  } else if (tiles < 128 || (tiles < 384 && steps >= 128)) {
    S = (512 + tiles - 1) / tiles;
  }
  if (forced >= 2) S = forced;
  S = std::min<int64_t>(S, std::min<int64_t>(16, steps / 8));
  if (S < 2) return sp;
  sp.S = S;
  sp.bytes = S * M * N * 4;
  return sp;
}

// Which prefill kernel: the register-weight kernel with the largest tile that still gives
// the GPU enough workgroups. 256 x 256 above 768 tokens when that makes 112+ tiles (each
// weight dequantized once per 256 activation rows: 14336 x 4096 INT4 g128 M=2048 244 ->
// 219 us, M=8192 ~945 -> 883 us against 128 x 128); else 128 x 128 when that makes 192+
// tiles (14336 x 4096 M=256: 55 us against 77 with 128 x 256 tiles); else 64-row tiles,
// 128 weight rows wide, or for INT4 64 wide once that still leaves fewer than 128 tiles
// (measured, us, 128 x 128 -> chosen shape: 14336 x 4096 M=128 INT4 42.7 -> 34.7, INT8
// 47.6 -> 31.8; 896 x 4864 M=256 INT4 46.3 -> 37.0, INT8 54.4 -> 34.6; 4864 x 896 M=128
// INT4 14.9 -> 10.2; 3584 x 18944 M=256 INT4 168 -> 133, INT8 195 -> 121; 896 x 4864
// M=2048 INT4 96 (256 x 256) -> 41). LSQ_GEMM=reg|wide|mid|small|lds forces 128 x 128,
// 256 x 256, 64 x 128, 64 x 64 or the LDS-weight kernel (tests, tuning). Returns the
// register-weight shape, or -1 for the LDS-weight kernel.
int rw_shape(int64_t M, int64_t N, bool w4) {
  const char* e = std::getenv("LSQ_GEMM");
  if (e && e[0] == 'r') return 0;
  if (e && e[0] == 'w') return 1;
  if (e && e[0] == 'm') return 2;
  if (e && e[0] == 's') return 3;
  if (e && e[0] == 'l') return -1;
  if (M <= 64) return 2;  // (batched-decode sizes: one 64-row tile, split over K)
  auto tiles = [&](int64_t bm, int64_t bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
  if (M > 768 && tiles(256, 256) >= 112) return 1;
  if (tiles(128, 128) >= 192) return 0;
  return w4 && tiles(64, 128) < 128 ? 3 : 2;
}

template <int DT, int KIND, bool GROUPED>
int launch_kind(const LinearArgs& a, hipStream_t s) {
  const int shape = rw_shape(a.M, a.N, KIND == kW4Tiled || KIND == kW4Canon);
  if (shape >= 0) {
    const GemmSplit sp = gemm_split_plan(a.M, a.N, a.K, shape);
    if (sp.S >= 2 && a.part && a.part_bytes >= sp.bytes) {
      LinearArgs as = a;
      as.ksplit = static_cast<int>(sp.S);
      const int rc = launch_rw<DT, KIND, GROUPED, true>(as, shape, s);
      if (rc != LSQ_OK) return rc;
      return launch_split_merge<DT>(a.part, static_cast<int>(sp.S), a.M, a.N, a.bias, a.bias_dt, a.y, a.ldy, s);
    }
    return launch_rw<DT, KIND, GROUPED, false>(a, shape, s);
  }
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

bool gemm_takes_batch(int64_t M, int64_t N, int64_t K) {
  const char* e = std::getenv("LSQ_BATCH_GEMM");
  if (M <= 16 || M > 64 || (e && e[0] == '0')) return false;
  if (e && e[0] == '1') return true;
  return M >= 24 && K >= 12288 && (N + kTileN - 1) / kTileN <= 256;
}

int64_t gemm_split_bytes(int64_t M, int64_t N, int64_t K) {
  if (M <= 16 || (M <= 64 && !gemm_takes_batch(M, N, K))) return 0;  // (the decode kernels take the rest)
  int64_t b = 0;
  for (const bool w4 : {false, true}) b = std::max(b, gemm_split_plan(M, N, K, rw_shape(M, N, w4)).bytes);
  return b;
}

}  // namespace lsq
