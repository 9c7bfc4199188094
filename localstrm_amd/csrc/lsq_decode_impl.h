// Decode-shaped GEMV kernel, M <= 64 tokens with all activations in LDS (gfx950): the kernel
// and its launch helpers, shared by lsq_decode.hip (weight-only entry) and
// lsq_decode_a8.hip (W8A8 entry), which compile their instantiations in parallel.
//
// Decode-shaped weight-only GEMV, M <= 64 tokens with all activations in LDS.
//
// GPU form of QuantizedLinear.forward (src/kernels/quantization.py:129-141) for the
// decode step, where the reference dequantizes the whole [N, K] weight and calls
// F.linear. Here the weights are streamed from HBM exactly once and never materialized.
//
// Work split. Output rows are cut into 16-row tiles (the N side of one
// v_mfma_f32_16x16x32 MFMA) and K into 128-column tiles. The weights are read from the
// tiled layouts (lsq_internal.h: one contiguous 1 KB per wavefront load, each wave
// streaming a contiguous run of tiles, which HBM serves near its streaming rate) or, for
// callers without a tiled copy, from the canonical row-major layouts. A workgroup owns RG x RT row
// tiles and all of K; its RG x KS waves each take RT row tiles and one of KS contiguous
// K slices. Partial sums of the KS slices are added through LDS at the end, in slice
// order, so results do not depend on timing.
//
// Tokens: MB blocks of 16 token rows (MB = 1, 2, 4 for up to 16, 32, 64 tokens); every
// unpacked weight operand feeds MB MFMAs. The launcher uses this kernel whenever the
// activations fit in LDS (e.g. 64 tokens up to K ~ 1100, 32 up to ~2300, 16 up to ~4600).
//
// Prologue. Before the first MFMA each workgroup stages, once, the activations
// x[0:M, 0:K] into LDS (row stride K + 8 elements, already in the column order the
// weight unpack produces, plus one all-zero row), per (128-column tile, token) sums of
// x, used to remove the INT4 nibble bias, and the workgroup's scales and bias as fp32
// (rounded to the activation type). The first D weight steps are issued before the
// staging completes, so their HBM latency overlaps it; after the prologue only the
// weight stream uses the in-order vmcnt counter.
//
// Main loop. Each lane streams 16 bytes (INT4: 32 weights) or 2 x 16 bytes (INT8: 32
// weights) per (row tile, k tile) with non-temporal loads, D steps ahead of use, and
// turns them into the B operand of 4 MFMAs in registers:
//   * INT8: v_cvt_f32_i32 with SDWA byte sign-extension, then v_cvt_pk_bf16_f32 (fp16:
//     v_cvt_pkrtz_f16_f32); integers |q| <= 128 are exact in both types.
//   * INT4: a nibble u = q + 8 OR-ed into the mantissa of 128.0 (bf16 0x4300; fp16
//     1024.0, 0x6400) is exactly 128 + u; the constant part, off = 136 (fp16: 1032),
//     is removed per 128-column tile as s * (acc - off * sum(x)), or once at the end for
//     per-channel scales.
// The activation (A operand) comes from LDS; lanes of token rows >= M read an all-zero
// row (all such lanes of a quad read the same address, an LDS broadcast).
//
// Numerics: every weight product q * x is exact in the fp32 MFMA accumulator; the scale
// is applied in fp32 per group (or per row), then the bias rounded to T, then one
// rounding to T. The reference rounds each dequantized weight round_T(q * s) first and
// then sums in its BLAS order; the two differ by bf16 rounding of the weights, far
// inside the 1e-2 relative contract.

#pragma once

#include "lsq_common.h"
#include "lsq_internal.h"
#include "lsq_decode.h"
#include "lsq_mfma16.h"

#include <atomic>
#include <type_traits>
#include <cstdlib>
#include <cstring>

namespace lsq {
namespace {

constexpr int kXB = 8;  // activation chunks (16 B) per thread per batch, large-M staging
constexpr int kSB = 8;  // scale dwords in flight per thread while staging

// LDS layout, shared by kernel and host: staged activations (M rows + one zero row),
// per-(k tile, token) activation sums, per-token totals, the workgroup's scales and bias
// as fp32 (already rounded to the activation type), cross-slice partial sums.
struct DecodeLds {
  int64_t xs, xsum, xtot, ss, sb, red, xch, total;
};

// Bytes of one staged activation row: K + 8 16-bit values, or (W8A8) K + 16 int8 values.
__host__ __device__ constexpr int64_t x_row_bytes(int64_t K, bool a8) {
  return a8 ? K + 16 : (K + 8) * 2;
}

__host__ __device__ inline DecodeLds decode_lds(int64_t M, int64_t K, int rows, int64_t ngs,
                                                int red_floats, int mp, bool a8,
                                                int xch_floats = 0) {
  DecodeLds l;
  const int64_t nkt = K / kTileK;
  l.xs = 0;
  l.xsum = align16((M + 1) * x_row_bytes(K, a8));
  l.xtot = l.xsum + nkt * mp * 4;
  l.ss = l.xtot + mp * 4;
  l.sb = l.ss + align16(rows * ngs * 4);
  l.red = l.sb + align16(rows * 4);
  l.xch = l.red + static_cast<int64_t>(red_floats) * 4;
  l.total = l.xch + static_cast<int64_t>(xch_floats) * 4;
  return l;
}

// Decode `nd` staged dwords (kSB per thread in `v`, dword index u * NT + tid + t0) of a
// float array with dtype `dt` holding `nelem` elements into dst[] as round_T fp32
// (EXACT: the stored value itself, widened to fp32).
template <int DT, int NT, bool EXACT>
__device__ __forceinline__ void put_floats(const uint32_t (&v)[kSB], int t0, int tid, int dt,
                                           int nelem, float* dst) {
  auto cvt = [](float f) { return EXACT ? f : Act<DT>::round(f); };
#pragma unroll
  for (int u = 0; u < kSB; ++u) {
    const int t = t0 + u * NT + tid;
    if (dt == LSQ_F32) {
      if (t < nelem) dst[t] = cvt(dword_elem(v[u], 0, dt));
    } else {
      if (2 * t < nelem) dst[2 * t] = cvt(dword_elem(v[u], 0, dt));
      if (2 * t + 1 < nelem) dst[2 * t + 1] = cvt(dword_elem(v[u], 1, dt));
    }
  }
}

typedef int i32x4 __attribute__((ext_vector_type(4)));

// W8A8 modes of the decode kernel: activations pre-quantized to int8 (x_q, scale_x from
// lsq_act_quant_i8), or quantized inside the kernel from the T-typed x.
constexpr int kA8Pre = 1, kA8Fused = 2;

// 16-byte activation chunks each thread loads in the prologue's first batch: 8192 chunks
// per 512-thread workgroup covers 16 tokens at K = 4096, 32 at 2048, 64 at 1024.
__host__ __device__ constexpr int prologue_chunks(int nt) {
  return nt >= 8192 ? 1 : (nt >= 512 ? 8192 / nt : 16);
}

// Max of a non-negative float (as its bits) over each row of 16 lanes, in every lane of the
// row (DPP; the bit order of non-negative floats is their value order, NaN above all).
__device__ __forceinline__ uint32_t row16_umax(uint32_t v) {
  v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0xB1, 0xF, 0xF, false)));
  v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x4E, 0xF, 0xF, false)));
  v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x141, 0xF, 0xF, false)));
  v = max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x140, 0xF, 0xF, false)));
  return v;
}

// v_mfma_i32_16x16x64_i8 on registers kept as f32x4 bit patterns (the accumulator
// arrays are shared with the floating-point paths).
__device__ __forceinline__ f32x4 mma_i8(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_bit_cast(
      f32x4, __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, a),
                                                   __builtin_bit_cast(i32x4, b),
                                                   __builtin_bit_cast(i32x4, c), 0, 0, 0));
}

template <int DT, int KIND, int RT, int RG, int KS, int D, bool GROUPED, int MB, int A8>
__global__ void __launch_bounds__(64 * RG * KS) decode_kernel(LinearArgs p) {
  static_assert(!A8 || (KIND == kW8Tiled && !GROUPED), "W8A8 streams the tiled INT8 layout");
  constexpr int MP = 16 * MB;  // token rows covered: MB blocks of 16
  constexpr int NT = 64 * RG * KS;
  // bytes per activation as loaded, and activations per 16-byte chunk
  constexpr int XB = A8 == kA8Pre ? 1 : static_cast<int>(sizeof(typename Act<DT>::storage));
  constexpr int XE = 16 / XB;
  constexpr bool W4 = KIND == kW4Tiled || KIND == kW4Canon;
  constexpr bool TILED = KIND == kW4Tiled || KIND == kW8Tiled;
  constexpr int LPT = W4 ? 1 : 2;  // 16-byte weight loads per lane per (row tile, k tile)
  constexpr int kTileB = W4 ? kTileBytes : kTileBytes8;
  // bytes between consecutive k tiles of one lane, and between a lane's two INT8 loads
  constexpr int kStride = TILED ? kTileB : (W4 ? kTileK / 2 : kTileK);
  constexpr int kHalf = KIND == kW8Tiled ? kTileBytes8 / 2 : 64;
  constexpr int ROWS = RG * RT * kTileN;
  constexpr int RED = KS > 1 ? (KS - 1) * RG * RT * MB * 4 * 64 : 0;
  extern __shared__ __align__(16) unsigned char smem[];
  using S = typename Act<DT>::storage;

  const int M = static_cast<int>(p.M), N = static_cast<int>(p.N), K = static_cast<int>(p.K);
  const int nkt = K / kTileK;
  const int nrt = (N + kTileN - 1) / kTileN;
  const int ng = static_cast<int>(p.ngroups);
  const int ngs = GROUPED ? ng : 1;  // scale columns per row
  const int gtiles = static_cast<int>(p.group / kTileK);
  const int ldxb = static_cast<int>(x_row_bytes(K, A8 != 0));  // LDS bytes per staged row

  // SiLU.mul epilogue: each up-row wave hands its outputs to the gate-row wave beside it
  const bool act = !A8 && p.act == LSQ_ACT_SILU_MUL;  // uniform
  const int XCH = act ? (RG / 2) * RT * MB * 4 * 64 : 0;
  const DecodeLds L = decode_lds(M, K, ROWS, ngs, RED, MP, A8 != 0, XCH);
  unsigned char* xs = smem + L.xs;
  float* xsum = reinterpret_cast<float*>(smem + L.xsum);
  float* xtot = reinterpret_cast<float*>(smem + L.xtot);
  float* ss = reinterpret_cast<float*>(smem + L.ss);
  float* sb = reinterpret_cast<float*>(smem + L.sb);
  float* red = reinterpret_cast<float*>(smem + L.red);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform per wave
  const int rg = wid % RG;
  uint32_t* xmax = reinterpret_cast<uint32_t*>(xtot);  // fused W8A8: per-token max|x| bits
  if (A8 == kA8Fused && tid < MP) xmax[tid] = 0u;
  const int ks = wid / RG;
  const int r = lane & 15;
  const int q = lane >> 4;
  const int rt_wg = blockIdx.x * RG * RT;  // first row tile of the workgroup
  const int row0 = rt_wg * kTileN;
  const int rows_valid = min(ROWS, N - row0);
  const int rtl = rg * RT;  // first row tile of this wave, counted within the workgroup
  const int k_lo = ks * nkt / KS;
  const int nsteps = (ks + 1) * nkt / KS - k_lo;

  // ---- descriptors over what this workgroup reads
  const int es_s = p.scale_dt == LSQ_F32 ? 4 : 2;
  const int es_b = p.bias_dt == LSQ_F32 ? 4 : 2;
  const rsrc_t rx = make_rsrc(p.x, static_cast<uint32_t>(((M - 1) * p.ldx + K) * XB));
  const uint8_t* wbase;
  uint32_t wbytes;
  if (TILED) {
    wbase = p.w + static_cast<int64_t>(rt_wg) * nkt * kTileB;
    wbytes = static_cast<uint32_t>(min(RG * RT, nrt - rt_wg) * nkt * kTileB);
  } else {
    const int row_bytes = W4 ? K / 2 : K;
    wbase = p.w + static_cast<int64_t>(row0) * row_bytes;
    wbytes = static_cast<uint32_t>(rows_valid * row_bytes);
  }
  const rsrc_t rw = make_rsrc(wbase, wbytes);
  const int nsc = rows_valid * ngs;  // scale elements of this workgroup
  const int nsd = (nsc * es_s + 3) / 4;
  // The dword holding the last 16-bit element may extend 2 bytes past the array; an
  // aligned dword never crosses a page, so reading it is always safe.
  const rsrc_t rs = make_rsrc(static_cast<const uint8_t*>(p.scale) +
                                  static_cast<int64_t>(row0) * ngs * es_s,
                              static_cast<uint32_t>(nsd * 4));
  const int nbd = p.bias ? (rows_valid * es_b + 3) / 4 : 0;
  const rsrc_t rb = make_rsrc(p.bias ? static_cast<const uint8_t*>(p.bias) +
                                           static_cast<int64_t>(row0) * es_b
                                     : static_cast<const uint8_t*>(p.scale),
                              static_cast<uint32_t>(nbd * 4));

  // ---- prologue loads, in the order their data is needed: activations, scales, bias,
  // then the first D weight steps.
  const int K8 = K / XE;  // 16-byte chunks per activation row
  const int nchunks = M * K8;
  auto x_off = [&](int c) -> uint32_t {
    const int m = c / K8;
    return c < nchunks ? static_cast<uint32_t>((m * p.ldx + (c - m * K8) * XE) * XB) : kOOB;
  };
  // First batch: XS chunks per thread, all issued at once (one memory round trip):
  // 8192 chunks per 512-thread workgroup covers 16 tokens at K = 4096, 32 at 2048, 64 at
  // 1024. Larger inputs take a second, batched pass after the weight stream is issued.
  constexpr int XS = prologue_chunks(NT);
  u32x4 xv[XS];
#pragma unroll
  for (int u = 0; u < XS; ++u)
    if (u * NT < nchunks) xv[u] = bload16<0>(rx, x_off(u * NT + tid));  // uniform skip
  uint32_t sv[kSB];
#pragma unroll
  for (int u = 0; u < kSB; ++u) {
    const int t = u * NT + tid;
    if (u * NT < nsd) sv[u] = bload4(rs, t < nsd ? t * 4 : kOOB);  // uniform skip
  }
  const uint32_t bv = bload4(rb, tid < nbd ? tid * 4 : kOOB);  // ROWS * 4 bytes <= 4 * NT
  float sxv = 0.f;  // pre-quantized W8A8: this thread's token scale
  if (A8 == kA8Pre && tid < M) sxv = p.xscale[tid];
  // ---- activations -> LDS (in the unpack's column order) and per-(k tile, token) sums
  // Sum of a float over each row of 16 lanes, in every lane of the row (DPP, no LDS).
  auto row16_sum = [](float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
    return v;
  };
  auto put_x = [&](const auto& v, int c0, auto nb) {
#pragma unroll
    for (int u = 0; u < decltype(nb)::value; ++u) {
      if (c0 + u * NT >= nchunks) break;  // uniform
      const int c = c0 + u * NT + tid;
      const int m = c / K8;
      const int c8 = c - m * K8;
      float sum = 0.f;
      if (c < nchunks) {
        *reinterpret_cast<u32x4*>(xs + m * ldxb + c8 * 16) = KIND == kW4Canon ? permute_canon(v[u]) : v[u];
        if constexpr (W4) {
#pragma unroll
          for (int e = 0; e < 4; ++e) sum += Mma<DT>::lo(v[u][e]) + Mma<DT>::hi(v[u][e]);
        }
      }
      if constexpr (W4) {
        // 16 consecutive lanes hold the 16 chunks of one (token, k tile); all valid or none
        sum = row16_sum(sum);
        if (c < nchunks && (lane & 15) == 0) xsum[(c8 / 16) * MP + m] = sum;
      }
    }
  };
  // Staging of what the prologue loaded, done after the first weight steps are issued:
  // these loads were issued before the weights, so waiting for them leaves the weight
  // loads in flight.
  // Fused W8A8: per-token max|x| (16-lane DPP max, then one LDS atomic max per row of 16
  // lanes, which always lie in one token row since K8 and NT are multiples of 16), then
  // each thread quantizes the chunks it holds and stores them as int8 rows.
  auto put_xq = [&]() {
    lds_barrier();  // xmax[] zeroed at entry
#pragma unroll
    for (int u = 0; u < XS; ++u) {
      if (u * NT >= nchunks) break;  // uniform
      const int c = u * NT + tid;
      uint32_t mx = 0u;
      if (c < nchunks) {
#pragma unroll
        for (int e = 0; e < XE; ++e) {
          const float f = XB == 4 ? __uint_as_float(xv[u][e])
                                  : Act<DT>::to_f32(static_cast<uint16_t>(xv[u][e >> 1] >> (16 * (e & 1))));
          mx = max(mx, __float_as_uint(fabsf(f)));
        }
      }
      mx = row16_umax(mx);
      if (c < nchunks && (lane & 15) == 0) atomicMax(&xmax[c / K8], mx);
    }
    lds_barrier();
#pragma unroll
    for (int u = 0; u < XS; ++u) {
      if (u * NT >= nchunks) break;  // uniform
      const int c = u * NT + tid;
      if (c < nchunks) {
        const int m = c / K8;
        const int c8 = c - m * K8;
        const float sc = a8_scale<DT>(__uint_as_float(xmax[m]));
        const float rc = __builtin_amdgcn_rcpf(sc);
        uint32_t o[XE / 4];
#pragma unroll
        for (int d = 0; d < XE / 4; ++d) {
          uint32_t b = 0;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int ee = 4 * d + e;
            const float f = XB == 4 ? __uint_as_float(xv[u][ee])
                                    : Act<DT>::to_f32(static_cast<uint16_t>(xv[u][ee >> 1] >> (16 * (ee & 1))));
            b |= (static_cast<uint32_t>(quant_i8_fast(f, sc, rc)) & 0xFFu) << (8 * e);
          }
          o[d] = b;
        }
        if constexpr (XE == 8) *reinterpret_cast<uint2*>(xs + m * ldxb + c8 * 8) = make_uint2(o[0], o[1]);
        else *reinterpret_cast<uint32_t*>(xs + m * ldxb + c8 * 4) = o[0];
      }
    }
  };
  auto stage_first = [&]() {
    if constexpr (A8 == kA8Fused) put_xq();
    else put_x(xv, 0, std::integral_constant<int, XS>());
    put_floats<DT, NT, (A8 != 0)>(sv, 0, tid, p.scale_dt, nsc, ss);
    // W8A8 adds the bias as stored (widened to fp32); weight-only rounds it to T first
    auto cvt = [](float f) { return A8 ? f : Act<DT>::round(f); };
    if (p.bias && tid < nbd) {
      if (es_b == 4) {
        sb[tid] = cvt(dword_elem(bv, 0, LSQ_F32));
      } else {
        if (2 * tid < rows_valid) sb[2 * tid] = cvt(dword_elem(bv, 0, p.bias_dt));
        if (2 * tid + 1 < rows_valid) sb[2 * tid + 1] = cvt(dword_elem(bv, 1, p.bias_dt));
      }
    }
    if (A8 == kA8Pre && tid < MP) xtot[tid] = sxv;
  };
  // Keep the scheduler from moving any of the loads above below the weight stream:
  // their consumers then wait only for them, not for the weights.
  __builtin_amdgcn_sched_barrier(0);

  // Weight stream: a ring of D k-tile steps per wave; refills past the end of the slice
  // are out-of-range loads (no memory traffic), so every load is unconditional and the
  // compiler waits for exactly the step being consumed while D - 1 stay in flight.
  u32x4 wbuf[D][RT][LPT];
  auto issue = [&](u32x4 (&wv)[RT][LPT], int st) {
    const int kt = k_lo + st;
    const bool real = st < nsteps;
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      const int lt = rtl + i;
      const uint32_t off = TILED ? static_cast<uint32_t>((lt * nkt + kt) * kTileB + lane * 16)
                                 : static_cast<uint32_t>((lt * kTileN + r) * (W4 ? K / 2 : K) +
                                                         kt * kStride + q * 16);
      wv[i][0] = bload16<kNT>(rw, real ? off : kOOB);
      if (LPT == 2) wv[i][LPT - 1] = bload16<kNT>(rw, real ? off + kHalf : kOOB);
    }
  };
#pragma unroll
  for (int s = 0; s < D; ++s) issue(wbuf[s], s);

  stage_first();
  // Activations or scales beyond the first batch (many tokens, or many scale groups) are
  // loaded and staged now, while the first D weight steps are in flight (the loop's waits
  // also cover the weights, which are needed next anyway).
  // (the fused W8A8 launch is only made when all activations fit in the first batch)
  const bool big = nchunks > NT * XS || nsd > NT * kSB;  // uniform
  if (big) {
    for (int c0 = NT * XS; A8 != kA8Fused && c0 < nchunks; c0 += NT * kXB) {
      u32x4 xb[kXB];
#pragma unroll
      for (int u = 0; u < kXB; ++u) xb[u] = bload16<0>(rx, x_off(c0 + u * NT + tid));
      put_x(xb, c0, std::integral_constant<int, kXB>());
    }
    for (int t0 = NT * kSB; t0 < nsd; t0 += NT * kSB) {
#pragma unroll
      for (int u = 0; u < kSB; ++u) {
        const int t = t0 + u * NT + tid;
        sv[u] = bload4(rs, t < nsd ? t * 4 : kOOB);
      }
      put_floats<DT, NT, (A8 != 0)>(sv, t0, tid, p.scale_dt, nsc, ss);
    }
  }
  // row M: zeros, read by lanes of token rows >= M (K bytes for int8 rows, 2 K for 16-bit)
  for (int c = tid; c < (A8 ? K / 16 : K / 8); c += NT)
    *reinterpret_cast<u32x4*>(xs + M * ldxb + c * 16) = u32x4{0u, 0u, 0u, 0u};
  lds_barrier();
  if (W4 && !GROUPED) {
    if (tid < MP) {
      float t = 0.f;
      if (tid < M)
        for (int kt = 0; kt < nkt; ++kt) t += xsum[kt * MP + tid];
      xtot[tid] = t;
    }
    lds_barrier();
  }

  // ---- main loop
  f32x4 acc[RT][MB];
#pragma unroll
  for (int i = 0; i < RT; ++i)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[i][mb] = f32x4{0.f, 0.f, 0.f, 0.f};
  const unsigned char* xrow[MB];  // token rows >= M read the zero row
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) xrow[mb] = xs + min(16 * mb + r, M) * ldxb;
  // Constants of the INT4 unpack in registers, so it selects v_and_or_b32 (VOP3 has no
  // literal operands on gfx9).
  uint32_t nib_mask = 0, magic = 0;
  if constexpr (W4) {
    asm volatile("v_mov_b32 %0, 0x000f000f" : "=v"(nib_mask));
    asm volatile("v_mov_b32 %0, %1" : "=v"(magic) : "i"(Mma<DT>::kMagic));
  }

  const int nblocks = (nsteps + D - 1) / D;
  for (int b = 0; b < nblocks; ++b) {
#pragma unroll
    for (int s = 0; s < D; ++s) {
      const int st = b * D + s;
      // Order within a step: LDS reads (independent of the weights, so they overlap the
      // wait for this step's weights), unpack, refill of the ring slot just freed, then
      // the MFMAs and the scale math, so that the next load leaves before the MFMA chain.
      const bool live = st < nsteps;  // uniform; dead steps of the last block only refill
      const int kt = k_lo + st;
      if constexpr (A8) {
        // W8A8: the raw int8 weights are the B operand of v_mfma_i32_16x16x64_i8 as
        // loaded; lane quad q, load j holds columns 32 q + 16 j .. +15 of the k tile,
        // and the activation operand is the same 16 columns of the token row.
        u32x4 a8[MB][2], b8[RT][2];
        if (live) {
#pragma unroll
          for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int j = 0; j < 2; ++j)
              a8[mb][j] = *reinterpret_cast<const u32x4*>(xrow[mb] + kt * kTileK + 32 * q + 16 * j);
#pragma unroll
          for (int i = 0; i < RT; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) b8[i][j] = wbuf[s][i][j];
        }
        issue(wbuf[s], st + D);
        if (live) {
#pragma unroll
          for (int i = 0; i < RT; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
              for (int mb = 0; mb < MB; ++mb) acc[i][mb] = mma_i8(a8[mb][j], b8[i][j], acc[i][mb]);
        }
      } else {
        u32x4 a[MB][4];
        f32x4 xo[MB];
        float scg[RT];
        u32x4 bb[RT][4];
        if (live) {
#pragma unroll
          for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int d = 0; d < 4; ++d)
              a[mb][d] = *reinterpret_cast<const u32x4*>(xrow[mb] + (kt * kTileK + a_col<KIND>(q, d)) * 2);
          if (W4 && GROUPED) {
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
              xo[mb] = *reinterpret_cast<const f32x4*>(xsum + kt * MP + 16 * mb + 4 * q);
            const int g = gtiles == 1 ? kt : kt / gtiles;
#pragma unroll
            for (int i = 0; i < RT; ++i) scg[i] = ss[((rtl + i) * kTileN + r) * ngs + g];
          }
#pragma unroll
          for (int i = 0; i < RT; ++i)
#pragma unroll
            for (int d = 0; d < 4; ++d)
              bb[i][d] = W4 ? unpack_w4(wbuf[s][i][0][d], nib_mask, magic)
                            : convert_w8<DT>(wbuf[s][i][d >> 1][2 * (d & 1)],
                                             wbuf[s][i][d >> 1][2 * (d & 1) + 1]);
        }
        issue(wbuf[s], st + D);
        if (live) {
#pragma unroll
          for (int i = 0; i < RT; ++i) {
            if (W4 && GROUPED) {
              f32x4 dacc[MB];
#pragma unroll
              for (int mb = 0; mb < MB; ++mb) dacc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
              for (int d = 0; d < 4; ++d)
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) dacc[mb] = Mma<DT>::mma(a[mb][d], bb[i][d], dacc[mb]);
#pragma unroll
              for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                  acc[i][mb][e] = fmaf(scg[i], fmaf(-Mma<DT>::kOff4, xo[mb][e], dacc[mb][e]), acc[i][mb][e]);
            } else {
#pragma unroll
              for (int d = 0; d < 4; ++d)
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) acc[i][mb] = Mma<DT>::mma(a[mb][d], bb[i][d], acc[i][mb]);
            }
          }
        }
      }
    }
  }

  // ---- cross-slice reduction (fixed slice order), epilogue
  if (KS > 1) {
    if (ks > 0) {
#pragma unroll
      for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            red[(((((ks - 1) * RG + rg) * RT + i) * MB + mb) * 4 + e) * 64 + lane] = acc[i][mb][e];
    }
    lds_barrier();
    if (ks == 0) {  // (waves of the other slices stay alive for the SiLU.mul barrier)
#pragma unroll
      for (int kk = 0; kk < KS - 1; ++kk)
#pragma unroll
        for (int i = 0; i < RT; ++i)
#pragma unroll
          for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float v = red[((((kk * RG + rg) * RT + i) * MB + mb) * 4 + e) * 64 + lane];
              if constexpr (A8)  // int32 partial sums (exact, in any order)
                acc[i][mb][e] = __int_as_float(__float_as_int(acc[i][mb][e]) + __float_as_int(v));
              else
                acc[i][mb][e] += v;
            }
    }
  }

  S* y = static_cast<S*>(p.y);
  if constexpr (!A8) {
    if (act) {
      // Row tile 2t holds gate rows 16t.., tile 2t + 1 the up rows of the same outputs
      // (RT == 1 and RG even, so the pair is waves rg, rg + 1 of one workgroup). Each
      // value is first rounded to T as its own layer would output it; then
      // y = round_T(round_T(silu(g)) * u), as F.silu(gate) * up evaluates it.
      float* xch = reinterpret_cast<float*>(smem + L.xch);
      const int rl = rtl * kTileN + r;
      const float sc = GROUPED ? 1.f : ss[rl];
      const float bias = p.bias ? sb[rl] : 0.f;
      float vt[MB][4];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float v = acc[0][mb][e];
          if constexpr (W4 && !GROUPED) v = fmaf(-Mma<DT>::kOff4, xtot[16 * mb + 4 * q + e], v);
          vt[mb][e] = Act<DT>::round(opaque(GROUPED ? v + bias : fmaf(v, sc, bias)));
        }
      const bool up = (rg & 1) != 0;
      if (ks == 0 && up) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int e = 0; e < 4; ++e) xch[(((rg >> 1) * MB + mb) * 4 + e) * 64 + lane] = vt[mb][e];
      }
      lds_barrier();
      if (ks == 0 && !up) {
        const int j = ((rt_wg + rtl) >> 1) * kTileN + r;  // output column
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int m = 16 * mb + 4 * q + e;
            const float g = vt[mb][e];
            const float u = xch[(((rg >> 1) * MB + mb) * 4 + e) * 64 + lane];
            const float sg = Act<DT>::round(opaque(g / (1.f + expf(-g))));
            // fp32 product, then the rounding to T (not one fused multiply-round)
            if (m < M && 2 * j < N) y[static_cast<int64_t>(m) * p.ldy + j] = Act<DT>::from_f32(opaque(sg * u));
          }
      }
      return;
    }
  }
  if (ks > 0) return;
#pragma unroll
  for (int i = 0; i < RT; ++i) {
    const int rl = (rtl + i) * kTileN + r;  // row within the workgroup
    const int n = row0 + rl;
    const float sc = GROUPED ? 1.f : ss[rl];
    const float bias = p.bias ? sb[rl] : 0.f;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = 16 * mb + 4 * q + e;
        if (m < M && n < N) {
          if constexpr (A8) {
            // float(acc) * (sx * sw) [+ bias], each an fp32 rounding, then round to T
            const float sxm = A8 == kA8Fused ? a8_scale<DT>(xtot[m]) : xtot[m];
            float v = mul_nc(static_cast<float>(__float_as_int(acc[i][mb][e])), mul_nc(sxm, sc));
            if (p.bias) v = add_nc(v, bias);
            y[static_cast<int64_t>(m) * p.ldy + n] = Act<DT>::from_f32(opaque(v));
          } else {
            float v = acc[i][mb][e];
            if constexpr (W4 && !GROUPED) v = fmaf(-Mma<DT>::kOff4, xtot[m], v);
            // scale and bias as one explicit FMA, so every code shape rounds alike
            y[static_cast<int64_t>(m) * p.ldy + n] = Act<DT>::from_f32(opaque(GROUPED ? v + bias : fmaf(v, sc, bias)));
          }
        }
      }
  }
}

// ------------------------------------------------------------------ launch

struct Cfg {
  int rt, rg, ks, d;
};

// Configurations compiled in (rt, rg, ks, d). The first one is the fallback default.
#define LSQ_DECODE_CONFIGS(X) \
  X(1, 8, 1, 4)               \
  X(1, 4, 2, 8)               \
  X(1, 2, 4, 4)               \
  X(1, 1, 8, 4)               \
  X(1, 2, 2, 8)               \
  X(1, 2, 4, 8)               \
  X(1, 1, 4, 8)               \
  X(1, 4, 4, 4)               \
  X(1, 8, 1, 6)               \
  X(1, 6, 2, 4)

int g_max_lds = -1;

int max_lds_bytes() {
  int v = g_max_lds;
  if (v < 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
      v = 64 * 1024;
    g_max_lds = v;
  }
  return v;
}

// LSQ_DECODE_CFG="rt,rg,ks,d" overrides the heuristic with a compiled-in configuration
// (for tuning sweeps); read once.
bool env_cfg(Cfg* out) {
  static int state = 0;  // 0 unread, 1 none, 2 set
  static Cfg c{};
  if (state == 0) {
    const char* e = std::getenv("LSQ_DECODE_CFG");
    state = 1;
    if (e && std::sscanf(e, "%d,%d,%d,%d", &c.rt, &c.rg, &c.ks, &c.d) == 4) state = 2;
  }
  if (state == 2) *out = c;
  return state == 2;
}

// Every wave streams one row tile over one K slice. Large layers: at most one workgroup
// per CU, 2 K slices per row tile where that still fits (see below). Small layers: split K
// so that there are at least ~1024 waves, each with at least a few k tiles.
Cfg pick_cfg(int kind, int64_t M, int64_t N, int64_t K) {
  Cfg c;
  if (env_cfg(&c)) return c;
  (void)M;
  const int64_t nrt = (N + kTileN - 1) / kTileN;
  const int64_t nkt = K / kTileK;
  // INT8 moves twice the bytes per tile and keeps a 6-step ring busy (measured 3-7 %
  // faster than 4 at 18944 x 3584); INT4 is fastest with 4.
  // Large N: up to 1536 row tiles (N <= 24576), 6 row tiles x 2 K slices per workgroup
  // keep every workgroup on its own CU (198 at N = 18944, 12 waves each); measured 9-14 %
  // faster than 8 row tiles of unsplit K (148 workgroups, 108 CUs idle) at 18944 x 3584,
  // INT8 and INT4, M = 1 to 16. Beyond that, 8 row tiles of unsplit K.
  if (nrt >= 1024) {
    if (nrt <= 6 * 256 && nkt >= 8) return Cfg{1, 6, 2, 4};
    return (kind == kW8 || kind == kW8Tiled) ? Cfg{1, 8, 1, 6} : Cfg{1, 8, 1, 4};
  }
  // Fewer than 8 k tiles (K < 1024, e.g. hidden 896): split K 4 ways over pairs of row
  // tiles (N up to ~8K), 2 ways over 4 row tiles above; measured 20-26 % faster than 8 row
  // tiles of unsplit K at 896 x 896 and 4864 x 896 (M = 1 and 32), which launch 7-38
  // workgroups.
  if (nkt < 8) return nrt < 512 ? Cfg{1, 2, 4, 4} : Cfg{1, 4, 2, 8};
  if (nrt * 2 >= 1024 || nkt < 16) return Cfg{1, 4, 2, 8};
  if (nrt * 4 >= 1024 || nkt < 32) return Cfg{1, 2, 4, 4};
  return Cfg{1, 1, 8, 4};
}

template <int DT, int KIND, int RT, int RG, int KS, int D, bool GROUPED, int MB, int A8>
int launch_one(const LinearArgs& a, hipStream_t s) {
  constexpr int RED = KS > 1 ? (KS - 1) * RG * RT * MB * 4 * 64 : 0;
  if (A8 == kA8Fused) {  // every activation chunk must be in the prologue's first batch
    constexpr int XE = 16 / static_cast<int>(sizeof(typename Act<DT>::storage));
    if (a.M * (a.K / XE) > int64_t(64 * RG * KS) * prologue_chunks(64 * RG * KS)) return LSQ_E_LAYOUT;
  }
  const bool grouped = a.group < a.K;
  const int XCH = (!A8 && a.act == LSQ_ACT_SILU_MUL) ? (RG / 2) * RT * MB * 4 * 64 : 0;
  if (XCH && (RT != 1 || RG % 2 != 0)) return LSQ_E_LAYOUT;
  const DecodeLds L = decode_lds(a.M, a.K, RG * RT * kTileN, grouped ? a.ngroups : 1, RED, 16 * MB,
                                 A8 != 0, XCH);
  if (L.total > max_lds_bytes()) return LSQ_E_LAYOUT;
  auto kern = decode_kernel<DT, KIND, RT, RG, KS, D, GROUPED, MB, A8>;
  if (L.total > 64 * 1024) {
    static std::atomic<int> attr_set{0};
    if (!attr_set.load(std::memory_order_acquire)) {
      const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                               hipFuncAttributeMaxDynamicSharedMemorySize,
                                               max_lds_bytes());
      if (e != hipSuccess) return static_cast<int>(e);
      attr_set.store(1, std::memory_order_release);
    }
  }
  const int64_t nrt = (a.N + kTileN - 1) / kTileN;
  const dim3 grid(static_cast<unsigned>((nrt + RG * RT - 1) / (RG * RT)));
  kern<<<grid, dim3(64 * RG * KS), static_cast<size_t>(L.total), s>>>(a);
  return static_cast<int>(hipGetLastError());
}

template <int DT, int KIND, bool GROUPED, int A8 = 0>
int launch_kind(const LinearArgs& a, hipStream_t s) {
  Cfg c = pick_cfg(KIND, a.M, a.N, a.K);
  if (a.act && (c.rt != 1 || c.rg % 2 != 0)) c = Cfg{1, 2, 4, 4};  // gate / up tile pairs
  if (a.M > 16) {
    // 17..64 tokens in 2 or 4 blocks of 16; only the configurations pick_cfg returns
#define LSQ_TRY_MB(RT_, RG_, KS_, D_)                                                   \
    if (c.rt == RT_ && c.rg == RG_ && c.ks == KS_ && c.d == D_)                          \
      return a.M <= 32 ? launch_one<DT, KIND, RT_, RG_, KS_, D_, GROUPED, 2, A8>(a, s)   \
                       : launch_one<DT, KIND, RT_, RG_, KS_, D_, GROUPED, 4, A8>(a, s);
    LSQ_TRY_MB(1, 8, 1, 4)
    LSQ_TRY_MB(1, 4, 2, 8)
    LSQ_TRY_MB(1, 2, 4, 4)
    LSQ_TRY_MB(1, 1, 8, 4)
    LSQ_TRY_MB(1, 6, 2, 4)
#undef LSQ_TRY_MB
    return a.M <= 32 ? launch_one<DT, KIND, 1, 8, 1, 4, GROUPED, 2, A8>(a, s)
                     : launch_one<DT, KIND, 1, 8, 1, 4, GROUPED, 4, A8>(a, s);
  }
#define LSQ_TRY(RT_, RG_, KS_, D_)                                        \
  if (c.rt == RT_ && c.rg == RG_ && c.ks == KS_ && c.d == D_)             \
    return launch_one<DT, KIND, RT_, RG_, KS_, D_, GROUPED, 1, A8>(a, s);
  LSQ_DECODE_CONFIGS(LSQ_TRY)
#undef LSQ_TRY
  return launch_one<DT, KIND, 1, 8, 1, 4, GROUPED, 1, A8>(a, s);
}

}  // namespace

}  // namespace lsq
