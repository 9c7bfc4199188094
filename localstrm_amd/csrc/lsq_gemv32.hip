// Decode GEMV for fp32 activations, 1..8 tokens per launch, on the tiled INT4 / INT8 layouts
// (gfx950).
//
// GPU form of QuantizedLinear.forward (src/kernels/quantization.py:104-141) when x is fp32,
// the type the reference's CPU path runs in: y = x W^T + b with every weight formed as the
// reference's dequantize() forms it, W = round_fp32(q * s) (q = u - 8 for INT4), and the
// products summed in fp32 with fmaf. At one or two tokens the arithmetic (a conversion, the
// scale product and one FMA per token and weight) keeps pace with the weight stream on the
// VALU; at 8 tokens it bounds the kernel (an fp32 MFMA taking the rounded weights as its B
// operand would take over the FMAs there).
//
// Work split as the 1..16-token GEMV (lsq_gemv.hip): balanced ranges of whole 16-row tiles
// per workgroup, the workgroup's (row tile, k tile) units cut into W contiguous runs, one
// per wave, a run spanning at most two row tiles. Lane l of a unit owns row l & 15 and the
// 32 columns 32 (l >> 4) .. +31 of the k tile (the tiled layouts' lane order: lsq_internal.h),
// so it needs 32 consecutive activations per token, read from the workgroup's LDS copy of
// x; the four lanes of a row add their sums with two shuffles at the end of the run, and
// the last wave of a row tile to arrive adds the waves' sums in wave order (fixed order:
// results do not depend on timing).

#include "lsq_common.h"
#include "lsq_internal.h"
#include "lsq_decode.h"

#include <atomic>
#include <cstdlib>

namespace lsq {
namespace {

// LDS layout (byte offsets): per-wave row sums (two slots of MT x 16 floats), one arrival
// counter per row tile, x [MT][K] as fp32, the workgroup's scales [rows][ngs] and bias as
// fp32.
struct G32Lds {
  int64_t red, cnt, xs, ss, sb, total;
};

__host__ __device__ inline G32Lds g32_lds(int64_t MT, int64_t K, int64_t rows, int64_t ngs, int W) {
  G32Lds l;
  l.red = 0;
  l.cnt = int64_t(W) * 2 * MT * 16 * 4;
  l.xs = (l.cnt + int64_t(W) * 4 + 15) & ~int64_t(15);
  l.ss = l.xs + MT * K * 4;
  l.sb = l.ss + rows * ngs * 4;
  l.total = l.sb + rows * 4;
  return l;
}

// Byte J of v as a float (v_cvt_f32_ubyte J: the compiler otherwise extracts bytes 1-3
// with a separate v_bfe_u32 each).
template <int J>
__device__ __forceinline__ float ubyte_f32(uint32_t v) {
  float f;
  if constexpr (J == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(f) : "v"(v));
  else if constexpr (J == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(f) : "v"(v));
  else if constexpr (J == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(f) : "v"(v));
  else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(f) : "v"(v));
  return f;
}

template <bool W4, bool GROUPED, int MT, int W, int D>
__global__ void __launch_bounds__(64 * W) gemv32_kernel(LinearArgs p) {
  constexpr int NT = 64 * W;
  constexpr int kTileB = W4 ? kTileBytes : kTileBytes8;
  constexpr int LPT = W4 ? 1 : 2;  // 16-byte weight loads per lane per unit
  extern __shared__ __align__(16) unsigned char smem[];

  const int M = static_cast<int>(p.M), N = static_cast<int>(p.N), K = static_cast<int>(p.K);
  const int nkt = K / kTileK;
  const int nrt = (N + kTileN - 1) / kTileN;
  const int ngs = GROUPED ? static_cast<int>(p.ngroups) : 1;
  const int gshift = GROUPED ? __builtin_ctz(static_cast<uint32_t>(p.group / kTileK)) : 0;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, q = lane >> 4;
  // row tiles of this workgroup: the first `rem` take base + 1
  const int G = gridDim.x, b = blockIdx.x;
  const int base = nrt / G, rem = nrt - base * G;
  const int rt_lo = b * base + min(b, rem);
  const int R = base + (b < rem ? 1 : 0);
  const int rmax = base + (rem > 0 ? 1 : 0);
  const int T = R * nkt;
  const int t_lo = wid * T / W, t_hi = (wid + 1) * T / W;
  const int row0 = rt_lo * kTileN;
  const int rows_valid = min(R * kTileN, N - row0);

  const G32Lds L = g32_lds(MT, K, int64_t(rmax) * kTileN, ngs, W);
  float* red = reinterpret_cast<float*>(smem + L.red);
  int* cnt = reinterpret_cast<int*>(smem + L.cnt);
  float* xs = reinterpret_cast<float*>(smem + L.xs);
  float* ss = reinterpret_cast<float*>(smem + L.ss);
  float* sb = reinterpret_cast<float*>(smem + L.sb);

  // ---- the weight ring: unit i of this wave's run is k tile kt0 + i of its first row
  // tile, or (from kt0 + i = nkt on) of the next one; refills past the run are
  // out-of-range loads (no data moved, no branch)
  const rsrc_t rw = make_rsrc(p.w + static_cast<int64_t>(rt_lo) * nkt * kTileB,
                              static_cast<uint32_t>(R * nkt * kTileB));
  const int rt_first = t_lo / nkt;
  const int kt0 = t_lo - rt_first * nkt;
  const uint32_t u_base = static_cast<uint32_t>(t_lo * kTileB + lane * 16);
  u32x4 wbuf[D][LPT];
  auto issue = [&](u32x4 (&wv)[LPT], int i) {
    const uint32_t off = t_lo + i < t_hi ? u_base + static_cast<uint32_t>(i * kTileB) : kOOB;
    wv[0] = bload16<kNT>(rw, off);
    if (LPT == 2) wv[LPT - 1] = bload16<kNT>(rw, off == kOOB ? kOOB : off + kTileB / 2);
  };
#pragma unroll
  for (int s = 0; s < D; ++s) issue(wbuf[s], s);

  // ---- prologue: x, the scales and the bias of the workgroup's rows, as fp32, into LDS
  {
    const int k4 = K / 4;
    for (int c = tid; c < M * k4; c += NT) {
      const int m = c / k4, kc = c - m * k4;
      *reinterpret_cast<float4*>(xs + m * K + 4 * kc) =
          *reinterpret_cast<const float4*>(static_cast<const float*>(p.x) + static_cast<int64_t>(m) * p.ldx + 4 * kc);
    }
    for (int i = tid; i < rows_valid * ngs; i += NT)
      ss[i] = load_as_f32(p.scale, p.scale_dt, static_cast<int64_t>(row0) * ngs + i);
    for (int i = tid; i < rows_valid; i += NT)
      sb[i] = p.bias ? load_as_f32(p.bias, p.bias_dt, row0 + i) : 0.f;
    if (tid < R) cnt[tid] = 0;
  }
  lds_barrier();

  // ---- main loop: per unit, 32 weights of row r against 32 activations per token
  float acc_a[MT], acc_b[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) acc_a[m] = acc_b[m] = 0.f;
  const int n_my = t_hi - t_lo;
  const float* srow_a = ss + (rt_first * kTileN + r) * ngs;
  const float* srow_b = srow_a + kTileN * ngs;
  for (int i0 = 0; i0 < n_my; i0 += D) {
#pragma unroll
    for (int s = 0; s < D; ++s) {
      const int i = i0 + s;
      const bool live = i < n_my;  // uniform
      const int kk = kt0 + i;
      const bool second = kk >= nkt;  // uniform
      const int kt = second ? kk - nkt : kk;
      u32x4 wv[LPT];
#pragma unroll
      for (int l = 0; l < LPT; ++l) wv[l] = wbuf[s][l];
      issue(wbuf[s], i + D);
      if (live) {
        const float sc = (second ? srow_b : srow_a)[GROUPED ? (kt >> gshift) : 0];
        const float c8 = -8.f * sc;  // exact
        const float* xk = xs + kt * kTileK + 32 * q;
        float part[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) part[m] = 0.f;
#pragma unroll
        for (int d = 0; d < 4; ++d) {  // 8 columns 32 q + 8 d .. +7 per step
          float wq[8];
          if constexpr (W4) {
            // nibble p holds column 8 d + tiled_nibble_k(p); byte j of `lo` / `hi` is nibble
            // 2 j / 2 j + 1 (v_cvt_f32_ubyte j). (u - 8) s = fma(u, s, -8 s) with one
            // rounding: u s and -8 s are exact, so this is round_fp32((u - 8) s).
            const uint32_t wd = wv[0][d];
            const uint32_t lo = wd & 0x0F0F0F0Fu, hi = (wd >> 4) & 0x0F0F0F0Fu;
            wq[tiled_nibble_k(0)] = fmaf(ubyte_f32<0>(lo), sc, c8);
            wq[tiled_nibble_k(1)] = fmaf(ubyte_f32<0>(hi), sc, c8);
            wq[tiled_nibble_k(2)] = fmaf(ubyte_f32<1>(lo), sc, c8);
            wq[tiled_nibble_k(3)] = fmaf(ubyte_f32<1>(hi), sc, c8);
            wq[tiled_nibble_k(4)] = fmaf(ubyte_f32<2>(lo), sc, c8);
            wq[tiled_nibble_k(5)] = fmaf(ubyte_f32<2>(hi), sc, c8);
            wq[tiled_nibble_k(6)] = fmaf(ubyte_f32<3>(lo), sc, c8);
            wq[tiled_nibble_k(7)] = fmaf(ubyte_f32<3>(hi), sc, c8);
          } else {
            const uint32_t w0 = wv[d >> 1][2 * (d & 1)], w1 = wv[d >> 1][2 * (d & 1) + 1];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              wq[e] = mul_rn(static_cast<float>(static_cast<int8_t>(w0 >> (8 * e))), sc);
              wq[4 + e] = mul_rn(static_cast<float>(static_cast<int8_t>(w1 >> (8 * e))), sc);
            }
          }
#pragma unroll
          for (int m = 0; m < MT; ++m) {
            const float4 x0 = *reinterpret_cast<const float4*>(xk + m * K + 8 * d);
            const float4 x1 = *reinterpret_cast<const float4*>(xk + m * K + 8 * d + 4);
            float v = part[m];
            v = fmaf(x0.x, wq[0], v); v = fmaf(x0.y, wq[1], v); v = fmaf(x0.z, wq[2], v); v = fmaf(x0.w, wq[3], v);
            v = fmaf(x1.x, wq[4], v); v = fmaf(x1.y, wq[5], v); v = fmaf(x1.z, wq[6], v); v = fmaf(x1.w, wq[7], v);
            part[m] = v;
          }
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          acc_a[m] = second ? acc_a[m] : acc_a[m] + part[m];
          acc_b[m] = second ? acc_b[m] + part[m] : acc_b[m];
        }
      }
    }
  }

  // ---- epilogue: the 4 lanes of a row, then the waves of a row tile in wave order
  auto first_wave = [&](int j) { return (j * nkt * W + W - 1) / T; };
  auto last_wave = [&](int j) { return ((j + 1) * nkt * W - 1) / T; };
  float* y = static_cast<float*>(p.y);
  auto finish = [&](int j) {  // lanes 0..15: row r of row tile j
    if (lane < 16) {
      const int rl = j * kTileN + r;
      const int n = row0 + rl;
      const int wb = last_wave(j);
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        float v = 0.f;
        for (int w2 = first_wave(j); w2 <= wb; ++w2) {
          const int slot = (w2 * R) / W == j ? 0 : 1;
          v += red[((w2 * 2 + slot) * MT + m) * 16 + r];
        }
        if (m < M && n < N) y[static_cast<int64_t>(m) * p.ldy + n] = v + sb[rl];
      }
    }
  };
  auto publish = [&](int j, int slot, float (&acc)[MT]) {
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      float v = acc[m];
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      if (lane < 16) red[((wid * 2 + slot) * MT + m) * 16 + r] = v;
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the sums are in LDS before the count
    int old = 0;
    if (lane == 0) old = atomicAdd(&cnt[j], 1);
    old = __builtin_amdgcn_readfirstlane(old);
    if (old == last_wave(j) - first_wave(j)) finish(j);
  };
  publish(rt_first, 0, acc_a);
  if (kt0 + n_my > nkt) publish(rt_first + 1, 1, acc_b);
}

// ------------------------------------------------------------------ launch

int g_gemv32_max_lds = -1;

int gemv32_max_lds() {
  int v = g_gemv32_max_lds;
  if (v < 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
      v = 64 * 1024;
    g_gemv32_max_lds = v;
  }
  return v;
}

template <bool W4, bool GROUPED, int MT, int W>
int gemv32_one(const LinearArgs& a, int grid, hipStream_t s) {
  constexpr int D = 3;
  const int64_t nrt = (a.N + kTileN - 1) / kTileN;
  const int64_t rmax = (nrt + grid - 1) / grid, rmin = nrt / grid;
  const int64_t nkt = a.K / kTileK;
  // a wave's run stays within two row tiles (R <= W) and is never empty (T >= W)
  if (rmax > W || rmin * nkt < W) return LSQ_E_LAYOUT;
  const G32Lds L = g32_lds(MT, a.K, rmax * kTileN, GROUPED ? a.ngroups : 1, W);
  if (L.total > gemv32_max_lds()) return LSQ_E_LAYOUT;
  auto kern = gemv32_kernel<W4, GROUPED, MT, W, D>;
  if (L.total > 64 * 1024) {
    static std::atomic<int> attr_set{0};
    if (!attr_set.load(std::memory_order_acquire)) {
      const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, gemv32_max_lds());
      if (e != hipSuccess) return static_cast<int>(e);
      attr_set.store(1, std::memory_order_release);
    }
  }
  kern<<<dim3(static_cast<unsigned>(grid)), dim3(64 * W), static_cast<size_t>(L.total), s>>>(a);
  return static_cast<int>(hipGetLastError());
}

template <bool W4, bool GROUPED, int MT>
int gemv32_mt(const LinearArgs& a, hipStream_t s) {
  // at most 256 workgroups of whole row tiles (one per CU), 16 waves when every wave gets
  // 16+ units, else 8 or 4
  const int64_t nrt = (a.N + kTileN - 1) / kTileN;
  const int64_t nkt = a.K / kTileK;
  const int64_t rpw = (nrt + 255) / 256;
  const int64_t grid = (nrt + rpw - 1) / rpw;
  const int64_t units = (nrt / grid) * nkt;  // of the smallest workgroup
  if (units >= 16 * 2) return gemv32_one<W4, GROUPED, MT, 16>(a, static_cast<int>(grid), s);
  if (units >= 8) return gemv32_one<W4, GROUPED, MT, 8>(a, static_cast<int>(grid), s);
  return gemv32_one<W4, GROUPED, MT, 4>(a, static_cast<int>(grid), s);
}

// MT token rows per lane (the rows from M up to MT are computed and dropped)
template <bool W4, bool GROUPED>
int gemv32_kind(const LinearArgs& a, hipStream_t s) {
  if (a.M == 1) return gemv32_mt<W4, GROUPED, 1>(a, s);
  if (a.M == 2) return gemv32_mt<W4, GROUPED, 2>(a, s);
  if (a.M <= 4) return gemv32_mt<W4, GROUPED, 4>(a, s);
  return gemv32_mt<W4, GROUPED, 8>(a, s);
}

// LSQ_GEMV32=0 turns this kernel off (the generic kernel then takes fp32 activations).
bool gemv32_enabled() {
  const char* e = std::getenv("LSQ_GEMV32");
  return !(e && e[0] == '0');
}

}  // namespace

int launch_gemv32(int kind, const LinearArgs& a, hipStream_t s) {
  if (!gemv32_enabled() || a.act != LSQ_ACT_NONE || a.xscale) return LSQ_E_LAYOUT;
  if (kind != kW4Tiled && kind != kW8Tiled) return LSQ_E_LAYOUT;
  if (a.M < 1 || a.M > 8 || a.K % kTileK != 0 || a.K < kTileK || a.N < 1) return LSQ_E_LAYOUT;
  // 16-byte activation loads
  if ((reinterpret_cast<uintptr_t>(a.x) & 15) || a.ldx % 4) return LSQ_E_LAYOUT;
  if ((reinterpret_cast<uintptr_t>(a.w) & 15)) return LSQ_E_LAYOUT;
  const bool w4 = kind == kW4Tiled;
  const bool grouped = w4 && a.group < a.K;
  if (grouped && (a.group % kTileK != 0 || ((a.group / kTileK) & (a.group / kTileK - 1)) != 0)) return LSQ_E_LAYOUT;
  // 32-bit buffer range of one workgroup's weights (<= 16 row tiles of K)
  if (int64_t(16) * (a.K / kTileK) * kTileBytes8 >= (int64_t(1) << 31)) return LSQ_E_LAYOUT;
  if (!w4) return gemv32_kind<false, false>(a, s);
  return grouped ? gemv32_kind<true, true>(a, s) : gemv32_kind<true, false>(a, s);
}

}  // namespace lsq
