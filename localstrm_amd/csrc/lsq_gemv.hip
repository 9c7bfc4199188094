// Decode GEMV for 1..16 tokens on the tiled INT4 / INT8 layouts (gfx950).
//
// GPU form of QuantizedLinear.forward (src/kernels/quantization.py:129-141) for the decode
// step: y = x W^T + b with the weights streamed from HBM once, unpacked in registers into
// the B operand of v_mfma_f32_16x16x32_{bf16,f16}, never materialized.
//
// Work split. The weight matrix is a sequence of (16-row tile, 128-column k tile) units,
// 1 KB (INT4) or 2 KB (INT8) each, stored row tile after row tile (lsq_internal.h). The
// grid's G workgroups take contiguous, balanced ranges of whole row tiles (sizes differing
// by at most one), so no output row is shared between workgroups and no
// cross-workgroup merge is needed (measured: merging through device-scope fences costs
// 7-25 us per launch on MI355X, through write-through stores and a counter 1.3 us). Inside
// a workgroup the R x nkt units are cut into W equal contiguous runs, one per wave; a run
// covers at most two row tiles (R <= W), so each wave keeps two accumulators. At the end
// each wave puts its (one or two) partial sums into LDS slots of its own and counts itself
// in per row tile; the last wave to arrive adds the slots in wave order, so results do not
// depend on timing, and no wave waits at a workgroup barrier for the slowest one.
//
// Streaming. Each wave keeps a ring of D units in flight (non-temporal 16-byte buffer
// loads, 1 KB contiguous per wavefront load; refills past the run are out-of-range loads
// that move no data, so the ring never needs a branch, which would make the compiler drain
// it). Measured on MI355X: a plain read of 35 MB is fastest with ~8 MB in flight over the
// whole chip (e.g. 4096 waves x 2 KB); the launcher picks G, W and D accordingly.
//
// Prologue (once per workgroup, loads issued before the weight ring so that waiting for
// them leaves the weights in flight): activations x[0:M] into LDS (row stride K + 8, plus
// one all-zero row read by the lanes of token rows >= M), per (k tile, token) sums of x
// for the INT4 nibble bias, the workgroup's scales and bias as fp32 rounded to T.
//
// Arithmetic (same as the LDS-staged decode kernel): INT4 nibble u OR-ed into the mantissa
// of 128.0 (bf16) / 1024.0 (fp16) is exactly 128 + u, the offset 136 / 1032 removed per k
// tile through the activation sums as s * (acc - off * sum(x)); INT8 bytes converted
// exactly through fp32. Every product is exact in the fp32 accumulator; group scales are
// applied per k tile in fp32, per-channel scales once at the end, then the bias rounded to
// T, then one rounding to T.

#include "lsq_common.h"
#include "lsq_internal.h"
#include "lsq_decode.h"
#include "lsq_mfma16.h"

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstdlib>

namespace lsq {

template <int DT>
int launch_split_merge(const float* part, int S, int64_t M, int64_t N, const void* bias, int bias_dt,
                       void* y, int64_t ldy, hipStream_t s);

namespace {

// LDS layout (byte offsets), shared by kernel and host: partial sums `red` (two slots per
// wave of NE x 64 floats), one arrival counter per row tile, the staged activations
// (M + 1 rows), per-(k tile, token) activation sums, the workgroup's scales and bias as
// 16-bit values of the activation type T (round_T of the stored values, which is what the
// reference multiplies by; a copy of the stored bits when they already are T).
struct GemvLds {
  int64_t red, cnt, xs, xsum, ss, sb, total;
};

__host__ __device__ inline GemvLds gemv_lds(int64_t M, int64_t K, int64_t rows, int64_t ngs, int W, int NE) {
  GemvLds l;
  const int64_t nkt = K / kTileK;
  l.red = 0;
  l.cnt = int64_t(W) * 2 * NE * 64 * 4;
  l.xs = align16(l.cnt + int64_t(W) * 4);
  l.xsum = l.xs + align16((M + 1) * (K + 8) * 2);
  l.ss = l.xsum + align16(nkt * 16 * 4);
  l.sb = l.ss + align16(rows * ngs * 2);
  l.total = l.sb + align16(rows * 2);
  return l;
}

// Scale groups per row the LDS layout holds: all ngs, or with S > 1 slices of at most
// kst k tiles the most one slice can touch (it may straddle a group boundary).
__host__ __device__ inline int gemv_lds_groups(int ngs, int S, int kst, int gtiles, bool grouped) {
  if (S <= 1 || !grouped) return ngs;
  const int g = (kst + gtiles - 1) / gtiles + 1;
  return g < ngs ? g : ngs;
}

// Sum of a float over each row of 16 lanes, in every lane of the row (DPP).
__device__ __forceinline__ float row16_add(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
  return v;
}

constexpr int kGemvSB = 4;  // scale dwords in flight per thread while staging

// Activation chunks (16 B) each thread loads per staging batch: enough for MT tokens at
// K = 4096 in one batch, at most 4 (8 for 16 tokens, so that 16 tokens at K = 3584, 115
// KB, stage in one batch of 16 waves and the weight ring is issued alongside).
__host__ __device__ constexpr int gemv_xb(int mt, int nt) {
  return mt * 512 / nt < 1 ? 1 : (mt * 512 / nt > (mt == 16 ? 8 : 4) ? (mt == 16 ? 8 : 4) : mt * 512 / nt);
}

// Units of the wave run [t_lo, t_hi) of wave `w` among W over T units.
__device__ __forceinline__ int run_lo(int w, int T, int W) {
  return w * T / W;  // T <= 16 row tiles x 2^14 k tiles: no overflow
}

template <int DT, bool W4, bool GROUPED, int MT, int W, int D, bool SPLIT>
__global__ void __launch_bounds__(64 * W) gemv_kernel(LinearArgs p) {
  constexpr int NT = 64 * W;
  constexpr int kTileB = W4 ? kTileBytes : kTileBytes8;
  constexpr int LPT = W4 ? 1 : 2;       // 16-byte weight loads per lane per unit
  constexpr int NE = MT < 4 ? MT : 4;   // accumulator elements per lane that can hold tokens
  constexpr int XB = gemv_xb(MT, NT);
  extern __shared__ __align__(16) unsigned char smem[];
  using S = typename Act<DT>::storage;

  const int M = static_cast<int>(p.M), N = static_cast<int>(p.N);
  // K slices (split-K: workgroup b takes slice b % NS of row-tile range b / NS; NS = 1
  // otherwise). `nkt` counts the k tiles of this workgroup's slice, which start at k tile
  // `kt_s0` of the layer's `nkt_all`.
  const int NS = SPLIT ? p.ksplit : 1;  // (a constant 1 in the unsplit instances)
  const int nkt_all = static_cast<int>(p.K / kTileK);
  const int sl = NS > 1 ? static_cast<int>(blockIdx.x) % NS : 0;
  const int kt_s0 = sl * nkt_all / NS;
  const int nkt = (sl + 1) * nkt_all / NS - kt_s0;
  const int K = nkt * kTileK;  // columns of the slice
  const int kmax = ((nkt_all + NS - 1) / NS) * kTileK;  // the widest slice (LDS layout)
  const int nrt = (N + kTileN - 1) / kTileN;
  const int ngs = GROUPED ? static_cast<int>(p.ngroups) : 1;
  const int gtiles = static_cast<int>(p.group / kTileK);
  const int gshift = __builtin_ctz(static_cast<uint32_t>(gtiles));  // k tiles per group: a power of two
  // scale groups staged per row: all of them, or with a split those of the slice
  const int gs0 = NS > 1 && GROUPED ? kt_s0 >> gshift : 0;
  const int ngs_s = NS > 1 && GROUPED ? ((kt_s0 + nkt - 1) >> gshift) - gs0 + 1 : ngs;
  const int ngs_lds = gemv_lds_groups(ngs, NS, kmax / kTileK, gtiles, GROUPED);
  const int ldxb = (kmax + 8) * 2;  // LDS bytes per staged activation row

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, q = lane >> 4;
  // Row tiles: the first `rem` workgroups take base + 1, the others base (one 32-bit
  // division; the code before the first load is on every wave's critical path).
  const int G = gridDim.x / NS;
  const int b = blockIdx.x / NS;
  const int base = nrt / G;
  const int rem = nrt - base * G;
  const int rt_lo = b * base + min(b, rem);
  const int R = base + (b < rem ? 1 : 0);  // row tiles of this workgroup (1 <= R <= W)
  const int rmax = base + (rem > 0 ? 1 : 0);  // the largest R of the grid (LDS sizing)
  const int T = R * nkt;                   // units of this workgroup
  const int t_lo = run_lo(wid, T, W), t_hi = run_lo(wid + 1, T, W);
  const int row0 = rt_lo * kTileN;
  const int rows_valid = min(R * kTileN, N - row0);

  const GemvLds L = gemv_lds(M, kmax, int64_t(rmax) * kTileN, ngs_lds, W, NE);
  unsigned char* xs = smem + L.xs;
  float* red = reinterpret_cast<float*>(smem + L.red);
  int* cnt = reinterpret_cast<int*>(smem + L.cnt);
  float* xsum = reinterpret_cast<float*>(smem + L.xsum);
  uint16_t* ss = reinterpret_cast<uint16_t*>(smem + L.ss);
  uint16_t* sb = reinterpret_cast<uint16_t*>(smem + L.sb);

  // ---- descriptors over what this workgroup reads
  const int es_s = p.scale_dt == LSQ_F32 ? 4 : 2;
  const int es_b = p.bias_dt == LSQ_F32 ? 4 : 2;
  const rsrc_t rx = make_rsrc(static_cast<const uint16_t*>(p.x) + static_cast<int64_t>(kt_s0) * kTileK,
                              static_cast<uint32_t>(((M - 1) * p.ldx + K) * 2));
  const rsrc_t rw = make_rsrc(p.w + static_cast<int64_t>(rt_lo) * nkt_all * kTileB,
                              static_cast<uint32_t>(R * nkt_all * kTileB));
  const int nsc = rows_valid * ngs;
  const int nsd = (nsc * es_s + 3) / 4;
  const int nse = rows_valid * ngs_s;  // scale elements staged (split: one per load)
  // The dword holding the last 16-bit element may extend 2 bytes past the array; an
  // aligned dword never crosses a page, so reading it is always safe.
  const rsrc_t rs = make_rsrc(static_cast<const uint8_t*>(p.scale) + static_cast<int64_t>(row0) * ngs * es_s,
                              static_cast<uint32_t>(nsd * 4));
  const int nbd = p.bias ? (rows_valid * es_b + 3) / 4 : 0;
  const rsrc_t rb = make_rsrc(p.bias ? static_cast<const uint8_t*>(p.bias) + static_cast<int64_t>(row0) * es_b
                                     : static_cast<const uint8_t*>(p.scale),
                              static_cast<uint32_t>(nbd * 4));

  // ---- prologue. When the activations, scales and bias fit one batch of loads per thread
  // (the decode shapes), every load of the batch is issued unconditionally (out-of-range
  // offsets where a thread has nothing to load) and before the weight ring, so that the
  // compiler's waits for them are exact and leave the weights in flight (a load that may
  // be skipped makes it wait conservatively, draining the ring). Otherwise everything is
  // staged first, then the ring is issued.
  const int K8 = K / 8;  // 16-byte chunks per activation row
  const int nch = M * K8;
  // c / K8 as a multiply-high: exact while c * K8 < 2^32 (c < 2^17 chunks, K8 < 2^15)
  const uint32_t k8_magic = MT == 1 ? 0u : 0xFFFFFFFFu / static_cast<uint32_t>(K8) + 1u;
  auto row_of = [&](int c) {
    return MT == 1 ? 0 : static_cast<int>(__umulhi(static_cast<uint32_t>(c), k8_magic));
  };
  auto x_off = [&](int c) -> uint32_t {
    const int m = row_of(c);
    return c < nch ? static_cast<uint32_t>((m * p.ldx + (c - m * K8) * 8) * 2) : kOOB;
  };
  // Unit i of this wave's run: k tile kt0 + i of the run's first row tile, or (from
  // kt0 + i = nkt on) of the next one; in memory a row tile holds all nkt_all k tiles.
  const int rt_first = t_lo / nkt;
  const int kt0 = t_lo - rt_first * nkt;
  const int u_base = (rt_first * nkt_all + kt_s0 + kt0) * kTileB + lane * 16;
  const int u_skip = (nkt_all - nkt) * kTileB;  // into the next row tile (0 without split)
  u32x4 wbuf[D][LPT];
  auto issue = [&](u32x4 (&wv)[LPT], int i) {
    const bool real = t_lo + i < t_hi;
    const uint32_t off = static_cast<uint32_t>(u_base + i * kTileB + (kt0 + i >= nkt ? u_skip : 0));
    wv[0] = bload16<kNT>(rw, real ? off : kOOB);
    if (LPT == 2) wv[LPT - 1] = bload16<kNT>(rw, real ? off + kTileB / 2 : kOOB);
  };
  auto put_x = [&](const u32x4 (&v)[XB], int c0) {
#pragma unroll
    for (int u = 0; u < XB; ++u) {
      if (c0 + u * NT >= nch) break;  // uniform
      const int c = c0 + u * NT + tid;
      const int m = row_of(c);
      const int c8 = c - m * K8;
      float sum = 0.f;
      if (c < nch) {
        *reinterpret_cast<u32x4*>(xs + m * ldxb + c8 * 16) = v[u];
        if constexpr (W4) {
#pragma unroll
          for (int e = 0; e < 4; ++e) sum += Mma<DT>::lo(v[u][e]) + Mma<DT>::hi(v[u][e]);
        }
      }
      if constexpr (W4) {
        // lanes 16a..16a+15 hold the 16 chunks of one (token, k tile): all valid or none
        sum = row16_add(sum);
        if (c < nch && (lane & 15) == 0) xsum[(c8 >> 4) * 16 + m] = sum;
      }
    }
  };
  auto load_x = [&](u32x4 (&v)[XB], int c0) {
#pragma unroll
    for (int u = 0; u < XB; ++u) v[u] = bload16<0>(rx, x_off(c0 + u * NT + tid));
  };
  // Split: element e of the staged scales is group gs0 + e % ngs_s of row e / ngs_s.
  auto s_byte = [&](int e) {
    const int row = e / ngs_s;
    return static_cast<uint32_t>((row * ngs + gs0 + (e - row * ngs_s)) * es_s);
  };
  auto load_s = [&](uint32_t (&v)[kGemvSB], int t0) {
#pragma unroll
    for (int u = 0; u < kGemvSB; ++u) {
      const int t = t0 + u * NT + tid;
      if (NS > 1)
        v[u] = bload4(rs, t < nse ? s_byte(t) & ~3u : kOOB);
      else
        v[u] = bload4(rs, t < nsd ? t * 4 : kOOB);
    }
  };
  auto put_scales = [&](const uint32_t (&v)[kGemvSB], int t0) {
    if (NS > 1) {  // uniform
#pragma unroll
      for (int u = 0; u < kGemvSB; ++u) {
        const int t = t0 + u * NT + tid;
        if (t < nse) ss[t] = Act<DT>::from_f32(dword_elem(v[u], (s_byte(t) >> 1) & 1, p.scale_dt));
      }
      return;
    }
    if (p.scale_dt == DT) {  // uniform: already T, copy the stored bits
#pragma unroll
      for (int u = 0; u < kGemvSB; ++u) {
        const int t = t0 + u * NT + tid;
        if (t < nsd) reinterpret_cast<uint32_t*>(ss)[t] = v[u];
      }
      return;
    }
#pragma unroll
    for (int u = 0; u < kGemvSB; ++u) {
      const int t = t0 + u * NT + tid;
      if (p.scale_dt == LSQ_F32) {
        if (t < nsc) ss[t] = Act<DT>::from_f32(dword_elem(v[u], 0, LSQ_F32));
      } else {
        if (2 * t < nsc) ss[2 * t] = Act<DT>::from_f32(dword_elem(v[u], 0, p.scale_dt));
        if (2 * t + 1 < nsc) ss[2 * t + 1] = Act<DT>::from_f32(dword_elem(v[u], 1, p.scale_dt));
      }
    }
  };
  auto put_bias = [&](uint32_t bv) {
    if (p.bias && tid < nbd) {
      if (es_b == 4) {
        sb[tid] = Act<DT>::from_f32(dword_elem(bv, 0, LSQ_F32));
      } else {
        if (2 * tid < rows_valid) sb[2 * tid] = Act<DT>::from_f32(dword_elem(bv, 0, p.bias_dt));
        if (2 * tid + 1 < rows_valid) sb[2 * tid + 1] = Act<DT>::from_f32(dword_elem(bv, 1, p.bias_dt));
      }
    }
  };
  // (bias: rows * 4 <= 16 W * 4 bytes, one dword per thread at most)
  const int nsl = NS > 1 ? nse : nsd;  // scale loads
  if (nch <= NT * XB && nsl <= NT * kGemvSB) {  // uniform
    u32x4 xv[XB];
    uint32_t sv[kGemvSB];
    load_x(xv, 0);
    load_s(sv, 0);
    const uint32_t bv = bload4(rb, tid < nbd ? tid * 4 : kOOB);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < D; ++s) issue(wbuf[s], s);
    put_x(xv, 0);
    put_scales(sv, 0);
    put_bias(bv);
  } else {
    for (int c0 = 0; c0 < nch; c0 += NT * XB) {
      u32x4 xv[XB];
      load_x(xv, c0);
      put_x(xv, c0);
    }
    for (int t0 = 0; t0 < nsl; t0 += NT * kGemvSB) {
      uint32_t sv[kGemvSB];
      load_s(sv, t0);
      put_scales(sv, t0);
    }
    put_bias(bload4(rb, tid < nbd ? tid * 4 : kOOB));
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < D; ++s) issue(wbuf[s], s);
  }
  // row M: zeros; sums of token rows >= M: zero
  for (int c = tid; c < K8; c += NT) *reinterpret_cast<u32x4*>(xs + M * ldxb + c * 16) = u32x4{0u, 0u, 0u, 0u};
  if constexpr (W4) {
    for (int i = tid; i < nkt * 16; i += NT)
      if ((i & 15) >= M) xsum[i] = 0.f;
  }
  if (tid < R) cnt[tid] = 0;
  lds_barrier();

  // ---- main loop over this wave's run of units. Unit i of the run is k tile kt0 + i of
  // the run's first row tile, or (once kt0 + i reaches nkt: `second`) k tile kt0 + i - nkt
  // of the next one; each unit's sum goes into acc_a or acc_b accordingly (uniform).
  f32x4 acc_a = {0.f, 0.f, 0.f, 0.f}, acc_b = {0.f, 0.f, 0.f, 0.f};
  const int n_my = t_hi - t_lo;
  const unsigned char* xrow = xs + min(r, M) * ldxb + 32 * q * 2;
  // this lane's scale row in the run's first and second row tile
  const uint16_t* srow_a = ss + (rt_first * kTileN + r) * ngs_s;
  const uint16_t* srow_b = srow_a + kTileN * ngs_s;
  uint32_t nib_mask = 0, magic = 0;
  if constexpr (W4) {
    // constants in registers, so that the unpack selects v_and_or_b32
    asm volatile("v_mov_b32 %0, 0x000f000f" : "=v"(nib_mask));
    asm volatile("v_mov_b32 %0, %1" : "=v"(magic) : "i"(Mma<DT>::kMagic));
  }
  for (int i0 = 0; i0 < n_my; i0 += D) {
#pragma unroll
    for (int s = 0; s < D; ++s) {
      const int i = i0 + s;
      const bool live = i < n_my;  // uniform
      const int kk = kt0 + i;
      const bool second = kk >= nkt;  // uniform
      const int kt = second ? kk - nkt : kk;
      u32x4 a[4], bb[4];
      float xo[NE], scg = 0.f;
      if (live) {
#pragma unroll
        for (int d = 0; d < 4; ++d) a[d] = *reinterpret_cast<const u32x4*>(xrow + (kt * kTileK + 8 * d) * 2);
        if constexpr (W4 && GROUPED) {
          if constexpr (NE == 1) {
            xo[0] = xsum[kt * 16 + 4 * q];
          } else {
            const f32x4 x4 = *reinterpret_cast<const f32x4*>(xsum + kt * 16 + 4 * q);
#pragma unroll
            for (int e = 0; e < NE; ++e) xo[e] = x4[e];
          }
          scg = Act<DT>::to_f32((second ? srow_b : srow_a)[((kt_s0 + kt) >> gshift) - gs0]);
        }
#pragma unroll
        for (int d = 0; d < 4; ++d)
          bb[d] = W4 ? unpack_w4(wbuf[s][0][d], nib_mask, magic)
                     : convert_w8<DT>(wbuf[s][d >> 1][2 * (d & 1)], wbuf[s][d >> 1][2 * (d & 1) + 1]);
      }
      issue(wbuf[s], i + D);
      if (live) {
        f32x4 dacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int d = 0; d < 4; ++d) dacc = Mma<DT>::mma(a[d], bb[d], dacc);
#pragma unroll
        for (int e = 0; e < NE; ++e) {
          float v = dacc[e];
          if constexpr (W4 && GROUPED) v = scg * fmaf(-Mma<DT>::kOff4, xo[e], v);
          // (selects, not a branch: the compiler would copy whole accumulators around one)
          acc_a[e] = second ? acc_a[e] : acc_a[e] + v;
          acc_b[e] = second ? acc_b[e] + v : acc_b[e];
        }
      }
    }
  }
  // ---- epilogue without a workgroup barrier. Every wave has a non-empty run (the launcher
  // ensures T >= W). The waves contributing to row tile j are wa(j)..wb(j), those holding
  // its first and last unit (the wave of unit u is ((u + 1) W - 1) / T); wave w's first row
  // tile is w R / W. Each wave stores its partial sum of a row tile into its own LDS slot
  // and counts itself in; the last to arrive adds the slots in wave order (fixed, so the
  // result does not depend on arrival order) and writes the outputs.
  auto first_wave = [&](int j) { return (j * nkt * W + W - 1) / T; };
  auto last_wave = [&](int j) { return ((j + 1) * nkt * W - 1) / T; };
  S* y = static_cast<S*>(p.y);
  auto finish = [&](int j) {
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    const int wb = last_wave(j);
    for (int w2 = first_wave(j); w2 <= wb; ++w2) {
      const int slot = (w2 * R) / W == j ? 0 : 1;
#pragma unroll
      for (int e = 0; e < NE; ++e) v[e] += red[((w2 * 2 + slot) * NE + e) * 64 + lane];
    }
    const int rl = j * kTileN + r;
    const int n = row0 + rl;
    const float sc = GROUPED ? 1.f : Act<DT>::to_f32(ss[rl]);
    const float bias = p.bias ? Act<DT>::to_f32(sb[rl]) : 0.f;
#pragma unroll
    for (int e = 0; e < NE; ++e) {
      const int m = 4 * q + e;
      float val = v[e];
      if constexpr (W4 && !GROUPED) {
        float tot = 0.f;
        for (int k2 = 0; k2 < nkt; ++k2) tot += xsum[k2 * 16 + m];
        val = fmaf(-Mma<DT>::kOff4, tot, val);
      }
      if (m < M && n < N) {
        if (NS > 1)  // this slice's scaled sum; the bias and the rounding come in the merge
          p.part[(static_cast<int64_t>(sl) * M + m) * N + n] = GROUPED ? val : val * sc;
        else
          y[static_cast<int64_t>(m) * p.ldy + n] = Act<DT>::from_f32(opaque(GROUPED ? val + bias : fmaf(val, sc, bias)));
      }
    }
  };
  auto publish = [&](int j, int slot, const f32x4& part) {
#pragma unroll
    for (int e = 0; e < NE; ++e) red[((wid * 2 + slot) * NE + e) * 64 + lane] = part[e];
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the partial is in LDS before the count
    int old = 0;
    if (lane == 0) old = atomicAdd(&cnt[j], 1);
    old = __builtin_amdgcn_readfirstlane(old);
    if (old == last_wave(j) - first_wave(j)) finish(j);
  };
  publish(rt_first, 0, acc_a);
  if (kt0 + n_my > nkt) publish(rt_first + 1, 1, acc_b);
}

// ------------------------------------------------------------------ launch

struct GemvCfg {
  int rpw, w, d;  // row tiles per workgroup (target), waves per workgroup, ring depth
};

// LSQ_GEMV_CFG="rpw,w,d" overrides the heuristic (for tuning sweeps); LSQ_GEMV=0 turns
// this kernel off (the LDS-staged decode kernel then takes these shapes). Both are read
// at every launch (a getenv, far below the cost of the call), so a process can switch.
bool gemv_enabled() {
  const char* e = std::getenv("LSQ_GEMV");
  return !(e && e[0] == '0');
}

bool env_cfg(GemvCfg* out) {
  const char* e = std::getenv("LSQ_GEMV_CFG");
  GemvCfg c{};
  if (e && std::sscanf(e, "%d,%d,%d", &c.rpw, &c.w, &c.d) == 3) {
    *out = c;
    return true;
  }
  return false;
}

// One workgroup per CU at most, row tiles balanced to +-1 over the grid (18944 x 3584:
// 237 workgroups of 4-5 row tiles), 16 waves of ~9 units each with a ring of 3: measured
// on MI355X this keeps ~8-11 MB of weights in flight, the bare-read optimum; fewer waves
// when the layer has few k tiles, so that no wave's run is empty.
GemvCfg pick_gemv(int64_t nrt, int64_t nkt) {
  GemvCfg c;
  if (env_cfg(&c)) return c;
  // Layers with fewer than 1024 row tiles stay on the LDS-staged decode kernel, measured
  // faster there (3584 x 18944: 10.7 vs 11.0-11.4 us; 4864 x 896: 4.0 vs 4.4 us).
  if (nrt < 1024) return GemvCfg{0, 0, 0};
  const int rpw = static_cast<int>((nrt + 255) / 256);
  const int64_t units = (nrt / ((nrt + rpw - 1) / rpw)) * nkt;  // units of the smallest workgroup
  const int w = units >= 16 ? 16 : (units >= 8 ? 8 : 4);
  return GemvCfg{rpw, w, 3};
}

// Split-K plan for layers of at most 512 row tiles whose activations are too large for
// the LDS-staged decode kernel (more than 96 KB: 4+ tokens at K = 18944, 16 at K = 4864),
// which the chunked decode kernel serves otherwise (down projections: 3584 x 18944,
// 4096 x 14336, 896 x 4864). K is cut into S slices of at least 4 k tiles, with x of one
// slice no larger than one staging batch of 16 waves (16 KB for one token, 32 KB up to 4,
// 64 KB up to 16: then its loads are issued together with the weight ring), and about one
// workgroup per CU: `ranges` balanced row-tile ranges of at most 16 row tiles, times S.
// Measured (us, INT4 g128, unsplit -> split): 3584 x 18944 M=4 25.6 -> 15.4, M=16
// 26.4 -> 18.1 (S = 5..20: 18.1-27.3), 4096 x 14336 M=16 20.9 -> 16.4; smaller x stays
// unsplit (3584 x 18944 M=2: 11.9 unsplit, 14.8-15.2 split), as do wider layers
// (14336 x 4096 M=16: 13.9 unsplit, 15.2 split). S = 1: no split. LSQ_SPLITK=0 turns the
// split off, LSQ_SPLITK=n forces n slices (read at every call).
struct GemvSplit {
  int64_t S, ranges, bytes;
};

GemvSplit gemv_split_plan(int64_t M, int64_t N, int64_t K) {
  const int64_t nrt = (N + kTileN - 1) / kTileN;
  const int64_t nkt = K / kTileK;
  GemvSplit sp{1, 0, 0};
  if (M < 1 || M > 16 || K % kTileK != 0 || nrt >= 1024 || nkt < 8) return sp;
  const char* e = std::getenv("LSQ_SPLITK");
  if (e && e[0] == '0') return sp;
  const int64_t forced = e ? std::atoi(e) : 0;  // LSQ_SPLITK=n >= 2: n slices (sweeps)
  if (forced < 2 && (nrt > 512 || M * K * 2 <= 96 * 1024)) return sp;
  const int64_t rmin_ranges = (nrt + 15) / 16;
  const int64_t batch = int64_t(16) * 1024 * std::min(4, gemv_xb(M == 1 ? 1 : (M <= 4 ? 4 : 16), 1024));
  int64_t S = (M * K * 2 + batch - 1) / batch;
  if (S < 1) S = 1;
  for (; S <= nkt / 4; ++S) {
    const int64_t ranges = std::min(nrt, std::max(rmin_ranges, int64_t(256) / S));
    if (ranges * S >= 192) break;
  }
  if (forced >= 2) S = forced;
  if (S < 2 || S > nkt / 4 || S > 16) return sp;  // (the merge adds at most 16 slices)
  sp.S = S;
  sp.ranges = std::min(nrt, std::max(rmin_ranges, int64_t(256) / S));
  sp.bytes = S * M * N * 4;
  return sp;
}

int g_gemv_max_lds = -1;

int gemv_max_lds() {
  int v = g_gemv_max_lds;
  if (v < 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
      v = 64 * 1024;
    g_gemv_max_lds = v;
  }
  return v;
}

template <int DT, bool W4, bool GROUPED, int MT, int W, int D, bool SPLIT>
int gemv_one(const LinearArgs& a, int grid, hipStream_t s) {
  // grid = row-tile ranges x a.ksplit K slices
  const int S = a.ksplit;
  const int64_t nrt = (a.N + kTileN - 1) / kTileN;
  const int64_t ranges = grid / S;
  const int64_t rmax = (nrt + ranges - 1) / ranges;
  const int64_t rmin = nrt / ranges;
  const int64_t nkt = a.K / kTileK;
  const int64_t kst_min = nkt / S, kst_max = (nkt + S - 1) / S;  // k tiles per slice
  // a wave's run stays within two row tiles (R <= W) and is never empty (T >= W)
  if (rmax > W || rmin * kst_min < W) return LSQ_E_LAYOUT;
  constexpr int NE = MT < 4 ? MT : 4;
  const int ngs = GROUPED ? static_cast<int>(a.ngroups) : 1;
  const GemvLds L = gemv_lds(a.M, kst_max * kTileK, rmax * kTileN,
                             gemv_lds_groups(ngs, S, static_cast<int>(kst_max), static_cast<int>(a.group / kTileK), GROUPED),
                             W, NE);
  if (L.total > gemv_max_lds()) return LSQ_E_LAYOUT;
  auto kern = gemv_kernel<DT, W4, GROUPED, MT, W, D, SPLIT>;
  if (L.total > 64 * 1024) {
    static std::atomic<int> attr_set{0};
    if (!attr_set.load(std::memory_order_acquire)) {
      const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, gemv_max_lds());
      if (e != hipSuccess) return static_cast<int>(e);
      attr_set.store(1, std::memory_order_release);
    }
  }
  kern<<<dim3(static_cast<unsigned>(grid)), dim3(64 * W), static_cast<size_t>(L.total), s>>>(a);
  return static_cast<int>(hipGetLastError());
}

template <int DT, bool W4, bool GROUPED, int MT, bool SPLIT>
int gemv_mt(const LinearArgs& a, const GemvCfg& c, int grid, hipStream_t s) {
#define LSQ_GEMV_TRY(W_, D_) \
  if (c.w == W_ && c.d == D_) return gemv_one<DT, W4, GROUPED, MT, W_, D_, SPLIT>(a, grid, s);
  LSQ_GEMV_TRY(16, 3)
  LSQ_GEMV_TRY(8, 3)
  LSQ_GEMV_TRY(4, 3)
  if constexpr (!SPLIT) {  // (the split launcher uses ring depth 3 only)
    LSQ_GEMV_TRY(16, 2)
    LSQ_GEMV_TRY(8, 2)
    LSQ_GEMV_TRY(4, 2)
  }
#undef LSQ_GEMV_TRY
  return LSQ_E_LAYOUT;
}

template <int DT, bool W4, bool GROUPED, bool SPLIT>
int gemv_grid(const LinearArgs& a, const GemvCfg& c, int grid, hipStream_t s) {
  if (a.M == 1) return gemv_mt<DT, W4, GROUPED, 1, SPLIT>(a, c, grid, s);
  if (a.M <= 4) return gemv_mt<DT, W4, GROUPED, 4, SPLIT>(a, c, grid, s);
  return gemv_mt<DT, W4, GROUPED, 16, SPLIT>(a, c, grid, s);
}

// y[m, n] = round_T(sum over slices s = 0.. S-1, in that order, of part[s][m][n] +
// round_T(bias[n])): the merge of the split-K GEMV. Each thread takes 4 consecutive
// outputs (16-byte loads; N % 4 == 0, else one output per thread) and issues every slice's
// load before the first add, so the kernel costs about one memory round trip.
template <int DT, int V>
__global__ void __launch_bounds__(256) gemv_merge_kernel(const float* __restrict__ part, int S, int M, int N,
                                                         const void* bias, int bias_dt,
                                                         typename Act<DT>::storage* __restrict__ y, int64_t ldy) {
  constexpr int kMaxS = 16;
  const int64_t MN = int64_t(M) * N;
  const int64_t i = (int64_t(blockIdx.x) * 256 + threadIdx.x) * V;  // first output
  if (i >= MN) return;
  const int m = static_cast<int>(i / N), n = static_cast<int>(i - int64_t(m) * N);
  float v[kMaxS][V];
#pragma unroll
  for (int sl = 0; sl < kMaxS; ++sl) {
    if (sl < S) {
      if constexpr (V == 4) {
        const float4 t = *reinterpret_cast<const float4*>(part + sl * MN + i);
        v[sl][0] = t.x; v[sl][1] = t.y; v[sl][2] = t.z; v[sl][3] = t.w;
      } else {
        v[sl][0] = part[sl * MN + i];
      }
    }
  }
  const uint16_t* b16 = static_cast<const uint16_t*>(bias);
#pragma unroll
  for (int e = 0; e < V; ++e) {
    float acc = v[0][e];
#pragma unroll
    for (int sl = 1; sl < kMaxS; ++sl)
      if (sl < S) acc += v[sl][e];
    if (bias) {
      const int nn = n + e;
      const float bv = bias_dt == LSQ_F32 ? static_cast<const float*>(bias)[nn]
                                          : (bias_dt == LSQ_BF16 ? bf16_to_f32(b16[nn]) : f16_to_f32(b16[nn]));
      acc = opaque(acc + Act<DT>::round(bv));
    }
    y[static_cast<int64_t>(m) * ldy + n + e] = Act<DT>::from_f32(acc);
  }
}

template <int DT, bool W4, bool GROUPED>
int gemv_kind(const LinearArgs& a, hipStream_t s) {
  const int64_t nrt = (a.N + kTileN - 1) / kTileN;
  const int64_t nkt = a.K / kTileK;
  const GemvCfg c = pick_gemv(nrt, nkt);
  if (c.rpw >= 1) {
    const int64_t rpw = c.rpw;
    const int64_t grid = (nrt + rpw - 1) / rpw;
    if (grid < 1 || grid > 65535) return LSQ_E_LAYOUT;
    return gemv_grid<DT, W4, GROUPED, false>(a, c, static_cast<int>(grid), s);
  }
  // Fewer than 1024 row tiles: the split-K form when it applies and a workspace is given.
  const GemvSplit sp = gemv_split_plan(a.M, a.N, a.K);
  if (sp.S < 2 || !a.part || a.part_bytes < sp.bytes) return LSQ_E_LAYOUT;
  const int64_t units = (nrt / sp.ranges) * (nkt / sp.S);  // of the smallest workgroup
  const GemvCfg cs{1, units >= 16 ? 16 : (units >= 8 ? 8 : 4), 3};
  LinearArgs as = a;
  as.ksplit = sp.S;
  const int rc = gemv_grid<DT, W4, GROUPED, true>(as, cs, static_cast<int>(sp.ranges * sp.S), s);
  if (rc != LSQ_OK) return rc;
  return launch_split_merge<DT>(a.part, static_cast<int>(sp.S), a.M, a.N, a.bias, a.bias_dt, a.y, a.ldy, s);
}

}  // namespace

template <int DT>
int launch_gemv(int kind, const LinearArgs& a, hipStream_t s) {
  if (!gemv_enabled() || a.act != LSQ_ACT_NONE || a.xscale) return LSQ_E_LAYOUT;
  if (kind != kW4Tiled && kind != kW8Tiled) return LSQ_E_LAYOUT;
  if (a.M < 1 || a.M > 16 || a.K % kTileK != 0 || a.K < kTileK || a.N < 1) return LSQ_E_LAYOUT;
  const bool w4 = kind == kW4Tiled;
  const bool grouped = w4 && a.group < a.K;
  if (grouped && (a.group % kTileK != 0 || ((a.group / kTileK) & (a.group / kTileK - 1)) != 0)) return LSQ_E_LAYOUT;
  auto aligned4 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 3) == 0; };
  if (!aligned4(a.scale) || (a.bias && !aligned4(a.bias))) return LSQ_E_LAYOUT;
  // 32-bit buffer ranges: activations, and one workgroup's weights (<= 16 row tiles of K)
  if (((a.M - 1) * a.ldx + a.K) * 2 >= (int64_t(1) << 31)) return LSQ_E_LAYOUT;
  if (int64_t(16) * (a.K / kTileK) * kTileBytes8 >= (int64_t(1) << 31)) return LSQ_E_LAYOUT;
  if (!w4) return gemv_kind<DT, false, false>(a, s);
  return grouped ? gemv_kind<DT, true, true>(a, s) : gemv_kind<DT, true, false>(a, s);
}

template <int DT>
int launch_split_merge(const float* part, int S, int64_t M, int64_t N, const void* bias, int bias_dt,
                       void* y, int64_t ldy, hipStream_t s) {
  using St = typename Act<DT>::storage;
  if (S < 1 || S > 16) return LSQ_E_SHAPE;
  const int64_t outs = M * N;
  if (N % 4 == 0 && (reinterpret_cast<uintptr_t>(part) & 15) == 0) {
    gemv_merge_kernel<DT, 4><<<dim3(static_cast<unsigned>((outs / 4 + 255) / 256)), dim3(256), 0, s>>>(
        part, S, static_cast<int>(M), static_cast<int>(N), bias, bias_dt, static_cast<St*>(y), ldy);
  } else {
    gemv_merge_kernel<DT, 1><<<dim3(static_cast<unsigned>((outs + 255) / 256)), dim3(256), 0, s>>>(
        part, S, static_cast<int>(M), static_cast<int>(N), bias, bias_dt, static_cast<St*>(y), ldy);
  }
  return static_cast<int>(hipGetLastError());
}
template int launch_split_merge<LSQ_BF16>(const float*, int, int64_t, int64_t, const void*, int, void*, int64_t, hipStream_t);
template int launch_split_merge<LSQ_F16>(const float*, int, int64_t, int64_t, const void*, int, void*, int64_t, hipStream_t);

int64_t gemv_split_bytes(int64_t M, int64_t N, int64_t K) {
  if (!gemv_enabled()) return 0;
  return gemv_split_plan(M, N, K).bytes;
}

template int launch_gemv<LSQ_BF16>(int, const LinearArgs&, hipStream_t);
template int launch_gemv<LSQ_F16>(int, const LinearArgs&, hipStream_t);

}  // namespace lsq
