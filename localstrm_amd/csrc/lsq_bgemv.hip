// Batched decode GEMV for 17..64 tokens on the tiled INT4 / INT8 layouts (gfx950).
//
// GPU form of QuantizedLinear.forward (src/kernels/quantization.py:129-141) for a batch of
// decode tokens (the engine's batched decode step, src/engine/model_runner.py:199-205).
//
// Work split. As in the 1..16-token GEMV (lsq_gemv.hip) the workgroups take balanced,
// contiguous ranges of whole 16-row tiles (at most 1, 3 or 5 by layer size: 56 workgroups
// at N = 896, 203 at 9728, 237 at 18944), so no output is shared between workgroups.
// Inside a workgroup 8 waves (two per SIMD, so that one wave's VALU work overlaps the
// other's MFMAs) split K and the tokens: wave w takes k tiles p, p + 4, p + 8, ...
// (p = w % 4) of token half h = w / 4, for all the workgroup's row tiles. A wave thus needs only the activations of its own k tiles and tokens: it DMAs
// them (buffer_load ... lds, 1 KB contiguous per instruction) into an LDS slab of its own,
// double-buffered, and reads them back in MFMA operand order; x is read once per
// workgroup, and the main loop has no workgroup barrier, so the waves never wait for each
// other (the two waves of a phase both unpack its weights). At the end the 4 phases'
// partial sums are added in LDS in phase order (deterministic), behind one barrier.
//
// Per k tile a wave has the row tiles' weights (INT4 1 KB, INT8 2 KB each; register ring)
// and its activation slab (16 MT token rows x 128 columns, MT 16-token blocks per wave) in
// flight two k tiles ahead;
// loads past the end of the wave's k tiles or past the workgroup's rows are out of range
// (zero, no memory traffic), so the ring has no branch and a k tile past the end adds
// zeros. Then MT x 4 v_mfma_f32_16x16x32 per row tile, ordered so that consecutive MFMAs
// never wait for each other's accumulator. Arithmetic as in the other decode kernels:
// INT4 nibble u OR-ed into the exact 128 + u (bf16) / 1024 + u (fp16); group-wise, each
// k tile's sum is formed in its own accumulator, the offset 136 / 1032 removed through the
// per-(token, k tile) activation sums (MFMAs against a ones operand) and the group scale
// applied in fp32; per channel the sums run over all of K and the offset and row scale
// are applied at the end; INT8 is converted exactly. Every product is exact in fp32.
//
// The workgroup's scales are converted once to 16-bit T values in LDS (round_T of the
// stored value, what the reference multiplies by), behind one barrier, so the loop reads
// them without branching on their storage type.

#include "lsq_common.h"
#include "lsq_internal.h"
#include "lsq_decode.h"
#include "lsq_mfma16.h"

#include <algorithm>
#include <atomic>
#include <cstdlib>

namespace lsq {
namespace {

constexpr int kBgPhases = 4;              // k phases: wave w takes k tiles w % 4 + 4 i
constexpr int kBgHalves = 2;              // token halves: wave w takes tokens of half w / 4
constexpr int kBgWaves = kBgPhases * kBgHalves;
constexpr int kBgRows = 5;   // row tiles per workgroup, at most (layers of 769+ row tiles)
constexpr int kBgDepth = 2;  // k tiles in flight per wave

// 16 bytes per lane from `r` at per-lane offset `voff` into LDS at `lds` + 16 * lane (a
// device function of its own: host compilation never sees the builtin, and with it in the
// kernel body clang emitted no host launch stub for this kernel).
__device__ __forceinline__ void dma16(rsrc_t r, unsigned char* lds, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, 0, 0, 0);
}

// LDS: per wave kBgDepth activation slabs of 16 MT rows x 256 bytes (16-byte chunk c of
// row t stored at position c ^ (t & 15)), then the scales of the workgroup's rows as
// 16-bit T values [row][group]. The epilogue reuses the slabs for the waves' partial sums
// [wave][row tile][token block][element][lane] (fp32; 5 KB x MT per wave, within the
// 8 KB x MT of its slabs).
__host__ __device__ constexpr int bgemv_slab(int mt) { return 16 * mt * 256; }
__host__ __device__ constexpr int bgemv_slabs_bytes(int mt) { return kBgWaves * kBgDepth * bgemv_slab(mt); }
__host__ __device__ inline int64_t bgemv_lds(int mt, int rm, int64_t ngs) {
  return bgemv_slabs_bytes(mt) + (int64_t(rm) * kTileN * ngs * 2 + 15) / 16 * 16;
}
static_assert(kBgRows * 4 * 64 * 4 <= kBgDepth * 16 * 256, "the partial sums must fit the activation slabs");

template <int DT, bool W4, bool GROUPED, int MT, int RM, bool SPLIT>
__global__ void __launch_bounds__(64 * kBgWaves) bgemv_kernel(LinearArgs p) {
  constexpr int P = kBgPhases, D = kBgDepth;
  constexpr int kTileB = W4 ? kTileBytes : kTileBytes8;
  constexpr int LPT = W4 ? 1 : 2;    // 16-byte weight loads per lane per unit
  constexpr int kDma = 16 * MT / 4;  // DMA instructions per slab (4 rows = 1 KB each)
  constexpr int kSlab = bgemv_slab(MT);
  constexpr int kOps = RM * LPT + kDma;  // VMEM instructions of one unit
  extern __shared__ __align__(16) unsigned char smem[];
  using S = typename Act<DT>::storage;

  const int M = static_cast<int>(p.M), N = static_cast<int>(p.N), K = static_cast<int>(p.K);
  // K slices (split-K: workgroup b takes slice b % NS of row-tile range b / NS; NS = 1
  // otherwise); `nkt` counts this slice's k tiles, from k tile `kt_s0` of `nkt_all`.
  const int NS = SPLIT ? p.ksplit : 1;  // (a constant 1 in the unsplit instances)
  const int nkt_all = K / kTileK;
  const int sl = NS > 1 ? static_cast<int>(blockIdx.x) % NS : 0;
  const int kt_s0 = sl * nkt_all / NS;
  const int nkt = (sl + 1) * nkt_all / NS - kt_s0;
  const int nrt = (N + kTileN - 1) / kTileN;
  const int ngs = GROUPED ? static_cast<int>(p.ngroups) : 1;
  const int gshift = GROUPED ? __builtin_ctz(static_cast<uint32_t>(p.group / kTileK)) : 0;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ph = wid % P, half = wid / P;  // k phase, token half
  const int r = lane & 15, q = lane >> 4;
  // row tiles: the first `rem` workgroups take base + 1, the others base
  const int G = gridDim.x / NS;
  const int b = blockIdx.x / NS;
  const int base = nrt / G;
  const int rem = nrt - base * G;
  const int rt_lo = b * base + min(b, rem);
  const int R = base + (b < rem ? 1 : 0);  // 1 <= R <= RM (the launcher checks)
  const int row0 = rt_lo * kTileN;
  const int rows_valid = min(R * kTileN, N - row0);
  const int n_my = (nkt - ph + P - 1) / P;  // this wave's k tiles: ph + P i, i < n_my

  // ---- descriptors over what this workgroup reads
  const rsrc_t rx = make_rsrc(p.x, static_cast<uint32_t>(((M - 1) * p.ldx + K) * 2));
  const rsrc_t rw = make_rsrc(p.w + static_cast<int64_t>(rt_lo) * nkt_all * kTileB,
                              static_cast<uint32_t>(R * nkt_all * kTileB));
  const int es_s = p.scale_dt == LSQ_F32 ? 4 : 2;
  // (the dword holding the last 16-bit element may reach 2 bytes past the array; an
  // aligned dword never crosses a page)
  const rsrc_t rs = make_rsrc(static_cast<const uint8_t*>(p.scale) + static_cast<int64_t>(row0) * ngs * es_s,
                              static_cast<uint32_t>((rows_valid * ngs * es_s + 3) & ~3));

  // ---- unit i of this wave (k tile ph + P i) into ring slot s: the weights into
  // registers, then the activation slab into LDS. DMA instruction j fills slab rows
  // 4j .. 4j + 3 (lane l: row 4j + (l >> 4), position l & 15, holding column chunk
  // (l & 15) ^ (row & 15)); the whole offset is per lane, so the descriptor's range check
  // covers it: a token row >= M lies past the range (rows * ldx >= it since ldx >= K), and
  // so does a unit past the end (kOOB).
  unsigned char* slabs = smem + wid * D * kSlab;
  uint32_t xoff[kDma];
#pragma unroll
  for (int j = 0; j < kDma; ++j) {
    const int row = 4 * j + (lane >> 4);  // slab row; token 16 MT half + row
    xoff[j] = static_cast<uint32_t>((16 * MT * half + row) * p.ldx * 2 + 16 * ((lane & 15) ^ (row & 15)));
  }
  u32x4 wv[D][RM][LPT];
  auto issue = [&](int s, int i) {
    const int kt = ph + P * i;
    const bool real = i < n_my;
#pragma unroll
    for (int rt = 0; rt < RM; ++rt) {
      // row tiles >= R lie past the weight descriptor
      const uint32_t off = static_cast<uint32_t>((rt * nkt_all + kt_s0 + kt) * kTileB + lane * 16);
      wv[s][rt][0] = bload16<kNT>(rw, real ? off : kOOB);
      if (LPT == 2) wv[s][rt][LPT - 1] = bload16<kNT>(rw, real ? off + kTileB / 2 : kOOB);
    }
    const uint32_t kx = static_cast<uint32_t>((kt_s0 + kt) * kTileK * 2);
    unsigned char* dst = slabs + s * kSlab;
#pragma unroll
    for (int j = 0; j < kDma; ++j)
      dma16(rx, dst + j * 1024, real ? xoff[j] + kx : kOOB);
  };

  // ---- the ring first, then the scales into LDS (one barrier)
#pragma unroll
  for (int s = 0; s < D; ++s) {
    issue(s, s);
    __builtin_amdgcn_sched_barrier(0);
  }
  uint16_t* ss = reinterpret_cast<uint16_t*>(smem + bgemv_slabs_bytes(MT));
  {
    const int nsc = rows_valid * ngs;      // stored scales of this workgroup
    const int nsd = (nsc * es_s + 3) / 4;  // their dwords
    for (int t = tid; t < nsd; t += 64 * kBgWaves) {
      const uint32_t v = bload4(rs, static_cast<uint32_t>(t) * 4u);
      if (p.scale_dt == LSQ_F32) {
        ss[t] = Act<DT>::from_f32(__uint_as_float(v));
      } else {
        if (2 * t < nsc) ss[2 * t] = Act<DT>::from_f32(dword_elem(v, 0, p.scale_dt));
        if (2 * t + 1 < nsc) ss[2 * t + 1] = Act<DT>::from_f32(dword_elem(v, 1, p.scale_dt));
      }
    }
  }
  lds_barrier();
  // this lane's row of each row tile (rows past the workgroup read row 0's scales: their
  // outputs are never stored)
  int srow[RM];
#pragma unroll
  for (int rt = 0; rt < RM; ++rt) srow[rt] = (rt * kTileN + r < rows_valid ? rt * kTileN + r : 0) * ngs;

  f32x4 acc[RM][MT];
  f32x4 xst[MT];  // per-channel INT4: activation sums over all of this wave's k tiles
#pragma unroll
  for (int rt = 0; rt < RM; ++rt)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[rt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < MT; ++t) xst[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  uint32_t nib_mask = 0, magic = 0, ones = 0;
  if constexpr (W4) {
    // constants in registers, so that the unpack selects v_and_or_b32
    asm volatile("v_mov_b32 %0, 0x000f000f" : "=v"(nib_mask));
    asm volatile("v_mov_b32 %0, %1" : "=v"(magic) : "i"(Mma<DT>::kMagic));
    asm volatile("v_mov_b32 %0, %1" : "=v"(ones) : "i"(Mma<DT>::kOne2));
  }
  const u32x4 ones4 = {ones, ones, ones, ones};
  const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};

  // one k tile from ring slot s (unit i; a unit past the end holds x = 0: it adds zeros)
  auto step = [&](int s, int i) {
    // this unit's weights and activation slab have landed: every VMEM instruction issued
    // after them belongs to the later units of the ring (the compiler does not track the
    // slab, which no register receives)
    constexpr int kAfter = (D - 1) * kOps;
    __builtin_amdgcn_s_waitcnt((kAfter & 15) | (7 << 4) | (15 << 8) | ((kAfter >> 4) << 14));
    __builtin_amdgcn_sched_barrier(0);
    const unsigned char* slab = slabs + s * kSlab;
    // lane (r, q) of token block t, MFMA d: row 16 t + r, column chunk 4 q + d
    auto xop = [&](int t, int d) {
      const int row = 16 * t + r;
      return *reinterpret_cast<const u32x4*>(slab + row * 256 + (((4 * q + d) ^ r) << 4));
    };
    if constexpr (W4 && GROUPED) {
      f32x4 part[RM][MT], xsd[MT];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        u32x4 xa[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) xa[t] = xop(t, d);
#pragma unroll
        for (int t = 0; t < MT; ++t) xsd[t] = Mma<DT>::mma(xa[t], ones4, d ? xsd[t] : zero4);
#pragma unroll
        for (int rt = 0; rt < RM; ++rt) {
          const u32x4 bb = unpack_w4(wv[s][rt][0][d], nib_mask, magic);
#pragma unroll
          for (int t = 0; t < MT; ++t) part[rt][t] = Mma<DT>::mma(xa[t], bb, d ? part[rt][t] : zero4);
        }
      }
      const int g = min((kt_s0 + ph + P * i) >> gshift, ngs - 1);
#pragma unroll
      for (int rt = 0; rt < RM; ++rt) {
        const float sc = Act<DT>::to_f32(ss[srow[rt] + g]);
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[rt][t][e] += sc * fmaf(-Mma<DT>::kOff4, xsd[t][e], part[rt][t][e]);
      }
    } else {
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        u32x4 xa[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) xa[t] = xop(t, d);
        if constexpr (W4) {
#pragma unroll
          for (int t = 0; t < MT; ++t) xst[t] = Mma<DT>::mma(xa[t], ones4, xst[t]);
        }
#pragma unroll
        for (int rt = 0; rt < RM; ++rt) {
          const u32x4 bb = W4 ? unpack_w4(wv[s][rt][0][d], nib_mask, magic)
                              : convert_w8<DT>(wv[s][rt][d >> 1][2 * (d & 1)], wv[s][rt][d >> 1][2 * (d & 1) + 1]);
#pragma unroll
          for (int t = 0; t < MT; ++t) acc[rt][t] = Mma<DT>::mma(xa[t], bb, acc[rt][t]);
        }
      }
    }
    // the slab's reads are done before its refill is issued
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  };

  for (int i0 = 0; i0 < n_my; i0 += D) {
#pragma unroll
    for (int s = 0; s < D; ++s) {
      step(s, i0 + s);
      __builtin_amdgcn_sched_barrier(0);
      issue(s, i0 + s + D);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // ---- epilogue: every wave is done with its slabs (and their DMAs) before the partial
  // sums reuse them; one barrier, then the 4 phases of each token half added in order
  __builtin_amdgcn_s_waitcnt(0);
  lds_barrier();
  float* red = reinterpret_cast<float*>(smem);
  constexpr int kPart = RM * MT * 4 * 64;  // floats per wave
#pragma unroll
  for (int rt = 0; rt < RM; ++rt)
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float v = acc[rt][t][e];
        if constexpr (W4 && !GROUPED) v = fmaf(-Mma<DT>::kOff4, xst[t][e], v);
        red[wid * kPart + ((rt * MT + t) * 4 + e) * 64 + lane] = v;
      }
  lds_barrier();
  S* y = static_cast<S*>(p.y);
  const int es_b = p.bias_dt == LSQ_F32 ? 4 : 2;
  const rsrc_t rb = make_rsrc(p.bias ? static_cast<const uint8_t*>(p.bias) + static_cast<int64_t>(row0) * es_b
                                     : static_cast<const uint8_t*>(p.scale),
                              p.bias ? static_cast<uint32_t>((rows_valid * es_b + 3) & ~3) : 0u);
  for (int idx = tid; idx < kBgHalves * kPart; idx += 64 * kBgWaves) {
    const int hf = idx / kPart, pi = idx - hf * kPart;
    const int ln = pi & 63, e = (pi >> 6) & 3;
    const int t = (pi >> 8) % MT, rt = (pi >> 8) / MT;
    const int m = 16 * (MT * hf + t) + 4 * (ln >> 4) + e;
    const int nl = rt * kTileN + (ln & 15);
    if (m >= M || nl >= rows_valid) continue;
    float v = red[(P * hf) * kPart + pi];
#pragma unroll
    for (int w = 1; w < P; ++w) v += red[(P * hf + w) * kPart + pi];
    const uint32_t ebb = static_cast<uint32_t>(nl * es_b);
    const float bias = p.bias ? Act<DT>::round(dword_elem(bload4(rb, ebb & ~3u), (ebb >> 1) & 1, p.bias_dt)) : 0.f;
    if (NS > 1) {  // this slice's scaled sum; the bias and the rounding come in the merge
      p.part[(static_cast<int64_t>(sl) * M + m) * N + row0 + nl] = GROUPED ? v : v * Act<DT>::to_f32(ss[nl]);
      continue;
    }
    const float out = GROUPED ? v + bias : fmaf(v, Act<DT>::to_f32(ss[nl]), bias);
    y[static_cast<int64_t>(m) * p.ldy + row0 + nl] = Act<DT>::from_f32(opaque(out));
  }
}

// ------------------------------------------------------------------ launch

// LSQ_BGEMV=0 turns this kernel off, LSQ_BGEMV=1 uses it for every shape it covers. By
// default it serves the shapes where it measured faster than the decode kernels: INT4 at
// 33..64 tokens (18944 x 3584, M = 64: 23.3 vs 32.0 us) and at 17..32 tokens below 1000
// row tiles (896 x 4864 M = 20: 7.8 vs 13.2 us; 9728 x 896 M = 32: 6.5 vs 7.5 us), INT8
// up to 256 row tiles (896 x 4864 M = 32: 10.2 vs 12.1 us; 4096 x 14336 M = 64: 38 vs
// 49 us). Larger INT8 layers (their weights are streamed once per token half, 2 KB per
// tile) and INT4 up to 32 tokens at 1000+ row tiles measured slower (INT8 18944 x 3584
// M = 64 30.6 vs 25.2 us, 9728 x 896 M = 32 7.7 vs 7.1 us; INT4 18944 x 3584 M = 32
// 17.8 vs 16.9 us).
int bgemv_mode() {
  const char* e = std::getenv("LSQ_BGEMV");
  return e && e[0] == '0' ? 0 : (e && e[0] == '1' ? 1 : 2);
}

int g_bgemv_max_lds = -1;

int bgemv_max_lds() {
  int v = g_bgemv_max_lds;
  if (v < 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
      v = 64 * 1024;
    g_bgemv_max_lds = v;
  }
  return v;
}

template <int DT, bool W4, bool GROUPED, int MT, int RM, bool SPLIT>
int bgemv_one(const LinearArgs& a, int grid, hipStream_t s) {
  auto kern = bgemv_kernel<DT, W4, GROUPED, MT, RM, SPLIT>;
  const int64_t lds = bgemv_lds(MT, RM, GROUPED ? a.ngroups : 1);
  if (lds > bgemv_max_lds()) return LSQ_E_LAYOUT;
  if (lds > 64 * 1024) {
    static std::atomic<int> attr_set{0};
    if (!attr_set.load(std::memory_order_acquire)) {
      const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, bgemv_max_lds());
      if (e != hipSuccess) return static_cast<int>(e);
      attr_set.store(1, std::memory_order_release);
    }
  }
  bgemv_kernel<DT, W4, GROUPED, MT, RM, SPLIT><<<dim3(static_cast<unsigned>(grid)), dim3(64 * kBgWaves), static_cast<size_t>(lds), s>>>(a);
  return static_cast<int>(hipGetLastError());
}

template <int DT, bool W4, bool GROUPED, int RM, bool SPLIT = false>
int bgemv_kind(const LinearArgs& a, int grid, hipStream_t s) {
  // token blocks per wave: two halves of 1 (up to 32 tokens) or 2 (up to 64) blocks
  return a.M <= 32 ? bgemv_one<DT, W4, GROUPED, 1, RM, SPLIT>(a, grid, s)
                   : bgemv_one<DT, W4, GROUPED, 2, RM, SPLIT>(a, grid, s);
}

// Split-K plan for small-N layers with many k tiles (at most 128 row tiles, 16+ k tiles:
// the Qwen2.5-0.5B down projection 896 x 4864), where one workgroup per row tile leaves
// most CUs idle and each wave walks ~nkt / 4 k tiles: S slices of ~10 k tiles (2-3 per
// wave), one row tile per workgroup, at most 512 workgroups; the merge adds the slices in
// order. LSQ_SPLITK=0 turns it off, LSQ_SPLITK=n forces n slices.
struct BgSplit {
  int64_t S, bytes;
};

BgSplit bgemv_split_plan(int64_t M, int64_t N, int64_t K) {
  BgSplit sp{1, 0};
  const int64_t nrt = (N + kTileN - 1) / kTileN;
  const int64_t nkt = K / kTileK;
  if (M <= 16 || M > 64 || K % kTileK != 0 || nrt > 128 || nkt < 16) return sp;
  const char* e = std::getenv("LSQ_SPLITK");
  if (e && e[0] == '0') return sp;
  const int64_t forced = e ? std::atoi(e) : 0;
  int64_t S = forced >= 2 ? forced : (nkt + 9) / 10;
  S = std::min<int64_t>(S, std::min<int64_t>(16, nkt));
  if (forced < 2) S = std::min<int64_t>(S, 512 / nrt);
  if (S < 2) return sp;
  sp.S = S;
  sp.bytes = S * M * N * 4;
  return sp;
}

// Row tiles per workgroup: 1 up to 256 row tiles, 3 up to 768, 5 beyond (at most 256
// workgroups each way but for 769..999 row tiles, 154-200 workgroups).
template <int DT, bool W4, bool GROUPED>
int bgemv_rows(const LinearArgs& a, int64_t nrt, hipStream_t s) {
  if (nrt <= 256) return bgemv_kind<DT, W4, GROUPED, 1>(a, static_cast<int>(nrt), s);
  if (nrt <= 768) return bgemv_kind<DT, W4, GROUPED, 3>(a, static_cast<int>((nrt + 2) / 3), s);
  return bgemv_kind<DT, W4, GROUPED, kBgRows>(a, static_cast<int>((nrt + kBgRows - 1) / kBgRows), s);
}

}  // namespace

template <int DT>
int launch_bgemv(int kind, const LinearArgs& a, hipStream_t s) {
  const int mode = bgemv_mode();
  if (mode == 0 || a.act != LSQ_ACT_NONE || a.xscale) return LSQ_E_LAYOUT;
  if (kind != kW4Tiled && kind != kW8Tiled) return LSQ_E_LAYOUT;
  if (a.M <= 16 || a.M > 64 || a.K % kTileK != 0 || a.K < kTileK || a.N < 1) return LSQ_E_LAYOUT;
  const bool w4 = kind == kW4Tiled;
  // Every workgroup owns whole row tiles (1, 3 or 5 by layer size: 896 x 4864 runs 56
  // workgroups of one, 9728 x 896 203 of three, 18944 x 3584 237 of five).
  const int64_t nrt = (a.N + kTileN - 1) / kTileN;
  if (mode == 2 && (w4 ? (a.M <= 32 && nrt >= 1000) : nrt > 256)) return LSQ_E_LAYOUT;
  const bool grouped = w4 && a.group < a.K;
  if (grouped && (a.group % kTileK != 0 || ((a.group / kTileK) & (a.group / kTileK - 1)) != 0)) return LSQ_E_LAYOUT;
  auto aligned4 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 3) == 0; };
  if (!aligned4(a.scale) || (a.bias && !aligned4(a.bias))) return LSQ_E_LAYOUT;
  if ((nrt + kBgRows - 1) / kBgRows > 65535) return LSQ_E_LAYOUT;
  // 32-bit buffer offsets: 64 token rows of x (a token row past M is out of range by its
  // row offset alone), one workgroup's weights and scales
  if ((int64_t(64) * a.ldx + a.K) * 2 >= (int64_t(1) << 31)) return LSQ_E_LAYOUT;
  if (int64_t(kBgRows) * (a.K / kTileK) * kTileBytes8 >= (int64_t(1) << 31)) return LSQ_E_LAYOUT;
  const BgSplit sp = bgemv_split_plan(a.M, a.N, a.K);
  if (sp.S >= 2 && a.part && a.part_bytes >= sp.bytes) {
    // one row tile per workgroup, times S slices
    LinearArgs as = a;
    as.ksplit = static_cast<int>(sp.S);
    const int grid = static_cast<int>(nrt * sp.S);
    const int rc = !w4 ? bgemv_kind<DT, false, false, 1, true>(as, grid, s)
                       : (grouped ? bgemv_kind<DT, true, true, 1, true>(as, grid, s)
                                  : bgemv_kind<DT, true, false, 1, true>(as, grid, s));
    if (rc != LSQ_OK) return rc;
    return launch_split_merge<DT>(a.part, static_cast<int>(sp.S), a.M, a.N, a.bias, a.bias_dt, a.y, a.ldy, s);
  }
  if (!w4) return bgemv_rows<DT, false, false>(a, nrt, s);
  return grouped ? bgemv_rows<DT, true, true>(a, nrt, s) : bgemv_rows<DT, true, false>(a, nrt, s);
}

int64_t bgemv_split_bytes(int64_t M, int64_t N, int64_t K) {
  if (bgemv_mode() == 0) return 0;
  return bgemv_split_plan(M, N, K).bytes;
}

template int launch_bgemv<LSQ_BF16>(int, const LinearArgs&, hipStream_t);
template int launch_bgemv<LSQ_F16>(int, const LinearArgs&, hipStream_t);

}  // namespace lsq
