// Decode-shaped weight-only GEMM for small batches whose activations do not fit in LDS,
// M <= 64 tokens (gfx950).
//
// GPU form of QuantizedLinear.forward (src/kernels/quantization.py:129-141) for batched
// decode steps. Same weight stream and in-register unpack as lsq_decode_impl.h: each wave
// owns one 16-row tile of W and one of KS K slices, streams its tiles once from HBM
// through a ring of kD k-tile steps in registers, and turns them into the B operands of
// v_mfma_f32_16x16x32. What changes is the activation side: the tokens of a layer with
// large K no longer fit in LDS at once (17 at K = 3584, 4 at K = 18944), so the workgroup
// streams x (padded to 16, 32 or 64 rows) through LDS in chunks of kCT k tiles per slice, double-buffered, with one barrier per chunk. Every
// token block of 16 (MB of them) reuses each unpacked weight operand, so the unpack cost
// per weight is shared by up to 64 tokens. Small-N layers split K into KS slices so that
// more waves stream; the slices' partial sums are added through LDS in slice order.
//
// Chunk pipeline (chunk c lives in LDS buffer c & 1). At the start of chunk c all
// waves pass one barrier (chunk c is visible, chunk c - 1 is finished); the workgroup
// then writes chunk c + 1, already in registers, into the other buffer with its
// per-(k tile, token) activation sums (16-lane DPP reductions), issues the global loads
// of a later chunk into the register set just freed, and computes chunk c. The
// activation loads of a chunk are issued one (INT8) or two (INT4) chunks before they are
// needed, and the weight loads issued after them stay in flight across the wait.
//
// Numerics as in lsq_decode_impl.h: weight products are exact in the fp32 accumulators; the
// INT4 nibble bias (and the magic exponent) is removed per 128-column tile with the
// activation sums, group scales are applied per tile in fp32, per-channel scales and
// the bias at the end, then one rounding to T.

#include "lsq_mfma16.h"

#include <atomic>
#include <cstdlib>

namespace lsq {
namespace {

constexpr int kCT = 2;  // k tiles per activation chunk
constexpr int kD = 8;   // weight ring depth in k tiles; a multiple of 2 * kCT

// LDS layout shared by kernel and host: per K slice, two activation chunk buffers (mp rows
// of kCT * 128 columns, row stride ldxs elements) and their per-(k tile, token) sums; the
// workgroup's scales as T (round_T(s) is a T value, so 16 bits hold it exactly; at
// K = 18944 that leaves room for 4 K slices) and its bias as round_T fp32; the
// cross-slice partial sums.
struct MbLds {
  int64_t xs, xsum, ss, sb, red, dummy, total;
  int ldxs;
};

__host__ __device__ inline MbLds mb_lds(int mp, int rows, int64_t ngs, int ks, int red_floats) {
  MbLds l;
  l.ldxs = kCT * kTileK + 8;  // +8: rows r and r + 1 start 4 banks apart
  l.xs = 0;
  l.xsum = align16(int64_t(ks) * 2 * mp * l.ldxs * 2);
  l.ss = l.xsum + int64_t(ks) * 2 * kCT * mp * 4;
  l.sb = l.ss + align16(rows * ngs * 2);
  l.red = l.sb + align16(rows * 4);
  l.dummy = l.red + int64_t(red_floats) * 4;  // 16-byte sink for stores of padding threads
  l.total = l.dummy + 32;
  return l;
}

template <int DT, int KIND, int MB, int RG, int KS, bool GROUPED>
__global__ void __launch_bounds__(64 * RG * KS) decode_mb_kernel(LinearArgs p) {
  constexpr int NT = 64 * RG * KS;
  constexpr bool W4 = KIND == kW4Tiled || KIND == kW4Canon;
  constexpr bool TILED = KIND == kW4Tiled || KIND == kW8Tiled;
  constexpr int LPT = W4 ? 1 : 2;  // 16-byte weight loads per lane per k tile
  constexpr int kTileB = W4 ? kTileBytes : kTileBytes8;
  constexpr int kStride = TILED ? kTileB : (W4 ? kTileK / 2 : kTileK);
  constexpr int kHalf = KIND == kW8Tiled ? kTileBytes8 / 2 : 64;
  constexpr int MP = 16 * MB;                 // token rows held per chunk (zero padded)
  constexpr int ROWS = RG * kTileN;
  constexpr int PIECES = kCT * kTileK / 8;    // 16-byte pieces per chunk row
  constexpr int SP = MP * PIECES;             // pieces per slice per chunk
  constexpr int XL = (KS * SP + NT - 1) / NT;  // activation loads per thread per chunk
  constexpr int RED = KS > 1 ? (KS - 1) * RG * MB * 4 * 64 : 0;
  static_assert(kD % (2 * kCT) == 0, "the ring block must hold whole pairs of chunks");
  extern __shared__ __align__(16) unsigned char smem[];
  using S = typename Act<DT>::storage;

  const int M = static_cast<int>(p.M), N = static_cast<int>(p.N), K = static_cast<int>(p.K);
  const int nkt = K / kTileK;
  const int nrt = (N + kTileN - 1) / kTileN;
  const int ng = static_cast<int>(p.ngroups);
  const int ngs = GROUPED ? ng : 1;
  const int gtiles = static_cast<int>(p.group / kTileK);
  // k tile -> group without a divide (a branch) in the loop: floor(kt / gtiles) =
  // mulhi(kt, ceil(2^32 / gtiles)), exact for kt, gtiles < 2^16
  const uint32_t gmagic = gtiles > 1 ? static_cast<uint32_t>((0x100000000ull + gtiles - 1) / gtiles) : 0u;
  // K slices: slice s owns k tiles [s * nkt / KS, (s + 1) * nkt / KS); every slice runs
  // the same number of chunks (that of the longest one), so all waves meet at the same
  // barriers.
  auto kt_lo = [&](int sl) { return sl * nkt / KS; };
  const int ntmax = (nkt + KS - 1) / KS;
  const int nchunks = (ntmax + kCT - 1) / kCT;

  const MbLds L = mb_lds(MP, ROWS, ngs, KS, RED);
  const int ldxs = L.ldxs;
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem + L.xs);
  float* xsum = reinterpret_cast<float*>(smem + L.xsum);
  S* ss = reinterpret_cast<S*>(smem + L.ss);
  float* sb = reinterpret_cast<float*>(smem + L.sb);
  float* red = reinterpret_cast<float*>(smem + L.red);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rg = wid % RG;  // row tile within the workgroup
  const int ks = wid / RG;  // K slice
  const int r = lane & 15;
  const int q = lane >> 4;
  const int rt_wg = blockIdx.x * RG;
  const int row0 = rt_wg * kTileN;
  const int rows_valid = min(ROWS, N - row0);
  const int my_lo = kt_lo(ks);
  const int my_nt = kt_lo(ks + 1) - my_lo;

  // ---- descriptors over what this workgroup reads
  const int es_s = p.scale_dt == LSQ_F32 ? 4 : 2;
  const int es_b = p.bias_dt == LSQ_F32 ? 4 : 2;
  const rsrc_t rx = make_rsrc(p.x, static_cast<uint32_t>(((M - 1) * p.ldx + K) * 2));
  const uint8_t* wbase;
  uint32_t wbytes;
  if (TILED) {
    wbase = p.w + static_cast<int64_t>(rt_wg) * nkt * kTileB;
    wbytes = static_cast<uint32_t>(min(RG, nrt - rt_wg) * nkt * kTileB);
  } else {
    const int row_bytes = W4 ? K / 2 : K;
    wbase = p.w + static_cast<int64_t>(row0) * row_bytes;
    wbytes = static_cast<uint32_t>(rows_valid * row_bytes);
  }
  const rsrc_t rw = make_rsrc(wbase, wbytes);
  const int nsc = rows_valid * ngs;
  // (the dword holding the last 16-bit element may reach 2 bytes past the array; an
  // aligned dword never crosses a page)
  const rsrc_t rs = make_rsrc(static_cast<const uint8_t*>(p.scale) + static_cast<int64_t>(row0) * ngs * es_s,
                              static_cast<uint32_t>((nsc * es_s + 3) & ~3));
  const rsrc_t rb = make_rsrc(p.bias ? static_cast<const uint8_t*>(p.bias) + static_cast<int64_t>(row0) * es_b
                                     : static_cast<const uint8_t*>(p.scale),
                              p.bias ? static_cast<uint32_t>((rows_valid * es_b + 3) & ~3) : 0u);

  // ---- scales (as T) and bias (round_T fp32) of the workgroup's rows -> LDS
  for (int t = tid; t < nsc; t += NT) {
    const uint32_t eb = static_cast<uint32_t>(t * es_s);
    ss[t] = Act<DT>::from_f32(Act<DT>::round(dword_elem(bload4(rs, eb & ~3u), (eb >> 1) & 1, p.scale_dt)));
  }
  if (p.bias) {
    for (int t = tid; t < rows_valid; t += NT) {
      const uint32_t eb = static_cast<uint32_t>(t * es_b);
      sb[t] = Act<DT>::round(dword_elem(bload4(rb, eb & ~3u), (eb >> 1) & 1, p.bias_dt));
    }
  }

  // ---- activation chunks: piece i of chunk c is slice i / SP, token (i % SP) / PIECES,
  // columns of that slice's chunk c: 8 (i % PIECES) .. +7; tokens >= M and columns past
  // the slice read as zeros.
  // XSETS register sets: chunk c + 1 is written to LDS at the start of chunk c from the
  // set its loads went into XSETS chunks earlier, so each chunk's loads have XSETS chunk
  // periods to land (INT4 takes two; INT8, whose weight ring holds twice the registers,
  // one).
  constexpr int XSETS = W4 ? 2 : 1;
  u32x4 xr[XSETS][XL];
  auto load_x = [&](int c, int set) {
#pragma unroll
    for (int u = 0; u < XL; ++u) {
      const int i = u * NT + tid;
      const int sl = i / SP;
      const int j = i - sl * SP;
      const int m = j / PIECES;
      const int k = (kt_lo(sl) + c * kCT) * kTileK + (j - m * PIECES) * 8;
      xr[set][u] = bload16<0>(rx, (i < KS * SP && m < M && k < kt_lo(sl + 1) * kTileK && c < nchunks)
                                       ? static_cast<uint32_t>((m * p.ldx + k) * 2) : kOOB);
    }
  };
  // Sum of a float over each row of 16 lanes, in every lane of the row (DPP, no LDS).
  auto row16_sum = [](float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
    return v;
  };
  auto put_x = [&](int b, int set) {
#pragma unroll
    for (int u = 0; u < XL; ++u) {
      const int i = u * NT + tid;
      const int sl = i / SP;
      const int j = i - sl * SP;
      const int m = j / PIECES;
      const int pc = j - m * PIECES;
      const u32x4 v = xr[set][u];
      const bool ok = i < KS * SP;  // padding threads store into the sink (no branch)
      uint16_t* xb = xs + ((sl * 2 + b) * MP + m) * ldxs;
      u32x4* dst = ok ? reinterpret_cast<u32x4*>(xb + pc * 8) : reinterpret_cast<u32x4*>(smem + L.dummy);
      *dst = KIND == kW4Canon ? permute_canon(v) : v;
      if (W4) {
        float sum = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) sum += Mma<DT>::lo(v[e]) + Mma<DT>::hi(v[e]);
        // the 16 pieces of one (slice, token, k tile) sit in one 16-lane row
        // (every lane of the row stores the same value: a store from one lane in 16 would
        // be a divergent branch, at which the compiler drains all global loads in flight)
        sum = row16_sum(sum);
        *(ok ? &xsum[((sl * 2 + b) * kCT + pc / 16) * MP + m] : reinterpret_cast<float*>(smem + L.dummy)) = sum;
      }
    }
  };

  // ---- weight ring: kD k-tile steps per wave over its slice; refills past the end are
  // out-of-range loads (no memory traffic), so every load is unconditional.
  u32x4 wbuf[kD][LPT];
  auto issue = [&](u32x4 (&wv)[LPT], int st) {
    const int kt = my_lo + st;
    const bool real = st < my_nt;
    const uint32_t off = TILED ? static_cast<uint32_t>((rg * nkt + kt) * kTileB + lane * 16)
                               : static_cast<uint32_t>((rg * kTileN + r) * (W4 ? K / 2 : K) +
                                                       kt * kStride + q * 16);
    wv[0] = bload16<kNT>(rw, real ? off : kOOB);
    if (LPT == 2) wv[LPT - 1] = bload16<kNT>(rw, real ? off + kHalf : kOOB);
  };

  load_x(0, 0);
  put_x(0, 0);
#pragma unroll
  for (int c = 1; c <= XSETS; ++c) load_x(c, c % XSETS);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int s = 0; s < kD; ++s) issue(wbuf[s], s);

  f32x4 acc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
  uint32_t nib_mask, magic;  // INT4 unpack constants in registers (VOP3 takes no literal)
  asm volatile("v_mov_b32 %0, 0x000f000f" : "=v"(nib_mask));
  asm volatile("v_mov_b32 %0, %1" : "=v"(magic) : "i"(Mma<DT>::kMagic));
  const S* srow = ss + (rg * kTileN + r) * ngs;

  const int nblocks = (nchunks * kCT + kD - 1) / kD;
  for (int b = 0; b < nblocks; ++b) {
#pragma unroll
    for (int s = 0; s < kD; ++s) {
      const int st = b * kD + s;
      if (s % kCT == 0) {
        const int c = st / kCT;
        if (c < nchunks) {  // uniform
          lds_barrier();    // chunk c visible to all waves; chunk c - 1 finished by all
          if (c + 1 < nchunks) {
            // (b * kD + s) / kCT = 4 b + s / kCT and 4 is a multiple of XSETS, so the set
            // is static
            put_x((c + 1) & 1, (s / kCT + 1) % XSETS);
            load_x(c + 1 + XSETS, (s / kCT + 1) % XSETS);
          }
        }
      }
      // Per k tile: unpack the ring slot and refill it, both unconditionally (a ring
      // register written on only some paths makes the compiler load into a temporary and
      // copy it over after draining every load in flight), then the LDS reads and MB
      // interleaved MFMA chains.
      const bool live = st < my_nt;  // uniform
      const int kBuf = (s / kCT) & 1;  // (b * kD + s) / kCT has the parity of s / kCT
      const uint16_t* xb = xs + (ks * 2 + kBuf) * MP * ldxs + (s % kCT) * kTileK;
      const float* xsb = xsum + ((ks * 2 + kBuf) * kCT + (s % kCT)) * MP;
      u32x4 a[MB][4];
      f32x4 xo[MB];
      float sc = 1.f;
      u32x4 bb[4];
#pragma unroll
      for (int d = 0; d < 4; ++d)
        bb[d] = W4 ? unpack_w4(wbuf[s][0][d], nib_mask, magic)
                   : convert_w8<DT>(wbuf[s][d >> 1][2 * (d & 1)], wbuf[s][d >> 1][2 * (d & 1) + 1]);
      issue(wbuf[s], st + kD);
      if (live) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int d = 0; d < 4; ++d)
            a[mb][d] = *reinterpret_cast<const u32x4*>(xb + (16 * mb + r) * ldxs + a_col<KIND>(q, d));
        if (W4) {
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) xo[mb] = *reinterpret_cast<const f32x4*>(xsb + 16 * mb + 4 * q);
        }
        if (GROUPED) {
          const uint32_t kt = static_cast<uint32_t>(my_lo + st);
          sc = Act<DT>::to_f32(srow[gtiles == 1 ? kt : __umulhi(kt, gmagic)]);
        }
        if (W4) {
          f32x4 dacc[MB];
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) dacc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int d = 0; d < 4; ++d)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) dacc[mb] = Mma<DT>::mma(a[mb][d], bb[d], dacc[mb]);
#pragma unroll
          for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float v = fmaf(-Mma<DT>::kOff4, xo[mb][e], dacc[mb][e]);
              acc[mb][e] = GROUPED ? fmaf(sc, v, acc[mb][e]) : acc[mb][e] + v;
            }
        } else {
#pragma unroll
          for (int d = 0; d < 4; ++d)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) acc[mb] = Mma<DT>::mma(a[mb][d], bb[d], acc[mb]);
        }
      }
    }
  }

  // ---- cross-slice reduction (fixed slice order), epilogue
  if (KS > 1) {
    if (ks > 0) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          red[((((ks - 1) * RG + rg) * MB + mb) * 4 + e) * 64 + lane] = acc[mb][e];
    }
    lds_barrier();
    if (ks > 0) return;
#pragma unroll
    for (int kk = 0; kk < KS - 1; ++kk)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          acc[mb][e] += red[(((kk * RG + rg) * MB + mb) * 4 + e) * 64 + lane];
  }

  // per-channel scale, bias, one rounding to T
  S* y = static_cast<S*>(p.y);
  const int rl = rg * kTileN + r;
  const int n = row0 + rl;
  if (n < N) {
    const float sc = GROUPED ? 1.f : Act<DT>::to_f32(ss[rl]);
    const float bias = p.bias ? sb[rl] : 0.f;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = 16 * mb + 4 * q + e;
        if (m < M) {
          const float v = acc[mb][e];
          y[static_cast<int64_t>(m) * p.ldy + n] = Act<DT>::from_f32(opaque(GROUPED ? v + bias : fmaf(v, sc, bias)));
        }
      }
  }
}

// ------------------------------------------------------------------ launch

int mb_max_lds() {
  static int v = -1;
  if (v < 0) {
    int dev = 0, x = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&x, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
      x = 64 * 1024;
    v = x;
  }
  return v;
}

// Workgroup shape (row tiles RG x K slices KS): 8 row tiles when that still leaves
// enough workgroups (one pass over x serves 128 rows), 4 for mid-size N; small N (fewer
// than 256 row tiles) splits K so that more waves stream the weights (4 slices of 2 row
// tiles up to 32 tokens, 2 for 64, within LDS). LSQ_DECODE_MB_RG=4|8 forces RG (tuning).
struct MbCfg {
  int rg, ks;
};

MbCfg pick_mb(int64_t N, int64_t K, int mb) {
  static int env = -1;
  if (env < 0) {
    const char* e = std::getenv("LSQ_DECODE_MB_RG");
    env = e ? std::atoi(e) : 0;
  }
  if (env == 4 || env == 8) return MbCfg{env, 1};
  const int64_t nrt = (N + kTileN - 1) / kTileN;
  // up to 32 tokens and 1536 row tiles: 6 row tiles x 2 K slices, one workgroup per CU
  // (198 at N = 18944; measured 9-17 % faster than 148 of 8 x 1 at 32 tokens; 64 tokens
  // would need more registers than 12 waves per CU leave)
  if (mb == 2 && nrt >= 8 * 128 && nrt <= 6 * 256) return MbCfg{6, 2};
  if (nrt >= 8 * 128) return MbCfg{8, 1};
  // 4 row tiles of unsplit K while that still makes ~200 workgroups or K is short (under
  // 32 k tiles); otherwise split K: INT4 4096 x 14336 at 4-32 tokens 65-68 -> 32-34 us
  // with 128 workgroups of 2 x 4 instead of 64 of 4 x 1
  const int64_t nkt = K / kTileK;
  if (nrt >= 256 && (nkt < 32 || nrt >= 800)) return MbCfg{4, 1};
  return MbCfg{2, mb == 2 ? 4 : 2};
}

template <int DT, int KIND, int MB, int RG, int KS, bool GROUPED>
int launch_one(const LinearArgs& a, hipStream_t s) {
  constexpr int RED = KS > 1 ? (KS - 1) * RG * MB * 4 * 64 : 0;
  const MbLds L = mb_lds(16 * MB, RG * kTileN, GROUPED ? a.ngroups : 1, KS, RED);
  if (L.total > mb_max_lds()) return LSQ_E_LAYOUT;
  auto kern = decode_mb_kernel<DT, KIND, MB, RG, KS, GROUPED>;
  if (L.total > 64 * 1024) {
    static std::atomic<int> attr_set{0};
    if (!attr_set.load(std::memory_order_acquire)) {
      const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, mb_max_lds());
      if (e != hipSuccess) return static_cast<int>(e);
      attr_set.store(1, std::memory_order_release);
    }
  }
  const int64_t nrt = (a.N + kTileN - 1) / kTileN;
  const dim3 grid(static_cast<unsigned>((nrt + RG - 1) / RG));
  kern<<<grid, dim3(64 * RG * KS), static_cast<size_t>(L.total), s>>>(a);
  return static_cast<int>(hipGetLastError());
}

// The staged group scales grow with K (rows x K / group floats), so at large K a split
// configuration can exceed LDS: then fewer K slices (2, then 1 with 4 row tiles) are
// tried before the caller falls back to the prefill GEMM.
template <int DT, int KIND, bool GROUPED>
int launch_kind(const LinearArgs& a, hipStream_t s) {
  int rc = LSQ_E_LAYOUT;
  if (a.M <= 16) {  // one block of 16 tokens (3584 x 18944, INT4: 41 -> 27 us against two)
    const MbCfg c = pick_mb(a.N, a.K, 2);
    if (c.rg == 6) rc = launch_one<DT, KIND, 1, 6, 2, GROUPED>(a, s);
    else if (c.ks == 4) rc = launch_one<DT, KIND, 1, 2, 4, GROUPED>(a, s);
    else rc = c.rg == 8 ? launch_one<DT, KIND, 1, 8, 1, GROUPED>(a, s) : launch_one<DT, KIND, 1, 4, 1, GROUPED>(a, s);
    if (rc == LSQ_E_LAYOUT && c.ks == 4) rc = launch_one<DT, KIND, 1, 2, 2, GROUPED>(a, s);
    if (rc == LSQ_E_LAYOUT && c.ks > 1) rc = launch_one<DT, KIND, 1, 4, 1, GROUPED>(a, s);
    return rc;
  }
  if (a.M <= 32) {
    const MbCfg c = pick_mb(a.N, a.K, 2);
    if (c.rg == 6) rc = launch_one<DT, KIND, 2, 6, 2, GROUPED>(a, s);
    else if (c.ks == 4) rc = launch_one<DT, KIND, 2, 2, 4, GROUPED>(a, s);
    else rc = c.rg == 8 ? launch_one<DT, KIND, 2, 8, 1, GROUPED>(a, s) : launch_one<DT, KIND, 2, 4, 1, GROUPED>(a, s);
    if (rc == LSQ_E_LAYOUT && c.ks == 4) rc = launch_one<DT, KIND, 2, 2, 2, GROUPED>(a, s);
    if (rc == LSQ_E_LAYOUT && c.ks > 1) rc = launch_one<DT, KIND, 2, 4, 1, GROUPED>(a, s);
    return rc;
  }
  const MbCfg c = pick_mb(a.N, a.K, 4);
  if (c.ks == 2) rc = launch_one<DT, KIND, 4, 2, 2, GROUPED>(a, s);
  else rc = c.rg == 8 ? launch_one<DT, KIND, 4, 8, 1, GROUPED>(a, s) : launch_one<DT, KIND, 4, 4, 1, GROUPED>(a, s);
  if (rc == LSQ_E_LAYOUT && c.ks > 1) rc = launch_one<DT, KIND, 4, 4, 1, GROUPED>(a, s);
  return rc;
}

}  // namespace

template <int DT>
int launch_decode_mb(int kind, const LinearArgs& a, hipStream_t s) {
  if (a.M < 1 || a.M > 64 || a.K % kTileK != 0 || a.K < kTileK) return LSQ_E_LAYOUT;
  const bool grouped = kind != kW8 && kind != kW8Tiled && a.group < a.K;
  if (grouped && a.group % kTileK != 0) return LSQ_E_LAYOUT;
  auto aligned4 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 3) == 0; };
  if (!aligned4(a.scale) || (a.bias && !aligned4(a.bias))) return LSQ_E_LAYOUT;
  // 32-bit descriptor ranges: activations, and the weight rows of one workgroup
  if (((a.M - 1) * a.ldx + a.K) * 2 >= (int64_t(1) << 31)) return LSQ_E_LAYOUT;
  if (int64_t(128) * a.K >= (int64_t(1) << 31)) return LSQ_E_LAYOUT;
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

template int launch_decode_mb<LSQ_BF16>(int, const LinearArgs&, hipStream_t);
template int launch_decode_mb<LSQ_F16>(int, const LinearArgs&, hipStream_t);

}  // namespace lsq
