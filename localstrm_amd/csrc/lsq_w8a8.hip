// W8A8 linear layer: int8 weights x per-token int8 activations on the int8 MFMA (gfx950).
//
// GPU form of Int8GEMMLinear.forward (src/kernels/quantization.py:379-447), the MLP layer
// of the reference's 'hybrid_int8' mode. The reference quantizes the activations with a
// chain of elementwise kernels (:411-414), pads M to a multiple of 32 (:416-422), calls
// torch._int_mm (:425) and rescales in fp32 (:431-440). Here:
//
//  * the decode kernel's W8A8 modes (lsq_decode_impl.h) for M <= 64 while x_q fits its
//    LDS: int8 weights streamed once from the tiled layout straight into
//    v_mfma_i32_16x16x64_i8, no conversion; for small x (M * K <= 16384) every workgroup
//    quantizes x itself while staging it, so the layer is one launch;
//  * act_quant_kernel otherwise: one workgroup per token row: max|x| (exact in the input
//    type), the scale, and the int8 row, from x held in registers;
//  * w8a8_gemm_kernel for larger M (and 17..64 tokens whose x_q exceeds that LDS): both
//    operands DMA'd from HBM into LDS (64 x 128 or 256 x 256 tiles, several stages ahead)
//    and fed to v_mfma_i32_32x32x32_i8; the fp32 rescale and bias are the epilogue.
//
// Exactness. The int32 sum of int8 products is exact in any order (|sum| < 2^31 for
// K < 131072), so the only roundings are the reference's own elementwise ones:
//   scale_x = clamp(round_T(max|x| * fp32(1/127)), min = round_T(1e-8))
//     (torch evaluates a tensor / Python-scalar division on the GPU as a product with the
//     fp32 reciprocal; the clamp bound is the scalar converted to T, 0 for fp16)
//   x_q     = clamp(rint(fp32(x) / scale_x), -128, 127)   (IEEE division, NaN -> 0)
//   y       = round_T( fp32(acc) * (scale_x * scale_w)  [+ fp32(bias)] )
// each product and sum rounded once to fp32, never fused, so the output is bit-identical
// to the reference's sequence of elementwise kernels.
//
// Weights. The reference stores weight_q_t [K, N] (int8, N contiguous) for _int_mm. The
// kernels read the tiled INT8 layout (lsq_internal.h, 16 x 128 tiles of 2 KB) built from
// weight_q_t by lsq_w8a8_retile, with K padded to a multiple of 128 with zero columns
// (the activation workspace is padded the same way, so the padding adds nothing).

#include "lsq_common.h"
#include "lsq_internal.h"
#include "lsq_decode.h"

#include <atomic>
#include <cstdlib>
#include <cstring>
#include <mutex>

namespace lsq {
namespace {

__host__ __device__ constexpr int64_t pad_k(int64_t K) { return (K + kTileK - 1) / kTileK * kTileK; }

// ============================================================ activation quantization

constexpr int kAqR = 4;     // 16-byte chunks per thread kept in registers between passes

// NaN-propagating max (torch.max returns NaN for a row holding one).
__device__ __forceinline__ float nan_max(float a, float b) { return (b > a || b != b) ? b : a; }

// NT threads per token row: 256, or 1024 for rows longer than 256 threads hold in
// registers (more than 8192 bf16 / fp16 or 4096 fp32 values, which would otherwise be read
// twice) when the rows are few.
template <int DT, int NT>
__global__ void __launch_bounds__(NT) act_quant_kernel(const void* __restrict__ x, int64_t ldx,
                                                          int K, int Kz, bool vec,
                                                          int8_t* __restrict__ xq, int64_t ldq,
                                                          float* __restrict__ sx) {
  using S = typename Act<DT>::storage;
  constexpr int E = 16 / static_cast<int>(sizeof(S));  // elements per 16-byte chunk
  __shared__ float wmax[NT / 64];
  const int m = blockIdx.x;
  const int tid = threadIdx.x;
  const S* xr = static_cast<const S*>(x) + static_cast<int64_t>(m) * ldx;
  int8_t* qr = xq + static_cast<int64_t>(m) * ldq;
  auto elem = [](u32x4 v, int e) -> float {
    if constexpr (E == 4) return __uint_as_float(v[e]);
    else return Act<DT>::to_f32(static_cast<uint16_t>(v[e >> 1] >> (16 * (e & 1))));
  };

  // pass 1: max |x| (exact: |x| of a T value is a T value)
  const int nch = vec ? K / E : 0;
  u32x4 v[kAqR];
  float mx = 0.f;
#pragma unroll
  for (int r = 0; r < kAqR; ++r) {
    const int c = tid + r * NT;
    if (c < nch) {
      v[r] = *reinterpret_cast<const u32x4*>(xr + c * E);
#pragma unroll
      for (int e = 0; e < E; ++e) mx = nan_max(mx, fabsf(elem(v[r], e)));
    }
  }
  for (int c = tid + kAqR * NT; c < nch; c += NT) {
    const u32x4 w = *reinterpret_cast<const u32x4*>(xr + c * E);
#pragma unroll
    for (int e = 0; e < E; ++e) mx = nan_max(mx, fabsf(elem(w, e)));
  }
  for (int k = nch * E + tid; k < K; k += NT) mx = nan_max(mx, fabsf(Act<DT>::to_f32(xr[k])));
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = nan_max(mx, __shfl_xor(mx, off, 64));
  if ((tid & 63) == 0) wmax[tid >> 6] = mx;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < NT / 64; ++w) mx = nan_max(mx, wmax[w]);

  const float s = a8_scale<DT>(mx);
  const float rs = __builtin_amdgcn_rcpf(s);
  if (tid == 0) sx[m] = s;

  // pass 2: quantize, E int8 per chunk. The product with rcp(s) decides every element
  // that is not within 2^-10 of a half-integer (the argument of quant_i8_fast); a chunk
  // holding any other element (a near-tie, s = 0, a non-finite value) takes the exact
  // division for all its elements, which agrees with the product wherever that decides,
  // so the common case runs without a branch per element.
  auto put = [&](int c, u32x4 w) {
    int qv[E];
    bool exact = false;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const float t = mul_nc(elem(w, e), rs);
      const float q = __builtin_rintf(t);
      exact |= !(__builtin_fabsf(t - q) < 0.5f - 0x1p-10f);
      qv[e] = static_cast<int>(__builtin_amdgcn_fmed3f(q, -128.f, 127.f));
    }
    if (exact) {
#pragma unroll
      for (int e = 0; e < E; ++e) qv[e] = quant_i8(elem(w, e), s);
    }
    uint32_t o[E / 4];
#pragma unroll
    for (int d = 0; d < E / 4; ++d) {
      uint32_t b = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) b |= (static_cast<uint32_t>(qv[4 * d + e]) & 0xFFu) << (8 * e);
      o[d] = b;
    }
    if constexpr (E == 8) *reinterpret_cast<uint2*>(qr + c * E) = make_uint2(o[0], o[1]);
    else *reinterpret_cast<uint32_t*>(qr + c * E) = o[0];
  };
#pragma unroll
  for (int r = 0; r < kAqR; ++r) {
    const int c = tid + r * NT;
    if (c < nch) put(c, v[r]);
  }
  for (int c = tid + kAqR * NT; c < nch; c += NT) put(c, *reinterpret_cast<const u32x4*>(xr + c * E));
  for (int k = nch * E + tid; k < K; k += NT) qr[k] = static_cast<int8_t>(quant_i8_fast(Act<DT>::to_f32(xr[k]), s, rs));
  for (int k = K + tid; k < Kz; k += NT) qr[k] = 0;  // padding columns
}

template <int DT>
int launch_act_quant(const void* x, int64_t ldx, int64_t M, int64_t K, int64_t Kz, int8_t* xq,
                     int64_t ldq, float* sx, hipStream_t s) {
  using S = typename Act<DT>::storage;
  constexpr int E = 16 / static_cast<int>(sizeof(S));
  const bool vec = (reinterpret_cast<uintptr_t>(x) & 15) == 0 && ldx % E == 0 &&
                   (reinterpret_cast<uintptr_t>(xq) & 7) == 0 && ldq % 8 == 0;
  // rows past what 256 threads keep in registers, on few rows: 1024 threads (K = 18944
  // bf16, M = 64: 12.8 -> 7.1 us; at M = 2048, where 256-thread rows already fill the GPU,
  // 31.1 -> 33.7, so those keep 256)
  if (K > int64_t(256) * kAqR * E && M <= 512)
    act_quant_kernel<DT, 1024><<<dim3(static_cast<unsigned>(M)), dim3(1024), 0, s>>>(
        x, ldx, static_cast<int>(K), static_cast<int>(Kz), vec, xq, ldq, sx);
  else
    act_quant_kernel<DT, 256><<<dim3(static_cast<unsigned>(M)), dim3(256), 0, s>>>(
        x, ldx, static_cast<int>(K), static_cast<int>(Kz), vec, xq, ldq, sx);
  return static_cast<int>(hipGetLastError());
}

// ============================================================ re-tile from weight_q_t

// One thread per dword of the tiled layout: dword (tile, half j, lane l, d) holds
// W[16 rt + (l & 15)][128 kt + 32 (l >> 4) + 16 j + 4 d + e], e = 0..3, with
// W[n][k] = weight_q_t[k][n]; zero past N or K.
__global__ void w8a8_retile_kernel(const int8_t* __restrict__ wt, uint32_t* __restrict__ tiled,
                                   int64_t N, int64_t K, int64_t nkt, int64_t total) {
  const int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  if (i >= total) return;
  const int d = static_cast<int>(i & 3);
  const int l = static_cast<int>((i >> 2) & 63);
  const int j = static_cast<int>((i >> 8) & 1);
  const int64_t tile = i >> 9;
  const int64_t rt = tile / nkt, kt = tile - rt * nkt;
  const int64_t n = 16 * rt + (l & 15);
  const int64_t k0 = 128 * kt + 32 * (l >> 4) + 16 * j + 4 * d;
  uint32_t v = 0;
  if (n < N) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (k0 + e < K) v |= (static_cast<uint32_t>(static_cast<uint8_t>(wt[(k0 + e) * N + n]))) << (8 * e);
  }
  tiled[i] = v;
}

// Inverse: one thread per element of weight_q_t [K, N].
__global__ void w8a8_untile_kernel(const int8_t* __restrict__ tiled, int8_t* __restrict__ wt,
                                   int64_t N, int64_t K, int64_t nkt) {
  const int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  if (i >= N * K) return;
  const int64_t k = i / N, n = i - k * N;
  const int64_t rt = n >> 4, kt = k >> 7;
  const int c = static_cast<int>(k & 127);
  const int l = static_cast<int>(n & 15) + 16 * (c >> 5);
  const int j = (c >> 4) & 1;
  wt[i] = tiled[(rt * nkt + kt) * kTileBytes8 + j * (kTileBytes8 / 2) + l * 16 + (c & 15)];
}

// ============================================================ prefill GEMM
//
// A workgroup computes a 256 x 256 tile of y with 8 waves in a 2 x 4 layout; each wave
// owns 128 x 64 outputs as 4 x 2 blocks of v_mfma_i32_32x32x32_i8 (int32 accumulators).
// K advances BK columns per step; the x_q tile [256, BK] and the weight tile [256 rows,
// BK] both go from HBM / L2 into LDS with buffer_load ... lds into NST stages, the DMA
// NST - 1 steps ahead, one barrier per step. The barrier sits before the step's last
// sub-step of MFMAs: right after it the next step's first operands are read from the
// next stage while those MFMAs run, so the MFMA pipe does not drain at the barrier. Both
// LDS tiles store row r's 16-byte chunk c at position c ^ ((r / (256 / BK)) % (BK / 16)),
// so the 16-byte MFMA operand reads (16 rows at one chunk) spread over all 64 banks.
// Consecutive workgroups take consecutive M tiles of one N tile (they share its weights
// in L2), and, unless the blocked order below applies, each starts at a different k step
// (K rotation) so that the ~32 workgroups resident on one XCD do not all miss on the same
// activation tile at once; the int32 sums do not depend on the order.
constexpr int QNT = 512;  // 8 waves, 2 (M) x 4 (N)
__host__ __device__ constexpr int w8a8_lds(int bm, int bn, int bk, int nst) { return nst * (bm + bn) * bk; }

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ i32x16 mma32_i8(u32x4 a, u32x4 b, i32x16 c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, a),
                                               __builtin_bit_cast(i32x4, b), c, 0, 0, 0);
}

// s_waitcnt immediate: vmcnt(n), lgkmcnt(0) (expcnt left alone)
__host__ __device__ constexpr int wait_vm(int n) { return (n & 15) | (7 << 4) | ((n >> 4) << 14); }

template <int DT, int QBM, int QBN, int BK, int NST, bool SPLIT>
__global__ void __launch_bounds__(QNT) w8a8_gemm_kernel(LinearArgs p) {
  static_assert(BK == 64 || BK == 128, "k step of 64 or 128 columns");
  static_assert(NST >= 2 && NST <= 8, "2..8 LDS stages");
  constexpr int A = NST - 1;         // steps the DMA runs ahead
  constexpr int KK = BK / 32;        // MFMA sub-steps per step
  constexpr int CPR = BK / 16;       // 16-byte chunks per tile row
  constexpr int RPL = 256 / BK;      // tile rows per 256 bytes (one pass over the 64 banks)
  constexpr int RPI = 1024 / BK;     // tile rows one DMA instruction fills (1 KB)
  constexpr int QWTM = QBM / 2, QWTN = QBN / 4;  // a wave's outputs
  constexpr int QFM = QWTM / 32, QFN = QWTN / 32;  // its 32 x 32 MFMA blocks
  constexpr int kXT = QBM * BK, kWT = QBN * BK;    // bytes of the two operand tiles
  constexpr int kBx = QBM / RPI / (QNT / 64);      // DMA instructions per wave and step: x
  constexpr int kBw = QBN / RPI / (QNT / 64);      // and weights
  constexpr int kB = kBx + kBw;
  static_assert(kBx >= 1 && kBw >= 1 && QFM >= 1 && QFN >= 1, "tile too small for 8 waves");
  extern __shared__ __align__(16) unsigned char smem[];
  using S = typename Act<DT>::storage;
  const int M = static_cast<int>(p.M), N = static_cast<int>(p.N), K = static_cast<int>(p.K);
  // split-K (SPLIT): workgroup b takes K slice b % NS of tile b / NS, steps
  // [st_lo, st_lo + nsteps) of the layer's nsteps_all, and writes its int32 sums to the
  // workspace p.part [NS][M][N]; the merge kernel adds the slices and rescales
  const int NS = SPLIT ? p.ksplit : 1;
  const int tile = SPLIT ? static_cast<int>(blockIdx.x) / NS : static_cast<int>(blockIdx.x);
  const int sl = SPLIT ? static_cast<int>(blockIdx.x) % NS : 0;
  const int nsteps_all = K / BK;
  const int st_lo = sl * nsteps_all / NS;
  const int nsteps = (sl + 1) * nsteps_all / NS - st_lo;
  const int nkt = K / kTileK;  // k tiles of the weight layout
  const int mtiles = (M + QBM - 1) / QBM;
  // Tile order as in the weight-only prefill GEMM (lsq_gemm.hip, gemm_rw_kernel): groups
  // of 4 M tiles, XCD x (workgroups are dealt to the 8 XCDs round-robin) taking the x-th
  // eighth of that order, so the workgroups resident on one XCD form a 4 x 8 block of
  // tiles and, with no K rotation, share activation and weight tiles in that XCD's L2
  // (14336 x 4096: M=2048 155 -> 146 us, M=8192 535 -> 519 us); M fastest otherwise.
  int mt = tile % mtiles;
  int nt = tile / mtiles;
  const int ntiles = (N + QBN - 1) / QBN;
  const bool blocked = !SPLIT && mtiles % 4 == 0 && (mtiles * ntiles) % 8 == 0;
  if (blocked) {
    const int L = (blockIdx.x & 7) * (mtiles * ntiles / 8) + (blockIdx.x >> 3);
    const int r = L % (4 * ntiles);
    mt = 4 * (L / (4 * ntiles)) + (r & 3);
    nt = r >> 2;
  }
  const int m0 = mt * QBM, n0 = nt * QBN;
  const int rows_m = min(QBM, M - m0);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wid & 1, wn = wid >> 1;
  const int rot = blocked || SPLIT ? 0 : (((blockIdx.x >> 3) & 31) * nsteps) >> 5;
  // k step of pipeline step st; steps past the end repeat the last one (their stage is
  // never read), so every wave issues the same DMAs in every step and waits exact counts
  auto gstep = [&](int st) {
    const int g = min(st, nsteps - 1) + rot;
    return st_lo + (g >= nsteps ? g - nsteps : g);
  };
  auto xs_at = [&](int buf) { return smem + buf * (kXT + kWT); };
  auto ws_at = [&](int buf) { return smem + buf * (kXT + kWT) + kXT; };
  auto swz = [](int r) { return (r / RPL) & (CPR - 1); };

  // ---- descriptors: rows past M and row tiles past N read zeros (the row part of every
  // offset is in the range-checked per-lane offset; the scalar offset carries the k step)
  const rsrc4_t rx = make_rsrc4(static_cast<const int8_t*>(p.x) + static_cast<int64_t>(m0) * p.ldx,
                                static_cast<uint32_t>((rows_m - 1) * p.ldx + K));
  const int rt0 = n0 / kTileN;
  const int nrt = (N + kTileN - 1) / kTileN;
  const rsrc4_t rw = make_rsrc4(p.w + static_cast<int64_t>(rt0) * nkt * kTileBytes8,
                                static_cast<uint32_t>(min(QBN / kTileN, nrt - rt0) * nkt * kTileBytes8));

  // One wave DMA instruction fills RPI rows of a tile (1 KB): lane l writes row
  // rb + l / CPR at position l % CPR, i.e. chunk (l % CPR) ^ swz(row). A tiled weight row
  // r's 16-byte chunk of k tile columns 16 c' .. +15 is lane (r & 15) + 16 (c' >> 1) of
  // half (c' & 1) of its 2 KB tile; a step starting at column k0 % 128 of its k tile adds
  // 16 lanes (256 bytes) per 32 columns of that start, through the scalar offset.
  uint32_t xo[kBx], wo[kBw];
#pragma unroll
  for (int b = 0; b < kBx; ++b) {
    const int r = (wid * kBx + b) * RPI + lane / CPR;
    xo[b] = static_cast<uint32_t>(r * p.ldx + ((lane % CPR) ^ swz(r)) * 16);
  }
#pragma unroll
  for (int b = 0; b < kBw; ++b) {
    const int r = (wid * kBw + b) * RPI + lane / CPR;
    const int c = (lane % CPR) ^ swz(r);
    wo[b] = static_cast<uint32_t>((r >> 4) * nkt * kTileBytes8 + (c & 1) * (kTileBytes8 / 2) +
                                  ((r & 15) + 16 * (c >> 1)) * 16);
  }
  auto issue = [&](int st, int buf) {
    const int k0 = gstep(st) * BK;
    const int sw = (k0 >> 7) * kTileBytes8 + ((k0 & 127) >> 5) * 256;
#pragma unroll
    for (int b = 0; b < kBw; ++b) {
      if (b < kBx) dma16_async(rx, xs_at(buf) + (wid * kBx + b) * RPI * BK, xo[b], static_cast<uint32_t>(k0));
      dma16_async(rw, ws_at(buf) + (wid * kBw + b) * RPI * BK, wo[b], static_cast<uint32_t>(sw));
    }
#pragma unroll
    for (int b = kBw; b < kBx; ++b)
      dma16_async(rx, xs_at(buf) + (wid * kBx + b) * RPI * BK, xo[b], static_cast<uint32_t>(k0));
  };

  i32x16 acc[QFM][QFN];
#pragma unroll
  for (int i = 0; i < QFM; ++i)
#pragma unroll
    for (int j = 0; j < QFN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0;
  // MFMA operands: lane l reads row (l & 31) of a 32-row block, 16 columns at
  // 32 kk + 16 (l >> 5), i.e. chunk 2 kk + (l >> 5), through the swizzle (32-row blocks
  // keep swz: 32 is a multiple of RPL * CPR).
  const int frow = lane & 31;
  auto frag_off = [&](int kk) { return frow * BK + (((2 * kk + (lane >> 5)) ^ swz(frow)) << 4); };
  u32x4 a[2][QFM], b[2][QFN];
  auto load = [&](int buf, int kk, u32x4 (&aa)[QFM], u32x4 (&bb)[QFN]) {
    const unsigned char* xb = xs_at(buf) + wm * QWTM * BK;
    const unsigned char* wb = ws_at(buf) + wn * QWTN * BK;
    const int off = frag_off(kk);
#pragma unroll
    for (int i = 0; i < QFM; ++i) aa[i] = *reinterpret_cast<const u32x4*>(xb + 32 * i * BK + off);
#pragma unroll
    for (int j = 0; j < QFN; ++j) bb[j] = *reinterpret_cast<const u32x4*>(wb + 32 * j * BK + off);
  };

  // prologue: steps 0 .. A-1 in flight, step 0 landed
#pragma unroll
  for (int st = 0; st < A; ++st) issue(st, st);
  __builtin_amdgcn_s_waitcnt(wait_vm((A - 1) * kB));
  lds_barrier();
  load(0, 0, a[0], b[0]);
  for (int st = 0; st < nsteps; ++st) {
    const int buf = st % NST;
    // into the stage read in step st - 1 (all its reads completed before that step's
    // barrier)
    issue(st + A, (st + A) % NST);
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      if (kk + 1 < KK) {
        load(buf, kk + 1, a[(kk + 1) & 1], b[(kk + 1) & 1]);
      } else {
        // step st + 1 landed (steps st + 2 .. st + A stay in flight), every wave's reads
        // of this stage done; then the next step's first operands
        __builtin_amdgcn_s_waitcnt(wait_vm((A - 1) * kB));
        lds_barrier();
        load((st + 1) % NST, 0, a[(kk + 1) & 1], b[(kk + 1) & 1]);
      }
#pragma unroll
      for (int i = 0; i < QFM; ++i)
#pragma unroll
        for (int j = 0; j < QFN; ++j) acc[i][j] = mma32_i8(a[kk & 1][i], b[kk & 1][j], acc[i][j]);
    }
  }
  // the DMAs of steps past the end may still be writing their stages
  __builtin_amdgcn_s_waitcnt(wait_vm(0));
  lds_barrier();

  if constexpr (SPLIT) {  // this slice's exact int32 sums
    int* part = reinterpret_cast<int*>(p.part) + static_cast<int64_t>(sl) * M * N;
#pragma unroll
    for (int i = 0; i < QFM; ++i)
#pragma unroll
      for (int j = 0; j < QFN; ++j) {
        const int n = n0 + wn * QWTN + 32 * j + (lane & 31);
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int m = m0 + wm * QWTM + 32 * i + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
          if (m < M && n < N) part[static_cast<int64_t>(m) * N + n] = acc[i][j][v];
        }
      }
    return;
  }

  // ---- epilogue: y = fp32(acc) * (sx[m] * sw[n]) [+ fp32(bias[n])], rounded to T
  float* sxs = reinterpret_cast<float*>(smem);  // the tile's token scales (LDS is free now)
  if (tid < QBM) sxs[tid] = tid < rows_m ? p.xscale[m0 + tid] : 0.f;
  lds_barrier();
  float swn[QFN], bsn[QFN];
#pragma unroll
  for (int j = 0; j < QFN; ++j) {
    const int n = n0 + wn * QWTN + 32 * j + (lane & 31);
    swn[j] = n < N ? load_as_f32(p.scale, p.scale_dt, n) : 0.f;
    bsn[j] = (p.bias && n < N) ? load_as_f32(p.bias, p.bias_dt, n) : 0.f;
  }
  S* y = static_cast<S*>(p.y);
#pragma unroll
  for (int i = 0; i < QFM; ++i)
#pragma unroll
    for (int j = 0; j < QFN; ++j) {
      const int n = n0 + wn * QWTN + 32 * j + (lane & 31);
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int ml = wm * QWTM + 32 * i + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        const int m = m0 + ml;
        if (m < M && n < N) {
          float r = mul_nc(static_cast<float>(acc[i][j][v]), mul_nc(sxs[ml], swn[j]));
          if (p.bias) r = add_nc(r, bsn[j]);
          y[static_cast<int64_t>(m) * p.ldy + n] = Act<DT>::from_f32(opaque(r));
        }
      }
    }
}

int g_max_lds_q = -1;

int max_lds_q() {
  int v = g_max_lds_q;
  if (v < 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
      v = 64 * 1024;
    g_max_lds_q = v;
  }
  return v;
}

// y[m, n] = round_T(fp32(sum over the S slices of part[s][m][n]) * (sx[m] * sw[n])
// [+ fp32(bias[n])]): the split GEMM's merge. The int32 sum is exact in any order, and the
// rescale is the GEMM epilogue's, operation for operation, so the result is the unsplit
// kernel's bit for bit. Every slice's load is issued before the first add.
template <int DT>
__global__ void __launch_bounds__(256) w8a8_merge_kernel(const int* __restrict__ part, int S, int M, int N,
                                                         const float* __restrict__ sx, const void* sw, int sw_dt,
                                                         const void* bias, int bias_dt,
                                                         typename Act<DT>::storage* __restrict__ y, int64_t ldy) {
  constexpr int kMaxS = 16;
  const int64_t MN = int64_t(M) * N;
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= MN) return;
  const int m = static_cast<int>(i / N), n = static_cast<int>(i - int64_t(m) * N);
  int v[kMaxS];
#pragma unroll
  for (int s = 0; s < kMaxS; ++s) v[s] = s < S ? part[s * MN + i] : 0;
  int acc = 0;
#pragma unroll
  for (int s = 0; s < kMaxS; ++s) acc += v[s];
  float r = mul_nc(static_cast<float>(acc), mul_nc(sx[m], load_as_f32(sw, sw_dt, n)));
  if (bias) r = add_nc(r, load_as_f32(bias, bias_dt, n));
  y[static_cast<int64_t>(m) * ldy + n] = Act<DT>::from_f32(opaque(r));
}

// Split-K plan for the GEMM's tiles when they are fewer than 128 and K is long: the 64 x
// 128 tiles (up to 192 tokens where 256 x 256 tiles leave fewer than 256 workgroups) with
// 16+ k tiles, slices of at least 4 k tiles; the 256 x 256 tiles with 32+ steps of 64
// columns, slices of at least 8 steps (both: K >= 2048). S = min(16, 256 / tiles) slices bring the grid to
// about 256 workgroups; the workspace holds S x M x N int32 sums. 3584 x 18944: 28 small
// tiles at M = 64, S = 9; 112 large tiles at M = 2048, S = 2. LSQ_W8A8_SPLITK=0 turns it
// off, =n forces n slices (tests, sweeps).
struct W8a8Split {
  int64_t S, bytes;
};

bool w8a8_small_tiles(int64_t M, int64_t N) {
  return M <= 192 && ((M + 255) / 256) * ((N + 255) / 256) < 256;
}

W8a8Split w8a8_split_plan(int64_t M, int64_t N, int64_t Kp) {
  W8a8Split sp{1, 0};
  const char* e = std::getenv("LSQ_W8A8_SPLITK");
  if (e && e[0] == '0') return sp;
  const int64_t forced = e ? std::atoi(e) : 0;
  if (M < 1 || Kp % kTileK != 0) return sp;
  const bool small = w8a8_small_tiles(M, N);
  const int64_t tiles = small ? ((M + 63) / 64) * ((N + 127) / 128) : ((M + 255) / 256) * ((N + 255) / 256);
  const int64_t steps = small ? Kp / 128 : Kp / 64;  // pipeline steps of the tile shape
  const int64_t min_steps = small ? 4 : 8;          // per slice
  int64_t S = forced >= 2 ? forced : (tiles < 128 && steps >= 4 * min_steps ? std::min<int64_t>(16, 256 / tiles) : 1);
  if (forced < 2) S = std::min<int64_t>(S, steps / min_steps);
  if (S < 2 || S > 16 || S > steps) return sp;
  sp.S = S;
  sp.bytes = S * M * N * 4;
  return sp;
}

template <int DT, int BM, int BN, int BK, int NST, bool SPLIT = false>
int launch_w8a8_gemm_as(const LinearArgs& a, hipStream_t s) {
  constexpr int lds = w8a8_lds(BM, BN, BK, NST);
  if (lds > max_lds_q()) return LSQ_E_LAYOUT;
  if (int64_t(BN / kTileN) * a.K * kTileN >= (int64_t(1) << 31)) return LSQ_E_LAYOUT;
  auto kern = w8a8_gemm_kernel<DT, BM, BN, BK, NST, SPLIT>;
  static std::atomic<int> attr_set{0};
  if (!attr_set.load(std::memory_order_acquire)) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return static_cast<int>(e);
    attr_set.store(1, std::memory_order_release);
  }
  const int64_t tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN) * (SPLIT ? a.ksplit : 1);
  if (tiles > INT32_MAX) return LSQ_E_SHAPE;
  kern<<<dim3(static_cast<unsigned>(tiles)), dim3(QNT), lds, s>>>(a);
  return static_cast<int>(hipGetLastError());
}

template <int DT>
int launch_w8a8_gemm(const LinearArgs& a, hipStream_t s) {
  if (a.K % kTileK != 0 || a.K < kTileK || !a.xscale) return LSQ_E_LAYOUT;
  if ((a.M - 1) * a.ldx + a.K >= (int64_t(1) << 31) || (a.ldx % 16) != 0) return LSQ_E_LAYOUT;
  // LSQ_W8A8_GEMM=1: 256 x 256 tiles, 128-column steps, two stages; =2: 256 x 256, 64-column
  // steps, three stages; =3: 64 x 128 tiles, 128-column steps, six stages (tests,
  // comparisons). Default 256 x 256, 64 columns, four stages: M=2048 at 14336 x 4096
  // 157 -> 145 us against the first, M=8192 543 -> 506 us; three stages measured the same.
  // Up to 192 tokens where 256 x 256 tiles leave fewer than 256 workgroups, the 64 x 128
  // tiles (18944 x 3584: M=96 50.4 -> 45.3 us, M=128 56.1 -> 46.8, M=192 59.7 -> 48.5;
  // M=256 equal, M=512 67 -> 104).
  const char* e = std::getenv("LSQ_W8A8_GEMM");
  const int v = e ? std::atoi(e) : 0;
  if (v == 1) return launch_w8a8_gemm_as<DT, 256, 256, 128, 2>(a, s);
  if (v == 2) return launch_w8a8_gemm_as<DT, 256, 256, 64, 3>(a, s);
  const bool small = v == 3 || (v == 0 && w8a8_small_tiles(a.M, a.N));
  // with the caller's workspace, split K where the tiles are few (long-K layers)
  const W8a8Split sp = v == 0 ? w8a8_split_plan(a.M, a.N, a.K) : W8a8Split{1, 0};
  if (sp.S >= 2 && a.part && a.part_bytes >= sp.bytes && (reinterpret_cast<uintptr_t>(a.part) & 3) == 0) {
    LinearArgs as = a;
    as.ksplit = static_cast<int>(sp.S);
    const int rc = small ? launch_w8a8_gemm_as<DT, 64, 128, 128, 6, true>(as, s)
                         : launch_w8a8_gemm_as<DT, 256, 256, 64, 4, true>(as, s);
    if (rc != LSQ_OK) return rc;
    const int64_t outs = a.M * a.N;
    using St = typename Act<DT>::storage;
    w8a8_merge_kernel<DT><<<dim3(static_cast<unsigned>((outs + 255) / 256)), dim3(256), 0, s>>>(
        reinterpret_cast<const int*>(a.part), static_cast<int>(sp.S), static_cast<int>(a.M),
        static_cast<int>(a.N), a.xscale, a.scale, a.scale_dt, a.bias, a.bias_dt, static_cast<St*>(a.y), a.ldy);
    return static_cast<int>(hipGetLastError());
  }
  return small ? launch_w8a8_gemm_as<DT, 64, 128, 128, 6>(a, s) : launch_w8a8_gemm_as<DT, 256, 256, 64, 4>(a, s);
}

// LSQ_W8A8_PATH selects a path for comparisons and tests: "gemm" sends every M to the
// GEMM kernel, "unfused" quantizes activations in their own kernel for decode shapes too,
// "fused" quantizes inside the decode kernel whenever x fits its first load batch.
bool path_is(const char* want) {
  const char* e = std::getenv("LSQ_W8A8_PATH");
  return e && std::strcmp(e, want) == 0;
}

// Every workgroup of the fused decode quantizes all of x again, which costs more than
// the separate quantization launch once a workgroup's share passes ~16K activations
// (measured: 18944 x 3584 gains 3.5 us at M = 1, loses 2.4 us at M = 8). One or two
// long rows still gain (3584 x 18944: M = 1 24.0 -> 18.4 us, M = 2 25.6 -> 23.5 us;
// 4096 x 14336 at M = 4 loses 6 us).
constexpr int64_t kFusedMaxElems = 16384;
constexpr int64_t kFusedMaxElemsTwoRows = 40960;
bool fuse_quant(int64_t M, int64_t K) {
  return M * K <= kFusedMaxElems || (M <= 2 && M * K <= kFusedMaxElemsTwoRows);
}

// M <= 64: the decode kernel quantizing x itself when x is small (above) and fits its
// first load batch; otherwise x is quantized by act_quant_kernel and the decode kernel
// streams x_q while it fits in LDS; else the GEMM (64 x 128 tiles, split over K with the
// caller's workspace), or the decode kernel in token blocks (the weights are streamed
// once per block, at most 8 blocks). M > 64, or no block fits: the GEMM on x_q.
template <int DT>
int run_w8a8(const LinearArgs& ax, const LinearArgs& a, hipStream_t s) {
  const bool gemm = path_is("gemm");
  const bool fused = path_is("fused") || (fuse_quant(ax.M, ax.K) && !path_is("unfused"));
  if (a.M <= 64 && !gemm && fused) {
    const int rc = launch_decode_a8<DT>(ax, true, s);
    if (rc != LSQ_E_LAYOUT) return rc;
  }
  // a.x / a.xscale are the caller's x_q / scale_x workspace
  int rc = launch_act_quant<DT>(ax.x, ax.ldx, a.M, ax.K, a.K,
                                const_cast<int8_t*>(static_cast<const int8_t*>(a.x)), a.ldx,
                                const_cast<float*>(a.xscale), s);
  if (rc != LSQ_OK) return rc;
  if (a.M <= 64 && !gemm) {
    rc = launch_decode_a8<DT>(a, false, s);
    if (rc != LSQ_E_LAYOUT) return rc;
    // x_q does not fit the decode kernel's LDS. With the workspace, the split-K GEMM
    // (3584 x 18944: M=16 66.6 -> 33.0 us, M=32 121 -> 34.0, M=64 185 -> 35.5; 896 x 4864
    // M=32 18.5 -> 15.9). Without it, the GEMM's 64 x 128 tiles past 32 tokens, or past 16
    // on layers of 16+ such tiles (18944 x 3584: M=48 33.0 -> 27.1 us; 3584 x 18944 M=32
    // 121 -> 92); else token blocks of the decode kernel (896 x 4864 M=32: 18.5 us blocks,
    // 30.2 unsplit GEMM over 7 tiles).
    const W8a8Split sp = w8a8_split_plan(a.M, a.N, a.K);
    const bool split = sp.S >= 2 && a.part && a.part_bytes >= sp.bytes;
    const int64_t tiles = ((a.M + 63) / 64) * ((a.N + 127) / 128);
    if (split || (a.M > 16 && (a.M > 32 || tiles >= 16))) return launch_w8a8_gemm<DT>(a, s);
    using Sy = typename Act<DT>::storage;
    // At most 8 passes over W: at small N the GEMM launches few workgroups (14 at
    // N = 3584), and 8 passes of the decode kernel still beat it (3584 x 18944, 8 tokens
    // in 2 blocks of 4: 263 -> ~52 us).
    for (int64_t blk : {int64_t(32), int64_t(16), int64_t(8), int64_t(4), int64_t(2)}) {
      if (blk >= a.M || (a.M + blk - 1) / blk > 8) continue;
      LinearArgs b = a;
      b.M = blk;
      rc = launch_decode_a8<DT>(b, false, s);  // block 0; LSQ_E_LAYOUT: does not fit, nothing ran
      if (rc == LSQ_E_LAYOUT) continue;
      if (rc != LSQ_OK) return rc;
      for (int64_t m0 = blk; m0 < a.M; m0 += blk) {
        b.x = static_cast<const int8_t*>(a.x) + m0 * a.ldx;
        b.y = static_cast<Sy*>(a.y) + m0 * a.ldy;
        b.xscale = a.xscale + m0;
        b.M = a.M - m0 < blk ? a.M - m0 : blk;
        rc = launch_decode_a8<DT>(b, false, s);
        if (rc != LSQ_OK) return rc;
      }
      return LSQ_OK;
    }
  }
  return launch_w8a8_gemm<DT>(a, s);
}

bool valid_dt(int dt) { return dt == LSQ_F32 || dt == LSQ_F16 || dt == LSQ_BF16; }

}  // namespace
}  // namespace lsq

using namespace lsq;

extern "C" int64_t lsq_w8a8_tiled_bytes(int64_t N, int64_t K) {
  if (N <= 0 || K <= 0) return 0;
  return (N + kTileN - 1) / kTileN * kTileN * pad_k(K);
}

extern "C" int lsq_w8a8_retile(const int8_t* weight_q_t, int8_t* tiled, int64_t N, int64_t K,
                               void* stream) {
  if (N < 0 || K < 0) return LSQ_E_SHAPE;
  if (N == 0 || K == 0) return LSQ_OK;
  if (!weight_q_t || !tiled) return LSQ_E_NULL;
  if (reinterpret_cast<uintptr_t>(tiled) & 15) return LSQ_E_ALIGN;
  const int64_t nkt = pad_k(K) / kTileK;
  const int64_t total = lsq_w8a8_tiled_bytes(N, K) / 4;
  const int64_t blocks = (total + 255) / 256;
  if (blocks > INT32_MAX) return LSQ_E_SHAPE;
  w8a8_retile_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       static_cast<hipStream_t>(stream)>>>(weight_q_t, reinterpret_cast<uint32_t*>(tiled),
                                                           N, K, nkt, total);
  return static_cast<int>(hipGetLastError());
}

extern "C" int lsq_w8a8_untile(const int8_t* tiled, int8_t* weight_q_t, int64_t N, int64_t K,
                               void* stream) {
  if (N < 0 || K < 0) return LSQ_E_SHAPE;
  if (N == 0 || K == 0) return LSQ_OK;
  if (!weight_q_t || !tiled) return LSQ_E_NULL;
  const int64_t blocks = (N * K + 255) / 256;
  if (blocks > INT32_MAX) return LSQ_E_SHAPE;
  w8a8_untile_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       static_cast<hipStream_t>(stream)>>>(tiled, weight_q_t, N, K, pad_k(K) / kTileK);
  return static_cast<int>(hipGetLastError());
}

extern "C" int lsq_act_quant_i8(const void* x, int64_t ldx, int dtype, int64_t M, int64_t K,
                                int8_t* x_q, int64_t ldq, float* scale_x, void* stream) {
  if (M < 0 || K < 1 || ldx < K || ldq < K) return LSQ_E_SHAPE;
  if (M > INT32_MAX || K > INT32_MAX / 2) return LSQ_E_SHAPE;
  if (!valid_dt(dtype)) return LSQ_E_DTYPE;
  if (M == 0) return LSQ_OK;
  if (!x || !x_q || !scale_x) return LSQ_E_NULL;
  const int64_t kz = pad_k(K) < ldq ? pad_k(K) : ldq;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case LSQ_F32: return launch_act_quant<LSQ_F32>(x, ldx, M, K, kz, x_q, ldq, scale_x, s);
    case LSQ_F16: return launch_act_quant<LSQ_F16>(x, ldx, M, K, kz, x_q, ldq, scale_x, s);
    default: return launch_act_quant<LSQ_BF16>(x, ldx, M, K, kz, x_q, ldq, scale_x, s);
  }
}

namespace {

// lsq_w8a8_linear with an optional split-K workspace (part / part_bytes; NULL / 0: none).
int w8a8_linear(const void* x, int64_t ldx, const int8_t* tiled, const void* scale_w, int scale_w_dtype,
                const void* bias, int bias_dtype, void* y, int64_t ldy, int dtype, int64_t M, int64_t N,
                int64_t K, int8_t* x_q, float* scale_x, void* part, int64_t part_bytes, void* stream) {
  if (M < 0 || N < 0 || K < 1 || ldx < K || ldy < N) return LSQ_E_SHAPE;
  if (M > INT32_MAX / 2 || N > INT32_MAX / 2 || K >= 131072) return LSQ_E_SHAPE;
  if (!valid_dt(dtype) || !valid_dt(scale_w_dtype) || (bias && !valid_dt(bias_dtype))) return LSQ_E_DTYPE;
  if (M == 0 || N == 0) return LSQ_OK;
  if (!x || !tiled || !scale_w || !y || !x_q || !scale_x) return LSQ_E_NULL;
  if ((reinterpret_cast<uintptr_t>(tiled) & 15) || (reinterpret_cast<uintptr_t>(x_q) & 15))
    return LSQ_E_ALIGN;
  if (M > INT32_MAX || K > INT32_MAX / 2) return LSQ_E_SHAPE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t kp = pad_k(K);
  // ax: the layer on x as given (fused decode; K must be a multiple of 128 there);
  // a: the same layer on the quantized workspace x_q [M, kp]
  const uint8_t* tw = reinterpret_cast<const uint8_t*>(tiled);
  LinearArgs ax{x, ldx, tw, scale_w, scale_w_dtype, bias, bias_dtype, y, ldy, M, N, K, kp, 1, nullptr};
  LinearArgs a{x_q, kp, tw, scale_w, scale_w_dtype, bias, bias_dtype, y, ldy, M, N, kp, kp, 1, scale_x};
  if (part && part_bytes > 0) {
    a.part = static_cast<float*>(part);
    a.part_bytes = part_bytes;
  }
  int rc;
  switch (dtype) {
    case LSQ_F32: rc = run_w8a8<LSQ_F32>(ax, a, s); break;
    case LSQ_F16: rc = run_w8a8<LSQ_F16>(ax, a, s); break;
    default: rc = run_w8a8<LSQ_BF16>(ax, a, s); break;
  }
  return rc == LSQ_E_LAYOUT ? LSQ_E_SHAPE : rc;
}

}  // namespace

extern "C" int lsq_w8a8_linear(const void* x, int64_t ldx, const int8_t* tiled,
                               const void* scale_w, int scale_w_dtype, const void* bias,
                               int bias_dtype, void* y, int64_t ldy, int dtype, int64_t M,
                               int64_t N, int64_t K, int8_t* x_q, float* scale_x, void* stream) {
  return w8a8_linear(x, ldx, tiled, scale_w, scale_w_dtype, bias, bias_dtype, y, ldy, dtype, M, N, K, x_q,
                     scale_x, nullptr, 0, stream);
}

extern "C" int64_t lsq_w8a8_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M < 1 || N < 1 || K < 1 || M > INT32_MAX / 2 || N > INT32_MAX / 2 || K >= 131072) return 0;
  const int64_t b = w8a8_split_plan(M, N, pad_k(K)).bytes;
  return b > 0 ? (b + 255) / 256 * 256 : 0;
}

extern "C" int lsq_w8a8_linear_ws(const void* x, int64_t ldx, const int8_t* tiled, const void* scale_w,
                                  int scale_w_dtype, const void* bias, int bias_dtype, void* y, int64_t ldy,
                                  int dtype, int64_t M, int64_t N, int64_t K, int8_t* x_q, float* scale_x,
                                  void* workspace, int64_t workspace_bytes, void* stream) {
  if (workspace && (reinterpret_cast<uintptr_t>(workspace) & 15)) return LSQ_E_ALIGN;
  return w8a8_linear(x, ldx, tiled, scale_w, scale_w_dtype, bias, bias_dtype, y, ldy, dtype, M, N, K, x_q,
                     scale_x, workspace, workspace ? workspace_bytes : 0, stream);
}

// ---- Allocation-free W8A8 entry point ----
//
// `scratch` replaces the caller's x_q / scale_x workspace: x_q [M, round_up(K, 128)] int8
// at offset 0, scale_x [M] fp32 at the next multiple of 256 bytes. Every GPU the library
// runs on holds its own copy until the process ends. In host code `scratch` names a
// host-side stand-in, never device memory: kernels get the address hipGetSymbolAddress
// returns for the device, resolved once per device (with that device current) and kept in
// g_scratch. Nothing in it has to start at zero: the activation quantizer writes every
// x_q byte the GEMM or GEMV reads (the K padding included) and every scale, before they
// are read, on the caller's stream. Calls that overlap on one GPU share the array and race.
static __device__ __align__(256) uint8_t scratch[LSQ_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::atomic<uint8_t*> g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

// This device's address of `scratch`; `dev` is current when called.
int scratch_on(int dev, uint8_t** out) {
  if (dev < 0 || dev >= kMaxDevices) return static_cast<int>(hipErrorInvalidDevice);
  uint8_t* p = g_scratch[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (!p) {
      void* addr = nullptr;
      const hipError_t e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return static_cast<int>(e);
      if (!addr) return static_cast<int>(hipErrorInvalidSymbol);
      p = static_cast<uint8_t*>(addr);
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return LSQ_OK;
}

}  // namespace

extern "C" int lsq_w8a8_linear_noalloc(const void* x, int64_t ldx, const int8_t* tiled,
                                       const void* scale_w, int scale_w_dtype, const void* bias,
                                       int bias_dtype, void* y, int64_t ldy, int dtype, int64_t M,
                                       int64_t N, int64_t K, void* stream) {
  if (M < 0 || N < 0 || K < 1 || ldx < K || ldy < N) return LSQ_E_SHAPE;
  if (M > INT32_MAX / 2 || N > INT32_MAX / 2 || K >= 131072) return LSQ_E_SHAPE;
  // x_q rows, then the scales 256-byte aligned; checked before any HIP call
  const int64_t xq_bytes = (M * pad_k(K) + 255) / 256 * 256;
  if (xq_bytes + M * static_cast<int64_t>(sizeof(float)) > LSQ_NOALLOC_SCRATCH_BYTES) return LSQ_E_SCRATCH;
  if (M == 0 || N == 0) return LSQ_OK;
  if (!x || !tiled || !scale_w || !y) return LSQ_E_NULL;
  // the stream's device, which the kernels run on; the scratch address is per device
  hipStream_t s = static_cast<hipStream_t>(stream);
  int cur = 0, dev = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return static_cast<int>(e);
  dev = cur;
  if (s) {
    e = hipStreamGetDevice(s, &dev);
    if (e != hipSuccess) return static_cast<int>(e);
  }
  uint8_t* base = nullptr;
  int rc;
  if (dev == cur) {
    rc = scratch_on(dev, &base);
  } else {
    e = hipSetDevice(dev);
    if (e != hipSuccess) return static_cast<int>(e);
    rc = scratch_on(dev, &base);
    e = hipSetDevice(cur);
    if (rc == LSQ_OK && e != hipSuccess) rc = static_cast<int>(e);
  }
  if (rc != LSQ_OK) return rc;
  return lsq_w8a8_linear(x, ldx, tiled, scale_w, scale_w_dtype, bias, bias_dtype, y, ldy, dtype, M, N, K,
                         reinterpret_cast<int8_t*>(base), reinterpret_cast<float*>(base + xq_bytes), stream);
}
