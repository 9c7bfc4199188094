// Decode-shaped (small M) weight-only GEMV kernels: declarations shared with the
// dispatcher in lsq_linear.hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lsq {

// How the weight operand is stored in HBM.
enum WeightKind : int {
  kW8 = 0,       // int8 [N, K] row-major (QuantizedLinear.weight_q)
  kW4Tiled = 1,  // INT4 re-tiled by lsq_w4_retile (16x128 tiles of 1 KB)
  kW4Canon = 2,  // INT4 canonical packed [N, K/2] (QuantizedLinear.weight_packed)
  kW8Tiled = 3,  // int8 re-tiled by lsq_w8_retile (16x128 tiles of 2 KB)
};

struct LinearArgs {
  const void* x;       // activations [M, K], row stride ldx (elements)
  int64_t ldx;
  const uint8_t* w;    // weights, layout per WeightKind
  const void* scale;   // [N, ngroups] (per-channel: ngroups == 1)
  int scale_dt;
  const void* bias;    // [N] or nullptr
  int bias_dt;
  void* y;             // output [M, N], row stride ldy (elements)
  int64_t ldy;
  int64_t M, N, K;
  int64_t group;       // columns per scale group (== K for per-channel)
  int64_t ngroups;
  const float* xscale = nullptr;  // W8A8 only: per-token activation scales [M]
  int act = 0;                    // LSQ_ACT_SILU_MUL: gate / up rows interleaved by 16-row
                                  // tiles, y [M, N / 2] = silu(gate) * up (decode kernel only)
  float* part = nullptr;          // split-K workspace: fp32 partial sums [ksplit][M][N]
  int64_t part_bytes = 0;         // its size (0: no split)
  int ksplit = 1;                 // K slices of the split-K GEMV (set by its launcher)
};

// Launches the LDS-staged decode kernel when the shape fits it (M <= 64, K % 128 == 0,
// group % 128 == 0, activations small enough to stage in LDS). Returns LSQ_E_LAYOUT
// without launching anything when it does not fit.
template <int DT>
int launch_decode(int kind, const LinearArgs& a, hipStream_t s);

// W8A8 decode: w the tiled INT8 layout, scale the per-row weight scale;
// y = float(sum_k xq * wq) * (scale_x[m] * scale[n]) (+ bias), each step one fp32
// rounding, then one rounding to the output type DT. fused = false: x is the per-token
// quantized int8 activation [M, K] (row stride ldx bytes) with its scales in xscale.
// fused = true: x is the DT-typed activation (row stride ldx elements, 16-byte aligned)
// and every workgroup quantizes it while staging (only when all of x fits the prologue's
// first load batch). Same fit rules as launch_decode otherwise.
template <int DT>
int launch_decode_a8(const LinearArgs& a, bool fused, hipStream_t s);

// Decode GEMV for 1..16 tokens on the tiled INT4 / INT8 layouts (lsq_gemv.hip): whole row
// tiles per workgroup, balanced over the grid; on layers of fewer than 1024 row tiles with
// a workspace (a.part), split over K slices, the slices' fp32 sums added by a second
// kernel in slice order. Returns LSQ_E_LAYOUT without launching anything for shapes,
// layouts or modes it does not cover (canonical layouts, the SiLU.mul epilogue, W8A8,
// activations too large for LDS).
template <int DT>
int launch_gemv(int kind, const LinearArgs& a, hipStream_t s);

// Workspace bytes launch_gemv's split-K path needs for this shape (0: it does not split).
int64_t gemv_split_bytes(int64_t M, int64_t N, int64_t K);

// Workspace bytes launch_bgemv's split-K path needs for this shape (0: it does not split).
int64_t bgemv_split_bytes(int64_t M, int64_t N, int64_t K);

// y[m, n] = round_T(sum over s < S, in order, of part[s][m][n] + round_T(bias[n])): the
// merge of the split-K GEMV kernels (lsq_gemv.hip).
template <int DT>
int launch_split_merge(const float* part, int S, int64_t M, int64_t N, const void* bias, int bias_dt,
                       void* y, int64_t ldy, hipStream_t s);

// Batched decode GEMV for 17..64 tokens on the tiled layouts of layers with ~1000+ row
// tiles (lsq_bgemv.hip): whole row tiles per workgroup, K split over its waves, each wave's
// activations DMA'd into an LDS slab of its own. Returns LSQ_E_LAYOUT without launching
// anything for what it does not cover.
template <int DT>
int launch_bgemv(int kind, const LinearArgs& a, hipStream_t s);

// Batched decode, 16 < M <= 64 tokens (activations streamed through LDS in chunks).
// Same contract as launch_decode.
template <int DT>
int launch_decode_mb(int kind, const LinearArgs& a, hipStream_t s);

// Decode GEMV for fp32 activations and outputs, 1..8 tokens per launch (the dispatcher
// runs more tokens in blocks of 8), on the tiled layouts
// (lsq_gemv32.hip): each weight formed as round_fp32(q * s), products summed with fmaf on
// the VALU. Returns LSQ_E_LAYOUT without launching anything for what it does not cover
// (canonical layouts, more tokens, activations or scales too large for LDS).
int launch_gemv32(int kind, const LinearArgs& a, hipStream_t s);

}  // namespace lsq
