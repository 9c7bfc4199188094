// Prefill-shaped GEMM (M > 16 tokens): declaration shared with the dispatcher in
// lsq_linear.hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lsq_decode.h"

namespace lsq {

// Launches the LDS-dequant MFMA GEMM when the shape fits it (fp16/bf16 activations,
// K % 128 == 0, group % 128 == 0, tiled or canonical weights). Returns LSQ_E_LAYOUT
// without launching anything when it does not fit.
template <int DT>
int launch_gemm(int kind, const LinearArgs& a, hipStream_t s);

// Workspace bytes launch_gemm's split-K path needs for this shape (0: it does not split).
int64_t gemm_split_bytes(int64_t M, int64_t N, int64_t K);

// Whether 17..64 tokens go to the split-K GEMM instead of the decode kernels: layers of at
// most 256 16-row tiles with a long K (12288+), from 24 tokens (down projections such as
// 3584 x 18944 or 4096 x 14336: one 64-row tile per 128 weight rows, K cut into up to 16
// slices). LSQ_BATCH_GEMM=1 / 0 forces it for every 17..64-token call / turns it off.
bool gemm_takes_batch(int64_t M, int64_t N, int64_t K);

}  // namespace lsq
