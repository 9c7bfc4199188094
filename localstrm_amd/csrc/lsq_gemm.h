// Prefill-shaped GEMM entry (M > 64) shared by the INT8 and INT4 paths.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lsq {

// Returns LSQ_E_LAYOUT when the shape is outside what the GEMM kernels cover; the
// caller then uses the generic kernel.
template <int DT>
int launch_gemm(bool w4, const void* x, int64_t ldx, const uint8_t* w, const void* scale,
                int scale_dt, int64_t group, int64_t ngroups, const void* bias, int bias_dt,
                void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, hipStream_t s);

}  // namespace lsq
