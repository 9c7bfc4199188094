// Prefill-shaped GEMM (M > 64): placeholder until the LDS-dequant MFMA kernel lands.
#include "lsq_common.h"
#include "lsq_gemm.h"

namespace lsq {

template <int DT>
int launch_gemm(bool, const void*, int64_t, const uint8_t*, const void*, int, int64_t, int64_t,
                const void*, int, void*, int64_t, int64_t, int64_t, int64_t, hipStream_t) {
  return LSQ_E_LAYOUT;
}

template int launch_gemm<LSQ_F16>(bool, const void*, int64_t, const uint8_t*, const void*, int,
                                  int64_t, int64_t, const void*, int, void*, int64_t, int64_t,
                                  int64_t, int64_t, hipStream_t);
template int launch_gemm<LSQ_BF16>(bool, const void*, int64_t, const uint8_t*, const void*, int,
                                   int64_t, int64_t, const void*, int, void*, int64_t, int64_t,
                                   int64_t, int64_t, hipStream_t);

}  // namespace lsq
