// W8A8 decode entry point (the kernel and its W8A8 modes are in lsq_decode_impl.h).

#include "lsq_decode_impl.h"

namespace lsq {

template <int DT>
int launch_decode_a8(const LinearArgs& a, bool fused, hipStream_t s) {
  if (a.M < 1 || a.M > 64 || a.K % kTileK != 0 || a.K < kTileK) return LSQ_E_LAYOUT;
  if (!fused && !a.xscale) return LSQ_E_LAYOUT;
  auto aligned4 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 3) == 0; };
  if (!aligned4(a.scale) || (a.bias && !aligned4(a.bias))) return LSQ_E_LAYOUT;
  const int64_t xb = fused ? static_cast<int64_t>(sizeof(typename Act<DT>::storage)) : 1;
  if (fused && ((reinterpret_cast<uintptr_t>(a.x) & 15) || (a.ldx * xb) % 16)) return LSQ_E_LAYOUT;
  if (((a.M - 1) * a.ldx + a.K) * xb >= (int64_t(1) << 31)) return LSQ_E_LAYOUT;
  if (int64_t(128) * a.K >= (int64_t(1) << 31)) return LSQ_E_LAYOUT;
  return fused ? launch_kind<DT, kW8Tiled, false, kA8Fused>(a, s)
               : launch_kind<DT, kW8Tiled, false, kA8Pre>(a, s);
}

template int launch_decode_a8<LSQ_F32>(const LinearArgs&, bool, hipStream_t);
template int launch_decode_a8<LSQ_F16>(const LinearArgs&, bool, hipStream_t);
template int launch_decode_a8<LSQ_BF16>(const LinearArgs&, bool, hipStream_t);

}  // namespace lsq
