// Weight-only decode entry point (the kernel is in lsq_decode_impl.h).

#include "lsq_decode_impl.h"

namespace lsq {

template <int DT>
int launch_decode(int kind, const LinearArgs& a, hipStream_t s) {
  if (a.M < 1 || a.M > 64 || a.K % kTileK != 0 || a.K < kTileK) return LSQ_E_LAYOUT;
  const bool grouped = kind != kW8 && a.group < a.K;
  if (grouped && a.group % kTileK != 0) return LSQ_E_LAYOUT;
  // Buffer descriptors: 4-byte aligned scale / bias bases, 32-bit byte ranges.
  auto aligned4 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 3) == 0; };
  if (!aligned4(a.scale) || (a.bias && !aligned4(a.bias))) return LSQ_E_LAYOUT;
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

template int launch_decode<LSQ_BF16>(int, const LinearArgs&, hipStream_t);
template int launch_decode<LSQ_F16>(int, const LinearArgs&, hipStream_t);

}  // namespace lsq
