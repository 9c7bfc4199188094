// Measurement floors for benchmarks (no counterpart in the reference).
//
// lsq_probe_empty: one empty workgroup, the cost of a launch itself (graph or stream node).
// lsq_probe_read: a bare streaming read of a buffer, with nothing computed and one small
// store per lane of each workgroup's first wave: the time any kernel that must stream the
// same bytes with the same launch cannot beat. Each workgroup reads a contiguous share,
// its waves taking interleaved 1 KB pieces (64 lanes x 16 bytes), 4 loads in flight per
// lane; refills past the end go to an out-of-range buffer offset (they return zeros and
// touch no memory), so every wave issues the same instruction stream.

#include "lsq_common.h"

namespace lsq {
namespace {

constexpr int kReadDepth = 4;
constexpr uint32_t kOOB = 0x80000000u;

__global__ void __launch_bounds__(64) empty_kernel() {}

__global__ void __launch_bounds__(1024) read_kernel(const uint8_t* __restrict__ buf, uint32_t nbytes,
                                                   float* __restrict__ sink) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(buf), 0, nbytes, 0x00020000);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, waves = blockDim.x >> 6;
  const uint32_t pieces = (nbytes + 1023u) / 1024u;
  const uint32_t per_wg = (pieces + gridDim.x - 1) / gridDim.x;
  const uint32_t first = blockIdx.x * per_wg + wid;                  // this wave's first piece
  const uint32_t end = min(pieces, (blockIdx.x + 1) * per_wg);       // past this workgroup's share
  const uint32_t cnt = first < end ? (end - first + waves - 1) / waves : 0;
  const uint32_t base = first * 1024u + lane * 16u, step = waves * 1024u;
  u32x4 acc = {0, 0, 0, 0};
  u32x4 v[kReadDepth];
#pragma unroll
  for (int s = 0; s < kReadDepth; ++s)
    v[s] = __builtin_amdgcn_raw_buffer_load_b128(r, s < static_cast<int>(cnt) ? base + s * step : kOOB, 0, 2);
  for (uint32_t i = 0; i < cnt; i += kReadDepth) {
#pragma unroll
    for (int s = 0; s < kReadDepth; ++s) {
      acc ^= v[s];
      const uint32_t j = i + kReadDepth + s;
      v[s] = __builtin_amdgcn_raw_buffer_load_b128(r, j < cnt ? base + j * step : kOOB, 0, 2);
    }
  }
  if (wid == 0) sink[blockIdx.x * 64 + lane] = static_cast<float>((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) & 0xFFu);
}

}  // namespace
}  // namespace lsq

using namespace lsq;

extern "C" int lsq_probe_empty(void* stream) {
  empty_kernel<<<dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream)>>>();
  return static_cast<int>(hipGetLastError());
}

extern "C" int lsq_probe_read(const void* buf, int64_t bytes, float* sink, int grid, int block, void* stream) {
  if (bytes < 1 || bytes >= (int64_t(1) << 31) || grid < 1 || grid > 65536 || block < 64 || block > 1024 ||
      block % 64 != 0)
    return LSQ_E_SHAPE;
  if (!buf || !sink) return LSQ_E_NULL;
  read_kernel<<<dim3(static_cast<unsigned>(grid)), dim3(static_cast<unsigned>(block)), 0,
                static_cast<hipStream_t>(stream)>>>(static_cast<const uint8_t*>(buf),
                                                    static_cast<uint32_t>(bytes), sink);
  return static_cast<int>(hipGetLastError());
}
