// Dequantization, INT4 unpack and INT4 re-tiling kernels (gfx950).
//
// dequant_w8 / dequant_w4 are the GPU form of QuantizedLinear.dequantize
// (src/kernels/quantization.py:104-127). They are bit-exact with the reference's
// `weight_q.to(T) * scale.to(T)` because q (<= 8 significant bits) times a T-rounded
// scale is formed with one fp32 multiply and rounded once to T.
// These kernels are HBM-bound elementwise passes; each thread handles a run of 8
// consecutive columns of one row so loads and stores stay contiguous across a wave.

#include "lsq_common.h"
#include "lsq_internal.h"

namespace lsq {

constexpr int kDqRun = 8;  // columns per thread

template <int DT>
__global__ void __launch_bounds__(256) dequant_w8_kernel(const int8_t* __restrict__ wq,
                                                         const void* __restrict__ scale,
                                                         int scale_dt,
                                                         typename Act<DT>::storage* __restrict__ out,
                                                         int64_t N, int64_t K) {
  const int64_t runs = (K + kDqRun - 1) / kDqRun;
  const int64_t total = N * runs;
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t n = t / runs;
    const int64_t k0 = (t - n * runs) * kDqRun;
    const float s = Act<DT>::round(load_as_f32(scale, scale_dt, n));
    const int8_t* src = wq + n * K + k0;
    typename Act<DT>::storage* dst = out + n * K + k0;
#pragma unroll
    for (int j = 0; j < kDqRun; ++j) {
      if (k0 + j < K) dst[j] = Act<DT>::from_f32(mul_rn(static_cast<float>(src[j]), s));
    }
  }
}

template <int DT>
__global__ void __launch_bounds__(256) dequant_w4_kernel(const uint8_t* __restrict__ wp,
                                                         const void* __restrict__ scale,
                                                         int scale_dt, int64_t group,
                                                         typename Act<DT>::storage* __restrict__ out,
                                                         int64_t N, int64_t K) {
  const int64_t runs = (K + kDqRun - 1) / kDqRun;
  const int64_t total = N * runs;
  const int64_t kb = (K + 1) / 2;
  const int64_t ng = (K + group - 1) / group;
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t n = t / runs;
    const int64_t k0 = (t - n * runs) * kDqRun;
    const uint8_t* src = wp + n * kb + k0 / 2;
    typename Act<DT>::storage* dst = out + n * K + k0;
#pragma unroll
    for (int j = 0; j < kDqRun; ++j) {
      const int64_t k = k0 + j;
      if (k < K) {
        const uint8_t byte = src[j >> 1];
        const int q = static_cast<int>((j & 1) ? (byte >> 4) : (byte & 0xF)) - 8;
        const float s = Act<DT>::round(load_as_f32(scale, scale_dt, n * ng + k / group));
        dst[j] = Act<DT>::from_f32(mul_rn(static_cast<float>(q), s));
      }
    }
  }
}

__global__ void __launch_bounds__(256) unpack_w4_kernel(const uint8_t* __restrict__ wp,
                                                        int8_t* __restrict__ out, int64_t N,
                                                        int64_t K) {
  const int64_t kb = (K + 1) / 2;
  const int64_t total = N * kb;
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t n = t / kb;
    const int64_t j = t - n * kb;
    const uint8_t byte = wp[t];
    out[n * K + 2 * j] = static_cast<int8_t>((byte & 0xF) - 8);
    if (2 * j + 1 < K) out[n * K + 2 * j + 1] = static_cast<int8_t>((byte >> 4) - 8);
  }
}

// Tiled INT4 layout: see tiled_nibble_k() in lsq_internal.h. One thread per output dword.
__global__ void __launch_bounds__(256) retile_w4_kernel(const uint8_t* __restrict__ wp,
                                                        uint32_t* __restrict__ tiled, int64_t N,
                                                        int64_t K) {
  const int64_t nkt = K / kTileK;
  const int64_t nrt = (N + kTileN - 1) / kTileN;
  const int64_t total = nrt * nkt * (kTileBytes / 4);
  const int64_t kb = K / 2;
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t tile = t / (kTileBytes / 4);
    const int w = static_cast<int>(t - tile * (kTileBytes / 4));
    const int lane = w >> 2, d = w & 3;
    const int64_t rt = tile / nkt, kt = tile - rt * nkt;
    const int64_t n = rt * kTileN + (lane & 15);
    uint32_t v = 0;
    if (n < N) {
      const int64_t kbase = kt * kTileK + (lane >> 4) * 32 + 8 * d;
      const uint32_t c = *reinterpret_cast<const uint32_t*>(wp + n * kb + kbase / 2);
#pragma unroll
      for (int p = 0; p < 8; ++p) v |= ((c >> (4 * tiled_nibble_k(p))) & 0xFu) << (4 * p);
    }
    tiled[t] = v;
  }
}

__global__ void __launch_bounds__(256) untile_w4_kernel(const uint32_t* __restrict__ tiled,
                                                        uint8_t* __restrict__ wp, int64_t N,
                                                        int64_t K) {
  const int64_t nkt = K / kTileK;
  const int64_t nrt = (N + kTileN - 1) / kTileN;
  const int64_t total = nrt * nkt * (kTileBytes / 4);
  const int64_t kb = K / 2;
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t tile = t / (kTileBytes / 4);
    const int w = static_cast<int>(t - tile * (kTileBytes / 4));
    const int lane = w >> 2, d = w & 3;
    const int64_t rt = tile / nkt, kt = tile - rt * nkt;
    const int64_t n = rt * kTileN + (lane & 15);
    if (n >= N) continue;
    const int64_t kbase = kt * kTileK + (lane >> 4) * 32 + 8 * d;
    const uint32_t v = tiled[t];
    uint32_t c = 0;
#pragma unroll
    for (int p = 0; p < 8; ++p) c |= ((v >> (4 * p)) & 0xFu) << (4 * tiled_nibble_k(p));
    *reinterpret_cast<uint32_t*>(wp + n * kb + kbase / 2) = c;
  }
}

// Tiled INT8 layout (lsq_internal.h). One thread per output dword.
__global__ void __launch_bounds__(256) retile_w8_kernel(const uint32_t* __restrict__ wq,
                                                        uint32_t* __restrict__ tiled, int64_t N,
                                                        int64_t K) {
  const int64_t nkt = K / kTileK;
  const int64_t nrt = (N + kTileN - 1) / kTileN;
  const int64_t total = nrt * nkt * (kTileBytes8 / 4);
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t tile = t / (kTileBytes8 / 4);
    const int w = static_cast<int>(t - tile * (kTileBytes8 / 4));
    const int j = w >> 8, lane = (w >> 2) & 63, d = w & 3;
    const int64_t rt = tile / nkt, kt = tile - rt * nkt;
    const int64_t n = rt * kTileN + (lane & 15);
    const int64_t col = kt * kTileK + (lane >> 4) * 32 + j * 16 + d * 4;
    tiled[t] = n < N ? wq[(n * K + col) / 4] : 0u;
  }
}

__global__ void __launch_bounds__(256) untile_w8_kernel(const uint32_t* __restrict__ tiled,
                                                        uint32_t* __restrict__ wq, int64_t N,
                                                        int64_t K) {
  const int64_t nkt = K / kTileK;
  const int64_t nrt = (N + kTileN - 1) / kTileN;
  const int64_t total = nrt * nkt * (kTileBytes8 / 4);
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t tile = t / (kTileBytes8 / 4);
    const int w = static_cast<int>(t - tile * (kTileBytes8 / 4));
    const int j = w >> 8, lane = (w >> 2) & 63, d = w & 3;
    const int64_t rt = tile / nkt, kt = tile - rt * nkt;
    const int64_t n = rt * kTileN + (lane & 15);
    if (n >= N) continue;
    const int64_t col = kt * kTileK + (lane >> 4) * 32 + j * 16 + d * 4;
    wq[(n * K + col) / 4] = tiled[t];
  }
}

static inline int elementwise_grid(int64_t work) {
  int64_t blocks = (work + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (blocks < 1) blocks = 1;
  return static_cast<int>(blocks);
}

}  // namespace lsq

using namespace lsq;

extern "C" int lsq_dequant_w8(const int8_t* weight_q, const void* scale, int scale_dtype,
                              void* w_out, int out_dtype, int64_t N, int64_t K, void* stream) {
  if (!weight_q || !scale || !w_out) return LSQ_E_NULL;
  if (N < 0 || K < 0) return LSQ_E_SHAPE;
  if (scale_dtype != LSQ_F32 && scale_dtype != LSQ_F16 && scale_dtype != LSQ_BF16) return LSQ_E_DTYPE;
  if (N == 0 || K == 0) return LSQ_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int grid = elementwise_grid(N * ((K + kDqRun - 1) / kDqRun));
  switch (out_dtype) {
    case LSQ_F32:
      dequant_w8_kernel<LSQ_F32><<<grid, 256, 0, s>>>(weight_q, scale, scale_dtype, static_cast<float*>(w_out), N, K);
      break;
    case LSQ_F16:
      dequant_w8_kernel<LSQ_F16><<<grid, 256, 0, s>>>(weight_q, scale, scale_dtype, static_cast<uint16_t*>(w_out), N, K);
      break;
    case LSQ_BF16:
      dequant_w8_kernel<LSQ_BF16><<<grid, 256, 0, s>>>(weight_q, scale, scale_dtype, static_cast<uint16_t*>(w_out), N, K);
      break;
    default:
      return LSQ_E_DTYPE;
  }
  return static_cast<int>(hipGetLastError());
}

extern "C" int lsq_dequant_w4(const uint8_t* weight_packed, const void* scale, int scale_dtype,
                              int64_t group_size, void* w_out, int out_dtype, int64_t N,
                              int64_t K, void* stream) {
  if (!weight_packed || !scale || !w_out) return LSQ_E_NULL;
  if (N < 0 || K < 0) return LSQ_E_SHAPE;
  if (group_size < 1) return LSQ_E_GROUP;
  if (scale_dtype != LSQ_F32 && scale_dtype != LSQ_F16 && scale_dtype != LSQ_BF16) return LSQ_E_DTYPE;
  if (N == 0 || K == 0) return LSQ_OK;
  const int64_t group = group_size < K ? group_size : K;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int grid = elementwise_grid(N * ((K + kDqRun - 1) / kDqRun));
  switch (out_dtype) {
    case LSQ_F32:
      dequant_w4_kernel<LSQ_F32><<<grid, 256, 0, s>>>(weight_packed, scale, scale_dtype, group,
                                                      static_cast<float*>(w_out), N, K);
      break;
    case LSQ_F16:
      dequant_w4_kernel<LSQ_F16><<<grid, 256, 0, s>>>(weight_packed, scale, scale_dtype, group,
                                                      static_cast<uint16_t*>(w_out), N, K);
      break;
    case LSQ_BF16:
      dequant_w4_kernel<LSQ_BF16><<<grid, 256, 0, s>>>(weight_packed, scale, scale_dtype, group,
                                                       static_cast<uint16_t*>(w_out), N, K);
      break;
    default:
      return LSQ_E_DTYPE;
  }
  return static_cast<int>(hipGetLastError());
}

extern "C" int lsq_unpack_w4(const uint8_t* weight_packed, int8_t* q_out, int64_t N, int64_t K,
                             void* stream) {
  if (!weight_packed || !q_out) return LSQ_E_NULL;
  if (N < 0 || K < 0) return LSQ_E_SHAPE;
  if (N == 0 || K == 0) return LSQ_OK;
  unpack_w4_kernel<<<elementwise_grid(N * ((K + 1) / 2)), 256, 0, static_cast<hipStream_t>(stream)>>>(
      weight_packed, q_out, N, K);
  return static_cast<int>(hipGetLastError());
}

extern "C" int64_t lsq_w4_tiled_bytes(int64_t N, int64_t K) {
  if (N <= 0 || K <= 0 || K % kTileK != 0) return 0;
  return ((N + kTileN - 1) / kTileN) * (K / kTileK) * kTileBytes;
}

extern "C" int lsq_w4_retile(const uint8_t* weight_packed, uint8_t* tiled, int64_t N, int64_t K,
                             void* stream) {
  if (!weight_packed || !tiled) return LSQ_E_NULL;
  if (N <= 0 || K <= 0) return LSQ_E_SHAPE;
  if (K % kTileK != 0) return LSQ_E_LAYOUT;
  if ((reinterpret_cast<uintptr_t>(weight_packed) & 3) || (reinterpret_cast<uintptr_t>(tiled) & 15))
    return LSQ_E_ALIGN;
  const int64_t dwords = lsq_w4_tiled_bytes(N, K) / 4;
  retile_w4_kernel<<<elementwise_grid(dwords), 256, 0, static_cast<hipStream_t>(stream)>>>(
      weight_packed, reinterpret_cast<uint32_t*>(tiled), N, K);
  return static_cast<int>(hipGetLastError());
}

extern "C" int lsq_w4_untile(const uint8_t* tiled, uint8_t* weight_packed, int64_t N, int64_t K,
                             void* stream) {
  if (!weight_packed || !tiled) return LSQ_E_NULL;
  if (N <= 0 || K <= 0) return LSQ_E_SHAPE;
  if (K % kTileK != 0) return LSQ_E_LAYOUT;
  if ((reinterpret_cast<uintptr_t>(weight_packed) & 3) || (reinterpret_cast<uintptr_t>(tiled) & 15))
    return LSQ_E_ALIGN;
  const int64_t dwords = lsq_w4_tiled_bytes(N, K) / 4;
  untile_w4_kernel<<<elementwise_grid(dwords), 256, 0, static_cast<hipStream_t>(stream)>>>(
      reinterpret_cast<const uint32_t*>(tiled), weight_packed, N, K);
  return static_cast<int>(hipGetLastError());
}

extern "C" int64_t lsq_w8_tiled_bytes(int64_t N, int64_t K) {
  if (N <= 0 || K <= 0 || K % kTileK != 0) return 0;
  return ((N + kTileN - 1) / kTileN) * (K / kTileK) * kTileBytes8;
}

extern "C" int lsq_w8_retile(const int8_t* weight_q, int8_t* tiled, int64_t N, int64_t K,
                             void* stream) {
  if (!weight_q || !tiled) return LSQ_E_NULL;
  if (N <= 0 || K <= 0) return LSQ_E_SHAPE;
  if (K % kTileK != 0) return LSQ_E_LAYOUT;
  if ((reinterpret_cast<uintptr_t>(weight_q) & 3) || (reinterpret_cast<uintptr_t>(tiled) & 15))
    return LSQ_E_ALIGN;
  const int64_t dwords = lsq_w8_tiled_bytes(N, K) / 4;
  retile_w8_kernel<<<elementwise_grid(dwords), 256, 0, static_cast<hipStream_t>(stream)>>>(
      reinterpret_cast<const uint32_t*>(weight_q), reinterpret_cast<uint32_t*>(tiled), N, K);
  return static_cast<int>(hipGetLastError());
}

extern "C" int lsq_w8_untile(const int8_t* tiled, int8_t* weight_q, int64_t N, int64_t K,
                             void* stream) {
  if (!weight_q || !tiled) return LSQ_E_NULL;
  if (N <= 0 || K <= 0) return LSQ_E_SHAPE;
  if (K % kTileK != 0) return LSQ_E_LAYOUT;
  if ((reinterpret_cast<uintptr_t>(weight_q) & 3) || (reinterpret_cast<uintptr_t>(tiled) & 15))
    return LSQ_E_ALIGN;
  const int64_t dwords = lsq_w8_tiled_bytes(N, K) / 4;
  untile_w8_kernel<<<elementwise_grid(dwords), 256, 0, static_cast<hipStream_t>(stream)>>>(
      reinterpret_cast<const uint32_t*>(tiled), reinterpret_cast<uint32_t*>(weight_q), N, K);
  return static_cast<int>(hipGetLastError());
}
