// Weight quantization on the GPU: the per-channel INT8 / INT4 steps of
// QuantizedLinear.from_float (src/kernels/quantization.py:72-94, the CPU staging of the
// quantized loader :593-610) and the group-wise INT4 of this library, written straight
// into the canonical and/or the tiled layouts.
//
// Exactness. The reference computes in fp32 on the CPU, and so do these kernels, with the
// same operations, each rounded once:
//   max     = max_k |w[n, k]| over the row (per channel) or over a group of columns:
//             exact in any order;
//   scale   = max(max / qmax, fp32(1e-8)) with an IEEE division (qmax 127 or 7; the CPU
//             divides, where torch on a GPU would multiply by the rounded reciprocal);
//   grouped: the stored scale is scale rounded to its dtype (RNE), and q is computed
//            against that stored value, as the layer dequantizes with it;
//   q       = clamp(rint(w / scale), qmin, qmax) with an IEEE division and rint's
//             round-half-to-even (torch.round).
// Rows holding NaN or infinities give unspecified q (so does the reference's .to(int8)).
//
// Two launches: one wave per (row, group) reduces max|w| and writes the scale, then one
// thread per output dword (tiled layouts) or element / byte (canonical layouts) quantizes.

#include "lsq_common.h"
#include "lsq_internal.h"

namespace lsq {
namespace {

template <int WT>
__device__ __forceinline__ float load_w(const void* w, int64_t i) {
  return Act<WT>::to_f32(static_cast<const typename Act<WT>::storage*>(w)[i]);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

__device__ __forceinline__ void store_scale(void* out, int64_t i, int sdt, float v) {
  if (sdt == LSQ_F32) static_cast<float*>(out)[i] = v;
  else if (sdt == LSQ_F16) static_cast<uint16_t*>(out)[i] = f32_to_f16(v);
  else static_cast<uint16_t*>(out)[i] = f32_to_bf16(v);
}

__device__ __forceinline__ float read_scale(const void* s, int64_t i, int sdt) {
  if (sdt == LSQ_F32) return static_cast<const float*>(s)[i];
  const uint16_t b = static_cast<const uint16_t*>(s)[i];
  return sdt == LSQ_F16 ? Act<LSQ_F16>::to_f32(b) : Act<LSQ_BF16>::to_f32(b);
}

// One wave per (row n, group g): scale[n * G + g] of the columns [g * gs, min(K, g * gs + gs)).
template <int WT>
__global__ void __launch_bounds__(256) scale_kernel(const void* __restrict__ w, int64_t ldw, int64_t N,
                                                   int64_t K, int64_t gs, int64_t G, float qmax,
                                                   void* __restrict__ scale, int sdt) {
  const int lane = threadIdx.x & 63;
  const int64_t pairs = N * G;
  const int64_t waves = static_cast<int64_t>(gridDim.x) * (blockDim.x >> 6);
  for (int64_t pw = blockIdx.x * static_cast<int64_t>(blockDim.x >> 6) + (threadIdx.x >> 6); pw < pairs;
       pw += waves) {
    const int64_t n = pw / G, g = pw - n * G;
    const int64_t k0 = g * gs, k1 = min(K, k0 + gs);
    float m = 0.f;
    for (int64_t k = k0 + lane; k < k1; k += 64) m = fmaxf(m, fabsf(load_w<WT>(w, n * ldw + k)));
    m = wave_max(m);
    if (lane == 0) store_scale(scale, pw, sdt, fmaxf(__fdiv_rn(m, qmax), 1e-8f));
  }
}

__device__ __forceinline__ int quant(float v, float s, float lo, float hi) {
  return static_cast<int>(fminf(fmaxf(rintf(__fdiv_rn(v, s)), lo), hi));
}

// INT8 canonical [N, K]: one thread per element.
template <int WT>
__global__ void __launch_bounds__(256) q8_kernel(const void* __restrict__ w, int64_t ldw, int64_t N, int64_t K,
                                                const float* __restrict__ scale, int8_t* __restrict__ q) {
  const int64_t total = N * K;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t n = i / K, k = i - n * K;
    q[i] = static_cast<int8_t>(quant(load_w<WT>(w, n * ldw + k), scale[n], -128.f, 127.f));
  }
}

// INT8 tiled (K % 128 == 0): one thread per dword, as the tiled layout defines it.
template <int WT>
__global__ void __launch_bounds__(256) q8_tiled_kernel(const void* __restrict__ w, int64_t ldw, int64_t N,
                                                      int64_t K, const float* __restrict__ scale,
                                                      uint32_t* __restrict__ tiled) {
  const int64_t nkt = K / kTileK;
  const int64_t total = (N + kTileN - 1) / kTileN * nkt * (kTileBytes8 / 4);
  for (int64_t t = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; t < total;
       t += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t tile = t / (kTileBytes8 / 4);
    const int wd = static_cast<int>(t - tile * (kTileBytes8 / 4));
    const int j = wd >> 8, lane = (wd >> 2) & 63, d = wd & 3;
    const int64_t rt = tile / nkt, kt = tile - rt * nkt;
    const int64_t n = rt * kTileN + (lane & 15);
    uint32_t v = 0;
    if (n < N) {
      const int64_t col = kt * kTileK + (lane >> 4) * 32 + j * 16 + d * 4;
      const float s = scale[n];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        v |= (static_cast<uint32_t>(quant(load_w<WT>(w, n * ldw + col + e), s, -128.f, 127.f)) & 0xFFu) << (8 * e);
    }
    tiled[t] = v;
  }
}

// The scale q of column k is computed against: the unrounded fp32 row scale (per channel,
// the reference's steps) or the stored group scale.
struct W4Scale {
  const void* s;
  int sdt;
  int64_t G, gs;
  __device__ __forceinline__ float at(int64_t n, int64_t k) const {
    return G == 1 ? static_cast<const float*>(s)[n] : read_scale(s, n * G + k / gs, sdt);
  }
};

// INT4 canonical packed [N, ceil(K/2)]: one thread per byte (low nibble = even column;
// an odd K leaves the last high nibble 0).
template <int WT>
__global__ void __launch_bounds__(256) q4_kernel(const void* __restrict__ w, int64_t ldw, int64_t N, int64_t K,
                                                W4Scale sc, uint8_t* __restrict__ packed) {
  const int64_t kb = (K + 1) / 2;
  const int64_t total = N * kb;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t n = i / kb, b = i - n * kb;
    const int64_t k = 2 * b;
    const uint32_t lo = static_cast<uint32_t>(quant(load_w<WT>(w, n * ldw + k), sc.at(n, k), -8.f, 7.f) + 8);
    uint32_t hi = 0;
    if (k + 1 < K) hi = static_cast<uint32_t>(quant(load_w<WT>(w, n * ldw + k + 1), sc.at(n, k + 1), -8.f, 7.f) + 8);
    packed[i] = static_cast<uint8_t>(lo | (hi << 4));
  }
}

// INT4 tiled (K % 128 == 0): dword d of lane l of tile (rt, kt) holds, in nibble p, column
// 128 kt + 32 (l >> 4) + 8 d + tiled_nibble_k(p) of row 16 rt + (l & 15).
template <int WT>
__global__ void __launch_bounds__(256) q4_tiled_kernel(const void* __restrict__ w, int64_t ldw, int64_t N,
                                                      int64_t K, W4Scale sc, uint32_t* __restrict__ tiled) {
  const int64_t nkt = K / kTileK;
  const int64_t total = (N + kTileN - 1) / kTileN * nkt * (kTileBytes / 4);
  for (int64_t t = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; t < total;
       t += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t tile = t / (kTileBytes / 4);
    const int wd = static_cast<int>(t - tile * (kTileBytes / 4));
    const int lane = wd >> 2, d = wd & 3;
    const int64_t rt = tile / nkt, kt = tile - rt * nkt;
    const int64_t n = rt * kTileN + (lane & 15);
    uint32_t v = 0;
    if (n < N) {
      const int64_t kbase = kt * kTileK + (lane >> 4) * 32 + 8 * d;
      const float s = sc.at(n, kbase);  // the 8 columns lie in one group (groups are >= 8 wide here)
#pragma unroll
      for (int p = 0; p < 8; ++p) {
        const int64_t k = kbase + tiled_nibble_k(p);
        v |= static_cast<uint32_t>(quant(load_w<WT>(w, n * ldw + k), s, -8.f, 7.f) + 8) << (4 * p);
      }
    }
    tiled[t] = v;
  }
}

int grid_for(int64_t work) {
  int64_t blocks = (work + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  return static_cast<int>(blocks < 1 ? 1 : blocks);
}

bool float_dt(int dt) { return dt == LSQ_F32 || dt == LSQ_F16 || dt == LSQ_BF16; }

template <int WT>
int run_w8(const void* w, int64_t ldw, int64_t N, int64_t K, float* scale, int8_t* q, int8_t* tiled,
           hipStream_t s) {
  scale_kernel<WT><<<grid_for(N * 64), 256, 0, s>>>(w, ldw, N, K, K, 1, 127.f, scale, LSQ_F32);
  if (q) q8_kernel<WT><<<grid_for(N * K), 256, 0, s>>>(w, ldw, N, K, scale, q);
  if (tiled)
    q8_tiled_kernel<WT><<<grid_for(lsq_w8_tiled_bytes(N, K) / 4), 256, 0, s>>>(
        w, ldw, N, K, scale, reinterpret_cast<uint32_t*>(tiled));
  return static_cast<int>(hipGetLastError());
}

template <int WT>
int run_w4(const void* w, int64_t ldw, int64_t N, int64_t K, int64_t gs, int64_t G, void* scale, int sdt,
           uint8_t* packed, uint8_t* tiled, hipStream_t s) {
  scale_kernel<WT><<<grid_for(N * G * 64), 256, 0, s>>>(w, ldw, N, K, gs, G, 7.f, scale, sdt);
  const W4Scale sc{scale, sdt, G, gs};
  if (packed) q4_kernel<WT><<<grid_for(N * ((K + 1) / 2)), 256, 0, s>>>(w, ldw, N, K, sc, packed);
  if (tiled)
    q4_tiled_kernel<WT><<<grid_for(lsq_w4_tiled_bytes(N, K) / 4), 256, 0, s>>>(
        w, ldw, N, K, sc, reinterpret_cast<uint32_t*>(tiled));
  return static_cast<int>(hipGetLastError());
}

}  // namespace
}  // namespace lsq

using namespace lsq;

extern "C" int lsq_quantize_w8(const void* w, int w_dtype, int64_t ldw, int64_t N, int64_t K, float* scale,
                               int8_t* weight_q, int8_t* tiled, void* stream) {
  if (N < 0 || K < 0 || ldw < K) return LSQ_E_SHAPE;
  if (!float_dt(w_dtype)) return LSQ_E_DTYPE;
  if (N == 0 || K == 0) return LSQ_OK;
  if (!w || !scale || (!weight_q && !tiled)) return LSQ_E_NULL;
  if (tiled && K % kTileK != 0) return LSQ_E_LAYOUT;
  if (tiled && (reinterpret_cast<uintptr_t>(tiled) & 15)) return LSQ_E_ALIGN;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (w_dtype) {
    case LSQ_F32: return run_w8<LSQ_F32>(w, ldw, N, K, scale, weight_q, tiled, s);
    case LSQ_F16: return run_w8<LSQ_F16>(w, ldw, N, K, scale, weight_q, tiled, s);
    default: return run_w8<LSQ_BF16>(w, ldw, N, K, scale, weight_q, tiled, s);
  }
}

extern "C" int lsq_quantize_w4(const void* w, int w_dtype, int64_t ldw, int64_t N, int64_t K, int64_t group_size,
                               void* scale, int scale_dtype, uint8_t* weight_packed, uint8_t* tiled,
                               void* stream) {
  if (N < 0 || K < 0 || ldw < K) return LSQ_E_SHAPE;
  if (group_size < 0) return LSQ_E_GROUP;
  if (!float_dt(w_dtype) || !float_dt(scale_dtype)) return LSQ_E_DTYPE;
  const bool per_channel = group_size == 0 || group_size >= K;
  if (per_channel && scale_dtype != LSQ_F32) return LSQ_E_DTYPE;
  if (N == 0 || K == 0) return LSQ_OK;
  if (!w || !scale || (!weight_packed && !tiled)) return LSQ_E_NULL;
  if (tiled && K % kTileK != 0) return LSQ_E_LAYOUT;
  // a tiled dword's 8 columns share one scale: groups of a multiple of 8 columns
  if (tiled && !per_channel && group_size % 8 != 0) return LSQ_E_LAYOUT;
  if (tiled && (reinterpret_cast<uintptr_t>(tiled) & 15)) return LSQ_E_ALIGN;
  const int64_t gs = per_channel ? K : group_size;
  const int64_t G = per_channel ? 1 : (K + gs - 1) / gs;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (w_dtype) {
    case LSQ_F32: return run_w4<LSQ_F32>(w, ldw, N, K, gs, G, scale, scale_dtype, weight_packed, tiled, s);
    case LSQ_F16: return run_w4<LSQ_F16>(w, ldw, N, K, gs, G, scale, scale_dtype, weight_packed, tiled, s);
    default: return run_w4<LSQ_BF16>(w, ldw, N, K, gs, G, scale, scale_dtype, weight_packed, tiled, s);
  }
}
