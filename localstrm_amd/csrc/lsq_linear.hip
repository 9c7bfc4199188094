// Weight-only quantized linear layer: y = x W^T + b with INT8 / INT4 W (gfx950).
//
// GPU form of QuantizedLinear.forward (src/kernels/quantization.py:129-141), which in the
// reference materializes W = dequantize(x.dtype) and then calls F.linear. This file holds
// the C entry points and the dispatch between the kernels; none materializes W in HBM:
//
//  * decode GEMV (lsq_gemv.hip): M <= 16 on the tiled layouts, whole row tiles per
//    workgroup balanced over the grid;
//  * batched decode GEMV (lsq_bgemv.hip): 17 <= M <= 64 on the tiled layouts of the larger
//    layers;
//  * fp32 decode GEMV (lsq_gemv32.hip): fp32 activations, M <= 8, tiled layouts, on the
//    VALU with the reference's per-weight fp32 dequantization;
//  * decode (lsq_decode_impl.h): M <= 64, fp16/bf16, K % 128 == 0, all activations staged in
//    LDS once (the common decode case; up to 64 tokens when x fits in LDS);
//  * chunked decode (lsq_decode_mb.hip): M <= 64 when x does not fit (large K, e.g. 4
//    tokens at K = 18944 or 17 at K = 3584), activations streamed through LDS;
//  * prefill GEMM (lsq_gemm.hip): M > 64 (and the shapes above that fit neither decode),
//    two MFMA kernels chosen by M;
//  * generic kernel (below): any dtype / shape / group size, exact per-element dequant and
//    fp32 FMA. Used for what the fast kernels do not cover (fp32 activations beyond 8
//    tokens or on the canonical layouts, odd K or group sizes).

#include <algorithm>

#include "lsq_common.h"
#include "lsq_internal.h"
#include "lsq_gemm.h"
#include "lsq_decode.h"

#include <cstdlib>
#include <cstring>

namespace lsq {

// ============================================================ generic kernel

constexpr int kGenMB = 8;  // activation rows per wavefront

// Byte offset of weight (n, k) in the tiled layouts (lsq_internal.h), and for INT4 which
// nibble of that byte (1 = high) holds it.
__device__ __forceinline__ int64_t tiled_w4_byte(int64_t n, int64_t k, int64_t nkt, int* hi) {
  const int c = static_cast<int>(k & (kTileK - 1));
  const int e = c & 7;
  const int p = (e & 1) ? 4 + (e >> 1) : (e >> 1);  // nibble position with tiled_nibble_k(p) == e
  const int lane = (c >> 5) * 16 + static_cast<int>(n & (kTileN - 1));
  *hi = p & 1;
  return ((n / kTileN) * nkt + k / kTileK) * kTileBytes + lane * 16 + ((c >> 3) & 3) * 4 + (p >> 1);
}

__device__ __forceinline__ int64_t tiled_w8_byte(int64_t n, int64_t k, int64_t nkt) {
  const int c = static_cast<int>(k & (kTileK - 1));
  const int lane = (c >> 5) * 16 + static_cast<int>(n & (kTileN - 1));
  return ((n / kTileN) * nkt + k / kTileK) * kTileBytes8 + ((c >> 4) & 1) * 1024 + lane * 16 + (c & 15);
}

// `tiled` (optional): the weights in the tiled layout, read instead of `w` when given.
template <int DT, bool W4>
__global__ void __launch_bounds__(256) linear_generic_kernel(
    const typename Act<DT>::storage* __restrict__ x, int64_t ldx, const void* __restrict__ w,
    const uint8_t* __restrict__ tiled, const void* __restrict__ scale, int scale_dt, int64_t group,
    const void* __restrict__ bias, int bias_dt, typename Act<DT>::storage* __restrict__ y,
    int64_t ldy, int64_t M, int64_t N, int64_t K) {
  const int lane = threadIdx.x & 63;
  const int64_t n = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t m0 = blockIdx.y * (int64_t)kGenMB;
  if (n >= N) return;
  const int64_t ng = (K + group - 1) / group;
  float acc[kGenMB];
#pragma unroll
  for (int i = 0; i < kGenMB; ++i) acc[i] = 0.f;
  const int64_t nkt = K / kTileK;
  for (int64_t k = lane; k < K; k += 64) {
    int q;
    float s;
    if (W4) {
      int hi = static_cast<int>(k & 1);
      const uint8_t byte = tiled ? tiled[tiled_w4_byte(n, k, nkt, &hi)]
                                 : static_cast<const uint8_t*>(w)[n * ((K + 1) / 2) + (k >> 1)];
      q = static_cast<int>(hi ? (byte >> 4) : (byte & 0xF)) - 8;
      s = load_as_f32(scale, scale_dt, n * ng + k / group);
    } else {
      q = tiled ? static_cast<int8_t>(tiled[tiled_w8_byte(n, k, nkt)]) : static_cast<const int8_t*>(w)[n * K + k];
      s = load_as_f32(scale, scale_dt, n);
    }
    const float wv = dequant_elem<DT>(q, Act<DT>::round(s));
#pragma unroll
    for (int i = 0; i < kGenMB; ++i) {
      if (m0 + i < M) acc[i] = fmaf(Act<DT>::to_f32(x[(m0 + i) * ldx + k]), wv, acc[i]);
    }
  }
  const float b = bias ? Act<DT>::round(load_as_f32(bias, bias_dt, n)) : 0.f;
#pragma unroll
  for (int i = 0; i < kGenMB; ++i) {
    const float v = wave_sum(acc[i]);
    if (lane == 0 && m0 + i < M) y[(m0 + i) * ldy + n] = Act<DT>::from_f32(v + b);
  }
}

// ------------------------------------------------------------ generic launch

template <int DT>
static int launch_generic(bool w4, const void* x, int64_t ldx, const void* w, const uint8_t* tiled,
                          const void* scale, int scale_dt, int64_t group, const void* bias, int bias_dt,
                          void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, hipStream_t s) {
  using S = typename Act<DT>::storage;
  const dim3 grid(static_cast<unsigned>((N + 3) / 4), static_cast<unsigned>((M + kGenMB - 1) / kGenMB));
  if (grid.y > 65535u) return LSQ_E_SHAPE;
  if (w4)
    linear_generic_kernel<DT, true><<<grid, 256, 0, s>>>(static_cast<const S*>(x), ldx, w, tiled, scale,
                                                         scale_dt, group, bias, bias_dt,
                                                         static_cast<S*>(y), ldy, M, N, K);
  else
    linear_generic_kernel<DT, false><<<grid, 256, 0, s>>>(static_cast<const S*>(x), ldx, w, tiled, scale,
                                                          scale_dt, group, bias, bias_dt,
                                                          static_cast<S*>(y), ldy, M, N, K);
  return static_cast<int>(hipGetLastError());
}

static int check_common(const void* x, int64_t ldx, const void* w, const void* tiled, const void* scale,
                        void* y, int64_t ldy, int dtype, int bias_dt, const void* bias, int64_t M,
                        int64_t N, int64_t K) {
  // An empty x or y (M, N or K zero) may come with a NULL data pointer, as torch gives
  // for zero-element tensors; such a pointer is never dereferenced. The canonical weights
  // may be NULL when the tiled copy is given.
  if ((!w && !tiled) || !scale) return LSQ_E_NULL;
  if ((!x && M > 0 && K > 0) || (!y && M > 0 && N > 0)) return LSQ_E_NULL;
  if (M < 0 || N < 0 || K < 0 || ldx < K || ldy < N) return LSQ_E_SHAPE;
  if (N > INT32_MAX / 2 || K > INT32_MAX / 2 || M > INT32_MAX / 2) return LSQ_E_SHAPE;
  if (dtype != LSQ_F32 && dtype != LSQ_F16 && dtype != LSQ_BF16) return LSQ_E_DTYPE;
  if (bias && bias_dt != LSQ_F32 && bias_dt != LSQ_F16 && bias_dt != LSQ_BF16) return LSQ_E_DTYPE;
  return LSQ_OK;
}

// The fast kernels read x with 16-byte loads at column offsets that are multiples of 8.
static bool x_aligned16(const void* x, int64_t ldx) {
  return (reinterpret_cast<uintptr_t>(x) & 15) == 0 && (ldx % 8) == 0;
}

template <int DT>
static int dispatch(bool w4, const void* x, int64_t ldx, const uint8_t* w, const uint8_t* tiled,
                    const void* scale, int scale_dt, int64_t group, const void* bias, int bias_dt,
                    void* y, int64_t ldy, int64_t M, int64_t N, int64_t K, hipStream_t s,
                    int act = LSQ_ACT_NONE, void* ws = nullptr, int64_t ws_bytes = 0) {
  const int64_t ng = (K + group - 1) / group;
  if constexpr (DT != LSQ_F32) {
    const void* wf = tiled ? static_cast<const void*>(tiled) : static_cast<const void*>(w);
    const bool mfma_ok = K % kTileK == 0 && x_aligned16(x, ldx) && (reinterpret_cast<uintptr_t>(wf) & 15) == 0;
    if (act != LSQ_ACT_NONE) {  // the fused epilogue exists in the decode kernel only
      if (!mfma_ok || M > 64) return LSQ_E_LAYOUT;
      LinearArgs a{x, ldx, tiled ? tiled : w, scale, scale_dt, bias, bias_dt, y, ldy,
                   M, N, K, group, ng};
      a.act = act;
      return launch_decode<DT>(w4 ? (tiled ? kW4Tiled : kW4Canon) : (tiled ? kW8Tiled : kW8), a, s);
    }
    if (mfma_ok) {
      LinearArgs a{x, ldx, tiled ? tiled : w, scale, scale_dt, bias, bias_dt, y, ldy,
                   M, N, K, group, ng};
      a.part = static_cast<float*>(ws);
      a.part_bytes = ws ? ws_bytes : 0;
      const int kind = w4 ? (tiled ? kW4Tiled : kW4Canon) : (tiled ? kW8Tiled : kW8);
      // decode with all activations in LDS; else (x too large for LDS, e.g. 4 tokens at
      // K = 18944) the chunked decode; else the prefill GEMM
      // 17..64 tokens on long-K, small-N layers: the split-K GEMM, when the workspace for
      // its slices is there (gemm_takes_batch)
      const bool batch_gemm = M > 16 && M <= 64 && gemm_takes_batch(M, N, K) && ws &&
                              ws_bytes >= gemm_split_bytes(M, N, K);
      int rc = LSQ_E_LAYOUT;
      if (M <= 16) rc = launch_gemv<DT>(kind, a, s);
      if (!batch_gemm) {
        if (rc == LSQ_E_LAYOUT && M > 16 && M <= 64) rc = launch_bgemv<DT>(kind, a, s);
        if (rc == LSQ_E_LAYOUT && M <= 64) rc = launch_decode<DT>(kind, a, s);
        if (rc == LSQ_E_LAYOUT && M <= 64) rc = launch_decode_mb<DT>(kind, a, s);
      }
      if (rc == LSQ_E_LAYOUT && M > 16) rc = launch_gemm<DT>(kind, a, s);
      if (rc != LSQ_E_LAYOUT) return rc;
    }
  } else {
    // fp32 activations on tiled weights: the VALU decode GEMV, in blocks of 8 tokens past 8
    // (18944 x 3584 INT4, against the generic kernel: M=9 449 -> 52 us, M=16 606 -> 76,
    // M=64 2196 -> 276; 14336 x 4096 M=256 7902 -> 966); a block that does not fit (the
    // first: nothing has run) leaves the layer to the generic kernel
    if (tiled && act == LSQ_ACT_NONE && K % kTileK == 0 && M >= 1) {
      for (int64_t m0 = 0; m0 < M; m0 += 8) {
        const int64_t mb = M - m0 < 8 ? M - m0 : 8;
        LinearArgs a{static_cast<const float*>(x) + m0 * ldx, ldx, tiled, scale, scale_dt, bias, bias_dt,
                     static_cast<float*>(y) + m0 * ldy, ldy, mb, N, K, group, ng};
        const int rc = launch_gemv32(w4 ? kW4Tiled : kW8Tiled, a, s);
        if (rc == LSQ_E_LAYOUT && m0 == 0) break;
        if (rc != LSQ_OK) return rc == LSQ_E_LAYOUT ? LSQ_E_SHAPE : rc;
        if (m0 + mb == M) return LSQ_OK;
      }
    }
  }
  if (act != LSQ_ACT_NONE) return LSQ_E_LAYOUT;
  return launch_generic<DT>(w4, x, ldx, w, tiled, scale, scale_dt, group, bias, bias_dt, y, ldy, M, N,
                            K, s);
}

// ============================================================ SiLU.mul over interleaved rows

// out[m, j] = round_T(round_T(silu(g)) * u), g = in[m, 32 (j / 16) + j % 16] and
// u = in[m, 32 (j / 16) + 16 + j % 16]: the 16-row gate / up interleave of a fused
// gate / up layer (F.silu(gate_proj(x)) * up_proj(x), modeling_qwen2.py:46-48).
template <int DT>
__global__ void __launch_bounds__(256) silu_mul_kernel(const typename Act<DT>::storage* __restrict__ in,
                                                       int64_t ldi, typename Act<DT>::storage* __restrict__ out,
                                                       int64_t ldo, int64_t M, int64_t I) {
  const int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
  if (i >= M * I) return;
  const int64_t m = i / I, j = i - m * I;
  const int64_t c = 32 * (j >> 4) + (j & 15);
  const float g = Act<DT>::to_f32(in[m * ldi + c]);
  const float u = Act<DT>::to_f32(in[m * ldi + c + 16]);
  const float sg = Act<DT>::round(opaque(g / (1.f + expf(-g))));
  out[m * ldo + j] = Act<DT>::from_f32(opaque(sg * u));  // fp32 product, then round to T
}

template <int DT>
static int launch_silu_mul(const void* in, int64_t ldi, void* out, int64_t ldo, int64_t M, int64_t I,
                           hipStream_t s) {
  using S = typename Act<DT>::storage;
  const int64_t blocks = (M * I + 255) / 256;
  if (blocks > INT32_MAX) return LSQ_E_SHAPE;
  silu_mul_kernel<DT><<<dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s>>>(
      static_cast<const S*>(in), ldi, static_cast<S*>(out), ldo, M, I);
  return static_cast<int>(hipGetLastError());
}

}  // namespace lsq

using namespace lsq;

extern "C" int lsq_version(void) { return 100; }

extern "C" const char* lsq_status_string(int status) {
  switch (status) {
    case LSQ_OK: return "success";
    case LSQ_E_NULL: return "lsq: a required pointer is NULL";
    case LSQ_E_SHAPE: return "lsq: M, N or K out of range, or leading dimension smaller than the row";
    case LSQ_E_DTYPE: return "lsq: unsupported dtype code";
    case LSQ_E_GROUP: return "lsq: group_size must be >= 1";
    case LSQ_E_LAYOUT: return "lsq: the tiled weight layouts need K % 128 == 0";
    case LSQ_E_ALIGN: return "lsq: pointer or leading dimension not aligned as required";
    case LSQ_E_SCRATCH:
      return "lsq: the call needs more than the allocation-free entry point's fixed scratch "
             "(LSQ_NOALLOC_SCRATCH_BYTES); use lsq_w8a8_linear with a workspace";
    default: break;
  }
  if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
  return "lsq: unknown status";
}

static int w8_linear(const void* x, int64_t ldx, const int8_t* weight_q, const int8_t* tiled,
                     const void* scale, int scale_dtype, const void* bias, int bias_dtype, void* y,
                     int64_t ldy, int dtype, int64_t M, int64_t N, int64_t K, void* stream, int act,
                     void* ws = nullptr, int64_t ws_bytes = 0) {
  const int64_t ny = act == LSQ_ACT_SILU_MUL ? N / 2 : N;  // output columns
  const int rc = check_common(x, ldx, weight_q, tiled, scale, y, ldy, dtype, bias_dtype, bias, M, ny, K);
  if (rc != LSQ_OK) return rc;
  if (act != LSQ_ACT_NONE && (act != LSQ_ACT_SILU_MUL || N % 32 != 0)) return LSQ_E_LAYOUT;
  if (scale_dtype != LSQ_F32 && scale_dtype != LSQ_F16 && scale_dtype != LSQ_BF16) return LSQ_E_DTYPE;
  if (tiled && (reinterpret_cast<uintptr_t>(tiled) & 15)) return LSQ_E_ALIGN;
  if (tiled && K % kTileK != 0) return LSQ_E_LAYOUT;
  if (ws && ((reinterpret_cast<uintptr_t>(ws) & 15) || ws_bytes < 0)) return LSQ_E_ALIGN;
  if (M == 0 || N == 0) return LSQ_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint8_t* w = reinterpret_cast<const uint8_t*>(weight_q);
  const uint8_t* t = reinterpret_cast<const uint8_t*>(tiled);
  const int64_t group = K > 0 ? K : 1;
  switch (dtype) {
    case LSQ_F32: return dispatch<LSQ_F32>(false, x, ldx, w, t, scale, scale_dtype, group, bias, bias_dtype, y, ldy, M, N, K, s, act, ws, ws_bytes);
    case LSQ_F16: return dispatch<LSQ_F16>(false, x, ldx, w, t, scale, scale_dtype, group, bias, bias_dtype, y, ldy, M, N, K, s, act, ws, ws_bytes);
    default: return dispatch<LSQ_BF16>(false, x, ldx, w, t, scale, scale_dtype, group, bias, bias_dtype, y, ldy, M, N, K, s, act, ws, ws_bytes);
  }
}

extern "C" int lsq_w8_linear(const void* x, int64_t ldx, const int8_t* weight_q,
                             const int8_t* tiled, const void* scale, int scale_dtype,
                             const void* bias, int bias_dtype, void* y, int64_t ldy, int dtype,
                             int64_t M, int64_t N, int64_t K, void* stream) {
  return w8_linear(x, ldx, weight_q, tiled, scale, scale_dtype, bias, bias_dtype, y, ldy, dtype, M,
                   N, K, stream, LSQ_ACT_NONE);
}

extern "C" int lsq_w8_linear_ws(const void* x, int64_t ldx, const int8_t* weight_q,
                                const int8_t* tiled, const void* scale, int scale_dtype,
                                const void* bias, int bias_dtype, void* y, int64_t ldy, int dtype,
                                int64_t M, int64_t N, int64_t K, void* workspace,
                                int64_t workspace_bytes, void* stream) {
  return w8_linear(x, ldx, weight_q, tiled, scale, scale_dtype, bias, bias_dtype, y, ldy, dtype, M,
                   N, K, stream, LSQ_ACT_NONE, workspace, workspace_bytes);
}

extern "C" int lsq_w8_linear_act(const void* x, int64_t ldx, const int8_t* weight_q,
                                 const int8_t* tiled, const void* scale, int scale_dtype,
                                 const void* bias, int bias_dtype, void* y, int64_t ldy, int dtype,
                                 int64_t M, int64_t N, int64_t K, int act, void* stream) {
  return w8_linear(x, ldx, weight_q, tiled, scale, scale_dtype, bias, bias_dtype, y, ldy, dtype, M,
                   N, K, stream, act);
}

static int w4_linear(const void* x, int64_t ldx, const uint8_t* weight_packed, const uint8_t* tiled,
                     const void* scale, int scale_dtype, int64_t group_size, const void* bias,
                     int bias_dtype, void* y, int64_t ldy, int dtype, int64_t M, int64_t N, int64_t K,
                     void* stream, int act, void* ws = nullptr, int64_t ws_bytes = 0) {
  const int64_t ny = act == LSQ_ACT_SILU_MUL ? N / 2 : N;  // output columns
  const int rc = check_common(x, ldx, weight_packed, tiled, scale, y, ldy, dtype, bias_dtype, bias, M, ny, K);
  if (rc != LSQ_OK) return rc;
  if (act != LSQ_ACT_NONE && (act != LSQ_ACT_SILU_MUL || N % 32 != 0)) return LSQ_E_LAYOUT;
  if (group_size < 1) return LSQ_E_GROUP;
  if (scale_dtype != LSQ_F32 && scale_dtype != LSQ_F16 && scale_dtype != LSQ_BF16) return LSQ_E_DTYPE;
  if (tiled && (reinterpret_cast<uintptr_t>(tiled) & 15)) return LSQ_E_ALIGN;
  if (tiled && K % kTileK != 0) return LSQ_E_LAYOUT;
  if (ws && ((reinterpret_cast<uintptr_t>(ws) & 15) || ws_bytes < 0)) return LSQ_E_ALIGN;
  if (M == 0 || N == 0) return LSQ_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t group = K > 0 ? (group_size < K ? group_size : K) : 1;
  switch (dtype) {
    case LSQ_F32: return dispatch<LSQ_F32>(true, x, ldx, weight_packed, tiled, scale, scale_dtype, group, bias, bias_dtype, y, ldy, M, N, K, s, act, ws, ws_bytes);
    case LSQ_F16: return dispatch<LSQ_F16>(true, x, ldx, weight_packed, tiled, scale, scale_dtype, group, bias, bias_dtype, y, ldy, M, N, K, s, act, ws, ws_bytes);
    default: return dispatch<LSQ_BF16>(true, x, ldx, weight_packed, tiled, scale, scale_dtype, group, bias, bias_dtype, y, ldy, M, N, K, s, act, ws, ws_bytes);
  }
}

extern "C" int lsq_w4_linear(const void* x, int64_t ldx, const uint8_t* weight_packed,
                             const uint8_t* tiled, const void* scale, int scale_dtype,
                             int64_t group_size, const void* bias, int bias_dtype, void* y,
                             int64_t ldy, int dtype, int64_t M, int64_t N, int64_t K, void* stream) {
  return w4_linear(x, ldx, weight_packed, tiled, scale, scale_dtype, group_size, bias, bias_dtype, y,
                   ldy, dtype, M, N, K, stream, LSQ_ACT_NONE);
}

extern "C" int lsq_w4_linear_ws(const void* x, int64_t ldx, const uint8_t* weight_packed,
                                const uint8_t* tiled, const void* scale, int scale_dtype,
                                int64_t group_size, const void* bias, int bias_dtype, void* y,
                                int64_t ldy, int dtype, int64_t M, int64_t N, int64_t K,
                                void* workspace, int64_t workspace_bytes, void* stream) {
  return w4_linear(x, ldx, weight_packed, tiled, scale, scale_dtype, group_size, bias, bias_dtype, y,
                   ldy, dtype, M, N, K, stream, LSQ_ACT_NONE, workspace, workspace_bytes);
}

extern "C" int64_t lsq_linear_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M < 0 || N < 0 || K < 0) return 0;
  const int64_t b = std::max({gemv_split_bytes(M, N, K), bgemv_split_bytes(M, N, K), gemm_split_bytes(M, N, K)});
  return (b + 255) / 256 * 256;
}

extern "C" int lsq_w4_linear_act(const void* x, int64_t ldx, const uint8_t* weight_packed,
                                 const uint8_t* tiled, const void* scale, int scale_dtype,
                                 int64_t group_size, const void* bias, int bias_dtype, void* y,
                                 int64_t ldy, int dtype, int64_t M, int64_t N, int64_t K, int act,
                                 void* stream) {
  return w4_linear(x, ldx, weight_packed, tiled, scale, scale_dtype, group_size, bias, bias_dtype, y,
                   ldy, dtype, M, N, K, stream, act);
}

extern "C" int lsq_silu_mul(const void* in, int64_t ld_in, void* out, int64_t ld_out, int dtype,
                            int64_t M, int64_t I, void* stream) {
  if (M < 0 || I < 0 || I % 16 != 0 || ld_in < 2 * I || ld_out < I) return LSQ_E_SHAPE;
  if (dtype != LSQ_F32 && dtype != LSQ_F16 && dtype != LSQ_BF16) return LSQ_E_DTYPE;
  if (M == 0 || I == 0) return LSQ_OK;
  if (!in || !out) return LSQ_E_NULL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case LSQ_F32: return launch_silu_mul<LSQ_F32>(in, ld_in, out, ld_out, M, I, s);
    case LSQ_F16: return launch_silu_mul<LSQ_F16>(in, ld_in, out, ld_out, M, I, s);
    default: return launch_silu_mul<LSQ_BF16>(in, ld_in, out, ld_out, M, I, s);
  }
}
