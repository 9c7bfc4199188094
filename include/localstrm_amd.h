/*
 * localstrm_amd: weight-only quantized linear layer for AMD Instinct MI355X (gfx950).
 *
 * C ABI of liblsq.so. Every entry point takes plain device pointers, sizes and a
 * hipStream_t (passed as void* so this header needs no HIP include), enqueues its
 * kernels on that stream and returns without synchronizing. The return value is a
 * status: 0 on success, a negative LSQ_E* code for a rejected argument, or a positive
 * hipError_t from the launch. lsq_status_string() turns either into text.
 *
 * Shapes follow the reference's QuantizedLinear (src/kernels/quantization.py:34-149):
 *   N = out_features (weight rows), K = in_features, M = tokens (rows of x).
 *   INT8: weight_q int8 [N, K] row-major, scale [N] (the [N,1] buffer; fp32 in the
 *         reference, any of the three dtype codes after a module dtype cast).
 *   INT4: weight_packed uint8 [N, (K+1)/2] row-major; byte j of row n holds
 *         (q[n,2j]+8) | (q[n,2j+1]+8) << 4   (quantization.py:86-91);
 *         scale [N, G] in fp32 or bf16 with G = ceil(K / group_size). A group_size
 *         >= K is the reference's per-output-channel INT4 (quantization.py:80-83).
 * Activation / output dtype T is one of LSQ_F32, LSQ_F16, LSQ_BF16. Dequantization is
 * the closed form of quantization.py:106-122 evaluated in T:
 *   W[n,k] = round_T( T(q[n,k]) * round_T(scale[n, k / group_size]) )
 * and the linear layer is F.linear (quantization.py:141): y = x W^T + round_T(bias),
 * fp32 accumulation, one rounding to T at the end.
 */
#ifndef LOCALSTRM_AMD_H
#define LOCALSTRM_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes for activations, outputs, scales and bias */
#define LSQ_F32 0
#define LSQ_F16 1
#define LSQ_BF16 2
#define LSQ_I8 3               /* KV cache entries only (lsq_paged_attention_decode) */

/* epilogues of lsq_w8_linear_act / lsq_w4_linear_act */
#define LSQ_ACT_NONE 0
#define LSQ_ACT_SILU_MUL 1     /* y = silu(gate) * up over gate / up rows interleaved by 16 */

/* argument errors (negative); positive values are hipError_t */
#define LSQ_OK 0
#define LSQ_E_NULL (-1)        /* a required pointer is NULL */
#define LSQ_E_SHAPE (-2)       /* M, N or K out of range, or a leading dim < row length */
#define LSQ_E_DTYPE (-3)       /* unsupported dtype code */
#define LSQ_E_GROUP (-4)       /* group_size < 1 */
#define LSQ_E_LAYOUT (-5)      /* tiled layouts need K % 128 == 0 */
#define LSQ_E_ALIGN (-6)       /* pointer or leading dim not aligned as the kernel needs */
#define LSQ_E_SCRATCH (-7)     /* the call needs more than LSQ_NOALLOC_SCRATCH_BYTES */

/* Library version (major*10000 + minor*100 + patch). No reference counterpart. */
int lsq_version(void);

/* Text for a status code returned by any entry point. Never NULL. */
const char* lsq_status_string(int status);

/* Dequantize INT8 per-output-channel weights to dtype out_dtype.
 * Replaces QuantizedLinear.dequantize for quant_type "int8"
 * (src/kernels/quantization.py:104-108): W = weight_q.to(T) * scale.to(T). */
int lsq_dequant_w8(const int8_t* weight_q, const void* scale, int scale_dtype, void* w_out,
                   int out_dtype, int64_t N, int64_t K, void* stream);

/* Dequantize packed INT4 weights (group-wise scales) to dtype out_dtype.
 * Replaces QuantizedLinear.dequantize for quant_type "int4"
 * (src/kernels/quantization.py:109-122); group_size >= K is the reference's per-channel
 * case, smaller groups are the group-wise extension W[n,k] = q * scale[n, k/group_size]. */
int lsq_dequant_w4(const uint8_t* weight_packed, const void* scale, int scale_dtype,
                   int64_t group_size, void* w_out, int out_dtype, int64_t N, int64_t K,
                   void* stream);

/* Unpack INT4 nibbles to int8 q in [-8, 7], [N, K] row-major.
 * The integer half of quantization.py:113-121 (the `unpacked` tensor). */
int lsq_unpack_w4(const uint8_t* weight_packed, int8_t* q_out, int64_t N, int64_t K,
                  void* stream);

/* Bytes of the tiled INT4 layout for an [N, K] weight (0 if K % 128 != 0).
 * No reference counterpart: the reference keeps only the canonical layout. */
int64_t lsq_w4_tiled_bytes(int64_t N, int64_t K);

/* Re-tile canonical packed INT4 weights into the decode layout: 16-row x 128-column
 * tiles of 1024 contiguous bytes, each 64-lane wavefront load reading one tile with
 * 16 bytes per lane, nibbles ordered for the in-register bf16/fp16 unpack. Rows past N
 * are zero-filled. Derived from weight_packed as produced by
 * src/kernels/quantization.py:86-91; the canonical buffer is left untouched. */
int lsq_w4_retile(const uint8_t* weight_packed, uint8_t* tiled, int64_t N, int64_t K,
                  void* stream);

/* Inverse of lsq_w4_retile (for round-trip checks). */
int lsq_w4_untile(const uint8_t* tiled, uint8_t* weight_packed, int64_t N, int64_t K,
                  void* stream);

/* Bytes of the tiled INT8 layout for an [N, K] weight (0 if K % 128 != 0).
 * No reference counterpart: the reference keeps only the row-major weight_q. */
int64_t lsq_w8_tiled_bytes(int64_t N, int64_t K);

/* Re-tile row-major int8 weights into the decode layout: 16-row x 128-column tiles of
 * 2048 contiguous bytes (two 1 KB halves, each read by one 64-lane wavefront load with
 * 16 bytes per lane). Rows past N are zero-filled. Derived from weight_q as produced by
 * src/kernels/quantization.py:72-78; weight_q is left untouched. */
int lsq_w8_retile(const int8_t* weight_q, int8_t* tiled, int64_t N, int64_t K, void* stream);

/* Inverse of lsq_w8_retile (for round-trip checks). */
int lsq_w8_untile(const int8_t* tiled, int8_t* weight_q, int64_t N, int64_t K, void* stream);

/* y[M, N] = x[M, K] @ dequant(W8)^T + round_T(bias).
 * Replaces QuantizedLinear.forward for quant_type "int8"
 * (src/kernels/quantization.py:129-141). x and y have dtype `dtype`, row strides ldx and
 * ldy (elements); bias is NULL or [N] of bias_dtype (rounded to `dtype` first, as
 * quantization.py:135-140 casts it). `tiled` is NULL or the output of lsq_w8_retile for
 * the same weights; when given, every kernel reads it instead of weight_q, and weight_q
 * may be NULL (a module on a GPU keeps only the tiled copy). */
int lsq_w8_linear(const void* x, int64_t ldx, const int8_t* weight_q, const int8_t* tiled,
                  const void* scale, int scale_dtype, const void* bias, int bias_dtype, void* y,
                  int64_t ldy, int dtype, int64_t M, int64_t N, int64_t K, void* stream);

/* y[M, N] = x[M, K] @ dequant(W4)^T + round_T(bias).
 * Replaces QuantizedLinear.forward for quant_type "int4"
 * (src/kernels/quantization.py:129-141), extended with group-wise scales.
 * `tiled` is NULL or the output of lsq_w4_retile for the same weights; when given, every
 * kernel reads it instead of weight_packed, and weight_packed may be NULL (a module on a
 * GPU keeps only the tiled copy). */
int lsq_w4_linear(const void* x, int64_t ldx, const uint8_t* weight_packed,
                  const uint8_t* tiled, const void* scale, int scale_dtype,
                  int64_t group_size, const void* bias, int bias_dtype, void* y, int64_t ldy,
                  int dtype, int64_t M, int64_t N, int64_t K, void* stream);

/* ---- The same forwards with a caller-provided workspace ----
 * Same contract and results as lsq_w8_linear / lsq_w4_linear (the same reference lines,
 * quantization.py:129-141), plus `workspace` (device memory, 16-byte aligned, or NULL) of
 * `workspace_bytes`. With at least lsq_linear_workspace_bytes(M, N, K) bytes, decode
 * calls on down-projection-shaped layers split K over workgroups (4-16 tokens whose
 * activations exceed 96 KB on layers of at most 512 16-row tiles, e.g. 3584 x 18944;
 * 17-64 tokens on layers of at most 128 row tiles with 16+ 128-column tiles, e.g.
 * 896 x 4864), and so do prefill calls whose GEMM tiles would leave the GPU short of
 * workgroups (small N, or long K: e.g. 896 x 4864 or 3584 x 18944 at 65-256 tokens):
 * each slice's fp32 partial sums go to the workspace and a second kernel adds
 * them in slice order, adds the bias and rounds to T. With a smaller or NULL workspace
 * these calls behave exactly like the plain entry points. The workspace is scratch for
 * the duration of the call on `stream` (its contents are not read before being written). */
int64_t lsq_linear_workspace_bytes(int64_t M, int64_t N, int64_t K);
int lsq_w8_linear_ws(const void* x, int64_t ldx, const int8_t* weight_q, const int8_t* tiled,
                     const void* scale, int scale_dtype, const void* bias, int bias_dtype, void* y,
                     int64_t ldy, int dtype, int64_t M, int64_t N, int64_t K, void* workspace,
                     int64_t workspace_bytes, void* stream);
int lsq_w4_linear_ws(const void* x, int64_t ldx, const uint8_t* weight_packed,
                     const uint8_t* tiled, const void* scale, int scale_dtype,
                     int64_t group_size, const void* bias, int bias_dtype, void* y, int64_t ldy,
                     int dtype, int64_t M, int64_t N, int64_t K, void* workspace,
                     int64_t workspace_bytes, void* stream);

/* ---- Fused gate / up with the SiLU.mul epilogue ----
 * The MLP of the reference's decoder layers computes down_proj(silu(gate_proj(x)) *
 * up_proj(x)) (modeling_qwen2.py:46-48), two launches and two elementwise kernels. No
 * reference counterpart for these entry points: they serve a gate / up pair fused into one
 * weight whose rows alternate 16 gate rows and the 16 up rows of the same outputs (row
 * tile 2t = gate rows 16t..16t+15, tile 2t+1 = up rows 16t..16t+15), N = 2 * I rows,
 * N % 32 == 0. With act = LSQ_ACT_SILU_MUL, y is [M, I] (row stride ldy >= I) and
 *   y[m, j] = round_T( round_T(silu(g)) * u ),  g, u = the two layers' outputs in T
 * (each as lsq_w8_linear / lsq_w4_linear computes it). The fused epilogue runs in the
 * decode kernel (fp16 / bf16, M <= 64, K % 128 == 0, x in LDS); other shapes return
 * LSQ_E_LAYOUT without launching anything: run the plain entry point on the interleaved
 * weight and lsq_silu_mul on its output. act = LSQ_ACT_NONE is the plain entry point. */
int lsq_w8_linear_act(const void* x, int64_t ldx, const int8_t* weight_q, const int8_t* tiled,
                      const void* scale, int scale_dtype, const void* bias, int bias_dtype,
                      void* y, int64_t ldy, int dtype, int64_t M, int64_t N, int64_t K, int act,
                      void* stream);
int lsq_w4_linear_act(const void* x, int64_t ldx, const uint8_t* weight_packed,
                      const uint8_t* tiled, const void* scale, int scale_dtype,
                      int64_t group_size, const void* bias, int bias_dtype, void* y, int64_t ldy,
                      int dtype, int64_t M, int64_t N, int64_t K, int act, void* stream);

/* out[m, j] = round_T(round_T(silu(g)) * u) from the interleaved output in [M, 2 I] (row
 * stride ld_in) of a fused gate / up layer: g = in[m, 32 (j/16) + j%16], u the element 16
 * further. I % 16 == 0. No reference counterpart (F.silu(gate) * up, modeling_qwen2.py:48). */
int lsq_silu_mul(const void* in, int64_t ld_in, void* out, int64_t ld_out, int dtype, int64_t M,
                 int64_t I, void* stream);

/* ---- W8A8: Int8GEMMLinear (the MLP layers of the reference's 'hybrid_int8' mode) ----
 * Weights: weight_q_t int8 [K, N] (N contiguous) and scale_w_t [N] (fp32 in the
 * reference, any dtype code after a module cast), as Int8GEMMLinear stores them
 * (src/kernels/quantization.py:309-319, from_float :326-353). Activations are quantized per token:
 *   scale_x[m] = clamp(round_T(max_k |x[m,k]| * fp32(1/127)), min = round_T(1e-8))
 *   x_q[m,k]   = clamp(rint(fp32(x[m,k]) / scale_x[m]), -128, 127)     (NaN -> 0)
 * (quantization.py:411-414; torch evaluates the division by the Python scalar 127 on the
 * GPU as a product with the fp32 reciprocal) and the output is
 *   y[m,n] = round_T( fp32(sum_k x_q[m,k] * w[k,n]) * (scale_x[m] * scale_w[n]) + fp32(bias[n]) )
 * with every product and sum one fp32 rounding (quantization.py:425-447): bit-exact. */

/* Bytes of the W8A8 tiled weight layout: the tiled INT8 layout of the [N, K] weight with
 * K padded to a multiple of 128 by zero columns. No reference counterpart. */
int64_t lsq_w8a8_tiled_bytes(int64_t N, int64_t K);

/* Re-tile weight_q_t [K, N] (the layout torch._int_mm consumes, quantization.py:309-313)
 * into the W8A8 tiled layout. No reference counterpart; weight_q_t is left untouched. */
int lsq_w8a8_retile(const int8_t* weight_q_t, int8_t* tiled, int64_t N, int64_t K, void* stream);

/* Inverse of lsq_w8a8_retile (for round-trip checks). */
int lsq_w8a8_untile(const int8_t* tiled, int8_t* weight_q_t, int64_t N, int64_t K, void* stream);

/* Per-token activation quantization of x [M, K] (dtype `dtype`, row stride ldx elements)
 * into x_q [M, ldq] int8 and scale_x [M] fp32. Replaces quantization.py:411-414. Columns
 * K .. min(ldq, round_up(K, 128)) - 1 of x_q are set to 0. */
int lsq_act_quant_i8(const void* x, int64_t ldx, int dtype, int64_t M, int64_t K, int8_t* x_q,
                     int64_t ldq, float* scale_x, void* stream);

/* y [M, N] (dtype `dtype`, row stride ldy) = W8A8 linear of x [M, K] (same dtype, row
 * stride ldx). Replaces Int8GEMMLinear.forward's native path, quantization.py:404-447
 * (activation quantization, torch._int_mm, rescale, bias, cast). `tiled` is the output of
 * lsq_w8a8_retile; bias is NULL or [N] of bias_dtype. x_q [M, round_up(K, 128)] int8
 * (16-byte aligned) and scale_x [M] fp32 are the caller's workspace for the quantized
 * activations and their scales; decode-sized calls quantize inside the GEMV kernel and
 * leave them untouched, so their contents afterwards are unspecified (lsq_act_quant_i8
 * computes them on their own). 1 <= K < 131072. */
int lsq_w8a8_linear(const void* x, int64_t ldx, const int8_t* tiled, const void* scale_w,
                    int scale_w_dtype, const void* bias, int bias_dtype, void* y, int64_t ldy,
                    int dtype, int64_t M, int64_t N, int64_t K, int8_t* x_q, float* scale_x,
                    void* stream);

/* lsq_w8a8_linear with a caller-provided workspace (the same reference lines,
 * quantization.py:404-447, and the same result bit for bit): `workspace` (device memory,
 * 16-byte aligned, or NULL) of `workspace_bytes`. With at least
 * lsq_w8a8_workspace_bytes(M, N, K) bytes, calls whose int8 GEMM would leave the GPU short
 * of workgroups on a long K (fewer than 128 output tiles of 64 x 128, up to 192 tokens, or
 * of 256 x 256 above, with 2048+ columns: e.g. 3584 x 18944 at any M up to ~2048) split K
 * over workgroups; each slice's int32
 * sums go to the workspace and a second kernel adds them (exact), rescales, adds the bias
 * and rounds to T, as the unsplit GEMM does. Such calls then also take the GEMM below 17
 * tokens when x_q does not fit the decode kernel. With a smaller or NULL workspace they
 * behave exactly like lsq_w8a8_linear. The workspace is scratch for the duration of the
 * call on `stream`. lsq_w8a8_workspace_bytes is 0 for shapes that never split. */
int64_t lsq_w8a8_workspace_bytes(int64_t M, int64_t N, int64_t K);
int lsq_w8a8_linear_ws(const void* x, int64_t ldx, const int8_t* tiled, const void* scale_w,
                       int scale_w_dtype, const void* bias, int bias_dtype, void* y, int64_t ldy,
                       int dtype, int64_t M, int64_t N, int64_t K, int8_t* x_q, float* scale_x,
                       void* workspace, int64_t workspace_bytes, void* stream);

/* Bytes of the fixed device array behind lsq_w8a8_linear_noalloc, one per GPU. */
#define LSQ_NOALLOC_SCRATCH_BYTES (8 * 1024 * 1024)

/* lsq_w8a8_linear without the x_q / scale_x workspace: the same kernels and the same
 * result bit for bit, with the quantized activations staged in a fixed device array of
 * LSQ_NOALLOC_SCRATCH_BYTES that the library holds on each GPU it runs on until the
 * process ends. No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc); it calls no hipMalloc / hipFree. The first call on a device resolves that
 * device's copy of the array (hipGetSymbolAddress; the device is the stream's). Limit:
 * round_up(M * round_up(K, 128), 256) + 4 * M <= LSQ_NOALLOC_SCRATCH_BYTES (M <= 2046 at
 * K = 4096), else LSQ_E_SCRATCH before any HIP call. Calls that overlap on one GPU (other
 * streams, other threads) share the array and race: serialize them. */
int lsq_w8a8_linear_noalloc(const void* x, int64_t ldx, const int8_t* tiled, const void* scale_w,
                            int scale_w_dtype, const void* bias, int bias_dtype, void* y,
                            int64_t ldy, int dtype, int64_t M, int64_t N, int64_t K, void* stream);

/* ---- Paged attention for one decode step (INT8 or T-typed KV cache) ----
 * Replaces paged_attention_decode (src/kernels/paged_attention.py:33-173) for a query of
 * one token per sequence: query [B, H, D] (the reference's [B, H, 1, D]), k_pool / v_pool
 * [num_blocks, block_size, Hkv, D] of kv_dtype (LSQ_I8 with k_scales / v_scales
 * [num_blocks, block_size, Hkv] of scale_dtype, or the query's dtype with NULL scales),
 * block_tables int64 [B, >= ceil(max_seq_len / block_size)] (row stride bt_stride),
 * seq_lens int64 [B]. A table entry e < 0 stands for block e + num_blocks (Python
 * indexing, as the reference's gather k_cache_pool[sub_tables]); an entry outside
 * [-num_blocks, num_blocks) masks its token (the reference's gather would raise
 * IndexError there). A token t of sequence b attends when its entry is in range,
 * t < max_seq_len and, without a mask, t < seq_lens[b]; with a mask (bool bytes, row stride mask_stride, one row per
 * sequence or, mask_rows_per_b = Hkv, one per (sequence, KV head) as the reference's
 * repeat_interleave'd mask), when mask[row][t]. head_mapping 0: query head h uses KV head
 * h / (H / Hkv) ("contiguous"); 1: h % Hkv ("interleaved"). Keys / values are dequantized
 * as round_T(k * scale) (the reference's keys.to(T) * k_scales), scores scaled by
 * 1 / sqrt(D), softmax and the value sum in fp32, out [B, H, D] rounded once to T.
 * H / Hkv <= 16, D in {64, 128} (an fp32 cache: 64), num_blocks * block_size * Hkv < 2^31.
 * workspace: lsq_paged_attention_workspace_bytes(...)
 * bytes of device memory (0 when max_seq_len <= 256; then it may be NULL). */
int64_t lsq_paged_attention_workspace_bytes(int64_t B, int64_t H, int64_t D, int64_t max_seq_len);
int lsq_paged_attention_decode(const void* query, const void* k_pool, const void* v_pool,
                               int kv_dtype, const void* k_scales, const void* v_scales,
                               int scale_dtype, const int64_t* block_tables, int64_t bt_stride,
                               const int64_t* seq_lens, const uint8_t* mask, int64_t mask_stride,
                               int64_t mask_rows_per_b, void* out, int dtype, int64_t B,
                               int64_t H, int64_t Hkv, int64_t D, int64_t block_size,
                               int64_t num_blocks, int64_t max_seq_len, int head_mapping,
                               void* workspace, int64_t workspace_bytes, void* stream);

/* ---- Weight quantization on the GPU ----
 * Replace the CPU quantization of QuantizedLinear.from_float / Int8GEMMLinear.from_float
 * (src/kernels/quantization.py:72-94, :341-344; the loader stages it at :593-610) for
 * weights already in device memory, with the same fp32 steps and results bit for bit:
 * scale = max(max|w| / qmax, fp32(1e-8)) per row (qmax 127 / 7; IEEE division), q =
 * clamp(rint(w / scale), qmin, qmax) (IEEE division, round half to even). w [N, K] is
 * f32 / f16 / bf16 with row stride ldw elements. Writes the canonical layout, the tiled
 * layout (16-byte aligned, K % 128 == 0), or both; NULL skips one, not both. Rows holding
 * NaN or infinities give unspecified q (as the reference's float -> int8 cast of NaN). */

/* INT8 per channel: scale [N] fp32, weight_q [N, K] int8, tiled as lsq_w8_retile writes
 * it (which is also the W8A8 tiled layout at K % 128 == 0). */
int lsq_quantize_w8(const void* w, int w_dtype, int64_t ldw, int64_t N, int64_t K, float* scale,
                    int8_t* weight_q, int8_t* tiled, void* stream);

/* INT4: group_size 0 or >= K is the reference's per-channel INT4 (scale [N] fp32,
 * scale_dtype must be LSQ_F32); 1 <= group_size < K quantizes each group of group_size
 * columns against its scale rounded to scale_dtype (stored [N, ceil(K / group_size)]).
 * weight_packed [N, ceil(K/2)] (low nibble = even column), tiled as lsq_w4_retile writes
 * it (group_size a multiple of 8 there). */
int lsq_quantize_w4(const void* w, int w_dtype, int64_t ldw, int64_t N, int64_t K, int64_t group_size,
                    void* scale, int scale_dtype, uint8_t* weight_packed, uint8_t* tiled, void* stream);

/* ---- Measurement floors (no reference counterpart; for benchmarks) ----
 * lsq_probe_empty launches one empty workgroup: the cost of a launch itself.
 * lsq_probe_read streams `bytes` (1 .. 2^31 - 1) of `buf` once with 16-byte loads and
 * computes nothing: `grid` workgroups of `block` threads (64..1024, a multiple of 64), each
 * reading a contiguous share with 4 loads in flight per lane, write grid * 64 floats to
 * `sink` (so the loads are kept). Its time is a floor for any kernel that must stream the
 * same bytes in one launch on this device. */
int lsq_probe_empty(void* stream);
int lsq_probe_read(const void* buf, int64_t bytes, float* sink, int grid, int block, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LOCALSTRM_AMD_H */
