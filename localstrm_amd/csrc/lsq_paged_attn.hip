// Paged attention for one decode step, with an INT8 or T-typed KV cache (gfx950).
//
// GPU form of paged_attention_decode (src/kernels/paged_attention.py:33-173): one query
// token per sequence attends to its cached keys / values, which live in fixed-size blocks
// of a shared pool found through the sequence's block table. The reference gathers every
// block into a contiguous copy, dequantizes it (keys.to(T) * scales), expands the GQA
// heads and calls F.scaled_dot_product_attention. Here nothing is copied:
//
//  * paged_attn_i8_kernel (INT8 cache, fp16 / bf16 queries; the default there): one
//    workgroup per (sequence, KV head, split of one or more chunks) whose 4 or 8 waves
//    each take 64 tokens of a 256- or 512-token chunk with an online softmax of their own
//    (no barrier until the end); scores and P x V on the MFMA with the probabilities used
//    where the scores leave them and the values read transposed out of LDS
//    (ds_read_b64_tr_b8); keys and values dequantized in registers; described at the
//    kernel;
//  * paged_attn_mfma_kernel (fp16 / bf16 queries with a T cache, or LSQ_PAGED_KERNEL=mfma):
//    one workgroup per (sequence, KV head, split), the chunk's scores, softmax and P x V
//    shared by its four waves through LDS, an online softmax across the split's chunks,
//    each chunk's loads issued while the previous one finishes; described at the kernel;
//  * paged_attn_split_kernel (fp32, or LSQ_PAGED_KERNEL=valu): one workgroup per
//    (sequence, KV head, split of 256 tokens);
//    thread t takes token t of the split: it walks the block table to the token's row,
//    dequantizes its key (round_T(k * scale)) and forms the scores of all G query heads
//    that share this KV head (q of the G heads in LDS); softmax statistics per head over
//    the split; then lane d of each wave accumulates p * v for 64 of the split's tokens
//    (value rows read coalesced, one row per token), the four waves' partials added in
//    LDS. One split writes the normalized output; several write (max, sum, partial
//    output) to the caller's workspace;
//  * paged_attn_combine_kernel: rescales and adds the splits of each (sequence, head).
// Every key / value byte (plus its scale) is read once per step; at decode sizes the time
// is set by each workgroup's chain of dependent loads and barriers more than by bandwidth.
//
// Numerics: scores and softmax in fp32 with the SDPA default scale 1 / sqrt(D), the
// value sum in fp32, one rounding to T at the end; keys and values are the T-valued
// dequantized entries, as the reference feeds them to SDPA.

#include "lsq_common.h"
#include "lsq_mfma16.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <type_traits>

namespace lsq {
namespace {

constexpr int kPaNT = 256;   // threads per workgroup = tokens per split
constexpr int kPaMaxG = 16;  // query heads per KV head

struct PagedArgs {
  const void* q;          // [B, H, D] (dtype DT)
  const void* kp;         // [NB, BS, Hkv, D] int8 or DT
  const void* vp;
  const void* ks;         // [NB, BS, Hkv] scales (int8 cache only)
  const void* vs;
  int scale_dt;
  const int64_t* bt;      // block tables, row stride ldbt
  int64_t ldbt;
  int64_t nb;             // blocks in the pools: a table entry outside [-nb, nb) masks its token
  const int64_t* sl;      // sequence lengths [B]
  const uint8_t* mask;    // optional boolean mask rows (row stride ldm), else sl decides
  int64_t ldm;
  int mask_rows_per_b;    // 1 or Hkv (a mask repeated per KV head)
  void* out;              // [B, H, D] (dtype DT)
  float* ws;              // [B, H, nsplit, D + 2] partials when nsplit > 1
  int B, H, Hkv, G, BS, nsplit, max_sl, interleaved;
  int cps;                // chunks per split (kPaNT tokens, 512 for the 8-wave kernel; VALU kernel: 1)
  int bs_m16;             // ceil(2^16 / BS) for BS < 64 (block / slot of a token, wave kernel)
  float sm_scale;
};

// Dequantized key / value element e of a 16-byte chunk (int8: 16 elements, T: 8), as T.
template <int DT, bool I8>
__device__ __forceinline__ float kv_elem(u32x4 v, int e, float s) {
  if constexpr (I8) {
    const int q = static_cast<int8_t>(v[e >> 2] >> (8 * (e & 3)));
    return Act<DT>::round(opaque(static_cast<float>(q) * s));
  } else if constexpr (DT == LSQ_F32) {
    return __uint_as_float(v[e]);
  } else {
    return Act<DT>::to_f32(static_cast<uint16_t>(v[e >> 1] >> (16 * (e & 1))));
  }
}

// The aligned dword holding scale i (fp32, or 16-bit f16 / bf16) of a per-row scale
// array, loaded without branching on the dtype so that several such loads are in flight
// together (a load inside a dtype branch is waited for before the branch ends); convert
// with dword_elem(w, scale_half(dt, i), dt). A 16-bit element's dword never crosses a page.
__device__ __forceinline__ uint32_t load_scale_word(const void* p, int dt, int64_t i) {
  const int64_t off = dt == LSQ_F32 ? 4 * i : 2 * i;
  return *reinterpret_cast<const uint32_t*>(static_cast<const unsigned char*>(p) + (off & ~int64_t(3)));
}
__device__ __forceinline__ int scale_half(int dt, int64_t i) { return dt == LSQ_F32 ? 0 : static_cast<int>(i & 1); }

// Max / sum of a float over each row of 16 lanes, in every lane of the row (DPP).
__device__ __forceinline__ float dpp_f(float v, int ctrl) {
  switch (ctrl) {
    case 0: return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
    case 1: return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
    case 2: return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
    default: return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
  }
}
__device__ __forceinline__ float row16_max(float v) {
#pragma unroll
  for (int c = 0; c < 4; ++c) v = fmaxf(v, dpp_f(v, c));
  return v;
}
__device__ __forceinline__ float row16_sum(float v) {
#pragma unroll
  for (int c = 0; c < 4; ++c) v += dpp_f(v, c);
  return v;
}

template <int DT, bool I8, int D>
__global__ void __launch_bounds__(kPaNT) paged_attn_split_kernel(PagedArgs p) {
  using S = typename Act<DT>::storage;
  constexpr int ESZ = I8 ? 1 : static_cast<int>(sizeof(S));  // bytes per cache element
  constexpr int EPC = 16 / ESZ;                              // elements per 16-byte chunk
  constexpr int kVtLd = kPaNT + 16;                          // transposed tile row (bytes)
  __shared__ __align__(16) float qs[kPaMaxG * D];
  __shared__ __align__(16) float sp[kPaMaxG * kPaNT];
  __shared__ float stat[2 * kPaMaxG];  // per head: max, sum
  __shared__ __align__(16) float vsc[kPaNT];
  __shared__ __align__(16) unsigned char tile[D * kVtLd * ESZ];  // values, vt[d][token]
  __shared__ __align__(16) float accs[4 * kPaMaxG * D];           // per-wave partial outputs

  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int G = p.G;
  auto head = [&](int g) { return p.interleaved ? g * p.Hkv + kvh : kvh * G + g; };
  const S* q = static_cast<const S*>(p.q);
  for (int i = tid; i < G * D; i += kPaNT) {
    const int g = i / D, d = i - (i / D) * D;
    qs[i] = Act<DT>::to_f32(q[(static_cast<int64_t>(b) * p.H + head(g)) * D + d]);
  }
  const int seq = static_cast<int>(p.sl[b]);
  auto valid_tok = [&](int t) -> bool {
    if (t >= p.max_sl) return false;
    if (p.mask) {
      const int row = b * p.mask_rows_per_b + (p.mask_rows_per_b > 1 ? kvh : 0);
      return p.mask[static_cast<int64_t>(row) * p.ldm + t] != 0;
    }
    return t < seq;
  };

  // ---- this thread's token: pool row (-1: masked), key and value rows. Loads are
  // unconditional (a masked token reads row 0, its results are discarded) so that they
  // are all in flight together.
  const int t0 = split * kPaNT;
  const int t = t0 + tid;
  // The block table entry is read for every token below max_seq_len (the table holds
  // ceil(max_seq_len / block_size) entries per sequence), so its load does not wait for
  // the sequence length; only valid tokens use it.
  int64_t blk = t < p.max_sl ? p.bt[static_cast<int64_t>(b) * p.ldbt + t / p.BS] : 0;
  if (blk < 0) blk += p.nb;  // a negative entry counts from the end, as Python indexing does
  const bool valid = valid_tok(t) && blk >= 0 && blk < p.nb;
  int my_row = -1;
  if (valid) my_row = static_cast<int>((blk * p.BS + t % p.BS) * p.Hkv + kvh);
  const int64_t lrow = my_row < 0 ? 0 : my_row;
  const uint32_t ksw = I8 ? load_scale_word(p.ks, p.scale_dt, lrow) : 0u;
  const uint32_t vsw = I8 ? load_scale_word(p.vs, p.scale_dt, lrow) : 0u;
  u32x4 kraw[D / EPC], vraw[D / EPC];
  {
    const unsigned char* kr = static_cast<const unsigned char*>(p.kp) + lrow * D * ESZ;
    const unsigned char* vr = static_cast<const unsigned char*>(p.vp) + lrow * D * ESZ;
#pragma unroll
    for (int c = 0; c < D / EPC; ++c) kraw[c] = *reinterpret_cast<const u32x4*>(kr + c * 16);
#pragma unroll
    for (int c = 0; c < D / EPC; ++c) vraw[c] = *reinterpret_cast<const u32x4*>(vr + c * 16);
  }
  const float ks = I8 ? dword_elem(ksw, scale_half(p.scale_dt, lrow), p.scale_dt) : 1.f;
  const float vs = I8 ? dword_elem(vsw, scale_half(p.scale_dt, lrow), p.scale_dt) : 1.f;
  // value row -> transposed tile (elements as stored), scale (0 for a masked token)
#pragma unroll
  for (int c = 0; c < D / EPC; ++c)
#pragma unroll
    for (int e = 0; e < EPC; ++e) {
      const int d = c * EPC + e;
      if constexpr (I8)
        tile[d * kVtLd + tid] = static_cast<unsigned char>(vraw[c][e >> 2] >> (8 * (e & 3)));
      else if constexpr (ESZ == 4)
        reinterpret_cast<uint32_t*>(tile)[d * kVtLd + tid] = vraw[c][e];
      else
        reinterpret_cast<uint16_t*>(tile)[d * kVtLd + tid] =
            static_cast<uint16_t>(vraw[c][e >> 1] >> (16 * (e & 1)));
    }
  vsc[tid] = my_row < 0 ? 0.f : vs;
  __syncthreads();

  // ---- scores: the key, dequantized once to T-valued floats, against each head's q
  constexpr float kNegInf = -__builtin_huge_valf();
#pragma unroll
  for (int h0 = 0; h0 < D; h0 += 64) {  // 64 dimensions at a time (registers)
    float kf[64];
#pragma unroll
    for (int e = 0; e < 64; ++e) {
      const int d = h0 + e;
      const u32x4 w = kraw[d / EPC];
      const int ee = d % EPC;
      if constexpr (I8) {
        const int qv = static_cast<int8_t>(w[ee >> 2] >> (8 * (ee & 3)));
        kf[e] = Act<DT>::round(opaque(static_cast<float>(qv) * ks));
      } else if constexpr (DT == LSQ_F32) {
        kf[e] = __uint_as_float(w[ee]);
      } else {
        kf[e] = Act<DT>::to_f32(static_cast<uint16_t>(w[ee >> 1] >> (16 * (ee & 1))));
      }
    }
    for (int g = 0; g < G; ++g) {
      float dot = 0.f;
#pragma unroll
      for (int e = 0; e < 64; e += 4) {
        const f32x4 qv = *reinterpret_cast<const f32x4*>(&qs[g * D + h0 + e]);
        dot = fmaf(qv[0], kf[e], fmaf(qv[1], kf[e + 1], fmaf(qv[2], kf[e + 2], fmaf(qv[3], kf[e + 3], dot))));
      }
      float* dst = &sp[g * kPaNT + tid];
      if (h0 + 64 < D) *dst = (h0 == 0 ? 0.f : *dst) + dot;
      else *dst = valid ? ((h0 == 0 ? 0.f : *dst) + dot) * p.sm_scale : kNegInf;
    }
  }

  // ---- softmax statistics per head over the split: thread (g = tid / 16, part = tid % 16)
  // reduces 16 of head g's 256 scores from LDS, then the 16 parts by DPP within a row
  __syncthreads();
  const int hg = tid >> 4, part = tid & 15;
  if (hg < G) {
    float m = kNegInf;
#pragma unroll
    for (int e = 0; e < 16; e += 4) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(&sp[hg * kPaNT + part * 16 + e]);
      m = fmaxf(fmaxf(m, fmaxf(v[0], v[1])), fmaxf(v[2], v[3]));
    }
    m = row16_max(m);
    if (part == 0) stat[hg] = m;
  }
  __syncthreads();
  for (int g = 0; g < G; ++g) {
    const float sv = sp[g * kPaNT + tid];
    sp[g * kPaNT + tid] = sv == kNegInf ? 0.f : __expf(sv - stat[g]);  // all masked: m = -inf
  }
  __syncthreads();
  if (hg < G) {
    float l = 0.f;
#pragma unroll
    for (int e = 0; e < 16; e += 4) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(&sp[hg * kPaNT + part * 16 + e]);
      l += (v[0] + v[1]) + (v[2] + v[3]);
    }
    l = row16_sum(l);
    if (part == 0) stat[kPaMaxG + hg] = l;
  }

  // ---- p * v: wave w takes tokens [64 w, 64 w + 64), lane d (then d + 64) one dimension;
  // the 64 values of the lane's dimension come from the transposed tile, 16 bytes a read
  const int tw = wid * 64;
#pragma unroll
  for (int j = 0; j < D / 64; ++j) {
    const int d = lane + 64 * j;
    float vv[64];
#pragma unroll
    for (int c = 0; c < 64 * ESZ / 16; ++c) {
      const u32x4 w = *reinterpret_cast<const u32x4*>(&tile[(d * kVtLd + tw) * ESZ + c * 16]);
#pragma unroll
      for (int e = 0; e < 16 / ESZ; ++e) {
        const int tt = c * (16 / ESZ) + e;
        float v;
        if constexpr (I8) {
          const int qv = static_cast<int8_t>(w[e >> 2] >> (8 * (e & 3)));
          v = Act<DT>::round(opaque(static_cast<float>(qv) * vsc[tw + tt]));
        } else if constexpr (DT == LSQ_F32) {
          v = __uint_as_float(w[e]);  // (fp32 caches are staged 4 bytes an element)
        } else {
          v = Act<DT>::to_f32(static_cast<uint16_t>(w[e >> 1] >> (16 * (e & 1))));
        }
        vv[tt] = vsc[tw + tt] == 0.f ? 0.f : v;  // masked token: its row may hold anything
      }
    }
    for (int g = 0; g < G; ++g) {
      float a = 0.f;
#pragma unroll
      for (int e = 0; e < 64; e += 4) {
        const f32x4 pg = *reinterpret_cast<const f32x4*>(&sp[g * kPaNT + tw + e]);
        a = fmaf(pg[0], vv[e], fmaf(pg[1], vv[e + 1], fmaf(pg[2], vv[e + 2], fmaf(pg[3], vv[e + 3], a))));
      }
      accs[(wid * kPaMaxG + g) * D + d] = a;
    }
  }
  __syncthreads();

  for (int i = tid; i < G * D; i += kPaNT) {
    const int g = i / D, d = i - (i / D) * D;
    const float a = (accs[(0 * kPaMaxG + g) * D + d] + accs[(1 * kPaMaxG + g) * D + d]) +
                    (accs[(2 * kPaMaxG + g) * D + d] + accs[(3 * kPaMaxG + g) * D + d]);
    const float m = stat[g], l = stat[kPaMaxG + g];
    const int64_t oh = static_cast<int64_t>(b) * p.H + head(g);
    if (p.nsplit == 1) {
      static_cast<S*>(p.out)[oh * D + d] = Act<DT>::from_f32(opaque(a / l));
    } else {
      float* w = p.ws + (oh * p.nsplit + split) * (D + 2);
      if (d == 0) { w[0] = m; w[1] = l; }
      w[2 + d] = a;
    }
  }
}


// fp16 / bf16 queries on v_mfma_f32_16x16x32 (the G heads padded to the 16 rows of the
// MFMA). A workgroup takes p.cps consecutive chunks of 256 tokens. Per chunk, scores:
// A = q (row = head), B = the dequantized keys of 16 tokens (column = token); lane l of
// wave w owns token 64 w + 16 tt + (l & 15) of the chunk for tt = 0..3 and dims
// 32 j + 8 (l >> 4) .. +7 of it, which it loads, dequantizes to T and packs as the B
// operand, and whose value bytes it writes into the transposed tile. Value sum: A = the
// probabilities rounded to T (as flash-attention kernels feed P to the second product),
// B = 8 consecutive tokens' values of one dim from the transposed tile, accumulated in
// registers across chunks with the running max / sum of an online softmax (the partial
// sums rescaled by e^(m_old - m_new) per head).
template <int DT, bool I8, int D>
__global__ void __launch_bounds__(kPaNT) paged_attn_mfma_kernel(PagedArgs p) {
  using S = typename Act<DT>::storage;
  constexpr int ESZ = I8 ? 1 : 2;
  constexpr int kQLd = D + 8;        // q rows (T elements), padded against bank conflicts
  constexpr int kSpLd = kPaNT + 4;   // score / probability rows (floats)
  constexpr int kVtLd = kPaNT + 16 / ESZ;  // transposed value rows (elements)
  __shared__ __align__(16) uint16_t qs[16 * kQLd];
  __shared__ __align__(16) float sp[16 * kSpLd];
  __shared__ float stat[3 * 16];     // per head: running max, running sum, rescale factor
  __shared__ __align__(16) float vsc[kPaNT];
  __shared__ __align__(16) unsigned char tile[D * kVtLd * ESZ];
  __shared__ __align__(16) float accs[4 * kPaMaxG * D];

  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int r16 = lane & 15, q4 = lane >> 4;
  const int G = p.G;
  auto head = [&](int g) { return p.interleaved ? g * p.Hkv + kvh : kvh * G + g; };
  const S* q = static_cast<const S*>(p.q);
  for (int i = tid; i < 16 * D; i += kPaNT) {
    const int g = i / D, d = i - (i / D) * D;
    qs[g * kQLd + d] = g < G ? q[(static_cast<int64_t>(b) * p.H + head(g)) * D + d] : uint16_t(0);
  }
  if (tid < 16) {
    stat[tid] = -__builtin_huge_valf();
    stat[16 + tid] = 0.f;
    stat[32 + tid] = 0.f;
  }
  const int seq = static_cast<int>(p.sl[b]);

  // This workgroup's chunks of kPaNT tokens: [c_lo, c_hi). Each chunk is loaded while the
  // previous one finishes: its block-table entries one chunk ahead, its keys, values and
  // scales as soon as the previous chunk's are consumed (after its scores and value
  // tile), so the softmax and value sum of a chunk overlap the next chunk's loads.
  const int nchunk = (p.max_sl + kPaNT - 1) / kPaNT;
  const int c_lo = split * p.cps;
  const int c_hi = min(c_lo + p.cps, nchunk);
  auto tok = [&](int c, int tt) { return c * kPaNT + wid * 64 + tt * 16 + r16; };
  // Block-table entries are read for every token below max_seq_len (the table holds
  // ceil(max_seq_len / block_size) entries per sequence): these loads do not wait for
  // the sequence length, and only valid tokens use them.
  // The loads are unconditional (tokens past max_seq_len read the last column, and are
  // masked later): a load under a per-lane condition makes the compiler wait for it at
  // the end of the condition. An entry outside [-nb, nb) becomes -1 (its token is masked);
  // a negative one counts from the end, as Python indexing does.
  auto load_bt = [&](int c, int64_t (&blk)[4]) {
    if (c < c_hi) {  // uniform; then max_seq_len > 0
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const int t = min(tok(c, tt), p.max_sl - 1);
        blk[tt] = p.bt[static_cast<int64_t>(b) * p.ldbt + t / p.BS];
      }
    }
  };
  auto block_of = [&](int64_t e) -> int {
    const int64_t i = e < 0 ? e + p.nb : e;
    return (i >= 0 && i < p.nb) ? static_cast<int>(i) : -1;
  };
  using Chunk = typename std::conditional<I8, uint2, u32x4>::type;  // 8 elements
  Chunk kc[4][D / 32], vc[4][D / 32];
  uint32_t ksw[4], vsw[4];  // raw scale words, converted when the chunk is used
  int shalf[4];
  bool val[4];
  // Keys, values and scales of the lane's 4 tokens of chunk c (a masked token, or a chunk
  // past the last, reads row 0 and its results are discarded).
  // No load here sits inside a data-dependent branch, so all of them are in flight
  // together (mask bytes first, then rows, scales, keys and values).
  auto load_kv = [&](int c, const int64_t (&blk)[4]) {
    const bool live = c < c_hi;
    unsigned char mk[4] = {1, 1, 1, 1};
    if (p.mask && live) {  // uniform; a mask row holds max_seq_len entries
      const int64_t mrow = static_cast<int64_t>(b * p.mask_rows_per_b + (p.mask_rows_per_b > 1 ? kvh : 0)) * p.ldm;
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) mk[tt] = p.mask[mrow + min(tok(c, tt), p.max_sl - 1)];
    }
    int row[4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const int t = tok(c, tt);
      const int bi = block_of(blk[tt]);
      val[tt] = live && t < p.max_sl && (p.mask ? mk[tt] != 0 : t < seq) && bi >= 0;
      row[tt] = val[tt] ? (bi * p.BS + t % p.BS) * p.Hkv + kvh : 0;
    }
    if constexpr (I8) {
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        ksw[tt] = load_scale_word(p.ks, p.scale_dt, row[tt]);
        vsw[tt] = load_scale_word(p.vs, p.scale_dt, row[tt]);
        shalf[tt] = scale_half(p.scale_dt, row[tt]);
      }
    }
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const unsigned char* kr = static_cast<const unsigned char*>(p.kp) + static_cast<int64_t>(row[tt]) * D * ESZ;
      const unsigned char* vr = static_cast<const unsigned char*>(p.vp) + static_cast<int64_t>(row[tt]) * D * ESZ;
#pragma unroll
      for (int j = 0; j < D / 32; ++j) {
        kc[tt][j] = *reinterpret_cast<const Chunk*>(kr + (32 * j + 8 * q4) * ESZ);
        vc[tt][j] = *reinterpret_cast<const Chunk*>(vr + (32 * j + 8 * q4) * ESZ);
      }
    }
  };
  int64_t blk_next[4] = {0, 0, 0, 0};
  load_bt(c_lo, blk_next);
  load_kv(c_lo, blk_next);
  load_bt(c_lo + 1, blk_next);

  constexpr float kNegInf = -__builtin_huge_valf();
  f32x4 oacc[D / 16];
#pragma unroll
  for (int dt = 0; dt < D / 16; ++dt) oacc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  __syncthreads();  // q rows and the running statistics are in LDS
  u32x4 qa[D / 32];
#pragma unroll
  for (int j = 0; j < D / 32; ++j) qa[j] = *reinterpret_cast<const u32x4*>(&qs[r16 * kQLd + 32 * j + 8 * q4]);
  const int hg = tid >> 4, part = tid & 15;

  for (int c = c_lo; c < c_hi; ++c) {
    float ksc[4], vscl[4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      ksc[tt] = I8 ? dword_elem(ksw[tt], shalf[tt], p.scale_dt) : 1.f;
      vscl[tt] = I8 ? dword_elem(vsw[tt], shalf[tt], p.scale_dt) : 1.f;
    }
    // ---- values -> transposed tile (a masked token's values as 0), scales
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const int tl = wid * 64 + tt * 16 + r16;
#pragma unroll
      for (int j = 0; j < D / 32; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int d = 32 * j + 8 * q4 + e;
          if constexpr (I8) {
            const uint32_t w = e < 4 ? vc[tt][j].x : vc[tt][j].y;
            tile[d * kVtLd + tl] = val[tt] ? static_cast<unsigned char>(w >> (8 * (e & 3))) : 0;
          } else {
            const uint32_t w = vc[tt][j][e >> 1];
            reinterpret_cast<uint16_t*>(tile)[d * kVtLd + tl] = val[tt] ? static_cast<uint16_t>(w >> (16 * (e & 1))) : 0;
          }
        }
      if (q4 == 0) vsc[tl] = val[tt] ? vscl[tt] : 0.f;
    }
    // ---- scores on the MFMA: A = q rows (head r16, dims 32 j + 8 q4 ..), B = keys
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < D / 32; ++j) {
        u32x4 kb;
        if constexpr (I8) {
          float kf[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const uint32_t w = e < 4 ? kc[tt][j].x : kc[tt][j].y;
            kf[e] = Act<DT>::round(opaque(static_cast<float>(static_cast<int8_t>(w >> (8 * (e & 3)))) * ksc[tt]));
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) kb[e] = Mma<DT>::pack2(kf[2 * e], kf[2 * e + 1]);
        } else {
          kb = kc[tt][j];
        }
        acc = Mma<DT>::mma(qa[j], kb, acc);
      }
      const int tl = wid * 64 + tt * 16 + r16;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int g = 4 * q4 + e;
        if (g < G) sp[g * kSpLd + tl] = val[tt] ? acc[e] * p.sm_scale : kNegInf;
      }
    }
    // ---- the next chunk's loads (registers free now), then its table entries' refill
    if (c + 1 < c_hi) {  // uniform
      load_kv(c + 1, blk_next);
      load_bt(c + 2, blk_next);  // (the loads above already hold their row offsets)
    }
    __syncthreads();

    // ---- online softmax per head (16 threads a head, DPP row reductions): new running
    // max, factor rescaling what was summed so far, exp, running sum
    if (hg < G) {
      float m = kNegInf;
#pragma unroll
      for (int e = 0; e < 16; e += 4) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(&sp[hg * kSpLd + part * 16 + e]);
        m = fmaxf(fmaxf(m, fmaxf(v[0], v[1])), fmaxf(v[2], v[3]));
      }
      m = row16_max(m);
      if (part == 0) {
        const float mo = stat[hg];
        const float mn = fmaxf(mo, m);
        stat[32 + hg] = mo == kNegInf ? 0.f : __expf(mo - mn);
        stat[hg] = mn;
      }
    }
    __syncthreads();
    for (int g = 0; g < G; ++g) {
      const float sv = sp[g * kSpLd + tid];
      sp[g * kSpLd + tid] = sv == kNegInf ? 0.f : __expf(sv - stat[g]);
    }
    __syncthreads();
    if (hg < G) {
      float l = 0.f;
#pragma unroll
      for (int e = 0; e < 16; e += 4) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(&sp[hg * kSpLd + part * 16 + e]);
        l += (v[0] + v[1]) + (v[2] + v[3]);
      }
      l = row16_sum(l);
      if (part == 0) stat[16 + hg] = fmaf(stat[16 + hg], stat[32 + hg], l);
    }

    // ---- value sum on the MFMA: wave w over its 64 tokens in 2 steps of 32, into the
    // running sums rescaled to the new max (rows g >= G hold nothing used)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float f = stat[32 + ((4 * q4 + e) & 15)];
#pragma unroll
      for (int dt = 0; dt < D / 16; ++dt) oacc[dt][e] *= f;
    }
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const int tb = wid * 64 + st * 32 + 8 * q4;  // the lane's 8 tokens
      u32x4 pa;
      {
        const f32x4 p0 = *reinterpret_cast<const f32x4*>(&sp[r16 * kSpLd + tb]);
        const f32x4 p1 = *reinterpret_cast<const f32x4*>(&sp[r16 * kSpLd + tb + 4]);
        pa[0] = Mma<DT>::pack2(p0[0], p0[1]);
        pa[1] = Mma<DT>::pack2(p0[2], p0[3]);
        pa[2] = Mma<DT>::pack2(p1[0], p1[1]);
        pa[3] = Mma<DT>::pack2(p1[2], p1[3]);
      }
      float sc8[8];
      if constexpr (I8) {
        const f32x4 s0 = *reinterpret_cast<const f32x4*>(&vsc[tb]);
        const f32x4 s1 = *reinterpret_cast<const f32x4*>(&vsc[tb + 4]);
#pragma unroll
        for (int e = 0; e < 4; ++e) { sc8[e] = s0[e]; sc8[4 + e] = s1[e]; }
      }
#pragma unroll
      for (int dt = 0; dt < D / 16; ++dt) {
        const int d = 16 * dt + r16;
        u32x4 vb;
        if constexpr (I8) {
          const uint2 w = *reinterpret_cast<const uint2*>(&tile[d * kVtLd + tb]);
          float vf[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const uint32_t ww = e < 4 ? w.x : w.y;
            vf[e] = Act<DT>::round(opaque(static_cast<float>(static_cast<int8_t>(ww >> (8 * (e & 3)))) * sc8[e]));
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) vb[e] = Mma<DT>::pack2(vf[2 * e], vf[2 * e + 1]);
        } else {
          vb = *reinterpret_cast<const u32x4*>(&reinterpret_cast<const uint16_t*>(tile)[d * kVtLd + tb]);
        }
        oacc[dt] = Mma<DT>::mma(pa, vb, oacc[dt]);
      }
    }
    __syncthreads();  // the tile, scales and probabilities are free for the next chunk
  }

#pragma unroll
  for (int dt = 0; dt < D / 16; ++dt)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int g = 4 * q4 + e;
      if (g < G) accs[(wid * kPaMaxG + g) * D + 16 * dt + r16] = oacc[dt][e];
    }
  __syncthreads();

  for (int i = tid; i < G * D; i += kPaNT) {
    const int g = i / D, d = i - (i / D) * D;
    const float a = (accs[(0 * kPaMaxG + g) * D + d] + accs[(1 * kPaMaxG + g) * D + d]) +
                    (accs[(2 * kPaMaxG + g) * D + d] + accs[(3 * kPaMaxG + g) * D + d]);
    const float m = stat[g], l = stat[16 + g];
    const int64_t oh = static_cast<int64_t>(b) * p.H + head(g);
    if (p.nsplit == 1) {
      static_cast<S*>(p.out)[oh * D + d] = Act<DT>::from_f32(opaque(a / l));
    } else {
      float* w = p.ws + (oh * p.nsplit + split) * (D + 2);
      if (d == 0) { w[0] = m; w[1] = l; }
      w[2 + d] = a;
    }
  }
}

// ---------------------------------------------------------------------------------------
// INT8 KV cache, fp16 / bf16 queries (the default for that cache): waves that work on
// their own. Wave w of a workgroup of NW (4 or 8) takes tokens 64 w .. 64 w + 63 of each
// 64 NW-token chunk of the split (four 16-token tiles) with an online softmax of its own,
// so the waves meet once, at the end, where their (max, sum, partial output) are merged in
// LDS.
//  * Scores as S^T = K q^T on v_mfma_f32_16x16x32: A = the dequantized keys of a tile
//    (row = token; lane l loads D / 4 contiguous bytes of token l & 15, so one k step of
//    the product takes dims D / 4 (l >> 4) + 8 s .. +7, and q is loaded in the same
//    order), B = q^T (column = head, zero past G). A lane then holds the scores of one
//    head (l & 15) for tokens 4 (l >> 4) .. +3 of each tile: the running max and sum are
//    per lane, the max shared by a head's 4 lanes through two shuffles.
//  * Value sum as O^T = V^T P^T: B = the probabilities where the scores left them (k
//    index 8 G + e of a 32-token step is token 4 G + e of its first tile for e < 4 and
//    16 + 4 G + e - 4 of its second, G = l >> 4), A = the values of those tokens for 16
//    dims. The wave stores its values in LDS as loaded (a token's bytes per lane) and
//    reads them back transposed with ds_read_b64_tr_b8, which hands lane 16 G + 8 h + j
//    byte j of the 8-byte rows addressed by lanes 16 G + h + 2 i, i = 0..7. O^T leaves a
//    lane with one head's outputs, so rescaling by e^(m_old - m_new) is per lane too.
//  * Dequantization in registers: byte b ^ 0x80 placed under the fp16 exponent of 1024
//    (v_perm) is exactly 1024 + 128 + k; minus 1152 gives k; times an fp16 scale rounds
//    once (v_pk_mul_f16), which is round_T(k * s), the reference's keys.to(T) * scales.
//    Other scale / query types go through fp32 as in the kernels above.
//  * Loads: a chunk's block-table entries one chunk ahead, its keys, values and scales
//    while the previous chunk's softmax and value sum run.
constexpr int kI8Tok = 64;  // tokens per wave and chunk (4 tiles of 16)

// Row stride (bytes) of a wave's value tile in LDS.
__host__ __device__ constexpr int i8_vld(int d) { return d + 16; }

typedef _Float16 f16x2v __attribute__((ext_vector_type(2)));

// 8 int8 (two dwords) -> 8 fp16 values k exactly, as 4 packed pairs (element e of the
// result = byte e).
__device__ __forceinline__ void i8x8_to_f16(uint32_t w0, uint32_t w1, f16x2v (&h)[4]) {
  const uint32_t u0 = w0 ^ 0x80808080u, u1 = w1 ^ 0x80808080u;
  const f16x2v off = {static_cast<_Float16>(1152.f), static_cast<_Float16>(1152.f)};
  h[0] = __builtin_bit_cast(f16x2v, __builtin_amdgcn_perm(u0, 0x64646464u, 0x00050004u)) - off;
  h[1] = __builtin_bit_cast(f16x2v, __builtin_amdgcn_perm(u0, 0x64646464u, 0x00070006u)) - off;
  h[2] = __builtin_bit_cast(f16x2v, __builtin_amdgcn_perm(u1, 0x64646464u, 0x00050004u)) - off;
  h[3] = __builtin_bit_cast(f16x2v, __builtin_amdgcn_perm(u1, 0x64646464u, 0x00070006u)) - off;
}

// Two fp32 values -> packed T pair, round to nearest even.
template <int DT>
__device__ __forceinline__ uint32_t pack_rne(float a, float b) {
  if constexpr (DT == LSQ_F16) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, f16x2v));
  } else {
    return Mma<LSQ_BF16>::pack2(a, b);
  }
}

// Operand of 8 dequantized elements round_T(k_e * s_e). FAST: T = fp16 with fp16 scales
// (s2[j] = the scales of elements 2 j, 2 j + 1 as an fp16 pair); otherwise sf[e] in fp32.
template <int DT, bool FAST>
__device__ __forceinline__ u32x4 i8x8_dequant(uint32_t w0, uint32_t w1, const f16x2v (&s2)[4], const float (&sf)[8]) {
  f16x2v h[4];
  i8x8_to_f16(w0, w1, h);
  u32x4 r;
  if constexpr (FAST) {
#pragma unroll
    for (int j = 0; j < 4; ++j) r[j] = __builtin_bit_cast(uint32_t, h[j] * s2[j]);
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      r[j] = pack_rne<DT>(opaque(static_cast<float>(h[j][0]) * sf[2 * j]), opaque(static_cast<float>(h[j][1]) * sf[2 * j + 1]));
  }
  return r;
}

template <int DT, int D, bool FAST, int NW>
__global__ void __launch_bounds__(64 * NW) paged_attn_i8_kernel(PagedArgs p) {
  constexpr int KB = D / 4;          // bytes of a token row per lane
  constexpr int NL = KB / 16;        // 16-byte loads per lane per token (1 or 2)
  constexpr int KS = D / 32;         // k steps of the score product
  constexpr int DTL = D / 16;        // 16-dim tiles of the value sum
  constexpr int VLD = i8_vld(D);
  constexpr float kNegInf = -__builtin_huge_valf();
  constexpr float kLog2e = 1.4426950408889634f;
  constexpr int NT = 64 * NW;        // threads
  constexpr int CH = NW * kI8Tok;    // tokens per chunk
  using S = typename Act<DT>::storage;
  __shared__ __align__(16) unsigned char vt[NW * kI8Tok * VLD];  // values; merge sums after
  __shared__ __align__(16) float vsc[NW * kI8Tok];               // value scales (0: invalid)
  __shared__ __align__(16) unsigned char vok[NW * kI8Tok];       // token valid
  __shared__ float ml[NW * 16 * 2];                              // per wave and head: max, sum
  static_assert(NW * kI8Tok * VLD >= NW * 16 * D * 4, "merge sums alias the value tiles");

  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int r16 = lane & 15, q4 = lane >> 4;
  const int G = p.G;
  auto head = [&](int g) { return p.interleaved ? g * p.Hkv + kvh : kvh * G + g; };
  unsigned char* vtw = vt + wid * kI8Tok * VLD;
  float* vscw = vsc + wid * kI8Tok;
  unsigned char* vokw = vok + wid * kI8Tok;

  // q^T operand: lane (head r16, group q4), k step s -> q[head][KB q4 + 8 s .. +7]
  u32x4 qb[KS];
  {
    const bool hv = r16 < G;
    const S* qrow = static_cast<const S*>(p.q) + (static_cast<int64_t>(b) * p.H + head(hv ? r16 : 0)) * D + KB * q4;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(qrow + 8 * s);
      qb[s] = hv ? v : u32x4{0u, 0u, 0u, 0u};
    }
  }
  const int seq = static_cast<int>(p.sl[b]);
  const int nchunk = (p.max_sl + CH - 1) / CH;
  const int c_lo = split * p.cps;
  const int c_hi = min(c_lo + p.cps, nchunk);
  // tokens below `lim` may be attended (a mask decides among them); the table holds
  // ceil(max_seq_len / block_size) entries per sequence, read for every token below
  // max_seq_len (later tokens read the last one and are masked)
  const int lim = p.mask ? p.max_sl : min(p.max_sl, seq);
  const int qmax = p.max_sl > 0 ? (p.max_sl - 1) / p.BS : 0;
  const int BS = p.BS;
  const int64_t* btrow = p.bt + static_cast<int64_t>(b) * p.ldbt;

  // Block-table entry and in-block slot of token T0 + 16 tt + r16 (T0 = this wave's first
  // token of chunk c): one uniform division per chunk, then per lane a wrap (BS >= 64) or
  // a multiply-high by ceil(2^16 / BS) (exact: remainders stay below 64 + BS).
  int64_t blk[4] = {0, 0, 0, 0};
  int slot[4] = {0, 0, 0, 0}, slot_n[4] = {0, 0, 0, 0};
  auto load_bt = [&](int c, int (&sl_out)[4]) {
    if (c < c_hi) {  // uniform; then max_seq_len > 0
      const int T0 = c * CH + wid * kI8Tok;
      const int qb0 = T0 / BS, rb0 = T0 - qb0 * BS;
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const int rm = rb0 + 16 * tt + r16;
        int qa;
        if (BS >= 64) qa = rm >= BS ? 1 : 0;
        else qa = static_cast<int>((static_cast<uint32_t>(rm) * static_cast<uint32_t>(p.bs_m16)) >> 16);
        sl_out[tt] = rm - qa * BS;
        blk[tt] = btrow[min(qb0 + qa, qmax)];
      }
    }
  };
  auto block_of = [&](int64_t e) -> int {
    const int64_t i = e < 0 ? e + p.nb : e;
    return (i >= 0 && i < p.nb) ? static_cast<int>(i) : -1;
  };
  u32x4 kr[4][NL], vr[4][NL];
  uint32_t ksw[4], vsw[4];
  int shalf[4];
  bool val[4];
  const int es_s = p.scale_dt == LSQ_F32 ? 4 : 2;
  // Keys, values and scales of tiles 2 h, 2 h + 1 of chunk c (an invalid token, or a
  // chunk past the last, reads row 0; its results are discarded). Branch-free except
  // for the (uniform) mask, so the compiler's waits for them are exact.
  // the mask row (a mask row holds max_seq_len entries), or without a mask a byte that is
  // always there (the first table entry), so that the load needs no branch
  const bool usem = p.mask != nullptr;
  const unsigned char* mrow = usem ? p.mask + static_cast<int64_t>(b * p.mask_rows_per_b + (p.mask_rows_per_b > 1 ? kvh : 0)) * p.ldm
                                   : reinterpret_cast<const unsigned char*>(p.bt);
  auto load_half = [&](int c, int h) {  // (c < c_hi: then max_seq_len > 0)
    const int T0 = c * CH + wid * kI8Tok;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int tt = 2 * h + u;
      const int t = T0 + 16 * tt + r16;
      const bool mok = mrow[usem ? min(t, p.max_sl - 1) : 0] != 0 || !usem;
      const int bi = block_of(blk[tt]);
      // the row does not wait for the mask byte: a masked token reads its own row
      const bool in = t < lim && bi >= 0;
      val[tt] = in && mok;
      const int row = in ? (bi * BS + slot[tt]) * p.Hkv + kvh : 0;
      const int64_t so = (static_cast<int64_t>(row) * es_s) & ~int64_t(3);
      ksw[tt] = *reinterpret_cast<const uint32_t*>(static_cast<const unsigned char*>(p.ks) + so);
      vsw[tt] = *reinterpret_cast<const uint32_t*>(static_cast<const unsigned char*>(p.vs) + so);
      shalf[tt] = scale_half(p.scale_dt, row);
      const int64_t ro = static_cast<int64_t>(row) * D + KB * q4;
#pragma unroll
      for (int i = 0; i < NL; ++i) {
        kr[tt][i] = *reinterpret_cast<const u32x4*>(static_cast<const unsigned char*>(p.kp) + ro + 16 * i);
        vr[tt][i] = *reinterpret_cast<const u32x4*>(static_cast<const unsigned char*>(p.vp) + ro + 16 * i);
      }
    }
  };
  if (c_lo < c_hi) {  // uniform
    load_bt(c_lo, slot);
    load_half(c_lo, 0);
    load_half(c_lo, 1);
    load_bt(c_lo + 1, slot_n);
  }

  const float c2 = p.sm_scale * kLog2e;  // scores in the log2 domain
  float m_run = kNegInf, l_run = 0.f;
  f32x4 ot[DTL];
#pragma unroll
  for (int t = 0; t < DTL; ++t) ot[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  // ds_read_b64_tr_b8 source row / column of this lane: token pi(q4, i) of a 32-token
  // step (i = (lane & 15) >> 1), dims 8 (lane & 1) .. +7 of a 16-dim tile
  const int tr_i = r16 >> 1;
  const int tr_row = tr_i < 4 ? 4 * q4 + tr_i : 16 + 4 * q4 + tr_i - 4;
  const int tr_col = 8 * (lane & 1);

  for (int c = c_lo; c < c_hi; ++c) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      // ---- values of tiles 2 h, 2 h + 1 (as loaded), their scales and validity into LDS
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int tt = 2 * h + u;
        const int tl = tt * 16 + r16;
#pragma unroll
        for (int i = 0; i < NL; ++i) *reinterpret_cast<u32x4*>(vtw + tl * VLD + KB * q4 + 16 * i) = vr[tt][i];
        if (q4 == 0) {
          vscw[tl] = val[tt] ? dword_elem(vsw[tt], shalf[tt], p.scale_dt) : 0.f;
          vokw[tl] = val[tt] ? 1 : 0;
        }
      }
      // ---- scores S^T of the two tiles: A = keys (token r16), B = q^T
      f32x4 sc[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int tt = 2 * h + u;
        const float ks = dword_elem(ksw[tt], shalf[tt], p.scale_dt);
        f16x2v s2[4];
        float sf[8];
        if constexpr (FAST) {
          const _Float16 kh = static_cast<_Float16>(ks);  // exact: an fp16 scale
#pragma unroll
          for (int j = 0; j < 4; ++j) s2[j] = f16x2v{kh, kh};
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) sf[e] = ks;
        }
        sc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const int i = (8 * s) / 16, o = ((8 * s) % 16) / 4;  // dwords o, o + 1 of load i
          const u32x4 a = i8x8_dequant<DT, FAST>(kr[tt][i][o], kr[tt][i][o + 1], s2, sf);
          sc[u] = Mma<DT>::mma(a, qb[s], sc[u]);
        }
      }
      // ---- this half's registers are free: the next chunk's loads for them
      if (c + 1 < c_hi) {  // uniform
        if (h == 0) {
#pragma unroll
          for (int tt = 0; tt < 4; ++tt) slot[tt] = slot_n[tt];
        }
        load_half(c + 1, h);
        if (h == 1) load_bt(c + 2, slot_n);
      }
      // ---- online softmax of head r16 over this lane's 8 tokens of the two tiles
      float cmax = kNegInf;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const uint32_t ok = *reinterpret_cast<const uint32_t*>(vokw + (2 * h + u) * 16 + 4 * q4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sc[u][e] = ((ok >> (8 * e)) & 0xFF) ? sc[u][e] * c2 : kNegInf;
          cmax = fmaxf(cmax, sc[u][e]);
        }
      }
      cmax = fmaxf(cmax, __shfl_xor(cmax, 16));
      cmax = fmaxf(cmax, __shfl_xor(cmax, 32));
      const float m_new = fmaxf(m_run, cmax);
      const float msub = m_new == kNegInf ? 0.f : m_new;  // (an all-invalid run: every p is 0)
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) sc[u][e] = __builtin_amdgcn_exp2f(sc[u][e] - msub);
      const float lsum = (sc[0][0] + sc[0][1]) + (sc[0][2] + sc[0][3]) + ((sc[1][0] + sc[1][1]) + (sc[1][2] + sc[1][3]));
      const float f = __builtin_amdgcn_exp2f(m_run - msub);  // 0 while m_run is -inf
      l_run = fmaf(l_run, f, lsum);
#pragma unroll
      for (int t = 0; t < DTL; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) ot[t][e] *= f;
      m_run = m_new;
      // ---- value sum O^T += V^T P^T over the half's 32 tokens
      u32x4 pb;
      pb[0] = pack_rne<DT>(sc[0][0], sc[0][1]);
      pb[1] = pack_rne<DT>(sc[0][2], sc[0][3]);
      pb[2] = pack_rne<DT>(sc[1][0], sc[1][1]);
      pb[3] = pack_rne<DT>(sc[1][2], sc[1][3]);
      // scales of the step's tokens pi(q4, 0..7)
      const f32x4 s0 = *reinterpret_cast<const f32x4*>(vscw + 32 * h + 4 * q4);
      const f32x4 s1 = *reinterpret_cast<const f32x4*>(vscw + 32 * h + 16 + 4 * q4);
      float sf[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
      f16x2v s2[4];
      if constexpr (FAST) {
#pragma unroll
        for (int j = 0; j < 4; ++j) s2[j] = f16x2v{static_cast<_Float16>(sf[2 * j]), static_cast<_Float16>(sf[2 * j + 1])};
      }
      const unsigned char* src = vtw + (32 * h + tr_row) * VLD + tr_col;
#pragma unroll
      for (int t = 0; t < DTL; ++t) {
        typedef int v2i __attribute__((ext_vector_type(2)));
        const v2i raw = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
            (__attribute__((address_space(3))) v2i*)(src + 16 * t));
        const u32x4 a = i8x8_dequant<DT, FAST>(static_cast<uint32_t>(raw[0]), static_cast<uint32_t>(raw[1]), s2, sf);
        ot[t] = Mma<DT>::mma(a, pb, ot[t]);
      }
    }
  }

  // ---- merge the waves: sum of the head over its 4 lanes, then (max, sum, O^T) in LDS
  l_run += __shfl_xor(l_run, 16);
  l_run += __shfl_xor(l_run, 32);
  __syncthreads();  // every wave is done with its value tile (the sums alias them)
  float* accs = reinterpret_cast<float*>(vt);  // [wave][head][D]
#pragma unroll
  for (int t = 0; t < DTL; ++t)
#pragma unroll
    for (int e = 0; e < 4; ++e) accs[(wid * 16 + r16) * D + 16 * t + 4 * q4 + e] = ot[t][e];
  if (q4 == 0) {
    ml[(wid * 16 + r16) * 2] = m_run;
    ml[(wid * 16 + r16) * 2 + 1] = l_run;
  }
  __syncthreads();
  for (int i = tid; i < G * D; i += NT) {
    const int g = i / D, d = i - (i / D) * D;
    float M = kNegInf;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, ml[(w * 16 + g) * 2]);
    const float Ms = M == kNegInf ? 0.f : M;
    float a = 0.f, l = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float fw = __builtin_amdgcn_exp2f(ml[(w * 16 + g) * 2] - Ms);  // 0 for an empty wave
      a = fmaf(fw, accs[(w * 16 + g) * D + d], a);
      l = fmaf(fw, ml[(w * 16 + g) * 2 + 1], l);
    }
    const int64_t oh = static_cast<int64_t>(b) * p.H + head(g);
    if (p.nsplit == 1) {
      static_cast<S*>(p.out)[oh * D + d] = Act<DT>::from_f32(opaque(a / l));
    } else {
      // the combine kernel works in the natural-log domain
      float* w = p.ws + (oh * p.nsplit + split) * (D + 2);
      if (d == 0) { w[0] = M == kNegInf ? M : M / kLog2e; w[1] = l; }
      w[2 + d] = a;
    }
  }
}

// One workgroup of D threads per (sequence, head): out = sum_s e^(m_s - M) acc_s /
// sum_s e^(m_s - M) l_s over the splits. (A ticket in the split kernel would save this
// launch, but the device-scope release / acquire it needs writes back and invalidates
// each XCD's L2 per workgroup, which measured 3.5 x slower.)
template <int DT, int D>
__global__ void __launch_bounds__(D) paged_attn_combine_kernel(PagedArgs p) {
  using S = typename Act<DT>::storage;
  const int64_t oh = blockIdx.x;
  const int d = threadIdx.x;
  const float* w = p.ws + oh * p.nsplit * (D + 2);
  constexpr float kNegInf = -__builtin_huge_valf();
  // splits in batches of 8 whose loads are all in flight before any is used
  constexpr int kB = 8;
  float M = kNegInf, a = 0.f, l = 0.f;
  for (int s0 = 0; s0 < p.nsplit; s0 += kB) {
    float ms[kB], ls[kB], as[kB];
#pragma unroll
    for (int u = 0; u < kB; ++u) {
      const int sp_ = s0 + u < p.nsplit ? s0 + u : s0;  // past the end: a repeat, skipped
      ms[u] = w[sp_ * (D + 2)];
      ls[u] = w[sp_ * (D + 2) + 1];
      as[u] = w[sp_ * (D + 2) + 2 + d];
    }
    float Mb = M;
#pragma unroll
    for (int u = 0; u < kB; ++u)
      if (s0 + u < p.nsplit) Mb = fmaxf(Mb, ms[u]);
    // rescale what was summed so far to the new running max
    const float r = (M == kNegInf || Mb == kNegInf) ? 0.f : __expf(M - Mb);
    a *= r;
    l *= r;
#pragma unroll
    for (int u = 0; u < kB; ++u) {
      if (s0 + u < p.nsplit) {
        const float f = ms[u] == kNegInf ? 0.f : __expf(ms[u] - Mb);
        l = fmaf(f, ls[u], l);
        a = fmaf(f, as[u], a);
      }
    }
    M = Mb;
  }
  static_cast<S*>(p.out)[oh * D + d] = Act<DT>::from_f32(opaque(a / l));
}

// LSQ_PAGED_KERNEL=valu runs the VALU split kernel for fp16 / bf16 too, =mfma the
// block-wide MFMA kernel for an INT8 cache too (comparisons).
bool paged_valu() {
  const char* e = std::getenv("LSQ_PAGED_KERNEL");
  return e && e[0] == 'v';
}
bool paged_block_mfma() {
  const char* e = std::getenv("LSQ_PAGED_KERNEL");
  return e && e[0] == 'm';
}

// Chunks of kPaNT tokens per workgroup of the MFMA kernel (each split loops over its
// chunks with the next chunk's loads in flight). Measured on the Qwen2.5-0.5B attention
// shapes: one chunk per workgroup is fastest up to ~768 (sequence, KV head, chunk)
// triples, since the per-workgroup chain of dependent loads and barriers is what takes
// the time; beyond that, or past 16 splits per sequence (the merge kernel then walks many
// partials), two or more. LSQ_PAGED_CHUNKS=n forces n chunks per split (tuning).
int paged_chunks_per_split(int64_t pairs, int nchunk) {
  const char* e = std::getenv("LSQ_PAGED_CHUNKS");
  const int forced = e ? std::atoi(e) : 0;
  int64_t cps = forced > 0 ? forced : 1;
  if (forced <= 0) {
    const int64_t work = pairs * nchunk;
    cps = std::max<int64_t>((work + 767) / 768, (nchunk + 15) / 16);
  }
  return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(cps, nchunk)));
}

// Waves per workgroup of the INT8 wave-wise kernel. At ~150 VGPRs a CU holds three
// 4-wave workgroups (256-token chunks) but one 8-wave workgroup (512-token chunks, two per
// split: 1024 tokens per workgroup). 8 waves when their grid G8 (pairs x ceil(max_sl /
// 1024)) fills one round of 256 CUs nearly or exactly (192 < G8 <= 256), or when it needs
// at most two rounds while the 4-wave grid (`grid4`) needs more than one round of 768.
// Measured per layer (us, 4 -> 8 waves): batch 64 x 2048 tokens 20.7 -> 19.6, 128 x 1024
// 20.4 -> 16.6, 16 x 8192 22.3 -> 19.7, 256 x 1024 38.7 -> 31.2; outside the rule 8 waves
// lost (128 x 2048 31.1 -> 34.1, 256 x 512 17.3 -> 21.2, 32 x 2048 14.8 -> 16.5).
// LSQ_PAGED_WAVES=4|8 forces one (tuning, tests).
int paged_i8_waves(int64_t pairs, int max_sl, int64_t grid4) {
  const char* e = std::getenv("LSQ_PAGED_WAVES");
  if (e && (std::atoi(e) == 4 || std::atoi(e) == 8)) return std::atoi(e);
  const int64_t g8 = pairs * ((max_sl + 1023) / 1024);
  return (g8 > 192 && g8 <= 256) || (g8 <= 512 && grid4 > 768) ? 8 : 4;
}

template <int DT, bool I8, int D>
int launch_paged(const PagedArgs& a0, hipStream_t s) {
  PagedArgs a = a0;
  const bool mfma = DT != LSQ_F32 && !paged_valu();
  // INT8 cache: the wave-wise kernel (its q operand is read 16 bytes at a time)
  const bool waves = DT != LSQ_F32 && I8 && mfma && !paged_block_mfma() && (reinterpret_cast<uintptr_t>(a.q) & 15) == 0;
  const int64_t pairs = int64_t(a.B) * a.Hkv;
  const int nchunk4 = a.max_sl > 0 ? (a.max_sl + kPaNT - 1) / kPaNT : 1;
  const int cps4 = mfma ? paged_chunks_per_split(pairs, nchunk4) : 1;
  const int nw = waves ? paged_i8_waves(pairs, a.max_sl, pairs * ((nchunk4 + cps4 - 1) / cps4)) : 4;
  if (nw == 8) {
    const int nchunk = a.max_sl > 0 ? (a.max_sl + 511) / 512 : 1;
    const char* ce = std::getenv("LSQ_PAGED_CHUNKS");  // (forced: n chunks per split)
    a.cps = ce && std::atoi(ce) > 0 ? std::min(std::atoi(ce), nchunk) : std::min(2, nchunk);
    a.nsplit = (nchunk + a.cps - 1) / a.cps;
  } else {
    a.cps = cps4;
    a.nsplit = (nchunk4 + cps4 - 1) / cps4;
  }
  const dim3 grid(static_cast<unsigned>(a.nsplit), static_cast<unsigned>(a.Hkv), static_cast<unsigned>(a.B));
  if constexpr (DT != LSQ_F32) {
    const bool fast = DT == LSQ_F16 && a.scale_dt == LSQ_F16;
    if (waves && nw == 8) {
      if (fast) paged_attn_i8_kernel<DT, D, true, 8><<<grid, dim3(512), 0, s>>>(a);
      else paged_attn_i8_kernel<DT, D, false, 8><<<grid, dim3(512), 0, s>>>(a);
    } else if (waves) {
      if (fast) paged_attn_i8_kernel<DT, D, true, 4><<<grid, dim3(256), 0, s>>>(a);
      else paged_attn_i8_kernel<DT, D, false, 4><<<grid, dim3(256), 0, s>>>(a);
    } else if (mfma) {
      paged_attn_mfma_kernel<DT, I8, D><<<grid, dim3(kPaNT), 0, s>>>(a);
    } else {
      paged_attn_split_kernel<DT, I8, D><<<grid, dim3(kPaNT), 0, s>>>(a);
    }
  } else {
    paged_attn_split_kernel<DT, I8, D><<<grid, dim3(kPaNT), 0, s>>>(a);
  }
  if (a.nsplit > 1)
    paged_attn_combine_kernel<DT, D><<<dim3(static_cast<unsigned>(a.B * a.H)), dim3(D), 0, s>>>(a);
  return static_cast<int>(hipGetLastError());
}

template <int DT>
int launch_paged_dt(const PagedArgs& a, bool i8, int D, hipStream_t s) {
  if (D == 64) return i8 ? launch_paged<DT, true, 64>(a, s) : launch_paged<DT, false, 64>(a, s);
  if constexpr (DT == LSQ_F32) {  // an fp32 value tile of 256 x 128 does not fit in LDS
    if (!i8) return LSQ_E_SHAPE;
    return launch_paged<DT, true, 128>(a, s);
  } else {
    return i8 ? launch_paged<DT, true, 128>(a, s) : launch_paged<DT, false, 128>(a, s);
  }
}

}  // namespace
}  // namespace lsq

using namespace lsq;

extern "C" int64_t lsq_paged_attention_workspace_bytes(int64_t B, int64_t H, int64_t D, int64_t max_seq_len) {
  if (B <= 0 || H <= 0 || D <= 0 || max_seq_len <= 0) return 0;
  const int64_t nsplit = (max_seq_len + kPaNT - 1) / kPaNT;
  return nsplit > 1 ? B * H * nsplit * (D + 2) * static_cast<int64_t>(sizeof(float)) : 0;
}

extern "C" int lsq_paged_attention_decode(
    const void* query, const void* k_pool, const void* v_pool, int kv_dtype, const void* k_scales,
    const void* v_scales, int scale_dtype, const int64_t* block_tables, int64_t bt_stride,
    const int64_t* seq_lens, const uint8_t* mask, int64_t mask_stride, int64_t mask_rows_per_b,
    void* out, int dtype, int64_t B, int64_t H, int64_t Hkv, int64_t D, int64_t block_size,
    int64_t num_blocks, int64_t max_seq_len, int head_mapping, void* workspace, int64_t workspace_bytes,
    void* stream) {
  const bool dt_ok = dtype == LSQ_F32 || dtype == LSQ_F16 || dtype == LSQ_BF16;
  const bool i8 = kv_dtype == LSQ_I8;
  if (!dt_ok || (!i8 && kv_dtype != dtype)) return LSQ_E_DTYPE;
  if (i8 && scale_dtype != LSQ_F32 && scale_dtype != LSQ_F16 && scale_dtype != LSQ_BF16) return LSQ_E_DTYPE;
  if (B < 0 || H < 1 || Hkv < 1 || H % Hkv != 0 || H / Hkv > kPaMaxG || (D != 64 && D != 128) ||
      block_size < 1 || num_blocks < 0 || max_seq_len < 0 ||
      bt_stride < (max_seq_len + block_size - 1) / block_size)
    return LSQ_E_SHAPE;
  // pool rows (block, slot, KV head) are addressed with 32 bits
  if (num_blocks * block_size * Hkv >= (int64_t(1) << 31)) return LSQ_E_SHAPE;
  if (mask && (mask_rows_per_b != 1 && mask_rows_per_b != Hkv)) return LSQ_E_SHAPE;
  if (mask && mask_stride < max_seq_len) return LSQ_E_SHAPE;
  // masked tokens read pool row 0 (their results discarded): an empty pool has none
  if (num_blocks == 0 && max_seq_len > 0 && B > 0) return LSQ_E_SHAPE;
  if (B == 0) return LSQ_OK;
  if (!query || !k_pool || !v_pool || !block_tables || !seq_lens || !out) return LSQ_E_NULL;
  if (i8 && (!k_scales || !v_scales)) return LSQ_E_NULL;
  if ((reinterpret_cast<uintptr_t>(k_pool) & 15) || (reinterpret_cast<uintptr_t>(v_pool) & 15))
    return LSQ_E_ALIGN;
  if (B > 65535 || Hkv > 65535 || B * H > INT32_MAX) return LSQ_E_SHAPE;
  const int64_t nsplit = max_seq_len > 0 ? (max_seq_len + kPaNT - 1) / kPaNT : 1;
  if (nsplit > 1 && (!workspace || workspace_bytes < lsq_paged_attention_workspace_bytes(B, H, D, max_seq_len)))
    return LSQ_E_NULL;
  PagedArgs a{};
  a.q = query; a.kp = k_pool; a.vp = v_pool; a.ks = k_scales; a.vs = v_scales;
  a.scale_dt = scale_dtype; a.bt = block_tables; a.ldbt = bt_stride; a.nb = num_blocks; a.sl = seq_lens;
  a.mask = mask; a.ldm = mask_stride; a.mask_rows_per_b = static_cast<int>(mask_rows_per_b);
  a.out = out; a.ws = static_cast<float*>(workspace);
  a.B = static_cast<int>(B); a.H = static_cast<int>(H); a.Hkv = static_cast<int>(Hkv);
  a.G = static_cast<int>(H / Hkv); a.BS = static_cast<int>(block_size);
  a.nsplit = static_cast<int>(nsplit); a.max_sl = static_cast<int>(max_seq_len);
  a.interleaved = head_mapping != 0;
  a.sm_scale = 1.0f / std::sqrt(static_cast<float>(D));
  a.bs_m16 = block_size < 64 ? static_cast<int>((65536 + block_size - 1) / block_size) : 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case LSQ_F32: return launch_paged_dt<LSQ_F32>(a, i8, static_cast<int>(D), s);
    case LSQ_F16: return launch_paged_dt<LSQ_F16>(a, i8, static_cast<int>(D), s);
    default: return launch_paged_dt<LSQ_BF16>(a, i8, static_cast<int>(D), s);
  }
}
