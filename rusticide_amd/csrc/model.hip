// model.hip -- the decoder forward pass around the quantized matrix products,
// on the device: Decoder::forward_batch and greedy generation
// (crates/rusticide-transformer/src/decoder.rs:57-136,
//  crates/rusticide-model/src/generate.rs:35-124).
//
// Every projection goes through rh_matmul_batch_device (the fused decode
// GEMV, or the MFMA GEMM for prefill chunks); the kernels here do what lies
// between them, each following the reference's arithmetic step for step:
//   * RMSNorm: squares summed in order from -0.0 by one lane, then
//     x / sqrt(mean + eps) * w (portable/norm.rs:8-14, transformer norm.rs:10-14);
//   * RoPE, adjacent pairs: fma(lo, cos, -(hi*sin)), fma(hi, cos, lo*sin)
//     (portable/rope.rs:7-23) with cos/sin from a table the host computes
//     with its libm at decoder creation, the same calls the CPU path makes;
//   * attention per (token, head): the eight-lane fused dot over the head
//     (rusticide-simd/src/float.rs:23-36) / sqrt(head_dim), max-subtracted
//     softmax summed in order from 0.0, then mix_rows' fused accumulation in
//     row order (float.rs:52-62, attention.rs:41-57);
//   * SiLU * up, residual adds (portable/elementwise.rs);
//   * greedy pick: NaN as -inf, total order, the last maximum wins
//     (sampling/src/sampler.rs:75-87, filters.rs:37-43).
// exp is rh::expf_ref (rh_math.h), which returns the bits of the libm expf
// the CPU path calls.
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <new>
#include <type_traits>
#include <utility>
#include <vector>

#include "../../include/rusticide_hip.h"
#include "rh_device.h"
#include "rh_internal.h"
#include "rh_math.h"

namespace rh {
namespace {

constexpr uint32_t kNormThreads = 256;



// Element e of row `row` of token_embd (Matrix::copy_row's dequantization,
// weights.rs:120-150): f32 rows of `pitch` bytes, or Q4_K / Q6_K in the unit
// layout with `pitch` blocks a row.
__device__ __forceinline__ float embed_value(uint32_t type_id, const uint8_t* data, size_t pitch, uint32_t row,
                                             uint32_t e) {
  if (type_id == 0u) return reinterpret_cast<const float*>(data + static_cast<size_t>(row) * pitch)[e];
  return unit_weight(data, type_id, row * static_cast<uint32_t>(pitch) + e / 256u, e % 256u);
}

// Token rows of token_embd into hidden.
__global__ __launch_bounds__(256) void embed_kernel(uint32_t type_id, const uint8_t* data, size_t pitch,
                                                    const uint32_t* tokens, uint32_t width, float* hidden) {
  const uint32_t t = blockIdx.y;
  const uint32_t row = tokens[t];
  float* out = hidden + static_cast<size_t>(t) * width;
  for (uint32_t e = blockIdx.x * 256u + threadIdx.x; e < width; e += gridDim.x * 256u)
    out[e] = embed_value(type_id, data, pitch, row, e);
}

// hidden[t] (+= the residual delta, stored by weight row: delta[e*n + t],
// or with TM token-major: delta[t*width + e]),
// then normed[t] = normalize(hidden[t], weight) for tokens t >= norm_from.
// One workgroup of TH threads per token; each thread keeps its PER elements
// (e = tid + TH k) in registers from the first load to the last store, so
// every global load is issued up front.
constexpr uint32_t kMaxNormPer = 32;  // widths up to 256 * 32 = 8192

// QUANT: the normalized row is not stored as f32 but quantized to Q8_K into
// q8 (token t - norm_from), as quantize_super_kernel would from the f32 row;
// width must then be a multiple of 256.
// PL: the delta is a split GEMM's token-major planes (SplitOut: planes
// `np` of rows_pad x n floats each, at `pl`), summed here in plane order as
// gemm_combine_kernel would, so that GEMM needs no combine launch.
constexpr uint32_t kPlaneBatch = 8;  // planes requested at once

template <uint32_t PER, bool QUANT, uint32_t TH, bool TM, bool PL = false>
__global__ __launch_bounds__(TH) void add_norm_kernel(float* __restrict__ hidden, const float* __restrict__ delta,
                                                      uint32_t n, uint32_t width, const float* __restrict__ weight,
                                                      float eps, uint32_t norm_from, float* __restrict__ normed,
                                                      Q8Dev q8, const float* __restrict__ pl, uint32_t np,
                                                      uint32_t rows_pad) {
  extern __shared__ __align__(16) float sq[];
  __shared__ float s_rms;
  const uint32_t t = blockIdx.x, tid = threadIdx.x;
  float* h = hidden + static_cast<size_t>(t) * width;
  const bool norm = t >= norm_from;  // uniform over the workgroup
  float v[PER], wt[PER], dl[PER];
#pragma unroll
  for (uint32_t k = 0; k < PER; k++) {
    const uint32_t e = tid + k * TH;
    if (e < width) {
      v[k] = h[e];
      if (delta) dl[k] = TM ? delta[static_cast<size_t>(t) * width + e] : delta[static_cast<size_t>(e) * n + t];
      if (norm) wt[k] = weight[e];
    }
  }
  if constexpr (PL) {
    // plane 0, then planes 1.. one addition at a time; each batch of planes
    // requested before its first addition (indices clamped to the last)
    const size_t psz = static_cast<size_t>(rows_pad) * n;
    const float* base = pl + static_cast<size_t>(t) * rows_pad;
    for (uint32_t p0 = 0; p0 < np; p0 += kPlaneBatch) {
      float pv[kPlaneBatch][PER];
#pragma unroll
      for (uint32_t j = 0; j < kPlaneBatch; j++)
#pragma unroll
        for (uint32_t k = 0; k < PER; k++) {
          const uint32_t e = min(tid + k * TH, width - 1u);
          pv[j][k] = base[static_cast<size_t>(min(p0 + j, np - 1u)) * psz + e];
        }
#pragma unroll
      for (uint32_t j = 0; j < kPlaneBatch; j++)
#pragma unroll
        for (uint32_t k = 0; k < PER; k++)
          if (p0 + j < np) dl[k] = p0 + j == 0 ? pv[j][k] : dl[k] + pv[j][k];
    }
  }
  if (delta || PL) {
#pragma unroll
    for (uint32_t k = 0; k < PER; k++) {
      const uint32_t e = tid + k * TH;
      if (e < width) {
        v[k] += dl[k];
        h[e] = v[k];
      }
    }
  }
  if (!norm) return;
#pragma unroll
  for (uint32_t k = 0; k < PER; k++) {
    const uint32_t e = tid + k * TH;
    if (e < width) {
      const float s = v[k] * v[k];
      sq[wave_sum_index(e)] = s;
    }
  }
  // the rest of the last 32-value chunk holds the sum's identity
  if (tid < ((width + 31u) & ~31u) - width) sq[wave_sum_index(width + tid)] = -0.0f;
  __syncthreads();
  if (tid < 64u) {
    // the squares summed in order from -0.0 (f32 Sum), by wave 0
    const float sum = ordered_sum_wave(sq, width, -0.0f);
    if (tid == 0) {
      const float mean = __fdiv_rn(sum, static_cast<float>(width));
      s_rms = sqrt_rn(mean + eps);
    }
  }
  __syncthreads();
  const float rms = s_rms;
  if constexpr (QUANT) {
    // the squares are summed: their LDS takes the normalized row, which each
    // wave then quantizes a 256-value block at a time
#pragma unroll
    for (uint32_t k = 0; k < PER; k++) {
      const uint32_t e = tid + k * TH;
      if (e < width) sq[e] = __fdiv_rn(v[k], rms) * wt[k];
    }
    __syncthreads();
    const uint32_t lane = tid & 63u;
    for (uint32_t sb = tid >> 6; sb < width / 256u; sb += TH / 64u) {
      float f[4];
#pragma unroll
      for (int i = 0; i < 4; i++) f[i] = sq[sb * 256u + lane * 4u + static_cast<uint32_t>(i)];
      quantize_super_block(f, lane, t - norm_from, sb, q8);
    }
    return;
  }
  float* o = normed + static_cast<size_t>(t - norm_from) * width;
#pragma unroll
  for (uint32_t k = 0; k < PER; k++) {
    const uint32_t e = tid + k * TH;
    if (e < width) {
      const float x = __fdiv_rn(v[k], rms);
      o[e] = x * wt[k];
    }
  }
}

using AddNormFn = void (*)(float*, const float*, uint32_t, uint32_t, const float*, float, uint32_t, float*, Q8Dev,
                          const float*, uint32_t, uint32_t);

// Dynamic LDS of add_norm_kernel: the squares in the ordered sum's layout
// (at least width floats, which the QUANT form reuses for the row).
size_t add_norm_lds(uint32_t width) {
  const size_t n = wave_sum_floats(width);
  return (n > width ? n : width) * 4u;
}

// The add_norm_kernel instance for a row width (<= 256 * kMaxNormPer) and
// its workgroup size: rows of 2048 values or more take 512 threads, so that
// eight waves quantize eight 256-value blocks at once (a 2048-wide QUANT
// norm of 64 tokens: 5.1 against 5.9 us with 256 threads).
struct AddNorm {
  AddNormFn fn;
  uint32_t threads;
};

template <bool QUANT = false, bool TM = false, bool PL = false>
AddNorm add_norm_for(uint32_t width) {
  if (width >= 2048u) {
    if (width <= 4u * 512u) return {add_norm_kernel<4, QUANT, 512, TM, PL>, 512u};
    if (width <= 8u * 512u) return {add_norm_kernel<8, QUANT, 512, TM, PL>, 512u};
    return {add_norm_kernel<kMaxNormPer / 2u, QUANT, 512, TM, PL>, 512u};
  }
  if (width <= 4u * kNormThreads) return {add_norm_kernel<4, QUANT, kNormThreads, TM, PL>, kNormThreads};
  return {add_norm_kernel<8, QUANT, kNormThreads, TM, PL>, kNormThreads};
}

// q/k/v from the projections (stored by weight row, x[e*n + t]): q rotated
// into token-major rows, k rotated and v copied into the cache at positions
// start + t. One thread per rotation pair (q, k) or value element (v).
__global__ __launch_bounds__(256) void qkv_post_kernel(const float* qr, const float* kr, const float* vr, uint32_t n,
                                                       uint32_t width, uint32_t kv, uint32_t head_dim,
                                                       const float* rcos, const float* rsin, uint32_t start,
                                                       float* q, float* kcache, float* vcache) {
  const uint32_t t = blockIdx.y;
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  const uint32_t pairs = head_dim / 2u;
  const uint32_t pos = start + t;
  const uint32_t qp = width / 2u, kp = kv / 2u;
  if (i < qp + kp) {
    const bool is_q = i < qp;
    const uint32_t e = 2u * (is_q ? i : i - qp);
    const float* src = is_q ? qr : kr;
    const float lo = src[static_cast<size_t>(e) * n + t], hi = src[static_cast<size_t>(e + 1u) * n + t];
    const uint32_t p = (e % head_dim) / 2u;
    const float c = rcos[static_cast<size_t>(pos) * pairs + p], s = rsin[static_cast<size_t>(pos) * pairs + p];
    const float hs = hi * s, ls = lo * s;
    const float nlo = __builtin_fmaf(lo, c, -hs), nhi = __builtin_fmaf(hi, c, ls);
    float* dst = is_q ? q + static_cast<size_t>(t) * width : kcache + static_cast<size_t>(pos) * kv;
    dst[e] = nlo;
    dst[e + 1u] = nhi;
  } else if (i < qp + kp + kv) {
    const uint32_t e = i - qp - kp;
    vcache[static_cast<size_t>(pos) * kv + e] = vr[static_cast<size_t>(e) * n + t];
  }
}

constexpr uint32_t kAttnThreads = 256;
constexpr uint32_t kVTile = 64;  // value rows per LDS tile

constexpr uint32_t kMaxHeadDim = 128;

// LDS floats attention_kernel needs for `rows` cached rows: the query head
// (up to kMaxHeadDim), a reduction area, the weights, and two value tiles of
// kVTile * 64 floats (kVTile rows up to head_dim 64, half as many above).
inline size_t attention_lds_floats(size_t rows) {
  return kMaxHeadDim + 64u + ((rows + 3u) & ~size_t{3}) + 2u * kVTile * 64u;
}

// Value rows per tile of attention_kernel.
__host__ __device__ constexpr uint32_t tile_rows(uint32_t hd) { return hd <= 64u ? kVTile : kVTile / 2u; }

// Value rows r0..r0+count of one kv head into registers, one tile's share
// per thread (HD = 64: 16 f32x4 per row, 16 threads a row).
template <uint32_t HD>
struct VTileRegs {
  static constexpr uint32_t kPer = HD ? kVTile * HD / 4u / kAttnThreads : kVTile * 64u / kAttnThreads;
  using T = typename std::conditional<HD != 0, f32x4, float>::type;
  T v[kPer];
  // Every thread loads unconditionally (rows past count re-read row
  // count - 1, which store() drops): a load under a condition into this
  // array would make the compiler keep it in scratch and wait for each load.
  __device__ __forceinline__ void load(const float* vcache, uint32_t kv, uint32_t off, uint32_t hd, uint32_t r0,
                                       uint32_t count) {
#pragma unroll
    for (uint32_t k = 0; k < kPer; k++) {
      const uint32_t f = threadIdx.x + k * kAttnThreads;
      if constexpr (HD != 0) {
        const uint32_t r = f / (HD / 4u), c = f % (HD / 4u);
        const uint32_t rr = r < count ? r : count - 1u;
        v[k] = *reinterpret_cast<const T*>(vcache + static_cast<size_t>(r0 + rr) * kv + off + 4u * c);
      } else {
        const uint32_t r = f / hd, c = f % hd;
        const uint32_t rr = r < count ? r : count - 1u;
        v[k] = vcache[static_cast<size_t>(r0 + rr) * kv + off + c];
      }
    }
  }
  // load() for head_dim HD, rows from `start` on read from vnew (the batch's
  // value projection, token-major with rows of kv floats) instead of vcache
  __device__ __forceinline__ void load_split(const float* vcache, const float* vnew, uint32_t start, uint32_t kv,
                                             uint32_t off, uint32_t r0, uint32_t count) {
    static_assert(HD != 0, "head_dim fixed");
#pragma unroll
    for (uint32_t k = 0; k < kPer; k++) {
      const uint32_t f = threadIdx.x + k * kAttnThreads;
      const uint32_t r = f / (HD / 4u), c = f % (HD / 4u);
      const uint32_t row = r0 + (r < count ? r : count - 1u);
      const float* src = row >= start ? vnew + static_cast<size_t>(row - start) * kv : vcache + static_cast<size_t>(row) * kv;
      v[k] = *reinterpret_cast<const T*>(src + off + 4u * c);
    }
  }
  __device__ __forceinline__ void store(float* tile, uint32_t hd, uint32_t count) const {
#pragma unroll
    for (uint32_t k = 0; k < kPer; k++) {
      const uint32_t f = threadIdx.x + k * kAttnThreads;
      if constexpr (HD != 0) {
        if (f / (HD / 4u) < count) reinterpret_cast<T*>(tile)[f] = v[k];
      } else {
        if (f / hd < count && f < kVTile * hd) tile[f] = v[k];
      }
    }
  }
};

// dot (float.rs:23-36) for head_dim 64: eight fused lanes over the eight
// 8-wide chunks.
__device__ __forceinline__ void lanes64(const float* qh, const f32x4 (&k4)[16], float (&acc)[8]) {
#pragma unroll
  for (int c = 0; c < 8; c++) {
    const f32x4 a = k4[2 * c], b = k4[2 * c + 1];
    acc[0] = __builtin_fmaf(qh[8 * c + 0], a.x, acc[0]);
    acc[1] = __builtin_fmaf(qh[8 * c + 1], a.y, acc[1]);
    acc[2] = __builtin_fmaf(qh[8 * c + 2], a.z, acc[2]);
    acc[3] = __builtin_fmaf(qh[8 * c + 3], a.w, acc[3]);
    acc[4] = __builtin_fmaf(qh[8 * c + 4], b.x, acc[4]);
    acc[5] = __builtin_fmaf(qh[8 * c + 5], b.y, acc[5]);
    acc[6] = __builtin_fmaf(qh[8 * c + 6], b.z, acc[6]);
    acc[7] = __builtin_fmaf(qh[8 * c + 7], b.w, acc[7]);
  }
}

// The dot's lanes summed in order from -0.0, plus the tail, over the scale
// (attention.rs:189-207 divides each score by sqrt(head_dim)).
__device__ __forceinline__ float score_from_lanes(const float (&acc)[8], float tail, float scale) {
  float s = -0.0f;
#pragma unroll
  for (int l = 0; l < 8; l++) s += acc[l];
  return __fdiv_rn(s + tail, scale);
}

// f32 order as unsigned keys, for DPP maxima: a larger float, a larger key;
// NaN maps to 0, below every number, and back to a NaN.
__device__ __forceinline__ uint32_t max_key(float f) {
  const uint32_t b = __float_as_uint(f);
  return f != f ? 0u : (b >> 31) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float max_key_float(uint32_t k) {
  return __uint_as_float((k >> 31) ? (k & 0x7fffffffu) : ~k);
}

// softmax (norm.rs:17-30) of the scores w[0..rows) in place, given each
// thread's maximum of the scores it wrote: the maximum over the workgroup
// (exact in any order), exp(x - max), the sum in order from 0.0 on one lane,
// and the division. The caller synchronizes before reading w.
__device__ __forceinline__ void softmax_rows(float* w, uint32_t rows, float mx, float* red) {
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  // the maximum over each half-wave as an order-preserving key (DPP), then
  // the two halves; NaN keys are the smallest, so NaN scores drop out as
  // fmaxf drops them
  mx = max_key_float(half_max_u32(max_key(mx)));
  mx = fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(mx), 0)),
             __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mx), 32)));
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  for (uint32_t i = tid; i < rows; i += kAttnThreads) w[i] = expf_ref(w[i] - mx);
  __syncthreads();
  if (tid == 0) red[4] = ordered_sum(w, rows, 0.0f);  // portable/norm.rs: `let mut sum = 0.0`
  __syncthreads();
  const float sum = red[4];
  for (uint32_t i = tid; i < rows; i += kAttnThreads) w[i] = __fdiv_rn(w[i], sum);
}

// mix_rows (float.rs:52-62) over one staged value tile: output lane `lane`
// adds rows 0..count of the tile in order, one fused multiply-add each.
__device__ __forceinline__ float mix_tile(const float* cur, const float* wr, uint32_t count, uint32_t hd,
                                          uint32_t lane, float acc) {
  uint32_t r = 0;
  for (; r + 16u <= count; r += 16u) {
    float v[16];
#pragma unroll
    for (int k = 0; k < 16; k++) v[k] = cur[(r + k) * hd + lane];
#pragma unroll
    for (int k = 0; k < 16; k++) acc = __builtin_fmaf(v[k], wr[r + k], acc);
  }
  for (; r < count; r++) acc = __builtin_fmaf(cur[r * hd + lane], wr[r], acc);
  return acc;
}

// One workgroup per (query head, token): scores over cached rows
// 0..=start+t, softmax, then the weighted sum of value rows
// (attention.rs:41-57,189-207). HD = 64 specializes head_dim; HD = 0 reads
// it at run time (any even head_dim <= kMaxHeadDim; above 64 the value tiles
// hold 32 rows and the row chains of output lanes 64.. run on wave 1).
template <uint32_t HD>
__global__ __launch_bounds__(kAttnThreads) void attention_kernel(const float* q, const float* kcache,
                                                                 const float* vcache, uint32_t width, uint32_t kv,
                                                                 uint32_t head_dim, uint32_t group, float scale,
                                                                 uint32_t start, float* mixed) {
  extern __shared__ __align__(16) float sh[];
  const uint32_t hd = HD ? HD : head_dim;
  const uint32_t h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
  const uint32_t rows = start + t + 1u;
  const uint32_t tr = tile_rows(hd);
  float* qh = sh;                      // [kMaxHeadDim]
  float* red = sh + kMaxHeadDim;       // [64]
  float* w = red + 64;                 // [rows rounded up to 4]
  float* vt = w + ((rows + 3u) & ~3u);  // [2][kVTile * 64]
  const uint32_t off = (h / group) * hd;
  if (tid < hd) qh[tid] = q[static_cast<size_t>(t) * width + h * hd + tid];
  __syncthreads();
  // dot (float.rs:23-36): eight fused lanes over whole chunks, lanes summed
  // in order from -0.0, then the unfused tail summed from -0.0. One cached
  // row per thread, its loads issued before the arithmetic.
  float mx = -INFINITY;
  for (uint32_t i = tid; i < rows; i += kAttnThreads) {
    const float* kr = kcache + static_cast<size_t>(i) * kv + off;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float tail = -0.0f;
    if constexpr (HD == 64u) {
      f32x4 k4[16];
#pragma unroll
      for (int c = 0; c < 16; c++) k4[c] = reinterpret_cast<const f32x4*>(kr)[c];
      lanes64(qh, k4, acc);
    } else {
      const uint32_t chunks = hd / 8u;
      for (uint32_t c = 0; c < chunks; c++)
#pragma unroll
        for (int l = 0; l < 8; l++) acc[l] = __builtin_fmaf(qh[8u * c + l], kr[8u * c + l], acc[l]);
      for (uint32_t e = 8u * chunks; e < hd; e++) {
        const float p = qh[e] * kr[e];
        tail += p;
      }
    }
    const float score = score_from_lanes(acc, tail, scale);
    w[i] = score;
    mx = fmaxf(mx, score);
  }
  softmax_rows(w, rows, mx, red);
  // mix_rows (float.rs:52-62): out starts at 0.0, each row fused in order.
  // Value tiles are staged through LDS by every thread, a tile ahead of
  // the first wave's chain of fused adds.
  const uint32_t tiles = (rows + tr - 1u) / tr;
  VTileRegs<HD> regs;
  regs.load(vcache, kv, off, hd, 0u, rows < tr ? rows : tr);
  regs.store(vt, hd, rows < tr ? rows : tr);
  __syncthreads();
  float acc = 0.0f;
  for (uint32_t tile = 0; tile < tiles; tile++) {
    const uint32_t r0 = tile * tr;
    const uint32_t count = rows - r0 < tr ? rows - r0 : tr;
    const bool more = tile + 1u < tiles;
    const uint32_t nr0 = r0 + tr, ncount = more ? (rows - nr0 < tr ? rows - nr0 : tr) : 0u;
    if (more) regs.load(vcache, kv, off, hd, nr0, ncount);
    if (tid < hd) acc = mix_tile(vt + (tile & 1u) * kVTile * 64u, w + r0, count, hd, tid, acc);
    if (more) regs.store(vt + ((tile + 1u) & 1u) * kVTile * 64u, hd, ncount);
    __syncthreads();
  }
  if (tid < hd) mixed[static_cast<size_t>(t) * width + h * hd + tid] = acc;
}

// attention_kernel<64> for the G query heads of one kv head (G = 4 or 8):
// one workgroup per (kv head, token) forms the G heads' scores, softmaxes
// and value mixes with attention_kernel's arithmetic, reading each key and
// value row once for all G heads (a 64-token prefill of 32/4 heads: 256
// workgroups instead of 2048). In the scores thread tid takes head tid % G
// and rows tid / G + (256 / G) k: the G lanes of a row read its 16-byte
// pieces together, so a load instruction touches 64 / G rows, not 64 (a
// 64-row score pass: 1.3 against 3.9 us); the mix gives every thread the
// output lane tid % 64 of heads tid / 64 + 4k. With QUANT the G heads'
// outputs, G / 4 whole 256-value blocks of the token's mixed row, are
// quantized to Q8_K into q8 as quantize_super_kernel would from that row,
// and not stored.
// With ROPE, qkv_post_kernel's work for the batch is done here too, so it
// needs no launch of its own: q is the raw query projection, token-major;
// keys and values of the batch's rows (start on) come raw from kr and vr
// (token-major, kv floats a row), the keys rotated as they are read, and
// the workgroups of a kv head's token t append its row start + t to the
// caches (no workgroup of the launch reads those cache rows).
template <uint32_t G, bool QUANT, bool ROPE>
__global__ __launch_bounds__(kAttnThreads) void attention_group_kernel(const float* q, float* kcache, float* vcache,
                                                                       uint32_t width, uint32_t kv, float scale,
                                                                       uint32_t start, float* mixed, Q8Dev q8,
                                                                       const float* kr, const float* vr,
                                                                       const float* rcos, const float* rsin) {
  static_assert(G == 4u || G == 8u, "four or eight query heads per kv head");
  constexpr uint32_t HD = 64u, L = kAttnThreads / G;  // lanes per head in the scores
  extern __shared__ __align__(16) float sh[];
  const uint32_t g = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
  constexpr uint32_t QS = HD + 4u;  // LDS floats per query head: the G heads' reads fall on distinct banks
  // ws: LDS floats per head's weights, 4 more than a multiple of 4, so that
  // the G lanes summing the G heads at once read distinct banks
  const uint32_t rows = start + t + 1u, ws = ((rows + 3u) & ~3u) + 4u;
  float* qh = sh;                // [G][QS]; with QUANT later the outputs
  float* red = qh + G * QS;      // [64]: the waves' maxima, then the sums
  float* w = red + 64;           // [G][ws]
  float* vt = w + G * ws;        // [2][kVTile * 64]
  const uint32_t off = g * HD;
  // the first value tile goes out with the query heads (its registers stay
  // live over the scores' loop only as 16 floats)
  constexpr uint32_t kPairs = HD / 2u;
  VTileRegs<HD> regs;
  if constexpr (ROPE)
    regs.load_split(vcache, vr, start, kv, off, 0u, rows < kVTile ? rows : kVTile);
  else
    regs.load(vcache, kv, off, HD, 0u, rows < kVTile ? rows : kVTile);
  if constexpr (ROPE) {
    // qkv_post_kernel's rotation of the G query heads (pair p of head j), and
    // of this token's key row into the cache (threads of the first head)
    const uint32_t pos = start + t;
    for (uint32_t pi = tid; pi < G * kPairs; pi += kAttnThreads) {
      const uint32_t jh = pi / kPairs, p = pi % kPairs;
      const float* src = q + static_cast<size_t>(t) * width + (g * G + jh) * HD;
      const float lo = src[2u * p], hi = src[2u * p + 1u];
      const float c = rcos[static_cast<size_t>(pos) * kPairs + p], sn = rsin[static_cast<size_t>(pos) * kPairs + p];
      const float hs = hi * sn, ls = lo * sn;
      qh[jh * QS + 2u * p] = __builtin_fmaf(lo, c, -hs);
      qh[jh * QS + 2u * p + 1u] = __builtin_fmaf(hi, c, ls);
      if (jh == 0u) {
        const float* ks = kr + static_cast<size_t>(t) * kv + off;
        const float klo = ks[2u * p], khi = ks[2u * p + 1u];
        const float khs = khi * sn, kls = klo * sn;
        float* kd = kcache + static_cast<size_t>(pos) * kv + off;
        kd[2u * p] = __builtin_fmaf(klo, c, -khs);
        kd[2u * p + 1u] = __builtin_fmaf(khi, c, kls);
      }
    }
    if (tid >= 64u && tid < 64u + HD / 4u)
      reinterpret_cast<f32x4*>(vcache + static_cast<size_t>(pos) * kv + off)[tid - 64u] =
          reinterpret_cast<const f32x4*>(vr + static_cast<size_t>(t) * kv + off)[tid - 64u];
  } else {
    for (uint32_t i = tid; i < G * HD; i += kAttnThreads)
      qh[(i / HD) * QS + i % HD] = q[static_cast<size_t>(t) * width + g * G * HD + i];
  }
  __syncthreads();
  const uint32_t j = tid % G, i0 = tid / G;
  float* wj = w + j * ws;
  float mx = -INFINITY;
  for (uint32_t i = i0; i < rows; i += L) {
    // ROPE: a batch row (i >= start) is read raw and rotated here with
    // qkv_post_kernel's expressions; the rotation's table loads are
    // unconditional (a cached row drops their result)
    const bool fresh = ROPE && i >= start;
    const float* krow = fresh ? kr + static_cast<size_t>(i - start) * kv + off : kcache + static_cast<size_t>(i) * kv + off;
    f32x4 k4[16];
#pragma unroll
    for (int c = 0; c < 16; c++) k4[c] = reinterpret_cast<const f32x4*>(krow)[c];
    if constexpr (ROPE) {
      f32x4 cs[8], sn[8];
#pragma unroll
      for (int c = 0; c < 8; c++) {
        cs[c] = reinterpret_cast<const f32x4*>(rcos + static_cast<size_t>(i) * kPairs)[c];
        sn[c] = reinterpret_cast<const f32x4*>(rsin + static_cast<size_t>(i) * kPairs)[c];
      }
#pragma unroll
      for (int c = 0; c < 16; c++) {
        f32x4 r = k4[c];
#pragma unroll
        for (int u = 0; u < 2; u++) {
          // pair 2c + u: elements 2u, 2u + 1 of the chunk
          const float co = cs[c >> 1][2 * (c & 1) + u], si = sn[c >> 1][2 * (c & 1) + u];
          const float lo = k4[c][2 * u], hi = k4[c][2 * u + 1];
          const float hs = hi * si, ls = lo * si;
          r[2 * u] = __builtin_fmaf(lo, co, -hs);
          r[2 * u + 1] = __builtin_fmaf(hi, co, ls);
        }
        k4[c] = fresh ? r : k4[c];
      }
    }
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    lanes64(qh + j * QS, k4, acc);
    const float score = score_from_lanes(acc, -0.0f, scale);
    wj[i] = score;
    mx = fmaxf(mx, score);
  }
  // softmax_rows per head: the maximum over the head's lanes (exact in any
  // order; every lane's is a number, fmaxf having dropped NaN scores), exp,
  // the sum in order from 0.0 on one lane of the head, the division
  const uint32_t wave = tid >> 6;
#pragma unroll
  for (uint32_t o = G; o < 64u; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, static_cast<int>(o), 64));
  if ((tid & 63u) < G) red[wave * G + j] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[j], red[G + j]), fmaxf(red[2u * G + j], red[3u * G + j]));
  for (uint32_t i = i0; i < rows; i += L) wj[i] = expf_ref(wj[i] - mx);
  __syncthreads();
  if (i0 == 0) red[32u + j] = ordered_sum(wj, rows, 0.0f);  // portable/norm.rs: `let mut sum = 0.0`
  __syncthreads();
  const float sum = red[32u + j];
  for (uint32_t i = i0; i < rows; i += L) wj[i] = __fdiv_rn(wj[i], sum);
  regs.store(vt, HD, rows < kVTile ? rows : kVTile);
  __syncthreads();
  // mix_rows: each output lane's chain of fused adds over the rows in order
  const uint32_t d = tid & 63u, jp = tid >> 6;
  float acc[G / 4u];
#pragma unroll
  for (uint32_t k = 0; k < G / 4u; k++) acc[k] = 0.0f;
  const uint32_t tiles = (rows + kVTile - 1u) / kVTile;
  for (uint32_t tile = 0; tile < tiles; tile++) {
    const uint32_t r0 = tile * kVTile;
    const uint32_t count = rows - r0 < kVTile ? rows - r0 : kVTile;
    const bool more = tile + 1u < tiles;
    const uint32_t nr0 = r0 + kVTile, ncount = more ? (rows - nr0 < kVTile ? rows - nr0 : kVTile) : 0u;
    if (more) {
      if constexpr (ROPE)
        regs.load_split(vcache, vr, start, kv, off, nr0, ncount);
      else
        regs.load(vcache, kv, off, HD, nr0, ncount);
    }
    const float* cur = vt + (tile & 1u) * kVTile * 64u;
    uint32_t r = 0;
    for (; r + 16u <= count; r += 16u) {
      float v[16];
#pragma unroll
      for (int k = 0; k < 16; k++) v[k] = cur[(r + k) * HD + d];
#pragma unroll
      for (int k = 0; k < 16; k++)
#pragma unroll
        for (uint32_t h = 0; h < G / 4u; h++) acc[h] = __builtin_fmaf(v[k], w[(jp + 4u * h) * ws + r0 + r + k], acc[h]);
    }
    for (; r < count; r++) {
      const float v = cur[r * HD + d];
#pragma unroll
      for (uint32_t h = 0; h < G / 4u; h++) acc[h] = __builtin_fmaf(v, w[(jp + 4u * h) * ws + r0 + r], acc[h]);
    }
    if (more) regs.store(vt + ((tile + 1u) & 1u) * kVTile * 64u, HD, ncount);
    __syncthreads();
  }
  if constexpr (!QUANT) {
#pragma unroll
    for (uint32_t h = 0; h < G / 4u; h++)
      mixed[static_cast<size_t>(t) * width + (g * G + jp + 4u * h) * HD + d] = acc[h];
  } else {
    // block h of the group holds heads 4h .. 4h + 3, head jp + 4h at jp * 64
#pragma unroll
    for (uint32_t h = 0; h < G / 4u; h++) qh[h * 256u + jp * HD + d] = acc[h];
    __syncthreads();
    const uint32_t lane = tid & 63u;
    if (wave < G / 4u) {
      const f32x4 v = reinterpret_cast<const f32x4*>(qh + wave * 256u)[lane];
      const float f[4] = {v[0], v[1], v[2], v[3]};
      quantize_super_block(f, lane, t, g * G / 4u + wave, q8);
    }
  }
}

using AttnGroupFn = void (*)(const float*, float*, float*, uint32_t, uint32_t, float, uint32_t, float*, Q8Dev,
                            const float*, const float*, const float*, const float*);
constexpr size_t kMaxLdsBytes = 160u * 1024u;  // a gfx950 workgroup's LDS

// LDS floats attention_group_kernel needs for `rows` cached rows.
inline size_t attention_group_lds_floats(size_t group, size_t rows) {
  return group * 68u + 64u + group * (((rows + 3u) & ~size_t{3}) + 4u) + 2u * kVTile * 64u;
}

// Value tile rows r0.. (below `rows`) of one kv head for head_dim 64, a
// f32x4 per thread and k; row `start` comes from the projection `vnew`.
// Loads are unconditional (rows past the end re-read row `start`, and
// store_v_tile drops them) so the tile stays in registers.
constexpr uint32_t kStepVTiles = 4;  // value tiles a step loads before its first wait
constexpr uint32_t kTileF4 = kVTile * 64u / 4u / kAttnThreads;

__device__ __forceinline__ void load_v_tile(f32x4 (&v)[kTileF4], const float* vcache, const float* vnew, uint32_t kv,
                                            uint32_t off, uint32_t r0, uint32_t rows, uint32_t start) {
#pragma unroll
  for (uint32_t k = 0; k < kTileF4; k++) {
    const uint32_t f = threadIdx.x + k * kAttnThreads, row = r0 + (f >> 4);
    const uint32_t rr = row < rows ? row : start;
    const float* src = rr == start ? vnew : vcache + static_cast<size_t>(rr) * kv + off;
    v[k] = reinterpret_cast<const f32x4*>(src)[f & 15u];
  }
}

__device__ __forceinline__ void store_v_tile(float* tile, const f32x4 (&v)[kTileF4], uint32_t r0, uint32_t rows) {
#pragma unroll
  for (uint32_t k = 0; k < kTileF4; k++) {
    const uint32_t f = threadIdx.x + k * kAttnThreads;
    if (r0 + (f >> 4) < rows) reinterpret_cast<f32x4*>(tile)[f] = v[k];
  }
}

// One token at position `start` with head_dim 64: qkv_post_kernel and
// attention_kernel in one launch, with their arithmetic. Each workgroup (one
// per query head) rotates its q and its kv head's new key row itself, with
// qkv_post_kernel's expressions, and takes the new value row from the
// projection; the first workgroup of each kv head appends the new key and
// value rows to the cache (no workgroup of the launch reads that row from
// the cache). Every global load -- each thread's first cached key row, the
// RoPE inputs, the new value row and up to kStepVTiles value tiles -- is
// issued before the first wait, so the step waits on memory once.
__global__ __launch_bounds__(kAttnThreads) void attention_step_kernel(
    const float* qr, const float* kr, const float* vr, const float* rcos, const float* rsin, float* kcache,
    float* vcache, uint32_t kv, uint32_t group, float scale, uint32_t start, float* mixed) {
  constexpr uint32_t hd = 64u;
  extern __shared__ __align__(16) float sh[];
  const uint32_t h = blockIdx.x, tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t rows = start + 1u;
  float* qh = sh;                        // [64]
  float* red = sh + 64;                  // [64]
  float* w = sh + 128;                   // [rows rounded up to 4]
  float* vt = w + ((rows + 3u) & ~3u);   // [2][kVTile * 64]
  float* knew = vt + kVTile * 64u;       // the rotated new key, in tile buffer 1 until the values need it
  const uint32_t off = (h / group) * hd;
  const bool appends = h % group == 0u;
  const float* vnew = vr + off;

  // RoPE inputs (qkv_post_kernel): threads 0..31 the query's pairs, 32..63
  // the new key's. Issued first: loads return in order, and the rotation and
  // the barrier after it need only these.
  float lo = 0.0f, hi = 0.0f, cs = 0.0f, sn = 0.0f;
  const uint32_t pair = tid & 31u;
  if (tid < 64u) {
    const float* src = tid < 32u ? qr + static_cast<size_t>(h) * hd : kr + off;
    lo = src[2u * pair];
    hi = src[2u * pair + 1u];
    cs = rcos[static_cast<size_t>(start) * (hd / 2u) + pair];
    sn = rsin[static_cast<size_t>(start) * (hd / 2u) + pair];
  }
  // this thread's first cached key row (row 0, unused, when it has none)
  f32x4 k4[16];
  const float* k0 = kcache + static_cast<size_t>(tid < start ? tid : 0u) * kv + off;
#pragma unroll
  for (int c = 0; c < 16; c++) k4[c] = reinterpret_cast<const f32x4*>(k0)[c];
  const f32x4 vrow = reinterpret_cast<const f32x4*>(vnew)[tid & 15u];
  f32x4 vtile[kStepVTiles][kTileF4];
#pragma unroll
  for (uint32_t t = 0; t < kStepVTiles; t++) load_v_tile(vtile[t], vcache, vnew, kv, off, t * kVTile, rows, start);

  if (tid < 64u) {
    const float hs = hi * sn, ls = lo * sn;
    const float nlo = __builtin_fmaf(lo, cs, -hs), nhi = __builtin_fmaf(hi, cs, ls);
    float* dst = tid < 32u ? qh : knew;
    dst[2u * pair] = nlo;
    dst[2u * pair + 1u] = nhi;
  }
  __syncthreads();
  if (appends) {
    if (tid < 16u)
      reinterpret_cast<f32x4*>(kcache + static_cast<size_t>(start) * kv + off)[tid] =
          reinterpret_cast<const f32x4*>(knew)[tid];
    else if (tid >= 64u && tid < 80u)
      reinterpret_cast<f32x4*>(vcache + static_cast<size_t>(start) * kv + off)[tid - 64u] = vrow;
  }

  float mx = -INFINITY;
  for (uint32_t i = tid; i < rows; i += kAttnThreads) {
    f32x4 kk[16];
    if (i == start) {
#pragma unroll
      for (int c = 0; c < 16; c++) kk[c] = reinterpret_cast<const f32x4*>(knew)[c];
    } else if (i == tid) {
#pragma unroll
      for (int c = 0; c < 16; c++) kk[c] = k4[c];
    } else {
#pragma unroll
      for (int c = 0; c < 16; c++)
        kk[c] = reinterpret_cast<const f32x4*>(kcache + static_cast<size_t>(i) * kv + off)[c];
    }
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    lanes64(qh, kk, acc);
    const float score = score_from_lanes(acc, -0.0f, scale);
    w[i] = score;
    mx = fmaxf(mx, score);
  }
  softmax_rows(w, rows, mx, red);

  // mix_rows over the value tiles, staged through the two LDS buffers a tile
  // ahead of wave 0's chain; tiles past kStepVTiles are loaded here
  const uint32_t tiles = (rows + kVTile - 1u) / kVTile;
  float acc = 0.0f;
  store_v_tile(vt, vtile[0], 0u, rows);
  __syncthreads();
#pragma unroll
  for (uint32_t t = 0; t < kStepVTiles; t++) {
    if (t < tiles) {
      const uint32_t r0 = t * kVTile, count = rows - r0 < kVTile ? rows - r0 : kVTile;
      float* next = vt + ((t + 1u) & 1u) * kVTile * 64u;
      if (t + 1u < tiles) {
        if (t + 1u < kStepVTiles) {
          store_v_tile(next, vtile[t + 1u < kStepVTiles ? t + 1u : 0u], r0 + kVTile, rows);
        } else {
          f32x4 v[kTileF4];
          load_v_tile(v, vcache, vnew, kv, off, r0 + kVTile, rows, start);
          store_v_tile(next, v, r0 + kVTile, rows);
        }
      }
      if (wave == 0) acc = mix_tile(vt + (t & 1u) * kVTile * 64u, w + r0, count, hd, lane, acc);
      __syncthreads();
    }
  }
  for (uint32_t t = kStepVTiles; t < tiles; t++) {
    const uint32_t r0 = t * kVTile, count = rows - r0 < kVTile ? rows - r0 : kVTile;
    if (t + 1u < tiles) {
      f32x4 v[kTileF4];
      load_v_tile(v, vcache, vnew, kv, off, r0 + kVTile, rows, start);
      store_v_tile(vt + ((t + 1u) & 1u) * kVTile * 64u, v, r0 + kVTile, rows);
    }
    if (wave == 0) acc = mix_tile(vt + (t & 1u) * kVTile * 64u, w + r0, count, hd, lane, acc);
    __syncthreads();
  }
  if (wave == 0) mixed[static_cast<size_t>(h) * hd + lane] = acc;
}

// mix_rows (float.rs:52-62) for output lane `lane` over value rows 0..rows
// held in LDS at 64 floats a row, with the weights w: one fused add per row
// in order from 0.0. Batches of 16 rows (values and weights) are read while
// the previous batch is added; the scheduling barriers keep the compiler from
// sinking the reads below the adds.
struct MixBatch {
  float v[16];
  f32x4 w[4];
};

__device__ __forceinline__ void mix_load(MixBatch& b, const float* col, const float* w) {
#pragma unroll
  for (int k = 0; k < 16; k++) b.v[k] = col[k * 64];
#pragma unroll
  for (int k = 0; k < 4; k++) b.w[k] = reinterpret_cast<const f32x4*>(w)[k];
}

__device__ __forceinline__ float mix_add(float acc, const MixBatch& b) {
#pragma unroll
  for (int k = 0; k < 16; k++) acc = __builtin_fmaf(b.v[k], b.w[k >> 2][k & 3], acc);
  return acc;
}

__device__ __forceinline__ float mix_lds(const float* va, const float* w, uint32_t rows, uint32_t lane) {
  const float* col = va + lane;
  float acc = 0.0f;
  uint32_t r = 0;
  if (rows >= 16u) {
    MixBatch a, b;
    mix_load(a, col, w);
    for (r = 16u; r + 32u <= rows; r += 32u) {
      mix_load(b, col + r * 64u, w + r);
      __builtin_amdgcn_sched_barrier(0);
      acc = mix_add(acc, a);
      mix_load(a, col + (r + 16u) * 64u, w + r + 16u);
      __builtin_amdgcn_sched_barrier(0);
      acc = mix_add(acc, b);
    }
    if (r + 16u <= rows) {
      mix_load(b, col + r * 64u, w + r);
      __builtin_amdgcn_sched_barrier(0);
      acc = mix_add(acc, a);
      acc = mix_add(acc, b);
      r += 16u;
    } else {
      acc = mix_add(acc, a);
    }
  }
  for (; r < rows; r++) acc = __builtin_fmaf(col[r * 64u], w[r], acc);
  return acc;
}

// attention_step_kernel's arithmetic for up to kStepLdsRows rows (the new
// one included), with its memory traffic rearranged. The key rows arrive by
// coalesced loads (16 lanes per 256-byte row) and pass through LDS, padded to
// kKeyStride floats a row so that one row per thread reads back without bank
// conflicts; the value rows, loaded in the same first burst, wait in
// registers and take the keys' place once every score is computed. The
// softmax denominator is ordered_sum_wave's (the sequential sum's bits), and
// wave 0 divides and mixes from LDS. Three barriers in all.
constexpr uint32_t kStepLdsRows = 224;
static_assert(kStepLdsRows <= 256u, "ordered_sum_wave4 sums at most 256 values");
constexpr uint32_t kKeyStride = 68;

inline size_t attention_step_lds_bytes(uint32_t nk) {
  const uint32_t cap = 16u * nk;
  return 4u * (cap * kKeyStride + cap + wave_sum_floats(cap) + 64u + 8u);
}

template <uint32_t NK>  // rows <= 16 * NK
__global__ __launch_bounds__(kAttnThreads) void attention_step_lds_kernel(
    const float* qr, const float* kr, const float* vr, const float* rcos, const float* rsin, float* kcache,
    float* vcache, uint32_t kv, uint32_t group, float scale, uint32_t start, float* mixed) {
  constexpr uint32_t hd = 64u, cap = 16u * NK;
  extern __shared__ __align__(16) float sh[];
  float* ka = sh;                         // [cap][kKeyStride] keys, then [cap][64] values
  float* w = ka + cap * kKeyStride;       // [cap] softmax weights
  float* ws = w + cap;                    // the exps, in order
  float* qh = ws + wave_sum_floats(cap);  // [64] the rotated query
  float* red = qh + 64;                   // [8]
  const uint32_t h = blockIdx.x, tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t rows = start + 1u;
  const uint32_t off = (h / group) * hd;
  const bool appends = h % group == 0u;
  const float* vnew = vr + off;

  // RoPE inputs first (threads 0..31 the query's pairs, 32..63 the new
  // key's): loads return in issue order and the rotation needs only these
  float lo = 0.0f, hi = 0.0f, cs = 0.0f, sn = 0.0f;
  const uint32_t pair = tid & 31u;
  if (tid < 64u) {
    const float* src = tid < 32u ? qr + static_cast<size_t>(h) * hd : kr + off;
    lo = src[2u * pair];
    hi = src[2u * pair + 1u];
    cs = rcos[static_cast<size_t>(start) * (hd / 2u) + pair];
    sn = rsin[static_cast<size_t>(start) * (hd / 2u) + pair];
  }
  // chunk k of this thread: row (tid / 16) + 16k, floats 4 (tid % 16) ..;
  // rows from `start` on read row 0 (keys, not stored) or the new value row
  const uint32_t col = tid & 15u;
  f32x4 kc[NK], vc[NK];
#pragma unroll
  for (uint32_t k = 0; k < NK; k++) {
    const uint32_t row = (tid >> 4) + 16u * k;
    kc[k] = reinterpret_cast<const f32x4*>(kcache + static_cast<size_t>(row < start ? row : 0u) * kv + off)[col];
  }
#pragma unroll
  for (uint32_t k = 0; k < NK; k++) {
    const uint32_t row = (tid >> 4) + 16u * k;
    const float* src = row < start ? vcache + static_cast<size_t>(row) * kv + off : vnew;
    vc[k] = reinterpret_cast<const f32x4*>(src)[col];
  }
  __builtin_amdgcn_sched_barrier(0);

  // qkv_post_kernel's rotation: the query to qh, the new key to key row start
  if (tid < 64u) {
    const float hs = hi * sn, ls = lo * sn;
    const float nlo = __builtin_fmaf(lo, cs, -hs), nhi = __builtin_fmaf(hi, cs, ls);
    float* dst = tid < 32u ? qh : ka + start * kKeyStride;
    dst[2u * pair] = nlo;
    dst[2u * pair + 1u] = nhi;
  }
#pragma unroll
  for (uint32_t k = 0; k < NK; k++) {
    const uint32_t row = (tid >> 4) + 16u * k;
    if (row < start) reinterpret_cast<f32x4*>(ka + row * kKeyStride)[col] = kc[k];
  }
  __syncthreads();
  if (appends) {
    if (tid < 16u)
      reinterpret_cast<f32x4*>(kcache + static_cast<size_t>(start) * kv + off)[tid] =
          reinterpret_cast<const f32x4*>(ka + start * kKeyStride)[tid];
    else if (tid >= 64u && tid < 80u)
      reinterpret_cast<f32x4*>(vcache + static_cast<size_t>(start) * kv + off)[tid - 64u] =
          reinterpret_cast<const f32x4*>(vnew)[tid - 64u];
  }

  // thread i scores row i (rows <= cap <= the workgroup's threads)
  float sc = 0.0f, mx = -INFINITY;
  if (tid < rows) {
    f32x4 kk[16];
#pragma unroll
    for (int c = 0; c < 16; c++) kk[c] = reinterpret_cast<const f32x4*>(ka + tid * kKeyStride)[c];
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    lanes64(qh, kk, acc);
    sc = score_from_lanes(acc, -0.0f, scale);
    mx = fmaxf(mx, sc);
  }
  // softmax_rows' maximum
  mx = max_key_float(half_max_u32(max_key(mx)));
  mx = fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(mx), 0)),
             __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mx), 32)));
  if (lane == 0) red[wave] = mx;
  __syncthreads();  // and every key has been read
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
#pragma unroll
  for (uint32_t k = 0; k < NK; k++) {
    const uint32_t row = (tid >> 4) + 16u * k;
    reinterpret_cast<f32x4*>(ka + row * 64u)[col] = vc[k];
  }
  // the exps in order, -0.0 (the sum's identity) up to a multiple of 4
  if (tid < rows)
    ws[tid] = expf_ref(sc - mx);
  else if (tid < ((rows + 3u) & ~3u))
    ws[tid] = -0.0f;
  __syncthreads();
  if (wave != 0) return;
  // portable/norm.rs: the sum from 0.0 in order (runs of 4 a lane: rows <=
  // 256), then each exp over it
  const float sum = ordered_sum_wave4(ws, rows, 0.0f);
  for (uint32_t i = lane; i < rows; i += 64u) w[i] = __fdiv_rn(ws[i], sum);
  mixed[static_cast<size_t>(h) * hd + lane] = mix_lds(ka, w, rows, lane);
}

// hf[t][e] = silu(gate) * up, both stored by weight row (x[e*n + t])
// (feed_forward.rs:51-66, portable/elementwise.rs:6-9).
__global__ __launch_bounds__(256) void silu_mul_kernel(const float* gate, const float* up, uint32_t n, uint32_t len,
                                                       float* hf) {
  const size_t i = static_cast<size_t>(blockIdx.x) * 256u + threadIdx.x;
  if (i >= static_cast<size_t>(n) * len) return;
  const uint32_t t = static_cast<uint32_t>(i / len), e = static_cast<uint32_t>(i % len);
  const float g = gate[static_cast<size_t>(e) * n + t];
  const float den = 1.0f + expf_ref(-g);
  const float s = __fdiv_rn(g, den);
  hf[i] = s * up[static_cast<size_t>(e) * n + t];
}

// silu_mul_kernel's values for tokens t0 .. t0+3 (t0 = 4 blockIdx.y) of the
// 256-value block blockIdx.x, quantized to Q8_K into q as quantize_super_kernel
// would from hf: one launch instead of two, and hf never leaves the chip.
// Thread i reads weight row 256 blockIdx.x + i of gate and up, the four
// tokens side by side (one 16-byte load when n is a multiple of 4; TM: gate
// and up token-major, rows of fw values, so each token's load runs along
// the rows); wave w then quantizes token t0 + w's block from LDS.
template <bool TM>
__global__ __launch_bounds__(256) void silu_quant_kernel(const float* gate, const float* up, uint32_t n, uint32_t fw,
                                                         Q8Dev q) {
  __shared__ __align__(16) float blk[4][256];
  const uint32_t tid = threadIdx.x, sb = blockIdx.x, t0 = 4u * blockIdx.y;
  const size_t at = static_cast<size_t>(sb * 256u + tid) * n + t0;
  float g[4], u[4];
  if constexpr (TM) {
#pragma unroll
    for (uint32_t j = 0; j < 4u; j++) {
      // tokens past n read token n - 1 (wave j then stores nothing)
      const size_t o = static_cast<size_t>(min(t0 + j, n - 1u)) * fw + sb * 256u + tid;
      g[j] = gate[o];
      u[j] = up[o];
    }
  } else if ((n & 3u) == 0) {
    const float4 gv = *reinterpret_cast<const float4*>(gate + at);
    const float4 uv = *reinterpret_cast<const float4*>(up + at);
    g[0] = gv.x, g[1] = gv.y, g[2] = gv.z, g[3] = gv.w;
    u[0] = uv.x, u[1] = uv.y, u[2] = uv.z, u[3] = uv.w;
  } else {
#pragma unroll
    for (uint32_t j = 0; j < 4u; j++) {
      const bool in = t0 + j < n;
      g[j] = in ? gate[at + j] : 0.0f;
      u[j] = in ? up[at + j] : 0.0f;
    }
  }
#pragma unroll
  for (uint32_t j = 0; j < 4u; j++) {
    const float den = 1.0f + expf_ref(-g[j]);
    blk[j][tid] = __fdiv_rn(g[j], den) * u[j];
  }
  __syncthreads();
  const uint32_t w = tid >> 6, lane = tid & 63u;
  if (t0 + w >= n) return;
  const float4 v = reinterpret_cast<const float4*>(blk[w])[lane];
  const float f[4] = {v.x, v.y, v.z, v.w};
  quantize_super_block(f, lane, t0 + w, sb, q);
}


// Greedy pick over the logits: NaN as -inf, max by total order, the last
// maximum wins; out[0] = token, out[1] = 1 when some logit is finite. When
// `tokens` is given the token is also appended at tokens[count[0]] (the
// generation's record), count[0] advanced, and count[1] set for good once a
// pick finds no finite logit. When `hidden` is given, the picked token's
// embedding row (token_embd's type emb_type at emb_data, row pitch
// emb_pitch as matrix_pitch gives it) is
// written there: the next step's input.
// Each thread issues all of its loads (32 a pass, clamped into range) before
// it looks at any, and the record's count is read first of all: the pick
// waits on one memory round trip, not one per eight loads.
// The pick's end over a 1024-thread workgroup, each thread holding the best
// code and the finite flag of its share: the workgroup's maximum goes to
// out / the record, and (hidden set) the picked row of token_embd to hidden.
__device__ __forceinline__ void pick_finish(uint64_t best, uint32_t fin, uint32_t cnt, uint32_t* out,
                                            uint32_t* tokens, uint32_t* count, uint32_t emb_type,
                                            const uint8_t* emb_data, size_t emb_pitch, uint32_t width,
                                            float* hidden) {
  __shared__ uint32_t shi[16], slo[16], sfin[16];
  __shared__ uint32_t s_pick;
  best = wave_max_code(best);
  fin = __ballot(fin != 0u) ? 1u : 0u;
  const uint32_t wv = threadIdx.x >> 6;
  if ((threadIdx.x & 63u) == 0) {
    shi[wv] = static_cast<uint32_t>(best >> 32);
    slo[wv] = static_cast<uint32_t>(best);
    sfin[wv] = fin;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t b = 0;
    uint32_t f = 0;
    for (uint32_t w = 0; w < 16u; w++) {
      const uint64_t c = (static_cast<uint64_t>(shi[w]) << 32) | slo[w];
      b = c > b ? c : b;
      f |= sfin[w];
    }
    const uint32_t idx = static_cast<uint32_t>(b);
    out[0] = idx;
    out[1] = f;
    if (tokens) {
      tokens[cnt] = idx;
      count[0] = cnt + 1u;
      if (!f) count[1] = 1u;
    }
    s_pick = idx;
  }
  if (!hidden) return;  // uniform
  __syncthreads();
  for (uint32_t e = threadIdx.x; e < width; e += 1024u) hidden[e] = embed_value(emb_type, emb_data, emb_pitch, s_pick, e);
}

__global__ __launch_bounds__(1024) void argmax_kernel(const float* logits, uint32_t n, uint32_t* out,
                                                      uint32_t* tokens, uint32_t* count, uint32_t emb_type,
                                                      const uint8_t* emb_data, size_t emb_pitch, uint32_t width,
                                                      float* hidden) {
  constexpr uint32_t kPer = 32;
  uint32_t cnt = 0;
  if (tokens && threadIdx.x == 0) cnt = count[0];
  uint64_t best = 0;
  uint32_t fin = 0;
  for (uint32_t base = 0; base < n; base += kPer * 1024u) {  // uniform
    float v[kPer];
#pragma unroll
    for (uint32_t j = 0; j < kPer; j++) {
      const uint32_t i = base + threadIdx.x + j * 1024u;
      v[j] = logits[i < n ? i : n - 1u];
    }
#pragma unroll
    for (uint32_t j = 0; j < kPer; j++) {
      const uint32_t i = base + threadIdx.x + j * 1024u;
      const bool in = i < n;
      fin |= in && __builtin_isfinite(v[j]) ? 1u : 0u;
      const uint64_t c = pick_code(total_key(v[j] != v[j] ? -INFINITY : v[j]), i);
      best = in && c > best ? c : best;
    }
  }
  pick_finish(best, fin, cnt, out, tokens, count, emb_type, emb_data, emb_pitch, width, hidden);
}

// The same pick from the output launch's per-workgroup partials (PickPart,
// written by the norm-fused output GEMV): n records of 16 bytes instead of
// every logit. The maximum of maxima is the maximum, in the same order.
__global__ __launch_bounds__(1024) void argmax_parts_kernel(const PickPart* parts, uint32_t n, uint32_t* out,
                                                            uint32_t* tokens, uint32_t* count, uint32_t emb_type,
                                                            const uint8_t* emb_data, size_t emb_pitch,
                                                            uint32_t width, float* hidden) {
  uint32_t cnt = 0;
  if (tokens && threadIdx.x == 0) cnt = count[0];
  uint64_t best = 0;
  uint32_t fin = 0;
  for (uint32_t i = threadIdx.x; i < n; i += 1024u) {
    const PickPart p = parts[i];
    best = p.code > best ? p.code : best;
    fin |= p.fin;
  }
  pick_finish(best, fin, cnt, out, tokens, count, emb_type, emb_data, emb_pitch, width, hidden);
}

// the float functions of the kernels above, one per element (test hook)
__global__ __launch_bounds__(256) void math_kernel(uint32_t op, const float* a, const float* b, float* y, size_t n) {
  const size_t i = static_cast<size_t>(blockIdx.x) * 256u + threadIdx.x;
  if (i >= n) return;
  if (op == RH_MATH_EXPF) y[i] = expf_ref(a[i]);
  else if (op == RH_MATH_SQRT) y[i] = sqrt_rn(a[i]);
  else y[i] = __fdiv_rn(a[i], b[i]);
}

// One wave: values[0..n) into the ordered sum's LDS layout, then the sum.
__global__ __launch_bounds__(64) void ordered_sum_kernel(const float* values, uint32_t n, float init, float* out,
                                                         uint32_t* rounds) {
  extern __shared__ __align__(16) float buf[];
  const uint32_t padded = (n + 31u) & ~31u;
  for (uint32_t i = threadIdx.x; i < padded; i += 64u) buf[wave_sum_index(i)] = i < n ? values[i] : -0.0f;
  __syncthreads();
  const float s = ordered_sum_wave(buf, n, init, rounds);
  if (threadIdx.x == 0) *out = s;
}

constexpr size_t kMaxOrderedSumTest = 8192;

// ordered_sum_wave4 over values[0..n), n <= 256, in its plain layout.
__global__ __launch_bounds__(64) void ordered_sum4_kernel(const float* values, uint32_t n, float init, float* out,
                                                          uint32_t* rounds) {
  __shared__ __align__(16) float buf[256];
  for (uint32_t i = threadIdx.x; i < 256u; i += 64u) buf[i] = i < n ? values[i] : -0.0f;
  __syncthreads();
  const float s = ordered_sum_wave4(buf, n, init, rounds);
  if (threadIdx.x == 0) *out = s;
}

}  // namespace
}  // namespace rh

using namespace rh;

struct rh_decoder {
  rh_ctx* ctx = nullptr;
  int device = 0;  // freeing needs no live context
  hipStream_t stream = nullptr;
  rh_decoder_config c{};
  struct Block {
    const rh_matrix *q, *k, *v, *o, *gate, *up, *down;
    float *attn_norm, *ffn_norm;
  };
  std::vector<Block> blocks;
  const rh_matrix* token_embd = nullptr;
  const rh_matrix* output = nullptr;
  float* output_norm = nullptr;
  float *rope_cos = nullptr, *rope_sin = nullptr;
  float *keys = nullptr, *values = nullptr;
  size_t kv = 0;
  size_t cached = 0;  // positions stored in every layer
  // activations for up to `cap` tokens
  size_t cap = 0;
  float *hidden = nullptr, *normed = nullptr, *delta = nullptr, *qr = nullptr, *kr = nullptr, *vr = nullptr;
  float* hidden2 = nullptr;  // the residual's other buffer on the norm-fused path
  bool fuse_norm = false;    // one-token forwards fold each RMSNorm into the GEMV after it
  bool quant_norm = false;   // batches quantize the normed rows in the norm kernel
  bool quant_ffn = false;    // batches quantize silu(gate) * up in silu_quant_kernel
  bool quant_attn = false;   // batches quantize the attention output in attention_group_kernel
  bool fuse_output_norm = false;  // one-token forwards fold the output norm into the output matrix's launch
  Q8Dev q8;                  // that activation, for up to `cap` tokens
  float *q = nullptr, *mixed = nullptr, *gate = nullptr, *up = nullptr, *hf = nullptr;
  float* logits = nullptr;
  uint32_t* tokens = nullptr;  // the chunk's token ids
  uint32_t* pick = nullptr;    // argmax: [token, any finite]
  // the output launch's per-workgroup pick partials, and how many the last
  // one-token forward wrote (0: none; the pick then reads the logits)
  PickPart* pick_parts = nullptr;
  uint32_t pick_n = 0;
  uint32_t* record = nullptr;  // generated tokens
  uint32_t* count = nullptr;   // [recorded, a pick found no finite logit]
  size_t record_cap = 0;
  // graphs of batched forwards, keyed by (tokens, start), each valid while
  // the buffers whose addresses it captured stay where they are
  struct Graph {
    size_t n, start;
    uint64_t ctx_gen, acts_gen, used;
    hipGraphExec_t exec;
  };
  std::vector<Graph> graphs;
  uint64_t acts_gen = 0, graph_clock = 0;
  bool use_graphs = false;
};

namespace {

constexpr size_t kPrefillChunk = 64;  // model/src/generate.rs:70

bool is_kquant_matrix(const rh_matrix* m) {
  const uint32_t t = rh_matrix_type(m);
  return t == RH_TYPE_Q4_K || t == RH_TYPE_Q6_K;
}

template <typename T>
hipError_t dmalloc(T** p, size_t n) {
  return hipMalloc(reinterpret_cast<void**>(p), (n ? n : 1) * sizeof(T));
}

// Destroys a graph exec once no replay of it can still be queued: work on
// the decoder's stream (a replay launched earlier in the same call) drains
// first.
void destroy_exec(rh_decoder* d, hipGraphExec_t exec) {
  hipStreamSynchronize(d->stream);
  hipGraphExecDestroy(exec);
}

void drop_graphs(rh_decoder* d) {
  for (rh_decoder::Graph& g : d->graphs) destroy_exec(d, g.exec);
  d->graphs.clear();
}

void free_acts(rh_decoder* d) {
  drop_graphs(d);
  d->acts_gen++;
  if (d->hidden2) hipFree(d->hidden2);
  d->hidden2 = nullptr;
  for (void* p : {static_cast<void*>(d->hidden), static_cast<void*>(d->normed), static_cast<void*>(d->delta),
                  static_cast<void*>(d->qr), static_cast<void*>(d->kr), static_cast<void*>(d->vr),
                  static_cast<void*>(d->q), static_cast<void*>(d->mixed), static_cast<void*>(d->gate),
                  static_cast<void*>(d->up), static_cast<void*>(d->hf), static_cast<void*>(d->tokens),
                  static_cast<void*>(d->q8.quants), static_cast<void*>(d->q8.scales), static_cast<void*>(d->q8.sums),
                  static_cast<void*>(d->q8.sums16)})
    if (p) hipFree(p);
  d->q8 = Q8Dev{};
  d->hidden = d->normed = d->delta = d->qr = d->kr = d->vr = d->q = d->mixed = d->gate = d->up = d->hf = nullptr;
  d->tokens = nullptr;
  d->cap = 0;
}

hipError_t ensure_acts(rh_decoder* d, size_t n) {
  if (d->cap >= n) return hipSuccess;
  hipError_t e = hipStreamSynchronize(d->stream);
  if (e != hipSuccess) return e;
  free_acts(d);
  const size_t w = d->c.embedding_length, f = d->c.feed_forward_length, kv = d->kv;
  if ((e = dmalloc(&d->hidden, n * w)) != hipSuccess || (e = dmalloc(&d->normed, n * w)) != hipSuccess ||
      (e = dmalloc(&d->delta, n * w)) != hipSuccess || (e = dmalloc(&d->qr, n * w)) != hipSuccess ||
      (e = dmalloc(&d->kr, n * kv)) != hipSuccess || (e = dmalloc(&d->vr, n * kv)) != hipSuccess ||
      (e = dmalloc(&d->q, n * w)) != hipSuccess || (e = dmalloc(&d->mixed, n * w)) != hipSuccess ||
      (e = dmalloc(&d->gate, n * f)) != hipSuccess || (e = dmalloc(&d->up, n * f)) != hipSuccess ||
      (e = dmalloc(&d->hf, n * f)) != hipSuccess || (e = dmalloc(&d->tokens, n)) != hipSuccess ||
      (e = dmalloc(&d->hidden2, w)) != hipSuccess) {
    free_acts(d);
    return e;
  }
  // the Q8_K activation of a batch (the layout ensure_q8 gives matmul_batch),
  // wide enough for either matrix input: a normed row (w) or the FFN's (f)
  const size_t wq = w > f ? w : f;
  const size_t qstride = (wq + 255u) / 256u * 256u, bstride = (qstride / 32u + 7u) / 8u * 8u;
  if ((e = dmalloc(&d->q8.quants, n * qstride)) != hipSuccess ||
      (e = dmalloc(&d->q8.scales, n * bstride)) != hipSuccess || (e = dmalloc(&d->q8.sums, n * bstride)) != hipSuccess ||
      (e = dmalloc(&d->q8.sums16, 2 * n * bstride)) != hipSuccess) {
    free_acts(d);
    return e;
  }
  d->q8.qstride = qstride;
  d->q8.bstride = bstride;
  d->q8.n_blocks = w / 256u * 8u;
  d->cap = n;
  return hipSuccess;
}

rh_status mm(rh_decoder* d, const float* in, size_t n, size_t width, std::initializer_list<rh_job> jobs) {
  std::vector<rh_job> v(jobs);
  return rh_matmul_batch_device(d->ctx, in, n * width, n, v.data(), v.size(), d->stream);
}

// The decoder's Q8_K activation as rows of `width` values (a multiple of 256).
Q8Dev q8_for(const rh_decoder* d, size_t width) {
  Q8Dev q = d->q8;
  q.n_blocks = width / 256u * 8u;
  return q;
}

// mm over the decoder's Q8_K activation (d->q8, which a QUANT norm or
// silu_quant_kernel filled) for rows of `width` values.
// defer: a split launch leaves its token-major planes there (SplitOut).
rh_status mm_q8(rh_decoder* d, size_t n, size_t width, std::initializer_list<rh_job> jobs, bool token_major = false,
                SplitOut* defer = nullptr) {
  std::vector<rh_job> v(jobs);
  return matmul_q8_device(d->ctx, q8_for(d, width), width, n, v.data(), v.size(), d->stream, token_major, defer);
}

#define RHD(expr)                                   \
  do {                                              \
    hipError_t e_ = (expr);                         \
    if (e_ != hipSuccess) return RH_ERR_DEVICE;     \
  } while (0)
#define RHS(expr)                                   \
  do {                                              \
    rh_status s_ = (expr);                          \
    if (s_ != RH_OK) return s_;                     \
  } while (0)

// Decoder::forward_on_pool (decoder.rs:74-107) for n tokens whose ids are
// in device memory at `tokens`, at positions start..start+n; leaves the last token's
// logits in d->logits.
rh_status forward_one_fused(rh_decoder* d, const uint32_t* tokens, size_t start, bool embedded);

// `embedded`: a one-token forward on the norm-fused path whose embedding row
// the greedy pick already wrote to hidden.
rh_status forward_device(rh_decoder* d, const uint32_t* tokens, size_t n, size_t start, bool embedded = false) {
  d->pick_n = 0;  // set again by a one-token output launch that writes pick partials
  if (n == 1 && d->fuse_norm) return forward_one_fused(d, tokens, start, embedded);
  const rh_decoder_config& c = d->c;
  const uint32_t w = static_cast<uint32_t>(c.embedding_length), kv = static_cast<uint32_t>(d->kv);
  const uint32_t f = static_cast<uint32_t>(c.feed_forward_length), hd = static_cast<uint32_t>(c.head_dim);
  const uint32_t nn = static_cast<uint32_t>(n);
  hipStream_t s = d->stream;
  const rh_matrix* E = d->token_embd;
  hipLaunchKernelGGL(embed_kernel, dim3((w + 255u) / 256u, nn), dim3(256), 0, s, rh_matrix_type(E),
                     matrix_data(E), matrix_pitch(E), tokens, w, d->hidden);
  RHD(hipGetLastError());
  const float scale = ::sqrtf(static_cast<float>(c.head_dim));
  const size_t norm_lds = add_norm_lds(w);
  const uint32_t grp = static_cast<uint32_t>(c.head_count / c.head_count_kv);
  const size_t glds = attention_group_lds_floats(grp, start + n) * 4u;
  const bool grouped = hd == 64u && (grp == 4u || grp == 8u) && glds <= kMaxLdsBytes;
  // when both producers of the residual delta (the O and down matrices) are
  // k-quant GEMMs over Q8_K operands, they store it token-major and the
  // norms read it coalesced
  const bool tm = grouped && d->quant_attn && d->quant_ffn && n >= rh_gemm_min_tokens();
  const AddNorm norm_fn = tm ? add_norm_for<false, true>(w) : add_norm_for(w);
  // a batch whose normed rows feed only k-quant GEMMs gets them as Q8_K
  // straight from the norm kernel
  const bool qn = d->quant_norm && n >= 2;
  // with those and the token-major path, the QKV GEMM stores q, k and v
  // token-major too and the grouped attention does qkv_post_kernel's work
  const bool rope_in_attn = tm && qn;
  const AddNorm norm_in = qn ? (tm ? add_norm_for<true, true>(w) : add_norm_for<true>(w)) : norm_fn;
  // the FFN norm that sums a split O launch's planes itself (no combine)
  const AddNorm norm_pl = qn ? add_norm_for<true, true, true>(w) : add_norm_for<false, true, true>(w);
  const float* pending = nullptr;  // the residual the next norm adds first
  for (size_t l = 0; l < d->blocks.size(); l++) {
    const rh_decoder::Block& b = d->blocks[l];
    hipLaunchKernelGGL(norm_in.fn, dim3(nn), dim3(norm_in.threads), norm_lds, s, d->hidden, pending, nn, w,
                       b.attn_norm, c.rms_norm_eps, 0u, d->normed, d->q8, nullptr, 0u, 0u);
    RHD(hipGetLastError());
    if (qn)
      RHS(mm_q8(d, n, w, {{b.q, d->qr, n * w}, {b.k, d->kr, n * kv}, {b.v, d->vr, n * kv}}, rope_in_attn));
    else
      RHS(mm(d, d->normed, n, w, {{b.q, d->qr, n * w}, {b.k, d->kr, n * kv}, {b.v, d->vr, n * kv}}));
    float* kc = d->keys + l * c.context_length * kv;
    float* vc = d->values + l * c.context_length * kv;
    SplitOut o_planes;
    if (!rope_in_attn) {
      const uint32_t work = w / 2u + kv / 2u + kv;
      hipLaunchKernelGGL(qkv_post_kernel, dim3((work + 255u) / 256u, nn), dim3(256), 0, s, d->qr, d->kr, d->vr, nn,
                         w, kv, hd, d->rope_cos, d->rope_sin, static_cast<uint32_t>(start), d->q, kc, vc);
      RHD(hipGetLastError());
    }
    if (grouped) {
      // the kv head's query heads together; the output as the O matrix's
      // Q8_K operand when it takes one
      const bool qa = d->quant_attn;
      AttnGroupFn fn;
      if (grp == 8u)
        fn = rope_in_attn ? attention_group_kernel<8, true, true>
                          : qa ? attention_group_kernel<8, true, false> : attention_group_kernel<8, false, false>;
      else
        fn = rope_in_attn ? attention_group_kernel<4, true, true>
                          : qa ? attention_group_kernel<4, true, false> : attention_group_kernel<4, false, false>;
      hipLaunchKernelGGL(fn, dim3(static_cast<uint32_t>(c.head_count_kv), nn), dim3(kAttnThreads), glds, s,
                         rope_in_attn ? d->qr : d->q, kc, vc, w, kv, scale, static_cast<uint32_t>(start), d->mixed,
                         q8_for(d, w), d->kr, d->vr, d->rope_cos, d->rope_sin);
      RHD(hipGetLastError());
      if (qa)
        RHS(mm_q8(d, n, w, {{b.o, d->delta, n * w}}, tm, tm ? &o_planes : nullptr));
      else
        RHS(mm(d, d->mixed, n, w, {{b.o, d->delta, n * w}}));
    } else {
      const size_t att_lds = attention_lds_floats(start + n) * 4u;
      hipLaunchKernelGGL(hd == 64u ? attention_kernel<64> : attention_kernel<0>,
                         dim3(static_cast<uint32_t>(c.head_count), nn), dim3(kAttnThreads), att_lds, s, d->q, kc,
                         vc, w, kv, hd, grp, scale, static_cast<uint32_t>(start), d->mixed);
      RHD(hipGetLastError());
      RHS(mm(d, d->mixed, n, w, {{b.o, d->delta, n * w}}));
    }
    if (o_planes.planes)
      hipLaunchKernelGGL(norm_pl.fn, dim3(nn), dim3(norm_pl.threads), norm_lds, s, d->hidden, nullptr, nn, w,
                         b.ffn_norm, c.rms_norm_eps, 0u, d->normed, d->q8, o_planes.terms, o_planes.planes,
                         o_planes.rows_pad);
    else
      hipLaunchKernelGGL(norm_in.fn, dim3(nn), dim3(norm_in.threads), norm_lds, s, d->hidden, d->delta, nn, w,
                         b.ffn_norm, c.rms_norm_eps, 0u, d->normed, d->q8, nullptr, 0u, 0u);
    RHD(hipGetLastError());
    if (qn)
      RHS(mm_q8(d, n, w, {{b.gate, d->gate, n * f}, {b.up, d->up, n * f}}, tm));
    else
      RHS(mm(d, d->normed, n, w, {{b.gate, d->gate, n * f}, {b.up, d->up, n * f}}));
    if (d->quant_ffn && n >= 2) {
      // gate and up are token-major where the k-quant GEMM stored them so
      hipLaunchKernelGGL(tm && qn ? silu_quant_kernel<true> : silu_quant_kernel<false>,
                         dim3(f / 256u, (nn + 3u) / 4u),
                         dim3(256), 0, s, d->gate, d->up, nn, f, q8_for(d, f));
      RHD(hipGetLastError());
      RHS(mm_q8(d, n, f, {{b.down, d->delta, n * w}}, tm));
    } else {
      const size_t total = n * f;
      hipLaunchKernelGGL(silu_mul_kernel, dim3(static_cast<uint32_t>((total + 255u) / 256u)), dim3(256), 0, s,
                         d->gate, d->up, nn, f, d->hf);
      RHD(hipGetLastError());
      RHS(mm(d, d->hf, n, f, {{b.down, d->delta, n * w}}));
    }
    pending = d->delta;
  }
  // the last residual for every token, then the last token's output norm
  hipLaunchKernelGGL(norm_fn.fn, dim3(nn), dim3(norm_fn.threads), norm_lds, s, d->hidden, pending, nn, w,
                     d->output_norm, c.rms_norm_eps, nn - 1u, d->normed, Q8Dev{}, nullptr, 0u, 0u);
  RHD(hipGetLastError());
  const rh_matrix* out = d->output ? d->output : d->token_embd;
  RHS(mm(d, d->normed, 1, w, {{out, d->logits, c.vocab_size}}));
  d->cached = start + n;
  return RH_OK;
}

// forward_device for one token with the layers' RMSNorms folded into the
// fused GEMV after them (NormIn): the residual h + delta is formed inside the
// QKV and gate/up launches, the first workgroup of each writing it to the
// other hidden buffer. Same arithmetic as the add_norm path, value for value.
rh_status forward_one_fused(rh_decoder* d, const uint32_t* tokens, size_t start, bool embedded) {
  const rh_decoder_config& c = d->c;
  const uint32_t w = static_cast<uint32_t>(c.embedding_length), kv = static_cast<uint32_t>(d->kv);
  const uint32_t f = static_cast<uint32_t>(c.feed_forward_length), hd = static_cast<uint32_t>(c.head_dim);
  hipStream_t s = d->stream;
  const rh_matrix* E = d->token_embd;
  if (!embedded) {
    hipLaunchKernelGGL(embed_kernel, dim3((w + 255u) / 256u, 1u), dim3(256), 0, s, rh_matrix_type(E),
                       matrix_data(E), matrix_pitch(E), tokens, w, d->hidden);
    RHD(hipGetLastError());
  }
  const float scale = ::sqrtf(static_cast<float>(c.head_dim));
  float* h = d->hidden;
  float* h2 = d->hidden2;
  const float* pending = nullptr;  // the residual the next norm adds first
  for (size_t l = 0; l < d->blocks.size(); l++) {
    const rh_decoder::Block& b = d->blocks[l];
    NormIn an{};
    an.delta = pending;
    an.weight = b.attn_norm;
    an.eps = c.rms_norm_eps;
    an.hidden_out = pending ? h2 : nullptr;
    const rh_job qkv[3] = {{b.q, d->qr, w}, {b.k, d->kr, kv}, {b.v, d->vr, kv}};
    RHS(matmul_norm_device(d->ctx, h, an, w, qkv, 3, s));
    if (pending) std::swap(h, h2);
    float* kc = d->keys + l * c.context_length * kv;
    float* vc = d->values + l * c.context_length * kv;
    const size_t att_lds = attention_lds_floats(start + 1) * 4u;
    const uint32_t group = static_cast<uint32_t>(c.head_count / c.head_count_kv);
    if (hd == 64u && start + 1u <= kStepLdsRows && tuning().attn_lds) {
      // 16-row groups, rounded up to an even count: 7 kernels cover every row count
      const uint32_t nk = ((static_cast<uint32_t>(start) + 1u + 31u) / 32u) * 2u;
      void* k = nk == 2u ? reinterpret_cast<void*>(attention_step_lds_kernel<2>)
              : nk == 4u ? reinterpret_cast<void*>(attention_step_lds_kernel<4>)
              : nk == 6u ? reinterpret_cast<void*>(attention_step_lds_kernel<6>)
              : nk == 8u ? reinterpret_cast<void*>(attention_step_lds_kernel<8>)
              : nk == 10u ? reinterpret_cast<void*>(attention_step_lds_kernel<10>)
              : nk == 12u ? reinterpret_cast<void*>(attention_step_lds_kernel<12>)
                          : reinterpret_cast<void*>(attention_step_lds_kernel<14>);
      const float* qr = d->qr;
      const float* kr = d->kr;
      const float* vr = d->vr;
      const float* rc = d->rope_cos;
      const float* rs = d->rope_sin;
      uint32_t kv32 = static_cast<uint32_t>(kv), st = static_cast<uint32_t>(start);
      float sc = scale;
      uint32_t gr = group;
      float* mixed = d->mixed;
      void* args[] = {&qr, &kr, &vr, &rc, &rs, &kc, &vc, &kv32, &gr, &sc, &st, &mixed};
      RHD(hipLaunchKernel(k, dim3(static_cast<uint32_t>(c.head_count)), dim3(kAttnThreads), args,
                          attention_step_lds_bytes(nk), s));
    } else if (hd == 64u) {
      hipLaunchKernelGGL(attention_step_kernel, dim3(static_cast<uint32_t>(c.head_count)), dim3(kAttnThreads),
                         att_lds, s, d->qr, d->kr, d->vr, d->rope_cos, d->rope_sin, kc, vc, kv, group, scale,
                         static_cast<uint32_t>(start), d->mixed);
    } else {
      const uint32_t work = w / 2u + kv / 2u + kv;
      hipLaunchKernelGGL(qkv_post_kernel, dim3((work + 255u) / 256u, 1u), dim3(256), 0, s, d->qr, d->kr, d->vr, 1u,
                         w, kv, hd, d->rope_cos, d->rope_sin, static_cast<uint32_t>(start), d->q, kc, vc);
      RHD(hipGetLastError());
      hipLaunchKernelGGL(attention_kernel<0>, dim3(static_cast<uint32_t>(c.head_count), 1u), dim3(kAttnThreads),
                         att_lds, s, d->q, kc, vc, w, kv, hd, group, scale, static_cast<uint32_t>(start), d->mixed);
    }
    RHD(hipGetLastError());
    RHS(mm(d, d->mixed, 1, w, {{b.o, d->delta, w}}));
    NormIn fn{};
    fn.delta = d->delta;
    fn.weight = b.ffn_norm;
    fn.eps = c.rms_norm_eps;
    fn.hidden_out = h2;
    if (gate_up_pairable(b.gate, b.up, w)) {
      // gate and up rows side by side in one launch, which writes silu(gate) * up
      RHS(matmul_norm_silu_device(d->ctx, h, fn, w, b.gate, b.up, d->hf, f, s));
    } else {
      const rh_job gu[2] = {{b.gate, d->gate, f}, {b.up, d->up, f}};
      RHS(matmul_norm_device(d->ctx, h, fn, w, gu, 2, s));
      hipLaunchKernelGGL(silu_mul_kernel, dim3((f + 255u) / 256u), dim3(256), 0, s, d->gate, d->up, 1u, f, d->hf);
      RHD(hipGetLastError());
    }
    std::swap(h, h2);
    RHS(mm(d, d->hf, 1, f, {{b.down, d->delta, w}}));
    pending = d->delta;
  }
  // the output norm folds into the output matrix's launch as the layers'
  // norms do (eight blocks per team keep that grid on the chip at once);
  // an output matrix the norm-fused kernels cannot take keeps the separate
  // norm kernel
  const rh_matrix* out = d->output ? d->output : d->token_embd;
  if (d->fuse_output_norm) {
    NormIn fo{};
    fo.delta = pending;
    fo.weight = d->output_norm;
    fo.eps = c.rms_norm_eps;
    fo.pick = d->pick_parts;
    fo.grid_out = &d->pick_n;
    const rh_job lm{out, d->logits, c.vocab_size};
    RHS(matmul_norm_device(d->ctx, h, fo, w, &lm, 1, s));
  } else {
    const AddNorm an = add_norm_for(w);
    hipLaunchKernelGGL(an.fn, dim3(1), dim3(an.threads), add_norm_lds(w), s, h, pending, 1u, w, d->output_norm,
                       c.rms_norm_eps, 0u, d->normed, Q8Dev{}, nullptr, 0u, 0u);
    RHD(hipGetLastError());
    RHS(mm(d, d->normed, 1, w, {{out, d->logits, c.vocab_size}}));
  }
  d->cached = start + 1;
  return RH_OK;
}

}  // namespace

extern "C" {

void rh_rope_table_host(size_t positions, size_t columns, float theta, float* cos_out, float* sin_out) {
  const size_t pairs = columns / 2;
  for (size_t pos = 0; pos < positions; pos++)
    for (size_t p = 0; p < pairs; p++) {
      const float exponent = -static_cast<float>(2 * p) / static_cast<float>(columns);
      const float angle = static_cast<float>(pos) * ::powf(theta, exponent);
      cos_out[pos * pairs + p] = ::cosf(angle);
      sin_out[pos * pairs + p] = ::sinf(angle);
    }
}

void rh_expf_host(const float* x, float* y, size_t n) {
  for (size_t i = 0; i < n; i++) y[i] = expf_ref(x[i]);
}

void rh_sqrt_host(const float* x, const float* start, float* y, size_t n) {
  for (size_t i = 0; i < n; i++) y[i] = start ? sqrt_fix(x[i], start[i]) : sqrt_rn(x[i]);
}

rh_status rh_math_device(rh_ctx* ctx, uint32_t op, const float* a, const float* b, float* y, size_t n) {
  const bool binary = op == RH_MATH_DIV;
  if (!ctx || op > RH_MATH_DIV || (n && (!a || !y || (binary && !b)))) return RH_ERR_INVALID_ARGUMENT;
  if (n == 0) return RH_OK;
  if (hipSetDevice(ctx_device(ctx)) != hipSuccess) return RH_ERR_DEVICE;
  hipStream_t s = static_cast<hipStream_t>(rh_stream(ctx));
  float *da = nullptr, *db = nullptr, *dy = nullptr;
  if (dmalloc(&da, n) != hipSuccess || dmalloc(&dy, n) != hipSuccess || (binary && dmalloc(&db, n) != hipSuccess)) {
    hipFree(da);
    hipFree(dy);
    return RH_ERR_OUT_OF_MEMORY;
  }
  hipError_t e = hipMemcpyAsync(da, a, n * 4, hipMemcpyHostToDevice, s);
  if (e == hipSuccess && binary) e = hipMemcpyAsync(db, b, n * 4, hipMemcpyHostToDevice, s);
  if (e == hipSuccess) {
    hipLaunchKernelGGL(math_kernel, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0, s, op, da, db, dy,
                       n);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipMemcpyAsync(y, dy, n * 4, hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  hipFree(da);
  hipFree(db);
  hipFree(dy);
  return e == hipSuccess ? RH_OK : RH_ERR_DEVICE;
}

rh_status rh_ordered_sum_device(rh_ctx* ctx, const float* values, size_t n, float init, float* sum,
                                uint32_t* rounds) {
  if (!ctx || !sum || n > kMaxOrderedSumTest || (n && !values)) return RH_ERR_INVALID_ARGUMENT;
  if (hipSetDevice(ctx_device(ctx)) != hipSuccess) return RH_ERR_DEVICE;
  hipStream_t s = static_cast<hipStream_t>(rh_stream(ctx));
  float *dv = nullptr, *dout = nullptr;
  uint32_t* dr = nullptr;
  if (dmalloc(&dv, n + 1) != hipSuccess || dmalloc(&dout, 1) != hipSuccess ||
      hipMalloc(reinterpret_cast<void**>(&dr), 4) != hipSuccess) {
    hipFree(dv);
    hipFree(dout);
    return RH_ERR_OUT_OF_MEMORY;
  }
  hipError_t e = n ? hipMemcpyAsync(dv, values, n * 4, hipMemcpyHostToDevice, s) : hipSuccess;
  if (e == hipSuccess) e = hipMemsetAsync(dr, 0, 4, s);
  if (e == hipSuccess) {
    hipLaunchKernelGGL(ordered_sum_kernel, dim3(1), dim3(64), wave_sum_floats(static_cast<uint32_t>(n)) * 4u + 16u,
                       s, dv, static_cast<uint32_t>(n), init, dout, dr);
    e = hipGetLastError();
  }
  uint32_t r = 0;
  if (e == hipSuccess) e = hipMemcpyAsync(sum, dout, 4, hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipMemcpyAsync(&r, dr, 4, hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (rounds) *rounds = r;
  hipFree(dv);
  hipFree(dout);
  hipFree(dr);
  return e == hipSuccess ? RH_OK : RH_ERR_DEVICE;
}

rh_status rh_greedy_pick_device(rh_ctx* ctx, const float* logits, size_t n, uint32_t* token, uint32_t* finite) {
  if (!ctx || !token || !finite || n == 0 || n > 0xFFFFFFFFu || !logits) return RH_ERR_INVALID_ARGUMENT;
  if (hipSetDevice(ctx_device(ctx)) != hipSuccess) return RH_ERR_DEVICE;
  hipStream_t s = static_cast<hipStream_t>(rh_stream(ctx));
  float* dl = nullptr;
  uint32_t* dout = nullptr;
  if (dmalloc(&dl, n) != hipSuccess || hipMalloc(reinterpret_cast<void**>(&dout), 8) != hipSuccess) {
    hipFree(dl);
    return RH_ERR_OUT_OF_MEMORY;
  }
  hipError_t e = hipMemcpyAsync(dl, logits, n * 4, hipMemcpyHostToDevice, s);
  if (e == hipSuccess) {
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, s, dl, static_cast<uint32_t>(n), dout, nullptr, nullptr,
                       0u, nullptr, size_t{0}, 0u, nullptr);
    e = hipGetLastError();
  }
  uint32_t o[2] = {0, 0};
  if (e == hipSuccess) e = hipMemcpyAsync(o, dout, 8, hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  *token = o[0];
  *finite = o[1];
  hipFree(dl);
  hipFree(dout);
  return e == hipSuccess ? RH_OK : RH_ERR_DEVICE;
}

rh_status rh_ordered_sum4_device(rh_ctx* ctx, const float* values, size_t n, float init, float* sum,
                                 uint32_t* rounds) {
  if (!ctx || !sum || n > 256u || (n && !values)) return RH_ERR_INVALID_ARGUMENT;
  if (hipSetDevice(ctx_device(ctx)) != hipSuccess) return RH_ERR_DEVICE;
  hipStream_t s = static_cast<hipStream_t>(rh_stream(ctx));
  float *dv = nullptr, *dout = nullptr;
  uint32_t* dr = nullptr;
  if (dmalloc(&dv, n + 1) != hipSuccess || dmalloc(&dout, 1) != hipSuccess ||
      hipMalloc(reinterpret_cast<void**>(&dr), 4) != hipSuccess) {
    hipFree(dv);
    hipFree(dout);
    return RH_ERR_OUT_OF_MEMORY;
  }
  hipError_t e = n ? hipMemcpyAsync(dv, values, n * 4, hipMemcpyHostToDevice, s) : hipSuccess;
  if (e == hipSuccess) e = hipMemsetAsync(dr, 0, 4, s);
  if (e == hipSuccess) {
    hipLaunchKernelGGL(ordered_sum4_kernel, dim3(1), dim3(64), 0, s, dv, static_cast<uint32_t>(n), init, dout, dr);
    e = hipGetLastError();
  }
  uint32_t r = 0;
  if (e == hipSuccess) e = hipMemcpyAsync(sum, dout, 4, hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipMemcpyAsync(&r, dr, 4, hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (rounds) *rounds = r;
  hipFree(dv);
  hipFree(dout);
  hipFree(dr);
  return e == hipSuccess ? RH_OK : RH_ERR_DEVICE;
}

rh_status rh_decoder_new(rh_ctx* ctx, const rh_decoder_config* config, const rh_decoder_weights* weights,
                         rh_decoder** out) {
  if (!ctx || !config || !weights || !out || !weights->token_embd || !weights->output_norm || !weights->blocks)
    return RH_ERR_INVALID_ARGUMENT;
  *out = nullptr;
  const rh_decoder_config& c = *config;
  // DecoderConfig::validate (transformer/src/config.rs:55-80), plus this
  // kernel set's limits: head_dim <= 128, embedding_length <= 8192, attention
  // weights for the whole context in one workgroup's LDS (160 KiB on gfx950:
  // context_length <= 32,576), f32/Q4_K/Q6_K embedding rows
  int lds_max = 0;
  if (hipSetDevice(ctx_device(ctx)) != hipSuccess ||
      hipDeviceGetAttribute(&lds_max, hipDeviceAttributeMaxSharedMemoryPerBlock, ctx_device(ctx)) != hipSuccess)
    return RH_ERR_DEVICE;
  if (c.head_count == 0 || c.head_count_kv == 0 || c.head_count % c.head_count_kv != 0 || c.head_dim == 0 ||
      c.head_dim % 2 != 0 || c.head_count * c.head_dim != c.embedding_length || c.block_count == 0 ||
      c.feed_forward_length == 0 || c.context_length == 0 || c.vocab_size == 0 || c.head_dim > kMaxHeadDim ||
      c.embedding_length > kMaxNormPer * kNormThreads ||
      attention_lds_floats(c.context_length) * 4u > static_cast<size_t>(lds_max))
    return RH_ERR_INVALID_CONFIG;
  const uint32_t et = rh_matrix_type(weights->token_embd);
  if ((et != RH_TYPE_F32 && et != RH_TYPE_Q4_K && et != RH_TYPE_Q6_K) ||
      rh_matrix_cols(weights->token_embd) != c.embedding_length || rh_matrix_rows(weights->token_embd) < c.vocab_size)
    return RH_ERR_SHAPE_MISMATCH;
  if (hipSetDevice(ctx_device(ctx)) != hipSuccess) return RH_ERR_DEVICE;
  rh_decoder* d = new (std::nothrow) rh_decoder();
  if (!d) return RH_ERR_OUT_OF_MEMORY;
  d->ctx = ctx;
  d->device = ctx_device(ctx);
  d->stream = static_cast<hipStream_t>(rh_stream(ctx));
  d->c = c;
  d->kv = c.head_count_kv * c.head_dim;
  d->token_embd = weights->token_embd;
  d->output = weights->output;
  const size_t w = c.embedding_length;
  auto upload = [&](const float* host, float** dev) -> bool {
    return dmalloc(dev, w) == hipSuccess &&
           hipMemcpy(*dev, host, w * 4, hipMemcpyHostToDevice) == hipSuccess;
  };
  bool ok = upload(weights->output_norm, &d->output_norm);
  for (size_t l = 0; ok && l < c.block_count; l++) {
    const rh_decoder_block& b = weights->blocks[l];
    rh_decoder::Block x{b.attn_q, b.attn_k, b.attn_v, b.attn_output, b.ffn_gate, b.ffn_up, b.ffn_down, nullptr,
                        nullptr};
    ok = b.attn_q && b.attn_k && b.attn_v && b.attn_output && b.ffn_gate && b.ffn_up && b.ffn_down &&
         b.attn_norm && b.ffn_norm && upload(b.attn_norm, &x.attn_norm) && upload(b.ffn_norm, &x.ffn_norm);
    d->blocks.push_back(x);
  }
  // RoPE angles for every position, with the host libm (portable/rope.rs:7-23)
  const size_t pairs = c.head_dim / 2;
  std::vector<float> hc(c.context_length * pairs), hs(c.context_length * pairs);
  rh_rope_table_host(c.context_length, c.head_dim, c.rope_freq_base, hc.data(), hs.data());
  ok = ok && dmalloc(&d->rope_cos, hc.size()) == hipSuccess && dmalloc(&d->rope_sin, hs.size()) == hipSuccess &&
       hipMemcpy(d->rope_cos, hc.data(), hc.size() * 4, hipMemcpyHostToDevice) == hipSuccess &&
       hipMemcpy(d->rope_sin, hs.data(), hs.size() * 4, hipMemcpyHostToDevice) == hipSuccess;
  const size_t cache = c.block_count * c.context_length * d->kv;
  ok = ok && dmalloc(&d->keys, cache) == hipSuccess && dmalloc(&d->values, cache) == hipSuccess &&
       dmalloc(&d->logits, c.vocab_size) == hipSuccess && dmalloc(&d->pick, 2) == hipSuccess &&
       dmalloc(&d->pick_parts, c.vocab_size) == hipSuccess &&
       dmalloc(&d->count, 2) == hipSuccess;
  if (!ok) {
    rh_decoder_free(d);
    return RH_ERR_OUT_OF_MEMORY;
  }
  // one-token forwards fold the norms into the GEMVs when every normed
  // projection is a k-quant matrix that takes the whole row in its preload;
  // RUSTICIDE_HIP_NORM_FUSE=0 keeps the separate norm kernels (same bits)
  auto fusable = [&](const rh_matrix* m) {
    const uint32_t t = rh_matrix_type(m);
    return rh_matrix_cols(m) == w && norm_fusable(t, w, static_cast<uint32_t>(w / 256u));
  };
  bool fuse = true;
  for (const rh_decoder::Block& b : d->blocks)
    fuse = fuse && fusable(b.q) && fusable(b.k) && fusable(b.v) && fusable(b.gate) && fusable(b.up);
  const char* env = std::getenv("RUSTICIDE_HIP_NORM_FUSE");
  d->fuse_norm = fuse && !(env && env[0] == '0');
  // batches quantize the normed rows in the norm kernel when every matrix
  // reading them is a k-quant GEMM operand; RUSTICIDE_HIP_NORM_QUANT=0 keeps
  // the f32 rows and matmul_batch's own quantize (same bits)
  bool quant = w % 256 == 0;
  for (const rh_decoder::Block& b : d->blocks)
    for (const rh_matrix* m : {b.q, b.k, b.v, b.gate, b.up})
      quant = quant && is_kquant_matrix(m) && rh_matrix_cols(m) == w;
  const rh_matrix* om = d->output ? d->output : d->token_embd;
  d->fuse_output_norm = d->fuse_norm && fusable(om);
  // graphs of batched forwards are opt-in (RUSTICIDE_HIP_GRAPHS=1): on
  // ROCm 7.2 replaying the ~290 launches of a 64-token prefill as a graph
  // takes as long as issuing them (3.30 against 3.25 ms)
  const char* genv = std::getenv("RUSTICIDE_HIP_GRAPHS");
  d->use_graphs = genv && genv[0] == '1';
  const char* qenv = std::getenv("RUSTICIDE_HIP_NORM_QUANT");
  d->quant_norm = quant && !(qenv && qenv[0] == '0');
  // likewise the FFN's down input, when every down matrix is a k-quant
  bool qffn = c.feed_forward_length % 256 == 0;
  for (const rh_decoder::Block& b : d->blocks)
    qffn = qffn && is_kquant_matrix(b.down) && rh_matrix_cols(b.down) == c.feed_forward_length;
  d->quant_ffn = qffn && !(qenv && qenv[0] == '0');
  // and the attention output, the O matrix's input, where the grouped
  // attention kernel forms it (head_dim 64, four or eight heads a kv head)
  const size_t grp = c.head_count_kv ? c.head_count / c.head_count_kv : 0;
  bool qattn = c.head_dim == 64 && (grp == 4 || grp == 8) && w % 256 == 0;
  for (const rh_decoder::Block& b : d->blocks)
    qattn = qattn && is_kquant_matrix(b.o) && rh_matrix_cols(b.o) == w;
  d->quant_attn = qattn && !(qenv && qenv[0] == '0');
  *out = d;
  return RH_OK;
}

void rh_decoder_free(rh_decoder* d) {
  if (!d) return;
  // the context (and its stream) may already be destroyed: drain the device
  hipSetDevice(d->device);
  hipDeviceSynchronize();
  free_acts(d);
  for (auto& b : d->blocks) {
    if (b.attn_norm) hipFree(b.attn_norm);
    if (b.ffn_norm) hipFree(b.ffn_norm);
  }
  for (void* p : {static_cast<void*>(d->output_norm), static_cast<void*>(d->rope_cos),
                  static_cast<void*>(d->rope_sin), static_cast<void*>(d->keys), static_cast<void*>(d->values),
                  static_cast<void*>(d->logits), static_cast<void*>(d->pick), static_cast<void*>(d->record),
                  static_cast<void*>(d->count), static_cast<void*>(d->pick_parts)})
    if (p) hipFree(p);
  delete d;
}

void rh_decoder_reset(rh_decoder* d) {
  if (d) d->cached = 0;
}

size_t rh_decoder_position(const rh_decoder* d) { return d ? d->cached : 0; }

}  // extern "C"

namespace {

constexpr size_t kMaxGraphs = 8;

// forward_device for a batch (n >= 2) whose ids are in d->tokens, through a
// graph of the same launches: the first call for (n, start) runs eagerly
// (which sizes every buffer) and then captures the forward; later calls
// replay it while no buffer it captured has moved. A failed capture leaves
// the eager result and no graph.
rh_status forward_cached(rh_decoder* d, size_t n, size_t start) {
  d->pick_n = 0;  // a replayed batch writes no pick partials
  if (n < 2 || !d->use_graphs) return forward_device(d, d->tokens, n, start);
  const uint64_t cg = ctx_scratch_generation(d->ctx);
  for (size_t i = 0; i < d->graphs.size(); i++) {
    rh_decoder::Graph& g = d->graphs[i];
    if (g.n != n || g.start != start) continue;
    if (g.ctx_gen == cg && g.acts_gen == d->acts_gen) {
      g.used = ++d->graph_clock;
      RHD(hipGraphLaunch(g.exec, d->stream));
      d->cached = start + n;
      return RH_OK;
    }
    destroy_exec(d, g.exec);
    d->graphs.erase(d->graphs.begin() + static_cast<std::ptrdiff_t>(i));
    break;
  }
  RHS(forward_device(d, d->tokens, n, start));
  const uint64_t cg2 = ctx_scratch_generation(d->ctx), ag = d->acts_gen;
  const size_t cached = d->cached;
  if (hipStreamBeginCapture(d->stream, hipStreamCaptureModeThreadLocal) != hipSuccess) {
    (void)hipGetLastError();
    return RH_OK;
  }
  const rh_status cs = forward_device(d, d->tokens, n, start);
  hipGraph_t graph = nullptr;
  const hipError_t ee = hipStreamEndCapture(d->stream, &graph);
  d->cached = cached;
  hipGraphExec_t exec = nullptr;
  const bool ok = cs == RH_OK && ee == hipSuccess && graph &&
                  hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0) == hipSuccess;
  if (graph) hipGraphDestroy(graph);
  (void)hipGetLastError();
  if (!ok || ctx_scratch_generation(d->ctx) != cg2 || d->acts_gen != ag) {
    if (exec) hipGraphExecDestroy(exec);
    return RH_OK;
  }
  if (d->graphs.size() == kMaxGraphs) {
    size_t lru = 0;
    for (size_t i = 1; i < d->graphs.size(); i++)
      if (d->graphs[i].used < d->graphs[lru].used) lru = i;
    destroy_exec(d, d->graphs[lru].exec);
    d->graphs.erase(d->graphs.begin() + static_cast<std::ptrdiff_t>(lru));
  }
  d->graphs.push_back(rh_decoder::Graph{n, start, cg2, ag, ++d->graph_clock, exec});
  return RH_OK;
}

}  // namespace

extern "C" {

rh_status rh_decoder_forward_batch(rh_decoder* d, const uint32_t* tokens, size_t n, size_t start, float* logits,
                                   size_t logits_len) {
  if (!d || (!tokens && n) || (!logits && logits_len)) return RH_ERR_INVALID_ARGUMENT;
  // decoder.rs:111-136: the batch is checked before anything changes
  if (n == 0) return RH_ERR_INVALID_CONFIG;
  if (start + n > d->c.context_length || start + n < start) return RH_ERR_CONTEXT_FULL;
  for (size_t i = 0; i < n; i++)
    if (tokens[i] >= d->c.vocab_size) return RH_ERR_INVALID_CONFIG;
  if (start != d->cached) return RH_ERR_CACHE_POSITION;  // cache.rs:56-61
  if (hipSetDevice(ctx_device(d->ctx)) != hipSuccess) return RH_ERR_DEVICE;
  if (ensure_acts(d, n) != hipSuccess) return RH_ERR_OUT_OF_MEMORY;
  RHD(hipMemcpyAsync(d->tokens, tokens, n * 4, hipMemcpyHostToDevice, d->stream));
  RHS(forward_cached(d, n, start));
  const size_t m = logits_len < d->c.vocab_size ? logits_len : d->c.vocab_size;
  if (m) RHD(hipMemcpyAsync(logits, d->logits, m * 4, hipMemcpyDeviceToHost, d->stream));
  RHD(hipStreamSynchronize(d->stream));
  return RH_OK;
}

rh_status rh_decoder_generate_greedy(rh_decoder* d, const uint32_t* prompt, size_t n, size_t max_tokens,
                                     uint32_t* out, size_t* n_out) {
  if (!d || !n_out || (!prompt && n) || (!out && max_tokens)) return RH_ERR_INVALID_ARGUMENT;
  *n_out = 0;
  // generate.rs:45-48
  if (n >= d->c.context_length) return RH_ERR_CONTEXT_FULL;
  if (n == 0) return RH_ERR_INVALID_CONFIG;
  for (size_t i = 0; i < n; i++)
    if (prompt[i] >= d->c.vocab_size) return RH_ERR_INVALID_CONFIG;
  if (hipSetDevice(ctx_device(d->ctx)) != hipSuccess) return RH_ERR_DEVICE;
  if (ensure_acts(d, n < kPrefillChunk ? n : kPrefillChunk) != hipSuccess) return RH_ERR_OUT_OF_MEMORY;
  if (d->record_cap < max_tokens) {
    RHD(hipStreamSynchronize(d->stream));
    if (d->record) hipFree(d->record);
    d->record = nullptr;
    d->record_cap = 0;
    if (dmalloc(&d->record, max_tokens) != hipSuccess) return RH_ERR_OUT_OF_MEMORY;
    d->record_cap = max_tokens;
  }
  hipStream_t s = d->stream;
  // prefill (generate.rs:70-81): reset, then chunks of 64
  d->cached = 0;
  for (size_t st = 0; st < n; st += kPrefillChunk) {
    const size_t m = n - st < kPrefillChunk ? n - st : kPrefillChunk;
    RHD(hipMemcpyAsync(d->tokens, prompt + st, m * 4, hipMemcpyHostToDevice, s));
    RHS(forward_cached(d, m, st));
  }
  RHD(hipMemsetAsync(d->count, 0, 8, s));
  // decode_loop (generate.rs:83-111): pick, then forward the pick; the pick
  // stays on the device and feeds the next step's embedding
  size_t position = n;
  size_t emitted = 0;
  for (size_t i = 0; i < max_tokens; i++) {
    // on the norm-fused path the pick also writes the next step's embedding
    const rh_matrix* E = d->token_embd;
    float* next = d->fuse_norm ? d->hidden : nullptr;
    const uint32_t width = static_cast<uint32_t>(d->c.embedding_length);
    if (d->pick_n)  // the last forward was a one-token step whose output launch wrote partials
      hipLaunchKernelGGL(argmax_parts_kernel, dim3(1), dim3(1024), 0, s, d->pick_parts, d->pick_n, d->pick,
                         d->record, d->count, rh_matrix_type(E), matrix_data(E), matrix_pitch(E), width, next);
    else
      hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, s, d->logits,
                         static_cast<uint32_t>(d->c.vocab_size), d->pick, d->record, d->count, rh_matrix_type(E),
                         matrix_data(E), matrix_pitch(E), width, next);
    RHD(hipGetLastError());
    emitted++;
    if (position == d->c.context_length) break;
    RHS(forward_device(d, d->pick, 1, position, d->fuse_norm));
    position++;
  }
  uint32_t flag[2] = {0, 0};
  if (emitted) RHD(hipMemcpyAsync(out, d->record, emitted * 4, hipMemcpyDeviceToHost, s));
  RHD(hipMemcpyAsync(flag, d->count, 8, hipMemcpyDeviceToHost, s));
  RHD(hipStreamSynchronize(s));
  if (flag[1]) return RH_ERR_NO_VALID_TOKENS;  // sampler.rs:84-85
  *n_out = emitted;
  return RH_OK;
}

}  // extern "C"
