// gemm.hip -- prefill GEMM on gfx950 matrix cores: Q4_K / Q6_K weights (their
// GGUF blocks, in the unit layout of rh_device.h) against Q8_K-quantized
// activations of many tokens, bit-identical to rusticide's CPU integer path.
//
// The CPU path (crates/rusticide-kernels/src/portable/int_dot.rs:142-204)
// forms, per 256-weight super-block b of row r and token t, exact integers
//   Q4_K: isum = sum_j sc_j * sum_l q*a, msum = sum_j m_j * bsum_j
//   Q6_K: isum = sum_s sc_s * sum_l (q-32)*a
// and one float term per block, added in block order. Here the integers come
// from int8 MFMA (v_mfma_i32_32x32x32_i8), exact in i32:
//   * the sub-block scale is folded into the weight and the product split
//     into two int8 planes: Q4_K w = sc*q with sc = 8*sh + sl, planes sh*q
//     and sl*q (0..105), isum = 8*hi + lo; Q6_K w = sc*(q-32) = 128*hi + lo
//     (lo in 0..127, hi in -32..31), isum = 128*hi + lo. Two accumulators
//     take the planes side by side over the block's eight 32-deep steps, so
//     each activation fragment is read from LDS once for both;
//   * the Q4_K min term needs only the block sums: with bsum = 128*bh + bl
//     (bl in 0..127), msum = 128 * sum_j m_j*bh_j + sum_j m_j*bl_j, two MFMAs
//     whose 32-deep operands carry the eight (m_j, bl_j) / (m_j, bh_j) pairs
//     in one lane group and zeros elsewhere. Each lane gives A and B the same
//     k for the same byte, so the order MFMA sums k in does not matter.
// The float combine is the CPU path's, per block, in block order, one
// accumulator per (row, token) in one lane.
//
// Split K: when the row and token tiles give too few workgroups to fill the
// chip (a 64-token prefill of a 2048-row matrix is 16 of them), blockIdx.z
// takes a segment of seg_len blocks. Segment 0 forms the in-order sum over its
// blocks as usual; every later segment stores each of its blocks' float terms,
// and gemm_combine_kernel continues segment 0's sum with them in block order.
// That is the unsplit sequence of float additions, so the bits do not change.
#include <algorithm>
#include <cstdlib>

#include "rh_device.h"
#include "rh_internal.h"

namespace rh {

namespace {

constexpr uint32_t kStride = 272;   // LDS bytes per 256-byte row: +16 spreads the banks

typedef int32_t v4i __attribute__((ext_vector_type(4)));
typedef int32_t v16i __attribute__((ext_vector_type(16)));

__device__ __forceinline__ uint32_t gemm_job(const GemvJobs& jobs, uint32_t wg) {
  uint32_t j = 0;
#pragma unroll
  for (uint32_t i = 1; i < static_cast<uint32_t>(kMaxJobs); i++)
    if (i < jobs.n && wg >= jobs.j[i].wg_begin) j = i;
  return j;
}

// 6-bit scale and min of Q4_K sub-block j from the header dwords
// (ggml get_scale_min_k4, quantize/src/q4_k.rs:17-25).
__device__ __forceinline__ void q4k_scale_min(const u32x4& hd, uint32_t j, uint32_t& sc, uint32_t& m) {
  if (j < 4u) {
    sc = bfe(hd.y, 8u * j, 6);
    m = bfe(hd.z, 8u * j, 6);
  } else {
    const uint32_t jj = j - 4u;
    sc = bfe(hd.w, 8u * jj, 4) | (bfe(hd.y, 8u * jj + 6u, 2) << 4);
    m = bfe(hd.w, 8u * jj + 4u, 4) | (bfe(hd.z, 8u * jj + 6u, 2) << 4);
  }
}

// Terms of a split launch: plane 0 holds segment 0's sums, plane 1 + b -
// seg_len the term of block b >= seg_len; each plane is [rows_pad][tokens]
// over the launch's row tiles.
struct SplitTerms {
  float* terms;        // nullptr: no split
  uint32_t seg_len;    // blocks per segment
  uint32_t rows_pad;   // kRowsWG x the launch's workgroups along rows
  uint32_t tmajor;     // 1: each plane token-major, [token][rows_pad]
  uint32_t planes;     // 1 + blocks - seg_len
  uint32_t* counters;  // non-null: the tiles' arrival counts (split_fixup)
};

// Offset of (padded row r, token t) within a plane.
__device__ __forceinline__ size_t plane_at(const SplitTerms& sp, uint32_t r, size_t t, size_t tokens) {
  return sp.tmajor ? t * sp.rows_pad + r : static_cast<size_t>(r) * tokens + t;
}

constexpr uint32_t kRowsWG = 128;  // rows a GEMM workgroup owns

// ------------------------------------------------------------ split fixup
// The end of a split launch without gemm_combine_kernel. Each workgroup, its
// planes stored, counts itself in at its tile's counter (device scope); the
// last of the tile's gridDim.z segments to arrive sums the tile's planes,
// plane 0 then planes 1.. one addition at a time as gemm_combine_kernel
// does (the same bits), stores the outputs and sets the counter back to 0
// for the next launch. No workgroup waits on another. The planes are
// [rows_pad][tokens] and tokens come in multiples of 4 (the host checks): a
// thread's slot is four consecutive tokens of a row, one 16-byte load a
// plane.
//
// Coherence without cache maintenance: the workgroups of a tile may sit on
// different XCDs, whose L2 caches are not coherent with one another. The
// planes are therefore stored device-coherent (relaxed device-scope atomic
// stores: sc1, written through the L2) and read device-coherent (sc1 buffer
// loads); each wave waits for its stores to complete (vmcnt(0)) before the
// workgroup's barrier, and one lane's counter increment follows the
// barrier, so a workgroup that finds the count complete reads every plane
// as stored. A release/acquire pair of fences instead writes back and
// invalidates the whole L2 of an XCD per workgroup: a 64-token prefill
// measured 2.35 ms that way against 2.04 with the separate combine launch.
constexpr uint32_t kFixupPlanes = 8;  // planes requested at once per slot
// Launches of more planes combine in gemm_combine_kernel: one workgroup
// reading a tile's planes in several rounds is slower than the separate
// launch (a 64-token prefill's 21-plane down GEMMs: 18.4-21.2 us with the
// fixup against 16.3-18.9 with the combine; its 8-plane QKV GEMM 11.8
// against 14.5).
constexpr uint32_t kFixupMaxPlanes = 1 + kFixupPlanes;
constexpr int kCoherentSc1 = 16;      // cache-policy bit sc1 of a buffer load
constexpr int kBufferRsrcWord3 = 0x00020000;  // gfx9 buffer resource: raw 32-bit dwords

// A plane value, stored device-coherent when a fixup reads it.
__device__ __forceinline__ void store_plane(float* p, float v, bool coherent) {
  if (coherent) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else *p = v;
}

// A lane's 16 values of one token into a plane: register 4q + u holds row
// 8q + 4g + u of the wave's 32 (the MFMA's D layout), so a token-major
// plane takes them as four 16-byte stores of four consecutive rows (a store
// instruction then writes 32 bytes a token instead of 4). A fixup's planes
// (device-coherent stores) are never token-major.
__device__ __forceinline__ void store_lane_plane(const SplitTerms& sp, float* plane, uint32_t r0, uint32_t g,
                                                 size_t tok, size_t T, const float (&v)[16]) {
  const bool coherent = sp.counters != nullptr;
  if (sp.tmajor && !coherent) {
    float* p = plane + tok * sp.rows_pad + r0 + 4u * g;
#pragma unroll
    for (int q = 0; q < 4; q++)
      *reinterpret_cast<f32x4*>(p + 8u * q) = f32x4{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
    return;
  }
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const uint32_t m = 8u * static_cast<uint32_t>(i >> 2) + 4u * g + static_cast<uint32_t>(i & 3);
    store_plane(plane + plane_at(sp, r0 + m, tok, T), v[i], coherent);
  }
}

// Token-major outputs from [rows_pad][tokens] planes go through `tile`
// (LDS, 32*NT tokens x kTileStride floats): the sums are stored there by row
// and read back by token, so the outputs are stored in runs of four rows.
constexpr uint32_t kTileStride = kRowsWG + 4u;

template <int NT>
__device__ __forceinline__ void split_fixup(const GemvJobs& jobs, const SplitTerms& sp, size_t T, uint32_t tok0,
                                            uint32_t* last, float* tile) {
  // every wave's plane stores complete before one lane counts the
  // workgroup in
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  uint32_t* const ctr = sp.counters + blockIdx.y * gridDim.x + blockIdx.x;
  if (threadIdx.x == 0)
    *last = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u == gridDim.z;
  __syncthreads();
  if (!*last) return;
  // kSlots slots a thread, slot (row sl / kCols, tokens 4 (sl % kCols) ..);
  // byte offsets within the planes (below 2^31, the host checks); slots
  // past the tile's tokens read its first and store nothing
  constexpr uint32_t kCols = 8u * NT, kSlots = kRowsWG * kCols / 256u, kAhead = kFixupPlanes / NT;
  const uint32_t tw = static_cast<uint32_t>(min(static_cast<size_t>(32u * NT), T - tok0));
  const uint32_t n4 = 4u * sp.rows_pad * static_cast<uint32_t>(T), R0 = blockIdx.x * kRowsWG;
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(sp.terms, 0, static_cast<int>(n4 * sp.planes), kBufferRsrcWord3);
  uint32_t base[kSlots];
  f32x4 y[kSlots];
#pragma unroll
  for (uint32_t k = 0; k < kSlots; k++) {
    const uint32_t sl = threadIdx.x + 256u * k, r = sl / kCols, c = sl % kCols;
    base[k] = 4u * ((R0 + r) * static_cast<uint32_t>(T) + tok0 + 4u * (4u * c < tw ? c : 0u));
    y[k] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, base[k], 0, kCoherentSc1));
  }
  for (uint32_t p0 = 1; p0 < sp.planes; p0 += kAhead) {
    f32x4 v[kAhead][kSlots];
#pragma unroll
    for (uint32_t j = 0; j < kAhead; j++)
#pragma unroll
      for (uint32_t k = 0; k < kSlots; k++)
        v[j][k] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                rs, min(p0 + j, sp.planes - 1u) * n4 + base[k], 0, kCoherentSc1));
#pragma unroll
    for (uint32_t j = 0; j < kAhead; j++)
#pragma unroll
      for (uint32_t k = 0; k < kSlots; k++)
        if (p0 + j < sp.planes) y[k] += v[j][k];
  }
  const GemvJob& J = jobs.j[gemm_job(jobs, blockIdx.x)];
  const bool runs = J.tmajor && J.rows % 4u == 0 && (reinterpret_cast<uintptr_t>(J.out) & 15u) == 0;
#pragma unroll
  for (uint32_t k = 0; k < kSlots; k++) {
    const uint32_t sl = threadIdx.x + 256u * k, r = sl / kCols, c = sl % kCols;
    if (J.tmajor) {  // into the tile, by row
#pragma unroll
      for (uint32_t e = 0; e < 4u; e++) tile[(4u * c + e) * kTileStride + r] = y[k][e];
    } else {
      const uint32_t row = (blockIdx.x - J.wg_begin) * kRowsWG + r;
      if (4u * c >= tw || row >= J.rows) continue;
#pragma unroll
      for (uint32_t e = 0; e < 4u; e++) {
        const size_t tok = tok0 + 4u * c + e;
        const size_t o = static_cast<size_t>(row) * T + tok;
        if (o < J.out_len) J.out[o] = y[k][e];
      }
    }
  }
  if (J.tmajor) {  // the tile back by token: (token sl / 32, rows 4 (sl % 32) ..)
    __syncthreads();
#pragma unroll
    for (uint32_t k = 0; k < kSlots; k++) {
      const uint32_t sl = threadIdx.x + 256u * k, t = sl / 32u, rq = sl % 32u;
      const uint32_t row = (blockIdx.x - J.wg_begin) * kRowsWG + 4u * rq;
      const size_t tok = tok0 + t;
      if (t >= tw || row >= J.rows) continue;
      const f32x4 v = *reinterpret_cast<const f32x4*>(tile + t * kTileStride + 4u * rq);
      if (runs) {
        const size_t o = tok * J.rows + row;
        if (o + 4u <= J.out_len) *reinterpret_cast<f32x4*>(J.out + o) = v;
        continue;
      }
#pragma unroll
      for (uint32_t e = 0; e < 4u; e++) {
        const size_t o = tok * J.rows + row + e;
        if (row + e < J.rows && o < J.out_len) J.out[o] = v[e];
      }
    }
  }
  if (threadIdx.x == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------------ row-owning form
// A workgroup of 4 waves owns kRowsWG = 128 rows x 32*NT tokens; wave w owns
// rows 32w.. of the tile outright. Each lane loads the raw bytes of its own
// row's block (lane = row + 32*g, g the lane's 16-deep half of every 32-deep
// step) and dequantizes them straight into the MFMA A operand: no weight
// plane passes through LDS and no two waves dequantize the same row. Only
// the activation tile (the B operand, shared by the four waves) is staged in
// LDS, double-buffered: block b+1's bytes are loaded into registers while
// block b's MFMAs run and stored into the other buffer after them, one
// barrier a block.
//
// Planes: Q4_K's w = sc*q is split along the scale, sc = 8*sh + sl (sh, sl
// in 0..7), so each plane byte sh*q or sl*q (at most 105) is one packed
// 16-bit multiply of four nibbles; isum = 8*hi + lo. Q6_K keeps w = sc*(q-32)
// = 128*hi + lo. Both sums are exact in i32.
//
// The matrices are in the unit layout (rh_device.h): the lane's pieces of a
// block sit at fixed 16-byte-aligned offsets of its group of 16 blocks.

typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pk_mul_u16(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, a) * __builtin_bit_cast(u16x2, b));
}

// The raw bytes one lane holds for one block of its row.
// Q4_K: hd = d, dmin, scales[12]; qs[p] = qs[32p + 16g .. +16].
// Q6_K: ql0[h] = ql[64h + 16g ..], ql1[h] = ql[64h + 32 + 16g ..],
//       qh[h] = qh[32h + 16g ..], sc = scales[16], d in the low half of dw.
template <int FMT>
struct LaneRaw;
template <>
struct LaneRaw<12> {
  u32x4 hd, qs[4];
};
template <>
struct LaneRaw<14> {
  u32x4 ql0[2], ql1[2], qh[2], sc;
  uint32_t dw;
};

// The lane's pieces of block b of its row from the unit layout (rh_device.h):
// block e = row * ub + b sits at position tw of group e >> 4, every piece at
// a 16-byte-aligned offset.
__device__ __forceinline__ void load_lane_raw(LaneRaw<12>& x, const GemvJob& J, uint32_t row, uint32_t b,
                                              uint32_t g) {
  const uint32_t e = row * J.ub + b, tw = e & 15u;
  const uint8_t* u = J.w + static_cast<size_t>(e >> 4) * kUnitBytesQ4;
  x.hd = load16(u + 16u * tw);
  x.qs[0] = load16(u + 256u + 64u * tw + 16u * g);
  x.qs[1] = load16(u + 256u + 64u * tw + 32u + 16u * g);
  x.qs[2] = load16(u + 1280u + 64u * tw + 16u * g);
  x.qs[3] = load16(u + 1280u + 64u * tw + 32u + 16u * g);
}

__device__ __forceinline__ void load_lane_raw(LaneRaw<14>& x, const GemvJob& J, uint32_t row, uint32_t b,
                                              uint32_t g) {
  const uint32_t e = row * J.ub + b, tw = e & 15u;
  const uint8_t* u = J.w + static_cast<size_t>(e >> 4) * kUnitBytesQ6;
#pragma unroll
  for (uint32_t h = 0; h < 2u; h++) {
    x.ql0[h] = load16(u + 64u * tw + 16u * (2u * h + g));
    x.ql1[h] = load16(u + 1024u + 64u * tw + 16u * (2u * h + g));
    x.qh[h] = load16(u + 2048u + 64u * tw + 16u * (2u * h + g));
  }
  x.sc = load16(u + 3072u + 16u * tw);
  x.dw = *reinterpret_cast<const uint16_t*>(u + 3328u + 2u * tw);
}

// The two A planes of 32-deep step kk for this lane (its row, k = 32kk + 16g ..).
__device__ __forceinline__ void lane_planes(const LaneRaw<12>& x, uint32_t kk, uint32_t, v4i& hi, v4i& lo) {
  uint32_t sc, m;
  q4k_scale_min(x.hd, kk, sc, m);
  const uint32_t sh = (sc >> 3) * 0x00010001u, sl = (sc & 7u) * 0x00010001u;
  const u32x4 c = x.qs[kk >> 1];
  const uint32_t s4 = 4u * (kk & 1u);
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t nib = (c[i] >> s4) & 0x0F0F0F0Fu;
    hi[i] = static_cast<int32_t>(pk_mul_u16(nib, sh));
    lo[i] = static_cast<int32_t>(pk_mul_u16(nib, sl));
  }
}

// Q6_K: four 6-bit bytes q as w = sc * (q - 32) in hi/lo planes (w = 128*hi
// + lo, lo in 0..127). The bytes are spread into 16-bit lanes and multiplied
// with one packed multiply-add each ((q - 32)*sc fits i16: |w| <= 4096),
// then the planes' bytes are gathered back with v_perm_b32.
__device__ __forceinline__ void q6_split(uint32_t q, int32_t sc, uint32_t& hi, uint32_t& lo) {
  typedef int16_t i16x2 __attribute__((ext_vector_type(2)));
  const i16x2 scv{static_cast<int16_t>(sc), static_cast<int16_t>(sc)};
  const i16x2 off{static_cast<int16_t>(-32 * sc), static_cast<int16_t>(-32 * sc)};
  // bytes 0,2 -> lanes of qe; bytes 1,3 -> lanes of qo (zero high bytes)
  const uint32_t qe = __builtin_amdgcn_perm(0u, q, 0x0c020c00u);
  const uint32_t qo = __builtin_amdgcn_perm(0u, q, 0x0c030c01u);
  const i16x2 we = __builtin_bit_cast(i16x2, qe) * scv + off;
  const i16x2 wo = __builtin_bit_cast(i16x2, qo) * scv + off;
  const uint32_t ue = __builtin_bit_cast(uint32_t, we), uo = __builtin_bit_cast(uint32_t, wo);
  // bytes (we.lo, wo.lo, we.hi, wo.hi) -> low byte of each 16-bit product
  lo = __builtin_amdgcn_perm(uo, ue, 0x06020400u) & 0x7F7F7F7Fu;
  const i16x2 he = we >> static_cast<int16_t>(7), ho = wo >> static_cast<int16_t>(7);
  hi = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, ho), __builtin_bit_cast(uint32_t, he), 0x06020400u);
}

__device__ __forceinline__ void lane_planes(const LaneRaw<14>& x, uint32_t kk, uint32_t g, v4i& hi, v4i& lo) {
  // k = 128h + 32r + l (q6_k.rs:13-43): ql[64h + 32(r&1) + l] (high nibble
  // for r >= 2), qh[32h + l] bits 2r..2r+1, scale 8h + 2r + l/16
  const uint32_t h = kk >> 2, r = kk & 3u;
  const u32x4 ql = (r & 1u) ? x.ql1[h] : x.ql0[h];
  const u32x4 qh = x.qh[h];
  const uint32_t s = 8u * h + 2u * r + g;
  const int32_t sc = __builtin_amdgcn_sbfe(static_cast<int32_t>(x.sc[s >> 2]), 8u * (s & 3u), 8);
  const uint32_t nsh = 4u * (r >> 1);
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t qv = ((ql[i] >> nsh) & 0x0F0F0F0Fu) | (((qh[i] >> (2u * r)) << 4) & 0x30303030u);
    uint32_t hw, lw;
    q6_split(qv, sc, hw, lw);
    hi[i] = static_cast<int32_t>(hw);
    lo[i] = static_cast<int32_t>(lw);
  }
}

// Q4_K's mins as the msum MFMA's A operand (k = j in lane group 0): with
// the activation's block sums as B (bsum_j = 128*bh_j + bl_j, bl_j in
// 0..127), msum = 128 * sum_j m_j*bh_j + sum_j m_j*bl_j from two MFMAs.
__device__ __forceinline__ v4i lane_mins(const LaneRaw<12>& x, uint32_t g) {
  uint32_t w0 = 0, w1 = 0;
#pragma unroll
  for (uint32_t j = 0; j < 8u; j++) {
    uint32_t sc, m;
    q4k_scale_min(x.hd, j, sc, m);
    if (j < 4u) w0 |= m << (8u * j);
    else w1 |= m << (8u * (j - 4u));
  }
  return v4i{g == 0 ? static_cast<int32_t>(w0) : 0, g == 0 ? static_cast<int32_t>(w1) : 0, 0, 0};
}

__device__ __forceinline__ float2 lane_d(const LaneRaw<12>& x) { return make_float2(f16_lo(x.hd.x), f16_hi(x.hd.x)); }
__device__ __forceinline__ float2 lane_d(const LaneRaw<14>& x) { return make_float2(f16_lo(x.dw), 0.0f); }

template <int NT>
constexpr size_t rows_kernel_lds() {
  // act [2][32NT][kStride] | d8 [2][32NT] | bs [2][32NT][16] | rowd [4][32]
  return 2u * 32u * NT * kStride + 2u * 32u * NT * 4u + 2u * 32u * NT * 16u + 4u * 32u * 8u;
}

template <int FMT, int NT, bool SPLIT>
__global__ __launch_bounds__(256) void gemm_kq_rows_kernel(GemvJobs jobs, Q8Dev q, size_t tokens,
                                                           SplitTerms split) {
  constexpr uint32_t BN = 32u * NT;
  extern __shared__ __align__(16) uint8_t lds[];
  int8_t* actT = reinterpret_cast<int8_t*>(lds);                          // [2][BN][kStride]
  float* d8T = reinterpret_cast<float*>(lds + 2u * BN * kStride);         // [2][BN]
  uint8_t* bsT = reinterpret_cast<uint8_t*>(d8T + 2u * BN);               // [2][BN][16]
  float2* rowdT = reinterpret_cast<float2*>(bsT + 2u * BN * 16u);         // [4][32]

  const GemvJob& J = jobs.j[gemm_job(jobs, blockIdx.x)];
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6, g = lane >> 5, ml = lane & 31u;
  const uint32_t row0 = (blockIdx.x - J.wg_begin) * kRowsWG;
  const uint32_t arow = min(row0 + 32u * wave + ml, J.rows - 1u);
  const uint32_t tok0 = blockIdx.y * BN;
  const uint32_t nb = J.nb;
  const uint32_t seg = SPLIT ? blockIdx.z : 0u;
  const uint32_t b_begin = SPLIT ? seg * split.seg_len : 0u;
  const uint32_t b_end = SPLIT ? min(nb, b_begin + split.seg_len) : nb;
  const bool store_terms = SPLIT && seg > 0u;
  const size_t T = tokens;
  const uint32_t last = static_cast<uint32_t>(T - 1);
  const uint32_t qs32 = static_cast<uint32_t>(q.qstride), bs32 = static_cast<uint32_t>(q.bstride);
  // staging: BN*256 activation bytes in 16-byte chunks over 256 threads; the
  // first BN threads also take one token's d8 (and Q4_K block sums)
  constexpr int ACH = static_cast<int>(BN) * 16 / 256;
  const uint32_t stok = min(tok0 + (tid & (BN - 1u)), last);

  LaneRaw<FMT> raw, nxt;
  u32x4 ar[ACH];
  u32x4 sr0{}, sr1{};
  float d8r = 0.0f;
  auto load_act = [&](uint32_t b) {
#pragma unroll
    for (int c = 0; c < ACH; c++) {
      const uint32_t chunk = tid + static_cast<uint32_t>(c) * 256u;
      const uint32_t tok = min(tok0 + (chunk >> 4), last);
      ar[c] = load16(reinterpret_cast<const uint8_t*>(q.quants + (__umul24(tok, qs32) + b * 256u +
                                                                  (chunk & 15u) * 16u)));
    }
    if (tid < BN) {
      const uint32_t o = __umul24(stok, bs32) + b * 8u;
      d8r = q.scales[o];
      if (FMT == 12) {
        sr0 = load16(reinterpret_cast<const uint8_t*>(q.sums + o));
        sr1 = load16(reinterpret_cast<const uint8_t*>(q.sums + o + 4));
      }
    }
  };
  auto store_act = [&](uint32_t buf) {
    int8_t* a = actT + buf * BN * kStride;
#pragma unroll
    for (int c = 0; c < ACH; c++) {
      const uint32_t chunk = tid + static_cast<uint32_t>(c) * 256u;
      *reinterpret_cast<u32x4*>(a + (chunk >> 4) * kStride + (chunk & 15u) * 16u) = ar[c];
    }
    if (tid < BN) {
      d8T[buf * BN + tid] = d8r;
      if (FMT == 12) {
        // bsum_j = 128*bh_j + bl_j, bl_j in 0..127 (|bsum_j| <= 32*128)
        const int32_t s8[8] = {static_cast<int32_t>(sr0.x), static_cast<int32_t>(sr0.y),
                               static_cast<int32_t>(sr0.z), static_cast<int32_t>(sr0.w),
                               static_cast<int32_t>(sr1.x), static_cast<int32_t>(sr1.y),
                               static_cast<int32_t>(sr1.z), static_cast<int32_t>(sr1.w)};
        uint32_t bl[2] = {0u, 0u}, bh[2] = {0u, 0u};
#pragma unroll
        for (int j = 0; j < 8; j++) {
          bl[j >> 2] |= (static_cast<uint32_t>(s8[j]) & 0x7fu) << (8 * (j & 3));
          bh[j >> 2] |= (static_cast<uint32_t>(s8[j] >> 7) & 0xffu) << (8 * (j & 3));
        }
        *reinterpret_cast<u32x4*>(bsT + (buf * BN + tid) * 16u) = u32x4{bl[0], bl[1], bh[0], bh[1]};
      }
    }
  };

  float y[NT][16];
#pragma unroll
  for (int t = 0; t < NT; t++)
#pragma unroll
    for (int i = 0; i < 16; i++) y[t][i] = -0.0f;

  if (b_begin < b_end) {
    load_lane_raw(raw, J, arow, b_begin, g);
    load_act(b_begin);
    store_act(0u);
    __syncthreads();
  }
  for (uint32_t b = b_begin; b < b_end; b++) {
    const uint32_t cur = (b - b_begin) & 1u;
    const bool more = b + 1u < b_end;
    if (more) {
      // the next block's weights go out a whole block ahead: each lane's
      // 16-byte pieces come from 32 different rows, a long round trip
      load_lane_raw(nxt, J, arow, b + 1u, g);
      load_act(b + 1u);
    }
    // this block's (d, dmin) of the wave's rows, for the D layout's rows
    if (g == 0) rowdT[wave * 32u + ml] = lane_d(raw);
    const int8_t* a = actT + cur * BN * kStride;
    v16i acc_h[NT], acc_l[NT];
#pragma unroll
    for (uint32_t kk = 0; kk < 8u; kk++) {
      v4i Ah, Al;
      lane_planes(raw, kk, g, Ah, Al);
#pragma unroll
      for (int t = 0; t < NT; t++) {
        const v4i Bv = *reinterpret_cast<const v4i*>(a + (32u * t + ml) * kStride + 32u * kk + 16u * g);
        acc_h[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(Ah, Bv, kk ? acc_h[t] : v16i{}, 0, 0, 0);
        acc_l[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(Al, Bv, kk ? acc_l[t] : v16i{}, 0, 0, 0);
      }
    }
    v4i Am{};
    if constexpr (FMT == 12) Am = lane_mins(raw, g);
    float* plane = store_terms ? split.terms + static_cast<size_t>(1u + b - split.seg_len) * split.rows_pad * T
                               : nullptr;
#pragma unroll
    for (int t = 0; t < NT; t++) {
      const uint32_t tl = 32u * t + ml;  // the lane's token column of this tile
      const float d8 = d8T[cur * BN + tl];
      v16i acc_m{};
      if constexpr (FMT == 12) {
        const u32x4 bs = *reinterpret_cast<const u32x4*>(bsT + (cur * BN + tl) * 16u);
        const v4i Bh{g == 0 ? static_cast<int32_t>(bs.z) : 0, g == 0 ? static_cast<int32_t>(bs.w) : 0, 0, 0};
        const v4i Bl{g == 0 ? static_cast<int32_t>(bs.x) : 0, g == 0 ? static_cast<int32_t>(bs.y) : 0, 0, 0};
        acc_m = __builtin_amdgcn_mfma_i32_32x32x32_i8(Am, Bh, v16i{}, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 16; i++) acc_m[i] <<= 7;
        acc_m = __builtin_amdgcn_mfma_i32_32x32x32_i8(Am, Bl, acc_m, 0, 0, 0);
      }
      // the block's float term per (row, token), added in block order
      // (D layout: lane n + 32*((m/4)%2), register 4*(m/8) + m%4)
      float tv[16];
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const uint32_t m = 8u * static_cast<uint32_t>(i >> 2) + 4u * g + static_cast<uint32_t>(i & 3);
        const float2 dd = rowdT[wave * 32u + m];
        const int32_t isum = FMT == 12 ? (acc_h[t][i] << 3) + acc_l[t][i] : (acc_h[t][i] << 7) + acc_l[t][i];
        float term;
        if constexpr (FMT == 12) {
          // int_dot.rs:169: d8 * d.mul_add(isum, -(dmin * msum))
          const float neg = -(dd.y * static_cast<float>(acc_m[i]));
          term = d8 * __builtin_fmaf(dd.x, static_cast<float>(isum), neg);
        } else {
          // int_dot.rs:203: (d * d8) * isum
          const float sd = dd.x * d8;
          term = sd * static_cast<float>(isum);
        }
        if (store_terms) tv[i] = term;
        else y[t][i] += term;
      }
      if (store_terms && tok0 + tl < T)
        store_lane_plane(split, plane, blockIdx.x * kRowsWG + 32u * wave, g, tok0 + tl, T, tv);
    }
    if (more) {
      store_act(cur ^ 1u);
      raw = nxt;
    }
    __syncthreads();
  }
  if (SPLIT && !store_terms) {  // segment 0 of a split launch: plane 0 (padded rows too)
#pragma unroll
    for (int t = 0; t < NT; t++)
      if (tok0 + 32u * t + ml < T)
        store_lane_plane(split, split.terms, blockIdx.x * kRowsWG + 32u * wave, g, tok0 + 32u * t + ml, T, y[t]);
  } else if (!SPLIT && J.tmajor && J.rows % 4u == 0 && (reinterpret_cast<uintptr_t>(J.out) & 15u) == 0) {
    // token-major outputs, four consecutive rows a 16-byte store (whole
    // groups of four rows are inside the job or past it)
#pragma unroll
    for (int t = 0; t < NT; t++) {
      const size_t tok = tok0 + 32u * t + ml;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const uint32_t row = row0 + 32u * wave + 8u * static_cast<uint32_t>(q) + 4u * g;
        const size_t idx = tok * J.rows + row;
        if (row < J.rows && tok < T && idx + 4u <= J.out_len)
          *reinterpret_cast<f32x4*>(J.out + idx) =
              f32x4{y[t][4 * q], y[t][4 * q + 1], y[t][4 * q + 2], y[t][4 * q + 3]};
      }
    }
  } else if (!SPLIT) {
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const uint32_t m = 8u * static_cast<uint32_t>(i >> 2) + 4u * g + static_cast<uint32_t>(i & 3);
      const uint32_t row = row0 + 32u * wave + m;
#pragma unroll
      for (int t = 0; t < NT; t++) {
        const size_t tok = tok0 + 32u * t + ml;
        const size_t idx = J.tmajor ? tok * J.rows + row : static_cast<size_t>(row) * T + tok;
        if (row < J.rows && tok < T && idx < J.out_len) J.out[idx] = y[t][i];
      }
    }
  }
  if constexpr (SPLIT) {
    __shared__ uint32_t fix_last;
    static_assert(32u * NT * kTileStride * 4u <= rows_kernel_lds<NT>(), "the fixup's tile fits the LDS");
    if (split.counters) split_fixup<NT>(jobs, split, T, tok0, &fix_last, reinterpret_cast<float*>(lds));
  }
}

// The end of a split launch: per (row, token), segment 0's sum plus the later
// blocks' terms, one addition at a time in block order.
// Each thread owns two consecutive (row, token) slots (a plane holds a
// multiple of 64 of them) and requests up to kCombineAhead planes at once,
// clamped to the last plane, before its first addition: the combine waits on
// memory once for up to that many planes (a 64-token prefill's planes number
// 8-21), not once per plane. The additions stay one plane at a time, in block
// order.
constexpr uint32_t kCombineAhead = 24;

// tmajor: the planes are [tokens][rows_pad] (written so for token-major
// outputs, which are then stored in runs of consecutive rows).
__global__ __launch_bounds__(256) void gemm_combine_kernel(GemvJobs jobs, const float* __restrict__ terms,
                                                           uint32_t planes, uint32_t rows_pad, size_t tokens,
                                                           uint32_t bm, uint32_t tmajor) {
  const size_t n = static_cast<size_t>(rows_pad) * tokens;
  const size_t idx = (static_cast<size_t>(blockIdx.x) * 256u + threadIdx.x) * 2u;
  if (idx >= n) return;
  f32x2 y = *reinterpret_cast<const f32x2*>(terms + idx);
  for (uint32_t p0 = 1; p0 < planes; p0 += kCombineAhead) {
    f32x2 v[kCombineAhead];
#pragma unroll
    for (uint32_t k = 0; k < kCombineAhead; k++) {
      const uint32_t p = min(p0 + k, planes - 1u);
      v[k] = *reinterpret_cast<const f32x2*>(terms + static_cast<size_t>(p) * n + idx);
    }
#pragma unroll
    for (uint32_t k = 0; k < kCombineAhead; k++)
      if (p0 + k < planes) y += v[k];
  }
  if (tmajor) {
    // both slots are one token's rows grow, grow + 1 of one row tile
    const size_t tok = idx / rows_pad;
    const uint32_t grow = static_cast<uint32_t>(idx - tok * rows_pad);
    const GemvJob& J = jobs.j[gemm_job(jobs, grow / bm)];
    const uint32_t row = grow - J.wg_begin * bm;
    if (J.tmajor) {
      const size_t o = tok * J.rows + row;
      if (row + 1u < J.rows && o + 2u <= J.out_len && (reinterpret_cast<uintptr_t>(J.out + o) & 7u) == 0) {
        *reinterpret_cast<f32x2*>(J.out + o) = y;
        return;
      }
    }
#pragma unroll
    for (uint32_t e = 0; e < 2u; e++) {
      const uint32_t r = row + e;
      const size_t o = J.tmajor ? tok * J.rows + r : static_cast<size_t>(r) * tokens + tok;
      if (r < J.rows && o < J.out_len) J.out[o] = y[e];
    }
    return;
  }
#pragma unroll
  for (int e = 0; e < 2; e++) {
    const uint32_t grow = static_cast<uint32_t>((idx + e) / tokens);
    const size_t tok = idx + e - static_cast<size_t>(grow) * tokens;
    const GemvJob& J = jobs.j[gemm_job(jobs, grow / bm)];
    const uint32_t row = grow - J.wg_begin * bm;
    const size_t o = J.tmajor ? tok * J.rows + row : static_cast<size_t>(row) * tokens + tok;
    if (row < J.rows && o < J.out_len) J.out[o] = y[e];
  }
}

// Workgroups along rows (tiles of bm rows), with each job's first one
// recorded in wg_begin.
uint32_t row_tiles(GemvJobs& jobs, uint32_t bm) {
  uint32_t wgs = 0;
  for (uint32_t i = 0; i < jobs.n; i++) {
    jobs.j[i].wg_begin = wgs;
    wgs += (jobs.j[i].rows + bm - 1u) / bm;
  }
  return wgs;
}

struct SplitPlan {
  uint32_t segs = 1, seg_len = 0, planes = 0, rows_pad = 0;
};

// Splits K when the launch has fewer than `below` workgroups, aiming at
// kSplitTarget; every job must have the same block count. Below 2 blocks, or
// with Tuning::gemm_split off, nothing is split.
constexpr uint32_t kSplitTarget = 512;

SplitPlan plan_split(GemvJobs jobs, size_t tokens, uint32_t bm, uint32_t bn, uint32_t below) {
  SplitPlan p;
  const uint32_t wgs = row_tiles(jobs, bm);
  if (wgs == 0 || jobs.n == 0) return p;
  const uint32_t nb = jobs.j[0].nb;
  for (uint32_t i = 1; i < jobs.n; i++)
    if (jobs.j[i].nb != nb) return p;
  if (!tuning().gemm_split) return p;
  const size_t base = static_cast<size_t>(wgs) * ((tokens + bn - 1) / bn);
  if (nb < 2 || base >= below) return p;
  const uint32_t want = static_cast<uint32_t>(std::min<size_t>(nb, (kSplitTarget + base - 1) / base));
  if (want < 2) return p;
  p.seg_len = (nb + want - 1) / want;
  p.segs = (nb + p.seg_len - 1) / p.seg_len;
  if (p.segs < 2) return SplitPlan{};
  p.planes = 1 + nb - p.seg_len;
  p.rows_pad = wgs * bm;
  return p;
}

// The launch a batch gets: 32*nt tokens a workgroup, and the K split.
struct GemmPlan {
  int nt = 2, bn = 64;
  SplitPlan split;
};

GemmPlan plan_gemm(const GemvJobs& jobs, size_t tokens) {
  GemmPlan g;
  GemvJobs jj = jobs;
  const uint32_t wgs = row_tiles(jj, kRowsWG);
  const uint32_t cus = static_cast<uint32_t>(device_cus());
  if (const int bn = tuning().gemm_bn) {
    g.nt = bn <= 32 ? 1 : 2;
  } else {
    // two 32-token tiles a wave (half the dequantization per MFMA) when
    // that still gives every CU a workgroup
    g.nt = static_cast<size_t>(wgs) * ((tokens + 63) / 64) >= cus ? 2 : 1;
  }
  g.bn = 32 * g.nt;
  // K is split below half a workgroup per CU when rows are long (16 blocks
  // or more) or the grid is under a quarter of the CUs; a short row split
  // over a moderate grid measured slower than unsplit (Q4_K 5632x2048 x 64
  // tokens, 88 workgroups: 19.5 against 15.7 us)
  uint32_t below = cus / 2u;
  if (jobs.n && jobs.j[0].nb < 16u && static_cast<size_t>(wgs) * ((tokens + g.bn - 1) / g.bn) >= cus / 4u)
    below = 0;
  g.split = plan_split(jj, tokens, kRowsWG, static_cast<uint32_t>(g.bn), below);
  return g;
}

template <int FMT, int NT>
hipError_t launch_rows(GemvJobs jobs, const Q8Dev& q, size_t tokens, const SplitPlan& plan, float* terms,
                       hipStream_t s, SplitOut* defer, uint32_t* counters) {
  const uint32_t wgs = row_tiles(jobs, kRowsWG);
  if (wgs == 0) return hipSuccess;
  const uint32_t tiles = static_cast<uint32_t>((tokens + 32u * NT - 1) / (32u * NT));
  constexpr size_t lds = rows_kernel_lds<NT>();
  const bool split = plan.segs > 1 && terms;
  if (!split) {
    hipLaunchKernelGGL((gemm_kq_rows_kernel<FMT, NT, false>), dim3(wgs, tiles), dim3(256), lds, s, jobs, q,
                       tokens, SplitTerms{nullptr, 0u, 0u, 0u, 0u, nullptr});
    return hipGetLastError();
  }
  // the last segment of each tile sums its planes (split_fixup) when they
  // are few, the tiles fit the counters, the tokens come in fours and the
  // planes' byte offsets in 31 bits
  const bool fixup = !defer && counters && tokens % 4u == 0 &&
                     static_cast<size_t>(wgs) * tiles <= kFixupTiles && tuning().gemm_fixup &&
                     plan.planes <= kFixupMaxPlanes &&
                     static_cast<size_t>(plan.planes) * plan.rows_pad * tokens * sizeof(float) <= 0x7fffffffu;
  // token-major planes for the caller, and for the combine of token-major
  // outputs (its reads and stores then both run along rows; every job of a
  // launch has the same tmajor); the fixup's device-coherent plane stores
  // run along tokens ([rows_pad][tokens]) and it transposes through LDS
  const uint32_t tplanes = defer || (!fixup && jobs.j[0].tmajor) ? 1u : 0u;
  hipLaunchKernelGGL((gemm_kq_rows_kernel<FMT, NT, true>), dim3(wgs, tiles, plan.segs), dim3(256), lds, s,
                     jobs, q, tokens,
                     SplitTerms{terms, plan.seg_len, plan.rows_pad, tplanes, plan.planes, fixup ? counters : nullptr});
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess || fixup) return e;
  if (defer) {  // the caller sums the token-major planes in block order itself
    *defer = SplitOut{terms, plan.planes, plan.rows_pad};
    return hipSuccess;
  }
  const size_t n = static_cast<size_t>(plan.rows_pad) * tokens;  // a multiple of 64
  hipLaunchKernelGGL(gemm_combine_kernel, dim3(static_cast<uint32_t>((n / 2u + 255u) / 256u)), dim3(256), 0, s, jobs,
                     terms, plan.planes, plan.rows_pad, tokens, kRowsWG, tplanes);
  return hipGetLastError();
}

template <int FMT>
hipError_t launch_rows_fmt(const GemvJobs& jobs, const Q8Dev& q, size_t tokens, const GemmPlan& g, float* terms,
                           hipStream_t s, SplitOut* defer, uint32_t* counters) {
  return g.nt == 2 ? launch_rows<FMT, 2>(jobs, q, tokens, g.split, terms, s, defer, counters)
                   : launch_rows<FMT, 1>(jobs, q, tokens, g.split, terms, s, defer, counters);
}

}  // namespace

bool gemm_fits(size_t tokens, size_t qstride) {
  return tokens < (size_t{1} << 24) && qstride < (size_t{1} << 24) && tokens * qstride <= size_t{0xffffffffu};
}

size_t gemm_split_bytes(uint32_t type_id, const GemvJobs& jobs, size_t tokens) {
  if (tokens == 0 || (type_id != 12u && type_id != 14u)) return 0;
  const SplitPlan p = plan_gemm(jobs, tokens).split;
  return p.segs > 1 ? static_cast<size_t>(p.planes) * p.rows_pad * tokens * sizeof(float) : 0;
}

hipError_t launch_gemm(uint32_t type_id, const GemvJobs& jobs, const Q8Dev& q, size_t tokens, float* terms,
                       hipStream_t s, SplitOut* defer, uint32_t* counters) {
  if (defer) *defer = SplitOut{};
  if (tokens == 0) return hipSuccess;
  if (!gemm_fits(tokens, q.qstride)) return hipErrorInvalidValue;
  const GemmPlan g = plan_gemm(jobs, tokens);
  if (type_id == 12u) return launch_rows_fmt<12>(jobs, q, tokens, g, terms, s, defer, counters);
  if (type_id == 14u) return launch_rows_fmt<14>(jobs, q, tokens, g, terms, s, defer, counters);
  return hipErrorInvalidValue;
}

}  // namespace rh
