// gemm.hip -- prefill GEMM on gfx950 matrix cores: Q4_K / Q6_K weights in
// their native GGUF blocks against Q8_K-quantized activations of many tokens,
// bit-identical to rusticide's CPU integer path.
//
// The CPU path (crates/rusticide-kernels/src/portable/int_dot.rs:142-204)
// forms, per 256-weight super-block b of row r and token t, exact integers
//   Q4_K: isum = sum_j sc_j * sum_l q*a, msum = sum_j m_j * bsum_j
//   Q6_K: isum = sum_s sc_s * sum_l (q-32)*a
// and one float term per block, added in block order. Here the integers come
// from int8 MFMA (v_mfma_i32_32x32x32_i8), exact in i32:
//   * the sub-block scale is folded into the weight, w = sc*q (Q4_K: 0..945;
//     Q6_K: sc*(q-32), -4096..4064), split into two int8 planes w = 128*hi +
//     lo (lo in 0..127). Two accumulators take the hi and the lo plane side
//     by side over the block's eight 32-deep steps (each activation fragment
//     read from LDS once for both); isum = 128*hi + lo;
//   * the Q4_K min term needs only the block sums: with bsum = 128*bh + bl
//     (bl in 0..127), msum = 128 * sum_j m_j*bh_j + sum_j m_j*bl_j, two MFMAs
//     whose 32-deep operands carry the eight (m_j, bl_j) / (m_j, bh_j) pairs
//     in one lane group and zeros elsewhere. Each lane gives A and B the same
//     k for the same byte, so the order MFMA sums k in does not matter.
// The float combine is the CPU path's, per block, in block order, one
// accumulator per (row, token) in one lane.
//
// Tiles: a workgroup of 4 waves owns 64 rows x BN tokens; wave w computes rows
// 32*(w&1).. and tokens (w>>1)*BN/2.. as BN/64 32x32 MFMA tiles. Per block:
// weights are dequantized into LDS planes once per workgroup, the block's
// activation tile and block-sum bytes are copied in, and the next block's raw
// bytes are already in flight in registers while the MFMAs of this one run.
//
// Split K: when the row and token tiles give too few workgroups to fill the
// chip (a 64-token prefill of a 2048-row matrix is 32 of them), blockIdx.z
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

constexpr uint32_t kThreads = 256;
constexpr uint32_t kBM = 64;        // rows per workgroup
constexpr uint32_t kStride = 272;   // LDS bytes per 256-byte row: +16 spreads the banks

typedef int32_t v4i __attribute__((ext_vector_type(4)));
typedef int32_t v16i __attribute__((ext_vector_type(16)));
typedef int16_t s16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t gemm_job(const GemvJobs& jobs, uint32_t wg) {
  uint32_t j = 0;
#pragma unroll
  for (uint32_t i = 1; i < static_cast<uint32_t>(kMaxJobs); i++)
    if (i < jobs.n && wg >= jobs.j[i].wg_begin) j = i;
  return j;
}

// Raw bytes one thread holds for one block of its row (thread = row*4 + p).
// Q4_K: w[0] header (d, dmin, scales[12]), w[1..2] qs[32p..32p+32).
// Q6_K: the GEMV kernels' lane windows for h = p>>1, gq = p&1: w[0] ql at
// 64h+16gq, w[1] ql at 64h+32+16gq, w[2] qh at 32h+16gq, w[3] scales, w[4]
// the fifth dwords of those windows and of the scales (holding d).
struct WRaw {
  u32x4 w[5];
};

template <int FMT>
__device__ __forceinline__ void load_wraw(WRaw& x, const uint8_t* row, uint32_t b, uint32_t p) {
  if (FMT == 12) {
    const uint8_t* blk = row + static_cast<size_t>(b) * 144u;
    x.w[0] = load16(blk);
    x.w[1] = load16(blk + 16u + 32u * p);
    x.w[2] = load16(blk + 32u + 32u * p);
  } else {
    const uint32_t h = p >> 1, gq = p & 1u;
    const uint8_t* base = row + static_cast<size_t>(b) * 210u - 2u * (b & 1u);
    x.w[0] = load16_a4(base + 64u * h + 16u * gq);
    x.w[1] = load16_a4(base + 64u * h + 32u + 16u * gq);
    x.w[2] = load16_a4(base + 128u + 32u * h + 16u * gq);
    x.w[3] = load16_a4(base + 192u);
    x.w[4] = u32x4{load4(base + 64u * h + 16u * gq + 16u), load4(base + 64u * h + 48u + 16u * gq),
                   load4(base + 144u + 32u * h + 16u * gq), load4(base + 208u)};
  }
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

// Four unsigned nibble bytes q (0..15) times sc (0..63) as the hi/lo planes:
// the products are formed two at a time in 16-bit lanes (< 2^16, no carry).
// Both factors are below 2^24, so the full-rate 24-bit multiply is exact.
__device__ __forceinline__ void split4_u(uint32_t q, uint32_t sc, uint32_t& hi, uint32_t& lo) {
  const uint32_t pe = __umul24(q & 0x00FF00FFu, sc);
  const uint32_t po = __umul24((q >> 8) & 0x00FF00FFu, sc);
  lo = (pe & 0x007F007Fu) | ((po & 0x007F007Fu) << 8);
  hi = ((pe >> 7) & 0x00FF00FFu) | (((po >> 7) & 0x00FF00FFu) << 8);
}

// Four six-bit bytes q (0..63) as sc * (q - 32) (sc signed) in hi/lo planes:
// w = 128*hi + lo, lo in 0..127, hi in -32..31 (two's complement bytes). The
// products are formed two at a time in signed 16-bit lanes (|w| <= 4096).
__device__ __forceinline__ void split4_s(uint32_t q, int32_t sc, uint32_t& hi, uint32_t& lo) {
  const s16x2 scv{static_cast<int16_t>(sc), static_cast<int16_t>(sc)};
  const s16x2 off{static_cast<int16_t>(-32 * sc), static_cast<int16_t>(-32 * sc)};
  const uint32_t qe = q & 0x00FF00FFu, qo = (q >> 8) & 0x00FF00FFu;
  const s16x2 we = __builtin_bit_cast(s16x2, qe) * scv + off;
  const s16x2 wo = __builtin_bit_cast(s16x2, qo) * scv + off;
  const uint32_t ue = __builtin_bit_cast(uint32_t, we), uo = __builtin_bit_cast(uint32_t, wo);
  lo = (ue & 0x007F007Fu) | ((uo & 0x007F007Fu) << 8);
  const s16x2 he = we >> static_cast<int16_t>(7), ho = wo >> static_cast<int16_t>(7);
  hi = (__builtin_bit_cast(uint32_t, he) & 0x00FF00FFu) | ((__builtin_bit_cast(uint32_t, ho) & 0x00FF00FFu) << 8);
}

// LDS: hi [64][272] | lo [64][272] | act [BN][272] | mins [64][8] u8 |
//      bsb [BN][16] (bl_0..7, bh_0..7) | rowd [64] float2 (d, dmin) | d8 [BN]
// Terms of a split launch: plane 0 holds segment 0's sums, plane 1 + b -
// seg_len the term of block b >= seg_len; each plane is [rows_pad][tokens]
// over the launch's 64-row tiles.
struct SplitTerms {
  float* terms;       // nullptr: no split
  uint32_t seg_len;   // blocks per segment
  uint32_t rows_pad;  // 64 x the launch's workgroups along rows
};

template <int FMT, int BN, bool SPLIT>
__global__ __launch_bounds__(256) void gemm_kq_kernel(GemvJobs jobs, Q8Dev q, size_t tokens, SplitTerms split) {
  extern __shared__ __align__(16) uint8_t lds[];
  int8_t* hiT = reinterpret_cast<int8_t*>(lds);
  int8_t* loT = hiT + kBM * kStride;
  int8_t* actT = loT + kBM * kStride;
  uint8_t* minsT = reinterpret_cast<uint8_t*>(actT + BN * kStride);
  uint8_t* bsT = minsT + kBM * 8u;
  float2* rowd = reinterpret_cast<float2*>(bsT + BN * 16u);
  float* d8T = reinterpret_cast<float*>(rowd + kBM);

  const GemvJob& J = jobs.j[gemm_job(jobs, blockIdx.x)];
  const uint32_t row0 = (blockIdx.x - J.wg_begin) * kBM;
  const uint32_t tok0 = blockIdx.y * BN;
  const uint32_t nb = J.nb;
  const uint32_t seg = SPLIT ? blockIdx.z : 0u;
  const uint32_t b_begin = SPLIT ? seg * split.seg_len : 0u;
  const uint32_t b_end = SPLIT ? min(nb, b_begin + split.seg_len) : nb;
  const bool store_terms = SPLIT && seg > 0u;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t wm = wave & 1u, wn = wave >> 1;
  constexpr int NT = BN / 64;  // 32x32 tiles per wave along tokens

  // staging roles: one row quarter per thread for the weights, 16-byte
  // chunks of the activation tile, one token's block sums for tid < BN
  const uint32_t sr = tid >> 2, sp = tid & 3u;
  const uint32_t srow = min(row0 + sr, J.rows - 1u);
  const uint8_t* wrow = J.w + __umul24(srow, static_cast<uint32_t>(J.stride));
  constexpr int ACH = BN * 16 / 256;  // activation chunks per thread
  const size_t T = tokens;
  // the launch keeps tokens * qstride below 2^32 and both below 2^24: the
  // activation offsets are exact 32-bit values from 24-bit multiplies
  const uint32_t last = static_cast<uint32_t>(T - 1);
  const uint32_t qs32 = static_cast<uint32_t>(q.qstride), bs32 = static_cast<uint32_t>(q.bstride);
  const uint32_t stok = min(tok0 + (tid & (BN - 1)), last);

  WRaw wr;
  u32x4 ar[ACH];
  u32x4 sr0{}, sr1{};
  float d8r = 0.0f;
  auto prefetch = [&](uint32_t b) {
    load_wraw<FMT>(wr, wrow, b, sp);
#pragma unroll
    for (int c = 0; c < ACH; c++) {
      const uint32_t chunk = tid + static_cast<uint32_t>(c) * kThreads;
      const uint32_t n = chunk >> 4, k = (chunk & 15u) * 16u;
      const uint32_t tok = min(tok0 + n, last);
      ar[c] = load16(reinterpret_cast<const uint8_t*>(q.quants + (__umul24(tok, qs32) + b * 256u + k)));
    }
    if (tid < static_cast<uint32_t>(BN)) {
      const uint32_t o = __umul24(stok, bs32) + b * 8u;
      d8r = q.scales[o];
      if (FMT == 12) {
        sr0 = load16(reinterpret_cast<const uint8_t*>(q.sums + o));
        sr1 = load16(reinterpret_cast<const uint8_t*>(q.sums + o + 4));
      }
    }
  };

  v16i acc_i[NT], acc_m[NT];
  float y[NT][16];
#pragma unroll
  for (int t = 0; t < NT; t++)
#pragma unroll
    for (int i = 0; i < 16; i++) y[t][i] = -0.0f;

  if (b_begin < b_end) prefetch(b_begin);
  for (uint32_t b = b_begin; b < b_end; b++) {
    // raw bytes -> LDS planes
    if (FMT == 12) {
      const u32x4 hd = wr.w[0];
      uint32_t sc0, m0, sc1, m1;
      q4k_scale_min(hd, 2u * sp, sc0, m0);
      q4k_scale_min(hd, 2u * sp + 1u, sc1, m1);
      // qs[32p + l]: low nibble -> k = 64p + l (sub-block 2p), high -> 64p + 32 + l
      uint32_t h0[8], l0[8], h1[8], l1[8];
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const uint32_t v = wr.w[1 + (i >> 2)][i & 3];
        split4_u(v & 0x0F0F0F0Fu, sc0, h0[i], l0[i]);
        split4_u((v >> 4) & 0x0F0F0F0Fu, sc1, h1[i], l1[i]);
      }
      int8_t* hrow = hiT + sr * kStride + 64u * sp;
      int8_t* lrow = loT + sr * kStride + 64u * sp;
#pragma unroll
      for (int i = 0; i < 8; i += 4) {
        *reinterpret_cast<u32x4*>(hrow + 4 * i) = u32x4{h0[i], h0[i + 1], h0[i + 2], h0[i + 3]};
        *reinterpret_cast<u32x4*>(lrow + 4 * i) = u32x4{l0[i], l0[i + 1], l0[i + 2], l0[i + 3]};
        *reinterpret_cast<u32x4*>(hrow + 32 + 4 * i) = u32x4{h1[i], h1[i + 1], h1[i + 2], h1[i + 3]};
        *reinterpret_cast<u32x4*>(lrow + 32 + 4 * i) = u32x4{l1[i], l1[i + 1], l1[i + 2], l1[i + 3]};
      }
      minsT[sr * 8u + 2u * sp] = static_cast<uint8_t>(m0);
      minsT[sr * 8u + 2u * sp + 1u] = static_cast<uint8_t>(m1);
      if (sp == 0) rowd[sr] = make_float2(f16_lo(hd.x), f16_hi(hd.x));
      if (tid < static_cast<uint32_t>(BN)) {
        // bsum_j = 128*bh_j + bl_j, bl_j in 0..127 (|bsum_j| <= 32*127)
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
        *reinterpret_cast<u32x4*>(bsT + tid * 16u) = u32x4{bl[0], bl[1], bh[0], bh[1]};
      }
    } else {
      const uint32_t h = sp >> 1, gq = sp & 1u;
      const uint32_t sh = 2u * (b & 1u);
      const u32x4 A = wr.w[0], B = wr.w[1], C = wr.w[2], W = wr.w[3], E = wr.w[4];
      const u32x4 a{__builtin_amdgcn_alignbyte(A.y, A.x, sh), __builtin_amdgcn_alignbyte(A.z, A.y, sh),
                    __builtin_amdgcn_alignbyte(A.w, A.z, sh), __builtin_amdgcn_alignbyte(E.x, A.w, sh)};
      const u32x4 bq{__builtin_amdgcn_alignbyte(B.y, B.x, sh), __builtin_amdgcn_alignbyte(B.z, B.y, sh),
                     __builtin_amdgcn_alignbyte(B.w, B.z, sh), __builtin_amdgcn_alignbyte(E.y, B.w, sh)};
      const u32x4 c{__builtin_amdgcn_alignbyte(C.y, C.x, sh), __builtin_amdgcn_alignbyte(C.z, C.y, sh),
                    __builtin_amdgcn_alignbyte(C.w, C.z, sh), __builtin_amdgcn_alignbyte(E.z, C.w, sh)};
      const uint32_t X0 = __builtin_amdgcn_alignbyte(W.y, W.x, sh);
      const uint32_t X1 = __builtin_amdgcn_alignbyte(W.z, W.y, sh);
      const uint32_t X2 = __builtin_amdgcn_alignbyte(W.w, W.z, sh);
      const uint32_t X3 = __builtin_amdgcn_alignbyte(E.w, W.w, sh);
      const uint32_t slo = h ? X2 : X0, shi = h ? X3 : X1;
      // run r, 16-group gq: scales[8h + 2r + gq] (int_dot.rs:199)
      int32_t scr[4];
      scr[0] = __builtin_amdgcn_sbfe(static_cast<int32_t>(slo), 8u * gq, 8);
      scr[1] = __builtin_amdgcn_sbfe(static_cast<int32_t>(slo), 8u * gq + 16u, 8);
      scr[2] = __builtin_amdgcn_sbfe(static_cast<int32_t>(shi), 8u * gq, 8);
      scr[3] = __builtin_amdgcn_sbfe(static_cast<int32_t>(shi), 8u * gq + 16u, 8);
      // element 128h + 32r + 16gq + l holds run r's value l (q6_k.rs:13-43)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        uint32_t hw[4], lw[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
          const uint32_t qv = r == 0 ? (a[k] & 0x0F0F0F0Fu) | ((c[k] << 4) & 0x30303030u)
                            : r == 1 ? (bq[k] & 0x0F0F0F0Fu) | ((c[k] << 2) & 0x30303030u)
                            : r == 2 ? ((a[k] >> 4) & 0x0F0F0F0Fu) | (c[k] & 0x30303030u)
                                     : ((bq[k] >> 4) & 0x0F0F0F0Fu) | ((c[k] >> 2) & 0x30303030u);
          split4_s(qv, scr[r], hw[k], lw[k]);
        }
        const uint32_t k0 = 128u * h + 32u * static_cast<uint32_t>(r) + 16u * gq;
        *reinterpret_cast<u32x4*>(hiT + sr * kStride + k0) = u32x4{hw[0], hw[1], hw[2], hw[3]};
        *reinterpret_cast<u32x4*>(loT + sr * kStride + k0) = u32x4{lw[0], lw[1], lw[2], lw[3]};
      }
      if (sp == 0) rowd[sr] = make_float2(f16_lo(E.w >> (8u * sh)), 0.0f);
    }
#pragma unroll
    for (int cch = 0; cch < ACH; cch++) {
      const uint32_t chunk = tid + static_cast<uint32_t>(cch) * kThreads;
      *reinterpret_cast<u32x4*>(actT + (chunk >> 4) * kStride + (chunk & 15u) * 16u) = ar[cch];
    }
    if (tid < static_cast<uint32_t>(BN)) d8T[tid] = d8r;
    __syncthreads();
    if (b + 1u < b_end) prefetch(b + 1u);

    const uint32_t arow = 32u * wm + (lane & 31u);
    const uint32_t g = lane >> 5;  // the lane's 16-byte k group of a 32-deep step
    uint32_t bcol[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) bcol[t] = static_cast<uint32_t>(BN / 2) * wn + 32u * static_cast<uint32_t>(t) + (lane & 31u);
#pragma unroll
    for (int t = 0; t < NT; t++) acc_i[t] = v16i{};
    v16i acc_l[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) acc_l[t] = v16i{};
    // hi and lo planes side by side per 32-deep step: each activation
    // fragment is read from LDS once
#pragma unroll
    for (uint32_t kk = 0; kk < 8u; kk++) {
      const uint32_t ko = 32u * kk + 16u * g;
      const v4i Ah = *reinterpret_cast<const v4i*>(hiT + arow * kStride + ko);
      const v4i Al = *reinterpret_cast<const v4i*>(loT + arow * kStride + ko);
#pragma unroll
      for (int t = 0; t < NT; t++) {
        const v4i Bv = *reinterpret_cast<const v4i*>(actT + bcol[t] * kStride + ko);
        acc_i[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(Ah, Bv, acc_i[t], 0, 0, 0);
        acc_l[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(Al, Bv, acc_l[t], 0, 0, 0);
      }
    }
    if (FMT == 12) {
      // msum: (m_j, bh_j) then x128, then (m_j, bl_j), in lane group 0
      const uint32_t mw0 = g == 0 ? *reinterpret_cast<const uint32_t*>(minsT + arow * 8u) : 0u;
      const uint32_t mw1 = g == 0 ? *reinterpret_cast<const uint32_t*>(minsT + arow * 8u + 4u) : 0u;
      const v4i Am{static_cast<int32_t>(mw0), static_cast<int32_t>(mw1), 0, 0};
#pragma unroll
      for (int t = 0; t < NT; t++) {
        const u32x4 bs = *reinterpret_cast<const u32x4*>(bsT + bcol[t] * 16u);
        const v4i Bh{g == 0 ? static_cast<int32_t>(bs.z) : 0, g == 0 ? static_cast<int32_t>(bs.w) : 0, 0, 0};
        acc_m[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(Am, Bh, v16i{}, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 16; i++) acc_m[t][i] <<= 7;
        const v4i Bl{g == 0 ? static_cast<int32_t>(bs.x) : 0, g == 0 ? static_cast<int32_t>(bs.y) : 0, 0, 0};
        acc_m[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(Am, Bl, acc_m[t], 0, 0, 0);
      }
    }
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
      for (int i = 0; i < 16; i++) acc_i[t][i] = (acc_i[t][i] << 7) + acc_l[t][i];
    // the block's float term per (row, token), added in block order
    // (D layout: lane n + 32*((m/4)%2), register 4*(m/8) + m%4)
    float d8n[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) d8n[t] = d8T[bcol[t]];
    float* plane = store_terms ? split.terms + static_cast<size_t>(1u + b - split.seg_len) * split.rows_pad * T
                               : nullptr;
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const uint32_t m = 32u * wm + 8u * static_cast<uint32_t>(i >> 2) + 4u * g + static_cast<uint32_t>(i & 3);
      const float2 dd = rowd[m];
#pragma unroll
      for (int t = 0; t < NT; t++) {
        float term;
        if (FMT == 12) {
          // int_dot.rs:169: d8 * d.mul_add(isum, -(dmin * msum))
          const float neg = -(dd.y * static_cast<float>(acc_m[t][i]));
          term = d8n[t] * __builtin_fmaf(dd.x, static_cast<float>(acc_i[t][i]), neg);
        } else {
          // int_dot.rs:203: (d * d8) * isum
          const float s = dd.x * d8n[t];
          term = s * static_cast<float>(acc_i[t][i]);
        }
        if (store_terms) {
          const size_t tok = tok0 + static_cast<uint32_t>(BN / 2) * wn + 32u * static_cast<uint32_t>(t) + (lane & 31u);
          if (tok < T) plane[static_cast<size_t>(blockIdx.x * kBM + m) * T + tok] = term;
        } else {
          y[t][i] += term;
        }
      }
    }
    __syncthreads();
  }
  if (store_terms) return;

  const uint32_t g = lane >> 5;
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const uint32_t m = 32u * wm + 8u * static_cast<uint32_t>(i >> 2) + 4u * g + static_cast<uint32_t>(i & 3);
    const uint32_t row = row0 + m;
    if (row >= J.rows) continue;
#pragma unroll
    for (int t = 0; t < NT; t++) {
      const size_t tok = tok0 + static_cast<uint32_t>(BN / 2) * wn + 32u * static_cast<uint32_t>(t) + (lane & 31u);
      if (SPLIT) {  // segment 0 of a split launch: plane 0
        if (tok < T) split.terms[static_cast<size_t>(blockIdx.x * kBM + m) * T + tok] = y[t][i];
        continue;
      }
      const size_t idx = static_cast<size_t>(row) * T + tok;
      if (tok < T && idx < J.out_len) J.out[idx] = y[t][i];
    }
  }
}

// The end of a split launch: per (row, token), segment 0's sum plus the later
// blocks' terms, one addition at a time in block order.
// Each thread owns four consecutive (row, token) slots (a plane holds a
// multiple of 64 of them) and keeps eight planes of loads in flight; the
// additions stay one plane at a time, in block order.
__global__ __launch_bounds__(256) void gemm_combine_kernel(GemvJobs jobs, const float* __restrict__ terms,
                                                           uint32_t planes, uint32_t rows_pad, size_t tokens) {
  const size_t n = static_cast<size_t>(rows_pad) * tokens;
  const size_t idx = (static_cast<size_t>(blockIdx.x) * 256u + threadIdx.x) * 4u;
  if (idx >= n) return;
  f32x4 y = *reinterpret_cast<const f32x4*>(terms + idx);
  uint32_t p = 1;
  for (; p + 8u <= planes; p += 8u) {
    f32x4 v[8];
#pragma unroll
    for (int k = 0; k < 8; k++) v[k] = *reinterpret_cast<const f32x4*>(terms + static_cast<size_t>(p + k) * n + idx);
#pragma unroll
    for (int k = 0; k < 8; k++) y += v[k];
  }
  for (; p < planes; p++) y += *reinterpret_cast<const f32x4*>(terms + static_cast<size_t>(p) * n + idx);
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const uint32_t grow = static_cast<uint32_t>((idx + e) / tokens);
    const size_t tok = idx + e - static_cast<size_t>(grow) * tokens;
    const GemvJob& J = jobs.j[gemm_job(jobs, grow / kBM)];
    const uint32_t row = grow - J.wg_begin * kBM;
    const size_t o = static_cast<size_t>(row) * tokens + tok;
    if (row < J.rows && o < J.out_len) J.out[o] = y[e];
  }
}

int token_tile(size_t tokens) {
  // Tuning::gemm_bn forces the token tile (64 or 128 here), for tuning
  if (const int bn = tuning().gemm_bn) return bn == 256 ? 128 : bn;
  return tokens >= 512 ? 128 : 64;
}

// Workgroups along rows, with each job's first one recorded in wg_begin.
uint32_t row_tiles(GemvJobs& jobs) {
  uint32_t wgs = 0;
  for (uint32_t i = 0; i < jobs.n; i++) {
    jobs.j[i].wg_begin = wgs;
    wgs += (jobs.j[i].rows + kBM - 1u) / kBM;
  }
  return wgs;
}

struct SplitPlan {
  uint32_t segs = 1, seg_len = 0, planes = 0, rows_pad = 0;
};

// Splits K when the launch has fewer than kSplitBelow workgroups, aiming at
// kSplitTarget; every job must have the same block count. Below 2 blocks, or
// with Tuning::gemm_split off, nothing is split.
constexpr uint32_t kSplitBelow = 128, kSplitTarget = 512;

SplitPlan plan_split(GemvJobs jobs, size_t tokens) {
  SplitPlan p;
  const uint32_t wgs = row_tiles(jobs);
  if (wgs == 0 || jobs.n == 0) return p;
  const uint32_t nb = jobs.j[0].nb;
  for (uint32_t i = 1; i < jobs.n; i++)
    if (jobs.j[i].nb != nb) return p;
  if (!tuning().gemm_split) return p;
  const size_t tiles = (tokens + token_tile(tokens) - 1) / token_tile(tokens);
  const size_t base = static_cast<size_t>(wgs) * tiles;
  if (nb < 2 || base >= kSplitBelow) return p;
  const uint32_t want = static_cast<uint32_t>(std::min<size_t>(nb, (kSplitTarget + base - 1) / base));
  if (want < 2) return p;
  p.seg_len = (nb + want - 1) / want;
  p.segs = (nb + p.seg_len - 1) / p.seg_len;
  if (p.segs < 2) return SplitPlan{};
  p.planes = 1 + nb - p.seg_len;
  p.rows_pad = wgs * kBM;
  return p;
}

template <int FMT, int BN>
hipError_t launch_bn(GemvJobs jobs, const Q8Dev& q, size_t tokens, const SplitPlan& plan, float* terms,
                     hipStream_t s) {
  const uint32_t wgs = row_tiles(jobs);
  if (wgs == 0) return hipSuccess;
  const uint32_t tiles = static_cast<uint32_t>((tokens + BN - 1) / BN);
  const size_t lds = 2u * kBM * kStride + BN * kStride + kBM * 8u + BN * 16u + kBM * 8u + BN * 4u;
  const bool split = plan.segs > 1 && terms;
  if (!split) {
    hipLaunchKernelGGL((gemm_kq_kernel<FMT, BN, false>), dim3(wgs, tiles), dim3(kThreads), lds, s, jobs, q, tokens,
                       SplitTerms{nullptr, 0u, 0u});
    return hipGetLastError();
  }
  hipLaunchKernelGGL((gemm_kq_kernel<FMT, BN, true>), dim3(wgs, tiles, plan.segs), dim3(kThreads), lds, s, jobs, q,
                     tokens, SplitTerms{terms, plan.seg_len, plan.rows_pad});
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const size_t n = static_cast<size_t>(plan.rows_pad) * tokens;  // a multiple of 64
  hipLaunchKernelGGL(gemm_combine_kernel, dim3(static_cast<uint32_t>((n / 4u + 255u) / 256u)), dim3(256), 0, s, jobs,
                     terms, plan.planes, plan.rows_pad, tokens);
  return hipGetLastError();
}

}  // namespace

bool gemm_fits(size_t tokens, size_t qstride) {
  return tokens < (size_t{1} << 24) && qstride < (size_t{1} << 24) && tokens * qstride <= size_t{0xffffffffu};
}

size_t gemm_split_bytes(uint32_t type_id, const GemvJobs& jobs, size_t tokens) {
  if (tokens == 0 || (type_id != 12u && type_id != 14u)) return 0;
  const SplitPlan p = plan_split(jobs, tokens);
  return p.segs > 1 ? static_cast<size_t>(p.planes) * p.rows_pad * tokens * sizeof(float) : 0;
}

hipError_t launch_gemm(uint32_t type_id, const GemvJobs& jobs, const Q8Dev& q, size_t tokens, float* terms,
                       hipStream_t s) {
  if (tokens == 0) return hipSuccess;
  if (!gemm_fits(tokens, q.qstride)) return hipErrorInvalidValue;
  const SplitPlan plan = plan_split(jobs, tokens);
  const int bn = token_tile(tokens);
  if (type_id == 12u)
    return bn == 128 ? launch_bn<12, 128>(jobs, q, tokens, plan, terms, s)
                     : launch_bn<12, 64>(jobs, q, tokens, plan, terms, s);
  if (type_id == 14u)
    return bn == 128 ? launch_bn<14, 128>(jobs, q, tokens, plan, terms, s)
                     : launch_bn<14, 64>(jobs, q, tokens, plan, terms, s);
  return hipErrorInvalidValue;
}

}  // namespace rh
