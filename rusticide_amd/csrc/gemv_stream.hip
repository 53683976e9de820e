// gemv_stream.hip -- decode GEMV (one or two tokens) that streams rows past
// lanes with a fixed column assignment.
//
// Every lane owns the same columns of every row it visits, so the quantized
// activation of those columns (and everything derived from the activation
// alone: block sums, d8, Q6_K's -32 offsets, I2_S's quant sums) is loaded into
// registers once per wave. No LDS and no barrier: a wave issues the loads of
// U row groups at once, decodes them in registers and reduces in-wave.
//
// k-quants: 4 lanes per 256-weight block, BP blocks per pass (a row segment
// of 4*BP lanes), P passes per row. A block's integer sums are reduced over
// its quad with DPP; its float term is formed exactly as
// portable/int_dot.rs:169 (Q4_K) or :203 (Q6_K) does; the segment's first
// lane then adds the terms of the row in block order from -0.0, the order of
// portable/int_dot/rows.rs:59. Results are bit-identical to the CPU path.
//
// I2_S: LPR lanes per row, each owning up to CPL 16-byte chunks; the i32 dot
// is reduced with wrapping adds (order-free) and scaled once per row
// (portable/ternary.rs:48-58).
#include <cstdlib>

#include "rh_device.h"
#include "rh_internal.h"

namespace rh {

namespace {

constexpr uint32_t kWaves = 4;  // waves per workgroup

struct StreamGeom {
  uint32_t bp;      // blocks per pass (k-quants) / lanes per row (I2_S)
  uint32_t groups;  // row groups per wave
};

// The wave's job and first row group; waves of a job are contiguous.
__device__ __forceinline__ uint32_t wave_job(const GemvJobs& jobs, uint32_t gw) {
  uint32_t j = 0;
#pragma unroll
  for (uint32_t i = 1; i < static_cast<uint32_t>(kMaxJobs); i++)
    if (i < jobs.n && gw >= jobs.j[i].wg_begin) j = i;
  return j;
}

// Two register buffers of U row groups each: the loads of the next U groups
// are in flight while the current U groups are decoded, so the memory system
// never idles behind the wave's own arithmetic. `groups` is a multiple of U.
template <int U, typename Buf, typename Load, typename Compute>
__device__ __forceinline__ void pipeline(Load& load, Compute& compute, uint32_t groups) {
  Buf x, y;
  load(x, 0u);
  for (uint32_t it = 0; it < groups; it += 2u * U) {
    load(y, it + U);
    compute(x, it);
    if (it + U >= groups) break;
    load(x, it + 2u * U);
    compute(y, it + U);
  }
}

// Q4_K -------------------------------------------------------------------
template <int T, int P, int U>
__global__ __launch_bounds__(256) void q4k_stream_kernel(GemvJobs jobs, Q8Dev q, StreamGeom geo,
                                                         size_t tokens, size_t t0) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t gw = blockIdx.x * kWaves + (threadIdx.x >> 6);
  const GemvJob& J = jobs.j[wave_job(jobs, gw)];
  const uint32_t BP = geo.bp, LPR = 4u * BP, RW = 64u / LPR;
  const uint32_t nb = J.nb;
  static_assert(P == 1 || P == 2, "one or two passes");
  const uint32_t rsub = lane / LPR, bl = (lane % LPR) >> 2, p4 = lane & 3u;
  const uint32_t j0 = 2u * (p4 >> 1), e0 = 16u * (p4 & 1u);
  const bool min_lane = (p4 & 1u) == 0;

  // activation of this lane's columns, per pass and token
  u32x4 act[P][T][4];
  int32_t S[P][T][4];
  float d8[P][T];
#pragma unroll
  for (int k = 0; k < P; k++) {
    const uint32_t b = k * BP + bl;
    const uint32_t bb = b < nb ? b : 0u;
#pragma unroll
    for (int t = 0; t < T; t++) {
      const int8_t* a = q.quants + (t0 + t) * q.qstride + bb * 256u + 32u * j0 + e0;
      act[k][t][0] = load16(reinterpret_cast<const uint8_t*>(a));
      act[k][t][1] = load16(reinterpret_cast<const uint8_t*>(a + 32));
      act[k][t][2] = load16(reinterpret_cast<const uint8_t*>(a + 128));
      act[k][t][3] = load16(reinterpret_cast<const uint8_t*>(a + 160));
      const int32_t* s = q.sums + (t0 + t) * q.bstride + bb * 8u + j0;
      S[k][t][0] = s[0];
      S[k][t][1] = s[1];
      S[k][t][2] = s[4];
      S[k][t][3] = s[5];
      d8[k][t] = q.scales[(t0 + t) * q.bstride + bb * 8u];
    }
  }

  const uint32_t g0 = (gw - J.wg_begin) * geo.groups;
  const uint32_t seg0 = rsub * LPR;
  struct Raw {
    u32x4 hd, c0, c1;
  };
  auto load = [&](Raw (&r)[U][P], uint32_t it) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const uint32_t row = (g0 + it + u) * RW + rsub;
#pragma unroll
      for (int k = 0; k < P; k++) {
        const uint32_t b = k * BP + bl;
        if (it < geo.groups && row < J.rows && b < nb) {
          const uint8_t* blk = J.w + static_cast<size_t>(row) * J.stride + static_cast<size_t>(b) * 144u;
          r[u][k].hd = load16(blk);
          r[u][k].c0 = load16(blk + 16u + 16u * p4);
          r[u][k].c1 = load16(blk + 80u + 16u * p4);
        } else {
          r[u][k].hd = r[u][k].c0 = r[u][k].c1 = u32x4{0, 0, 0, 0};
        }
      }
    }
  };
  auto compute = [&](const Raw (&r)[U][P], uint32_t it) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const uint32_t row = (g0 + it + u) * RW + rsub;
      float term[P][T];
#pragma unroll
      for (int k = 0; k < P; k++) {
        const u32x4 h = r[u][k].hd;
        const int32_t sc0 = static_cast<int32_t>(bfe(h.y, 8u * j0, 6));
        const int32_t sc1 = static_cast<int32_t>(bfe(h.y, 8u * j0 + 8u, 6));
        const int32_t sc2 = static_cast<int32_t>(bfe(h.w, 8u * j0, 4) | (bfe(h.y, 8u * j0 + 6u, 2) << 4));
        const int32_t sc3 = static_cast<int32_t>(bfe(h.w, 8u * j0 + 8u, 4) | (bfe(h.y, 8u * j0 + 14u, 2) << 4));
        const int32_t m0 = static_cast<int32_t>(bfe(h.z, 8u * j0, 6));
        const int32_t m1 = static_cast<int32_t>(bfe(h.z, 8u * j0 + 8u, 6));
        const int32_t m2 = static_cast<int32_t>(bfe(h.w, 8u * j0 + 4u, 4) | (bfe(h.z, 8u * j0 + 6u, 2) << 4));
        const int32_t m3 = static_cast<int32_t>(bfe(h.w, 8u * j0 + 12u, 4) | (bfe(h.z, 8u * j0 + 14u, 2) << 4));
        const float d = f16_lo(h.x), dmin = f16_hi(h.x);
        uint32_t lo0[4], hi0[4], lo1[4], hi1[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
          lo0[i] = r[u][k].c0[i] & 0x0F0F0F0Fu;
          hi0[i] = (r[u][k].c0[i] >> 4) & 0x0F0F0F0Fu;
          lo1[i] = r[u][k].c1[i] & 0x0F0F0F0Fu;
          hi1[i] = (r[u][k].c1[i] >> 4) & 0x0F0F0F0Fu;
        }
#pragma unroll
        for (int t = 0; t < T; t++) {
          int32_t D0 = 0, D1 = 0, D2 = 0, D3 = 0;
#pragma unroll
          for (int i = 0; i < 4; i++) {
            D0 = dot4(lo0[i], act[k][t][0][i], D0);
            D1 = dot4(hi0[i], act[k][t][1][i], D1);
            D2 = dot4(lo1[i], act[k][t][2][i], D2);
            D3 = dot4(hi1[i], act[k][t][3][i], D3);
          }
          int32_t isum = sc0 * D0 + sc1 * D1 + sc2 * D2 + sc3 * D3;
          int32_t msum = min_lane ? (m0 * S[k][t][0] + m1 * S[k][t][1] + m2 * S[k][t][2] + m3 * S[k][t][3]) : 0;
          isum = quad_sum(isum);
          msum = quad_sum(msum);
          // int_dot.rs:169: d8 * d.mul_add(isum, -(dmin * msum))
          const float neg = -(dmin * static_cast<float>(msum));
          term[k][t] = d8[k][t] * __builtin_fmaf(d, static_cast<float>(isum), neg);
        }
      }
      // the row's terms in block order, from -0.0 (rows.rs:59)
#pragma unroll
      for (int t = 0; t < T; t++) {
        float s = -0.0f;
        auto gather = [&](float tk, uint32_t first) {
          for (uint32_t i = 0; i < BP; i++) {
            const float v = __shfl(tk, static_cast<int>(seg0 + 4u * i), 64);
            if (first + i < nb) s += v;
          }
        };
        gather(term[0][t], 0u);
        if (P > 1) gather(term[P - 1][t], BP);
        const size_t idx = static_cast<size_t>(row) * tokens + t0 + t;
        if (lane == seg0 && row < J.rows && idx < J.out_len) J.out[idx] = s;
      }
    }
  };
  pipeline<U, Raw[U][P]>(load, compute, geo.groups);
}

// Q6_K -------------------------------------------------------------------
template <int T, int P, int U>
__global__ __launch_bounds__(256) void q6k_stream_kernel(GemvJobs jobs, Q8Dev q, StreamGeom geo,
                                                         size_t tokens, size_t t0) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t gw = blockIdx.x * kWaves + (threadIdx.x >> 6);
  const GemvJob& J = jobs.j[wave_job(jobs, gw)];
  const uint32_t BP = geo.bp, LPR = 4u * BP, RW = 64u / LPR;
  const uint32_t nb = J.nb;
  const uint32_t rsub = lane / LPR, bl = (lane % LPR) >> 2, p4 = lane & 3u;
  const uint32_t h = p4 >> 1, gq = p4 & 1u;

  u32x4 act[P][T][4];
  int32_t bias[P][T][4];
  float d8[P][T];
#pragma unroll
  for (int k = 0; k < P; k++) {
    const uint32_t b = k * BP + bl;
    const uint32_t bb = b < nb ? b : 0u;
#pragma unroll
    for (int t = 0; t < T; t++) {
      const int8_t* a = q.quants + (t0 + t) * q.qstride + bb * 256u + 128u * h + 16u * gq;
#pragma unroll
      for (int r = 0; r < 4; r++) act[k][t][r] = load16(reinterpret_cast<const uint8_t*>(a + 32 * r));
      // -32 * the activation sum of run r's 16 values (the six_bit offset,
      // int_dot.rs:174-176, folded into the dot's starting value)
      const int32_t* s16 = q.sums16 + 2u * (t0 + t) * q.bstride + bb * 16u + 8u * h + gq;
#pragma unroll
      for (int r = 0; r < 4; r++) bias[k][t][r] = -32 * s16[2 * r];
      d8[k][t] = q.scales[(t0 + t) * q.bstride + bb * 8u];
    }
  }

  const uint32_t g0 = (gw - J.wg_begin) * geo.groups;
  const uint32_t seg0 = rsub * LPR;
  // raw aligned dwords of one lane's windows, realigned after they arrive.
  // Rows start 16-byte aligned, so block b sits (210*b) mod 4 = 2*(b & 1)
  // bytes past a dword boundary.
  struct Raw {
    u32x4 A, B, C, W, E;  // E: the fifth dwords of A, B, C and dwords 4, 5 of W
  };
  auto load = [&](Raw (&r)[U][P], uint32_t it) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const uint32_t row = (g0 + it + u) * RW + rsub;
#pragma unroll
      for (int k = 0; k < P; k++) {
        const uint32_t b = k * BP + bl;
        Raw& x = r[u][k];
        if (it < geo.groups && row < J.rows && b < nb) {
          const uint8_t* blk = J.w + static_cast<size_t>(row) * J.stride + static_cast<size_t>(b) * 210u;
          const uint8_t* base = blk - 2u * (b & 1u);
          // ql[64h+16gq..], ql[64h+32+16gq..], qh[32h+16gq..] (quantize/src/q6_k.rs:13-43)
          x.A = load16_a4(base + 64u * h + 16u * gq);
          x.B = load16_a4(base + 64u * h + 32u + 16u * gq);
          x.C = load16_a4(base + 128u + 32u * h + 16u * gq);
          // scales[16] at 192 and d at 208
          x.W = load16_a4(base + 192u);
          x.E = u32x4{load4(base + 64u * h + 16u * gq + 16u), load4(base + 64u * h + 48u + 16u * gq),
                      load4(base + 144u + 32u * h + 16u * gq), load4(base + 208u)};
        } else {
          x.A = x.B = x.C = x.W = x.E = u32x4{0, 0, 0, 0};
        }
      }
    }
  };
  auto compute = [&](const Raw (&r)[U][P], uint32_t it) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const uint32_t row = (g0 + it + u) * RW + rsub;
      float term[P][T];
#pragma unroll
      for (int k = 0; k < P; k++) {
        const Raw& x = r[u][k];
        const uint32_t sh = 2u * ((k * BP + bl) & 1u);
        const u32x4 a{__builtin_amdgcn_alignbyte(x.A.y, x.A.x, sh), __builtin_amdgcn_alignbyte(x.A.z, x.A.y, sh),
                      __builtin_amdgcn_alignbyte(x.A.w, x.A.z, sh), __builtin_amdgcn_alignbyte(x.E.x, x.A.w, sh)};
        const u32x4 bq{__builtin_amdgcn_alignbyte(x.B.y, x.B.x, sh), __builtin_amdgcn_alignbyte(x.B.z, x.B.y, sh),
                       __builtin_amdgcn_alignbyte(x.B.w, x.B.z, sh), __builtin_amdgcn_alignbyte(x.E.y, x.B.w, sh)};
        const u32x4 c{__builtin_amdgcn_alignbyte(x.C.y, x.C.x, sh), __builtin_amdgcn_alignbyte(x.C.z, x.C.y, sh),
                      __builtin_amdgcn_alignbyte(x.C.w, x.C.z, sh), __builtin_amdgcn_alignbyte(x.E.z, x.C.w, sh)};
        const uint32_t X0 = __builtin_amdgcn_alignbyte(x.W.y, x.W.x, sh);
        const uint32_t X1 = __builtin_amdgcn_alignbyte(x.W.z, x.W.y, sh);
        const uint32_t X2 = __builtin_amdgcn_alignbyte(x.W.w, x.W.z, sh);
        const uint32_t X3 = __builtin_amdgcn_alignbyte(x.E.w, x.W.w, sh);
        // d sits at bytes 208..209: within dword 4 of the window for either shift
        const uint32_t X4 = x.E.w >> (8u * sh);
        const uint32_t slo = h ? X2 : X0, shi = h ? X3 : X1;
        // scale of run r, 16-group gq: scales[8h + 2r + gq] (int_dot.rs:199)
        const int32_t sc0 = __builtin_amdgcn_sbfe(static_cast<int32_t>(slo), 8u * gq, 8);
        const int32_t sc1 = __builtin_amdgcn_sbfe(static_cast<int32_t>(slo), 8u * gq + 16u, 8);
        const int32_t sc2 = __builtin_amdgcn_sbfe(static_cast<int32_t>(shi), 8u * gq, 8);
        const int32_t sc3 = __builtin_amdgcn_sbfe(static_cast<int32_t>(shi), 8u * gq + 16u, 8);
        const float d = f16_lo(X4);
        uint32_t q0[4], q1[4], q2[4], q3[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
          q0[i] = (a[i] & 0x0F0F0F0Fu) | ((c[i] << 4) & 0x30303030u);
          q1[i] = (bq[i] & 0x0F0F0F0Fu) | ((c[i] << 2) & 0x30303030u);
          q2[i] = ((a[i] >> 4) & 0x0F0F0F0Fu) | (c[i] & 0x30303030u);
          q3[i] = ((bq[i] >> 4) & 0x0F0F0F0Fu) | ((c[i] >> 2) & 0x30303030u);
        }
#pragma unroll
        for (int t = 0; t < T; t++) {
          int32_t D0 = bias[k][t][0], D1 = bias[k][t][1], D2 = bias[k][t][2], D3 = bias[k][t][3];
#pragma unroll
          for (int i = 0; i < 4; i++) {
            D0 = dot4(q0[i], act[k][t][0][i], D0);
            D1 = dot4(q1[i], act[k][t][1][i], D1);
            D2 = dot4(q2[i], act[k][t][2][i], D2);
            D3 = dot4(q3[i], act[k][t][3][i], D3);
          }
          const int32_t isum = quad_sum(sc0 * D0 + sc1 * D1 + sc2 * D2 + sc3 * D3);
          // int_dot.rs:203: (d * d8) * isum
          const float dd = d * d8[k][t];
          term[k][t] = dd * static_cast<float>(isum);
        }
      }
#pragma unroll
      for (int t = 0; t < T; t++) {
        float s = -0.0f;
        auto gather = [&](float tk, uint32_t first) {
          for (uint32_t i = 0; i < BP; i++) {
            const float v = __shfl(tk, static_cast<int>(seg0 + 4u * i), 64);
            if (first + i < nb) s += v;
          }
        };
        gather(term[0][t], 0u);
        if (P > 1) gather(term[P - 1][t], BP);
        const size_t idx = static_cast<size_t>(row) * tokens + t0 + t;
        if (lane == seg0 && row < J.rows && idx < J.out_len) J.out[idx] = s;
      }
    }
  };
  pipeline<U, Raw[U][P]>(load, compute, geo.groups);
}

// I2_S -------------------------------------------------------------------
template <int T, int CPL, int U>
__global__ __launch_bounds__(256) void i2s_stream_kernel(GemvJobs jobs, Q8Dev q, StreamGeom geo,
                                                         size_t tokens, size_t t0, int32_t* raw) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t gw = blockIdx.x * kWaves + (threadIdx.x >> 6);
  const GemvJob& J = jobs.j[wave_job(jobs, gw)];
  const uint32_t LPR = geo.bp, RW = 64u / LPR;
  const uint32_t nchunk = 2u * J.nb;
  const uint32_t rsub = lane / LPR, cl = lane % LPR;

  u32x4 act[CPL][T][4];
#pragma unroll
  for (int i = 0; i < CPL; i++) {
    const uint32_t c = cl + i * LPR;
    const uint32_t cc = c < nchunk ? c : 0u;
#pragma unroll
    for (int t = 0; t < T; t++) {
      const int8_t* a = q.quants + (t0 + t) * q.qstride + 128u * (cc >> 1) + 16u * (cc & 1u);
#pragma unroll
      for (int L = 0; L < 4; L++) act[i][t][L] = load16(reinterpret_cast<const uint8_t*>(a + 32 * L));
    }
  }
  // sum of the quants the row's blocks cover (ternary.rs:39), per token
  uint32_t qsum[T];
#pragma unroll
  for (int t = 0; t < T; t++) {
    uint32_t acc = 0;
    for (uint32_t i = lane; i < 4u * J.nb; i += 64u) acc += static_cast<uint32_t>(q.sums[(t0 + t) * q.bstride + i]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc += static_cast<uint32_t>(__shfl_xor(static_cast<int>(acc), off, 64));
    qsum[t] = acc;
  }
  float divisor[T];
#pragma unroll
  for (int t = 0; t < T; t++) divisor[t] = q.n_blocks ? q.scales[(t0 + t) * q.bstride] : 0.0f;

  const uint32_t g0 = (gw - J.wg_begin) * geo.groups;
  struct Raw {
    u32x4 w;
  };
  auto load = [&](Raw (&r)[U][CPL], uint32_t it) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const uint32_t row = (g0 + it + u) * RW + rsub;
#pragma unroll
      for (int i = 0; i < CPL; i++) {
        const uint32_t c = cl + i * LPR;
        if (it < geo.groups && row < J.rows && c < nchunk)
          r[u][i].w = load16(J.w + static_cast<size_t>(row) * J.stride + 16u * c);
        else
          r[u][i].w = u32x4{0, 0, 0, 0};  // code 0 adds nothing to sum(code * q)
      }
    }
  };
  auto compute = [&](const Raw (&r)[U][CPL], uint32_t it) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const uint32_t row = (g0 + it + u) * RW + rsub;
      uint32_t acc[T];
#pragma unroll
      for (int t = 0; t < T; t++) acc[t] = 0;
#pragma unroll
      for (int i = 0; i < CPL; i++) {
        uint32_t c6[4], c4[4], c2[4], c0[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
          const uint32_t x = r[u][i].w[k];
          c6[k] = (x >> 2) & 0x30303030u;  // shift 6, times 16
          c4[k] = x & 0x30303030u;         // shift 4, times 16
          c2[k] = x & 0x0C0C0C0Cu;         // shift 2, times 4
          c0[k] = x & 0x03030303u;         // shift 0
        }
#pragma unroll
        for (int t = 0; t < T; t++) {
          int32_t P16 = 0, P4 = 0, P1 = 0;
#pragma unroll
          for (int k = 0; k < 4; k++) {
            P16 = dot4(c6[k], act[i][t][0][k], P16);
            P16 = dot4(c4[k], act[i][t][1][k], P16);
            P4 = dot4(c2[k], act[i][t][2][k], P4);
            P1 = dot4(c0[k], act[i][t][3][k], P1);
          }
          acc[t] += static_cast<uint32_t>(P1 + (P4 >> 2) + (P16 >> 4));
        }
      }
#pragma unroll
      for (int t = 0; t < T; t++) {
        uint32_t v = acc[t];
        for (uint32_t off = LPR >> 1; off > 0; off >>= 1)
          v += static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), static_cast<int>(off), 64));
        // sum(code * q) over the row's chunks minus sum(q) over its blocks
        const int32_t dot = static_cast<int32_t>(v - qsum[t]);
        const size_t idx = static_cast<size_t>(row) * tokens + t0 + t;
        if (cl == 0 && row < J.rows && idx < J.out_len) {
          if (raw) raw[idx] = dot;
          else J.out[idx] = q.n_blocks ? __fdiv_rn(static_cast<float>(dot), divisor[t]) * J.scale : 0.0f;
        }
      }
    }
  };
  pipeline<U, Raw[U][CPL]>(load, compute, geo.groups);
}

template <typename K>
hipError_t launch(K kernel, GemvJobs& jobs, uint32_t rw, uint32_t groups_hint, const Q8Dev& q,
                  StreamGeom geo, size_t tokens, size_t t0, hipStream_t s, int32_t* raw, bool ternary) {
  (void)groups_hint;
  uint32_t waves = 0;
  for (uint32_t i = 0; i < jobs.n; i++) {
    jobs.j[i].wg_begin = waves;  // first wave of the job
    const uint32_t groups = (jobs.j[i].rows + rw - 1u) / rw;
    waves += (groups + geo.groups - 1u) / geo.groups;
  }
  const uint32_t wgs = (waves + kWaves - 1u) / kWaves;
  if (wgs == 0) return hipSuccess;
  if (ternary)
    hipLaunchKernelGGL(reinterpret_cast<void (*)(GemvJobs, Q8Dev, StreamGeom, size_t, size_t, int32_t*)>(kernel),
                       dim3(wgs), dim3(256), 0, s, jobs, q, geo, tokens, t0, raw);
  else
    hipLaunchKernelGGL(reinterpret_cast<void (*)(GemvJobs, Q8Dev, StreamGeom, size_t, size_t)>(kernel),
                       dim3(wgs), dim3(256), 0, s, jobs, q, geo, tokens, t0);
  return hipGetLastError();
}

uint32_t pow2_at_least(uint32_t v) {
  uint32_t p = 1;
  while (p < v) p <<= 1;
  return p;
}

// Row groups per wave, a multiple of U: about `target` waves over the launch
// (RUSTICIDE_HIP_STREAM_WAVES overrides the default of 2048, for tuning).
uint32_t groups_per_wave(uint32_t total_groups, uint32_t U) {
  uint32_t target = 2048u;
  if (const char* v = std::getenv("RUSTICIDE_HIP_STREAM_WAVES")) {
    const long n = std::strtol(v, nullptr, 10);
    if (n > 0) target = static_cast<uint32_t>(n);
  }
  uint32_t g = (total_groups + target - 1u) / target;
  g = g < U ? U : g;
  return (g + U - 1u) / U * U;
}

}  // namespace

bool launch_gemv_stream(uint32_t type_id, GemvJobs jobs, const Q8Dev& q, size_t tokens, size_t t0,
                        size_t tn, hipStream_t s, int32_t* raw, hipError_t* err) {
  *err = hipSuccess;
  if (tn < 1 || tn > 2 || jobs.n == 0) return false;
  const uint32_t nb = jobs.j[0].nb;
  uint32_t total_rows = 0;
  for (uint32_t i = 0; i < jobs.n; i++) {
    if (jobs.j[i].nb != nb) return false;  // one geometry per launch
    total_rows += jobs.j[i].rows;
  }
  if (nb == 0) return false;
  if (type_id == 12u || type_id == 14u) {
    const uint32_t bp = nb >= 16u ? 16u : pow2_at_least(nb);
    const uint32_t passes = (nb + bp - 1u) / bp;
    if (passes > 2u) return false;
    // two passes hold twice the activation registers: one row group per stage
    const uint32_t U = passes == 1 ? 2u : 1u;
    const uint32_t rw = 64u / (4u * bp);
    StreamGeom geo{bp, groups_per_wave((total_rows + rw - 1u) / rw, U)};
    void* k = nullptr;
    if (type_id == 12u)
      k = passes == 1 ? (tn == 1 ? reinterpret_cast<void*>(q4k_stream_kernel<1, 1, 2>)
                                 : reinterpret_cast<void*>(q4k_stream_kernel<2, 1, 2>))
                      : (tn == 1 ? reinterpret_cast<void*>(q4k_stream_kernel<1, 2, 1>)
                                 : reinterpret_cast<void*>(q4k_stream_kernel<2, 2, 1>));
    else
      k = passes == 1 ? (tn == 1 ? reinterpret_cast<void*>(q6k_stream_kernel<1, 1, 2>)
                                 : reinterpret_cast<void*>(q6k_stream_kernel<2, 1, 2>))
                      : (tn == 1 ? reinterpret_cast<void*>(q6k_stream_kernel<1, 2, 1>)
                                 : reinterpret_cast<void*>(q6k_stream_kernel<2, 2, 1>));
    *err = launch(k, jobs, rw, 0, q, geo, tokens, t0, s, nullptr, false);
    return true;
  }
  if (type_id == 36u) {
    constexpr uint32_t U = 2;
    const uint32_t nchunk = 2u * nb;
    const uint32_t lpr = nchunk <= 48u ? 32u : 64u;
    const uint32_t cpl = (nchunk + lpr - 1u) / lpr;
    if (cpl > 2u) return false;
    const uint32_t rw = 64u / lpr;
    StreamGeom geo{lpr, groups_per_wave((total_rows + rw - 1u) / rw, U)};
    void* k = cpl == 1 ? (tn == 1 ? reinterpret_cast<void*>(i2s_stream_kernel<1, 1, U>)
                                  : reinterpret_cast<void*>(i2s_stream_kernel<2, 1, U>))
                       : (tn == 1 ? reinterpret_cast<void*>(i2s_stream_kernel<1, 2, U>)
                                  : reinterpret_cast<void*>(i2s_stream_kernel<2, 2, U>));
    *err = launch(k, jobs, rw, 0, q, geo, tokens, t0, s, raw, true);
    return true;
  }
  return false;
}

}  // namespace rh
