// gemv_kq.hip -- persistent decode GEMV for the k-quants (Q4_K, Q6_K) on gfx950.
//
// A resident workgroup stages the quantized activation of its tokens in LDS
// once, then walks row tiles of every matrix in the launch with a grid
// stride. The weight loads of the next tile are issued before the current
// tile is decoded, so each workgroup keeps a tile of HBM traffic in flight
// while its arithmetic runs, and no workgroup waits for a second generation.
//
// Inside a tile each 4-lane team decodes up to two 256-weight super-blocks in
// registers: integer sums with v_dot4_i32_i8 and DPP quad reductions (exact),
// then the block's float term exactly as the CPU path forms it
// (crates/rusticide-kernels/src/portable/int_dot.rs:169 for Q4_K, :203 for
// Q6_K). The terms of a row are added in block order from -0.0 by one lane
// (portable/int_dot/rows.rs:59), so outputs are bit-identical to the CPU path.
#include <cstdlib>

#include "rh_device.h"
#include "rh_internal.h"

namespace rh {

namespace {

constexpr uint32_t kThreads = 256;
constexpr uint32_t kTeams = kThreads / 4u;
constexpr int kNI = 2;  // blocks per team per tile

__device__ __forceinline__ uint32_t tile_job(const GemvJobs& jobs, uint32_t gt) {
  uint32_t j = 0;
#pragma unroll
  for (uint32_t i = 1; i < static_cast<uint32_t>(kMaxJobs); i++)
    if (i < jobs.n && gt >= jobs.j[i].wg_begin) j = i;
  return j;
}

struct TileGeom {
  uint32_t R;      // rows per tile
  uint32_t nbmax;  // largest blocks-per-row of the launch
  uint32_t tiles;  // tiles over all jobs
};

// Raw bytes of one team's block: Q4_K uses w[0..2] (header, two quarters of
// qs); Q6_K uses all five (ql, ql, qh windows, scales, fifth dwords + d).
struct Raw {
  u32x4 w[5];
};

template <int FMT>
__device__ __forceinline__ void load_block(Raw& x, const uint8_t* row, uint32_t b, uint32_t p) {
  if (FMT == 12) {
    const uint8_t* blk = row + static_cast<size_t>(b) * 144u;
    x.w[0] = load16(blk);
    x.w[1] = load16(blk + 16u + 16u * p);
    x.w[2] = load16(blk + 80u + 16u * p);
  } else {
    // rows start 16-byte aligned: block b sits 2*(b & 1) bytes past a dword
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

// LDS: act [T][nbmax*256] i8 | d8 [T][nbmax] f32 | side [T][nbmax*16] i32
// (Q4_K: the 8 block sums; Q6_K: -32 * the 16 run sums) | terms [2][R][nbmax][T]
template <int FMT, int T>
__global__ __launch_bounds__(256) void gemv_kq_kernel(GemvJobs jobs, Q8Dev q, TileGeom geo, size_t tokens,
                                                      size_t t0) {
  extern __shared__ __align__(16) uint8_t lds[];
  const uint32_t nbmax = geo.nbmax, R = geo.R;
  const uint32_t abytes = nbmax * 256u;
  int8_t* act = reinterpret_cast<int8_t*>(lds);
  float* d8 = reinterpret_cast<float*>(lds + T * abytes);
  int32_t* side = reinterpret_cast<int32_t*>(d8 + T * nbmax);
  float* terms = reinterpret_cast<float*>(side + T * nbmax * 16u);
  const uint32_t tstride = R * nbmax * T;  // one of the two term buffers

  const uint32_t team = threadIdx.x >> 2, p = threadIdx.x & 3u;

  // the first tile's weights are requested before anything else
  Raw bufa[kNI], bufb[kNI];
  auto issue = [&](Raw (&buf)[kNI], uint32_t gt) {
    if (gt >= geo.tiles) return;  // uniform
    const GemvJob& J = jobs.j[tile_job(jobs, gt)];
    const uint32_t row0 = (gt - J.wg_begin) * R;
    const uint32_t nrows = min(R, J.rows - row0);
    const uint32_t nb = J.nb, total = nrows * nb;
#pragma unroll
    for (int i = 0; i < kNI; i++) {
      const uint32_t g = team + i * kTeams;
      const uint32_t gg = g < total ? g : 0u;  // spare teams re-read block 0
      const uint32_t r = nb ? gg / nb : 0u, b = gg - r * nb;
      load_block<FMT>(buf[i], J.w + static_cast<size_t>(row0 + r) * J.stride, b, p);
    }
  };
  uint32_t gt = blockIdx.x;
  issue(bufa, gt);

  // stage the activation once per workgroup; chunk c of block b goes to
  // chunk c ^ (b & 15) so the teams of a wave read distinct LDS banks
  for (uint32_t t = 0; t < static_cast<uint32_t>(T); t++) {
    const int8_t* src = q.quants + (t0 + t) * q.qstride;
    for (uint32_t i = threadIdx.x * 16u; i < abytes; i += kThreads * 16u) {
      const uint32_t b = i >> 8, c = (i >> 4) & 15u;
      *reinterpret_cast<u32x4*>(act + t * abytes + (b << 8) + ((c ^ (b & 15u)) << 4)) =
          *reinterpret_cast<const u32x4*>(src + i);
    }
  }
  auto swz = [](const int8_t* act_t, uint32_t b, uint32_t k) {
    return act_t + (b << 8) + ((((k >> 4) ^ (b & 15u))) << 4);
  };
  for (uint32_t i = threadIdx.x; i < T * nbmax * 16u; i += kThreads) {
    const uint32_t t = i / (nbmax * 16u), k = i - t * nbmax * 16u;
    if (FMT == 12) {
      if (k < nbmax * 8u) {
        const size_t src = (t0 + t) * q.bstride + k;
        side[t * nbmax * 16u + k] = q.sums[src];
        if ((k & 7u) == 0) d8[t * nbmax + k / 8u] = q.scales[src];
      }
    } else {
      side[i] = -32 * q.sums16[2u * (t0 + t) * q.bstride + k];
      if ((k & 15u) == 0) d8[t * nbmax + k / 16u] = q.scales[(t0 + t) * q.bstride + k / 2u];
    }
  }
  __syncthreads();

  const uint32_t h = p >> 1, gq = p & 1u;           // Q6_K lane roles
  const uint32_t j0 = 2u * (p >> 1), e0 = 16u * (p & 1u);  // Q4_K lane roles
  const bool min_lane = (p & 1u) == 0;

  // one tile from the register set `cur`, after the next tile's loads go
  // into `nxt`; the two sets alternate (a copy between them would wait for
  // the loads just issued)
  auto tile = [&](const Raw (&cur)[kNI], Raw (&nxt)[kNI], uint32_t k, uint32_t gt) {
    issue(nxt, gt + gridDim.x);
    const GemvJob& J = jobs.j[tile_job(jobs, gt)];
    const uint32_t row0 = (gt - J.wg_begin) * R;
    const uint32_t nrows = min(R, J.rows - row0);
    const uint32_t nb = J.nb, total = nrows * nb;
    float* tb = terms + (k & 1u) * tstride;
#pragma unroll
    for (int it = 0; it < kNI; it++) {
      const uint32_t g = team + it * kTeams;
      if (g >= total) break;  // uniform over the team
      const uint32_t r = g / nb, b = g - r * nb;
      const Raw& x = cur[it];
      if (FMT == 12) {
        const u32x4 hd = x.w[0];
        // 6-bit scales/mins of sub-blocks j0, j0+1, j0+4, j0+5 (ggml
        // get_scale_min_k4, quantize/src/q4_k.rs:17-25)
        const int32_t sc0 = static_cast<int32_t>(bfe(hd.y, 8u * j0, 6));
        const int32_t sc1 = static_cast<int32_t>(bfe(hd.y, 8u * j0 + 8u, 6));
        const int32_t sc2 = static_cast<int32_t>(bfe(hd.w, 8u * j0, 4) | (bfe(hd.y, 8u * j0 + 6u, 2) << 4));
        const int32_t sc3 = static_cast<int32_t>(bfe(hd.w, 8u * j0 + 8u, 4) | (bfe(hd.y, 8u * j0 + 14u, 2) << 4));
        const int32_t m0 = static_cast<int32_t>(bfe(hd.z, 8u * j0, 6));
        const int32_t m1 = static_cast<int32_t>(bfe(hd.z, 8u * j0 + 8u, 6));
        const int32_t m2 = static_cast<int32_t>(bfe(hd.w, 8u * j0 + 4u, 4) | (bfe(hd.z, 8u * j0 + 6u, 2) << 4));
        const int32_t m3 = static_cast<int32_t>(bfe(hd.w, 8u * j0 + 12u, 4) | (bfe(hd.z, 8u * j0 + 14u, 2) << 4));
        const float d = f16_lo(hd.x), dmin = f16_hi(hd.x);
        uint32_t lo0[4], hi0[4], lo1[4], hi1[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
          lo0[i] = x.w[1][i] & 0x0F0F0F0Fu;
          hi0[i] = (x.w[1][i] >> 4) & 0x0F0F0F0Fu;
          lo1[i] = x.w[2][i] & 0x0F0F0F0Fu;
          hi1[i] = (x.w[2][i] >> 4) & 0x0F0F0F0Fu;
        }
#pragma unroll
        for (int t = 0; t < T; t++) {
          const int8_t* at = act + t * abytes;
          const uint32_t k0 = e0 + 32u * j0;
          const u32x4 a0 = *reinterpret_cast<const u32x4*>(swz(at, b, k0));
          const u32x4 a1 = *reinterpret_cast<const u32x4*>(swz(at, b, k0 + 32u));
          const u32x4 a2 = *reinterpret_cast<const u32x4*>(swz(at, b, k0 + 128u));
          const u32x4 a3 = *reinterpret_cast<const u32x4*>(swz(at, b, k0 + 160u));
          int32_t D0 = 0, D1 = 0, D2 = 0, D3 = 0;
#pragma unroll
          for (int i = 0; i < 4; i++) {
            D0 = dot4(lo0[i], a0[i], D0);
            D1 = dot4(hi0[i], a1[i], D1);
            D2 = dot4(lo1[i], a2[i], D2);
            D3 = dot4(hi1[i], a3[i], D3);
          }
          int32_t isum = __mul24(sc0, D0) + __mul24(sc1, D1) + __mul24(sc2, D2) + __mul24(sc3, D3);
          const int32_t* S = side + t * nbmax * 16u + b * 8u + j0;
          int32_t msum =
              min_lane ? (__mul24(m0, S[0]) + __mul24(m1, S[1]) + __mul24(m2, S[4]) + __mul24(m3, S[5])) : 0;
          isum = quad_sum(isum);
          msum = quad_sum(msum);
          if (p == 0) {
            // int_dot.rs:169: d8 * d.mul_add(isum, -(dmin * msum))
            const float neg = -(dmin * static_cast<float>(msum));
            tb[(r * nbmax + b) * T + t] = d8[t * nbmax + b] * __builtin_fmaf(d, static_cast<float>(isum), neg);
          }
        }
      } else {
        const uint32_t sh = 2u * (b & 1u);
        const u32x4 A = x.w[0], B = x.w[1], C = x.w[2], W = x.w[3], E = x.w[4];
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
        // scale of run r, 16-group gq: scales[8h + 2r + gq] (int_dot.rs:199)
        const int32_t sc0 = __builtin_amdgcn_sbfe(static_cast<int32_t>(slo), 8u * gq, 8);
        const int32_t sc1 = __builtin_amdgcn_sbfe(static_cast<int32_t>(slo), 8u * gq + 16u, 8);
        const int32_t sc2 = __builtin_amdgcn_sbfe(static_cast<int32_t>(shi), 8u * gq, 8);
        const int32_t sc3 = __builtin_amdgcn_sbfe(static_cast<int32_t>(shi), 8u * gq + 16u, 8);
        const float d = f16_lo(E.w >> (8u * sh));  // bytes 208..209
        // six-bit weights, offset by 32 through the dot's starting value
        // (q6_k.rs:10-11, int_dot.rs:174-176)
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
          const int8_t* at = act + t * abytes;
          const uint32_t k0 = 128u * h + 16u * gq;
          const u32x4 a0 = *reinterpret_cast<const u32x4*>(swz(at, b, k0));
          const u32x4 a1 = *reinterpret_cast<const u32x4*>(swz(at, b, k0 + 32u));
          const u32x4 a2 = *reinterpret_cast<const u32x4*>(swz(at, b, k0 + 64u));
          const u32x4 a3 = *reinterpret_cast<const u32x4*>(swz(at, b, k0 + 96u));
          const int32_t* bb = side + t * nbmax * 16u + b * 16u + 8u * h + gq;
          int32_t D0 = bb[0], D1 = bb[2], D2 = bb[4], D3 = bb[6];
#pragma unroll
          for (int i = 0; i < 4; i++) {
            D0 = dot4(q0[i], a0[i], D0);
            D1 = dot4(q1[i], a1[i], D1);
            D2 = dot4(q2[i], a2[i], D2);
            D3 = dot4(q3[i], a3[i], D3);
          }
          const int32_t isum = quad_sum(__mul24(sc0, D0) + __mul24(sc1, D1) + __mul24(sc2, D2) + __mul24(sc3, D3));
          if (p == 0) {
            // int_dot.rs:203: read_f16_le(block, 208) * span.scales[0] * lossy(sum)
            const float dd = d * d8[t * nbmax + b];
            tb[(r * nbmax + b) * T + t] = dd * static_cast<float>(isum);
          }
        }
      }
    }
    __syncthreads();
    // each row's terms in block order, from -0.0 (rows.rs:59)
    for (uint32_t i = threadIdx.x; i < nrows * T; i += kThreads) {
      const uint32_t r = i / T, t = i - r * T;
      float s = -0.0f;
      for (uint32_t b = 0; b < nb; b++) s += tb[(r * nbmax + b) * T + t];
      const size_t idx = static_cast<size_t>(row0 + r) * tokens + t0 + t;
      if (idx < J.out_len) J.out[idx] = s;
    }
  };
  for (uint32_t k = 0; gt < geo.tiles; k += 2u, gt += 2u * gridDim.x) {
    tile(bufa, bufb, k, gt);
    if (gt + gridDim.x >= geo.tiles) break;
    tile(bufb, bufa, k + 1u, gt + gridDim.x);
  }
}

size_t kq_lds_bytes(uint32_t T, uint32_t nbmax, uint32_t R) {
  return static_cast<size_t>(T) * nbmax * 256u + T * nbmax * 4u + T * nbmax * 64u + 2u * R * nbmax * T * 4u;
}

uint32_t kq_rows(uint32_t nb) {
  const uint32_t R = static_cast<uint32_t>(kNI) * kTeams / nb;
  return R < 1u ? 1u : R;
}

template <int FMT, int T>
hipError_t launch_kq(GemvJobs jobs, const Q8Dev& q, uint32_t nbmax, size_t tokens, size_t t0, hipStream_t s) {
  const uint32_t R = kq_rows(nbmax);
  uint32_t tiles = 0;
  for (uint32_t i = 0; i < jobs.n; i++) {
    jobs.j[i].wg_begin = tiles;  // first tile of the job
    tiles += (jobs.j[i].rows + R - 1u) / R;
  }
  if (tiles == 0) return hipSuccess;
  const size_t lds = kq_lds_bytes(T, nbmax, R);
  // resident workgroups: measured once per (format, tokens, shape) bucket
  static int per_cu[2][8] = {};
  int& occ = per_cu[FMT == 12 ? 0 : 1][T - 1];
  if (occ == 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, gemv_kq_kernel<FMT, T>, kThreads, lds) != hipSuccess || n < 1)
      n = 1;
    occ = n;
  }
  int cus = 256;
  int dev = 0;
  if (hipGetDevice(&dev) == hipSuccess) hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  uint32_t grid = static_cast<uint32_t>(occ) * static_cast<uint32_t>(cus);
  if (const char* v = std::getenv("RUSTICIDE_HIP_KQ_GRID")) {
    const long g = std::strtol(v, nullptr, 10);
    if (g > 0) grid = static_cast<uint32_t>(g);
  }
  grid = grid < tiles ? grid : tiles;
  TileGeom geo{R, nbmax, tiles};
  hipLaunchKernelGGL((gemv_kq_kernel<FMT, T>), dim3(grid), dim3(kThreads), lds, s, jobs, q, geo, tokens, t0);
  return hipGetLastError();
}

}  // namespace

size_t gemv_kq_max_tokens(uint32_t nb) {
  // a tile's teams cover kNI * kTeams blocks: wider rows go to the LDS kernels
  if (nb == 0 || nb > static_cast<uint32_t>(kNI) * kTeams) return 0;
  for (uint32_t t = 4; t >= 1; t--)
    if (kq_lds_bytes(t, nb, kq_rows(nb)) <= 64u * 1024u) return t;
  return 0;
}

hipError_t launch_gemv_kq(uint32_t type_id, const GemvJobs& jobs, const Q8Dev& q, uint32_t nbmax, size_t tokens,
                          size_t t0, size_t tn, hipStream_t s) {
  if (type_id == 12u) {
    switch (tn) {
      case 1: return launch_kq<12, 1>(jobs, q, nbmax, tokens, t0, s);
      case 2: return launch_kq<12, 2>(jobs, q, nbmax, tokens, t0, s);
      case 3: return launch_kq<12, 3>(jobs, q, nbmax, tokens, t0, s);
      case 4: return launch_kq<12, 4>(jobs, q, nbmax, tokens, t0, s);
      default: return hipErrorInvalidValue;
    }
  }
  switch (tn) {
    case 1: return launch_kq<14, 1>(jobs, q, nbmax, tokens, t0, s);
    case 2: return launch_kq<14, 2>(jobs, q, nbmax, tokens, t0, s);
    case 3: return launch_kq<14, 3>(jobs, q, nbmax, tokens, t0, s);
    case 4: return launch_kq<14, 4>(jobs, q, nbmax, tokens, t0, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace rh
