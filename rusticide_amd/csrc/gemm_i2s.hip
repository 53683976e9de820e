// gemm_i2s.hip -- prefill GEMM for I2_S ternary weights against I8_S
// activations on gfx950 int8 matrix cores, bit-identical to rusticide's CPU
// path.
//
// The CPU path (crates/rusticide-kernels/src/portable/ternary.rs:11-57) forms,
// per (row, token), the i32 dot sum(code * q) - sum(q) over the row's
// 128-weight blocks with wrapping adds, then (dot as f32) / s * scale. Since
// code*q - q = (code - 1)*q, the weights enter v_mfma_i32_32x32x32_i8 as
// code - 1 in {-1, 0, 1, 2} (code 3 is +2, quantize/src/i2_s.rs:96-104) and
// the activations as their I8_S quants; the MFMA's i32 sums are exact (modulo
// 2^32, as the wrapping adds are). There is no per-block float work: one
// division and one product per output.
//
// Tiles: a workgroup of four waves owns 128 rows x BN tokens, and wave w owns
// rows 32w .. 32w + 32 outright. For 32-deep step kk of a block, lane
// row + 32g needs weights 32kk + 16g .. + 16 of its row, which sit in packed
// bytes 16g .. 16g + 16 at shift 6 - 2kk (quantize/src/i2_s.rs:12-21): one
// 16-byte load a block gives the lane all four steps' A operands, decoded in
// registers. Only the activation tile (the B operand, shared by the four
// waves) goes through LDS, double-buffered, one barrier a block.
//
// The loop is latency-bound on its loads (a block's MFMAs are 4 BN/32 of
// them a wave), so each block's bytes are requested kAhead blocks before
// they are used: block k's registers are set k % (kAhead + 1), and the loop
// is unrolled over the sets so that each is named by a constant (a register
// copy between sets would wait for the newest loads too). Every load is
// unconditional (past the last block it reads the last block again), so the
// loads in flight are counted exactly at each wait.
#include "rh_device.h"
#include "rh_internal.h"

namespace rh {

namespace {

constexpr uint32_t kThreads = 256;
constexpr uint32_t kRowsWG = 128;  // rows per workgroup, 32 a wave
constexpr uint32_t kRow = 144;     // LDS bytes per 128-byte activation row: +16 spreads the banks
constexpr int kAhead = 3;          // blocks requested ahead

typedef int32_t v4i __attribute__((ext_vector_type(4)));
typedef int32_t v16i __attribute__((ext_vector_type(16)));

__device__ __forceinline__ uint32_t job_index(const GemvJobs& jobs, uint32_t wg) {
  uint32_t j = 0;
#pragma unroll
  for (uint32_t i = 1; i < static_cast<uint32_t>(kMaxJobs); i++)
    if (i < jobs.n && wg >= jobs.j[i].wg_begin) j = i;
  return j;
}

// Four 2-bit codes (one per byte, 0..3) minus one: a byte table lookup
// (v_perm_b32 picks byte c of 0x020100FF: -1, 0, 1, 2 for codes 0..3).
__device__ __forceinline__ uint32_t codes_minus_one(uint32_t x) {
  return __builtin_amdgcn_perm(0u, 0x020100FFu, x);
}

template <int BN>
__global__ __launch_bounds__(256) void gemm_i2s_kernel(GemvJobs jobs, Q8Dev q, size_t tokens, int32_t* raw) {
  extern __shared__ __align__(16) uint8_t lds[];
  constexpr int NTT = BN / 32;             // 32-token tiles per wave
  constexpr int ACH = BN * 8 / kThreads;   // 16-byte activation chunks per thread per block
  constexpr int NS = kAhead + 1;           // register sets
  const GemvJob& J = jobs.j[job_index(jobs, blockIdx.x)];
  const uint32_t row0 = (blockIdx.x - J.wg_begin) * kRowsWG + 32u * (threadIdx.x >> 6);
  const uint32_t tok0 = blockIdx.y * BN;
  const uint32_t nb = J.nb;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, g = lane >> 5, ml = lane & 31u;
  const size_t T = tokens;

  // the lane's row (clamped to the last) and half-block; the thread's
  // activation chunks: token tok0 + chunk/8, bytes 16 (chunk % 8) ..
  const uint8_t* wr = J.w + static_cast<size_t>(min(row0 + ml, J.rows - 1u)) * J.stride + 16u * g;
  const int8_t* arow[ACH];
#pragma unroll
  for (int c = 0; c < ACH; c++) {
    const uint32_t chunk = tid + static_cast<uint32_t>(c) * kThreads;
    const size_t tok = min(static_cast<size_t>(tok0 + (chunk >> 3)), T - 1);
    arow[c] = q.quants + tok * q.qstride + (chunk & 7u) * 16u;
  }

  // a block's registers: the lane's packed weights and its activation chunks
  struct Set {
    u32x4 w;
    u32x4 a[ACH];
  };
  auto load = [&](Set& x, uint32_t b) {
    x.w = load16(wr + static_cast<size_t>(b) * 32u);
#pragma unroll
    for (int c = 0; c < ACH; c++)
      x.a[c] = load16(reinterpret_cast<const uint8_t*>(arow[c] + static_cast<size_t>(b) * 128u));
  };
  auto store_a = [&](const Set& x, uint32_t buf) {
    uint8_t* at = lds + buf * BN * kRow;
#pragma unroll
    for (int c = 0; c < ACH; c++) {
      const uint32_t chunk = tid + static_cast<uint32_t>(c) * kThreads;
      *reinterpret_cast<u32x4*>(at + (chunk >> 3) * kRow + (chunk & 7u) * 16u) = x.a[c];
    }
  };

  v16i acc[NTT];
#pragma unroll
  for (int t = 0; t < NTT; t++) acc[t] = v16i{};

  Set S[NS];
  if (nb) {
#pragma unroll
    for (int k = 0; k < kAhead; k++) load(S[k], min(static_cast<uint32_t>(k), nb - 1u));
    store_a(S[0], 0u);
    __syncthreads();
  }
  for (uint32_t b0 = 0; b0 < nb; b0 += NS) {
#pragma unroll
    for (int ph = 0; ph < NS; ph++) {
      const uint32_t b = b0 + static_cast<uint32_t>(ph);
      if (b >= nb) break;
      load(S[(ph + kAhead) % NS], min(b + kAhead, nb - 1u));
      const u32x4 w = S[ph].w;
      const int8_t* at = reinterpret_cast<const int8_t*>(lds + (b & 1u) * BN * kRow);
#pragma unroll
      for (uint32_t kk = 0; kk < 4u; kk++) {
        const uint32_t shift = 6u - 2u * kk;
        v4i A;
#pragma unroll
        for (int i = 0; i < 4; i++) A[i] = static_cast<int32_t>(codes_minus_one((w[i] >> shift) & 0x03030303u));
#pragma unroll
        for (int t = 0; t < NTT; t++) {
          const v4i Bv = *reinterpret_cast<const v4i*>(at + (32u * t + ml) * kRow + 32u * kk + 16u * g);
          acc[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, Bv, acc[t], 0, 0, 0);
        }
      }
      // block b+1's activation (requested kAhead - 1 blocks ago) to the other buffer
      if (b + 1u < nb) store_a(S[(ph + 1) % NS], (b & 1u) ^ 1u);
      __syncthreads();
    }
  }

  // ternary.rs:53-57: (dot as f32) / s * scale, 0 without an activation
  // (D layout: lane n + 32*((m/4)%2), register 4*(m/8) + m%4)
#pragma unroll
  for (int t = 0; t < NTT; t++) {
    const size_t tok = tok0 + 32u * t + ml;
    if (tok >= T) continue;
    const float s = q.n_blocks ? q.scales[tok * q.bstride] : 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const uint32_t m = 8u * static_cast<uint32_t>(i >> 2) + 4u * g + static_cast<uint32_t>(i & 3);
      const uint32_t row = row0 + m;
      if (row >= J.rows) continue;
      const size_t idx = static_cast<size_t>(row) * T + tok;
      if (idx >= J.out_len) continue;
      const int32_t dot = acc[t][i];
      if (raw) raw[idx] = dot;
      else J.out[idx] = q.n_blocks ? __fdiv_rn(static_cast<float>(dot), s) * J.scale : 0.0f;
    }
  }
}

template <int BN>
hipError_t launch_bn(GemvJobs jobs, const Q8Dev& q, size_t tokens, int32_t* raw, hipStream_t s) {
  uint32_t wgs = 0;
  for (uint32_t i = 0; i < jobs.n; i++) {
    jobs.j[i].wg_begin = wgs;
    wgs += (jobs.j[i].rows + kRowsWG - 1u) / kRowsWG;
  }
  if (wgs == 0) return hipSuccess;
  const uint32_t tiles = static_cast<uint32_t>((tokens + BN - 1) / BN);
  hipLaunchKernelGGL((gemm_i2s_kernel<BN>), dim3(wgs, tiles), dim3(kThreads), 2u * BN * kRow, s, jobs, q, tokens,
                     raw);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm_i2s(const GemvJobs& jobs, const Q8Dev& q, size_t tokens, int32_t* raw, hipStream_t s) {
  if (tokens == 0 || jobs.n == 0) return hipSuccess;
  // 64 tokens a workgroup when that still gives every CU one and a half
  // workgroups, else 32 (6912x2560: 23.6 against 26.0 us at 512 tokens,
  // 61.6 against 74.3 at 2048; 2560x6912 at 512 tokens: 28.3 against 33.1 at
  // 64, its 160 workgroups too few); tuning().gemm_bn forces it
  uint32_t row_tiles = 0;
  for (uint32_t i = 0; i < jobs.n; i++) row_tiles += (jobs.j[i].rows + kRowsWG - 1u) / kRowsWG;
  const size_t wgs64 = static_cast<size_t>(row_tiles) * ((tokens + 63) / 64);
  int bn = 2u * wgs64 >= 3u * static_cast<size_t>(device_cus()) ? 64 : 32;
  if (const int v = tuning().gemm_bn) bn = v <= 32 ? 32 : 64;
  return bn == 64 ? launch_bn<64>(jobs, q, tokens, raw, s) : launch_bn<32>(jobs, q, tokens, raw, s);
}

}  // namespace rh
