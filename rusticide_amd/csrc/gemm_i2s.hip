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
// Tiles: a workgroup of 4 waves owns 128 rows x BN tokens; wave (wm, wn)
// computes rows 64*wm.. as two 32-row tiles and tokens (BN/2)*wn.. as BN/64
// 32-token tiles. K advances one 128-weight block per step through two LDS
// stages. Two register sets carry the packed codes and quants of the next
// two blocks: block b+1 is stored to LDS while block b's MFMAs run, from
// loads issued two steps earlier.
#include "rh_device.h"
#include "rh_internal.h"

namespace rh {

namespace {

constexpr uint32_t kThreads = 256;
constexpr uint32_t kTM = 128;      // rows per workgroup
constexpr uint32_t kRow = 144;     // LDS bytes per 128-byte row: +16 spreads the banks

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
constexpr size_t stage_bytes() { return (kTM + BN) * kRow; }

template <int BN>
__global__ __launch_bounds__(256) void gemm_i2s_kernel(GemvJobs jobs, Q8Dev q, size_t tokens, int32_t* raw) {
  extern __shared__ __align__(16) uint8_t lds[];
  constexpr int NT = BN / 64;                 // 32-token tiles per wave
  constexpr int ACH = BN * 8 / kThreads;      // 16-byte activation chunks per thread per block
  const GemvJob& J = jobs.j[job_index(jobs, blockIdx.x)];
  const uint32_t row0 = (blockIdx.x - J.wg_begin) * kTM;
  const uint32_t tok0 = blockIdx.y * BN;
  const uint32_t nb = J.nb;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t wm = wave & 1u, wn = wave >> 1;
  const uint32_t g = lane >> 5;
  const size_t T = tokens;

  // staging roles: half a block's 32 packed bytes of one row; ACH 16-byte
  // chunks of the activation tile
  const uint32_t sr = tid >> 1, sh = tid & 1u;
  const uint8_t* wrow = J.w + static_cast<size_t>(min(row0 + sr, J.rows - 1u)) * J.stride + 16u * sh;
  const int8_t* arow[ACH];
#pragma unroll
  for (int c = 0; c < ACH; c++) {
    const uint32_t chunk = tid + static_cast<uint32_t>(c) * kThreads;
    const size_t tok = min(static_cast<size_t>(tok0 + (chunk >> 3)), T - 1);
    arow[c] = q.quants + tok * q.qstride + (chunk & 7u) * 16u;
  }

  struct Regs {
    u32x4 w;
    u32x4 a[ACH];
  };
  auto load = [&](Regs& r, uint32_t b) {
    r.w = load16(wrow + static_cast<size_t>(b) * 32u);
#pragma unroll
    for (int c = 0; c < ACH; c++)
      r.a[c] = load16(reinterpret_cast<const uint8_t*>(arow[c] + static_cast<size_t>(b) * 128u));
  };
  // packed byte j (0..31) of a block holds weights j, j+32, j+64, j+96 at
  // shifts 6, 4, 2, 0 (quantize/src/i2_s.rs:12-21)
  auto store = [&](const Regs& r, uint32_t stage) {
    uint8_t* wt = lds + stage * stage_bytes<BN>() + sr * kRow + 16u * sh;
#pragma unroll
    for (uint32_t k = 0; k < 4u; k++) {
      const uint32_t shift = 6u - 2u * k;
      const u32x4 v{codes_minus_one((r.w.x >> shift) & 0x03030303u), codes_minus_one((r.w.y >> shift) & 0x03030303u),
                    codes_minus_one((r.w.z >> shift) & 0x03030303u), codes_minus_one((r.w.w >> shift) & 0x03030303u)};
      *reinterpret_cast<u32x4*>(wt + 32u * k) = v;
    }
    uint8_t* at = lds + stage * stage_bytes<BN>() + kTM * kRow;
#pragma unroll
    for (int c = 0; c < ACH; c++) {
      const uint32_t chunk = tid + static_cast<uint32_t>(c) * kThreads;
      *reinterpret_cast<u32x4*>(at + (chunk >> 3) * kRow + (chunk & 7u) * 16u) = r.a[c];
    }
  };

  v16i acc[2][NT];
#pragma unroll
  for (int rt = 0; rt < 2; rt++)
#pragma unroll
    for (int t = 0; t < NT; t++) acc[rt][t] = v16i{};
  uint32_t arow_l[2], brow_l[NT];
#pragma unroll
  for (int rt = 0; rt < 2; rt++) arow_l[rt] = 64u * wm + 32u * static_cast<uint32_t>(rt) + (lane & 31u);
#pragma unroll
  for (int t = 0; t < NT; t++) brow_l[t] = static_cast<uint32_t>(BN / 2) * wn + 32u * static_cast<uint32_t>(t) + (lane & 31u);

  auto compute = [&](uint32_t stage) {
    const int8_t* wt = reinterpret_cast<const int8_t*>(lds + stage * stage_bytes<BN>());
    const int8_t* at = wt + kTM * kRow;
#pragma unroll
    for (uint32_t kk = 0; kk < 4u; kk++) {
      const uint32_t ko = 32u * kk + 16u * g;
      v4i A[2], B[NT];
#pragma unroll
      for (int rt = 0; rt < 2; rt++) A[rt] = *reinterpret_cast<const v4i*>(wt + arow_l[rt] * kRow + ko);
#pragma unroll
      for (int t = 0; t < NT; t++) B[t] = *reinterpret_cast<const v4i*>(at + brow_l[t] * kRow + ko);
#pragma unroll
      for (int rt = 0; rt < 2; rt++)
#pragma unroll
        for (int t = 0; t < NT; t++) acc[rt][t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[rt], B[t], acc[rt][t], 0, 0, 0);
    }
  };

  // block b's MFMAs run from stage b&1 while block b+1 (in the register set
  // loaded two steps ago) goes to the other stage; the set it frees takes
  // block b+3
  Regs r0, r1;
  if (nb) {
    load(r0, 0);
    if (nb > 1u) load(r1, 1u);
    store(r0, 0);
    __syncthreads();
    if (nb > 2u) load(r0, 2u);
  }
  for (uint32_t b = 0; b < nb; b += 2u) {
    compute(0);
    if (b + 1u < nb) store(r1, 1);
    __syncthreads();
    if (b + 3u < nb) load(r1, b + 3u);
    if (b + 1u < nb) {
      compute(1);
      if (b + 2u < nb) store(r0, 0);
      __syncthreads();
      if (b + 4u < nb) load(r0, b + 4u);
    }
  }

  // ternary.rs:53-57: (dot as f32) / s * scale, 0 without an activation
  // (D layout: lane n + 32*((m/4)%2), register 4*(m/8) + m%4)
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const size_t tok = tok0 + brow_l[t];
    if (tok >= T) continue;
    const float s = q.n_blocks ? q.scales[tok * q.bstride] : 0.0f;
#pragma unroll
    for (int rt = 0; rt < 2; rt++)
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const uint32_t m = 64u * wm + 32u * static_cast<uint32_t>(rt) + 8u * static_cast<uint32_t>(i >> 2) + 4u * g +
                           static_cast<uint32_t>(i & 3);
        const uint32_t row = row0 + m;
        if (row >= J.rows) continue;
        const size_t idx = static_cast<size_t>(row) * T + tok;
        if (idx >= J.out_len) continue;
        const int32_t dot = acc[rt][t][i];
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
    wgs += (jobs.j[i].rows + kTM - 1u) / kTM;
  }
  if (wgs == 0) return hipSuccess;
  const uint32_t tiles = static_cast<uint32_t>((tokens + BN - 1) / BN);
  hipLaunchKernelGGL((gemm_i2s_kernel<BN>), dim3(wgs, tiles), dim3(kThreads), 2u * stage_bytes<BN>(), s, jobs, q,
                     tokens, raw);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm_i2s(const GemvJobs& jobs, const Q8Dev& q, size_t tokens, int32_t* raw, hipStream_t s) {
  if (tokens == 0 || jobs.n == 0) return hipSuccess;
  // 64 tokens a workgroup up to 1023 tokens (512: 26.4 against 31.8 us at
  // 128), 128 from 1024 (2048: 77-79 against 88 us at 64; 256 is slower at
  // every size: one workgroup per CU); tuning().gemm_bn forces it
  const int bn = tuning().gemm_bn ? tuning().gemm_bn : tokens >= 1024 ? 128 : 64;
  return bn == 256 ? launch_bn<256>(jobs, q, tokens, raw, s)
       : bn == 128 ? launch_bn<128>(jobs, q, tokens, raw, s)
                   : launch_bn<64>(jobs, q, tokens, raw, s);
}

}  // namespace rh
