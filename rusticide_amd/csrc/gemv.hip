// gemv.hip -- decode GEMV on gfx950: Q4_K / Q6_K / I2_S weights in their
// native GGUF block layouts against device-quantized activations.
//
// Work split: a workgroup of 256 lanes owns R consecutive rows of one matrix
// (several matrices share a launch, as matmul_batch shares one parallel
// region: crates/rusticide-kernels/src/matmul.rs:229-248). The activation of
// every token in the launch is staged in LDS once per workgroup.
//
// k-quants: a team of 4 lanes decodes one 256-weight super-block in
// registers from three 16-byte loads per lane, forms the block's integer sums
// with v_dot4_i32_i8 and DPP quad reductions (exact, so their order is free),
// and writes the block's float term. The terms of a row are then added in
// block order from -0.0 by one lane, which is the order of the CPU path
// (portable/int_dot/rows.rs:9-12,59): the result is bit-identical.
//
// I2_S: a team of 8 lanes walks a row 16 bytes at a time; the i32 dot is
// order-free (wrapping) and is scaled once per row, as portable/ternary.rs:48-58.
#include "rh_device.h"
#include "rh_internal.h"
#include "rh_math.h"

namespace rh {

namespace {

constexpr uint32_t kThreads = 256;

__device__ __forceinline__ uint32_t find_job(const GemvJobs& jobs) {
  uint32_t j = 0;
#pragma unroll
  for (uint32_t i = 1; i < static_cast<uint32_t>(kMaxJobs); i++)
    if (i < jobs.n && blockIdx.x >= jobs.j[i].wg_begin) j = i;
  return j;
}

// Copies `bytes` (a multiple of 16) of each token's quants into LDS.
template <int T>
__device__ __forceinline__ void stage_quants(int8_t* act, uint32_t bytes, const Q8Dev& q, size_t t0) {
  for (uint32_t t = 0; t < static_cast<uint32_t>(T); t++) {
    const int8_t* src = q.quants + (t0 + t) * q.qstride;
    for (uint32_t i = threadIdx.x * 16u; i < bytes; i += kThreads * 16u)
      *reinterpret_cast<u32x4*>(act + t * bytes + i) = *reinterpret_cast<const u32x4*>(src + i);
  }
}

// Each 4-lane team decodes up to NI blocks. Their weight loads are issued
// first, before the activation is staged and before the barrier, so every
// resident workgroup has all of its rows in flight from its first cycles and
// the decode of one workgroup overlaps the loads of the others.
// As stage_quants, for the k-quants: 16-byte chunk c of 256-byte block b is
// stored at chunk c ^ (b & 15). The teams of a wave read the same chunk
// offsets of different blocks at once; unswizzled those all land in the same
// few LDS banks (a 256-byte block stride is a whole number of bank rows).
template <int T, uint32_t NT = kThreads>
__device__ __forceinline__ void stage_quants_swizzled(int8_t* act, uint32_t bytes, const Q8Dev& q, size_t t0) {
  for (uint32_t t = 0; t < static_cast<uint32_t>(T); t++) {
    const int8_t* src = q.quants + (t0 + t) * q.qstride;
    for (uint32_t i = threadIdx.x * 16u; i < bytes; i += NT * 16u) {
      const uint32_t b = i >> 8, c = (i >> 4) & 15u;
      *reinterpret_cast<u32x4*>(act + t * bytes + (b << 8) + ((c ^ (b & 15u)) << 4)) =
          *reinterpret_cast<const u32x4*>(src + i);
    }
  }
}

// The address of activation byte k (a multiple of 16) of block b of token t.
__device__ __forceinline__ const int8_t* swz(const int8_t* act_t, uint32_t b, uint32_t k) {
  return act_t + (b << 8) + ((((k >> 4) ^ (b & 15u))) << 4);
}

// Q8Kind::SuperBlock quantization (portable/q8.rs:64-98) of the first nq
// 256-value blocks of T tokens (x[t * width + ...]) straight into the LDS
// tiles the k-quant kernels read: quants swizzled as stage_quants_swizzled
// lays them out, d8[t][b] the block's step, and per token
//   FMT 12: side[t][8b + j]  = the sum of 32-block j's quants;
//   FMT 14: side[t][16b + k] = -32 * the sum of 16-run k's quants.
// A 32-lane half-wave owns one block, 8 values per lane; a round covers K
// blocks per half-wave. The kernels load the first round before their weight
// loads: vector memory returns in issue order, so x loaded after the weights
// could not be quantized until every weight had arrived.
// Each block is reduced with DPP: amax over the magnitudes (q8.rs:12-25; a
// NaN never enters it), then the first value whose magnitude is amax
// (q8.rs:26-32) as the minimum of (index, sign) keys -- every candidate is
// +-amax, so its sign is all the index selects. The arithmetic after that is
// quantize_super_kernel's, so the bits are the same.
template <int K>
struct XRound {
  float f[K][8];
};

struct XGeom {
  const float* x;  // token t0
  size_t width;
  uint32_t nq;     // blocks quantized per token: min(nb, width / 256)
  uint32_t total;  // T * nq
};

template <int T>
__device__ __forceinline__ XGeom x_geom(const float* x, size_t width, uint32_t nb) {
  XGeom g;
  g.x = x;
  g.width = width;
  g.nq = width / 256u < nb ? static_cast<uint32_t>(width / 256u) : nb;
  g.total = static_cast<uint32_t>(T) * g.nq;
  return g;
}

template <int K, uint32_t NT = kThreads>
__device__ __forceinline__ void load_x_round(XRound<K>& xr, const XGeom& g, uint32_t u0) {
  const uint32_t hl = threadIdx.x & 31u, hw = threadIdx.x >> 5;
#pragma unroll
  for (uint32_t k = 0; k < static_cast<uint32_t>(K); k++) {
    const uint32_t u = u0 + hw + k * (NT / 32u);
    if (u >= g.total) {
#pragma unroll
      for (int i = 0; i < 8; i++) xr.f[k][i] = 0.0f;
      continue;
    }
    const uint32_t t = u / g.nq, b = u - t * g.nq;
    const float* v = g.x + t * g.width + static_cast<size_t>(b) * 256u + 8u * hl;
    // dword-aligned 16-byte loads, whatever x's and the width's alignment: no
    // branch for the compiler to join (a join between these loads and the
    // weight loads after them makes it wait for x before issuing the weights)
    const u32x4 lo = load16_a4(reinterpret_cast<const uint8_t*>(v));
    const u32x4 hi = load16_a4(reinterpret_cast<const uint8_t*>(v + 4));
#pragma unroll
    for (int i = 0; i < 4; i++) {
      xr.f[k][i] = __uint_as_float(lo[i]);
      xr.f[k][4 + i] = __uint_as_float(hi[i]);
    }
  }
}

template <int FMT, int K, uint32_t NT = kThreads>
__device__ __forceinline__ void quantize_x_round(const XRound<K>& xr, const XGeom& g, uint32_t u0, uint32_t nb,
                                                 int8_t* act, float* d8, int32_t* side) {
  const uint32_t hl = threadIdx.x & 31u, hw = threadIdx.x >> 5;
  const uint32_t abytes = nb * 256u;
#pragma unroll
  for (uint32_t k = 0; k < static_cast<uint32_t>(K); k++) {
    const uint32_t u = u0 + hw + k * (NT / 32u);
    if (u >= g.total) break;  // uniform over the half-wave
    const uint32_t t = u / g.nq, b = u - t * g.nq;
    const float* f = xr.f[k];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float m = __builtin_fabsf(f[i]);
      amax = m > amax ? m : amax;
    }
    amax = __uint_as_float(half_max_u32(__float_as_uint(amax)));
    uint32_t key = 0xffffffffu;
#pragma unroll
    for (int i = 7; i >= 0; i--)
      if (__builtin_fabsf(f[i]) == amax) key = 2u * (8u * hl + static_cast<uint32_t>(i)) + (__float_as_uint(f[i]) >> 31);
    key = half_min_u32(key);
    const float max = key == 0xffffffffu ? 0.0f : ((key & 1u) ? -amax : amax);
    const float inverse = (max == 0.0f) ? 0.0f : __fdiv_rn(-127.0f, max);
    const float step = (max == 0.0f) ? 0.0f : __fdiv_rn(1.0f, inverse);
    uint32_t packed[2] = {0u, 0u};
    int32_t s = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float prod = f[i] * inverse;
      const int32_t qv = round_to_i8(prod);
      s += qv;
      packed[i >> 2] |= (static_cast<uint32_t>(qv) & 0xffu) << (8 * (i & 3));
    }
    // byte 8*hl of block b: chunk hl/2, stored at chunk (hl/2) ^ (b & 15)
    uint32_t* dst = reinterpret_cast<uint32_t*>(act + t * abytes + (b << 8) + (((hl >> 1) ^ (b & 15u)) << 4) +
                                                8u * (hl & 1u));
    dst[0] = packed[0];
    dst[1] = packed[1];
    const int32_t s16 = s + static_cast<int32_t>(dpp<0xB1>(static_cast<uint32_t>(s)));
    const int32_t s32 = s16 + static_cast<int32_t>(dpp<0x4E>(static_cast<uint32_t>(s16)));
    if (FMT == 12) {
      if ((hl & 3u) == 0) side[t * nb * 8u + b * 8u + (hl >> 2)] = s32;
    } else {
      if ((hl & 1u) == 0) side[t * nb * 16u + b * 16u + (hl >> 1)] = -32 * s16;
    }
    if (hl == 0) d8[t * nb + b] = step;
  }
}

// The residual add and RMSNorm on a one-token preload that holds the whole
// row (NormIn): each lane forms v = h + delta for its values and their
// squares in LDS, one lane sums the squares in element order, then every
// lane replaces its values with (v / rms) * weight -- the arithmetic of the
// decoder's add_norm kernel, value for value. norm_load issues the delta and
// weight loads with the activation's, before the matrix loads (loads return
// in issue order); norm_apply runs after them.
template <int K>
struct NormRound {
  float d[K][8];
  float w[K][8];
};

template <int K, uint32_t NT = kThreads>
__device__ __forceinline__ void norm_load(NormRound<K>& nr, const XGeom& g, const NormIn& nrm) {
  const uint32_t hl = threadIdx.x & 31u, hw = threadIdx.x >> 5;
#pragma unroll
  for (uint32_t k = 0; k < static_cast<uint32_t>(K); k++) {
    const uint32_t u = hw + k * (NT / 32u);
    const size_t e0 = static_cast<size_t>(u < g.total ? u : 0u) * 256u + 8u * hl;
    const u32x4 w0 = load16(reinterpret_cast<const uint8_t*>(nrm.weight + e0));
    const u32x4 w1 = load16(reinterpret_cast<const uint8_t*>(nrm.weight + e0 + 4));
    // without a delta the weights are read twice and the copy discarded: a
    // branch around these loads would make the compiler wait for them at
    // its join, before the weight loads behind it
    const float* dsrc = nrm.delta ? nrm.delta : nrm.weight;
    const u32x4 d0 = load16(reinterpret_cast<const uint8_t*>(dsrc + e0));
    const u32x4 d1 = load16(reinterpret_cast<const uint8_t*>(dsrc + e0 + 4));
#pragma unroll
    for (int i = 0; i < 4; i++) {
      nr.w[k][i] = __uint_as_float(w0[i]);
      nr.w[k][4 + i] = __uint_as_float(w1[i]);
      nr.d[k][i] = __uint_as_float(d0[i]);
      nr.d[k][4 + i] = __uint_as_float(d1[i]);
    }
  }
}

template <int K, uint32_t NT = kThreads>
__device__ __forceinline__ void norm_apply(XRound<K>& xr, const NormRound<K>& nr, const XGeom& g, const NormIn& nrm,
                                           float* sq, float* s_rms) {
  const uint32_t hl = threadIdx.x & 31u, hw = threadIdx.x >> 5;
#pragma unroll
  for (uint32_t k = 0; k < static_cast<uint32_t>(K); k++) {
    const uint32_t u = hw + k * (NT / 32u);
    if (u >= g.total) continue;
    const uint32_t e0 = u * 256u + 8u * hl;
    float s2[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      float v = xr.f[k][i];
      if (nrm.delta) v += nr.d[k][i];
      xr.f[k][i] = v;
      s2[i] = v * v;
      if (nrm.hidden_out && blockIdx.x == 0) nrm.hidden_out[e0 + i] = v;
    }
    // 8 consecutive values stay inside one 32-value chunk of the layout
    float4* dst = reinterpret_cast<float4*>(sq + wave_sum_index(e0));
    dst[0] = float4{s2[0], s2[1], s2[2], s2[3]};
    dst[1] = float4{s2[4], s2[5], s2[6], s2[7]};
  }
  __syncthreads();
  if (threadIdx.x < 64u) {
    // the squares summed in order from -0.0 (f32 Sum), by wave 0
    const uint32_t n = g.total * 256u;
    const float sum = ordered_sum_wave(sq, n, -0.0f);
    if (threadIdx.x == 0) {
      const float mean = __fdiv_rn(sum, static_cast<float>(n));
      *s_rms = sqrt_rn(mean + nrm.eps);
    }
  }
  __syncthreads();
  const float rms = *s_rms;
#pragma unroll
  for (uint32_t k = 0; k < static_cast<uint32_t>(K); k++) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float xv = __fdiv_rn(xr.f[k][i], rms);
      xr.f[k][i] = xv * nr.w[k][i];
    }
  }
}

// The rounds after the first (which the kernel quantizes from its preload).
template <int FMT, int K, uint32_t NT = kThreads>
__device__ __forceinline__ void quantize_x_rest(const XGeom& g, uint32_t nb, int8_t* act, float* d8,
                                                int32_t* side) {
  for (uint32_t u0 = static_cast<uint32_t>(K) * (NT / 32u); u0 < g.total;
       u0 += static_cast<uint32_t>(K) * (NT / 32u)) {
    XRound<K> xr;
    load_x_round<K, NT>(xr, g, u0);
    quantize_x_round<FMT, K, NT>(xr, g, u0, nb, act, d8, side);
  }
}

// Blocks per team whose weight loads a k-quant kernel issues before its
// activation prologue; the rest go out one per block computed, `ahead`
// blocks in front. A wave whose loads all go out at once stalls on issue
// once its CU's memory queue is full, which holds back the prologue (the
// quantize, and the norm in the norm-fused kernels) and every dot behind it.
template <int NI, bool NORM>
constexpr int issue_ahead() { return NI < 2 ? NI : 2; }

// The rows of a k-quant workgroup. PAIR (a gate/up launch): the workgroup
// takes nh rows of the job's w from row0 on as its rows 0..nh-1, and the
// same rows of w2 as its rows nh..2nh-1.
struct WgRows {
  // The job's first matrix and the byte offset of its second (a pair's up
  // rows), the offset pinned in SGPRs: a per-lane select between J.w and
  // J.w2 otherwise becomes a per-lane load of the pointer itself, whose wait
  // (loads return in issue order) holds every weight load behind the
  // activation loads issued before it. A pointer passed through the pin
  // would lose its global address space (flat loads).
  const uint8_t* w1;
  uint64_t d2;
  uint32_t row0, nrows, nh;
  // row_of's chunk map: row = ((r >> cs) * nwg + w) << cs | (r & mask).
  // Contiguous rows are the case cs = 0, nwg = 1, w = row0, so the map has
  // no branch (a branch between two blocks' loads makes the compiler wait
  // for the first block's loads at the join).
  uint32_t cs, nwg, w, mask;
};

template <bool PAIR>
__device__ __forceinline__ WgRows wg_rows(const GemvJob& J, uint32_t R) {
  const uint32_t per = PAIR ? R / 2u : R;
  const uint32_t w = blockIdx.x - J.wg_begin;
  uint64_t d2 = PAIR ? reinterpret_cast<uintptr_t>(J.w2) - reinterpret_cast<uintptr_t>(J.w) : 0u;
  asm volatile("" : "+s"(d2));
  if (!PAIR && J.il) {
    const uint32_t cs = J.il - 1u;
    return WgRows{J.w, d2, 0u, per, per, cs, J.rows / per, w, (1u << cs) - 1u};
  }
  const uint32_t row0 = w * per;
  const uint32_t nh = min(per, J.rows - row0);
  return WgRows{J.w, d2, row0, PAIR ? 2u * nh : nh, nh, 0u, 1u, row0, 0u};
}

// The matrix row of workgroup row r (not of a pair's second half).
__device__ __forceinline__ uint32_t row_of(const WgRows& g, uint32_t r) {
  return ((__umul24(r >> g.cs, g.nwg) + g.w) << g.cs) | (r & g.mask);
}

// The group of 16 blocks (the unit layout, rh_device.h) holding block fb of
// workgroup row r, for the fixed-column walk: a wave's step reads one group,
// its team tw at position tw.
template <bool PAIR>
__device__ __forceinline__ const uint8_t* unit_at(const WgRows& g, uint32_t r, uint32_t fb, uint32_t nb,
                                                  uint32_t ubytes) {
  const bool second = PAIR && r >= g.nh;
  const uint8_t* m = g.w1 + (second ? g.d2 : 0u);
  const uint32_t row = PAIR ? g.row0 + (second ? r - g.nh : r) : row_of(g, r);
  return m + ((row * nb + fb) >> 4) * ubytes;
}

// nb terms t[0], t[S], t[2S], ... summed in order from -0.0, the LDS reads
// of each run of 8 (then 4) issued together: one read latency a run, not
// one a term.
template <int S>
__device__ __forceinline__ float terms_sum(const float* t, uint32_t nb) {
  float s = -0.0f;
  uint32_t b = 0;
  for (; b + 8u <= nb; b += 8u) {
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; k++) v[k] = t[(b + k) * S];
#pragma unroll
    for (int k = 0; k < 8; k++) s += v[k];
  }
  if (b + 4u <= nb) {
    float v[4];
#pragma unroll
    for (int k = 0; k < 4; k++) v[k] = t[(b + k) * S];
#pragma unroll
    for (int k = 0; k < 4; k++) s += v[k];
    b += 4u;
  }
  for (; b < nb; b++) s += t[b * S];
  return s;
}

// Each row's block terms summed in block order from -0.0
// (portable/int_dot/rows.rs:9-12,59) and written; PAIR writes
// silu(gate) * up with silu_mul's expressions (portable/elementwise.rs:6-9).
// PICK (one token, a norm-fused launch): with `pick` set, the workgroup also
// writes the greedy pick's partial over its rows to pick[blockIdx.x].
template <int T, bool PAIR, uint32_t NT = kThreads, bool PICK = false>
__device__ __forceinline__ void write_rows(const GemvJob& J, const WgRows& g, const float* terms, uint32_t nb,
                                           uint32_t nbmax, size_t tokens, size_t t0, PickPart* pick = nullptr) {
  if constexpr (PAIR) {
    static_assert(T == 1, "a gate/up pair serves one token");
    for (uint32_t r = threadIdx.x; r < g.nh; r += NT) {
      const float gs = terms_sum<1>(terms + __umul24(r, nbmax), nb);
      const float us = terms_sum<1>(terms + __umul24(r + g.nh, nbmax), nb);
      const float den = 1.0f + expf_ref(-gs);
      const float sg = __fdiv_rn(gs, den);
      const size_t idx = static_cast<size_t>(g.row0 + r) * tokens + t0;
      if (idx < J.out_len) J.out[idx] = sg * us;
    }
  } else {
    const bool want = PICK && pick != nullptr;  // uniform
    uint64_t best = 0;
    uint32_t fin = 0;
    for (uint32_t i = threadIdx.x; i < g.nrows * T; i += NT) {
      const uint32_t r = i / T, t = i - r * T;
      const float s = terms_sum<T>(terms + __umul24(r, nbmax) * T + t, nb);
      const uint32_t row = row_of(g, r);
      const size_t idx = static_cast<size_t>(row) * tokens + t0 + t;
      if (idx < J.out_len) {
        J.out[idx] = s;
        if (want) {
          fin |= __builtin_isfinite(s) ? 1u : 0u;
          const uint64_t c = pick_code(total_key(s != s ? -INFINITY : s), row);
          best = c > best ? c : best;
        }
      }
    }
    if constexpr (PICK) {
      if (!want) return;
      __shared__ uint64_t s_best[NT / 64u];
      __shared__ uint32_t s_fin[NT / 64u];
      best = wave_max_code(best);
      fin = __ballot(fin != 0u) ? 1u : 0u;
      if ((threadIdx.x & 63u) == 0) {
        s_best[threadIdx.x >> 6] = best;
        s_fin[threadIdx.x >> 6] = fin;
      }
      __syncthreads();
      if (threadIdx.x == 0) {
        PickPart part{0, 0, 0};
        for (uint32_t w = 0; w < NT / 64u; w++) {
          part.code = s_best[w] > part.code ? s_best[w] : part.code;
          part.fin |= s_fin[w];
        }
        pick[blockIdx.x] = part;
      }
    }
  }
}

// Where a team finds its blocks. A workgroup's teams take team blocks
// g = team + i * NT/4, i = 0..NI-1, of its rows x nb blocks in row-major
// order. The general walk divides each g into (row g / nb, block g % nb) and
// finds that block's group and position in the unit layout (rh_device.h);
// when a wave's 16 teams take the 16 blocks of one group, its loads read
// consecutive bytes.
// FIX (nb a power of two up to NT/4: rows of 256, 512, ... values): g % nb
// is the same for every i, so the team keeps one
// block column fb, its row advances by step = NT/4/nb an iteration, and the
// activation a team reads is the same for all of its blocks and leaves the
// loop. A wave's 16 teams take the 16 blocks of one group, each at its own
// position, and the group's address advances by a constant stride (row_of is
// affine in i: step is a whole number of interleaved chunks, and the
// launcher checks that every wave's rows start a group).
template <bool PAIR, uint32_t NT, bool FIX>
struct BlockWalk {
  const GemvJob& J;
  const WgRows& wr;
  uint32_t nb, total, team, bbytes;
  float inv_nb;
  uint32_t r0, fb, step, delta;  // FIX
  const uint8_t* p0;             // FIX: the team's first block (block 0 of row 0 for a spare team)

  __device__ __forceinline__ BlockWalk(const GemvJob& j, const WgRows& w, uint32_t block_bytes)
      : J(j), wr(w), nb(j.nb), total(w.nrows * j.nb), team(threadIdx.x >> 2), bbytes(block_bytes) {
    inv_nb = nb ? 1.0f / static_cast<float>(nb) : 0.0f;
    r0 = fb = step = delta = 0u;
    p0 = nullptr;
    if constexpr (FIX) {
      const uint32_t sh = static_cast<uint32_t>(__builtin_ctz(nb));
      r0 = team >> sh;
      fb = team & (nb - 1u);
      step = (NT / 4u) >> sh;
      // matrix rows an iteration, times the unit layout's bytes a row
      delta = (((step >> wr.cs) * wr.nwg) << wr.cs) * nb * bbytes;
      const bool in = r0 < wr.nrows;
      p0 = unit_at<PAIR>(wr, in ? r0 : 0u, in ? fb : 0u, nb, 16u * bbytes);
    }
  }
  // whether team block i lies in the workgroup's rows (uniform over a team)
  __device__ __forceinline__ bool live(int i) const {
    if constexpr (FIX) return r0 + static_cast<uint32_t>(i) * step < wr.nrows;
    return team + static_cast<uint32_t>(i) * (NT / 4u) < total;
  }
  // the workgroup row and block of team block i
  __device__ __forceinline__ void rb(int i, uint32_t& r, uint32_t& b) const {
    if constexpr (FIX) {
      r = r0 + static_cast<uint32_t>(i) * step;
      b = fb;
    } else {
      const uint32_t g = team + static_cast<uint32_t>(i) * (NT / 4u);
      r = static_cast<uint32_t>((static_cast<float>(g) + 0.5f) * inv_nb);
      b = g - __umul24(r, nb);
    }
  }
  // the group of team block i and the block's position tw in it; a spare
  // team re-reads a block of its own
  __device__ __forceinline__ const uint8_t* addr(int i, uint32_t& tw) const {
    if constexpr (FIX) {
      tw = team & 15u;
      const uint32_t r = r0 + static_cast<uint32_t>(i) * step;
      if constexpr (PAIR) return r < wr.nrows ? unit_at<true>(wr, r, fb, nb, 16u * bbytes) : p0;
      return r < wr.nrows ? p0 + static_cast<uint32_t>(i) * delta : p0;
    } else {
      // g = r*nb + b with g < 8*128: a float reciprocal divides exactly here
      const uint32_t g = team + static_cast<uint32_t>(i) * (NT / 4u);
      const uint32_t gg = g < total ? g : 0u;
      const uint32_t r = static_cast<uint32_t>((static_cast<float>(gg) + 0.5f) * inv_nb), b = gg - __umul24(r, nb);
      const bool second = PAIR && r >= wr.nh;
      const uint8_t* m = wr.w1 + (second ? wr.d2 : 0u);
      const uint32_t row = PAIR ? wr.row0 + (second ? r - wr.nh : r) : row_of(wr, r);
      const uint32_t e = row * J.ub + b;  // the matrix's unit blocks stay below 2^32
      tw = e & 15u;
      return m + (e >> 4) * (16u * bbytes);
    }
  }
};

// One 4-lane team's share of a k-quant block: decoded once per block (the
// scales and the lane's 16 bytes of each run), then against each token's
// activation. The term is valid in lane p == 0 of the team after the quad
// sums, which every lane runs.

// Q4_K: lane p takes sub-blocks j0, j0+1, j0+4, j0+5 (j0 = 2(p >> 1)),
// bytes 16(p & 1).. of each (quantize/src/q4_k.rs:17-25, ggml
// get_scale_min_k4 for the 6-bit scales and mins).
struct Q4Dec {
  int32_t sc[4], m[4];
  float d, dmin;
  uint32_t lo0[4], hi0[4], lo1[4], hi1[4];
};

__device__ __forceinline__ Q4Dec q4k_decode(const u32x4& h, const u32x4& c0, const u32x4& c1, uint32_t j0) {
  Q4Dec q;
  q.sc[0] = static_cast<int32_t>(bfe(h.y, 8u * j0, 6));
  q.sc[1] = static_cast<int32_t>(bfe(h.y, 8u * j0 + 8u, 6));
  q.sc[2] = static_cast<int32_t>(bfe(h.w, 8u * j0, 4) | (bfe(h.y, 8u * j0 + 6u, 2) << 4));
  q.sc[3] = static_cast<int32_t>(bfe(h.w, 8u * j0 + 8u, 4) | (bfe(h.y, 8u * j0 + 14u, 2) << 4));
  q.m[0] = static_cast<int32_t>(bfe(h.z, 8u * j0, 6));
  q.m[1] = static_cast<int32_t>(bfe(h.z, 8u * j0 + 8u, 6));
  q.m[2] = static_cast<int32_t>(bfe(h.w, 8u * j0 + 4u, 4) | (bfe(h.z, 8u * j0 + 6u, 2) << 4));
  q.m[3] = static_cast<int32_t>(bfe(h.w, 8u * j0 + 12u, 4) | (bfe(h.z, 8u * j0 + 14u, 2) << 4));
  q.d = f16_lo(h.x);
  q.dmin = f16_hi(h.x);
#pragma unroll
  for (int k = 0; k < 4; k++) {
    q.lo0[k] = c0[k] & 0x0F0F0F0Fu;
    q.hi0[k] = (c0[k] >> 4) & 0x0F0F0F0Fu;
    q.lo1[k] = c1[k] & 0x0F0F0F0Fu;
    q.hi1[k] = (c1[k] >> 4) & 0x0F0F0F0Fu;
  }
  return q;
}

// a: the activation quants of the lane's four runs; s: their 32-block sums
// (S[0], S[1], S[4], S[5] of the block, read by the min lanes); dd8: d8.
__device__ __forceinline__ float q4k_term(const Q4Dec& q, const u32x4& a0, const u32x4& a1, const u32x4& a2,
                                          const u32x4& a3, const int32_t (&s)[4], float dd8, bool min_lane) {
  int32_t D0 = 0, D1 = 0, D2 = 0, D3 = 0;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    D0 = dot4(q.lo0[k], a0[k], D0);
    D1 = dot4(q.hi0[k], a1[k], D1);
    D2 = dot4(q.lo1[k], a2[k], D2);
    D3 = dot4(q.hi1[k], a3[k], D3);
  }
  // 24-bit multiplies are exact here: |D| < 2^17, sums of 32 quants < 2^12,
  // scales and mins below 64
  int32_t isum = __mul24(q.sc[0], D0) + __mul24(q.sc[1], D1) + __mul24(q.sc[2], D2) + __mul24(q.sc[3], D3);
  int32_t msum =
      min_lane ? (__mul24(q.m[0], s[0]) + __mul24(q.m[1], s[1]) + __mul24(q.m[2], s[2]) + __mul24(q.m[3], s[3])) : 0;
  isum = quad_sum(isum);
  msum = quad_sum(msum);
  // int_dot.rs:169: d8 * d.mul_add(isum, -(dmin * msum))
  const float neg = -(q.dmin * static_cast<float>(msum));
  return dd8 * __builtin_fmaf(q.d, static_cast<float>(isum), neg);
}

// Q6_K: lane p (h = p >> 1, gq = p & 1) takes runs of ql[64h+16gq..],
// ql[64h+32+16gq..] and qh[32h+16gq..] (q6_k.rs:13-43), four 16-groups of
// half h.
struct Q6Dec {
  int32_t sc[4];
  float d;
  uint32_t q0[4], q1[4], q2[4], q3[4];
};

__device__ __forceinline__ Q6Dec q6k_decode(const u32x4& a, const u32x4& bq, const u32x4& c, uint2 S, uint32_t D,
                                            uint32_t gq) {
  Q6Dec q;
  // scale of run r, 16-group gq: scales[8h + 2r + gq] (int_dot.rs:199)
  q.sc[0] = __builtin_amdgcn_sbfe(static_cast<int32_t>(S.x), 8u * gq, 8);
  q.sc[1] = __builtin_amdgcn_sbfe(static_cast<int32_t>(S.x), 8u * gq + 16u, 8);
  q.sc[2] = __builtin_amdgcn_sbfe(static_cast<int32_t>(S.y), 8u * gq, 8);
  q.sc[3] = __builtin_amdgcn_sbfe(static_cast<int32_t>(S.y), 8u * gq + 16u, 8);
  q.d = f16_lo(D);  // bytes 208..209
#pragma unroll
  for (int k = 0; k < 4; k++) {
    q.q0[k] = (a[k] & 0x0F0F0F0Fu) | ((c[k] << 4) & 0x30303030u);
    q.q1[k] = (bq[k] & 0x0F0F0F0Fu) | ((c[k] << 2) & 0x30303030u);
    q.q2[k] = ((a[k] >> 4) & 0x0F0F0F0Fu) | (c[k] & 0x30303030u);
    q.q3[k] = ((bq[k] >> 4) & 0x0F0F0F0Fu) | ((c[k] >> 2) & 0x30303030u);
  }
  return q;
}

// a: the activation quants of the lane's four runs; bias: -32 x their
// 16-run quant sums; dd8: d8.
__device__ __forceinline__ float q6k_term(const Q6Dec& q, const u32x4& a0, const u32x4& a1, const u32x4& a2,
                                          const u32x4& a3, const int32_t (&bias)[4], float dd8) {
  int32_t D0 = bias[0], D1 = bias[1], D2 = bias[2], D3 = bias[3];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    D0 = dot4(q.q0[k], a0[k], D0);
    D1 = dot4(q.q1[k], a1[k], D1);
    D2 = dot4(q.q2[k], a2[k], D2);
    D3 = dot4(q.q3[k], a3[k], D3);
  }
  // |D| < 2^20 and |scale| <= 128: the 24-bit multiplies are exact
  const int32_t isum =
      quad_sum(__mul24(q.sc[0], D0) + __mul24(q.sc[1], D1) + __mul24(q.sc[2], D2) + __mul24(q.sc[3], D3));
  // int_dot.rs:203: read_f16_le(block, 208) * span.scales[0] * lossy(sum)
  const float dd = q.d * dd8;
  return dd * static_cast<float>(isum);
}

// Q4_K x Q8_K --------------------------------------------------------------
// LDS: act [T][nbmax*256] i8 | d8 [T][nbmax] f32 | sums [T][nbmax*8] i32 |
//      terms [R][nbmax][T] f32
// FQ: 0 reads the activation q holds; 1 or 4 quantizes x in the kernel,
// preloading FQ blocks per half-wave before the weights.
// NORM (T = 1, the whole row in the preload): x is the hidden state and the
// kernel applies the NormIn residual add and RMSNorm before quantizing.
// FIX: see BlockWalk (one token).
template <int T, int NI, int FQ, bool NORM, bool PAIR, uint32_t NT, bool FIX>
__device__ __forceinline__ void q4k_body(const GemvJob& J, const Q8Dev& q, const float* __restrict__ x, size_t width,
                                         uint32_t R, uint32_t nbmax, size_t tokens, size_t t0, const NormIn& nrm,
                                         uint8_t* lds) {
  const uint32_t abytes = nbmax * 256u;
  int8_t* act = reinterpret_cast<int8_t*>(lds);
  float* d8 = reinterpret_cast<float*>(lds + T * abytes);
  int32_t* sums = reinterpret_cast<int32_t*>(d8 + T * nbmax);
  float* terms = reinterpret_cast<float*>(sums + T * nbmax * 8u);

  const WgRows wr = wg_rows<PAIR>(J, R);
  const BlockWalk<PAIR, NT, FIX> walk(J, wr, 144u);
  const uint32_t p = threadIdx.x & 3u;

  const XGeom xg = x_geom<T>(FQ ? x + t0 * width : nullptr, width, nbmax);
  XRound<FQ ? FQ : 1> xr;
  if (FQ) load_x_round<FQ ? FQ : 1, NT>(xr, xg, 0u);
  NormRound<FQ ? FQ : 1> nr;
  if constexpr (NORM) norm_load<FQ ? FQ : 1, NT>(nr, xg, nrm);
  // the activation's loads go out before any weight load (loads return in
  // issue order: the prologue waits only for these)
  __builtin_amdgcn_sched_barrier(0);
  u32x4 hd[NI], c0[NI], c1[NI];
  // the unit layout (rh_device.h): the block's header at 16 tw, the lane's
  // pieces of qs[0..64) and qs[64..128) at 256 / 1280 + 64 tw + 16p; the
  // quants are read nontemporal (once per launch)
  auto issue = [&](int i) {
    uint32_t tw;
    const uint8_t* grp = walk.addr(i, tw);
    hd[i] = load16(grp + 16u * tw);
    c0[i] = load16_nt(grp + 256u + 64u * tw + 16u * p);
    c1[i] = load16_nt(grp + 1280u + 64u * tw + 16u * p);
  };
  constexpr int ahead = issue_ahead<NI, NORM>();
#pragma unroll
  for (int i = 0; i < ahead; i++) issue(i);

  if constexpr (NORM) norm_apply<FQ ? FQ : 1, NT>(xr, nr, xg, nrm, reinterpret_cast<float*>(lds + nrm.lds_offset),
                                    reinterpret_cast<float*>(lds + nrm.lds_offset) + wave_sum_floats(xg.total * 256u));
  if (FQ) {
    quantize_x_round<12, FQ ? FQ : 1, NT>(xr, xg, 0u, nbmax, act, d8, sums);
    quantize_x_rest<12, FQ ? FQ : 1, NT>(xg, nbmax, act, d8, sums);
  } else {
    stage_quants_swizzled<T, NT>(act, abytes, q, t0);
    for (uint32_t i = threadIdx.x; i < T * nbmax * 8u; i += NT) {
      const uint32_t t = i / (nbmax * 8u), k = i - t * nbmax * 8u;
      const size_t src = (t0 + t) * q.bstride + k;
      sums[i] = q.sums[src];
      if ((k & 7u) == 0) d8[t * nbmax + k / 8u] = q.scales[src];
    }
  }
  __syncthreads();

  const uint32_t j0 = 2u * (p >> 1), e0 = 16u * (p & 1u);
  const uint32_t k0 = e0 + 32u * j0;
  const bool min_lane = (p & 1u) == 0;
  // FIX: the team's activation quants, 32-block sums and d8, read once
  u32x4 fa[4] = {};
  int32_t fs[4] = {};
  float fd8 = 0.0f;
  if constexpr (FIX) {
    fa[0] = *reinterpret_cast<const u32x4*>(swz(act, walk.fb, k0));
    fa[1] = *reinterpret_cast<const u32x4*>(swz(act, walk.fb, k0 + 32u));
    fa[2] = *reinterpret_cast<const u32x4*>(swz(act, walk.fb, k0 + 128u));
    fa[3] = *reinterpret_cast<const u32x4*>(swz(act, walk.fb, k0 + 160u));
    const int32_t* S = sums + walk.fb * 8u + j0;
    fs[0] = S[0];
    fs[1] = S[1];
    fs[2] = S[4];
    fs[3] = S[5];
    fd8 = d8[walk.fb];
  }
#pragma unroll
  for (int it = 0; it < NI; it++) {
    if (it + ahead < NI) issue(it + ahead);
    if (!walk.live(it)) break;  // uniform over the team
    uint32_t r, b;
    walk.rb(it, r, b);
    const Q4Dec q = q4k_decode(hd[it], c0[it], c1[it], j0);
#pragma unroll
    for (int t = 0; t < T; t++) {
      u32x4 a0 = fa[0], a1 = fa[1], a2 = fa[2], a3 = fa[3];
      int32_t sv[4] = {fs[0], fs[1], fs[2], fs[3]};
      float dd8 = fd8;
      if constexpr (!FIX) {
        const int8_t* at = act + t * abytes;
        a0 = *reinterpret_cast<const u32x4*>(swz(at, b, k0));
        a1 = *reinterpret_cast<const u32x4*>(swz(at, b, k0 + 32u));
        a2 = *reinterpret_cast<const u32x4*>(swz(at, b, k0 + 128u));
        a3 = *reinterpret_cast<const u32x4*>(swz(at, b, k0 + 160u));
        const int32_t* S = sums + t * nbmax * 8u + b * 8u + j0;
        sv[0] = S[0];
        sv[1] = S[1];
        sv[2] = S[4];
        sv[3] = S[5];
        dd8 = d8[t * nbmax + b];
      }
      const float term = q4k_term(q, a0, a1, a2, a3, sv, dd8, min_lane);
      if (p == 0) terms[(__umul24(r, nbmax) + b) * T + t] = term;
    }
  }
  __syncthreads();
  write_rows<T, PAIR, NT, NORM && !PAIR && T == 1>(J, wr, terms, J.nb, nbmax, tokens, t0, nrm.pick);
}

// FIX: every job's nb is a power of two up to NT/4 (the launch checks). It is
// a kernel of its own rather than a branch in one: at the join of two walks
// the compiler merges their pending loads and then waits for the activation
// before issuing the first weights.
template <int T, int NI, int FQ, bool NORM, bool PAIR = false, uint32_t NT = kThreads, bool FIX = false>
__global__ __launch_bounds__(NT) void gemv_q4k_kernel(GemvJobs jobs, Q8Dev q, const float* __restrict__ x,
                                                       size_t width, uint32_t R, uint32_t nbmax, size_t tokens,
                                                       size_t t0, NormIn nrm) {
  extern __shared__ __align__(16) uint8_t lds[];
  static_assert(!FIX || T == 1, "fixed columns: one token");
  q4k_body<T, NI, FQ, NORM, PAIR, NT, FIX>(jobs.j[find_job(jobs)], q, x, width, R, nbmax, tokens, t0, nrm, lds);
}

// The same kernel with the activation's scalars first: the build preloads
// leading scalar arguments into SGPRs (-amdgpu-kernarg-preload-count), so the
// activation's first loads need no kernel-argument load (kq_preloads).
template <int T, int NI, int FQ, bool NORM, bool PAIR = false, uint32_t NT = kThreads, bool FIX = false>
__global__ __launch_bounds__(NT) void gemv_q4k_kernel_pl(const float* __restrict__ x, size_t width, uint32_t R,
                                                          uint32_t nbmax, size_t tokens, size_t t0, GemvJobs jobs,
                                                          Q8Dev q, NormIn nrm) {
  extern __shared__ __align__(16) uint8_t lds[];
  q4k_body<T, NI, FQ, NORM, PAIR, NT, FIX>(jobs.j[find_job(jobs)], q, x, width, R, nbmax, tokens, t0, nrm, lds);
}

// Q6_K x Q8_K --------------------------------------------------------------
// LDS: act [T][nbmax*256] i8 | d8 [T][nbmax] f32 | bias [T][nbmax*16] i32
//      (-32 * the activation sum of each 16-run) | terms [R][nbmax][T] f32
// FQ: 0 reads the activation q holds; 1 or 4 quantizes x in the kernel,
// preloading FQ blocks per half-wave before the weights.
template <int T, int NI, int FQ, bool NORM, bool PAIR, uint32_t NT, bool FIX>
__device__ __forceinline__ void q6k_body(const GemvJob& J, const Q8Dev& q, const float* __restrict__ x, size_t width,
                                         uint32_t R, uint32_t nbmax, size_t tokens, size_t t0, const NormIn& nrm,
                                         uint8_t* lds) {
  const uint32_t abytes = nbmax * 256u;
  int8_t* act = reinterpret_cast<int8_t*>(lds);
  float* d8 = reinterpret_cast<float*>(lds + T * abytes);
  int32_t* bias = reinterpret_cast<int32_t*>(d8 + T * nbmax);
  float* terms = reinterpret_cast<float*>(bias + T * nbmax * 16u);

  const WgRows wr = wg_rows<PAIR>(J, R);
  const BlockWalk<PAIR, NT, FIX> walk(J, wr, 210u);
  const uint32_t p = threadIdx.x & 3u;
  const uint32_t h = p >> 1, gq = p & 1u;

  // A, B: ql[64h+16gq..], ql[64h+32+16gq..]; C: qh[32h+16gq..]; S: the
  // eight scales of half h; D: d (q6_k.rs:13-43).
  const XGeom xg = x_geom<T>(FQ ? x + t0 * width : nullptr, width, nbmax);
  XRound<FQ ? FQ : 1> xr;
  if (FQ) load_x_round<FQ ? FQ : 1, NT>(xr, xg, 0u);
  NormRound<FQ ? FQ : 1> nr;
  if constexpr (NORM) norm_load<FQ ? FQ : 1, NT>(nr, xg, nrm);
  // the activation's loads go out before any weight load (loads return in
  // issue order: the prologue waits only for these)
  __builtin_amdgcn_sched_barrier(0);
  u32x4 A[NI], B[NI], C[NI];
  uint2 S[NI];
  uint32_t D[NI];
  // the unit layout (rh_device.h): the lane's pieces A, B, C at
  // 64 tw + 16p, 1024 + 64 tw + 16p, 2048 + 64 tw + 16p (nontemporal, as in
  // q4k_body), the block's scales at 3072 + 16 tw, d at 3328 + 2 tw
  auto issue = [&](int i) {
    uint32_t tw;
    const uint8_t* grp = walk.addr(i, tw);
    A[i] = load16_nt(grp + 64u * tw + 16u * p);
    B[i] = load16_nt(grp + 1024u + 64u * tw + 16u * p);
    C[i] = load16_nt(grp + 2048u + 64u * tw + 16u * p);
    S[i] = *reinterpret_cast<const uint2*>(grp + 3072u + 16u * tw + 8u * h);
    D[i] = *reinterpret_cast<const uint16_t*>(grp + 3328u + 2u * tw);
  };
  constexpr int ahead = issue_ahead<NI, NORM>();
#pragma unroll
  for (int i = 0; i < ahead; i++) issue(i);

  if constexpr (NORM) norm_apply<FQ ? FQ : 1, NT>(xr, nr, xg, nrm, reinterpret_cast<float*>(lds + nrm.lds_offset),
                                    reinterpret_cast<float*>(lds + nrm.lds_offset) + wave_sum_floats(xg.total * 256u));
  if (FQ) {
    quantize_x_round<14, FQ ? FQ : 1, NT>(xr, xg, 0u, nbmax, act, d8, bias);
    quantize_x_rest<14, FQ ? FQ : 1, NT>(xg, nbmax, act, d8, bias);
  } else {
    stage_quants_swizzled<T, NT>(act, abytes, q, t0);
    for (uint32_t i = threadIdx.x; i < T * nbmax * 16u; i += NT) {
      const uint32_t t = i / (nbmax * 16u), k = i - t * nbmax * 16u;
      bias[i] = -32 * q.sums16[2u * (t0 + t) * q.bstride + k];
      if ((k & 15u) == 0) d8[t * nbmax + k / 16u] = q.scales[(t0 + t) * q.bstride + k / 2u];
    }
  }
  __syncthreads();

  const uint32_t k0 = 128u * h + 16u * gq;
  // FIX: the team's activation quants, 16-run biases and d8, read once
  u32x4 fa[4] = {};
  int32_t fb4[4] = {};
  float fd8 = 0.0f;
  if constexpr (FIX) {
    fa[0] = *reinterpret_cast<const u32x4*>(swz(act, walk.fb, k0));
    fa[1] = *reinterpret_cast<const u32x4*>(swz(act, walk.fb, k0 + 32u));
    fa[2] = *reinterpret_cast<const u32x4*>(swz(act, walk.fb, k0 + 64u));
    fa[3] = *reinterpret_cast<const u32x4*>(swz(act, walk.fb, k0 + 96u));
    const int32_t* bb = bias + walk.fb * 16u + 8u * h + gq;
    fb4[0] = bb[0];
    fb4[1] = bb[2];
    fb4[2] = bb[4];
    fb4[3] = bb[6];
    fd8 = d8[walk.fb];
  }
#pragma unroll
  for (int it = 0; it < NI; it++) {
    if (it + ahead < NI) issue(it + ahead);
    if (!walk.live(it)) break;  // uniform over the team
    uint32_t r, b;
    walk.rb(it, r, b);
    const Q6Dec q = q6k_decode(A[it], B[it], C[it], S[it], D[it], gq);
#pragma unroll
    for (int t = 0; t < T; t++) {
      u32x4 a0 = fa[0], a1 = fa[1], a2 = fa[2], a3 = fa[3];
      int32_t bv[4] = {fb4[0], fb4[1], fb4[2], fb4[3]};
      float dd8 = fd8;
      if constexpr (!FIX) {
        const int8_t* at = act + t * abytes;
        a0 = *reinterpret_cast<const u32x4*>(swz(at, b, k0));
        a1 = *reinterpret_cast<const u32x4*>(swz(at, b, k0 + 32u));
        a2 = *reinterpret_cast<const u32x4*>(swz(at, b, k0 + 64u));
        a3 = *reinterpret_cast<const u32x4*>(swz(at, b, k0 + 96u));
        const int32_t* bb = bias + t * nbmax * 16u + b * 16u + 8u * h + gq;
        bv[0] = bb[0];
        bv[1] = bb[2];
        bv[2] = bb[4];
        bv[3] = bb[6];
        dd8 = d8[t * nbmax + b];
      }
      const float term = q6k_term(q, a0, a1, a2, a3, bv, dd8);
      if (p == 0) terms[(__umul24(r, nbmax) + b) * T + t] = term;
    }
  }
  __syncthreads();
  write_rows<T, PAIR, NT, NORM && !PAIR && T == 1>(J, wr, terms, J.nb, nbmax, tokens, t0, nrm.pick);
}

// FIX: every job's nb is a power of two up to NT/4 (the launch checks). It is
// a kernel of its own rather than a branch in one: at the join of two walks
// the compiler merges their pending loads and then waits for the activation
// before issuing the first weights.
template <int T, int NI, int FQ, bool NORM, bool PAIR = false, uint32_t NT = kThreads, bool FIX = false>
__global__ __launch_bounds__(NT) void gemv_q6k_kernel(GemvJobs jobs, Q8Dev q, const float* __restrict__ x,
                                                       size_t width, uint32_t R, uint32_t nbmax, size_t tokens,
                                                       size_t t0, NormIn nrm) {
  extern __shared__ __align__(16) uint8_t lds[];
  static_assert(!FIX || T == 1, "fixed columns: one token");
  q6k_body<T, NI, FQ, NORM, PAIR, NT, FIX>(jobs.j[find_job(jobs)], q, x, width, R, nbmax, tokens, t0, nrm, lds);
}

// The same kernel with the activation's scalars first: the build preloads
// leading scalar arguments into SGPRs (-amdgpu-kernarg-preload-count), so the
// activation's first loads need no kernel-argument load (kq_preloads).
template <int T, int NI, int FQ, bool NORM, bool PAIR = false, uint32_t NT = kThreads, bool FIX = false>
__global__ __launch_bounds__(NT) void gemv_q6k_kernel_pl(const float* __restrict__ x, size_t width, uint32_t R,
                                                          uint32_t nbmax, size_t tokens, size_t t0, GemvJobs jobs,
                                                          Q8Dev q, NormIn nrm) {
  extern __shared__ __align__(16) uint8_t lds[];
  q6k_body<T, NI, FQ, NORM, PAIR, NT, FIX>(jobs.j[find_job(jobs)], q, x, width, R, nbmax, tokens, t0, nrm, lds);
}

// I2_S x I8_S --------------------------------------------------------------
// LDS: act [T][nbmax*128] i8 | prefix [T][nbmax+1] i32 (sums of the first 4b
// activation blocks) | divisor [T] f32
template <int T>
__global__ __launch_bounds__(256) void gemv_i2s_kernel(GemvJobs jobs, Q8Dev q, uint32_t R,
                                                       uint32_t nbmax, size_t tokens, size_t t0,
                                                       int32_t* raw) {
  extern __shared__ __align__(16) uint8_t lds[];
  const uint32_t abytes = nbmax * 128u;
  int8_t* act = reinterpret_cast<int8_t*>(lds);
  int32_t* prefix = reinterpret_cast<int32_t*>(lds + T * abytes);
  float* divisor = reinterpret_cast<float*>(prefix + T * (nbmax + 1u));

  const GemvJob& J = jobs.j[find_job(jobs)];
  const uint32_t row0 = (blockIdx.x - J.wg_begin) * R;
  const uint32_t nrows = min(R, J.rows - row0);
  const uint32_t nb = J.nb;

  stage_quants<T>(act, abytes, q, t0);
  if (threadIdx.x < static_cast<uint32_t>(T)) {
    const uint32_t t = threadIdx.x;
    const int32_t* s = q.sums + (t0 + t) * q.bstride;
    uint32_t acc = 0;
    prefix[t * (nbmax + 1u)] = 0;
    for (uint32_t b = 0; b < nbmax; b++) {
      acc += static_cast<uint32_t>(s[4u * b]) + static_cast<uint32_t>(s[4u * b + 1u]) +
             static_cast<uint32_t>(s[4u * b + 2u]) + static_cast<uint32_t>(s[4u * b + 3u]);
      prefix[t * (nbmax + 1u) + b + 1u] = static_cast<int32_t>(acc);
    }
    divisor[t] = q.n_blocks ? q.scales[(t0 + t) * q.bstride] : 0.0f;
  }
  __syncthreads();

  const uint32_t team = threadIdx.x >> 3, u = threadIdx.x & 7u;
  const uint32_t nchunk = 2u * nb;
  for (uint32_t r = team; r < nrows; r += kThreads / 8u) {
    const uint8_t* row = J.w + static_cast<size_t>(row0 + r) * J.stride;
    uint32_t acc[T];
#pragma unroll
    for (int t = 0; t < T; t++) acc[t] = 0;
    for (uint32_t c = u; c < nchunk; c += 8u) {
      const u32x4 w = load16(row + 16u * c);
      const uint32_t block = c >> 1, half = c & 1u;
      uint32_t c6[4], c4[4], c2[4], c0[4];
#pragma unroll
      for (int k = 0; k < 4; k++) {
        c6[k] = (w[k] >> 2) & 0x30303030u;  // code of shift 6, times 16
        c4[k] = w[k] & 0x30303030u;         // shift 4, times 16
        c2[k] = w[k] & 0x0C0C0C0Cu;         // shift 2, times 4
        c0[k] = w[k] & 0x03030303u;         // shift 0
      }
#pragma unroll
      for (int t = 0; t < T; t++) {
        const int8_t* a = act + t * abytes + 128u * block + 16u * half;
        const u32x4 a0 = *reinterpret_cast<const u32x4*>(a);
        const u32x4 a1 = *reinterpret_cast<const u32x4*>(a + 32u);
        const u32x4 a2 = *reinterpret_cast<const u32x4*>(a + 64u);
        const u32x4 a3 = *reinterpret_cast<const u32x4*>(a + 96u);
        int32_t P16 = 0, P4 = 0, P1 = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
          P16 = dot4(c6[k], a0[k], P16);
          P16 = dot4(c4[k], a1[k], P16);
          P4 = dot4(c2[k], a2[k], P4);
          P1 = dot4(c0[k], a3[k], P1);
        }
        acc[t] += static_cast<uint32_t>(P1 + (P4 >> 2) + (P16 >> 4));
      }
    }
#pragma unroll
    for (int t = 0; t < T; t++) {
      const uint32_t total = octet_sum(acc[t]);
      if (u == 0) {
        // ternary.rs:39,41: sum(code*q) - sum(q), wrapping
        const int32_t dot = static_cast<int32_t>(total - static_cast<uint32_t>(prefix[t * (nbmax + 1u) + nb]));
        const size_t idx = static_cast<size_t>(row0 + r) * tokens + t0 + t;
        if (idx < J.out_len) {
          if (raw) {
            raw[idx] = dot;
          } else {
            // ternary.rs:53-57: (dot as f32) / s * scale; 0 without a scale
            const float s = divisor[t];
            J.out[idx] = q.n_blocks ? __fdiv_rn(static_cast<float>(dot), s) * J.scale : 0.0f;
          }
        }
      }
    }
  }
}

// I2_S x I8_S, fused -------------------------------------------------------
// The workgroup quantizes its tokens itself (Q8Kind::Row, portable/q8.rs:38-49,
// 99-105, the arithmetic of quantize_row_kernel). Each lane keeps 4
// consecutive values of every 1024 in registers, loaded for the first token
// before the weights. One workgroup reduction
// gives the row's last NaN and its largest magnitude; without a NaN (the
// usual case) that fixes the divisor, and only a row with a NaN needs a
// second reduction, of the magnitudes after that NaN. The quants of the first
// nkeep values then go to LDS with one sum per 32.
constexpr uint32_t kFusedRowPasses = 8;  // rows of up to 8192 values

// Workgroup maxima of (p, m) over its 4 waves; `slot` alternates between
// calls so that one barrier per reduction suffices.
template <uint32_t NW = kThreads / 64u>  // waves in the workgroup
__device__ __forceinline__ void wg_max_pair(int32_t& p, uint32_t& m, int32_t* red, uint32_t slot) {
  p = half_max_i32(p);
  m = half_max_u32(m);
  p = max(__builtin_amdgcn_readlane(p, 0), __builtin_amdgcn_readlane(p, 32));
  m = max(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(m), 0)),
          static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(m), 32)));
  int32_t* r = red + slot * 2u * NW;
  if ((threadIdx.x & 63u) == 0) {
    r[threadIdx.x >> 6] = p;
    r[NW + (threadIdx.x >> 6)] = static_cast<int32_t>(m);
  }
  __syncthreads();
  p = r[0];
  m = static_cast<uint32_t>(r[NW]);
#pragma unroll
  for (uint32_t w = 1; w < NW; w++) {
    p = max(p, r[w]);
    m = max(m, static_cast<uint32_t>(r[NW + w]));
  }
}

struct RowX {
  float f[kFusedRowPasses][4];
};

// Token t's values into registers: 4 consecutive values of every 1024.
__device__ __forceinline__ void load_row_x(RowX& r, const float* __restrict__ v, uint32_t n, bool aligned) {
#pragma unroll
  for (uint32_t k = 0; k < kFusedRowPasses; k++) {
    const uint32_t e = 4u * threadIdx.x + 4u * kThreads * k;  // n is a multiple of 32
    if (e < n && aligned) {
      const u32x4 q4 = load16(reinterpret_cast<const uint8_t*>(v + e));
#pragma unroll
      for (uint32_t i = 0; i < 4; i++) r.f[k][i] = __uint_as_float(q4[i]);
    } else {
#pragma unroll
      for (uint32_t i = 0; i < 4; i++) r.f[k][i] = e < n ? v[e + i] : 0.0f;
    }
  }
}

// Token t from its registers into the LDS tiles; `slot` alternates the
// reduction scratch between calls.
__device__ __forceinline__ void quantize_row_regs(const RowX& r, uint32_t t, uint32_t n, uint32_t nkeep,
                                                  int8_t* act, int32_t* qs32, float* divisor, int32_t* red,
                                                  uint32_t& slot) {
  const uint32_t lane = threadIdx.x & 63u;
  int32_t last_nan = -1;
  float all_max = 0.0f;
#pragma unroll
  for (uint32_t k = 0; k < kFusedRowPasses; k++)
#pragma unroll
    for (uint32_t i = 0; i < 4; i++) {
      const uint32_t e = 4u * threadIdx.x + 4u * kThreads * k + i;
      const float m = __builtin_fabsf(r.f[k][i]);
      if (e < n && r.f[k][i] != r.f[k][i]) last_nan = static_cast<int32_t>(e);
      all_max = m > all_max ? m : all_max;  // NaN never enters
    }
  int32_t p = last_nan;
  uint32_t mb = __float_as_uint(all_max);
  wg_max_pair(p, mb, red, slot);
  slot ^= 1u;
  // C's MAX from 1e-5 in f64: a NaN restarts the maximum at the next value
  // (without the floor); a trailing NaN leaves it NaN
  double mx;
  if (p < 0) {
    mx = static_cast<double>(__uint_as_float(mb));
    mx = 1e-5 > mx ? 1e-5 : mx;
  } else {
    float after = 0.0f;
#pragma unroll
    for (uint32_t k = 0; k < kFusedRowPasses; k++)
#pragma unroll
      for (uint32_t i = 0; i < 4; i++) {
        const uint32_t e = 4u * threadIdx.x + 4u * kThreads * k + i;
        const float m = __builtin_fabsf(r.f[k][i]);
        if (e < n && static_cast<int32_t>(e) > p) after = m > after ? m : after;
      }
    int32_t unused = -1;
    uint32_t ab = __float_as_uint(after);
    wg_max_pair(unused, ab, red, slot);
    slot ^= 1u;
    mx = p == static_cast<int32_t>(n) - 1 ? __builtin_nan("") : static_cast<double>(__uint_as_float(ab));
  }
  const float div = static_cast<float>(127.0 / mx);
#pragma unroll
  for (uint32_t k = 0; k < kFusedRowPasses; k++) {
    const uint32_t base = 4u * threadIdx.x + 4u * kThreads * k;
    int32_t qv[4];
    int32_t s = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float prod = r.f[k][i] * div;
      qv[i] = round_row_to_i8(prod);
      s += qv[i];
    }
    // a 32-block is 8 lanes of 4 values
    int32_t s32 = s + static_cast<int32_t>(dpp<0xB1>(static_cast<uint32_t>(s)));
    s32 += static_cast<int32_t>(dpp<0x4E>(static_cast<uint32_t>(s32)));
    s32 += static_cast<int32_t>(dpp<0x141>(static_cast<uint32_t>(s32)));
    if (base < nkeep) {
      *reinterpret_cast<uint32_t*>(act + t * nkeep + base) =
          (static_cast<uint32_t>(qv[0]) & 0xffu) | ((static_cast<uint32_t>(qv[1]) & 0xffu) << 8) |
          ((static_cast<uint32_t>(qv[2]) & 0xffu) << 16) | (static_cast<uint32_t>(qv[3]) << 24);
      if ((lane & 7u) == 0) qs32[t * (nkeep / 32u) + base / 32u] = s32;
    }
  }
  if (threadIdx.x == 0) divisor[t] = div;
}

// LDS: act [T][nbmax*128] i8 | qs32 [T][nbmax*4] i32 | divisor [T] f32 |
// reduction scratch. A team of lpr lanes (a power of two) owns a row of each
// of the workgroup's G row groups; lane l holds chunks l, l + lpr, ... (CPL
// of them) of 16 bytes of each, all loaded before the activation is
// quantized, so one quantization serves G groups of rows.
template <int T, int CPL, int G>
__global__ __launch_bounds__(256) void gemv_i2s_fused_kernel(GemvJobs jobs, const float* __restrict__ x,
                                                             size_t width, uint32_t nq, uint32_t nbmax,
                                                             uint32_t lpr, size_t tokens, size_t t0,
                                                             int32_t* raw) {
  extern __shared__ __align__(16) uint8_t lds[];
  const uint32_t nkeep = nbmax * 128u;
  int8_t* act = reinterpret_cast<int8_t*>(lds);
  int32_t* qs32 = reinterpret_cast<int32_t*>(lds + T * nkeep);
  float* divisor = reinterpret_cast<float*>(qs32 + T * nbmax * 4u);
  int32_t* red = reinterpret_cast<int32_t*>(divisor + T);  // [2 slots][2][waves]

  const GemvJob& J = jobs.j[find_job(jobs)];
  const uint32_t R = kThreads / lpr;
  const uint32_t r = threadIdx.x / lpr, cl = threadIdx.x & (lpr - 1u);
  const uint32_t row0 = (blockIdx.x - J.wg_begin) * R * static_cast<uint32_t>(G) + r;
  const uint32_t nchunk = 2u * J.nb;
  // token t0's values first: loads return in issue order (see load_x_round)
  const float* xt = x + t0 * width;
  const uint32_t n = nq * 32u;
  const bool aligned = ((reinterpret_cast<uintptr_t>(xt) | (width * 4u)) & 15u) == 0;
  RowX rx;
  load_row_x(rx, xt, n, aligned);
  u32x4 w[G][CPL];
#pragma unroll
  for (int gi = 0; gi < G; gi++) {
    const uint32_t row = row0 + static_cast<uint32_t>(gi) * R;
#pragma unroll
    for (int i = 0; i < CPL; i++) {
      const uint32_t c = cl + static_cast<uint32_t>(i) * lpr;
      w[gi][i] = (row < J.rows && c < nchunk)
                     ? load16(J.w + __umul24(row, static_cast<uint32_t>(J.stride)) + 16u * c)
                     : u32x4{0, 0, 0, 0};
    }
  }

  uint32_t slot = 0;
  quantize_row_regs(rx, 0u, n, nkeep, act, qs32, divisor, red, slot);
  for (uint32_t t = 1; t < static_cast<uint32_t>(T); t++) {
    load_row_x(rx, xt + t * width, n, aligned);
    quantize_row_regs(rx, t, n, nkeep, act, qs32, divisor, red, slot);
  }
  __syncthreads();

#pragma unroll
  for (int gi = 0; gi < G; gi++) {
    const uint32_t row = row0 + static_cast<uint32_t>(gi) * R;
    const bool live = row < J.rows;
    uint32_t acc[T];
#pragma unroll
    for (int t = 0; t < T; t++) acc[t] = 0;
#pragma unroll
    for (int i = 0; i < CPL; i++) {
      const uint32_t c = cl + static_cast<uint32_t>(i) * lpr;
      if (c >= nchunk) break;
      uint32_t c6[4], c4[4], c2[4], c0[4];
#pragma unroll
      for (int k = 0; k < 4; k++) {
        c6[k] = (w[gi][i][k] >> 2) & 0x30303030u;  // code of shift 6, times 16
        c4[k] = w[gi][i][k] & 0x30303030u;         // shift 4, times 16
        c2[k] = w[gi][i][k] & 0x0C0C0C0Cu;         // shift 2, times 4
        c0[k] = w[gi][i][k] & 0x03030303u;         // shift 0
      }
#pragma unroll
      for (int t = 0; t < T; t++) {
        const int8_t* a = act + t * nkeep + 128u * (c >> 1) + 16u * (c & 1u);
        const u32x4 a0 = *reinterpret_cast<const u32x4*>(a);
        const u32x4 a1 = *reinterpret_cast<const u32x4*>(a + 32u);
        const u32x4 a2 = *reinterpret_cast<const u32x4*>(a + 64u);
        const u32x4 a3 = *reinterpret_cast<const u32x4*>(a + 96u);
        int32_t P16 = 0, P4 = 0, P1 = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
          P16 = dot4(c6[k], a0[k], P16);
          P16 = dot4(c4[k], a1[k], P16);
          P4 = dot4(c2[k], a2[k], P4);
          P1 = dot4(c0[k], a3[k], P1);
        }
        acc[t] += static_cast<uint32_t>(P1 + (P4 >> 2) + (P16 >> 4));
      }
    }
    // ternary.rs:39,41: minus the sum of the quants of the row's blocks (wrapping)
#pragma unroll
    for (int t = 0; t < T; t++)
      for (uint32_t k = cl; k < 4u * J.nb; k += lpr) acc[t] -= static_cast<uint32_t>(qs32[t * nbmax * 4u + k]);
#pragma unroll
    for (int t = 0; t < T; t++) {
      uint32_t v = acc[t];
      for (uint32_t off = lpr >> 1; off > 0; off >>= 1)
        v += static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), static_cast<int>(off), 64));
      const size_t idx = static_cast<size_t>(row) * tokens + t0 + t;
      if (cl == 0 && live && idx < J.out_len) {
        const int32_t dot = static_cast<int32_t>(v);
        if (raw) raw[idx] = dot;
        // ternary.rs:53-57: (dot as f32) / s * scale; 0 without a scale
        else J.out[idx] = nq ? __fdiv_rn(static_cast<float>(dot), divisor[t]) * J.scale : 0.0f;
      }
    }
  }
}

// I2_S x I8_S, one token ----------------------------------------------------
// The decode case of the kernel above, arranged so that each step waits for
// its own inputs only. Every global load is unconditional (addresses clamped,
// surplus values masked in registers), so the number of loads in flight is
// known where each is used: the activation's loads go out first and the
// weights' after them, and since loads complete in issue order the
// activation's quantization waits for its own loads while the weights are
// still arriving. The sum of the quants that ternary.rs:39,41 subtracts is the
// same for every row of a job: it is reduced once, beside the quantization,
// rather than per row. A team of LPR lanes owns a row; lane l of the team
// holds chunks l, l + LPR, ... (CPL of them) of 16 bytes. Job fields are read
// into registers once.
// LDS: act [nkeep] i8 | red [2 slots][2][waves] i32 | qsw [waves] i32
template <uint32_t NT, int LPR, int CPL, bool ONE_JOB>
__global__ __launch_bounds__(NT) void gemv_i2s_one_kernel(GemvJobs jobs, const float* __restrict__ x, uint32_t n,
                                                           uint32_t nkeep, size_t tokens, size_t t0, int32_t* raw) {
  extern __shared__ __align__(16) uint8_t lds[];
  constexpr uint32_t kWaves = NT / 64u;
  constexpr uint32_t R = NT / static_cast<uint32_t>(LPR);
  constexpr uint32_t kPasses = 4u * kThreads * kFusedRowPasses / (4u * NT);  // rows of up to 8192 values
  int8_t* act = reinterpret_cast<int8_t*>(lds);
  int32_t* red = reinterpret_cast<int32_t*>(lds + nkeep);  // nkeep is a multiple of 128
  int32_t* qsw = red + 4u * kWaves;

  // a launch of one job reads it at a fixed offset, without find_job's
  // dependent round trip
  const GemvJob& J = jobs.j[ONE_JOB ? 0u : find_job(jobs)];
  const uint8_t* const wbase = J.w;
  const uint32_t stride = J.stride, rows = J.rows, nb = J.nb;
  float* const out = J.out;
  const size_t out_len = J.out_len;
  const float scale = J.scale;
  const uint32_t cl = threadIdx.x & static_cast<uint32_t>(LPR - 1);
  const uint32_t row = (blockIdx.x - J.wg_begin) * R + threadIdx.x / static_cast<uint32_t>(LPR);
  const uint32_t nchunk = 2u * nb;

  // the activation (x: token t0's n values): 4 consecutive values of every
  // 1024 per lane; positions past n read the last 4 values and are zeroed below
  f32x4 xv[kPasses];
#pragma unroll
  for (uint32_t k = 0; k < kPasses; k++) {
    const uint32_t e = min(4u * threadIdx.x + 4u * NT * k, n - 4u);
    const u32x4 v = load16_a4(reinterpret_cast<const uint8_t*>(x + e));
    xv[k] = f32x4{__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3])};
  }
  // then the weights (rows past the job's last read its last row)
  // (a matrix stays below 4 GiB, rows below 2^24: the 24-bit product is exact)
  const uint8_t* wrow = wbase + __umul24(min(row, rows - 1u), stride);
  u32x4 w[CPL];
#pragma unroll
  for (int i = 0; i < CPL; i++) {
    const uint32_t c = min(cl + static_cast<uint32_t>(i * LPR), nchunk - 1u);
    w[i] = load16_nt(wrow + 16u * c);  // read once: nontemporal
  }
  // the scalars the stores need, loaded now rather than after the dot (the
  // compiler otherwise reloads them there, one dependent round trip each)
  __asm__ volatile("" ::"s"(out), "s"(out_len), "s"(scale), "s"(tokens), "s"(t0), "s"(raw));
  // keep the weights' loads ahead of the quantization (the scheduler would
  // otherwise sink them below the activation's first use)
  __builtin_amdgcn_sched_barrier(0);

  // C's MAX over |x| from 1e-5 in f64 (portable/q8.rs:38-49). Without a NaN
  // or an infinity in the row (the usual case) that is its largest magnitude,
  // floored at 1e-5, and the quants need no NaN rule; a row with either takes
  // the exact path below. Only the passes that hold values are computed.
  const uint32_t npass = (n + 4u * NT - 1u) / (4u * NT);
  float all_max = 0.0f;
  bool has_nan = false;
#pragma unroll
  for (uint32_t k = 0; k < kPasses; k++) {
    if (k < npass) {
      if (4u * NT * (k + 1u) > n) {  // the last pass may run past n
        const bool in = 4u * threadIdx.x + 4u * NT * k < n;
#pragma unroll
        for (int i = 0; i < 4; i++) xv[k][i] = in ? xv[k][i] : 0.0f;
      }
      // maxNum: a NaN never enters the maximum
      all_max = __builtin_fmaxf(all_max, __builtin_fmaxf(__builtin_fabsf(xv[k][0]), __builtin_fabsf(xv[k][1])));
      all_max = __builtin_fmaxf(all_max, __builtin_fmaxf(__builtin_fabsf(xv[k][2]), __builtin_fabsf(xv[k][3])));
      has_nan |= __builtin_isunordered(xv[k][0], xv[k][1]) | __builtin_isunordered(xv[k][2], xv[k][3]);
    }
  }
  int32_t p = has_nan ? 0 : -1;
  uint32_t mb = __float_as_uint(all_max);
  wg_max_pair<kWaves>(p, mb, red, 0u);
  const bool exact = p >= 0 || mb == 0x7f800000u;  // a NaN, or an infinity
  double mx;
  if (p < 0) {
    mx = static_cast<double>(__uint_as_float(mb));
    mx = 1e-5 > mx ? 1e-5 : mx;
  } else {
    // a NaN restarts the maximum at the next value (without the floor); a
    // trailing NaN leaves it NaN
    int32_t last_nan = -1;
#pragma unroll
    for (uint32_t k = 0; k < kPasses; k++)
      if (k < npass)
#pragma unroll
        for (uint32_t i = 0; i < 4; i++)
          if (xv[k][i] != xv[k][i]) last_nan = static_cast<int32_t>(4u * threadIdx.x + 4u * NT * k + i);
    uint32_t unused = 0;
    wg_max_pair<kWaves>(last_nan, unused, red, 1u);
    float after = 0.0f;
#pragma unroll
    for (uint32_t k = 0; k < kPasses; k++)
      if (k < npass)
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) {
          const int32_t e = static_cast<int32_t>(4u * threadIdx.x + 4u * NT * k + i);
          const float m = __builtin_fabsf(xv[k][i]);
          if (e > last_nan) after = m > after ? m : after;
        }
    int32_t none = -1;
    uint32_t ab = __float_as_uint(after);
    wg_max_pair<kWaves>(none, ab, red, 0u);  // slot 0 is free again after slot 1's barrier
    mx = last_nan == static_cast<int32_t>(n) - 1 ? __builtin_nan("") : static_cast<double>(__uint_as_float(ab));
  }
  const float div = static_cast<float>(127.0 / mx);

  // the quants into LDS (round_row_to_i8; on the usual path every product is
  // finite and within +-127.5, so a clamp replaces the NaN rule); the sum of
  // those of the job's blocks, per wave
  const uint32_t ncover = 128u * nb;
  int32_t qsum = 0;
#pragma unroll
  for (uint32_t k = 0; k < kPasses; k++) {
    if (k < npass) {
      const uint32_t base = 4u * threadIdx.x + 4u * NT * k;
      int32_t qv[4];
      if (!exact) {
#pragma unroll
        for (int i = 0; i < 4; i++)
          qv[i] = static_cast<int32_t>(__builtin_amdgcn_fmed3f(__builtin_rintf(xv[k][i] * div), -128.0f, 127.0f));
      } else {
#pragma unroll
        for (int i = 0; i < 4; i++) qv[i] = round_row_to_i8(xv[k][i] * div);
      }
      // bytes q0 q1 q2 q3, low first
      const uint32_t lo = __builtin_amdgcn_perm(static_cast<uint32_t>(qv[1]), static_cast<uint32_t>(qv[0]), 0x0c0c0400u);
      const uint32_t hi = __builtin_amdgcn_perm(static_cast<uint32_t>(qv[3]), static_cast<uint32_t>(qv[2]), 0x04000c0cu);
      const uint32_t packed = lo | hi;
      if (base < nkeep) *reinterpret_cast<uint32_t*>(act + base) = packed;
      if (base < ncover) qsum = dot4(packed, 0x01010101u, qsum);
    }
  }
  uint32_t ws = static_cast<uint32_t>(qsum);
  ws += dpp<0xB1>(ws);
  ws += dpp<0x4E>(ws);
  ws += dpp<0x141>(ws);
  ws += dpp<0x140>(ws);
  ws += static_cast<uint32_t>(__builtin_amdgcn_ds_swizzle(static_cast<int>(ws), 0x401F));
  ws = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(ws), 0)) +
       static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(ws), 32));
  if ((threadIdx.x & 63u) == 0) qsw[threadIdx.x >> 6] = static_cast<int32_t>(ws);
  __syncthreads();
  uint32_t qtotal = 0;
#pragma unroll
  for (uint32_t v = 0; v < kWaves; v++) qtotal += static_cast<uint32_t>(qsw[v]);

  uint32_t acc = 0;
#pragma unroll
  for (int i = 0; i < CPL; i++) {
    const uint32_t craw = cl + static_cast<uint32_t>(i * LPR);
    const uint32_t c = min(craw, nchunk - 1u);
    const uint32_t live = craw < nchunk ? 0xffffffffu : 0u;
    const int8_t* a = act + 128u * (c >> 1) + 16u * (c & 1u);
    const u32x4 a0 = *reinterpret_cast<const u32x4*>(a);
    const u32x4 a1 = *reinterpret_cast<const u32x4*>(a + 32u);
    const u32x4 a2 = *reinterpret_cast<const u32x4*>(a + 64u);
    const u32x4 a3 = *reinterpret_cast<const u32x4*>(a + 96u);
    int32_t P16 = 0, P4 = 0, P1 = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const uint32_t wk = w[i][k] & live;
      P16 = dot4((wk >> 2) & 0x30303030u, a0[k], P16);  // code of shift 6, times 16
      P16 = dot4(wk & 0x30303030u, a1[k], P16);         // shift 4, times 16
      P4 = dot4(wk & 0x0C0C0C0Cu, a2[k], P4);           // shift 2, times 4
      P1 = dot4(wk & 0x03030303u, a3[k], P1);           // shift 0
    }
    acc += static_cast<uint32_t>(P1 + (P4 >> 2) + (P16 >> 4));
  }
  // the team's sum, left in every lane of it (wrapping)
  acc += dpp<0xB1>(acc);
  acc += dpp<0x4E>(acc);
  if constexpr (LPR >= 8) acc += dpp<0x141>(acc);
  if constexpr (LPR >= 16) acc += dpp<0x140>(acc);
  if constexpr (LPR >= 32) acc += static_cast<uint32_t>(__builtin_amdgcn_ds_swizzle(static_cast<int>(acc), 0x401F));
  if constexpr (LPR == 64)
    acc = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(acc), 0)) +
          static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(acc), 32));
  if (cl == 0 && row < rows) {
    const size_t idx = static_cast<size_t>(row) * tokens + t0;
    if (idx < out_len) {
      // ternary.rs:39,41: sum(code*q) - sum(q), wrapping
      const int32_t dot = static_cast<int32_t>(acc - qtotal);
      if (raw) raw[idx] = dot;
      // ternary.rs:53-57: (dot as f32) / s * scale
      else out[idx] = __fdiv_rn(static_cast<float>(dot), div) * scale;
    }
  }
}

// The team sum of gemv_i2s_one_kernel's row accumulators, left in every lane
// of the team (wrapping).
template <int LPR>
__device__ __forceinline__ uint32_t i2s_team_sum(uint32_t acc) {
  acc += dpp<0xB1>(acc);
  acc += dpp<0x4E>(acc);
  if constexpr (LPR >= 8) acc += dpp<0x141>(acc);
  if constexpr (LPR >= 16) acc += dpp<0x140>(acc);
  if constexpr (LPR >= 32) acc += static_cast<uint32_t>(__builtin_amdgcn_ds_swizzle(static_cast<int>(acc), 0x401F));
  if constexpr (LPR == 64)
    acc = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(acc), 0)) +
          static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(acc), 32));
  return acc;
}

// The sum of v over the wave, in every lane (wrapping).
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += dpp<0x141>(v);
  v += dpp<0x140>(v);
  v += static_cast<uint32_t>(__builtin_amdgcn_ds_swizzle(static_cast<int>(v), 0x401F));
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 0)) +
         static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 32));
}

// I2_S x a pre-quantized I8_S activation (Q8Kind::Row), T tokens: the layout
// of gemv_i2s_one_kernel with the quantization replaced by a copy. Every load
// is unconditional: the tokens' quants (nkeep bytes each, at most 8192) and
// the 32-block sums of the job's blocks go out first, the weights after
// them; the quants go to LDS and each token's sum of quants (ternary.rs:39,41
// subtracts it) is reduced once per workgroup.
// LDS: act [T][nkeep] i8 | qsw [T][waves] i32
template <int T, int LPR, int CPL>
__global__ __launch_bounds__(256) void gemv_i2s_q8_kernel(GemvJobs jobs, Q8Dev q, uint32_t nkeep, size_t tokens,
                                                          size_t t0, int32_t* raw) {
  extern __shared__ __align__(16) uint8_t lds[];
  constexpr uint32_t kWaves = kThreads / 64u;
  constexpr uint32_t R = kThreads / static_cast<uint32_t>(LPR);
  constexpr uint32_t ACH = 2u * static_cast<uint32_t>(T);  // 16-byte chunks a thread: nkeep <= 8192
  int8_t* act = reinterpret_cast<int8_t*>(lds);
  int32_t* qsw = reinterpret_cast<int32_t*>(lds + T * nkeep);

  const GemvJob& J = jobs.j[find_job(jobs)];
  const uint8_t* const wbase = J.w;
  const uint32_t stride = J.stride, rows = J.rows, nb = J.nb;
  float* const out = J.out;
  const size_t out_len = J.out_len;
  const float scale = J.scale;
  const uint32_t cl = threadIdx.x & static_cast<uint32_t>(LPR - 1);
  const uint32_t row = (blockIdx.x - J.wg_begin) * R + threadIdx.x / static_cast<uint32_t>(LPR);
  const uint32_t nchunk = 2u * nb;
  const uint32_t qs32 = static_cast<uint32_t>(q.qstride), bs32 = static_cast<uint32_t>(q.bstride);

  // the tokens' quants: chunk c of token t is c + t * cpt (past the last,
  // the last chunk again, not stored)
  const uint32_t cpt = nkeep / 16u, nch = static_cast<uint32_t>(T) * cpt;
  u32x4 ar[ACH];
#pragma unroll
  for (uint32_t i = 0; i < ACH; i++) {
    const uint32_t c = min(threadIdx.x + i * kThreads, nch - 1u);
    const uint32_t t = T == 1 ? 0u : c / cpt, k = c - t * cpt;
    ar[i] = load16(reinterpret_cast<const uint8_t*>(q.quants) + (t0 + t) * qs32 + 16u * k);
  }
  // the job's 32-block sums, one a thread and token (4 nb <= 256)
  int32_t sv[T];
#pragma unroll
  for (int t = 0; t < T; t++) sv[t] = q.sums[(t0 + t) * bs32 + min(threadIdx.x, 4u * nb - 1u)];
  // the weights (rows past the job's last read its last row)
  const uint8_t* wrow = wbase + __umul24(min(row, rows - 1u), stride);
  u32x4 w[CPL];
#pragma unroll
  for (int i = 0; i < CPL; i++) {
    const uint32_t c = min(cl + static_cast<uint32_t>(i * LPR), nchunk - 1u);
    w[i] = load16_nt(wrow + 16u * c);  // read once: nontemporal
  }
  __asm__ volatile("" ::"s"(out), "s"(out_len), "s"(scale), "s"(tokens), "s"(t0), "s"(raw));
  __builtin_amdgcn_sched_barrier(0);

#pragma unroll
  for (uint32_t i = 0; i < ACH; i++) {
    const uint32_t c = threadIdx.x + i * kThreads;
    if (c < nch) {
      const uint32_t t = T == 1 ? 0u : c / cpt, k = c - t * cpt;
      *reinterpret_cast<u32x4*>(act + t * nkeep + 16u * k) = ar[i];
    }
  }
#pragma unroll
  for (int t = 0; t < T; t++) {
    const uint32_t ws = wave_sum_u32(threadIdx.x < 4u * nb ? static_cast<uint32_t>(sv[t]) : 0u);
    if ((threadIdx.x & 63u) == 0) qsw[t * kWaves + (threadIdx.x >> 6)] = static_cast<int32_t>(ws);
  }
  __syncthreads();

  uint32_t acc[T];
#pragma unroll
  for (int t = 0; t < T; t++) acc[t] = 0;
#pragma unroll
  for (int i = 0; i < CPL; i++) {
    const uint32_t craw = cl + static_cast<uint32_t>(i * LPR);
    const uint32_t c = min(craw, nchunk - 1u);
    const uint32_t live = craw < nchunk ? 0xffffffffu : 0u;
    uint32_t c6[4], c4[4], c2[4], c0[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const uint32_t wk = w[i][k] & live;
      c6[k] = (wk >> 2) & 0x30303030u;  // code of shift 6, times 16
      c4[k] = wk & 0x30303030u;         // shift 4, times 16
      c2[k] = wk & 0x0C0C0C0Cu;         // shift 2, times 4
      c0[k] = wk & 0x03030303u;         // shift 0
    }
#pragma unroll
    for (int t = 0; t < T; t++) {
      const int8_t* a = act + t * nkeep + 128u * (c >> 1) + 16u * (c & 1u);
      const u32x4 a0 = *reinterpret_cast<const u32x4*>(a);
      const u32x4 a1 = *reinterpret_cast<const u32x4*>(a + 32u);
      const u32x4 a2 = *reinterpret_cast<const u32x4*>(a + 64u);
      const u32x4 a3 = *reinterpret_cast<const u32x4*>(a + 96u);
      int32_t P16 = 0, P4 = 0, P1 = 0;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        P16 = dot4(c6[k], a0[k], P16);
        P16 = dot4(c4[k], a1[k], P16);
        P4 = dot4(c2[k], a2[k], P4);
        P1 = dot4(c0[k], a3[k], P1);
      }
      acc[t] += static_cast<uint32_t>(P1 + (P4 >> 2) + (P16 >> 4));
    }
  }
#pragma unroll
  for (int t = 0; t < T; t++) {
    const uint32_t v = i2s_team_sum<LPR>(acc[t]);
    uint32_t qtotal = 0;
#pragma unroll
    for (uint32_t u = 0; u < kWaves; u++) qtotal += static_cast<uint32_t>(qsw[t * kWaves + u]);
    const size_t idx = static_cast<size_t>(row) * tokens + t0 + t;
    if (cl == 0 && row < rows && idx < out_len) {
      // ternary.rs:39,41: sum(code*q) - sum(q), wrapping
      const int32_t dot = static_cast<int32_t>(v - qtotal);
      if (raw) {
        raw[idx] = dot;
      } else {
        // ternary.rs:53-57: (dot as f32) / s * scale; 0 without a scale
        const float s = q.n_blocks ? q.scales[(t0 + t) * bs32] : 0.0f;
        out[idx] = q.n_blocks ? __fdiv_rn(static_cast<float>(dot), s) * scale : 0.0f;
      }
    }
  }
}

// Dense f32 ---------------------------------------------------------------
// rusticide-simd/src/float.rs:23-36: eight fused lanes over the whole chunks,
// the lanes added in order from -0.0, then the unfused tail (from -0.0).
// A team of 8 lanes per row keeps exactly those eight accumulators.
template <int T>
__global__ __launch_bounds__(256) void gemv_dense_kernel(GemvJobs jobs, const float* __restrict__ x,
                                                         size_t width, uint32_t R, size_t tokens,
                                                         size_t t0) {
  const GemvJob& J = jobs.j[find_job(jobs)];
  const uint32_t row0 = (blockIdx.x - J.wg_begin) * R;
  const uint32_t nrows = min(R, J.rows - row0);
  const uint32_t n = J.nb;  // elements both operands hold
  const uint32_t team = threadIdx.x >> 3, i = threadIdx.x & 7u;
  const uint32_t chunks = n / 8u;
  for (uint32_t r = team; r < nrows; r += kThreads / 8u) {
    const float* w = reinterpret_cast<const float*>(J.w + static_cast<size_t>(row0 + r) * J.stride);
#pragma unroll
    for (int t = 0; t < T; t++) {
      const float* xt = x + (t0 + t) * width;
      float acc = 0.0f;
      for (uint32_t c = 0; c < chunks; c++) acc = __builtin_fmaf(w[8u * c + i], xt[8u * c + i], acc);
      float lanes[8];
#pragma unroll
      for (int k = 0; k < 8; k++) lanes[k] = __shfl(acc, (threadIdx.x & ~7u) + k, 64);
      if (i == 0) {
        float tail = -0.0f;
        for (uint32_t k = 8u * chunks; k < n; k++) {
          const float prod = w[k] * xt[k];
          tail += prod;
        }
        float s = -0.0f;
#pragma unroll
        for (int k = 0; k < 8; k++) s += lanes[k];
        const size_t idx = static_cast<size_t>(row0 + r) * tokens + t0 + t;
        if (idx < J.out_len) J.out[idx] = s + tail;
      }
    }
  }
}

// Dequantize one row (Matrix::copy_row, model/src/weights.rs:120-150) -------
__global__ __launch_bounds__(256) void dequantize_row_kernel(uint32_t type_id, const uint8_t* m, size_t pitch,
                                                             uint32_t row, uint32_t nb, float scale, float* out,
                                                             size_t out_len) {
  const uint32_t bs = type_id == 36u ? 128u : 256u;
  const size_t n = min(static_cast<size_t>(nb) * bs, out_len);
  for (size_t e = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x; e < n;
       e += static_cast<size_t>(gridDim.x) * kThreads) {
    const uint32_t b = static_cast<uint32_t>(e / bs), l = static_cast<uint32_t>(e % bs);
    float v;
    if (type_id == 12u || type_id == 14u) {
      v = unit_weight(m, type_id, row * static_cast<uint32_t>(pitch) + b, l);
    } else {  // quantize/src/i2_s.rs:15-21 then i2_s_apply_scale (:33-37)
      const uint8_t byte = m[static_cast<size_t>(row) * pitch + static_cast<size_t>(b) * 32u + l % 32u];
      const uint32_t code = (byte >> (6u - 2u * (l / 32u))) & 3u;
      const float c = static_cast<float>(code) - 1.0f;
      v = c * scale;
    }
    out[e] = v;
  }
}

template <int T>
size_t lds_bytes(uint32_t type_id, uint32_t nbmax, uint32_t R) {
  if (type_id == 12u) return T * nbmax * 256u + T * nbmax * 4u + T * nbmax * 32u + R * nbmax * T * 4u;
  if (type_id == 14u) return T * nbmax * 256u + T * nbmax * 4u + T * nbmax * 64u + R * nbmax * T * 4u;
  if (type_id == 36u) return T * nbmax * 128u + T * (nbmax + 1u) * 4u + T * 4u;
  return 0;
}

// Blocks per 4-lane team in the k-quant kernels (1, 2 or 4), chosen per
// launch: the smallest that lets every workgroup of the grid be resident at
// once, so no rows wait for a second generation of workgroups.
// Tuning::gemv_ni forces it and Tuning::interleave = false keeps every
// workgroup's rows contiguous, for tuning.
bool interleave_rows() { return tuning().interleave; }

uint32_t forced_blocks_per_team() { return static_cast<uint32_t>(tuning().gemv_ni); }

// Lanes of a one-round one-token workgroup for a 17- to 32-block row: a
// half-wave quantizes each block.
uint32_t onepass_lanes(uint32_t nb) { return nb <= 24u ? 768u : 1024u; }

// Rows per workgroup: one per 8-lane team for I2_S and dense rows; for the
// k-quants, whole rows of nb blocks over 64 teams of ni blocks each.
uint32_t rows_per_wg(uint32_t type_id, uint32_t nb, uint32_t ni) {
  if (type_id == 36u || type_id == 0u) return 32u;
  const uint32_t R = ni * (kThreads / 4u) / nb;
  return R < 1u ? 1u : R;
}

// A k-quant GEMV kernel and the order of its arguments: `preload` kernels
// are the _pl forms (the activation's scalars first, loaded into SGPRs before
// the first instruction), the others take the jobs first.
struct KqFn {
  void* fn = nullptr;
  bool preload = false;
  explicit operator bool() const { return fn != nullptr; }
};

// Preloaded arguments measured faster for the decode's launches (TinyLlama
// step 671.3-673.6 against 677.5-678.3 us) and slower for the eight-block
// launches without a norm (the output-sized one-round GEMV, 32000x2048 Q6_K:
// 11.20-11.23 against 10.99-11.10 us), which keep theirs in memory.
template <int NI, bool NORM>
constexpr bool kq_preloads() { return NI != 8 || NORM; }

template <int FMT, int T, int NI, int FQ, bool NORM = false, bool PAIR = false, uint32_t NT = kThreads,
          bool FIX = false>
KqFn kq_kernel() {
  if constexpr (kq_preloads<NI, NORM>())
    return {FMT == 12 ? reinterpret_cast<void*>(gemv_q4k_kernel_pl<T, NI, FQ, NORM, PAIR, NT, FIX>)
                      : reinterpret_cast<void*>(gemv_q6k_kernel_pl<T, NI, FQ, NORM, PAIR, NT, FIX>),
            true};
  else
    return {FMT == 12 ? reinterpret_cast<void*>(gemv_q4k_kernel<T, NI, FQ, NORM, PAIR, NT, FIX>)
                      : reinterpret_cast<void*>(gemv_q6k_kernel<T, NI, FQ, NORM, PAIR, NT, FIX>),
            false};
}

// The fixed-column kernels of the one-token, one-round launches (an empty
// KqFn where none is built): 1, 2, 4 or 8 blocks per team (8: not for a pair);
// norm-fused (pair or not) and plain.
template <int FMT, uint32_t NT>
KqFn kq_fix_kernel_nt(uint32_t ni, bool norm, bool pair) {
  if (norm && pair) {
    return ni == 1u ? kq_kernel<FMT, 1, 1, 1, true, true, NT, true>()
           : ni == 2u ? kq_kernel<FMT, 1, 2, 1, true, true, NT, true>()
           : ni == 4u ? kq_kernel<FMT, 1, 4, 1, true, true, NT, true>()
                      : KqFn{};
  }
  if (pair) return KqFn{};
  if (norm) {
    return ni == 1u ? kq_kernel<FMT, 1, 1, 1, true, false, NT, true>()
           : ni == 2u ? kq_kernel<FMT, 1, 2, 1, true, false, NT, true>()
           : ni == 4u ? kq_kernel<FMT, 1, 4, 1, true, false, NT, true>()
           : ni == 8u ? kq_kernel<FMT, 1, 8, 1, true, false, NT, true>()
                      : KqFn{};
  }
  return ni == 1u ? kq_kernel<FMT, 1, 1, 1, false, false, NT, true>()
         : ni == 2u ? kq_kernel<FMT, 1, 2, 1, false, false, NT, true>()
         : ni == 4u ? kq_kernel<FMT, 1, 4, 1, false, false, NT, true>()
         : ni == 8u ? kq_kernel<FMT, 1, 8, 1, false, false, NT, true>()
                    : KqFn{};
}

KqFn kq_fix_kernel(uint32_t type_id, uint32_t ni, bool norm, bool pair, uint32_t nt) {
  if (nt == kThreads)
    return type_id == 12u ? kq_fix_kernel_nt<12, kThreads>(ni, norm, pair)
                          : kq_fix_kernel_nt<14, kThreads>(ni, norm, pair);
  return type_id == 12u ? kq_fix_kernel_nt<12, 2u * kThreads>(ni, norm, pair)
                        : kq_fix_kernel_nt<14, 2u * kThreads>(ni, norm, pair);
}

// The 512-lane one-token kernels: 128 teams of ni blocks each take the rows
// that 64 teams of 2*ni take at 256 lanes (nullptr where none is built).
template <int FMT>
KqFn kq_wide_kernel_fmt(uint32_t fq, uint32_t ni, bool norm, bool pair) {
  constexpr uint32_t W = 2u * kThreads;
  if (norm) {
    if (fq != 1u) return KqFn{};
    if (pair) {
      return ni == 1u ? kq_kernel<FMT, 1, 1, 1, true, true, W>() : ni == 2u ? kq_kernel<FMT, 1, 2, 1, true, true, W>()
             : ni == 4u                                            ? kq_kernel<FMT, 1, 4, 1, true, true, W>()
                                                                   : KqFn{};
    }
    return ni == 1u ? kq_kernel<FMT, 1, 1, 1, true, false, W>() : ni == 2u ? kq_kernel<FMT, 1, 2, 1, true, false, W>()
           : ni == 4u ? kq_kernel<FMT, 1, 4, 1, true, false, W>()
           : ni == 8u ? kq_kernel<FMT, 1, 8, 1, true, false, W>()
                      : KqFn{};
  }
  if (pair) return KqFn{};
  if (fq == 1u)
    return ni == 1u ? kq_kernel<FMT, 1, 1, 1, false, false, W>() : ni == 2u ? kq_kernel<FMT, 1, 2, 1, false, false, W>()
           : ni == 4u ? kq_kernel<FMT, 1, 4, 1, false, false, W>()
           : ni == 8u ? kq_kernel<FMT, 1, 8, 1, false, false, W>()
                      : KqFn{};
  if (fq == 4u)
    return ni == 1u ? kq_kernel<FMT, 1, 1, 4, false, false, W>() : ni == 2u ? kq_kernel<FMT, 1, 2, 4, false, false, W>()
           : ni == 4u                                              ? kq_kernel<FMT, 1, 4, 4, false, false, W>()
                                                                   : KqFn{};
  return KqFn{};
}

KqFn kq_wide_kernel(uint32_t type_id, uint32_t fq, uint32_t ni, bool norm, bool pair) {
  return type_id == 12u ? kq_wide_kernel_fmt<12>(fq, ni, norm, pair) : kq_wide_kernel_fmt<14>(fq, ni, norm, pair);
}

// The one-token kernels with a half-wave for every block of a 17- to
// 32-block activation (768 or 1024 lanes, one block per team).
template <uint32_t NT>
KqFn kq_onepass_kernel_nt(uint32_t type_id) {
  return type_id == 12u ? kq_kernel<12, 1, 1, 4, false, false, NT, false>()
                        : kq_kernel<14, 1, 1, 4, false, false, NT, false>();
}

KqFn kq_onepass_kernel(uint32_t type_id, uint32_t nt) {
  return nt == 768u ? kq_onepass_kernel_nt<768u>(type_id) : kq_onepass_kernel_nt<1024u>(type_id);
}

// The norm-fused decode kernels: one token, four blocks per team (two for a
// single-round launch that would leave most CUs idle), the row preloaded in
// one (FQ 1) or four (FQ 4) rounds; `pair` for a gate/up job.
KqFn kq_norm_kernel(uint32_t type_id, uint32_t fq, bool pair, uint32_t ni) {
  if (ni == 8u && fq == 1u && !pair)
    return type_id == 12u ? kq_kernel<12, 1, 8, 1, true>() : kq_kernel<14, 1, 8, 1, true>();
  if (ni == 2u && fq == 1u) {
    if (pair) return type_id == 12u ? kq_kernel<12, 1, 2, 1, true, true>() : kq_kernel<14, 1, 2, 1, true, true>();
    return type_id == 12u ? kq_kernel<12, 1, 2, 1, true>() : kq_kernel<14, 1, 2, 1, true>();
  }
  if (pair) {
    if (type_id == 12u) return fq == 1u ? kq_kernel<12, 1, 4, 1, true, true>() : kq_kernel<12, 1, 4, 4, true, true>();
    return fq == 1u ? kq_kernel<14, 1, 4, 1, true, true>() : kq_kernel<14, 1, 4, 4, true, true>();
  }
  if (type_id == 12u) return fq == 1u ? kq_kernel<12, 1, 4, 1, true>() : kq_kernel<12, 1, 4, 4, true>();
  return fq == 1u ? kq_kernel<14, 1, 4, 1, true>() : kq_kernel<14, 1, 4, 4, true>();
}

template <int FMT, int T, int FQ>
KqFn kq_kernel_ni(uint32_t ni) {
  // eight blocks per team: one-token fused launches only
  if constexpr (T == 1 && FQ != 0)
    if (ni == 8u) return kq_kernel<FMT, T, 8, FQ>();
  return ni == 4u ? kq_kernel<FMT, T, 4, FQ>() : ni == 2u ? kq_kernel<FMT, T, 2, FQ>() : kq_kernel<FMT, T, 1, FQ>();
}

// fq: 0 (a separately quantized activation), 1 or 4 (fused, preload depth)
template <int T>
KqFn kq_kernel_for(uint32_t type_id, uint32_t ni, uint32_t fq) {
  if (fq == 0u) return type_id == 12u ? kq_kernel_ni<12, T, 0>(ni) : kq_kernel_ni<14, T, 0>(ni);
  if (fq == 1u) return type_id == 12u ? kq_kernel_ni<12, T, 1>(ni) : kq_kernel_ni<14, T, 1>(ni);
  return type_id == 12u ? kq_kernel_ni<12, T, 4>(ni) : kq_kernel_ni<14, T, 4>(ni);
}

// Resident workgroups per CU of one kernel at an LDS size (1 KiB buckets).
int resident_wgs_per_cu(const void* kernel, size_t lds) {
  struct Entry {
    const void* k;
    size_t bucket;
    int n;
  };
  static thread_local Entry cache[64];
  static thread_local int used = 0;
  const size_t bucket = lds / 1024u;
  for (int i = 0; i < used; i++)
    if (cache[i].k == kernel && cache[i].bucket == bucket) return cache[i].n;
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, kThreads, (bucket + 1u) * 1024u) != hipSuccess ||
      n < 1)
    n = 1;
  if (used < 64) cache[used++] = Entry{kernel, bucket, n};
  return n;
}

// The 64 teams of a workgroup cover at most 64 * NI blocks: a row of nb
// blocks needs NI >= nb / 64.
uint32_t min_blocks_per_team(uint32_t nb) {
  return nb <= 64u ? 1u : nb <= 128u ? 2u : 4u;
}

// The fused kernels take four blocks per team: measured on MI355X at the
// TinyLlama / BitNet decode shapes, NI = 4 is the fastest or within 1%
// everywhere (fewer, longer-lived workgroups amortize the quantize prologue),
// except for one-token launches of three or more workgroups per CU, which
// take eight (Q6_K 32000x2048: 12.5 us against 13.1 us).
// The others take the smallest NI that keeps every workgroup resident.
template <int T>
uint32_t choose_blocks_per_team(uint32_t type_id, uint32_t nb, uint32_t total_rows, uint32_t fq) {
  const uint32_t floor_ni = min_blocks_per_team(nb);
  if (uint32_t forced = forced_blocks_per_team()) {
    if (forced == 8u && (T != 1 || !fq)) forced = 4u;  // eight: one-token fused kernels only
    return forced > floor_ni ? forced : floor_ni;
  }
  if (fq) {
    // every workgroup quantizes the whole activation: when four blocks per
    // team would give three or more workgroups per CU (a 32000-row output
    // matrix), eight halve that repeated work; when four would leave most
    // CUs idle (64 workgroups for the 2048x2048 attention output), two
    // spread the rows over twice the workgroups
    const uint32_t r4 = rows_per_wg(type_id, nb, 4u);
    const uint32_t wgs4 = (total_rows + r4 - 1u) / r4;
    const uint32_t cus = static_cast<uint32_t>(device_cus());
    if (T == 1 && wgs4 >= 3u * cus) return 8u;
    if (T == 1 && 2u * wgs4 < cus && floor_ni <= 2u) return 2u;
    return 4u;
  }
  for (uint32_t ni : {1u, 2u, 4u}) {
    if (ni < floor_ni) continue;
    const uint32_t R = rows_per_wg(type_id, nb, ni);
    const uint32_t wgs = (total_rows + R - 1u) / R;
    const int per_cu = resident_wgs_per_cu(kq_kernel_for<T>(type_id, ni, fq).fn, lds_bytes<T>(type_id, nb, R));
    if (wgs <= static_cast<uint32_t>(per_cu * device_cus())) return ni;
  }
  return 4u;
}

// One grouped launch. FUSED: the k-quant kernels quantize x themselves
// (T <= kMaxFusedTokens); otherwise they read the activation q holds.
template <int T>
hipError_t launch_i2s_q8(GemvJobs jobs, const Q8Dev& q, size_t tokens, size_t t0, hipStream_t s, int32_t* raw);

}  // namespace

size_t units_bytes(uint32_t type_id, size_t rows, size_t nb) {
  const size_t groups = (rows * nb + 15u) / 16u;
  return groups * 16u * (type_id == 12u ? 144u : 210u);
}

namespace {

template <int T, bool FUSED>
hipError_t launch_t(uint32_t type_id, GemvJobs jobs, const Q8Dev& q, const float* x, size_t width,
                    size_t tokens, size_t t0, hipStream_t s, int32_t* raw, const NormIn* norm = nullptr) {
  uint32_t nbmax = 0, total_rows = 0;
  for (uint32_t i = 0; i < jobs.n; i++) {
    nbmax = jobs.j[i].nb > nbmax ? jobs.j[i].nb : nbmax;
    total_rows += jobs.j[i].rows;
  }
  // Rows whose blocks the input does not reach still get an output (-0.0 for
  // the k-quants, as an empty f32 sum); size everything for at least one block.
  const uint32_t nbl = nbmax ? nbmax : 1u;
  const bool kquant = type_id == 12u || type_id == 14u;
  // fused: preload every block of a one-round activation, else 4 per half-wave
  uint32_t fq = 0u;
  if (FUSED) {
    const size_t nq = width / 256u < nbmax ? width / 256u : nbmax;
    fq = static_cast<size_t>(T) * nq <= kThreads / 32u ? 1u : 4u;
  }
  uint32_t ni = norm ? 4u : kquant ? choose_blocks_per_team<T>(type_id, nbl, total_rows, fq) : 1u;
  // a norm-fused launch of fewer workgroups than half the CUs (Q/K/V: 80)
  // takes two blocks per team, as choose_blocks_per_team does for the others
  const bool pair_job = jobs.n == 1u && jobs.j[0].w2 != nullptr;
  if (norm && T == 1 && fq == 1u && !pair_job && min_blocks_per_team(nbl) <= 2u) {
    const uint32_t r4 = rows_per_wg(type_id, nbl, 4u);
    uint32_t wgs4 = 0;
    for (uint32_t i = 0; i < jobs.n; i++) wgs4 += (jobs.j[i].rows + r4 - 1u) / r4;
    if (2u * wgs4 < static_cast<uint32_t>(device_cus())) ni = 2u;
    // an output-sized launch (32000 rows: 1000 workgroups at four) takes
    // eight, so the grid fits on the chip at once
    if (wgs4 >= 3u * static_cast<uint32_t>(device_cus())) ni = 8u;
  }
  // Tuning::norm_ni forces the norm-fused one-token launches, for tuning
  if (const int v = tuning().norm_ni)
    if (norm && T == 1 && fq == 1u && min_blocks_per_team(nbl) <= 2u) ni = static_cast<uint32_t>(v);
  // A one-round launch of eight blocks per team (an output-sized matrix)
  // takes 512 lanes and twice the rows per workgroup when that still gives
  // 15/16 of the CUs a workgroup: half the activation quantizations (32000x2048
  // Q6_K: 250 workgroups, 12.03-12.22 against 12.33-12.58 us). The
  // norm-fused output launch of the decoder keeps 256 (1-2 us a token
  // slower at 512). Tuning::kq_nt and Tuning::norm_nt force it (512) or keep
  // 256.
  bool wide8 = false;
  if (T == 1 && FUSED && fq == 1u && ni == 8u && !pair_job) {
    const uint32_t r8 = rows_per_wg(type_id, nbl, 16u);
    uint32_t w8 = 0;
    for (uint32_t i = 0; i < jobs.n; i++) w8 += (jobs.j[i].rows + r8 - 1u) / r8;
    const int forced = norm ? tuning().norm_nt : tuning().kq_nt;
    wide8 = forced ? forced == 512 : !norm && 16u * w8 >= 15u * static_cast<uint32_t>(device_cus());
  }
  uint32_t R = rows_per_wg(type_id, nbl, wide8 ? 16u : ni);
  // A one-token grid of between one and two workgroups per CU leaves some
  // CUs twice the rows of others and repeats the activation prologue once
  // per workgroup: it takes one workgroup per CU instead, 512 lanes and the
  // blocks per team that hold its rows (the gate/up pair: 256 workgroups of
  // 22 + 22 rows at four blocks a team, 8.36 against 9.57 us). Grids below
  // one workgroup per CU keep their shape (more workgroups measured slower:
  // Q/K/V 7.52 against 6.57 us), and so do the eight-block output launches
  // (the rule above). Tuning::kq_balance = false keeps every grid, and so
  // does a forced 256-lane shape (Tuning::kq_nt, Tuning::norm_nt).
  bool balanced = false;
  if (T == 1 && FUSED && kquant && !wide8 && ni < 8u && tuning().kq_balance &&
      (norm ? tuning().norm_nt : tuning().kq_nt) != 256) {
    const uint32_t cus = static_cast<uint32_t>(device_cus());
    const uint32_t per0 = pair_job ? R / 2u : R;
    uint32_t wcur = 0;
    for (uint32_t i = 0; i < jobs.n; i++) wcur += (jobs.j[i].rows + per0 - 1u) / per0;
    if (per0 > 0u && wcur > cus && wcur < 2u * cus) {
      const uint32_t rows_main = pair_job ? jobs.j[0].rows : total_rows;
      const uint32_t per = (rows_main + cus - 1u) / cus;
      const uint32_t R2 = pair_job ? 2u * per : per;
      const uint32_t need = (R2 * nbl + 2u * kThreads / 4u - 1u) / (2u * kThreads / 4u);
      const uint32_t nib = need <= 1u ? 1u : need <= 2u ? 2u : need <= 4u ? 4u : need <= 8u ? 8u : 0u;
      if (nib && (!pair_job || R2 >= 2u) && kq_wide_kernel(type_id, fq, nib, norm != nullptr, pair_job)) {
        R = R2;
        ni = nib;
        balanced = true;
      }
    }
  }
  // A one-token row of 17 to 32 blocks (5632 or 8192 values) leaves a
  // 512-lane workgroup's 16 half-waves a second round of quantization, which
  // every wave then waits for at the barrier: 768 lanes (up to 24 blocks)
  // or 1024 (up to 32) quantize it in one round, with one block a team, when
  // that grid still fits one workgroup per CU (2048x5632: Q6_K 5.45 against
  // 6.37 us, Q4_K 4.85 against 5.32; Q4_K 2048x8192 at 1024 lanes: 5.95
  // against 7.1). Larger grids measured slower (4096x5632: 6.7 against 6.1
  // us) and keep their shape. Tuning::kq_onepass = false keeps every grid.
  uint32_t onepass_nt = 0u;
  if (T == 1 && FUSED && kquant && !norm && !pair_job && fq == 4u && nbl > 16u && nbl <= 32u &&
      tuning().kq_onepass) {
    const uint32_t nt1 = onepass_lanes(nbl);
    const uint32_t r1 = (nt1 / 4u) / nbl;
    uint32_t w1 = 0;
    for (uint32_t i = 0; i < jobs.n; i++) w1 += (jobs.j[i].rows + r1 - 1u) / r1;
    if (w1 <= static_cast<uint32_t>(device_cus())) {
      onepass_nt = nt1;
      R = r1;
      ni = 1u;
      balanced = false;
    }
  }
  // a gate/up pair: one norm-fused job, R/2 rows of each matrix per workgroup
  const bool pair = jobs.n == 1u && jobs.j[0].w2 != nullptr;
  if (pair && (!norm || !kquant || R < 2u)) return hipErrorInvalidValue;
  const uint32_t per = pair ? R / 2u : R;
  uint32_t wgs = 0;
  for (uint32_t i = 0; i < jobs.n; i++) {
    if (i > 0 && jobs.j[i].w2) return hipErrorInvalidValue;
    jobs.j[i].wg_begin = wgs;
    wgs += (jobs.j[i].rows + per - 1u) / per;
  }
  if (wgs == 0) return hipSuccess;
  // one k-quant matrix whose rows tile a grid of at least one workgroup per
  // CU exactly: interleave its workgroups over chunks of one iteration's rows
  // (64 teams / nb blocks). Smaller grids measured no gain.
  jobs.j[0].il = 0u;
  if (kquant && jobs.n == 1u && !pair && nbl <= 64u && 64u % nbl == 0u && jobs.j[0].rows == wgs * per &&
      (wgs >= static_cast<uint32_t>(device_cus()) || wide8) && interleave_rows()) {
    const uint32_t c = 64u / nbl;
    if (per % c == 0u) jobs.j[0].il = static_cast<uint32_t>(__builtin_ctz(c)) + 1u;
  }
  if (type_id == 0u) {
    hipLaunchKernelGGL(gemv_dense_kernel<T>, dim3(wgs), dim3(kThreads), 0, s, jobs, x, width, R,
                       tokens, t0);
    return hipGetLastError();
  }
  size_t lds = lds_bytes<T>(type_id, nbl, R);
  if (kquant) {
    // the fused kernels quantize blocks [0, nbmax) of x, which width covers
    const float* xin = FUSED ? x : nullptr;
    NormIn nrm{};
    KqFn k;
    if (norm) {
      // the squares of the row (and the rms) after the kernel's own LDS
      nrm = *norm;
      nrm.lds_offset = static_cast<uint32_t>((lds + 15u) / 16u * 16u);
      lds = nrm.lds_offset + static_cast<size_t>(wave_sum_floats(nbl * 256u)) * 4u + 16u;
      k = kq_norm_kernel(type_id, fq, pair, ni);
    } else {
      k = kq_kernel_for<T>(type_id, ni, fq);
    }
    // A one-token grid of fewer workgroups than CUs takes 512 lanes and half
    // the blocks per team: the same rows and the same one quantization per
    // workgroup, twice the waves to cover the weight loads' latency (Q6_K
    // 2048x5632: 6.6-6.75 against 7.45 us; Q4_K 5632x2048: 4.9 against 5.1).
    // The 500-workgroup 32000x2048 output launch keeps 256 (12.3 against
    // 12.9). Tuning::kq_nt and Tuning::norm_nt force it.
    uint32_t nt = kThreads, nit = ni;
    if (onepass_nt) {
      // each workgroup's rows are whole groups of 16 blocks where R * nb is a
      // multiple of 16 (2048x5632 takes 8 rows of 22 blocks, 11 groups), so
      // each load instruction of a wave reads consecutive bytes
      k = kq_onepass_kernel(type_id, onepass_nt);
      nt = onepass_nt;
    } else if (balanced) {
      k = kq_wide_kernel(type_id, fq, ni, norm != nullptr, pair);
      nt = 2u * kThreads;
    } else if (wide8) {
      if (const KqFn kw = kq_wide_kernel(type_id, fq, 8u, norm != nullptr, pair)) {
        k = kw;
        nt = 2u * kThreads;
      } else {
        return hipErrorNotSupported;  // every one-round eight-block form is built
      }
    } else if (T == 1 && FUSED && ni >= 2u) {
      const int forced = norm ? tuning().norm_nt : tuning().kq_nt;
      const bool wide = forced ? forced == 512 : wgs < static_cast<uint32_t>(device_cus());
      const KqFn kw = wide ? kq_wide_kernel(type_id, fq, ni / 2u, norm != nullptr, pair) : KqFn{};
      if (kw) {
        k = kw;
        nt = 2u * kThreads;
        nit = ni / 2u;
      }
    }
    // One token, one preload round, and every job's blocks a power of two
    // no larger than the teams covering whole rows, with every wave's rows
    // starting a group of 16 blocks: the fixed-column walk (BlockWalk).
    // Tuning::kq_fix = false keeps the general walk.
    if (!onepass_nt && T == 1 && FUSED && fq == 1u && tuning().kq_fix) {
      bool fix = true;
      for (uint32_t i = 0; i < jobs.n; i++) {
        const GemvJob& j = jobs.j[i];
        const uint32_t b = j.nb;
        fix = fix && b != 0u && (b & (b - 1u)) == 0u && b <= nt / 4u && b == j.ub;
        // rows per group of 16 blocks; a workgroup's first row, and an
        // interleave chunk, must be whole groups
        const uint32_t rpu = b != 0u && b < 16u ? 16u / b : 1u;
        fix = fix && (j.il ? (1u << (j.il - 1u)) % rpu == 0u : per % rpu == 0u);
        // a pair's up rows start at workgroup row nh = min(per, rows - row0):
        // the last workgroup's nh is whole groups only when rows is
        fix = fix && (!pair || j.rows % rpu == 0u);
      }
      const KqFn kf = fix ? kq_fix_kernel(type_id, nit, norm != nullptr, pair, nt) : KqFn{};
      if (kf) k = kf;
    }
    if (!k) return hipErrorNotSupported;
    // the argument order of the kernel chosen (KqFn::preload)
    void* args_jobs[] = {&jobs, const_cast<Q8Dev*>(&q), &xin, &width, const_cast<uint32_t*>(&R),
                         const_cast<uint32_t*>(&nbl), &tokens, &t0, &nrm};
    void* args_pl[] = {&xin, &width, const_cast<uint32_t*>(&R), const_cast<uint32_t*>(&nbl), &tokens, &t0,
                       &jobs, const_cast<Q8Dev*>(&q), &nrm};
    if (norm && norm->grid_out) *norm->grid_out = wgs;
    return hipLaunchKernel(k.fn, dim3(wgs), dim3(nt), k.preload ? args_pl : args_jobs, lds, s);
  }
  if (tuning().i2s_one) {
    const hipError_t e = launch_i2s_q8<T>(jobs, q, tokens, t0, s, raw);
    if (e != hipErrorNotSupported) return e;
  }
  hipLaunchKernelGGL(gemv_i2s_kernel<T>, dim3(wgs), dim3(kThreads), lds, s, jobs, q, R, nbl, tokens, t0, raw);
  return hipGetLastError();
}

}  // namespace

size_t gemv_max_tokens(uint32_t type_id, uint32_t nb) {
  // LDS per workgroup stays within 64 KiB at the largest tile (NI = 4)
  const uint32_t nbl = nb ? nb : 1u;
  if ((type_id == 12u || type_id == 14u) && nbl > 4u * (kThreads / 4u)) return 0;
  const uint32_t R = rows_per_wg(type_id, nbl, 4u);
  size_t t = kMaxTokens;
  while (t > 1) {
    size_t need = 0;
    switch (t) {
      case 8: need = lds_bytes<8>(type_id, nbl, R); break;
      case 7: need = lds_bytes<7>(type_id, nbl, R); break;
      case 6: need = lds_bytes<6>(type_id, nbl, R); break;
      case 5: need = lds_bytes<5>(type_id, nbl, R); break;
      case 4: need = lds_bytes<4>(type_id, nbl, R); break;
      case 3: need = lds_bytes<3>(type_id, nbl, R); break;
      default: need = lds_bytes<2>(type_id, nbl, R); break;
    }
    if (need <= 64u * 1024u) break;
    t--;
  }
  return lds_bytes<1>(type_id, nbl, R) <= 64u * 1024u ? t : 0;
}

hipError_t launch_gemv(uint32_t type_id, const GemvJobs& jobs, const Q8Dev& q, const float* x,
                       size_t width, size_t tokens, size_t t0, size_t tn, hipStream_t s,
                       int32_t* raw) {
  switch (tn) {
    case 1: return launch_t<1, false>(type_id, jobs, q, x, width, tokens, t0, s, raw);
    case 2: return launch_t<2, false>(type_id, jobs, q, x, width, tokens, t0, s, raw);
    case 3: return launch_t<3, false>(type_id, jobs, q, x, width, tokens, t0, s, raw);
    case 4: return launch_t<4, false>(type_id, jobs, q, x, width, tokens, t0, s, raw);
    case 5: return launch_t<5, false>(type_id, jobs, q, x, width, tokens, t0, s, raw);
    case 6: return launch_t<6, false>(type_id, jobs, q, x, width, tokens, t0, s, raw);
    case 7: return launch_t<7, false>(type_id, jobs, q, x, width, tokens, t0, s, raw);
    case 8: return launch_t<8, false>(type_id, jobs, q, x, width, tokens, t0, s, raw);
    default: return hipErrorInvalidValue;
  }
}

bool gemv_fused_ok(uint32_t type_id, size_t width, size_t tn) {
  if (type_id == 12u || type_id == 14u) return tn >= 1 && tn <= kMaxFusedTokens;
  if (type_id == 36u) return tn >= 1 && tn <= 2 && width / 32u * 32u <= 4u * kThreads * kFusedRowPasses;
  return false;
}

namespace {

constexpr uint32_t kI2sMinWgs = 256;  // one per CU

template <int T>
hipError_t launch_i2s_fused(GemvJobs jobs, const float* x, size_t width, size_t tokens, size_t t0,
                            hipStream_t s, int32_t* raw) {
  uint32_t nbmax = 0;
  for (uint32_t i = 0; i < jobs.n; i++) nbmax = jobs.j[i].nb > nbmax ? jobs.j[i].nb : nbmax;
  const uint32_t nbl = nbmax ? nbmax : 1u;
  const uint32_t nq = static_cast<uint32_t>(width / 32u);
  // two chunks per lane at most: nbl <= 64 (8192 values) gives lpr <= 64
  const uint32_t nchunk = 2u * nbl;
  uint32_t lpr = 8u;
  while (lpr < 64u && 2u * lpr < nchunk) lpr <<= 1;
  const uint32_t cpl = (nchunk + lpr - 1u) / lpr;
  if (cpl > 2u) return hipErrorInvalidValue;
  const uint32_t R = kThreads / lpr;
  // G row groups per workgroup: the most that still leave at least
  // kI2sMinWgs workgroups (each repeats the activation's quantization);
  // Tuning::i2s_groups forces it, for tuning
  auto count = [&](uint32_t g) {
    uint32_t n = 0;
    for (uint32_t i = 0; i < jobs.n; i++) n += (jobs.j[i].rows + R * g - 1u) / (R * g);
    return n;
  };
  uint32_t G = 1;
  while (G < 4u && count(2u * G) >= kI2sMinWgs) G *= 2u;
  if (const int v = tuning().i2s_groups) G = static_cast<uint32_t>(v);
  uint32_t wgs = 0;
  for (uint32_t i = 0; i < jobs.n; i++) {
    jobs.j[i].wg_begin = wgs;
    wgs += (jobs.j[i].rows + R * G - 1u) / (R * G);
  }
  if (wgs == 0) return hipSuccess;
  const size_t lds = T * nbl * 128u + T * nbl * 16u + T * 4u + 4u * (kThreads / 64u) * 4u;
  void* k;
  if (cpl == 1u)
    k = G == 4u ? reinterpret_cast<void*>(gemv_i2s_fused_kernel<T, 1, 4>)
      : G == 2u ? reinterpret_cast<void*>(gemv_i2s_fused_kernel<T, 1, 2>)
                : reinterpret_cast<void*>(gemv_i2s_fused_kernel<T, 1, 1>);
  else
    k = G == 4u ? reinterpret_cast<void*>(gemv_i2s_fused_kernel<T, 2, 4>)
      : G == 2u ? reinterpret_cast<void*>(gemv_i2s_fused_kernel<T, 2, 2>)
                : reinterpret_cast<void*>(gemv_i2s_fused_kernel<T, 2, 1>);
  void* args[] = {&jobs, const_cast<float**>(&x), &width, const_cast<uint32_t*>(&nq), const_cast<uint32_t*>(&nbl),
                  &lpr, &tokens, &t0, &raw};
  return hipLaunchKernel(k, dim3(wgs), dim3(kThreads), args, lds, s);
}

template <uint32_t NT, int LPR, int CPL>
void* i2s_one_kernel(bool one_job) {
  return one_job ? reinterpret_cast<void*>(gemv_i2s_one_kernel<NT, LPR, CPL, true>)
                 : reinterpret_cast<void*>(gemv_i2s_one_kernel<NT, LPR, CPL, false>);
}

// The kernels built: 256 threads at every team width with 1-8 chunks a lane;
// 512 threads at 16-64 lanes with 1-4 chunks; 1024 at 32-64 lanes with 1-2
// (a row of at most 128 chunks never needs more at those widths).
template <uint32_t NT, int LPR>
void* i2s_one_pick(uint32_t cpl, bool one_job) {
  constexpr uint32_t kMaxCpl = NT == 256u ? 8u : NT == 512u ? 4u : 2u;
  if (cpl == 0u || cpl > kMaxCpl) return nullptr;
  if constexpr (NT == 256u) {
    switch (cpl) {
      case 1: return i2s_one_kernel<NT, LPR, 1>(one_job);
      case 2: return i2s_one_kernel<NT, LPR, 2>(one_job);
      case 3: return i2s_one_kernel<NT, LPR, 3>(one_job);
      case 4: return i2s_one_kernel<NT, LPR, 4>(one_job);
      case 5: return i2s_one_kernel<NT, LPR, 5>(one_job);
      case 6: return i2s_one_kernel<NT, LPR, 6>(one_job);
      case 7: return i2s_one_kernel<NT, LPR, 7>(one_job);
      default: return i2s_one_kernel<NT, LPR, 8>(one_job);
    }
  } else if constexpr (NT == 512u) {
    switch (cpl) {
      case 1: return i2s_one_kernel<NT, LPR, 1>(one_job);
      case 2: return i2s_one_kernel<NT, LPR, 2>(one_job);
      case 3: return i2s_one_kernel<NT, LPR, 3>(one_job);
      default: return i2s_one_kernel<NT, LPR, 4>(one_job);
    }
  } else {
    return cpl == 1u ? i2s_one_kernel<NT, LPR, 1>(one_job) : i2s_one_kernel<NT, LPR, 2>(one_job);
  }
}

void* i2s_one_for(uint32_t nt, uint32_t lpr, uint32_t cpl, bool one_job) {
  if (nt == 256u)
    return lpr == 8u ? i2s_one_pick<256, 8>(cpl, one_job) : lpr == 16u ? i2s_one_pick<256, 16>(cpl, one_job)
         : lpr == 32u ? i2s_one_pick<256, 32>(cpl, one_job) : i2s_one_pick<256, 64>(cpl, one_job);
  if (nt == 512u)
    return lpr == 16u ? i2s_one_pick<512, 16>(cpl, one_job) : lpr == 32u ? i2s_one_pick<512, 32>(cpl, one_job)
         : lpr == 64u ? i2s_one_pick<512, 64>(cpl, one_job) : nullptr;
  if (nt == 1024u)
    return lpr == 32u ? i2s_one_pick<1024, 32>(cpl, one_job) : lpr == 64u ? i2s_one_pick<1024, 64>(cpl, one_job)
                      : nullptr;
  return nullptr;
}

// One token of I2_S on gemv_i2s_one_kernel; hipErrorNotSupported for shapes
// it does not take (the two-token kernel serves those).
hipError_t launch_i2s_one(GemvJobs jobs, const float* x, size_t width, size_t tokens, size_t t0, hipStream_t s,
                          int32_t* raw) {
  uint32_t nbmax = 0, nbmin = ~0u;
  for (uint32_t i = 0; i < jobs.n; i++) {
    nbmax = jobs.j[i].nb > nbmax ? jobs.j[i].nb : nbmax;
    nbmin = jobs.j[i].nb < nbmin ? jobs.j[i].nb : nbmin;
  }
  const uint32_t n = static_cast<uint32_t>(width / 32u) * 32u;
  if (jobs.n == 0 || nbmin == 0 || n < 32u || n > 4u * kThreads * kFusedRowPasses) return hipErrorNotSupported;
  const uint32_t nchunk = 2u * nbmax;
  // lanes per row at 256 threads: the fewest that hold a row in at most 8
  // chunks each. Each workgroup repeats the activation's quantization, so
  // fewer and fuller workgroups win even below one per CU (6912x2560: 216
  // workgroups of 32 rows beat 432 of 16; 2560x6912: 160 of 16 beat 320 of
  // 8). Wider workgroups keep the rows a workgroup takes and give each lane
  // a smaller share of the quantization and of the row.
  // tuning().i2s_nt and tuning().i2s_lpr force them.
  uint32_t lpr = 8;
  while (lpr < 64u && (nchunk + lpr - 1u) / lpr > 8u) lpr *= 2u;
  // 512 threads for rows of more than 4096 values (2560x6912: 5.8 against
  // 6.2-6.4 us; 6912x2560 keeps 256: 4.3-4.9 against 5.1)
  uint32_t nt = tuning().i2s_nt ? static_cast<uint32_t>(tuning().i2s_nt) : n > 4096u ? 512u : 256u;
  lpr = lpr * (nt / 256u) > 64u ? 64u : lpr * (nt / 256u);
  if (const int v = tuning().i2s_lpr) lpr = static_cast<uint32_t>(v);
  const uint32_t cpl = (nchunk + lpr - 1u) / lpr;
  void* k = i2s_one_for(nt, lpr, cpl, jobs.n == 1u);
  if (!k) return hipErrorNotSupported;
  const uint32_t R = nt / lpr;
  uint32_t wgs = 0;
  for (uint32_t i = 0; i < jobs.n; i++) {
    jobs.j[i].wg_begin = wgs;
    wgs += (jobs.j[i].rows + R - 1u) / R;
  }
  if (wgs == 0) return hipSuccess;
  uint32_t nkeep = nbmax * 128u;
  const size_t lds = nkeep + 4u * (4u + 1u) * (nt / 64u);
  const float* xt = x + t0 * width;
  void* args[] = {&jobs, const_cast<float**>(&xt), const_cast<uint32_t*>(&n), &nkeep, &tokens, &t0, &raw};
  return hipLaunchKernel(k, dim3(wgs), dim3(nt), args, lds, s);
}

template <int T, int LPR>
void* i2s_q8_pick(uint32_t cpl) {
  if constexpr (T == 1) {
    switch (cpl) {
      case 1: return reinterpret_cast<void*>(gemv_i2s_q8_kernel<1, LPR, 1>);
      case 2: return reinterpret_cast<void*>(gemv_i2s_q8_kernel<1, LPR, 2>);
      case 3: return reinterpret_cast<void*>(gemv_i2s_q8_kernel<1, LPR, 3>);
      case 4: return reinterpret_cast<void*>(gemv_i2s_q8_kernel<1, LPR, 4>);
      case 5: return reinterpret_cast<void*>(gemv_i2s_q8_kernel<1, LPR, 5>);
      case 6: return reinterpret_cast<void*>(gemv_i2s_q8_kernel<1, LPR, 6>);
      case 7: return reinterpret_cast<void*>(gemv_i2s_q8_kernel<1, LPR, 7>);
      case 8: return reinterpret_cast<void*>(gemv_i2s_q8_kernel<1, LPR, 8>);
      default: return nullptr;
    }
  } else {
    // only the forms whose registers hold their chunks (no scratch): four
    // chunks a lane up to seven tokens, eight up to three; gemv_i2s_kernel
    // takes the rest
    if (cpl <= 4u) {
      if constexpr (T <= 7) return reinterpret_cast<void*>(gemv_i2s_q8_kernel<T, LPR, 4>);
      return nullptr;
    }
    if (cpl <= 8u) {
      if constexpr (T <= 3) return reinterpret_cast<void*>(gemv_i2s_q8_kernel<T, LPR, 8>);
      return nullptr;
    }
    return nullptr;
  }
}

// T tokens of I2_S against a pre-quantized activation on gemv_i2s_q8_kernel;
// hipErrorNotSupported for shapes it does not take.
template <int T>
hipError_t launch_i2s_q8(GemvJobs jobs, const Q8Dev& q, size_t tokens, size_t t0, hipStream_t s, int32_t* raw) {
  uint32_t nbmax = 0, nbmin = ~0u;
  for (uint32_t i = 0; i < jobs.n; i++) {
    nbmax = jobs.j[i].nb > nbmax ? jobs.j[i].nb : nbmax;
    nbmin = jobs.j[i].nb < nbmin ? jobs.j[i].nb : nbmin;
  }
  if (jobs.n == 0 || nbmin == 0 || nbmax > 64u) return hipErrorNotSupported;
  // 32-bit activation offsets (the launchers keep tokens * qstride below 2^32)
  if ((t0 + T) * q.qstride > 0xffffffffu || (t0 + T) * q.bstride > 0xffffffffu) return hipErrorNotSupported;
  const uint32_t nchunk = 2u * nbmax;
  uint32_t lpr = 8;
  while (lpr < 64u && (nchunk + lpr - 1u) / lpr > 8u) lpr *= 2u;
  if (const int v = tuning().i2s_lpr) lpr = static_cast<uint32_t>(v);
  const uint32_t cpl = (nchunk + lpr - 1u) / lpr;
  void* k = lpr == 8u ? i2s_q8_pick<T, 8>(cpl) : lpr == 16u ? i2s_q8_pick<T, 16>(cpl)
          : lpr == 32u ? i2s_q8_pick<T, 32>(cpl) : i2s_q8_pick<T, 64>(cpl);
  if (!k) return hipErrorNotSupported;
  const uint32_t R = kThreads / lpr;
  uint32_t wgs = 0;
  for (uint32_t i = 0; i < jobs.n; i++) {
    jobs.j[i].wg_begin = wgs;
    wgs += (jobs.j[i].rows + R - 1u) / R;
  }
  if (wgs == 0) return hipSuccess;
  uint32_t nkeep = nbmax * 128u;
  const size_t lds = static_cast<size_t>(T) * nkeep + static_cast<size_t>(T) * 4u * (kThreads / 64u);
  void* args[] = {&jobs, const_cast<Q8Dev*>(&q), &nkeep, &tokens, &t0, &raw};
  return hipLaunchKernel(k, dim3(wgs), dim3(kThreads), args, lds, s);
}

}  // namespace

bool norm_fusable(uint32_t type_id, size_t width, uint32_t nbmax) {
  // the whole row in the preload: every block of x quantized, at most four
  // rounds of eight half-waves
  return (type_id == 12u || type_id == 14u) && width % 256u == 0 && width / 256u == nbmax && nbmax >= 1u &&
         nbmax <= 4u * (kThreads / 32u);
}

hipError_t launch_gemv_fused(uint32_t type_id, const GemvJobs& jobs, const float* x, size_t width,
                             size_t tokens, size_t t0, size_t tn, hipStream_t s, int32_t* raw, const NormIn* norm) {
  if (!gemv_fused_ok(type_id, width, tn)) return hipErrorInvalidValue;
  if (norm) {
    uint32_t nbmax = 0;
    for (uint32_t i = 0; i < jobs.n; i++) nbmax = jobs.j[i].nb > nbmax ? jobs.j[i].nb : nbmax;
    if (tn != 1 || tokens != 1 || !norm_fusable(type_id, width, nbmax)) return hipErrorInvalidValue;
    const Q8Dev none{};
    return launch_t<1, true>(type_id, jobs, none, x, width, tokens, t0, s, nullptr, norm);
  }
  if (type_id == 36u) {
    if (tn == 1 && tuning().i2s_one) {
      const hipError_t e = launch_i2s_one(jobs, x, width, tokens, t0, s, raw);
      if (e != hipErrorNotSupported) return e;
    }
    return tn == 1 ? launch_i2s_fused<1>(jobs, x, width, tokens, t0, s, raw)
                   : launch_i2s_fused<2>(jobs, x, width, tokens, t0, s, raw);
  }
  const Q8Dev none{};
  switch (tn) {
    case 1: return launch_t<1, true>(type_id, jobs, none, x, width, tokens, t0, s, nullptr);
    case 2: return launch_t<2, true>(type_id, jobs, none, x, width, tokens, t0, s, nullptr);
    case 3: return launch_t<3, true>(type_id, jobs, none, x, width, tokens, t0, s, nullptr);
    case 4: return launch_t<4, true>(type_id, jobs, none, x, width, tokens, t0, s, nullptr);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_dequantize_row(uint32_t type_id, const uint8_t* mat, size_t pitch, uint32_t row, uint32_t nb,
                                 float scale, float* out, size_t out_len, hipStream_t s) {
  const size_t n = static_cast<size_t>(nb) * (type_id == 36u ? 128u : 256u);
  const size_t m = n < out_len ? n : out_len;
  if (m == 0) return hipSuccess;
  const uint32_t grid = static_cast<uint32_t>((m + kThreads - 1) / kThreads);
  hipLaunchKernelGGL(dequantize_row_kernel, dim3(grid < 1024u ? grid : 1024u), dim3(kThreads), 0, s,
                     type_id, mat, pitch, row, nb, scale, out, out_len);
  return hipGetLastError();
}

}  // namespace rh
