// rh_device.h -- device helpers shared by the gfx950 kernels.
//
// Every kernel here is built with -ffp-contract=off: a float expression is
// evaluated one IEEE operation at a time, and fused multiply-adds appear only
// where the source calls fmaf(), matching the places rusticide's CPU path calls
// mul_add. Division uses __fdiv_rn (correctly rounded), never a reciprocal.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace rh {

// 16 bytes loaded with a 4-byte alignment guarantee only: LLVM lowers this to
// one global_load_dwordx4, which needs dword alignment.
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
// A native 4-float vector. HIP's float4 is a struct whose copies become
// memcpy, which keeps register arrays of it in scratch when they live across
// branches; arrays of this type stay in registers.
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ u32x4 load16(const uint8_t* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

// A 16-byte load marked nontemporal, for weights a decode GEMV reads once per
// launch in whole consecutive lines (the unit layout; I2_S rows). The lm_head
// GEMV measured 10.4-10.6 against 11.0-11.2 us with it, a 22-layer decode
// 630-634 against 676 us per token.
__device__ __forceinline__ u32x4 load16_nt(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

__device__ __forceinline__ u32x4 load16_a4(const uint8_t* p) {
  u32x4_a4 v = *reinterpret_cast<const u32x4_a4*>(p);
  return u32x4{v.x, v.y, v.z, v.w};
}

__device__ __forceinline__ uint32_t load4(const uint8_t* p) {
  return *reinterpret_cast<const uint32_t*>(p);
}

// 16 and 8 bytes at any byte address: the HSA ABI runs global memory in
// unaligned-access mode, and LLVM lowers these to one global_load_dwordx4 /
// global_load_dwordx2 each.
__device__ __forceinline__ u32x4 load16_any(const uint8_t* p) {
  u32x4 v;
  __builtin_memcpy(&v, p, 16);
  return v;
}
__device__ __forceinline__ uint2 load8_any(const uint8_t* p) {
  uint2 v;
  __builtin_memcpy(&v, p, 8);
  return v;
}

// The 16 bytes at p, where p is only 2-byte aligned: five aligned dwords
// funnel-shifted by (p & 3) bytes. Reads up to 4 bytes past p + 16.
__device__ __forceinline__ u32x4 load16_unaligned(const uint8_t* p) {
  const uint32_t sh = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p) & 3u);
  const uint8_t* base = p - sh;
  u32x4 v = load16_a4(base);
  uint32_t e = load4(base + 16);
  return u32x4{__builtin_amdgcn_alignbyte(v.y, v.x, sh), __builtin_amdgcn_alignbyte(v.z, v.y, sh),
               __builtin_amdgcn_alignbyte(v.w, v.z, sh), __builtin_amdgcn_alignbyte(e, v.w, sh)};
}

// Exact IEEE half -> float widening (v_cvt_f32_f16).
__device__ __forceinline__ float f16_lo(uint32_t w) {
  _Float16 h;
  uint16_t b = static_cast<uint16_t>(w & 0xffffu);
  __builtin_memcpy(&h, &b, 2);
  return static_cast<float>(h);
}
__device__ __forceinline__ float f16_hi(uint32_t w) { return f16_lo(w >> 16); }

// Four signed byte products accumulated into c (v_dot4_i32_i8, no clamp).
__device__ __forceinline__ int32_t dot4(uint32_t a, uint32_t b, int32_t c) {
  return __builtin_amdgcn_sdot4(static_cast<int32_t>(a), static_cast<int32_t>(b), c, false);
}

__device__ __forceinline__ uint32_t bfe(uint32_t v, uint32_t off, uint32_t width) {
  return __builtin_amdgcn_ubfe(v, off, width);
}

// Sum over the 4 lanes of a quad (DPP quad_perm); exact for integers.
__device__ __forceinline__ int32_t quad_sum(int32_t v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
  v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
  return v;
}

// One DPP lane permutation of v (every source lane is valid for the
// patterns used here: quad_perm, row_half_mirror, row_mirror).
template <int CTRL>
__device__ __forceinline__ uint32_t dpp(uint32_t v) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(static_cast<int>(v), static_cast<int>(v), CTRL, 0xF, 0xF, false));
}

// Maximum / minimum over each aligned group of 32 lanes, left in every lane:
// xor 1 and 2 (quad_perm), the 8-lane and 16-lane mirrors, then xor 16
// (ds_swizzle in bit mode). Unsigned; non-negative floats compare as their bits.
__device__ __forceinline__ uint32_t half_max_u32(uint32_t v) {
  v = max(v, dpp<0xB1>(v));
  v = max(v, dpp<0x4E>(v));
  v = max(v, dpp<0x141>(v));
  v = max(v, dpp<0x140>(v));
  return max(v, static_cast<uint32_t>(__builtin_amdgcn_ds_swizzle(static_cast<int>(v), 0x401F)));
}
__device__ __forceinline__ uint32_t half_min_u32(uint32_t v) {
  v = min(v, dpp<0xB1>(v));
  v = min(v, dpp<0x4E>(v));
  v = min(v, dpp<0x141>(v));
  v = min(v, dpp<0x140>(v));
  return min(v, static_cast<uint32_t>(__builtin_amdgcn_ds_swizzle(static_cast<int>(v), 0x401F)));
}
__device__ __forceinline__ int32_t half_max_i32(int32_t v) {
  v = max(v, static_cast<int32_t>(dpp<0xB1>(static_cast<uint32_t>(v))));
  v = max(v, static_cast<int32_t>(dpp<0x4E>(static_cast<uint32_t>(v))));
  v = max(v, static_cast<int32_t>(dpp<0x141>(static_cast<uint32_t>(v))));
  v = max(v, static_cast<int32_t>(dpp<0x140>(static_cast<uint32_t>(v))));
  return max(v, __builtin_amdgcn_ds_swizzle(v, 0x401F));
}

// Sum over aligned groups of 8 lanes; exact (wrapping) for integers.
__device__ __forceinline__ uint32_t octet_sum(uint32_t v) {
  v += static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), 1, 64));
  v += static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), 2, 64));
  v += static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), 4, 64));
  return v;
}

// Q8Kind::SuperBlock round_to_i8 (portable/q8.rs:114-116): ties to even,
// clamp to +-127, NaN to 0.
__device__ __forceinline__ int32_t round_to_i8(float v) {
  float r = __builtin_rintf(v);
  if (r != r) return 0;
  r = r < -127.0f ? -127.0f : r;
  r = r > 127.0f ? 127.0f : r;
  return static_cast<int32_t>(r);
}

// Q8Kind::Row round_row_to_i8 (portable/q8.rs:128-130): ties to even, then a
// saturating cast to [-128, 127] with NaN to 0.
__device__ __forceinline__ int32_t round_row_to_i8(float v) {
  const float r = __builtin_rintf(v);
  const float c = __builtin_fminf(__builtin_fmaxf(r, -128.0f), 127.0f);  // NaN r gives -128 here
  return r != r ? 0 : static_cast<int32_t>(c);
}

// ((s + p[0]) + p[1]) + ... on one lane, from 16-byte aligned LDS. The sum is
// a chain of dependent adds; each batch of 28 values is loaded while the
// previous batch is added (the scheduling barriers keep the compiler from
// sinking the loads below the adds), so LDS latency does not stall the chain.
// Two batches in flight stay under the 15 outstanding LDS reads a wait can
// name, so the adds wait for their own batch only.
constexpr uint32_t kSumBatch4 = 7;  // float4 per batch
constexpr uint32_t kSumBatch = 4u * kSumBatch4;

__device__ __forceinline__ void load_batch(const float* p, float4 (&v)[kSumBatch4]) {
#pragma unroll
  for (uint32_t j = 0; j < kSumBatch4; j++) v[j] = reinterpret_cast<const float4*>(p)[j];
}

__device__ __forceinline__ float add_batch(float s, const float4 (&v)[kSumBatch4]) {
#pragma unroll
  for (uint32_t j = 0; j < kSumBatch4; j++) {
    s += v[j].x;
    s += v[j].y;
    s += v[j].z;
    s += v[j].w;
  }
  return s;
}

__device__ __forceinline__ float ordered_sum(const float* p, uint32_t n, float s) {
  uint32_t i = 0;
  if (n >= kSumBatch) {
    float4 a[kSumBatch4], b[kSumBatch4];
    load_batch(p, a);
    for (i = kSumBatch; i + 2u * kSumBatch <= n; i += 2u * kSumBatch) {
      load_batch(p + i, b);
      __builtin_amdgcn_sched_barrier(0);
      s = add_batch(s, a);
      load_batch(p + i + kSumBatch, a);
      __builtin_amdgcn_sched_barrier(0);
      s = add_batch(s, b);
    }
    if (i + kSumBatch <= n) {
      load_batch(p + i, b);
      __builtin_amdgcn_sched_barrier(0);
      s = add_batch(s, a);
      s = add_batch(s, b);
      i += kSumBatch;
    } else {
      s = add_batch(s, a);
    }
  }
  for (; i < n; i++) s += p[i];
  return s;
}

// Wave-parallel ordered sum ---------------------------------------------------
//
// ordered_sum's exact result, ((init + p[0]) + p[1]) + ... in float, from one
// full wave: the values are cut into one run of 32-value chunks per lane, and
// each lane adds its run as a chain from a guessed start. The result is
// accepted only when every lane's chain is shown to start exactly where the
// previous lane's ended (lane 0 starts at init): then, by induction over the
// runs, the last lane's end is the sequential sum bit for bit. The guesses
// only decide how fast that happens.
//
// Guesses: an approximate sum of every run, then an exclusive prefix sum (in
// double) of those, gives approximate starts; one chain per lane from there
// gives each run's increment (end minus start). While the running sum stays
// in one binade, an add rounds to the same grid whatever the start, except
// for ties to even, which follow the start's last bit: so an increment is
// nearly independent of where its run starts, and the prefix sum of the
// increments puts every lane within an ulp of its true start. Each checking
// round then chains every run from three candidate starts -- the guess and
// the floats one ulp either side -- and maps each chain's end to the
// candidate of the next lane it equals (or to none). The maps compose (a
// byte permutation, v_perm_b32), and a prefix composition tells every lane
// which of its candidates is the true start. A round that leaves some lane
// unresolved has proved the lanes before it exact; the next guesses come
// from their increments. After kWaveSumRounds checking rounds one chain runs
// on from the last exact lane, so the result is exact in every case (NaN,
// infinity and signed values included) and the cost is bounded.
//
// Layout: value i sits at float index 36*(i/32) + i%32 of p (16-byte aligned
// LDS): the 16-byte reads of 16 consecutive lanes fall on distinct banks.
// Indices from n up to the next multiple of 32 must hold -0.0, the exact
// identity of float addition (x + -0.0 == x for every x, -0.0 included).
constexpr uint32_t kWaveSumRounds = 6;

__host__ __device__ constexpr uint32_t wave_sum_index(uint32_t i) { return (i >> 5) * 36u + (i & 31u); }
__host__ __device__ constexpr uint32_t wave_sum_floats(uint32_t n) { return ((n + 31u) >> 5) * 36u; }

__device__ __forceinline__ void load_chunk(const float* p, float4 (&v)[8]) {
#pragma unroll
  for (uint32_t j = 0; j < 8u; j++) v[j] = reinterpret_cast<const float4*>(p)[j];
}

// Three chains over one chunk, in element order.
__device__ __forceinline__ void chain3(float (&s)[3], const float4 (&v)[8]) {
#pragma unroll
  for (uint32_t j = 0; j < 8u; j++) {
    const float x[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      s[0] += x[i];
      s[1] += x[i];
      s[2] += x[i];
    }
  }
}

__device__ __forceinline__ float chain1(float s, const float4 (&v)[8]) {
#pragma unroll
  for (uint32_t j = 0; j < 8u; j++) {
    s += v[j].x;
    s += v[j].y;
    s += v[j].z;
    s += v[j].w;
  }
  return s;
}

// An approximate sum of one chunk (pairwise; only a guess).
__device__ __forceinline__ float tree_chunk(const float4 (&v)[8]) {
  float t[8];
#pragma unroll
  for (uint32_t j = 0; j < 8u; j++) t[j] = (v[j].x + v[j].y) + (v[j].z + v[j].w);
  return ((t[0] + t[1]) + (t[2] + t[3])) + ((t[4] + t[5]) + (t[6] + t[7]));
}

// DPP moves (GFX9 controls): row_shr:1/2/4/8 within rows of 16 lanes,
// row_bcast:15 (into rows 1 and 3) and row_bcast:31 (into rows 2 and 3) for
// a Hillis-Steele scan; wave_shr:1 (lane i reads lane i-1) and wave_shl:1
// (lane i reads lane i+1) across the wave. Lanes without a source, or
// outside ROWS, read `fill`.
constexpr int kDppWaveShl1 = 0x130;
constexpr int kDppWaveShr1 = 0x138;

template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ uint32_t dpp_fill(uint32_t v, uint32_t fill) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(static_cast<int>(fill), static_cast<int>(v), CTRL, ROWS, 0xF, false));
}

template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ double dpp_fill0_f64(double v) {
  const uint64_t b = static_cast<uint64_t>(__double_as_longlong(v));
  const uint64_t lo = dpp_fill<CTRL, ROWS>(static_cast<uint32_t>(b), 0u);
  const uint64_t hi = dpp_fill<CTRL, ROWS>(static_cast<uint32_t>(b >> 32), 0u);
  return __longlong_as_double(static_cast<long long>((hi << 32) | lo));
}

// Inclusive prefix sum over the 64 lanes (approximate: it only makes
// guesses).
__device__ __forceinline__ double wave_prefix_sum(double v) {
  v += dpp_fill0_f64<0x111>(v);
  v += dpp_fill0_f64<0x112>(v);
  v += dpp_fill0_f64<0x114>(v);
  v += dpp_fill0_f64<0x118>(v);
  v += dpp_fill0_f64<0x142, 0xA>(v);
  v += dpp_fill0_f64<0x143, 0xC>(v);
  return v;
}

// Start guesses from increments: lane k gets init + the increments of lanes
// 0..k-1, rounded to float; lane 0 gets init itself (the shift's fill), so
// no lane-dependent branch surrounds the cross-lane moves.
__device__ __forceinline__ float guess_starts(double d, float init) {
  const float end = static_cast<float>(static_cast<double>(init) + wave_prefix_sum(d));
  return __uint_as_float(dpp_fill<kDppWaveShr1>(__float_as_uint(end), __float_as_uint(init)));
}

// A map from {0, 1, 2, 3} to itself as 4 bytes (byte i = image of i); 3 is
// "none" and maps to itself. map_after(hi, lo) applies lo first: v_perm_b32
// picks byte lo[i] of hi for every byte i.
constexpr uint32_t kMapIdentity = 0x03020100u;
__device__ __forceinline__ uint32_t map_after(uint32_t hi, uint32_t lo) { return __builtin_amdgcn_perm(hi, hi, lo); }

// Exclusive prefix composition over the 64 lanes: lane k gets
// map_{k-1} o ... o map_0 (lane 0 the identity).
__device__ __forceinline__ uint32_t wave_prefix_maps_excl(uint32_t m) {
  m = map_after(m, dpp_fill<0x111>(m, kMapIdentity));
  m = map_after(m, dpp_fill<0x112>(m, kMapIdentity));
  m = map_after(m, dpp_fill<0x114>(m, kMapIdentity));
  m = map_after(m, dpp_fill<0x118>(m, kMapIdentity));
  m = map_after(m, dpp_fill<0x142, 0xA>(m, kMapIdentity));
  m = map_after(m, dpp_fill<0x143, 0xC>(m, kMapIdentity));
  return dpp_fill<kDppWaveShr1>(m, kMapIdentity);
}

// Called by all 64 lanes of one wave with the same p, n and init; returns the
// sum in every lane. `rounds`, when given, receives the checking rounds used
// (lane 0 writes it; kWaveSumRounds + 1 means the closing sequential chain
// ran). The cross-lane moves (DPP, ballot, readlane) read every lane, so
// each runs as a statement of its own at the function's top level, never
// inside a lane-dependent branch or a conditional expression: a C++ ?:
// evaluates only the operand it picks, and a move run with some lanes off
// reads fills in their place.
__device__ __forceinline__ float ordered_sum_wave(const float* p, uint32_t n, float init,
                                                  uint32_t* rounds = nullptr) {
  const uint32_t lane = __lane_id();
  const uint32_t chunks = (n + 31u) >> 5;
  if (chunks == 0) return init;
  const uint32_t per = (chunks + 63u) >> 6;           // chunks per lane
  const uint32_t lanes = (chunks + per - 1u) / per;   // lanes holding values
  const uint32_t mine = lane < lanes ? min(per, chunks - lane * per) : 0u;
  const float* run = p + (mine ? lane * per * 36u : 0u);

  float4 v[8];
  double d = 0.0;  // this lane's increment, as well as known
  if (mine) {
    load_chunk(run, v);
    float t = tree_chunk(v);
    for (uint32_t c = 1; c < mine; c++) {
      float4 w[8];
      load_chunk(run + c * 36u, w);
      t += tree_chunk(w);
    }
    d = t;
  }
  // one chain from the approximate start refines the increment
  {
    const float g = guess_starts(d, init);
    float e = g;
    if (mine) {
      e = chain1(e, v);
      for (uint32_t c = 1; c < mine; c++) {
        float4 w[8];
        load_chunk(run + c * 36u, w);
        e = chain1(e, w);
      }
    }
    d = static_cast<double>(e) - static_cast<double>(g);
  }

  uint32_t r = 0, first_bad = 0;
  float end = init;
  bool done = false;
  while (true) {
    r++;
    const float g = guess_starts(d, init);
    const uint32_t gb = __float_as_uint(g);
    const float cand[3] = {g, __uint_as_float(gb - 1u), __uint_as_float(gb + 1u)};
    float s[3] = {cand[0], cand[1], cand[2]};
    if (mine) {
      chain3(s, v);
      for (uint32_t c = 1; c < mine; c++) {
        float4 w[8];
        load_chunk(run + c * 36u, w);
        chain3(s, w);
      }
    }
    // which candidate of the next lane each end is: bits equal, one below,
    // one above (the move kept out of DPP combining, as in ordered_sum_wave4)
    uint32_t next = dpp_fill<kDppWaveShl1>(gb, 0u);
    asm volatile("" : "+v"(next));
    uint32_t map = 0x03000000u;
#pragma unroll
    for (int i = 0; i < 3; i++) {
      const uint32_t delta = __float_as_uint(s[i]) - next;
      const uint32_t j = delta == 0u ? 0u : delta == 0xFFFFFFFFu ? 1u : delta == 1u ? 2u : 3u;
      map |= j << (8 * i);
    }
    if (lane + 1u >= lanes) map = kMapIdentity;
    // lane 0 starts at candidate 0 (init); lane k at the image of 0 under
    // the maps of the lanes before it
    const uint32_t state = wave_prefix_maps_excl(map) & 0xFFu;
    const float mine_end = state == 1u ? s[1] : state == 2u ? s[2] : s[0];
    const uint64_t bad = __ballot(lane < lanes && state == 3u);
    if (bad == 0) {
      end = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine_end), static_cast<int>(lanes - 1u)));
      done = true;
      break;
    }
    first_bad = static_cast<uint32_t>(__builtin_ctzll(bad));  // >= 1: lane 0 is always resolved
    end = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine_end), static_cast<int>(first_bad - 1u)));
    if (r == kWaveSumRounds) break;
    const float start = state == 1u ? cand[1] : state == 2u ? cand[2] : cand[0];
    d = lane < first_bad ? static_cast<double>(mine_end) - static_cast<double>(start)
                         : static_cast<double>(s[0]) - static_cast<double>(cand[0]);
  }
  if (!done) {
    // `end` is the exact sum of the runs before lane first_bad
    for (uint32_t c = first_bad * per; c < chunks; c++) {
      float4 w[8];
      load_chunk(p + c * 36u, w);
      end = chain1(end, w);
    }
    r++;
  }
  if (rounds && lane == 0) *rounds = r;
  return end;
}

// ordered_sum_wave for at most 256 values in plain order: p 16-byte aligned,
// -0.0 from n up to the next multiple of 4. Lane l holds values 4l..4l+3,
// so every chain is 4 additions long where ordered_sum_wave's are 32 (a
// softmax over a few hundred rows spread 1-7 lanes of 32). Same contract
// and the same rounds.
__device__ __forceinline__ float ordered_sum_wave4(const float* p, uint32_t n, float init,
                                                   uint32_t* rounds = nullptr) {
  const uint32_t lane = __lane_id();
  const uint32_t lanes = (n + 3u) >> 2;  // lanes holding values
  if (lanes == 0) return init;
  const bool mine = lane < lanes;
  float v[4] = {-0.0f, -0.0f, -0.0f, -0.0f};
  if (mine) {
    const f32x4 t = reinterpret_cast<const f32x4*>(p)[lane];
    v[0] = t[0];
    v[1] = t[1];
    v[2] = t[2];
    v[3] = t[3];
  }
  double d = mine ? static_cast<double>((v[0] + v[1]) + (v[2] + v[3])) : 0.0;
  {
    // one chain from the approximate start refines the increment
    const float g = guess_starts(d, init);
    float e = g;
#pragma unroll
    for (int i = 0; i < 4; i++) e += v[i];
    d = mine ? static_cast<double>(e) - static_cast<double>(g) : 0.0;
  }
  uint32_t r = 0, first_bad = 0;
  float end = init;
  bool done = false;
  while (true) {
    r++;
    const float g = guess_starts(d, init);
    const uint32_t gb = __float_as_uint(g);
    const float cand[3] = {g, __uint_as_float(gb - 1u), __uint_as_float(gb + 1u)};
    float s[3] = {cand[0], cand[1], cand[2]};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      s[0] += v[i];
      s[1] += v[i];
      s[2] += v[i];
    }
    uint32_t next = dpp_fill<kDppWaveShl1>(gb, 0u);
    // kept out of the compiler's DPP combining: folded into the subtraction
    // below as v_subrev_u32_dpp wave_shl:1 it read wrong lanes on gfx950
    asm volatile("" : "+v"(next));
    // the next lane's candidate each end is: ulp distance 0, -1, +1 are 0,
    // 1, 2 (2|delta| - (delta < 0)), any other none; in arithmetic, so that
    // no lane-dependent branch appears
    uint32_t map = 0x03000000u;
#pragma unroll
    for (int i = 0; i < 3; i++) {
      const uint32_t delta = __float_as_uint(s[i]) - next;
      const uint32_t neg = delta >> 31;
      const uint32_t mag = min(neg ? 0u - delta : delta, 2u);
      map |= min(2u * mag - neg, 3u) << (8 * i);
    }
    if (lane + 1u >= lanes) map = kMapIdentity;
    const uint32_t state = wave_prefix_maps_excl(map) & 0xFFu;
    const float mine_end = state == 1u ? s[1] : state == 2u ? s[2] : s[0];
    const uint64_t bad = __ballot(mine && state == 3u);
    if (bad == 0) {
      end = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine_end), static_cast<int>(lanes - 1u)));
      done = true;
      break;
    }
    first_bad = static_cast<uint32_t>(__builtin_ctzll(bad));  // >= 1: lane 0 is always resolved
    end = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine_end), static_cast<int>(first_bad - 1u)));
    if (r == kWaveSumRounds) break;
    const float start = state == 1u ? cand[1] : state == 2u ? cand[2] : cand[0];
    d = lane < first_bad ? static_cast<double>(mine_end) - static_cast<double>(start)
                         : static_cast<double>(s[0]) - static_cast<double>(cand[0]);
  }
  if (!done) {
    // `end` is the exact sum of the runs before lane first_bad
    for (uint32_t i = 4u * first_bad; i < 4u * lanes; i++) end += p[i];
    r++;
  }
  if (rounds && lane == 0) *rounds = r;
  return end;
}


// Q8Kind::SuperBlock (portable/q8.rs:64-98) of one 256-value block held by a
// wave, values lane*4 .. lane*4+3 in f: the quants, the eight 32-block
// scales and the 32- and 16-run sums of token t, super-block sb, written to
// q (a Q8Dev).
template <class Q>
__device__ __forceinline__ void quantize_super_block(const float (&f)[4], uint32_t lane, size_t t, uint32_t sb,
                                                     const Q& q) {
  // amax: f32::max folded from 0.0 (q8.rs:12-14,19-25). Comparisons keep a
  // NaN from ever entering the running maximum, as maxNum does; the result
  // is a non-negative float or +inf, whose bits order like u32 (DPP within
  // each half-wave, then the two halves).
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    float m = __builtin_fabsf(f[i]);
    amax = m > amax ? m : amax;
  }
  const uint32_t ab = half_max_u32(__float_as_uint(amax));
  amax = __uint_as_float(max(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(ab), 0)),
                             static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(ab), 32))));
  // The first element, in order, whose magnitude is amax (q8.rs:26-32).
  uint32_t idx = 256u;
#pragma unroll
  for (int i = 3; i >= 0; i--)
    if (__builtin_fabsf(f[i]) == amax) idx = lane * 4u + i;
  idx = half_min_u32(idx);
  idx = min(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(idx), 0)),
            static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(idx), 32)));
  // the owner of element idx broadcasts it (no dependent reload)
  const uint32_t sel = idx & 3u;
  const float mine = sel == 0 ? f[0] : sel == 1 ? f[1] : sel == 2 ? f[2] : f[3];
  const float owned =
      __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), static_cast<int>((idx >> 2) & 63u)));
  const float max = idx < 256u ? owned : 0.0f;
  const float inverse = (max == 0.0f) ? 0.0f : __fdiv_rn(-127.0f, max);
  const float step = (max == 0.0f) ? 0.0f : __fdiv_rn(1.0f, inverse);

  int32_t qv[4];
  int32_t s = 0;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    float prod = f[i] * inverse;
    qv[i] = round_to_i8(prod);
    s += qv[i];
  }
  uint32_t packed = (static_cast<uint32_t>(qv[0]) & 0xffu) | ((static_cast<uint32_t>(qv[1]) & 0xffu) << 8) |
                    ((static_cast<uint32_t>(qv[2]) & 0xffu) << 16) | (static_cast<uint32_t>(qv[3]) << 24);
  *reinterpret_cast<uint32_t*>(q.quants + t * q.qstride + static_cast<size_t>(sb) * 256u + lane * 4u) = packed;
  // sums per 16 (a quad: quad_perm swaps) and per 32 (two quads: the
  // half-row mirror)
  uint32_t s16 = static_cast<uint32_t>(s);
  s16 += dpp<0xB1>(s16);
  s16 += dpp<0x4E>(s16);
  const uint32_t s32 = s16 + dpp<0x141>(s16);
  const size_t b0 = t * q.bstride + static_cast<size_t>(sb) * 8u;
  if ((lane & 3u) == 0) q.sums16[2 * t * q.bstride + static_cast<size_t>(sb) * 16u + lane / 4u] = static_cast<int32_t>(s16);
  if ((lane & 7u) == 0) q.sums[b0 + lane / 8u] = static_cast<int32_t>(s32);
  if (lane < 8u) q.scales[b0 + lane] = step;
}

// ---------------------------------------------------------------- greedy pick
// (sampling/src/filters.rs:37-43: NaN as -inf, f32::total_cmp, the last
// maximum wins)
// f32::total_cmp's order as an i32 key.
__device__ __forceinline__ int32_t total_key(float f) {
  const int32_t b = __float_as_int(f);
  return b ^ static_cast<int32_t>(static_cast<uint32_t>(b >> 31) >> 1);
}

// (key, index) as one unsigned 64-bit value in the pick's order: the
// total-order key (made unsigned) above the index (a larger index wins a
// tie: the last maximum). Keys of real logits are above INT32_MIN (a NaN
// enters as -inf), so 0 stands for "no logit".
__device__ __forceinline__ uint64_t pick_code(int32_t key, uint32_t idx) {
  return (static_cast<uint64_t>(static_cast<uint32_t>(key) ^ 0x80000000u) << 32) | idx;
}

// The maximum code over the wave, in every lane: the keys first, then the
// indices among the lanes holding the largest key.
__device__ __forceinline__ uint64_t wave_max_code(uint64_t c) {
  uint32_t hi = static_cast<uint32_t>(c >> 32);
  uint32_t m = half_max_u32(hi);
  m = max(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(m), 0)),
          static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(m), 32)));
  uint32_t lo = hi == m ? static_cast<uint32_t>(c) : 0u;
  lo = half_max_u32(lo);
  lo = max(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(lo), 0)),
           static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(lo), 32)));
  return (static_cast<uint64_t>(m) << 32) | lo;
}

// The pick's partial over a set of logits (one workgroup's rows): the
// largest code and whether any logit is finite.
struct PickPart {
  uint64_t code;
  uint32_t fin;
  uint32_t pad;
};

// ---------------------------------------------------------------- unit layout
// Q4_K and Q6_K matrices live in HBM once, in the unit layout: the blocks in
// row-major order (block e = row * blocks_per_row + column), cut into groups
// of 16, each group laid out the way a wave of 16 four-lane teams reads it
// (lane l = 4 * tw + p of the team at position tw). Group g of a matrix
// starts at g * kUnitBytes{Q4,Q6}; block e is at position tw = e & 15 of
// group e >> 4.
//   Q4_K (2304 bytes): headers (d, dmin, scales[12]) [16][16] at 16 tw |
//     qs[0..64) of block tw at 256 + 64 tw | qs[64..128) at 1280 + 64 tw.
//   Q6_K (3360 bytes): ql[64h + x], x < 32, at 64 tw + 32h + x |
//     ql[64h + 32 + x] at 1024 + 64 tw + 32h + x | qh[c] at 2048 + 64 tw + c |
//     scales[16] at 3072 + 16 tw | d at 3328 + 2 tw.
// So a team lane p's 16-byte pieces of its block sit at one offset each
// (Q4_K: 256 + 64 tw + 16p, 1280 + 64 tw + 16p; Q6_K: 64 tw + 16p,
// 1024 + 64 tw + 16p, 2048 + 64 tw + 16p), and a wave whose 16 teams read the
// 16 blocks of a group reads 1 KB of consecutive bytes per load.
constexpr uint32_t kUnitBytesQ4 = 16u * 144u;
constexpr uint32_t kUnitBytesQ6 = 16u * 210u;

__device__ __forceinline__ const uint8_t* unit_group(const uint8_t* m, uint32_t type_id, uint32_t e) {
  return m + static_cast<size_t>(e >> 4) * (type_id == 12u ? kUnitBytesQ4 : kUnitBytesQ6);
}

// Byte c of block e in its GGUF order (Q4_K 0..143, Q6_K 0..209).
__device__ __forceinline__ uint8_t unit_byte(const uint8_t* m, uint32_t type_id, uint32_t e, uint32_t c) {
  const uint8_t* g = unit_group(m, type_id, e);
  const uint32_t tw = e & 15u;
  if (type_id == 12u) {
    if (c < 16u) return g[16u * tw + c];
    c -= 16u;
    return c < 64u ? g[256u + 64u * tw + c] : g[1280u + 64u * tw + (c - 64u)];
  }
  if (c < 128u) {
    const uint32_t h = c >> 6, x = c & 63u;
    return x < 32u ? g[64u * tw + 32u * h + x] : g[1024u + 64u * tw + 32u * h + (x - 32u)];
  }
  if (c < 192u) return g[2048u + 64u * tw + (c - 128u)];
  if (c < 208u) return g[3072u + 16u * tw + (c - 192u)];
  return g[3328u + 2u * tw + (c - 208u)];
}

// Weight l (0..255) of Q4_K / Q6_K block e, dequantized as Matrix::copy_row
// does (quantize/src/q4_k.rs:32-66, q6_k.rs:13-43), from the unit layout.
__device__ __forceinline__ float unit_weight(const uint8_t* m, uint32_t type_id, uint32_t e, uint32_t l) {
  auto byte = [&](uint32_t c) { return static_cast<uint32_t>(unit_byte(m, type_id, e, c)); };
  if (type_id == 12u) {
    const float d = f16_lo(byte(0) | (byte(1) << 8)), dmin = f16_lo(byte(2) | (byte(3) << 8));
    const uint32_t j = l / 32u, li = l % 32u;
    uint32_t sc, mn;
    if (j < 4u) {
      sc = byte(4u + j) & 63u;
      mn = byte(8u + j) & 63u;
    } else {
      sc = (byte(8u + j) & 0x0Fu) | ((byte(j) >> 6) << 4);
      mn = (byte(8u + j) >> 4) | ((byte(4u + j) >> 6) << 4);
    }
    const uint32_t qb = byte(16u + 32u * (j / 2u) + li);
    const uint32_t qv = (j & 1u) ? (qb >> 4) : (qb & 0x0Fu);
    const float ds = d * static_cast<float>(sc), dm = dmin * static_cast<float>(mn);
    const float prod = ds * static_cast<float>(qv);
    return prod - dm;
  }
  const float d = f16_lo(byte(208) | (byte(209) << 8));
  const uint32_t hh = l / 128u, rr = (l % 128u) / 32u, li = l % 32u;
  const uint32_t low = byte(64u * hh + 32u * (rr & 1u) + li);
  const uint32_t high = byte(128u + 32u * hh + li);
  const uint32_t nib = rr < 2u ? (low & 0x0Fu) : (low >> 4);
  const int32_t qv = static_cast<int32_t>(nib | (((high >> (2u * rr)) & 3u) << 4)) - 32;
  const float sc = static_cast<float>(static_cast<int8_t>(byte(192u + 8u * hh + 2u * rr + li / 16u)));
  const float ds = d * sc;
  return ds * static_cast<float>(qv);
}

}  // namespace rh
