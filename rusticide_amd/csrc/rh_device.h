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

__device__ __forceinline__ u32x4 load16(const uint8_t* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

__device__ __forceinline__ u32x4 load16_a4(const uint8_t* p) {
  u32x4_a4 v = *reinterpret_cast<const u32x4_a4*>(p);
  return u32x4{v.x, v.y, v.z, v.w};
}

__device__ __forceinline__ uint32_t load4(const uint8_t* p) {
  return *reinterpret_cast<const uint32_t*>(p);
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

}  // namespace rh
