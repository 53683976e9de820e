// quantize.hip -- the activation quantizers on the device.
//
// SuperBlock (ggml Q8_K) follows crates/rusticide-kernels/src/portable/q8.rs:64-98;
// Row (bitnet.cpp's legacy I8_S) follows portable/q8.rs:38-49 and :99-105.
// Both produce exactly the quants, scales and sums the CPU path produces.
#include "rh_device.h"
#include "rh_internal.h"

namespace rh {

// One wave per 256-element super-block, four values per lane.
__global__ __launch_bounds__(256) void quantize_super_kernel(const float* __restrict__ x,
                                                             size_t width, uint32_t n_super,
                                                             Q8Dev q) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t sb = blockIdx.x * 4u + (threadIdx.x >> 6);
  const size_t t = blockIdx.y;
  if (sb >= n_super) return;  // wave-uniform
  // one 16-byte load a lane (rows are whole super blocks, x 16-byte aligned)
  const float4 v = *reinterpret_cast<const float4*>(x + t * width + static_cast<size_t>(sb) * 256u + lane * 4u);
  const float f[4] = {v.x, v.y, v.z, v.w};
  quantize_super_block(f, lane, t, sb, q);
}

// One 1024-lane workgroup per token, four consecutive values per lane per
// pass, all held in registers: the row divisor in f64 with C's MAX
// semantics, then the quants. A NaN element restarts the running maximum at
// the next element (q8.rs:42-45), so the divisor depends on the elements
// after the last NaN only; a trailing NaN makes it NaN.
constexpr uint32_t kRowThreads = 1024;
constexpr uint32_t kRowPasses = 4;  // up to 16384 values per token

__device__ __forceinline__ int block_max_i(int v, int* red) {
  for (int off = 32; off > 0; off >>= 1) {
    const int o = __shfl_xor(v, off, 64);
    v = o > v ? o : v;
  }
  const uint32_t wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63u) == 0) red[wave] = v;
  __syncthreads();
  int m = red[0];
  for (uint32_t w = 1; w < kRowThreads / 64u; w++) m = red[w] > m ? red[w] : m;
  return m;
}

__device__ __forceinline__ float block_max_f(float v, float* red) {
  for (int off = 32; off > 0; off >>= 1) {
    const float o = __shfl_xor(v, off, 64);
    v = o > v ? o : v;
  }
  const uint32_t wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63u) == 0) red[wave] = v;
  __syncthreads();
  float m = red[0];
  for (uint32_t w = 1; w < kRowThreads / 64u; w++) m = red[w] > m ? red[w] : m;
  return m;
}

__global__ __launch_bounds__(1024) void quantize_row_kernel(const float* __restrict__ x, size_t width,
                                                            uint32_t n_blocks, Q8Dev q) {
  __shared__ int s_i[kRowThreads / 64u];
  __shared__ float s_f[kRowThreads / 64u];
  const size_t t = blockIdx.x;
  const float* v = x + t * width;
  const uint32_t n = n_blocks * 32u;
  const uint32_t lane = threadIdx.x & 63u;
  float f[kRowPasses][4];
  int last_nan = -1;
#pragma unroll
  for (uint32_t k = 0; k < kRowPasses; k++) {
    const uint32_t base = 4u * threadIdx.x + 4u * kRowThreads * k;
#pragma unroll
    for (uint32_t i = 0; i < 4; i++) {
      const uint32_t e = base + i;
      f[k][i] = e < n ? v[e] : 0.0f;
      if (e < n && f[k][i] != f[k][i]) last_nan = static_cast<int>(e);
    }
  }
  const int p = block_max_i(last_nan, s_i);
  float mag_max = 0.0f;
#pragma unroll
  for (uint32_t k = 0; k < kRowPasses; k++)
#pragma unroll
    for (uint32_t i = 0; i < 4; i++) {
      const uint32_t e = 4u * threadIdx.x + 4u * kRowThreads * k + i;
      const float m = __builtin_fabsf(f[k][i]);
      if (e < n && static_cast<int>(e) > p) mag_max = m > mag_max ? m : mag_max;
    }
  const float mm = block_max_f(mag_max, s_f);
  double mx;
  if (p < 0) {
    mx = static_cast<double>(mm);
    mx = 1e-5 > mx ? 1e-5 : mx;
  } else if (p == static_cast<int>(n) - 1) {
    mx = __builtin_nan("");
  } else {
    mx = static_cast<double>(mm);
  }
  const float divisor = static_cast<float>(127.0 / mx);

#pragma unroll
  for (uint32_t k = 0; k < kRowPasses; k++) {
    const uint32_t base = 4u * threadIdx.x + 4u * kRowThreads * k;
    if (4u * kRowThreads * k >= n) break;  // uniform
    int32_t qv[4];
    int32_t s = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float prod = f[k][i] * divisor;
      qv[i] = round_row_to_i8(prod);
      s += qv[i];
    }
    // a 32-block is 8 lanes of 4; lanes past n belong to whole blocks past n
    int32_t s32 = s + __shfl_xor(s, 1, 64);
    s32 += __shfl_xor(s32, 2, 64);
    s32 += __shfl_xor(s32, 4, 64);
    if (base < n) {
      const uint32_t packed = (static_cast<uint32_t>(qv[0]) & 0xffu) | ((static_cast<uint32_t>(qv[1]) & 0xffu) << 8) |
                              ((static_cast<uint32_t>(qv[2]) & 0xffu) << 16) | (static_cast<uint32_t>(qv[3]) << 24);
      *reinterpret_cast<uint32_t*>(q.quants + t * q.qstride + base) = packed;
      if ((lane & 7u) == 0) {
        q.sums[t * q.bstride + base / 32u] = s32;
        q.scales[t * q.bstride + base / 32u] = divisor;
      }
    }
  }
}

// The same arithmetic with one wave per token (four tokens per workgroup):
// lane l holds the 16-byte chunks l, l+64, ... of the row in registers, so
// both reductions stay inside the wave and every load is issued at once. For
// rows of at most 256*P values whose width is a multiple of 4, and batches of
// 512 tokens or more.
template <uint32_t P>
__global__ __launch_bounds__(256) void quantize_row_wave_kernel(const float* __restrict__ x, size_t width,
                                                                uint32_t n_blocks, size_t tokens, Q8Dev q) {
  const size_t t = static_cast<size_t>(blockIdx.x) * 4u + (threadIdx.x >> 6);
  if (t >= tokens) return;  // whole waves
  const uint32_t lane = threadIdx.x & 63u;
  const float* v = x + t * width;
  const uint32_t n = n_blocks * 32u;  // a multiple of 32: chunks are all in or all out
  // every load issued unconditionally (chunks past n read chunk 0 and are
  // then zeroed), so the compiler emits no branch around them
  float4 f[P];
#pragma unroll
  for (uint32_t k = 0; k < P; k++) {
    const uint32_t base = 4u * (lane + 64u * k);
    f[k] = *reinterpret_cast<const float4*>(v + (base < n ? base : 0u));
  }
  int last_nan = -1;
#pragma unroll
  for (uint32_t k = 0; k < P; k++) {
    const uint32_t base = 4u * (lane + 64u * k);
    const bool in = base < n;
    if (!in) f[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    last_nan = (in && f[k].x != f[k].x) ? static_cast<int>(base) : last_nan;
    last_nan = (in && f[k].y != f[k].y) ? static_cast<int>(base + 1u) : last_nan;
    last_nan = (in && f[k].z != f[k].z) ? static_cast<int>(base + 2u) : last_nan;
    last_nan = (in && f[k].w != f[k].w) ? static_cast<int>(base + 3u) : last_nan;
  }
  const int p = half_max_i32(last_nan);
  const int pw = max(__builtin_amdgcn_readlane(p, 0), __builtin_amdgcn_readlane(p, 32));
  float mag_max = 0.0f;
#pragma unroll
  for (uint32_t k = 0; k < P; k++) {
    const uint32_t base = 4u * (lane + 64u * k);
    const float e[4] = {f[k].x, f[k].y, f[k].z, f[k].w};
#pragma unroll
    for (uint32_t i = 0; i < 4u; i++) {
      const float m = __builtin_fabsf(e[i]);
      mag_max = (base + i < n && static_cast<int>(base + i) > pw && m > mag_max) ? m : mag_max;
    }
  }
  // magnitudes are non-negative floats or +inf: their bits order like u32
  const uint32_t mb = half_max_u32(__float_as_uint(mag_max));
  const float mm = __uint_as_float(max(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(mb), 0)),
                                       static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(mb), 32))));
  double mx;
  if (pw < 0) {
    mx = static_cast<double>(mm);
    mx = 1e-5 > mx ? 1e-5 : mx;
  } else if (pw == static_cast<int>(n) - 1) {
    mx = __builtin_nan("");
  } else {
    mx = static_cast<double>(mm);
  }
  const float divisor = static_cast<float>(127.0 / mx);
#pragma unroll
  for (uint32_t k = 0; k < P; k++) {
    const uint32_t base = 4u * (lane + 64u * k);
    if (64u * 4u * k >= n) break;  // uniform
    const float e[4] = {f[k].x, f[k].y, f[k].z, f[k].w};
    int32_t qv[4];
    int32_t s = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float prod = e[i] * divisor;
      qv[i] = round_row_to_i8(prod);
      s += qv[i];
    }
    // a 32-block is the 8 lanes 8j..8j+7: quad sums, then the half-row mirror
    uint32_t s32 = static_cast<uint32_t>(s);
    s32 += dpp<0xB1>(s32);
    s32 += dpp<0x4E>(s32);
    s32 += dpp<0x141>(s32);
    if (base < n) {
      const uint32_t packed = (static_cast<uint32_t>(qv[0]) & 0xffu) | ((static_cast<uint32_t>(qv[1]) & 0xffu) << 8) |
                              ((static_cast<uint32_t>(qv[2]) & 0xffu) << 16) | (static_cast<uint32_t>(qv[3]) << 24);
      *reinterpret_cast<uint32_t*>(q.quants + t * q.qstride + base) = packed;
      if ((lane & 7u) == 0) {
        q.sums[t * q.bstride + base / 32u] = static_cast<int32_t>(s32);
        q.scales[t * q.bstride + base / 32u] = divisor;
      }
    }
  }
}

// Rows wider than the register-resident kernel holds: three passes over
// global memory, one workgroup per token.
__global__ __launch_bounds__(256) void quantize_row_wide_kernel(const float* __restrict__ x, size_t width,
                                                                uint32_t n_blocks, Q8Dev q) {
  __shared__ int s_last_nan;
  __shared__ float s_max[4];
  __shared__ int s_nan_wave[4];
  const size_t t = blockIdx.x;
  const float* v = x + t * width;
  const uint32_t n = n_blocks * 32u;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;

  int last_nan = -1;
  for (uint32_t i = tid; i < n; i += 256u)
    if (v[i] != v[i]) last_nan = static_cast<int>(i);
  for (int off = 32; off > 0; off >>= 1) {
    int o = __shfl_xor(last_nan, off, 64);
    last_nan = o > last_nan ? o : last_nan;
  }
  if (lane == 0) s_nan_wave[wave] = last_nan;
  __syncthreads();
  if (tid == 0) {
    int m = s_nan_wave[0];
    for (int w = 1; w < 4; w++) m = s_nan_wave[w] > m ? s_nan_wave[w] : m;
    s_last_nan = m;
  }
  __syncthreads();
  const int p = s_last_nan;
  float mag_max = 0.0f;
  for (uint32_t i = tid; i < n; i += 256u) {
    if (static_cast<int>(i) > p) {
      float m = __builtin_fabsf(v[i]);
      mag_max = m > mag_max ? m : mag_max;
    }
  }
  for (int off = 32; off > 0; off >>= 1) {
    float o = __shfl_xor(mag_max, off, 64);
    mag_max = o > mag_max ? o : mag_max;
  }
  if (lane == 0) s_max[wave] = mag_max;
  __syncthreads();
  float mm = s_max[0];
  for (int w = 1; w < 4; w++) mm = s_max[w] > mm ? s_max[w] : mm;
  double mx;
  if (p < 0) {
    mx = static_cast<double>(mm);
    mx = 1e-5 > mx ? 1e-5 : mx;
  } else if (p == static_cast<int>(n) - 1) {
    mx = __builtin_nan("");
  } else {
    mx = static_cast<double>(mm);
  }
  const float divisor = static_cast<float>(127.0 / mx);

  for (uint32_t base = tid * 4u; base < n; base += 1024u) {
    int32_t qv[4];
    int32_t s = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      float prod = v[base + i] * divisor;
      qv[i] = round_row_to_i8(prod);
      s += qv[i];
    }
    uint32_t packed = (static_cast<uint32_t>(qv[0]) & 0xffu) | ((static_cast<uint32_t>(qv[1]) & 0xffu) << 8) |
                      ((static_cast<uint32_t>(qv[2]) & 0xffu) << 16) | (static_cast<uint32_t>(qv[3]) << 24);
    *reinterpret_cast<uint32_t*>(q.quants + t * q.qstride + base) = packed;
    int32_t s32 = s + __shfl_xor(s, 1, 64);
    s32 += __shfl_xor(s32, 2, 64);
    s32 += __shfl_xor(s32, 4, 64);
    if ((lane & 7u) == 0) {
      q.sums[t * q.bstride + base / 32u] = s32;
      q.scales[t * q.bstride + base / 32u] = divisor;
    }
  }
}

hipError_t launch_quantize_super(const float* x, size_t width, size_t tokens, const Q8Dev& q,
                                 hipStream_t s) {
  const uint32_t n_super = static_cast<uint32_t>(width / 256u);
  if (n_super == 0 || tokens == 0) return hipSuccess;
  dim3 grid((n_super + 3u) / 4u, static_cast<uint32_t>(tokens));
  hipLaunchKernelGGL(quantize_super_kernel, grid, dim3(256), 0, s, x, width, n_super, q);
  return hipGetLastError();
}

hipError_t launch_quantize_row(const float* x, size_t width, size_t tokens, const Q8Dev& q,
                               hipStream_t s) {
  const uint32_t n_blocks = static_cast<uint32_t>(width / 32u);
  if (n_blocks == 0 || tokens == 0) return hipSuccess;
  const uint32_t n = n_blocks * 32u;
  // one wave per token pays off once there are enough tokens to fill the
  // chip; fewer tokens spread each row over a 1024-lane workgroup instead
  if (width % 4u == 0 && n <= 256u * 32u && tokens >= 512u) {
    const dim3 grid(static_cast<uint32_t>((tokens + 3u) / 4u));
    if (n <= 256u * 8u)
      hipLaunchKernelGGL(quantize_row_wave_kernel<8>, grid, dim3(256), 0, s, x, width, n_blocks, tokens, q);
    else if (n <= 256u * 16u)
      hipLaunchKernelGGL(quantize_row_wave_kernel<16>, grid, dim3(256), 0, s, x, width, n_blocks, tokens, q);
    else
      hipLaunchKernelGGL(quantize_row_wave_kernel<32>, grid, dim3(256), 0, s, x, width, n_blocks, tokens, q);
    return hipGetLastError();
  }
  if (n_blocks * 32u <= 4u * kRowThreads * kRowPasses)
    hipLaunchKernelGGL(quantize_row_kernel, dim3(static_cast<uint32_t>(tokens)), dim3(kRowThreads), 0, s, x,
                       width, n_blocks, q);
  else
    hipLaunchKernelGGL(quantize_row_wide_kernel, dim3(static_cast<uint32_t>(tokens)), dim3(256), 0, s, x,
                       width, n_blocks, q);
  return hipGetLastError();
}

}  // namespace rh
