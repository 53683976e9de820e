// stream_read.hip -- bench hooks: a plain streaming read of device memory,
// the measured bandwidth ceiling the GEMV kernels are compared with, and a
// bounded hold that keeps the stream busy while the host queues a timed run.
//
// Every lane reads 16-byte words in a grid stride (nontemporal, as the GEMV
// weights are used once) and XORs them together so the loads stay live; each
// workgroup leaves one word in the sink. No arithmetic of the product path
// runs here. 2048 workgroups: the fastest grid measured on MI355X for a
// 54 MB read (1024: 5.4 TB/s, 2048: 6.0, 4096 and more: 5.7-5.8).
#include "rh_device.h"
#include "rh_internal.h"

namespace rh {
namespace {

constexpr uint32_t kThreads = 256;

__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4* __restrict__ p, size_t n16, uint32_t* sink) {
  __shared__ uint32_t red[kThreads / 64];
  uint32_t acc = 0;
  const size_t stride = static_cast<size_t>(gridDim.x) * kThreads;
  for (size_t i = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x; i < n16; i += stride) {
    const u32x4 v = __builtin_nontemporal_load(p + i);
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  acc ^= static_cast<uint32_t>(__shfl_xor(static_cast<int>(acc), 32, 64));
  acc = half_max_u32(acc);  // any lane-combining fold keeps the loads live
  if ((threadIdx.x & 63u) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) sink[blockIdx.x] = red[0] ^ red[1] ^ red[2] ^ red[3];
}

// One wave that returns once the constant-rate clock has advanced `ticks`
// (or after kMaxSpins polls, whichever comes first), so every wave ends.
constexpr uint32_t kMaxSpins = 4u << 20;

__global__ __launch_bounds__(64) void hold_kernel(uint64_t ticks) {
  const uint64_t t0 = static_cast<uint64_t>(wall_clock64());
  for (uint32_t i = 0; i < kMaxSpins; i++) {
    if (static_cast<uint64_t>(wall_clock64()) - t0 >= ticks) break;
    __builtin_amdgcn_s_sleep(8);
  }
}

}  // namespace
}  // namespace rh

extern "C" rh_status rh_hold_device(rh_ctx* ctx, uint32_t microseconds, void* stream) {
  using namespace rh;
  if (!ctx || microseconds > RH_HOLD_MAX_US) return RH_ERR_INVALID_ARGUMENT;
  if (microseconds == 0) return RH_OK;
  if (hipSetDevice(ctx_device(ctx)) != hipSuccess) return RH_ERR_DEVICE;
  int khz = 0;
  if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, ctx_device(ctx)) != hipSuccess || khz <= 0)
    return RH_ERR_DEVICE;
  const uint64_t ticks = static_cast<uint64_t>(microseconds) * static_cast<uint64_t>(khz) / 1000u;
  const hipStream_t s = stream ? static_cast<hipStream_t>(stream) : static_cast<hipStream_t>(rh_stream(ctx));
  hipLaunchKernelGGL(hold_kernel, dim3(1), dim3(64), 0, s, ticks);
  return hipGetLastError() == hipSuccess ? RH_OK : RH_ERR_DEVICE;
}

extern "C" rh_status rh_stream_read_device(rh_ctx* ctx, const void* const* buffers, size_t n_buffers, size_t bytes,
                                            size_t launches, uint32_t* sink) {
  using namespace rh;
  if (!ctx || !sink || bytes % 16u != 0 || (launches && (!buffers || n_buffers == 0)))
    return RH_ERR_INVALID_ARGUMENT;
  for (size_t i = 0; i < n_buffers && launches; i++)
    if (!buffers[i] || reinterpret_cast<uintptr_t>(buffers[i]) % 16u != 0) return RH_ERR_INVALID_ARGUMENT;
  if (bytes == 0 || launches == 0) return RH_OK;
  if (hipSetDevice(ctx_device(ctx)) != hipSuccess) return RH_ERR_DEVICE;
  const hipStream_t s = static_cast<hipStream_t>(rh_stream(ctx));
  for (size_t i = 0; i < launches; i++) {
    hipLaunchKernelGGL(stream_read_kernel, dim3(RH_STREAM_READ_SINK_WORDS), dim3(kThreads), 0, s,
                       static_cast<const u32x4*>(buffers[i % n_buffers]), bytes / 16u, sink);
    if (hipGetLastError() != hipSuccess) return RH_ERR_DEVICE;
  }
  return RH_OK;
}
