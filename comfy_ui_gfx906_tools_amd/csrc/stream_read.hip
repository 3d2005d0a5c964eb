// The HBM read floor of a single kernel call: `bytes` bytes read once with 16-byte loads (every
// lane keeps four loads in flight), folded into one xor word per workgroup so the loads cannot be
// dropped. The skinny-M W4A16 kernels read their weights once per call; this is the same bytes
// with no arithmetic, the reference point their GB/s is compared with.
#include "common.hpp"
#include "launch.hpp"

namespace qlinear {

namespace {

constexpr int kSrThreads = 512;

__global__ __launch_bounds__(kSrThreads) void stream_read_kernel(const u32x4* __restrict__ p, size_t n16,
                                                                 uint32_t* __restrict__ out) {
  __shared__ uint32_t red[kSrThreads / kWave];
  const size_t stride = (size_t)gridDim.x * kSrThreads;
  u32x4 acc = {0u, 0u, 0u, 0u};
  size_t i = (size_t)blockIdx.x * kSrThreads + threadIdx.x;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const u32x4 a = __builtin_nontemporal_load(p + i), b = __builtin_nontemporal_load(p + i + stride);
    const u32x4 c = __builtin_nontemporal_load(p + i + 2 * stride), d = __builtin_nontemporal_load(p + i + 3 * stride);
    acc ^= a ^ b ^ c ^ d;
  }
  for (; i < n16; i += stride) acc ^= __builtin_nontemporal_load(p + i);
  uint32_t v = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v ^= (uint32_t)__shfl_xor((int)v, off, kWave);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t r = 0;
#pragma unroll
    for (int w = 0; w < kSrThreads / kWave; ++w) r ^= red[w];
    out[blockIdx.x] = r;
  }
}

}  // namespace

hipError_t stream_read_launch(const void* buf, int64_t bytes, uint32_t* out, int workgroups, hipStream_t stream) {
  hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)workgroups), dim3(kSrThreads), 0, stream, (const u32x4*)buf,
                     (size_t)(bytes / 16), out);
  return hipGetLastError();
}

}  // namespace qlinear
