// Quantizer kernels for gfx950.
//
// quantize_int4: symmetric block-32 int4 with the reference's packing
//   (nodes/ComfyUI-Gfx906Int4/ops.py:108-126: scale = clamp_min(amax, 1e-8) / 7,
//   codes = clamp(round_half_even(x / scale), -8, 7), byte j = code[2j] | code[2j+1] << 4).
//   rule 0 divides the amax by 7 (torch on CPU), rule 1 multiplies by fl(1/7) (torch's
//   scalar-divisor path on GPU and csrc/int4_gemm_scaled.hip:210-211). One thread per block.
// quantize_int8_per_token: s = max(amax(row), 1e-8) * fl(1/127),
//   q = clamp(rint(x / s), -127, 127) (csrc/int8_gemm.hip:215-246, block widened to the row).
//   One 256-thread workgroup per row; rows of K % 8 == 0 up to 16384 stay in registers.
// repack_q4_0: lossless ggml Q4_0 -> native layout (nodes/ComfyUI-Gfx906Int4/ops.py:129-164).
#include "common.hpp"
#include "launch.hpp"

namespace qlinear {

namespace {

constexpr int kQThreads = 256;

template <int DT>
__device__ __forceinline__ void load32(const void* x, size_t base, float (&v)[32]) {
  if constexpr (DT == kF32) {
    const u32x4* p = (const u32x4*)((const float*)x + base);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const u32x4 w = p[c];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // copy the element out first: bit_cast of a vector subscript reads the vector's first bytes
        const uint32_t bits = w[e];
        v[4 * c + e] = __builtin_bit_cast(float, bits);
      }
    }
  } else {
    const u32x4* p = (const u32x4*)((const uint16_t*)x + base);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const u32x4 w = p[c];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t lo = w[e] & 0xFFFFu, hi = w[e] >> 16;
        v[8 * c + 2 * e] = DT == kBF16 ? bf16_bits_to_f32(lo) : f16_bits_to_f32(lo);
        v[8 * c + 2 * e + 1] = DT == kBF16 ? bf16_bits_to_f32(hi) : f16_bits_to_f32(hi);
      }
    }
  }
}

template <int DT>
__global__ __launch_bounds__(kQThreads) void quantize_int4_kernel(const void* __restrict__ x,
                                                                  u32x4* __restrict__ packed,
                                                                  float* __restrict__ scale,
                                                                  long long blocks, int rule) {
  const long long b = (long long)blockIdx.x * kQThreads + threadIdx.x;
  if (b >= blocks) return;
  float v[32];
  load32<DT>(x, (size_t)b * 32, v);
  float amax = 0.0f;
#pragma unroll
  for (int e = 0; e < 32; ++e) amax = fmaxf(amax, fabsf(v[e]));
  amax = fmaxf(amax, 1e-8f);
  const float s = rule == 0 ? __fdiv_rn(amax, 7.0f) : __fmul_rn(amax, 1.0f / 7.0f);
  const float rcp = __fdiv_rn(1.0f, s);
  u32x4 out = {0u, 0u, 0u, 0u};
  float qv[32];
  rint_quot_n<32>(v, s, rcp, qv);
#pragma unroll
  for (int e = 0; e < 32; ++e) {
    const float q = fminf(fmaxf(qv[e], -8.0f), 7.0f);
    out[e / 8] |= ((uint32_t)(int)q & 0xFu) << (4 * (e % 8));
  }
  packed[b] = out;
  scale[b] = s;
}

template <int DT>
__global__ __launch_bounds__(kQThreads) void quantize_int8_row_kernel(const void* __restrict__ x,
                                                                      int8_t* __restrict__ q,
                                                                      float* __restrict__ scale,
                                                                      int K) {
  __shared__ float red[kQThreads / kWave];
  const int row = blockIdx.x;
  const size_t base = (size_t)row * K;
  float amax = 0.0f;
  for (int k = threadIdx.x; k < K; k += kQThreads) amax = fmaxf(amax, fabsf(read_elem(x, DT, base + k)));
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, kWave));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = red[0];
#pragma unroll
  for (int w = 1; w < kQThreads / kWave; ++w) amax = fmaxf(amax, red[w]);
  const float s = __fmul_rn(fmaxf(amax, 1e-8f), 1.0f / 127.0f);
  if (threadIdx.x == 0) scale[row] = s;
  const float rcp = __fdiv_rn(1.0f, s);
  for (int k = threadIdx.x; k < K; k += kQThreads) {
    const float v = read_elem(x, DT, base + k);
    float qv;
    rint_quot_n<1>(&v, s, rcp, &qv);
    q[base + k] = (int8_t)(int)fminf(fmaxf(qv, -127.0f), 127.0f);
  }
}

// Same rule, for K % 8 == 0 and K <= 8 * kQThreads * kQ8Vec: each thread reads its 8-element
// vectors once (16-byte loads for 16-bit x) and keeps them in registers between the row maximum
// and the quantize pass; 8 codes leave as one 8-byte store.
constexpr int kQ8Vec = 8;
template <int DT>
__global__ __launch_bounds__(kQThreads) void quantize_int8_row_vec_kernel(const void* __restrict__ x,
                                                                          int8_t* __restrict__ q,
                                                                          float* __restrict__ scale, int K) {
  __shared__ float red[kQThreads / kWave];
  const int row = blockIdx.x;
  const size_t base = (size_t)row * K;
  const int nv = K / 8;
  float v[kQ8Vec][8];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < kQ8Vec; ++i) {
    const int vi = threadIdx.x + i * kQThreads;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[i][e] = 0.0f;
    if (vi < nv) {
      if constexpr (DT == kF32) {
        const u32x4 lo = *(const u32x4*)((const float*)x + base + 8 * vi);
        const u32x4 hi = *(const u32x4*)((const float*)x + base + 8 * vi + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t a = lo[e], b = hi[e];
          v[i][e] = __builtin_bit_cast(float, a);
          v[i][4 + e] = __builtin_bit_cast(float, b);
        }
      } else {
        const u32x4 w = *(const u32x4*)((const uint16_t*)x + base + 8 * vi);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t lo = w[e] & 0xFFFFu, hi = w[e] >> 16;
          v[i][2 * e] = DT == kBF16 ? bf16_bits_to_f32(lo) : f16_bits_to_f32(lo);
          v[i][2 * e + 1] = DT == kBF16 ? bf16_bits_to_f32(hi) : f16_bits_to_f32(hi);
        }
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[i][e]));
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, kWave));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = red[0];
#pragma unroll
  for (int w = 1; w < kQThreads / kWave; ++w) amax = fmaxf(amax, red[w]);
  const float s = __fmul_rn(fmaxf(amax, 1e-8f), 1.0f / 127.0f);
  if (threadIdx.x == 0) scale[row] = s;
  const float rcp = __fdiv_rn(1.0f, s);
#pragma unroll
  for (int i = 0; i < kQ8Vec; ++i) {
    const int vi = threadIdx.x + i * kQThreads;
    if (vi < nv) {
      uint32_t lo = 0, hi = 0;
      float qv[8];
      rint_quot_n<8>(v[i], s, rcp, qv);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t c = (uint32_t)(int)fminf(fmaxf(qv[e], -127.0f), 127.0f) & 0xFFu;
        if (e < 4)
          lo |= c << (8 * e);
        else
          hi |= c << (8 * (e - 4));
      }
      typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
      *(u32x2*)(q + base + 8 * vi) = u32x2{lo, hi};
    }
  }
}

// ggml Q4_0 -> native layout, one thread per 32-element block: the 18-byte block (fp16 d, then
// 16 bytes whose byte i holds elements i (low nibble) and i + 16 (high nibble) as q + 8) becomes
// 16 bytes of two's-complement nibbles in element order (byte j = elements 2j | 2j+1 << 4) and
// the fp32 scale d (exact widening). Blocks are only 2-byte aligned: read as 9 halfwords.
__global__ __launch_bounds__(kQThreads) void repack_q4_0_kernel(const uint16_t* __restrict__ raw,
                                                                u32x4* __restrict__ packed,
                                                                float* __restrict__ scale, long long blocks) {
  const long long b = (long long)blockIdx.x * kQThreads + threadIdx.x;
  if (b >= blocks) return;
  const uint16_t* src = raw + b * 9;
  uint32_t e[32];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t hw = src[1 + i];  // bytes 2i, 2i+1 of the quants
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const uint32_t byte = (hw >> (8 * k)) & 0xFFu;
      e[2 * i + k] = ((byte & 0xFu) - 8u) & 0xFu;          // element 2i + k
      e[2 * i + k + 16] = (((byte >> 4) & 0xFu) - 8u) & 0xFu;  // element 2i + k + 16
    }
  }
  u32x4 out = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int j = 0; j < 32; ++j) out[j / 8] |= e[j] << (4 * (j % 8));
  packed[b] = out;
  scale[b] = f16_bits_to_f32(src[0]);
}

// Block-32 int8 quantize, the reference's quantize_int8_kernel rule (csrc/int8_gemm.hip:215-246):
// one thread per 32-element block, s = max(amax, 1e-8) * (1/127), q = clamp(rint(v / s), -127, 127),
// the block read with 16-byte loads and its 32 codes written as two 16-byte stores.
template <int DT>
__global__ __launch_bounds__(kQThreads) void quantize_int8_block32_kernel(const void* __restrict__ x,
                                                                          int8_t* __restrict__ q,
                                                                          float* __restrict__ scale, long blocks) {
  const long b = (long)blockIdx.x * kQThreads + threadIdx.x;
  if (b >= blocks) return;
  const size_t base = (size_t)b * 32;
  float v[32];
  if constexpr (DT == kF32) {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const u32x4 w = *(const u32x4*)((const float*)x + base + 4 * c);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t bits = w[e];
        v[4 * c + e] = __builtin_bit_cast(float, bits);
      }
    }
  } else {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const u32x4 w = *(const u32x4*)((const uint16_t*)x + base + 8 * c);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t lo = w[e] & 0xFFFFu, hi = w[e] >> 16;
        v[8 * c + 2 * e] = DT == kBF16 ? bf16_bits_to_f32(lo) : f16_bits_to_f32(lo);
        v[8 * c + 2 * e + 1] = DT == kBF16 ? bf16_bits_to_f32(hi) : f16_bits_to_f32(hi);
      }
    }
  }
  float amax = 0.0f;
#pragma unroll
  for (int e = 0; e < 32; ++e) amax = fmaxf(amax, fabsf(v[e]));
  const float s = __fmul_rn(fmaxf(amax, 1e-8f), 1.0f / 127.0f);
  const float rcp = __fdiv_rn(1.0f, s);
  u32x4 out[2];
  float qv[32];
  rint_quot_n<32>(v, s, rcp, qv);
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    uint32_t word = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int c = (int)fminf(fmaxf(qv[4 * w + e], -127.0f), 127.0f);
      word |= (uint32_t)(c & 0xFF) << (8 * e);
    }
    out[w >> 2][w & 3] = word;
  }
  *(u32x4*)(q + base) = out[0];
  *(u32x4*)(q + base + 16) = out[1];
  scale[b] = s;
}

}  // namespace

hipError_t repack_q4_0_launch(const void* raw, void* packed, float* scale, int64_t blocks, hipStream_t stream) {
  const dim3 grid((unsigned)((blocks + kQThreads - 1) / kQThreads));
  hipLaunchKernelGGL(repack_q4_0_kernel, grid, dim3(kQThreads), 0, stream, (const uint16_t*)raw, (u32x4*)packed, scale,
                     (long long)blocks);
  return hipGetLastError();
}

hipError_t quantize_int4_launch(int dtype, int rule, const void* x, void* packed, float* scale,
                                int64_t rows, int64_t K, hipStream_t stream) {
  const long long blocks = (long long)rows * (K / 32);
  const dim3 grid((unsigned)((blocks + kQThreads - 1) / kQThreads));
  switch (dtype) {
    case kF32:
      hipLaunchKernelGGL(quantize_int4_kernel<kF32>, grid, dim3(kQThreads), 0, stream, x, (u32x4*)packed,
                         scale, blocks, rule);
      break;
    case kF16:
      hipLaunchKernelGGL(quantize_int4_kernel<kF16>, grid, dim3(kQThreads), 0, stream, x, (u32x4*)packed,
                         scale, blocks, rule);
      break;
    default:
      hipLaunchKernelGGL(quantize_int4_kernel<kBF16>, grid, dim3(kQThreads), 0, stream, x, (u32x4*)packed,
                         scale, blocks, rule);
      break;
  }
  return hipGetLastError();
}

hipError_t quantize_int8_per_token_launch(int dtype, const void* x, int8_t* q, float* scale, int64_t M,
                                          int64_t K, hipStream_t stream) {
  const dim3 grid((unsigned)M);
  // 16-byte loads need 16-byte aligned rows: K % 8 == 0 and an aligned base (checked by the caller)
  if (K % 8 == 0 && K <= 8 * kQThreads * kQ8Vec && ((uintptr_t)x & 15) == 0 && ((uintptr_t)q & 7) == 0) {
    switch (dtype) {
      case kF32:
        hipLaunchKernelGGL(quantize_int8_row_vec_kernel<kF32>, grid, dim3(kQThreads), 0, stream, x, q, scale, (int)K);
        break;
      case kF16:
        hipLaunchKernelGGL(quantize_int8_row_vec_kernel<kF16>, grid, dim3(kQThreads), 0, stream, x, q, scale, (int)K);
        break;
      default:
        hipLaunchKernelGGL(quantize_int8_row_vec_kernel<kBF16>, grid, dim3(kQThreads), 0, stream, x, q, scale,
                           (int)K);
        break;
    }
    return hipGetLastError();
  }
  switch (dtype) {
    case kF32:
      hipLaunchKernelGGL(quantize_int8_row_kernel<kF32>, grid, dim3(kQThreads), 0, stream, x, q, scale, (int)K);
      break;
    case kF16:
      hipLaunchKernelGGL(quantize_int8_row_kernel<kF16>, grid, dim3(kQThreads), 0, stream, x, q, scale, (int)K);
      break;
    default:
      hipLaunchKernelGGL(quantize_int8_row_kernel<kBF16>, grid, dim3(kQThreads), 0, stream, x, q, scale, (int)K);
      break;
  }
  return hipGetLastError();
}

hipError_t quantize_int8_block32_launch(int dtype, const void* x, int8_t* q, float* scale, int64_t blocks,
                                       hipStream_t stream) {
  const dim3 grid((unsigned)((blocks + kQThreads - 1) / kQThreads));
  switch (dtype) {
    case kF32:
      hipLaunchKernelGGL(quantize_int8_block32_kernel<kF32>, grid, dim3(kQThreads), 0, stream, x, q, scale, (long)blocks);
      break;
    case kF16:
      hipLaunchKernelGGL(quantize_int8_block32_kernel<kF16>, grid, dim3(kQThreads), 0, stream, x, q, scale, (long)blocks);
      break;
    default:
      hipLaunchKernelGGL(quantize_int8_block32_kernel<kBF16>, grid, dim3(kQThreads), 0, stream, x, q, scale,
                         (long)blocks);
      break;
  }
  return hipGetLastError();
}

}  // namespace qlinear
