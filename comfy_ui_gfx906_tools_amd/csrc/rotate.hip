// Activation rotation fused into the fp16 staging pass (gfx950): for a layer whose weights were
// folded through the block-diagonal rotation R = H diag(signs) / sqrt(g) (Sylvester Hadamard H of
// order g, nodes/ComfyUI-Gfx906Int4/ops.py:43-105), the activation of the forward must be rotated
// the same way, y = x_g R^T per group of g along K. Instead of the reference's fp32 matmul
// (ops.py:176-179) this pass computes, per row, y_g = H (signs * x_g) / sqrt(g) with a fast
// Walsh-Hadamard transform in registers and DPP lane moves, and writes y directly as the row-scaled
// fp16 operand of the W4A16 GEMM (x16 = y * 2^-e, row_scale = 2^e, max |y| * 2^-e in
// [2^14, 2^15) before the fp16 rounding), so the rotation costs one HBM pass.
//
// One 256-thread block per row; thread t holds elements 8t + 2048 r (r < R). Butterfly strides
// 1, 2, 4 are inside a thread's 8 values, strides 8 .. g/2 pair thread t with t ^ (stride / 8)
// by DPP moves (a group spans g / 8 <= 16 aligned threads: within one 16-lane DPP row). K % g == 0,
// so a group is either wholly inside the row or wholly past it; the exchanges run on every lane.
#include "common.hpp"
#include "launch.hpp"

namespace qlinear {

namespace {

template <int DT>
__device__ __forceinline__ void load8_row(const void* p, size_t i, float (&v)[8]) {
  if constexpr (DT == kF32) {
    const f32x4 lo = *(const f32x4*)((const float*)p + i);
    const f32x4 hi = *(const f32x4*)((const float*)p + i + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = lo[e];
      v[4 + e] = hi[e];
    }
  } else {
    const u32x4 w = *(const u32x4*)((const uint16_t*)p + i);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t word = w[e];
      v[2 * e] = DT == kBF16 ? bf16_bits_to_f32(word & 0xFFFFu) : f16_bits_to_f32(word & 0xFFFFu);
      v[2 * e + 1] = DT == kBF16 ? bf16_bits_to_f32(word >> 16) : f16_bits_to_f32(word >> 16);
    }
  }
}

// Value of lane t ^ D (D = 1, 2, 4, 8; within a 16-lane DPP row) by DPP moves, no LDS round trip:
// xor 1 and xor 2 are quad permutations; xor 4 = (xor 7: row_half_mirror) then (xor 3: quad
// [3,2,1,0]); xor 8 = (xor 15: row_mirror) then (xor 7: row_half_mirror).
template <int kCtrl>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, 0xF, 0xF, false));
}
template <int D>
__device__ __forceinline__ float lane_xor(float v) {
  if constexpr (D == 1) return dpp_mov<0xB1>(v);
  else if constexpr (D == 2) return dpp_mov<0x4E>(v);
  else if constexpr (D == 4) return dpp_mov<0x1B>(dpp_mov<0x141>(v));
  else return dpp_mov<0x141>(dpp_mov<0x140>(v));
}

template <int XDT, int G, int R>
__global__ __launch_bounds__(256) void rotate_rows_to_f16_kernel(const void* __restrict__ x,
                                                                 const float* __restrict__ signs,
                                                                 _Float16* __restrict__ x16,
                                                                 float* __restrict__ row_scale, int K,
                                                                 float inv_sqrt_g) {
  __shared__ float red[4];
  const int t = threadIdx.x;
  const size_t base = (size_t)blockIdx.x * K;
  // the signs of this thread's 8 positions within their group (2048 is a multiple of G)
  float sg[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) sg[e] = signs[(8 * t) % G + e];
  float v[R][8];
  float amax = 0.0f;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int k = 8 * t + 2048 * r;
    if (k < K) {
      load8_row<XDT>(x, base + k, v[r]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[r][e] = 0.0f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) v[r][e] *= sg[e];
    // strides 1, 2, 4 within the thread: (a, b) -> (a + b, a - b)
#pragma unroll
    for (int h = 1; h < 8; h <<= 1)
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (!(e & h)) {
          const float a = v[r][e], b = v[r][e + h];
          v[r][e] = a + b;
          v[r][e + h] = a - b;
        }
    // strides 8 .. G/2 across threads t and t ^ d, d = stride / 8: the lower thread keeps a + b,
    // the upper one a - b (a = the lower thread's value)
    static_for<0, 4>([&](auto sc) {
      constexpr int d = 1 << decltype(sc)::value;
      if constexpr (d < G / 8) {
        const bool upper = (t & d) != 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float other = lane_xor<d>(v[r][e]);
          v[r][e] = upper ? other - v[r][e] : v[r][e] + other;
        }
      }
    });
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      v[r][e] *= inv_sqrt_g;
      if (k < K) amax = fmaxf(amax, fabsf(v[r][e]));
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, kWave));
  if ((t & 63) == 0) red[t >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  int ex = 0;
  if (amax > 0.0f && amax <= 3.0e38f) {
    int E;
    frexpf(amax, &E);  // amax = f * 2^E, f in [0.5, 1)
    ex = E - 15;
  }
  if (t == 0) row_scale[blockIdx.x] = ldexpf(1.0f, ex);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int k = 8 * t + 2048 * r;
    if (k < K) {
      u32x4 o;
#pragma unroll
      for (int q = 0; q < 4; ++q) o[q] = pack2_f16(ldexpf(v[r][2 * q], -ex), ldexpf(v[r][2 * q + 1], -ex));
      *(u32x4*)(x16 + base + k) = o;
    }
  }
}

template <int XDT, int G>
hipError_t rotate_launch_r(const void* x, const float* signs, void* x16, float* rs, int64_t M, int64_t K,
                           hipStream_t st) {
  const dim3 grid((unsigned)M), block(256);
  const float inv = (float)(1.0 / __builtin_sqrt((double)G));
  if (K <= 2048)
    hipLaunchKernelGGL((rotate_rows_to_f16_kernel<XDT, G, 1>), grid, block, 0, st, x, signs, (_Float16*)x16, rs,
                       (int)K, inv);
  else if (K <= 4096)
    hipLaunchKernelGGL((rotate_rows_to_f16_kernel<XDT, G, 2>), grid, block, 0, st, x, signs, (_Float16*)x16, rs,
                       (int)K, inv);
  else if (K <= 8192)
    hipLaunchKernelGGL((rotate_rows_to_f16_kernel<XDT, G, 4>), grid, block, 0, st, x, signs, (_Float16*)x16, rs,
                       (int)K, inv);
  else
    hipLaunchKernelGGL((rotate_rows_to_f16_kernel<XDT, G, 8>), grid, block, 0, st, x, signs, (_Float16*)x16, rs,
                       (int)K, inv);
  return hipGetLastError();
}

template <int XDT>
hipError_t rotate_launch_g(int group, const void* x, const float* signs, void* x16, float* rs, int64_t M, int64_t K,
                           hipStream_t st) {
  switch (group) {
    case 32: return rotate_launch_r<XDT, 32>(x, signs, x16, rs, M, K, st);
    case 64: return rotate_launch_r<XDT, 64>(x, signs, x16, rs, M, K, st);
    default: return rotate_launch_r<XDT, 128>(x, signs, x16, rs, M, K, st);
  }
}

}  // namespace

hipError_t rotate_rows_to_f16_launch(int x_dtype, int group, const void* x, const float* signs, void* x16,
                                     float* row_scale, int64_t M, int64_t K, hipStream_t stream) {
  switch (x_dtype) {
    case kF32: return rotate_launch_g<kF32>(group, x, signs, x16, row_scale, M, K, stream);
    case kF16: return rotate_launch_g<kF16>(group, x, signs, x16, row_scale, M, K, stream);
    default: return rotate_launch_g<kBF16>(group, x, signs, x16, row_scale, M, K, stream);
  }
}

}  // namespace qlinear
