// Fused DiT block glue around the W4A16 linears (gfx950, wave64): the element-wise work a
// Flux-style block does between its projections, one HBM pass each instead of a chain of
// torch ops with fp32 intermediates.
//
//  * adaln_to_f16_kernel: LayerNorm (no affine) of a row, then (1 + scale) * y + shift, written
//    as the row-scaled fp16 operand of the W4A16 GEMM (the format of rows_to_scaled_f16_kernel:
//    max |y| * 2^-e in [2^14, 2^15) before the fp16 rounding, row_scale = 2^e), as the plain row,
//    or as the per-token int8 operand of the W8A8 GEMM.
//  * qk_norm_rope_kernel: splits a qkv projection [L, 3, H, D] into q, k, v [H, L_out, D] at row
//    offset l0, with RMSNorm over D (learned scale) and the RoPE pair rotation on q and k.
//  * gated_residual_kernel: out = x + gate * y with gate broadcast over rows.
//  * heads_to_f16_kernel: rows of an attention output in the head-major layout [H, L, D], optionally
//    followed by the same row of a second [L, E] tensor, gathered into the row-scaled fp16 operand
//    of the next GEMM (the head transpose, a concatenation and the staging pass in one).
//
// Every value is computed in fp32 and rounded once to the output type.
#include "common.hpp"
#include "launch.hpp"

#include <algorithm>

namespace qlinear {
namespace {

template <int DT>
__device__ __forceinline__ void load8(const void* p, size_t i, float (&v)[8]) {
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

template <int DT>
__device__ __forceinline__ void store8(void* p, size_t i, const float (&v)[8]) {
  if constexpr (DT == kF32) {
    f32x4 lo, hi;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      lo[e] = v[e];
      hi[e] = v[4 + e];
    }
    *(f32x4*)((float*)p + i) = lo;
    *(f32x4*)((float*)p + i + 4) = hi;
  } else {
    u32x4 w;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      w[e] = DT == kBF16 ? pack2_bf16(v[2 * e], v[2 * e + 1]) : pack2_f16(v[2 * e], v[2 * e + 1]);
    *(u32x4*)((uint16_t*)p + i) = w;
  }
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

// Sum over the 256-thread block (4 waves) in a fixed order; `red` is this reduction's own
// 4-slot array, so successive reductions need no barrier between them.
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}
__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// One 256-thread block per row; thread t holds elements 8t + 2048 r (r < R) in registers, so the
// row is read from HBM once. K % 8 == 0, K <= 2048 R. OUT: kOperandF16 the row-scaled fp16 operand
// of the W4A16 GEMM, kOperandPlain the row in x's dtype, kOperandI8 the per-token int8 operand of the
// W8A8 GEMM: the row rounded to x's dtype, then quantized by qlinear_quantize_int8_per_token's
// rule (s = fl(max(amax, 1e-8) * fl(1/127)), q = clamp(rint(v / s), -127, 127), IEEE division),
// row_scale[m] = s.
template <int XDT, int MDT, int R, int OUT>
__global__ __launch_bounds__(256) void adaln_to_f16_kernel(const void* __restrict__ x, const void* __restrict__ shift,
                                                           const void* __restrict__ scale, void* __restrict__ out,
                                                           float* __restrict__ row_scale, int K, float eps) {
  __shared__ float red[3][4];
  const size_t base = (size_t)blockIdx.x * K;
  float v[R][8];
  float s = 0.0f;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int k = threadIdx.x * 8 + r * 2048;
    if (k < K) {
      load8<XDT>(x, base + k, v[r]);
#pragma unroll
      for (int e = 0; e < 8; ++e) s += v[r][e];
    }
  }
  const float mean = block_sum(s, red[0]) / (float)K;
  float q = 0.0f;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int k = threadIdx.x * 8 + r * 2048;
    if (k < K) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = v[r][e] - mean;
        q += d * d;
      }
    }
  }
  const float rstd = 1.0f / sqrtf(block_sum(q, red[1]) / (float)K + eps);
  float amax = 0.0f;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int k = threadIdx.x * 8 + r * 2048;
    if (k < K) {
      float sh[8], sc[8];
      load8<MDT>(shift, k, sh);
      load8<MDT>(scale, k, sc);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v[r][e] = (v[r][e] - mean) * rstd * (1.0f + sc[e]) + sh[e];
        if constexpr (OUT == kOperandI8) v[r][e] = round_to(XDT, v[r][e]);
        amax = fmaxf(amax, fabsf(v[r][e]));
      }
    }
  }
  if constexpr (OUT == kOperandPlain) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int k = threadIdx.x * 8 + r * 2048;
      if (k < K) store8<XDT>(out, base + k, v[r]);
    }
    return;
  }
  amax = block_max(amax, red[2]);
  if constexpr (OUT == kOperandI8) {
    const float s = __fmul_rn(fmaxf(amax, 1e-8f), 1.0f / 127.0f);
    if (threadIdx.x == 0) row_scale[blockIdx.x] = s;
    const float rcp = __fdiv_rn(1.0f, s);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int k = threadIdx.x * 8 + r * 2048;
      if (k < K) {
        uint32_t w[2] = {0u, 0u};
        float qv[8];
        rint_quot_n<8>(v[r], s, rcp, qv);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int c = (int)fminf(fmaxf(qv[e], -127.0f), 127.0f);
          w[e >> 2] |= ((uint32_t)c & 0xFFu) << (8 * (e & 3));
        }
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        *(u32x2*)((int8_t*)out + base + k) = u32x2{w[0], w[1]};
      }
    }
    return;
  }
  int ex = 0;
  if (amax > 0.0f && amax <= 3.0e38f) {
    int E;
    frexpf(amax, &E);  // amax = f * 2^E, f in [0.5, 1)
    ex = E - 15;
  }
  if (threadIdx.x == 0) row_scale[blockIdx.x] = ldexpf(1.0f, ex);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int k = threadIdx.x * 8 + r * 2048;
    if (k < K) {
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = ldexpf(v[r][e], -ex);
      store8<kF16>(out, base + k, o);
    }
  }
}

// One wave per (token l, head h); lane j holds the pair (2j, 2j + 1) of the 128-wide head, which is
// also the RoPE pair. q and k: y = x * rsqrt(mean(x^2) + eps) * norm_scale, then
// (y0, y1) -> (c y0 - s y1, s y0 + c y1) with c, s = cos/sin[l0 + l][j]; v is copied.
template <int DT>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(const void* __restrict__ qkv, const void* __restrict__ qn,
                                                           const void* __restrict__ kn, const float* __restrict__ cosv,
                                                           const float* __restrict__ sinv, void* __restrict__ qo,
                                                           void* __restrict__ ko, void* __restrict__ vo, int L, int H,
                                                           int L_out, int l0, float eps) {
  constexpr int D = 128;
  const int lane = threadIdx.x & 63;
  const long w = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (w >= (long)L * H) return;  // whole waves exit together: no barrier below
  const int l = (int)(w / H), h = (int)(w % H);
  const size_t in_row = (size_t)l * 3 * H * D + (size_t)h * D + 2 * lane;
  const size_t out_row = ((size_t)h * L_out + (size_t)(l0 + l)) * D + 2 * lane;
  const float c = cosv[(size_t)(l0 + l) * (D / 2) + lane];
  const float s = sinv[(size_t)(l0 + l) * (D / 2) + lane];
  const uint16_t* in = (const uint16_t*)qkv;
  auto to_f = [](uint32_t b) { return DT == kBF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b); };
  auto pack = [](float a, float b) { return DT == kBF16 ? pack2_bf16(a, b) : pack2_f16(a, b); };
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const uint32_t word = *(const uint32_t*)(in + in_row + (size_t)t * H * D);
    const float x0 = to_f(word & 0xFFFFu), x1 = to_f(word >> 16);
    const float ms = wave_sum(x0 * x0 + x1 * x1) / (float)D;
    const float rs = 1.0f / sqrtf(ms + eps);
    const uint32_t nw = *(const uint32_t*)((const uint16_t*)(t == 0 ? qn : kn) + 2 * lane);
    const float y0 = x0 * rs * to_f(nw & 0xFFFFu), y1 = x1 * rs * to_f(nw >> 16);
    *(uint32_t*)((uint16_t*)(t == 0 ? qo : ko) + out_row) = pack(c * y0 - s * y1, s * y0 + c * y1);
  }
  *(uint32_t*)((uint16_t*)vo + out_row) = *(const uint32_t*)(in + in_row + (size_t)2 * H * D);
}

// out[m, k] = x[m, k] + gate[k] * y[m, k] (out may be x); 8 elements per thread, grid-stride over
// M * K / 8 chunks, each read and written by one thread.
template <int DT>
__global__ __launch_bounds__(256) void gated_residual_kernel(void* out, const void* x, const void* __restrict__ gate,
                                                             const void* __restrict__ y, long chunks, int K) {
  for (long c = (long)blockIdx.x * 256 + threadIdx.x; c < chunks; c += (long)gridDim.x * 256) {
    const size_t i = (size_t)c * 8;
    const int k = (int)(i % (size_t)K);
    float a[8], g[8], b[8];
    load8<DT>(x, i, a);
    load8<DT>(gate, k, g);
    load8<DT>(y, i, b);
#pragma unroll
    for (int e = 0; e < 8; ++e) a[e] = a[e] + g[e] * b[e];
    store8<DT>(out, i, a);
  }
}

// One 256-thread block per output row l; thread t holds row elements 8t + 2048 r (r < R): element
// p < H * 128 is o[p / 128, l0 + l, p % 128], element p >= H * 128 is extra[l, p - H * 128].
// OUT as for adaln_to_f16_kernel: the row-scaled fp16 operand, the gathered row itself (DT), or
// the per-token int8 operand (the gathered values are the inputs themselves, so no rounding comes
// first).
template <int DT, int R, int OUT>
__global__ __launch_bounds__(256) void heads_to_f16_kernel(const void* __restrict__ o, const void* __restrict__ extra,
                                                           void* __restrict__ out, float* __restrict__ row_scale,
                                                           int H, int L_all, int l0, int E) {
  constexpr int D = 128;
  __shared__ float red[4];
  const int l = blockIdx.x;
  const int HD = H * D, Kt = HD + E;
  float v[R][8];
  float amax = 0.0f;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int p = threadIdx.x * 8 + r * 2048;
    if (p < Kt) {
      if (p < HD)
        load8<DT>(o, ((size_t)(p / D) * L_all + (size_t)(l0 + l)) * D + (p % D), v[r]);
      else
        load8<DT>(extra, (size_t)l * E + (p - HD), v[r]);
#pragma unroll
      for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[r][e]));
    }
  }
  if constexpr (OUT == kOperandPlain) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int p = threadIdx.x * 8 + r * 2048;
      if (p < Kt) store8<DT>(out, (size_t)l * Kt + p, v[r]);
    }
    return;
  }
  amax = block_max(amax, red);
  if constexpr (OUT == kOperandI8) {  // the rule of qlinear_quantize_int8_per_token
    const float s = __fmul_rn(fmaxf(amax, 1e-8f), 1.0f / 127.0f);
    if (threadIdx.x == 0) row_scale[l] = s;
    const float rcp = __fdiv_rn(1.0f, s);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int p = threadIdx.x * 8 + r * 2048;
      if (p < Kt) {
        uint32_t w[2] = {0u, 0u};
        float qv[8];
        rint_quot_n<8>(v[r], s, rcp, qv);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int c = (int)fminf(fmaxf(qv[e], -127.0f), 127.0f);
          w[e >> 2] |= ((uint32_t)c & 0xFFu) << (8 * (e & 3));
        }
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        *(u32x2*)((int8_t*)out + (size_t)l * Kt + p) = u32x2{w[0], w[1]};
      }
    }
    return;
  }
  int ex = 0;
  if (amax > 0.0f && amax <= 3.0e38f) {
    int E2;
    frexpf(amax, &E2);  // amax = f * 2^E2, f in [0.5, 1)
    ex = E2 - 15;
  }
  if (threadIdx.x == 0) row_scale[l] = ldexpf(1.0f, ex);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int p = threadIdx.x * 8 + r * 2048;
    if (p < Kt) {
      float q[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) q[e] = ldexpf(v[r][e], -ex);
      store8<kF16>(out, (size_t)l * Kt + p, q);
    }
  }
}

template <int XDT, int MDT, int OUT>
hipError_t adaln_launch_r(const void* x, const void* shift, const void* scale, void* out, float* rs, int64_t M,
                          int64_t K, float eps, hipStream_t st) {
  const dim3 grid((unsigned)M), block(256);
  if (K <= 2048)
    hipLaunchKernelGGL((adaln_to_f16_kernel<XDT, MDT, 1, OUT>), grid, block, 0, st, x, shift, scale, out, rs, (int)K,
                       eps);
  else if (K <= 4096)
    hipLaunchKernelGGL((adaln_to_f16_kernel<XDT, MDT, 2, OUT>), grid, block, 0, st, x, shift, scale, out, rs, (int)K,
                       eps);
  else if (K <= 8192)
    hipLaunchKernelGGL((adaln_to_f16_kernel<XDT, MDT, 4, OUT>), grid, block, 0, st, x, shift, scale, out, rs, (int)K,
                       eps);
  else
    hipLaunchKernelGGL((adaln_to_f16_kernel<XDT, MDT, 8, OUT>), grid, block, 0, st, x, shift, scale, out, rs, (int)K,
                       eps);
  return hipGetLastError();
}

template <int XDT, int OUT>
hipError_t adaln_launch_x(int mod_dtype, const void* x, const void* shift, const void* scale, void* out, float* rs,
                          int64_t M, int64_t K, float eps, hipStream_t st) {
  switch (mod_dtype) {
    case kF32: return adaln_launch_r<XDT, kF32, OUT>(x, shift, scale, out, rs, M, K, eps, st);
    case kF16: return adaln_launch_r<XDT, kF16, OUT>(x, shift, scale, out, rs, M, K, eps, st);
    default: return adaln_launch_r<XDT, kBF16, OUT>(x, shift, scale, out, rs, M, K, eps, st);
  }
}

template <int OUT>
hipError_t adaln_launch_o(int x_dtype, int mod_dtype, const void* x, const void* shift, const void* scale, void* out,
                          float* row_scale, int64_t M, int64_t K, float eps, hipStream_t stream) {
  switch (x_dtype) {
    case kF32: return adaln_launch_x<kF32, OUT>(mod_dtype, x, shift, scale, out, row_scale, M, K, eps, stream);
    case kF16: return adaln_launch_x<kF16, OUT>(mod_dtype, x, shift, scale, out, row_scale, M, K, eps, stream);
    default: return adaln_launch_x<kBF16, OUT>(mod_dtype, x, shift, scale, out, row_scale, M, K, eps, stream);
  }
}

}  // namespace

hipError_t adaln_launch(int out_kind, int x_dtype, int mod_dtype, const void* x, const void* shift, const void* scale,
                        void* out, float* row_scale, int64_t M, int64_t K, float eps, hipStream_t stream) {
  switch (out_kind) {
    case kOperandF16: return adaln_launch_o<kOperandF16>(x_dtype, mod_dtype, x, shift, scale, out, row_scale, M, K, eps, stream);
    case kOperandPlain:
      return adaln_launch_o<kOperandPlain>(x_dtype, mod_dtype, x, shift, scale, out, row_scale, M, K, eps, stream);
    case kOperandI8: return adaln_launch_o<kOperandI8>(x_dtype, mod_dtype, x, shift, scale, out, row_scale, M, K, eps, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t qk_norm_rope_launch(int dtype, const void* qkv, const void* q_norm, const void* k_norm, const float* cosv,
                               const float* sinv, void* q, void* k, void* v, int64_t L, int64_t H, int64_t L_out,
                               int64_t l0, float eps, hipStream_t stream) {
  const long waves = (long)L * H;
  const dim3 grid((unsigned)((waves + 3) / 4)), block(256);
  if (dtype == kBF16)
    hipLaunchKernelGGL(qk_norm_rope_kernel<kBF16>, grid, block, 0, stream, qkv, q_norm, k_norm, cosv, sinv, q, k, v,
                       (int)L, (int)H, (int)L_out, (int)l0, eps);
  else
    hipLaunchKernelGGL(qk_norm_rope_kernel<kF16>, grid, block, 0, stream, qkv, q_norm, k_norm, cosv, sinv, q, k, v,
                       (int)L, (int)H, (int)L_out, (int)l0, eps);
  return hipGetLastError();
}

template <int DT, int OUT>
static hipError_t heads_launch_r(const void* o, const void* extra, void* x16, float* rs, int64_t H, int64_t L_all,
                                 int64_t l0, int64_t rows, int64_t E, hipStream_t st) {
  const int64_t Kt = H * 128 + E;
  const dim3 grid((unsigned)rows), block(256);
#define QL_HEADS(R)                                                                                       \
  hipLaunchKernelGGL((heads_to_f16_kernel<DT, R, OUT>), grid, block, 0, st, o, extra, x16, rs, (int)H, (int)L_all, \
                     (int)l0, (int)E)
  if (Kt <= 2048)
    QL_HEADS(1);
  else if (Kt <= 4096)
    QL_HEADS(2);
  else if (Kt <= 8192)
    QL_HEADS(4);
  else
    QL_HEADS(8);
#undef QL_HEADS
  return hipGetLastError();
}

template <int OUT>
static hipError_t heads_launch_o(int dtype, const void* o, int64_t H, int64_t L_all, int64_t l0, int64_t rows,
                                 const void* extra, int64_t E, void* out, float* row_scale, hipStream_t stream) {
  return dtype == kBF16 ? heads_launch_r<kBF16, OUT>(o, extra, out, row_scale, H, L_all, l0, rows, E, stream)
                        : heads_launch_r<kF16, OUT>(o, extra, out, row_scale, H, L_all, l0, rows, E, stream);
}

hipError_t heads_gather_launch(int out_kind, int dtype, const void* o, int64_t H, int64_t L_all, int64_t l0,
                               int64_t rows, const void* extra, int64_t E, void* out, float* row_scale,
                               hipStream_t stream) {
  switch (out_kind) {
    case kOperandF16: return heads_launch_o<kOperandF16>(dtype, o, H, L_all, l0, rows, extra, E, out, row_scale, stream);
    case kOperandPlain:
      return heads_launch_o<kOperandPlain>(dtype, o, H, L_all, l0, rows, extra, E, out, row_scale, stream);
    case kOperandI8: return heads_launch_o<kOperandI8>(dtype, o, H, L_all, l0, rows, extra, E, out, row_scale, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t gated_residual_launch(int dtype, void* out, const void* x, const void* gate, const void* y, int64_t M,
                                 int64_t K, hipStream_t stream) {
  const long chunks = (long)(M * K / 8);
  const long blocks = std::min<long>((chunks + 255) / 256, 8192);
  const dim3 grid((unsigned)blocks), block(256);
  switch (dtype) {
    case kF32:
      hipLaunchKernelGGL(gated_residual_kernel<kF32>, grid, block, 0, stream, out, x, gate, y, chunks, (int)K);
      break;
    case kF16:
      hipLaunchKernelGGL(gated_residual_kernel<kF16>, grid, block, 0, stream, out, x, gate, y, chunks, (int)K);
      break;
    default:
      hipLaunchKernelGGL(gated_residual_kernel<kBF16>, grid, block, 0, stream, out, x, gate, y, chunks, (int)K);
      break;
  }
  return hipGetLastError();
}

}  // namespace qlinear
