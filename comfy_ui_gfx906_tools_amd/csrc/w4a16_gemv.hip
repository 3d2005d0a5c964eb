// W4A16 for a handful of activation rows (M <= 4): y[M,N] = x[M,K] @ (q[N,K] * s[N,K/32])^T
// (+ bias), bf16 or fp16 x read as is, q packed int4 in the reference layout
// (nodes/ComfyUI-Gfx906Int4/ops.py:108-126), fp32 group scales. HBM-bound: every weight byte is
// read once and feeds M multiply-adds, so the kernel is built around streaming the packed weights
// at full bandwidth with as little VALU work per weight as possible; no MFMA (a 16-row MFMA tile
// would be at most a quarter full).
//
// * About four waves per SIMD, each looping over its output columns n = w, w + W, w + 2W, ...
//   (W = waves in the grid). Lane i takes the quant groups g = i, i + 64, ... (kR of them) of
//   a column: 16 contiguous bytes (32 nibbles) each, so one load instruction reads 1 KiB of one
//   weight row. The weights and scales of the next kD columns (kD = max(2, 6 / kR)) are in flight by
//   DMA into a wave-private LDS ring while a column is computed: enough bytes in flight for HBM
//   latency, and memory and arithmetic overlap within every wave.
// * Dequant without conversion instructions: with u = nibble ^ 8 = code + 8 in [0, 15], the
//   16-bit pattern  magic | u  is the number c + u exactly, c = 128 in bf16 (magic 0x4300, 7
//   mantissa bits) and c = 1024 in fp16 (0x6400). One v_bitop3_b32 on the dword shifted by 4i
//   (mask 0x000F000F, the xor with 8 folded in) builds the pair (c + u_i, c + u_{i+4}) of its
//   nibbles i and i + 4, so 8 weights take 7 bit operations (three shifts, four bitop3). The
//   activations are arranged to match once per wave and kept in registers: pairs
//   (x_i, x_{i+4}), i = 0..3, of every 8.
// * v_dot2_f32_{bf16,f16} multiplies two such pairs exactly and adds in fp32, so a group gives
//   D = sum x_k (c + u_k); its contribution is s * (D - E) with E = (c + 8) * sum x_k over the
//   group, computed once per (row, group) with the activations, so that D - E = sum x_k code_k.
//   Codes and activations enter exactly; the roundings are those of the fp32 sums (the c terms
//   cancel there: with c = 1024 the sums carry about 10 bits more magnitude than the result,
//   which still leaves a relative error near 1e-4 of max|y| at K = 4096).
// * A column's 64 lane sums are combined by DPP within rows of 16 lanes and v_readlane of the
//   four row sums (a fixed order: deterministic); lane (column index % 64) keeps the result and
//   the wave stores all its columns at the end, so the loop issues no stores and its vmcnt waits
//   count weight loads only.
#include <algorithm>

#include "common.hpp"
#include "launch.hpp"

namespace qlinear {

namespace {

constexpr int kGvWaves = 4;  // waves per workgroup (independent)
// Four waves per SIMD, each with 6 / kR (at least 2) columns in flight: against two waves with
// 12 / kR columns (the same bytes in flight per CU), each wave owns half the columns, so less of
// its arithmetic trails the last load (measured at M = 1: K = 4096, N = 10240 9.24 -> 8.95 us;
// 3072 -> 18432 11.7 -> 10.9 us; with a single column in flight at K = 8192 it lost, 7.7 -> 8.1 us).
// LDS: 4 waves x kD x kR x 1.25 KiB per workgroup, at most 40 KiB, so four workgroups fit a CU.
constexpr int kGvDepth = 6;
constexpr int kGvWavesPerSimd = 4;

template <bool kBf16>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  if constexpr (kBf16) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
  } else {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c, false);
  }
}

// v + DPP-permuted v (dpp_ctrl kCtrl), all lanes enabled
template <int kCtrl>
__device__ __forceinline__ float add_dpp(float v) {
  const int t = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, 0xF, 0xF, false);
  return v + __builtin_bit_cast(float, t);
}

// Sum over the 64 lanes, the same value in every lane: butterflies within each row of 16 lanes
// (quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror, row_mirror), then the four row sums.
__device__ __forceinline__ float wave_sum(float v) {
  v = add_dpp<0xB1>(v);
  v = add_dpp<0x4E>(v);
  v = add_dpp<0x141>(v);
  v = add_dpp<0x140>(v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return (r0 + r1) + (r2 + r3);
}

// kR quant groups per lane and column (K <= 2048 kR), kM activation rows (M <= kM).
template <bool kBf16, int kM, int kR>
__global__ __launch_bounds__(64 * kGvWaves) void w4a16_gemv_kernel(W4A16Params p) {
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(blockIdx.x * kGvWaves + (threadIdx.x >> 6));
  const int W = gridDim.x * kGvWaves;
  const int M = p.M, N = p.N, K = p.K;
  const int G = K / kGroup;  // quant groups per column
  const int ncols = w < N ? (N - w + W - 1) / W : 0;  // <= 64 (the launcher sizes the grid)
  constexpr uint32_t kMagic = kBf16 ? 0x43004300u : 0x64006400u;
  constexpr float kC = kBf16 ? 128.0f : 1024.0f;  // value of the magic alone
  // (c + u_0, c + u_4) from the raw nibbles n_0 (bits 0-3) and n_4 (bits 16-19) of v:
  // ((v & 0x000F000F) ^ 0x00080008) | magic = (v & 0x000F000F) ^ (magic | 0x00080008), as the
  // magic has no bits in the nibble field -- one v_bitop3_b32 (truth table 0x6A: (a & b) ^ c).
  auto pair = [](uint32_t v) { return __builtin_amdgcn_bitop3_b32(v, 0x000F000Fu, kMagic | 0x00080008u, 0x6A); };

  // ---- weight loads of column i into LDS buffer b -------------------------------------------
  // DMA (buffer_load ... lds) into a wave-private LDS ring of kD column buffers, each kR KiB of
  // weights then kR x 256 B of scales; lane i's 16 B (4 B) land at 16 i (4 i) of each block, which
  // it reads back itself. Loads into LDS write no registers, so the compiler adds no waits of its
  // own; the loop waits for exactly the loads it needs. A resource per column row: columns past N
  // and groups past K read zeros (a zero scale then zeroes the group). Every call issues exactly
  // 2 kR loads.
  constexpr int kColBytes = kR * (1024 + 256);
  constexpr int kD = kGvDepth / kR >= 2 ? kGvDepth / kR : 2;  // columns in flight per wave
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kGvWaves * kD * kColBytes];
  uint8_t* const mine = lds + (threadIdx.x >> 6) * kD * kColBytes;
  auto issue = [&](int i, auto bc) {
    constexpr int b = decltype(bc)::value;
    const int n = w + i * W;
    const bool live = i < ncols;
    const rsrc_t rw = make_rsrc((const uint8_t*)p.wq + (size_t)(live ? n : 0) * (K / 2), live ? (uint32_t)(K / 2) : 0u);
    const rsrc_t rs = make_rsrc(p.ws + (size_t)(live ? n : 0) * G, live ? (uint32_t)G * 4 : 0u);
    uint8_t* const buf = mine + b * kColBytes;
#pragma unroll
    for (int r = 0; r < kR; ++r) {
      buf_load16_lds(rw, buf + r * 1024, (uint32_t)(lane * 16), r * 1024);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(buf + kR * 1024 + r * 256),
                                               4, (uint32_t)(lane * 4), r * 256, 0, 0);
    }
  };
  // ---- activations: pairs matching the dequant, and the per-group offsets E -----------------
  // Group g = 64 r + lane of row m: 32 values = 4 chunks of 8; chunk q gives the dot pairs
  // (x0, x4), (x1, x5), (x2, x6), (x3, x7), in the order the weight dword of chunk q is expanded.
  // The activation loads go first, then the weight loads of the first kD columns, then the
  // arithmetic on the activations: in-order vmcnt then lets it wait for the activations only.
  u32x4 xv[kR][kM][4];
#pragma unroll
  for (int r = 0; r < kR; ++r)
#pragma unroll
    for (int m = 0; m < kM; ++m) {
      const bool row = m < M;
      const rsrc_t rx = make_rsrc((const uint16_t*)p.x + (size_t)(row ? m : 0) * K, row ? (uint32_t)K * 2 : 0u);
#pragma unroll
      for (int q = 0; q < 4; ++q) xv[r][m][q] = buf_load16(rx, (uint32_t)(lane * 64 + q * 16), r * 4096);
    }
  __builtin_amdgcn_sched_barrier(0);
  static_for<0, kD>([&](auto bc) { issue(decltype(bc)::value, bc); });
  __builtin_amdgcn_sched_barrier(0);
  uint32_t xp[kR][kM][16];
  float e[kR][kM];
#pragma unroll
  for (int r = 0; r < kR; ++r)
#pragma unroll
    for (int m = 0; m < kM; ++m) {
      float xs = 0.0f;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const u32x4 v = xv[r][m][q];
        // v = (x0 x1)(x2 x3)(x4 x5)(x6 x7), low half first -> (x0 x4)(x1 x5)(x2 x6)(x3 x7)
        xp[r][m][4 * q + 0] = __builtin_amdgcn_perm(v[2], v[0], 0x05040100u);
        xp[r][m][4 * q + 1] = __builtin_amdgcn_perm(v[2], v[0], 0x07060302u);
        xp[r][m][4 * q + 2] = __builtin_amdgcn_perm(v[3], v[1], 0x05040100u);
        xp[r][m][4 * q + 3] = __builtin_amdgcn_perm(v[3], v[1], 0x07060302u);
        auto f = [&](uint32_t bits) { return kBf16 ? bf16_bits_to_f32(bits) : f16_bits_to_f32(bits); };
#pragma unroll
        for (int t = 0; t < 4; ++t) xs += f(v[t] & 0xFFFFu) + f(v[t] >> 16);
      }
      e[r][m] = (kC + 8.0f) * xs;
    }

  // ---- column loop ------------------------------------------------------------------------------
  float res[kM];
#pragma unroll
  for (int m = 0; m < kM; ++m) res[m] = 0.0f;
  typedef __attribute__((address_space(3))) const u32x4* lds_u32x4_ptr;
  typedef __attribute__((address_space(3))) const float* lds_f32_ptr;
  auto compute = [&](int i, auto bc) {
    constexpr int b = decltype(bc)::value;
    const uint32_t base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)(mine + b * kColBytes);
    float acc[kM];
#pragma unroll
    for (int m = 0; m < kM; ++m) acc[m] = 0.0f;
#pragma unroll
    for (int r = 0; r < kR; ++r) {
      const u32x4 wr = *(lds_u32x4_ptr)(base + r * 1024 + lane * 16);
      const float sr = *(lds_f32_ptr)(base + kR * 1024 + r * 256 + lane * 4);
      uint32_t pr[16];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t wq = wr[q];
        pr[4 * q + 0] = pair(wq);
        pr[4 * q + 1] = pair(wq >> 4);
        pr[4 * q + 2] = pair(wq >> 8);
        pr[4 * q + 3] = pair(wq >> 12);
      }
#pragma unroll
      for (int m = 0; m < kM; ++m) {
        float d = 0.0f;
#pragma unroll
        for (int k = 0; k < 16; ++k) d = dot2<kBf16>(pr[k], xp[r][m][k], d);
        acc[m] = fmaf(sr, d - e[r][m], acc[m]);
      }
    }
#pragma unroll
    for (int m = 0; m < kM; ++m) {
      const float v = wave_sum(acc[m]);
      res[m] = lane == i ? v : res[m];
    }
  };
  // Entering the wait of column i (ring slot i % kD), the loads in flight are those of columns
  // i .. i + kD - 1. A slot is refilled only after this wave's reads of it have returned.
  for (int i0 = 0; i0 < ncols; i0 += kD) {
    bool done = false;
    static_for<0, kD>([&](auto bc) {
      constexpr int b = decltype(bc)::value;
      if (done || i0 + b >= ncols) {
        done = true;
        return;
      }
      wait_vmcnt<(kD - 1) * 2 * kR>();
      compute(i0 + b, bc);
      wait_lgkm();
      issue(i0 + b + kD, bc);
    });
  }
  wait_vmcnt<0>();  // no DMA into LDS may outlive the wave

  // ---- epilogue: lane j stores column w + j W -----------------------------------------------
  if (lane < ncols) {
    const int n = w + lane * W;
    const float bv = p.bias ? read_elem(p.bias, p.out_dtype, n) : 0.0f;
#pragma unroll
    for (int m = 0; m < kM; ++m) {
      if (m < M) {
        float out = res[m] * (p.row_scale ? p.row_scale[m] : 1.0f) + bv;
        if (p.act == kActGeluTanh) out = gelu_tanh(round_to(p.out_dtype, out));
        write_elem(p.y, p.out_dtype, (size_t)m * N + n, out);
      }
    }
  }
}

}  // namespace

hipError_t w4a16_gemv_launch(bool bf16, const W4A16Params& p, hipStream_t stream) {
  // kGvWavesPerSimd waves per SIMD, at least one column per wave, at most 64 columns per wave
  const int waves = std::max(std::min(4 * kGvWavesPerSimd * std::max(p.cus, 1), p.N), (p.N + 63) / 64);
  const dim3 grid((unsigned)((waves + kGvWaves - 1) / kGvWaves)), block(64 * kGvWaves);
  const int kr = p.K <= 2048 ? 1 : p.K <= 4096 ? 2 : 4;
  const int km = p.M <= 1 ? 1 : p.M <= 2 ? 2 : 4;
#define QL_GV(B, MM, RR) hipLaunchKernelGGL((w4a16_gemv_kernel<B, MM, RR>), grid, block, 0, stream, p)
#define QL_GV_R(B, MM)     \
  if (kr == 1)             \
    QL_GV(B, MM, 1);       \
  else if (kr == 2)        \
    QL_GV(B, MM, 2);       \
  else                     \
    QL_GV(B, MM, 4);
  if (km == 4 && kr == 4) return hipErrorInvalidValue;  // excluded by w4a16 planning (K * M <= 16384)
  if (bf16) {
    if (km == 1) {
      QL_GV_R(true, 1)
    } else if (km == 2) {
      QL_GV_R(true, 2)
    } else if (kr == 1) {
      QL_GV(true, 4, 1);
    } else {
      QL_GV(true, 4, 2);
    }
  } else {
    if (km == 1) {
      QL_GV_R(false, 1)
    } else if (km == 2) {
      QL_GV_R(false, 2)
    } else if (kr == 1) {
      QL_GV(false, 4, 1);
    } else {
      QL_GV(false, 4, 2);
    }
  }
#undef QL_GV_R
#undef QL_GV
  return hipGetLastError();
}

}  // namespace qlinear
