// Block-scaled int4 (W4A4) and int8 GEMMs on gfx950 with the reference's numerics (nodes/ComfyUI-Gfx906Int4/csrc/
// int4_gemm_scaled.hip:53-191, 229-246): A [M, K/2] and B [N, K/2] packed int4 (two's-complement
// nibbles, low nibble first), scales As [M, K/qb], Bs [N, K/qb] fp32, qb = 32 or 16. For every
// quant block in K order: ip = exact int32 dot of the block's codes, then
// acc = fmaf(float(ip), as * bs, acc); finally y = acc (+ bias) rounded to the output dtype.
// Split-K (splits > 1, int4): K is cut into ranges of stages_per_split 128-K stages (the
// reference's k-tiles of 4 blocks of 32), each range accumulates from 0 into an fp32 partial, and
// w4a4_splitk_reduce_kernel forms y = ((0 + p_0) + p_1) + ... (+ bias) in split order, the
// reference's splitk_reduce_kernel (int4_gemm_scaled.hip:182-191). The result is bit-identical to
// those sequences.
//
// * One quant block of 32 K is exactly the K of v_mfma_i32_16x16x32_i8, so each MFMA yields one
//   block's integer dot for a 16 x 16 fragment (with qb = 16, two MFMAs per block, each with the
//   other half's lanes zeroed). The nibbles go to the high half of each byte (code * 16): the
//   MFMA returns 256 * ip exactly (|256 ip| <= 2^19), and the A scales are taken as as * 2^-8
//   (exact), so fmaf(float(256 ip), (as * 2^-8) * bs, acc) rounds exactly like the reference's
//   fmaf(float(ip), as * bs, acc) (the two products are the same real number).
// * int8 (block-32 gemm_int8, csrc/int8_gemm.hip:66-213 of the reference, same per-block fmaf order):
//   the codes go to the MFMA as they are (partial = ip), scales unscaled.
// * 128 x 128 tile per 256-thread workgroup, 4 waves as 2 x 2, each 64 x 64 = 4 x 4 fragments.
//   A stage is 64 B of codes per row (4 int4 blocks or 2 int8 blocks): global -> registers -> LDS, double
//   buffered, one barrier per stage. In LDS a row keeps, per lane group j, the 4 dwords (one per
//   block) that lane group j feeds to the MFMA, so a lane reads its operands for the whole stage
//   with one 16-byte read; scales are stored block-major so a lane's 4 rows are one 16-byte read.
// * Lane (r, j) of a fragment supplies row r and K slots 8j .. 8j+7 of the block: int4, dword j of
//   the row's 16-byte block (even K in the low dword, odd K in the high one -- A and B use the same
//   slot order, so the dot is unchanged); int8, bytes 8j .. 8j+7 of the 32-byte block. The
//   accumulator lane layout is (row 4j + e, column r).
#include "common.hpp"
#include "launch.hpp"

namespace qlinear {

namespace {

constexpr int kW4BM = 128, kW4BN = 128;
constexpr int kW4RowBytes = 64;  // code bytes per row per stage (4 int4 blocks or 2 int8 blocks)
constexpr int kW4GroupM = kW4A4GroupM;

// 8 codes of a dword (K = 2t in the low nibble of byte t, 2t + 1 in the high one) as 8 int8 lanes
// holding code * 16: low dword = even K, high dword = odd K.
__device__ __forceinline__ long unpack_x16(uint32_t w) {
  const uint32_t even = (w << 4) & 0xF0F0F0F0u;
  const uint32_t odd = w & 0xF0F0F0F0u;
  return (long)(((uint64_t)odd << 32) | even);
}

template <int SUB, bool kI8>
__global__ __launch_bounds__(256) void w4a4_gemm_kernel(W4A4Params p) {
  constexpr int kBlkBytes = kI8 ? 32 : 16;               // code bytes per quant block of 32 K
  constexpr int kW4StageBlocks = kW4RowBytes / kBlkBytes;
  constexpr int kChunksPerBlk = kBlkBytes / 16;
  constexpr int kScaleCols = SUB * kW4StageBlocks;  // scale columns per stage
  __shared__ __attribute__((aligned(16))) uint8_t lds_a[2][kW4BM * kW4RowBytes];
  __shared__ __attribute__((aligned(16))) uint8_t lds_b[2][kW4BN * kW4RowBytes];
  __shared__ __attribute__((aligned(16))) float lds_as[2][kScaleCols][kW4BM];
  __shared__ __attribute__((aligned(16))) float lds_bs[2][kScaleCols][kW4BN];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int r16 = lane & 15, j4 = lane >> 4;
  const int M = p.M, N = p.N, K = p.K;
  const int KB = K / 32;                     // quant blocks of 32 along K
  const int SC = KB * SUB;                   // scale columns per row
  const int S = (KB + kW4StageBlocks - 1) / kW4StageBlocks;

  const int g = xcd_remap(blockIdx.x, gridDim.x);
  int tm, tn;
  tile_coords(g, p.tiles_m, p.tiles_n, kW4GroupM, tm, tn);
  // this workgroup's K range in stages: all of K, or split blockIdx.y's share (possibly empty)
  const int s_first = p.splits > 1 ? (int)blockIdx.y * p.stages_per_split : 0;
  const int s_end = p.splits > 1 ? min(S, s_first + p.stages_per_split) : S;
  const int m0 = tm * kW4BM, n0 = tn * kW4BN;
  const uint8_t* A = (const uint8_t*)p.a;
  const uint8_t* B = (const uint8_t*)p.b;
  const size_t row_bytes = (size_t)K * kBlkBytes / 32;

  // ---- stage loads: 512 16-byte chunks of A and of B (row c / 4, block c % 4), 128 x kScaleCols
  //      scales of each ------------------------------------------------------------------------
  u32x4 ra[2], rb[2];
  float rsa[kScaleCols];
  auto load_regs = [&](int s) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c = tid + 256 * i, r = c >> 2;
      const int kb = s * kW4StageBlocks + (c & 3) / kChunksPerBlk, part = (c & 3) % kChunksPerBlk;
      const bool ka = kb < KB;
      const size_t off = (size_t)kb * kBlkBytes + 16 * part;
      ra[i] = (ka && m0 + r < M) ? *(const u32x4*)(A + (size_t)(m0 + r) * row_bytes + off) : u32x4{0u, 0u, 0u, 0u};
      rb[i] = (ka && n0 + r < N) ? *(const u32x4*)(B + (size_t)(n0 + r) * row_bytes + off) : u32x4{0u, 0u, 0u, 0u};
    }
    // threads 0-127: A scales of row tid (taken as as * 2^-8); 128-255: B scales of row tid - 128
    const int r = tid & 127;
    const bool is_a = tid < 128;
    const int gr = (is_a ? m0 : n0) + r;
    const bool rok = gr < (is_a ? M : N);
    const float* sp = is_a ? p.as : p.bs;
#pragma unroll
    for (int q = 0; q < kScaleCols; ++q) {
      const int col = s * kScaleCols + q;
      const float v = (rok && col < SC) ? sp[(size_t)gr * SC + col] : 0.0f;
      rsa[q] = (is_a && !kI8) ? v * 0.00390625f : v;
    }
  };
  auto store_lds = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c = tid + 256 * i, r = c >> 2, q = c & 3;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // int4: chunk q = block q, dword j -> lane group j, slot q; int8: chunk q = half q % 2 of block
        // q / 2, dword j -> lane group 2 (q % 2) + j / 2, slot 2 (q / 2) + j % 2
        const int grp = kI8 ? 2 * (q & 1) + (j >> 1) : j;
        const int slot = kI8 ? 2 * (q >> 1) + (j & 1) : q;
        const int off = r * kW4RowBytes + ((grp ^ (r & 3)) << 4) + 4 * slot;
        *(uint32_t*)(lds_a[buf] + off) = ra[i][j];
        *(uint32_t*)(lds_b[buf] + off) = rb[i][j];
      }
    }
    const int r = tid & 127;
    float(*dst)[kW4BM] = tid < 128 ? lds_as[buf] : lds_bs[buf];
#pragma unroll
    for (int q = 0; q < kScaleCols; ++q) dst[q][r] = rsa[q];
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int fm = 0; fm < 4; ++fm)
#pragma unroll
    for (int fn = 0; fn < 4; ++fn) acc[fm][fn] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  load_regs(s_first);
  store_lds(0);
  __syncthreads();
  for (int s = s_first; s < s_end; ++s) {
    const int buf = (s - s_first) & 1;
    if (s + 1 < s_end) load_regs(s + 1);
    u32x4 a_raw[4], b_raw[4];
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      const int ra_row = wm * 64 + f * 16 + r16, rb_row = wn * 64 + f * 16 + r16;
      a_raw[f] = *(const u32x4*)(lds_a[buf] + ra_row * kW4RowBytes + ((j4 ^ (ra_row & 3)) << 4));
      b_raw[f] = *(const u32x4*)(lds_b[buf] + rb_row * kW4RowBytes + ((j4 ^ (rb_row & 3)) << 4));
    }
    const int nb = min(kW4StageBlocks, KB - s * kW4StageBlocks);  // uniform
#pragma unroll
    for (int b = 0; b < kW4StageBlocks; ++b) {
      if (b >= nb) break;
      auto operand = [&](const u32x4& raw) -> long {
        if constexpr (kI8)
          return (long)(((uint64_t)raw[2 * b + 1] << 32) | raw[2 * b]);
        else
          return unpack_x16(raw[b]);
      };
      long bop[4];
#pragma unroll
      for (int fn = 0; fn < 4; ++fn) bop[fn] = operand(b_raw[fn]);
#pragma unroll
      for (int sub = 0; sub < SUB; ++sub) {
        long aop[4];
#pragma unroll
        for (int fm = 0; fm < 4; ++fm) {
          const long v = operand(a_raw[fm]);
          aop[fm] = (SUB == 1 || (j4 >> 1) == sub) ? v : 0l;  // qb = 16: K slots of this half only
        }
        i32x4 part[4][4];
#pragma unroll
        for (int fm = 0; fm < 4; ++fm)
#pragma unroll
          for (int fn = 0; fn < 4; ++fn)
            part[fm][fn] = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop[fm], bop[fn], i32x4{0, 0, 0, 0}, 0, 0, 0);
        const int q = b * SUB + sub;
        f32x4 sa[4];
        float sb[4];
#pragma unroll
        for (int fm = 0; fm < 4; ++fm) sa[fm] = *(const f32x4*)&lds_as[buf][q][wm * 64 + fm * 16 + 4 * j4];
#pragma unroll
        for (int fn = 0; fn < 4; ++fn) sb[fn] = lds_bs[buf][q][wn * 64 + fn * 16 + r16];
#pragma unroll
        for (int fm = 0; fm < 4; ++fm)
#pragma unroll
          for (int fn = 0; fn < 4; ++fn)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              acc[fm][fn][e] = __builtin_fmaf((float)part[fm][fn][e], sa[fm][e] * sb[fn], acc[fm][fn][e]);
      }
    }
    if (s + 1 < s_end) store_lds(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue: y = acc (+ bias), rounded once to the output dtype; a split's partial goes out
  //      as plain fp32 without bias ------------------------------------------------------------
  const bool split = p.splits > 1;
  void* dst = split ? (void*)(p.partial + (size_t)blockIdx.y * M * N) : p.y;
  const int dst_dtype = split ? (int)kF32 : p.out_dtype;
  const void* bias = split ? nullptr : p.bias;
#pragma unroll
  for (int fn = 0; fn < 4; ++fn) {
    const int n = n0 + wn * 64 + fn * 16 + r16;
    if (n >= N) continue;
    const float bv = bias ? read_elem(bias, p.out_dtype, n) : 0.0f;
#pragma unroll
    for (int fm = 0; fm < 4; ++fm)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + wm * 64 + fm * 16 + 4 * j4 + e;
        if (m >= M) continue;
        float v = acc[fm][fn][e];
        if (bias) v = v + bv;
        write_elem(dst, dst_dtype, (size_t)m * N + n, v);
      }
  }
}

// y[i] = ((0 + partial[0][i]) + partial[1][i]) + ... (+ bias[i % N]) in fp32, rounded once to the
// output dtype: the reference's split-K reduction, element by element.
__global__ __launch_bounds__(256) void w4a4_splitk_reduce_kernel(const float* __restrict__ partial,
                                                                 const void* __restrict__ bias, void* __restrict__ y,
                                                                 int out_dtype, int splits, long MN, int N) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= MN) return;
  float v = 0.0f;
  for (int s = 0; s < splits; ++s) v += partial[(size_t)s * MN + i];
  if (bias) v += read_elem(bias, out_dtype, (size_t)(i % N));
  write_elem(y, out_dtype, (size_t)i, v);
}

}  // namespace

hipError_t w4a4_launch(int qblock, const W4A4Params& p, hipStream_t stream) {
  const int splits = p.splits > 1 ? p.splits : 1;
  const dim3 grid((unsigned)(p.tiles_m * p.tiles_n), (unsigned)splits), block(256);
  if (qblock == 32)
    hipLaunchKernelGGL((w4a4_gemm_kernel<1, false>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((w4a4_gemm_kernel<2, false>), grid, block, 0, stream, p);
  if (splits > 1) {
    const long MN = (long)p.M * p.N;
    hipLaunchKernelGGL(w4a4_splitk_reduce_kernel, dim3((unsigned)((MN + 255) / 256)), dim3(256), 0, stream,
                       (const float*)p.partial, p.bias, p.y, p.out_dtype, splits, MN, p.N);
  }
  return hipGetLastError();
}

hipError_t int8_block32_launch(const W4A4Params& p, hipStream_t stream) {
  W4A4Params q = p;
  q.splits = 1;
  const dim3 grid((unsigned)(p.tiles_m * p.tiles_n)), block(256);
  hipLaunchKernelGGL((w4a4_gemm_kernel<1, true>), grid, block, 0, stream, q);
  return hipGetLastError();
}

}  // namespace qlinear
