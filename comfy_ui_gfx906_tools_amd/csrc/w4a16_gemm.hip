// W4A16 GEMM for gfx950: y[M,N] = x[M,K] @ (q[N,K] * s[N,K/32])^T (+ bias), x fp16/bf16,
// q packed int4 in the reference layout (nodes/ComfyUI-Gfx906Int4/ops.py:108-126), fp32 group
// scales, fp32 MFMA accumulation.
//
// The reference computes this product as dequantize-then-matmul (nodes.py:43-52, 116) and its
// production kernel is a W4A4 v_dot8 GEMM (csrc/int4_gemm_scaled.hip:53-180); neither is the
// shape of this kernel. Design, per 256-thread workgroup (4 waves side by side along N) and a
// BM x BN output tile:
//
// * A (activations) is staged HBM -> LDS with global_load_lds_dwordx4, 128 K per stage, double
//   buffered in two distinct arrays. A row of a stage is 256 B = 16 chunks of 16 B; chunk c of
//   row r sits at slot c ^ (r & 15), so the 16 rows an MFMA operand read touches hit 16
//   distinct bank groups. Rows past M are clamped to row M-1 (their outputs are never stored);
//   K past the end is clamped to the last chunk and meets zero weights.
// * B (weights) never touches LDS. Lane (c = l%16, j = l/16) of a wave loads 16 B of weight row
//   n = col0 + c: the whole 32-element quant group j of the stage, with its one scale, and
//   dequantizes it in registers (dequant8: int4 -> q*s -> fp16/bf16). The MFMA K-slot map is
//   permuted to match: MFMA i of a stage takes, in K-slot block j, elements 32j + 8i .. +7; A is
//   read from LDS with the same map (chunk 4j + i), so every lane's load is one group.
// * Each wave owns a (16*WM) x (16*WN) sub-tile of 16x16 accumulators (v_mfma_f32_16x16x32).
//   With WM = 16 the dequant costs 0.5 element per MFMA.
// * Optional row scales (the fp16 route for bf16 activations): x arrives pre-scaled per row by
//   2^-e (exact) and the epilogue multiplies by 2^e (exact).
// * Scheduling: every workgroup runs one K range of one tile. The first dp_tiles tiles are
//   whole (kernel instance kCut = false); each remaining tile is cut into ksplit K ranges
//   (kCut = true, launched next on the same stream) whose fp32 partials a third kernel sums in
//   piece order (deterministic), with bias and row scale. Stream order makes the partials
//   visible to the reduction -- no fences or counters inside the GEMM, which on MI355X's
//   per-XCD L2s would force L2 write-backs.
#include "common.hpp"
#include "launch.hpp"

namespace qlinear {

namespace {

constexpr int kStageK = 128;        // K per pipeline stage (16-bit elements)
constexpr int kRowBytes = 256;      // one A row of a stage
constexpr int kGroupsPerStage = 4;  // 128 / 32
constexpr int kGroupM = 8;
constexpr int kWaves = 4;

template <bool kBf16, int WM, int WN, bool kCut, bool kRegA>
__global__ __launch_bounds__(64 * kWaves) void w4a16_gemm_kernel(W4A16Params p) {
  constexpr int BM = 16 * WM;
  constexpr int BN = 16 * WN * kWaves;
  constexpr int kStageBytes = BM * kRowBytes;
  constexpr int kBlocksPerWave = BM / 4 / kWaves;  // 1 KiB LDS blocks each wave fills per stage
  static_assert(BM % (4 * kWaves) == 0, "A tile must split into whole 1 KiB blocks per wave");
  // Two distinct arrays (not one indexed by stage parity): the compiler's alias analysis then
  // sees that operand reads of one buffer never touch the DMA target of the other, and does not
  // wait for the next stage's loads before the current stage's MFMAs.
  __shared__ __attribute__((aligned(1024))) uint8_t lds0[kStageBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t lds1[kStageBytes];

  const int lane = threadIdx.x & 63;
  const int wn = threadIdx.x >> 6;
  const int r16 = lane & 15, j4 = lane >> 4;
  const int M = p.M, N = p.N, K = p.K;
  const int groups = K / kGroup;
  const int S = p.stages;  // steps of two stages

  const uint16_t* __restrict__ x = (const uint16_t*)p.x;

  // ---- this workgroup's segment ----------------------------------------------------------
  const int g = xcd_remap(blockIdx.x, gridDim.x);
  int t, s0, s1;
  if constexpr (!kCut) {
    t = g;
    s0 = 0;
    s1 = S;
  } else {
    t = p.dp_tiles + g / p.ksplit;
    const int piece = g - (t - p.dp_tiles) * p.ksplit;
    s0 = (int)((long long)piece * S / p.ksplit);
    s1 = (int)((long long)(piece + 1) * S / p.ksplit);
  }
  int tm, tn;
  tile_coords(t, p.tiles_m, p.tiles_n, kGroupM, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;

  // ---- B addressing ------------------------------------------------------------------------
  const uint8_t* bptr[WN];
  const float* sptr[WN];
  bool bok[WN];
#pragma unroll
  for (int fn = 0; fn < WN; ++fn) {
    const int n = n0 + (wn * WN + fn) * 16 + r16;
    bok[fn] = n < N;
    const int nc = min(n, N - 1);
    bptr[fn] = (const uint8_t*)p.wq + (size_t)nc * (K / 2);
    sptr[fn] = p.ws + (size_t)nc * groups;
  }

  // A staging, either HBM -> LDS directly (global_load_lds_dwordx4) or through registers
  // (global_load_dwordx4, then ds_write_b128 at the end of the stage). Same LDS layout.
  u32x4 areg[kRegA ? kBlocksPerWave : 1];
  auto a_src = [&](int s, int q) {
    const int blk = wn * kBlocksPerWave + q;
    const int row = blk * 4 + j4;
    const int lch = r16 ^ (row & 15);
    const int gm = min(m0 + row, M - 1);
    const int gk = min(s * kStageK + lch * 8, K - 8);
    return x + (size_t)gm * K + gk;
  };
  auto issue_a = [&](int s, uint8_t* buf) {
#pragma unroll
    for (int q = 0; q < kBlocksPerWave; ++q) {
      if constexpr (kRegA) {
        areg[q] = *(const u32x4*)a_src(s, q);
      } else {
        load_lds16(a_src(s, q), buf + (wn * kBlocksPerWave + q) * 1024);
      }
    }
  };
  auto commit_a = [&](uint8_t* buf) {
    if constexpr (kRegA) {
#pragma unroll
      for (int q = 0; q < kBlocksPerWave; ++q) *(u32x4*)(buf + (wn * kBlocksPerWave + q) * 1024 + lane * 16) = areg[q];
    }
  };
  // Raw loads only; the zero-scale select for columns past N / groups past K is applied by the
  // stage that consumes them, so no wait is forced right after the loads are issued.
  auto load_b = [&](int s, u32x4 (&raw)[WN], float (&sc)[WN]) {
    const int kgc = min(s * kGroupsPerStage + j4, groups - 1);
#pragma unroll
    for (int fn = 0; fn < WN; ++fn) {
      raw[fn] = *(const u32x4*)(bptr[fn] + (size_t)kgc * 16);
      sc[fn] = sptr[fn][kgc];
    }
  };

  f32x4 acc[WM][WN];
#pragma unroll
  for (int fm = 0; fm < WM; ++fm)
#pragma unroll
    for (int fn = 0; fn < WN; ++fn) acc[fm][fn] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Two register sets for the raw weights, alternating with the two LDS buffers.
  u32x4 rawA[WN], rawB[WN];
  float scA[WN], scB[WN];

  // One pipeline stage: operands of stage s are in `cur` (LDS) and raw/scr (registers); stage s+1
  // is fetched into `nxt` and raw_n/sc_n. Order matters: the stage's own registers are consumed
  // (first dequant, first operand reads) before the next loads are issued, so the waits the
  // compiler places for them never also wait for the next stage's loads.
  auto stage = [&](int s, int s_end, const uint8_t* cur, uint8_t* nxt, u32x4 (&raw)[WN], float (&scr)[WN],
                   u32x4 (&raw_n)[WN], float (&sc_n)[WN]) {
    wait_vmem();
    __syncthreads();
    float sc[WN], neg8s[WN];
    const bool kok = s * kGroupsPerStage + j4 < groups;
#pragma unroll
    for (int fn = 0; fn < WN; ++fn) {
      sc[fn] = (bok[fn] && kok) ? scr[fn] : 0.0f;  // zero scale -> exact zero weights
      neg8s[fn] = -8.0f * sc[fn];
    }
    u32x4 b[WN];
#pragma unroll
    for (int fn = 0; fn < WN; ++fn) b[fn] = dequant8<kBf16>(raw[fn][0], sc[fn], neg8s[fn]);

    // A operand blocks q = i * WM + fm (K-step i, 16-row block fm); ring of three registers,
    // reads issued two blocks ahead of their MFMAs
    const uint8_t* abase = cur + r16 * kRowBytes;
    auto a_addr = [&](int q) {
      const int i = q / WM, fm = q % WM;
      return (const u32x4*)(abase + fm * 16 * kRowBytes + (((4 * j4 + i) ^ r16) * 16));
    };
    constexpr int kBlocks = 4 * WM;
    u32x4 ar[3];
    ar[0] = *a_addr(0);
    if (kBlocks > 1) ar[1] = *a_addr(1);
    __builtin_amdgcn_sched_barrier(0);

    if (s + 1 < s_end) {
      issue_a(s + 1, nxt);
      load_b(s + 1, raw_n, sc_n);
    }

    u32x4 bn[WN];
#pragma unroll
    for (int q = 0; q < kBlocks; ++q) {
      const int i = q / WM, fm = q % WM;
      if (q + 2 < kBlocks) ar[(q + 2) % 3] = *a_addr(q + 2);
      if (fm == 0 && i > 0) {
#pragma unroll
        for (int fn = 0; fn < WN; ++fn) b[fn] = bn[fn];
      }
#pragma unroll
      for (int fn = 0; fn < WN; ++fn) acc[fm][fn] = mfma16<kBf16>(ar[q % 3], b[fn], acc[fm][fn]);
      // dequant of K-step i+1, spread over the 16-row blocks: column block fn goes with row
      // block fn % WM (all of them with the first row block when WM == 1)
      if (i < 3) {
#pragma unroll
        for (int fn = 0; fn < WN; ++fn)
          if (fn % WM == fm) bn[fn] = dequant8<kBf16>(raw[fn][i + 1], sc[fn], neg8s[fn]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (s + 1 < s_end) commit_a(nxt);
  };

  // Segments are counted in steps of two stages (256 K), so both halves of the unrolled loop
  // body run unconditionally and the accumulators stay in one register class.
  const int s_end = 2 * s1;
  issue_a(2 * s0, lds0);
  commit_a(lds0);
  load_b(2 * s0, rawA, scA);
  // Drain the kernel-argument scalar loads: with none pending, the compiler can wait for LDS
  // operand reads with partial lgkmcnt counts instead of lgkmcnt(0).
  wait_lgkm();
  for (int sp = s0; sp < s1; ++sp) {
    stage(2 * sp, s_end, lds0, lds1, rawA, scA, rawB, scB);
    stage(2 * sp + 1, s_end, lds1, lds0, rawB, scB, rawA, scA);
  }

  // ---- epilogue ----------------------------------------------------------------------------
  // A whole tile goes to y (row scale, bias, out dtype); a cut tile's piece goes as plain fp32 to
  // its partial slot, a tile-local [BM][BN] array. Same store loop for both.
  void* dst = p.y;
  int dst_m0 = m0, dst_n0 = n0, dst_M = M, dst_N = N, dst_dtype = p.out_dtype;
  const void* bias = p.bias;
  const float* row_scale = p.row_scale;
  if constexpr (kCut) {
    dst = p.partial + (size_t)g * (BM * BN);
    dst_m0 = 0;
    dst_n0 = 0;
    dst_M = BM;
    dst_N = BN;
    dst_dtype = kF32;
    bias = nullptr;
    row_scale = nullptr;
  }
  float bv[WN];
#pragma unroll
  for (int fn = 0; fn < WN; ++fn) {
    const int n = dst_n0 + (wn * WN + fn) * 16 + r16;
    bv[fn] = (bias && n < dst_N) ? read_elem(bias, dst_dtype, n) : 0.0f;
  }
  // one 16-row block at a time, fenced, so the row scales and addresses of all rows are never
  // live together
#pragma unroll
  for (int fm = 0; fm < WM; ++fm) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = dst_m0 + fm * 16 + 4 * j4 + e;
      if (m >= dst_M) continue;
      const float rs = row_scale ? row_scale[m] : 1.0f;
#pragma unroll
      for (int fn = 0; fn < WN; ++fn) {
        const int n = dst_n0 + (wn * WN + fn) * 16 + r16;
        if (n < dst_N) write_elem(dst, dst_dtype, (size_t)m * dst_N + n, acc[fm][fn][e] * rs + bv[fn]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Sums the ksplit fp32 partials of every cut tile in piece order, applies the row scale and the
// bias, and stores y. Grid: (cut tiles) x (BM*BN / 1024) workgroups of 256 threads, 4 elements
// per thread.
__global__ __launch_bounds__(256) void w4a16_reduce_kernel(W4A16Params p, int BM, int BN) {
  const int tl = blockIdx.y;  // cut tile index
  const int t = p.dp_tiles + tl;
  int tm, tn;
  tile_coords(t, p.tiles_m, p.tiles_n, kGroupM, tm, tn);
  const int idx = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (idx >= BM * BN) return;
  const size_t tile_elems = (size_t)BM * BN;
  const float* first = p.partial + (size_t)tl * p.ksplit * tile_elems;
  f32x4 v = *(const f32x4*)(first + idx);
  for (int q = 1; q < p.ksplit; ++q) {
    const f32x4 w = *(const f32x4*)(first + (size_t)q * tile_elems + idx);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] += w[e];
  }
  const int m = tm * BM + idx / BN;
  if (m >= p.M) return;
  const float rs = p.row_scale ? p.row_scale[m] : 1.0f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int n = tn * BN + idx % BN + e;
    if (n >= p.N) continue;
    const float bv = p.bias ? read_elem(p.bias, p.out_dtype, n) : 0.0f;
    write_elem(p.y, p.out_dtype, (size_t)m * p.N + n, v[e] * rs + bv);
  }
}

// x [M, K] (fp32 / fp16 / bf16) -> x16 [M, K] fp16 scaled by 2^-e_m per row, row_scale[m] = 2^e_m,
// with e_m chosen so that max |x16| lies in [2^14, 2^15): every bf16 value maps exactly (fp16
// keeps 11 mantissa bits), and no row can overflow fp16. One workgroup per row; 8 elements per
// thread and step (16-byte loads for 16-bit inputs), the row read twice (max, then convert; the
// second read hits L2).
template <int DT>
__global__ __launch_bounds__(256) void rows_to_scaled_f16_kernel(const void* __restrict__ x,
                                                                 _Float16* __restrict__ x16,
                                                                 float* __restrict__ row_scale, int K) {
  __shared__ float red[4];
  const int row = blockIdx.x;
  const size_t base = (size_t)row * K;
  auto load8 = [&](int k, float (&v)[8]) {
    if constexpr (DT == kF32) {
      const u32x4 lo = *(const u32x4*)((const float*)x + base + k);
      const u32x4 hi = *(const u32x4*)((const float*)x + base + k + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t a = lo[e], b = hi[e];
        v[e] = __builtin_bit_cast(float, a);
        v[4 + e] = __builtin_bit_cast(float, b);
      }
    } else {
      const u32x4 w = *(const u32x4*)((const uint16_t*)x + base + k);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t word = w[e];
        v[2 * e] = DT == kBF16 ? bf16_bits_to_f32(word & 0xFFFFu) : f16_bits_to_f32(word & 0xFFFFu);
        v[2 * e + 1] = DT == kBF16 ? bf16_bits_to_f32(word >> 16) : f16_bits_to_f32(word >> 16);
      }
    }
  };
  float amax = 0.0f;
  for (int k = threadIdx.x * 8; k < K; k += 256 * 8) {
    float v[8];
    load8(k, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[e]));
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, kWave));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  int e = 0;
  if (amax > 0.0f && amax <= 3.0e38f) {
    int E;
    frexpf(amax, &E);  // amax = f * 2^E, f in [0.5, 1)
    e = E - 15;
  }
  if (threadIdx.x == 0) row_scale[row] = ldexpf(1.0f, e);
  for (int k = threadIdx.x * 8; k < K; k += 256 * 8) {
    float v[8];
    load8(k, v);
    u32x4 out;
#pragma unroll
    for (int q = 0; q < 4; ++q) out[q] = pack2_f16(ldexpf(v[2 * q], -e), ldexpf(v[2 * q + 1], -e));
    *(u32x4*)(x16 + base + k) = out;
  }
}

}  // namespace

// ---- host-side launch ------------------------------------------------------------------------
// A staging through registers for tiles up to 128 rows (the LDS-DMA path makes the compiler
// wait for operand reads with lgkmcnt(0)); 256-row tiles keep the DMA path (no registers left).
#ifndef QL_A_REG_MAX_WM
#define QL_A_REG_MAX_WM 8
#endif

template <bool kBf16, int WM>
static hipError_t launch_cfg(const W4A16Params& p, hipStream_t stream) {
  constexpr int BM = 16 * WM, BN = 16 * 4 * kWaves;
  constexpr bool kRegA = WM <= QL_A_REG_MAX_WM;
  const int tiles = p.tiles_m * p.tiles_n;
  if (p.dp_tiles > 0)
    hipLaunchKernelGGL((w4a16_gemm_kernel<kBf16, WM, 4, false, kRegA>), dim3(p.dp_tiles), dim3(64 * kWaves), 0,
                       stream, p);
  const int cut = tiles - p.dp_tiles;
  if (cut > 0) {
    hipLaunchKernelGGL((w4a16_gemm_kernel<kBf16, WM, 4, true, kRegA>), dim3(cut * p.ksplit), dim3(64 * kWaves), 0,
                       stream, p);
    hipLaunchKernelGGL(w4a16_reduce_kernel, dim3((BM * BN + 1023) / 1024, cut), dim3(256), 0, stream, p, BM, BN);
  }
  return hipGetLastError();
}

const W4A16Config& w4a16_config(int id) {
  // {id, BM, BN}; every config is 4 waves side by side, each 16*WM rows x 64 columns
  static const W4A16Config cfgs[] = {
      {0, 256, 256},  // WM 16
      {1, 128, 256},  // WM 8
      {2, 64, 256},   // WM 4
      {3, 16, 256},   // WM 1
  };
  return cfgs[id];
}

hipError_t w4a16_launch(int cfg, bool bf16, const W4A16Params& p, hipStream_t stream) {
#define QL_CASE(ID, WM) \
  case ID:              \
    return bf16 ? launch_cfg<true, WM>(p, stream) : launch_cfg<false, WM>(p, stream);
  switch (cfg) {
    QL_CASE(0, 16)
    QL_CASE(1, 8)
    QL_CASE(2, 4)
    QL_CASE(3, 1)
    default:
      return hipErrorInvalidValue;
  }
#undef QL_CASE
}

hipError_t rows_to_scaled_f16_launch(int dtype, const void* x, void* x16, float* row_scale, int64_t M,
                                     int64_t K, hipStream_t stream) {
  const dim3 grid((unsigned)M);
  switch (dtype) {
    case kF32:
      hipLaunchKernelGGL(rows_to_scaled_f16_kernel<kF32>, grid, dim3(256), 0, stream, x, (_Float16*)x16, row_scale,
                         (int)K);
      break;
    case kF16:
      hipLaunchKernelGGL(rows_to_scaled_f16_kernel<kF16>, grid, dim3(256), 0, stream, x, (_Float16*)x16, row_scale,
                         (int)K);
      break;
    default:
      hipLaunchKernelGGL(rows_to_scaled_f16_kernel<kBF16>, grid, dim3(256), 0, stream, x, (_Float16*)x16,
                         row_scale, (int)K);
      break;
  }
  return hipGetLastError();
}

}  // namespace qlinear
