// W4A16 GEMM for gfx950: y[M,N] = x[M,K] @ (q[N,K] * s[N,K/32])^T (+ bias), x bf16/fp16,
// q packed int4 in the reference layout (nodes/ComfyUI-Gfx906Int4/ops.py:108-126), fp32 group
// scales, fp32 MFMA accumulation.
//
// The reference computes this product as dequantize-then-matmul (nodes.py:43-52, 116) and its
// production kernel is a W4A4 v_dot8 GEMM (csrc/int4_gemm_scaled.hip:53-180); neither is the
// shape of this kernel. Design, per workgroup of NWM x NWN waves and a BM x BN output tile:
//
// * A (activations) is staged HBM -> LDS with global_load_lds_dwordx4, 128 K per stage, double
//   buffered. A row of a stage is 256 B = 16 chunks of 16 B; chunk c of row r sits at
//   slot c ^ (r & 15), so the 16 rows an MFMA operand read touches hit 16 distinct bank groups.
//   Rows past M are clamped to row M-1 (their outputs are never stored); K past the end is
//   clamped to the last chunk and meets zero weights.
// * B (weights) never touches LDS. Lane (c = l%16, j = l/16) of a wave loads 16 B of weight
//   row n = col0 + c: the whole 32-element quant group j of the stage, with its one scale, and
//   dequantizes it in registers (dequant8: int4 -> q*s -> bf16/fp16). The MFMA K-slot map is
//   permuted to match: MFMA i of a stage takes, in K-slot block j, elements 32j + 8i .. +7.
//   A is read from LDS with the same map (chunk 4j + i), so every lane's load is one group.
// * Each wave owns a 16*WM x 16*WN sub-tile: WM*WN accumulators of 16x16, v_mfma_f32_16x16x32.
//   With WM = 16 a wave's dequant work is 0.5 element per MFMA, which hides under the MFMA.
// * Scheduling: every workgroup runs exactly one K range of one tile. The first dp_tiles tiles
//   are whole (one workgroup each); each remaining tile is cut into ksplit K ranges, so a grid
//   that would leave CUs idle in its last wave is evened out. A cut tile is finished by the
//   workgroup that arrives last on its counter: it sums the fp32 partials of all pieces in
//   piece order (deterministic), adds the bias and stores. No workgroup ever waits on another.
//   (One segment per workgroup keeps the accumulators' live range simple enough for the
//   register allocator to leave them in AGPRs.)
#include "common.hpp"
#include "launch.hpp"

namespace qlinear {

namespace {

constexpr int kStageK = 128;          // K per pipeline stage (16-bit elements); S counts
                                      // steps of two stages
constexpr int kRowBytes = 256;        // one A row of a stage
constexpr int kGroupsPerStage = 4;    // 128 / 32
constexpr int kGroupM = 8;

template <bool kBf16, int WM, int WN, int NWM, int NWN>
__global__ __launch_bounds__(64 * NWM * NWN) void w4a16_gemm_kernel(W4A16Params p) {
  constexpr int NW = NWM * NWN;
  constexpr int BM = 16 * WM * NWM;
  constexpr int BN = 16 * WN * NWN;
  constexpr int kStageBytes = BM * kRowBytes;
  constexpr int kBlocksPerWave = BM / 4 / NW;  // 1024-B LDS blocks each wave fills per stage
  static_assert(BM % (4 * NW) == 0, "A tile must split into whole 1 KiB blocks per wave");
  // Two distinct arrays (not one indexed by stage parity): the compiler's alias analysis then
  // sees that operand reads of one buffer never touch the DMA target of the other, and does
  // not wait for the next stage's loads before the current stage's MFMAs.
  __shared__ __attribute__((aligned(1024))) uint8_t lds0[kStageBytes];
  __shared__ __attribute__((aligned(1024))) uint8_t lds1[kStageBytes];
  __shared__ int s_last;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave / NWN, wn = wave % NWN;
  const int r16 = lane & 15, j4 = lane >> 4;
  const int M = p.M, N = p.N, K = p.K;
  const int groups = K / kGroup;
  const size_t wrow = (size_t)K / 2;
  const int S = p.stages;

  const uint16_t* __restrict__ x = (const uint16_t*)p.x;
  const uint8_t* __restrict__ wq = (const uint8_t*)p.wq;
  const float* __restrict__ ws = p.ws;

  const int g = xcd_remap(blockIdx.x, gridDim.x);

  f32x4 acc[WM][WN];

  // ---- one K-stage range [s0, s1) of tile t --------------------------------------------
  auto run_segment = [&](int t, int s0, int s1, int& m0, int& n0) {
    int tm, tn;
    tile_coords(t, p.tiles_m, p.tiles_n, kGroupM, tm, tn);
    m0 = tm * BM;
    n0 = tn * BN;

    const uint8_t* bptr[WN];
    const float* sptr[WN];
    bool bok[WN];
#pragma unroll
    for (int fn = 0; fn < WN; ++fn) {
      const int n = n0 + (wn * WN + fn) * 16 + r16;
      bok[fn] = n < N;
      const int nc = min(n, N - 1);
      bptr[fn] = wq + (size_t)nc * wrow;
      sptr[fn] = ws + (size_t)nc * groups;
    }

    auto issue_a = [&](int s, uint8_t* buf) {
#pragma unroll
      for (int q = 0; q < kBlocksPerWave; ++q) {
        const int blk = wave * kBlocksPerWave + q;
        const int row = blk * 4 + j4;
        const int lch = r16 ^ (row & 15);
        const int gm = min(m0 + row, M - 1);
        const int gk = min(s * kStageK + lch * 8, K - 8);
        load_lds16(x + (size_t)gm * K + gk, buf + blk * 1024);
      }
    };
    // Raw loads only; the zero-scale select for columns past N / groups past K is applied by
    // the stage that consumes them, so no wait is forced right after the loads are issued.
    auto load_b = [&](int s, u32x4 (&raw)[WN], float (&sc)[WN]) {
      const int kgc = min(s * kGroupsPerStage + j4, groups - 1);
#pragma unroll
      for (int fn = 0; fn < WN; ++fn) {
        raw[fn] = *(const u32x4*)(bptr[fn] + (size_t)kgc * 16);
        sc[fn] = sptr[fn][kgc];
      }
    };

#pragma unroll
    for (int fm = 0; fm < WM; ++fm)
#pragma unroll
      for (int fn = 0; fn < WN; ++fn) acc[fm][fn] = f32x4{0.f, 0.f, 0.f, 0.f};

    u32x4 rawn[WN];
    float scn[WN];
    // one pipeline stage: operands of stage s are in `cur`; stage s+1 is fetched into `nxt`
    auto stage = [&](int s, int k_end, const uint8_t* cur, uint8_t* nxt) {
      wait_vmem();
      __syncthreads();
      u32x4 raw[WN];
      float sc[WN], neg8s[WN];
      const bool kok = s * kGroupsPerStage + j4 < groups;
#pragma unroll
      for (int fn = 0; fn < WN; ++fn) {
        raw[fn] = rawn[fn];
        sc[fn] = (bok[fn] && kok) ? scn[fn] : 0.0f;  // zero scale -> exact zero weights
        neg8s[fn] = -8.0f * sc[fn];
      }
      if (s + 1 < k_end) {
        issue_a(s + 1, nxt);
        load_b(s + 1, rawn, scn);
      }
      const uint8_t* abase = cur + (wm * WM * 16 + r16) * kRowBytes;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        u32x4 b[WN];
#pragma unroll
        for (int fn = 0; fn < WN; ++fn) b[fn] = dequant8<kBf16>(raw[fn][i], sc[fn], neg8s[fn]);
        const int pch = (4 * j4 + i) ^ r16;
#pragma unroll
        for (int fm = 0; fm < WM; ++fm) {
          const u32x4 a = *(const u32x4*)(abase + fm * 16 * kRowBytes + pch * 16);
#pragma unroll
          for (int fn = 0; fn < WN; ++fn) acc[fm][fn] = mfma16<kBf16>(a, b[fn], acc[fm][fn]);
        }
        // keep each K-step's operand reads and dequant inside the step: bounds live registers
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    // Segments are counted in steps of two stages (256 K), so both halves of the unrolled
    // loop body run unconditionally and the accumulators stay in one register class.
    const int k_end = 2 * s1;  // first stage not in this segment
    issue_a(2 * s0, lds0);
    load_b(2 * s0, rawn, scn);
    for (int sp = s0; sp < s1; ++sp) {
      stage(2 * sp, k_end, lds0, lds1);
      stage(2 * sp + 1, k_end, lds1, lds0);
    }
    __syncthreads();  // the next segment refills both LDS buffers
  };

  // ---- epilogues -----------------------------------------------------------------------
  auto store_tile = [&](int m0, int n0) {
#pragma unroll
    for (int fn = 0; fn < WN; ++fn) {
      const int n = n0 + (wn * WN + fn) * 16 + r16;
      if (n >= N) continue;
      const float bv = p.bias ? read_elem(p.bias, p.out_dtype, n) : 0.0f;
#pragma unroll
      for (int fm = 0; fm < WM; ++fm) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int m = m0 + (wm * WM + fm) * 16 + 4 * j4 + e;
          if (m < M) write_elem(p.y, p.out_dtype, (size_t)m * N + n, __fadd_rn(acc[fm][fn][e], bv));
        }
      }
    }
  };
  auto partial_index = [&](int fm, int fn, int e) {
    const int lm = (wm * WM + fm) * 16 + 4 * j4 + e;
    const int ln = (wn * WN + fn) * 16 + r16;
    return lm * BN + ln;
  };

  // ---- this workgroup's segment ----------------------------------------------------------
  int t, s0, s1, piece = 0;
  if (g < p.dp_tiles) {
    t = g;
    s0 = 0;
    s1 = S;
  } else {
    const int r = g - p.dp_tiles;
    t = p.dp_tiles + r / p.ksplit;
    piece = r - (t - p.dp_tiles) * p.ksplit;
    s0 = (int)((long long)piece * S / p.ksplit);
    s1 = (int)((long long)(piece + 1) * S / p.ksplit);
  }
  int m0, n0;
  run_segment(t, s0, s1, m0, n0);
  if (g < p.dp_tiles) {
    store_tile(m0, n0);
    return;
  }

  // ---- cut tile: publish this piece, the last arriving piece finishes the tile ------------
  const size_t tile_elems = (size_t)BM * BN;
  float* part = p.partial + (size_t)(g - p.dp_tiles) * tile_elems;  // slot = (tile, piece)
#pragma unroll
  for (int fm = 0; fm < WM; ++fm)
#pragma unroll
    for (int fn = 0; fn < WN; ++fn)
#pragma unroll
      for (int e = 0; e < 4; ++e) part[partial_index(fm, fn, e)] = acc[fm][fn][e];
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned old = atomicAdd(&p.counters[t - p.dp_tiles], 1u);
    s_last = (old == (unsigned)(p.ksplit - 1));
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  const float* first = p.partial + (size_t)(t - p.dp_tiles) * p.ksplit * tile_elems;
  for (int idx = threadIdx.x * 4; idx < BM * BN; idx += NW * 64 * 4) {
    f32x4 v = *(const f32x4*)(first + idx);
    for (int q = 1; q < p.ksplit; ++q) {
      const f32x4 w = *(const f32x4*)(first + (size_t)q * tile_elems + idx);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = __fadd_rn(v[e], w[e]);
    }
    const int m = m0 + idx / BN;
    if (m >= M) continue;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int n = n0 + idx % BN + e;
      if (n >= N) continue;
      const float bv = p.bias ? read_elem(p.bias, p.out_dtype, n) : 0.0f;
      write_elem(p.y, p.out_dtype, (size_t)m * N + n, __fadd_rn(v[e], bv));
    }
  }
  if (threadIdx.x == 0) p.counters[t - p.dp_tiles] = 0u;  // ready for the next call
}

}  // namespace

// ---- host-side launch ------------------------------------------------------------------------
template <bool kBf16, int WM, int WN, int NWM, int NWN>
static hipError_t launch_cfg(const W4A16Params& p, int grid, hipStream_t stream) {
  hipLaunchKernelGGL((w4a16_gemm_kernel<kBf16, WM, WN, NWM, NWN>), dim3(grid), dim3(64 * NWM * NWN), 0,
                     stream, p);
  return hipGetLastError();
}

const W4A16Config& w4a16_config(int id) {
  // {id, BM, BN}
  static const W4A16Config cfgs[] = {
      {0, 256, 256},  // WM 16, WN 4, 1 x 4 waves
      {1, 128, 256},  // WM 8
      {2, 64, 256},   // WM 4
      {3, 16, 256},   // WM 1
  };
  return cfgs[id];
}

hipError_t w4a16_launch(int cfg, bool bf16, const W4A16Params& p, int grid, hipStream_t stream) {
#define QL_CASE(ID, WM)                                                   \
  case ID:                                                                \
    return bf16 ? launch_cfg<true, WM, 4, 1, 4>(p, grid, stream)          \
                : launch_cfg<false, WM, 4, 1, 4>(p, grid, stream);
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

}  // namespace qlinear
