// W8A8 GEMM for gfx950: acc[m,n] = sum_k xq[m,k] * wq[n,k] in int32 on v_mfma_i32_16x16x64_i8
// (exact integer arithmetic), epilogue y = float(acc) * (sx[m] * sw[n]) (+ bias[n]) with every
// step rounded in fp32 -- the scale-product order of the reference's int8 kernel
// (csrc/int8_gemm.hip:191-193, 209), whose block-32 scales become one per token and one per
// output channel here. out_dtype kI32 stores the raw accumulators.
//
// Same skeleton as w4a16_gemm.hip: A staged HBM -> LDS by global_load_lds_dwordx4 (256 K per
// stage, XOR-swizzled 16-byte chunks), B loaded straight into registers, lane (c, j) holding
// 64 contiguous bytes of weight row col0 + c (K elements 64j .. 64j+63 of the stage); MFMA i
// takes bytes 16i .. 16i+15 of them, so A is read at chunk 4j + i.
#include "common.hpp"
#include "launch.hpp"

namespace qlinear {

namespace {

constexpr int kStageK8 = 256;  // int8 K per stage = 256 bytes per A row
constexpr int kRowBytes8 = 256;
constexpr int kGroupM8 = kW8A8GroupM;

template <int WM, int WN, int NWM, int NWN>
__global__ __launch_bounds__(64 * NWM * NWN) void w8a8_gemm_kernel(W8A8Params p) {
  constexpr int NW = NWM * NWN;
  constexpr int BM = 16 * WM * NWM;
  constexpr int BN = 16 * WN * NWN;
  constexpr int kStageBytes = BM * kRowBytes8;
  constexpr int kBlocksPerWave = BM / 4 / NW;
  static_assert(BM % (4 * NW) == 0, "A tile must split into whole 1 KiB blocks per wave");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * kStageBytes];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave / NWN, wn = wave % NWN;
  const int r16 = lane & 15, j4 = lane >> 4;
  const int M = p.M, N = p.N, K = p.K;
  const int S = p.stages;

  const int g = xcd_remap(blockIdx.x, gridDim.x);
  int tm, tn;
  tile_coords(g, p.tiles_m, p.tiles_n, kGroupM8, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;

  const int8_t* bptr[WN];
  bool bok[WN];
#pragma unroll
  for (int fn = 0; fn < WN; ++fn) {
    const int n = n0 + (wn * WN + fn) * 16 + r16;
    bok[fn] = n < N;
    bptr[fn] = p.wq + (size_t)min(n, N - 1) * K;
  }

  auto issue_a = [&](int s, int buf) {
#pragma unroll
    for (int q = 0; q < kBlocksPerWave; ++q) {
      const int blk = wave * kBlocksPerWave + q;
      const int row = blk * 4 + j4;
      const int lch = r16 ^ lds_swz(row & 15);
      const int gm = min(m0 + row, M - 1);
      const int gk = min(s * kStageK8 + lch * 16, K - 16);
      load_lds16(p.xq + (size_t)gm * K + gk, lds + buf * kStageBytes + blk * 1024);
    }
  };
  auto load_b = [&](int s, u32x4 (&raw)[WN][4]) {
#pragma unroll
    for (int fn = 0; fn < WN; ++fn) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int k = s * kStageK8 + 64 * j4 + 16 * i;
        const bool ok = bok[fn] && k < K;
        const u32x4 v = *(const u32x4*)(bptr[fn] + min(k, K - 16));
        raw[fn][i] = ok ? v : u32x4{0u, 0u, 0u, 0u};  // zero weights past K / N
      }
    }
  };

  i32x4 acc[WM][WN];
#pragma unroll
  for (int fm = 0; fm < WM; ++fm)
#pragma unroll
    for (int fn = 0; fn < WN; ++fn) acc[fm][fn] = i32x4{0, 0, 0, 0};

  u32x4 rawn[WN][4];
  issue_a(0, 0);
  load_b(0, rawn);
  for (int s = 0; s < S; ++s) {
    wait_vmem();
    __syncthreads();
    u32x4 raw[WN][4];
#pragma unroll
    for (int fn = 0; fn < WN; ++fn)
#pragma unroll
      for (int i = 0; i < 4; ++i) raw[fn][i] = rawn[fn][i];
    const int buf = s & 1;
    if (s + 1 < S) {
      issue_a(s + 1, buf ^ 1);
      load_b(s + 1, rawn);
    }
    const uint8_t* abase = lds + buf * kStageBytes + (wm * WM * 16 + r16) * kRowBytes8;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int pch = (4 * j4 + i) ^ lds_swz(r16);
#pragma unroll
      for (int fm = 0; fm < WM; ++fm) {
        const u32x4 a = *(const u32x4*)(abase + fm * 16 * kRowBytes8 + pch * 16);
#pragma unroll
        for (int fn = 0; fn < WN; ++fn) acc[fm][fn] = mfma16_i8(a, raw[fn][i], acc[fm][fn]);
      }
    }
  }

#pragma unroll
  for (int fn = 0; fn < WN; ++fn) {
    const int n = n0 + (wn * WN + fn) * 16 + r16;
    if (n >= N) continue;
    const float swv = p.out_dtype == kI32 ? 0.0f : p.sw[n];
    const float bv = (p.bias && p.out_dtype != kI32) ? read_elem(p.bias, p.out_dtype, n) : 0.0f;
#pragma unroll
    for (int fm = 0; fm < WM; ++fm) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + (wm * WM + fm) * 16 + 4 * j4 + e;
        if (m >= M) continue;
        const size_t idx = (size_t)m * N + n;
        if (p.out_dtype == kI32) {
          ((int32_t*)p.y)[idx] = acc[fm][fn][e];
        } else {
          // each step rounded separately, as the reference's order: no contraction into an FMA
#pragma clang fp contract(off)
          float v = __fmul_rn((float)acc[fm][fn][e], __fmul_rn(p.sx[m], swv));
          if (p.bias) v = __fadd_rn(v, bv);
          write_elem(p.y, p.out_dtype, idx, v);
        }
      }
    }
  }
}

}  // namespace

const W8A8Config& w8a8_config(int id) {
  static const W8A8Config cfgs[] = {
      {0, 256, 256},  // WM 16, WN 4, 1 x 4 waves
      {1, 128, 256},
      {2, 64, 256},
      {3, 16, 256},
  };
  return cfgs[id];
}

template <int WM>
static hipError_t launch8(const W8A8Params& p, int grid, hipStream_t stream) {
  hipLaunchKernelGGL((w8a8_gemm_kernel<WM, 4, 1, 4>), dim3(grid), dim3(256), 0, stream, p);
  return hipGetLastError();
}

hipError_t w8a8_launch(int cfg, const W8A8Params& p, int grid, hipStream_t stream) {
  switch (cfg) {
    case 0: return launch8<16>(p, grid, stream);
    case 1: return launch8<8>(p, grid, stream);
    case 2: return launch8<4>(p, grid, stream);
    case 3: return launch8<1>(p, grid, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace qlinear
