// W4A16 for up to 16 activation rows on MFMA: y[M,N] = x[M,K] @ (q[N,K] * s[N,K/32])^T (+ bias),
// bf16 or fp16 x read as is (no staging pass), q packed int4 in the reference layout
// (nodes/ComfyUI-Gfx906Int4/ops.py:108-126), fp32 group scales. HBM-bound like the M <= 4
// kernel, but the products run on v_mfma_f32_16x16x32_{bf16,f16}, whose 16 columns hold up to 16
// activation rows, so the VALU work per weight does not grow with M.
//
// * A workgroup owns B blocks of 16 output columns for all M rows (B = 1, 2 or 3, chosen by the
//   caller from N and the CU count); its 8 waves split K into 8 slices of gw quant groups
//   (gw = 4 ceil(G / 32) <= 16) and sum their partial results through LDS at the end, in wave
//   order (deterministic). Every workgroup reads all of x (M K 2 bytes, from L2), so larger B
//   means less x traffic per weight byte; B = 3 takes 120 KiB of LDS (one workgroup per CU).
// * Every load is issued at the start, nothing is recycled: each wave DMAs its B x 16 columns x
//   gw groups of packed weights (4 KiB per block) and their scales (1 KiB per block) into a
//   wave-private LDS region and holds its activation slice (16 rows x gw groups, 16 B per lane
//   and group) in registers.
//   The whole weight matrix is in flight from the first microseconds, which is what a one-shot
//   read of a few tens of MB needs to approach the HBM rate.
// * Per group t: A = the 16 activation rows of its 32 K, B = the 16 columns' weights as exact
//   16-bit numbers c + u (u = code + 8, built by v_bitop3 as in the M <= 4 kernel). One MFMA with
//   B = -(c + 8) in every slot gives -E = -(c + 8) * (sum of each row's 32 activations), in the
//   output layout, once per group; one MFMA per column block with C = -E then gives
//   D = sum x * code (exact products, fp32 sums). Lane l holds outputs of column l % 16 only, so
//   the group scale is one value per lane: acc += s * D.
// * Weights reach LDS as one 1 KiB DMA per (group quad, block): 16 columns x 4 groups, column r's
//   group 4tq + tt in 16-byte slot tt ^ (r / 4 % 4) of its 64 bytes, so the B-operand read (16
//   columns x 4 dwords of one group) touches 64 distinct banks and every 4-lane quad of the DMA
//   fetches one aligned 64-byte piece. The loads are issued in compute order and each (quad,
//   block) waits only for its own, so the arithmetic overlaps the stream.
// * Groups past this wave's slice or past K read zeros (out-of-range buffer offsets), rows past M
//   and columns past N likewise; K % 128 == 0, K <= 4096.
#include "common.hpp"
#include "launch.hpp"

namespace qlinear {

namespace {

constexpr int kSkWaves = 8;                 // K slices per workgroup
constexpr int kSkMaxGW = 16;                // quant groups per wave
constexpr int kSkColBytes = kSkMaxGW * 16;  // one column's slice of packed weights

// kSkBlocks 16-column blocks per workgroup (1-3)
template <bool kBf16, int kSkBlocks>
__global__ __launch_bounds__(64 * kSkWaves) void w4a16_skinny_kernel(W4A16Params p) {
  constexpr int kSkWBytes = kSkBlocks * 16 * kSkColBytes;   // 4 KiB of weights per wave and block
  constexpr int kSkSBytes = kSkBlocks * 16 * kSkMaxGW * 4;  // 1 KiB of scales per wave and block
  constexpr int kSkWaveBytes = kSkWBytes + kSkSBytes;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kSkWaves * kSkWaveBytes];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int M = p.M, N = p.N, K = p.K;
  const int G = K / kGroup;
  const int gw = 4 * ((G + 4 * kSkWaves - 1) / (4 * kSkWaves));
  const int g0 = w * gw;
  const int ng = max(0, min(gw, G - g0));  // this wave's groups: a multiple of 4 (G % 4 == 0)
  const int n0 = blockIdx.x * (16 * kSkBlocks);
  uint8_t* const mine = lds + w * kSkWaveBytes;
  const int r16 = lane & 15, q = lane >> 4;
  constexpr uint32_t kMagic = kBf16 ? 0x43004300u : 0x64006400u;
  constexpr float kC = kBf16 ? 128.0f : 1024.0f;  // value of the magic alone
  // (c + u_0, c + u_4) from nibbles 0 and 4 of v: one v_bitop3_b32 ((a & b) ^ c, table 0x6A)
  auto pair = [](uint32_t v) {
    return (uint32_t)__builtin_amdgcn_bitop3_b32(v, 0x000F000Fu, kMagic | 0x00080008u, 0x6A);
  };

  // ---- activations first (in-order vmcnt: the E pass below waits for them only) ---------------
  // lane (m = r16, q) of group t: x[m][32 (g0 + t) + 8q .. +7]
  const rsrc_t rx = make_rsrc(p.x, (uint32_t)((size_t)M * K * 2));
  // Every load below is issued unconditionally (an unused one gets an out-of-range offset and
  // reads zeros): no branches around loads, so the compiler's vmcnt bookkeeping and the waits
  // further down see one fixed sequence.
  auto pick = [](bool valid, uint32_t off) {
    uint32_t v = valid ? off : kOobOffset;
    asm volatile("" : "+v"(v));
    return v;
  };
  u32x4 xv[kSkMaxGW];
#pragma unroll
  for (int t = 0; t < kSkMaxGW; ++t)
    xv[t] = buf_load16(rx, pick(t < ng, (uint32_t)((r16 * K + (g0 + t) * kGroup + 8 * q) * 2)), 0);
  __builtin_amdgcn_sched_barrier(0);

  // ---- scales, then weights, by DMA -----------------------------------------------------------
  // scales [column][group] per block: lane i -> column i / 4, groups 4 (i % 4) .. +3
  const rsrc_t rw = make_rsrc(p.wq, (uint32_t)((size_t)N * (K / 2)));
  const rsrc_t rsc = make_rsrc(p.ws, (uint32_t)((size_t)N * G * 4));
#pragma unroll
  for (int b = 0; b < kSkBlocks; ++b) {
    const int gq = 4 * (lane & 3);
    const uint32_t vs = pick(gq < ng, (uint32_t)(((n0 + 16 * b + (lane >> 2)) * G + g0 + gq) * 4));
    buf_load16_lds(rsc, mine + kSkWBytes + b * 1024, vs, 0);
  }
  // weights: one 1 KiB instruction per (group quad tq, block b), issued in compute order; lane i ->
  // column r = i / 4, slot i % 4 holding group 4tq + ((i % 4) ^ (r / 4 % 4))
  {
    const int r = lane >> 2;
    const int tt = (lane & 3) ^ ((r >> 2) & 3);
#pragma unroll
    for (int tq = 0; tq < kSkMaxGW / 4; ++tq)
#pragma unroll
      for (int b = 0; b < kSkBlocks; ++b) {
        const uint32_t vo = pick(4 * tq < ng, (uint32_t)((n0 + 16 * b + r) * (K / 2) + (g0 + 4 * tq + tt) * 16));
        buf_load16_lds(rw, mine + (tq * kSkBlocks + b) * 1024, vo, 0);
      }
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- activations to dequant order ----------------------------------------------------------
  // (x0 x1)(x2 x3)(x4 x5)(x6 x7) -> (x0 x4)(x1 x5)(x2 x6)(x3 x7), matching pair(w >> 4i)
  u32x4 xp[kSkMaxGW];
#pragma unroll
  for (int t = 0; t < kSkMaxGW; ++t) {
    const u32x4 v = xv[t];
    xp[t] = u32x4{__builtin_amdgcn_perm(v[2], v[0], 0x05040100u), __builtin_amdgcn_perm(v[2], v[0], 0x07060302u),
                  __builtin_amdgcn_perm(v[3], v[1], 0x05040100u), __builtin_amdgcn_perm(v[3], v[1], 0x07060302u)};
  }

  // ---- products, each (group quad, block) as soon as its weights have landed -------------------
  // -(c + 8) as a 16-bit pair: bf16 -136 (0xC308), fp16 -1032 (0xE408)
  constexpr uint32_t kNegC8 = kBf16 ? 0xC308C308u : 0xE408E408u;
  const u32x4 negc8 = u32x4{kNegC8, kNegC8, kNegC8, kNegC8};
  constexpr int kWLoads = kSkMaxGW / 4 * kSkBlocks;  // weight instructions after the scales
  typedef __attribute__((address_space(3))) const uint32_t* lds_u32_ptr;
  typedef __attribute__((address_space(3))) const f32x4* lds_f32x4_ptr;
  const uint32_t base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)mine;
  const uint32_t wrow = base + (uint32_t)(r16 * 64 + 4 * q);
  const int wswz = (r16 >> 2) & 3;
  const uint32_t srow = base + (uint32_t)(kSkWBytes + r16 * 64);
  f32x4 acc[kSkBlocks];
#pragma unroll
  for (int b = 0; b < kSkBlocks; ++b) acc[b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  static_for<0, kSkMaxGW / 4>([&](auto tqc) {
    constexpr int tq = decltype(tqc)::value;
    if (4 * tq >= ng) return;
    f32x4 negE[4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) negE[tt] = mfma16<kBf16>(xp[4 * tq + tt], negc8, f32x4{0.0f, 0.0f, 0.0f, 0.0f});
    static_for<0, kSkBlocks>([&](auto bc) {
      constexpr int b = decltype(bc)::value;
      wait_vmcnt<kWLoads - 1 - (tq * kSkBlocks + b)>();
      // scales of column r16, groups 4tq .. 4tq + 3
      const f32x4 sc = *(lds_f32x4_ptr)(srow + b * 1024 + 16 * tq);
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const uint32_t wd = *(lds_u32_ptr)(wrow + (tq * kSkBlocks + b) * 1024 + ((tt ^ wswz) << 4));
        const u32x4 wv = u32x4{pair(wd), pair(wd >> 4), pair(wd >> 8), pair(wd >> 12)};
        const f32x4 d = mfma16<kBf16>(xp[4 * tq + tt], wv, negE[tt]);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[b][i] = fmaf(sc[tt], d[i], acc[b][i]);
      }
    });
  });

  // ---- sum the 8 K slices in wave order, epilogue ------------------------------------------------
  // lane l of block b holds column 16b + l % 16, rows 4(l / 16) + i; each wave writes its partials
  // over its own (already consumed) weight region.
  wait_vmcnt<0>();  // the DMA of unused quads (zeros) has landed too
  wait_lgkm();
#pragma unroll
  for (int b = 0; b < kSkBlocks; ++b) *(f32x4*)(mine + (b * 64 + lane) * 16) = acc[b];
  __syncthreads();
  constexpr int kCols = 16 * kSkBlocks;
  for (int tid = threadIdx.x; tid < 16 * kCols; tid += 64 * kSkWaves) {  // no barrier below
    const int m = tid / kCols, nl = tid % kCols;  // 16 rows x kCols columns
    const int b = nl >> 4;
    const int l = 16 * (m >> 2) + (nl & 15), i = m & 3;
    float v = 0.0f;
#pragma unroll
    for (int ww = 0; ww < kSkWaves; ++ww) v += ((const float*)(lds + ww * kSkWaveBytes))[(b * 64 + l) * 4 + i];
    const int n = n0 + nl;
    if (m < M && n < N) {
      float out = v * (p.row_scale ? p.row_scale[m] : 1.0f) + (p.bias ? read_elem(p.bias, p.out_dtype, n) : 0.0f);
      if (p.act == kActGeluTanh) out = gelu_tanh(round_to(p.out_dtype, out));
      write_elem(p.y, p.out_dtype, (size_t)m * N + n, out);
    }
  }
}

template <int kSkBlocks>
hipError_t skinny_launch_b(bool bf16, const W4A16Params& p, hipStream_t stream) {
  const dim3 grid((unsigned)((p.N + 16 * kSkBlocks - 1) / (16 * kSkBlocks))), block(64 * kSkWaves);
  if (bf16)
    hipLaunchKernelGGL((w4a16_skinny_kernel<true, kSkBlocks>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((w4a16_skinny_kernel<false, kSkBlocks>), grid, block, 0, stream, p);
  return hipGetLastError();
}

}  // namespace

hipError_t w4a16_skinny_launch(bool bf16, int blocks, const W4A16Params& p, hipStream_t stream) {
  switch (blocks) {
    case 1: return skinny_launch_b<1>(bf16, p, stream);
    case 2: return skinny_launch_b<2>(bf16, p, stream);
    default: return skinny_launch_b<3>(bf16, p, stream);
  }
}

}  // namespace qlinear
