// W4A16 GEMM for gfx950: y[M,N] = x[M,K] @ (q[N,K] * s[N,K/32])^T (+ bias), x fp16/bf16,
// q packed int4 in the reference layout (nodes/ComfyUI-Gfx906Int4/ops.py:108-126), fp32 group
// scales, fp32 MFMA accumulation.
//
// The reference computes this product as dequantize-then-matmul (nodes.py:43-52, 116) and its
// production kernel is a W4A4 v_dot8 GEMM (csrc/int4_gemm_scaled.hip:53-180); neither is the
// shape of this kernel. Design, per 256-thread workgroup (4 waves side by side along N, one wave
// per SIMD) and a BM x 256 output tile:
//
// * The cost that bounds this kernel is instruction issue: a SIMD issues one VALU or MFMA
//   instruction per 4 cycles, and one v_mfma_f32_16x16x32 occupies the matrix core for 16, so a
//   wave has 3 VALU slots per MFMA. The int4 -> 16-bit dequant costs 19 VALU per 8 weights, paid
//   once per weight per workgroup, so its cost per MFMA falls with the tile height: 2.4 VALU per
//   MFMA at BM = 128, 1.2 at BM = 256 (the large-M tile).
// * All global reads are raw buffer loads: a per-lane offset fixed for the whole K loop plus a
//   scalar offset bumped per stage, so the loop has no vector address arithmetic; rows past M,
//   columns past N and K past the end fall outside the buffer range and read as zeros.
// * A (activations): 128 K per stage, staged HBM -> registers -> LDS, double buffered in two
//   distinct LDS arrays. A row of a stage is 256 B = 16 chunks of 16 B; chunk c of row r sits
//   at slot c ^ lds_swz(r & 15), so an MFMA operand read is free of bank conflicts.
// * B (weights) never touches LDS. Lane (c = l%16, j = l/16) of a wave loads 16 B of weight row
//   n = col0 + c: the whole 32-element quant group j of the stage, with its one scale, and
//   dequantizes it in registers (dequant8: int4 -> q*s -> fp16/bf16). The MFMA K-slot map is
//   permuted to match: MFMA i of a stage takes, in K-slot block j, elements 32j + 8i .. +7; A is
//   read from LDS with the same map (chunk 4j + i), so every lane's load is one group.
// * Each wave owns a (16*WM) x 64 sub-tile of 16x16 accumulators (v_mfma_f32_16x16x32).
// * Pipeline, per stage s: issue the global loads of stage s+1 (B first, then A); run the
//   stage's MFMAs with operand reads kD fragments ahead and the next K-step's dequant spread
//   between them; kD fragments before the end, store the staged A of s+1 to the other LDS
//   buffer, dequantize K-step 0 of s+1, pass the workgroup barrier and issue the first operand
//   reads of s+1 -- the stage's last MFMAs then cover both the barrier and the read latency.
// * Optional row scales (the fp16 route for bf16 activations): x arrives pre-scaled per row by
//   2^-e (exact) and the epilogue multiplies by 2^e (exact).
// * Optional column scales (fp16 dequant): column n's group scales are multiplied by 2^-e_n
//   (exact) before q * s is rounded to fp16, and the epilogue multiplies by 2^e_n (exact), with
//   e_n from the column's scales (col_scales_kernel). Weights of any fp32 scale then dequantize
//   into fp16's normal range instead of overflowing (|s| > 8188) or going subnormal
//   (|s| < 2^-14). Columns already in range have factor 1, and a wave whose 64 columns all do
//   takes the plain epilogue (the factors cost nothing for ordinary checkpoints).
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
constexpr int kGroupM = kW4A16GroupM;
constexpr int kWaves = 4;
constexpr int kWN = 4;              // 16-column blocks per wave

template <bool kBf16, int WM, bool kCut, bool kKTail>
__global__ __launch_bounds__(64 * kWaves) void w4a16_gemm_kernel(W4A16Params p) {
  constexpr int WN = kWN;
  constexpr int BM = 16 * WM;
  constexpr int BN = 16 * WN * kWaves;
  constexpr int kStageBytes = BM * kRowBytes;
  constexpr int kLoadsA = BM / 16;        // 1 KiB (4-row) blocks each wave stages per stage
  constexpr int kQ = 4 * WM;              // operand fragments per stage: 4 K-steps x WM row blocks
  constexpr int kD = WM < 3 ? WM : 3;     // operand read-ahead, in fragments
  constexpr int kR = kD + 1;              // operand register ring
  static_assert(kQ % kR == 0, "the operand ring must restart at every stage");
  // kNB stage buffers in a ring, loads issued kNB-1 stages ahead: three for tiles up to 128 rows
  // (96 KiB of LDS), two for 256-row tiles (3 x 64 KiB would exceed the 160 KiB of a CU).
  constexpr int kNB = w4a16_nbuf(WM);
  constexpr int kLoadsPerStage = 2 * WN + kLoadsA;  // vmem instructions of one load_stage
  constexpr bool kRolled = kNB == 2;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kNB * kStageBytes];

  const int lane = threadIdx.x & 63;
  const int wn = threadIdx.x >> 6;
  const int r16 = lane & 15, j4 = lane >> 4;
  const int M = p.M, N = p.N, K = p.K;
  const int groups = K / kGroup;
  const int S = p.stages;                      // loop steps of kNB stages
  const int s_real = (K + kStageK - 1) / kStageK;  // stages that hold data

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

  // ---- buffer resources and per-lane offsets ----------------------------------------------
  // Per-lane offsets are fixed for the whole K loop; the stage (and, for A, the 16-row group of
  // the load, for B / scales the 16-column block) goes into the scalar offset.
  // Every tile of this kernel starts inside M and N (tile_coords gives tm < tiles_m, tn < tiles_n),
  // so rows and cols are >= 1. (A max(0, .) here costs 8-9 VGPRs in the K-cut instances and
  // measurably slows them.)
  const int rows = min(M - m0, BM), cols = min(N - n0, BN);
  const rsrc_t rs_a = make_rsrc((const uint16_t*)p.x + (size_t)m0 * K, (uint32_t)rows * K * 2);
  const rsrc_t rs_b = make_rsrc((const uint8_t*)p.wq + (size_t)n0 * (K / 2), (uint32_t)cols * (K / 2));
  // scales [N, K/32], or group-major [K/32, N] (scales_kn: a stage's 4 groups of the tile's
  // columns are 4 runs of BN * 4 bytes instead of BN runs of 16; the range ends at the tile's last
  // column of the last group row, and a column past N of an earlier row reads a scale of the next
  // row, which only enters that column's own accumulators, never stored)
  const int kn = p.scales_kn;
  const rsrc_t rs_s = kn ? make_rsrc(p.ws + n0, (uint32_t)((groups - 1) * N + cols) * 4)
                         : make_rsrc(p.ws + (size_t)n0 * groups, (uint32_t)cols * groups * 4);
  // A: wave wn stages rows [wn*BM/4, (wn+1)*BM/4) in kLoadsA loads of 4 rows; load q covers row
  // wn*BM/4 + 4q + j4, whose swizzle depends on q % 4 only
  constexpr int kVoA = kLoadsA < 4 ? kLoadsA : 4;
  uint32_t vo_a[kVoA];
  auto a_row = [&](int q) { return (wn * kLoadsA + q) * 4 + j4; };
  auto a_lch = [&](int q) { return r16 ^ lds_swz(a_row(q) & 15); };
#pragma unroll
  for (int q = 0; q < kVoA; ++q) vo_a[q] = (uint32_t)(a_row(q) * K + a_lch(q) * 8) * 2;
  const uint32_t a_q4_step = 16u * K * 2;  // four loads further down = 16 rows
  const int col0 = wn * WN * 16 + r16;
  const uint32_t vo_b = (uint32_t)col0 * (K / 2) + j4 * 16;
  const uint32_t vo_s = kn ? ((uint32_t)j4 * N + col0) * 4 : ((uint32_t)col0 * groups + j4) * 4;
  const uint32_t b_fn_step = 16u * (K / 2), s_fn_step = kn ? 16u * 4 : 16u * groups * 4;
  const uint32_t s_stage = kn ? (uint32_t)kGroupsPerStage * N * 4 : (uint32_t)kGroupsPerStage * 4;

  // Global loads of stage s: B (raw int4 + scales) into registers, then A straight into the LDS
  // buffer `dst`, one vector-memory instruction per call (index l < kLoadsPerStage), so a stage's
  // loads can be spread between MFMAs: issued in one burst they fill the address FIFO of the
  // CU's texture unit and the wave, which issues in order, stalls its MFMAs behind them. With
  // kKTail (K not a multiple of 128) a stage that reaches past K masks the chunks / groups past
  // the end with an out-of-range offset. `live` false turns every load into an out-of-range one
  // (a stage past the segment): no memory traffic, no branch.
  const rsrc_t rs_none = make_rsrc(p.ws, 0);
  auto load_one = [&](int l, int s, bool live, u32x4 (&raw)[WN], float (&sc)[WN], uint8_t* dst) {
    if (l < 2 * WN) {
      uint32_t vb = vo_b, vs = vo_s;
      if constexpr (kKTail) {
        const bool gok = s * kGroupsPerStage + j4 < groups;
        vb = gok ? vb : kOobOffset;
        vs = gok ? vs : kOobOffset;
      }
      if (l < WN) {
        raw[l] = buf_load16(live ? rs_b : rs_none, vb, s * 64 + l * b_fn_step);
      } else {
        sc[l - WN] = buf_load_f32(live ? rs_s : rs_none, vs, s * s_stage + (l - WN) * s_fn_step);
      }
    } else {
      const int q = l - 2 * WN;
      uint32_t va = vo_a[q % kVoA];
      if constexpr (kKTail) va = s * kStageK + a_lch(q) * 8 < K ? va : kOobOffset;
      buf_load16_lds(live ? rs_a : rs_none, dst + (wn * kLoadsA + q) * 1024, va, s * 256 + (q / 4) * a_q4_step);
    }
  };
  auto load_stage = [&](int s, bool live, u32x4 (&raw)[WN], float (&sc)[WN], uint8_t* dst) {
#pragma unroll
    for (int l = 0; l < kLoadsPerStage; ++l) load_one(l, s, live, raw, sc, dst);
  };
  // operand fragment q = i * WM + fm of a stage: rows fm*16 + (l % 16), K-step i (chunk 4j + i).
  // One lane address per (buffer, K-step), kept opaque to the optimizer so it does not fold the
  // buffer offset into the immediate (which tops out at 64 KiB) and materialize an address per
  // fragment; the row block fm*4 KiB is the ds_read immediate.
  typedef __attribute__((address_space(3))) const u32x4* lds_frag_ptr;
  const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)lds;
  uint32_t fbase[kNB][4];
#pragma unroll
  for (int k = 0; k < kNB; ++k)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      fbase[k][i] = lds_base + k * kStageBytes + r16 * kRowBytes + (((4 * j4 + i) ^ lds_swz(r16)) * 16);
      asm volatile("" : "+v"(fbase[k][i]));
    }
  auto frag = [&](int k, int q) {
    const int i = q / WM, fm = q % WM;
    return *(lds_frag_ptr)(fbase[k][i] + fm * 16 * kRowBytes);
  };

  // Accumulators start as the result of an MFMA on zeros rather than as a plain zero constant:
  // the compiler then keeps them in AGPRs across the K loop instead of copying every one between
  // AGPRs and VGPRs at each loop iteration.
  f32x4 acc[WM][WN];
#pragma unroll
  for (int fm = 0; fm < WM; ++fm)
#pragma unroll
    for (int fn = 0; fn < WN; ++fn)
      acc[fm][fn] = mfma16<kBf16>(u32x4{0u, 0u, 0u, 0u}, u32x4{0u, 0u, 0u, 0u}, f32x4{0.f, 0.f, 0.f, 0.f});

  // Column factors (fp16 dequant): the lane's weight columns n0 + col0 + 16 fn dequantize with
  // their group scales times 1 / col_scale[n] (an exact power of two), undone in the epilogue.
  // Loaded here, ahead of the prologue's loads; csd is formed after the prologue's wait, so the
  // load's latency hides behind the first stage's.
  float csv[WN], csd[WN];
  {
    const float* cs_p = p.col_scale;
#pragma unroll
    for (int fn = 0; fn < WN; ++fn) {
      const int n = n0 + col0 + 16 * fn;
      csv[fn] = (cs_p && n < N) ? cs_p[n] : 1.0f;
    }
  }

  // kNB register sets for the raw weights, rotating with the LDS buffers.
  u32x4 raw[kNB][WN];
  float sc[kNB][WN];
  u32x4 b[WN], bn[WN];  // dequantized weights of the current / the next K-step
  u32x4 ar[kR];         // operand ring

  // One pipeline stage s, held in ring slot k = s % kNB. Entering: buffer k holds A of stage s
  // (published by the last barrier), raw[k]/sc[k] its weights, bn its dequantized K-step 0,
  // ar[0..kD-1] its first kD operand fragments (reads issued); the loads of stages s+1 ..
  // s+kNB-2 are in flight. Fragment q sits in ring slot q % kR.
  // Unrolled (kc = ring slot as a constant): the loop body holds kNB stages with fixed slots.
  // Rolled (kRolled, two buffers, 256-row tiles): one stage per loop iteration; the LDS slot is a
  // runtime value (per-stage base addresses fcur / fnxt), the weights of s+1 land in raw[1] and
  // move to raw[0] at the end. 256 accumulators leave the register allocator no spare AGPRs, and
  // a two-stage loop body makes it shuffle them between stages; one stage per iteration does not.
  auto stage = [&](auto kc, int s, int s_end) {
    constexpr int k = kRolled ? 0 : decltype(kc)::value;
    constexpr int k1 = kRolled ? 1 : (k + 1) % kNB, kl = kRolled ? 1 : (k + kNB - 1) % kNB;
    const int s_load = s + kNB - 1;
    const bool live = s_load < s_end;
    const int slot = kRolled ? (s & 1) : k;  // LDS buffer of stage s
    uint32_t fcur[4], fnxt[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      fcur[i] = kRolled ? fbase[0][i] + slot * kStageBytes : fbase[k][i];
      fnxt[i] = kRolled ? fbase[0][i] + (slot ^ 1) * kStageBytes : fbase[k1 % kNB][i];
    }
    auto fragb = [&](const uint32_t (&fb)[4], int q) {
      const int i = q / WM, fm = q % WM;
      return *(lds_frag_ptr)(fb[i] + fm * 16 * kRowBytes);
    };
    uint8_t* const ldst = lds + (kRolled ? (slot ^ 1) : kl) * kStageBytes;  // target of the loads
    float neg8s[WN];
#pragma unroll
    for (int fn = 0; fn < WN; ++fn) neg8s[fn] = -8.0f * sc[k][fn];
    static_for<0, kQ>([&](auto qc) {
      constexpr int q = decltype(qc)::value;
      constexpr int i = q / WM, fm = q % WM;
      if constexpr (fm == 0) {
#pragma unroll
        for (int fn = 0; fn < WN; ++fn) b[fn] = bn[fn];
      }
      // this step's share of the loads of stage s+kNB-1, spread over the first kLoadWindow steps
      // (all before the hand-over; with two buffers in the first half, as the hand-over waits
      // for them)
      constexpr int kLoadWindow = kNB == 2 ? kQ / 2 : kQ - kD;
      static_for<0, kLoadsPerStage>([&](auto lc) {
        constexpr int l = decltype(lc)::value;
        if constexpr (l * kLoadWindow / kLoadsPerStage == q)
          load_one(l, s_load, live, raw[kl], sc[kl], ldst);
      });
      if constexpr (q == kQ - kD) {
        // hand-over to stage s+1: its K-step 0 dequantized, its A (loaded into buffer k1 since
        // kNB-2 stages ago) complete, the barrier; from here the ring reads the first fragments
        // of s+1, and the MFMAs q .. kQ-1 of this stage cover the barrier and their latency
#pragma unroll
        for (int fn = 0; fn < WN; ++fn) {
          sc[k1][fn] *= csd[fn];  // the scales of s+1, each multiplied by its column factor once
          bn[fn] = dequant8<kBf16>(raw[k1][fn][0], sc[k1][fn], -8.0f * sc[k1][fn]);
        }
        wait_vmcnt<(kNB - 2) * kLoadsPerStage>();  // this wave's loads of s+1 have landed
        wait_lgkm();                                // its operand reads of buffer k are done
        barrier_no_fence();
      }
      if constexpr (q + kD < kQ) {
        ar[(q + kD) % kR] = fragb(fcur, q + kD);
      } else {
        ar[(q + kD) % kR] = fragb(fnxt, q + kD - kQ);  // past the segment: read, never used
      }
#pragma unroll
      for (int fn = 0; fn < WN; ++fn) acc[fm][fn] = mfma16<kBf16>(b[fn], ar[q % kR], acc[fm][fn]);
      // dequant of K-step i+1, spread over the row blocks of K-step i
      if constexpr (i < 3) {
#pragma unroll
        for (int fn = 0; fn < WN; ++fn)
          if ((WM >= 4 ? fn * (WM / 4) : fn % WM) == fm) bn[fn] = dequant8<kBf16>(raw[k][fn][i + 1], sc[k][fn], neg8s[fn]);
      }
      __builtin_amdgcn_sched_barrier(0);
    });
    if constexpr (kRolled) {
#pragma unroll
      for (int fn = 0; fn < WN; ++fn) {
        raw[0][fn] = raw[1][fn];
        sc[0][fn] = sc[1][fn];
      }
    }
  };

  // ---- prologue: stages up to kNB-2 ahead in flight, the first one published -----------------
  // Stages at or past s_end (the segment's end, or the last stage holding data) load nothing.
  const int s_first = kNB * s0;
  const int s_end = min(kNB * s1, s_real);
  static_for<0, kNB - 1>([&](auto kc) {
    constexpr int k = decltype(kc)::value;
    load_stage(s_first + k, s_first + k < s_end, raw[k], sc[k], lds + k * kStageBytes);
  });
  wait_vmcnt<(kNB - 2) * kLoadsPerStage>();
#pragma unroll
  for (int fn = 0; fn < WN; ++fn) {
    csd[fn] = pow2_recip(csv[fn]);
    sc[0][fn] *= csd[fn];
    bn[fn] = dequant8<kBf16>(raw[0][fn][0], sc[0][fn], -8.0f * sc[0][fn]);
  }
  barrier_no_fence();
#pragma unroll
  for (int d = 0; d < kD; ++d) ar[d] = frag(0, d);

  // Segments are counted in steps of kNB stages, so every stage of the unrolled loop body has a
  // fixed ring slot and the accumulators stay in one register class.
  if constexpr (kRolled) {
    for (int st = s_first; st < kNB * s1; ++st) stage(ic<0>{}, st, s_end);
  } else {
    for (int sp = s0; sp < s1; ++sp) {
      static_for<0, kNB>([&](auto kc) { stage(kc, kNB * sp + decltype(kc)::value, s_end); });
    }
  }

  // ---- epilogue ----------------------------------------------------------------------------
  // The MFMAs take the weights as their first operand, so each 16x16 block holds y^T: lane l has
  // y[m][n .. n+3] for m = block row + l % 16, n = block column + 4 * (l / 16) -- four adjacent
  // outputs, stored with one 8-byte (16-bit out) or 16-byte (fp32 out) store.
  // A whole tile goes to y (row scale, bias, out dtype); a cut tile's piece goes as plain fp32 to
  // its partial slot, a tile-local [BM][BN] array. Same store loop for both.
  void* dst = p.y;
  int dst_m0 = m0, dst_n0 = n0, dst_M = M, dst_N = N, dst_dtype = p.out_dtype, dst_act = p.act;
  const void* bias = p.bias;
  const float* row_scale = p.row_scale;
  const float* col_scale = p.col_scale;
  const void* resid = p.residual;
  if constexpr (kCut) {
    resid = nullptr;
    dst = p.partial + (size_t)g * (BM * BN);
    dst_m0 = 0;
    dst_n0 = 0;
    dst_M = BM;
    dst_N = BN;
    dst_dtype = kF32;
    dst_act = kActNone;
    bias = nullptr;
    row_scale = nullptr;
    col_scale = nullptr;
  }
  const bool vec = dst_N % 4 == 0 && ((uintptr_t)dst & 15) == 0;
  float bv[WN][4];
#pragma unroll
  for (int fn = 0; fn < WN; ++fn) {
    const int n = dst_n0 + (wn * WN + fn) * 16 + 4 * j4;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      bv[fn][e] = (bias && n + e < dst_N) ? read_elem(bias, p.out_dtype == kBF16AsF16 ? kBF16 : p.out_dtype, n + e)
                                          : 0.0f;
  }
  // The wave's output columns are the columns of its K loop (csd). When every one has factor 1
  // (ordinary checkpoints) the plain epilogue runs; the choice is uniform over the wave.
  bool col_one = true;
#pragma unroll
  for (int fn = 0; fn < WN; ++fn) col_one = col_one && csd[fn] == 1.0f;
  const bool scaled_cols = col_scale != nullptr && __builtin_amdgcn_ballot_w64(!col_one) != 0;
  auto store_tile = [&](auto kc) {
    constexpr bool kColScaled = decltype(kc)::value;
    float cu[WN][4];
#pragma unroll
    for (int fn = 0; fn < WN; ++fn) {
      const int n = dst_n0 + (wn * WN + fn) * 16 + 4 * j4;
#pragma unroll
      for (int e = 0; e < 4; ++e) cu[fn][e] = (kColScaled && n + e < dst_N) ? col_scale[n + e] : 1.0f;
    }
#pragma unroll
    for (int fm = 0; fm < WM; ++fm) {
      const int m = dst_m0 + fm * 16 + r16;
      if (m < dst_M) {
        const float rs = row_scale ? row_scale[m] : 1.0f;
        // kBF16AsF16: the row's fp16 storage factor from its bound (see f16_row_factor); the
        // tile column 0 workgroup's wave 0 publishes 2^e_m
        const int rnd = dst_dtype == kBF16AsF16 ? (int)kBF16 : dst_dtype;
        float rdown = 1.0f;
        if (dst_dtype == kBF16AsF16) {
          float up;
          f16_row_factor(w4a16_row_bound(rs, p.out_bound[0], p.out_bound[1]), rdown, up);
          if (tn == 0 && wn == 0 && j4 == 0) p.out_row_scale[m] = up;
        }
#pragma unroll
        for (int fn = 0; fn < WN; ++fn) {
          const int n = dst_n0 + (wn * WN + fn) * 16 + 4 * j4;
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            v[e] = kColScaled ? acc[fm][fn][e] * rs * cu[fn][e] + bv[fn][e] : acc[fm][fn][e] * rs + bv[fn][e];
            if (dst_act == kActGeluTanh) v[e] = gelu_tanh(round_to(rnd, v[e]));
            if (dst_dtype == kBF16AsF16) v[e] = round_to(kBF16, v[e]) * rdown;  // exact in fp16
          }
          const size_t off = (size_t)m * dst_N + n;
          const int st = dst_dtype == kBF16AsF16 ? (int)kF16 : dst_dtype;  // storage dtype
          if (resid) {  // gated residual on the rounded outputs (uniform over the workgroup)
            const size_t goff = (size_t)(m / p.gate_rows) * dst_N + n;
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (n + e < dst_N)
                v[e] = read_elem(resid, st, off + e) + read_elem(p.gate, st, goff + e) * round_to(st, v[e]);
          }
          if (vec && n + 3 < dst_N) {
            if (st == kF32) {
              *(f32x4*)((float*)dst + off) = f32x4{v[0], v[1], v[2], v[3]};
            } else {
              typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
              const bool bf = st == kBF16;
              const u32x2 w = {bf ? pack2_bf16(v[0], v[1]) : pack2_f16(v[0], v[1]),
                               bf ? pack2_bf16(v[2], v[3]) : pack2_f16(v[2], v[3])};
              *(u32x2*)((uint16_t*)dst + off) = w;
            }
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (n + e < dst_N) write_elem(dst, st, off + e, v[e]);
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  if (scaled_cols) {
    store_tile(ic<1>{});
  } else {
    store_tile(ic<0>{});
  }
}

// Sums the ksplit fp32 partials of every cut tile in piece order, applies the row and column
// scales and the bias, and stores y. Grid: (cut tiles) x (BM*BN / 1024) workgroups of 256 threads, 4 elements
// per thread.
__global__ __launch_bounds__(256) void w4a16_reduce_kernel(W4A16Params p, int BM, int BN, int group_m) {
  const int tl = blockIdx.y;  // cut tile index
  const int t = p.dp_tiles + tl;
  int tm, tn;
  tile_coords(t, p.tiles_m, p.tiles_n, group_m, tm, tn);
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
  const bool as_f16 = p.out_dtype == kBF16AsF16;
  const int rnd = as_f16 ? (int)kBF16 : p.out_dtype;  // the logical output dtype
  float rdown = 1.0f;
  if (as_f16) {  // the row's fp16 storage factor; the thread holding the tile's column 0 publishes it
    float up;
    f16_row_factor(w4a16_row_bound(rs, p.out_bound[0], p.out_bound[1]), rdown, up);
    if (tn == 0 && idx % BN == 0) p.out_row_scale[m] = up;
  }
  const int n0 = tn * BN + idx % BN;  // a multiple of 4
  f32x4 cu = {1.0f, 1.0f, 1.0f, 1.0f};
  if (p.col_scale) {
    if (n0 + 3 < p.N) {
      cu = *(const f32x4*)(p.col_scale + n0);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) cu[e] = n0 + e < p.N ? p.col_scale[n0 + e] : 1.0f;
    }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int n = n0 + e;
    if (n >= p.N) continue;
    const float bv = p.bias ? read_elem(p.bias, rnd, n) : 0.0f;
    float out = v[e] * rs * cu[e] + bv;
    if (p.act == kActGeluTanh) out = gelu_tanh(round_to(rnd, out));
    if (as_f16) out = round_to(kBF16, out) * rdown;  // exact in fp16
    if (p.residual)  // gated residual on the rounded output
      out = read_elem(p.residual, rnd, (size_t)m * p.N + n) +
            read_elem(p.gate, rnd, (size_t)(m / p.gate_rows) * p.N + n) * round_to(rnd, out);
    write_elem(p.y, as_f16 ? (int)kF16 : p.out_dtype, (size_t)m * p.N + n, out);
  }
}

// x [M, K] (fp32 / fp16 / bf16) -> x16 [M, K] fp16 scaled by 2^-e_m per row, row_scale[m] = 2^e_m,
// with e_m chosen so that max |x16| lies in [2^14, 2^15): every bf16 value maps exactly (fp16
// keeps 11 mantissa bits), and no row can overflow fp16. One workgroup per row, 8 elements per
// thread and step (16-byte loads for 16-bit inputs). R > 0 (K <= 2048 R): thread t holds elements
// 8t + 2048 r (r < R) in registers, all R loads issued before the first use, the row read once.
// R = 0 (longer rows): a strided loop, the row read twice (max, then convert; the second read
// hits L2).
template <int DT, int R>
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
  auto store8 = [&](int k, const float (&v)[8], int e) {
    u32x4 out;
#pragma unroll
    for (int q = 0; q < 4; ++q) out[q] = pack2_f16(ldexpf(v[2 * q], -e), ldexpf(v[2 * q + 1], -e));
    *(u32x4*)(x16 + base + k) = out;
  };
  auto row_exponent = [&](float amax) {
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
    return e;
  };
  float amax = 0.0f;
  if constexpr (R > 0) {
    float v[R][8];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int k = threadIdx.x * 8 + 2048 * r;
      if (k < K) {
        load8(k, v[r]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[r][e] = 0.0f;
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[r][e]));
    const int e = row_exponent(amax);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int k = threadIdx.x * 8 + 2048 * r;
      if (k < K) store8(k, v[r], e);
    }
  } else {
    for (int k = threadIdx.x * 8; k < K; k += 256 * 8) {
      float v[8];
      load8(k, v);
#pragma unroll
      for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[e]));
    }
    const int e = row_exponent(amax);
    for (int k = threadIdx.x * 8; k < K; k += 256 * 8) {
      float v[8];
      load8(k, v);
      store8(k, v, e);
    }
  }
}

// Per-column power-of-two factors of the fp16 dequant: one wave per column n. A column whose
// dequantized weights q s already lie in fp16's normal range for every code (every nonzero |s| >=
// 2^-14 and 8 max |s| <= 65504) gets 1, so the tile kernels compute exactly what a plain fp16
// dequant computes; any other column gets 2^e with 8 max |s| 2^-e in [2^14, 2^15) (|q s| <= 8 |s|
// for codes in [-8, 7]): q s 2^-e is then a normal fp16 number for every code of the column's
// largest group and overflows for none. e is clamped to [-126, 126] (2^e and 2^-e both normal
// fp32); a column whose largest scale is not finite gets 1. Four columns per 256-thread
// workgroup.
__global__ __launch_bounds__(256) void col_scales_kernel(const float* __restrict__ ws, float* __restrict__ cs, int N,
                                                         int groups) {
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (n >= N) return;
  const float* row = ws + (size_t)n * groups;
  float mx = 0.0f, mn = INFINITY;
  for (int g = lane; g < groups; g += kWave) {
    const float a = fabsf(row[g]);
    mx = fmaxf(mx, a);
    if (a > 0.0f) mn = fminf(mn, a);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    mx = fmaxf(mx, __shfl_xor(mx, off, kWave));
    mn = fminf(mn, __shfl_xor(mn, off, kWave));
  }
  if (lane == 0) {
    int e = 0;
    const bool in_range = mn >= 0x1p-14f && 8.0f * mx <= 65504.0f;
    if (!in_range && mx > 0.0f && mx <= 3.4028235e38f) {
      int E;
      frexpf(mx, &E);  // mx = f 2^E, f in [0.5, 1): 8 mx in [2^(E+2), 2^(E+3))
      e = min(max(E - 12, -126), 126);
    }
    cs[n] = ldexpf(1.0f, e);
  }
}

// Group-major copy of the scales: kn[g][n] = ws[n][g]. 32 x 32 blocks through LDS (a padded row
// keeps the column reads conflict free), so both the reads and the writes are 128-byte runs.
// 256 threads: thread (tx, ty) moves rows ty, ty + 8, ty + 16, ty + 24 of the block.
__global__ __launch_bounds__(256) void scales_kn_kernel(const float* __restrict__ ws, float* __restrict__ kn, int N,
                                                        int groups) {
  __shared__ float tile[32][33];
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  const int n0 = blockIdx.x * 32, g0 = blockIdx.y * 32;
#pragma unroll
  for (int r = 0; r < 32; r += 8) {
    const int n = n0 + ty + r, g = g0 + tx;
    if (n < N && g < groups) tile[ty + r][tx] = ws[(size_t)n * groups + g];
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 32; r += 8) {
    const int g = g0 + ty + r, n = n0 + tx;
    if (n < N && g < groups) kn[(size_t)g * N + n] = tile[tx][ty + r];
  }
}

// Per-column L1 norms of the dequantized weight, one wave per column (4 per workgroup), and the
// workgroup's maximum into partial[blockIdx.x]: sum over groups of |s_g| * sum of |codes| (the
// integer sums are exact; the fp32 products and sum round, which the 2^-10 margin of the final
// bound covers for K up to 2^22).
__global__ __launch_bounds__(256) void w4a16_col_l1_kernel(const uint8_t* __restrict__ wq, const float* __restrict__ ws,
                                                           int N, int K, float* __restrict__ partial) {
  __shared__ float red[4];
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  float sum = 0.0f;
  if (n < N) {
    const int groups = K / kGroup;
    const uint8_t* row = wq + (size_t)n * (K / 2);
    for (int g = lane; g < groups; g += kWave) {
      const u32x4 w = *(const u32x4*)(row + (size_t)g * 16);
      int a = 0;
#pragma unroll
      for (int d = 0; d < 4; ++d)
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const int c = (int)((w[d] >> (4 * t)) & 0xFu);
          a += c >= 8 ? 16 - c : c;
        }
      sum += fabsf(ws[(size_t)n * groups + g]) * (float)a;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off, kWave);
  }
  if (lane == 0) red[threadIdx.x >> 6] = sum;
  __syncthreads();
  if (threadIdx.x == 0) partial[blockIdx.x] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// bound[0] = max over the partial maxima * (1 + 2^-10), bound[1] = max |bias|: one workgroup.
__global__ __launch_bounds__(256) void w4a16_bound_reduce_kernel(const float* __restrict__ partial, int np,
                                                                 const void* __restrict__ bias, int bias_dtype, int N,
                                                                 float* __restrict__ bound) {
  __shared__ float red[2][4];
  float a = 0.0f, b = 0.0f;
  for (int i = threadIdx.x; i < np; i += 256) a = fmaxf(a, partial[i]);
  if (bias)
    for (int i = threadIdx.x; i < N; i += 256) b = fmaxf(b, fabsf(read_elem(bias, bias_dtype, (size_t)i)));
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    a = fmaxf(a, __shfl_xor(a, off, kWave));
    b = fmaxf(b, __shfl_xor(b, off, kWave));
  }
  if ((threadIdx.x & 63) == 0) {
    red[0][threadIdx.x >> 6] = a;
    red[1][threadIdx.x >> 6] = b;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    bound[0] = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3])) * (1.0f + 0x1p-10f);
    bound[1] = fmaxf(fmaxf(red[1][0], red[1][1]), fmaxf(red[1][2], red[1][3]));
  }
}

template <int DT>
hipError_t rows_launch_r(const void* x, void* x16, float* row_scale, int64_t M, int64_t K, hipStream_t stream) {
  const dim3 grid((unsigned)M), block(256);
  if (K <= 2048)
    hipLaunchKernelGGL((rows_to_scaled_f16_kernel<DT, 1>), grid, block, 0, stream, x, (_Float16*)x16, row_scale,
                       (int)K);
  else if (K <= 4096)
    hipLaunchKernelGGL((rows_to_scaled_f16_kernel<DT, 2>), grid, block, 0, stream, x, (_Float16*)x16, row_scale,
                       (int)K);
  else if (K <= 8192)
    hipLaunchKernelGGL((rows_to_scaled_f16_kernel<DT, 4>), grid, block, 0, stream, x, (_Float16*)x16, row_scale,
                       (int)K);
  else if (K <= 16384)
    hipLaunchKernelGGL((rows_to_scaled_f16_kernel<DT, 8>), grid, block, 0, stream, x, (_Float16*)x16, row_scale,
                       (int)K);
  else
    hipLaunchKernelGGL((rows_to_scaled_f16_kernel<DT, 0>), grid, block, 0, stream, x, (_Float16*)x16, row_scale,
                       (int)K);
  return hipGetLastError();
}

}  // namespace

// ---- host-side launch ------------------------------------------------------------------------
template <bool kBf16, int WM, bool kKTail>
static hipError_t launch_cfg(const W4A16Params& p, hipStream_t stream) {
  constexpr int BM = 16 * WM, BN = 16 * kWN * kWaves;
  const int tiles = p.tiles_m * p.tiles_n;
  if (p.dp_tiles > 0)
    hipLaunchKernelGGL((w4a16_gemm_kernel<kBf16, WM, false, kKTail>), dim3(p.dp_tiles), dim3(64 * kWaves), 0, stream,
                       p);
  const int cut = tiles - p.dp_tiles;
  if (cut > 0) {
    hipLaunchKernelGGL((w4a16_gemm_kernel<kBf16, WM, true, kKTail>), dim3(cut * p.ksplit), dim3(64 * kWaves), 0,
                       stream, p);
    hipLaunchKernelGGL(w4a16_reduce_kernel, dim3((BM * BN + 1023) / 1024, cut), dim3(256), 0, stream, p, BM, BN,
                       kGroupM);
  }
  return hipGetLastError();
}

template <bool kBf16, int WM>
static hipError_t launch_k(const W4A16Params& p, hipStream_t stream) {
  // K a multiple of 128 (every stage full): no K masking in the loads
  return p.K % kStageK == 0 ? launch_cfg<kBf16, WM, false>(p, stream) : launch_cfg<kBf16, WM, true>(p, stream);
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

int w4a16_steps(int cfg, int64_t K) {
  const int wm = w4a16_config(cfg).BM / 16;
  const int64_t per_step = (int64_t)kStageK * w4a16_nbuf(wm);
  return (int)((K + per_step - 1) / per_step);
}

hipError_t w4a16_launch(int cfg, bool bf16, const W4A16Params& p, hipStream_t stream) {
#define QL_CASE(ID, WM) \
  case ID:              \
    return bf16 ? launch_k<true, WM>(p, stream) : launch_k<false, WM>(p, stream);
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
  switch (dtype) {
    case kF32: return rows_launch_r<kF32>(x, x16, row_scale, M, K, stream);
    case kF16: return rows_launch_r<kF16>(x, x16, row_scale, M, K, stream);
    default: return rows_launch_r<kBF16>(x, x16, row_scale, M, K, stream);
  }
}

hipError_t w4a16_reduce_launch(const W4A16Params& p, int BM, int BN, int group_m, hipStream_t stream) {
  const int cut = p.tiles_m * p.tiles_n - p.dp_tiles;
  if (cut > 0)
    hipLaunchKernelGGL(w4a16_reduce_kernel, dim3((BM * BN + 1023) / 1024, cut), dim3(256), 0, stream, p, BM, BN,
                       group_m);
  return hipGetLastError();
}

hipError_t w4a16_out_bound_launch(const void* w_q4, const float* w_scale, const void* bias, int bias_dtype, int64_t N,
                                  int64_t K, float* bound, hipStream_t stream) {
  const int np = (int)((N + 3) / 4);
  hipLaunchKernelGGL(w4a16_col_l1_kernel, dim3((unsigned)np), dim3(256), 0, stream, (const uint8_t*)w_q4, w_scale,
                     (int)N, (int)K, bound + 2);
  hipLaunchKernelGGL(w4a16_bound_reduce_kernel, dim3(1), dim3(256), 0, stream, (const float*)(bound + 2), np, bias,
                     bias_dtype, (int)N, bound);
  return hipGetLastError();
}

hipError_t scales_kn_launch(const float* w_scale, float* w_scale_kn, int64_t N, int64_t groups, hipStream_t stream) {
  hipLaunchKernelGGL(scales_kn_kernel, dim3((unsigned)((N + 31) / 32), (unsigned)((groups + 31) / 32)), dim3(256), 0,
                     stream, w_scale, w_scale_kn, (int)N, (int)groups);
  return hipGetLastError();
}

hipError_t col_scales_launch(const float* w_scale, float* col_scale, int64_t N, int64_t groups, hipStream_t stream) {
  hipLaunchKernelGGL(col_scales_kernel, dim3((unsigned)((N + 3) / 4)), dim3(256), 0, stream, w_scale, col_scale,
                     (int)N, (int)groups);
  return hipGetLastError();
}

}  // namespace qlinear
