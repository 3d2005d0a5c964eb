// W4A16 GEMM for large M on gfx950: y[M,N] = x[M,K] @ (q[N,K] * s[N,K/32])^T (+ bias), x fp16
// (or bf16), q packed int4 in the reference layout (nodes/ComfyUI-Gfx906Int4/ops.py:108-126),
// fp32 group scales, fp32 MFMA accumulation. Same arithmetic as w4a16_gemm.hip; a different
// shape of workgroup, for M in the thousands.
//
// One 512-thread workgroup (8 waves, two per SIMD) computes a 256 x 256 output tile:
//
// * Waves sit 2 (along M) x 4 (along N); each owns 128 rows x 64 columns as 4 x 2 blocks of
//   v_mfma_f32_32x32x16 (128 fp32 accumulators). Two waves per SIMD let one wave's dequant run
//   on the VALU while the other's MFMAs run on the matrix core.
// * Everything a stage needs arrives by DMA straight into LDS (buffer_load ... lds), 64 K per
//   stage: activations (256 rows x 128 B), raw int4 weights (256 columns x 32 B) and the group
//   scales (256 columns x 2 x 4 B), 42 KiB per stage, three stage buffers; the loads of stage
//   s+2 are issued during stage s.
// * The weights are the MFMA's first operand (rows of the 32x32 block = output columns n), the
//   activations its second (block columns = rows m of y). Lane (c = l % 32, h = l / 32) of a
//   weight fragment holds column c and quant group h of the stage: one 16-byte read from LDS
//   gives the lane the 32 nibbles of its group; K-step t of the stage dequantizes dword t (8
//   weights) in registers. The K-slot map of an MFMA is therefore: slot block h of K-step t =
//   K elements 32h + 8t .. +7 of the stage, and the activation fragment is read with the same
//   map (row m, 16-byte chunk 4h + t).
// * LDS swizzles (swz_a, swz_b) make every 16-byte operand read conflict free: activation rows
//   are 128 B, weight columns 32 B.
// * Rows past M, columns past N read zeros (buffer range checks); K must be a multiple of 64.
// * Optional column factors (fp16 dequant, as in w4a16_gemm.hip): column n's scales are read as
//   s / col_scale[n] and the epilogue multiplies by col_scale[n], both exact powers of two, so the
//   dequantized weights stay in fp16's normal range for any fp32 scale.
// * Epilogue: lane (m, h) of an accumulator block holds y[m][n .. n+3] for n = 8b + 4h, b = 0..3
//   (the transpose of the MFMA's row-major output): bias, optional exact row and column scales,
//   rounding to the output dtype, one 8- or 16-byte store per 4 outputs.
#include "common.hpp"
#include "launch.hpp"

namespace qlinear {

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kT256StageK = 64;
constexpr int kT256NBuf = 3;
constexpr int kT256GroupM = kTile256GroupM;

template <bool kBf16>
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (kBf16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                  0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                 0);
  }
}

// 4-byte DMA (buffer_load_dword ... lds): lane i writes lds_base + 4 * i.
__device__ __forceinline__ void buf_load4_lds(rsrc_t r, void* lds_base, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_base, 4, voff, soff, 0, 0);
}

// LDS swizzles. A 16-byte operand read (ds_read_b128) is served 16 lanes (256 B) or 32 lanes
// (512 B) at a time; both are conflict free when the lanes of a pass hit distinct 16-byte slots
// of the 256- or 512-byte window. Activation reads take rows r .. r+31 (lanes 0-31) at one logical
// chunk: with 128-byte rows, rows of equal r & 1 (256-byte pass) and of equal r & 3 (512-byte
// pass) must use distinct physical chunks, which needs bits 1-3 and bits 2-4 of r to each map
// one-to-one onto the chunk: chunk ^ (bits 1-3 of r) ^ (bit 4 of r). Weight reads take columns
// n .. n+31 at one half: columns n and n + 8 (256-byte pass) and n and n + 16 (512-byte pass)
// must use different halves: half ^ bit 3 ^ bit 4 of n.
__device__ __forceinline__ int swz_a(int r) { return ((r >> 1) & 7) ^ ((r >> 4) & 1); }
__device__ __forceinline__ int swz_b(int n) { return ((n >> 3) & 1) ^ ((n >> 4) & 1); }

// Waves sit kWavesM (along M) x kWavesN (along N); each owns (32 WM) rows x (32 WN) columns as
// WM x WN blocks of v_mfma_f32_32x32x16. The tile is BM = 32 WM kWavesM rows by
// BN = 32 WN kWavesN columns.
// A workgroup computes sub-tile (g % kSub) along M of the (kSub BM) x 256 tile p.tile_base + g / kSub
// (grouped tile order): kSub = 1 for whole tiles, 2 for the 128-row halves that the last,
// partly filled round of 256-row tiles is cut into. kCut: K piece g % ksplit of the BM x 256 tile
// p.tile_base + g / ksplit, its fp32 partial written to slot g of p.partial (summed, with the
// epilogue, by w4a16_reduce_kernel) -- for the few-tile shapes of small M, where whole tiles would
// leave most CUs idle.
template <bool kBf16, int kWavesM, int kWavesN, int WM, int WN, int kSub, bool kCut = false, int kNBuf = kT256NBuf>
__global__ __launch_bounds__(64 * kWavesM * kWavesN) void w4a16_tile256_kernel(W4A16Params p) {
  constexpr int kWaves = kWavesM * kWavesN;
  constexpr int BM = 32 * WM * kWavesM, BN = 32 * WN * kWavesN;
  // activation rows of a stage buffer: BM rounded up to whole DMA rounds (8 rows per wave); the
  // rows past BM (224-row tiles: 224 .. 255) lie outside the activation descriptor and read zeros
  constexpr int kARows = (BM + 8 * kWavesM * kWavesN - 1) / (8 * kWavesM * kWavesN) * (8 * kWavesM * kWavesN);
  constexpr int kABytes = kARows * kT256StageK * 2;  // activations: kARows rows x 128 B
  constexpr int kBBytes = BN * kT256StageK / 2;  // weights: BN columns x 32 B
  constexpr int kSBytes = BN * 2 * 4;            // scales: BN columns x 2 groups x 4 B
  constexpr int kStageBytes = kABytes + kBBytes + kSBytes;
  // DMA instructions per wave and stage: activations in 1 KiB blocks (8 rows), weights in 1 KiB
  // blocks (32 columns), scales in 256 B blocks (32 columns)
  constexpr int nA = kARows / 8 / kWaves, nB = BN / 32 / kWaves, nS = BN / 32 / kWaves;
  constexpr int nL = nA + nB + nS;
  static_assert(nA * 8 * kWaves == kARows && nB * 32 * kWaves == BN && nB >= 1, "DMA blocks must split evenly");
  static_assert(nL <= 4 * WM * WN, "the loads of a stage are spread over the MFMAs of a stage");
  static_assert(kNBuf >= 3 && kNBuf * kStageBytes <= 160 * 1024, "stage ring: 3 or more buffers in 160 KiB of LDS");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kNBuf * kStageBytes];

  const int lane = threadIdx.x & 63;
  // the wave index is uniform across the wave: in a scalar register, LDS destinations of the DMA
  // (M0) and other per-wave values are computed with scalar instructions
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = w / kWavesN, wn = w % kWavesN;
  const int c32 = lane & 31, h = lane >> 5;
  const int M = p.M, N = p.N, K = p.K;
  const int S = K / kT256StageK;

  static_assert((BM * kSub == 256 || kSub == 1) && BN == 256 && (!kCut || kSub == 1), "sub-tiles of a 256 x 256 tile");
  const int g = xcd_remap(blockIdx.x, gridDim.x);
  int tm, tn;
  tile_coords(p.tile_base + (kCut ? g / p.ksplit : g / kSub), p.tiles_m, p.tiles_n, kT256GroupM, tm, tn);
  const int m0 = tm * (BM * kSub) + (kCut ? 0 : (g % kSub) * BM), n0 = tn * BN;
  // this workgroup's stages [sb, sb + Sl): all of K, or K piece g % ksplit
  int sb = 0, Sl = S;
  if constexpr (kCut) {
    const int piece = g % p.ksplit;
    sb = (int)((long long)piece * S / p.ksplit);
    Sl = (int)((long long)(piece + 1) * S / p.ksplit) - sb;
  }
  // The second 128-row half of the last tile row lies wholly past M when M % 256 is in (0, 128]:
  // nothing to compute or store. The exit is uniform over the workgroup and precedes every barrier
  // and DMA. (Without it `rows` would be negative and the activation descriptor's range would wrap
  // to ~4 GB past the end of x.)
  if (m0 >= M) return;
  const int rows = max(0, min(M - m0, BM)), cols = max(0, min(N - n0, BN));

  const rsrc_t rs_a = make_rsrc((const uint16_t*)p.x + (size_t)m0 * K, (uint32_t)rows * K * 2);
  const rsrc_t rs_b = make_rsrc((const uint8_t*)p.wq + (size_t)n0 * (K / 2), (uint32_t)cols * (K / 2));
  // Group scales, column-major [N, K/32] (the reference's layout): a stage's two groups of a column
  // are 8 bytes of that column's own row, so every column costs a memory request per stage (256
  // requests of 8 bytes: measured to halve the weight stream's rate where it is memory-bound).
  // Group-major [K/32, N] (scales_kn): a stage's scales of the tile are two 1 KiB runs. The range
  // ends at the tile's last column of the last group row; a column past N in an earlier row reads
  // a scale of the next row, which only enters that column's own accumulators (each output column
  // has its own weights and scales), and those are never stored.
  const int kn = p.scales_kn;
  const rsrc_t rs_s = kn ? make_rsrc(p.ws + n0, (uint32_t)((K / 32 - 1) * N + cols) * 4)
                         : make_rsrc(p.ws + (size_t)n0 * (K / 32), (uint32_t)cols * (K / 32) * 4);
  const uint32_t s_stage = kn ? (uint32_t)N * 8 : 8u;  // bytes from one stage's scales to the next
  const rsrc_t rs_none = make_rsrc(p.ws, 0);

  // ---- DMA lane offsets (fixed for the K loop; the stage goes into the scalar offset) --------
  // activation block kb = w nA + q: rows 8kb .. 8kb+7; lane i: row 8kb + i/8, physical chunk i%8
  //   holding logical chunk (i%8) ^ swz_a(row)
  uint32_t vo_a[nA];
#pragma unroll
  for (int q = 0; q < nA; ++q) {
    const int r = 8 * (w * nA + q) + (lane >> 3);
    vo_a[q] = (uint32_t)(r * K + 8 * ((lane & 7) ^ swz_a(r))) * 2;
  }
  // weight block kb = w nB + q: columns 32kb .. 32kb+31; lane i: column 32kb + i/2, physical half
  //   i%2 holding group (i%2) ^ swz_b(column). Scale block likewise, lane i: group i%2.
  uint32_t vo_b[nB], vo_s[nS];
#pragma unroll
  for (int q = 0; q < nB; ++q) {
    const int n = 32 * (w * nB + q) + (lane >> 1);
    vo_b[q] = (uint32_t)n * (K / 2) + 16 * ((lane & 1) ^ swz_b(n));
    vo_s[q] = kn ? ((uint32_t)(lane & 1) * N + n) * 4 : ((uint32_t)n * (K / 32) + (lane & 1)) * 4;
  }

  // LDS layout: the three activation stage buffers, then the three weight buffers, then the three
  // scale buffers, so that every operand read of buffers 0 and 1 (and the weight and scale reads of
  // all three) fits the 16-bit immediate offset of ds_read from one base register.
  constexpr int kOffB = kNBuf * kABytes, kOffS = kOffB + kNBuf * kBBytes;
  // DMA instruction l (0 .. nL-1) of this wave's share of stage s into ring buffer `buf`. A stage
  // past the end loads through an empty resource (no traffic, no branch).
  // (s counts this workgroup's stages; the K position is sb + s)
  auto load_one = [&](int l, int s, int buf) {
    const bool live = s < Sl;
    const int sg = sb + s;
    if (l < nA) {
      buf_load16_lds(live ? rs_a : rs_none, lds + buf * kABytes + (w * nA + l) * 1024, vo_a[l], sg * 128);
    } else if (l < nA + nB) {
      const int q = l - nA;
      buf_load16_lds(live ? rs_b : rs_none, lds + kOffB + buf * kBBytes + (w * nB + q) * 1024, vo_b[q], sg * 32);
    } else {
      const int q = l - nA - nB;
      buf_load4_lds(live ? rs_s : rs_none, lds + kOffS + buf * kSBytes + (w * nS + q) * 256, vo_s[q], sg * s_stage);
    }
  };
  auto load_stage = [&](int s, int buf) {
#pragma unroll
    for (int l = 0; l < nL; ++l) load_one(l, s, buf);
  };

  // ---- LDS read addresses ------------------------------------------------------------------
  // activation fragment (m-block j, K-step t): row wm*32*WM + 32j + c32, logical chunk 4h + t.
  // The swizzle depends only on bits 1-4 of the row, those of c32, so one base per K-step serves
  // every m-block (+ j * 4 KiB).
  // Base addresses are kept opaque to the optimizer, which would otherwise fold each buffer's offset
  // into a separate register per (buffer, K-step) instead of using the immediate field.
  typedef __attribute__((address_space(3))) const u32x4* lds_frag_ptr;
  const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)lds;
  constexpr int kImm = 65536;  // ds_read immediate offsets are below 64 KiB
  // buffers [0, kFarBuf) are read from a_base, the rest from a_far; each group's immediates (buffer
  // offset + m-block offset, up to 4 KiB (WM - 1)) stay below 64 KiB
  constexpr int kFarBuf = [] {
    int f = kNBuf;
    while (f > 1 && (f - 1) * kABytes + 4096 * (WM - 1) >= kImm) --f;
    return f;
  }();
  static_assert(kFarBuf == kNBuf || (kNBuf - 1 - kFarBuf) * kABytes + 4096 * (WM - 1) < kImm,
                "activation buffers must split into two groups within the ds_read immediate range");
  uint32_t a_base[4], a_far[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int r = wm * 32 * WM + c32;
    a_base[t] = lds_base + (uint32_t)(r * 128 + (((4 * h + t) ^ swz_a(r)) * 16));
    a_far[t] = a_base[t] + kFarBuf * kABytes;
    asm volatile("" : "+v"(a_base[t]), "+v"(a_far[t]));
  }
  // weight fragment (n-block i): column wn*32*WN + 32i + c32, group h of the stage
  uint32_t b_base[WN], s_base[WN];
#pragma unroll
  for (int i = 0; i < WN; ++i) {
    const int n = wn * 32 * WN + 32 * i + c32;
    b_base[i] = lds_base + (uint32_t)(kOffB + n * 32 + 16 * (h ^ swz_b(n)));
    s_base[i] = lds_base + (uint32_t)(kOffS + n * 8 + 4 * h);
    asm volatile("" : "+v"(b_base[i]), "+v"(s_base[i]));
  }
  auto read_a = [&](int buf, int t, int j) {
    return buf >= kFarBuf ? *(lds_frag_ptr)(a_far[t] + (buf - kFarBuf) * kABytes + j * 4096)
                          : *(lds_frag_ptr)(a_base[t] + buf * kABytes + j * 4096);
  };
  auto read_b = [&](int buf, int i) { return *(lds_frag_ptr)(b_base[i] + buf * kBBytes); };
  auto read_s = [&](int buf, int i) {
    return *(__attribute__((address_space(3))) const float*)(s_base[i] + buf * kSBytes);
  };

  // Accumulators start as the result of an MFMA on zeros rather than as a zero constant, which
  // keeps the compiler from copying them between register files at every loop iteration.
  f32x16 acc[WN][WM];
  {
    f32x16 z;
#pragma unroll
    for (int e = 0; e < 16; ++e) z[e] = 0.0f;
#pragma unroll
    for (int i = 0; i < WN; ++i)
#pragma unroll
      for (int j = 0; j < WM; ++j) acc[i][j] = mfma32<kBf16>(u32x4{0u, 0u, 0u, 0u}, u32x4{0u, 0u, 0u, 0u}, z);
  }

  // ---- main loop ----------------------------------------------------------------------------
  // Stage s sits in ring buffer s % kNBuf. Entering stage s: its raw weights, scales and the
  // activation fragments of K-step 0 are in registers (reads issued), the loads of stages s+1 ..
  // s+kNBuf-2 are in flight, and buffer (s-1) % kNBuf is free (every wave passed the barrier at
  // the end of stage s-1). During stage s each wave issues its loads of stage s+kNBuf-1 into it,
  // spread evenly over the stage's MFMAs: issued in a burst, the DMA instructions of all waves
  // fill the texture unit's address FIFO and stall the MFMAs queued behind them. Before the
  // stage's last K-step every wave waits for its own loads of s+1 and passes the barrier (after
  // which stage s+1 is complete in LDS and nobody reads buffer s % kNBuf any more); the last
  // K-step's MFMAs then cover the reads of s+1's first fragments.
  // Each activation fragment register is refilled in place with the fragment of the next K-step
  // (of the next stage after the last K-step) right after its last MFMA of this K-step, so the
  // reads have the rest of the K-step's MFMAs to land and only one set of fragments is live.
  constexpr int kSlots = 4 * WM * WN;  // MFMAs per wave and stage
  // DMA instruction l of stage s+kNBuf-1 goes after MFMA slot l * kSlots / nL of stage s; the ones
  // before the last K-step (slot < 3 WM WN) are issued before that K-step's wait, which must let
  // exactly those and the loads of stages s+2 .. s+kNBuf-2 stay outstanding (vmcnt counts this
  // wave's loads in issue order)
  constexpr int kPreWait = [] {
    int c = 0;
    for (int l = 0; l < nL; ++l) c += (l * kSlots / nL < 3 * WM * WN) ? 1 : 0;
    return c;
  }();
  u32x4 raw[WN], a[WM], b[WN], bn[WN];
  float sc[WN];
  // Column factors (fp16 dequant): the lane's weight column n dequantizes with its group scales
  // times 1 / col_scale[n] (an exact power of two), undone in the epilogue.
  float csd[WN];
  auto first_weights = [&](auto bc) {
    constexpr int bf = decltype(bc)::value;
#pragma unroll
    for (int i = 0; i < WN; ++i) {
      raw[i] = read_b(bf, i);
      sc[i] = read_s(bf, i) * csd[i];
    }
  };
  auto stage = [&](auto bc, int s) {
    constexpr int bf = decltype(bc)::value;
    constexpr int bf1 = (bf + 1) % kNBuf, bfl = (bf + kNBuf - 1) % kNBuf;
    float n8s[WN];
#pragma unroll
    for (int i = 0; i < WN; ++i) {
      n8s[i] = -8.0f * sc[i];
      bn[i] = dequant8<kBf16>(raw[i][0], sc[i], n8s[i]);
    }
    static_for<0, 4>([&](auto tc) {
      constexpr int t = decltype(tc)::value;
#pragma unroll
      for (int i = 0; i < WN; ++i) b[i] = bn[i];
      if constexpr (t == 3) {
        // this wave's reads of buffer bf are complete (the last ones fill a[] for this K-step)
        // and its loads of stage s+1 have landed; after the barrier every wave's have
        wait_lgkm();
        wait_vmcnt<(kNBuf - 3) * nL + kPreWait>();
        barrier_no_fence();
        first_weights(ic<bf1>{});
      }
      static_for<0, WM>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        static_for<0, WN>([&](auto ic_) {
          constexpr int i = decltype(ic_)::value;
          constexpr int slot = (t * WM + j) * WN + i;
          acc[i][j] = mfma32<kBf16>(b[i], a[j], acc[i][j]);
          static_for<0, nL>([&](auto lc) {
            constexpr int l = decltype(lc)::value;
            if constexpr (l * kSlots / nL == slot) {
              load_one(l, s + kNBuf - 1, bfl);
              __builtin_amdgcn_sched_barrier(0);
            }
          });
        });
        a[j] = t < 3 ? read_a(bf, t + 1, j) : read_a(bf1, 0, j);
        if constexpr (t < 3 && j < WN) bn[j] = dequant8<kBf16>(raw[j][t + 1], sc[j], n8s[j]);
      });
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  // ---- prologue: stages 0 .. kNBuf-2 in flight, stage 0 published ---------------------------
  // The column factors load first; csd is formed after the wait for stage 0, so their latency
  // hides behind the stage loads.
  {
    const float* cs_p = p.col_scale;
    asm volatile("" : "+s"(cs_p));
#pragma unroll
    for (int i = 0; i < WN; ++i) {
      const int n = n0 + wn * 32 * WN + 32 * i + c32;
      csd[i] = (cs_p && n < N) ? cs_p[n] : 1.0f;
    }
  }
#pragma unroll
  for (int i = 0; i < kNBuf - 1; ++i) load_stage(i, i);
  wait_vmcnt<(kNBuf - 2) * nL>();
#pragma unroll
  for (int i = 0; i < WN; ++i) csd[i] = pow2_recip(csd[i]);
  barrier_no_fence();
  first_weights(ic<0>{});
#pragma unroll
  for (int j = 0; j < WM; ++j) a[j] = read_a(0, 0, j);

  int s = 0;
  if constexpr (kNBuf == 3) {
    // (written out: the generic form below costs the register-tight 256 x 64-per-wave variant
    // a spill of its accumulators)
    for (; s + 3 <= Sl; s += 3) {
      stage(ic<0>{}, s);
      stage(ic<1>{}, s + 1);
      stage(ic<2>{}, s + 2);
    }
    if (s < Sl) stage(ic<0>{}, s++);
    if (s < Sl) stage(ic<1>{}, s++);
  } else {
    for (; s + kNBuf <= Sl; s += kNBuf) static_for<0, kNBuf>([&](auto bc) { stage(bc, s + decltype(bc)::value); });
    // the last Sl % kNBuf stages (s is a multiple of kNBuf here: stage s + b sits in buffer b)
    static_for<0, kNBuf - 1>([&](auto bc) {
      if (s + decltype(bc)::value < Sl) stage(bc, s + decltype(bc)::value);
    });
  }

  if constexpr (kCut) {
    wait_vmcnt<0>();  // the DMA issued for stages past the piece (zeros into LDS) has landed
    // K piece: the raw fp32 accumulators to partial slot g, a [BM][BN] row-major tile; lane (c32, h)
    // of block (i, j) holds row 32j + c32 (of this wave's rows), columns 8 bq + 4h .. +3 of n-block i
    float* dst = p.partial + (size_t)g * (BM * BN);
#pragma unroll
    for (int j = 0; j < WM; ++j)
#pragma unroll
      for (int i = 0; i < WN; ++i)
#pragma unroll
        for (int bq = 0; bq < 4; ++bq) {
          const int r = wm * 32 * WM + 32 * j + c32, c = wn * 32 * WN + 32 * i + 8 * bq + 4 * h;
          *(f32x4*)(dst + (size_t)r * BN + c) =
              f32x4{acc[i][j][4 * bq], acc[i][j][4 * bq + 1], acc[i][j][4 * bq + 2], acc[i][j][4 * bq + 3]};
        }
    return;
  }

  // ---- epilogue ----------------------------------------------------------------------------
  // The gated residual epilogue is not built into variant 2 (4 waves of 256 x 64), whose
  // accumulators leave no registers for it; the C ABI rejects it there.
  constexpr bool kResidual = !(kWavesM == 1 && kWavesN == 4);
  // v = acc * row_scale * col_scale + bias (both scales exact powers of two); with the GELU
  // epilogue v is first rounded to the output dtype
  // (the unfused sequence's linear output) and then passed through gelu_tanh. Bias and row
  // scales go to registers before any store (y may alias them as far as the compiler knows).
  // (The pointers pass through an empty asm statement so the loads are not hoisted above the K
  // loop, where their registers would be live across it.)
  const void* bias_p = p.bias;
  const float* rs_p = p.row_scale;
  const float* cu_p = p.col_scale;
  asm volatile("" : "+s"(bias_p), "+s"(rs_p), "+s"(cu_p));
  float bv[WN][4][4], rsj[WM];
#pragma unroll
  for (int i = 0; i < WN; ++i)
#pragma unroll
    for (int bq = 0; bq < 4; ++bq)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int n = n0 + wn * 32 * WN + 32 * i + 8 * bq + 4 * h + e;
        bv[i][bq][e] = (bias_p && n < N) ? read_elem(bias_p, p.out_dtype == kBF16AsF16 ? kBF16 : p.out_dtype, n)
                                         : 0.0f;
      }
  // When every column of the tile has factor 1 (ordinary checkpoints) the plain epilogue runs.
  // Each wave checks all BN columns (BN / 64 per lane), so the choice is uniform over the
  // workgroup: the 16-bit epilogue below passes workgroup barriers.
  bool col_one = true;
  if (cu_p) {
#pragma unroll
    for (int e = 0; e < BN / 64; ++e) {
      const int n = n0 + (BN / 64) * lane + e;
      col_one = col_one && (n >= N || cu_p[n] == 1.0f);
    }
  }
  const bool scaled_cols = __builtin_amdgcn_ballot_w64(!col_one) != 0;
#pragma unroll
  for (int j = 0; j < WM; ++j) {
    const int m = m0 + wm * 32 * WM + 32 * j + c32;
    rsj[j] = (rs_p && m < M) ? rs_p[m] : 1.0f;
  }
  // kBF16AsF16 output: row m is stored as fp16 times 2^-e_m, 2^e_m from the row's bound (its input
  // row factor and the weight's bound); the tile column 0 workgroups publish 2^e_m, one lane a row.
  float rdown[WM];
#pragma unroll
  for (int j = 0; j < WM; ++j) rdown[j] = 1.0f;
  if (p.out_dtype == kBF16AsF16) {
    const float wl1 = p.out_bound[0], bmax = p.out_bound[1];
#pragma unroll
    for (int j = 0; j < WM; ++j) {
      float up;
      f16_row_factor(w4a16_row_bound(rsj[j], wl1, bmax), rdown[j], up);
      const int m = m0 + wm * 32 * WM + 32 * j + c32;
      if (tn == 0 && wn == 0 && h == 0 && m < M) p.out_row_scale[m] = up;
    }
  }
  // The epilogue is instantiated per (activation, output dtype), so that its per-value code has no
  // branches; one uniform dispatch selects the instance.
  auto epilogue = [&](auto actc, auto odtc, auto colc) {
    constexpr int kAct = decltype(actc)::value, kOdt = decltype(odtc)::value;
    constexpr bool kColScaled = decltype(colc)::value;
    constexpr int kRnd = kOdt == kBF16AsF16 ? (int)kBF16 : kOdt;  // the logical output dtype
    float cu[WN][4][4];
#pragma unroll
    for (int i = 0; i < WN; ++i)
#pragma unroll
      for (int bq = 0; bq < 4; ++bq)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int n = n0 + wn * 32 * WN + 32 * i + 8 * bq + 4 * h + e;
          cu[i][bq][e] = (kColScaled && n < N) ? cu_p[n] : 1.0f;
        }
    auto value = [&](int i, int j, int bq, int e) {
      float v = kColScaled ? acc[i][j][4 * bq + e] * rsj[j] * cu[i][bq][e] + bv[i][bq][e]
                           : acc[i][j][4 * bq + e] * rsj[j] + bv[i][bq][e];
      if constexpr (kAct == kActGeluTanh) v = gelu_tanh(round_to(kRnd, v));
      if constexpr (kOdt == kBF16AsF16) v = round_to(kBF16, v) * rdown[j];  // exact in fp16
      return v;
    };
    if constexpr (kOdt == kF32) {
      // fp32: lane (m, h) stores 4 adjacent outputs (16 B) per accumulator quarter
      const bool vec = (N % 4) == 0 && (((uintptr_t)p.y) & 15) == 0;
#pragma unroll
      for (int j = 0; j < WM; ++j) {
        const int m = m0 + wm * 32 * WM + 32 * j + c32;
        if (m >= M) continue;
#pragma unroll
        for (int i = 0; i < WN; ++i)
#pragma unroll
          for (int bq = 0; bq < 4; ++bq) {
            const int n = n0 + wn * 32 * WN + 32 * i + 8 * bq + 4 * h;
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = value(i, j, bq, e);
            const size_t off = (size_t)m * N + n;
            if (kResidual && p.residual) {  // gated residual (uniform over the workgroup)
              const float* rp = (const float*)p.residual + off;
              const float* gp = (const float*)p.gate + (size_t)(m / p.gate_rows) * N + n;
#pragma unroll
              for (int e = 0; e < 4; ++e)
                if (n + e < N) v[e] = rp[e] + gp[e] * v[e];
            }
            if (vec && n + 3 < N) {
              *(f32x4*)((float*)p.y + off) = f32x4{v[0], v[1], v[2], v[3]};
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                if (n + e < N) ((float*)p.y)[off + e] = v[e];
            }
          }
      }
    } else {
      // 16-bit outputs go through LDS, half a tile (kHalfRows rows x BN columns) at a time, so that
      // each wave stores whole 512-byte row segments with 16-byte lanes instead of 8-byte pieces
      // of 32 different rows. LDS row r holds 16-byte chunk c at slot c ^ (r & 31): the 8-byte
      // writes of a wave (32 rows x 2 halves of one chunk) and the 16-byte reads (2 rows x 32
      // chunks) are both conflict free. The stage buffers are free once every wave is past its
      // last MFMA and the DMA loads issued for stages past the end (which write zeros) have landed.
      // halves of whole 32-row blocks: BM / 2, or 128 + 96 rows for 224-row tiles
      constexpr int kHalfRows = (BM / 2 + 31) / 32 * 32;
      constexpr int kChunks = BN / 8;  // 16-byte chunks per row
      static_assert(kHalfRows * BN * 2 <= kNBuf * kStageBytes, "half a tile must fit the stage buffers");
      wait_vmcnt<0>();
      wait_lgkm();
      barrier_no_fence();
      const bool vec = (N % 8) == 0 && (((uintptr_t)p.y) & 15) == 0;
      const bool rvec = vec && ((((uintptr_t)p.residual) | ((uintptr_t)p.gate)) & 15) == 0;
      static_for<0, 2>([&](auto hc) {
        constexpr int half = decltype(hc)::value;
        static_for<0, WM>([&](auto jc) {
          constexpr int j = decltype(jc)::value;
          if ((wm * 32 * WM + 32 * j) / kHalfRows != half) return;
          const int r = wm * 32 * WM + 32 * j - half * kHalfRows + c32;
#pragma unroll
          for (int i = 0; i < WN; ++i)
#pragma unroll
            for (int bq = 0; bq < 4; ++bq) {
              const int c = wn * 32 * WN + 32 * i + 8 * bq + 4 * h;  // tile column of the lane's 4 outputs
              uint32_t lo, hi;
              if constexpr (kOdt == kBF16) {
                lo = pack2_bf16(value(i, j, bq, 0), value(i, j, bq, 1));
                hi = pack2_bf16(value(i, j, bq, 2), value(i, j, bq, 3));
              } else {  // fp16, and kBF16AsF16 (values already exact fp16 numbers)
                lo = pack2_f16(value(i, j, bq, 0), value(i, j, bq, 1));
                hi = pack2_f16(value(i, j, bq, 2), value(i, j, bq, 3));
              }
              typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
              *(u32x2*)(lds + r * (BN * 2) + (((c >> 3) ^ (r & 31)) << 4) + (c & 7) * 2) = u32x2{lo, hi};
            }
        });
        barrier_no_fence();
#pragma unroll
        for (int k = 0; k < kHalfRows * kChunks / (64 * kWaves); ++k) {
          const int q = threadIdx.x + k * 64 * kWaves;
          const int r = q / kChunks, c = q % kChunks;
          u32x4 v = *(const u32x4*)(lds + r * (BN * 2) + ((c ^ (r & 31)) << 4));
          const int m = m0 + half * kHalfRows + r, n = n0 + 8 * c;
          // (a short second half, 224-row tiles: staged rows past the tile are not this tile's)
          if (half * kHalfRows + r < BM && m < M && n < N) {
            uint16_t* dst = (uint16_t*)p.y + (size_t)m * N + n;
            if constexpr ((kOdt == kBF16 || kOdt == kF16) && kResidual) {
              if (p.residual)  // gated residual on the rounded outputs (uniform over the workgroup)
                v = gated_residual8<kOdt>(v, (const uint16_t*)p.residual + (size_t)m * N + n,
                                          (const uint16_t*)p.gate + (size_t)(m / p.gate_rows) * N + n, min(8, N - n), rvec);
            }
            if (vec && n + 8 <= N) {
              *(u32x4*)dst = v;
            } else {
              for (int e = 0; e < 8 && n + e < N; ++e) dst[e] = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
            }
          }
        }
        if constexpr (half == 0) barrier_no_fence();
      });
    }
  };
  const bool gelu = p.act == kActGeluTanh;
  auto run = [&](auto colc) {
    switch (p.out_dtype) {
      case kF32:
        gelu ? epilogue(ic<kActGeluTanh>{}, ic<kF32>{}, colc) : epilogue(ic<kActNone>{}, ic<kF32>{}, colc);
        break;
      case kF16:
        gelu ? epilogue(ic<kActGeluTanh>{}, ic<kF16>{}, colc) : epilogue(ic<kActNone>{}, ic<kF16>{}, colc);
        break;
      case kBF16AsF16:  // variant 1 and its halves only (the C ABI rejects it for the others)
        if constexpr (kWavesM == 1 && kWavesN == 8)
          gelu ? epilogue(ic<kActGeluTanh>{}, ic<kBF16AsF16>{}, colc) : epilogue(ic<kActNone>{}, ic<kBF16AsF16>{}, colc);
        break;
      default:
        gelu ? epilogue(ic<kActGeluTanh>{}, ic<kBF16>{}, colc) : epilogue(ic<kActNone>{}, ic<kBF16>{}, colc);
        break;
    }
  };
  if (scaled_cols) {
    run(ic<1>{});
  } else {
    run(ic<0>{});
  }
}

template <bool kBf16, int kWavesM, int kWavesN, int WM, int WN>
hipError_t launch_variant(const W4A16Params& p, hipStream_t stream) {
  W4A16Params q = p;
  const int tiles = p.tiles_m * p.tiles_n;
  const int whole = p.dp_tiles;  // tiles run whole; the rest as 128-row halves
  if (whole > 0) {
    q.tile_base = 0;
    hipLaunchKernelGGL((w4a16_tile256_kernel<kBf16, kWavesM, kWavesN, WM, WN, 1>), dim3(whole),
                       dim3(64 * kWavesM * kWavesN), 0, stream, q);
  }
  if (whole < tiles) {
    q.tile_base = whole;
    hipLaunchKernelGGL((w4a16_tile256_kernel<kBf16, 1, 8, 4, 1, 2>), dim3(2 * (tiles - whole)), dim3(512), 0, stream,
                       q);
  }
  return hipGetLastError();
}

// Stage buffers of the short tiles: as many as fit 160 KiB of LDS (64 rows: 8 x 18 KiB, 128 rows:
// 6 x 26 KiB). With few rows a stage is a few hundred cycles of MFMA, far less than a trip to
// HBM, so only a deep ring of loads in flight keeps the weight stream going.
constexpr int rows_nbuf(int wm) { return wm == 2 ? 8 : wm == 4 ? 6 : kT256NBuf; }

// Variant 1 with tiles of p.tile_rows (64, 128 or 256) rows: the first dp_tiles whole, the rest cut
// into ksplit K pieces whose partials w4a16_reduce_kernel sums (tile order of this kernel).
template <bool kBf16, int WM>
hipError_t launch_rows(const W4A16Params& p, hipStream_t stream) {
  constexpr int kNB = rows_nbuf(WM);
  W4A16Params q = p;
  const int tiles = p.tiles_m * p.tiles_n;
  if (p.dp_tiles > 0) {
    q.tile_base = 0;
    hipLaunchKernelGGL((w4a16_tile256_kernel<kBf16, 1, 8, WM, 1, 1, false, kNB>), dim3(p.dp_tiles), dim3(512), 0,
                       stream, q);
  }
  const int cut = tiles - p.dp_tiles;
  if (cut > 0) {
    q.tile_base = p.dp_tiles;
    hipLaunchKernelGGL((w4a16_tile256_kernel<kBf16, 1, 8, WM, 1, 1, true, kNB>), dim3(cut * p.ksplit), dim3(512), 0,
                       stream, q);
    const hipError_t e = w4a16_reduce_launch(q, 32 * WM, 256, kTile256GroupM, stream);
    if (e != hipSuccess) return e;
  }
  return hipGetLastError();
}

// Variant 1 with 224-row tiles, all whole: a single round of tiles where 256-row tiles would leave
// CUs idle (the plan takes it only then; the activation stages keep the 256-row layout).
template <bool kBf16>
hipError_t launch_rows224(const W4A16Params& p, hipStream_t stream) {
  if (p.ksplit != 1 || p.dp_tiles != p.tiles_m * p.tiles_n) return hipErrorInvalidValue;
  W4A16Params q = p;
  q.tile_base = 0;
  hipLaunchKernelGGL((w4a16_tile256_kernel<kBf16, 1, 8, 7, 1, 1>), dim3(p.dp_tiles), dim3(512), 0, stream, q);
  return hipGetLastError();
}

}  // namespace

hipError_t w4a16_tile256_launch(int variant, bool bf16, const W4A16Params& p, hipStream_t stream) {
  switch (variant) {
    case 0:  // 8 waves, 2 x 4, each 128 x 64
      return bf16 ? launch_variant<true, 2, 4, 4, 2>(p, stream) : launch_variant<false, 2, 4, 4, 2>(p, stream);
    case 1:  // 8 waves, 1 x 8, each 256 x 32; with K pieces, or 64 / 128 / 224-row tiles, per the plan
      if (p.ksplit > 1 || p.tile_rows != 256) {
        switch (p.tile_rows) {
          case 64: return bf16 ? launch_rows<true, 2>(p, stream) : launch_rows<false, 2>(p, stream);
          case 128: return bf16 ? launch_rows<true, 4>(p, stream) : launch_rows<false, 4>(p, stream);
          case 224: return bf16 ? launch_rows224<true>(p, stream) : launch_rows224<false>(p, stream);
          case 256: return bf16 ? launch_rows<true, 8>(p, stream) : launch_rows<false, 8>(p, stream);
          default: return hipErrorInvalidValue;
        }
      }
      return bf16 ? launch_variant<true, 1, 8, 8, 1>(p, stream) : launch_variant<false, 1, 8, 8, 1>(p, stream);
    case 2:  // 4 waves, 1 x 4, each 256 x 64
      return bf16 ? launch_variant<true, 1, 4, 8, 2>(p, stream) : launch_variant<false, 1, 4, 8, 2>(p, stream);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace qlinear
