// W8A8 GEMM for large M on gfx950: acc[m,n] = sum_k xq[m,k] * wq[n,k] in int32 on
// v_mfma_i32_32x32x32_i8 (exact integer arithmetic), epilogue y = float(acc) * (sx[m] * sw[n])
// (+ bias[n]) with every step rounded in fp32 -- the scale-product order of the reference's int8
// kernel (csrc/int8_gemm.hip:191-193, 209), whose block-32 scales become one per token and one
// per output channel here. out_dtype kI32 stores the raw accumulators.
//
// One 512-thread workgroup (8 waves, two per SIMD) computes a 256 x 256 output tile:
//
// * Waves sit 2 (along M) x 4 (along N); each owns 128 rows x 64 columns as 4 x 2 blocks of
//   32 x 32 int32 accumulators (128 registers). With no dequant in this kernel the cost to keep
//   low is LDS operand reads: 12 KiB per wave and 64 K, which the 2 x 4 layout halves against
//   a 1 x 8 one.
// * Activations and weights arrive by DMA straight into LDS (buffer_load ... lds), 64 K (bytes)
//   per stage: 256 rows x 64 B of each, 32 KiB per stage, four stage buffers, the loads of stage
//   s+3 spread over the MFMAs of stage s (issued in a burst they fill the texture unit's address
//   FIFO). Each wave issues 4 DMA instructions per stage.
// * The weights are the MFMA's first operand (rows of a 32 x 32 block = output columns n), the
//   activations its second (block columns = rows m of y). K-step t (32 K) of a stage: lane
//   (c = l % 32, h = l / 32) supplies row c, K bytes 32t + 16h .. +15, i.e. 16-byte chunk 2t + h
//   of the 64-byte row, for both operands.
// * LDS rows are 64 B; chunk q of row r sits at slot q ^ swz8(r): the 32 lanes of a 16-byte
//   operand read (rows r .. r+31, one chunk) hit distinct 16-byte bank groups whether the LDS
//   serves 16 lanes (256 B) or 32 lanes (512 B) at a time.
// * Rows past M, columns past N read zeros (buffer range checks); K must be a multiple of 64.
// * Epilogue: lane (m, h) of an accumulator block holds acc[m][n .. n+3] for n = 8b + 4h,
//   b = 0..3. 16-bit outputs are staged through LDS for whole-row stores.
#include "common.hpp"
#include "launch.hpp"

namespace qlinear {

namespace {

typedef int i32x16 __attribute__((ext_vector_type(16)));

constexpr int kQ8StageK = 64;  // int8 K (= bytes) per stage
constexpr int kQ8NBuf = 4;
constexpr int kQ8GroupM = kW8A8T256GroupM;
constexpr int kQ8WavesM = 2, kQ8WavesN = 4, kQ8WM = 4, kQ8WN = 2;
constexpr int kQ8Waves = kQ8WavesM * kQ8WavesN;
constexpr int kQ8BM = 32 * kQ8WM * kQ8WavesM, kQ8BN = 32 * kQ8WN * kQ8WavesN;  // 256 x 256
constexpr int kQ8ABytes = kQ8BM * kQ8StageK;                                    // 16 KiB
constexpr int kQ8BBytes = kQ8BN * kQ8StageK;                                    // 16 KiB

__device__ __forceinline__ i32x16 mfma32_i8(u32x4 a, u32x4 b, i32x16 c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, a), __builtin_bit_cast(i32x4, b), c, 0, 0,
                                              0);
}

// chunk q of a 64-byte row r at slot q ^ swz8(r): rows of equal r % 4 (256-byte pass) and of equal
// r % 8 (512-byte pass) must use distinct slots, which needs bits 2-3 and bits 3-4 of r to map
// one-to-one onto the 2-bit slot: (bit 2 ^ bit 4, bit 3).
__device__ __forceinline__ int swz8(int r) { return (((r >> 2) & 1) ^ ((r >> 4) & 1)) | (((r >> 3) & 1) << 1); }

__global__ __launch_bounds__(64 * kQ8Waves) void w8a8_tile256_kernel(W8A8Params p) {
  constexpr int nA = kQ8BM / 16 / kQ8Waves, nB = kQ8BN / 16 / kQ8Waves;  // 1 KiB DMA blocks (16 rows)
  constexpr int nL = nA + nB;
  constexpr int kSlots = 2 * kQ8WM * kQ8WN;  // MFMAs per wave and stage
  static_assert(nA * 16 * kQ8Waves == kQ8BM && nB * 16 * kQ8Waves == kQ8BN, "DMA blocks must split evenly");
  static_assert(kQ8BM == kQ8BN && 64 * kQ8Waves == 2 * kQ8BN, "one epilogue factor load per thread and table");
  constexpr int kOffB = kQ8NBuf * kQ8ABytes;
  constexpr int kOffF = kQ8NBuf * (kQ8ABytes + kQ8BBytes);
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kOffF + 3 * kQ8BN * 4];

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = w / kQ8WavesN, wn = w % kQ8WavesN;
  const int c32 = lane & 31, h = lane >> 5;
  const int M = p.M, N = p.N, K = p.K;
  const int S = K / kQ8StageK;

  const int g = xcd_remap(blockIdx.x, gridDim.x);
  int tm, tn;
  tile_coords(g, p.tiles_m, p.tiles_n, kQ8GroupM, tm, tn);
  const int m0 = tm * kQ8BM, n0 = tn * kQ8BN;
  // clamped at 0 so a descriptor range can never wrap (tiles start inside M and N here)
  const int rows = max(0, min(M - m0, kQ8BM)), cols = max(0, min(N - n0, kQ8BN));
  const rsrc_t rs_a = make_rsrc(p.xq + (size_t)m0 * K, (uint32_t)rows * K);
  const rsrc_t rs_b = make_rsrc(p.wq + (size_t)n0 * K, (uint32_t)cols * K);
  const rsrc_t rs_none = make_rsrc(p.xq, 0);

  // ---- DMA lane offsets: block kb (16 rows) of the stage; lane i: row 16kb + i/4, physical chunk
  // i%4 holding logical chunk (i%4) ^ swz8(row) ------------------------------------------------
  uint32_t vo_a[nA], vo_b[nB];
#pragma unroll
  for (int q = 0; q < nA; ++q) {
    const int r = 16 * (w * nA + q) + (lane >> 2);
    vo_a[q] = (uint32_t)(r * K + 16 * ((lane & 3) ^ swz8(r)));
  }
#pragma unroll
  for (int q = 0; q < nB; ++q) {
    const int r = 16 * (w * nB + q) + (lane >> 2);
    vo_b[q] = (uint32_t)(r * K + 16 * ((lane & 3) ^ swz8(r)));
  }
  auto load_one = [&](int l, int s, int buf) {
    const bool live = s < S;
    if (l < nA) {
      buf_load16_lds(live ? rs_a : rs_none, lds + buf * kQ8ABytes + (w * nA + l) * 1024, vo_a[l], s * kQ8StageK);
    } else {
      const int q = l - nA;
      buf_load16_lds(live ? rs_b : rs_none, lds + kOffB + buf * kQ8BBytes + (w * nB + q) * 1024, vo_b[q],
                     s * kQ8StageK);
    }
  };

  // ---- LDS read addresses: operand fragment of block row c32 (+ 32 per block), K-step t, half h --
  // The swizzle of rows wm*128 + 32j + c32 (A) and wn*64 + 32i + c32 (B) depends on c32 only.
  typedef __attribute__((address_space(3))) const u32x4* lds_frag_ptr;
  const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)lds;
  uint32_t a_base[2], b_base[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const uint32_t slot = (uint32_t)(((2 * t + h) ^ swz8(c32)) * 16);
    a_base[t] = lds_base + (uint32_t)((wm * 32 * kQ8WM + c32) * kQ8StageK) + slot;
    b_base[t] = lds_base + (uint32_t)(kOffB + (wn * 32 * kQ8WN + c32) * kQ8StageK) + slot;
    asm volatile("" : "+v"(a_base[t]), "+v"(b_base[t]));
  }
  auto read_a = [&](int buf, int t, int j) { return *(lds_frag_ptr)(a_base[t] + buf * kQ8ABytes + j * 2048); };
  auto read_b = [&](int buf, int t, int i) { return *(lds_frag_ptr)(b_base[t] + buf * kQ8BBytes + i * 2048); };

  // ---- main loop ----------------------------------------------------------------------------
  // Stage s sits in ring buffer s % 4. Entering stage s: the fragments of its K-step 0 are being
  // read, the loads of s+1 and s+2 are in flight, buffer (s+3) % 4 is free. During stage s each
  // wave issues its loads of s+3, one after every kSlots / nL MFMAs; before the last K-step it
  // waits for its loads of s+1 (leaving s+2 and the part of s+3 already issued in flight), passes
  // the barrier, and the last K-step's MFMAs cover the first reads of s+1.
  constexpr int kPreWait = [] {
    int c = 0;
    for (int l = 0; l < nL; ++l) c += (l * kSlots / nL < kQ8WM * kQ8WN) ? 1 : 0;
    return c;
  }();
  i32x16 acc[kQ8WN][kQ8WM];
#pragma unroll
  for (int i = 0; i < kQ8WN; ++i)
#pragma unroll
    for (int j = 0; j < kQ8WM; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0;
  u32x4 a[kQ8WM], b[kQ8WN];
  auto stage = [&](auto bc, int s) {
    constexpr int bf = decltype(bc)::value;
    constexpr int bf1 = (bf + 1) % kQ8NBuf, bf3 = (bf + 3) % kQ8NBuf;
    static_for<0, 2>([&](auto tc) {
      constexpr int t = decltype(tc)::value;
      if constexpr (t == 1) {
        wait_lgkm();
        wait_vmcnt<nL + kPreWait>();
        barrier_no_fence();
      }
      // weights of this K-step in registers (read ahead at the previous step's end)
      static_for<0, kQ8WM>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        static_for<0, kQ8WN>([&](auto ic_) {
          constexpr int i = decltype(ic_)::value;
          constexpr int slot = (t * kQ8WM + j) * kQ8WN + i;
          acc[i][j] = mfma32_i8(b[i], a[j], acc[i][j]);
          static_for<0, nL>([&](auto lc) {
            constexpr int l = decltype(lc)::value;
            if constexpr (l * kSlots / nL == slot) {
              load_one(l, s + 3, bf3);
              __builtin_amdgcn_sched_barrier(0);
            }
          });
          // the last use of b[i] in this K-step: refill it with the next K-step's fragment
          if constexpr (j == kQ8WM - 1) b[i] = t == 0 ? read_b(bf, 1, i) : read_b(bf1, 0, i);
        });
        a[j] = t == 0 ? read_a(bf, 1, j) : read_a(bf1, 0, j);
      });
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  // ---- epilogue factors: sw[256], bias[256], sx[256] as fp32 in LDS past the stage ring -------
  // Loaded before the stage loads, so the prologue's wait for stage 0 covers them; the barrier of
  // the first stage publishes the LDS writes.
  float* const lds_f = (float*)(lds + kOffF);
  const int odt = p.out_dtype;
  float f0 = 0.0f, f1 = 0.0f;
  if (odt != kI32) {
    const int t = threadIdx.x;
    if (t < kQ8BN) {
      const int n = n0 + t;
      f0 = n < N ? p.sw[n] : 0.0f;
      f1 = (p.bias && n < N) ? read_elem(p.bias, odt, n) : 0.0f;
    } else {
      const int m = m0 + t - kQ8BN;
      f0 = m < M ? p.sx[m] : 0.0f;
    }
  }

  // ---- prologue: stages 0, 1, 2 in flight, stage 0 published ----------------------------------
#pragma unroll
  for (int s0 = 0; s0 < 3; ++s0)
#pragma unroll
    for (int l = 0; l < nL; ++l) load_one(l, s0, s0);
  wait_vmcnt<2 * nL>();
  if (odt != kI32) {
    const int t = threadIdx.x;
    if (t < kQ8BN) {
      lds_f[t] = f0;
      lds_f[kQ8BN + t] = f1;
    } else {
      lds_f[2 * kQ8BN + t - kQ8BN] = f0;
    }
  }
  barrier_no_fence();
#pragma unroll
  for (int j = 0; j < kQ8WM; ++j) a[j] = read_a(0, 0, j);
#pragma unroll
  for (int i = 0; i < kQ8WN; ++i) b[i] = read_b(0, 0, i);

  int s = 0;
  for (; s + 4 <= S; s += 4) {
    stage(ic<0>{}, s);
    stage(ic<1>{}, s + 1);
    stage(ic<2>{}, s + 2);
    stage(ic<3>{}, s + 3);
  }
  if (s < S) stage(ic<0>{}, s++);
  if (s < S) stage(ic<1>{}, s++);
  if (s < S) stage(ic<2>{}, s++);

  // ---- epilogue ----------------------------------------------------------------------------
  auto epilogue = [&](auto odtc) {
    constexpr int kOdt = decltype(odtc)::value;
    const bool has_bias = p.bias != nullptr;
    // lane (c32, h) of column block i uses columns 32i + 8bq + 4h + e of the wave's 64
    const float* f_sw = lds_f + wn * 32 * kQ8WN + 4 * h;
    const float* f_bias = f_sw + kQ8BN;
    float sxv[kQ8WM];
#pragma unroll
    for (int j = 0; j < kQ8WM; ++j) sxv[j] = kOdt == kI32 ? 0.0f : lds_f[2 * kQ8BN + wm * 32 * kQ8WM + 32 * j + c32];
    float swv[4][4], bv[4][4];
    auto factors = [&](int i) {
      if constexpr (kOdt != kI32) {
#pragma unroll
        for (int bq = 0; bq < 4; ++bq) {
          const f32x4 sv = *(const f32x4*)(f_sw + 32 * i + 8 * bq);
          const f32x4 bb = *(const f32x4*)(f_bias + 32 * i + 8 * bq);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            swv[bq][e] = sv[e];
            bv[bq][e] = bb[e];
          }
        }
      }
    };
    // float(acc) * (sx * sw) (+ bias), each operation rounded in fp32
    auto value = [&](int i, int j, int bq, int e) {
      float v = __fmul_rn((float)acc[i][j][4 * bq + e], __fmul_rn(sxv[j], swv[bq][e]));
      if (has_bias) v = __fadd_rn(v, bv[bq][e]);
      return v;
    };
    if constexpr (kOdt == kF32 || kOdt == kI32) {
      const bool vec = (N % 4) == 0 && (((uintptr_t)p.y) & 15) == 0;
#pragma unroll
      for (int i = 0; i < kQ8WN; ++i) {
        factors(i);
#pragma unroll
        for (int j = 0; j < kQ8WM; ++j) {
          const int m = m0 + wm * 32 * kQ8WM + 32 * j + c32;
          if (m >= M) continue;
#pragma unroll
          for (int bq = 0; bq < 4; ++bq) {
            const int n = n0 + wn * 32 * kQ8WN + 32 * i + 8 * bq + 4 * h;
            const size_t off = (size_t)m * N + n;
            u32x4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e)
              v[e] = kOdt == kI32 ? (uint32_t)acc[i][j][4 * bq + e] : __builtin_bit_cast(uint32_t, value(i, j, bq, e));
            if (vec && n + 3 < N) {
              *(u32x4*)((uint32_t*)p.y + off) = v;
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                if (n + e < N) ((uint32_t*)p.y)[off + e] = v[e];
            }
          }
        }
      }
    } else {
      // 16-bit outputs through LDS, half a tile (128 rows x 256 columns, 64 KiB) at a time, whole
      // 512-byte row segments per wave; chunk c of staged row r at slot c ^ (r & 31).
      constexpr int kHalfRows = kQ8BM / 2, kChunks = kQ8BN / 8;
      wait_vmcnt<0>();  // the loads of stages past the end (which write zeros) have landed
      wait_lgkm();
      barrier_no_fence();
      const bool vec = (N % 8) == 0 && (((uintptr_t)p.y) & 15) == 0;
      static_for<0, 2>([&](auto hc) {
        constexpr int half = decltype(hc)::value;
#pragma unroll
        for (int i = 0; i < kQ8WN; ++i) {
          if ((wm * 32 * kQ8WM) / kHalfRows == half || (wm * 32 * kQ8WM + 32 * (kQ8WM - 1)) / kHalfRows == half)
            factors(i);
          static_for<0, kQ8WM>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            if ((wm * 32 * kQ8WM + 32 * j) / kHalfRows != half) return;
            const int r = wm * 32 * kQ8WM + 32 * j - half * kHalfRows + c32;
#pragma unroll
            for (int bq = 0; bq < 4; ++bq) {
              const int c = wn * 32 * kQ8WN + 32 * i + 8 * bq + 4 * h;
              uint32_t lo, hi;
              if constexpr (kOdt == kBF16) {
                lo = pack2_bf16(value(i, j, bq, 0), value(i, j, bq, 1));
                hi = pack2_bf16(value(i, j, bq, 2), value(i, j, bq, 3));
              } else {
                lo = pack2_f16(value(i, j, bq, 0), value(i, j, bq, 1));
                hi = pack2_f16(value(i, j, bq, 2), value(i, j, bq, 3));
              }
              typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
              *(u32x2*)(lds + r * (kQ8BN * 2) + (((c >> 3) ^ (r & 31)) << 4) + (c & 7) * 2) = u32x2{lo, hi};
            }
          });
        }
        barrier_no_fence();
#pragma unroll
        for (int k = 0; k < kHalfRows * kChunks / (64 * kQ8Waves); ++k) {
          const int q = threadIdx.x + k * 64 * kQ8Waves;
          const int r = q / kChunks, c = q % kChunks;
          const u32x4 v = *(const u32x4*)(lds + r * (kQ8BN * 2) + ((c ^ (r & 31)) << 4));
          const int m = m0 + half * kHalfRows + r, n = n0 + 8 * c;
          if (m < M && n < N) {
            uint16_t* dst = (uint16_t*)p.y + (size_t)m * N + n;
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
  switch (odt) {
    case kI32: epilogue(ic<kI32>{}); break;
    case kF32: epilogue(ic<kF32>{}); break;
    case kF16: epilogue(ic<kF16>{}); break;
    default: epilogue(ic<kBF16>{}); break;
  }
  wait_vmcnt<0>();  // no DMA into LDS outlives the workgroup
}

}  // namespace

hipError_t w8a8_tile256_launch(const W8A8Params& p, hipStream_t stream) {
  hipLaunchKernelGGL(w8a8_tile256_kernel, dim3(p.tiles_m * p.tiles_n), dim3(64 * kQ8Waves), 0, stream, p);
  return hipGetLastError();
}

}  // namespace qlinear
