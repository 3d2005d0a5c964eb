// Shared device helpers for the gfx950 (CDNA4, wave64) quantized-linear kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace qlinear {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

enum DType { kF32 = 0, kF16 = 1, kBF16 = 2, kI32 = 3 };
// Epilogue-internal output mode of the W4A16 kernels: each value is rounded to bf16 (the logical
// output dtype) and stored as the exact fp16 number value * 2^-e_m of its row m (see
// f16_row_factor), so the next GEMM takes it as its row-scaled fp16 operand without a staging pass.
constexpr int kBF16AsF16 = 5;

// The fp16 storage factor of an output row whose values are bounded in magnitude by b: down = 2^-e
// and up = 2^e with b * 2^-e in [2^14, 2^15) (e clamped to [-126, 126]; 1 for b = 0 or not finite).
// A bf16 value v with |v| <= b then maps to v * 2^-e <= 2^15 (1 + 2^-8) < 65504 exactly whenever
// |v| >= 2^(e - 17): the rows' values within 2^-31 of the bound keep all their bits.
__device__ __forceinline__ void f16_row_factor(float b, float& down, float& up) {
  int e = 0;
  if (b > 0.0f && b <= 3.4028235e38f) {
    int E;
    frexpf(b, &E);  // b = f 2^E, f in [0.5, 1)
    e = min(max(E - 15, -126), 126);
  }
  down = ldexpf(1.0f, -e);
  up = ldexpf(1.0f, e);
}
// The bound of an output row of x @ W^T + bias (optionally through GELU) from the row's input
// factor rs (max |x[m, :]| < 2^15 rs, as every row-scaled fp16 operand here guarantees) and the
// weight's bound {max_n sum_k |W_nk|, max_n |bias_n|}: |y| <= 2^15 rs max_n ||W_n||_1 + max|bias|,
// and |gelu(v)| <= max(|v|, 0.17). Rounding of this fp32 evaluation is covered by the 1e-4 factor.
__device__ __forceinline__ float w4a16_row_bound(float rs, float wl1, float bmax) {
  return (32768.0f * rs * wl1) * 1.0001f + bmax + 0.17f;
}

constexpr int kWave = 64;
constexpr int kGroup = 32;  // int4 quant group along K (ops.py BLOCK = 32)

// ---- scalar conversions ------------------------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __builtin_bit_cast(float, bits16 << 16);
}
__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}
// Round-to-nearest-even pack of two fp32 into one dword (v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32).
__device__ __forceinline__ uint32_t pack2_bf16(float lo, float hi) {
  bf16x2 v;
  v[0] = (__bf16)lo;
  v[1] = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, v);
}
// One v_cvt_pk_f16_f32 (round to nearest even) for the pair. Converting as a 2-vector also keeps
// the compiler from fusing a producing fp32 fma into v_fma_mix{lo,hi}_f16, whose half-register
// writes chain the two halves of the result dword.
__device__ __forceinline__ uint32_t pack2_f16(float lo, float hi) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, f16x2));
}

// 1 / c for a power of two c = 2^e, e in [-126, 126] (the column factors of the fp16 dequant):
// the exponent field reflected about the bias, one integer subtract and exact.
__device__ __forceinline__ float pow2_recip(float c) {
  return __builtin_bit_cast(float, 0x7F000000u - __builtin_bit_cast(uint32_t, c));
}

// Read element i of a buffer of dtype code dt as fp32.
__device__ __forceinline__ float read_elem(const void* p, int dt, size_t i) {
  if (dt == kF32) return ((const float*)p)[i];
  const uint32_t b = ((const uint16_t*)p)[i];
  return dt == kBF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
}

// Write fp32 v as dtype dt (RNE) to element i.
__device__ __forceinline__ void write_elem(void* p, int dt, size_t i, float v) {
  if (dt == kF32) {
    ((float*)p)[i] = v;
  } else if (dt == kBF16) {
    ((__bf16*)p)[i] = (__bf16)v;
  } else {
    ((_Float16*)p)[i] = (_Float16)v;
  }
}

// Round v to the 16-bit dtype dt (kBF16 / kF16, RNE) and back to fp32; fp32 passes through.
__device__ __forceinline__ float round_to(int dt, float v) {
  if (dt == kBF16) return (float)(__bf16)v;
  if (dt == kF16) return (float)(_Float16)v;
  return v;
}

// Gated residual on 8 consecutive 16-bit outputs (dtype DT, packed pairs in w, each already the
// rounded output value v): residual + gate * v in fp32 (the product of two 16-bit numbers is
// exact in fp32, so only the sum rounds before the final rounding to DT). cnt < 8 (the row's end)
// reads only the first cnt residuals and gates; vec allows the 16-byte loads.
template <int DT>
__device__ __forceinline__ u32x4 gated_residual8(u32x4 w, const uint16_t* res, const uint16_t* gate, int cnt,
                                                 bool vec) {
  u32x4 r = {0u, 0u, 0u, 0u}, g = {0u, 0u, 0u, 0u};
  if (vec && cnt == 8) {
    r = *(const u32x4*)res;
    g = *(const u32x4*)gate;
  } else {
    for (int e = 0; e < cnt; ++e) {
      r[e >> 1] |= (uint32_t)res[e] << (16 * (e & 1));
      g[e >> 1] |= (uint32_t)gate[e] << (16 * (e & 1));
    }
  }
  auto f = [](uint32_t bits) { return DT == kBF16 ? bf16_bits_to_f32(bits) : f16_bits_to_f32(bits); };
  u32x4 o;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float lo = f(r[q] & 0xFFFFu) + f(g[q] & 0xFFFFu) * f(w[q] & 0xFFFFu);
    const float hi = f(r[q] >> 16) + f(g[q] >> 16) * f(w[q] >> 16);
    o[q] = DT == kBF16 ? pack2_bf16(lo, hi) : pack2_f16(lo, hi);
  }
  return o;
}

// GELU, tanh approximation, in fp32: 0.5 x (1 + tanh(u)), u = sqrt(2/pi) (x + 0.044715 x^3), the
// form of torch.nn.functional.gelu(approximate="tanh") that the reference's DiT MLP applies between
// its two linears. Evaluated through the identity 0.5 (1 + tanh(u)) =
// 1 / (1 + e^(-2u)): one exp2 and one reciprocal instead of a tanhf (about 30 instructions), so
// the epilogue of a 4608 x 12288 output does not stall the GEMM. Relative error a few fp32 ulp,
// below the rounding of a 16-bit output. x -> -inf gives 1 / inf = 0 and -0.0; x -> +inf gives x.
__device__ __forceinline__ float gelu_tanh(float x) {
  // -2 u log2(e) = x (c1 + c2 x^2)
  const float c1 = -2.0f * 0.7978845608028654f * 1.4426950408889634f;
  const float c2 = c1 * 0.044715f;
  const float t = x * (c1 + c2 * (x * x));
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(t));
}

// rint(fl(v / s)) of a quantizer whose codes satisfy |v / s| <= 128 (scale s = amax * c,
// c <= 1/7), bit for bit, with a multiplication by r = fl(1 / s) (computed once per scale) in
// place of the division: v r = (v / s)(1 + d1)(1 + d2) with |d1|, |d2| <= 2^-24 lies within
// 128 * 2^-23 (1 + 2^-24) < 2^-15.9 of v / s, so the two round to the same integer unless v / s
// lies that close to a half-integer (ties go to even in both). Those, and NaN, take the exact
// quotient: where |frac(v r) - 1/2| <= 2^-15. (y - floor(y) is exact for |y| < 2^23.)
__device__ __forceinline__ bool quot_near_half(float y) { return !(fabsf((y - floorf(y)) - 0.5f) > 0x1p-15f); }
// N values at a time: the multiplications for all of them, the exact quotients only in a block
// that a wave skips unless one of its lanes needs it (one value in about 2^13)
template <int N>
__device__ __forceinline__ void rint_quot_n(const float* v, float s, float r, float* q) {
  bool need = false;
#pragma unroll
  for (int e = 0; e < N; ++e) {
    const float y = __fmul_rn(v[e], r);
    q[e] = rintf(y);
    need |= quot_near_half(y);
  }
  if (need) {
#pragma unroll
    for (int e = 0; e < N; ++e)
      if (quot_near_half(__fmul_rn(v[e], r))) q[e] = rintf(__fdiv_rn(v[e], s));
  }
}

// ---- compile-time loops ----------------------------------------------------------------------
// static_for<B, E>(f) calls f(std::integral_constant<int, i>{}) for i = B .. E-1 as straight-line
// code: the index is a constant expression inside f, so register arrays indexed by it stay in
// registers whatever the compiler's unrolling heuristics decide about loop size.
template <int I>
struct ic {
  static constexpr int value = I;
};
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(ic<B>{});
    static_for<B + 1, E>(f);
  }
}

// ---- int4 -> 16-bit dequant in registers ---------------------------------------------------
// One packed dword holds 8 consecutive K elements: nibble t (bits 4t..4t+3) is element t,
// two's complement (the reference's packing, ops.py:119-121). Returns the 8 values q*s
// rounded to bf16/fp16, natural order, two per dword (element 2b in the low half of dword b).
// u = nibble ^ 8 = q + 8 is exact as a byte; fmaf(u, s, -8s) = q*s rounded once in fp32
// (the product is exact inside the FMA and -8s is exact), then one RNE rounding to 16 bits.
template <bool kBf16>
__device__ __forceinline__ u32x4 dequant8(uint32_t w, float s, float neg8s) {
  const uint32_t ev = (w & 0x0F0F0F0Fu) ^ 0x08080808u;         // bytes: u0 u2 u4 u6
  const uint32_t od = ((w >> 4) & 0x0F0F0F0Fu) ^ 0x08080808u;  // bytes: u1 u3 u5 u7
  u32x4 r;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const float lo = fmaf((float)((ev >> (8 * b)) & 0xFFu), s, neg8s);
    const float hi = fmaf((float)((od >> (8 * b)) & 0xFFu), s, neg8s);
    r[b] = kBf16 ? pack2_bf16(lo, hi) : pack2_f16(lo, hi);
  }
  return r;
}

// ---- MFMA wrappers (v_mfma_f32_16x16x32_{bf16,f16}, v_mfma_i32_16x16x64_i8) ----------------
// Operand layout (lane l of 64): A supplies row l%16, B supplies column l%16, each with the
// 8 (16-bit) or 16 (int8) K values of K-slot block l/16; D lane l holds column l%16,
// rows 4*(l/16) + 0..3. The kernels only rely on A and B using the same K-slot map.
template <bool kBf16>
__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (kBf16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                  __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                 __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}
__device__ __forceinline__ i32x4 mfma16_i8(u32x4 a, u32x4 b, i32x4 c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, a),
                                              __builtin_bit_cast(i32x4, b), c, 0, 0, 0);
}

// ---- direct global -> LDS 16-byte loads (global_load_lds_dwordx4) ----------------------------
// Lane i of the wave writes its 16 bytes to lds_base + 16*i; lds_base must be wave-uniform.
__device__ __forceinline__ void load_lds16(const void* gptr, void* lds_base) {
  __builtin_amdgcn_global_load_lds(gptr, (__attribute__((address_space(3))) void*)lds_base, 16, 0, 0);
}
// ---- raw buffer loads ------------------------------------------------------------------------
// A buffer resource covers [base, base + bytes); a load whose offset (per-lane voffset + wave-uniform
// soffset) lies at or past `bytes` returns zeros instead of touching memory. The kernels use this
// for every edge (rows past M, columns past N, K past the end) and advance through K by bumping
// the scalar offset, so no per-stage vector address arithmetic is needed.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int kRsrcWord3 = 0x00020000;      // gfx9 V# word 3: 32-bit data format, raw access
constexpr uint32_t kOobOffset = 0x80000000u;  // voffset that is out of range for every resource here

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kRsrcWord3);
}
__device__ __forceinline__ u32x4 buf_load16(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
}
__device__ __forceinline__ float buf_load_f32(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}

// Buffer load of 16 B per lane straight into LDS (buffer_load_dwordx4 ... lds): lane i of the wave
// writes lds_base + 16*i; lds_base must be wave-uniform. Out-of-range lanes write zeros.
__device__ __forceinline__ void buf_load16_lds(rsrc_t r, void* lds_base, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_base, 16, voff, soff, 0,
                                           0);
}

// s_waitcnt as a real instruction (not inline asm), so the compiler's own wait insertion knows
// which counters are already drained. gfx9 encoding: vmcnt [3:0]+[15:14], expcnt [6:4],
// lgkmcnt [11:8]; a field at its maximum means "do not wait" on that counter.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }   // vmcnt(0)
// vmcnt(N): at most N vector-memory instructions of this wave still outstanding (in issue order)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit field");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | 0x0F70);
}
__device__ __forceinline__ void wait_lgkm() { __builtin_amdgcn_s_waitcnt(0xC07F); }   // lgkmcnt(0)

// ---- LDS layout of 256-byte operand rows ----------------------------------------------------
// A stage row is 16 chunks of 16 B; logical chunk c of row r is stored in slot c ^ lds_swz(r & 15).
// An MFMA operand read (ds_read_b128) has lane l fetch row l % 16, chunk 4 * (l / 16) + i. The LDS
// serves such a read 32 lanes (512 B, all 128 banks) at a time, so the 32 chunks of lanes 0-31
// (rows 0-15, chunk blocks 0 and 1; likewise 32-63) must land in 32 distinct 16-byte bank
// groups of the 512-byte line formed by rows r and r ^ 1. lds_swz is the bit permutation
// (r1 r2 r0 r3) of r: the 8 rows of one parity then use chunk offsets that are distinct and never
// differ by 4 (the gap between chunk blocks 0 and 1), and all 16 rows together are still
// conflict-free for 16-lane (256 B) service.
__device__ __forceinline__ int lds_swz(int r) { return ((r >> 1) & 3) | ((r & 1) << 2) | (r & 8); }

// Workgroup barrier without the memory fence of __syncthreads(): the fence would also wait for
// every outstanding global load (vmcnt(0)), including prefetches meant to stay in flight across
// the barrier. Callers wait for exactly what the barrier publishes (wait_vmcnt / wait_lgkm)
// first; the empty asm statements keep the compiler from moving memory accesses across it.
__device__ __forceinline__ void barrier_no_fence() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// ---- workgroup -> tile order ---------------------------------------------------------------
// Workgroups are dispatched round-robin over the 8 XCDs (each with its own L2). Renumber them
// so that consecutive logical ids run on the same XCD and share A/B panels in its L2.
__host__ __device__ __forceinline__ int xcd_remap(int g, int G) {
  constexpr int kXcd = 8;
  const int xcd = g % kXcd, local = g / kXcd;
  const int per = G / kXcd, rem = G % kXcd;
  return xcd < rem ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
}

// Grouped ("super-tile") order: kGroupM tile-rows walk the N tiles together.
__host__ __device__ __forceinline__ void tile_coords(int t, int tiles_m, int tiles_n, int group_m, int& tm,
                                                     int& tn) {
  const int per_group = group_m * tiles_n;
  const int grp = t / per_group;
  const int first_m = grp * group_m;
  const int gsize = tiles_m - first_m < group_m ? tiles_m - first_m : group_m;
  const int r = t - grp * per_group;
  tm = first_m + r % gsize;
  tn = r / gsize;
}

}  // namespace qlinear
