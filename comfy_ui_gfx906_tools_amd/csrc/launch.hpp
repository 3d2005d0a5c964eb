// Host-side launch interface between the C ABI (capi.cpp) and the kernel files.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace qlinear {

enum Activation { kActNone = 0, kActGeluTanh = 1 };

// Tile rows that walk the tile columns together in each kernel's grouped tile order
// (tile_coords in common.hpp); the launch-plan check in capi.cpp enumerates with the same values.
constexpr int kW4A16GroupM = 8;     // w4a16_gemm.hip, configurations 0-3
constexpr int kTile256GroupM = 4;   // w4a16_tile256.hip
constexpr int kW4A4GroupM = 8;      // w4a4_gemm.hip
constexpr int kW8A8GroupM = 8;      // w8a8_gemm.hip
constexpr int kW8A8T256GroupM = 4;  // w8a8_tile256.hip

struct W4A16Params {
  const void* x;         // [M, K] bf16 / fp16
  const void* wq;        // [N, K/2] packed int4
  const float* ws;       // [N, K/32], or [K/32, N] (group-major) when scales_kn
  const void* bias;      // [N] out dtype, or null
  void* y;               // [M, N] out dtype
  const float* row_scale;  // [M] power-of-two factor applied in the epilogue, or null
  // [N] power-of-two factor 2^e_n per output column, or null (tile kernels, fp16 dequant): the
  // group scales of column n are multiplied by 2^-e_n before the fp16 rounding of q * s and the
  // epilogue multiplies by 2^e_n, so every column's dequantized weights sit in fp16's normal range
  const float* col_scale;
  // out_dtype kBF16AsF16: {max_n ||W_n||_1, max_n |bias_n|} (w4a16_out_bound_launch) and the
  // output's fp16 row factors 2^e_m [M], written by the kernels
  const float* out_bound;
  float* out_row_scale;
  float* partial;        // partial tiles of the cut tiles: (tiles - dp_tiles) * ksplit slots of BM * BN fp32
  int M, N, K;
  int out_dtype;
  int act;               // epilogue activation: kActNone or kActGeluTanh (256 x 256 kernel only)
  int tiles_m, tiles_n;
  int stages;            // K loop steps: ceil(K / (128 * w4a16_nbuf(WM)))
  int dp_tiles;          // tiles processed whole, one workgroup each
  int ksplit;            // K pieces of every tile past dp_tiles (>= 2 when any)
  int tile_base;         // 256 x 256 kernel: first tile of the launch (set by the launcher)
  int tile_rows;         // 256-column kernel, variant 1: tile height 64, 128 or 256
  int scales_kn;         // ws is group-major [K/32, N] (qlinear_w4a16_scales_kn)
  // Gated residual epilogue (or null): y = residual + gate[m / gate_rows] * v, v the output as it
  // would be stored (rounded to out_dtype), in fp32, rounded once more; residual [M, N] and gate
  // [ceil(M / gate_rows), N] in out_dtype; y may be residual itself (each element is read and
  // written by the same thread)
  const void* residual;
  const void* gate;
  int gate_rows;
  int cus;               // compute units of the device (grid sizing)
};

struct W4A16Config {
  int id, BM, BN;
};

// LDS stage buffers of the W4A16 kernel for a tile of 16*WM rows: three (loads two stages ahead)
// while they fit, two for 256-row tiles.
constexpr int w4a16_nbuf(int WM) { return WM >= 16 ? 2 : 3; }
// K loop steps (of w4a16_nbuf stages of 128 K) for config `cfg`
int w4a16_steps(int cfg, int64_t K);

const W4A16Config& w4a16_config(int id);
hipError_t w4a16_launch(int cfg, bool bf16, const W4A16Params& p, hipStream_t stream);
// 256 x 256 tiles, 32x32x16 MFMA (w4a16_tile256.hip), K % 64 == 0. Variant 0: 8 waves as 2 x 4
// (128 x 64 each); 1: 8 waves as 1 x 8 (256 x 32); 2: 4 waves as 1 x 4 (256 x 64). The first
// p.dp_tiles tiles (grouped order) run whole, the rest as two 128-row halves each (second launch).
constexpr int kTile256Variants = 3;
hipError_t w4a16_tile256_launch(int variant, bool bf16, const W4A16Params& p, hipStream_t stream);
// Activation rows up to 4, bf16 / fp16 x as is, K <= 8192 and M * K <= 16384 (w4a16_gemv.hip):
// VALU dot products on exact integer codes, columns streamed by four waves per SIMD.
constexpr int kGemvMaxM = 4, kGemvMaxK = 8192, kGemvMaxMK = 16384;
hipError_t w4a16_gemv_launch(bool bf16, const W4A16Params& p, hipStream_t stream);
// MFMA kernel for M <= 16 (w4a16_skinny.hip): `blocks` (1-3) blocks of 16 columns per workgroup,
// K split over its 8 waves; K % 128 == 0, K <= 4096.
constexpr int kSkinnyMaxM = 16, kSkinnyMaxK = 4096, kSkinnyMaxBlocks = 3;
hipError_t w4a16_skinny_launch(bool bf16, int blocks, const W4A16Params& p, hipStream_t stream);
hipError_t rows_to_scaled_f16_launch(int dtype, const void* x, void* x16, float* row_scale, int64_t M,
                                     int64_t K, hipStream_t stream);
// Sums the ksplit fp32 partials [BM][BN] of every cut tile (tiles p.dp_tiles .. of the grouped order
// with group_m tile rows) in piece order and applies the epilogue (w4a16_gemm.hip).
hipError_t w4a16_reduce_launch(const W4A16Params& p, int BM, int BN, int group_m, hipStream_t stream);
// col_scale[n] = 2^e_n with 8 max_g |w_scale[n, g]| * 2^-e_n in [2^14, 2^15), e_n clamped to
// [-126, 126]; 1 for a column whose scales are all zero or not finite (w4a16_gemm.hip).
// w_scale [N, groups] -> w_scale_kn [groups, N] (group-major copy read by the tile kernels)
// one read of `bytes` bytes (a multiple of 16) by `workgroups` workgroups; xor words to out[workgroups]
hipError_t stream_read_launch(const void* buf, int64_t bytes, uint32_t* out, int workgroups, hipStream_t stream);
hipError_t scales_kn_launch(const float* w_scale, float* w_scale_kn, int64_t N, int64_t groups, hipStream_t stream);
hipError_t col_scales_launch(const float* w_scale, float* col_scale, int64_t N, int64_t groups, hipStream_t stream);
// bound[0] = max_n sum_k |q_nk s_n,k/32| (1 + 2^-10), bound[1] = max_n |bias_n| (0 without bias);
// bound[2 ..] holds per-workgroup partial maxima, (N + 3) / 4 floats (w4a16_gemm.hip).
hipError_t w4a16_out_bound_launch(const void* w_q4, const float* w_scale, const void* bias, int bias_dtype, int64_t N,
                                  int64_t K, float* bound, hipStream_t stream);

struct W8A8Params {
  const int8_t* xq;      // [M, K]
  const float* sx;       // [M]
  const int8_t* wq;      // [N, K]
  const float* sw;       // [N]
  const void* bias;      // [N] out dtype, or null
  void* y;               // [M, N]
  int M, N, K;
  int out_dtype;         // kF32 / kF16 / kBF16 / kI32
  int tiles_m, tiles_n;
  int stages;            // K / 256
};

struct W8A8Config {
  int id, BM, BN;
};
const W8A8Config& w8a8_config(int id);
hipError_t w8a8_launch(int cfg, const W8A8Params& p, int grid, hipStream_t stream);
// 256 x 256-tile int8 MFMA kernel for M > 128 (grid = tiles_m * tiles_n of 256 x 256)
constexpr int kW8A8Tile256 = 256;
hipError_t w8a8_tile256_launch(const W8A8Params& p, hipStream_t stream);

hipError_t quantize_int4_launch(int dtype, int rule, const void* x, void* packed, float* scale,
                                int64_t rows, int64_t K, hipStream_t stream);
hipError_t repack_q4_0_launch(const void* raw, void* packed, float* scale, int64_t blocks, hipStream_t stream);
hipError_t quantize_int8_per_token_launch(int dtype, const void* x, int8_t* q, float* scale,
                                          int64_t M, int64_t K, hipStream_t stream);

// W4A4 GEMM with the reference's per-block fmaf accumulation (w4a4_gemm.hip).
struct W4A4Params {
  const void* a;         // [M, K/2] packed int4
  const float* as;       // [M, K/qb]
  const void* b;         // [N, K/2] packed int4
  const float* bs;       // [N, K/qb]
  const void* bias;      // [N] out dtype, or null
  void* y;               // [M, N] out dtype
  int M, N, K;
  int out_dtype;
  int tiles_m, tiles_n;  // 128 x 128 tiles
  // split-K (int4 only): splits > 1 cuts K into ranges of stages_per_split 128-K stages; split s
  // writes its fp32 partial [M, N] (no bias) to partial + s * M * N, summed by a second kernel
  int splits, stages_per_split;
  float* partial;
};
hipError_t w4a4_launch(int qblock, const W4A4Params& p, hipStream_t stream);
// The same kernel with int8 codes ([M, K] / [N, K], block-32 scales): the reference's gemm_int8.
hipError_t int8_block32_launch(const W4A4Params& p, hipStream_t stream);
hipError_t quantize_int8_block32_launch(int dtype, const void* x, int8_t* q, float* scale, int64_t blocks,
                                       hipStream_t stream);

// Activation rotation + fp16 staging in one pass (rotate.hip): group 32 / 64 / 128, K % group == 0,
// K <= 16384.
hipError_t rotate_rows_to_f16_launch(int x_dtype, int group, const void* x, const float* signs, void* x16,
                                     float* row_scale, int64_t M, int64_t K, hipStream_t stream);

// Fused DiT block glue (dit_fused.hip). K % 8 == 0 and K <= 16384 for the LayerNorm kernel;
// head dim 128 for the q/k kernel; K % 8 == 0 for the residual.
// adaLN of rows of x into: kOperandF16 the row-scaled fp16 W4A16 operand (+ row_scale), kOperandPlain
// x's dtype, kOperandI8 the per-token int8 W8A8 operand (+ its scales in row_scale)
constexpr int kOperandF16 = 0, kOperandPlain = 1, kOperandI8 = 2;
hipError_t adaln_launch(int out_kind, int x_dtype, int mod_dtype, const void* x, const void* shift, const void* scale,
                        void* out, float* row_scale, int64_t M, int64_t K, float eps, hipStream_t stream);
hipError_t qk_norm_rope_launch(int dtype, const void* qkv, const void* q_norm, const void* k_norm, const float* cosv,
                               const float* sinv, void* q, void* k, void* v, int64_t L, int64_t H, int64_t L_out,
                               int64_t l0, float eps, hipStream_t stream);
hipError_t gated_residual_launch(int dtype, void* out, const void* x, const void* gate, const void* y, int64_t M,
                                 int64_t K, hipStream_t stream);
hipError_t heads_gather_launch(int out_kind, int dtype, const void* o, int64_t H, int64_t L_all, int64_t l0,
                               int64_t rows, const void* extra, int64_t E, void* out, float* row_scale,
                               hipStream_t stream);

}  // namespace qlinear
