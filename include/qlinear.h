/*
 * qlinear.h -- C ABI of libqlinear.so, the gfx950 (MI355X) quantized-linear engine.
 *
 * Plain pointers, sizes and an opaque stream. The library never allocates or frees:
 * every buffer, workspace included, is passed in by the caller (PyTorch's caching
 * allocator on the Python side), and every launch goes on the caller's HIP stream.
 *
 * Return value of every entry point: 0 (QL_OK) or one of the QL_ERR_* codes below;
 * qlinear_last_error() then returns a message naming expected vs actual, kept per host
 * thread. Entry points are re-entrant and keep no global mutable state beyond a
 * per-device, lock-protected cache of the CU count.
 *
 * Layouts shared with the reference (luna-niemitalo/comfy_ui_gfx906_tools):
 *   packed int4 weight  int8  [N, K/2]  byte j of a row = code[2j] & 0xF | (code[2j+1] & 0xF) << 4,
 *                                       codes two's complement in [-8, 7]
 *                                       (nodes/ComfyUI-Gfx906Int4/ops.py:108-126)
 *   group scales        fp32  [N, K/32] one scale per 32 consecutive K elements (ops.py:215)
 *   dtype codes         0 = fp32, 1 = fp16, 2 = bf16 (csrc/binding.cpp:45-50); 3 = int32 is an
 *                       output-only code of this library (raw W8A8 accumulators)
 * All row-major, rows contiguous; pointers 16-byte aligned.
 */
#ifndef QLINEAR_H
#define QLINEAR_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum qlinear_dtype { QL_F32 = 0, QL_F16 = 1, QL_BF16 = 2, QL_I32 = 3 };

enum qlinear_status {
  QL_OK = 0,
  QL_ERR_ARG = 1,       /* null pointer, bad enum, bad option */
  QL_ERR_SHAPE = 2,     /* sizes inconsistent or out of the supported range */
  QL_ERR_DTYPE = 3,     /* dtype not supported for this operand */
  QL_ERR_ALIGN = 4,     /* pointer not 16-byte aligned */
  QL_ERR_WORKSPACE = 5, /* workspace missing or too small */
  QL_ERR_LAUNCH = 6,    /* HIP runtime error at launch */
  QL_ERR_DEVICE = 7     /* HIP device query failed */
};

/* Message for the last failing call on this host thread ("" if none). */
const char* qlinear_last_error(void);

/* ABI version of this header: (major << 16) | minor. 2.0: qlinear_w4a16_gemm takes col_scale;
 * 3.0: qlinear_w4a16_gemm(_noalloc) take w_scale_kn; 4.0: and residual. */
int qlinear_abi_version(void);

/* ---------------------------------------------------------------------------------------
 * W4A16 linear: y[M,N] = x[M,K] @ dequant(w_q4, w_scale)^T (+ bias[N]).
 * Replaces the pair ext.quantize_int4 + ext.gemm_int4 that int4_linear calls
 * (nodes/ComfyUI-Gfx906Int4/ops.py:181-182; csrc/binding.cpp:53-112; dispatchers
 * csrc/int4_gemm_scaled.hip:248-269): the activation is not quantized here, the weight is
 * dequantized in registers and fed to 16-bit MFMA with fp32 accumulation.
 *   x_dtype   QL_F16: fp16 MFMA on x as given; if row_scale is not NULL, row m of the product
 *             is multiplied by row_scale[m] in the epilogue (x as written by qlinear_rows_to_f16).
 *             QL_BF16 / QL_F32: by default each row of x is first scaled by an exact power of
 *             two into an fp16 copy (in the workspace, as qlinear_rows_to_f16 does) and the
 *             weights dequantize to fp16 -- 8x less weight rounding than bf16 -- and the
 *             epilogue scales back exactly. With QL_W4A16_BF16_MFMA in flags, bf16 x is fed to
 *             bf16 MFMA directly (the reference's own bf16 dequant-then-matmul numerics; no
 *             staging pass; the automatic choice then stays on the tile kernels 0-6).
 *             row_scale must be NULL for these dtypes.
 *   out_dtype QL_F32, QL_F16 or QL_BF16; bias (optional, may be NULL) has dtype out_dtype
 *   K % 32 == 0, K >= 32; M >= 0 (M == 0 launches nothing)
 *   splits    0 = automatic (under-filled last waves are cut into K pieces),
 *             1 = one workgroup per output tile, 2..64 = that many K pieces per tile.
 *   w_scale_kn [K/32, N] fp32 from qlinear_w4a16_scales_kn(w_scale), or NULL (below).
 *   col_scale [N] fp32 from qlinear_w4a16_col_scales(w_scale), or NULL (then computed into the
 *             workspace by the call); read only by the tile kernels on the fp16 route.
 *   workspace device memory of qlinear_w4a16_workspace_bytes(...) bytes (NULL when that is 0),
 *             scratch for the fp16 staging copy, the column factors and split-K partial tiles;
 *             no initial contents needed. Calls sharing one workspace must be ordered (same
 *             stream).
 * ------------------------------------------------------------------------------------- */
#define QL_W4A16_BF16_MFMA 1 /* flags bit, see above */
/* flags bit: GELU (tanh approximation) epilogue, y = gelu(round(x @ W^T + bias)) with the linear's
 * result first rounded to out_dtype, then gelu_tanh in fp32 and rounded again -- the sequence
 * Linear -> nn.GELU(approximate="tanh") of the DiT MLP, in one kernel (no counterpart in the
 * reference's extension, whose GELU is a separate torch op). */
#define QL_W4A16_GELU_TANH 2
/* flags bit: store the output as the next GEMM's row-scaled fp16 operand instead of bfloat16.
 * Each value is computed exactly as for out_dtype QL_BF16 (GELU included) and rounded to bf16,
 * then stored as the fp16 number value * 2^-e_m, exact for every value of row m above 2^-31 of
 * the row's bound B_m = 2^15 rs_m max_n ||W_n||_1 (1 + 1e-4) + max|bias| + 0.17 (rs_m = the input
 * row factor: max |x[m, :]| < 2^15 rs_m; 0.17 bounds GELU's negative lobe), with 2^-e_m B_m in
 * [2^14, 2^15) so nothing overflows; out_row_scale[m] = 2^e_m. Pass y (fp16 [M, N]) and
 * out_row_scale to the next qlinear_w4a16_gemm as x (QL_F16) and row_scale: the bf16 activation
 * between two linears without the staging pass. out_dtype must be QL_BF16 (the logical dtype),
 * bias bfloat16; x float16 with row_scale, or bfloat16 / float32 x on the fp16 route; out_bound
 * from qlinear_w4a16_out_bound for this w_q4 / w_scale / bias. Tile kernels 0-3 and 5 only (the
 * automatic plan never picks another). No counterpart in the reference, whose linears each read
 * and write their activations. */
#define QL_W4A16_F16_ROWSCALED 4
/* flags bit: gated residual epilogue, y = residual + gate[m / gate_rows] (.) v, where v is the
 * output as it would otherwise be stored (bias, activation, rounded to out_dtype) and the sum is
 * formed in fp32 (the product of two 16-bit numbers is exact there) and rounded to out_dtype: the
 * result of this GEMM followed by the elementwise kernel x + gate * y, in one pass (a DiT block's
 * "x = x + gate * linear(h)"). residual [M, N] and gate [ceil(M / gate_rows), N] have out_dtype,
 * aligned to their elements; y may be residual itself (in place), any other overlap is undefined.
 * Described by the ql_w4a16_residual passed as `residual` (NULL without this flag). Not with
 * QL_W4A16_F16_ROWSCALED; tile kernels 0-5 only (the automatic plan picks no other). No
 * counterpart in the reference, whose linears end at the bias. */
#define QL_W4A16_GATED_RESIDUAL 16
typedef struct ql_w4a16_residual {
  const void* residual; /* [M, N], out_dtype */
  const void* gate;     /* [ceil(M / gate_rows), N], out_dtype */
  int64_t gate_rows;    /* output rows per gate row: M for one gate row, L for [B, L, N] outputs */
} ql_w4a16_residual;
/* flags bits 8-11: 0 = automatic kernel choice, c + 1 = force kernel configuration c
 * (0-3: 256 / 128 / 64 / 16-row x 256-column tiles, 4 waves; 4-6: 256-column tiles with 8 waves
 * as 2 x 4, 8 waves as 1 x 8, 4 waves as 1 x 4, K % 64 == 0; 256 x 256 tiles, a last round at
 * most half full run as 128-row halves; 5 also takes the tile height and K pieces its plan
 * picks: 64 / 128 rows for M <= 64 / 128, 224 rows where that fills a single round better, and
 * K pieces (fp32 partials summed in order) when the tiles fill at most a third of the CUs; 7: M <= 4,
 * K <= 8192, bfloat16/float16 x read as given, VALU dot products on the exact integer codes with
 * the group scale applied in fp32 -- the automatic choice for M = 1; 8: M <= 16, K % 128 == 0,
 * K <= 4096, bfloat16/float16 x read as given, MFMA on the exact integer codes with the group
 * scale applied in fp32 -- the automatic choice for 2 <= M <= 16 where it applies). For tuning
 * and tests; results agree to rounding. */
#define QL_W4A16_CFG_SHIFT 8
#define QL_W4A16_CFG_MASK (0xF << QL_W4A16_CFG_SHIFT)
#define QL_W4A16_CFG(c) (((c) + 1) << QL_W4A16_CFG_SHIFT)

size_t qlinear_w4a16_workspace_bytes(int x_dtype, int64_t M, int64_t N, int64_t K, int splits,
                                     int flags, int device);

int qlinear_w4a16_gemm(int x_dtype, int out_dtype, const void* x, const float* row_scale,
                       const void* w_q4, const float* w_scale, const float* w_scale_kn,
                       const float* col_scale, const void* bias, void* y, const float* out_bound,
                       float* out_row_scale, const ql_w4a16_residual* residual, int64_t M,
                       int64_t N, int64_t K, int splits, int flags, void* workspace,
                       size_t workspace_bytes, void* stream);

/* Group-major copy of the group scales: w_scale_kn[g * N + n] = w_scale[n * (K/32) + g]
 * ([K/32, N] fp32, N * K / 8 bytes). Passed as w_scale_kn to qlinear_w4a16_gemm (NULL there =
 * read w_scale), the tile kernels (configurations 0-6) read it instead of w_scale: a stage of a
 * 256-column tile then needs its scales as a few runs of 1 KiB rather than 8-16 bytes from each of
 * 256 column rows. Measured on MI355X for a weight stream like the skinny-M GEMMs' (N = 65536,
 * K = 4096, no arithmetic): 68 us with the column rows, 40 us group-major, 35 us with no scales
 * at all. The results are the same bit for bit; only the addresses change. w_scale itself is
 * still read by the direct kernels (7, 8: whole column rows, already long runs) and by the
 * column-factor pass. Depends only on w_scale: compute once per weight and keep it with the
 * weight. No counterpart in the reference (its scales stay [N, K/32]). */
int qlinear_w4a16_scales_kn(const float* w_scale, float* w_scale_kn, int64_t N, int64_t K,
                            void* stream);

/* The weight's output bound for QL_W4A16_F16_ROWSCALED: bound[0] = max_n sum_k |dequant W_nk| *
 * (1 + 2^-10), bound[1] = max_n |bias_n| (0 when bias is NULL). bound holds
 * QL_W4A16_OUT_BOUND_FLOATS(N) floats (the rest is scratch of the two-pass reduction). Depends
 * only on w_q4, w_scale and bias: compute once per weight. */
#define QL_W4A16_OUT_BOUND_FLOATS(N) (2 + ((N) + 3) / 4)
int qlinear_w4a16_out_bound(const void* w_q4, const float* w_scale, const void* bias, int bias_dtype,
                            int64_t N, int64_t K, float* bound, void* stream);

/* Allocation-free variant of qlinear_w4a16_gemm, with the same arguments, checks and results
 * minus the workspace. No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that forbid it).
 * Its workspace is a static device array of QL_W4A16_NOALLOC_SCRATCH_BYTES in the library, one
 * per GPU, held from the library's load until the process ends; the call makes no hipMalloc,
 * hipFree or other allocation. A call whose plan needs more scratch than that (see
 * qlinear_w4a16_workspace_bytes) fails with QL_ERR_WORKSPACE before launching anything. Every
 * call on one GPU shares that GPU's array: calls that overlap on one GPU (different streams or
 * host threads without ordering) race on it; calls on one stream are ordered. The scratch needs
 * no initial contents (each call writes what it reads). */
#define QL_W4A16_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int qlinear_w4a16_gemm_noalloc(int x_dtype, int out_dtype, const void* x, const float* row_scale,
                               const void* w_q4, const float* w_scale, const float* w_scale_kn,
                               const float* col_scale, const void* bias, void* y,
                               const float* out_bound, float* out_row_scale,
                               const ql_w4a16_residual* residual, int64_t M, int64_t N, int64_t K,
                               int splits, int flags, void* stream);

/* Column factors of the fp16 dequant: col_scale[n] = 2^e_n with 8 * max_g |w_scale[n, g]| * 2^-e_n
 * in [2^14, 2^15) (e_n clamped to [-126, 126]; 1 for a column whose scales are all 0 or not
 * finite). The tile kernels (configurations 0-6 on the fp16 route) dequantize column n as
 * fp16(q * s * 2^-e_n) and multiply the column by 2^e_n in the epilogue, so weights of any fp32
 * scale keep 11 significant bits without overflow (the reference's bf16 dequant, nodes.py:116,
 * keeps the full exponent range too); where q * s is a normal fp16 number the result is the
 * same bit for bit. qlinear_w4a16_gemm computes them into its workspace when col_scale is NULL
 * (one small launch per call); a caller that keeps them with the weight computes them once here
 * and passes them in. They depend only on w_scale. K % 32 == 0. No counterpart in the reference. */
int qlinear_w4a16_col_scales(const float* w_scale, float* col_scale, int64_t N, int64_t K,
                             void* stream);

/* Staging pass of the fp16 route: x[M,K] (fp32/fp16/bf16, K % 8 == 0) -> x16[M,K] fp16 with
 * row m scaled by 2^-e_m, row_scale[m] = 2^e_m, e_m chosen so max|x16[m,:]| is in [2^14, 2^15)
 * (exact for bf16 and fp16 inputs). No counterpart in the reference, whose activations go to
 * int4 instead (csrc/int4_gemm_scaled.hip:193-220). */
int qlinear_rows_to_f16(int x_dtype, const void* x, void* x16, float* row_scale, int64_t M,
                        int64_t K, void* stream);

/* Number of workgroups per output tile that splits == 0 resolves to; mirrors
 * ext.gemm_int4_auto_splits (csrc/binding.cpp:36-43, 359-362). */
int qlinear_w4a16_auto_splits(int64_t M, int64_t N, int64_t K, int device);

/* Rotated fp16 staging: per row, every group of `group` (32, 64 or 128) elements along K becomes
 * y_g = H (signs * x_g) / sqrt(group) (Sylvester Hadamard H; signs fp32 +-1 [group]), i.e.
 * x_g R^T with R = H diag(signs) / sqrt(group), then is written as qlinear_rows_to_f16 writes
 * (x16 = y * 2^-e_m, row_scale[m] = 2^e_m; pass both to qlinear_w4a16_gemm with x_dtype QL_F16).
 * Replaces the fp32 activation rotation of a rotated layer's forward (ops.py:176-179,
 * apply_group_rotation ops.py:85-105) plus the staging pass. K % group == 0, K <= 16384. */
int qlinear_rotate_rows_to_f16(int x_dtype, const void* x, const float* signs, int group, void* x16,
                               float* row_scale, int64_t M, int64_t K, void* stream);

/* ---------------------------------------------------------------------------------------
 * Symmetric block-32 int4 quantize + pack of a float matrix x[rows, K] (fp32/fp16/bf16):
 *   scale = max(amax(block), 1e-8) / 7      (rule 0, torch on CPU: ops.py:115-116)
 *   scale = max(amax(block), 1e-8) * (1/7)  (rule 1, torch on GPU and the reference's own
 *                                            kernel: csrc/int4_gemm_scaled.hip:210-211)
 *   code  = clamp(rint(x / scale), -8, 7), packed two per byte as above.
 * Replaces quantize_pack_int4 (ops.py:108-126) for device-resident weights, and
 * quantize_int4_dispatch (csrc/int4_gemm_scaled.hip:248-252) for activations.
 * ------------------------------------------------------------------------------------- */
int qlinear_quantize_int4(int x_dtype, int rule, const void* x, void* packed, float* scale,
                          int64_t rows, int64_t K, void* stream);

/* ---------------------------------------------------------------------------------------
 * Lossless ggml Q4_0 -> native layout of a weight [rows, K]: rows * K/32 blocks of 18 bytes
 * (fp16 d, then 16 bytes whose byte i holds elements i and i + 16 as offset-binary nibbles)
 * become w_q4 [rows, K/2] (two's-complement nibbles, element 2j in the low nibble of byte j)
 * and w_scale [rows, K/32] fp32 = d. Replaces repack_q4_0_native (ops.py:129-164) for
 * device-resident GGUF tensors. raw 2-byte aligned, packed 16-byte aligned.
 * ------------------------------------------------------------------------------------- */
int qlinear_repack_q4_0(const void* raw, int8_t* packed, float* scale, int64_t rows, int64_t K,
                        void* stream);

/* ---------------------------------------------------------------------------------------
 * Per-token int8 quantize of activations x[M,K] (fp32/fp16/bf16):
 *   s[m] = max(amax(row m), 1e-8) * (1/127); q = clamp(rint(x / s), -127, 127)
 * The reference's int8 rule (csrc/int8_gemm.hip:215-246, quantize_int8_dispatch :280) with
 * the block widened from 32 to the whole row.
 * ------------------------------------------------------------------------------------- */
int qlinear_quantize_int8_per_token(int x_dtype, const void* x, int8_t* q, float* scale,
                                    int64_t M, int64_t K, void* stream);

/* ---------------------------------------------------------------------------------------
 * W8A8 linear: acc[m,n] = sum_k xq[m,k] * wq[n,k] in int32 (exact), then
 *   y = float(acc) * (x_scale[m] * w_scale[n]) (+ bias[n]), each step rounded in fp32,
 * the scale-product order of csrc/int8_gemm.hip:191-193, 209. out_dtype QL_I32 stores the
 * raw accumulators (x_scale, w_scale and bias are then ignored). K % 64 == 0.
 * Counterpart of gemm_int8_dispatch (csrc/int8_gemm.hip:287-295) with per-token x
 * per-channel scales instead of block-32 scales.
 * ------------------------------------------------------------------------------------- */
int qlinear_w8a8_gemm(int out_dtype, const int8_t* xq, const float* x_scale, const int8_t* wq,
                      const float* w_scale, const void* bias, void* y, int64_t M, int64_t N,
                      int64_t K, void* stream);

/* ---------------------------------------------------------------------------------------
 * W4A4 linear with the reference's production numerics: a_q4 [M, K/2] (activations from
 * qlinear_quantize_int4, rule 1) and b_q4 [N, K/2] packed int4, scales a_scale [M, K/qblock],
 * b_scale [N, K/qblock] fp32, qblock 32 or 16. For each quant block in K order:
 *   ip = exact int32 dot of the block's codes; acc = fmaf(float(ip), a_scale * b_scale, acc)
 * then y = acc (+ bias) rounded once to out_dtype (bias of dtype out_dtype). splits > 1 (at most
 * 8): K is cut into ranges of ceil(k_tiles / splits) k-tiles of 128 K (k_tiles = ceil(K / 128)),
 * each range accumulates from 0 into an fp32 partial [M, N] in the workspace, and
 * y = ((0 + p_0) + p_1) + ... (+ bias) in split order. splits 0 = the reference's automatic
 * choice (qlinear_w4a4_auto_splits). Bit-identical to gemm_dispatch (csrc/int4_gemm_scaled.hip:
 * 254-269, kernel :53-191, split-K :182-191, 229-246) with the same splits. Counterpart of
 * ext.gemm_int4 (csrc/binding.cpp:70-112). workspace: qlinear_w4a4_workspace_bytes(...) bytes
 * (splits * M * N fp32 when splits > 1, else none). K % 32 == 0; a_q4, b_q4 16-byte aligned.
 * ------------------------------------------------------------------------------------- */
int qlinear_w4a4_gemm(int out_dtype, const void* a_q4, const float* a_scale, const void* b_q4,
                      const float* b_scale, const void* bias, void* y, int64_t M, int64_t N,
                      int64_t K, int qblock, int splits, void* workspace, size_t workspace_bytes,
                      void* stream);
/* The split count splits = 0 resolves to, the reference's auto_splits (csrc/binding.cpp:36-43,
 * gemm_int4_auto_splits :359-362) with this device's CU count: 1 when ceil(M/64) * ceil(N/64)
 * tiles fill 2 per CU, else min(ceil(12 * 2 CUs / (5 tiles)), 8, max(1, k_tiles / 8)). A
 * negative value is -status on bad arguments. */
int qlinear_w4a4_auto_splits(int64_t M, int64_t N, int64_t K, int device);
/* Workspace bytes of qlinear_w4a4_gemm for these arguments (0 when no split-K, or on bad
 * arguments). */
size_t qlinear_w4a4_workspace_bytes(int64_t M, int64_t N, int64_t K, int splits, int device);

/* ---------------------------------------------------------------------------------------
 * Block-32 int8, the reference's gemm_int8 / quantize_int8 (csrc/int8_gemm.hip:66-252,
 * gemm_int8_dispatch / quantize_int8_dispatch :280-295; ext.quantize_int8 / ext.gemm_int8,
 * csrc/binding.cpp:173-217):
 *   quantize: per 32 elements s = max(amax, 1e-8) * (1/127), q = clamp(rint(x / s), -127, 127)
 *             -> q int8 [rows, K], scale fp32 [rows, K/32]
 *   gemm:     per block in K order ip = exact int32 dot, acc = fmaf(float(ip), as * bs, acc);
 *             y = acc (+ bias, dtype out_dtype) rounded to out_dtype. Bit-identical to the
 *             reference's kernel (any of its tile configs: they share this order).
 * K % 32 == 0; x / q / a / b 16-byte aligned.
 * ------------------------------------------------------------------------------------- */
int qlinear_quantize_int8_block32(int x_dtype, const void* x, int8_t* q, float* scale, int64_t rows,
                                  int64_t K, void* stream);
int qlinear_gemm_int8_block32(int out_dtype, const int8_t* a, const float* a_scale, const int8_t* b,
                              const float* b_scale, const void* bias, void* y, int64_t M, int64_t N,
                              int64_t K, void* stream);

/* ---------------------------------------------------------------------------------------
 * Fused DiT block glue. No counterpart in the reference: its node patches only the Linears of
 * ComfyUI's Flux model (nodes/ComfyUI-Gfx906Int4/nodes.py:71-124, 447-599) and the layer norms,
 * modulation, QK-norm, RoPE and gated residuals run as separate torch ops around them. Each entry
 * point is one HBM pass, computes in fp32 and rounds once.
 * ------------------------------------------------------------------------------------- */
/* adaLN: y = LayerNorm(x[m, :]) (no affine, biased variance, eps) * (1 + scale) + shift, with
 * shift / scale [K] shared by all rows (one batch item), written as the fp16 operand of
 * qlinear_w4a16_gemm: x16 = y * 2^-e_m rounded to fp16, e_m such that max|y[m, :]| * 2^-e_m is in
 * [2^14, 2^15) (after the rounding, max|x16[m, :]| <= 2^15), row_scale[m] = 2^e_m
 * (pass both to qlinear_w4a16_gemm with x_dtype QL_F16). x fp32/fp16/bf16, shift/scale of
 * mod_dtype; K % 8 == 0, K <= 16384; x, shift, scale, x16 16-byte aligned. */
int qlinear_adaln_modulate_f16(int x_dtype, const void* x, int mod_dtype, const void* shift,
                               const void* scale, void* x16, float* row_scale, int64_t M,
                               int64_t K, float eps, void* stream);

/* The same adaLN row y written as out_kind says:
 *   QL_OPERAND_F16_ROWSCALED  as qlinear_adaln_modulate_f16 (out = x16 fp16, row_scale = 2^e_m);
 *   QL_OPERAND_PLAIN          y rounded to x's dtype, out [M, K] of that dtype (row_scale unused);
 *   QL_OPERAND_I8_PER_TOKEN   the W8A8 GEMM's operand: y rounded to x's dtype, then quantized as
 *                           qlinear_quantize_int8_per_token quantizes it (out int8 [M, K],
 *                           row_scale[m] = the token's scale) -- the PLAIN output followed by
 *                           that quantizer, bit for bit, without the round trip of the bf16 row
 *                           through HBM (the reference quantizes in a launch of its own,
 *                           ops.py:181, csrc/int8_gemm.hip:215-246).
 * out 16-byte aligned (8-byte for int8). */
#define QL_OPERAND_F16_ROWSCALED 0
#define QL_OPERAND_PLAIN 1
#define QL_OPERAND_I8_PER_TOKEN 2
int qlinear_adaln_modulate(int out_kind, int x_dtype, const void* x, int mod_dtype,
                           const void* shift, const void* scale, void* out, float* row_scale,
                           int64_t M, int64_t K, float eps, void* stream);

/* QK-norm + RoPE + head split of a qkv projection [L, 3, H, D] (q, k, v blocks of H heads):
 * q[h, l_offset + l, :] = rope(rmsnorm(q_in[l, h, :]) * q_norm), likewise k with k_norm,
 * v[h, l_offset + l, :] = v_in[l, h, :]; q, k, v are [H, L_out, D] (the attention layout), so
 * two calls with offsets 0 and L_txt assemble a joint text + image sequence. rmsnorm = x *
 * rsqrt(mean(x^2) + eps); rope rotates pairs (2j, 2j + 1) by cos/sin[l_offset + l, j] (fp32
 * [L_out, D/2]). dtype fp16/bf16 for qkv, norms and outputs; D == 128; 4-byte alignment. */
int qlinear_qk_norm_rope(int dtype, const void* qkv, const void* q_norm, const void* k_norm,
                         const float* cos_t, const float* sin_t, void* q, void* k, void* v,
                         int64_t L, int64_t H, int64_t D, int64_t L_out, int64_t l_offset,
                         float eps, void* stream);

/* Attention output to the next GEMM's operand: row l of x16 [rows, H * D + E] is the head-major
 * o[:, l_offset + l, :] ([H, L_all, D], the layout attention returns) flattened over heads,
 * followed by extra[l, :] ([rows, E], may be NULL with E == 0), written as qlinear_rows_to_f16
 * writes (row-scaled fp16, row_scale[l] = 2^e_l). dtype fp16/bf16 for o and extra; D == 128,
 * E % 8 == 0, H * D + E <= 16384; o, extra, x16 16-byte aligned. */
int qlinear_heads_to_f16(int dtype, const void* o, int64_t H, int64_t L_all, int64_t D,
                         int64_t l_offset, int64_t rows, const void* extra, int64_t E, void* x16,
                         float* row_scale, void* stream);

/* The same gathered row written as out_kind says (the QL_OPERAND_* kinds of
 * qlinear_adaln_modulate): QL_OPERAND_F16_ROWSCALED as qlinear_heads_to_f16; QL_OPERAND_PLAIN the
 * row in `dtype` ([rows, H * D + E], row_scale unused); QL_OPERAND_I8_PER_TOKEN the W8A8 operand,
 * the row quantized as qlinear_quantize_int8_per_token quantizes it (int8 out, row_scale[l] = the
 * token's scale) -- the producer of a W8A8 proj / linear2 writing its operand directly. out 16-byte
 * aligned (8-byte for int8). */
int qlinear_heads_gather(int out_kind, int dtype, const void* o, int64_t H, int64_t L_all,
                         int64_t D, int64_t l_offset, int64_t rows, const void* extra, int64_t E,
                         void* out, float* row_scale, void* stream);

/* Measurement: one read of `bytes` bytes of buf (a multiple of 16, 16-byte aligned) by one
 * workgroup per CU with 16-byte loads, folded to one xor word per workgroup into out (as many
 * uint32 as the device has CUs). The single-kernel HBM read floor the skinny-M W4A16 kernels
 * (which read their weights once per call) are measured against. No counterpart in the reference. */
int qlinear_stream_read(const void* buf, int64_t bytes, uint32_t* out, void* stream);

/* Gated residual: out[m, k] = x[m, k] + gate[k] * y[m, k]; out may be x (in place) but must
 * not overlap it otherwise; out, x, gate, y of one dtype (fp32/fp16/bf16), K % 8 == 0, 16-byte
 * aligned. */
int qlinear_gated_residual(int dtype, void* out, const void* x, const void* gate, const void* y,
                           int64_t M, int64_t K, void* stream);

/* ---------------------------------------------------------------------------------------
 * Host-only self-check of the launch plans (no GPU needed, nothing launched). No counterpart in
 * the reference. For op 0 (qlinear_w4a16_gemm, any x_dtype / splits / flags), 1
 * (qlinear_w8a8_gemm) or 2 (qlinear_w4a4_gemm with `splits` >= 1) and a CU count `cus`, walks
 * every workgroup of every launch the entry point would make through the kernels' own
 * workgroup -> tile mapping and returns QL_OK if every output tile (and every K piece or 128-row
 * half of one) is covered exactly once, every workgroup starts inside M x N (or is a 256 x 256
 * half wholly past M, which the kernel leaves before any memory access), and the workspace holds
 * every split-K partial; otherwise a status with the first violation in qlinear_last_error().
 * ------------------------------------------------------------------------------------- */
int qlinear_check_launch_plan(int op, int x_dtype, int64_t M, int64_t N, int64_t K, int splits,
                              int flags, int cus);
/* The plan qlinear_w4a16_gemm makes on a device with `cus` compute units, host only: info[0] =
 * kernel configuration (0-8), [1] / [2] = tile rows / columns, [3] = tiles run whole, [4] = tiles,
 * [5] = K pieces of each remaining tile, [6] = 1 when x is staged to fp16 first. No counterpart in
 * the reference (its tile shape is fixed). */
int qlinear_w4a16_describe_plan(int x_dtype, int64_t M, int64_t N, int64_t K, int splits, int flags,
                                int cus, int* info);

#ifdef __cplusplus
}
#endif

#endif /* QLINEAR_H */
