"""CPU oracle for the quantized-linear hot path -- TEST INFRASTRUCTURE ONLY.

This module restates, in numpy, the reference's arithmetic for the path that libqlinear.so
implements on gfx950. It is imported only by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, and only as the checker (or the timed CPU baseline), never as the product:
the product path (comfy_ui_gfx906_tools_amd) has no CPU fallback and never imports it.

Reference: luna-niemitalo/comfy_ui_gfx906_tools, paths relative to /root/reference.
Every function cites the file:line it follows and names the tests that pin it
(tests/test_oracle.py); none is "parity unpinned".
"""
from __future__ import annotations

import numpy as np

BLOCK = 32  # nodes/ComfyUI-Gfx906Int4/ops.py:196
F32_1E8 = np.float32(1e-8)
RECIP7 = np.float32(1.0) / np.float32(7.0)      # fl(1/7), the reference kernel's constant
RECIP127 = np.float32(1.0) / np.float32(127.0)  # fl(1/127)


# ---------------------------------------------------------------------------------------------
# 16-bit float helpers (numpy has fp16 but no bf16)
# ---------------------------------------------------------------------------------------------
def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16, returned as uint16 bit patterns; NaN stays NaN.
    Pinned by test_bf16_rounding_matches_torch."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(a)
    if nan.any():
        rounded = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), rounded)
    return rounded


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_to_bf16(a: np.ndarray) -> np.ndarray:
    """fp32 values rounded (RNE) to the nearest bf16, returned as fp32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(a))


def round_to_dtype(a: np.ndarray, dtype: str) -> np.ndarray:
    """Round fp32 values to 'float32' | 'float16' | 'bfloat16' (RNE), returned as fp32."""
    a = np.asarray(a, dtype=np.float32)
    if dtype == "float32":
        return a
    if dtype == "float16":
        return a.astype(np.float16).astype(np.float32)
    if dtype == "bfloat16":
        return round_to_bf16(a)
    raise ValueError(dtype)


# ---------------------------------------------------------------------------------------------
# int4 weight format
# ---------------------------------------------------------------------------------------------
def int4_scale(amax: np.ndarray, rule: str = "div") -> np.ndarray:
    """Group scale from the group's absolute maximum.
    rule 'div':   clamp_min(amax, 1e-8) / 7.0        -- ops.py:115-116 evaluated by torch on CPU
                                                      (IEEE division)
    rule 'recip': max(amax, 1e-8) * fl(1/7)          -- int4_gemm_scaled.hip:210-211 (and torch's
                                                      scalar-divisor path on GPU, per that
                                                      comment)
    Pinned by test_int4_scale_rules (exact rational arithmetic)."""
    amax = np.maximum(np.asarray(amax, dtype=np.float32), F32_1E8)
    if rule == "div":
        return (amax / np.float32(7.0)).astype(np.float32)
    if rule == "recip":
        return (amax * RECIP7).astype(np.float32)
    raise ValueError(rule)


def quantize_pack_int4(t: np.ndarray, block: int = BLOCK, rule: str = "div"):
    """ops.py:108-126. t [..., K] float -> (packed int8 [..., K/2], scale fp32 [..., K/block]).
    codes = clamp(round_half_even(t / scale), -8, 7); byte j = code[2j] & 0xF | (code[2j+1] & 0xF) << 4.
    Pinned by test_pack_layout_hand_bytes, test_quantize_exact_grid, test_round_half_even_ties,
    test_zero_block, test_int4_scale_rules."""
    t = np.asarray(t, dtype=np.float32)
    K = t.shape[-1]
    assert K % block == 0, f"last dim {K} not divisible by block {block}"
    rows = t.shape[:-1]
    tb = t.reshape(-1, K // block, block)
    amax = np.abs(tb).max(axis=-1, keepdims=True)
    scale = int4_scale(amax, rule)
    codes = np.clip(np.rint(tb / scale), -8, 7).astype(np.int32).reshape(-1, K)
    lo = codes[:, 0::2] & 0xF
    hi = codes[:, 1::2] & 0xF
    packed = (lo | (hi << 4)).astype(np.uint8).view(np.int8)
    return packed.reshape(*rows, K // 2), scale.reshape(*rows, K // block).astype(np.float32)


def unpack_int4(packed: np.ndarray) -> np.ndarray:
    """Inverse of the packing above: int8 [..., K/2] -> int8 codes [..., K] in [-8, 7]
    (two's-complement nibbles; low nibble first). Pinned by test_unpack_matches_reference_decode
    (the reference's own dword decode, int4_train_test.py:46-52) and the hand-byte test."""
    b = np.asarray(packed).view(np.uint8)
    lo = (b & 0xF).astype(np.int16)
    hi = (b >> 4).astype(np.int16)
    codes = np.stack([lo, hi], axis=-1).reshape(*b.shape[:-1], b.shape[-1] * 2)
    return np.where(codes > 7, codes - 16, codes).astype(np.int8)


def dequant_int4(packed: np.ndarray, scale: np.ndarray, block: int = BLOCK) -> np.ndarray:
    """codes * scale (repeated over each block), fp32: the exact product of a 4-bit integer and an
    fp32 scale rounded once to fp32 (nodes.py:51-52, `q * scale`)."""
    codes = unpack_int4(packed).astype(np.float32)
    s = np.repeat(np.asarray(scale, dtype=np.float32), block, axis=-1)
    return (codes * s).astype(np.float32)


def quantize_dequantize_int4(t: np.ndarray, block: int = BLOCK, rule: str = "div") -> np.ndarray:
    """nodes.py:43-52 (Gfx906Int4Patch's w4a16 fake-quant): RTN int4 then back to float32.
    Rows whose K is not a multiple of block are returned unchanged (nodes.py:46-47)."""
    t = np.asarray(t, dtype=np.float32)
    if t.shape[-1] % block:
        return t
    p, s = quantize_pack_int4(t, block, rule)
    return dequant_int4(p, s, block).reshape(t.shape)


def w4a16_reference(x: np.ndarray, packed: np.ndarray, scale: np.ndarray, bias: np.ndarray | None = None,
                    block: int = BLOCK) -> np.ndarray:
    """The W4A16 parity target: y = x.float() @ dequant(W)^T (+ bias), nodes.py:43-52 + 116
    followed by the stock matmul. Accumulated in float64 so the oracle's own rounding is far
    below the kernel's. Pinned by test_w4a16_reference_bruteforce, test_w4a16_exact_on_grid,
    test_w4a16_linearity."""
    xf = np.asarray(x, dtype=np.float32).astype(np.float64)
    w = dequant_int4(packed, scale, block).astype(np.float64)
    y = xf @ w.T
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float32).astype(np.float64)
    return y


# ---------------------------------------------------------------------------------------------
# ggml Q4_0 -> native repack
# ---------------------------------------------------------------------------------------------
Q4_0_TYPE_SIZE = 18


def ggml_q4_0_dequant(raw: np.ndarray, out_features: int, in_features: int) -> np.ndarray:
    """The ggml Q4_0 block definition: 18 bytes = fp16 d + 16 bytes qs;
    x[i] = d * ((qs[i] & 0xF) - 8), x[i + 16] = d * ((qs[i] >> 4) - 8), i < 16.
    The product is formed in fp32 from the fp16 d. Used to pin repack_q4_0_native."""
    blocks = np.asarray(raw).view(np.uint8).reshape(-1, Q4_0_TYPE_SIZE)
    d = blocks[:, :2].copy().view(np.float16).astype(np.float32).reshape(-1, 1)
    qs = blocks[:, 2:].astype(np.int32)
    vals = np.concatenate([(qs & 0xF) - 8, (qs >> 4) - 8], axis=1).astype(np.float32)
    return (vals * d).reshape(out_features, in_features)


def repack_q4_0_native(raw: np.ndarray, out_features: int, in_features: int, block: int = BLOCK):
    """ops.py:129-164: lossless ggml Q4_0 -> native layout. Offset-binary nibbles (q - 8 stored
    as q) become two's complement ((n - 8) & 0xF); the split-half element order of a Q4_0 block
    (byte i = elem i | elem i+16 << 4) becomes interleaved (byte j = elem 2j | elem 2j+1 << 4);
    the fp16 d becomes an fp32 scale. Pinned by test_q4_0_repack_* (ggml definition)."""
    n_blocks = in_features // block
    blocks = np.asarray(raw).view(np.uint8).reshape(out_features * n_blocks, Q4_0_TYPE_SIZE)
    scale = blocks[:, :2].copy().view(np.float16).astype(np.float32).reshape(out_features, n_blocks)
    qs = blocks[:, 2:].astype(np.int32)
    lo = ((qs & 0xF) - 8) & 0xF
    hi = (((qs >> 4) & 0xF) - 8) & 0xF
    elems = np.concatenate([lo, hi], axis=1)  # element order 0..31 of each block
    packed = (elems[:, 0::2] | (elems[:, 1::2] << 4)).astype(np.uint8).view(np.int8)
    return packed.reshape(out_features, in_features // 2), scale


# ---------------------------------------------------------------------------------------------
# Hadamard group rotation
# ---------------------------------------------------------------------------------------------
def hadamard(n: int) -> np.ndarray:
    """ops.py:43-51: Sylvester construction H_{2k} = [[H, H], [H, -H]], scaled by 1/sqrt(n).
    Pinned by test_hadamard_* (orthonormal, symmetric, +-1/sqrt(n) entries, scipy)."""
    assert n & (n - 1) == 0, f"Hadamard order {n} must be a power of two"
    h = np.ones((1, 1), dtype=np.float32)
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return (h / np.float32(n ** 0.5)).astype(np.float32)


def choose_rotation_group(in_features: int, max_group: int = 128, min_group: int = 32):
    """ops.py:54-65: largest power of two <= max_group dividing in_features, or None."""
    g = max_group
    while g >= min_group:
        if in_features % g == 0:
            return g
        g //= 2
    return None


def group_rotation(signs: np.ndarray) -> np.ndarray:
    """ops.py:68-82: R = H * signs (column scaling), signs in {-1, +1}. The signs come from
    torch's CPU generator seeded with 0 ^ group (ops.py:79-80); tests load them from the
    fixture tests/golden/rotation_signs.npz made by that exact call."""
    g = signs.shape[0]
    return (hadamard(g) * signs.astype(np.float32)[None, :]).astype(np.float32)


def apply_group_rotation(t: np.ndarray, R: np.ndarray) -> np.ndarray:
    """ops.py:85-105: every group-sized chunk of the last dim, as a row vector v, becomes v @ R^T."""
    g = R.shape[0]
    flat = np.asarray(t, dtype=np.float32).reshape(-1, g)
    return (flat.astype(np.float64) @ R.T.astype(np.float64)).astype(np.float32).reshape(t.shape)


# ---------------------------------------------------------------------------------------------
# int8
# ---------------------------------------------------------------------------------------------
def quantize_int8_rows(x: np.ndarray, block: int | None = None):
    """int8_gemm.hip:215-246 with the block widened to `block` (None = the whole row, the
    per-token variant): s = max(amax, 1e-8) * fl(1/127); q = clamp(rint(x / s), -127, 127).
    Returns (int8 q like x, fp32 s [rows] (per-token) or [rows, K/block]).
    Pinned by test_int8_quantizer_*."""
    x = np.asarray(x, dtype=np.float32)
    M, K = x.shape
    blk = K if block is None else block
    xb = x.reshape(M, K // blk, blk)
    amax = np.abs(xb).max(axis=-1, keepdims=True)
    s = (np.maximum(amax, F32_1E8) * RECIP127).astype(np.float32)
    q = np.clip(np.rint(xb / s), -127, 127).astype(np.int8).reshape(M, K)
    s = s.reshape(M, K // blk)
    return q, (s[:, 0] if block is None else s)


def int8_matmul_exact(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """sum_k a[m,k] * b[n,k] in int64 (exact). The W8A8 int32 accumulator must equal this."""
    return np.asarray(a, dtype=np.int64) @ np.asarray(b, dtype=np.int64).T


def int8_matmul_exact_f64(a: np.ndarray, b: np.ndarray, chunk: int = 512) -> np.ndarray:
    """int8_matmul_exact through float64 BLAS (all the host's cores): int8 codes are exact in
    float64 and every partial sum of K products stays below 127 * 128 * K < 2^53 for K < 2^38, so
    each product and sum is exact and the result equals the int64 matmul. Rows in chunks to bound
    the float64 copies. Returns int64."""
    a = np.asarray(a)
    bt = np.asarray(b, dtype=np.float64).T
    if a.shape[1] >= (1 << 38):
        raise ValueError("K too large for an exact float64 accumulation")
    out = np.empty((a.shape[0], bt.shape[1]), dtype=np.int64)
    for r in range(0, a.shape[0], chunk):
        out[r:r + chunk] = (a[r:r + chunk].astype(np.float64) @ bt).astype(np.int64)
    return out


def w8a8_epilogue(acc: np.ndarray, sx: np.ndarray, sw: np.ndarray, bias: np.ndarray | None = None) -> np.ndarray:
    """float(acc) * (sx[m] * sw[n]) (+ bias[n]), each operation rounded in fp32 -- the order of
    int8_gemm.hip:191-193 (fmaf(float(ip), as * bs, 0)) and :209 (v += bias). Returns fp32."""
    f = np.asarray(acc, dtype=np.int64).astype(np.float32)
    p = (np.asarray(sx, dtype=np.float32)[:, None] * np.asarray(sw, dtype=np.float32)[None, :]).astype(np.float32)
    y = (f * p).astype(np.float32)
    if bias is not None:
        y = (y + np.asarray(bias, dtype=np.float32)[None, :]).astype(np.float32)
    return y


def gemm_int8_block32(aq, as_, bq, bs, bias=None, block: int = 32) -> np.ndarray:
    """int8_gemm.hip:66-213: per 32-block int32 partial, then acc = fmaf(float(ip), as*bs, acc)
    in K order, + bias. fmaf is emulated exactly: the product of an int (< 2^24 in magnitude) and
    an fp32 is exact in float64, and the sum is rounded once via a float64 two-sum correction."""
    aq = np.asarray(aq, dtype=np.int64)
    bq = np.asarray(bq, dtype=np.int64)
    M, K = aq.shape
    N = bq.shape[0]
    acc = np.zeros((M, N), dtype=np.float32)
    for kb in range(K // block):
        ip = aq[:, kb * block:(kb + 1) * block] @ bq[:, kb * block:(kb + 1) * block].T
        sc = (np.asarray(as_, np.float32)[:, kb][:, None] * np.asarray(bs, np.float32)[:, kb][None, :]).astype(np.float32)
        acc = fmaf32(ip.astype(np.float32), sc, acc)
    if bias is not None:
        acc = (acc + np.asarray(bias, dtype=np.float32)[None, :]).astype(np.float32)
    return acc


def fmaf32(a: np.ndarray, b: np.ndarray, c: np.ndarray) -> np.ndarray:
    """Correctly rounded fp32 fused multiply-add of fp32 inputs (C fmaf). a*b is exact in float64
    (24 + 24 bits). s = RN64(a*b + c) rounds to the same fp32 as the exact sum unless s sits
    exactly on an fp32 midpoint; then the TwoSum error term e = (a*b + c) - s decides the side.
    Pinned by test_fmaf32_matches_fractions."""
    a, b, c = np.broadcast_arrays(np.asarray(a, np.float32), np.asarray(b, np.float32), np.asarray(c, np.float32))
    p = a.astype(np.float64) * b.astype(np.float64)
    c64 = c.astype(np.float64)
    s = p + c64
    bb = s - p
    e = (p - (s - bb)) + (c64 - bb)
    r = s.astype(np.float32)
    r64 = r.astype(np.float64)
    with np.errstate(invalid="ignore"):
        toward = np.where(s > r64, np.float32(np.inf), np.float32(-np.inf)).astype(np.float32)
        n = np.nextafter(r, toward)
        mid = (r64 + n.astype(np.float64)) / 2
        tie = np.isfinite(s) & (s != r64) & (s == mid)
    if tie.any():
        up = e > 0
        down = e < 0
        hi = np.maximum(r, n)
        lo = np.minimum(r, n)
        r = np.where(tie & up, hi, np.where(tie & down, lo, r)).astype(np.float32)
    return r


# ---------------------------------------------------------------------------------------------
# W4A4 (the reference's production numerics): block-32 int4 activations x int4 weights
# ---------------------------------------------------------------------------------------------
def gemm_int4_w4a4(a_packed, a_scale, b_packed, b_scale, bias=None, block: int = 32, splits: int = 1) -> np.ndarray:
    """int4_gemm_scaled.hip:53-180 (SUB=1): per 32-block int32 dot of the signed nibbles, then
    acc = fmaf(float(ip), as*bs, acc) in K order, + bias (fp32 result). splits > 1: the split-K
    association of gemm_split_k below."""
    a = unpack_int4(a_packed).astype(np.int64)
    b = unpack_int4(b_packed).astype(np.int64)
    if splits > 1:
        return gemm_split_k(a, a_scale, b, b_scale, bias, block, splits)
    return gemm_int8_block32(a, a_scale, b, b_scale, bias, block)


def gemm_split_k(aq, as_, bq, bs, bias, block: int, splits: int) -> np.ndarray:
    """The reference's split-K gemm_int4 (int4_gemm_scaled.hip:229-246 launch, :123-129 K range,
    :182-191 reduce): K is cut into k-tiles of 4 loads of 32 codes (128 K); split s takes k-tiles
    [s t, min(k_tiles, (s + 1) t)) with t = ceil(k_tiles / splits) (possibly none), accumulates
    its blocks from 0 in K order exactly as the unsplit kernel, and the partials are summed in
    fp32 as v = ((0 + p_0) + p_1) + ..., then + bias. Pinned by test_split_k_* (tests/test_oracle.py)."""
    aq = np.asarray(aq, dtype=np.int64)
    bq = np.asarray(bq, dtype=np.int64)
    M, K = aq.shape
    N = bq.shape[0]
    k_tiles = (K // 32 + 3) // 4
    per = (k_tiles + splits - 1) // splits
    v = np.zeros((M, N), dtype=np.float32)
    for s in range(splits):
        k_lo = min(K, s * per * 128)
        k_hi = min(K, (s + 1) * per * 128)
        if k_hi > k_lo:
            sl = slice(k_lo // block, k_hi // block)
            part = gemm_int8_block32(aq[:, k_lo:k_hi], np.asarray(as_)[:, sl], bq[:, k_lo:k_hi], np.asarray(bs)[:, sl],
                                     None, block)
        else:
            part = np.zeros((M, N), dtype=np.float32)
        v = (v + part).astype(np.float32)
    if bias is not None:
        v = (v + np.asarray(bias, dtype=np.float32)[None, :]).astype(np.float32)
    return v


def reference_auto_splits(M: int, N: int, K: int, cus: int) -> int:
    """binding.cpp:21-43 auto_splits (gemm_tiles / gemm_k_tiles of int4_gemm_scaled.hip:271-272):
    64 x 64 tiles; none when they fill 2 workgroups per CU, else ceil(12 slots / (5 tiles)) capped at
    8 and at k_tiles / 8 (at least 1). Pinned by test_reference_auto_splits (the reference's own sweep
    notes, binding.cpp:31-35)."""
    tiles = ((M + 63) // 64) * ((N + 63) // 64)
    slots = cus * 2
    if tiles >= slots or tiles == 0:
        return 1
    max_splits = min(8, max(1, ((K // 32 + 3) // 4) // 8))
    wanted = (12 * slots + 5 * tiles - 1) // (5 * tiles)
    return min(wanted, max_splits)
