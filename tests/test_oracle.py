"""Pins the CPU oracle (oracle/qlinear_oracle.py) on the CPU: closed forms, exact rational
arithmetic, brute force on tiny inputs, the format definitions (ggml Q4_0, two's-complement
nibbles), library routines (torch's bf16 cast, scipy's Hadamard) and the committed fixtures.
Each check is chosen so that a plausible mistake in the oracle (a dropped term, a swapped nibble,
a wrong rounding rule, a transposed operand) fails it. No GPU needed."""
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import qlinear_oracle as orc
from tests.conftest import golden_path


# ---- exact-rounding helpers (independent of the oracle) ------------------------------------
def _f32_nearest(q: Fraction) -> np.float32:
    """Correctly rounded (RNE) fp32 of an exact rational, by bracketing."""
    r = np.float32(float(q))  # float() of a Fraction is correctly rounded to float64
    cands = {r, np.nextafter(r, np.float32(np.inf)), np.nextafter(r, np.float32(-np.inf))}
    best = None
    for c in sorted(cands):
        d = abs(Fraction(float(c)) - q)
        if best is None or d < best[0] or (d == best[0] and (int(c.view(np.uint32)) & 1) == 0):
            best = (d, c)
    return np.float32(best[1])


def _decode_dwords(packed: np.ndarray) -> np.ndarray:
    """The reference test's decode (develop/experiments/2026-10-11/int4_train_test.py:46-52):
    view the bytes as little-endian int32 words; element e of a word is bits 4e..4e+3,
    sign-extended as a 4-bit two's-complement value. Written here with arithmetic shifts."""
    words = np.ascontiguousarray(packed).view(np.int32)
    out = np.empty(words.shape + (8,), dtype=np.int32)
    for e in range(8):
        out[..., e] = (words << (28 - 4 * e)) >> 28  # arithmetic shift sign-extends the nibble
    return out.reshape(packed.shape[0], -1)


# ---- 16-bit helpers ------------------------------------------------------------------------
def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2**32, 200_000, dtype=np.uint64).astype(np.uint32)
    # add exact ties (low half 0x8000) with odd and even kept halves, subnormals, inf, max
    ties = (rng.integers(0, 2**16, 5000, dtype=np.uint64).astype(np.uint32) << 16) | 0x8000
    special = np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x7F7FFFFF, 0x00000001, 0x007FFFFF,
                        0x3F808000, 0x3F818000, 0x7F7F8000], dtype=np.uint32)
    a = np.concatenate([bits, ties, special]).view(np.float32)
    a = a[~np.isnan(a)]
    ours = orc.f32_to_bf16_bits(a)
    theirs = torch.from_numpy(a.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)
    assert np.isnan(orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(np.array([np.nan], np.float32)))).all()


def test_round_to_dtype_float16_and_float32():
    a = np.array([1.0 + 2**-11, 1.0 + 3 * 2**-11, 65504.0, 1e-8], np.float32)
    assert np.array_equal(orc.round_to_dtype(a, "float16"), np.array([1.0, 1.0 + 2**-9, 65504.0, 0.0], np.float32))
    assert orc.round_to_dtype(a, "float32") is not None and np.array_equal(orc.round_to_dtype(a, "float32"), a)
    with pytest.raises(ValueError):
        orc.round_to_dtype(a, "int8")


# ---- int4 scale rules ------------------------------------------------------------------------
def test_int4_scale_rules():
    rng = np.random.default_rng(1)
    amax = np.concatenate([np.abs(rng.standard_normal(3000).astype(np.float32)) * 0.05,
                           np.array([0.0, 1e-9, 7.0, 1.0, 3.0e38], np.float32)])
    div = orc.int4_scale(amax, "div")
    rec = orc.int4_scale(amax, "recip")
    r7 = _f32_nearest(Fraction(1, 7))
    assert orc.RECIP7 == r7
    for a, d, r in zip(amax, div, rec):
        a = max(Fraction(float(a)), Fraction(float(np.float32(1e-8))))
        assert d == _f32_nearest(a / 7), (a, d)
        assert r == _f32_nearest(a * Fraction(float(r7))), (a, r)
    # the rules are distinct on ordinary data (so tests can tell which one a kernel uses)
    assert (div != rec).sum() > 100
    with pytest.raises(ValueError):
        orc.int4_scale(amax, "other")


# ---- int4 pack / unpack ----------------------------------------------------------------------
def test_pack_layout_hand_bytes():
    # amax 7 -> scale exactly 1 (7/7), so codes are the values themselves
    t = np.zeros((1, 32), np.float32)
    t[0, :6] = [1, -1, 7, -7, 0, 3]
    t[0, 31] = -2
    packed, scale = orc.quantize_pack_int4(t)
    assert scale.tolist() == [[1.0]]
    b = packed.view(np.uint8)[0]
    # byte j = code[2j] & 0xF | (code[2j+1] & 0xF) << 4
    assert b[0] == (1 | (0xF << 4))        # 1, -1
    assert b[1] == (7 | (0x9 << 4))        # 7, -7
    assert b[2] == (0 | (3 << 4))          # 0, 3
    assert b[15] == (0 | (0xE << 4))       # 0, -2
    assert packed.dtype == np.int8 and packed.shape == (1, 16)
    assert np.array_equal(orc.unpack_int4(packed)[0], t[0].astype(np.int8))


def test_unpack_matches_reference_decode():
    rng = np.random.default_rng(2)
    raw = rng.integers(-128, 128, (7, 48), dtype=np.int16).astype(np.int8)  # K = 96
    assert np.array_equal(orc.unpack_int4(raw).astype(np.int32), _decode_dwords(raw))
    # every byte value decodes to the pair of signed nibbles
    allb = np.arange(256, dtype=np.uint8).view(np.int8).reshape(1, 256)
    u = orc.unpack_int4(allb)[0].astype(int)
    for v in range(256):
        lo, hi = v & 0xF, v >> 4
        assert u[2 * v] == (lo - 16 if lo > 7 else lo) and u[2 * v + 1] == (hi - 16 if hi > 7 else hi)


def test_quantize_exact_grid():
    rng = np.random.default_rng(3)
    codes = rng.integers(-7, 8, (5, 128)).astype(np.int32)
    codes[:, ::32] = 7  # amax of every group = 7 * s exactly
    s = (2.0 ** rng.integers(-12, 0, (5, 4))).astype(np.float32)
    t = (codes.reshape(5, 4, 32) * s[..., None]).reshape(5, 128).astype(np.float32)
    for rule in ("div", "recip"):
        packed, scale = orc.quantize_pack_int4(t, rule=rule)
        if rule == "div":
            assert np.array_equal(scale, s)
        assert np.array_equal(orc.unpack_int4(packed).astype(np.int32), codes)
    assert np.array_equal(orc.dequant_int4(*orc.quantize_pack_int4(t)), t)


def test_round_half_even_ties():
    t = np.zeros((1, 32), np.float32)
    t[0, :8] = [7, 0.5, 1.5, 2.5, -0.5, -2.5, 3.5, -6.5]
    packed, _ = orc.quantize_pack_int4(t)
    assert orc.unpack_int4(packed)[0, :8].tolist() == [7, 0, 2, 2, 0, -2, 4, -6]


def test_zero_block():
    t = np.zeros((2, 64), np.float32)
    t[1, 32:] = 0.25
    packed, scale = orc.quantize_pack_int4(t)
    assert scale[0, 0] == _f32_nearest(Fraction(float(np.float32(1e-8))) / 7)
    assert scale[0, 1] == scale[0, 0] and scale[1, 0] == scale[0, 0]
    assert not orc.unpack_int4(packed)[0].any()
    assert (orc.unpack_int4(packed)[1, 32:] == 7).all()


def test_quantize_general_vs_bruteforce():
    """Random weights against a per-element Fraction computation of the reference rule."""
    rng = np.random.default_rng(4)
    t = (rng.standard_normal((3, 64)) * 0.02).astype(np.float32)
    packed, scale = orc.quantize_pack_int4(t)
    codes = orc.unpack_int4(packed)
    for r in range(3):
        for gi in range(2):
            blk = t[r, 32 * gi: 32 * gi + 32]
            s = _f32_nearest(Fraction(float(np.abs(blk).max())) / 7)
            assert scale[r, gi] == s
            for k in range(32):
                q = np.float32(blk[k]) / s  # IEEE fp32 division, as torch's t / scale
                c = int(np.clip(np.rint(q), -8, 7))
                assert codes[r, 32 * gi + k] == c
    # the -8 code never arises from round-to-nearest of |v/s| <= 7
    assert codes.min() >= -7


def test_quantize_dequantize_ragged_passthrough():
    t = np.ones((2, 40), np.float32)
    assert orc.quantize_dequantize_int4(t) is not None and np.array_equal(orc.quantize_dequantize_int4(t), t)
    t2 = np.linspace(-1, 1, 64, dtype=np.float32).reshape(1, 64)
    p, s = orc.quantize_pack_int4(t2)
    assert np.array_equal(orc.quantize_dequantize_int4(t2), orc.dequant_int4(p, s))


# ---- W4A16 reference ---------------------------------------------------------------------
def test_w4a16_reference_bruteforce():
    rng = np.random.default_rng(5)
    M, N, K = 3, 4, 64
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    packed, scale = orc.quantize_pack_int4(w)
    codes = orc.unpack_int4(packed)
    y = orc.w4a16_reference(x, packed, scale, bias)
    for m in range(M):
        for n in range(N):
            acc = Fraction(0)
            for k in range(K):
                wv = Fraction(float(np.float32(codes[n, k]) * scale[n, k // 32]))  # one fp32 rounding
                acc += Fraction(float(x[m, k])) * wv
            acc += Fraction(float(bias[n]))
            assert abs(float(acc) - y[m, n]) <= 1e-12 * max(1.0, abs(float(acc)))
    # operands are not transposed: a rank-one check
    assert y.shape == (M, N)


def test_w4a16_exact_on_grid():
    rng = np.random.default_rng(6)
    M, N, K = 5, 6, 96
    x = rng.integers(-4, 5, (M, K)).astype(np.float32)
    codes = rng.integers(-8, 8, (N, K))
    s = np.full((N, K // 32), 0.5, np.float32)
    packed = ((codes[:, 0::2] & 0xF) | ((codes[:, 1::2] & 0xF) << 4)).astype(np.uint8).view(np.int8)
    y = orc.w4a16_reference(x, packed, s)
    assert np.array_equal(y, (x.astype(np.int64) @ codes.T.astype(np.int64)) * 0.5)


def test_w4a16_linearity():
    rng = np.random.default_rng(7)
    # dyadic inputs, so 2*x1 + x2 is exact in fp32 and only the oracle's own arithmetic is tested
    x1 = (rng.integers(-2048, 2048, (4, 64)) / 1024).astype(np.float32)
    x2 = (rng.integers(-2048, 2048, (4, 64)) / 1024).astype(np.float32)
    p, s = orc.quantize_pack_int4((rng.standard_normal((8, 64)) * 0.1).astype(np.float32))
    lhs = orc.w4a16_reference(2 * x1 + x2, p, s)
    rhs = 2 * orc.w4a16_reference(x1, p, s) + orc.w4a16_reference(x2, p, s)
    assert np.allclose(lhs, rhs, rtol=0, atol=1e-9)


# ---- ggml Q4_0 repack --------------------------------------------------------------------------
def _q4_0_blocks(rng, n):
    d = (rng.standard_normal(n) * 0.01).astype(np.float16)
    qs = rng.integers(0, 256, (n, 16), dtype=np.uint16).astype(np.uint8)
    raw = np.concatenate([d.view(np.uint8).reshape(n, 2), qs], axis=1)
    return raw, d, qs


def test_q4_0_repack_hand_block():
    # one block: d = 0.5, qs[i] = (i | (15 - i) << 4): elem i = i - 8, elem i+16 = 7 - i
    qs = np.array([i | ((15 - i) << 4) for i in range(16)], np.uint8)
    raw = np.concatenate([np.array([0.5], np.float16).view(np.uint8), qs])[None, :]
    x = orc.ggml_q4_0_dequant(raw, 1, 32)[0]
    assert x.tolist() == [0.5 * (i - 8) for i in range(16)] + [0.5 * (7 - i) for i in range(16)]
    packed, scale = orc.repack_q4_0_native(raw, 1, 32)
    assert scale.tolist() == [[0.5]]
    assert orc.unpack_int4(packed)[0].tolist() == [i - 8 for i in range(16)] + [7 - i for i in range(16)]
    # the -8 code survives the repack (elem 0 = 0 - 8)
    assert packed.view(np.uint8)[0, 0] & 0xF == 0x8


def test_q4_0_repack_lossless_random():
    rng = np.random.default_rng(8)
    out_f, in_f = 6, 128
    raw, _, _ = _q4_0_blocks(rng, out_f * in_f // 32)
    packed, scale = orc.repack_q4_0_native(raw, out_f, in_f)
    assert packed.shape == (out_f, in_f // 2) and scale.shape == (out_f, in_f // 32)
    assert np.array_equal(orc.dequant_int4(packed, scale), orc.ggml_q4_0_dequant(raw, out_f, in_f))


# ---- Hadamard rotation -------------------------------------------------------------------------
@pytest.mark.parametrize("n", [1, 2, 32, 128])
def test_hadamard_properties(n):
    import scipy.linalg
    h = orc.hadamard(n)
    assert np.allclose(h @ h.T, np.eye(n), atol=1e-6)
    assert np.array_equal(h, h.T)
    assert np.allclose(np.abs(h), 1 / np.sqrt(n))
    assert np.allclose(h * np.sqrt(n), scipy.linalg.hadamard(n))


def test_choose_rotation_group():
    assert orc.choose_rotation_group(3072) == 128
    assert orc.choose_rotation_group(12288) == 128
    assert orc.choose_rotation_group(96) == 32
    assert orc.choose_rotation_group(64) == 64
    assert orc.choose_rotation_group(48) is None
    assert orc.choose_rotation_group(3072, max_group=64) == 64


def test_rotation_signs_fixture_and_orthogonality():
    f = np.load(golden_path("rotation_signs.npz"))
    for g in (32, 64, 128):
        signs = f[f"signs_{g}"]
        gen = torch.Generator(device="cpu").manual_seed(0 ^ g)
        assert np.array_equal(signs, (torch.randint(0, 2, (g,), generator=gen).float() * 2 - 1).numpy())
        R = orc.group_rotation(signs)
        assert np.allclose(R @ R.T, np.eye(g), atol=1e-6)
        assert np.allclose(R, orc.hadamard(g) @ np.diag(signs))


def test_apply_group_rotation_block_diagonal():
    rng = np.random.default_rng(9)
    signs = np.where(rng.random(32) < 0.5, -1.0, 1.0)
    R = orc.group_rotation(signs)
    t = rng.standard_normal((3, 96)).astype(np.float32)
    got = orc.apply_group_rotation(t, R)
    big = np.kron(np.eye(3), R.astype(np.float64))  # block-diagonal rotation of each row
    assert np.allclose(got, (t.astype(np.float64) @ big.T).astype(np.float32), atol=1e-6)
    # folding R into W and rotating x leaves x @ W^T unchanged: (x R^T)(W R^T)^T = x W^T
    w = rng.standard_normal((5, 96)).astype(np.float32)
    assert np.allclose(got @ orc.apply_group_rotation(w, R).T, t @ w.T, atol=1e-4)


# ---- int8 ------------------------------------------------------------------------------------------
def test_int8_quantizer_closed_form():
    x = np.zeros((3, 64), np.float32)
    x[0, :4] = [127.0, 0.5, -63.5, 1.5]  # amax 127: s = fl(127 * fl(1/127))
    x[2, 7] = -2.0
    q, s = orc.quantize_int8_rows(x)
    r127 = _f32_nearest(Fraction(1, 127))
    assert orc.RECIP127 == r127
    assert s[0] == _f32_nearest(Fraction(127) * Fraction(float(r127)))
    assert s[1] == _f32_nearest(Fraction(float(np.float32(1e-8))) * Fraction(float(r127)))
    assert not q[1].any()
    assert q[2, 7] == -127 and s[2] == _f32_nearest(Fraction(2) * Fraction(float(r127)))
    for k in range(4):
        assert q[0, k] == int(np.rint(np.float32(x[0, k]) / s[0]))


def test_int8_quantizer_blocked_and_bounds():
    rng = np.random.default_rng(10)
    x = (rng.standard_normal((4, 96)) * 3).astype(np.float32)
    q, s = orc.quantize_int8_rows(x, block=32)
    assert s.shape == (4, 3) and q.dtype == np.int8 and np.abs(q.astype(int)).max() == 127
    for b in range(3):
        q2, s2 = orc.quantize_int8_rows(np.ascontiguousarray(x[:, 32 * b:32 * b + 32]))
        assert np.array_equal(q2, q[:, 32 * b:32 * b + 32]) and np.array_equal(s2, s[:, b])


def test_int8_matmul_exact_bruteforce():
    rng = np.random.default_rng(11)
    a = rng.integers(-127, 128, (3, 70), dtype=np.int16).astype(np.int8)
    b = rng.integers(-127, 128, (5, 70), dtype=np.int16).astype(np.int8)
    got = orc.int8_matmul_exact(a, b)
    for m in range(3):
        for n in range(5):
            assert got[m, n] == sum(int(a[m, k]) * int(b[n, k]) for k in range(70))
    big = np.full((1, 12288), -127, np.int8)
    assert orc.int8_matmul_exact(big, big)[0, 0] == 12288 * 127 * 127


def test_int8_matmul_exact_f64_equals_int64():
    """The float64-BLAS form is exact: equal to the int64 matmul (itself pinned by brute force
    above) on random codes, on the extreme codes at large K, and across its row chunks."""
    rng = np.random.default_rng(13)
    a = rng.integers(-128, 128, (70, 3072), dtype=np.int16).astype(np.int8)
    b = rng.integers(-128, 128, (33, 3072), dtype=np.int16).astype(np.int8)
    assert np.array_equal(orc.int8_matmul_exact_f64(a, b, chunk=16), orc.int8_matmul_exact(a, b))
    big = np.full((2, 65536), -128, np.int8)
    got = orc.int8_matmul_exact_f64(big, big)
    assert got.dtype == np.int64 and got[1, 1] == 65536 * 128 * 128


def test_w8a8_epilogue_rounding_order():
    rng = np.random.default_rng(12)
    acc = rng.integers(-2**24, 2**24, (4, 5))
    sx = rng.random(4).astype(np.float32) * 0.01
    sw = rng.random(5).astype(np.float32) * 0.01
    bias = rng.standard_normal(5).astype(np.float32)
    y = orc.w8a8_epilogue(acc, sx, sw, bias)
    for m in range(4):
        for n in range(5):
            f = _f32_nearest(Fraction(int(acc[m, n])))
            p = _f32_nearest(Fraction(float(sx[m])) * Fraction(float(sw[n])))
            v = _f32_nearest(Fraction(float(f)) * Fraction(float(p)))
            v = _f32_nearest(Fraction(float(v)) + Fraction(float(bias[n])))
            assert y[m, n] == v


def test_fmaf32_matches_fractions():
    rng = np.random.default_rng(13)
    n = 3000
    a = rng.standard_normal(n).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    c = rng.standard_normal(n).astype(np.float32)
    # adversarial: c = -RN(a*b) (cancellation) and products landing on fp32 midpoints
    c[:500] = -(a[:500] * b[:500])
    a[500:1000] = np.float32(1.0) + np.float32(2.0 ** -23) * rng.integers(1, 64, 500).astype(np.float32)
    b[500:1000] = np.float32(1.0) + np.float32(2.0 ** -23) * rng.integers(1, 64, 500).astype(np.float32)
    c[500:1000] = np.float32(2.0 ** -24) * rng.choice([-1, 1], 500).astype(np.float32)
    c[1000:1200] = np.float32(2.0 ** 30)
    # exact fp32 midpoints a*b = 1 + (u+v)2^-12 + uv 2^-24 (uv odd) nudged by a c far below
    # float64's resolution: RN64(a*b + c) lands on the midpoint and only c's sign decides
    u = 2 * rng.integers(0, 500, 400) + 1
    v = 2 * rng.integers(0, 500, 400) + 1
    a[1200:1600] = (1.0 + u * 2.0 ** -12).astype(np.float32)
    b[1200:1600] = (1.0 + v * 2.0 ** -12).astype(np.float32)
    c[1200:1600] = (rng.choice([-1.0, 1.0], 400) * 2.0 ** -80).astype(np.float32)
    got = orc.fmaf32(a, b, c)
    for i in range(n):
        exact = Fraction(float(a[i])) * Fraction(float(b[i])) + Fraction(float(c[i]))
        assert got[i] == _f32_nearest(exact), i


def test_gemm_int8_block32_bruteforce():
    rng = np.random.default_rng(14)
    M, N, K = 6, 7, 256
    aq = rng.integers(-127, 128, (M, K), dtype=np.int16).astype(np.int8)
    bq = rng.integers(-127, 128, (N, K), dtype=np.int16).astype(np.int8)
    as_ = rng.random((M, K // 32)).astype(np.float32) * 0.01
    bs = rng.random((N, K // 32)).astype(np.float32) * 0.01
    bias = rng.standard_normal(N).astype(np.float32)
    got = orc.gemm_int8_block32(aq, as_, bq, bs, bias)
    for m in range(M):
        for n in range(N):
            acc = np.float32(0)
            for kb in range(K // 32):
                ip = sum(int(aq[m, k]) * int(bq[n, k]) for k in range(32 * kb, 32 * kb + 32))
                sc = _f32_nearest(Fraction(float(as_[m, kb])) * Fraction(float(bs[n, kb])))
                acc = _f32_nearest(Fraction(ip) * Fraction(float(sc)) + Fraction(float(acc)))
            acc = _f32_nearest(Fraction(float(acc)) + Fraction(float(bias[n])))
            assert got[m, n] == acc


def test_gemm_int4_w4a4_matches_unpacked_int8_path():
    rng = np.random.default_rng(15)
    a = rng.standard_normal((3, 64)).astype(np.float32)
    w = rng.standard_normal((4, 64)).astype(np.float32)
    ap, as_ = orc.quantize_pack_int4(a, rule="recip")
    wp, ws = orc.quantize_pack_int4(w, rule="recip")
    got = orc.gemm_int4_w4a4(ap, as_, wp, ws)
    want = orc.gemm_int8_block32(orc.unpack_int4(ap), as_, orc.unpack_int4(wp), ws)
    assert np.array_equal(got, want)
    # and it approximates the float product of the dequantized operands
    deq = orc.dequant_int4(ap, as_).astype(np.float64) @ orc.dequant_int4(wp, ws).T.astype(np.float64)
    assert np.allclose(got, deq, rtol=1e-5, atol=1e-5)


def test_split_k_bruteforce_fractions():
    """gemm_split_k against exact rationals on a tiny case whose split boundaries are written out:
    K = 384 is 3 k-tiles of 128; 2 splits take k-tiles {0, 1} (K 0-255) and {2} (K 256-383), each
    accumulated from 0 with correctly rounded fmaf, then v = (0 + p0) + p1, + bias, each rounded to
    fp32. 3 splits take one k-tile each; 4 splits leave the last one empty."""
    rng = np.random.default_rng(21)
    M, N, K = 2, 3, 384
    aq = rng.integers(-8, 8, (M, K))
    bq = rng.integers(-8, 8, (N, K))
    as_ = rng.uniform(0.01, 1.0, (M, K // 32)).astype(np.float32)
    bs = rng.uniform(0.01, 1.0, (N, K // 32)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)

    def partial(m, n, k_lo, k_hi):
        acc = Fraction(0)
        for kb in range(k_lo // 32, k_hi // 32):
            ip = sum(int(aq[m, k]) * int(bq[n, k]) for k in range(32 * kb, 32 * kb + 32))
            sc = _f32_nearest(Fraction(float(as_[m, kb])) * Fraction(float(bs[n, kb])))
            acc = Fraction(float(_f32_nearest(Fraction(ip) * Fraction(float(sc)) + acc)))
        return acc

    for splits, ranges in ((2, [(0, 256), (256, 384)]), (3, [(0, 128), (128, 256), (256, 384)]),
                           (4, [(0, 128), (128, 256), (256, 384), (384, 384)])):
        got = orc.gemm_split_k(aq, as_, bq, bs, bias, 32, splits)
        for m in range(M):
            for n in range(N):
                v = Fraction(0)
                for lo, hi in ranges:
                    v = Fraction(float(_f32_nearest(v + partial(m, n, lo, hi))))
                v = _f32_nearest(v + Fraction(float(bias[n])))
                assert got[m, n] == v, (splits, m, n)


def test_split_k_is_a_reassociation_of_the_unsplit_sum():
    """One split is the unsplit kernel; on an exactly representable grid (integer codes, power-of-
    two scales, small K) every association gives the same fp32 sum, so any split count must equal
    the unsplit result; on random data the split result stays within a few fp32 ulp of it."""
    rng = np.random.default_rng(22)
    M, N, K = 5, 7, 1280
    ap, bp = (((c[:, 0::2] & 0xF) | ((c[:, 1::2] & 0xF) << 4)).astype(np.uint8).view(np.int8)
              for c in (rng.integers(-8, 8, (M, K)), rng.integers(-8, 8, (N, K))))
    s2a = (2.0 ** rng.integers(-6, 0, (M, K // 32))).astype(np.float32)
    s2b = (2.0 ** rng.integers(-6, 0, (N, K // 32))).astype(np.float32)
    ref = orc.gemm_int4_w4a4(ap, s2a, bp, s2b)
    for splits in (1, 2, 3, 7, 8):
        assert np.array_equal(orc.gemm_int4_w4a4(ap, s2a, bp, s2b, splits=splits), ref), splits
    ra = rng.uniform(0.01, 1.0, (M, K // 32)).astype(np.float32)
    rb = rng.uniform(0.01, 1.0, (N, K // 32)).astype(np.float32)
    ref = orc.gemm_int4_w4a4(ap, ra, bp, rb).astype(np.float64)
    got = orc.gemm_int4_w4a4(ap, ra, bp, rb, splits=4).astype(np.float64)
    assert np.abs(got - ref).max() <= 8 * np.spacing(np.abs(ref).max().astype(np.float32))
    assert not np.array_equal(got, ref)  # the association does differ somewhere on random data
    # qblock 16: two scales per 32-K load, same k-tile boundaries
    sa16 = rng.uniform(0.01, 1.0, (M, K // 16)).astype(np.float32)
    sb16 = rng.uniform(0.01, 1.0, (N, K // 16)).astype(np.float32)
    r16 = orc.gemm_int4_w4a4(ap, sa16, bp, sb16, block=16).astype(np.float64)
    g16 = orc.gemm_int4_w4a4(ap, sa16, bp, sb16, block=16, splits=3).astype(np.float64)
    assert np.abs(g16 - r16).max() <= 8 * np.spacing(np.abs(r16).max().astype(np.float32))


def test_reference_auto_splits():
    """The reference's split choice, checked against its own sweep notes (binding.cpp:31-35, on a
    60-CU gfx906: 4-5 splits best for M=192 N=1536 = 72 tiles, 3 for 96 tiles) and its guards: no
    split once the 64 x 64 tiles fill 2 per CU, none when K has fewer than 16 k-tiles of 128."""
    assert orc.reference_auto_splits(192, 1536, 6144, 60) == 4
    assert orc.reference_auto_splits(256, 1536, 6144, 60) == 3      # 96 tiles
    assert orc.reference_auto_splits(4608, 3072, 3072, 60) == 1     # fills the GPU
    assert orc.reference_auto_splits(192, 1536, 1024, 60) == 1      # 8 k-tiles: too short to split
    assert orc.reference_auto_splits(64, 96, 3072, 256) == 3        # 24 k-tiles: at most 3
    assert orc.reference_auto_splits(1, 64, 16384, 256) == 8        # capped at 8


# ---- committed fixtures --------------------------------------------------------------------------
def test_golden_w4a16_small():
    f = np.load(golden_path("w4a16_small.npz"))
    x = orc.bf16_bits_to_f32(f["x_bf16_bits"])
    packed, scale = orc.quantize_pack_int4(f["w_float"], rule="div")
    assert np.array_equal(packed, f["w_q4"]) and np.array_equal(scale, f["w_scale"])
    assert np.array_equal(orc.w4a16_reference(x, packed, scale, f["bias"]), f["y_ref"])


def test_golden_w8a8_small():
    f = np.load(golden_path("w8a8_small.npz"))
    x = orc.bf16_bits_to_f32(f["x_bf16_bits"])
    xq, sx = orc.quantize_int8_rows(x)
    wq, sw = orc.quantize_int8_rows(f["w_float"])
    assert np.array_equal(xq, f["xq"]) and np.array_equal(sx, f["sx"])
    assert np.array_equal(wq, f["wq"]) and np.array_equal(sw, f["sw"])
    acc = orc.int8_matmul_exact(xq, wq)
    assert np.array_equal(acc, f["acc"])
    assert np.array_equal(orc.round_to_dtype(orc.w8a8_epilogue(acc, sx, sw), "bfloat16"), f["y_bf16"])
