"""The C ABI on the CPU: libqlinear.so loads, exports every function include/qlinear.h declares
with the arity the header gives, the ctypes table matches the header, and the argument checks
that run before any HIP call return the documented status codes and messages. No entry point
here reaches a device query or a launch (there is no GPU in this container)."""
import ctypes
import os
import re
import subprocess

import pytest

from tests.conftest import ROOT

HEADER = os.path.join(ROOT, "include", "qlinear.h")
LIB = os.path.join(ROOT, "comfy_ui_gfx906_tools_amd", "libqlinear.so")

QL_OK, QL_ERR_ARG, QL_ERR_SHAPE, QL_ERR_DTYPE, QL_ERR_ALIGN, QL_ERR_WORKSPACE = 0, 1, 2, 3, 4, 5


def _header_functions():
    """name -> number of parameters, parsed from the prototypes in include/qlinear.h."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"\b(?:int|size_t|const char\*)\s+(qlinear_\w+)\s*\(([^)]*)\)\s*;", text):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else len(params.split(","))
    return out


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.skip("libqlinear.so not built (python -m comfy_ui_gfx906_tools_amd.build)")
    from comfy_ui_gfx906_tools_amd import _lib
    return _lib.load_library(LIB)


def test_header_parses():
    fns = _header_functions()
    assert {"qlinear_w4a16_gemm", "qlinear_w8a8_gemm", "qlinear_quantize_int4", "qlinear_last_error"} <= set(fns)
    assert fns["qlinear_w4a16_gemm"] == 21 and fns["qlinear_abi_version"] == 0


def test_every_declared_symbol_is_exported(lib):
    fns = _header_functions()
    dyn = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in dyn.splitlines() if " T " in line}
    missing = sorted(set(fns) - exported)
    assert not missing, f"declared in include/qlinear.h but not exported: {missing}"
    for name in fns:
        assert getattr(lib, name) is not None


def test_ctypes_table_matches_header(lib):
    from comfy_ui_gfx906_tools_amd import _lib
    fns = _header_functions()
    assert set(_lib.SIGNATURES) == set(fns)
    for name, (_, args) in _lib.SIGNATURES.items():
        assert len(args) == fns[name], name


def test_abi_version_and_error_text(lib):
    assert lib.qlinear_abi_version() >> 16 == 4
    assert isinstance(lib.qlinear_last_error(), bytes)


def _err(lib):
    return lib.qlinear_last_error().decode()


def test_w4a16_argument_checks(lib):
    def f(*a):  # every argument but w_scale_kn and residual (NULL: the checks below do not use them)
        return lib.qlinear_w4a16_gemm(*a[:6], None, *a[6:11], None, *a[11:])
    # bad activation dtype (int32)
    assert f(3, 0, None, None, None, None, None, None, None, None, None, 4, 64, 64, 0, 0, None, 0, None) == QL_ERR_DTYPE
    assert "x dtype" in _err(lib)
    assert f(2, 3, None, None, None, None, None, None, None, None, None, 4, 64, 64, 0, 0, None, 0, None) == QL_ERR_DTYPE
    # K not a multiple of the 32-wide group
    assert f(2, 2, None, None, None, None, None, None, None, None, None, 4, 64, 48, 0, 0, None, 0, None) == QL_ERR_SHAPE
    assert "K % 32 == 0" in _err(lib) and "K=48" in _err(lib)
    assert f(2, 2, None, None, None, None, None, None, None, None, None, 4, 0, 64, 0, 0, None, 0, None) == QL_ERR_SHAPE
    assert f(2, 2, None, None, None, None, None, None, None, None, None, 4, 64, 64, 65, 0, None, 0, None) == QL_ERR_ARG
    assert f(2, 2, None, None, None, None, None, None, None, None, None, 4, 64, 64, 0, 4, None, 0, None) == QL_ERR_ARG
    # row scales are only meaningful for fp16 activations staged by qlinear_rows_to_f16
    assert f(2, 2, None, ctypes.c_void_p(16), None, None, None, None, None, None, None, 4, 64, 64, 0, 0, None, 0, None) == QL_ERR_ARG
    # M == 0 is a no-op that succeeds (binding.cpp:64, 93 of the reference return empty outputs)
    assert f(2, 2, None, None, None, None, None, None, None, None, None, 0, 64, 64, 0, 0, None, 0, None) == QL_OK
    assert f(2, 2, None, None, None, None, None, None, None, None, None, 4, 64, 64, 0, 0, None, 0, None) == QL_ERR_ARG
    assert "null" in _err(lib)
    assert f(1, 2, ctypes.c_void_p(8), None, ctypes.c_void_p(16), ctypes.c_void_p(16), None, None, ctypes.c_void_p(16), None, None,
             4, 64, 64, 0, 0, None, 0, None) == QL_ERR_ALIGN
    # forced kernel configurations (flags bits 8-11 = configuration + 1): 0-8 exist; the 256 x 256
    # configurations 4-6 need K % 64 == 0 and whole tiles
    cfg = lambda c: (c + 1) << 8  # noqa: E731
    assert f(2, 2, None, None, None, None, None, None, None, None, None, 0, 64, 64, 0, cfg(9), None, 0, None) == QL_ERR_ARG
    assert "configuration 9 does not exist" in _err(lib)
    # configuration 8 (MFMA, M <= 16): 16-bit x, K % 128 == 0, K <= 4096, no K split
    assert f(2, 2, None, None, None, None, None, None, None, None, None, 0, 64, 128, 0, cfg(8), None, 0, None) == QL_OK
    assert f(0, 2, None, None, None, None, None, None, None, None, None, 0, 64, 128, 0, cfg(8), None, 0, None) == QL_ERR_SHAPE
    assert f(2, 2, None, None, None, None, None, None, None, None, None, 17, 64, 128, 0, cfg(8), None, 0, None) == QL_ERR_SHAPE
    assert f(2, 2, None, None, None, None, None, None, None, None, None, 1, 64, 96, 0, cfg(8), None, 0, None) == QL_ERR_SHAPE
    assert f(2, 2, None, None, None, None, None, None, None, None, None, 1, 64, 4224, 0, cfg(8), None, 0, None) == QL_ERR_SHAPE
    assert "K % 128 == 0" in _err(lib)
    assert f(2, 2, None, None, None, None, None, None, None, None, None, 0, 64, 128, 2, cfg(8), None, 0, None) == QL_ERR_ARG
    assert "no K split" in _err(lib)
    # configuration 7 (VALU, M <= 4): 16-bit x, K <= 8192
    assert f(0, 2, None, None, None, None, None, None, None, None, None, 0, 64, 64, 0, cfg(7), None, 0, None) == QL_ERR_SHAPE
    assert f(2, 2, None, None, None, None, None, None, None, None, None, 5, 64, 64, 0, cfg(7), None, 0, None) == QL_ERR_SHAPE
    assert f(2, 2, None, None, None, None, None, None, None, None, None, 1, 64, 8224, 0, cfg(7), None, 0, None) == QL_ERR_SHAPE
    for c in range(8):
        assert f(2, 2, None, None, None, None, None, None, None, None, None, 0, 64, 64, 0, cfg(c), None, 0, None) == QL_OK
    for c in (4, 5, 6):
        assert f(2, 2, None, None, None, None, None, None, None, None, None, 0, 64, 96, 0, cfg(c), None, 0, None) == QL_ERR_SHAPE
        assert "K % 64 == 0" in _err(lib)
    for c in (4, 6):  # variants 0 and 2 run whole tiles; variant 1 (configuration 5) takes K pieces
        assert f(2, 2, None, None, None, None, None, None, None, None, None, 0, 64, 128, 2, cfg(c), None, 0, None) == QL_ERR_ARG
        assert "whole tiles" in _err(lib)
    assert f(2, 2, None, None, None, None, None, None, None, None, None, 0, 64, 128, 2, cfg(5), None, 0, None) == QL_OK


def test_w4a16_gated_residual_argument_checks(lib):
    from comfy_ui_gfx906_tools_amd import _lib
    f = lib.qlinear_w4a16_gemm
    P = ctypes.c_void_p(256)  # never dereferenced: every call below fails its checks first
    res = _lib.Residual(256, 512, 4)
    bad_rows = _lib.Residual(256, 512, 0)
    odd = _lib.Residual(257, 512, 4)
    GR = 16
    args = lambda r, flags, od=2: (2, od, P, None, P, P, None, None, None, P, None, None, r, 8, 64, 64, 0, flags,  # noqa: E731
                                   None, 0, None)
    assert f(*args(None, GR)) == QL_ERR_ARG and "exactly when" in _err(lib)
    assert f(*args(ctypes.addressof(res), 0)) == QL_ERR_ARG
    assert f(*args(ctypes.addressof(bad_rows), GR)) == QL_ERR_ARG and "gate_rows" in _err(lib)
    assert f(*args(ctypes.addressof(odd), GR)) == QL_ERR_ALIGN
    assert f(*args(ctypes.addressof(res), GR | 4)) == QL_ERR_ARG and "do not combine" in _err(lib)
    assert f(*args(ctypes.addressof(res), GR | (8 << 8))) == QL_ERR_ARG and "configurations 0-5" in _err(lib)
    assert f(*args(ctypes.addressof(res), GR | (7 << 8))) == QL_ERR_ARG  # variant 2 of the 256 x 256 kernel
    # host-side plan queries see the flag: the direct kernels are never planned with it
    assert _lib.load_library().qlinear_check_launch_plan(0, 2, 8, 4096, 4096, 0, GR, 256) == 0


def test_quantizer_and_w8a8_argument_checks(lib):
    assert lib.qlinear_quantize_int4(2, 2, None, None, None, 4, 64, None) == QL_ERR_ARG
    assert lib.qlinear_quantize_int4(2, 0, None, None, None, 4, 40, None) == QL_ERR_SHAPE
    assert lib.qlinear_quantize_int4(3, 0, None, None, None, 4, 64, None) == QL_ERR_DTYPE
    assert lib.qlinear_quantize_int4(2, 0, None, None, None, 0, 64, None) == QL_OK
    # Q4_0 repack: K % 32, null pointers, a source that is not 2-byte aligned
    assert lib.qlinear_repack_q4_0(None, None, None, 4, 48, None) == QL_ERR_SHAPE
    assert lib.qlinear_repack_q4_0(None, None, None, 0, 64, None) == QL_OK
    assert lib.qlinear_repack_q4_0(None, None, None, 4, 64, None) == QL_ERR_ARG
    assert lib.qlinear_repack_q4_0(ctypes.c_void_p(17), ctypes.c_void_p(256), ctypes.c_void_p(512), 4, 64,
                                   None) == QL_ERR_ALIGN
    assert lib.qlinear_quantize_int8_per_token(3, None, None, None, 4, 64, None) == QL_ERR_DTYPE
    assert lib.qlinear_quantize_int8_per_token(2, None, None, None, 4, 64, None) == QL_ERR_ARG
    assert lib.qlinear_w8a8_gemm(2, None, None, None, None, None, None, 4, 64, 96, None) == QL_ERR_SHAPE
    assert "K % 64 == 0" in _err(lib)
    assert lib.qlinear_w8a8_gemm(7, None, None, None, None, None, None, 4, 64, 128, None) == QL_ERR_DTYPE
    assert lib.qlinear_w8a8_gemm(2, None, None, None, None, None, None, 0, 64, 128, None) == QL_OK
    assert lib.qlinear_w8a8_gemm(2, ctypes.c_void_p(16), None, ctypes.c_void_p(16), None, None, ctypes.c_void_p(16),
                                 4, 64, 128, None) == QL_ERR_ARG  # float output needs both scale vectors
    assert lib.qlinear_rows_to_f16(2, None, None, None, 4, 12, None) == QL_ERR_SHAPE
    assert lib.qlinear_rows_to_f16(3, None, None, None, 4, 16, None) == QL_ERR_DTYPE


def test_w4a4_entry_point_checks_arguments(lib):
    p16 = ctypes.c_void_p(256)
    f = lib.qlinear_w4a4_gemm
    assert f(3, None, None, None, None, None, None, 4, 64, 64, 32, 1, None, 0, None) == QL_ERR_DTYPE
    assert f(0, None, None, None, None, None, None, 4, 64, 64, 8, 1, None, 0, None) == QL_ERR_ARG
    assert f(0, None, None, None, None, None, None, 4, 64, 48, 32, 1, None, 0, None) == QL_ERR_SHAPE
    assert f(0, None, None, None, None, None, None, 0, 64, 64, 32, 0, None, 0, None) == QL_OK
    assert f(0, None, None, None, None, None, None, 4, 64, 64, 32, 1, None, 0, None) == QL_ERR_ARG
    assert f(0, ctypes.c_void_p(264), p16, p16, p16, None, p16, 4, 64, 64, 16, 1, None, 0, None) == QL_ERR_ALIGN
    assert f(0, p16, ctypes.c_void_p(258), p16, p16, None, p16, 4, 64, 64, 16, 1, None, 0, None) == QL_ERR_ALIGN
    # split-K: at most 8 splits (binding.cpp MAX_SPLITS), and a workspace of splits * M * N fp32
    assert f(0, p16, p16, p16, p16, None, p16, 4, 64, 64, 32, 9, None, 0, None) == QL_ERR_ARG
    assert "splits" in _err(lib)
    assert f(0, p16, p16, p16, p16, None, p16, 4, 64, 64, 32, 2, None, 0, None) == QL_ERR_WORKSPACE
    assert "2048 bytes" in _err(lib)
    assert lib.qlinear_w4a4_workspace_bytes(4, 64, 64, 2, 0) == 2 * 4 * 64 * 4
    assert lib.qlinear_w4a4_workspace_bytes(4, 64, 64, 1, 0) == 0


def test_int8_block32_entry_points_check_arguments(lib):
    p16 = ctypes.c_void_p(256)
    qz, gm = lib.qlinear_quantize_int8_block32, lib.qlinear_gemm_int8_block32
    assert qz(3, None, None, None, 4, 64, None) == QL_ERR_DTYPE
    assert qz(2, None, None, None, 4, 48, None) == QL_ERR_SHAPE
    assert qz(2, None, None, None, 0, 64, None) == QL_OK
    assert qz(2, None, None, None, 4, 64, None) == QL_ERR_ARG
    assert qz(2, ctypes.c_void_p(264), p16, p16, 4, 64, None) == QL_ERR_ALIGN
    assert gm(3, None, None, None, None, None, None, 4, 64, 64, None) == QL_ERR_DTYPE
    assert gm(0, None, None, None, None, None, None, 4, 64, 40, None) == QL_ERR_SHAPE
    assert gm(0, None, None, None, None, None, None, 0, 64, 64, None) == QL_OK
    assert gm(0, None, None, None, None, None, None, 4, 64, 64, None) == QL_ERR_ARG
    assert gm(0, p16, p16, ctypes.c_void_p(264), p16, None, p16, 4, 64, 64, None) == QL_ERR_ALIGN


def test_fused_dit_entry_points_check_arguments(lib):
    """The fused DiT glue entry points reject bad arguments before any launch."""
    p16 = ctypes.c_void_p(256)
    adaln = lib.qlinear_adaln_modulate_f16
    assert adaln(3, None, 2, None, None, None, None, 4, 64, 1e-6, None) == QL_ERR_DTYPE
    assert adaln(2, None, 3, None, None, None, None, 4, 64, 1e-6, None) == QL_ERR_DTYPE
    assert adaln(2, None, 2, None, None, None, None, 4, 60, 1e-6, None) == QL_ERR_SHAPE
    assert adaln(2, None, 2, None, None, None, None, 4, 16392, 1e-6, None) == QL_ERR_SHAPE
    assert "K <= 16384" in _err(lib)
    assert adaln(2, None, 2, None, None, None, None, 4, 64, -1.0, None) == QL_ERR_ARG
    assert adaln(2, None, 2, None, None, None, None, 0, 64, 1e-6, None) == QL_OK
    assert adaln(2, None, 2, None, None, None, None, 4, 64, 1e-6, None) == QL_ERR_ARG
    assert adaln(2, ctypes.c_void_p(258), 2, p16, p16, p16, p16, 4, 64, 1e-6, None) == QL_ERR_ALIGN
    qk = lib.qlinear_qk_norm_rope
    assert qk(0, None, None, None, None, None, None, None, None, 4, 2, 128, 4, 0, 1e-6, None) == QL_ERR_DTYPE
    assert qk(2, None, None, None, None, None, None, None, None, 4, 2, 64, 4, 0, 1e-6, None) == QL_ERR_SHAPE
    assert qk(2, None, None, None, None, None, None, None, None, 4, 2, 128, 6, 3, 1e-6, None) == QL_ERR_SHAPE
    assert "l_offset" in _err(lib)
    assert qk(2, None, None, None, None, None, None, None, None, 0, 2, 128, 6, 3, 1e-6, None) == QL_OK
    assert qk(2, None, None, None, None, None, None, None, None, 4, 2, 128, 6, 2, 1e-6, None) == QL_ERR_ARG
    assert qk(2, p16, p16, p16, p16, p16, p16, p16, ctypes.c_void_p(258), 4, 2, 128, 6, 2, 1e-6,
              None) == QL_ERR_ALIGN
    hd = lib.qlinear_heads_to_f16
    assert hd(0, None, 2, 8, 128, 0, 8, None, 0, None, None, None) == QL_ERR_DTYPE
    assert hd(2, None, 2, 8, 64, 0, 8, None, 0, None, None, None) == QL_ERR_SHAPE
    assert hd(2, None, 2, 8, 128, 4, 5, None, 0, None, None, None) == QL_ERR_SHAPE  # rows past L
    assert hd(2, None, 2, 8, 128, 0, 8, None, 12, None, None, None) == QL_ERR_SHAPE  # E % 8
    assert hd(2, None, 24, 8, 128, 0, 8, None, 16384, None, None, None) == QL_ERR_SHAPE  # row too long
    assert hd(2, None, 2, 8, 128, 0, 0, None, 0, None, None, None) == QL_OK
    assert hd(2, p16, 2, 8, 128, 0, 8, None, 8, p16, p16, None) == QL_ERR_ARG  # E > 0 needs extra
    assert hd(2, p16, 2, 8, 128, 0, 8, ctypes.c_void_p(264), 8, p16, p16, None) == QL_ERR_ALIGN
    res = lib.qlinear_gated_residual
    assert res(3, None, None, None, None, 4, 64, None) == QL_ERR_DTYPE
    assert res(2, None, None, None, None, 4, 12, None) == QL_ERR_SHAPE
    assert res(2, None, None, None, None, 0, 64, None) == QL_OK
    assert res(2, None, None, None, None, 4, 64, None) == QL_ERR_ARG
    assert res(2, p16, ctypes.c_void_p(264), p16, p16, 4, 64, None) == QL_ERR_ALIGN


def test_error_text_is_per_thread(lib):
    import threading
    assert lib.qlinear_quantize_int4(3, 0, None, None, None, 4, 64, None) == QL_ERR_DTYPE
    main_msg = _err(lib)
    seen = {}

    def other():
        seen["before"] = lib.qlinear_last_error().decode()
        lib.qlinear_w8a8_gemm(2, None, None, None, None, None, None, 4, 64, 96, None)
        seen["after"] = lib.qlinear_last_error().decode()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["before"] == "" and "K % 64" in seen["after"]
    assert _err(lib) == main_msg
