"""ctypes binding of libqlinear.so (C ABI in include/qlinear.h) for torch tensors.

The reference binds its kernels through a pybind11 torch extension
(nodes/ComfyUI-Gfx906Int4/csrc/binding.cpp:364-392). Here the boundary is a plain C ABI and
this module is the thin Python side of it: it checks tensors, makes them contiguous (copies,
like binding.cpp:89-90), allocates outputs and workspaces with torch's caching allocator,
passes raw pointers plus the current HIP stream, and turns a non-zero status into
RuntimeError carrying the library's message. There is no CPU fallback: a missing library or a
CPU tensor is an error.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

_PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG_DIR, "libqlinear.so")

# dtype codes of the C ABI (csrc/binding.cpp:45-50 of the reference, plus int32)
QL_F32, QL_F16, QL_BF16, QL_I32 = 0, 1, 2, 3
_DTYPE_CODE = {torch.float32: QL_F32, torch.float16: QL_F16, torch.bfloat16: QL_BF16, torch.int32: QL_I32}

W4A16_BF16_MFMA = 1  # flags: bf16 activations straight into bf16 MFMA (see include/qlinear.h)
W4A16_GELU_TANH = 2  # flags: fused GELU-tanh epilogue
W4A16_F16_ROWSCALED = 4  # flags: output stored as the next GEMM's row-scaled fp16 operand
W4A16_GATED_RESIDUAL = 16  # flags: y = residual + gate * output (ql_w4a16_residual)
W4A16_CFG_SHIFT = 8  # flags bits 8-11: forced kernel configuration + 1 (QL_W4A16_CFG)
W4A16_TILE256 = 4    # configuration id of the 256 x 256, 8-wave kernel
W4A16_NOALLOC_SCRATCH_BYTES = 32 << 20  # QL_W4A16_NOALLOC_SCRATCH_BYTES

RULE_DIV = 0    # scale = amax / 7        (torch on CPU)
RULE_RECIP = 1  # scale = amax * fl(1/7)  (torch on GPU; the reference kernel)

_lib = None
_lib_lock = threading.Lock()

_c_size_t = ctypes.c_size_t
_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_c_vp = ctypes.c_void_p

# name -> (restype, argtypes); must match include/qlinear.h
SIGNATURES = {
    "qlinear_last_error": (ctypes.c_char_p, []),
    "qlinear_abi_version": (_c_int, []),
    "qlinear_w4a16_workspace_bytes": (_c_size_t, [_c_int, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_int]),
    "qlinear_w4a16_gemm": (_c_int, [_c_int, _c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
                                    _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_vp, _c_size_t, _c_vp]),
    "qlinear_w4a16_scales_kn": (_c_int, [_c_vp, _c_vp, _c_i64, _c_i64, _c_vp]),
    "qlinear_stream_read": (_c_int, [_c_vp, _c_i64, _c_vp, _c_vp]),
    "qlinear_w4a16_col_scales": (_c_int, [_c_vp, _c_vp, _c_i64, _c_i64, _c_vp]),
    "qlinear_w4a16_out_bound": (_c_int, [_c_vp, _c_vp, _c_vp, _c_int, _c_i64, _c_i64, _c_vp, _c_vp]),
    "qlinear_w4a16_gemm_noalloc": (_c_int, [_c_int, _c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
                                            _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_vp]),
    "qlinear_rows_to_f16": (_c_int, [_c_int, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_vp]),
    "qlinear_w4a16_auto_splits": (_c_int, [_c_i64, _c_i64, _c_i64, _c_int]),
    "qlinear_quantize_int4": (_c_int, [_c_int, _c_int, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_vp]),
    "qlinear_quantize_int8_per_token": (_c_int, [_c_int, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_vp]),
    "qlinear_repack_q4_0": (_c_int, [_c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_vp]),
    "qlinear_w8a8_gemm": (_c_int, [_c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp]),
    "qlinear_adaln_modulate_f16": (_c_int, [_c_int, _c_vp, _c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64,
                                            ctypes.c_float, _c_vp]),
    "qlinear_heads_gather": (_c_int, [_c_int, _c_int, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64,
                                      _c_vp, _c_vp, _c_vp]),
    "qlinear_adaln_modulate": (_c_int, [_c_int, _c_int, _c_vp, _c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64,
                                        ctypes.c_float, _c_vp]),
    "qlinear_qk_norm_rope": (_c_int, [_c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64,
                                      _c_i64, _c_i64, _c_i64, ctypes.c_float, _c_vp]),
    "qlinear_w4a4_gemm": (_c_int, [_c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_int,
                                   _c_int, _c_vp, _c_size_t, _c_vp]),
    "qlinear_w4a4_auto_splits": (_c_int, [_c_i64, _c_i64, _c_i64, _c_int]),
    "qlinear_check_launch_plan": (_c_int, [_c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_int]),
    "qlinear_w4a16_describe_plan": (_c_int, [_c_int, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_vp]),
    "qlinear_w4a4_workspace_bytes": (_c_size_t, [_c_i64, _c_i64, _c_i64, _c_int, _c_int]),
    "qlinear_rotate_rows_to_f16": (_c_int, [_c_int, _c_vp, _c_vp, _c_int, _c_vp, _c_vp, _c_i64, _c_i64, _c_vp]),
    "qlinear_heads_to_f16": (_c_int, [_c_int, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp,
                                      _c_vp, _c_vp]),
    "qlinear_quantize_int8_block32": (_c_int, [_c_int, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_vp]),
    "qlinear_gemm_int8_block32": (_c_int, [_c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64,
                                           _c_vp]),
    "qlinear_gated_residual": (_c_int, [_c_int, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_vp]),
}


class Residual(ctypes.Structure):
    """ql_w4a16_residual of include/qlinear.h."""
    _fields_ = [("residual", ctypes.c_void_p), ("gate", ctypes.c_void_p), ("gate_rows", ctypes.c_int64)]


def load_library(path: str = LIB_PATH):
    """Load libqlinear.so once (thread-safe). Raises if it is missing: build it with
    `python -m comfy_ui_gfx906_tools_amd.build`."""
    global _lib
    if _lib is not None:
        return _lib
    with _lib_lock:
        if _lib is None:
            if not os.path.exists(path):
                raise RuntimeError(f"{path} is missing: build it with `python -m comfy_ui_gfx906_tools_amd.build` "
                                   "(this engine has no CPU fallback)")
            lib = ctypes.CDLL(path)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def _check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load_library().qlinear_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (status {rc}): {msg}")


def _dev_tensor(t: torch.Tensor, name: str) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise RuntimeError(f"{name} must be on a GPU device, got {t.device} (no CPU fallback)")
    t = t.contiguous()
    if t.data_ptr() % 16:
        t = t.clone()  # fresh caching-allocator block: 16-byte aligned
    return t


def _stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


class _Workspaces:
    """Device workspaces, one per (device, stream): calls that share one must be ordered, and
    work on one stream is. Grown on demand. Every call writes the parts of the workspace it
    reads (staged activations, row scales, split-K partial tiles) before reading them, so the
    memory needs no initialisation."""

    def __init__(self):
        self._bufs: dict[tuple[int, int], torch.Tensor] = {}
        self._lock = threading.Lock()

    def get(self, device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
        key = (device.index, stream)
        with self._lock:
            buf = self._bufs.get(key)
            if buf is None or buf.numel() < nbytes:
                buf = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
                self._bufs[key] = buf
            return buf


_workspaces = _Workspaces()


def rows_to_f16(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Exact per-row power-of-two scaling of x [M, K] into fp16: (x16 [M, K], row_scale [M])."""
    lib = load_library()
    x = _dev_tensor(x, "x")
    if x.dtype not in (torch.float32, torch.float16, torch.bfloat16) or x.dim() != 2:
        raise RuntimeError(f"x must be a float32/float16/bfloat16 [M, K] tensor, got {x.dtype} {tuple(x.shape)}")
    M, K = x.shape
    x16 = torch.empty((M, K), dtype=torch.float16, device=x.device)
    rs = torch.empty((M,), dtype=torch.float32, device=x.device)
    if M == 0:
        return x16, rs
    with torch.cuda.device(x.device):
        rc = lib.qlinear_rows_to_f16(_DTYPE_CODE[x.dtype], x.data_ptr(), x16.data_ptr(), rs.data_ptr(), M, K,
                                     _stream_ptr(x.device))
    _check(rc, "rows_to_f16")
    return x16, rs


def w4a16_col_scales(w_scale: torch.Tensor) -> torch.Tensor:
    """Per-column power-of-two factors of the fp16 dequant for w_scale [N, K/32] (fp32 [N]):
    col[n] = 2^e_n with 8 max|w_scale[n, :]| 2^-e_n in [2^14, 2^15) (include/qlinear.h)."""
    lib = load_library()
    w_scale = _dev_tensor(w_scale, "w_scale")
    if w_scale.dtype != torch.float32 or w_scale.dim() != 2:
        raise RuntimeError(f"w_scale must be a float32 [N, K/32] tensor, got {w_scale.dtype} {tuple(w_scale.shape)}")
    N, G = w_scale.shape
    cs = torch.empty((N,), dtype=torch.float32, device=w_scale.device)
    with torch.cuda.device(w_scale.device):
        rc = lib.qlinear_w4a16_col_scales(w_scale.data_ptr(), cs.data_ptr(), N, G * 32, _stream_ptr(w_scale.device))
    _check(rc, "w4a16_col_scales")
    return cs


def stream_read(buf: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """One read of buf's bytes (qlinear_stream_read, the single-kernel HBM read floor); returns the
    per-workgroup xor words (uint32 as int32, one per CU)."""
    lib = load_library()
    buf = _dev_tensor(buf, "buf")
    nbytes = buf.numel() * buf.element_size()
    cus = torch.cuda.get_device_properties(buf.device).multi_processor_count
    if out is None:
        out = torch.empty((cus,), dtype=torch.int32, device=buf.device)
    with torch.cuda.device(buf.device):
        rc = lib.qlinear_stream_read(buf.data_ptr(), nbytes - nbytes % 16, out.data_ptr(), _stream_ptr(buf.device))
    _check(rc, "stream_read")
    return out


def w4a16_scales_kn(w_scale: torch.Tensor) -> torch.Tensor:
    """Group-major copy of the group scales: fp32 [K/32, N] with out[g, n] = w_scale[n, g]
    (qlinear_w4a16_scales_kn). Passed as w4a16_gemm(..., scales_kn=...), the tile kernels read
    it in place of w_scale: the same results, fewer memory requests."""
    lib = load_library()
    w_scale = _dev_tensor(w_scale, "w_scale")
    if w_scale.dtype != torch.float32 or w_scale.dim() != 2:
        raise RuntimeError(f"w_scale must be a float32 [N, K/32] tensor, got {w_scale.dtype} {tuple(w_scale.shape)}")
    N, G = w_scale.shape
    out = torch.empty((G, N), dtype=torch.float32, device=w_scale.device)
    with torch.cuda.device(w_scale.device):
        rc = lib.qlinear_w4a16_scales_kn(w_scale.contiguous().data_ptr(), out.data_ptr(), N, G * 32,
                                         _stream_ptr(w_scale.device))
    _check(rc, "w4a16_scales_kn")
    return out


def cached_scales_kn(w_scale: torch.Tensor) -> torch.Tensor | None:
    """w4a16_scales_kn(w_scale), kept on the w_scale tensor object and recomputed when the tensor
    is modified in place (version counter) or used from another stream; None for tensors without
    a version counter (inference-mode tensors), for which the GEMM reads w_scale itself."""
    try:
        version = w_scale._version
    except RuntimeError:
        return None
    stream = _stream_ptr(w_scale.device)
    hit = getattr(w_scale, "_qlinear_scales_kn", None)
    if hit is not None and hit[0] == version and hit[1] == stream:
        return hit[2]
    kn = w4a16_scales_kn(w_scale)
    try:
        w_scale._qlinear_scales_kn = (version, stream, kn)
    except (AttributeError, RuntimeError):
        pass
    return kn


def w4a16_out_bound(w_q4: torch.Tensor, w_scale: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """{max_n ||dequant W_n||_1 (1 + 2^-10), max_n |bias_n|} (fp32 [2] on the weight's device): the
    bound the row-scaled fp16 output (w4a16_gemm(..., f16_rowscaled=True)) derives its row factors
    from."""
    lib = load_library()
    w_q4 = _dev_tensor(w_q4, "w_q4")
    w_scale = _dev_tensor(w_scale, "w_scale")
    N = w_q4.shape[0]
    K = w_q4.shape[1] * 2
    if w_scale.dtype != torch.float32 or w_scale.numel() != N * (K // 32):
        raise RuntimeError(f"w_scale must be float32 [{N}, {K // 32}], got {w_scale.dtype} {tuple(w_scale.shape)}")
    if bias is not None:
        bias = _dev_tensor(bias, "bias")
        if bias.numel() != N or bias.dtype not in (torch.float32, torch.float16, torch.bfloat16):
            raise RuntimeError(f"bias must be a float [{N}] tensor, got {bias.dtype} {tuple(bias.shape)}")
    buf = torch.empty((2 + (N + 3) // 4,), dtype=torch.float32, device=w_q4.device)
    with torch.cuda.device(w_q4.device):
        rc = lib.qlinear_w4a16_out_bound(w_q4.data_ptr(), w_scale.data_ptr(),
                                         bias.data_ptr() if bias is not None else None,
                                         _DTYPE_CODE[bias.dtype] if bias is not None else QL_F32, N, K,
                                         buf.data_ptr(), _stream_ptr(w_q4.device))
    _check(rc, "w4a16_out_bound")
    return buf[:2]


def cached_out_bound(w_q4: torch.Tensor, w_scale: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
    """w4a16_out_bound kept on the w_q4 tensor object, recomputed when w_q4, w_scale or bias change
    (version counters, identity) or the stream differs."""
    try:
        key = (w_q4._version, id(w_scale), w_scale._version, id(bias), bias._version if bias is not None else 0,
               _stream_ptr(w_q4.device))
    except RuntimeError:  # inference-mode tensors keep no version counter
        return w4a16_out_bound(w_q4, w_scale, bias)
    hit = getattr(w_q4, "_qlinear_out_bound", None)
    if hit is not None and hit[0] == key:
        return hit[1]
    b = w4a16_out_bound(w_q4, w_scale, bias)
    try:
        w_q4._qlinear_out_bound = (key, b)
    except (AttributeError, RuntimeError):
        pass
    return b


def cached_col_scales(w_scale: torch.Tensor) -> torch.Tensor | None:
    """w4a16_col_scales(w_scale), kept on the w_scale tensor object and recomputed when the tensor
    is modified in place (torch's version counter), moved, or used from another stream. None for
    tensors without a version counter (inference-mode tensors): the GEMM then computes the factors
    in its workspace."""
    try:
        version = w_scale._version
    except RuntimeError:
        return None
    stream = _stream_ptr(w_scale.device)
    hit = getattr(w_scale, "_qlinear_col_scale", None)
    if hit is not None and hit[0] == version and hit[1] == stream:
        return hit[2]
    cs = w4a16_col_scales(w_scale)
    try:
        w_scale._qlinear_col_scale = (version, stream, cs)
    except (AttributeError, RuntimeError):
        pass
    return cs


def w4a16_gemm(x: torch.Tensor, w_q4: torch.Tensor, w_scale: torch.Tensor, bias: torch.Tensor | None = None,
               out_dtype: torch.dtype | None = None, splits: int = 0, bf16_mfma: bool = False,
               row_scale: torch.Tensor | None = None, config: int | None = None,
               gelu: bool = False, col_scale: torch.Tensor | None = None, noalloc: bool = False,
               f16_rowscaled: bool = False, out_bound: torch.Tensor | None = None,
               scales_kn: torch.Tensor | None = None, residual: torch.Tensor | None = None,
               gate: torch.Tensor | None = None, out: torch.Tensor | None = None):
    """y[M, N] = x[M, K] @ dequant(w_q4, w_scale)^T (+ bias) on the gfx950 W4A16 kernel.
    x: fp16/bf16/fp32 [M, K]; w_q4: int8 [N, K/2]; w_scale: fp32 [N, K/32]; bias: out_dtype [N].
    bf16 and fp32 activations go through the exact row-scaled fp16 staging unless bf16_mfma is
    set (then bf16 x meets bf16-rounded weights, the reference's bf16 dequant numerics).
    row_scale (fp16 x only): per-row factor from rows_to_f16, applied in the epilogue.
    config: force kernel configuration 0-6 (include/qlinear.h, QL_W4A16_CFG); None = automatic.
    gelu: fused GELU-tanh epilogue (QL_W4A16_GELU_TANH): gelu(round(y)), as Linear -> GELU.
    col_scale: the fp16 dequant's column factors (w4a16_col_scales of this w_scale); None = the
    GEMM computes them in its workspace.
    noalloc: run qlinear_w4a16_gemm_noalloc (the library's static scratch instead of a workspace
    from torch's allocator; calls needing more than QL_W4A16_NOALLOC_SCRATCH_BYTES raise).
    f16_rowscaled: the bf16 result (out_dtype must be bfloat16) stored as the next GEMM's row-scaled
    fp16 operand (QL_W4A16_F16_ROWSCALED); returns (y16 fp16 [M, N], row_scale fp32 [M]) to pass on
    as (x, row_scale). out_bound: w4a16_out_bound of this weight and bias (computed when None).
    scales_kn: w4a16_scales_kn of this w_scale (group-major, read by the tile kernels), or None.
    residual, gate: the gated residual epilogue (QL_W4A16_GATED_RESIDUAL), y = residual + gate * y:
    residual out_dtype [M, N]; gate out_dtype [G, N] with M % G == 0, row m taking gate row
    m // (M // G) (G = the batch of a [B, L, N] activation). out: the output tensor (out_dtype
    [M, N], contiguous), e.g. residual itself for the in-place update; None = a new tensor."""
    lib = load_library()
    x = _dev_tensor(x, "x")
    w_q4 = _dev_tensor(w_q4, "w_q4")
    w_scale = _dev_tensor(w_scale, "w_scale")
    if x.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise RuntimeError(f"x dtype {x.dtype} unsupported, expected bfloat16, float16 or float32")
    if w_q4.dtype not in (torch.int8, torch.uint8) or w_scale.dtype != torch.float32:
        raise RuntimeError(f"w_q4 must be int8 and w_scale float32, got {w_q4.dtype} / {w_scale.dtype}")
    if x.dim() != 2 or w_q4.dim() != 2:
        raise RuntimeError(f"expected x [M, K] and w_q4 [N, K/2], got {tuple(x.shape)} / {tuple(w_q4.shape)}")
    M, K = x.shape
    N = w_q4.shape[0]
    if w_q4.shape[1] * 2 != K or w_scale.numel() != N * (K // 32):
        raise RuntimeError(f"expected w_q4 [{N}, {K // 2}] and w_scale [{N}, {K // 32}] for x [{M}, {K}], "
                           f"got {tuple(w_q4.shape)} / {tuple(w_scale.shape)}")
    if not (x.device == w_q4.device == w_scale.device):
        raise RuntimeError(f"x, w_q4, w_scale must share a device, got {x.device} / {w_q4.device} / {w_scale.device}")
    out_dtype = out_dtype or x.dtype
    if out_dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise RuntimeError(f"out dtype {out_dtype} unsupported")
    if bias is not None:
        bias = _dev_tensor(bias, "bias")
        if bias.dtype != out_dtype or bias.numel() != N:
            raise RuntimeError(f"bias must be {out_dtype} [{N}], got {bias.dtype} {tuple(bias.shape)}")
    if out is not None:
        if f16_rowscaled or out.dtype != out_dtype or tuple(out.shape) != (M, N) or not out.is_contiguous() \
                or out.device != x.device:
            raise RuntimeError(f"out must be a contiguous {out_dtype} [{M}, {N}] tensor on {x.device}")
        y = out
    else:
        y = torch.empty((M, N), dtype=torch.float16 if f16_rowscaled else out_dtype, device=x.device)
    res_arg = None
    if residual is not None or gate is not None:
        if residual is None or gate is None:
            raise RuntimeError("the gated residual needs both residual and gate")
        residual, gate = _dev_tensor(residual, "residual"), _dev_tensor(gate, "gate")
        if residual.dtype != out_dtype or tuple(residual.shape) != (M, N) or not residual.is_contiguous():
            raise RuntimeError(f"residual must be a contiguous {out_dtype} [{M}, {N}] tensor, got {residual.dtype} "
                               f"{tuple(residual.shape)}")
        gate2 = gate.reshape(-1, N).contiguous() if N and gate.numel() % N == 0 else gate
        G = gate2.shape[0] if gate2.dim() == 2 else 0
        if gate.dtype != out_dtype or G < 1 or M % G != 0:
            raise RuntimeError(f"gate must be a {out_dtype} [G, {N}] tensor with {M} % G == 0, got "
                               f"{gate.dtype} {tuple(gate.shape)}")
        if residual.device != x.device or gate.device != x.device:
            raise RuntimeError("residual and gate must be on the device of x")
        res_arg = Residual(residual.data_ptr(), gate2.data_ptr(), M // G if M else 1)
    out_rs = None
    if f16_rowscaled:
        if out_dtype != torch.bfloat16:
            raise RuntimeError(f"f16_rowscaled rounds to bfloat16; out_dtype {out_dtype} given")
        out_rs = torch.empty((M,), dtype=torch.float32, device=x.device)
        if out_bound is None:
            out_bound = w4a16_out_bound(w_q4, w_scale, bias)
        out_bound = _dev_tensor(out_bound, "out_bound")
    if M == 0:
        return (y, out_rs) if f16_rowscaled else y
    flags = (W4A16_BF16_MFMA if bf16_mfma else 0) | (W4A16_GELU_TANH if gelu else 0) | \
        (W4A16_F16_ROWSCALED if f16_rowscaled else 0) | (W4A16_GATED_RESIDUAL if res_arg is not None else 0)
    res_ptr = ctypes.addressof(res_arg) if res_arg is not None else None
    if config is not None:
        flags |= (int(config) + 1) << W4A16_CFG_SHIFT
    xdt = _DTYPE_CODE[x.dtype]
    if row_scale is not None:
        row_scale = _dev_tensor(row_scale, "row_scale")
        if x.dtype != torch.float16 or row_scale.dtype != torch.float32 or row_scale.numel() != M:
            raise RuntimeError(f"row_scale needs float16 x and a float32 [{M}] tensor, got x {x.dtype}, "
                               f"row_scale {row_scale.dtype} {tuple(row_scale.shape)}")
    if col_scale is not None:
        col_scale = _dev_tensor(col_scale, "col_scale")
        if col_scale.dtype != torch.float32 or col_scale.numel() != N or col_scale.device != x.device:
            raise RuntimeError(f"col_scale must be a float32 [{N}] tensor on {x.device}, got {col_scale.dtype} "
                               f"{tuple(col_scale.shape)} on {col_scale.device}")
    if scales_kn is not None:
        scales_kn = _dev_tensor(scales_kn, "scales_kn")
        if scales_kn.dtype != torch.float32 or tuple(scales_kn.shape) != (K // 32, N) or scales_kn.device != x.device:
            raise RuntimeError(f"scales_kn must be a float32 [{K // 32}, {N}] tensor on {x.device}, got "
                               f"{scales_kn.dtype} {tuple(scales_kn.shape)} on {scales_kn.device}")
    kn_ptr = scales_kn.data_ptr() if scales_kn is not None else None
    with torch.cuda.device(x.device):
        stream = _stream_ptr(x.device)
        if noalloc:
            rc = lib.qlinear_w4a16_gemm_noalloc(xdt, _DTYPE_CODE[out_dtype], x.data_ptr(),
                                                row_scale.data_ptr() if row_scale is not None else None,
                                                w_q4.data_ptr(), w_scale.data_ptr(), kn_ptr,
                                                col_scale.data_ptr() if col_scale is not None else None,
                                                bias.data_ptr() if bias is not None else None, y.data_ptr(),
                                                out_bound.data_ptr() if out_bound is not None else None,
                                                out_rs.data_ptr() if out_rs is not None else None, res_ptr,
                                                M, N, K, splits, flags, stream)
            _check(rc, "w4a16_gemm_noalloc")
            return (y, out_rs) if f16_rowscaled else y
        nbytes = lib.qlinear_w4a16_workspace_bytes(xdt, M, N, K, splits, flags, x.device.index)
        ws = _workspaces.get(x.device, stream, nbytes) if nbytes else None
        rc = lib.qlinear_w4a16_gemm(xdt, _DTYPE_CODE[out_dtype], x.data_ptr(),
                                    row_scale.data_ptr() if row_scale is not None else None,
                                    w_q4.data_ptr(), w_scale.data_ptr(), kn_ptr,
                                    col_scale.data_ptr() if col_scale is not None else None,
                                    bias.data_ptr() if bias is not None else None, y.data_ptr(),
                                    out_bound.data_ptr() if out_bound is not None else None,
                                    out_rs.data_ptr() if out_rs is not None else None, res_ptr, M, N, K,
                                    splits, flags, ws.data_ptr() if ws is not None else None,
                                    ws.numel() if ws is not None else 0, stream)
    _check(rc, "w4a16_gemm")
    return (y, out_rs) if f16_rowscaled else y


def w4a16_describe_plan(M: int, N: int, K: int, x_dtype: torch.dtype = torch.bfloat16, splits: int = 0,
                        config: int | None = None, cus: int | None = None) -> dict:
    """The launch plan qlinear_w4a16_gemm makes (kernel configuration, tile shape, whole tiles, K
    pieces, staging), for `cus` compute units (default: the current GPU's). Host only."""
    if cus is None:
        cus = torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count
    flags = 0 if config is None else (int(config) + 1) << W4A16_CFG_SHIFT
    info = (ctypes.c_int * 7)()
    _check(load_library().qlinear_w4a16_describe_plan(_DTYPE_CODE[x_dtype], M, N, K, splits, flags, int(cus),
                                                      ctypes.cast(info, ctypes.c_void_p)), "w4a16_describe_plan")
    return {"config": info[0], "tile_rows": info[1], "tile_cols": info[2], "whole_tiles": info[3],
            "tiles": info[4], "k_pieces": info[5], "staged": bool(info[6])}


def w4a16_auto_splits(M: int, N: int, K: int, device: torch.device | int | None = None) -> int:
    """K pieces per tile that splits=0 resolves to for [M, K] x [N, K]^T (1 = unsplit)."""
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device("cuda", device) \
        if isinstance(device, int) else device
    rc = load_library().qlinear_w4a16_auto_splits(M, N, K, dev.index)
    if rc < 0:
        _check(-rc, "w4a16_auto_splits")
    return rc


def quantize_int4(x: torch.Tensor, rule: int = RULE_RECIP) -> tuple[torch.Tensor, torch.Tensor]:
    """Block-32 int4 quantize + pack of a device tensor [..., K] -> (int8 [..., K/2], fp32 [..., K/32])."""
    lib = load_library()
    x = _dev_tensor(x, "x")
    if x.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise RuntimeError(f"unsupported dtype {x.dtype}, expected float32/float16/bfloat16")
    K = x.shape[-1]
    if K % 32 != 0:
        raise RuntimeError(f"last dim {K} not divisible by block 32")
    rows = x.numel() // K if K else 0
    packed = torch.empty((*x.shape[:-1], K // 2), dtype=torch.int8, device=x.device)
    scale = torch.empty((*x.shape[:-1], K // 32), dtype=torch.float32, device=x.device)
    if rows == 0:
        return packed, scale
    with torch.cuda.device(x.device):
        rc = lib.qlinear_quantize_int4(_DTYPE_CODE[x.dtype], rule, x.data_ptr(), packed.data_ptr(), scale.data_ptr(),
                                       rows, K, _stream_ptr(x.device))
    _check(rc, "quantize_int4")
    return packed, scale


def repack_q4_0(raw: torch.Tensor, out_features: int, in_features: int) -> tuple[torch.Tensor, torch.Tensor]:
    """ggml Q4_0 bytes of a [out_features, in_features] weight (device tensor) -> (int8
    [out, in/2], fp32 [out, in/32]) in the native layout, by the HIP kernel."""
    lib = load_library()
    raw = _dev_tensor(raw, "raw").reshape(-1)
    nbytes = raw.numel() * raw.element_size()
    if in_features % 32 != 0 or nbytes != out_features * (in_features // 32) * 18:
        raise RuntimeError(f"Q4_0 data of {nbytes} bytes does not hold a [{out_features}, {in_features}] weight "
                           f"(expected {out_features * (in_features // 32) * 18} bytes, in_features % 32 == 0)")
    packed = torch.empty((out_features, in_features // 2), dtype=torch.int8, device=raw.device)
    scale = torch.empty((out_features, in_features // 32), dtype=torch.float32, device=raw.device)
    if out_features == 0:
        return packed, scale
    with torch.cuda.device(raw.device):
        rc = lib.qlinear_repack_q4_0(raw.data_ptr(), packed.data_ptr(), scale.data_ptr(), out_features, in_features,
                                     _stream_ptr(raw.device))
    _check(rc, "repack_q4_0")
    return packed, scale


def quantize_int8_per_token(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row int8 quantize: x [M, K] -> (int8 [M, K], fp32 [M])."""
    lib = load_library()
    x = _dev_tensor(x, "x")
    if x.dtype not in (torch.float32, torch.float16, torch.bfloat16) or x.dim() != 2:
        raise RuntimeError(f"x must be a float32/float16/bfloat16 [M, K] tensor, got {x.dtype} {tuple(x.shape)}")
    M, K = x.shape
    q = torch.empty((M, K), dtype=torch.int8, device=x.device)
    s = torch.empty((M,), dtype=torch.float32, device=x.device)
    if M == 0:
        return q, s
    with torch.cuda.device(x.device):
        rc = lib.qlinear_quantize_int8_per_token(_DTYPE_CODE[x.dtype], x.data_ptr(), q.data_ptr(), s.data_ptr(), M, K,
                                                 _stream_ptr(x.device))
    _check(rc, "quantize_int8_per_token")
    return q, s


def w8a8_gemm(xq: torch.Tensor, x_scale: torch.Tensor, wq: torch.Tensor, w_scale: torch.Tensor,
              bias: torch.Tensor | None = None, out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """int8 x int8 -> int32 GEMM with per-token x per-channel rescale. out_dtype torch.int32
    returns the raw accumulators."""
    lib = load_library()
    xq = _dev_tensor(xq, "xq")
    wq = _dev_tensor(wq, "wq")
    if xq.dtype != torch.int8 or wq.dtype != torch.int8 or xq.dim() != 2 or wq.dim() != 2:
        raise RuntimeError(f"expected int8 xq [M, K] and wq [N, K], got {xq.dtype} {tuple(xq.shape)} / "
                           f"{wq.dtype} {tuple(wq.shape)}")
    M, K = xq.shape
    N = wq.shape[0]
    if wq.shape[1] != K:
        raise RuntimeError(f"K mismatch: xq {tuple(xq.shape)} vs wq {tuple(wq.shape)}")
    if out_dtype not in _DTYPE_CODE:
        raise RuntimeError(f"out dtype {out_dtype} unsupported")
    sx = sw = None
    if out_dtype != torch.int32:
        sx = _dev_tensor(x_scale, "x_scale")
        sw = _dev_tensor(w_scale, "w_scale")
        if sx.dtype != torch.float32 or sw.dtype != torch.float32 or sx.numel() != M or sw.numel() != N:
            raise RuntimeError(f"scales must be float32 [{M}] / [{N}], got {sx.dtype} {tuple(sx.shape)} / "
                               f"{sw.dtype} {tuple(sw.shape)}")
        if bias is not None:
            bias = _dev_tensor(bias, "bias")
            if bias.dtype != out_dtype or bias.numel() != N:
                raise RuntimeError(f"bias must be {out_dtype} [{N}], got {bias.dtype} {tuple(bias.shape)}")
    else:
        bias = None
    y = torch.empty((M, N), dtype=out_dtype, device=xq.device)
    if M == 0:
        return y
    with torch.cuda.device(xq.device):
        rc = lib.qlinear_w8a8_gemm(_DTYPE_CODE[out_dtype], xq.data_ptr(), sx.data_ptr() if sx is not None else None,
                                   wq.data_ptr(), sw.data_ptr() if sw is not None else None,
                                   bias.data_ptr() if bias is not None else None, y.data_ptr(), M, N, K,
                                   _stream_ptr(xq.device))
    _check(rc, "w8a8_gemm")
    return y


def quantize_int8_block32(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Block-32 int8 quantize of x [M, K] -> (int8 [M, K], fp32 [M, K/32])."""
    lib = load_library()
    x = _dev_tensor(x, "x")
    if x.dim() != 2 or x.shape[1] % 32 != 0 or x.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise RuntimeError(f"x must be a float32/float16/bfloat16 [M, K] tensor with K % 32 == 0, got {x.dtype} "
                           f"{list(x.shape)}")
    M, K = x.shape
    q = torch.empty((M, K), dtype=torch.int8, device=x.device)
    s = torch.empty((M, K // 32), dtype=torch.float32, device=x.device)
    if M == 0:
        return q, s
    with torch.cuda.device(x.device):
        rc = lib.qlinear_quantize_int8_block32(_DTYPE_CODE[x.dtype], x.data_ptr(), q.data_ptr(), s.data_ptr(), M, K,
                                               _stream_ptr(x.device))
    _check(rc, "quantize_int8_block32")
    return q, s


def gemm_int8_block32(a: torch.Tensor, a_scale: torch.Tensor, b: torch.Tensor, b_scale: torch.Tensor,
                      bias: torch.Tensor | None = None, out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """[M, N] = block-32 int8 A [M, K] x B [N, K]^T with the reference's per-block fmaf order."""
    lib = load_library()
    a, b = _dev_tensor(a, "A"), _dev_tensor(b, "B")
    if a.device != b.device:
        raise RuntimeError("A and B must be on the same device")
    if a.dtype != torch.int8 or b.dtype != torch.int8:
        raise RuntimeError("A and B must be int8")
    if a.dim() != 2 or b.dim() != 2 or a.shape[1] != b.shape[1] or a.shape[1] % 32 != 0:
        raise RuntimeError(f"expected A [M, K], B [N, K], K % 32 == 0; got A {list(a.shape)} B {list(b.shape)}")
    M, N, K = a.shape[0], b.shape[0], a.shape[1]
    a_scale, b_scale = _dev_tensor(a_scale, "A_scale"), _dev_tensor(b_scale, "B_scale")
    if a_scale.dtype != torch.float32 or b_scale.dtype != torch.float32:
        raise RuntimeError("scales must be float32")
    if a_scale.numel() != M * (K // 32) or b_scale.numel() != N * (K // 32):
        raise RuntimeError(f"scales must be [M, K/32] / [N, K/32], got {list(a_scale.shape)} / {list(b_scale.shape)}")
    if out_dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise RuntimeError(f"unsupported dtype {out_dtype}, expected float32/float16/bfloat16")
    if bias is not None:
        bias = _dev_tensor(bias, "bias")
        if bias.dtype != out_dtype or bias.numel() != N:
            raise RuntimeError(f"bias must be {out_dtype} [{N}], got {bias.dtype} {list(bias.shape)}")
    y = torch.empty((M, N), dtype=out_dtype, device=a.device)
    if M == 0:
        return y
    with torch.cuda.device(a.device):
        rc = lib.qlinear_gemm_int8_block32(_DTYPE_CODE[out_dtype], a.data_ptr(), a_scale.data_ptr(), b.data_ptr(),
                                           b_scale.data_ptr(), bias.data_ptr() if bias is not None else None,
                                           y.data_ptr(), M, N, K, _stream_ptr(a.device))
    _check(rc, "gemm_int8_block32")
    return y


def rotate_rows_to_f16(x: torch.Tensor, signs: torch.Tensor, group: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-group rotation x_g -> H (signs * x_g) / sqrt(group) of x [M, K], written as the W4A16
    GEMM's fp16 operand: (x16 [M, K] fp16, row_scale [M] fp32)."""
    lib = load_library()
    x = _dev_tensor(x, "x")
    signs = _dev_tensor(signs, "signs").float().reshape(-1)
    if x.dim() != 2 or x.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise RuntimeError(f"x must be a float32/float16/bfloat16 [M, K] tensor, got {x.dtype} {tuple(x.shape)}")
    if signs.numel() != group:
        raise RuntimeError(f"signs must have {group} elements, got {signs.numel()}")
    M, K = x.shape
    x16 = torch.empty((M, K), dtype=torch.float16, device=x.device)
    rs = torch.empty((M,), dtype=torch.float32, device=x.device)
    with torch.cuda.device(x.device):
        rc = lib.qlinear_rotate_rows_to_f16(_DTYPE_CODE[x.dtype], x.data_ptr(), signs.data_ptr(), int(group),
                                            x16.data_ptr(), rs.data_ptr(), M, K, _stream_ptr(x.device))
    _check(rc, "rotate_rows_to_f16")
    return x16, rs


def w4a4_auto_splits(M: int, N: int, K: int, device: torch.device | int | None = None) -> int:
    """The split-K count splits=0 resolves to in w4a4_gemm (the reference's auto_splits rule)."""
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device("cuda", device) \
        if isinstance(device, int) else device
    rc = load_library().qlinear_w4a4_auto_splits(M, N, K, dev.index)
    if rc < 0:
        _check(-rc, "w4a4_auto_splits")
    return rc


def w4a4_gemm(a_q4: torch.Tensor, a_scale: torch.Tensor, b_q4: torch.Tensor, b_scale: torch.Tensor,
              bias: torch.Tensor | None = None, out_dtype: torch.dtype = torch.float32,
              qblock: int = 32, splits: int = 1) -> torch.Tensor:
    """y[M, N] from block-scaled int4 activations (quantize_int4) and int4 weights with the
    reference's per-block fmaf accumulation in K order and, for splits > 1 (0 = the reference's
    automatic choice), its per-split fp32 partials summed in split order (see include/qlinear.h)."""
    lib = load_library()
    a_q4, b_q4 = _dev_tensor(a_q4, "A_packed"), _dev_tensor(b_q4, "B_packed")
    if a_q4.device != b_q4.device:
        raise RuntimeError(f"A and B must be on the same device, got {a_q4.device} / {b_q4.device}")
    if a_q4.dtype != torch.int8 or b_q4.dtype != torch.int8:
        raise RuntimeError(f"packed tensors must be int8, got {a_q4.dtype} / {b_q4.dtype}")
    if a_q4.dim() != 2 or b_q4.dim() != 2 or a_q4.shape[1] != b_q4.shape[1] or a_q4.shape[1] % 16 != 0:
        raise RuntimeError(f"expected A [M, K/2], B [N, K/2], K % 32 == 0; got A {tuple(a_q4.shape)} B "
                           f"{tuple(b_q4.shape)}")
    if qblock not in (32, 16):
        raise RuntimeError(f"qblock must be 32 or 16, got {qblock}")
    a_scale, b_scale = _dev_tensor(a_scale, "A_scale"), _dev_tensor(b_scale, "B_scale")
    if a_scale.dtype != torch.float32 or b_scale.dtype != torch.float32:
        raise RuntimeError("scales must be float32")
    M, N, K = a_q4.shape[0], b_q4.shape[0], a_q4.shape[1] * 2
    if a_scale.numel() != M * K // qblock or b_scale.numel() != N * K // qblock:
        raise RuntimeError(f"scales must be [M, K/{qblock}] / [N, K/{qblock}] = {M * K // qblock} / {N * K // qblock} "
                           f"elements, got {a_scale.numel()} / {b_scale.numel()}")
    if out_dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise RuntimeError(f"unsupported dtype {out_dtype}, expected float32/float16/bfloat16")
    if bias is not None:
        bias = _dev_tensor(bias, "bias")
        if bias.dtype != out_dtype:
            raise RuntimeError(f"bias dtype {bias.dtype} != out dtype {out_dtype}")
        if bias.numel() != N:
            raise RuntimeError(f"bias must have {N} elements, got {bias.numel()}")
    if not 0 <= int(splits) <= 8:
        raise RuntimeError(f"splits must be in [0, 8], got {splits}")
    y = torch.empty((M, N), dtype=out_dtype, device=a_q4.device)
    if M == 0:
        return y
    with torch.cuda.device(a_q4.device):
        stream = _stream_ptr(a_q4.device)
        nbytes = lib.qlinear_w4a4_workspace_bytes(M, N, K, int(splits), a_q4.device.index)
        ws = _workspaces.get(a_q4.device, stream, nbytes) if nbytes else None
        rc = lib.qlinear_w4a4_gemm(_DTYPE_CODE[out_dtype], a_q4.data_ptr(), a_scale.data_ptr(), b_q4.data_ptr(),
                                   b_scale.data_ptr(), bias.data_ptr() if bias is not None else None, y.data_ptr(),
                                   M, N, K, qblock, int(splits), ws.data_ptr() if ws is not None else None,
                                   ws.numel() if ws is not None else 0, stream)
    _check(rc, "w4a4_gemm")
    return y


# ---- fused DiT block glue (csrc/dit_fused.hip) -----------------------------------------------
def adaln_modulate_f16(x: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor,
                       eps: float = 1e-6) -> tuple[torch.Tensor, torch.Tensor]:
    """LayerNorm(x) * (1 + scale) + shift for x [M, K] (shift / scale [K], shared by every row),
    returned as the W4A16 GEMM's fp16 operand: (x16 [M, K] fp16, row_scale [M] fp32), to be
    passed to w4a16_gemm(x16, ..., row_scale=row_scale)."""
    lib = load_library()
    x = _dev_tensor(x, "x")
    shift = _dev_tensor(shift, "shift").reshape(-1)
    scale = _dev_tensor(scale, "scale").reshape(-1)
    if x.dim() != 2 or x.dtype not in _DTYPE_CODE or x.dtype == torch.int32:
        raise RuntimeError(f"x must be a float [M, K] tensor, got {x.dtype} {tuple(x.shape)}")
    M, K = x.shape
    if shift.dtype != scale.dtype or shift.numel() != K or scale.numel() != K or shift.dtype == torch.int32:
        raise RuntimeError(f"shift and scale must be float [{K}] tensors of one dtype, got {shift.dtype} "
                           f"{tuple(shift.shape)} / {scale.dtype} {tuple(scale.shape)}")
    x16 = torch.empty((M, K), dtype=torch.float16, device=x.device)
    rs = torch.empty((M,), dtype=torch.float32, device=x.device)
    with torch.cuda.device(x.device):
        rc = lib.qlinear_adaln_modulate_f16(_DTYPE_CODE[x.dtype], x.data_ptr(), _DTYPE_CODE[shift.dtype],
                                            shift.data_ptr(), scale.data_ptr(), x16.data_ptr(), rs.data_ptr(), M, K,
                                            float(eps), _stream_ptr(x.device))
    _check(rc, "adaln_modulate_f16")
    return x16, rs


OPERAND_F16_ROWSCALED, OPERAND_PLAIN, OPERAND_I8_PER_TOKEN = 0, 1, 2


def adaln_modulate(x: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor, out: str = "f16",
                   eps: float = 1e-6):
    """LayerNorm(x) * (1 + scale) + shift for x [M, K] (shift / scale [K]) written as `out`:
    "f16" -> (x16 fp16 [M, K], row_scale fp32 [M]) as adaln_modulate_f16; "plain" -> the row in
    x's dtype [M, K]; "i8" -> (q int8 [M, K], scale fp32 [M]), the W8A8 GEMM's per-token operand
    (the plain output quantized by quantize_int8_per_token's rule, in the same pass)."""
    lib = load_library()
    kinds = {"f16": OPERAND_F16_ROWSCALED, "plain": OPERAND_PLAIN, "i8": OPERAND_I8_PER_TOKEN}
    if out not in kinds:
        raise RuntimeError(f"out must be one of {sorted(kinds)}, got {out!r}")
    x = _dev_tensor(x, "x")
    shift = _dev_tensor(shift, "shift").reshape(-1)
    scale = _dev_tensor(scale, "scale").reshape(-1)
    if x.dim() != 2 or x.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise RuntimeError(f"x must be a float [M, K] tensor, got {x.dtype} {tuple(x.shape)}")
    M, K = x.shape
    if shift.dtype != scale.dtype or shift.numel() != K or scale.numel() != K or shift.dtype == torch.int32:
        raise RuntimeError(f"shift and scale must be float [{K}] tensors of one dtype, got {shift.dtype} "
                           f"{tuple(shift.shape)} / {scale.dtype} {tuple(scale.shape)}")
    odt = {"f16": torch.float16, "plain": x.dtype, "i8": torch.int8}[out]
    y = torch.empty((M, K), dtype=odt, device=x.device)
    rs = torch.empty((M,), dtype=torch.float32, device=x.device) if out != "plain" else None
    with torch.cuda.device(x.device):
        rc = lib.qlinear_adaln_modulate(kinds[out], _DTYPE_CODE[x.dtype], x.data_ptr(), _DTYPE_CODE[shift.dtype],
                                        shift.data_ptr(), scale.data_ptr(), y.data_ptr(),
                                        rs.data_ptr() if rs is not None else None, M, K, float(eps),
                                        _stream_ptr(x.device))
    _check(rc, "adaln_modulate")
    return y if out == "plain" else (y, rs)


def qk_norm_rope(qkv: torch.Tensor, q_norm: torch.Tensor, k_norm: torch.Tensor, cos: torch.Tensor,
                 sin: torch.Tensor, heads: int, out: tuple | None = None, l_offset: int = 0,
                 eps: float = 1e-6) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """qkv [L, 3 * heads * 128] -> q, k, v [heads, L_out, 128] with RMSNorm (scales q_norm /
    k_norm [128]) and RoPE (cos / sin fp32 [L_out, 64]) on q and k, written to rows
    [l_offset, l_offset + L) of `out` (three [heads, L_out, 128] tensors; new ones with
    L_out = L when None)."""
    lib = load_library()
    qkv = _dev_tensor(qkv, "qkv")
    if qkv.dtype not in (torch.bfloat16, torch.float16) or qkv.dim() != 2 or qkv.shape[1] != 3 * heads * 128:
        raise RuntimeError(f"qkv must be a bfloat16/float16 [L, {3 * heads * 128}] tensor, got {qkv.dtype} "
                           f"{tuple(qkv.shape)}")
    L = qkv.shape[0]
    qn = _dev_tensor(q_norm, "q_norm").to(qkv.dtype)
    kn = _dev_tensor(k_norm, "k_norm").to(qkv.dtype)
    cos = _dev_tensor(cos, "cos").float().reshape(-1, 64)
    sin = _dev_tensor(sin, "sin").float().reshape(-1, 64)
    if out is None:
        out = tuple(torch.empty((heads, L, 128), dtype=qkv.dtype, device=qkv.device) for _ in range(3))
    for t in out:
        if t.dtype != qkv.dtype or t.dim() != 3 or t.shape[0] != heads or t.shape[2] != 128 or not t.is_contiguous():
            raise RuntimeError(f"outputs must be contiguous {qkv.dtype} [{heads}, L_out, 128] tensors, got {t.dtype} "
                               f"{tuple(t.shape)}")
    L_out = out[0].shape[1]
    if cos.shape[0] != L_out or sin.shape[0] != L_out or qn.numel() != 128 or kn.numel() != 128:
        raise RuntimeError(f"cos / sin must be [{L_out}, 64] and the norm scales [128]")
    with torch.cuda.device(qkv.device):
        rc = lib.qlinear_qk_norm_rope(_DTYPE_CODE[qkv.dtype], qkv.data_ptr(), qn.data_ptr(), kn.data_ptr(),
                                      cos.data_ptr(), sin.data_ptr(), out[0].data_ptr(), out[1].data_ptr(),
                                      out[2].data_ptr(), L, heads, 128, L_out, l_offset, float(eps),
                                      _stream_ptr(qkv.device))
    _check(rc, "qk_norm_rope")
    return out


def gated_residual(x: torch.Tensor, gate: torch.Tensor, y: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """x + gate * y for x, y [..., K] and gate [K] (one dtype), into `out` (a new tensor when None;
    `out` may be x itself for the in-place update)."""
    lib = load_library()
    x = _dev_tensor(x, "x")
    K = x.shape[-1]
    gate = _dev_tensor(gate, "gate").reshape(-1)
    y = _dev_tensor(y, "y")
    if x.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise RuntimeError(f"dtype {x.dtype} unsupported")
    if gate.dtype != x.dtype or y.dtype != x.dtype or gate.numel() != K or y.shape != x.shape:
        raise RuntimeError(f"gate [{K}] and y {tuple(x.shape)} must have x's dtype {x.dtype}, got {gate.dtype} "
                           f"{tuple(gate.shape)} / {y.dtype} {tuple(y.shape)}")
    if out is None:
        out = torch.empty_like(x)
    elif not (out.is_cuda and out.is_contiguous() and out.data_ptr() % 16 == 0 and out.shape == x.shape
              and out.dtype == x.dtype):
        raise RuntimeError("out must be a contiguous, 16-byte aligned GPU tensor of x's shape and dtype")
    with torch.cuda.device(x.device):
        rc = lib.qlinear_gated_residual(_DTYPE_CODE[x.dtype], out.data_ptr(), x.data_ptr(), gate.data_ptr(),
                                        y.data_ptr(), x.numel() // K if K else 0, K, _stream_ptr(x.device))
    _check(rc, "gated_residual")
    return out


def heads_to_f16(o: torch.Tensor, l_offset: int = 0, rows: int | None = None,
                 extra: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Rows [l_offset, l_offset + rows) of an attention output o [H, L, 128] flattened over heads,
    each followed by the same row of `extra` [rows, E], as the W4A16 GEMM's fp16 operand:
    (x16 [rows, H * 128 + E] fp16, row_scale [rows] fp32)."""
    lib = load_library()
    o = _dev_tensor(o, "o")
    if o.dim() != 3 or o.shape[2] != 128 or o.dtype not in (torch.bfloat16, torch.float16):
        raise RuntimeError(f"o must be a bfloat16/float16 [H, L, 128] tensor, got {o.dtype} {tuple(o.shape)}")
    H, L = o.shape[0], o.shape[1]
    rows = L - l_offset if rows is None else rows
    E = 0
    if extra is not None:
        extra = _dev_tensor(extra, "extra")
        if extra.dtype != o.dtype or extra.dim() != 2 or extra.shape[0] != rows:
            raise RuntimeError(f"extra must be a {o.dtype} [{rows}, E] tensor, got {extra.dtype} {tuple(extra.shape)}")
        E = extra.shape[1]
    x16 = torch.empty((rows, H * 128 + E), dtype=torch.float16, device=o.device)
    rs = torch.empty((rows,), dtype=torch.float32, device=o.device)
    with torch.cuda.device(o.device):
        rc = lib.qlinear_heads_to_f16(_DTYPE_CODE[o.dtype], o.data_ptr(), H, L, 128, l_offset, rows,
                                      extra.data_ptr() if extra is not None else None, E, x16.data_ptr(),
                                      rs.data_ptr(), _stream_ptr(o.device))
    _check(rc, "heads_to_f16")
    return x16, rs


def heads_gather(o: torch.Tensor, l_offset: int = 0, rows: int | None = None, extra: torch.Tensor | None = None,
                 out: str = "f16"):
    """heads_to_f16's gathered rows written as `out`: "f16" -> (x16, row_scale) as heads_to_f16;
    "plain" -> the rows in o's dtype [rows, H * 128 + E]; "i8" -> (q int8, scale fp32 [rows]), the
    W8A8 GEMM's per-token operand (quantize_int8_per_token's rule, in the same pass)."""
    lib = load_library()
    kinds = {"f16": OPERAND_F16_ROWSCALED, "plain": OPERAND_PLAIN, "i8": OPERAND_I8_PER_TOKEN}
    if out not in kinds:
        raise RuntimeError(f"out must be one of {sorted(kinds)}, got {out!r}")
    o = _dev_tensor(o, "o")
    if o.dim() != 3 or o.shape[2] != 128 or o.dtype not in (torch.bfloat16, torch.float16):
        raise RuntimeError(f"o must be a bfloat16/float16 [H, L, 128] tensor, got {o.dtype} {tuple(o.shape)}")
    H, L = o.shape[0], o.shape[1]
    rows = L - l_offset if rows is None else rows
    E = 0
    if extra is not None:
        extra = _dev_tensor(extra, "extra")
        if extra.dtype != o.dtype or extra.dim() != 2 or extra.shape[0] != rows:
            raise RuntimeError(f"extra must be a {o.dtype} [{rows}, E] tensor, got {extra.dtype} {tuple(extra.shape)}")
        E = extra.shape[1]
    odt = {"f16": torch.float16, "plain": o.dtype, "i8": torch.int8}[out]
    y = torch.empty((rows, H * 128 + E), dtype=odt, device=o.device)
    rs = torch.empty((rows,), dtype=torch.float32, device=o.device) if out != "plain" else None
    with torch.cuda.device(o.device):
        rc = lib.qlinear_heads_gather(kinds[out], _DTYPE_CODE[o.dtype], o.data_ptr(), H, L, 128, l_offset, rows,
                                      extra.data_ptr() if extra is not None else None, E, y.data_ptr(),
                                      rs.data_ptr() if rs is not None else None, _stream_ptr(o.device))
    _check(rc, "heads_gather")
    return y if out == "plain" else (y, rs)
