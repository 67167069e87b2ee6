"""MI355X (gfx950) kernel library for better-benchmark's oracle API.

`libhip_oracles.so` (built by hip_oracles/build.py from csrc/*.hip) exports
the C ABI declared in include/hip_oracles.h.  This module opens it with
ctypes and wraps each entry point in a torch-facing function that checks
the operands on the host, allocates outputs with torch, and launches on
torch's current HIP stream (so calls are capturable by torch.cuda.graph).

There is no fallback: if the library is missing or a tensor is not on a
ROCm device, the wrappers raise.
"""
from __future__ import annotations

import ctypes
import re
import threading
import weakref
from pathlib import Path

import torch  # imported before the .so so the process has one HIP runtime

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "libhip_oracles.so"
HEADER_PATH = PKG_DIR.parents[1] / "include" / "hip_oracles.h"
ABI_VERSION = 4

_c_i64 = ctypes.c_int64
_c_ptr = ctypes.c_void_p
_c_f32 = ctypes.c_float

# Signatures of every exported symbol (mirrors include/hip_oracles.h).
_SIGNATURES = {
    "hipo_abi_version": (ctypes.c_int, []),
    "hipo_last_error": (ctypes.c_char_p, []),
    "hipo_row_mean_f32": (ctypes.c_int, [_c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_ptr]),
    "hipo_bias_gelu_nchw_to_nhwc_bf16": (
        ctypes.c_int, [_c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_ptr]),
    "hipo_scaled_masked_softmax_bf16": (
        ctypes.c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_f32, _c_ptr]),
    "hipo_residual_layernorm_bf16": (
        ctypes.c_int,
        [_c_ptr] * 8 + [_c_i64, _c_i64, _c_f32, _c_ptr]),
    "hipo_rmsnorm_bf16": (
        ctypes.c_int, [_c_ptr] * 4 + [_c_i64, _c_i64, _c_f32, _c_ptr]),
    "hipo_rmsnorm_ex_bf16": (
        ctypes.c_int, [_c_ptr] * 6 + [_c_i64, _c_i64, _c_f32, _c_f32, ctypes.c_int, _c_ptr]),
    "hipo_scaled_bias_softmax_bf16": (
        ctypes.c_int,
        [_c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_f32,
         _c_ptr]),
    "hipo_spatial_mean_workspace_bytes": (ctypes.c_size_t, [_c_i64, _c_i64, _c_i64]),
    "hipo_spatial_mean_nhwc_bf16": (
        ctypes.c_int, [_c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_ptr, ctypes.c_size_t, _c_ptr]),
    "hipo_batchnorm_nhwc_workspace_bytes": (ctypes.c_size_t, [_c_i64] * 4),
    "hipo_batchnorm_nhwc_act_pad_bf16": (
        ctypes.c_int,
        [_c_ptr] * 8 + [_c_i64] * 6 + [_c_f32] * 3 + [ctypes.c_int, _c_ptr, ctypes.c_size_t,
                                                   _c_ptr]),
    "hipo_batchnorm_nchw_mean_workspace_bytes": (ctypes.c_size_t, [_c_i64] * 3),
    "hipo_batchnorm_nchw_act_mean_bf16": (
        ctypes.c_int,
        [_c_ptr] * 8 + [_c_i64] * 3 + [_c_f32] * 3 + [ctypes.c_int, _c_ptr, ctypes.c_size_t,
                                                   _c_ptr]),
    "hipo_batchnorm_workspace_bytes": (ctypes.c_size_t, [_c_i64, _c_i64, _c_i64]),
    "hipo_batchnorm_train_fwd_f32": (
        ctypes.c_int,
        [_c_ptr] * 8 + [_c_i64, _c_i64, _c_i64, _c_f32, _c_f32, ctypes.c_int,
                        _c_ptr, ctypes.c_size_t, _c_ptr]),
    "hipo_batchnorm_noalloc_error": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(ctypes.c_uint32),
                                                    ctypes.c_int]),
    "hipo_flat_copy": (ctypes.c_int, [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr]),
    "hipo_flat_copy2": (ctypes.c_int, [_c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_ptr]),
    "hipo_hold_copy_f32": (ctypes.c_int, [_c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, _c_ptr]),
    "hipo_gelu_tanh_bf16": (ctypes.c_int, [_c_ptr, _c_ptr, _c_i64, _c_ptr]),
    "hipo_gelu_tanh_f32": (ctypes.c_int, [_c_ptr, _c_ptr, _c_i64, _c_ptr]),
    "hipo_transpose_last2": (
        ctypes.c_int, [_c_ptr, _c_ptr, _c_i64, _c_i64, _c_i64, ctypes.c_int, _c_ptr]),
    "hipo_row_mean_bf16": (ctypes.c_int, [_c_ptr, _c_ptr, _c_i64, _c_i64, ctypes.c_int, _c_ptr]),
    "hipo_gelu_erf_bwd_colsum_workspace_bytes": (ctypes.c_size_t, [_c_i64, _c_i64]),
    "hipo_gelu_erf_bwd_colsum_bf16": (
        ctypes.c_int, [_c_ptr] * 4 + [_c_i64, _c_i64, _c_ptr, ctypes.c_size_t, _c_ptr]),
    "hipo_batchnorm_train_fwd_f32_noalloc": (
        ctypes.c_int,
        [_c_ptr] * 8 + [_c_i64, _c_i64, _c_i64, _c_f32, _c_f32, ctypes.c_int, _c_ptr]),
}

_lib = None
_lib_lock = threading.Lock()


class HipOraclesUnavailable(RuntimeError):
    """libhip_oracles.so is missing or unusable."""


def header_symbols(header: Path = HEADER_PATH) -> list[str]:
    """Names of the functions include/hip_oracles.h declares."""
    text = header.read_text()
    return sorted(set(re.findall(r"\b(hipo_[a-z0-9_]+)\s*\(", text)))


def load_library(path: str | Path | None = None):
    """Open (once) and return the ctypes handle; raises if unavailable."""
    global _lib
    with _lib_lock:
        if _lib is not None and path is None:
            return _lib
        p = Path(path) if path is not None else LIB_PATH
        if not p.exists():
            raise HipOraclesUnavailable(
                f"{p} not found: build it with "
                f"`python better-benchmark_amd/hip_oracles/build.py` "
                f"(or __graft_entry__.build())")
        lib = ctypes.CDLL(str(p))
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        got = lib.hipo_abi_version()
        if got != ABI_VERSION:
            raise HipOraclesUnavailable(
                f"{p}: ABI version {got}, expected {ABI_VERSION}")
        if path is None:
            _lib = lib
        return lib


def _check(rc: int, what: str) -> None:
    if rc != 0:
        msg = _lib.hipo_last_error().decode(errors="replace") if _lib else ""
        raise RuntimeError(f"hip_oracles.{what} failed (code {rc}): {msg}")


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _require_rocm(*tensors: torch.Tensor) -> torch.device:
    dev = tensors[0].device
    for t in tensors:
        _require(isinstance(t, torch.Tensor), "expected tensors")
        _require(t.device.type == "cuda",
                 f"hip_oracles runs on the ROCm device only, got a {t.device} tensor")
        _require(t.device == dev, "all operands must be on one device")
    _require(torch.version.hip is not None, "torch is not a ROCm build")
    return dev


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


# ---------------------------------------------------------------------------
# Op wrappers
# ---------------------------------------------------------------------------

def row_mean(x: torch.Tensor) -> torch.Tensor:
    """fp32 mean over the last dim of a 2-D fp32 tensor -> [rows]."""
    lib = load_library()
    dev = _require_rocm(x)
    _require(x.dtype == torch.float32 and x.dim() == 2, "row_mean: x must be 2-D fp32")
    _require(x.stride(1) == 1 or x.shape[1] <= 1, "row_mean: last dim must be contiguous")
    rows, cols = x.shape
    out = torch.empty(rows, dtype=torch.float32, device=dev)
    row_stride = x.stride(0) if rows > 1 else cols
    with torch.cuda.device(dev):
        _check(lib.hipo_row_mean_f32(_ptr(x), _ptr(out), rows, cols,
                                     max(row_stride, cols), _stream(dev)),
               "row_mean")
    return out


def bias_gelu_nchw_to_nhwc(x: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    """gelu_tanh(x + bias[None,:,None,None]) written channels-last (bf16)."""
    lib = load_library()
    dev = _require_rocm(x, bias)
    _require(x.dtype == torch.bfloat16 and bias.dtype == torch.bfloat16,
             "bias_gelu: bf16 operands required")
    _require(x.dim() == 4 and x.is_contiguous(), "bias_gelu: x must be contiguous NCHW")
    n, c, h, w = x.shape
    _require(bias.shape == (c,) and bias.is_contiguous(), "bias_gelu: bias must be [C]")
    out = torch.empty((n, c, h, w), dtype=torch.bfloat16, device=dev,
                      memory_format=torch.channels_last)
    with torch.cuda.device(dev):
        _check(lib.hipo_bias_gelu_nchw_to_nhwc_bf16(_ptr(x), _ptr(bias), _ptr(out),
                                                    n, c, h * w, _stream(dev)),
               "bias_gelu_nchw_to_nhwc")
    return out


def gelu_tanh(x: torch.Tensor) -> torch.Tensor:
    """0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))) of a contiguous bf16
    or fp32 tensor, same shape: bf16 correctly rounded per element, fp32 as
    x / (1 + e^(-2u)) to a few ulps."""
    lib = load_library()
    dev = _require_rocm(x)
    _require(x.dtype in (torch.bfloat16, torch.float32), "gelu_tanh: bf16 or fp32 x required")
    _require(x.is_contiguous(), "gelu_tanh: x must be contiguous")
    y = torch.empty_like(x, memory_format=torch.contiguous_format)
    fn = lib.hipo_gelu_tanh_bf16 if x.dtype == torch.bfloat16 else lib.hipo_gelu_tanh_f32
    with torch.cuda.device(dev):
        _check(fn(_ptr(x), _ptr(y), x.numel(), _stream(dev)), "gelu_tanh")
    return y


def transpose_last2(x: torch.Tensor) -> torch.Tensor:
    """x.transpose(-2, -1).contiguous() for a contiguous tensor of >= 2 dims
    with 2- or 4-byte elements, moved bit for bit."""
    lib = load_library()
    dev = _require_rocm(x)
    _require(x.dim() >= 2 and x.is_contiguous(), "transpose_last2: contiguous x, >= 2 dims")
    _require(x.element_size() in (2, 4), "transpose_last2: 2- or 4-byte elements required")
    *lead, rows, cols = x.shape
    y = torch.empty((*lead, cols, rows), dtype=x.dtype, device=dev)
    batch = 1
    for d in lead:
        batch *= d
    with torch.cuda.device(dev):
        _check(lib.hipo_transpose_last2(_ptr(x), _ptr(y), batch, rows, cols,
                                        x.element_size(), _stream(dev)), "transpose_last2")
    return y


def row_mean_bf16(x: torch.Tensor, *, relu: bool = False) -> torch.Tensor:
    """bf16 mean over the last dim of a contiguous 2-D bf16 tensor (fp32 sum,
    one rounding), of relu(x) with relu=True -> [rows] bf16."""
    lib = load_library()
    dev = _require_rocm(x)
    _require(x.dtype == torch.bfloat16 and x.dim() == 2 and x.is_contiguous(),
             "row_mean_bf16: x must be contiguous 2-D bf16")
    rows, cols = x.shape
    _require(cols >= 1 or rows == 0, "row_mean_bf16: mean over zero elements")
    out = torch.empty(rows, dtype=torch.bfloat16, device=dev)
    with torch.cuda.device(dev):
        _check(lib.hipo_row_mean_bf16(_ptr(x), _ptr(out), rows, cols, 1 if relu else 0,
                                      _stream(dev)), "row_mean_bf16")
    return out


def gelu_erf_bwd_colsum(grad: torch.Tensor, x: torch.Tensor):
    """GELU(erf) backward and its column sum for contiguous 2-D bf16 grad and
    x [rows, cols] (cols a multiple of 8): y = bf16(grad * d(x)) with d the
    correctly rounded fp32 GELU'(x), and colsum = bf16(sum over rows of y)
    as fp32.  Returns (y [rows, cols] bf16, colsum [cols] fp32)."""
    lib = load_library()
    dev = _require_rocm(grad, x)
    _require(grad.dtype == torch.bfloat16 and x.dtype == torch.bfloat16,
             "gelu_erf_bwd: bf16 operands required")
    _require(grad.dim() == 2 and grad.shape == x.shape and grad.is_contiguous()
             and x.is_contiguous(), "gelu_erf_bwd: grad and x must be contiguous [rows, cols]")
    rows, cols = x.shape
    _require(cols % 8 == 0, "gelu_erf_bwd: cols must be a multiple of 8")
    y = torch.empty((rows, cols), dtype=torch.bfloat16, device=dev)
    colsum = torch.empty(cols, dtype=torch.float32, device=dev)
    need = int(lib.hipo_gelu_erf_bwd_colsum_workspace_bytes(rows, cols))
    ws = torch.empty(need, dtype=torch.uint8, device=dev) if need else None
    with torch.cuda.device(dev):
        _check(lib.hipo_gelu_erf_bwd_colsum_bf16(
            _ptr(grad), _ptr(x), _ptr(y), _ptr(colsum), rows, cols,
            None if ws is None else _ptr(ws), need, _stream(dev)), "gelu_erf_bwd_colsum")
    return y, colsum


def scaled_masked_softmax(x: torch.Tensor, mask: torch.Tensor, scale: float) -> torch.Tensor:
    """softmax(x * scale + mask, -1) for bf16 x [B, Q, K], mask [Q, K]."""
    lib = load_library()
    dev = _require_rocm(x, mask)
    _require(x.dtype == torch.bfloat16 and mask.dtype == torch.bfloat16,
             "masked_softmax: bf16 operands required")
    _require(x.dim() == 3 and x.is_contiguous(), "masked_softmax: x must be contiguous [B,Q,K]")
    b, q, k = x.shape
    _require(mask.dim() == 2 and tuple(mask.shape) == (q, k) and mask.stride(1) == 1,
             "masked_softmax: mask must be [Q, K] with unit inner stride")
    if q > 1 and mask.stride(0) < k:
        # Rows that overlap (a mask broadcast over Q): the kernel addresses
        # row q at q * row_stride and needs row_stride >= K.
        mask = mask.contiguous()
    mstride = mask.stride(0) if q > 1 else k
    out = torch.empty_like(x)
    with torch.cuda.device(dev):
        _check(lib.hipo_scaled_masked_softmax_bf16(_ptr(x), _ptr(mask), _ptr(out),
                                                   b, q, k, mstride,
                                                   float(scale), _stream(dev)),
               "scaled_masked_softmax")
    return out


# bf16 zeros [K] per (device, K): the mask row of softmax_lastdim.
_zero_rows: dict = {}


def softmax_lastdim(x: torch.Tensor) -> torch.Tensor:
    """softmax(x, -1) of a contiguous bf16 tensor (fp32 max, exp, sum and
    division, bf16 out): hipo_scaled_masked_softmax_bf16 over [rows, 1, K]
    with scale 1 and one zero mask row (s = fma(x, 1, 0) = x exactly).  The
    zero row is allocated on a device's first call with that K, which
    therefore must not be inside a graph capture."""
    lib = load_library()
    dev = _require_rocm(x)
    _require(x.dtype == torch.bfloat16, "softmax: bf16 operand required")
    _require(x.dim() >= 1 and x.is_contiguous(), "softmax: x must be contiguous")
    k = x.shape[-1]
    out = torch.empty_like(x)
    if x.numel() == 0:
        return out
    key = (dev.index, k)
    zero = _zero_rows.get(key)
    if zero is None:
        _require(not torch.cuda.is_current_stream_capturing(),
                 "softmax: the first call for this K must run outside graph capture")
        zero = _zero_rows[key] = torch.zeros(k, dtype=torch.bfloat16, device=dev)
    with torch.cuda.device(dev):
        _check(lib.hipo_scaled_masked_softmax_bf16(_ptr(x), _ptr(zero), _ptr(out),
                                                   x.numel() // k, 1, k, k, 1.0,
                                                   _stream(dev)),
               "softmax_lastdim")
    return out


def residual_layernorm(x, residual, gamma, beta, eps: float, *, outputs: str = "all"):
    """(h, y, mean, rstd) of LayerNorm(x + residual) over the last dim;
    outputs="y" returns y alone and writes nothing else, outputs="hy"
    returns (h, y) and writes no statistics."""
    lib = load_library()
    dev = _require_rocm(x, residual, gamma, beta)
    for t in (x, residual, gamma, beta):
        _require(t.dtype == torch.bfloat16 and t.is_contiguous(),
                 "residual_layernorm: contiguous bf16 operands required")
    _require(x.dim() == 2 and residual.shape == x.shape, "residual_layernorm: x, residual [R, C]")
    rows, cols = x.shape
    _require(gamma.shape == (cols,) and beta.shape == (cols,), "residual_layernorm: gamma/beta [C]")
    _require(outputs in ("all", "y", "hy"),
             "residual_layernorm: outputs must be 'all', 'y' or 'hy'")
    y = torch.empty_like(x)
    if outputs == "all":
        h = torch.empty_like(x)
        mean = torch.empty(rows, dtype=torch.float32, device=dev)
        rstd = torch.empty(rows, dtype=torch.float32, device=dev)
        ptrs = (_ptr(h), _ptr(mean), _ptr(rstd))
    elif outputs == "hy":
        h = torch.empty_like(x)
        ptrs = (_ptr(h), None, None)
    else:
        ptrs = (None, None, None)
    with torch.cuda.device(dev):
        _check(lib.hipo_residual_layernorm_bf16(
            _ptr(x), _ptr(residual), _ptr(gamma), _ptr(beta), ptrs[0], _ptr(y),
            ptrs[1], ptrs[2], rows, cols, float(eps), _stream(dev)),
            "residual_layernorm")
    if outputs == "all":
        return h, y, mean, rstd
    return (h, y) if outputs == "hy" else y


def rmsnorm(x, gamma, eps: float):
    """(y, rstd) of RMSNorm(x) over the last dim."""
    lib = load_library()
    dev = _require_rocm(x, gamma)
    for t in (x, gamma):
        _require(t.dtype == torch.bfloat16 and t.is_contiguous(),
                 "rmsnorm: contiguous bf16 operands required")
    _require(x.dim() == 2, "rmsnorm: x must be [R, C]")
    rows, cols = x.shape
    _require(gamma.shape == (cols,), "rmsnorm: gamma must be [C]")
    y = torch.empty_like(x)
    rstd = torch.empty(rows, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _check(lib.hipo_rmsnorm_bf16(_ptr(x), _ptr(gamma), _ptr(y), _ptr(rstd),
                                     rows, cols, float(eps), _stream(dev)),
               "rmsnorm")
    return y, rstd


def rmsnorm_ex(x, gamma, eps: float, *, residual=None, scale: float = 1.0, mode: int = 0,
               want_rstd: bool = False, want_h: bool = False):
    """RMSNorm over the last dim with an optional residual (h = bf16(x + r)),
    an output scale and the eager rounding order: mode 0 = torch rms_norm
    (one rounding), mode 1 = HF T5 (bf16(h*rstd), then *gamma, then *scale,
    each rounded).  Returns y, or (y, rstd) with want_rstd; with want_h
    (needs a residual) h comes first: (h, y) or (h, y, rstd)."""
    lib = load_library()
    ops = (x, gamma) if residual is None else (x, gamma, residual)
    dev = _require_rocm(*ops)
    for t in ops:
        _require(t.dtype == torch.bfloat16 and t.is_contiguous(),
                 "rmsnorm_ex: contiguous bf16 operands required")
    _require(x.dim() == 2, "rmsnorm_ex: x must be [R, C]")
    rows, cols = x.shape
    _require(gamma.shape == (cols,), "rmsnorm_ex: gamma must be [C]")
    _require(residual is None or residual.shape == x.shape, "rmsnorm_ex: residual [R, C]")
    _require(mode in (0, 1), "rmsnorm_ex: mode must be 0 or 1")
    _require(not want_h or residual is not None, "rmsnorm_ex: h needs a residual")
    y = torch.empty_like(x)
    h = torch.empty_like(x) if want_h else None
    rstd = torch.empty(rows, dtype=torch.float32, device=dev) if want_rstd else None
    with torch.cuda.device(dev):
        _check(lib.hipo_rmsnorm_ex_bf16(
            _ptr(x), None if residual is None else _ptr(residual), _ptr(gamma),
            None if h is None else _ptr(h), _ptr(y), None if rstd is None else _ptr(rstd),
            rows, cols, float(eps), float(scale), int(mode), _stream(dev)), "rmsnorm_ex")
    out = (y, rstd) if want_rstd else (y,)
    out = ((h,) + out) if want_h else out
    return out if len(out) > 1 else out[0]


def scaled_bias_softmax(x, bias, scale: float, heads: int):
    """softmax(x * scale + bias, -1) for bf16 x [B, Q, K] and a bias
    [B / heads, Q, K] (any layout with unit inner stride and 8-aligned row and
    batch strides) shared by `heads` consecutive batch entries."""
    lib = load_library()
    dev = _require_rocm(x, bias)
    _require(x.dtype == torch.bfloat16 and bias.dtype == torch.bfloat16,
             "bias_softmax: bf16 operands required")
    _require(x.dim() == 3 and x.is_contiguous(), "bias_softmax: x must be contiguous [B,Q,K]")
    b, q, k = x.shape
    _require(heads >= 1 and b % heads == 0, "bias_softmax: heads must divide the batch")
    _require(bias.dim() == 3 and tuple(bias.shape) == (b // heads, q, k) and bias.stride(2) == 1,
             "bias_softmax: bias must be [B / heads, Q, K] with unit inner stride")
    if q > 1 and bias.stride(1) < k:
        bias = bias.contiguous()  # rows that overlap: the kernel needs row stride >= K
    rs = bias.stride(1) if q > 1 else k
    bs = bias.stride(0) if b // heads > 1 else 0
    out = torch.empty_like(x)
    with torch.cuda.device(dev):
        _check(lib.hipo_scaled_bias_softmax_bf16(_ptr(x), _ptr(bias), _ptr(out), b, q, k,
                                                 rs, bs, heads, float(scale),
                                                 _stream(dev)),
               "scaled_bias_softmax")
    return out


def spatial_mean_nhwc(x, keepdim: bool = True):
    """Mean over H, W of a channels-last bf16 [N, C, H, W] tensor ->
    [N, C, 1, 1] (keepdim) or [N, C], contiguous bf16."""
    lib = load_library()
    dev = _require_rocm(x)
    _require(x.dtype == torch.bfloat16 and x.dim() == 4, "spatial_mean: bf16 NCHW tensor")
    n, c, h, w = x.shape
    _require(x.is_contiguous(memory_format=torch.channels_last),
             "spatial_mean: x must be stored channels-last")
    out = torch.empty((n, c, 1, 1) if keepdim else (n, c), dtype=torch.bfloat16, device=dev)
    need = int(lib.hipo_spatial_mean_workspace_bytes(n, h * w, c))
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=dev) if need else None
    with torch.cuda.device(dev):
        _check(lib.hipo_spatial_mean_nhwc_bf16(_ptr(x), _ptr(out), n, h * w, c,
                                               None if ws is None else _ptr(ws), need,
                                               _stream(dev)),
               "spatial_mean_nhwc")
    return out


def batchnorm_workspace_bytes(n: int, c: int, hw: int) -> int:
    return int(load_library().hipo_batchnorm_workspace_bytes(n, c, hw))


# One zero-filled BatchNorm workspace per device, kept for the process: the
# single-pass kernel keeps its exchange state (completion count, epoch,
# tagged slots) there between calls, so it must start zeroed and must not be
# handed to two calls that can run at the same time.  A workspace that is
# replaced by a larger one is retired, never freed: a hipGraph captured
# earlier holds its raw address (ctypes keeps no reference to the tensor),
# and its replays keep using it, with their own epoch state, safely.
_bn_workspaces: dict[int, torch.Tensor] = {}
_bn_retired: dict[int, list[torch.Tensor]] = {}
# Caller-provided workspaces seen by batchnorm_train, so their error words are
# checked too (weak: the caller owns them).
_bn_caller_workspaces: "weakref.WeakValueDictionary[int, torch.Tensor]" = (
    weakref.WeakValueDictionary())
_bn_ws_lock = threading.Lock()

# Byte offset of the sticky error word in a BatchNorm workspace.
BN_ERROR_WORD_OFFSET = 8


class HipOraclesDeviceFault(RuntimeError):
    """A kernel reported a fault through its error word (a bounded
    cross-workgroup wait timed out; the affected outputs are NaN)."""


def batchnorm_cached_workspace(dev: torch.device, nbytes: int) -> torch.Tensor:
    """The device's shared workspace, grown (zero-filled) to at least nbytes.
    The workspace it replaces stays allocated for the rest of the process."""
    with _bn_ws_lock:
        ws = _bn_workspaces.get(dev.index)
        if ws is None or ws.numel() < nbytes:
            _require(not torch.cuda.is_current_stream_capturing(),
                     "batchnorm: the workspace is allocated on first use; call once "
                     "outside graph capture (or pass workspace=) before capturing")
            if ws is not None:
                _bn_retired.setdefault(dev.index, []).append(ws)
            ws = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=dev)
            _bn_workspaces[dev.index] = ws
        return ws


def batchnorm_train(x, gamma, beta, running_mean, running_var, *, momentum: float,
                    eps: float, relu: bool = True, workspace: torch.Tensor | None = None):
    """(y, save_mean, save_invstd); running_mean/var are updated in place.

    workspace: zero-filled uint8 device memory of at least
    batchnorm_workspace_bytes(n, c, h*w) bytes, reused unmodified across calls
    that are ordered on one stream.  Default: the device's shared workspace
    (callers issuing BatchNorm on several streams at once pass their own)."""
    lib = load_library()
    dev = _require_rocm(x, gamma, beta, running_mean, running_var)
    _require(x.dim() == 4 and x.dtype == torch.float32 and x.is_contiguous(),
             "batchnorm: x must be contiguous NCHW fp32")
    n, c, h, w = x.shape
    for t in (gamma, beta, running_mean, running_var):
        _require(t.dtype == torch.float32 and t.shape == (c,) and t.is_contiguous(),
                 "batchnorm: gamma/beta/running stats must be contiguous fp32 [C]")
    need = int(lib.hipo_batchnorm_workspace_bytes(n, c, h * w))
    if workspace is None:
        workspace = batchnorm_cached_workspace(dev, need)
    else:
        _require(workspace.device == dev and workspace.is_contiguous(),
                 "batchnorm: workspace must be contiguous memory on x's device")
        _bn_caller_workspaces[workspace.data_ptr()] = workspace
    _require(workspace.numel() * workspace.element_size() >= need,
             "batchnorm: workspace too small")
    y = torch.empty_like(x)
    save_mean = torch.empty(c, dtype=torch.float32, device=dev)
    save_invstd = torch.empty(c, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _check(lib.hipo_batchnorm_train_fwd_f32(
            _ptr(x), _ptr(gamma), _ptr(beta), _ptr(running_mean), _ptr(running_var),
            _ptr(y), _ptr(save_mean), _ptr(save_invstd), n, c, h * w,
            float(momentum), float(eps), 1 if relu else 0,
            _ptr(workspace), workspace.numel() * workspace.element_size(), _stream(dev)),
            "batchnorm_train")
    return y, save_mean, save_invstd


def flat_copy(src: torch.Tensor, dst: torch.Tensor, read_bytes: int | None = None,
              write_bytes: int | None = None) -> None:
    """Measurement yardstick: read `read_bytes` of src and write `write_bytes`
    of dst in one launch with the oracle kernels' access style (default: all
    of each).  Sizes are multiples of 1024 bytes."""
    lib = load_library()
    dev = _require_rocm(src, dst)
    _require(src.is_contiguous() and dst.is_contiguous(), "flat_copy: contiguous buffers")
    rb = src.numel() * src.element_size() if read_bytes is None else int(read_bytes)
    wb = dst.numel() * dst.element_size() if write_bytes is None else int(write_bytes)
    _require(rb <= src.numel() * src.element_size() and wb <= dst.numel() * dst.element_size(),
             "flat_copy: sizes exceed the buffers")
    with torch.cuda.device(dev):
        _check(lib.hipo_flat_copy(_ptr(src), rb, _ptr(dst), wb, _stream(dev)), "flat_copy")


def flat_copy2(src0: torch.Tensor, src1: torch.Tensor, dst0: torch.Tensor,
               dst1: torch.Tensor) -> None:
    """Measurement yardstick: copy src0 -> dst0 and src1 -> dst1 in one
    launch, four streams in lockstep (the residual LayerNorm's pattern).  All
    four buffers contiguous, the same size, a multiple of 1024 bytes."""
    lib = load_library()
    dev = _require_rocm(src0, src1, dst0, dst1)
    nb = src0.numel() * src0.element_size()
    for t in (src0, src1, dst0, dst1):
        _require(t.is_contiguous() and t.numel() * t.element_size() == nb,
                 "flat_copy2: four contiguous buffers of one size")
    with torch.cuda.device(dev):
        _check(lib.hipo_flat_copy2(_ptr(src0), _ptr(src1), _ptr(dst0), _ptr(dst1), nb,
                                   _stream(dev)), "flat_copy2")


def hold_copy(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """Measurement yardstick: y = x for an fp32 NCHW [N, C, H, W] tensor with
    the single-pass BatchNorm kernel's access pattern (slabs held in
    registers from their loads to their stores, no exchange, no arithmetic
    on the values)."""
    lib = load_library()
    dev = _require_rocm(x)
    _require(x.dtype == torch.float32 and x.dim() == 4 and x.is_contiguous(),
             "hold_copy: a contiguous fp32 [N, C, H, W] tensor required")
    y = torch.empty_like(x) if out is None else out
    _require(y.shape == x.shape and y.dtype == x.dtype and y.is_contiguous(),
             "hold_copy: out must match x")
    n, c, h, w = x.shape
    with torch.cuda.device(dev):
        _check(lib.hipo_hold_copy_f32(_ptr(x), _ptr(y), n, c, h * w, _stream(dev)), "hold_copy")
    return y


_BN_ACTS = {None: 0, "none": 0, "relu": 1, "silu": 2}


def _bn_bf16_params(what, c, dev, gamma, beta, running_mean, running_var):
    for t in (gamma, beta, running_mean, running_var):
        _require(t.device == dev and t.dtype == torch.float32 and t.numel() == c
                 and t.is_contiguous(),
                 f"{what}: gamma/beta/running stats must be contiguous fp32 [C]")


def batchnorm_nhwc_act_pad(x, gamma, beta, running_mean, running_var, *, momentum: float,
                           eps: float, var_scale: float, act: str | None = "silu",
                           pad_bottom: int = 0, pad_right: int = 0):
    """BatchNorm training forward of a channels-last bf16 [N, C, H, W] tensor
    with fp32 statistics, an activation and a zero pad of the bottom/right
    border.  Returns (save_mean [1, C, 1, 1], save_rstd [1, C, 1, 1], out
    [N, C, H + pad_bottom, W + pad_right] channels-last bf16); running_mean
    / running_var are updated in place."""
    lib = load_library()
    dev = _require_rocm(x)
    _require(x.dim() == 4 and x.dtype == torch.bfloat16
             and x.is_contiguous(memory_format=torch.channels_last),
             "batchnorm_nhwc: x must be a channels-last bf16 [N, C, H, W] tensor")
    _require(act in _BN_ACTS, f"batchnorm_nhwc: act must be one of {sorted(map(str, _BN_ACTS))}")
    n, c, h, w = x.shape
    _bn_bf16_params("batchnorm_nhwc", c, dev, gamma, beta, running_mean, running_var)
    out = torch.empty((n, c, h + pad_bottom, w + pad_right), dtype=torch.bfloat16, device=dev,
                      memory_format=torch.channels_last)
    save_mean = torch.empty((1, c, 1, 1), dtype=torch.float32, device=dev)
    save_rstd = torch.empty((1, c, 1, 1), dtype=torch.float32, device=dev)
    need = int(lib.hipo_batchnorm_nhwc_workspace_bytes(n, h, w, c))
    ws = torch.empty(max(need, 16), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        _check(lib.hipo_batchnorm_nhwc_act_pad_bf16(
            _ptr(x), _ptr(gamma), _ptr(beta), _ptr(running_mean), _ptr(running_var),
            _ptr(save_mean), _ptr(save_rstd), _ptr(out), n, h, w, c, int(pad_bottom),
            int(pad_right), float(momentum), float(eps), float(var_scale), _BN_ACTS[act],
            _ptr(ws), ws.numel(), _stream(dev)), "batchnorm_nhwc_act_pad")
    return save_mean, save_rstd, out


def batchnorm_nchw_act_mean(x, gamma, beta, running_mean, running_var, *, momentum: float,
                            eps: float, var_scale: float, act: str | None = "relu"):
    """BatchNorm training forward of a contiguous NCHW bf16 tensor with fp32
    statistics, an activation and the mean over H, W.  Returns (save_mean
    [1, C, 1, 1], save_rstd [1, C, 1, 1], out [N, C] bf16); running_mean /
    running_var are updated in place."""
    lib = load_library()
    dev = _require_rocm(x)
    _require(x.dim() == 4 and x.dtype == torch.bfloat16 and x.is_contiguous(),
             "batchnorm_nchw: x must be a contiguous NCHW bf16 tensor")
    _require(act in _BN_ACTS, f"batchnorm_nchw: act must be one of {sorted(map(str, _BN_ACTS))}")
    n, c, h, w = x.shape
    _bn_bf16_params("batchnorm_nchw", c, dev, gamma, beta, running_mean, running_var)
    out = torch.empty((n, c), dtype=torch.bfloat16, device=dev)
    save_mean = torch.empty((1, c, 1, 1), dtype=torch.float32, device=dev)
    save_rstd = torch.empty((1, c, 1, 1), dtype=torch.float32, device=dev)
    need = int(lib.hipo_batchnorm_nchw_mean_workspace_bytes(n, c, h * w))
    ws = torch.empty(max(need, 16), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        _check(lib.hipo_batchnorm_nchw_act_mean_bf16(
            _ptr(x), _ptr(gamma), _ptr(beta), _ptr(running_mean), _ptr(running_var),
            _ptr(save_mean), _ptr(save_rstd), _ptr(out), n, c, h * w, float(momentum),
            float(eps), float(var_scale), _BN_ACTS[act], _ptr(ws), ws.numel(), _stream(dev)),
            "batchnorm_nchw_act_mean")
    return save_mean, save_rstd, out


def _error_word(ws: torch.Tensor) -> torch.Tensor:
    raw = ws.view(torch.uint8) if ws.dtype != torch.uint8 else ws
    return raw[BN_ERROR_WORD_OFFSET:BN_ERROR_WORD_OFFSET + 4].view(torch.int32)


def _known_workspaces(dev: torch.device | None):
    with _bn_ws_lock:
        found = list(_bn_workspaces.items())
        found += [(d, w) for d, ws in _bn_retired.items() for w in ws]
        found += [(w.device.index, w) for w in list(_bn_caller_workspaces.values())]
    return [w for d, w in found if dev is None or d == dev.index]


def batchnorm_error_flag(dev: torch.device | None = None, *,
                         workspace: torch.Tensor | None = None) -> int:
    """Sticky error word of a BatchNorm workspace: nonzero once an exchange
    wait of the single-pass kernel has timed out (that channel's outputs and
    running statistics are then NaN).  `workspace` selects a caller-provided
    workspace; by default the device's shared one.  Synchronises."""
    if workspace is None:
        d = dev or torch.device("cuda", torch.cuda.current_device())
        workspace = _bn_workspaces.get(d.index)
        if workspace is None:
            return 0
    return int(_error_word(workspace).item())


def device_faults(dev: torch.device | None = None, *, clear: bool = True) -> list[str]:
    """Faults recorded by kernels in every BatchNorm workspace this process has
    used on `dev` (all devices if None): the shared, retired and caller-provided
    ones, and the allocation-free entry point's static scratch array.  With
    `clear`, each reported word is reset to zero, so the next check sees only
    new faults.  Synchronises."""
    out = []
    for ws in _known_workspaces(dev):
        word = _error_word(ws)
        v = int(word.item())
        if v:
            out.append(f"batchnorm_train_fwd_f32: exchange wait timed out "
                       f"(error word {v:#x}, workspace {ws.data_ptr():#x} on {ws.device}); "
                       f"its outputs and running statistics are NaN")
            if clear:
                word.zero_()
    # The allocation-free entry point's static scratch array, per device.
    lib = load_library()
    devices = [dev.index] if dev is not None else range(torch.cuda.device_count())
    for d in devices:
        w = ctypes.c_uint32(0)
        _check(lib.hipo_batchnorm_noalloc_error(int(d), ctypes.byref(w), 1 if clear else 0),
               "batchnorm_noalloc_error")
        if w.value:
            out.append(f"batchnorm_train_fwd_f32_noalloc: exchange wait timed out "
                       f"(error word {w.value:#x} in the static scratch array of cuda:{d}); "
                       f"its outputs and running statistics are NaN")
    return out


def raise_on_device_faults(dev: torch.device | None = None) -> None:
    """Raise HipOraclesDeviceFault if any kernel recorded a fault (see
    device_faults); the words are cleared first."""
    faults = device_faults(dev, clear=True)
    if faults:
        raise HipOraclesDeviceFault("; ".join(faults))


__all__ = [
    "HipOraclesUnavailable", "LIB_PATH", "load_library", "header_symbols",
    "row_mean", "bias_gelu_nchw_to_nhwc", "scaled_masked_softmax",
    "residual_layernorm", "rmsnorm", "rmsnorm_ex", "scaled_bias_softmax", "spatial_mean_nhwc",
    "batchnorm_nhwc_act_pad", "batchnorm_nchw_act_mean",
    "batchnorm_workspace_bytes", "batchnorm_train",
    "batchnorm_cached_workspace", "batchnorm_error_flag", "BN_ERROR_WORD_OFFSET",
    "HipOraclesDeviceFault", "device_faults", "raise_on_device_faults", "flat_copy",
    "flat_copy2",
    "hold_copy",
    "gelu_erf_bwd_colsum",
]
