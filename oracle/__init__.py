"""CPU oracle for the HIP kernels -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker (or as the timed CPU baseline),
never as the thing shipped: the product path (hip_oracles) has no CPU
fallback and fails loudly without its HIP library.

The arithmetic lives in oracle/hipo_ref.c (compiled by oracle/build.py);
this module passes torch CPU tensors to it through ctypes.  Each function
restates the eager semantics of one repro module; see hipo_ref.c for the
reference files it follows.  How each function is pinned (closed forms,
brute force, ATen eager, golden fixtures) is in tests/test_oracle_pins.py.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "_build" / "libhipo_ref.so"

_lib = None

_i64 = ctypes.c_int64
_p = ctypes.c_void_p
_f = ctypes.c_float
_i = ctypes.c_int

_SIGS = {
    "ref_abi_version": (_i, []),
    "ref_max_threads": (_i, []),
    "ref_row_mean_f32": (None, [_p, _p, _i64, _i64, _i]),
    "ref_bias_gelu_nchw_to_nhwc_bf16": (None, [_p, _p, _p, _i64, _i64, _i64, _i, _i]),
    "ref_scaled_masked_softmax_bf16": (None, [_p, _p, _p, _i64, _i64, _i64, _i64, _f, _i]),
    "ref_residual_layernorm_bf16": (None, [_p] * 8 + [_i64, _i64, _f, _i]),
    "ref_rmsnorm_bf16": (None, [_p] * 4 + [_i64, _i64, _f, _i]),
    "ref_batchnorm_train_f32": (None, [_p] * 8 + [_i64, _i64, _i64, _f, _f, _i, _i]),
    "ref_scaled_bias_softmax_bf16": (
        None, [_p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _f, _i]),
    "ref_spatial_mean_nhwc_bf16": (None, [_p, _p, _i64, _i64, _i64, _i]),
    "ref_rmsnorm_ex_bf16": (None, [_p] * 5 + [_i64, _i64, _f, _f, _i, _i]),
    "ref_batchnorm_nhwc_act_pad_bf16": (
        None, [_p] * 8 + [_i64] * 6 + [_f, _f, _f, _i, _i]),
    "ref_batchnorm_nchw_act_mean_bf16": (None, [_p] * 8 + [_i64] * 3 + [_f, _f, _f, _i, _i]),
    "ref_gelu_tanh_bf16": (None, [_p, _p, _i64, _i]),
    "ref_gelu_tanh_f32": (None, [_p, _p, _i64, _i]),
    "ref_transpose_last2": (None, [_p, _p, _i64, _i64, _i64, _i, _i]),
    "ref_row_mean_bf16": (None, [_p, _p, _i64, _i64, _i, _i]),
    "ref_gelu_erf_grad_f32": (None, [_p, _p, _i64, _i]),
    "ref_gelu_erf_bwd_colsum_bf16": (None, [_p] * 4 + [_i64, _i64, _i]),
}

_ACTS = {None: 0, "none": 0, "relu": 1, "silu": 2}


def load():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            from oracle.build import build
            build()
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def default_threads() -> int:
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        return int(env)
    return max(1, min(os.cpu_count() or 1, 16))


def _cpu(t: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    assert t.dtype == dtype, f"expected {dtype}, got {t.dtype}"
    return t.detach().to("cpu").contiguous()


def _th(threads):
    return default_threads() if threads is None else int(threads)


def row_mean(x: torch.Tensor, threads=None) -> torch.Tensor:
    x = _cpu(x, torch.float32)
    rows, cols = x.shape
    out = torch.empty(rows, dtype=torch.float32)
    load().ref_row_mean_f32(x.data_ptr(), out.data_ptr(), rows, cols, _th(threads))
    return out


def bias_gelu_nchw_to_nhwc(x, bias, *, round_t: bool = True, threads=None):
    x = _cpu(x, torch.bfloat16)
    bias = _cpu(bias, torch.bfloat16)
    n, c, h, w = x.shape
    out = torch.empty((n, c, h, w), dtype=torch.bfloat16, memory_format=torch.channels_last)
    load().ref_bias_gelu_nchw_to_nhwc_bf16(x.data_ptr(), bias.data_ptr(), out.data_ptr(),
                                           n, c, h * w, 1 if round_t else 0, _th(threads))
    return out


def scaled_masked_softmax(x, mask, scale: float, threads=None):
    x = _cpu(x, torch.bfloat16)
    mask = _cpu(mask, torch.bfloat16)
    b, q, k = x.shape
    assert tuple(mask.shape) == (q, k)
    out = torch.empty_like(x)
    load().ref_scaled_masked_softmax_bf16(x.data_ptr(), mask.data_ptr(), out.data_ptr(),
                                          b, q, k, k, float(scale), _th(threads))
    return out


def residual_layernorm(x, residual, gamma, beta, eps: float, threads=None):
    x, residual = _cpu(x, torch.bfloat16), _cpu(residual, torch.bfloat16)
    gamma, beta = _cpu(gamma, torch.bfloat16), _cpu(beta, torch.bfloat16)
    rows, cols = x.shape
    h, y = torch.empty_like(x), torch.empty_like(x)
    mean = torch.empty(rows, dtype=torch.float32)
    rstd = torch.empty(rows, dtype=torch.float32)
    load().ref_residual_layernorm_bf16(
        x.data_ptr(), residual.data_ptr(), gamma.data_ptr(), beta.data_ptr(),
        h.data_ptr(), y.data_ptr(), mean.data_ptr(), rstd.data_ptr(),
        rows, cols, float(eps), _th(threads))
    return h, y, mean, rstd


def rmsnorm(x, gamma, eps: float, threads=None):
    x, gamma = _cpu(x, torch.bfloat16), _cpu(gamma, torch.bfloat16)
    rows, cols = x.shape
    y = torch.empty_like(x)
    rstd = torch.empty(rows, dtype=torch.float32)
    load().ref_rmsnorm_bf16(x.data_ptr(), gamma.data_ptr(), y.data_ptr(), rstd.data_ptr(),
                            rows, cols, float(eps), _th(threads))
    return y, rstd


def batchnorm_train(x, gamma, beta, running_mean, running_var, *, momentum: float,
                    eps: float, relu: bool = True, threads=None):
    """Returns (y, save_mean, save_invstd, running_mean', running_var').

    The running statistics are updated on CPU copies, which are returned.
    """
    x = _cpu(x, torch.float32)
    gamma, beta = _cpu(gamma, torch.float32), _cpu(beta, torch.float32)
    rm = _cpu(running_mean, torch.float32).clone()
    rv = _cpu(running_var, torch.float32).clone()
    n, c, h, w = x.shape
    y = torch.empty_like(x)
    sm = torch.empty(c, dtype=torch.float32)
    si = torch.empty(c, dtype=torch.float32)
    load().ref_batchnorm_train_f32(
        x.data_ptr(), gamma.data_ptr(), beta.data_ptr(), rm.data_ptr(), rv.data_ptr(),
        y.data_ptr(), sm.data_ptr(), si.data_ptr(), n, c, h * w,
        float(momentum), float(eps), 1 if relu else 0, _th(threads))
    return y, sm, si, rm, rv


def scaled_bias_softmax(x, bias, scale: float, heads: int, threads=None):
    """softmax(x * scale + bias[b / heads]) for x [B, Q, K], bias [B / heads, Q, K]."""
    x = _cpu(x, torch.bfloat16)
    bias = _cpu(bias, torch.bfloat16)
    b, q, k = x.shape
    assert b % heads == 0 and tuple(bias.shape) == (b // heads, q, k)
    out = torch.empty_like(x)
    load().ref_scaled_bias_softmax_bf16(x.data_ptr(), bias.data_ptr(), out.data_ptr(),
                                        b, q, k, k, q * k, heads, float(scale), _th(threads))
    return out


def spatial_mean_nhwc(x, threads=None):
    """Mean over H, W of a bf16 [N, C, H, W] tensor -> [N, C, 1, 1]."""
    assert x.dtype == torch.bfloat16
    n, c, h, w = x.shape
    xl = x.detach().to("cpu").contiguous(memory_format=torch.channels_last)
    out = torch.empty((n, c, 1, 1), dtype=torch.bfloat16)
    load().ref_spatial_mean_nhwc_bf16(xl.data_ptr(), out.data_ptr(), n, h * w, c, _th(threads))
    return out


def rmsnorm_ex(x, gamma, eps: float, *, residual=None, scale: float = 1.0, mode: int = 0,
               threads=None):
    """(y, rstd) of the RMSNorm with an optional residual, scale and rounding
    order (mode 0: torch rms_norm, mode 1: HF T5)."""
    x, gamma = _cpu(x, torch.bfloat16), _cpu(gamma, torch.bfloat16)
    res = None if residual is None else _cpu(residual, torch.bfloat16)
    rows, cols = x.shape
    y = torch.empty_like(x)
    rstd = torch.empty(rows, dtype=torch.float32)
    load().ref_rmsnorm_ex_bf16(x.data_ptr(), None if res is None else res.data_ptr(),
                               gamma.data_ptr(), y.data_ptr(), rstd.data_ptr(), rows, cols,
                               float(eps), float(scale), int(mode), _th(threads))
    return y, rstd


def _bn_params(c, gamma, beta, running_mean, running_var):
    gamma, beta = _cpu(gamma, torch.float32), _cpu(beta, torch.float32)
    rm = _cpu(running_mean, torch.float32).clone()
    rv = _cpu(running_var, torch.float32).clone()
    assert gamma.numel() == beta.numel() == rm.numel() == rv.numel() == c
    return gamma, beta, rm, rv


def batchnorm_nhwc_act_pad(x, gamma, beta, running_mean, running_var, *, momentum: float,
                           eps: float, var_scale: float, act=None, pad_bottom: int = 0,
                           pad_right: int = 0, threads=None):
    """bf16 BatchNorm-train + activation + bottom/right zero pad.  Returns
    (save_mean [1,C,1,1], save_rstd [1,C,1,1], out channels-last, rm', rv')."""
    assert x.dtype == torch.bfloat16
    n, c, h, w = x.shape
    xl = x.detach().to("cpu").contiguous(memory_format=torch.channels_last)
    gamma, beta, rm, rv = _bn_params(c, gamma, beta, running_mean, running_var)
    out = torch.empty((n, c, h + pad_bottom, w + pad_right), dtype=torch.bfloat16,
                      memory_format=torch.channels_last)
    sm = torch.empty((1, c, 1, 1), dtype=torch.float32)
    sr = torch.empty((1, c, 1, 1), dtype=torch.float32)
    load().ref_batchnorm_nhwc_act_pad_bf16(
        xl.data_ptr(), gamma.data_ptr(), beta.data_ptr(), rm.data_ptr(), rv.data_ptr(),
        sm.data_ptr(), sr.data_ptr(), out.data_ptr(), n, h, w, c, int(pad_bottom),
        int(pad_right), float(momentum), float(eps), float(var_scale), _ACTS[act], _th(threads))
    return sm, sr, out, rm, rv


def batchnorm_nchw_act_mean(x, gamma, beta, running_mean, running_var, *, momentum: float,
                            eps: float, var_scale: float, act=None, threads=None):
    """bf16 NCHW BatchNorm-train + activation + mean over H, W.  Returns
    (save_mean [1,C,1,1], save_rstd [1,C,1,1], out [N, C], rm', rv')."""
    x = _cpu(x, torch.bfloat16)
    n, c, h, w = x.shape
    gamma, beta, rm, rv = _bn_params(c, gamma, beta, running_mean, running_var)
    out = torch.empty((n, c), dtype=torch.bfloat16)
    sm = torch.empty((1, c, 1, 1), dtype=torch.float32)
    sr = torch.empty((1, c, 1, 1), dtype=torch.float32)
    load().ref_batchnorm_nchw_act_mean_bf16(
        x.data_ptr(), gamma.data_ptr(), beta.data_ptr(), rm.data_ptr(), rv.data_ptr(),
        sm.data_ptr(), sr.data_ptr(), out.data_ptr(), n, c, h * w, float(momentum),
        float(eps), float(var_scale), _ACTS[act], _th(threads))
    return sm, sr, out, rm, rv


def gelu_tanh(x, threads=None):
    """GELU(tanh) of a bf16 or fp32 tensor, evaluated in fp64 and rounded
    once; same shape, contiguous."""
    assert x.dtype in (torch.bfloat16, torch.float32), x.dtype
    x = x.detach().to("cpu").contiguous()
    y = torch.empty_like(x)
    fn = load().ref_gelu_tanh_bf16 if x.dtype == torch.bfloat16 else load().ref_gelu_tanh_f32
    fn(x.data_ptr(), y.data_ptr(), x.numel(), _th(threads))
    return y


def transpose_last2(x, threads=None):
    """x.transpose(-2, -1) made contiguous, element bits copied."""
    x = x.detach().to("cpu").contiguous()
    *lead, rows, cols = x.shape
    y = torch.empty((*lead, cols, rows), dtype=x.dtype)
    batch = 1
    for d in lead:
        batch *= d
    load().ref_transpose_last2(x.data_ptr(), y.data_ptr(), batch, rows, cols,
                               x.element_size(), _th(threads))
    return y


def row_mean_bf16(x, *, relu: bool = False, threads=None):
    """bf16 mean over the last dim of a 2-D bf16 tensor (of relu(x) with
    relu=True), fp64 sum, one rounding -> [rows]."""
    x = _cpu(x, torch.bfloat16)
    rows, cols = x.shape
    out = torch.empty(rows, dtype=torch.bfloat16)
    load().ref_row_mean_bf16(x.data_ptr(), out.data_ptr(), rows, cols, 1 if relu else 0,
                             _th(threads))
    return out


def gelu_erf_grad(x, threads=None):
    """The fp32 derivative of GELU(erf), Phi(t) + t phi(t), of every element
    of a bf16 tensor: fp64, one rounding; same shape."""
    x = _cpu(x, torch.bfloat16)
    d = torch.empty(x.shape, dtype=torch.float32)
    load().ref_gelu_erf_grad_f32(x.data_ptr(), d.data_ptr(), x.numel(), _th(threads))
    return d


def gelu_erf_bwd_colsum(grad, x, threads=None):
    """(y, colsum) of the GELU(erf) backward + column sum graph for 2-D bf16
    grad and x: y = bf16(grad * d(x)) with the fp32 d above, colsum =
    bf16(fp64 sum over rows of y) as fp32."""
    grad = _cpu(grad, torch.bfloat16)
    x = _cpu(x, torch.bfloat16)
    assert grad.shape == x.shape and x.dim() == 2, (grad.shape, x.shape)
    rows, cols = x.shape
    y = torch.empty((rows, cols), dtype=torch.bfloat16)
    colsum = torch.empty(cols, dtype=torch.float32)
    load().ref_gelu_erf_bwd_colsum_bf16(grad.data_ptr(), x.data_ptr(), y.data_ptr(),
                                        colsum.data_ptr(), rows, cols, _th(threads))
    return y, colsum
