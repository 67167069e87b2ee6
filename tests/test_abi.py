"""The C-ABI library loads without a GPU and exports exactly what
include/hip_oracles.h declares; host-side argument checks fail with
HIPO_EINVAL and a message before anything is launched (no GPU needed)."""
import ctypes
import subprocess
import sys

import pytest

import hip_oracles

HIPO_EINVAL = 1000


@pytest.fixture(scope="module")
def lib():
    return hip_oracles.load_library()


def test_header_symbols_are_exported(lib):
    declared = hip_oracles.header_symbols()
    assert len(declared) >= 9
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in include/hip_oracles.h but not exported"
    assert set(declared) == set(hip_oracles._SIGNATURES), "ctypes signatures out of sync"


def test_exported_names_match_header():
    out = subprocess.run(["nm", "-D", "--defined-only", str(hip_oracles.LIB_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T hipo_" in line}
    assert exported == set(hip_oracles.header_symbols())


def test_abi_version_and_error_string(lib):
    assert lib.hipo_abi_version() == hip_oracles.ABI_VERSION == 4
    assert lib.hipo_last_error() == b""


@pytest.mark.parametrize("call,msg", [
    (lambda l: l.hipo_row_mean_f32(None, None, -1, 4, 4, None), b"negative"),
    (lambda l: l.hipo_row_mean_f32(None, None, 4, 8, 4, None), b"row_stride"),
    (lambda l: l.hipo_row_mean_f32(None, None, 4, 8, 8, None), b"null"),
    (lambda l: l.hipo_bias_gelu_nchw_to_nhwc_bf16(None, None, None, 2, 8, 8, None), b"null"),
    (lambda l: l.hipo_scaled_masked_softmax_bf16(1, 1, 1, 2, 4, 8, 4, 1.0, None), b"mask_row_stride"),
    (lambda l: l.hipo_residual_layernorm_bf16(None, None, None, None, None, None, None, None,
                                              4, 0, 1e-5, None), b"cols"),
    (lambda l: l.hipo_rmsnorm_bf16(None, None, None, None, -2, 8, 1e-5, None), b"negative"),
    (lambda l: l.hipo_rmsnorm_bf16(1, 1, 1, None, 2, 8, 1e-5, None), b"null"),
    (lambda l: l.hipo_rmsnorm_ex_bf16(1, None, 1, None, 1, None, 2, 8, 1e-5, 1.0, 2, None), b"mode"),
    (lambda l: l.hipo_rmsnorm_ex_bf16(1, None, 1, 1, 1, None, 2, 8, 1e-5, 1.0, 0, None), b"residual"),
    (lambda l: l.hipo_rmsnorm_ex_bf16(None, None, 1, None, 1, None, 2, 8, 1e-5, 1.0, 0, None), b"null"),
    (lambda l: l.hipo_scaled_bias_softmax_bf16(1, 1, 1, 6, 4, 8, 8, 0, 4, 1.0, None), b"heads"),
    (lambda l: l.hipo_scaled_bias_softmax_bf16(1, 1, 1, 6, 4, 8, 8, -8, 3, 1.0, None),
     b"mask_batch_stride"),
    (lambda l: l.hipo_spatial_mean_nhwc_bf16(1, 1, 2, 0, 8, None, 0, None), b"spatial"),
    (lambda l: l.hipo_spatial_mean_nhwc_bf16(16, 16, 64, 4096, 256, None, 0, None), b"workspace"),
    (lambda l: l.hipo_batchnorm_train_fwd_f32(1, 1, 1, 1, 1, 1, 1, 1, 2, 4, 9, 0.1, 1e-5, 1,
                                              1, 0, None), b"workspace"),
    (lambda l: l.hipo_batchnorm_train_fwd_f32(None, 1, 1, 1, 1, 1, 1, 1, 2, 4, 9, 0.1, 1e-5, 1,
                                              1, 1 << 20, None), b"null"),
    (lambda l: l.hipo_batchnorm_nhwc_act_pad_bf16(*[1] * 8, 2, 4, 4, 8, 1, 1, 0.1, 1e-3, 1.0, 3,
                                                  16, 1 << 20, None), b"act"),
    (lambda l: l.hipo_batchnorm_nhwc_act_pad_bf16(*[1] * 8, 2, 4, 4, 8, 1, 1, 0.1, 1e-3, 1.0, 2,
                                                  16, 8, None), b"workspace"),
    (lambda l: l.hipo_batchnorm_nhwc_act_pad_bf16(*[1] * 8, 2, 4, 4, 8, 1, 1, 0.1, 1e-3, 1.0, 2,
                                                  8, 1 << 20, None), b"aligned"),
    (lambda l: l.hipo_batchnorm_nhwc_act_pad_bf16(None, *[1] * 7, 2, 4, 4, 8, 0, 0, 0.1, 1e-3, 1.0,
                                                  0, 16, 1 << 20, None), b"null"),
    (lambda l: l.hipo_batchnorm_nhwc_act_pad_bf16(*[1] * 8, 0, 4, 4, 8, 0, 0, 0.1, 1e-3, 1.0, 0,
                                                  16, 1 << 20, None), b"empty reduction"),
    (lambda l: l.hipo_batchnorm_nhwc_act_pad_bf16(*[1] * 8, 2, 4, 4, 8, -1, 0, 0.1, 1e-3, 1.0, 0,
                                                  16, 1 << 20, None), b"negative"),
    (lambda l: l.hipo_batchnorm_nchw_act_mean_bf16(*[1] * 8, 2, 8, 49, 0.1, 1e-5, 1.0, 5,
                                                   16, 1 << 20, None), b"act"),
    (lambda l: l.hipo_batchnorm_nchw_act_mean_bf16(*[1] * 8, 5, 8, 49, 0.1, 1e-5, 1.0, 1,
                                                   16, 64, None), b"workspace"),
    (lambda l: l.hipo_batchnorm_nchw_act_mean_bf16(*[1] * 7, None, 5, 8, 49, 0.1, 1e-5, 1.0, 1,
                                                   16, 1 << 20, None), b"null"),
    (lambda l: l.hipo_batchnorm_nchw_act_mean_bf16(*[1] * 8, 5, 8, 0, 0.1, 1e-5, 1.0, 1,
                                                   16, 1 << 20, None), b"empty reduction"),
    (lambda l: l.hipo_gelu_erf_bwd_colsum_bf16(16, 16, 16, 16, 4, 12, 16, 1 << 20, None),
     b"multiple of 8"),
    (lambda l: l.hipo_gelu_erf_bwd_colsum_bf16(16, 16, 16, 16, -1, 16, 16, 1 << 20, None),
     b"negative"),
    (lambda l: l.hipo_gelu_erf_bwd_colsum_bf16(16, 16, 16, None, 4, 16, 16, 1 << 20, None),
     b"colsum"),
    (lambda l: l.hipo_gelu_erf_bwd_colsum_bf16(None, 16, 16, 16, 4, 16, 16, 1 << 20, None),
     b"null"),
    (lambda l: l.hipo_gelu_erf_bwd_colsum_bf16(8, 16, 16, 16, 4, 16, 16, 1 << 20, None),
     b"aligned"),
    (lambda l: l.hipo_gelu_erf_bwd_colsum_bf16(16, 16, 16, 16, 4096, 3072, 16, 8, None),
     b"workspace"),
])
def test_argument_errors_before_launch(lib, call, msg):
    assert call(lib) == HIPO_EINVAL
    assert msg in lib.hipo_last_error()


def test_empty_inputs_are_no_ops(lib):
    assert lib.hipo_row_mean_f32(None, None, 0, 16, 16, None) == 0
    assert lib.hipo_bias_gelu_nchw_to_nhwc_bf16(None, None, None, 0, 8, 8, None) == 0
    assert lib.hipo_scaled_masked_softmax_bf16(None, None, None, 3, 0, 8, 8, 1.0, None) == 0
    assert lib.hipo_scaled_bias_softmax_bf16(None, None, None, 0, 4, 8, 8, 0, 1, 1.0, None) == 0
    assert lib.hipo_rmsnorm_ex_bf16(None, None, None, None, None, None, 0, 8, 1e-5, 1.0, 0, None) == 0
    assert lib.hipo_spatial_mean_nhwc_bf16(None, None, 0, 64, 8, None, 0, None) == 0
    assert lib.hipo_batchnorm_nhwc_act_pad_bf16(*[None] * 8, 2, 4, 4, 0, 1, 1, 0.1, 1e-3, 1.0, 2,
                                                None, 0, None) == 0
    assert lib.hipo_batchnorm_nchw_act_mean_bf16(*[None] * 8, 2, 0, 49, 0.1, 1e-5, 1.0, 1,
                                                 None, 0, None) == 0
    assert lib.hipo_gelu_erf_bwd_colsum_bf16(None, None, None, None, 0, 0, None, 0, None) == 0
    assert lib.hipo_last_error() == b""


def test_spatial_mean_workspace_bytes(lib):
    # one slice per image when there are enough images or few positions
    assert lib.hipo_spatial_mean_workspace_bytes(128, 36, 1536) == 0
    assert lib.hipo_spatial_mean_workspace_bytes(0, 64, 8) == 0
    # [128, 256, 64, 64]: 16-group channel blocks, 256 workgroups, no slices
    assert lib.hipo_spatial_mean_workspace_bytes(128, 4096, 256) == 0
    # [64, 256, 64, 64]: four position slices -> fp32 partials [64, 4, 256]
    assert lib.hipo_spatial_mean_workspace_bytes(64, 4096, 256) == 64 * 4 * 256 * 4
    # C not a multiple of 8: the scalar kernel, no workspace
    assert lib.hipo_spatial_mean_workspace_bytes(4, 4096, 100) == 0


def test_bf16_batchnorm_workspace_bytes(lib):
    """(mean, M2) fp32 pairs per slice and channel.  Channels-last: slices of
    a multiple of 512 rows, at most about 512 of them; NCHW: one slice per 4
    images."""
    assert lib.hipo_batchnorm_nhwc_workspace_bytes(128, 28, 28, 240) == 196 * 240 * 8
    assert lib.hipo_batchnorm_nhwc_workspace_bytes(128, 112, 112, 96) == 448 * 96 * 8
    assert lib.hipo_batchnorm_nhwc_workspace_bytes(1, 3, 3, 20) == 1 * 20 * 8
    assert lib.hipo_batchnorm_nhwc_workspace_bytes(0, 3, 3, 20) == 0
    assert lib.hipo_batchnorm_nchw_mean_workspace_bytes(128, 1024, 49) == 32 * 1024 * 8
    assert lib.hipo_batchnorm_nchw_mean_workspace_bytes(5, 8, 9) == 2 * 8 * 8
    assert lib.hipo_batchnorm_nchw_mean_workspace_bytes(5, 8, 0) == 0


def test_noalloc_error_query_without_a_call(lib):
    """hipo_batchnorm_noalloc_error before the allocation-free entry point has
    run on a device: word 0, no device call; bad arguments are rejected."""
    import ctypes
    w = ctypes.c_uint32(7)
    assert lib.hipo_batchnorm_noalloc_error(0, ctypes.byref(w), 1) == 0 and w.value == 0
    assert lib.hipo_batchnorm_noalloc_error(0, None, 0) == HIPO_EINVAL
    assert b"null" in lib.hipo_last_error()
    assert lib.hipo_batchnorm_noalloc_error(-1, ctypes.byref(w), 0) == HIPO_EINVAL
    assert lib.hipo_batchnorm_noalloc_error(64, ctypes.byref(w), 0) == HIPO_EINVAL


def test_yardstick_argument_checks(lib):
    """The two-stream yardstick rejects bad arguments on the host, before
    any device call: sizes that are not positive multiples of 1 KiB, null or
    misaligned pointers."""
    import ctypes
    buf = ctypes.create_string_buffer(4096 + 16)
    base = (ctypes.addressof(buf) + 15) // 16 * 16
    p = ctypes.c_void_p(base)
    assert lib.hipo_flat_copy2(p, p, p, p, 1000, None) != 0
    assert "multiple of 1024" in lib.hipo_last_error().decode()
    assert lib.hipo_flat_copy2(p, None, p, p, 1024, None) != 0
    assert "null" in lib.hipo_last_error().decode()
    q = ctypes.c_void_p(base + 4)
    assert lib.hipo_flat_copy2(p, q, p, p, 1024, None) != 0
    assert "aligned" in lib.hipo_last_error().decode()


def test_hold_copy_argument_checks(lib):
    """The BatchNorm hold-copy yardstick rejects, on the host, sizes that are
    not positive, null pointers and shapes outside the single-pass geometry
    (H*W not a multiple of 4) before any device call."""
    import ctypes
    buf = ctypes.create_string_buffer(4096 + 16)
    p = ctypes.c_void_p((ctypes.addressof(buf) + 15) // 16 * 16)
    assert lib.hipo_hold_copy_f32(p, p, 0, 4, 4, None) != 0
    assert "positive" in lib.hipo_last_error().decode()
    assert lib.hipo_hold_copy_f32(None, p, 2, 4, 4, None) != 0
    assert "null" in lib.hipo_last_error().decode()
    assert lib.hipo_hold_copy_f32(p, p, 2, 4, 49, None) != 0
    assert "geometry" in lib.hipo_last_error().decode()


def test_gelu_bwd_workspace_bytes(lib):
    """fp64 column partials, one row per row block: none up to 256 rows (one
    launch); 8-row blocks up to 1024 rows; 256-row blocks for one or two
    512-column blocks, halved (to 32 at least) while they give fewer than
    192 workgroups; rows * blocks / 2048 rows held to [64, 128] (up to 8
    column blocks) or [32, 128]."""
    assert lib.hipo_gelu_erf_bwd_colsum_workspace_bytes(25216, 3072) == 346 * 3072 * 8
    assert lib.hipo_gelu_erf_bwd_colsum_workspace_bytes(175360, 3072) == 1370 * 3072 * 8
    assert lib.hipo_gelu_erf_bwd_colsum_workspace_bytes(32768, 1024) == 128 * 1024 * 8
    assert lib.hipo_gelu_erf_bwd_colsum_workspace_bytes(2048, 10240) == 64 * 10240 * 8
    assert lib.hipo_gelu_erf_bwd_colsum_workspace_bytes(128, 3072) == 0
    assert lib.hipo_gelu_erf_bwd_colsum_workspace_bytes(256, 16) == 0
    assert lib.hipo_gelu_erf_bwd_colsum_workspace_bytes(257, 3072) == 33 * 3072 * 8
    assert lib.hipo_gelu_erf_bwd_colsum_workspace_bytes(1000, 16) == 125 * 16 * 8
    # two column blocks, 8192 rows: 64-row blocks (128 x 2 = 256 workgroups)
    assert lib.hipo_gelu_erf_bwd_colsum_workspace_bytes(8192, 768) == 128 * 768 * 8
    # 25216 rows: 256-row blocks already give 99 x 2 = 198 workgroups
    assert lib.hipo_gelu_erf_bwd_colsum_workspace_bytes(25216, 768) == 99 * 768 * 8
    # 2048 rows of one column block: halved down to the 32-row floor
    assert lib.hipo_gelu_erf_bwd_colsum_workspace_bytes(2048, 512) == 64 * 512 * 8
    # grid.y holds at most 65535 row blocks: longer tensors get longer blocks
    rows = 10 ** 8
    rpb = -(-rows // 65535)
    assert lib.hipo_gelu_erf_bwd_colsum_workspace_bytes(rows, 8) == -(-rows // rpb) * 8 * 8
    assert lib.hipo_gelu_erf_bwd_colsum_workspace_bytes(0, 16) == 0
    assert lib.hipo_gelu_erf_bwd_colsum_workspace_bytes(16, 0) == 0


def test_batchnorm_workspace_bytes(lib):
    assert lib.hipo_batchnorm_workspace_bytes(0, 4, 4) == 0
    n = lib.hipo_batchnorm_workspace_bytes(128, 256, 3136)
    assert 0 < n < (1 << 24)
    assert hip_oracles.batchnorm_workspace_bytes(128, 256, 3136) == n


def test_error_message_is_per_thread(lib):
    import threading
    assert lib.hipo_row_mean_f32(None, None, -1, 4, 4, None) == HIPO_EINVAL
    seen = []
    th = threading.Thread(target=lambda: seen.append(lib.hipo_last_error()))
    th.start()
    th.join()
    assert seen == [b""] and b"negative" in lib.hipo_last_error()


def test_wrappers_reject_cpu_tensors_without_fallback():
    import torch
    with pytest.raises(ValueError, match="ROCm device"):
        hip_oracles.row_mean(torch.randn(4, 4))
    with pytest.raises(ValueError):
        hip_oracles.bias_gelu_nchw_to_nhwc(torch.randn(1, 8, 2, 2).bfloat16(),
                                           torch.zeros(8).bfloat16())


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(hip_oracles.HipOraclesUnavailable):
        hip_oracles.load_library(tmp_path / "nope.so")


def test_bench_refuses_multi_gpu():
    import pathlib
    root = pathlib.Path(__file__).resolve().parents[1]
    proc = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "2"],
                          capture_output=True, text=True, timeout=120)
    assert proc.returncode == 2 and "one GPU" in proc.stderr
