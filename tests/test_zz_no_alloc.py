"""The allocation-free BatchNorm entry point against the workspace one.

hipo_batchnorm_train_fwd_f32_noalloc keeps its workspace in a file-scope
device array instead of a caller allocation.  Called through the C ABI, it
must give bit-identical outputs (y, save_mean, save_invstd and the updated
running statistics) to hipo_batchnorm_train_fwd_f32 with a zeroed caller
workspace on the same inputs: the same kernels run in both.  Two calls in a
row, the second on a smaller shape (the array keeps the first call's state),
plus a shape beyond the array's size, which must be rejected.
"""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

SHAPES = [
    (128, 256, 56, 56),  # the BASELINE config: the single-pass kernel
    (16, 24, 7, 7),      # smaller, HW % 4 != 0: one workgroup per channel
    (32, 64, 28, 28),    # smaller again, single pass with another slab plan
]


def _inputs(shape, seed):
    g = torch.Generator().manual_seed(seed)
    n, c, h, w = shape
    x = torch.randn(shape, generator=g) * 2 + 0.5
    gamma = 1 + 0.1 * torch.randn(c, generator=g)
    beta = 0.1 * torch.randn(c, generator=g)
    rm = 0.1 * torch.randn(c, generator=g)
    rv = 1 + 0.1 * torch.rand(c, generator=g)
    return x, gamma, beta, rm, rv


def _run(lib, dev, shape, seed, noalloc):
    n, c, h, w = shape
    x, gamma, beta, rm, rv = (t.to(dev) for t in _inputs(shape, seed))
    y = torch.empty_like(x)
    save_mean = torch.empty(c, device=dev)
    save_invstd = torch.empty(c, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    ptrs = [t.data_ptr() for t in (x, gamma, beta, rm, rv, y, save_mean, save_invstd)]
    if noalloc:
        rc = lib.hipo_batchnorm_train_fwd_f32_noalloc(*ptrs, n, c, h * w, 0.1, 1e-5, 1, stream)
    else:
        need = lib.hipo_batchnorm_workspace_bytes(n, c, h * w)
        ws = torch.zeros(need, dtype=torch.uint8, device=dev)
        rc = lib.hipo_batchnorm_train_fwd_f32(*ptrs, n, c, h * w, 0.1, 1e-5, 1,
                                              ws.data_ptr(), need, stream)
    assert rc == 0, lib.hipo_last_error().decode()
    torch.cuda.synchronize(dev)
    return [t.cpu() for t in (y, save_mean, save_invstd, rm, rv)]


def test_noalloc_matches_workspace_entry_point(rocm_device):
    import hip_oracles
    lib = hip_oracles.load_library()
    names = ("y", "save_mean", "save_invstd", "running_mean", "running_var")
    for k, shape in enumerate(SHAPES):
        print(f"noalloc vs workspace: shape {shape}", flush=True)
        want = _run(lib, rocm_device, shape, 100 + k, noalloc=False)
        got = _run(lib, rocm_device, shape, 100 + k, noalloc=True)
        for name, a, b in zip(names, got, want):
            assert torch.isfinite(a).all(), f"{shape} {name}: non-finite values"
            assert torch.equal(a, b), (f"{shape} {name}: max |diff| "
                                       f"{(a - b).abs().max().item():.3e}")


def test_noalloc_rejects_shapes_beyond_the_scratch_array(rocm_device):
    import hip_oracles
    lib = hip_oracles.load_library()
    n, c, hw = 2, 1 << 20, 1  # a workspace of tens of MiB
    assert lib.hipo_batchnorm_workspace_bytes(n, c, hw) > 4 << 20
    stream = torch.cuda.current_stream(rocm_device).cuda_stream
    p = ctypes.c_void_p(16)  # never dereferenced: rejected before any launch
    rc = lib.hipo_batchnorm_train_fwd_f32_noalloc(p, p, p, p, p, p, p, p, n, c, hw, 0.1, 1e-5,
                                                  1, stream)
    assert rc == 1000  # HIPO_EINVAL
    assert "scratch array" in lib.hipo_last_error().decode()


def test_noalloc_forced_timeout_is_reported(rocm_device, monkeypatch):
    """Failure injection from the host on the allocation-free path
    (HIPO_TEST_FORCE_BN_TIMEOUT: every exchange wait looks for a tag no
    workgroup publishes, gives up after a few polls, and the kernel exits
    normally): the outputs and running statistics are NaN, the sticky error
    word in the static scratch array is reported by device_faults() (read
    through hipo_batchnorm_noalloc_error) and cleared, and the next call
    without injection matches the workspace entry point again."""
    import hip_oracles
    lib = hip_oracles.load_library()
    shape = SHAPES[0]  # the single-pass kernel with its cross-workgroup exchange
    _run(lib, rocm_device, shape, 5, noalloc=True)  # the array is set up
    hip_oracles.device_faults()  # start clean
    monkeypatch.setenv("HIPO_TEST_FORCE_BN_TIMEOUT", "1")
    out = _run(lib, rocm_device, shape, 5, noalloc=True)
    for name, t in zip(("y", "save_mean", "save_invstd", "running_mean", "running_var"), out):
        assert torch.isnan(t).all(), f"{name} not poisoned after a timed-out exchange"
    faults = hip_oracles.device_faults()
    assert len(faults) == 1 and "noalloc" in faults[0] and "timed out" in faults[0], faults
    assert hip_oracles.device_faults() == [], "the error word was not cleared"
    monkeypatch.delenv("HIPO_TEST_FORCE_BN_TIMEOUT")
    got = _run(lib, rocm_device, shape, 6, noalloc=True)
    want = _run(lib, rocm_device, shape, 6, noalloc=False)
    for name, a, b in zip(("y", "save_mean", "save_invstd", "running_mean", "running_var"),
                          got, want):
        assert torch.equal(a, b), f"after the injected timeout: {name}"
    assert hip_oracles.device_faults() == []

