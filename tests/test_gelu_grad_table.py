"""The GELU(erf) backward kernel's d(t) table, pinned on the CPU.

csrc/gelu_bwd.hip multiplies the gradient by d(t) = Phi(t) + t phi(t) (the
derivative of GELU(t) = t Phi(t)) read from csrc/gelu_grad_table.h, indexed
by the bits of the bf16 input t with the exponent clamped to [100, 131].
Here the committed table is regenerated (mpmath at 96 bits), the clamped
rows are checked to stand for every input they cover, and the whole
mapping -- restated in Python from the kernel's indexing -- is compared over
all 65536 bf16 inputs with the CPU oracle's fp64 evaluation (libm erfc /
exp, rounded once to fp32).  Independently of both: scipy's normal CDF,
finite differences of GELU itself, and closed forms.
"""
import importlib.util
import math
import struct
from pathlib import Path

import pytest
import torch

import oracle as ref

mpmath = pytest.importorskip("mpmath")

ROOT = Path(__file__).resolve().parents[1]
GEN = ROOT / "better-benchmark_amd" / "hip_oracles" / "gen_gelu_grad_table.py"


@pytest.fixture(scope="module")
def gen():
    spec = importlib.util.spec_from_file_location("gen_gelu_grad_table", GEN)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="module")
def table(gen):
    return gen.table()


def _f32(bits):
    return struct.unpack("<f", struct.pack("<I", bits & 0xFFFFFFFF))[0]


def _all_bf16():
    return torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)


def _kernel_d(gen, table, tb):
    """The kernel's d for the bf16 bits tb: the clamped magnitude's entry,
    NaN for inf and NaN inputs."""
    mag = tb & 0x7FFF
    if mag >= 0x7F80:
        return float("nan")
    mc = min(max(mag, gen.E_LO << 7), (gen.E_HI << 7) | 0x7F) - (gen.E_LO << 7)
    return _f32(table[(gen.PER_SIGN if tb & 0x8000 else 0) + mc])


def test_committed_table_is_current(gen):
    assert gen.main(["--check"]) == 0, "csrc/gelu_grad_table.h differs from the generator"


def test_clamped_rows_stand_for_their_inputs(gen, table):
    gen.check_clamped_rows(table)  # raises on the first input whose d differs


def test_mapping_equals_the_oracle_on_every_bf16_input(gen, table):
    d = ref.gelu_erf_grad(_all_bf16()).tolist()
    for tb in range(65536):
        want = d[tb]
        got = _kernel_d(gen, table, tb)
        if math.isnan(want) or math.isnan(got):
            assert math.isnan(want) and math.isnan(got), hex(tb)
        else:
            assert got == want, (hex(tb), got, want)


def test_table_against_scipy_normal_cdf(gen, table):
    """scipy's ndtr (an independent Phi) in fp64, rounded to fp32: equal to
    the table but for fp64's own error at a rounding boundary."""
    special = pytest.importorskip("scipy.special")
    import numpy as np
    idx = np.arange(2 * gen.PER_SIGN)
    sign = np.where(idx >= gen.PER_SIGN, -1.0, 1.0)
    e = (idx % gen.PER_SIGN) // 128 + gen.E_LO
    m = idx % 128
    t = sign * np.ldexp(128.0 + m, e - 127 - 7)
    want = (special.ndtr(t) + t * np.exp(-0.5 * t * t) / math.sqrt(2 * math.pi)).astype(np.float32)
    got = np.array(table, dtype=np.uint32).view(np.float32)
    inner = (e > gen.E_LO) & (e < gen.E_HI)  # the clamped rows are checked on their own
    diff = np.nonzero(inner & (got != want))[0]
    ulps = np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
    assert diff.size <= 4 and (ulps[diff] <= 1).all(), [(int(i), got[i], want[i]) for i in diff[:8]]


def test_table_is_the_derivative_of_gelu(gen, table):
    """Central differences of GELU(t) = t Phi(t) = t erfc(-t / sqrt 2) / 2
    (step 2^-12, error ~1e-8) at every 3rd inner entry."""
    def gelu(t):
        return t * math.erfc(-t / math.sqrt(2.0)) / 2

    h = 2.0 ** -12
    for i in range(0, 2 * gen.PER_SIGN, 3):
        e = (i % gen.PER_SIGN) // 128 + gen.E_LO
        if e in (gen.E_LO, gen.E_HI) or e > 130:
            continue
        t = (-1.0 if i >= gen.PER_SIGN else 1.0) * math.ldexp(128 + i % 128, e - 127 - 7)
        fd = (gelu(t + h) - gelu(t - h)) / (2 * h)
        assert abs(_f32(table[i]) - fd) <= 1e-7 + 1e-6 * abs(fd), (t, _f32(table[i]), fd)


def test_closed_forms(gen, table):
    d = ref.gelu_erf_grad(torch.tensor(
        [0.0, -0.0, 16.0, -16.0, 3e38, -3e38, float("inf"), float("-inf"), float("nan"),
         1e-40]).to(torch.bfloat16)).tolist()
    assert d[0] == 0.5 and d[1] == 0.5 and d[9] == 0.5, "d(0) = 1/2"
    assert d[2] == 1.0 and d[4] == 1.0, "d(t) -> 1"
    assert d[3] == 0.0 and d[5] == 0.0, "d(t) -> 0 from below"
    assert all(math.isnan(v) for v in d[6:9]), "inf * 0 in the graph's t * exp(-t^2 / 2)"
    # d(t) + d(-t) = 1 (Phi(t) + Phi(-t) = 1, the t phi terms cancel)
    for i in range(gen.PER_SIGN):
        s = _f32(table[i]) + _f32(table[gen.PER_SIGN + i])
        assert abs(s - 1.0) <= 2 ** -23, (i, s)
    # the maximum of d: 1.1289 at t = sqrt(2) (d' = phi (2 - t^2) = 0)
    assert abs(max(_f32(v) for v in table) - 1.1289) < 1e-3
