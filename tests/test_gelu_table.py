"""The GELU kernel's bf16 -> bf16 mapping, pinned on the CPU.

csrc/bias_gelu_nhwc.hip maps the bits of t = bf16(x + bias) to the bits of
GELU_tanh(t) with a table (csrc/gelu_table.h) for 2^-10 <= |t| < 16 and bit
arithmetic elsewhere.  Here the committed table is regenerated, and the whole
mapping -- restated in Python from the kernel's rules -- is compared over all
65536 bf16 inputs with the exact function evaluated by mpmath and rounded to
nearest even: every finite input must match, except that below 2^-125 the
kernel rounds t / 2 (ties to even) where the exact value sits a hair off the
tie.  Independently of mpmath, the table's values are checked against
closed forms (GELU(t) = t for large t, t / 2 for tiny t, GELU(0) = 0) and
against the CPU oracle's fp64 evaluation away from the far negative tail.
"""
import importlib.util
import math
from pathlib import Path

import pytest

mpmath = pytest.importorskip("mpmath")

ROOT = Path(__file__).resolve().parents[1]
GEN = ROOT / "better-benchmark_amd" / "hip_oracles" / "gen_gelu_table.py"


@pytest.fixture(scope="module")
def gen():
    spec = importlib.util.spec_from_file_location("gen_gelu_table", GEN)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_committed_table_is_current(gen):
    assert gen.main(["--check"]) == 0, "csrc/gelu_table.h differs from the generator"


def _kernel_mapping(gen, table):
    """The kernel's gelu_bits, restated."""
    lo = gen.E_LO << 7
    hi = (gen.E_HI + 1) << 7

    def f(tb):
        mag = tb & 0x7FFF
        off = (mag - lo) & 0xFFFFFFFF
        if off < gen.PER_SIGN:
            return table[off + (gen.PER_SIGN if tb & 0x8000 else 0)]
        if mag < 0x100:  # +-0 and subnormal results: t / 2, nearest even
            return gen.to_bf16(gen.bf16_value(tb) / 2)
        if mag < lo:
            return tb - 0x80
        if not tb & 0x8000 or mag > 0x7F80:
            return tb
        return 0x7FC0 if mag == 0x7F80 else 0x8000

    return f


def test_mapping_is_the_correctly_rounded_gelu(gen):
    table = gen.table()
    f = _kernel_mapping(gen, table)
    mismatches = []
    for tb in range(65536):
        mag = tb & 0x7FFF
        got = f(tb)
        if mag > 0x7F80:                       # NaN in -> NaN out
            assert (got & 0x7FFF) > 0x7F80
            continue
        if mag == 0x7F80:                      # +inf -> +inf, -inf -> NaN
            assert got == (0x7F80 if tb < 0x8000 else 0x7FC0)
            continue
        want = gen.to_bf16(gen.gelu_tanh_exact(gen.bf16_value(tb)))
        if got != want:
            mismatches.append((tb, got, want))
    # only ties of t / 2 below 2^-125 may differ, by one subnormal ulp
    for tb, got, want in mismatches:
        assert (tb & 0x7FFF) < 0x100 and abs((got & 0x7FFF) - (want & 0x7FFF)) == 1, \
            (hex(tb), hex(got), hex(want))
    assert len(mismatches) <= 128


def test_table_closed_forms_and_fp64(gen):
    table = gen.table()
    per = gen.PER_SIGN
    # t in [8, 16): GELU(t) = t;  smallest |t| = 2^-10: t / 2
    for m in range(128):
        assert table[(gen.E_HI - gen.E_LO) * 128 + m] == (gen.E_HI << 7) | m
    assert table[0] == ((gen.E_LO - 1) << 7)              # GELU(2^-10) -> 2^-11
    assert table[per] == 0x8000 | ((gen.E_LO - 1) << 7)   # GELU(-2^-10) -> -2^-11
    # against an independent fp64 evaluation of the tanh form (accurate
    # while 1 + tanh(u) does not cancel: t > -5)
    for i, v in enumerate(table):
        tb = (0x8000 if i >= per else 0) | (((i % per) // 128 + gen.E_LO) << 7) | (i % 128)
        t = float(gen.bf16_value(tb))
        if t <= -5.0:
            continue
        y = 0.5 * t * (1.0 + math.tanh(0.7978845608028654 * (t + 0.044715 * t ** 3)))
        want = gen.to_bf16(mpmath.mpf(y))
        assert abs((v & 0x7FFF) - (want & 0x7FFF)) <= 1 and (v & 0x8000) == (want & 0x8000), \
            (hex(tb), hex(v), hex(want))
