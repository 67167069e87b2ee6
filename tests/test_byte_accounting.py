"""byte_accounting: the effective-byte rules, restating the reference's
test_byte_accounting.py:12-154 (dense, embedding, gather, index_select,
index_put, scatter, slice, downstream reduction of index_put, id reuse) and
tests/test_bench_accounting.py:85-101 (naive alias dedup), plus the
closed-form byte counts of the six BASELINE configs and the MI355X SOL
table."""
import pytest
import torch

from byte_accounting import (HBM_PEAK_BYTES_PER_S, achieved_gbps, count_bytes_effective,
                             count_bytes_naive, count_unique_tensor_bytes, sol_fraction, sol_us)


def nb(t):
    return t.numel() * t.element_size()


class M(torch.nn.Module):
    def __init__(self, fn):
        super().__init__()
        self.fn = fn

    def forward(self, *a):
        return self.fn(*a)


def test_dense_elementwise():
    a, b = torch.randn(4, 5), torch.randn(4, 5)
    out = a + b
    assert count_bytes_effective(M(lambda a, b: a + b), [a, b]) == nb(a) + nb(b) + nb(out)


def test_embedding_gather_index_select_charge_results():
    w, idx = torch.randn(1000, 16), torch.tensor([1, 3, 7, 9])
    out = torch.ops.aten.embedding.default(w, idx)
    got = count_bytes_effective(M(lambda w, i: torch.ops.aten.embedding.default(w, i)), [w, idx])
    assert got == nb(out) + nb(idx) + nb(out)
    assert got < count_bytes_naive([w, idx], out)
    src, gi = torch.randn(2, 100), torch.tensor([[1, 3, 5], [2, 4, 6]])
    out = torch.gather(src, 1, gi)
    assert count_bytes_effective(M(lambda s, i: torch.ops.aten.gather.default(s, 1, i)), [src, gi]) \
        == nb(out) + nb(gi) + nb(out)
    src = torch.randn(100, 16, dtype=torch.float16)
    si = torch.tensor([1, 3, 5, 7, 9])
    out = src.index_select(0, si)
    assert count_bytes_effective(M(lambda s, i: torch.ops.aten.index_select.default(s, 0, i)),
                                 [src, si]) == nb(out) + nb(si) + nb(out)


def test_index_put_and_scatter_charge_updates():
    idx, vals = torch.tensor([1, 3, 5]), torch.randn(3, 16)

    def ip(i, v):
        return torch.ops.aten.index_put.default(torch.zeros(100, 16), [i], v, False)
    got = count_bytes_effective(M(ip), [idx, vals])
    assert got == nb(idx) + nb(vals) + nb(vals)
    assert got < count_bytes_naive([idx, vals], ip(idx, vals))
    sidx = torch.tensor([[1] * 16, [3] * 16, [5] * 16])
    src = torch.randn(3, 16)

    def sc(i, s):
        return torch.ops.aten.scatter.src(torch.zeros(100, 16), 0, i, s)
    assert count_bytes_effective(M(sc), [sidx, src]) == nb(sidx) + nb(src) + nb(src)


def test_slice_charges_accessed_portion():
    x = torch.randn(8, 128, 100)
    got = count_bytes_effective(M(lambda x: torch.ops.aten.slice.Tensor(x, 1, 0, 64) + 1.0), [x])
    assert got == 2 * 8 * 64 * 100 * 4
    assert got < count_bytes_naive([x], x[:, :64] + 1)


def test_downstream_reduction_of_index_put():
    idx, vals = torch.tensor([1, 3, 5]), torch.randn(3, 16)

    def f(i, v):
        up = torch.ops.aten.index_put.default(torch.zeros(100, 16), [i], v, False)
        return torch.ops.aten.sum.dim_IntList(up, [0])
    assert count_bytes_effective(M(f), [idx, vals]) == nb(idx) + nb(vals) + 16 * 4


def test_id_reuse_does_not_leak_sparse_write():
    src, idx = torch.randn(10, 16), torch.tensor([1, 3, 5])

    def f(s, i):
        up = torch.ops.aten.index_put.default(torch.zeros(100, 16), [i], s[:3], False)
        up.sum(dim=0)
        return s.sum(dim=0)
    assert count_bytes_effective(M(f), [src, idx]) == nb(src) + nb(idx) + 16 * 4


def test_naive_dedups_output_aliases():
    a = torch.randn(10)
    out = a * 2
    assert count_bytes_naive([a], (out, out, out.view(10))) == nb(a) + nb(out)
    assert count_unique_tensor_bytes([out, out[:5]]) == nb(out) + 20


def test_inputs_returned_unchanged_are_not_writes():
    a = torch.randn(6)
    assert count_bytes_effective(M(lambda a: (a * 2, a)), [a]) == nb(a) * 2


def test_meta_outputs_are_distinct():
    """On meta tensors every storage pointer is 0; distinct outputs of equal
    size must still be charged separately."""
    x = torch.empty(16, 8, device="meta")
    assert count_bytes_effective(M(lambda x: (x + 1, x * 2)), [x]) == 3 * 16 * 8 * 4


# Closed forms of the BASELINE configs (algorithmic R + W bytes)
EXPECTED = {
    "mean_lastdim_f32": 134_217_728 + 32_768,
    "pointwise_bias_gelu_tanh_nhwc": 205_521_408 + 205_520_896,
    "amax_sum_scaled_masked_softmax": 807_403_520 + 805_306_368,
    "var_mean_residual_layernorm": 268_451_840 + 268_566_528,
    "mean_rmsnorm": 134_225_920 + 134_283_264,
    # running stats are updated inside native_batch_norm and returned as the
    # (never produced) inputs, so they are not charged as writes
    "var_mean_batchnorm_train_relu": 411_045_888 + 411_043_840,
}


@pytest.mark.parametrize("rid", list(EXPECTED))
def test_baseline_config_bytes(rid):
    from conftest import CANONICAL
    from oracle_harness import effective_bytes, get_repro_instance
    from repro_harness import load_shape_configs
    cfg = next(iter(load_shape_configs(str(CANONICAL / rid / "repro.py")).values()))
    meta = [torch.empty_strided(s["shape"], s["stride"], dtype=getattr(torch, s["dtype"]),
                                device="meta") for s in cfg["inputs"]]
    assert effective_bytes(get_repro_instance(CANONICAL / rid), meta) == EXPECTED[rid]


def test_sol_table():
    assert HBM_PEAK_BYTES_PER_S["MI355X"] == 8.0e12
    assert sol_us(8_000_000) == pytest.approx(1.0)
    assert achieved_gbps(8_000_000, 2.0) == pytest.approx(4000.0)
    assert sol_fraction(8_000_000, 2.0) == pytest.approx(0.5)
    assert sol_us(134_250_496) == pytest.approx(16.78, abs=0.01)
