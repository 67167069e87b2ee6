"""pytest setup: put the package directory and the repo root on sys.path
(the reference's tests/conftest.py does the same for its root), and
register the `gpu` marker."""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "better-benchmark_amd"
for p in (str(PKG), str(ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)

CANONICAL = PKG / "repros" / "canonical"
REPRO_IDS = [
    "mean_lastdim_f32",
    "pointwise_bias_gelu_tanh_nhwc",
    "amax_sum_scaled_masked_softmax",
    "var_mean_residual_layernorm",
    "mean_rmsnorm",
    "var_mean_batchnorm_train_relu",
]


# Residual add + LayerNorm corpus families on one kernel, by what they
# return: y2 = y viewed [R, C]; h_y2 = (h, y); h_y2x3 = (h, three views of
# y); y3_y2x3 = (y, three views of it); y3_y2 = (y, a view of it).
LN_FAMILY_OUTPUTS = {
    "var_mean_0ada225c0a04": "y2",
    "var_mean_96edf0542ecd": "y2",
    "var_mean_f4578c128d74": "h_y2",
    "var_mean_b19e82f2a47b": "h_y2x3",
    "var_mean_393456b916a6": "y3_y2x3",
    "var_mean_45f7dfd4a983": "y3_y2",
}

# Residual add + RMSNorm corpus families on one kernel: (mode, first output,
# views of y after it) -- mode 1 rounds bf16(h * rstd) before the gamma
# product, mode 0 once at the end; the first output is h (the bf16 sum), y
# ([b, s, C]) or nothing; the views use the graph's shape parameters 1..n.
RMS_FAMILY_OUTPUTS = {
    "mean_f08c75b5f21f": (1, "", 1),
    "mean_db9733790220": (1, "", 1),
    "mean_8818e35b12aa": (1, "h", 1),
    "mean_c033ad4c69ca": (1, "h", 3),
    "mean_f21cc667fe83": (0, "h", 1),
    "mean_426e2409482e": (1, "y", 16),
    "mean_4dace6865eee": (1, "y", 12),
    "mean_bf2ed36e56df": (1, "h", 3),
    "mean_d28c6a07654f": (1, "h", 2),
    "mean_41e8bba10b8b": (1, "h", 2),
}

# Corpus families the kernels generalise to (the reference's canonical dir
# names, their shape points and model counts).
VARIANT_IDS = [
    "mean_c9e1a8113328",
    "mean_4462ce967d63",
    "amax_sum_20ccc18dda60",
    "var_mean_80e7ff4dee7f",
    "var_mean_ceb5c315290a",
    "var_mean_mean_19ffdb35cc67",
    "pointwise_2d969ac9ad59",
    "pointwise_021e90d9c17d",
    "mean_b402ee209d0b",
    "amax_sum_fa4cc85fe5ad",
] + list(LN_FAMILY_OUTPUTS) + list(RMS_FAMILY_OUTPUTS) + [
    "sum_139a3020e8bf",
]


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs the ROCm device (MI355X)")


@pytest.fixture(scope="session")
def rocm_device():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    return torch.device("cuda:0")
