"""
MI355X oracle for mean_lastdim_f32: x.mean(dim=-1) on fp32 [R, C].

Kernel: hipo_row_mean_f32 (libhip_oracles.so) -- up to 8 waves per row,
non-temporal 16-byte lane-interleaved loads (1 KiB per load instruction),
fp32 accumulation, DPP wave reduction, fixed-order LDS combine.  Algorithmic bytes: 4 R C + 4 R.
Replaces the Triton body of the reference's
repros/canonical/mean_c9e1a8113328/oracle.py:95 (row mode, :45).
"""
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
import hip_oracles  # noqa: E402
from oracle_harness import oracle_impl, oracle_main  # noqa: E402


@oracle_impl(hardware="MI355X", point="b84ae979", description="row mean, waves per row")
@oracle_impl(hardware="MI355X", description="row mean, shape-general")
def oracle_forward(inputs):
    (x,) = inputs
    return hip_oracles.row_mean(x)


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
