"""
MI355X oracle for amax_sum_scaled_masked_softmax:
softmax(scores * 0.125 + mask, -1), bf16 in/out, fp32 max and sum.

Kernel: hipo_scaled_masked_softmax_bf16 -- the row in registers (one wave
per row at K = 1024, two non-temporal 16-byte loads per lane, 8 rows per
workgroup), DPP max and sum, the [Q, K] mask row re-read from cache for
every batch entry.  Algorithmic
bytes: 2 B Q K (read) + 2 Q K (mask) + 2 B Q K (write).
Replaces the Triton body of the reference's
repros/canonical/amax_sum_20ccc18dda60/oracle.py:63.
"""
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))
import hip_oracles  # noqa: E402
from oracle_harness import oracle_impl, oracle_main  # noqa: E402

SCALE = 0.125  # the graph constant of repro.py


@oracle_impl(hardware="MI355X", point="134a1d74", description="masked softmax, rows in registers")
@oracle_impl(hardware="MI355X", description="masked softmax, shape-general")
def oracle_forward(inputs):
    x, mask = inputs
    return hip_oracles.scaled_masked_softmax(x, mask, SCALE)


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
