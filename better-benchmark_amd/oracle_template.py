"""Template for an MI355X oracle.py (copy into repros/canonical/<repro_id>/).

The MI355X counterpart of the reference's scripts/oracle_template.py: the
same module contract (an `oracle_forward(inputs, **cfg)` registered with
`@oracle_impl`, the standalone `--check/--bench` CLI), with the Triton body
replaced by a call into a C-ABI HIP kernel library.

Contract (scope invariant):
  * `oracle_forward` takes exactly the inputs `Repro()(*inputs)` takes (the
    repro's `make_inputs`) and returns the same outputs: count, shapes,
    dtypes and strides; in-place updates (running statistics) happen on the
    same input tensors and those tensors are returned.
  * Outputs and workspaces are allocated with torch on the inputs' device;
    the kernel call enqueues on torch's current stream and does nothing
    else (no allocation, synchronisation or host copy), so `bench_oracle`
    can capture it in a hipGraph.
  * No CPU or eager fallback: a missing library or a non-ROCm tensor is an
    error, never a silent substitute.
  * Registrations: `point="<shape_hash>"` for every shapes.json point the
    kernel was tuned on, and one shape-general `@oracle_impl(hardware=
    "MI355X")` if it handles other shapes correctly.  Launch parameters
    given as extra keyword arguments reach `oracle_forward` as kwargs.

Steps for a new pattern:
  1. Write the kernel and its `extern "C"` entry point in
     hip_oracles/csrc/<name>.hip, declare it in include/hip_oracles.h, add
     the source to hip_oracles/build.py and the signature to
     hip_oracles/__init__.py (_SIGNATURES + a wrapper doing the host-side
     checks and allocations).
  2. Copy this file to the canonical dir as oracle.py, fill in
     `oracle_forward` and the registrations.
  3. `python oracle.py --check --all-shapes` (eager comparison at every
     point), then `python oracle.py --bench --all-shapes`.
"""
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[3]))  # the package dir
import hip_oracles  # noqa: E402,F401  (the kernel library)
from oracle_harness import oracle_impl, oracle_main  # noqa: E402


# @oracle_impl(hardware="MI355X", point="<shape_hash>", description="...")
@oracle_impl(hardware="MI355X", description="TODO: what this kernel computes")
def oracle_forward(inputs):
    """Same inputs and outputs as Repro()(*inputs)."""
    raise NotImplementedError("call the hip_oracles wrapper of the new kernel here")


if __name__ == "__main__":
    raise SystemExit(oracle_main(__file__, oracle_forward))
