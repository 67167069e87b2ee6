"""Effective byte accounting and the HBM speed-of-light table.

`count_bytes_effective(mod, inputs)` runs one eager forward of a repro under
a TorchDispatchMode and returns the bytes a perfectly fused kernel must
move: each external input is charged once (only the part any dense op
actually reads through a view), sparse reads (embedding / gather / index /
index_select / take) are charged at result size, sparse updates (scatter*,
index_put) are charged at update size, and each distinct output is charged
once.  Same rules as the reference's counter (reference:
byte_accounting.py:54-66, 142-293); the implementation here is separate.

The reference has no peak-bandwidth table (its SOL is a measured memcopy);
HBM_PEAK_BYTES_PER_S adds the published MI355X figure so oracle timings can
be reported as a fraction of the HBM roofline.  The counter also works on
"meta" tensors, so full-size byte counts need no device memory.
"""
from __future__ import annotations

from collections.abc import Iterable
from typing import Any

import torch
from torch.utils import _pytree
from torch.utils._python_dispatch import TorchDispatchMode

#: Published peak HBM bandwidth (bytes/s) per hardware kind.
HBM_PEAK_BYTES_PER_S = {
    "MI355X": 8.0e12,   # HBM3E, 8 TB/s
    "MI350X": 8.0e12,
    "MI325X": 6.0e12,
    "MI300X": 5.3e12,
}


def sol_us(nbytes: int, hardware: str = "MI355X") -> float:
    """Time (µs) to move `nbytes` at the hardware's peak HBM bandwidth."""
    return nbytes / HBM_PEAK_BYTES_PER_S[hardware] * 1e6


def achieved_gbps(nbytes: int, us: float) -> float:
    """Achieved bandwidth in GB/s (1e9 B/s) for `nbytes` moved in `us` µs."""
    return nbytes / (us * 1e-6) / 1e9 if us > 0 else 0.0


def sol_fraction(nbytes: int, us: float, hardware: str = "MI355X") -> float:
    """Achieved / peak HBM bandwidth."""
    return achieved_gbps(nbytes, us) * 1e9 / HBM_PEAK_BYTES_PER_S[hardware] if us > 0 else 0.0


def tensor_nbytes(tensor: torch.Tensor) -> int:
    return tensor.numel() * tensor.element_size()


def tensor_alias_key(tensor: torch.Tensor) -> tuple[int, int, int, int]:
    """(storage id, storage offset, numel, element size) identity of a view.

    The storage id is its data pointer; meta tensors have no data (every
    pointer is 0), so for them the StorageImpl address stands in.
    """
    try:
        storage = tensor.untyped_storage()
        base = storage._cdata if tensor.device.type == "meta" else storage.data_ptr()
    except RuntimeError:
        base = tensor.data_ptr()
    return (base, tensor.storage_offset(), tensor.nelement(), tensor.element_size())


def _tensors(values: Any):
    for leaf in _pytree.tree_leaves(values):
        if isinstance(leaf, torch.Tensor):
            yield leaf


def count_unique_tensor_bytes(values: Any) -> int:
    """Bytes of the tensors in a nested value, counting exact aliases once."""
    seen, total = set(), 0
    for t in _tensors(values):
        key = tensor_alias_key(t)
        if key not in seen:
            seen.add(key)
            total += tensor_nbytes(t)
    return total


def count_bytes_naive(inputs: Any, outputs: Any) -> int:
    """All input tensor bytes plus unique output bytes."""
    return sum(tensor_nbytes(t) for t in _tensors(inputs)) + count_unique_tensor_bytes(outputs)


def count_bytes_effective(mod, inputs: Iterable[Any]) -> int:
    """Effective reads of external inputs plus final output writes."""
    with _EffectiveByteCounter() as counter:
        with torch.no_grad():
            outputs = mod(*inputs)
    return counter.total(outputs)


_VIEW_OPS = frozenset({
    "aten.alias.default", "aten.as_strided.default", "aten.detach.default",
    "aten.expand.default", "aten.flatten.using_ints", "aten.permute.default",
    "aten.reshape.default", "aten.select.int", "aten.slice.Tensor",
    "aten.squeeze.default", "aten.squeeze.dim", "aten.squeeze.dims",
    "aten.t.default", "aten.transpose.int", "aten.unsqueeze.default",
    "aten.view.default", "aten._unsafe_view.default",
})

_SPARSE_SOURCE_OPS = frozenset({
    "aten.embedding.default", "aten.gather.default", "aten.index.Tensor",
    "aten.index_select.default", "aten.take.default",
})

_SCATTER_PREFIXES = ("aten.scatter.", "aten.scatter_add.", "aten.scatter_reduce.")


class _EffectiveByteCounter(TorchDispatchMode):
    """Dispatch-level tracker of which external bytes a region touches.

    Tensors are identified by id(); every tensor the region creates is kept
    alive for the counter's lifetime so ids are never recycled.
    """

    def __init__(self):
        super().__init__()
        self._alive: list[torch.Tensor] = []
        self._made: set[int] = set()          # ids of tensors ops returned
        self._view_root: dict[int, int] = {}  # view id -> root id
        self._ext_size: dict[int, int] = {}   # external root id -> nbytes
        self._dense_read: dict[int, int] = {} # root -> max bytes read densely
        self._sparse_read: dict[int, int] = {}
        self._sparse_write: dict[int, int] = {}  # result id -> update bytes

    def _root_of(self, tid: int) -> int:
        seen = set()
        while tid in self._view_root and tid not in seen:
            seen.add(tid)
            tid = self._view_root[tid]
        return tid

    def _note_operand(self, t: torch.Tensor) -> None:
        root = self._root_of(id(t))
        if root not in self._made and root not in self._ext_size:
            self._ext_size[root] = tensor_nbytes(t)

    def _dense(self, t: torch.Tensor) -> None:
        root = self._root_of(id(t))
        if root in self._ext_size:
            self._dense_read[root] = max(self._dense_read.get(root, 0), tensor_nbytes(t))

    def _sparse(self, t: torch.Tensor, nbytes: int) -> None:
        root = self._root_of(id(t))
        if root in self._ext_size:
            self._sparse_read[root] = self._sparse_read.get(root, 0) + nbytes

    def __torch_dispatch__(self, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        name = str(func)
        operands = list(_tensors((args, kwargs)))
        for t in operands:
            self._note_operand(t)

        result = func(*args, **kwargs)
        produced = list(_tensors(result))
        self._alive.extend(produced)
        for t in produced:
            self._made.add(id(t))

        first = args[0] if args and isinstance(args[0], torch.Tensor) else None
        if name in _VIEW_OPS and first is not None:
            root = self._root_of(id(first))
            for t in produced:
                self._view_root[id(t)] = root
            return result

        skip: set[int] = set()
        if name in _SPARSE_SOURCE_OPS and first is not None:
            skip.add(id(first))
            self._sparse(first, count_unique_tensor_bytes(result))
        if name.startswith(_SCATTER_PREFIXES):
            nb = self._update_bytes(args, result, src_pos=3)
            if len(args) >= 4 and isinstance(args[3], torch.Tensor):
                skip.add(id(args[3]))
                self._sparse(args[3], nb)
            for t in produced:
                self._sparse_write[id(t)] = nb
        if name == "aten.index_put.default":
            nb = self._update_bytes(args, result, src_pos=2)
            if len(args) >= 3 and isinstance(args[2], torch.Tensor):
                skip.add(id(args[2]))
                self._sparse(args[2], nb)
            for t in produced:
                self._sparse_write[id(t)] = nb
        for t in operands:
            if id(t) not in skip:
                self._dense(t)
        return result

    @staticmethod
    def _update_bytes(args, result, src_pos: int) -> int:
        full = count_unique_tensor_bytes(result)
        src = args[src_pos] if len(args) > src_pos else None
        if isinstance(src, torch.Tensor):
            return min(tensor_nbytes(src), full)
        if src_pos == 3 and len(args) >= 3 and isinstance(args[2], torch.Tensor):
            # scatter with a scalar value: one element per index entry
            out = next(_tensors(result), None)
            esize = out.element_size() if out is not None else 1
            return min(args[2].numel() * esize, full)
        return full

    def read_bytes(self) -> int:
        total = 0
        for root, size in self._ext_size.items():
            if root in self._dense_read:
                total += min(self._dense_read[root], size)
            else:
                total += min(self._sparse_read.get(root, 0), size)
        return total

    def write_bytes(self, outputs: Any) -> int:
        seen, total = set(), 0
        for t in _tensors(outputs):
            key = tensor_alias_key(t)
            if key in seen:
                continue
            seen.add(key)
            root = self._root_of(id(t))
            if root in self._ext_size and id(t) not in self._made:
                continue  # an input handed back unchanged by identity
            nbytes = tensor_nbytes(t)
            if id(t) in self._sparse_write:
                nbytes = min(self._sparse_write[id(t)], nbytes)
            total += nbytes
        return total

    def total(self, outputs: Any) -> int:
        return self.read_bytes() + self.write_bytes(outputs)
