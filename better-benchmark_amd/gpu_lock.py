"""Per-GPU advisory benchmark locks and ROCm GPU discovery.

The ROCm counterpart of the reference's scripts/gpu_lock.py (and
scripts/with_gpu_lock.py): the same lock protocol, so every benchmark that
opts in serialises on one GPU, with discovery through ROCm instead of
nvidia-smi.

Lock protocol (reference scripts/gpu_lock.py:60-205, 247-300):
  - one lock file per GPU, `<lock dir>/gpu_<index>.lock`, taken with
    `flock` (exclusive for timing, shared for set-up work);
  - the holder writes `pid=`, `gpu=`, `device_kind=`, `mode=`, `label=`,
    `acquired_unix=` lines into the file;
  - a waiter that finds the holder's pid dead for longer than the stale
    grace period raises TimeoutError naming the holder instead of waiting
    forever; an optional timeout does the same for a live holder.
The lock directory and the file names are the ones
oracle_harness._gpu_exclusive_lock uses, so the two interoperate.

Discovery: `index` is the device's position in the ROCr-visible list (the
number HIP_VISIBLE_DEVICES takes).  The order comes from the KFD topology
under /sys/class/kfd/kfd/topology/nodes (GPU nodes are the ones with SIMDs,
in node order, which is the order ROCr enumerates them); product names come
from `rocm-smi --showproductname --json`, matched by KFD node id (rocm-smi's
own card numbering follows DRM and need not match ROCr's).  Without the
KFD tree, rocm-smi's list is used as is; without either, one unknown device.
A HIP_VISIBLE_DEVICES (or CUDA_VISIBLE_DEVICES) list in the environment
restricts the result to those indices; ROCR_VISIBLE_DEVICES renumbers.

CLI (reference scripts/with_gpu_lock.py):
    python -m gpu_lock --gpu 0 -- python bench.py
    python -m gpu_lock --device-kind MI355X -- python bench.py
runs the command with HIP_VISIBLE_DEVICES set to the locked GPU.
"""
from __future__ import annotations

import argparse
import contextlib
import fcntl
import json
import os
import re
import subprocess
import sys
import time
from pathlib import Path
from typing import Iterator

DEFAULT_LOCK_DIR = Path(os.environ.get("COMPILE_UTILS_GPU_LOCK_DIR",
                                       "/tmp/compile_utils_gpu_locks"))
STALE_LOCK_GRACE_S = float(os.environ.get("COMPILE_UTILS_GPU_LOCK_STALE_GRACE_S", "5"))
KFD_TOPOLOGY = Path("/sys/class/kfd/kfd/topology/nodes")

#: Product names this module recognises, most specific first.
KNOWN_DEVICE_KINDS = ("MI355X", "MI350X", "MI325X", "MI300X", "MI300A", "MI250X", "MI210")
#: gfx target -> product kind (the gfx950 part is MI355X here; MI350X shares
#: the ISA but the product name, when available, wins).
ARCH_KINDS = {"gfx950": "MI355X", "gfx942": "MI300X", "gfx90a": "MI250X"}
VISIBILITY_VARS = ("HIP_VISIBLE_DEVICES", "CUDA_VISIBLE_DEVICES")


def device_kind_from_name(name: str, arch: str | None = None) -> str:
    """Product kind from a device / product name, else from the gfx target."""
    lowered = name.lower()
    for token in KNOWN_DEVICE_KINDS:
        if token.lower() in lowered:
            return token
    if arch and arch.split(":")[0] in ARCH_KINDS:
        return ARCH_KINDS[arch.split(":")[0]]
    return name.strip().replace(" ", "_") or "UNKNOWN"


def gfx_from_target_version(version: int) -> str:
    """KFD `gfx_target_version` (major*10000 + minor*100 + stepping) -> gfx name."""
    major, minor, step = version // 10000, (version // 100) % 100, version % 100
    return f"gfx{major}{minor:x}{step:x}"


def _parse_rocm_smi_json(text: str) -> list[dict[str, str]]:
    data = json.loads(text)
    cards = []
    for key, fields in data.items():
        m = re.fullmatch(r"card(\d+)", key)
        if not m or not isinstance(fields, dict):
            continue
        name = (fields.get("Card Series") or fields.get("Card Model")
                or fields.get("Device Name") or fields.get("Card SKU") or "UNKNOWN")
        arch = fields.get("GFX Version") or fields.get("gfx_version") or ""
        node = str(fields.get("Node ID", "")).strip()
        cards.append((int(m.group(1)), str(name), str(arch), node))
    cards.sort()
    return [{"index": str(i), "name": name, "kind": device_kind_from_name(name, arch),
             "node": node}
            for i, name, arch, node in cards]


def _discover_rocm_smi() -> list[dict[str, str]]:
    try:
        out = subprocess.run(["rocm-smi", "--showproductname", "--json"],
                             capture_output=True, text=True, timeout=30)
    except Exception:
        return []
    if out.returncode != 0 or not out.stdout.strip():
        return []
    try:
        return _parse_rocm_smi_json(out.stdout)
    except (ValueError, AttributeError):
        return []


def _discover_kfd(topology: Path = KFD_TOPOLOGY) -> list[dict[str, str]]:
    """GPU agents from the KFD topology, in node order (the ROCr order)."""
    if not topology.is_dir():
        return []
    nodes = []
    for node in topology.iterdir():
        if not node.name.isdigit():
            continue
        try:
            props = dict(line.split(None, 1) for line in
                         (node / "properties").read_text().splitlines() if " " in line)
        except OSError:
            continue
        if int(props.get("simd_count", "0").strip() or 0) <= 0:
            continue  # CPU node
        arch = gfx_from_target_version(int(props.get("gfx_target_version", "0").strip() or 0))
        try:
            name = (node / "name").read_text().strip() or arch
        except OSError:
            name = arch
        nodes.append((int(node.name), name, arch))
    nodes.sort()
    return [{"index": str(i), "name": name, "kind": device_kind_from_name(name, arch),
             "node": str(node_id)}
            for i, (node_id, name, arch) in enumerate(nodes)]


def _visible_filter(devices: list[dict[str, str]], env=None) -> list[dict[str, str]]:
    env = os.environ if env is None else env
    for var in VISIBILITY_VARS:
        raw = env.get(var)
        if raw is None or not raw.strip():
            continue
        wanted = [tok.strip() for tok in raw.split(",") if tok.strip()]
        by_index = {d["index"]: d for d in devices}
        return [by_index[i] for i in wanted if i in by_index]
    return devices


def discover_gpus(env=None) -> list[dict[str, str]]:
    """index/name/kind records of the GPUs this process may use."""
    env = os.environ if env is None else env
    devices = _discover_kfd()
    smi = _discover_rocm_smi()
    if devices:
        by_node = {d["node"]: d for d in smi if d.get("node")}
        devices = [{**d, "name": by_node[d["node"]]["name"], "kind": by_node[d["node"]]["kind"]}
                   if d["node"] in by_node else d for d in devices]
    else:
        devices = smi
    rocr = env.get("ROCR_VISIBLE_DEVICES")
    if devices and rocr and rocr.strip():
        # ROCr renumbers: index k is the k-th device of its list.
        by_index = {d["index"]: d for d in devices}
        picked = [by_index[t.strip()] for t in rocr.split(",") if t.strip() in by_index]
        devices = [{**d, "index": str(k)} for k, d in enumerate(picked)]
    devices = _visible_filter(devices, env)
    return devices or [{"index": "0", "name": "UNKNOWN", "kind": "UNKNOWN"}]


def matching_gpus(device_kind: str | None = None) -> list[dict[str, str]]:
    devices = discover_gpus()
    if not device_kind:
        return devices
    wanted = device_kind.lower()
    return [d for d in devices if d["kind"].lower() == wanted or wanted in d["name"].lower()]


# ---------------------------------------------------------------------------
# Locks
# ---------------------------------------------------------------------------

def _write_lock_metadata(fd: int, *, gpu: str, label: str, device_kind: str = "",
                         mode: str = "exclusive") -> None:
    os.ftruncate(fd, 0)
    os.write(fd, (f"pid={os.getpid()}\ngpu={gpu}\ndevice_kind={device_kind}\n"
                  f"mode={mode}\nlabel={label}\nacquired_unix={time.time():.0f}\n").encode())
    os.fsync(fd)


def read_lock_metadata(lock_path: Path) -> dict[str, str]:
    try:
        text = Path(lock_path).read_text()
    except OSError:
        return {}
    meta = {}
    for line in text.splitlines():
        key, sep, value = line.partition("=")
        if sep:
            meta[key.strip()] = value.strip()
    return meta


def pid_is_alive(pid: str | None) -> bool | None:
    """True / False for a parseable pid, None when there is no usable pid."""
    if not pid:
        return None
    try:
        value = int(pid)
    except ValueError:
        return None
    if value <= 0:
        return False
    try:
        os.kill(value, 0)
    except ProcessLookupError:
        return False
    except PermissionError:
        return True
    return True


def _describe_holder(meta: dict[str, str]) -> str:
    fields = [f"{k}={meta[k]}" for k in
              ("pid", "gpu", "device_kind", "mode", "label", "acquired_unix") if meta.get(k)]
    return ", ".join(fields) if fields else "unknown holder"


def _check_stale(lock_path: Path, stale_since: float | None, now: float) -> float | None:
    """Track how long the holder's pid has been dead; raise past the grace."""
    meta = read_lock_metadata(lock_path)
    if pid_is_alive(meta.get("pid")) is not False:
        return None
    stale_since = now if stale_since is None else stale_since
    if now - stale_since >= STALE_LOCK_GRACE_S:
        raise TimeoutError(f"GPU lock appears stale: {lock_path} reports dead "
                           f"{_describe_holder(meta)}")
    return stale_since


def _acquire(lock_path: Path, op: int, *, timeout_s: float | None, what: str,
             poll_s: float) -> int:
    fd = os.open(lock_path, os.O_CREAT | os.O_RDWR, 0o666)
    start = time.monotonic()
    stale_since = None
    while True:
        try:
            fcntl.flock(fd, op | fcntl.LOCK_NB)
            return fd
        except BlockingIOError:
            now = time.monotonic()
            try:
                stale_since = _check_stale(lock_path, stale_since, now)
            except TimeoutError:
                os.close(fd)
                raise
            if timeout_s is not None and now - start >= timeout_s:
                os.close(fd)
                raise TimeoutError(f"Timed out waiting for {what}: {lock_path} "
                                   f"({_describe_holder(read_lock_metadata(lock_path))})")
            time.sleep(poll_s)


@contextlib.contextmanager
def gpu_lock(gpu: int | str = 0, *, lock_dir: Path | str | None = None,
             timeout_s: float | None = None, label: str = "") -> Iterator[Path]:
    """Exclusive advisory lock of one GPU (for any timing)."""
    directory = Path(lock_dir) if lock_dir is not None else DEFAULT_LOCK_DIR
    directory.mkdir(parents=True, exist_ok=True)
    lock_path = directory / f"gpu_{gpu}.lock"
    fd = _acquire(lock_path, fcntl.LOCK_EX, timeout_s=timeout_s,
                  what=f"GPU {gpu} lock", poll_s=1.0)
    try:
        _write_lock_metadata(fd, gpu=str(gpu), label=label)
        yield lock_path
    finally:
        fcntl.flock(fd, fcntl.LOCK_UN)
        os.close(fd)


@contextlib.contextmanager
def gpu_shared_lock(gpu: int | str = 0, *, lock_dir: Path | str | None = None,
                    timeout_s: float | None = None, label: str = "") -> Iterator[Path]:
    """Shared advisory lock of one GPU (set-up work that must not overlap a
    timing window, but may overlap other set-up work)."""
    directory = Path(lock_dir) if lock_dir is not None else DEFAULT_LOCK_DIR
    directory.mkdir(parents=True, exist_ok=True)
    lock_path = directory / f"gpu_{gpu}.lock"
    fd = _acquire(lock_path, fcntl.LOCK_SH, timeout_s=timeout_s,
                  what=f"shared GPU {gpu} lock", poll_s=0.1)
    try:
        _write_lock_metadata(fd, gpu=str(gpu), label=label, mode="shared")
        yield lock_path
    finally:
        fcntl.flock(fd, fcntl.LOCK_UN)
        os.close(fd)


@contextlib.contextmanager
def gpu_lock_for_kind(device_kind: str | None = None, *,
                      lock_dir: Path | str | None = None, timeout_s: float | None = None,
                      label: str = "", devices=None) -> Iterator[dict[str, str]]:
    """Exclusive lock of any free GPU of a kind; yields its record plus
    `lock_path`.  `devices` overrides discovery (a list of records)."""
    directory = Path(lock_dir) if lock_dir is not None else DEFAULT_LOCK_DIR
    directory.mkdir(parents=True, exist_ok=True)
    start = time.monotonic()
    stale: dict[Path, float | None] = {}
    while True:
        cands = devices if devices is not None else matching_gpus(device_kind)
        if devices is not None and device_kind:
            want = device_kind.lower()
            cands = [d for d in cands if d["kind"].lower() == want or want in d["name"].lower()]
        if not cands:
            have = ", ".join(f"{d['index']}:{d['kind']}:{d['name']}" for d in
                             (devices if devices is not None else discover_gpus()))
            raise RuntimeError(f"No GPUs match device kind {device_kind!r}. Available: {have}")
        for dev in cands:
            lock_path = directory / f"gpu_{dev['index']}.lock"
            fd = os.open(lock_path, os.O_CREAT | os.O_RDWR, 0o666)
            try:
                fcntl.flock(fd, fcntl.LOCK_EX | fcntl.LOCK_NB)
            except BlockingIOError:
                try:
                    stale[lock_path] = _check_stale(lock_path, stale.get(lock_path),
                                                    time.monotonic())
                finally:
                    os.close(fd)
                continue
            try:
                _write_lock_metadata(fd, gpu=dev["index"], device_kind=dev["kind"],
                                     label=label, mode="exclusive")
                yield {**dev, "lock_path": str(lock_path)}
            finally:
                fcntl.flock(fd, fcntl.LOCK_UN)
                os.close(fd)
            return
        if timeout_s is not None and time.monotonic() - start >= timeout_s:
            raise TimeoutError(f"Timed out waiting for GPU kind {device_kind!r}")
        time.sleep(1.0)


def child_env_for_gpu(index: str, env=None) -> dict[str, str]:
    """Environment for a child process pinned to GPU `index` (a ROCr-visible
    index): HIP_VISIBLE_DEVICES = index, no competing CUDA_VISIBLE_DEVICES."""
    out = dict(os.environ if env is None else env)
    out.pop("CUDA_VISIBLE_DEVICES", None)
    out["HIP_VISIBLE_DEVICES"] = str(index)
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="Run a command holding a per-GPU lock.")
    ap.add_argument("--gpu", default=None, help="GPU index to lock and expose")
    ap.add_argument("--device-kind", default=None, help="GPU kind to lock, e.g. MI355X")
    ap.add_argument("--lock-dir", type=Path, default=None)
    ap.add_argument("--timeout-s", type=float, default=None)
    ap.add_argument("--label", default="")
    ap.add_argument("command", nargs=argparse.REMAINDER)
    args = ap.parse_args(argv)
    command = args.command[1:] if args.command and args.command[0] == "--" else args.command
    if not command:
        ap.error("missing command after --")
    label = args.label or " ".join(command[:4])
    if args.device_kind:
        with gpu_lock_for_kind(args.device_kind, lock_dir=args.lock_dir,
                               timeout_s=args.timeout_s, label=label) as dev:
            print(f"[gpu-lock] acquired {dev['lock_path']} ({dev['kind']} {dev['name']})",
                  flush=True)
            return subprocess.run(command, env=child_env_for_gpu(dev["index"])).returncode
    gpu = "0" if args.gpu is None else str(args.gpu)
    with gpu_lock(gpu, lock_dir=args.lock_dir, timeout_s=args.timeout_s,
                  label=label) as lock_path:
        print(f"[gpu-lock] acquired {lock_path}", flush=True)
        return subprocess.run(command, env=child_env_for_gpu(gpu)).returncode


if __name__ == "__main__":
    sys.exit(main())
