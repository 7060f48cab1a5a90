"""Helpers to drive the C++17 drop-in layer through tests/cxx/bin/dropin_probe
(raw little-endian files in, raw files out)."""
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
PROBE = os.path.join(HERE, "cxx", "bin", "dropin_probe")
ROOT = os.path.dirname(HERE)
BIN = os.path.join(ROOT, "cwlb-spmm_amd", "bin")


class ProbeError(Exception):
    def __init__(self, kind, msg):
        super().__init__(f"{kind}: {msg}")
        self.kind = kind
        self.msg = msg


def probe(*args, cwd=None, timeout=300, env=None):
    if not os.path.exists(PROBE):
        raise RuntimeError(f"{PROBE} missing: build with __graft_entry__.build()")
    r = subprocess.run([PROBE, *map(str, args)], capture_output=True, text=True, cwd=cwd,
                       timeout=timeout, env=None if env is None else {**os.environ, **env})
    out = r.stdout
    if r.returncode == 3:
        line = [ln for ln in out.splitlines() if "EXC " in ln][-1]
        _, kind, msg = line[line.index("EXC "):].split(" ", 2)
        raise ProbeError(kind, msg)
    if r.returncode != 0:
        raise RuntimeError(f"probe {args[0]} exited {r.returncode}: {r.stderr[-2000:]}")
    return out


def write_csr(path, rp, ci, val):
    rp, ci, val = (np.asarray(rp, np.int32), np.asarray(ci, np.int32),
                   np.asarray(val, np.float32))
    with open(path, "wb") as f:
        np.array([len(rp) - 1, len(ci)], np.int64).tofile(f)
        rp.tofile(f)
        ci.tofile(f)
        val.tofile(f)


def write_order(path, origin, rp, ci, val):
    with open(path, "wb") as f:
        np.array([len(origin), len(ci)], np.int64).tofile(f)
        for a, t in ((origin, np.int32), (rp, np.int32), (ci, np.int32), (val, np.float32)):
            np.asarray(a, t).tofile(f)


def read_order(path):
    raw = open(path, "rb").read()
    n, nnz = np.frombuffer(raw[:16], np.int64)
    off = 16
    out = []
    for cnt, t in ((n, np.int32), (n + 1, np.int32), (nnz, np.int32), (nnz, np.float32)):
        a = np.frombuffer(raw[off:off + 4 * int(cnt)], t).copy()
        off += 4 * int(cnt)
        out.append(a)
    return tuple(out)


def read_csr(path):
    raw = open(path, "rb").read()
    n, nnz = np.frombuffer(raw[:16], np.int64)
    off = 16
    rp = np.frombuffer(raw[off:off + 4 * (n + 1)], np.int32).copy()
    off += 4 * (n + 1)
    ci = np.frombuffer(raw[off:off + 4 * nnz], np.int32).copy()
    off += 4 * nnz
    val = np.frombuffer(raw[off:off + 4 * nnz], np.float32).copy()
    return rp, ci, val


def write_f32(path, a):
    np.ascontiguousarray(a, np.float32).tofile(path)


def write_tasks(path, tasks):
    np.ascontiguousarray(tasks, np.int32).reshape(-1).tofile(path)
