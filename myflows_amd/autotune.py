"""Opt-in empirical GEMM plans (MFHIP_GEMM_AUTOTUNE=1): for each (layout, M, N, K) the MFMA
engine's tiles and split-K counts are timed on this device and the fastest is kept, in a JSON file
per shape under MFHIP_AUTOTUNE_CACHE (default: ``myflows_amd/_gemm_plans``). The reference's
``ops/cuda_native/autotune.py:1-195`` plays the same role for its register engine.

Each measurement writes ``{"identity", "layout", "shape", "candidates", "selected"}``. A file is
used only when its identity (device name, arch, CU count, HIP runtime, library build) and shape
match. Every one-group tile adds each output's K terms in the same order, so all unsplit
candidates of one K-group count must agree bit for bit; a disagreement raises instead of being
stored.
"""

from __future__ import annotations

import fcntl
import hashlib
import json
import os
import random
import statistics
import time
from contextlib import contextmanager
from functools import lru_cache
from pathlib import Path

import torch

from . import native

VERSION = 1
SPLIT_CHOICES = (1, 2, 3, 4, 6, 8, 12, 16, 24, 32, 48, 64)
LAYOUTS = ("NN", "NT", "TN")


def _library_digest():
    path = native.LIBRARY_PATH
    return hashlib.sha256(path.read_bytes()).hexdigest()[:16] if path.exists() else "missing"


@lru_cache(maxsize=8)
def device_identity(device_index):
    props = torch.cuda.get_device_properties(device_index)
    identity = {"name": props.name, "arch": getattr(props, "gcnArchName", ""), "cus": props.multi_processor_count,
                "hip": torch.version.hip, "library": _library_digest(), "version": VERSION}
    return hashlib.sha256(json.dumps(identity, sort_keys=True).encode()).hexdigest()[:24], identity


def cache_root():
    configured = os.environ.get("MFHIP_AUTOTUNE_CACHE")
    return Path(configured) if configured else Path(__file__).resolve().parent / "_gemm_plans"


def plan_file(layout, m, n, k, device_index=None):
    key, _ = device_identity(torch.cuda.current_device() if device_index is None else device_index)
    return cache_root() / key / f"{layout}-{m}x{n}x{k}.json"


def read_plan(path, layout, shape, identity):
    """(tile, requested slices) from a stored measurement, or None if it is missing or stale."""
    try:
        record = json.loads(Path(path).read_text(encoding="utf-8"))
        if record["identity"] != identity or record["layout"] != layout or record["shape"] != list(shape):
            return None
        tile, requested = record["selected"]["tile"], record["selected"]["requested_slices"]
        native._plan_code(tile, requested)  # still a valid plan of this library
        return tile, requested
    except (OSError, ValueError, KeyError, TypeError):
        return None


def write_plan(path, record):
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    scratch = path.with_name(f"{path.name}.{os.getpid()}.tmp")
    scratch.write_text(json.dumps(record, indent=1, allow_nan=False), encoding="utf-8")
    os.replace(scratch, path)


@contextmanager
def _locked(directory):
    directory.mkdir(parents=True, exist_ok=True)
    with open(directory / ".lock", "w") as handle:
        fcntl.flock(handle, fcntl.LOCK_EX)
        try:
            yield
        finally:
            fcntl.flock(handle, fcntl.LOCK_UN)


def candidates(m, n, k, workspace_budget_bytes):
    """[(tile, requested, slices, workspace bytes)] with one entry per distinct slice count."""
    rows = []
    for tile, entry in native.tile_catalog().items():
        seen = set()
        for requested in SPLIT_CHOICES:
            slices = native._slices(k, requested, entry[-1])
            if slices in seen:
                continue
            seen.add(slices)
            workspace = 4 * slices * m * n if slices > 1 else 0
            if workspace <= workspace_budget_bytes:
                rows.append((tile, requested, slices, workspace))
    return rows


def measure(layout, m, n, k, repeats=3, rounds=3, seed=197):
    """Time every candidate plan of one GEMM shape; returns the record that write_plan stores."""
    trans_a, trans_b = layout == "TN", layout == "NT"
    gen = torch.Generator(device="cuda").manual_seed(seed)
    a = torch.randn((k, m) if trans_a else (m, k), device="cuda", generator=gen)
    b = torch.randn((n, k) if trans_b else (k, n), device="cuda", generator=gen)
    out = torch.empty((m, n), device="cuda")
    free, total = torch.cuda.mem_get_info()
    budget = max(0, int(free) - max(512 << 20, int(total) // 8))
    rows = [{"tile": t, "requested_slices": r, "slices": s, "workspace_bytes": w, "times_ms": []}
            for t, r, s, w in candidates(m, n, k, budget)]
    launch = lambda row: native.gemm(a, b, trans_a=trans_a, trans_b=trans_b, out=out,
                                     plan=(row["tile"], row["requested_slices"]))
    reference_bits = {}
    for row in rows:  # correctness pass: the unsplit tiles of one K-group count must give the same bits
        launch(row)
        if row["slices"] == 1:
            bits, groups = out.clone(), native.tile_groups(row["tile"])
            if groups not in reference_bits:
                reference_bits[groups] = bits
            elif not torch.equal(bits, reference_bits[groups]):
                raise ArithmeticError(f"unsplit tile {row['tile']} changed the summation order of {layout} {m}x{n}x{k}")
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    order = random.Random(2201)
    began = time.monotonic()
    for _ in range(rounds):
        order.shuffle(rows)
        for row in rows:
            start.record()
            for _ in range(repeats):
                launch(row)
            stop.record()
            stop.synchronize()
            row["times_ms"].append(start.elapsed_time(stop) / repeats)
    for row in rows:
        row["median_ms"] = statistics.median(row["times_ms"])
    best = min(rows, key=lambda row: row["median_ms"])
    auto_tile, auto_slices = native.gemm_plan(m, n, k)
    _, identity = device_identity(torch.cuda.current_device())
    return {"identity": identity, "layout": layout, "shape": [m, n, k], "candidates": rows, "selected": best,
            "automatic": {"tile": auto_tile, "slices": auto_slices}, "seconds": time.monotonic() - began}


@lru_cache(maxsize=4096)
def _selected(root, device_index, layout, m, n, k):
    path = plan_file(layout, m, n, k, device_index)
    _, identity = device_identity(device_index)
    found = read_plan(path, layout, (m, n, k), identity)
    if found:
        return found
    with _locked(path.parent):
        found = read_plan(path, layout, (m, n, k), identity)  # another process may have measured it
        if found:
            return found
        record = measure(layout, m, n, k)
        write_plan(path, record)
        return record["selected"]["tile"], record["selected"]["requested_slices"]


def selected_plan(layout, m, n, k):
    """(tile name, requested split count) for an op(A) op(B) GEMM of this shape on this device."""
    if layout not in LAYOUTS or min(m, n, k) < 1:
        raise ValueError("expected layout NN, NT or TN and positive GEMM dimensions")
    return _selected(str(cache_root()), torch.cuda.current_device(), layout, int(m), int(n), int(k))
