"""Autotuned GEMM plans: the on-disk record round trip and its validation (CPU), and one real
measurement on the GPU."""

import json

import pytest
import torch

from myflows_amd import autotune, native


def test_plan_record_round_trip_and_stale_records(tmp_path):
    identity = {"name": "gfx950 test", "cus": 256}
    record = {"identity": identity, "layout": "TN", "shape": [64, 576, 72384],
              "selected": {"tile": "64x128", "requested_slices": 8}, "candidates": []}
    path = tmp_path / "key" / "TN-64x576x72384.json"
    autotune.write_plan(path, record)
    assert autotune.read_plan(path, "TN", (64, 576, 72384), identity) == ("64x128", 8)
    assert autotune.read_plan(path, "NN", (64, 576, 72384), identity) is None  # another layout
    assert autotune.read_plan(path, "TN", (64, 576, 72385), identity) is None  # another shape
    assert autotune.read_plan(path, "TN", (64, 576, 72384), {**identity, "cus": 304}) is None  # another device
    record["selected"]["tile"] = "7x7"
    path.write_text(json.dumps(record))
    assert autotune.read_plan(path, "TN", (64, 576, 72384), identity) is None  # not a plan of this library
    path.write_text("{not json")
    assert autotune.read_plan(path, "TN", (64, 576, 72384), identity) is None


def test_candidates_are_distinct_and_within_budget():
    rows = autotune.candidates(64, 576, 72384, workspace_budget_bytes=64 << 20)
    assert rows and all(w <= 64 << 20 for *_, w in rows)
    for tile in native.tile_catalog():
        slices = [s for t, _, s, _ in rows if t == tile]
        assert len(slices) == len(set(slices)) and 1 in slices
    with pytest.raises(ValueError):
        autotune.selected_plan("TT", 4, 4, 4)


@pytest.mark.gpu
def test_measured_plan_is_stored_and_used(tmp_path, monkeypatch):
    monkeypatch.setenv("MFHIP_AUTOTUNE_CACHE", str(tmp_path))
    record = autotune.measure("TN", 96, 80, 2560, repeats=1, rounds=1)  # raises if unsplit tiles disagree
    assert record["selected"]["median_ms"] == min(c["median_ms"] for c in record["candidates"])
    tile, requested = autotune.selected_plan("TN", 96, 80, 2560)
    assert autotune.plan_file("TN", 96, 80, 2560).exists()
    monkeypatch.setenv("MFHIP_GEMM_AUTOTUNE", "1")
    gen = torch.Generator(device="cuda").manual_seed(3)
    a, b = torch.randn((2560, 96), device="cuda", generator=gen), torch.randn((2560, 80), device="cuda", generator=gen)
    tuned = native.gemm(a, b, trans_a=True)
    explicit = native.gemm(a, b, trans_a=True, plan=(tile, requested))
    assert torch.equal(tuned, explicit)
