"""bench.py's reading of the committed traffic summary (CPU only)."""

import json
import runpy
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def _bench():
    return runpy.run_path(str(ROOT / "bench.py"), run_name="bench_contract")


def test_traffic_summary_is_reported_for_its_own_sources(tmp_path, monkeypatch):
    """A summary whose digest names the current sources is reported as is."""
    bench = _bench()
    data = json.loads((ROOT / "profiles" / "traffic.json").read_text())
    digest = bench["source_digest"]()
    data["_sources"] = digest
    (tmp_path / "profiles").mkdir()
    (tmp_path / "profiles" / "traffic.json").write_text(json.dumps(data))
    load = bench["load_traffic"]
    monkeypatch.setitem(load.__globals__, "ROOT", str(tmp_path))
    monkeypatch.setitem(load.__globals__, "source_digest", lambda: digest)
    assert load("gemm_fp8_block") == data["gemm_fp8_block"]


def test_stale_traffic_summary_is_not_reported(tmp_path, monkeypatch):
    """A summary taken on other sources is ignored (traffic null), not
    reported as if it described the current kernels."""
    bench = _bench()
    data = json.loads((ROOT / "profiles" / "traffic.json").read_text())
    data["_sources"] = "0" * 16
    (tmp_path / "profiles").mkdir()
    (tmp_path / "profiles" / "traffic.json").write_text(json.dumps(data))
    load = bench["load_traffic"]
    monkeypatch.setitem(load.__globals__, "ROOT", str(tmp_path))
    monkeypatch.setitem(load.__globals__, "source_digest", lambda: "1" * 16)
    assert load("gemm_fp8_block") is None
