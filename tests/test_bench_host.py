"""Host-side pieces of bench.py that need no GPU: the metric names per
workload and the HBM traffic figure read from the committed counter summary
(reported only while the live launch tuning is the one it was measured
with)."""
import argparse
import importlib.util
from pathlib import Path

import _dip_hip as K

ROOT = Path(__file__).resolve().parent.parent


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _args(**kw):
    base = dict(checkpoint=None, shape="qwen3-32b", keep=0.6, layers=None)
    base.update(kw)
    return argparse.Namespace(**base)


def test_metric_names():
    b = _bench()
    assert b.metric_name(_args()) == b.METRIC
    assert "Qwen3-8B" in b.metric_name(_args(shape="qwen3-8b"))
    assert "keep=0.3" in b.metric_name(_args(keep=0.3))
    assert b.metric_name(_args(layers=8)) != b.METRIC
    assert "checkpoint" in b.metric_name(_args(checkpoint="/x"))


def test_traffic_from_the_committed_summary():
    b = _bench()
    text = (ROOT / "profiles" / "hbm_traffic_qwen3-32b_keep0.6.md").read_text()
    line = next(l for l in text.splitlines() if l.startswith("traffic_bytes_per_launch:"))
    table = dict(item.split("=") for item in line.split(":", 1)[1].split())
    # every stage the bench names, at least the algorithmic bytes of the gate
    assert set(table) == {"gate_silu", "topk_spec_up", "down_gather"}
    assert int(table["gate_silu"]) >= 25600 * 2640
    old = K.get_tuning("spec_margin")
    try:
        live = b.measured_traffic("qwen3-32b", 0.6, "gate_silu", K)
        assert live == int(table["gate_silu"])
        assert b.measured_traffic("qwen3-8b", 0.6, "gate_silu", K) is None  # no summary
        K.set_tuning("spec_margin", old + 1)  # other tuning: the figure no longer applies
        assert b.measured_traffic("qwen3-32b", 0.6, "gate_silu", K) is None
    finally:
        K.set_tuning("spec_margin", old)
