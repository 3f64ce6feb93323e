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
        assert b.measured_traffic("qwen3-32b", 0.3, "gate_silu", K) is None  # no summary
        K.set_tuning("spec_margin", old + 1)  # other tuning: the figure no longer applies
        assert b.measured_traffic("qwen3-32b", 0.6, "gate_silu", K) is None
    finally:
        K.set_tuning("spec_margin", old)


def test_probe_library_is_separate_and_checks_its_arguments():
    """The read-ceiling probes are a library of their own (bench.py --ceiling
    loads it); the decode library exports none of them.  Bad arguments are
    rejected before any launch (no GPU needed)."""
    import ctypes
    lib = ctypes.CDLL(str(ROOT / "dynamic-input-pruning_amd" / "libdip_probe.so"))
    _p, _i64, _i = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    lib.dip_probe_read.argtypes = [_p, ctypes.c_size_t, _i, _i, _p, _p]
    lib.dip_probe_gather.argtypes = [_p, _i64, _i64, _p, _i64, _i, _i, _p, _p]
    buf = (ctypes.c_uint8 * 64)()
    p = ctypes.addressof(buf) + (-ctypes.addressof(buf) % 16)
    assert lib.dip_probe_read(None, 16, 1, 4, p, None) == -1
    assert lib.dip_probe_read(p, 24, 1, 4, p, None) == -2
    assert lib.dip_probe_read(p + 2, 32, 1, 4, p, None) == -3
    assert lib.dip_probe_read(p, 32, 0, 4, p, None) == -6
    assert lib.dip_probe_read(p, 32, 1, 3, p, None) == -6
    assert lib.dip_probe_gather(p, 100, 2560, None, 10, 1, 4, p, None) == -1
    assert lib.dip_probe_gather(p, 100, 2600, p, 10, 1, 4, p, None) == -2
    assert lib.dip_probe_gather(p, 100, 8192, p, 10, 1, 4, p, None) == -2
    assert lib.dip_probe_gather(p, 0, 2560, p, 10, 1, 4, p, None) == -2
    assert lib.dip_probe_gather(p, 100, 2560, p, 10, 1, 5, p, None) == -6
    assert not hasattr(K.lib, "dip_probe_read") and not hasattr(K.lib, "dip_gather_probe")


def test_cache_aware_mode_refuses_the_profiler(monkeypatch, capsys):
    """bench.py --ca exits with status 3 before any GPU call when rocprofv3's
    environment is present, and runs otherwise (here: no variable set)."""
    b = _bench()
    for n in [n for n in list(__import__("os").environ) if n.startswith("ROCPROF")]:
        monkeypatch.delenv(n)
    assert b.profiler_env() == []
    monkeypatch.setenv("ROCPROF_OUTPUT_PATH", "/tmp/prof")
    assert b.profiler_env() == ["ROCPROF_OUTPUT_PATH"]
    assert b.main(["--ca", "0.3"]) == 3
    assert "does not run under rocprofv3" in capsys.readouterr().err


def test_timeline_refuses_the_dense_route(capsys):
    """--timeline reads the DIP step's per-workgroup stamps; at keep >= 0.999
    the stack runs the dense route (no top-k launch), so the mode exits with
    status 2 before any GPU call."""
    b = _bench()
    assert b.main(["--timeline", "--keep", "1.0"]) == 2
    assert "dense route" in capsys.readouterr().err


def test_traffic_of_the_dense_route():
    """keep 1.0 (the dense route) has its own summary: the stages the dense
    stack times, each at least the I weight rows it must read."""
    b = _bench()
    for stage in ("gate_silu", "up_gather_h", "down_gather"):
        v = b.measured_traffic("qwen3-32b", 1.0, stage, K)
        assert v is not None and v >= 25600 * 2640, stage
    assert b.measured_traffic("qwen3-32b", 1.0, "topk_spec_up", K) is None
