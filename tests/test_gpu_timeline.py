"""The timeline build of the library (libdip_hip_timeline.so): bench.py
--timeline decodes a short stack with it and reads every decode kernel's
per-workgroup stamps back through dip_timeline_read.  Run in a child process,
since the bindings load one library per process."""
import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.mark.gpu
@pytest.mark.parametrize("shape", ["qwen3-32b", "qwen3-8b"])
def test_layer_timeline_is_ordered(shape):
    out = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--timeline", "--shape", shape,
                          "--layers", "3", "--steps", "4", "--warmup", "2"],
                         capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr[-2000:]
    rec = json.loads(out.stdout.strip().splitlines()[-1])
    ks = rec["kernels"]
    # hidden 4096 on a full 256-CU gfx950: the down partials' launch reduces
    # them itself (no reduce kernel); hidden 5120 keeps the reduce launch
    import torch
    props = torch.cuda.get_device_properties(0)
    in_launch = (shape == "qwen3-8b" and props.gcnArchName.startswith("gfx950")
                 and props.multi_processor_count == 256)
    assert list(ks) == ["gate", "topk_spec_up", "down_partials"] + ([] if in_launch
                                                                    else ["down_reduce"])
    for name, k in ks.items():
        assert k["finished"] > 0, name
        assert k["first_start"] <= k["last_start"] <= k["last_end"], name
        assert k["first_end"] <= k["end_p50"] <= k["last_end"], name
    assert ks["gate"]["first_start"] == 0.0
    # stream order: each kernel's workgroups start after the previous one's end
    order = list(ks)
    for a, b in zip(order, order[1:]):
        assert ks[b]["first_start"] >= ks[a]["last_end"], (a, b)
        assert rec["gap_us"][f"{a}->{b}"] >= 0
    # the down grid pads row blocks to a multiple of 8 XCDs: padding tiles
    # start but never reach the end of the kernel
    assert ks["down_partials"]["finished"] <= ks["down_partials"]["workgroups"]
    # one layer's kernels fit in one layer period
    assert rec["layer_span_us"] <= rec["layer_period_us"] * 1.5
