"""The timeline build of the library (libdip_hip_timeline.so): bench.py
--timeline decodes a short stack with it and reads every decode kernel's
per-workgroup stamps back through dip_timeline_read.  Run in a child process,
since the bindings load one library per process."""
import json
import os
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


_XCD_SCRIPT = """
import os, sys
sys.path[:0] = [sys.argv[1], sys.argv[2], sys.argv[3]]
import numpy as np
import torch
import _dip_hip as K
import dip_oracle as O
from gpu_util import dev, dev_bf16
H, I = 4096, 12288
L = O.make_layer(H, I, seed=5)
D = {n: (dev_bf16(v) if v.dtype == np.uint16 else dev(v)) for n, v in L.items()}
gm = K.scales_group_major(D["down_t_sc"])
x = dev_bf16(O.make_x(H, seed=9))
# the speculative step (state given) with group-major scales: its down
# launch reduces its own partials
st = K.mlp_state(torch.device("cuda:0"))
K.mlp_decode(D["gate_qw"], D["gate_sc"], D["up_qw"], D["up_sc"], D["down_t_qw"], D["down_t_sc"],
             x, O.keep_count(I, 0.6), state=st, down_t_sc_gm=gm)
torch.cuda.synchronize()
for name in ("gate", "down_partials"):
    start, end, xcc = K.timeline_read(name)
    print(name, len(xcc), " ".join(str(int(v)) for v in xcc), flush=True)
"""


@pytest.mark.gpu
def test_workgroups_equal_mod_8_share_an_xcd(tmp_path):
    """The down launch's in-launch reduce relies on the dispatcher placing
    workgroup b on XCD (b + c) mod 8 for one c per launch: every tile of a
    column block runs on one XCD, so its partials and arrival counter stay in
    that XCD's L2.  The timeline build records each workgroup's XCC_ID."""
    import torch
    props = torch.cuda.get_device_properties(0)
    if not (props.gcnArchName.startswith("gfx950") and props.multi_processor_count == 256):
        pytest.skip("the in-launch reduce runs on a full 256-CU gfx950 only")
    script = tmp_path / "xcd.py"
    script.write_text(_XCD_SCRIPT)
    env = dict(os.environ,
               DIP_HIP_LIB=str(ROOT / "dynamic-input-pruning_amd" / "libdip_hip_timeline.so"))
    print("xcd grouping subprocess H=4096 I=12288", flush=True)
    out = subprocess.run([sys.executable, str(script), str(ROOT / "dynamic-input-pruning_amd"),
                          str(ROOT / "oracle"), str(ROOT / "tests")],
                         capture_output=True, text=True, timeout=300, env=env)
    assert out.returncode == 0, out.stdout[-2000:] + out.stderr[-4000:]
    lines = [l.split() for l in out.stdout.splitlines() if l.split()[:1] in (["gate"],
                                                                            ["down_partials"])]
    assert [l[0] for l in lines] == ["gate", "down_partials"]
    for l in lines:
        blocks, xcc = int(l[1]), [int(v) for v in l[2:]]
        assert blocks == len(xcc) >= 64, l[0]
        assert sorted(set(xcc[:8])) == list(range(8)), (l[0], xcc[:8])
        assert all(xcc[b] == xcc[b % 8] for b in range(blocks)), l[0]
