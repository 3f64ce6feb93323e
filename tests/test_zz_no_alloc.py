"""dip_mlp_decode_noalloc (the decode step whose workspace is the library's
per-GPU scratch array) against dip_mlp_decode with a caller workspace,
through the C ABI: calls in a row, each with a smaller layer than the one
before, with and without the speculation state, with and without the group-major copy of
down_t's scales, plus a shape the scratch cannot hold.  Outputs must be
bit-identical (the same kernels on the same inputs).  In a fresh process the
very first call is made inside a HIP graph capture (the scratch address is
looked up then), the graph is replayed several times, and eager calls leave
the device's free memory unchanged."""
import os
import subprocess
import sys
import textwrap
from pathlib import Path

import numpy as np
import pytest
import torch

import dip_oracle as O
from gpu_util import dev, dev_bf16, host_bf16

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def K():
    import _dip_hip
    return _dip_hip


def _layer(H, I, seed):
    L = O.make_layer(H, I, seed=seed)
    return L, {n: (dev_bf16(v) if v.dtype == np.uint16 else dev(v)) for n, v in L.items()}


def _outs(H, I, k, fill):
    d = torch.device("cuda:0")
    return (torch.full((H,), fill, dtype=torch.bfloat16, device=d),
            torch.full((I,), fill, dtype=torch.bfloat16, device=d),
            torch.full((k,), -7, dtype=torch.int32, device=d),
            torch.full((k,), fill, dtype=torch.bfloat16, device=d))


@pytest.mark.parametrize("spec,gm", [(False, False), (True, False), (False, True), (True, True)],
                         ids=["stagewise", "speculative", "stagewise-gm", "speculative-gm"])
def test_noalloc_equals_workspace_entry_point(K, spec, gm):
    _noalloc_cases(K, spec, gm)


def _noalloc_cases(K, spec, use_gm):
    # each call smaller than the one before; hidden 4096 takes the down
    # launch that reduces its own partials (arrival counters in the scratch)
    # in the speculative step with group-major scales on a full 256-CU gfx950
    cases = [(5120, 25600, 0.6, 0), (4096, 12288, 0.6, 2), (1024, 3072, 0.3, 1)]
    st_ref = K.mlp_state(torch.device("cuda:0")) if spec else None
    st_new = K.mlp_state(torch.device("cuda:0")) if spec else None
    for H, I, keep, seed in cases:
        print(f"noalloc case H={H} I={I} keep={keep} spec={spec}", flush=True)
        L, D = _layer(H, I, seed)
        gm = K.scales_group_major(D["down_t_sc"]) if use_gm else None
        k = O.keep_count(I, keep)
        for tok in range(2):
            x = dev_bf16(O.make_x(H, seed=100 + tok))
            ref = K.mlp_decode(D["gate_qw"], D["gate_sc"], D["up_qw"], D["up_sc"], D["down_t_qw"],
                               D["down_t_sc"], x, k, state=st_ref, down_t_sc_gm=gm)
            y, g, idx, h = _outs(H, I, k, 3.0)
            K.mlp_decode_noalloc(D["gate_qw"], D["gate_sc"], D["up_qw"], D["up_sc"],
                                 D["down_t_qw"], D["down_t_sc"], x, k, y=y, g=g, idx=idx, h=h,
                                 state=st_new, down_t_sc_gm=gm)
            torch.cuda.synchronize()
            for name, a, b in zip(("y", "g", "idx", "h"), ref, (y, g, idx, h)):
                assert torch.equal(a, b), (name, H, I, tok)
            if spec:
                assert torch.equal(st_ref, st_new)
            # and against the oracle: idx bit-exact on the device's g
            assert np.array_equal(idx.cpu().numpy(), O.topk_select(host_bf16(g), k))


def test_noalloc_rejects_shapes_beyond_the_scratch(K):
    H, I = 16384, 65536
    nbytes = K.lib.dip_mlp_workspace_size(H, I, I)
    assert nbytes > 16 << 20
    st = K.lib.dip_mlp_decode_noalloc(16, 16, 16, 16, 16, 16, None, 16, 16, 16, 16, 16, H, I, I,
                                      None, None)
    assert st == -7 and b"no-alloc scratch" in K.lib.dip_status_string(st)


_CAPTURE_SCRIPT = textwrap.dedent("""
    import sys
    import numpy as np
    import torch
    sys.path[:0] = [sys.argv[1], sys.argv[2], sys.argv[3]]
    import _dip_hip as K
    import dip_oracle as O
    from gpu_util import dev, dev_bf16

    H, I = int(sys.argv[4]), int(sys.argv[5])
    k = O.keep_count(I, 0.6)
    L = O.make_layer(H, I, seed=3)
    D = {n: (dev_bf16(v) if v.dtype == np.uint16 else dev(v)) for n, v in L.items()}
    W = [D[n] for n in ("gate_qw", "gate_sc", "up_qw", "up_sc", "down_t_qw", "down_t_sc")]
    gm = K.scales_group_major(D["down_t_sc"])
    x = dev_bf16(O.make_x(H, seed=7))
    out = [torch.empty(H, dtype=torch.bfloat16, device="cuda"),
           torch.empty(I, dtype=torch.bfloat16, device="cuda"),
           torch.empty(k, dtype=torch.int32, device="cuda"),
           torch.empty(k, dtype=torch.bfloat16, device="cuda")]
    st_new = K.mlp_state(torch.device("cuda:0"))
    torch.cuda.synchronize()
    # the first call of the process on this device, under capture
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            K.mlp_decode_noalloc(*W, x, k, y=out[0], g=out[1], idx=out[2], h=out[3],
                                 state=st_new, down_t_sc_gm=gm)
    torch.cuda.synchronize()
    st_ref = K.mlp_state(torch.device("cuda:0"))
    for rep in range(4):
        x.copy_(dev_bf16(O.make_x(H, seed=20 + rep)))
        torch.randn(1000, device="cuda").sum().item()  # unrelated eager work
        graph.replay()
        ref = K.mlp_decode(*W, x, k, state=st_ref, down_t_sc_gm=gm)
        torch.cuda.synchronize()
        for name, a, b in zip(("y", "g", "idx", "h"), ref, out):
            assert torch.equal(a, b), (name, rep)
        assert torch.equal(st_ref, st_new), rep
    # eager calls allocate nothing: the device's free memory stays the same
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    for rep in range(3):
        K.mlp_decode_noalloc(*W, x, k, y=out[0], g=out[1], idx=out[2], h=out[3],
                             state=st_new, down_t_sc_gm=gm)
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0
    print("capture-first ok", flush=True)
""")


# hidden 4096: the replays run the down launch that reduces its own partials
# with its arrival counters in the scratch
@pytest.mark.parametrize("H,I", [(2560, 9728), (4096, 12288)])
def test_noalloc_first_call_under_graph_capture(tmp_path, H, I):
    root = Path(__file__).resolve().parents[1]
    script = tmp_path / "capture_first.py"
    script.write_text(_CAPTURE_SCRIPT)
    paths = [str(root / "dynamic-input-pruning_amd"), str(root / "oracle"), str(root / "tests")]
    print(f"noalloc capture-first subprocess H={H} I={I}", flush=True)
    proc = subprocess.run([sys.executable, str(script), *paths, str(H), str(I)], capture_output=True, text=True,
                          timeout=300, env=dict(os.environ))
    assert proc.returncode == 0, proc.stdout[-2000:] + proc.stderr[-4000:]
    assert "capture-first ok" in proc.stdout
