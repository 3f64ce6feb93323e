"""dip_mlp_decode_noalloc (the decode step whose workspace is the library's
per-GPU scratch array) against dip_mlp_decode with a caller workspace,
through the C ABI: two calls in a row, the second with a smaller layer, with
and without the speculation state (both step forms), with and without the
group-major copy of down_t's scales, plus a shape the scratch cannot hold.
Outputs must be bit-identical (the same kernels on the same inputs)."""
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


@pytest.mark.parametrize("spec,step,gm", [(False, 0, False), (True, 0, False), (True, 1, False),
                                          (True, 2, False), (False, 0, True), (True, 0, True),
                                          (True, 2, True)],
                         ids=["stagewise", "four-launch", "fused", "split", "stagewise-gm",
                              "four-launch-gm", "split-gm"])
def test_noalloc_equals_workspace_entry_point(K, spec, step, gm):
    old = K.get_tuning("step")
    K.set_tuning("step", step)
    try:
        _noalloc_cases(K, spec, gm)
    finally:
        K.set_tuning("step", old)


def _noalloc_cases(K, spec, use_gm):
    cases = [(5120, 25600, 0.6, 0), (1024, 3072, 0.3, 1)]   # second call smaller
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
