"""The down stage's in-launch (XCD-local) reduce: with the group-major scales
and out_features a multiple of 2048 (at most 8192), the decode step's down
kernel lets the last tile of each column block sum its partials inside the
same launch on a full 256-CU gfx950.  It must give y bit for bit as the
reduce launch does (the same summation order), leave its arrival counters at
zero for the next call on the same workspace, and do so for any row-block
count."""
import numpy as np
import pytest
import torch

import dip_oracle as O
from gpu_util import dev, dev_bf16, host_bf16, random_bf16, random_int4

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def K():
    import _dip_hip
    return _dip_hip


def _bits(t):
    return t.view(torch.int16)


def _counters(K):
    ws = K._ws_cache[(torch.cuda.current_device(), "down")]
    return ws[:8192]


@pytest.mark.parametrize("out_f", [2048, 4096, 8192, 5120])
def test_in_launch_reduce_same_bits_over_successive_calls(K, out_f):
    """Successive calls on one workspace with 1, 1, 2, 9, 12 and 17 row
    blocks (k of 1, 256, 257, 2049, 3000 and 4100 of 4100 rows): y and h_out
    bit for bit those of the general kernel and its reduce launch (no
    group-major scales), y within the oracle's bar, and every arrival counter
    back at zero after each call.  out_f 5120 (20 column blocks) keeps the
    reduce launch."""
    rng = np.random.default_rng(out_f)
    rows = 4100
    qw, sc = random_int4(rng, rows, out_f)
    d_qw, d_sc = dev(qw), dev_bf16(sc)
    gm = K.scales_group_major(d_sc)
    for k in (1, 256, 257, 2049, 3000, rows):
        idx = np.sort(rng.permutation(rows)[:k]).astype(np.int32)
        h_full = random_bf16(rng, rows)
        d_h, d_idx = dev_bf16(h_full), dev(idx)
        outs = []
        for g in (None, gm):
            h_out = torch.empty(k, dtype=torch.bfloat16, device="cuda")
            y = K.int4_gather_down_by_channel(d_qw, d_sc, d_h, d_idx, h_out=h_out, scales_gm=g)
            outs.append((y.clone(), h_out))
        torch.cuda.synchronize()
        assert torch.equal(_bits(outs[0][0]), _bits(outs[1][0])), k
        assert torch.equal(_bits(outs[0][1]), _bits(outs[1][1])), k
        assert int(_counters(K).count_nonzero()) == 0, k
        ref = O.down_f64(qw, sc, h_full[idx], rows=idx)
        err = np.abs(O.bf16_to_f32(host_bf16(outs[1][0])) - ref).max() / np.abs(ref).max()
        assert err < 1e-2, (k, err)


def test_in_launch_reduce_bad_ids(K):
    """Out-of-range channel ids poison their tiles' partials, so every
    output of the in-launch reduce is NaN too, as through the reduce launch,
    and the counters still end at zero."""
    rng = np.random.default_rng(17)
    rows, k, out_f = 600, 300, 2048
    qw, sc = random_int4(rng, rows, out_f)
    idx = np.sort(rng.permutation(rows)[:k]).astype(np.int32)
    idx[[5, 100]] = [rows, -3]
    h_full = random_bf16(rng, rows)
    d_qw, d_sc, d_h, d_idx = dev(qw), dev_bf16(sc), dev_bf16(h_full), dev(idx)
    gm = K.scales_group_major(d_sc)
    outs = [K.int4_gather_down_by_channel(d_qw, d_sc, d_h, d_idx, scales_gm=g).clone()
            for g in (None, gm)]
    torch.cuda.synchronize()
    assert torch.equal(_bits(outs[0]), _bits(outs[1]))
    assert torch.isnan(outs[1].float()).all()
    assert int(_counters(K).count_nonzero()) == 0


def test_decode_step_8b_in_launch_reduce_matches_stage_by_stage(K):
    """The Qwen3-8B decode step (hidden 4096: the in-launch reduce) against
    the same step without the layer state (five launches, reduce launch),
    three tokens: y, g, idx and h bit for bit."""
    from dip_stack import DIPStack
    gen = torch.Generator(device="cuda").manual_seed(4)
    st = DIPStack(4096, 12288, 1, 0.6, "cuda:0", seed=9)
    lw = st.w[0]
    state = K.mlp_state(torch.device("cuda:0"))
    for t in range(3):
        x = torch.randn(4096, device="cuda", generator=gen).to(torch.bfloat16)
        a = K.mlp_decode(lw["gate_qw"], lw["gate_sc"], lw["up_qw"], lw["up_sc"], lw["down_t_qw"],
                         lw["down_t_sc"], x, st.k, state=state, down_t_sc_gm=lw["down_t_sc_gm"])
        b = K.mlp_decode(lw["gate_qw"], lw["gate_sc"], lw["up_qw"], lw["up_sc"], lw["down_t_qw"],
                         lw["down_t_sc"], x, st.k)
        torch.cuda.synchronize()
        for u, v in zip(a, b):
            u = u.view(torch.int16) if u.dtype == torch.bfloat16 else u
            v = v.view(torch.int16) if v.dtype == torch.bfloat16 else v
            assert torch.equal(u, v), t
