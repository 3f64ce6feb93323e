"""The two-tier split of contiguous row-dot GEMVs (DIP_TUNE_ROW_TIERS, on by
default): at two workgroups per CU, the first workgroup on each CU takes
more rows per lane group than the second where a split was measured (the
SiLU gate at hidden 5120 with 12 < rows / (8 * CUs) <= 13: 9 rows and the
rest, the Qwen3-32B gate; at hidden 4096 with rows = 6 * 8 * CUs: 5 and 1,
the Qwen3-8B gate; the plain GEMV at 5120 columns with rows = 5 * 8 * CUs
and at 8192 columns with rows = 5 * 4 * CUs: 4 and 1, the Qwen3-32B q|k|v
and o projections).  Each row is still one group's dot product in the same
order, so the output must be bit for bit the even split's, at the row
counts on both sides of each rule; the even split is pinned to the oracle
by the kernel tests, and the split's outputs are checked against the oracle
here too."""
import numpy as np
import pytest
import torch

import dip_oracle as O
from gpu_util import dev, dev_bf16, host_bf16, random_bf16, random_int4, rel_err, ulp_diff

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def K():
    import _dip_hip
    return _dip_hip


def _groups_per_tier():
    return torch.cuda.get_device_properties(0).multi_processor_count * 8


@pytest.mark.parametrize("hidden,tier_units", [(5120, 12), (5120, 12.0001), (5120, 12.5),
                                               (5120, 13), (5120, 13.0001), (4096, 5.9995),
                                               (4096, 6), (4096, 6.0001)])
def test_gate_tiers_same_bits_as_even_split(K, hidden, tier_units):
    rows = int(np.ceil(tier_units * _groups_per_tier()))
    print(f"gate tiers rows={rows} hidden={hidden}", flush=True)
    rng = np.random.default_rng(rows)
    qw, sc = random_int4(rng, rows, hidden)
    x = random_bf16(rng, hidden)
    qd, sd, xd = dev(qw), dev_bf16(sc), dev_bf16(x)
    assert K.get_tuning("row_tiers") == 1
    split = K.int4_gemv(qd, sd, xd, act=1)
    try:
        K.set_tuning("row_tiers", 0)
        even = K.int4_gemv(qd, sd, xd, act=1)
    finally:
        K.set_tuning("row_tiers", 1)
    torch.cuda.synchronize()
    assert torch.equal(split, even)
    # against the oracle: SiLU of the pre-activation (within one bf16 ulp of
    # the correctly rounded SiLU), the pre-activation itself within the
    # reference's relative error
    pre = host_bf16(K.int4_gemv(qd, sd, xd))
    assert rel_err(pre, O.gemv_f64(qw, sc, x)) < 1e-2
    d = ulp_diff(host_bf16(split), O.silu_bf16(pre))
    assert d.max() <= 1 and (d > 0).mean() < 1e-3


@pytest.mark.parametrize("H,I", [(5120, 25600), (4096, 12288)])
def test_gate_tiers_in_the_decode_step(K, H, I):
    """The speculative decode step at the Qwen3-32B and Qwen3-8B shapes: y,
    g, idx and h with the split equal those with the even split, token after
    token."""
    keep = 0.6
    L = O.make_layer(H, I, seed=11)
    D = {n: (dev_bf16(v) if v.dtype == np.uint16 else dev(v)) for n, v in L.items()}
    gm = K.scales_group_major(D["down_t_sc"])
    k = O.keep_count(I, keep)
    st = [K.mlp_state(torch.device("cuda:0")) for _ in range(2)]
    for tok in range(3):
        print(f"gate tiers decode H={H} token {tok}", flush=True)
        x = dev_bf16(O.make_x(H, seed=40 + tok))
        outs = []
        for tiers in (1, 0):
            K.set_tuning("row_tiers", tiers)
            try:
                outs.append(K.mlp_decode(D["gate_qw"], D["gate_sc"], D["up_qw"], D["up_sc"],
                                         D["down_t_qw"], D["down_t_sc"], x, k, state=st[tiers],
                                         down_t_sc_gm=gm))
            finally:
                K.set_tuning("row_tiers", 1)
        torch.cuda.synchronize()
        for name, a, b in zip(("y", "g", "idx", "h"), *outs):
            assert torch.equal(a, b), (name, tok)
        assert np.array_equal(outs[0][2].cpu().numpy(), O.topk_select(host_bf16(outs[0][1]), k))


@pytest.mark.parametrize("H,I", [(5120, 25600), (4096, 12288)])
def test_gate_tiers_with_the_folded_rmsnorm(K, H, I):
    """The decode step with the post-attention RMSNorm folded into the gate
    (the whole-model decode's MLP): the split and the even split give the
    same y, g, idx, h, residual and x, token after token."""
    L = O.make_layer(H, I, seed=13)
    D = {n: (dev_bf16(v) if v.dtype == np.uint16 else dev(v)) for n, v in L.items()}
    W = [D[n] for n in ("gate_qw", "gate_sc", "up_qw", "up_sc", "down_t_qw", "down_t_sc")]
    gm = K.scales_group_major(D["down_t_sc"])
    k = O.keep_count(I, 0.6)
    gen = torch.Generator(device="cuda").manual_seed(H)
    w = (1 + 0.1 * torch.randn(H, device="cuda", generator=gen)).to(torch.bfloat16)
    st = [K.mlp_state(torch.device("cuda:0")) for _ in range(2)]
    for tok in range(3):
        print(f"gate tiers rmsnorm decode H={H} token {tok}", flush=True)
        res = (torch.randn(H, device="cuda", generator=gen) * 3).to(torch.bfloat16)
        add = torch.randn(H, device="cuda", generator=gen).to(torch.bfloat16)
        outs = []
        for tiers in (1, 0):
            K.set_tuning("row_tiers", tiers)
            try:
                res_out, x_out = torch.empty_like(res), torch.empty_like(res)
                o = K.mlp_decode_rmsnorm(*W, res, add, w, 1e-6, k, res_out=res_out, x_out=x_out,
                                         state=st[tiers], down_t_sc_gm=gm)
                outs.append([v.clone() for v in o[:4]] + [res_out, x_out])
            finally:
                K.set_tuning("row_tiers", 1)
        torch.cuda.synchronize()
        for name, a, b in zip(("y", "g", "idx", "h", "res", "x"), *outs):
            assert torch.equal(a, b), (name, tok)


@pytest.mark.parametrize("cols,units", [(5120, 5), (5120, 4.9995), (5120, 5.0005), (8192, 5),
                                        (8192, 4.999), (8192, 5.001)])
def test_plain_gemv_tiers_same_bits_as_even_split(K, cols, units):
    """The plain GEMV (the q|k|v and o projections' kernel), and with the
    folded RMSNorm where the width has it."""
    lanes = 64 if cols == 8192 else 32
    rows = int(np.ceil(units * _groups_per_tier() * 32 / lanes))
    print(f"plain gemv tiers rows={rows} cols={cols}", flush=True)
    rng = np.random.default_rng(rows + cols)
    qw, sc = random_int4(rng, rows, cols)
    x = random_bf16(rng, cols)
    qd, sd, xd = dev(qw), dev_bf16(sc), dev_bf16(x)
    gen = torch.Generator(device="cuda").manual_seed(cols)
    add = torch.randn(cols, device="cuda", generator=gen).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(cols, device="cuda", generator=gen)).to(torch.bfloat16)
    outs = []
    for tiers in (1, 0):
        K.set_tuning("row_tiers", tiers)
        try:
            o = [K.int4_gemv(qd, sd, xd)]
            if cols == 5120:
                o.append(K.int4_gemv_rmsnorm(qd, sd, xd, add, w, 1e-6))
            outs.append(o)
        finally:
            K.set_tuning("row_tiers", 1)
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    assert rel_err(host_bf16(outs[0][0]), O.gemv_f64(qw, sc, x)) < 1e-2


@pytest.mark.parametrize("hidden,tier_units", [(5120, 12), (5120, 12.0001), (5120, 12.5),
                                               (5120, 13), (4096, 6), (4096, 6.0001)])
def test_up_h_tiers_same_bits_as_even_split(K, hidden, tier_units):
    """The gathered up rows with h (dip_up_gather_h) take the gate's split at
    the gate's row counts (the keep >= 0.999 step gathers every channel):
    same bits as the even split, in a shuffled row order, and h = bf16(g[c] *
    u[c]) against the oracle."""
    k = int(np.ceil(tier_units * _groups_per_tier()))
    print(f"up+h tiers k={k} hidden={hidden}", flush=True)
    rng = np.random.default_rng(k + 1)
    qw, sc = random_int4(rng, k, hidden)
    x = random_bf16(rng, hidden)
    g = random_bf16(rng, k)
    idx = rng.permutation(k).astype(np.int32)
    qd, sd, xd, gd = dev(qw), dev_bf16(sc), dev_bf16(x), dev_bf16(g)
    idd = dev(idx)
    assert K.get_tuning("row_tiers") == 1
    split = K.up_gather_h(qd, sd, xd, idd, gd)
    try:
        K.set_tuning("row_tiers", 0)
        even = K.up_gather_h(qd, sd, xd, idd, gd)
    finally:
        K.set_tuning("row_tiers", 1)
    torch.cuda.synchronize()
    assert torch.equal(split, even)
    u = host_bf16(K.int4_gather_gemv(qd, sd, xd, idd))
    assert rel_err(u, O.gemv_f64(qw, sc, x)[idx]) < 1e-2
    assert np.array_equal(host_bf16(split), O.h_bf16(g[idx], u))
