"""The group-major copy of down_t's scales (dip_scales_group_major) and the
down stage reading it: the copy is the exact transpose of the scale matrix,
and every entry point that takes it gives the same bits as without it (the
same scale values reach the same arithmetic; only their addresses differ)."""
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
    return t.view(torch.int16) if t.dtype == torch.bfloat16 else t


@pytest.mark.parametrize("rows,groups", [(25600, 40), (12288, 32), (1000, 24), (130, 70), (1, 1)])
def test_scales_group_major_is_the_transpose(K, rows, groups):
    rng = np.random.default_rng(rows + groups)
    sc = random_bf16(rng, rows * groups).reshape(rows, groups)
    gm = K.scales_group_major(dev_bf16(sc))
    assert tuple(gm.shape) == (groups, rows)
    assert np.array_equal(host_bf16(gm), np.ascontiguousarray(sc.T))


@pytest.mark.parametrize("rows,k,out_f", [(25600, 15360, 5120), (12288, 7373, 4096),
                                          (3000, 1000, 384), (500, 500, 1024),
                                          (300, 1, 1024), (300, 7, 2048), (300, 257, 1024),
                                          (4000, 2049, 5120)])
def test_down_by_channel_same_bits_with_group_major_scales(K, rows, k, out_f):
    """out_f 384 runs the 4-lane tiles, the others the 8-lane ones (with the
    group-major copy: the decode step's kernel); k = rows selects every row;
    k of 1, 7, 257 and 2049 leave tiles and slots partly empty."""
    rng = np.random.default_rng(k)
    qw, sc = random_int4(rng, rows, out_f)
    idx = np.sort(rng.permutation(rows)[:k]).astype(np.int32)
    h_full = random_bf16(rng, rows)
    d_qw, d_sc, d_h, d_idx = dev(qw), dev_bf16(sc), dev_bf16(h_full), dev(idx)
    gm = K.scales_group_major(d_sc)
    outs = []
    for g in (None, gm):
        h_out = torch.empty(k, dtype=torch.bfloat16, device="cuda")
        y = K.int4_gather_down_by_channel(d_qw, d_sc, d_h, d_idx, h_out=h_out, scales_gm=g)
        outs.append((y.clone(), h_out))
    assert torch.equal(_bits(outs[0][0]), _bits(outs[1][0]))
    assert torch.equal(_bits(outs[0][1]), _bits(outs[1][1]))
    ref = O.down_f64(qw, sc, h_full[idx], rows=idx)
    err = np.abs(O.bf16_to_f32(host_bf16(outs[1][0])) - ref).max() / np.abs(ref).max()
    assert err < 1e-2


def test_down_by_channel_bad_ids_same_bits_with_group_major_scales(K):
    """Out-of-range channel ids poison y (NaN) and read row 0 for h_out, the
    same bits through the decode step's kernel as through the general one."""
    rng = np.random.default_rng(11)
    rows, k, out_f = 600, 300, 1024
    qw, sc = random_int4(rng, rows, out_f)
    idx = np.sort(rng.permutation(rows)[:k]).astype(np.int32)
    idx[[5, 100]] = [rows, -3]
    h_full = random_bf16(rng, rows)
    d_qw, d_sc, d_h, d_idx = dev(qw), dev_bf16(sc), dev_bf16(h_full), dev(idx)
    gm = K.scales_group_major(d_sc)
    outs = []
    for g in (None, gm):
        h_out = torch.empty(k, dtype=torch.bfloat16, device="cuda")
        y = K.int4_gather_down_by_channel(d_qw, d_sc, d_h, d_idx, h_out=h_out, scales_gm=g)
        outs.append((y.clone(), h_out))
    assert torch.equal(_bits(outs[0][0]), _bits(outs[1][0]))
    assert torch.equal(_bits(outs[0][1]), _bits(outs[1][1]))
    assert torch.isnan(outs[1][0].float()).all()
    assert _bits(outs[1][1])[5].item() == _bits(dev_bf16(h_full[:1]))[0].item()


def test_group_major_scales_rejected_with_wrong_shape(K):
    rng = np.random.default_rng(3)
    qw, sc = random_int4(rng, 256, 512)
    d_sc = dev_bf16(sc)
    with pytest.raises(RuntimeError, match="scales_gm"):
        K.int4_gather_down_by_channel(dev(qw), d_sc, dev_bf16(random_bf16(rng, 256)),
                                      dev(np.arange(10, dtype=np.int32)), scales_gm=d_sc)


@pytest.mark.parametrize("H,I,keep", [(5120, 25600, 0.6), (4096, 12288, 0.3)])
@pytest.mark.parametrize("spec", [False, True], ids=["stagewise", "four-launch"])
def test_mlp_decode_same_bits_with_group_major_scales(K, H, I, keep, spec):
    L = O.make_layer(H, I, seed=11)
    D = {n: (dev_bf16(v) if v.dtype == np.uint16 else dev(v)) for n, v in L.items()}
    gm = K.scales_group_major(D["down_t_sc"])
    k = O.keep_count(I, keep)
    W = (D["gate_qw"], D["gate_sc"], D["up_qw"], D["up_sc"], D["down_t_qw"], D["down_t_sc"])
    states = [K.mlp_state(torch.device("cuda:0")) if spec else None for _ in range(2)]
    for tok in range(3):  # the speculation state evolves the same way on both
        x = dev_bf16(O.make_x(H, seed=40 + tok))
        a = [t.clone() for t in K.mlp_decode(*W, x, k, state=states[0])]
        b = [t.clone() for t in K.mlp_decode(*W, x, k, state=states[1], down_t_sc_gm=gm)]
        for name, u, v in zip(("y", "g", "idx", "h"), a, b):
            assert torch.equal(_bits(u), _bits(v)), (name, tok)
        assert np.array_equal(b[2].cpu().numpy(), O.topk_select(host_bf16(b[1]), k))


@pytest.mark.parametrize("rows,out_f", [(25600, 5120), (12288, 4096), (3000, 1152), (777, 1024)])
@pytest.mark.parametrize("use_gm", [True, False], ids=["gm", "row-major"])
def test_down_by_channel_without_indices_is_every_row(K, rows, out_f, use_gm):
    """indices=None (the dense route's every-row down: position j is row j,
    no id list) gives the bits of indices = 0..rows-1, with and without the
    group-major scales, on the shapes of each down kernel (hidden 5120: the
    reduce launch; 4096: the in-launch reduce on a full gfx950; 1152: four
    lanes per row segment; 1024: one row block short), and y within 1e-2 of
    the oracle's fp64 sum."""
    print(f"down without indices rows={rows} out={out_f} gm={use_gm}", flush=True)
    rng = np.random.default_rng(rows + out_f + use_gm)
    qw, sc = random_int4(rng, rows, out_f)
    h = random_bf16(rng, rows)
    qd, sd, hd = dev(qw), dev_bf16(sc), dev_bf16(h)
    gm = K.scales_group_major(sd) if use_gm else None
    every = K.int4_gather_down_by_channel(qd, sd, hd, None, scales_gm=gm)
    ar = torch.arange(rows, dtype=torch.int32, device="cuda")
    ref = K.int4_gather_down_by_channel(qd, sd, hd, ar, scales_gm=gm)
    torch.cuda.synchronize()
    assert torch.equal(_bits(every), _bits(ref))
    y64 = O.down_f64(qw, sc, h)
    err = np.abs(O.bf16_to_f32(host_bf16(every)) - y64).max() / np.abs(y64).max()
    assert err < 1e-2
