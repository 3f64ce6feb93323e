"""GPU parity of the decode step with speculative up rows.

dip_mlp_decode with a layer state runs four launches: the gate, one launch
holding the top-k select and the up rows (with h) of the channels the
state's speculation key picks, the down partials and the down reduce.
Whatever the state holds, g, idx and h must be bit-identical to the
stage-by-stage step (no state), which the other GPU tests pin against the
oracle.  y is the same sum of the same exact products, read by channel
instead of by position; it must agree to within a few fp32 roundings: one
bf16 ulp, except where the sum cancels to near zero; a missing or doubled
channel moves y by about 1/sqrt(k) of its size.  For a given state the step
is deterministic.  The state itself must then hold the magnitude key of rank
k + margin of the call's g.
"""
import numpy as np
import pytest
import torch

import dip_oracle as O
from gpu_util import host_bf16, rel_err, ulp_diff

pytestmark = pytest.mark.gpu

MARGIN_PER_1024 = 8  # DIP_TUNE_SPEC_MARGIN default


@pytest.fixture(scope="module")
def K():
    import _dip_hip
    return _dip_hip


def _weights(H, I, seed):
    from quantize import quantize_tensor_int4_groupwise
    gen = torch.Generator(device="cuda").manual_seed(seed)
    out = []
    for _ in range(3):
        q, s = quantize_tensor_int4_groupwise(
            torch.randn(I, H, device="cuda", generator=gen) * 0.02)
        out += [q, s]
    return out  # gate_qw, gate_sc, up_qw, up_sc, down_t_qw, down_t_sc


def _x(H, seed):
    gen = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn(H, device="cuda", generator=gen).to(torch.bfloat16)


def _bits(t):
    return t.view(torch.int16) if t.dtype == torch.bfloat16 else t


def _step(K, W, x, k, state=None):
    return [t.clone() for t in K.mlp_decode(*W, x, k, state=state)]


def _assert_same(a, b, what):
    for name, u, v in zip(("y", "g", "idx", "h"), a, b):
        assert torch.equal(_bits(u), _bits(v)), f"{what}: {name} differs"


def _assert_y_close(u, v, what):
    """Two fp32 sums of the same exact products in different groupings, each
    rounded to bf16: every output within one bf16 ulp, except where the sum
    cancels to near zero (|y| below 1e-3 of max|y|), where the two may differ
    by fp32 rounding of the large terms (at most 1e-4 of max|y|).  A missing
    or doubled channel moves y by about 1/sqrt(k) of max|y| (> 1e-2)."""
    yu, yv = host_bf16(u), host_bf16(v)
    a = O.bf16_to_f32(yu).astype(np.float64)
    b = O.bf16_to_f32(yv).astype(np.float64)
    top = max(np.abs(b).max(), 1e-30)
    small = np.abs(b) < 1e-3 * top
    d = ulp_diff(yu, yv)
    assert (d[~small] <= 1).all(), f"{what}: y differs by {d[~small].max()} ulps"
    assert (np.abs(a - b)[small] <= 1e-4 * top).all(), f"{what}: near-zero y"
    assert np.abs(a - b).max() <= 4e-3 * top, f"{what}: y rel err"


def _assert_step(a, b, what):
    """g, idx, h bit-identical; y close (another fp32 summation order)."""
    for name, u, v in zip(("g", "idx", "h"), a[1:], b[1:]):
        assert torch.equal(_bits(u), _bits(v)), f"{what}: {name} differs"
    _assert_y_close(a[0], b[0], what)


def _state(key):
    """A decode state holding the speculation key in use and the next one."""
    return torch.tensor([key, key, 0, 0], dtype=torch.int32, device="cuda")


def _assert_next_state(K, state, g, k, margin, what, first=False):
    """The state a call leaves: its rank k + margin key as the next key, the
    key it used in [0] (0 after the first call)."""
    st = state.cpu().numpy().view(np.uint32)
    assert st[1] == _rank_key(g, k + margin), what
    if first:
        assert st[0] == 0, what  # a zeroed state speculates on every channel


def _rank_key(g, r):
    """Magnitude key (|bf16 bits|) of rank r (1 = largest) among the values
    that are not NaN; 0 when there are fewer than r."""
    keys = host_bf16(g).astype(np.int64) & 0x7FFF
    keys = np.sort(keys[keys <= 0x7F80])[::-1]
    return int(keys[r - 1]) if r <= len(keys) else 0


@pytest.mark.parametrize("H,I,keep", [(5120, 25600, 0.6), (4096, 12288, 0.3), (2560, 9728, 0.6)])
def test_spec_matches_stagewise(K, H, I, keep):
    W = _weights(H, I, seed=H)
    k = O.keep_count(I, keep)
    state = K.mlp_state("cuda")
    margin = I * MARGIN_PER_1024 // 1024
    for t in range(4):
        x = _x(H, 100 + t)
        st0 = state.clone()
        got = _step(K, W, x, k, state)
        ref = _step(K, W, x, k)
        _assert_step(got, ref, f"H={H} token {t}")
        _assert_same(_step(K, W, x, k, st0), got, f"H={H} token {t}: same state, same bits")
        _assert_next_state(K, state, ref[1], k, margin, t, first=t == 0)


def test_spec_any_state_value(K):
    """Forced speculation keys: all channels, none (every selected channel is
    a residual row of the select workgroups), the exact cut, half of the
    selection, a wide margin, +inf."""
    H, I = 4096, 12288
    W = _weights(H, I, seed=7)
    k = O.keep_count(I, 0.6)
    x = _x(H, 5)
    ref = _step(K, W, x, k)
    g = ref[1]
    keys = [0, 0xFFFF, _rank_key(g, k), _rank_key(g, k // 2), _rank_key(g, k + 2000), 0x7F80,
            0x7FFF, 1]
    for key in keys:
        got = _step(K, W, x, k, _state(key))
        _assert_step(got, ref, f"key {key:#x}")


def test_spec_unfilled_slots_use_channel_0(K):
    """Fewer than k channels are nonzero: the unfilled slots point at channel
    0, whose h must be computed even when it is neither selected nor
    speculated on (including h = bf16(0 * u), which keeps u's sign)."""
    H, I = 2560, 9728
    W = _weights(H, I, seed=9)
    gs = W[1].clone()
    gs[200:] = 0            # g = silu(0) = 0 for all but 200 channels
    gs[0] = 0               # channel 0 among the zeros
    W0 = [W[0], gs] + W[2:]
    k = O.keep_count(I, 0.3)
    x = _x(H, 6)
    ref = _step(K, W0, x, k)
    assert (ref[2][200:] == 0).all()  # unfilled slots hold channel 0
    for key in (0, 1, 0xFFFF, _rank_key(ref[1], 100)):
        _assert_step(_step(K, W0, x, k, _state(key)), ref, f"key {key:#x}")
    gs[0] = W[1][0]         # channel 0 nonzero again
    ref = _step(K, W0, x, k)
    for key in (0, 0xFFFF):
        _assert_step(_step(K, W0, x, k, _state(key)), ref, f"key {key:#x}, channel 0 live")


def test_spec_margin_knob(K):
    H, I = 2560, 9728
    W = _weights(H, I, seed=11)
    k = O.keep_count(I, 0.6)
    try:
        for m in (0, 1024):
            K.set_tuning("spec_margin", m)
            state = K.mlp_state("cuda")
            for t in range(3):
                x = _x(H, 30 + t)
                ref = _step(K, W, x, k)
                _assert_step(_step(K, W, x, k, state), ref, f"margin {m} token {t}")
                _assert_next_state(K, state, ref[1], k, I * m // 1024, f"margin {m}")
    finally:
        K.set_tuning("spec_margin", MARGIN_PER_1024)


def test_spec_unsupported_width_runs_stagewise(K):
    """A width without a speculative instantiation runs the stage-by-stage
    step and leaves the state alone."""
    H, I = 1024, 3072
    W = _weights(H, I, seed=13)
    k = O.keep_count(I, 0.6)
    x = _x(H, 8)
    state = K.mlp_state("cuda")
    _assert_same(_step(K, W, x, k, state), _step(K, W, x, k), "H=1024")
    assert (state == 0).all()


def test_spec_stack_graph_replays(K):
    """A 3-layer stack with speculation captured as one HIP graph: every
    replay (new x each time, eager work and synchronisation in between)
    equals the stage-by-stage eager run of the same weights."""
    from dip_stack import DIPStack
    H, I = 2560, 9728
    spec = DIPStack(H, I, 3, 0.6, "cuda", seed=21, spec=True)
    plain = DIPStack(H, I, 3, 0.6, "cuda", seed=21, spec=False)
    for name in ("gate_qw", "up_qw", "down_t_qw"):
        assert torch.equal(spec.w[2][name], plain.w[2][name])
    spec.capture()
    for rep in range(4):
        x = _x(H, 50 + rep)
        for y in spec.y:
            y.zero_()
        torch.randn(1000, device="cuda").sum().item()    # unrelated eager work
        spec.step(x)
        plain.x.copy_(x)
        plain.run_token()
        torch.cuda.synchronize()
        for a, b in zip(spec.y, plain.y):
            _assert_y_close(a, b, f"replay {rep}")


def test_mlp_decode_rmsnorm_equals_mlp_decode_on_its_x(K):
    """The decode step with the post-attention RMSNorm folded into the gate:
    the residual it writes is bf16(res + add), its x is within one bf16 ulp
    of the separate RMSNorm kernel's, and y, g, idx and h equal
    mlp_decode's on that x, bit for bit, over several tokens (speculative
    and stage-by-stage)."""
    from quantize import quantize_tensor_int4_groupwise
    for H, I in [(5120, 25600), (2560, 9728)]:
        print(f"mlp_decode_rmsnorm H={H} I={I}", flush=True)
        gen = torch.Generator(device="cuda").manual_seed(H)
        W = []
        for _ in range(3):
            W += list(quantize_tensor_int4_groupwise(
                torch.randn(I, H, device="cuda", generator=gen) * 0.02))
        k = O.keep_count(I, 0.6)
        w = (1 + 0.1 * torch.randn(H, device="cuda", generator=gen)).to(torch.bfloat16)
        for state in (K.mlp_state("cuda"), None):
            for t in range(3):
                res = (torch.randn(H, device="cuda", generator=gen) * 3).to(torch.bfloat16)
                add = torch.randn(H, device="cuda", generator=gen).to(torch.bfloat16)
                res_out = torch.empty_like(res)
                x_out = torch.empty_like(res)
                a = [v.clone() for v in K.mlp_decode_rmsnorm(*W, res, add, w, 1e-6, k,
                                                             res_out=res_out, x_out=x_out,
                                                             state=state)]
                assert torch.equal(res_out.view(torch.int16), (res + add).view(torch.int16))
                x_sep = torch.empty_like(res)
                K.add_rmsnorm((res + add).clone(), None, w, x_sep, 1e-6)
                d = ulp_diff(x_out.view(torch.int16).cpu().numpy().view(np.uint16),
                             x_sep.view(torch.int16).cpu().numpy().view(np.uint16))
                assert d.max() <= 1
                b = [v.clone() for v in K.mlp_decode(*W, x_out, k)]
                if state is None:
                    _assert_same(a[:4], b, f"H={H} token {t}")
                else:
                    _assert_step(a[:4], b, f"H={H} token {t} (state)")


def test_stack_qwen3_32b_shape_two_layers(K):
    """A 2-layer DIPStack at the Qwen3-32B layer shape (H=5120, I=25600,
    keep 0.6) with per-layer speculation state and the shared workspace,
    replayed as one HIP graph: over 3 tokens every layer's y is within 1e-2
    of the oracle's decode forward on that layer's weights, and the shared
    idx (the last layer's) is the top-k of the shared g."""
    from dip_stack import DIPStack
    H, I = 5120, 25600
    stack = DIPStack(H, I, 2, 0.6, "cuda", seed=31, spec=True)
    host = [tuple(lw[n].cpu().numpy() if n.endswith("_qw") else host_bf16(lw[n])
                  for n in ("gate_qw", "gate_sc", "up_qw", "up_sc", "down_t_qw", "down_t_sc"))
            for lw in stack.w]
    stack.capture()
    for t in range(3):
        x = O.make_x(H, seed=40 + t)
        stack.step(torch.from_numpy(x.view(np.int16)).to("cuda").view(torch.bfloat16))
        torch.cuda.synchronize()
        g_h = host_bf16(stack.g)
        assert np.array_equal(stack.idx.cpu().numpy(), O.topk_select(g_h, stack.k)), t
        for i, w in enumerate(host):
            ref = O.dip_forward(*w, x, stack.k)
            err = rel_err(host_bf16(stack.y[i]), ref["y_f64"])
            print(f"token {t} layer {i}: rel err {err:.2e}", flush=True)
            assert err < 1e-2, (t, i)


def test_stack_dense_route_at_keep_one(K):
    """keep >= 0.999 routes every layer to the dense computation, as the
    reference does (dip_stream_predispatch.py:177-179 -> _dense): no top-k,
    idx = 0..I-1, g and h = bf16(g * u) within the step's ulp bounds of the
    oracle's dense forward, y within 1e-2 of it (and of the reference's literal
    bf16-weight dense route) on every layer, replayed as one HIP graph; the
    stage timing names the three dense launches."""
    from dip_stack import DIPStack
    H, I = 2560, 9728
    stack = DIPStack(H, I, 2, 1.0, "cuda", seed=17, spec=True)
    assert stack.dense and stack.k == I
    host = [tuple(lw[n].cpu().numpy() if n.endswith("_qw") else host_bf16(lw[n])
                  for n in ("gate_qw", "gate_sc", "up_qw", "up_sc", "down_t_qw", "down_t_sc"))
            for lw in stack.w]
    stack.capture()
    for t in range(3):
        x = O.make_x(H, seed=60 + t)
        stack.step(torch.from_numpy(x.view(np.int16)).to("cuda").view(torch.bfloat16))
        torch.cuda.synchronize()
        assert np.array_equal(stack.idx.cpu().numpy(), np.arange(I, dtype=np.int32))
        for i, w in enumerate(host):
            ref = O.dense_forward(*w, x)
            if i == len(host) - 1:  # g and h are shared: the last layer's
                # g = silu(bf16(gate . x)): fp32 summation order may move it
                # by up to 2 ulps; h = bf16(g * u) on the device's g
                g_h = host_bf16(stack.g)
                d = ulp_diff(g_h, ref["g"])
                assert d.max() <= 2 and (d > 0).mean() < 5e-3, t
                hd = ulp_diff(host_bf16(stack.h), O.h_bf16(g_h, ref["u"]))
                assert (hd > 0).mean() < 0.02, t
            err = rel_err(host_bf16(stack.y[i]), ref["y_f64"])
            lit = rel_err(host_bf16(stack.y[i]), O.dense_literal_forward(*w, x)["y_f64"])
            print(f"dense token {t} layer {i}: rel err {err:.2e} (literal {lit:.2e})", flush=True)
            assert err < 1e-2 and lit < 2e-2, (t, i)
    st = stack.stage_times_ms(reps=1, samples=1)
    assert list(st) == ["gate_silu", "up_gather_h", "down_gather"]
