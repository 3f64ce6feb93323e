"""GPU: the one-token decode kernels of a Qwen3 decoder layer
(dip_add_rmsnorm, dip_qk_norm_rope_cache, dip_decode_attention) against the
math of transformers' Qwen3 modules (Qwen3RMSNorm.forward,
apply_rotary_pos_emb, scaled-dot-product attention) restated with torch ops
on the same bf16 inputs.

Bars: the residual add and the value-cache copy are bit-exact; RMSNorm and
the rotary embedding round at the modules' points but sum the squares in a
different order, so outputs may differ by one bf16 ulp on a few elements;
attention is compared with an fp64 softmax at the reference's
max|err|/max|ref| < 1e-2 and 2 bf16 ulps per element (outputs near zero:
1e-5 of the largest)."""
import math

import numpy as np
import pytest
import torch

from gpu_util import ulp_diff

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def K():
    import _dip_hip
    return _dip_hip


def _bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)


def _hf_rmsnorm(x, w, eps):
    """Qwen3RMSNorm.forward on bf16 input (last dimension)."""
    xf = x.float()
    var = xf.pow(2).mean(-1, keepdim=True)
    return w * (xf * torch.rsqrt(var + eps)).to(torch.bfloat16)


def _rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def _tables(max_len, hd=128, theta=1e6):
    inv = 1.0 / (theta ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))
    f = torch.arange(max_len, dtype=torch.float32)[:, None] * inv[None, :]
    t = torch.cat((f, f), -1)
    return t.cos().to(torch.bfloat16).cuda(), t.sin().to(torch.bfloat16).cuda()


@pytest.mark.parametrize("n", [128, 1000, 2560, 4096, 5120, 8192])
def test_add_rmsnorm(K, n):
    print(f"add_rmsnorm n={n}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(n)
    h = (torch.randn(n, device="cuda", generator=g) * 3).to(torch.bfloat16)
    add = torch.randn(n, device="cuda", generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(n, device="cuda", generator=g)).to(torch.bfloat16)
    eps = 1e-6
    h2 = h + add
    ref = _hf_rmsnorm(h2, w, eps)
    hk = h.clone()
    out = torch.empty_like(h)
    K.add_rmsnorm(hk, add, w, out, eps)
    assert torch.equal(hk.view(torch.int16), h2.view(torch.int16))
    d = ulp_diff(_bits(out), _bits(ref))
    assert d.max() <= 1 and (d > 0).mean() < 0.01
    # without the add: h is left as it is
    h3 = h.clone()
    K.add_rmsnorm(h3, None, w, out, eps)
    assert torch.equal(h3.view(torch.int16), h.view(torch.int16))
    d = ulp_diff(_bits(out), _bits(_hf_rmsnorm(h, w, eps)))
    assert d.max() <= 1 and (d > 0).mean() < 0.01


@pytest.mark.parametrize("nh,nkv,pos", [(64, 8, 5), (4, 2, 0), (40, 8, 127), (16, 16, 31)])
def test_qk_norm_rope_cache(K, nh, nkv, pos):
    print(f"qk_norm_rope_cache nh={nh} nkv={nkv} pos={pos}", flush=True)
    hd, max_len, eps = 128, 128, 1e-6
    g = torch.Generator(device="cuda").manual_seed(nh * 7 + pos)
    qkv = (torch.randn((nh + 2 * nkv) * hd, device="cuda", generator=g) * 2).to(torch.bfloat16)
    qn = (1 + 0.1 * torch.randn(hd, device="cuda", generator=g)).to(torch.bfloat16)
    kn = (1 + 0.1 * torch.randn(hd, device="cuda", generator=g)).to(torch.bfloat16)
    cos, sin = _tables(max_len)
    kc = torch.full((nkv, max_len, hd), 0.5, dtype=torch.bfloat16, device="cuda")
    vc = torch.full((nkv, max_len, hd), -0.25, dtype=torch.bfloat16, device="cuda")
    kc0, vc0 = kc.clone(), vc.clone()
    q_out = torch.empty(nh * hd, dtype=torch.bfloat16, device="cuda")
    p = torch.tensor([pos], dtype=torch.long, device="cuda")
    K.qk_norm_rope_cache(qkv, qn, kn, cos, sin, p, q_out, kc, vc, nh, nkv, eps)

    q = _hf_rmsnorm(qkv[: nh * hd].view(nh, hd), qn, eps)
    k = _hf_rmsnorm(qkv[nh * hd:(nh + nkv) * hd].view(nkv, hd), kn, eps)
    v = qkv[(nh + nkv) * hd:].view(nkv, hd)
    c, s = cos[pos], sin[pos]
    q_ref = q * c + _rotate_half(q) * s
    k_ref = k * c + _rotate_half(k) * s
    d = ulp_diff(_bits(q_out), _bits(q_ref))
    assert d.max() <= 1 and (d > 0).mean() < 0.01
    d = ulp_diff(_bits(kc[:, pos]), _bits(k_ref))
    assert d.max() <= 1 and (d > 0).mean() < 0.01
    assert torch.equal(vc[:, pos].view(torch.int16), v.view(torch.int16))
    others = [i for i in range(max_len) if i != pos]
    assert torch.equal(kc[:, others], kc0[:, others])
    assert torch.equal(vc[:, others], vc0[:, others])
    # a position outside the cache writes no cache row
    K.qk_norm_rope_cache(qkv, qn, kn, cos, sin, torch.tensor([max_len], device="cuda"), q_out,
                         kc0, vc0, nh, nkv, eps)
    assert bool((kc0 == 0.5).all()) and bool((vc0 == -0.25).all())


def _attn_ref(q, kc, vc, pos, scale):
    nh, hd = q.shape
    nkv = kc.shape[0]
    G = nh // nkv
    qd = q.double().cpu().view(nkv, G, hd)
    kd = kc[:, : pos + 1].double().cpu()
    vd = vc[:, : pos + 1].double().cpu()
    s = torch.einsum("kgd,kpd->kgp", qd, kd) * scale
    p = torch.softmax(s, dim=-1)
    return torch.einsum("kgp,kpd->kgd", p, vd).reshape(nh, hd)


@pytest.mark.parametrize("nh,nkv", [(8, 8), (4, 2), (32, 8), (40, 8), (64, 8), (64, 4)])
def test_decode_attention(K, nh, nkv):
    hd, max_len = 128, 300
    g = torch.Generator(device="cuda").manual_seed(nh + nkv)
    q = torch.randn(nh, hd, device="cuda", generator=g).to(torch.bfloat16)
    kc = torch.randn(nkv, max_len, hd, device="cuda", generator=g).to(torch.bfloat16)
    vc = torch.randn(nkv, max_len, hd, device="cuda", generator=g).to(torch.bfloat16)
    scale = 1 / math.sqrt(hd)
    ws = torch.zeros(K.decode_attention_workspace_bytes(nh, hd, max_len), dtype=torch.uint8,
                     device="cuda")
    for pos in (0, 1, 31, 32, 33, 63, 64, 200, max_len - 1):
        print(f"decode_attention nh={nh} nkv={nkv} pos={pos}", flush=True)
        out = torch.empty(nh * hd, dtype=torch.bfloat16, device="cuda")
        K.decode_attention(q.view(-1), kc, vc, torch.tensor([pos], device="cuda"), out, scale, ws)
        ref = _attn_ref(q, kc, vc, pos, scale)
        got = out.view(nh, hd).double().cpu()
        assert float((got - ref).abs().max() / ref.abs().max()) < 1e-2
        # per element: within 2 bf16 ulps of the rounded fp64 value, or (for
        # outputs near zero, where fp32 cancellation dominates) within
        # 1e-5 of the largest output
        ulps = ulp_diff(_bits(out), _bits(ref.float().to(torch.bfloat16))).reshape(nh, hd)
        err = (got - ref).abs().numpy()
        assert not ((ulps > 2) & (err > 1e-5 * float(ref.abs().max()))).any()


@pytest.mark.parametrize("cap", [128, 1024])
@pytest.mark.parametrize("nh,nkv", [(4, 4), (4, 2), (24, 8), (32, 8), (40, 8), (64, 8), (64, 4)])
def test_decode_attention_fused_matches_split(K, nh, nkv, cap):
    """The one-launch norm + rotary + cache write + attention against the
    two-step path on the same inputs: the cache rows bit for bit (and no
    other row touched), the output within the attention bars of the fp64
    reference taken on the two-step path's q, and within 2 ulps of the split
    attention where that is built for the grouping."""
    # cap 128: the 4-wave launch; 1024 (the limit): 16 waves
    hd, max_len, eps = 128, min(cap, K.decode_attention_fused_max_len()), 1e-6
    scale = 1 / math.sqrt(hd)
    g = torch.Generator(device="cuda").manual_seed(7 * nh + nkv)
    qn = (1 + 0.1 * torch.randn(hd, device="cuda", generator=g)).to(torch.bfloat16)
    kn = (1 + 0.1 * torch.randn(hd, device="cuda", generator=g)).to(torch.bfloat16)
    cos, sin = _tables(max_len)
    base_k = torch.randn(nkv, max_len, hd, device="cuda", generator=g).to(torch.bfloat16)
    base_v = torch.randn(nkv, max_len, hd, device="cuda", generator=g).to(torch.bfloat16)
    for pos in sorted({0, 15, 16, 31, 32, 100, max_len // 2 + 3, max_len - 1}):
        print(f"decode_attention_fused nh={nh} nkv={nkv} max_len={max_len} pos={pos}", flush=True)
        qkv = (torch.randn((nh + 2 * nkv) * hd, device="cuda", generator=g) * 2).to(torch.bfloat16)
        p = torch.tensor([pos], device="cuda")
        kc1, vc1 = base_k.clone(), base_v.clone()
        q = torch.empty(nh * hd, dtype=torch.bfloat16, device="cuda")
        K.qk_norm_rope_cache(qkv, qn, kn, cos, sin, p, q, kc1, vc1, nh, nkv, eps)
        # the split path is built for groups of 1, 2, 4, 5, 8 and 16 query
        # heads; the fused one for any grouping
        split = None
        if nh // nkv in (1, 2, 4, 5, 8, 16):
            split = torch.empty(nh * hd, dtype=torch.bfloat16, device="cuda")
            K.decode_attention(q, kc1, vc1, p, split, scale)
        kc2, vc2 = base_k.clone(), base_v.clone()
        fused = torch.empty(nh * hd, dtype=torch.bfloat16, device="cuda")
        K.decode_attention_fused(qkv, qn, kn, cos, sin, p, kc2, vc2, fused, nh, nkv, eps, scale)
        assert torch.equal(kc1.view(torch.int16), kc2.view(torch.int16))
        assert torch.equal(vc1.view(torch.int16), vc2.view(torch.int16))
        ref = _attn_ref(q.view(nh, hd), kc1, vc1, pos, scale)
        got = fused.view(nh, hd).double().cpu()
        assert float((got - ref).abs().max() / ref.abs().max()) < 1e-2
        ulps = ulp_diff(_bits(fused), _bits(ref.float().to(torch.bfloat16))).reshape(nh, hd)
        err = (got - ref).abs().numpy()
        assert not ((ulps > 2) & (err > 1e-5 * float(ref.abs().max()))).any()
        if split is not None:
            assert ulp_diff(_bits(fused), _bits(split)).max() <= 2


@pytest.mark.parametrize("rows,cols", [(10240, 5120), (6144, 4096), (5120, 2560), (77, 5120)])
def test_int4_gemv_rmsnorm(K, rows, cols):
    """The GEMV with the input RMSNorm folded in: the residual it writes is
    bf16(h + add) bit for bit; its output is the GEMV of the normalised x,
    within the GEMV bars of the oracle on the x torch's Qwen3RMSNorm math
    gives (the sums of squares run in another order, so x may differ by a
    bf16 ulp in a few places)."""
    import dip_oracle as O
    from gpu_util import dev, dev_bf16, gemv_abs_terms, host_bf16, random_int4, rel_err
    print(f"int4_gemv_rmsnorm rows={rows} cols={cols}", flush=True)
    rng = np.random.default_rng(rows + cols)
    qw, sc = random_int4(rng, rows, cols)
    g = torch.Generator(device="cuda").manual_seed(rows)
    h = (torch.randn(cols, device="cuda", generator=g) * 3).to(torch.bfloat16)
    add = torch.randn(cols, device="cuda", generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(cols, device="cuda", generator=g)).to(torch.bfloat16)
    h_out = torch.full_like(h, 7.0)
    out = K.int4_gemv_rmsnorm(dev(qw), dev_bf16(sc), h, add, w, 1e-6, h_out=h_out)
    assert torch.equal(h_out.view(torch.int16), (h + add).view(torch.int16))
    x = _bits(_hf_rmsnorm(h + add, w, 1e-6))
    ref = O.gemv_f64(qw, sc, x)
    got = host_bf16(out)
    assert rel_err(got, ref) < 1e-2
    assert float(np.max(np.abs(O.bf16_to_f32(got) - ref)) / np.max(np.abs(ref))) < 1e-2
    # no residual addend and no residual written
    out2 = K.int4_gemv_rmsnorm(dev(qw), dev_bf16(sc), h, None, w, 1e-6)
    ref2 = O.gemv_f64(qw, sc, _bits(_hf_rmsnorm(h, w, 1e-6)))
    assert rel_err(host_bf16(out2), ref2) < 1e-2
    with pytest.raises(RuntimeError):   # the residual written over its own input
        K.int4_gemv_rmsnorm(dev(qw), dev_bf16(sc), h, add, w, 1e-6, h_out=h)


@pytest.mark.parametrize("cols", [5120, 4096, 2560])
def test_int4_gemv_rmsnorm_special_values(K, cols):
    """The folded RMSNorm's roundings (one v_cvt_pk_bf16_f32 per pair) on
    special values: the residual bf16(h + add) it writes equals torch's bit
    for bit with signed zeros, cancellation, subnormals and the largest
    finite values, where the output stays within the GEMV bars; and with
    +-inf and NaN inputs (NaN becomes 0x7FC0), where every output is NaN."""
    import dip_oracle as O
    from gpu_util import dev, dev_bf16, host_bf16, random_int4, rel_err
    print(f"int4_gemv_rmsnorm special values cols={cols}", flush=True)
    rng = np.random.default_rng(cols + 1)
    rows = 64
    qw, sc = random_int4(rng, rows, cols)
    g = torch.Generator(device="cuda").manual_seed(cols + 1)
    h = (torch.randn(cols, device="cuda", generator=g) * 3).to(torch.bfloat16)
    add = torch.randn(cols, device="cuda", generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(cols, device="cuda", generator=g)).to(torch.bfloat16)
    # (h, add) bit pairs: +-0, subnormal sums, the smallest normal, a large
    # value (its square still finite), cancellation to +0, 1 + tiny (ties and
    # rounding)
    pairs = [(0x0000, 0x8000), (0x8000, 0x8000), (0x0001, 0x0001), (0x807F, 0x0001),
             (0x0080, 0x8001), (0x5F00, 0x0000), (0x4040, 0xC040), (0x3F80, 0x3381),
             (0xBF81, 0x3381), (0x3F80, 0x3B80)]
    hb, ab = h.view(torch.int16), add.view(torch.int16)
    for i, (x, y) in enumerate(pairs):
        hb[37 * i + 5] = x - 65536 if x > 32767 else x
        ab[37 * i + 5] = y - 65536 if y > 32767 else y
    h_out = torch.full_like(h, 7.0)
    out = K.int4_gemv_rmsnorm(dev(qw), dev_bf16(sc), h, add, w, 1e-6, h_out=h_out)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(h_out), _bits(h + add))
    ref = O.gemv_f64(qw, sc, _bits(_hf_rmsnorm(h + add, w, 1e-6)))
    assert rel_err(host_bf16(out), ref) < 1e-2
    # non-finite residuals: +-inf, inf - inf, and a NaN with a payload
    for i, (x, y) in enumerate([(0x7F80, 0x3F80), (0xFF80, 0x0000), (0x7F80, 0xFF80),
                                (0x7FC1, 0x3F80), (0xFFC0, 0x0000)]):
        hb[41 * i + 3] = x - 65536 if x > 32767 else x
        ab[41 * i + 3] = y - 65536 if y > 32767 else y
    out = K.int4_gemv_rmsnorm(dev(qw), dev_bf16(sc), h, add, w, 1e-6, h_out=h_out)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(h_out), _bits(h + add))
    assert 0x7FC0 in set(_bits(h_out).tolist())
    assert torch.isnan(out.float()).all()


def test_decode_attention_rejects_bad_arguments(K):
    q = torch.zeros(3 * 128, dtype=torch.bfloat16, device="cuda")
    kc = torch.zeros(2, 16, 128, dtype=torch.bfloat16, device="cuda")
    out = torch.empty_like(q)
    with pytest.raises(RuntimeError):   # 3 query heads over 2 kv heads
        K.decode_attention(q, kc, kc, torch.zeros(1, dtype=torch.long, device="cuda"), out, 1.0)
    with pytest.raises(RuntimeError):   # pos on the host
        K.decode_attention(q[:256], kc, kc, torch.zeros(1, dtype=torch.long), out[:256], 1.0)
