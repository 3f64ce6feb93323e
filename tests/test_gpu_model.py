"""GPU: whole-model integration.  A small random-weight Qwen3 is written in
the reference's int4 checkpoint layout and loaded with load_streaming_dip /
load_dip_ca; DIPDecoder's HIP-graph decode is checked bit for bit against
its own eager steps and against transformers' incremental forward on the same
modules, against the same checkpoint on the CPU with the oracle's GEMV and
DIP MLP, and (keep 1.0) against the modules' dense route.

Tolerances are on max|err|/max|ref| of the logits (the reference's metric):
the paths share the int4 kernels but differ in attention kernels and bf16
rounding points, and a top-k boundary channel may flip between them."""
import numpy as np
import pytest
import torch

import dip_oracle as O
from gpu_util import assert_fp32_close, dev, dev_bf16, gemv_abs_terms, host_bf16, random_bf16, \
    random_int4, rel_err
from model_util import assert_confident_argmax, max_rel, oracle_model, teacher_forced_logits, \
    tiny_config, tiny_model, write_checkpoint

pytestmark = pytest.mark.gpu

# "spec": hidden 2560 runs the speculative up path; "stagewise": hidden 512
# runs the five-launch path.
CONFIGS = {"spec": dict(hidden=2560, inter=3072, heads=4, kv_heads=2, head_dim=128, vocab=1024),
           "stagewise": dict(hidden=512, inter=1024, heads=4, kv_heads=1, head_dim=128, vocab=512)}
KEEP = 0.6
PLEN, NEW = 6, 10


@pytest.fixture(scope="module", params=list(CONFIGS))
def ckpt(request, tmp_path_factory):
    cfg = tiny_config(**CONFIGS[request.param])
    d = tmp_path_factory.mktemp(request.param)
    write_checkpoint(tiny_model(cfg, seed=len(request.param)), d)
    return request.param, d, cfg


@pytest.fixture(scope="module")
def streaming(ckpt):
    from dip_stream_predispatch import load_streaming_dip
    name, d, cfg = ckpt
    print(f"load_streaming_dip {name}", flush=True)
    model, tok, sdips = load_streaming_dip(d, keep_ratio=KEEP)
    prompt = torch.randint(0, cfg.vocab_size, (1, PLEN), generator=torch.Generator().manual_seed(9))
    return model, sdips, prompt


def test_loader_swaps_every_mlp(ckpt, streaming):
    from dip_stream_predispatch import StreamingDIPMlp
    from qlinear import QuantLinear
    name, d, cfg = ckpt
    model, sdips, _ = streaming
    assert len(sdips) == cfg.num_hidden_layers
    for layer, s in zip(model.model.layers, sdips):
        assert layer.mlp is s and isinstance(s, StreamingDIPMlp)
        assert s.k == O.keep_count(cfg.intermediate_size, KEEP)
        for p in ("q_proj", "k_proj", "v_proj", "o_proj"):
            q = getattr(layer.self_attn, p)
            assert isinstance(q, QuantLinear) and q.qweight.is_cuda
    assert all(t.is_cuda for t in model.parameters())


def test_graph_decode_equals_eager(ckpt, streaming):
    from dip_model import DIPDecoder
    model, _, prompt = streaming
    print(f"graph vs eager decode {ckpt[0]}", flush=True)
    seq_g, log_g = DIPDecoder(model, 32, use_graph=True).generate(prompt, NEW, return_logits=True)
    seq_e, log_e = DIPDecoder(model, 32, use_graph=False).generate(prompt, NEW, return_logits=True)
    assert torch.equal(seq_g, seq_e)
    assert torch.equal(log_g, log_e)


def test_graph_decode_real_shapes_equals_eager():
    """Two layers of the Qwen3-32B shape with its full 151936-token
    vocabulary (synthetic weights): every graph replay's logits equal the
    eager step's bit for bit, with the eager lm_head and argmax between
    replays."""
    from dip_model import DIPDecoder, qwen3_config, synthetic_model
    print("graph vs eager decode, qwen3-32b shape, 2 layers", flush=True)
    cfg = qwen3_config("qwen3-32b", num_hidden_layers=2)
    model, _ = synthetic_model(cfg, 0.6, "cuda:0", seed=3)
    prompt = torch.randint(0, cfg.vocab_size, (1, 8), generator=torch.Generator().manual_seed(1))
    seq_g, log_g = DIPDecoder(model, 40, use_graph=True).generate(prompt, 16, return_logits=True)
    seq_e, log_e = DIPDecoder(model, 40, use_graph=False).generate(prompt, 16, return_logits=True)
    assert torch.equal(seq_g, seq_e)
    assert torch.equal(log_g, log_e)


@pytest.mark.parametrize("keep,bound", [(KEEP, 8e-2), (1.0, 2e-2)])
def test_fused_decode_matches_module_path(ckpt, streaming, keep, bound):
    """The fused decode kernels against the same step through the HF
    modules' PyTorch ops (same int4 GEMVs and DIP MLPs), teacher-forced on
    the fused path's tokens.  The two differ by bf16 rounding (sum order
    in RMSNorm, fp32 attention); at keep 0.6 such a difference in an MLP
    input can swap a channel at the top-k boundary, and in a random-weight
    model each swap moves y by about 1/sqrt(k) of its size, hence the wider
    bound there."""
    from dip_model import DIPDecoder
    from dip_stream_predispatch import load_streaming_dip
    name, d, cfg = ckpt
    model, _, prompt = streaming
    if keep != KEEP:
        model, _, _ = load_streaming_dip(d, keep_ratio=keep)
    print(f"fused vs module decode {name} keep {keep}", flush=True)
    dec = DIPDecoder(model, 32)
    assert dec.fused
    seq, got = dec.generate(prompt, NEW, return_logits=True)
    ref = teacher_forced_logits(DIPDecoder(model, 32, use_graph=False, fused=False), seq, PLEN)
    err = max_rel(got, ref)
    print(f"  max_rel {err:.3e}", flush=True)
    assert err < bound
    assert_confident_argmax(got, ref, bound)


@pytest.mark.parametrize("long_kind", ["split", "one-launch-16-waves"])
def test_long_cache_decode_matches_short(ckpt, streaming, long_kind):
    """A longer cache against a 32-row one (the 4-wave one-launch
    attention), teacher-forced on the same tokens: beyond the one-launch
    limit (the split path: norm + rotary + cache write, per-chunk partials,
    merge), and at 300 rows (the 16-wave one-launch attention)."""
    from dip_model import DIPDecoder
    import _dip_hip as K
    model, _, prompt = streaming
    print(f"long ({long_kind}) vs short cache decode {ckpt[0]}", flush=True)
    short = DIPDecoder(model, 32)
    split = long_kind == "split"
    long_ = DIPDecoder(model, K.decode_attention_fused_max_len() + 88 if split else 300)
    assert short._attn_one_launch and long_._attn_one_launch != split
    seq, got = long_.generate(prompt, NEW, return_logits=True)
    ref = teacher_forced_logits(short, seq, PLEN)
    err = max_rel(got, ref)
    print(f"  max_rel {err:.3e}", flush=True)
    assert err < 8e-2
    assert_confident_argmax(got, ref, 8e-2)


def test_module_decode_equals_hf_incremental_forward(ckpt, streaming):
    """DIPDecoder's module path (fused=False) is transformers' own
    incremental forward, one token at a time with its DynamicCache, through
    the same StreamingDIPMlp and QuantLinear modules: bit for bit."""
    from transformers import DynamicCache
    from dip_model import DIPDecoder
    model, _, prompt = streaming
    print(f"module decode vs HF incremental forward {ckpt[0]}", flush=True)
    seq, got = DIPDecoder(model, 32, fused=False).generate(prompt, NEW, return_logits=True)
    seq = seq.cuda()
    ref = []
    with torch.no_grad():
        cache = DynamicCache(config=model.config)
        out = model(input_ids=seq[:, :PLEN], past_key_values=cache, use_cache=True)
        ref.append(out.logits[0, -1].float())
        for t in range(PLEN, PLEN + NEW - 1):
            out = model(input_ids=seq[:, t:t + 1], past_key_values=cache, use_cache=True)
            ref.append(out.logits[0, -1].float())
    assert torch.equal(got, torch.stack(ref))


@pytest.mark.parametrize("keep,bound", [(KEEP, 8e-2), (1.0, 2e-2)])
def test_decode_matches_cpu_oracle_model(ckpt, streaming, keep, bound):
    """The same checkpoint on the CPU with every projection and MLP from the
    oracle (fp64 GEMV sums rounded to bf16, bit-exact threshold top-k), fed
    the GPU's tokens.  At keep 1.0 nothing is selected away, so the two
    differ by rounding only; at keep 0.6 a bf16-level difference in an MLP
    input can swap a channel at the top-k boundary, and in a random-weight
    model each swap moves y by about 1/sqrt(k) of its size, hence the wider
    bound."""
    from dip_model import DIPDecoder
    from dip_stream_predispatch import load_streaming_dip
    name, d, cfg = ckpt
    print(f"decode vs CPU oracle model {name} keep {keep}", flush=True)
    model, _, prompt = streaming
    if keep != KEEP:
        model, _, _ = load_streaming_dip(d, keep_ratio=keep)
    seq, got = DIPDecoder(model, 32).generate(prompt, NEW, return_logits=True)
    cpu = oracle_model(d, keep)
    ref = teacher_forced_logits(DIPDecoder(cpu, 32, use_graph=False), seq, PLEN)
    err = max_rel(got, ref)
    print(f"  max_rel {err:.3e}", flush=True)
    assert err < bound
    assert_confident_argmax(got, ref, bound)


class _DenseRoute(torch.nn.Module):
    """A StreamingDIPMlp forced onto its dense route for every input."""

    def __init__(self, sdip):
        super().__init__()
        self.sdip = sdip

    def forward(self, x):
        return self.sdip._dense(x)


def test_keep_one_matches_dense_route(ckpt):
    """At keep 1.0 the DIP MLP selects every channel, so decoding equals the
    modules' dense route (dip_stream_predispatch.py:206-215: dequantized
    gate/up GEMMs and the transposed down) on every token."""
    from dip_model import DIPDecoder, swap_modules
    from dip_stream_predispatch import load_streaming_dip
    name, d, cfg = ckpt
    print(f"keep 1.0 vs dense route {name}", flush=True)
    prompt = torch.randint(0, cfg.vocab_size, (1, PLEN), generator=torch.Generator().manual_seed(2))
    full, _, sdips = load_streaming_dip(d, keep_ratio=1.0)
    assert all(s.k == cfg.intermediate_size for s in sdips)
    seq, got = DIPDecoder(full, 32).generate(prompt, NEW, return_logits=True)
    names = [f"model.layers.{i}.mlp" for i in range(len(sdips))]
    swap_modules(full, names, [_DenseRoute(s) for s in sdips])
    ref = teacher_forced_logits(DIPDecoder(full, 32, use_graph=False), seq, PLEN)
    err = max_rel(got, ref)
    print(f"  max_rel {err:.3e}", flush=True)
    assert err < 3e-2


def test_cache_aware_model_calibrates_and_decodes(ckpt, streaming):
    """load_dip_ca + calibrate_cache over a short greedy generation: every
    decode call is counted (k per call), each layer's cache holds the
    cache_frac most selected channels, and decoding with the cache gives the
    streaming model's logits up to the down sum's channel order."""
    from dip_ca import load_dip_ca, calibrate_cache
    from dip_model import DIPDecoder
    name, d, cfg = ckpt
    model, _, prompt = streaming
    print(f"cache-aware model {name}", flush=True)
    ca_model, tok, cas = load_dip_ca(d, keep_ratio=KEEP, cache_frac=0.3)
    calib = 6
    counts = calibrate_cache(ca_model, tok, cas, prompt, calib_tokens=calib)
    for c, cnt in zip(cas, counts):
        assert int(cnt.sum()) == c.k * (calib - 1)
        assert c.cache_ids.numel() == c.cache_n == int(round(c.inter * 0.3))
        hot, id2slot = O.hot_set(cnt.cpu().numpy(), c.cache_n)
        assert np.array_equal(c.cache_ids.cpu().numpy(), hot)
        assert np.array_equal(c.id2slot.cpu().numpy(), id2slot)
    with pytest.raises(ValueError):
        DIPDecoder(ca_model, 32, use_graph=True)
    seq, ref = DIPDecoder(model, 32).generate(prompt, NEW, return_logits=True)
    got = teacher_forced_logits(DIPDecoder(ca_model, 32, use_graph=False), seq.cuda(), PLEN)
    err = max_rel(got, ref)
    print(f"  max_rel {err:.3e}  hits {cas[0].buf.last_n_hit} misses {cas[0].buf.last_n_miss}",
          flush=True)
    assert err < 2e-2
    # determinism, as the reference checks it (tests/test_ca_determinism.py:
    # 16-50: two generations, identical output): two greedy generates of the
    # cache-aware model give the same tokens and bit-identical logits
    dec = DIPDecoder(ca_model, 32, use_graph=False)
    s1, l1 = dec.generate(prompt, NEW, return_logits=True)
    s2, l2 = dec.generate(prompt, NEW, return_logits=True)
    assert torch.equal(s1, s2) and torch.equal(l1, l2)


@pytest.mark.parametrize("cols", [256, 512, 1024, 2048, 2560, 4096, 5120, 8192])
def test_quantlinear_decode_route(cols):
    """QuantLinear on one GPU token runs the int4 GEMV: the fp64 oracle's
    bars, and within bf16 rounding of the dense dequant + F.linear route."""
    from qlinear import QuantLinear
    rng = np.random.default_rng(cols)
    rows = 384
    qw, sc = random_int4(rng, rows, cols)
    x = random_bf16(rng, cols)
    lin = QuantLinear(cols, rows).cuda()
    lin.qweight.copy_(dev(qw))
    lin.scales.copy_(dev_bf16(sc))
    xd = dev_bf16(x)
    y = lin(xd.view(1, 1, cols))
    assert y.shape == (1, 1, rows)
    got = host_bf16(y.view(-1))
    ref = O.gemv_f64(qw, sc, x)
    assert rel_err(got, ref) < 1e-2
    assert_fp32_close(got, ref, gemv_abs_terms(qw, sc, x))
    dense = lin(torch.stack([xd, xd]).view(1, 2, cols))[0, 0]
    assert max_rel(y.view(-1).float(), dense.float()) < 1e-2
