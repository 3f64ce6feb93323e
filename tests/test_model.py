"""Whole-model integration on the CPU: the projection swap of the reference's
loaders (qlinear.py:91-106), the checkpoint -> model key mapping of
load_quantized_qwen3 (qlinear.py:109-166), and DIPDecoder's decode step
against transformers' own Qwen3 forward on the same modules (fp32, so the
two differ by summation order only)."""
import pytest
import torch
import torch.nn as nn
from safetensors import safe_open
from safetensors.torch import save_file

from model_util import max_rel, teacher_forced_logits, tiny_config, tiny_model, write_checkpoint


def test_replace_linears_swaps_the_seven_projections():
    from transformers import Qwen3ForCausalLM
    from qlinear import QuantLinear, _replace_linears_with_quant
    cfg = tiny_config(layers=3)
    m = Qwen3ForCausalLM(cfg)
    shapes = {n: (mod.in_features, mod.out_features) for n, mod in m.named_modules()
              if isinstance(mod, nn.Linear)}
    names = _replace_linears_with_quant(m)
    assert len(names) == 7 * 3
    assert sorted({n.rsplit(".", 1)[1] for n in names}) == sorted(
        ["q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"])
    for n in names:
        q = m.get_submodule(n)
        assert isinstance(q, QuantLinear) and (q.in_features, q.out_features) == shapes[n]
        assert q.qweight.shape == (q.out_features, q.in_features // 2)
    assert type(m.lm_head) is nn.Linear and type(m.model.embed_tokens) is nn.Embedding


@pytest.mark.parametrize("heads,kv_heads", [(4, 2), (4, 4), (8, 1)])
def test_decoder_step_matches_hf_forward(heads, kv_heads):
    """Prefill + one step per token reproduces the logits of one causal HF
    forward over the whole sequence at every position."""
    from dip_model import DIPDecoder
    cfg = tiny_config(heads=heads, kv_heads=kv_heads)
    m = tiny_model(cfg, seed=heads * 10 + kv_heads)
    seq = torch.randint(0, cfg.vocab_size, (1, 14), generator=torch.Generator().manual_seed(3))
    with torch.no_grad():
        ref = m(seq).logits[0]
    dec = DIPDecoder(m, max_len=40, use_graph=False)
    got = teacher_forced_logits(dec, seq, 5)
    assert int(dec.pos) == 13
    assert max_rel(got, ref[4:13]) < 1e-5


def test_decoder_generate_matches_hf_generate():
    from dip_model import DIPDecoder
    cfg = tiny_config()
    m = tiny_model(cfg, seed=7)
    ids = torch.randint(0, cfg.vocab_size, (1, 6), generator=torch.Generator().manual_seed(4))
    with torch.no_grad():
        ref = m.generate(ids, max_new_tokens=12, do_sample=False, pad_token_id=0)
    out = DIPDecoder(m, max_len=32, use_graph=False).generate(ids, 12)
    assert torch.equal(out, ref)


def test_decoder_limits():
    from dip_model import DIPDecoder
    cfg = tiny_config()
    m = tiny_model(cfg, seed=1)
    dec = DIPDecoder(m, max_len=8, use_graph=False)
    with pytest.raises(ValueError):
        dec.prefill(torch.zeros(1, 8, dtype=torch.long))
    with pytest.raises(ValueError):
        dec.generate(torch.zeros(1, 4, dtype=torch.long), 5)
    eos_seq = dec.generate(torch.zeros(1, 2, dtype=torch.long), 6)
    first = int(eos_seq[0, 2])
    cut = dec.generate(torch.zeros(1, 2, dtype=torch.long), 6, eos_token_id=first)
    assert cut.shape[1] == 3 and int(cut[0, 2]) == first


def test_load_quantized_qwen3_maps_every_tensor(tmp_path):
    """The int4 baseline model read from the checkpoint equals an HF model
    holding bf16(q*s) projection weights and the other tensors in bf16."""
    from transformers import AutoModelForCausalLM
    from dip_checkpoint import ST_NAME
    from qlinear import dequantize, load_quantized_qwen3
    cfg = tiny_config()
    src = tiny_model(cfg, seed=11)
    write_checkpoint(src, tmp_path)
    model, tok = load_quantized_qwen3(tmp_path, device="cpu")
    assert tok is None
    ref = AutoModelForCausalLM.from_config(cfg, dtype=torch.bfloat16).eval()
    sd = {}
    with safe_open(str(tmp_path / ST_NAME), framework="pt", device="cpu") as f:
        for key in f.keys():
            if key.endswith(".qweight"):
                base = key[: -len(".qweight")]
                sd[base + ".weight"] = dequantize(f.get_tensor(key), f.get_tensor(base + ".scales"))
            elif not key.endswith(".scales"):
                sd[key] = f.get_tensor(key)
    ref.load_state_dict(sd, strict=True)
    seq = torch.randint(0, cfg.vocab_size, (1, 9), generator=torch.Generator().manual_seed(5))
    with torch.no_grad():
        assert torch.equal(model(seq).logits, ref(seq).logits)


def test_loader_rejects_missing_and_misshapen_tensors(tmp_path):
    from dip_checkpoint import ST_NAME
    from qlinear import load_quantized_qwen3
    write_checkpoint(tiny_model(tiny_config(), seed=2), tmp_path)
    path = tmp_path / ST_NAME
    with safe_open(str(path), framework="pt", device="cpu") as f:
        full = {k: f.get_tensor(k) for k in f.keys()}
    part = dict(full)
    del part["model.layers.1.self_attn.k_norm.weight"]
    save_file(part, str(path))
    with pytest.raises(ValueError, match="no tensor"):
        load_quantized_qwen3(tmp_path, device="cpu")
    bad = dict(full)
    bad["model.norm.weight"] = bad["model.norm.weight"][:-1].clone()
    save_file(bad, str(path))
    with pytest.raises(ValueError, match="shape"):
        load_quantized_qwen3(tmp_path, device="cpu")
