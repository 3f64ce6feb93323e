"""The reference's int4 checkpoint format (scripts/quantize.py:66-151) as
written and read by dip_checkpoint, on the CPU: which tensors are quantized,
the stored layout and dtypes, the quantizer's bytes against the oracle, the
quant config and the layer order of the MLP loader."""
import json

import numpy as np
import pytest
import torch
from safetensors import safe_open

import dip_checkpoint as C
import dip_oracle as O


def test_should_quantize_matches_reference_rule():
    yes = ["model.layers.0.self_attn.q_proj.weight", "model.layers.3.self_attn.k_proj.weight",
           "model.layers.3.self_attn.v_proj.weight", "model.layers.3.self_attn.o_proj.weight",
           "model.layers.9.mlp.gate_proj.weight", "model.layers.9.mlp.up_proj.weight",
           "model.layers.9.mlp.down_proj.weight"]
    no = ["model.embed_tokens.weight", "lm_head.weight", "model.norm.weight",
          "model.layers.0.input_layernorm.weight", "model.layers.0.self_attn.q_norm.weight",
          "model.layers.0.self_attn.q_proj.bias", "model.layers.0.mlp.gate_proj.qweight"]
    assert all(C.should_quantize(n) for n in yes)
    assert not any(C.should_quantize(n) for n in no)


def _state(H=256, I=512, layers=(0, 1, 10), seed=0):
    g = torch.Generator().manual_seed(seed)
    sd = {"model.embed_tokens.weight": torch.randn(64, H, generator=g),
          "model.norm.weight": torch.ones(H)}
    for i in layers:
        p = f"model.layers.{i}"
        sd[f"{p}.input_layernorm.weight"] = torch.ones(H)
        sd[f"{p}.self_attn.q_proj.weight"] = torch.randn(H, H, generator=g) * 0.02
        sd[f"{p}.mlp.gate_proj.weight"] = torch.randn(I, H, generator=g) * 0.02
        sd[f"{p}.mlp.up_proj.weight"] = torch.randn(I, H, generator=g) * 0.02
        sd[f"{p}.mlp.down_proj.weight"] = torch.randn(H, I, generator=g) * 0.02
    return sd


def test_write_read_layout(tmp_path):
    sd = _state()
    st = C.save_int4_checkpoint(tmp_path, sd)
    cfg = json.loads((tmp_path / "quant_config.json").read_text())
    assert cfg == C.QUANT_CONFIG
    assert C.read_quant_config(tmp_path) == cfg
    with safe_open(str(st), framework="pt", device="cpu") as f:
        keys = set(f.keys())
        for name, w in sd.items():
            if C.should_quantize(name):
                base = name[:-len(".weight")]
                assert name not in keys
                q, s = f.get_tensor(base + ".qweight"), f.get_tensor(base + ".scales")
                assert q.dtype == torch.int8 and s.dtype == torch.bfloat16
                assert tuple(q.shape) == (w.shape[0], w.shape[1] // 2)
                assert tuple(s.shape) == (w.shape[0], w.shape[1] // 128)
                oq, os_ = O.quantize_int4_groupwise(w.numpy())
                assert np.array_equal(q.numpy(), oq)
                assert np.array_equal(s.view(torch.int16).numpy().view(np.uint16), os_)
            else:
                kept = f.get_tensor(name)
                assert kept.dtype == torch.bfloat16
                assert torch.equal(kept, w.to(torch.bfloat16))
    assert C.mlp_names(st) == ["model.layers.0.mlp", "model.layers.1.mlp", "model.layers.10.mlp"]


def test_quant_config_mismatch_is_rejected(tmp_path):
    C.save_int4_checkpoint(tmp_path, _state(layers=(0,)))
    cfg = dict(C.QUANT_CONFIG, group_size=64)
    (tmp_path / "quant_config.json").write_text(json.dumps(cfg))
    with pytest.raises(ValueError, match="group_size"):
        C.read_quant_config(tmp_path)


def test_incomplete_mlp_is_skipped(tmp_path):
    sd = _state(layers=(0, 1))
    del sd["model.layers.1.mlp.down_proj.weight"]
    st = C.save_int4_checkpoint(tmp_path, sd)
    assert C.mlp_names(st) == ["model.layers.0.mlp"]
