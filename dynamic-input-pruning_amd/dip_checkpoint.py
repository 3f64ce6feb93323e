"""The reference's int4 checkpoint on disk, read into resident DIP MLPs.

Format (written by the reference's scripts/quantize.py:106-151):
  * <dir>/model_int4.safetensors: every weight `<name>.weight` that
    should_quantize selects (the q/k/v/o and gate/up/down projections) is
    stored as `<name>.qweight` (int8 [out, in/2], low nibble = even column)
    and `<name>.scales` (bf16 [out, in/128]); every other tensor is kept,
    fp32 ones cast to bf16;
  * <dir>/quant_config.json: the quantizer's parameters (QUANT_CONFIG).
The MLP loader (dip_stream_predispatch.py:218-246) reads, for every decoder
MLP `<m>` (e.g. `model.layers.7.mlp`), `<m>.{gate,up,down}_proj.{qweight,
scales}` and builds a StreamingDIPMlp, transposing down once.  Here every
MLP is read straight to the GPU and down is transposed there
(dip_transpose_down_int4, bit-identical to the reference's CPU route).
"""
from __future__ import annotations

import json
import re
from pathlib import Path

import torch
from safetensors import safe_open
from safetensors.torch import save_file

import _dip_hip as K
from quantize import GROUP_SIZE, QMAX, quantize_tensor_int4_groupwise

ST_NAME = "model_int4.safetensors"
QUANT_CONFIG = {  # scripts/quantize.py:142-149
    "quant_method": "self_int4_symmetric_groupwise",
    "group_size": GROUP_SIZE,
    "bits": 4,
    "symmetric": True,
    "packing": "two_int4_per_int8_low_even_high_odd",
    "qmax": QMAX,
}
_PROJ = ("gate_proj", "up_proj", "down_proj")


def should_quantize(name: str) -> bool:
    """The reference's selection (scripts/quantize.py:66-80): `.weight`
    tensors of the attention and MLP projections, never embeddings, norms or
    lm_head."""
    if not name.endswith(".weight"):
        return False
    lname = name.lower()
    if "embed_tokens" in lname or "lm_head" in lname or "norm" in lname:
        return False
    return any(p in lname for p in ("q_proj", "k_proj", "v_proj", "o_proj") + _PROJ)


def quantize_state_dict(sd: dict) -> dict:
    """The reference's per-tensor loop (scripts/quantize.py:106-124) on a state
    dict: selected weights -> .qweight/.scales, fp32 others -> bf16."""
    out = {}
    for name, t in sd.items():
        if should_quantize(name):
            base = name[: -len(".weight")]
            q, s = quantize_tensor_int4_groupwise(t)
            out[base + ".qweight"] = q.cpu().contiguous()
            out[base + ".scales"] = s.cpu().contiguous()
        else:
            out[name] = (t.to(torch.bfloat16) if t.dtype == torch.float32 else t).cpu().contiguous()
    return out


def save_int4_checkpoint(out_dir, state_dict: dict) -> Path:
    """Quantize `state_dict` and write model_int4.safetensors + quant_config.json
    into `out_dir` (scripts/quantize.py:126-151)."""
    out_dir = Path(out_dir)
    out_dir.mkdir(parents=True, exist_ok=True)
    save_file(quantize_state_dict(state_dict), str(out_dir / ST_NAME))
    with open(out_dir / "quant_config.json", "w") as f:
        json.dump(QUANT_CONFIG, f, indent=2)
    return out_dir / ST_NAME


def read_quant_config(ckpt_dir) -> dict:
    """quant_config.json, checked against the format the kernels read."""
    path = Path(ckpt_dir) / "quant_config.json"
    with open(path) as f:
        cfg = json.load(f)
    for key in ("group_size", "bits", "symmetric", "packing"):
        if cfg.get(key) != QUANT_CONFIG[key]:
            raise ValueError(f"{path}: {key}={cfg.get(key)!r}, this build reads "
                             f"{QUANT_CONFIG[key]!r}")
    return cfg


def _natural_key(name: str):
    return [int(p) if p.isdigit() else p for p in re.split(r"(\d+)", name)]


def mlp_names(st_path) -> list:
    """Every module `<m>` with all six `<m>.{gate,up,down}_proj.{qweight,scales}`
    tensors, in layer order."""
    with safe_open(str(st_path), framework="pt", device="cpu") as f:
        keys = set(f.keys())
    found = []
    for key in keys:
        if key.endswith(".gate_proj.qweight"):
            m = key[: -len(".gate_proj.qweight")]
            if all(f"{m}.{p}.{t}" in keys for p in _PROJ for t in ("qweight", "scales")):
                found.append(m)
    return sorted(found, key=_natural_key)


def iter_mlp_layers(ckpt_dir, device="cuda:0", names=None):
    """Per MLP (layer order) a dict {'name', 'gate_qw', 'gate_sc', 'up_qw',
    'up_sc', 'down_t_qw', 'down_t_sc'} resident on `device`, read one layer
    at a time; down is transposed to [inter, hidden/2] on the GPU
    (dip_stream_predispatch.py:100-120)."""
    ckpt_dir = Path(ckpt_dir)
    read_quant_config(ckpt_dir)
    st_path = ckpt_dir / ST_NAME
    names = mlp_names(st_path) if names is None else list(names)
    if not names:
        raise ValueError(f"{st_path}: no MLP with gate/up/down qweight and scales")
    dev = torch.device(device)
    with safe_open(str(st_path), framework="pt", device="cpu") as f:
        keys = set(f.keys())
        for m in names:
            missing = [f"{m}.{p}.{t}" for p in _PROJ for t in ("qweight", "scales")
                       if f"{m}.{p}.{t}" not in keys]
            if missing:
                raise ValueError(f"{st_path}: missing {missing}")
            t = {f"{p.split('_')[0]}_{kind}": f.get_tensor(f"{m}.{p}.{full}").to(dev)
                 for p in _PROJ for kind, full in (("qw", "qweight"), ("sc", "scales"))}
            d_qw, d_sc = K.transpose_down_int4(t.pop("down_qw"), t.pop("down_sc"))
            inter, hidden = t["up_qw"].shape[0], t["up_qw"].shape[1] * 2
            if t["gate_qw"].shape != (inter, hidden // 2) or d_qw.shape != (inter, hidden // 2):
                raise ValueError(f"{m}: gate/up/down shapes disagree")
            yield dict(name=m, down_t_qw=d_qw, down_t_sc=d_sc, **t)


def load_mlp_layers(ckpt_dir, device="cuda:0", names=None) -> list:
    """Every MLP of the checkpoint as iter_mlp_layers yields them."""
    return list(iter_mlp_layers(ckpt_dir, device, names))


def load_streaming_mlps(ckpt_dir, keep_ratio=0.6, device="cuda:0", names=None):
    """The MLP half of the reference's load_streaming_dip
    (dip_stream_predispatch.py:218-246): one StreamingDIPMlp per MLP of the
    checkpoint, all sharing one SharedBuffers.  Returns (names, modules,
    shared)."""
    from dip_stream_predispatch import SharedBuffers, StreamingDIPMlp
    layers = load_mlp_layers(ckpt_dir, device, names)
    first = layers[0]
    inter = first["up_qw"].shape[0]
    out_f = first["down_t_qw"].shape[1] * 2
    k = max(1, int(round(inter * keep_ratio)))
    shared = SharedBuffers(k, first["up_qw"].shape[1], first["up_sc"].shape[1], out_f,
                           out_f // GROUP_SIZE, device)
    mods = [StreamingDIPMlp(L["gate_qw"], L["gate_sc"], L["up_qw"], L["up_sc"], L["down_t_qw"],
                            L["down_t_sc"], shared, keep_ratio, device, down_transposed=True)
            for L in layers]
    return [L["name"] for L in layers], mods, shared
