"""A small random-weight Qwen3 for the whole-model tests: transformers builds
it from a config (no download), its state dict is written in the
reference's int4 checkpoint layout, and the norm weights are randomised so a
skipped or misplaced norm changes the logits."""
from __future__ import annotations

import numpy as np
import torch
import torch.nn as nn


def tiny_config(hidden=256, inter=512, layers=2, heads=4, kv_heads=2, head_dim=64, vocab=512,
                max_pos=512, rope_theta=1e6):
    from transformers import Qwen3Config
    return Qwen3Config(vocab_size=vocab, hidden_size=hidden, intermediate_size=inter,
                       num_hidden_layers=layers, num_attention_heads=heads,
                       num_key_value_heads=kv_heads, head_dim=head_dim,
                       max_position_embeddings=max_pos,
                       rope_parameters={"rope_type": "default", "rope_theta": rope_theta},
                       tie_word_embeddings=False)


def tiny_model(cfg, seed=0, dtype=torch.float32):
    from transformers import Qwen3ForCausalLM
    torch.manual_seed(seed)
    m = Qwen3ForCausalLM(cfg).eval()
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for name, p in m.named_parameters():
            if name.endswith("norm.weight"):
                p.copy_(1.0 + 0.1 * torch.randn(p.shape, generator=g))
    return m.to(dtype)


def write_checkpoint(model, out_dir):
    """config.json + model_int4.safetensors + quant_config.json."""
    from dip_checkpoint import save_int4_checkpoint
    model.config.save_pretrained(str(out_dir))
    sd = {k: v.detach().float() if v.is_floating_point() else v
          for k, v in model.state_dict().items()}
    save_int4_checkpoint(out_dir, sd)
    return out_dir


def max_rel(a: torch.Tensor, b: torch.Tensor) -> float:
    """max|a - b| / max|b| (the reference's comparison metric)."""
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


def assert_confident_argmax(got: torch.Tensor, ref: torch.Tensor, bound: float) -> int:
    """Every row whose reference top-1 logit beats its top-2 by more than
    twice the allowed error (bound * max|ref|) must pick the same token;
    rows with a smaller margin may flip within the tolerance.  Returns how
    many rows were checked."""
    got, ref = got.detach().float().cpu(), ref.detach().float().cpu()
    tol = bound * float(ref.abs().max())
    top2 = ref.topk(2, dim=-1).values
    sure = (top2[:, 0] - top2[:, 1]) > 2 * tol
    assert torch.equal(got.argmax(-1)[sure], ref.argmax(-1)[sure])
    return int(sure.sum())


def teacher_forced_logits(dec, seq: torch.Tensor, plen: int) -> torch.Tensor:
    """Logits the decoder gives at positions plen-1 .. len-2 of `seq` [1, L]
    when fed the tokens of `seq` (prefill of the first plen, then one step
    per token)."""
    out = [dec.prefill(seq[:, :plen]).float().cpu()]
    for t in range(plen, seq.shape[1] - 1):
        dec.tok.fill_(int(seq[0, t]))
        out.append(dec.step().float().cpu())
    return torch.stack(out)


class OracleDIPMlp(nn.Module):
    """The DIP MLP on the CPU from the oracle: the decode path
    (dip_stream_predispatch.py:176-204) for one-token inputs, the dense path
    (:206-215) otherwise; int4 tensors as numpy arrays, down transposed."""

    def __init__(self, gate_qw, gate_sc, up_qw, up_sc, down_qw, down_sc, keep_ratio):
        super().__init__()
        import dip_oracle as O
        self.O = O
        npy = lambda t: t.numpy() if t.dtype == torch.int8 else t.view(torch.int16).numpy().view(np.uint16)
        self.w = [npy(gate_qw), npy(gate_sc), npy(up_qw), npy(up_sc)]
        self.w += list(O.transpose_down_to_int4(npy(down_qw), npy(down_sc)))
        self.k = O.keep_count(up_qw.shape[0], keep_ratio)

    def forward(self, x):
        O = self.O
        rows = x.reshape(-1, x.shape[-1]).to(torch.bfloat16).view(torch.int16).numpy()
        decode = x.dim() == 3 and x.shape[1] == 1
        ys = []
        for r in rows:
            xb = r.view(np.uint16)
            res = O.dip_forward(*self.w, xb, self.k) if decode else O.dense_forward(*self.w, xb)
            ys.append(torch.from_numpy(res["y"].view(np.int16).copy()).view(torch.bfloat16))
        return torch.stack(ys).reshape(*x.shape[:-1], -1).to(x.dtype)


class OracleLinear(nn.Module):
    """A QuantLinear on the CPU from the oracle: one-token inputs through the
    fp64 GEMV rounded to bf16 (what the GPU's int4 GEMV computes), longer
    inputs through the host dequant + F.linear route."""

    def __init__(self, ql):
        super().__init__()
        import dip_oracle as O
        self.O = O
        self.ql = ql
        self.qw = ql.qweight.numpy()
        self.sc = ql.scales.view(torch.int16).numpy().view(np.uint16)

    def forward(self, x):
        if x.numel() != self.ql.in_features:
            return self.ql(x)
        xb = x.reshape(-1).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        y = self.O.gemv_bf16(self.qw, self.sc, xb)
        y = torch.from_numpy(y.view(np.int16).copy()).view(torch.bfloat16)
        return y.to(x.dtype).reshape(*x.shape[:-1], -1)


def oracle_model(ckpt_dir, keep_ratio):
    """The checkpoint's model on the CPU with OracleLinear projections and
    OracleDIPMlp MLPs."""
    from safetensors import safe_open
    from dip_checkpoint import ST_NAME
    from dip_model import build_empty_model, load_tensors, mlp_module_names, swap_modules
    model = build_empty_model(ckpt_dir)
    names = mlp_module_names(model)
    mods = []
    with safe_open(str(ckpt_dir / ST_NAME), framework="pt", device="cpu") as f:
        for n in names:
            t = [f.get_tensor(f"{n}.{p}_proj.{s}") for p in ("gate", "up", "down")
                 for s in ("qweight", "scales")]
            mods.append(OracleDIPMlp(*t, keep_ratio))
    swap_modules(model, names, mods)
    load_tensors(model, ckpt_dir / ST_NAME, "cpu", skip_prefixes=names)
    from qlinear import QuantLinear
    qnames = [n for n, m in model.named_modules() if isinstance(m, QuantLinear)]
    swap_modules(model, qnames, [OracleLinear(model.get_submodule(n)) for n in qnames])
    return model
