"""Whole-model integration: an HF Qwen3 built from an int4 checkpoint with
its MLPs swapped for DIP modules, and a decode loop captured in one HIP graph.

Loading follows the reference's sequence (dip_stream_predispatch.py:218-289,
dip_ca.py:199-269, qlinear.py:109-166): build the architecture of
`config.json` with empty weights, swap the seven projections for QuantLinear,
swap each decoder MLP for a DIP module, then load every other tensor of
model_int4.safetensors.  One MI355X holds the whole model in HBM, so every
tensor goes to one device; there is no offload map.

``DIPDecoder`` runs greedy decoding.  The prompt goes through the HF forward
(the reference's prefill: the DIP modules take their dense route for
sequences longer than one token), then its key/value cache is copied into a
static cache and every further token runs one decode step that reads nothing
from the host: embedding, per layer RMSNorm -> q/k/v projections (int4 GEMV)
-> q/k RMSNorm -> rotary embedding from a precomputed table -> cache write
at the device-side position -> attention over the static cache with a
position mask -> o projection -> RMSNorm -> DIP MLP, then the final norm,
lm_head and argmax.  With ``use_graph`` the step up to the final norm (and
the position update) is captured once in a HIP graph and replayed per token;
lm_head and argmax run after each replay on the same stream.
The step uses the model's own modules, so the decode math is the HF model's
(transformers' Qwen3DecoderLayer / Qwen3Attention forward).
"""
from __future__ import annotations

from pathlib import Path

import torch
import torch.nn as nn
import torch.nn.functional as F
from safetensors import safe_open

from qlinear import _replace_linears_with_quant

# Rotary types whose inverse frequencies are fixed at construction; the
# dynamic ones recompute them from the sequence length at run time.
_STATIC_ROPE = ("default", "linear", "yarn", "llama3")


def build_empty_model(ckpt_dir, dtype=torch.bfloat16):
    """The causal LM of `ckpt_dir/config.json` with weights on the meta device
    (buffers computed at construction, such as rotary frequencies, stay
    real) and QuantLinear projections."""
    from accelerate import init_empty_weights
    from transformers import AutoConfig, AutoModelForCausalLM
    config = AutoConfig.from_pretrained(str(ckpt_dir))
    with init_empty_weights():
        model = AutoModelForCausalLM.from_config(config, dtype=dtype)
    _replace_linears_with_quant(model)
    return model.eval()


def mlp_module_names(model: nn.Module) -> list:
    """Names of the modules holding gate/up/down QuantLinear projections, in
    model order (the reference's selection, dip_stream_predispatch.py:231-233)."""
    from qlinear import QuantLinear
    return [n for n, m in model.named_modules()
            if all(hasattr(m, p) for p in ("gate_proj", "up_proj", "down_proj"))
            and isinstance(m.up_proj, QuantLinear)]


def swap_modules(model: nn.Module, names, modules) -> None:
    """Put each module of `modules` where `model.<name>` was."""
    for name, mod in zip(names, modules):
        parent_name, _, attr = name.rpartition(".")
        setattr(model.get_submodule(parent_name) if parent_name else model, attr, mod)


def _set_tensor(model: nn.Module, key: str, value: torch.Tensor, device) -> None:
    mod_name, _, attr = key.rpartition(".")
    mod = model.get_submodule(mod_name) if mod_name else model
    if attr in mod._parameters:
        old = mod._parameters[attr]
    elif attr in mod._buffers:
        old = mod._buffers[attr]
    else:
        raise KeyError(f"{key}: the model has no such parameter or buffer")
    if tuple(old.shape) != tuple(value.shape):
        raise ValueError(f"{key}: checkpoint shape {tuple(value.shape)}, model "
                         f"{tuple(old.shape)}")
    dt = old.dtype if old.dtype.is_floating_point and value.dtype.is_floating_point else value.dtype
    t = value.to(device=device, dtype=dt)
    if attr in mod._parameters:
        mod._parameters[attr] = nn.Parameter(t, requires_grad=False)
    else:
        mod._buffers[attr] = t


def load_tensors(model: nn.Module, st_path, device, skip_prefixes=()) -> None:
    """Load every tensor of `st_path` into `model` on `device`, except those
    under a module named in `skip_prefixes` (the swapped MLPs, whose weights
    their DIP modules already hold).  Ties lm_head to the embedding when the
    config says so and the checkpoint has no lm_head, moves the buffers made
    at construction to `device`, and raises if any parameter or buffer is
    still empty."""
    device = torch.device(device)
    skip = tuple(p + "." for p in skip_prefixes)
    with safe_open(str(st_path), framework="pt", device="cpu") as f:
        keys = list(f.keys())
        for key in keys:
            if key.startswith(skip):
                continue
            _set_tensor(model, key, f.get_tensor(key), device)
    if getattr(model.config, "tie_word_embeddings", False) and "lm_head.weight" not in keys:
        model.lm_head.weight = model.get_input_embeddings().weight
    _finish(model, device, st_path)


def _finish(model: nn.Module, device, source) -> None:
    """Move the buffers made at construction to `device`; raise if any
    parameter or buffer is still empty."""
    for mod in model.modules():
        for name, buf in list(mod._buffers.items()):
            if buf is not None and not buf.is_meta and buf.device != device:
                mod._buffers[name] = buf.to(device)
    empty = [n for n, t in list(model.named_parameters()) + list(model.named_buffers())
             if t.is_meta]
    if empty:
        raise ValueError(f"{source}: no tensor for {len(empty)} model entries, e.g. "
                         f"{empty[:4]}")


# Published Qwen3 architectures (the models' config.json values).
QWEN3_SHAPES = {
    "qwen3-32b": dict(hidden_size=5120, intermediate_size=25600, num_hidden_layers=64,
                      num_attention_heads=64, num_key_value_heads=8),
    "qwen3-8b": dict(hidden_size=4096, intermediate_size=12288, num_hidden_layers=36,
                     num_attention_heads=32, num_key_value_heads=8),
}


def qwen3_config(shape: str = "qwen3-32b", **overrides):
    """A Qwen3Config of a published model's shape (vocabulary 151936, head
    dim 128, rope theta 1e6, untied embeddings)."""
    from transformers import Qwen3Config
    kw = dict(QWEN3_SHAPES[shape], vocab_size=151936, head_dim=128, rms_norm_eps=1e-6,
              max_position_embeddings=40960, tie_word_embeddings=False,
              rope_parameters={"rope_type": "default", "rope_theta": 1e6})
    kw.update(overrides)
    return Qwen3Config(**kw)


def synthetic_model(config, keep_ratio: float = 0.6, device="cuda:0", seed: int = 0,
                    std: float = 0.02):
    """A causal LM of `config` with N(0, std) weights drawn on the device, for
    benchmarks (no checkpoint needed): every projection quantized int4 g128
    with the reference quantizer rule (QuantLinear buffers), every MLP a
    StreamingDIPMlp whose down is drawn and quantized directly in the
    transposed layout, norm weights 1, embedding and lm_head bf16.
    Returns (model, list of the StreamingDIPMlp modules)."""
    import _dip_hip as K
    from accelerate import init_empty_weights
    from transformers import AutoModelForCausalLM
    from dip_stream_predispatch import SharedBuffers, StreamingDIPMlp
    from qlinear import QuantLinear
    device = torch.device(device)
    with init_empty_weights():
        model = AutoModelForCausalLM.from_config(config, dtype=torch.bfloat16)
    _replace_linears_with_quant(model)
    model.eval()
    gen = torch.Generator(device=device).manual_seed(seed)

    def draw(*shape):
        return torch.randn(*shape, device=device, generator=gen) * std

    H, I = config.hidden_size, config.intermediate_size
    k = max(1, int(round(I * keep_ratio)))
    shared = SharedBuffers(k, H // 2, H // 128, H, H // 128, device)
    names = mlp_module_names(model)
    mods = []
    for _ in names:
        w = [K.quantize_int4(draw(I, H)) for _ in range(3)]
        mods.append(StreamingDIPMlp(*w[0], *w[1], *w[2], shared, keep_ratio, device,
                                    down_transposed=True))
    swap_modules(model, names, mods)
    for name, mod in model.named_modules():
        if isinstance(mod, QuantLinear):
            qw, sc = K.quantize_int4(draw(mod.out_features, mod.in_features))
            mod._buffers["qweight"], mod._buffers["scales"] = qw, sc
    for name, p in list(model.named_parameters()):
        if p.is_meta:
            t = (torch.ones(p.shape, device=device) if name.endswith("norm.weight")
                 else draw(*p.shape))
            _set_tensor(model, name, t.to(torch.bfloat16), device)
    if getattr(config, "tie_word_embeddings", False):
        model.lm_head.weight = model.get_input_embeddings().weight
    _finish(model, device, "synthetic_model")
    return model, mods


def load_tokenizer(ckpt_dir):
    """The checkpoint's tokenizer, or None when the directory holds none."""
    ckpt_dir = Path(ckpt_dir)
    if not any((ckpt_dir / f).exists() for f in ("tokenizer.json", "tokenizer_config.json")):
        return None
    from transformers import AutoTokenizer
    return AutoTokenizer.from_pretrained(str(ckpt_dir))


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


class DIPDecoder:
    """Greedy decoding of a Qwen3 causal LM with a static key/value cache and
    a HIP-graph decode step.  Batch size 1, as the reference's decode.

    Args:
      model:     a Qwen3ForCausalLM-shaped model (model.model.layers[i] with
                 self_attn.{q,k,v,o}_proj, q_norm, k_norm, input_layernorm,
                 post_attention_layernorm and mlp); any MLP module works.
      max_len:   cache length (prompt + generated tokens).  Up to 1024 rows
                 the attention runs in one launch per layer, beyond it on
                 the three-launch split path, so the default covers the
                 reference's benchmark (a short prompt + 64 tokens) on the
                 fast path; pass more for longer sequences.
      use_graph: capture the decode step in a HIP graph (needs a GPU and MLP
                 modules that read nothing back to the host per token; a
                 module says it does with `graph_capturable = False`).
      fused:     run the layer's non-MLP steps with this library's decode
                 kernels instead of the HF modules' PyTorch ops: one fused
                 q|k|v GEMV with the residual add and the input RMSNorm
                 folded in; q/k norm + rotary + cache write + attention in
                 one launch for caches of up to 1024 rows, else three; the
                 o projection; the post-attention residual add and RMSNorm
                 folded into the DIP MLP's gate (7 launches per layer, 9 for
                 long caches).  None: whenever the model fits them (GPU,
                 bf16, head_dim 128, int4 attention projections).
    """

    def __init__(self, model: nn.Module, max_len: int = 1024, use_graph: bool = True,
                 fused=None):
        inner = model.model
        cfg = model.config
        self.model = model
        self.layers = list(inner.layers)
        emb = inner.embed_tokens.weight
        self.device, self.dtype = emb.device, emb.dtype
        att = self.layers[0].self_attn
        self.hd = att.head_dim
        self.nh = cfg.num_attention_heads
        self.nkv = cfg.num_key_value_heads
        if any(getattr(L.self_attn, "sliding_window", None) for L in self.layers):
            raise ValueError("sliding-window attention layers are not supported")
        rot = inner.rotary_emb
        if rot.rope_type not in _STATIC_ROPE:
            raise ValueError(f"rope type {rot.rope_type!r}: frequencies change with length")
        self.max_len = int(max_len)
        pos = torch.arange(self.max_len, dtype=torch.float32, device=self.device)
        freqs = pos[:, None] * rot.inv_freq.to(self.device, torch.float32)[None, :]
        table = torch.cat((freqs, freqs), dim=-1)
        self.cos = (table.cos() * rot.attention_scaling).to(self.dtype)
        self.sin = (table.sin() * rot.attention_scaling).to(self.dtype)
        shape = (len(self.layers), self.nkv, self.max_len, self.hd)
        self.k_cache = torch.zeros(shape, dtype=self.dtype, device=self.device)
        self.v_cache = torch.zeros(shape, dtype=self.dtype, device=self.device)
        self._cols = torch.arange(self.max_len, device=self.device)
        self.tok = torch.zeros(1, dtype=torch.long, device=self.device)
        self.pos = torch.zeros(1, dtype=torch.long, device=self.device)
        supported = self._fused_supported()
        if fused and not supported:
            raise ValueError("fused decode needs a GPU, bf16 weights, head_dim 128, int4 "
                             "attention projections and a supported head grouping")
        self.fused = supported if fused is None else bool(fused)
        if self.fused:
            self._setup_fused()
        self.use_graph = bool(use_graph) and self.device.type == "cuda"
        if self.use_graph:
            bad = [i for i, L in enumerate(self.layers)
                   if not getattr(L.mlp, "graph_capturable", True)]
            if bad:
                raise ValueError(f"the MLPs of layers {bad[:4]} synchronise with the host "
                                 "per token and cannot be captured; use use_graph=False")
        self.graph = None
        self._graph_out = None

    # -- fused decode kernels -------------------------------------------------
    def _fused_supported(self) -> bool:
        from qlinear import QuantLinear, _GEMV_COLS
        if self.device.type != "cuda" or self.dtype != torch.bfloat16 or self.hd != 128:
            return False
        if self.nh % self.nkv or self.nh // self.nkv not in (1, 2, 4, 5, 8, 16):
            return False
        hidden = self.model.config.hidden_size
        if hidden > 8192 or hidden not in _GEMV_COLS or self.nh * self.hd not in _GEMV_COLS:
            return False
        for L in self.layers:
            a = L.self_attn
            if not all(isinstance(getattr(a, p), QuantLinear)
                       for p in ("q_proj", "k_proj", "v_proj", "o_proj")):
                return False
            if a.q_norm.variance_epsilon != a.k_norm.variance_epsilon:
                return False
        return True

    def _setup_fused(self) -> None:
        """Concatenate each layer's q/k/v projections into one [q|k|v]
        matrix (the projections keep views into it, so nothing is stored
        twice) and allocate the per-token buffers of the fused step."""
        import _dip_hip as K
        from dip_stream_predispatch import StreamingDIPMlp
        self._K = K
        self.hidden = self.model.config.hidden_size
        dev, bf = self.device, torch.bfloat16
        self._qkv_w = []
        for L in self.layers:
            a = L.self_attn
            parts = (a.q_proj, a.k_proj, a.v_proj)
            qw = torch.cat([p.qweight for p in parts])
            sc = torch.cat([p.scales for p in parts])
            r = 0
            for p in parts:
                n = p.out_features
                p._buffers["qweight"], p._buffers["scales"] = qw[r:r + n], sc[r:r + n]
                r += n
            self._qkv_w.append((qw, sc))
        self._mlp_fns = [(lambda x, m=L.mlp: m._decode_one(x))
                         if isinstance(L.mlp, StreamingDIPMlp) else
                         (lambda x, m=L.mlp, H=self.hidden: m(x.view(1, 1, H)).reshape(-1))
                         for L in self.layers]
        # two residual buffers: the q|k|v GEMV with the input RMSNorm folded in
        # reads one and writes the updated residual to the other
        self._hres = [torch.empty(self.hidden, dtype=bf, device=dev) for _ in range(2)]
        self._norm_gemv = self.hidden in K.NORM_GEMV_COLS
        self._mlp_norm = [self._norm_gemv and isinstance(L.mlp, StreamingDIPMlp)
                          for L in self.layers]
        self._x = torch.empty(self.hidden, dtype=bf, device=dev)
        self._a = torch.empty(self.hidden, dtype=bf, device=dev)
        self._qkv = torch.empty((self.nh + 2 * self.nkv) * self.hd, dtype=bf, device=dev)
        self._q = torch.empty(self.nh * self.hd, dtype=bf, device=dev)
        self._o = torch.empty(self.nh * self.hd, dtype=bf, device=dev)
        self._attn_ws = torch.zeros(K.decode_attention_workspace_bytes(self.nh, self.hd,
                                                                       self.max_len),
                                    dtype=torch.uint8, device=dev)
        # short caches: norm + rotary + cache write + attention in one launch
        # (one workgroup per kv head); longer ones split the cache over many
        # workgroups (three launches)
        self._attn_one_launch = self.max_len <= K.decode_attention_fused_max_len()

    def _body_fused(self) -> torch.Tensor:
        K = self._K
        inner = self.model.model
        H = self.hidden
        h, other = self._hres
        torch.index_select(inner.embed_tokens.weight, 0, self.tok, out=h.view(1, H))
        y = None
        for i, L in enumerate(self.layers):
            a = L.self_attn
            qw, sc = self._qkv_w[i]
            n_in = L.input_layernorm
            if self._norm_gemv:
                # residual add + input RMSNorm inside the q|k|v GEMV
                K.int4_gemv_rmsnorm(qw, sc, h, y, n_in.weight, n_in.variance_epsilon,
                                    h_out=other if y is not None else None, out=self._qkv)
                if y is not None:
                    h, other = other, h
            else:
                K.add_rmsnorm(h, y, n_in.weight, self._x, n_in.variance_epsilon)
                K.int4_gemv(qw, sc, self._x, out=self._qkv)
            if self._attn_one_launch:
                K.decode_attention_fused(self._qkv, a.q_norm.weight, a.k_norm.weight, self.cos,
                                         self.sin, self.pos, self.k_cache[i], self.v_cache[i],
                                         self._o, self.nh, self.nkv, a.q_norm.variance_epsilon,
                                         a.scaling)
            else:
                K.qk_norm_rope_cache(self._qkv, a.q_norm.weight, a.k_norm.weight, self.cos,
                                     self.sin, self.pos, self._q, self.k_cache[i],
                                     self.v_cache[i], self.nh, self.nkv,
                                     a.q_norm.variance_epsilon)
                K.decode_attention(self._q, self.k_cache[i], self.v_cache[i], self.pos, self._o,
                                   a.scaling, ws=self._attn_ws)
            K.int4_gemv(a.o_proj.qweight, a.o_proj.scales, self._o, out=self._a)
            pn = L.post_attention_layernorm
            if self._mlp_norm[i]:
                # residual add + post-attention RMSNorm inside the MLP's gate
                y = L.mlp.decode_rmsnorm(h, self._a, pn.weight, pn.variance_epsilon, other,
                                         self._x)
                h, other = other, h
            else:
                K.add_rmsnorm(h, self._a, pn.weight, self._x, pn.variance_epsilon)
                y = self._mlp_fns[i](self._x)
        K.add_rmsnorm(h, y, inner.norm.weight, self._x, inner.norm.variance_epsilon)
        return self._x.view(1, 1, H)

    # -- one decode step (device-side token and position) ---------------------
    def _body(self) -> torch.Tensor:
        if self.fused:
            return self._body_fused()
        return self._body_modules()

    def _body_modules(self) -> torch.Tensor:
        """Embedding of `tok` at `pos` through every layer and the final norm
        (the part the graph captures); returns the hidden state [1, 1, H]."""
        inner = self.model.model
        hd = self.hd
        h = inner.embed_tokens(self.tok).view(1, 1, -1)
        cos = self.cos.index_select(0, self.pos).view(1, 1, 1, hd)
        sin = self.sin.index_select(0, self.pos).view(1, 1, 1, hd)
        mask = torch.where(self._cols > self.pos, float("-inf"), 0.0).to(self.dtype).view(
            1, 1, 1, self.max_len)
        for i, layer in enumerate(self.layers):
            a = layer.self_attn
            x = layer.input_layernorm(h)
            q = a.q_norm(a.q_proj(x).view(1, 1, -1, hd)).transpose(1, 2)
            k = a.k_norm(a.k_proj(x).view(1, 1, -1, hd)).transpose(1, 2)
            v = a.v_proj(x).view(1, 1, -1, hd).transpose(1, 2)
            q = q * cos + _rotate_half(q) * sin
            k = k * cos + _rotate_half(k) * sin
            self.k_cache[i].index_copy_(1, self.pos, k[0])
            self.v_cache[i].index_copy_(1, self.pos, v[0])
            # query head j reads key/value head j // (nh / nkv); the one-token
            # queries of a group are the rows of one attention call, so the
            # cache is read once per kv head and never repeated
            qg = q.reshape(1, self.nkv, self.nh // self.nkv, hd)
            o = F.scaled_dot_product_attention(qg, self.k_cache[i:i + 1], self.v_cache[i:i + 1],
                                               attn_mask=mask, scale=a.scaling)
            h = h + a.o_proj(o.reshape(1, 1, -1))
            h = h + layer.mlp(layer.post_attention_layernorm(h))
        return inner.norm(h)

    def _head(self, h: torch.Tensor) -> torch.Tensor:
        """lm_head and the greedy choice, outside any graph: over a full
        vocabulary both are library calls (a GEMV and a many-workgroup
        reduction) that may clear their own scratch with a memset, which a
        captured graph does not replay reliably."""
        logits = self.model.lm_head(h).view(-1)
        self.tok.copy_(logits.argmax().view(1))
        return logits

    @torch.no_grad()
    def step(self) -> torch.Tensor:
        """Decode the token in `self.tok` at position `self.pos`; afterwards
        `self.tok` holds the argmax and `self.pos` has advanced by one.
        Returns the logits."""
        if not self.use_graph or self.graph is None:
            h = self._body()
            self.pos.add_(1)
            logits = self._head(h)
            if self.use_graph:
                # the first step ran eagerly (it also made every lazily
                # created buffer); capture the same body for later tokens
                torch.cuda.synchronize(self.device)
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    self._graph_out = self._body()
                    self.pos.add_(1)
                self.graph = g
            return logits
        self.graph.replay()
        return self._head(self._graph_out)

    # -- prompt ---------------------------------------------------------------
    @torch.no_grad()
    def prefill(self, input_ids: torch.Tensor) -> torch.Tensor:
        """Run the prompt [1, P] through the HF forward, copy its key/value
        cache into the static cache, set `tok` to the argmax of the last
        logits and `pos` to P.  Returns the last logits."""
        from transformers import DynamicCache
        ids = input_ids.to(self.device).view(1, -1)
        plen = ids.shape[1]
        if plen < 1 or plen >= self.max_len:
            raise ValueError(f"prompt length {plen} outside [1, {self.max_len})")
        cache = DynamicCache(config=self.model.config)
        out = self.model(input_ids=ids, past_key_values=cache, use_cache=True)
        for i, layer in enumerate(cache.layers):
            self.k_cache[i, :, :plen].copy_(layer.keys[0])
            self.v_cache[i, :, :plen].copy_(layer.values[0])
        logits = out.logits[0, -1]
        self.tok.copy_(logits.argmax().view(1))
        self.pos.fill_(plen)
        return logits

    @torch.no_grad()
    def generate(self, input_ids: torch.Tensor, max_new_tokens: int, eos_token_id=None,
                 return_logits: bool = False):
        """Greedy continuation of `input_ids` [1, P]: the prompt followed by up
        to `max_new_tokens` tokens (cut after the first `eos_token_id`), as
        HF's generate(do_sample=False) returns it for batch 1.  With
        `return_logits` also the logits of every generated token."""
        ids = input_ids.to(self.device).view(1, -1)
        plen = ids.shape[1]
        if plen + max_new_tokens > self.max_len:
            raise ValueError(f"{plen} + {max_new_tokens} tokens exceed max_len {self.max_len}")
        toks = torch.empty(max_new_tokens, dtype=torch.long, device=self.device)
        logs = []
        # every generation starts from fresh speculation keys, so the same
        # prompt gives the same tokens and logits bit for bit
        for m in self.model.modules():
            if hasattr(m, "reset_speculation"):
                m.reset_speculation()
        last = self.prefill(ids)
        for t in range(max_new_tokens):
            if return_logits:
                logs.append(last.float().clone())
            toks[t:t + 1].copy_(self.tok)
            if t + 1 < max_new_tokens:
                last = self.step()
        out = toks.cpu()
        if eos_token_id is not None:
            eos = set(eos_token_id if isinstance(eos_token_id, (list, tuple)) else [eos_token_id])
            for t, v in enumerate(out.tolist()):
                if v in eos:
                    out = out[: t + 1]
                    break
        seq = torch.cat([ids[0].cpu(), out]).view(1, -1)
        return (seq, torch.stack(logs)) if return_logits else seq
