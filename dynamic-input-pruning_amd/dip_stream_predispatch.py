"""Selective DIP MLP with resident int4 weights (drop-in for the reference's
dip_stream_predispatch.py:77-215).

The reference keeps up/down in pinned host memory and, per decode token,
gathers the k selected rows on the CPU and copies them over PCIe before two
gather kernels run.  On MI355X all MLP weights fit in HBM (a 64-layer Qwen3-32B
MLP stack is ~13 GB of 288 GB), so this module keeps gate, up and the
transposed down resident and runs the whole decode step on the GPU:

    dip_mlp_decode:  gate GEMV + SiLU
                  -> one launch: the bit-exact threshold top-k, and meanwhile
                     h = bf16(g * bf16(up . x)) for the channels this layer's
                     previous token ranked highest (then any selected ones
                     they missed)
                  -> transposed-down gather of h[idx] (deterministic
                     two-stage sum)

with no host synchronisation, so consecutive layers (and HIP-graph captures of
them) run back to back.  Constructor arguments, attributes and routing follow
the reference; ``forward`` of a non-decode input (prefill) takes the dense
route of the reference's ``_dense`` (every channel), with the gate and up
projections on the int4 MFMA GEMM for short prompts.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

import _dip_hip as K
from qlinear import GROUP_SIZE, dequantize, int4_linear, int4_linear_t, _unpack_int4
from quantize import pack_int4

# The reference decides these from which kernel .so files it found; here the
# HIP library is mandatory (importing _dip_hip raised otherwise).
_use_gather = True
_use_down = True


def _unpack_int4_rows(qweight):
    """int8 [R, C/2] packed -> int8 [R, C] in [-8, 7]
    (dip_stream_predispatch.py:77-90)."""
    return _unpack_int4(qweight)


def _pack_int4_rows(q):
    """int8 [R, C] in [-8, 7] -> packed int8 [R, C/2]
    (dip_stream_predispatch.py:93-97)."""
    return pack_int4(q)


def _transpose_down_to_int4(down_qw, down_sc):
    """down [out, inter] int4 -> down_t [inter, out/2] int4 + scales
    [inter, out/128] (dip_stream_predispatch.py:100-120): bf16 dequantize,
    transpose, fp32, re-quantize g128 along `out` with the quantizer's rule.
    Device tensors use the HIP transpose kernel; the result is bit-identical
    to the host route."""
    if down_qw.is_cuda:
        return K.transpose_down_int4(down_qw, down_sc)
    w = dequantize(down_qw, down_sc)
    wt = w.t().contiguous().float()
    inter, out_f = wt.shape
    assert out_f % GROUP_SIZE == 0
    wg = wt.reshape(inter, out_f // GROUP_SIZE, GROUP_SIZE)
    scales = (wg.abs().amax(dim=2, keepdim=True) / 7.0).clamp(min=1e-8)
    q = torch.round(wg / scales).clamp(-8, 7).to(torch.int8).reshape(inter, out_f)
    return _pack_int4_rows(q), scales.squeeze(-1).to(torch.bfloat16)


class SharedBuffers:
    """Per-stack scratch shared by every layer (layers run one after the other
    on one stream, as in dip_stream_predispatch.py:123-138).

    The reference holds staging copies of the k selected up/down rows here;
    with resident weights nothing is staged, so this holds the per-token
    intermediates (g, idx, h) and the kernels' workspace instead."""

    def __init__(self, k, up_in_packed, up_ngroups, down_out, down_ngroups, device):
        self.k = int(k)
        self.device = torch.device(device)
        self.hidden = int(up_in_packed) * 2
        self.down_out = int(down_out)
        assert self.hidden == up_ngroups * GROUP_SIZE
        assert self.down_out == down_ngroups * GROUP_SIZE
        self.local_idx = torch.arange(self.k, dtype=torch.int32, device=self.device)
        self.idx = torch.empty(self.k, dtype=torch.int32, device=self.device)
        self.h = torch.empty(self.k, dtype=torch.bfloat16, device=self.device)
        self._g = {}
        self._all = {}
        self._ws = None

    def g(self, inter: int) -> torch.Tensor:
        t = self._g.get(inter)
        if t is None:
            t = self._g[inter] = torch.empty(inter, dtype=torch.bfloat16, device=self.device)
        return t

    def all_rows(self, inter: int):
        """(arange(inter) int32, h [inter]) for the keep >= 0.999 route."""
        t = self._all.get(inter)
        if t is None:
            t = self._all[inter] = (torch.arange(inter, dtype=torch.int32, device=self.device),
                                    torch.empty(inter, dtype=torch.bfloat16, device=self.device))
        return t

    def workspace(self, hidden: int, inter: int, k: int) -> torch.Tensor:
        need = K.mlp_workspace_bytes(hidden, inter, max(k, inter))
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.zeros(need, dtype=torch.uint8, device=self.device)
        return self._ws


class StreamingDIPMlp(nn.Module):
    """DIP MLP for decode (dip_stream_predispatch.py:141-215), all weights
    resident on `device`.

    Args follow the reference; ``down_qw/down_sc`` are in checkpoint layout
    [out, inter/2] and are transposed once here, unless ``down_transposed``
    says they already are [inter, out/2]."""

    def __init__(self, gate_qw, gate_sc, up_qw, up_sc, down_qw, down_sc, shared,
                 keep_ratio=0.6, device="cuda:0", down_transposed=False):
        super().__init__()
        self.keep_ratio = keep_ratio
        self.device = torch.device(device)
        self.buf = shared

        self.gate_qw = gate_qw.to(self.device).contiguous()
        self.gate_sc = gate_sc.to(self.device).contiguous()
        self.up_qw = up_qw.to(self.device).contiguous()
        self.up_sc = up_sc.to(self.device).contiguous()
        self.inter = up_qw.shape[0]
        if down_transposed:
            dn_t_qw, dn_t_sc = down_qw, down_sc
        else:
            dn_t_qw, dn_t_sc = _transpose_down_to_int4(down_qw.to(self.device),
                                                       down_sc.to(self.device))
        self.down_t_qw = dn_t_qw.to(self.device).contiguous()
        self.down_t_sc = dn_t_sc.to(self.device).contiguous()
        # a group-major copy of the same scales (2 bytes per channel and
        # group): the decode step's down tiles read a column group of many
        # channels at once, which this layout keeps in a few cache lines
        self.down_t_sc_gm = K.scales_group_major(self.down_t_sc)
        self.out_features = self.down_t_qw.shape[1] * 2
        self.k = shared.k
        # which channels the next token's up rows are speculated on: it
        # decides which workgroup handles which channel, so it never changes
        # g, idx or h, and y only within fp32 rounding (the grouping of the
        # down sum); reset_speculation() makes the next call repeat a fresh
        # module's bits
        self._spec_state = K.mlp_state(self.device)

    def reset_speculation(self):
        """Forget the speculation key (the next call speculates on every
        channel, as the first call of a new module does)."""
        self._spec_state.zero_()

    def _gate(self, x):
        """gate_proj(x) (dip_stream_predispatch.py:166-174)."""
        if x.dim() == 3 and x.shape[1] == 1:
            out = torch.stack([K.int4_gemv(self.gate_qw, self.gate_sc, x[b, 0].to(torch.bfloat16))
                               for b in range(x.shape[0])])
            return out.reshape(x.shape[0], 1, -1)
        return int4_linear(x, self.gate_qw, self.gate_sc)

    def _decode_one(self, xv: torch.Tensor) -> torch.Tensor:
        b = self.buf
        hidden = self.out_features
        if self.keep_ratio >= 0.999:
            # Reference routes keep >= 0.999 to _dense (:177-179): all rows.
            idx, h = b.all_rows(self.inter)
            g = b.g(self.inter)
            K.int4_gemv(self.gate_qw, self.gate_sc, xv, act=1, out=g)
            K.up_gather_h(self.up_qw, self.up_sc, xv, idx, g, out=h)
            return K.int4_gather_down(self.down_t_qw, self.down_t_sc, h)
        ws = b.workspace(hidden, self.inter, self.k)
        y, _, _, _ = K.mlp_decode(self.gate_qw, self.gate_sc, self.up_qw, self.up_sc,
                                  self.down_t_qw, self.down_t_sc, xv, self.k,
                                  g=b.g(self.inter), idx=b.idx, h=b.h, ws=ws,
                                  state=self._spec_state, down_t_sc_gm=self.down_t_sc_gm)
        return y

    def decode_rmsnorm(self, res, add, norm_w, eps, res_out, x_out):
        """One decode token with the preceding RMSNorm folded in (the whole-
        model decode loop): x_out = RMSNorm(res + add) * norm_w, res_out =
        res + add, returns this module's y for x_out (the same values as
        forward on x_out)."""
        b = self.buf
        if self.keep_ratio >= 0.999 or self.out_features not in K.NORM_GEMV_COLS:
            res_out.copy_(res)
            K.add_rmsnorm(res_out, add, norm_w, x_out, eps)
            return self._decode_one(x_out)
        ws = b.workspace(self.out_features, self.inter, self.k)
        y, _, _, _, _ = K.mlp_decode_rmsnorm(
            self.gate_qw, self.gate_sc, self.up_qw, self.up_sc, self.down_t_qw, self.down_t_sc,
            res, add, norm_w, eps, self.k, res_out=res_out, x_out=x_out, g=b.g(self.inter),
            idx=b.idx, h=b.h, ws=ws, state=self._spec_state, down_t_sc_gm=self.down_t_sc_gm)
        return y

    def forward(self, x):
        if x.dim() != 3 or x.shape[1] != 1:
            return self._dense(x)
        xdt = x.dtype
        ys = [self._decode_one(x[i, 0].to(torch.bfloat16)) for i in range(x.shape[0])]
        return torch.stack(ys).to(xdt).reshape(x.shape[0], 1, -1)

    def _dense(self, x):
        """Prefill route (dip_stream_predispatch.py:206-215): every channel; the
        gate and up projections through int4_linear (the int4 GEMM for short
        prompts), down through its dequantized transpose."""
        g = F.silu(self._gate(x))
        u = int4_linear(x, self.up_qw, self.up_sc)
        h = g * u
        return int4_linear_t(h, self.down_t_qw, self.down_t_sc)

    # Introspection used by tests: the intermediates of the last decode call.
    def last_selection(self):
        return self.buf.idx, self.buf.h, self.buf.g(self.inter)


def load_streaming_dip(ckpt_dir, gpu_mem_gib=10, cpu_mem_gib=60, keep_ratio=0.6,
                       device="cuda:0"):
    """The reference's whole-model loader (dip_stream_predispatch.py:218-289):
    the causal LM of `ckpt_dir/config.json` with QuantLinear projections,
    every decoder MLP replaced by a StreamingDIPMlp (one SharedBuffers for
    all), and the remaining tensors of model_int4.safetensors loaded.
    Returns (model, tokenizer or None, list of the StreamingDIPMlp modules).

    Every tensor is resident on `device` (a whole int4 Qwen3-32B fits one
    MI355X), so the reference's accelerate offload sizes gpu_mem_gib /
    cpu_mem_gib are accepted for call compatibility only."""
    from pathlib import Path
    from dip_checkpoint import ST_NAME, load_streaming_mlps
    from dip_model import (build_empty_model, load_tensors, load_tokenizer, mlp_module_names,
                           swap_modules)
    ckpt_dir = Path(ckpt_dir)
    model = build_empty_model(ckpt_dir)
    names = mlp_module_names(model)
    if not names:
        raise ValueError(f"{ckpt_dir}: the model has no gate/up/down MLP")
    _, sdips, _ = load_streaming_mlps(ckpt_dir, keep_ratio, device, names=names)
    swap_modules(model, names, sdips)
    load_tensors(model, ckpt_dir / ST_NAME, device, skip_prefixes=names)
    return model, load_tokenizer(ckpt_dir), sdips
