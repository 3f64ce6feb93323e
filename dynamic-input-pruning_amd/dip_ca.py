"""Cache-aware DIP (drop-in for the reference's dip_ca.py:58-196, 300-309).

The most frequently selected channels of each layer keep their up/down rows
resident in HBM; each decode token splits its k selected channels into hits
(resident) and misses (streamed from a pinned host copy).  Per token:

    GPU : gate GEMV + SiLU + top-k (bit-exact reference order)
          -> hit/miss assembly through id2slot            (dip_ca_assemble)
    host: read n_hit/n_miss and the miss ids (the one sync the reference also
          has, dip_ca.py:139-146); gather the miss rows into pinned staging
          with native threads
    GPU : hits' up GEMV + h runs while the misses cross PCIe on a side stream
          -> misses' up GEMV + h -> dual-source transposed-down gather

The combined order is [hits in idx order, misses in idx order] with
src 0 = hit / 1 = miss and row = resident slot / staging row, exactly as the
reference builds it (dip_ca.py:158-171).  The hot set is ordered by
key = count * I - id, descending (dip_ca.py:300-308); resident slots follow
ascending channel id (dip_ca.py:107-113).
"""
from __future__ import annotations

import os
import time

import torch
import torch.nn as nn
import torch.nn.functional as F

import _dip_hip as K
from qlinear import GROUP_SIZE, dequantize, int4_linear, int4_linear_t
from dip_stream_predispatch import _transpose_down_to_int4, _use_gather, _use_down  # noqa: F401

_use_ca_fused = True


def hot_ids_from_counts(counts: torch.Tensor) -> torch.Tensor:
    """Channels ordered by (selection count desc, id asc) via the single key
    count * I - id (dip_ca.py:305-307)."""
    cnt = counts.to(torch.long)
    inter = cnt.numel()
    key = cnt * inter - torch.arange(inter, dtype=torch.long, device=cnt.device)
    return key.argsort(descending=True)


class CABuffers:
    """Staging for the streamed misses, sized for the worst case of k misses
    (dip_ca.py:58-70), plus the per-token intermediates."""

    def __init__(self, k, up_in_packed, up_ngroups, down_out, down_ngroups, device):
        self.device = torch.device(device)
        self.k = int(k)
        dev = self.device
        self.gpu_up_qw = torch.empty(k, up_in_packed, dtype=torch.int8, device=dev)
        self.gpu_up_sc = torch.empty(k, up_ngroups, dtype=torch.bfloat16, device=dev)
        self.pin_up_qw = torch.empty(k, up_in_packed, dtype=torch.int8).pin_memory()
        self.pin_up_sc = torch.empty(k, up_ngroups, dtype=torch.bfloat16).pin_memory()
        self.gpu_dn_qw = torch.empty(k, down_out // 2, dtype=torch.int8, device=dev)
        self.gpu_dn_sc = torch.empty(k, down_ngroups, dtype=torch.bfloat16, device=dev)
        self.pin_dn_qw = torch.empty(k, down_out // 2, dtype=torch.int8).pin_memory()
        self.pin_dn_sc = torch.empty(k, down_ngroups, dtype=torch.bfloat16).pin_memory()
        self.copy_stream = torch.cuda.Stream(device=dev)
        self.h = torch.empty(k, dtype=torch.bfloat16, device=dev)
        self._g = {}
        # the per-token read-back: n_hit, n_miss and the miss ids
        self.host_counts = torch.empty(2, dtype=torch.int32).pin_memory()
        self.host_miss = torch.empty(k, dtype=torch.int32).pin_memory()
        # host threads of the native miss gather (default: this process's
        # cores but one, for the thread that queues the copies, at most 15;
        # with the copies on two DMA engines, 15 gathered faster than 8 on a
        # 16-core share)
        self.host_threads = int(os.environ.get(
            "DIP_HOST_THREADS", str(max(1, min(15, len(os.sched_getaffinity(0)) - 1)))))
        # miss rows per gather / copy chunk: each chunk's H2D copy runs while
        # the host gathers the next one
        self.stream_chunk = int(os.environ.get("DIP_STREAM_CHUNK", "2048"))
        # statistics of the last forward (hit rate, bytes streamed)
        self.last_n_hit = 0
        self.last_n_miss = 0
        # when a list: one (bytes, seconds of the gather-and-queue call, ms
        # of copy-stream time of its H2D copies) per streamed miss set; the
        # call then also waits for its copies
        self.transfers = None

    def g(self, inter: int) -> torch.Tensor:
        t = self._g.get(inter)
        if t is None:
            t = self._g[inter] = torch.empty(inter, dtype=torch.bfloat16, device=self.device)
        return t


class CADIPMlp(nn.Module):
    """MLP with a resident channel cache (dip_ca.py:73-196)."""

    # each decode token reads the hit/miss counts back to the host
    graph_capturable = False

    def __init__(self, gate_qw, gate_sc, up_qw, up_sc, down_qw, down_sc, buf,
                 keep_ratio=0.6, cache_frac=0.3, device="cuda:0", down_transposed=False):
        super().__init__()
        self.device = torch.device(device)
        self.keep_ratio = keep_ratio
        self.buf = buf

        self.gate_qw = gate_qw.to(self.device).contiguous()
        self.gate_sc = gate_sc.to(self.device).contiguous()

        # full up / down_t pinned on the host: the source of streamed misses
        self.up_qw = up_qw.cpu().contiguous().pin_memory()
        self.up_sc = up_sc.cpu().contiguous().pin_memory()
        self.inter = up_qw.shape[0]
        if down_transposed:
            dn_t_qw, dn_t_sc = down_qw, down_sc
        else:
            dn_t_qw, dn_t_sc = _transpose_down_to_int4(down_qw.to(self.device),
                                                       down_sc.to(self.device))
        self.down_t_qw = dn_t_qw.cpu().contiguous().pin_memory()
        self.down_t_sc = dn_t_sc.cpu().contiguous().pin_memory()
        self.out_features = self.down_t_qw.shape[1] * 2

        self.k = int(round(self.inter * keep_ratio))
        self.cache_n = int(round(self.inter * cache_frac))

        self.register_buffer("cache_ids", torch.empty(0, dtype=torch.long), persistent=False)
        self.register_buffer("id2slot", torch.full((self.inter,), -1, dtype=torch.long),
                             persistent=False)
        self._res_up_qw = None
        self._res_up_sc = None
        self._res_dn_qw = None
        self._res_dn_sc = None

    def set_cache(self, hot_ids):
        """Make the first cache_n of `hot_ids` resident (dip_ca.py:107-117)."""
        hot_ids = hot_ids[: self.cache_n].cpu().sort().values
        self.cache_ids = hot_ids.to(self.device)
        id2 = torch.full((self.inter,), -1, dtype=torch.long)
        id2[hot_ids] = torch.arange(len(hot_ids))
        self.id2slot = id2.to(self.device)
        self._res_up_qw = self.up_qw[hot_ids].to(self.device)
        self._res_up_sc = self.up_sc[hot_ids].to(self.device)
        self._res_dn_qw = self.down_t_qw[hot_ids].to(self.device)
        self._res_dn_sc = self.down_t_sc[hot_ids].to(self.device)

    def _gate(self, x):
        if x.dim() == 3 and x.shape[1] == 1:
            out = torch.stack([K.int4_gemv(self.gate_qw, self.gate_sc, x[b, 0].to(torch.bfloat16))
                               for b in range(x.shape[0])])
            return out.reshape(x.shape[0], 1, -1)
        return int4_linear(x, self.gate_qw, self.gate_sc)

    def _stream_misses(self, miss_ids_cpu: torch.Tensor, n_miss: int):
        """Pinned row gather of the misses + async H2D on the copy stream
        (dip_ca.py:146-156) as one native call: host threads gather the up
        and down_t rows of buf.stream_chunk misses at a time, and each
        chunk's copies are queued as soon as it is gathered, so they run
        while the next chunk is gathered."""
        b = self.buf
        pins = (b.pin_up_qw, b.pin_up_sc, b.pin_dn_qw, b.pin_dn_sc)
        # No wait on the compute stream: _decode_one synchronised it on the
        # host before the read-back, so the previous layer's reads of the
        # staging rows are done, and the hits' GEMV queued since reads only
        # resident rows.  The copies therefore overlap that GEMV.
        timing = b.transfers is not None
        t0 = time.perf_counter()
        ms = K.host_stream_rows((self.up_qw, self.up_sc, self.down_t_qw, self.down_t_sc),
                                miss_ids_cpu, pins,
                                (b.gpu_up_qw, b.gpu_up_sc, b.gpu_dn_qw, b.gpu_dn_sc),
                                chunk_rows=b.stream_chunk, threads=b.host_threads,
                                stream=b.copy_stream, timing=timing)
        if timing:
            nbytes = n_miss * sum(p.stride(0) * p.element_size() for p in pins)
            b.transfers.append((nbytes, time.perf_counter() - t0, ms))

    def _decode_one(self, xv: torch.Tensor) -> torch.Tensor:
        b = self.buf
        g, idx = K.gate_silu_topk(self.gate_qw, self.gate_sc, xv, self.k, g=b.g(self.inter))
        combined, src, row, miss, counts = K.ca_assemble(self.id2slot, idx)
        # one read-back of the counts and the miss ids (the host sync the
        # reference also has, dip_ca.py:139-146)
        b.host_counts.copy_(counts, non_blocking=True)
        b.host_miss.copy_(miss, non_blocking=True)
        torch.cuda.current_stream(self.device).synchronize()
        n_hit, n_miss = (int(v) for v in b.host_counts)
        b.last_n_hit, b.last_n_miss = n_hit, n_miss
        h = b.h[: self.k]
        if n_hit:  # runs on the GPU while the host gathers the misses
            K.ca_fused_gemv(self._res_up_qw, self._res_up_sc, b.gpu_up_qw, b.gpu_up_sc, xv,
                            src[:n_hit], row[:n_hit], g=g, gid=combined[:n_hit], out=h[:n_hit])
        if n_miss:
            self._stream_misses(b.host_miss[:n_miss], n_miss)
            torch.cuda.current_stream(self.device).wait_stream(b.copy_stream)
            K.ca_fused_gemv(self._res_up_qw, self._res_up_sc, b.gpu_up_qw, b.gpu_up_sc, xv,
                            src[n_hit:], row[n_hit:], g=g, gid=combined[n_hit:], out=h[n_hit:])
        return K.ca_down(self._res_dn_qw, self._res_dn_sc, b.gpu_dn_qw, b.gpu_dn_sc, h, src, row)

    def forward(self, x):
        if x.dim() != 3 or x.shape[1] != 1 or self.keep_ratio >= 0.999 or self._res_up_qw is None:
            return self._dense(x)
        xdt = x.dtype
        ys = [self._decode_one(x[i, 0].to(torch.bfloat16)) for i in range(x.shape[0])]
        return torch.stack(ys).to(xdt).reshape(x.shape[0], 1, -1)

    def _dense(self, x):
        """Prefill route (dip_ca.py:190-196), as StreamingDIPMlp._dense."""
        g = F.silu(self._gate(x))
        u = int4_linear(x, self.up_qw.to(self.device), self.up_sc.to(self.device))
        h = g * u
        return int4_linear_t(h, self.down_t_qw.to(self.device), self.down_t_sc.to(self.device))


def zipf_counts(inter: int, k: int, tokens: int = 128, s: float = 1.1, seed: int = 0):
    """Synthetic stand-in for the selection counts calibrate_cache gathers
    over generate (dip_ca.py:272-309): channel popularity follows Zipf(s)
    over a seeded random ranking of the channels, and each of `tokens`
    synthetic tokens selects k distinct channels, drawn without replacement
    with probability proportional to popularity (Gumbel top-k: the k largest
    log(w) + Gumbel noise are a draw of k items without replacement
    proportional to w).  Returns int64 counts [inter] on the host."""
    if not 0 < k <= inter:
        raise ValueError(f"need 0 < k <= inter, got k={k} inter={inter}")
    gen = torch.Generator().manual_seed(seed)
    rank = torch.randperm(inter, generator=gen)  # rank[c] = popularity rank of channel c
    logw = -s * torch.log1p(rank.double())       # log(1 / (rank + 1)^s)
    u = torch.rand(tokens, inter, generator=gen, dtype=torch.float64).clamp_(1e-300, 1.0)
    keys = logw.unsqueeze(0) - torch.log(-torch.log(u))
    sel = keys.topk(k, dim=1).indices
    return torch.bincount(sel.reshape(-1), minlength=inter).to(torch.long)


def calibrate_cache_from_counts(cas, counts):
    """Apply the reference's hot-set rule (dip_ca.py:300-308) to per-layer
    selection counts gathered by any calibration pass."""
    for c, cnt in zip(cas, counts):
        c.set_cache(hot_ids_from_counts(cnt))


def load_dip_ca(ckpt_dir, gpu_mem_gib=10, cpu_mem_gib=60, keep_ratio=0.6, cache_frac=0.3,
                device="cuda:0"):
    """The reference's cache-aware whole-model loader (dip_ca.py:199-269):
    the causal LM of `ckpt_dir/config.json` with QuantLinear projections and
    every decoder MLP replaced by a CADIPMlp (one CABuffers for all), the
    remaining tensors loaded on `device`.  The caches are empty until
    calibrate_cache (or calibrate_cache_from_counts) fills them; until then
    the modules take their dense route.  Returns (model, tokenizer or None,
    list of the CADIPMlp modules).  gpu_mem_gib / cpu_mem_gib are accepted
    for call compatibility (no offload map: the non-MLP weights are
    resident, the MLP weights live pinned on the host by design)."""
    from pathlib import Path
    from dip_checkpoint import ST_NAME, iter_mlp_layers
    from dip_model import (build_empty_model, load_tensors, load_tokenizer, mlp_module_names,
                           swap_modules)
    ckpt_dir = Path(ckpt_dir)
    model = build_empty_model(ckpt_dir)
    names = mlp_module_names(model)
    if not names:
        raise ValueError(f"{ckpt_dir}: the model has no gate/up/down MLP")
    buf, cas = None, []
    for L in iter_mlp_layers(ckpt_dir, device, names):
        if buf is None:
            inter = L["up_qw"].shape[0]
            out_f = L["down_t_qw"].shape[1] * 2
            buf = CABuffers(int(round(inter * keep_ratio)), L["up_qw"].shape[1],
                            L["up_sc"].shape[1], out_f, out_f // GROUP_SIZE, device)
        cas.append(CADIPMlp(L["gate_qw"], L["gate_sc"], L["up_qw"], L["up_sc"], L["down_t_qw"],
                            L["down_t_sc"], buf, keep_ratio, cache_frac, device,
                            down_transposed=True))
        del L
    swap_modules(model, names, cas)
    load_tensors(model, ckpt_dir / ST_NAME, device, skip_prefixes=names)
    return model, load_tokenizer(ckpt_dir), cas


def calibrate_cache(model, tok, cas, prompt, calib_tokens=30):
    """Count how often each channel is selected over a short greedy
    generation, then make each layer's most selected channels resident
    (dip_ca.py:272-309).  `prompt` is a string (run through the tokenizer's
    chat template, as the reference does) or a token-id tensor [1, P].

    The forward hooks select with the module's own gate + SiLU + top-k
    kernel and count on the GPU, so the pass adds no host synchronisation;
    the hot set follows the reference's (count desc, id asc) order."""
    counts = [torch.zeros(c.inter, dtype=torch.long, device=c.device) for c in cas]

    def make_hook(lid, c):
        def hook(module, inp, out):
            x = inp[0]
            if x.dim() == 3 and x.shape[1] == 1:
                for b in range(x.shape[0]):
                    _, idx = K.gate_silu_topk(c.gate_qw, c.gate_sc, x[b, 0].to(torch.bfloat16),
                                              c.k)
                    counts[lid].index_add_(0, idx.long(),
                                           torch.ones_like(idx, dtype=torch.long))
        return hook

    handles = [c.register_forward_hook(make_hook(lid, c)) for lid, c in enumerate(cas)]
    if isinstance(prompt, str):
        if tok is None:
            raise ValueError("a text prompt needs a tokenizer")
        ids = tok.apply_chat_template([{"role": "user", "content": prompt}],
                                      add_generation_prompt=True, return_tensors="pt")
        if not torch.is_tensor(ids):
            ids = ids["input_ids"]
    else:
        ids = torch.as_tensor(prompt).view(1, -1)
    dev = cas[0].device
    pad = tok.eos_token_id if tok is not None else model.config.eos_token_id
    try:
        with torch.no_grad():
            model.generate(ids.to(dev), max_new_tokens=calib_tokens, do_sample=False,
                           use_cache=True, pad_token_id=pad)
    finally:
        for h in handles:
            h.remove()
    calibrate_cache_from_counts(cas, [c.cpu() for c in counts])
    return counts
