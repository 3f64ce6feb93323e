"""A resident stack of DIP MLP layers decoding one token at a time.

This is the MLP half of the reference's decode loop (64 x StreamingDIPMlp
inside Qwen3DecoderLayer, gen_utils.py:49-93 / dip_stream_predispatch.py:
176-204) without the attention half: every layer's int4 gate/up/down_t stays
in HBM, the per-token intermediates (g, idx, h) and the kernels' workspace are
shared by all layers (they run in stream order), and one token through all
layers can be captured as a single HIP graph.

Synthetic weights follow the benchmark configs: N(0, 0.02) draws quantized
with the reference quantizer rule, drawn and quantized on the GPU.  Down is
quantized directly in the transposed layout [inter, hidden] (same format as
the reference's dequant -> transpose -> requant route, which the tests pin
separately) so building a 64-layer Qwen3-32B stack takes seconds.
"""
from __future__ import annotations

import ctypes

import torch

import _dip_hip as K
from quantize import quantize_tensor_int4_groupwise

SHAPES = {
    "qwen3-32b": dict(hidden=5120, inter=25600, layers=64),
    "qwen3-8b": dict(hidden=4096, inter=12288, layers=36),
}


def keep_count(inter: int, keep_ratio: float) -> int:
    """k = max(1, int(round(I * keep))) (dip_stream_predispatch.py:248)."""
    return max(1, int(round(inter * keep_ratio)))


def bytes_per_layer(hidden: int, inter: int, k: int) -> int:
    """Algorithmic HBM bytes of one decode step of one layer: the gate is read
    in full, up and down_t only on the k selected rows; one row is hidden/2
    packed bytes + hidden/128 bf16 scales."""
    row = hidden // 2 + 2 * (hidden // 128)
    return inter * row + 2 * k * row


class DIPStack:
    def __init__(self, hidden: int, inter: int, layers: int, keep_ratio: float = 0.6,
                 device="cuda:0", seed: int = 0, spec: bool = True, weights=None,
                 scales_gm: bool = True):
        self.hidden, self.inter, self.layers = hidden, inter, layers
        self.keep_ratio = keep_ratio
        # keep >= 0.999: every channel, without a top-k, as the reference
        # routes it (dip_stream_predispatch.py:177-179 -> _dense)
        self.dense = keep_ratio >= 0.999
        self.k = inter if self.dense else keep_count(inter, keep_ratio)
        self.device = torch.device(device)
        dev = self.device
        if weights is not None:  # per layer: gate/up/down_t qweight + scales on `device`
            self.w = [{n: lw[n] for n in ("gate_qw", "gate_sc", "up_qw", "up_sc", "down_t_qw",
                                          "down_t_sc")} for lw in weights]
        else:
            gen = torch.Generator(device=dev).manual_seed(seed)
            self.w = []
            for _ in range(layers):
                lw = {}
                for name in ("gate", "up", "down_t"):
                    q, s = quantize_tensor_int4_groupwise(
                        torch.randn(inter, hidden, device=dev, generator=gen) * 0.02)
                    lw[name + "_qw"], lw[name + "_sc"] = q, s
                self.w.append(lw)
        # the group-major copy of down_t's scales the down stage reads
        # (None: it reads the [inter, hidden/128] scales themselves)
        for lw in self.w:
            lw["down_t_sc_gm"] = K.scales_group_major(lw["down_t_sc"]) if scales_gm else None
        self.x = torch.empty(hidden, dtype=torch.bfloat16, device=dev)
        self.y = [torch.empty(hidden, dtype=torch.bfloat16, device=dev) for _ in range(layers)]
        self.g = torch.empty(inter, dtype=torch.bfloat16, device=dev)
        self.idx = (torch.arange(inter, dtype=torch.int32, device=dev) if self.dense
                    else torch.empty(self.k, dtype=torch.int32, device=dev))
        self.h = torch.empty(self.k, dtype=torch.bfloat16, device=dev)
        self.ws = torch.zeros(K.mlp_workspace_bytes(hidden, inter, self.k), dtype=torch.uint8,
                              device=dev)
        # per-layer speculation state (None: every step runs stage by stage)
        self.spec = spec
        self.state = [K.mlp_state(dev) for _ in range(layers)] if spec else [None] * layers
        self.graph = None

    @classmethod
    def from_checkpoint(cls, ckpt_dir, keep_ratio: float = 0.6, device="cuda:0",
                        spec: bool = True, scales_gm: bool = True):
        """Every MLP of an int4 checkpoint in the reference's format
        (dip_checkpoint), resident on `device`, in layer order."""
        from dip_checkpoint import load_mlp_layers
        layers = load_mlp_layers(ckpt_dir, device)
        inter, hidden = layers[0]["up_qw"].shape[0], layers[0]["up_qw"].shape[1] * 2
        return cls(hidden, inter, len(layers), keep_ratio, device, spec=spec, weights=layers,
                   scales_gm=scales_gm)

    @property
    def down_launches(self) -> int:
        """Launches of the decode step's down stage: 1 when its last tiles
        reduce the partial sums inside the launch (the speculative step's
        down kernel with the group-major scales, hidden a multiple of 2048 up
        to 8192, on a full 256-CU gfx950: the rule of
        dip_int4_gather_down_by_channel), else 2 (partials + reduce)."""
        props = torch.cuda.get_device_properties(self.device)
        xcd_local = ((self.spec or self.dense) and self.w[0]["down_t_sc_gm"] is not None
                     and self.hidden % 2048 == 0 and self.hidden <= 8192
                     and props.gcnArchName.startswith("gfx950")
                     and props.multi_processor_count == 256)
        return 1 if xcd_local else 2

    @property
    def bytes_per_token(self) -> int:
        return self.layers * bytes_per_layer(self.hidden, self.inter, self.k)

    def reset_speculation(self):
        """Zero every layer's speculation state (the next token speculates on
        every channel, as the first token of a new stack does)."""
        for st in self.state:
            if st is not None:
                st.zero_()

    def _dense_layer(self, lw, y, stream):
        """One layer over every channel (keep >= 0.999): g = SiLU(gate x),
        h[c] = bf16(g[c] * bf16(up[c] . x)) for every c (idx = 0..I-1), y =
        down over every row in order (no id list; the group-major scales
        when present); the down workspace is the stack's own."""
        lib = K.lib
        H, I = self.hidden, self.inter
        down_ws = self.ws.data_ptr() + 512
        down_n = (lib.dip_gather_down_workspace_size(I, H) + 255) // 256 * 256
        K._check(lib.dip_int4_gemv(lw["gate_qw"].data_ptr(), lw["gate_sc"].data_ptr(),
                                   self.x.data_ptr(), self.g.data_ptr(), I, H, 1, stream),
                 "dense gate")
        K._check(lib.dip_up_gather_h(lw["up_qw"].data_ptr(), lw["up_sc"].data_ptr(),
                                     self.x.data_ptr(), self.idx.data_ptr(), self.g.data_ptr(),
                                     self.h.data_ptr(), I, H, I, stream), "dense up")
        gm = lw["down_t_sc_gm"]
        K._check(lib.dip_int4_gather_down_by_channel(
            lw["down_t_qw"].data_ptr(), lw["down_t_sc"].data_ptr(),
            None if gm is None else gm.data_ptr(), self.h.data_ptr(), None, y.data_ptr(),
            None, I, H, I, ctypes.c_void_p(down_ws), down_n, stream), "dense down")

    def run_token(self):
        """All layers on self.x, in stream order (one dip_mlp_decode each;
        at keep >= 0.999 the three dense launches)."""
        if self.dense:
            st = torch.cuda.current_stream(self.device).cuda_stream
            for lw, y in zip(self.w, self.y):
                self._dense_layer(lw, y, st)
            return
        for lw, y, st in zip(self.w, self.y, self.state):
            K.mlp_decode(lw["gate_qw"], lw["gate_sc"], lw["up_qw"], lw["up_sc"],
                         lw["down_t_qw"], lw["down_t_sc"], self.x, self.k, y=y, g=self.g,
                         idx=self.idx, h=self.h, ws=self.ws, state=st,
                         down_t_sc_gm=lw["down_t_sc_gm"])

    def capture(self):
        """Capture run_token() as one HIP graph (after an eager warm-up)."""
        s = torch.cuda.Stream(device=self.device)
        s.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(s):
            self.run_token()
        torch.cuda.current_stream(self.device).wait_stream(s)
        torch.cuda.synchronize(self.device)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.run_token()
        torch.cuda.synchronize(self.device)

    def step(self, x_t: torch.Tensor):
        """Decode one token: feed x_t into the captured graph's input buffer
        and replay all layers."""
        self.x.copy_(x_t, non_blocking=True)
        self.graph.replay()

    # -- per-stage timing --------------------------------------------------
    def stage_graphs(self):
        """One HIP graph per kernel stage, each launching that stage for every
        layer back to back (on the intermediates the last token left).  With
        speculation: gate_silu, gate_topk (gate + the top-k / speculative-up
        launch) and down_gather (h by channel); without: gate_silu, gate_topk,
        up_gather_h and down_gather; at keep >= 0.999 (no top-k): gate_silu,
        up_gather_h (every row) and down_gather (every row, h by channel)."""
        lib = K.lib
        H, I, k = self.hidden, self.inter, self.k
        # the decode step's workspace: [0, 512) top-k state | the down
        # workspace (dip_gather_down_workspace_size, 256-byte aligned) | h by
        # channel
        topk_bytes = 512
        ws_ptr = self.ws.data_ptr()
        down_ws = ws_ptr + topk_bytes
        down_n = (lib.dip_gather_down_workspace_size(k, H) + 255) // 256 * 256
        h_full = down_ws + down_n
        x = self.x.data_ptr()

        def gate(st):
            for lw in self.w:
                K._check(lib.dip_int4_gemv(lw["gate_qw"].data_ptr(), lw["gate_sc"].data_ptr(), x,
                                           self.g.data_ptr(), I, H, 1, st), "gate")

        def gate_topk(st):
            for lw, state in zip(self.w, self.state):
                if self.spec:
                    K._check(lib.dip_gate_silu_topk_spec(
                        lw["gate_qw"].data_ptr(), lw["gate_sc"].data_ptr(),
                        lw["up_qw"].data_ptr(), lw["up_sc"].data_ptr(), x, self.g.data_ptr(),
                        self.idx.data_ptr(), h_full, I, H, k, ws_ptr, topk_bytes,
                        state.data_ptr(), st), "gate_topk_spec")
                else:
                    K._check(lib.dip_gate_silu_topk(lw["gate_qw"].data_ptr(),
                                                    lw["gate_sc"].data_ptr(), x,
                                                    self.g.data_ptr(), self.idx.data_ptr(), I, H,
                                                    k, ws_ptr, topk_bytes, st), "gate_topk")

        def up(st):
            for lw in self.w:
                K._check(lib.dip_up_gather_h(lw["up_qw"].data_ptr(), lw["up_sc"].data_ptr(), x,
                                             self.idx.data_ptr(), self.g.data_ptr(),
                                             self.h.data_ptr(), I, H, k, st), "up")

        def down_dense(st):
            for lw, y in zip(self.w, self.y):
                gm = lw["down_t_sc_gm"]
                K._check(lib.dip_int4_gather_down_by_channel(
                    lw["down_t_qw"].data_ptr(), lw["down_t_sc"].data_ptr(),
                    None if gm is None else gm.data_ptr(), self.h.data_ptr(), None,
                    y.data_ptr(), None, I, H, k, ctypes.c_void_p(down_ws), down_n, st),
                    "dense down")

        def down(st):
            for lw, y in zip(self.w, self.y):
                if self.spec:
                    gm = lw["down_t_sc_gm"]
                    K._check(lib.dip_int4_gather_down_by_channel(
                        lw["down_t_qw"].data_ptr(), lw["down_t_sc"].data_ptr(),
                        None if gm is None else gm.data_ptr(), h_full,
                        self.idx.data_ptr(), y.data_ptr(), self.h.data_ptr(), I, H, k,
                        ctypes.c_void_p(down_ws), down_n, st), "down_by_channel")
                else:
                    K._check(lib.dip_int4_gather_down(lw["down_t_qw"].data_ptr(),
                                                      lw["down_t_sc"].data_ptr(),
                                                      self.h.data_ptr(), self.idx.data_ptr(),
                                                      y.data_ptr(), I, H, k,
                                                      ctypes.c_void_p(down_ws), down_n, st),
                             "down")

        if self.dense:  # every channel, no top-k
            stages = [("gate_silu", gate), ("up_gather_h", up), ("down_gather", down_dense)]
        else:
            stages = [("gate_silu", gate), ("gate_topk", gate_topk)]
            if not self.spec:
                stages.append(("up_gather_h", up))
            stages.append(("down_gather", down))
        graphs = {}
        for name, fn in stages:
            s = torch.cuda.Stream(device=self.device)
            s.wait_stream(torch.cuda.current_stream(self.device))
            with torch.cuda.stream(s):
                fn(s.cuda_stream)
            torch.cuda.current_stream(self.device).wait_stream(s)
            torch.cuda.synchronize(self.device)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                fn(torch.cuda.current_stream(self.device).cuda_stream)
            graphs[name] = g
        return graphs

    def stage_times_ms(self, reps: int = 3, samples: int = 5):
        """Average duration of one launch of each kernel stage: each stage's
        graph (one launch per layer, back to back) is replayed `reps` times
        between two HIP events on the replaying stream, time / (layers *
        reps); of `samples` such averages the median is kept, so one
        disturbed sample does not move the figure.  The top-k stage (with
        speculation: the top-k / speculative-up launch) reads the g its gate
        launch wrote, so its time is that of gate + top-k minus that of the
        gate alone."""
        import statistics
        self.run_token()
        torch.cuda.synchronize(self.device)
        graphs = self.stage_graphs()
        stream = torch.cuda.current_stream(self.device)
        out = {}
        for name, g in graphs.items():
            g.replay()
            means = []
            for _ in range(samples):
                e0 = torch.cuda.Event(enable_timing=True)
                e1 = torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                for _ in range(reps):
                    g.replay()
                e1.record(stream)
                torch.cuda.synchronize(self.device)
                means.append(e0.elapsed_time(e1) / (reps * self.layers))
            out[name] = statistics.median(means)
        if self.dense:
            return out
        topk = max(out.pop("gate_topk") - out["gate_silu"], 0.0)
        res = {"gate_silu": out["gate_silu"]}
        if self.spec:
            res["topk_spec_up"] = topk
        else:
            res["topk"] = topk
            res["up_gather_h"] = out["up_gather_h"]
        res["down_gather"] = out["down_gather"]
        return res
