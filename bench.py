"""Benchmark: DIP MLP decode tok/s on the Qwen3-32B-shape 64-layer int4 stack
(keep 0.6) on one MI355X, with achieved HBM GB/s against the 8 TB/s peak.

    python bench.py [--gpus 1] [--steps 256] [--warmup 16] [--shape qwen3-32b]
                    [--keep 0.6] [--cpu-seconds 20] [--no-cpu]

A step is one decode token through all layers (64 layers,
H=5120, I=25600, k=15360, every layer resident in HBM).  Weights are
synthetic N(0, 0.02) draws quantized int4 g128; x_t ~ N(0, 1) bf16, a fresh
vector per token.  One token = one HIP-graph replay of all layers; the timed
region covers exactly `steps` tokens, bracketed by device synchronisation.

Besides the JSON line's `value` (tok/s) it reports:
  roofline      the longest single-kernel stage's algorithmic bytes / its
                average duration (HIP events around each launch, on its
                stream);
  step_*        whole-token bytes / time against the same peak;
  cpu_baseline  the reference's forward run literally with PyTorch CPU ops
                (oracle.torch_cpu_forward) on one layer of the same weights,
                on this host's cores, scaled to tok/s of the full stack.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "dynamic-input-pruning_amd"))

# Kernel arguments in device memory (a HIP runtime option, read when the
# runtime starts, so before torch touches the GPU): the decode graph's four
# launches per layer dispatch slightly faster (2.490 -> 2.471 ms per token on
# the Qwen3-32B stack).  An explicit setting in the environment wins.
os.environ.setdefault("HIP_FORCE_DEV_KERNARG", "1")

HBM_PEAK_GBS = 8000.0
METRIC = "DIP MLP decode tok/s, Qwen3-32B shape int4 k=0.6; achieved HBM GB/s vs peak"


def metric_name(args) -> str:
    """The headline metric's name for its own workload (Qwen3-32B shape,
    keep 0.6, synthetic weights); other workloads name theirs."""
    if args.checkpoint:
        return f"DIP MLP decode tok/s, checkpoint MLPs int4 keep={args.keep:g}; achieved HBM GB/s vs peak"
    if args.shape == "qwen3-32b" and args.keep == 0.6 and not args.layers:
        return METRIC
    shape = {"qwen3-32b": "Qwen3-32B", "qwen3-8b": "Qwen3-8B"}.get(args.shape, args.shape)
    layers = f" {args.layers}-layer" if args.layers else ""
    return f"DIP MLP decode tok/s, {shape} shape{layers} int4 keep={args.keep:g}; achieved HBM GB/s vs peak"


def cpu_baseline(stack, seconds: float):
    """Time the reference's CPU path on layer 0 of the stack (bounded sample)."""
    import numpy as np
    import torch
    sys.path.insert(0, str(ROOT / "oracle"))
    import dip_oracle as O

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    lw = stack.w[0]
    t = {k: v.cpu() for k, v in lw.items()}
    x = torch.randn(stack.hidden, generator=torch.Generator().manual_seed(123)).to(torch.bfloat16)
    args = (t["gate_qw"], t["gate_sc"], t["up_qw"], t["up_sc"], t["down_t_qw"], t["down_t_sc"],
            x, stack.k)
    O.torch_cpu_forward(*args)  # warm-up
    times = []
    t0 = time.perf_counter()
    while True:
        a = time.perf_counter()
        O.torch_cpu_forward(*args)
        times.append(time.perf_counter() - a)
        if len(times) >= 3 and time.perf_counter() - t0 > seconds:
            break
        if len(times) >= 50:
            break
    t_layer = float(np.median(times))
    return {
        "value": 1.0 / (t_layer * stack.layers),
        "unit": "tok/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"reference forward with PyTorch CPU ops (dequantize per call, F.linear, "
                   f"F.silu, top-k, index_select, matmul) on 1 layer of the same "
                   f"H={stack.hidden} I={stack.inter} k={stack.k} weights, median of "
                   f"{len(times)} runs = {t_layer * 1e3:.1f} ms/layer, scaled to "
                   f"{stack.layers} layers"),
    }


def measured_traffic(shape: str, keep: float, stage: str, K):
    """HBM bytes per launch of `stage` from the committed counter summary
    (profiles/hbm_traffic_<shape>_keep<keep>.md: FETCH_SIZE / WRITE_SIZE
    passes scaled against a device copy), or None when there is none for this
    workload or it was measured under other launch tuning."""
    path = ROOT / "profiles" / f"hbm_traffic_{shape}_keep{keep:g}.md"
    if not path.exists():
        return None
    tuning, table = None, {}
    for line in path.read_text().splitlines():
        if line.startswith("tuning:"):
            tuning = {}
            for item in line.split(":", 1)[1].split():
                name, val = item.split("=")
                tuning[name] = int(val)
        elif line.startswith("traffic_bytes_per_launch:"):
            for item in line.split(":", 1)[1].split():
                name, val = item.split("=")
                table[name] = int(val)
    # every knob, by name, as it was when the counters were read
    live = {name: K.get_tuning(name) for name in K.TUNE}
    if tuning != live:
        return None
    return table.get(stage)


def whole_model(args) -> int:
    """Greedy decode of a whole synthetic Qwen3 (int4 attention projections,
    DIP MLPs at --keep, bf16 embedding and lm_head) through DIPDecoder's
    HIP-graph step.  Reports decode-only tok/s (HIP events over `steps`
    graph replays after `warmup`) and tok/s the way the reference's
    gen_utils.benchmark_decode measures it (wall time of a greedy generate of
    64 new tokens, prompt prefill included, mean of 3 runs after a warmup
    run), plus the weight bytes one token reads."""
    import torch
    from dip_model import DIPDecoder, qwen3_config, synthetic_model
    from qlinear import QuantLinear
    dev = torch.device("cuda:0")
    over = {"num_hidden_layers": args.layers} if args.layers else {}
    cfg = qwen3_config(args.shape, **over)
    print(f"[bench] building whole {args.shape} model ({cfg.num_hidden_layers} layers) "
          f"keep={args.keep}", file=sys.stderr, flush=True)
    model, mods = synthetic_model(cfg, args.keep, dev, seed=0)
    plen, gen_new = 32, 64
    dec = DIPDecoder(model, max_len=plen + max(args.warmup + args.steps, gen_new) + 1)
    prompt = torch.randint(0, cfg.vocab_size, (1, plen), generator=torch.Generator().manual_seed(0))
    print("[bench] model built; prefill + warmup", file=sys.stderr, flush=True)
    dec.prefill(prompt)
    for _ in range(args.warmup):
        dec.step()
    torch.cuda.synchronize()
    print("[bench] timing decode steps", file=sys.stderr, flush=True)
    stream = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.steps):
        dec.step()
    e1.record(stream)
    torch.cuda.synchronize()
    ms_step = e0.elapsed_time(e1) / args.steps
    print(f"[bench] {ms_step:.3f} ms per decode step; timing generate", file=sys.stderr,
          flush=True)
    dec.generate(prompt, gen_new)
    runs = []
    for _ in range(3):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        dec.generate(prompt, gen_new)
        torch.cuda.synchronize()
        runs.append(gen_new / (time.perf_counter() - t0))
    proj = sum(m.qweight.numel() + 2 * m.scales.numel() for m in model.modules()
               if isinstance(m, QuantLinear))
    H, I, k = cfg.hidden_size, cfg.intermediate_size, mods[0].k
    row = H // 2 + 2 * (H // 128)
    mlp = len(mods) * (I + 2 * k) * row
    head = model.lm_head.weight.numel() * 2
    out = {
        "metric": "whole-model greedy decode tok/s, synthetic " + args.shape +
                  f" int4, DIP MLPs keep {args.keep}",
        "value": round(1000.0 / ms_step, 2), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 5),
        "higher_is_better": True, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"{args.shape}-shape whole model, batch 1, prompt {plen}, "
                               "HIP-graph decode step", "layers": cfg.num_hidden_layers,
                   "keep": args.keep, "k": k},
        "reference_method_tok_s": round(sum(runs) / len(runs), 2),
        "reference_method": f"greedy generate of {gen_new} tokens incl. {plen}-token prefill, "
                            "wall clock, mean of 3 after 1 warmup",
        "weight_bytes_per_token": {"projections_int4": proj, "dip_mlps": mlp,
                                   "lm_head_bf16": head, "total": proj + mlp + head},
        "weight_gbs": round((proj + mlp + head) / (ms_step * 1e-3) / 1e9, 1),
    }
    print(json.dumps(out), flush=True)
    return 0


def profiler_env():
    """Names of the environment variables rocprofv3 sets for its tool
    library in the profiled process (ROCPROF_OUTPUT_PATH, ROCPROF_STATS, ...):
    non-empty when this process runs under the profiler."""
    return sorted(n for n in os.environ if n.startswith(("ROCPROF_", "ROCPROFILER_")))


def release_cache_aware(*objs):
    """Return everything the cache-aware run holds to the HIP runtime while
    the runtime (and a profiler's tool library, when there is one) is still
    up: the modules' pinned up/down_t (8.6 GB at the Qwen3-32B shape) and the
    staging buffers go back to torch's pinned-host cache when their last
    reference goes, and that cache only frees them with hipHostFree from a
    static destructor at process exit unless it is emptied here."""
    import gc
    import torch
    torch.cuda.synchronize()
    for o in objs:
        if isinstance(o, list):
            o.clear()
    del objs
    gc.collect()
    torch.cuda.empty_cache()
    torch._C._host_emptyCache()
    torch.cuda.synchronize()


def cache_aware(args) -> int:
    """Cache-aware DIP decode (the reference's CADIPMlp, dip_ca.py:127-188)
    on the --shape stack: every layer keeps round(I * cache_frac) channels'
    up/down_t rows resident in HBM, picked by the reference's hot-set key
    (dip_ca.py:300-308) from seeded Zipf(1.1) selection counts over 128
    synthetic tokens (dip_ca.zipf_counts); the full up/down_t live pinned in
    host memory and each token's misses are gathered there by native threads
    and copied over PCIe on a side stream in chunks (a chunk's copy overlaps
    the next chunk's gather, and the hits' up GEMV runs meanwhile).  Every layer reads
    x_t, as in the resident stack.  Prints one JSON line: tok/s (wall clock,
    the per-layer hit/miss read-back included), the mean hit rate, the PCIe
    rate of the miss copies (bytes / the summed copy-stream time of the
    chunks) and the rate of the whole miss stream (gather and copies, from
    the call to the last copy's end)."""
    import numpy as np
    import torch
    from dip_ca import CABuffers, CADIPMlp, calibrate_cache_from_counts, zipf_counts
    from dip_stack import SHAPES, keep_count
    from quantize import quantize_tensor_int4_groupwise

    dev = torch.device("cuda:0")
    shape = dict(SHAPES[args.shape])
    if args.layers:
        shape["layers"] = args.layers
    H, I, L = shape["hidden"], shape["inter"], shape["layers"]
    k = keep_count(I, args.keep)
    print(f"[bench] building cache-aware {args.shape} stack {shape} keep={args.keep} "
          f"cache_frac={args.ca}", file=sys.stderr, flush=True)
    buf = CABuffers(k, H // 2, H // 128, H, H // 128, dev)
    gen = torch.Generator(device=dev).manual_seed(0)
    cas = []
    for layer in range(L):
        w = []
        for _ in range(3):  # gate, up, down_t
            w += quantize_tensor_int4_groupwise(
                torch.randn(I, H, device=dev, generator=gen) * 0.02)
        cas.append(CADIPMlp(*w, buf, args.keep, args.ca, dev, down_transposed=True))
        if (layer + 1) % 16 == 0:
            print(f"[bench] {layer + 1}/{L} layers built", file=sys.stderr, flush=True)
    gen = torch.Generator(device=dev).manual_seed(1)
    n_tok = args.warmup + args.steps
    if args.ca_calib == "stream":
        # anisotropic synthetic hidden states: a fixed direction mu plus
        # iid noise of the same norm, so that some channels are selected
        # far more often than others (as in real decode); the hot set comes
        # from the selections of 64 calibration tokens of the same
        # distribution, disjoint from the timed ones
        import _dip_hip as K
        mu = torch.randn(H, device=dev, generator=gen)

        def draw(n):
            return (mu + torch.randn(n, H, device=dev, generator=gen)).to(torch.bfloat16)

        calib = draw(64)
        counts = []
        for c in cas:
            cnt = torch.zeros(I, dtype=torch.long, device=dev)
            for t in range(calib.shape[0]):
                _, idx = K.gate_silu_topk(c.gate_qw, c.gate_sc, calib[t], c.k)
                cnt.index_add_(0, idx.long(), torch.ones_like(idx, dtype=torch.long))
            counts.append(cnt.cpu())
        xs = draw(n_tok)
        calib_desc = "selections of 64 calibration tokens (fixed direction + noise)"
    else:
        counts = [zipf_counts(I, k, tokens=128, s=1.1, seed=1000 + layer) for layer in range(L)]
        xs = torch.randn(n_tok, H, device=dev, generator=gen).to(torch.bfloat16)
        calib_desc = "Zipf(1.1) selection counts over 128 synthetic tokens (random x: hits = cache_frac)"
    calibrate_cache_from_counts(cas, counts)
    cache_n = cas[0].cache_n
    row = H // 2 + 2 * (H // 128)
    print(f"[bench] caches set: {cache_n} resident channels per layer "
          f"({2 * cache_n * row / 1e6:.1f} MB)", file=sys.stderr, flush=True)

    hits = []

    def token(i):
        x = xs[i].view(1, 1, H)
        with torch.no_grad():
            for c in cas:
                c(x)
                hits.append(buf.last_n_hit)

    for i in range(args.warmup):
        token(i)
    torch.cuda.synchronize()
    hits.clear()
    buf.transfers = []
    w0 = time.perf_counter()
    for i in range(args.warmup, n_tok):
        token(i)
        if (i - args.warmup + 1) % 8 == 0:
            print(f"[bench] {i - args.warmup + 1}/{args.steps} tokens", file=sys.stderr,
                  flush=True)
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    tr = buf.transfers
    buf.transfers = None
    miss_bytes = sum(t[0] for t in tr)
    copy_s = sum(t[2] for t in tr) * 1e-3
    stream_s = sum(t[1] for t in tr)
    ms_step = wall * 1e3 / args.steps
    hit_rate = float(np.mean(hits)) / k
    out = {
        "metric": "cache-aware DIP MLP decode tok/s, Qwen3 shape int4, misses over PCIe",
        "value": round(1000.0 / ms_step, 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": f"{args.shape}-shape {L}-layer cache-aware DIP MLP decode, batch 1, "
                        f"keep {args.keep}, cache_frac {args.ca}, hot set from {calib_desc}",
            "hidden": H, "inter": I, "layers": L, "k": k, "cache_n": cache_n,
            "host_threads": buf.host_threads, "stream_chunk_rows": buf.stream_chunk,
        },
        "hit_rate": round(hit_rate, 4),
        "miss_bytes_per_token": int(miss_bytes / args.steps),
        "pcie_gbs": round(miss_bytes / copy_s / 1e9, 2) if copy_s > 0 else None,
        "copy_ms_per_token": round(copy_s * 1e3 / args.steps, 3),
        # host gather + queued copies, until the last copy ends
        "miss_stream_gbs": round(miss_bytes / stream_s / 1e9, 2) if stream_s > 0 else None,
        "miss_stream_ms_per_token": round(stream_s * 1e3 / args.steps, 3),
    }
    print(json.dumps(out), flush=True)
    release_cache_aware(cas, hits, tr)
    del cas, buf, xs, counts, hits, tr
    release_cache_aware()
    return 0


def read_ceiling(args) -> int:
    """The read bandwidth this GPU gives the decode step's two access
    patterns, swept over bytes in flight, with the probe kernels of
    libdip_probe.so (csrc/probe/dip_probe.hip; loads only, no arithmetic):
      * contiguous: the gate matrix's bytes (67.584 MB) read front to back,
        grid-stride;
      * gather: 15360 sorted random rows of 2560 B out of 25600 (the up/down
        rows at keep 0.6), each row read whole by one 32-lane group;
      * rows: all 25600 rows the same way (the gate's pattern);
    for workgroups of 256 threads in {1, 2, 3, 4, 8} per CU and each
    thread or group holding {1, 2, 4, 8} loads (rows) in flight.  Rotating:
    every launch reads the next of 8 buffers (541 MB in all) or 12 gather
    matrices (472 MB of rows touched), more than the 256 MB memory-side
    cache holds; resident: every launch re-reads the same buffer, which the
    memory-side cache then serves.  Each figure is HIP events around one
    replay of a HIP graph of `--steps` back-to-back launches (the median of
    5), so it includes one launch boundary per launch, as the decode step's
    stage figures do.  One JSON line."""
    import ctypes
    import torch

    lib = ctypes.CDLL(str(ROOT / "dynamic-input-pruning_amd" / "libdip_probe.so"))
    _p, _i64, _i = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    lib.dip_probe_read.argtypes = [_p, ctypes.c_size_t, _i, _i, _p, _p]
    lib.dip_probe_gather.argtypes = [_p, _i64, _i64, _p, _i64, _i, _i, _p, _p]
    lib.dip_probe_read.restype = lib.dip_probe_gather.restype = _i

    dev = torch.device("cuda:0")
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    reps = max(8, args.steps)
    stream = torch.cuda.current_stream(dev)

    def cur():
        return torch.cuda.current_stream(dev).cuda_stream

    def check(st, what):
        if st != 0:
            raise RuntimeError(f"{what} failed with status {st}")

    def timed(fn):
        """us per launch: `reps` back-to-back launches captured in one HIP
        graph (as the decode step runs), the median of 5 replays."""
        s = torch.cuda.Stream(device=dev)
        s.wait_stream(stream)
        with torch.cuda.stream(s):
            fn(0)
        stream.wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for r in range(reps):
                fn(r)
        g.replay()
        torch.cuda.synchronize()
        ts = []
        for _ in range(5):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            g.replay()
            e1.record(stream)
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1) * 1000.0 / reps)
        return sorted(ts)[2]

    wpcs, rings = (1, 2, 3, 4, 8), (1, 2, 4, 8)
    out = {"metric": "HBM read ceiling (probe kernels, loads only)", "unit": "TB/s",
           "reps": reps, "cus": cus, "threads_per_wg": 256}
    nbytes = 67584000
    bufs = [torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1) for _ in range(8)]
    sweep = {}
    for wpc in wpcs:
        for ring in rings:
            us = timed(lambda r: check(lib.dip_probe_read(bufs[r % 8].data_ptr(), nbytes,
                                                          wpc * cus, ring, sink.data_ptr(),
                                                          cur()), "read"))
            sweep[f"wpc{wpc}_ring{ring}"] = {"us": round(us, 2), "TB/s": round(nbytes / us / 1e6, 3)}
            print(f"[ceiling] read 67.6MB rotating wpc={wpc} ring={ring}: {us:.2f} us",
                  file=sys.stderr, flush=True)
    best = min(sweep, key=lambda n: sweep[n]["us"])
    wpc, ring = (int(v) for v in best.replace("wpc", "").split("_ring"))
    us = timed(lambda r: check(lib.dip_probe_read(bufs[0].data_ptr(), nbytes, wpc * cus, ring,
                                                  sink.data_ptr(), cur()), "read"))
    out["read_67.6MB"] = {"rotating": sweep, "best_rotating": best,
                          "resident_at_best": {"us": round(us, 2),
                                               "TB/s": round(nbytes / us / 1e6, 3)}}
    dst = torch.empty_like(bufs[0])
    us = timed(lambda r: dst.copy_(bufs[r % 8]))
    out["d2d_copy_67.6MB"] = {"us": round(us, 2), "TB/s_read_plus_write": round(2 * nbytes / us / 1e6, 3)}
    del bufs, dst
    torch.cuda.empty_cache()

    n, k, rb, nmat = 25600, 15360, 2560, 12
    gen = torch.Generator(device="cpu").manual_seed(5)
    mats, idxs = [], []
    for _ in range(nmat):
        mats.append(torch.ones(n, rb, dtype=torch.uint8, device=dev))
        idxs.append(torch.sort(torch.randperm(n, generator=gen)[:k]).values.to(torch.int32).to(dev))
    sweep = {}
    for wpc in wpcs:
        for ring in rings:
            us = timed(lambda r: check(lib.dip_probe_gather(
                mats[r % nmat].data_ptr(), n, rb, idxs[r % nmat].data_ptr(), k, wpc * cus, ring,
                sink.data_ptr(), cur()), "gather"))
            sweep[f"wpc{wpc}_ring{ring}"] = {"us": round(us, 2), "TB/s": round(k * rb / us / 1e6, 3)}
            print(f"[ceiling] gather rotating wpc={wpc} ring={ring}: {us:.2f} us",
                  file=sys.stderr, flush=True)
    best = min(sweep, key=lambda n_: sweep[n_]["us"])
    wpc, ring = (int(v) for v in best.replace("wpc", "").split("_ring"))
    us = timed(lambda r: check(lib.dip_probe_gather(mats[0].data_ptr(), n, rb, idxs[0].data_ptr(),
                                                    k, wpc * cus, ring, sink.data_ptr(),
                                                    cur()), "gather"))
    out["gather_15360x2560B_of_25600"] = {"rotating": sweep, "best_rotating": best,
                                          "resident_at_best": {"us": round(us, 2),
                                                               "TB/s": round(k * rb / us / 1e6, 3)}}
    # the gate's pattern: every row, whole, one row per 32-lane group
    allrows = torch.arange(n, dtype=torch.int32, device=dev)
    sweep = {}
    for wpc in wpcs:
        for ring in rings:
            us = timed(lambda r: check(lib.dip_probe_gather(
                mats[r % nmat].data_ptr(), n, rb, allrows.data_ptr(), n, wpc * cus, ring,
                sink.data_ptr(), cur()), "rows"))
            sweep[f"wpc{wpc}_ring{ring}"] = {"us": round(us, 2), "TB/s": round(n * rb / us / 1e6, 3)}
            print(f"[ceiling] all rows rotating wpc={wpc} ring={ring}: {us:.2f} us",
                  file=sys.stderr, flush=True)
    best = min(sweep, key=lambda n_: sweep[n_]["us"])
    out["rows_25600x2560B"] = {"rotating": sweep, "best_rotating": best}
    print(json.dumps(out), flush=True)
    return 0


def timeline(args) -> int:
    """One layer's timeline from the timeline build of the library
    (libdip_hip_timeline.so, per-workgroup wall-clock stamps in the decode
    step's four kernels): the stack decodes `steps` tokens from its captured
    graph, then the last layer's records give each kernel's first and last
    workgroup start, the spread of workgroup ends and the gaps between the
    kernels, in microseconds from the gate's first workgroup start, next to
    the layer period (token time / layers).  Prints its own JSON line."""
    if args.keep >= 0.999:
        print("--timeline reads the DIP step's kernels; keep >= 0.999 runs the dense route "
              "(no top-k launch)", file=sys.stderr)
        return 2
    import numpy as np
    lib_path = ROOT / "dynamic-input-pruning_amd" / "libdip_hip_timeline.so"
    if not lib_path.exists():
        print(f"{lib_path} is not built; run __graft_entry__.build()", file=sys.stderr)
        return 2
    os.environ["DIP_HIP_LIB"] = str(lib_path)
    import torch
    import _dip_hip as K
    from dip_stack import SHAPES, DIPStack

    dev = torch.device("cuda:0")
    shape = dict(SHAPES[args.shape])
    if args.layers:
        shape["layers"] = args.layers
    print(f"[bench] timeline build, {args.shape} stack {shape} keep={args.keep}", file=sys.stderr,
          flush=True)
    stack = DIPStack(shape["hidden"], shape["inter"], shape["layers"], args.keep, dev, seed=0)
    gen = torch.Generator(device=dev).manual_seed(7)
    xs = (torch.randn(args.warmup + args.steps, stack.hidden, device=dev, generator=gen)
          .to(torch.bfloat16))
    stack.capture()
    for i in range(args.warmup):
        stack.step(xs[i])
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(args.warmup, args.warmup + args.steps):
        stack.step(xs[i])
    e1.record()
    torch.cuda.synchronize()
    ms_token = e0.elapsed_time(e1) / args.steps
    period = ms_token * 1e3 / stack.layers

    def layer(recs):
        """Per-kernel statistics of one layer's records, in microseconds from
        the gate's first workgroup start."""
        t0 = int(recs["gate"][0].min())
        us = lambda v: (float(v) - t0) * 0.01
        kernels = {}
        for name, (start, end, xcc) in recs.items():
            if len(start) == 0:  # not launched (the in-launch reduce has no reduce kernel)
                continue
            wg_end = np.where(end >= start[:, None], end, 0).max(axis=1)
            done = wg_end > 0  # workgroups whose waves reached the end (not padding tiles)
            ends = wg_end[done]
            kernels[name] = {
                "workgroups": int(len(start)), "finished": int(done.sum()),
                "first_start": us(start.min()), "last_start": us(start.max()),
                "first_end": us(ends.min()), "end_p10": us(np.percentile(ends, 10)),
                "end_p50": us(np.percentile(ends, 50)), "end_p90": us(np.percentile(ends, 90)),
                "last_end": us(ends.max()),
                "end_mean_by_xcc": {int(x): us(ends[xcc[done] == x].mean())
                                    for x in sorted(set(xcc[done].tolist()))},
            }
        return kernels

    # the stamps hold the last layer of the last token: 5 samples, one token
    # replayed before each, and every figure below is the median over them
    samples = []
    for j in range(5):
        stack.step(xs[(args.warmup + j) % len(xs)])
        torch.cuda.synchronize()
        samples.append(layer({name: K.timeline_read(name) for name in K.TIMELINE_KERNELS}))
    med = lambda vals: round(float(np.median(vals)), 2)
    kernels = {}
    for name in samples[0]:
        ks = [smp[name] for smp in samples]
        kernels[name] = {f: (ks[0][f] if f in ("workgroups", "finished") else
                             {x: med([k[f][x] for k in ks if x in k[f]]) for x in ks[0][f]}
                             if f == "end_mean_by_xcc" else med([k[f] for k in ks]))
                         for f in ks[0]}
    order = [n for n in K.TIMELINE_KERNELS if n in kernels]
    gaps = {f"{a}->{b}": med([smp[b]["first_start"] - smp[a]["last_end"] for smp in samples])
            for a, b in zip(order, order[1:])}
    spans = {n: med([smp[n]["last_end"] - smp[n]["first_start"] for smp in samples])
             for n in order}
    span = med([smp[order[-1]]["last_end"] for smp in samples])
    out = {
        "metric": "one decode layer's timeline (per-workgroup wall-clock stamps)",
        "unit": "us", "shape": args.shape, "layers": stack.layers, "keep": args.keep,
        "steps": args.steps, "ms_per_token": round(ms_token, 5), "layer_period_us": round(period, 2),
        "layer_span_us": span,
        # the launch gap to the next layer's gate, with the per-token graph
        # launch and input copy spread over the layers
        "rest_of_period_us": round(period - span, 2),
        "span_us": spans, "gap_us": gaps, "kernels": kernels,
        "note": "timeline build (stamps add a few stores per workgroup); the last layer of the "
                "last token, median of 5 tokens; microseconds from the gate's first workgroup "
                "start",
    }
    print(json.dumps(out))
    return 0


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--shape", default="qwen3-32b")
    ap.add_argument("--layers", type=int, default=None)
    ap.add_argument("--checkpoint", default=None,
                    help="bench the MLP stack of an int4 checkpoint in the reference's format "
                         "(model_int4.safetensors + quant_config.json) instead of synthetic weights")
    ap.add_argument("--keep", type=float, default=0.6)
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-spec", action="store_true",
                    help="run every layer stage by stage (no speculative up rows during the "
                         "top-k); same outputs, five launches per layer instead of four")
    ap.add_argument("--no-gm", action="store_true",
                    help="the down stage reads down_t's [inter, hidden/128] scales instead of "
                         "their group-major copy")
    ap.add_argument("--eager", action="store_true",
                    help="launch every kernel eagerly instead of replaying the captured graph "
                         "(for counter collection, which profiles each dispatch)")
    ap.add_argument("--whole-model", action="store_true",
                    help="instead of the MLP stack, time greedy decode of a whole synthetic "
                         "Qwen3 of --shape (attention, DIP MLPs, lm_head) with the HIP-graph "
                         "decode loop; prints its own JSON line")
    ap.add_argument("--ca", type=float, default=None, metavar="CACHE_FRAC",
                    help="instead of the resident stack, time cache-aware DIP decode with this "
                         "fraction of channels resident (misses streamed from pinned host "
                         "memory over PCIe); prints its own JSON line")
    ap.add_argument("--ca-calib", choices=("zipf", "stream"), default="zipf",
                    help="--ca hot set: seeded Zipf counts with iid random x (hits equal "
                         "cache_frac), or the counted selections of 64 calibration tokens of an "
                         "anisotropic decode stream (fixed direction + noise) that the timed "
                         "tokens also follow")
    ap.add_argument("--ceiling", action="store_true",
                    help="instead of the decode step, sweep the read bandwidth of the step's "
                         "access patterns with the probe kernels of libdip_probe.so; prints its "
                         "own JSON line")
    ap.add_argument("--timeline", action="store_true",
                    help="instead of the bench line, decode with the timeline build of the "
                         "library (libdip_hip_timeline.so) and print one layer's per-kernel "
                         "workgroup start/end times and the gaps between the kernels")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="after the timed run, copy a buffer of this many MiB device to device "
                         "(the reference transfer for scaling HBM byte counters)")
    args = ap.parse_args(argv)

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures the single-GPU DIP decode path; multi-GPU runs are not "
              "part of this build (--gpus must be 1)", file=sys.stderr)
        return 2

    if args.ceiling:
        return read_ceiling(args)
    if args.timeline:
        return timeline(args)
    if args.whole_model:
        return whole_model(args)
    if args.ca is not None:
        prof = profiler_env()
        if prof:
            # checked before any GPU call: a profiled cache-aware run has
            # ended in a segmentation fault at exit (after its result)
            print("bench.py --ca does not run under rocprofv3 (found " + ", ".join(prof[:3]) +
                  "); its copy rates come from the bench's own HIP events", file=sys.stderr)
            return 3
        return cache_aware(args)

    import torch
    import _dip_hip as K
    from dip_stack import SHAPES, DIPStack

    dev = torch.device("cuda:0")
    if args.checkpoint:
        print(f"[bench] loading MLPs of {args.checkpoint} keep={args.keep}", file=sys.stderr,
              flush=True)
        stack = DIPStack.from_checkpoint(args.checkpoint, args.keep, dev, spec=not args.no_spec,
                                         scales_gm=not args.no_gm)
        shape = dict(hidden=stack.hidden, inter=stack.inter, layers=stack.layers)
    else:
        shape = dict(SHAPES[args.shape])
        if args.layers:
            shape["layers"] = args.layers
        print(f"[bench] building {args.shape} stack {shape} keep={args.keep}", file=sys.stderr,
              flush=True)
        stack = DIPStack(shape["hidden"], shape["inter"], shape["layers"], args.keep, dev, seed=0,
                         spec=not args.no_spec, scales_gm=not args.no_gm)
    gen = torch.Generator(device=dev).manual_seed(1)
    n_tok = args.warmup + args.steps
    xs = (torch.randn(n_tok, shape["hidden"], device=dev, generator=gen)).to(torch.bfloat16)
    if args.eager:
        def run(x_t):
            stack.x.copy_(x_t, non_blocking=True)
            stack.run_token()
    else:
        stack.capture()
        print("[bench] graph captured", file=sys.stderr, flush=True)
        run = stack.step

    for i in range(args.warmup):
        run(xs[i])
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    w0 = time.perf_counter()
    e0.record(stream)
    for i in range(args.warmup, n_tok):
        run(xs[i])
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    ms_total = e0.elapsed_time(e1)
    ms_step = ms_total / args.steps
    tok_s = 1000.0 / ms_step
    step_gbs = stack.bytes_per_token / (ms_step * 1e-3) / 1e9
    print(f"[bench] {args.steps} tokens: {ms_step:.4f} ms/token (wall {wall:.3f} s)",
          file=sys.stderr, flush=True)

    if args.copy_mib:
        src = torch.empty(args.copy_mib << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    if args.eager:
        # counter-collection runs: every dispatch above was eager; no graph
        # replays and no CPU baseline follow
        print(json.dumps({"metric": metric_name(args), "value": round(tok_s, 2), "unit": "tok/s",
                          "eager": True, "ms_per_step": round(ms_step, 5)}), flush=True)
        return 0

    # per-stage kernel durations: HIP events around graph replays of each
    # stage's launches (one per layer, back to back)
    stages = stack.stage_times_ms(reps=3)
    H, I, k = stack.hidden, stack.inter, stack.k
    row = H // 2 + 2 * (H // 128)
    stage_bytes = {"gate_silu": I * row, "topk": 2 * I + 4 * k,
                   "up_gather_h": k * row, "down_gather": k * row,
                   # top-k + the up rows of the k selected channels (rows
                   # speculated on but not selected are not counted)
                   "topk_spec_up": 2 * I + 4 * k + k * row}
    # the roofline names one kernel: the longest single-kernel stage (where
    # the down stage is two launches, the partial-sum kernel and its
    # reduction, it is reported in stage_ms only)
    down_launches = stack.down_launches
    single = {name: v for name, v in stages.items()
              if name != "down_gather" or down_launches == 1}
    dom = max(single, key=single.get)
    ach = stage_bytes[dom] / (stages[dom] * 1e-3) / 1e9
    roofline = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(ach / HBM_PEAK_GBS, 4),
                "traffic": None if args.checkpoint else measured_traffic(args.shape, args.keep,
                                                                         dom, K),
                "kernel": dom, "bytes_per_launch": stage_bytes[dom],
                "avg_launch_ms": round(stages[dom], 5)}
    print(f"[bench] stages (ms): {json.dumps({k_: round(v, 5) for k_, v in stages.items()})}",
          file=sys.stderr, flush=True)

    cpu = None
    if not args.no_cpu:
        print("[bench] timing CPU baseline", file=sys.stderr, flush=True)
        cpu = cpu_baseline(stack, args.cpu_seconds)

    out = {
        "metric": metric_name(args),
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic" if not args.checkpoint else "checkpoint weights, synthetic x",
        "config": {
            "workload": (f"{args.shape}-shape" if not args.checkpoint else "checkpoint") +
                        f" {stack.layers}-layer int4 g128 DIP MLP decode, "
                        f"batch 1, keep {args.keep}, weights resident in HBM",
            "hidden": H, "inter": I, "layers": stack.layers, "k": k,
            "weights": ("int4 g128 symmetric, bf16 scales; " +
                        ("N(0,0.02) draws" if not args.checkpoint else "from the checkpoint")),
            "activations": "bf16, fp32 accumulate",
            "route": ("dense: every channel, no top-k (keep >= 0.999, as the reference "
                      "routes it)" if stack.dense else "DIP: gate, top-k, k up and down rows"),
            "speculative_up": not args.no_spec and not stack.dense,
            "down_scales": "row-major" if args.no_gm else "group-major copy",
            "down_reduce": "in the partials' launch (XCD-local)" if down_launches == 1
                           else "separate launch",
            "bytes_per_token": stack.bytes_per_token,
        },
        "step_hbm_gbs": round(step_gbs, 1),
        "step_roofline_frac": round(step_gbs / HBM_PEAK_GBS, 4),
        "stage_ms": {k_: round(v, 5) for k_, v in stages.items()},
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
