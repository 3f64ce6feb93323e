"""The cache-aware module (CADIPMlp, dip_ca.py:73-196) at the Qwen3-32B layer
shape with a Zipf-calibrated cache (keep 0.6, cache_frac 0.3): the resident
set follows the reference's hot-set key (dip_ca.py:300-308, 107-113), the
hit/miss split and y match the oracle's CADIPMlp restatement on the device's
top-k, and each token's streamed misses are the bytes of their rows.

Bars: cache ids and id2slot exact, n_hit exact, y max|err|/max|ref| <= 1e-2
against the fp64 down over the oracle's [hits, misses] rows."""
import numpy as np
import pytest
import torch

import dip_oracle as O
from gpu_util import dev, dev_bf16, host_bf16, rel_err

pytestmark = pytest.mark.gpu

H, I, KEEP, FRAC = 5120, 25600, 0.6, 0.3


@pytest.fixture(scope="module")
def layer():
    print("building a Qwen3-32B-shape layer on the CPU oracle", flush=True)
    return O.make_layer(H, I, seed=4)


def test_ca_module_zipf_cache_matches_oracle(layer):
    from dip_ca import CABuffers, CADIPMlp, calibrate_cache_from_counts, zipf_counts
    L = layer
    d = torch.device("cuda:0")
    k = O.keep_count(I, KEEP)
    buf = CABuffers(k, H // 2, H // 128, H, H // 128, d)
    m = CADIPMlp(dev(L["gate_qw"]), dev_bf16(L["gate_sc"]), dev(L["up_qw"]),
                 dev_bf16(L["up_sc"]), dev(L["down_t_qw"]), dev_bf16(L["down_t_sc"]), buf,
                 KEEP, FRAC, d, down_transposed=True)
    counts = zipf_counts(I, k, tokens=128, s=1.1, seed=9)
    calibrate_cache_from_counts([m], [counts])
    hot, id2slot = O.hot_set(counts.numpy(), m.cache_n)
    assert m.cache_n == round(I * FRAC)
    assert np.array_equal(m.cache_ids.cpu().numpy(), hot)
    assert np.array_equal(m.id2slot.cpu().numpy(), id2slot)

    buf.transfers = []
    misses = []
    for seed in (1, 2):
        x = O.make_x(H, seed=seed)
        print(f"CA decode token seed={seed}", flush=True)
        y = m(dev_bf16(x).reshape(1, 1, -1))
        idx = O.topk_select(host_bf16(buf.g(I)), k)
        ref = O.ca_forward(L["gate_qw"], L["gate_sc"], L["up_qw"], L["up_sc"], L["down_t_qw"],
                           L["down_t_sc"], id2slot, x, k, idx=idx)
        assert buf.last_n_hit == ref["n_hit"] and buf.last_n_miss == k - ref["n_hit"]
        misses.append(k - ref["n_hit"])
        err = rel_err(host_bf16(y.reshape(-1)), ref["y_f64"])
        print(f"  n_hit={ref['n_hit']} of k={k}, y rel err {err:.2e}", flush=True)
        assert err < 1e-2
    torch.cuda.synchronize()
    row = H // 2 + 2 * (H // 128)
    assert [t[0] for t in buf.transfers] == [n * 2 * row for n in misses]
    assert all(t[2] > 0 for t in buf.transfers)
    buf.transfers = None


def test_host_stream_rows_matches_index_select():
    """The native gather + chunked H2D copy puts exactly src[ids] into the
    device rows, for chunk sizes that divide n, do not, and exceed it; rows
    past n are left untouched."""
    import _dip_hip as K
    d = torch.device("cuda:0")
    g = torch.Generator().manual_seed(0)
    rows, n = 5000, 1234
    srcs = [torch.randint(-128, 127, (rows, 2560), dtype=torch.int8, generator=g),
            torch.randn(rows, 40, generator=g).to(torch.bfloat16)]
    ids = torch.randperm(rows, generator=g)[:n].to(torch.int32)
    pins = [torch.empty(n, *s.shape[1:], dtype=s.dtype).pin_memory() for s in srcs]
    for chunk in (617, 500, 4096):
        dsts = [torch.full((n + 3, *s.shape[1:]), 7, dtype=s.dtype, device=d) for s in srcs]
        ms = K.host_stream_rows(srcs, ids, pins, dsts, chunk_rows=chunk, threads=8,
                                timing=(chunk == 500))
        torch.cuda.synchronize()
        for s_, d_ in zip(srcs, dsts):
            assert torch.equal(d_[:n].cpu(), s_[ids.long()]), chunk
            assert bool((d_[n:].cpu() == 7).all())
        assert (ms is None) == (chunk != 500) and (ms is None or ms > 0)
    with pytest.raises(RuntimeError):
        K.host_stream_rows(srcs, torch.tensor([rows], dtype=torch.int32), pins, dsts)


def test_ca_module_chunk_size_does_not_change_y(layer):
    """The chunked miss stream (one chunk, many small chunks, the default)
    gives identical bits: chunking only moves when rows are copied."""
    from dip_ca import CABuffers, CADIPMlp, calibrate_cache_from_counts, zipf_counts
    L = layer
    d = torch.device("cuda:0")
    k = O.keep_count(I, KEEP)
    buf = CABuffers(k, H // 2, H // 128, H, H // 128, d)
    m = CADIPMlp(dev(L["gate_qw"]), dev_bf16(L["gate_sc"]), dev(L["up_qw"]),
                 dev_bf16(L["up_sc"]), dev(L["down_t_qw"]), dev_bf16(L["down_t_sc"]), buf,
                 KEEP, FRAC, d, down_transposed=True)
    calibrate_cache_from_counts([m], [zipf_counts(I, k, tokens=128, seed=10)])
    x = dev_bf16(O.make_x(H, seed=3)).reshape(1, 1, -1)
    ys = []
    for chunk in (k, 333, 2048):
        buf.stream_chunk = chunk
        ys.append(m(x))
    assert torch.equal(ys[0], ys[1]) and torch.equal(ys[0], ys[2])


@pytest.mark.parametrize("case", ["all_hits", "all_misses"])
def test_ca_module_all_hits_and_all_misses(layer, case):
    """The split's extremes: every selected channel resident (no rows
    streamed) and none resident (every row streamed, no hit GEMV)."""
    from dip_ca import CABuffers, CADIPMlp
    L = layer
    d = torch.device("cuda:0")
    k = O.keep_count(I, KEEP)
    x = O.make_x(H, seed=5)
    g = O.silu_bf16(O.gemv_bf16(L["gate_qw"], L["gate_sc"], x))
    idx = O.topk_select(g, k)
    frac = 1.0 if case == "all_hits" else FRAC
    buf = CABuffers(k, H // 2, H // 128, H, H // 128, d)
    m = CADIPMlp(dev(L["gate_qw"]), dev_bf16(L["gate_sc"]), dev(L["up_qw"]),
                 dev_bf16(L["up_sc"]), dev(L["down_t_qw"]), dev_bf16(L["down_t_sc"]), buf,
                 KEEP, frac, d, down_transposed=True)
    if case == "all_hits":
        hot = torch.arange(I)
    else:  # the first cache_n channels the token does not select
        unselected = np.setdiff1d(np.arange(I), idx)
        hot = torch.from_numpy(unselected[: m.cache_n].astype(np.int64))
    m.set_cache(hot)
    print(f"CA {case}: cache_n={m.cache_n}", flush=True)
    y = m(dev_bf16(x).reshape(1, 1, -1))
    idx_dev = O.topk_select(host_bf16(buf.g(I)), k)
    id2slot = m.id2slot.cpu().numpy()
    ref = O.ca_forward(L["gate_qw"], L["gate_sc"], L["up_qw"], L["up_sc"], L["down_t_qw"],
                       L["down_t_sc"], id2slot, x, k, idx=idx_dev)
    assert buf.last_n_hit == ref["n_hit"] == (k if case == "all_hits" else 0)
    assert rel_err(host_bf16(y.reshape(-1)), ref["y_f64"]) < 1e-2


def _bits(t):
    """The tensor's storage as int64 values (an exact checksum of its bits)."""
    return t.view(torch.int16 if t.element_size() == 2 else torch.int8).to(torch.int64)


def test_host_stream_rows_from_two_threads():
    """Two host threads stream rows at once, each on its own stream into its
    own device rows: every call gets exactly src[ids] (the calls take the
    library's second copy stream one at a time), and work queued on each
    caller's stream after its call sees all of that call's rows."""
    import threading
    import _dip_hip as K
    d = torch.device("cuda:0")
    g = torch.Generator().manual_seed(5)
    rows, n = 4000, 1500
    srcs = [torch.randint(-128, 127, (rows, 2560), dtype=torch.int8, generator=g),
            torch.randn(rows, 40, generator=g).to(torch.bfloat16),
            torch.randint(-128, 127, (rows, 2560), dtype=torch.int8, generator=g),
            torch.randn(rows, 40, generator=g).to(torch.bfloat16)]
    jobs = []
    for j in range(2):
        ids = torch.randperm(rows, generator=g)[:n].to(torch.int32)
        pins = [torch.empty(n, *s.shape[1:], dtype=s.dtype).pin_memory() for s in srcs]
        dsts = [torch.full((n, *s.shape[1:]), 3, dtype=s.dtype, device=d) for s in srcs]
        jobs.append((ids, pins, dsts, torch.cuda.Stream(device=d)))
    sums = [None, None]
    errors = []

    def run(j):
        ids, pins, dsts, st = jobs[j]
        try:
            for rep in range(5):
                with torch.cuda.stream(st):
                    K.host_stream_rows(srcs, ids, pins, dsts, chunk_rows=512, threads=4)
                    # queued after the call on the same stream: sees every row
                    sums[j] = [_bits(t).sum() for t in dsts]
                st.synchronize()
        except Exception as e:  # reported below
            errors.append(e)

    ts = [threading.Thread(target=run, args=(j,)) for j in range(2)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors, errors
    torch.cuda.synchronize()
    for j, (ids, pins, dsts, st) in enumerate(jobs):
        for s_, d_, got in zip(srcs, dsts, sums[j]):
            want = s_[ids.long()]
            assert torch.equal(d_.cpu(), want), j
            assert int(got.cpu()) == int(_bits(want).sum()), j
