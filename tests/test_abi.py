"""C ABI checks that need no GPU: the library loads, exports every entry point
include/dip_hip.h declares, rejects bad arguments before any launch, and its
host-side row gather is correct."""
import ctypes
import re

import numpy as np
import pytest
import torch

import _dip_hip as K


def _declared():
    text = K.HEADER_PATH.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dip_[a-z0-9_]+)\s*\(", text)))


def test_exports_every_declared_symbol():
    names = _declared()
    assert len(names) >= 20
    for n in names:
        assert hasattr(K.lib, n), n
    assert set(names) == set(K._SIGS), set(names) ^ set(K._SIGS)


def test_status_strings():
    assert K.status_string(0) == "ok"
    for code in (-1, -2, -3, -4, -5, -6):
        assert K.status_string(code) not in ("ok", "unknown status")
    # the bindings are written for exactly this ABI version (include/dip_hip.h)
    header = int(re.search(r"#define DIP_VERSION (\d+)", K.HEADER_PATH.read_text()).group(1))
    assert K.lib.dip_version() == header == K.ABI_VERSION
    assert K.lib.dip_topk_max_n() == 65536


def _fake(n=16):
    """An aligned host pointer that is never dereferenced by a rejected call."""
    buf = (ctypes.c_uint8 * (n + 16))()
    addr = ctypes.addressof(buf)
    return buf, addr + (-addr % 16)


def test_argument_rejection_before_launch():
    keep, p = _fake()
    L = K.lib
    # NULL weights
    assert L.dip_int4_gemv(None, p, p, p, 8, 128, 0, None) == -1
    # in_features not a multiple of 128
    assert L.dip_int4_gemv(p, p, p, p, 8, 100, 0, None) == -2
    # misaligned weights
    assert L.dip_int4_gemv(p + 1, p, p, p, 8, 128, 0, None) == -3
    # unsupported width (no instantiation): 384 = 12 chunks
    # (validated by launch dispatch, which runs no kernel for unknown shapes)
    # bad activation
    assert L.dip_int4_gemv(p, p, p, p, 8, 128, 5, None) == -6
    # top-k: n too large, workspace missing/small
    assert L.dip_topk_select(p, p, 1 << 20, 5, p, 1 << 20, None) == -2
    assert L.dip_topk_select(p, p, 100, 5, None, 0, None) == -5
    assert L.dip_topk_select(p, p, 100, 5, p, 16, None) == -5
    # down: workspace too small
    need = L.dip_gather_down_workspace_size(15360, 5120)
    assert need > 0
    assert L.dip_int4_gather_down(p, p, p, None, p, 15360, 5120, 15360, p, need - 1, None) == -5
    # contiguous down with k > rows
    assert L.dip_int4_gather_down(p, p, p, None, p, 10, 5120, 11, p, need, None) == -2
    # mlp: k > inter, missing outputs
    ws = L.dip_mlp_workspace_size(5120, 25600, 15360)
    assert L.dip_mlp_decode(p, p, p, p, p, p, None, p, p, p, p, p, 5120, 25600, 30000, p, ws, p,
                            None) == -2
    assert L.dip_mlp_decode(p, p, p, p, p, p, None, p, p, None, p, p, 5120, 25600, 100, p, ws, p,
                            None) == -1
    assert L.dip_mlp_decode(p, p, p, p, p, p, None, p, p, p, p, p, 5120, 25600, 15360, p, ws - 1,
                            p, None) == -5
    # speculative first half: missing state, k = 0, unsupported width, misaligned state
    tw = L.dip_topk_workspace_size(25600)
    assert L.dip_gate_silu_topk_spec(p, p, p, p, p, p, p, p, 25600, 5120, 100, p, tw, None,
                                     None) == -1
    assert L.dip_gate_silu_topk_spec(p, p, p, p, p, p, p, p, 25600, 5120, 0, p, tw, p,
                                     None) == -2
    assert L.dip_gate_silu_topk_spec(p, p, p, p, p, p, p, p, 25600, 1024, 100, p, tw, p,
                                     None) == -4
    assert L.dip_gate_silu_topk_spec(p, p, p, p, p, p, p, p, 25600, 5120, 100, p, tw, p + 2,
                                     None) == -3
    assert L.dip_gate_silu_topk_spec(p, p, p, p, p, p, p, p, 25600, 5120, 100, p, 8, p,
                                     None) == -5
    # no indices: every row in order, so k may not exceed the rows
    assert L.dip_int4_gather_down_by_channel(p, p, None, p, None, p, None, 10, 5120, 20, p,
                                             need, None) == -2
    # group-major scales: NULL, shapes
    assert L.dip_scales_group_major(None, p, 10, 40, None) == -1
    assert L.dip_scales_group_major(p, p, -1, 40, None) == -2
    assert L.dip_scales_group_major(p, p, 10, 0, None) == -2
    assert L.dip_mlp_state_size() == 16  # speculation key (twice), key band, spare
    assert not hasattr(L, "dip_read_probe")  # the probes live in libdip_probe.so
    assert L.dip_set_tuning(3, 1) == -6  # the removed step-form knob
    assert L.dip_get_tuning(3) == -6
    assert L.dip_get_tuning(4) == 1  # the two-tier gate split: on by default
    assert L.dip_set_tuning(4, 2) == -6
    assert L.dip_set_tuning(4, -1) == -6
    assert L.dip_set_tuning(2, 1025) == -6
    assert L.dip_set_tuning(2, -1) == -6
    assert L.dip_set_tuning(1, 7) == -6
    assert L.dip_get_tuning(0) == 0  # row-dot grids: automatic by default
    assert L.dip_set_tuning(0, 17) == -6
    assert L.dip_set_tuning(0, -1) == -6
    assert L.dip_set_tuning(99, 1) == -6
    assert L.dip_get_tuning(99) == -6
    assert L.dip_dequant_rows(p, p, None, p, 10, 5, 128, 0, None) == -2
    assert L.dip_ca_assemble(None, p, p, p, p, p, p, 10, 5, None) == -1
    # MLP step with the RMSNorm in its gate: unsupported width, aliasing
    assert L.dip_mlp_decode_rmsnorm(p, p, p, p, p, p, None, p, None, p, 1e-6, None, p, p, p, p,
                                    p, 1024, 3072, 100, p, 1 << 20, None, None) == -4
    assert L.dip_mlp_decode_rmsnorm(p, p, p, p, p, p, None, p, None, p, 1e-6, None, p, p, p, p,
                                    p, 5120, 3072, 100, p, 1 << 20, None, None) == -6
    # GEMV with the RMSNorm prologue: unsupported width, aliasing, NULL h
    assert L.dip_int4_gemv_rmsnorm(p, p, p, None, p, 1e-6, None, p, 8, 1024, None) == -4
    assert L.dip_int4_gemv_rmsnorm(p, p, p, None, p, 1e-6, p, p, 8, 5120, None) == -6
    assert L.dip_int4_gemv_rmsnorm(p, p, None, None, p, 1e-6, None, p, 8, 5120, None) == -1
    # transposed prompt GEMM: NULL, output width, zero tokens, workspace
    assert L.dip_int4_gemm_t(None, p, p, p, 4, 128, 64, p, 16, None) == -1
    assert L.dip_int4_gemm_t(p, p, p, p, 4, 100, 64, p, 16, None) == -2
    assert L.dip_int4_gemm_t(p, p, None, None, 0, 128, 64, None, 0, None) == 0
    assert L.dip_int4_gemm_t_workspace_size(0, 5120, 25600) == 0
    # prompt GEMM: NULL weights, width not a multiple of 128, no tokens (no
    # buffers needed), misaligned x
    assert L.dip_int4_gemm(None, p, p, p, 4, 64, 128, None) == -1
    assert L.dip_int4_gemm(p, p, p, p, 4, 64, 100, None) == -2
    assert L.dip_int4_gemm(p, p, None, None, 0, 64, 128, None) == 0
    assert L.dip_int4_gemm(p, p, None, p, 4, 64, 128, None) == -1
    assert L.dip_int4_gemm(p, p, p + 2, p, 4, 64, 128, None) == -3
    # decode steps: NULL / size / head_dim / alignment / grouping / workspace
    assert L.dip_add_rmsnorm(None, None, p, p, 128, 1e-6, None) == -1
    assert L.dip_add_rmsnorm(p, None, p, p, 0, 1e-6, None) == -2
    assert L.dip_add_rmsnorm(p, None, p, p, 8193, 1e-6, None) == -2
    assert L.dip_add_rmsnorm(p, None, p, p, 100, 1e-6, None) == -2
    assert L.dip_add_rmsnorm(p + 2, None, p, p, 128, 1e-6, None) == -3
    assert L.dip_add_rmsnorm(p, None, p, p, 128, -1.0, None) == -6
    assert L.dip_qk_norm_rope_cache(p, p, p, p, p, p, p, p, None, 4, 2, 128, 16, 1e-6,
                                    None) == -1
    assert L.dip_qk_norm_rope_cache(p, p, p, p, p, p, p, p, p, 4, 2, 64, 16, 1e-6, None) == -4
    assert L.dip_qk_norm_rope_cache(p, p, p, p, p, p, p, p, p, 0, 2, 128, 16, 1e-6, None) == -2
    assert L.dip_qk_norm_rope_cache(p + 2, p, p, p, p, p, p, p, p, 4, 2, 128, 16, 1e-6,
                                    None) == -3
    big = 1 << 20
    assert L.dip_decode_attention(p, p, p, p, p, 6, 4, 128, 16, 1.0, p, big, None) == -2
    assert L.dip_decode_attention(p, p, p, p, p, 6, 2, 128, 16, 1.0, p, big, None) == -4
    assert L.dip_decode_attention(p, p, p, p, p, 8, 2, 128, 16, 1.0, p, 16, None) == -5
    assert L.dip_decode_attention(p, p, p, p, p, 8, 2, 96, 16, 1.0, p, big, None) == -4
    assert L.dip_decode_attention_fused_max_len() == 1024
    assert L.dip_decode_attention_fused(p, p, p, p, p, p, p, p, p, 8, 2, 128, 1025, 1e-6, 1.0,
                                        None) == -2
    assert L.dip_decode_attention_fused(p, p, p, p, p, p, p, p, p, 7, 2, 128, 64, 1e-6, 1.0,
                                        None) == -2
    assert L.dip_decode_attention_fused(p, p, p, p, p, p, p, p, None, 8, 2, 128, 64, 1e-6, 1.0,
                                        None) == -1
    del keep


def test_workspace_sizes():
    L = K.lib
    assert L.dip_topk_workspace_size(25600) >= 16
    # down: 8 KB of arrival counters (the in-launch reduce), then one fp32
    # row of `out` per block of 256 selected positions
    need = L.dip_gather_down_workspace_size(15360, 5120)
    assert need == 8192 + 60 * 5120 * 4
    assert L.dip_gather_down_workspace_size(15361, 5120) == 8192 + 61 * 5120 * 4
    assert L.dip_gather_down_workspace_size(1, 128) == 8192 + 128 * 4
    # decode: 512 B of top-k state, the down workspace, h by channel
    assert L.dip_mlp_workspace_size(5120, 25600, 15360) == 512 + need + 2 * 25600
    # attention partials: (m, l, 128 sums) per query head per 32 cache rows
    assert L.dip_decode_attention_workspace_size(64, 128, 300) == 10 * 64 * 130 * 4
    assert L.dip_decode_attention_workspace_size(64, 96, 300) == 0


def test_host_gather_rows():
    rng = np.random.default_rng(0)
    src = torch.from_numpy(rng.integers(-128, 128, size=(300, 2560), dtype=np.int8))
    ids = torch.from_numpy(rng.permutation(300)[:111].astype(np.int32))
    for threads in (1, 3, 8):
        dst = torch.zeros(200, 2560, dtype=torch.int8)
        K.host_gather_rows(src, ids, dst, threads=threads)
        assert torch.equal(dst[:111], src[ids.long()])
        assert torch.all(dst[111:] == 0)
    sc = torch.from_numpy(rng.standard_normal((300, 40)).astype(np.float32)).to(torch.bfloat16)
    dst = torch.zeros(111, 40, dtype=torch.bfloat16)
    K.host_gather_rows(sc, ids, dst, threads=4)
    assert torch.equal(dst, sc[ids.long()])
    bad = torch.tensor([5, 300], dtype=torch.int32)
    with pytest.raises(RuntimeError):
        K.host_gather_rows(src, bad, torch.zeros(2, 2560, dtype=torch.int8))


def test_host_gather_rows_multi_and_pool_reuse():
    """Several matrices in one pass, thread counts above and below the row
    count, and many back-to-back jobs on the persistent pool."""
    rng = np.random.default_rng(1)
    srcs = [torch.from_numpy(rng.integers(-128, 128, size=(400, 2560), dtype=np.int8)),
            torch.from_numpy(rng.standard_normal((400, 40)).astype(np.float32)).to(torch.bfloat16),
            torch.from_numpy(rng.integers(-128, 128, size=(400, 96), dtype=np.int8))]
    for rep in range(50):
        n = int(rng.integers(1, 300))
        ids = torch.from_numpy(rng.integers(0, 400, size=n).astype(np.int32))
        dsts = [torch.zeros(n + 2, *s.shape[1:], dtype=s.dtype) for s in srcs]
        K.host_gather_rows_multi(srcs, ids, dsts, threads=(1, 3, 8, 16)[rep % 4])
        for s, d in zip(srcs, dsts):
            assert torch.equal(d[:n], s[ids.long()])
            assert torch.all(d[n:] == 0)
    with pytest.raises(RuntimeError):
        K.host_gather_rows_multi(srcs, torch.tensor([0, 400], dtype=torch.int32),
                                 [torch.zeros(2, *s.shape[1:], dtype=s.dtype) for s in srcs])
    with pytest.raises(RuntimeError):  # row counts differ
        K.host_gather_rows_multi([srcs[0], srcs[1][:10]], torch.tensor([0], dtype=torch.int32),
                                 [torch.zeros(1, 2560, dtype=torch.int8),
                                  torch.zeros(1, 40, dtype=torch.bfloat16)])


def test_host_gather_pool_under_concurrent_callers():
    """Several host threads calling the gather at once (ctypes releases the
    GIL): the persistent pool runs their jobs one after another and every
    caller gets exactly its own rows."""
    import threading
    rng = np.random.default_rng(2)
    src = torch.from_numpy(rng.integers(-128, 128, size=(500, 640), dtype=np.int8))
    sc = torch.from_numpy(rng.standard_normal((500, 5)).astype(np.float32)).to(torch.bfloat16)
    errors = []

    def worker(seed):
        r = np.random.default_rng(seed)
        try:
            for _ in range(40):
                n = int(r.integers(1, 400))
                ids = torch.from_numpy(r.integers(0, 500, size=n).astype(np.int32))
                d0 = torch.empty(n, 640, dtype=torch.int8)
                d1 = torch.empty(n, 5, dtype=torch.bfloat16)
                K.host_gather_rows_multi([src, sc], ids, [d0, d1], threads=int(r.integers(1, 9)))
                if not (torch.equal(d0, src[ids.long()]) and torch.equal(d1, sc[ids.long()])):
                    errors.append(seed)
                    return
        except Exception as e:  # surfaced below
            errors.append(repr(e))

    threads = [threading.Thread(target=worker, args=(s,)) for s in range(6)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors


@pytest.mark.skipif(torch.cuda.is_available(), reason="copies into host stand-ins: CPU only")
def test_host_stream_rows_gathers_on_the_pool_without_a_device():
    """The miss stream's gather runs on the pool's threads while the calling
    thread waits for each chunk and queues its copies; with no device every
    copy fails, so the call returns HIP's status after the whole gather
    (staging rows exact, destinations never written).  Repeated calls with
    chunk sizes that do and do not divide n reuse the pool."""
    rng = np.random.default_rng(3)
    rows, n = 3000, 1700
    srcs = [torch.from_numpy(rng.integers(-128, 128, size=(rows, 2560), dtype=np.int8)),
            torch.from_numpy(rng.standard_normal((rows, 40)).astype(np.float32)).to(torch.bfloat16)]
    a = ctypes.addressof
    arr = lambda ts: (ctypes.c_void_p * len(ts))(*[t.data_ptr() for t in ts])  # noqa: E731
    rb = (ctypes.c_int64 * 2)(2560, 80)
    for chunk in (500, 1700, 333, 4096):
        ids = torch.from_numpy(rng.integers(0, rows, size=n).astype(np.int32))
        pins = [torch.zeros(n, *s.shape[1:], dtype=s.dtype) for s in srcs]
        dsts = [torch.zeros(n, *s.shape[1:], dtype=s.dtype) for s in srcs]
        a_s, a_p, a_d = arr(srcs), arr(pins), arr(dsts)
        st = K.lib.dip_host_stream_rows(a(a_s), a(a_p), a(a_d), a(rb), 2, ids.data_ptr(), n, rows,
                                        chunk, 8, None, None)
        assert st > 0, st  # a hipError_t from the first copy
        for p, s in zip(pins, srcs):
            assert torch.equal(p, s[ids.long()]), chunk
        assert all(not d.any() for d in dsts)


def test_host_stream_rows_rejects_before_any_copy():
    L = K.lib
    p = ctypes.c_void_p(16)
    arr = (ctypes.c_void_p * 1)(16)
    rb = (ctypes.c_int64 * 1)(64)
    ids_bad = (ctypes.c_int32 * 2)(0, 10)
    a = ctypes.addressof
    # chunk_rows <= 0, then an id past src_rows: both before any HIP call
    assert L.dip_host_stream_rows(a(arr), a(arr), a(arr), a(rb), 1, a(ids_bad), 2, 10, 0, 4, None,
                                  None) == -6
    assert L.dip_host_stream_rows(a(arr), a(arr), a(arr), a(rb), 1, a(ids_bad), 2, 10, 64, 4, None,
                                  None) == -2
    # nothing to stream: OK without touching the device
    assert L.dip_host_stream_rows(a(arr), a(arr), a(arr), a(rb), 1, a(ids_bad), 0, 10, 64, 4, None,
                                  None) == 0
    assert L.dip_host_stream_rows(None, None, None, None, 1, p, 2, 10, 64, 4, None, None) == -1


def test_python_layer_rejects_host_tensors():
    qw = torch.zeros(8, 64, dtype=torch.int8)
    sc = torch.zeros(8, 1, dtype=torch.bfloat16)
    x = torch.zeros(128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="HIP device"):
        K.int4_gemv(qw, sc, x)
    with pytest.raises(RuntimeError, match="multiple of 128"):
        K.int4_gemv(torch.zeros(8, 50, dtype=torch.int8), sc, x)
    with pytest.raises(RuntimeError, match="must be torch.bfloat16"):
        K.int4_gemv(qw, sc.float(), x)


def test_timeline_entry_point():
    """dip_timeline_read: the product build records nothing and says so; the
    timeline build (libdip_hip_timeline.so, the same sources with per-workgroup
    stamps) carries the same ABI and rejects bad arguments before any HIP
    call."""
    buf = np.zeros(286728 // 8, dtype=np.uint64)
    assert ctypes.sizeof(ctypes.c_uint64) * buf.size == 2048 * 8 * 17 + 2048 * 4 + 8
    L = K.lib
    assert L.dip_timeline_read(0, buf.ctypes.data) == -4  # DIP_ERR_UNSUPPORTED
    assert L.dip_timeline_read(0, None) == -1
    assert L.dip_timeline_read(4, buf.ctypes.data) == -6
    path = K.LIB_PATH.parent / "libdip_hip_timeline.so"
    assert path.exists(), "the timeline build is built with the library"
    T = ctypes.CDLL(str(path))
    assert T.dip_version() == K.ABI_VERSION
    for n in _declared():
        assert hasattr(T, n), n
    T.dip_timeline_read.argtypes = [ctypes.c_int, ctypes.c_void_p]
    assert T.dip_timeline_read(1, None) == -1
    assert T.dip_timeline_read(-1, buf.ctypes.data) == -6
