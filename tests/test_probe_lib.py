"""The bench-only read-probe library (libdip_probe.so, csrc/probe/dip_probe.hip):
it loads apart from the decode library, exports its two entry points,
rejects bad arguments before any launch, and on the GPU runs the gather at
small k (groups past the k-th row load nothing) and every ring depth."""
import ctypes
from pathlib import Path

import pytest

PROBE = Path(__file__).resolve().parent.parent / "dynamic-input-pruning_amd" / "libdip_probe.so"


def _lib():
    if not PROBE.exists():
        pytest.fail(f"{PROBE} is not built (dynamic-input-pruning_amd/build.py builds it)")
    lib = ctypes.CDLL(str(PROBE))
    _p, _i64, _i = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    lib.dip_probe_read.argtypes = [_p, ctypes.c_size_t, _i, _i, _p, _p]
    lib.dip_probe_gather.argtypes = [_p, _i64, _i64, _p, _i64, _i, _i, _p, _p]
    lib.dip_probe_read.restype = lib.dip_probe_gather.restype = _i
    return lib


def _aligned(n=64):
    buf = (ctypes.c_uint8 * (n + 16))()
    addr = ctypes.addressof(buf)
    return buf, addr + (-addr % 16)


def test_probe_library_is_separate_and_exports_its_entry_points():
    lib = _lib()
    assert hasattr(lib, "dip_probe_read") and hasattr(lib, "dip_probe_gather")
    # the decode library no longer carries the probes
    import _dip_hip as K
    assert not hasattr(K.lib, "dip_probe_read")
    assert not hasattr(K.lib, "dip_probe_gather")


def test_probe_argument_rejection_before_launch():
    lib = _lib()
    keep, p = _aligned()
    R, G = lib.dip_probe_read, lib.dip_probe_gather
    assert R(None, 64, 1, 1, p, None) == -1
    assert R(p, 64, 1, 1, None, None) == -1
    assert R(p, 0, 1, 1, p, None) == -2
    assert R(p, 65, 1, 1, p, None) == -2
    assert R(p + 1, 64, 1, 1, p, None) == -3
    assert R(p, 64, 0, 1, p, None) == -6
    assert R(p, 64, 1 << 17, 1, p, None) == -6
    assert R(p, 64, 1, 3, p, None) == -6
    # gather: rows of whole 512-byte segments, at most 8 per row
    assert G(None, 4, 512, p, 1, 1, 1, p, None) == -1
    assert G(p, 4, 512, None, 1, 1, 1, p, None) == -1
    assert G(p, 0, 512, p, 1, 1, 1, p, None) == -2
    assert G(p, 4, 512, p, 0, 1, 1, p, None) == -2
    assert G(p, 4, 500, p, 1, 1, 1, p, None) == -2
    assert G(p, 4, 512 * 9, p, 1, 1, 1, p, None) == -2
    assert G(p, 4, 512, p, 1 << 31, 1, 1, p, None) == -2
    assert G(p + 1, 4, 512, p, 1, 1, 1, p, None) == -3
    assert G(p, 4, 512, p, 1, 0, 1, p, None) == -6
    assert G(p, 4, 512, p, 1, 1, 5, p, None) == -6


@pytest.mark.gpu
def test_probe_gather_small_k_and_every_ring():
    """k far below the number of row groups (16 per CU): the groups without
    a row return before loading an index, so nothing is read past idx."""
    import torch

    lib = _lib()
    dev = torch.device("cuda:0")
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    n, rb = 64, 2560
    rows = torch.ones(n, rb, dtype=torch.uint8, device=dev)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    for k in (1, 3, 17, n):
        # exactly k indices: a read past the end would leave this allocation
        idx = torch.arange(k, dtype=torch.int32, device=dev).flip(0).contiguous()
        for ring in (1, 2, 4, 8):
            for wgs in (1, 2 * cus):
                st = lib.dip_probe_gather(rows.data_ptr(), n, rb, idx.data_ptr(), k, wgs, ring,
                                          sink.data_ptr(), stream)
                assert st == 0, (k, ring, wgs, st)
    buf = torch.ones(1 << 20, dtype=torch.uint8, device=dev)
    for ring in (1, 2, 4, 8):
        assert lib.dip_probe_read(buf.data_ptr(), buf.numel(), 2 * cus, ring, sink.data_ptr(),
                                  stream) == 0
    torch.cuda.synchronize()
    # the fold of all-ones words never equals the sink's magic value
    assert sink.cpu().tolist() == [0, 0, 0, 0]
