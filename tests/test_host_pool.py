"""The host thread pool of the cache-aware miss gather
(dynamic-input-pruning_amd/csrc/dip_host_pool.h) on the CPU.

A program that uses the pool and returns from main at once must exit
cleanly: the pool's destructor, run by the exit handlers, waits for a job in
flight, stops and joins the workers.  tests/host_pool_exit.cpp is built with
ThreadSanitizer and with AddressSanitizer (g++; host code only) and run; any
sanitizer report or a non-zero exit fails.  The library itself is also
loaded in fresh interpreters that gather rows on the pool and exit right
after the call."""
import shutil
import subprocess
import sys
import textwrap
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "dynamic-input-pruning_amd" / "csrc"
DRIVER = Path(__file__).resolve().parent / "host_pool_exit.cpp"
LIB = ROOT / "dynamic-input-pruning_amd" / "libdip_hip.so"


@pytest.mark.parametrize("san", ["thread", "address"])
def test_pool_exits_cleanly_under_sanitizer(tmp_path, san):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    exe = tmp_path / f"pool_{san}"
    cmd = ["g++", "-std=c++17", "-O1", "-g", f"-fsanitize={san}", "-fno-omit-frame-pointer",
           f"-I{CSRC}", str(DRIVER), "-o", str(exe), "-pthread"]
    subprocess.run(cmd, check=True, capture_output=True, text=True, timeout=240)
    for args in (["30", "8"], ["5", "63"], ["1", "2"]):
        p = subprocess.run([str(exe), *args], capture_output=True, text=True, timeout=120)
        assert p.returncode == 0, (args, p.returncode, p.stderr[-2000:])
        assert "Sanitizer" not in p.stderr, p.stderr[-2000:]
        assert "bad 0" in p.stdout


def test_library_process_exits_right_after_a_pool_call():
    if not LIB.exists():
        pytest.skip("libdip_hip.so not built")
    code = textwrap.dedent(f"""
        import ctypes, numpy as np
        lib = ctypes.CDLL({str(LIB)!r})
        f = lib.dip_host_gather_rows
        f.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int64] * 3 + [ctypes.c_int]
        src = np.arange(4096 * 256, dtype=np.uint8).reshape(4096, 256)
        ids = np.random.default_rng(0).integers(0, 4096, size=2048).astype(np.int32)
        dst = np.zeros((2048, 256), np.uint8)
        st = f(src.ctypes.data, ids.ctypes.data, dst.ctypes.data, 2048, 256, 4096, 16)
        assert st == 0 and np.array_equal(dst, src[ids])
    """)
    for _ in range(5):
        p = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True,
                           timeout=120)
        assert p.returncode == 0, p.stderr[-2000:]
