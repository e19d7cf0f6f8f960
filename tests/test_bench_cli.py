"""bench.py's command-line contract that needs no GPU: it measures one GPU only."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert r.stdout == ""


def test_ceilings_library_exports_its_entry_points():
    """bench.py's measured ceilings come from a separate diagnostic library built beside bench.py."""
    import ctypes
    lib = ctypes.CDLL(os.path.join(ROOT, "bench_ceilings.so"))
    assert hasattr(lib, "fhipc_mfma_fp8_rate") and hasattr(lib, "fhipc_l2_stream")
