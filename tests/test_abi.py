"""The C ABI library (CPU): it loads without a GPU, exports every entry point
include/t0hip.h declares, the Python binding binds exactly those, and the
host-only entry points validate their arguments."""
import ctypes as C
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    src = open(os.path.join(ROOT, "include", "t0hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(t0h_[a-z0-9_]+)\s*\(", src)))


def test_every_declared_symbol_is_exported(t0hip):
    names = declared()
    assert len(names) >= 25
    L = C.CDLL(t0hip.LIB_PATH)
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    assert sorted(t0hip.SYMBOLS) == names


def test_probe_library_is_separate(t0hip):
    """The benchmark's streaming-read helper lives in its own library, outside the C ABI: it
    exports its two entry points, rejects bad sizes before touching a device, and
    libt0hip.so exports none of them."""
    path = os.path.join(ROOT, "t0-web_amd", "libt0probe.so")
    if not os.path.exists(path):
        pytest.skip("libt0probe.so not built")
    P = C.CDLL(path)
    P.t0p_stream_read.argtypes = [C.c_void_p, C.c_size_t, C.c_void_p, C.c_void_p]
    P.t0p_stream_read_out_words.argtypes = [C.c_size_t]
    P.t0p_stream_read_out_words.restype = C.c_size_t
    assert P.t0p_stream_read_out_words(65536) == 1 and P.t0p_stream_read_out_words(65552) == 2
    assert P.t0p_stream_read(None, 64, None, None) != 0
    assert P.t0p_stream_read(C.c_void_p(16), 24, C.c_void_p(16), None) != 0  # not a multiple of 16
    L = C.CDLL(t0hip.LIB_PATH)
    assert not hasattr(L, "t0p_stream_read")


def test_abi_version_and_no_device(t0hip):
    assert t0hip.lib().t0h_abi_version() == 1
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    with pytest.raises(t0hip.T0HipError) as e:
        t0hip.Engine(0)
    assert e.value.status == "NO_DEVICE"


def test_host_entry_points_validate(t0hip):
    with pytest.raises(t0hip.T0HipError) as e:
        t0hip.synth_model_gguf(t0hip.make_config(embed_dim=100, num_heads=3))
    assert e.value.status == "INVALID_ARG"
    with pytest.raises(t0hip.T0HipError) as e:
        t0hip.export_gguf(b"not a gguf at all", 8)
    assert e.value.status == "GGUF_MAGIC"
    L = t0hip.lib()
    assert L.t0h_gguf_inspect(None, 0, None, None) == -2  # empty input: bad magic
    assert L.t0h_forecast(None, None, 1, 1, 1, None, 0) == -1
    assert L.t0h_model_config(None, None) == -1
    x = np.zeros(64, np.float32)
    out = np.zeros(10, np.uint8)
    assert L.t0h_quantize(8, x.ctypes.data_as(C.c_void_p), 64, out.ctypes.data_as(C.c_void_p), 10) == -1
    # the GEMM entry points refuse base pointers their 16-byte vector accesses cannot use
    P = C.c_void_p
    assert L.t0h_gemm_q(8, P(0x1008), P(0x2000), None, P(0x3000), 1, 64, 64, 0, None) == -1
    assert L.t0h_gemm_q(8, P(0x1000), P(0x2000), P(0x4002), P(0x3000), 1, 64, 64, 0, None) == -1
    assert L.t0h_gemm_f16(8, P(0x1000), P(0x2004), None, P(0x3000), 1, 64, 64, 0, 0, None) == -1
    assert b"16-byte aligned" in L.t0h_last_error()


def test_no_cpu_fallback_in_product():
    """The product package never imports or loads the oracle."""
    pkg = os.path.join(ROOT, "t0-web_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".cpp", ".hip", ".h")):
                text = open(os.path.join(dirpath, f), errors="ignore").read()
                assert "t0ref" not in text and "libt0ref" not in text, f


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus N > 1 (or a multi-rank launch) exits with status 2 and says
    so, before it touches torch or the GPU."""
    import subprocess
    import sys
    for args, env in ((["--gpus", "2"], {}), ([], {"WORLD_SIZE": "2"})):
        r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                           env={**os.environ, **env}, timeout=60)
        assert r.returncode == 2, r.stderr
        assert "one GPU only" in r.stderr and r.stdout == ""
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--steps", "0"], capture_output=True, text=True,
                       timeout=60)
    assert r.returncode == 2 and "at least 1" in r.stderr
