"""The C ABI library loads and exports every symbol include/rlxq.h declares, and
host-side argument checks answer without a GPU."""
import ctypes as C
import subprocess

import pytest

import rlxq


def test_library_exports_every_declared_symbol():
    L = rlxq.lib()
    declared = rlxq.declared_symbols()
    assert "rlxq_dequant_matmul" in declared and "rlxq_dm_matmul" in declared
    missing = [s for s in declared if not hasattr(L, s)]
    assert not missing, missing


def test_exports_nothing_else():
    out = subprocess.run(["nm", "-D", "--defined-only", str(rlxq.LIBPATH)], capture_output=True, text=True,
                         check=True).stdout
    names = {line.split()[-1] for line in out.splitlines() if line.strip()}
    assert names == set(rlxq.declared_symbols())


def test_strerror_and_version():
    assert rlxq.strerror(0) == "ok"
    assert rlxq.strerror(rlxq.E_SHAPE) == "bad shape"
    assert rlxq.lib().rlxq_version().decode().startswith("rlxq ")


def test_row_bytes():
    rb = rlxq.lib().rlxq_row_bytes
    assert rb(rlxq.GGUF_Q4_1, 4096) == 2560
    assert rb(rlxq.GGUF_Q8_0, 2048) == 2176
    assert rb(rlxq.GGUF_Q4_0, 64) == 36
    assert rb(rlxq.GGUF_Q4_1, 33) == -1
    assert rb(99, 64) == -1


def test_null_context_is_rejected():
    L = rlxq.lib()
    assert L.rlxq_dequant_matmul(None, 3, 32, None, 0, None, None, None, 0, 1, 32, 1, None, 0, None) == rlxq.E_NULL
    assert L.rlxq_destroy(None) == rlxq.E_NULL
    assert L.rlxq_dm_matmul(None, None, 0, None, 0, 0, 0, 0, 3, None) == rlxq.E_NULL
    assert L.rlxq_init(0, None) == rlxq.E_NULL


def test_init_without_gfx950_fails_cleanly():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    h = C.c_void_p()
    rc = rlxq.lib().rlxq_init(0, C.byref(h))
    assert rc in (rlxq.E_DEVICE, rlxq.E_HIP) and not h.value


EXAMPLE = rlxq.PKG / "lib" / "examples" / "decode_gemv"


def test_plain_c_caller_links_and_runs():
    """examples/decode_gemv.c: the ABI from plain C (no Python, no torch).
    Without a gfx950 device it must stop cleanly with status 77."""
    import torch

    assert EXAMPLE.exists(), "build the package first (python rlx-models_amd/build.py)"
    if torch.cuda.is_available():
        pytest.skip("a GPU is present: tests/test_gemv_gpu.py runs it for real")
    r = subprocess.run([str(EXAMPLE)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 77, r.stdout + r.stderr
