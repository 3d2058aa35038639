"""Bounded corruption loop over the checkpoint readers: the reference's GGUF
header fixture (tests/golden/bonsai2_manifest.gguf) and its bench_matmul_rlx
safetensors weights (tests/golden/bench_matmul_rlx_model.safetensors), each
truncated at a spread of lengths and hit by random single-byte flips, then
opened and walked through the reader's whole API (tensor infos, take_packed,
metadata / reads).  A corrupt file must give an error status, never a crash.
Run by tests/sanitize_run.py under AddressSanitizer and UBSan; also runnable
alone:

    python tests/checkpoint_fuzz.py [--flips N] [--cuts N]
"""
from __future__ import annotations

import argparse
import ctypes as C
import os
import sys
import tempfile
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT / "rlx-models_amd"))
FIXTURE = ROOT / "tests" / "golden" / "bonsai2_manifest.gguf"
ST_FIXTURE = ROOT / "tests" / "golden" / "bench_matmul_rlx_model.safetensors"


def walk(path: str) -> str:
    """Opens `path` and reads everything the API exposes; returns 'ok' or the
    error status of the first failure."""
    import rlxq

    L = rlxq.lib()
    h = C.c_void_p()
    rc = L.rlxq_gguf_open(path.encode(), C.byref(h))
    try:
        if rc != 0:
            L.rlxq_gguf_last_error(h)
            return f"open:{rc}"
        L.rlxq_gguf_version(h)
        L.rlxq_gguf_data_offset(h)
        for i in range(int(L.rlxq_gguf_tensor_count(h))):
            ti = rlxq.GgufTensorInfo()
            if L.rlxq_gguf_tensor_info(h, i, C.byref(ti)) != 0:
                continue
            sch, nd, nb = C.c_int(), C.c_int(), C.c_int64()
            shape = (C.c_int64 * 4)()
            L.rlxq_gguf_take_packed(h, ti.name, C.byref(sch), shape, C.byref(nd), C.byref(nb))
            L.rlxq_gguf_find_tensor(h, ti.name)
            if 0 <= ti.nbytes <= 1 << 16:
                buf = (C.c_uint8 * max(int(ti.nbytes), 1))()
                L.rlxq_gguf_read(h, ti.name, buf, ti.nbytes)
        for i in range(int(L.rlxq_gguf_meta_count(h))):
            ty, el, cnt = C.c_int(), C.c_int(), C.c_uint64()
            if L.rlxq_gguf_meta_type(h, i, C.byref(ty), C.byref(el), C.byref(cnt)) != 0:
                continue
            L.rlxq_gguf_meta_key(h, i)
            for j in list(range(min(cnt.value, 4))) + [cnt.value]:   # the last probe is out of range
                v, f = C.c_int64(), C.c_double()
                s, n = C.c_char_p(), C.c_uint64()
                L.rlxq_gguf_meta_int(h, i, j, C.byref(v))
                L.rlxq_gguf_meta_float(h, i, j, C.byref(f))
                L.rlxq_gguf_meta_str(h, i, j, C.byref(s), C.byref(n))
        return "ok"
    finally:
        L.rlxq_gguf_close(h)


def walk_mlx(path: str) -> str:
    """The same for the safetensors / MLX reader."""
    import rlxq

    L = rlxq.lib()
    h = C.c_void_p()
    rc = L.rlxq_mlx_open(path.encode(), C.byref(h))
    try:
        if rc != 0:
            L.rlxq_mlx_last_error(h)
            return f"open:{rc}"
        b, g, m = C.c_int(), C.c_int(), C.c_int()
        L.rlxq_mlx_quantization(h, C.byref(b), C.byref(g), C.byref(m))
        for i in range(int(L.rlxq_mlx_tensor_count(h))):
            ti = rlxq.MlxTensorInfo()
            if L.rlxq_mlx_tensor_info(h, i, C.byref(ti)) != 0:
                continue
            L.rlxq_mlx_find_tensor(h, ti.name)
            p = rlxq.MlxPacked()
            L.rlxq_mlx_take_packed(h, ti.name, C.byref(p))
            if 0 <= ti.nbytes <= 1 << 21:
                buf = (C.c_uint8 * max(int(ti.nbytes), 1))()
                L.rlxq_mlx_read(h, ti.name, buf, ti.nbytes)
                fl = (C.c_float * max(int(ti.nbytes) // 2, 1))()
                L.rlxq_mlx_read_f32(h, ti.name, fl, max(int(ti.nbytes) // 2, 1))
        return "ok"
    finally:
        L.rlxq_mlx_close(h)


def corrupt(data: bytes, suffix: str, walker, cuts_n: int, flips: int, rng, d: str, flip_end: int = 1 << 20) -> dict:
    import numpy as np

    outcomes: dict[str, int] = {}
    p = os.path.join(d, "f" + suffix)
    cuts = sorted(set(np.linspace(0, len(data), cuts_n, dtype=np.int64).tolist()) | set(range(0, 64)))
    for n in cuts:
        Path(p).write_bytes(data[:n])
        r = walker(p)
        outcomes[r] = outcomes.get(r, 0) + 1
    for _ in range(flips):
        b = bytearray(data)
        pos = int(rng.integers(0, min(len(b), flip_end)))
        b[pos] ^= int(rng.integers(1, 256))
        Path(p).write_bytes(bytes(b))
        r = walker(p)
        outcomes[r] = outcomes.get(r, 0) + 1
    return outcomes


def main(argv=None) -> int:
    import numpy as np

    ap = argparse.ArgumentParser()
    ap.add_argument("--flips", type=int, default=300)
    ap.add_argument("--cuts", type=int, default=300)
    a = ap.parse_args(argv)
    rng = np.random.default_rng(0)
    with tempfile.TemporaryDirectory() as d:
        og = corrupt(FIXTURE.read_bytes(), ".gguf", walk, a.cuts, a.flips, rng, d)
        # only the header of the safetensors file is parsed: flips go there
        st = ST_FIXTURE.read_bytes()
        hdr = 8 + int.from_bytes(st[:8], "little")
        os_ = corrupt(st, ".safetensors", walk_mlx, a.cuts, a.flips, rng, d, flip_end=hdr)
    assert walk(str(FIXTURE)) == "ok" and walk_mlx(str(ST_FIXTURE)) == "ok"
    print(f"checkpoint fuzz: {FIXTURE.name} outcomes {og}; {ST_FIXTURE.name} (flips in its header) outcomes {os_}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
