"""ctypes face of the C oracle (liboracle.so) -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, as the checker.  The product (librlxq.so and the rlxq package)
never imports it.

Every function here forwards to rlxq_oracle.c, whose header cites the
reference file:line each routine restates.  Arrays are numpy, C-contiguous.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIBPATH = Path(os.environ.get("RLXQ_ORACLE_LIB", HERE / "liboracle.so"))

Q8_0, Q4_0, Q4_1, MLX4, MLX8, INT8_BLOCK, Q4_K, Q6_K = 1, 2, 3, 4, 5, 6, 7, 8
Q5_K, Q3_K, Q2_K, Q8_K = 10, 11, 12, 13
BLOCK_BYTES = {Q8_0: 34, Q4_0: 18, Q4_1: 20, Q4_K: 144, Q6_K: 210, Q5_K: 176, Q3_K: 110, Q2_K: 84, Q8_K: 292}
KQUANTS = (Q4_K, Q6_K, Q5_K, Q3_K, Q2_K, Q8_K)

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIBPATH.exists():
            raise RuntimeError(f"{LIBPATH} missing: run `python rlx-models_amd/build.py`")
        L = C.CDLL(str(LIBPATH))
        P, I64, I = C.c_void_p, C.c_int64, C.c_int
        sig = {
            "orc_f32_to_f16": (C.c_uint16, [C.c_float]),
            "orc_f16_to_f32": (C.c_float, [C.c_uint16]),
            "orc_f32_to_bf16": (C.c_uint16, [C.c_float]),
            "orc_bf16_to_f32": (C.c_float, [C.c_uint16]),
            "orc_f32_to_f16_n": (None, [P, I64, P]),
            "orc_f16_to_f32_n": (None, [P, I64, P]),
            "orc_f32_to_bf16_n": (None, [P, I64, P]),
            "orc_bf16_to_f32_n": (None, [P, I64, P]),
            "orc_block_bytes": (I64, [I]),
            "orc_row_bytes": (I64, [I, I64]),
            "orc_quantize": (I, [I, P, I64, P]),
            "orc_dequantize": (I, [I, P, I64, P]),
            "orc_q4k_scale_min": (None, [P, I, C.POINTER(I), C.POINTER(I)]),
            "orc_q3k_scale": (I, [P, I]),
            "orc_mlx_pack": (I, [P, I64, I64, I, P]),
            "orc_mlx_dequantize": (I, [P, P, P, I64, I64, I, I, P]),
            "orc_matmul_f64": (I, [I, P, P, I64, I64, I64, P]),
            "orc_matmul_refl": (I, [I, P, P, I64, I64, I64, P]),
            "orc_matmul_refl_par": (I, [I, P, P, I64, I64, I64, P, I]),
            "orc_mlx_matmul_f64": (I, [P, P, P, P, I64, I64, I64, I, I, P]),
            "orc_grouped_matmul_f64": (I, [I, P, P, P, I64, I64, I64, I64, P]),
            "orc_topk_softmax": (I, [P, I64, I64, I64, I, P, P]),
            "orc_moe_f64": (I, [I, P, P, P, P, I64, I64, I64, I64, I64, P]),
            "orc_quantize_act_int8": (I, [P, I64, I64, P, P]),
            "orc_quantize_int8_col": (I, [P, I64, I64, P, P]),
            "orc_w8a8_matmul": (I, [P, P, P, P, I64, I64, I64, P]),
            "orc_int8_block_matmul_f64": (I, [P, P, P, P, I64, I64, I64, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _chk(rc: int, what: str) -> None:
    if rc != 0:
        raise ValueError(f"oracle {what} failed: rc={rc}")


# ---- conversions -----------------------------------------------------------
def f32_to_f16_bits(a) -> np.ndarray:
    a = _f32(a).ravel()
    out = np.empty(a.size, np.uint16)
    lib().orc_f32_to_f16_n(_p(a), a.size, _p(out))
    return out


def f16_bits_to_f32(b) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16).ravel()
    out = np.empty(b.size, np.float32)
    lib().orc_f16_to_f32_n(_p(b), b.size, _p(out))
    return out


def f32_to_bf16_bits(a) -> np.ndarray:
    a = _f32(a)
    flat = a.ravel()
    out = np.empty(flat.size, np.uint16)
    lib().orc_f32_to_bf16_n(_p(flat), flat.size, _p(out))
    return out.reshape(a.shape)


def bf16_bits_to_f32(b) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    flat = b.ravel()
    out = np.empty(flat.size, np.float32)
    lib().orc_bf16_to_f32_n(_p(flat), flat.size, _p(out))
    return out.reshape(b.shape)


# ---- GGUF codecs -----------------------------------------------------------
def row_bytes(scheme: int, k: int) -> int:
    return int(lib().orc_row_bytes(scheme, k))


def quantize(scheme: int, w) -> np.ndarray:
    """Quantize an [N, K] float matrix (K % 32 == 0) into packed rows [N, row_bytes]."""
    w = _f32(w)
    n, k = w.shape
    out = np.empty((n, row_bytes(scheme, k)), np.uint8)
    _chk(lib().orc_quantize(scheme, _p(w), w.size, _p(out)), "quantize")
    return out


def dequantize(scheme: int, packed, k: int) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    rb = row_bytes(scheme, k)
    n = packed.size // rb
    out = np.empty((n, k), np.float32)
    _chk(lib().orc_dequantize(scheme, _p(packed), n * k, _p(out)), "dequantize")
    return out


# ---- MLX affine ------------------------------------------------------------
def mlx_pack(codes, bits: int) -> np.ndarray:
    codes = np.ascontiguousarray(codes, dtype=np.uint32)
    rows, cols = codes.shape
    out = np.empty((rows, cols * bits // 32), np.uint32)
    _chk(lib().orc_mlx_pack(_p(codes), rows, cols, bits, _p(out)), "mlx_pack")
    return out


def mlx_dequantize(wq, scales, biases, cols: int, bits: int, group: int) -> np.ndarray:
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    scales, biases = _f32(scales), _f32(biases)
    rows = wq.shape[0]
    out = np.empty((rows, cols), np.float32)
    _chk(lib().orc_mlx_dequantize(_p(wq), _p(scales), _p(biases), rows, cols, bits, group, _p(out)),
         "mlx_dequantize")
    return out


# ---- matmuls ---------------------------------------------------------------
def matmul_f64(scheme: int, x, packed, n: int) -> np.ndarray:
    x = _f32(x)
    m, k = x.shape
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    y = np.empty((m, n), np.float64)
    _chk(lib().orc_matmul_f64(scheme, _p(x), _p(packed), m, k, n, _p(y)), "matmul_f64")
    return y


def matmul_refl(scheme: int, x, packed, n: int, threads: int | None = None) -> np.ndarray:
    x = _f32(x)
    m, k = x.shape
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    y = np.empty((m, n), np.float32)
    if threads is None:
        _chk(lib().orc_matmul_refl(scheme, _p(x), _p(packed), m, k, n, _p(y)), "matmul_refl")
    else:
        _chk(lib().orc_matmul_refl_par(scheme, _p(x), _p(packed), m, k, n, _p(y), threads), "matmul_refl_par")
    return y


def mlx_matmul_f64(x, wq, scales, biases, n: int, bits: int, group: int) -> np.ndarray:
    x = _f32(x)
    m, k = x.shape
    wq = np.ascontiguousarray(wq, dtype=np.uint32)
    scales, biases = _f32(scales), _f32(biases)
    y = np.empty((m, n), np.float64)
    _chk(lib().orc_mlx_matmul_f64(_p(x), _p(wq), _p(scales), _p(biases), m, k, n, bits, group, _p(y)),
         "mlx_matmul_f64")
    return y


def grouped_matmul_f64(scheme: int, x, bank, expert_idx, n: int, num_experts: int) -> np.ndarray:
    x = _f32(x)
    rows, k = x.shape
    bank = np.ascontiguousarray(bank, dtype=np.uint8)
    idx = _f32(expert_idx)
    y = np.empty((rows, n), np.float64)
    _chk(lib().orc_grouped_matmul_f64(scheme, _p(x), _p(bank), _p(idx), rows, k, n, num_experts, _p(y)),
         "grouped_matmul_f64")
    return y


def topk_softmax(logits, k: int, renorm: bool = False):
    logits = _f32(logits)
    rows, e = logits.shape
    ids = np.empty((rows, k), np.int32)
    probs = np.empty((rows, k), np.float32)
    _chk(lib().orc_topk_softmax(_p(logits), rows, e, k, int(renorm), _p(ids), _p(probs)), "topk_softmax")
    return ids, probs


def moe_f64(scheme: int, x, bank, ids, probs, n: int, num_experts: int) -> np.ndarray:
    x = _f32(x)
    rows, k = x.shape
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    probs = _f32(probs)
    topk = ids.shape[1]
    bank = np.ascontiguousarray(bank, dtype=np.uint8)
    y = np.empty((rows, n), np.float64)
    _chk(lib().orc_moe_f64(scheme, _p(x), _p(bank), _p(ids), _p(probs), rows, topk, k, n, num_experts, _p(y)),
         "moe_f64")
    return y


# ---- int8 ------------------------------------------------------------------
def quantize_act_int8(x):
    x = _f32(x)
    rows, cols = x.shape
    q = np.empty((rows, cols), np.int8)
    s = np.empty(rows, np.float32)
    _chk(lib().orc_quantize_act_int8(_p(x), rows, cols, _p(q), _p(s)), "quantize_act_int8")
    return q, s


def quantize_int8_col(w):
    w = _f32(w)
    k, n = w.shape
    q = np.empty((k, n), np.int8)
    s = np.empty(n, np.float32)
    _chk(lib().orc_quantize_int8_col(_p(w), k, n, _p(q), _p(s)), "quantize_int8_col")
    return q, s


def w8a8_matmul(qx, sx, qw, sw) -> np.ndarray:
    qx = np.ascontiguousarray(qx, dtype=np.int8)
    qw = np.ascontiguousarray(qw, dtype=np.int8)
    sx, sw = _f32(sx), _f32(sw)
    m, k = qx.shape
    n = qw.shape[1]
    y = np.empty((m, n), np.float32)
    _chk(lib().orc_w8a8_matmul(_p(qx), _p(sx), _p(qw), _p(sw), m, k, n, _p(y)), "w8a8_matmul")
    return y


def int8_block_matmul_f64(x, wq, scale, zp=None) -> np.ndarray:
    x = _f32(x)
    m, k = x.shape
    wq = np.ascontiguousarray(wq, dtype=np.int8)
    n = wq.shape[1]
    scale = _f32(scale)
    zp = np.zeros(n, np.float32) if zp is None else _f32(zp)
    y = np.empty((m, n), np.float64)
    _chk(lib().orc_int8_block_matmul_f64(_p(x), _p(wq), _p(scale), _p(zp), m, k, n, _p(y)), "int8_block")
    return y


# ---- seeded synthetic weights in the shape of the benchmark configs ---------
def synth_q4_1(rng: np.random.Generator, n: int, k: int) -> np.ndarray:
    """Q4_1 rows with codes ~U{0..15}, d ~U(0.005, 0.05), m ~U(-0.4, 0) (fp16)."""
    nb = n * (k // 32)
    blk = np.empty((nb, 20), np.uint8)
    d = f32_to_f16_bits(rng.uniform(0.005, 0.05, nb).astype(np.float32))
    mn = f32_to_f16_bits(rng.uniform(-0.4, 0.0, nb).astype(np.float32))
    blk[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    blk[:, 2:4] = mn.view(np.uint8).reshape(nb, 2)
    blk[:, 4:20] = rng.integers(0, 256, (nb, 16), dtype=np.uint8)
    return blk.reshape(n, -1)


def synth_q8_0(rng: np.random.Generator, n: int, k: int, lo=0.002, hi=0.02) -> np.ndarray:
    """Q8_0 rows with q ~U{-127..127}, d ~U(lo, hi) (fp16)."""
    nb = n * (k // 32)
    blk = np.empty((nb, 34), np.uint8)
    d = f32_to_f16_bits(rng.uniform(lo, hi, nb).astype(np.float32))
    blk[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    blk[:, 2:34] = rng.integers(-127, 128, (nb, 32), dtype=np.int8).view(np.uint8)
    return blk.reshape(n, -1)


def synth_q4_0(rng: np.random.Generator, n: int, k: int) -> np.ndarray:
    nb = n * (k // 32)
    blk = np.empty((nb, 18), np.uint8)
    d = f32_to_f16_bits(rng.uniform(0.005, 0.05, nb).astype(np.float32))
    blk[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    blk[:, 2:18] = rng.integers(0, 256, (nb, 16), dtype=np.uint8)
    return blk.reshape(n, -1)


def synth_q4_k(rng: np.random.Generator, n: int, k: int) -> np.ndarray:
    """Q4_K rows (K % 256 == 0): codes ~U{0..15}, 6-bit scales and mins
    ~U{0..63} packed as GGML does, d ~U(0.0005, 0.002) and dmin ~U(0.0005,
    0.005) (fp16), so that d*sc spans Q4_1-like step sizes."""
    nb = n * (k // 256)
    blk = np.empty((nb, 144), np.uint8)
    d = f32_to_f16_bits(rng.uniform(0.0005, 0.002, nb).astype(np.float32))
    dm = f32_to_f16_bits(rng.uniform(0.0005, 0.005, nb).astype(np.float32))
    blk[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    blk[:, 2:4] = dm.view(np.uint8).reshape(nb, 2)
    blk[:, 4:16] = q4k_pack_scales(rng.integers(0, 64, (nb, 8)), rng.integers(0, 64, (nb, 8)))
    blk[:, 16:144] = rng.integers(0, 256, (nb, 128), dtype=np.uint8)
    return blk.reshape(n, -1)


def synth_q6_k(rng: np.random.Generator, n: int, k: int) -> np.ndarray:
    """Q6_K rows (K % 256 == 0): random 6-bit codes (ql / qh bytes), int8
    scales ~U{-64..63}, d ~U(0.0002, 0.001) fp16."""
    nb = n * (k // 256)
    blk = np.empty((nb, 210), np.uint8)
    blk[:, 0:192] = rng.integers(0, 256, (nb, 192), dtype=np.uint8)
    blk[:, 192:208] = rng.integers(-64, 64, (nb, 16), dtype=np.int8).view(np.uint8)
    d = f32_to_f16_bits(rng.uniform(0.0002, 0.001, nb).astype(np.float32))
    blk[:, 208:210] = d.view(np.uint8).reshape(nb, 2)
    return blk.reshape(n, -1)


def synth_q5_k(rng: np.random.Generator, n: int, k: int) -> np.ndarray:
    """Q5_K rows (K % 256 == 0): random qh / qs bytes (5-bit codes), 6-bit
    scales and mins ~U{0..63} in the Q4_K packing, d ~U(0.0003, 0.001) and
    dmin ~U(0.0005, 0.005) fp16."""
    nb = n * (k // 256)
    blk = np.empty((nb, 176), np.uint8)
    d = f32_to_f16_bits(rng.uniform(0.0003, 0.001, nb).astype(np.float32))
    dm = f32_to_f16_bits(rng.uniform(0.0005, 0.005, nb).astype(np.float32))
    blk[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    blk[:, 2:4] = dm.view(np.uint8).reshape(nb, 2)
    blk[:, 4:16] = q4k_pack_scales(rng.integers(0, 64, (nb, 8)), rng.integers(0, 64, (nb, 8)))
    blk[:, 16:176] = rng.integers(0, 256, (nb, 160), dtype=np.uint8)
    return blk.reshape(n, -1)


def synth_q3_k(rng: np.random.Generator, n: int, k: int) -> np.ndarray:
    """Q3_K rows (K % 256 == 0): random hmask / qs bytes, sixteen 6-bit
    scales ~U{0..63} in GGML's block_q3_K packing, d ~U(0.0002, 0.001) fp16."""
    nb = n * (k // 256)
    blk = np.empty((nb, 110), np.uint8)
    blk[:, 0:96] = rng.integers(0, 256, (nb, 96), dtype=np.uint8)
    blk[:, 96:108] = q3k_pack_scales(rng.integers(0, 64, (nb, 16)))
    d = f32_to_f16_bits(rng.uniform(0.0002, 0.001, nb).astype(np.float32))
    blk[:, 108:110] = d.view(np.uint8).reshape(nb, 2)
    return blk.reshape(n, -1)


def synth_q2_k(rng: np.random.Generator, n: int, k: int) -> np.ndarray:
    """Q2_K rows (K % 256 == 0): random scale bytes (4-bit scale and min),
    random 2-bit codes, d ~U(0.001, 0.004) and dmin ~U(0.0005, 0.002) fp16."""
    nb = n * (k // 256)
    blk = np.empty((nb, 84), np.uint8)
    blk[:, 0:80] = rng.integers(0, 256, (nb, 80), dtype=np.uint8)
    d = f32_to_f16_bits(rng.uniform(0.001, 0.004, nb).astype(np.float32))
    dm = f32_to_f16_bits(rng.uniform(0.0005, 0.002, nb).astype(np.float32))
    blk[:, 80:82] = d.view(np.uint8).reshape(nb, 2)
    blk[:, 82:84] = dm.view(np.uint8).reshape(nb, 2)
    return blk.reshape(n, -1)


def synth_q8_k(rng: np.random.Generator, n: int, k: int) -> np.ndarray:
    """Q8_K rows (K % 256 == 0): f32 d ~U(0.0002, 0.001), int8 codes
    ~U{-127..127}, and the 16 int16 sums of 16 codes that the format carries."""
    nb = n * (k // 256)
    blk = np.empty((nb, 292), np.uint8)
    blk[:, 0:4] = rng.uniform(0.0002, 0.001, nb).astype(np.float32).view(np.uint8).reshape(nb, 4)
    q = rng.integers(-127, 128, (nb, 256)).astype(np.int8)
    blk[:, 4:260] = q.view(np.uint8)
    blk[:, 260:292] = q.astype(np.int16).reshape(nb, 16, 16).sum(-1).astype(np.int16).view(np.uint8).reshape(nb, 32)
    return blk.reshape(n, -1)


def q3k_pack_scales(sc) -> np.ndarray:
    """The 12 bytes that hold sixteen 6-bit Q3_K scales ([..., 16], 0..63), in
    GGML's block_q3_K packing: byte t < 8 holds the low nibbles of scales t
    (bits 0-3) and t + 8 (bits 4-7); byte 8 + t holds bits 4-5 of scales t,
    t + 4, t + 8, t + 12 at bits 0-1, 2-3, 4-5, 6-7."""
    sc = np.asarray(sc, np.int64)
    out = np.empty(sc.shape[:-1] + (12,), np.uint8)
    out[..., 0:8] = (sc[..., 0:8] & 15) | ((sc[..., 8:16] & 15) << 4)
    hi = sc >> 4
    out[..., 8:12] = hi[..., 0:4] | (hi[..., 4:8] << 2) | (hi[..., 8:12] << 4) | (hi[..., 12:16] << 6)
    return out


def q3k_scale(q12, s: int) -> int:
    q = np.ascontiguousarray(q12, dtype=np.uint8)
    return int(lib().orc_q3k_scale(_p(q), s))


def q4k_pack_scales(sc, mn) -> np.ndarray:
    """The 12 bytes that hold eight 6-bit scales and mins ([..., 8] each), in
    GGML's block_q4_K packing: bytes 0-3 sc[0..3] | (sc[4..7] >> 4) << 6,
    bytes 4-7 mn[0..3] | (mn[4..7] >> 4) << 6, bytes 8-11 (sc[4..7] & 15) |
    (mn[4..7] & 15) << 4."""
    sc = np.asarray(sc, np.int64)
    mn = np.asarray(mn, np.int64)
    out = np.empty(sc.shape[:-1] + (12,), np.uint8)
    out[..., 0:4] = (sc[..., 0:4] & 63) | ((sc[..., 4:8] >> 4) << 6)
    out[..., 4:8] = (mn[..., 0:4] & 63) | ((mn[..., 4:8] >> 4) << 6)
    out[..., 8:12] = (sc[..., 4:8] & 15) | ((mn[..., 4:8] & 15) << 4)
    return out


def q4k_scale_min(q12, s: int) -> tuple[int, int]:
    q = np.ascontiguousarray(q12, dtype=np.uint8)
    sc, mn = C.c_int(), C.c_int()
    lib().orc_q4k_scale_min(_p(q), s, C.byref(sc), C.byref(mn))
    return sc.value, mn.value


def synth(scheme: int, rng: np.random.Generator, n: int, k: int) -> np.ndarray:
    return {Q4_1: synth_q4_1, Q8_0: synth_q8_0, Q4_0: synth_q4_0, Q4_K: synth_q4_k, Q6_K: synth_q6_k,
            Q5_K: synth_q5_k, Q3_K: synth_q3_k, Q2_K: synth_q2_k, Q8_K: synth_q8_k}[scheme](rng, n, k)


# ---- MXFP4 (QuantScheme::MlxMxfp4), in numpy ---------------------------------
# crates/rlx-models-core/src/mxfp4_pack.rs: layout :26-33 (codes [rows, k/2],
# element c in byte c/2, low nibble when c is even; E8M0 exponent bytes
# [rows, k/32], b meaning 2^(b-127)), E2M1 table :56-58, encoder :64-128 and
# :196-250, decoder :263-281 (exp2 with the exponent clamped, :130-135).
MXFP4 = 9
E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0])


def e8m0_value(b) -> np.ndarray:
    """2^(b-127) as the reference decodes it: (b clamped to 0..254) << 7 as
    bf16 bits, so b = 0 is 0.0 and b = 255 is 2^127 (mxfp4_pack.rs:130-135)."""
    e = np.clip(np.asarray(b, np.int64), 0, 254)
    return np.where(e == 0, 0.0, np.ldexp(1.0, (e - 127).astype(np.int64)))


def mxfp4_nibbles(codes, rows: int, k: int) -> np.ndarray:
    c = np.asarray(codes, np.uint8).reshape(rows, k // 2)
    return np.stack([c & 15, c >> 4], axis=-1).reshape(rows, k)


def mxfp4_dequantize(codes, scales, rows: int, k: int) -> np.ndarray:
    """f64 [rows, k]: E2M1(code) * scale; `scales` are E8M0 bytes (uint8) or
    the decoded scales as bf16 bits (uint16)."""
    s = np.asarray(scales).reshape(rows, k // 32)
    sc = e8m0_value(s) if s.dtype == np.uint8 else bf16_bits_to_f32(s).astype(np.float64)
    return E2M1[mxfp4_nibbles(codes, rows, k)] * np.repeat(sc, 32, axis=1)


def e8m0_exponent(amax) -> np.ndarray:
    """Smallest b with 6 * 2^(b-127) >= amax, 127 for a zero, negative or
    non-finite amax (mxfp4_pack.rs:116-128)."""
    a = np.asarray(amax, np.float32).astype(np.float64)
    ok = np.isfinite(a) & (a > 0)
    safe = np.where(ok, a, 1.0)
    e = np.clip(np.ceil(np.log2(safe / 6.0)), -127, 127).astype(np.int64)
    for _ in range(3):
        e = np.where((e < 127) & (np.ldexp(6.0, e) < safe), e + 1, e)
        e = np.where((e > -127) & (np.ldexp(6.0, e - 1) >= safe), e - 1, e)
    return np.where(ok, e + 127, 127).astype(np.uint8)


def e2m1_code(v, scale) -> np.ndarray:
    """Nearest E2M1 code of v / scale, ties to even, sign kept (also for
    -0.0); a non-finite ratio saturates to +-6 (mxfp4_pack.rs:64-112)."""
    v = np.asarray(v, np.float32)
    scale = np.asarray(scale, np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.where(scale > 0, v / np.where(scale > 0, scale, 1), np.float32(0.0)).astype(np.float32)
    a = np.abs(r)
    mag = np.select([a <= 0.25, a < 0.75, a <= 1.25, a < 1.75, a <= 2.5, a < 3.5, a <= 5.0],
                    [0, 1, 2, 3, 4, 5, 6], 7).astype(np.uint8)
    code = np.where(np.signbit(r), mag | 8, mag).astype(np.uint8)
    return np.where(np.isfinite(r), code, np.where(np.signbit(r), 0x0F, 0x07)).astype(np.uint8)


def mxfp4_quantize(w) -> tuple[np.ndarray, np.ndarray]:
    """Row-major f32 [rows, k] -> (codes uint8 [rows, k/2], E8M0 bytes uint8
    [rows, k/32]), the reference encoder (mxfp4_pack.rs:196-250)."""
    w = np.asarray(w, np.float32)
    rows, k = w.shape
    g = w.reshape(rows, k // 32, 32)
    eb = e8m0_exponent(np.max(np.abs(g), axis=2))
    scale = e8m0_value(eb).astype(np.float32)
    nib = e2m1_code(g, scale[:, :, None]).reshape(rows, k)
    codes = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
    return codes, eb


def mxfp4_matmul_f64(x, codes, scales, n: int) -> np.ndarray:
    x = np.asarray(x, np.float64)
    return x @ mxfp4_dequantize(codes, scales, n, x.shape[1]).T


def synth_mxfp4(rng: np.random.Generator, n: int, k: int) -> tuple[np.ndarray, np.ndarray]:
    """MXFP4 rows from N(0, 0.02) weights through the reference encoder."""
    return mxfp4_quantize((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
