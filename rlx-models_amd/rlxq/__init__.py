"""Python binding of librlxq (include/rlxq.h) for tests, smoke and bench.

The product is the C ABI; this module only forwards device pointers of torch
tensors (torch is plumbing for HBM allocations and streams here).  Loading
fails loudly when librlxq.so has not been built: there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

PKG = Path(__file__).resolve().parent.parent
LIBPATH = Path(os.environ.get("RLXQ_LIB", PKG / "lib" / "librlxq.so"))
HEADER = PKG.parent / "include" / "rlxq.h"

GGUF_Q8_0, GGUF_Q4_0, GGUF_Q4_1, MLX_AFFINE4, MLX_AFFINE8, INT8_BLOCK, GGUF_Q4_K, GGUF_Q6_K = 1, 2, 3, 4, 5, 6, 7, 8
MLX_MXFP4 = 9
GGUF_Q5_K, GGUF_Q3_K, GGUF_Q2_K, GGUF_Q8_K = 10, 11, 12, 13
F32, BF16, U8 = 0, 1, 2
MOE_EXPAND, MOE_COMBINE, MOE_EXPAND_SWIGLU = 0, 1, 2
OK = 0
PROBE_MFMA, PROBE_READ, PROBE_READ4, PROBE_TILE20 = 0, 1, 2, 3
E_NULL, E_SHAPE, E_SCHEME, E_ALIGN, E_DTYPE, E_HIP, E_NOMEM, E_INDEX, E_NOKERNEL, E_DEVICE = range(-1, -11, -1)
E_IO, E_FORMAT, E_NOTFOUND, E_TAKEN, E_SCRATCH = range(-11, -16, -1)
NOALLOC_SCRATCH_BYTES = 64 << 20   # RLXQ_NOALLOC_SCRATCH_BYTES

_lib = None


class GgufTensorInfo(C.Structure):
    """rlxq_gguf_tensor."""
    _fields_ = [("name", C.c_char_p), ("ggml_type", C.c_int32), ("n_dims", C.c_int32),
                ("dims", C.c_int64 * 4), ("offset", C.c_uint64), ("nbytes", C.c_int64), ("scheme", C.c_int32)]


class MlxTensorInfo(C.Structure):
    """rlxq_mlx_tensor."""
    _fields_ = [("name", C.c_char_p), ("dtype", C.c_int32), ("n_dims", C.c_int32), ("shape", C.c_int64 * 8),
                ("nbytes", C.c_int64), ("file", C.c_char_p), ("offset", C.c_uint64)]


class MlxPacked(C.Structure):
    """rlxq_mlx_packed."""
    _fields_ = [("scheme", C.c_int32), ("bits", C.c_int32), ("group_size", C.c_int32),
                ("out_features", C.c_int64), ("in_features", C.c_int64), ("codes", C.c_char_p),
                ("scales", C.c_char_p), ("biases", C.c_char_p), ("codes_nbytes", C.c_int64),
                ("scales_nbytes", C.c_int64), ("biases_nbytes", C.c_int64), ("slab_dtype", C.c_int32)]


ST_DTYPES = {1: "BOOL", 2: "U8", 3: "I8", 4: "U16", 5: "I16", 6: "F16", 7: "BF16", 8: "U32", 9: "I32", 10: "F32",
             11: "U64", 12: "I64", 13: "F64", 14: "F8_E4M3", 15: "F8_E5M2"}
MLX_MODE_NONE, MLX_MODE_AFFINE, MLX_MODE_MXFP4 = 0, 1, 2


class RlxqError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"rlxq status {status}: {msg}")
        self.status = status


def lib() -> C.CDLL:
    """Loads librlxq.so (raises if it is missing)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIBPATH.exists():
        raise RuntimeError(f"{LIBPATH} is missing: build it with `python rlx-models_amd/build.py`")
    L = C.CDLL(str(LIBPATH))
    P, I, I64, S = C.c_void_p, C.c_int, C.c_int64, C.c_size_t
    sig = {
        "rlxq_init": (I, [I, C.POINTER(P)]),
        "rlxq_destroy": (I, [P]),
        "rlxq_strerror": (C.c_char_p, [I]),
        "rlxq_last_error": (C.c_char_p, [P]),
        "rlxq_last_kernel": (C.c_char_p, [P]),
        "rlxq_version": (C.c_char_p, []),
        "rlxq_row_bytes": (I64, [I, I64]),
        "rlxq_reserve_workspace": (I, [P, P, S]),
        "rlxq_workspace_bytes": (I64, [P, P]),
        "rlxq_workspace_retired_bytes": (I64, [P, P]),
        "rlxq_peak_probe": (I, [P, I, P, I64, P, C.POINTER(I64), P]),
        "rlxq_release_stream": (I, [P, P]),
        "rlxq_dequant_matmul": (I, [P, I, I, P, I, P, P, P, I, I64, I64, I64, P, I, P]),
        "rlxq_dequant_matmul_noalloc": (I, [P, I, I, P, I, P, P, P, I, I64, I64, I64, P, I, P]),
        "rlxq_dequant_grouped_matmul": (I, [P, I, I, P, I, P, P, P, I, P, I64, I64, I64, I64, P, I, P]),
        "rlxq_moe_grouped": (I, [P, I, I, P, I, P, P, P, I64, I64, I64, I64, I64, P, I, P]),
        "rlxq_moe_route": (I, [P, P, I64, I64, I64, I, P, P, P]),
        "rlxq_swiglu": (I, [P, P, I, I64, I64, P, I, P]),
        "rlxq_w8a8_gemm": (I, [P, P, I, P, P, I64, I64, I64, P, I, P]),
        "rlxq_quantize_act_int8": (I, [P, P, I, I64, I64, P, P, P]),
        "rlxq_dequantize": (I, [P, I, I, P, P, P, I, I64, I64, P, P]),
        "rlxq_dm_try_new": (I, [I, C.POINTER(P)]),
        "rlxq_dm_free": (None, [P]),
        "rlxq_dm_last_error": (C.c_char_p, [P]),
        "rlxq_dm_matmul": (I, [P, P, S, P, S, S, S, S, I, P]),
        "rlxq_dm_grouped_matmul": (I, [P, P, S, P, S, P, S, S, S, S, S, I, P]),
        "rlxq_dm_grouped_swiglu": (I, [P, P, S, P, S, P, S, I, P, S, I, P, S, I, S, S, S, S, P]),
        "rlxq_dm_upload_count": (I64, [P]),
        "rlxq_gguf_open": (I, [C.c_char_p, C.POINTER(P)]),
        "rlxq_gguf_close": (None, [P]),
        "rlxq_gguf_last_error": (C.c_char_p, [P]),
        "rlxq_gguf_version": (I, [P]),
        "rlxq_gguf_data_offset": (I64, [P]),
        "rlxq_gguf_tensor_count": (I64, [P]),
        "rlxq_gguf_find_tensor": (I64, [P, C.c_char_p]),
        "rlxq_gguf_tensor_info": (I, [P, I64, C.POINTER(GgufTensorInfo)]),
        "rlxq_gguf_take_packed": (I, [P, C.c_char_p, C.POINTER(I), C.POINTER(I64), C.POINTER(I),
                                      C.POINTER(I64)]),
        "rlxq_gguf_read": (I, [P, C.c_char_p, P, S]),
        "rlxq_gguf_upload": (I, [P, C.c_char_p, P, S, P]),
        "rlxq_gguf_meta_count": (I64, [P]),
        "rlxq_gguf_meta_find": (I64, [P, C.c_char_p]),
        "rlxq_gguf_meta_key": (C.c_char_p, [P, I64]),
        "rlxq_gguf_meta_type": (I, [P, I64, C.POINTER(I), C.POINTER(I), C.POINTER(C.c_uint64)]),
        "rlxq_gguf_meta_int": (I, [P, I64, C.c_uint64, C.POINTER(I64)]),
        "rlxq_gguf_meta_float": (I, [P, I64, C.c_uint64, C.POINTER(C.c_double)]),
        "rlxq_gguf_meta_str": (I, [P, I64, C.c_uint64, C.POINTER(C.c_char_p), C.POINTER(C.c_uint64)]),
        "rlxq_mlx_open": (I, [C.c_char_p, C.POINTER(P)]),
        "rlxq_mlx_close": (None, [P]),
        "rlxq_mlx_last_error": (C.c_char_p, [P]),
        "rlxq_mlx_quantization": (I, [P, C.POINTER(I), C.POINTER(I), C.POINTER(I)]),
        "rlxq_mlx_tensor_count": (I64, [P]),
        "rlxq_mlx_find_tensor": (I64, [P, C.c_char_p]),
        "rlxq_mlx_tensor_info": (I, [P, I64, C.POINTER(MlxTensorInfo)]),
        "rlxq_mlx_take_packed": (I, [P, C.c_char_p, C.POINTER(MlxPacked)]),
        "rlxq_mlx_read": (I, [P, C.c_char_p, P, S]),
        "rlxq_mlx_read_f32": (I, [P, C.c_char_p, P, S]),
        "rlxq_mlx_upload": (I, [P, C.c_char_p, P, S, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def declared_symbols() -> list[str]:
    """Function names declared in include/rlxq.h."""
    import re

    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rlxq_\w+)\s*\(", text)))


def strerror(status: int) -> str:
    return lib().rlxq_strerror(status).decode()


def _ptr(t) -> int | None:
    if t is None:
        return None
    return t.data_ptr()


def _stream(stream) -> int | None:
    if stream is None:
        import torch

        return torch.cuda.current_stream().cuda_stream or None
    return int(stream)


def _dt(t) -> int:
    import torch

    if t.dtype == torch.float32:
        return F32
    if t.dtype == torch.bfloat16:
        return BF16
    if t.dtype == torch.uint8:
        return U8
    raise TypeError(f"unsupported dtype {t.dtype}")


# ---- argument checks -------------------------------------------------------
# The C entry points check shapes, schemes and alignment, but they receive raw
# device pointers: they cannot see a tensor's size, layout or device.  These
# checks run before every call of the wrappers below and raise ValueError, so
# a wrong n, num_experts or output buffer never reaches a kernel.

_PACKED = (GGUF_Q8_0, GGUF_Q4_0, GGUF_Q4_1, MLX_AFFINE4, MLX_AFFINE8, GGUF_Q4_K, GGUF_Q6_K, MLX_MXFP4,
           GGUF_Q5_K, GGUF_Q3_K, GGUF_Q2_K, GGUF_Q8_K)


def packed_row_bytes(scheme: int, k: int) -> int:
    """Bytes of one packed weight row of K elements (-1 if K does not fit
    the scheme): GGUF blocks, MLX u32 codes, MXFP4 code bytes."""
    if scheme == MLX_AFFINE4 or scheme == MLX_MXFP4:
        return k // 2 if k > 0 and k % 32 == 0 else -1
    if scheme == MLX_AFFINE8:
        return k if k > 0 and k % 32 == 0 else -1
    return int(lib().rlxq_row_bytes(scheme, k))


def _need(cond, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _nbytes(t) -> int:
    return t.numel() * t.element_size()


def _tensor(t, name: str, dtypes=None, ndim=None):
    _need(t is not None, f"{name} is required")
    _need(hasattr(t, "data_ptr") and hasattr(t, "is_contiguous"), f"{name} must be a tensor")
    _need(t.is_contiguous(), f"{name} must be contiguous (got strides {tuple(t.stride())})")
    if dtypes is not None:
        _need(t.dtype in dtypes, f"{name} has dtype {t.dtype}, expected one of {[str(d) for d in dtypes]}")
    if ndim is not None:
        _need(t.dim() == ndim, f"{name} must be {ndim}-D (got shape {tuple(t.shape)})")


def _on_device(device: int, **tensors) -> None:
    for name, t in tensors.items():
        if t is not None:
            _need(t.is_cuda and (t.device.index or 0) == device,
                  f"{name} is on {t.device}, the context is on cuda:{device}")


def _act_dtypes():
    import torch

    return (torch.float32, torch.bfloat16)


def _check_weights(scheme: int, group: int, w, scales, biases, rows: int, k: int, what: str) -> None:
    """w (and the MLX / MXFP4 / Int8Block slabs) hold at least `rows` packed
    rows of K weights (rows = N, or E * N for an expert bank).  What the C
    entry point checks itself (scheme, K against the scheme, group size, slab
    dtypes, NULL slabs) is left to it, so its status codes reach the caller."""
    import torch

    _tensor(w, f"{what}: w")
    if scheme == INT8_BLOCK:
        _need(w.dtype in (torch.int8, torch.uint8), f"{what}: Int8Block weights are int8 [K, N]")
        _need(_nbytes(w) >= k * rows, f"{what}: w holds {_nbytes(w)} B, [K={k}, N={rows}] int8 needs {k * rows}")
        for nm, t in (("scales", scales), ("zero points", biases)):
            if t is not None:
                _tensor(t, f"{what}: {nm}")
                _need(t.numel() >= rows, f"{what}: {nm} have {t.numel()} elements, N = {rows}")
        return
    if scheme not in _PACKED:
        return
    rb = packed_row_bytes(scheme, k)
    if rb <= 0:
        return
    _need(_nbytes(w) >= rows * rb, f"{what}: w holds {_nbytes(w)} B, {rows} rows of {rb} B need {rows * rb}")
    if scheme in (MLX_AFFINE4, MLX_AFFINE8, MLX_MXFP4):
        g = 32 if scheme == MLX_MXFP4 else group
        if g <= 0 or k % g:
            return
        per = rows * (k // g)
        slabs = (("scales", scales),) if scheme == MLX_MXFP4 else (("scales", scales), ("biases", biases))
        for nm, t in slabs:
            if t is not None:
                _tensor(t, f"{what}: {nm}")
                _need(t.numel() >= per, f"{what}: {nm} has {t.numel()} elements, [{rows}, {k // g}] needs {per}")
        if scheme != MLX_MXFP4 and scales is not None and biases is not None:
            _need(scales.dtype == biases.dtype, f"{what}: scales and biases must share a dtype")


def _check_out(y, shape, what: str) -> None:
    _tensor(y, f"{what}: y", _act_dtypes())
    _need(tuple(y.shape) == tuple(shape), f"{what}: y has shape {tuple(y.shape)}, expected {tuple(shape)}")


def check_dense(x, w, scheme: int, n: int, *, group: int = 32, scales=None, biases=None, y=None,
                device=None) -> None:
    """Raises ValueError unless the dense call's tensors fit each other."""
    _tensor(x, "dequant_matmul: x", _act_dtypes(), 2)
    m, k = x.shape
    _need(n >= 0, "dequant_matmul: n must be >= 0")
    _check_weights(scheme, group, w, scales, biases, n, k, "dequant_matmul")
    if y is not None:
        _check_out(y, (m, n), "dequant_matmul")
    if device is not None:
        _on_device(device, x=x, w=w, scales=scales, biases=biases, y=y)


def check_grouped(x, bank, expert_idx, scheme: int, n: int, num_experts: int, *, group: int = 32, scales=None,
                  biases=None, y=None, device=None) -> None:
    import torch

    _tensor(x, "grouped_matmul: x", _act_dtypes(), 2)
    rows, k = x.shape
    _need(num_experts > 0 and n >= 0, "grouped_matmul: need num_experts > 0 and n >= 0")
    _check_weights(scheme, group, bank, scales, biases, num_experts * n, k, "grouped_matmul")
    _tensor(expert_idx, "grouped_matmul: expert_idx", (torch.float32,))
    _need(expert_idx.numel() == rows, f"grouped_matmul: expert_idx has {expert_idx.numel()} entries, rows = {rows}")
    if y is not None:
        _check_out(y, (rows, n), "grouped_matmul")
    if device is not None:
        _on_device(device, x=x, bank=bank, expert_idx=expert_idx, scales=scales, biases=biases, y=y)


def check_moe(x, bank, ids, probs, scheme: int, mode: int, n: int, num_experts: int, *, y=None,
              device=None) -> None:
    import torch

    _need(mode in (MOE_EXPAND, MOE_COMBINE, MOE_EXPAND_SWIGLU), f"moe_grouped: unknown mode {mode}")
    _tensor(ids, "moe_grouped: ids", (torch.int32,), 2)
    rows, top_k = ids.shape
    _tensor(x, "moe_grouped: x", _act_dtypes(), 2)
    k = x.shape[1]
    want_rows = rows * top_k if mode == MOE_COMBINE else rows
    _need(x.shape[0] == want_rows, f"moe_grouped: x has {x.shape[0]} rows, this mode needs {want_rows}")
    _need(num_experts > 0 and n >= 0, "moe_grouped: need num_experts > 0 and n >= 0")
    _need(mode != MOE_EXPAND_SWIGLU or n % 2 == 0, "moe_grouped: EXPAND_SWIGLU needs an even n (gate|up)")
    _check_weights(scheme, 32, bank, None, None, num_experts * n, k, "moe_grouped")
    if mode == MOE_COMBINE:
        _tensor(probs, "moe_grouped: probs", (torch.float32,), 2)
        _need(tuple(probs.shape) == (rows, top_k), f"moe_grouped: probs has shape {tuple(probs.shape)}")
    if y is not None:
        width = n // 2 if mode == MOE_EXPAND_SWIGLU else n
        _check_out(y, (rows if mode == MOE_COMBINE else rows * top_k, width), "moe_grouped")
    if device is not None:
        _on_device(device, x=x, bank=bank, ids=ids, probs=probs if mode == MOE_COMBINE else None, y=y)


def check_w8a8(x, wq, w_scale, n: int, *, y=None, device=None) -> None:
    import torch

    _tensor(x, "w8a8_gemm: x", _act_dtypes(), 2)
    m, k = x.shape
    _tensor(wq, "w8a8_gemm: wq", (torch.int8,))
    _need(wq.numel() >= k * n, f"w8a8_gemm: wq has {wq.numel()} elements, [K={k}, N={n}] needs {k * n}")
    _tensor(w_scale, "w8a8_gemm: w_scale", (torch.float32,))
    _need(w_scale.numel() >= n, f"w8a8_gemm: w_scale has {w_scale.numel()} elements, N = {n}")
    if y is not None:
        _check_out(y, (m, n), "w8a8_gemm")
    if device is not None:
        _on_device(device, x=x, wq=wq, w_scale=w_scale, y=y)


class Context:
    """Owns an rlxq_ctx on one device (rlxq_init / rlxq_destroy)."""

    def __init__(self, device: int = 0):
        self.device = device
        h = C.c_void_p()
        rc = lib().rlxq_init(device, C.byref(h))
        if rc != OK:
            raise RlxqError(rc, f"rlxq_init({device}): {strerror(rc)}")
        self.h = h

    def close(self) -> None:
        if getattr(self, "h", None):
            lib().rlxq_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc: int, what: str) -> None:
        if rc != OK:
            raise RlxqError(rc, f"{what}: {strerror(rc)}: {lib().rlxq_last_error(self.h).decode()}")

    @property
    def last_kernel(self) -> str:
        return lib().rlxq_last_kernel(self.h).decode()

    def reserve_workspace(self, nbytes: int, *, stream=None) -> None:
        """Sizes the context scratch of `stream` to at least nbytes (before a
        graph capture)."""
        self._check(lib().rlxq_reserve_workspace(self.h, _stream(stream), nbytes), "reserve_workspace")

    def workspace_bytes(self, *, stream=None) -> int:
        return int(lib().rlxq_workspace_bytes(self.h, _stream(stream)))

    def peak_probe(self, kind: int, work: int, *, buf=None, sink, stream=None) -> int:
        """rlxq_peak_probe: launches the probe on `stream`, returns the flops
        (PROBE_MFMA) or bytes (PROBE_READ, PROBE_READ4, PROBE_TILE20) it
        issues."""
        cnt = C.c_int64(0)
        rc = lib().rlxq_peak_probe(self.h, kind, _ptr(buf), work, _ptr(sink), C.byref(cnt), _stream(stream))
        self._check(rc, "peak_probe")
        return int(cnt.value)

    def workspace_retired_bytes(self, *, stream=None) -> int:
        """Bytes of replaced scratch buffers `stream` still holds."""
        return int(lib().rlxq_workspace_retired_bytes(self.h, _stream(stream)))

    def release_stream(self, *, stream=None) -> None:
        """Frees the scratch buffers of `stream` after waiting for it."""
        self._check(lib().rlxq_release_stream(self.h, _stream(stream)), "release_stream")

    def bind_dequant_matmul(self, x, w, scheme: int, n: int, *, y, stream, group: int = 32, scales=None,
                            biases=None):
        """A zero-argument callable that runs dequant_matmul on these tensors.

        The C arguments are converted once, as a compiled caller's FFI binding
        holds them, so a call costs the C entry point and not this module's
        argument handling (decode launches are a few microseconds each).  The
        tensors must stay alive while the callable is used."""
        check_dense(x, w, scheme, n, group=group, scales=scales, biases=biases, y=y, device=self.device)
        m, k = x.shape
        sb = _dt(scales) if scales is not None else F32
        fn = lib().rlxq_dequant_matmul
        args = (self.h, C.c_int(scheme), C.c_int(group), C.c_void_p(_ptr(x)), C.c_int(_dt(x)), C.c_void_p(_ptr(w)),
                C.c_void_p(_ptr(scales)), C.c_void_p(_ptr(biases)), C.c_int(sb), C.c_int64(m), C.c_int64(k),
                C.c_int64(n), C.c_void_p(_ptr(y)), C.c_int(_dt(y)), C.c_void_p(_stream(stream)))

        def call():
            rc = fn(*args)
            if rc != OK:
                self._check(rc, "dequant_matmul")

        return call

    def dequant_matmul(self, x, w, scheme: int, n: int, *, group: int = 32, scales=None, biases=None,
                       y=None, y_dtype=None, stream=None):
        """y[m, n] = x[m, k] . dequant(w)^T; returns y (allocated if not given)."""
        import torch

        check_dense(x, w, scheme, n, group=group, scales=scales, biases=biases, y=y, device=self.device)
        m, k = x.shape
        if y is None:
            y = torch.empty((m, n), dtype=y_dtype or torch.float32, device=x.device)
        sb = _dt(scales) if scales is not None else F32
        rc = lib().rlxq_dequant_matmul(self.h, scheme, group, _ptr(x), _dt(x), _ptr(w), _ptr(scales), _ptr(biases),
                                       sb, m, k, n, _ptr(y), _dt(y), _stream(stream))
        self._check(rc, "dequant_matmul")
        return y

    def dequant_matmul_noalloc(self, x, w, scheme: int, n: int, *, y, group: int = 32, scales=None, biases=None,
                               stream=None):
        """rlxq_dequant_matmul_noalloc into the caller's y: no device memory is
        allocated (the scratch is the library's static per-GPU array)."""
        check_dense(x, w, scheme, n, group=group, scales=scales, biases=biases, y=y, device=self.device)
        m, k = x.shape
        sb = _dt(scales) if scales is not None else F32
        rc = lib().rlxq_dequant_matmul_noalloc(self.h, scheme, group, _ptr(x), _dt(x), _ptr(w), _ptr(scales),
                                               _ptr(biases), sb, m, k, n, _ptr(y), _dt(y), _stream(stream))
        self._check(rc, "dequant_matmul_noalloc")
        return y

    def dequantize(self, w, scheme: int, rows: int, k: int, *, group: int = 32, scales=None, biases=None,
                   out=None, stream=None):
        import torch

        _need(rows >= 0 and k > 0, "dequantize: need rows >= 0 and k > 0")
        _need(scheme != INT8_BLOCK, "dequantize: Int8Block has no packed rows")
        _check_weights(scheme, group, w, scales, biases, rows, k, "dequantize")
        if out is None:
            out = torch.empty((rows, k), dtype=torch.float32, device=w.device)
        _tensor(out, "dequantize: out", (torch.float32,))
        _need(tuple(out.shape) == (rows, k), f"dequantize: out has shape {tuple(out.shape)}, expected {(rows, k)}")
        _on_device(self.device, w=w, scales=scales, biases=biases, out=out)
        sb = _dt(scales) if scales is not None else F32
        rc = lib().rlxq_dequantize(self.h, scheme, group, _ptr(w), _ptr(scales), _ptr(biases), sb, rows, k,
                                   _ptr(out), _stream(stream))
        self._check(rc, "dequantize")
        return out

    def grouped_matmul(self, x, bank, expert_idx, scheme: int, n: int, num_experts: int, *, group: int = 32,
                       scales=None, biases=None, y=None, y_dtype=None, stream=None):
        import torch

        check_grouped(x, bank, expert_idx, scheme, n, num_experts, group=group, scales=scales, biases=biases, y=y,
                      device=self.device)
        rows, k = x.shape
        if y is None:
            y = torch.empty((rows, n), dtype=y_dtype or torch.float32, device=x.device)
        sb = _dt(scales) if scales is not None else F32
        rc = lib().rlxq_dequant_grouped_matmul(self.h, scheme, group, _ptr(x), _dt(x), _ptr(bank), _ptr(scales),
                                               _ptr(biases), sb, _ptr(expert_idx), rows, k, n, num_experts,
                                               _ptr(y), _dt(y), _stream(stream))
        self._check(rc, "dequant_grouped_matmul")
        return y

    def moe_grouped(self, x, bank, ids, probs, scheme: int, mode: int, n: int, num_experts: int, *,
                    y=None, y_dtype=None, stream=None):
        import torch

        check_moe(x, bank, ids, probs, scheme, mode, n, num_experts, y=y, device=self.device)
        rows, top_k = ids.shape
        k = x.shape[1]
        out_rows = rows if mode == MOE_COMBINE else rows * top_k
        width = n // 2 if mode == MOE_EXPAND_SWIGLU else n
        if y is None:
            y = torch.empty((out_rows, width), dtype=y_dtype or torch.float32, device=x.device)
        rc = lib().rlxq_moe_grouped(self.h, scheme, mode, _ptr(x), _dt(x), _ptr(bank), _ptr(ids), _ptr(probs),
                                    rows, top_k, k, n, num_experts, _ptr(y), _dt(y), _stream(stream))
        self._check(rc, "moe_grouped")
        return y

    def moe_route(self, logits, top_k: int, renorm: bool, *, stream=None):
        import torch

        _tensor(logits, "moe_route: logits", (torch.float32,), 2)
        _on_device(self.device, logits=logits)
        rows, e = logits.shape
        ids = torch.empty((rows, top_k), dtype=torch.int32, device=logits.device)
        probs = torch.empty((rows, top_k), dtype=torch.float32, device=logits.device)
        rc = lib().rlxq_moe_route(self.h, _ptr(logits), rows, e, top_k, int(renorm), _ptr(ids), _ptr(probs),
                                  _stream(stream))
        self._check(rc, "moe_route")
        return ids, probs

    def swiglu(self, gu, inter: int, *, out=None, out_dtype=None, stream=None):
        import torch

        _tensor(gu, "swiglu: gu", _act_dtypes(), 2)
        _need(gu.shape[1] == 2 * inter, f"swiglu: gu has {gu.shape[1]} columns, 2 * inter = {2 * inter}")
        rows = gu.shape[0]
        if out is None:
            out = torch.empty((rows, inter), dtype=out_dtype or gu.dtype, device=gu.device)
        _check_out(out, (rows, inter), "swiglu")
        _on_device(self.device, gu=gu, out=out)
        rc = lib().rlxq_swiglu(self.h, _ptr(gu), _dt(gu), rows, inter, _ptr(out), _dt(out), _stream(stream))
        self._check(rc, "swiglu")
        return out

    def quantize_act_int8(self, x, *, stream=None):
        import torch

        _tensor(x, "quantize_act_int8: x", _act_dtypes(), 2)
        _on_device(self.device, x=x)
        m, k = x.shape
        q = torch.empty((m, k), dtype=torch.int8, device=x.device)
        s = torch.empty((m,), dtype=torch.float32, device=x.device)
        rc = lib().rlxq_quantize_act_int8(self.h, _ptr(x), _dt(x), m, k, _ptr(q), _ptr(s), _stream(stream))
        self._check(rc, "quantize_act_int8")
        return q, s

    def w8a8_gemm(self, x, wq, w_scale, n: int, *, y=None, y_dtype=None, stream=None):
        import torch

        check_w8a8(x, wq, w_scale, n, y=y, device=self.device)
        m, k = x.shape
        if y is None:
            y = torch.empty((m, n), dtype=y_dtype or torch.float32, device=x.device)
        rc = lib().rlxq_w8a8_gemm(self.h, _ptr(x), _dt(x), _ptr(wq), _ptr(w_scale), m, k, n, _ptr(y), _dt(y),
                                  _stream(stream))
        self._check(rc, "w8a8_gemm")
        return y


class DeviceMatmul:
    """The host-slice session API (rlxq_dm_*), mirroring rlx-laguna's DeviceMatmul."""

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        rc = lib().rlxq_dm_try_new(device, C.byref(h))
        if rc != OK:
            raise RlxqError(rc, f"rlxq_dm_try_new({device}): {strerror(rc)}")
        self.h = h

    def close(self) -> None:
        if getattr(self, "h", None):
            lib().rlxq_dm_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc: int) -> None:
        if rc != OK:
            raise RlxqError(rc, lib().rlxq_dm_last_error(self.h).decode())

    @property
    def uploads(self) -> int:
        return int(lib().rlxq_dm_upload_count(self.h))

    def matmul(self, x, w_bytes, m: int, k: int, n: int, scheme: int):
        import numpy as np

        x = np.ascontiguousarray(x, dtype=np.float32).ravel()
        w_bytes = np.ascontiguousarray(w_bytes, dtype=np.uint8).ravel()
        y = np.empty(m * n, np.float32)
        rc = lib().rlxq_dm_matmul(self.h, x.ctypes.data, x.size, w_bytes.ctypes.data, w_bytes.size, m, k, n,
                                  scheme, y.ctypes.data)
        self._check(rc)
        return y

    def grouped_matmul(self, x, w_bytes, expert_idx, m: int, k: int, n: int, num_experts: int, scheme: int):
        import numpy as np

        x = np.ascontiguousarray(x, dtype=np.float32).ravel()
        w_bytes = np.ascontiguousarray(w_bytes, dtype=np.uint8).ravel()
        idx = np.ascontiguousarray(expert_idx, dtype=np.float32).ravel()
        y = np.empty(m * n, np.float32)
        rc = lib().rlxq_dm_grouped_matmul(self.h, x.ctypes.data, x.size, w_bytes.ctypes.data, w_bytes.size,
                                          idx.ctypes.data, idx.size, m, k, n, num_experts, scheme, y.ctypes.data)
        self._check(rc)
        return y

    def grouped_swiglu(self, x, expert_idx, w_gate, gate_scheme: int, w_up, up_scheme: int, w_down,
                       down_scheme: int, m: int, h: int, inter: int, num_experts: int):
        """down(silu(gate(x)) * up(x)) per row (DeviceMatmul::grouped_swiglu,
        crates/rlx-laguna/src/device_matmul.rs:221-296): f32 [m * h]."""
        import numpy as np

        x = np.ascontiguousarray(x, dtype=np.float32).ravel()
        idx = np.ascontiguousarray(expert_idx, dtype=np.float32).ravel()
        ws = [np.ascontiguousarray(w, dtype=np.uint8).ravel() for w in (w_gate, w_up, w_down)]
        y = np.empty(m * h, np.float32)
        rc = lib().rlxq_dm_grouped_swiglu(self.h, x.ctypes.data, x.size, idx.ctypes.data, idx.size,
                                          ws[0].ctypes.data, ws[0].size, gate_scheme, ws[1].ctypes.data,
                                          ws[1].size, up_scheme, ws[2].ctypes.data, ws[2].size, down_scheme,
                                          m, h, inter, num_experts, y.ctypes.data)
        self._check(rc)
        return y


class GgufTensor:
    """One tensor info of a GGUF file: `shape` innermost first, as stored."""

    def __init__(self, ti: GgufTensorInfo):
        self.name = ti.name.decode()
        self.dtype = int(ti.ggml_type)
        self.shape = [int(ti.dims[d]) for d in range(ti.n_dims)]
        self.offset = int(ti.offset)
        self.nbytes = int(ti.nbytes)
        self.scheme = int(ti.scheme)

    def __repr__(self):
        return f"GgufTensor({self.name!r}, type={self.dtype}, shape={self.shape}, nbytes={self.nbytes})"


class GgufFile:
    """A GGUF checkpoint through rlxq_gguf_* (GgufFile / GgufLoader's packed
    path: crates/rlx-models-core/src/weight_loader.rs:1360-1486)."""

    def __init__(self, path):
        h = C.c_void_p()
        rc = lib().rlxq_gguf_open(str(path).encode(), C.byref(h))
        if rc != OK:
            msg = lib().rlxq_gguf_last_error(h).decode() if h else strerror(rc)
            lib().rlxq_gguf_close(h)
            raise RlxqError(rc, msg)
        self.h = h
        L = lib()
        self.version = int(L.rlxq_gguf_version(h))
        self.data_offset = int(L.rlxq_gguf_data_offset(h))
        self.tensors = {}
        for i in range(int(L.rlxq_gguf_tensor_count(h))):
            ti = GgufTensorInfo()
            self._check(L.rlxq_gguf_tensor_info(h, i, C.byref(ti)))
            t = GgufTensor(ti)
            self.tensors[t.name] = t

    def close(self) -> None:
        if getattr(self, "h", None):
            lib().rlxq_gguf_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc: int) -> None:
        if rc != OK:
            raise RlxqError(rc, lib().rlxq_gguf_last_error(self.h).decode() or strerror(rc))

    def get(self, name: str):
        return self.tensors.get(name)

    def keys(self) -> list:
        L = lib()
        return [L.rlxq_gguf_meta_key(self.h, i).decode() for i in range(int(L.rlxq_gguf_meta_count(self.h)))]

    def meta(self, key: str):
        """The value of a metadata key: int, float, bool, str or a list of them."""
        L = lib()
        i = int(L.rlxq_gguf_meta_find(self.h, key.encode()))
        if i < 0:
            raise KeyError(key)
        ty, el, cnt = C.c_int(), C.c_int(), C.c_uint64()
        self._check(L.rlxq_gguf_meta_type(self.h, i, C.byref(ty), C.byref(el), C.byref(cnt)))

        def one(j):
            if el.value == 8:
                sp, n = C.c_char_p(), C.c_uint64()
                self._check(L.rlxq_gguf_meta_str(self.h, i, j, C.byref(sp), C.byref(n)))
                return C.string_at(sp, n.value).decode("utf-8", "replace")
            if el.value in (6, 12):
                v = C.c_double()
                self._check(L.rlxq_gguf_meta_float(self.h, i, j, C.byref(v)))
                return v.value
            v = C.c_int64()
            self._check(L.rlxq_gguf_meta_int(self.h, i, j, C.byref(v)))
            return bool(v.value) if el.value == 7 else v.value

        if ty.value == 9:
            return [one(j) for j in range(cnt.value)]
        return one(0)

    def take_packed(self, name: str):
        """(scheme, shape outermost first, nbytes), or None for a tensor the
        kernels do not read packed (not taken then); raises on a second take."""
        sch, nd, nb = C.c_int(), C.c_int(), C.c_int64()
        shape = (C.c_int64 * 4)()
        self._check(lib().rlxq_gguf_take_packed(self.h, name.encode(), C.byref(sch), shape, C.byref(nd),
                                                C.byref(nb)))
        if sch.value == 0:
            return None
        return sch.value, [int(shape[d]) for d in range(nd.value)], int(nb.value)

    def read(self, name: str):
        import numpy as np

        t = self.tensors[name]
        out = np.empty(max(t.nbytes, 0), np.uint8)
        self._check(lib().rlxq_gguf_read(self.h, name.encode(), out.ctypes.data, out.size))
        return out

    def upload(self, name: str, dst, *, stream=None):
        """The tensor's bytes into the device tensor `dst` (pread + pinned staging)."""
        nbytes = dst.numel() * dst.element_size()
        self._check(lib().rlxq_gguf_upload(self.h, name.encode(), _ptr(dst), nbytes, _stream(stream)))
        return dst


class MlxFile:
    """An MLX (mlx-community) checkpoint through rlxq_mlx_*: a directory or
    one .safetensors file (MlxLoader and take_packed_mlx:
    crates/rlx-models-core/src/weight_loader.rs:906-1012)."""

    def __init__(self, path):
        h = C.c_void_p()
        rc = lib().rlxq_mlx_open(str(path).encode(), C.byref(h))
        if rc != OK:
            msg = lib().rlxq_mlx_last_error(h).decode() if h else strerror(rc)
            lib().rlxq_mlx_close(h)
            raise RlxqError(rc, msg)
        self.h = h
        L = lib()
        self.tensors = {}
        for i in range(int(L.rlxq_mlx_tensor_count(h))):
            ti = MlxTensorInfo()
            self._check(L.rlxq_mlx_tensor_info(h, i, C.byref(ti)))
            self.tensors[ti.name.decode()] = {"dtype": ST_DTYPES[ti.dtype],
                                              "shape": [int(ti.shape[d]) for d in range(ti.n_dims)],
                                              "nbytes": int(ti.nbytes), "file": ti.file.decode(),
                                              "offset": int(ti.offset)}
        b, g, m = C.c_int(), C.c_int(), C.c_int()
        self._check(L.rlxq_mlx_quantization(h, C.byref(b), C.byref(g), C.byref(m)))
        self.quantization = (b.value, g.value, m.value)

    def close(self) -> None:
        if getattr(self, "h", None):
            lib().rlxq_mlx_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc: int) -> None:
        if rc != OK:
            raise RlxqError(rc, lib().rlxq_mlx_last_error(self.h).decode() or strerror(rc))

    def take_packed(self, key: str):
        """The packed Linear as a dict, or None when `key` is not packed in a
        form the kernels read (not taken then); raises on a second take."""
        p = MlxPacked()
        self._check(lib().rlxq_mlx_take_packed(self.h, key.encode(), C.byref(p)))
        if p.scheme == 0:
            return None
        return {"scheme": p.scheme, "bits": p.bits, "group_size": p.group_size, "n": p.out_features,
                "k": p.in_features, "codes": p.codes.decode(), "scales": p.scales.decode(),
                "biases": p.biases.decode() if p.biases else None, "codes_nbytes": p.codes_nbytes,
                "scales_nbytes": p.scales_nbytes, "biases_nbytes": p.biases_nbytes,
                "slab_dtype": ST_DTYPES[p.slab_dtype]}

    def read(self, name: str):
        import numpy as np

        out = np.empty(self.tensors[name]["nbytes"], np.uint8)
        self._check(lib().rlxq_mlx_read(self.h, name.encode(), out.ctypes.data, out.size))
        return out

    def read_f32(self, name: str):
        import numpy as np

        t = self.tensors[name]
        out = np.empty(int(np.prod(t["shape"])) if t["shape"] else 1, np.float32)
        self._check(lib().rlxq_mlx_read_f32(self.h, name.encode(), out.ctypes.data, out.size))
        return out.reshape(t["shape"])

    def upload(self, name: str, dst, *, stream=None):
        nbytes = dst.numel() * dst.element_size()
        self._check(lib().rlxq_mlx_upload(self.h, name.encode(), _ptr(dst), nbytes, _stream(stream)))
        return dst
