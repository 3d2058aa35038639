"""CPU tests of the Python binding's argument checks (rlxq.check_*): tensor
sizes, layout, dtypes of index operands and devices that the C entry points
cannot see through raw pointers are rejected with ValueError before anything
is launched.  No GPU is needed: the checks run on CPU tensors, and a Context
built without a device shows that its methods raise before calling the C ABI."""
import pytest
import torch

import rlxq

Q4_1 = rlxq.GGUF_Q4_1


def _u8(n):
    return torch.zeros(n, dtype=torch.uint8)


def test_dense_sizes_ok_then_device():
    x = torch.zeros((2, 64), dtype=torch.bfloat16)
    w = _u8(8 * 40)   # 8 rows of 2 Q4_1 blocks
    y = torch.zeros((2, 8))
    rlxq.check_dense(x, w, Q4_1, 8, y=y)               # sizes fit
    with pytest.raises(ValueError, match="context is on cuda:0"):
        rlxq.check_dense(x, w, Q4_1, 8, y=y, device=0)  # CPU tensors


@pytest.mark.parametrize("case", ["w_short", "y_shape", "y_dtype", "x_strided", "x_1d", "n_too_big"])
def test_dense_rejects(case):
    x = torch.zeros((2, 64), dtype=torch.bfloat16)
    w = _u8(8 * 40)
    y = torch.zeros((2, 8))
    n = 8
    if case == "w_short":
        w = w[:-1]
    elif case == "y_shape":
        y = torch.zeros((2, 7))
    elif case == "y_dtype":
        y = torch.zeros((2, 8), dtype=torch.float16)
    elif case == "x_strided":
        x = torch.zeros((64, 2), dtype=torch.bfloat16).t()
    elif case == "x_1d":
        x = torch.zeros((64,), dtype=torch.bfloat16)
    elif case == "n_too_big":
        n, y = 9, torch.zeros((2, 9))
    with pytest.raises(ValueError):
        rlxq.check_dense(x, w, Q4_1, n, y=y)


def test_mlx_and_int8_slabs():
    x = torch.zeros((1, 128))
    codes = _u8(4 * 64)   # 4 rows, 4-bit
    sc = torch.zeros((4, 2))
    bi = torch.zeros((4, 2))
    rlxq.check_dense(x, codes, rlxq.MLX_AFFINE4, 4, group=64, scales=sc, biases=bi)
    with pytest.raises(ValueError, match="biases"):
        rlxq.check_dense(x, codes, rlxq.MLX_AFFINE4, 4, group=64, scales=sc, biases=bi[:3])
    with pytest.raises(ValueError, match="share a dtype"):
        rlxq.check_dense(x, codes, rlxq.MLX_AFFINE4, 4, group=64, scales=sc, biases=bi.to(torch.bfloat16))
    wq = torch.zeros((128, 16), dtype=torch.int8)
    rlxq.check_dense(x, wq, rlxq.INT8_BLOCK, 16, scales=torch.ones(16))
    with pytest.raises(ValueError, match="int8"):
        rlxq.check_dense(x, wq[:100], rlxq.INT8_BLOCK, 16, scales=torch.ones(16))
    with pytest.raises(ValueError, match="scales"):
        rlxq.check_dense(x, wq, rlxq.INT8_BLOCK, 16, scales=torch.ones(15))


def test_grouped_and_moe():
    x = torch.zeros((3, 64), dtype=torch.bfloat16)
    E, n = 4, 8
    bank = _u8(E * n * 40)
    idx = torch.zeros(3)
    rlxq.check_grouped(x, bank, idx, Q4_1, n, E)
    with pytest.raises(ValueError, match="w holds"):
        rlxq.check_grouped(x, bank, idx, Q4_1, n, E + 1)        # num_experts beyond the bank
    with pytest.raises(ValueError, match="expert_idx"):
        rlxq.check_grouped(x, bank, idx.to(torch.int32), Q4_1, n, E)
    with pytest.raises(ValueError, match="entries"):
        rlxq.check_grouped(x, bank, idx[:2], Q4_1, n, E)
    ids = torch.zeros((3, 2), dtype=torch.int32)
    probs = torch.zeros((3, 2))
    rlxq.check_moe(x, bank, ids, None, Q4_1, rlxq.MOE_EXPAND, n, E, y=torch.zeros((6, n)))
    rlxq.check_moe(x, bank, ids, None, Q4_1, rlxq.MOE_EXPAND_SWIGLU, n, E, y=torch.zeros((6, n // 2)))
    x6 = torch.zeros((6, 64), dtype=torch.bfloat16)
    rlxq.check_moe(x6, bank, ids, probs, Q4_1, rlxq.MOE_COMBINE, n, E, y=torch.zeros((3, n)))
    with pytest.raises(ValueError, match="rows"):
        rlxq.check_moe(x, bank, ids, probs, Q4_1, rlxq.MOE_COMBINE, n, E)
    with pytest.raises(ValueError, match="ids"):
        rlxq.check_moe(x, bank, ids.long(), None, Q4_1, rlxq.MOE_EXPAND, n, E)
    with pytest.raises(ValueError, match="probs"):
        rlxq.check_moe(x6, bank, ids, None, Q4_1, rlxq.MOE_COMBINE, n, E)
    with pytest.raises(ValueError, match="y has shape"):
        rlxq.check_moe(x, bank, ids, None, Q4_1, rlxq.MOE_EXPAND_SWIGLU, n, E, y=torch.zeros((6, n)))


def test_w8a8():
    x = torch.zeros((2, 64))
    wq = torch.zeros((64, 32), dtype=torch.int8)
    rlxq.check_w8a8(x, wq, torch.ones(32), 32)
    with pytest.raises(ValueError, match="wq"):
        rlxq.check_w8a8(x, wq, torch.ones(32), 33)
    with pytest.raises(ValueError, match="wq"):
        rlxq.check_w8a8(x, wq.to(torch.uint8), torch.ones(32), 32)
    with pytest.raises(ValueError, match="w_scale"):
        rlxq.check_w8a8(x, wq, torch.ones(31), 32)


def test_context_methods_check_before_the_c_call():
    """A Context without a device: a bad argument must raise ValueError from
    the binding, never reach the C entry point (whose handle is NULL here)."""
    c = rlxq.Context.__new__(rlxq.Context)
    c.h, c.device = None, 0
    x = torch.zeros((2, 64), dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        c.dequant_matmul(x, _u8(10), Q4_1, 8)
    with pytest.raises(ValueError):
        c.grouped_matmul(x, _u8(8 * 40), torch.zeros(2), Q4_1, 8, 2)
    with pytest.raises(ValueError):
        c.moe_grouped(x, _u8(8 * 40), torch.zeros((2, 2), dtype=torch.int32), None, Q4_1, rlxq.MOE_EXPAND, 8, 2)
    with pytest.raises(ValueError):
        c.w8a8_gemm(x, torch.zeros((64, 8), dtype=torch.int8), torch.ones(7), 8)
    with pytest.raises(ValueError):
        c.swiglu(torch.zeros((2, 9)), 4)
    with pytest.raises(ValueError):
        c.bind_dequant_matmul(x, _u8(8 * 40), Q4_1, 8, y=torch.zeros((2, 8)), stream=0)   # CPU tensors


def test_packed_row_bytes():
    assert rlxq.packed_row_bytes(Q4_1, 4096) == 2560
    assert rlxq.packed_row_bytes(rlxq.GGUF_Q8_0, 4096) == 4352
    assert rlxq.packed_row_bytes(rlxq.MLX_AFFINE4, 4096) == 2048
    assert rlxq.packed_row_bytes(rlxq.MLX_AFFINE8, 4096) == 4096
    assert rlxq.packed_row_bytes(rlxq.MLX_MXFP4, 4096) == 2048
    assert rlxq.packed_row_bytes(rlxq.GGUF_Q4_K, 4096) == 2304
    assert rlxq.packed_row_bytes(Q4_1, 100) == -1
