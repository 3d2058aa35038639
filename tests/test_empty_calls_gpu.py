"""Empty calls through the C ABI: zero activation rows, zero output
columns, zero entries or zero routed rows are valid and do nothing (the
reference's ops take empty batches; nothing is launched and nothing is
written), while negative sizes are shape errors.  Every entry point of the
hot path is called with real device pointers and a sentinel-filled output,
which must come back unchanged."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

Q4_1, F32, BF16 = 3, 0, 1


def _bufs():
    import torch

    x = torch.ones((4, 256), device="cuda")
    w = torch.zeros((64 * 160,), device="cuda", dtype=torch.uint8)
    y = torch.full((4, 64), 7.0, device="cuda")
    return x, w, y


def _unchanged(y):
    import torch

    torch.cuda.synchronize()
    assert bool((y == 7.0).all())


def test_dense_empty(ctx):
    import rlxq

    L = rlxq.lib()
    x, w, y = _bufs()
    for fn in (L.rlxq_dequant_matmul, L.rlxq_dequant_matmul_noalloc):
        for m, n in ((0, 64), (4, 0), (0, 0)):
            assert fn(ctx.h, Q4_1, 32, x.data_ptr(), F32, w.data_ptr(), None, None, F32, m, 256, n,
                      y.data_ptr(), F32, None) == rlxq.OK
        assert fn(ctx.h, Q4_1, 32, x.data_ptr(), F32, w.data_ptr(), None, None, F32, -1, 256, 64,
                  y.data_ptr(), F32, None) == rlxq.E_SHAPE
        assert fn(ctx.h, Q4_1, 32, x.data_ptr(), F32, w.data_ptr(), None, None, F32, 4, 0, 64,
                  y.data_ptr(), F32, None) == rlxq.E_SHAPE
    _unchanged(y)


def test_grouped_moe_and_helpers_empty(ctx):
    import torch
    import rlxq

    L = rlxq.lib()
    x, w, y = _bufs()
    idx = torch.zeros((4,), device="cuda")
    ids = torch.zeros((4, 2), device="cuda", dtype=torch.int32)
    probs = torch.full((4, 2), 0.5, device="cuda")
    logits = torch.zeros((4, 8), device="cuda")
    assert L.rlxq_dequant_grouped_matmul(ctx.h, Q4_1, 32, x.data_ptr(), F32, w.data_ptr(), None, None, F32,
                                         idx.data_ptr(), 0, 256, 64, 2, y.data_ptr(), F32, None) == rlxq.OK
    assert L.rlxq_dequant_grouped_matmul(ctx.h, Q4_1, 32, x.data_ptr(), F32, w.data_ptr(), None, None, F32,
                                         idx.data_ptr(), -1, 256, 64, 2, y.data_ptr(), F32, None) == rlxq.E_SHAPE
    for mode in (rlxq.MOE_EXPAND, rlxq.MOE_COMBINE, rlxq.MOE_EXPAND_SWIGLU):
        assert L.rlxq_moe_grouped(ctx.h, Q4_1, mode, x.data_ptr(), F32, w.data_ptr(), ids.data_ptr(),
                                  probs.data_ptr(), 0, 2, 256, 64, 2, y.data_ptr(), F32, None) == rlxq.OK
    ids_before = ids.clone()
    assert L.rlxq_moe_route(ctx.h, logits.data_ptr(), 0, 8, 2, 1, ids.data_ptr(), probs.data_ptr(), None) == rlxq.OK
    assert L.rlxq_swiglu(ctx.h, x.data_ptr(), F32, 0, 32, y.data_ptr(), F32, None) == rlxq.OK
    assert L.rlxq_swiglu(ctx.h, x.data_ptr(), F32, 4, 0, y.data_ptr(), F32, None) == rlxq.OK
    assert L.rlxq_dequantize(ctx.h, Q4_1, 32, w.data_ptr(), None, None, F32, 0, 256, y.data_ptr(), None) == rlxq.OK
    q = torch.zeros((4, 256), device="cuda", dtype=torch.int8)
    s = torch.full((4,), 7.0, device="cuda")
    assert L.rlxq_quantize_act_int8(ctx.h, x.data_ptr(), F32, 0, 256, q.data_ptr(), s.data_ptr(), None) == rlxq.OK
    wq = torch.zeros((256, 64), device="cuda", dtype=torch.int8)
    sw = torch.ones((64,), device="cuda")
    assert L.rlxq_w8a8_gemm(ctx.h, x.data_ptr(), F32, wq.data_ptr(), sw.data_ptr(), 0, 256, 64, y.data_ptr(),
                            F32, None) == rlxq.OK
    _unchanged(y)
    torch.cuda.synchronize()
    assert bool((s == 7.0).all()) and bool((ids == ids_before).all())
