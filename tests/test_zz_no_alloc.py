"""rlxq_dequant_matmul_noalloc against rlxq_dequant_matmul through the C ABI:
the same kernels on the library's static scratch array, so the outputs are
bit-identical.  Two calls in a row, the second smaller (the array keeps the
first call's contents), on paths that use scratch: prefill split-K partial
sums, batched-decode prepared activations, Int8Block split-K; plus the
rejection of a call that needs more than RLXQ_NOALLOC_SCRATCH_BYTES."""
import numpy as np
import pytest

from conftest import announce

pytestmark = pytest.mark.gpu


def _q4_1(orc, rng, n, k):
    import torch

    return torch.from_numpy(orc.synth_q4_1(rng, n, k)).cuda()


def _x(rng, m, k):
    import torch

    return torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).cuda().to(torch.bfloat16)


@pytest.mark.parametrize("first,second", [
    ((256, 12288, 4096, "bf16"), (16, 4096, 2048, "f32")),    # split-K GEMM, then batched decode
    ((64, 4096, 6144, "f32"), (8, 4096, 1024, "f32")),        # batched decode, larger then smaller
])
def test_noalloc_matches_dequant_matmul(ctx, orc, first, second):
    import torch
    import rlxq

    rng = np.random.default_rng(77)
    for (m, k, n, yd) in (first, second):
        announce(f"noalloc Q4_1 m={m} k={k} n={n} y={yd}")
        w = _q4_1(orc, rng, n, k)
        x = _x(rng, m, k)
        ydt = torch.bfloat16 if yd == "bf16" else torch.float32
        want = ctx.dequant_matmul(x, w, rlxq.GGUF_Q4_1, n, y_dtype=ydt)
        kern = ctx.last_kernel
        y = torch.full((m, n), float("nan"), dtype=ydt, device="cuda")
        ctx.dequant_matmul_noalloc(x, w, rlxq.GGUF_Q4_1, n, y=y)
        torch.cuda.synchronize()
        assert ctx.last_kernel == kern
        assert torch.equal(y, want), f"m={m} k={k} n={n}: no-allocation result differs"
        ref = orc.matmul_f64(orc.Q4_1, x.float().cpu().numpy(), w.cpu().numpy(), n)
        rel = float(np.max(np.abs(y.float().cpu().numpy() - ref)) / np.max(np.abs(ref)))
        assert rel <= (8e-3 if yd == "bf16" else 1e-3)


def test_noalloc_int8_block_twice(ctx, orc):
    import torch
    import rlxq

    rng = np.random.default_rng(78)
    for (m, k, n) in ((32, 4096, 2048), (3, 2048, 1024)):
        announce(f"noalloc Int8Block m={m} k={k} n={n}")
        wq = torch.from_numpy(rng.integers(-127, 128, (k, n), dtype=np.int8)).cuda()
        sc = torch.from_numpy(rng.uniform(0.001, 0.01, n).astype(np.float32)).cuda()
        x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).cuda()
        want = ctx.dequant_matmul(x, wq, rlxq.INT8_BLOCK, n, group=k, scales=sc)
        y = torch.full((m, n), float("nan"), device="cuda")
        ctx.dequant_matmul_noalloc(x, wq, rlxq.INT8_BLOCK, n, group=k, scales=sc, y=y)
        torch.cuda.synchronize()
        assert torch.equal(y, want)


def test_noalloc_rejects_oversized_scratch(ctx, orc):
    import torch
    import rlxq

    rng = np.random.default_rng(79)
    m, k, n = 3072, 12288, 4096       # f32 output: the exact GEMM's f16 activations alone are 72 MiB
    w = _q4_1(orc, rng, n, k)
    x = _x(rng, m, k)
    y = torch.zeros((m, n), device="cuda")
    announce("noalloc oversized call is rejected before any launch")
    with pytest.raises(rlxq.RlxqError) as e:
        ctx.dequant_matmul_noalloc(x, w, rlxq.GGUF_Q4_1, n, y=y)
    assert e.value.status == rlxq.E_SCRATCH
    torch.cuda.synchronize()
    assert float(y.abs().max()) == 0.0
