"""Seeded random shapes across the dense op's routing boundaries (the M=1
register GEMVs and their K split, the multi-row GEMVs, batched decode from 5
rows, the prefill GEMM from 64 rows, split-K on every family), for every
GGUF format, f32 or bf16 activations and f32 or bf16 output, against the
oracle in float64 from the activations the kernel saw.  Bars: 1e-3 for f32
output, 2e-2 for bf16 output.  Each case names its kernel, so a failure
points at the path; the shapes are drawn once from a fixed seed."""
import numpy as np
import pytest

from conftest import announce
from test_gemv_gpu import _t, _x_as, rel_err, want_f64

pytestmark = pytest.mark.gpu

SCHEMES = {"q8_0": 1, "q4_0": 2, "q4_1": 3, "q4_k": 7, "q6_k": 8, "q5_k": 10, "q3_k": 11, "q2_k": 12, "q8_k": 13}
KQ = {7, 8, 10, 11, 12, 13}


def _cases(count=72, seed=20261202):
    rng = np.random.default_rng(seed)
    out = []
    names = list(SCHEMES)
    for i in range(count):
        name = names[i % len(names)]
        sch = SCHEMES[name]
        m = int(rng.choice([1, 1, 2, 3, 4, 5, 7, 16, 17, 33, 64, 65, 100, 256, 257, 300]))
        # (Q8_0 and Q4_0 rows of an odd block count are refused: K % 64)
        unit = 256 if sch in KQ else (64 if sch in (1, 2) else 32)
        k = unit * int(rng.integers(1, (12288 if m <= 4 else 4096) // unit + 1))
        n = int(rng.choice([3, 16, 77, 128, 300, 520, 1031, 2048]))
        xdt = str(rng.choice(["f32", "bf16"]))
        ydt = str(rng.choice(["f32", "f32", "bf16"]))
        out.append((name, m, k, n, xdt, ydt))
    return out


@pytest.mark.parametrize("case", _cases(), ids=lambda c: "-".join(map(str, c)))
def test_fuzz_dense(ctx, orc, case):
    import torch

    name, m, k, n, xdt, ydt = case
    sch = SCHEMES[name]
    announce(f"fuzz {case}")
    rng = np.random.default_rng(m * 100003 + k * 31 + n)
    packed = orc.synth(sch, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    xt, xv = _x_as(x, xdt)
    y = ctx.dequant_matmul(xt, _t(packed), sch, n, y_dtype=torch.bfloat16 if ydt == "bf16" else torch.float32)
    kern = ctx.last_kernel
    torch.cuda.synchronize()
    got = y.float().cpu().numpy()
    assert rel_err(got, want_f64(orc, sch, xv, packed, k)) <= (2e-2 if ydt == "bf16" else 1e-3), kern


@pytest.mark.parametrize("name", ["q8_0", "q4_0"])
def test_odd_block_rows_refused(ctx, orc, name):
    """Q8_0 / Q4_0 rows of an odd block count start 2 bytes off a dword every
    other row; the kernels read block pairs as dwords, so the call is refused
    before any launch (RLXQ_E_ALIGN), as the header documents."""
    import torch
    import rlxq

    sch = SCHEMES[name]
    k, n = 32 * 49, 8
    packed = orc.synth(sch, np.random.default_rng(5), n, k)
    y = torch.full((2, n), 7.0, device="cuda")
    with pytest.raises(rlxq.RlxqError) as e:
        ctx.dequant_matmul(_t(np.ones((2, k), np.float32)), _t(packed), sch, n, y=y)
    assert e.value.status == rlxq.E_ALIGN
    torch.cuda.synchronize()
    assert bool((y == 7.0).all())
