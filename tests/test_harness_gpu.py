"""The bench_matmul_rlx harness flow (crates/bench_matmul_rlx/src/graph.rs:
75-150, weights.rs:20-33) on this library: its own weights file
(tests/golden/bench_matmul_rlx_model.safetensors, w [512, 512] and b [512])
read with rlxq_mlx_*, w packed to GGUF Q8_0 with the reference's encoder rule
(crates/rlx-flint/src/quant.rs:86-95; the op's weight is w transposed, since
the harness computes x . w), the DequantMatMul run on the GPU through the C
ABI, then the graph's Add and Relu.  Checked against the oracle's float64
contraction of the same Q8_0 weights (1e-3, the op's bar) and against the
harness's dense f32 graph (cosine > 0.9999, the tolerance the reference uses
for quantized matmuls, crates/rlx-models/tests/gguf_legacy_quant_matmul.rs:156)."""
from pathlib import Path

import numpy as np
import pytest

from conftest import announce

pytestmark = pytest.mark.gpu

FIXTURE = Path(__file__).resolve().parent / "golden" / "bench_matmul_rlx_model.safetensors"


def test_bench_matmul_rlx_flow(ctx, orc):
    import torch
    import rlxq

    f = rlxq.MlxFile(FIXTURE)
    w = f.read_f32("w")          # [in 512, out 512]: the harness computes x . w
    b = f.read_f32("b")
    f.close()
    wt = np.ascontiguousarray(w.T)                    # [out, in]: the op's W
    packed = orc.quantize(orc.Q8_0, wt)
    rng = np.random.default_rng(0)
    x = rng.standard_normal((32, 512)).astype(np.float32)   # the graph's input [1, 32, 512]
    announce("bench_matmul_rlx flow: Q8_0 512x512, 32 rows")
    xt = torch.from_numpy(x).cuda()
    y = ctx.dequant_matmul(xt, torch.from_numpy(packed).cuda(), rlxq.GGUF_Q8_0, 512)
    out = torch.relu(y + torch.from_numpy(b).cuda())
    torch.cuda.synchronize()
    got = out.cpu().numpy().astype(np.float64)
    lin = orc.matmul_f64(orc.Q8_0, x, packed, 512)
    want_q = np.maximum(lin + b, 0.0)
    assert float(np.max(np.abs(got - want_q)) / np.max(np.abs(want_q))) <= 1e-3
    dense = np.maximum(x.astype(np.float64) @ w.astype(np.float64) + b, 0.0)
    cos = float((got * dense).sum() / np.sqrt((got * got).sum() * (dense * dense).sum()))
    assert cos > 0.9999, cos
