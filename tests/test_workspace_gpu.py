"""Context scratch across HIP graph capture: a buffer that growth replaces
stays valid for graphs captured before (one used under capture is retired,
not freed, until rlxq_release_stream / rlxq_destroy), reserve / release work
per stream, and an ascending run of sizes grows the scratch geometrically
and frees the replaced buffers once their work is done."""
import numpy as np
import pytest

from conftest import announce

pytestmark = pytest.mark.gpu


def test_graph_replay_after_scratch_growth(ctx, orc):
    import torch
    import rlxq

    rng = np.random.default_rng(31)
    m, k, n = 16, 4096, 1024          # batched decode: prepared activations in the scratch
    packed = orc.synth_q4_1(rng, n, k)
    w = torch.from_numpy(packed).cuda()
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).cuda().to(torch.bfloat16)
    want = orc.matmul_f64(orc.Q4_1, x.float().cpu().numpy(), packed, n)
    s = torch.cuda.Stream()
    announce("workspace: eager call on a side stream")
    with torch.cuda.stream(s):
        y_eager = ctx.dequant_matmul(x, w, rlxq.GGUF_Q4_1, n)
    s.synchronize()
    size0 = ctx.workspace_bytes(stream=s.cuda_stream)
    assert size0 > 0
    rel = float(np.max(np.abs(y_eager.cpu().numpy() - want)) / np.max(np.abs(want)))
    assert rel <= 1e-3

    announce("workspace: capture")
    y = torch.zeros((m, n), device="cuda")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        ctx.dequant_matmul(x, w, rlxq.GGUF_Q4_1, n, y=y)
    torch.cuda.synchronize()

    announce("workspace: grow the stream's scratch after the capture")
    with torch.cuda.stream(s):
        ctx.reserve_workspace(size0 + (48 << 20))
        xb = torch.from_numpy(rng.standard_normal((64, 12288)).astype(np.float32)).cuda().to(torch.bfloat16)
        wb = torch.from_numpy(orc.synth_q4_1(rng, 2048, 12288)).cuda()
        ctx.dequant_matmul(xb, wb, rlxq.GGUF_Q4_1, 2048)
    s.synchronize()
    assert ctx.workspace_bytes(stream=s.cuda_stream) >= size0 + (48 << 20)

    for r in range(3):
        announce(f"workspace: replay {r}")
        y.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, y_eager), f"replay {r} differs from the eager result"
        # eager work on the same stream between replays
        with torch.cuda.stream(s):
            ctx.dequant_matmul(x, w, rlxq.GGUF_Q4_1, n)
        s.synchronize()
    del g
    torch.cuda.synchronize()
    ctx.release_stream(stream=s.cuda_stream)
    assert ctx.workspace_bytes(stream=s.cuda_stream) == 0
    # a released stream gets fresh scratch on its next call
    with torch.cuda.stream(s):
        y2 = ctx.dequant_matmul(x, w, rlxq.GGUF_Q4_1, n)
    s.synchronize()
    assert torch.equal(y2, y_eager)
    ctx.release_stream(stream=s.cuda_stream)


def test_ascending_sizes_grow_geometrically_and_free_retired(ctx, orc):
    """A chunked-prefill-like run of ascending M on one stream (batched-decode
    kernels: prepared activations and split-K partials in the scratch): the
    scratch grows by at least half each time, so the count of growths stays
    logarithmic, and the buffers it replaced (never used under capture) are
    freed by later calls once their work has finished."""
    import torch
    import rlxq

    rng = np.random.default_rng(5)
    k, n = 12288, 256                 # small N, long K: split-K partials
    packed = orc.synth_q4_1(rng, n, k)
    w = torch.from_numpy(packed).cuda()
    s = torch.cuda.Stream()
    sp = s.cuda_stream
    sizes, growths = [], 0
    with torch.cuda.stream(s):
        for m in range(5, 257, 3):
            announce(f"workspace ascending m={m}")
            x = torch.randn((m, k), device="cuda").to(torch.bfloat16)
            ctx.dequant_matmul(x, w, rlxq.GGUF_Q4_1, n)
            b = ctx.workspace_bytes(stream=sp)
            if sizes and b > sizes[-1]:
                growths += 1
                assert b >= sizes[-1] * 3 // 2, (m, b, sizes[-1])
            sizes.append(b)
            # replaced buffers never exceed twice the live one
            assert ctx.workspace_retired_bytes(stream=sp) < 2 * b
    s.synchronize()
    assert growths <= 12, growths
    # once the stream's work is done, the next call frees every retired buffer
    with torch.cuda.stream(s):
        x = torch.randn((5, k), device="cuda").to(torch.bfloat16)
        y = ctx.dequant_matmul(x, w, rlxq.GGUF_Q4_1, n)
    s.synchronize()
    assert ctx.workspace_retired_bytes(stream=sp) == 0
    want = orc.matmul_f64(orc.Q4_1, x.float().cpu().numpy(), packed, n)
    assert float(np.max(np.abs(y.cpu().numpy() - want)) / np.max(np.abs(want))) <= 1e-3
    ctx.release_stream(stream=sp)
    assert ctx.workspace_retired_bytes(stream=sp) == 0
