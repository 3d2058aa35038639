"""GGUF checkpoint -> device -> kernel, through the C ABI: rlxq_gguf_take_packed
gives the scheme and [out, in] shape (weight_loader.rs:1444-1486),
rlxq_gguf_upload streams the bytes through pinned staging onto the device
(high_level_runner.rs:474-499), and the kernels compute on them as stored.
Bars: the uploaded bytes equal the file's exactly; the products meet the
oracle at max|got - want| / max|want| <= 1e-3 (f32 accumulate)."""
import time

import numpy as np
import pytest

from conftest import announce
from rlxq.gguf_writer import F32, Q4_1, Q4_K, Q6_K, Q8_0, write_gguf
from test_gemv_gpu import _t, rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _u8(nbytes):
    import torch

    return torch.empty(nbytes, dtype=torch.uint8, device="cuda")


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory, orc):
    """A small checkpoint: one tensor per served scheme, an expert stack, an
    F32 norm, and a 71 MB Q8_0 tensor that takes three staging rounds."""
    import rlxq

    rng = np.random.default_rng(31)
    specs = [  # name, ggml type, scheme, out rows, in
        ("blk.0.attn_q.weight", Q4_1, rlxq.GGUF_Q4_1, 384, 1024),
        ("blk.0.ffn_up.weight", Q4_K, rlxq.GGUF_Q4_K, 256, 1536),
        ("blk.0.ffn_down.weight", Q6_K, rlxq.GGUF_Q6_K, 192, 768),
        ("output.weight", Q8_0, rlxq.GGUF_Q8_0, 16384, 4096),
    ]
    tensors, packed = [], {}
    for name, gt, sch, n, k in specs:
        w = orc.synth(sch, rng, n, k).ravel()
        packed[name] = (sch, n, k, w)
        tensors.append((name, gt, [k, n], w.tobytes()))
    E, n, k = 4, 320, 512
    bank = orc.synth_q4_1(rng, E * n, k).ravel()
    packed["blk.0.ffn_gate_exps.weight"] = (rlxq.GGUF_Q4_1, n, k, bank)
    tensors.append(("blk.0.ffn_gate_exps.weight", Q4_1, [k, n, E], bank.tobytes()))
    norm = rng.standard_normal(1024).astype(np.float32)
    tensors.append(("blk.0.attn_norm.weight", F32, [1024], norm.tobytes()))
    path = tmp_path_factory.mktemp("gguf") / "model.gguf"
    write_gguf(path, [("general.architecture", "str", "qwen3")], tensors, alignment=64)
    f = rlxq.GgufFile(path)
    yield f, packed, norm
    f.close()


@pytest.mark.parametrize("name", ["blk.0.attn_q.weight", "blk.0.ffn_up.weight", "blk.0.ffn_down.weight",
                                  "output.weight"])
def test_take_upload_matmul(ctx, orc, ckpt, name):
    import torch

    f, packed, _ = ckpt
    sch, n, k, w = packed[name]
    announce(f"gguf take+upload+matmul {name} scheme={sch} [{n}, {k}]")
    got = f.take_packed(name)
    assert got == (sch, [n, k], w.size)
    dev = _u8(w.size)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    f.upload(name, dev)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    print(f"upload {w.size / 1e6:.1f} MB in {dt * 1e3:.2f} ms ({w.size / dt / 1e9:.2f} GB/s)", flush=True)
    assert np.array_equal(dev.cpu().numpy(), w)
    rng = np.random.default_rng(5)
    m = 3
    x = rng.standard_normal((m, k)).astype(np.float32)
    y = ctx.dequant_matmul(_t(x), dev, sch, n)
    torch.cuda.synchronize()
    assert rel_err(y.cpu().numpy(), orc.matmul_f64(sch, x, w, n)) <= TOL


def test_expert_stack_upload_grouped(ctx, orc, ckpt):
    """A 3-D expert stack [in, out, E] as stored comes out as [E, out, in]
    and serves the grouped op directly."""
    import torch

    f, packed, _ = ckpt
    name = "blk.0.ffn_gate_exps.weight"
    sch, n, k, bank = packed[name]
    announce(f"gguf expert stack {name}")
    got = f.take_packed(name)
    assert got == (sch, [4, n, k], bank.size)
    dev = _u8(bank.size)
    f.upload(name, dev)
    rng = np.random.default_rng(6)
    x = rng.standard_normal((10, k)).astype(np.float32)
    idx = (np.arange(10) * 3 % 4).astype(np.float32)
    y = ctx.grouped_matmul(_t(x), dev, _t(idx), sch, n, 4)
    torch.cuda.synchronize()
    assert rel_err(y.cpu().numpy(), orc.grouped_matmul_f64(sch, x, bank, idx, n, 4)) <= TOL


def test_uncompressed_and_errors(ckpt):
    import rlxq
    import torch

    f, _, norm = ckpt
    name = "blk.0.attn_norm.weight"
    announce("gguf uncompressed tensor + upload errors")
    assert f.take_packed(name) is None
    dev = _u8(norm.size * 4)
    f.upload(name, dev)
    torch.cuda.synchronize()
    assert np.array_equal(dev.cpu().numpy().view(np.float32), norm)
    with pytest.raises(rlxq.RlxqError) as e:
        f.upload(name, _u8(norm.size * 4 - 1))
    assert e.value.status == rlxq.E_SHAPE
    with pytest.raises(rlxq.RlxqError) as e:
        f.upload("missing.weight", dev)
    assert e.value.status == rlxq.E_NOTFOUND
