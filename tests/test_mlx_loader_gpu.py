"""MLX checkpoints end to end on the GPU: a written mlx-community style
checkpoint is opened with rlxq_mlx_*, each packed Linear taken
(take_packed_mlx), its codes / scale / bias tensors uploaded as stored with
rlxq_mlx_upload, and the dense DequantMatMul run on them; the bytes on the
device equal the file's, and the outputs match the oracle's float64
contraction of the same codes and slabs within 1e-3 (f32 output)."""
import numpy as np
import pytest

from conftest import announce
from test_mlx_loader import _bf16, rlxq_pack

pytestmark = pytest.mark.gpu


def _dev_bytes(f, name):
    import torch

    t = torch.empty(f.tensors[name]["nbytes"], dtype=torch.uint8, device="cuda")
    f.upload(name, t)
    return t


def test_mlx_checkpoint_through_the_kernels(tmp_path, ctx, orc):
    import torch
    import rlxq
    from rlxq.safetensors_writer import write_mlx_dir

    rng = np.random.default_rng(11)
    specs = {"model.layers.0.mlp.down_proj": (96, 512, 4, 64), "model.layers.0.self_attn.o_proj": (64, 256, 8, 32),
             "model.layers.0.mlp.up_proj": (80, 256, 4, 128)}
    tensors, bf, truth = {}, [], {}
    for key, (n, k, bits, g) in specs.items():
        codes = rng.integers(0, 1 << bits, (n, k)).astype(np.uint32)
        wq = rlxq_pack(codes, bits)
        sc = _bf16(rng.uniform(0.01, 0.1, (n, k // g)))
        bi = _bf16(rng.uniform(-0.5, 0.1, (n, k // g)))
        tensors.update({key + ".weight": wq, key + ".scales": sc, key + ".biases": bi})
        bf += [key + ".scales", key + ".biases"]
        truth[key] = (wq, orc.bf16_bits_to_f32(sc), orc.bf16_bits_to_f32(bi))
    quant = {"group_size": 64, "bits": 4, "model.layers.0.self_attn.o_proj": {"group_size": 32, "bits": 8},
             "model.layers.0.mlp.up_proj": {"group_size": 128, "bits": 4}}
    write_mlx_dir(tmp_path, [tensors], quant, bf16=tuple(bf))
    f = rlxq.MlxFile(tmp_path)
    for key, (n, k, bits, g) in specs.items():
        announce(f"mlx checkpoint {key} bits={bits} group={g}")
        p = f.take_packed(key)
        assert (p["n"], p["k"], p["bits"], p["group_size"]) == (n, k, bits, g)
        w = _dev_bytes(f, p["codes"])
        sc = _dev_bytes(f, p["scales"]).view(torch.bfloat16)
        bi = _dev_bytes(f, p["biases"]).view(torch.bfloat16)
        torch.cuda.synchronize()
        assert np.array_equal(w.cpu().numpy(), f.read(p["codes"]))
        for xdt in (torch.float32, torch.bfloat16):
            x = torch.from_numpy(rng.standard_normal((3, k)).astype(np.float32)).cuda().to(xdt)
            y = ctx.dequant_matmul(x, w, p["scheme"], n, group=g, scales=sc, biases=bi)
            torch.cuda.synchronize()
            wq, s32, b32 = truth[key]
            wd = orc.mlx_dequantize(wq, s32, b32, k, bits, g).astype(np.float64)
            want = x.float().cpu().numpy().astype(np.float64) @ wd.T
            err = float(np.max(np.abs(y.cpu().numpy() - want)) / np.max(np.abs(want)))
            assert err <= 1e-3, (key, xdt, err)
    f.close()


def test_mxfp4_checkpoint_through_the_kernels(tmp_path, ctx, orc):
    import torch
    import rlxq
    from rlxq.safetensors_writer import write_mlx_dir

    rng = np.random.default_rng(12)
    n, k = 128, 512
    codes = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    eb = rng.integers(115, 126, (n, k // 32), dtype=np.uint8)
    write_mlx_dir(tmp_path, [{"m.weight": codes.view(np.uint32).reshape(n, k // 8), "m.scales": eb}],
                  {"group_size": 32, "bits": 4, "mode": "mxfp4"})
    f = rlxq.MlxFile(tmp_path)
    p = f.take_packed("m")
    announce("mlx checkpoint mxfp4")
    w = _dev_bytes(f, p["codes"])
    s = _dev_bytes(f, p["scales"])
    x = torch.from_numpy(rng.standard_normal((2, k)).astype(np.float32)).cuda().to(torch.bfloat16)
    y = ctx.dequant_matmul(x, w, rlxq.MLX_MXFP4, n, scales=s)
    torch.cuda.synchronize()
    want = x.float().cpu().numpy().astype(np.float64) @ orc.mxfp4_dequantize(codes, eb, n, k).T
    err = float(np.max(np.abs(y.cpu().numpy() - want)) / np.max(np.abs(want)))
    assert err <= 1e-3
    f.close()
