"""CPU tests of the MLX checkpoint reader (rlxq_mlx_*): the safetensors
layout pinned on the reference's own harness weights
(crates/bench_matmul_rlx/weights/model.safetensors, copied byte for byte to
tests/golden/bench_matmul_rlx_model.safetensors: tensors "w" F32 [512, 512]
and "b" F32 [512] as crates/bench_matmul_rlx/src/graph.rs:88-118 binds them,
read as little-endian f32 as src/weights.rs:20-33 does), and take_packed_mlx's
rules (weight_loader.rs:906-1012, load_proj standard_decoder.rs:590-645) on
written mlx-community style checkpoints."""
import hashlib
import json
import struct
from pathlib import Path

import numpy as np
import pytest

import rlxq
from rlxq.safetensors_writer import safetensors_bytes, write_mlx_dir, write_safetensors

FIXTURE = Path(__file__).resolve().parent / "golden" / "bench_matmul_rlx_model.safetensors"
FIXTURE_SHA256 = "e48ef101d07987c9d4d2763d3b4b96db1b49a5d278fe2721f7e83bba939d6cdb"


def test_harness_fixture():
    assert hashlib.sha256(FIXTURE.read_bytes()).hexdigest() == FIXTURE_SHA256
    f = rlxq.MlxFile(FIXTURE)
    assert set(f.tensors) == {"w", "b"}
    assert f.tensors["w"]["dtype"] == "F32" and f.tensors["w"]["shape"] == [512, 512]
    assert f.tensors["b"]["dtype"] == "F32" and f.tensors["b"]["shape"] == [512]
    assert f.quantization == (0, 0, rlxq.MLX_MODE_NONE)
    raw = FIXTURE.read_bytes()
    n = struct.unpack("<Q", raw[:8])[0]
    for name in ("w", "b"):
        t = f.tensors[name]
        got = f.read(name)
        assert got.tobytes() == raw[t["offset"]:t["offset"] + t["nbytes"]]
        assert t["offset"] >= 8 + n
        v = f.read_f32(name)
        assert np.array_equal(v.ravel().view(np.uint32), got.view(np.uint32))
        assert np.all(np.isfinite(v))
    with pytest.raises(rlxq.RlxqError) as e:
        f.take_packed("w")                      # no "w.weight": not an MLX Linear
    assert e.value.status == rlxq.E_NOTFOUND
    f.close()


def _bf16(a):
    return (np.asarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def _linear(rng, n, k, bits, group, slab="bf16"):
    if 32 % bits:   # (a packing the kernels do not read: only its shape matters)
        wq = rng.integers(0, 1 << 32, (n, k * bits // 32), dtype=np.uint64).astype(np.uint32)
    else:
        wq = rlxq_pack(rng.integers(0, 1 << bits, (n, k)).astype(np.uint32), bits)
    sc = rng.uniform(0.01, 0.1, (n, k // group)).astype(np.float32)
    bi = rng.uniform(-0.5, 0.1, (n, k // group)).astype(np.float32)
    if slab == "bf16":
        return wq, _bf16(sc), _bf16(bi)
    if slab == "f16":
        return wq, sc.astype(np.float16), bi.astype(np.float16)
    return wq, sc, bi


def rlxq_pack(codes, bits):
    """u32 words, codes LSB first (the MLX packing, mlx_affine.rs:272-288)."""
    per = 32 // bits
    c = codes.reshape(codes.shape[0], -1, per).astype(np.uint64)
    w = np.zeros(c.shape[:2], np.uint64)
    for i in range(per):
        w |= c[:, :, i] << np.uint64(bits * i)
    return w.astype(np.uint32)


def _ckpt(tmp_path, index=False):
    rng = np.random.default_rng(3)
    t = {}
    bf = []
    for key, (n, k, bits, g, slab) in {
        "model.layers.0.mlp.down_proj": (64, 256, 4, 64, "bf16"),
        "model.layers.0.self_attn.q_proj": (32, 128, 8, 32, "bf16"),    # per-layer override
        "model.layers.0.self_attn.k_proj": (32, 128, 4, 64, "f16"),
        "model.layers.0.mlp.gate_proj": (32, 128, 3, 64, "bf16"),       # 3-bit: not read by the kernels
    }.items():
        wq, sc, bi = _linear(rng, n, k, bits, g, slab)
        t[key + ".weight"], t[key + ".scales"], t[key + ".biases"] = wq, sc, bi
        if slab == "bf16":
            bf += [key + ".scales", key + ".biases"]
    t["model.embed_tokens.weight"] = rng.standard_normal((16, 128)).astype(np.float16)
    t["lm_head.weight"] = rng.integers(0, 1 << 32, (16, 16), dtype=np.uint64).astype(np.uint32)
    t["lm_head.scales"] = _bf16(np.ones((16, 2)))
    t["lm_head.biases"] = _bf16(np.zeros((16, 2)))
    bf += ["lm_head.scales", "lm_head.biases"]
    q = {"group_size": 64, "bits": 4, "model.layers.0.self_attn.q_proj": {"group_size": 32, "bits": 8},
         "model.layers.0.mlp.gate_proj": {"group_size": 64, "bits": 3}, "lm_head": False}
    names = sorted(t)
    shards = [{n: t[n] for n in names[: len(names) // 2]}, {n: t[n] for n in names[len(names) // 2:]}]
    write_mlx_dir(tmp_path, shards if index else [t], q, index=index, bf16=tuple(bf))
    return t


@pytest.mark.parametrize("index", [False, True])
def test_take_packed_rules(tmp_path, index):
    t = _ckpt(tmp_path, index)
    f = rlxq.MlxFile(tmp_path)
    assert f.quantization == (4, 64, rlxq.MLX_MODE_AFFINE)
    assert len(f.tensors) == len(t)
    p = f.take_packed("model.layers.0.mlp.down_proj")
    assert p["scheme"] == rlxq.MLX_AFFINE4 and (p["n"], p["k"], p["group_size"]) == (64, 256, 64)
    assert p["slab_dtype"] == "BF16" and p["biases"] == "model.layers.0.mlp.down_proj.biases"
    assert p["codes_nbytes"] == 64 * 256 // 2 and p["scales_nbytes"] == 64 * 4 * 2
    assert np.array_equal(f.read(p["codes"]).view(np.uint32).reshape(64, 32), t[p["codes"]])
    with pytest.raises(rlxq.RlxqError) as e:
        f.take_packed("model.layers.0.mlp.down_proj")
    assert e.value.status == rlxq.E_TAKEN
    q = f.take_packed("model.layers.0.self_attn.q_proj")        # the per-layer entry
    assert q["scheme"] == rlxq.MLX_AFFINE8 and (q["k"], q["group_size"]) == (128, 32)
    k = f.take_packed("model.layers.0.self_attn.k_proj")
    assert k["scheme"] == rlxq.MLX_AFFINE4 and k["slab_dtype"] == "F16"
    sc = f.read_f32(k["scales"])
    assert np.array_equal(sc, t[k["scales"]].astype(np.float32))   # f16 -> f32 exact
    bf = f.read_f32("model.layers.0.mlp.down_proj.scales")
    assert np.array_equal(bf.view(np.uint32) >> 16, t["model.layers.0.mlp.down_proj.scales"].astype(np.uint32))
    assert f.take_packed("model.layers.0.mlp.gate_proj") is None   # 3-bit: the caller's dense path
    assert f.take_packed("lm_head") is None                        # switched off by `false`
    assert f.take_packed("model.embed_tokens") is None   # F16 .weight, no .scales: dense
    f.close()


def test_mxfp4_checkpoint(tmp_path):
    rng = np.random.default_rng(5)
    n, k = 48, 256
    codes = rng.integers(0, 256, (n, k // 2), dtype=np.uint8).view(np.uint32)   # [n, k/8] words
    eb = rng.integers(115, 126, (n, k // 32), dtype=np.uint8)
    write_mlx_dir(tmp_path, [{"m.weight": codes.reshape(n, k // 8), "m.scales": eb}],
                  {"group_size": 32, "bits": 4, "mode": "mxfp4"})
    f = rlxq.MlxFile(tmp_path)
    assert f.quantization == (4, 32, rlxq.MLX_MODE_MXFP4)
    p = f.take_packed("m")
    assert p["scheme"] == rlxq.MLX_MXFP4 and p["biases"] is None and p["slab_dtype"] == "U8"
    assert (p["n"], p["k"]) == (n, k)
    f.close()


def test_single_file_and_errors(tmp_path):
    good = safetensors_bytes({"a": np.arange(6, dtype=np.float32).reshape(2, 3)}, {"x": "y"})
    (tmp_path / "one.safetensors").write_bytes(good)
    f = rlxq.MlxFile(tmp_path / "one.safetensors")
    assert f.tensors["a"]["shape"] == [2, 3]
    assert np.array_equal(f.read_f32("a"), np.arange(6, dtype=np.float32).reshape(2, 3))
    f.close()
    n = struct.unpack("<Q", good[:8])[0]
    hdr = json.loads(good[8:8 + n])

    def with_header(h, tail=None):
        b = json.dumps(h).encode()
        data = good[8 + n:] if tail is None else tail
        return struct.pack("<Q", len(b)) + b + data

    bad_off = dict(hdr, a=dict(hdr["a"], data_offsets=[0, 28]))
    bad_dt = dict(hdr, a=dict(hdr["a"], dtype="Q4"))
    bad_size = dict(hdr, a=dict(hdr["a"], shape=[2, 4]))
    cases = {
        "truncated_len": (good[:5], rlxq.E_FORMAT, "header length"),
        "len_past_end": (struct.pack("<Q", 1 << 40) + good[8:], rlxq.E_FORMAT, "does not fit"),
        "not_json": (struct.pack("<Q", 4) + b"{a:1" + good[12:], rlxq.E_FORMAT, "JSON"),
        "offsets": (with_header(bad_off), rlxq.E_FORMAT, "data_offsets"),
        "dtype": (with_header(bad_dt), rlxq.E_FORMAT, "unknown dtype"),
        "size": (with_header(bad_size), rlxq.E_FORMAT, "do not match"),
        "cut_data": (good[:-4], rlxq.E_FORMAT, "data_offsets"),
    }
    for name, (data, status, msg) in cases.items():
        p = tmp_path / f"{name}.safetensors"
        p.write_bytes(data)
        with pytest.raises(rlxq.RlxqError) as e:
            rlxq.MlxFile(p)
        assert e.value.status == status and msg in str(e.value), (name, str(e.value))
    with pytest.raises(rlxq.RlxqError) as e:
        rlxq.MlxFile(tmp_path / "missing")
    assert e.value.status == rlxq.E_IO
    (tmp_path / "empty").mkdir()
    with pytest.raises(rlxq.RlxqError) as e:
        rlxq.MlxFile(tmp_path / "empty")
    assert e.value.status == rlxq.E_NOTFOUND


@pytest.mark.parametrize("cfg", [
    {"quantization_config": {"quant_method": "gptq", "bits": 4, "group_size": 128, "desc_act": False}},
    {"quantization_config": {"quant_method": "fp8", "weight_block_size": [128, 128], "fmt": "e4m3"}},
    {"quantization_config": {"quant_method": "mxfp4", "modules_to_not_convert": ["lm_head"]}},
    {"quantization": {"mode": "none"}},
    {"quantization": 4},
], ids=["gptq", "fp8", "gpt-oss", "no-bits", "not-object"])
def test_non_mlx_quantization_blocks_read_as_unquantized(tmp_path, cfg):
    """Only an mlx-lm `quantization` object with bits or group_size marks an
    MLX checkpoint (dir_is_mlx_quant, crates/rlx-models-core/src/
    weight_registry.rs:27-41); GPTQ / AWQ / fp8 / gpt-oss `quantization_config`
    blocks and other `quantization` values leave the tensors unquantized."""
    rng = np.random.default_rng(1)
    wq = rng.integers(0, 1 << 32, (32, 16), dtype=np.uint64).astype(np.uint32)
    (tmp_path / "model.safetensors").write_bytes(
        safetensors_bytes({"m.weight": wq, "m.scales": _bf16(np.ones((32, 2))), "m.biases": _bf16(np.zeros((32, 2)))}))
    (tmp_path / "config.json").write_text(json.dumps(dict(cfg, model_type="qwen3")))
    f = rlxq.MlxFile(tmp_path)
    assert f.quantization == (0, 0, rlxq.MLX_MODE_NONE)
    assert f.take_packed("m") is None
    assert f.tensors["m.weight"]["shape"] == [32, 16]
    f.close()
