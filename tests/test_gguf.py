"""The GGUF reader (rlxq_gguf_*), on the CPU.

Pinned two ways:
- against the reference's own fixture, tests/golden/bonsai2_manifest.gguf:
  a byte copy of crates/rlx-qwen35/tests/fixtures/bonsai2_manifest.gguf, the
  real header of a published 27B checkpoint with its 851 tensor infos
  (crates/rlx-qwen35/tests/bonsai2_manifest.rs:1-10).  Every figure asserted
  below is one the reference's tests assert on that file (:29-130) through
  its GGUF parser (external crate rlx_gguf ^0.2.19), so a mis-read string
  length, array, dimension list or alignment fails here;
- against files written from the published layout (rlxq/gguf_writer.py),
  for what that header does not hold: tensor data, alignment other than 32,
  version 2, the packed-take rules and every error path.
"""
import hashlib
from pathlib import Path

import numpy as np
import pytest

from rlxq.gguf_writer import BF16, F16, F32, Q2_K, Q3_K, Q4_0, Q4_1, Q4_K, Q5_K, Q6_K, Q8_0, Q8_K, gguf_bytes, write_gguf

FIXTURE = Path(__file__).parent / "golden" / "bonsai2_manifest.gguf"
FIXTURE_SHA256 = "a5f3ba541001c302e16a2005bb5aa7d4464ca71ad384f109cbc3a9d2ecdc7726"


@pytest.fixture(scope="module")
def bonsai():
    import rlxq

    f = rlxq.GgufFile(FIXTURE)
    yield f
    f.close()


# ------------------------------------------------- the reference's fixture
def test_fixture_is_the_reference_copy():
    assert hashlib.sha256(FIXTURE.read_bytes()).hexdigest() == FIXTURE_SHA256


def test_bonsai_tensor_infos(bonsai):
    """bonsai2_manifest.rs:1-10 (851 tensor infos) and :29-50 (402 tensors
    of ggml type 143, token_embd among them; output.weight separate :68)."""
    assert bonsai.version == 3
    assert len(bonsai.tensors) == 851
    assert sum(t.dtype == 143 for t in bonsai.tensors.values()) == 402
    assert bonsai.get("token_embd.weight").dtype == 143
    assert bonsai.get("output.weight") is not None
    assert bonsai.get("no.such.tensor") is None


def test_bonsai_config_keys(bonsai):
    """The values Qwen35Config::from_gguf reads (crates/rlx-qwen35/src/
    config.rs:128-230) and bonsai2_manifest.rs:52-69 asserts."""
    m = bonsai.meta
    assert m("general.architecture") == "qwen35"
    assert m("qwen35.block_count") == 64
    assert m("qwen35.embedding_length") == 5120
    assert m("qwen35.feed_forward_length") == 17408
    assert m("qwen35.attention.head_count") == 24
    assert m("qwen35.attention.head_count_kv") == 4
    assert m("qwen35.full_attention_interval") == 4
    assert m("qwen35.ssm.state_size") == 128
    assert m("qwen35.ssm.group_count") == 16
    assert m("qwen35.ssm.time_step_rank") == 48
    assert m("qwen35.ssm.inner_size") == 6144
    assert m("qwen35.rope.dimension_sections") == [11, 11, 10, 0]
    with pytest.raises(KeyError):
        m("qwen35.no_such_key")


def test_bonsai_hadamard_block(bonsai):
    """bonsai2_manifest.rs:71-109 through PrismHadamard::from_gguf
    (crates/rlx-qwen35/src/prism_hadamard.rs:91-160): block size 1024, 401
    folded weights, token_embd inverse-only, output folded, every folded
    weight a real tensor whose input width the block divides, and sign
    vectors of widths 5120 / 6144 / 17408, all +-1 and none all +1."""
    m = bonsai.meta
    assert m("prism.hadamard.block_size") == 1024
    folded = m("prism.hadamard.weight_names")
    assert len(folded) == len(set(folded)) == 401
    assert m("prism.hadamard.inverse_weight_names") == ["token_embd.weight"]
    assert "token_embd.weight" not in folded and "output.weight" in folded
    for name in folded:
        t = bonsai.get(name)
        assert t is not None and t.shape[0] % 1024 == 0, name
    widths = m("prism.hadamard.sign_widths")
    assert widths == [5120, 6144, 17408]
    signs = np.array(m("prism.hadamard.sign_values"))
    assert signs.size == sum(widths)
    assert set(np.unique(signs)) <= {-1, 1}
    for seg in np.split(signs, np.cumsum(widths)[:-1]):
        assert (seg < 0).any()


def test_bonsai_every_ternary_weight_accounted_for(bonsai):
    """bonsai2_manifest.rs:111-130: every type-143 tensor is folded or
    inverse."""
    folded = set(bonsai.meta("prism.hadamard.weight_names"))
    inverse = set(bonsai.meta("prism.hadamard.inverse_weight_names"))
    assert [t.name for t in bonsai.tensors.values() if t.dtype == 143 and t.name not in folded | inverse] == []


def test_bonsai_data_layout(bonsai):
    """The header ends at byte 178842 (the file is the header alone); with no
    general.alignment the data section starts at the next multiple of 32.
    Offsets are aligned, and no tensor of a known layout (F32, BF16) runs
    into the next one."""
    import rlxq

    assert FIXTURE.stat().st_size == 178842
    assert bonsai.data_offset == 178848
    ts = sorted(bonsai.tensors.values(), key=lambda t: t.offset)
    assert all((t.offset - bonsai.data_offset) % 32 == 0 for t in ts)
    for a, b in zip(ts, ts[1:]):
        if a.nbytes >= 0:
            assert a.offset + a.nbytes <= b.offset, a.name
    norm = bonsai.get("output_norm.weight")
    assert norm.dtype == 0 and norm.shape == [5120] and norm.nbytes == 5120 * 4
    bf = [t for t in ts if t.dtype == BF16]
    assert len(bf) == 96 and all(t.nbytes == 2 * int(np.prod(t.shape)) for t in bf)
    assert bonsai.get("token_embd.weight").nbytes == -1   # type 143: no fixed layout here
    with pytest.raises(rlxq.RlxqError) as e:
        bonsai.read("output_norm.weight")
    assert e.value.status == rlxq.E_IO and "past the end" in str(e.value)


# --------------------------------------------------------- written files
def _blob(nbytes, seed):
    return np.random.default_rng(seed).integers(0, 256, nbytes, dtype=np.uint8).tobytes()


# (name, ggml type, dims innermost first, bytes per block, elements per block)
LAYOUT = [
    ("blk.0.attn_q.weight", Q4_1, [256, 48], 20, 32),
    ("blk.0.ffn_down.weight", Q8_0, [96, 64], 34, 32),
    ("blk.0.attn_k.weight", Q4_0, [64, 16], 18, 32),
    ("blk.0.ffn_up.weight", Q4_K, [512, 24], 144, 256),
    ("blk.0.ffn_gate.weight", Q6_K, [256, 40], 210, 256),
    ("blk.0.ffn_gate_exps.weight", Q4_1, [64, 24, 3], 20, 32),
    ("blk.0.attn_norm.weight", F32, [64], 4, 1),
    ("token_embd.weight", F16, [32, 10], 2, 1),
    ("blk.1.attn_q.weight", Q5_K, [256, 8], 176, 256),
    ("output.weight", BF16, [32, 7], 2, 1),
    ("blk.1.attn_k.weight", 6, [64, 4], 22, 32),          # Q5_0: not served, stays unpacked
    ("blk.1.ffn_up.weight", Q3_K, [256, 6], 110, 256),
    ("blk.1.ffn_down.weight", Q2_K, [512, 3], 84, 256),
    ("blk.1.ffn_gate.weight", Q8_K, [256, 5], 292, 256),
]


def _tensors():
    out = []
    for i, (name, gt, dims, bb, be) in enumerate(LAYOUT):
        n = int(np.prod(dims)) // be * bb
        out.append((name, gt, dims, _blob(n, i)))
    return out


META = [
    ("general.architecture", "str", "qwen3"),
    ("general.name", "str", "tést"),
    ("qwen3.block_count", "u32", 2),
    ("qwen3.context_length", "u64", 40960),
    ("qwen3.rope.freq_base", "f32", 1000000.0),
    ("qwen3.eps", "f64", 1e-6),
    ("qwen3.flag", "bool", True),
    ("qwen3.i8", "i8", -5),
    ("qwen3.i16", "i16", -300),
    ("qwen3.u16", "u16", 65535),
    ("qwen3.i32", "i32", -70000),
    ("qwen3.i64", "i64", -(1 << 40)),
    ("qwen3.u8", "u8", 200),
    ("tokenizer.ggml.tokens", "arr", ("str", ["a", "bc", "", "ü"])),
    ("qwen3.sections", "arr", ("i32", [3, -1, 4])),
    ("qwen3.scales", "arr", ("f32", [0.5, 1.5])),
]


@pytest.mark.parametrize("version,alignment", [(3, None), (2, None), (3, 64), (3, 8)])
def test_written_file_round_trip(tmp_path, version, alignment):
    import rlxq

    tensors = _tensors()
    path = tmp_path / "m.gguf"
    offsets = write_gguf(path, META, tensors, version=version, alignment=alignment)
    f = rlxq.GgufFile(path)
    assert f.version == version
    assert len(f.tensors) == len(tensors)
    for name, gt, dims, data in tensors:
        t = f.get(name)
        assert (t.dtype, t.shape, t.offset, t.nbytes) == (gt, dims, offsets[name], len(data)), name
        assert f.read(name).tobytes() == data, name
    assert f.meta("general.name") == "tést"
    assert f.meta("qwen3.block_count") == 2 and f.meta("qwen3.context_length") == 40960
    assert f.meta("qwen3.rope.freq_base") == 1000000.0 and f.meta("qwen3.eps") == 1e-6
    assert f.meta("qwen3.flag") is True
    assert [f.meta(f"qwen3.{k}") for k in ("i8", "i16", "u16", "i32", "i64", "u8")] == \
        [-5, -300, 65535, -70000, -(1 << 40), 200]
    assert f.meta("tokenizer.ggml.tokens") == ["a", "bc", "", "ü"]
    assert f.meta("qwen3.sections") == [3, -1, 4] and f.meta("qwen3.scales") == [0.5, 1.5]
    if alignment:
        assert f.meta("general.alignment") == alignment
    assert f.data_offset % (alignment or 32) == 0
    f.close()


def test_take_packed_rules(tmp_path):
    """take_packed (weight_loader.rs:1444-1486): packed types give their
    scheme and the shape reversed to outermost first and are taken once;
    a second take fails ("weight already taken"); uncompressed and unserved
    types give None and stay untaken; a missing name is "tensor missing"."""
    import rlxq

    path = tmp_path / "m.gguf"
    write_gguf(path, META, _tensors())
    f = rlxq.GgufFile(path)
    want = {
        "blk.0.attn_q.weight": (rlxq.GGUF_Q4_1, [48, 256], 48 * 8 * 20),
        "blk.0.ffn_down.weight": (rlxq.GGUF_Q8_0, [64, 96], 64 * 3 * 34),
        "blk.0.attn_k.weight": (rlxq.GGUF_Q4_0, [16, 64], 16 * 2 * 18),
        "blk.0.ffn_up.weight": (rlxq.GGUF_Q4_K, [24, 512], 24 * 2 * 144),
        "blk.0.ffn_gate.weight": (rlxq.GGUF_Q6_K, [40, 256], 40 * 210),
        "blk.0.ffn_gate_exps.weight": (rlxq.GGUF_Q4_1, [3, 24, 64], 3 * 24 * 2 * 20),
        "blk.1.attn_q.weight": (rlxq.GGUF_Q5_K, [8, 256], 8 * 176),
        "blk.1.ffn_up.weight": (rlxq.GGUF_Q3_K, [6, 256], 6 * 110),
        "blk.1.ffn_down.weight": (rlxq.GGUF_Q2_K, [3, 512], 3 * 2 * 84),
        "blk.1.ffn_gate.weight": (rlxq.GGUF_Q8_K, [5, 256], 5 * 292),
    }
    for name, w in want.items():
        assert f.get(name).scheme == w[0]
        assert f.take_packed(name) == w, name
        with pytest.raises(rlxq.RlxqError) as e:
            f.take_packed(name)
        assert e.value.status == rlxq.E_TAKEN and "already taken" in str(e.value)
        assert f.read(name).size == w[2]   # reading bytes does not depend on the taken mark
    for name in ("blk.0.attn_norm.weight", "token_embd.weight", "output.weight", "blk.1.attn_k.weight"):
        assert f.get(name).scheme == 0
        assert f.take_packed(name) is None
        assert f.take_packed(name) is None   # not taken
    with pytest.raises(rlxq.RlxqError) as e:
        f.take_packed("blk.9.attn_q.weight")
    assert e.value.status == rlxq.E_NOTFOUND and "tensor missing" in str(e.value)
    f.close()


def test_block_layouts_match_the_kernels(tmp_path):
    """Packed bytes per row agree with rlxq_row_bytes for the schemes the
    kernels read (Q4_0 18, Q4_1 20, Q8_0 34 B per 32; Q4_K 144, Q6_K 210,
    Q5_K 176, Q3_K 110, Q2_K 84, Q8_K 292 B per 256: block_q6_K is ql[128] +
    qh[64] + scales[16] + d, the reference's probe block,
    weight_loader.rs:573-581)."""
    import rlxq

    path = tmp_path / "m.gguf"
    write_gguf(path, [], _tensors())
    f = rlxq.GgufFile(path)
    for t in f.tensors.values():
        if t.scheme:
            rows = int(np.prod(t.shape[1:]))
            assert rlxq.lib().rlxq_row_bytes(t.scheme, t.shape[0]) * rows == t.nbytes, t.name
    f.close()


def _expect_open_error(path, status, text):
    import rlxq

    with pytest.raises(rlxq.RlxqError) as e:
        rlxq.GgufFile(path)
    assert e.value.status == status and text in str(e.value), str(e.value)


def test_open_errors(tmp_path):
    import rlxq

    good, _ = gguf_bytes(META, _tensors())
    cases = {
        "missing": None,
        "magic": gguf_bytes(META, _tensors(), magic=b"GGML")[0],
        "v1": gguf_bytes(META, _tensors(), version=1)[0],
        "truncated": good[:200],
        "empty": b"",
        "align3": gguf_bytes(META, _tensors(), alignment=3)[0],
        "dup_tensor": gguf_bytes([], [_tensors()[0], _tensors()[0]])[0],
        "dup_key": gguf_bytes([META[0], META[0]], [])[0],
        "dims5": gguf_bytes([], [("x", F32, [1, 1, 1, 1, 2], b"\0" * 8)])[0],
    }
    want = {
        "missing": (rlxq.E_IO, "cannot open"),
        "magic": (rlxq.E_FORMAT, "bad magic"),
        "v1": (rlxq.E_FORMAT, "unsupported version 1"),
        "truncated": (rlxq.E_FORMAT, "truncated"),
        "empty": (rlxq.E_FORMAT, "bad magic"),
        "align3": (rlxq.E_FORMAT, "power of two"),
        "dup_tensor": (rlxq.E_FORMAT, "duplicate tensor"),
        "dup_key": (rlxq.E_FORMAT, "duplicate key"),
        "dims5": (rlxq.E_FORMAT, "5 dims"),
    }
    for name, data in cases.items():
        p = tmp_path / f"{name}.gguf"
        if data is not None:
            p.write_bytes(data)
        _expect_open_error(p, *want[name])
    # an 8-byte element type whose byte size wraps 64 bits: elements below
    # 2^62, elements x 8 past 2^64 (it would wrap to 8 bytes)
    p = tmp_path / "wrap.gguf"
    p.write_bytes(gguf_bytes([], [("w", 28, [(1 << 61) + 1], b"\0" * 8)])[0])
    _expect_open_error(p, rlxq.E_FORMAT, "too large")
    # a huge count is rejected before anything is allocated for it
    bad = bytearray(good)
    bad[8:16] = (1 << 60).to_bytes(8, "little")
    p = tmp_path / "count.gguf"
    p.write_bytes(bytes(bad))
    _expect_open_error(p, rlxq.E_FORMAT, "counts exceed")


def test_data_errors(tmp_path):
    """A file cut inside the data section opens (the header is whole) but
    the cut tensor cannot be read; a short destination is refused."""
    import rlxq

    tensors = _tensors()
    data, offsets = gguf_bytes(META, tensors)
    last = tensors[-1]
    p = tmp_path / "cut.gguf"
    p.write_bytes(data[: offsets[last[0]] + 5])
    f = rlxq.GgufFile(p)
    assert f.read(tensors[0][0]).tobytes() == tensors[0][3]
    with pytest.raises(rlxq.RlxqError) as e:
        f.read(last[0])
    assert e.value.status == rlxq.E_IO
    buf = np.empty(3, np.uint8)
    rc = rlxq.lib().rlxq_gguf_read(f.h, tensors[0][0].encode(), buf.ctypes.data, buf.size)
    assert rc == rlxq.E_SHAPE
    with pytest.raises(rlxq.RlxqError) as e:
        f.take_packed("nope")
    assert e.value.status == rlxq.E_NOTFOUND
    f.close()
