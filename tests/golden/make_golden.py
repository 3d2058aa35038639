"""Writes the golden fixtures of the quantized-matmul path (tests/golden/*.npz).

The reference ships no golden vectors for this path (its tests compute their
oracle in-test from closed forms), so the fixtures here are frozen outputs of
this repository's CPU oracle (oracle/rlxq_oracle.c, float64 contraction) on
seeded inputs: M=4, K=256, N=64 per scheme, plus one grouped-expert case, one
MoE combine case, the int8 cases and the Qwen3 decode shapes' first rows.
Every array is numeric (loadable with numpy.load(allow_pickle=False)), and
MANIFEST.txt records each file's sha256.

    python tests/golden/make_golden.py      # rewrites the fixtures
"""
import hashlib
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))
from oracle import oracle as orc  # noqa: E402

M, K, N = 4, 256, 64


def x_for(rng, m, k):
    return rng.standard_normal((m, k)).astype(np.float32)


def gguf_case(scheme, seed):
    rng = np.random.default_rng(seed)
    packed = orc.synth(scheme, rng, N, K)
    x = x_for(rng, M, K)
    return dict(x=x, w=packed, dequant=orc.dequantize(scheme, packed, K), y=orc.matmul_f64(scheme, x, packed, N),
                scheme=np.int32(scheme), n=np.int32(N))


def mlx_case(bits, group, seed):
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 1 << bits, (N, K)).astype(np.uint32)
    wq = orc.mlx_pack(codes, bits)
    sc = rng.uniform(0.01, 0.1, (N, K // group)).astype(np.float32)
    bi = rng.uniform(-0.5, 0.1, (N, K // group)).astype(np.float32)
    x = x_for(rng, M, K)
    return dict(x=x, w=wq, scales=sc, biases=bi, dequant=orc.mlx_dequantize(wq, sc, bi, K, bits, group),
                y=orc.mlx_matmul_f64(x, wq, sc, bi, N, bits, group), bits=np.int32(bits), group=np.int32(group),
                n=np.int32(N))


def grouped_case(seed):
    rng = np.random.default_rng(seed)
    E, R = 4, 6
    bank = np.concatenate([orc.synth(orc.Q4_1, rng, N, K) for _ in range(E)])
    idx = np.array([(7 * r + 1) % E for r in range(R)], np.float32)
    x = x_for(rng, R, K)
    return dict(x=x, bank=bank, expert_idx=idx, y=orc.grouped_matmul_f64(orc.Q4_1, x, bank, idx, N, E),
                num_experts=np.int32(E), n=np.int32(N))


def moe_case(seed):
    rng = np.random.default_rng(seed)
    E, R, TOPK = 8, 3, 2
    bank = np.concatenate([orc.synth(orc.Q4_1, rng, N, K) for _ in range(E)])
    logits = rng.standard_normal((R, E)).astype(np.float32)
    ids, probs = orc.topk_softmax(logits, TOPK, renorm=True)
    x = x_for(rng, R, K)  # one row per token; every slot of a token sees it
    return dict(x=x, bank=bank, logits=logits, ids=ids, probs=probs,
                y=orc.moe_f64(orc.Q4_1, x, bank, ids, probs, N, E), num_experts=np.int32(E), n=np.int32(N))


def int8_case(seed):
    rng = np.random.default_rng(seed)
    x = x_for(rng, M, K)
    w = (rng.standard_normal((K, N)) * 0.05).astype(np.float32)
    qw, sw = orc.quantize_int8_col(w)
    qx, sx = orc.quantize_act_int8(x)
    zp = rng.standard_normal(N).astype(np.float32)
    return dict(x=x, qw=qw, sw=sw, qx=qx, sx=sx, zp=zp, y_w8a8=orc.w8a8_matmul(qx, sx, qw, sw),
                y_i8b=orc.int8_block_matmul_f64(x, qw, sw), y_i8b_zp=orc.int8_block_matmul_f64(x, qw, sw, zp))


CASES = {
    "q8_0": lambda: gguf_case(orc.Q8_0, 10),
    "q4_0": lambda: gguf_case(orc.Q4_0, 11),
    "q4_1": lambda: gguf_case(orc.Q4_1, 12),
    "mlx4_g32": lambda: mlx_case(4, 32, 13),
    "mlx8_g64": lambda: mlx_case(8, 64, 14),
    "grouped_q4_1": lambda: grouped_case(15),
    "moe_q4_1": lambda: moe_case(16),
    "int8": lambda: int8_case(17),
}


def main() -> int:
    lines = []
    for name, make in CASES.items():
        path = HERE / f"{name}.npz"
        np.savez_compressed(path, **make())
        lines.append(f"{hashlib.sha256(path.read_bytes()).hexdigest()}  {path.name}")
    (HERE / "MANIFEST.txt").write_text("\n".join(lines) + "\n")
    print("\n".join(lines))
    return 0


if __name__ == "__main__":
    sys.exit(main())
