"""Builds librlxq.so (gfx950 code objects embedded) and the CPU oracle.

    python rlx-models_amd/build.py            # everything
    python rlx-models_amd/build.py --no-oracle

Outputs (git-ignored, they travel with the tree to the GPU box):
    rlx-models_amd/lib/librlxq.so        the product: C ABI of include/rlxq.h
    rlx-models_amd/lib/co/*.co           intermediate gfx950 code objects
    oracle/liboracle.so                  CPU restatement (tests/bench only)
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import hashlib
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
KDIR = PKG / "csrc" / "kernels"
HDIR = PKG / "csrc" / "host"
LIB = PKG / "lib"
CO = LIB / "co"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = str(ROCM / "bin" / "hipcc")

# Code objects the host library embeds (rlxq.cpp RLXQ_EMBED lines), with the
# number of parts each kernel file is compiled in (-DRLXQ_PART=i gives
# <name><i>.co; the parts build in parallel).  A name without a source file is
# embedded empty and skipped at load time.
CODE_OBJECTS = (("gemv", 6), ("misc", 1), ("gemm", 1), ("moe", 5), ("int8", 1), ("skinny", 1))

HIP_FLAGS = [
    "--genco", "--offload-arch=gfx950", "-O3", "-std=c++17",
    # No packed fp32 arithmetic (v_pk_*_f32) in any kernel: its forms have
    # given silent wrong results on this hardware pool.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd: list[str], what: str) -> None:
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"{what} failed ({r.returncode}):\n{' '.join(cmd)}\n{out}")


def _inputs_digest(src: Path, defs: list[str]) -> str:
    h = hashlib.sha256()
    h.update(" ".join([*HIP_FLAGS, *defs]).encode())
    for p in [src, *sorted(KDIR.glob("*.h"))]:
        h.update(p.name.encode())
        h.update(p.read_bytes())
    return h.hexdigest()


def build_code_objects(cached: bool = False) -> None:
    """hipcc --genco of every kernel part.  With cached=True (development
    only) a part whose source, kernel headers and flags are unchanged since its
    last build is kept."""
    CO.mkdir(parents=True, exist_ok=True)
    jobs = []
    for name, parts in CODE_OBJECTS:
        src = KDIR / f"{name}.hip"
        for i in range(parts):
            dst = CO / (f"{name}{i}.co" if parts > 1 else f"{name}.co")
            if not src.exists():
                dst.write_bytes(b"")
                continue
            defs = [f"-DRLXQ_PART={i}"] if parts > 1 else []
            stamp = dst.with_suffix(".sha256")
            digest = _inputs_digest(src, defs)
            if cached and dst.exists() and stamp.exists() and stamp.read_text() == digest:
                continue
            jobs.append((dst.stem, [HIPCC, *HIP_FLAGS, *defs, "-I", str(KDIR), str(src), "-o", str(dst)], stamp, digest))

    def one(job):
        stem, cmd, stamp, digest = job
        stamp.unlink(missing_ok=True)
        _run(cmd, f"hipcc {stem}")
        stamp.write_text(digest)

    with cf.ThreadPoolExecutor(max_workers=min(8, max(1, len(jobs)))) as ex:
        for f in [ex.submit(one, j) for j in jobs]:
            f.result()


def build_host_hip_objects() -> list[str]:
    """Host translation units that also hold device data (noalloc.hip: the
    static scratch array of the no-allocation entry point), compiled by hipcc
    into position-independent objects for the g++ link."""
    odir = LIB / "obj"
    odir.mkdir(parents=True, exist_ok=True)
    objs = []
    for src in sorted(HDIR.glob("*.hip")):
        obj = odir / f"{src.stem}.o"
        cmd = [HIPCC, "-c", "-fPIC", "--offload-arch=gfx950", "-O2", "-std=c++17",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
               "-I", str(ROOT / "include"), "-I", str(HDIR), "-I", str(KDIR), str(src), "-o", str(obj)]
        _run(cmd, f"hipcc -c {src.name}")
        objs.append(str(obj))
    return objs


# CPU sanitizer build of the host code (tests/sanitize_run.py): AddressSanitizer
# and UndefinedBehaviorSanitizer on the g++ translation units only (the
# code objects are embedded unchanged).
SANITIZE_FLAGS = ["-fsanitize=address,undefined", "-fno-omit-frame-pointer", "-fno-sanitize-recover=undefined",
                  "-g", "-O1"]
SANDIR = LIB / "sanitize"


def build_host(sanitize: bool = False) -> Path:
    outdir = SANDIR if sanitize else LIB
    outdir.mkdir(parents=True, exist_ok=True)
    out = outdir / "librlxq.so"
    tmp = outdir / "librlxq.so.tmp"
    srcs = sorted(str(p) for p in HDIR.glob("*.cpp")) + build_host_hip_objects()
    cmd = [
        "g++", "-std=c++17", *(SANITIZE_FLAGS if sanitize else ["-O2"]), "-fPIC", "-shared", "-pthread",
        "-D__HIP_PLATFORM_AMD__", f"-DRLXQ_CO_DIR=\"{CO}\"",
        "-I", str(ROOT / "include"), "-I", str(HDIR), "-I", str(KDIR), "-I", str(ROCM / "include"),
        *srcs, "-o", str(tmp),
        "-L", str(ROCM / "lib"), "-lamdhip64", f"-Wl,-rpath,{ROCM / 'lib'}",
        "-Wl,--version-script=" + str(HDIR / "exports.map"),
    ]
    _run(cmd, "g++ librlxq")
    os.replace(tmp, out)
    return out


def build_examples() -> list[Path]:
    """The plain-C callers of the ABI in examples/, linked against librlxq.so."""
    outs = []
    (LIB / "examples").mkdir(parents=True, exist_ok=True)
    for src in sorted((PKG / "examples").glob("*.c")):
        out = LIB / "examples" / src.stem
        cmd = ["gcc", "-std=c99", "-O2", "-Wall", "-D__HIP_PLATFORM_AMD__", "-I", str(ROOT / "include"),
               "-I", str(ROCM / "include"), str(src), "-o", str(out), "-L", str(LIB), "-lrlxq",
               f"-Wl,-rpath,{LIB}", "-L", str(ROCM / "lib"), "-lamdhip64", f"-Wl,-rpath,{ROCM / 'lib'}", "-lm"]
        _run(cmd, f"gcc {src.name}")
        outs.append(out)
    return outs


def build_oracle(sanitize: bool = False) -> Path:
    odir = ROOT / "oracle"
    outdir = SANDIR if sanitize else odir
    outdir.mkdir(parents=True, exist_ok=True)
    out = outdir / "liboracle.so"
    tmp = outdir / "liboracle.so.tmp"
    # -ffp-contract=off keeps every multiply-add rounded where the restated
    # reference rounds; x86-64-v3 (AVX2 + FMA) so fmaf() is one instruction on
    # any host the GPU box may have.
    cmd = ["gcc", "-std=c11", *(SANITIZE_FLAGS if sanitize else ["-O3"]), "-march=x86-64-v3", "-ffp-contract=off",
           "-fopenmp", "-fPIC", "-shared", str(odir / "rlxq_oracle.c"), "-o", str(tmp), "-lm"]
    _run(cmd, "gcc liboracle")
    os.replace(tmp, out)
    return out


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--no-oracle", action="store_true")
    ap.add_argument("--host-only", action="store_true", help="relink librlxq.so from existing code objects")
    ap.add_argument("--cached", action="store_true", help="keep code objects whose inputs are unchanged (development)")
    ap.add_argument("--sanitize", action="store_true",
                    help="only the CPU sanitizer build of librlxq and the oracle, into lib/sanitize/ "
                         "(needs the code objects of a normal build)")
    a = ap.parse_args(argv)
    if shutil.which("g++") is None or not Path(HIPCC).exists():
        raise RuntimeError("need g++ and hipcc")
    if a.sanitize:
        build_host(sanitize=True)
        build_oracle(sanitize=True)
        return 0
    if not a.host_only:
        build_code_objects(cached=a.cached)
    build_host()
    build_examples()
    if not a.no_oracle:
        build_oracle()
    return 0


if __name__ == "__main__":
    sys.exit(main())
