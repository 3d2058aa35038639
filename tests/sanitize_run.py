"""CPU sanitizer run of the host code: builds librlxq's host translation
units and the oracle with AddressSanitizer + UndefinedBehaviorSanitizer
(rlx-models_amd/build.py --sanitize, into rlx-models_amd/lib/sanitize/), then
runs, with those libraries loaded through RLXQ_LIB / RLXQ_ORACLE_LIB and the
ASan runtime preloaded into Python:
  * the CPU tests of the GGUF reader, the C ABI, the oracle, the golden
    fixtures and the binding's argument checks;
  * tests/checkpoint_fuzz.py (truncations and byte flips of the reference's
    GGUF and safetensors fixtures).
No GPU is used.  Exit status 0 means every step passed with no sanitizer
report (reports abort the process: halt_on_error).

    python tests/sanitize_run.py
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def main() -> int:
    subprocess.run([sys.executable, str(ROOT / "rlx-models_amd" / "build.py"), "--sanitize"], check=True)
    asan = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True,
                          check=True).stdout.strip()
    ubsan = subprocess.run(["gcc", "-print-file-name=libubsan.so"], capture_output=True, text=True,
                           check=True).stdout.strip()
    san = ROOT / "rlx-models_amd" / "lib" / "sanitize"
    env = dict(os.environ)
    env.update({
        "RLXQ_LIB": str(san / "librlxq.so"),
        "RLXQ_ORACLE_LIB": str(san / "liboracle.so"),
        "LD_PRELOAD": f"{asan}:{ubsan}",
        # the interpreter itself is not instrumented and keeps memory until
        # exit: leak reports would be its own
        "ASAN_OPTIONS": "detect_leaks=0:halt_on_error=1:abort_on_error=1:verify_asan_link_order=0",
        "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1",
        "OMP_NUM_THREADS": "2",
    })
    steps = [
        [sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider", "-m", "not gpu",
         "tests/test_gguf.py", "tests/test_abi.py", "tests/test_oracle.py", "tests/test_golden.py",
         "tests/test_wrapper_checks.py", "tests/test_mlx_loader.py"],
        [sys.executable, "tests/checkpoint_fuzz.py"],
    ]
    for cmd in steps:
        print("[sanitize]", " ".join(cmd[1:]), flush=True)
        r = subprocess.run(cmd, cwd=ROOT, env=env)
        if r.returncode != 0:
            print(f"[sanitize] failed with status {r.returncode}", flush=True)
            return r.returncode
    print("[sanitize] all steps passed under ASan + UBSan", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
