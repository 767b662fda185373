"""Ahead-of-time build of libllamatov_hip.so for gfx950.

Replaces the reference's JIT chain (swipl emitter -> .cu -> nvcc -cubin, content-addressed
by SHA-1; bpd/lib/fact_dispatch.py:74-109, bpd/lib/dev_residency.py:363-385): every kernel
is hand-written HIP compiled once, in-tree, into one shared library.  The library records
the SHA-256 of its sources next to itself so a stale build is detectable.
"""
from __future__ import annotations

import hashlib
import os
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
INCLUDE = PKG_DIR.parent / "include"
LIB_NAME = "libllamatov_hip.so"
LIB_PATH = PKG_DIR / LIB_NAME
ARCH = os.environ.get("LT_OFFLOAD_ARCH", "gfx950")

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fvisibility=hidden",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results straight into VGPRs: the prefill GEMM folds every MFMA result with VALU
    # arithmetic, which would otherwise first copy each of them out of the AGPRs
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wno-unused-command-line-argument",
]


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def source_digest() -> str:
    h = hashlib.sha256()
    for p in sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.h")) + list(INCLUDE.glob("*.h"))):
        h.update(p.name.encode())
        h.update(p.read_bytes())
    return h.hexdigest()


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    raise RuntimeError(f"hipcc not found under {rocm}; ROCm is required to build {LIB_NAME}")


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print("[build]", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{r.stdout}\n{r.stderr}")


def build(verbose: bool = True, jobs: int | None = None) -> Path:
    """Compile every HIP source into llamatov_amd/libllamatov_hip.so (always recompiles):
    one object per source, compiled in parallel, then one shared-library link."""
    from concurrent.futures import ThreadPoolExecutor
    import tempfile

    out_tmp = LIB_PATH.with_suffix(".so.tmp")
    srcs = sources()
    with tempfile.TemporaryDirectory(prefix="lt_build_") as tmp:
        objs = [Path(tmp) / (s.stem + ".o") for s in srcs]
        n = jobs or min(len(srcs), max(1, min(8, len(os.sched_getaffinity(0)))))
        with ThreadPoolExecutor(max_workers=n) as ex:
            list(ex.map(lambda so: _run([hipcc(), *HIP_FLAGS, "-c", str(so[0]), "-o", str(so[1])], verbose),
                        zip(srcs, objs)))
        _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(out_tmp)],
             verbose)
    os.replace(out_tmp, LIB_PATH)
    (PKG_DIR / (LIB_NAME + ".sha256")).write_text(source_digest() + "\n")
    return LIB_PATH


def is_stale() -> bool:
    stamp = PKG_DIR / (LIB_NAME + ".sha256")
    if not LIB_PATH.exists() or not stamp.exists():
        return True
    return stamp.read_text().strip() != source_digest()


if __name__ == "__main__":
    build()
    sys.exit(0)
