"""Build the gfx950 HIP library in-tree with hipcc (no torch extension machinery).

    python -m nexusquant_amd.build        # -> nexusquant_amd/lib/libnqamd.so
"""

from __future__ import annotations

import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB_DIR = os.path.join(HERE, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libnqamd.so")
ARCH = os.environ.get("NQ_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "-shared",
    f"--offload-arch={ARCH}",
    # parity: the kernels follow an explicit rounding order, no FMA contraction
    "-ffp-contract=off",
    # packed fp32 VALU ops stay disabled on this hardware pool
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


# Per-source flags.  The scorers read every MFMA result with VALU instructions;
# accumulators in VGPRs save one v_accvgpr_read per element.
SOURCE_FLAGS = {
    "nq_score.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "nq_keykey.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; the gfx950 library cannot be built")


def sources():
    return sorted(glob.glob(os.path.join(HERE, "csrc", "*.hip")))


def source_hash() -> str:
    """sha256 (hex, 16 digits) of everything the library is built from: the
    kernel sources and headers, the public header and the compiler flags.
    The build embeds it (nq_source_hash()); _lib.load() recomputes it and
    refuses a library built from other sources."""
    import hashlib
    h = hashlib.sha256()
    files = sorted(glob.glob(os.path.join(HERE, "csrc", "*.hip")) + glob.glob(os.path.join(HERE, "csrc", "*.h"))
                   + glob.glob(os.path.join(ROOT, "include", "*.h")))
    for path in files:
        h.update(os.path.relpath(path, ROOT).encode() + b"\0")
        with open(path, "rb") as f:
            h.update(f.read())
        h.update(b"\0")
    h.update(" ".join(HIPCC_FLAGS).encode())
    for name in sorted(SOURCE_FLAGS):
        h.update((name + ":" + " ".join(SOURCE_FLAGS[name])).encode())
    return h.hexdigest()[:16]


def _run(cmd, verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed with status {res.returncode}: {' '.join(cmd[-3:])}")


def build(verbose: bool = False, jobs: int = 0) -> str:
    """Compile every csrc/*.hip to an object in parallel (outside the tree), then link."""
    import tempfile
    from concurrent.futures import ThreadPoolExecutor
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = LIB_PATH + ".tmp"
    inc = ["-I", os.path.join(ROOT, "include")]
    compile_flags = [f for f in HIPCC_FLAGS if f != "-shared"] + [f'-DNQ_SOURCE_HASH="{source_hash()}"']
    jobs = jobs or min(len(sources()), os.cpu_count() or 1, 16)
    with tempfile.TemporaryDirectory(prefix="nqamd_build_") as objdir:
        objs = [os.path.join(objdir, os.path.basename(src) + ".o") for src in sources()]
        with ThreadPoolExecutor(max_workers=jobs) as pool:
            list(pool.map(lambda so: _run([hipcc(), *compile_flags, *SOURCE_FLAGS.get(os.path.basename(so[0]), []),
                                           *inc, "-c", so[0], "-o", so[1]], verbose),
                          zip(sources(), objs)))
        _run([hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", tmp, *objs], verbose)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
