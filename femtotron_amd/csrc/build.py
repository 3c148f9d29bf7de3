"""Build libfemtohip.so (gfx950) from the HIP sources in this directory.

    python -m femtotron_amd.csrc.build          # or femtotron_amd.csrc.build.build()

Every source is compiled by hipcc for gfx950 only, in parallel, into
``_build/`` next to this file, and linked into ``femtotron_amd/libfemtohip.so``.
A build always recompiles (it is the "does it build" check); loaders only
look for the finished library.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

CSRC = Path(__file__).resolve().parent
PKG = CSRC.parent
REPO = PKG.parent
INCLUDE = REPO / "include"
OUT = PKG / "libfemtohip.so"
BUILD_DIR = CSRC / "_build"

ARCH = "gfx950"
SOURCES = sorted([p for p in CSRC.iterdir() if p.suffix in (".hip", ".cpp")])

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Packed fp32 (v_pk_*_f32) code generation stays off for all device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]

# MFMA accumulators in VGPRs: the attention softmax rescales its output
# accumulators every key block, which in AGPRs costs a read and a write per
# register per block.  The GEMM keeps its 256 accumulator registers per lane in
# AGPRs (one wave per SIMD, 128 x 128 outputs each), so it is built without.
VGPR_FORM = ["-mllvm", "-amdgpu-mfma-vgpr-form"]
AGPR_FORM_SOURCES = {"fh_gemm.hip"}


def flags_for(src: Path) -> list:
    return COMMON_FLAGS + ([] if src.name in AGPR_FORM_SOURCES else VGPR_FORM)


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the femtohip library needs ROCm's hipcc")


def _compile(src: Path) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc(), *flags_for(src), "-x", "hip", "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stdout}\n{res.stderr}")
    # hipcc's host pass does not know the packed-fp32 feature name; drop that
    # (harmless) warning and show anything else.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    extra = [ln for ln in res.stderr.splitlines() if ln.strip() and noise not in ln]
    if extra:
        sys.stderr.write("\n".join(extra) + "\n")
    return obj


def build(verbose: bool = True) -> Path:
    BUILD_DIR.mkdir(exist_ok=True)
    jobs = min(len(SOURCES), max(1, min(16, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"[femtohip] built {OUT} from {len(SOURCES)} sources for {ARCH}")
    return OUT


if __name__ == "__main__":
    build()
