"""Build libthundersync_hip.so for gfx950 from csrc/*.hip, in-tree.

Each translation unit is compiled with hipcc for gfx950 only and linked into
one shared library next to this file.  The packed-FP32 instruction feature is
switched off for every device compile (-packed-fp32-ops): the kernels are
written with scalar float arithmetic and must not be vectorised into packed
FP32 instructions.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
INCLUDE = HERE.parent / "include"
LIB_NAME = "libthundersync_hip.so"
ARCH = "gfx950"


def hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found (looked at $HIPCC, /opt/rocm/bin/hipcc, PATH)")


def device_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-munsafe-fp-atomics",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        f"-I{INCLUDE}",
        "-Wno-unused-result",
    ]


# Extra code-generation flags per translation unit.  attention_dq.hip: the dQ
# kernel's S/dP tiles and dQ accumulators fit the VGPRs, and MFMA results
# written to VGPRs spare it per-tile copies out of the accumulation registers.
FILE_FLAGS = {
    "attention_dq.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    # the one-wave-per-head dK/dV kernel: S and dP in VGPRs (MFMA results in
    # VGPRs), its dK/dV accumulators in the accumulation registers through
    # inline assembly
    "attention_dkdv_wave.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    # the head-dim-256 dK/dV kernel with 32 keys per wave: likewise
    "attention_dkdv256.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


def _compile(src: Path, obj: Path) -> tuple[Path, str]:
    cmd = [hipcc(), *device_flags(), *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    log = "\n".join(
        line for line in (proc.stdout + proc.stderr).splitlines() if noise not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{log}")
    return obj, log


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every csrc/*.hip and link the shared library; return its path."""
    build_dir = HERE / "_build"
    build_dir.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(sources), max(1, (os.cpu_count() or 2) - 1), 8)
    with concurrent.futures.ThreadPoolExecutor(jobs) as pool:
        futures = [pool.submit(_compile, s, build_dir / (s.stem + ".o")) for s in sources]
        objects = []
        for f in futures:
            obj, log = f.result()
            if verbose and log.strip():
                print(log, file=sys.stderr)
            objects.append(obj)
    out = HERE / LIB_NAME
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}{proc.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    path = build(verbose=True)
    print(path)
