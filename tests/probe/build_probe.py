"""Build tests/probe/libts_probe.so, the test suite's hardware-probe library.

The probes (ts_probe.hip) are one-wave kernels that pin lane layouts and LDS
behaviour for tests/test_probe_gpu.py; they live in a library of their own
so that the operator library exports only operators.  Same gfx950 flags as
the operator library (thundersync_amd/_build.py).
"""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
LIB_PATH = HERE / "libts_probe.so"


def build() -> Path:
    if str(ROOT) not in sys.path:
        sys.path.insert(0, str(ROOT))
    from thundersync_amd import _build

    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [_build.hipcc(), *_build.device_flags(), "-shared", str(HERE / "ts_probe.hip"), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on ts_probe.hip:\n{proc.stdout}{proc.stderr}")
    tmp.replace(LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build())
