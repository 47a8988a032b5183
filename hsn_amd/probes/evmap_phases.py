"""Build and run the event-map phase timeline (``evmap_phases.hip``) on the current GPU.

``python -m hsn_amd.probes.evmap_phases [N]`` (one reset in N positions, default 256, 0 for
none) compiles the probe with the library's hipcc flags into
``_build/evmap_phases`` (the event-map kernels with their phase-stamp hooks on) and prints its
report: for the forward and the backward at the ref shape, when each phase edge is reached
(mean and largest over the wavefronts), the spread of each phase's span and of the workgroups'
ends, and the back-to-back launch durations of the instrumented build."""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

from hsn_amd import build as _build

HERE = Path(__file__).resolve().parent


def compile_probe() -> Path:
    out = _build.BUILD / "evmap_phases"
    _build.BUILD.mkdir(exist_ok=True)
    cmd = [_build.hipcc(), *_build.HIP_FLAGS, str(HERE / "evmap_phases.hip"), "-o", str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on evmap_phases.hip:\n{proc.stderr[-4000:]}")
    return out


def main() -> int:
    exe = compile_probe()
    print(f"built {exe}", flush=True)
    return subprocess.run([str(exe), *sys.argv[1:]]).returncode


if __name__ == "__main__":
    sys.exit(main())
