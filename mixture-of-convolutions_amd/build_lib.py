"""Build libmoc_hip.so (gfx950) from csrc/ with hipcc.

    python mixture-of-convolutions_amd/build_lib.py [--jobs N]

Objects go to csrc/_build/, the shared library next to the Python package
(moc/libmoc_hip.so), where moc/_lib.py loads it.  Every call recompiles.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
CSRC = PKG_ROOT / "csrc"
BUILD = CSRC / "_build"
LIB = PKG_ROOT / "moc" / "libmoc_hip.so"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fno-gpu-rdc",
    # packed FP32 VALU ops are kept out of the device code on this pool
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in VGPRs: the kernels read every result on VALU right away,
    # and AGPR results would cost a v_accvgpr_read per value
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-command-line-argument",
]


def _compile(src: Path, extra: tuple[str, ...] = (), build_dir: Path = BUILD) -> Path:
    obj = build_dir / (src.stem + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    msgs = [ln for ln in (res.stdout + res.stderr).splitlines()
            if "packed-fp32-ops' is not a recognized feature" not in ln]
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n" + "\n".join(msgs))
    if msgs:
        print("\n".join(msgs), file=sys.stderr)
    return obj


def build(jobs: int | None = None, verbose: bool = True, defines: tuple[str, ...] = (),
          out: Path = LIB) -> Path:
    """Compile csrc/*.hip and link ``out``; ``defines`` are extra -D flags."""
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    build_dir = BUILD if not defines else BUILD / ("_".join(defines).replace("=", "-"))
    build_dir.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    jobs = jobs or min(len(sources), max(1, (os.cpu_count() or 4)))
    extra = tuple(f"-D{d}" for d in defines)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda src: _compile(src, extra, build_dir), sources))
    LIB_OUT = Path(out)
    tmp = LIB_OUT.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("link failed:\n" + res.stdout + res.stderr)
    os.replace(tmp, LIB_OUT)
    if verbose:
        print(f"built {LIB_OUT} from {len(sources)} sources")
    return LIB_OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("-D", dest="defines", action="append", default=[],
                    help="extra preprocessor define, e.g. -D MOC_BWD_MIN_WAVES=2")
    ap.add_argument("--out", default=str(LIB))
    a = ap.parse_args()
    build(a.jobs, defines=tuple(a.defines), out=Path(a.out))
