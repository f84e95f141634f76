"""Builds liblocali_amd.so (HIP kernels for gfx950 + the host slot planner).

Each translation unit under locali_amd/csrc is compiled by hipcc in its own
process (the kernel variants are split by bit width and dtype so they build
in parallel), then linked in-tree next to this file. `python -m
locali_amd.build` builds from scratch; `--incremental` reuses objects whose
source hash (sources + headers + flags) is unchanged.
"""

from __future__ import annotations

import argparse
import hashlib
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
OBJ = PKG / "_build"
LIB = PKG / "liblocali_amd.so"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
COMMON = ["-O3", "-std=c++17", "-fPIC", f"-I{INCLUDE}", f"-I{CSRC}"]
# MFMA results go straight to VGPRs (no accumulator-register round trips).
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang",
          "-packed-fp32-ops", "-munsafe-fp-atomics", "-mllvm", "-amdgpu-mfma-vgpr-form"]


def sources() -> list[Path]:
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


def _flags(src: Path) -> list[str]:
    if src.suffix == ".hip":
        return COMMON + DEVICE + ["-x", "hip"]
    return COMMON + ["-Wall", "-Wextra"]


def _digest(src: Path) -> str:
    h = hashlib.sha256()
    for hdr in sorted(list(CSRC.glob("*.hpp")) + list(INCLUDE.glob("*.h"))):
        h.update(hdr.read_bytes())
    h.update(src.read_bytes())
    h.update(" ".join(_flags(src)).encode())
    return h.hexdigest()[:16]


def _compile(src: Path, incremental: bool) -> Path:
    out = OBJ / f"{src.stem}.{_digest(src)}.o"
    if incremental and out.exists():
        return out
    for stale in OBJ.glob(f"{src.stem}.*.o"):
        stale.unlink()
    cmd = [HIPCC, *_flags(src), "-c", str(src), "-o", str(out)]
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    noise = "is not a recognized feature for this target"
    log = "\n".join(line for line in proc.stdout.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"compile failed: {src.name}\n{log}")
    if log.strip():
        print(log, file=sys.stderr)
    return out


def build(incremental: bool = False, jobs: int | None = None, verbose: bool = True) -> Path:
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    OBJ.mkdir(exist_ok=True)
    srcs = sources()
    jobs = jobs or min(16, os.cpu_count() or 4, len(srcs))
    # Longest translation units first so the pool drains evenly.
    srcs.sort(key=lambda p: -p.stat().st_size)
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(lambda s: _compile(s, incremental), srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed\n{proc.stdout}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(objs)} translation units")
    return LIB


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--incremental", action="store_true")
    ap.add_argument("-j", "--jobs", type=int, default=None)
    args = ap.parse_args(argv)
    build(incremental=args.incremental, jobs=args.jobs)


if __name__ == "__main__":
    main()
