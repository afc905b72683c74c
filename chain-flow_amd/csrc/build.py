"""Build libcfhip.so (every HIP source in this directory) for gfx950 with hipcc.

    python chain-flow_amd/csrc/build.py [--jobs N]

The library lands next to the Python package (chain-flow_amd/chain_flow_amd/libcfhip.so), so it
travels with the source tree; objects go to chain-flow_amd/csrc/_build/.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import re
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
INCLUDE = ROOT / "include"
OUT = HERE.parent / "chain_flow_amd" / "libcfhip.so"
BUILD = HERE / "_build"
ARCH = "gfx950"

# -packed-fp32-ops off: hipcc must not fuse fp32 pairs into packed-math instructions.
HIPFLAGS = ["-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC", "-Wall", "-Wno-unused-function",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            f"-I{INCLUDE}", f"-I{HERE}"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libcfhip.so)")


def sources():
    return sorted(HERE.glob("*.hip"))


def compile_one(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    # the resource-usage remarks name every kernel that spills registers to scratch memory
    cmd = [hipcc(), *HIPFLAGS, "-Rpass-analysis=kernel-resource-usage", "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{r.stdout}\n{r.stderr}")
    noise = "is not a recognized feature for this target"
    lines = r.stderr.splitlines()
    spills, name = [], None
    for line in lines:
        if "remark: Function Name:" in line:
            name = line.split("Function Name:")[1].split("[")[0].strip()
        elif "remark:" in line and "ScratchSize [bytes/lane]:" in line:
            n = int(line.split("ScratchSize [bytes/lane]:")[1].split("[")[0])
            if n > 0 and name:
                spills.append(f"{name} ({n} B/lane)")
    if spills:
        print(f"{src.name}: {len(spills)} kernel(s) use scratch (register spills): " + "; ".join(spills[:6]),
              file=sys.stderr)
    # drop the remarks and the source-context lines that follow them
    ctx = re.compile(r"^\s*(\d+\s*)?[|^]|^In file included from")
    warn = "\n".join(line for line in lines if noise not in line and "remark:" not in line and line.strip()
                     and not ctx.match(line) and "kernel-resource-usage" not in line)
    if warn.strip():
        print(warn, file=sys.stderr)
    return obj


def build(jobs: int = 8, verbose: bool = True) -> Path:
    BUILD.mkdir(exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(compile_one, srcs))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT} from {len(srcs)} sources")
    return OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=8)
    build(ap.parse_args().jobs)
