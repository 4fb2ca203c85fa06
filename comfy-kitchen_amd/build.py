"""Build the gfx950 C-ABI library libckh.so in-tree (no JIT, no torch extension).

    python comfy-kitchen_amd/build.py            # build (always recompiles)

Every csrc/*.hip file is compiled by hipcc for gfx950 only and linked into
comfy_kitchen/backends/hip/libckh.so, which the "hip" backend loads with ctypes.
benchlib/*.hip (kernels bench.py times for comparison, e.g. the copy floor) is linked
into benchlib/libckh_bench.so, and tests/hw/*.hip (exhaustive hardware-identity checks)
into tests/hw/libckh_hwcheck.so, both separate from the product library.

Flags: -O3; no fast-math (the quantizers need IEEE division and exact rounding);
-ffp-contract=off so no multiply-add is fused behind the kernels' back (the kernels
call __fmaf_rn where a fused multiply-add is intended); packed-FP32 instructions are
disabled for the device pass.  Code object v5 is used because the extension runs inside
torch's bundled HIP runtime (same SONAME as /opt/rocm's), which may be older than hipcc.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parent
CSRC = HERE / "csrc"
OUT = HERE / "comfy_kitchen" / "backends" / "hip" / "libckh.so"
BENCHLIB = HERE / "benchlib"
HWCHECK = REPO / "tests" / "hw"  # test-only: exhaustive hardware-identity sweeps
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-mcode-object-version=5",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fno-gpu-rdc",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{REPO / 'include'}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    cand = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(cand).exists():
        raise RuntimeError("hipcc not found; ROCm is required to build libckh.so")
    return cand


# Most per-lane scratch (private memory) bytes a kernel may use.  A private array the
# compiler fails to keep in registers (e.g. behind a call it did not inline) lands in scratch
# memory and can make a kernel ten times slower without changing its results; the build
# fails instead.  The MXFP8 tile kernel spills 2-3 registers in some instantiations (12 bytes).
SCRATCH_LIMIT = 16


def _compile(src: Path, obj: Path) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, "-Rpass-analysis=kernel-resource-usage", "-fno-caret-diagnostics", "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    lines = [l for l in res.stderr.splitlines() if noise not in l]
    err = "\n".join(l for l in lines if "kernel-resource-usage" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    kernel = "?"
    for l in lines:
        if "Function Name:" in l:
            kernel = l.split("Function Name:")[1].split()[0]
        elif "ScratchSize [bytes/lane]:" in l:
            n = int(l.split("ScratchSize [bytes/lane]:")[1].split()[0])
            if n > SCRATCH_LIMIT:
                raise RuntimeError(f"{src.name}: kernel {kernel} uses {n} bytes/lane of scratch "
                                   f"(limit {SCRATCH_LIMIT}): a private array left memory-resident")


def _link(sources: list[Path], out: Path, objdir: Path, verbose: bool) -> Path:
    objdir.mkdir(parents=True, exist_ok=True)
    objs = [objdir / (s.stem + ".o") for s in sources]
    workers = min(len(sources), int(os.environ.get("MAX_JOBS", "8")), 8)
    with cf.ThreadPoolExecutor(max_workers=max(workers, 1)) as ex:
        list(ex.map(_compile, sources, objs))
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-mcode-object-version=5", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out.relative_to(REPO)} from {len(sources)} sources")
    return out


def build(verbose: bool = True) -> Path:
    _link(sorted(CSRC.glob("*.hip")), OUT, HERE / "_build", verbose)
    bench = sorted(BENCHLIB.glob("*.hip"))
    if bench:
        _link(bench, BENCHLIB / "libckh_bench.so", HERE / "_build" / "benchlib", verbose)
    hw = sorted(HWCHECK.glob("*.hip"))
    if hw:
        _link(hw, HWCHECK / "libckh_hwcheck.so", HERE / "_build" / "hwcheck", verbose)
    return OUT


if __name__ == "__main__":
    build()
