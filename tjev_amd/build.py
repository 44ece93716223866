"""Build libtjev_gdn.so for gfx950 in-tree: PARTS hipcc jobs per (chunk, head dim) pair of
csrc/gdn_shapes.def plus the C ABI, linked with ``hipcc -shared``.

    python -m tjev_amd.build [-j JOBS]
"""

from __future__ import annotations

import argparse
import os
import re
import shutil
import subprocess
import sys
import time
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OUT = HERE / "_build"
LIB = HERE / "libtjev_gdn.so"
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # packed fp32 instructions stay off in every GPU build of this library
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


# units built once: the C ABI, the gated RMSNorm and the decode step
EXTRA_UNITS = ("gdn_api", "gdn_norm", "gdn_decode")
# object files per (chunk, head dim) pair: the launch sequences with the small kernels (part 0),
# then one per large kernel family (gdn_inst.hip's GDN_PART)
PARTS = 6
# per-object backend options, measured at the model shape: the output kernel (part 3) runs 1%
# faster under the scheduler strategy that groups memory instructions; every other family is
# as fast or slower under it (k_bwd_grads by a third)
PART_FLAGS = {(128, 128, 3): ["-mllvm", "--amdgpu-sched-strategy=max-memory-clause"]}


def unit_flags(c: int, d: int, part: int) -> list[str]:
    """The defines and backend options of one gdn_inst.hip object."""
    return [f"-DGDN_C={c}", f"-DGDN_D={d}", f"-DGDN_PART={part}", *PART_FLAGS.get((c, d, part), [])]


def shapes() -> list[tuple[int, int]]:
    text = (CSRC / "gdn_shapes.def").read_text()
    return [(int(c), int(d)) for c, d in re.findall(r"GDN_SHAPE\((\d+),\s*(\d+)\)", text)]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the GDN library needs ROCm's hipcc")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        noise = "is not a recognized feature for this target"
        err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{err}")


def build(jobs: int | None = None, verbose: bool = False, verify: bool = True) -> Path:
    """Compile every kernel unit and link the library (always rebuilds). ``verify`` also runs
    the merged-LDS-access check of ds_check.py on every unit and fails the build if any
    access was miscompiled."""
    hipcc = _hipcc()
    OUT.mkdir(exist_ok=True)
    units = []
    for c, d in shapes():
        for part in range(PARTS):
            obj = OUT / f"gdn_inst_c{c}_d{d}_p{part}.o"
            units.append([hipcc, *FLAGS, *unit_flags(c, d, part), "-c", str(CSRC / "gdn_inst.hip"), "-o", str(obj)])
    for name in EXTRA_UNITS:
        units.append([hipcc, *FLAGS, "-c", str(CSRC / f"{name}.hip"), "-o", str(OUT / f"{name}.o")])
    t0 = time.time()
    with ThreadPoolExecutor(max_workers=jobs or min(len(units), os.cpu_count() or 4)) as pool:
        checks = []
        if verify:
            from .ds_check import check_source, check_unit

            checks = [pool.submit(check_unit, c, d, part) for c, d in shapes() for part in range(PARTS)]
            checks += [pool.submit(check_source, CSRC / f"{name}.hip") for name in EXTRA_UNITS]
        list(pool.map(_run, units))
        bad = [line for f in checks for line in f.result()]
    if bad:
        raise RuntimeError("miscompiled merged LDS accesses (ds_check):\n" + "\n".join(bad[:10]))
    objs = [u[-1] for u in units]
    tmp = LIB.with_suffix(".so.tmp")
    _run([hipcc, *FLAGS, "-shared", "-o", str(tmp), *objs])
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} in {time.time() - t0:.1f}s ({len(units)} units)")
    return LIB


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("-j", "--jobs", type=int, default=None)
    ap.add_argument("--no-verify", action="store_true", help="skip the merged-LDS-access check")
    args = ap.parse_args(argv)
    build(args.jobs, verbose=True, verify=not args.no_verify)
    return 0


if __name__ == "__main__":
    sys.exit(main())
