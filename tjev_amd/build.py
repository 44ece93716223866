"""Build libtjev_gdn.so for gfx950 in-tree: PARTS hipcc jobs per (chunk, head dim) pair of
csrc/gdn_shapes.def plus the C ABI, linked with ``hipcc -shared``. ``--lds-poison`` builds the
debug library libtjev_gdn_lds_poison.so instead: every kernel fills its LDS with NaN bytes before
its own code runs (-DGDN_LDS_POISON), over the shapes its tests run.

    python -m tjev_amd.build [-j JOBS] [--lds-poison]
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
LDS_POISON_LIB = HERE / "libtjev_gdn_lds_poison.so"
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


def shapes(lds_poison: bool = False) -> list[tuple[int, int]]:
    """The (chunk, head dim) pairs of gdn_shapes.def: its #else branch for the library, its
    GDN_LDS_POISON branch for the LDS-poison debug library."""
    text = (CSRC / "gdn_shapes.def").read_text()
    poison, full = text.split("#ifdef GDN_LDS_POISON", 1)[1].split("#else", 1)
    part = poison if lds_poison else full.split("#endif", 1)[0]
    return [(int(c), int(d)) for c, d in re.findall(r"GDN_SHAPE\((\d+),\s*(\d+)\)", part)]


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


def build(jobs: int | None = None, verbose: bool = False, verify: bool = True, lds_poison: bool = False) -> Path:
    """Compile every kernel unit and link the library (always rebuilds). ``verify`` also runs
    the merged-LDS-access check of ds_check.py on every unit and fails the build if any
    access was miscompiled. ``lds_poison``: the LDS-poison debug library (its own objects and
    shapes, -DGDN_LDS_POISON), checked the same way."""
    hipcc = _hipcc()
    out = OUT / "lds_poison" if lds_poison else OUT
    lib = LDS_POISON_LIB if lds_poison else LIB
    extra = ["-DGDN_LDS_POISON"] if lds_poison else []
    out.mkdir(parents=True, exist_ok=True)
    units = []
    for c, d in shapes(lds_poison):
        for part in range(PARTS):
            obj = out / f"gdn_inst_c{c}_d{d}_p{part}.o"
            units.append([hipcc, *FLAGS, *extra, *unit_flags(c, d, part), "-c", str(CSRC / "gdn_inst.hip"), "-o",
                          str(obj)])
    for name in EXTRA_UNITS:
        units.append([hipcc, *FLAGS, *extra, "-c", str(CSRC / f"{name}.hip"), "-o", str(out / f"{name}.o")])
    t0 = time.time()
    with ThreadPoolExecutor(max_workers=jobs or min(len(units), os.cpu_count() or 4)) as pool:
        checks = []
        if verify:
            from .ds_check import check_source

            checks = [pool.submit(check_source, CSRC / "gdn_inst.hip", [*extra, *unit_flags(c, d, part)])
                      for c, d in shapes(lds_poison) for part in range(PARTS)]
            checks += [pool.submit(check_source, CSRC / f"{name}.hip", extra) for name in EXTRA_UNITS]
        list(pool.map(_run, units))
        bad = [line for f in checks for line in f.result()]
    if bad:
        raise RuntimeError("miscompiled merged LDS accesses (ds_check):\n" + "\n".join(bad[:10]))
    objs = [u[-1] for u in units]
    tmp = lib.with_suffix(".so.tmp")
    _run([hipcc, *FLAGS, "-shared", "-o", str(tmp), *objs])
    os.replace(tmp, lib)
    if verbose:
        print(f"built {lib} in {time.time() - t0:.1f}s ({len(units)} units)")
    return lib


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("-j", "--jobs", type=int, default=None)
    ap.add_argument("--no-verify", action="store_true", help="skip the merged-LDS-access check")
    ap.add_argument("--lds-poison", action="store_true", help="build the LDS-poison debug library")
    args = ap.parse_args(argv)
    build(args.jobs, verbose=True, verify=not args.no_verify, lds_poison=args.lds_poison)
    return 0


if __name__ == "__main__":
    sys.exit(main())
