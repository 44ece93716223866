"""Guard against a miscompile of merged LDS accesses in ROCm 7.2's AMDGPU backend.

The SI load/store optimizer pairs two LDS accesses off one base register into a
ds_{read,write}2_b{32,64}. In some kernels of this library it emitted the first offset scaled
wrongly (two fp32 stores at byte offsets 272 and 336 became ``ds_write2_b32 ... 17, 84``, the
first store landing 204 bytes early). This check compiles one kernel unit with the machine IR
printed before and after that pass and verifies that every merged access keeps the byte
offsets of the two accesses it replaced, up to one common base shift (the pass may rebase),
for the pairs whose originals addressed off one base register.

    python -m tjev_amd.ds_check [C D ...]
"""

from __future__ import annotations

import re
import subprocess
import sys

from .build import CSRC, FLAGS, PARTS, _hipcc, shapes, unit_flags

_SINGLE = re.compile(r"DS_(WRITE|READ)_B(32|64)\w*\s(%\d+)[^,]*,.*?,\s*(\d+),\s*0,\s*implicit"
                     r".*?(?:into|from) %ir\.([\w.]+)")
_PAIR = re.compile(r"DS_(WRITE|READ)2(ST64)?_B(32|64)\w*\s.*?,\s*(\d+),\s*(\d+),\s*0,\s*implicit"
                   r".*?(?:into|from) %ir\.([\w.]+).*?(?:into|from) %ir\.([\w.]+)")


def check_unit(c: int, d: int, part: int) -> list[str]:
    """Wrongly merged LDS accesses of one part of the (chunk c, head dim d) kernel unit (empty
    if none)."""
    return check_source(CSRC / "gdn_inst.hip", unit_flags(c, d, part))


def check_source(src, defines=()) -> list[str]:
    """Wrongly merged LDS accesses of one HIP source's device code (empty if none)."""
    cmd = [_hipcc(), *FLAGS, *defines, "--cuda-device-only", "-S", "-o", "/dev/null", str(src),
           "-mllvm", "-print-before=si-load-store-opt", "-mllvm", "-print-after=si-load-store-opt"]
    return bad_merges(subprocess.run(cmd, capture_output=True, text=True).stderr)


def bad_merges(text: str) -> list[str]:
    """The wrongly merged LDS accesses in a machine-IR dump printed before and after the SI
    load/store optimizer."""
    parts = re.split(r"# \*\*\* IR Dump (?:Before|After) SI Load Store Optimizer[^\n]*\n", text)[1:]
    bad = []
    for before, after in zip(parts[0::2], parts[1::2]):
        name = re.search(r"name:\s+(\S+)", before)
        # (base register, byte offset) of every single access before the pass
        single = {m.group(5): (m.group(3), int(m.group(4))) for m in _SINGLE.finditer(before)}
        for m in _PAIR.finditer(after):
            unit = (64 if m.group(2) else 1) * (4 if m.group(3) == "32" else 8)
            o0, o1, a, b = int(m.group(4)) * unit, int(m.group(5)) * unit, m.group(6), m.group(7)
            if a not in single or b not in single or single[a][0] != single[b][0]:
                continue  # only accesses off one base register have offsets to compare
            oa, ob = single[a][1], single[b][1]
            if (o0 - oa) != (o1 - ob) and (o0 - ob) != (o1 - oa):
                bad.append(f"{name.group(1) if name else '?'}: {m.group(0)[:60]}... merged from byte offsets "
                           f"{oa}, {ob}")
    return bad


def main(argv: list[str] | None = None) -> int:
    argv = sys.argv[1:] if argv is None else argv
    units = [(int(argv[i]), int(argv[i + 1])) for i in range(0, len(argv), 2)] if argv else shapes()
    failed = 0
    for c, d in units:
        bad = [line for part in range(PARTS) for line in check_unit(c, d, part)]
        print(f"chunk {c} dim {d}: {len(bad)} wrongly merged LDS accesses")
        for line in bad[:5]:
            print("   ", line)
        failed += bool(bad)
    return 1 if failed else 0


if __name__ == "__main__":
    sys.exit(main())
