"""Build-time guard on the kernels' register use: reads the kernel-resource-usage remarks that the
Makefile writes per HIP unit (build/<unit>.res, from hipcc -Rpass-analysis=kernel-resource-usage)
and fails when any kernel uses scratch memory, spills registers or has a dynamic stack.

Why: the tile kernels wait on exact vector-memory counts (s_waitcnt vmcnt(N) with N counted from
the static issue order of their copies and loads: wide_kernel.hpp CHUNK_WAIT / PRO_WAIT /
short_wait, slab_kernel.hpp's ring waits). A scratch spill is a vector-memory operation too; the
compiler would place it between the counted ones, and a wait would then let a copy still in
flight be read. A kernel with zero scratch has no such operation.

  python3 check_resources.py [build_dir]     # prints the table, exit status 1 on a violation
"""
import glob
import os
import re
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
FIELDS = {"VGPRs": "vgpr", "AGPRs": "agpr", "ScratchSize [bytes/lane]": "scratch",
          "SGPRs Spill": "sgpr_spill", "VGPRs Spill": "vgpr_spill", "Dynamic Stack": "dyn_stack",
          "LDS Size [bytes/block]": "lds", "Occupancy [waves/SIMD]": "occupancy"}
_NAME = re.compile(r"remark: Function Name: (\S+)")
_FIELD = re.compile(r"remark:\s+([^:]+(?:\[[^\]]*\])?): (\S+) \[-Rpass-analysis")


def parse(path):
    """{kernel symbol: {field: value}} of one remarks file."""
    out, cur = {}, None
    with open(path, errors="replace") as f:
        for line in f:
            m = _NAME.search(line)
            if m:
                cur = out.setdefault(m.group(1), {})
                continue
            m = _FIELD.search(line)
            if m and cur is not None and m.group(1).strip() in FIELDS:
                v = m.group(2)
                cur[FIELDS[m.group(1).strip()]] = (v == "True") if v in ("True", "False") else int(v)
    return out


def collect(build_dir):
    files = sorted(glob.glob(os.path.join(build_dir, "*.res")))
    kernels = {}
    for p in files:
        for name, r in parse(p).items():
            kernels[name] = dict(r, unit=os.path.basename(p)[:-4])
    return files, kernels


def violations(kernels):
    return [(n, r) for n, r in kernels.items()
            if r.get("scratch", 0) or r.get("sgpr_spill", 0) or r.get("vgpr_spill", 0)
            or r.get("dyn_stack", False)]


def family(name):
    for fam in ("wide_kernel", "slab_kernel", "direct_kernel", "reduce_splitk_kernel",
                "repack_rows_kernel", "prep"):
        if fam in name:
            return fam
    return "other"


def main(argv):
    build_dir = argv[1] if len(argv) > 1 else os.path.join(HERE, "build")
    files, kernels = collect(build_dir)
    if not files or not kernels:
        print(f"check_resources: no resource remarks under {build_dir} (build with make first)")
        return 1
    fams = {}
    for n, r in kernels.items():
        fams.setdefault(family(n), []).append(r)
    print(f"check_resources: {len(kernels)} kernels in {len(files)} units")
    for fam, rs in sorted(fams.items()):
        print(f"  {fam:22s} {len(rs):4d} kernels  VGPR <= {max(r.get('vgpr', 0) for r in rs):3d}  "
              f"AGPR <= {max(r.get('agpr', 0) for r in rs):3d}  "
              f"scratch max {max(r.get('scratch', 0) for r in rs)} B/lane")
    bad = violations(kernels)
    for n, r in bad:
        print(f"  SCRATCH/SPILL: {n} ({r['unit']}): {r}")
    return 1 if bad else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
