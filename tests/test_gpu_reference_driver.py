"""The reference's own test program against this library.

oracle/Makefile (target refdriver) compiles the reference's tests/test_gemm.cpp where it lies,
unchanged, against this library's headers (include/mxfp6/) and static archive in place of the
reference's: the switch a user of the reference makes. Run without arguments, the program first
checks the reference's routing table, then runs its correctness section -- the routed gemm on
nineteen shapes (128x128, 128x384 and split-K paths among them, gemm_force_tile with the
reference's own scale groupings, a workspace handed over where none is needed) against its CPU
reference GEMM with its own bound, printing one "OK" or "FAIL<<<" line each -- and then times
seven large shapes. This test asserts every correctness line; the routing-table lines check the
reference router's own tile choices, which this library's fitted router does not reproduce by
design (each route it picks is covered by the parity tests), so they are printed, not asserted.
The timing section needs minutes of host-side quantisation at K = 105728; the program is stopped
once its correctness section has reported.
"""
import os
import re
import subprocess
import time

import pytest

from gpu_util import say

pytestmark = pytest.mark.gpu

EXE = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle", "_ref",
                   "test_gemm_on_this_library")
# one line per verify* call of test_gemm.cpp's correctness section: "  MxNxK -> MTxNT[ +ws] : OK",
# "  compact MxNxK (Kp=..) -> MTxNT : NaNs=0 OK", "  128x128 MxNxK : OK", "  128x384 MxNxK : OK"
VERIFY = re.compile(r"^\s+(?:compact |128x128 |128x384 )?\s*\d+x\s*\d+x\s*\d+(?: \(Kp=\d+\))?"
                    r"(?: -> \d+x\d+(?: \+ws)?)? : (?:NaNs=\d+ )?(OK|FAIL<<<)\s*$")
N_VERIFY = 19


def test_reference_test_program_correctness_section():
    if not os.path.exists(EXE):
        pytest.skip("oracle/_ref/test_gemm_on_this_library not built (needs the reference's "
                    "sources: make -C oracle refdriver)")
    proc = subprocess.Popen([EXE], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                            bufsize=1)
    lines, verdict, t0 = [], None, time.time()
    try:
        for line in proc.stdout:
            line = line.rstrip("\n")
            lines.append(line)
            if VERIFY.match(line) or "CORRECTNESS" in line or "all OK" in line:
                say("  " + line)
            if line.strip() in ("all OK", "CORRECTNESS FAILED"):
                verdict = line.strip()
                break
            if time.time() - t0 > 240:
                break
    finally:
        proc.kill()
        proc.wait()
    verify = [m for m in (VERIFY.match(s) for s in lines) if m]
    routing = [s for s in lines if s.lstrip().startswith(("route ", "choose_tile", "covers ",
                                                          "tile covers", "split", "workspace"))]
    say(f"  routing-table lines (the reference router's choices, not asserted): {len(routing)}")
    for s in routing[-6:]:
        say("  " + s)
    assert len(verify) == N_VERIFY, f"{len(verify)} correctness lines, expected {N_VERIFY}"
    bad = [m.group(0) for m in verify if m.group(1) != "OK"]
    assert not bad, "correctness lines failed:\n" + "\n".join(bad)
    # the program's own verdict counts the routing table too; every correctness line is OK, so
    # a failing verdict can only come from the routing table
    assert verdict in ("all OK", "CORRECTNESS FAILED"), "the correctness section did not finish"
