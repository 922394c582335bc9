"""Routing and split-K planning (host only).

The oracle's restatement of the reference router is pinned by the reference's own routing table
(tests/test_gemm.cpp:262-299) and by the reference library itself over a sweep. The library's
own MI355X router is checked for what the public contract requires of any router: the tile it
returns divides the shape (full coverage), its scale grouping is one the kernels read, and the
workspace query agrees with the split the launch uses.
"""
import json
import os

import numpy as np
import pytest

GOLD = os.path.join(os.path.dirname(__file__), "golden")
with open(os.path.join(GOLD, "ref_routing.json")) as f:
    REF = json.load(f)

IMPLEMENTED = {(128, 128, 2, 2), (128, 256, 2, 4), (128, 384, 4, 3), (256, 256, 4, 4),
               (256, 192, 4, 3)}


def _kpad(K):
    return (K + 191) // 192 * 192


def test_oracle_router_reference_table(orc):
    for M, N, K, MT, NT in REF["cases"]:
        t = orc.choose_tile_ref(M, N, _kpad(K))
        assert (t[0], t[1]) == (MT, NT), (M, N, K, t)


def test_oracle_router_matches_reference_library(orc, ref_lib):
    import ctypes as C
    t = (C.c_int * 4)()
    for M in range(128, 8193, 384):
        for N in range(128, 24577, 640):
            for K in (512, 4096, 16128, 32768, 105728):
                Kp = _kpad(K)
                ref_lib.ref_choose_tile(M, N, Kp, t)
                assert orc.choose_tile_ref(M, N, Kp) == tuple(t), (M, N, K)
                assert orc.splitk_s_ref(M, N, Kp) * M * N * 4 == \
                    (ref_lib.ref_gemm_workspace_size(M, N, Kp) or M * N * 4), (M, N, K)


def test_oracle_split_plan_reference_cases(orc):
    for M, N, K in REF["no_split"]:
        assert orc.splitk_s_ref(M, N, _kpad(K)) == 1
    for M, N, K in REF["degenerate"]:
        orc.splitk_s_ref(M, N, _kpad(K))  # must return, not trap
    # the narrow-N / large-K benchmark shape splits 4 ways in the reference
    assert orc.splitk_s_ref(2048, 1024, _kpad(105728)) == 4


def test_router_covers_every_multiple_of_128(mx):
    bad = 0
    for M in range(128, 16385, 128):
        for N in range(128, 24577, 128):
            for K in (512, 16128, 105728):
                t = mx.choose_tile(M, N, _kpad(K))
                if M % t[0] or N % t[1] or tuple(t) not in IMPLEMENTED:
                    bad += 1
    assert bad == 0


def test_workspace_matches_split(mx):
    for M in (128, 256, 1024, 2048, 4096, 8192):
        for N in (128, 256, 384, 1024, 5120, 6144, 8192):
            for K in (1024, 4096, 16128, 105728):
                Kp = _kpad(K)
                S = mx.splitk_segments(M, N, Kp)
                rp = mx.repacks_a(M, N, Kp)
                ws = mx.workspace_size(M, N, Kp)
                # split partials first, then the repacked A at the next 256-byte boundary
                split = S * M * N * 4 if S > 1 else 0
                want = (split + 255) // 256 * 256 + (M * Kp // 4 * 3 if rp else 0)
                assert ws == want, (M, N, K, S, rp, ws)
                assert mx.plan_workspace_size(M, N, Kp, S, rp) == want
                if S > 1:
                    assert Kp // 192 // S >= 8 and S <= 16  # every segment >= 8 K-tiles


def test_router_degenerate_shapes_do_not_trap(mx):
    for M, N, K in REF["degenerate"] + [[0, 0, 192], [-128, 256, 192], [128, 128, 0]]:
        mx.choose_tile(M, N, _kpad(K))
        assert mx.workspace_size(M, N, _kpad(K)) == 0


def test_router_benchmark_shapes(mx):
    # the MI355X routing of the five benchmark workloads (256x256 or 256x192 whenever the grid has
    # >= 64 workgroups, else cost: CU waves x workgroup work, ties to the larger tile). Split counts
    # follow the CU-wave time model: 160 workgroups over 551 K-tiles take 3 segments (480
    # workgroups, two waves of a third of K each: 2/3 of the unsplit time), 32 workgroups take 8.
    want = {
        (256, 256, 1024): ((128, 128, 2, 2), 1),
        (8192, 8192, 8192): ((256, 256, 4, 4), 1),
        (2048, 6144, 16128): ((256, 192, 4, 3), 1),
        (2048, 1024, 105728): ((256, 256, 4, 4), 8),
        (2048, 5120, 105728): ((256, 256, 4, 4), 3),
    }
    for (M, N, K), exp in want.items():
        t = mx.choose_tile(M, N, _kpad(K))
        S = mx.splitk_segments(M, N, _kpad(K))
        assert (tuple(t), S) == exp, (M, N, K, t, S)
    # A is repacked where the output has >= 8 tile columns
    for (M, N, K), rp in {(8192, 8192, 8192): True, (2048, 6144, 16128): True,
                          (2048, 1024, 105728): False, (2048, 5120, 105728): True,
                          (256, 256, 1024): False}.items():
        assert mx.repacks_a(M, N, _kpad(K)) == rp, (M, N, K)
