"""Helpers of the GPU parity tests: upload a Problem, run a library entry point through the C
ABI, read D back as float32. torch provides device memory and the stream only."""
import sys

import numpy as np
import torch

import mxfp6_amd as mx

TORCH_OUT = {0: torch.float32, 1: torch.float16, 2: torch.bfloat16}


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def routed_shape(cands, want):
    """The first (M, N, K) of cands whose routed plan (tile, K segments, A repacked) satisfies
    want(tile, S, repack): tests that need a given route search for it, so that a refit of the
    router's model cannot silently move them off it."""
    for M, N, K in cands:
        Kp = mx.kpad(K)
        if want(tuple(mx.choose_tile(M, N, Kp)), mx.splitk_segments(M, N, Kp),
                mx.repacks_a(M, N, Kp)):
            return M, N, K
    raise AssertionError("no candidate shape reaches the route")


class DevProblem:
    """Device copies of a Problem's operands laid out for one tile's scale grouping."""

    def __init__(self, p: mx.Problem, tile, dev="cuda"):
        self.p = p
        self.tile = tuple(tile)
        bsh, sa, sb = p.layouts(tile)
        self.a = torch.from_numpy(p.a_packed).to(dev)
        self.bsh = torch.from_numpy(bsh).to(dev)
        self.sa = torch.from_numpy(sa).to(dev)
        self.sb = torch.from_numpy(sb).to(dev)

    def out(self, out_type):
        n = self.p.M * self.p.N * mx.OUT_BYTES[out_type]
        return torch.full((n,), 0x5A, dtype=torch.uint8, device=self.a.device)

    def ptrs(self):
        return self.a.data_ptr(), self.bsh.data_ptr(), self.sa.data_ptr(), self.sb.data_ptr()


def to_f32(buf: torch.Tensor, out_type, M, N) -> np.ndarray:
    return buf.view(TORCH_OUT[out_type]).float().reshape(M, N).cpu().numpy()


def run_routed(dp: DevProblem, out_type, with_ws=True, stream=None, ws_kind="preferred"):
    """ws_kind: "preferred" (the plan's whole workspace, repack included) or "split" (exactly
    gemm_workspace_size's bytes, the reference's meaning: A is then read row-major)."""
    p = dp.p
    size = mx.preferred_workspace_size if ws_kind == "preferred" else mx.workspace_size
    ws_bytes = size(p.M, p.N, p.Kp) if with_ws else 0
    ws = torch.empty(max(ws_bytes, 4), dtype=torch.uint8, device="cuda") if ws_bytes else None
    D = dp.out(out_type)
    a, b, sa, sb = dp.ptrs()
    say(f"  gemm {p.M}x{p.N}x{p.K} (Kp {p.Kp}) out {mx.OUT_NAMES[out_type]} tile {dp.tile} "
        f"ws {ws_bytes}")
    rc = mx.gemm(out_type, p.M, p.N, p.Kp, a, b, sa, sb, D.data_ptr(), p.a_row_bytes,
                 ws.data_ptr() if ws is not None else 0, ws_bytes,
                 stream=None if stream is None else stream.cuda_stream)
    assert rc == 0, mx.STATUS.get(rc, rc)
    torch.cuda.synchronize()
    return to_f32(D, out_type, p.M, p.N)


def run_forced(dp: DevProblem, out_type):
    p = dp.p
    D = dp.out(out_type)
    a, b, sa, sb = dp.ptrs()
    say(f"  force {dp.tile} {p.M}x{p.N}x{p.K} out {mx.OUT_NAMES[out_type]}")
    rc = mx.gemm_force_tile(out_type, p.M, p.N, p.Kp, dp.tile, a, b, sa, sb, D.data_ptr(),
                            p.a_row_bytes)
    if rc == 4:
        import pytest
        pytest.skip(f"tile {dp.tile} has no pipelined-kernel instantiation")
    assert rc == 0, mx.STATUS.get(rc, rc)
    torch.cuda.synchronize()
    return to_f32(D, out_type, p.M, p.N)


def run_direct(dp: DevProblem, out_type, splits=1):
    p = dp.p
    ws_bytes = splits * p.M * p.N * 4 if splits > 1 else 0
    ws = torch.empty(max(ws_bytes, 4), dtype=torch.uint8, device="cuda")
    D = dp.out(out_type)
    a, b, sa, sb = dp.ptrs()
    say(f"  direct {p.M}x{p.N}x{p.K} groups {dp.tile[2:]} out {mx.OUT_NAMES[out_type]} S {splits}")
    rc = mx.gemm_direct(out_type, p.M, p.N, p.Kp, dp.tile[2], dp.tile[3], a, b, sa, sb,
                        D.data_ptr(), p.a_row_bytes, splits, ws.data_ptr() if ws_bytes else 0,
                        ws_bytes)
    assert rc == 0, mx.STATUS.get(rc, rc)
    torch.cuda.synchronize()
    return to_f32(D, out_type, p.M, p.N)


def run_explicit(dp: DevProblem, out_type, splits=1, a_layout=0, a_dev=None):
    """a_layout 2 reads A from a_dev (a device tensor holding A preshuffled)."""
    p = dp.p
    ws_bytes = mx.plan_workspace_size(p.M, p.N, p.Kp, splits, a_layout == 1)
    ws = torch.empty(max(ws_bytes, 4), dtype=torch.uint8, device="cuda")
    D = dp.out(out_type)
    a, b, sa, sb = dp.ptrs()
    if a_dev is not None:
        a = a_dev.data_ptr()
    say(f"  explicit {dp.tile} {p.M}x{p.N}x{p.K} out {mx.OUT_NAMES[out_type]} S {splits} "
        f"A layout {a_layout}")
    rc = mx.gemm_explicit(out_type, p.M, p.N, p.Kp, dp.tile, splits, a, b, sa, sb, D.data_ptr(),
                          p.a_row_bytes, ws.data_ptr() if ws_bytes else 0, ws_bytes,
                          a_layout=a_layout)
    assert rc == 0, mx.STATUS.get(rc, rc)
    torch.cuda.synchronize()
    return to_f32(D, out_type, p.M, p.N)
