"""Parity at the benchmark workloads' full sizes (8192^3 FP16; 2048x6144x16128 FP16;
2048x1024x105728 FP16 split-K; 2048x5120x105728 BF16 split-K), through the routed gemm().

The FP64 oracle is too slow for every element at these sizes, so three checks cover the output:
  * sampled rows and sampled columns, every element of each, against the FP64 oracle at the
    usual per-element bar (columns come from the transposed problem: D^T = B^T A^T);
  * every row sum and every column sum of D against FP64 GEMVs of the exactly dequantised
    operands (column sums = (1^T A) B, row sums = A (B 1)), within the sum of the per-element bars
    of that row or column (1e-5 * sum|ab| for the FP32 accumulation, plus half an ulp of the
    output format per element, 2^-11 |D| for FP16 and 2^-8 |D| for BF16, plus the smallest
    subnormal step);
  * the total sum (a checksum of the checksums) against 1^T A B 1.
A tile written to the wrong place, a missing or doubled K segment, or a scale group applied to
the wrong rows moves some row or column sum by far more than its bound.
"""
import numpy as np
import pytest

import checks
import mxfp6_amd as mx
import oracle
from gpu_util import say, TORCH_OUT

pytestmark = pytest.mark.gpu

SEED = 0x4D584636
WORKLOADS = {
    "c2": (8192, 8192, 8192, mx.OUT_F16, (mx.DIST_NORMAL, 1.0), (mx.DIST_NORMAL, 1.0)),
    "c3": (2048, 6144, 16128, mx.OUT_F16, (mx.DIST_NORMAL, 2.0), (mx.DIST_UNIFORM, 1.0)),
    "c4": (2048, 1024, 105728, mx.OUT_F16, (mx.DIST_NORMAL, 1.0), (mx.DIST_NORMAL, 1.0)),
    "c5": (2048, 5120, 105728, mx.OUT_BF16, (mx.DIST_STUDENT_T3, 1.0), (mx.DIST_STUDENT_T3, 1.0)),
}


def _check_lines(D, R, ab, out_type):
    if out_type == mx.OUT_F32:
        checks.check_f32(D, R, ab)
    else:
        checks.check_lowp(D, R, mx.OUT_NAMES[out_type])


@pytest.mark.parametrize("name", sorted(WORKLOADS))
def test_full_size_workload(name):
    import torch

    M, N, K, ot, (da, sa_), (db, sb_) = WORKLOADS[name]
    say(f"full-size parity {name}: {M}x{N}x{K} out {mx.OUT_NAMES[ot]}")
    p = mx.make_problem(M, N, K, da, sa_, db, sb_, seed=SEED ^ int(name[1:]))
    tile = mx.choose_tile(M, N, p.Kp)
    bsh, sa, sb = p.layouts(tile)
    dev = "cuda"
    dA = torch.from_numpy(p.a_packed).to(dev)
    dB, dsa, dsb = (torch.from_numpy(x).to(dev) for x in (bsh, sa, sb))
    ws_bytes = mx.preferred_workspace_size(M, N, p.Kp)
    ws = torch.empty(max(ws_bytes, 4), dtype=torch.uint8, device=dev)
    D = torch.full((M * N * mx.OUT_BYTES[ot],), 0x5A, dtype=torch.uint8, device=dev)
    rc = mx.gemm(ot, M, N, p.Kp, dA.data_ptr(), dB.data_ptr(), dsa.data_ptr(), dsb.data_ptr(),
                 D.data_ptr(), p.a_row_bytes, ws.data_ptr(), ws_bytes)
    assert rc == 0, mx.STATUS.get(rc, rc)
    torch.cuda.synchronize()
    Dt = D.view(TORCH_OUT[ot]).reshape(M, N)
    D64 = Dt.double()
    col_sum = D64.sum(dim=0).cpu().numpy()
    row_sum = D64.sum(dim=1).cpu().numpy()
    col_abs = D64.abs().sum(dim=0).cpu().numpy()
    row_abs = D64.abs().sum(dim=1).cpu().numpy()
    total = float(D64.sum().item())
    rows = np.r_[0:3, M // 2 - 1:M // 2 + 2, M - 3:M, 257, 1023 % M]
    cols = np.r_[0:3, N // 2 - 1:N // 2 + 2, N - 3:N, 191, 4095 % N]
    Drows = Dt[torch.from_numpy(rows).to(dev)].float().cpu().numpy()
    Dcols = Dt[:, torch.from_numpy(cols).to(dev)].float().cpu().numpy().T
    del D64, Dt, D, dA, dB, ws
    torch.cuda.empty_cache()

    # every element of the sampled rows and columns
    R, ab = oracle.gemm_f64(p.a_packed, p.a_row_bytes, p.a_scales, p.b_packed, p.b_row_bytes,
                            p.b_scales, M, N, K, rows=rows)
    _check_lines(Drows, R, ab, ot)
    Rc, abc = oracle.gemm_f64(p.b_packed, p.b_row_bytes, p.b_scales, p.a_packed, p.a_row_bytes,
                              p.a_scales, N, M, K, rows=cols)
    _check_lines(Dcols, Rc, abc, ot)

    # row and column checksums against FP64 GEMVs of the dequantised operands
    Af = oracle.dequant_f32(p.a_packed, p.a_row_bytes, p.a_scales, M, K)
    Bf = oracle.dequant_f32(p.b_packed, p.b_row_bytes, p.b_scales, N, K)   # B^T: [N][K]
    rc_col, rc_row = checks.check_checksums(col_sum, row_sum, col_abs, row_abs, total, Af, Bf, ot)
    say(f"  {name}: rows/cols exact to the bar; checksum error / bound: columns {rc_col:.3f}, "
        f"rows {rc_row:.3f}")
