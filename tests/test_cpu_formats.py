"""Element formats, packing, quantisers and the workload generator (CPU only).

Three implementations meet here: the library (product, mxfp6_amd), the oracle's C restatement
(oracle/), and the reference's own code compiled from its sources (oracle/_ref). The oracle is
pinned by fixtures (OCP value table, hand-derived packing KATs, PCG32 reference output) and by
brute force; the library must equal it byte for byte.
"""
import json
import math
import os

import numpy as np
import pytest

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _load(name):
    with open(os.path.join(GOLD, name)) as f:
        return json.load(f)


def _values_table():
    mags = _load("e2m3_table.json")["magnitudes"]
    return [m for m in mags] + [-m for m in mags]


# ---- FP6 E2M3 decode -----------------------------------------------------------------------------

def test_e2m3_decode_matches_ocp_table(mx, orc):
    table = _values_table()
    for code in range(64):
        want = table[code]
        assert orc.lib().o_fp6_decode(code) == want, code
        assert mx.lib().mxfp6_fp6_e2m3_to_float(code) == want, code


def test_e2m3_decode_reference(ref_lib):
    table = _values_table()
    for code in range(64):
        assert ref_lib.ref_fp6_decode(code) == table[code]


# ---- FP6 E2M3 encode -----------------------------------------------------------------------------

def _encode_probe_values():
    mags = _load("e2m3_table.json")["magnitudes"]
    vals = set()
    for i, m in enumerate(mags):
        vals.add(m)
        if i + 1 < len(mags):
            mid = (m + mags[i + 1]) / 2  # exact ties
            vals.update([mid, np.nextafter(np.float32(mid), np.float32(0)),
                         np.nextafter(np.float32(mid), np.float32(10))])
    vals.update([7.5, 7.6, 7.75, 8.0, 100.0, 1e30, np.float32(np.finfo(np.float32).max),
                 1e-30, 1e-45, 0.0625, 0.0624, 0.0626, 0.9375, 1.9375, 3.875, 7.25, 6.75])
    rng = np.random.default_rng(1)
    dense = np.concatenate([np.linspace(0, 9, 20001), rng.uniform(0, 8, 20000),
                            np.exp(rng.uniform(-20, 3, 5000))])
    vals.update(float(v) for v in dense)
    out = []
    for v in vals:
        out.extend([np.float32(v), np.float32(-v)])
    out.append(np.float32(-0.0))
    return out


def _brute_nearest(v: float, table_mags):
    """Independent rule: nearest magnitude, ties to the even code, saturating at 7.5."""
    a = min(abs(float(v)), 7.5)
    best, bd = 0, math.inf
    for c, m in enumerate(table_mags):
        d = abs(a - m)
        if d < bd or (d == bd and c % 2 == 0 and best % 2 == 1):
            best, bd = c, d
    sign = 0x20 if v < 0 else 0
    return sign | best


def test_e2m3_encode_product_equals_oracle_bruteforce(mx, orc):
    mags = _load("e2m3_table.json")["magnitudes"]
    vals = _encode_probe_values()
    enc_p = mx.lib().mxfp6_float_to_fp6_e2m3
    enc_o = orc.lib().o_fp6_encode
    for v in vals[::7]:  # python brute force on a subsample
        assert enc_o(v) == _brute_nearest(v, mags), v
    for v in vals:
        assert enc_p(v) == enc_o(v), (float(v), enc_p(v), enc_o(v))


def test_e2m3_encode_reference(mx, ref_lib):
    enc_p = mx.lib().mxfp6_float_to_fp6_e2m3
    for v in _encode_probe_values():
        assert enc_p(v) == ref_lib.ref_fp6_encode(v), float(v)


def test_e2m3_roundtrip_every_code(mx):
    for code in range(64):
        v = mx.lib().mxfp6_fp6_e2m3_to_float(code)
        back = mx.lib().mxfp6_float_to_fp6_e2m3(v)
        if code == 0x20:  # -0.0 encodes as +0 (v < 0 is false)
            assert back == 0
        else:
            assert back == code, code


# ---- E8M0 ------------------------------------------------------------------------------------------

def test_e8m0_decode_closed_form(mx, orc):
    for u in range(255):
        assert mx.lib().mxfp6_e8m0_to_float(u) == np.float32(2.0 ** (u - 127)), u
        assert orc.lib().o_e8m0_decode(u) == 2.0 ** (u - 127)
    assert math.isnan(mx.lib().mxfp6_e8m0_to_float(255))
    assert math.isnan(orc.lib().o_e8m0_decode(255))


def test_e8m0_encode_reference(mx, ref_lib):
    rng = np.random.default_rng(2)
    vals = [np.float32(x) for x in np.exp(rng.uniform(-87, 87, 20000))]
    vals += [np.float32(2.0 ** e) for e in range(-126, 128)] + [np.float32(0), np.float32(-1),
                                                                np.float32(1.4142135), np.float32(1.4142137)]
    for v in vals:
        assert mx.lib().mxfp6_float_to_e8m0(v) == ref_lib.ref_e8m0_encode(v), float(v)


# ---- packing -------------------------------------------------------------------------------------

def test_pack_kat(mx, orc):
    import ctypes as C
    for case in _load("pack_kat.json")["cases"]:
        codes = np.array(case["codes"], dtype=np.uint8)
        want = np.array(case["bytes"], dtype=np.uint8)
        assert np.array_equal(orc.pack(codes), want)
        out = np.zeros(3, dtype=np.uint8)
        assert mx.lib().mxfp6_pack_fp6(codes.ctypes.data, 4, out.ctypes.data) == 0
        assert np.array_equal(out, want), case
        back = np.zeros(4, dtype=np.uint8)
        assert mx.lib().mxfp6_unpack_fp6(want.ctypes.data, 4, back.ctypes.data) == 0
        assert np.array_equal(back, codes)
    assert mx.lib().mxfp6_pack_fp6(C.c_void_p(1), 6, C.c_void_p(1)) != 0  # n % 4 != 0


def test_pack_random_three_ways(mx, orc, ref_lib):
    rng = np.random.default_rng(3)
    codes = rng.integers(0, 64, 4096, dtype=np.uint8)
    want = orc.pack(codes)
    out = np.zeros_like(want)
    mx.lib().mxfp6_pack_fp6(codes.ctypes.data, codes.size, out.ctypes.data)
    assert np.array_equal(out, want)
    r = np.zeros_like(want)
    ref_lib.ref_pack(codes.ctypes.data, codes.size, r.ctypes.data)
    assert np.array_equal(r, want)
    assert np.array_equal(orc.unpack(want, codes.size), codes)


# ---- quantize_to_mxfp6 (reference rule) ---------------------------------------------------------

def _special_matrix(rows, cols, seed):
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 1, (rows, cols)).astype(np.float32)
    x[0, :32] = 0.0                                   # all-zero block -> scale 127
    x[0, 32:64] = 7.5                                 # amax / 7.5 exactly a power of two
    x[1, :32] = rng.normal(0, 1e-38, 32)             # tiny (clamped scale code 0 region)
    x[1, 32:64] = rng.normal(0, 1e30, 32)            # huge
    x[2, :32] = 2.0 ** rng.integers(-10, 10, 32)      # powers of two
    x[2, 32:64] = -0.0
    x[3] *= 1e-3
    return x


@pytest.mark.parametrize("rows,cols", [(8, 64), (37, 256), (64, 1024)])
def test_quantize_ref_rule_three_ways(mx, orc, ref_lib, rows, cols):
    x = _special_matrix(rows, cols, rows * cols)
    po, so = orc.quantize_ref(x)
    pp, sp = mx.quantize(x)
    assert np.array_equal(sp, so) and np.array_equal(pp, po)
    pr = np.empty_like(po)
    sr = np.empty_like(so)
    ref_lib.ref_quantize(x.ctypes.data, rows, cols, pr.ctypes.data, sr.ctypes.data)
    assert np.array_equal(sr, so) and np.array_equal(pr, po)


def test_quantize_scale_rule_closed_form(mx):
    # amax = 7.5 * 2^e exactly -> scale 2^e; amax slightly above -> 2^(e+1)
    for e in (-20, -3, 0, 5, 40):
        x = np.zeros((1, 32), dtype=np.float32)
        x[0, 5] = 7.5 * 2.0 ** e
        _, s = mx.quantize(x)
        assert s[0, 0] == e + 127
        x[0, 5] = np.nextafter(np.float32(7.5 * 2.0 ** e), np.float32(np.inf))
        _, s = mx.quantize(x)
        assert s[0, 0] == e + 128


def test_dequantize_matches_reference(mx, ref_lib):
    x = _special_matrix(16, 256, 9)
    p, s = mx.quantize(x)
    d = mx.dequantize(p, s, 16, 256)
    r = np.empty_like(d)
    ref_lib.ref_dequantize(p.ctypes.data, s.ctypes.data, 16, 256, r.ctypes.data)
    assert np.array_equal(d.view(np.uint32), r.view(np.uint32))


def test_preprocess_b_matches_reference(mx, ref_lib):
    rng = np.random.default_rng(4)
    B = rng.normal(0, 1, (192, 64)).astype(np.float32)
    p, s = mx.preprocess_b(B)
    pr, sr = np.empty_like(p), np.empty_like(s)
    ref_lib.ref_preprocess_b(B.ctypes.data, 192, 64, pr.ctypes.data, sr.ctypes.data)
    assert np.array_equal(p, pr) and np.array_equal(s, sr)


# ---- workload generator (PCG32 + OCP MX rule) -----------------------------------------------------

def test_pcg32_known_answer(mx):
    kat = _load("pcg32_kat.json")
    o = kat["outputs"]
    v = mx.gen_values(1, 32, mx.DIST_UNIFORM, 1.0, kat["seed"], kat["stream"])[0]
    for i in range(3):
        u = ((o[2 * i] >> 5) * 67108864.0 + (o[2 * i + 1] >> 6)) / 9007199254740992.0
        assert v[i] == np.float32(2.0 * u - 1.0), i


def test_generator_rows_are_one_stream(mx):
    # row r starts at draw r * K * draws_per_value: two rows of K == one row of 2K
    for dist in (mx.DIST_NORMAL, mx.DIST_UNIFORM, mx.DIST_STUDENT_T3):
        two = mx.gen_values(2, 64, dist, 1.0, 7, 3)
        one = mx.gen_values(1, 128, dist, 1.0, 7, 3)
        assert np.array_equal(two.ravel(), one.ravel()), dist
        # thread count does not change the stream
        assert np.array_equal(mx.gen_values(9, 64, dist, 1.0, 7, 3, nthreads=1),
                              mx.gen_values(9, 64, dist, 1.0, 7, 3, nthreads=4))


def test_generator_distributions(mx):
    n = mx.gen_values(64, 4096, mx.DIST_NORMAL, 2.0, 11, 1).ravel().astype(np.float64)
    assert abs(n.mean()) < 0.02 and abs(n.std() - 2.0) < 0.02
    assert abs((np.abs(n) > 2 * 1.96).mean() - 0.05) < 0.005
    u = mx.gen_values(64, 4096, mx.DIST_UNIFORM, 1.0, 11, 2).ravel().astype(np.float64)
    assert u.min() >= -1 and u.max() < 1 and abs(u.mean()) < 0.01 and abs(u.var() - 1 / 3) < 0.01
    t = mx.gen_values(64, 4096, mx.DIST_STUDENT_T3, 1.0, 11, 3).ravel().astype(np.float64)
    # t(3): P(|T| > 3.182) = 0.05, variance 3 (heavy tails)
    assert abs((np.abs(t) > 3.182446).mean() - 0.05) < 0.005
    assert np.median(np.abs(t)) == pytest.approx(0.7649, abs=0.02)


@pytest.mark.parametrize("dist,sigma", [(0, 1.0), (0, 2.0), (1, 1.0), (2, 1.0)])
def test_generator_quantisation_is_ocp_rule(mx, orc, dist, sigma):
    rows, K = 48, 1024
    x = mx.gen_values(rows, K, dist, sigma, 0x4D584636, 1)
    po, so = orc.quantize_ocp(x)
    pp, sp = mx.gen_operand(rows, K, dist, sigma, 0x4D584636, 1)
    assert np.array_equal(sp, so)
    assert np.array_equal(pp, po)


def test_ocp_scale_rule_bruteforce(orc):
    # o_quantize_ocp against the rule written as arithmetic on exponents (python, independent)
    rng = np.random.default_rng(5)
    x = (rng.standard_t(3, (16, 256)) * 10.0 ** rng.uniform(-3, 3, (16, 1))).astype(np.float32)
    _, s = orc.quantize_ocp(x)
    amax = np.abs(x.reshape(16, 8, 32)).max(axis=2).astype(np.float64)
    want = np.clip(np.floor(np.log2(amax)).astype(int) - 2 + 127, 0, 254)
    assert np.array_equal(s.astype(int), want)


def test_generator_padding_and_tails(mx):
    K, Kp = 1024, 1152
    p, s = mx.gen_operand(4, K, mx.DIST_NORMAL, 1.0, 1, 2, row_bytes=Kp // 4 * 3, scale_cols=Kp // 32)
    p = p.reshape(4, Kp // 4 * 3)
    assert (p[:, K // 4 * 3:] == 0).all()
    assert (s[:, K // 32:] == 127).all()
