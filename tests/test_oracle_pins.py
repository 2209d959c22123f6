"""Pins the CPU oracle to the reference's own printed outputs.

The reference's arithmetic library (xlnscpp) is an absent submodule, so the
oracle restates it; these tests check the restatement against every figure the
reference's tests committed (tests/golden/reference_figures.json, copied from
results/sum32-evidence/*.txt and convert.jsonl) by re-running the reference
tests' own deterministic input generators:
  - lns-backend/tests/test-lns16-sum32.cpp (LCG 0x2545F4914F6CDD1D), and
  - lns-backend/tests/test-lns-backend.cpp (closed-form patterns and the LCG
    0x9E3779B97F4A7C15 of the K=1536 case),
plus closed-form and brute-force invariants of the formats.
"""
import json
import math
import os

import numpy as np
import pytest

import oracle_lib as O

HERE = os.path.dirname(os.path.abspath(__file__))
FIG = json.load(open(os.path.join(HERE, "golden", "reference_figures.json")))
M64 = (1 << 64) - 1


@pytest.fixture(scope="module")
def L():
    return O.lib()


# ---------------------------------------------------------------- formats --

def test_xlns16_known_codes(L):
    # unit-tests-lns16-base.txt div values: fp2xlns16(5)=297, (6)=330, (9)=405,
    # (0.1)=-425, (7)=359, (100)=850 in log units
    for v, code in ((5.0, 297), (6.0, 330), (9.0, 405), (0.1, -425), (7.0, 359), (100.0, 850),
                    (10.0, 425), (2.0, 128), (0.5, -128), (1.0, 0)):
        c = L.lno16_from_f32(v)
        assert c & 0x8000 == 0
        assert (c & 0x7fff) - 0x4000 == code, v
        c = L.lno16_from_f32(-v)
        assert c & 0x8000 and (c & 0x7fff) - 0x4000 == code


def test_xlns16_printed_div_values(L):
    # test-lns-backend.cpp:509-549 div cases (inputs of the reference test)
    f = FIG["unit_tests"]["base"]

    def div(a, b):
        return ["%.6f" % L.lno16_to_f32(L.lno16_div(L.lno16_from_f32(x), L.lno16_from_f32(y))) for x, y in zip(a, b)]

    assert div([8, -6, 5, 1, 0.5, -0.25, 100, -3], [2, 3, -1, 4, 0.5, 0.1, 7, -6]) == f["div"]
    assert div([8, -6, 5, 1, 0.5, -0.25], [2] * 6) == f["div_scalar"]
    a2 = [8, -6, 5, 1, 4, -2, 9, 3, 1, 2, 6, -4]
    assert div(a2, [2, -1] * 6) == f["div_2d"]


def test_xlns16_decode_is_seven_digit_decimal(L):
    # 2^(1355/128) prints as 1537.0380, 2^(491/128) as 14.280130 in the reference
    assert "%.4f" % L.lno16_to_f32(0x4000 + 1355) == "1537.0380"
    assert "%.6f" % L.lno16_to_f32(0x4000 + 491) == "14.280130"
    assert "%.6f" % L.lno16_to_f32(0x4000 + 202) == "2.985816"


def test_mul_div_recip_closed_form(L):
    rng = np.random.default_rng(1)
    a = rng.integers(0x4000 - 3000, 0x4000 + 3000, 2000)
    b = rng.integers(0x4000 - 3000, 0x4000 + 3000, 2000)
    for x, y in zip(a, b):
        sx, sy = int(rng.integers(0, 2)) << 15, int(rng.integers(0, 2)) << 15
        p = L.lno16_mul(int(x) | sx, int(y) | sy)
        assert p == ((sx ^ sy) | (int(x) + int(y) - 0x4000))
        q = L.lno16_div(int(x) | sx, int(y) | sy)
        assert q == ((sx ^ sy) | (int(x) - int(y) + 0x4000))
        r = L.lno16_recip(int(x) | sx)
        assert r == (sx | (0x8000 - int(x)))
    # overflow saturates, underflow gives a (signed) zero
    assert L.lno16_mul(0x7f00, 0x7f00) == 0x7fff
    assert L.lno16_mul(0x8100, 0x0100) == 0x8000
    assert L.lno16_mul(0x0100, 0x0100) == 0x0000


def test_sqrt_rounds_half_away(L):
    for l in range(-5000, 5000, 7):
        s = L.lno16_sqrt(0x4000 + l)
        want = math.ceil(l / 2) if l >= 0 else math.floor(l / 2)
        assert (s & 0x7fff) - 0x4000 == want and s & 0x8000 == 0


def test_widen_narrow_roundtrip(L):
    # test-lns16-sum32.cpp:57-68: narrow(widen(x)) == x for all codes
    for x in range(65536):
        assert L.lno16_narrow_sum32(L.lno16_widen(x)) == x


def test_canonical_order_is_real_order(L):
    rng = np.random.default_rng(3)
    codes = rng.integers(1, 65536, 400)
    codes = [int(c) for c in codes if c & 0x7fff]
    vals = [float(L.lno16_to_f32(c)) for c in codes]
    for i in range(len(codes) - 1):
        a, b = codes[i], codes[i + 1]
        if vals[i] != vals[i + 1]:
            assert bool(L.lno16_gt(a, b)) == (vals[i] > vals[i + 1])
    assert all(L.lno16_gt(c, 0xffff) for c in codes if c != 0xffff)


def test_sb_db_tables_match_gaussian_logs(L):
    sb = O.table("lno16_sb_table", 1281, np.int16)
    db = O.table("lno16_db_table", 1281, np.int16)
    d = np.arange(1281)
    exact_sb = 128 * np.log2(1 + 2.0 ** (-d / 128))
    assert np.all(np.abs(sb - exact_sb) <= 0.5 + 1e-9)
    exact_db = 128 * np.log2(1 - 2.0 ** (-d[1:] / 128))
    # db rounds like (int)(x + .5) on log2(2^(d/128) - 1): correctly rounded
    # for d >= 128, one step toward zero short of that below (negative
    # argument, truncation rounds up)
    err = db[1:] - exact_db
    assert np.all(np.abs(err[127:]) <= 0.5 + 1e-9)
    assert np.all((err[:127] > 0) & (err[:127] < 1.5))
    assert sb[1092] == 0 and sb[1091] == 1   # stagnation point of base sums


# ------------------------------------------------------------- conversion --

# -------------------------------------------------- standalone sum32 test --

class _Lcg:
    """test-lns16-sum32.cpp:25-29"""

    def __init__(self):
        self.s = 0x2545F4914F6CDD1D

    def __call__(self):
        self.s = (self.s * 6364136223846793005 + 1442695040888963407) & M64
        return ((self.s >> 11) & ((1 << 53) - 1)) / float(1 << 53)


def _ideal16(v):
    if v == 0.0:
        return 0
    l = math.log2(abs(v)) * 128.0
    c = (math.floor(l + 0.5) if l >= 0 else -math.floor(-l + 0.5)) + 0x4000
    c = max(0, min(0x7FFF, c))
    return (0x8000 if v < 0 else 0) | c


def _ulp(a, b):
    if (a & 0x8000) != (b & 0x8000):
        return 0x7FFF
    return abs((a & 0x7FFF) - (b & 0x7FFF))


@pytest.fixture(scope="module")
def standalone(L):
    """Re-runs test-lns16-sum32.cpp's five checks with its own LCG stream."""
    rnd = _Lcg()
    out = {}
    f2x, x2f = L.lno16_from_f32, L.lno16_to_f32
    wb = ws = tb = ts = cnt = 0
    for _ in range(200000):
        ea = rnd() * 40.0 - 20.0
        eb = ea + rnd() * 40.0 - 20.0
        va, vb = 2.0 ** ea, 2.0 ** eb
        if rnd() < 0.5:
            va = -va
        if rnd() < 0.5:
            vb = -vb
        a, b = f2x(np.float32(va)), f2x(np.float32(vb))
        ex = float(x2f(a)) + float(x2f(b))
        if ex == 0.0:
            continue
        w = _ideal16(ex)
        db = _ulp(L.lno16_add(a, b), w)
        ds = _ulp(L.lno16_narrow_sum32(L.lno32_add(a << 16, b << 16)), w)
        wb, ws, tb, ts, cnt = max(wb, db), max(ws, ds), tb + db, ts + ds, cnt + 1
    out["two_term"] = {"n": cnt, "base_max": wb, "base_mean": "%.3f" % (tb / cnt),
                       "sum32_max": ws, "sum32_mean": "%.3f" % (ts / cnt)}
    stag = {}
    for n in (128, 370, 512, 1536, 8960, 65536):
        v = np.full(n, 0x4000, np.uint16)
        stag[str(n)] = {"base": "%.4f" % float(x2f(O.sum16(O.BASE, v))),
                        "sum32": "%.4f" % float(x2f(O.sum16(O.SUM32, v)))}
    out["stagnation"] = stag
    dots = {}
    for K in (1536, 8960):
        srb = srs = 0.0
        wins = 0
        for _ in range(64):
            u = np.array([rnd() for _ in range(2 * K)])
            a = O.f2x16((u[0::2] * 2.0 - 1.0).astype(np.float32))
            b = O.f2x16((u[1::2] * 2.0 - 1.0).astype(np.float32))
            da, dbb = O.x2f16(a).astype(np.float64), O.x2f16(b).astype(np.float64)
            exact = 0.0
            for x, y in zip(da, dbb):
                exact += x * y
            gb = float(x2f(O.vec_dot16(O.BASE, a, b)))
            gs = float(x2f(O.vec_dot16(O.SUM32, a, b)))
            rb, rs = abs(gb - exact) / abs(exact), abs(gs - exact) / abs(exact)
            srb, srs, wins = srb + rb, srs + rs, wins + (rs < rb)
        dots[str(K)] = {"base": "%.3f" % (srb / 64 * 100), "sum32": "%.3f" % (srs / 64 * 100), "wins": wins}
    out["long_dot"] = dots
    rms = {}
    for n in (576, 1536):
        x = np.array([f2x(np.float32(rnd() * 2.0 - 1.0)) for _ in range(n)], np.uint16)
        xf = O.x2f16(x).astype(np.float64)
        sq = 0.0
        for v in xf:
            sq += v * v
        inv = 1.0 / math.sqrt(sq / n + 1e-6)
        eps = f2x(np.float32(1e-6))
        rb_ = O.x2f16(O.rms_norm_row16(O.BASE, x, eps)).astype(np.float64)
        rs_ = O.x2f16(O.rms_norm_row16(O.SUM32, x, eps)).astype(np.float64)
        want = xf * inv
        den = np.maximum(np.abs(want), 1e-6)
        rms[str(n)] = {"base": "%.3f" % (np.max(np.abs(rb_ - want) / den) * 100),
                       "sum32": "%.3f" % (np.max(np.abs(rs_ - want) / den) * 100)}
    out["rms_norm"] = rms
    return out


# ------------------------------------------------ backend unit-test suite --

A_K2 = np.array([[2, 8], [5, 1], [4, 2], [8, 6]], np.float32)
B_K2 = np.array([[10, 5], [9, 9], [5, 4]], np.float32)


def _long_operands():
    """test-lns-backend.cpp:221-245"""
    rng = 0x9E3779B97F4A7C15
    K, M, N = 1536, 8, 4
    vals = np.empty(M * K + N * K, np.float32)
    for i in range(vals.size):
        rng = (rng * 6364136223846793005 + 1442695040888963407) & M64
        vals[i] = np.float32(((rng >> 32) & 0xFFFFFFFF) / 2147483648.0 - 1.0)
    return vals[: M * K].reshape(M, K), vals[M * K:].reshape(N, K)


def _mm_long_figures(out, a, b):
    ref = b.astype(np.float64) @ a.astype(np.float64).T
    err = out.astype(np.float64) - ref
    rms = math.sqrt((ref ** 2).mean())
    return {"max_over_rms": "%.4f" % (np.abs(err).max() / rms * 100), "rms_ref": "%.4f" % rms,
            "nrmse": "%.4f" % (math.sqrt((err ** 2).sum() / (ref ** 2).sum()) * 100)}


def _softmax_case(ne00, ne01, scale, masked):
    """test-lns-backend.cpp:908-935 inputs and float reference"""
    i = np.arange(ne00)[None, :]
    r = np.arange(ne01)[:, None]
    u = ((i * 37 + r * 101) % 97).astype(np.float32) / np.float32(97.0)
    a = (np.float32(8.0) * (u - np.float32(0.5))).astype(np.float32)
    mask = None
    if masked:
        mask = np.zeros((ne01, ne00), np.float32)
        mask[np.broadcast_to((i >= ne00 - 1 - r) | ((i % 13) == 5), mask.shape)] = -np.inf
    want = np.empty_like(a)
    for rr in range(ne01):
        t = (a[rr] * np.float32(scale) + (mask[rr] if masked else np.float32(0))).astype(np.float32)
        t = np.exp((t - t.max()).astype(np.float32)).astype(np.float32)
        s = np.float32(0)
        for v in t:
            s = np.float32(s + v)
        want[rr] = (t / s).astype(np.float32)
    return a, mask, want


SOFTMAX_CASES = {"short": (8, 4, 1.0, False), "long": (512, 4, 1.0, False), "scaled": (512, 4, 0.125, False),
                 "masked": (64, 8, 1.0, True), "masked_scaled": (256, 4, 0.125, True)}


def _rms_case(ne00, ne01, eps=1e-5):
    """test-lns-backend.cpp:1004-1022 inputs and float reference"""
    i = np.arange(ne00)[None, :]
    r = np.arange(ne01)[:, None]
    u = ((i * 53 + r * 19) % 89).astype(np.float32) / np.float32(89.0)
    a = (np.float32(6.0) * (u - np.float32(0.5))).astype(np.float32)
    want = np.empty_like(a)
    for rr in range(ne01):
        ss = float(np.sum(a[rr].astype(np.float64) ** 2))
        want[rr] = a[rr] * (np.float32(1.0) / np.sqrt(np.float32(ss / ne00) + np.float32(eps)))
    return a, want


def test_swiglu_lns32_printed():
    # xlns32_silu is in the absent xlnscpp library: the oracle's definition
    # (sigmoid in double, fp2xlns32) reproduces the eight values the
    # reference printed for lns32_swiglu, to their six decimals
    gate = np.array([-3.0, -1.0, 0.0, 2.0, 1.5, -0.5, 4.0, -2.0], np.float32)
    up = np.array([0.5, -2.0, 3.0, 1.0, -1.0, 4.0, 0.25, 2.0], np.float32)
    got = ["%.6f" % v for v in O.swiglu32(gate, up)]
    assert got == FIG["unit_tests"]["lns32"]["swiglu"]
    # and they differ from the float swiglu in the last printed digits only
    want = gate / (1 + np.exp(-gate.astype(np.float64))) * up
    assert np.abs(O.swiglu32(gate, up) - want).max() < 2e-6


def test_lns32_elementwise_closed_forms():
    # add / mul of values exactly representable in xlns32 (powers of two)
    a = np.array([1.0, 2.0, -4.0, 0.5, 8.0], np.float32)
    b = np.array([1.0, 2.0, 4.0, 0.5, -8.0], np.float32)
    assert np.array_equal(O.mul32(a, b), a * b)
    assert np.array_equal(O.add32(a, b)[[0, 1, 3]], (a + b)[[0, 1, 3]])
    assert O.add32(a, b)[2] == 0.0 and O.add32(a, b)[4] == 0.0   # exact cancellation
    # rope at position 0 is the identity up to the xlns32 round trip
    x = np.random.default_rng(3).standard_normal((2, 3, 8)).astype(np.float32)
    y = O.rope32(x, np.zeros(2, np.int32), 8, 0, 10000.0)
    assert np.array_equal(y, O.x2f32(O.f2x32(x)))
    # rope is a rotation: norms of pairs kept to xlns32 precision
    y = O.rope32(x, np.array([5, 9], np.int32), 8, 0, 10000.0)
    n0 = np.hypot(x[..., 0::2], x[..., 1::2])
    n1 = np.hypot(y[..., 0::2], y[..., 1::2])
    assert np.abs(n1 - n0).max() < 1e-5


@pytest.mark.parametrize("w32", [False, True])
def test_scale_closed_forms(w32):
    # powers of two are exact codes in both formats, so x s is exact (zero is
    # the smallest code, not an exact zero, under multiplication)
    x = np.array([1.0, -2.0, 0.5, 4.0, -0.25], np.float32)
    for s in (2.0, -0.5, 1.0):
        assert np.array_equal(O.scale(w32, x, s), x * s)
    # b only enters when non-zero: 0 s + b is b's round trip, x s - x s cancels,
    # and 1 + 1 is exactly 2
    rt = O.x2f32(O.f2x32(np.float32([0.3]))) if w32 else O.x2f16(O.f2x16(np.float32([0.3])))
    assert O.scale(w32, np.float32([0.0]), 3.0, 0.3)[0] == rt[0]
    assert O.scale(w32, np.float32([2.0]), 4.0, -8.0)[0] == 0.0
    assert O.scale(w32, np.float32([1.0]), 1.0, 1.0)[0] == 2.0
    # generic values: the product's error stays within the format's step
    v = np.random.default_rng(9).standard_normal(256).astype(np.float32)
    rel = np.abs(O.scale(w32, v, 0.7) / (v * np.float32(0.7)) - 1)
    assert rel.max() < (1e-6 if w32 else 2 ** (1 / 128) - 1 + 1e-6) * 2


# ------------------------------------------------------------- Monte LFSR --

def test_lfsr_contract(L):
    # test-lns-cuda-parity.cpp:559-570
    assert not O.monte_set(0)
    O.monte_set(7)
    assert L.lno_lfsr_step(7) == FIG["lfsr"]["step_of_7"]
    s, seen = 7, 0
    while True:
        s = L.lno_lfsr_step(s)
        seen += 1
        if s == 7:
            break
    assert seen == FIG["lfsr"]["period"]
    for n in (0, 1, 2, 100, 65534, 65535, 123457):
        s = 7
        for _ in range(n % 65535):
            s = L.lno_lfsr_step(s)
        assert L.lno_lfsr_jump(7, n) == s
    start = np.zeros(1, np.uint16)
    L.lno_monte_reserve(5, start.ctypes.data)
    assert start[0] == 7 and O.monte_get() == L.lno_lfsr_jump(7, 5)
    O.monte_set(7)


# ------------------------------------------------------------ MUL_MAT_ID --

@pytest.mark.parametrize("mode", ["base", "monte", "lpvip", "sum32", "lns32"])
def test_mul_mat_id_is_mul_mat_per_slot_in_order(mode):
    # each (token, slot) output is the pinned mul_mat of the slot's expert and
    # activation row s % ne11, run in the order t, s (so Monte draws continue
    # from one slot to the next exactly as in the reference's loop)
    rng = np.random.default_rng(21)
    E, M, K, T, neu, ne11 = 5, 24, 40, 3, 4, 2
    w = (rng.standard_normal((E, M, K)) * 0.1).astype(np.float32)
    x = rng.standard_normal((T, ne11, K)).astype(np.float32)
    ids = rng.integers(0, E, (T, neu)).astype(np.int32)
    m = None if mode == "lns32" else O.MODES[mode]
    O.monte_set(7)
    got = O.mul_mat_id(m, w, x, ids)
    after = O.monte_get()
    O.monte_set(7)
    for t in range(T):
        for s in range(neu):
            xr = x[t, s % ne11][None]
            e = ids[t, s]
            want = O.mul_mat32(w[e], xr) if m is None else O.mul_mat16(m, O.f2x16(w[e]), xr)
            assert np.array_equal(got[t, s].view(np.uint32), want[0].view(np.uint32)), (t, s)
    assert O.monte_get() == after
    if m == O.MONTE:
        assert after == O.lib().lno_lfsr_jump(7, T * neu * M * (K - 1))
