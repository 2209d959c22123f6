"""Every figure the reference printed for this path, asserted exactly.

The CPU oracle (oracle/lns_oracle.c) is checked against three committed
evidence sets of the reference:

  * results/sum32-evidence/unit-tests-*.txt: test-lns-backend.cpp's suite,
    one file per sum mode and one for LNS32 (2026-08-20, the pinned
    xlnscpp);
  * results/sum32-evidence/standalone-sum32-invariants.txt:
    test-lns16-sum32.cpp;
  * experiments/dot-product-scaling/results/{synth,convert,monte}.jsonl:
    dot-bench.cpp, whose operands tests/synth/synth_stats.cpp regenerates
    with the same libstdc++ generators, so its six-digit statistics over
    4096 outputs per K (monte.jsonl: 2048 outputs, 32 reps from per-rep
    LFSR seeds, and the rep averages) are exact pins.  That experiment ran
    on the post-merge libraries (experiments/README.md:28-37).

Where the oracle's restatement disagrees with a printed figure, the test is a
strict xfail that names the figure: the disagreement is reported, never
absorbed by a tolerance.  lpvip is contradicted by both evidence sets; the
restated Monte adder reproduces 13 of its 15 unit-test figures and no
experiment row; xlns32_alt (sum32 / LNS32) misses two unit-test figures and
the experiment's signed rows.  The two evidence sets also contradict each other
for xlns32: test_xlns32_evidence_sets_disagree shows it.
"""
import json
import math
import os
import subprocess

import numpy as np
import pytest

import oracle_lib as O
import test_oracle_pins as P

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
FIG = json.load(open(os.path.join(HERE, "golden", "reference_figures.json")))
SYNTH = json.load(open(os.path.join(HERE, "golden", "synth_rows.json")))["rows"]
UT = FIG["unit_tests"]

MONTE_REASON = ("parity contradicted: the restated xlns16_add_monte (xlnscpp xlns16monte.cpp is absent; "
                "the restatement is fitted to the printed figures) misses this figure")
LPVIP_REASON = ("parity contradicted: the restated xlns32_add_lpvip (xlnscpp xlns32lpvip.cpp is absent) "
                "does not reproduce the reference's printed lpvip figures")
X32_REASON = ("parity contradicted: the restated xlns32_alt adder misses this figure "
              "(its sb/db table layout is not in the reference)")


# ------------------------------------------------- test-lns-backend suite --

def _ramp(n, start, step):
    """fill_ramp (test-lns-backend.cpp:295-299), in float"""
    return (np.float32(start) + np.float32(step) * np.arange(n, dtype=np.float32)).astype(np.float32)


# (name, K, M (the test's N), n_expert, ne11, ids) of test-lns-backend.cpp:408-468
MM_ID_CASES = [
    ("non_broadcast", 8, 4, 6, 3, [[0, 2, 5], [1, 3, 4], [5, 0, 1], [2, 2, 3]]),
    ("broadcast_1", 8, 5, 8, 1, [[0, 1, 2, 7], [3, 4, 5, 6], [1, 1, 0, 7]]),
    ("partial_2", 6, 3, 5, 2, [[0, 4, 2, 1], [3, 0, 4, 2]]),
    ("dst_lns16", 8, 5, 8, 1, [[0, 1, 2, 7], [3, 4, 5, 6], [1, 1, 0, 7]]),
]


def _mm_id_case(K, M, E, ne11, ids):
    """test-lns-backend.cpp:326-343 inputs and the float reference (:301-324)"""
    ids = np.array(ids, np.int32)
    T, neu = ids.shape
    w = _ramp(K * M * E, -1.5, 0.07)
    x = _ramp(K * ne11 * T, 0.3, -0.05)
    for e in range(E):
        w[e * M * K] = np.float32(w[e * M * K] + np.float32(0.25) * np.float32(e))
    for t in range(T):
        for i in range(ne11):
            x[(t * ne11 + i) * K] = np.float32(x[(t * ne11 + i) * K] + np.float32(0.1) * np.float32(t + i))
    w, x = w.reshape(E, M, K), x.reshape(T, ne11, K)
    want = np.zeros((T, neu, M), np.float32)
    for t in range(T):
        for s in range(neu):
            a = x[t, s % ne11]
            for m in range(M):
                acc = np.float32(0)
                for k in range(K):
                    acc = np.float32(acc + np.float32(w[ids[t, s], m, k] * a[k]))
                want[t, s, m] = acc
    return w, x, ids, want


def _scaled_max(out, want):
    return np.max(np.abs(out - want) / np.maximum(np.abs(want), np.float32(1.0)))


def _suite(mode):
    """The figures of one unit-tests-*.txt, computed in the suite's order
    (test-lns-backend.cpp:1326-1343) so that Monte draws continue from LFSR
    state 7 through every reduction exactly as in the reference run."""
    lns32 = mode == "lns32"
    m = None if lns32 else O.MODES[mode]
    O.monte_set(7)
    got = {}
    out = O.mul_mat32(P.A_K2, P.B_K2) if lns32 else O.mul_mat16_f32w(m, P.A_K2, P.B_K2)
    got["mul_mat_k2"] = ["%.2f" % v for v in out.ravel()]
    a, b = P._long_operands()
    out = O.mul_mat32(a, b) if lns32 else O.mul_mat16_f32w(m, a, b)
    got["mul_mat_long"] = P._mm_long_figures(out, a, b)
    mid = {}
    for name, K, M, E, ne11, ids in MM_ID_CASES:
        if lns32 and name == "dst_lns16":
            continue
        w, x, idv, want = _mm_id_case(K, M, E, ne11, ids)
        mid[name] = "%.4f" % (_scaled_max(O.mul_mat_id(m, w, x, idv), want) * 100)
    got["mul_mat_id"] = mid
    sm = {}
    for case, args in P.SOFTMAX_CASES.items():
        x, mask, want = P._softmax_case(*args)
        out = O.soft_max32(x, mask, args[2]) if lns32 else O.soft_max16(m, x, mask, args[2])
        sm[case] = "%.6f" % np.abs(out - want).max()
    got["softmax"] = sm
    rms = {}
    for key, shape in (("short", (16, 3)), ("576", (576, 3))):
        x, want = P._rms_case(*shape)
        out = O.rms_norm32(x, 1e-5) if lns32 else O.rms_norm16(m, x, 1e-5)
        rms[key] = "%.4f" % (_scaled_max(out, want) * 100)
    got["rms_norm"] = rms
    O.monte_set(7)
    return got


_SUITES = {}


def suite(mode):
    if mode not in _SUITES:
        _SUITES[mode] = _suite(mode)
    return _SUITES[mode]


def _figures(mode):
    u = UT[mode]
    out = [("mul_mat_k2", None), ("mul_mat_long", None)]
    out += [("mul_mat_id", k) for k in u["mul_mat_id"]]
    out += [("softmax", k) for k in u["softmax"]]
    out += [("rms_norm", k) for k in u["rms_norm"]]
    return out


# figures the restated adders miss, by mode
CONTRADICTED = {
    "monte": {("mul_mat_long", None): MONTE_REASON + " (K=1536 NRMSE 4.9245% vs 4.7150%)",
              ("softmax", "masked_scaled"): MONTE_REASON + " (0.000287 vs 0.000494)"},
    "lns32": {("mul_mat_long", None): X32_REASON + " (K=1536 NRMSE 0.0124% vs 0.0122%, max 0.0367% vs 0.0327%)",
              ("mul_mat_id", "broadcast_1"): X32_REASON + " (0.0000% vs 0.0001%)"},
}


def _cases():
    for mode in ("base", "sum32", "lns32", "monte", "lpvip"):
        for fig, key in _figures(mode):
            marks = ()
            if mode == "lpvip":
                marks = (pytest.mark.xfail(strict=True, reason=LPVIP_REASON),)
            elif (fig, key) in CONTRADICTED.get(mode, {}):
                marks = (pytest.mark.xfail(strict=True, reason=CONTRADICTED[mode][(fig, key)]),)
            yield pytest.param(mode, fig, key, marks=marks, id="%s-%s%s" % (mode, fig, "" if key is None else "-" + key))


@pytest.mark.parametrize("mode,fig,key", list(_cases()))
def test_unit_suite_figure(mode, fig, key):
    got, want = suite(mode)[fig], UT[mode][fig]
    if key is not None:
        got, want = got[key], want[key]
    assert got == want


def test_monte_k2_and_mul_mat_id_equal_base_in_reference():
    # what the reference's Monte figures say on their own: every K <= 8 sum
    # (the K=2 mul_mat and all four mul_mat_id cases) printed the base value
    for fig in ("mul_mat_k2", "mul_mat_id"):
        assert UT["monte"][fig] == UT["base"][fig]


# ------------------------------------------------- standalone sum32 check --

@pytest.fixture(scope="module")
def standalone():
    return P.standalone.__wrapped__(O.lib())


@pytest.mark.parametrize("part", ["two_term", "stagnation", "rms_norm"])
def test_standalone_exact(standalone, part):
    assert standalone[part] == FIG["standalone"][part]


def test_standalone_long_dot_k1536(standalone):
    assert standalone["long_dot"]["1536"] == FIG["standalone"]["long_dot"]["1536"]


@pytest.mark.xfail(strict=True, reason=X32_REASON + " (K=8960: mean 0.211% vs 0.198%, better in 63 vs 64)")
def test_standalone_long_dot_k8960(standalone):
    assert standalone["long_dot"]["8960"] == FIG["standalone"]["long_dot"]["8960"]


def test_standalone_long_dot_base(standalone):
    for K in ("1536", "8960"):
        assert standalone["long_dot"][K]["base"] == FIG["standalone"]["long_dot"][K]["base"]


# ------------------------------------------ dot-product-scaling experiment --

SYNTH_EXE = os.path.join(HERE, "synth", "synth_stats")


@pytest.fixture(scope="module")
def synth_exe():
    src = os.path.join(HERE, "synth", "synth_stats.cpp")
    osrc = os.path.join(ROOT, "oracle", "lns_oracle.c")
    if not os.path.exists(SYNTH_EXE) or os.path.getmtime(SYNTH_EXE) < max(os.path.getmtime(src),
                                                                           os.path.getmtime(osrc)):
        obj = SYNTH_EXE + ".oracle.o"
        subprocess.check_call(["gcc", "-O2", "-c", osrc, "-o", obj])
        subprocess.check_call(["g++", "-O2", "-std=c++17", "-I", os.path.join(ROOT, "oracle"), src, obj,
                               "-o", SYNTH_EXE, "-lm"])
    return SYNTH_EXE


def _run_synth(exe, cfg, dist, kmin, kmax, variant=0):
    out = subprocess.run([exe, "synth", cfg, dist, str(kmin), str(kmax), str(variant)],
                         capture_output=True, text=True, check=True).stdout
    return {json.loads(l)["K"]: json.loads(l)["acc"] for l in out.splitlines()}


def _ref_rows(cfg, dist, kmax):
    return {r["K"]: r["acc"] for r in SYNTH if r["config"] == cfg and r["dist"] == dist and r["K"] <= kmax}


def _fmt(acc):
    return {k: "%.6g" % v for k, v in acc.items()}


def _synth_case(exe, cfg, dist, kmax, variant=0):
    want = _ref_rows(cfg, dist, kmax)
    got = _run_synth(exe, cfg, dist, min(want), max(want), variant)
    return {K: _fmt(got[K]) for K in want}, {K: _fmt(v) for K, v in want.items()}


@pytest.mark.parametrize("dist", ["signed", "positive", "attn"])
def test_synth_base_rows(synth_exe, dist):
    # base mode and the xlns16 conversions: every row K = 16..16384 to all
    # six printed digits of all five statistics
    got, want = _synth_case(synth_exe, "base", dist, 16384)
    assert got == want


def _mode_case(cfg, dist, reason, kmax=1024):
    return pytest.param(cfg, dist, kmax, marks=pytest.mark.xfail(strict=True, reason=reason), id="%s-%s" % (cfg, dist))


EXP_REASON = " (the experiment ran the post-merge libraries, experiments/README.md:28-37)"


@pytest.mark.parametrize("cfg,dist,kmax", [
    *[_mode_case("monte", d, MONTE_REASON + EXP_REASON) for d in ("signed", "positive", "attn")],
    *[_mode_case("lpvip", d, LPVIP_REASON + EXP_REASON) for d in ("signed", "positive", "attn")],
    *[_mode_case("sum32", d, X32_REASON + EXP_REASON) for d in ("signed", "positive", "attn")],
    *[_mode_case("xlns32", d, X32_REASON + EXP_REASON) for d in ("signed", "positive", "attn")],
])
def test_synth_mode_rows(synth_exe, cfg, dist, kmax):
    got, want = _synth_case(synth_exe, cfg, dist, kmax)
    assert got == want


MONTE_ROWS = json.load(open(os.path.join(HERE, "golden", "monte_rows.json")))["rows"]


def _monte_reps(exe, dist, kmax):
    """The oracle's statistics in the Monte experiment's form (rep 0's acc
    statistics and the averages over 1, 2, 4, ... 32 reps, each rep from
    its own LFSR seed), as synth_stats monte prints them"""
    out = subprocess.run([exe, "monte", dist, "16", str(kmax), "32", "2048"], capture_output=True, text=True,
                         check=True).stdout
    acc, avg = {}, {}
    for line in out.splitlines():
        d = json.loads(line)
        if "avg" in d:
            avg.setdefault(d["avg"]["K"], []).append({k: "%.6g" % d["avg"][k] for k in ("bias", "sd", "rms")})
        else:
            acc[d["K"]] = _fmt(d["acc"])
    return acc, avg


@pytest.mark.xfail(strict=True, reason=MONTE_REASON + EXP_REASON)
@pytest.mark.parametrize("dist", ["signed", "positive", "attn"])
def test_monte_rep_rows(synth_exe, dist):
    # results/monte.jsonl: 2048 outputs per K, 32 reps with per-rep LFSR
    # seeds; rep 0's five statistics and the rep-averaged bias, sd and rms,
    # every row K = 16..1024 to all six printed digits
    want = {r["K"]: r for r in MONTE_ROWS if r["dist"] == dist and r["K"] <= 1024}
    acc, avg = _monte_reps(synth_exe, dist, 1024)
    assert {K: acc[K] for K in want} == {K: _fmt(r["acc"]) for K, r in want.items()}
    assert {K: avg[K] for K in want} == {
        K: [{k: "%.6g" % a[k] for k in ("bias", "sd", "rms")} for a in r["avg"]] for K, r in want.items()}


def test_xlns32_evidence_sets_disagree(synth_exe, standalone):
    """The experiment's xlns32 sb is recovered exactly, and it is not the
    unit-test era's: with it (lno32_set_variant(1)) every positive-operand
    xlns32 row of synth.jsonl matches to all six digits (only sb runs
    there), yet the standalone test's sum of 8960 ones comes out code 1681
    where standalone-sum32-invariants.txt:10 printed code 1680.  No single
    sb satisfies both sets."""
    got, want = _synth_case(synth_exe, "xlns32", "positive", 16384, variant=1)
    assert got == want
    L = O.lib()
    old = L.lno32_set_variant(1)
    try:
        s = 0x40000000
        for _ in range(8959):
            s = L.lno32_add(s, 0x40000000)
    finally:
        L.lno32_set_variant(old)
    assert L.lno16_narrow_sum32(s) - 0x4000 == 1681
    assert FIG["standalone"]["stagnation"]["8960"]["sum32"] == "%.4f" % L.lno16_to_f32(0x4000 + 1680)
    assert standalone["stagnation"]["8960"]["sum32"] == "%.4f" % L.lno16_to_f32(0x4000 + 1680)


def _convert(exe, fmt):
    out = subprocess.run([exe, "convert", fmt], capture_output=True, text=True, check=True).stdout
    return json.loads(out)


@pytest.mark.parametrize("fmt", ["xlns16", "xlns32"])
def test_convert_rows_exact(synth_exe, fmt):
    # fp2xlns16 / xlns162fp (tables) and fp2xlns32 / xlns322fp (libm) over
    # the experiment's 4M log-uniform values, every statistic to six digits
    got = _convert(synth_exe, fmt)
    want = FIG["convert_" + fmt]
    for k, v in want.items():
        if k.startswith("_"):
            continue
        assert "%.6g" % got[k] == "%.6g" % v, k
