"""CPU checks of the product library: it loads without a GPU, exports every
function include/*.h declares, and its arithmetic tables equal the oracle's
independent restatement (no compute call needs a GPU here)."""
import ctypes
import os
import re

import numpy as np
import pytest

import oracle_lib as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def lnship():
    import lnship as m
    if not os.path.exists(m.LIB_PATH):
        pytest.fail("liblnship.so is not built (run __graft_entry__.build())")
    return m


def _declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b((?:lnship|ggml_backend)\w*)\s*\(", text)))


# which in-tree library implements each public header
LIBRARY_OF = {"lnship.h": "liblnship.so", "ggml-lnship.h": "libggml-lnship.so"}


def test_every_header_has_a_library():
    headers = sorted(h for h in os.listdir(os.path.join(ROOT, "include")) if h.endswith(".h"))
    assert headers == sorted(LIBRARY_OF)


@pytest.mark.parametrize("header", sorted(LIBRARY_OF))
def test_library_exports_every_declared_symbol(lnship, header):
    path = os.path.join(os.path.dirname(lnship.LIB_PATH), LIBRARY_OF[header])
    if header == "ggml-lnship.h":
        # its ggml imports come from the test host stub
        import ggml_host
        ggml_host.build_stub()
        ctypes.CDLL(ggml_host.STUB_SO, mode=ctypes.RTLD_GLOBAL)
    L = ctypes.CDLL(path)
    names = _declared(header)
    assert names
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_cvt16_table_equals_oracle(lnship):
    assert np.array_equal(lnship.host_table("cvt16", np.uint16), O.table("lno16_cvt_table", 1 << 17, np.uint16))


def test_rev16_table_equals_oracle(lnship):
    got = lnship.host_table("rev16", np.float32)
    want = O.x2f16(np.arange(65536, dtype=np.uint16))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_gauss16_tables_equal_oracle(lnship):
    g = lnship.host_table("gauss16", np.int16)
    n = g.size // 2
    sb, db = O.table("lno16_sb_table", 1281, np.int16), O.table("lno16_db_table", 1281, np.int16)
    assert np.array_equal(g[:1281], sb) and np.array_equal(g[n:n + 1281], db)
    assert np.all(g[1281:n] == 0) and np.all(g[n + 1281:] == 0)


def test_monte_table_encodes_the_oracle_adder(lnship):
    # (sb e, sb m, db e, db m) per distance: the base table x 64 and no draw
    # below the dither range, then the oracle's threshold F(d) (0 at the end)
    g = lnship.host_table("gauss16m", np.int32).reshape(-1, 4)
    n = g.shape[0]
    sb, db = O.table("lno16_sb_table", 1281, np.int16), O.table("lno16_db_table", 1281, np.int16)
    F = np.zeros(n, np.int32)
    O.lib().lno16_monte_threshold_n(0, n, F.ctypes.data)
    start = int(np.argmax(F > 0))
    assert start == 1091 and F[n - 1] == 0 and F[n - 2] > 0
    assert np.array_equal(g[:start, 0], sb[:start].astype(np.int32) * 64) and np.all(g[:start, 1] == 0)
    assert np.array_equal(g[:start, 2], db[:start].astype(np.int32) * 64) and np.all(g[:start, 3] == 0)
    assert np.array_equal(g[start:, 0], F[start:]) and np.all(g[start:, 1] == 63)
    assert np.array_equal(g[start:, 2], 64 - F[start:]) and np.all(g[start:, 3] == -1)
    # the draw of every entry against the oracle's rule, for every draw r
    r = np.arange(64, dtype=np.int32)[:, None]
    for e, m, sign in ((g[:, 0], g[:, 1], 1), (g[:, 2], g[:, 3], -1)):
        adj = (e[None, :] + ((r ^ (m[None, :] >> 31)) & m[None, :])) >> 6
        want = np.where(np.arange(n) < start, e[None, :] >> 6, sign * ((F[None, :] + r) >> 6))
        assert np.array_equal(adj, want)


def test_exp16_table_equals_oracle(lnship):
    assert np.array_equal(lnship.host_table("exp16", np.uint16), O.table("lno16_exp_table", 1 << 16, np.uint16))


def test_tab32_equals_oracle(lnship):
    t = lnship.host_table("tab32", np.int32)
    sb, sbf, db, dbf, dlo, dhi = (O.table32(k) for k in ("sb", "sbf", "db", "dbf", "dlo", "dhi"))
    parts = [dlo, dhi, sb, sbf, db[2048:], dbf]
    assert t.size == sum(p.size for p in parts)
    assert np.array_equal(t, np.concatenate(parts))


def test_lfsr_sequence_equals_oracle(lnship):
    seq = lnship.host_table("lfsr_seq", np.uint16)
    L = O.lib()
    s = 1
    for i in range(0, 65535, 997):
        assert seq[i] == L.lno_lfsr_jump(1, i)
    for st in (7, 1, 0xB403, 12345):
        for n in (0, 1, 65534, 65535, 10 ** 9 + 7):
            assert lnship.lfsr_jump(st, n) == L.lno_lfsr_jump(st, n)


def test_draw_accounting_matches_reference_formula(lnship):
    # test-lns-cuda-parity.cpp:77-105: K-1 per dot, n-1 per softmax row, n per rms row
    L = lnship.lib()
    assert L.lnship16_mul_mat_draws(lnship.MONTE, 576, 1536, 5, 2, 3) == 1536 * 5 * 6 * 575
    assert L.lnship16_mul_mat_draws(lnship.MONTE, 0, 1536, 5, 1, 1) == 0
    assert L.lnship16_mul_mat_draws(lnship.SUM32, 576, 1536, 5, 1, 1) == 0
    assert L.lnship16_soft_max_draws(lnship.MONTE, 128, 9) == 9 * 127
    assert L.lnship16_rms_norm_draws(lnship.MONTE, 576, 3) == 3 * 576


def test_calls_without_init_fail_loudly(lnship):
    # no device here: every compute entry point must refuse, never fall back
    L = lnship.lib()
    rc = L.lnship16_from_f32(None, None, 16, None)
    assert rc != 0


def test_rope_table_uses_the_float_recurrence(lnship):
    # lns_rope (src/lns-ops.cpp:1225-1247): t *= powf(base, -2/n_dims), cosf / sinf
    libm = ctypes.CDLL("libm.so.6")
    for fn in ("cosf", "sinf", "powf"):
        getattr(libm, fn).restype = ctypes.c_float
    libm.cosf.argtypes = libm.sinf.argtypes = [ctypes.c_float]
    libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]
    n_dims, n_pos = 64, 40
    got = np.empty(n_pos * n_dims, np.float32)
    assert lnship.lib().lnship_rope_table(10000.0, n_dims, n_pos, ctypes.c_void_p(got.ctypes.data)) == 0
    ts = np.float32(libm.powf(10000.0, np.float32(-2.0) / np.float32(n_dims)))
    for p in range(n_pos):
        t = np.float32(p)
        for j in range(n_dims // 2):
            assert got[(p * 32 + j) * 2] == np.float32(libm.cosf(t))
            assert got[(p * 32 + j) * 2 + 1] == np.float32(libm.sinf(t))
            t = np.float32(t * ts)
