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


def test_fused_row_limits(lnship):
    # the fused one-row kernels hold their rows in LDS beside the tables, so
    # callers ask for their limits before fusing (lnship_max_row 5 and 6)
    L = lnship.lib()
    rms_mm = L.lnship_max_row(5, lnship.SUM32)
    # the three-node launch takes SmolLM2's and Llama-1B's rows, but fewer
    # than the rms_norm node alone: a ggml graph may hold rows in between
    assert 2048 <= rms_mm < L.lnship_max_row(0, lnship.SUM32)
    assert rms_mm % 8 == 0
    for m in (lnship.BASE, lnship.MONTE, lnship.LPVIP):
        assert L.lnship_max_row(5, m) == 0
    assert L.lnship_max_row(6, lnship.MONTE) == 0
    for m in (lnship.BASE, lnship.LPVIP, lnship.SUM32):
        glu = L.lnship_max_row(6, m)
        assert glu >= 8192 and glu % 8 == 0   # Llama-1B's FFN


def test_attn_decode_refuses_wide_heads_before_any_device_call(lnship):
    # lnship_max_row(4) holds for head_dim <= 256; a wider head at that n_kv
    # does not fit LDS and must be refused as a size error, not fail at launch
    L = lnship.lib()
    n_kv = L.lnship_max_row(4, lnship.SUM32)
    fake = ctypes.c_void_p(0x1000)   # never dereferenced: the size check comes first
    a = lnship.AttnArgs()
    a.q = a.k_cache = a.v_cache = a.dst = fake.value
    a.cache_m, a.n_head, a.n_head_kv, a.n_kv, a.scale = n_kv, 8, 8, n_kv, 0.125
    ERANGE, ENOINIT = -4, -3   # include/lnship.h: enum lnship_error
    for hd, want in ((1024, ERANGE), (4096, ERANGE)):
        a.head_dim = hd
        assert L.lnship16_attn_decode(lnship.SUM32, ctypes.byref(a), None) == want
        assert b"LDS" in L.lnship_last_error()
    # a head_dim within the limit passes the checks and then needs a device
    a.head_dim = 64
    assert L.lnship16_attn_decode(lnship.SUM32, ctypes.byref(a), None) == ENOINIT
    # the LNS32 one: its own cell limit (xlns32 codes), the same refusals
    n32 = L.lnship_max_row(7, 0)
    assert 2048 <= n32 < n_kv
    a.n_kv = a.cache_m = n32
    assert L.lnship32_attn_decode(ctypes.byref(a), None) == ENOINIT
    a.head_dim = 256   # the limit's head_dim
    assert L.lnship32_attn_decode(ctypes.byref(a), None) == ENOINIT
    a.n_kv = a.cache_m = n32 + 8
    assert L.lnship32_attn_decode(ctypes.byref(a), None) == ERANGE
    a.n_kv = a.cache_m = n32
    a.head_dim = 1024
    assert L.lnship32_attn_decode(ctypes.byref(a), None) == ERANGE


def test_q4_k_host_to_float():
    # the test ggml host's Q4_K to_float (ggml's published block layout)
    # equals the graph check's numpy restatement, and a hand-made block
    # decodes to the values its fields name
    import ggml_host as G
    import ggml_graph_check as C
    G.build_stub()
    stub = ctypes.CDLL(G.STUB_SO)
    stub.ggml_get_type_traits.restype = ctypes.c_void_p
    stub.ggml_get_type_traits.argtypes = [ctypes.c_int]

    class Traits(ctypes.Structure):
        _fields_ = [("type_name", ctypes.c_char_p), ("blck_size", ctypes.c_int64),
                    ("blck_size_interleave", ctypes.c_int64), ("type_size", ctypes.c_size_t),
                    ("is_quantized", ctypes.c_bool),
                    ("to_float", ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64))]

    tr = Traits.from_address(stub.ggml_get_type_traits(12))
    assert (tr.type_name, tr.blck_size, tr.type_size, tr.is_quantized) == (b"q4_K", 256, 144, True)
    rng = np.random.default_rng(5)
    raw, want = C.q4_k(3, 512, rng)
    got = np.empty(3 * 512, np.float32)
    tr.to_float(raw.ctypes.data, got.ctypes.data, got.size)
    assert np.array_equal(got.view(np.uint32), want.reshape(-1).view(np.uint32))
    # d = 1, dmin = 0.5; pair j: scale j + 1, min 2j (6-bit packing of
    # pairs 4-7 spread over three bytes); quants 0..15 repeating
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.array([1.0], np.float16).view(np.uint8)
    blk[2:4] = np.array([0.5], np.float16).view(np.uint8)
    sc, mn = list(range(1, 9)), [2 * j for j in range(8)]
    for j in range(4):
        blk[4 + j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        blk[8 + j] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        blk[12 + j] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    blk[16:] = np.arange(128, dtype=np.uint8) % 16 * 17   # both nibbles l % 16
    out = np.empty(256, np.float32)
    tr.to_float(blk.ctypes.data, out.ctypes.data, 256)
    for j in range(8):
        q = np.arange(32) % 16
        assert np.array_equal(out[32 * j:32 * j + 32], (sc[j] * q - 0.5 * mn[j]).astype(np.float32))


def test_positive_sum_pair_image(lnship):
    # the row kernels' positive-sum adder: per sb interval the node and the
    # slope scaled by 2^10 (near grid, fraction scaled by 2^9) or 2^9 (far
    # grid, fraction by 2^4), both 24-bit signed operands of
    # v_mul_hi_i32_i24; the high word of their product is then exactly
    # floor((t1 - t0) * f / 2^sh), the oracle's interpolation term
    img = lnship.host_table("pos32", np.int32).reshape(-1, 2)
    L = O.lib()
    sb = O.table32("sb")
    sbf = O.table32("sbf")
    nn = sb.size - 1
    assert np.array_equal(img[:nn, 0], sb[:-1])
    assert np.array_equal(img[:nn, 1].astype(np.int64), (sb[1:].astype(np.int64) - sb[:-1]) << 10)
    # the far grid, extended with zeros out to every distance below 2^31
    nf = ((1 << 31) - 12 * (1 << 23)) >> 19
    far = np.zeros(nf + 1, np.int64)
    far[:sbf.size] = sbf
    assert img.shape[0] >= nn + nf
    assert np.array_equal(img[nn:nn + nf, 0], far[:-1])
    assert np.array_equal(img[nn:nn + nf, 1].astype(np.int64), (far[1:] - far[:-1]) << 9)
    assert sbf[-1] == 0 and np.all(np.abs(img[:, 1].astype(np.int64)) <= 1 << 23)
    # the product identity on every fraction of the steepest intervals
    for t, sc, fs, sh in ((img[:nn], 10, 9, 13), (img[nn:nn + nf], 9, 4, 19)):
        i = int(np.argmin(t[:, 1]))
        f = np.arange(1 << sh, dtype=np.int64)
        slope = int(t[i, 1]) >> sc
        assert np.array_equal((int(t[i, 1]) * (f << fs)) >> 32, (slope * f) >> sh)


def test_rope_attn_decode_checks_its_store_arguments_first(lnship):
    # lnship16_rope_attn_decode takes the token's rope and cache stores with
    # the attention: every store argument must describe the same heads and
    # caches, one token of one sequence; a mismatch is refused before any
    # device call, a matching pair then needs a device
    L = lnship.lib()
    fake = ctypes.c_void_p(0x1000).value   # never dereferenced: the checks come first
    EINVAL, ENOINIT = -1, -3   # include/lnship.h: enum lnship_error
    nh, nkv, hd, n_ctx = 9, 3, 64, 256

    def pair():
        a = lnship.AttnArgs()
        a.k_cache, a.v_cache, a.dst, a.mask = fake, fake + 64, fake + 128, fake + 192
        a.cache_m, a.k_slice, a.v_slice, a.scale = n_ctx, hd * n_ctx, hd * n_ctx, 0.125
        a.n_head, a.n_head_kv, a.head_dim, a.n_kv = nh, nkv, hd, 200
        q = lnship.QkvStoreArgs(fake, (nh + 2 * nkv) * hd, fake + 256, 1, nh, nkv, hd, hd, fake + 320, None,
                                fake, fake + 64, n_ctx, hd * n_ctx, hd * n_ctx, None, 0)
        return q, a

    q, a = pair()
    assert L.lnship16_rope_attn_decode(lnship.SUM32, ctypes.byref(q), ctypes.byref(a), None) == ENOINIT
    # args.q may be null: the fused rope forms the queries
    assert not a.q
    for field, value in (("ntok", 2), ("n_head", nh - 1), ("n_head_kv", 1), ("head_dim", 60),
                         ("rope_n_dims", 63), ("rope_n_dims", 72), ("qkv_ld", (nh + 2 * nkv) * hd - 1),
                         ("k_cache", fake + 8), ("v_cache", fake + 8), ("cache_m", n_ctx + 8), ("k_slice", 8),
                         ("v_slice", 8), ("seq", fake), ("qkv", None), ("pos", None), ("cos_sin", None)):
        q, a = pair()
        setattr(q, field, value)
        assert L.lnship16_rope_attn_decode(lnship.SUM32, ctypes.byref(q), ctypes.byref(a), None) == EINVAL, field
    q, a = pair()
    assert L.lnship16_rope_attn_decode(lnship.MONTE, ctypes.byref(q), ctypes.byref(a), None) == EINVAL
    assert L.lnship16_rope_attn_decode(lnship.SUM32, None, ctypes.byref(a), None) == EINVAL


def test_rope_attn_decode_seqs_checks_its_store_arguments_first(lnship):
    # lnship16_rope_attn_decode_seqs: one token per sequence in the store
    # arguments, no seq map, sequence s's cells where the attention reads
    # them (seq_stride = n_head_kv * k_slice); every mode, Monte included;
    # mismatches are refused before any device call
    L = lnship.lib()
    fake = ctypes.c_void_p(0x1000).value   # never dereferenced: the checks come first
    EINVAL, ENOINIT = -1, -3   # include/lnship.h: enum lnship_error
    nh, nkv, hd, n_ctx, nseq = 9, 3, 64, 256, 4

    def triple():
        a = lnship.AttnArgs()
        a.k_cache, a.v_cache, a.dst, a.mask = fake, fake + 64, fake + 128, fake + 192
        a.cache_m, a.k_slice, a.v_slice, a.scale = n_ctx, hd * n_ctx, hd * n_ctx, 0.125
        a.n_head, a.n_head_kv, a.head_dim, a.n_kv = nh, nkv, hd, 200
        q = lnship.QkvStoreArgs(fake, (nh + 2 * nkv) * hd, fake + 256, nseq, nh, nkv, hd, hd, fake + 320, None,
                                fake, fake + 64, n_ctx, hd * n_ctx, hd * n_ctx, None, nkv * hd * n_ctx)
        return q, a, lnship.attn_seqs(nseq, (1, 2, 3))

    for mode in (lnship.BASE, lnship.MONTE, lnship.LPVIP, lnship.SUM32):
        q, a, sq = triple()
        assert L.lnship16_rope_attn_decode_seqs(mode, ctypes.byref(q), ctypes.byref(a), ctypes.byref(sq),
                                                None) == ENOINIT, mode
    for field, value in (("ntok", nseq - 1), ("ntok", 1), ("seq", fake), ("seq_stride", nkv * hd * n_ctx + 8),
                         ("n_head", nh - 1), ("head_dim", 60), ("rope_n_dims", 63),
                         ("qkv_ld", (nh + 2 * nkv) * hd - 1), ("k_cache", fake + 8), ("cache_m", n_ctx + 8),
                         ("v_slice", 8), ("qkv", None), ("pos", None), ("cos_sin", None)):
        q, a, sq = triple()
        setattr(q, field, value)
        assert L.lnship16_rope_attn_decode_seqs(lnship.MONTE, ctypes.byref(q), ctypes.byref(a), ctypes.byref(sq),
                                                None) == EINVAL, field
    q, a, sq = triple()
    assert L.lnship16_rope_attn_decode_seqs(lnship.SUM32, ctypes.byref(q), ctypes.byref(a), None, None) == EINVAL
    assert L.lnship16_rope_attn_decode_seqs(lnship.SUM32, None, ctypes.byref(a), ctypes.byref(sq), None) == EINVAL
    # one sequence: seq_stride is not read
    q, a, sq = triple()
    q.ntok, q.seq_stride, sq.n_seq = 1, 0, 1
    assert L.lnship16_rope_attn_decode_seqs(lnship.MONTE, ctypes.byref(q), ctypes.byref(a), ctypes.byref(sq),
                                            None) == ENOINIT


def test_attn_decode_seqs_checks_arguments_first(lnship):
    # lnship16_attn_decode_seqs runs every mode, Monte with the three nodes'
    # starts; its arguments and the sequence count are checked before any
    # device call (a valid call then needs the device)
    L = lnship.lib()
    fake = ctypes.c_void_p(0x1000).value   # never dereferenced: the checks come first
    EINVAL, ENOINIT, ERANGE = -1, -3, -4   # include/lnship.h: enum lnship_error
    a = lnship.AttnArgs()
    a.q, a.k_cache, a.v_cache, a.dst, a.mask = fake, fake + 64, fake + 128, fake + 192, fake + 256
    a.cache_m, a.k_slice, a.v_slice, a.scale = 512, 64 * 512, 64 * 512, 0.125
    a.n_head, a.n_head_kv, a.head_dim, a.n_kv = 9, 3, 64, 320
    for mode in (lnship.BASE, lnship.MONTE, lnship.LPVIP, lnship.SUM32):
        sq = lnship.attn_seqs(8, (1, 2, 3))
        assert L.lnship16_attn_decode_seqs(mode, ctypes.byref(a), ctypes.byref(sq), None) == ENOINIT, mode
        # the limit of the cells is that of lnship16_attn_decode, Monte included
        lim = L.lnship_max_row(8, mode)
        assert lim >= 4096 and (mode == lnship.MONTE or lim == L.lnship_max_row(4, mode))
    for n_seq in (0, -1, 0x7fffff):
        sq = lnship.attn_seqs(n_seq)
        assert L.lnship16_attn_decode_seqs(lnship.MONTE, ctypes.byref(a), ctypes.byref(sq), None) == EINVAL, n_seq
    assert L.lnship16_attn_decode_seqs(lnship.SUM32, ctypes.byref(a), None, None) == EINVAL
    # lnship16_attn_decode itself still refuses Monte (it has no starts)
    assert L.lnship16_attn_decode(lnship.MONTE, ctypes.byref(a), None) == EINVAL
    assert L.lnship_max_row(4, lnship.MONTE) == 0
    a.n_kv = L.lnship_max_row(8, lnship.MONTE) + 8
    a.cache_m = a.n_kv
    sq = lnship.attn_seqs(2)
    assert L.lnship16_attn_decode_seqs(lnship.MONTE, ctypes.byref(a), ctypes.byref(sq), None) == ERANGE


def test_ctypes_structs_match_the_header(lnship, tmp_path):
    # every argument struct the Python mirror passes by pointer has the
    # header's size and field offsets (a C program built from include/lnship.h
    # prints them; gcc on the host, nothing launched)
    import subprocess
    structs = {"lnship_mul_mat_args": lnship.MulMatArgs, "lnship_soft_max_args": lnship.SoftMaxArgs,
               "lnship_mul_mat_id_args": lnship.MulMatIdArgs, "lnship_qkv_store_args": lnship.QkvStoreArgs,
               "lnship_attn_args": lnship.AttnArgs, "lnship_attn_seqs": lnship.AttnSeqs}
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "lnship.h"', "int main(void) {"]
    for cname, py in structs.items():
        lines.append('printf("%s size %%zu\\n", sizeof(%s));' % (cname, cname))
        for f in py._fields_:
            lines.append('printf("%s %s %%zu\\n", offsetof(%s, %s));' % (cname, f[0], cname, f[0]))
    lines += ["return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    inc = os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "include")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-I", inc, str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    got = {tuple(l.split()[:2]): int(l.split()[2]) for l in out if l}
    for cname, py in structs.items():
        assert got[(cname, "size")] == ctypes.sizeof(py), cname
        for f in py._fields_:
            assert got[(cname, f[0])] == getattr(py, f[0]).offset, (cname, f[0])


def test_lpvip_db_range_checks_its_range_first(lnship):
    # d = 0 (exact cancellation, never a db) and ranges past 2^32 are refused
    # before any device call; a valid range then needs the device
    L = lnship.lib()
    fake = ctypes.c_void_p(0x1000)
    EINVAL, ENOINIT = -1, -3   # include/lnship.h: enum lnship_error
    assert L.lnship_lpvip_db_range(0, 8, fake, None) == EINVAL
    assert L.lnship_lpvip_db_range(0xffffffff, 2, fake, None) == EINVAL
    assert L.lnship_lpvip_db_range(1, 8, None, None) == EINVAL
    assert L.lnship_lpvip_db_range(1, 8, fake, None) == ENOINIT
