"""GPU parity of the decode GEMVs that take the graph node before them into
their launch, bit for bit against the CPU oracle of the separate nodes and
against the library's separate launches:
- lnship16_rms_norm_mul_mat: rms_norm, norm MUL and mul_mat (lns_rms_norm,
  lns_mul, lns_mul_mat: src/lns-ops.cpp:701-736, :468-530, :293-384).  The
  kernel starts the mul_mat's chains from a predicted rms scale and runs them
  again when the rms chain's scale differs; the skew hook makes every
  prediction wrong, so the second pass is checked too.
- lnship16_swiglu_mul_mat: swiglu and the mul_mat with its residual ADD
  (lns_swiglu, src/lns-ops.cpp:809-862, then lns_mul_mat and lns_add)."""
import ctypes

import numpy as np
import pytest
import torch

import oracle_lib as O

pytestmark = pytest.mark.gpu

EPS = 1e-5


@pytest.fixture(scope="module")
def ln():
    import lnship
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    lnship.init()
    return lnship


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def P(t):
    return ctypes.c_void_p(t.data_ptr())


def same_bits(got, want, what):
    g, w = np.ascontiguousarray(got), np.ascontiguousarray(want)
    assert g.shape == w.shape, (what, g.shape, w.shape)
    bad = np.nonzero(g.view(np.uint32).ravel() != w.view(np.uint32).ravel())[0]
    assert bad.size == 0, f"{what}: {bad.size}/{g.size} differ; first at {bad[0]}: got {g.ravel()[bad[0]]!r} " \
                          f"want {w.ravel()[bad[0]]!r}"


def oracle(x, wn, w):
    """The three nodes on the CPU: rms_norm, MUL by wn (both through xlns16
    and back to F32 between nodes), then the sum32 mul_mat."""
    h = O.rms_norm16(O.SUM32, x[None, :], EPS)
    hc = O.f2x16(h)
    wc = O.f2x16(np.broadcast_to(wn, h.shape).copy())
    mul = np.vectorize(lambda a, b: O.lib().lno16_mul(int(a), int(b)), otypes=[np.uint16])
    h = O.x2f16(mul(hc, wc))
    return O.mul_mat16_f32w(O.SUM32, w[None, None], h[None, None])[0, 0, 0]


def fused(ln, x, wn, wp, K, M):
    out = torch.empty(M, dtype=torch.float32, device="cuda")
    dx, dwn = dev(x), dev(wn)
    ln.check(ln.lib().lnship16_rms_norm_mul_mat(O.SUM32, P(dx), P(dwn), ctypes.c_float(EPS), P(wp), P(out), K, M,
                                                ln._stream()))
    return host(out)


def two_launch(ln, x, wn, wp, K, M):
    dx, dwn = dev(x[None, :]), dev(wn)
    h = torch.empty_like(dx)
    ln.check(ln.lib().lnship16_rms_norm_mul(O.SUM32, P(dx), P(dwn), P(h), K, 1, ctypes.c_float(EPS), 7, None, 0,
                                            ln._stream()))
    return host(ln.mul_mat16(O.SUM32, wp, h, K, M))[0]


def case(rng, K, M, xscale):
    x = (rng.standard_normal(K) * xscale).astype(np.float32)
    wn = (rng.standard_normal(K) * 0.5 + 1.0).astype(np.float32)
    w = (rng.standard_normal((M, K)) * 0.02).astype(np.float32)
    return x, wn, w


# SmolLM2's decode shapes (QKV 960, up|gate 3072 over d_model 576), rows
# around the 192 chain lanes of a workgroup, K tails, tiny and wide rows
SHAPES = [(576, 960, 1.0), (576, 3072, 0.05), (577, 193, 3.0), (13, 5, 30.0), (1, 1, 1.0), (2048, 400, 0.02),
          (576, 191, 1e-3)]


@pytest.mark.parametrize("K,M,xscale", SHAPES)
def test_rms_norm_mul_mat_equals_three_nodes(ln, K, M, xscale):
    print(f"\n[rms_norm_mul_mat] K={K} M={M} xscale={xscale}", flush=True)
    rng = np.random.default_rng(K * 7919 + M)
    x, wn, w = case(rng, K, M, xscale)
    wp = ln.pack16(dev(w))
    want = oracle(x, wn, w)
    same_bits(fused(ln, x, wn, wp, K, M), want, f"fused K={K} M={M}")
    same_bits(two_launch(ln, x, wn, wp, K, M), want, f"two launches K={K} M={M}")


@pytest.mark.parametrize("skew", [1, -1, 9])
def test_rms_norm_mul_mat_mispredicted_scale(ln, skew):
    # every prediction off by skew codes: the result comes from the second pass
    print(f"\n[rms_norm_mul_mat] skew={skew}", flush=True)
    rng = np.random.default_rng(100 + skew)
    prev = ln.lib().lnship_test_predict_skew(skew)
    try:
        for K, M, xscale in [(576, 960, 1.0), (577, 193, 3.0), (13, 5, 30.0)]:
            x, wn, w = case(rng, K, M, xscale)
            wp = ln.pack16(dev(w))
            same_bits(fused(ln, x, wn, wp, K, M), oracle(x, wn, w), f"skew {skew} K={K} M={M}")
    finally:
        ln.lib().lnship_test_predict_skew(prev)


def test_rms_norm_mul_mat_logits_shape(ln):
    # the tied output layer's shape (vocab 49152 rows), against the two launches
    print("\n[rms_norm_mul_mat] K=576 M=49152", flush=True)
    rng = np.random.default_rng(5)
    K, M = 576, 49152
    x, wn, w = case(rng, K, M, 0.3)
    wp = ln.pack16(dev(w))
    same_bits(fused(ln, x, wn, wp, K, M), two_launch(ln, x, wn, wp, K, M), "logits shape")


def test_rms_norm_mul_mat_refuses_other_modes(ln):
    x = torch.ones(8, device="cuda")
    wp = ln.pack16(torch.ones(4, 8, device="cuda"))
    out = torch.empty(4, device="cuda")
    for mode in (O.BASE, O.MONTE, O.LPVIP):
        rc = ln.lib().lnship16_rms_norm_mul_mat(mode, P(x), P(x), ctypes.c_float(EPS), P(wp), P(out), 8, 4,
                                                ln._stream())
        assert rc == -1, (mode, rc)
        assert b"sum32 only" in ln.lib().lnship_last_error()


def swiglu_oracle(gate, up):
    L = O.lib()
    L.lno16_swiglu_f32.argtypes = [ctypes.c_void_p] * 2 + [ctypes.c_int64, ctypes.c_void_p]
    sw = np.empty_like(gate)
    L.lno16_swiglu_f32(O._ptr(gate), O._ptr(up), gate.size, O._ptr(sw))
    return sw


@pytest.mark.parametrize("mode", ["base", "lpvip", "sum32"])
@pytest.mark.parametrize("K,M", [(1536, 576), (13, 5), (1537, 193)])
def test_swiglu_mul_mat_equals_two_nodes(ln, mode, K, M):
    # the down projection's shape (up | gate rows of 2K, residual in place)
    print(f"\n[swiglu_mul_mat] {mode} K={K} M={M}", flush=True)
    m = O.MODES[mode]
    rng = np.random.default_rng(K + 31 * M)
    ug = (rng.standard_normal(2 * K) * 0.7).astype(np.float32)
    w = (rng.standard_normal((M, K)) * 0.02).astype(np.float32)
    resid = rng.standard_normal(M).astype(np.float32)
    wp = ln.pack16(dev(w))
    dug = dev(ug)
    gate_p, up_p = ctypes.c_void_p(dug.data_ptr() + 4 * K), P(dug)
    # without the residual: against the oracle
    out = torch.empty(M, device="cuda")
    ln.check(ln.lib().lnship16_swiglu_mul_mat(m, gate_p, up_p, P(wp), None, P(out), K, M, ln._stream()))
    want = O.mul_mat16_f32w(m, w[None, None], swiglu_oracle(ug[K:].copy(), ug[:K].copy())[None, None, None])[0, 0, 0]
    same_bits(host(out), want, f"swiglu_mul_mat {mode} K={K} M={M}")
    # with the residual, written over it: against lnship16_swiglu, then the mul_mat with its ADD
    x = dev(resid)
    ln.check(ln.lib().lnship16_swiglu_mul_mat(m, gate_p, up_p, P(wp), P(x), P(x), K, M, ln._stream()))
    sw = torch.empty(1, K, device="cuda")
    ln.check(ln.lib().lnship16_swiglu(gate_p, 2 * K, up_p, 2 * K, P(sw), K, 1, ln._stream()))
    ref = dev(resid)
    ln.mul_mat16_raw(m, wp.data_ptr(), sw.data_ptr(), ref.data_ptr(), K, M, 1, residual=P(ref))
    same_bits(host(x), host(ref), f"swiglu_mul_mat + residual {mode} K={K} M={M}")


def test_swiglu_mul_mat_refuses_monte(ln):
    x = torch.ones(16, device="cuda")
    wp = ln.pack16(torch.ones(4, 8, device="cuda"))
    out = torch.empty(4, device="cuda")
    assert ln.lib().lnship16_swiglu_mul_mat(O.MONTE, P(x), P(x), P(wp), None, P(out), 8, 4, ln._stream()) == -1


# ---- lnship16_mul_mat's prologue fields: the node before the product ---------
# (rms_norm_w: RMS_NORM and the norm MUL; glu_up: the GLU node's swiglu) in the
# launch of a mul_mat of N activation rows, every mode, Monte with the
# rms_norm node's own start: against the oracle of the separate nodes (Monte:
# one LFSR sequence through them in graph order) and against the library's
# separate launches with the residual ADD


def mm_args(ln, wp, x_ptr, out, K, M, N, seed, x_ld=0, residual=None):
    sd, st, off = ln.seed_fields(seed)
    return ln.MulMatArgs(wp.data_ptr(), x_ptr, out.data_ptr(), K, M, N, 1, 1, 1, 1, x_ld, 0, sd, 0, 0, 0, 0, st,
                         off or 0, residual)


def rms_mul_oracle(mode, x, wn, w, s0):
    """rms_norm (Monte from s0), the MUL by wn, then the mul_mat (Monte: the
    LFSR where rms_norm left it), F32 between the nodes."""
    O.monte_set(s0)
    h = O.rms_norm16(mode, x, EPS)
    mul = np.vectorize(lambda a, b: O.lib().lno16_mul(int(a), int(b)), otypes=[np.uint16])
    h = O.x2f16(mul(O.f2x16(h), O.f2x16(np.broadcast_to(wn, h.shape).copy())))
    return O.mul_mat16_f32w(mode, w[None, None], h[None, None])[0, 0]


@pytest.mark.parametrize("mode", ["base", "monte", "lpvip", "sum32"])
@pytest.mark.parametrize("K,M,N", [(576, 960, 8), (577, 193, 3), (13, 5, 1), (1536, 576, 2), (576, 3072, 8),
                                   (576, 700, 16), (200, 300, 40)])
def test_mul_mat_rms_prologue_equals_three_nodes(ln, mode, K, M, N):
    # (16 and 40 rows: launches of several columns per workgroup, where the
    # rms chains of the columns share wave 0)
    print(f"\n[mul_mat rms prologue] {mode} K={K} M={M} N={N}", flush=True)
    m = O.MODES[mode]
    L = ln.lib()
    rng = np.random.default_rng(K + 17 * M + 5 * N)
    x = (rng.standard_normal((N, K)) * 1.5).astype(np.float32)
    wn = (rng.standard_normal(K) * 0.5 + 1.0).astype(np.float32)
    w = (rng.standard_normal((M, K)) * 0.02).astype(np.float32)
    resid = rng.standard_normal((N, M)).astype(np.float32)
    wp, dx, dwn = ln.pack16(dev(w)), dev(x), dev(wn)
    s0 = 3001
    d_rms = L.lnship16_rms_norm_draws(m, K, N)
    s1 = L.lnship_lfsr_jump(s0, d_rms)

    def fused(seeds, residual=None):
        out = dev(resid) if residual is not None else torch.full((N, M), float("nan"), device="cuda")
        a = mm_args(ln, wp, dx.data_ptr(), out, K, M, N, seeds[1], residual=out.data_ptr() if residual else None)
        rsd, _, roff = ln.seed_fields(seeds[0])
        a.rms_norm_w, a.rms_eps, a.rms_seed, a.rms_offset = dwn.data_ptr(), EPS, rsd, roff or 0
        ln.check(L.lnship16_mul_mat(m, ctypes.byref(a), ln._stream()))
        return host(out)

    got = fused((s0, s1))
    if M * K * N <= 8_000_000:
        same_bits(got, rms_mul_oracle(m, x, wn, w, s0), f"rms prologue {mode} K={K} M={M} N={N} vs oracle")
    # the residual ADD, against the library's rms_norm_mul and mul_mat launches
    h = torch.empty(N, K, device="cuda")
    ln.check(L.lnship16_rms_norm_mul(m, P(dx), P(dwn), P(h), K, N, ctypes.c_float(EPS), s0, None, 0, ln._stream()))
    ref = dev(resid)
    ln.mul_mat16_raw(m, wp.data_ptr(), h.data_ptr(), ref.data_ptr(), K, M, N, seed=s1, residual=P(ref))
    same_bits(fused((s0, s1), residual=True), host(ref), f"rms prologue + residual {mode} K={K} M={M} N={N}")
    if mode == "monte":
        # both starts read from one device state, with their offsets
        S = 777
        st = torch.tensor([S], dtype=torch.int16, device="cuda")
        g2 = fused(((st, 5), (st, 5 + d_rms)))
        want = fused((L.lnship_lfsr_jump(S, 5), L.lnship_lfsr_jump(S, 5 + d_rms)))
        same_bits(g2, want, f"rms prologue monte K={K} N={N}: state vs seeds")
        if K >= 64:   # (a 13-term row may round alike from other draws)
            assert not np.array_equal(want, got), "other starts, other draws"


@pytest.mark.parametrize("mode", ["base", "monte", "lpvip", "sum32"])
@pytest.mark.parametrize("K,M,N", [(1536, 576, 8), (13, 5, 3), (1537, 193, 1)])
def test_mul_mat_glu_prologue_equals_two_nodes(ln, mode, K, M, N):
    # the down projection of a decode step: gate | up rows of 2K (x_ld 2K),
    # the residual ADD in place
    print(f"\n[mul_mat glu prologue] {mode} K={K} M={M} N={N}", flush=True)
    m = O.MODES[mode]
    L = ln.lib()
    rng = np.random.default_rng(K + 31 * M + N)
    ug = (rng.standard_normal((N, 2 * K)) * 0.7).astype(np.float32)
    w = (rng.standard_normal((M, K)) * 0.02).astype(np.float32)
    resid = rng.standard_normal((N, M)).astype(np.float32)
    wp, dug = ln.pack16(dev(w)), dev(ug)
    gate_p, up_p = dug.data_ptr() + 4 * K, dug.data_ptr()
    s0 = 1234
    out = torch.full((N, M), float("nan"), device="cuda")
    a = mm_args(ln, wp, gate_p, out, K, M, N, s0, x_ld=2 * K)
    a.glu_up = up_p
    ln.check(L.lnship16_mul_mat(m, ctypes.byref(a), ln._stream()))
    sw = np.stack([swiglu_oracle(ug[n, K:].copy(), ug[n, :K].copy()) for n in range(N)])
    O.monte_set(s0)
    same_bits(host(out), O.mul_mat16_f32w(m, w[None, None], sw[None, None])[0, 0],
              f"glu prologue {mode} K={K} M={M} N={N} vs oracle")
    x = dev(resid)
    a = mm_args(ln, wp, gate_p, x, K, M, N, s0, x_ld=2 * K, residual=x.data_ptr())
    a.glu_up = up_p
    ln.check(L.lnship16_mul_mat(m, ctypes.byref(a), ln._stream()))
    swd = torch.empty(N, K, device="cuda")
    ln.check(L.lnship16_swiglu(ctypes.c_void_p(gate_p), 2 * K, ctypes.c_void_p(up_p), 2 * K, P(swd), K, N,
                               ln._stream()))
    ref = dev(resid)
    ln.mul_mat16_raw(m, wp.data_ptr(), swd.data_ptr(), ref.data_ptr(), K, M, N, seed=s0, residual=P(ref))
    same_bits(host(x), host(ref), f"glu prologue + residual {mode} K={K} M={M} N={N}")


def test_mul_mat_prologue_rows_too_long(ln):
    # a row that does not fit LDS beside the tables: LNSHIP_ERANGE before
    # any launch (the caller runs the nodes apart), dst untouched
    L = ln.lib()
    K, M = 100000, 8
    wp = ln.pack16(torch.zeros(M, K, device="cuda"))
    x = torch.ones(1, K, device="cuda")
    out = torch.full((1, M), 7.0, device="cuda")
    for mode in (O.BASE, O.SUM32):
        a = mm_args(ln, wp, x.data_ptr(), out, K, M, 1, 7)
        a.rms_norm_w, a.rms_eps = x.data_ptr(), EPS
        assert L.lnship16_mul_mat(mode, ctypes.byref(a), ln._stream()) == -4, mode
    wp32 = ln.pack32(torch.zeros(M, K, device="cuda"))
    a = mm_args(ln, wp32, x.data_ptr(), out, K, M, 1, 0)
    a.rms_norm_w, a.rms_eps = x.data_ptr(), EPS
    assert L.lnship32_mul_mat(ctypes.byref(a), ln._stream()) == -4
    assert np.all(host(out) == 7.0)


def test_mul_mat_prologue_refusals(ln):
    # both nodes at once, several activation slices: refused, nothing
    # launched; lnship32_mul_mat_noalloc takes neither
    L = ln.lib()
    wp = ln.pack16(torch.ones(4, 8, device="cuda"))
    x = torch.ones(2, 8, device="cuda")
    out = torch.empty(2, 4, device="cuda")
    a = mm_args(ln, wp, x.data_ptr(), out, 8, 4, 2, 7)
    a.rms_norm_w, a.glu_up = x.data_ptr(), x.data_ptr()
    assert L.lnship16_mul_mat(O.BASE, ctypes.byref(a), ln._stream()) == -1
    a = mm_args(ln, wp, x.data_ptr(), out, 8, 4, 1, 7)
    a.ne12 = a.ne02 = 2
    a.rms_norm_w = x.data_ptr()
    assert L.lnship16_mul_mat(O.BASE, ctypes.byref(a), ln._stream()) == -1
    a = mm_args(ln, wp, x.data_ptr(), out, 8, 4, 2, 7)
    a.glu_up = x.data_ptr()
    assert L.lnship32_mul_mat_noalloc(ctypes.byref(a), ln._stream()) == -1
    a.rms_norm_w = x.data_ptr()
    assert L.lnship32_mul_mat(ctypes.byref(a), ln._stream()) == -1


# ---- the same prologues in lnship32_mul_mat (LNS32: lns32_rms_norm,
# lns32_mul, lns32_swiglu, then lns32_mul_mat, src32/lns32-ops.cpp), and its
# one-column launches that convert their own activations


@pytest.mark.parametrize("K,M,N", [(2048, 3072, 1), (2048, 300, 1), (13, 5, 1), (77, 96, 3), (4096, 256, 1)])
def test_mul_mat32_rms_prologue_equals_three_nodes(ln, K, M, N):
    print(f"\n[mul_mat32 rms prologue] K={K} M={M} N={N}", flush=True)
    L = ln.lib()
    rng = np.random.default_rng(4 * K + M + N)
    x = (rng.standard_normal((N, K)) * 1.5).astype(np.float32)
    wn = (rng.standard_normal(K) * 0.5 + 1.0).astype(np.float32)
    w = (rng.standard_normal((M, K)) * 0.02).astype(np.float32)
    resid = rng.standard_normal((N, M)).astype(np.float32)
    wp, dx, dwn = ln.pack32(dev(w)), dev(x), dev(wn)
    h = O.mul32(O.rms_norm32(x, EPS), wn)
    want = O.mul_mat32(w, h)
    for residual in (False, True):
        out = dev(resid) if residual else torch.full((N, M), float("nan"), device="cuda")
        a = mm_args(ln, wp, dx.data_ptr(), out, K, M, N, 0, residual=out.data_ptr() if residual else None)
        a.rms_norm_w, a.rms_eps = dwn.data_ptr(), EPS
        ln.check(L.lnship32_mul_mat(ctypes.byref(a), ln._stream()))
        if not residual:
            same_bits(host(out), want, f"mul_mat32 rms prologue K={K} M={M} N={N} vs oracle")
        else:
            ref = dev(resid)
            ln.mul_mat32_raw(wp.data_ptr(), dev(h).data_ptr(), ref.data_ptr(), K, M, N, residual=P(ref))
            same_bits(host(out), host(ref), f"mul_mat32 rms prologue + residual K={K} M={M} N={N}")


@pytest.mark.parametrize("K,M", [(2048, 512), (13, 5), (1537, 193)])
def test_mul_mat32_glu_prologue_equals_two_nodes(ln, K, M):
    print(f"\n[mul_mat32 glu prologue] K={K} M={M}", flush=True)
    L = ln.lib()
    rng = np.random.default_rng(K + 7 * M)
    ug = (rng.standard_normal(2 * K) * 0.7).astype(np.float32)
    w = (rng.standard_normal((M, K)) * 0.02).astype(np.float32)
    wp, dug = ln.pack32(dev(w)), dev(ug)
    out = torch.full((1, M), float("nan"), device="cuda")
    a = mm_args(ln, wp, dug.data_ptr() + 4 * K, out, K, M, 1, 0, x_ld=2 * K)
    a.glu_up = dug.data_ptr()
    ln.check(L.lnship32_mul_mat(ctypes.byref(a), ln._stream()))
    want = O.mul_mat32(w, O.swiglu32(ug[K:].copy(), ug[:K].copy())[None])
    same_bits(host(out), want, f"mul_mat32 glu prologue K={K} M={M} vs oracle")


@pytest.mark.parametrize("K,M,N,nslices", [(2048, 3072, 1, 1), (64, 768, 1, 32), (768, 64, 1, 32), (2048, 32000, 1, 1),
                                           (8192, 2048, 1, 1), (3, 7, 2, 1), (2048, 512, 4, 1)])
def test_mul_mat32_own_conversion_equals_staged(ln, K, M, N, nslices):
    # lnship32_mul_mat's one-column launches convert their activations into
    # LDS themselves; lnship32_mul_mat_noalloc converts them first (k_act) in
    # every case: the two agree bit for bit, GQA broadcast (32 activation
    # slices over 8 weight slices) and the 32000-row output shape included
    print(f"\n[mul_mat32 own conversion] K={K} M={M} N={N} slices={nslices}", flush=True)
    L = ln.lib()
    rng = np.random.default_rng(K + M + 13 * N + nslices)
    ne02 = max(1, nslices // 4)
    w = (rng.standard_normal((ne02, M, K)) * 0.05).astype(np.float32)
    x = (rng.standard_normal((nslices, N, K))).astype(np.float32)
    wp, dx = ln.pack32(dev(w)), dev(x)
    outs = []
    for fn in (L.lnship32_mul_mat, L.lnship32_mul_mat_noalloc):
        out = torch.full((nslices, N, M), float("nan"), device="cuda")
        a = ln.MulMatArgs(wp.data_ptr(), dx.data_ptr(), out.data_ptr(), K, M, N, ne02, 1, nslices, 1, 0, 0, 0, 0, 0, 0,
                          0, None, 0, None)
        rc = fn(ctypes.byref(a), ln._stream())
        if rc == -4:   # the fixed block of noalloc holds at most 1 Mi codes
            pytest.skip("beyond the fixed scratch")
        ln.check(rc)
        outs.append(host(out))
    same_bits(outs[0], outs[1], f"own conversion K={K} M={M} N={N} slices={nslices}")
    if M * K * N * nslices <= 4_000_000:
        same_bits(outs[0], O.mul_mat32(w, x, ne02=ne02), f"own conversion K={K} M={M} vs oracle")
