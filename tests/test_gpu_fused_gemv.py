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
