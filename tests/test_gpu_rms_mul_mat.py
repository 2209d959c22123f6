"""GPU parity of lnship16_rms_norm_mul_mat, the decode step's rms_norm, norm
MUL and mul_mat in one launch (lns_rms_norm, lns_mul, lns_mul_mat:
src/lns-ops.cpp:701-736, :468-530, :293-384), bit for bit against the CPU
oracle of the three nodes and against the library's two-launch path.

The kernel starts the mul_mat's chains from a predicted rms scale and runs
them again when the rms chain's scale differs; the skew hook makes every
prediction wrong, so the second pass is checked too."""
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
