"""lnship32_mul_mat_noalloc, the entry point that allocates nothing, through
the C ABI: its outputs equal lnship32_mul_mat's bit for bit on consecutive
calls (the second smaller than the first, so stale staging from the first
call is overwritten where it is read), up to and at its 1 Mi-code limit, and
a larger call is refused before anything runs."""
import ctypes

import numpy as np
import pytest

import oracle_lib as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

LIMIT = 1 << 20   # activation codes the fixed scratch holds


@pytest.fixture(scope="module")
def ln():
    import lnship
    lnship.init()
    return lnship


def _run(ln, fn, wp, x, out, K, M, ne12):
    N = x.shape[-2]
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    a = ln.MulMatArgs(p(wp), p(x), p(out), K, M, N, 1, 1, ne12, 1, 0, 0, 0, 0, 0, 0, 0, None, 0, None)
    return getattr(ln.lib(), fn)(ctypes.byref(a), ln._stream())


def _case(ln, K, M, N, ne12, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((M, K)) * 0.02).astype(np.float32)
    x = rng.standard_normal((ne12, N, K)).astype(np.float32)
    wp = ln.pack32(torch.from_numpy(w).cuda())
    xd = torch.from_numpy(x).cuda()
    ref = torch.full((ne12, N, M), float("nan"), device="cuda")
    got = torch.full((ne12, N, M), float("nan"), device="cuda")
    return w, x, wp, xd, ref, got


def test_noalloc_equals_mul_mat_on_consecutive_calls(ln):
    # (K, M, N, ne12): the first call fills most of the fixed block, the
    # second is smaller; the third is exactly at the limit
    for K, M, N, ne12, seed in ((2048, 96, 100, 4, 1), (576, 300, 3, 1, 2), (2048, 40, 512, 1, 3)):
        print(f"\n[noalloc] K={K} M={M} N={N} ne12={ne12}", flush=True)
        assert ne12 * N * ((K + 7) // 8 * 8) <= LIMIT
        w, x, wp, xd, ref, got = _case(ln, K, M, N, ne12, seed)
        assert _run(ln, "lnship32_mul_mat", wp, xd, ref, K, M, ne12) == 0
        assert _run(ln, "lnship32_mul_mat_noalloc", wp, xd, got, K, M, ne12) == 0
        torch.cuda.synchronize()
        r, g = ref.cpu().numpy(), got.cpu().numpy()
        assert np.array_equal(g.view(np.uint32), r.view(np.uint32)), (K, M, N, ne12)
        if K * M * N * ne12 < 2e6:   # and the small one against the oracle as well
            want = O.mul_mat32(w, x.reshape(ne12 * N, K)).reshape(ne12, N, M)
            assert np.array_equal(g.view(np.uint32), want.view(np.uint32))


def test_noalloc_refuses_beyond_its_block(ln):
    K, M, N = 2048, 8, 513                      # 513 * 2048 codes > 1 Mi
    print(f"\n[noalloc] refused K={K} N={N}", flush=True)
    w, x, wp, xd, ref, got = _case(ln, K, M, N, 1, 4)
    assert _run(ln, "lnship32_mul_mat_noalloc", wp, xd, got, K, M, 1) == -4   # LNSHIP_ERANGE
    assert b"fixed scratch" in ln.lib().lnship_last_error()
    torch.cuda.synchronize()
    assert torch.isnan(got).all()               # nothing ran
