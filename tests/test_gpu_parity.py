"""GPU parity: the gfx950 kernels against the CPU oracle, bit for bit.

Follows the reference's parity harness (lns-backend/tests/
test-lns-cuda-parity.cpp:158-171 memcmp, cases :255-366): mul_mat with N not
a multiple of the column tile, K=1536 / 4096 / 1, N=1, GQA and 4-D broadcast,
rms_norm and soft_max with singleton rows and padded masks, Monte from equal
LFSR states.  Inputs are seeded; every case prints its name before it runs.
"""
import numpy as np
import pytest

import oracle_lib as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

MODES = ["base", "monte", "lpvip", "sum32"]


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


def same_bits(got, want, what):
    g, w = np.ascontiguousarray(got), np.ascontiguousarray(want)
    assert g.shape == w.shape, (what, g.shape, w.shape)
    gb, wb = g.view(np.uint32), w.view(np.uint32)
    bad = np.nonzero(gb.ravel() != wb.ravel())[0]
    assert bad.size == 0, f"{what}: {bad.size}/{g.size} differ; first at {bad[0]}: got {g.ravel()[bad[0]]!r} want {w.ravel()[bad[0]]!r}"


# ---------------------------------------------------------------- conversion --

def test_from_f32_16_every_bucket(ln):
    # every 2^15-wide bucket of float bit patterns: lowest, highest, middle
    b = np.arange(1 << 17, dtype=np.uint64) << 15
    bits = np.concatenate([b, b + 0x7FFF, b + 0x4321]).astype(np.uint32)
    x = bits.view(np.float32)
    got = host(ln.from_f32_16(dev(x))).view(np.uint16)
    assert np.array_equal(got, O.f2x16(x))


def test_to_f32_16_every_code(ln):
    codes = np.arange(65536, dtype=np.uint16)
    got = host(ln.to_f32_16(dev(codes.view(np.int16))))
    same_bits(got, O.x2f16(codes), "xlns16 -> f32")


def _x32_add_cases(rng):
    """xlns32 code pairs (x, y) over the adder's cases: every cotransformation
    split d = (dh << 12) + dl with dl in {0, 1, 2, 4095, random} for each dh
    and dh in {0, 1, 4095, random} for each dl, distances out to 30 binades,
    d = 0, and logs at both ends of the field (clamp at 0, saturation)."""
    B = 1 << 23
    d = []
    dh = np.arange(4096, dtype=np.int64)
    for dl in (0, 1, 2, 4095, None):
        d.append((dh << 12) + (rng.integers(0, 4096, 4096) if dl is None else dl))
    dl = np.arange(4096, dtype=np.int64)
    for h in (0, 1, 4095, None):
        d.append(((rng.integers(0, 4096, 4096) if h is None else h) << 12) + dl)
    d.append(rng.integers(1 << 24, 30 * B, 8192))
    d.append(np.zeros(256, np.int64))
    d = np.concatenate(d)
    a = rng.integers(32 * B, (1 << 31) - 32 * B, d.size)
    b = np.where(rng.integers(0, 2, d.size) == 1, a + d, a - d)
    # half the pairs with opposite signs (the db and cotransformation cases)
    sa = rng.integers(0, 2, d.size).astype(np.int64)
    sb = np.where(np.arange(d.size) % 2 == 0, 1 - sa, rng.integers(0, 2, d.size))
    # the ends: tiny logs that cancel below 0, large ones that overflow
    lo = rng.integers(0, 1 << 22, 2048)
    hi = rng.integers((1 << 31) - (1 << 22), 1 << 31, 2048)
    a = np.concatenate([a, lo, hi, hi])
    b = np.concatenate([b, lo + rng.integers(0, 1 << 12, 2048), hi - rng.integers(0, 1 << 23, 2048),
                        rng.integers((1 << 31) - (1 << 24), 1 << 31, 2048)])
    sa = np.concatenate([sa, np.zeros(2048, np.int64), np.zeros(4096, np.int64)])
    sb = np.concatenate([sb, np.ones(2048, np.int64), np.zeros(4096, np.int64)])
    x = (a | (sa << 31)).astype(np.uint32)
    y = (b | (sb << 31)).astype(np.uint32)
    return x, y


def test_xlns32_lds_adder_every_case(ln):
    # the adder over its LDS image (sentinels, extended far grid, descriptor
    # caps) in the three forms the kernels run, against xlns32_add
    import ctypes
    x, y = _x32_add_cases(np.random.default_rng(73))
    add = O.lib().lno32_add
    want = np.array([add(int(p), int(q)) for p, q in zip(x, y)], np.uint32)
    m = np.uint32(0x7FFFFFFF)
    want_pos = np.array([add(int(p), int(q)) for p, q in zip(x & m, y & m)], np.uint32)
    dx, dy = dev(x.view(np.int32)), dev(y.view(np.int32))
    for form, ref in ((0, want), (1, want), (2, want_pos)):
        print(f"\n[xlns32 LDS adder] form {form}, {x.size} pairs", flush=True)
        out = torch.empty_like(dx)
        ln.check(ln.lib().lnship32_add_lds(form, ctypes.c_void_p(dx.data_ptr()), ctypes.c_void_p(dy.data_ptr()),
                                            ctypes.c_void_p(out.data_ptr()), x.size, ln._stream()))
        got = host(out).view(np.uint32)
        bad = np.nonzero(got != ref)[0]
        assert bad.size == 0, (f"form {form}: {bad.size} differ; first x={x[bad[0]]:#x} y={y[bad[0]]:#x}: "
                               f"got {got[bad[0]]:#x} want {ref[bad[0]]:#x}")


def test_xlns32_positive_adders_every_grid_node(ln):
    # the two positive-sum forms (2: over the adder's image, 3: over the
    # pair image of the row kernels) at every sb grid node and its
    # neighbours, random distances to 30 binades and the saturating end,
    # against xlns32_add
    import ctypes
    rng = np.random.default_rng(29)
    B = 1 << 23
    near = np.arange(0, 12 * B + 1, 1 << 13, dtype=np.int64)
    far = np.arange(12 * B, 24 * B + 1, 1 << 19, dtype=np.int64)
    d = np.concatenate([near, near + 1, near + (1 << 13) - 1, far, far + 1, far + (1 << 19) - 1, far - 1,
                        rng.integers(0, 30 * B, 1 << 16), np.array([0, 24 * B - 1, 24 * B, 24 * B + 1])])
    d = d[d >= 0]
    a = rng.integers(32 * B, (1 << 31) - 32 * B, d.size)
    b = np.where(rng.integers(0, 2, d.size) == 1, a + d, a - d)
    hi = rng.integers((1 << 31) - (1 << 22), 1 << 31, 2048)
    x = np.concatenate([a, hi]).astype(np.uint32)
    y = np.concatenate([b, rng.integers((1 << 31) - (1 << 24), 1 << 31, 2048)]).astype(np.uint32)
    add = O.lib().lno32_add
    want = np.array([add(int(p), int(q)) for p, q in zip(x, y)], np.uint32)
    dx, dy = dev(x.view(np.int32)), dev(y.view(np.int32))
    for form in (2, 3):
        print(f"\n[xlns32 positive adder] form {form}, {x.size} pairs", flush=True)
        out = torch.empty_like(dx)
        ln.check(ln.lib().lnship32_add_lds(form, ctypes.c_void_p(dx.data_ptr()), ctypes.c_void_p(dy.data_ptr()),
                                            ctypes.c_void_p(out.data_ptr()), x.size, ln._stream()))
        got = host(out).view(np.uint32)
        bad = np.nonzero(got != want)[0]
        assert bad.size == 0, (f"form {form}: {bad.size} differ; first x={x[bad[0]]:#x} y={y[bad[0]]:#x}: "
                               f"got {got[bad[0]]:#x} want {want[bad[0]]:#x}")


def test_xlns32_conversion_sampled(ln):
    rng = np.random.default_rng(11)
    bits = rng.integers(0, 1 << 32, 1 << 20, dtype=np.uint64).astype(np.uint32)
    special = np.array([0, 0x80000000, 0x3F800000, 0x7F800000, 0xFF800000, 0x7FC00000, 1, 0x807FFFFF,
                        0x00800000, 0x7F7FFFFF], dtype=np.uint32)
    x = np.concatenate([bits, special]).view(np.float32)
    got = host(ln.from_f32_32(dev(x))).view(np.uint32)
    want = O.f2x32(x)
    assert np.array_equal(got, want), int(np.sum(got != want))
    codes = rng.integers(0, 1 << 32, 1 << 20, dtype=np.uint64).astype(np.uint32)
    back = host(ln.to_f32_32(dev(codes.view(np.int32))))
    same_bits(back, O.x2f32(codes), "xlns32 -> f32")


# ------------------------------------------------------------------- mul_mat --

def _mm_case(ln, mode, K, M, N, ne02=1, ne03=1, ne12=1, ne13=1, seed=0, wscale=0.02, lfsr=7):
    print(f"\n[mul_mat] mode={mode} K={K} M={M} N={N} w=({ne03},{ne02}) x=({ne13},{ne12})", flush=True)
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((ne03, ne02, M, K)) * wscale).astype(np.float32)
    x = rng.standard_normal((ne13, ne12, N, K)).astype(np.float32)
    m = O.MODES[mode]
    O.monte_set(lfsr)
    want = O.mul_mat16_f32w(m, w, x, ne02, ne03)
    wp = ln.pack16(dev(w))
    got = host(ln.mul_mat16(m, wp, dev(x), K, M, ne02, ne03, seed=lfsr))
    same_bits(got, want, f"mul_mat {mode} K={K} M={M} N={N}")
    if m == O.MONTE:
        # the oracle's LFSR advanced by exactly the draws the kernel reserves
        assert O.monte_get() == O.lib().lno_lfsr_jump(lfsr, ln.mul_mat_draws(m, K, M, N, ne12, ne13))


@pytest.mark.parametrize("mode", MODES)
def test_mul_mat_c1_gemv(ln, mode):
    # 1536x576 weight times 576x1, and K=1536 with 576 rows
    _mm_case(ln, mode, 576, 1536, 1, seed=1)
    _mm_case(ln, mode, 1536, 576, 1, seed=2)


@pytest.mark.parametrize("mode", MODES)
def test_mul_mat_ragged_shapes(ln, mode):
    _mm_case(ln, mode, 256, 67, 5, seed=3)          # N=5: not a multiple of the column tile
    _mm_case(ln, mode, 4096, 70, 7, seed=4)         # long K, N=7
    _mm_case(ln, mode, 1, 33, 3, seed=5)            # K=1
    _mm_case(ln, mode, 13, 300, 9, seed=6)          # K not a multiple of 8
    _mm_case(ln, mode, 64, 513, 130, seed=7)        # several column tiles and row blocks


@pytest.mark.parametrize("mode", MODES)
def test_mul_mat_broadcast(ln, mode):
    _mm_case(ln, mode, 64, 40, 3, ne02=3, ne12=9, seed=8)                # GQA: 9 query heads over 3 kv heads
    _mm_case(ln, mode, 32, 24, 2, ne02=2, ne03=2, ne12=4, ne13=6, seed=9)  # 4-D broadcast


def test_mul_mat_same_sign_long(ln):
    # same-sign K=2048: the stagnation regime of base sums
    for mode in MODES:
        print(f"\n[mul_mat same sign] {mode}", flush=True)
        rng = np.random.default_rng(10)
        w = np.abs(rng.standard_normal((1, 1, 96, 2048))).astype(np.float32)
        x = np.abs(rng.standard_normal((1, 1, 4, 2048))).astype(np.float32)
        O.monte_set(7)
        want = O.mul_mat16_f32w(O.MODES[mode], w, x)
        got = host(ln.mul_mat16(O.MODES[mode], ln.pack16(dev(w)), dev(x), 2048, 96))
        same_bits(got, want, f"same-sign {mode}")


def test_mul_mat_monte_seeds(ln):
    # equal LFSR states give equal results; a different state gives another
    for lfsr in (7, 1, 0xB403, 65535):
        _mm_case(ln, "monte", 128, 64, 3, seed=12, lfsr=lfsr)


def test_monte_start_from_device_state(ln):
    # ops given (device state, offset) start where the 16-bit seed
    # lfsr_jump(state, offset) would, and lnship_lfsr_advance moves the state
    rng = np.random.default_rng(14)
    w = (rng.standard_normal((1, 1, 64, 96)) * 0.05).astype(np.float32)
    x = rng.standard_normal((1, 1, 3, 96)).astype(np.float32)
    xr = rng.standard_normal((5, 200)).astype(np.float32)
    xs = (rng.standard_normal((2, 3, 70)) * 2).astype(np.float32)
    wp = ln.pack16(dev(w))
    jump = O.lib().lno_lfsr_jump
    for s0, off in ((7, 0), (0xB403, 12345), (65535, 70000), (1, 65534)):
        print(f"\n[monte device state] state={s0:#06x} offset={off}", flush=True)
        st = torch.tensor([s0 - 65536 if s0 >= 32768 else s0], dtype=torch.int16, device="cuda")
        start = jump(s0, off)
        O.monte_set(start)
        same_bits(host(ln.mul_mat16(O.MONTE, wp, dev(x), 96, 64, seed=(st, off))), O.mul_mat16_f32w(O.MONTE, w, x),
                  f"mul_mat from state {s0} + {off}")
        O.monte_set(start)
        same_bits(host(ln.rms_norm16(O.MONTE, dev(xr), 1e-5, seed=(st, off))), O.rms_norm16(O.MONTE, xr, 1e-5),
                  f"rms_norm from state {s0} + {off}")
        O.monte_set(start)
        same_bits(host(ln.soft_max16(O.MONTE, dev(xs), None, 0.5, seed=(st, off))),
                  O.soft_max16(O.MONTE, xs, None, 0.5), f"soft_max from state {s0} + {off}")
        ln.lfsr_advance(st, off)
        assert int(host(st)[0]) & 0xFFFF == start


def test_mul_mat_f16_weights(ln):
    # F16 sources (the KV-cache operand of kq / kqv): converted as F32 values
    rng = np.random.default_rng(13)
    K, M, N = 64, 256, 4
    w16 = (rng.standard_normal((M, K)) * 0.5).astype(np.float16)
    x = rng.standard_normal((N, K)).astype(np.float32)
    want = O.mul_mat16_f32w(O.SUM32, w16.astype(np.float32), x)
    got = host(ln.mul_mat16(O.SUM32, ln.pack16(dev(w16)), dev(x), K, M))
    same_bits(got, want, "f16 weights")


def test_mul_mat_lns16_code_weights(ln):
    # GGML_TYPE_LNS16 weights: xlns16 codes packed as they are (no F32 round
    # trip, which would move about half of them)
    rng = np.random.default_rng(15)
    K, M, N = 200, 130, 3
    codes = rng.integers(0, 65536, (M, K)).astype(np.uint16)
    x = rng.standard_normal((N, K)).astype(np.float32)
    for mode in MODES:
        print(f"\n[mul_mat lns16 weights] {mode}", flush=True)
        O.monte_set(7)
        want = O.mul_mat16(O.MODES[mode], codes, x)
        got = host(ln.mul_mat16(O.MODES[mode], ln.pack16(dev(codes.view(np.int16))), dev(x), K, M))
        same_bits(got, want, f"lns16 weights {mode}")


def _sample(n, step):
    return np.unique(np.concatenate([np.arange(0, n, step), [n - 1]]))


# Shapes that select each workgroup shape of the xlns32-accumulating GEMVs on
# a 256-CU MI355X: (columns per lane, column groups), and whether the
# activations fit in LDS next to the tables.  Each output depends on its own
# row and column only, so the big shapes are checked exactly on a sample of
# rows x columns (every column group and wave slot is hit).
X32_SHAPES = [
    # K,    M,    N      lane cols x groups
    (21, 64, 1),      # 1 x 1
    (21, 64, 384),    # 1 x 2
    (21, 70, 768),    # 1 x 4, ragged rows
    (21, 64, 2000),   # 2 x 4, ragged columns
    (21, 300, 2048),  # 4 x 4
    (21, 1024, 2048),  # 8 x 4, activations in LDS
    (1000, 1024, 2048),  # 8 x 4, activations from global memory
    (1701, 300, 2040),  # 4 x 4, activations from global memory, K tail
]


@pytest.mark.parametrize("K,M,N", X32_SHAPES)
def test_mul_mat_sum32_workgroup_shapes(ln, K, M, N):
    print(f"\n[mul_mat sum32 shape] K={K} M={M} N={N}", flush=True)
    rng = np.random.default_rng(K * 7 + M + N)
    w = (rng.standard_normal((M, K)) * 0.02).astype(np.float32)
    x = rng.standard_normal((N, K)).astype(np.float32)
    got = host(ln.mul_mat16(O.SUM32, ln.pack16(dev(w)), dev(x), K, M))
    rows, cols = (_sample(M, 13), _sample(N, 31)) if K * M * N > 5e7 else (np.arange(M), np.arange(N))
    want = O.mul_mat16_f32w(O.SUM32, w[rows][None, None], x[cols][None, None])
    same_bits(got[cols][:, rows], want.reshape(len(cols), len(rows)), f"sum32 K={K} M={M} N={N}")


@pytest.mark.parametrize("K,M,N", X32_SHAPES[:5] + [(1000, 300, 2040)])
def test_mul_mat_lns32_workgroup_shapes(ln, K, M, N):
    print(f"\n[mul_mat lns32 shape] K={K} M={M} N={N}", flush=True)
    rng = np.random.default_rng(K * 5 + M + N)
    w = (rng.standard_normal((M, K)) * 0.02).astype(np.float32)
    x = rng.standard_normal((N, K)).astype(np.float32)
    got = host(ln.mul_mat32(ln.pack32(dev(w)), dev(x), K, M))
    rows, cols = (_sample(M, 13), _sample(N, 31)) if K * M * N > 5e7 else (np.arange(M), np.arange(N))
    want = O.mul_mat32(w[rows], x[cols])
    same_bits(got[cols][:, rows], want.reshape(len(cols), len(rows)), f"lns32 K={K} M={M} N={N}")


def test_mul_mat_lns32(ln):
    for (K, M, N, seed) in ((576, 300, 1, 20), (1536, 64, 5, 21), (9, 40, 3, 22)):
        print(f"\n[mul_mat lns32] K={K} M={M} N={N}", flush=True)
        rng = np.random.default_rng(seed)
        w = (rng.standard_normal((M, K)) * 0.02).astype(np.float32)
        x = rng.standard_normal((N, K)).astype(np.float32)
        want = O.mul_mat32(w, x)
        got = host(ln.mul_mat32(ln.pack32(dev(w)), dev(x), K, M))
        same_bits(got, want, f"lns32 mul_mat K={K}")


# ------------------------------------------------------------------ rms_norm --

@pytest.mark.parametrize("mode", MODES)
def test_rms_norm(ln, mode):
    rng = np.random.default_rng(30)
    for shape in ((1, 576), (128, 576), (3, 2, 2048), (5, 1), (70, 16)):
        print(f"\n[rms_norm] {mode} {shape}", flush=True)
        x = rng.standard_normal(shape).astype(np.float32)
        O.monte_set(7)
        want = O.rms_norm16(O.MODES[mode], x, 1e-5)
        got = host(ln.rms_norm16(O.MODES[mode], dev(x), 1e-5, seed=7))
        same_bits(got, want, f"rms_norm {mode} {shape}")


def test_rms_norm_lns32(ln):
    rng = np.random.default_rng(31)
    for shape in ((1, 576), (9, 2048), (4, 1)):
        x = rng.standard_normal(shape).astype(np.float32)
        same_bits(host(ln.rms_norm32(dev(x), 1e-5)), O.rms_norm32(x, 1e-5), f"rms_norm lns32 {shape}")


def _elementwise16(fn, a, b):
    """The oracle's LNS16 elementwise op on F32 arrays (b broadcast over a):
    both through xlns16, fn on the codes, back to F32 (lns_add / lns_mul)."""
    ca, cb = O.f2x16(a), O.f2x16(np.broadcast_to(b, a.shape).copy())
    f = np.vectorize(lambda x, y: fn(int(x), int(y)), otypes=[np.uint16])
    return O.x2f16(f(ca, cb))


@pytest.mark.parametrize("mode", MODES)
def test_rms_norm_mul(ln, mode):
    # RMS_NORM then MUL by the norm weight row, in one launch
    import ctypes
    rng = np.random.default_rng(32)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    for shape in ((1, 576), (70, 16), (3, 1)):
        print(f"\n[rms_norm_mul] {mode} {shape}", flush=True)
        x = rng.standard_normal(shape).astype(np.float32)
        w = (rng.standard_normal(shape[1]) * 2).astype(np.float32)
        w[0] = 0.0
        O.monte_set(7)
        want = _elementwise16(O.lib().lno16_mul, O.rms_norm16(O.MODES[mode], x, 1e-5), w)
        out = torch.empty(shape, dtype=torch.float32, device="cuda")
        dx, dw = dev(x), dev(w)
        ln.check(ln.lib().lnship16_rms_norm_mul(O.MODES[mode], P(dx), P(dw), P(out), shape[1], shape[0],
                                                ctypes.c_float(1e-5), 7, None, 0, ln._stream()))
        same_bits(host(out), want, f"rms_norm_mul {mode} {shape}")


def test_rms_norm_mul_lns32(ln):
    import ctypes
    rng = np.random.default_rng(33)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    for shape in ((1, 576), (9, 2048), (4, 1)):
        x = rng.standard_normal(shape).astype(np.float32)
        w = (rng.standard_normal(shape[1]) * 2).astype(np.float32)
        want = O.mul32(O.rms_norm32(x, 1e-5), w)
        out = torch.empty(shape, dtype=torch.float32, device="cuda")
        dx, dw = dev(x), dev(w)
        ln.check(ln.lib().lnship32_rms_norm_mul(P(dx), P(dw), P(out), shape[1], shape[0], ctypes.c_float(1e-5),
                                                ln._stream()))
        same_bits(host(out), want, f"rms_norm_mul lns32 {shape}")


def _narrow_cases(rng):
    """(name, K, M, weights, activations) for the one-column sum32 GEMV"""
    cases = []
    for K, M in ((576, 576), (1536, 576), (576, 1000), (13, 37), (1, 5)):
        cases.append((f"N(0,0.02) K={K} M={M}", K, M, (rng.standard_normal((M, K)) * 0.02).astype(np.float32),
                      rng.standard_normal(K).astype(np.float32)))
    K, M = 700, 96
    # magnitudes over 2^-60 .. 2^60 (every grid: near, far, past the
    # essential zero), zeros among them
    w = (rng.standard_normal((M, K)) * np.exp2(rng.uniform(-60, 60, (M, K)))).astype(np.float32)
    w[:, ::17] = 0.0
    cases.append(("wide range", K, M, w, (rng.standard_normal(K) * np.exp2(rng.uniform(-20, 20, K))).astype(np.float32)))
    # exact and near cancellations: pairs of equal terms of opposite signs
    x = rng.standard_normal(K).astype(np.float32)
    x[1::2] = -x[0::2]
    w2 = np.repeat((rng.standard_normal((M, K // 2)) * 0.5).astype(np.float32), 2, axis=1)
    w2[:, 1::4] *= np.float32(1.01)
    cases.append(("cancellations", K, M, w2, x))
    # one sign: only sb
    cases.append(("positive", K, M, np.abs(rng.standard_normal((M, K))).astype(np.float32),
                  np.abs(rng.standard_normal(K)).astype(np.float32)))
    return cases


@pytest.mark.parametrize("width", [0, 16])
@pytest.mark.parametrize("mode", MODES)
def test_gemv_narrow_waves_columns(ln, mode, width):
    # the single-chain GEMV with several columns (the batched decode's) in
    # every mode, on the narrow waves the launch picks (4 to 32 rows; 300,
    # 4608 and 24576 chains) and with 64 rows (width 0), against the oracle
    L = ln.lib()
    prev = L.lnship_test_decode_width(width)
    try:
        for (K, M, N) in ((576, 576, 8), (1536, 100, 3), (64, 3072, 8)):
            _mm_case(ln, mode, K, M, N, seed=K + N)
    finally:
        L.lnship_test_decode_width(prev)


@pytest.mark.parametrize("width", [0, 16])
def test_sum32_gemv_narrow_waves(ln, width):
    # the one-column sum32 GEMV with 16 rows per wave (the default) and with
    # 64 (width 0) against the oracle, plain and with the residual ADD, on
    # shapes and values that reach every table of the adder (the decoder
    # tests run the default width, the swiglu prologue included)
    L = ln.lib()
    rng = np.random.default_rng(4242)
    prev = L.lnship_test_decode_width(width)
    try:
        for name, K, M, w, x in _narrow_cases(rng):
            print(f"\n[sum32 gemv] width={width} {name}", flush=True)
            wp = ln.pack16(dev(w))
            want = O.mul_mat16_f32w(O.SUM32, w[None, None], x[None, None, None])[0, 0, 0]
            got = host(ln.mul_mat16(O.SUM32, wp, dev(x[None]), K, M))
            same_bits(got.reshape(-1), want, f"width {width} {name}")
            r = rng.standard_normal(M).astype(np.float32)
            acc = dev(r)
            ln.mul_mat16_raw(O.SUM32, wp.data_ptr(), dev(x[None]).data_ptr(), acc.data_ptr(), K, M, 1,
                             residual=acc.data_ptr())
            same_bits(host(acc), _elementwise16(O.lib().lno16_add, want[None], r[None])[0],
                      f"width {width} {name} residual")
    finally:
        L.lnship_test_decode_width(prev)


@pytest.mark.parametrize("width", [0, 16])
def test_lns32_gemv_narrow_waves(ln, width):
    # the one-column xlns32 GEMV (the LNS32 decoder's) with 16 rows per wave
    # and with 64, against the oracle, plain and with the residual ADD
    L = ln.lib()
    rng = np.random.default_rng(4343)
    prev = L.lnship_test_decode_width(width)
    try:
        for name, K, M, w, x in _narrow_cases(rng):
            print(f"\n[xlns32 gemv] width={width} {name}", flush=True)
            wp, dx = ln.pack32(dev(w)), dev(x[None])
            want = O.mul_mat32(w, x[None])
            y = torch.empty(1, M, device="cuda")
            ln.mul_mat32_raw(wp.data_ptr(), dx.data_ptr(), y.data_ptr(), K, M, 1)
            same_bits(host(y), want, f"width {width} {name}")
            r = rng.standard_normal((1, M)).astype(np.float32)
            acc = dev(r)
            ln.mul_mat32_raw(wp.data_ptr(), dx.data_ptr(), acc.data_ptr(), K, M, 1, residual=acc.data_ptr())
            same_bits(host(acc), O.add32(want, r), f"width {width} {name} residual")
    finally:
        L.lnship_test_decode_width(prev)


@pytest.mark.parametrize("mode", MODES + ["lns32"])
def test_mul_mat_residual(ln, mode):
    # the ADD after a mul_mat fused into it, in place (dst = residual), as
    # the decoder's attention output and down projections use it
    rng = np.random.default_rng(34)
    for (K, M, N) in ((576, 576, 1), (1536, 70, 3), (13, 33, 2)):
        print(f"\n[mul_mat residual] {mode} K={K} M={M} N={N}", flush=True)
        w = (rng.standard_normal((M, K)) * 0.02).astype(np.float32)
        x = rng.standard_normal((N, K)).astype(np.float32)
        r = rng.standard_normal((N, M)).astype(np.float32)
        r[0, :2] = [0.0, -1.5]
        acc = dev(r)
        if mode == "lns32":
            want = O.add32(O.mul_mat32(w, x), r)
            wp, dx = ln.pack32(dev(w)), dev(x)
            ln.mul_mat32_raw(wp.data_ptr(), dx.data_ptr(), acc.data_ptr(), K, M, N, residual=acc.data_ptr())
        else:
            m = O.MODES[mode]
            O.monte_set(7)
            want = _elementwise16(O.lib().lno16_add, O.mul_mat16_f32w(m, w[None, None], x[None, None])[0, 0], r)
            wp, dx = ln.pack16(dev(w)), dev(x)
            ln.mul_mat16_raw(m, wp.data_ptr(), dx.data_ptr(), acc.data_ptr(), K, M, N, seed=7,
                             residual=acc.data_ptr())
        same_bits(host(acc), want, f"mul_mat residual {mode} K={K} M={M} N={N}")


@pytest.mark.parametrize("w32", [False, True], ids=["lns16", "lns32"])
def test_rope_store_kv_fused(ln, w32):
    # the fused launch writes exactly what rope + two store_kv launches write
    # (the decoder tests pin both against the oracle's graph), caches and q
    # included, with two sequences and positions out of order
    import ctypes
    rng = np.random.default_rng(35)
    L, st = ln.lib(), ln._stream()
    P = lambda t, off=0: ctypes.c_void_p(t.data_ptr() + off * t.element_size())
    T, nh, nkv, hd, n_ctx = 3, 4, 2, 16, 24
    nqkv = (nh + 2 * nkv) * hd
    qkv = dev((rng.standard_normal((T, nqkv)) * 2).astype(np.float32))
    pos = dev(np.array([5, 0, 17], np.int32))
    seq = dev(np.array([1, 0, 1], np.int32))
    rt = np.empty(n_ctx * hd, np.float32)
    ln.check(L.lnship_rope_table(ctypes.c_float(10000.0), hd, n_ctx, ctypes.c_void_p(rt.ctypes.data)))
    cs = dev(rt)
    kslice = ((hd + 7) // 8 * 8) * n_ctx
    vslice = kslice
    seq_stride = nkv * kslice
    dt = torch.int32 if w32 else torch.int16
    pre = "lnship32_" if w32 else "lnship16_"
    outs = []
    for fused in (False, True):
        kc = torch.full((2 * seq_stride,), 0x1234, dtype=dt, device="cuda")
        vc = torch.full((2 * seq_stride,), 0x1234, dtype=dt, device="cuda")
        q = torch.full((T * nh * hd,), 7.0, dtype=torch.float32, device="cuda")
        if fused:
            a = ln.QkvStoreArgs(P(qkv), nqkv, P(pos), T, nh, nkv, hd, hd, P(cs), P(q), P(kc), P(vc), n_ctx, kslice,
                                vslice, P(seq), seq_stride)
            ln.check(getattr(L, pre + "rope_store_kv")(ctypes.byref(a), st))
        else:
            ln.check(getattr(L, pre + "rope")(P(qkv), nqkv, P(pos), T, nh, hd, hd, 0, P(cs), P(q), st))
            ln.check(getattr(L, pre + "store_kv")(P(qkv, nh * hd), nqkv, P(pos), T, nkv, hd, hd, P(cs), P(kc), n_ctx,
                                                  kslice, 0, P(seq), seq_stride, st))
            ln.check(getattr(L, pre + "store_kv")(P(qkv, (nh + nkv) * hd), nqkv, P(pos), T, nkv, hd, 0, P(cs), P(vc),
                                                  n_ctx, vslice, 1, P(seq), seq_stride, st))
        outs.append((host(q), host(kc), host(vc)))
    for name, g, w in zip(("q", "k cache", "v cache"), outs[1], outs[0]):
        assert np.array_equal(g.view(np.uint32) if g.dtype == np.float32 else g,
                              w.view(np.uint32) if w.dtype == np.float32 else w), name


@pytest.mark.parametrize("w32", [False, True])
def test_rope_store_kv_position_out_of_range(ln, w32):
    # a position at or beyond the cache's n_ctx rows is reported as an index
    # error, and nothing is written for that token (no cache cell, no query
    # row); the other tokens are stored as usual
    import ctypes
    rng = np.random.default_rng(36)
    L, st = ln.lib(), ln._stream()
    P = lambda t, off=0: ctypes.c_void_p(t.data_ptr() + off * t.element_size())
    T, nh, nkv, hd, n_ctx = 3, 2, 1, 16, 16
    nqkv = (nh + 2 * nkv) * hd
    qkv = dev((rng.standard_normal((T, nqkv)) * 2).astype(np.float32))
    rt = np.empty(n_ctx * hd, np.float32)
    ln.check(L.lnship_rope_table(ctypes.c_float(10000.0), hd, n_ctx, ctypes.c_void_p(rt.ctypes.data)))
    cs = dev(rt)
    kslice = hd * n_ctx
    dt = torch.int32 if w32 else torch.int16
    pre = "lnship32_" if w32 else "lnship16_"
    bad = ctypes.c_int64(0)
    L.lnship_index_error(ctypes.byref(bad), st)   # clear
    outs = []
    for p_last in (7, n_ctx):
        pos = dev(np.array([2, 5, p_last], np.int32))
        kc = torch.full((kslice,), 0x1234, dtype=dt, device="cuda")
        vc = torch.full((kslice,), 0x1234, dtype=dt, device="cuda")
        q = torch.full((T * nh * hd,), 7.0, dtype=torch.float32, device="cuda")
        a = ln.QkvStoreArgs(P(qkv), nqkv, P(pos), T, nh, nkv, hd, hd, P(cs), P(q), P(kc), P(vc), n_ctx, kslice,
                            kslice, None, 0)
        ln.check(getattr(L, pre + "rope_store_kv")(ctypes.byref(a), st))
        outs.append((host(q).reshape(T, nh * hd), host(kc), host(vc)))
        if p_last == n_ctx:
            assert L.lnship_index_error(ctypes.byref(bad), st) == 1 and bad.value == n_ctx
        else:
            assert L.lnship_index_error(ctypes.byref(bad), st) == 0
    (q_ok, k_ok, v_ok), (q_bad, k_bad, v_bad) = outs
    assert np.array_equal(q_bad[:2].view(np.uint32), q_ok[:2].view(np.uint32))
    assert np.all(q_bad[2] == 7.0)                     # the refused token's query row untouched
    fill = 0x1234
    # the refused token wrote no cache cell: the caches equal the valid run's
    # with position 7's cells left at the fill value
    k_want, v_want = k_ok.copy(), v_ok.copy()
    for d in range(hd):
        k_want[((d >> 3) * n_ctx + 7) * 8 + (d & 7)] = fill
        v_want[((7 >> 3) * hd + d) * 8 + (7 & 7)] = fill
    assert np.array_equal(k_bad, k_want) and np.array_equal(v_bad, v_want)


# ------------------------------------------------------------------- softmax --

def _causal(nq, nkv):
    m = np.zeros((nq, nkv), np.float32)
    for i in range(nq):
        m[i, nkv - nq + i + 1:] = -np.inf
    return m


def _underflowing(rng):
    # rows whose exps are exactly zero (log 0) in the middle, at the end, or
    # everywhere but the maximum: the chain stops after the last nonzero one
    x = rng.standard_normal((6, 96)).astype(np.float32)
    x[0, 40:] = -1e4
    x[1, 10:50] = -1e4
    x[2, :] = -1e4
    x[2, 7] = 0.0
    x[3, ::3] = -3e4
    x[4, 95] = 50.0
    x[5, 0] = 50.0
    return x


@pytest.mark.parametrize("mode", MODES)
def test_soft_max(ln, mode):
    rng = np.random.default_rng(40)
    m = O.MODES[mode]
    cases = [
        ("c1 9x128x128", (rng.standard_normal((9, 128, 128)) * 3).astype(np.float32), None, 0.125),
        ("c1 causal", (rng.standard_normal((9, 128, 128)) * 3).astype(np.float32), _causal(128, 128), 0.125),
        ("300x3x2", rng.standard_normal((2, 3, 300)).astype(np.float32), None, 1.0),
        ("padded mask", rng.standard_normal((4, 5, 64)).astype(np.float32),
         np.where(rng.random((8, 64)) < 0.2, -np.inf, rng.standard_normal((8, 64))).astype(np.float32), 0.5),
        ("1100 wide", rng.standard_normal((3, 1100)).astype(np.float32), _causal(3, 1100), 1.0),
        ("singleton", rng.standard_normal((7, 1)).astype(np.float32), None, 1.0),
        ("underflow", _underflowing(rng), None, 1.0),
    ]
    for name, x, mask, scale in cases:
        print(f"\n[soft_max] {mode} {name}", flush=True)
        O.monte_set(7)
        want = O.soft_max16(m, x, mask, scale)
        got = host(ln.soft_max16(m, dev(x), dev(mask) if mask is not None else None, scale, seed=7))
        same_bits(got, want, f"soft_max {mode} {name}")


def test_soft_max_lns32(ln):
    rng = np.random.default_rng(41)
    x = (rng.standard_normal((3, 16, 128)) * 3).astype(np.float32)
    mask = _causal(16, 128)
    same_bits(host(ln.soft_max32(dev(x), dev(mask), 0.125)), O.soft_max32(x, mask, 0.125), "soft_max lns32")
    same_bits(host(ln.soft_max32(dev(x), None, 1.0)), O.soft_max32(x, None, 1.0), "soft_max lns32 unmasked")
    u = _underflowing(rng)
    same_bits(host(ln.soft_max32(dev(u), None, 1.0)), O.soft_max32(u, None, 1.0), "soft_max lns32 underflow")


# ------------------------------------------------- LNS32 elementwise ops --

def test_elementwise_lns32(ln):
    import ctypes
    L = ln.lib()
    st = ln._stream()
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    rng = np.random.default_rng(41)
    a = (rng.standard_normal((37, 24)) * 3).astype(np.float32)
    b = rng.standard_normal(24).astype(np.float32)
    a[0, :4] = [0.0, -0.0, 1e-30, -7.5]
    b[:4] = [0.0, 2.0, -1e-30, 7.5]                   # zeros, tiny, exact cancellation
    da, db = dev(a), dev(b)
    for name, fn in (("add", O.add32), ("mul", O.mul32)):
        print(f"\n[lns32 {name}]", flush=True)
        out = torch.empty_like(da)
        ln.check(getattr(L, "lnship32_" + name)(P(da), P(db), a.size, b.size, P(out), st))
        same_bits(host(out), fn(a, b), f"lns32 {name}")
    print("[lns32 swiglu]", flush=True)
    g = (rng.standard_normal((5, 2 * 40)) * 4).astype(np.float32)
    g[0, :3] = [0.0, 90.0, -90.0]
    dg = dev(g)
    out = torch.empty((5, 40), dtype=torch.float32, device="cuda")
    ln.check(L.lnship32_swiglu(ctypes.c_void_p(dg.data_ptr() + 40 * 4), 80, P(dg), 80, P(out), 40, 5, st))
    same_bits(host(out), O.swiglu32(g[:, 40:], g[:, :40]), "lns32 swiglu")
    for neox, n_dims in ((0, 16), (1, 16), (0, 10)):
        print(f"[lns32 rope] neox={neox} n_dims={n_dims}", flush=True)
        x = rng.standard_normal((3, 4, 16)).astype(np.float32)
        pos = np.array([0, 7, 300], np.int32)
        cs = np.empty(512 * n_dims, np.float32)
        ln.check(L.lnship_rope_table(10000.0, n_dims, 512, ctypes.c_void_p(cs.ctypes.data)))
        dx, dpos, dcs = dev(x), dev(pos), dev(cs)
        out = torch.empty_like(dx)
        ln.check(L.lnship32_rope(P(dx), 64, P(dpos), 3, 4, 16, n_dims, neox, P(dcs), P(out), st))
        same_bits(host(out), O.rope32(x, pos, n_dims, neox, 10000.0), f"lns32 rope neox={neox} n_dims={n_dims}")


# ---------------------------------------- SCALE and data movement (C ABI) --

def test_scale_both_formats(ln):
    import ctypes
    L, st = ln.lib(), ln._stream()
    rng = np.random.default_rng(61)
    x = (rng.standard_normal(1 << 20) * 5).astype(np.float32)
    x[:4] = [0.0, -0.0, 1e-30, -3e38]
    for w32, fn in ((False, L.lnship16_scale), (True, L.lnship32_scale)):
        for s, b in ((0.125, 0.0), (-1.5, 0.25), (3.0, -7.0)):
            print(f"\n[scale] w32={w32} s={s} b={b}", flush=True)
            xd, yd = dev(x), torch.empty(x.size, dtype=torch.float32, device="cuda")
            ln.check(fn(ctypes.c_void_p(xd.data_ptr()), ctypes.c_void_p(yd.data_ptr()), x.size, s, b, st))
            same_bits(host(yd), O.scale(w32, x, s, b), f"scale w32={w32} s={s} b={b}")


def test_row_index_out_of_range_is_reported(ln):
    # a bad index leaves its row unwritten and is reported once; the good rows land
    import ctypes
    L, st = ln.lib(), ln._stream()
    V = lambda *v: (ctypes.c_int64 * len(v))(*v)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    tab = dev(np.arange(40, dtype=np.float32).reshape(10, 4))
    ids = dev(np.array([3, 10, 0], np.int32))
    out = torch.full((3, 4), -1.0, dtype=torch.float32, device="cuda")
    print("\n[get_rows] index 10 of 10 rows", flush=True)
    ln.check(L.lnship_get_rows(P(tab), 0, V(4, 10, 1, 1), V(4, 16, 160, 160), P(ids), V(3, 1, 1), V(4, 12, 12),
                               P(out), V(4, 16, 48, 48), st))
    bad = ctypes.c_int64()
    assert L.lnship_index_error(ctypes.byref(bad), st) == 1 and bad.value == 10
    assert L.lnship_index_error(ctypes.byref(bad), st) == 0
    got = host(out)
    assert np.array_equal(got[0], np.arange(12, 16)) and np.array_equal(got[2], np.arange(4))
    assert np.all(got[1] == -1.0)
    print("[set_rows] index -1", flush=True)
    src = dev(np.ones((2, 4), np.float32))
    ids64 = dev(np.array([-1, 9], np.int64))
    dst = torch.zeros((10, 4), dtype=torch.float16, device="cuda")
    ln.check(L.lnship_set_rows(P(src), V(4, 2, 1, 1), V(4, 16, 32, 32), P(ids64), 1, V(2, 1, 1), V(8, 16, 16),
                               P(dst), 1, V(4, 10, 1, 1), V(2, 8, 80, 80), st))
    assert L.lnship_index_error(ctypes.byref(bad), st) == 1 and bad.value == -1
    d = host(dst).astype(np.float32)
    assert np.all(d[9] == 1.0) and np.all(d[:9] == 0.0)


# ------------------------------------------------------------ MUL_MAT_ID --

MM_ID_CASES = [
    # (n_expert, M, K, T, n_expert_used, ne11): decode, prefill with the
    # activation broadcast over slots, a K tail and one row per workgroup edge
    (8, 1536, 576, 1, 2, 1),
    (8, 256, 576, 9, 4, 1),
    (4, 70, 13, 5, 4, 2),
    (16, 65, 1024, 2, 8, 8),
]


@pytest.mark.parametrize("mode", MODES + ["lns32"])
def test_mul_mat_id(ln, mode):
    m = None if mode == "lns32" else O.MODES[mode]
    for E, M, K, T, neu, ne11 in MM_ID_CASES:
        print(f"\n[mul_mat_id] {mode} experts={E} M={M} K={K} T={T} used={neu} ne11={ne11}", flush=True)
        rng = np.random.default_rng(E * 1000 + M + K)
        w = (rng.standard_normal((E, M, K)) * 0.05).astype(np.float32)
        x = rng.standard_normal((T, ne11, K)).astype(np.float32)
        ids = rng.integers(0, E, (T, neu)).astype(np.int32)
        O.monte_set(7)
        want = O.mul_mat_id(m, w, x, ids)
        wp = ln.pack32(dev(w)) if m is None else ln.pack16(dev(w))
        got = host(ln.mul_mat_id(m, wp, dev(x), dev(ids), K, M, E, seed=7))
        same_bits(got, want, f"mul_mat_id {mode} E={E} M={M} K={K}")
        if m == O.MONTE:
            assert O.monte_get() == O.lib().lno_lfsr_jump(7, ln.lib().lnship16_mul_mat_id_draws(m, K, M, neu, T))


def test_mul_mat_id_expert_out_of_range(ln):
    import ctypes
    w = np.ones((3, 64, 16), np.float32)
    x = np.ones((2, 1, 16), np.float32)
    ids = np.array([[0, 3], [2, 1]], np.int32)
    print("\n[mul_mat_id] expert 3 of 3", flush=True)
    out = torch.full((2, 2, 64), -1.0, dtype=torch.float32, device="cuda")
    ln.mul_mat_id(O.SUM32, ln.pack16(dev(w)), dev(x), dev(ids), 16, 64, 3, out=out)
    bad = ctypes.c_int64()
    assert ln.lib().lnship_index_error(ctypes.byref(bad), ln._stream()) == 1 and bad.value == 3
    got = host(out)
    want = O.mul_mat_id(O.SUM32, w, x, np.array([[0, 0], [2, 1]], np.int32))
    assert np.all(got[0, 1] == -1.0)
    same_bits(got[0, 0], want[0, 0], "slot before the bad expert")
    same_bits(got[1], want[1], "token after the bad expert")


@pytest.mark.parametrize("mode,n_kv,big_tail,skew,hd", [
    ("base", 1, False, 0, 64), ("base", 13, False, 0, 64), ("base", 256, False, 0, 64), ("base", 256, True, 0, 64),
    ("lpvip", 13, False, 0, 64), ("lpvip", 256, False, 0, 64), ("lpvip", 256, True, 0, 64), ("sum32", 1, False, 0, 64),
    ("sum32", 13, False, 0, 64), ("sum32", 256, False, 0, 64), ("sum32", 256, True, 0, 64), ("sum32", 520, False, 0, 64),
    ("sum32", 2048, False, 0, 64), ("sum32", 1, False, 1, 64), ("sum32", 13, False, -1, 64),
    ("sum32", 256, True, 3, 64), ("sum32", 520, False, -7, 64),
    # head dims off the group of eight: the score chains end inside a group
    ("sum32", 13, False, 0, 36), ("sum32", 200, False, 0, 72), ("sum32", 77, True, 2, 100),
    ("base", 200, False, 0, 72)])
def test_attn_decode_equals_three_nodes(ln, mode, n_kv, big_tail, skew, hd):
    # lnship16_attn_decode against K^T q, soft_max and V p run as three ops
    # (the library's own launches, and the oracle's), on
    # the SmolLM2 head shape (9 query heads over 3 kv heads of 64), random
    # caches and a causal mask that hides the last cells.  Past the last
    # nonzero exp the KQV chain stops only where the remaining products add
    # nothing; big_tail puts values of 1e35 in the masked cells of V, so that
    # they would not and the chain runs on.  sum32 starts the KQV chains from
    # a predicted soft_max total; skew makes that prediction wrong, so the
    # result comes from the rerun
    import ctypes
    m = O.MODES[mode]
    nh, nkv, n_ctx = 9, 3, max(256, (n_kv + 255) // 256 * 256)
    rng = np.random.default_rng(n_kv)
    print(f"\n[attn decode] {mode} n_kv={n_kv} big_tail={big_tail} skew={skew} head_dim={hd}", flush=True)
    pos = max(0, n_kv - 1 - n_kv // 5)
    v = (rng.standard_normal((nkv, hd, n_ctx)) * 0.5).astype(np.float32)
    if big_tail:
        v[:, :, pos + 1:n_kv] *= np.float32(1e35)
    kf = (rng.standard_normal((nkv, n_ctx, hd)) * 0.5).astype(np.float32)
    kc = ln.pack16(dev(kf))
    vc = ln.pack16(dev(v))
    kslice, vslice = ln.kp(hd) * n_ctx, ln.kp(n_ctx) * hd
    qf = (rng.standard_normal(nh * hd) * 2).astype(np.float32)
    maskf = np.where(np.arange(n_kv) <= pos, 0.0, -np.inf).astype(np.float32)
    q = dev(qf)
    mask = dev(maskf)
    scale = 0.125
    P = lambda t: t.data_ptr()
    kq = torch.empty(nh * n_kv, device="cuda")
    ln.mul_mat16_raw(m, P(kc), P(q), P(kq), hd, n_kv, 1, ne02=nkv, ne12=nh, x_ld=nh * hd, x_slice=hd,
                     w_mstride=n_ctx, w_slice=kslice)
    p = ln.soft_max16(m, kq.view(1, nh, 1, n_kv), mask.view(1, 1, 1, n_kv), scale)
    want = torch.empty(nh * hd, device="cuda")
    ln.mul_mat16_raw(m, P(vc), P(p), P(want), n_kv, hd, 1, ne02=nkv, ne12=nh, x_ld=n_kv, x_slice=n_kv,
                     w_slice=vslice, dst_ld=nh * hd, dst_slice=hd)
    got = torch.full((nh * hd,), float("nan"), device="cuda")
    a = ln.AttnArgs(P(q), P(kc), P(vc), n_ctx, kslice, vslice, P(mask), scale, P(got), nh, nkv, hd, n_kv)
    prev = ln.lib().lnship_test_predict_skew(skew)
    try:
        ln.check(ln.lib().lnship16_attn_decode(m, ctypes.byref(a), ln._stream()))
    finally:
        ln.lib().lnship_test_predict_skew(prev)
    same_bits(host(got), host(want), f"attn decode {mode} n_kv={n_kv} skew={skew}")
    # and against the oracle's three ops: the GQA kq product (query head h on
    # kv head h / 3), the masked soft_max, then the kqv product
    kq_o = O.mul_mat16_f32w(m, kf[None, :, :n_kv], qf.reshape(1, nh, 1, hd), ne02=nkv)[0]
    p_o = O.soft_max16(m, kq_o, maskf[None], scale)
    want_o = O.mul_mat16_f32w(m, v[None, :, :, :n_kv], p_o[None], ne02=nkv)[0]
    same_bits(host(got), want_o.reshape(-1), f"attn decode {mode} n_kv={n_kv} skew={skew} vs oracle")
    if mode == "sum32" and n_kv == 13 and not big_tail:
        # Monte is refused (its draws run across the three nodes in graph order)
        assert ln.lib().lnship16_attn_decode(O.MONTE, ctypes.byref(a), ln._stream()) != 0
        assert ln.lib().lnship_max_row(4, O.MONTE) == 0 and ln.lib().lnship_max_row(4, m) >= 4096


@pytest.mark.parametrize("mode,nseq,n_kv,hd,big_tail", [
    ("monte", 1, 13, 64, False), ("monte", 1, 256, 64, False), ("monte", 3, 256, 64, False), ("monte", 8, 512, 64, False),
    ("monte", 3, 200, 72, True), ("base", 3, 256, 64, False), ("base", 8, 512, 64, True), ("lpvip", 3, 256, 64, False),
    ("lpvip", 8, 320, 64, False), ("sum32", 3, 256, 64, True), ("sum32", 8, 512, 64, False), ("sum32", 2, 77, 36, False)])
def test_attn_decode_seqs_equals_three_nodes(ln, mode, nseq, n_kv, hd, big_tail):
    # lnship16_attn_decode_seqs against the batched decode step's three ops:
    # K^T q with ggml's 4-D broadcast (sequence s on its own caches), the
    # masked soft_max and V p, the library's own launches, each with its own
    # Monte start; sequences at different positions (each its own mask row).
    # Monte runs twice: with the three starts as seeds, and read from a
    # device state with offsets (as in a captured graph).  big_tail puts
    # values of 1e35 in V past a sequence's last position, where the KQV
    # chain may not stop
    import ctypes
    m = O.MODES[mode]
    nh, nkv, n_ctx = 9, 3, max(256, (n_kv + 255) // 256 * 256)
    rng = np.random.default_rng(7000 + 10 * nseq + n_kv + hd)
    print(f"\n[attn decode seqs] {mode} n_seq={nseq} n_kv={n_kv} head_dim={hd} big_tail={big_tail}", flush=True)
    L, P = ln.lib(), (lambda t: t.data_ptr())
    pos = [int(x) for x in rng.integers(max(0, n_kv // 3), n_kv, nseq)]
    pos[0] = n_kv - 1
    v = (rng.standard_normal((nseq, nkv, hd, n_ctx)) * 0.5).astype(np.float32)
    if big_tail:
        for s in range(nseq):
            v[s, :, :, pos[s] + 1:n_kv] *= np.float32(1e35)
    kf = (rng.standard_normal((nseq, nkv, n_ctx, hd)) * 0.5).astype(np.float32)
    kc = ln.pack16(dev(kf.reshape(nseq * nkv, n_ctx, hd)))
    vc = ln.pack16(dev(v.reshape(nseq * nkv, hd, n_ctx)))
    kslice, vslice = ln.kp(hd) * n_ctx, ln.kp(n_ctx) * hd
    q = dev((rng.standard_normal(nseq * nh * hd) * 2).astype(np.float32))
    maskf = np.where(np.arange(n_kv)[None, :] <= np.array(pos)[:, None], 0.0, -np.inf).astype(np.float32)
    mask = dev(maskf)
    scale = 0.125
    d_kq = L.lnship16_mul_mat_draws(m, hd, n_kv, 1, nh, nseq)
    d_sm = L.lnship16_soft_max_draws(m, n_kv, nh * nseq)
    s0 = 4242
    s1 = L.lnship_lfsr_jump(s0, d_kq)
    s2 = L.lnship_lfsr_jump(s1, d_sm)
    kq = torch.empty(nseq * nh * n_kv, device="cuda")
    ln.mul_mat16_raw(m, P(kc), P(q), P(kq), hd, n_kv, 1, ne02=nkv, ne03=nseq, ne12=nh, ne13=nseq, x_ld=nh * hd,
                     x_slice=hd, seed=s0, w_mstride=n_ctx, w_slice=kslice)
    p = ln.soft_max16(m, kq.view(nseq, nh, 1, n_kv), mask.view(nseq, 1, 1, n_kv), scale, seed=s1)
    want = torch.empty(nseq * nh * hd, device="cuda")
    ln.mul_mat16_raw(m, P(vc), P(p), P(want), n_kv, hd, 1, ne02=nkv, ne03=nseq, ne12=nh, ne13=nseq, x_ld=n_kv,
                     x_slice=n_kv, seed=s2, w_slice=vslice, dst_ld=nh * hd, dst_slice=hd)
    a_args = lambda out: ln.AttnArgs(P(q), P(kc), P(vc), n_ctx, kslice, vslice, P(mask), scale, P(out), nh, nkv, hd,
                                     n_kv)
    got = torch.full((nseq * nh * hd,), float("nan"), device="cuda")
    sq = ln.attn_seqs(nseq, (s0, s1, s2))
    ln.check(L.lnship16_attn_decode_seqs(m, ctypes.byref(a_args(got)), ctypes.byref(sq), ln._stream()))
    same_bits(host(got), host(want), f"attn decode seqs {mode} n_seq={nseq} n_kv={n_kv}")
    if mode == "monte":
        # the starts read on the device: state S, offsets 0, d_kq, d_kq + d_sm
        S = 911
        st = torch.tensor([S], dtype=torch.int16, device="cuda")
        got2 = torch.full((nseq * nh * hd,), float("nan"), device="cuda")
        sq2 = ln.attn_seqs(nseq, ((st, 0), (st, d_kq), (st, d_kq + d_sm)))
        ln.check(L.lnship16_attn_decode_seqs(m, ctypes.byref(a_args(got2)), ctypes.byref(sq2), ln._stream()))
        got3 = torch.full((nseq * nh * hd,), float("nan"), device="cuda")
        sq3 = ln.attn_seqs(nseq, (S, L.lnship_lfsr_jump(S, d_kq), L.lnship_lfsr_jump(S, d_kq + d_sm)))
        ln.check(L.lnship16_attn_decode_seqs(m, ctypes.byref(a_args(got3)), ctypes.byref(sq3), ln._stream()))
        same_bits(host(got2), host(got3), f"attn decode seqs monte n_seq={nseq} n_kv={n_kv}: state vs seeds")
        assert not np.array_equal(host(got3), host(got)), "other starts, other draws"


@pytest.mark.parametrize("mode,n_kv,nd,hd,pos", [
    ("sum32", 1, 64, 64, 0), ("sum32", 13, 64, 64, 12), ("sum32", 256, 64, 64, 200), ("sum32", 520, 64, 64, 517),
    ("sum32", 200, 32, 64, 150), ("sum32", 77, 72, 72, 60), ("base", 256, 64, 64, 200), ("lpvip", 13, 64, 64, 9),
    ("sum32", 256, 64, 64, 300)])
def test_rope_attn_decode_equals_two_launches(ln, mode, n_kv, nd, hd, pos):
    # lnship16_rope_attn_decode against lnship16_rope_store_kv (one token)
    # then lnship16_attn_decode: the attention output and both whole caches
    # bit for bit, on the SmolLM2 head counts with random caches, a causal
    # mask and partial rotations (nd < hd); at pos 300 with n_kv 256 the new
    # cell lies past the attended cells (it is stored, not read)
    import ctypes
    rng = np.random.default_rng(1000 + n_kv + pos)
    L, st = ln.lib(), ln._stream()
    m = O.MODES[mode]
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    nh, nkv, n_ctx = 9, 3, 768
    print(f"\n[rope attn decode] {mode} n_kv={n_kv} rope dims={nd} head_dim={hd} pos={pos}", flush=True)
    nqkv = (nh + 2 * nkv) * hd
    qkv = dev((rng.standard_normal(nqkv) * 2).astype(np.float32))
    rt = np.empty(n_ctx * nd, np.float32)
    ln.check(L.lnship_rope_table(ctypes.c_float(10000.0), nd, n_ctx, ctypes.c_void_p(rt.ctypes.data)))
    cs = dev(rt)
    posd = dev(np.array([pos], np.int32))
    kf = (rng.standard_normal((nkv, n_ctx, hd)) * 0.5).astype(np.float32)
    vf = (rng.standard_normal((nkv, hd, n_ctx)) * 0.5).astype(np.float32)
    kslice, vslice = ln.kp(hd) * n_ctx, ln.kp(n_ctx) * hd
    maskf = np.where(np.arange(n_kv) <= pos, 0.0, -np.inf).astype(np.float32)
    mask = dev(maskf)
    outs = []
    for fused in (False, True):
        kc, vc = ln.pack16(dev(kf)), ln.pack16(dev(vf))
        q = torch.full((nh * hd,), 7.0, dtype=torch.float32, device="cuda")
        got = torch.full((nh * hd,), float("nan"), device="cuda")
        qs = ln.QkvStoreArgs(P(qkv), nqkv, P(posd), 1, nh, nkv, hd, nd, P(cs), P(q), P(kc), P(vc), n_ctx, kslice,
                             vslice, None, 0)
        a = ln.AttnArgs(P(q), P(kc), P(vc), n_ctx, kslice, vslice, P(mask), 0.125, P(got), nh, nkv, hd, n_kv)
        if fused:
            ln.check(L.lnship16_rope_attn_decode(m, ctypes.byref(qs), ctypes.byref(a), st))
        else:
            ln.check(L.lnship16_rope_store_kv(ctypes.byref(qs), st))
            ln.check(L.lnship16_attn_decode(m, ctypes.byref(a), st))
        outs.append((host(got), host(kc), host(vc)))
    (w_att, w_k, w_v), (g_att, g_k, g_v) = outs
    assert np.array_equal(g_k, w_k) and np.array_equal(g_v, w_v), "caches"
    same_bits(g_att, w_att, f"rope attn decode {mode} n_kv={n_kv}")


@pytest.mark.parametrize("mode,nseq,n_kv,nd,hd", [
    ("monte", 1, 256, 64, 64), ("monte", 8, 512, 64, 64), ("monte", 3, 77, 32, 64), ("base", 3, 256, 64, 64),
    ("lpvip", 8, 320, 64, 64), ("sum32", 8, 512, 64, 64), ("sum32", 2, 60, 72, 72)])
def test_rope_attn_decode_seqs_equals_two_launches(ln, mode, nseq, n_kv, nd, hd):
    # lnship16_rope_attn_decode_seqs against lnship16_rope_store_kv (one token
    # per sequence, seq = 0..n_seq-1) then lnship16_attn_decode_seqs with the
    # same Monte starts: the attention output and both whole caches bit for
    # bit; the sequences at different positions (the first past the attended
    # cells: stored, not read), qkv rows wider than the heads
    import ctypes
    rng = np.random.default_rng(2000 + 10 * nseq + n_kv + nd)
    L, st = ln.lib(), ln._stream()
    m = O.MODES[mode]
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    nh, nkv, n_ctx = 9, 3, 768
    print(f"\n[rope attn decode seqs] {mode} n_seq={nseq} n_kv={n_kv} rope dims={nd} head_dim={hd}", flush=True)
    nqkv = (nh + 2 * nkv) * hd
    ld = nqkv + 8
    qkv = dev((rng.standard_normal(nseq * ld) * 2).astype(np.float32))
    rt = np.empty(n_ctx * nd, np.float32)
    ln.check(L.lnship_rope_table(ctypes.c_float(10000.0), nd, n_ctx, ctypes.c_void_p(rt.ctypes.data)))
    cs = dev(rt)
    pos = [int(x) for x in rng.integers(max(0, n_kv // 3), n_kv, nseq)]
    pos[0] = n_kv + 5
    posd = dev(np.array(pos, np.int32))
    seq_ids = torch.arange(nseq, dtype=torch.int32, device="cuda")
    kf = (rng.standard_normal((nseq * nkv, n_ctx, hd)) * 0.5).astype(np.float32)
    vf = (rng.standard_normal((nseq * nkv, hd, n_ctx)) * 0.5).astype(np.float32)
    kslice, vslice = ln.kp(hd) * n_ctx, ln.kp(n_ctx) * hd
    maskf = np.where(np.arange(n_kv)[None, :] <= np.array(pos)[:, None], 0.0, -np.inf).astype(np.float32)
    mask = dev(maskf)
    seeds = (4242, 999, 31337)
    outs = []
    for fused in (False, True):
        kc, vc = ln.pack16(dev(kf)), ln.pack16(dev(vf))
        q = torch.full((nseq * nh * hd,), 7.0, dtype=torch.float32, device="cuda")
        got = torch.full((nseq * nh * hd,), float("nan"), device="cuda")
        qs = ln.QkvStoreArgs(P(qkv), ld, P(posd), nseq, nh, nkv, hd, nd, P(cs), P(q), P(kc), P(vc), n_ctx, kslice,
                             vslice, None if fused else P(seq_ids), nkv * kslice)
        a = ln.AttnArgs(P(q), P(kc), P(vc), n_ctx, kslice, vslice, P(mask), 0.125, P(got), nh, nkv, hd, n_kv)
        sq = ln.attn_seqs(nseq, seeds)
        if fused:
            ln.check(L.lnship16_rope_attn_decode_seqs(m, ctypes.byref(qs), ctypes.byref(a), ctypes.byref(sq), st))
        else:
            ln.check(L.lnship16_rope_store_kv(ctypes.byref(qs), st))
            ln.check(L.lnship16_attn_decode_seqs(m, ctypes.byref(a), ctypes.byref(sq), st))
        outs.append((host(got), host(kc), host(vc)))
    (w_att, w_k, w_v), (g_att, g_k, g_v) = outs
    assert np.array_equal(g_k, w_k) and np.array_equal(g_v, w_v), "caches"
    assert not np.array_equal(g_k, host(ln.pack16(dev(kf)))), "the cells were stored"
    same_bits(g_att, w_att, f"rope attn decode seqs {mode} n_seq={nseq} n_kv={n_kv}")


def test_rope_attn_decode_seqs_position_out_of_range(ln):
    # a sequence at a position at or beyond the cache is recorded as an index
    # error; its caches and dst rows are left alone, the other sequence runs
    import ctypes
    L, st = ln.lib(), ln._stream()
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    nh, nkv, hd, n_ctx, n_kv, nseq = 2, 1, 16, 16, 8, 2
    nqkv = (nh + 2 * nkv) * hd
    qkv = dev(np.ones(nseq * nqkv, np.float32))
    rt = np.empty(n_ctx * hd, np.float32)
    ln.check(L.lnship_rope_table(ctypes.c_float(10000.0), hd, n_ctx, ctypes.c_void_p(rt.ctypes.data)))
    cs = dev(rt)
    posd = dev(np.array([3, n_ctx], np.int32))
    kc = torch.full((nseq * hd * n_ctx,), 0x1234, dtype=torch.int16, device="cuda")
    vc = torch.full((nseq * hd * n_ctx,), 0x1234, dtype=torch.int16, device="cuda")
    got = torch.full((nseq * nh * hd,), 7.0, device="cuda")
    mask = dev(np.zeros(nseq * n_kv, np.float32))
    bad = ctypes.c_int64(0)
    L.lnship_index_error(ctypes.byref(bad), st)   # clear
    qs = ln.QkvStoreArgs(P(qkv), nqkv, P(posd), nseq, nh, nkv, hd, hd, P(cs), None, P(kc), P(vc), n_ctx, hd * n_ctx,
                         hd * n_ctx, None, hd * n_ctx)
    a = ln.AttnArgs(None, P(kc), P(vc), n_ctx, hd * n_ctx, hd * n_ctx, P(mask), 0.25, P(got), nh, nkv, hd, n_kv)
    sq = ln.attn_seqs(nseq)
    ln.check(L.lnship16_rope_attn_decode_seqs(O.SUM32, ctypes.byref(qs), ctypes.byref(a), ctypes.byref(sq), st))
    assert L.lnship_index_error(ctypes.byref(bad), st) == 1 and bad.value == n_ctx
    k, v, g = host(kc), host(vc), host(got)
    assert np.all(k[hd * n_ctx:] == 0x1234) and np.all(v[hd * n_ctx:] == 0x1234) and np.all(g[nh * hd:] == 7.0)
    assert np.any(k[:hd * n_ctx] != 0x1234) and np.all(np.isfinite(g[:nh * hd])) and np.any(g[:nh * hd] != 7.0)


def test_rope_attn_decode_position_out_of_range(ln):
    # a position at or beyond the cache is recorded as an index error, and
    # neither the caches nor dst are written
    import ctypes
    L, st = ln.lib(), ln._stream()
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    nh, nkv, hd, n_ctx, n_kv = 2, 1, 16, 16, 8
    nqkv = (nh + 2 * nkv) * hd
    qkv = dev(np.ones(nqkv, np.float32))
    rt = np.empty(n_ctx * hd, np.float32)
    ln.check(L.lnship_rope_table(ctypes.c_float(10000.0), hd, n_ctx, ctypes.c_void_p(rt.ctypes.data)))
    cs = dev(rt)
    posd = dev(np.array([n_ctx], np.int32))
    kc = torch.full((hd * n_ctx,), 0x1234, dtype=torch.int16, device="cuda")
    vc = torch.full((hd * n_ctx,), 0x1234, dtype=torch.int16, device="cuda")
    got = torch.full((nh * hd,), 7.0, device="cuda")
    bad = ctypes.c_int64(0)
    L.lnship_index_error(ctypes.byref(bad), st)   # clear
    qs = ln.QkvStoreArgs(P(qkv), nqkv, P(posd), 1, nh, nkv, hd, hd, P(cs), None, P(kc), P(vc), n_ctx, hd * n_ctx,
                         hd * n_ctx, None, 0)
    a = ln.AttnArgs(None, P(kc), P(vc), n_ctx, hd * n_ctx, hd * n_ctx, None, 0.25, P(got), nh, nkv, hd, n_kv)
    ln.check(L.lnship16_rope_attn_decode(O.SUM32, ctypes.byref(qs), ctypes.byref(a), st))
    assert L.lnship_index_error(ctypes.byref(bad), st) == 1 and bad.value == n_ctx
    assert np.all(host(kc) == 0x1234) and np.all(host(vc) == 0x1234) and np.all(host(got) == 7.0)


@pytest.mark.parametrize("n_kv,masked,big_tail,hd", [
    (1, False, False, 64), (13, True, False, 64), (256, True, False, 64), (256, True, True, 64),
    (520, True, False, 64), (768, True, False, 64), (1024, False, False, 64), (1024, True, False, 64),
    (200, True, False, 128), (13, True, False, 36), (200, True, True, 72)])
def test_attn32_decode_equals_three_nodes(ln, n_kv, masked, big_tail, hd):
    # lnship32_attn_decode (LNS32) against kq, soft_max and kqv run as three
    # ops, the library's launches and the oracle's, on the Llama-1B head
    # geometry (32 query heads over 8 kv heads), random xlns32 caches and a
    # causal mask that hides the last cells; big_tail puts values of 1e35 in
    # the masked cells of V (their products still run through the chain)
    import ctypes
    nh, nkv, n_ctx = 32, 8, max(256, (n_kv + 255) // 256 * 256)
    rng = np.random.default_rng(n_kv + hd)
    print(f"\n[attn32 decode] n_kv={n_kv} masked={masked} big_tail={big_tail} hd={hd}", flush=True)
    pos = max(0, n_kv - 1 - n_kv // 5) if masked else n_kv - 1
    kf = (rng.standard_normal((nkv, n_ctx, hd)) * 0.5).astype(np.float32)
    vf = (rng.standard_normal((nkv, hd, n_ctx)) * 0.5).astype(np.float32)
    if big_tail:
        vf[:, :, pos + 1:n_kv] *= np.float32(1e35)
    kc, vc = ln.pack32(dev(kf)), ln.pack32(dev(vf))
    kslice, vslice = ln.kp(hd) * n_ctx, ln.kp(n_ctx) * hd
    qf = (rng.standard_normal(nh * hd) * 2).astype(np.float32)
    maskf = np.where(np.arange(n_kv) <= pos, 0.0, -np.inf).astype(np.float32)
    q, mask = dev(qf), dev(maskf)
    scale = 0.125
    P = lambda t: t.data_ptr()
    kq = torch.empty(nh * n_kv, device="cuda")
    ln.mul_mat32_raw(P(kc), P(q), P(kq), hd, n_kv, 1, ne02=nkv, ne12=nh, x_ld=nh * hd, x_slice=hd,
                     w_mstride=n_ctx, w_slice=kslice)
    p = ln.soft_max32(kq.view(1, nh, 1, n_kv), mask.view(1, 1, 1, n_kv), scale)
    want = torch.empty(nh * hd, device="cuda")
    ln.mul_mat32_raw(P(vc), P(p), P(want), n_kv, hd, 1, ne02=nkv, ne12=nh, x_ld=n_kv, x_slice=n_kv,
                     w_slice=vslice, dst_ld=nh * hd, dst_slice=hd)
    got = torch.full((nh * hd,), float("nan"), device="cuda")
    a = ln.AttnArgs(P(q), P(kc), P(vc), n_ctx, kslice, vslice, P(mask), scale, P(got), nh, nkv, hd, n_kv)
    ln.check(ln.lib().lnship32_attn_decode(ctypes.byref(a), ln._stream()))
    same_bits(host(got), host(want), f"attn32 decode n_kv={n_kv}")
    kq_o = O.mul_mat32(kf[None, :, :n_kv], qf.reshape(1, nh, 1, hd), ne02=nkv)[0]
    p_o = O.soft_max32(kq_o, maskf[None], scale)
    want_o = O.mul_mat32(vf[None, :, :, :n_kv], p_o[None], ne02=nkv)[0]
    same_bits(host(got), want_o.reshape(-1), f"attn32 decode n_kv={n_kv} vs oracle")
    assert ln.lib().lnship_max_row(7, 0) >= 2048


def test_lpvip_db_every_distance_below_one_binade(ln):
    # lpvip's exact branch (d below one binade, opposite signs) against the
    # host's libm for every d, and the Mitchell branch just above it (d = 0
    # is exact cancellation, handled before db)
    import ctypes
    n = (1 << 23) + (1 << 20)
    print(f"\n[lpvip db] d = 1 .. {n}", flush=True)
    out = torch.empty(n, dtype=torch.int32, device="cuda")
    ln.check(ln.lib().lnship_lpvip_db_range(1, n, ctypes.c_void_p(out.data_ptr()), ln._stream()))
    want = np.empty(n, np.int32)
    O.lib().lno32_lpvip_db_n(1, n, want.ctypes.data)
    got = host(out)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} differ; first d={bad[0] + 1}: got {got[bad[0]]} want {want[bad[0]]}"
