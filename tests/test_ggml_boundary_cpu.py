"""CPU checks of the ggml boundary (libggml-lnship.so) through a test-only
ggml host: struct layout, the registry / device / backend vtables, the op
predicates with their audit reasons, the environment controls and the Monte
state API.  Nothing here needs a GPU; each environment case runs in a fresh
interpreter because the backend reads its environment once per process.

Reference behaviour mirrored: lns-backend/common/lns-backend-framework.h
(vtables, check, audit), common/lns-op-support.h (predicates),
common/lns-backend-config.h (GGML_LNS_BACKEND, LNS_DISABLE_OPS,
LNS_ENABLE_OPS, LNS_OP_AUDIT), cuda/lns-cuda-ops.cpp (the GPU backend's extra
predicates), include/ggml-lns.h (Monte state).
"""
import ctypes
import json
import os
import subprocess
import sys
import textwrap

import numpy as np
import pytest

import ggml_host as G
import oracle_lib as O

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def host():
    if not os.path.exists(G.BACKEND_SO):
        pytest.fail("libggml-lnship.so is not built (run __graft_entry__.build())")
    return G.Host()


def test_tensor_layout_matches_ggml(host):
    # sizeof(struct ggml_tensor) is 336 on LP64 (ggml's GGML_TENSOR_SIZE)
    assert host.stub.ggml_host_sizeof_tensor() == 336 == ctypes.sizeof(G.Tensor)
    assert host.stub.ggml_host_offsetof_src() == 152 == G.Tensor.src.offset
    assert host.stub.ggml_host_offsetof_data() == 248 == G.Tensor.data.offset
    assert host.stub.ggml_host_offsetof_name() == 256 == G.Tensor.name.offset


def test_registry(host):
    for w32, name in ((False, b"LNSHIP16"), (True, b"LNSHIP32")):
        r = host.reg(w32)
        assert r.api_version == 2
        assert G.call(r.iface.get_name, ctypes.c_char_p, (ctypes.addressof(r), ctypes.c_void_p)) == name
        n = G.call(r.iface.get_device_count, ctypes.c_size_t, (ctypes.addressof(r), ctypes.c_void_p))
        assert n in (0, 1)
        if n == 0:
            assert host.init(w32) is None


def test_proc_address_exports_monte_state(host):
    for w32 in (False, True):
        r = host.reg(w32)
        for fn in ("ggml_backend_lnship16_monte_get_state", "ggml_backend_lnship16_monte_set_state",
                   "ggml_backend_lnship16_monte_reserve"):
            p = G.call(r.iface.get_proc_address, ctypes.c_void_p, (ctypes.addressof(r), ctypes.c_void_p),
                       (fn.encode(), ctypes.c_char_p))
            if w32:
                assert p is None
            else:
                assert p == ctypes.cast(getattr(host.lib, fn), ctypes.c_void_p).value
        assert G.call(r.iface.get_proc_address, ctypes.c_void_p, (ctypes.addressof(r), ctypes.c_void_p),
                      (b"no_such_function", ctypes.c_char_p)) is None


def test_device_slots(host):
    for w32 in (False, True):
        d = host.device(w32)
        a = (ctypes.addressof(d), ctypes.c_void_p)
        name = G.call(d.iface.get_name, ctypes.c_char_p, a)
        assert name == (b"LNSHIP32" if w32 else b"LNSHIP16")
        desc = G.call(d.iface.get_description, ctypes.c_char_p, a).decode()
        assert desc.startswith("Logarithmic Number System on HIP (xlns32" if w32 else
                               "Logarithmic Number System on HIP (xlns16, sum=base")
        assert G.call(d.iface.get_type, ctypes.c_int, a) == 3   # ACCEL
        p = G.DevProps()
        G.call(d.iface.get_props, None, a, (ctypes.addressof(p), ctypes.c_void_p))
        assert p.name == name and p.type == 3
        assert (p.caps.async_, p.caps.host_buffer, p.caps.buffer_from_host_ptr, p.caps.events) == \
            (False, False, True, False)
        cpu_buft = host.stub.ggml_backend_cpu_buffer_type
        cpu_buft.restype = ctypes.c_void_p
        assert G.call(d.iface.get_buffer_type, ctypes.c_void_p, a) == cpu_buft()
        assert G.call(d.iface.supports_buft, ctypes.c_bool, a, (cpu_buft(), ctypes.c_void_p))
        assert not G.call(d.iface.supports_buft, ctypes.c_bool, a, (12345, ctypes.c_void_p))
        # slots the reference leaves empty
        for slot in ("get_host_buffer_type", "event_new", "event_free", "event_synchronize"):
            assert getattr(d.iface, slot) is None
        assert d.iface.offload_op == d.iface.supports_op


# ---- op predicates ---------------------------------------------------------

def _mm(h, src0_type="f32", K=576, M=1536, N=3, ne02=1, ne12=1, src1_type="f32", nb0=None):
    a = h.tensor([K, M, ne02], src0_type, weights=True, name="blk.0.ffn_up.weight")
    if nb0 is not None:
        a.nb[0] = nb0
    b = h.tensor([K, N, ne12], src1_type, name="attn_norm-0")
    return h.tensor([M, N, ne12], "f32", op="MUL_MAT", src=(a, b), name="ffn_up-0")


def _verdicts(h, w32=False):
    f = lambda **kw: h.tensor(**kw)
    x = f(ne=[576, 3], name="x")
    cases = {}
    cases["mm_f32"] = _mm(h)
    cases["mm_f16"] = _mm(h, "f16")
    cases["mm_q8_0"] = _mm(h, "q8_0")
    cases["mm_lns16_src0"] = _mm(h, "lns16")
    cases["mm_src1_f16"] = _mm(h, src1_type="f16")
    cases["mm_strided_rows"] = _mm(h, nb0=8)
    cases["mm_gqa"] = _mm(h, K=64, M=256, N=3, ne02=3, ne12=9)
    cases["mm_partial_bcast"] = _mm(h, K=64, M=256, N=3, ne02=3, ne12=4)
    cases["rms"] = f(ne=[576, 3], op="RMS_NORM", src=(x,), fparams={0: 1e-5})
    cases["rms_f16"] = f(ne=[576, 3], op="RMS_NORM", src=(f(ne=[576, 3], type_name="f16"),), fparams={0: 1e-5})
    long_row = f(ne=[1 << 18, 1])
    cases["rms_long"] = f(ne=[1 << 18, 1], op="RMS_NORM", src=(long_row,), fparams={0: 1e-5})
    kq = f(ne=[256, 3, 9])
    mask = f(ne=[256, 4])
    cases["softmax"] = f(ne=[256, 3, 9], op="SOFT_MAX", src=(kq, mask), fparams={0: 0.125, 1: 0.0})
    cases["softmax_nomask"] = f(ne=[256, 3, 9], op="SOFT_MAX", src=(kq,), fparams={0: 0.125, 1: 0.0})
    cases["softmax_sinks"] = f(ne=[256, 3, 9], op="SOFT_MAX", src=(kq, mask, f(ne=[9])), fparams={0: 0.125})
    cases["softmax_alibi"] = f(ne=[256, 3, 9], op="SOFT_MAX", src=(kq, mask), fparams={0: 0.125, 1: 8.0})
    cases["softmax_small_mask"] = f(ne=[256, 3, 9], op="SOFT_MAX", src=(kq, f(ne=[128, 4])), fparams={0: 1.0})
    cases["add_bcast"] = f(ne=[576, 3], op="ADD", src=(x, f(ne=[576])))
    cases["add_bad_bcast"] = f(ne=[576, 3], op="ADD", src=(x, f(ne=[575])))
    cases["mul_f16"] = f(ne=[576, 3], op="MUL", src=(x, f(ne=[576], type_name="f16")))
    swi = h.stub.ggml_host_glu(b"SWIGLU")
    geg = h.stub.ggml_host_glu(b"GEGLU")
    ug = f(ne=[3072, 3])
    cases["swiglu_fused"] = f(ne=[1536, 3], op="GLU", src=(ug,), params=(swi, 0))
    cases["swiglu_split"] = f(ne=[1536, 3], op="GLU", src=(f(ne=[1536, 3]), f(ne=[1536, 3])), params=(swi, 0))
    cases["swiglu_odd"] = f(ne=[1536, 3], op="GLU", src=(f(ne=[3071, 3]),), params=(swi, 0))
    cases["geglu"] = f(ne=[1536, 3], op="GLU", src=(ug,), params=(geg, 0))
    cases["silu"] = f(ne=[576, 3], op="UNARY", src=(x,), params=(h.stub.ggml_host_unary(b"SILU"),))
    q = f(ne=[64, 9, 3])
    pos = f(ne=[3], type_name="i32")
    rp = {5: 10000.0, 6: 1.0, 7: 0.0, 8: 1.0}
    cases["rope"] = f(ne=[64, 9, 3], op="ROPE", src=(q, pos), params=(0, 64, 0), fparams=rp)
    cases["rope_neox"] = f(ne=[64, 9, 3], op="ROPE", src=(q, pos), params=(0, 64, 2), fparams=rp)
    cases["rope_mrope"] = f(ne=[64, 9, 3], op="ROPE", src=(q, pos), params=(0, 64, 8), fparams=rp)
    cases["rope_yarn"] = f(ne=[64, 9, 3], op="ROPE", src=(q, pos), params=(0, 64, 0), fparams={**rp, 7: 1.0})
    cases["rope_short_pos"] = f(ne=[64, 9, 3], op="ROPE", src=(q, f(ne=[2], type_name="i32")), params=(0, 64, 0),
                                fparams=rp)
    cases["rope_odd_dims"] = f(ne=[64, 9, 3], op="ROPE", src=(q, pos), params=(0, 63, 0), fparams=rp)
    cases["view"] = f(ne=[576, 3], op="VIEW", src=(x,))
    cases["get_rows"] = f(ne=[576, 3], op="GET_ROWS", src=(x, pos))
    wexp = h.tensor([576, 256, 8], "q8_0", weights=True, name="blk.0.ffn_up_exps.weight")
    xe = f(ne=[576, 1, 3])
    cases["mm_id"] = f(ne=[256, 2, 3], op="MUL_MAT_ID", src=(wexp, xe, f(ne=[2, 3], type_name="i32")))
    cases["mm_id_i64_ids"] = f(ne=[256, 2, 3], op="MUL_MAT_ID", src=(wexp, xe, f(ne=[2, 3], type_name="i64")))
    cases["mm_id_bad_bcast"] = f(ne=[256, 3, 3], op="MUL_MAT_ID",
                                 src=(wexp, f(ne=[576, 2, 3]), f(ne=[3, 3], type_name="i32")))
    cases["scale"] = f(ne=[576, 3], op="SCALE", src=(x,), fparams={0: 0.125, 1: 0.0})
    xt = f(ne=[3, 576], nb=[4 * 576, 4, 4 * 576 * 3, 4 * 576 * 3])
    cases["scale_strided"] = f(ne=[3, 576], op="SCALE", src=(xt,), fparams={0: 0.125, 1: 0.0})
    cases["cpy"] = f(ne=[576, 3], type_name="f16", op="CPY", src=(x,))
    cases["set_rows"] = f(ne=[576, 8], type_name="f16", op="SET_ROWS", src=(x, f(ne=[3], type_name="i64")))
    return {k: h.check(t, w32) for k, t in cases.items()}


EXPECT16 = {
    "mm_f32": (True, "lnship_mul_mat"),
    "mm_f16": (True, "lnship_mul_mat"),
    "mm_q8_0": (True, "lnship_mul_mat"),
    "mm_lns16_src0": (True, "lnship_mul_mat"),
    "mm_src1_f16": (False, "mul_mat_requires_src1_f32_and_convertible_src0"),
    "mm_strided_rows": (False, "mul_mat_requires_contiguous_rows"),
    "mm_gqa": (True, "lnship_mul_mat"),
    "mm_partial_bcast": (False, "lnship_mul_mat_requires_whole_broadcast"),
    "rms": (True, "unary_like_requires_src0_f32"),
    "rms_f16": (False, "unary_like_requires_src0_f32"),
    "rms_long": (False, "lnship_row_too_long"),
    "softmax": (True, "soft_max_f32"),
    "softmax_nomask": (True, "soft_max_f32"),
    "softmax_sinks": (False, "soft_max_sinks_unsupported"),
    "softmax_alibi": (False, "soft_max_alibi_unsupported"),
    "softmax_small_mask": (False, "lnship_soft_max_mask_smaller_than_src0"),
    "add_bcast": (True, "binary_requires_f32_srcs"),
    "add_bad_bcast": (False, "lnship_binary_requires_repeatable_src1"),
    "mul_f16": (False, "binary_requires_f32_srcs"),
    "swiglu_fused": (True, "glu_fused_requires_even_src0_and_half_width_dst"),
    "swiglu_split": (True, "glu_split_requires_matching_f32_contiguous_inputs"),
    "swiglu_odd": (False, "glu_fused_requires_even_src0_and_half_width_dst"),
    "geglu": (False, "unsupported_glu_op"),
    "silu": (False, "unsupported_unary_op"),
    "rope": (True, "lnship_rope"),
    "rope_neox": (True, "lnship_rope"),
    "rope_mrope": (False, "rope_mode_unsupported"),
    "rope_yarn": (False, "rope_scaling_unsupported"),
    "rope_short_pos": (False, "lnship_rope_requires_i32_positions"),
    "rope_odd_dims": (False, "lnship_rope_requires_even_n_dims"),
    "view": (True, "supported_view_or_noop"),
    "get_rows": (False, "lnship_get_rows_requires_hbm_dst"),
    "mm_id": (True, "lnship_mul_mat_id"),
    "mm_id_i64_ids": (False, "mul_mat_id_requires_src1_f32_and_i32_ids_and_convertible_src0"),
    "mm_id_bad_bcast": (False, "lnship_mul_mat_id_shape"),
    "scale": (True, "requires_contiguous_f32_src0_and_dst"),
    "scale_strided": (False, "requires_contiguous_f32_src0_and_dst"),
    "cpy": (False, "lnship_copy_requires_hbm_dst"),
    "set_rows": (False, "lnship_set_rows_requires_hbm_dst"),
}


def test_lnship16_predicates(host):
    got = _verdicts(host)
    bad = {k: (got[k], v) for k, v in EXPECT16.items() if got[k] != v}
    assert not bad, bad


def test_lnship32_claims(host):
    # the xlns32 backend runs the hot ops and the Llama graph's elementwise
    # ops (cuda/lns-cuda-kernels.cuh:161-355 instantiate them for xlns32 too)
    got = _verdicts(host, w32=True)
    for k in ("mm_f32", "mm_q8_0", "mm_gqa", "rms", "softmax", "view", "add_bcast", "swiglu_fused", "rope", "scale",
              "mm_id"):
        assert got[k][0], (k, got[k])
    for k in ("geglu", "silu", "get_rows", "cpy", "set_rows", "mm_lns16_src0"):
        assert not got[k][0], (k, got[k])
    # xlns32 rows take 4 bytes of LDS each
    assert got["rms_long"] == (False, "lnship_row_too_long")


# ---- environment (fresh interpreter per case) --------------------------------

PRELUDE = textwrap.dedent("""
    import ctypes, sys
    sys.path.insert(0, {tests!r})
    import ggml_host as G
    h = G.Host()
    x = h.tensor([576, 3], name="attn_norm-0")
    w = h.tensor([576, 1536], weights=True, name="blk.0.ffn_up.weight")
    mm = h.tensor([1536, 3], op="MUL_MAT", src=(w, x), name="ffn_up-0")
    w2 = h.tensor([1536, 576], weights=True, name="blk.0.ffn_down.weight")
    mm2 = h.tensor([576, 3], op="MUL_MAT", src=(w2, h.tensor([1536, 3], name="ffn_gate_par-0")), name="ffn_down-0")
    rms = h.tensor([576, 3], op="RMS_NORM", src=(x,), fparams={{0: 1e-5}}, name="norm-0")
""").format(tests=HERE)


def _run(code, **env):
    e = {k: v for k, v in os.environ.items()
         if k not in ("GGML_LNS_BACKEND", "LNS_DISABLE_OPS", "LNS_ENABLE_OPS", "LNS_OP_AUDIT", "GGML_LNS16_SUM")}
    e.update(env)
    r = subprocess.run([sys.executable, "-c", PRELUDE + textwrap.dedent(code)], env=e, capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    return r.stdout, r.stderr


def test_default_selection_leaves_ops_to_the_cpu_backend():
    out, err = _run("print(h.supports_op(mm), h.supports_op(rms))", LNS_OP_AUDIT="1")
    assert out.split() == ["False", "False"]
    recs = [json.loads(l) for l in err.splitlines() if l.startswith("{")]
    assert recs and all(r["reason"] == "disabled_by_env" and r["backend"] == "LNSHIP16" for r in recs)


def test_selection_aliases():
    for sel, want16, want32 in (("hip16", True, False), ("hip", True, False), ("hip32", False, True),
                                ("LNSHIP16", True, False), ("lnship32,16", False, True), ("cuda16", False, False)):
        out, _ = _run("print(h.supports_op(mm), h.supports_op(mm, w32=True))", GGML_LNS_BACKEND=sel)
        assert out.split() == [str(want16), str(want32)], sel


def test_unknown_selection_token_warns_and_falls_back():
    out, err = _run("print(h.supports_op(mm))", GGML_LNS_BACKEND="nonsense")
    assert out.split() == ["False"] and "ignoring unknown GGML_LNS_BACKEND token 'nonsense'" in err


def test_disable_and_enable_lists():
    code = "print(h.supports_op(mm), h.supports_op(mm2), h.supports_op(rms))"
    cases = ((dict(LNS_DISABLE_OPS="mul_mat"), ["False", "False", "True"]),
             (dict(LNS_DISABLE_OPS="ffn_down"), ["True", "False", "True"]),
             (dict(LNS_DISABLE_OPS="MUL_MAT:<ffn_gate*"), ["True", "False", "True"]),
             (dict(LNS_DISABLE_OPS="RMS_NORM:blk*"), ["True", "True", "True"]),
             (dict(LNS_ENABLE_OPS="RMS_NORM"), ["False", "False", "True"]),
             (dict(LNS_ENABLE_OPS=""), ["False", "False", "False"]))
    for env, want in cases:
        out, _ = _run(code, GGML_LNS_BACKEND="hip16", **env)
        assert out.split() == want, env


def test_audit_record_format():
    _, err = _run("h.supports_op(mm)", GGML_LNS_BACKEND="hip16", LNS_OP_AUDIT="1", GGML_LNS16_SUM="sum32")
    rec = json.loads([l for l in err.splitlines() if l.startswith("{")][0])
    assert list(rec) == ["event", "backend", "sum_mode", "op", "desc", "supported", "dst_type", "src_types",
                         "shape", "reason"]
    assert rec["event"] == "lns_supports_op" and rec["sum_mode"] == "sum32" and rec["op"] == "MUL_MAT"
    assert rec["supported"] is True and rec["src_types"] == ["f32", "f32", "null", "null"]
    assert rec["shape"] == [1536, 3, 1, 1] and rec["reason"] == "lnship_mul_mat"


def test_sum_mode_in_description():
    for mode in ("base", "lpvip", "sum32", "monte"):
        out, _ = _run("""
            d = h.device()
            print(G.call(d.iface.get_description, ctypes.c_char_p, (ctypes.addressof(d), ctypes.c_void_p)).decode())
        """, GGML_LNS16_SUM=mode)
        assert ("sum=%s" % mode) in out
        assert ("monte=pure16" in out) == (mode == "monte")


def test_bad_sum_mode_aborts():
    e = dict(os.environ, GGML_LNS16_SUM="fast")
    r = subprocess.run([sys.executable, "-c", PRELUDE + "h.reg()"], env=e, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode != 0 and "GGML_LNS16_SUM must be one of" in r.stderr


def test_monte_bylpvip_refused():
    # the reference's GGML_LNS16_MONTE_BYLPVIP build is not available: asking
    # for it in a Monte run stops with a message instead of running pure16
    e = dict(os.environ, GGML_LNS16_SUM="monte", GGML_LNS16_MONTE_BYLPVIP="ON")
    r = subprocess.run([sys.executable, "-c", PRELUDE + "h.reg()"], env=e, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode != 0 and "monte=bylpvip is not available" in r.stderr
    for off in ("OFF", "0"):
        e = dict(os.environ, GGML_LNS16_SUM="monte", GGML_LNS16_MONTE_BYLPVIP=off)
        r = subprocess.run([sys.executable, "-c", PRELUDE + "h.reg()"], env=e, capture_output=True, text=True,
                           timeout=120)
        assert r.returncode == 0, r.stderr[-500:]


def test_data_movement_claimed_for_hbm_destinations():
    # with the HBM buffer type, CPY / CONT / GET_ROWS / SET_ROWS whose
    # destination is not allocated yet (the scheduler places it in this
    # backend's buffer type) are claimed; a destination in host memory, a bad
    # shape or a quantized destination are left to the CPU backend
    out, _ = _run("""
        def unalloc(t):
            t.buffer = None
            return t
        ids = h.tensor([3], "i32")
        ids64 = h.tensor([3], "i64")
        cases = [
            unalloc(h.tensor([576, 3], "f16", op="CPY", src=(x,))),
            unalloc(h.tensor([576, 3], op="CONT", src=(x,))),
            unalloc(h.tensor([576, 3], op="GET_ROWS", src=(h.tensor([576, 100], weights=True), ids))),
            unalloc(h.tensor([576, 3], op="GET_ROWS", src=(h.tensor([576, 100], "q8_0", weights=True), ids))),
            unalloc(h.tensor([576, 8], "f16", op="SET_ROWS", src=(x, ids64))),
            unalloc(h.tensor([576, 8], "f16", op="SET_ROWS", src=(x, ids))),
            h.tensor([576, 3], "f16", op="CPY", src=(x,)),
            unalloc(h.tensor([576, 2], op="GET_ROWS", src=(h.tensor([576, 100]), ids))),
            unalloc(h.tensor([576, 8], "f16", op="SET_ROWS", src=(x, h.tensor([2], "i64")))),
            unalloc(h.tensor([576, 3], "q8_0", op="CPY", src=(x,))),
        ]
        print(" ".join(str(h.check(t)[0]) for t in cases))
    """, GGML_LNS_BACKEND="hip", GGML_LNS_HIP_BUFFERS="device")
    assert out.split() == ["True"] * 6 + ["False"] * 4


def test_bad_sum_policy_aborts():
    for policy, msg in (("MUL_MAT", "is not selector=mode"), ("MUL_MAT=fast", "is not available"),
                        ("SOFT_MAX=monte", "monte only as GGML_LNS16_SUM")):
        e = dict(os.environ, GGML_LNS16_SUM="sum32", LNS16_SUM_POLICY=policy)
        r = subprocess.run([sys.executable, "-c", PRELUDE + "h.reg()"], env=e, capture_output=True, text=True,
                           timeout=120)
        assert r.returncode != 0 and msg in r.stderr, (policy, r.stderr[-500:])
    e = dict(os.environ, GGML_LNS16_SUM="base", LNS16_SUM_POLICY="MUL_MAT=sum32, SOFT_MAX:kq*=lpvip")
    r = subprocess.run([sys.executable, "-c", PRELUDE + "h.reg()"], env=e, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0 and "LNS16_SUM_POLICY with 2 rules (default sum=base)" in r.stderr, r.stderr[-500:]


def test_monte_state_api():
    out, _ = _run("""
        L = h.lib
        s = ctypes.c_uint16()
        print(L.ggml_backend_lnship16_monte_get_state(ctypes.byref(s)), s.value)
        print(L.ggml_backend_lnship16_monte_reserve(1000, ctypes.byref(s)), s.value)
        L.ggml_backend_lnship16_monte_get_state(ctypes.byref(s)); print(s.value)
        print(L.ggml_backend_lnship16_monte_set_state(0), L.ggml_backend_lnship16_monte_set_state(12345))
        L.ggml_backend_lnship16_monte_reserve(70000, ctypes.byref(s)); print(s.value)
        L.ggml_backend_lnship16_monte_get_state(ctypes.byref(s)); print(s.value)
    """, GGML_LNS16_SUM="monte")
    lines = out.split("\n")
    assert lines[0] == "True 7" and lines[1] == "True 7"
    assert int(lines[2]) == _lfsr(7, 1000)
    assert lines[3] == "False True" and int(lines[4]) == 12345
    assert int(lines[5]) == _lfsr(12345, 70000)


def _lfsr(state, n):
    """n single steps of the oracle's LFSR (src/lns-ops.cpp:182-188), an
    independent check of the backend's closed-form jump."""
    step = O.lib().lno_lfsr_step
    step.restype = ctypes.c_uint16
    step.argtypes = [ctypes.c_uint16]
    for _ in range(n):
        state = step(state)
    return state


def test_monte_api_is_inert_in_other_modes():
    out, _ = _run("""
        L = h.lib
        s = ctypes.c_uint16()
        print(L.ggml_backend_lnship16_monte_get_state(ctypes.byref(s)),
              L.ggml_backend_lnship16_monte_set_state(5), L.ggml_backend_lnship16_monte_reserve(3, ctypes.byref(s)))
    """, GGML_LNS16_SUM="sum32")
    assert out.split() == ["False", "False", "False"]
