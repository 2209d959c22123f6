"""Runs a small ggml graph through the LNSHIP16 (or LNSHIP32) backend on the
GPU and checks every node against the oracle, bit for bit (TEST
INFRASTRUCTURE; run by tests/test_gpu_ggml.py, one process per summation
mode because the backend reads GGML_LNS16_SUM once).

The graph has the shapes and layouts llama.cpp hands the reference's
LNSCUDA16 backend (cuda/lns-cuda-ops.cpp): an rms_norm and norm-weight MUL,
a fused QKV MUL_MAT on F32 weights, RoPE on a strided view of it, the GQA kq
MUL_MAT on an F16 KV-cache tensor against a permuted view, a masked
SOFT_MAX, a Q8_0-weight and a Q4_K-weight MUL_MAT, SWIGLU fused and split, ADD with flat and
general broadcasts, an F16-weight MUL_MAT, a repeated MUL_MAT that hits the
weight cache, an unmasked SOFT_MAX, a MUL_MAT_ID over six experts and a
MUL_MAT on GGML_TYPE_LNS16 weights (xlns16 codes, used as they are).  The oracle runs the same ops in
graph order, so Monte draws are reserved in the same sequence.

With --policy the backend runs under LNS16_SUM_POLICY and the oracle takes
each node's summation mode from the same rules (op names, "OP:glob" on the
node name, or a glob).

With --device-buffers (GGML_LNS_HIP_BUFFERS=device) the inputs, the KV
cache, the F32 / F16 weights and every node live in the backend's device
buffers, and results are read back through the buffer interface.

With --movement: SCALE, CPY / CONT, GET_ROWS and SET_ROWS on HBM tensors
(the KV-cache writes and row gathers of a device-resident graph).

Usage: python ggml_graph_check.py --mode base|monte|lpvip|sum32 [--policy RULES] [--device-buffers] [--w32]
       python ggml_graph_check.py --movement [--w32]
Exit status 0 when every node matches.
"""
import argparse
import ctypes
import fnmatch
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

import ggml_host as G  # noqa: E402
import oracle_lib as O  # noqa: E402


def q8_0(w, rng):
    """w [M, K] -> (block bytes, the F32 values the blocks decode to)."""
    M, K = w.shape
    blocks = w.reshape(M, K // 32, 32)
    d = (np.abs(blocks).max(axis=2) / 127.0).astype(np.float16)
    d[d == 0] = np.float16(1.0)
    q = np.clip(np.rint(blocks / d.astype(np.float32)[..., None]), -127, 127).astype(np.int8)
    raw = np.zeros((M, K // 32, 34), np.uint8)
    raw[..., :2] = d.view(np.uint8).reshape(M, K // 32, 2)
    raw[..., 2:] = q.view(np.uint8)
    deq = q.astype(np.float32) * d.astype(np.float32)[..., None]
    return raw.reshape(-1), deq.reshape(M, K)


def q4_k(M, K, rng):
    """Random Q4_K blocks for an [M, K] weight (K a multiple of 256) -> (block
    bytes, the F32 values they decode to).  ggml's published layout: per 256
    values a half d, a half dmin, 12 bytes of eight 6-bit (scale, min) pairs
    and 128 bytes of 4-bit quants (value = d * scale * q - dmin * min)."""
    nb = M * (K // 256)
    raw = np.zeros((nb, 144), np.uint8)
    d = (rng.uniform(0.5, 1.5, nb) * 0.02 / 63).astype(np.float16)
    dmin = (rng.uniform(0.5, 1.5, nb) * 0.02 / 63).astype(np.float16)
    raw[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    raw[:, 2:4] = dmin.view(np.uint8).reshape(nb, 2)
    raw[:, 4:16] = rng.integers(0, 256, (nb, 12), dtype=np.uint8)
    raw[:, 16:] = rng.integers(0, 256, (nb, 128), dtype=np.uint8)
    sb = raw[:, 4:16].astype(np.int32)
    sc = np.zeros((nb, 8), np.int32)
    mn = np.zeros((nb, 8), np.int32)
    for j in range(4):
        sc[:, j] = sb[:, j] & 63
        mn[:, j] = sb[:, j + 4] & 63
        sc[:, j + 4] = (sb[:, j + 8] & 15) | ((sb[:, j] >> 6) << 4)
        mn[:, j + 4] = (sb[:, j + 8] >> 4) | ((sb[:, j + 4] >> 6) << 4)
    q = raw[:, 16:].reshape(nb, 4, 32).astype(np.int32)
    nib = np.stack([q & 15, q >> 4], axis=2).reshape(nb, 8, 32)   # sub-block 2r: low, 2r + 1: high nibbles
    dd = d.astype(np.float32)[:, None] * sc.astype(np.float32)
    dm = dmin.astype(np.float32)[:, None] * mn.astype(np.float32)
    deq = dd[:, :, None] * nib.astype(np.float32) - dm[:, :, None]
    return raw.reshape(-1), deq.astype(np.float32).reshape(M, K)


def oracle_fns():
    L = O.lib()
    for name, args in (("lno16_add_f32", [ctypes.c_void_p] * 2 + [ctypes.c_int64] * 2 + [ctypes.c_void_p]),
                       ("lno16_mul_f32", [ctypes.c_void_p] * 2 + [ctypes.c_int64] * 2 + [ctypes.c_void_p]),
                       ("lno16_swiglu_f32", [ctypes.c_void_p] * 2 + [ctypes.c_int64, ctypes.c_void_p]),
                       ("lno16_rope_f32", [ctypes.c_void_p] * 2 + [ctypes.c_int64] * 3 +
                        [ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_void_p])):
        fn = getattr(L, name)
        fn.restype = None
        fn.argtypes = args
    return L


def P(a):
    return ctypes.c_void_p(a.ctypes.data)


def binop(fn, a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    out = np.empty_like(a)
    fn(P(a), P(b), a.size, b.size, P(out))
    return out


def policy_modes(policy, default):
    """mode_of(op, name) under LNS16_SUM_POLICY rules (the forms this check uses)."""
    rules = []
    for rule in filter(None, (r.strip() for r in (policy or "").split(","))):
        sel, mode = rule.rsplit("=", 1)
        rules.append((sel, O.MODES[mode]))

    def mode_of(op, name):
        for sel, mode in rules:
            if sel.upper() == op:
                return mode
            if ":" in sel:
                o, pat = sel.split(":", 1)
                if o.upper() == op and fnmatch.fnmatch(name, pat):
                    return mode
            elif fnmatch.fnmatch(name, sel):
                return mode
        return default
    return mode_of


FLAG_OUTPUT = 2


def mark_outputs(nodes, fused):
    """Flags every checked node as a graph output, so each op runs on its own;
    with fused, the nodes that feed only the next node (RMS_NORM before its
    norm-weight MUL, MUL_MAT before its residual ADD) stay unflagged, so
    graph_compute fuses the pairs, and are left out of the check (a fused
    pair does not write the intermediate tensor).  "mm_self" stays unflagged
    too but is checked: its ADD reads the product's own activation and writes
    over it in place, a pair graph_compute must not fuse.  Returns the
    checked keys.  "rms1" -> "mul1" -> "qkv1" is a decode step's norm and
    q|k|v product (one row): in sum32 graph_compute runs the three as one
    launch, in the other modes the first two.  "rms2" -> "mul2" -> "mm2" is
    such a row too long for the three-node launch: the pair runs fused and
    "mul2" is written."""
    skip = {"rms", "mm", "down", "rms1", "mul1", "rms2"} if fused else set()
    noflag = {"mm_self", "mul2"} if fused else set()
    for k, tn in nodes.items():
        if k not in skip and k not in noflag:
            tn.flags |= FLAG_OUTPUT
    return [k for k in nodes if k not in skip]


def run16(mode_name, policy=None, dev=False, fused=False):
    m = O.MODES[mode_name]
    mode_of = policy_modes(policy, m)
    L = oracle_fns()
    h = G.Host()
    # with dev, activations, caches and F32 / F16 weights live in the
    # backend's device buffers (weights in one of WEIGHTS usage, so the
    # weight cache sees them); the Q8_0 weight stays in host memory
    act = h.device_buffer(64 << 20) if dev else None
    wts = h.device_buffer(16 << 20) if dev else None
    if dev:
        h.stub.ggml_host_set_usage.argtypes = [ctypes.c_void_p, ctypes.c_int]
        h.stub.ggml_host_set_usage(wts.addr, G.USAGE_WEIGHTS)
    rng = np.random.default_rng(1234)
    f32 = lambda *s, scale=1.0, loc=0.0: (rng.standard_normal(s) * scale + loc).astype(np.float32)
    T, E, H, HKV, D, NKV = 3, 576, 9, 3, 64, 256
    x0 = f32(T, E)
    g = f32(E, scale=0.1, loc=1.0)
    wqkv = f32(E + 2 * HKV * D, E, scale=0.02)
    kc = (rng.standard_normal((HKV, NKV, D)) * 0.5).astype(np.float16)
    pos = np.array([100, 101, 102], np.int32)
    mask = np.zeros((4, NKV), np.float32)
    for t in range(4):
        mask[t, 101 + t:] = -np.inf
    wq8_raw, wq8 = q8_0(f32(256, E, scale=0.02), rng)
    bias = f32(T, 1)
    x1 = f32(T, 1536)
    w2 = (rng.standard_normal((E, 1536)) * 0.02).astype(np.float16)
    z = f32(2, 5, 100, scale=3.0)
    wmoe = f32(6, 96, 64, scale=0.05)
    xmoe = f32(T, 1, 64)
    ids_moe = np.array([[5, 0], [2, 2], [1, 4]], np.int32)
    w_codes = O.f2x16(f32(200, E, scale=0.05))   # GGML_TYPE_LNS16 weights
    xs = f32(T, E)
    wself = f32(E, E, scale=0.02)
    xdec = f32(1, E)
    wq4_raw, wq4 = q4_k(128, 768, rng)
    x4 = f32(T, 768)
    # a decode row longer than lnship16_rms_norm_mul_mat holds in LDS: with
    # fusion on, graph_compute runs its RMS_NORM -> MUL pair and the MUL_MAT
    K2 = int(G.lnship_max_row(5, O.SUM32)) + 8
    xdec2 = f32(1, K2)
    g2 = f32(K2, scale=0.1, loc=1.0)
    wlong = f32(64, K2, scale=0.02)

    t = lambda *a, **k: h.tensor(*a, device=None if k.get("weights") else act, **k)
    tw = lambda *a, **k: h.tensor(*a, device=wts, **k)
    X0 = t([E, T], data=x0, name="inp")
    Gw = tw([E], data=g, weights=True, name="blk.0.attn_norm.weight")
    WQKV = tw([E, E + 2 * HKV * D], data=wqkv, weights=True, name="blk.0.attn_qkv.weight")
    KC = t([D, NKV, HKV], "f16", data=kc, name="cache_k_l0")
    POS = t([T], "i32", data=pos, name="inp_pos")
    MASK = t([NKV, 4], data=mask, name="kq_mask")
    WQ8 = h.tensor([E, 256], "q8_0", data=wq8_raw, weights=True, name="blk.0.ffn_up.weight")
    BIAS = t([1, T], data=bias, name="bias")
    X1 = t([1536, T], data=x1, name="ffn_inp")
    W2 = tw([1536, E], "f16", data=w2, weights=True, name="blk.0.ffn_down.weight")
    Z = t([100, 5, 2], data=z, name="scores")
    WMOE = tw([64, 96, 6], data=wmoe, weights=True, name="blk.0.ffn_up_exps.weight")
    WL16 = tw([E, 200], "lns16", data=w_codes, weights=True, name="blk.0.attn_k_lns16.weight")
    XMOE = t([64, 1, T], data=xmoe, name="ffn_moe_inp")
    IDS = t([2, T], "i32", data=ids_moe, name="ffn_moe_topk")
    WQ4 = h.tensor([768, 128], "q4_k", data=wq4_raw, weights=True, name="blk.0.ffn_gate.weight")
    X4 = t([768, T], data=x4, name="ffn_inp_q4")
    G2 = tw([K2], data=g2, weights=True, name="blk.1.attn_norm.weight")
    WLONG = tw([K2, 64], data=wlong, weights=True, name="blk.1.attn_q.weight")
    swi = h.stub.ggml_host_glu(b"SWIGLU")

    nodes = {}
    nodes["rms"] = t([E, T], op="RMS_NORM", src=(X0,), fparams={0: 1e-5}, name="norm-0")
    nodes["mul"] = t([E, T], op="MUL", src=(nodes["rms"], Gw), name="attn_norm-0")
    nodes["qkv"] = t([E + 2 * HKV * D, T], op="MUL_MAT", src=(WQKV, nodes["mul"]), name="qkv-0")
    qv = t([D, H, T], op="VIEW", src=(nodes["qkv"],), data=nodes["qkv"].data,
           nb=[4, D * 4, (E + 2 * HKV * D) * 4, (E + 2 * HKV * D) * 4 * T], name="q-0")
    nodes["rope"] = t([D, H, T], op="ROPE", src=(qv, POS), params=(0, D, 0),
                      fparams={5: 10000.0, 6: 1.0, 7: 0.0, 8: 1.0}, name="Qcur-0")
    qp = t([D, T, H], op="PERMUTE", src=(nodes["rope"],), data=nodes["rope"].data,
           nb=[4, D * H * 4, D * 4, D * H * T * 4], name="q-perm-0")
    nodes["kq"] = t([NKV, T, H], op="MUL_MAT", src=(KC, qp), name="kq-0")
    nodes["softmax"] = t([NKV, T, H], op="SOFT_MAX", src=(nodes["kq"], MASK), fparams={0: 0.125, 1: 0.0},
                         name="kq_soft_max-0")
    nodes["ug"] = t([256, T], op="MUL_MAT", src=(WQ8, nodes["mul"]), name="ffn_up-0")
    nodes["swiglu"] = t([128, T], op="GLU", src=(nodes["ug"],), params=(swi, 0), name="ffn_swiglu-0")
    ga = t([128, T], op="VIEW", src=(nodes["ug"],), data=nodes["ug"].data, nb=[4, 1024, 1024 * T, 1024 * T],
           name="gate-0")
    ua = t([128, T], op="VIEW", src=(nodes["ug"],), data=nodes["ug"].data + 512, nb=[4, 1024, 1024 * T, 1024 * T],
           name="up-0")
    nodes["swiglu_split"] = t([128, T], op="GLU", src=(ga, ua), params=(swi, 0), name="ffn_swiglu_split-0")
    nodes["add"] = t([E, T], op="ADD", src=(X0, nodes["mul"]), name="ffn_inp-0")
    nodes["add_bcast"] = t([E, T], op="ADD", src=(X0, BIAS), name="bias_add-0")
    nodes["down"] = t([E, T], op="MUL_MAT", src=(W2, X1), name="ffn_out-0")
    nodes["down_res"] = t([E, T], op="ADD", src=(X0, nodes["down"]), name="l_out-0")   # residual first
    nodes["qkv_again"] = t([E + 2 * HKV * D, T], op="MUL_MAT", src=(WQKV, nodes["mul"]), name="qkv-1")
    nodes["softmax_nomask"] = t([100, 5, 2], op="SOFT_MAX", src=(Z,), fparams={0: 1.0, 1: 0.0}, name="sm-1")
    nodes["moe"] = t([96, 2, T], op="MUL_MAT_ID", src=(WMOE, XMOE, IDS), name="ffn_moe_up-0")
    nodes["mm_lns16"] = t([200, T], op="MUL_MAT", src=(WL16, nodes["mul"]), name="k_lns16-0")
    # y = W x + x with y written over x (an in-place residual that is the
    # product's own activation)
    XS = t([E, T], data=xs.copy(), name="self_inp")   # overwritten in place
    WS = tw([E, E], data=wself, weights=True, name="blk.0.self.weight")
    nodes["mm_self"] = t([E, T], op="MUL_MAT", src=(WS, XS), name="self_mm-0")
    nodes["add_self"] = t([E, T], op="ADD", src=(XS, nodes["mm_self"]), data=XS.data, name="self_out-0")
    # one decode row: its norm, the norm MUL and the q|k|v product
    XD = t([E, 1], data=xdec, name="inp_dec")
    nodes["rms1"] = t([E, 1], op="RMS_NORM", src=(XD,), fparams={0: 1e-5}, name="norm-1")
    nodes["mul1"] = t([E, 1], op="MUL", src=(nodes["rms1"], Gw), name="attn_norm-1")
    nodes["qkv1"] = t([E + 2 * HKV * D, 1], op="MUL_MAT", src=(WQKV, nodes["mul1"]), name="qkv-2")
    # a Q4_K weight (ggml's to_float, then converted and cached)
    nodes["mm_q4k"] = t([128, T], op="MUL_MAT", src=(WQ4, X4), name="ffn_gate_q4-0")
    XD2 = t([K2, 1], data=xdec2, name="inp_dec_long")
    nodes["rms2"] = t([K2, 1], op="RMS_NORM", src=(XD2,), fparams={0: 1e-5}, name="norm-2")
    nodes["mul2"] = t([K2, 1], op="MUL", src=(nodes["rms2"], G2), name="attn_norm-2")
    nodes["mm2"] = t([64, 1], op="MUL_MAT", src=(WLONG, nodes["mul2"]), name="q-2")
    order = ["rms", "mul", "qkv", "view_q", "rope", "perm_q", "kq", "softmax", "ug", "swiglu", "view_g", "view_u",
             "swiglu_split", "add", "add_bcast", "down", "down_res", "qkv_again", "softmax_nomask", "moe", "mm_lns16",
             "mm_self", "add_self", "rms1", "mul1", "qkv1", "mm_q4k", "rms2", "mul2", "mm2"]
    views = {"view_q": qv, "perm_q": qp, "view_g": ga, "view_u": ua}
    graph = [views[k] if k in views else nodes[k] for k in order]

    checked = mark_outputs(nodes, fused)
    be = h.init()
    if be is None:
        print(json.dumps({"error": "no GPU: LNSHIP16 init returned NULL"}))
        return 1
    rc = h.compute(be, graph)
    assert rc == 0, rc

    # oracle, same op order (Monte draws in graph order)
    O.monte_set(7)
    want = {}
    want["rms"] = O.rms_norm16(mode_of("RMS_NORM", "norm-0"), x0, 1e-5)
    want["mul"] = binop(L.lno16_mul_f32, want["rms"], g)
    want["qkv"] = O.mul_mat16(mode_of("MUL_MAT", "qkv-0"), O.f2x16(wqkv), want["mul"])
    q = np.ascontiguousarray(want["qkv"][:, :E].reshape(T, H, D))
    want["rope"] = np.empty_like(q)
    L.lno16_rope_f32(P(q), P(pos), T, H, D, D, 0, 10000.0, P(want["rope"]))
    qperm = np.ascontiguousarray(want["rope"].transpose(1, 0, 2))
    want["kq"] = O.mul_mat16_f32w(mode_of("MUL_MAT", "kq-0"), kc.astype(np.float32)[None], qperm[None], ne02=HKV)[0]
    want["softmax"] = O.soft_max16(mode_of("SOFT_MAX", "kq_soft_max-0"), want["kq"], mask, 0.125)
    want["ug"] = O.mul_mat16_f32w(mode_of("MUL_MAT", "ffn_up-0"), wq8, want["mul"])
    sw = np.empty((T, 128), np.float32)
    gate, up = np.ascontiguousarray(want["ug"][:, :128]), np.ascontiguousarray(want["ug"][:, 128:])
    L.lno16_swiglu_f32(P(gate), P(up), gate.size, P(sw))
    want["swiglu"] = sw
    want["swiglu_split"] = sw
    want["add"] = binop(L.lno16_add_f32, x0, want["mul"])
    want["add_bcast"] = binop(L.lno16_add_f32, x0, np.repeat(bias, E, axis=1))
    want["down"] = O.mul_mat16_f32w(mode_of("MUL_MAT", "ffn_out-0"), w2.astype(np.float32), x1)
    want["down_res"] = binop(L.lno16_add_f32, x0, want["down"])
    want["qkv_again"] = O.mul_mat16(mode_of("MUL_MAT", "qkv-1"), O.f2x16(wqkv), want["mul"])
    want["softmax_nomask"] = O.soft_max16(mode_of("SOFT_MAX", "sm-1"), z, None, 1.0)
    want["moe"] = O.mul_mat_id(mode_of("MUL_MAT_ID", "ffn_moe_up-0"), wmoe, xmoe, ids_moe)
    want["mm_lns16"] = O.mul_mat16(mode_of("MUL_MAT", "k_lns16-0"), w_codes, want["mul"])
    want["mm_self"] = O.mul_mat16(mode_of("MUL_MAT", "self_mm-0"), O.f2x16(wself), xs)
    want["add_self"] = binop(L.lno16_add_f32, xs, want["mm_self"])
    want["rms1"] = O.rms_norm16(mode_of("RMS_NORM", "norm-1"), xdec, 1e-5)
    want["mul1"] = binop(L.lno16_mul_f32, want["rms1"], g)
    want["qkv1"] = O.mul_mat16(mode_of("MUL_MAT", "qkv-2"), O.f2x16(wqkv), want["mul1"])
    want["mm_q4k"] = O.mul_mat16_f32w(mode_of("MUL_MAT", "ffn_gate_q4-0"), wq4, x4)
    want["rms2"] = O.rms_norm16(mode_of("RMS_NORM", "norm-2"), xdec2, 1e-5)
    want["mul2"] = binop(L.lno16_mul_f32, want["rms2"], g2)
    want["mm2"] = O.mul_mat16(mode_of("MUL_MAT", "q-2"), O.f2x16(wlong), want["mul2"])

    # the decode row's three nodes run as one launch only in sum32; otherwise
    # the norm MUL is written and checked like the other nodes
    triple = mode_of("RMS_NORM", "norm-1") == O.SUM32 and mode_of("MUL_MAT", "qkv-2") == O.SUM32
    if fused and not triple:
        checked.append("mul1")
    report = {}
    for k in checked:
        got = h.f32_of(nodes[k], act).reshape(want[k].shape)
        bad = int(np.count_nonzero(got.view(np.uint32) != want[k].view(np.uint32)))
        report[k] = bad
    if act is None:   # fused away: host tensors never written (still zeros)
        for k in nodes.keys() - set(checked):
            report[k + "_written"] = int(np.count_nonzero(h.f32_of(nodes[k])))
    if O.MODES[mode_name] == O.MODES["monte"]:
        s = ctypes.c_uint16()
        h.lib.ggml_backend_lnship16_monte_get_state(ctypes.byref(s))
        report["monte_state_matches"] = int(s.value == O.monte_get())
    h.free(be)
    print(json.dumps({"mode": mode_name, "device_buffers": dev, "fused": fused, "mismatches": report}), flush=True)
    ok = all(v == 0 for k, v in report.items() if k != "monte_state_matches")
    return 0 if ok and report.get("monte_state_matches", 1) == 1 else 1


def run32(dev=False, fused=False):
    h = G.Host()
    rng = np.random.default_rng(99)
    f32 = lambda *s, scale=1.0: (rng.standard_normal(s) * scale).astype(np.float32)
    T, K, M, D, H = 2, 2048, 512, 64, 4
    x = f32(T, K)
    g = f32(K, scale=0.1) + 1.0
    w = f32(M, K, scale=0.02)
    kq = f32(4, T, 200, scale=3.0)
    mask = np.zeros((T, 200), np.float32)
    mask[0, 150:] = -np.inf
    res = f32(T, M)
    qk = f32(T, H, D)
    pos = np.array([7, 300], np.int32)
    wmoe = f32(4, 40, 256, scale=0.05)
    xmoe = f32(T, 2, 256)
    ids_moe = np.array([[3, 0], [1, 1]], np.int32)
    act = h.device_buffer(32 << 20, w32=True) if dev else None
    t = lambda *a, **k: h.tensor(*a, device=act, **k)
    X = t([K, T], data=x, name="inp")
    Gw = t([K], data=g, name="blk.0.attn_norm.weight")
    W = t([K, M], data=w, weights=True, name="blk.0.ffn_up.weight")
    KQ = t([200, T, 4], data=kq, name="kq")
    MASK = t([200, T], data=mask, name="kq_mask")
    RES = t([M, T], data=res, name="res")
    QK = t([D, H, T], data=qk, name="q")
    POS = t([T], "i32", data=pos, name="inp_pos")
    WMOE = t([256, 40, 4], data=wmoe, weights=True, name="blk.0.ffn_up_exps.weight")
    XMOE = t([256, 2, T], data=xmoe, name="ffn_moe_inp")
    IDS = t([2, T], "i32", data=ids_moe, name="ffn_moe_topk")
    swi = h.stub.ggml_host_glu(b"SWIGLU")
    nodes = {"rms": t([K, T], op="RMS_NORM", src=(X,), fparams={0: 1e-6}, name="norm-0")}
    nodes["mul"] = t([K, T], op="MUL", src=(nodes["rms"], Gw), name="attn_norm-0")
    nodes["mm"] = t([M, T], op="MUL_MAT", src=(W, nodes["mul"]), name="ffn_up-0")
    nodes["add"] = t([M, T], op="ADD", src=(nodes["mm"], RES), name="ffn_out-0")
    nodes["swiglu"] = t([M // 2, T], op="GLU", src=(nodes["add"],), params=(swi, 0), name="ffn_swiglu-0")
    nodes["rope"] = t([D, H, T], op="ROPE", src=(QK, POS), params=(0, D, 0),
                      fparams={5: 10000.0, 6: 1.0, 7: 0.0, 8: 1.0}, name="Qcur-0")
    nodes["softmax"] = t([200, T, 4], op="SOFT_MAX", src=(KQ, MASK), fparams={0: 0.125, 1: 0.0}, name="sm-0")
    nodes["moe"] = t([40, 2, T], op="MUL_MAT_ID", src=(WMOE, XMOE, IDS), name="ffn_moe_up-0")
    checked = mark_outputs(nodes, fused)
    be = h.init(w32=True)
    if be is None:
        print(json.dumps({"error": "no GPU: LNSHIP32 init returned NULL"}))
        return 1
    assert h.compute(be, list(nodes.values())) == 0
    want = {"rms": O.rms_norm32(x, 1e-6)}
    want["mul"] = O.mul32(want["rms"], g)
    want["mm"] = O.mul_mat32(w, want["mul"])
    want["add"] = O.add32(want["mm"], res)
    want["swiglu"] = O.swiglu32(want["add"][:, :M // 2], want["add"][:, M // 2:])
    want["rope"] = O.rope32(qk, pos, D, 0, 10000.0)
    want["softmax"] = O.soft_max32(kq, mask, 0.125)
    want["moe"] = O.mul_mat_id(None, wmoe, xmoe, ids_moe)
    report = {}
    for k in checked:
        got = h.f32_of(nodes[k], act).reshape(want[k].shape)
        report[k] = int(np.count_nonzero(got.view(np.uint32) != want[k].view(np.uint32)))
    if act is None:   # fused away: host tensors never written (still zeros)
        for k in nodes.keys() - set(checked):
            report[k + "_written"] = int(np.count_nonzero(h.f32_of(nodes[k])))
    h.free(be)
    print(json.dumps({"mode": "lns32", "device_buffers": dev, "fused": fused, "mismatches": report}), flush=True)
    return 0 if all(v == 0 for v in report.values()) else 1


def run_movement(w32=False):
    """SCALE and the data movement of a device-resident graph (CPY, CONT,
    GET_ROWS, SET_ROWS) with every tensor in the HBM buffer type except the
    host-side tables and indices named below; expected values from numpy
    (no LNS arithmetic) and, for SCALE, the oracle."""
    h = G.Host()
    rng = np.random.default_rng(5)
    f32 = lambda *s: rng.standard_normal(s).astype(np.float32)
    act = h.device_buffer(16 << 20, w32=w32)
    t = lambda *a, **k: h.tensor(*a, device=act, **k)
    x = f32(3, 64)
    X = t([64, 3], data=x, name="x")
    nodes, want, f16 = {}, {}, set()

    # llama.cpp's KV write: set_rows(cache view [128, 32], k_cur [128, 3], k_idxs i64 [3])
    kcur = f32(3, 128)
    cache = np.zeros((32, 128), np.float16)
    KCUR = t([128, 3], data=kcur, name="k_cur")
    CACHE = t([128, 32], "f16", data=cache, name="cache_k_l0")
    idx = np.array([5, 17, 30], np.int64)
    IDX = t([3], "i64", data=idx, name="k_idxs")
    nodes["set_rows"] = t([128, 32], "f16", op="SET_ROWS", src=(KCUR, IDX), data=CACHE.data, name="k_stored")
    c = cache.copy()
    c[idx] = kcur.astype(np.float16)
    want["set_rows"], f16 = c, f16 | {"set_rows"}
    # F32 destination, indices in host memory (int32), broadcast over slices
    vs = f32(4, 3, 16)
    VS = t([16, 3, 4], data=vs, name="v_src")
    VD = t([16, 10, 4], data=np.zeros((4, 10, 16), np.float32), name="v_dst")
    vid = np.array([[9, 0, 4], [1, 2, 3]], np.int32)
    VID = h.tensor([3, 2], "i32", data=vid, name="v_idxs")
    nodes["set_rows_bcast"] = t([16, 10, 4], op="SET_ROWS", src=(VS, VID), data=VD.data, name="v_stored")
    d = np.zeros((4, 10, 16), np.float32)
    for i03 in range(4):
        for r in range(3):
            d[i03, vid[i03 % 2, r]] = vs[i03, r]
    want["set_rows_bcast"] = d

    # the older KV write: CPY of F32 rows into an F16 cache view at row 7
    cache2 = np.zeros((32, 64), np.float16)
    CACHE2 = t([64, 32], "f16", data=cache2, name="cache_v_l0")
    nodes["cpy_f16"] = t([64, 3], "f16", op="CPY", src=(X,), data=CACHE2.data + 7 * 64 * 2,
                         nb=[2, 128, 128 * 3, 128 * 3], name="v_view")
    want["cpy_f16"] = x.astype(np.float16)
    f16 |= {"cpy_f16"}
    # CONT of a permuted view; CPY from a host tensor; CPY F16 -> F32
    XT = t([3, 64], op="PERMUTE", src=(X,), data=X.data, nb=[256, 4, 768, 768], name="x_t")
    nodes["cont"] = t([3, 64], op="CONT", src=(XT,), name="x_t_cont")
    want["cont"] = np.ascontiguousarray(x.T)
    xh = f32(2, 40)
    XH = h.tensor([40, 2], data=xh, name="host_rows")
    nodes["cpy_host_src"] = t([40, 2], "f16", op="CPY", src=(XH,), name="host_rows_f16")
    want["cpy_host_src"], f16 = xh.astype(np.float16), f16 | {"cpy_host_src"}
    hv = (f32(5, 12) * 4).astype(np.float16)
    HV = t([12, 5], "f16", data=hv, name="half_vals")
    nodes["cpy_f16_f32"] = t([12, 5], op="CPY", src=(HV,), name="half_vals_f32")
    want["cpy_f16_f32"] = hv.astype(np.float32)

    # GET_ROWS: F16 table in HBM with device ids; host F32 and Q8_0 tables;
    # a 3-D gather (ids [4, 3] over three table slices)
    tab16 = (f32(50, 64) * 0.5).astype(np.float16)
    TAB16 = t([64, 50], "f16", data=tab16, name="tab16")
    gid = np.array([49, 0, 7, 7], np.int32)
    GID = t([4], "i32", data=gid, name="inp_out_ids")
    nodes["get_rows_f16"] = t([64, 4], op="GET_ROWS", src=(TAB16, GID), name="rows16")
    want["get_rows_f16"] = tab16[gid].astype(np.float32)
    tab = f32(50, 64)
    TAB = h.tensor([64, 50], data=tab, weights=True, name="token_embd.weight")
    GIDH = h.tensor([4], "i32", data=gid, name="inp_tokens")
    nodes["get_rows_host"] = t([64, 4], op="GET_ROWS", src=(TAB, GIDH), name="inp_embd")
    want["get_rows_host"] = tab[gid]
    q8raw, q8 = q8_0(f32(50, 64), rng)
    TABQ = h.tensor([64, 50], "q8_0", data=q8raw, weights=True, name="token_embd_q8.weight")
    nodes["get_rows_q8"] = t([64, 4], op="GET_ROWS", src=(TABQ, GID), name="inp_embd_q8")
    want["get_rows_q8"] = q8[gid]
    tab3 = f32(3, 10, 16)
    TAB3 = t([16, 10, 3], data=tab3, name="tab3")
    gid3 = np.array([[0, 9, 3, 3], [1, 1, 2, 8], [5, 4, 0, 9]], np.int32)
    GID3 = t([4, 3], "i32", data=gid3, name="ids3")
    nodes["get_rows_3d"] = t([16, 4, 3], op="GET_ROWS", src=(TAB3, GID3), name="rows3")
    want["get_rows_3d"] = np.stack([tab3[s][gid3[s]] for s in range(3)])

    # SCALE in the backend's arithmetic
    nodes["scale"] = t([64, 3], op="SCALE", src=(X,), fparams={0: 0.125, 1: 0.0}, name="kq_scaled")
    want["scale"] = O.scale(w32, x, 0.125)
    nodes["scale_bias"] = t([64, 3], op="SCALE", src=(X,), fparams={0: 1.5, 1: 0.25}, name="scaled_biased")
    want["scale_bias"] = O.scale(w32, x, 1.5, 0.25)

    be = h.init(w32=w32)
    if be is None:
        print(json.dumps({"error": "no GPU: init returned NULL"}))
        return 1
    assert h.compute(be, [XT] + list(nodes.values())) == 0
    report = {}
    for k, tn in nodes.items():
        if k in f16:
            got = act.get(tn, want[k].size * 2).view(np.float16).reshape(want[k].shape)
            report[k] = int(np.count_nonzero(got.view(np.uint16) != want[k].view(np.uint16)))
        else:
            got = h.f32_of(tn, act).reshape(want[k].shape)
            report[k] = int(np.count_nonzero(got.view(np.uint32) != want[k].view(np.uint32)))
    h.free(be)
    print(json.dumps({"mode": "movement32" if w32 else "movement16", "mismatches": report}), flush=True)
    return 0 if all(v == 0 for v in report.values()) else 1


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--mode", default="base")
    ap.add_argument("--w32", action="store_true")
    ap.add_argument("--policy", default=None)
    ap.add_argument("--device-buffers", action="store_true")
    ap.add_argument("--movement", action="store_true", help="SCALE and the data-movement ops (HBM buffers)")
    ap.add_argument("--fused", action="store_true",
                    help="leave RMS_NORM -> MUL and MUL_MAT -> ADD intermediates unflagged, so the pairs fuse")
    a = ap.parse_args()
    if a.policy is not None:
        os.environ["LNS16_SUM_POLICY"] = a.policy
    if a.fused:   # node-pair fusion is opt-in
        os.environ["GGML_LNS_HIP_FUSE"] = "1"
    if a.device_buffers or a.movement:
        os.environ["GGML_LNS_HIP_BUFFERS"] = "device"
    if a.movement:
        sys.exit(run_movement(a.w32))
    sys.exit(run32(a.device_buffers, a.fused) if a.w32 else run16(a.mode, a.policy, a.device_buffers, a.fused))
