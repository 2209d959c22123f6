"""Benchmark: SmolLM2-135M-shape LNS16 decoder on one MI355X.

Workload: 30 layers, d_model 576, 9 / 3 heads of 64, SwiGLU 1536, vocab 49152,
random-init N(0, 0.02) weights stored as xlns16, LNS16 sum32 mode; a
128-token uniform-random prompt, then greedy decode.  A step is one decoded
token (the whole graph: 271 mul_mats, 61 rms_norms, 30 soft_maxes and the
elementwise ops), replayed from a captured HIP graph; the next token is the
device-side argmax, so the timed loop never waits for the host.

Prints one JSON line with decode tok/s (value), prefill tok/s, weight
mul_mat GMAC/s, the roofline of the dominant kernel (the decode GEMV) and the
single-threaded CPU oracle timed on this host on a bounded sample.  The line
also carries BASELINE config 5's prefill GEMM (prefill_gemm: GMAC/s in sum32
and base against the VALU-issue roofline, parity and the oracle's rate on a
slice of it), config 3 (c3: 8 sequences x 256-token prompts, batched decode
in monte and lpvip) and config 4 (c4: the LNS32 1B-shape decoder).
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "xlns-ggml-backend_amd"))

METRIC = "LNS16 mul_mat GMAC/s (sum32) + tok/s prefill/decode, SmolLM2-135M shape"
HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=120)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--mode", default="sum32", choices=["base", "monte", "lpvip", "sum32", "all"])
    ap.add_argument("--prompt", type=int, default=None, help="prompt tokens (128; 512 with --lns32)")
    ap.add_argument("--cpu-tokens", type=int, default=3, help="decode tokens of the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill-gemm", action="store_true",
                    help="leave BASELINE config 5's GEMM (GMAC/s, sum32 and base) out of the default line")
    ap.add_argument("--no-configs", action="store_true",
                    help="leave BASELINE configs 3 (monte and lpvip, 8 sequences) and 4 (LNS32 1B shape) out of the "
                         "default line")
    ap.add_argument("--no-graph", action="store_true", help="decode eagerly instead of replaying a HIP graph")
    ap.add_argument("--split-attn", action="store_true",
                    help="run a decode step's kq, soft_max and kqv as three launches (not one fused attention)")
    ap.add_argument("--split-rope", action="store_true",
                    help="LNS16 decode: the query rope and the cache stores as a launch of their own, apart from the "
                         "fused attention")
    ap.add_argument("--split-rms", action="store_true",
                    help="decode: rms_norm + MUL (sum32) and swiglu as launches of their own, apart from the "
                         "mul_mat after them")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the prompt and the decode steps, then one recorded eager step: prints the decode "
                         "launches' algorithmic bytes (for HBM counter runs; with --prompt 1 every lnship16_mul_mat "
                         "launch of the run is a decode-step launch)")
    ap.add_argument("--calib-copy", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB three times (HBM counter calibration)")
    ap.add_argument("--ops", choices=["decode", "prefill", "all"],
                    help="only time single ops (decode GEMVs, C5 prefill GEMM / rms_norm / soft_max), one JSON "
                         "line each, in --mode (or every mode with --mode all)")
    ap.add_argument("--reps", type=int, default=5, help="launches timed per op with --ops")
    ap.add_argument("--batch", type=int, default=1, metavar="S",
                    help="BASELINE config 3: S independent sequences, each prompt prefilled on its own, then "
                         "batched greedy decode (one token per sequence per step); prints its own JSON line")
    ap.add_argument("--ggml", action="store_true",
                    help="the PCIe-inclusive rate of the ggml boundary: BASELINE config 1 ops through graph_compute "
                         "on host buffers next to the same ops on HBM-resident data; prints its own JSON line")
    ap.add_argument("--lns32", action="store_true",
                    help="BASELINE config 4: the LNS32 1B-shape decoder (prompt defaults to 512 tokens); prints its "
                         "own JSON line")
    args, rest = ap.parse_known_args()
    if rest:
        ap.error("unrecognized arguments: %s" % " ".join(rest))
    return args


def _ops_modes(mode):
    return ["base", "sum32", "monte", "lpvip"] if mode == "all" else [mode]


def run_ops(args):
    """Per-op timings on synthetic data (HIP events around back-to-back
    launches on the current stream).  GEMVs report ns per dependent step,
    K steps per output chain; C5 reports GMAC/s."""
    import torch
    import lnship
    torch.cuda.set_device(0)
    lnship.init()
    gen = torch.Generator(device="cuda").manual_seed(0)
    randn = lambda *s: torch.randn(*s, device="cuda", generator=gen)

    def timed(fn, reps):
        fn()
        torch.cuda.synchronize()
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(reps):
            fn()
        e.record()
        e.synchronize()
        return s.elapsed_time(e) * 1e3 / reps

    def line(**kw):
        print(json.dumps(kw), flush=True)

    if args.ops in ("decode", "all"):
        line(op="chain_floor", **chain_floor(lnship, torch))
        # LNS32 (xlns32 weights, 4 B each) at the Llama-1B shape of BASELINE
        # config 4: q / o, k / v, gate|up, down, lm_head
        for K, M in ((2048, 2048), (2048, 512), (2048, 16384), (8192, 2048), (2048, 32000)):
            wp = lnship.pack32(randn(M, K) * 0.02)
            x = randn(1, K)
            us = timed(lambda: lnship.mul_mat32(wp, x, K, M), args.reps)
            line(op="mul_mat", mode="lns32", K=K, M=M, N=1, us=round(us, 2), ns_per_step=round(us * 1e3 / K, 2),
                 gbs=round((4 * K * M + 4 * K + 4 * M) / us / 1e3, 3))
        x = randn(1, 2048)
        us = timed(lambda: lnship.rms_norm32(x, 1e-5), args.reps)
        line(op="rms_norm", mode="lns32", rows=1, n=2048, us=round(us, 2), ns_per_step=round(us * 1e3 / 2048, 2))
    for mname in _ops_modes(args.mode):
        m = lnship.MODES[mname]
        if args.ops in ("decode", "all"):
            # SmolLM2 decode shapes: qkv, o, up|gate, down, lm_head
            for K, M in ((576, 960), (576, 576), (576, 3072), (1536, 576), (576, 49152)):
                wp = lnship.pack16(randn(M, K) * 0.02)
                x = randn(1, K)
                us = timed(lambda: lnship.mul_mat16(m, wp, x, K, M), args.reps)
                line(op="mul_mat", mode=mname, K=K, M=M, N=1, us=round(us, 2), ns_per_step=round(us * 1e3 / K, 2),
                     gbs=round((2 * K * M + 4 * K + 4 * M) / us / 1e3, 3))
            x = randn(1, 576)
            us = timed(lambda: lnship.rms_norm16(m, x, 1e-5), args.reps)
            line(op="rms_norm", mode=mname, rows=1, n=576, us=round(us, 2), ns_per_step=round(us * 1e3 / 576, 2))
        if args.ops in ("prefill", "all"):
            K, M, T = 2048, 8192, 512
            wp = lnship.pack16(randn(M, K) * 0.02)
            x = randn(T, K)
            # a 5-25 ms launch: at least ten of them per figure
            us = timed(lambda: lnship.mul_mat16(m, wp, x, K, M), max(10, args.reps))
            line(op="mul_mat", mode=mname, K=K, M=M, N=T, us=round(us, 2), gmacs=round(K * M * T / us / 1e3, 2))
            x = randn(512, 2048)
            us = timed(lambda: lnship.rms_norm16(m, x, 1e-5), args.reps)
            line(op="rms_norm", mode=mname, rows=512, n=2048, us=round(us, 2))
            s = randn(32, 512, 512) * 3
            mask = torch.triu(torch.full((512, 512), float("-inf"), device="cuda"), 1)
            us = timed(lambda: lnship.soft_max16(m, s, mask, 0.125), args.reps)
            line(op="soft_max", mode=mname, heads=32, rows=512, n=512, us=round(us, 2))


def batch_measure(mode_name, S, prompt_n, warmup, steps, graph=True):
    """S sequences of the SmolLM2-shape model in one mode: each prompt_n-token
    prompt is prefilled on its own, then warmup + steps batched decode steps
    (one token per sequence; weight GEMVs see S columns, attention is batched
    over the sequences' own KV caches).  Every step replays one HIP graph
    (Monte ops read their LFSR start from a device state the graph advances).
    Returns decode tok/s over the timed steps, ms per step, prefill tok/s and
    the KV view length."""
    import numpy as np
    import torch
    import lnship
    from lnship import llama
    torch.cuda.set_device(0)
    lnship.init()
    cfg = llama.SMOLLM2_135M
    weights = llama.synthetic_weights(cfg, seed=1234, std=0.02)
    model = llama.LlamaLNS16(cfg, weights, mode=lnship.MODES[mode_name], n_seq=S)
    rng = np.random.default_rng(2024)
    prompts = [[int(t) for t in rng.integers(0, cfg.n_vocab, prompt_n)] for _ in range(S)]
    torch.cuda.synchronize()
    tp = time.perf_counter()
    first = [model.eval(prompts[s], seq=s).argmax() for s in range(S)]
    torch.cuda.synchronize()
    t_prefill = time.perf_counter() - tp
    tok_dev = torch.stack(first).to(torch.int32)

    def step():
        nonlocal tok_dev
        out = model.decode_graph_batch(tok_dev) if graph else model.eval_batch(tok_dev.tolist())
        tok_dev = out.argmax(dim=1).to(torch.int32)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    ts = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    t_decode = time.perf_counter() - ts
    res = {"decode_tok_s": round(S * steps / t_decode, 3), "ms_per_step": round(t_decode / steps * 1e3, 4),
           "prefill_tok_s": round(S * prompt_n / t_prefill, 3), "n_kv": model.batch_n_kv()}
    del model
    torch.cuda.empty_cache()
    return res


def run_batch(args):
    """BASELINE config 3 on its own line (--batch S): batch_measure in --mode."""
    S = args.batch
    r = batch_measure(args.mode, S, args.prompt, args.warmup, args.steps, graph=not args.no_graph)
    print(json.dumps({
        "metric": "LNS16 batched decode tok/s, %d sequences, SmolLM2-135M shape" % S,
        "value": r["decode_tok_s"], "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": r["ms_per_step"], "higher_is_better": True,
        "dtype": "xlns16", "data": "synthetic (as the default workload)",
        "config": {"workload": "BASELINE config 3: %d x %d-token prompts, then batched greedy decode" % (S, args.prompt),
                   "mode": args.mode, "sequences": S, "n_kv": r["n_kv"],
                   "graph": "eager" if args.no_graph else "hipGraph per decode step"},
        "prefill_tok_s": r["prefill_tok_s"]}), flush=True)


def calib_copy(mib):
    """A plain device-to-device copy of known size: what FETCH_SIZE / WRITE_SIZE
    read for it scales the same counters read for the LNS kernels."""
    import torch
    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calib": "copy", "bytes_read": n * 4, "bytes_written": n * 4}), flush=True)


def replay_call(model, ln, torch, call):
    """Launches one recorded GEMV call again on the current stream."""
    w, x_ptr, dst_ptr, K, M, N, kw = call
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if "norm" in kw:
        ln.check(ln.lib().lnship16_rms_norm_mul_mat(model.mode, x_ptr, kw["norm"], model.cfg.eps, ctypes.c_void_p(w),
                                                    dst_ptr, K, M, st))
    elif "glu_up" in kw:
        ln.check(ln.lib().lnship16_swiglu_mul_mat(model.mode, x_ptr, kw["glu_up"], ctypes.c_void_p(w),
                                                  kw["residual"], dst_ptr, K, M, st))
    elif "pre" in kw:
        # lnship16_mul_mat with the node before it in its launch
        p = kw["pre"]
        a = ln.MulMatArgs(w, x_ptr, dst_ptr, K, M, N, 1, 1, 1, 1, p["x_ld"], 0, 7, 0, 0, 0, 0, None, 0,
                          kw["residual"])
        if p["rms_w"] is not None:
            a.rms_norm_w, a.rms_eps, a.rms_seed = p["rms_w"], model.cfg.eps, 7
        else:
            a.glu_up = p["glu_up"]
        ln.check(ln.lib().lnship16_mul_mat(model.mode, ctypes.byref(a), st))
    else:
        ln.mul_mat16_raw(model.mode, w, x_ptr, dst_ptr, K, M, N, seed=7, stream=st, **kw)


def gemv_roofline(model, ln, torch, reps=4):
    """Records the GEMV launches of one eager decode step, captures them
    `reps` times over into one HIP graph and times a replay between two HIP
    events on the replay stream.  Returns (algorithmic bytes per launch,
    average launch us, launches per token); a launch is one lnship16_mul_mat
    call (one k_mm16 kernel when its activation rows fit in LDS next to the
    tables, as at every decode shape) or one lnship16_rms_norm_mul_mat call
    (one k_mm16_rms kernel: the rms_norm before the GEMV runs inside it)."""
    calls = record_decode_step(model, torch)
    # the launches go into one HIP graph so host-side launch cost stays out
    # of the device time between the events
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            for call in calls:
                replay_call(model, ln, torch, call)
    g.replay()
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    s.record()
    g.replay()
    e.record()
    e.synchronize()
    n = len(calls)
    total_us = s.elapsed_time(e) * 1e3 / reps
    return launch_bytes(calls) / n, total_us / n, n


def record_decode_step(model, torch):
    """Runs one eager decode step at the last timed position (its KV row is
    rewritten; nothing reads it afterwards), so the launches have the timed
    steps' shapes, and returns its GEMV calls: lnship16_mul_mat's, and
    lnship16_rms_norm_mul_mat's with the norm row as kw["norm"]."""
    c = model.cfg
    calls = []
    orig, orig_rms, orig_glu, orig_pre = model._mm, model._rms_mm, model._glu_mm, model._mm_pre

    def record_mm(w, x_ptr, dst_ptr, K, M, N, **kw):
        orig(w, x_ptr, dst_ptr, K, M, N, **kw)
        calls.append((w, x_ptr, dst_ptr, K, M, N, kw))

    def record_rms_mm(x_ptr, wn_ptr, w, h_ptr, dst_ptr, K, M, T, step=False):
        # split or with the prologue: records through record_mm / record_pre
        orig_rms(x_ptr, wn_ptr, w, h_ptr, dst_ptr, K, M, T, step=step)
        if T == 1 and model.fused_rms:
            calls.append((w, x_ptr, dst_ptr, K, M, 1, {"norm": wn_ptr}))

    def record_glu_mm(gate_ptr, up_ptr, w, resid_ptr, dst_ptr, K, M):
        orig_glu(gate_ptr, up_ptr, w, resid_ptr, dst_ptr, K, M)
        calls.append((w, gate_ptr, dst_ptr, K, M, 1, {"glu_up": up_ptr, "residual": resid_ptr}))

    def record_pre(w, x_ptr, dst_ptr, K, M, N, rms_w=None, glu_up=None, residual=None, x_ld=0):
        ok = orig_pre(w, x_ptr, dst_ptr, K, M, N, rms_w=rms_w, glu_up=glu_up, residual=residual, x_ld=x_ld)
        if ok:
            calls.append((w, x_ptr, dst_ptr, K, M, N,
                          {"pre": {"rms_w": rms_w, "glu_up": glu_up, "x_ld": x_ld}, "residual": residual}))
        return ok

    model._mm, model._rms_mm, model._glu_mm, model._mm_pre = record_mm, record_rms_mm, record_glu_mm, record_pre
    try:
        tok = model._buf("rtok", 1, torch.int32)
        pos = model._buf("rpos", 1, torch.int32)
        tok.fill_(1)
        pos.fill_(model.n_past - 1)
        from lnship.llama import n_kv_for
        model.forward(1, tok, pos, n_kv_for(model.n_past, c.n_ctx))
        torch.cuda.synchronize()
    finally:
        model._mm, model._rms_mm, model._glu_mm, model._mm_pre = orig, orig_rms, orig_glu, orig_pre
    return calls


def launch_bytes(calls):
    """Algorithmic bytes of GEMV calls: xlns16 weights once per weight
    slice, F32 in / out, the F32 residual read by the launches that fuse the
    ADD after them, the F32 norm row read by those that fuse the rms_norm
    before them, and the F32 up row read by those that fuse the swiglu
    before them."""
    return sum(2 * K * M * kw.get("ne02", 1) + 4 * K * N * kw.get("ne12", 1)
               + 4 * M * N * kw.get("ne12", 1) * (2 if kw.get("residual") is not None else 1)
               + (4 * K if "norm" in kw or "glu_up" in kw or "pre" in kw else 0)
               for _, _, _, K, M, N, kw in calls)


def chain_bound(model, ln, torch, mode):
    """The dependent-step bound of one decode token.  steps: the sum over the
    token's launches of their chain length (K per mul_mat, n per rms_norm row,
    n - 1 per soft_max row; head_dim + 2 n_kv - 1 for the fused decode
    attention, whose KQ, soft_max and KQV chains run one after another; K
    for a fused rms_norm + mul_mat, whose rms chain runs beside the GEMV's);
    a launch's chains run side by side and the launches one after another.  ns_per_step: the slope of GEMV launch time
    against K at M = 576 (K = 576 and 1536, each a graph of 20 launches timed
    between HIP events on the replay stream), so each launch's fixed cost
    stays out of it.  bound_tok_s = 1 / (steps * ns_per_step)."""
    c = model.cfg
    steps = []
    orig = (model._mm, model._rms_mul, model._softmax, model._attn, model._rms_mm, model._glu_mm, model._mm_pre)

    def mm(w, x_ptr, dst_ptr, K, M, N, **kw):
        steps.append(K)
        orig[0](w, x_ptr, dst_ptr, K, M, N, **kw)

    def rms(x_ptr, w_ptr, dst_ptr, ncols, nrows):
        steps.append(ncols)
        orig[1](x_ptr, w_ptr, dst_ptr, ncols, nrows)

    def sm(x_ptr, ne, mask_ptr, mne, scale, dst_ptr):
        steps.append(ne[0] - 1)
        orig[2](x_ptr, ne, mask_ptr, mne, scale, dst_ptr)

    def attn(args, store=None):
        steps.append(args.head_dim + 2 * args.n_kv - 1)
        if store is None:
            orig[3](args)
        else:
            orig[3](args, store)

    def rms_mm(x_ptr, wn_ptr, w, h_ptr, dst_ptr, K, M, T, step=False):
        if T == 1 and model.fused_rms:
            steps.append(K)
        # split: counted by rms and mm; with the prologue by pre
        orig[4](x_ptr, wn_ptr, w, h_ptr, dst_ptr, K, M, T, step=step)

    def pre(w, x_ptr, dst_ptr, K, M, N, rms_w=None, glu_up=None, residual=None, x_ld=0):
        # the rms chain, then the GEMV's (the scale is not predicted here)
        ok = orig[6](w, x_ptr, dst_ptr, K, M, N, rms_w=rms_w, glu_up=glu_up, residual=residual, x_ld=x_ld)
        if ok:
            steps.append(2 * K if rms_w is not None else K)
        return ok

    def glu_mm(gate_ptr, up_ptr, w, resid_ptr, dst_ptr, K, M):
        steps.append(K)
        orig[5](gate_ptr, up_ptr, w, resid_ptr, dst_ptr, K, M)

    (model._mm, model._rms_mul, model._softmax, model._attn, model._rms_mm, model._glu_mm,
     model._mm_pre) = (mm, rms, sm, attn, rms_mm, glu_mm, pre)
    try:
        tok = model._buf("rtok", 1, torch.int32)
        pos = model._buf("rpos", 1, torch.int32)
        tok.fill_(1)
        pos.fill_(model.n_past - 1)   # the last timed position again (its KV row is rewritten)
        from lnship.llama import n_kv_for
        model.forward(1, tok, pos, n_kv_for(model.n_past, c.n_ctx))
        torch.cuda.synchronize()
    finally:
        (model._mm, model._rms_mul, model._softmax, model._attn, model._rms_mm, model._glu_mm,
         model._mm_pre) = orig
    st = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    us = {}
    M = 576
    for K in (576, 1536):
        g0 = torch.Generator(device="cpu").manual_seed(K)
        wp = ln.pack16((torch.randn(M, K, generator=g0) * 0.02).cuda())
        x = torch.randn(1, K, generator=g0).cuda()
        y = torch.empty(1, M, device="cuda")
        launch = lambda: ln.mul_mat16_raw(ln.MODES[mode], wp.data_ptr(), x.data_ptr(), y.data_ptr(), K, M, 1,
                                          seed=7, stream=st())
        launch()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(20):
                launch()
        g.replay()
        s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s_ev.record()
        g.replay()
        e_ev.record()
        e_ev.synchronize()
        us[K] = s_ev.elapsed_time(e_ev) * 1e3 / 20
    ns_step = (us[1536] - us[576]) * 1e3 / (1536 - 576)
    total = sum(steps)
    floor = chain_floor(ln, torch)
    return {"steps_per_token": total, "ns_per_step": round(ns_step, 2),
            "launch_us_k576": round(us[576], 2), "launch_us_k1536": round(us[1536], 2),
            "bound_tok_s": round(1e9 / (total * ns_step), 3), "chain_launches_per_token": len(steps),
            "floor_ns": floor["two_lds_round_trips_add_ns"], "floor_frac": round(floor["two_lds_round_trips_add_ns"] / ns_step, 4),
            "floor": floor}


def chain_floor(ln, torch, steps=200000):
    """What gfx950 itself needs per dependent step on one wave
    (lnship_chain_probe, HIP events on the current stream): one and two
    dependent LDS round trips (a pointer chase), two round trips plus one
    dependent VALU op (the least an LNS addition can be: a table read whose
    value addresses a second one, then an add), and one dependent VALU op."""
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    out = {}
    for key, rt, v in (("lds_round_trip_ns", 1, 0), ("two_lds_round_trips_ns", 2, 0),
                       ("two_lds_round_trips_add_ns", 2, 1), ("dependent_valu_ns", 0, 8)):
        ns = ctypes.c_double()
        ln.check(ln.lib().lnship_chain_probe(rt, v, steps, st, ctypes.byref(ns)))
        out[key] = round(ns.value / (8 if key == "dependent_valu_ns" else 1), 3)
    return out


def measured_traffic(mode):
    """HBM bytes per decode mul_mat launch from the committed rocprofv3 PMC
    summary (FETCH_SIZE and WRITE_SIZE passes scaled by a plain copy), or None
    when no summary exists for this mode."""
    p = os.path.join(ROOT, "profiles", "k_mm16_decode_%s_traffic.json" % mode)
    try:
        with open(p) as f:
            d = json.load(f)
        return d["bytes_per_mul_mat"], os.path.relpath(p, ROOT)
    except (OSError, KeyError, ValueError):
        return None, None


def device_clock_ghz():
    """The device's peak engine clock (hipDeviceAttributeClockRate, kHz)."""
    hip = ctypes.CDLL("libamdhip64.so")
    v = ctypes.c_int()
    if hip.hipDeviceGetAttribute(ctypes.byref(v), 5, 0) != 0:   # 5 = hipDeviceAttributeClockRate
        return None
    return v.value / 1e6


def prefill_gemm(ln, torch, np, cpu=True, reps=10):
    """BASELINE config 5's GEMM (K 2048, M 8192 outputs, N 512 tokens, xlns16
    weights N(0, 0.02), activations N(0, 1)) in sum32 and base: mean launch
    time of `reps` back-to-back launches between HIP events on the launch
    stream, GMAC/s, and the VALU-issue roofline 256 CUs x peak clock x 64 lanes
    / VALU instructions per MAC (from the committed rocprofv3 counters).
    With cpu, the single-threaded C oracle is timed on a slice of the same
    product (256 rows x 8 tokens) and the GPU's outputs there are compared
    with its bit for bit."""
    K, M, T = 2048, 8192, 512
    gen = torch.Generator(device="cuda").manual_seed(5)
    w = torch.randn(M, K, device="cuda", generator=gen) * 0.02
    x = torch.randn(T, K, device="cuda", generator=gen)
    wp = ln.pack16(w)
    clock = device_clock_ghz()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    try:
        with open(os.path.join(ROOT, "profiles", "k_mm16_prefill_c5_valu.json")) as f:
            prof = json.load(f)
    except (OSError, ValueError):
        prof = {}
    out = {"workload": "mul_mat K=2048, M=8192, N=512 (BASELINE config 5), xlns16 weights N(0,0.02), "
                       "activations N(0,1), %d launches timed with HIP events" % reps,
           "macs_per_launch": K * M * T, "peak_clock_ghz": clock, "cus": cus}
    sample = None
    if cpu:
        sys.path.insert(0, os.path.join(ROOT, "tests"))
        import oracle_lib as O
        ms, ns = 512, 64
        w_codes = O.f2x16(w[:ms].cpu().numpy())
        x_s = np.ascontiguousarray(x[:ns].cpu().numpy())
    for mname in ("sum32", "base"):
        m = ln.MODES[mname]
        y = ln.mul_mat16(m, wp, x, K, M)
        torch.cuda.synchronize()
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(reps):
            ln.mul_mat16(m, wp, x, K, M)
        e.record()
        e.synchronize()
        us = s.elapsed_time(e) * 1e3 / reps
        gmacs = K * M * T / us / 1e3
        r = {"us_per_launch": round(us, 2), "gmacs": round(gmacs, 2)}
        vpm = prof.get(mname, {}).get("valu_per_mac")
        if vpm and clock:
            peak = cus * clock * 64 / vpm
            r["roofline"] = {"bound": "valu", "valu_per_mac": vpm, "peak_gmacs": round(peak, 1),
                             "frac": round(gmacs / peak, 4), "lds_busy": prof[mname].get("lds_busy"),
                             "lds_bank_conflict_rate": prof[mname].get("lds_bank_conflict_rate"),
                             "source": "profiles/k_mm16_prefill_c5_valu.json"}
        if cpu:
            with _one_core():
                t0 = time.perf_counter()
                want = O.mul_mat16(O.MODES[mname], w_codes, x_s)
                dt = time.perf_counter() - t0
            got = np.ascontiguousarray(y[:ns, :ms].cpu().numpy(), np.float32)
            r["cpu_baseline"] = {"value": round(ms * ns * K / dt / 1e9, 5), "unit": "GMAC/s", "cores": 1,
                                 "kind": "port", "sample": "%d rows x %d tokens of the same product, single-threaded "
                                                           "C oracle (%.2f s)" % (ms, ns, dt)}
            r["parity"] = {"bit_exact": bool(np.array_equal(got.view(np.uint32), want.view(np.uint32))),
                           "outputs": ms * ns}
        out[mname] = r
    return out


def cpu_baseline(cfg, weights, mode, n_tokens):
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O
    from llama_oracle import LlamaOracle16
    m = O.MODES[mode]
    cpu = LlamaOracle16(cfg, weights, m)
    with _one_core() as core:
        ref = [cpu.eval([1, 2])]
        t0 = time.perf_counter()
        tok = 3
        for _ in range(n_tokens):
            logits = cpu.eval([tok])
            ref.append(logits)
            tok = int(logits.argmax())
        dt = time.perf_counter() - t0
    return {"value": round(n_tokens / dt, 4), "unit": "tok/s", "cores": 1, "kind": "port",
            "sample": f"{n_tokens} decode tokens after a 2-token prompt, full SmolLM2-135M shape, "
                      f"{mode}, single-threaded C oracle pinned to core {core} ({dt:.1f} s)",
            "cpu": _cpu_name(), "nproc": len(os.sched_getaffinity(0))}, ref


def logits_parity(model, ref, torch, np):
    """The GPU model replays the CPU baseline's sample from position 0 (the
    2-token prompt, then each decode token from a HIP graph) and compares
    every logit with the oracle's, bit for bit."""
    model.restart()
    # the model returns its logits buffer: copy each step's before the next
    got = [model.eval([1, 2]).clone()]
    tok = 3
    for _ in ref[1:]:
        got.append(model.decode_graph(tok).clone())
        tok = int(torch.argmax(got[-1]))
    torch.cuda.synchronize()
    differ = 0
    for g, r in zip(got, ref):
        g = np.ascontiguousarray(g.cpu().numpy(), np.float32).view(np.uint32)
        differ += int(np.count_nonzero(g != np.ascontiguousarray(r, np.float32).view(np.uint32)))
    return {"bit_exact": differ == 0, "logits": sum(int(r.size) for r in ref), "differ": differ,
            "sample": "the cpu_baseline sample: logits of the 2-token prompt and of %d graph-replayed decode "
                      "tokens, GPU against the CPU oracle" % (len(ref) - 1)}


class _one_core:
    """Pins the calling thread to the first core it may run on (the oracle is
    single-threaded), and restores its affinity afterwards."""

    def __enter__(self):
        self.saved = os.sched_getaffinity(0)
        core = min(self.saved)
        os.sched_setaffinity(0, {core})
        return core

    def __exit__(self, *exc):
        os.sched_setaffinity(0, self.saved)
        return False


def _cpu_name():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              f"(multi-GPU sharding is a design note, not part of this build)", file=sys.stderr)
        sys.exit(2)
    if args.calib_copy:
        calib_copy(args.calib_copy)
        return
    if args.ops:
        run_ops(args)
        return
    if args.mode == "all":
        sys.exit("bench.py: --mode all is for --ops only")
    if args.ggml:
        run_ggml(args)
        return
    if args.lns32:
        run_lns32(args)
        return
    if args.prompt is None:
        args.prompt = 128
    if args.batch > 1:
        run_batch(args)
        return
    import numpy as np
    import torch
    import lnship
    from lnship import llama

    torch.cuda.set_device(0)
    lnship.init()
    cfg = llama.SMOLLM2_135M
    mode = lnship.MODES[args.mode]
    t0 = time.perf_counter()
    weights = llama.synthetic_weights(cfg, seed=1234, std=0.02)
    model = llama.LlamaLNS16(cfg, weights, mode=mode)
    model.fused_rms = model.fused_rms and not args.split_rms
    model.fused_glu = model.fused_glu and not args.split_rms
    model.fused_attn = model.fused_attn and not args.split_attn
    model.fused_rope = not args.split_rope
    torch.cuda.synchronize()
    t_setup = time.perf_counter() - t0

    rng = np.random.default_rng(2024)
    prompt = [int(t) for t in rng.integers(0, cfg.n_vocab, args.prompt)]
    # prefill (timed once; the first call pays the one-time kernel setup, so
    # run it on a scratch model state first)
    model.eval(prompt[:8])
    model.n_past = 0
    torch.cuda.synchronize()
    tp = time.perf_counter()
    logits = model.eval(prompt)
    torch.cuda.synchronize()
    t_prefill = time.perf_counter() - tp

    tok_dev = torch.argmax(logits).to(torch.int32).reshape(1)
    use_graph = not args.no_graph

    def step():
        nonlocal tok_dev
        if use_graph:
            out = model.decode_graph(tok_dev)
        else:
            out = model.eval([int(tok_dev.item())])
        tok_dev = torch.argmax(out).to(torch.int32).reshape(1)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ts = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t_decode = time.perf_counter() - ts

    decode_tok_s = args.steps / t_decode
    if args.decode_only:
        calls = record_decode_step(model, torch)
        print(json.dumps({"decode_only": True, "mode": args.mode, "prompt_tokens": args.prompt,
                          "decode_steps": args.warmup + args.steps + 1, "launches_per_token": len(calls),
                          "bytes_per_launch": int(launch_bytes(calls) / len(calls)),
                          "decode_tok_s": round(decode_tok_s, 3)}), flush=True)
        return
    macs_per_token = cfg.n_layer * (
        (cfg.n_head + 2 * cfg.n_head_kv) * cfg.head_dim * cfg.n_embd + cfg.n_embd * cfg.n_head * cfg.head_dim +
        3 * cfg.n_ff * cfg.n_embd) + cfg.n_vocab * cfg.n_embd
    b_launch, us_launch, n_launch = gemv_roofline(model, lnship, torch)
    achieved = b_launch / (us_launch * 1e-6) / 1e9
    chain = chain_bound(model, lnship, torch, args.mode)
    chain["frac"] = round(decode_tok_s / chain["bound_tok_s"], 4)
    traffic, traffic_src = measured_traffic(args.mode)
    out = {
        "metric": METRIC,
        "value": round(decode_tok_s, 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t_decode / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "xlns16",
        "data": "synthetic: splitmix64/Box-Muller N(0,0.02) weights stored as xlns16, uniform token ids",
        "config": {"workload": "SmolLM2-135M-shape decoder, LNS16 %s, %d-token prompt then greedy decode "
                               "(one decoded token per step)" % (args.mode, args.prompt),
                   "mode": args.mode, "prompt_tokens": args.prompt, "n_kv": llama.n_kv_for(model.n_past, cfg.n_ctx),
                   "graph": "hipGraph per decode step" if use_graph else "eager"},
        "prefill_tok_s": round(args.prompt / t_prefill, 3),
        "mul_mat_gmacs": round(macs_per_token * decode_tok_s / 1e9, 4),
        "weight_macs_per_token": macs_per_token,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 3), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 6), "traffic": traffic,
                     "traffic_source": traffic_src,
                     "kernel": "decode GEMV launches: lnship16_mul_mat (k_mm16<%s, NC=1>, activations converted "
                               "in-kernel; the down projections with the swiglu before them inside the launch "
                               "through lnship16_swiglu_mul_mat)%s" % (
                                   args.mode, " and lnship16_rms_norm_mul_mat (k_mm16_rms, the rms_norm before the "
                                              "GEMV inside it)" if model.fused_rms else ""),
                     "launches_per_token": n_launch, "avg_launch_us": round(us_launch, 3),
                     "bytes_per_launch": int(b_launch)},
        "chain_bound": chain,
        "reference_published": {"rtx2050_sum32_decode_tok_s": 7.31,
                                "source": "experiments/layer-by-layer/CPU-vs-GPU.md:21 (Q4_K_M, 5-token prompt)"},
        "setup_s": round(t_setup, 2),
    }
    if not args.no_cpu:
        out["cpu_baseline"], ref = cpu_baseline(cfg, weights, args.mode, args.cpu_tokens)
        out["parity"] = logits_parity(model, ref, torch, np)
        if not out["parity"]["bit_exact"]:
            print("bench.py: GPU logits differ from the CPU oracle's", file=sys.stderr)
    if not args.no_prefill_gemm:
        out["prefill_gemm"] = prefill_gemm(lnship, torch, np, cpu=not args.no_cpu)
    if not args.no_configs:
        del model
        torch.cuda.empty_cache()
        out["c3"] = other_configs_c3()
        out["c4"] = other_configs_c4()
    print(json.dumps(out), flush=True)


# BASELINE configs 3 and 4 in the default line, each at its named shape, with
# fewer timed decode steps than their own lines take by default
C3_SEQS, C3_PROMPT, C3_WARMUP, C3_STEPS = 8, 256, 1, 63
C4_PROMPT, C4_WARMUP, C4_STEPS = 512, 2, 24


def other_configs_c3():
    """8 independent 256-token prompts, each prefilled on
    its own, then 64 graph-replayed batched greedy decode steps (the first
    one untimed), in monte and lpvip."""
    res = {"workload": "BASELINE config 3: %d x %d-token prompts, prefill each, then %d batched greedy decode "
                       "steps (%d timed)" % (C3_SEQS, C3_PROMPT, C3_WARMUP + C3_STEPS, C3_STEPS),
           "sequences": C3_SEQS, "timed_steps": C3_STEPS, "unit": "tok/s (all sequences)"}
    for mode in ("monte", "lpvip"):
        res[mode] = batch_measure(mode, C3_SEQS, C3_PROMPT, C3_WARMUP, C3_STEPS)
    return res


def other_configs_c4():
    """the LNS32 1B-shape decoder, 512-token prompt, then
    graph-replayed greedy decode (the first C4_WARMUP + C4_STEPS tokens of
    its 256)."""
    r, _ = lns32_measure(C4_PROMPT, C4_WARMUP, C4_STEPS)
    r["workload"] = ("BASELINE config 4: LNS32 Llama-style 1B-shape decoder, %d-token prompt, then greedy decode "
                     "(%d timed steps)" % (C4_PROMPT, C4_STEPS))
    r["unit"] = "tok/s"
    return r


def run_ggml(args):
    """BASELINE config 1's ops through libggml-lnship.so's graph_compute, as
    llama.cpp drives the backend: host (CPU-buffer) tensors, so each call
    uploads its activations, runs the kernels and downloads the output (the
    weights are cached on the device after the first call, as the reference's
    weight cache does); then with the tensors in the backend's device buffer
    type; beside them, the same op on device-resident data through the C ABI.
    Median wall time of one synchronised call over --reps calls."""
    import numpy as np
    import torch
    os.environ.setdefault("GGML_LNS16_SUM", args.mode if args.mode != "all" else "sum32")
    os.environ["GGML_LNS_HIP_BUFFERS"] = "device"   # host tensors stay host; the device leg uses the HBM type
    mode_name = os.environ["GGML_LNS16_SUM"]
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import ggml_host as G
    import lnship
    torch.cuda.set_device(0)
    lnship.init()
    h = G.Host()
    be = h.init()
    rng = np.random.default_rng(7)
    reps = max(args.reps, 20)
    f32 = lambda *s_, scale=1.0: (rng.standard_normal(s_) * scale).astype(np.float32)
    res = []

    def wall(fn):
        # median wall time of one synchronised call (a stall in one call
        # does not move it)
        fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts)) * 1e6

    mode = lnship.MODES[mode_name]
    hbm = h.device_buffer(64 << 20)
    for (K, M) in ((576, 1536), (1536, 576)):
        w, x = f32(M, K, scale=0.02), f32(1, K)
        W = h.tensor([K, M], data=w, weights=True, name="w")
        X = h.tensor([K, 1], data=x, name="x")
        D = h.tensor([M, 1], op="MUL_MAT", src=(W, X), name="y")
        us_b = wall(lambda: h.compute(be, [D]))
        Xh = h.tensor([K, 1], data=x, name="x", device=hbm)
        Dh = h.tensor([M, 1], op="MUL_MAT", src=(W, Xh), name="y", device=hbm)
        us_h = wall(lambda: h.compute(be, [Dh]))
        wp, xd = lnship.pack16(torch.from_numpy(w).cuda()), torch.from_numpy(x).cuda()
        us_d = wall(lambda: lnship.mul_mat16(mode, wp, xd, K, M))
        res.append({"op": "mul_mat", "K": K, "M": M, "N": 1, "boundary_us": round(us_b, 2),
                    "boundary_hbm_us": round(us_h, 2), "device_us": round(us_d, 2), "pcie_bytes": 4 * (K + M),
                    "boundary_weight_gbs": round(2 * K * M / us_b / 1e3, 3)})
    x = f32(1, 576)
    X = h.tensor([576, 1], data=x, name="x")
    D = h.tensor([576, 1], op="RMS_NORM", src=(X,), fparams={0: 1e-5}, name="n")
    Xh = h.tensor([576, 1], data=x, name="x", device=hbm)
    Dh = h.tensor([576, 1], op="RMS_NORM", src=(Xh,), fparams={0: 1e-5}, name="n", device=hbm)
    xd = torch.from_numpy(x).cuda()
    res.append({"op": "rms_norm", "n": 576, "rows": 1, "boundary_us": round(wall(lambda: h.compute(be, [D])), 2),
                "boundary_hbm_us": round(wall(lambda: h.compute(be, [Dh])), 2),
                "device_us": round(wall(lambda: lnship.rms_norm16(mode, xd, 1e-5)), 2), "pcie_bytes": 8 * 576})
    z = f32(9, 128, 128, scale=3.0)
    Z = h.tensor([128, 128, 9], data=z, name="kq")
    D = h.tensor([128, 128, 9], op="SOFT_MAX", src=(Z,), fparams={0: 0.125, 1: 0.0}, name="p")
    Zh = h.tensor([128, 128, 9], data=z, name="kq", device=hbm)
    Dh = h.tensor([128, 128, 9], op="SOFT_MAX", src=(Zh,), fparams={0: 0.125, 1: 0.0}, name="p", device=hbm)
    zd = torch.from_numpy(z).cuda()
    res.append({"op": "soft_max", "ne": [128, 128, 9], "boundary_us": round(wall(lambda: h.compute(be, [D])), 2),
                "boundary_hbm_us": round(wall(lambda: h.compute(be, [Dh])), 2),
                "device_us": round(wall(lambda: lnship.soft_max16(mode, zd, None, 0.125)), 2),
                "pcie_bytes": 8 * z.size})
    h.free(be)
    print(json.dumps({"metric": "ggml boundary PCIe-inclusive latency per op (BASELINE config 1 shapes)",
                      "mode": mode_name, "reps": reps, "ops": res,
                      "note": "boundary_us: graph_compute wall time with host tensors (upload, kernels, download, "
                              "sync); boundary_hbm_us: graph_compute with the tensors in the backend's device buffer "
                              "type (GGML_LNS_HIP_BUFFERS=device); device_us: the same op on HBM-resident tensors "
                              "through the C ABI, wall time with launch"}), flush=True)


def lns32_weights(cfg, seed, std, torch):
    """Random-init weights of the architecture on the device (N(0, std^2),
    torch's seeded generator; norm weights ones)."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    e, f, d = cfg.n_embd, cfg.n_ff, cfg.head_dim
    nq, nkv = cfg.n_head * d, cfg.n_head_kv * d
    r = lambda *shape: torch.randn(*shape, generator=g, device="cuda") * std
    w = {"tok_embd": r(cfg.n_vocab, e), "out_norm": torch.ones(e, device="cuda"), "layers": []}
    for _ in range(cfg.n_layer):
        w["layers"].append({"attn_norm": torch.ones(e, device="cuda"), "wq": r(nq, e), "wk": r(nkv, e),
                            "wv": r(nkv, e), "wo": r(e, nq), "ffn_norm": torch.ones(e, device="cuda"),
                            "w_gate": r(f, e), "w_up": r(f, e), "w_down": r(e, f)})
    return w


def lns32_measure(prompt_n, warmup, steps, graph=True, split_attn=False):
    """the LNS32 backend's graph on a Llama-style 1B-shape
    decoder (16 layers, d 2048, 32 / 8 heads x 64, SwiGLU 8192, vocab 32000),
    random-init N(0, 0.02) weights packed as xlns32 (4 bytes per weight).
    Prefill of the prompt, then greedy decode from a replayed HIP graph.  The
    roofline is the decode's weight stream: every token reads each packed
    weight once.  Returns the figures and the weights (for the CPU leg)."""
    import numpy as np
    import torch
    import lnship
    from lnship import llama

    torch.cuda.set_device(0)
    lnship.init()
    cfg = llama.LLAMA_1B
    t0 = time.perf_counter()
    weights = lns32_weights(cfg, 4321, 0.02, torch)
    model = llama.LlamaLNS32(cfg, weights)
    model.fused_attn = model.fused_attn and not split_attn
    torch.cuda.synchronize()
    t_setup = time.perf_counter() - t0
    rng = np.random.default_rng(2024)
    prompt = [int(t) for t in rng.integers(0, cfg.n_vocab, prompt_n)]
    model.eval(prompt[:8])
    model.n_past = 0
    torch.cuda.synchronize()
    tp = time.perf_counter()
    logits = model.eval(prompt)
    torch.cuda.synchronize()
    t_prefill = time.perf_counter() - tp
    tok_dev = torch.argmax(logits).to(torch.int32).reshape(1)

    def step():
        nonlocal tok_dev
        out = model.decode_graph(tok_dev) if graph else model.eval([int(tok_dev.item())])
        tok_dev = torch.argmax(out).to(torch.int32).reshape(1)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    ts = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    t_decode = time.perf_counter() - ts
    tok_s = steps / t_decode
    wbytes = model.weight_bytes_per_token()
    achieved = wbytes * tok_s / 1e9
    res = {"decode_tok_s": round(tok_s, 3), "ms_per_step": round(t_decode / steps * 1e3, 4),
           "prefill_tok_s": round(prompt_n / t_prefill, 3), "n_kv": llama.n_kv_for(model.n_past, cfg.n_ctx),
           "weight_stream": {"achieved": round(achieved, 3), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                             "frac": round(achieved / HBM_PEAK_GBS, 6), "weight_bytes_per_token": wbytes},
           "setup_s": round(t_setup, 2)}
    del model
    torch.cuda.empty_cache()
    return res, weights


def run_lns32(args):
    """BASELINE config 4 on its own line (--lns32): lns32_measure, and the
    oracle's LNS32 graph timed on the host beside it."""
    from lnship import llama
    prompt_n = args.prompt if args.prompt is not None else 512
    r, weights = lns32_measure(prompt_n, args.warmup, args.steps, graph=not args.no_graph,
                               split_attn=args.split_attn)
    ws = r["weight_stream"]
    out = {
        "metric": "LNS32 decode tok/s and weight-stream HBM GB/s, 1B-shape Llama decoder",
        "value": r["decode_tok_s"], "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": r["ms_per_step"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "xlns32",
        "data": "synthetic: torch-seeded N(0,0.02) weights packed as xlns32, uniform token ids",
        "config": {"workload": "BASELINE config 4: LNS32 Llama-style 1B-shape decoder, %d-token prompt then "
                               "greedy decode (one decoded token per step)" % prompt_n,
                   "prompt_tokens": prompt_n, "n_kv": r["n_kv"],
                   "graph": "eager" if args.no_graph else "hipGraph per decode step"},
        "prefill_tok_s": r["prefill_tok_s"],
        "roofline": {"bound": "hbm", "achieved": ws["achieved"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": ws["frac"], "traffic": None,
                     "kernel": "whole decode token: xlns32 weights read once per token",
                     "weight_bytes_per_token": ws["weight_bytes_per_token"]},
        "setup_s": r["setup_s"],
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline_lns32(llama.LLAMA_1B, weights, __import__("torch"))
    print(json.dumps(out), flush=True)


def cpu_baseline_lns32(cfg, weights, torch):
    """The oracle's LNS32 graph at the 1B width on the host: one decode token
    after a 2-token prompt through the embedding, norm and output alone (t0)
    and through layer 0 as well (t1); a 16-layer token is t0 + 16 (t1 - t0)."""
    import dataclasses
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from llama_oracle import LlamaOracle32
    h = lambda t: t.detach().float().cpu().numpy()
    w1 = {"tok_embd": h(weights["tok_embd"]), "out_norm": h(weights["out_norm"]),
          "layers": [{k: h(v) for k, v in weights["layers"][0].items()}]}
    cfg1 = dataclasses.replace(cfg, n_layer=1)
    cpu = LlamaOracle32(cfg1, w1)
    times = []
    with _one_core() as core:
        for n_layers in (0, 1):
            cpu.n_past = 0
            cpu.eval([1, 2], n_layers=n_layers)
            t0 = time.perf_counter()
            cpu.eval([3], n_layers=n_layers)
            times.append(time.perf_counter() - t0)
    per_tok = times[0] + cfg.n_layer * (times[1] - times[0])
    return {"value": round(1.0 / per_tok, 5), "unit": "tok/s", "cores": 1, "kind": "port",
            "sample": "one decode token after a 2-token prompt at the 1B width, single-threaded C oracle "
                      "pinned to core %d: embedding + output %.2f s, plus layer 0 %.2f s; scaled to 16 layers" %
                      (core, times[0], times[1] - times[0]),
            "cpu": _cpu_name(), "nproc": len(os.sched_getaffinity(0))}


if __name__ == "__main__":
    main()
