"""CPU audit of the LNS32 decoder's launch arguments at a full context.

LlamaLNS32 (lnship/llama.py) builds every launch of a decode step from its
own buffers: the weights, both KV caches, the rope table, the causal mask
and the grow-only step buffers that a captured HIP graph keeps.  Here the
decoder is built on CPU tensors and the library is replaced by a recorder,
so nothing runs; each recorded call's footprint - the elements its entry
point reads and writes, as include/lnship.h states them for those arguments
- must lie inside one live allocation.  The steps audited are those of the
Llama-1B shape (head geometry, widths and n_ctx 1024 of BASELINE config 4,
two of its sixteen identical layers): a 512-token prompt, and decode steps
through decode_graph at n_past 1022 and 1023, where the KV view is the whole
cache (n_kv = n_ctx = 1024) and the last position is n_ctx - 1, with a
decode step's kq, soft_max and kqv as three launches and as one
lnship32_attn_decode launch.

The footprints are the kernels' own extents: k_mm32 / k_mm16 lanes of rows
m >= M return before any load, and weight / activation prefetches past the
last group of eight k reload that group (min(g, last)), so a mul_mat reads
no code beyond round8(K) of its rows.
"""
import ctypes
import dataclasses

import pytest
import torch

import lnship
from lnship import llama

F32 = 4


class Recorder:
    """Stands in for liblnship.so: records each call with copies of the
    argument structs it was passed by reference, and returns success."""

    def __init__(self):
        self.calls = []

    def __getattr__(self, name):
        if not name.startswith("lnship"):
            raise AttributeError(name)

        def call(*args):
            rec = []
            for a in args:
                obj = getattr(a, "_obj", None)   # ctypes.byref(struct)
                if obj is not None:
                    a = type(obj).from_buffer_copy(obj)
                elif isinstance(a, ctypes.c_void_p):
                    a = a.value or 0
                rec.append(a)
            self.calls.append((name, rec))
            if name == "lnship_max_row":
                return 1 << 20
            return 0
        return call


class _Graph:
    def replay(self):
        pass


def _ptr(v):
    return v.value if isinstance(v, ctypes.c_void_p) else (v or 0)


def footprints(name, a):
    """(pointer, bytes, what) for each buffer a call touches, from its
    arguments and the access pattern include/lnship.h documents."""
    out = []
    if name == "lnship32_pack":
        # the source is the caller's F32 weight (a temporary of the
        # constructor); the packed cache is what the decoder keeps
        src, src_is_f16, src_ld, src_slice, dst, K, M, ns = a[:8]
        out.append((dst, ns * lnship.kp(K) * M * 4, "pack dst"))
    elif name == "lnship32_rms_norm_mul":
        src, w, dst, ncols, nrows = a[:5]
        out += [(src, nrows * ncols * F32, "rms src"), (w, ncols * F32, "rms weight"),
                (dst, nrows * ncols * F32, "rms dst")]
    elif name == "lnship32_mul_mat":
        m = a[0]
        K, M, N = m.K, m.M, m.N
        kp = lnship.kp(K)
        wms = m.w_mstride or M
        wsl = m.w_slice or kp * wms
        # weight code (k, m) of a slice at ((k / 8) * w_mstride + m) * 8 + k % 8, k < round8(K)
        w_ext = (m.ne02 * m.ne03 - 1) * wsl + ((kp // 8 - 1) * wms + M) * 8
        x_ld = m.x_ld or K
        x_sl = m.x_slice or N * x_ld
        d_ld = m.dst_ld or M
        d_sl = m.dst_slice or N * d_ld
        ns = m.ne12 * m.ne13
        out += [(m.w, w_ext * 4, "mul_mat w"), (m.x, ((ns - 1) * x_sl + (N - 1) * x_ld + K) * F32, "mul_mat x"),
                (m.dst, ((ns - 1) * d_sl + (N - 1) * d_ld + M) * F32, "mul_mat dst")]
        if m.residual:
            out.append((m.residual, ((ns - 1) * d_sl + (N - 1) * d_ld + M) * F32, "mul_mat residual"))
        # the nodes before the product: the norm row (K floats), the up rows
        # laid out as x
        if m.rms_norm_w:
            out.append((m.rms_norm_w, K * F32, "mul_mat rms_norm_w"))
        if m.glu_up:
            out.append((m.glu_up, ((ns - 1) * x_sl + (N - 1) * x_ld + K) * F32, "mul_mat glu_up"))
    elif name == "lnship32_rope_store_kv":
        q = a[0]
        hd, nh, nkv = q.head_dim, q.n_head, q.n_head_kv
        p_max = q.cache_m - 1   # positions are checked against n_ctx = cache_m on the host and the device
        out += [(q.qkv, ((q.ntok - 1) * q.qkv_ld + (nh + 2 * nkv) * hd) * F32, "rope qkv"),
                (q.pos, q.ntok * 4, "rope pos"),
                (q.cos_sin, (p_max + 1) * q.rope_n_dims * F32, "rope table"),
                (q.q_dst, q.ntok * nh * hd * F32, "rope q_dst"),
                # key (h, p, d) at h * k_slice + ((d / 8) * cache_m + p) * 8 + d % 8
                (q.k_cache, ((nkv - 1) * q.k_slice + ((lnship.kp(hd) // 8 - 1) * q.cache_m + p_max) * 8 + 8) * 4,
                 "k cache"),
                # value (h, p, d) at h * v_slice + ((p / 8) * head_dim + d) * 8 + p % 8
                (q.v_cache, ((nkv - 1) * q.v_slice + ((p_max // 8) * hd + hd - 1) * 8 + 8) * 4, "v cache")]
    elif name == "lnship32_attn_decode":
        q = a[0]
        hd, nh, nkv, n = q.head_dim, q.n_head, q.n_head_kv, q.n_kv
        out += [(q.q, nh * hd * F32, "attn q"), (q.dst, nh * hd * F32, "attn dst"),
                # key cell j < n_kv, dim d: k_slice per kv head, groups of eight dims cache_m * 8 codes apart
                (q.k_cache, ((nkv - 1) * q.k_slice + ((lnship.kp(hd) // 8 - 1) * q.cache_m + n - 1) * 8 + 8) * 4,
                 "attn k cache"),
                # value dim d, cell j: groups of eight cells head_dim * 8 codes apart
                (q.v_cache, ((nkv - 1) * q.v_slice + lnship.kp(n) * hd) * 4, "attn v cache")]
        if q.mask:
            out.append((q.mask, n * F32, "attn mask"))
    elif name == "lnship32_soft_max":
        s = a[0]
        ne, mne = list(s.src_ne), list(s.mask_ne)
        n = ne[0] * ne[1] * ne[2] * ne[3]
        out += [(s.src, n * F32, "soft_max src"), (s.dst, n * F32, "soft_max dst")]
        if s.mask:
            # mask row i1 of plane (i2 % mask_ne[2], i3 % mask_ne[3])
            last = ((min(mne[3], ne[3]) - 1) * mne[2] * mne[1] + (min(mne[2], ne[2]) - 1) * mne[1] + ne[1] - 1)
            out.append((s.mask, (last * mne[0] + ne[0]) * F32, "soft_max mask"))
    elif name == "lnship32_add":
        x, b, n, nb, dst = a[:5]
        out += [(x, n * F32, "add a"), (b, nb * F32, "add b"), (dst, n * F32, "add dst")]
    elif name == "lnship32_swiglu":
        gate, gate_ld, up, up_ld, dst, ncols, nrows = a[:7]
        out += [(gate, ((nrows - 1) * gate_ld + ncols) * F32, "swiglu gate"),
                (up, ((nrows - 1) * up_ld + ncols) * F32, "swiglu up"), (dst, nrows * ncols * F32, "swiglu dst")]
    elif name == "lnship_causal_mask":
        pos, ntok, n_kv, mask = a[:4]
        out += [(pos, ntok * 4, "mask pos"), (mask, ntok * n_kv * F32, "mask")]
    elif name in ("lnship_init", "lnship_rope_table", "lnship_max_row"):
        pass   # no device memory (the rope table is filled in host memory)
    else:
        raise AssertionError("no footprint for " + name)
    return [(_ptr(p), nbytes, what) for p, nbytes, what in out]


def allocations(model):
    ts = [model.tok_embd, model.tok_embd_f32, model.out_norm, model.cos_sin, *model.kcache, *model.vcache,
          *model._bufs.values()]
    for L in model.layers:
        ts += list(L.values())
    spans = {}
    for t in ts:
        st = t.untyped_storage()
        spans[st.data_ptr()] = st.nbytes()
    return sorted(spans.items())


def audit(calls, allocs):
    checked = 0
    for name, args in calls:
        for p, nbytes, what in footprints(name, args):
            assert p, f"{name}: {what} is a null pointer"
            assert nbytes > 0, f"{name}: {what} spans no bytes"
            inside = [(b, n) for b, n in allocs if b <= p and p + nbytes <= b + n]
            assert inside, (f"{name}: {what} [{p:#x}, +{nbytes}) lies outside every allocation: "
                            f"{[(hex(b), n) for b, n in allocs if b <= p < b + n]}")
            checked += 1
    return checked


@pytest.fixture
def recorded(monkeypatch):
    rec = Recorder()
    for mod in (lnship, llama):
        monkeypatch.setattr(mod, "lib", lambda: rec)
        monkeypatch.setattr(mod, "init", lambda device=None: None)
    monkeypatch.setattr(torch.cuda, "current_stream", lambda *a: type("S", (), {"cuda_stream": 0})())
    monkeypatch.setattr(torch.cuda, "synchronize", lambda *a: None)
    return rec


def _model(rec):
    cfg = dataclasses.replace(llama.LLAMA_1B, n_layer=2)
    e, f, hd = cfg.n_embd, cfg.n_ff, cfg.head_dim
    z = lambda *s: torch.empty(*s)   # never read: nothing runs
    layers = [{"attn_norm": z(e), "wq": z(cfg.n_head * hd, e), "wk": z(cfg.n_head_kv * hd, e),
               "wv": z(cfg.n_head_kv * hd, e), "wo": z(e, cfg.n_head * hd), "ffn_norm": z(e),
               "w_up": z(f, e), "w_gate": z(f, e), "w_down": z(e, f)} for _ in range(cfg.n_layer)]
    model = llama.LlamaLNS32(cfg, {"tok_embd": z(cfg.n_vocab, e), "out_norm": z(e), "layers": layers},
                             device="cpu")
    model._capture = lambda run: (_Graph(), run())
    return cfg, model


def test_lns32_decode_at_full_context_stays_inside_its_allocations(recorded):
    cfg, model = _model(recorded)
    assert cfg.n_ctx == 1024
    n_init = audit(recorded.calls, allocations(model))   # the weight packing
    recorded.calls.clear()
    # a 512-token prompt (audited before later steps could regrow a buffer),
    # then decode up to the last cell of the cache
    model.eval(list(range(512)))
    n_prompt = audit(recorded.calls, allocations(model))
    recorded.calls.clear()
    model.n_past = cfg.n_ctx - 2
    tok = torch.zeros(1, dtype=torch.int32)
    model.decode_graph(tok)
    model.decode_graph(tok)
    assert model.n_past == cfg.n_ctx
    # the steps' KV views covered the whole cache (kq, soft_max and kqv as
    # three ops at this n_kv)
    kq = [a[0] for n, a in recorded.calls if n == "lnship32_mul_mat" and a[0].w_mstride == cfg.n_ctx]
    assert kq and max(m.M for m in kq) == cfg.n_ctx
    kqv = [a[0] for n, a in recorded.calls if n == "lnship32_mul_mat" and a[0].w_slice == model.vslice]
    assert kqv and max(m.K for m in kqv) == cfg.n_ctx
    # q|k|v and up|gate take their rms_norm and norm MUL in their launch
    pre = [a[0] for n, a in recorded.calls if n == "lnship32_mul_mat" and a[0].rms_norm_w]
    assert len(pre) == 2 * cfg.n_layer   # (the second step replays the graph)
    n = audit(recorded.calls, allocations(model))
    # the same steps with the attention as one launch over the whole cache
    # (the second step replays the graph the first one captured)
    recorded.calls.clear()
    model._graphs.clear()
    model._attn_max_kv = cfg.n_ctx
    model.n_past = cfg.n_ctx - 2
    model.decode_graph(tok)
    model.decode_graph(tok)
    att = [a[0] for n, a in recorded.calls if n == "lnship32_attn_decode"]
    assert len(att) == cfg.n_layer and max(q.n_kv for q in att) == cfg.n_ctx
    n += audit(recorded.calls, allocations(model))
    assert n_init > 0 and n_prompt > 0 and n > 30 * cfg.n_layer
    # and a step past the cache is refused on the host before any launch
    recorded.calls.clear()
    with pytest.raises(ValueError):
        model.decode_graph(tok)
    assert not [c for c in recorded.calls if c[0] != "lnship_max_row"]


def test_audit_catches_a_view_past_the_cache(recorded):
    # the footprint check itself: a KV view one cell longer than the cache
    # is reported
    cfg, model = _model(recorded)
    recorded.calls.clear()
    model._attn_max_kv = cfg.n_ctx
    model.n_past = cfg.n_ctx - 1
    model.forward(1, torch.zeros(1, dtype=torch.int32), torch.full((1,), cfg.n_ctx - 1, dtype=torch.int32),
                  cfg.n_ctx)
    calls = []
    for name, args in recorded.calls:
        if name == "lnship32_attn_decode":
            m = type(args[0]).from_buffer_copy(args[0])
            m.n_kv = cfg.n_ctx + 8
            args = [m]
        calls.append((name, args))
    assert any(n == "lnship32_attn_decode" for n, _ in calls)
    with pytest.raises(AssertionError, match="outside every allocation"):
        audit(calls, allocations(model))
