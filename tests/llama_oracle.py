"""CPU oracles of the Llama-architecture decoder in LNS16 and LNS32 (test
infrastructure).

The same graph as lnship.llama (llama.cpp's llama graph as the reference's
LNS16 backend computes it), built from the oracle's op drivers: mul_mat
(src/lns-ops.cpp:293-384), rms_norm (:701-736), soft_max (:643-695), add /
mul (:468-530), swiglu (:812-868), rope (:1199-1281), get_rows of LNS16
weights (:1003-1050).  The KV cache holds IEEE half values, as llama.cpp's
F16 cache does.  Monte ops draw from the oracle's process-global LFSR in
graph order.  With n_seq > 1 each sequence has its own KV cache; eval(tokens,
seq) runs one sequence's tokens and eval_batch(tokens) one decode step of
every sequence, attention batched over sequences in the 4th dimension, as
lnship.llama does.
"""
import ctypes
import math

import numpy as np

import oracle_lib as O

KV_PAD = 256


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data)


def n_kv_for(n_used, n_ctx):
    return min(n_ctx, max(KV_PAD, ((n_used + KV_PAD - 1) // KV_PAD) * KV_PAD))


def _binop(fn, a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    out = np.empty_like(a)
    fn(_ptr(a), _ptr(b), a.size, b.size, _ptr(out))
    return out


class LlamaOracle16:
    def __init__(self, cfg, weights, mode, lfsr=7, n_seq=1):
        L = O.lib()
        for name, args in (("lno16_add_f32", [ctypes.c_void_p] * 2 + [ctypes.c_int64] * 2 + [ctypes.c_void_p]),
                           ("lno16_mul_f32", [ctypes.c_void_p] * 2 + [ctypes.c_int64] * 2 + [ctypes.c_void_p]),
                           ("lno16_swiglu_f32", [ctypes.c_void_p] * 2 + [ctypes.c_int64, ctypes.c_void_p]),
                           ("lno16_rope_f32", [ctypes.c_void_p] * 2 + [ctypes.c_int64] * 3 +
                            [ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_void_p])):
            fn = getattr(L, name)
            fn.restype = None
            fn.argtypes = args
        self.L, self.cfg, self.mode = L, cfg, mode
        O.monte_set(lfsr)
        c = cfg
        # LNS16 weight tensors: the codes of the F32 init values
        self.tok_embd = O.f2x16(weights["tok_embd"])                  # [vocab, e]
        self.out_norm = weights["out_norm"]
        self.layers = []
        for W in weights["layers"]:
            self.layers.append({
                "attn_norm": W["attn_norm"], "ffn_norm": W["ffn_norm"],
                "wqkv": O.f2x16(np.concatenate([W["wq"], W["wk"], W["wv"]])),
                "wo": O.f2x16(W["wo"]),
                "wug": O.f2x16(np.concatenate([W["w_up"], W["w_gate"]])),
                "wdown": O.f2x16(W["w_down"]),
            })
        self.n_seq = n_seq
        self.kcache = [np.zeros((n_seq, c.n_ctx, c.n_head_kv, c.head_dim), np.float16) for _ in range(c.n_layer)]
        self.vcache = [np.zeros((n_seq, c.n_ctx, c.n_head_kv, c.head_dim), np.float16) for _ in range(c.n_layer)]
        self.past = [0] * n_seq

    def _rope(self, x, pos):
        c = self.cfg
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty_like(x)
        pos = np.ascontiguousarray(pos, np.int32)
        self.L.lno16_rope_f32(_ptr(x), _ptr(pos), x.shape[0], x.shape[1], x.shape[2], c.head_dim, 0,
                              c.rope_theta, _ptr(out))
        return out

    @property
    def n_past(self):
        return self.past[0]

    def eval(self, tokens, seq=0):
        """Appends tokens to sequence seq; returns the logits of the last one."""
        p0 = self.past[seq]
        pos = np.arange(p0, p0 + len(tokens), dtype=np.int32)
        out = self._graph(tokens, pos, [seq] * len(tokens), n_kv_for(p0 + len(tokens), self.cfg.n_ctx), False)
        self.past[seq] += len(tokens)
        return out

    def eval_batch(self, tokens):
        """One decode step of every sequence; returns logits [n_seq][n_vocab]."""
        pos = np.asarray(self.past, dtype=np.int32)
        out = self._graph(tokens, pos, list(range(self.n_seq)), n_kv_for(max(self.past) + 1, self.cfg.n_ctx), True)
        self.past = [p + 1 for p in self.past]
        return out

    def _graph(self, tokens, pos, seqs, n_kv, batch):
        c, m = self.cfg, self.mode
        T = len(tokens)
        e, hd, nh, nkv, f = c.n_embd, c.head_dim, c.n_head, c.n_head_kv, c.n_ff
        nq = nh * hd
        mask = np.where(np.arange(n_kv)[None, :] <= pos[:, None], 0.0, -np.inf).astype(np.float32)
        x = O.x2f16(self.tok_embd[np.asarray(tokens)])                 # get_rows of LNS16 -> F32
        for il, W in enumerate(self.layers):
            last = il == c.n_layer - 1
            h = O.rms_norm16(m, x, c.eps)
            h = _binop(self.L.lno16_mul_f32, h, W["attn_norm"])
            qkv = O.mul_mat16(m, W["wqkv"], h)                          # [T, nq + 2 nkv hd]
            q = self._rope(qkv[:, :nq].reshape(T, nh, hd), pos)
            k = self._rope(qkv[:, nq:nq + nkv * hd].reshape(T, nkv, hd), pos)
            v = qkv[:, nq + nkv * hd:].reshape(T, nkv, hd)
            for t in range(T):
                self.kcache[il][seqs[t], pos[t]] = k[t].astype(np.float16)
                self.vcache[il][seqs[t], pos[t]] = v[t].astype(np.float16)
            if batch:
                # one query row per sequence, sequences in the 4th dimension
                kw = self.kcache[il][:, :n_kv].astype(np.float32).transpose(0, 2, 1, 3)   # [S, nkv, n_kv, hd]
                kq = O.mul_mat16_f32w(m, kw, q[:, :, None, :], ne02=nkv, ne03=T)        # [S, nh, 1, n_kv]
                kq = O.soft_max16(m, kq, mask[:, None, None, :], 1.0 / math.sqrt(hd))
                vw = self.vcache[il][:, :n_kv].astype(np.float32).transpose(0, 2, 3, 1)   # [S, nkv, hd, n_kv]
                att = O.mul_mat16_f32w(m, vw, kq, ne02=nkv, ne03=T)                   # [S, nh, 1, hd]
                att = np.ascontiguousarray(att.reshape(T, nq))
            else:
                s = seqs[0]
                kw = self.kcache[il][s, :n_kv].astype(np.float32).transpose(1, 0, 2)   # [nkv, n_kv, hd]
                kq = O.mul_mat16_f32w(m, kw[None], q.transpose(1, 0, 2)[None], ne02=nkv)  # [1, nh, T, n_kv]
                kq = O.soft_max16(m, kq[0], mask, 1.0 / math.sqrt(hd))
                vw = self.vcache[il][s, :n_kv].astype(np.float32).transpose(1, 2, 0)   # [nkv, hd, n_kv]
                att = O.mul_mat16_f32w(m, vw[None], kq[None], ne02=nkv)[0]          # [nh, T, hd]
                att = np.ascontiguousarray(att.transpose(1, 0, 2).reshape(T, nq))
            o = O.mul_mat16(m, W["wo"], att)
            if last and not batch:
                o, x = o[-1:], x[-1:]
            x = _binop(self.L.lno16_add_f32, o, x)
            h = O.rms_norm16(m, x, c.eps)
            h = _binop(self.L.lno16_mul_f32, h, W["ffn_norm"])
            ug = O.mul_mat16(m, W["wug"], h)
            up, gate = np.ascontiguousarray(ug[:, :f]), np.ascontiguousarray(ug[:, f:])
            sw = np.empty_like(up)
            self.L.lno16_swiglu_f32(_ptr(gate), _ptr(up), up.size, _ptr(sw))
            d = O.mul_mat16(m, W["wdown"], sw)
            x = _binop(self.L.lno16_add_f32, d, x)
        h = O.rms_norm16(m, x if batch else x[-1:], c.eps)
        h = _binop(self.L.lno16_mul_f32, h, self.out_norm)
        logits = O.mul_mat16(m, self.tok_embd, h)
        return logits if batch else logits[0]


class LlamaOracle32:
    """The same graph as the reference's LNS32 backend computes it
    (src32/lns32-ops.cpp): get_rows copies the F32 embedding rows (:707-745),
    every other op converts its F32 operands with fp2xlns32 (weights once:
    the conversion of an F32 weight does not depend on the call), the KV
    cache holds IEEE half values (kq / kqv convert them, :64-79), one
    sequence."""

    def __init__(self, cfg, weights):
        self.cfg = cfg
        c = cfg
        self.tok_embd_f32 = np.ascontiguousarray(weights["tok_embd"], np.float32)
        self.tok_embd = O.f2x32(self.tok_embd_f32)                     # [vocab, e] codes
        self.out_norm = weights["out_norm"]
        self.layers = []
        for W in weights["layers"]:
            self.layers.append({
                "attn_norm": W["attn_norm"], "ffn_norm": W["ffn_norm"],
                "wqkv": O.f2x32(np.concatenate([W["wq"], W["wk"], W["wv"]])),
                "wo": O.f2x32(W["wo"]),
                "wug": O.f2x32(np.concatenate([W["w_up"], W["w_gate"]])),
                "wdown": O.f2x32(W["w_down"]),
            })
        self.kcache = [np.zeros((c.n_ctx, c.n_head_kv, c.head_dim), np.float16) for _ in range(c.n_layer)]
        self.vcache = [np.zeros((c.n_ctx, c.n_head_kv, c.head_dim), np.float16) for _ in range(c.n_layer)]
        self.n_past = 0

    def eval(self, tokens, n_layers=None):
        """Appends tokens; returns the logits of the last one.  n_layers runs
        only the first layers (a bounded sample for timing)."""
        c = self.cfg
        T = len(tokens)
        p0 = self.n_past
        pos = np.arange(p0, p0 + T, dtype=np.int32)
        n_kv = n_kv_for(p0 + T, c.n_ctx)
        e, hd, nh, nkv, f = c.n_embd, c.head_dim, c.n_head, c.n_head_kv, c.n_ff
        nq = nh * hd
        mask = np.where(np.arange(n_kv)[None, :] <= pos[:, None], 0.0, -np.inf).astype(np.float32)
        x = self.tok_embd_f32[np.asarray(tokens)]
        layers = self.layers if n_layers is None else self.layers[:n_layers]
        for il, W in enumerate(layers):
            last = il == c.n_layer - 1
            h = O.mul32(O.rms_norm32(x, c.eps), W["attn_norm"])
            qkv = O.mul_mat32_codes(W["wqkv"], h)
            q = O.rope32(qkv[:, :nq].reshape(T, nh, hd), pos, hd, 0, c.rope_theta)
            k = O.rope32(qkv[:, nq:nq + nkv * hd].reshape(T, nkv, hd), pos, hd, 0, c.rope_theta)
            v = qkv[:, nq + nkv * hd:].reshape(T, nkv, hd)
            self.kcache[il][pos] = k.astype(np.float16)
            self.vcache[il][pos] = v.astype(np.float16)
            kw = self.kcache[il][:n_kv].astype(np.float32).transpose(1, 0, 2)       # [nkv, n_kv, hd]
            kq = O.mul_mat32(kw[None], q.transpose(1, 0, 2)[None], ne02=nkv)       # [1, nh, T, n_kv]
            kq = O.soft_max32(kq[0], mask, 1.0 / math.sqrt(hd))
            vw = self.vcache[il][:n_kv].astype(np.float32).transpose(1, 2, 0)       # [nkv, hd, n_kv]
            att = O.mul_mat32(vw[None], kq[None], ne02=nkv)[0]                      # [nh, T, hd]
            att = np.ascontiguousarray(att.transpose(1, 0, 2).reshape(T, nq))
            o = O.mul_mat32_codes(W["wo"], att)
            if last:
                o, x = o[-1:], x[-1:]
            x = O.add32(o, x)
            h = O.mul32(O.rms_norm32(x, c.eps), W["ffn_norm"])
            ug = O.mul_mat32_codes(W["wug"], h)
            sw = O.swiglu32(ug[:, f:], ug[:, :f])
            x = O.add32(O.mul_mat32_codes(W["wdown"], sw), x)
        self.n_past += T
        h = O.mul32(O.rms_norm32(x[-1:], c.eps), self.out_norm)
        return O.mul_mat32_codes(self.tok_embd, h)[0]
