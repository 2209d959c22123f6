"""A Llama-architecture decoder running every op on the gfx950 LNS kernels.

The graph is llama.cpp's llama graph (non-flash attention) as the reference's
LNS16 backend computes it, op by op, with F32 at op boundaries:

  x = get_rows(tok_embd, tokens)                         (LNS16 weights decoded)
  per layer:  h = rms_norm(x) * attn_norm
              q, k, v = Wq h, Wk h, Wv h                  (one fused launch)
              q, k = rope(q), rope(k)                      (normal pairs)
              K/V cache <- f16(k), f16(v)                  (kept as packed LNS16)
              p = soft_max(K^T q * 1/sqrt(d) + causal mask) over n_kv = pad(n, 256)
              x = Wo (V p) + x                             (last layer: then last token only)
              h = rms_norm(x) * ffn_norm
              x = Wdown swiglu(Wgate h, Wup h) + x         (up | gate fused)
  logits = tok_embd^T (rms_norm(x_last) * out_norm)        (tied output)

Fusing Q|K|V and up|gate into one matrix keeps the Monte draw order of the
separate ops: outputs of a mul_mat take draws in (row, column) order, so the
fused rows enumerate Q's outputs, then K's, then V's.  A single-sequence
decode step runs K^T q, soft_max and V p in one launch (lnship16_attn_decode,
and in Monte and for a batched step of several sequences
lnship16_attn_decode_seqs, which takes the three ops' Monte starts;
bit-identical to the three ops; fused_attn = False runs the three), the
query rope and the cache stores inside it (fused_rope).  A single-row sum32
step runs each rms_norm, its norm MUL and the mul_mat that reads them in one
launch (lnship16_rms_norm_mul_mat, its scale predicted, bit-identical to the
three; fused_rms = False runs them apart).  A single-row step outside Monte
forms swiglu inside the down projection's launch (lnship16_swiglu_mul_mat;
fused_glu = False runs the two).  The other decode steps (a batched step, a
Monte token) run the rms_norm and norm MUL, or the swiglu, inside the launch
of the mul_mat that reads them through lnship16_mul_mat's prologue fields
(fused_pre = False runs them apart).

With n_seq > 1 the model holds that many independent sequences, each with
its own KV cache, as llama.cpp's per-sequence KV streams.  A sequence's
prompt runs on its own (eval with seq=s); a batched decode step (eval_batch)
takes one token per sequence: the weight mul_mats see N = n_seq columns and
attention runs over all sequences at once through the 4th dimension
(kq = K_s^T q_s and kqv = V_s p_s for each sequence s, masked per sequence).

Activations, weights and the KV cache live in HBM; nothing is copied back to
the host except the logits the caller asks for.
"""
import ctypes
import math
from dataclasses import dataclass

import numpy as np

from . import (BASE, MONTE, LPVIP, SUM32, AttnArgs, QkvStoreArgs, attn_seqs, check, init, kp, lfsr_advance, lib,
               mul_mat16_raw, mul_mat32_raw, seed_fields)

KV_PAD = 256   # llama.cpp pads the KV view to 256 cells without flash attention


@dataclass
class LlamaConfig:
    n_layer: int = 30
    n_embd: int = 576
    n_head: int = 9
    n_head_kv: int = 3
    head_dim: int = 64
    n_ff: int = 1536
    n_vocab: int = 49152
    n_ctx: int = 512
    rope_theta: float = 10000.0
    eps: float = 1e-5


SMOLLM2_135M = LlamaConfig()


def splitmix_normal(seed, n, std):
    """n samples of N(0, std^2): splitmix64 uniforms, Box-Muller in double, cast to float32."""
    n2 = (n + 1) // 2
    i = np.arange(2 * n2, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = (np.uint64(seed) * np.uint64(0x9E3779B97F4A7C15) + (i + np.uint64(1)) * np.uint64(0x9E3779B97F4A7C15))
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    u = ((z >> np.uint64(11)).astype(np.float64) + 0.5) * (1.0 / 9007199254740992.0)
    u1, u2 = u[0::2], u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    out = np.empty(2 * n2, dtype=np.float64)
    out[0::2] = r * np.cos(2.0 * np.pi * u2)
    out[1::2] = r * np.sin(2.0 * np.pi * u2)
    return (out[:n] * std).astype(np.float32)


def synthetic_weights(cfg, seed=1234, std=0.02):
    """Random-init weights of the architecture (F32, host).  Norm weights are
    ones, as a freshly initialised RMSNorm; matrices are N(0, std^2)."""
    e, f, d = cfg.n_embd, cfg.n_ff, cfg.head_dim
    nq, nkv = cfg.n_head * d, cfg.n_head_kv * d
    w = {"tok_embd": splitmix_normal(seed, cfg.n_vocab * e, std).reshape(cfg.n_vocab, e),
         "out_norm": np.ones(e, np.float32), "layers": []}
    for il in range(cfg.n_layer):
        s = seed + 1000 * (il + 1)
        w["layers"].append({
            "attn_norm": np.ones(e, np.float32),
            "wq": splitmix_normal(s + 1, nq * e, std).reshape(nq, e),
            "wk": splitmix_normal(s + 2, nkv * e, std).reshape(nkv, e),
            "wv": splitmix_normal(s + 3, nkv * e, std).reshape(nkv, e),
            "wo": splitmix_normal(s + 4, e * nq, std).reshape(e, nq),
            "ffn_norm": np.ones(e, np.float32),
            "w_gate": splitmix_normal(s + 5, f * e, std).reshape(f, e),
            "w_up": splitmix_normal(s + 6, f * e, std).reshape(f, e),
            "w_down": splitmix_normal(s + 7, e * f, std).reshape(e, f),
        })
    return w


def n_kv_for(n_used, n_ctx):
    return min(n_ctx, max(KV_PAD, ((n_used + KV_PAD - 1) // KV_PAD) * KV_PAD))


class LlamaLNS16:
    """The decoder on one GPU; mode is the xlns16 summation mode."""

    def __init__(self, cfg, weights, mode=SUM32, lfsr=7, n_seq=1):
        import torch
        init()
        self.cfg, self.mode, self.lfsr, self.n_seq = cfg, mode, lfsr, n_seq
        self.torch = torch
        # decode attention in one launch where the op takes the cells
        self.fused_attn = True
        # and with it, the query rope and the cache stores of the token
        # (lnship16_rope_attn_decode, bit-identical to the two launches)
        self.fused_rope = True
        # sum32, one row: rms_norm, the norm MUL and the mul_mat after them in
        # one launch (lnship16_rms_norm_mul_mat, bit-identical to the three),
        # where the row fits the kernel's LDS
        self.fused_rms = mode == SUM32 and cfg.n_embd <= lib().lnship_max_row(5, mode)
        # one row outside Monte: swiglu inside the down projection's launch
        # (lnship16_swiglu_mul_mat, bit-identical to the two nodes), where the
        # activation row fits LDS
        self.fused_glu = mode != MONTE and cfg.n_ff <= lib().lnship_max_row(6, mode)
        # the rows of a decode step (one token, or one per sequence): the
        # rms_norm and norm MUL, or the swiglu, inside the launch of the
        # mul_mat that reads them (lnship16_mul_mat's prologue fields,
        # bit-identical to the separate nodes), where the rows fit LDS
        self.fused_pre = True
        self._attn_max_kv = lib().lnship_max_row(8, mode)
        dev = torch.device("cuda", torch.cuda.current_device())
        self.dev = dev
        c = cfg
        from . import pack16
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
        self.tok_embd = pack16(t(weights["tok_embd"]))           # K = n_embd, M = n_vocab
        self.out_norm = t(weights["out_norm"])
        self.layers = []
        for L in weights["layers"]:
            self.layers.append({
                "attn_norm": t(L["attn_norm"]),
                "wqkv": pack16(t(np.concatenate([L["wq"], L["wk"], L["wv"]]))),
                "wo": pack16(t(L["wo"])),
                "ffn_norm": t(L["ffn_norm"]),
                "wug": pack16(t(np.concatenate([L["w_up"], L["w_gate"]]))),
                "wdown": pack16(t(L["w_down"])),
            })
        hd, nkv = c.head_dim, c.n_head_kv
        # packed LNS16 caches, per layer and sequence: K [nkv][hd/8][n_ctx][8],
        # V [nkv][n_ctx/8][hd][8]; the sequences' caches follow each other
        self.kslice = kp(hd) * c.n_ctx
        self.vslice = kp(c.n_ctx) * hd
        assert self.kslice == self.vslice
        self.seq_stride = nkv * self.kslice
        self.kcache = [torch.zeros(n_seq * self.seq_stride, dtype=torch.int16, device=dev) for _ in range(c.n_layer)]
        self.vcache = [torch.zeros(n_seq * self.seq_stride, dtype=torch.int16, device=dev) for _ in range(c.n_layer)]
        rt = np.empty(c.n_ctx * hd, np.float32)
        check(lib().lnship_rope_table(c.rope_theta, hd, c.n_ctx, ctypes.c_void_p(rt.ctypes.data)))
        self.cos_sin = t(rt)
        self.seq_ids = torch.arange(n_seq, dtype=torch.int32, device=dev)
        self.past = [0] * n_seq
        self._bufs = {}
        self._graphs = {}
        # Monte under HIP graphs: the ops of a captured step read their LFSR
        # start from this device state (a jump of the draws before them in
        # the step), and the step ends by advancing it past all its draws
        self.lfsr_dev = torch.zeros(1, dtype=torch.int16, device=dev)
        self._dev_draws = None      # draws so far of the step being built on lfsr_dev
        self._lfsr_synced = False   # lfsr_dev holds self.lfsr

    @property
    def n_past(self):
        """Tokens held by sequence 0."""
        return self.past[0]

    @n_past.setter
    def n_past(self, v):
        self.past[0] = v

    def restart(self, lfsr=7):
        """Empties every sequence's KV cache (positions restart at 0) and puts
        the Monte LFSR back at lfsr; captured graphs stay valid."""
        self.past = [0] * self.n_seq
        self.lfsr = lfsr
        self._lfsr_synced = False

    # -- buffers --------------------------------------------------------------
    def _buf(self, name, n, dtype=None):
        """A grow-only device buffer.  A captured HIP graph keeps the
        addresses it was captured with, so growing a buffer first drops every
        captured graph (together with the tensors they reference); they are
        captured again on their next use."""
        torch = self.torch
        dtype = dtype or torch.float32
        b = self._bufs.get(name)
        if b is None or b.numel() < n:
            if b is not None and self._graphs:
                torch.cuda.synchronize()
                self._graphs.clear()
            b = torch.empty(max(n, 1), dtype=dtype, device=self.dev)
            self._bufs[name] = b
        return b

    def _check_ctx(self, first, T, n_kv=None):
        """Positions first .. first + T - 1 and a KV view of n_kv cells must
        fit the n_ctx cells of the caches and the rope table."""
        n_ctx = self.cfg.n_ctx
        if first < 0 or T < 0 or first + T > n_ctx:
            raise ValueError("context full: positions %d..%d do not fit n_ctx=%d" % (first, first + T - 1, n_ctx))
        if n_kv is not None and not 0 < n_kv <= n_ctx:
            raise ValueError("KV view of %d cells outside 1..n_ctx=%d" % (n_kv, n_ctx))

    def _seed(self, draws):
        """Monte: where an op's LFSR draws start, then advance past them (graph
        order).  Eagerly that is the 16-bit state itself; in a step built for
        a HIP graph it is (lfsr_dev, offset): the op jumps from the state the
        replay finds on the device."""
        if self.mode != MONTE:
            return self.lfsr
        if self._dev_draws is not None:
            off = self._dev_draws
            self._dev_draws += draws
            return (self.lfsr_dev, off)
        s = self.lfsr
        self.lfsr = lib().lnship_lfsr_jump(s, draws)
        self._lfsr_synced = False
        return s

    def _device_seeded(self, run):
        """run() with the Monte ops seeded from lfsr_dev, then lfsr_dev advanced
        past the draws they took; returns (run's result, draws)."""
        if self.mode != MONTE:
            return run(), 0
        self._dev_draws = 0
        try:
            out = run()
            draws = self._dev_draws
            lfsr_advance(self.lfsr_dev, draws)
        finally:
            self._dev_draws = None
        return out, draws

    def _replay(self, key, build):
        """Replays the graph of key (capturing build() first if needed) and
        keeps self.lfsr and lfsr_dev in step; returns the graph's output."""
        if key not in self._graphs:
            self._graphs[key] = self._capture(lambda: self._device_seeded(build))
            self._lfsr_synced = False   # the warm-up run advanced lfsr_dev
        g, (out, draws) = self._graphs[key]
        if self.mode == MONTE:
            if not self._lfsr_synced:
                self.lfsr_dev.fill_(self.lfsr - 65536 if self.lfsr >= 32768 else self.lfsr)
            g.replay()
            self.lfsr = lib().lnship_lfsr_jump(self.lfsr, draws)
            self._lfsr_synced = True
        else:
            g.replay()
        return out

    # -- ops --------------------------------------------------------------------
    def _mm(self, w, x_ptr, dst_ptr, K, M, N, **kw):
        ne12, ne13 = kw.get("ne12", 1), kw.get("ne13", 1)
        draws = lib().lnship16_mul_mat_draws(self.mode, K, M, N, ne12, ne13)
        mul_mat16_raw(self.mode, w, x_ptr, dst_ptr, K, M, N, seed=self._seed(draws), stream=self._stream, **kw)

    def _mm_pre(self, w, x_ptr, dst_ptr, K, M, N, rms_w=None, glu_up=None, residual=None, x_ld=0):
        """dst (+)= W pre(x) for N rows of K in one launch, pre being the
        node(s) before the mul_mat: rms_norm and the MUL by the norm row rms_w,
        or swiglu(x, glu_up) (lnship16_mul_mat's prologue fields; Monte: the
        rms_norm's draws, then the product's, in graph order).  False, with
        nothing run and no draws taken, where the launch cannot stage its
        rows beside the tables."""
        from . import MulMatArgs
        L = lib()
        saved = (self.lfsr, self._dev_draws, self._lfsr_synced)
        rs = self._seed(L.lnship16_rms_norm_draws(self.mode, K, N)) if rms_w is not None else 0
        sd, st, off = seed_fields(self._seed(L.lnship16_mul_mat_draws(self.mode, K, M, N, 1, 1)))
        a = MulMatArgs(ctypes.c_void_p(w), x_ptr, dst_ptr, K, M, N, 1, 1, 1, 1, x_ld, 0, sd, 0, 0, 0, 0, st,
                       off or 0, residual)
        if rms_w is not None:
            rsd, rst, roff = seed_fields(rs)
            # (one device state, or none, for both nodes' starts)
            assert (rst is None) == (st is None), "the two nodes' starts come from one place"
            a.rms_norm_w, a.rms_eps, a.rms_seed, a.rms_offset = rms_w, self.cfg.eps, rsd, roff or 0
        else:
            a.glu_up = glu_up
        rc = L.lnship16_mul_mat(self.mode, ctypes.byref(a), self._stream)
        if rc == -4:   # LNSHIP_ERANGE: the rows do not fit beside the tables
            self.lfsr, self._dev_draws, self._lfsr_synced = saved
            return False
        check(rc)
        return True

    def _rms_mul(self, x_ptr, w_ptr, dst_ptr, ncols, nrows):
        """rms_norm of nrows rows, then the MUL by the norm weight row w, in
        one launch (the MUL takes no draws)."""
        sd, st, off = seed_fields(self._seed(lib().lnship16_rms_norm_draws(self.mode, ncols, nrows)))
        check(lib().lnship16_rms_norm_mul(self.mode, x_ptr, w_ptr, dst_ptr, ncols, nrows, self.cfg.eps, sd, st,
                                          off or 0, self._stream))

    def _softmax(self, x_ptr, ne, mask_ptr, mne, scale, dst_ptr):
        from . import SoftMaxArgs
        nrows = ne[1] * ne[2] * ne[3]
        sd, st, off = seed_fields(self._seed(lib().lnship16_soft_max_draws(self.mode, ne[0], nrows)))
        a = SoftMaxArgs(x_ptr, (ctypes.c_int64 * 4)(*ne), mask_ptr, (ctypes.c_int64 * 4)(*mne), scale, dst_ptr, sd,
                        st, off)
        check(lib().lnship16_soft_max(self.mode, ctypes.byref(a), self._stream))

    def _rms_mm(self, x_ptr, wn_ptr, w, h_ptr, dst_ptr, K, M, T, step=False):
        """dst = W (rms_norm(x) * wn) for T rows of K: for one sum32 row in one
        launch (its scale predicted), for the rows of a decode step (step) in
        one launch, else rms_norm + MUL into h, then the mul_mat."""
        if T == 1 and self.fused_rms:
            check(lib().lnship16_rms_norm_mul_mat(self.mode, x_ptr, wn_ptr, self.cfg.eps, ctypes.c_void_p(w), dst_ptr,
                                                  K, M, self._stream))
        elif not (step and self.fused_pre and self._mm_pre(w, x_ptr, dst_ptr, K, M, T, rms_w=wn_ptr)):
            self._rms_mul(x_ptr, wn_ptr, h_ptr, K, T)
            self._mm(w, h_ptr, dst_ptr, K, M, T)

    def _glu_mm(self, gate_ptr, up_ptr, w, resid_ptr, dst_ptr, K, M):
        """dst = resid + W swiglu(gate, up) for one row of K, in one launch."""
        check(lib().lnship16_swiglu_mul_mat(self.mode, gate_ptr, up_ptr, ctypes.c_void_p(w), resid_ptr, dst_ptr, K, M,
                                            self._stream))

    def _attn_seqs(self, args, nseq, store=None):
        """The decode attention of one token in each of nseq sequences, with
        the Monte starts of the three nodes it replaces, taken in their order;
        with store (the tokens' rope and cache stores), the two in one launch."""
        L, nh, hd, n_kv = lib(), args.n_head, args.head_dim, args.n_kv
        seeds = (self._seed(L.lnship16_mul_mat_draws(self.mode, hd, n_kv, 1, nh, nseq)),
                 self._seed(L.lnship16_soft_max_draws(self.mode, n_kv, nh * nseq)),
                 self._seed(L.lnship16_mul_mat_draws(self.mode, n_kv, hd, 1, nh, nseq)))
        sq = attn_seqs(nseq, seeds)
        if store is None:
            check(L.lnship16_attn_decode_seqs(self.mode, ctypes.byref(args), ctypes.byref(sq), self._stream))
        else:
            check(L.lnship16_rope_attn_decode_seqs(self.mode, ctypes.byref(store), ctypes.byref(args),
                                                   ctypes.byref(sq), self._stream))

    def _attn(self, args, store=None):
        """The decode attention; with store (the token's rope and cache
        stores), the two in one launch."""
        if store is None:
            check(lib().lnship16_attn_decode(self.mode, ctypes.byref(args), self._stream))
        else:
            check(lib().lnship16_rope_attn_decode(self.mode, ctypes.byref(store), ctypes.byref(args), self._stream))

    # -- forward -------------------------------------------------------------------
    def forward(self, T, tokens_dev, pos_dev, n_kv, seq=0, batch=False):
        """Runs T tokens at positions pos_dev[0..T) (device int32) against a
        KV view of n_kv cells.  Without batch all T tokens belong to sequence
        seq and the device logits of the last one are returned; with batch
        T == n_seq, token s belongs to sequence s, and the logits of every
        token come back ([n_seq][n_vocab])."""
        torch, c, L = self.torch, self.cfg, lib()
        if batch and T != self.n_seq:
            raise ValueError("batched forward: %d tokens for %d sequences" % (T, self.n_seq))
        self._check_ctx(0, T, n_kv)
        self._stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        st = self._stream
        e, hd, nh, nkv, f = c.n_embd, c.head_dim, c.n_head, c.n_head_kv, c.n_ff
        nq, nqkv = nh * hd, (nh + 2 * nkv) * hd
        P = lambda b, off=0: ctypes.c_void_p(b.data_ptr() + off * b.element_size())
        x = self._buf("x", T * e)
        h = self._buf("h", T * e)
        qkv = self._buf("qkv", T * nqkv)
        q = self._buf("q", T * nq)
        kq = self._buf("kq", nh * T * n_kv)
        att = self._buf("att", T * nq)
        o = self._buf("o", T * e)
        ug = self._buf("ug", T * 2 * f)
        sw = self._buf("sw", T * f)
        mask = self._buf("mask", T * n_kv)
        logits = self._buf("logits", (T if batch else 1) * c.n_vocab)
        nseq = self.n_seq if batch else 1
        cbase = 0 if batch else seq * self.seq_stride   # cache offset (codes) of the attended sequence
        seq_ids = P(self.seq_ids) if batch else None
        check(L.lnship16_get_rows_packed(P(self.tok_embd), e, c.n_vocab, P(tokens_dev), T, P(x), st))
        check(L.lnship_causal_mask(P(pos_dev), T, n_kv, P(mask), st))
        for il, W in enumerate(self.layers):
            last = il == c.n_layer - 1
            self._rms_mm(P(x), P(W["attn_norm"]), W["wqkv"].data_ptr(), P(h), P(qkv), e, nqkv, T,
                         step=T == 1 or batch)
            # rope(q) and the K / V cache stores (k rotated) in one launch
            qs = QkvStoreArgs(P(qkv), nqkv, P(pos_dev), T, nh, nkv, hd, hd, P(self.cos_sin), P(q),
                              P(self.kcache[il], cbase), P(self.vcache[il], cbase), c.n_ctx, self.kslice,
                              self.vslice, seq_ids, self.seq_stride)
            Tq = 1 if batch else T   # query rows per sequence
            fused = (T == 1 or batch) and self.fused_attn and n_kv <= self._attn_max_kv
            # Monte and batched steps: lnship16_(rope_)attn_decode_seqs
            seqs = fused and (batch or self.mode == MONTE)
            if not (fused and self.fused_rope):
                check(L.lnship16_rope_store_kv(ctypes.byref(qs), st))
            if seqs:
                # the fused rope finds sequence s's cells without the seq map
                qs.seq = None
                self._attn_seqs(AttnArgs(P(q), P(self.kcache[il], cbase), P(self.vcache[il], cbase), c.n_ctx,
                                         self.kslice, self.vslice, P(mask), 1.0 / math.sqrt(hd), P(att), nh, nkv, hd,
                                         n_kv), nseq, qs if self.fused_rope else None)
            elif fused:
                # the three nodes below in one launch, bit for bit (and the
                # rope and cache stores above it, with fused_rope)
                self._attn(AttnArgs(P(q), P(self.kcache[il], cbase), P(self.vcache[il], cbase), c.n_ctx,
                                    self.kslice, self.vslice, P(mask), 1.0 / math.sqrt(hd), P(att), nh, nkv, hd,
                                    n_kv), qs if self.fused_rope else None)
            else:
                # kq[s][h][t][j] = K_s,j . q_s,t (GQA: query head h reads kv head h / (nh / nkv))
                self._mm(self.kcache[il].data_ptr() + 2 * cbase, P(q), P(kq), hd, n_kv, Tq, ne02=nkv, ne03=nseq,
                         ne12=nh, ne13=nseq, x_ld=nq, x_slice=hd, w_mstride=c.n_ctx, w_slice=self.kslice)
                self._softmax(P(kq), (n_kv, Tq, nh, nseq), P(mask), (n_kv, Tq, 1, nseq), 1.0 / math.sqrt(hd),
                              P(kq))
                # att[s, t][h*hd + d] = sum_j V_s[j][d] p[s][h][t][j]
                self._mm(self.vcache[il].data_ptr() + 2 * cbase, P(kq), P(att), n_kv, hd, Tq, ne02=nkv,
                         ne03=nseq, ne12=nh, ne13=nseq, x_ld=n_kv, x_slice=Tq * n_kv, w_slice=self.vslice,
                         dst_ld=nq, dst_slice=hd)
            # after the last layer's attention only the output rows go on
            rows = 1 if last and not batch else T
            r0 = (T - rows) * e
            if rows == T:   # x += Wo att: the residual ADD inside the mul_mat
                self._mm(W["wo"].data_ptr(), P(att), P(x), nq, e, T, residual=P(x))
            else:
                self._mm(W["wo"].data_ptr(), P(att), P(o), nq, e, T)
                check(L.lnship16_add(P(o, r0), P(x, r0), rows * e, rows * e, P(x), st))
            step = rows == 1 or batch
            self._rms_mm(P(x), P(W["ffn_norm"]), W["wug"].data_ptr(), P(h), P(ug), e, 2 * f, rows, step=step)
            if rows == 1 and self.fused_glu:   # x += Wdown swiglu(gate, up), one launch
                self._glu_mm(P(ug, f), P(ug), W["wdown"].data_ptr(), P(x), P(x), f, e)
            elif not (step and self.fused_pre and self._mm_pre(W["wdown"].data_ptr(), P(ug, f), P(x), f, e, rows,
                                                              glu_up=P(ug), residual=P(x), x_ld=2 * f)):
                check(L.lnship16_swiglu(P(ug, f), 2 * f, P(ug), 2 * f, P(sw), f, rows, st))
                self._mm(W["wdown"].data_ptr(), P(sw), P(x), f, e, rows, residual=P(x))
        nout = T if batch else 1
        self._rms_mm(P(x), P(self.out_norm), self.tok_embd.data_ptr(), P(h), P(logits), e, c.n_vocab, nout)
        if batch:
            return logits[: T * c.n_vocab].view(T, c.n_vocab)
        return logits[: c.n_vocab]

    def eval(self, tokens, seq=0):
        """Appends tokens (host list) to sequence seq; returns the device
        logits of the last one."""
        torch = self.torch
        T = len(tokens)
        p0 = self.past[seq]
        self._check_ctx(p0, T)
        tok = self._buf("tok", T, torch.int32)
        pos = self._buf("pos", T, torch.int32)
        tok[:T].copy_(torch.tensor(tokens, dtype=torch.int32))
        pos[:T].copy_(torch.arange(p0, p0 + T, dtype=torch.int32))
        n_kv = n_kv_for(p0 + T, self.cfg.n_ctx)
        out = self.forward(T, tok, pos, n_kv, seq=seq)
        self.past[seq] += T
        return out

    def eval_batch(self, tokens):
        """One decode step of every sequence: tokens[s] is appended to
        sequence s.  Returns the device logits [n_seq][n_vocab]."""
        torch = self.torch
        if len(tokens) != self.n_seq:
            raise ValueError("eval_batch: %d tokens for %d sequences" % (len(tokens), self.n_seq))
        self._check_ctx(max(self.past), 1)
        tok = self._buf("btok", self.n_seq, torch.int32)
        pos = self._buf("bpos", self.n_seq, torch.int32)
        tok[: self.n_seq].copy_(torch.tensor(tokens, dtype=torch.int32))
        pos[: self.n_seq].copy_(torch.tensor(self.past, dtype=torch.int32))
        out = self.forward(self.n_seq, tok, pos, self.batch_n_kv(), batch=True)
        self.past = [p + 1 for p in self.past]
        return out

    def batch_n_kv(self):
        """KV view of a batched step: the longest sequence's, padded."""
        return n_kv_for(max(self.past) + 1, self.cfg.n_ctx)

    def decode_graph_batch(self, tok_dev, n_kv=None):
        """eval_batch through a captured HIP graph, with the n_seq tokens
        already on the device.  Returns the device logits.  Monte ops read
        their LFSR start from lfsr_dev, so one graph serves every step."""
        torch = self.torch
        self._check_ctx(max(self.past), 1)
        n_kv = n_kv or self.batch_n_kv()
        self._check_ctx(max(self.past), 1, n_kv)
        tok = self._buf("gbtok", self.n_seq, torch.int32)
        pos = self._buf("gbpos", self.n_seq, torch.int32)
        tok[: self.n_seq].copy_(tok_dev[: self.n_seq])
        pos[: self.n_seq].copy_(torch.tensor(self.past, dtype=torch.int32))
        out = self._replay(("batch", n_kv), lambda: self.forward(self.n_seq, tok, pos, n_kv, batch=True))
        self.past = [p + 1 for p in self.past]
        return out

    def _capture(self, run):
        """Warms the library's scratch and the buffers with one eager run,
        then captures run() into a HIP graph; returns (graph, output)."""
        torch = self.torch
        run()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                out = run()
        torch.cuda.current_stream().wait_stream(s)
        return g, out

    def decode_graph(self, token, n_kv=None):
        """One decode step of sequence 0 through a captured HIP graph; token
        is a host int or a one-element device int32 tensor.  Returns the
        device logits.  Monte ops read their LFSR start from lfsr_dev, so
        one graph serves every step."""
        torch = self.torch
        self._check_ctx(self.n_past, 1)
        n_kv = n_kv or n_kv_for(self.n_past + 1, self.cfg.n_ctx)
        self._check_ctx(self.n_past, 1, n_kv)
        tok = self._buf("gtok", 1, torch.int32)
        pos = self._buf("gpos", 1, torch.int32)
        if isinstance(token, torch.Tensor):
            tok[:1].copy_(token.reshape(-1)[:1])
        else:
            tok.fill_(int(token))
        pos.fill_(self.n_past)
        out = self._replay(n_kv, lambda: self.forward(1, tok, pos, n_kv))
        self.n_past += 1
        return out


# the most cells for which LlamaLNS32 runs a decode step's attention as one
# launch (one kq chain per lane of a 256-lane workgroup)
ATTN32_FUSED_KV = 256

LLAMA_1B = LlamaConfig(n_layer=16, n_embd=2048, n_head=32, n_head_kv=8, head_dim=64, n_ff=8192, n_vocab=32000,
                       n_ctx=1024)


class LlamaLNS32:
    """The decoder as the reference's LNS32 backend computes it
    (src32/lns32-ops.cpp), one sequence: get_rows copies the F32 embedding
    rows (:707-745), every other op runs in xlns32 with F32 at its boundaries,
    the weights are packed xlns32 (4 bytes each) and the KV cache holds the
    xlns32 codes of the IEEE-half-rounded K / V values (llama.cpp's F16 cache
    as lns32_mul_mat converts it, :64-79).  weights may hold host arrays or
    device tensors (float32)."""

    def __init__(self, cfg, weights, device=None):
        import torch
        init()
        self.cfg = cfg
        self.torch = torch
        # device: where the weights, caches and buffers live (default the
        # current GPU; a CPU device lets a test audit the launch arguments
        # against the allocations with a recording stand-in for the library)
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.dev = dev
        c = cfg
        from . import pack32

        def t(a):
            if isinstance(a, torch.Tensor):
                return a.to(dev, torch.float32).contiguous()
            return torch.from_numpy(np.ascontiguousarray(a)).to(dev)

        self.tok_embd_f32 = t(weights["tok_embd"])                  # [vocab, e]: get_rows
        self.tok_embd = pack32(self.tok_embd_f32)                    # the tied output matrix
        self.out_norm = t(weights["out_norm"])
        self.layers = []
        for L in weights["layers"]:
            cat = lambda *a: torch.cat([t(x) for x in a]) if isinstance(a[0], torch.Tensor) else t(np.concatenate(a))
            self.layers.append({
                "attn_norm": t(L["attn_norm"]),
                "wqkv": pack32(cat(L["wq"], L["wk"], L["wv"])),
                "wo": pack32(t(L["wo"])),
                "ffn_norm": t(L["ffn_norm"]),
                "wug": pack32(cat(L["w_up"], L["w_gate"])),
                "wdown": pack32(t(L["w_down"])),
            })
        hd, nkv = c.head_dim, c.n_head_kv
        self.kslice = kp(hd) * c.n_ctx
        self.vslice = kp(c.n_ctx) * hd
        assert self.kslice == self.vslice
        self.kcache = [torch.zeros(nkv * self.kslice, dtype=torch.int32, device=dev) for _ in range(c.n_layer)]
        self.vcache = [torch.zeros(nkv * self.kslice, dtype=torch.int32, device=dev) for _ in range(c.n_layer)]
        # a single-token step's kq, soft_max and kqv in one launch
        # (lnship32_attn_decode, bit-identical to the three ops) where one
        # round of its workgroup's 256 lanes holds the cells' kq chains: past
        # that the separate kq GEMV, whose chains spread over many CUs, wins
        # (at n_kv 768 the fused step is 1 % slower); fused_attn = False runs
        # the three ops
        self.fused_attn = True
        self._attn_max_kv = min(lib().lnship_max_row(7, 0), ATTN32_FUSED_KV)
        # one row: the rms_norm and norm MUL inside the launch of the mul_mat
        # that reads them (lnship32_mul_mat's rms_norm_w, bit-identical to the
        # separate nodes) where the row fits LDS; False runs them apart
        self.fused_pre = True
        rt = np.empty(c.n_ctx * hd, np.float32)
        check(lib().lnship_rope_table(c.rope_theta, hd, c.n_ctx, ctypes.c_void_p(rt.ctypes.data)))
        self.cos_sin = t(rt)
        self.n_past = 0
        self._bufs = {}
        self._graphs = {}

    _buf = LlamaLNS16._buf
    _check_ctx = LlamaLNS16._check_ctx
    _capture = LlamaLNS16._capture

    def weight_bytes_per_token(self):
        """Bytes of packed weights one decode token reads (4 per weight)."""
        c = self.cfg
        e, f, hd = c.n_embd, c.n_ff, c.head_dim
        per_layer = (c.n_head + 2 * c.n_head_kv) * hd * e + e * c.n_head * hd + 2 * f * e + e * f
        return 4 * (c.n_layer * per_layer + c.n_vocab * e)

    def forward(self, T, tokens_dev, pos_dev, n_kv):
        """Runs T tokens at positions pos_dev[0..T) (device int32) against a
        KV view of n_kv cells; returns the device logits of the last one."""
        torch, c, L = self.torch, self.cfg, lib()
        self._check_ctx(0, T, n_kv)
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        e, hd, nh, nkv, f = c.n_embd, c.head_dim, c.n_head, c.n_head_kv, c.n_ff
        nq, nqkv = nh * hd, (nh + 2 * nkv) * hd
        P = lambda b, off=0: ctypes.c_void_p(b.data_ptr() + off * b.element_size())
        mm = lambda w, x, dst, K, M, N, **kw: mul_mat32_raw(w, x, dst, K, M, N, stream=st, **kw)
        x = self._buf("x", T * e)
        h = self._buf("h", T * e)

        def rms_mm(x_ptr, wn_ptr, w, dst_ptr, K, M, rows):
            """dst = W (rms_norm(x) * wn) for rows rows of K: for one row in
            one launch (lnship32_mul_mat's rms_norm_w), else rms_norm + MUL
            into h, then the mul_mat."""
            if rows == 1 and self.fused_pre:
                from . import MulMatArgs
                a = MulMatArgs(w, x_ptr, dst_ptr, K, M, 1, 1, 1, 1, 1, 0, 0, 0, 0, 0, 0, 0, None, 0, None)
                a.rms_norm_w, a.rms_eps = wn_ptr, c.eps
                rc = L.lnship32_mul_mat(ctypes.byref(a), st)
                if rc != -4:   # LNSHIP_ERANGE: the row does not fit beside the tables
                    check(rc)
                    return
            check(L.lnship32_rms_norm_mul(x_ptr, wn_ptr, P(h), K, rows, c.eps, st))
            mm(w, P(h), dst_ptr, K, M, rows)
        qkv = self._buf("qkv", T * nqkv)
        q = self._buf("q", T * nq)
        kq = self._buf("kq", nh * T * n_kv)
        att = self._buf("att", T * nq)
        o = self._buf("o", T * e)
        ug = self._buf("ug", T * 2 * f)
        sw = self._buf("sw", T * f)
        mask = self._buf("mask", T * n_kv)
        logits = self._buf("logits", c.n_vocab)
        # GET_ROWS of an F32 table is a row copy
        torch.index_select(self.tok_embd_f32, 0, tokens_dev[:T].long(), out=x[: T * e].view(T, e))
        check(L.lnship_causal_mask(P(pos_dev), T, n_kv, P(mask), st))
        from . import SoftMaxArgs
        for il, W in enumerate(self.layers):
            last = il == c.n_layer - 1
            rms_mm(P(x), P(W["attn_norm"]), W["wqkv"].data_ptr(), P(qkv), e, nqkv, T)
            qs = QkvStoreArgs(P(qkv), nqkv, P(pos_dev), T, nh, nkv, hd, hd, P(self.cos_sin), P(q),
                              P(self.kcache[il]), P(self.vcache[il]), c.n_ctx, self.kslice, self.vslice, None, 0)
            check(L.lnship32_rope_store_kv(ctypes.byref(qs), st))
            if T == 1 and self.fused_attn and n_kv <= self._attn_max_kv:
                # the three nodes below in one launch, bit for bit
                aa = AttnArgs(P(q), P(self.kcache[il]), P(self.vcache[il]), c.n_ctx, self.kslice, self.vslice,
                              P(mask), 1.0 / math.sqrt(hd), P(att), nh, nkv, hd, n_kv)
                check(L.lnship32_attn_decode(ctypes.byref(aa), st))
            else:
                mm(self.kcache[il].data_ptr(), P(q), P(kq), hd, n_kv, T, ne02=nkv, ne12=nh, x_ld=nq, x_slice=hd,
                   w_mstride=c.n_ctx, w_slice=self.kslice)
                a = SoftMaxArgs(P(kq), (ctypes.c_int64 * 4)(n_kv, T, nh, 1), P(mask),
                                (ctypes.c_int64 * 4)(n_kv, T, 1, 1), 1.0 / math.sqrt(hd), P(kq), 0)
                check(L.lnship32_soft_max(ctypes.byref(a), st))
                mm(self.vcache[il].data_ptr(), P(kq), P(att), n_kv, hd, T, ne02=nkv, ne12=nh, x_ld=n_kv,
                   x_slice=T * n_kv, w_slice=self.vslice, dst_ld=nq, dst_slice=hd)
            rows = 1 if last else T
            r0 = (T - rows) * e
            if rows == T:   # x += Wo att: the residual ADD inside the mul_mat
                mm(W["wo"].data_ptr(), P(att), P(x), nq, e, T, residual=P(x))
            else:
                mm(W["wo"].data_ptr(), P(att), P(o), nq, e, T)
                check(L.lnship32_add(P(o, r0), P(x, r0), rows * e, rows * e, P(x), st))
            rms_mm(P(x), P(W["ffn_norm"]), W["wug"].data_ptr(), P(ug), e, 2 * f, rows)
            check(L.lnship32_swiglu(P(ug, f), 2 * f, P(ug), 2 * f, P(sw), f, rows, st))
            mm(W["wdown"].data_ptr(), P(sw), P(x), f, e, rows, residual=P(x))
        check(L.lnship32_rms_norm_mul(P(x), P(self.out_norm), P(h), e, 1, c.eps, st))
        mm(self.tok_embd.data_ptr(), P(h), P(logits), e, c.n_vocab, 1)
        return logits[: c.n_vocab]

    def restart(self):
        """Empties the KV cache (positions restart at 0); captured graphs stay
        valid."""
        self.n_past = 0

    def eval(self, tokens):
        """Appends tokens (host list); returns the device logits of the last one."""
        torch = self.torch
        T = len(tokens)
        p0 = self.n_past
        self._check_ctx(p0, T)
        tok = self._buf("tok", T, torch.int32)
        pos = self._buf("pos", T, torch.int32)
        tok[:T].copy_(torch.tensor(tokens, dtype=torch.int32))
        pos[:T].copy_(torch.arange(p0, p0 + T, dtype=torch.int32))
        out = self.forward(T, tok, pos, n_kv_for(p0 + T, self.cfg.n_ctx))
        self.n_past += T
        return out

    def decode_graph(self, token, n_kv=None):
        """One decode step through a captured HIP graph; token is a host int or
        a device int32 tensor of one element.  Returns the device logits."""
        torch = self.torch
        self._check_ctx(self.n_past, 1)
        n_kv = n_kv or n_kv_for(self.n_past + 1, self.cfg.n_ctx)
        self._check_ctx(self.n_past, 1, n_kv)
        tok = self._buf("gtok", 1, torch.int32)
        pos = self._buf("gpos", 1, torch.int32)
        if isinstance(token, torch.Tensor):
            tok[:1].copy_(token.reshape(-1)[:1])
        else:
            tok.fill_(int(token))
        pos.fill_(self.n_past)
        if n_kv not in self._graphs:
            self._graphs[n_kv] = self._capture(lambda: self.forward(1, tok, pos, n_kv))
        g, out = self._graphs[n_kv]
        g.replay()
        self.n_past += 1
        return out
