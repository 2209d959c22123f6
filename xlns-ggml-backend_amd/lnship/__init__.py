"""Python binding of the gfx950 LNS kernels (liblnship.so, include/lnship.h).

Device memory and streams come from torch (torch.cuda tensors on ROCm); every
call goes through the C ABI.  There is no CPU fallback: if liblnship.so is
missing or no GPU is visible, the calls raise.
"""
import ctypes
import os

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_DIR, "liblnship.so")

BASE, MONTE, LPVIP, SUM32 = 0, 1, 2, 3
MODES = {"base": BASE, "monte": MONTE, "lpvip": LPVIP, "sum32": SUM32}

_lib = None
_ready = set()

c_i64 = ctypes.c_int64
c_p = ctypes.c_void_p


class LnshipError(RuntimeError):
    pass


class MulMatArgs(ctypes.Structure):
    _fields_ = [("w", c_p), ("x", c_p), ("dst", c_p), ("K", c_i64), ("M", c_i64), ("N", c_i64),
                ("ne02", c_i64), ("ne03", c_i64), ("ne12", c_i64), ("ne13", c_i64),
                ("x_ld", c_i64), ("x_slice", c_i64), ("monte_seed", ctypes.c_uint16),
                ("w_mstride", c_i64), ("w_slice", c_i64), ("dst_ld", c_i64), ("dst_slice", c_i64),
                ("monte_state", c_p), ("monte_offset", ctypes.c_uint64), ("residual", c_p),
                ("rms_norm_w", c_p), ("rms_eps", ctypes.c_float), ("rms_seed", ctypes.c_uint16),
                ("rms_offset", ctypes.c_uint64), ("glu_up", c_p)]


class SoftMaxArgs(ctypes.Structure):
    _fields_ = [("src", c_p), ("src_ne", c_i64 * 4), ("mask", c_p), ("mask_ne", c_i64 * 4),
                ("scale", ctypes.c_float), ("dst", c_p), ("monte_seed", ctypes.c_uint16),
                ("monte_state", c_p), ("monte_offset", ctypes.c_uint64)]


class MulMatIdArgs(ctypes.Structure):
    _fields_ = [("w", c_p), ("x", c_p), ("ids", c_p), ("dst", c_p), ("K", c_i64), ("M", c_i64),
                ("n_expert", c_i64), ("n_expert_used", c_i64), ("n_tokens", c_i64), ("ne11", c_i64),
                ("x_ld", c_i64), ("ids_ld", c_i64), ("monte_seed", ctypes.c_uint16),
                ("monte_state", c_p), ("monte_offset", ctypes.c_uint64)]


class QkvStoreArgs(ctypes.Structure):
    _fields_ = [("qkv", c_p), ("qkv_ld", c_i64), ("pos", c_p), ("ntok", c_i64), ("n_head", c_i64),
                ("n_head_kv", c_i64), ("head_dim", c_i64), ("rope_n_dims", ctypes.c_int), ("cos_sin", c_p),
                ("q_dst", c_p), ("k_cache", c_p), ("v_cache", c_p), ("cache_m", c_i64), ("k_slice", c_i64),
                ("v_slice", c_i64), ("seq", c_p), ("seq_stride", c_i64)]


class AttnArgs(ctypes.Structure):
    _fields_ = [("q", c_p), ("k_cache", c_p), ("v_cache", c_p), ("cache_m", c_i64), ("k_slice", c_i64),
                ("v_slice", c_i64), ("mask", c_p), ("scale", ctypes.c_float), ("dst", c_p), ("n_head", c_i64),
                ("n_head_kv", c_i64), ("head_dim", c_i64), ("n_kv", c_i64)]


class AttnSeqs(ctypes.Structure):
    _fields_ = [("n_seq", c_i64), ("monte_seed", ctypes.c_uint16 * 3), ("monte_state", c_p),
                ("monte_offset", ctypes.c_uint64 * 3)]


def attn_seqs(n_seq, seeds=(0, 0, 0)):
    """lnship_attn_seqs for n_seq sequences; seeds: the kq, soft_max and kqv
    nodes' Monte seed arguments (seed_fields forms: all three 16-bit states,
    or all three (state, offset) pairs on one device state)."""
    a = AttnSeqs()
    a.n_seq = n_seq
    state = None
    for i, sd in enumerate(seeds):
        seed, st, off = seed_fields(sd)
        a.monte_seed[i] = seed
        a.monte_offset[i] = off or 0
        if st is not None:
            state = st
    a.monte_state = state
    return a


def build():
    import subprocess
    subprocess.check_call(["make", "-s", "-C", PKG_DIR])


def lib():
    """Loads liblnship.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise LnshipError(f"{LIB_PATH} is missing: build it with __graft_entry__.build()")
    L = ctypes.CDLL(LIB_PATH)
    sigs = {
        "lnship_init": (ctypes.c_int, []),
        "lnship_last_error": (ctypes.c_char_p, []),
        "lnship_chain_probe": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, c_i64, c_p, ctypes.POINTER(ctypes.c_double)]),
        "lnship_version": (ctypes.c_char_p, []),
        "lnship_host_table": (c_p, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_size_t)]),
        "lnship16_from_f32": (ctypes.c_int, [c_p, c_p, c_i64, c_p]),
        "lnship16_to_f32": (ctypes.c_int, [c_p, c_p, c_i64, c_p]),
        "lnship32_from_f32": (ctypes.c_int, [c_p, c_p, c_i64, c_p]),
        "lnship32_to_f32": (ctypes.c_int, [c_p, c_p, c_i64, c_p]),
        "lnship16_pack": (ctypes.c_int, [c_p, ctypes.c_int, c_i64, c_i64, c_p, c_i64, c_i64, c_i64, c_p]),
        "lnship32_pack": (ctypes.c_int, [c_p, ctypes.c_int, c_i64, c_i64, c_p, c_i64, c_i64, c_i64, c_p]),
        "lnship16_mul_mat": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(MulMatArgs), c_p]),
        "lnship32_mul_mat": (ctypes.c_int, [ctypes.POINTER(MulMatArgs), c_p]),
        "lnship32_mul_mat_noalloc": (ctypes.c_int, [ctypes.POINTER(MulMatArgs), c_p]),
        "lnship16_rms_norm": (ctypes.c_int, [ctypes.c_int, c_p, c_p, c_i64, c_i64, ctypes.c_float,
                                             ctypes.c_uint16, c_p]),
        "lnship16_rms_norm_state": (ctypes.c_int, [ctypes.c_int, c_p, c_p, c_i64, c_i64, ctypes.c_float,
                                                   c_p, ctypes.c_uint64, c_p]),
        "lnship32_rms_norm": (ctypes.c_int, [c_p, c_p, c_i64, c_i64, ctypes.c_float, c_p]),
        "lnship16_rms_norm_mul": (ctypes.c_int, [ctypes.c_int, c_p, c_p, c_p, c_i64, c_i64, ctypes.c_float,
                                                 ctypes.c_uint16, c_p, ctypes.c_uint64, c_p]),
        "lnship32_rms_norm_mul": (ctypes.c_int, [c_p, c_p, c_p, c_i64, c_i64, ctypes.c_float, c_p]),
        "lnship16_rms_norm_mul_mat": (ctypes.c_int, [ctypes.c_int, c_p, c_p, ctypes.c_float, c_p, c_p, c_i64,
                                                     c_i64, c_p]),
        "lnship16_swiglu_mul_mat": (ctypes.c_int, [ctypes.c_int, c_p, c_p, c_p, c_p, c_p, c_i64, c_i64, c_p]),
        "lnship16_rope_store_kv": (ctypes.c_int, [ctypes.POINTER(QkvStoreArgs), c_p]),
        "lnship16_attn_decode": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(AttnArgs), c_p]),
        "lnship16_attn_decode_seqs": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(AttnArgs), ctypes.POINTER(AttnSeqs),
                                                     c_p]),
        "lnship16_rope_attn_decode": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(QkvStoreArgs),
                                                     ctypes.POINTER(AttnArgs), c_p]),
        "lnship16_rope_attn_decode_seqs": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(QkvStoreArgs),
                                                          ctypes.POINTER(AttnArgs), ctypes.POINTER(AttnSeqs), c_p]),
        "lnship32_attn_decode": (ctypes.c_int, [ctypes.POINTER(AttnArgs), c_p]),
        "lnship_max_row": (c_i64, [ctypes.c_int, ctypes.c_int]),
        "lnship32_rope_store_kv": (ctypes.c_int, [ctypes.POINTER(QkvStoreArgs), c_p]),
        "lnship16_soft_max": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(SoftMaxArgs), c_p]),
        "lnship32_soft_max": (ctypes.c_int, [ctypes.POINTER(SoftMaxArgs), c_p]),
        "lnship16_mul_mat_draws": (ctypes.c_uint64, [ctypes.c_int, c_i64, c_i64, c_i64, c_i64, c_i64]),
        "lnship16_soft_max_draws": (ctypes.c_uint64, [ctypes.c_int, c_i64, c_i64]),
        "lnship16_rms_norm_draws": (ctypes.c_uint64, [ctypes.c_int, c_i64, c_i64]),
        "lnship_lfsr_jump": (ctypes.c_uint16, [ctypes.c_uint16, ctypes.c_uint64]),
        "lnship_lfsr_advance": (ctypes.c_int, [c_p, ctypes.c_uint64, c_p]),
        "lnship16_mul_mat_id": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(MulMatIdArgs), c_p]),
        "lnship32_mul_mat_id": (ctypes.c_int, [ctypes.POINTER(MulMatIdArgs), c_p]),
        "lnship16_mul_mat_id_draws": (ctypes.c_uint64, [ctypes.c_int, c_i64, c_i64, c_i64, c_i64]),
        "lnship16_scale": (ctypes.c_int, [c_p, c_p, c_i64, ctypes.c_float, ctypes.c_float, c_p]),
        "lnship32_scale": (ctypes.c_int, [c_p, c_p, c_i64, ctypes.c_float, ctypes.c_float, c_p]),
        "lnship_copy": (ctypes.c_int, [c_p, ctypes.c_int, c_p, c_p, c_p, ctypes.c_int, c_p, c_p, c_p]),
        "lnship_get_rows": (ctypes.c_int, [c_p, ctypes.c_int, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_p]),
        "lnship_set_rows": (ctypes.c_int, [c_p, c_p, c_p, c_p, ctypes.c_int, c_p, c_p, c_p, ctypes.c_int, c_p, c_p,
                                           c_p]),
        "lnship_index_error": (ctypes.c_int, [ctypes.POINTER(c_i64), c_p]),
        "lnship_lpvip_db_range": (ctypes.c_int, [ctypes.c_uint32, ctypes.c_uint32, c_p, c_p]),
        "lnship32_add_lds": (ctypes.c_int, [ctypes.c_int, c_p, c_p, c_p, c_i64, c_p]),
        "lnship_test_predict_skew": (ctypes.c_int, [ctypes.c_int]),
        "lnship_test_decode_width": (ctypes.c_int, [ctypes.c_int]),
        "lnship16_add": (ctypes.c_int, [c_p, c_p, c_i64, c_i64, c_p, c_p]),
        "lnship16_mul": (ctypes.c_int, [c_p, c_p, c_i64, c_i64, c_p, c_p]),
        "lnship16_swiglu": (ctypes.c_int, [c_p, c_i64, c_p, c_i64, c_p, c_i64, c_i64, c_p]),
        "lnship16_get_rows_packed": (ctypes.c_int, [c_p, c_i64, c_i64, c_p, c_i64, c_p, c_p]),
        "lnship16_rope": (ctypes.c_int, [c_p, c_i64, c_p, c_i64, c_i64, c_i64, ctypes.c_int, ctypes.c_int, c_p, c_p,
                                         c_p]),
        "lnship16_store_kv": (ctypes.c_int, [c_p, c_i64, c_p, c_i64, c_i64, c_i64, ctypes.c_int, c_p, c_p, c_i64,
                                             c_i64, ctypes.c_int, c_p, c_i64, c_p]),
        "lnship32_add": (ctypes.c_int, [c_p, c_p, c_i64, c_i64, c_p, c_p]),
        "lnship32_mul": (ctypes.c_int, [c_p, c_p, c_i64, c_i64, c_p, c_p]),
        "lnship32_swiglu": (ctypes.c_int, [c_p, c_i64, c_p, c_i64, c_p, c_i64, c_i64, c_p]),
        "lnship32_rope": (ctypes.c_int, [c_p, c_i64, c_p, c_i64, c_i64, c_i64, ctypes.c_int, ctypes.c_int, c_p, c_p,
                                         c_p]),
        "lnship32_store_kv": (ctypes.c_int, [c_p, c_i64, c_p, c_i64, c_i64, c_i64, ctypes.c_int, c_p, c_p, c_i64,
                                             c_i64, ctypes.c_int, c_p, c_i64, c_p]),
        "lnship_causal_mask": (ctypes.c_int, [c_p, c_i64, c_i64, c_p, c_p]),
        "lnship_rope_table": (ctypes.c_int, [ctypes.c_float, ctypes.c_int, c_i64, c_p]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def host_table(name, dtype):
    """Host copy of one of the library's arithmetic tables (numpy; no GPU)."""
    import numpy as np
    n = ctypes.c_size_t(0)
    p = lib().lnship_host_table(name.encode(), ctypes.byref(n))
    if not p:
        raise LnshipError(lib().lnship_last_error().decode())
    buf = (ctypes.c_char * n.value).from_address(p)
    return np.frombuffer(buf, dtype=dtype).copy()


def check(rc):
    if rc != 0:
        raise LnshipError(f"lnship error {rc}: {lib().lnship_last_error().decode()}")


def init(device=None):
    """Uploads the tables to the current (or given) torch device."""
    import torch
    if not torch.cuda.is_available():
        raise LnshipError("no GPU visible: the LNS kernels have no CPU fallback")
    dev = torch.cuda.current_device() if device is None else device
    with torch.cuda.device(dev):
        if dev not in _ready:
            check(lib().lnship_init())
            _ready.add(dev)


def _stream():
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def kp(K):
    return (K + 7) & ~7


# ---- conversions -------------------------------------------------------------

def from_f32_16(x):
    import torch
    init()
    x = x.contiguous()
    out = torch.empty(x.shape, dtype=torch.int16, device=x.device)
    check(lib().lnship16_from_f32(_p(x), _p(out), x.numel(), _stream()))
    return out


def to_f32_16(v):
    import torch
    init()
    v = v.contiguous()
    out = torch.empty(v.shape, dtype=torch.float32, device=v.device)
    check(lib().lnship16_to_f32(_p(v), _p(out), v.numel(), _stream()))
    return out


def from_f32_32(x):
    import torch
    init()
    x = x.contiguous()
    out = torch.empty(x.shape, dtype=torch.int32, device=x.device)
    check(lib().lnship32_from_f32(_p(x), _p(out), x.numel(), _stream()))
    return out


def to_f32_32(v):
    import torch
    init()
    v = v.contiguous()
    out = torch.empty(v.shape, dtype=torch.float32, device=v.device)
    check(lib().lnship32_to_f32(_p(v), _p(out), v.numel(), _stream()))
    return out


def pack16(w, dtype=None):
    """w [..., M, K] (float32, float16, or int16 xlns16 codes) -> k8-interleaved xlns16 cache [slices, Kp*M] (int16)."""
    import torch
    init()
    w = w.contiguous()
    K, M = w.shape[-1], w.shape[-2]
    ns = w.numel() // max(1, K * M)
    out = torch.empty((ns, kp(K) * M), dtype=torch.int16, device=w.device)
    src_type = 2 if w.dtype == torch.int16 else int(w.dtype == torch.float16)   # int16: xlns16 codes
    check(lib().lnship16_pack(_p(w), src_type, K, K * M, _p(out), K, M, ns, _stream()))
    return out


def pack32(w):
    import torch
    init()
    w = w.contiguous()
    K, M = w.shape[-1], w.shape[-2]
    ns = w.numel() // max(1, K * M)
    out = torch.empty((ns, kp(K) * M), dtype=torch.int32, device=w.device)
    check(lib().lnship32_pack(_p(w), int(w.dtype == torch.float16), K, K * M, _p(out), K, M, ns, _stream()))
    return out


# ---- ops ---------------------------------------------------------------------

def seed_fields(seed):
    """A Monte seed argument -> (monte_seed, monte_state, monte_offset).

    seed is either the 16-bit start state itself, or a pair (state, offset):
    a device uint16 (tensor or pointer) holding the LFSR state, read when the
    op runs, and the jump from it to the op's first draw."""
    if isinstance(seed, tuple):
        st, off = seed
        return 0, (st if isinstance(st, int) else _p(st)), off
    return seed, None, 0


def _mm_args(wp, x, out, K, M, ne02, ne03, seed):
    N = x.shape[-2]
    ne12 = x.shape[-3] if x.dim() >= 3 else 1
    ne13 = x.shape[-4] if x.dim() >= 4 else 1
    sd, st, off = seed_fields(seed)
    return MulMatArgs(_p(wp), _p(x), _p(out), K, M, N, ne02, ne03, ne12, ne13, 0, 0, sd, 0, 0, 0, 0, st, off)


def mul_mat16_raw(mode, w_ptr, x_ptr, dst_ptr, K, M, N, ne02=1, ne03=1, ne12=1, ne13=1, x_ld=0, x_slice=0,
                  seed=7, w_mstride=0, w_slice=0, dst_ld=0, dst_slice=0, stream=None, residual=None):
    """mul_mat on raw device pointers (ints), with every stride of the C ABI;
    residual (a pointer laid out as dst) adds the following ADD node."""
    sd, st, off = seed_fields(seed)
    a = MulMatArgs(w_ptr, x_ptr, dst_ptr, K, M, N, ne02, ne03, ne12, ne13, x_ld, x_slice, sd,
                   w_mstride, w_slice, dst_ld, dst_slice, st, off, residual)
    check(lib().lnship16_mul_mat(mode, ctypes.byref(a), stream if stream is not None else _stream()))


def mul_mat16(mode, wp, x, K, M, ne02=1, ne03=1, seed=7, out=None):
    """wp: packed weights (pack16), x: [ne13, ne12, N, K] float32 -> [..., N, M] float32."""
    import torch
    init()
    x = x.contiguous()
    if out is None:
        out = torch.empty(x.shape[:-1] + (M,), dtype=torch.float32, device=x.device)
    a = _mm_args(wp, x, out, K, M, ne02, ne03, seed)
    check(lib().lnship16_mul_mat(mode, ctypes.byref(a), _stream()))
    return out


def mul_mat32_raw(w_ptr, x_ptr, dst_ptr, K, M, N, ne02=1, ne03=1, ne12=1, ne13=1, x_ld=0, x_slice=0,
                  w_mstride=0, w_slice=0, dst_ld=0, dst_slice=0, stream=None, residual=None):
    """xlns32 mul_mat on raw device pointers (ints), with every stride of the
    C ABI; residual as in mul_mat16_raw."""
    a = MulMatArgs(w_ptr, x_ptr, dst_ptr, K, M, N, ne02, ne03, ne12, ne13, x_ld, x_slice, 0,
                   w_mstride, w_slice, dst_ld, dst_slice, None, 0, residual)
    check(lib().lnship32_mul_mat(ctypes.byref(a), stream if stream is not None else _stream()))


def mul_mat32(wp, x, K, M, ne02=1, ne03=1, out=None):
    import torch
    init()
    x = x.contiguous()
    if out is None:
        out = torch.empty(x.shape[:-1] + (M,), dtype=torch.float32, device=x.device)
    a = _mm_args(wp, x, out, K, M, ne02, ne03, 0)
    check(lib().lnship32_mul_mat(ctypes.byref(a), _stream()))
    return out


def mul_mat_id(mode, wp, x, ids, K, M, n_expert, seed=7, out=None):
    """MUL_MAT_ID: wp packed experts (pack16 / pack32 of [n_expert, M, K]),
    x [T, ne11, K] float32, ids [T, n_expert_used] int32 (device) ->
    [T, n_expert_used, M] float32.  mode None: xlns32."""
    import torch
    init()
    x = x.contiguous()
    ids = ids.contiguous()
    T, ne11 = x.shape[0], x.shape[1]
    neu = ids.shape[1]
    if out is None:
        out = torch.empty((T, neu, M), dtype=torch.float32, device=x.device)
    sd, st, off = seed_fields(seed)
    a = MulMatIdArgs(_p(wp), _p(x), _p(ids), _p(out), K, M, n_expert, neu, T, ne11, 0, 0, sd, st, off)
    if mode is None:
        check(lib().lnship32_mul_mat_id(ctypes.byref(a), _stream()))
    else:
        check(lib().lnship16_mul_mat_id(mode, ctypes.byref(a), _stream()))
    return out


def rms_norm16(mode, x, eps, seed=7, out=None):
    import torch
    init()
    x = x.contiguous()
    if out is None:
        out = torch.empty_like(x)
    ncols = x.shape[-1]
    sd, st, off = seed_fields(seed)
    if st is not None:
        check(lib().lnship16_rms_norm_state(mode, _p(x), _p(out), ncols, x.numel() // max(1, ncols), eps, st, off,
                                            _stream()))
    else:
        check(lib().lnship16_rms_norm(mode, _p(x), _p(out), ncols, x.numel() // max(1, ncols), eps, sd,
                                      _stream()))
    return out


def rms_norm32(x, eps, out=None):
    import torch
    init()
    x = x.contiguous()
    if out is None:
        out = torch.empty_like(x)
    ncols = x.shape[-1]
    check(lib().lnship32_rms_norm(_p(x), _p(out), ncols, x.numel() // max(1, ncols), eps, _stream()))
    return out


def _ne4(shape):
    s = list(shape)[::-1]
    return (c_i64 * 4)(*(s + [1] * (4 - len(s))))


def _sm_args(x, mask, scale, out, seed):
    ne = _ne4(x.shape)
    mne = _ne4(mask.shape) if mask is not None else (c_i64 * 4)(*ne)
    sd, st, off = seed_fields(seed)
    return SoftMaxArgs(_p(x), ne, _p(mask), mne, scale, _p(out), sd, st, off)


def soft_max16(mode, x, mask=None, scale=1.0, seed=7, out=None):
    import torch
    init()
    x = x.contiguous()
    mask = mask.contiguous() if mask is not None else None
    if out is None:
        out = torch.empty_like(x)
    a = _sm_args(x, mask, scale, out, seed)
    check(lib().lnship16_soft_max(mode, ctypes.byref(a), _stream()))
    return out


def soft_max32(x, mask=None, scale=1.0, out=None):
    import torch
    init()
    x = x.contiguous()
    mask = mask.contiguous() if mask is not None else None
    if out is None:
        out = torch.empty_like(x)
    a = _sm_args(x, mask, scale, out, 0)
    check(lib().lnship32_soft_max(ctypes.byref(a), _stream()))
    return out


def mul_mat_draws(mode, K, M, N, ne12=1, ne13=1):
    return lib().lnship16_mul_mat_draws(mode, K, M, N, ne12, ne13)


def lfsr_jump(state, n):
    return lib().lnship_lfsr_jump(state, n)


def lfsr_advance(state, draws):
    """state (a device uint16 tensor) <- lfsr_jump(state, draws), in stream order."""
    init()
    check(lib().lnship_lfsr_advance(_p(state), draws, _stream()))
