"""ctypes loader for the CPU oracle (oracle/liblnsoracle.so).

Test infrastructure: only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg use this module, and only as the checker.
"""
import ctypes
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE_SO = os.environ.get("LNS_ORACLE_SO", os.path.join(ORACLE_DIR, "liblnsoracle.so"))

BASE, MONTE, LPVIP, SUM32 = 0, 1, 2, 3
MODES = {"base": BASE, "monte": MONTE, "lpvip": LPVIP, "sum32": SUM32}

_lib = None

u16, u32, i64, f32 = ctypes.c_uint16, ctypes.c_uint32, ctypes.c_int64, ctypes.c_float
P = ctypes.c_void_p
SZ = ctypes.c_size_t


def build():
    subprocess.check_call(["make", "-s", "-C", ORACLE_DIR])


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(ORACLE_SO):
        build()
    L = ctypes.CDLL(ORACLE_SO)
    sig = {
        "lno_init": (ctypes.c_int, []),
        "lno16_from_f32": (u16, [f32]),
        "lno16_to_f32": (f32, [u16]),
        "lno16_from_f32_n": (None, [P, P, SZ]),
        "lno16_to_f32_n": (None, [P, P, SZ]),
        "lno16_mul": (u16, [u16, u16]),
        "lno16_div": (u16, [u16, u16]),
        "lno16_add": (u16, [u16, u16]),
        "lno16_sub": (u16, [u16, u16]),
        "lno16_sqrt": (u16, [u16]),
        "lno16_recip": (u16, [u16]),
        "lno16_exp": (u16, [u16]),
        "lno16_gt": (ctypes.c_int, [u16, u16]),
        "lno16_cvt_table": (P, []),
        "lno16_sb_table": (P, []),
        "lno16_db_table": (P, []),
        "lno16_exp_table": (P, []),
        "lno16_widen": (u32, [u16]),
        "lno16_narrow_sum32": (u16, [u32]),
        "lno16_narrow_lpvip": (u16, [u32]),
        "lno16_sum": (u16, [ctypes.c_int, P, SZ, P]),
        "lno16_vec_dot": (u16, [ctypes.c_int, P, P, SZ, P]),
        "lno16_rms_norm_row": (None, [ctypes.c_int, P, P, SZ, u16, P]),
        "lno16_softmax_row": (None, [ctypes.c_int, P, P, P, SZ, u16, P]),
        "lno16_add_monte": (u16, [u16, u16, P]),
        "lno16_monte_threshold_n": (None, [ctypes.c_int, ctypes.c_int, P]),
        "lno16_lpvip_add": (u32, [u32, u16]),
        "lno32_lpvip_db_n": (None, [u32, u32, P]),
        "lno_lfsr_step": (u16, [u16]),
        "lno_lfsr_jump": (u16, [u16, ctypes.c_uint64]),
        "lno_monte_get_state": (ctypes.c_int, [P]),
        "lno_monte_set_state": (ctypes.c_int, [u16]),
        "lno_monte_reserve": (ctypes.c_int, [ctypes.c_uint64, P]),
        "lno32_from_f32": (u32, [f32]),
        "lno32_to_f32": (f32, [u32]),
        "lno32_from_f32_n": (None, [P, P, SZ]),
        "lno32_to_f32_n": (None, [P, P, SZ]),
        "lno32_mul": (u32, [u32, u32]),
        "lno32_div": (u32, [u32, u32]),
        "lno32_add": (u32, [u32, u32]),
        "lno32_set_variant": (ctypes.c_int, [ctypes.c_int]),
        "lno32_sub": (u32, [u32, u32]),
        "lno32_sqrt": (u32, [u32]),
        "lno32_recip": (u32, [u32]),
        "lno32_exp": (u32, [u32]),
        "lno32_gt": (ctypes.c_int, [u32, u32]),
        "lno32_table": (P, [ctypes.c_char_p, ctypes.POINTER(SZ)]),
        "lno32_vec_dot": (u32, [P, P, SZ]),
        "lno32_rms_norm_row": (None, [P, P, SZ, u32]),
        "lno32_softmax_row": (None, [P, P, P, SZ, u32]),
        "lno16_mul_mat": (None, [ctypes.c_int, P, P, P, i64, i64, i64, i64, i64, i64, i64]),
        "lno16_mul_mat_f32w": (None, [ctypes.c_int, P, P, P, i64, i64, i64, i64, i64, i64, i64]),
        "lno16_soft_max": (None, [ctypes.c_int, P, P, P, P, f32, P]),
        "lno16_rms_norm": (None, [ctypes.c_int, P, i64, i64, f32, P]),
        "lno32_mul_mat": (None, [P, P, P, i64, i64, i64, i64, i64, i64, i64]),
        "lno32_mul_mat_lnsw": (None, [P, P, P, i64, i64, i64, i64, i64, i64, i64]),
        "lno32_soft_max": (None, [P, P, P, P, f32, P]),
        "lno32_rms_norm": (None, [P, i64, i64, f32, P]),
        "lno32_silu": (u32, [u32]),
        "lno16_mul_mat_id": (None, [ctypes.c_int, P, P, P, P, i64, i64, i64, i64, i64, i64]),
        "lno32_mul_mat_id": (None, [P, P, P, P, i64, i64, i64, i64, i64, i64]),
        "lno16_scale_f32": (None, [P, i64, f32, f32, P]),
        "lno32_scale_f32": (None, [P, i64, f32, f32, P]),
        "lno32_add_f32": (None, [P, P, i64, i64, P]),
        "lno32_mul_f32": (None, [P, P, i64, i64, P]),
        "lno32_swiglu_f32": (None, [P, P, i64, P]),
        "lno32_rope_f32": (None, [P, P, i64, i64, i64, ctypes.c_int, ctypes.c_int, f32, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    L.lno_init()
    _lib = L
    return L


# ---- numpy conveniences --------------------------------------------------

def f2x16(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().lno16_from_f32_n(_ptr(x), _ptr(out), x.size)
    return out


def x2f16(v):
    v = np.ascontiguousarray(v, dtype=np.uint16)
    out = np.empty(v.shape, dtype=np.float32)
    lib().lno16_to_f32_n(_ptr(v), _ptr(out), v.size)
    return out


def f2x32(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint32)
    lib().lno32_from_f32_n(_ptr(x), _ptr(out), x.size)
    return out


def x2f32(v):
    v = np.ascontiguousarray(v, dtype=np.uint32)
    out = np.empty(v.shape, dtype=np.float32)
    lib().lno32_to_f32_n(_ptr(v), _ptr(out), v.size)
    return out


def table(name, n, dtype):
    p = getattr(lib(), name)()
    buf = (ctypes.c_char * (n * np.dtype(dtype).itemsize)).from_address(p)
    return np.frombuffer(buf, dtype=dtype).copy()


def table32(name):
    n = SZ(0)
    p = lib().lno32_table(name.encode(), ctypes.byref(n))
    buf = (ctypes.c_char * (n.value * 4)).from_address(p)
    return np.frombuffer(buf, dtype=np.int32).copy()


def sum16(mode, a, lfsr=None):
    a = np.ascontiguousarray(a, dtype=np.uint16)
    st = np.array([lfsr if lfsr is not None else 7], dtype=np.uint16)
    return lib().lno16_sum(mode, _ptr(a), a.size, _ptr(st))


def vec_dot16(mode, a, b, lfsr=None):
    a = np.ascontiguousarray(a, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    st = np.array([lfsr if lfsr is not None else 7], dtype=np.uint16)
    return lib().lno16_vec_dot(mode, _ptr(a), _ptr(b), a.size, _ptr(st))


def rms_norm_row16(mode, x, eps, lfsr=None):
    x = np.ascontiguousarray(x, dtype=np.uint16)
    out = np.empty_like(x)
    st = np.array([lfsr if lfsr is not None else 7], dtype=np.uint16)
    lib().lno16_rms_norm_row(mode, _ptr(x), _ptr(out), x.size, eps, _ptr(st))
    return out


def mul_mat16(mode, w_codes, x, ne02=1, ne03=1):
    """w_codes [ne03, ne02, M, K] uint16, x [ne13, ne12, N, K] float32 -> [ne13, ne12, N, M]"""
    w = np.ascontiguousarray(w_codes, dtype=np.uint16)
    x = np.ascontiguousarray(x, dtype=np.float32)
    K = w.shape[-1]
    M = w.shape[-2]
    N = x.shape[-2]
    ne12 = x.shape[-3] if x.ndim >= 3 else 1
    ne13 = x.shape[-4] if x.ndim >= 4 else 1
    out = np.zeros(x.shape[:-1] + (M,), dtype=np.float32)
    lib().lno16_mul_mat(mode, _ptr(w), _ptr(x), _ptr(out), K, M, N, ne02, ne03, ne12, ne13)
    return out


def mul_mat16_f32w(mode, w, x, ne02=1, ne03=1):
    w = np.ascontiguousarray(w, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    K = w.shape[-1]
    M = w.shape[-2]
    N = x.shape[-2]
    ne12 = x.shape[-3] if x.ndim >= 3 else 1
    ne13 = x.shape[-4] if x.ndim >= 4 else 1
    out = np.zeros(x.shape[:-1] + (M,), dtype=np.float32)
    lib().lno16_mul_mat_f32w(mode, _ptr(w), _ptr(x), _ptr(out), K, M, N, ne02, ne03, ne12, ne13)
    return out


def _ne4(shape):
    s = list(shape)[::-1]
    return np.array(s + [1] * (4 - len(s)), dtype=np.int64)


def soft_max16(mode, src, mask=None, scale=1.0):
    src = np.ascontiguousarray(src, dtype=np.float32)
    out = np.empty_like(src)
    ne = _ne4(src.shape)
    if mask is not None:
        mask = np.ascontiguousarray(mask, dtype=np.float32)
        mne = _ne4(mask.shape)
    else:
        mne = ne.copy()
    lib().lno16_soft_max(mode, _ptr(src), _ptr(ne), _ptr(mask), _ptr(mne), scale, _ptr(out))
    return out


def rms_norm16(mode, src, eps):
    src = np.ascontiguousarray(src, dtype=np.float32)
    out = np.empty_like(src)
    ncols = src.shape[-1]
    lib().lno16_rms_norm(mode, _ptr(src), ncols, src.size // max(ncols, 1), eps, _ptr(out))
    return out


def mul_mat32(w, x, ne02=1, ne03=1):
    w = np.ascontiguousarray(w, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    K = w.shape[-1]
    M = w.shape[-2]
    N = x.shape[-2]
    ne12 = x.shape[-3] if x.ndim >= 3 else 1
    ne13 = x.shape[-4] if x.ndim >= 4 else 1
    out = np.zeros(x.shape[:-1] + (M,), dtype=np.float32)
    lib().lno32_mul_mat(_ptr(w), _ptr(x), _ptr(out), K, M, N, ne02, ne03, ne12, ne13)
    return out


def mul_mat32_codes(w_codes, x, ne02=1, ne03=1):
    """mul_mat32 with the weights already converted to xlns32 codes."""
    w = np.ascontiguousarray(w_codes, dtype=np.uint32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    K = w.shape[-1]
    M = w.shape[-2]
    N = x.shape[-2]
    ne12 = x.shape[-3] if x.ndim >= 3 else 1
    ne13 = x.shape[-4] if x.ndim >= 4 else 1
    out = np.zeros(x.shape[:-1] + (M,), dtype=np.float32)
    lib().lno32_mul_mat_lnsw(_ptr(w), _ptr(x), _ptr(out), K, M, N, ne02, ne03, ne12, ne13)
    return out


def _binop32(fn, a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    out = np.empty_like(a)
    fn(_ptr(a), _ptr(b), a.size, b.size, _ptr(out))
    return out


def add32(a, b):
    """lns32_add of F32 tensors, b repeated over a's rows."""
    return _binop32(lib().lno32_add_f32, a, b)


def mul32(a, b):
    """lns32_mul of F32 tensors, b repeated over a's rows."""
    return _binop32(lib().lno32_mul_f32, a, b)


def mul_mat_id(mode, w, x, ids):
    """MUL_MAT_ID: w [n_expert][M][K] F32 (xlns16 via fp2xlns16, or xlns32
    when mode is None), x [T][ne11][K] F32, ids [T][n_expert_used] int32
    -> [T][n_expert_used][M] F32."""
    w = np.ascontiguousarray(w, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    ids = np.ascontiguousarray(ids, np.int32)
    E, M, K = w.shape
    T, ne11, _ = x.shape
    neu = ids.shape[1]
    out = np.zeros((T, neu, M), np.float32)
    if mode is None:
        lib().lno32_mul_mat_id(_ptr(w), _ptr(x), _ptr(ids), _ptr(out), K, M, E, neu, T, ne11)
    else:
        wc = f2x16(w)
        lib().lno16_mul_mat_id(mode, _ptr(wc), _ptr(x), _ptr(ids), _ptr(out), K, M, E, neu, T, ne11)
    return out


def scale(w32, x, s, b=0.0):
    """SCALE (y = x s, + b when b != 0) in xlns16 (w32 False) or xlns32."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    (lib().lno32_scale_f32 if w32 else lib().lno16_scale_f32)(_ptr(x), x.size, s, b, _ptr(out))
    return out


def swiglu32(gate, up):
    gate = np.ascontiguousarray(gate, np.float32)
    up = np.ascontiguousarray(up, np.float32)
    out = np.empty_like(up)
    lib().lno32_swiglu_f32(_ptr(gate), _ptr(up), up.size, _ptr(out))
    return out


def rope32(x, pos, n_dims, neox, freq_base):
    """x [ntok][nhead][ne0] F32, pos [ntok] int32."""
    x = np.ascontiguousarray(x, np.float32)
    pos = np.ascontiguousarray(pos, np.int32)
    out = np.empty_like(x)
    lib().lno32_rope_f32(_ptr(x), _ptr(pos), x.shape[0], x.shape[1], x.shape[2], n_dims, neox, freq_base,
                         _ptr(out))
    return out


def soft_max32(src, mask=None, scale=1.0):
    src = np.ascontiguousarray(src, dtype=np.float32)
    out = np.empty_like(src)
    ne = _ne4(src.shape)
    if mask is not None:
        mask = np.ascontiguousarray(mask, dtype=np.float32)
        mne = _ne4(mask.shape)
    else:
        mne = ne.copy()
    lib().lno32_soft_max(_ptr(src), _ptr(ne), _ptr(mask), _ptr(mne), scale, _ptr(out))
    return out


def rms_norm32(src, eps):
    src = np.ascontiguousarray(src, dtype=np.float32)
    out = np.empty_like(src)
    ncols = src.shape[-1]
    lib().lno32_rms_norm(_ptr(src), ncols, src.size // max(ncols, 1), eps, _ptr(out))
    return out


def monte_set(state):
    return lib().lno_monte_set_state(state)


def monte_get():
    st = np.zeros(1, dtype=np.uint16)
    lib().lno_monte_get_state(_ptr(st))
    return int(st[0])
