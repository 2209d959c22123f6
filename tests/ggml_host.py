"""A test-only ggml host for the LNSHIP backends (TEST INFRASTRUCTURE).

ctypes mirrors of the ggml structures the backends read (ggml_tensor, the
leading members of ggml_cgraph) and fill (registry / device / backend
vtables, device props), over tests/ggml_host/libggml_host.so, which stands in
for the ggml-base functions libggml-lnship.so imports.  Tests build small
graphs of host tensors backed by numpy arrays and call the backend through
its vtables the way ggml's scheduler does.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
STUB_SRC = os.path.join(HERE, "ggml_host", "ggml_host.c")
STUB_SO = os.path.join(HERE, "ggml_host", "libggml_host.so")
BACKEND_SO = os.path.join(ROOT, "xlns-ggml-backend_amd", "libggml-lnship.so")
ABI_DIR = os.path.join(ROOT, "xlns-ggml-backend_amd", "csrc")

FLAG_COMPUTE = 16
USAGE_ANY, USAGE_WEIGHTS, USAGE_COMPUTE = 0, 1, 2
TYPES = {"f32": (0, 4, 1), "f16": (1, 2, 1), "q8_0": (8, 34, 32), "q4_k": (12, 144, 256), "i32": (26, 4, 1), "i64": (27, 8, 1), "lns16": (43, 2, 1)}


LNSHIP_SO = os.path.join(ROOT, "xlns-ggml-backend_amd", "liblnship.so")


def lnship_max_row(which, mode):
    """liblnship's row limits (no GPU needed)."""
    lib = ctypes.CDLL(LNSHIP_SO)
    lib.lnship_max_row.restype = ctypes.c_int64
    lib.lnship_max_row.argtypes = [ctypes.c_int, ctypes.c_int]
    return lib.lnship_max_row(which, mode)


def build_stub():
    """Compiles the stub when it is missing or older than its source."""
    if os.path.exists(STUB_SO) and os.path.getmtime(STUB_SO) >= os.path.getmtime(STUB_SRC):
        return
    subprocess.check_call(["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-Wall", "-I" + ABI_DIR,
                           "-o", STUB_SO, STUB_SRC])


class Tensor(ctypes.Structure):
    _fields_ = [("type", ctypes.c_int), ("buffer", ctypes.c_void_p), ("ne", ctypes.c_int64 * 4),
                ("nb", ctypes.c_size_t * 4), ("op", ctypes.c_int), ("op_params", ctypes.c_int32 * 16),
                ("flags", ctypes.c_int32), ("src", ctypes.c_void_p * 10), ("view_src", ctypes.c_void_p),
                ("view_offs", ctypes.c_size_t), ("data", ctypes.c_void_p), ("name", ctypes.c_char * 64),
                ("extra", ctypes.c_void_p), ("padding", ctypes.c_char * 8)]


class Graph(ctypes.Structure):
    _fields_ = [("size", ctypes.c_int), ("n_nodes", ctypes.c_int), ("n_leafs", ctypes.c_int),
                ("nodes", ctypes.POINTER(ctypes.POINTER(Tensor))), ("rest", ctypes.c_void_p * 16)]


BACKEND_SLOTS = ["get_name", "free", "set_tensor_async", "get_tensor_async", "set_tensor_2d_async",
                 "get_tensor_2d_async", "cpy_tensor_async", "synchronize", "graph_plan_create", "graph_plan_free",
                 "graph_plan_update", "graph_plan_compute", "graph_compute", "event_record", "event_wait",
                 "graph_optimize"]
DEVICE_SLOTS = ["get_name", "get_description", "get_memory", "get_type", "get_props", "init_backend",
                "get_buffer_type", "get_host_buffer_type", "buffer_from_host_ptr", "supports_op", "supports_buft",
                "offload_op", "event_new", "event_free", "event_synchronize"]
REG_SLOTS = ["get_name", "get_device_count", "get_device", "get_proc_address"]


class BackendI(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in BACKEND_SLOTS]


class Backend(ctypes.Structure):
    _fields_ = [("guid", ctypes.c_void_p), ("iface", BackendI), ("device", ctypes.c_void_p),
                ("context", ctypes.c_void_p)]


class DeviceI(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in DEVICE_SLOTS]


class Device(ctypes.Structure):
    _fields_ = [("iface", DeviceI), ("reg", ctypes.c_void_p), ("context", ctypes.c_void_p)]


class RegI(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in REG_SLOTS]


class Reg(ctypes.Structure):
    _fields_ = [("api_version", ctypes.c_int), ("iface", RegI), ("context", ctypes.c_void_p)]


class DevCaps(ctypes.Structure):
    _fields_ = [("async_", ctypes.c_bool), ("host_buffer", ctypes.c_bool), ("buffer_from_host_ptr", ctypes.c_bool),
                ("events", ctypes.c_bool)]


class DevProps(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("description", ctypes.c_char_p), ("memory_free", ctypes.c_size_t),
                ("memory_total", ctypes.c_size_t), ("type", ctypes.c_int), ("device_id", ctypes.c_char_p),
                ("caps", DevCaps)]


class BufferTypeI(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("get_name", "alloc_buffer", "get_alignment", "get_max_size",
                                               "get_alloc_size", "is_host")]


class BufferType(ctypes.Structure):
    _fields_ = [("iface", BufferTypeI), ("device", ctypes.c_void_p), ("context", ctypes.c_void_p)]


class BufferI(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("free_buffer", "get_base", "init_tensor", "memset_tensor",
                                               "set_tensor", "get_tensor", "cpy_tensor", "clear", "reset")]


class Buffer(ctypes.Structure):
    _fields_ = [("iface", BufferI), ("buft", ctypes.c_void_p), ("context", ctypes.c_void_p),
                ("size", ctypes.c_size_t), ("usage", ctypes.c_int)]


class DeviceBuffer:
    """A buffer of the backend's device buffer type, handed out by a bump
    allocator (256-byte aligned, as the type asks)."""

    def __init__(self, host, addr):
        self.host, self.addr = host, addr
        self.buf = ctypes.cast(addr, ctypes.POINTER(Buffer)).contents
        self.base = call(self.buf.iface.get_base, ctypes.c_void_p, (addr, ctypes.c_void_p))
        self.used = 0

    def alloc(self, nbytes):
        off = (self.used + 255) // 256 * 256
        assert off + nbytes <= self.buf.size, "device buffer too small"
        self.used = off + nbytes
        return self.base + off

    def set(self, t, arr):
        a = np.ascontiguousarray(arr)
        call(self.buf.iface.set_tensor, None, (self.addr, ctypes.c_void_p), (ctypes.addressof(t), ctypes.c_void_p),
             (a.ctypes.data, ctypes.c_void_p), (0, ctypes.c_size_t), (a.nbytes, ctypes.c_size_t))

    def get(self, t, nbytes):
        out = np.empty(nbytes, np.uint8)
        call(self.buf.iface.get_tensor, None, (self.addr, ctypes.c_void_p), (ctypes.addressof(t), ctypes.c_void_p),
             (out.ctypes.data, ctypes.c_void_p), (0, ctypes.c_size_t), (nbytes, ctypes.c_size_t))
        return out

    def free(self):
        call(self.buf.iface.free_buffer, None, (self.addr, ctypes.c_void_p))


def call(addr, restype, *args_and_types):
    """Calls a vtable slot: call(addr, restype, (value, ctype), ...)."""
    fn = ctypes.CFUNCTYPE(restype, *[t for _, t in args_and_types])(addr)
    return fn(*[v for v, _ in args_and_types])


class Host:
    def __init__(self):
        build_stub()
        self.stub = ctypes.CDLL(STUB_SO, mode=ctypes.RTLD_GLOBAL)
        self.lib = ctypes.CDLL(BACKEND_SO)
        s, L = self.stub, self.lib
        for name in ("ggml_host_op", "ggml_host_glu", "ggml_host_unary"):
            getattr(s, name).argtypes = [ctypes.c_char_p]
            getattr(s, name).restype = ctypes.c_int
        s.ggml_host_buffer.argtypes = [ctypes.c_int]
        s.ggml_host_buffer.restype = ctypes.c_void_p
        for name in ("ggml_host_sizeof_tensor", "ggml_host_offsetof_data", "ggml_host_offsetof_name",
                     "ggml_host_offsetof_src"):
            getattr(s, name).restype = ctypes.c_size_t
        for name in ("ggml_backend_lnship16_reg", "ggml_backend_lnship32_reg", "ggml_backend_lnship16_init",
                     "ggml_backend_lnship32_init"):
            getattr(L, name).restype = ctypes.c_void_p
            getattr(L, name).argtypes = []
        L.ggml_backend_is_lnship.argtypes = [ctypes.c_void_p]
        L.ggml_backend_is_lnship.restype = ctypes.c_bool
        L.ggml_backend_lnship16_monte_get_state.argtypes = [ctypes.POINTER(ctypes.c_uint16)]
        L.ggml_backend_lnship16_monte_set_state.argtypes = [ctypes.c_uint16]
        L.ggml_backend_lnship16_monte_reserve.argtypes = [ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint16)]
        for name in ("ggml_backend_lnship16_monte_get_state", "ggml_backend_lnship16_monte_set_state",
                     "ggml_backend_lnship16_monte_reserve"):
            getattr(L, name).restype = ctypes.c_bool
        for name in ("ggml_backend_lnship16_check_op", "ggml_backend_lnship32_check_op"):
            getattr(L, name).argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_char_p)]
            getattr(L, name).restype = ctypes.c_bool
        self.keep = []
        self.weights_buf = s.ggml_host_buffer(USAGE_WEIGHTS)
        self.compute_buf = s.ggml_host_buffer(USAGE_COMPUTE)

    # ---- tensors ----
    def tensor(self, ne, type_name="f32", data=None, nb=None, op="NONE", src=(), params=(), fparams=None,
               name="", weights=False, device=None):
        """A host tensor, or with device (a DeviceBuffer) one in device
        memory.  data: a numpy array (kept alive; copied in for a device
        tensor) or an address (a view's); nb defaults to the contiguous
        strides of ggml."""
        tid, tsize, blck = TYPES[type_name]
        ne = list(ne) + [1] * (4 - len(ne))
        t = Tensor()
        t.type = tid
        t.ne[:] = ne
        if nb is None:
            nb = [tsize, tsize * (ne[0] // blck)]
            nb += [nb[1] * ne[1], nb[1] * ne[1] * ne[2]]
        t.nb[:] = nb
        t.op = self.stub.ggml_host_op(op.encode())
        assert t.op >= 0, op
        for i, p in enumerate(params):
            t.op_params[i] = p
        for i, f in (fparams or {}).items():
            t.op_params[i] = int(np.array([f], np.float32).view(np.int32)[0])
        for i, sct in enumerate(src):
            t.src[i] = ctypes.addressof(sct) if sct is not None else None
        t.name = name.encode()
        if device is not None:
            t.buffer = device.addr
            if isinstance(data, int):
                t.data = data
            else:
                t.data = device.alloc(max(nb[3] * ne[3], 4))
                if data is not None:
                    device.set(t, data)
            t.flags = FLAG_COMPUTE if op not in ("NONE",) else 0
            self.keep.append(t)
            return t
        if data is None:
            nbytes = nb[3] * ne[3]
            data = np.zeros(max(nbytes, 4) // 4 + 1, np.float32)
        if isinstance(data, np.ndarray):
            self.keep.append(data)
            t.data = data.ctypes.data
        else:
            t.data = data
        t.buffer = self.weights_buf if weights else self.compute_buf
        t.flags = FLAG_COMPUTE if op not in ("NONE",) else 0
        self.keep.append(t)
        return t

    def device_buffer(self, size, w32=False):
        """A buffer of the device's default buffer type (the HBM type when
        GGML_LNS_HIP_BUFFERS=device)."""
        d = self.device(w32)
        buft = call(d.iface.get_buffer_type, ctypes.c_void_p, (ctypes.addressof(d), ctypes.c_void_p))
        bt = ctypes.cast(buft, ctypes.POINTER(BufferType)).contents
        addr = call(bt.iface.alloc_buffer, ctypes.c_void_p, (buft, ctypes.c_void_p), (size, ctypes.c_size_t))
        assert addr, "alloc_buffer failed"
        db = DeviceBuffer(self, addr)
        self.keep.append(db)
        return db

    def f32_of(self, t, device=None):
        """Contiguous F32 copy or view of an F32 tensor's data."""
        n = t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3]
        if device is not None:
            return device.get(t, n * 4).view(np.float32).reshape(t.ne[3], t.ne[2], t.ne[1], t.ne[0])
        return np.ctypeslib.as_array((ctypes.c_float * n).from_address(t.data)).reshape(
            t.ne[3], t.ne[2], t.ne[1], t.ne[0])

    def graph(self, nodes):
        arr = (ctypes.POINTER(Tensor) * len(nodes))(*[ctypes.pointer(n) for n in nodes])
        g = Graph(len(nodes), len(nodes), 0, arr)
        self.keep.append((arr, g))
        return g

    # ---- registry / device / backend ----
    def reg(self, w32=False):
        p = (self.lib.ggml_backend_lnship32_reg if w32 else self.lib.ggml_backend_lnship16_reg)()
        return ctypes.cast(p, ctypes.POINTER(Reg)).contents

    def device(self, w32=False):
        r = self.reg(w32)
        p = call(r.iface.get_device, ctypes.c_void_p, (ctypes.addressof(r), ctypes.c_void_p), (0, ctypes.c_size_t))
        return ctypes.cast(p, ctypes.POINTER(Device)).contents

    def supports_op(self, t, w32=False):
        d = self.device(w32)
        return call(d.iface.supports_op, ctypes.c_bool, (ctypes.addressof(d), ctypes.c_void_p),
                    (ctypes.addressof(t), ctypes.c_void_p))

    def check(self, t, w32=False):
        reason = ctypes.c_char_p()
        fn = self.lib.ggml_backend_lnship32_check_op if w32 else self.lib.ggml_backend_lnship16_check_op
        ok = fn(ctypes.addressof(t), ctypes.byref(reason))
        return bool(ok), reason.value.decode()

    def init(self, w32=False):
        p = (self.lib.ggml_backend_lnship32_init if w32 else self.lib.ggml_backend_lnship16_init)()
        return ctypes.cast(p, ctypes.POINTER(Backend)).contents if p else None

    def compute(self, backend, nodes):
        g = self.graph(nodes)
        return call(backend.iface.graph_compute, ctypes.c_int, (ctypes.addressof(backend), ctypes.c_void_p),
                    (ctypes.addressof(g), ctypes.c_void_p))

    def free(self, backend):
        call(backend.iface.free, None, (ctypes.addressof(backend), ctypes.c_void_p))
