"""A ctypes stand-in for the host side of ggml's backend API.

It lays out ggml_tensor / ggml_cgraph and walks the plugin's vtables
(registry -> device -> buffer type -> buffer -> backend) the way ggml-backend
does when llama.cpp loads a backend from GGML_BACKEND_PATH, so the plugin can
be exercised without a llama.cpp checkout.  Struct layouts follow ggml at
llama.cpp 0ec4027a2 as used by the reference plugin (src/ggml-xdna.cpp:361-376,
398-403, 461-489, 516-528, 599-621, 660-671, 696-713).
"""
import ctypes as C

# Any value works for a host that has no ggml_op_name(): the plugin is told
# which op id is MUL_MAT.  This one differs from the compat struct's 18 on
# purpose, so a plugin that hard-codes either is caught.
HOST_OP_MUL_MAT = 29
HOST_OP_RMS_NORM = 24

TYPE_F32 = 0
TYPE_Q4_0 = 2

STATUS_SUCCESS = 0
STATUS_FAILED = -1


class Tensor(C.Structure):
    _fields_ = [
        ("type", C.c_int32),
        ("buffer", C.c_void_p),
        ("ne", C.c_int64 * 4),
        ("nb", C.c_size_t * 4),
        ("op", C.c_int32),
        ("op_params", C.c_int32 * 16),
        ("flags", C.c_int32),
        ("src", C.c_void_p * 10),
        ("view_src", C.c_void_p),
        ("view_offs", C.c_size_t),
        ("data", C.c_void_p),
        ("name", C.c_char * 64),
        ("extra", C.c_void_p),
        ("padding", C.c_char * 8),
    ]


class CGraph(C.Structure):
    _fields_ = [
        ("size", C.c_int),
        ("n_nodes", C.c_int),
        ("n_leafs", C.c_int),
        ("nodes", C.POINTER(C.POINTER(Tensor))),
        ("grads", C.c_void_p),
        ("grad_accs", C.c_void_p),
        ("leafs", C.c_void_p),
    ]


class DevCaps(C.Structure):
    _fields_ = [("async_", C.c_bool), ("host_buffer", C.c_bool), ("buffer_from_host_ptr", C.c_bool),
                ("events", C.c_bool), ("mmap_support", C.c_bool)]


class DevProps(C.Structure):
    _fields_ = [("name", C.c_char_p), ("description", C.c_char_p), ("type", C.c_int),
                ("memory_free", C.c_size_t), ("memory_total", C.c_size_t), ("device_id", C.c_char_p),
                ("caps", DevCaps)]


class CompatTensor(C.Structure):
    """struct ggml_tensor_mi355x of include/ggml-mi355x.h (host pointers)."""
    _fields_ = [
        ("type", C.c_int32),
        ("ne", C.c_int64 * 4),
        ("nb", C.c_size_t * 4),
        ("op", C.c_uint32),
        ("op_params", C.c_int32 * 16),
        ("flags", C.c_int32),
        ("src", C.c_void_p * 10),
        ("data", C.c_void_p),
        ("name", C.c_char * 64),
        ("extra", C.c_void_p),
    ]


COMPAT_OP_RMS_NORM = 15
COMPAT_OP_MUL_MAT = 18

assert C.sizeof(Tensor) == 336
assert CGraph.nodes.offset == 16


def bind_compat(lib):
    """ctypes signatures of the plugin's exported (non-vtable) entry points."""
    lib.ggml_backend_init.restype = C.c_void_p
    lib.ggml_backend_init.argtypes = []
    lib.ggml_backend_score.restype = C.c_int
    lib.ggml_backend_mi355x_reg.restype = C.c_void_p
    lib.ggml_backend_mi355x_init.restype = C.c_void_p
    lib.ggml_backend_mi355x_init.argtypes = [C.c_size_t]
    lib.ggml_backend_is_mi355x.restype = C.c_bool
    lib.ggml_backend_is_mi355x.argtypes = [C.c_void_p]
    lib.ggml_backend_mi355x_free.restype = None
    lib.ggml_backend_mi355x_free.argtypes = [C.c_void_p]
    lib.ggml_backend_mi355x_buffer_type.restype = C.c_void_p
    lib.ggml_backend_mi355x_buffer_type.argtypes = [C.c_size_t]
    lib.ggml_backend_mi355x_host_buffer_type.restype = C.c_void_p
    lib.ggml_backend_mi355x_graph_compute.restype = C.c_int
    lib.ggml_backend_mi355x_graph_compute.argtypes = [C.c_void_p, C.c_void_p]
    lib.ggml_backend_mi355x_supports_op.restype = C.c_bool
    lib.ggml_backend_mi355x_supports_op.argtypes = [C.c_void_p, C.POINTER(CompatTensor)]
    lib.ggml_backend_mi355x_compute_graph.restype = C.c_bool
    lib.ggml_backend_mi355x_compute_graph.argtypes = [C.c_void_p, C.POINTER(C.POINTER(CompatTensor)), C.c_size_t]
    lib.ggml_backend_mi355x_set_op_mul_mat.restype = C.c_bool
    lib.ggml_backend_mi355x_set_op_mul_mat.argtypes = [C.c_int]
    lib.ggml_backend_mi355x_load_iq_grids_from_ggml.restype = C.c_int
    lib.ggml_backend_mi355x_set_kernel_variant.restype = C.c_bool
    lib.ggml_backend_mi355x_set_kernel_variant.argtypes = [C.c_void_p, C.c_int]
    lib.ggml_backend_mi355x_set_group_mode.restype = C.c_bool
    lib.ggml_backend_mi355x_set_group_mode.argtypes = [C.c_void_p, C.c_int]
    return lib

GROUPS_SERVER, GROUPS_LAUNCH = 0, 1
USAGE_ANY, USAGE_WEIGHTS, USAGE_COMPUTE = 0, 1, 2

_P = C.c_void_p
# (slot index, restype, argtypes) of every vtable entry the host calls
BUF = {
    "free_buffer": (0, None, [_P]),
    "get_base": (1, _P, [_P]),
    "init_tensor": (2, C.c_int, [_P, _P]),
    "memset_tensor": (3, None, [_P, _P, C.c_uint8, C.c_size_t, C.c_size_t]),
    "set_tensor": (4, None, [_P, _P, _P, C.c_size_t, C.c_size_t]),
    "get_tensor": (5, None, [_P, _P, _P, C.c_size_t, C.c_size_t]),
    "cpy_tensor": (8, C.c_bool, [_P, _P, _P]),
    "clear": (9, None, [_P, C.c_uint8]),
}
BUF_SLOTS = 14
BUFT = {
    "get_name": (0, C.c_char_p, [_P]),
    "alloc_buffer": (1, _P, [_P, C.c_size_t]),
    "get_alignment": (3, C.c_size_t, [_P]),
    "get_max_size": (4, C.c_size_t, [_P]),
    "get_alloc_size": (5, C.c_size_t, [_P, _P]),
    "is_host": (7, C.c_bool, [_P]),
}
DEV = {
    "get_name": (0, C.c_char_p, [_P]),
    "get_description": (1, C.c_char_p, [_P]),
    "get_memory": (2, None, [_P, C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]),
    "get_type": (3, C.c_int, [_P]),
    "get_props": (4, None, [_P, C.POINTER(DevProps)]),
    "init_backend": (5, _P, [_P, C.c_char_p]),
    "get_buffer_type": (6, _P, [_P]),
    "get_host_buffer_type": (7, _P, [_P]),
    "supports_op": (9, C.c_bool, [_P, _P]),
    "supports_buft": (10, C.c_bool, [_P, _P]),
    "offload_op": (11, C.c_bool, [_P, _P]),
}
REG = {
    "get_name": (0, C.c_char_p, [_P]),
    "get_device_count": (1, C.c_size_t, [_P]),
    "get_device": (2, _P, [_P, C.c_size_t]),
    "get_proc_address": (3, _P, [_P, C.c_char_p]),
}
BACKEND = {
    "get_name": (0, C.c_char_p, [_P]),
    "free": (1, None, [_P]),
    "set_tensor_async": (2, None, [_P, _P, _P, C.c_size_t, C.c_size_t]),
    "get_tensor_async": (3, None, [_P, _P, _P, C.c_size_t, C.c_size_t]),
    "synchronize": (7, None, [_P]),
    "graph_compute": (12, C.c_int, [_P, _P]),
}


def _addr(p):
    return p if isinstance(p, int) else C.addressof(p) if isinstance(p, C.Structure) else p.value


def vcall(table, iface_addr, name, *args):
    """Call slot `name` of the function-pointer table at iface_addr."""
    slot, res, argt = table[name]
    fp = C.c_void_p.from_address(iface_addr + slot * C.sizeof(C.c_void_p)).value
    if not fp:
        raise NotImplementedError(f"vtable slot {name} is empty")
    return C.CFUNCTYPE(res, *argt)(fp)(*args)


def slot_filled(iface_addr, slot):
    return bool(C.c_void_p.from_address(iface_addr + slot * C.sizeof(C.c_void_p)).value)


class Reg:
    """ggml_backend_reg: {int api_version; iface(4); context}."""

    def __init__(self, addr):
        self.addr = addr
        self.api_version = C.c_int.from_address(addr).value
        self.iface = addr + 8

    def call(self, name, *args):
        return vcall(REG, self.iface, name, self.addr, *args)

    def device(self, i):
        d = self.call("get_device", i)
        return Device(d) if d else None


class Device:
    """ggml_backend_device: {iface(15); reg; context}."""

    def __init__(self, addr):
        self.addr = addr
        self.iface = addr

    def call(self, name, *args):
        return vcall(DEV, self.iface, name, self.addr, *args)

    def buffer_type(self):
        return BufferType(self.call("get_buffer_type"))

    def host_buffer_type(self):
        return BufferType(self.call("get_host_buffer_type"))

    def props(self):
        p = DevProps()
        self.call("get_props", C.byref(p))
        return p

    def supports_op(self, t):
        return bool(self.call("supports_op", C.addressof(t)))

    def backend(self):
        b = self.call("init_backend", None)
        return Backend(b) if b else None


class BufferType:
    """ggml_backend_buffer_type: {iface(8); device; context}."""

    def __init__(self, addr):
        self.addr = addr
        self.iface = addr

    def call(self, name, *args):
        return vcall(BUFT, self.iface, name, self.addr, *args)

    def name(self):
        return self.call("get_name").decode()

    def alloc(self, size):
        b = self.call("alloc_buffer", size)
        if not b:
            raise MemoryError("alloc_buffer returned NULL")
        return Buffer(b)


class Buffer:
    """ggml_backend_buffer: {iface(14); buft; context; size; usage}.

    Tensors are placed in the buffer by a bump allocator honouring the buffer
    type's alignment, as ggml-alloc does."""

    def __init__(self, addr):
        self.addr = addr
        self.iface = addr
        off = BUF_SLOTS * C.sizeof(C.c_void_p)
        self.buft = C.c_void_p.from_address(addr + off).value
        self.size = C.c_size_t.from_address(addr + off + 16).value
        self.base = self.call("get_base")
        self.align = BufferType(self.buft).call("get_alignment")
        self.next = 0
        self.keep = []

    def call(self, name, *args):
        return vcall(BUF, self.iface, name, self.addr, *args)

    def place(self, t, nbytes):
        """Give tensor `t` the next aligned `nbytes` of this buffer."""
        off = (self.next + self.align - 1) // self.align * self.align
        if off + nbytes > self.size:
            raise MemoryError("buffer full")
        self.next = off + nbytes
        t.buffer = self.addr
        t.data = self.base + off
        self.call("init_tensor", C.addressof(t))
        self.keep.append(t)
        return t

    def set(self, t, arr, offset=0):
        arr = memoryview(arr).cast("B")
        src = (C.c_uint8 * len(arr)).from_buffer_copy(arr)
        self.call("set_tensor", C.addressof(t), C.addressof(src), offset, len(arr))

    def get(self, t, nbytes, offset=0):
        dst = (C.c_uint8 * nbytes)()
        self.call("get_tensor", C.addressof(t), C.addressof(dst), offset, nbytes)
        return bytes(dst)

    def set_usage(self, usage):
        """ggml_backend_buffer_set_usage: the field after size."""
        C.c_int.from_address(self.addr + BUF_SLOTS * C.sizeof(C.c_void_p) + 24).value = usage

    def free(self):
        if self.addr:
            self.call("free_buffer")
            self.addr = None


class Backend:
    """ggml_backend: {guid; iface(16); device; context}."""

    def __init__(self, addr):
        self.addr = addr
        self.iface = addr + 8

    def call(self, name, *args):
        return vcall(BACKEND, self.iface, name, self.addr, *args)

    def compute(self, nodes):
        arr = (C.POINTER(Tensor) * len(nodes))(*[C.pointer(n) for n in nodes])
        g = CGraph(size=len(nodes), n_nodes=len(nodes), n_leafs=0, nodes=arr)
        return self.call("graph_compute", C.addressof(g))

    def free(self):
        if self.addr:
            self.call("free")
            self.addr = None


def tensor(type_, ne, nb=None, name=b""):
    """A ggml_tensor with contiguous strides for `type_` (nb[0] = element or
    block bytes as ggml sets it)."""
    t = Tensor()
    t.type = type_
    ne = list(ne) + [1] * (4 - len(ne))
    for i, v in enumerate(ne):
        t.ne[i] = v
    if nb is not None:
        for i, v in enumerate(nb):
            t.nb[i] = v
    t.name = name
    return t


def contiguous_nb(elem_bytes, block, ne):
    nb = [elem_bytes, elem_bytes * (ne[0] // block)]
    nb.append(nb[1] * ne[1])
    nb.append(nb[2] * (ne[2] if len(ne) > 2 else 1))
    return nb


def mul_mat(w, x, out_ne, op=HOST_OP_MUL_MAT, name=b"mm"):
    """dst = MUL_MAT(w, x): dst->ne = {N, M, ...}, F32."""
    d = tensor(TYPE_F32, out_ne, contiguous_nb(4, 1, list(out_ne) + [1] * (4 - len(out_ne))), name)
    d.op = op
    d.src[0] = C.addressof(w)
    d.src[1] = C.addressof(x)
    d._keep = (w, x)
    return d
