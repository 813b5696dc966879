"""ctypes mirror of the scrapgpu_ C API exported by libscrapgpu_hip.so (include/scrapgpu/*.h).

This is host plumbing for the tests and the benchmark: every computation happens in the C++/HIP
library. Loading fails loudly when the library has not been built (``python -m
scrapgpulibrary_amd.build``); there is no fallback.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("SCRAPGPU_HIP_LIB") or os.path.join(PKG, "libscrapgpu_hip.so")

# status (include/scrapgpu/status.h)
OK, UNSUPPORTED, INVALID_ARGUMENT, OUT_OF_MEMORY, BACKEND_ERROR, DEVICE_LOST = range(6)
STATUS_NAMES = ["OK", "UNSUPPORTED", "INVALID_ARGUMENT", "OUT_OF_MEMORY", "BACKEND_ERROR", "DEVICE_LOST"]
# dtypes / layouts (include/scrapgpu/tensor.h)
F32, F16, I32, I64, I16, BF16 = 0, 1, 2, 3, 4, 5
Q4_0, Q8_0, Q4_K, Q6_K = 16, 17, 32, 33
QTYPES = (Q4_0, Q8_0, Q4_K, Q6_K)
NATURAL, R32 = 0, 1
BLOCK = {F32: 1, F16: 1, BF16: 1, I32: 1, Q4_0: 32, Q8_0: 32, Q4_K: 256, Q6_K: 256}
TYPE_SIZE = {F32: 4, F16: 2, BF16: 2, I32: 4, Q4_0: 18, Q8_0: 34, Q4_K: 144, Q6_K: 210}
NAMES = {Q4_0: "q4_0", Q8_0: "q8_0", Q4_K: "q4_k", Q6_K: "q6_k", F32: "f32"}
# ops (include/scrapgpu/op.h)
OP_ADD, OP_GET_ROWS, OP_MUL_MAT, OP_MUL_MAT_ID, OP_MUL_MAT_MULTI = 10, 23, 28, 29, 103


class TensorDesc(C.Structure):
    _fields_ = [("struct_size", C.c_size_t), ("dtype", C.c_int), ("ne", C.c_int64 * 4), ("nb", C.c_uint64 * 4),
                ("buffer", C.c_void_p), ("offset", C.c_uint64), ("layout", C.c_int)]


class OpDesc(C.Structure):
    _fields_ = [("struct_size", C.c_size_t), ("op", C.c_int), ("inputs", C.POINTER(TensorDesc)), ("input_count", C.c_size_t),
                ("outputs", C.POINTER(TensorDesc)), ("output_count", C.c_size_t), ("params", C.c_void_p),
                ("params_size", C.c_size_t)]


class GetRowsParams(C.Structure):
    _fields_ = [("struct_size", C.c_size_t), ("indices_are_i64", C.c_int)]


class MulMatIdParams(C.Structure):
    _fields_ = [("struct_size", C.c_size_t), ("n_used", C.c_uint32), ("max_prompt_tokens", C.c_uint32)]


class MulMatParams(C.Structure):
    _fields_ = [("struct_size", C.c_size_t), ("allow_broadcast", C.c_int)]


class DeviceInfo(C.Structure):
    _fields_ = [("struct_size", C.c_size_t), ("name", C.c_char_p), ("vendor", C.c_char_p), ("platform_name", C.c_char_p),
                ("driver_version", C.c_char_p), ("backend_name", C.c_char_p), ("reported_api_version", C.c_char_p),
                ("used_api_version", C.c_char_p), ("generation", C.c_int), ("generation_reason", C.c_char_p),
                ("total_memory_bytes", C.c_uint64), ("max_allocation_reported_bytes", C.c_uint64),
                ("max_allocation_used_bytes", C.c_uint64), ("max_work_group_size", C.c_uint64),
                ("local_memory_bytes", C.c_uint64), ("compute_units", C.c_uint32), ("warp_or_wave_width", C.c_uint32),
                ("quirks", C.c_uint64), ("probed_quirks", C.c_uint64), ("tuning_profile_name", C.c_char_p),
                ("tuning_overrides", C.c_char_p)]


class PlanNode(C.Structure):
    _fields_ = [("struct_size", C.c_size_t), ("op", OpDesc), ("output_use_count", C.c_uint32)]


class PlanDesc(C.Structure):
    _fields_ = [("struct_size", C.c_size_t), ("nodes", C.POINTER(PlanNode)), ("node_count", C.c_size_t)]


_lib = None

_SIGS = {
    "scrapgpu_get_abi_version": (C.c_uint32, []),
    "scrapgpu_status_string": (C.c_char_p, [C.c_int]),
    "scrapgpu_last_error": (C.c_char_p, []),
    "scrapgpu_clear_last_error": (None, []),
    "scrapgpu_set_last_error": (None, [C.c_char_p]),
    "scrapgpu_device_info_init": (C.c_int, [C.c_void_p, C.c_size_t]),
    "scrapgpu_get_device_count": (C.c_size_t, []),
    "scrapgpu_get_device": (C.c_int, [C.c_size_t, C.POINTER(C.c_void_p)]),
    "scrapgpu_device_get_info": (C.c_int, [C.c_void_p, C.c_void_p]),
    "scrapgpu_buffer_alloc": (C.c_int, [C.c_void_p, C.c_size_t, C.POINTER(C.c_void_p)]),
    "scrapgpu_buffer_free": (C.c_int, [C.c_void_p]),
    "scrapgpu_buffer_write": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p, C.c_size_t, C.c_int]),
    "scrapgpu_buffer_read": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p, C.c_size_t, C.c_int]),
    "scrapgpu_buffer_copy": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p, C.c_uint64, C.c_size_t, C.c_int]),
    "scrapgpu_buffer_fill": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64, C.c_size_t, C.c_uint8, C.c_int]),
    "scrapgpu_stream_create": (C.c_int, [C.c_void_p, C.POINTER(C.c_void_p)]),
    "scrapgpu_stream_free": (C.c_int, [C.c_void_p]),
    "scrapgpu_stream_sync": (C.c_int, [C.c_void_p]),
    "scrapgpu_dtype_block_size": (C.c_size_t, [C.c_int]),
    "scrapgpu_dtype_type_size": (C.c_size_t, [C.c_int]),
    "scrapgpu_tensor_row_size": (C.c_size_t, [C.c_int, C.c_int64]),
    "scrapgpu_tensor_is_contiguous": (C.c_int, [C.POINTER(TensorDesc)]),
    "scrapgpu_tensor_r32_eligible": (C.c_int, [C.POINTER(TensorDesc)]),
    "scrapgpu_tensor_upload": (C.c_int, [C.c_void_p, C.POINTER(TensorDesc), C.c_void_p, C.c_size_t]),
    "scrapgpu_tensor_download": (C.c_int, [C.c_void_p, C.POINTER(TensorDesc), C.c_void_p, C.c_size_t]),
    "scrapgpu_op_desc_validate": (C.c_int, [C.POINTER(OpDesc)]),
    "scrapgpu_op_supported": (C.c_int, [C.c_void_p, C.POINTER(OpDesc), C.POINTER(C.c_char_p)]),
    "scrapgpu_op_execute": (C.c_int, [C.c_void_p, C.POINTER(OpDesc)]),
    "scrapgpu_register_backend": (C.c_int, [C.c_void_p]),
    "scrapgpu_unregister_all_backends": (None, []),
    "scrapgpu_plan_build": (C.c_int, [C.c_void_p, C.POINTER(PlanDesc), C.POINTER(C.c_void_p)]),
    "scrapgpu_plan_execute": (C.c_int, [C.c_void_p, C.c_void_p]),
    "scrapgpu_plan_free": (C.c_int, [C.c_void_p]),
    "scrapgpu_hip_register": (C.c_int, []),
    "scrapgpu_hip_quantize": (C.c_int, [C.c_void_p, C.POINTER(TensorDesc), C.POINTER(TensorDesc)]),
    "scrapgpu_hip_dequantize": (C.c_int, [C.c_void_p, C.POINTER(TensorDesc), C.POINTER(TensorDesc)]),
    "scrapgpu_hip_fill_normal": (C.c_int, [C.c_void_p, C.POINTER(TensorDesc), C.c_uint64, C.c_float, C.c_float]),
    "scrapgpu_hip_profile_enable": (C.c_int, [C.c_int]),
    "scrapgpu_hip_profile_reset": (C.c_int, []),
    "scrapgpu_hip_profile_read": (C.c_int, [C.c_size_t, C.POINTER(C.c_char_p), C.POINTER(C.c_uint64), C.POINTER(C.c_double),
                                            C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    "scrapgpu_hip_stream_native": (C.c_void_p, [C.c_void_p]),
    "scrapgpu_hip_op_execute_static": (C.c_int, [C.c_void_p, C.POINTER(OpDesc)]),
    "scrapgpu_hip_last_launch": (C.c_int, [C.c_char_p, C.c_size_t, C.POINTER(C.c_uint64)]),
}


def lib():
    """The loaded library; raises if it was not built (no fallback path exists)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m scrapgpulibrary_amd.build`")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


class ScrapError(RuntimeError):
    def __init__(self, status: int, what: str):
        self.status = status
        msg = lib().scrapgpu_last_error().decode(errors="replace")
        super().__init__(f"{what}: {STATUS_NAMES[status] if 0 <= status < 6 else status}: {msg}")


def check(status: int, what: str = "scrapgpu call") -> None:
    if status != OK:
        raise ScrapError(status, what)


def row_bytes(dtype: int, ne0: int) -> int:
    return (ne0 + BLOCK[dtype] - 1) // BLOCK[dtype] * TYPE_SIZE[dtype]


def tdesc(dtype: int, ne, buffer=None, offset: int = 0, layout: int = NATURAL, nb=None) -> TensorDesc:
    """A contiguous tensor descriptor (ggml order: ne[0] innermost)."""
    ne = list(ne) + [1] * (4 - len(ne))
    t = TensorDesc()
    t.struct_size = C.sizeof(TensorDesc)
    t.dtype = dtype
    for i in range(4):
        t.ne[i] = ne[i]
    if nb is None:
        nb = [TYPE_SIZE[dtype], row_bytes(dtype, max(ne[0], 1))]
        nb.append(nb[1] * max(ne[1], 1))
        nb.append(nb[2] * max(ne[2], 1))
    for i in range(4):
        t.nb[i] = nb[i]
    t.buffer = buffer.handle if isinstance(buffer, Buffer) else buffer
    t.offset = offset
    t.layout = layout
    return t


def nbytes(t: TensorDesc) -> int:
    bs = BLOCK[t.dtype]
    if bs == 1:
        n = TYPE_SIZE[t.dtype]
        return n + sum((max(t.ne[i], 1) - 1) * t.nb[i] for i in range(4))
    n = t.ne[0] * t.nb[0] // bs
    return n + sum((max(t.ne[i], 1) - 1) * t.nb[i] for i in range(1, 4))


def mul_mat_op(w: TensorDesc, x: TensorDesc, y: TensorDesc, allow_broadcast: int = 0):
    """(OpDesc, keep-alive tuple) for MUL_MAT y = W x."""
    ins = (TensorDesc * 2)(w, x)
    outs = (TensorDesc * 1)(y)
    p = MulMatParams(C.sizeof(MulMatParams), allow_broadcast)
    op = OpDesc(C.sizeof(OpDesc), OP_MUL_MAT, ins, 2, outs, 1, C.cast(C.pointer(p), C.c_void_p), C.sizeof(p))
    return op, (ins, outs, p)


def mul_mat_id_op(w: TensorDesc, x: TensorDesc, ids: TensorDesc, y: TensorDesc, n_used: int):
    """(OpDesc, keep-alive tuple) for MUL_MAT_ID y[:, i, t] = W[:, :, ids[i, t]] x[:, i or 0, t]."""
    ins = (TensorDesc * 3)(w, x, ids)
    outs = (TensorDesc * 1)(y)
    p = MulMatIdParams(C.sizeof(MulMatIdParams), n_used, 0)
    op = OpDesc(C.sizeof(OpDesc), OP_MUL_MAT_ID, ins, 3, outs, 1, C.cast(C.pointer(p), C.c_void_p), C.sizeof(p))
    return op, (ins, outs, p)


def get_rows_op(w: TensorDesc, ids: TensorDesc, y: TensorDesc):
    """(OpDesc, keep-alive tuple) for GET_ROWS y[:, a, b, c] = row ids[a, b, c] of slice (b, c) of W."""
    ins = (TensorDesc * 2)(w, ids)
    outs = (TensorDesc * 1)(y)
    p = GetRowsParams(C.sizeof(GetRowsParams), 0)
    op = OpDesc(C.sizeof(OpDesc), OP_GET_ROWS, ins, 2, outs, 1, C.cast(C.pointer(p), C.c_void_p), C.sizeof(p))
    return op, (ins, outs, p)


def multi_op(ws, x: TensorDesc, ys):
    n = len(ws)
    ins = (TensorDesc * (n + 1))(*ws, x)
    outs = (TensorDesc * n)(*ys)
    op = OpDesc(C.sizeof(OpDesc), OP_MUL_MAT_MULTI, ins, n + 1, outs, n, None, 0)
    return op, (ins, outs)


class Buffer:
    def __init__(self, device: "Device", size: int):
        self.device = device
        h = C.c_void_p()
        check(lib().scrapgpu_buffer_alloc(device.handle, size, C.byref(h)), f"buffer_alloc({size})")
        self.handle = h.value
        self.size = size

    def free(self):
        if self.handle:
            check(lib().scrapgpu_buffer_free(self.handle), "buffer_free")
            self.handle = None


class Stream:
    def __init__(self, device: "Device"):
        h = C.c_void_p()
        check(lib().scrapgpu_stream_create(device.handle, C.byref(h)), "stream_create")
        self.handle = h.value
        self.device = device

    def sync(self):
        check(lib().scrapgpu_stream_sync(self.handle), "stream_sync")

    def free(self):
        if self.handle:
            check(lib().scrapgpu_stream_free(self.handle), "stream_free")
            self.handle = None

    # ---- transfers of numpy arrays
    def upload(self, t: TensorDesc, arr: np.ndarray, size: int | None = None):
        a = np.ascontiguousarray(arr)
        n = a.nbytes if size is None else size
        check(lib().scrapgpu_tensor_upload(self.handle, C.byref(t), a.ctypes.data, n), "tensor_upload")

    def download(self, t: TensorDesc, dtype=np.float32, count: int | None = None) -> np.ndarray:
        n = nbytes(t)
        out = np.empty(n, np.uint8)
        check(lib().scrapgpu_tensor_download(self.handle, C.byref(t), out.ctypes.data, n), "tensor_download")
        out = out.view(dtype)
        return out if count is None else out[:count]

    def write(self, buf: Buffer, offset: int, arr: np.ndarray):
        a = np.ascontiguousarray(arr)
        check(lib().scrapgpu_buffer_write(self.handle, buf.handle, offset, a.ctypes.data, a.nbytes, 1), "buffer_write")

    def read(self, buf: Buffer, offset: int, size: int) -> np.ndarray:
        out = np.empty(size, np.uint8)
        check(lib().scrapgpu_buffer_read(self.handle, buf.handle, offset, out.ctypes.data, size, 1), "buffer_read")
        return out

    def execute(self, op: OpDesc):
        check(lib().scrapgpu_op_execute(self.handle, C.byref(op)), "op_execute")

    def quantize(self, src: TensorDesc, dst: TensorDesc):
        check(lib().scrapgpu_hip_quantize(self.handle, C.byref(src), C.byref(dst)), "hip_quantize")

    def dequantize(self, src: TensorDesc, dst: TensorDesc):
        check(lib().scrapgpu_hip_dequantize(self.handle, C.byref(src), C.byref(dst)), "hip_dequantize")

    def fill_normal(self, t: TensorDesc, seed: int, mean: float = 0.0, std: float = 1.0):
        check(lib().scrapgpu_hip_fill_normal(self.handle, C.byref(t), seed, mean, std), "hip_fill_normal")


class Device:
    def __init__(self, index: int = 0):
        check(lib().scrapgpu_hip_register(), "hip_register")
        if index >= lib().scrapgpu_get_device_count():
            raise RuntimeError("no gfx950 device registered by the hip backend")
        h = C.c_void_p()
        check(lib().scrapgpu_get_device(index, C.byref(h)), "get_device")
        self.handle = h.value

    def info(self) -> DeviceInfo:
        info = DeviceInfo()
        check(lib().scrapgpu_device_info_init(C.byref(info), C.sizeof(info)))
        check(lib().scrapgpu_device_get_info(self.handle, C.byref(info)), "device_get_info")
        return info

    def alloc(self, size: int) -> Buffer:
        return Buffer(self, size)

    def stream(self) -> Stream:
        return Stream(self)

    def supported(self, op: OpDesc):
        r = C.c_char_p()
        st = lib().scrapgpu_op_supported(self.handle, C.byref(op), C.byref(r))
        return st, (r.value.decode() if r.value else "")


def last_launch() -> tuple[str, int]:
    """(form, work-groups) of this thread's last matvec / matmul launch (scrapgpu_hip_last_launch)."""
    buf = C.create_string_buffer(96)
    grid = C.c_uint64()
    check(lib().scrapgpu_hip_last_launch(buf, 96, C.byref(grid)), "hip_last_launch")
    return buf.value.decode(), grid.value


def profile_table() -> list[dict]:
    """Per-kernel rows of the library's event profiler (scrapgpu_hip_profile_read)."""
    rows = []
    i = 0
    name, n, ms, by, fl = C.c_char_p(), C.c_uint64(), C.c_double(), C.c_double(), C.c_double()
    while lib().scrapgpu_hip_profile_read(i, C.byref(name), C.byref(n), C.byref(ms), C.byref(by), C.byref(fl)) == OK:
        rows.append({"name": name.value.decode(), "launches": n.value, "ms": ms.value, "bytes": by.value, "flops": fl.value})
        i += 1
    return rows
