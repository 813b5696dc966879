"""CPU oracle of the quantized MUL_MAT path -- TEST INFRASTRUCTURE ONLY.

ctypes bindings over ``oracle/liboracle.so`` (the C restatement in ``oracle/oracle.c`` of the
reference's ``src/core/ref``) and, when it was built in this container, ``oracle/_ref/
libscrapgpu_ref.so`` (the reference's own CPU implementation compiled from its sources).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` import
this package. The product library never loads it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libscrapgpu_ref.so")

F32, F16, I32, BF16, Q4_0, Q8_0, Q4_K, Q6_K = 0, 1, 2, 5, 16, 17, 32, 33
QTYPES = (Q4_0, Q8_0, Q4_K, Q6_K)
FTYPES = (F32, F16, BF16)
NAMES = {F32: "f32", F16: "f16", BF16: "bf16", Q4_0: "q4_0", Q8_0: "q8_0", Q4_K: "q4_k", Q6_K: "q6_k"}
BLOCK = {F32: 1, F16: 1, BF16: 1, Q4_0: 32, Q8_0: 32, Q4_K: 256, Q6_K: 256}
TYPE_SIZE = {F32: 4, F16: 2, BF16: 2, Q4_0: 18, Q8_0: 34, Q4_K: 144, Q6_K: 210}


def build(ref: bool = False) -> None:
    """Compiles liboracle.so (and _ref when asked and the reference sources exist)."""
    subprocess.run(["make", "-s", "-C", HERE, "liboracle.so"], check=True)
    if ref and os.path.isdir("/root/reference/src"):
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


class SgoTensor(C.Structure):
    _fields_ = [("dtype", C.c_int32), ("ne", C.c_int64 * 4), ("nb", C.c_uint64 * 4), ("data", C.c_void_p)]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        L.sgo_half_to_float.restype = C.c_float
        L.sgo_half_to_float.argtypes = [C.c_uint16]
        L.sgo_float_to_half.restype = C.c_uint16
        L.sgo_float_to_half.argtypes = [C.c_float]
        L.sgo_half_to_float_n.argtypes = [C.c_void_p, C.c_void_p, C.c_int64]
        L.sgo_float_to_half_n.argtypes = [C.c_void_p, C.c_void_p, C.c_int64]
        L.sgo_dequantize.argtypes = [C.c_int32, C.c_void_p, C.c_void_p, C.c_int64]
        L.sgo_quantize.argtypes = [C.c_int32, C.c_void_p, C.c_void_p, C.c_int64]
        L.sgo_mul_mat.argtypes = [C.POINTER(SgoTensor)] * 3 + [C.c_int]
        L.sgo_mul_mat_mt.argtypes = [C.POINTER(SgoTensor)] * 3 + [C.c_int, C.c_int]
        L.sgo_mul_mat_id.argtypes = [C.POINTER(SgoTensor)] * 4
        L.sgo_get_rows.argtypes = [C.POINTER(SgoTensor)] * 3
        for f in (L.sgo_r32_pack, L.sgo_r32_unpack):
            f.argtypes = [C.c_int32, C.c_int64, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p]
        _lib = L
    return _lib


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


def row_bytes(dtype: int, K: int) -> int:
    return K // BLOCK[dtype] * TYPE_SIZE[dtype]


def float_to_bf16(x: np.ndarray) -> np.ndarray:
    """bf16 bit patterns of float32 x, rounded to nearest even (NaNs kept quiet), as the
    reference's st_bf16 (src/core/ref/ops.cpp:43-52)."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (b & 0x7FFFFFFF) > 0x7F800000
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) & 0xFFFF
    return np.where(nan, (b >> 16) | 0x40, r).astype(np.uint16)


def bf16_to_float(h: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def half_to_float(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().sgo_half_to_float_n(_p(h), _p(out), h.size)
    return out


def float_to_half(f: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().sgo_float_to_half_n(_p(f), _p(out), f.size)
    return out


def quantize(dtype: int, x: np.ndarray, threads: int = 1) -> np.ndarray:
    """Natural-layout blocks of the float array x (its size a multiple of the block size). Blocks
    are quantized independently, so `threads` > 1 splits x into runs of whole blocks quantized in
    parallel (ctypes releases the GIL); the bytes are the same."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    bs, ts = BLOCK[dtype], TYPE_SIZE[dtype]
    out = np.zeros(x.size // bs * ts, np.uint8)
    nblk = x.size // bs
    if threads <= 1 or nblk < 4096:
        st = lib().sgo_quantize(dtype, _p(x), _p(out), x.size)
        if st != 0:
            raise ValueError(f"sgo_quantize status {st}")
        return out
    import concurrent.futures as cf

    cuts = [nblk * i // threads for i in range(threads + 1)]

    def run(i):
        b0, b1 = cuts[i], cuts[i + 1]
        xs, qs = x[b0 * bs:b1 * bs], out[b0 * ts:b1 * ts]
        return lib().sgo_quantize(dtype, _p(xs), _p(qs), xs.size) if b1 > b0 else 0

    with cf.ThreadPoolExecutor(threads) as ex:
        sts = list(ex.map(run, range(threads)))
    if any(sts):
        raise ValueError(f"sgo_quantize status {max(sts)}")
    return out


def dequantize(dtype: int, q: np.ndarray, n: int) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    out = np.empty(n, np.float32)
    st = lib().sgo_dequantize(dtype, _p(q), _p(out), n)
    if st != 0:
        raise ValueError(f"sgo_dequantize status {st}")
    return out


def _tensor(dtype: int, arr: np.ndarray, ne, nb) -> SgoTensor:
    t = SgoTensor()
    t.dtype = dtype
    for i in range(4):
        t.ne[i] = ne[i]
        t.nb[i] = nb[i]
    t.data = _p(arr)
    return t


def mul_mat(dtype: int, w: np.ndarray, K: int, M: int, x: np.ndarray, threads: int = 1) -> np.ndarray:
    """y[n, m] = sum_k W[m, k] x[n, k] for one contiguous slice: w holds M rows of natural blocks
    (float rows: float32 [M, K] for F32, the uint16 bit patterns [M, K] for F16 and BF16), x is
    float32 [N, K]. Returns float32 [N, M]."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, K)
    N = x.shape[0]
    rb = row_bytes(dtype, K)
    w = np.ascontiguousarray(w).view(np.uint8).reshape(-1)
    assert w.size == rb * M, (w.size, rb, M)
    y = np.zeros((N, M), np.float32)
    tw = _tensor(dtype, w, (K, M, 1, 1), (TYPE_SIZE[dtype], rb, rb * M, rb * M))
    tx = _tensor(F32, x, (K, N, 1, 1), (4, 4 * K, 4 * K * N, 4 * K * N))
    ty = _tensor(F32, y, (M, N, 1, 1), (4, 4 * M, 4 * M * N, 4 * M * N))
    st = lib().sgo_mul_mat_mt(C.byref(tw), C.byref(tx), C.byref(ty), 0, threads)
    if st != 0:
        raise ValueError(f"sgo_mul_mat status {st}")
    return y


def mul_mat_id(dtype: int, w: np.ndarray, K: int, M: int, E: int, x: np.ndarray, ids: np.ndarray) -> np.ndarray:
    """MUL_MAT_ID on contiguous tensors: w holds E experts of M rows of natural blocks, x is float32
    [T, n1, K] (n1 = 1 or n_used), ids int32 [T, n_used]. Returns float32 [T, n_used, M]; raises
    ValueError on a status other than OK (an expert index out of range)."""
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    T, nu = ids.shape
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(T, -1, K)
    n1 = x.shape[1]
    rb = row_bytes(dtype, K)
    w = np.ascontiguousarray(w).view(np.uint8).reshape(-1)
    assert w.size == rb * M * E
    y = np.zeros((T, nu, M), np.float32)
    tw = _tensor(dtype, w, (K, M, E, 1), (TYPE_SIZE[dtype], rb, rb * M, rb * M * E))
    tx = _tensor(F32, x, (K, n1, T, 1), (4, 4 * K, 4 * K * n1, 4 * K * n1 * T))
    ti = _tensor(I32, ids, (nu, T, 1, 1), (4, 4 * nu, 4 * nu * T, 4 * nu * T))
    ty = _tensor(F32, y, (M, nu, T, 1), (4, 4 * M, 4 * M * nu, 4 * M * nu * T))
    st = lib().sgo_mul_mat_id(C.byref(tw), C.byref(tx), C.byref(ti), C.byref(ty))
    if st != 0:
        raise ValueError(f"sgo_mul_mat_id status {st}")
    return y


def get_rows(dtype: int, w: np.ndarray, K: int, R: int, ids: np.ndarray) -> np.ndarray:
    """GET_ROWS of one slice: w holds R rows of natural blocks, ids int32 [n]. Returns float32 [n, K]."""
    ids = np.ascontiguousarray(ids, dtype=np.int32).reshape(-1)
    n = ids.size
    rb = row_bytes(dtype, K)
    w = np.ascontiguousarray(w).view(np.uint8).reshape(-1)
    y = np.zeros((n, K), np.float32)
    tw = _tensor(dtype, w, (K, R, 1, 1), (TYPE_SIZE[dtype], rb, rb * R, rb * R))
    ti = _tensor(I32, ids, (n, 1, 1, 1), (4, 4 * n, 4 * n, 4 * n))
    ty = _tensor(F32, y, (K, n, 1, 1), (4, 4 * K, 4 * K * n, 4 * K * n))
    st = lib().sgo_get_rows(C.byref(tw), C.byref(ti), C.byref(ty))
    if st != 0:
        raise ValueError(f"sgo_get_rows status {st}")
    return y


def mul_mat_strided(w: SgoTensor, x: SgoTensor, y: SgoTensor, allow_broadcast: int = 1) -> int:
    """Raw call on caller-built descriptors (arbitrary strides / slices / broadcast)."""
    return lib().sgo_mul_mat(C.byref(w), C.byref(x), C.byref(y), allow_broadcast)


def tensor(dtype: int, arr: np.ndarray, ne, nb) -> SgoTensor:
    return _tensor(dtype, arr, ne, nb)


def r32_pack(dtype: int, K: int, M: int, slices: int, nat: np.ndarray) -> np.ndarray:
    nat = np.ascontiguousarray(nat, dtype=np.uint8)
    rep = np.zeros_like(nat)
    st = lib().sgo_r32_pack(dtype, K, M, slices, _p(nat), _p(rep))
    if st != 0:
        raise ValueError(f"sgo_r32_pack status {st}")
    return rep


def r32_unpack(dtype: int, K: int, M: int, slices: int, rep: np.ndarray) -> np.ndarray:
    rep = np.ascontiguousarray(rep, dtype=np.uint8)
    nat = np.zeros_like(rep)
    st = lib().sgo_r32_unpack(dtype, K, M, slices, _p(rep), _p(nat))
    if st != 0:
        raise ValueError(f"sgo_r32_unpack status {st}")
    return nat


# ------------------------------------------------------------------------------------------------
# deterministic synthetic inputs: splitmix64 + Box-Muller in float64, rounded to float32
# ------------------------------------------------------------------------------------------------

def normal(n: int, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    """n samples of N(mean, std) as float32 (numpy only; the bytes are the input, the generator
    need not match anything else)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    return (rng.standard_normal(n) * std + mean).astype(np.float32)


# ------------------------------------------------------------------------------------------------
# the reference compiled from source (only in the build container)
# ------------------------------------------------------------------------------------------------

_ref = None


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def ref():
    global _ref
    if _ref is None:
        L = C.CDLL(REF_PATH)
        L.scrapgpu_ref_quantize.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_int64]
        L.scrapgpu_ref_dequantize.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_int64]
        L.scrapgpu_ref_execute.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p]
        L.ref_r32_move.argtypes = [C.c_int, C.c_int64, C.c_int64, C.c_int64, C.c_void_p, C.c_void_p, C.c_int]
        _ref = L
    return _ref


def ref_quantize(dtype: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.size // BLOCK[dtype] * TYPE_SIZE[dtype], np.uint8)
    assert ref().scrapgpu_ref_quantize(dtype, _p(x), _p(out), x.size) == 0
    return out


def ref_dequantize(dtype: int, q: np.ndarray, n: int) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    out = np.empty(n, np.float32)
    assert ref().scrapgpu_ref_dequantize(dtype, _p(q), _p(out), n) == 0
    return out


def ref_r32(dtype: int, K: int, M: int, slices: int, data: np.ndarray, pack: bool) -> np.ndarray:
    data = np.ascontiguousarray(data, dtype=np.uint8).copy()
    out = np.zeros_like(data)
    if pack:
        st = ref().ref_r32_move(dtype, K, M, slices, _p(data), _p(out), 1)
    else:
        st = ref().ref_r32_move(dtype, K, M, slices, _p(out), _p(data), 0)
    assert st == 0
    return out


class _RefTensorDesc(C.Structure):
    # scrapgpu_tensor_desc (reference include/scrapgpu/tensor.h:29-37)
    _fields_ = [("struct_size", C.c_size_t), ("dtype", C.c_int), ("ne", C.c_int64 * 4), ("nb", C.c_uint64 * 4),
                ("buffer", C.c_void_p), ("offset", C.c_uint64), ("layout", C.c_int)]


class _RefOpDesc(C.Structure):
    _fields_ = [("struct_size", C.c_size_t), ("op", C.c_int), ("inputs", C.c_void_p), ("input_count", C.c_size_t),
                ("outputs", C.c_void_p), ("output_count", C.c_size_t), ("params", C.c_void_p), ("params_size", C.c_size_t)]


class _RefMulMatParams(C.Structure):
    _fields_ = [("struct_size", C.c_size_t), ("allow_broadcast", C.c_int)]


def ref_mul_mat(dtype: int, w: np.ndarray, K: int, M: int, x: np.ndarray) -> np.ndarray:
    """scrapgpu_ref_execute(MUL_MAT) of the reference on one contiguous slice."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, K)
    N = x.shape[0]
    w = np.ascontiguousarray(w).view(np.uint8).reshape(-1)
    rb = row_bytes(dtype, K)
    y = np.zeros((N, M), np.float32)
    ins = (_RefTensorDesc * 2)()
    outs = (_RefTensorDesc * 1)()

    def fill(t, dt, ne, nb):
        t.struct_size = C.sizeof(_RefTensorDesc)
        t.dtype = dt
        for i in range(4):
            t.ne[i] = ne[i]
            t.nb[i] = nb[i]
        t.offset = 0
        t.layout = 0

    fill(ins[0], dtype, (K, M, 1, 1), (TYPE_SIZE[dtype], rb, rb * M, rb * M))
    fill(ins[1], F32, (K, N, 1, 1), (4, 4 * K, 4 * K * N, 4 * K * N))
    fill(outs[0], F32, (M, N, 1, 1), (4, 4 * M, 4 * M * N, 4 * M * N))
    p = _RefMulMatParams(C.sizeof(_RefMulMatParams), 0)
    op = _RefOpDesc(C.sizeof(_RefOpDesc), 28, C.addressof(ins), 2, C.addressof(outs), 1, C.addressof(p), C.sizeof(p))
    in_ptrs = (C.c_void_p * 2)(_p(w), _p(x))
    out_ptrs = (C.c_void_p * 1)(_p(y))
    st = ref().scrapgpu_ref_execute(C.byref(op), in_ptrs, out_ptrs)
    assert st == 0, st
    return y


class _RefMulMatIdParams(C.Structure):
    _fields_ = [("struct_size", C.c_size_t), ("n_used", C.c_uint32), ("max_prompt_tokens", C.c_uint32)]


class _RefGetRowsParams(C.Structure):
    _fields_ = [("struct_size", C.c_size_t), ("indices_are_i64", C.c_int)]


def _ref_fill(t, dt, ne, nb):
    t.struct_size = C.sizeof(_RefTensorDesc)
    t.dtype = dt
    for i in range(4):
        t.ne[i] = ne[i]
        t.nb[i] = nb[i]
    t.offset = 0
    t.layout = 0


def ref_mul_mat_id(dtype: int, w: np.ndarray, K: int, M: int, E: int, x: np.ndarray, ids: np.ndarray):
    """scrapgpu_ref_execute(MUL_MAT_ID) of the reference on contiguous tensors (shapes as
    mul_mat_id). Returns (status, y)."""
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    T, nu = ids.shape
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(T, -1, K)
    n1 = x.shape[1]
    rb = row_bytes(dtype, K)
    w = np.ascontiguousarray(w).view(np.uint8).reshape(-1)
    y = np.zeros((T, nu, M), np.float32)
    ins = (_RefTensorDesc * 3)()
    outs = (_RefTensorDesc * 1)()
    _ref_fill(ins[0], dtype, (K, M, E, 1), (TYPE_SIZE[dtype], rb, rb * M, rb * M * E))
    _ref_fill(ins[1], F32, (K, n1, T, 1), (4, 4 * K, 4 * K * n1, 4 * K * n1 * T))
    _ref_fill(ins[2], I32, (nu, T, 1, 1), (4, 4 * nu, 4 * nu * T, 4 * nu * T))
    _ref_fill(outs[0], F32, (M, nu, T, 1), (4, 4 * M, 4 * M * nu, 4 * M * nu * T))
    p = _RefMulMatIdParams(C.sizeof(_RefMulMatIdParams), nu, 0)
    op = _RefOpDesc(C.sizeof(_RefOpDesc), 29, C.addressof(ins), 3, C.addressof(outs), 1, C.addressof(p), C.sizeof(p))
    in_ptrs = (C.c_void_p * 3)(_p(w), _p(x), _p(ids))
    out_ptrs = (C.c_void_p * 1)(_p(y))
    st = ref().scrapgpu_ref_execute(C.byref(op), in_ptrs, out_ptrs)
    return st, y


def ref_get_rows(dtype: int, w: np.ndarray, K: int, R: int, ids: np.ndarray):
    """scrapgpu_ref_execute(GET_ROWS) of the reference on one slice. Returns (status, y [n, K])."""
    ids = np.ascontiguousarray(ids, dtype=np.int32).reshape(-1)
    n = ids.size
    rb = row_bytes(dtype, K)
    w = np.ascontiguousarray(w).view(np.uint8).reshape(-1)
    y = np.zeros((n, K), np.float32)
    ins = (_RefTensorDesc * 2)()
    outs = (_RefTensorDesc * 1)()
    _ref_fill(ins[0], dtype, (K, R, 1, 1), (TYPE_SIZE[dtype], rb, rb * R, rb * R))
    _ref_fill(ins[1], I32, (n, 1, 1, 1), (4, 4 * n, 4 * n, 4 * n))
    _ref_fill(outs[0], F32, (K, n, 1, 1), (4, 4 * K, 4 * K * n, 4 * K * n))
    p = _RefGetRowsParams(C.sizeof(_RefGetRowsParams), 0)
    op = _RefOpDesc(C.sizeof(_RefOpDesc), 23, C.addressof(ins), 2, C.addressof(outs), 1, C.addressof(p), C.sizeof(p))
    in_ptrs = (C.c_void_p * 2)(_p(w), _p(ids))
    out_ptrs = (C.c_void_p * 1)(_p(y))
    st = ref().scrapgpu_ref_execute(C.byref(op), in_ptrs, out_ptrs)
    return st, y
