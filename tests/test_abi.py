"""The C-ABI boundary on the CPU: exports, struct layouts, header hygiene, core rules, dispatch.

Mirrors the reference's contract tests (tests/core/core_contract_tests.cpp, public_headers_{c,cpp},
the fake-backend pattern of tests/core/compat_tests.cpp:13-31). No GPU is touched: on a machine
without a gfx950 device scrapgpu_hip_register() registers zero devices.
"""
import ctypes as C
import glob
import os
import re
import subprocess
import tempfile

import pytest

import scrapgpulibrary_amd as sg

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INC = os.path.join(ROOT, "include")
REF_INC = "/root/reference/include"


def declared_functions():
    names = set()
    for h in glob.glob(os.path.join(INC, "scrapgpu", "*.h")):
        text = open(h).read()
        names.update(re.findall(r"SCRAPGPU_API\s+[^;(]*?\b(scrapgpu_\w+)\s*\(", text))
    return sorted(names)


def test_library_exports_every_declared_function():
    out = subprocess.run(["nm", "-D", "--defined-only", sg.LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    names = declared_functions()
    assert len(names) > 40
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    lib = sg.lib()
    for n in names:
        getattr(lib, n)


PROBE = r"""
#include <stdio.h>
#include <stddef.h>
#include "scrapgpu/backend.h"
#define P(T) printf(#T " %zu\n", sizeof(T));
#define O(T, f) printf(#T "." #f " %zu\n", offsetof(T, f));
int main(void) {
    P(scrapgpu_tensor_desc) O(scrapgpu_tensor_desc, dtype) O(scrapgpu_tensor_desc, ne) O(scrapgpu_tensor_desc, nb)
    O(scrapgpu_tensor_desc, buffer) O(scrapgpu_tensor_desc, offset) O(scrapgpu_tensor_desc, layout)
    P(scrapgpu_op_desc) O(scrapgpu_op_desc, op) O(scrapgpu_op_desc, inputs) O(scrapgpu_op_desc, input_count)
    O(scrapgpu_op_desc, outputs) O(scrapgpu_op_desc, output_count) O(scrapgpu_op_desc, params) O(scrapgpu_op_desc, params_size)
    P(scrapgpu_mul_mat_params) O(scrapgpu_mul_mat_params, allow_broadcast)
    P(scrapgpu_mul_mat_id_params) O(scrapgpu_mul_mat_id_params, n_used) O(scrapgpu_mul_mat_id_params, max_prompt_tokens)
    P(scrapgpu_get_rows_params) O(scrapgpu_get_rows_params, indices_are_i64)
    P(scrapgpu_device_info) O(scrapgpu_device_info, generation) O(scrapgpu_device_info, total_memory_bytes)
    O(scrapgpu_device_info, compute_units) O(scrapgpu_device_info, warp_or_wave_width) O(scrapgpu_device_info, quirks)
    O(scrapgpu_device_info, tuning_overrides)
    P(scrapgpu_plan_node) O(scrapgpu_plan_node, op) O(scrapgpu_plan_node, output_use_count)
    P(scrapgpu_plan_desc) O(scrapgpu_plan_desc, nodes) O(scrapgpu_plan_desc, node_count)
    P(scrapgpu_backend_vtable) O(scrapgpu_backend_vtable, get_device_count) O(scrapgpu_backend_vtable, op_supported)
    O(scrapgpu_backend_vtable, plan_free) O(scrapgpu_backend_vtable, stream_create) O(scrapgpu_backend_vtable, op_execute)
    O(scrapgpu_backend_vtable, stream_device)
    printf("SCRAPGPU_OP_MUL_MAT %d\nSCRAPGPU_OP_MUL_MAT_MULTI %d\nSCRAPGPU_DTYPE_Q6_K %d\nSCRAPGPU_LAYOUT_R32 %d\n",
           (int) SCRAPGPU_OP_MUL_MAT, (int) SCRAPGPU_OP_MUL_MAT_MULTI, (int) SCRAPGPU_DTYPE_Q6_K, (int) SCRAPGPU_LAYOUT_R32);
    printf("SCRAPGPU_OP_MUL_MAT_ID %d\nSCRAPGPU_OP_GET_ROWS %d\nSCRAPGPU_DTYPE_I32 %d\n",
           (int) SCRAPGPU_OP_MUL_MAT_ID, (int) SCRAPGPU_OP_GET_ROWS, (int) SCRAPGPU_DTYPE_I32);
    printf("ABI %u.%u\n", SCRAPGPU_ABI_VERSION_MAJOR, SCRAPGPU_ABI_VERSION_MINOR);
    return 0;
}
"""


def probe(include_dir):
    with tempfile.TemporaryDirectory() as d:
        src = os.path.join(d, "probe.c")
        exe = os.path.join(d, "probe")
        open(src, "w").write(PROBE)
        subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", include_dir, src, "-o", exe], check=True)
        return subprocess.run([exe], capture_output=True, text=True, check=True).stdout


def test_struct_layouts_match_ctypes():
    lines = dict(l.rsplit(" ", 1) for l in probe(INC).splitlines())
    assert int(lines["scrapgpu_tensor_desc"]) == C.sizeof(sg.TensorDesc)
    assert int(lines["scrapgpu_op_desc"]) == C.sizeof(sg.OpDesc)
    assert int(lines["scrapgpu_device_info"]) == C.sizeof(sg.DeviceInfo)
    assert int(lines["scrapgpu_plan_node"]) == C.sizeof(sg.PlanNode)
    assert int(lines["scrapgpu_mul_mat_params"]) == C.sizeof(sg.MulMatParams)
    assert int(lines["scrapgpu_mul_mat_id_params"]) == C.sizeof(sg.MulMatIdParams)
    assert int(lines["scrapgpu_get_rows_params"]) == C.sizeof(sg.GetRowsParams)
    assert int(lines["SCRAPGPU_OP_MUL_MAT_ID"]) == sg.OP_MUL_MAT_ID
    assert int(lines["SCRAPGPU_OP_GET_ROWS"]) == sg.OP_GET_ROWS
    assert int(lines["scrapgpu_tensor_desc.layout"]) == sg.TensorDesc.layout.offset
    assert int(lines["SCRAPGPU_OP_MUL_MAT"]) == sg.OP_MUL_MAT
    assert int(lines["SCRAPGPU_LAYOUT_R32"]) == sg.R32


@pytest.mark.skipif(not os.path.isdir(REF_INC), reason="reference headers absent (GPU box)")
def test_struct_layouts_match_reference_headers():
    # the drop-in claim: the same sizes, offsets, enum values and ABI version as the reference
    assert probe(INC) == probe(REF_INC)


def test_headers_compile_as_c99_and_cpp():
    with tempfile.TemporaryDirectory() as d:
        for lang, std, ext in (("c", "-std=c99", "c"), ("c++", "-std=c++11", "cpp")):
            src = os.path.join(d, "h." + ext)
            open(src, "w").write("".join(f'#include "scrapgpu/{os.path.basename(h)}"\n'
                                         for h in sorted(glob.glob(os.path.join(INC, "scrapgpu", "*.h")))) + "int main(void){return 0;}\n")
            cc = "gcc" if lang == "c" else "g++"
            subprocess.run([cc, std, "-Wall", "-Wextra", "-Werror", "-pedantic", "-I", INC, src, "-o", os.path.join(d, "a.out")], check=True)


# ---------------------------------------------------------------------------------------------
# core behaviour without a GPU
# ---------------------------------------------------------------------------------------------

def test_version_status_and_last_error():
    L = sg.lib()
    assert L.scrapgpu_get_abi_version() == (0 << 16) | 4
    assert L.scrapgpu_status_string(sg.DEVICE_LOST) == b"DEVICE_LOST"
    assert L.scrapgpu_status_string(77) == b"UNKNOWN"
    L.scrapgpu_set_last_error(b"hello")
    assert L.scrapgpu_last_error() == b"hello"
    L.scrapgpu_clear_last_error()
    assert L.scrapgpu_last_error() == b""


def test_tensor_helpers():
    L = sg.lib()
    assert (L.scrapgpu_dtype_block_size(sg.Q4_K), L.scrapgpu_dtype_type_size(sg.Q4_K)) == (256, 144)
    assert (L.scrapgpu_dtype_block_size(sg.Q6_K), L.scrapgpu_dtype_type_size(sg.Q6_K)) == (256, 210)
    assert (L.scrapgpu_dtype_block_size(sg.Q8_0), L.scrapgpu_dtype_type_size(sg.Q8_0)) == (32, 34)
    assert L.scrapgpu_tensor_row_size(sg.Q4_0, 64) == 36
    assert L.scrapgpu_tensor_row_size(sg.Q4_0, 33) == 36  # blocks rounded up
    t = sg.tdesc(sg.Q4_0, (64, 33, 2))
    assert L.scrapgpu_tensor_is_contiguous(C.byref(t)) == 1
    # 33 rows x 36 B = 1188: not a multiple of 16 with 2 slices -> not R32-eligible (tensor.h:348-361)
    assert L.scrapgpu_tensor_r32_eligible(C.byref(t)) == 0
    t1 = sg.tdesc(sg.Q4_0, (64, 33, 1))
    assert L.scrapgpu_tensor_r32_eligible(C.byref(t1)) == 1
    t2 = sg.tdesc(sg.Q6_K, (256, 72, 3))
    assert L.scrapgpu_tensor_r32_eligible(C.byref(t2)) == 1
    f = sg.tdesc(sg.F32, (64, 4))
    assert L.scrapgpu_tensor_r32_eligible(C.byref(f)) == 0
    part = sg.tdesc(sg.Q4_0, (48, 4))  # partial block per row
    assert L.scrapgpu_tensor_r32_eligible(C.byref(part)) == 0
    strided = sg.tdesc(sg.F32, (4, 4), nb=[4, 20, 80, 80])
    assert L.scrapgpu_tensor_is_contiguous(C.byref(strided)) == 0


def test_op_validation_rules():
    L = sg.lib()
    w, x, y = sg.tdesc(sg.Q4_K, (256, 8)), sg.tdesc(sg.F32, (256, 1)), sg.tdesc(sg.F32, (8, 1))
    op, keep = sg.mul_mat_op(w, x, y)
    assert L.scrapgpu_op_desc_validate(C.byref(op)) == sg.OK
    bad = sg.OpDesc.from_buffer_copy(op)
    bad.params = None
    bad.params_size = 0
    assert L.scrapgpu_op_desc_validate(C.byref(bad)) == sg.INVALID_ARGUMENT
    assert b"params" in L.scrapgpu_last_error()
    y16 = sg.tdesc(sg.F16, (8, 1))
    op2, keep2 = sg.mul_mat_op(w, x, y16)
    assert L.scrapgpu_op_desc_validate(C.byref(op2)) == sg.INVALID_ARGUMENT
    small = sg.OpDesc.from_buffer_copy(op)
    small.struct_size = 8
    assert L.scrapgpu_op_desc_validate(C.byref(small)) == sg.INVALID_ARGUMENT
    multi, k3 = sg.multi_op([w, w, w, w], x, [y, y, y, y])  # n = 4 > 3
    assert L.scrapgpu_op_desc_validate(C.byref(multi)) == sg.INVALID_ARGUMENT
    multi, k3 = sg.multi_op([w, w], x, [y, y])
    assert L.scrapgpu_op_desc_validate(C.byref(multi)) == sg.OK
    unknown = sg.OpDesc.from_buffer_copy(op)
    unknown.op = 999
    assert L.scrapgpu_op_desc_validate(C.byref(unknown)) == sg.INVALID_ARGUMENT
    reason = C.c_char_p()
    assert L.scrapgpu_op_supported(None, C.byref(op), C.byref(reason)) == sg.UNSUPPORTED
    assert reason.value


def test_hip_register_without_gpu_is_ok():
    L = sg.lib()
    assert L.scrapgpu_hip_register() == sg.OK
    assert L.scrapgpu_hip_register() == sg.OK  # idempotent
    if L.scrapgpu_get_device_count() == 0:
        d = C.c_void_p()
        assert L.scrapgpu_get_device(0, C.byref(d)) == sg.UNSUPPORTED


# ---------------------------------------------------------------------------------------------
# registry dispatch through a fake backend (the pattern of tests/core/compat_tests.cpp:13-31)
# ---------------------------------------------------------------------------------------------

ST = C.c_int
VP = C.c_void_p
FN = {
    "get_device_count": C.CFUNCTYPE(C.c_size_t, VP),
    "get_device": C.CFUNCTYPE(ST, VP, C.c_size_t, C.POINTER(VP)),
    "device_get_info": C.CFUNCTYPE(ST, VP, VP),
    "buffer_alloc": C.CFUNCTYPE(ST, VP, C.c_size_t, C.POINTER(VP)),
    "buffer_free": C.CFUNCTYPE(ST, VP),
    "buffer_write": C.CFUNCTYPE(ST, VP, VP, C.c_uint64, VP, C.c_size_t, C.c_int),
    "buffer_read": C.CFUNCTYPE(ST, VP, VP, C.c_uint64, VP, C.c_size_t, C.c_int),
    "buffer_copy": C.CFUNCTYPE(ST, VP, VP, C.c_uint64, VP, C.c_uint64, C.c_size_t, C.c_int),
    "buffer_fill": C.CFUNCTYPE(ST, VP, VP, C.c_uint64, C.c_size_t, C.c_uint8, C.c_int),
    "stream_sync": C.CFUNCTYPE(ST, VP),
    "op_supported": C.CFUNCTYPE(ST, VP, VP, VP),
    "plan_build": C.CFUNCTYPE(ST, VP, VP, C.POINTER(VP)),
    "plan_execute": C.CFUNCTYPE(ST, VP, VP),
    "plan_free": C.CFUNCTYPE(ST, VP),
}
ORDER = list(FN)


class Vtable(C.Structure):
    # the full scrapgpu_backend_vtable; the ABI 0.3/0.4 tail stays NULL in this fake
    _fields_ = ([("struct_size", C.c_size_t), ("name", C.c_char_p), ("userdata", VP)] + [(n, FN[n]) for n in ORDER] +
                [(n, VP) for n in ("stream_create", "stream_free", "tensor_upload", "tensor_download", "op_execute", "stream_device")])


def test_fake_backend_dispatch_and_short_vtable():
    L = sg.lib()
    calls = []
    vt = Vtable()
    objs = {}

    def header(key):
        # every object starts with a pointer to the owning vtable (scrapgpu_object_header)
        if key not in objs:
            objs[key] = (C.c_void_p * 2)(C.addressof(registered[0]), None) if registered else None
        return objs[key]

    registered = []

    def get_device_count(ud):
        return 1

    def get_device(ud, idx, out):
        out[0] = C.addressof(header("dev"))
        return 0

    def buffer_alloc(dev, size, out):
        calls.append(("alloc", size))
        out[0] = C.addressof(header("buf"))
        return 0

    def buffer_free(buf):
        calls.append(("free",))
        return 0

    impls = {"get_device_count": get_device_count, "get_device": get_device, "buffer_alloc": buffer_alloc, "buffer_free": buffer_free}
    keep = []
    for n in ORDER:
        f = FN[n](impls[n]) if n in impls else FN[n]()
        keep.append(f)
        setattr(vt, n, f)
    vt.name = b"fake"
    # registered as an ABI 0.2 backend (struct_size ends at plan_free): the core pads its copy
    vt.struct_size = Vtable.plan_free.offset + C.sizeof(C.c_void_p)
    L.scrapgpu_unregister_all_backends()
    assert L.scrapgpu_register_backend(C.byref(vt)) == sg.OK
    # objects carry the backend's own table in their header; the core dispatches through it
    registered.append(vt)
    try:
        assert L.scrapgpu_get_device_count() == 1
        dev = C.c_void_p()
        assert L.scrapgpu_get_device(0, C.byref(dev)) == sg.OK
        buf = C.c_void_p()
        assert L.scrapgpu_buffer_alloc(dev, 123, C.byref(buf)) == sg.OK
        assert calls == [("alloc", 123)]
        # entries past the short table are UNSUPPORTED with a reason, not a crash
        st = C.c_void_p()
        assert L.scrapgpu_stream_create(dev, C.byref(st)) == sg.UNSUPPORTED
        assert L.scrapgpu_last_error()
        assert L.scrapgpu_buffer_free(buf) == sg.OK
        # objects outlive their backend's registration: after unregister_all they are dispatched
        # through their header's own table (freeing them still reaches the backend), and a table
        # registered again is called through its new copy
        b1, b2 = C.c_void_p(), C.c_void_p()
        assert L.scrapgpu_buffer_alloc(dev, 1, C.byref(b1)) == sg.OK
        assert L.scrapgpu_buffer_alloc(dev, 2, C.byref(b2)) == sg.OK
        L.scrapgpu_unregister_all_backends()
        assert L.scrapgpu_get_device_count() == 0
        assert L.scrapgpu_buffer_free(b1) == sg.OK
        assert L.scrapgpu_register_backend(C.byref(vt)) == sg.OK
        assert L.scrapgpu_register_backend(C.byref(vt)) == sg.OK  # re-registration: one entry
        assert L.scrapgpu_get_device_count() == 1
        assert L.scrapgpu_buffer_free(b2) == sg.OK
        assert calls[-4:] == [("alloc", 1), ("alloc", 2), ("free",), ("free",)]
        # an object without a usable header table is rejected
        stray = (C.c_void_p * 2)(None, None)
        assert L.scrapgpu_buffer_free(C.addressof(stray)) == sg.INVALID_ARGUMENT
        # incomplete vtables are refused
        bad = Vtable.from_buffer_copy(vt)
        bad.name = None
        assert L.scrapgpu_register_backend(C.byref(bad)) == sg.INVALID_ARGUMENT
    finally:
        L.scrapgpu_unregister_all_backends()
