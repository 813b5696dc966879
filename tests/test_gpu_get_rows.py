"""GPU parity of GET_ROWS on R32 weights (the embedding lookup before the path) against the CPU
oracle, bit for bit, through the C-ABI only. Reference semantics: src/core/ref/ops.cpp:690-721
and src/backends/opencl11/kernels/get_set_rows.cl:8-33."""
import os

import numpy as np
import pytest

import oracle as O
import scrapgpulibrary_amd as sg
from tests.gpu_util import upload_weights

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(__file__), "golden", "mul_mat_id_get_rows.npz")


def run_get_rows(dev, st, dtype, w, K, R, ids, slices=1, y_pad=0):
    """dst [n2, n1, n0, K] (+ y_pad floats of row padding) for src0 = `slices` slices of R rows."""
    ids = np.ascontiguousarray(ids, np.int32)
    n2, n1, n0 = ids.shape
    wb, wt = upload_weights(dev, st, dtype, w, K, R, slices=slices)
    ib = dev.alloc(ids.nbytes)
    it = sg.tdesc(sg.I32, (n0, n1, n2), ib)
    st.upload(it, ids)
    row = K + y_pad
    yb = dev.alloc(4 * row * n0 * n1 * n2)
    yt = sg.tdesc(sg.F32, (K, n0, n1, n2), yb, nb=[4, 4 * row, 4 * row * n0, 4 * row * n0 * n1])
    op, keep = sg.get_rows_op(wt, it, yt)
    st.execute(op)
    st.sync()
    flat = sg.tdesc(sg.F32, (row * n0 * n1 * n2,), yb)  # the padded rows, read back whole
    y = st.download(flat).reshape(n2, n1, n0, row)[..., :K].copy()
    for b in (wb, ib, yb):
        b.free()
    return y


@pytest.mark.parametrize("dtype", sg.QTYPES, ids=lambda d: sg.NAMES[d])
def test_golden_get_rows(hip, dtype):
    """The reference's own GET_ROWS outputs (scrapgpu_ref_execute), bit for bit."""
    dev, st = hip
    g = np.load(GOLD)
    name = sg.NAMES[dtype]
    K = 256 if sg.BLOCK[dtype] == 256 else 96
    w, ids, want = g[f"{name}_gr_w"], g[f"{name}_gr_ids"], g[f"{name}_gr_y"]
    y = run_get_rows(dev, st, dtype, w, K, 37, ids.reshape(1, 1, -1))
    assert np.array_equal(y.reshape(-1, K).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("dtype", sg.QTYPES, ids=lambda d: sg.NAMES[d])
def test_get_rows_slices_and_strides(hip, dtype):
    """3 slices of 70 rows (a partial R32 group), ids [4, 3, 1] with repeats and both ends, a
    padded destination row stride; every row equal to the oracle's dequantized row."""
    dev, st = hip
    K, R, S = 4 * sg.BLOCK[dtype], 70, 3
    w = O.quantize(dtype, O.normal(K * R * S, 61, 0.0, 1.0))
    deq = O.dequantize(dtype, w, K * R * S).reshape(S, R, K)
    ids = np.array([[[0, 69, 33, 33], [64, 65, 1, 2], [31, 32, 63, 0]]], np.int32)
    y = run_get_rows(dev, st, dtype, w, K, R, ids, slices=S, y_pad=8)
    for b in range(3):
        assert np.array_equal(y[0, b].view(np.uint32), deq[b][ids[0, b]].view(np.uint32))


def test_get_rows_clamps_out_of_range(hip):
    dev, st = hip
    dtype, K, R = sg.Q6_K, 256, 40
    w = O.quantize(dtype, O.normal(K * R, 71, 0.0, 1.0))
    deq = O.dequantize(dtype, w, K * R).reshape(R, K)
    ids = np.array([[[-3, 40, 7]]], np.int32)
    y = run_get_rows(dev, st, dtype, w, K, R, ids)
    assert np.array_equal(y[0, 0].view(np.uint32), deq[[0, R - 1, 7]].view(np.uint32))
