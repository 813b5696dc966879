"""scrapgpu_hip_op_execute_static: the no-allocation variant of scrapgpu_op_execute, through the
C-ABI. Its output must equal scrapgpu_op_execute's (the same kernels run on the same inputs, so
bit for bit) on consecutive calls that share the static scratch, the second on a smaller input;
an op needing more scratch than the static array holds is refused with a reason."""
import ctypes as C

import numpy as np
import pytest

import oracle as O
import scrapgpulibrary_amd as sg
from tests.gpu_util import quantized, upload_weights

pytestmark = pytest.mark.gpu


def _run(dev, st, wt, x, M, static):
    N, K = x.shape
    xb = dev.alloc(x.nbytes)
    xt = sg.tdesc(sg.F32, (K, N), xb)
    st.upload(xt, x)
    yb = dev.alloc(4 * M * N)
    st.write(yb, 0, np.full(M * N, np.nan, np.float32))
    yt = sg.tdesc(sg.F32, (M, N), yb)
    op, keep = sg.mul_mat_op(wt, xt, yt)
    if static:
        sg.check(sg.lib().scrapgpu_hip_op_execute_static(st.handle, C.byref(op)), "hip_op_execute_static")
    else:
        st.execute(op)
    st.sync()
    y = st.download(yt).reshape(N, M).copy()
    xb.free()
    yb.free()
    return y


@pytest.mark.parametrize("dtype,K", [(sg.Q4_K, 4096), (sg.Q6_K, 4096), (sg.Q4_K, 12288)], ids=["q4_k", "q6_k", "q4_k_long_k"])
def test_static_scratch_matches_op_execute(hip, dtype, K):
    """K = 12288 over 4 row tiles per CU: the decode column runs in K chunks, whose arrival counts
    are the static ones."""
    dev, st = hip
    M = 1536 if K == 4096 else 64 * dev.info().compute_units
    q, _ = quantized(dtype, K, M, 1500)
    wb, wt = upload_weights(dev, st, dtype, q, K, M)
    # prefill at 512 tokens (f16 x in the scratch), then 64 tokens (the narrow GEMM: x in fragment
    # order), then one decode column (no scratch): each against scrapgpu_op_execute and the oracle
    for N in ((512, 64, 1) if K == 4096 else (64, 1)):  # (512 tokens at K = 12288 need more than the static scratch)
        x = O.normal(N * K, 1501 + N).reshape(N, K)
        y_static = _run(dev, st, wt, x, M, True)
        form = sg.last_launch()[0]
        y_plain = _run(dev, st, wt, x, M, False)
        assert np.array_equal(y_static.view(np.uint32), y_plain.view(np.uint32)), f"N={N} [{form}]: outputs differ"
        ref = O.mul_mat(dtype, q, K, M, x, threads=8)
        e = float(np.sum((y_static.astype(np.float64) - ref) ** 2) / np.sum(ref.astype(np.float64) ** 2))
        assert e <= (1e-7 if N <= 8 else 5e-5), f"N={N}: NMSE {e:.3e}"
    wb.free()


def test_static_scratch_wide_64_token_forms(hip):
    """The wide GEMM's 64-token forms through the static scratch: 6144x4096 at 512 tokens (192-row
    tiles, 2 K groups) and then at 256 tokens (384-row tiles, K split over work-groups, partial
    sums in the static scratch), each bit for bit equal to scrapgpu_op_execute's output."""
    dev, st = hip
    K, M = 4096, 6144
    q, _ = quantized(sg.Q4_K, K, M, 1520)
    wb, wt = upload_weights(dev, st, sg.Q4_K, q, K, M)
    for N in (512, 256):
        x = O.normal(N * K, 1521 + N).reshape(N, K)
        y_static = _run(dev, st, wt, x, M, True)
        form = sg.last_launch()[0]
        if dev.info().compute_units == 256:
            assert form.startswith("gemm wide w=12 kg=2 bn=64" if N == 512 else "gemm wide w=12 kg=1 bn=64 rg=1 split=4"), form
        y_plain = _run(dev, st, wt, x, M, False)
        assert np.array_equal(y_static.view(np.uint32), y_plain.view(np.uint32)), f"N={N} [{form}]: outputs differ"
        ref = O.mul_mat(sg.Q4_K, q, K, M, x, threads=8)
        e = float(np.sum((y_static.astype(np.float64) - ref) ** 2) / np.sum(ref.astype(np.float64) ** 2))
        assert e <= 5e-5, f"N={N}: NMSE {e:.3e}"
    wb.free()


def test_static_scratch_256_row_tiles(hip):
    """The wide GEMM's 8-wave form (256-row x 128-token tiles, one work-group per CU) through the
    static scratch: 4096x4096 at 2048 tokens (256 tiles, K whole), then 64 tokens (the narrow
    GEMM), each bit for bit equal to scrapgpu_op_execute's output."""
    dev, st = hip
    K, M = 4096, 4096
    q, _ = quantized(sg.Q4_K, K, M, 1525)
    wb, wt = upload_weights(dev, st, sg.Q4_K, q, K, M)
    for N in (2048, 64):
        x = O.normal(N * K, 1526 + N).reshape(N, K)
        y_static = _run(dev, st, wt, x, M, True)
        form = sg.last_launch()[0]
        if dev.info().compute_units == 256:
            assert form.startswith("gemm wide w=8 kg=1 bn=128 rg=1 split=1" if N == 2048 else "gemm narrow"), form
        y_plain = _run(dev, st, wt, x, M, False)
        assert np.array_equal(y_static.view(np.uint32), y_plain.view(np.uint32)), f"N={N} [{form}]: outputs differ"
        ref = O.mul_mat(sg.Q4_K, q, K, M, x, threads=8)
        e = float(np.sum((y_static.astype(np.float64) - ref) ** 2) / np.sum(ref.astype(np.float64) ** 2))
        assert e <= 5e-5, f"N={N}: NMSE {e:.3e}"
    wb.free()


def test_static_scratch_stream_k_shape(hip):
    """12288x5632 at 768 tokens: scrapgpu_op_execute runs it in the stream-K form (192 384-row
    tiles, fewer than the CUs, 44 stages each); the static entry point runs another GEMM form (the
    stream-K slots do not fit its array), so its output is checked against the oracle (NMSE) and
    for being the same on two calls in a row, not for bit equality with the stream-K output."""
    dev, st = hip
    K, M, N = 5632, 12288, 768
    q, _ = quantized(sg.Q4_K, K, M, 1530)
    wb, wt = upload_weights(dev, st, sg.Q4_K, q, K, M)
    x = O.normal(N * K, 1531).reshape(N, K)
    y_plain = _run(dev, st, wt, x, M, False)
    plain_form = sg.last_launch()[0]
    y_static = _run(dev, st, wt, x, M, True)
    static_form = sg.last_launch()[0]
    y_again = _run(dev, st, wt, x, M, True)
    if dev.info().compute_units == 256:
        assert "stream-k" in plain_form, plain_form
    assert "stream-k" not in static_form, static_form
    assert np.array_equal(y_static.view(np.uint32), y_again.view(np.uint32))
    ref = O.mul_mat(sg.Q4_K, q, K, M, x, threads=8)
    for y, form in ((y_static, static_form), (y_plain, plain_form)):
        e = float(np.sum((y.astype(np.float64) - ref) ** 2) / np.sum(ref.astype(np.float64) ** 2))
        assert e <= 5e-5, f"[{form}]: NMSE {e:.3e}"
    wb.free()


def test_static_scratch_float_matvec_many_columns(hip):
    """F32 weights at 4096 tokens run the exact float matvec (no scratch): the static entry point
    runs them instead of refusing them for scratch they do not use."""
    dev, st = hip
    K, M, N = 4096, 64, 4096
    w = O.normal(M * K, 1540, 0.0, 0.02).astype(np.float32)
    wb = dev.alloc(w.nbytes)
    st.write(wb, 0, w.view(np.uint8).reshape(-1))
    wt = sg.tdesc(sg.F32, (K, M), wb)
    x = O.normal(N * K, 1541).reshape(N, K)
    y_static = _run(dev, st, wt, x, M, True)
    y_plain = _run(dev, st, wt, x, M, False)
    assert np.array_equal(y_static.view(np.uint32), y_plain.view(np.uint32))
    ref = O.mul_mat(sg.F32, w, K, M, x, threads=8)
    e = float(np.sum((y_static.astype(np.float64) - ref) ** 2) / np.sum(ref.astype(np.float64) ** 2))
    assert e <= 1e-10, f"NMSE {e:.3e}"
    wb.free()


def test_static_scratch_refuses_large_ops(hip):
    dev, st = hip
    K, M, N = 12288, 256, 2048  # 2 N K = 48 MiB of f16 activations > 32 MiB
    q, _ = quantized(sg.Q4_K, K, M, 1502)
    wb, wt = upload_weights(dev, st, sg.Q4_K, q, K, M)
    xb, yb = dev.alloc(4 * N * K), dev.alloc(4 * M * N)
    op, keep = sg.mul_mat_op(wt, sg.tdesc(sg.F32, (K, N), xb), sg.tdesc(sg.F32, (M, N), yb))
    stt = sg.lib().scrapgpu_hip_op_execute_static(st.handle, C.byref(op))
    assert stt == sg.UNSUPPORTED
    assert b"static scratch" in sg.lib().scrapgpu_last_error()
    for b in (wb, xb, yb):
        b.free()


def test_static_scratch_float_weights(hip):
    """F16 weights: the 64-column GEMM (x in the static scratch) and the one-column matvec (no
    scratch) equal scrapgpu_op_execute bit for bit, on two calls in a row."""
    dev, st = hip
    K, M = 2048, 512
    w = O.normal(M * K, 1510, 0.0, 0.02).astype(np.float16).view(np.uint16)
    wb = dev.alloc(w.nbytes)
    st.write(wb, 0, w.view(np.uint8).reshape(-1))
    wt = sg.tdesc(sg.F16, (K, M), wb)
    for N in (64, 1):
        x = O.normal(N * K, 1511 + N).reshape(N, K)
        y_static = _run(dev, st, wt, x, M, True)
        y_plain = _run(dev, st, wt, x, M, False)
        assert np.array_equal(y_static.view(np.uint32), y_plain.view(np.uint32)), f"N={N}: outputs differ"
        ref = O.mul_mat(sg.F16, w, K, M, x, threads=8)
        e = float(np.sum((y_static.astype(np.float64) - ref) ** 2) / np.sum(ref.astype(np.float64) ** 2))
        assert e <= (1e-10 if N == 1 else 1e-6), f"N={N}: NMSE {e:.3e}"
    wb.free()
