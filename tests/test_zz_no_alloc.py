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
    # prefill at 512 tokens (f16 x in the scratch), then 64 tokens (split-K partials as well), then
    # one decode column (no scratch): each against scrapgpu_op_execute and the oracle
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
