"""Helpers of the GPU parity tests: upload oracle-quantized weights as R32, run MUL_MAT through the
C-ABI, compare with the oracle."""
import numpy as np

import oracle as O
import scrapgpulibrary_amd as sg


def nmse(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = float(np.sum(b * b))
    num = float(np.sum((a - b) ** 2))
    return num / den if den > 0 else num


def upload_weights(dev, st, dtype, qbytes, K, M, slices=1, layout=sg.R32):
    buf = dev.alloc(max(qbytes.nbytes, 1))
    t = sg.tdesc(dtype, (K, M, slices, 1), buf, layout=layout)
    st.upload(t, qbytes)
    return buf, t


def run_mul_mat(dev, st, dtype, q, K, M, x, bufs=None):
    """y [N, M] = W x for one slice of R32 weights `q` (natural bytes) and x [N, K]."""
    N = x.shape[0]
    wb, wt = upload_weights(dev, st, dtype, q, K, M)
    xb = dev.alloc(x.nbytes)
    xt = sg.tdesc(sg.F32, (K, N), xb)
    st.upload(xt, x)
    yb = dev.alloc(4 * M * N)
    yt = sg.tdesc(sg.F32, (M, N), yb)
    op, keep = sg.mul_mat_op(wt, xt, yt)
    st.execute(op)
    st.sync()
    y = st.download(yt).reshape(N, M).copy()
    for b in (wb, xb, yb):
        b.free()
    return y


def check_matvec(y, ref, x, w_deq, tol_nmse=1e-7):
    """The decode gates: NMSE <= 1e-7 and max|err| <= 1e-4 * ||x||_2 * max|w| (per column)."""
    e = nmse(y, ref)
    assert e <= tol_nmse, f"NMSE {e:.3e} > {tol_nmse}"
    wmax = float(np.max(np.abs(w_deq)))
    for n in range(x.shape[0]):
        bound = 1e-4 * float(np.linalg.norm(x[n].astype(np.float64))) * wmax
        err = float(np.max(np.abs(y[n].astype(np.float64) - ref[n])))
        assert err <= bound, f"column {n}: max abs err {err:.3e} > {bound:.3e}"
    return e


def quantized(dtype, K, M, seed, std=0.02):
    w = O.normal(K * M, seed, 0.0, std)
    q = O.quantize(dtype, w)
    return q, O.dequantize(dtype, q, K * M).reshape(M, K)
