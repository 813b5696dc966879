"""Decode matvec (N <= 8) precision where the activations' outliers do not dominate y, and
non-finite activations, against the CPU oracle (the reference's fp32 MUL_MAT restated,
src/core/ref/ops.cpp:958-980; its GPU kernel computes the same fp32 sums, mul_mv_k.cl:151-180).

The decode kernels carry x as three int8 planes per 32-element segment, exact to 1.03 * 2^-24 of
the segment's largest |x|. The hard case for such a representation is an outlier channel whose
weights are zero or tiny: the outlier then sets the segment's scale while contributing nothing to
y, and every other element's precision is measured against it. Here each 32-element segment holds
one +-100 sigma channel (the same channel in every token) and that channel's weights are exactly
zero or ~1e-4 (before quantization), for all four formats, N = 1 and 8, K = 4096 and 12288, and
at the Qwen3-8B gate+up (MUL_MAT_MULTI of two 12288 x 4096 Q4_K) and down (4096 x 12288 Q6_K)
shapes. Gates: NMSE <= 1e-7 and max-abs <= 1e-4 ||x||_2 max|w| per column.

Non-finite x: the reference's fp32 dot product gives +-Inf where an Inf meets a non-zero weight,
NaN where it meets a zero weight, where +Inf and -Inf terms meet, and wherever x holds a NaN.
Segments with a non-finite element (or all elements below 2^-90) are summed in fp32 by the kernel
instead of through the planes, so each output must have the oracle's class (NaN / +Inf / -Inf /
finite), and the finite outputs its value within the decode gates. Every kernel form is reached:
the one-column burst, its K-chunked form, the streaming form (K past 64 steps), the multi-column
form on 32x32x32 MFMAs (one K chunk and several), the 16x16x64 multi-column form with its x
pre-pass (x not 16-byte aligned), the streaming multi-column form (several slices), and
MUL_MAT_ID.
"""
import os

import numpy as np
import pytest

import oracle as O
import scrapgpulibrary_amd as sg
from tests.gpu_util import check_matvec, nmse, run_mul_mat, upload_weights

pytestmark = pytest.mark.gpu

THREADS = min(16, os.cpu_count() or 1)


def outlier_x(N, K, seed):
    """N(0, 1) with one +-100 element per 32-element segment; pos[g] = its channel in segment g."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((N, K))
    pos = rng.integers(0, 32, K // 32)
    x.reshape(N, K // 32, 32)[:, np.arange(K // 32), pos] = 100.0 * rng.choice([-1.0, 1.0], (N, K // 32))
    return x.astype(np.float32), np.arange(K // 32) * 32 + pos


def small_weights_at(dtype, K, M, cols, wstd, seed):
    """M x K weights ~ N(0, 0.02) whose columns `cols` are ~ N(0, wstd) (0: exactly zero), quantized
    by the oracle: (natural bytes, dequantized weights)."""
    w = O.normal(K * M, seed, 0.0, 0.02).reshape(M, K)
    w[:, cols] = O.normal(M * cols.size, seed + 1, 0.0, 1.0).reshape(M, cols.size) * wstd
    q = O.quantize(dtype, w, threads=THREADS)
    return q, O.dequantize(dtype, q, K * M).reshape(M, K)


@pytest.mark.parametrize("wstd", [0.0, 1e-4], ids=["zero_w", "tiny_w"])
@pytest.mark.parametrize("N", [1, 8])
@pytest.mark.parametrize("K", [4096, 12288])
@pytest.mark.parametrize("dtype", sg.QTYPES, ids=lambda d: sg.NAMES[d])
def test_outliers_on_small_weights(hip, dtype, K, N, wstd):
    dev, st = hip
    M = 256
    x, pos = outlier_x(N, K, 2000 + N)
    q, deq = small_weights_at(dtype, K, M, pos, wstd, 2100 + K % 97)
    y = run_mul_mat(dev, st, dtype, q, K, M, x)
    ref = O.mul_mat(dtype, q, K, M, x, threads=THREADS)
    e = check_matvec(y, ref, x, deq)
    print(f"{sg.NAMES[dtype]} K={K} N={N} w_std={wstd}: NMSE {e:.3e} ({sg.last_launch()[0]})", flush=True)


def tiled(dtype, K, M, cols, wstd, seed):
    """M rows as copies of 96 rows built by small_weights_at (rows are independent)."""
    q0, d0 = small_weights_at(dtype, K, 96, cols, wstd, seed)
    reps = -(-M // 96)
    return np.tile(q0, reps)[: M * (q0.size // 96)], np.tile(d0, (reps, 1))[:M]


@pytest.mark.parametrize("N", [1, 8])
@pytest.mark.parametrize("shape", ["gate_up", "down"])
def test_outliers_on_small_weights_qwen3_shapes(hip, shape, N):
    """The config-3 layer's largest products at their real shapes: gate+up as one MUL_MAT_MULTI
    of two 12288 x 4096 Q4_K weights, down as 4096 x 12288 Q6_K (each weight's outlier channels
    carry zero weights)."""
    dev, st = hip
    dtype, K, Ms = (sg.Q4_K, 4096, (12288, 12288)) if shape == "gate_up" else (sg.Q6_K, 12288, (4096,))
    x, pos = outlier_x(N, K, 2200 + N)
    xb = dev.alloc(x.nbytes)
    xt = sg.tdesc(sg.F32, (K, N), xb)
    st.upload(xt, x)
    bufs, wts, yts, refs = [xb], [], [], []
    for i, M in enumerate(Ms):
        q, deq = tiled(dtype, K, M, pos, 0.0, 2300 + i)
        wb, wt = upload_weights(dev, st, dtype, q, K, M)
        yb = dev.alloc(4 * M * N)
        bufs += [wb, yb]
        wts.append(wt)
        yts.append(sg.tdesc(sg.F32, (M, N), yb))
        refs.append((O.mul_mat(dtype, q, K, M, x, threads=THREADS), deq))
    op, keep = sg.multi_op(wts, xt, yts) if len(Ms) > 1 else sg.mul_mat_op(wts[0], xt, yts[0])
    st.execute(op)
    st.sync()
    form = sg.last_launch()[0]
    for yt, (ref, deq), M in zip(yts, refs, Ms):
        e = check_matvec(st.download(yt).reshape(N, M), ref, x, deq)
        print(f"{shape} N={N} M={M}: NMSE {e:.3e} ({form})", flush=True)
    for b in bufs:
        b.free()


# ---- non-finite and tiny activations ----------------------------------------------------------

def special_x(N, K, seed, r=0):
    """N(0, 1) columns; column n carries pattern (n + r) % 5: 0: +Inf at k = 5 and a segment of
    1e-35-sized values; 1: -Inf at k = 300 and +Inf at k = 301 (one segment); 2: a NaN; 3: every
    element 1e-36-sized (every segment below the planes' 2^-90 floor); 4: finite, a segment of
    1e-35-sized values and one scaled 1e-26 (just above the floor)."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((N, K)).astype(np.float32)
    for n in range(N):
        p = (n + r) % 5
        if p == 0:
            x[n, 5] = np.inf
            x[n, 64:96] *= np.float32(1e-35)
        elif p == 1:
            x[n, 300] = -np.inf
            x[n, 301] = np.inf
        elif p == 2:
            x[n, K // 2 + 7] = np.nan
        elif p == 3:
            x[n] *= np.float32(1e-36)
        else:
            x[n, 64:96] *= np.float32(1e-35)
            x[n, 512:544] *= np.float32(1e-26)
    return x


def zero_cols(dtype, K, M, seed):
    """Weights ~ N(0, 0.02) whose even rows are exactly zero at the non-finite channels above
    (an Inf there gives NaN on those rows, +-Inf on the others)."""
    w = O.normal(K * M, seed, 0.0, 0.02).reshape(M, K)
    w[0::2, [5, 300, 301]] = 0.0
    q = O.quantize(dtype, w, threads=THREADS)
    return q, O.dequantize(dtype, q, K * M).reshape(M, K)


def check_special(y, ref, x, deq):
    """Same class per output (NaN, +Inf, -Inf, finite) as the oracle; finite outputs of each column
    within the decode gates."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    assert np.array_equal(np.isnan(y), np.isnan(ref)), f"NaN pattern differs: {np.argwhere(np.isnan(y) != np.isnan(ref))[:5]}"
    assert np.array_equal(np.isposinf(y), np.isposinf(ref)), "+Inf pattern differs"
    assert np.array_equal(np.isneginf(y), np.isneginf(ref)), "-Inf pattern differs"
    wmax = float(np.max(np.abs(deq)))
    for n in range(y.shape[0]):
        f = np.isfinite(ref[n])
        if not f.any():
            continue
        e = nmse(y[n, f], ref[n, f])
        assert e <= 1e-7, f"column {n}: NMSE {e:.3e}"
        xf = x[n][np.isfinite(x[n])].astype(np.float64)
        bound = 1e-4 * float(np.linalg.norm(xf)) * wmax
        err = float(np.max(np.abs(y[n, f] - ref[n, f])))
        assert err <= bound, f"column {n}: max abs err {err:.3e} > {bound:.3e}"
    return int(np.sum(~np.isfinite(ref)))


FORMS = {  # name: (K, M, N, slices, kernel form prefix, x offset in floats)
    "burst": (4096, 256, 1, 1, "burst rg=", 0),
    "burst_chunks": (12288, None, 1, 1, "burst-chunks", 0),
    "stream": (16640, 96, 1, 1, "stream nc=1", 0),
    "columns_2": (4096, 96, 2, 1, "columns mfma32 nc=2 chunks=4", 0),
    "columns_8": (4096, 200, 8, 1, "columns mfma32 nc=8 chunks=4", 0),
    "columns_one_chunk": (768, 96, 5, 1, "columns mfma32 nc=5 chunks=1", 0),
    "columns_long_k": (8192, 96, 4, 1, "columns mfma32 nc=4 chunks=4", 0),  # (32 steps: 2 x 4 waves, 8-step chunks)
    "columns_long_k_8": (12288, 200, 8, 1, "columns mfma32 nc=8 chunks=6", 0),
    "columns_unaligned_x": (12288, 96, 5, 1, "columns nc=5 chunks=3 pre", 1),
    "stream_columns": (4096, 64, 4, 2, "stream-columns nc=4", 0),
}


@pytest.mark.parametrize("form", list(FORMS))
@pytest.mark.parametrize("dtype", sg.QTYPES, ids=lambda d: sg.NAMES[d])
def test_nonfinite_activations(hip, dtype, form):
    dev, st = hip
    K, M, N, S, want, off = FORMS[form]
    if M is None:  # 4 row tiles per CU: the chunked burst
        M = 64 * dev.info().compute_units + 40
    q0, d0 = zero_cols(dtype, K, 96, 2400 + K % 97)
    reps = -(-M // 96)
    q, deq = np.tile(q0, reps)[: M * (q0.size // 96)], np.tile(d0, (reps, 1))[:M]
    wb, wt = upload_weights(dev, st, dtype, np.tile(q, S), K, M, slices=S)
    xb, yb = dev.alloc(4 * (K * N * S + off)), dev.alloc(4 * M * N * S)
    xt = sg.tdesc(sg.F32, (K, N, S), xb, offset=4 * off)
    yt = sg.tdesc(sg.F32, (M, N, S), yb)
    op, keep = sg.mul_mat_op(wt, xt, yt)
    for r in (0, 3):  # (one column: patterns 0 and 3)
        x = np.stack([special_x(N, K, 2500 + s, r + s) for s in range(S)])  # [S, N, K]
        st.upload(xt, x)
        st.execute(op)
        st.sync()
        got_form = sg.last_launch()[0]
        assert got_form.startswith(want), got_form
        y = st.download(yt).reshape(S, N, M)
        for s in range(S):
            ref = O.mul_mat(dtype, q, K, M, x[s], threads=THREADS)
            ns = check_special(y[s], ref, x[s], deq)
            print(f"{sg.NAMES[dtype]} {form} r={r} slice {s}: {ns} non-finite outputs match ({got_form})", flush=True)
    for b in (wb, xb, yb):
        b.free()


@pytest.mark.parametrize("dtype", sg.QTYPES, ids=lambda d: sg.NAMES[d])
def test_nonfinite_activations_mul_mat_id(hip, dtype):
    """MUL_MAT_ID's per-pair matvec (x per slot): each pair's output has the class and value of the
    oracle's MUL_MAT on its expert."""
    from tests.test_gpu_mul_mat_id import run_mul_mat_id

    dev, st = hip
    K, M, E, T, nu = 4096, 64, 4, 2, 4
    qs, ds = zip(*(zero_cols(dtype, K, M, 2600 + e) for e in range(E)))
    w = np.concatenate(qs)
    x = np.stack([special_x(nu, K, 2700 + t, t) for t in range(T)])  # [T, nu, K]
    ids = np.array([[0, 1, 2, 3], [3, 3, 1, 0]], np.int32)
    y = run_mul_mat_id(dev, st, dtype, w, K, M, E, x, ids)
    for t in range(T):
        for i in range(nu):
            e = ids[t, i]
            ref = O.mul_mat(dtype, qs[e], K, M, x[t, i][None, :], threads=THREADS)
            check_special(y[t, i][None, :], ref, x[t, i][None, :], ds[e])
