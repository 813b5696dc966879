"""The narrow GEMM (k_gemm_n: 9..128 tokens, one or two R32 groups per work-group, K split over
its waves and added in LDS): every quantized dtype against the oracle at the prefill gate (NMSE <= 5e-5, and
per token row), on shapes that reach its edges -- a partial last R32 group, token counts on both
sides of the 32-token fragment, a stage count below the waves (idle waves), an odd stage count
(Q4_0 / Q8_0), both wave counts (8 and 16) -- plus MUL_MAT_MULTI over weights whose row counts are
not multiples of 32, repeat launches (bit-identical), and a plan replay."""
import numpy as np
import pytest

import oracle as O
import scrapgpulibrary_amd as sg
from tests.gpu_util import nmse, quantized, upload_weights

pytestmark = pytest.mark.gpu

QT = (sg.Q4_0, sg.Q8_0, sg.Q4_K, sg.Q6_K)

# (K, M, N): M = 1000 and 333 end in a partial R32 group; 96 rows leave most CUs without a group
# (16 waves, or 64 tokens as two work-groups); 12288 and 8990 rows are 1-2 groups per CU (two
# groups per work-group; 8990 rows: an odd group count, the last work-group's second wave idle);
# K = 256 is 2 stages for 8-16 waves; K = 384 an odd stage count; 100 and 128 tokens run as two
# work-groups of 64 per group; 12288 / 12256 / 12224 rows at 33..128 tokens: 3 groups per
# work-group with the tokens in two halves (the last triple 1 or 2 groups short at 12256 / 12224)
SHAPES = [(4096, 1000, 9), (2048, 333, 17), (1536, 64, 32), (4096, 100, 33), (256, 40, 64), (12288, 96, 64),
          (4096, 12288, 64), (2048, 8990, 30), (384, 200, 48), (2048, 1000, 100), (1024, 64, 128),
          (4096, 12256, 100), (2048, 12224, 40)]


def cases():
    out = []
    for dt in QT:
        for K, M, N in SHAPES:
            if K % sg.BLOCK[dt] == 0:
                out.append((dt, K, M, N))
    return out


def run(hip, dt, q, K, M, x, off=0):
    """(two launches' y, form); off: x starts `off` floats into its buffer (off % 4 != 0: not
    16-byte aligned, the pre-pass's scalar path)."""
    dev, st = hip
    N = x.shape[0]
    wb, wt = upload_weights(dev, st, dt, q, K, M)
    xb = dev.alloc(x.nbytes + 4 * off)
    xt = sg.tdesc(sg.F32, (K, N), xb, offset=4 * off)
    st.upload(xt, x)
    yb = dev.alloc(4 * M * N)
    yt = sg.tdesc(sg.F32, (M, N), yb)
    op, keep = sg.mul_mat_op(wt, xt, yt)
    ys = []
    for _ in range(2):
        st.execute(op)
        st.sync()
        ys.append(st.download(yt).reshape(N, M).copy())
    form = sg.last_launch()[0]
    for b in (wb, xb, yb):
        b.free()
    return ys, form


def check(y, ref, what):
    e = nmse(y, ref)
    assert e <= 5e-5, f"{what}: NMSE {e:.3e}"
    for n in range(y.shape[0]):
        en = nmse(y[n], ref[n])
        assert en <= 2e-4, f"{what}: token {n} NMSE {en:.3e}"


@pytest.mark.parametrize("case", cases(), ids=lambda c: f"{O.NAMES[c[0]]}-K{c[1]}-M{c[2]}-N{c[3]}")
def test_narrow(hip, case):
    dt, K, M, N = case
    q, _ = quantized(dt, K, M, 7 + K + M)
    x = O.normal(N * K, 11 + N).reshape(N, K)
    # heavy-tailed rows and an outlier channel: the per-row f16 scaling of x
    x[0] *= 1000.0
    x[-1] *= 1e-3
    x[:, 5] *= 50.0
    (y, y2), form = run(hip, dt, q, K, M, x)
    assert form.startswith("gemm narrow"), form
    assert np.array_equal(y, y2), "repeat launch differs"
    ref = O.mul_mat(dt, q, K, M, x, threads=8)
    check(y, ref, f"{O.NAMES[dt]} {M}x{K} N={N} [{form}]")


@pytest.mark.parametrize("dt", QT, ids=lambda d: O.NAMES[d])
def test_narrow_unaligned_x(hip, dt):
    """x one float past a 16-byte boundary: the pre-pass reads it element by element."""
    K, M, N = 1024, 200, 40
    q, _ = quantized(dt, K, M, 21)
    x = O.normal(N * K, 22).reshape(N, K)
    (y, _), form = run(hip, dt, q, K, M, x, off=1)
    assert form.startswith("gemm narrow"), form
    check(y, O.mul_mat(dt, q, K, M, x, threads=8), f"{O.NAMES[dt]} unaligned x [{form}]")


@pytest.mark.parametrize("dt", QT, ids=lambda d: O.NAMES[d])
def test_narrow_multi(hip, dt):
    """MUL_MAT_MULTI: three weights (row counts 100, 257, 64) sharing x at 40 tokens, one launch."""
    dev, st = hip
    K, N, Ms = 2048, 40, (100, 257, 64)
    x = O.normal(N * K, 5).reshape(N, K)
    xb = dev.alloc(x.nbytes)
    xt = sg.tdesc(sg.F32, (K, N), xb)
    st.write(xb, 0, x)
    bufs, wts, yts, refs = [xb], [], [], []
    for j, M in enumerate(Ms):
        q, _ = quantized(dt, K, M, 60 + j)
        wb, wt = upload_weights(dev, st, dt, q, K, M)
        yb = dev.alloc(4 * M * N)
        bufs += [wb, yb]
        wts.append(wt)
        yts.append(sg.tdesc(sg.F32, (M, N), yb))
        refs.append(O.mul_mat(dt, q, K, M, x, threads=8))
    op, keep = sg.multi_op(wts, xt, yts)
    st.execute(op)
    st.sync()
    form = sg.last_launch()[0]
    assert form.startswith("gemm narrow"), form
    for M, yt, ref in zip(Ms, yts, refs):
        check(st.download(yt).reshape(N, M), ref, f"{O.NAMES[dt]} {M} rows of {Ms} N={N} [{form}]")
    for b in bufs:
        b.free()


@pytest.mark.parametrize("dt", QT, ids=lambda d: O.NAMES[d])
def test_narrow_multi_three_groups(hip, dt):
    """MUL_MAT_MULTI on the 3-groups-per-work-group form: 4096 + 4064 + 4128 rows (384 R32 groups
    together, triples straddling the weights) at 64 tokens."""
    dev, st = hip
    K, N, Ms = 1024, 64, (4096, 4064, 4128)
    x = O.normal(N * K, 15).reshape(N, K)
    xb = dev.alloc(x.nbytes)
    xt = sg.tdesc(sg.F32, (K, N), xb)
    st.write(xb, 0, x)
    bufs, wts, yts, refs = [xb], [], [], []
    for j, M in enumerate(Ms):
        q, _ = quantized(dt, K, M, 160 + j)
        wb, wt = upload_weights(dev, st, dt, q, K, M)
        yb = dev.alloc(4 * M * N)
        bufs += [wb, yb]
        wts.append(wt)
        yts.append(sg.tdesc(sg.F32, (M, N), yb))
        refs.append(O.mul_mat(dt, q, K, M, x, threads=8))
    op, keep = sg.multi_op(wts, xt, yts)
    st.execute(op)
    st.sync()
    form = sg.last_launch()[0]
    if dev.info().compute_units == 256:
        assert form.startswith("gemm narrow rw=3"), form
    for M, yt, ref in zip(Ms, yts, refs):
        check(st.download(yt).reshape(N, M), ref, f"{O.NAMES[dt]} {M} rows of {Ms} N={N} [{form}]")
    for b in bufs:
        b.free()


def test_narrow_plan_replays_shared_x(hip):
    """A plan of a Q4_K and a Q6_K product reading the same x at 48 tokens (the second reuses the
    first's fragment-ordered x), replayed as a graph with new x each time, every replay against
    the oracle."""
    import ctypes as C

    dev, st = hip
    L = sg.lib()
    K, N = 1024, 48
    specs = [(sg.Q4_K, 300, 90), (sg.Q6_K, 200, 91)]
    xb = dev.alloc(4 * K * N)
    xt = sg.tdesc(sg.F32, (K, N), xb)
    bufs, items = [xb], []
    for dt, M, seed in specs:
        q, _ = quantized(dt, K, M, seed)
        wb, wt = upload_weights(dev, st, dt, q, K, M)
        yb = dev.alloc(4 * M * N)
        yt = sg.tdesc(sg.F32, (M, N), yb)
        op, keep = sg.mul_mat_op(wt, xt, yt)
        bufs += [wb, yb]
        items.append((dt, M, q, yt, op, keep))
    nodes = (sg.PlanNode * 2)(*[sg.PlanNode(C.sizeof(sg.PlanNode), it[4], 0) for it in items])
    pd = sg.PlanDesc(C.sizeof(sg.PlanDesc), nodes, 2)
    plan = C.c_void_p()
    sg.check(L.scrapgpu_plan_build(dev.handle, C.byref(pd), C.byref(plan)), "plan_build")
    try:
        for rep in range(3):
            x = O.normal(N * K, 200 + rep).reshape(N, K)
            st.upload(xt, x)
            st.sync()
            sg.check(L.scrapgpu_plan_execute(st.handle, plan), "plan_execute")
            st.sync()
            for dt, M, q, yt, _, _ in items:
                check(st.download(yt).reshape(N, M), O.mul_mat(dt, q, K, M, x, threads=8), f"replay {rep} {O.NAMES[dt]}")
    finally:
        sg.check(L.scrapgpu_plan_free(plan), "plan_free")
    for b in bufs:
        b.free()


@pytest.mark.parametrize("dt,K,M,N", [(sg.Q4_K, 4096, 12288, 64), (sg.Q6_K, 2048, 500, 100), (sg.Q8_0, 1024, 64, 20)],
                         ids=["q4_k-2groups", "q6_k-100tok", "q8_0-idle-waves"])
def test_narrow_new_x_each_launch(hip, dt, K, M, N):
    """One op launched three times with new x (of growing magnitude) written before each: every
    launch converts and reads its own x."""
    dev, st = hip
    q, _ = quantized(dt, K, M, 300 + N)
    wb, wt = upload_weights(dev, st, dt, q, K, M)
    xb = dev.alloc(4 * N * K)
    xt = sg.tdesc(sg.F32, (K, N), xb)
    yb = dev.alloc(4 * M * N)
    yt = sg.tdesc(sg.F32, (M, N), yb)
    op, keep = sg.mul_mat_op(wt, xt, yt)
    for rep in range(3):
        x = O.normal(N * K, 310 + rep).reshape(N, K) * (10.0 ** (rep - 1))
        st.upload(xt, x)
        st.execute(op)
        st.sync()
        form = sg.last_launch()[0]
        assert form.startswith("gemm narrow"), form
        check(st.download(yt).reshape(N, M), O.mul_mat(dt, q, K, M, x, threads=8), f"launch {rep} [{form}]")
    for b in (wb, xb, yb):
        b.free()
