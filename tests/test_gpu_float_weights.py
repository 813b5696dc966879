"""MUL_MAT with float weights (F32 / F16 / BF16 rows in the natural layout) through the C-ABI,
against the oracle (the reference's exec_mul_mat restated, pinned by its golden vectors) and the
reference's golden vectors themselves. 1..8 columns run exact f32 products (the decode gate:
NMSE <= 1e-7 and max-abs <= 1e-4 ||x||_2 max|w|)."""
import os

import numpy as np
import pytest

import oracle as O
import scrapgpulibrary_amd as sg
from tests.gpu_util import check_matvec, nmse

pytestmark = pytest.mark.gpu

FT = (sg.F32, sg.F16, sg.BF16)
IDS = {sg.F32: "f32", sg.F16: "f16", sg.BF16: "bf16"}


def float_weights(dtype, M, K, seed, std=0.02):
    """(bytes as stored, the weights as f32) of M rows of K."""
    w = O.normal(M * K, seed, 0.0, std).reshape(M, K)
    if dtype == sg.F32:
        return w, w
    if dtype == sg.F16:
        h = w.astype(np.float16)
        return h.view(np.uint16), h.astype(np.float32)
    b = O.float_to_bf16(w)
    return b, O.bf16_to_float(b).reshape(M, K)


def run(dev, st, dtype, wbytes, K, M, x, row_stride=None, x_offset=0, check_form=True):
    """y [N, M] = W x, W uploaded with rows `row_stride` bytes apart (default: packed)."""
    N = x.shape[0]
    esz = sg.TYPE_SIZE[dtype]
    rs = row_stride or K * esz
    img = np.zeros((M, rs), np.uint8)
    img[:, :K * esz] = np.ascontiguousarray(wbytes).view(np.uint8).reshape(M, K * esz)
    wb = dev.alloc(img.nbytes)
    st.write(wb, 0, img)
    wt = sg.tdesc(dtype, (K, M), wb, nb=[esz, rs, rs * M, rs * M])
    xb = dev.alloc(x.nbytes + x_offset)
    xt = sg.tdesc(sg.F32, (K, N), xb, offset=x_offset)
    st.write(xb, x_offset, np.ascontiguousarray(x, np.float32))
    yb = dev.alloc(4 * M * N)
    yt = sg.tdesc(sg.F32, (M, N), yb)
    op, keep = sg.mul_mat_op(wt, xt, yt)
    st.execute(op)
    st.sync()
    form, grid = sg.last_launch()
    if check_form:
        ncp = 1 if N == 1 else 2 if N == 2 else 4 if N <= 4 else 8
        assert form == f"float rows=8 nc={ncp}", form
        assert grid == (M + 7) // 8, (form, grid)
    y = st.download(yt).reshape(N, M).copy()
    for b in (wb, xb, yb):
        b.free()
    return y


@pytest.mark.parametrize("dtype", FT, ids=lambda d: IDS[d])
@pytest.mark.parametrize("K,M,N", [(4096, 1000, 1), (4096, 256, 2), (520, 77, 3), (4096, 512, 4), (1536, 333, 5), (12288, 264, 8)])
def test_float_decode(hip, dtype, K, M, N):
    """Every dtype at 1..8 columns: a row tail (M not a multiple of 8), K not a multiple of the
    512-element step (520, 1536 over 4 waves), a long K."""
    dev, st = hip
    wbytes, wf = float_weights(dtype, M, K, 7000 + K + M)
    x = O.normal(N * K, 7001 + N).reshape(N, K)
    y = run(dev, st, dtype, wbytes, K, M, x)
    ref = O.mul_mat(dtype, wbytes, K, M, x, threads=8)
    e = check_matvec(y, ref, x, wf)
    assert e <= 1e-10, f"NMSE {e:.3e}"


@pytest.mark.parametrize("dtype", FT, ids=lambda d: IDS[d])
def test_float_golden(hip, dtype):
    """The reference's own outputs (tests/golden/float_weights.npz, scrapgpu_ref_execute) at 1, 3 and
    7 columns, with weights outside F16's normal range (subnormal, hundreds)."""
    dev, st = hip
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "float_weights.npz"))
    n = IDS[dtype]
    for M, N in ((24, 1), (23, 3), (37, 7)):
        k = f"{n}_mm_K72_M{M}_N{N}"
        w, x, yref = g[k + "_w"], g[k + "_x"], g[k + "_y"]
        y = run(dev, st, dtype, w, 72, M, x)
        assert np.allclose(y, yref, rtol=1e-5, atol=1e-5 * float(np.max(np.abs(yref)))), k
        assert nmse(y, yref) <= 1e-12, k


@pytest.mark.parametrize("dtype", FT, ids=lambda d: IDS[d])
def test_float_padded_rows_and_unaligned_x(hip, dtype):
    """Rows 48 bytes longer than K elements (the row stride is honoured), x 4 bytes past a 16-byte
    boundary (the scalar x loads)."""
    dev, st = hip
    K, M, N = 1024, 100, 3
    wbytes, wf = float_weights(dtype, M, K, 7100)
    x = O.normal(N * K, 7101).reshape(N, K)
    rs = K * sg.TYPE_SIZE[dtype] + 48
    y = run(dev, st, dtype, wbytes, K, M, x, row_stride=rs, x_offset=4)
    ref = O.mul_mat(dtype, wbytes, K, M, x, threads=8)
    check_matvec(y, ref, x, wf)


def test_float_slices_broadcast(hip):
    """F16 weights of 2 slices under x of 4 slices (allow_broadcast): slice i of x uses weight slice
    i // 2."""
    dev, st = hip
    K, M, N, S, SW = 512, 40, 2, 4, 2
    ws = [float_weights(sg.F16, M, K, 7200 + i) for i in range(SW)]
    img = np.concatenate([w[0].reshape(-1) for w in ws]).view(np.uint8)
    wb = dev.alloc(img.nbytes)
    st.write(wb, 0, img)
    rb = 2 * K
    wt = sg.tdesc(sg.F16, (K, M, SW), wb, nb=[2, rb, rb * M, rb * M * SW])
    x = O.normal(S * N * K, 7201).reshape(S, N, K)
    xb = dev.alloc(x.nbytes)
    xt = sg.tdesc(sg.F32, (K, N, S), xb)
    st.write(xb, 0, x)
    yb = dev.alloc(4 * M * N * S)
    yt = sg.tdesc(sg.F32, (M, N, S), yb)
    op, keep = sg.mul_mat_op(wt, xt, yt, allow_broadcast=1)
    st.execute(op)
    st.sync()
    y = st.download(yt).reshape(S, N, M)
    for i in range(S):
        wbytes, wf = ws[i // (S // SW)]
        ref = O.mul_mat(sg.F16, wbytes, K, M, x[i])
        check_matvec(y[i], ref, x[i], wf)
    for b in (wb, xb, yb):
        b.free()


@pytest.mark.parametrize("dtype", FT, ids=lambda d: IDS[d])
def test_float_multi(hip, dtype):
    """MUL_MAT_MULTI of three float weights sharing x (q / k / v shapes at 2 columns): one launch
    over all their rows."""
    dev, st = hip
    K, N, Ms = 2048, 2, (512, 128, 136)
    x = O.normal(N * K, 7300).reshape(N, K)
    xb = dev.alloc(x.nbytes)
    xt = sg.tdesc(sg.F32, (K, N), xb)
    st.write(xb, 0, x)
    bufs, wts, yts, refs = [xb], [], [], []
    for i, M in enumerate(Ms):
        wbytes, wf = float_weights(dtype, M, K, 7301 + i)
        wb = dev.alloc(wbytes.nbytes)
        st.write(wb, 0, np.ascontiguousarray(wbytes).view(np.uint8).reshape(-1))
        wts.append(sg.tdesc(dtype, (K, M), wb))
        yb = dev.alloc(4 * M * N)
        yts.append(sg.tdesc(sg.F32, (M, N), yb))
        bufs += [wb, yb]
        refs.append((O.mul_mat(dtype, wbytes, K, M, x), wf))
    op, keep = sg.multi_op(wts, xt, yts)
    st.execute(op)
    st.sync()
    form, grid = sg.last_launch()
    assert form == "float rows=8 nc=2" and grid == sum((M + 7) // 8 for M in Ms), (form, grid)
    for M, yt, (ref, wf) in zip(Ms, yts, refs):
        check_matvec(st.download(yt).reshape(N, M), ref, x, wf)
    for b in bufs:
        b.free()


def test_float_support_rules(hip):
    dev, st = hip
    K, M = 1024, 16
    wb, xb, yb = dev.alloc(4 * K * M), dev.alloc(4 * K * 16), dev.alloc(4 * M * 16)
    x, y = sg.tdesc(sg.F32, (K, 1), xb), sg.tdesc(sg.F32, (M, 1), yb)
    ok = sg.tdesc(sg.F16, (K, M), wb)
    assert dev.supported(sg.mul_mat_op(ok, x, y)[0])[0] == sg.OK
    k_odd = sg.tdesc(sg.F16, (K - 4, M), wb)
    stt, reason = dev.supported(sg.mul_mat_op(k_odd, sg.tdesc(sg.F32, (K - 4, 1), xb), y)[0])
    assert stt == sg.UNSUPPORTED and "multiple of 8" in reason
    unaligned = sg.tdesc(sg.F16, (K, M), wb, nb=[2, 2 * K + 8, (2 * K + 8) * M, (2 * K + 8) * M])
    stt, reason = dev.supported(sg.mul_mat_op(unaligned, x, y)[0])
    assert stt == sg.UNSUPPORTED and "16-byte" in reason
    i32 = sg.tdesc(sg.I32, (K, M), wb)  # not a MUL_MAT src0 dtype at all (the core's op rule)
    assert dev.supported(sg.mul_mat_op(i32, x, y)[0])[0] == sg.INVALID_ARGUMENT
    for b in (wb, xb, yb):
        b.free()


# ---- more than 8 columns ------------------------------------------------------------------------
# F16 / BF16 with K a multiple of 128: the MFMA GEMM (f16 operands for F16, the weights exact; bf16
# operands for BF16, x rounded to bf16): the prefill gate NMSE <= 5e-5, and tighter bounds that a
# lost bit of either operand would break. F32 and other K: the exact matvec per group of 8 columns.

PREFILL_NMSE = {sg.F16: 1e-6, sg.BF16: 2e-5}


@pytest.mark.parametrize("dtype", (sg.F16, sg.BF16), ids=lambda d: IDS[d])
@pytest.mark.parametrize("K,M,N", [(4096, 1000, 64), (2048, 384, 200), (512, 4096, 512), (1024, 8192, 9)])
def test_float_prefill_gemm(hip, dtype, K, M, N):
    dev, st = hip
    wbytes, wf = float_weights(dtype, M, K, 7400 + K + N)
    x = O.normal(N * K, 7401 + N).reshape(N, K)
    x[:, ::37] *= 100.0  # outlier channels: the per-row scaling of x keeps them in range
    y = run(dev, st, dtype, wbytes, K, M, x, check_form=False)
    form, _ = sg.last_launch()
    assert form.startswith("gemm w=4 kg=1"), form
    ref = O.mul_mat(dtype, wbytes, K, M, x, threads=8)
    e = nmse(y, ref)
    assert e <= PREFILL_NMSE[dtype], f"{IDS[dtype]} {M}x{K} N={N}: NMSE {e:.3e} [{form}]"


@pytest.mark.parametrize("dtype", (sg.F16, sg.BF16), ids=lambda d: IDS[d])
@pytest.mark.parametrize("K,M,N,split", [(1024, 24536, 500, 1), (4096, 12288, 380, 2)], ids=["fill", "k_split"])
def test_float_prefill_wide_gemm(hip, dtype, K, M, N, split):
    """F16 / BF16 on the wide GEMM (384-row x 128-token tiles, one 12-wave work-group per CU): a
    ragged shape whose tiles fill the CUs (the last row tile and token tile part empty), and one
    with K split over 2 work-groups per tile (96 tiles, the last token tile part empty; partials
    added by the split reduce)."""
    dev, st = hip
    wbytes, wf = float_weights(dtype, M, K, 7700 + K + N)
    x = O.normal(N * K, 7701 + N).reshape(N, K)
    x[:, ::41] *= 100.0
    y = run(dev, st, dtype, wbytes, K, M, x, check_form=False)
    form, _ = sg.last_launch()
    if dev.info().compute_units == 256:
        assert form.startswith(f"gemm wide w=12 kg=1 bn=128 rg=1 split={split}"), form
    else:
        assert form.startswith("gemm"), form
    ref = O.mul_mat(dtype, wbytes, K, M, x, threads=8)
    e = nmse(y, ref)
    assert e <= PREFILL_NMSE[dtype], f"{IDS[dtype]} {M}x{K} N={N}: NMSE {e:.3e} [{form}]"


@pytest.mark.parametrize("dtype,K,N", [(sg.F32, 1024, 20), (sg.F16, 520, 17), (sg.BF16, 72, 33)], ids=["f32", "f16_k520", "bf16_k72"])
def test_float_prefill_column_groups(hip, dtype, K, N):
    """F32 weights and K not a multiple of 128: exact products, 8 columns per launch."""
    dev, st = hip
    M = 300
    wbytes, wf = float_weights(dtype, M, K, 7500 + K)
    x = O.normal(N * K, 7501).reshape(N, K)
    y = run(dev, st, dtype, wbytes, K, M, x, check_form=False)
    assert sg.last_launch()[0] == f"float rows=8 column-groups={(N + 7) // 8}"
    ref = O.mul_mat(dtype, wbytes, K, M, x, threads=8)
    check_matvec(y, ref, x, wf)


@pytest.mark.parametrize("dtype", (sg.F16, sg.BF16), ids=lambda d: IDS[d])
def test_float_prefill_multi(hip, dtype):
    """A prefill MUL_MAT_MULTI of three float weights (q / k / v shapes): one GEMM over all rows."""
    dev, st = hip
    K, N, Ms = 1024, 96, (512, 128, 136)
    x = O.normal(N * K, 7600).reshape(N, K)
    xb = dev.alloc(x.nbytes)
    xt = sg.tdesc(sg.F32, (K, N), xb)
    st.write(xb, 0, x)
    bufs, wts, yts, refs = [xb], [], [], []
    for i, M in enumerate(Ms):
        wbytes, wf = float_weights(dtype, M, K, 7601 + i)
        wb = dev.alloc(wbytes.nbytes)
        st.write(wb, 0, np.ascontiguousarray(wbytes).view(np.uint8).reshape(-1))
        wts.append(sg.tdesc(dtype, (K, M), wb))
        yb = dev.alloc(4 * M * N)
        yts.append(sg.tdesc(sg.F32, (M, N), yb))
        bufs += [wb, yb]
        refs.append(O.mul_mat(dtype, wbytes, K, M, x, threads=8))
    op, keep = sg.multi_op(wts, xt, yts)
    st.execute(op)
    st.sync()
    form, _ = sg.last_launch()
    assert form.startswith("gemm w=4 kg=1"), form
    for M, yt, ref in zip(Ms, yts, refs):
        e = nmse(st.download(yt).reshape(N, M), ref)
        assert e <= PREFILL_NMSE[dtype], f"{M} rows: NMSE {e:.3e}"
    for b in bufs:
        b.free()


# ---- GET_ROWS -----------------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", (sg.F32, sg.F16), ids=lambda d: IDS[d])
def test_float_get_rows(hip, dtype):
    """GET_ROWS on F32 / F16 rows: the reference's golden rows (F16), and the oracle's rows for
    repeated, first and last indices; an index past the rows reads the last one (the GPU rule)."""
    dev, st = hip
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "float_weights.npz"))
    K, R = 72, 37
    if dtype == sg.F16:
        wbytes, rid, yref = g["f16_gr_w"], g["f16_gr_ids"], g["f16_gr_y"]
    else:
        wbytes = O.normal(K * R, 7700).reshape(R, K)
        rid = np.array([0, R - 1, 5, 5, 12, 30], np.int32)
        yref = O.get_rows(dtype, wbytes, K, R, rid)
    rid_dev = np.concatenate([rid, np.array([R + 5], np.int32)])
    wb = dev.alloc(np.ascontiguousarray(wbytes).nbytes)
    st.write(wb, 0, np.ascontiguousarray(wbytes).view(np.uint8).reshape(-1))
    ib, yb = dev.alloc(4 * rid_dev.size), dev.alloc(4 * K * rid_dev.size)
    st.write(ib, 0, rid_dev)
    wt = sg.tdesc(dtype, (K, R), wb)
    it = sg.tdesc(sg.I32, (rid_dev.size,), ib)
    yt = sg.tdesc(sg.F32, (K, rid_dev.size), yb)
    op, keep = sg.get_rows_op(wt, it, yt)
    st.execute(op)
    st.sync()
    y = st.download(yt).reshape(rid_dev.size, K)
    assert np.array_equal(y[:-1].view(np.uint32), np.asarray(yref).view(np.uint32))
    assert np.array_equal(y[-1].view(np.uint32), y[1].view(np.uint32))
    for b in (wb, ib, yb):
        b.free()


# ---- MUL_MAT_ID ---------------------------------------------------------------------------------

def run_mid(dev, st, dtype, wbytes, K, M, E, x, ids):
    T, nu = ids.shape
    n1 = x.shape[1]
    w = np.ascontiguousarray(wbytes).view(np.uint8).reshape(-1)
    wb = dev.alloc(w.nbytes)
    st.write(wb, 0, w)
    wt = sg.tdesc(dtype, (K, M, E), wb)
    xb, ib, yb = dev.alloc(x.nbytes), dev.alloc(ids.nbytes), dev.alloc(4 * M * nu * T)
    st.write(xb, 0, np.ascontiguousarray(x, np.float32))
    st.write(ib, 0, np.ascontiguousarray(ids, np.int32))
    xt, it, yt = sg.tdesc(sg.F32, (K, n1, T), xb), sg.tdesc(sg.I32, (nu, T), ib), sg.tdesc(sg.F32, (M, nu, T), yb)
    op, keep = sg.mul_mat_id_op(wt, xt, it, yt, nu)
    st.execute(op)
    st.sync()
    form, grid = sg.last_launch()
    y = st.download(yt).reshape(T, nu, M).copy()
    for b in (wb, xb, ib, yb):
        b.free()
    return y, form, grid


def test_float_mul_mat_id_golden(hip):
    """F16 experts: the reference's golden MUL_MAT_ID (scrapgpu_ref_execute)."""
    dev, st = hip
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "float_weights.npz"))
    K, M, E = 72, 40, 5
    y, form, grid = run_mid(dev, st, sg.F16, g["f16_mid_w"], K, M, E, g["f16_mid_x"], g["f16_mid_ids"])
    T, nu = g["f16_mid_ids"].shape
    assert form == "float rows=8 nc=1" and grid == (M + 7) // 8 * T * nu, (form, grid)
    assert nmse(y, g["f16_mid_y"]) <= 1e-12


@pytest.mark.parametrize("dtype", (sg.F32, sg.F16), ids=lambda d: IDS[d])
@pytest.mark.parametrize("shared", [True, False], ids=["x_shared", "x_per_slot"])
def test_float_mul_mat_id(hip, dtype, shared):
    """8 experts of 200 x 1024 at 2 slots over 20 tokens (many tokens stay on the per-pair matvec for
    float experts), against the oracle per pair; an id out of range reads the nearest expert."""
    dev, st = hip
    K, M, E, T, nu = 1024, 200, 8, 20, 2
    parts = [float_weights(dtype, M, K, 7800 + e) for e in range(E)]
    wbytes = np.concatenate([p[0].reshape(-1) for p in parts])
    ids = np.random.default_rng(7801).integers(0, E, (T, nu)).astype(np.int32)
    x = O.normal(T * (1 if shared else nu) * K, 7802).reshape(T, 1 if shared else nu, K)
    ref = O.mul_mat_id(dtype, wbytes, K, M, E, x, ids)
    ids_dev = ids.copy()
    ids_dev[3, 1] = E + 4  # clamped to E - 1 on the device
    y, form, _ = run_mid(dev, st, dtype, wbytes, K, M, E, x, ids_dev)
    assert form == "float rows=8 nc=1", form
    ids_c = np.minimum(ids_dev, E - 1)
    ref_c = O.mul_mat_id(dtype, wbytes, K, M, E, x, ids_c)
    for t in range(T):
        for i in range(nu):
            xc = x[t, i if not shared else 0][None, :]
            check_matvec(y[t, i][None, :], ref_c[t, i][None, :], xc, parts[ids_c[t, i]][1])
    assert np.array_equal(ref_c[0], ref[0])


def test_float_plan_replays(hip):
    """Float-weight products recorded in a plan (a HIP graph) and replayed with new x each time: an
    F16 decode column, a BF16 4-column product and an F16 prefill GEMM match the oracle on every
    replay."""
    import ctypes as C

    dev, st = hip
    L = sg.lib()
    K = 1024
    items = []
    for dtype, M, N, seed in ((sg.F16, 200, 1, 7900), (sg.BF16, 96, 4, 7901), (sg.F16, 384, 128, 7902)):
        wbytes, wf = float_weights(dtype, M, K, seed)
        wb = dev.alloc(wbytes.nbytes)
        st.write(wb, 0, np.ascontiguousarray(wbytes).view(np.uint8).reshape(-1))
        xb, yb = dev.alloc(4 * K * N), dev.alloc(4 * M * N)
        xt, yt = sg.tdesc(sg.F32, (K, N), xb), sg.tdesc(sg.F32, (M, N), yb)
        op, keep = sg.mul_mat_op(sg.tdesc(dtype, (K, M), wb), xt, yt)
        items.append(dict(dtype=dtype, M=M, N=N, w=wbytes, wf=wf, bufs=(wb, xb, yb), xt=xt, yt=yt, op=op, keep=keep))
    nodes = (sg.PlanNode * len(items))(*[sg.PlanNode(C.sizeof(sg.PlanNode), it["op"], 0) for it in items])
    pdesc = sg.PlanDesc(C.sizeof(sg.PlanDesc), nodes, len(items))
    plan = C.c_void_p()
    sg.check(L.scrapgpu_plan_build(dev.handle, C.byref(pdesc), C.byref(plan)), "plan_build")
    try:
        for rep in range(3):
            xs = []
            for i, it in enumerate(items):
                x = O.normal(it["N"] * K, 7950 + 10 * rep + i).reshape(it["N"], K)
                st.upload(it["xt"], x)
                xs.append(x)
            st.sync()
            sg.check(L.scrapgpu_plan_execute(st.handle, plan), "plan_execute")
            st.sync()
            for it, x in zip(items, xs):
                y = st.download(it["yt"]).reshape(it["N"], it["M"])
                ref = O.mul_mat(it["dtype"], it["w"], K, it["M"], x)
                if it["N"] > 8:
                    assert nmse(y, ref) <= PREFILL_NMSE[it["dtype"]], f"replay {rep}"
                else:
                    check_matvec(y, ref, x, it["wf"])
    finally:
        sg.check(L.scrapgpu_plan_free(plan), "plan_free")
        for it in items:
            for b in it["bufs"]:
                b.free()
