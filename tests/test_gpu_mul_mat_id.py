"""GPU parity of MUL_MAT_ID (expert matvecs with device-side ids) against the CPU oracle, through
the C-ABI only. Reference semantics: src/core/ref/ops.cpp:986-1024; the reference's GPU kernels
read the ids on the device and clamp them (src/backends/opencl11/kernels/mul_mv_r.cl:30-33)."""
import ctypes as C
import os

import numpy as np
import pytest

import oracle as O
import scrapgpulibrary_amd as sg
from tests.gpu_util import check_matvec, upload_weights

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(__file__), "golden", "mul_mat_id_get_rows.npz")


def run_mul_mat_id(dev, st, dtype, w, K, M, E, x, ids):
    """y [T, n_used, M] for experts `w` (natural bytes of E slices), x [T, n1, K], ids [T, n_used]."""
    T, nu = ids.shape
    n1 = x.shape[1]
    wb, wt = upload_weights(dev, st, dtype, w, K, M, slices=E)
    xb = dev.alloc(x.nbytes)
    xt = sg.tdesc(sg.F32, (K, n1, T), xb)
    st.upload(xt, x)
    ib = dev.alloc(ids.nbytes)
    it = sg.tdesc(sg.I32, (nu, T), ib)
    st.upload(it, np.ascontiguousarray(ids, np.int32))
    yb = dev.alloc(4 * M * nu * T)
    yt = sg.tdesc(sg.F32, (M, nu, T), yb)
    op, keep = sg.mul_mat_id_op(wt, xt, it, yt, nu)
    st.execute(op)
    st.sync()
    y = st.download(yt).reshape(T, nu, M).copy()
    for b in (wb, xb, ib, yb):
        b.free()
    return y


def check_pairs(y, ref, x, deq, ids):
    """The decode gates per (slot, token) pair: each output column against its expert's weights."""
    T, nu = ids.shape
    for t in range(T):
        for i in range(nu):
            xc = x[t, i if x.shape[1] > 1 else 0][None, :]
            check_matvec(y[t, i][None, :], ref[t, i][None, :], xc, deq[ids[t, i]])


@pytest.mark.parametrize("dtype", sg.QTYPES, ids=lambda d: sg.NAMES[d])
def test_golden_mul_mat_id(hip, dtype):
    """The reference's own MUL_MAT_ID outputs (scrapgpu_ref_execute, committed fixtures)."""
    dev, st = hip
    g = np.load(GOLD)
    name = sg.NAMES[dtype]
    K = 256 if sg.BLOCK[dtype] == 256 else 96
    M, E = 40, 5
    w, ids = g[f"{name}_mid_w"], g[f"{name}_mid_ids"]
    deq = O.dequantize(dtype, w, K * M * E).reshape(E, M, K)
    for n1 in (1, ids.shape[1]):
        x, want = g[f"{name}_mid_x{n1}"], g[f"{name}_mid_y{n1}"]
        y = run_mul_mat_id(dev, st, dtype, w, K, M, E, x, ids)
        check_pairs(y, want, x, deq, ids)


@pytest.mark.parametrize("dtype", sg.QTYPES, ids=lambda d: sg.NAMES[d])
@pytest.mark.parametrize("shared", [True, False], ids=["x_shared", "x_per_slot"])
def test_mul_mat_id_moe_shapes(hip, dtype, shared):
    """An MoE decode step: 8 experts of 2048 x 264 (a partial row group), 4 slots, 3 tokens."""
    dev, st = hip
    K, M, E, T, nu = 2048, 264, 8, 3, 4
    w = O.quantize(dtype, O.normal(K * M * E, 31, 0.0, 0.02))
    deq = O.dequantize(dtype, w, K * M * E).reshape(E, M, K)
    rng = np.random.default_rng(5)
    ids = np.stack([rng.permutation(E)[:nu] for _ in range(T)]).astype(np.int32)
    x = O.normal(T * (1 if shared else nu) * K, 32).reshape(T, 1 if shared else nu, K)
    y = run_mul_mat_id(dev, st, dtype, w, K, M, E, x, ids)
    ref = O.mul_mat_id(dtype, w, K, M, E, x, ids)
    check_pairs(y, ref, x, deq, ids)


def test_mul_mat_id_clamps_out_of_range_ids(hip):
    """Indices outside [0, E) select the nearest expert on the device (the reference's GPU rule);
    the CPU reference would report INVALID_ARGUMENT instead."""
    dev, st = hip
    dtype, K, M, E = sg.Q4_K, 512, 64, 3
    w = O.quantize(dtype, O.normal(K * M * E, 41, 0.0, 0.02))
    deq = O.dequantize(dtype, w, K * M * E).reshape(E, M, K)
    ids = np.array([[-5, 1], [3, 2], [1000, 0]], np.int32)
    x = O.normal(3 * K, 42).reshape(3, 1, K)
    y = run_mul_mat_id(dev, st, dtype, w, K, M, E, x, ids)
    clamped = np.clip(ids, 0, E - 1)
    check_pairs(y, O.mul_mat_id(dtype, w, K, M, E, x, clamped), x, deq, clamped)


def test_mul_mat_id_plan_reads_ids_on_device(hip):
    """A recorded plan (HIP graph) replayed after the ids changed in device memory follows them."""
    dev, st = hip
    dtype, K, M, E, T, nu = sg.Q8_0, 1024, 96, 6, 2, 2
    w = O.quantize(dtype, O.normal(K * M * E, 51, 0.0, 0.02))
    deq = O.dequantize(dtype, w, K * M * E).reshape(E, M, K)
    wb, wt = upload_weights(dev, st, dtype, w, K, M, slices=E)
    x = O.normal(T * K, 52).reshape(T, 1, K)
    xb = dev.alloc(x.nbytes)
    xt = sg.tdesc(sg.F32, (K, 1, T), xb)
    st.upload(xt, x)
    ib = dev.alloc(4 * nu * T)
    it = sg.tdesc(sg.I32, (nu, T), ib)
    yb = dev.alloc(4 * M * nu * T)
    yt = sg.tdesc(sg.F32, (M, nu, T), yb)
    op, keep = sg.mul_mat_id_op(wt, xt, it, yt, nu)
    nodes = (sg.PlanNode * 1)(sg.PlanNode(C.sizeof(sg.PlanNode), op, 0))
    pdesc = sg.PlanDesc(C.sizeof(sg.PlanDesc), nodes, 1)
    plan = C.c_void_p()
    sg.check(sg.lib().scrapgpu_plan_build(dev.handle, C.byref(pdesc), C.byref(plan)), "plan_build")
    try:
        for ids in (np.array([[0, 5], [2, 3]], np.int32), np.array([[4, 1], [1, 4]], np.int32), np.array([[3, 3], [0, 2]], np.int32)):
            st.upload(it, ids)
            sg.check(sg.lib().scrapgpu_plan_execute(st.handle, plan), "plan_execute")
            st.sync()
            y = st.download(yt).reshape(T, nu, M)
            check_pairs(y, O.mul_mat_id(dtype, w, K, M, E, x, ids), x, deq, ids)
    finally:
        sg.check(sg.lib().scrapgpu_plan_free(plan), "plan_free")
    for b in (wb, xb, ib, yb):
        b.free()


def test_mul_mat_id_support_rules(hip):
    dev, st = hip
    K, M, E = 256, 32, 4
    wb = dev.alloc(O.row_bytes(sg.Q4_K, K) * M * E)
    xb, ib, yb = dev.alloc(4 * K * 3), dev.alloc(4 * 2 * 3), dev.alloc(4 * M * 2 * 3)
    wt = sg.tdesc(sg.Q4_K, (K, M, E), wb, layout=sg.R32)
    xt = sg.tdesc(sg.F32, (K, 1, 3), xb)
    it = sg.tdesc(sg.I32, (2, 3), ib)
    yt = sg.tdesc(sg.F32, (M, 2, 3), yb)
    op, keep = sg.mul_mat_id_op(wt, xt, it, yt, 2)
    assert dev.supported(op)[0] == sg.OK
    op, keep = sg.mul_mat_id_op(wt, xt, it, sg.tdesc(sg.F32, (M, 3, 3), yb), 2)
    assert dev.supported(op)[0] == sg.INVALID_ARGUMENT
    op, keep = sg.mul_mat_id_op(sg.tdesc(sg.Q4_K, (K, M, E), wb), xt, it, yt, 2)
    stt, reason = dev.supported(op)
    assert stt == sg.UNSUPPORTED and "R32" in reason
    op, keep = sg.mul_mat_id_op(wt, xt, sg.tdesc(sg.F32, (2, 3), ib), yt, 2)
    assert dev.supported(op)[0] == sg.UNSUPPORTED
    for b in (wb, xb, ib, yb):
        b.free()


def check_grouped(y, ref, tol=5e-5):
    """The prefill tolerance (f16 MFMA path): NMSE over all pairs and for each pair."""
    from tests.gpu_util import nmse
    e = nmse(y, ref)
    assert e <= tol, f"NMSE {e:.3e}"
    T, nu, M = ref.shape
    for t in range(T):
        for i in range(nu):
            ep = nmse(y[t, i], ref[t, i])
            assert ep <= 20 * tol, f"pair (token {t}, slot {i}): NMSE {ep:.3e}"


@pytest.mark.parametrize("dtype", sg.QTYPES, ids=lambda d: sg.NAMES[d])
@pytest.mark.parametrize("shared", [True, False], ids=["x_shared", "x_per_slot"])
def test_mul_mat_id_grouped_prefill(hip, dtype, shared):
    """More than 8 tokens: pairs grouped by expert on the device, one MFMA GEMM (32-pair tiles,
    16 experts, 200 rows = a partial row tile)."""
    dev, st = hip
    K, M, E, T, nu = 512, 200, 16, 40, 4
    w = O.quantize(dtype, O.normal(K * M * E, 61, 0.0, 0.02))
    rng = np.random.default_rng(62)
    ids = np.stack([rng.permutation(E)[:nu] for _ in range(T)]).astype(np.int32)
    x = O.normal(T * (1 if shared else nu) * K, 63).reshape(T, 1 if shared else nu, K)
    y = run_mul_mat_id(dev, st, dtype, w, K, M, E, x, ids)
    check_grouped(y, O.mul_mat_id(dtype, w, K, M, E, x, ids))


@pytest.mark.parametrize("case", ["tiles64", "skewed", "clamped", "q8_0_ktail", "one_expert_one_slot", "w12_bn32", "w12_bn64"])
def test_mul_mat_id_grouped_cases(hip, case):
    """64-pair tiles (>= 16 pairs per expert); a skewed routing (most pairs on one expert, most
    experts empty); out-of-range ids (clamped on the device); a K that ends inside a stage."""
    dev, st = hip
    dtype, K, M, E, T, nu = sg.Q4_K, 512, 256, 4, 64, 2
    rng = np.random.default_rng(71)
    if case == "tiles64":
        E = 2
        ids = np.stack([rng.permutation(E)[:nu] for _ in range(T)]).astype(np.int32)
    elif case == "skewed":
        E, T, nu = 32, 96, 2
        ids = np.where(rng.random((T, nu)) < 0.8, 5, rng.integers(0, 3, (T, nu))).astype(np.int32)
        ids[:, 1] = np.where(ids[:, 0] == ids[:, 1], 31, ids[:, 1])
    elif case == "clamped":
        E, T, nu = 6, 24, 3
        ids = rng.integers(-4, E + 4, (T, nu)).astype(np.int32)
    elif case == "q8_0_ktail":
        dtype, K, E, T, nu = sg.Q8_0, 544, 5, 20, 3
        ids = np.stack([rng.permutation(E)[:nu] for _ in range(T)]).astype(np.int32)
    elif case == "one_expert_one_slot":
        E, T, nu = 1, 70, 1
        ids = np.zeros((T, nu), np.int32)
    else:
        # 128 experts of 384 rows: one 12-wave work-group per (expert, token tile); 4 pairs per
        # expert on average (32-pair tiles) or 16 (64-pair tiles)
        M, E, nu = 384, 128, 8
        T = 64 if case == "w12_bn32" else 256
        ids = np.stack([rng.permutation(E)[:nu] for _ in range(T)]).astype(np.int32)
    w = O.quantize(dtype, O.normal(K * M * E, 72, 0.0, 0.02))
    x = O.normal(T * K, 73).reshape(T, 1, K)
    y = run_mul_mat_id(dev, st, dtype, w, K, M, E, x, ids)
    check_grouped(y, O.mul_mat_id(dtype, w, K, M, E, x, np.clip(ids, 0, E - 1)))


@pytest.mark.parametrize("dtype", sg.QTYPES, ids=lambda d: sg.NAMES[d])
@pytest.mark.parametrize("shared", [True, False], ids=["x_shared", "x_per_slot"])
def test_mul_mat_id_grouped_wide(hip, dtype, shared):
    """The grouped MUL_MAT_ID on the wide GEMM's 384-row x 64-token tiles (12 waves, 16 pairs per
    expert on average, K a whole number of 128-element stages): 392 rows (a last row tile of 8),
    tiles of up to 32 pairs that skip their second token fragment. The form is pinned."""
    dev, st = hip
    K, M, E, T, nu = 512, 392, 64, 128, 8
    w = O.quantize(dtype, O.normal(K * M * E, 81, 0.0, 0.02))
    rng = np.random.default_rng(82)
    ids = np.stack([rng.permutation(E)[:nu] for _ in range(T)]).astype(np.int32)
    x = O.normal(T * (1 if shared else nu) * K, 83).reshape(T, 1 if shared else nu, K)
    y = run_mul_mat_id(dev, st, dtype, w, K, M, E, x, ids)
    if dev.info().compute_units == 256:
        assert sg.last_launch()[0] == "grouped wide w=12 bn=64", sg.last_launch()
    check_grouped(y, O.mul_mat_id(dtype, w, K, M, E, x, ids))


def test_mul_mat_id_grouped_plan_reads_ids_on_device(hip):
    """A recorded plan (HIP graph) of a grouped MUL_MAT_ID replayed after the ids changed in device
    memory: the routing runs on the device each replay."""
    dev, st = hip
    dtype, K, M, E, T, nu = sg.Q4_K, 256, 128, 8, 32, 2
    w = O.quantize(dtype, O.normal(K * M * E, 81, 0.0, 0.02))
    wb, wt = upload_weights(dev, st, dtype, w, K, M, slices=E)
    x = O.normal(T * K, 82).reshape(T, 1, K)
    xb = dev.alloc(x.nbytes)
    xt = sg.tdesc(sg.F32, (K, 1, T), xb)
    st.upload(xt, x)
    ib = dev.alloc(4 * nu * T)
    it = sg.tdesc(sg.I32, (nu, T), ib)
    yb = dev.alloc(4 * M * nu * T)
    yt = sg.tdesc(sg.F32, (M, nu, T), yb)
    op, keep = sg.mul_mat_id_op(wt, xt, it, yt, nu)
    nodes = (sg.PlanNode * 1)(sg.PlanNode(C.sizeof(sg.PlanNode), op, 0))
    pdesc = sg.PlanDesc(C.sizeof(sg.PlanDesc), nodes, 1)
    plan = C.c_void_p()
    sg.check(sg.lib().scrapgpu_plan_build(dev.handle, C.byref(pdesc), C.byref(plan)), "plan_build")
    rng = np.random.default_rng(83)
    try:
        for _ in range(3):
            ids = np.stack([rng.permutation(E)[:nu] for _ in range(T)]).astype(np.int32)
            st.upload(it, ids)
            sg.check(sg.lib().scrapgpu_plan_execute(st.handle, plan), "plan_execute")
            st.sync()
            y = st.download(yt).reshape(T, nu, M)
            check_grouped(y, O.mul_mat_id(dtype, w, K, M, E, x, ids))
    finally:
        sg.check(sg.lib().scrapgpu_plan_free(plan), "plan_free")
    for b in (wb, xb, ib, yb):
        b.free()


def test_mul_mat_id_plan_fuses_gate_up(hip):
    """A plan of a MoE layer's gate and up (same x and ids: one launch) and down (other x): every
    output against the oracle, on graph replays with new ids and in eager plan mode (profiler on),
    where the fused pair counts as one launch."""
    dev, st = hip
    E, nu, T, H, F = 8, 2, 1, 512, 256
    rng = np.random.default_rng(91)
    specs = [("gate", sg.Q4_K, H, F), ("up", sg.Q4_K, H, F), ("down", sg.Q6_K, F, H)]
    ws, bufs, descs = {}, [], {}
    for i, (name, dt, K, M) in enumerate(specs):
        w = O.quantize(dt, O.normal(K * M * E, 92 + i, 0.0, 0.02))
        b, t = upload_weights(dev, st, dt, w, K, M, slices=E)
        ws[name] = w
        descs[name] = t
        bufs.append(b)
    xh = O.normal(T * H, 95).reshape(T, 1, H)
    xf = O.normal(T * nu * F, 96).reshape(T, nu, F)
    xhb, xfb = dev.alloc(xh.nbytes), dev.alloc(xf.nbytes)
    xht, xft = sg.tdesc(sg.F32, (H, 1, T), xhb), sg.tdesc(sg.F32, (F, nu, T), xfb)
    st.upload(xht, xh)
    st.upload(xft, xf)
    ib = dev.alloc(4 * nu * T)
    it = sg.tdesc(sg.I32, (nu, T), ib)
    ybs = {name: dev.alloc(4 * M * nu * T) for name, _, _, M in specs}
    yts = {name: sg.tdesc(sg.F32, (M, nu, T), ybs[name]) for name, _, _, M in specs}
    ops = [sg.mul_mat_id_op(descs[name], xft if name == "down" else xht, it, yts[name], nu) for name, *_ in specs]
    nodes = (sg.PlanNode * 3)(*[sg.PlanNode(C.sizeof(sg.PlanNode), op, 0) for op, _ in ops])
    pdesc = sg.PlanDesc(C.sizeof(sg.PlanDesc), nodes, 3)
    plan = C.c_void_p()
    sg.check(sg.lib().scrapgpu_plan_build(dev.handle, C.byref(pdesc), C.byref(plan)), "plan_build")
    try:
        for rep in range(4):
            ids = np.stack([rng.permutation(E)[:nu] for _ in range(T)]).astype(np.int32)
            st.upload(it, ids)
            eager = rep == 3
            if eager:
                sg.lib().scrapgpu_hip_profile_reset()
                sg.lib().scrapgpu_hip_profile_enable(1)
            sg.check(sg.lib().scrapgpu_plan_execute(st.handle, plan), "plan_execute")
            st.sync()
            if eager:
                sg.lib().scrapgpu_hip_profile_enable(0)
                rows = sg.profile_table()
                assert sum(r["launches"] for r in rows) == 2, rows
            for name, dt, K, M in specs:
                x = xf if name == "down" else xh
                y = st.download(yts[name]).reshape(T, nu, M)
                deq = O.dequantize(dt, ws[name], K * M * E).reshape(E, M, K)
                check_pairs(y, O.mul_mat_id(dt, ws[name], K, M, E, x, ids), x, deq, ids)
    finally:
        sg.check(sg.lib().scrapgpu_plan_free(plan), "plan_free")
    for b in bufs + list(ybs.values()) + [xhb, xfb, ib]:
        b.free()


@pytest.mark.parametrize("form", ["tiled", "wide"])
def test_mul_mat_id_grouped_plan_shares_routing(hip, form):
    """A plan of a MoE layer at prefill size: down (its own x), then gate and up (the same x and
    ids): up runs its GEMM on gate's x pre-pass and routing (the form says shared-x). On graph
    replays with new ids, each output bit for bit equal to the op run alone and within the
    prefill tolerance of the oracle. tiled: 4-wave 32-pair tiles with the Q4_K single-fma x form;
    wide: the wide GEMM's 384-row x 64-pair tiles."""
    dev, st = hip
    if form == "tiled":
        E, nu, T, H, F = 16, 4, 40, 512, 256
    else:
        E, nu, T, H, F = 64, 8, 128, 512, 512
    rng = np.random.default_rng(97)
    specs = [("down", sg.Q6_K, F, H), ("gate", sg.Q4_K, H, F), ("up", sg.Q4_K, H, F)]
    ws, bufs, descs = {}, [], {}
    for i, (name, dt, K, M) in enumerate(specs):
        w = O.quantize(dt, O.normal(K * M * E, 98 + i, 0.0, 0.02))
        b, t = upload_weights(dev, st, dt, w, K, M, slices=E)
        ws[name] = w
        descs[name] = t
        bufs.append(b)
    xh = O.normal(T * H, 101).reshape(T, 1, H)
    xf = O.normal(T * nu * F, 102).reshape(T, nu, F)
    xhb, xfb = dev.alloc(xh.nbytes), dev.alloc(xf.nbytes)
    xht, xft = sg.tdesc(sg.F32, (H, 1, T), xhb), sg.tdesc(sg.F32, (F, nu, T), xfb)
    st.upload(xht, xh)
    st.upload(xft, xf)
    ib = dev.alloc(4 * nu * T)
    it = sg.tdesc(sg.I32, (nu, T), ib)
    ybs = {name: dev.alloc(4 * M * nu * T) for name, _, _, M in specs}
    yts = {name: sg.tdesc(sg.F32, (M, nu, T), ybs[name]) for name, _, _, M in specs}
    ops = [sg.mul_mat_id_op(descs[name], xft if name == "down" else xht, it, yts[name], nu) for name, *_ in specs]
    nodes = (sg.PlanNode * 3)(*[sg.PlanNode(C.sizeof(sg.PlanNode), op, 0) for op, _ in ops])
    pdesc = sg.PlanDesc(C.sizeof(sg.PlanDesc), nodes, 3)
    plan = C.c_void_p()
    sg.check(sg.lib().scrapgpu_plan_build(dev.handle, C.byref(pdesc), C.byref(plan)), "plan_build")
    try:
        for rep in range(3):
            ids = np.stack([rng.permutation(E)[:nu] for _ in range(T)]).astype(np.int32)
            st.upload(it, ids)
            eager = rep == 2
            if eager:  # (the profiler runs a plan eagerly: the last launch's form is readable)
                sg.lib().scrapgpu_hip_profile_reset()
                sg.lib().scrapgpu_hip_profile_enable(1)
            sg.check(sg.lib().scrapgpu_plan_execute(st.handle, plan), "plan_execute")
            st.sync()
            if eager:
                sg.lib().scrapgpu_hip_profile_enable(0)
                assert sg.last_launch()[0].endswith("shared-x"), sg.last_launch()
            got = {name: st.download(yts[name]).reshape(T, nu, M).copy() for name, _, _, M in specs}
            for (op, _), (name, dt, K, M) in zip(ops, specs):
                st.execute(op)
                st.sync()
                alone = st.download(yts[name]).reshape(T, nu, M)
                assert np.array_equal(got[name].view(np.uint32), alone.view(np.uint32)), f"rep {rep} {name}: plan and op differ"
                x = xf if name == "down" else xh
                check_grouped(got[name], O.mul_mat_id(dt, ws[name], K, M, E, x, ids))
    finally:
        sg.check(sg.lib().scrapgpu_plan_free(plan), "plan_free")
    for b in bufs + list(ybs.values()) + [xhb, xfb, ib]:
        b.free()


def test_mul_mat_id_decode_20_steps(hip):
    """A decode MUL_MAT_ID with K of 20 steps: the pairs keep 16 waves of 2 steps (the instances
    that read the expert id ahead of x), where a plain MUL_MAT of that K takes 10 waves."""
    dev, st = hip
    dtype, K, M, E, T, nu = sg.Q4_K, 5120, 96, 6, 1, 3
    w = O.quantize(dtype, O.normal(K * M * E, 111, 0.0, 0.02))
    rng = np.random.default_rng(112)
    ids = np.stack([rng.permutation(E)[:nu] for _ in range(T)]).astype(np.int32)
    x = O.normal(T * nu * K, 113).reshape(T, nu, K)
    y = run_mul_mat_id(dev, st, dtype, w, K, M, E, x, ids)
    assert sg.last_launch()[0] == "burst rg=1 W=16 spw=2", sg.last_launch()
    deq = O.dequantize(dtype, w, K * M * E).reshape(E, M, K)
    check_pairs(y, O.mul_mat_id(dtype, w, K, M, E, x, ids), x, deq, ids)
