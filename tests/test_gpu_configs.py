"""GPU parity at BASELINE.json's five workloads, at their real shapes, through the C-ABI.

Each product runs exactly as the benchmark (or a caller) runs it -- R32 upload, MUL_MAT or
MUL_MAT_MULTI, the kernel form the shape selects -- and every output row is compared with the CPU
oracle (the reference's MUL_MAT restated, src/core/ref/ops.cpp:891-984) on the same quantized bytes
and the same x, with the gates of the reference's GPU suite (tests/ops/ops_tests.cpp:702-727):
decode (N <= 8) NMSE <= 1e-7 and max-abs <= 1e-4 * ||x||_2 * max|w|; prefill NMSE <= 5e-5.

Weights: N(0, 0.02) drawn on the device (scrapgpu_hip_fill_normal), copied to the host and
quantized there by the oracle (the reference quantizer restated; its bytes are pinned by the
golden vectors), then uploaded as R32 natural bytes like any caller's. x ~ N(0, 1) (numpy).
Each test asserts the kernel form the shape selects (scrapgpu_hip_last_launch), so a change of
the selection rules cannot silently move a workload off the kernel it was tested on.
"""
import os

import numpy as np
import pytest

import oracle as O
import scrapgpulibrary_amd as sg
from tests.gpu_util import check_matvec, nmse, upload_weights

pytestmark = pytest.mark.gpu

THREADS = min(16, os.cpu_count() or 1)
_cache = {}


def weights(hip, dtype, K, M, seed):
    """(natural quantized bytes, R32 buffer, R32 desc) of an M x K weight ~ N(0, 0.02); cached."""
    key = (dtype, K, M, seed)
    if key not in _cache:
        dev, st = hip
        fb = dev.alloc(4 * K * M)
        ft = sg.tdesc(sg.F32, (K, M), fb)
        st.fill_normal(ft, seed=seed, mean=0.0, std=0.02)
        w = st.download(ft)
        fb.free()
        q = O.quantize(dtype, w, threads=THREADS)
        del w
        buf, t = upload_weights(dev, st, dtype, q, K, M)
        _cache[key] = (q, buf, t)
    return _cache[key]


@pytest.fixture(scope="module", autouse=True)
def _free_cache(hip):
    yield
    for _, buf, _ in _cache.values():
        buf.free()
    _cache.clear()


def run(hip, wts, x, multi=False):
    """Runs W x for the R32 weight descs `wts` (one MUL_MAT each, or one MUL_MAT_MULTI); returns
    ([y [N, M] per weight], (form, grid) of the last launch)."""
    dev, st = hip
    N, K = x.shape
    xb = dev.alloc(x.nbytes)
    xt = sg.tdesc(sg.F32, (K, N), xb)
    st.upload(xt, x)
    ybs = [dev.alloc(4 * t.ne[1] * N) for t in wts]
    yts = [sg.tdesc(sg.F32, (t.ne[1], N), b) for t, b in zip(wts, ybs)]
    if multi:
        op, keep = sg.multi_op(wts, xt, yts)
        st.execute(op)
        form = sg.last_launch()
    else:
        for wt, yt in zip(wts, yts):
            op, keep = sg.mul_mat_op(wt, xt, yt)
            st.execute(op)
            form = sg.last_launch()
    st.sync()
    ys = [st.download(yt).reshape(N, yt.ne[0]).copy() for yt in yts]
    for b in ybs + [xb]:
        b.free()
    return ys, form


def check(dtype, q, K, M, x, y, what):
    ref = O.mul_mat(dtype, q, K, M, x, threads=THREADS)
    if x.shape[0] <= 8:
        deq_max = float(np.max(np.abs(O.dequantize(dtype, q, K * M))))
        e = check_matvec(y, ref, x, np.array([deq_max]))
    else:
        e = nmse(y, ref)
        assert e <= 5e-5, f"{what}: NMSE {e:.3e}"
    print(f"{what}: NMSE {e:.3e}", flush=True)
    return e


def cus(hip):
    return hip[0].info().compute_units


def test_config1_q4_0_4096(hip):
    """examples/standalone_matmul.c -- Q4_0 W 4096 x 4096 ~ N(0, 0.02) in R32, x [1, 4096]."""
    K = M = 4096
    q, _, wt = weights(hip, sg.Q4_0, K, M, 0)
    x = O.normal(K, 0).reshape(1, K)
    (y,), (form, grid) = run(hip, [wt], x)
    assert form.startswith("burst"), form
    check(sg.Q4_0, q, K, M, x, y, f"Q4_0 {M}x{K} N=1 [{form}]")


@pytest.mark.parametrize("N", [1, 4, 8])
@pytest.mark.parametrize("K,M", [(4096, 11008), (11008, 4096)], ids=["up_gate", "down"])
def test_config2_q8_0_llama_mlp(hip, K, M, N):
    """Q8_0 decode at Llama-7B MLP shapes (11008 x 4096 and 4096 x 11008), batch 1, 4, 8."""
    q, _, wt = weights(hip, sg.Q8_0, K, M, 10 + K)
    x = O.normal(N * K, 20 + N).reshape(N, K)
    (y,), (form, grid) = run(hip, [wt], x)
    assert form.startswith("burst" if N == 1 else "columns"), form
    check(sg.Q8_0, q, K, M, x, y, f"Q8_0 {M}x{K} N={N} [{form}]")


QWEN = [("q", sg.Q4_K, 4096, 4096), ("k", sg.Q4_K, 4096, 1024), ("v", sg.Q4_K, 4096, 1024), ("o", sg.Q4_K, 4096, 4096),
        ("gate", sg.Q4_K, 4096, 12288), ("up", sg.Q4_K, 4096, 12288), ("down", sg.Q6_K, 12288, 4096)]


@pytest.mark.parametrize("group", [("q", "k", "v"), ("o",), ("gate", "up"), ("down",), ("gate",)],
                         ids=["qkv_multi", "o", "gate_up_multi", "down_q6_k", "gate"])
def test_config3_qwen3_8b_decode_layer(hip, group):
    """configs[2], the metric's workload: one Qwen3-8B Q4_K_M decode layer's products at bs = 1,
    launched as the benchmark launches them (q/k/v and gate/up as one MUL_MAT_MULTI each). The
    fused gate+up (24576 rows) selects the 48-row burst tiles, whose 16-row groups straddle R32
    groups -- the benchmark's roofline kernel."""
    spec = {n: (dt, K, M) for n, dt, K, M in QWEN}
    ws = [weights(hip, *spec[n], 300 + i) for i, n in enumerate(group)]
    K = spec[group[0]][1]
    x = O.normal(K, 31).reshape(1, K)
    ys, (form, grid) = run(hip, [w[2] for w in ws], x, multi=len(group) > 1)
    rows = sum(spec[n][2] for n in group)
    if group == ("gate", "up"):
        want = "burst rg=3" if rows >= 96 * cus(hip) else "burst rg=2" if rows >= 64 * cus(hip) else "burst rg=1"
        assert form.startswith(want), form
        assert grid == sum((spec[n][2] + 47) // 48 for n in group), (form, grid)
    else:
        assert form.startswith("burst"), form
    for n, (q, _, _), y in zip(group, ws, ys):
        dt, K, M = spec[n]
        check(dt, q, K, M, x, y, f"{n} {sg.NAMES[dt]} {M}x{K} N=1 [{form}]")


@pytest.mark.parametrize("dtype", [sg.Q4_0, sg.Q4_K], ids=["q4_0", "q4_k"])
@pytest.mark.parametrize("rg", [2, 3])
def test_burst_multi_row_tiles_ragged(hip, dtype, rg):
    """The 32- and 48-row burst tiles (N = 1, K = 4096) on a row count that is neither a multiple
    of the tile nor of the R32 group (the last group holds 8 rows), alone and as a 2-weight
    MUL_MAT_MULTI whose first weight ends inside a tile."""
    K = 4096
    M = (32 if rg == 2 else 48) * cus(hip) + 40  # rows * 1 slice >= 32 rg CUs, last R32 group of 8 rows
    q, _, wt = weights(hip, dtype, K, M, 400 + rg)
    x = O.normal(K, 41).reshape(1, K)
    # alone and as MULTI the row count per CU selects the tile height (32 rows from 24 per CU, 48 from 96)
    (y,), (form, grid) = run(hip, [wt], x)
    assert form.startswith("burst"), form
    check(dtype, q, K, M, x, y, f"{sg.NAMES[dtype]} {M}x{K} [{form}]")
    M2 = M + 24
    q2, _, wt2 = weights(hip, dtype, K, M2, 500 + rg)
    ys, (form, grid) = run(hip, [wt, wt2], x, multi=True)
    assert form.startswith(f"burst rg={rg}"), form
    assert grid == (M + 16 * rg - 1) // (16 * rg) + (M2 + 16 * rg - 1) // (16 * rg), (form, grid)
    check(dtype, q, K, M, x, ys[0], f"multi[0] {sg.NAMES[dtype]} {M}x{K} [{form}]")
    check(dtype, q2, K, M2, x, ys[1], f"multi[1] {sg.NAMES[dtype]} {M2}x{K} [{form}]")


@pytest.mark.parametrize("N", [64, 128, 512, 2048])
@pytest.mark.parametrize("K,M", [(4096, 12288), (12288, 4096)], ids=["12288x4096", "4096x12288"])
def test_config4_q4_k_prefill(hip, K, M, N):
    """Q4_K prefill, W 12288 x 4096 and 4096 x 12288, x [N, K] for N in {64, 128, 512, 2048}."""
    q, _, wt = weights(hip, sg.Q4_K, K, M, 600 + K)
    x = O.normal(N * K, 60 + N).reshape(N, K)
    (y,), (form, grid) = run(hip, [wt], x)
    assert form.startswith("gemm"), form
    if M == 4096 and N == 2048 and hip[0].info().compute_units == 256:
        assert form.startswith("gemm wide w=8 kg=1 bn=128 rg=1 split=1"), form  # (256 256-row tiles, one per CU)
    if M == 4096 and N == 512 and hip[0].info().compute_units == 256:
        assert form.startswith("gemm wide w=8 kg=1 bn=128 rg=1 split=4"), form  # (64 256-row tiles x 4 splits of K)
    check(sg.Q4_K, q, K, M, x, y, f"Q4_K {M}x{K} N={N} [{form}]")


@pytest.mark.parametrize("N", [1, 8, 64])
def test_config5_q6_k_lm_head(hip, N):
    """the Q6_K LM head, W 151936 x 4096, at batch 1, 8 and 64 (batch 1: 16-row tiles
    of 4 waves of 4 steps, the form for 16 or more tiles per CU)."""
    K, M = 4096, 151936
    q, _, wt = weights(hip, sg.Q6_K, K, M, 700)
    x = O.normal(N * K, 70 + N).reshape(N, K)
    (y,), (form, grid) = run(hip, [wt], x)
    assert form.startswith("burst" if N == 1 else "columns" if N <= 8 else "gemm"), form
    if N == 1 and cus(hip) == 256:
        assert form == "burst rg=1 W=4 spw=4", form
    check(sg.Q6_K, q, K, M, x, y, f"Q6_K {M}x{K} N={N} [{form}]")


def test_config5_q4_k_70b_mlp(hip):
    """the 70B-class Q4_K MLP matrix, W 28672 x 8192, at batch 1 (32 steps of K: two
    chunks of 16 steps on 48-row tiles, 16-row ones below 96 rows per CU)."""
    K, M = 8192, 28672
    q, _, wt = weights(hip, sg.Q4_K, K, M, 800)
    x = O.normal(K, 80).reshape(1, K)
    (y,), (form, grid) = run(hip, [wt], x)
    rg = 3 if M >= 96 * cus(hip) else 1
    assert form.startswith(f"burst-chunks rg={rg} W=8 spw=2 chunks=2"), form
    check(sg.Q4_K, q, K, M, x, y, f"Q4_K {M}x{K} N=1 [{form}]")
