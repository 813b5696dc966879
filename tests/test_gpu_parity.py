"""GPU parity of the hip backend against the CPU oracle, through the C-ABI only.

Covers the drop-in path end to end: R32 upload (device-side pack) and download, bit-exact
dequantization and quantization on the device, the decode matvec (N = 1..8) and the MFMA prefill
(N > 8) for Q4_0 / Q8_0 / Q4_K / Q6_K, ragged rows, slices / broadcast, strides, MUL_MAT_MULTI and
plans. The reference shapes of tests/ops/ops_tests.cpp:702-778 are included.
"""
import ctypes as C
import os

import numpy as np
import pytest

import oracle as O
import scrapgpulibrary_amd as sg
from tests.gpu_util import check_matvec, nmse, quantized, run_mul_mat, upload_weights

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(__file__), "golden", "quant_mulmat_r32.npz")


def test_device_info(hip):
    dev, st = hip
    info = dev.info()
    assert info.backend_name == b"hip"
    assert info.warp_or_wave_width == 64
    assert info.compute_units >= 1
    assert b"gfx950" in info.generation_reason


@pytest.mark.parametrize("dtype", sg.QTYPES, ids=lambda d: sg.NAMES[d])
@pytest.mark.parametrize("M,slices", [(1, 1), (40, 1), (72, 3), (100, 2)])
def test_r32_device_layout_matches_reference_pack(hip, dtype, M, slices):
    """Device bytes after an R32 upload == the oracle's (reference-pinned) pack; download == input."""
    dev, st = hip
    K = 2 * sg.BLOCK[dtype]
    nat = np.random.default_rng(M * 7 + dtype).integers(0, 256, O.row_bytes(dtype, K) * M * slices, dtype=np.uint8)
    buf, t = upload_weights(dev, st, dtype, nat, K, M, slices)
    raw = st.read(buf, 0, nat.nbytes)
    assert np.array_equal(raw, O.r32_pack(dtype, K, M, slices, nat))
    assert np.array_equal(st.download(t, np.uint8), nat)
    buf.free()


@pytest.mark.parametrize("dtype", sg.QTYPES, ids=lambda d: sg.NAMES[d])
def test_r32_partial_upload_keeps_tail(hip, dtype):
    """A partial upload (first `size` natural bytes) leaves the rest of the tensor intact."""
    dev, st = hip
    K, M = sg.BLOCK[dtype] * 2, 70
    rb = O.row_bytes(dtype, K)
    rng = np.random.default_rng(3)
    a = rng.integers(0, 256, rb * M, dtype=np.uint8)
    b = rng.integers(0, 256, rb * M, dtype=np.uint8)
    buf, t = upload_weights(dev, st, dtype, a, K, M)
    cut = rb * 33 + 5  # inside the second row group
    st.upload(t, b, size=cut)
    got = st.download(t, np.uint8)
    assert np.array_equal(got[:cut], b[:cut])
    assert np.array_equal(got[cut:], a[cut:])
    buf.free()


@pytest.mark.parametrize("dtype", sg.QTYPES, ids=lambda d: sg.NAMES[d])
@pytest.mark.parametrize("layout", [sg.NATURAL, sg.R32], ids=["natural", "r32"])
def test_dequantize_bit_exact(hip, dtype, layout):
    dev, st = hip
    g = np.load(GOLD)
    name = sg.NAMES[dtype]
    for key in ("quant", "raw"):
        q = g[f"{name}_{key}_q"]
        want = g[f"{name}_{key}_y"]
        K = sg.BLOCK[dtype]
        M = want.size // K
        buf, t = upload_weights(dev, st, dtype, q, K, M, layout=layout)
        fb = dev.alloc(want.nbytes)
        ft = sg.tdesc(sg.F32, (K, M), fb)
        st.dequantize(t, ft)
        got = st.download(ft)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"{key}: dequantization differs"
        buf.free()
        fb.free()
    # a larger tensor: oracle dequantization of N(0, 0.02) weights
    K, M = 4 * sg.BLOCK[dtype] * 4, 77
    q, _ = quantized(dtype, K, M, 11)
    buf, t = upload_weights(dev, st, dtype, q, K, M, layout=layout)
    fb = dev.alloc(4 * K * M)
    ft = sg.tdesc(sg.F32, (K, M), fb)
    st.dequantize(t, ft)
    assert np.array_equal(st.download(ft).view(np.uint32), O.dequantize(dtype, q, K * M).view(np.uint32))
    buf.free()
    fb.free()


@pytest.mark.parametrize("dtype", sg.QTYPES, ids=lambda d: sg.NAMES[d])
@pytest.mark.parametrize("layout", [sg.NATURAL, sg.R32], ids=["natural", "r32"])
def test_quantize_matches_reference_bytes(hip, dtype, layout):
    dev, st = hip
    g = np.load(GOLD)
    name = sg.NAMES[dtype]
    cases = [g[f"{name}_quant_x"]]
    K = 4 * sg.BLOCK[dtype]
    cases.append(O.normal(K * 33, 5, 0.0, 0.02))
    cases.append(O.normal(K * 33, 6, 0.0, 1.0))
    for x in cases:
        M = x.size // K if x.size % K == 0 else x.size // sg.BLOCK[dtype]
        KK = x.size // M
        want = O.quantize(dtype, x)
        fb = dev.alloc(x.nbytes)
        ft = sg.tdesc(sg.F32, (KK, M), fb)
        st.upload(ft, x)
        qb = dev.alloc(want.nbytes)
        qt = sg.tdesc(dtype, (KK, M), qb, layout=layout)
        st.quantize(ft, qt)
        got = st.download(qt, np.uint8)
        assert np.array_equal(got, want), f"quantized bytes differ ({np.count_nonzero(got != want)} bytes)"
        fb.free()
        qb.free()


@pytest.mark.parametrize("dtype", sg.QTYPES, ids=lambda d: sg.NAMES[d])
def test_golden_mul_mat(hip, dtype):
    """The reference's own MUL_MAT outputs (scrapgpu_ref_execute, committed fixtures)."""
    dev, st = hip
    g = np.load(GOLD)
    name = sg.NAMES[dtype]
    K = 256 if sg.BLOCK[dtype] == 256 else 96
    for M, N in ((24, 1), (24, 4), (37, 7), (37, 17)):
        pre = f"{name}_mm_K{K}_M{M}_N{N}"
        w, x, want = g[pre + "_w"], g[pre + "_x"], g[pre + "_y"]
        y = run_mul_mat(dev, st, dtype, w, K, M, x)
        deq = O.dequantize(dtype, w, K * M)
        if N <= 8:
            check_matvec(y, want, x, deq)
        else:
            assert nmse(y, want) <= 5e-5


@pytest.mark.parametrize("dtype", sg.QTYPES, ids=lambda d: sg.NAMES[d])
@pytest.mark.parametrize("N", [1, 2, 3, 4, 5, 6, 7, 8])
def test_matvec_decode(hip, dtype, N):
    dev, st = hip
    for K, M in ((4096, 96), (sg.BLOCK[dtype] * 3, 37), (2048, 1000)):
        q, deq = quantized(dtype, K, M, 100 + N)
        x = O.normal(N * K, 200 + N).reshape(N, K)
        y = run_mul_mat(dev, st, dtype, q, K, M, x)
        ref = O.mul_mat(dtype, q, K, M, x, threads=8)
        check_matvec(y, ref, x, deq)


@pytest.mark.parametrize("dtype", sg.QTYPES, ids=lambda d: sg.NAMES[d])
@pytest.mark.parametrize("K", [8448, 12288])
def test_matvec_decode_three_steps_per_wave(hip, dtype, K):
    """N = 1 with 33..48 steps of K (the Q6_K down projection's K = 12288): 16 waves of 3 steps;
    K = 8448 (33 steps) leaves the last waves 2."""
    dev, st = hip
    M = 200
    q, deq = quantized(dtype, K, M, 900 + K % 97)
    x = O.normal(K, 901).reshape(1, K)
    y = run_mul_mat(dev, st, dtype, q, K, M, x)
    ref = O.mul_mat(dtype, q, K, M, x, threads=8)
    check_matvec(y, ref, x, deq)


@pytest.mark.parametrize("dtype,K,rpc", [(sg.Q4_0, 12288, 64), (sg.Q4_K, 12288, 64), (sg.Q6_K, 11008, 64), (sg.Q8_0, 4352, 64),
                                         (sg.Q4_0, 8192, 96), (sg.Q4_K, 12288, 96), (sg.Q6_K, 8192, 96)],
                         ids=["q4_0", "q4_k", "q6_k_partial_chunk", "q8_0_one_step_chunk", "q4_0_48_row_tiles", "q4_k_48_row_tiles",
                              "q6_k_many_rows"])
def test_matvec_decode_long_k_chunks(hip, dtype, K, rpc):
    """N = 1 with K past 16 steps and 4 row tiles per CU: K in chunks of 16 steps over 8-wave
    work-groups of 16 rows (48 rows for Q4_0 / Q4_K from 96 rows per CU), the
    chunks' partial sums added by the last chunk of each row tile to arrive, which resets its
    count. Three launches in a row (the counts must be back at zero after each), each against the
    oracle and bit for bit equal to the first; K = 11008 ends in a chunk of 11 steps, K = 4352 in
    a chunk of one step; the row count leaves a partial last tile and a last R32 group of 8 rows.
    The launch shape is pinned."""
    dev, st = hip
    M = rpc * dev.info().compute_units + 40 # 4 (or 6) row tiles per CU (where chunks start), a partial last one
    rg = 3 if rpc >= 96 and dtype in (sg.Q4_0, sg.Q4_K) else 1
    q0, d0 = quantized(dtype, K, 96, 950)   # 96 rows, repeated (rows are independent)
    reps = -(-M // 96)
    q, deq = np.tile(q0, reps)[: M * (q0.size // 96)], np.tile(d0, (reps, 1))[:M]
    x = O.normal(K, 951).reshape(1, K)
    ref = O.mul_mat(dtype, q, K, M, x, threads=8)
    first = None
    for _ in range(3):
        y = run_mul_mat(dev, st, dtype, q, K, M, x)
        form, grid = sg.last_launch()
        nck = -(-(K // 256) // 16)
        assert form == f"burst-chunks rg={rg} W=8 spw=2 chunks={nck}" and grid == -(-M // (16 * rg)) * nck, (form, grid)
        check_matvec(y, ref, x, deq)
        if first is None:
            first = y
        assert np.array_equal(y.view(np.uint32), first.view(np.uint32))


def test_matvec_decode_long_k_chunks_multi(hip):
    """The chunked burst on 48-row tiles over a MUL_MAT_MULTI of two Q4_K weights (K = 8192, 32
    steps: 2 chunks) whose first weight ends inside a tile: each weight against the oracle, on two
    launches in a row."""
    dev, st = hip
    cus = dev.info().compute_units
    K, Ms = 8192, (48 * cus + 20, 48 * cus + 8)
    x = O.normal(K, 960).reshape(1, K)
    xb = dev.alloc(x.nbytes)
    xt = sg.tdesc(sg.F32, (K, 1), xb)
    st.upload(xt, x)
    bufs, wts, yts, refs = [xb], [], [], []
    for i, M in enumerate(Ms):
        q0, d0 = quantized(sg.Q4_K, K, 96, 961 + i)
        reps = -(-M // 96)
        q, deq = np.tile(q0, reps)[: M * (q0.size // 96)], np.tile(d0, (reps, 1))[:M]
        wb, wt = upload_weights(dev, st, sg.Q4_K, q, K, M)
        yb = dev.alloc(4 * M)
        bufs += [wb, yb]
        wts.append(wt)
        yts.append(sg.tdesc(sg.F32, (M, 1), yb))
        refs.append((O.mul_mat(sg.Q4_K, q, K, M, x, threads=8), deq))
    op, keep = sg.multi_op(wts, xt, yts)
    for _ in range(2):
        st.execute(op)
        st.sync()
        form, grid = sg.last_launch()
        assert form == "burst-chunks rg=3 W=8 spw=2 chunks=2" and grid == sum(-(-M // 48) for M in Ms) * 2, (form, grid)
        for yt, (ref, deq) in zip(yts, refs):
            check_matvec(st.download(yt).reshape(1, -1), ref, x, deq)
    for b in bufs:
        b.free()


@pytest.mark.parametrize("dtype,K,want", [(sg.Q4_0, 12288, "burst rg=1 W=12 spw=4"), (sg.Q4_K, 12288, "burst rg=1 W=12 spw=4"),
                                          (sg.Q4_0, 11264, "burst rg=1 W=11 spw=4"), (sg.Q4_K, 10240, "burst rg=1 W=10 spw=4"),
                                          (sg.Q6_K, 8448, "burst rg=1 W=9 spw=4"), (sg.Q8_0, 11264, "burst rg=1 W=15 spw=3"),
                                          (sg.Q8_0, 12288, "burst rg=1 W=16 spw=3"), (sg.Q8_0, 8448, "burst rg=1 W=11 spw=3"),
                                          (sg.Q4_0, 10016, "burst rg=1 W=10 spw=4"), (sg.Q8_0, 9248, "burst rg=1 W=13 spw=3")],
                         ids=["q4_0_48", "q4_k_48", "q4_0_44", "q4_k_40", "q6_k_33", "q8_0_44", "q8_0_48", "q8_0_33", "q4_0_ragged_40",
                              "q8_0_ragged_37"])
def test_matvec_decode_long_k_slices(hip, dtype, K, want):
    """N = 1 over 2 slices with K of 33..48 steps: ceil(steps / 4) waves of 4 steps (Q8_0:
    ceil(steps / 3) waves of 3; the last wave's loads past K discarded); no chunks (one slice
    only), 16-row tiles (the launch must show the form)."""
    dev, st = hip
    M, S = 320, 2
    q0, d0 = quantized(dtype, K, M, 952)
    q1, d1 = quantized(dtype, K, M, 953)
    wb, wt = upload_weights(dev, st, dtype, np.concatenate([q0, q1]), K, M, slices=S)
    x = O.normal(S * K, 954).reshape(S, 1, K)
    xb, yb = dev.alloc(x.nbytes), dev.alloc(4 * M * S)
    xt = sg.tdesc(sg.F32, (K, 1, S), xb)
    yt = sg.tdesc(sg.F32, (M, 1, S), yb)
    st.upload(xt, x)
    op, keep = sg.mul_mat_op(wt, xt, yt)
    st.execute(op)
    st.sync()
    form, grid = sg.last_launch()
    assert form == want and grid == M // 16 * S, (form, grid)
    y = st.download(yt).reshape(S, M)
    for sl, (q, deq) in enumerate(((q0, d0), (q1, d1))):
        check_matvec(y[sl:sl + 1], O.mul_mat(dtype, q, K, M, x[sl], threads=8), x[sl], deq)
    for b in (wb, xb, yb):
        b.free()


@pytest.mark.parametrize("dtype,K,M,want", [(sg.Q4_K, 3072, 320, "burst rg=1 W=6 spw=2"), (sg.Q8_0, 4352, 320, "burst rg=1 W=10 spw=2"),
                                            (sg.Q4_0, 5120, 320, "burst rg=1 W=10 spw=2"), (sg.Q6_K, 6144, 320, "burst rg=1 W=12 spw=2"),
                                            (sg.Q4_K, 7168, 6144, "burst rg=2 W=14 spw=2"), (sg.Q4_0, 5120, 13824, "burst rg=2 W=10 spw=2")],
                         ids=["q4_k_12", "q8_0_17", "q4_0_20", "q6_k_24", "q4_k_28_rg2", "q4_0_20_rg2"])
def test_matvec_decode_even_wave_counts(hip, dtype, K, M, want):
    """N = 1 with 9..32 steps of K: an even number of waves of 2 steps, the fewest that cover K
    (6, 10, 12, 14: not a power of two; the last wave's loads past K discarded), on 16- and 32-row
    tiles (the launch must show the form; from 64 rows per CU these K take the chunked form)."""
    dev, st = hip
    q, deq = quantized(dtype, K, M, 960 + K % 97)
    x = O.normal(K, 961).reshape(1, K)
    wb, wt = upload_weights(dev, st, dtype, q, K, M)
    xb, yb = dev.alloc(x.nbytes), dev.alloc(4 * M)
    xt, yt = sg.tdesc(sg.F32, (K, 1), xb), sg.tdesc(sg.F32, (M, 1), yb)
    st.upload(xt, x)
    op, keep = sg.mul_mat_op(wt, xt, yt)
    st.execute(op)
    st.sync()
    if dev.info().compute_units == 256:
        assert sg.last_launch()[0] == want, sg.last_launch()
    check_matvec(st.download(yt).reshape(1, M), O.mul_mat(dtype, q, K, M, x, threads=8), x, deq)
    for b in (wb, xb, yb):
        b.free()


@pytest.mark.parametrize("dtype", sg.QTYPES, ids=lambda d: sg.NAMES[d])
def test_matvec_k_split_repeated(hip, dtype):
    """Few row groups + long K (N = 2, 64 steps): the streaming matvec, whose waves split K and
    add their partial sums in LDS in wave order; three runs, each against the oracle."""
    dev, st = hip
    K, M, N = 16384, 64, 2
    q, deq = quantized(dtype, K, M, 7)
    x = O.normal(N * K, 8).reshape(N, K)
    ref = O.mul_mat(dtype, q, K, M, x, threads=8)
    for _ in range(3):
        y = run_mul_mat(dev, st, dtype, q, K, M, x)
        check_matvec(y, ref, x, deq)


@pytest.mark.parametrize("dtype", sg.QTYPES, ids=lambda d: sg.NAMES[d])
@pytest.mark.parametrize("N", [9, 16, 64, 130])
def test_prefill_mfma(hip, dtype, N):
    dev, st = hip
    K, M = 1024, 200
    q, _ = quantized(dtype, K, M, 300 + N)
    x = O.normal(N * K, 400 + N).reshape(N, K)
    y = run_mul_mat(dev, st, dtype, q, K, M, x)
    ref = O.mul_mat(dtype, q, K, M, x, threads=8)
    e = nmse(y, ref)
    assert e <= 5e-5, f"NMSE {e:.3e}"


@pytest.mark.parametrize("dtype,M,N,K", [(sg.Q4_0, 1536, 4096, 512), (sg.Q8_0, 1536, 4096, 544), (sg.Q4_K, 1536, 4096, 512),
                                         (sg.Q6_K, 1536, 4096, 512), (sg.Q4_K, 3500, 6592, 256)],
                         ids=["q4_0", "q8_0_ktail", "q4_k", "q6_k", "q4_k_partial_rows"])
def test_prefill_one_workgroup_per_cu(hip, dtype, M, N, K):
    """Shapes whose 384-row x 64-token tiles fill the CUs in whole rounds (or in many rounds):
    the matmul runs one 12-wave work-group per CU. Q8_0 with K = 544 ends in a partial stage;
    M = 3500 ends in a partial row tile."""
    dev, st = hip
    q, _ = quantized(dtype, K, M, 500 + M)
    x = O.normal(N * K, 501).reshape(N, K)
    y = run_mul_mat(dev, st, dtype, q, K, M, x)
    ref = O.mul_mat(dtype, q, K, M, x, threads=8)
    e = nmse(y, ref)
    assert e <= 5e-5, f"NMSE {e:.3e}"


@pytest.mark.parametrize("dtype,M,N,K", [(sg.Q4_K, 768, 4096, 2048), (sg.Q6_K, 384, 8192, 2048), (sg.Q4_0, 768, 4096, 2048),
                                         (sg.Q8_0, 768, 4096, 2016), (sg.Q4_K, 768, 4096, 2304), (sg.Q8_0, 768, 4096, 2080)],
                         ids=["q4_k_kgroups2", "q6_k_kgroups2", "q4_0_kgroups2", "q8_0_kgroups2_ktail", "q4_k_split", "q8_0_split_ktail"])
def test_prefill_workgroup_per_cu_few_tiles(hip, dtype, M, N, K):
    """Too few 384-row x 64-token tiles to fill the CUs (128). K = 2048 (16 stages): 2 K groups of
    6 row waves on 192-row tiles (256), added in LDS, on the wide GEMM's 64-token form. K = 2304 /
    2080 (18 / 17 stages, not two equal runs of whole groups of 4): K split in 2 over 12-wave
    work-groups (the wide GEMM's for K = 2304, the 64-token kernel's for the K tail), partials
    added in split order; Q8_0 with K = 2080 splits 17 stages into 8 + 9, the
    last one partial (K = 2016: 16 stages on the 64-token kernel's 2 K groups, the last one
    partial). The form is pinned on a 256-CU part."""
    dev, st = hip
    q, _ = quantized(dtype, K, M, 700 + M)
    x = O.normal(N * K, 701).reshape(N, K)
    y = run_mul_mat(dev, st, dtype, q, K, M, x)
    if dev.info().compute_units == 256:
        want = ("gemm wide w=12 kg=2 bn=64" if K == 2048 else "gemm w=12 kg=2 bn=64" if K == 2016
                else "gemm wide w=12 kg=1 bn=64 rg=1 split=2" if K == 2304 else "gemm w=12 kg=1 bn=64 rg=1 split=2")
        assert sg.last_launch()[0].startswith(want), sg.last_launch()
    ref = O.mul_mat(dtype, q, K, M, x, threads=8)
    e = nmse(y, ref)
    assert e <= 5e-5, f"NMSE {e:.3e}"


@pytest.mark.parametrize("dtype,M,N,K", [(sg.Q4_0, 512, 4096, 3072), (sg.Q4_K, 512, 4096, 3072), (sg.Q6_K, 512, 4096, 3072),
                                         (sg.Q8_0, 200, 8192, 3040), (sg.Q4_K, 512, 4096, 4096), (sg.Q6_K, 512, 4096, 4096),
                                         (sg.Q8_0, 512, 4096, 4064)],
                         ids=["q4_0", "q4_k", "q6_k", "q8_0_partial_rows_ktail", "q4_k_uneven", "q6_k_uneven", "q8_0_uneven_ktail"])
def test_prefill_k_groups(hip, dtype, M, N, K):
    """Shapes whose 128-row tiles fill the CUs: one 12-wave work-group per CU, 3 K groups added in
    LDS in group order (the wide GEMM's 64-token form where K is a whole number of 128-element
    stages, the 64-token kernel otherwise). K = 3072 splits into 3 equal runs; K = 4096 (32 stages)
    into 12 + 12 + 8 with 4 inactive stages in the last group. Q8_0 with K = 3040 / 4064 ends in a
    partial stage and M = 200 in a partial row tile. The form is pinned on a 256-CU part."""
    dev, st = hip
    q, _ = quantized(dtype, K, M, 600 + M)
    x = O.normal(N * K, 601).reshape(N, K)
    y = run_mul_mat(dev, st, dtype, q, K, M, x)
    if dev.info().compute_units == 256:
        want = "gemm wide w=12 kg=3 bn=64" if K % 128 == 0 else "gemm w=12 kg=3 bn=64"
        assert sg.last_launch()[0].startswith(want), sg.last_launch()
    ref = O.mul_mat(dtype, q, K, M, x, threads=8)
    e = nmse(y, ref)
    assert e <= 5e-5, f"NMSE {e:.3e}"


@pytest.mark.parametrize("K,M,N", [(2560, 200, 64), (2816, 200, 64), (1024, 1536, 4096), (3072, 512, 4096)])
def test_prefill_q4k_large_scales_and_split_groups(hip, K, M, N):
    """Q4_K prefill with rows whose sub-block scales (weights in the hundreds) or offsets (means
    near -3000) are beyond the single-fma form, mixed with ordinary rows; K = 20 or 22 stages, so
    the split-K halves start inside a group of 4 stages and K = 2816 ends in half a group; the
    1536 x 4096 shape runs on 12-wave work-groups. Every row set meets the NMSE bound on its own."""
    dev, st = hip
    w = O.normal(K * M, 77, 0.0, 0.02).reshape(M, K)
    w[0:10] *= 1e4                    # scales d * sc well above 32
    w[20:30] += -3000.0               # offsets 32 * dmin * m well above 32768
    w[40:45, :256] *= 1e4             # one large block in an ordinary row
    w[46:50, :32] *= 1e4              # one large sub-block: the row's two lanes disagree
    q = O.quantize(sg.Q4_K, w.reshape(-1))
    x = O.normal(N * K, 78).reshape(N, K)
    y = run_mul_mat(dev, st, sg.Q4_K, q, K, M, x)
    ref = O.mul_mat(sg.Q4_K, q, K, M, x, threads=8)
    assert np.all(np.isfinite(y))
    for rows in (slice(0, 10), slice(20, 30), slice(40, 45), slice(46, 50), slice(50, M)):
        e = nmse(y[:, rows], ref[:, rows])
        assert e <= 5e-5, f"rows {rows}: NMSE {e:.3e}"


@pytest.mark.parametrize("M,K,S,form", [(768, 256, 4, "gemm wide w=12 kg=1 bn=64"), (256, 3072, 4, "gemm wide w=12 kg=3 bn=64"), (768, 256, 8, "gemm wide w=12 kg=1 bn=128")],
                         ids=["one_k_group", "three_k_groups", "wide"])
def test_prefill_workgroup_per_cu_slices_broadcast_strides(hip, M, K, S, form):
    """The 12-wave prefill kernels over S x slices with 2 weight slices (broadcast r2 = S / 2) and
    padded x / y column strides, all on the wide GEMM: 384-row x 64-token tiles (M = 768, 4
    slices), its 64-token form's 3 K groups (K = 3072), and 384-row x 128-token tiles (8 slices), each filling the CUs
    with S slices x 2048 tokens (on a 256-CU part)."""
    dev, st = hip
    dtype, N = sg.Q4_K, 2048
    q0, _ = quantized(dtype, K, M, 11)
    q1, _ = quantized(dtype, K, M, 12)
    wb, wt = upload_weights(dev, st, dtype, np.concatenate([q0, q1]), K, M, slices=2)
    xs1, ys1 = K + 8, M + 4
    x = O.normal(S * N * xs1, 13).reshape(S, N, xs1)
    xb = dev.alloc(x.nbytes)
    xt = sg.tdesc(sg.F32, (K, N, S), xb, nb=[4, 4 * xs1, 4 * xs1 * N, 4 * xs1 * N * S])
    st.write(xb, 0, x)
    yb = dev.alloc(4 * ys1 * N * S)
    st.write(yb, 0, np.full(ys1 * N * S, -7.0, np.float32))
    yt = sg.tdesc(sg.F32, (M, N, S), yb, nb=[4, 4 * ys1, 4 * ys1 * N, 4 * ys1 * N * S])
    op, keep = sg.mul_mat_op(wt, xt, yt, allow_broadcast=1)
    st.execute(op)
    st.sync()
    if dev.info().compute_units == 256:
        assert sg.last_launch()[0].startswith(form), sg.last_launch()
    y = st.read(yb, 0, 4 * ys1 * N * S).view(np.float32).reshape(S, N, ys1)
    for s in range(S):
        ref = O.mul_mat(dtype, q0 if s // (S // 2) == 0 else q1, K, M, x[s, :, :K].copy(), threads=8)
        e = nmse(y[s, :, :M], ref)
        assert e <= 5e-5, f"slice {s}: NMSE {e:.3e}"
        assert np.all(y[s, :, M:] == -7.0), "padding of dst was written"
    for b in (wb, xb, yb):
        b.free()


def wide_tokens(dev, row_tiles, pad=0):
    """Tokens at which `row_tiles` 384-row x 128-token tiles fill the device's CUs in one round
    (less `pad`: a part-empty last token tile)."""
    cus = dev.info().compute_units
    assert (cus * 128) % row_tiles == 0, cus
    return cus * 128 // row_tiles - pad


@pytest.mark.parametrize("dtype,M,pad", [(sg.Q4_0, 3072, 0), (sg.Q8_0, 3072, 40), (sg.Q4_K, 3072, 0), (sg.Q6_K, 3072, 0),
                                         (sg.Q4_K, 6000, 40)],
                         ids=["q4_0", "q8_0_token_tail", "q4_k", "q6_k", "q4_k_row_tail"])
def test_prefill_wide_tiles(hip, dtype, M, pad):
    """The wide GEMM (384-row x 128-token tiles, one per CU, x tiles loaded straight into LDS,
    exact Q4_K dequantization): every dtype; a part-empty last token tile (tokens past N read the
    last token, outputs dropped); M = 6000 ends in a partial row tile. The launch form is pinned."""
    dev, st = hip
    K = 512
    N = wide_tokens(dev, (M + 383) // 384, pad)
    q, _ = quantized(dtype, K, M, 900 + M)
    x = O.normal(N * K, 901).reshape(N, K)
    wb, wt = upload_weights(dev, st, dtype, q, K, M)
    xb, yb = dev.alloc(x.nbytes), dev.alloc(4 * M * N)
    xt, yt = sg.tdesc(sg.F32, (K, N), xb), sg.tdesc(sg.F32, (M, N), yb)
    st.upload(xt, x)
    op, keep = sg.mul_mat_op(wt, xt, yt)
    st.execute(op)
    st.sync()
    form, grid = sg.last_launch()
    assert form.startswith("gemm wide w=12 kg=1"), form
    assert grid == (M + 383) // 384 * ((N + 127) // 128), (form, grid)
    y = st.download(yt).reshape(N, M)
    ref = O.mul_mat(dtype, q, K, M, x, threads=8)
    e = nmse(y, ref)
    assert e <= 5e-5, f"NMSE {e:.3e}"
    for b in (wb, xb, yb):
        b.free()


@pytest.mark.parametrize("dtype,K,pad", [(sg.Q4_K, 2048, 0), (sg.Q8_0, 2048, 0), (sg.Q4_0, 2048, 40), (sg.Q6_K, 4608, 0)],
                         ids=["q4_k", "q8_0", "q4_0_token_tail", "q6_k_uneven"])
def test_prefill_wide_k_groups(hip, dtype, K, pad):
    """The wide GEMM with 2 K groups of 6 row waves (192-row x 128-token tiles that fill the CUs
    where the 384-row ones do not): each group sums half of K, hands half of its token fragments'
    sums to the other group through LDS and stores the other half. K = 4608 (36 stages): groups
    of 20 stages, the second one's last 4 inactive."""
    dev, st = hip
    M = 3072
    N = wide_tokens(dev, M // 192, pad)
    q, _ = quantized(dtype, K, M, 930 + K)
    x = O.normal(N * K, 931).reshape(N, K)
    wb, wt = upload_weights(dev, st, dtype, q, K, M)
    xb, yb = dev.alloc(x.nbytes), dev.alloc(4 * M * N)
    xt, yt = sg.tdesc(sg.F32, (K, N), xb), sg.tdesc(sg.F32, (M, N), yb)
    st.upload(xt, x)
    op, keep = sg.mul_mat_op(wt, xt, yt)
    st.execute(op)
    st.sync()
    form, grid = sg.last_launch()
    assert form.startswith("gemm wide w=12 kg=2"), form
    assert grid == M // 192 * ((N + 127) // 128), (form, grid)
    y = st.download(yt).reshape(N, M)
    ref = O.mul_mat(dtype, q, K, M, x, threads=8)
    e = nmse(y, ref)
    assert e <= 5e-5, f"NMSE {e:.3e}"
    for b in (wb, xb, yb):
        b.free()


@pytest.mark.parametrize("dtype,N,extra", [(sg.Q6_K, 64, 0), (sg.Q8_0, 40, 0), (sg.Q4_K, 64, 100), (sg.Q4_0, 16, 0)],
                         ids=["q6_k", "q8_0_token_tail", "q4_k_row_tail", "q4_0_16_tokens"])
def test_prefill_wide_64_tokens(hip, dtype, N, extra):
    """The wide GEMM with 64-token wave tiles (few tokens, rows enough for a 384-row tile per CU,
    as in an LM head): a part-empty token tile (N = 40, 16) and a partial last row tile."""
    dev, st = hip
    K = 256
    M = 384 * dev.info().compute_units + extra
    q, _ = quantized(dtype, K, M, 960 + N)
    x = O.normal(N * K, 961).reshape(N, K)
    y = run_mul_mat(dev, st, dtype, q, K, M, x)
    form, grid = sg.last_launch()
    assert form.startswith("gemm wide w=12 kg=1 bn=64"), form
    assert grid == (M + 383) // 384, (form, grid)
    ref = O.mul_mat(dtype, q, K, M, x, threads=8)
    e = nmse(y, ref)
    assert e <= 5e-5, f"NMSE {e:.3e}"


def test_prefill_wide_q4k_large_scales(hip):
    """The wide GEMM's exact Q4_K form on rows with scales (weights in the hundreds) and offsets
    (means near -3000) far beyond the ordinary ones, mixed with ordinary rows."""
    dev, st = hip
    K, M = 512, 3072
    N = wide_tokens(dev, 8)
    w = O.normal(K * M, 79, 0.0, 0.02).reshape(M, K)
    w[0:10] *= 1e4
    w[20:30] += -3000.0
    w[40:45, :256] *= 1e4
    q = O.quantize(sg.Q4_K, w.reshape(-1))
    x = O.normal(N * K, 80).reshape(N, K)
    y = run_mul_mat(dev, st, sg.Q4_K, q, K, M, x)
    assert sg.last_launch()[0].startswith("gemm wide")
    ref = O.mul_mat(sg.Q4_K, q, K, M, x, threads=8)
    assert np.all(np.isfinite(y))
    for rows in (slice(0, 10), slice(20, 30), slice(40, 45), slice(50, M)):
        e = nmse(y[:, rows], ref[:, rows])
        assert e <= 5e-5, f"rows {rows}: NMSE {e:.3e}"


def test_prefill_wide_multi_per_weight_tiles(hip):
    """A prefill MUL_MAT_MULTI on the wide GEMM whose first weights are not whole 32-row groups
    (1000 + 1000 + 1072 rows): each weight owns its own 384-row tiles, the last one of each
    partial."""
    dev, st = hip
    dtype, K, Ms = sg.Q4_K, 512, (1000, 1000, 1072)
    N = wide_tokens(dev, 8)
    x = O.normal(N * K, 940).reshape(N, K)
    xb = dev.alloc(x.nbytes)
    xt = sg.tdesc(sg.F32, (K, N), xb)
    st.upload(xt, x)
    bufs, wts, yts, refs = [], [], [], []
    for i, M in enumerate(Ms):
        q, _ = quantized(dtype, K, M, 941 + i)
        b, t = upload_weights(dev, st, dtype, q, K, M)
        yb = dev.alloc(4 * M * N)
        bufs += [b, yb]
        wts.append(t)
        yts.append(sg.tdesc(sg.F32, (M, N), yb))
        refs.append(O.mul_mat(dtype, q, K, M, x, threads=8))
    op, keep = sg.multi_op(wts, xt, yts)
    st.execute(op)
    st.sync()
    form, grid = sg.last_launch()
    assert form.startswith("gemm wide"), form
    assert grid == sum((M + 383) // 384 for M in Ms) * ((N + 127) // 128), (form, grid)
    for M, yt, ref in zip(Ms, yts, refs):
        e = nmse(st.download(yt).reshape(N, M), ref)
        assert e <= 5e-5, f"{M} rows: NMSE {e:.3e}"
    for b in bufs + [xb]:
        b.free()


def sk_tokens(dev, row_tiles, stages, pad=0, extra=0):
    """Tokens at which `row_tiles` 384-row x 128-token tiles are fewer than the CUs but hold at
    least 32 stages of K per CU (the wide GEMM's stream-K form), plus `extra` token tiles, less
    `pad`."""
    cus = dev.info().compute_units
    ntw = -(-32 * cus // (row_tiles * stages)) + extra
    assert row_tiles * ntw < cus, (row_tiles, ntw, cus)
    return 128 * ntw - pad


def _sk_run(dev, st, dtype, K, Ms, N, seed):
    x = O.normal(N * K, seed).reshape(N, K)
    xb = dev.alloc(x.nbytes)
    xt = sg.tdesc(sg.F32, (K, N), xb)
    st.upload(xt, x)
    bufs, wts, yts, refs = [xb], [], [], []
    for i, M in enumerate(Ms):
        q, _ = quantized(dtype, K, M, seed + 1 + i)
        b, t = upload_weights(dev, st, dtype, q, K, M)
        yb = dev.alloc(4 * M * N)
        st.write(yb, 0, np.full(M * N, np.nan, np.float32))
        bufs += [b, yb]
        wts.append(t)
        yts.append(sg.tdesc(sg.F32, (M, N), yb))
        refs.append(O.mul_mat(dtype, q, K, M, x, threads=8))
    op, keep = sg.multi_op(wts, xt, yts) if len(Ms) > 1 else sg.mul_mat_op(wts[0], xt, yts[0])
    ys = []
    for rep in range(2):  # (the second launch finds the first one's partial slots in the scratch)
        st.execute(op)
        st.sync()
        ys.append([st.download(yt).reshape(N, M).copy() for M, yt in zip(Ms, yts)])
    form, grid = sg.last_launch()
    for b in bufs:
        b.free()
    return ys, refs, form, grid


@pytest.mark.parametrize("dtype,K,Ms,N,split", [(sg.Q4_K, 2048, (3000,), 2504, 1), (sg.Q6_K, 8192, (4096,), 500, 4),
                                              (sg.Q8_0, 4096, (2048, 2048), 1000, 2), (sg.Q4_0, 2048, (1000, 1000, 1048), 2500, 1)],
                         ids=["q4_k_row_and_token_tails", "q6_k_k_split", "q8_0_multi_packed", "q4_0_multi_per_weight_tiles"])
def test_prefill_wide_256_row_tiles(hip, dtype, K, Ms, N, split):
    """The wide GEMM's 8-wave form: 256-row x 128-token tiles, one work-group per CU, K split over
    `split` work-groups where that fills the CUs in one round (15/16 of them or more). A part-empty
    last row tile and token tile, K split with the partials added by the split reduce, a
    MUL_MAT_MULTI packed end to end and one whose weights own their row tiles; two launches
    bit-identical, every output within the prefill NMSE of the oracle."""
    dev, st = hip
    ys, refs, form, grid = _sk_run(dev, st, dtype, K, Ms, N, 990 + N)
    if dev.info().compute_units == 256:
        assert form.startswith(f"gemm wide w=8 kg=1 bn=128 rg=1 split={split}"), form
    for M, a, b, ref in zip(Ms, ys[0], ys[1], refs):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"{M} rows: launches differ"
        e = nmse(a, ref)
        assert e <= 5e-5, f"{sg.NAMES[dtype]} {M}x{K} N={N}: NMSE {e:.3e} [{form}]"


@pytest.mark.parametrize("dtype,K,Ms,N", [(sg.Q4_0, 2048, (98688,), 33), (sg.Q6_K, 2048, (49000, 49688), 64)],
                         ids=["q4_0_257_tiles", "q6_k_multi_per_weight_tiles"])
def test_prefill_wide_stream_k_64_tokens(hip, dtype, K, Ms, N):
    """Stream-K on the wide GEMM's 64-token tiles: 257-258 tiles of 384 rows (a second round of
    tiles at most a quarter full), so the CUs share all tiles' 2-stage units instead and the tiles
    cut between CUs are added from their partial slots by the reduce pass; a part-empty token tile
    and a MUL_MAT_MULTI whose weights own their row tiles; two launches bit-identical."""
    dev, st = hip
    ys, refs, form, grid = _sk_run(dev, st, dtype, K, Ms, N, 1200 + N)
    if dev.info().compute_units == 256:
        assert form.startswith("gemm wide stream-k w=12 kg=1 bn=64"), form
    for M, a, b, ref in zip(Ms, ys[0], ys[1], refs):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"{M} rows: launches differ"
        e = nmse(a, ref)
        assert e <= 5e-5, f"{sg.NAMES[dtype]} {M}x{K} N={N}: NMSE {e:.3e} [{form}]"


@pytest.mark.parametrize("dtype,K,Ms,pad", [(sg.Q6_K, 12288, (3102,), 60), (sg.Q8_0, 8192, (3840,), 100),
                                            (sg.Q4_K, 8192, (1000, 1000, 1072), 100), (sg.Q4_0, 8192, (1024, 1024, 1024), 0)],
                         ids=["q6_k_row_tail_scalar_y", "q8_0_token_tail", "q4_k_multi_per_weight_tiles", "q4_0_multi_packed"])
def test_prefill_wide_stream_k(hip, dtype, K, Ms, pad):
    """The wide GEMM's stream-K form: fewer 384-row tiles than CUs, each CU an equal run of 2-stage
    units over all tiles (a tile shared by several CUs is added from its partial slots in CU order
    by a reduce pass). A row tail with rows not a multiple of 4 (the reduce's scalar stores), a
    part-empty token tile, a MUL_MAT_MULTI whose weights own their row tiles (more tiles than all
    rows together need) and one run end to end; two launches bit-identical."""
    dev, st = hip
    M = sum(Ms)
    # (3072 rows: one token tile more than the minimum, where 192-row tiles would fill the CUs)
    N = sk_tokens(dev, (M + 383) // 384, K // 128, pad, extra=1 if M == 3072 else 0)
    ys, refs, form, grid = _sk_run(dev, st, dtype, K, Ms, N, 960 + len(Ms))
    assert form.startswith("gemm wide stream-k"), form
    assert grid == dev.info().compute_units, (form, grid)
    for M, a, b, ref in zip(Ms, ys[0], ys[1], refs):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"{M} rows: launches differ"
        e = nmse(a, ref)
        assert e <= 5e-5, f"{sg.NAMES[dtype]} {M}x{K} N={N}: NMSE {e:.3e} [{form}]"


def test_prefill_wide_multi_tiles_across_weights(hip):
    """A prefill MUL_MAT_MULTI on the wide GEMM: 3 weights of 1024 rows (32-row multiples), the
    384-row tiles running across their boundaries, each wave taking the weight its rows are in."""
    dev, st = hip
    dtype, K, Ms = sg.Q6_K, 512, (1024, 1024, 1024)
    N = wide_tokens(dev, 8)
    x = O.normal(N * K, 910).reshape(N, K)
    xb = dev.alloc(x.nbytes)
    xt = sg.tdesc(sg.F32, (K, N), xb)
    st.upload(xt, x)
    bufs, wts, yts, refs = [], [], [], []
    for i, M in enumerate(Ms):
        q, _ = quantized(dtype, K, M, 920 + i)
        b, t = upload_weights(dev, st, dtype, q, K, M)
        yb = dev.alloc(4 * M * N)
        bufs += [b, yb]
        wts.append(t)
        yts.append(sg.tdesc(sg.F32, (M, N), yb))
        refs.append(O.mul_mat(dtype, q, K, M, x, threads=8))
    op, keep = sg.multi_op(wts, xt, yts)
    st.execute(op)
    st.sync()
    assert sg.last_launch()[0].startswith("gemm wide"), sg.last_launch()
    for M, yt, ref in zip(Ms, yts, refs):
        e = nmse(st.download(yt).reshape(N, M), ref)
        assert e <= 5e-5, f"{M} rows: NMSE {e:.3e}"
    for b in bufs + [xb]:
        b.free()


@pytest.mark.parametrize("dtype", [sg.Q4_0, sg.Q4_K], ids=lambda d: sg.NAMES[d])
@pytest.mark.parametrize("N", [1, 4, 33])
def test_slices_broadcast_and_strides(hip, dtype, N):
    """src0 with 2 slices broadcast over src1's 4 (r2 = 2); x and y with padded column strides."""
    dev, st = hip
    K, M = 2 * sg.BLOCK[dtype], 40
    w2 = 2
    q0, d0 = quantized(dtype, K, M, 1)
    q1, d1 = quantized(dtype, K, M, 2)
    wq = np.concatenate([q0, q1])
    wb, wt = upload_weights(dev, st, dtype, wq, K, M, slices=w2)
    S = 4
    xs1 = K + 8  # padded column stride (floats)
    ys1 = M + 5
    x = O.normal(S * N * xs1, 9).reshape(S, N, xs1)
    xb = dev.alloc(x.nbytes)
    xt = sg.tdesc(sg.F32, (K, N, S), xb, nb=[4, 4 * xs1, 4 * xs1 * N, 4 * xs1 * N * S])
    st.write(xb, 0, x)
    yb = dev.alloc(4 * ys1 * N * S)
    st.write(yb, 0, np.full(ys1 * N * S, -7.0, np.float32))
    yt = sg.tdesc(sg.F32, (M, N, S), yb, nb=[4, 4 * ys1, 4 * ys1 * N, 4 * ys1 * N * S])
    op, keep = sg.mul_mat_op(wt, xt, yt, allow_broadcast=1)
    st.execute(op)
    st.sync()
    y = st.read(yb, 0, 4 * ys1 * N * S).view(np.float32).reshape(S, N, ys1)
    for s in range(S):
        qs, ds = (q0, d0) if s // 2 == 0 else (q1, d1)
        ref = O.mul_mat(dtype, qs, K, M, x[s, :, :K].copy())
        if N <= 8:
            check_matvec(y[s, :, :M], ref, x[s, :, :K], ds)
        else:
            assert nmse(y[s, :, :M], ref) <= 5e-5
        assert np.all(y[s, :, M:] == -7.0), "padding of dst was written"
    # the same op without allow_broadcast is refused
    op0, keep0 = sg.mul_mat_op(wt, xt, yt, allow_broadcast=0)
    stt, reason = dev.supported(op0)
    assert stt == sg.UNSUPPORTED and "broadcast" in reason
    for b in (wb, xb, yb):
        b.free()


def test_support_rules(hip):
    dev, st = hip
    K, M = 256, 32
    wb = dev.alloc(O.row_bytes(sg.Q4_K, K) * M)
    xb, yb = dev.alloc(4 * K), dev.alloc(4 * M)
    x, y = sg.tdesc(sg.F32, (K, 1), xb), sg.tdesc(sg.F32, (M, 1), yb)
    natural = sg.tdesc(sg.Q4_K, (K, M), wb, layout=sg.NATURAL)
    op, keep = sg.mul_mat_op(natural, x, y)
    stt, reason = dev.supported(op)
    assert stt == sg.UNSUPPORTED and "R32" in reason
    f32w = sg.tdesc(sg.F32, (K, M), wb)
    op, keep = sg.mul_mat_op(f32w, x, y)
    assert dev.supported(op)[0] == sg.OK  # float weights run from the natural layout
    f32r = sg.tdesc(sg.F32, (K, M), wb, layout=sg.R32)
    op, keep = sg.mul_mat_op(f32r, x, y)
    stt, reason = dev.supported(op)
    assert stt == sg.UNSUPPORTED and "natural" in reason
    r32 = sg.tdesc(sg.Q4_K, (K, M), wb, layout=sg.R32)
    op, keep = sg.mul_mat_op(r32, x, y)
    assert dev.supported(op)[0] == sg.OK
    bad_y = sg.tdesc(sg.F32, (M + 1, 1), yb)
    op, keep = sg.mul_mat_op(r32, x, bad_y)
    assert dev.supported(op)[0] == sg.INVALID_ARGUMENT
    for b in (wb, xb, yb):
        b.free()


@pytest.mark.parametrize("n", [2, 3])
def test_mul_mat_multi(hip, n):
    """tests/ops/ops_tests.cpp:751-778: n Q4_0 weights sharing one x."""
    dev, st = hip
    K, M = 96, 8
    ws, wts, qs = [], [], []
    for i in range(n):
        q, _ = quantized(sg.Q4_0, K, M, 50 + i, std=0.5)
        b, t = upload_weights(dev, st, sg.Q4_0, q, K, M)
        ws.append(b)
        wts.append(t)
        qs.append(q)
    x = O.normal(K, 60).reshape(1, K)
    xb = dev.alloc(x.nbytes)
    xt = sg.tdesc(sg.F32, (K, 1), xb)
    st.upload(xt, x)
    ybs = [dev.alloc(4 * M) for _ in range(n)]
    yts = [sg.tdesc(sg.F32, (M, 1), b) for b in ybs]
    op, keep = sg.multi_op(wts, xt, yts)
    st.execute(op)
    st.sync()
    for i in range(n):
        ref = O.mul_mat(sg.Q4_0, qs[i], K, M, x)
        assert nmse(st.download(yts[i]).reshape(1, M), ref) <= 1e-6
    for b in ws + ybs + [xb]:
        b.free()


@pytest.mark.parametrize("dtype", sg.QTYPES, ids=lambda d: sg.NAMES[d])
@pytest.mark.parametrize("N", [1, 3, 8])
def test_mul_mat_multi_fused_qkv_shapes(hip, dtype, N):
    """One fused launch for 3 weights of different row counts sharing x (QKV-like: 96 / 32 / 40 rows)."""
    dev, st = hip
    K = 4 * sg.BLOCK[dtype] if sg.BLOCK[dtype] == 256 else 1024
    Ms = (96, 32, 40)
    bufs, wts, qs, deqs = [], [], [], []
    for i, M in enumerate(Ms):
        q, d = quantized(dtype, K, M, 500 + i)
        b, t = upload_weights(dev, st, dtype, q, K, M)
        bufs.append(b)
        wts.append(t)
        qs.append(q)
        deqs.append(d)
    x = O.normal(N * K, 510 + N).reshape(N, K)
    xb = dev.alloc(x.nbytes)
    xt = sg.tdesc(sg.F32, (K, N), xb)
    st.upload(xt, x)
    ybs = [dev.alloc(4 * M * N) for M in Ms]
    yts = [sg.tdesc(sg.F32, (M, N), b) for M, b in zip(Ms, ybs)]
    sg.lib().scrapgpu_hip_profile_reset()
    sg.lib().scrapgpu_hip_profile_enable(1)
    op, keep = sg.multi_op(wts, xt, yts)
    st.execute(op)
    st.sync()
    sg.lib().scrapgpu_hip_profile_enable(0)
    rows = sg.profile_table()
    assert [r["name"] for r in rows] == [f"matvec_multi_{sg.NAMES[dtype]}"] and rows[0]["launches"] == 1
    for i, M in enumerate(Ms):
        ref = O.mul_mat(dtype, qs[i], K, M, x)
        check_matvec(st.download(yts[i]).reshape(N, M), ref, x, deqs[i])
    for b in bufs + ybs + [xb]:
        b.free()


@pytest.mark.parametrize("specs", [[(sg.Q4_K, 384), (sg.Q4_K, 200), (sg.Q6_K, 96)], [(sg.Q6_K, 96), (sg.Q4_K, 200), (sg.Q4_K, 64)]],
                         ids=["share_then_convert", "convert_then_share"])
def test_mul_mat_multi_prefill_shares_x(hip, specs):
    """Prefill MUL_MAT_MULTI (N = 64): consecutive products that read the same x in the same form
    share one x pre-pass (Q4_K, Q4_K); a Q6_K product converts x in its own form, and a Q4_K after
    it converts again. Every output against the oracle."""
    dev, st = hip
    K, N = 512, 64
    x = O.normal(N * K, 530).reshape(N, K)
    xb = dev.alloc(x.nbytes)
    xt = sg.tdesc(sg.F32, (K, N), xb)
    st.upload(xt, x)
    bufs, wts, yts, refs = [], [], [], []
    for i, (dt, M) in enumerate(specs):
        q, _ = quantized(dt, K, M, 540 + i)
        b, t = upload_weights(dev, st, dt, q, K, M)
        yb = dev.alloc(4 * M * N)
        bufs += [b, yb]
        wts.append(t)
        yts.append(sg.tdesc(sg.F32, (M, N), yb))
        refs.append(O.mul_mat(dt, q, K, M, x, threads=8))
    op, keep = sg.multi_op(wts, xt, yts)
    st.execute(op)
    st.sync()
    for (dt, M), yt, ref in zip(specs, yts, refs):
        e = nmse(st.download(yt).reshape(N, M), ref)
        assert e <= 5e-5, f"{sg.NAMES[dt]} {M} rows: NMSE {e:.3e}"
    for b in bufs + [xb]:
        b.free()


@pytest.mark.parametrize("Ms,K,N", [((200, 64, 40), 1024, 64), ((256, 128, 98), 4096, 64), ((768, 768), 256, 4096),
                                    ((512, 128, 128), 2048, 4096), ((512, 128, 128), 2304, 4096)],
                         ids=["small", "split_k_odd_rows", "workgroup_per_cu", "tiles_across_weights_kgroups2",
                              "tiles_across_weights_split_k"])
def test_mul_mat_multi_prefill_one_launch(hip, Ms, K, N):
    """Prefill MUL_MAT_MULTI of one dtype: one GEMM launch over all the weights' row tiles (split-K
    partials over all their rows, scattered back per weight; 98 rows take the scalar reduce; two
    768-row weights at 4096 tokens run on 12-wave work-groups; 512 + 128 + 128 rows as 192-row tiles
    that cross the weights' boundaries, 2 K groups, or at K = 2304 as 384-row tiles with K split
    in 2). Every output against the oracle."""
    dev, st = hip
    dtype = sg.Q4_K
    x = O.normal(N * K, 550).reshape(N, K)
    xb = dev.alloc(x.nbytes)
    xt = sg.tdesc(sg.F32, (K, N), xb)
    st.upload(xt, x)
    bufs, wts, yts, refs = [], [], [], []
    for i, M in enumerate(Ms):
        q, _ = quantized(dtype, K, M, 560 + i)
        b, t = upload_weights(dev, st, dtype, q, K, M)
        yb = dev.alloc(4 * M * N)
        bufs += [b, yb]
        wts.append(t)
        yts.append(sg.tdesc(sg.F32, (M, N), yb))
        refs.append(O.mul_mat(dtype, q, K, M, x, threads=8))
    op, keep = sg.multi_op(wts, xt, yts)
    sg.lib().scrapgpu_hip_profile_reset()
    sg.lib().scrapgpu_hip_profile_enable(1)
    st.execute(op)
    st.sync()
    sg.lib().scrapgpu_hip_profile_enable(0)
    rows = sg.profile_table()
    assert [r["launches"] for r in rows] == [1], rows
    for M, yt, ref in zip(Ms, yts, refs):
        e = nmse(st.download(yt).reshape(N, M), ref)
        assert e <= 5e-5, f"{M} rows: NMSE {e:.3e}"
    for b in bufs + [xb]:
        b.free()


@pytest.mark.parametrize("N", [1, 64])
def test_plan_fuses_mul_mats_sharing_x(hip, N):
    """A plan of separate MUL_MATs q, k, v (same x) and o (another x): the three run as one
    MUL_MAT_MULTI launch; every output against the oracle, on a graph replay and in eager plan mode
    (profiler on: 2 launches for the 4 nodes)."""
    dev, st = hip
    K, dtype = 512, sg.Q4_K
    Ms = {"q": 256, "k": 64, "v": 64, "o": 256}
    x1 = O.normal(N * K, 570).reshape(N, K)
    x2 = O.normal(N * K, 571).reshape(N, K)
    bufs, descs, qs, yts = [], {}, {}, {}
    x1b, x2b = dev.alloc(x1.nbytes), dev.alloc(x2.nbytes)
    x1t, x2t = sg.tdesc(sg.F32, (K, N), x1b), sg.tdesc(sg.F32, (K, N), x2b)
    st.upload(x1t, x1)
    st.upload(x2t, x2)
    for i, (name, M) in enumerate(Ms.items()):
        q, _ = quantized(dtype, K, M, 580 + i)
        b, t = upload_weights(dev, st, dtype, q, K, M)
        yb = dev.alloc(4 * M * N)
        bufs += [b, yb]
        descs[name], qs[name] = t, q
        yts[name] = sg.tdesc(sg.F32, (M, N), yb)
    ops = [sg.mul_mat_op(descs[n], x2t if n == "o" else x1t, yts[n]) for n in Ms]
    nodes = (sg.PlanNode * 4)(*[sg.PlanNode(C.sizeof(sg.PlanNode), op, 0) for op, _ in ops])
    pdesc = sg.PlanDesc(C.sizeof(sg.PlanDesc), nodes, 4)
    plan = C.c_void_p()
    sg.check(sg.lib().scrapgpu_plan_build(dev.handle, C.byref(pdesc), C.byref(plan)), "plan_build")
    try:
        for eager in (False, True):
            if eager:
                sg.lib().scrapgpu_hip_profile_reset()
                sg.lib().scrapgpu_hip_profile_enable(1)
            sg.check(sg.lib().scrapgpu_plan_execute(st.handle, plan), "plan_execute")
            st.sync()
            if eager:
                sg.lib().scrapgpu_hip_profile_enable(0)
                assert sum(r["launches"] for r in sg.profile_table()) == 2
            for n, M in Ms.items():
                x = x2 if n == "o" else x1
                y = st.download(yts[n]).reshape(N, M)
                ref = O.mul_mat(dtype, qs[n], K, M, x)
                assert nmse(y, ref) <= (1e-7 if N == 1 else 5e-5), n
    finally:
        sg.check(sg.lib().scrapgpu_plan_free(plan), "plan_free")
    for b in bufs + [x1b, x2b]:
        b.free()


def test_mul_mat_multi_mixed_dtypes_falls_back(hip):
    """Weights of different dtypes share x: one launch per product, same results."""
    dev, st = hip
    K, M = 512, 64
    specs = [(sg.Q4_K, 0), (sg.Q6_K, 1)]
    bufs, wts, refs = [], [], []
    x = O.normal(2 * K, 520).reshape(2, K)
    for dt, i in specs:
        q, d = quantized(dt, K, M, 530 + i)
        b, t = upload_weights(dev, st, dt, q, K, M)
        bufs.append(b)
        wts.append(t)
        refs.append((O.mul_mat(dt, q, K, M, x), d))
    xb = dev.alloc(x.nbytes)
    xt = sg.tdesc(sg.F32, (K, 2), xb)
    st.upload(xt, x)
    ybs = [dev.alloc(4 * M * 2) for _ in specs]
    yts = [sg.tdesc(sg.F32, (M, 2), b) for b in ybs]
    op, keep = sg.multi_op(wts, xt, yts)
    st.execute(op)
    st.sync()
    for (ref, d), yt in zip(refs, yts):
        check_matvec(st.download(yt).reshape(2, M), ref, x, d)
    for b in bufs + ybs + [xb]:
        b.free()


def test_plan_and_buffer_lifetime(hip):
    dev, st = hip
    L = sg.lib()
    K, M = 512, 64
    q, deq = quantized(sg.Q6_K, K, M, 70)
    wb, wt = upload_weights(dev, st, sg.Q6_K, q, K, M)
    x = O.normal(2 * K, 71).reshape(2, K)
    xb = dev.alloc(x.nbytes)
    xt = sg.tdesc(sg.F32, (K, 2), xb)
    st.upload(xt, x)
    yb = dev.alloc(4 * M * 2)
    yt = sg.tdesc(sg.F32, (M, 2), yb)
    op, keep = sg.mul_mat_op(wt, xt, yt)
    node = sg.PlanNode(C.sizeof(sg.PlanNode), op, 0)
    nodes = (sg.PlanNode * 1)(node)
    pd = sg.PlanDesc(C.sizeof(sg.PlanDesc), nodes, 1)
    plan = C.c_void_p()
    sg.check(L.scrapgpu_plan_build(dev.handle, C.byref(pd), C.byref(plan)), "plan_build")
    assert L.scrapgpu_buffer_free(wb.handle) == sg.INVALID_ARGUMENT  # referenced by a live plan
    for _ in range(2):
        sg.check(L.scrapgpu_plan_execute(st.handle, plan), "plan_execute")
    st.sync()
    check_matvec(st.download(yt).reshape(2, M), O.mul_mat(sg.Q6_K, q, K, M, x), x, deq)
    sg.check(L.scrapgpu_plan_free(plan), "plan_free")
    for b in (wb, xb, yb):
        b.free()


def test_profiler_counts_launches(hip):
    dev, st = hip
    L = sg.lib()
    K, M = 1024, 256
    q, _ = quantized(sg.Q4_K, K, M, 90)
    L.scrapgpu_hip_profile_reset()
    L.scrapgpu_hip_profile_enable(1)
    try:
        x = O.normal(K, 91).reshape(1, K)
        run_mul_mat(dev, st, sg.Q4_K, q, K, M, x)
    finally:
        L.scrapgpu_hip_profile_enable(0)
    rows = {r["name"]: r for r in sg.profile_table()}
    assert rows["matvec_q4_k"]["launches"] == 1
    assert rows["matvec_q4_k"]["bytes"] == O.row_bytes(sg.Q4_K, K) * M


def _plan(dev, ops):
    L = sg.lib()
    nodes = (sg.PlanNode * len(ops))(*[sg.PlanNode(C.sizeof(sg.PlanNode), op, 0) for op in ops])
    pd = sg.PlanDesc(C.sizeof(sg.PlanDesc), nodes, len(ops))
    plan = C.c_void_p()
    sg.check(L.scrapgpu_plan_build(dev.handle, C.byref(pd), C.byref(plan)), "plan_build")
    return plan


def test_plan_graph_replays_match_eager(hip):
    """A plan is recorded once as a HIP graph and replayed: every replay, with new inputs written
    and other eager work between the replays, matches the oracle; growing the stream's scratch
    and switching streams re-record it."""
    dev, st = hip
    L = sg.lib()
    K = 1024
    specs = [(sg.Q4_K, 256, 1, 100), (sg.Q8_0, 96, 4, 101), (sg.Q6_K, 160, 64, 102), (sg.Q4_0, 128, 1, 103)]
    items = []
    for dtype, M, N, seed in specs:
        q, deq = quantized(dtype, K, M, seed)
        wb, wt = upload_weights(dev, st, dtype, q, K, M)
        xb = dev.alloc(4 * K * N)
        xt = sg.tdesc(sg.F32, (K, N), xb)
        yb = dev.alloc(4 * M * N)
        yt = sg.tdesc(sg.F32, (M, N), yb)
        op, keep = sg.mul_mat_op(wt, xt, yt)
        items.append(dict(dtype=dtype, M=M, N=N, q=q, deq=deq, bufs=(wb, xb, yb), xt=xt, yt=yt, op=op, keep=keep))
    plan = _plan(dev, [it["op"] for it in items])
    st2 = dev.stream()
    try:
        for rep in range(5):
            if rep == 3:  # a large eager prefill grows the scratch of `st`: the graph is re-recorded
                q, _ = quantized(sg.Q4_K, 2048, 128, 110)
                run_mul_mat(dev, st, sg.Q4_K, q, 2048, 128, O.normal(512 * 2048, 111).reshape(512, 2048))
            stream = st2 if rep == 4 else st
            xs = []
            for i, it in enumerate(items):
                x = O.normal(it["N"] * K, 1000 * rep + i).reshape(it["N"], K)
                st.upload(it["xt"], x)
                xs.append(x)
            st.sync()
            sg.check(L.scrapgpu_plan_execute(stream.handle, plan), "plan_execute")
            stream.sync()
            for it, x in zip(items, xs):
                y = st.download(it["yt"]).reshape(it["N"], it["M"])
                ref = O.mul_mat(it["dtype"], it["q"], K, it["M"], x)
                if it["N"] > 8:
                    assert nmse(y, ref) <= 5e-5, f"replay {rep} {it['dtype']}"
                else:
                    check_matvec(y, ref, x, it["deq"])
    finally:
        sg.check(L.scrapgpu_plan_free(plan), "plan_free")
        st2.free()
        for it in items:
            for b in it["bufs"]:
                b.free()
