"""CPU pins of the oracle (oracle/oracle.c) -- no GPU needed.

Each oracle function is checked against something that does not restate it:
  * golden vectors written by the reference's own code compiled from source (tests/golden/);
  * the known-answer blocks and bit patterns of the reference's tests
    (tests/ref/ref_quant_tests.cpp:23-105,179-223; tests/r32/r32_tests.cpp:104-181;
    tests/ref/ref_ops_tests.cpp:754-771);
  * numpy's IEEE binary16 conversion (exhaustive half -> float, every exponent for float -> half);
  * fp64 brute-force dot products and round-trip error bounds;
  * the output checksums of the reference's tools/cpu_bench.cpp on its deterministic inputs
    (measured by compiling the reference in the build container);
  * the reference compiled from source, live, when oracle/_ref exists (build container only).
"""
import os

import numpy as np
import pytest

import oracle as O

GOLD = os.path.join(os.path.dirname(__file__), "golden", "quant_mulmat_r32.npz")


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD)


# ---------------------------------------------------------------------------------------------
# golden vectors of the reference
# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("dt", O.QTYPES, ids=lambda d: O.NAMES[d])
def test_golden_quantize_dequantize(gold, dt):
    n = O.NAMES[dt]
    x, q, y = gold[f"{n}_quant_x"], gold[f"{n}_quant_q"], gold[f"{n}_quant_y"]
    assert np.array_equal(O.quantize(dt, x), q)
    assert np.array_equal(O.dequantize(dt, q, x.size).view(np.uint32), y.view(np.uint32))
    raw, ry = gold[f"{n}_raw_q"], gold[f"{n}_raw_y"]
    assert np.array_equal(O.dequantize(dt, raw, ry.size).view(np.uint32), ry.view(np.uint32))


@pytest.mark.parametrize("dt", O.QTYPES, ids=lambda d: O.NAMES[d])
def test_golden_mul_mat(gold, dt):
    n = O.NAMES[dt]
    K = 256 if O.BLOCK[dt] == 256 else 96
    for M, N in ((24, 1), (24, 4), (37, 7), (37, 17)):
        p = f"{n}_mm_K{K}_M{M}_N{N}"
        y = O.mul_mat(dt, gold[p + "_w"], K, M, gold[p + "_x"])
        assert np.array_equal(y.view(np.uint32), gold[p + "_y"].view(np.uint32)), p


@pytest.mark.parametrize("dt", O.QTYPES, ids=lambda d: O.NAMES[d])
def test_golden_r32(gold, dt):
    n = O.NAMES[dt]
    Kr, Mr, S = 2 * O.BLOCK[dt], 40, 2
    nat = gold[f"{n}_r32_K{Kr}_M{Mr}_S{S}_nat"]
    rep = gold[f"{n}_r32_K{Kr}_M{Mr}_S{S}_rep"]
    assert np.array_equal(O.r32_pack(dt, Kr, Mr, S, nat), rep)
    assert np.array_equal(O.r32_unpack(dt, Kr, Mr, S, rep), nat)


# golden MUL_MAT_ID / GET_ROWS of the reference, and the independent checks: a MUL_MAT_ID output
# is the N = 1 MUL_MAT of the selected expert (pinned above); a GET_ROWS row is the dequantized row

GOLD_ID = os.path.join(os.path.dirname(__file__), "golden", "mul_mat_id_get_rows.npz")


@pytest.fixture(scope="module")
def gold_id():
    return np.load(GOLD_ID)


@pytest.mark.parametrize("dt", O.QTYPES, ids=lambda d: O.NAMES[d])
def test_golden_mul_mat_id(gold_id, dt):
    n = O.NAMES[dt]
    K = 256 if O.BLOCK[dt] == 256 else 96
    M, E = 40, 5
    w, ids = gold_id[f"{n}_mid_w"], gold_id[f"{n}_mid_ids"]
    rb = O.row_bytes(dt, K) * M
    for n1 in (1, ids.shape[1]):
        x, y = gold_id[f"{n}_mid_x{n1}"], gold_id[f"{n}_mid_y{n1}"]
        got = O.mul_mat_id(dt, w, K, M, E, x, ids)
        assert np.array_equal(got.view(np.uint32), y.view(np.uint32))
        for t in range(ids.shape[0]):
            for i in range(ids.shape[1]):
                e = ids[t, i]
                one = O.mul_mat(dt, w[e * rb:(e + 1) * rb], K, M, x[t, i if n1 > 1 else 0])
                assert np.array_equal(one[0].view(np.uint32), got[t, i].view(np.uint32))


def test_mul_mat_id_expert_out_of_range():
    w = O.quantize(O.Q4_0, O.normal(96 * 8 * 3, 3, 0.0, 0.02))
    x = O.normal(2 * 96, 4).reshape(2, 1, 96)
    for bad in (3, -1):
        with pytest.raises(ValueError):
            O.mul_mat_id(O.Q4_0, w, 96, 8, 3, x, np.array([[0], [bad]], np.int32))


@pytest.mark.parametrize("dt", O.QTYPES, ids=lambda d: O.NAMES[d])
def test_golden_get_rows(gold_id, dt):
    n = O.NAMES[dt]
    K = 256 if O.BLOCK[dt] == 256 else 96
    R = 37
    w, ids, y = gold_id[f"{n}_gr_w"], gold_id[f"{n}_gr_ids"], gold_id[f"{n}_gr_y"]
    got = O.get_rows(dt, w, K, R, ids)
    assert np.array_equal(got.view(np.uint32), y.view(np.uint32))
    deq = O.dequantize(dt, w, K * R).reshape(R, K)
    assert np.array_equal(got.view(np.uint32), deq[ids].view(np.uint32))
    with pytest.raises(ValueError):
        O.get_rows(dt, w, K, R, np.array([R], np.int32))


# float weights (F32 / F16 / BF16): golden vectors of the reference, and independent checks: the
# conversion against numpy's (F16) and the exact high-half rule (BF16), the product against an fp64
# dot of the converted weights

GOLD_F = os.path.join(os.path.dirname(__file__), "golden", "float_weights.npz")


@pytest.fixture(scope="module")
def gold_f():
    return np.load(GOLD_F)


def _as_float(dt, w):
    if dt == O.F32:
        return np.asarray(w, np.float32)
    if dt == O.F16:
        return np.asarray(w, np.uint16).view(np.float16).astype(np.float32)
    return O.bf16_to_float(w)


@pytest.mark.parametrize("dt", O.FTYPES, ids=lambda d: O.NAMES[d])
def test_golden_float_mul_mat(gold_f, dt):
    n = O.NAMES[dt]
    K = 72
    for M, N in ((24, 1), (23, 3), (37, 7), (37, 17)):
        k = f"{n}_mm_K{K}_M{M}_N{N}"
        w, x, y = gold_f[k + "_w"], gold_f[k + "_x"], gold_f[k + "_y"]
        got = O.mul_mat(dt, w, K, M, x)
        assert np.array_equal(got.view(np.uint32), y.view(np.uint32)), k
        wf = _as_float(dt, w).reshape(M, K).astype(np.float64)
        ref = x.astype(np.float64) @ wf.T
        bound = 2.0 * K * 2.0 ** -24 * (np.abs(x).astype(np.float64) @ np.abs(wf).T) + 1e-30
        assert np.all(np.abs(got - ref) <= bound), k


def test_float_weights_conversion():
    """bf16: the high half of the f32 bits, rounding to nearest even with ties; f16 rows through the
    oracle's half_to_float equal numpy's float16."""
    v = np.array([1.0, -2.5, 1.00390625, 1.005859375, 3e-39, 65504.0, np.inf, -0.0], np.float32)
    b = O.float_to_bf16(v)
    assert b.tolist() == [0x3F80, 0xC020, 0x3F80, 0x3F81, 0x0021, 0x4780, 0x7F80, 0x8000]
    w = np.arange(-300, 300, dtype=np.float32) * 0.37
    hb = w.astype(np.float16).view(np.uint16)
    one = np.ones((1, w.size), np.float32)
    y = O.mul_mat(O.F16, hb, w.size, 1, one)
    # (the increasing-k float sum: cumsum adds in order, np.sum would pair)
    assert y[0, 0] == np.cumsum(w.astype(np.float16).astype(np.float32), dtype=np.float32)[-1]


def test_golden_float_mul_mat_id_get_rows(gold_f):
    K, M, E = 72, 40, 5
    w, ids, x, y = gold_f["f16_mid_w"], gold_f["f16_mid_ids"], gold_f["f16_mid_x"], gold_f["f16_mid_y"]
    got = O.mul_mat_id(O.F16, w, K, M, E, x, ids)
    assert np.array_equal(got.view(np.uint32), y.view(np.uint32))
    R = 37
    wr, rid, g = gold_f["f16_gr_w"], gold_f["f16_gr_ids"], gold_f["f16_gr_y"]
    got = O.get_rows(O.F16, wr, K, R, rid)
    assert np.array_equal(got.view(np.uint32), g.view(np.uint32))
    assert np.array_equal(got, wr.reshape(R, K).view(np.float16).astype(np.float32)[rid])


# ---------------------------------------------------------------------------------------------
# the reference's known-answer tests
# ---------------------------------------------------------------------------------------------

def test_kat_q4_0():
    blk = np.zeros(18, np.uint8)
    blk[1] = 0x3C  # d = 1.0
    blk[2:18] = np.arange(16)
    y = O.dequantize(O.Q4_0, blk, 32)
    assert np.array_equal(y[:16], np.arange(16) - 8.0)
    assert np.all(y[16:] == -8.0)


def test_kat_q8_0():
    blk = np.zeros(34, np.uint8)
    blk[1] = 0x38  # d = 0.5
    blk[2:34] = (np.arange(32) - 16).astype(np.int8).view(np.uint8)
    assert np.array_equal(O.dequantize(O.Q8_0, blk, 32), (np.arange(32) - 16) * 0.5)


def test_kat_q4_k():
    blk = np.zeros(144, np.uint8)
    blk[1] = 0x3C  # d = 1, dmin = 0
    blk[4:8] = 32
    l = np.arange(128)
    blk[16:] = (l & 15) | ((l & 15) << 4)
    y = O.dequantize(O.Q4_K, blk, 256)
    assert np.array_equal(y[:128], 32.0 * (np.arange(128) & 15))
    assert np.all(y[128:] == 0.0)


def test_kat_q6_k():
    blk = np.zeros(210, np.uint8)
    blk[209] = 0x3C  # d = 1.0 at 208
    blk[192:208] = 8
    for half in range(2):
        for l in range(64):
            i = half * 64 + l
            blk[i] = (i % 16) | (((i + 3) % 16) << 4)
    y = O.dequantize(O.Q6_K, blk, 256)
    for n0 in (0, 128):
        for l in range(32):
            assert y[n0 + l] == 8.0 * ((l % 16) - 32)
            assert y[n0 + l + 32] == 8.0 * (((l + 32) % 16) - 32)
            assert y[n0 + l + 64] == 8.0 * (((l + 3) % 16) - 32)
            assert y[n0 + l + 96] == 8.0 * (((l + 35) % 16) - 32)


def test_f16_reference_bit_patterns():
    # tests/ref/ref_quant_tests.cpp:179-223
    f = np.array([1.0, -2.0, 0.5, 65504.0, 65520.0, 65512.0, -0.0, 5.960464477539063e-08, 2.9802322387695312e-08,
                  8.940696716308594e-08], np.float32)
    want = np.array([0x3C00, 0xC000, 0x3800, 0x7BFF, 0x7C00, 0x7BFF, 0x8000, 0x0001, 0x0000, 0x0002], np.uint16)
    assert np.array_equal(O.float_to_half(f), want)


def test_half_to_float_exhaustive():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.half_to_float(h)
    want = h.view(np.float16).astype(np.float32)
    finite = np.isfinite(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(got[np.isinf(want)], want[np.isinf(want)])


def test_float_to_half_every_exponent():
    rng = np.random.default_rng(1)
    exps = np.arange(256, dtype=np.uint32)
    mant = rng.integers(0, 1 << 23, (256, 512), dtype=np.uint32)
    mant[:, 0] = 0
    mant[:, 1] = 0x7FFFFF
    mant[:, 2] = 0x001000  # ties at the normal rounding point
    mant[:, 3] = 0x003000
    bits = (exps[:, None] << 23) | mant
    bits = np.concatenate([bits.ravel(), bits.ravel() | 0x80000000])
    f = bits.view(np.float32)
    got = O.float_to_half(f)
    finite = np.isfinite(f)
    with np.errstate(over="ignore"):
        want = f[finite].astype(np.float16).view(np.uint16)
    assert np.array_equal(got[finite], want)
    nan = np.isnan(f)
    assert np.all((got[nan] & 0x7FFF) == 0x7E00)  # quiet NaN, sign kept (f16.cpp:44-47)


def test_quantize_round_trip_bounds():
    # tests/ref/ref_quant_tests.cpp:112-158: max error as a fraction of amax
    rng = np.random.default_rng(12345)
    for dt, nblk, bound in ((O.Q4_0, 7, 1 / 7), (O.Q8_0, 5, 1 / 200), (O.Q4_K, 3, 0.10), (O.Q6_K, 3, 0.02)):
        n = O.BLOCK[dt] * nblk
        x = (rng.uniform(-1, 1, n) * 3).astype(np.float32)
        if O.BLOCK[dt] == 256:
            x[:256] = -1.0 - 0.5 * np.abs(rng.uniform(-1, 1, 256))
        y = O.dequantize(dt, O.quantize(dt, x), n)
        assert np.max(np.abs(x.astype(np.float64) - y)) <= bound * np.max(np.abs(x))
    z = np.zeros(32, np.float32)
    assert np.all(O.dequantize(O.Q4_0, O.quantize(O.Q4_0, z), 32) == 0.0)


# ---------------------------------------------------------------------------------------------
# MUL_MAT
# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("N", [1, 4, 16, 17])
def test_mul_mat_increasing_k_order(N):
    # tests/ref/ref_ops_tests.cpp:754-771: only an increasing-K float sum gives exactly 7
    w = np.tile(np.array([1e20, 1.0, -1e20, 3.0, 4.0], np.float32), 5)
    x = np.ones((N, 5), np.float32)
    assert np.all(O.mul_mat(O.F32, w, 5, 5, x) == 7.0)


@pytest.mark.parametrize("dt", O.QTYPES, ids=lambda d: O.NAMES[d])
def test_mul_mat_vs_fp64(dt):
    K, M = 2 * O.BLOCK[dt] * 4, 19
    q = O.quantize(dt, O.normal(K * M, 3, 0.0, 0.02))
    w = O.dequantize(dt, q, K * M).reshape(M, K).astype(np.float64)
    for N in (1, 3, 4, 9, 16, 21):
        x = O.normal(N * K, 4 + N).reshape(N, K)
        y = O.mul_mat(dt, q, K, M, x).astype(np.float64)
        ref = x.astype(np.float64) @ w.T
        assert np.max(np.abs(y - ref)) <= 1e-5 * np.max(np.abs(ref)) + 1e-6


def test_mul_mat_panel_equals_scalar():
    # N >= 4 takes the K-major panel path, N < 4 the scalar one: same bits for the same column
    K, M = 512, 33
    q = O.quantize(O.Q4_K, O.normal(K * M, 5, 0.0, 0.02))
    x = O.normal(17 * K, 6).reshape(17, K)
    y17 = O.mul_mat(O.Q4_K, q, K, M, x)
    for n in range(17):
        y1 = O.mul_mat(O.Q4_K, q, K, M, x[n:n + 1])
        assert np.array_equal(y1[0].view(np.uint32), y17[n].view(np.uint32))


def test_mul_mat_threads_identical():
    K, M = 1024, 77
    q = O.quantize(O.Q6_K, O.normal(K * M, 7, 0.0, 0.02))
    x = O.normal(5 * K, 8).reshape(5, K)
    assert np.array_equal(O.mul_mat(O.Q6_K, q, K, M, x, threads=1), O.mul_mat(O.Q6_K, q, K, M, x, threads=7))


@pytest.mark.parametrize("dt", [16, 17, 32, 33])
def test_quantize_threads_identical(dt):
    """quantize(threads=n) splits x into runs of whole blocks: the same bytes as one call."""
    x = O.normal(256 * 4099, 41, 0.0, 0.5)
    assert np.array_equal(O.quantize(dt, x, threads=7), O.quantize(dt, x))


def test_mul_mat_broadcast_and_strides():
    """dst[i2] = W[i2 / r2] x[i2] with padded strides (ops.cpp:909-917, ref_ops_tests.cpp:659-753)."""
    K, M, N = 64, 5, 3
    w = O.quantize(O.Q4_0, O.normal(K * M * 2, 9, 0.0, 0.5))
    rb = O.row_bytes(O.Q4_0, K)
    wt = O.tensor(O.Q4_0, w, (K, M, 2, 1), (18, rb, rb * M, rb * M * 2))
    xs = K + 3
    x = O.normal(xs * N * 4, 10)
    xt = O.tensor(O.F32, x, (K, N, 4, 1), (4, 4 * xs, 4 * xs * N, 4 * xs * N * 4))
    ys = M + 2
    y = np.full(ys * N * 4, -3.0, np.float32)
    yt = O.tensor(O.F32, y, (M, N, 4, 1), (4, 4 * ys, 4 * ys * N, 4 * ys * N * 4))
    assert O.mul_mat_strided(wt, xt, yt, 1) == 0
    yv = y.reshape(4, N, ys)
    xv = x.reshape(4, N, xs)
    for s in range(4):
        ws = w[(s // 2) * rb * M:(s // 2 + 1) * rb * M]
        assert np.array_equal(yv[s, :, :M], O.mul_mat(O.Q4_0, ws, K, M, xv[s, :, :K].copy()))
        assert np.all(yv[s, :, M:] == -3.0)
    assert O.mul_mat_strided(wt, xt, yt, 0) == 1  # broadcast refused without allow_broadcast


CPU_BENCH = [  # tools/cpu_bench.cpp inputs; checksums printed by the reference build (%.9g)
    (O.Q4_0, 4096, 4096, 1, 5216.86226),
    (O.Q8_0, 4096, 4096, 1, 723.419414),
    (O.Q4_K, 4096, 4096, 1, -718.604221),
    (O.Q6_K, 4096, 4096, 1, 893.870385),
    (O.Q4_K, 4096, 12288, 8, -38591.9616),
    (O.Q4_K, 4096, 4096, 64, 7066.97543),
]


@pytest.mark.parametrize("dt,K,M,N,checksum", CPU_BENCH)
def test_reference_cpu_bench_checksums(dt, K, M, N, checksum):
    i = np.arange(K * M, dtype=np.int64)
    w = (((i * 37 + 11) % 257) - 128).astype(np.float32) / np.float32(64.0)
    j = np.arange(K * N, dtype=np.int64)
    x = (((j * 17 + 3) % 251) - 125).astype(np.float32) / np.float32(128.0)
    q = O.quantize(dt, w)
    y = O.mul_mat(dt, q, K, M, x.reshape(N, K), threads=8)  # y[n, m]; the tool indexes m + n * M
    flat = y.reshape(-1).astype(np.float64)
    got = float(np.sum(flat * (np.arange(flat.size) % 17 + 1)))
    assert abs(got - checksum) <= 1e-8 * abs(checksum) + 1e-6, got


# ---------------------------------------------------------------------------------------------
# R32 layout (tests/r32/r32_tests.cpp)
# ---------------------------------------------------------------------------------------------

def test_r32_layout_q4_0_hand_checked():
    nat = np.zeros(3 * 36, np.uint8)
    for lane in range(3):
        for b in range(2):
            for i in range(18):
                nat[lane * 36 + b * 18 + i] = 1 + lane * 40 + b * 20 + i
    want = np.zeros(3 * 36, np.uint8)
    for lane in range(3):
        for b in range(2):
            for i in range(16):
                want[(b * 3 + lane) * 16 + i] = 1 + lane * 40 + b * 20 + 2 + i
            for j in range(2):
                want[96 + (b * 3 + lane) * 2 + j] = 1 + lane * 40 + b * 20 + j
    assert np.array_equal(O.r32_pack(O.Q4_0, 64, 3, 1, nat), want)


def test_r32_layout_q8_0_hand_checked():
    nat = np.zeros(2 * 34, np.uint8)
    for lane in range(2):
        for i in range(34):
            nat[lane * 34 + i] = 1 + lane * 50 + i
    want = np.zeros(2 * 34, np.uint8)
    for lane in range(2):
        for j in range(2):
            for i in range(16):
                want[(j * 2 + lane) * 16 + i] = (1 + lane * 50 + 2 + 16 * j + i) ^ 0x80
        for j in range(2):
            want[64 + lane * 2 + j] = 1 + lane * 50 + j
    assert np.array_equal(O.r32_pack(O.Q8_0, 32, 2, 1, nat), want)


@pytest.mark.parametrize("dt,K,M,S", [(O.Q4_0, 64, 33, 1), (O.Q4_0, 32, 64, 4), (O.Q4_0, 32, 1, 1), (O.Q8_0, 64, 40, 2),
                                      (O.Q4_K, 256, 33, 2), (O.Q4_K, 512, 16, 4), (O.Q6_K, 256, 72, 3), (O.Q6_K, 512, 32, 1)])
def test_r32_identity(dt, K, M, S):
    nat = ((np.arange(O.row_bytes(dt, K) * M * S) * 7 + 13) & 0xFF).astype(np.uint8)
    assert np.array_equal(O.r32_unpack(dt, K, M, S, O.r32_pack(dt, K, M, S, nat)), nat)


# ---------------------------------------------------------------------------------------------
# live comparison with the reference compiled from source (build container only)
# ---------------------------------------------------------------------------------------------

@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (the reference sources are absent)")
@pytest.mark.parametrize("dt", O.QTYPES, ids=lambda d: O.NAMES[d])
def test_live_reference(dt):
    rng = np.random.default_rng(99 + dt)
    for trial in range(4):
        n = O.BLOCK[dt] * int(rng.integers(1, 40))
        x = (rng.standard_normal(n) * [0.02, 1.0, 50.0, 1e-4][trial]).astype(np.float32)
        q = O.quantize(dt, x)
        assert np.array_equal(q, O.ref_quantize(dt, x))
        assert np.array_equal(O.dequantize(dt, q, n).view(np.uint32), O.ref_dequantize(dt, q, n).view(np.uint32))
    K, M = 4 * O.BLOCK[dt] if O.BLOCK[dt] == 32 else 512, 45
    q = O.quantize(dt, O.normal(K * M, 11, 0.0, 0.02))
    for N in (1, 2, 5, 16, 33):
        x = O.normal(N * K, 12 + N).reshape(N, K)
        assert np.array_equal(O.mul_mat(dt, q, K, M, x).view(np.uint32), O.ref_mul_mat(dt, q, K, M, x).view(np.uint32))
    nat = rng.integers(0, 256, O.row_bytes(dt, K) * 72 * 2, dtype=np.uint8)  # 72 rows: 16-byte slice stride
    assert np.array_equal(O.r32_pack(dt, K, 72, 2, nat), O.ref_r32(dt, K, 72, 2, nat, True))
    E, T, nu = 6, 4, 3
    w = O.quantize(dt, O.normal(K * M * E, 13, 0.0, 0.02))
    ids = rng.integers(0, E, (T, nu)).astype(np.int32)
    for n1 in (1, nu):
        x = O.normal(T * n1 * K, 14 + n1).reshape(T, n1, K)
        st, yr = O.ref_mul_mat_id(dt, w, K, M, E, x, ids)
        assert st == 0 and np.array_equal(O.mul_mat_id(dt, w, K, M, E, x, ids).view(np.uint32), yr.view(np.uint32))
    assert O.ref_mul_mat_id(dt, w, K, M, E, x, np.full((T, nu), E, np.int32))[0] == 2
    rid = rng.integers(0, M, 9).astype(np.int32)
    st, gr = O.ref_get_rows(dt, q, K, M, rid)
    assert st == 0 and np.array_equal(O.get_rows(dt, q, K, M, rid).view(np.uint32), gr.view(np.uint32))
