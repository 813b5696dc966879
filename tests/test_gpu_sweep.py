"""A seeded sweep of MUL_MAT shapes over every weight dtype (quantized R32 and float natural), 1..700
columns, odd M and K, slices with broadcast: each against the oracle at the gate of its path
(decode: NMSE <= 1e-7 and max-abs; prefill: NMSE <= 5e-5). It exercises the shape rules that pick
a kernel form, so every form a shape can reach is checked on shapes no other test chose."""
import numpy as np
import pytest

import oracle as O
import scrapgpulibrary_amd as sg
from tests.gpu_util import check_matvec, nmse

pytestmark = pytest.mark.gpu

DTYPES = (sg.Q4_0, sg.Q8_0, sg.Q4_K, sg.Q6_K, sg.F16, sg.BF16, sg.F32)


def cases(n=96, seed=20261202):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        dt = DTYPES[i % len(DTYPES)]
        blk = sg.BLOCK[dt] if dt not in (sg.F16, sg.BF16, sg.F32) else 8
        K = int(blk * rng.integers(max(1, 64 // blk), max(2, 6144 // blk) + 1))
        if dt in (sg.F16, sg.BF16) and rng.random() < 0.5:
            K = 128 * max(1, K // 128)  # (the GEMM's whole stages)
        M = int(rng.integers(1, 3000))
        N = int(rng.choice([1, 2, 3, 5, 8, 9, 17, 64, 100, 256, 700]))
        S = int(rng.choice([1, 1, 1, 2]))
        bc = int(rng.choice([1, 2])) if S == 2 else 1
        if S > 1:
            M = (M + 15) // 16 * 16  # (R32 slices must span whole 16-byte units)
        while M * K * N * S * bc > 6e8:
            N = max(1, N // 2)
        out.append((dt, K, M, N, S, bc))
    return out


def weights(dt, K, M, S, seed):
    w = O.normal(S * M * K, seed, 0.0, 0.02)
    if dt == sg.F32:
        return w.reshape(S, M * K), w.reshape(S, M, K)
    if dt == sg.F16:
        h = w.astype(np.float16)
        return h.view(np.uint16).reshape(S, -1), h.astype(np.float32).reshape(S, M, K)
    if dt == sg.BF16:
        b = O.float_to_bf16(w)
        return b.reshape(S, -1), O.bf16_to_float(b).reshape(S, M, K)
    q = O.quantize(dt, w, threads=8)
    return q.reshape(S, -1), O.dequantize(dt, q, S * M * K).reshape(S, M, K)


@pytest.mark.parametrize("case", cases(), ids=lambda c: f"{O.NAMES[c[0]]}-K{c[1]}-M{c[2]}-N{c[3]}-S{c[4]}x{c[5]}")
def test_sweep(hip, case):
    dt, K, M, N, S, bc = case
    dev, st = hip
    quant = dt in sg.QTYPES
    wq, wf = weights(dt, K, M, S, 31 + K + M)
    wbytes = np.ascontiguousarray(wq).view(np.uint8).reshape(-1)
    wb = dev.alloc(wbytes.nbytes)
    if quant:
        wt = sg.tdesc(dt, (K, M, S), wb, layout=sg.R32)
        st.upload(wt, wbytes)
    else:
        st.write(wb, 0, wbytes)
        wt = sg.tdesc(dt, (K, M, S), wb)
    SX = S * bc
    x = O.normal(SX * N * K, 32 + N).reshape(SX, N, K)
    xb, yb = dev.alloc(x.nbytes), dev.alloc(4 * M * N * SX)
    xt, yt = sg.tdesc(sg.F32, (K, N, SX), xb), sg.tdesc(sg.F32, (M, N, SX), yb)
    st.write(xb, 0, x)
    op, keep = sg.mul_mat_op(wt, xt, yt, allow_broadcast=1)
    st.execute(op)
    st.sync()
    form = sg.last_launch()[0]
    y = st.download(yt).reshape(SX, N, M)
    for s in range(SX):
        ws = s // bc
        ref = O.mul_mat(dt, wq[ws], K, M, x[s], threads=8)
        if N <= 8 or (not quant and (dt == sg.F32 or K % 128 != 0)):
            check_matvec(y[s], ref, x[s], wf[ws])
        else:
            e = nmse(y[s], ref)
            assert e <= 5e-5, f"slice {s}: NMSE {e:.3e} [{form}]"
    for b in (wb, xb, yb):
        b.free()


def multi_cases(n=24, seed=20261203):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        dt = DTYPES[i % len(DTYPES)]
        blk = sg.BLOCK[dt] if dt in sg.QTYPES else 128
        K = int(blk * rng.integers(max(1, 256 // blk), max(2, 4096 // blk) + 1))
        Ms = tuple(int(m) for m in rng.integers(1, 1500, int(rng.integers(2, 4))))
        N = int(rng.choice([1, 4, 8, 33, 128, 300]))
        out.append((dt, K, Ms, N))
    return out


@pytest.mark.parametrize("case", multi_cases(), ids=lambda c: f"{O.NAMES[c[0]]}-K{c[1]}-M{'+'.join(map(str, c[2]))}-N{c[3]}")
def test_sweep_multi(hip, case):
    """MUL_MAT_MULTI: 2-3 weights of one dtype sharing x (one fused launch where the form allows)."""
    dt, K, Ms, N = case
    dev, st = hip
    quant = dt in sg.QTYPES
    x = O.normal(N * K, 41 + N).reshape(N, K)
    xb = dev.alloc(x.nbytes)
    xt = sg.tdesc(sg.F32, (K, N), xb)
    st.write(xb, 0, x)
    bufs, wts, yts, refs = [xb], [], [], []
    for j, M in enumerate(Ms):
        wq, wf = weights(dt, K, M, 1, 43 + 7 * j + M)
        wbytes = np.ascontiguousarray(wq).view(np.uint8).reshape(-1)
        wb = dev.alloc(wbytes.nbytes)
        if quant:
            wt = sg.tdesc(dt, (K, M), wb, layout=sg.R32)
            st.upload(wt, wbytes)
        else:
            st.write(wb, 0, wbytes)
            wt = sg.tdesc(dt, (K, M), wb)
        yb = dev.alloc(4 * M * N)
        bufs += [wb, yb]
        wts.append(wt)
        yts.append(sg.tdesc(sg.F32, (M, N), yb))
        refs.append((O.mul_mat(dt, wq[0], K, M, x, threads=8), wf[0]))
    op, keep = sg.multi_op(wts, xt, yts)
    st.execute(op)
    st.sync()
    form = sg.last_launch()[0]
    for M, yt, (ref, wf) in zip(Ms, yts, refs):
        y = st.download(yt).reshape(N, M)
        if N <= 8 or (not quant and (dt == sg.F32 or K % 128 != 0)):
            check_matvec(y, ref, x, wf)
        else:
            e = nmse(y, ref)
            assert e <= 5e-5, f"{M} rows: NMSE {e:.3e} [{form}]"
    for b in bufs:
        b.free()


def id_cases(n=16, seed=20261204):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        dt = (sg.Q4_0, sg.Q8_0, sg.Q4_K, sg.Q6_K, sg.F16, sg.F32)[i % 6]
        blk = sg.BLOCK[dt] if dt in sg.QTYPES else 8
        K = int(blk * rng.integers(max(1, 256 // blk), max(2, 3072 // blk) + 1))
        M = int(rng.integers(1, 50)) * 16  # (R32 experts span whole 16-byte units)
        E = int(rng.integers(2, 40))
        nu = int(rng.integers(1, min(E, 8) + 1))
        T = int(rng.choice([1, 3, 9, 40, 128]))
        shared = bool(rng.integers(0, 2))
        out.append((dt, K, M, E, nu, T, shared))
    return out


@pytest.mark.parametrize("case", id_cases(), ids=lambda c: f"{O.NAMES[c[0]]}-K{c[1]}-M{c[2]}-E{c[3]}-u{c[4]}-T{c[5]}-{'shared' if c[6] else 'slots'}")
def test_sweep_mul_mat_id(hip, case):
    """MUL_MAT_ID: experts, slots and tokens of random sizes (the per-pair matvec and, for many
    tokens of quantized experts, the grouped GEMM), every pair against the oracle."""
    dt, K, M, E, nu, T, shared = case
    dev, st = hip
    quant = dt in sg.QTYPES
    wq, wf = weights(dt, K, M * E, 1, 51 + K + E)
    wbytes = np.ascontiguousarray(wq).view(np.uint8).reshape(-1)
    wb = dev.alloc(wbytes.nbytes)
    if quant:
        wt = sg.tdesc(dt, (K, M, E), wb, layout=sg.R32)
        st.upload(wt, wbytes)  # (the natural bytes of E slices, packed slice by slice)
    else:
        st.write(wb, 0, wbytes)
        wt = sg.tdesc(dt, (K, M, E), wb)
    rng = np.random.default_rng(52 + T)
    ids = np.stack([rng.permutation(E)[:nu] for _ in range(T)]).astype(np.int32)
    n1 = 1 if shared else nu
    x = O.normal(T * n1 * K, 53 + T).reshape(T, n1, K)
    xb, ib, yb = dev.alloc(x.nbytes), dev.alloc(ids.nbytes), dev.alloc(4 * M * nu * T)
    st.write(xb, 0, x)
    st.write(ib, 0, ids)
    xt, it, yt = sg.tdesc(sg.F32, (K, n1, T), xb), sg.tdesc(sg.I32, (nu, T), ib), sg.tdesc(sg.F32, (M, nu, T), yb)
    op, keep = sg.mul_mat_id_op(wt, xt, it, yt, nu)
    st.execute(op)
    st.sync()
    form = sg.last_launch()[0]
    y = st.download(yt).reshape(T, nu, M)
    ref = O.mul_mat_id(dt, wq[0], K, M, E, x, ids)
    # (the backend's rule: quantized experts, more than 8 tokens, at least 4 pairs per expert)
    grouped = quant and T > 8 and nu * T >= 4 * E
    if grouped:
        e = nmse(y, ref)
        assert e <= 5e-5, f"NMSE {e:.3e} [{form}]"
    else:
        wfe = wf[0].reshape(E, M, K)
        for t in range(T):
            for i in range(nu):
                xc = x[t, 0 if shared else i][None, :]
                check_matvec(y[t, i][None, :], ref[t, i][None, :], xc, wfe[ids[t, i]])
    for b in (wb, xb, ib, yb):
        b.free()
