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
