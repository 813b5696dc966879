"""Precision of the decode and prefill paths on activations with outliers, against the CPU oracle.

Real activations are not N(0, 1): a few channels carry values tens to hundreds of times the rest,
and their distribution is heavy-tailed. The decode matvec represents each 32-element segment of x
relative to its largest element, and the prefill GEMM scales each token row by a power of two
before its f16 conversion, so both are tested here on
  * outlier channels: N(0, 1) with one element of every 32-element segment at +-100 sigma;
  * heavy tails: Student-t with 3 degrees of freedom;
  * rows of very different magnitude (prefill only: the per-row power-of-two scaling);
for all four weight formats, K = 4096 and 12288, and N = 1, 8 (decode) and 512 (prefill), against
the gates of the decode path (NMSE <= 1e-7, max-abs <= 1e-4 ||x||_2 max|w|) and of the prefill
path (NMSE <= 5e-5).
"""
import numpy as np
import pytest

import oracle as O
import scrapgpulibrary_amd as sg
from tests.gpu_util import check_matvec, nmse, quantized, run_mul_mat

pytestmark = pytest.mark.gpu


def activations(kind, N, K, seed):
    rng = np.random.default_rng(seed)
    if kind == "outlier":
        x = rng.standard_normal((N, K))
        pos = rng.integers(0, 32, K // 32)  # one outlier channel per segment, the same in every token
        x.reshape(N, K // 32, 32)[:, np.arange(K // 32), pos] = 100.0 * rng.choice([-1.0, 1.0], (N, K // 32))
    elif kind == "student_t":
        x = rng.standard_t(3, (N, K))
    else:  # row magnitudes spread over 2^-20 .. 2^20
        x = rng.standard_normal((N, K)) * np.exp2(rng.integers(-20, 21, (N, 1)))
    return x.astype(np.float32)


@pytest.mark.parametrize("kind", ["outlier", "student_t"])
@pytest.mark.parametrize("N", [1, 8])
@pytest.mark.parametrize("K", [4096, 12288])
@pytest.mark.parametrize("dtype", sg.QTYPES, ids=lambda d: sg.NAMES[d])
def test_decode_outlier_activations(hip, dtype, K, N, kind):
    dev, st = hip
    M = 256
    q, deq = quantized(dtype, K, M, 1100 + K % 97)
    x = activations(kind, N, K, 1200 + N)
    y = run_mul_mat(dev, st, dtype, q, K, M, x)
    ref = O.mul_mat(dtype, q, K, M, x, threads=8)
    e = check_matvec(y, ref, x, deq)
    print(f"{sg.NAMES[dtype]} K={K} N={N} {kind}: NMSE {e:.3e}", flush=True)


@pytest.mark.parametrize("kind", ["outlier", "student_t", "row_scales"])
@pytest.mark.parametrize("K", [4096, 12288])
@pytest.mark.parametrize("dtype", sg.QTYPES, ids=lambda d: sg.NAMES[d])
def test_prefill_outlier_activations(hip, dtype, K, kind):
    dev, st = hip
    M, N = 384, 512
    q, _ = quantized(dtype, K, M, 1300 + K % 97)
    x = activations(kind, N, K, 1400)
    y = run_mul_mat(dev, st, dtype, q, K, M, x)
    ref = O.mul_mat(dtype, q, K, M, x, threads=8)
    e = nmse(y, ref)
    # the NMSE of each token row on its own: a row scaled far below the others must not lose its
    # precision to them
    worst = max(nmse(y[n], ref[n]) for n in range(N))
    print(f"{sg.NAMES[dtype]} K={K} N={N} {kind}: NMSE {e:.3e}, worst row {worst:.3e}", flush=True)
    assert e <= 5e-5, f"NMSE {e:.3e}"
    assert worst <= 5e-5, f"worst row NMSE {worst:.3e}"
