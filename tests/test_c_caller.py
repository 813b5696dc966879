"""The public C API used from a C99 program (tests/c/standalone_matmul.c, built with the library
by scrapgpulibrary_amd/build.py), as the reference's examples/standalone_matmul.c:115-195 uses
it: configs[0] of the benchmark set -- Q4_0 W 4096 x 4096 ~ N(0, 0.02) uploaded as R32, x [1, 4096]
~ N(0, 1) -- with the result checked against the CPU oracle."""
import os
import subprocess

import numpy as np
import pytest

import oracle as O
from scrapgpulibrary_amd import build as B
from tests.gpu_util import check_matvec


def _run(args, timeout=120):
    return subprocess.run([B.C_CALLER] + [str(a) for a in args], capture_output=True, text=True, timeout=timeout)


def test_c_caller_links_and_checks_arguments():
    assert os.path.exists(B.C_CALLER), "built by scrapgpulibrary_amd/build.py"
    r = _run([])
    assert r.returncode == 1 and "usage" in r.stderr
    if not os.path.exists("/dev/kfd"):  # no GPU here: the library loads and finds no device
        r = _run([4096, 4096, 1, "w", "x", "y"])
        assert r.returncode == 2 and "no gfx950 device" in r.stderr, r.stderr


@pytest.mark.gpu
def test_c_caller_config1_q4_0(tmp_path):
    K = M = 4096
    q = O.quantize(O.Q4_0, O.normal(K * M, 0, 0.0, 0.02))
    x = O.normal(K, 1).reshape(1, K)
    (tmp_path / "w.bin").write_bytes(q.tobytes())
    (tmp_path / "x.bin").write_bytes(x.tobytes())
    print("C caller: Q4_0 4096 x 4096, N = 1", flush=True)
    r = _run([K, M, 1, tmp_path / "w.bin", tmp_path / "x.bin", tmp_path / "y.bin"])
    assert r.returncode == 0, r.stderr
    print(r.stdout.strip(), flush=True)
    y = np.fromfile(tmp_path / "y.bin", np.float32).reshape(1, M)
    ref = O.mul_mat(O.Q4_0, q, K, M, x, threads=8)
    e = check_matvec(y, ref, x, O.dequantize(O.Q4_0, q, K * M))
    print(f"NMSE {e:.3e}", flush=True)
