"""bench.py's contract checked without a GPU: more than one GPU is refused with a message before any
device is touched, and the byte counts behind its metric are the ones BASELINE.json's workloads
state (the Qwen3-8B Q4_K_M decode token, the MoE token, the config matrices)."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402
import scrapgpulibrary_amd as sg  # noqa: E402


@pytest.mark.parametrize("argv,env", [(["--gpus", "2"], {}), (["--gpus", "8", "--steps", "1"], {}), ([], {"WORLD_SIZE": "2"})])
def test_more_than_one_gpu_is_refused(argv, env):
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py")] + argv, capture_output=True, text=True, timeout=120,
                       env={**os.environ, **env})
    assert r.returncode == 2, r.stderr
    assert "one GPU" in r.stderr and r.stdout == ""


def test_decode_token_bytes():
    # q, o 4096x4096, k, v 1024x4096, gate, up 12288x4096 in Q4_K and down 4096x12288 in Q6_K, 36 layers
    per_layer = sum(bench.weight_bytes(dt, K, M) for _, dt, K, M in bench.LAYER_SHAPES)
    assert per_layer == 2 * 9_437_184 + 2 * 2_359_296 + 2 * 28_311_552 + 41_287_680
    assert per_layer * bench.LAYERS == 4_374_134_784


def test_config_matrix_bytes():
    assert bench.weight_bytes(sg.Q4_0, 4096, 4096) == 9_437_184
    assert bench.weight_bytes(sg.Q8_0, 4096, 11008) == 47_906_816
    assert bench.weight_bytes(sg.Q4_K, 4096, 12288) == 28_311_552
    assert bench.weight_bytes(sg.Q6_K, 12288, 4096) == 41_287_680
    assert bench.weight_bytes(sg.Q6_K, 4096, 151936) == 510_504_960
    assert bench.weight_bytes(sg.Q4_K, 8192, 28672) == 132_120_576


def test_moe_token_bytes():
    # 48 layers x 8 selected experts x (gate, up Q4_K 2048->768; down Q6_K 768->2048)
    per_expert = 2 * bench.weight_bytes(sg.Q4_K, 2048, 768) + bench.weight_bytes(sg.Q6_K, 768, 2048)
    assert bench.MOE_LAYERS * bench.MOE_USED * per_expert == 1_174_929_408
