"""bench.py's command-line contract and the constants its roofline figures rest on (CPU only:
no case reaches the GPU)."""

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def _run(*args):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True, text=True,
                          timeout=120)


def test_more_than_one_gpu_is_refused_before_any_gpu_work():
    r = _run("--gpus", "2")
    assert r.returncode == 2
    assert "measures one GPU" in r.stderr and "--gpus 2" in r.stderr
    assert r.stdout == ""


def test_bad_step_counts_are_refused():
    r = _run("--steps", "0")
    assert r.returncode != 0 and "steps must be >= 1" in r.stderr


def test_decode_kernel_count_matches_the_step_graph():
    # The greedy pick with the embedding; per layer q/k/v GEMV, split attention, o, gate/up and
    # down GEMVs; then the LM head (its norm, the greedy keys and the advance in the same kernel).
    assert bench.decode_kernels_per_token(bench.SMOL) == 5 * 30 + 2 == 152


def test_decode_roofline_bytes_follow_the_model_shape():
    """162 MB a token: int8 layer weights, their per-output scales, the int8 LM head, the norm
    weights and the mean KV rows of positions 512 .. 639 (46,080 bytes a position)."""
    h, inter, layers, vocab = 576, 1536, 30, 49152
    q, kv = 9 * 64, 3 * 64
    per_layer_w = h * (q + 2 * kv) + q * h + h * 2 * inter + inter * h
    per_layer_scales = 4 * ((q + 2 * kv) + h + 2 * inter + h)
    norms = 4 * h * (2 * layers + 1)
    kv_row = 2 * layers * kv * 4  # k and v, fp32, every layer
    assert per_layer_w * layers == 106_168_320
    assert per_layer_scales * layers == 622_080
    assert vocab * h == 28_311_552
    assert norms == 140_544
    assert kv_row == 46_080
    assert bench.LLAMA_DECODE_BYTES == 106_168_320 + 622_080 + 28_311_552 + 140_544 + 46_080 * 576


def test_gemv_algorithmic_bytes():
    # W int8 + per-column scale + X + C, each once (the headline's 58,851,328 at m = 1).
    assert bench.gemv_bytes(1) == 4096 * 14336 + 4 * 14336 + 4 * 4096 + 4 * 14336 == 58_851_328
