"""The parts of bench.py's JSON contract that need no GPU: which roofline
bounds a launch, the committed traffic figures it reports, and the refusal
of more than one GPU."""
import pathlib
import subprocess
import sys

import pytest

REPO = pathlib.Path(__file__).resolve().parents[1]
sys.path.insert(0, str(REPO))

import bench  # noqa: E402  (imports no GPU code at module level)


class _Args:
    def __init__(self, layers, m_und, m_gen):
        self.layers, self.m_und, self.m_gen = layers, m_und, m_gen


def _layer_bytes(m_und, m_gen):
    """Algorithmic bytes of one config-2-shaped layer, as bench.py counts
    them: each weight set with rows once, activations and outputs once."""
    M = m_und + m_gen
    nsets = (m_und > 0) + (m_gen > 0)
    H, I, NQ, NKV = bench.HIDDEN, bench.INTER, bench.NQ, bench.NKV
    return (nsets * bench.FLOP_PER_ROW + 2 * M * (H + NQ + H + I)
            + 2 * M * (NQ + 2 * NKV + H + 2 * I + H))


def test_flop_per_row_is_the_layer_shapes():
    # q, k, v, o, gate, up, down of a Qwen3-8B-shaped layer
    H, I, NQ, NKV = 4096, 12288, 4096, 1024
    assert bench.FLOP_PER_ROW == 2 * (H * NQ + 2 * H * NKV + NQ * H + 2 * H * I + I * H)
    assert bench.FLOP_PER_ROW == 385875968


@pytest.mark.parametrize("m_und,m_gen,bound", [
    (128, 4096, "mfma"),   # config 2: the headline
    (128, 0, "hbm"),       # und-only prefill: the weights dominate
    (0, 256, "hbm"),
    (0, 1024, "mfma"),     # config 5's small split is above the ridge
])
def test_roofline_side_of_the_ridge(m_und, m_gen, bound):
    flop = bench.FLOP_PER_ROW * (m_und + m_gen)
    nbytes = _layer_bytes(m_und, m_gen)
    r = bench._roof(flop, nbytes, 1000.0, 2000.0, bench.PEAK_BF16, "TFLOP/s")
    assert r["bound"] == bound
    if bound == "hbm":
        assert r["unit"] == "GB/s" and r["peak"] == bench.PEAK_HBM
        assert r["achieved"] == 2000.0 and r["frac"] == round(2000.0 / 8000.0, 4)
    else:
        assert r["unit"] == "TFLOP/s" and r["peak"] == bench.PEAK_BF16
        assert r["frac"] == round(1000.0 / bench.PEAK_BF16, 4)


def test_ridge_is_peak_over_hbm():
    # exactly at the bf16 ridge (314.6 FLOP/B) the matrix cores bound it
    ridge = bench.PEAK_BF16 * 1e12 / (bench.PEAK_HBM * 1e9)
    assert bench._roof(ridge * 1e6, 1e6, 1.0, 1.0, bench.PEAK_BF16, "TFLOP/s")["bound"] == "mfma"
    assert bench._roof(ridge * 0.99e6, 1e6, 1.0, 1.0, bench.PEAK_BF16, "TFLOP/s")["bound"] == "hbm"


def test_committed_traffic_figures():
    c2 = bench.measured_traffic(_Args(1, 128, 4096))
    und = bench.measured_traffic(_Args(1, 128, 0))
    assert c2 is not None and und is not None
    # traffic beyond L2 is at least the algorithmic bytes of a launch
    assert c2 >= _layer_bytes(128, 4096) / 4
    assert und >= _layer_bytes(128, 0) / 4
    assert bench.measured_traffic(_Args(42, 128, 4096)) is None
    assert bench.measured_traffic(_Args(1, 4352, 12288)) is None


def test_more_than_one_gpu_is_refused():
    p = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert p.returncode == 2
    assert "one GPU only" in p.stderr
    assert p.stdout == ""
