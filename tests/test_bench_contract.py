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
    # the und-only split is profiled as the bench runs it: two layers
    # rotated (their weights exceed twice the Infinity Cache)
    assert bench.parse(["--m-und", "128", "--m-gen", "0"]).layers == 2
    und = bench.measured_traffic(_Args(2, 128, 0))
    assert c2 is not None and und is not None
    # traffic beyond L2 is at least the algorithmic bytes of a launch
    assert c2 >= _layer_bytes(128, 4096) / 4
    assert und >= _layer_bytes(128, 0) / 4
    assert bench.measured_traffic(_Args(42, 128, 4096)) is None
    assert bench.measured_traffic(_Args(1, 4352, 12288)) is None
    # the int8 kernel's figure is its own, at least its algorithmic bytes
    # (int8 weights and codes, f32 scales, bf16 output) and below bf16's
    c2_i8 = bench.measured_traffic(_Args(1, 128, 4096), int8=True)
    assert c2_i8 is not None and c2_i8 != c2
    work = bench.step_work(128, 4096, 1)
    assert c2_i8 >= work["i8_bytes"] / work["gemm_launches"]
    assert c2_i8 < c2
    assert bench.measured_traffic(_Args(2, 128, 0), int8=True) is None


def test_more_than_one_gpu_is_refused():
    p = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert p.returncode == 2
    assert "one GPU only" in p.stderr
    assert p.stdout == ""


# ---- per-launch arithmetic of a step (both tiers) ---------------------------

@pytest.mark.parametrize("layers", [1, 42])
def test_step_work_per_launch(layers):
    """FLOP and algorithmic bytes per GEMM launch do not depend on how many
    layers a step holds, and the int8 figures count int8 operands."""
    w = bench.step_work(128, 4096, layers)
    M = 4224
    assert w["gemm_launches"] == 4 * layers and w["quant_launches"] == 4 * layers
    assert w["flop"] / w["gemm_launches"] == bench.FLOP_PER_ROW * M / 4
    # bf16: both weight sets, inputs and outputs, 2 bytes each
    assert w["bf16_bytes"] / w["gemm_launches"] == _layer_bytes(128, 4096) / 4
    # int8: int8 weights (half the bf16 bytes) + f32 channel scales of both
    # sets, int8 inputs + one f32 scale per row per launch, bf16 outputs
    H, I, NQ, NKV = bench.HIDDEN, bench.INTER, bench.NQ, bench.NKV
    cols = NQ + 2 * NKV + H + 2 * I + H
    i8_layer = (2 * bench.FLOP_PER_ROW // 2 + 4 * 2 * cols
                + M * (H + NQ + H + I) + 16 * M + 2 * M * cols)
    assert w["i8_bytes"] / w["gemm_launches"] == i8_layer / 4
    assert 204e6 < w["i8_bytes"] / w["gemm_launches"] < 206e6
    # the quantiser reads bf16 and writes int8 + a scale per row
    assert w["quant_bytes"] / w["quant_launches"] == \
        (3 * M * (H + NQ + H + I) + 16 * M) / 4


def test_tier_result_divides_by_launches():
    """The int8 roofline uses the measured launch count: a 42-layer step's
    per-launch figures equal a 1-layer step's at the same kernel speed."""
    outs = []
    for layers in (1, 42):
        w = bench.step_work(128, 4096, layers)
        steps = 3
        k = {"gemm_ms": 0.17 * w["gemm_launches"] * steps,
             "pre_ms": 0.02 * w["quant_launches"] * steps,
             "post_ms": 0.05 * layers * steps, "calls": w["gemm_launches"] * steps}
        outs.append(bench.tier_result(w, 0.8 * layers, k, steps, True, None))
    a, b = outs
    for key in ("achieved", "frac", "avg_launch_ms", "alg_bytes_per_launch",
                "achieved_GBps", "split_reduce_ms_per_step"):
        if key == "split_reduce_ms_per_step":
            assert b["roofline"][key] == pytest.approx(42 * a["roofline"][key])
        else:
            assert b["roofline"][key] == pytest.approx(a["roofline"][key])
    assert a["roofline"]["frac"] < 1.0
    assert a["quant_kernel"]["achieved_GBps"] == b["quant_kernel"]["achieved_GBps"]
    assert a["value"] == b["value"]


def test_kernel_label_follows_the_knobs(monkeypatch):
    for k in ("U15H_WAVES", "U15H_MFMA16"):
        monkeypatch.delenv(k, raising=False)
    assert bench.kernel_label(False) == "mot_gemm_kernel<MmaBf16x16, kBf16, 4>"
    assert bench.kernel_label(True) == "mot_gemm_kernel<MmaI8x16, kDequantBf16, 4>"
    monkeypatch.setenv("U15H_WAVES", "4")
    assert bench.kernel_label(False) == "mot_gemm_kernel<MmaBf16x16, kBf16, 2>"
    monkeypatch.setenv("U15H_WAVES", "8")
    monkeypatch.setenv("U15H_MFMA16", "0")
    assert bench.kernel_label(False) == "mot_gemm_kernel<MmaBf16, kBf16, 4>"
    assert bench.kernel_label(True) == "mot_gemm_kernel<MmaI8, kDequantBf16, 4>"
    monkeypatch.setenv("U15H_MFMA16", "-1")
    assert bench.kernel_label(False) == "mot_gemm_kernel<MmaBf16, kBf16, 4>"
    assert bench.kernel_label(True) == "mot_gemm_kernel<MmaI8x16, kDequantBf16, 4>"


def test_kernel_label_names_the_skinny_route(monkeypatch):
    """bf16 steps whose groups all have <= 128 rows run the skinny kernels
    (the build by rows); int8, larger groups and U15H_SKINNY=0 the tiled
    kernel."""
    for k in ("U15H_WAVES", "U15H_MFMA16", "U15H_SKINNY"):
        monkeypatch.delenv(k, raising=False)
    assert bench.kernel_label(False, 1) == "skinny_dma_kernel<1>"
    assert bench.kernel_label(False, 64) == "skinny_lds_kernel<4, 4, 0, 1>"
    assert bench.kernel_label(False, 128).startswith("skinny_lds_kernel<8")
    assert bench.kernel_label(False, 129) == "mot_gemm_kernel<MmaBf16x16, kBf16, 4>"
    assert bench.kernel_label(True, 128) == "mot_gemm_kernel<MmaI8x16, kDequantBf16, 4>"
    assert bench.step_work(128, 0, 1)["max_rows"] == 128
    assert bench.step_work(128, 4096, 1)["max_rows"] == 4096
    monkeypatch.setenv("U15H_SKINNY", "0")
    assert bench.kernel_label(False, 128) == "mot_gemm_kernel<MmaBf16x16, kBf16, 4>"


def test_small_m_rotates_past_the_cache():
    """Below the ridge a pass cycles more than twice the 256 MB Infinity
    Cache of weights; above it one layer is the step."""
    assert bench.rotation_layers(128, 4096) == 1
    assert bench.rotation_layers(4352, 12288) == 1
    for mu, mg in ((128, 0), (0, 128), (64, 192), (1, 0)):
        n = bench.rotation_layers(mu, mg)
        sets = (mu > 0) + (mg > 0)
        assert n * sets * bench.LAYER_WEIGHT_BYTES >= 2 * bench.MALL_BYTES
        assert (n - 1) * sets * bench.LAYER_WEIGHT_BYTES < 2 * bench.MALL_BYTES
    a = bench.parse(["--m-und", "128", "--m-gen", "0"])
    assert a.layers == 2
    assert bench.parse([]).layers == 1
    assert bench.parse(["--workload", "c5"]).layers == 42


def test_timed_blocks_follow_their_kernel_pass():
    """Per tier: the warm-up (at least --warmup steps and --warmup-ms of
    time; the line reports the steps actually run), the per-kernel pass
    (events bound to the kernels' dispatches), then the contract's block,
    unprofiled, in the same steady state; the interleaved samples follow."""
    import inspect
    src = inspect.getsource(bench.main)
    w16 = src.index("warm(torch, runs, args.warmup, args.warmup_ms)")
    k16 = src.index("timed_step_kernels(torch, ops, runs, args.steps")
    t16 = src.index("timed_step(torch, runs, args.steps, 0)")
    w8 = src.index('warm(torch, arms["int8"], args.warmup, args.warmup_ms)')
    k8 = src.index('timed_step_kernels(torch, ops, arms["int8"], args.steps')
    t8 = src.index('timed_step(torch, arms["int8"], args.steps, 0)')
    inter = src.index("interleaved(torch, arms, args.steps, args.rounds)")
    assert w16 < k16 < t16 < w8 < k8 < t8 < inter
    assert '"warmup": n_warm' in src
    assert bench.parse([]).warmup_ms >= 100
    body = inspect.getsource(bench.timed_step_kernels)
    assert "profile_next_kernels" in body


def test_warm_runs_at_least_the_requested_steps_and_time():
    class _T:       # a torch stand-in: synchronize only
        class cuda:
            @staticmethod
            def synchronize():
                pass
    calls = []
    n = bench.warm(_T, [lambda: calls.append(1)], 5, 0.0)
    assert n == 5 and len(calls) == 5
    import time as _time
    slow = [lambda: _time.sleep(0.002)]
    n = bench.warm(_T, slow, 1, 30.0)
    assert n >= 8          # 30 ms of 2 ms steps, in doubling batches


@pytest.mark.parametrize("int8", [False, True])
def test_tier_result_checks_that_the_kernels_fit_the_step(int8):
    """launches x avg_launch_ms + reductions (+ quantisers) against the
    timed step: fits_step says whether the bracketed kernels add up to at
    most a step."""
    w = bench.step_work(128, 4096, 1)
    steps = 4
    k = {"gemm_ms": 0.30 * 4 * steps, "pre_ms": (0.015 * 4 * steps) if int8 else 0.0,
         "post_ms": 0.02 * steps, "calls": 4 * steps}
    per_step = (k["gemm_ms"] + k["pre_ms"] + k["post_ms"]) / steps
    ok = bench.tier_result(w, per_step * 1.01, k, steps, int8, None)["roofline"]
    assert ok["fits_step"] and ok["kernels_ms_per_step"] == pytest.approx(per_step)
    assert ok["avg_launch_ms"] * 4 + ok["split_reduce_ms_per_step"] <= per_step * 1.01
    bad = bench.tier_result(w, per_step * 0.97, k, steps, int8, None)["roofline"]
    assert not bad["fits_step"]


def test_vendor_shapes_are_the_gen_groups_projections():
    """--vendor times plain GEMMs at the gen group's own shapes: gate|up
    (N = 2I), down (K = I) and q|k|v (N = q + 2 kv) over the 4096 gen
    rows, and down over the und + gen rows as one matrix."""
    H, I, NQ, NKV = bench.HIDDEN, bench.INTER, bench.NQ, bench.NKV
    shapes = set(bench.VENDOR_SHAPES)
    assert (4096, 2 * I, H) in shapes
    assert (4096, H, I) in shapes
    assert (4096, NQ + 2 * NKV, H) in shapes
    assert (4224, H, I) in shapes
    a = bench.parse(["--vendor", "--vendor-shape", "4096x24576x4096"])
    assert a.vendor and a.vendor_shape == "4096x24576x4096"
    assert not bench.parse([]).vendor
