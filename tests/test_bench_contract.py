"""bench.py's contract that can be checked without a GPU: the one-GPU guard and
the committed traffic counters its roofline objects read."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


@pytest.mark.parametrize("n", [2, 8])
def test_more_than_one_gpu_exits_with_a_message(n):
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", str(n)],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert line["n_gpus"] == n and "one GPU" in line["error"]


def test_traffic_lines_cover_every_roofline_object():
    """Every `traffic` key bench.py looks up has a calibrated line in
    profiles/bench_hbm_traffic_counters.md, and each is at least the kernel's
    algorithmic bytes minus 1% (counters cannot read less than the data moved)."""
    t = bench.measured_traffic()
    algorithmic = {
        "gemm_fp8_nt_256": None,            # operands re-read from L2/MALL: no lower bound here
        "rmsnorm_fp8": 84_414_464,
        "rmsnorm_bwd": 100_671_488,
        "gemv_rowdot_m1": 58_767_488,
        "gemv_fp8_m16": 58_767_488,
        "gemv_fp8_m32": 59_787_264,
        "quant_dual": 270_532_608,
        "xent_fwd": 824_311_808,
        "xent_bwd": 1_648_459_776,
    }
    for key, lo in algorithmic.items():
        assert key in t, key
        if lo is not None:
            assert t[key] >= 0.99 * lo, (key, t[key], lo)


def test_default_warmup_covers_the_clock_ramp():
    """The ~30 ms clock ramp after idle is covered by the untimed clock-settle
    phase that runs before any --warmup the driver asks for (--warmup 5 included)."""
    old = sys.argv
    try:
        sys.argv = ["bench.py"]
        a = bench.parse()
    finally:
        sys.argv = old
    assert a.gpus == 1 and a.warmup >= 1 and a.steps >= 20
    assert bench.CLOCK_SETTLE_MS >= 40
    src = open(bench.__file__).read()
    main = src[src.index("def main():"):]
    # the settle phase precedes the warm-up steps and is reported in the JSON line
    assert main.index("CLOCK_SETTLE_MS") < main.index("range(args.warmup)")
    assert '"clock_settle"' in main


def test_power_sampler_degrades_to_a_reason_without_a_device():
    """Without a GPU (or without amdsmi access) the sustained-clock phase
    reports why it is unavailable instead of failing the bench line."""
    r = bench.PowerSampler().run(lambda: None, 0.01)
    assert set(r) == {"unavailable"} and r["unavailable"]


def test_power_phase_is_skipped_under_rocprofv3(monkeypatch):
    monkeypatch.delenv("ROCPROF_OUTPUT_PATH", raising=False)
    assert not bench.under_profiler()
    monkeypatch.setenv("ROCPROF_OUTPUT_PATH", "/tmp")
    assert bench.under_profiler()
