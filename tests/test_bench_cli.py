"""CPU checks of bench.py's contract pieces that need no GPU: the one-GPU
refusal, the committed profiles it reads its traffic and small-kernel
durations from, the C5 FLOP count and the roofline arithmetic."""

import importlib.util
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "4"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_committed_profiles_cover_what_the_bench_reads():
    b = _bench()
    # small kernels whose roofline comes from the committed kernel trace
    for name, grid in (("gdn_step_kernel", (8, 32, 1)),
                       ("decode_split_f32<64, 32, false>", (4, 8, 1)),
                       ("decode_combine<float, float, 1, 16>", (32, 1, 1)),
                       ("recurrent_rows_kernel<1>", (8, 32, 1)),
                       ("recurrent_finish_kernel<float>", (24, 1, 1))):
        ms = b._trace_avg_ms(name, grid)
        assert ms is not None and 0.0 < ms < 0.05, (name, ms)
    assert b._trace_avg_ms("no_such_kernel", (1, 1, 1)) is None
    traffic = b._measured_traffic()
    assert traffic is not None and 0.95 < traffic["traffic_over_alg"] < 1.2


def test_c5_flops_and_roofline_arithmetic():
    b = _bench()
    # 32 heads x 16 chunks of 2 C^2 (3 Dk + 2 Dv) + 6 C Dk Dv, C = 64, Dk = Dv = 128
    assert b.C5_BASELINE_FLOPS == 5_905_580_032
    r = b._roofline("k", "hbm", 8_000_000_000, 1.0)  # 8 GB in 1 ms = 8 TB/s
    assert r["achieved"] == 8000.0 and r["frac"] == 1.0 and r["unit"] == "GB/s"
    r = b._roofline("k", "mfma", 2_500_000_000, 0.001, work_name="flops")
    assert r["unit"] == "TFLOP/s" and abs(r["frac"] - 1.0) < 1e-9
