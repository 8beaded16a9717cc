"""bench.py's contract on the host: the multi-GPU refusal, the algorithmic
flop counts the roofline uses, and the traffic lookup in the committed
counter summary."""
import importlib.util
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def load_bench():
    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_more_than_one_gpu_is_refused_with_a_message():
    p = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert p.returncode == 2
    assert "one GPU" in p.stderr


def test_expert_flops_match_the_mixtral_roofline_figures():
    from moe_amd import synth

    b = load_bench()
    mx = synth.SHAPES["mixtral"]
    # 2·T·k·2·H·I for gate/up, 2·T·k·3·H·I for the layer (BASELINE's 360.8 GFLOP at T=512)
    assert abs(b.expert_flops(mx, 512, 2, up_only=True) - 240.52e9) < 0.01e9
    assert abs(b.expert_flops(mx, 512, 2) - 360.78e9) < 0.01e9
    v2 = synth.SHAPES["v2_lite"]  # the shared expert adds 2·T·3·H·I_s
    assert b.expert_flops(v2, 1, 6) == 2.0 * 6 * 3 * 2048 * 1408 + 2.0 * 3 * 2048 * 2816


def test_traffic_lookup_takes_the_prefill_launch():
    b = load_bench()
    doc = json.load(open(b.TRAFFIC_FILE))
    ups = [k for k in doc["kernels"] if k["kernel"].startswith("mfma_kernel<2, true")]
    assert ups, "the committed summary has the gate/up MFMA kernel"
    biggest = max(ups, key=lambda k: k["grid"])
    assert b.traffic_of("mfma_kernel<2, true") == biggest["hbm_bytes"]
    # The T=512 gate/up launch moves at least the 528.5 MB of weights it reads.
    assert biggest["hbm_bytes"] >= 528.4e6
    assert b.traffic_of("no_such_kernel") is None
