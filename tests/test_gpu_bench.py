"""bench.py on a workload other than the headline one: a dense configuration
(no router, the FFN as the one-expert stage) produces a complete JSON line
whose roofline names the plain attention kernel. Runs bench.py as a child
process, a few steps without the CPU baseline."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.gpu
def test_bench_dense_config_line():
    cmd = [sys.executable, os.path.join(ROOT, "bench.py"), "--config", "dense128", "--batch", "2", "--steps", "2",
           "--warmup", "1", "--no-cpu", "--stage-reps", "2"]
    print("running:", " ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=110, cwd=ROOT)
    print(r.stderr[-2000:])
    assert r.returncode == 0, r.stderr[-2000:]
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out["value"] > 0 and out["ms_per_step"] > 0
    assert out["config"]["batch"] == 2 and out["config"]["experts"] == 1
    assert "dense FFN" in out["config"]["workload"]
    # 270 windows: the 8-wave kernel, with the block's FFN in the same launch
    assert out["roofline"]["kernel"] == "prism_attn_d128_w8_ffn"
    assert 0 < out["roofline"]["frac"] < 1
    assert out["roofline"]["chain_launches"]["experts"] is None
    assert out["stages_ms"]["attention_routed"] is None and out["stages_ms"]["router_stage"] is None
    assert out["stages_ms"]["experts"] > 0 and out["stages_ms"]["attention_stage"] > 0
    assert out["expert_load"] is None
    assert out["batch1"]["us_per_frame"] > 0
    assert out["cpu_baseline"] is None
