"""bench.py's host-side contract, on the CPU (no GPU is touched):

- ``--gpus N`` with N > 1 exits with status 2 and a message before anything
  initialises a GPU (this build measures one GPU);
- the documented workloads and flags parse;
- the near-tie rule that judges the first CPU/GPU greedy divergence
  accepts a swap within twice the logit error plus the BF16 rounding of the
  logits and rejects a larger one, the rule tests/test_gpu_model.py applies
  per step."""
import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402  (module level: argparse, json, os, sys, time only)


@pytest.mark.parametrize("gpus", [2, 8])
def test_more_than_one_gpu_is_refused(gpus):
    done = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", str(gpus)],
                          capture_output=True, text=True, timeout=120,
                          env=dict(os.environ, HIP_VISIBLE_DEVICES=""))
    assert done.returncode == 2, done.stderr
    assert done.stdout == ""
    assert "one GPU" in done.stderr and f"--gpus {gpus}" in done.stderr


@pytest.mark.parametrize("argv, expect", [
    ([], {"workload": "e2e", "steps": 10, "warmup": 2, "prompt": 512, "decode_tokens": 0,
          "graph": "on"}),
    (["--workload", "gemv"], {"steps": 200, "warmup": 20, "launch": "plan"}),
    (["--workload", "prefill", "--tokens", "128", "--dtype", "bf16"],
     {"steps": 200, "tokens": 128, "dtype": "bf16"}),
    (["--workload", "ttft", "--prompt", "32"], {"steps": 20, "warmup": 5, "prompt": 32}),
    (["--workload", "tile", "--shape", "4096,1024,896", "--dtype", "bf16"],
     {"workload": "tile", "shape": "4096,1024,896", "dtype": "bf16"}),
    (["--steps", "3", "--warmup", "0", "--graph", "off", "--decode-tokens", "32"],
     {"steps": 3, "warmup": 0, "graph": "off", "decode_tokens": 32}),
])
def test_flags_parse(monkeypatch, argv, expect):
    monkeypatch.setattr(sys, "argv", ["bench.py", *argv])
    args = bench.parse()
    for k, v in expect.items():
        assert getattr(args, k) == v, (k, getattr(args, k), v)


def test_near_tie_rule():
    rng = np.random.default_rng(5)
    ref = rng.uniform(-5.0, 5.0, 1000)           # every other logit below 10 in size
    ref[7], ref[9] = 10.0, 9.98                  # oracle picks 7, 9 is 0.02 behind
    # BF16 rounding of the logits alone: 2^-8 * max|ref| = 0.039 > 0.02
    near = bench.near_tie_rule(ref.copy(), ref, 9, 7)
    assert near["near_tie"] and near["margin"] == pytest.approx(0.02)
    assert near["bound"] == pytest.approx(2.0 ** -8 * 10.0)
    far_ref = ref.copy()
    far_ref[9] = 9.0                               # 1.0 behind: not a tie
    far = bench.near_tie_rule(far_ref.copy(), far_ref, 9, 7)
    assert not far["near_tie"]
    # a logit error of 0.5 on one entry widens the bound by 1.0
    gpu = far_ref.copy()
    gpu[500] += 0.5
    widened = bench.near_tie_rule(gpu, far_ref, 9, 7)
    assert widened["bound"] == pytest.approx(1.0 + 2.0 ** -8 * 10.0)
    assert widened["near_tie"]
    assert widened["logits_cosine"] <= 1.0


def test_stats_of():
    s = bench.stats_of([1.0, 2.0, 3.0, 4.0, 100.0])
    assert s == {"mean": 22.0, "p50": 3.0, "p95": 80.8}
