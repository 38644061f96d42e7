"""The parts of the ``bench.py`` contract that need no GPU: the one-GPU refusal,
the clip workload's algorithmic bytes (48,750,656 B per call: unique inputs
plus the bf16 output), and the HBM traffic and utilisation figures read from
the committed rocprofv3 summaries."""

import subprocess
import sys
from pathlib import Path

import torch

import bench
from trifusion_amd.synthetic import algorithmic_bytes, clip_inputs

ROOT = Path(__file__).resolve().parent.parent


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)


def test_clip_algorithmic_bytes():
    w = bench.WORKLOAD
    args = clip_inputs(w["batch"], w["time"], heads=w["heads"], head_dim=w["head_dim"], state=w["state"],
                       rotary=w["rotary"], qk_heads=w["qk_heads"])
    assert algorithmic_bytes(args, out_dtype=torch.bfloat16) == 48_750_656


def test_committed_profile_figures_parse():
    traffic = bench.traffic_bytes()
    # reads are the input bytes; the streaming output stores write some 128-byte lines in parts
    assert traffic is not None and 48_750_656 <= traffic < 1.10 * 48_750_656
    counters = bench.utilisation_counters()
    assert counters is not None and 0 < counters["MfmaUtil"] < 100 and 0 < counters["VALUBusy"] < 100
