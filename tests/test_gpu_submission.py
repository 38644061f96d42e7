"""End to end on MI355X: ``trifusion-amd predict`` over a template directory
(WAV decoding, length buckets, the graph engine, the CSV writer) against the
oracle forward of each file on its own at its own length. Tolerance: sigmoid
probabilities within 1e-2 (as the model's parity test)."""

import csv
import json
import wave

import numpy as np
import pytest
import torch

from oracle.trifusion_model import trifusion_forward
from trifusion_amd import cli, runtime
from trifusion_amd.submission_format import OUTPUTS
from trifusion_amd.trifusion import TriFusion, TriFusionConfig

pytestmark = pytest.mark.gpu
SMALL = dict(dim=128, depth=2, heads=4, ffn_dim=256, state_dim=64, evidence_rank=16)
COLUMNS = ["ID", "VOICE_PRESENT_PROB", "FILE_FAKE_PROB", "MUSIC_PRESENT_PROB", "MUSIC_FAKE_PROB", "VOICE_FAKE_PROB"]
FILES = [("b", 16001, 1), ("a", 32000, 2), ("c", 64001, 1)]


def fixture(root):
    rng = np.random.default_rng(3)
    (root / "data/test").mkdir(parents=True)
    clips = {}
    for name, n, ch in FILES:
        ints = rng.integers(-12000, 12000, (n, ch)).astype("<i2")
        with wave.open(str(root / "data/test" / f"{name}.wav"), "wb") as w:
            w.setnchannels(ch)
            w.setsampwidth(2)
            w.setframerate(16000)
            w.writeframes(ints.tobytes())
        clips[name] = torch.from_numpy(ints.T.astype(np.float32) / 32768)
    with (root / "data/sample_submission.csv").open("w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=COLUMNS)
        w.writeheader()
        for name, _, _ in FILES:
            w.writerow({**dict.fromkeys(COLUMNS, 0), "ID": name})
    return clips


def test_predict_matches_oracle(tmp_path):
    clips = fixture(tmp_path)
    torch.manual_seed(5)
    model = TriFusion(TriFusionConfig(**SMALL)).eval()
    with torch.no_grad():
        for blk in model.blocks:
            for layer in (blk.e_gate, blk.gate):
                layer.weight.normal_(std=0.05)
                layer.bias.normal_(std=0.5)
    weights = tmp_path / "student.pt"
    runtime.save_student(model, weights)
    assert cli.main(["predict", "--weights", str(weights), "--root", str(tmp_path), "--padded-seconds", "8",
                     "--max-batch", "2", "--workers", "2"]) == 0
    with (tmp_path / "output/submission.csv").open() as f:
        reader = csv.DictReader(f)
        rows = list(reader)
        assert reader.fieldnames == COLUMNS
    assert [r["ID"] for r in rows] == [name for name, _, _ in FILES]
    report = json.loads((tmp_path / "output/runtime_report.json").read_text())
    assert report["files"] == 3 and report["batches"] == 3
    sd = torch.load(weights, weights_only=True)["model"]
    cfg = TriFusionConfig(**SMALL)
    worst = 0.0
    for row, (name, n, ch) in zip(rows, FILES):
        ref = trifusion_forward(sd, cfg, clips[name][None], torch.tensor([n]), torch.tensor([ch])).sigmoid()[0]
        got = torch.tensor([float(row[col]) for col in ("FILE_FAKE_PROB", "VOICE_FAKE_PROB", "MUSIC_FAKE_PROB",
                                                        "VOICE_PRESENT_PROB", "MUSIC_PRESENT_PROB")])
        worst = max(worst, (got - ref).abs().max().item())
    print(f"predict prob max diff {worst:.2e}", flush=True)
    assert worst <= 1e-2
    assert len(OUTPUTS) == 5
