"""Encoder forward, graph replay and checkpoint loading on MI355X.

Parity: sigmoid probabilities of the HIP encoder vs the CPU oracle forward on
the same parameters within 1e-2 absolute (the encoder tolerance); graph replay
vs eager: bitwise identical (reference docs/benchmarks.md:38-41 reports zero
difference between graph and eager).
"""

import pytest
import torch

from oracle.encoder import encoder_forward
from trifusion_amd import runtime
from trifusion_amd.model import Encoder, ModelConfig

pytestmark = pytest.mark.gpu
DEV = "cuda"
PROB_TOL = 1e-2


def make_model(depth=8, seed=0):
    torch.manual_seed(seed)
    model = Encoder(ModelConfig(depth=depth)).eval().requires_grad_(False)
    runtime.prepare_static_weights(model)
    return model.to(DEV)


def clip_audio(b, n, seed=551, channels=1):
    g = torch.Generator().manual_seed(seed)
    audio = torch.randint(-32768, 32768, (b, channels, n), generator=g).float() / 32768
    return audio


def test_configure_runtime_on_gfx950():
    runtime.configure_runtime()
    assert runtime.device_arch() == "gfx950"


def test_encoder_matches_oracle_full_length():
    model = make_model()
    audio = clip_audio(2, 64000)
    lengths = torch.full((2,), 64000)
    channels = torch.ones(2, dtype=torch.int64)
    eng = runtime.InferenceEngine(model)
    logits = eng.eager(audio.to(DEV), lengths.to(DEV), channels.to(DEV)).cpu()
    ref = encoder_forward(model.state_dict(), model.config, audio, lengths, channels)
    diff = (logits.sigmoid() - ref.sigmoid()).abs().max().item()
    print(f"prob max diff {diff:.2e}", flush=True)
    assert torch.isfinite(logits).all() and diff <= PROB_TOL


def test_encoder_matches_oracle_variable_lengths_and_stereo():
    model = make_model(depth=3, seed=1)
    audio = clip_audio(4, 48000, seed=3, channels=2)
    lengths = torch.tensor([48000, 20000, 7000, 31999])
    channels = torch.tensor([2, 1, 2, 1])
    eng = runtime.InferenceEngine(model)
    logits = eng.eager(audio.to(DEV), lengths.to(DEV), channels.to(DEV)).cpu()
    ref = encoder_forward(model.state_dict(), model.config, audio, lengths, channels)
    assert (logits.sigmoid() - ref.sigmoid()).abs().max().item() <= PROB_TOL


def test_graph_replay_equals_eager_across_replays():
    model = make_model()
    audio = clip_audio(16, 64000).to(DEV)
    lengths = torch.full((16,), 64000, device=DEV)
    channels = torch.ones(16, dtype=torch.int64, device=DEV)
    eng = runtime.InferenceEngine(model, graphs=True, max_graphs=1)
    eager = eng.eager(audio, lengths, channels).clone()
    outs = []
    for i in range(4):
        outs.append(eng(audio, lengths, channels))
        # unrelated eager work between replays
        other = clip_audio(16, 64000, seed=10 + i).to(DEV)
        eng.eager(other, lengths, channels)
        torch.cuda.synchronize()
    assert eng.graph_hits == 4
    for o in outs:
        assert torch.equal(o, eager)
    # new inputs through the same graph follow the new data
    other = clip_audio(16, 64000, seed=99).to(DEV)
    assert torch.equal(eng(other, lengths, channels), eng.eager(other, lengths, channels))


def test_load_student_round_trip(tmp_path):
    model = make_model(depth=2, seed=4)
    path = tmp_path / "s.pt"
    runtime.save_student(model.cpu(), path)
    loaded = runtime.load_student(path)
    audio = clip_audio(2, 32000).to(DEV)
    lengths = torch.full((2,), 32000, device=DEV)
    channels = torch.ones(2, dtype=torch.int64, device=DEV)
    a = runtime.InferenceEngine(loaded).eager(audio, lengths, channels)
    b = runtime.InferenceEngine(model.to(DEV)).eager(audio, lengths, channels)
    assert torch.equal(a, b)
    portable = runtime.load_student(path, optimized=False)
    c = runtime.InferenceEngine(portable).eager(audio, lengths, channels)
    assert (c.sigmoid() - a.sigmoid()).abs().max().item() <= PROB_TOL


def make_bidirectional(depth=2, seed=5):
    torch.manual_seed(seed)
    model = Encoder(ModelConfig(depth=depth, bidirectional=True)).eval().requires_grad_(False)
    runtime.prepare_static_weights(model)
    return model.to(DEV)


def test_bidirectional_encoder_matches_oracle():
    """Backward direction via the recurrence's reverse flag vs the oracle's
    explicitly reversed valid prefixes (reference model.py:174-184)."""
    model = make_bidirectional()
    audio = clip_audio(4, 48000, seed=7, channels=2)
    lengths = torch.tensor([48000, 20000, 7000, 31999])
    channels = torch.tensor([2, 1, 2, 1])
    eng = runtime.InferenceEngine(model)
    logits = eng.eager(audio.to(DEV), lengths.to(DEV), channels.to(DEV)).cpu()
    ref = encoder_forward(model.state_dict(), model.config, audio, lengths, channels)
    diff = (logits.sigmoid() - ref.sigmoid()).abs().max().item()
    print(f"bidirectional prob max diff {diff:.2e}", flush=True)
    assert torch.isfinite(logits).all() and diff <= PROB_TOL


def test_bidirectional_graph_replay_equals_eager():
    model = make_bidirectional(seed=6)
    audio = clip_audio(3, 32000, seed=8).to(DEV)
    lengths = torch.tensor([32000, 15000, 800], device=DEV)
    channels = torch.ones(3, dtype=torch.int64, device=DEV)
    eng = runtime.InferenceEngine(model, graphs=True)
    eager = eng.eager(audio, lengths, channels).clone()
    for _ in range(3):
        graph = eng(audio, lengths, channels)
        torch.cuda.synchronize()
        assert torch.equal(graph, eager)
        eng.eager(audio, lengths, channels)
    assert eng.graph_hits >= 2
