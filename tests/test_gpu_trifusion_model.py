"""The TriFusion-FP model (reference layout) on MI355X against the oracle's CPU
forward of the same state dict: sigmoid probabilities within 1e-2 (the model
tolerance), graph replay (with its side-stream branches) bitwise equal to the
one-stream eager forward, and a save/load round trip
through ``load_student``."""

import pytest
import torch

from oracle.trifusion_model import trifusion_forward
from trifusion_amd import runtime, trifusion
from trifusion_amd.trifusion import TriFusion, TriFusionConfig

pytestmark = pytest.mark.gpu
DEV = "cuda"
PROB_TOL = 1e-2
SMALL = dict(dim=128, depth=2, heads=4, ffn_dim=256, state_dim=64, evidence_rank=16)


def make_model(seed=0, **cfg):
    torch.manual_seed(seed)
    model = TriFusion(TriFusionConfig(**{**SMALL, **cfg})).eval().requires_grad_(False)
    with torch.no_grad():
        # the reference initialises the evidence and merge gates to zero; random
        # gates exercise the gated kernels inside the forward
        for blk in model.blocks:
            for layer in (blk.e_gate, blk.gate):
                layer.weight.normal_(std=0.05)
                layer.bias.normal_(std=0.5)
    del model.memory_head
    runtime.prepare_static_weights(model)
    return model.to(DEV)


def inputs(b=3, n=32000, seed=7):
    g = torch.Generator().manual_seed(seed)
    audio = torch.randint(-32768, 32768, (b, 2, n), generator=g).float() / 32768
    lengths = torch.tensor([n, 20000, 9000][:b])
    channels = torch.tensor([2, 1, 2][:b])
    return audio, lengths, channels


def test_trifusion_matches_oracle(monkeypatch):
    model = make_model()
    audio, lengths, channels = inputs()
    eng = runtime.InferenceEngine(model)
    # the fused block and front-stage kernels are the path under test
    calls = {"block": 0, "stage": 0}
    block_fused, stage = type(model.blocks[0]).forward_fused, trifusion.front_stage

    def count_block(*a, **k):
        calls["block"] += 1
        return block_fused(*a, **k)

    def count_stage(*a, **k):
        calls["stage"] += 1
        return stage(*a, **k)

    monkeypatch.setattr(type(model.blocks[0]), "forward_fused", count_block)
    monkeypatch.setattr(trifusion, "front_stage", count_stage)
    out = eng.eager(audio.to(DEV), lengths.to(DEV), channels.to(DEV)).cpu()
    assert calls == {"block": SMALL["depth"], "stage": 3}
    ref = trifusion_forward(model.state_dict(), model.config, audio, lengths, channels)
    diff = (out.sigmoid() - ref.sigmoid()).abs().max().item()
    print(f"trifusion prob max diff {diff:.2e}", flush=True)
    assert out.shape == (3, 5) and torch.isfinite(out).all()
    assert diff <= PROB_TOL


def test_trifusion_graph_replay_equals_eager(monkeypatch):
    """The captured graph forks the attention branches and the fine reads onto
    side streams (eager calls do not): every replay, with eager forwards of
    other inputs between them, equals the one-stream eager forward bitwise."""
    model = make_model(seed=1)
    audio, lengths, channels = (t.to(DEV) for t in inputs(seed=8))
    other = [t.to(DEV) for t in inputs(seed=10)]
    forks = []
    branch = trifusion.branch_stream

    def count_fork(device, slot=0):
        forks.append(slot)
        return branch(device, slot)

    monkeypatch.setattr(trifusion, "branch_stream", count_fork)
    eng = runtime.InferenceEngine(model, graphs=True)
    eager = eng.eager(audio, lengths, channels).clone()
    assert forks == []
    with trifusion.eager_forks():
        assert torch.equal(eng.eager(audio, lengths, channels), eager)
    assert sorted(set(forks)) == [0, 1]
    forks.clear()
    for _ in range(3):
        graph = eng(audio, lengths, channels)
        torch.cuda.synchronize()
        assert torch.equal(graph, eager)
        eng.eager(*other)
        torch.cuda.synchronize()
    assert eng.graph_hits >= 2
    # two forked warm-ups and the capture
    assert sorted(set(forks)) == [0, 1] and forks.count(0) == 3 * SMALL["depth"]


def test_short_clips_through_the_forked_graph():
    """0.2 s and 0.1 s clips (a few frames after the front end, one recurrence
    chunk, grids of one or two pooled rows): eager against the oracle, and the
    forked graph's replay bitwise against eager."""
    model = make_model(seed=5)
    g = torch.Generator().manual_seed(13)
    audio = torch.randint(-32768, 32768, (2, 1, 3200), generator=g).float() / 32768
    lengths, channels = torch.tensor([3200, 1600]), torch.tensor([1, 1])
    eng = runtime.InferenceEngine(model, graphs=True)
    dev = [t.to(DEV) for t in (audio, lengths, channels)]
    eager = eng.eager(*dev).clone()
    ref = trifusion_forward(model.state_dict(), model.config, audio, lengths, channels)
    diff = (eager.cpu().sigmoid() - ref.sigmoid()).abs().max().item()
    print(f"short clips prob max diff {diff:.2e}", flush=True)
    assert torch.isfinite(eager).all() and diff <= PROB_TOL
    for _ in range(2):
        graph = eng(*dev)
        torch.cuda.synchronize()
        assert torch.equal(graph, eager)


def test_forks_switched_off(monkeypatch):
    """With the branch forks switched off the captured forward stays on the
    caller's stream, and its replays still equal the eager forward bitwise."""
    model = make_model(seed=3)
    for blk in model.blocks:
        blk.branch_streams = False
    model.fork_fine = False
    audio, lengths, channels = (t.to(DEV) for t in inputs(seed=11))
    forks = []
    branch = trifusion.branch_stream

    def count_fork(device, slot=0):
        forks.append(slot)
        return branch(device, slot)

    monkeypatch.setattr(trifusion, "branch_stream", count_fork)
    eng = runtime.InferenceEngine(model, graphs=True)
    eager = eng.eager(audio, lengths, channels).clone()
    for _ in range(2):
        graph = eng(audio, lengths, channels)
        torch.cuda.synchronize()
        assert torch.equal(graph, eager)
    assert forks == [] and eng.graph_hits >= 1


def test_capture_error_in_a_fork_falls_back(monkeypatch):
    """An out-of-memory error raised inside the forked attention branch while
    the graph is captured: the side stream is joined back on the way out, so
    the capture ends cleanly, the engine sees the error, disables the shape
    and answers eagerly; the streams stay usable."""
    model = make_model(seed=4)
    audio, lengths, channels = (t.to(DEV) for t in inputs(seed=12))
    eng = runtime.InferenceEngine(model, graphs=True)
    eager = eng.eager(audio, lengths, channels).clone()
    cls = type(model.blocks[0])
    branch = cls._attention_branch

    def fail_in_capture(self, p, grids):
        if torch.cuda.is_current_stream_capturing():
            raise torch.cuda.OutOfMemoryError("forced inside the captured attention branch")
        return branch(self, p, grids)

    monkeypatch.setattr(cls, "_attention_branch", fail_in_capture)
    out = eng(audio, lengths, channels)
    torch.cuda.synchronize()
    assert torch.equal(out, eager)
    assert len(eng.disabled_shapes) == 1 and eng.graph_hits == 0
    monkeypatch.setattr(cls, "_attention_branch", branch)
    with trifusion.eager_forks():
        forked = eng.eager(audio, lengths, channels)
    torch.cuda.synchronize()
    assert torch.equal(forked, eager)


def test_load_student_round_trip(tmp_path):
    torch.manual_seed(2)
    model = TriFusion(TriFusionConfig(**SMALL)).eval()
    path = tmp_path / "student.pt"
    runtime.save_student(model, path)
    loaded = runtime.load_student(path, device=DEV)
    assert isinstance(loaded, TriFusion) and not hasattr(loaded, "memory_head")
    sd = model.state_dict()
    for k, v in loaded.state_dict().items():
        assert torch.equal(v.float().cpu(), sd[k].to(v.dtype).float()), k
    audio, lengths, channels = (t.to(DEV) for t in inputs(seed=9))
    out = runtime.InferenceEngine(loaded).eager(audio, lengths, channels)
    assert torch.isfinite(out).all()
