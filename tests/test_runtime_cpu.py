"""Host-side runtime logic without a GPU: checkpoint format and loading, and the
graph engine's cache / fallback policy (reference src/trifusion_l4/runtime.py)."""

import pytest
import torch

from trifusion_amd import runtime
from trifusion_amd.model import Encoder, ModelConfig

SMALL = dict(dim=64, depth=2, ffn_dim=96, state_dim=32, head_dim=32)


def small_model():
    torch.manual_seed(0)
    return Encoder(ModelConfig(**SMALL)).eval()


def test_checkpoint_round_trip(tmp_path):
    model = small_model()
    path = tmp_path / "student.pt"
    runtime.save_student(model, path)
    loaded = runtime.load_student(path, optimized=True, device="cpu")
    assert not any(p.requires_grad for p in loaded.parameters())
    assert loaded.blocks[0].gate_up.weight.dtype == torch.bfloat16  # GEMM weights cast once
    assert loaded.blocks[0].ff_norm.weight.dtype == torch.float32  # norms stay fp32
    assert loaded.blocks[0].mamba.dt_bias.dtype == torch.float32
    ref = model.state_dict()
    for k, v in loaded.state_dict().items():
        assert torch.equal(v.float(), ref[k].to(v.dtype).float()), k
    assert loaded.blocks[1].mamba.variant == "auto"
    assert runtime.load_student(path, optimized=False, device="cpu").blocks[0].mamba.variant == "generic"


def test_unknown_config_fields_rejected(tmp_path):
    model = small_model()
    path = tmp_path / "bad.pt"
    config = dict(SMALL, not_a_field=1)
    torch.save({"model_config": config, "model": model.state_dict()}, path)
    with pytest.raises(ValueError):
        runtime.load_student(path, device="cpu")


def test_training_only_keys_are_stripped_and_strict(tmp_path):
    model = small_model()
    state = dict(model.state_dict())
    state["memory_head.weight"] = torch.zeros(2, 2)
    state["kd_features.x"] = torch.zeros(1)
    path = tmp_path / "train.pt"
    torch.save({"model_config": SMALL, "model": state}, path)
    runtime.load_student(path, device="cpu")
    del state["head.bias"]
    torch.save({"model_config": SMALL, "model": state}, path)
    with pytest.raises(RuntimeError):
        runtime.load_student(path, device="cpu")


class FakeModel(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.calls = 0

    def forward(self, audio, lengths, channels):
        self.calls += 1
        return {"logits": audio.sum(-1)[:, :1].repeat(1, 5) + lengths[:, None].float()}


class FakeGraph:
    def __init__(self, fn):
        self.fn = fn
        self.replays = 0

    def replay(self):
        self.replays += 1
        self.fn()


@pytest.fixture
def fake_cuda(monkeypatch):
    state = {"reserved": 0, "oom": False}
    monkeypatch.setattr(torch.cuda, "empty_cache", lambda: None)
    monkeypatch.setattr(torch.cuda, "memory_reserved", lambda *a, **k: state["reserved"])

    def capture(self, x, l, c):
        if state["oom"]:
            raise torch.cuda.OutOfMemoryError("planted")
        out = self.model(x, l, c)["logits"].clone()
        return FakeGraph(lambda: out.copy_(self.model(x, l, c)["logits"])), out

    monkeypatch.setattr(runtime.InferenceEngine, "_capture", capture)
    monkeypatch.setattr(runtime.InferenceEngine, "eager", lambda self, a, l, c: self.model(a, l, c)["logits"])
    return state


def inputs(b=2, n=10, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.rand(b, 1, n, generator=g), torch.full((b,), n), torch.ones(b, dtype=torch.int64)


def test_engine_eager_when_graphs_off(fake_cuda):
    eng = runtime.InferenceEngine(FakeModel(), graphs=False)
    out = eng(*inputs())
    assert out.shape == (2, 5) and eng.graph_hits == 0 and not eng.cache


def test_engine_captures_once_and_replays(fake_cuda):
    model = FakeModel()
    eng = runtime.InferenceEngine(model, graphs=True)
    a = inputs(seed=1)
    first = eng(*a)
    second = eng(*inputs(seed=2))
    assert eng.graph_hits == 2 and len(eng.cache) == 1
    assert torch.equal(second, FakeModel()(*inputs(seed=2))["logits"])
    assert first.data_ptr() != second.data_ptr()  # owned results
    assert torch.equal(first, FakeModel()(*a)["logits"])  # not overwritten by the later replay


def test_engine_lru_eviction(fake_cuda):
    eng = runtime.InferenceEngine(FakeModel(), graphs=True, max_graphs=1)
    eng(*inputs(n=10))
    eng(*inputs(n=12))
    assert len(eng.cache) == 1 and list(eng.cache)[0][0] == (2, 1, 12)


def test_engine_oom_at_capture_disables_shape(fake_cuda):
    fake_cuda["oom"] = True
    eng = runtime.InferenceEngine(FakeModel(), graphs=True)
    out = eng(*inputs())
    assert out.shape == (2, 5)
    assert ((2, 1, 10), torch.float32) in eng.disabled_shapes and not eng.cache
    fake_cuda["oom"] = False
    eng(*inputs())
    assert eng.graph_hits == 0  # stays eager for that shape


def test_engine_reserved_limit_disables_shape(fake_cuda):
    fake_cuda["reserved"] = 10 * 2**30
    eng = runtime.InferenceEngine(FakeModel(), graphs=True, max_reserved_gib=1)
    eng(*inputs())
    assert ((2, 1, 10), torch.float32) in eng.disabled_shapes and eng.graph_hits == 0


def test_configure_runtime_requires_gpu(monkeypatch):
    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    with pytest.raises(RuntimeError):
        runtime.configure_runtime()
