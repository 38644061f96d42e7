"""Checkpoint loading, runtime configuration and hipGraph replay engine.

Same API and policies as the reference runtime (``src/trifusion_l4/runtime.py``):

``load_student(path, optimized=True, device="cuda")`` (``:11-47``)
    Reads a local model-only checkpoint ``{"model_config": {...}, "model": state}``
    with ``torch.load(weights_only=True, mmap=True)``, rejects unknown config
    keys, builds the model on the meta device, attaches the tensors with
    ``load_state_dict(strict=True, assign=True)``, freezes it and casts the GEMM
    weights to bf16. ``optimized=False`` selects the generic (fp32-FMA) recurrence
    kernel instead of the MFMA chunked scan.
``configure_runtime(threads=2, enforce_gfx950=True)`` (``:57-65``)
    Requires a ROCm GPU, by default a gfx950 (MI355X) one, sets the host thread
    count and disables TF32 and convolution autotuning.
``InferenceEngine(model, graphs=False, max_graphs=2, max_reserved_gib=19.5)`` (``:68-138``)
    LRU cache of captured graphs keyed on the audio shape and dtype; two warm-up
    passes on a side stream, one capture, inputs copied into static buffers and
    ``graph.replay()`` per call; an out-of-memory during capture or a reserved
    pool above the limit disables graphs for that shape and falls back to eager.
    On ROCm ``torch.cuda.CUDAGraph`` records a hipGraph.
"""

import gc
import time
from collections import OrderedDict
from dataclasses import fields

import torch

from .model import Encoder, ModelConfig
from .trifusion import TriFusion, TriFusionConfig, eager_forks


def _model_kind(config):
    """The TriFusion layout when the configuration's fields are those of the
    reference model (``model.py:14-34``), else the benchmark encoder."""
    keys = set(config)
    if keys <= {f.name for f in fields(TriFusionConfig)} and keys & {"heads", "evidence_rank", "backend"}:
        return TriFusion, TriFusionConfig
    if keys <= {f.name for f in fields(ModelConfig)}:
        return Encoder, ModelConfig
    raise ValueError("Unsupported model configuration fields")


def load_student(path, optimized=True, device="cuda"):
    saved = torch.load(path, map_location="cpu", weights_only=True, mmap=True)
    config = dict(saved["model_config"])
    cls, cfg = _model_kind(config)
    with torch.device("meta"):
        model = cls(cfg(**config))
    if cls is TriFusion:
        # the training-only head is not part of the deployed network (runtime.py:33-40)
        del model.memory_head
    state = {
        k: v for k, v in saved["model"].items() if not k.startswith(("kd_features.", "memory_head."))
    }
    model.load_state_dict(state, strict=True, assign=True)
    if cls is TriFusion:
        # the STFT window is a non-persistent buffer: materialise it (runtime.py:41-42)
        model.front.window = torch.hann_window(400, periodic=True)
    model.eval().requires_grad_(False)
    model.set_variant("auto" if optimized else "generic")
    if optimized:
        prepare_static_weights(model)
    return model.to(device)


def save_student(model, path):
    """Write a model-only checkpoint in the format ``load_student`` reads."""
    config = {f.name: getattr(model.config, f.name) for f in fields(type(model.config))}
    torch.save({"model_config": config, "model": model.state_dict()}, path)


# Layers whose weights feed a GEMM (or an implicit-GEMM convolution).
_MATMUL_LAYERS = (torch.nn.Linear, torch.nn.Conv1d, torch.nn.Conv2d)


def prepare_static_weights(model):
    """Store the weights of every matrix-product layer (linear, 1-d and 2-d
    convolution) in bf16 once, the dtype the autocast forward feeds its GEMMs,
    instead of casting them on every call. Norm weights and the recurrence's
    control parameters are not matrix-product layers and keep fp32."""
    for layer in model.modules():
        if isinstance(layer, _MATMUL_LAYERS):
            layer.to(dtype=torch.bfloat16)


def device_arch(index=0):
    return torch.cuda.get_device_properties(index).gcnArchName.split(":")[0]


def configure_runtime(threads=2, enforce_gfx950=True):
    """Process settings for inference: a ROCm GPU is required (a gfx950 one
    unless ``enforce_gfx950`` is False), ``threads`` host threads, fp32 GEMMs
    and convolutions without TF32, and no convolution autotuning (the same
    algorithms run in every call, so a captured graph matches the eager
    forward)."""
    if not torch.cuda.is_available():
        raise RuntimeError("A ROCm GPU is required")
    arch = device_arch()
    if enforce_gfx950 and arch != "gfx950":
        raise RuntimeError(f"This runtime is built for MI355X (gfx950), not {arch}")
    torch.set_num_threads(threads)
    flags = torch.backends
    flags.cuda.matmul.allow_tf32 = False
    flags.cudnn.allow_tf32 = False
    flags.cudnn.benchmark = False


def _release_cached_memory():
    gc.collect()
    torch.cuda.empty_cache()


class _Replay:
    """A captured forward: its graph, the static input tensors the graph reads
    and the logits buffer it writes."""

    __slots__ = ("graph", "static_inputs", "logits")

    def __init__(self, graph, static_inputs, logits):
        self.graph = graph
        self.static_inputs = static_inputs
        self.logits = logits

    def run(self, *inputs):
        for dst, src in zip(self.static_inputs, inputs):
            dst.copy_(src)
        self.graph.replay()
        # the caller owns its result: the next replay rewrites the buffer
        return self.logits.clone()


class InferenceEngine:
    """Runs a frozen model's forward, replaying captured graphs when ``graphs``.

    Graphs are cached per (audio shape, audio dtype), at most ``max_graphs`` of
    them, the least recently used one dropped first. A shape whose capture
    runs out of memory, or after whose capture torch's reserved pool exceeds
    ``max_reserved_gib``, is marked in ``disabled_shapes`` and runs eagerly from
    then on. ``graph_hits`` counts replays and ``graph_build_seconds`` the time
    spent building graphs. Calls are not thread-safe: serialise them.
    """

    def __init__(self, model, graphs=False, max_graphs=2, max_reserved_gib=19.5):
        self.model = model
        self.graphs = graphs
        self.max_graphs = max_graphs
        self.limit = int(max_reserved_gib * 2**30)
        self.cache = OrderedDict()
        self.disabled_shapes = set()
        self.graph_build_seconds = 0.0
        self.graph_hits = 0

    @torch.inference_mode()
    def eager(self, audio, lengths, channels):
        """One forward without a graph under bf16 autocast; the logits."""
        with torch.autocast("cuda", dtype=torch.bfloat16):
            result = self.model(audio, lengths, channels)
        return result["logits"]

    def clear(self):
        """Drop every cached graph and return the memory to the device."""
        self.cache.clear()
        _release_cached_memory()

    def _capture(self, audio, lengths, channels):
        """Record one forward reading ``audio``/``lengths``/``channels`` into a
        graph. Two eager forwards on a side stream come first, forking onto the
        branch streams as the capture will, so kernels are loaded and library
        handles and workspaces exist on every stream before capture."""
        caller = torch.cuda.current_stream()
        side = torch.cuda.Stream()
        side.wait_stream(caller)
        with torch.cuda.stream(side), eager_forks():
            self.eager(audio, lengths, channels)
            self.eager(audio, lengths, channels)
        caller.wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            logits = self.eager(audio, lengths, channels)
        return graph, logits

    def _disable(self, shape_key):
        self.disabled_shapes.add(shape_key)
        self.clear()

    def _build(self, shape_key, inputs):
        """Capture a graph for ``shape_key`` on copies of ``inputs``; None when
        the shape has to run eagerly instead."""
        while len(self.cache) >= self.max_graphs:
            self.cache.popitem(last=False)
        _release_cached_memory()
        began = time.perf_counter()
        static_inputs = tuple(t.clone() for t in inputs)
        try:
            graph, logits = self._capture(*static_inputs)
        except torch.cuda.OutOfMemoryError:
            static_inputs = None
            self._disable(shape_key)
            return None
        self.graph_build_seconds += time.perf_counter() - began
        if torch.cuda.memory_reserved() > self.limit:
            graph = logits = static_inputs = None
            self._disable(shape_key)
            return None
        replay = _Replay(graph, static_inputs, logits)
        self.cache[shape_key] = replay
        return replay

    @torch.inference_mode()
    def __call__(self, audio, lengths, channels):
        shape_key = (tuple(audio.shape), audio.dtype)
        if self.graphs and shape_key not in self.disabled_shapes:
            replay = self.cache.get(shape_key)
            if replay is None:
                replay = self._build(shape_key, (audio, lengths, channels))
            if replay is not None:
                self.cache.move_to_end(shape_key)
                self.graph_hits += 1
                return replay.run(audio, lengths, channels)
        return self.eager(audio, lengths, channels)
