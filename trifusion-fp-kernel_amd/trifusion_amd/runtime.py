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
from .trifusion import TriFusion, TriFusionConfig


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


def prepare_static_weights(model):
    """Cast frozen GEMM/conv parameters once; normalization and controls stay fp32."""
    for module in model.modules():
        if isinstance(module, (torch.nn.Linear, torch.nn.Conv1d, torch.nn.Conv2d)):
            module.to(dtype=torch.bfloat16)


def device_arch(index=0):
    return torch.cuda.get_device_properties(index).gcnArchName.split(":")[0]


def configure_runtime(threads=2, enforce_gfx950=True):
    if not torch.cuda.is_available():
        raise RuntimeError("A ROCm GPU is required")
    if enforce_gfx950 and device_arch() != "gfx950":
        raise RuntimeError("This runtime is built for MI355X (gfx950)")
    torch.set_num_threads(threads)
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    torch.backends.cudnn.benchmark = False


class InferenceEngine:
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
        with torch.autocast("cuda", dtype=torch.bfloat16):
            return self.model(audio, lengths, channels)["logits"]

    def clear(self):
        self.cache.clear()
        gc.collect()
        torch.cuda.empty_cache()

    def _capture(self, x, lengths, channels):
        """Warm up on a side stream, then record one forward into a graph."""
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            for _ in range(2):
                self.eager(x, lengths, channels)
        torch.cuda.current_stream().wait_stream(stream)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = self.eager(x, lengths, channels)
        return graph, out

    @torch.inference_mode()
    def __call__(self, audio, lengths, channels):
        key = (tuple(audio.shape), audio.dtype)
        if not self.graphs or key in self.disabled_shapes:
            return self.eager(audio, lengths, channels)
        if key not in self.cache:
            while len(self.cache) >= self.max_graphs:
                self.cache.popitem(last=False)
            gc.collect()
            torch.cuda.empty_cache()
            start = time.perf_counter()
            x = audio.clone()
            l = lengths.clone()
            c = channels.clone()
            try:
                graph, out = self._capture(x, l, c)
            except torch.cuda.OutOfMemoryError:
                del x, l, c
                self.clear()
                self.disabled_shapes.add(key)
                return self.eager(audio, lengths, channels)
            self.graph_build_seconds += time.perf_counter() - start
            if torch.cuda.memory_reserved() > self.limit:
                del graph, out, x, l, c
                self.clear()
                self.disabled_shapes.add(key)
                return self.eager(audio, lengths, channels)
            self.cache[key] = (graph, x, l, c, out)
        graph, x, l, c, out = self.cache[key]
        self.cache.move_to_end(key)
        x.copy_(audio)
        l.copy_(lengths)
        c.copy_(channels)
        graph.replay()
        self.graph_hits += 1
        # a later replay overwrites the graph's output buffer
        return out.clone()
