"""Offline inference over a submission template on one MI355X.

Behaviour of ``src/trifusion_l4/submission.py:run``: read the template and map
IDs to audio files, plan length-bucketed batches, load the checkpoint with the
static bf16 weight casts, run every batch through the graph engine (a batch
that runs out of HBM is retried file by file, eagerly, after the engine's
graphs are released), write the five sigmoid probabilities in template order
and a JSON runtime report next to it (``<root>/output``).
"""

import json
from pathlib import Path
import resource
import time

import numpy as np
import torch

from .audio import decoded_batches, inspect_audio, plan_batches
from .runtime import InferenceEngine, configure_runtime, load_student
from .submission_format import OUTPUTS, discover_inputs, write_submission


def _logits(engine, inputs):
    try:
        return engine(*inputs)
    except torch.cuda.OutOfMemoryError:
        pass
    # outside the handler, so the failed graph's activations can be released
    engine.clear()
    return torch.cat([engine.eager(*(x[i : i + 1] for x in inputs)) for i in range(inputs[0].shape[0])])


def run(root, weights, graphs=True, padded_seconds=64, max_batch=16, workers=4):
    """Predict every template row of ``root`` with the checkpoint ``weights``;
    returns the runtime report (also written to ``root/output/runtime_report.json``)."""
    start = time.perf_counter()
    configure_runtime(threads=2)
    columns, rows, aliases, paths = discover_inputs(root)
    records = [inspect_audio(i, p) for i, p in enumerate(paths)]
    plan = plan_batches(records, padded_seconds, max_batch, round_buckets=graphs)
    metadata_seconds = time.perf_counter() - start
    torch.cuda.reset_peak_memory_stats()
    model = load_student(weights, optimized=True)
    engine = InferenceEngine(model, graphs=graphs, max_graphs=1)
    model_load_seconds = time.perf_counter() - start - metadata_seconds
    result = np.full((len(rows), len(OUTPUTS)), np.nan, dtype=np.float32)
    seen = np.zeros(len(rows), dtype=bool)
    with torch.inference_mode():
        for batch in decoded_batches(plan, workers):
            indices = batch["indices"]
            if seen[indices].any():
                raise ValueError("An input was scheduled twice")
            inputs = [batch[k].cuda(non_blocking=True) for k in ("audio", "lengths", "channels")]
            result[indices] = _logits(engine, inputs).float().sigmoid().cpu().numpy()
            seen[indices] = True
    if not seen.all():
        raise ValueError("Missing predictions")
    output = Path(root) / "output"
    write_submission(output / "submission.csv", columns, rows, aliases, result)
    report = {
        "files": len(rows),
        "batches": len(plan),
        "wall_seconds": time.perf_counter() - start,
        "metadata_seconds": metadata_seconds,
        "model_load_seconds": model_load_seconds,
        "peak_process_rss_gib": resource.getrusage(resource.RUSAGE_SELF).ru_maxrss / 1024**2,
        "peak_allocated_gib": torch.cuda.max_memory_allocated() / 2**30,
        "peak_reserved_gib": torch.cuda.max_memory_reserved() / 2**30,
        "graph_build_seconds": engine.graph_build_seconds,
        "graph_hits": engine.graph_hits,
        "torch": torch.__version__,
        "gpu": torch.cuda.get_device_name(),
    }
    (output / "runtime_report.json").write_text(json.dumps(report, indent=2) + "\n")
    print(json.dumps(report), flush=True)
    return report
