"""Offline scoring of a submission template on one MI355X.

The job the reference's ``trifusion-l4 predict`` performs
(src/trifusion_l4/submission.py:16-73), built here from four pieces:

* ``_Stopwatch`` splits the wall time into the phases the report names
  (template and header scan, checkpoint load);
* ``_Scores`` holds one row of five probabilities per template row and accepts
  each row exactly once, so a planner mistake (a file scored twice, or never)
  fails the job instead of writing a wrong CSV;
* ``_score_bucket`` runs one length bucket through the graph engine; when the
  bucket's graph does not fit in HBM it drops the cached graphs and scores the
  bucket's files one at a time with eager launches;
* ``run`` wires them together and writes ``output/submission.csv`` (template
  row and column order, ``submission_format.write_submission``) and
  ``output/runtime_report.json`` with the keys in ``REPORT_KEYS``.
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

# runtime_report.json, in this order (reference src/trifusion_l4/submission.py:57-70)
REPORT_KEYS = ("files", "batches", "wall_seconds", "metadata_seconds", "model_load_seconds", "peak_process_rss_gib",
               "peak_allocated_gib", "peak_reserved_gib", "graph_build_seconds", "graph_hits", "torch", "gpu")
GIB = float(1 << 30)


class _Stopwatch:
    def __init__(self):
        self.origin = self.mark = time.perf_counter()

    def split(self):
        """Seconds since the previous split (or since construction)."""
        now = time.perf_counter()
        elapsed, self.mark = now - self.mark, now
        return elapsed

    def total(self):
        return time.perf_counter() - self.origin


class _Scores:
    def __init__(self, rows):
        self.table = np.full((rows, len(OUTPUTS)), np.nan, dtype=np.float32)
        self.done = np.zeros(rows, dtype=bool)

    def fill(self, rows, probabilities):
        rows = np.asarray(rows, dtype=np.int64)
        repeated = np.unique(rows).size != rows.size or self.done[rows].any()
        if repeated:
            raise RuntimeError(f"batch plan scores template rows {rows.tolist()} more than once")
        self.table[rows] = probabilities
        self.done[rows] = True

    def result(self):
        absent = np.flatnonzero(~self.done)
        if absent.size:
            raise RuntimeError(f"{absent.size} template rows were never scored (first: row {absent[0]})")
        return self.table


def _score_bucket(engine, audio, lengths, channels):
    """Sigmoid probabilities ``[B, 5]`` (float32, host) of one padded bucket."""
    try:
        logits = engine(audio, lengths, channels)
    except torch.cuda.OutOfMemoryError:
        logits = None  # the handler's frame holds the failed capture; release it first
    if logits is None:
        engine.clear()
        logits = torch.empty(audio.shape[0], len(OUTPUTS), device=audio.device)
        for i in range(audio.shape[0]):
            one = slice(i, i + 1)
            logits[one] = engine.eager(audio[one], lengths[one], channels[one]).float()
    return logits.float().sigmoid().cpu().numpy()


def run(root, weights, graphs=True, padded_seconds=64, max_batch=16, workers=4):
    """Score every template row under ``root`` with the checkpoint ``weights``;
    returns the runtime report, also written to ``root/output/runtime_report.json``."""
    clock = _Stopwatch()
    configure_runtime(threads=2)
    columns, rows, aliases, paths = discover_inputs(root)
    plan = plan_batches([inspect_audio(i, p) for i, p in enumerate(paths)], padded_seconds, max_batch,
                        round_buckets=graphs)
    scan_seconds = clock.split()

    torch.cuda.reset_peak_memory_stats()
    engine = InferenceEngine(load_student(weights, optimized=True), graphs=graphs, max_graphs=1)
    load_seconds = clock.split()

    scores = _Scores(len(rows))
    with torch.inference_mode():
        for bucket in decoded_batches(plan, workers):
            device_inputs = (bucket[name].to("cuda", non_blocking=True) for name in ("audio", "lengths", "channels"))
            scores.fill(bucket["indices"], _score_bucket(engine, *device_inputs))

    destination = Path(root) / "output"
    write_submission(destination / "submission.csv", columns, rows, aliases, scores.result())
    measured = {
        "files": len(rows),
        "batches": len(plan),
        "wall_seconds": clock.total(),
        "metadata_seconds": scan_seconds,
        "model_load_seconds": load_seconds,
        # ru_maxrss is in KiB on Linux
        "peak_process_rss_gib": resource.getrusage(resource.RUSAGE_SELF).ru_maxrss * 1024 / GIB,
        "peak_allocated_gib": torch.cuda.max_memory_allocated() / GIB,
        "peak_reserved_gib": torch.cuda.max_memory_reserved() / GIB,
        "graph_build_seconds": engine.graph_build_seconds,
        "graph_hits": engine.graph_hits,
        "torch": torch.__version__,
        "gpu": torch.cuda.get_device_name(),
    }
    report = {key: measured[key] for key in REPORT_KEYS}
    (destination / "runtime_report.json").write_text(json.dumps(report, indent=2) + "\n")
    print(json.dumps(report), flush=True)
    return report
