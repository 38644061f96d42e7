"""Host logic of the submission job (no GPU): each template row is scored
exactly once, and a bucket whose graph runs out of device memory is rescored
file by file after the engine drops its graphs."""

import numpy as np
import pytest
import torch

from trifusion_amd import submission


def test_scores_accept_each_row_once():
    scores = submission._Scores(4)
    scores.fill([2, 0], np.full((2, 5), 0.25, np.float32))
    with pytest.raises(RuntimeError, match="more than once"):
        scores.fill([1, 2], np.zeros((2, 5), np.float32))
    with pytest.raises(RuntimeError, match="more than once"):
        scores.fill([3, 3], np.zeros((2, 5), np.float32))
    with pytest.raises(RuntimeError, match="2 template rows were never scored"):
        scores.result()
    scores.fill([1, 3], np.full((2, 5), 0.75, np.float32))
    table = scores.result()
    assert table.shape == (4, 5) and np.array_equal(table[:, 0], [0.25, 0.75, 0.25, 0.75])


class FakeEngine:
    """Logit of a file = its length; the batched call fails when ``oom``."""

    def __init__(self, oom):
        self.oom, self.cleared, self.eager_calls = oom, 0, 0

    def _logits(self, lengths):
        return lengths.float()[:, None].expand(-1, 5).to(torch.bfloat16)

    def __call__(self, audio, lengths, channels):
        if self.oom:
            raise torch.cuda.OutOfMemoryError("graph capture ran out of memory")
        return self._logits(lengths)

    def clear(self):
        self.cleared += 1

    def eager(self, audio, lengths, channels):
        assert audio.shape[0] == 1 and self.cleared == 1
        self.eager_calls += 1
        return self._logits(lengths)


@pytest.mark.parametrize("oom", [False, True])
def test_score_bucket_falls_back_per_file(oom):
    lengths = torch.tensor([-2, 0, 1])
    engine = FakeEngine(oom)
    probs = submission._score_bucket(engine, torch.zeros(3, 1, 8), lengths, torch.ones(3, dtype=torch.int64))
    assert probs.dtype == np.float32 and probs.shape == (3, 5)
    np.testing.assert_allclose(probs[:, 3], 1 / (1 + np.exp(-lengths.numpy())), rtol=1e-6)
    assert (engine.cleared, engine.eager_calls) == ((1, 3) if oom else (0, 0))


def test_report_keys_are_the_runtime_report_format():
    assert submission.REPORT_KEYS == (
        "files", "batches", "wall_seconds", "metadata_seconds", "model_load_seconds", "peak_process_rss_gib",
        "peak_allocated_gib", "peak_reserved_gib", "graph_build_seconds", "graph_hits", "torch", "gpu")
