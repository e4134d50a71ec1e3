"""The bench's per-run checks (programs/harness.py DecoderState.check_capture, the checks of
benchmarks/decoder/run.py:107-132 that a timed sample can fail) on the CPU, with no device: a
capture equal to the expected state passes, and each kind of planted mistake is refused: a token,
a history row or the position off by one, a logit beyond the tolerance, a NaN logit, a row-normwise
error above 1e-4 that the elementwise tolerance admits, and an overwritten sentinel tail."""
import numpy as np
import pytest

from programs.harness import LOGITS_NORMWISE, SENTINEL, DecoderState

B, V, T, TAIL = 4, 64, 8, 16


def state():
    s = DecoderState.__new__(DecoderState)          # the checks read only the initial shapes
    s.initial = {"tokens": np.zeros(B, np.int32), "history": np.zeros((T, B), np.int32),
                 "position": np.zeros(1, np.int32), "logits": np.zeros((B, V), np.float32)}
    return s


def expected(rng):
    return {"steps": 3, "tokens": rng.integers(0, V, B).astype(np.int32),
            "history": rng.integers(0, V, (T, B)).astype(np.int32), "position": np.array([5], np.int32),
            "logits": rng.standard_normal((B, V)).astype(np.float32)}


def capture_of(e):
    def with_tail(a, dtype):
        return np.concatenate([np.asarray(a, dtype).ravel(), np.full(TAIL, SENTINEL, dtype)])
    return {"tokens": with_tail(e["tokens"], np.int32), "history": with_tail(e["history"], np.int32),
            "position": with_tail(e["position"], np.int32), "logits": with_tail(e["logits"], np.float32)}


def test_matching_capture_passes():
    e = expected(np.random.default_rng(1))
    found = state().check_capture(capture_of(e), e)
    assert found["logits_max_abs"] == 0.0 and found["logits_normwise"] == 0.0


@pytest.mark.parametrize("mistake", ["token", "history", "position", "logit", "nan", "normwise", "tail"])
def test_planted_mistake_is_refused(mistake):
    rng = np.random.default_rng(2)
    e = expected(rng)
    c = capture_of(e)
    if mistake == "token":
        c["tokens"][1] += 1
    elif mistake == "history":
        c["history"][B * 2 + 3] += 1
    elif mistake == "position":
        c["position"][0] += 1
    elif mistake == "logit":
        c["logits"][V + 7] += 1e-2
    elif mistake == "nan":
        c["logits"][5] = np.nan
    elif mistake == "normwise":
        # Within atol 2e-5 + rtol 3e-4 elementwise (0.2 at a logit of 1000), but 2e-4 of the row's
        # largest magnitude.
        row = np.zeros(V, np.float32)
        row[0] = 1000.0
        e["logits"][2] = row
        c["logits"][2 * V:3 * V] = row
        c["logits"][2 * V] = np.float32(1000.2)
        assert np.allclose(c["logits"][2 * V:3 * V], row, atol=2e-5, rtol=3e-4)
        assert 0.2 / 1000.0 > LOGITS_NORMWISE
    elif mistake == "tail":
        c["logits"][-1] = 0.0
    with pytest.raises(AssertionError):
        state().check_capture(c, e)
