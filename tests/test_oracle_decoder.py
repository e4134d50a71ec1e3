"""The NumPy decoder oracle reproduces the reference's recorded prompts and greedy tokens for
all 15 recorded configurations, and the product's synthetic input generator draws exactly the
oracle's inputs."""
import json
from pathlib import Path

import numpy as np
import pytest

from oracle import decoder as oracle
from programs.decoder_config import CONFIGS, Config
from programs.harness import synthetic_inputs

GOLDEN = json.loads((Path(__file__).parent / "golden" / "decoder_reference_results.json").read_text())["cases"]


@pytest.mark.parametrize("case", GOLDEN, ids=[f"{c['source'].split('/')[0]}-{c['name']}" for c in GOLDEN])
def test_oracle_tokens_match_reference_results(case):
    c = Config(**case["config"])
    initial, prompts = oracle.make_inputs(c, 123)
    assert prompts.tolist() == case["prompts"]
    final = oracle.expected(initial, c, c.steps)
    history = final["history"][c.context - 1:c.context - 1 + c.steps]
    assert history.tolist() == case["generated_tokens"]
    assert int(final["position"][0]) == c.context - 1 + c.steps


@pytest.mark.parametrize("init", ["baseline", "reference"])
@pytest.mark.parametrize("name", ["small", "wide", "deep"])
def test_synthetic_inputs_equal_oracle_inputs(name, init):
    c = CONFIGS[name]
    mine, prompts = synthetic_inputs(c, 123, init=init)
    ref, ref_prompts = oracle.initial_state(c, 123, init=init)
    assert np.array_equal(prompts, ref_prompts)
    assert set(mine) == set(ref)
    for key in ref:
        assert mine[key].dtype == ref[key].dtype and np.array_equal(mine[key], ref[key]), key


def test_rms_and_softmax_closed_forms():
    """Hand-checkable values: rms of a constant row is the gain; a one-position softmax is 1."""
    x = np.full((2, 8), 3.0, dtype=np.float32)
    out = oracle.rms(x, np.float32(2.0))
    assert np.allclose(out, 2.0 * 3.0 / np.sqrt(9.0 + 1e-5), rtol=1e-6)
    c = Config(batch=1, hidden=8, heads=2, layers=1, ffn=8, vocab=16, context=1, steps=1)
    arrays, _ = oracle.initial_state(c, 5)
    oracle.step(arrays, c)
    assert int(arrays["position"][0]) == 1
    assert arrays["tokens"][0] == int(np.argmax(arrays["logits"][0]))


def edge_rows(v, rng):
    """Logit rows that exercise the greedy scan's rules: ties, NaN, -0/+0, -inf rows."""
    rows = [rng.standard_normal(v).astype(np.float32) for _ in range(3)]
    tie = np.full(v, -1.0, np.float32)
    tie[[v // 3, v - 1]] = 2.0                                # equal maxima: the first index wins
    nan0 = rng.standard_normal(v).astype(np.float32)
    nan0[0] = np.nan                                          # NaN logit 0 is never displaced
    nans = rng.standard_normal(v).astype(np.float32)
    nans[rng.choice(v, v // 4, replace=False)] = np.nan
    nans[v // 2] = 50.0                                       # NaN elsewhere never wins
    zeros = np.full(v, -3.0, np.float32)
    zeros[[2, v - 2]] = [-0.0, 0.0]                           # -0 and +0 tie
    neg_inf = np.full(v, -np.inf, np.float32)                 # nothing beats logit 0
    nan_inf = np.full(v, -np.inf, np.float32)
    nan_inf[1::2] = np.nan
    return np.stack(rows + [tie, nan0, nans, zeros, neg_inf, nan_inf])


def scan_loop(row):
    # The kernel body's loop, element by element (workloads.py:170-183).
    best, winner = row[0], 0
    for v in range(1, len(row)):
        if row[v] > best:
            best, winner = row[v], v
    return winner


@pytest.mark.parametrize("v", [5, 129, 4100])
def test_greedy_scan_matches_the_scan_loop(v):
    logits = edge_rows(v, np.random.default_rng(v))
    expected = np.array([scan_loop(row) for row in logits], np.int32)
    assert np.array_equal(oracle.greedy_scan(logits), expected)
    clean = ~np.isnan(logits).any(axis=1)
    assert np.array_equal(oracle.greedy_scan(logits[clean]), logits[clean].argmax(axis=1))
