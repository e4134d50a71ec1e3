"""Independent requests (benchmarks/decoder/experiment.py:20-147): N invocations of one compiled
decode program share the read-only weights and RoPE table; each request has its own prompt,
mutable state, stream, heaps and workspaces, and all are submitted from one thread side by side
(`ckl.run_requests`). Every request's tokens, history, position, caches and logits must match the
oracle's steps from that request's own state (run.py:107-132 protocol, logits within 1e-4
row-normwise), and every mode, grouping and the serial order must leave the same state bit for
bit."""
import numpy as np
import pytest

import ckl
from oracle import decoder as oracle
from programs.decoder_config import CONFIGS, MUTABLE
from programs.harness import RequestGroup

pytestmark = pytest.mark.gpu

RUNS = (("graph", 1, True), ("graph", 1, False), ("graph", 16, False), ("stream", 1, False),
        ("ordinary", 1, False), ("capture", 1, False))


@pytest.mark.parametrize("name", ["small", "wide"])
def test_independent_requests_match_the_oracle(device, name):
    c = CONFIGS[name]
    requests = 4
    initial = [oracle.make_inputs(c, 123, init="baseline", prompt_seed=123 + i)[0] for i in range(requests)]
    group = RequestGroup(c, device, initial)
    # One set of weight buffers for all requests; separate mutable state.
    assert all(s.buffers["wq"] is group.states[0].buffers["wq"] for s in group.states)
    assert len({s.buffers["kc"].address for s in group.states}) == requests
    references = [oracle.expected(state.initial, c, c.steps) for state in group.states]
    results = {}
    for mode, batch, serial in RUNS:
        group.reset()
        timing = group.run(mode=mode, iterations=c.steps // batch, batch_size=batch, serial=serial)
        assert timing["wall_us"] > 0 and timing["span_us"] > 0, (mode, batch, serial)
        for state, reference in zip(group.states, references):
            state.verify(reference)
            assert state.logits_normwise <= 1e-4, (mode, batch, serial)
        results[(mode, batch, serial)] = [{k: s.download(k) for k in MUTABLE} for s in group.states]
    first = results[RUNS[0]]
    for key, states in results.items():
        for got, expected in zip(states, first):
            for k in MUTABLE:
                assert np.array_equal(got[k], expected[k]), (key, k)
    histories = [s["history"] for s in first]
    assert not np.array_equal(histories[0], histories[1]), "distinct prompts should give distinct tokens"


def test_run_requests_rejects_a_repeated_invocation(device):
    c = CONFIGS["small"]
    initial = [oracle.make_inputs(c, 123, init="baseline", prompt_seed=7)[0]]
    group = RequestGroup(c, device, initial)
    with pytest.raises(ValueError):
        ckl.run_requests([group.invocations[0], group.invocations[0]], mode="graph")
    with pytest.raises(ValueError):
        ckl.run_requests([], mode="graph")
