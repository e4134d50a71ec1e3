"""The reference's own recorded decoder results on the GPU: for every one of its 15 recorded
configurations (tests/golden/decoder_reference_results.json: benchmarks/decoder/results/deep-dive/
matrix.json and rtx5060ti.json), the tokens this backend generates in every run mode, with storage
reuse off and on, are exactly the recorded `generated_tokens`, and the whole state matches the
NumPy oracle (run.py:107-132 checks, logits within 1e-4 row-normwise).

The inputs are the reference's (oracle.make_inputs(init="reference"): its seed, weight scales and
prompts, which the oracle reproduces bit for bit, tests/test_oracle_decoder.py). Two starting
points are checked per configuration:
  * the GPU's own teacher-forced prefill of the context-1 prompt positions from the empty state
    (positions 0 .. context-2: case0's context of 1 makes the first generated step position 0),
    against the oracle's prefilled state;
  * 16 greedy steps from the oracle's prefilled state in each mode, one step per submission and
    16 steps per graph submission.
"""
import json
from pathlib import Path

import numpy as np
import pytest

from oracle import decoder as oracle
from programs.decoder_config import Config
from programs.harness import LOGITS_NORMWISE, DecoderSession, normwise_error

pytestmark = pytest.mark.gpu

GOLDEN = json.loads((Path(__file__).parent / "golden" / "decoder_reference_results.json").read_text())["cases"]
MODES = ("ordinary", "capture", "graph", "branches", "contracted", "stream")


@pytest.mark.parametrize("case", GOLDEN, ids=[f"{c['source'].split('/')[0]}-{c['name']}" for c in GOLDEN])
def test_recorded_tokens_on_the_gpu(device, case):
    c = Config(**case["config"])
    print(f"case {case['source']}:{case['name']} {c}", flush=True)
    initial, prompts = oracle.make_inputs(c, 123, init="reference")
    assert prompts.tolist() == case["prompts"]
    reference = oracle.expected(initial, c, c.steps)
    start = c.context - 1

    # The GPU's own prefill of positions 0 .. context-2 from the empty state.
    empty, _ = oracle.initial_state(c, 123, init="reference")
    prefill = DecoderSession(c, device, arrays=empty)
    prefill.prefill(prompts, mode="graph")
    for key in ("tokens", "position", "history"):
        assert np.array_equal(prefill.state.download(key), initial[key]), key
    for key in ("kc", "vc"):
        got = prefill.state.download(key)
        assert np.allclose(got[:, :, :, :start], initial[key][:, :, :, :start], atol=2e-5, rtol=3e-4), key
        assert np.array_equal(got[:, :, :, start:], initial[key][:, :, :, start:]), key
    if start:
        assert normwise_error(prefill.state.download("logits"), initial["logits"]) <= LOGITS_NORMWISE
    del prefill

    session = DecoderSession(c, device, arrays=initial)
    recorded = np.array(case["generated_tokens"], np.int32)
    for reuse, inv in session.invocations.items():
        for mode in MODES:
            for group in ((1, c.steps) if mode in ("graph", "capture") else (1,)):
                session.state.reset()
                for _ in range(c.steps // group):
                    inv.run(mode=mode, batch_size=group)
                history = session.state.download("history")[start:start + c.steps]
                assert np.array_equal(history, recorded), (reuse, mode, group)
                session.state.verify(reference)
                assert session.state.logits_normwise <= LOGITS_NORMWISE, (reuse, mode, group)
