"""The large decoder (B32 C2048 A16x128 L4 F5632 V32000, 1024-token prompt,
KV capacity 1040) against the NumPy oracle. The 1023-step prefill runs teacher-forced on the GPU
(programs.harness.DecoderSession.prefill); from that state, one step and a 16-step generation in
each run mode are compared with the oracle's steps from the same state (run.py:107-132 protocol:
exact tokens/history/position, f32 state within atol 2e-5 / rtol 3e-4, logits within 1e-4 relative
to each row's largest reference magnitude, unchanged weights, cache prefix and suffix untouched,
sentinel tails intact)."""
import pytest

from oracle import decoder as oracle
from programs.decoder_config import CONFIGS
from programs.harness import DecoderSession, synthetic_inputs

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def large(device):
    c = CONFIGS["large"]
    arrays, prompts = synthetic_inputs(c, 123, init="baseline")
    session = DecoderSession(c, device, arrays=arrays)
    session.prefill(prompts)
    references = {n: oracle.expected(session.state.initial, c, n) for n in (1, c.steps)}
    return c, session, references


def test_large_one_step_all_modes(large):
    c, session, references = large
    for reuse, inv in session.invocations.items():
        for mode in ("graph", "capture", "ordinary", "branches", "contracted", "stream"):
            session.state.reset()
            inv.run(mode=mode)
            assert session.state.verify(references[1], check_weights=False) < 2e-5, (reuse, mode)
            assert session.state.logits_normwise <= 1e-4, (reuse, mode)
    assert session.invocations[False].edge_count(mode="branches") == 24 * c.layers + 5


def test_large_generation_grouped_graph(large):
    c, session, references = large
    session.state.reset()
    session.invocations[True].run(mode="graph", batch_size=c.steps)
    assert session.state.verify(references[c.steps]) < 2e-5
    assert session.state.logits_normwise <= 1e-4


def test_large_generation_branch_graph(large):
    c, session, references = large
    session.state.reset()
    session.invocations[True].run(mode="branches", batch_size=c.steps)
    assert session.state.verify(references[c.steps], check_weights=False) < 2e-5
