"""The library's contract bodies (ckl.decoder_kernels) lower to exactly the canonical IR of the
reference's decoder kernels (benchmarks/decoder/workloads.py:33-188) and of its vector-pipeline
`update` (examples/vector_pipeline.py:11-16), for every specialisation the decode program and the
vector pipeline use; and the library serves every one of those specialisations.

The expected IR is data: tests/golden/workload_ir.json holds the SHA-256 of each reference
kernel's IR lowered by this package's frontend from the reference's source text (written by
tests/golden/make_workload_ir.py in the build container, where the reference checkout exists).
A contract body that differs from the reference's by one operation, operand order or constant
changes its hash.
"""
import hashlib
import json
import sys
from pathlib import Path

import pytest

from ckl import library

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))
FIXTURE = json.loads((GOLDEN / "workload_ir.json").read_text())

from make_workload_ir import programs, signature_key  # noqa: E402

LOWERED = dict(programs())


@pytest.mark.parametrize("label", sorted(FIXTURE))
def test_contract_bodies_lower_to_the_reference_kernels_ir(label):
    lowered = LOWERED[label]
    report = library.explain(lowered)
    seen = {}
    for spec, text in zip(lowered.specializations, lowered.kernels):
        kind, selection = report[spec.symbol]
        assert kind == "library", (spec.symbol, selection)
        assert selection.kernel.name == spec.definition.name
        seen[signature_key(spec.definition.name, spec.signature)] = hashlib.sha256(text.encode()).hexdigest()
    assert seen == FIXTURE[label]


def test_a_changed_body_is_not_served_by_the_library():
    """A body whose IR differs from the contract (here: the operands of rms_apply's product
    swapped) compiles from its own IR instead of running the library kernel."""
    import warnings

    import ckl
    from ckl.decoder_kernels import Activations, Gains, PerRequest

    @ckl.kernel
    def rms_apply(rows: Activations, inverse: PerRequest, gains: Gains, out: Activations,
                  which: ckl.constexpr[ckl.index]) -> None:
        col = ckl.global_id(0)
        row = ckl.global_id(1)
        if col < 64:
            out[row, col] = inverse[row] * rows[row, col] * gains[which, col]

    @ckl.program
    def normalize(rows: Activations, inverse: PerRequest, gains: Gains, out: Activations) -> None:
        ckl.launch(rms_apply, rows, inverse, gains, out, 0, grid=(1, 8), block=(64,))

    spec = {"rows": ckl.BufferSpec((8, 64), ckl.f32), "inverse": ckl.BufferSpec((8,), ckl.f32),
            "gains": ckl.BufferSpec((1, 64), ckl.f32), "out": ckl.BufferSpec((8, 64), ckl.f32)}
    with warnings.catch_warnings(record=True) as caught:
        warnings.simplefilter("always")
        report = library.explain(normalize.lower(signature=spec))
    assert [kind for kind, _ in report.values()] == ["jit"]
    assert any(issubclass(w.category, library.LibraryNameWarning) for w in caught)
