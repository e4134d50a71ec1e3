"""Storage planner: known-answer tests (tests/Core/MemoryPlannerTest.cpp:18-65 of the reference),
and agreement of the native planner with the reference planner compiled from its own sources
(oracle/_ref) and with the Python restatement (oracle/graph.py) on seeded random graphs."""
import random
import subprocess
from pathlib import Path

import pytest

from ckl import _native
from oracle import graph as oracle_graph

ROOT = Path(__file__).resolve().parents[1]
REF_PLANNER = ROOT / "oracle" / "_ref" / "ref_planner"

EDGES = [(0, 1), (1, 4), (2, 3), (3, 4), (4, 5), (5, 6)]
RESOURCES = [
    dict(bytes=1024, alignment=256, users=[0, 1]),                       # early
    dict(bytes=512, alignment=256, users=[2, 3]),                        # parallel branch
    dict(bytes=768, alignment=128, users=[5, 6]),                        # late
    dict(bytes=256, alignment=64, users=[0, 6], kind="persistent"),
    dict(bytes=4096, alignment=256, users=[0, 6], kind="external"),
]


def test_known_answer_plan():
    baseline, planned, out = _native.plan_storage(7, EDGES, RESOURCES)
    early, parallel, late, persistent, external = out
    assert external is None
    assert early["slot"] != parallel["slot"], "parallel lifetimes must not share storage"
    assert late["slot"] == early["slot"], "ordered compatible lifetimes share best-fit storage"
    assert persistent["slot"] not in (early["slot"], parallel["slot"])
    assert (baseline, planned) == (2560, 1792)
    assert late["shares_first"] == 0


def test_reuse_disabled_is_dedicated():
    baseline, planned, out = _native.plan_storage(7, EDGES, RESOURCES, reuse=False)
    assert planned == baseline == 2560
    assert out[0]["slot"] != out[2]["slot"]


def test_persistent_storage_is_not_recycled():
    _, _, out = _native.plan_storage(2, [(0, 1)], [dict(bytes=64, alignment=64, users=[0], kind="persistent"),
                                                   dict(bytes=64, alignment=64, users=[1])])
    assert out[0]["slot"] != out[1]["slot"]


def test_cycles_are_rejected_with_diagnostic():
    with pytest.raises(ValueError, match="memory-planning graph must be acyclic"):
        _native.plan_storage(2, [(0, 1), (1, 0)], [])


def test_invalid_alignment_and_users():
    with pytest.raises(ValueError, match="power of two"):
        _native.plan_storage(1, [], [dict(bytes=8, alignment=3, users=[0])])
    with pytest.raises(ValueError, match="at least one user"):
        _native.plan_storage(1, [], [dict(bytes=8, alignment=8, users=[])])


def reference_plan(count, edges, resources, reuse):
    kinds = {"temporary": 0, "persistent": 1, "external": 2}
    lines = [f"nodes {count} reuse {int(reuse)}"] + [f"edge {a} {b}" for a, b in edges]
    lines += [f"resource {r['bytes']} {r['alignment']} 0 {kinds[r.get('kind', 'temporary')]} " +
              " ".join(map(str, r["users"])) for r in resources]
    out = subprocess.run([str(REF_PLANNER)], input="\n".join(lines) + "\n", capture_output=True, text=True, check=True)
    rows = out.stdout.split("\n")
    if rows[0].startswith("error"):
        return rows[0]
    _, baseline, _, planned = rows[0].split()
    offsets = {}
    for row in rows[1:]:
        if row:
            _, k, heap, offset, slot, shares = row.split()
            offsets[int(k)] = int(offset)
    return int(baseline), int(planned), [offsets.get(k) for k in range(len(resources))]


def random_graph(rng, count):
    edges = sorted({(a, b) for a in range(count) for b in range(a + 1, count) if rng.random() < 0.15})
    resources = []
    for _ in range(rng.randrange(2, 12)):
        users = sorted(rng.sample(range(count), rng.randrange(1, 4)))
        kind = rng.choice(["temporary"] * 6 + ["persistent", "external"])
        resources.append(dict(bytes=rng.choice([4, 64, 100, 256, 1000, 4096]), alignment=rng.choice([64, 128, 256]),
                              users=users, kind=kind))
    return edges, resources


@pytest.mark.skipif(not REF_PLANNER.is_file(), reason="reference planner not built (make -C oracle)")
@pytest.mark.parametrize("seed", range(40))
def test_native_matches_reference_planner_on_random_graphs(seed):
    rng = random.Random(seed)
    count = rng.randrange(3, 24)
    edges, resources = random_graph(rng, count)
    for reuse in (True, False):
        ref = reference_plan(count, edges, resources, reuse)
        baseline, planned, out = _native.plan_storage(count, edges, resources, reuse)
        mine = (baseline, planned, [None if a is None else a["offset"] for a in out])
        assert mine == ref
        assert oracle_graph.plan(count, set(edges), resources, reuse) == ref
