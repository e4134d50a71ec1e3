"""Closed-form oracle for the dependency graph, storage planner and transitive reduction
(TEST INFRASTRUCTURE; see oracle/__init__.py).

Restated rules (the reference's algorithm, not its code):
  nodes      allocation, dispatch and free operations of the host function in program order
             (python/ckl/frontend/emitter.py:162-179, 406-427, 578-646; GraphAnalysis.cpp:405-416)
  edges      for i < j: an SSA edge when node j is a dispatch taking node i's allocation as an
             argument; a memory/lifetime edge when an access of i and an access of j touch
             resources that may alias (the same temporary, or any two host arguments) and at
             least one of them writes, allocates or frees (MemoryEffects.cpp:51-97;
             GraphAnalysis.cpp:436-491)
  reduction  among dispatch nodes, keep candidate -> target when no dispatch lies on a path
             between them (GraphAlgorithms.cpp:10-46)
  planner    graph-order slot reuse with least growth, 256-byte alignment
             (MemoryPlanner.cpp:19-204)
The decoder program is described per kernel by which arguments it reads and writes
(benchmarks/decoder/workloads.py:33-188); position accesses all cover element 0, so regions never
separate them.
Pinned by the reference's recorded topologies and heap sizes (tests/golden) for L = 1, 2, 8, by
the reference planner compiled from its sources (oracle/_ref), and by the closed-form edge rule
of the reference's randomized DAG test (tests/MLIR/test_semantics.py:98-125).
"""
from __future__ import annotations

READ, WRITE, ALLOC, FREE = 1, 2, 4, 8

# Per kernel: effect bits of each buffer argument, in argument order (scalars omitted).
KERNELS = {
    "embedding": (READ, READ, WRITE),
    "rms_stats": (READ, WRITE),
    "rms_apply": (READ, READ, READ, WRITE),
    "linear": (READ, READ, WRITE),
    "rope": (READ, READ, READ, WRITE),
    "append_kv": (READ, READ, WRITE, WRITE, READ),
    "attention_scores": (READ, READ, READ, WRITE),
    "softmax": (READ, READ, WRITE),
    "attention_values": (READ, READ, READ, WRITE),
    "add": (READ, READ, WRITE),
    "silu": (READ, WRITE),
    "multiply": (READ, READ, WRITE),
    "greedy": (READ, WRITE, WRITE, READ),
    "advance": (READ | WRITE,),
}


class Program:
    """Records nodes as the frontend orders them: alloc at creation, dispatch at launch, frees
    of all temporaries in reverse order at the end."""

    def __init__(self):
        self.nodes = []          # (kind, payload)
        self.temporaries = []    # (name, bytes)

    def empty(self, name, nbytes):
        self.temporaries.append((name, nbytes))
        self.nodes.append(("alloc", name))
        return name

    def launch(self, kernel, *buffers):
        bits = KERNELS[kernel]
        assert len(bits) == len(buffers), kernel
        self.nodes.append(("dispatch", (kernel, list(zip(buffers, bits)))))

    def finish(self):
        for name, _ in reversed(self.temporaries):
            self.nodes.append(("free", name))
        return self


def decoder_program(layers, batch, hidden, heads, capacity, ffn):
    """The decode program's node sequence (workloads.py:191-254)."""
    p = Program()
    bc, b, bat, bf = 4 * batch * hidden, 4 * batch, 4 * batch * heads * capacity, 4 * batch * ffn
    n = [0]

    def tmp(nbytes):
        n[0] += 1
        return p.empty(f"t{n[0]}", nbytes)

    x = tmp(bc)
    p.launch("embedding", "tokens", "emb", x)
    for _ in range(layers):
        inv, normed = tmp(b), tmp(bc)
        p.launch("rms_stats", x, inv)
        p.launch("rms_apply", x, inv, "norm1", normed)
        q, k, v = tmp(bc), tmp(bc), tmp(bc)
        p.launch("linear", normed, "wq", q)
        p.launch("linear", normed, "wk", k)
        p.launch("linear", normed, "wv", v)
        qr, kr = tmp(bc), tmp(bc)
        p.launch("rope", q, "sincos", "position", qr)
        p.launch("rope", k, "sincos", "position", kr)
        p.launch("append_kv", kr, v, "kc", "vc", "position")
        scores, probs = tmp(bat), tmp(bat)
        p.launch("attention_scores", qr, "kc", "position", scores)
        p.launch("softmax", scores, "position", probs)
        context = tmp(bc)
        p.launch("attention_values", probs, "vc", "position", context)
        projected = tmp(bc)
        p.launch("linear", context, "wo", projected)
        residual = tmp(bc)
        p.launch("add", x, projected, residual)
        inv2, normed2 = tmp(b), tmp(bc)
        p.launch("rms_stats", residual, inv2)
        p.launch("rms_apply", residual, inv2, "norm2", normed2)
        gate, up = tmp(bf), tmp(bf)
        p.launch("linear", normed2, "wg", gate)
        p.launch("linear", normed2, "wu", up)
        activated, product = tmp(bf), tmp(bf)
        p.launch("silu", gate, activated)
        p.launch("multiply", activated, up, product)
        down, next_x = tmp(bc), tmp(bc)
        p.launch("linear", product, "wd", down)
        p.launch("add", residual, down, next_x)
        x = next_x
    final_inv, final_x = tmp(b), tmp(bc)
    p.launch("rms_stats", x, final_inv)
    p.launch("rms_apply", x, final_inv, "final_norm", final_x)
    p.launch("linear", final_x, "lm", "logits")
    p.launch("greedy", "logits", "tokens", "history", "position")
    p.launch("advance", "position")
    return p.finish()


def accesses(node):
    kind, payload = node
    if kind == "alloc":
        return [(payload, ALLOC)]
    if kind == "free":
        return [(payload, FREE)]
    return payload[1]


def edges(program):
    temporaries = {name for name, _ in program.temporaries}
    alloc_node = {payload: i for i, (kind, payload) in enumerate(program.nodes) if kind == "alloc"}
    result = set()
    nodes = program.nodes
    for j, (kind, payload) in enumerate(nodes):
        if kind == "dispatch":
            for resource, _ in payload[1]:
                if resource in alloc_node and alloc_node[resource] != j:
                    result.add((alloc_node[resource], j))
    for i in range(len(nodes)):
        for j in range(i + 1, len(nodes)):
            for ra, ba in accesses(nodes[i]):
                for rb, bb in accesses(nodes[j]):
                    same = ra == rb
                    may = not same and ra not in temporaries and rb not in temporaries
                    if (same or may) and ((ba | bb) & (WRITE | ALLOC | FREE)):
                        result.add((i, j))
    return result


def closure(count, edge_set):
    reach = [0] * count
    for a, b in edge_set:
        reach[a] |= 1 << b
    for via in range(count):
        bit = 1 << via
        for a in range(count):
            if reach[a] & bit:
                reach[a] |= reach[via]
    return reach


def reduced_dependencies(program, edge_set):
    reach = closure(len(program.nodes), edge_set)
    dispatches = [i for i, (kind, _) in enumerate(program.nodes) if kind == "dispatch"]
    result = {}
    for t in dispatches:
        deps = []
        for c in dispatches:
            if c >= t or not reach[c] >> t & 1:
                continue
            if any(c < m < t and reach[c] >> m & 1 and reach[m] >> t & 1 for m in dispatches):
                continue
            deps.append(c)
        result[t] = deps
    return result


def plan(count, edge_set, resources, reuse=True):
    """resources: list of dict(bytes, alignment, users, kind in temporary/persistent/external).
    Returns (baseline, planned, offsets) with offsets[k] None for externals."""
    reach = closure(count, edge_set)

    def ordered(a, b):
        return bool(a["users"]) and bool(b["users"]) and all(
            x != y and reach[x] >> y & 1 for x in a["users"] for y in b["users"])

    def align(v, a):
        return (v + a - 1) // a * a

    slots, slot_of, baseline = [], {}, 0
    for k, r in enumerate(resources):
        if r["kind"] == "external":
            continue
        baseline += align(r["bytes"], r["alignment"])
        chosen, growth = None, None
        if reuse and r["kind"] == "temporary":
            for s, slot in enumerate(slots):
                if not slot["recyclable"]:
                    continue
                if all(ordered(r, resources[o]) or ordered(resources[o], r) for o in slot["residents"]):
                    g = max(slot["bytes"], r["bytes"]) - slot["bytes"]
                    if growth is None or g < growth:
                        chosen, growth = s, g
        if chosen is None:
            chosen = len(slots)
            slots.append(dict(bytes=r["bytes"], alignment=r["alignment"], recyclable=r["kind"] == "temporary", residents=[]))
        slot = slots[chosen]
        slot["bytes"] = max(slot["bytes"], r["bytes"])
        slot["alignment"] = max(slot["alignment"], r["alignment"])
        slot["residents"].append(k)
        slot_of[k] = chosen
    heap, heap_align = 0, 1
    for slot in slots:
        heap_align = max(heap_align, slot["alignment"])
        slot["offset"] = align(heap, slot["alignment"])
        heap = slot["offset"] + slot["bytes"]
    planned = align(heap, heap_align) if slots else 0
    offsets = [slots[slot_of[k]]["offset"] if k in slot_of else None for k in range(len(resources))]
    return baseline, planned, offsets


def decoder_plan(program, edge_set, reuse=True):
    """Planner inputs of the decoder: temporaries in first-access order over dispatch nodes."""
    sizes = dict(program.temporaries)
    order, users = [], {}
    for i, (kind, payload) in enumerate(program.nodes):
        if kind != "dispatch":
            continue
        for resource, _ in payload[1]:
            if resource not in users:
                users[resource] = []
                order.append(resource)
            if not users[resource] or users[resource][-1] != i:
                users[resource].append(i)
    resources = [dict(bytes=sizes[r], alignment=256, users=users[r], kind="temporary") for r in order if r in sizes]
    return plan(len(program.nodes), edge_set, resources, reuse)


def random_program_expected_edges(operations):
    """Closed form of tests/MLIR/test_semantics.py:107-114: explicit token edges plus every earlier
    dispatch on the same resource where either side writes."""
    expected = set()
    for target, (resource, effect, dependency) in enumerate(operations):
        if dependency is not None:
            expected.add((dependency, target))
        for source in range(target):
            other, other_effect, _ = operations[source]
            if other == resource and "write" in (effect, other_effect):
                expected.add((source, target))
    return expected
