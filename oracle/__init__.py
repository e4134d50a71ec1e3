"""CPU oracle for the CKL decode hot path (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package,
and only as the checker or the reported CPU baseline; the product path never calls it.

Modules:
  decoder.py  NumPy restatement of benchmarks/decoder/reference.py (numerics, seeded inputs,
              prefill) -- pinned by the reference's recorded greedy tokens (matrix.json,
              rtx5060ti.json) for its own configurations.
  graph.py    closed-form restatement of the dependency-edge rules, the storage planner and the
              transitive reduction -- pinned by the reference's recorded decoder topologies and
              heap sizes, by its test fixtures, and by the reference planner compiled from its
              own sources into oracle/_ref/ (Makefile in this directory).
"""
