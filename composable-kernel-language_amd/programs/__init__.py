"""CKL programs of the decode hot path (the reference's benchmarks/decoder/workloads.py and
examples/vector_pipeline.py), written against the ckl API."""
