"""Run decode steps of one decoder configuration for a kernel profiler.

Binds the decode program (storage reuse off: the plan of bench.py's headline "inferred" variant)
to seeded synthetic state, sets the position to the
configuration's prefill position (so attention covers context rows, as in the timed steps; the
cache contents do not change kernel durations) and executes `--steps` inferred steps in mode
"stream": the inferred graph's contracted launches issued on the stream, so a profiler sees every
launch of the step (same kernels, same order as the graph; `--mode graph` runs the graph itself,
to compare the two on the GPU clock). `--calibrate` adds four launches of
the vector_pipeline `update` kernel, a copy of known size (4 MiB read, 4 MiB written), for scaling
hardware byte counters.

    rocprofv3 --kernel-trace --stats -d out -- \\
        python3 composable-kernel-language_amd/programs/profile_step.py --config large
"""
from __future__ import annotations

import argparse
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
for path in (HERE.parent / "python", HERE.parent):
    sys.path.insert(0, str(path))

import numpy as np  # noqa: E402


def main() -> None:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--config", default="large")
    parser.add_argument("--steps", type=int, default=12)
    parser.add_argument("--calibrate", action="store_true")
    parser.add_argument("--mode", default="stream", choices=("stream", "graph"),
                        help="stream: the launches one by one; graph: the same launches as one hipGraph per step")
    args = parser.parse_args()

    import ckl
    from programs.decoder_config import CONFIGS
    from programs.harness import DecoderSession

    c = CONFIGS[args.config]
    device = ckl.Device()
    session = DecoderSession(c, device)
    state = session.state
    state.host["position"][0] = c.context - 1
    inv = session.invocations[False]   # the plan bench.py's headline "inferred" variant runs
    print(f"{args.config}: {inv.launch_count(mode='graph', batch_size=1)} launches per inferred step", flush=True)
    for _ in range(args.steps):
        state.reset(("position",))
        inv.run(mode=args.mode, batch_size=1)
    if args.calibrate:
        from programs import vector_pipeline as vp
        n = 1 << 20
        program = vp.lower(n).compile(fuse_pointwise=False, reuse_storage=True)
        spec = ckl.BufferSpec((n,), ckl.f32)
        src, dst = device.empty(spec), device.empty(spec)
        src.copy_from_host(np.zeros(n, np.float32))
        copy = program.bind(src, dst, 0.5)
        for _ in range(4):
            copy.run(mode="ordinary")
    print("done", flush=True)


if __name__ == "__main__":
    main()
