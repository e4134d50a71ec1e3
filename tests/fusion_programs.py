"""Programs for the pointwise-fusion tests (tests/test_fusion.py, tests/test_gpu_fusion.py).

Each one exercises one rule of the fusion pass (the reference's lib/Transforms/PointwiseFusion.cpp,
csrc/core/fusion.cpp here), as the reference's own fusion fixtures do:
  one_step       a single guarded pointwise launch: nothing to fuse, one dispatch stays;
  six_steps      a chain of six unary pointwise launches over single-use temporaries (written
                 with a program loop): one fused dispatch of six steps, no temporary left;
  fan_out        a temporary read by three launches and two two-input joins: no producer has a
                 single unary consumer, so all six dispatches stay;
  smooth_twice   two 3-point smoothing stencils (neighbour reads are not pointwise): both stay;
  scale_offset   multiply, then add (runtime scalars): fused, the product must still be rounded
                 to f32 before the addition, i.e. no contraction into an FMA
                 (tests/Runtime/test_pointwise_fusion.py:105-118 of the reference).
"""
import ckl

N = ckl.dim("N")
Line = ckl.Buffer[ckl.f32, (N,)]
THREADS = 256


@ckl.kernel
def axpb(x: Line, y: Line, a: ckl.f32, b: ckl.f32) -> None:
    """y = a * x + b."""
    i = ckl.global_id(0)
    if i < N:
        y[i] = a * x[i] + b


@ckl.kernel
def sum2(x: Line, y: Line, out: Line) -> None:
    i = ckl.global_id(0)
    if i < N:
        out[i] = x[i] + y[i]


@ckl.kernel
def smooth(x: Line, out: Line) -> None:
    """(x[i-1] + 2 x[i] + x[i+1]) / 4 inside, x[i] at the two ends."""
    i = ckl.global_id(0)
    if i < N:
        if i > 0:
            if i + 1 < N:
                out[i] = (x[i - 1] + 2.0 * x[i] + x[i + 1]) * 0.25
        if i == 0:
            out[i] = x[i]
        if i + 1 == N:
            out[i] = x[i]


@ckl.kernel
def scale(x: Line, out: Line, factor: ckl.f32) -> None:
    i = ckl.global_id(0)
    if i < N:
        out[i] = x[i] * factor


@ckl.kernel
def offset(x: Line, out: Line, bias: ckl.f32) -> None:
    i = ckl.global_id(0)
    if i < N:
        out[i] = x[i] + bias


@ckl.program
def one_step(src: Line, dst: Line) -> None:
    ckl.launch(axpb, src, dst, 0.75, -0.125, grid=(ckl.cdiv(N, THREADS),), block=(THREADS,))


@ckl.program
def six_steps(src: Line, dst: Line) -> None:
    current = src
    for step in range(5):
        following = ckl.empty_like(src)
        ckl.launch(axpb, current, following, 0.9375, 0.0625, grid=(ckl.cdiv(N, THREADS),), block=(THREADS,))
        current = following
    ckl.launch(axpb, current, dst, 0.9375, 0.0625, grid=(ckl.cdiv(N, THREADS),), block=(THREADS,))


@ckl.program
def fan_out(src: Line, other: Line, dst: Line) -> None:
    shared = ckl.empty_like(src)
    ckl.launch(axpb, src, shared, 1.5, 0.25, grid=(ckl.cdiv(N, THREADS),), block=(THREADS,))
    first = ckl.empty_like(src)
    second = ckl.empty_like(src)
    third = ckl.empty_like(src)
    ckl.launch(axpb, shared, first, -0.5, 1.0, grid=(ckl.cdiv(N, THREADS),), block=(THREADS,))
    ckl.launch(axpb, shared, second, 2.0, 0.0, grid=(ckl.cdiv(N, THREADS),), block=(THREADS,))
    ckl.launch(axpb, shared, third, 0.25, -1.0, grid=(ckl.cdiv(N, THREADS),), block=(THREADS,))
    joined = ckl.empty_like(src)
    ckl.launch(sum2, first, second, joined, grid=(ckl.cdiv(N, THREADS),), block=(THREADS,))
    ckl.launch(sum2, joined, third, dst, grid=(ckl.cdiv(N, THREADS),), block=(THREADS,))


@ckl.program
def smooth_twice(src: Line, dst: Line) -> None:
    once = ckl.empty_like(src)
    ckl.launch(smooth, src, once, grid=(ckl.cdiv(N, THREADS),), block=(THREADS,))
    ckl.launch(smooth, once, dst, grid=(ckl.cdiv(N, THREADS),), block=(THREADS,))


@ckl.program
def scale_offset(src: Line, dst: Line, factor: ckl.f32, bias: ckl.f32) -> None:
    product = ckl.empty_like(src)
    ckl.launch(scale, src, product, factor, grid=(ckl.cdiv(N, THREADS),), block=(THREADS,))
    ckl.launch(offset, product, dst, bias, grid=(ckl.cdiv(N, THREADS),), block=(THREADS,))


# name -> (program, dispatches left after the fusion pass)
CASES = {"one_step": (one_step, 1), "six_steps": (six_steps, 1), "fan_out": (fan_out, 6),
         "smooth_twice": (smooth_twice, 2)}
