// Hand-written gfx950 (CDNA4) kernels implementing the CKL decoder kernels of
// benchmarks/decoder/workloads.py:33-188 and the vector update of examples/vector_pipeline.py:11-16.
//
// Contract with the executor (csrc/runtime/runtime.cpp):
//   * every kernel takes ONE struct argument whose layout is the CKL kernel's arguments in
//     order (buffers as pointers, scalars by value) followed by int32 shape constants chosen by
//     the selection in python/ckl/library.py; the runtime packs it with natural alignment and
//     pads to 8 bytes, which is the layout of an aligned(8) C struct with the same fields;
//   * grids are one-dimensional; each kernel body takes the logical block index so the same
//     body serves the single launch `ckl_X` and the sibling-group launch `ckl_X_group`, which
//     runs up to kMaxGroup independent dispatches of one family in a single grid;
//   * every position-indexed access is bounds-checked against the cache capacity.
// The semantics (what each element equals) are those of the CKL bodies; only the work
// decomposition differs (wave64 reductions, LDS staging, 128-bit accesses).
#include <hip/hip_runtime.h>

#include <stdint.h>

#include "args.h"

using namespace ckl::kernels;

constexpr int kBlock = 256;

#define CKL_ENTRY_ATTR(name, Args, body, threads, attributes)                                        \
  extern "C" __global__ __launch_bounds__(threads) attributes void ckl_##name(const Args a) { body(a, blockIdx.x); } \
  extern "C" __global__ __launch_bounds__(threads) attributes void ckl_##name##_group(const Group<Args> g) { \
    int b = blockIdx.x, m = 0;                                                                        \
    while (m + 1 < g.count && b >= g.start[m + 1]) ++m;                                               \
    body(g.m[m], b - g.start[m]);                                                                     \
  }
#define CKL_ENTRY(name, Args, body) CKL_ENTRY_ATTR(name, Args, body, kBlock, )
// Streaming kernels that keep several loads in flight per lane trade occupancy for registers.
#define CKL_TWO_WAVES __attribute__((amdgpu_waves_per_eu(1, 2)))
#define CKL_ONE_WAVE __attribute__((amdgpu_waves_per_eu(1, 1)))

// ------------------------------------------------------------------ wave64 reductions (DPP)
template <int Ctrl> __device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), Ctrl, 0xF, 0xF, false));
}
template <int Ctrl> __device__ __forceinline__ int dppi(int v) {
  return __builtin_amdgcn_mov_dpp(v, Ctrl, 0xF, 0xF, false);
}
constexpr int kQuadXor1 = 0xB1;      // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;      // quad_perm [2,3,0,1]
constexpr int kRowHalfMirror = 0x141;
constexpr int kRowMirror = 0x140;

// Sum over all 64 lanes; every lane receives the result. Fixed combination order.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<kQuadXor1>(v);
  v += dpp<kQuadXor2>(v);
  v += dpp<kRowHalfMirror>(v);
  v += dpp<kRowMirror>(v);
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<kQuadXor1>(v));
  v = fmaxf(v, dpp<kQuadXor2>(v));
  v = fmaxf(v, dpp<kRowHalfMirror>(v));
  v = fmaxf(v, dpp<kRowMirror>(v));
  v = fmaxf(v, __shfl_xor(v, 16));
  v = fmaxf(v, __shfl_xor(v, 32));
  return v;
}

// Sum over aligned groups of `width` lanes (width a power of two <= 64).
__device__ __forceinline__ float group_sum(float v, int width) {
  if (width > 1) v += dpp<kQuadXor1>(v);
  if (width > 2) v += dpp<kQuadXor2>(v);
  if (width > 4) v += dpp<kRowHalfMirror>(v);
  if (width > 8) v += dpp<kRowMirror>(v);
  if (width > 16) v += __shfl_xor(v, 16);
  if (width > 32) v += __shfl_xor(v, 32);
  return v;
}

// (value, index) argmax combine: larger value wins, equal values keep the smaller index.
__device__ __forceinline__ void argmax_combine(float &v, int &i, float ov, int oi) {
  if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
}

__device__ __forceinline__ void wave_argmax(float &v, int &i) {
  float ov; int oi;
  ov = dpp<kQuadXor1>(v); oi = dppi<kQuadXor1>(i); argmax_combine(v, i, ov, oi);
  ov = dpp<kQuadXor2>(v); oi = dppi<kQuadXor2>(i); argmax_combine(v, i, ov, oi);
  ov = dpp<kRowHalfMirror>(v); oi = dppi<kRowHalfMirror>(i); argmax_combine(v, i, ov, oi);
  ov = dpp<kRowMirror>(v); oi = dppi<kRowMirror>(i); argmax_combine(v, i, ov, oi);
  ov = __shfl_xor(v, 16); oi = __shfl_xor(i, 16); argmax_combine(v, i, ov, oi);
  ov = __shfl_xor(v, 32); oi = __shfl_xor(i, 32); argmax_combine(v, i, ov, oi);
}

__device__ __forceinline__ int load_position(const int *position) { return *position; }

// Streaming loads: the `_nt` entry points read the data a launch reads exactly once (weight rows,
// cache rows) with the nontemporal cache policy (global_load ... nt); the executor selects them
// when that data is at least kStreamBytes (args.h). Measured on MI355X, per-workgroup contiguous
// reads of a 2 GiB buffer stream at ~7.1 TB/s this way against ~6.1 TB/s with the default
// policy; but a decode step whose few MB of weights stay in the caches between steps runs
// slower with it, and a branch between the two in one kernel costs the small launches too.
typedef float stream_float4 __attribute__((ext_vector_type(4)));
typedef float stream_float2 __attribute__((ext_vector_type(2)));
template <bool NT> __device__ __forceinline__ float4 load4(const float *p) {
  if constexpr (NT) {
    stream_float4 v = __builtin_nontemporal_load(reinterpret_cast<const stream_float4 *>(p));
    return make_float4(v.x, v.y, v.z, v.w);
  } else {
    return *reinterpret_cast<const float4 *>(p);
  }
}
template <bool NT> __device__ __forceinline__ float2 load2(const float *p) {
  if constexpr (NT) {
    stream_float2 v = __builtin_nontemporal_load(reinterpret_cast<const stream_float2 *>(p));
    return make_float2(v.x, v.y);
  } else {
    return *reinterpret_cast<const float2 *>(p);
  }
}
template <bool NT> __device__ __forceinline__ float load1(const float *p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  else return *p;
}

// Operands of chain kernels that may be a split linear's partial planes (PartialSource, args.h):
// the planes are added in g order starting from 0, as the linear's own combine (split_finish)
// does, so deferring the combine leaves every value bit-identical. `i` is the element index.
// The planes of a batch are loaded together (one round trip per kSourceBatch planes): indices
// past the last plane re-read it and add nothing (the running sum starts at +0 and is never -0,
// so skipping a term and adding +0 agree).
constexpr int kSourceBatch = 8;
template <int N> struct SourceVector { float v[N]; };
template <int N> __device__ __forceinline__ SourceVector<N> source_load(const float *p) {
  SourceVector<N> out;
  if constexpr (N == 4) {
    float4 v = *reinterpret_cast<const float4 *>(p);
    out.v[0] = v.x; out.v[1] = v.y; out.v[2] = v.z; out.v[3] = v.w;
  } else if constexpr (N == 2) {
    float2 v = *reinterpret_cast<const float2 *>(p);
    out.v[0] = v.x; out.v[1] = v.y;
  } else {
    out.v[0] = *p;
  }
  return out;
}
template <int N> __device__ __forceinline__ SourceVector<N> source(const PartialSource &src, const float *own, long i) {
  if (src.parts == 0) return source_load<N>(own + i);
  SourceVector<N> t;
#pragma unroll
  for (int e = 0; e < N; ++e) t.v[e] = 0.f;
  for (int g0 = 0; g0 < src.parts; g0 += kSourceBatch) {
    SourceVector<N> v[kSourceBatch];
#pragma unroll
    for (int j = 0; j < kSourceBatch; ++j)
      v[j] = source_load<N>(src.partials + long(min(g0 + j, src.parts - 1)) * src.planeStride + i);
#pragma unroll
    for (int j = 0; j < kSourceBatch; ++j)
#pragma unroll
      for (int e = 0; e < N; ++e) t.v[e] += g0 + j < src.parts ? v[j].v[e] : 0.f;
  }
  return t;
}
__device__ __forceinline__ float source1(const PartialSource &src, const float *own, long i) {
  return source<1>(src, own, i).v[0];
}
__device__ __forceinline__ float2 source2(const PartialSource &src, const float *own, long i) {
  SourceVector<2> t = source<2>(src, own, i);
  return make_float2(t.v[0], t.v[1]);
}
__device__ __forceinline__ float4 source4(const PartialSource &src, const float *own, long i) {
  SourceVector<4> t = source<4>(src, own, i);
  return make_float4(t.v[0], t.v[1], t.v[2], t.v[3]);
}

// ------------------------------------------------------------------ embedding
// dst[b, c] = table[tokens[b], c]   (workloads.py:33-39)
__device__ void embedding_body(const EmbeddingArgs &a, int block) {
  long i = long(block) * kBlock + threadIdx.x;
  if ((a.C & 3) == 0) {
    long per = a.C / 4;
    if (i >= long(a.B) * per) return;
    int b = int(i / per), c4 = int(i % per);
    int token = a.tokens[b];
    float4 v = token >= 0 && token < a.V ? reinterpret_cast<const float4 *>(a.table + long(token) * a.C)[c4]
                                         : make_float4(__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""));
    reinterpret_cast<float4 *>(a.dst + long(b) * a.C)[c4] = v;
  } else {
    if (i >= long(a.B) * a.C) return;
    int b = int(i / a.C), c = int(i % a.C);
    int token = a.tokens[b];
    a.dst[long(b) * a.C + c] = token >= 0 && token < a.V ? a.table[long(token) * a.C + c] : __builtin_nanf("");
  }
}
CKL_ENTRY(embedding, EmbeddingArgs, embedding_body)

// ------------------------------------------------------------------ rms_stats
// inv[b] = rsqrt(sum_c x[b,c]^2 / C + eps)   (workloads.py:42-49). The squares
// are accumulated with explicit FMAs, so the row chains below (which compute the same row sums
// from the values they produce) round exactly as this kernel does.
__device__ __forceinline__ float add_squares(float total, float4 v) {
  total = __builtin_fmaf(v.x, v.x, total);
  total = __builtin_fmaf(v.y, v.y, total);
  total = __builtin_fmaf(v.z, v.z, total);
  return __builtin_fmaf(v.w, v.w, total);
}
__device__ __forceinline__ float rms_inverse(float total, int C, float eps) {
  return 1.0f / __fsqrt_rn(total / float(C) + eps);
}
// Sum over the 256 threads of a workgroup: wave sums, then the four wave sums in order.
__device__ __forceinline__ float block_sum(float v) {
  __shared__ float waves[kBlock / 64];
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) waves[threadIdx.x >> 6] = v;
  __syncthreads();
  return (waves[0] + waves[1]) + (waves[2] + waves[3]);
}
// One 256-thread workgroup per row: thread t accumulates elements t, t+256, ... (float4 when
// C % 4 == 0) with explicit FMAs, then block_sum. The row chains below use the same order.
__device__ void rms_stats_body(const RmsStatsArgs &a, int block) {
  const int row = block;
  if (row >= a.B) return;
  const float *x = a.x + long(row) * a.C;
  float total = 0.f;
  if ((a.C & 3) == 0) {
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
#pragma unroll 4
    for (int c = threadIdx.x; c < a.C / 4; c += kBlock) total = add_squares(total, x4[c]);
  } else {
#pragma unroll 4
    for (int c = threadIdx.x; c < a.C; c += kBlock) total = __builtin_fmaf(x[c], x[c], total);
  }
  total = block_sum(total);
  if (threadIdx.x == 0) a.inv[row] = rms_inverse(total, a.C, a.eps);
}
CKL_ENTRY(rms_stats, RmsStatsArgs, rms_stats_body)

// ------------------------------------------------------------------ rms_apply
// dst[b, c] = x[b, c] * inv[b] * gain[layer, c]   (workloads.py:52-58)
__device__ __forceinline__ float4 rms_scale(float4 x, float s, float4 g) {
  return make_float4(x.x * s * g.x, x.y * s * g.y, x.z * s * g.z, x.w * s * g.w);
}
__device__ void rms_apply_body(const RmsApplyArgs &a, int block) {
  long i = long(block) * kBlock + threadIdx.x;
  const float *gain = a.gain + long(a.layer) * a.C;
  if ((a.C & 3) == 0) {
    long per = a.C / 4;
    if (i >= long(a.B) * per) return;
    int b = int(i / per), c4 = int(i % per);
    float s = a.inv[b];
    float4 x = reinterpret_cast<const float4 *>(a.x + long(b) * a.C)[c4];
    float4 g = reinterpret_cast<const float4 *>(gain)[c4];
    reinterpret_cast<float4 *>(a.dst + long(b) * a.C)[c4] = rms_scale(x, s, g);
  } else {
    if (i >= long(a.B) * a.C) return;
    int b = int(i / a.C), c = int(i % a.C);
    a.dst[i] = a.x[i] * a.inv[b] * gain[c];
  }
}
CKL_ENTRY(rms_apply, RmsApplyArgs, rms_apply_body)

// ------------------------------------------------------------------ row chains ending in rms
// [producer ->] rms_stats -> rms_apply as one launch of rms_stats's geometry (one 256-thread
// workgroup per row): the workgroup produces its row (embedding gather or residual add, written to
// the producer's dst), sums the squares of the values it produced in rms_stats's order, writes
// inv[row] (unless the executor cleared the pointer because nothing outside the chain reads inv),
// then scales the row. Each thread touches the same elements in every phase, so it only reads
// back its own writes. The executor runs a chain only when its buffers are pairwise disjoint or
// identical (csrc/runtime/chains.cpp). Per element the arithmetic is that of the separate
// kernels, so results are bit-identical.
__device__ __forceinline__ void rms_finish_row(const RmsStatsArgs &stats, const RmsApplyArgs &apply, int row,
                                               float total) {
  total = block_sum(total);
  const float s = rms_inverse(total, stats.C, stats.eps);
  if (threadIdx.x == 0 && stats.inv) stats.inv[row] = s;   // null: only the chain reads inv
  const int C = apply.C;
  const float *gain = apply.gain + long(apply.layer) * C;
  const float *x = apply.x + long(row) * C;
  float *dst = apply.dst + long(row) * C;
  if ((C & 3) == 0) {
#pragma unroll 4
    for (int c = threadIdx.x; c < C / 4; c += kBlock)
      reinterpret_cast<float4 *>(dst)[c] = rms_scale(reinterpret_cast<const float4 *>(x)[c], s,
                                                     reinterpret_cast<const float4 *>(gain)[c]);
  } else {
#pragma unroll 4
    for (int c = threadIdx.x; c < C; c += kBlock) dst[c] = x[c] * s * gain[c];
  }
}

// Row chains whose row fits in registers (C % 4 == 0 and C / 4 <= kRowRegisters * 256): thread t
// keeps its R float4 values of the row (elements t, t + 256, ..., rms_stats's order) and has the
// gain loaded with its operands, so the scale phase needs no memory round trip. Every operand load
// of the row is issued before the first add (unpredicated, index clamped to the row; a plane
// source of at most kSourceBatch planes loads them all at once); stores and sums cover the
// in-range elements only. The values are those of the loop versions above and below.
constexpr int kRowRegisters = 4;
template <int R, bool Planes> struct RowSource { float4 v[R][Planes ? kSourceBatch : 1]; };
template <int R, bool Planes>
__device__ __forceinline__ void row_source_issue(const PartialSource &src, const float *own, const long (&i)[R],
                                                 RowSource<R, Planes> &l) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if constexpr (Planes) {
#pragma unroll
      for (int j = 0; j < kSourceBatch; ++j)
        l.v[r][j] = *reinterpret_cast<const float4 *>(src.partials + long(min(j, src.parts - 1)) * src.planeStride + i[r]);
    } else {
      l.v[r][0] = *reinterpret_cast<const float4 *>(own + i[r]);
    }
  }
}
// The planes added in g order from +0, skipping indices past the last plane (source<N>'s sums).
template <int R, bool Planes>
__device__ __forceinline__ float4 row_source_value(const PartialSource &src, const RowSource<R, Planes> &l, int r) {
  if constexpr (!Planes) {
    return l.v[r][0];
  } else {
    float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < kSourceBatch; ++j) {
      const bool in = j < src.parts;
      t.x += in ? l.v[r][j].x : 0.f;
      t.y += in ? l.v[r][j].y : 0.f;
      t.z += in ? l.v[r][j].z : 0.f;
      t.w += in ? l.v[r][j].w : 0.f;
    }
    return t;
  }
}
// Stores the produced row, sums its squares, and finishes rms_stats -> rms_apply from registers.
template <int R>
__device__ __forceinline__ void rms_finish_registers(const RmsStatsArgs &stats, const RmsApplyArgs &apply, int row,
                                                     float *produced, const float4 (&v)[R], const float4 (&g)[R]) {
  const int n4 = apply.C / 4;
  float total = 0.f;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int c = int(threadIdx.x) + r * kBlock;
    if (c < n4) {
      reinterpret_cast<float4 *>(produced)[c] = v[r];
      total = add_squares(total, v[r]);
    }
  }
  total = block_sum(total);
  const float s = rms_inverse(total, stats.C, stats.eps);
  if (threadIdx.x == 0 && stats.inv) stats.inv[row] = s;
  float4 *dst = reinterpret_cast<float4 *>(apply.dst + long(row) * apply.C);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int c = int(threadIdx.x) + r * kBlock;
    if (c < n4) dst[c] = rms_scale(v[r], s, g[r]);
  }
}
template <int R>
__device__ __forceinline__ void row_gain(const RmsApplyArgs &apply, const int (&c)[R], float4 (&g)[R]) {
  const float4 *gain = reinterpret_cast<const float4 *>(apply.gain + long(apply.layer) * apply.C);
#pragma unroll
  for (int r = 0; r < R; ++r) g[r] = gain[c[r]];
}
template <int R, bool PlanesX, bool PlanesY>
__device__ void add_rms_registers(const AddRmsChainArgs &a, int row) {
  const int n4 = a.stats.C / 4;
  const long base = long(row) * a.stats.C;
  int c[R];
  long idx[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    c[r] = min(int(threadIdx.x) + r * kBlock, n4 - 1);
    idx[r] = base + 4 * c[r];
  }
  float4 g[R], v[R];
  row_gain<R>(a.apply, c, g);
  RowSource<R, PlanesX> x;
  RowSource<R, PlanesY> y;
  row_source_issue<R, PlanesX>(a.x, a.add.x, idx, x);
  row_source_issue<R, PlanesY>(a.y, a.add.y, idx, y);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float4 u = row_source_value<R, PlanesX>(a.x, x, r), w = row_source_value<R, PlanesY>(a.y, y, r);
    v[r] = make_float4(u.x + w.x, u.y + w.y, u.z + w.z, u.w + w.w);
  }
  rms_finish_registers<R>(a.stats, a.apply, row, a.add.dst + base, v, g);
}
template <int R, bool PlanesX>
__device__ void add_rms_registers(const AddRmsChainArgs &a, int row) {
  if (a.y.parts > 0) add_rms_registers<R, PlanesX, true>(a, row);
  else add_rms_registers<R, PlanesX, false>(a, row);
}
template <int R> __device__ void add_rms_registers(const AddRmsChainArgs &a, int row) {
  if (a.x.parts > 0) add_rms_registers<R, true>(a, row);
  else add_rms_registers<R, false>(a, row);
}
template <int R> __device__ void embedding_rms_registers(const EmbeddingRmsChainArgs &a, int row) {
  const EmbeddingArgs &e = a.embedding;
  const int n4 = e.C / 4;
  int c[R];
#pragma unroll
  for (int r = 0; r < R; ++r) c[r] = min(int(threadIdx.x) + r * kBlock, n4 - 1);
  float4 g[R], v[R];
  row_gain<R>(a.apply, c, g);
  const int token = e.tokens[row];
  const bool valid = token >= 0 && token < e.V;
  const float nan = __builtin_nanf("");
  const float4 *table = reinterpret_cast<const float4 *>(e.table + long(valid ? token : 0) * e.C);
#pragma unroll
  for (int r = 0; r < R; ++r) v[r] = table[c[r]];
#pragma unroll
  for (int r = 0; r < R; ++r) v[r] = valid ? v[r] : make_float4(nan, nan, nan, nan);
  rms_finish_registers<R>(a.stats, a.apply, row, e.dst + long(row) * e.C, v, g);
}
// Number of float4 values per thread when the row fits in registers, else 0.
__device__ __forceinline__ int row_registers(int C) {
  return (C & 3) == 0 && C / 4 <= kRowRegisters * kBlock ? (C / 4 + kBlock - 1) / kBlock : 0;
}

__device__ void rms_stats__rms_apply_body(const RmsChainArgs &a, int block) {
  const int row = block;
  if (row >= a.stats.B) return;
  const int C = a.stats.C;
  const float *x = a.stats.x + long(row) * C;
  float total = 0.f;
  if ((C & 3) == 0) {
#pragma unroll 4
    for (int c = threadIdx.x; c < C / 4; c += kBlock) total = add_squares(total, reinterpret_cast<const float4 *>(x)[c]);
  } else {
#pragma unroll 4
    for (int c = threadIdx.x; c < C; c += kBlock) total = __builtin_fmaf(x[c], x[c], total);
  }
  rms_finish_row(a.stats, a.apply, row, total);
}
CKL_ENTRY(rms_stats__rms_apply, RmsChainArgs, rms_stats__rms_apply_body)

__device__ void add__rms_stats__rms_apply_body(const AddRmsChainArgs &a, int block) {
  const int row = block;
  if (row >= a.stats.B) return;
  const int C = a.stats.C;
  if (a.x.parts <= kSourceBatch && a.y.parts <= kSourceBatch) {
    switch (row_registers(C)) {
      case 1: add_rms_registers<1>(a, row); return;
      case 2: add_rms_registers<2>(a, row); return;
      case 3: add_rms_registers<3>(a, row); return;
      case 4: add_rms_registers<4>(a, row); return;
      default: break;
    }
  }
  const long base = long(row) * C;
  float total = 0.f;
  if ((C & 3) == 0) {
    float4 *dst = reinterpret_cast<float4 *>(a.add.dst + base);
#pragma unroll 4
    for (int c = threadIdx.x; c < C / 4; c += kBlock) {
      float4 u = source4(a.x, a.add.x, base + 4 * c), w = source4(a.y, a.add.y, base + 4 * c);
      float4 v = make_float4(u.x + w.x, u.y + w.y, u.z + w.z, u.w + w.w);
      dst[c] = v;
      total = add_squares(total, v);
    }
  } else {
#pragma unroll 4
    for (int c = threadIdx.x; c < C; c += kBlock) {
      float v = source1(a.x, a.add.x, base + c) + source1(a.y, a.add.y, base + c);
      a.add.dst[base + c] = v;
      total = __builtin_fmaf(v, v, total);
    }
  }
  rms_finish_row(a.stats, a.apply, row, total);
}
CKL_ENTRY(add__rms_stats__rms_apply, AddRmsChainArgs, add__rms_stats__rms_apply_body)

__device__ void embedding__rms_stats__rms_apply_body(const EmbeddingRmsChainArgs &a, int block) {
  const int row = block;
  if (row >= a.stats.B) return;
  const EmbeddingArgs &e = a.embedding;
  const int C = e.C;
  switch (row_registers(C)) {
    case 1: embedding_rms_registers<1>(a, row); return;
    case 2: embedding_rms_registers<2>(a, row); return;
    case 3: embedding_rms_registers<3>(a, row); return;
    case 4: embedding_rms_registers<4>(a, row); return;
    default: break;
  }
  const int token = e.tokens[row];
  const bool valid = token >= 0 && token < e.V;
  const float nan = __builtin_nanf("");
  float total = 0.f;
  if ((C & 3) == 0) {
    const float4 *table = reinterpret_cast<const float4 *>(e.table + long(valid ? token : 0) * C);
    float4 *dst = reinterpret_cast<float4 *>(e.dst + long(row) * C);
#pragma unroll 4
    for (int c = threadIdx.x; c < C / 4; c += kBlock) {
      float4 v = valid ? table[c] : make_float4(nan, nan, nan, nan);
      dst[c] = v;
      total = add_squares(total, v);
    }
  } else {
#pragma unroll 4
    for (int c = threadIdx.x; c < C; c += kBlock) {
      float v = valid ? e.table[long(token) * C + c] : nan;
      e.dst[long(row) * C + c] = v;
      total = __builtin_fmaf(v, v, total);
    }
  }
  rms_finish_row(a.stats, a.apply, row, total);
}
CKL_ENTRY(embedding__rms_stats__rms_apply, EmbeddingRmsChainArgs, embedding__rms_stats__rms_apply_body)

// ------------------------------------------------------------------ linear
// dst[b, o] = sum_i x[b, i] * w[layer, i, o]   (workloads.py:61-69)
//
// The weight matrix is streamed from HBM exactly once per launch. The grid is
// rowTiles x kSplit x tilesN workgroups of 256 threads (4 waves): workgroup (rt, kg, tn) owns
// output tile tn (a column range) for batch-row tile rt over the reduction slice
// [kg*kChunk, (kg+1)*kChunk), which its 4 waves share.
//   ckl_linear_rowvec (vector, B <= 16): one batch row and 64 output columns (lane <-> column)
//           per workgroup, the reduction split over its waves;
//   ckl_linear_mfma<J>x<S> (f32 MFMA, B > 16): v_mfma_f32_32x32x2f32 over 32 batch rows; each lane
//           loads J = 1, 2 or 4 consecutive weight columns with one vector load, and MFMA j
//           accumulates columns {J*c + j}, so one wave owns a 32 x 32J tile; a wave streams
//           16*S reduction rows per stage. The K index is permuted so the A operand (x) is one
//           float4 load per 8 reduction rows.
// Partial tiles of the 4 waves are added through LDS in wave order. With kSplit > 1 every
// workgroup writes its partial tile to the workspace with agent-coherent stores and bumps the
// tile's completion counter; the last one to arrive adds the kSplit partials in kg order,
// writes dst and resets the counter, so the result is deterministic and replays need no reset.
//
// workspace: the zero page, then counters (rowTiles*tilesN uint32, padded to 256 B); partials:
// partial tiles float[kSplit][rowTiles*rowsPerTile][O] (rowsPerTile = 32 for MFMA, B for the
// vector path).

typedef float floatx16 __attribute__((ext_vector_type(16)));
// s_waitcnt immediate (gfx9 encoding) that waits for vmcnt == 0 only: outstanding vector memory
// operations of the wave, stores included, have completed.
constexpr int kWaitStores = 0x0F70;

// Workspace of the linear family (args.h): kLinearZeroPage bytes that stay zero (loads of
// padding read here, so they need neither a predicate nor a select on the loaded value), then the
// split completion counters; the partial planes have their own pointer.
constexpr int kZeroPage = kLinearZeroPage;
__device__ __forceinline__ unsigned *split_counters(const LinearArgs &a) {
  return reinterpret_cast<unsigned *>(a.workspace + kZeroPage);
}
__device__ __forceinline__ float *split_partials(const LinearArgs &a, bool) { return a.partials; }

// Cross-workgroup partial tiles live in the workspace and are written and read only with
// agent-scope atomic stores/loads (sc1: coherent across the MI355X's per-XCD L2 caches without
// the whole-L2 writeback/invalidate an agent-scope fence costs).
__device__ __forceinline__ void partial_store(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float partial_load(const float *p) {
  return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Returns true in every thread of the last workgroup to finish a split tile. Every wave waits
// until its agent-coherent partial stores have completed (s_waitcnt vmcnt(0)); after the
// workgroup barrier one thread bumps the tile's completion counter, so the workgroup that
// observes the final count reads every partial through the same coherent path.
__device__ __forceinline__ bool split_arrive(unsigned *counter, int parts) {
  __shared__ int last;
  __builtin_amdgcn_s_waitcnt(kWaitStores);
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned previous = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    int isLast = previous == unsigned(parts - 1);
    if (isLast) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = isLast;
  }
  __syncthreads();
  return last;
}

// Adds the kSplit partial tiles (rows [r0, r0+rows), columns [c0, c0+cols)) in split order
// and writes dst. The partials of kFinishBatch splits are loaded together, then added in order
// (the batch condition is uniform; agent-coherent loads of one address serialize, so indices past
// the end are skipped rather than clamped).
constexpr int kFinishBatch = 8;
__device__ void split_finish(const LinearArgs &a, const float *partial, long planeStride, int r0, int rows, int c0,
                             int cols) {
  for (int e = threadIdx.x; e < rows * cols; e += blockDim.x) {
    int r = r0 + e / cols, c = c0 + e % cols;
    if (r >= a.B || c >= a.O) continue;
    const float *p = partial + long(r) * a.O + c;
    float total = 0.f;
    for (int g0 = 0; g0 < a.kSplit; g0 += kFinishBatch) {
      float v[kFinishBatch];
#pragma unroll
      for (int j = 0; j < kFinishBatch; ++j) v[j] = g0 + j < a.kSplit ? partial_load(p + (g0 + j) * planeStride) : 0.f;
#pragma unroll
      for (int j = 0; j < kFinishBatch; ++j) total += v[j];
    }
    a.dst[long(r) * a.O + c] = total;
  }
}

template <int J, bool NT> __device__ __forceinline__ void load_columns(float (&out)[J], const float *p) {
  if constexpr (J == 4) {
    float4 v = load4<NT>(p);
    out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
  } else if constexpr (J == 2) {
    float2 v = load2<NT>(p);
    out[0] = v.x; out[1] = v.y;
  } else {
    out[0] = load1<NT>(p);
  }
}

template <int J> __device__ __forceinline__ void store_columns(float *p, const float (&v)[J]) {
  if constexpr (J == 4) *reinterpret_cast<float4 *>(p) = make_float4(v[0], v[1], v[2], v[3]);
  else if constexpr (J == 2) *reinterpret_cast<float2 *>(p) = make_float2(v[0], v[1]);
  else *p = v[0];
}

// One stage = 16*S reduction rows of one lane (2S 8-row super-steps): x[row][k+8u .. k+8u+3] and
// the lane's J weight columns of rows k+8u+i. Full stages load without predicates or selects, so
// the next stage's loads stay in flight under the current stage's MFMAs: a batch row >= B (x row
// clamped to 0) only feeds output row >= B and a column >= O (clamped to column 0) only feeds
// output column >= O, neither of which is stored. Tail stages (S = 1) zero reduction rows past k1
// (their addresses are clamped to row k1-1).
// M > 1: M weight matrices of one shape that multiply the same x (a shared-operand group); the
// stage holds one x fragment and each member's weight columns.
template <int J, int S, int M> struct MfmaStage {
  float x[2 * S][4];
  float w[M][2 * S][4][J];
};

// A prefetch past the wave's last full stage (`dead`, issued only to keep the loop free of
// conditional loads) reads the workspace's zero page instead: one cache line for the wave.
template <int J, int S, int M, bool Tail, bool NT>
__device__ __forceinline__ void mfma_load(MfmaStage<J, S, M> &st, const float *xr, const float *const (&w)[M], long O,
                                          int k, int k1, bool dead = false, const float *zero = nullptr) {
#pragma unroll
  for (int u = 0; u < 2 * S; ++u) {
    const int kk = k + 8 * u;
    if constexpr (!Tail) {
      float4 v = *reinterpret_cast<const float4 *>(dead ? zero : xr + kk);
      st.x[u][0] = v.x; st.x[u][1] = v.y; st.x[u][2] = v.z; st.x[u][3] = v.w;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (Tail) {
        const bool inside = kk + i < k1;
        const int kr = min(kk + i, k1 - 1);
        st.x[u][i] = inside ? xr[kr] : 0.f;
#pragma unroll
        for (int m = 0; m < M; ++m) {
          float c[J];
          load_columns<J, NT>(c, w[m] + long(kr) * O);
#pragma unroll
          for (int j = 0; j < J; ++j) st.w[m][u][i][j] = inside ? c[j] : 0.f;
        }
      } else {
#pragma unroll
        for (int m = 0; m < M; ++m) load_columns<J, NT>(st.w[m][u][i], dead ? zero : w[m] + long(kk + i) * O);
      }
    }
  }
}

// Each accumulator acc[m][j] sees the same sequence of products whatever M is, so a member of a
// shared-operand group computes exactly what it computes alone.
template <int J, int S, int M>
__device__ __forceinline__ void mfma_compute(const MfmaStage<J, S, M> &st, floatx16 (&acc)[M][J]) {
#pragma unroll
  for (int u = 0; u < 2 * S; ++u)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int m = 0; m < M; ++m)
#pragma unroll
        for (int j = 0; j < J; ++j)
          acc[m][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(st.x[u][i], st.w[m][u][i][j], acc[m][j], 0, 0, 0);
}

// `a` holds M member blocks that agree on x, B, I, O, layer and the tiling (M = 1: one linear);
// the workgroup computes its tile of every member from one stream of x fragments.
template <int J, int S, int M, bool NT>
__device__ void linear_mfma(const LinearArgs *a, int block, float *smem) {
  const LinearArgs &a0 = a[0];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform: scalar loop control
  const int m = lane & 31, s = lane >> 5;
  const int tn = block % a0.tilesN, rest = block / a0.tilesN;
  const int kg = rest % a0.kSplit, rt = rest / a0.kSplit;
  const int n = tn * 32 * J + J * m;               // first of this lane's J columns
  const bool colOk = n < a0.O;                     // host guarantees O % J == 0
  const int row = rt * 32 + m;
  const bool rowOk = row < a0.B;
  const float *xr = a0.x + long(rowOk ? row : 0) * a0.I;
  const float *w[M];
#pragma unroll
  for (int e = 0; e < M; ++e) w[e] = a[e].w + long(a0.layer) * a0.I * a0.O + (colOk ? n : 0);
  const int kb0 = min(kg * a0.kChunk, a0.I), kb1 = min(kb0 + a0.kChunk, a0.I);

  floatx16 acc[M][J];
#pragma unroll
  for (int e = 0; e < M; ++e)
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[e][j][r] = 0.f;

  // The slice is cut into 16*S-row stages dealt round-robin to the 4 waves (wave w takes stages
  // w, w+4, ...), so the waves of a workgroup stream neighbouring weight rows at any moment.
  // Full stages are double-buffered: stage u+1's loads are in flight while stage u feeds the
  // MFMAs (S sets how many bytes each wave keeps in flight). The loop body has no conditional
  // loads (the compiler would sink them into the condition and drain the load queue at the join);
  // with an even stage count the last prefetch is dead and reads the zero page. sched_barrier
  // keeps each stage's loads issued as one group ahead of the other stage's MFMAs. The ragged
  // rest of the slice is cut into 16-row tail stages, dealt round-robin after the full ones.
  constexpr int R = 16 * S;
  const int fullTotal = (kb1 - kb0) / R;
  const int full = fullTotal > wave ? (fullTotal - wave + 3) / 4 : 0;
  const int k = kb0 + R * wave + 4 * s;                // this lane's row in the wave's first stage
  const int k1 = kb1;
  const long O = a0.O;
  MfmaStage<J, S, M> sa, sb;
  int t = 0;
  if (full > 0) mfma_load<J, S, M, false, NT>(sa, xr, w, O, k, k1);
  for (; t + 1 < full; t += 2) {
    mfma_load<J, S, M, false, NT>(sb, xr, w, O, k + 4 * R * (t + 1), k1);
    __builtin_amdgcn_sched_barrier(0);
    mfma_compute<J, S, M>(sa, acc);
    __builtin_amdgcn_sched_barrier(0);
    mfma_load<J, S, M, false, NT>(sa, xr, w, O, k + 4 * R * min(t + 2, full - 1), k1, t + 2 >= full,
                                  reinterpret_cast<const float *>(a0.workspace));
    __builtin_amdgcn_sched_barrier(0);
    mfma_compute<J, S, M>(sb, acc);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (t < full) mfma_compute<J, S, M>(sa, acc);
  const int tailBase = kb0 + R * fullTotal;
  const int tailStages = (kb1 - tailBase + 15) / 16;
#pragma unroll 1
  for (int q = (wave - fullTotal % 4 + 4) % 4; q < tailStages; q += 4) {
    MfmaStage<J, 1, M> st;
    mfma_load<J, 1, M, true, NT>(st, xr, w, O, tailBase + 16 * q + 4 * s, k1);
    mfma_compute<J, 1, M>(st, acc);
  }

  // Every wave hands its accumulators to the others through LDS in one pass (EM members at a
  // time, one float4 per lane and register quad); wave w then adds, for each member and column,
  // the four waves' quads 4w .. 4w+3 (its rows {8w + 4s + q}) in wave order and stores the lane's
  // J columns of each row with one vector store, so the four waves share the epilogue. Partial
  // planes the consumer combines (deferred) are plain stores; planes combined here go through
  // the agent-coherent path. `smem` is 16-byte aligned: float4 LDS accesses at an offset of 4
  // (after a 4-byte static variable) are split by the hardware and cost more than the pass saves.
  constexpr int EM = linearEpilogueMembers(M, J);
  const int rowTiles = (a0.B + 31) / 32;
  float4 *quads = reinterpret_cast<float4 *>(smem);
#pragma unroll
  for (int e0 = 0; e0 < M; e0 += EM) {
    if (e0 > 0) __syncthreads();
#pragma unroll
    for (int e = 0; e < EM && e0 + e < M; ++e)
#pragma unroll
      for (int j = 0; j < J; ++j)
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
          quads[(((wave * EM + e) * J + j) * 4 + rb) * 64 + lane] = make_float4(
              acc[e0 + e][j][4 * rb], acc[e0 + e][j][4 * rb + 1], acc[e0 + e][j][4 * rb + 2], acc[e0 + e][j][4 * rb + 3]);
    __syncthreads();
#pragma unroll
    for (int e = 0; e < EM && e0 + e < M; ++e) {
      const LinearArgs &ae = a[e0 + e];
      float *partial = split_partials(ae, false);
      float sum[J][4];
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const float4 t = quads[((e * J + j) * 4 + wave) * 64 + lane];
        sum[j][0] = t.x; sum[j][1] = t.y; sum[j][2] = t.z; sum[j][3] = t.w;
#pragma unroll
        for (int v = 1; v < 4; ++v) {
          const float4 o = quads[(((v * EM + e) * J + j) * 4 + wave) * 64 + lane];
          sum[j][0] += o.x; sum[j][1] += o.y; sum[j][2] += o.z; sum[j][3] += o.w;
        }
      }
      if (colOk) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int i = rt * 32 + 8 * wave + 4 * s + q;   // row of accumulator register 4*wave + q
          float v[J];
#pragma unroll
          for (int j = 0; j < J; ++j) v[j] = sum[j][q];
          if (ae.kSplit > 1) {
            float *p = partial + long(kg) * rowTiles * 32 * O + long(i) * O + n;
            if (ae.deferred) {
              store_columns<J>(p, v);
            } else {
#pragma unroll
              for (int j = 0; j < J; ++j) partial_store(p + j, v[j]);
            }
          } else if (i < ae.B) {
            store_columns<J>(ae.dst + long(i) * O + n, v);
          }
        }
      }
      if (ae.kSplit > 1 && !ae.deferred) {
        unsigned *counters = split_counters(ae);
        if (split_arrive(counters + rt * ae.tilesN + tn, ae.kSplit))
          split_finish(ae, partial, long(rowTiles) * 32 * O, rt * 32, 32, tn * 32 * J, 32 * J);
      }
    }
  }
}

// Row-parallel vector path (B <= 16, latency-bound): workgroup (tn, b, kg) computes the 64
// outputs dst[b, 64*tn .. 64*tn+63] (lane <-> column) over the reduction slice kg of waves*64 rows;
// wave w owns 64 consecutive rows of it. Measured on MI355X, these few-microsecond kernels are
// bound by memory round trips and by the instruction count of the busiest wave, so each wave
// issues all 64 of its weight loads at once (unpredicated: a predicated load becomes its own
// round trip because the compiler drains the load queue where branches join; padding rows read
// the workspace's zero page), takes x[b, k] as wave-uniform scalar loads, and does 64 FMAs.
// Waves are combined through LDS in wave order; only reductions longer than 16*64 rows split
// across workgroups.
constexpr int kVectorRows = 64;
constexpr int kVectorWaves = 16;
// This wave's partial sum for output column tn*64 + lane of batch row b over its kVectorRows
// reduction rows of slice kg (the caller combines the waves in wave order).
// A lane's reduction rows [k0, k1) and weight column of one chunk; the weights are loaded
// (rows past k1 read the zero page) and then dotted with x, so x may come from memory or LDS.
struct RowvecSlice { int k0, k1; const float *w; };
__device__ __forceinline__ RowvecSlice rowvec_slice(const LinearArgs &a, int col, int chunk, int waves, int kg) {
  const int span = waves * kVectorRows;
  const int kb0 = kg * span, kb1 = min(kb0 + span, a.I);
  const int k0 = kb0 + chunk * kVectorRows, k1 = min(k0 + kVectorRows, kb1);
  return {k0, k1, a.w + long(a.layer) * a.I * a.O + long(k0) * a.O + (col < a.O ? col : 0)};
}
template <bool NT>
__device__ __forceinline__ void rowvec_load(const LinearArgs &a, const RowvecSlice &s, float (&wv)[kVectorRows]) {
  const float *zero = reinterpret_cast<const float *>(a.workspace);   // kZeroPage: 64 zero floats
  const int lane = threadIdx.x & 63;
  if (s.k1 - s.k0 == kVectorRows) {
#pragma unroll
    for (int u = 0; u < kVectorRows; ++u) wv[u] = load1<NT>(s.w + long(u) * a.O);
  } else if (s.k0 < s.k1) {
#pragma unroll
    for (int u = 0; u < kVectorRows; ++u) wv[u] = load1<NT>(s.k0 + u < s.k1 ? s.w + long(u) * a.O : zero + lane);
  }
}
// x(k) is x[b, k] for k in [k0, k1).
template <typename X>
__device__ __forceinline__ float rowvec_dot(const RowvecSlice &s, const float (&wv)[kVectorRows], X x) {
  float acc = 0.f;
  if (s.k1 - s.k0 == kVectorRows) {
#pragma unroll
    for (int u = 0; u < kVectorRows; ++u) acc += x(s.k0 + u) * wv[u];
  } else if (s.k0 < s.k1) {
#pragma unroll
    for (int u = 0; u < kVectorRows; ++u) acc += (s.k0 + u < s.k1 ? x(min(s.k0 + u, s.k1 - 1)) : 0.f) * wv[u];
  }
  return acc;
}
template <bool NT> __device__ __forceinline__ float rowvec_partial(const LinearArgs &a, int b, int tn, int kg) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const RowvecSlice s = rowvec_slice(a, tn * 64 + int(threadIdx.x & 63), wave, int(blockDim.x >> 6), kg);
  const float *__restrict__ xr = a.x + long(b) * a.I;
  float wv[kVectorRows];
  rowvec_load<NT>(a, s, wv);
  return rowvec_dot(s, wv, [&](int k) { return xr[k]; });
}

template <bool NT> __device__ void linear_rowvec_stream(const LinearArgs &a, int block) {
  __shared__ float red[kVectorWaves][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int waves = blockDim.x >> 6;
  const int tn = block % a.tilesN, rest = block / a.tilesN;
  const int b = rest % a.B, kg = rest / a.B;
  const int col = tn * 64 + lane;
  const bool colOk = col < a.O;
  red[wave][lane] = rowvec_partial<NT>(a, b, tn, kg);
  __syncthreads();
  if (wave != 0 || !colOk) {
    if (a.kSplit == 1 || a.deferred) return;
  } else {
    float v = red[0][lane];
    for (int v2 = 1; v2 < waves; ++v2) v += red[v2][lane];
    if (a.kSplit > 1) partial_store(split_partials(a, true) + (long(kg) * a.B + b) * a.O + col, v);
    else a.dst[long(b) * a.O + col] = v;
  }
  if (a.kSplit > 1 && !a.deferred && split_arrive(split_counters(a) + b * a.tilesN + tn, a.kSplit))
    split_finish(a, split_partials(a, true), long(a.B) * a.O, b, 1, tn * 64, 64);
}

template <int J, int S, bool NT = false> __device__ void linear_mfma_body(const LinearArgs &a, int block) {
  extern __shared__ __attribute__((aligned(16))) float smem[];
  linear_mfma<J, S, 1, NT>(&a, block, smem);
}
CKL_ENTRY_ATTR(linear_rowvec, LinearArgs, linear_rowvec_stream<false>, 1024, )
CKL_ENTRY_ATTR(linear_rowvec_nt, LinearArgs, linear_rowvec_stream<true>, 1024, )
// ckl_linear_mfma<J>x<S>: J weight columns per lane, 16*S reduction rows per stage.
CKL_ENTRY(linear_mfma1x1, LinearArgs, (linear_mfma_body<1, 1>))
CKL_ENTRY(linear_mfma1x1_nt, LinearArgs, (linear_mfma_body<1, 1, true>))
CKL_ENTRY(linear_mfma1x2, LinearArgs, (linear_mfma_body<1, 2>))
CKL_ENTRY_ATTR(linear_mfma1x4, LinearArgs, (linear_mfma_body<1, 4>), kBlock, CKL_TWO_WAVES)
CKL_ENTRY(linear_mfma2x1, LinearArgs, (linear_mfma_body<2, 1>))
CKL_ENTRY(linear_mfma2x1_nt, LinearArgs, (linear_mfma_body<2, 1, true>))
CKL_ENTRY_ATTR(linear_mfma2x2, LinearArgs, (linear_mfma_body<2, 2>), kBlock, CKL_TWO_WAVES)
CKL_ENTRY_ATTR(linear_mfma2x4, LinearArgs, (linear_mfma_body<2, 4>), kBlock, CKL_TWO_WAVES)
CKL_ENTRY_ATTR(linear_mfma4x1, LinearArgs, (linear_mfma_body<4, 1>), kBlock, CKL_TWO_WAVES)
CKL_ENTRY_ATTR(linear_mfma4x1_nt, LinearArgs, (linear_mfma_body<4, 1, true>), kBlock, CKL_TWO_WAVES)
CKL_ENTRY_ATTR(linear_mfma4x2, LinearArgs, (linear_mfma_body<4, 2>), kBlock, CKL_TWO_WAVES)
// ckl_linear_mfma<J>x1_shared<M>: M linears of one shape and tiling that multiply the same x
// (their blocks in a Group<LinearArgs>, count == M; grid = one member's grid). Each workgroup
// computes its tile of every member from one x stream, so the sibling projections of a decoder
// layer (q, k, v; gate, up) run as one grid of at most one workgroup per CU.
#define CKL_LINEAR_SHARED(J, M)                                                                       \
  extern "C" __global__ __launch_bounds__(kBlock) CKL_ONE_WAVE void ckl_linear_mfma##J##x1_shared##M( \
      const Group<LinearArgs> g) {                                                                    \
    extern __shared__ __attribute__((aligned(16))) float smem[];                                                                   \
    linear_mfma<J, 1, M, false>(g.m, blockIdx.x, smem);                             \
  }                                                                                                   \
  extern "C" __global__ __launch_bounds__(kBlock) CKL_ONE_WAVE void ckl_linear_mfma##J##x1_nt_shared##M( \
      const Group<LinearArgs> g) {                                                                    \
    extern __shared__ __attribute__((aligned(16))) float smem[];                                                                   \
    linear_mfma<J, 1, M, true>(g.m, blockIdx.x, smem);                              \
  }
CKL_LINEAR_SHARED(1, 2)
CKL_LINEAR_SHARED(1, 3)
CKL_LINEAR_SHARED(2, 2)
CKL_LINEAR_SHARED(2, 3)
CKL_LINEAR_SHARED(4, 2)
CKL_LINEAR_SHARED(4, 3)

// ------------------------------------------------------------------ rope
// Adjacent-pair rotation at position p (workloads.py:72-85):
//   dst[b,c] = s[b,c]*cos - s[b,c+1]*sin; dst[b,c+1] = s[b,c]*sin + s[b,c+1]*cos, c = h*2R + 2r.
// (first*cos - second*sin, first*sin + second*cos) with explicit FMAs, shared by rope and its chain.
__device__ __forceinline__ float2 rotate(float2 s, float2 cs) {
  return make_float2(__builtin_fmaf(s.x, cs.x, -(s.y * cs.y)), __builtin_fmaf(s.x, cs.y, s.y * cs.x));
}
// Two adjacent pairs (elements c .. c+3) and their two (cos, sin) entries, each one 128-bit access;
// each pair rounds exactly as `rotate` alone.
__device__ __forceinline__ float4 rotate2(float4 s, float4 cs) {
  const float2 lo = rotate(make_float2(s.x, s.y), make_float2(cs.x, cs.y));
  const float2 hi = rotate(make_float2(s.z, s.w), make_float2(cs.z, cs.w));
  return make_float4(lo.x, lo.y, hi.x, hi.y);
}
// Pairs a rope worker rotates: two when R is even (python/ckl/library.py sizes the grid alike),
// so its q, k and table accesses are 128 bits wide; one when R is odd.
__device__ __forceinline__ int rope_unit(int R) { return (R & 1) ? 1 : 2; }
__device__ __forceinline__ bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
// A source read 4 floats at a time at 16-byte-aligned element offsets stays aligned.
__device__ __forceinline__ bool aligned16(const PartialSource &src, const float *own) {
  return src.parts ? aligned16(src.partials) && (src.planeStride & 3) == 0 : aligned16(own);
}
__device__ void rope_body(const RopeArgs &a, int block) {
  const int unit = rope_unit(a.R), per = a.R / unit;
  long i = long(block) * kBlock + threadIdx.x;
  if (i >= long(a.B) * a.A * per) return;
  int p = load_position(a.position);
  if (p < 0 || p >= a.T) return;
  const int r = int(i % per) * unit;
  const long bh = i / per;
  const long c = bh * (2L * a.R) + 2 * r;               // = b*(2R*A) + h*2R + 2r
  const float *table = a.table + (long(p) * a.R + r) * 2;
  if (unit == 2 && aligned16(a.src) && aligned16(a.dst) && aligned16(a.table)) {
    *reinterpret_cast<float4 *>(a.dst + c) =
        rotate2(*reinterpret_cast<const float4 *>(a.src + c), *reinterpret_cast<const float4 *>(table));
    return;
  }
  for (int j = 0; j < unit; ++j)
    *reinterpret_cast<float2 *>(a.dst + c + 2 * j) =
        rotate(*reinterpret_cast<const float2 *>(a.src + c + 2 * j), *reinterpret_cast<const float2 *>(table + 2 * j));
}
CKL_ENTRY(rope, RopeArgs, rope_body)

// ------------------------------------------------------------------ append_kv
// kc[layer,b,h,p,d] = k[b,h*D+d]; vc[...] = v[...]   (workloads.py:88-97)
__device__ void append_kv_body(const AppendArgs &a, int block) {
  long i = long(block) * kBlock + threadIdx.x;
  int p = load_position(a.position);
  if (p < 0 || p >= a.T) return;
  if ((a.D & 3) == 0) {
    int per = a.D / 4;
    if (i >= long(a.B) * a.A * per) return;
    int d4 = int(i % per);
    long bh = i / per;
    long src = bh * a.D + 4 * d4;
    long dst = (((long(a.layer) * a.B * a.A) + bh) * a.T + p) * a.D + 4 * d4;
    *reinterpret_cast<float4 *>(a.kc + dst) = *reinterpret_cast<const float4 *>(a.k + src);
    *reinterpret_cast<float4 *>(a.vc + dst) = *reinterpret_cast<const float4 *>(a.v + src);
  } else {
    if (i >= long(a.B) * a.A * a.D) return;
    int d = int(i % a.D);
    long bh = i / a.D;
    long dst = (((long(a.layer) * a.B * a.A) + bh) * a.T + p) * a.D + d;
    a.kc[dst] = a.k[bh * a.D + d];
    a.vc[dst] = a.v[bh * a.D + d];
  }
}
CKL_ENTRY(append_kv, AppendArgs, append_kv_body)

// rope(q), rope(k) -> append_kv as one launch of rope's geometry: a worker rotates rope_unit(R)
// adjacent pairs of q and of k (128-bit accesses when R is even and the buffers allow), writes q's
// (and k's, unless only append reads it), and appends the rotated k and v's elements to the caches
// at the current position. (D = 2R, so element h*D + 2r of k and v is the same index c as the
// rotated pair.)
__device__ __forceinline__ void rope_append_pair(const RopeAppendChainArgs &a, long c, long row, const float *table) {
  const float2 cs = *reinterpret_cast<const float2 *>(table);
  *reinterpret_cast<float2 *>(a.q.dst + c) = rotate(source2(a.qsrc, a.q.src, c), cs);
  const float2 kr = rotate(source2(a.ksrc, a.k.src, c), cs);
  if (a.k.dst) *reinterpret_cast<float2 *>(a.k.dst + c) = kr;
  *reinterpret_cast<float2 *>(a.append.kc + row) = kr;
  *reinterpret_cast<float2 *>(a.append.vc + row) = source2(a.v, a.append.v, c);
}
__device__ void rope__rope__append_kv_body(const RopeAppendChainArgs &a, int block) {
  const RopeArgs &q = a.q, &k = a.k;
  const AppendArgs &ap = a.append;
  const int unit = rope_unit(q.R), per = q.R / unit;
  long i = long(block) * kBlock + threadIdx.x;
  if (i >= long(q.B) * q.A * per) return;
  int p = load_position(q.position);
  if (p < 0 || p >= q.T) return;
  const int r = int(i % per) * unit;
  const long bh = i / per;
  const long c = bh * (2L * q.R) + 2 * r;
  const long row = (((long(ap.layer) * ap.B * ap.A) + bh) * ap.T + p) * ap.D + 2 * r;
  const float *table = q.table + (long(p) * q.R + r) * 2;
  const bool wide = unit == 2 && aligned16(a.qsrc, q.src) && aligned16(a.ksrc, k.src) && aligned16(a.v, ap.v) &&
                    aligned16(q.dst) && (!k.dst || aligned16(k.dst)) && aligned16(q.table) && aligned16(ap.kc) &&
                    aligned16(ap.vc);
  if (!wide) {
    for (int j = 0; j < unit; ++j) rope_append_pair(a, c + 2 * j, row + 2 * j, table + 2 * j);
    return;
  }
  const float4 cs = *reinterpret_cast<const float4 *>(table);
  *reinterpret_cast<float4 *>(q.dst + c) = rotate2(source4(a.qsrc, q.src, c), cs);
  const float4 kr = rotate2(source4(a.ksrc, k.src, c), cs);
  if (k.dst) *reinterpret_cast<float4 *>(k.dst + c) = kr;
  *reinterpret_cast<float4 *>(ap.kc + row) = kr;
  *reinterpret_cast<float4 *>(ap.vc + row) = source4(a.v, ap.v, c);
}
CKL_ENTRY(rope__rope__append_kv, RopeAppendChainArgs, rope__rope__append_kv_body)

// ------------------------------------------------------------------ attention_scores
// scores[b,h,t] = (sum_d q[b,h*D+d] * kc[layer,b,h,t,d]) * scale for t <= p (workloads.py:100-111).
// One 256-thread workgroup per (b, h, 256-row chunk); each wave owns 64 consecutive cache rows.
// Rows are held in the vector layout below; a wave issues kScoreBatch float4 loads per lane before
// reducing any of them, so ~kScoreBatch KB per wave are in flight. Row addresses past the end
// re-read an early row of the wave and their results are dropped (the loads stay unpredicated).
// The row arithmetic is shared with the attention chains; rows the vector layout does not cover
// use the sequential dot product.
constexpr int kScoreBatch = 8;
__device__ __forceinline__ float score_scalar(const float *q, const float *key, int D) {
  float v = 0.f;
  for (int d = 0; d < D; ++d) v = __builtin_fmaf(q[d], key[d], v);
  return v;
}
// Vector layout of the scores: groups of G lanes hold one cache row, each lane P float4 pieces of
// it (pieces part + G*j, j < P): P = 1 and G = D/4 for D <= 32, P = 2 for D <= 64, else P = 4,
// with G = D/(4P) a power of two (8 lanes for D = 64 and 128, 16 for D = 256); other D (D = 96:
// G = 6) take the sequential dot product. A P = 3 instantiation for D = 96 would give it 8-lane
// groups, but it doubled the VGPRs of the rope/attention chain kernel for every D (69 -> 148,
// with scratch), so the chain ran 40% slower at D = 128; it is not instantiated. Each lane adds its 4P products with explicit FMAs in piece order, then
// the row is summed over its G lanes (group_sum), so with 8-lane groups a row costs three DPP
// steps instead of a 32-lane butterfly. A wave load covers 64/G rows; a lane keeps kScoreBatch
// pieces in flight (kScoreBatch/P rows).
__device__ __forceinline__ int score_pieces(int D) { return D <= 32 ? 1 : D <= 64 ? 2 : 4; }
__device__ __forceinline__ bool scores_vector_layout(int D) {
  if ((D & 3) || D > 256) return false;
  const int P = score_pieces(D), G = D / (4 * P);
  return G * 4 * P == D && (G & (G - 1)) == 0;        // G lanes a row: a power of two
}
// Partial dot product of a lane's P pieces of q and of one key row.
template <int P> __device__ __forceinline__ float dot_pieces(const float4 (&q)[P], const float4 *k) {
  float v = q[0].x * k[0].x;
  v = __builtin_fmaf(q[0].y, k[0].y, v);
  v = __builtin_fmaf(q[0].z, k[0].z, v);
  v = __builtin_fmaf(q[0].w, k[0].w, v);
#pragma unroll
  for (int j = 1; j < P; ++j) {
    v = __builtin_fmaf(q[j].x, k[j].x, v);
    v = __builtin_fmaf(q[j].y, k[j].y, v);
    v = __builtin_fmaf(q[j].z, k[j].z, v);
    v = __builtin_fmaf(q[j].w, k[j].w, v);
  }
  return v;
}
template <int P> struct KeyLayout {
  static constexpr int U = kScoreBatch / P;        // rows per lane per batch
  int G, rowsPerLoad, sub, part;
  __device__ explicit KeyLayout(int D) : G(D / (4 * P)), rowsPerLoad(64 / (D / (4 * P))) {
    const int lane = threadIdx.x & 63;
    sub = lane / G;
    part = lane % G;
  }
  __device__ int rowsPerBatch() const { return U * rowsPerLoad; }
  template <typename T> __device__ void loadQuery(float4 (&qv)[P], const T *q) const {
#pragma unroll
    for (int j = 0; j < P; ++j) qv[j] = reinterpret_cast<const float4 *>(q)[part + G * j];
  }
};
template <bool NT, int P> __device__ void attention_scores_rows(const ScoresArgs &a, const float *q, const float *keys,
                                                          float *scores, int w0, int w1) {
  const KeyLayout<P> k(a.D);
  float4 qv[P];
  k.loadQuery(qv, q);
  for (int base = w0; base < w1; base += k.rowsPerBatch()) {
    float4 kv[kScoreBatch];
#pragma unroll
    for (int u = 0; u < k.U; ++u) {
      int t = base + u * k.rowsPerLoad + k.sub;
      t = t < w1 ? t : min(w0 + k.sub, w1 - 1);    // past the end: re-read an early row, dropped
#pragma unroll
      for (int j = 0; j < P; ++j) kv[u * P + j] = load4<NT>(keys + long(t) * a.D + 4 * (k.part + k.G * j));
    }
#pragma unroll
    for (int u = 0; u < k.U; ++u) {
      float v = group_sum(dot_pieces<P>(qv, kv + u * P), k.G);
      int t = base + u * k.rowsPerLoad + k.sub;
      if (k.part == 0 && t < w1) scores[t] = v * a.scale;
    }
  }
}
template <bool NT> __device__ void attention_scores_body(const ScoresArgs &a, int block) {
  int chunks = (a.T + kBlock - 1) / kBlock;
  int chunk = block % chunks;
  long bh = block / chunks;
  if (bh >= long(a.B) * a.A) return;
  int p = load_position(a.position);
  int end = min(p + 1, a.T);
  int t0 = chunk * kBlock;
  if (p < 0 || t0 >= end) return;
  const float *q = a.q + bh * a.D;
  const float *keys = a.kc + (long(a.layer) * a.B * a.A + bh) * long(a.T) * a.D;
  float *scores = a.scores + bh * a.T;
  int tEnd = min(t0 + kBlock, end);
  if (scores_vector_layout(a.D)) {
    const int wave = threadIdx.x >> 6;
    const int w0 = t0 + wave * 64, w1 = min(w0 + 64, tEnd);
    switch (score_pieces(a.D)) {
      case 1: attention_scores_rows<NT, 1>(a, q, keys, scores, w0, w1); break;
      case 2: attention_scores_rows<NT, 2>(a, q, keys, scores, w0, w1); break;
      default: attention_scores_rows<NT, 4>(a, q, keys, scores, w0, w1); break;
    }
  } else {
    for (int t = t0 + threadIdx.x; t < tEnd; t += kBlock) scores[t] = score_scalar(q, keys + long(t) * a.D, a.D) * a.scale;
  }
}
CKL_ENTRY(attention_scores, ScoresArgs, attention_scores_body<false>)
CKL_ENTRY(attention_scores_nt, ScoresArgs, attention_scores_body<true>)

// ------------------------------------------------------------------ softmax
// probs[b,h,t] = exp(s[t] - max) / sum_t' exp(s[t'] - max) over t <= p (workloads.py:114-128).
// `rowThreads` (64 or 256) lanes per (b, h) row; each lane keeps up to kSoftmaxPerLane scores in
// registers (one read of the row, one write), longer rows stream three passes.
constexpr int kSoftmaxPerLane = 8;
constexpr int kValuesBlock = 512;

// Reduction over the `rowThreads` lanes of one row (a wave, or waves 0-3 of the workgroup). With
// rowThreads > 64 every thread of the workgroup must call it (it synchronizes the workgroup).
template <bool IsMax> __device__ __forceinline__ float row_reduce(float v, int rowThreads) {
  __shared__ float across[kValuesBlock / 64];
  v = IsMax ? wave_max(v) : wave_sum(v);
  if (rowThreads <= 64) return v;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) across[wave] = v;
  __syncthreads();
  float r = across[0];
  for (int w = 1; w < kBlock / 64; ++w) r = IsMax ? fmaxf(r, across[w]) : r + across[w];
  return r;
}

// Softmax of row `row` (scores `s`: a.scores' row, or its LDS copy in a chain) by the lanes with
// local index `local` < rowThreads (inactive lanes only take part in the synchronization).
// Probabilities go to a.probs (unless null) and, when `stage` is given, to stage[t] as well;
// `stage` may be `s` itself: every lane reads its elements before it writes them.
// `p` is the position (a.position[0]), loaded by the caller.
__device__ __forceinline__ void softmax_row(const SoftmaxArgs &a, const float *s, long row, int local, bool active,
                                            float *stage, int p) {
  int end = min(p + 1, a.T);
  if (p < 0) end = 0;
  float *out = a.probs ? a.probs + (active ? row : 0) * a.T : nullptr;   // null in a chain: LDS only
  if (end <= a.rowThreads * kSoftmaxPerLane) {
    float v[kSoftmaxPerLane];
    float m = -__builtin_inff();
#pragma unroll
    for (int u = 0; u < kSoftmaxPerLane; ++u) {
      int t = local + u * a.rowThreads;
      v[u] = active && t < end ? s[t] : -__builtin_inff();
      m = fmaxf(m, v[u]);
    }
    m = row_reduce<true>(m, a.rowThreads);
    float total = 0.f;
#pragma unroll
    for (int u = 0; u < kSoftmaxPerLane; ++u) {
      int t = local + u * a.rowThreads;
      v[u] = t < end ? expf(v[u] - m) : 0.f;
      total += v[u];
    }
    total = row_reduce<false>(total, a.rowThreads);
#pragma unroll
    for (int u = 0; u < kSoftmaxPerLane; ++u) {
      int t = local + u * a.rowThreads;
      if (active && t < end) {
        float q = v[u] / total;
        if (out) out[t] = q;
        if (stage) stage[t] = q;
      }
    }
  } else {
    float m = -__builtin_inff();
    for (int t = local; t < end; t += a.rowThreads) m = fmaxf(m, active ? s[t] : -__builtin_inff());
    m = row_reduce<true>(m, a.rowThreads);
    float total = 0.f;
    for (int t = local; t < end; t += a.rowThreads) total += active ? expf(s[t] - m) : 0.f;
    total = row_reduce<false>(total, a.rowThreads);
    for (int t = local; t < end; t += a.rowThreads)
      if (active) {
        float q = expf(s[t] - m) / total;
        if (out) out[t] = q;
        if (stage) stage[t] = q;
      }
  }
}

__device__ void softmax_body(const SoftmaxArgs &a, int block) {
  const int rowsPerBlock = kBlock / a.rowThreads;
  const int local = threadIdx.x % a.rowThreads;
  long row = long(block) * rowsPerBlock + threadIdx.x / a.rowThreads;
  const bool active = row < long(a.B) * a.A;       // uniform per row group (rowThreads divides kBlock)
  softmax_row(a, a.scores + (active ? row : 0) * a.T, row, local, active, nullptr, load_position(a.position));
}
CKL_ENTRY(softmax, SoftmaxArgs, softmax_body)

// ------------------------------------------------------------------ attention_values
// dst[b, h*D+d] = sum_{t<=p} probs[b,h,t] * vc[layer,b,h,t,d]   (workloads.py:131-142).
// One workgroup per (b, h) of blockDim.x <= kValuesBlock threads (a power of two, chosen from the
// cache capacity): groups of D/4 lanes own the float4 column slices of one row, blockDim/(D/4)
// row groups stride over t with kValuesBatch row loads per lane in flight; the partial float4
// sums are combined by a fixed-order tree in LDS. `probs` is the (b, h) row of probabilities
// (global memory, or LDS in the softmax chain).
constexpr int kValuesBatch = 8;
__device__ __forceinline__ bool values_vector_layout(int D) { return (D & 3) == 0 && D <= 4 * 64 && (64 % (D / 4)) == 0; }
// A thread's kValuesBatch cache-row loads of the values' vector layout, rows base + u*groups + g
// (rows past `end` re-read an early row; end > 0).
struct ValueBatch { float4 v[kValuesBatch]; };
template <bool NT>
__device__ __forceinline__ void load_value_batch(ValueBatch &vb, const float *values, int D, int base, int end) {
  const int width = D / 4, groups = int(blockDim.x) / width;
  const int g = threadIdx.x / width, part = threadIdx.x % width;
#pragma unroll
  for (int u = 0; u < kValuesBatch; ++u) {
    int t = base + u * groups + g;
    int tc = t < end ? t : min(g, end - 1);        // past the end: re-read an early row, weight 0
    vb.v[u] = load4<NT>(values + long(tc) * D + 4 * part);
  }
}
__device__ __forceinline__ const float *values_slab(const ValuesArgs &a, long bh) {
  return a.vc + (long(a.layer) * a.B * a.A + bh) * long(a.T) * a.D;
}
// `haveFirst`: `first` holds this thread's first batch (vector layout, end > 0). `p` is the
// position (a.position[0]), loaded by the caller.
template <bool NT>
__device__ __forceinline__ void attention_values_row(const ValuesArgs &a, long bh, const float *probs,
                                                     const ValueBatch &first, bool haveFirst, int p) {
  __shared__ float4 partial[kValuesBlock];
  int end = min(p + 1, a.T);
  if (p < 0) end = 0;
  const float *values = values_slab(a, bh);
  float *dst = a.dst + bh * a.D;
  if (values_vector_layout(a.D)) {
    const int width = a.D / 4, groups = int(blockDim.x) / width;
    const int g = threadIdx.x / width, part = threadIdx.x % width;
    const int step = kValuesBatch * groups;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    auto consume = [&](const ValueBatch &vb, int base) {
#pragma unroll
      for (int u = 0; u < kValuesBatch; ++u) {
        int t = base + u * groups + g;
        int tc = t < end ? t : min(g, end - 1);
        float pr = t < end ? probs[tc] : 0.f;
        acc.x = __builtin_fmaf(pr, vb.v[u].x, acc.x);
        acc.y = __builtin_fmaf(pr, vb.v[u].y, acc.y);
        acc.z = __builtin_fmaf(pr, vb.v[u].z, acc.z);
        acc.w = __builtin_fmaf(pr, vb.v[u].w, acc.w);
      }
    };
    int base = 0;
    if (haveFirst) {
      consume(first, 0);
      base = step;
    }
    for (; base < end; base += step) {
      ValueBatch vb;
      load_value_batch<NT>(vb, values, a.D, base, end);
      consume(vb, base);
    }
    partial[threadIdx.x] = acc;
    __syncthreads();
    for (int stride = groups / 2; stride > 0; stride /= 2) {
      if (g < stride) {
        float4 o = partial[threadIdx.x + stride * width];
        float4 s = partial[threadIdx.x];
        partial[threadIdx.x] = make_float4(s.x + o.x, s.y + o.y, s.z + o.z, s.w + o.w);
      }
      __syncthreads();
    }
    if (g == 0) reinterpret_cast<float4 *>(dst)[part] = partial[part];
  } else {
    for (int d = threadIdx.x; d < a.D; d += blockDim.x) {
      float acc = 0.f;
      for (int t = 0; t < end; ++t) acc = __builtin_fmaf(probs[t], values[long(t) * a.D + d], acc);
      dst[d] = acc;
    }
  }
}

template <bool NT> __device__ void attention_values_body(const ValuesArgs &a, int block) {
  long bh = block;
  if (bh >= long(a.B) * a.A) return;
  ValueBatch none;
  attention_values_row<NT>(a, bh, a.probs + bh * a.T, none, false, load_position(a.position));
}
CKL_ENTRY_ATTR(attention_values, ValuesArgs, attention_values_body<false>, kValuesBlock, )
CKL_ENTRY_ATTR(attention_values_nt, ValuesArgs, attention_values_body<true>, kValuesBlock, )

// softmax -> attention_values as one launch of attention_values's geometry (one workgroup per
// (b, h), blockDim >= rowThreads, checked by the executor): lanes [0, rowThreads) compute the
// row's softmax exactly as the softmax kernel does, writing probs and an LDS copy of the row
// (T <= kChainSoftmaxRow floats of dynamic shared memory), then the workgroup reduces the values
// from the LDS copy.
template <bool NT> __device__ void softmax__attention_values_body(const SoftmaxValuesChainArgs &a, int block) {
  extern __shared__ float rowProbs[];
  long bh = block;
  if (bh >= long(a.values.B) * a.values.A) return;
  const int rowThreads = a.softmax.rowThreads;
  softmax_row(a.softmax, a.softmax.scores + bh * a.softmax.T, bh, int(threadIdx.x) % rowThreads,
              int(threadIdx.x) < rowThreads, rowProbs, load_position(a.softmax.position));
  __syncthreads();
  ValueBatch none;
  attention_values_row<NT>(a.values, bh, rowProbs, none, false, load_position(a.values.position));
}
CKL_ENTRY_ATTR(softmax__attention_values, SoftmaxValuesChainArgs, softmax__attention_values_body<false>, kValuesBlock, )
CKL_ENTRY_ATTR(softmax__attention_values_nt, SoftmaxValuesChainArgs, softmax__attention_values_body<true>, kValuesBlock, )

// attention_scores -> softmax -> attention_values as one launch of attention_values's geometry
// (one workgroup per (b, h)): the workgroup computes the row's scores into LDS (the waves stride
// over cache rows, kScoreBatch row loads per lane in flight, each row reduced exactly as
// attention_scores does), the softmax in place in LDS, then the values from LDS. Scores and
// probabilities are also written to global memory unless the executor cleared those pointers
// (only the chain reads them).
// A wave's kScoreBatch cache-row loads of the scores' vector layout (groups of D/4 lanes hold one
// row as float4s): rows base + u*rowsPerLoad + sub; rows past `end` re-read an early row.
// A wave's batch of cache-row loads in the scores' vector layout (KeyLayout<P>): rows
// base + u*rowsPerLoad + sub for u < U, P pieces each; rows past `end` re-read an early row.
struct KeyBatch { float4 kv[kScoreBatch]; };
template <bool NT, int P>
__device__ __forceinline__ void load_key_batch(KeyBatch &kb, const float *keys, int D, const KeyLayout<P> &k, int base,
                                               int end) {
#pragma unroll
  for (int u = 0; u < k.U; ++u) {
    int t = base + u * k.rowsPerLoad + k.sub;
    t = t < end ? t : min(k.sub, end - 1);        // past the end: re-read an early row, dropped
#pragma unroll
    for (int j = 0; j < P; ++j) kb.kv[u * P + j] = load4<NT>(keys + long(t) * D + 4 * (k.part + k.G * j));
  }
}
template <int P>
__device__ __forceinline__ void score_key_batch(const KeyBatch &kb, const float4 (&qv)[P], const KeyLayout<P> &k, int base,
                                                int end, float scale, float *rowScores, float *scores) {
#pragma unroll
  for (int u = 0; u < k.U; ++u) {
    float v = group_sum(dot_pieces<P>(qv, kb.kv + u * P), k.G) * scale;
    int t = base + u * k.rowsPerLoad + k.sub;
    if (k.part == 0 && t < end) {
      rowScores[t] = v;
      if (scores) scores[t] = v;
    }
  }
}

// The scores -> softmax -> values row of (b, h) = bh with the query row `q` (global memory, or
// LDS in the rope chain) at position `p` (sc.position[0], loaded by the caller): scores into
// rowScores (LDS, T floats), softmax in place, values. With
// `haveFirst`, `first` holds the wave's first batch of cache rows (vector layout only). With
// `appended` (the rope chain, position in range), the key row at the position is read from LDS
// instead of the cache and `storesPending` waves wait for their cache-row stores before the
// barrier that precedes the values. The first batch of value rows is loaded before the softmax.
template <bool NT, int P>
__device__ __forceinline__ void attention_chain_row(const ScoresArgs &sc, const SoftmaxArgs &softmax,
                                                    const ValuesArgs &values, long bh, const float *q, int p,
                                                    float *rowScores, const KeyBatch &first, bool haveFirst,
                                                    const float *appended = nullptr, bool storesPending = false) {
  int end = min(p + 1, sc.T);
  if (p < 0) end = 0;
  const float *keys = sc.kc + (long(sc.layer) * sc.B * sc.A + bh) * long(sc.T) * sc.D;
  float *scores = sc.scores ? sc.scores + bh * sc.T : nullptr;
  const bool vector = scores_vector_layout(sc.D);
  if (vector) {
    const KeyLayout<P> k(sc.D);
    const int wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    float4 qv[P];
    k.loadQuery(qv, q);
    const int step = waves * k.rowsPerBatch();
    const int endG = appended ? end - 1 : end;       // the appended row comes from LDS
    int base = wave * k.rowsPerBatch();
    if (haveFirst) {
      score_key_batch(first, qv, k, base, endG, sc.scale, rowScores, scores);
      base += step;
    }
    for (; base < endG; base += step) {
      KeyBatch kb;
      load_key_batch<NT, P>(kb, keys, sc.D, k, base, endG);
      score_key_batch(kb, qv, k, base, endG, sc.scale, rowScores, scores);
    }
    if (appended && wave == 0) {
      // The row's score with the arithmetic of the cache path (any lane group reduces alike).
      float4 kv[P];
      k.loadQuery(kv, appended);
      float v = group_sum(dot_pieces<P>(qv, kv), k.G) * sc.scale;
      if ((threadIdx.x & 63) == 0) {
        rowScores[p] = v;
        if (scores) scores[p] = v;
      }
    }
  } else {
    for (int t = threadIdx.x; t < end; t += blockDim.x) {
      float v = score_scalar(q, keys + long(t) * sc.D, sc.D) * sc.scale;
      rowScores[t] = v;
      if (scores) scores[t] = v;
    }
  }
  if (storesPending) __builtin_amdgcn_s_waitcnt(kWaitStores);
  __syncthreads();
  ValueBatch vfirst;
  const bool haveV = values_vector_layout(values.D) && end > 0;
  if (haveV) load_value_batch<NT>(vfirst, values_slab(values, bh), values.D, 0, end);
  const int rowThreads = softmax.rowThreads;
  softmax_row(softmax, rowScores, bh, int(threadIdx.x) % rowThreads, int(threadIdx.x) < rowThreads, rowScores, p);
  __syncthreads();
  attention_values_row<NT>(values, bh, rowScores, vfirst, haveV, p);
}

template <bool NT>
__device__ void attention_scores__softmax__attention_values_body(const AttentionChainArgs &a, int block) {
  extern __shared__ float rowScores[];
  long bh = block;
  if (bh >= long(a.values.B) * a.values.A) return;
  KeyBatch none;
  const float *q = a.scores.q + bh * a.scores.D;
  const int p = load_position(a.scores.position);
  switch (score_pieces(a.scores.D)) {
    case 1: attention_chain_row<NT, 1>(a.scores, a.softmax, a.values, bh, q, p, rowScores, none, false); break;
    case 2: attention_chain_row<NT, 2>(a.scores, a.softmax, a.values, bh, q, p, rowScores, none, false); break;
    default: attention_chain_row<NT, 4>(a.scores, a.softmax, a.values, bh, q, p, rowScores, none, false); break;
  }
}
CKL_ENTRY_ATTR(attention_scores__softmax__attention_values, AttentionChainArgs,
               attention_scores__softmax__attention_values_body<false>, kValuesBlock, )
CKL_ENTRY_ATTR(attention_scores__softmax__attention_values_nt, AttentionChainArgs,
               attention_scores__softmax__attention_values_body<true>, kValuesBlock, )

// rope(q), rope(k) -> append_kv -> attention_scores -> softmax -> attention_values as one launch
// of attention_values's geometry: workgroup (b, h) first rotates its head's pairs of q and k at
// the current position (as rope does), writes the rotated q (and k, unless only append reads it),
// keeps the rotated q and k in LDS and appends the rotated k and v's row to the caches; then it
// runs the attention row as the attention chain does, with the query and the appended key row
// from LDS, the first batch of cache-row loads issued before the rotation, and the appending waves
// waiting for their stores before the values read the cache. The position is outside
// [0, T) only if the caller lets it run past the cache capacity; then rope and append write
// nothing and the attention reads q's buffer, as the separate dispatches would.
// Dynamic LDS: the row of T scores (padded to 4 floats), then the D-float query and key rows.
// Planes of a rotation operand requested up front (rope_attention_rows): a pair from each of the
// first kRopeRequest planes (a source of fewer planes re-reads its last one) or, without planes,
// the pair itself; sum_pair adds them as source2 does.
constexpr int kRopeRequest = 4;
__device__ __forceinline__ void request_pair(const PartialSource &src, const float *own, long i,
                                             float2 (&out)[kRopeRequest]) {
  if (src.parts == 0) {
    out[0] = *reinterpret_cast<const float2 *>(own + i);
    return;
  }
#pragma unroll
  for (int j = 0; j < kRopeRequest; ++j)
    out[j] = *reinterpret_cast<const float2 *>(src.partials + long(min(j, src.parts - 1)) * src.planeStride + i);
}
__device__ __forceinline__ float2 sum_pair(const PartialSource &src, const float2 (&in)[kRopeRequest]) {
  if (src.parts == 0) return in[0];
  float2 t = make_float2(0.f, 0.f);
#pragma unroll
  for (int j = 0; j < kRopeRequest; ++j) {
    t.x += j < src.parts ? in[j].x : 0.f;
    t.y += j < src.parts ? in[j].y : 0.f;
  }
  return t;
}
template <bool NT, int P>
__device__ void rope_attention_rows(const RopeAttentionChainArgs &a, int block) {
  extern __shared__ float rowScores[];
  const RopeArgs &q = a.q, &k = a.k;
  const AppendArgs &ap = a.append;
  const ScoresArgs &sc = a.scores;
  long bh = block;
  if (bh >= long(a.values.B) * a.values.A) return;
  float *qrow = rowScores + ((q.T + 3) & ~3);
  float *krow = qrow + ap.D;
  const int p = load_position(q.position);
  const bool inRange = p >= 0 && p < q.T;
  // Every wave's first batch of cache rows below p (rows >= p re-read an early row and are
  // dropped, as in the scores loop) is requested before the rotation and overlaps it; this
  // launch writes only row p of the cache.
  const int wave = threadIdx.x >> 6;
  const bool vector = scores_vector_layout(sc.D);
  const KeyLayout<P> layout(vector ? sc.D : 4 * P);
  const int firstBase = wave * layout.rowsPerBatch();
  const bool early = vector && inRange && p >= 1;
  // With one pair a thread and at most kRopeRequest planes a source, a thread's rotation operands
  // (its q, k and v pairs' planes and the (cos, sin) entry) are requested before the first key
  // batch, so that they are not queued behind the key rows every workgroup requests at once, and
  // added after the batch has been issued (in plane order, as source2 adds them).
  const bool requestFirst = inRange && q.R <= int(blockDim.x) && a.qsrc.parts <= kRopeRequest &&
                            a.ksrc.parts <= kRopeRequest && a.v.parts <= kRopeRequest;
  const int pair = threadIdx.x;
  const long pairIndex = bh * (2L * q.R) + 2 * pair;          // = b*(2R*A) + h*2R + 2r
  float2 qPlanes[kRopeRequest], kPlanes[kRopeRequest], vPlanes[kRopeRequest], pairTable = make_float2(0.f, 0.f);
  if (requestFirst && pair < q.R) {
    pairTable = *reinterpret_cast<const float2 *>(q.table + long(p) * q.R * 2 + 2 * pair);
    request_pair(a.qsrc, q.src, pairIndex, qPlanes);
    request_pair(a.ksrc, k.src, pairIndex, kPlanes);
    request_pair(a.v, ap.v, pairIndex, vPlanes);
  }
  KeyBatch first;
  if (early)
    load_key_batch<NT, P>(first, sc.kc + (long(sc.layer) * sc.B * sc.A + bh) * long(sc.T) * sc.D, sc.D, layout,
                          firstBase, p);
  if (requestFirst) {
    if (pair < q.R) {
      const long row0 = (((long(ap.layer) * ap.B * ap.A) + bh) * ap.T + p) * ap.D;
      const float2 qr = rotate(sum_pair(a.qsrc, qPlanes), pairTable);
      *reinterpret_cast<float2 *>(q.dst + pairIndex) = qr;
      *reinterpret_cast<float2 *>(qrow + 2 * pair) = qr;
      const float2 kr = rotate(sum_pair(a.ksrc, kPlanes), pairTable);
      if (k.dst) *reinterpret_cast<float2 *>(k.dst + pairIndex) = kr;
      *reinterpret_cast<float2 *>(krow + 2 * pair) = kr;
      *reinterpret_cast<float2 *>(ap.kc + row0 + 2 * pair) = kr;
      *reinterpret_cast<float2 *>(ap.vc + row0 + 2 * pair) = sum_pair(a.v, vPlanes);
    }
    if (!vector) __builtin_amdgcn_s_waitcnt(kWaitStores);
  } else if (inRange) {
    // One pair a thread, 64-bit accesses: this rotation runs while every wave holds its first batch
    // of key rows in registers, and the 128-bit form (two pairs a thread, 4-wide partial-plane sums)
    // raised the kernel from 69 to 196 VGPRs with scratch, occupancy 7 -> 2. The rotation and append
    // take ~2 us of the ~85 us launch (large decoder), and the standalone rope and rope -> append_kv
    // kernels use 128-bit accesses.
    const long row0 = (((long(ap.layer) * ap.B * ap.A) + bh) * ap.T + p) * ap.D;
    const float *table = q.table + long(p) * q.R * 2;
    for (int r = threadIdx.x; r < q.R; r += blockDim.x) {
      const long c = bh * (2L * q.R) + 2 * r;        // = b*(2R*A) + h*2R + 2r
      const float2 cs = *reinterpret_cast<const float2 *>(table + 2 * r);
      const float2 qr = rotate(source2(a.qsrc, q.src, c), cs);
      *reinterpret_cast<float2 *>(q.dst + c) = qr;
      *reinterpret_cast<float2 *>(qrow + 2 * r) = qr;
      const float2 kr = rotate(source2(a.ksrc, k.src, c), cs);
      if (k.dst) *reinterpret_cast<float2 *>(k.dst + c) = kr;
      *reinterpret_cast<float2 *>(krow + 2 * r) = kr;
      *reinterpret_cast<float2 *>(ap.kc + row0 + 2 * r) = kr;
      *reinterpret_cast<float2 *>(ap.vc + row0 + 2 * r) = source2(a.v, ap.v, c);
    }
    // The sequential dot product reads the appended key row from the cache after the barrier.
    if (!vector) __builtin_amdgcn_s_waitcnt(kWaitStores);
  }
  __syncthreads();
  // The barrier alone does not wait for vector stores: the waves that appended cache rows wait for
  // them before the barrier that precedes the values (the scores take the key row from LDS).
  attention_chain_row<NT, P>(a.scores, a.softmax, a.values, bh, inRange ? qrow : sc.q + bh * sc.D, p, rowScores,
                             first, early, inRange ? krow : nullptr, inRange && int(threadIdx.x & ~63) < q.R);
}
template <bool NT> __device__ void rope_attention_stream(const RopeAttentionChainArgs &a, int block) {
  switch (score_pieces(a.scores.D)) {
    case 1: rope_attention_rows<NT, 1>(a, block); break;
    case 2: rope_attention_rows<NT, 2>(a, block); break;
    default: rope_attention_rows<NT, 4>(a, block); break;
  }
}
CKL_ENTRY_ATTR(rope__rope__append_kv__attention_scores__softmax__attention_values, RopeAttentionChainArgs,
               rope_attention_stream<false>, kValuesBlock, )
CKL_ENTRY_ATTR(rope__rope__append_kv__attention_scores__softmax__attention_values_nt, RopeAttentionChainArgs,
               rope_attention_stream<true>, kValuesBlock, )

// ------------------------------------------------------------------ pointwise
// add: dst = x + y; multiply: dst = x * y; silu: dst = v / (1 + exp(-v)) (workloads.py:145-167).

template <int Op> __device__ __forceinline__ float binary(float x, float y) { return Op == 0 ? x + y : x * y; }

template <int Op> __device__ void binary_body(const BinaryArgs &a, int block) {
  long i = long(block) * kBlock + threadIdx.x;
  if ((a.n & 3) == 0) {
    if (i >= a.n / 4) return;
    float4 x = reinterpret_cast<const float4 *>(a.x)[i], y = reinterpret_cast<const float4 *>(a.y)[i];
    reinterpret_cast<float4 *>(a.dst)[i] =
        make_float4(binary<Op>(x.x, y.x), binary<Op>(x.y, y.y), binary<Op>(x.z, y.z), binary<Op>(x.w, y.w));
  } else if (i < a.n) {
    a.dst[i] = binary<Op>(a.x[i], a.y[i]);
  }
}
__device__ void add_body(const BinaryArgs &a, int block) { binary_body<0>(a, block); }
__device__ void multiply_body(const BinaryArgs &a, int block) { binary_body<1>(a, block); }
CKL_ENTRY(add, BinaryArgs, add_body)
CKL_ENTRY(multiply, BinaryArgs, multiply_body)

__device__ __forceinline__ float silu(float v) { return v / (1.0f + expf(-v)); }
__device__ void silu_body(const UnaryArgs &a, int block) {
  long i = long(block) * kBlock + threadIdx.x;
  if ((a.n & 3) == 0) {
    if (i >= a.n / 4) return;
    float4 v = reinterpret_cast<const float4 *>(a.src)[i];
    reinterpret_cast<float4 *>(a.dst)[i] = make_float4(silu(v.x), silu(v.y), silu(v.z), silu(v.w));
  } else if (i < a.n) {
    a.dst[i] = silu(a.src[i]);
  }
}
CKL_ENTRY(silu, UnaryArgs, silu_body)

// silu -> multiply as one launch of silu's geometry: element i (or float4 i) is activated,
// written to silu's dst and multiplied by multiply's y in the same thread.
// Both operands' loads (each at most kSourceBatch planes) issued before the activation.
template <bool PlanesS, bool PlanesY> __device__ void silu_multiply_float4(const SiluMultiplyChainArgs &a, long i) {
  const long idx[1] = {4 * i};
  RowSource<1, PlanesS> src;
  RowSource<1, PlanesY> y;
  row_source_issue<1, PlanesS>(a.src, a.silu.src, idx, src);
  row_source_issue<1, PlanesY>(a.y, a.multiply.y, idx, y);
  const float4 v = row_source_value<1, PlanesS>(a.src, src, 0);
  const float4 act = make_float4(silu(v.x), silu(v.y), silu(v.z), silu(v.w));
  if (a.silu.dst) reinterpret_cast<float4 *>(a.silu.dst)[i] = act;   // null: only multiply reads it
  const float4 u = row_source_value<1, PlanesY>(a.y, y, 0);
  reinterpret_cast<float4 *>(a.multiply.dst)[i] =
      make_float4(binary<1>(act.x, u.x), binary<1>(act.y, u.y), binary<1>(act.z, u.z), binary<1>(act.w, u.w));
}

__device__ void silu__multiply_body(const SiluMultiplyChainArgs &a, int block) {
  long i = long(block) * kBlock + threadIdx.x;
  const int n = a.silu.n;
  if ((n & 3) == 0 && a.src.parts <= kSourceBatch && a.y.parts <= kSourceBatch) {
    if (i >= n / 4) return;
    if (a.src.parts > 0) {
      if (a.y.parts > 0) silu_multiply_float4<true, true>(a, i);
      else silu_multiply_float4<true, false>(a, i);
    } else {
      if (a.y.parts > 0) silu_multiply_float4<false, true>(a, i);
      else silu_multiply_float4<false, false>(a, i);
    }
  } else if ((n & 3) == 0) {
    if (i >= n / 4) return;
    float4 v = source4(a.src, a.silu.src, 4 * i);
    float4 act = make_float4(silu(v.x), silu(v.y), silu(v.z), silu(v.w));
    if (a.silu.dst) reinterpret_cast<float4 *>(a.silu.dst)[i] = act;   // null: only multiply reads it
    float4 y = source4(a.y, a.multiply.y, 4 * i);
    reinterpret_cast<float4 *>(a.multiply.dst)[i] =
        make_float4(binary<1>(act.x, y.x), binary<1>(act.y, y.y), binary<1>(act.z, y.z), binary<1>(act.w, y.w));
  } else if (i < n) {
    float act = silu(source1(a.src, a.silu.src, i));
    if (a.silu.dst) a.silu.dst[i] = act;
    a.multiply.dst[i] = binary<1>(act, source1(a.y, a.multiply.y, i));
  }
}
CKL_ENTRY(silu__multiply, SiluMultiplyChainArgs, silu__multiply_body)


// Row-parallel linear chains. With one column tile (O <= 64) and one slice a rowvec workgroup
// holds a whole output row, so the row ops after the linear run in the same workgroup: linear ->
// add -> rms_stats -> rms_apply (the o and down projections of a narrow decoder), and, for any O
// and one slice, the two linears of one x -> silu -> multiply (gate/up). The linear columns are
// computed and combined exactly as linear_rowvec does. For the rms, C <= 64 keeps every value of
// the row in wave 0, the only wave with data in the 256-thread rms kernels, and the sums follow
// their order (float4 t or element t per thread, the wave sum, then the block sum's zeros).
// Row b's linear -> add -> rms_stats -> rms_apply with the row-parallel linear's arithmetic (all
// waves compute their chunk's partial; wave 0 adds them in wave order and finishes the row). Wave 0
// leaves the normalized row in `y` (LDS, C floats) and returns true; the other waves return false
// after the linear. Only a `writer` stores the chain's outputs (the linear's output, the sum, inv
// and the normalized row, each unless the executor cleared its pointer).
template <bool NT>
__device__ __forceinline__ bool front_rows(const LinearAddRmsChainArgs &a, int b, bool writer, float4 *y) {
  __shared__ float red[kVectorWaves][64];
  __shared__ float4 row4[16];
  const LinearArgs &l = a.linear;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int waves = blockDim.x >> 6;
  const int C = a.stats.C;
  float *rowf = reinterpret_cast<float *>(row4);
  const long base = long(b) * C;
  const bool vec = (C & 3) == 0;
  // The add's other operand and the gain are requested ahead of the linear's weights (every wave
  // loads them, unpredicated at clamped indices; wave 0 uses them), so the row ops after the
  // reduction wait for no further memory round trip.
  const float *gain = a.apply.gain + long(a.apply.layer) * C;
  const float other = (a.linearIsY ? a.add.x : a.add.y)[base + min(lane, C - 1)];
  const float4 gain4 = vec ? reinterpret_cast<const float4 *>(gain)[min(lane, C / 4 - 1)] : make_float4(0.f, 0.f, 0.f, 0.f);
  const float gain1 = gain[min(lane, C - 1)];
  red[wave][lane] = rowvec_partial<NT>(l, b, 0, 0);
  __syncthreads();
  if (wave != 0) return false;
  if (lane < C) {
    float v = red[0][lane];
    for (int v2 = 1; v2 < waves; ++v2) v += red[v2][lane];
    if (writer && l.dst) l.dst[long(b) * l.O + lane] = v;   // null: only add reads it
    const float h = a.linearIsY ? binary<0>(other, v) : binary<0>(v, other);
    if (writer) a.add.dst[base + lane] = h;
    rowf[lane] = h;
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float4 h4 = make_float4(0.f, 0.f, 0.f, 0.f);
  float h1 = 0.f, total = 0.f;
  if (vec) {
    if (lane < C / 4) {
      h4 = row4[lane];
      total = add_squares(total, h4);
    }
  } else if (lane < C) {
    h1 = rowf[lane];
    total = __builtin_fmaf(h1, h1, total);
  }
  total = wave_sum(total);
  total = (total + 0.f) + (0.f + 0.f);               // block_sum over four waves, three of them empty
  const float s = rms_inverse(total, C, a.stats.eps);
  if (writer && lane == 0 && a.stats.inv) a.stats.inv[b] = s;  // null: only the chain reads inv
  if (vec) {
    if (lane < C / 4) {
      const float4 r = rms_scale(h4, s, gain4);
      if (writer && a.apply.dst) reinterpret_cast<float4 *>(a.apply.dst + base)[lane] = r;
      y[lane] = r;
    }
  } else if (lane < C) {
    const float r = h1 * s * gain1;
    if (writer && a.apply.dst) a.apply.dst[base + lane] = r;
    reinterpret_cast<float *>(y)[lane] = r;
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  return true;
}

template <bool NT> __device__ void linear_add_rms_stream(const LinearAddRmsChainArgs &a, int block) {
  __shared__ float4 y[16];
  if (block >= a.linear.B) return;
  front_rows<NT>(a, block, true, y);
}
CKL_ENTRY_ATTR(linear_rowvec__add__rms_stats__rms_apply, LinearAddRmsChainArgs, linear_add_rms_stream<false>, 1024, )
CKL_ENTRY_ATTR(linear_rowvec__add__rms_stats__rms_apply_nt, LinearAddRmsChainArgs, linear_add_rms_stream<true>, 1024, )

template <bool NT> __device__ void linear_silu_stream(const LinearSiluChainArgs &a, int block) {
  __shared__ float red[2][kVectorWaves][64];
  const LinearArgs &g = a.gate, &u = a.up;
  const int tn = block % g.tilesN, b = block / g.tilesN;
  if (b >= g.B) return;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int waves = blockDim.x >> 6;
  red[0][wave][lane] = rowvec_partial<NT>(g, b, tn, 0);
  red[1][wave][lane] = rowvec_partial<NT>(u, b, tn, 0);
  __syncthreads();
  const int col = tn * 64 + lane;
  if (wave != 0 || col >= g.O) return;
  float gv = red[0][0][lane], uv = red[1][0][lane];
  for (int v2 = 1; v2 < waves; ++v2) gv += red[0][v2][lane];
  for (int v2 = 1; v2 < waves; ++v2) uv += red[1][v2][lane];
  const long i = long(b) * g.O + col;
  if (g.dst) g.dst[i] = gv;                          // null: only the chain reads them
  if (u.dst) u.dst[i] = uv;
  const float act = silu(gv);
  if (a.silu.dst) a.silu.dst[i] = act;
  a.multiply.dst[i] = binary<1>(act, uv);
}
CKL_ENTRY_ATTR(linear_rowvec__linear_rowvec__silu__multiply, LinearSiluChainArgs, linear_silu_stream<false>, 1024, )
CKL_ENTRY_ATTR(linear_rowvec__linear_rowvec__silu__multiply_nt, LinearSiluChainArgs, linear_silu_stream<true>, 1024, )

// linear -> add -> rms_stats -> rms_apply -> (linear, linear) -> silu -> multiply, for single-wave
// row-parallel linears (64-thread blocks: C <= 64, so the first linear's rows and the normalized
// row fit one wave): workgroup (tn, b) of the gate/up grid requests its gate and up weights with
// the first linear's, recomputes row b's first chain (front_rows), takes the normalized row from
// LDS as the x of its gate/up tile, and finishes as linear_silu_stream. Only the tn = 0 workgroup
// writes the first chain's outputs.
template <bool NT> __device__ void linear_add_rms_silu_stream(const LinearAddRmsSiluChainArgs &a, int block) {
  __shared__ float4 y4[16];
  const LinearSiluChainArgs &k = a.back;
  const LinearArgs &g = k.gate, &u = k.up;
  const int tn = block % g.tilesN, b = block / g.tilesN;
  if (b >= g.B) return;
  const int lane = threadIdx.x & 63;
  const float *yf = reinterpret_cast<const float *>(y4);
  const RowvecSlice gs = rowvec_slice(g, tn * 64 + lane, 0, 1, 0), us = rowvec_slice(u, tn * 64 + lane, 0, 1, 0);
  float gw[kVectorRows], uw[kVectorRows];
  rowvec_load<NT>(g, gs, gw);
  rowvec_load<NT>(u, us, uw);
  if (!front_rows<NT>(a.front, b, tn == 0, y4)) return;
  const float gv = rowvec_dot(gs, gw, [&](int kk) { return yf[kk]; });
  const float uv = rowvec_dot(us, uw, [&](int kk) { return yf[kk]; });
  const int col = tn * 64 + lane;
  if (col >= g.O) return;
  const long i = long(b) * g.O + col;
  if (g.dst) g.dst[i] = gv;                          // null: only the chain reads them
  if (u.dst) u.dst[i] = uv;
  const float act = silu(gv);
  if (k.silu.dst) k.silu.dst[i] = act;
  k.multiply.dst[i] = binary<1>(act, uv);
}
CKL_ENTRY_ATTR(linear_rowvec__add__rms_stats__rms_apply__linear_rowvec__linear_rowvec__silu__multiply,
               LinearAddRmsSiluChainArgs, linear_add_rms_silu_stream<false>, 64, )
CKL_ENTRY_ATTR(linear_rowvec__add__rms_stats__rms_apply__linear_rowvec__linear_rowvec__silu__multiply_nt,
               LinearAddRmsSiluChainArgs, linear_add_rms_silu_stream<true>, 64, )

// embedding -> rms_stats -> rms_apply -> `count` single-wave row-parallel linears of the normalized
// rows, C <= 64 and C % 4 == 0 (64-thread blocks): member m owns blocks [start[m], start[m+1]) of
// its tilesN x B grid. Each workgroup requests its tile's weights, gathers its row's embedding (a
// float4 per lane) and normalizes it with the chain's arithmetic (the 256-thread row's block sum,
// in which only wave 0 holds data), then computes its tile from the normalized row in LDS with the
// single-wave linear's arithmetic. Member 0's tile-0 workgroups write the row chain's outputs.
template <bool NT> __device__ void embedding_rms_linears_stream(const EmbeddingRmsLinearsChainArgs &a, int block) {
  __shared__ float4 y4[16];
  int m = 0;
  while (m + 1 < a.count && block >= a.start[m + 1]) ++m;
  const LinearArgs &l = a.back[m];
  const int local = block - a.start[m];
  const int tn = local % l.tilesN, b = local / l.tilesN;
  if (b >= l.B) return;
  const int lane = threadIdx.x & 63;
  const RowvecSlice ls = rowvec_slice(l, tn * 64 + lane, 0, 1, 0);
  float lw[kVectorRows];
  rowvec_load<NT>(l, ls, lw);
  const EmbeddingRmsChainArgs &f = a.front;
  const EmbeddingArgs &e = f.embedding;
  const int n4 = e.C / 4, c = min(lane, n4 - 1);
  const float4 g = reinterpret_cast<const float4 *>(f.apply.gain + long(f.apply.layer) * e.C)[c];
  const int token = e.tokens[b];
  const bool valid = token >= 0 && token < e.V;
  const float nan = __builtin_nanf("");
  float4 v = reinterpret_cast<const float4 *>(e.table + long(valid ? token : 0) * e.C)[c];
  v = valid ? v : make_float4(nan, nan, nan, nan);
  float total = lane < n4 ? add_squares(0.f, v) : 0.f;
  total = wave_sum(total);
  total = (total + 0.f) + (0.f + 0.f);               // block_sum over four waves, three of them empty
  const float s = rms_inverse(total, e.C, f.stats.eps);
  const float4 y = rms_scale(v, s, g);
  if (m == 0 && tn == 0) {
    if (lane < n4) {
      reinterpret_cast<float4 *>(e.dst + long(b) * e.C)[lane] = v;
      if (f.apply.dst) reinterpret_cast<float4 *>(f.apply.dst + long(b) * e.C)[lane] = y;
    }
    if (lane == 0 && f.stats.inv) f.stats.inv[b] = s;   // null: only the chain reads inv
  }
  if (lane < n4) y4[lane] = y;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const float *yf = reinterpret_cast<const float *>(y4);
  const float out = rowvec_dot(ls, lw, [&](int kk) { return yf[kk]; });
  const int col = tn * 64 + lane;
  if (col < l.O && l.dst) l.dst[long(b) * l.O + col] = out;
}
CKL_ENTRY_ATTR(embedding__rms_stats__rms_apply__linear_rowvec__linear_rowvec__linear_rowvec,
               EmbeddingRmsLinearsChainArgs, embedding_rms_linears_stream<false>, 64, )
CKL_ENTRY_ATTR(embedding__rms_stats__rms_apply__linear_rowvec__linear_rowvec__linear_rowvec_nt,
               EmbeddingRmsLinearsChainArgs, embedding_rms_linears_stream<true>, 64, )

// ------------------------------------------------------------------ greedy
// tokens[b] = history[p, b] = first index of the maximum logit (strict '>' scan from index 0,
// workloads.py:170-183): NaN logits never win, a NaN logit 0 is never displaced, +0 and -0 tie.
// A row of at most kGreedyRowLoads float4 per thread (V % 4 == 0; the library launches 1024
// threads for rows above kGreedyChunk logits) is one workgroup: each thread scans its float4s
// in index order with a strict '>' from -inf, so it keeps the first index of its maximum and
// never takes a NaN, and the threads' (value, index) pairs are reduced as 64-bit keys (ordered
// value bits << 32 | ~index: the maximum key is the largest value at the smallest index, -0 and
// +0 tie). A row with no key above -inf (all -inf or NaN) and a row whose logit 0 is NaN pick 0.
// Longer rows are cut into `chunks` slices of kGreedyChunk logits, one 256-thread workgroup
// each, which fold their slice's key into the row's key with an agent-scope atomic max and bump
// the row's counter; the last workgroup writes the token and resets key and counter.
// workspace: uint64 key[B], uint32 counter[B], then the uint32 row count of the greedy ->
// advance chain.
constexpr int kGreedyChunk = 4096;
constexpr int kGreedyRowLoads = 8;
constexpr int kGreedyMaxWaves = 16;

__device__ __forceinline__ unsigned long long greedy_key(float v, int index) {
  unsigned bits = __float_as_uint(v == 0.f ? 0.f : v);     // -0 ties with +0
  unsigned ordered = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
  return (static_cast<unsigned long long>(ordered) << 32) | (0xFFFFFFFFu - unsigned(index));
}

// The key of this thread's float4s of a one-workgroup row (see above).
__device__ __forceinline__ unsigned long long greedy_row_key(const float *logits, int V) {
  const float4 *row = reinterpret_cast<const float4 *>(logits);
  const int n4 = V / 4, step = blockDim.x;
  float4 x[kGreedyRowLoads];
#pragma unroll
  for (int u = 0; u < kGreedyRowLoads; ++u) x[u] = row[min(u * step + int(threadIdx.x), n4 - 1)];
  float best = -__builtin_inff();
  int index = -1;
#pragma unroll
  for (int u = 0; u < kGreedyRowLoads; ++u) {
    const int c = u * step + int(threadIdx.x);
    if (c < n4) {
      const float v[4] = {x[u].x, x[u].y, x[u].z, x[u].w};
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (v[e] > best) {
          best = v[e];
          index = 4 * c + e;
        }
    }
  }
  return index < 0 ? 0ull : greedy_key(best, index);
}

// Returns true in thread 0 of the workgroup that wrote row b's token; *position is the position
// it read.
__device__ __forceinline__ bool greedy_block(const GreedyArgs &a, int block, int *position) {
  __shared__ unsigned long long bestKey[kGreedyMaxWaves];
  const int b = block / a.chunks, chunk = block % a.chunks;
  if (b >= a.B) return false;
  const float *logits = a.logits + long(b) * a.V;
  // Thread 0 requests logit 0 and the position with the row, not after the reduction.
  float first = 0.f;
  int p = 0;
  if (threadIdx.x == 0) {
    first = logits[0];
    p = load_position(a.position);
  }
  unsigned long long key = 0;                               // below every real key
  if (a.chunks == 1 && (a.V & 3) == 0 && a.V / 4 <= kGreedyRowLoads * int(blockDim.x)) {
    key = greedy_row_key(logits, a.V);
  } else {
    const int v0 = chunk * kGreedyChunk, v1 = min(v0 + kGreedyChunk, a.V);
    float x[kGreedyChunk / kBlock];
#pragma unroll
    for (int u = 0; u < kGreedyChunk / kBlock; ++u) x[u] = logits[min(v0 + u * kBlock + int(threadIdx.x), v1 - 1)];
#pragma unroll
    for (int u = 0; u < kGreedyChunk / kBlock; ++u) {
      int k = v0 + u * kBlock + threadIdx.x;
      if (k < v1 && x[u] == x[u]) key = max(key, greedy_key(x[u], k));
    }
  }
#pragma unroll
  for (int offset = 32; offset > 0; offset /= 2) {
    unsigned long long other = __shfl_xor(key, offset);
    key = max(key, other);
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
  if (lane == 0) bestKey[wave] = key;
  __syncthreads();
  if (threadIdx.x != 0) return false;
  for (int w = 1; w < waves; ++w) key = max(key, bestKey[w]);
  bool finish = a.chunks == 1;
  if (!finish) {
    unsigned long long *keys = reinterpret_cast<unsigned long long *>(a.workspace);
    unsigned *counters = reinterpret_cast<unsigned *>(a.workspace + 8 * a.B);
    __hip_atomic_fetch_max(keys + b, key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(kWaitStores);
    unsigned previous = __hip_atomic_fetch_add(counters + b, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    finish = previous == unsigned(a.chunks - 1);
    if (finish) {
      key = __hip_atomic_load(keys + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(keys + b, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(counters + b, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if (!finish) return false;
  int winner = (first != first || key == 0) ? 0 : int(0xFFFFFFFFu - unsigned(key & 0xFFFFFFFFu));
  a.tokens[b] = winner;
  if (p >= 0 && p < a.T) a.history[long(p) * a.B + b] = winner;
  *position = p;
  return true;
}
__device__ void greedy_body(const GreedyArgs &a, int block) {
  int p;
  greedy_block(a, block, &p);
}
CKL_ENTRY_ATTR(greedy, GreedyArgs, greedy_body, 1024, )

// greedy -> advance as one launch of greedy's geometry: the thread that writes a row's token
// (its position load has returned: the history store's address uses it) counts the row; the one
// that counts the last row (every row has read the position by then) resets the count and
// stores position + 1, which is what advance computes.
__device__ void greedy__advance_body(const GreedyAdvanceChainArgs &a, int block) {
  int p;
  if (!greedy_block(a.greedy, block, &p)) return;
  unsigned *rows = reinterpret_cast<unsigned *>(a.greedy.workspace + 12 * a.greedy.B);
  unsigned previous = __hip_atomic_fetch_add(rows, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (previous == unsigned(a.greedy.B - 1)) {
    __hip_atomic_store(rows, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    a.advance.position[0] = p + 1;
  }
}
CKL_ENTRY_ATTR(greedy__advance, GreedyAdvanceChainArgs, greedy__advance_body, 1024, )

// linear -> greedy -> advance for a single-wave row-parallel linear of at most 16 tiles (the LM head
// of a narrow decoder): workgroup b computes row b's logits, wave w the columns of tile w with the
// linear's arithmetic, writes them, and picks the token from the values in registers: each lane's
// key (value bits, ~column) when its logit is above -inf, reduced as greedy_block does (logit 0
// NaN or no key above -inf: token 0); the row is then counted as in greedy__advance_body.
template <bool NT> __device__ void linear_greedy_advance_stream(const LinearGreedyAdvanceChainArgs &a, int block) {
  __shared__ unsigned long long bestKey[kGreedyMaxWaves];
  const LinearArgs &l = a.linear;
  const GreedyArgs &g = a.pick.greedy;
  const int b = block;
  if (b >= l.B) return;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), waves = blockDim.x >> 6;
  int p = 0;
  if (threadIdx.x == 0) p = load_position(g.position);
  const int col = wave * 64 + lane;
  const RowvecSlice sl = rowvec_slice(l, col, 0, 1, 0);
  const float *__restrict__ xr = l.x + long(b) * l.I;
  float wv[kVectorRows];
  rowvec_load<NT>(l, sl, wv);
  const float v = rowvec_dot(sl, wv, [&](int k) { return xr[k]; });
  if (col < l.O) l.dst[long(b) * l.O + col] = v;
  unsigned long long key = col < g.V && v > -__builtin_inff() ? greedy_key(v, col) : 0ull;
#pragma unroll
  for (int offset = 32; offset > 0; offset /= 2) key = max(key, __shfl_xor(key, offset));
  if (lane == 0) bestKey[wave] = key;
  __syncthreads();
  if (threadIdx.x != 0) return;
  for (int w = 1; w < waves; ++w) key = max(key, bestKey[w]);
  const int winner = (v != v || key == 0) ? 0 : int(0xFFFFFFFFu - unsigned(key & 0xFFFFFFFFu));   // v: logit 0
  g.tokens[b] = winner;
  if (p >= 0 && p < g.T) g.history[long(p) * g.B + b] = winner;
  unsigned *rows = reinterpret_cast<unsigned *>(g.workspace + 12 * g.B);
  if (__hip_atomic_fetch_add(rows, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == unsigned(g.B - 1)) {
    __hip_atomic_store(rows, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    a.pick.advance.position[0] = p + 1;
  }
}
CKL_ENTRY_ATTR(linear_rowvec__greedy__advance, LinearGreedyAdvanceChainArgs, linear_greedy_advance_stream<false>, 1024, )
CKL_ENTRY_ATTR(linear_rowvec__greedy__advance_nt, LinearGreedyAdvanceChainArgs, linear_greedy_advance_stream<true>, 1024, )

// ------------------------------------------------------------------ advance
// position[0] += 1   (workloads.py:186-188)
__device__ void advance_body(const AdvanceArgs &a, int block) {
  if (block == 0 && threadIdx.x == 0) a.position[0] = a.position[0] + 1;
}
CKL_ENTRY(advance, AdvanceArgs, advance_body)

// ------------------------------------------------------------------ vector update
// dst[i] = src[i] + bias for i < N   (examples/vector_pipeline.py:11-16)
__device__ void update_body(const UpdateArgs &a, int block) {
  long i = long(block) * kBlock + threadIdx.x;
  if ((a.n & 3) == 0) {
    if (i >= a.n / 4) return;
    float4 v = reinterpret_cast<const float4 *>(a.src)[i];
    reinterpret_cast<float4 *>(a.dst)[i] = make_float4(v.x + a.bias, v.y + a.bias, v.z + a.bias, v.w + a.bias);
  } else if (i < a.n) {
    a.dst[i] = a.src[i] + a.bias;
  }
}
CKL_ENTRY(update, UpdateArgs, update_body)
