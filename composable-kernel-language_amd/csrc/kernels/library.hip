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

#define CKL_ALIGN __attribute__((aligned(8)))
constexpr int kMaxGroup = 4;
constexpr int kBlock = 256;

template <typename Args> struct CKL_ALIGN Group {
  Args m[kMaxGroup];
  int start[kMaxGroup + 1];
  int count;
};

#define CKL_ENTRY_ATTR(name, Args, body, attributes)                                                 \
  extern "C" __global__ __launch_bounds__(kBlock) attributes void ckl_##name(const Args a) { body(a, blockIdx.x); } \
  extern "C" __global__ __launch_bounds__(kBlock) attributes void ckl_##name##_group(const Group<Args> g) { \
    int b = blockIdx.x, m = 0;                                                                        \
    while (m + 1 < g.count && b >= g.start[m + 1]) ++m;                                               \
    body(g.m[m], b - g.start[m]);                                                                     \
  }
#define CKL_ENTRY(name, Args, body) CKL_ENTRY_ATTR(name, Args, body, )
// Streaming kernels that keep several loads in flight per lane trade occupancy for registers.
#define CKL_TWO_WAVES __attribute__((amdgpu_waves_per_eu(1, 2)))

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

// ------------------------------------------------------------------ embedding
// dst[b, c] = table[tokens[b], c]   (workloads.py:33-39)
struct CKL_ALIGN EmbeddingArgs { const int *tokens; const float *table; float *dst; int B, C, V; };
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
// inv[b] = rsqrt(sum_c x[b,c]^2 / C + eps)   (workloads.py:42-49); one wave per row.
struct CKL_ALIGN RmsStatsArgs { const float *x; float *inv; float eps; int B, C; };
__device__ void rms_stats_body(const RmsStatsArgs &a, int block) {
  int lane = threadIdx.x & 63;
  int row = block * (kBlock / 64) + (threadIdx.x >> 6);
  if (row >= a.B) return;
  const float *x = a.x + long(row) * a.C;
  float total = 0.f;
  if ((a.C & 3) == 0) {
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    for (int c = lane; c < a.C / 4; c += 64) {
      float4 v = x4[c];
      total += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
  } else {
    for (int c = lane; c < a.C; c += 64) total += x[c] * x[c];
  }
  total = wave_sum(total);
  if (lane == 0) a.inv[row] = 1.0f / __fsqrt_rn(total / float(a.C) + a.eps);
}
CKL_ENTRY(rms_stats, RmsStatsArgs, rms_stats_body)

// ------------------------------------------------------------------ rms_apply
// dst[b, c] = x[b, c] * inv[b] * gain[layer, c]   (workloads.py:52-58)
struct CKL_ALIGN RmsApplyArgs { const float *x; const float *inv; const float *gain; float *dst; int B, C, layer; };
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
    reinterpret_cast<float4 *>(a.dst + long(b) * a.C)[c4] = make_float4(x.x * s * g.x, x.y * s * g.y, x.z * s * g.z, x.w * s * g.w);
  } else {
    if (i >= long(a.B) * a.C) return;
    int b = int(i / a.C), c = int(i % a.C);
    a.dst[i] = a.x[i] * a.inv[b] * gain[c];
  }
}
CKL_ENTRY(rms_apply, RmsApplyArgs, rms_apply_body)

// ------------------------------------------------------------------ linear
// dst[b, o] = sum_i x[b, i] * w[layer, i, o]   (workloads.py:61-69)
//
// The weight matrix is streamed from HBM exactly once per launch. The grid is
// rowTiles x kSplit x tilesN workgroups of 256 threads (4 waves): workgroup (rt, kg, tn) owns
// output tile tn (a column range) for batch-row tile rt over the reduction slice
// [kg*kChunk, (kg+1)*kChunk), which its 4 waves share.
//   ckl_linear (vector, B <= 16): lane <-> output column (64 per tile), rows accumulated in
//           VGPRs, x staged through LDS;
//   ckl_linear_mfma1/4 (f32 MFMA, B > 16): v_mfma_f32_32x32x2f32 over 32 batch rows; each lane loads
//           J = 1 / 4 consecutive weight columns with one vector load, and MFMA j accumulates
//           columns {J*c + j}, so one wave owns a 32 x 32J tile. The K index is permuted so the
//           A operand (x) is one float4 load per 8 reduction rows.
// Partial tiles of the 4 waves are added through LDS in wave order. With kSplit > 1 every
// workgroup writes its partial tile to the workspace with agent-coherent stores and bumps the
// tile's completion counter; the last one to arrive adds the kSplit partials in kg order,
// writes dst and resets the counter, so the result is deterministic and replays need no reset.
//
// workspace layout: counters (rowTiles*tilesN uint32, padded to 256 B), then partial tiles
// float[kSplit][rowTiles*rowsPerTile][O] (rowsPerTile = 32 for MFMA, B for the vector path).
struct CKL_ALIGN LinearArgs {
  const float *x; const float *w; float *dst; int B, I, O, layer;
  int tilesN, kSplit, kChunk, pad;
  unsigned char *workspace;
};
constexpr int kVectorRows = 16;

typedef float floatx16 __attribute__((ext_vector_type(16)));
// s_waitcnt immediate (gfx9 encoding) that waits for vmcnt == 0 only: outstanding vector memory
// operations of the wave, stores included, have completed.
constexpr int kWaitStores = 0x0F70;

__device__ __forceinline__ int counter_bytes(int count) { return (count * 4 + 255) & ~255; }

// Cross-workgroup partial tiles live in the workspace and are written and read only with
// agent-scope atomic stores/loads (sc1: coherent across the MI355X's per-XCD L2 caches without
// the whole-L2 writeback/invalidate an agent-scope fence costs).
__device__ __forceinline__ void partial_store(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float partial_load(const float *p) {
  return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Returns true in every thread of the last workgroup to finish a split tile. Only wave 0 of a
// workgroup writes its partial tile; it waits until those agent-coherent stores have completed
// (s_waitcnt vmcnt(0)) before bumping the tile's completion counter, so the workgroup that
// observes the final count reads every partial through the same coherent path.
__device__ __forceinline__ bool split_arrive(unsigned *counter, int parts, int wave) {
  __shared__ int last;
  if (wave == 0) {
    __builtin_amdgcn_s_waitcnt(kWaitStores);
    if (threadIdx.x == 0) {
      unsigned previous = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      int isLast = previous == unsigned(parts - 1);
      if (isLast) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last = isLast;
    }
  }
  __syncthreads();
  return last;
}

// Adds the kSplit partial tiles (rows [r0, r0+rows), columns [c0, c0+cols)) in split order
// and writes dst.
__device__ void split_finish(const LinearArgs &a, const float *partial, long planeStride, int r0, int rows, int c0,
                             int cols) {
  for (int e = threadIdx.x; e < rows * cols; e += kBlock) {
    int r = r0 + e / cols, c = c0 + e % cols;
    if (r >= a.B || c >= a.O) continue;
    float total = 0.f;
    for (int g = 0; g < a.kSplit; ++g) total += partial_load(partial + g * planeStride + long(r) * a.O + c);
    a.dst[long(r) * a.O + c] = total;
  }
}

template <int J> __device__ __forceinline__ void load_columns(float (&out)[J], const float *p) {
  if constexpr (J == 4) {
    float4 v = *reinterpret_cast<const float4 *>(p);
    out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
  } else if constexpr (J == 2) {
    float2 v = *reinterpret_cast<const float2 *>(p);
    out[0] = v.x; out[1] = v.y;
  } else {
    out[0] = *p;
  }
}

// 16 reduction rows of one lane (two 8-row super-steps): x[row][k+8u .. k+8u+3] and the lane's
// J weight columns of rows k+8u+i. Full stages load without predicates or selects, so the next
// stage's loads stay in flight under the current stage's MFMAs: a batch row >= B (x row clamped
// to 0) only feeds output row >= B and a column >= O (clamped to column 0) only feeds output
// column >= O, neither of which is stored. The tail stage zeroes reduction rows past k1 (their
// addresses are clamped to row k1-1).
template <int J> struct MfmaStage {
  float x[2][4];
  float w[2][4][J];
};

template <int J, bool Tail>
__device__ __forceinline__ void mfma_load(MfmaStage<J> &st, const float *xr, const float *w, long O, int k, int k1) {
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int kk = k + 8 * u;
    if constexpr (!Tail) {
      float4 v = *reinterpret_cast<const float4 *>(xr + kk);
      st.x[u][0] = v.x; st.x[u][1] = v.y; st.x[u][2] = v.z; st.x[u][3] = v.w;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (Tail) {
        const bool inside = kk + i < k1;
        const int kr = min(kk + i, k1 - 1);
        st.x[u][i] = inside ? xr[kr] : 0.f;
        float c[J];
        load_columns<J>(c, w + long(kr) * O);
#pragma unroll
        for (int j = 0; j < J; ++j) st.w[u][i][j] = inside ? c[j] : 0.f;
      } else {
        load_columns<J>(st.w[u][i], w + long(kk + i) * O);
      }
    }
  }
}

template <int J> __device__ __forceinline__ void mfma_compute(const MfmaStage<J> &st, floatx16 (&acc)[J]) {
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < J; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(st.x[u][i], st.w[u][i][j], acc[j], 0, 0, 0);
}

template <int J> __device__ void linear_mfma(const LinearArgs &a, int block, float *smem) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform: scalar loop control
  const int m = lane & 31, s = lane >> 5;
  const int tn = block % a.tilesN, rest = block / a.tilesN;
  const int kg = rest % a.kSplit, rt = rest / a.kSplit;
  const int n = tn * 32 * J + J * m;               // first of this lane's J columns
  const bool colOk = n < a.O;                      // host guarantees O % J == 0
  const int row = rt * 32 + m;
  const bool rowOk = row < a.B;
  const float *xr = a.x + long(rowOk ? row : 0) * a.I;
  const float *w = a.w + long(a.layer) * a.I * a.O + (colOk ? n : 0);
  const int kb0 = min(kg * a.kChunk, a.I), kb1 = min(kb0 + a.kChunk, a.I);

  floatx16 acc[J];
#pragma unroll
  for (int j = 0; j < J; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = 0.f;

  // The slice is cut into 16-row stages dealt round-robin to the 4 waves (wave w takes stages
  // w, w+4, ...), so the waves of a workgroup stream neighbouring weight rows at any moment.
  // Full stages are double-buffered: stage u+1's loads are in flight while stage u feeds the
  // MFMAs. The loop body has no conditional loads (the compiler would sink them into the
  // condition and drain the load queue at the join); with an even stage count the last prefetch
  // re-reads the last stage, an L2 hit. sched_barrier keeps each stage's loads issued as one
  // group ahead of the other stage's MFMAs. A ragged last stage is handled by its owner.
  const int fullTotal = (kb1 - kb0) / 16;
  const int full = fullTotal > wave ? (fullTotal - wave + 3) / 4 : 0;
  const int k = kb0 + 16 * wave + 4 * s;               // this lane's row in the wave's first stage
  const int k1 = kb1;
  MfmaStage<J> sa, sb;
  int t = 0;
  if (full > 0) mfma_load<J, false>(sa, xr, w, a.O, k, k1);
  for (; t + 1 < full; t += 2) {
    mfma_load<J, false>(sb, xr, w, a.O, k + 64 * (t + 1), k1);
    __builtin_amdgcn_sched_barrier(0);
    mfma_compute<J>(sa, acc);
    __builtin_amdgcn_sched_barrier(0);
    mfma_load<J, false>(sa, xr, w, a.O, k + 64 * min(t + 2, full - 1), k1);
    __builtin_amdgcn_sched_barrier(0);
    mfma_compute<J>(sb, acc);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (t < full) mfma_compute<J>(sa, acc);
  if (kb0 + 16 * fullTotal < kb1 && fullTotal % 4 == wave) {
    mfma_load<J, true>(sa, xr, w, a.O, kb0 + 16 * fullTotal + 4 * s, k1);
    mfma_compute<J>(sa, acc);
  }

  // Waves 1..3 hand their tiles to wave 0 through LDS; wave 0 adds them in wave order.
  if (wave > 0) {
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) smem[(((wave - 1) * J + j) * 16 + r) * 64 + lane] = acc[j][r];
  }
  __syncthreads();
  const int rowTiles = (a.B + 31) / 32;
  float *partial = reinterpret_cast<float *>(a.workspace + counter_bytes(rowTiles * a.tilesN));
  if (wave == 0) {
#pragma unroll 1
    for (int v = 1; v < 4; ++v)
#pragma unroll
      for (int j = 0; j < J; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[j][r] += smem[(((v - 1) * J + j) * 16 + r) * 64 + lane];
    // D[i][c] of MFMA j: i = 8*(r/4) + 4*s + r%4, c = lane%32 -> column n + j.
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int i = rt * 32 + 8 * (r / 4) + 4 * s + (r % 4);
      if (!colOk) continue;
      if (a.kSplit > 1) {
        float *p = partial + long(kg) * rowTiles * 32 * a.O + long(i) * a.O + n;
#pragma unroll
        for (int j = 0; j < J; ++j) partial_store(p + j, acc[j][r]);
      } else if (i < a.B) {
        float *p = a.dst + long(i) * a.O + n;
        if constexpr (J == 4) *reinterpret_cast<float4 *>(p) = make_float4(acc[0][r], acc[1][r], acc[2][r], acc[3][r]);
        else if constexpr (J == 2) *reinterpret_cast<float2 *>(p) = make_float2(acc[0][r], acc[1][r]);
        else *p = acc[0][r];
      }
    }
  }
  if (a.kSplit > 1) {
    unsigned *counters = reinterpret_cast<unsigned *>(a.workspace);
    if (split_arrive(counters + rt * a.tilesN + tn, a.kSplit, wave))
      split_finish(a, partial, long(rowTiles) * 32 * a.O, rt * 32, 32, tn * 32 * J, 32 * J);
  }
}

// Vector path: lane <-> column; x[B, kChunk slice] staged in LDS; B <= kVectorRows.
__device__ void linear_vector(const LinearArgs &a, int block, float *smem) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int tn = block % a.tilesN, kg = block / a.tilesN;
  const int col = tn * 64 + lane;
  const bool colOk = col < a.O;
  const int kb0 = kg * a.kChunk, kb1 = min(kb0 + a.kChunk, a.I);
  float *xs = smem;                                // [B][kChunk]
  float *red = smem + a.B * a.kChunk;              // [3][B][64]
  for (int e = threadIdx.x; e < a.B * a.kChunk; e += kBlock) {
    int r = e / a.kChunk, k = e % a.kChunk;
    xs[e] = kb0 + k < kb1 ? a.x[long(r) * a.I + kb0 + k] : 0.f;
  }
  __syncthreads();
  const int quarter = a.kChunk / 4;
  const int k0 = wave * quarter, k1 = min(k0 + quarter, kb1 - kb0);
  const float *w = a.w + long(a.layer) * a.I * a.O + long(kb0) * a.O + (colOk ? col : 0);
  float acc[kVectorRows];
#pragma unroll
  for (int r = 0; r < kVectorRows; ++r) acc[r] = 0.f;
  int k = k0;
  for (; k + 8 <= k1; k += 8) {
    float wv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) wv[u] = colOk ? w[long(k + u) * a.O] : 0.f;
#pragma unroll
    for (int u = 0; u < 8; ++u)
#pragma unroll
      for (int r = 0; r < kVectorRows; ++r)
        if (r < a.B) acc[r] += xs[r * a.kChunk + k + u] * wv[u];
  }
  for (; k < k1; ++k) {
    float wv = colOk ? w[long(k) * a.O] : 0.f;
#pragma unroll
    for (int r = 0; r < kVectorRows; ++r)
      if (r < a.B) acc[r] += xs[r * a.kChunk + k] * wv;
  }
  if (wave > 0)
#pragma unroll
    for (int r = 0; r < kVectorRows; ++r)
      if (r < a.B) red[((wave - 1) * a.B + r) * 64 + lane] = acc[r];
  __syncthreads();
  float *partial = reinterpret_cast<float *>(a.workspace + counter_bytes(a.tilesN));
  if (wave == 0 && colOk) {
#pragma unroll
    for (int r = 0; r < kVectorRows; ++r) {
      if (r >= a.B) continue;
      float v = ((acc[r] + red[r * 64 + lane]) + red[(a.B + r) * 64 + lane]) + red[(2 * a.B + r) * 64 + lane];
      if (a.kSplit > 1) partial_store(partial + long(kg) * a.B * a.O + long(r) * a.O + col, v);
      else a.dst[long(r) * a.O + col] = v;
    }
  }
  if (a.kSplit > 1) {
    unsigned *counters = reinterpret_cast<unsigned *>(a.workspace);
    if (split_arrive(counters + tn, a.kSplit, wave)) split_finish(a, partial, long(a.B) * a.O, 0, a.B, tn * 64, 64);
  }
}

__device__ void linear_body(const LinearArgs &a, int block) {
  extern __shared__ float smem[];
  linear_vector(a, block, smem);
}
__device__ void linear_mfma1_body(const LinearArgs &a, int block) {
  extern __shared__ float smem[];
  linear_mfma<1>(a, block, smem);
}
__device__ void linear_mfma4_body(const LinearArgs &a, int block) {
  extern __shared__ float smem[];
  linear_mfma<4>(a, block, smem);
}
CKL_ENTRY(linear, LinearArgs, linear_body)
CKL_ENTRY(linear_mfma1, LinearArgs, linear_mfma1_body)
CKL_ENTRY_ATTR(linear_mfma4, LinearArgs, linear_mfma4_body, CKL_TWO_WAVES)

// ------------------------------------------------------------------ rope
// Adjacent-pair rotation at position p (workloads.py:72-85):
//   dst[b,c] = s[b,c]*cos - s[b,c+1]*sin; dst[b,c+1] = s[b,c]*sin + s[b,c+1]*cos, c = h*2R + 2r.
struct CKL_ALIGN RopeArgs { const float *src; const float *table; const int *position; float *dst; int B, A, R, T; };
__device__ void rope_body(const RopeArgs &a, int block) {
  long i = long(block) * kBlock + threadIdx.x;
  long pairs = long(a.B) * a.A * a.R;
  if (i >= pairs) return;
  int p = load_position(a.position);
  if (p < 0 || p >= a.T) return;
  int r = int(i % a.R);
  long bh = i / a.R;
  int h = int(bh % a.A), b = int(bh / a.A);
  long c = long(b) * (2L * a.R * a.A) + long(h) * (2 * a.R) + 2 * r;
  float2 s = *reinterpret_cast<const float2 *>(a.src + c);
  float2 cs = *reinterpret_cast<const float2 *>(a.table + (long(p) * a.R + r) * 2);
  *reinterpret_cast<float2 *>(a.dst + c) = make_float2(s.x * cs.x - s.y * cs.y, s.x * cs.y + s.y * cs.x);
}
CKL_ENTRY(rope, RopeArgs, rope_body)

// ------------------------------------------------------------------ append_kv
// kc[layer,b,h,p,d] = k[b,h*D+d]; vc[...] = v[...]   (workloads.py:88-97)
struct CKL_ALIGN AppendArgs { const float *k; const float *v; float *kc; float *vc; const int *position; int L, B, A, T, D, layer; };
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

// ------------------------------------------------------------------ attention_scores
// scores[b,h,t] = (sum_d q[b,h*D+d] * kc[layer,b,h,t,d]) * scale for t <= p (workloads.py:100-111).
// One block per (b, h, 256-row chunk); lane groups of D/4 lanes reduce one cache row each.
struct CKL_ALIGN ScoresArgs { const float *q; const float *kc; const int *position; float *scores; float scale; int L, B, A, T, D, layer; };
__device__ void attention_scores_body(const ScoresArgs &a, int block) {
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
  if ((a.D & 3) == 0 && a.D <= 256 && (64 % (a.D / 4)) == 0) {
    int width = a.D / 4;                         // lanes per row
    int rowsPerWave = 64 / width;
    int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int sub = lane / width, part = lane % width;
    float4 qv = reinterpret_cast<const float4 *>(q)[part];
    for (int t = t0 + wave * rowsPerWave + sub; t - sub < tEnd; t += 4 * rowsPerWave) {
      float s = 0.f;
      if (t < tEnd) {
        float4 kv = reinterpret_cast<const float4 *>(keys + long(t) * a.D)[part];
        s = qv.x * kv.x + qv.y * kv.y + qv.z * kv.z + qv.w * kv.w;
      }
      s = group_sum(s, width);
      if (part == 0 && t < tEnd) scores[t] = s * a.scale;
    }
  } else {
    for (int t = t0 + threadIdx.x; t < tEnd; t += kBlock) {
      float s = 0.f;
      for (int d = 0; d < a.D; ++d) s += q[d] * keys[long(t) * a.D + d];
      scores[t] = s * a.scale;
    }
  }
}
CKL_ENTRY(attention_scores, ScoresArgs, attention_scores_body)

// ------------------------------------------------------------------ softmax
// probs[b,h,t] = exp(s[t] - max) / sum_t' exp(s[t'] - max) over t <= p (workloads.py:114-128).
// One wave per (b, h) row.
struct CKL_ALIGN SoftmaxArgs { const float *scores; const int *position; float *probs; int B, A, T; };
__device__ void softmax_body(const SoftmaxArgs &a, int block) {
  int lane = threadIdx.x & 63;
  long row = long(block) * (kBlock / 64) + (threadIdx.x >> 6);
  if (row >= long(a.B) * a.A) return;
  int p = load_position(a.position);
  int end = min(p + 1, a.T);
  if (p < 0) return;
  const float *s = a.scores + row * a.T;
  float *out = a.probs + row * a.T;
  float m = -__builtin_inff();
  for (int t = lane; t < end; t += 64) m = fmaxf(m, s[t]);
  m = wave_max(m);
  float total = 0.f;
  for (int t = lane; t < end; t += 64) total += expf(s[t] - m);
  total = wave_sum(total);
  for (int t = lane; t < end; t += 64) out[t] = expf(s[t] - m) / total;
}
CKL_ENTRY(softmax, SoftmaxArgs, softmax_body)

// ------------------------------------------------------------------ attention_values
// dst[b, h*D+d] = sum_{t<=p} probs[b,h,t] * vc[layer,b,h,t,d]   (workloads.py:131-142).
// One block per (b, h): lane groups of D/4 lanes own a float4 column slice; 256/(D/4) row
// groups stride over t; partial float4 sums are combined through LDS in a fixed order.
struct CKL_ALIGN ValuesArgs { const float *probs; const float *vc; const int *position; float *dst; int L, B, A, T, D, layer; };
__device__ void attention_values_body(const ValuesArgs &a, int block) {
  __shared__ float4 partial[kBlock];
  long bh = block;
  if (bh >= long(a.B) * a.A) return;
  int p = load_position(a.position);
  int end = min(p + 1, a.T);
  const float *probs = a.probs + bh * a.T;
  const float *values = a.vc + (long(a.layer) * a.B * a.A + bh) * long(a.T) * a.D;
  float *dst = a.dst + bh * a.D;
  if ((a.D & 3) == 0 && a.D <= 4 * kBlock && (kBlock % (a.D / 4)) == 0) {
    int width = a.D / 4, groups = kBlock / width;
    int g = threadIdx.x / width, part = threadIdx.x % width;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int t = g; t < end && p >= 0; t += groups) {
      float pr = probs[t];
      float4 v = reinterpret_cast<const float4 *>(values + long(t) * a.D)[part];
      acc.x += pr * v.x; acc.y += pr * v.y; acc.z += pr * v.z; acc.w += pr * v.w;
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
    for (int d = threadIdx.x; d < a.D; d += kBlock) {
      float acc = 0.f;
      for (int t = 0; t < end && p >= 0; ++t) acc += probs[t] * values[long(t) * a.D + d];
      dst[d] = acc;
    }
  }
}
CKL_ENTRY(attention_values, ValuesArgs, attention_values_body)

// ------------------------------------------------------------------ pointwise
// add: dst = x + y; multiply: dst = x * y; silu: dst = v / (1 + exp(-v)) (workloads.py:145-167).
struct CKL_ALIGN BinaryArgs { const float *x; const float *y; float *dst; int n; };
struct CKL_ALIGN UnaryArgs { const float *src; float *dst; int n; };

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

// ------------------------------------------------------------------ greedy
// tokens[b] = history[p, b] = first index of the maximum logit (strict '>' scan,
// workloads.py:170-183). One block per row; NaN logits never win unless at index 0.
struct CKL_ALIGN GreedyArgs { const float *logits; int *tokens; int *history; const int *position; int B, V, T; };
__device__ void greedy_body(const GreedyArgs &a, int block) {
  __shared__ float bestValue[kBlock / 64];
  __shared__ int bestIndex[kBlock / 64];
  int b = block;
  if (b >= a.B) return;
  const float *logits = a.logits + long(b) * a.V;
  float v = -__builtin_inff();
  int idx = 0x7fffffff;
  for (int k = threadIdx.x; k < a.V; k += kBlock) {
    float x = logits[k];
    if (x > v || (x == v && k < idx)) { v = x; idx = k; }
  }
  wave_argmax(v, idx);
  int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) { bestValue[wave] = v; bestIndex[wave] = idx; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kBlock / 64; ++w) argmax_combine(v, idx, bestValue[w], bestIndex[w]);
    float first = logits[0];
    int winner = first != first ? 0 : idx;   // a NaN first logit is never displaced
    int p = load_position(a.position);
    a.tokens[b] = winner;
    if (p >= 0 && p < a.T) a.history[long(p) * a.B + b] = winner;
  }
}
CKL_ENTRY(greedy, GreedyArgs, greedy_body)

// ------------------------------------------------------------------ advance
// position[0] += 1   (workloads.py:186-188)
struct CKL_ALIGN AdvanceArgs { int *position; };
__device__ void advance_body(const AdvanceArgs &a, int block) {
  if (block == 0 && threadIdx.x == 0) a.position[0] = a.position[0] + 1;
}
CKL_ENTRY(advance, AdvanceArgs, advance_body)

// ------------------------------------------------------------------ vector update
// dst[i] = src[i] + bias for i < N   (examples/vector_pipeline.py:11-16)
struct CKL_ALIGN UpdateArgs { const float *src; float *dst; float bias; int n; };
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
