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

#define CKL_ENTRY(name, Args, body)                                                                  \
  extern "C" __global__ __launch_bounds__(kBlock) void ckl_##name(const Args a) { body(a, blockIdx.x); } \
  extern "C" __global__ __launch_bounds__(kBlock) void ckl_##name##_group(const Group<Args> g) {      \
    int b = blockIdx.x, m = 0;                                                                        \
    while (m + 1 < g.count && b >= g.start[m + 1]) ++m;                                               \
    body(g.m[m], b - g.start[m]);                                                                     \
  }

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
// 64 output columns per block (one per lane); the 4 waves split the reduction range; x is
// staged through LDS in chunks and broadcast; the 4 partial sums are combined through LDS in a
// fixed order. Rows are processed in tiles of kRows.
struct CKL_ALIGN LinearArgs { const float *x; const float *w; float *dst; int B, I, O, layer; };
constexpr int kRows = 8;
constexpr int kChunk = 128;
__device__ void linear_body(const LinearArgs &a, int block) {
  __shared__ float xs[kRows][kChunk];
  __shared__ float partial[4][kRows][64];
  int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int o = block * 64 + lane;
  const float *w = a.w + long(a.layer) * a.I * a.O;
  for (int r0 = 0; r0 < a.B; r0 += kRows) {
    float acc[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r) acc[r] = 0.f;
    for (int k0 = 0; k0 < a.I; k0 += kChunk) {
      __syncthreads();
      for (int e = threadIdx.x; e < kRows * kChunk; e += kBlock) {
        int r = e / kChunk, k = e % kChunk;
        xs[r][k] = (r0 + r < a.B && k0 + k < a.I) ? a.x[long(r0 + r) * a.I + k0 + k] : 0.f;
      }
      __syncthreads();
      int kEnd = min(kChunk, a.I - k0);
      if (o < a.O) {
        for (int k = wave; k < kEnd; k += 4) {
          float wv = w[long(k0 + k) * a.O + o];
#pragma unroll
          for (int r = 0; r < kRows; ++r) acc[r] += xs[r][k] * wv;
        }
      }
    }
#pragma unroll
    for (int r = 0; r < kRows; ++r) partial[wave][r][lane] = acc[r];
    __syncthreads();
    for (int e = threadIdx.x; e < kRows * 64; e += kBlock) {
      int r = e / 64, c = e % 64;
      int oo = block * 64 + c;
      if (r0 + r < a.B && oo < a.O)
        a.dst[long(r0 + r) * a.O + oo] = ((partial[0][r][c] + partial[1][r][c]) + partial[2][r][c]) + partial[3][r][c];
    }
    __syncthreads();
  }
}
CKL_ENTRY(linear, LinearArgs, linear_body)

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
