// Argument blocks of the gfx950 kernel library (library.hip), shared with the HIP executor.
//
// Every library kernel takes ONE of these structs by value. Its layout is the CKL kernel's
// arguments in order (buffers as pointers, scalars by value) followed by the int32 shape
// constants chosen by python/ckl/library.py and, for some families, the workspace pointer the
// executor appends (ckl_workspace). The executor packs arguments with natural alignment and pads
// the block to 8 bytes, which is the layout of these aligned(8) structs.
//
// Chain entry points (several dependent dispatches executed as one launch in the inferred graph)
// take the member blocks back to back: struct { First first; Second second; ... }. The executor
// (csrc/runtime/chains.cpp) reads the members' packed blocks through these structs to decide
// whether a chain may run fused, and fills the chain block from them, clearing the pointers of
// hand-off buffers that only the chain reads (the kernels then do not write them).
#pragma once

#include <stdint.h>

#define CKL_ALIGN __attribute__((aligned(8)))

namespace ckl::kernels {

constexpr int kMaxGroup = 4;

// Sibling-group entry points: up to kMaxGroup independent dispatches of one family in one grid;
// member m owns logical blocks [start[m], start[m+1]).
template <typename Args> struct CKL_ALIGN Group {
  Args m[kMaxGroup];
  int start[kMaxGroup + 1];
  int count;
};

// dst[b, c] = table[tokens[b], c]   (workloads.py:33-39)
struct CKL_ALIGN EmbeddingArgs { const int *tokens; const float *table; float *dst; int B, C, V; };
// inv[b] = rsqrt(sum_c x[b,c]^2 / C + eps)   (workloads.py:42-49)
struct CKL_ALIGN RmsStatsArgs { const float *x; float *inv; float eps; int B, C; };
// dst[b, c] = x[b, c] * inv[b] * gain[layer, c]   (workloads.py:52-58)
struct CKL_ALIGN RmsApplyArgs { const float *x; const float *inv; const float *gain; float *dst; int B, C, layer; };
// dst[b, o] = sum_i x[b, i] * w[layer, i, o]   (workloads.py:61-69)
// With kSplit > 1 the reduction is split over workgroups that leave partial planes in
// `partials`; `deferred` = 0: the last workgroup of a tile adds them into dst; 1 (set by the
// executor, see PartialSource): dst is not written and the consumer adds the planes.
struct CKL_ALIGN LinearArgs {
  const float *x; const float *w; float *dst; int B, I, O, layer;
  int tilesN, kSplit, kChunk, deferred;
  unsigned char *workspace;
  float *partials;
};

// Workspace of the linear family, two ranges of the plan's workspace heap. `workspace` (state,
// reads zero at every launch, never shared): kLinearZeroPage bytes that stay zero (padding loads
// read them), then the split completion counters (uint32 per output tile, padded to 256 B; reset
// by the last workgroup of each tile). `partials` (null when kSplit = 1): the partial planes
// float[kSplit][rows][O], rows = B for the vector path (ckl_linear_rowvec) and 32 * ceil(B / 32)
// for the MFMA paths, live from the launch until the readers of dst have run.
constexpr int kLinearZeroPage = 256;
// The MFMA linear's epilogue hands the accumulators of EM members through LDS in one pass:
// 16 KB per member and weight column of a lane (4 waves x 16 registers x 64 lanes x 4 bytes), at
// most kLinearEpilogueBytes; a shared-operand launch of more members takes them EM at a time.
constexpr int kLinearEpilogueBytes = 128 * 1024;
constexpr int linearEpilogueMembers(int M, int J) {
  return M * J * 16384 <= kLinearEpilogueBytes ? M : (kLinearEpilogueBytes / (J * 16384) > 0 ? kLinearEpilogueBytes / (J * 16384) : 1);
}
constexpr uint64_t linearCounterBytes(uint64_t counters) { return (counters * 4 + 255) & ~uint64_t(255); }
constexpr uint64_t linearPlaneRows(int B, bool vector) { return vector ? uint64_t(B) : uint64_t((B + 31) / 32) * 32; }

// A consumer operand that is the sum of a split linear's partial planes (the linear's combine
// deferred to its consumer): value[i] = sum over g < parts of partials[g * planeStride + i], added
// in g order starting from 0 as the linear's own combine does. parts == 0: read the operand's
// own pointer.
struct CKL_ALIGN PartialSource { const float *partials; int64_t planeStride; int parts, pad; };
// adjacent-pair rotation at the current position   (workloads.py:72-85)
struct CKL_ALIGN RopeArgs { const float *src; const float *table; const int *position; float *dst; int B, A, R, T; };
// kc/vc[layer, b, h, p, :] = k/v[b, h*D : h*D+D]   (workloads.py:88-97)
struct CKL_ALIGN AppendArgs { const float *k; const float *v; float *kc; float *vc; const int *position; int L, B, A, T, D, layer; };
// scores[b, h, t] = q . kc[layer, b, h, t] * scale   (workloads.py:100-111)
struct CKL_ALIGN ScoresArgs { const float *q; const float *kc; const int *position; float *scores; float scale; int L, B, A, T, D, layer; };
// probs[b, h, :] = softmax(scores[b, h, :p+1])   (workloads.py:114-128)
struct CKL_ALIGN SoftmaxArgs { const float *scores; const int *position; float *probs; int B, A, T, rowThreads; };
// dst[b, h*D+d] = sum_t probs[b, h, t] * vc[layer, b, h, t, d]   (workloads.py:131-142)
struct CKL_ALIGN ValuesArgs { const float *probs; const float *vc; const int *position; float *dst; int L, B, A, T, D, layer; };
// add / multiply / silu over n elements   (workloads.py:145-167)
struct CKL_ALIGN BinaryArgs { const float *x; const float *y; float *dst; int n; };
struct CKL_ALIGN UnaryArgs { const float *src; float *dst; int n; };
// tokens[b] = history[p, b] = argmax logits[b, :]   (workloads.py:170-183)
struct CKL_ALIGN GreedyArgs {
  const float *logits; int *tokens; int *history; const int *position; int B, V, T, chunks;
  unsigned char *workspace;
};
// position[0] += 1   (workloads.py:186-188)
struct CKL_ALIGN AdvanceArgs { int *position; };
// dst[i] = src[i] + bias   (examples/vector_pipeline.py:11-16)
struct CKL_ALIGN UpdateArgs { const float *src; float *dst; float bias; int n; };

// Chains (member blocks back to back, in dispatch order).
struct CKL_ALIGN RmsChainArgs { RmsStatsArgs stats; RmsApplyArgs apply; };
struct CKL_ALIGN AddRmsChainArgs { BinaryArgs add; RmsStatsArgs stats; RmsApplyArgs apply; PartialSource x, y; };
struct CKL_ALIGN EmbeddingRmsChainArgs { EmbeddingArgs embedding; RmsStatsArgs stats; RmsApplyArgs apply; };
struct CKL_ALIGN SiluMultiplyChainArgs { UnaryArgs silu; BinaryArgs multiply; PartialSource src, y; };
struct CKL_ALIGN SoftmaxValuesChainArgs { SoftmaxArgs softmax; ValuesArgs values; };
struct CKL_ALIGN AttentionChainArgs { ScoresArgs scores; SoftmaxArgs softmax; ValuesArgs values; };
struct CKL_ALIGN RopeAppendChainArgs { RopeArgs q; RopeArgs k; AppendArgs append; PartialSource qsrc, ksrc, v; };
struct CKL_ALIGN GreedyAdvanceChainArgs { GreedyArgs greedy; AdvanceArgs advance; };
// Row-parallel linear (one tile, one slice: a workgroup owns a whole output row) -> add ->
// rms_stats -> rms_apply; linearIsY: the linear's output is add's y operand.
struct CKL_ALIGN LinearAddRmsChainArgs {
  LinearArgs linear; BinaryArgs add; RmsStatsArgs stats; RmsApplyArgs apply; int linearIsY, pad;
};
// Two row-parallel linears of one x (gate, up; one slice) -> silu(gate) -> multiply by up.
struct CKL_ALIGN LinearSiluChainArgs { LinearArgs gate; LinearArgs up; UnaryArgs silu; BinaryArgs multiply; };
// The two row chains above in one launch for single-wave row-parallel linears (C <= 64): every
// gate/up workgroup recomputes its row's linear -> add -> rms, the tile-0 workgroup writes them.
struct CKL_ALIGN LinearAddRmsSiluChainArgs { LinearAddRmsChainArgs front; LinearSiluChainArgs back; };
// embedding -> rms_stats -> rms_apply, then `count` (1 to 3) single-wave row-parallel linears of
// the normalized rows (layer 0's q, k, v): member m owns blocks [start[m], start[m+1]).
struct CKL_ALIGN EmbeddingRmsLinearsChainArgs { EmbeddingRmsChainArgs front; LinearArgs back[3]; int count, start[4], pad; };
// A single-wave row-parallel linear whose output row feeds greedy -> advance (the LM head): one
// workgroup per row, one wave per 64-column tile.
struct CKL_ALIGN LinearGreedyAdvanceChainArgs { LinearArgs linear; GreedyAdvanceChainArgs pick; };
// rope(q), rope(k) -> append_kv -> attention_scores -> softmax -> attention_values per (b, h).
struct CKL_ALIGN RopeAttentionChainArgs {
  RopeArgs q; RopeArgs k; AppendArgs append; ScoresArgs scores; SoftmaxArgs softmax; ValuesArgs values;
  PartialSource qsrc, ksrc, v;
};

// Entry points named <entry>_nt read their streamed operand (weights, the cache) with
// nontemporal loads; the executor selects them when that operand is at least this large.
constexpr int64_t kStreamBytes = int64_t(8) << 20;

// Largest row (in floats) an attention chain keeps in LDS.
constexpr int kChainSoftmaxRow = 8192;

} // namespace ckl::kernels
