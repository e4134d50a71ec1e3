// Chains: dependent library dispatches executed as one launch in the inferred graph.
//
// On MI355X every dependent kernel launch in a graph costs ~2.5 us of dispatch latency, which is
// most of the time of the decode step's row-local kernels. The kernel library therefore has chain
// entry points (csrc/kernels/library.hip) that run several dependent dispatches row by row in one
// grid: rms_stats -> rms_apply, add -> rms_stats -> rms_apply, embedding -> rms_stats ->
// rms_apply, silu -> multiply, rope(q), rope(k) -> append_kv -> attention_scores -> softmax ->
// attention_values (or the rope part alone, attention_scores -> softmax -> attention_values, or
// softmax -> attention_values), greedy -> advance, and for row-parallel linears whose workgroups
// hold whole rows, linear -> add -> rms_stats -> rms_apply and linear, linear -> silu -> multiply
// (both as one launch for single-wave linears). The plan itself (nodes, edges,
// argument blocks) is unchanged; only the inferred lowering contracts a chain into one unit.
//
// A chain is taken only when
//   * each member depends directly on the previous one (the two ropes of the rope chain are
//     independent of each other) and the members' entry points and the chain entry point come
//     from one code object;
//   * the members' argument blocks agree (the buffer one member writes is the one the next
//     reads, same shapes), read through the argument structs in csrc/kernels/args.h;
//   * every buffer range a member writes is disjoint from every other range of the chain, or
//     identical to it and accessed row by row in both (the chain runs member k of row r before
//     member k-1 of row r' is done, which is only equivalent for such ranges);
//   * contracting it (with the chains taken before) leaves the unit graph acyclic.
// A hand-off buffer that only the chain reads (rms_stats's inv, softmax's probs, silu's output)
// is kept in registers or LDS and not written when it is a temporary no other dispatch takes as
// an argument: its range then cannot conflict with storage the planner reused for it.
// Chains are found on one iteration of the plan and repeated for every iteration.
#include "runtime.h"

#include "../kernels/args.h"

#include <algorithm>
#include <cstddef>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <stdexcept>

namespace ckl::rt {
namespace {

using namespace ckl::kernels;

struct Range {
  uint64_t begin = 0, end = 0;
  bool written = false;
  bool rowed = false;      // row r is touched only by the worker of row r
  uint64_t rowBytes = 0;
};

Range rows(const void *p, uint64_t count, uint64_t rowBytes, bool written) {
  uint64_t a = reinterpret_cast<uint64_t>(p);
  return {a, a + count * rowBytes, written, true, rowBytes};
}

Range whole(const void *p, uint64_t bytes) {
  uint64_t a = reinterpret_cast<uint64_t>(p);
  return {a, a + bytes, false, false, 0};
}

bool tracing();

bool hazardFree(const std::vector<Range> &ranges) {
  for (size_t i = 0; i < ranges.size(); ++i)
    for (size_t j = i + 1; j < ranges.size(); ++j) {
      const Range &a = ranges[i], &b = ranges[j];
      if (!a.written && !b.written) continue;
      if (a.end <= b.begin || b.end <= a.begin) continue;
      bool identical = a.begin == b.begin && a.end == b.end && a.rowed && b.rowed && a.rowBytes == b.rowBytes;
      if (!identical) {
        if (tracing())
          std::fprintf(stderr, "[ckl chains] ranges %zu [%#llx, %#llx) and %zu [%#llx, %#llx) overlap\n", i,
                       (unsigned long long)a.begin, (unsigned long long)a.end, j, (unsigned long long)b.begin,
                       (unsigned long long)b.end);
        return false;
      }
    }
  return true;
}

// For launches in which several workgroups touch one row: every written range is disjoint from
// every other written range and from every range in `others` (no identical-rows exception).
bool writesDisjoint(const std::vector<Range> &written, const std::vector<Range> &others) {
  auto apart = [](const Range &a, const Range &b) { return a.end <= b.begin || b.end <= a.begin; };
  for (size_t i = 0; i < written.size(); ++i) {
    for (const Range &r : others)
      if (!apart(written[i], r)) return false;
    for (size_t j = i + 1; j < written.size(); ++j)
      if (!apart(written[i], written[j])) return false;
  }
  return true;
}

template <typename T> T block(const Launch &launch) {
  // Packed blocks are padded to 8 bytes, as are the aligned(8) structs.
  if (launch.arguments.size() != sizeof(T))
    throw std::logic_error("argument block of " + launch.name + " does not match the kernel library's layout");
  T value;
  std::memcpy(&value, launch.arguments.data(), sizeof(T));
  return value;
}

bool singleGrid(const Launch &l) { return l.grid[1] == 1 && l.grid[2] == 1 && l.block[1] == 1 && l.block[2] == 1; }

constexpr const char *kOverlap = "buffers overlap in a way row-by-row execution would change";

unsigned cdiv(uint64_t a, uint64_t b) { return unsigned((a + b - 1) / b); }

// Geometry of the rms chains: one 256-thread workgroup per row (rms_stats's geometry).
void rowGeometry(Launch &out, int rowsCount) {
  out.grid[0] = unsigned(rowsCount);
  out.block[0] = 256;
  out.shared = 0;
}

template <typename T> void setArguments(Launch &out, const T &chain) {
  out.arguments.resize(sizeof(T));
  std::memcpy(out.arguments.data(), &chain, sizeof(T));
}

// A buffer that only the chain reads: a temporary (a plan resource placed in a heap) that no
// dispatch outside the chain (in one iteration of the plan) takes as an argument. The chain keeps
// such a hand-off in registers or LDS and does not write it (its pointer is cleared in the block).
using Internal = std::function<bool(size_t member, const void *)>;
using Members = std::vector<const Launch *>;

const char *rmsTail(RmsStatsArgs &s, const RmsApplyArgs &p, size_t member, const Internal &internal,
                    std::vector<Range> &ranges) {
  if (s.x != p.x || s.inv != p.inv || s.B != p.B || s.C != p.C || s.B <= 0 || s.C <= 0 || p.layer < 0)
    return "rms_stats and rms_apply disagree on x, inv or shape";
  uint64_t row = 4ull * uint64_t(s.C);
  if (internal(member, s.inv)) s.inv = nullptr;
  ranges.push_back(rows(s.x, uint64_t(s.B), row, false));
  if (s.inv) ranges.push_back(rows(s.inv, uint64_t(s.B), 4, true));
  ranges.push_back(whole(p.gain + int64_t(p.layer) * s.C, row));
  ranges.push_back(rows(p.dst, uint64_t(s.B), row, true));
  return nullptr;
}

const char *rmsChain(const Members &m, const Internal &internal, Launch &out) {
  RmsChainArgs c{block<RmsStatsArgs>(*m[0]), block<RmsApplyArgs>(*m[1])};
  std::vector<Range> ranges;
  if (const char *why = rmsTail(c.stats, c.apply, 0, internal, ranges)) return why;
  if (!hazardFree(ranges)) return kOverlap;
  rowGeometry(out, c.stats.B);
  setArguments(out, c);
  return nullptr;
}

const char *addRmsChain(const Members &m, const Internal &internal, Launch &out) {
  AddRmsChainArgs c{block<BinaryArgs>(*m[0]), block<RmsStatsArgs>(*m[1]), block<RmsApplyArgs>(*m[2])};
  std::vector<Range> ranges;
  if (const char *why = rmsTail(c.stats, c.apply, 1, internal, ranges)) return why;
  if (c.add.dst != c.stats.x || int64_t(c.add.n) != int64_t(c.stats.B) * c.stats.C)
    return "add does not produce rms_stats's rows";
  uint64_t row = 4ull * uint64_t(c.stats.C), count = uint64_t(c.stats.B);
  ranges.push_back(rows(c.add.x, count, row, false));
  ranges.push_back(rows(c.add.y, count, row, false));
  ranges.push_back(rows(c.add.dst, count, row, true));
  if (!hazardFree(ranges)) return kOverlap;
  rowGeometry(out, c.stats.B);
  setArguments(out, c);
  return nullptr;
}

const char *embeddingRmsChain(const Members &m, const Internal &internal, Launch &out) {
  EmbeddingRmsChainArgs c{block<EmbeddingArgs>(*m[0]), block<RmsStatsArgs>(*m[1]), block<RmsApplyArgs>(*m[2])};
  const EmbeddingArgs &e = c.embedding;
  std::vector<Range> ranges;
  if (const char *why = rmsTail(c.stats, c.apply, 1, internal, ranges)) return why;
  if (e.dst != c.stats.x || e.B != c.stats.B || e.C != c.stats.C || e.V <= 0)
    return "embedding does not produce rms_stats's rows";
  uint64_t row = 4ull * uint64_t(e.C), count = uint64_t(e.B);
  ranges.push_back(rows(e.tokens, count, 4, false));
  ranges.push_back(whole(e.table, uint64_t(e.V) * row));
  ranges.push_back(rows(e.dst, count, row, true));
  if (!hazardFree(ranges)) return kOverlap;
  rowGeometry(out, e.B);
  setArguments(out, c);
  return nullptr;
}

const char *siluMultiplyChain(const Members &m, const Internal &internal, Launch &out) {
  SiluMultiplyChainArgs c{block<UnaryArgs>(*m[0]), block<BinaryArgs>(*m[1])};
  if (c.silu.dst != c.multiply.x || c.silu.n != c.multiply.n || c.silu.n <= 0)
    return "multiply does not consume silu's output";
  // Element i is owned by one thread in both members (float4 i when n % 4 == 0).
  uint64_t n = uint64_t(c.silu.n);
  if (internal(0, c.silu.dst)) c.silu.dst = nullptr;
  std::vector<Range> ranges{rows(c.silu.src, n, 4, false), rows(c.multiply.y, n, 4, false), rows(c.multiply.dst, n, 4, true)};
  if (c.silu.dst) ranges.push_back(rows(c.silu.dst, n, 4, true));
  if (!hazardFree(ranges)) return kOverlap;
  out.grid[0] = cdiv(n % 4 == 0 ? n / 4 : n, 256);
  out.block[0] = 256;
  out.shared = 0;
  setArguments(out, c);
  return nullptr;
}

const char *softmaxValuesChain(const Members &m, const Internal &internal, Launch &out) {
  SoftmaxValuesChainArgs c{block<SoftmaxArgs>(*m[0]), block<ValuesArgs>(*m[1])};
  const SoftmaxArgs &x = c.softmax;
  const ValuesArgs &v = c.values;
  const Launch &values = *m[1];
  if (x.probs != v.probs || x.position != v.position || x.B != v.B || x.A != v.A || x.T != v.T)
    return "attention_values does not consume softmax's rows";
  if (x.B <= 0 || x.A <= 0 || x.T <= 0 || x.T > kChainSoftmaxRow || v.D <= 0 || v.layer < 0)
    return "softmax row does not fit the chain's LDS copy";
  if ((x.rowThreads != 64 && x.rowThreads != 256) || values.block[0] < unsigned(x.rowThreads))
    return "attention_values workgroup is narrower than a softmax row";
  if (values.grid[0] != unsigned(x.B) * unsigned(x.A)) return "attention_values grid is not one workgroup per row";
  uint64_t bh = uint64_t(x.B) * uint64_t(x.A), row = 4ull * uint64_t(x.T);
  uint64_t slab = bh * uint64_t(x.T) * uint64_t(v.D);
  if (internal(0, x.probs)) c.softmax.probs = nullptr;
  std::vector<Range> ranges{rows(x.scores, bh, row, false), whole(x.position, 4),
                            whole(v.vc + int64_t(v.layer) * int64_t(slab), 4 * slab),
                            rows(v.dst, bh, 4ull * uint64_t(v.D), true)};
  if (c.softmax.probs) ranges.push_back(rows(x.probs, bh, row, true));
  if (!hazardFree(ranges)) return kOverlap;
  out.grid[0] = values.grid[0];
  out.block[0] = values.block[0];
  out.shared = unsigned(row);
  setArguments(out, c);
  return nullptr;
}

Range slab(const void *p, uint64_t bytes, bool written) {
  uint64_t a = reinterpret_cast<uint64_t>(p);
  return {a, a + bytes, written, false, 0};
}

const char *attentionChain(const Members &m, const Internal &internal, Launch &out) {
  AttentionChainArgs c{block<ScoresArgs>(*m[0]), block<SoftmaxArgs>(*m[1]), block<ValuesArgs>(*m[2])};
  const ScoresArgs &sc = c.scores;
  const SoftmaxArgs &x = c.softmax;
  const ValuesArgs &v = c.values;
  const Launch &values = *m[2];
  if (sc.scores != x.scores || x.probs != v.probs || sc.position != x.position || x.position != v.position)
    return "softmax and attention_values do not consume the scores chain";
  if (sc.B != x.B || sc.A != x.A || sc.T != x.T || x.B != v.B || x.A != v.A || x.T != v.T || sc.D != v.D)
    return "attention shapes disagree";
  if (x.B <= 0 || x.A <= 0 || x.T <= 0 || x.T > kChainSoftmaxRow || v.D <= 0 || v.layer < 0 || sc.layer < 0)
    return "attention row does not fit the chain's LDS copy";
  if ((x.rowThreads != 64 && x.rowThreads != 256) || values.block[0] < unsigned(x.rowThreads))
    return "attention_values workgroup is narrower than a softmax row";
  if (values.grid[0] != unsigned(x.B) * unsigned(x.A)) return "attention_values grid is not one workgroup per row";
  uint64_t bh = uint64_t(x.B) * uint64_t(x.A), row = 4ull * uint64_t(x.T), head = 4ull * uint64_t(v.D);
  uint64_t cache = bh * uint64_t(x.T) * uint64_t(v.D);
  if (internal(0, sc.scores)) c.scores.scores = nullptr;
  if (internal(1, x.probs)) c.softmax.probs = nullptr;
  std::vector<Range> ranges{rows(sc.q, bh, head, false), whole(x.position, 4),
                            whole(sc.kc + int64_t(sc.layer) * int64_t(cache), 4 * cache),
                            whole(v.vc + int64_t(v.layer) * int64_t(cache), 4 * cache), rows(v.dst, bh, head, true)};
  if (c.scores.scores) ranges.push_back(rows(sc.scores, bh, row, true));
  if (c.softmax.probs) ranges.push_back(rows(x.probs, bh, row, true));
  if (!hazardFree(ranges)) return kOverlap;
  out.grid[0] = values.grid[0];
  out.block[0] = values.block[0];
  out.shared = unsigned(row);
  setArguments(out, c);
  return nullptr;
}

const char *ropeAppendChain(const Members &m, const Internal &internal, Launch &out) {
  RopeAppendChainArgs c{block<RopeArgs>(*m[0]), block<RopeArgs>(*m[1]), block<AppendArgs>(*m[2])};
  const RopeArgs &q = c.q, &k = c.k;
  const AppendArgs &ap = c.append;
  if (q.table != k.table || q.position != k.position || q.position != ap.position || q.B != k.B || q.A != k.A ||
      q.R != k.R || q.T != k.T)
    return "the two ropes disagree on table, position or shape";
  if (ap.k != k.dst || ap.B != q.B || ap.A != q.A || ap.D != 2 * q.R || ap.T != q.T || ap.layer < 0 || ap.L <= ap.layer)
    return "append_kv does not take the rotated k";
  if (q.B <= 0 || q.A <= 0 || q.R <= 0 || q.T <= 0) return "empty rope";
  // A worker rotates two adjacent pairs when R is even (rope_unit in the kernel library).
  const uint64_t unit = (q.R & 1) ? 1 : 2;
  uint64_t workers = uint64_t(q.B) * uint64_t(q.A) * uint64_t(q.R) / unit, bytes = 8 * unit;
  uint64_t cache = uint64_t(ap.B) * uint64_t(ap.A) * uint64_t(ap.T) * uint64_t(ap.D);
  if (internal(1, k.dst)) c.k.dst = nullptr;
  std::vector<Range> ranges{rows(q.src, workers, bytes, false), rows(q.dst, workers, bytes, true),
                            rows(k.src, workers, bytes, false), rows(ap.v, workers, bytes, false),
                            whole(q.table, 8ull * uint64_t(q.T) * uint64_t(q.R)), whole(q.position, 4),
                            slab(ap.kc + int64_t(ap.layer) * int64_t(cache), 4 * cache, true),
                            slab(ap.vc + int64_t(ap.layer) * int64_t(cache), 4 * cache, true)};
  if (c.k.dst) ranges.push_back(rows(k.dst, workers, bytes, true));
  if (!hazardFree(ranges)) return kOverlap;
  out.grid[0] = cdiv(workers, 256);
  out.block[0] = 256;
  out.shared = 0;
  setArguments(out, c);
  return nullptr;
}

// rope(q), rope(k) -> append_kv -> attention_scores -> softmax -> attention_values: the rope chain
// and the attention chain of one layer, fused per (b, h). Every buffer is touched only in the
// worker's (b, h) rows: q, k, v and the outputs in rows of D floats, the caches in slabs of T*D.
const char *ropeAttentionChain(const Members &m, const Internal &internal, Launch &out) {
  RopeAttentionChainArgs c{block<RopeArgs>(*m[0]),   block<RopeArgs>(*m[1]),    block<AppendArgs>(*m[2]),
                           block<ScoresArgs>(*m[3]), block<SoftmaxArgs>(*m[4]), block<ValuesArgs>(*m[5]),
                           {}, {}, {}};
  const RopeArgs &q = c.q, &k = c.k;
  const AppendArgs &ap = c.append;
  const ScoresArgs &sc = c.scores;
  const SoftmaxArgs &x = c.softmax;
  const ValuesArgs &v = c.values;
  const Launch &values = *m[5];
  if (q.table != k.table || q.position != k.position || q.position != ap.position || q.B != k.B || q.A != k.A ||
      q.R != k.R || q.T != k.T)
    return "the two ropes disagree on table, position or shape";
  if (ap.k != k.dst || ap.B != q.B || ap.A != q.A || ap.D != 2 * q.R || ap.T != q.T || ap.layer < 0 || ap.L <= ap.layer)
    return "append_kv does not take the rotated k";
  if (sc.q != q.dst || sc.kc != ap.kc || v.vc != ap.vc || sc.layer != ap.layer || v.layer != ap.layer)
    return "the attention does not read the rotated q and the appended caches";
  if (sc.scores != x.scores || x.probs != v.probs || sc.position != q.position || x.position != q.position ||
      v.position != q.position)
    return "softmax and attention_values do not consume the scores chain";
  if (sc.B != q.B || sc.A != q.A || sc.T != q.T || sc.D != ap.D || x.B != q.B || x.A != q.A || x.T != q.T ||
      v.B != q.B || v.A != q.A || v.T != q.T || v.D != ap.D || v.L != ap.L || sc.L != ap.L)
    return "attention shapes disagree";
  if (q.B <= 0 || q.A <= 0 || q.R <= 0 || q.T <= 0 || q.T > kChainSoftmaxRow)
    return "attention row does not fit the chain's LDS copy";
  if ((x.rowThreads != 64 && x.rowThreads != 256) || values.block[0] < unsigned(x.rowThreads))
    return "attention_values workgroup is narrower than a softmax row";
  if (values.grid[0] != unsigned(q.B) * unsigned(q.A)) return "attention_values grid is not one workgroup per row";
  uint64_t bh = uint64_t(q.B) * uint64_t(q.A), head = 4ull * uint64_t(ap.D), row = 4ull * uint64_t(q.T);
  uint64_t slab = uint64_t(q.T) * head, cache = bh * uint64_t(q.T) * uint64_t(ap.D);
  if (internal(1, k.dst)) c.k.dst = nullptr;
  if (internal(3, sc.scores)) c.scores.scores = nullptr;
  if (internal(4, x.probs)) c.softmax.probs = nullptr;
  std::vector<Range> ranges{rows(q.src, bh, head, false), rows(k.src, bh, head, false), rows(ap.v, bh, head, false),
                            rows(q.dst, bh, head, true), whole(q.table, 8ull * uint64_t(q.T) * uint64_t(q.R)),
                            whole(q.position, 4), rows(ap.kc + int64_t(ap.layer) * int64_t(cache), bh, slab, true),
                            rows(ap.vc + int64_t(ap.layer) * int64_t(cache), bh, slab, true),
                            rows(v.dst, bh, head, true)};
  if (c.k.dst) ranges.push_back(rows(k.dst, bh, head, true));
  if (c.scores.scores) ranges.push_back(rows(sc.scores, bh, row, true));
  if (c.softmax.probs) ranges.push_back(rows(x.probs, bh, row, true));
  if (!hazardFree(ranges)) return kOverlap;
  out.grid[0] = values.grid[0];
  out.block[0] = values.block[0];
  out.shared = unsigned(16 * ((uint64_t(q.T) + 3) / 4) + 2 * head);   // T floats padded to a float4, then 2 x D
  setArguments(out, c);
  return nullptr;
}

// Row-parallel linear whose workgroup holds a whole output row (one tile, one slice) -> add ->
// rms_stats -> rms_apply: one workgroup per batch row.
const char *linearAddRmsChain(const Members &m, const Internal &internal, Launch &out) {
  LinearAddRmsChainArgs c{block<LinearArgs>(*m[0]), block<BinaryArgs>(*m[1]), block<RmsStatsArgs>(*m[2]),
                          block<RmsApplyArgs>(*m[3]), 0, 0};
  const LinearArgs &l = c.linear;
  const BinaryArgs &ad = c.add;
  const Launch &lin = *m[0];
  if (l.tilesN != 1 || l.kSplit != 1 || l.O > 64 || l.B <= 0 || l.I <= 0 || !l.workspace)
    return "the linear's output rows are not one workgroup's";
  if (lin.grid[0] != unsigned(l.B) || lin.block[0] > 1024) return "the linear does not run one workgroup per row";
  if (ad.x == ad.y) return "add takes one operand twice";
  if (ad.x == l.dst) c.linearIsY = 0;
  else if (ad.y == l.dst) c.linearIsY = 1;
  else return "add does not take the linear's output";
  if (int64_t(ad.n) != int64_t(l.B) * l.O) return "add does not cover the linear's rows";
  std::vector<Range> ranges;
  if (const char *why = rmsTail(c.stats, c.apply, 2, internal, ranges)) return why;
  if (ad.dst != c.stats.x || c.stats.C != l.O || c.stats.B != l.B) return "add does not produce rms_stats's rows";
  const uint64_t count = uint64_t(l.B), row = 4ull * uint64_t(l.O);
  const uint64_t matrix = 4ull * uint64_t(l.I) * uint64_t(l.O);
  if (internal(0, l.dst)) c.linear.dst = nullptr;
  ranges.push_back(rows(l.x, count, 4ull * uint64_t(l.I), false));
  ranges.push_back(whole(l.w + int64_t(l.layer) * l.I * l.O, matrix));
  ranges.push_back(whole(l.workspace, kLinearZeroPage));
  ranges.push_back(rows(c.linearIsY ? ad.x : ad.y, count, row, false));
  ranges.push_back(rows(ad.dst, count, row, true));
  if (c.linear.dst) ranges.push_back(rows(l.dst, count, row, true));
  if (!hazardFree(ranges)) return kOverlap;
  out.grid[0] = unsigned(l.B);
  out.block[0] = lin.block[0];
  out.shared = 0;
  setArguments(out, c);
  return nullptr;
}

// Two row-parallel linears of one x (one slice each) -> silu(first) -> multiply by the second.
const char *linearSiluChain(const Members &m, const Internal &internal, Launch &out) {
  LinearSiluChainArgs c{block<LinearArgs>(*m[0]), block<LinearArgs>(*m[1]), block<UnaryArgs>(*m[2]),
                        block<BinaryArgs>(*m[3])};
  const LinearArgs &g = c.gate, &u = c.up;
  const Launch &gl = *m[0], &ul = *m[1];
  if (g.kSplit != 1 || u.kSplit != 1 || g.x != u.x || g.B != u.B || g.I != u.I || g.O != u.O || g.tilesN != u.tilesN ||
      g.B <= 0 || g.O <= 0 || !g.workspace || !u.workspace)
    return "the two linears do not share x, shape and a single slice";
  if (gl.grid[0] != ul.grid[0] || gl.block[0] != ul.block[0] || gl.grid[0] != unsigned(g.tilesN) * unsigned(g.B))
    return "the two linears do not share the row-parallel geometry";
  if (c.silu.src != g.dst || c.multiply.x != c.silu.dst || c.multiply.y != u.dst)
    return "silu and multiply do not take the two linears' outputs";
  const int64_t n = int64_t(g.B) * g.O;
  if (c.silu.n != n || c.multiply.n != n) return "silu or multiply does not cover the linears' outputs";
  const uint64_t count = uint64_t(g.B), row = 4ull * uint64_t(g.O);
  const uint64_t matrix = 4ull * uint64_t(g.I) * uint64_t(g.O);
  if (internal(0, g.dst)) c.gate.dst = nullptr;
  if (internal(1, u.dst)) c.up.dst = nullptr;
  if (internal(2, c.silu.dst)) c.silu.dst = nullptr;
  std::vector<Range> ranges{rows(g.x, count, 4ull * uint64_t(g.I), false),
                            whole(g.w + int64_t(g.layer) * g.I * g.O, matrix),
                            whole(u.w + int64_t(u.layer) * u.I * u.O, matrix),
                            whole(g.workspace, kLinearZeroPage), whole(u.workspace, kLinearZeroPage),
                            rows(c.multiply.dst, count, row, true)};
  if (c.gate.dst) ranges.push_back(rows(g.dst, count, row, true));
  if (c.up.dst) ranges.push_back(rows(u.dst, count, row, true));
  if (c.silu.dst) ranges.push_back(rows(c.silu.dst, count, row, true));
  if (!hazardFree(ranges)) return kOverlap;
  out.grid[0] = gl.grid[0];
  out.block[0] = gl.block[0];
  out.shared = 0;
  setArguments(out, c);
  return nullptr;
}

// The two row chains above as one launch when both linears are single-wave (64-thread blocks:
// C <= 64): the gate/up grid, each workgroup recomputing its row's first chain. With several
// workgroups per row, every range one of them writes must be disjoint from every other range.
const char *linearAddRmsSiluChain(const Members &m, const Internal &internal, Launch &out) {
  const Members front(m.begin(), m.begin() + 4), back(m.begin() + 4, m.end());
  const Internal backInternal = [&](size_t index, const void *p) { return internal(index + 4, p); };
  Launch f = out, k = out;
  if (const char *why = linearAddRmsChain(front, internal, f)) return why;
  if (const char *why = linearSiluChain(back, backInternal, k)) return why;
  LinearAddRmsSiluChainArgs c{block<LinearAddRmsChainArgs>(f), block<LinearSiluChainArgs>(k)};
  const LinearArgs &o = c.front.linear, &g = c.back.gate, &u = c.back.up;
  if (f.block[0] != 64 || k.block[0] != 64) return "the linears are not single-wave row-parallel";
  if (g.x != c.front.apply.dst || g.B != o.B || g.I != c.front.stats.C)
    return "the gate and up linears do not multiply the normalized rows";
  if (internal(3, c.front.apply.dst)) c.front.apply.dst = nullptr;
  const uint64_t B = uint64_t(o.B), C = uint64_t(c.front.stats.C), F = uint64_t(g.O);
  const BinaryArgs &ad = c.front.add;
  std::vector<Range> ranges{whole(o.x, 4 * B * uint64_t(o.I)),
                            whole(o.w + int64_t(o.layer) * o.I * o.O, 4ull * uint64_t(o.I) * uint64_t(o.O)),
                            whole(c.front.linearIsY ? ad.x : ad.y, 4 * B * C),
                            whole(c.front.apply.gain + int64_t(c.front.apply.layer) * int64_t(C), 4 * C),
                            whole(g.w + int64_t(g.layer) * g.I * g.O, 4ull * uint64_t(g.I) * F),
                            whole(u.w + int64_t(u.layer) * u.I * u.O, 4ull * uint64_t(u.I) * F),
                            whole(o.workspace, kLinearZeroPage), whole(g.workspace, kLinearZeroPage),
                            whole(u.workspace, kLinearZeroPage)};
  std::vector<Range> written{whole(ad.dst, 4 * B * C), whole(c.back.multiply.dst, 4 * B * F)};
  if (c.front.apply.dst) written.push_back(whole(c.front.apply.dst, 4 * B * C));
  if (c.front.stats.inv) written.push_back(whole(c.front.stats.inv, 4 * B));
  if (o.dst) written.push_back(whole(o.dst, 4 * B * C));
  for (const void *p : {static_cast<const void *>(g.dst), static_cast<const void *>(u.dst),
                        static_cast<const void *>(c.back.silu.dst)})
    if (p) written.push_back(whole(p, 4 * B * F));
  if (!writesDisjoint(written, ranges)) return kOverlap;
  out.grid[0] = k.grid[0];
  out.block[0] = 64;
  out.shared = 0;
  setArguments(out, c);
  return nullptr;
}

const char *greedyAdvanceChain(const Members &m, const Internal &, Launch &out);

// A single-wave row-parallel linear of at most 16 tiles whose output rows are greedy's logits, then
// greedy -> advance: one workgroup per row (one wave per tile); the logits are still written.
const char *linearGreedyAdvanceChain(const Members &m, const Internal &internal, Launch &out) {
  const Members tail(m.begin() + 1, m.end());
  const Internal shifted = [&](size_t index, const void *p) { return internal(index + 1, p); };
  Launch pick = out;
  if (const char *why = greedyAdvanceChain(tail, shifted, pick)) return why;
  if (m[0]->arguments.size() != sizeof(LinearArgs)) return "the linear's block does not match the library layout";
  LinearGreedyAdvanceChainArgs c{block<LinearArgs>(*m[0]), block<GreedyAdvanceChainArgs>(pick)};
  const LinearArgs &l = c.linear;
  const GreedyArgs &g = c.pick.greedy;
  if (m[0]->block[0] != 64 || l.kSplit != 1 || l.tilesN < 1 || l.tilesN > 16 || l.dst != g.logits || l.O != g.V ||
      l.B != g.B || g.chunks != 1 || !l.workspace || m[0]->grid[0] != unsigned(l.tilesN) * unsigned(l.B))
    return "the linear is not a single-wave row-parallel projection to greedy's logits";
  const uint64_t B = uint64_t(l.B), V = uint64_t(l.O);
  const std::vector<Range> read{whole(l.x, 4 * B * uint64_t(l.I)),
                                whole(l.w + int64_t(l.layer) * l.I * l.O, 4ull * uint64_t(l.I) * V),
                                whole(l.workspace, kLinearZeroPage)};
  const std::vector<Range> written{whole(l.dst, 4 * B * V), whole(g.tokens, 4 * B),
                                   whole(g.history, 4ull * uint64_t(g.T) * B), whole(g.position, 4)};
  if (!writesDisjoint(written, read)) return kOverlap;
  out.grid[0] = unsigned(l.B);
  out.block[0] = 64u * unsigned(l.tilesN);
  out.shared = 0;
  setArguments(out, c);
  return nullptr;
}

// embedding -> rms_stats -> rms_apply, then single-wave row-parallel linears of the normalized rows
// (layer 0's q, k, v) as one launch of the linears' grids (C <= 64, C % 4 == 0), every workgroup
// recomputing its row's gather and rms. Several workgroups per row: written ranges must be
// disjoint from every other range.
const char *embeddingRmsLinearsChain(const Members &m, const Internal &internal, Launch &out) {
  const Members front(m.begin(), m.begin() + 3);
  Launch f = out;
  if (const char *why = embeddingRmsChain(front, internal, f)) return why;
  EmbeddingRmsLinearsChainArgs c{};
  c.front = block<EmbeddingRmsChainArgs>(f);
  const EmbeddingArgs &e = c.front.embedding;
  if (e.C % 4 || e.C > 64) return "the embedding row does not fit one wave's float4s";
  c.count = int(m.size() - 3);
  if (c.count < 1 || c.count > 3) return "the chain takes one to three linears";
  const uint64_t B = uint64_t(e.B), C = uint64_t(e.C);
  std::vector<Range> ranges{whole(e.tokens, 4 * B), whole(e.table, uint64_t(e.V) * 4 * C),
                            whole(c.front.apply.gain + int64_t(c.front.apply.layer) * int64_t(C), 4 * C)};
  std::vector<Range> written{whole(e.dst, 4 * B * C)};
  int start = 0;
  for (int k = 0; k < c.count; ++k) {
    const Launch &ll = *m[3 + size_t(k)];
    if (ll.arguments.size() != sizeof(LinearArgs)) return "a linear's block does not match the library layout";
    LinearArgs &l = c.back[k] = block<LinearArgs>(ll);
    if (ll.block[0] != 64 || l.kSplit != 1 || l.x != c.front.apply.dst || l.B != e.B || l.I != e.C || l.O <= 0 ||
        !l.workspace || ll.grid[0] != unsigned(l.tilesN) * unsigned(l.B))
      return "a linear is not a single-wave row-parallel projection of the normalized rows";
    c.start[k] = start;
    start += int(ll.grid[0]);
    ranges.push_back(whole(l.w + int64_t(l.layer) * l.I * l.O, 4ull * uint64_t(l.I) * uint64_t(l.O)));
    ranges.push_back(whole(l.workspace, kLinearZeroPage));
    if (l.dst) written.push_back(whole(l.dst, 4 * B * uint64_t(l.O)));
  }
  for (int k = c.count; k <= 3; ++k) c.start[k] = start;
  if (internal(2, c.front.apply.dst)) c.front.apply.dst = nullptr;
  if (c.front.apply.dst) written.push_back(whole(c.front.apply.dst, 4 * B * C));
  if (c.front.stats.inv) written.push_back(whole(c.front.stats.inv, 4 * B));
  if (!writesDisjoint(written, ranges)) return kOverlap;
  out.grid[0] = unsigned(start);
  out.block[0] = 64;
  out.shared = 0;
  setArguments(out, c);
  return nullptr;
}

const char *greedyAdvanceChain(const Members &m, const Internal &, Launch &out) {
  GreedyAdvanceChainArgs c{block<GreedyArgs>(*m[0]), block<AdvanceArgs>(*m[1])};
  const GreedyArgs &g = c.greedy;
  if (c.advance.position != g.position || !g.workspace || g.B <= 0 || g.V <= 0 || g.T <= 0 || g.chunks <= 0)
    return "advance does not step greedy's position";
  // The position is read by every row and written once after all reads (the chain's row count);
  // it must not overlap the other buffers.
  std::vector<Range> ranges{whole(g.logits, 4ull * uint64_t(g.B) * uint64_t(g.V)), rows(g.tokens, uint64_t(g.B), 4, true),
                            slab(g.history, 4ull * uint64_t(g.T) * uint64_t(g.B), true), slab(g.position, 4, true)};
  if (!hazardFree(ranges)) return kOverlap;
  const Launch &greedy = *m[0];
  out.grid[0] = greedy.grid[0];
  out.block[0] = greedy.block[0];
  out.shared = greedy.shared;
  setArguments(out, c);
  return nullptr;
}

using Successors = std::vector<std::vector<size_t>>;
using Matcher = std::vector<size_t> (*)(const Plan &, size_t head, const Successors &, const std::vector<bool> &taken);

// rope(q), rope(k) -> append_kv: the ropes are independent; append_kv takes the rotated k. The
// head may be either rope; the other is the nearest untaken rope (roles: q, k, append).
std::vector<size_t> matchRopeAppend(const Plan &plan, size_t head, const Successors &successors,
                                    const std::vector<bool> &taken) {
  const size_t n = plan.nodes.size();
  auto isRope = [&](size_t k) { return !taken[k] && plan.nodes[k].launch.name == "ckl_rope" && singleGrid(plan.nodes[k].launch); };
  auto appendOf = [&](size_t rope) {
    for (size_t s : successors[rope]) {
      const Launch &l = plan.nodes[s].launch;
      if (taken[s] || l.name != "ckl_append_kv" || !singleGrid(l)) continue;
      if (block<AppendArgs>(l).k == block<RopeArgs>(plan.nodes[rope].launch).dst) return s;
    }
    return n;
  };
  auto nearest = [&](auto accept) {
    size_t best = n;
    for (size_t k = 0; k < n; ++k)
      if (k != head && isRope(k) && accept(k) &&
          (best == n || (k > head ? k - head : head - k) < (best > head ? best - head : head - best)))
        best = k;
    return best;
  };
  if (!isRope(head)) return {};
  size_t append = appendOf(head);
  if (append != n) {
    size_t q = nearest([&](size_t) { return true; });
    if (q == n) return {};
    return {q, head, append};
  }
  size_t k = nearest([&](size_t r) { return appendOf(r) != n; });
  if (k == n) return {};
  return {head, k, appendOf(k)};
}

// The rope chain's three roles, then attention_scores taking the rotated q and reading the
// appended cache, softmax of its scores and attention_values of its probabilities.
std::vector<size_t> matchRopeAttention(const Plan &plan, size_t head, const Successors &successors,
                                       const std::vector<bool> &taken) {
  std::vector<size_t> roles = matchRopeAppend(plan, head, successors, taken);
  if (roles.size() != 3) return {};
  const void *rotatedQ = block<RopeArgs>(plan.nodes[roles[0]].launch).dst;
  auto next = [&](size_t from, const char *name, auto accept) {
    size_t found = plan.nodes.size();
    for (size_t s : successors[from]) {
      const Launch &l = plan.nodes[s].launch;
      if (!taken[s] && l.name == name && singleGrid(l) && accept(l) && s < found) found = s;
    }
    return found;
  };
  const size_t n = plan.nodes.size();
  size_t scores = next(roles[2], "ckl_attention_scores", [&](const Launch &l) { return block<ScoresArgs>(l).q == rotatedQ; });
  if (scores == n) return {};
  size_t softmax = next(scores, "ckl_softmax", [](const Launch &) { return true; });
  if (softmax == n) return {};
  size_t values = next(softmax, "ckl_attention_values", [](const Launch &) { return true; });
  if (values == n) return {};
  roles.insert(roles.end(), {scores, softmax, values});
  return roles;
}

std::vector<size_t> matchLinearSilu(const Plan &plan, size_t head, const Successors &successors,
                                    const std::vector<bool> &taken);

// linear -> add -> rms_stats -> rms_apply (each the first direct successor of that name), then
// the gate/up chain of a linear that reads the normalized rows.
std::vector<size_t> matchLinearAddRmsSilu(const Plan &plan, size_t head, const Successors &successors,
                                          const std::vector<bool> &taken) {
  const size_t n = plan.nodes.size();
  std::vector<size_t> roles{head};
  for (const char *name : {"ckl_add", "ckl_rms_stats", "ckl_rms_apply"}) {
    size_t found = n;
    for (size_t s : successors[roles.back()]) {
      const Launch &l = plan.nodes[s].launch;
      if (!taken[s] && l.name == name && singleGrid(l) && s < found) found = s;
    }
    if (found == n) return {};
    roles.push_back(found);
  }
  for (size_t s : successors[roles.back()]) {
    std::vector<size_t> back = matchLinearSilu(plan, s, successors, taken);
    if (back.size() == 4) {
      roles.insert(roles.end(), back.begin(), back.end());
      return roles;
    }
  }
  return {};
}

// embedding -> rms_stats -> rms_apply (each the first direct successor of that name), then the
// three row-parallel linears that multiply the normalized rows (in plan order).
std::vector<size_t> matchEmbeddingRmsLinears(const Plan &plan, size_t head, const Successors &successors,
                                             const std::vector<bool> &taken) {
  const size_t n = plan.nodes.size();
  std::vector<size_t> roles{head};
  for (const char *name : {"ckl_rms_stats", "ckl_rms_apply"}) {
    size_t found = n;
    for (size_t s : successors[roles.back()]) {
      const Launch &l = plan.nodes[s].launch;
      if (!taken[s] && l.name == name && singleGrid(l) && s < found) found = s;
    }
    if (found == n) return {};
    roles.push_back(found);
  }
  const Launch &apply = plan.nodes[roles.back()].launch;
  if (apply.arguments.size() != sizeof(RmsApplyArgs)) return {};
  const void *y = block<RmsApplyArgs>(apply).dst;
  std::vector<size_t> linears;
  for (size_t s : successors[roles.back()]) {
    const Launch &l = plan.nodes[s].launch;
    if (!taken[s] && l.name == "ckl_linear_rowvec" && singleGrid(l) && l.arguments.size() == sizeof(LinearArgs) &&
        block<LinearArgs>(l).x == y)
      linears.push_back(s);
  }
  if (linears.size() != 3) return {};
  std::sort(linears.begin(), linears.end());
  roles.insert(roles.end(), linears.begin(), linears.end());
  return roles;
}

// Two row-parallel linears of one x whose outputs meet in silu -> multiply: the head is the
// linear silu reads (roles: gate, up, silu, multiply).
std::vector<size_t> matchLinearSilu(const Plan &plan, size_t head, const Successors &successors,
                                    const std::vector<bool> &taken) {
  const size_t n = plan.nodes.size();
  auto rowvec = [&](size_t k) {
    const Launch &l = plan.nodes[k].launch;
    return !taken[k] && l.name == "ckl_linear_rowvec" && singleGrid(l) && l.arguments.size() == sizeof(LinearArgs);
  };
  if (!rowvec(head)) return {};
  const LinearArgs gate = block<LinearArgs>(plan.nodes[head].launch);
  size_t silu = n, multiply = n;
  for (size_t s : successors[head]) {
    const Launch &l = plan.nodes[s].launch;
    if (!taken[s] && l.name == "ckl_silu" && singleGrid(l) && l.arguments.size() == sizeof(UnaryArgs) &&
        block<UnaryArgs>(l).src == gate.dst && s < silu)
      silu = s;
  }
  if (silu == n) return {};
  const void *act = block<UnaryArgs>(plan.nodes[silu].launch).dst;
  for (size_t s : successors[silu]) {
    const Launch &l = plan.nodes[s].launch;
    if (!taken[s] && l.name == "ckl_multiply" && singleGrid(l) && l.arguments.size() == sizeof(BinaryArgs) &&
        block<BinaryArgs>(l).x == act && s < multiply)
      multiply = s;
  }
  if (multiply == n) return {};
  const void *y = block<BinaryArgs>(plan.nodes[multiply].launch).y;
  for (size_t d : plan.nodes[multiply].dependencies)
    if (d != head && rowvec(d) && block<LinearArgs>(plan.nodes[d].launch).dst == y) return {head, d, silu, multiply};
  return {};
}

struct Rule {
  std::vector<std::string> members;   // entry points, in role order (dependency order for a path)
  const char *entry;                  // chain entry point
  const char *(*build)(const Members &, const Internal &, Launch &);   // null, or why not
  Matcher match = nullptr;            // null: each member is a direct successor of the previous
  std::vector<std::array<size_t, 3>> deferrable = {};   // {role, member pointer offset, source offset}
};

const std::vector<Rule> &rules() {
  static const std::vector<Rule> table = {
      {{"ckl_rope", "ckl_rope", "ckl_append_kv", "ckl_attention_scores", "ckl_softmax", "ckl_attention_values"},
       "ckl_rope__rope__append_kv__attention_scores__softmax__attention_values", ropeAttentionChain, matchRopeAttention,
       {{0, offsetof(RopeArgs, src), offsetof(RopeAttentionChainArgs, qsrc)},
        {1, offsetof(RopeArgs, src), offsetof(RopeAttentionChainArgs, ksrc)},
        {2, offsetof(AppendArgs, v), offsetof(RopeAttentionChainArgs, v)}}},
      {{"ckl_linear_rowvec", "ckl_add", "ckl_rms_stats", "ckl_rms_apply", "ckl_linear_rowvec", "ckl_linear_rowvec",
        "ckl_silu", "ckl_multiply"},
       "ckl_linear_rowvec__add__rms_stats__rms_apply__linear_rowvec__linear_rowvec__silu__multiply",
       linearAddRmsSiluChain, matchLinearAddRmsSilu},
      {{"ckl_linear_rowvec", "ckl_add", "ckl_rms_stats", "ckl_rms_apply"}, "ckl_linear_rowvec__add__rms_stats__rms_apply",
       linearAddRmsChain},
      {{"ckl_linear_rowvec", "ckl_linear_rowvec", "ckl_silu", "ckl_multiply"},
       "ckl_linear_rowvec__linear_rowvec__silu__multiply", linearSiluChain, matchLinearSilu},
      {{"ckl_add", "ckl_rms_stats", "ckl_rms_apply"}, "ckl_add__rms_stats__rms_apply", addRmsChain, nullptr,
       {{0, offsetof(BinaryArgs, x), offsetof(AddRmsChainArgs, x)}, {0, offsetof(BinaryArgs, y), offsetof(AddRmsChainArgs, y)}}},
      {{"ckl_embedding", "ckl_rms_stats", "ckl_rms_apply", "ckl_linear_rowvec", "ckl_linear_rowvec", "ckl_linear_rowvec"},
       "ckl_embedding__rms_stats__rms_apply__linear_rowvec__linear_rowvec__linear_rowvec", embeddingRmsLinearsChain,
       matchEmbeddingRmsLinears},
      {{"ckl_embedding", "ckl_rms_stats", "ckl_rms_apply"}, "ckl_embedding__rms_stats__rms_apply", embeddingRmsChain},
      {{"ckl_rms_stats", "ckl_rms_apply"}, "ckl_rms_stats__rms_apply", rmsChain},
      {{"ckl_silu", "ckl_multiply"}, "ckl_silu__multiply", siluMultiplyChain, nullptr,
       {{0, offsetof(UnaryArgs, src), offsetof(SiluMultiplyChainArgs, src)},
        {1, offsetof(BinaryArgs, y), offsetof(SiluMultiplyChainArgs, y)}}},
      {{"ckl_attention_scores", "ckl_softmax", "ckl_attention_values"}, "ckl_attention_scores__softmax__attention_values",
       attentionChain},
      {{"ckl_softmax", "ckl_attention_values"}, "ckl_softmax__attention_values", softmaxValuesChain},
      {{"ckl_linear_rowvec", "ckl_greedy", "ckl_advance"}, "ckl_linear_rowvec__greedy__advance",
       linearGreedyAdvanceChain},
      {{"ckl_greedy", "ckl_advance"}, "ckl_greedy__advance", greedyAdvanceChain},
      {{"ckl_rope", "ckl_rope", "ckl_append_kv"}, "ckl_rope__rope__append_kv", ropeAppendChain, matchRopeAppend,
       {{0, offsetof(RopeArgs, src), offsetof(RopeAppendChainArgs, qsrc)},
        {1, offsetof(RopeArgs, src), offsetof(RopeAppendChainArgs, ksrc)},
        {2, offsetof(AppendArgs, v), offsetof(RopeAppendChainArgs, v)}}},
  };
  return table;
}

// Kahn's algorithm over the units given by `unit` (node -> unit id).
bool acyclic(const Plan &plan, const std::vector<size_t> &unit, size_t units) {
  std::vector<std::vector<size_t>> succ(units);
  std::vector<size_t> indegree(units, 0);
  for (size_t k = 0; k < plan.nodes.size(); ++k)
    for (size_t d : plan.nodes[k].dependencies)
      if (unit[d] != unit[k]) { succ[unit[d]].push_back(unit[k]); ++indegree[unit[k]]; }
  std::vector<size_t> ready;
  for (size_t u = 0; u < units; ++u) if (!indegree[u]) ready.push_back(u);
  size_t seen = 0;
  while (!ready.empty()) {
    size_t u = ready.back();
    ready.pop_back();
    ++seen;
    for (size_t s : succ[u]) if (!--indegree[s]) ready.push_back(s);
  }
  return seen == units;
}

} // namespace

// CKL_CHAIN_TRACE=1 reports every chain considered and why it was not taken (stderr).
namespace {
bool tracing() {
  static const bool on = [] {
    const char *v = std::getenv("CKL_CHAIN_TRACE");
    return v && std::strcmp(v, "1") == 0;
  }();
  return on;
}

void trace(size_t head, const Rule &rule, const char *outcome) {
  if (tracing()) std::fprintf(stderr, "[ckl chains] node %zu %s: %s\n", head, rule.entry, outcome);
}

} // namespace

std::vector<Chain> findChains(const Plan &plan, const std::vector<bool> &temporary,
                              std::vector<std::vector<size_t>> *refused) {
  const size_t n = plan.nodes.size();
  std::vector<std::vector<size_t>> successors(n);
  for (size_t k = 0; k < n; ++k) for (size_t d : plan.nodes[k].dependencies) successors[d].push_back(k);
  std::vector<size_t> unit(n);
  for (size_t k = 0; k < n; ++k) unit[k] = k;
  std::vector<bool> taken(n, false);
  std::vector<Chain> chains;
  for (size_t head = 0; head < n; ++head) {
    if (taken[head]) continue;
    const Launch &first = plan.nodes[head].launch;
    for (const Rule &rule : rules()) {
      if (first.name != rule.members[0] || !first.module || !singleGrid(first)) continue;
      std::vector<size_t> roles;
      if (rule.match) {
        roles = rule.match(plan, head, successors, taken);
        bool same = roles.size() == rule.members.size();
        for (size_t k = 0; same && k < roles.size(); ++k) same = plan.nodes[roles[k]].launch.module == first.module;
        if (!same) {
          trace(head, rule, "its members are not all present");
          continue;
        }
      } else {
        roles.push_back(head);
        for (size_t k = 1; k < rule.members.size(); ++k) {
          size_t found = n;
          for (size_t s : successors[roles.back()]) {
            const Launch &l = plan.nodes[s].launch;
            if (!taken[s] && l.name == rule.members[k] && l.module == first.module && singleGrid(l) && s < found) found = s;
          }
          if (found == n) break;
          roles.push_back(found);
        }
        if (roles.size() != rule.members.size()) {
          trace(head, rule, ("no dependent " + rule.members[roles.size()] + " follows").c_str());
          continue;
        }
      }
      std::vector<size_t> members = roles;
      std::sort(members.begin(), members.end());
      hipFunction_t function = nullptr, group = nullptr;
      if (hipModuleGetFunction(&function, first.module, rule.entry) != hipSuccess) {
        (void)hipGetLastError();
        trace(head, rule, "the code object has no such entry point");
        continue;
      }
      // A chain with a streaming member runs its nontemporal-load variant when there is one.
      std::string entry = rule.entry;
      bool streaming = false;
      for (size_t m : roles) streaming |= streams(plan.nodes[m].launch);
      if (streaming) {
        hipFunction_t variant = nullptr;
        if (hipModuleGetFunction(&variant, first.module, (entry + "_nt").c_str()) == hipSuccess) {
          function = variant;
          entry += "_nt";
        } else {
          (void)hipGetLastError();
        }
      }
      std::string groupName = entry + "_group";
      if (hipModuleGetFunction(&group, first.module, groupName.c_str()) != hipSuccess) {
        (void)hipGetLastError();
        group = nullptr;
      }
      // The plan resources (logical buffers, whatever storage they share) that member `index`
      // addresses with pointer `p` (the arguments of one dispatch are live together, so they
      // never share storage); internal when each is a temporary no other dispatch takes.
      auto internal = [&](size_t index, const void *p) {
        std::vector<int64_t> ids;
        const Launch &l = plan.nodes[roles.at(index)].launch;
        for (size_t slot = 0; slot < l.slotOffsets.size() && slot < l.slotResources.size(); ++slot) {
          uint64_t word = 0;
          if (l.slotResources[slot] < 0 || l.slotOffsets[slot] + 8 > l.arguments.size()) continue;
          std::memcpy(&word, l.arguments.data() + l.slotOffsets[slot], 8);
          if (word == reinterpret_cast<uint64_t>(p)) ids.push_back(l.slotResources[slot]);
        }
        if (ids.empty()) return false;
        for (int64_t id : ids)
          if (size_t(id) >= temporary.size() || !temporary[size_t(id)]) return false;
        for (size_t k = 0; k < n; ++k) {
          if (std::find(members.begin(), members.end(), k) != members.end()) continue;
          for (int64_t id : plan.nodes[k].launch.slotResources)
            if (std::find(ids.begin(), ids.end(), id) != ids.end()) return false;
        }
        return true;
      };
      std::vector<const Launch *> launches;
      for (size_t m : roles) launches.push_back(&plan.nodes[m].launch);
      Launch fused;
      fused.name = rule.entry;
      fused.module = first.module;
      fused.function = function;
      fused.groupFunction = group;
      if (const char *why = rule.build(launches, internal, fused)) {
        trace(head, rule, why);
        if (refused && why == kOverlap) refused->push_back(members);
        continue;
      }
      std::vector<size_t> trial = unit;
      for (size_t m : members) trial[m] = head;
      // Unit ids stay node indices: count them as the node range.
      if (!acyclic(plan, trial, n)) {
        trace(head, rule, "contracting it would create a cycle");
        continue;
      }
      trace(head, rule, "taken");
      unit = std::move(trial);
      for (size_t m : members) taken[m] = true;
      chains.push_back({std::move(members), std::move(fused), roles, rule.deferrable});
      break;
    }
  }
  return chains;
}

bool streams(const Launch &l) {
  const std::string &name = l.name;
  if (name.rfind("ckl_linear_mfma", 0) == 0 || name == "ckl_linear_rowvec") {
    if (l.arguments.size() != sizeof(LinearArgs)) return false;
    const LinearArgs a = block<LinearArgs>(l);
    return int64_t(a.I) * a.O * 4 >= kStreamBytes;
  }
  if (name == "ckl_attention_scores" && l.arguments.size() == sizeof(ScoresArgs)) {
    const ScoresArgs a = block<ScoresArgs>(l);
    return int64_t(a.B) * a.A * a.T * a.D * 4 >= kStreamBytes;
  }
  if (name == "ckl_attention_values" && l.arguments.size() == sizeof(ValuesArgs)) {
    const ValuesArgs a = block<ValuesArgs>(l);
    return int64_t(a.B) * a.A * a.T * a.D * 4 >= kStreamBytes;
  }
  return false;
}

bool sharesOperands(const std::vector<const Launch *> &members) {
  if (members.size() < 2 || members[0]->name.rfind("ckl_linear_mfma", 0) != 0) return false;
  const LinearArgs a = block<LinearArgs>(*members[0]);
  for (size_t k = 1; k < members.size(); ++k) {
    if (members[k]->name != members[0]->name) return false;
    const LinearArgs b = block<LinearArgs>(*members[k]);
    if (b.x != a.x || b.B != a.B || b.I != a.I || b.O != a.O || b.layer != a.layer || b.tilesN != a.tilesN ||
        b.kSplit != a.kSplit || b.kChunk != a.kChunk)
      return false;
  }
  return true;
}

std::map<size_t, Launch> deferCombines(const Plan &plan, const std::vector<bool> &temporary, std::vector<Chain> &chains) {
  auto slotAt = [](const Launch &l, size_t offset) -> int64_t {
    for (size_t s = 0; s < l.slotOffsets.size() && s < l.slotResources.size(); ++s)
      if (l.slotOffsets[s] == offset) return int64_t(s);
    return -1;
  };
  // Deferrable chain operands by the plan resource they read: {chain, source offset, node, slot}.
  struct Operand { size_t chain, source, node; int64_t slot; };
  std::map<int64_t, std::vector<Operand>> operands;
  for (size_t c = 0; c < chains.size(); ++c)
    for (const auto &[role, pointer, source] : chains[c].deferrable) {
      size_t node = chains[c].roles.at(role);
      int64_t slot = slotAt(plan.nodes[node].launch, pointer);
      if (slot < 0) continue;
      int64_t resource = plan.nodes[node].launch.slotResources[size_t(slot)];
      if (resource >= 0) operands[resource].push_back({c, source, node, slot});
    }
  std::map<size_t, Launch> patched;
  for (size_t p = 0; p < plan.nodes.size(); ++p) {
    const Launch &l = plan.nodes[p].launch;
    if (l.name.rfind("ckl_linear_", 0) != 0) continue;
    LinearArgs a = block<LinearArgs>(l);
    int64_t dstSlot = slotAt(l, offsetof(LinearArgs, dst));
    if (a.kSplit <= 1 || a.deferred || dstSlot < 0 || !a.workspace) continue;
    int64_t resource = l.slotResources[size_t(dstSlot)];
    if (resource < 0 || size_t(resource) >= temporary.size() || !temporary[size_t(resource)]) continue;
    auto found = operands.find(resource);
    if (found == operands.end()) continue;
    // Every other argument taking the resource must be one of the deferrable operands.
    bool all = true;
    for (size_t k = 0; k < plan.nodes.size() && all; ++k) {
      const Launch &consumer = plan.nodes[k].launch;
      for (size_t s = 0; s < consumer.slotResources.size() && all; ++s) {
        if (consumer.slotResources[s] != resource || (k == p && int64_t(s) == dstSlot)) continue;
        bool listed = false;
        for (const Operand &o : found->second) listed |= o.node == k && o.slot == int64_t(s);
        all = listed;
      }
    }
    const bool vector = l.name == "ckl_linear_rowvec";
    const uint64_t stride = linearPlaneRows(a.B, vector) * uint64_t(a.O);
    if (!all || stride % 4) continue;
    if (!a.partials) continue;
    PartialSource source{a.partials, int64_t(stride), a.kSplit, 0};
    for (const Operand &o : found->second) {
      std::vector<uint8_t> &bytes = chains[o.chain].launch.arguments;
      if (o.source + sizeof source > bytes.size()) throw std::logic_error("chain block has no room for a partial source");
      std::memcpy(bytes.data() + o.source, &source, sizeof source);
    }
    Launch deferred = l;
    a.deferred = 1;
    std::memcpy(deferred.arguments.data(), &a, sizeof a);
    if (tracing()) std::fprintf(stderr, "[ckl chains] node %zu %s: combine deferred to %zu readers\n", p, l.name.c_str(),
                                found->second.size());
    patched.emplace(p, std::move(deferred));
  }
  return patched;
}

} // namespace ckl::rt
