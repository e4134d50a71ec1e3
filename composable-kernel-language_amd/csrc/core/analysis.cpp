#include "analysis.h"

#include "sha256.h"

#include <algorithm>
#include <limits>
#include <set>
#include <sstream>
#include <unordered_map>
#include <unordered_set>

namespace ckl {

// ====================================================================== regions and aliasing
// lib/Core/MemoryEffects.cpp:51-223

Attr AccessRegion::attr() const {
  switch (kind) {
  case Whole: return Attr::string("whole");
  case Unknown: return Attr::string("unknown");
  default: return Attr::dictOf({{"length", Attr::integer(length)}, {"offset", Attr::integer(offset)}});
  }
}

bool hasConflictingAccesses(unsigned lhs, unsigned rhs) {
  constexpr unsigned nonRead = Write | Allocate | Free;
  return (lhs & nonRead) || (rhs & nonRead);
}

static bool isAllocOp(const Op *op) {
  return op && (op->name == "ckl.alloc" || op->name == "memref.alloc" || op->name == "memref.alloca");
}

bool isAllocationValue(const Value *value) { return value && value->def && isAllocOp(value->def) && value->index == 0; }

static bool isViewOp(const Op *op) {
  return op && (op->name == "ckl.view" || op->name == "ckl.subview" || op->name == "memref.subview" ||
                op->name == "memref.cast" || op->name == "memref.reinterpret_cast");
}

Value *getBaseResource(Value *value) {
  std::unordered_set<const Op *> visited;
  while (value->def && isViewOp(value->def) && !value->def->operands.empty()) {
    if (!visited.insert(value->def).second) break;
    value = value->def->operands[0];
  }
  return value;
}

Alias aliasWholeBuffers(Value *lhs, Value *rhs) {
  lhs = getBaseResource(lhs);
  rhs = getBaseResource(rhs);
  if (lhs == rhs) return Alias::Must;
  if (isAllocationValue(lhs) || isAllocationValue(rhs)) return Alias::No;
  return Alias::May;
}

static std::optional<int64_t> elementBytes(const Type &t) {
  unsigned width = Type::bitWidth(t.element);
  if (!width || width % 8) return std::nullopt;
  return int64_t(width / 8);
}

std::optional<AccessRegion> staticResourceRange(const Value *value) {
  const Type &t = value->type;
  if (!t.isMemRef() || !t.hasStaticShape() || !t.identityLayout) return std::nullopt;
  auto bytes = elementBytes(t);
  if (!bytes || t.element == Type::Index) return std::nullopt;
  int64_t elements = 1;
  for (int64_t d : t.shape) {
    if (d <= 0 || elements > std::numeric_limits<int64_t>::max() / d) return std::nullopt;
    elements *= d;
  }
  if (elements > std::numeric_limits<int64_t>::max() / *bytes) return std::nullopt;
  int64_t offset = 0;
  if (const Op *op = value->def) {
    if (op->name == "ckl.subview") {
      auto parent = staticResourceRange(op->operands[0]);
      const Attr *elementOffset = op->attr("offset");
      if (!parent || !elementOffset || elementOffset->kind != Attr::Int || elementOffset->i < 0 ||
          elementOffset->i > std::numeric_limits<int64_t>::max() / *bytes)
        return std::nullopt;
      int64_t local = elementOffset->i * *bytes;
      if (local > parent->length || elements * *bytes > parent->length - local) return std::nullopt;
      offset = parent->offset + local;
    } else if (isViewOp(op)) {
      return std::nullopt;   // unmodeled views are not zero-offset aliases
    }
  }
  return AccessRegion::interval(offset, elements * *bytes);
}

static std::optional<int64_t> constantInt(const Value *v) {
  if (!v->def || v->def->name != "arith.constant") return std::nullopt;
  const Attr *a = v->def->attr("value");
  if (!a || a->kind != Attr::Int) return std::nullopt;
  return a->i;
}

static AccessRegion operationAccessRegion(const Op *op, const Value *resource) {
  const Type &t = resource->type;
  if (t.isMemRef() && t.hasStaticShape() && t.identityLayout && (Type::bitWidth(t.element) % 8 == 0) &&
      (op->name == "ckl.load_element" || op->name == "ckl.store_element")) {
    size_t begin = op->name == "ckl.load_element" ? 1 : 2;
    if (op->operands.size() != begin + t.shape.size()) return AccessRegion::whole();
    int64_t linear = 0;
    for (size_t axis = 0; axis < t.shape.size(); ++axis) {
      auto index = constantInt(op->operands[begin + axis]);
      if (!index) return AccessRegion::whole();
      int64_t i = *index, extent = t.shape[axis];
      if (i < 0 || i >= extent || linear > (std::numeric_limits<int64_t>::max() - i) / extent)
        return AccessRegion::whole();
      linear = linear * extent + i;
    }
    int64_t bytes = Type::bitWidth(t.element) / 8;
    if (bytes && linear <= std::numeric_limits<int64_t>::max() / bytes)
      return AccessRegion::interval(linear * bytes, bytes);
  }
  return AccessRegion::whole();
}

AccessRegion composeAccessRegion(const Value *resource, const AccessRegion &relative) {
  if (relative.kind == AccessRegion::Unknown) return relative;
  auto range = staticResourceRange(resource);
  if (!range) return AccessRegion::whole();
  if (relative.kind == AccessRegion::Interval) {
    if (relative.offset > range->length || relative.length > range->length - relative.offset)
      return AccessRegion::unknown();
    return AccessRegion::interval(range->offset + relative.offset, relative.length);
  }
  if (resource != getBaseResource(const_cast<Value *>(resource))) return *range;
  return relative;
}

std::optional<AccessRegion> mergeAccessRegions(const std::optional<AccessRegion> &lhs, const AccessRegion &rhs) {
  if (!lhs) return rhs;
  if (lhs->kind == AccessRegion::Unknown || rhs.kind == AccessRegion::Unknown) return AccessRegion::unknown();
  if (lhs->kind != AccessRegion::Interval || rhs.kind != AccessRegion::Interval) return AccessRegion::whole();
  int64_t start = std::min(lhs->offset, rhs.offset);
  int64_t end = std::max(lhs->offset + lhs->length, rhs.offset + rhs.length);
  return AccessRegion::interval(start, end - start);
}

bool disjointRegions(const AccessRegion &a, const AccessRegion &b) {
  return a.kind == AccessRegion::Interval && b.kind == AccessRegion::Interval &&
         (a.offset + a.length <= b.offset || b.offset + b.length <= a.offset);
}

// ====================================================================== effect summaries
// lib/Analysis/EffectAnalysis.cpp:41-343

namespace {

bool isResourceType(const Type &t) { return t.isMemRef(); }

struct Effect {
  unsigned bits;
  Value *value;   // may be null
};

// Memory-effect model of the supported operations. `modeled` is false for operations whose
// effects are unknown; `recursive` for operations whose effects are those of their regions.
void operationEffects(Op *op, std::vector<Effect> &effects, bool &modeled, bool &recursive) {
  const std::string &n = op->name;
  modeled = true;
  recursive = false;
  auto starts = [&](const char *prefix) { return n.rfind(prefix, 0) == 0; };
  if (isAllocOp(op)) { effects.push_back({Allocate, op->results.empty() ? nullptr : op->result(0)}); return; }
  if (n == "ckl.free" || n == "memref.dealloc") { effects.push_back({Free, op->operands.empty() ? nullptr : op->operands[0]}); return; }
  if (n == "ckl.load" || n == "ckl.load_element" || n == "memref.load") { effects.push_back({Read, op->operands.at(0)}); return; }
  if (n == "ckl.store" || n == "ckl.store_element" || n == "memref.store") { effects.push_back({Write, op->operands.at(1)}); return; }
  if (n == "memref.copy") {   // whole-buffer copy: reads its source, writes its target
    effects.push_back({Read, op->operands.at(0)});
    effects.push_back({Write, op->operands.at(1)});
    return;
  }
  if (n == "ckl.atomic_rmw") {
    effects.push_back({Read, op->operands.at(1)});
    effects.push_back({Write, op->operands.at(1)});
    return;
  }
  if (n == "ckl.sync") {
    for (Value *v : op->operands) { effects.push_back({Read, v}); effects.push_back({Write, v}); }
    return;
  }
  if (starts("arith.") || starts("math.") || n == "ckl.thread_id" || n == "ckl.block_id" || n == "ckl.block_dim" ||
      n == "ckl.grid_dim" || n == "ckl.global_id" || isViewOp(op) || n == "scf.yield" || n == "scf.condition")
    return;
  if (n == "scf.if" || n == "scf.for" || n == "scf.while" || n == "scf.execute_region") { modeled = false; recursive = true; return; }
  modeled = false;
}

bool implementsAccessRegion(const Op *op) {
  return op->name == "ckl.load" || op->name == "ckl.store" || op->name == "ckl.load_element" ||
         op->name == "ckl.store_element" || op->name == "ckl.atomic_rmw";
}

std::vector<Value *> dispatchArguments(const Op *op) {
  size_t count = op->operands.size();
  if (const Attr *seg = op->attr("operandSegmentSizes"); seg && !seg->dense.empty()) count = size_t(seg->dense[0]);
  return std::vector<Value *>(op->operands.begin(), op->operands.begin() + std::min(count, op->operands.size()));
}

std::vector<Value *> dispatchDependencies(const Op *op) {
  size_t count = op->operands.size();
  if (const Attr *seg = op->attr("operandSegmentSizes"); seg && !seg->dense.empty()) count = size_t(seg->dense[0]);
  if (count >= op->operands.size()) return {};
  return std::vector<Value *>(op->operands.begin() + count, op->operands.end());
}

std::string symbolOf(const Op *op, const char *key) {
  const Attr *a = op->attr(key);
  if (!a || a->kind != Attr::Symbol || !a->nested.empty()) return {};
  return a->s;
}

class SummaryAnalysis {
public:
  SummaryAnalysis(Module &module, bool strict) : module(module), strict(strict) {}

  KernelSummary summarize(Op *function) {
    if (auto found = summaries.find(function); found != summaries.end()) return found->second;
    KernelSummary summary;
    size_t argc = argumentCount(function);
    summary.effects.assign(argc, 0);
    summary.regions.assign(argc, std::nullopt);
    if (function->isDeclaration()) {
      markUnknown(summary, function);
      if (strict) throw CompileError(where(function) + "cannot summarize an external function in strict mode");
      summaries[function] = summary;
      return summary;
    }
    if (!active.insert(function).second) {
      markUnknown(summary, function);
      if (strict) throw CompileError(where(function) + "recursive effect summaries are conservative and unavailable in strict mode");
      return summary;
    }
    for (auto &block : function->regions[0]->blocks)
      for (auto &op : block->ops) analyze(op.get(), function, summary);
    active.erase(function);
    summaries[function] = summary;
    return summary;
  }

  std::map<const Op *, KernelSummary> summaries;

private:
  Module &module;
  bool strict;
  std::set<const Op *> active;

  static std::string where(const Op *op) { return sourcePosition(op); }

  static size_t argumentCount(const Op *function) {
    if (Block *entry = function->entry()) return entry->args.size();
    if (const Attr *types = function->attr("ckl.argument_types")) return types->array.size();
    return 0;
  }
  static Type argumentType(const Op *function, size_t index) {
    if (Block *entry = function->entry()) return entry->args[index]->type;
    return function->attr("ckl.argument_types")->array[index].type;
  }

  void markUnknown(KernelSummary &summary, const Op *function) const {
    summary.unknown = true;
    summary.synchronizes = true;
    if (std::find(summary.orderingScopes.begin(), summary.orderingScopes.end(), "unknown") == summary.orderingScopes.end())
      summary.orderingScopes.push_back("unknown");
    for (size_t k = 0; k < summary.effects.size(); ++k) {
      if (!isResourceType(argumentType(function, k))) continue;
      summary.effects[k] |= Read | Write;
      summary.regions[k] = AccessRegion::unknown();
    }
  }

  void handleUnknown(Op *op, Op *function, KernelSummary &summary, const std::string &reason) {
    if (strict) throw CompileError(where(op) + "'" + op->name + "': " + reason + " in strict effect mode");
    markUnknown(summary, function);
  }

  void addEffect(Value *value, unsigned bits, Op *function, KernelSummary &summary, Op *source,
                 std::optional<AccessRegion> region) {
    Value *base = getBaseResource(value);
    if (!base->def && base->owner == function->entry()) {
      summary.effects[base->index] |= bits;
      AccessRegion r = composeAccessRegion(value, region ? *region : AccessRegion::whole());
      summary.regions[base->index] = mergeAccessRegions(summary.regions[base->index], r);
      return;
    }
    if (isAllocationValue(base)) return;
    handleUnknown(source, function, summary, "cannot resolve an effect to a function resource");
  }

  void applyCallee(Op *op, const std::vector<Value *> &actuals, Op *callee, Op *function, KernelSummary &summary) {
    KernelSummary calleeSummary = summarize(callee);
    if (actuals.size() != calleeSummary.effects.size()) {
      handleUnknown(op, function, summary, "callee argument count does not match its effect summary");
      return;
    }
    summary.synchronizes |= calleeSummary.synchronizes;
    summary.unknown |= calleeSummary.unknown;
    for (const std::string &scope : calleeSummary.orderingScopes)
      if (std::find(summary.orderingScopes.begin(), summary.orderingScopes.end(), scope) == summary.orderingScopes.end())
        summary.orderingScopes.push_back(scope);
    for (size_t k = 0; k < actuals.size(); ++k)
      if (calleeSummary.effects[k])
        addEffect(actuals[k], calleeSummary.effects[k], function, summary, op, calleeSummary.regions[k]);
  }

  void addScope(KernelSummary &summary, const std::string &scope) {
    if (std::find(summary.orderingScopes.begin(), summary.orderingScopes.end(), scope) == summary.orderingScopes.end())
      summary.orderingScopes.push_back(scope);
  }

  void analyze(Op *op, Op *function, KernelSummary &summary) {
    if (op->name == "func.return") return;
    if (op->name == "func.call") {
      Op *callee = module.lookup(symbolOf(op, "callee"));
      if (!callee || callee->name != "func.func") { handleUnknown(op, function, summary, "cannot resolve callee"); return; }
      applyCallee(op, op->operands, callee, function, summary);
      return;
    }
    if (op->name == "ckl.dispatch") {
      Op *callee = module.lookup(symbolOf(op, "kernel"));
      if (!callee || callee->name != "func.func") { handleUnknown(op, function, summary, "cannot resolve dispatched kernel"); return; }
      summary.synchronizes |= !dispatchDependencies(op).empty();
      applyCallee(op, dispatchArguments(op), callee, function, summary);
      return;
    }
    if (op->name == "ckl.atomic_rmw") {
      const Attr *ordering = op->attr("ordering");
      const Attr *scope = op->attr("scope");
      addScope(summary, (ordering ? ordering->s : std::string()) + "@" + (scope ? scope->s : std::string()));
    }
    if (op->name == "ckl.sync") {
      summary.synchronizes = true;
      const Attr *scope = op->attr("scope");
      addScope(summary, "sync@" + (scope ? scope->s : std::string()));
    }
    std::vector<Effect> effects;
    bool modeled, recursive;
    operationEffects(op, effects, modeled, recursive);
    if (modeled) {
      for (const Effect &effect : effects) {
        if (!effect.bits) continue;
        if (!effect.value) {
          if (op->name == "ckl.sync") continue;
          handleUnknown(op, function, summary, "memory effect has no addressable resource");
          continue;
        }
        AccessRegion region = implementsAccessRegion(op) ? operationAccessRegion(op, effect.value) : AccessRegion::whole();
        addEffect(effect.value, effect.bits, function, summary, op, region);
      }
    } else if (!recursive) {
      handleUnknown(op, function, summary, "operation has no complete memory-effect model");
    }
    for (auto &region : op->regions)
      for (auto &block : region->blocks)
        for (auto &nested : block->ops) analyze(nested.get(), function, summary);
  }
};

Attr effectList(unsigned bits) {
  std::vector<Attr> out;
  if (bits & Read) out.push_back(Attr::string("read"));
  if (bits & Write) out.push_back(Attr::string("write"));
  if (bits & Allocate) out.push_back(Attr::string("allocate"));
  if (bits & Free) out.push_back(Attr::string("free"));
  return Attr::arrayOf(out);
}

Attr materializeSummary(const Op *function, const KernelSummary &summary) {
  std::vector<Attr> accesses;
  for (size_t k = 0; k < summary.effects.size(); ++k) {
    if (!summary.effects[k]) continue;
    accesses.push_back(Attr::dictOf({{"arg", Attr::integer(int64_t(k))},
                                     {"effects", effectList(summary.effects[k])},
                                     {"region", summary.regions[k] ? summary.regions[k]->attr() : Attr::string("whole")}}));
  }
  std::vector<Attr> mayAlias;
  if (Block *entry = function->entry()) {
    for (size_t a = 0; a < entry->args.size(); ++a) {
      if (!isResourceType(entry->args[a]->type)) continue;
      for (size_t b = a + 1; b < entry->args.size(); ++b) {
        if (!isResourceType(entry->args[b]->type)) continue;
        if (aliasWholeBuffers(entry->args[a].get(), entry->args[b].get()) == Alias::May)
          mayAlias.push_back(Attr::arrayOf({Attr::integer(int64_t(a)), Attr::integer(int64_t(b))}));
      }
    }
  }
  std::vector<Attr> scopes;
  for (const std::string &s : summary.orderingScopes) scopes.push_back(Attr::string(s));
  return Attr::dictOf({{"accesses", Attr::arrayOf(accesses)},
                       {"may_alias", Attr::arrayOf(mayAlias)},
                       {"ordering_scopes", Attr::arrayOf(scopes)},
                       {"synchronizes", Attr::boolean(summary.synchronizes)},
                       {"unknown", Attr::boolean(summary.unknown)}});
}

} // namespace

std::map<const Op *, KernelSummary> deriveEffectSummaries(Module &module, bool strict) {
  SummaryAnalysis analysis(module, strict);
  std::map<const Op *, KernelSummary> result;
  for (Op *function : module.functions()) {
    KernelSummary summary = analysis.summarize(function);
    function->attrs["ckl.effect_summary"] = materializeSummary(function, summary);
    result[function] = summary;
  }
  return result;
}

// ====================================================================== graph
// lib/Analysis/GraphAnalysis.cpp:64-600

namespace {

std::string locationText(const Op *op) { return "loc(" + (op->loc.empty() ? std::string("unknown") : op->loc) + ")"; }

class Namer {
public:
  explicit Namer(const Op *function) : entry(function->entry()) {}
  std::string operator()(Value *value) {
    value = getBaseResource(value);
    if (!value->def && value->owner == entry) return "arg" + std::to_string(value->index);
    if (isAllocationValue(value)) {
      auto [it, inserted] = ids.try_emplace(value->def, unsigned(ids.size()));
      return "alloc" + std::to_string(it->second);
    }
    return "%" + (value->hint.empty() ? std::string("value") : value->hint);
  }

private:
  Block *entry;
  std::unordered_map<const Op *, unsigned> ids;
};

bool staticControl(const Op *op, const Op *host) {
  return host->regions[0]->blocks.size() == 1 && op->parentOp() == host && op->parent == host->entry();
}

std::optional<std::size_t> staticBytes(const Value *value) {
  const Type &t = value->type;
  if (!t.isMemRef() || !t.hasStaticShape() || !t.identityLayout) return std::nullopt;
  if (!(t.element == Type::F16 || t.element == Type::F32 || t.element == Type::F64 || t.element == Type::I1 ||
        t.element == Type::I8 || t.element == Type::I32 || t.element == Type::I64))
    return std::nullopt;
  std::size_t elementBytes = (Type::bitWidth(t.element) + 7) / 8;
  std::size_t elements = std::size_t(t.elementCount());
  if (!elementBytes || !elements || elements > std::numeric_limits<std::size_t>::max() / elementBytes ||
      elements * elementBytes > std::size_t(std::numeric_limits<int64_t>::max()))
    return std::nullopt;
  return elements * elementBytes;
}

std::optional<int> deviceOrdinal(const std::string &device) {
  for (const char *prefix : {"cuda:", "rocm:", "hip:"}) {
    size_t n = std::strlen(prefix);
    if (device.compare(0, n, prefix) == 0) {
      std::string rest = device.substr(n);
      if (rest.empty() || !std::all_of(rest.begin(), rest.end(), ::isdigit) || rest.size() > 9) return std::nullopt;
      return std::stoi(rest);
    }
  }
  return std::nullopt;
}

} // namespace

Attr EdgeReason::attr() const {
  return Attr::dictOf({{"alias", Attr::string(alias)}, {"detail", Attr::string(detail)},
                       {"from_location", Attr::string(from)}, {"kind", Attr::string(kind)},
                       {"resource", Attr::string(resource)}, {"to_location", Attr::string(to)}});
}

std::optional<Graph> buildGraph(Module &module, Op *function, const std::map<const Op *, KernelSummary> &summaries,
                                bool reuseStorage) {
  if (function->isDeclaration()) return std::nullopt;
  Graph graph;
  graph.source = function->symName();
  Namer name(function);

  // Nodes in pre-order walk order (GraphAnalysis.cpp:405-416).
  std::vector<Op *> order;
  for (auto &block : function->regions[0]->blocks)
    for (auto &op : block->ops) walkPreOrder(op.get(), [&](Op *o) { order.push_back(o); });
  for (Op *op : order) {
    if (op->name == "ckl.dispatch") {
      Op *callee = module.lookup(symbolOf(op, "kernel"));
      auto found = callee ? summaries.find(callee) : summaries.end();
      if (found == summaries.end())
        throw CompileError(locationText(function) + ": failed to bind a dispatch effect summary");
      const KernelSummary &summary = found->second;
      GraphNode node;
      node.id = unsigned(graph.nodes.size());
      node.kind = "dispatch";
      node.source = op;
      node.kernel = symbolOf(op, "kernel");
      node.orderingScopes = summary.orderingScopes;
      node.unknown = summary.unknown;
      node.synchronizes = summary.synchronizes;
      node.nestedControl = !staticControl(op, function);
      std::vector<Value *> actuals = dispatchArguments(op);
      std::vector<Attr> accesses;
      for (size_t arg = 0; arg < summary.effects.size(); ++arg) {
        if (!summary.effects[arg]) continue;
        if (arg >= actuals.size()) throw CompileError("failed to bind a dispatch effect summary");
        Value *resource = getBaseResource(actuals[arg]);
        AccessRegion region = composeAccessRegion(actuals[arg], summary.regions[arg] ? *summary.regions[arg] : AccessRegion::whole());
        node.accesses.push_back({resource, summary.effects[arg], region});
        accesses.push_back(Attr::dictOf({{"arg", Attr::integer(int64_t(arg))}, {"effects", effectList(summary.effects[arg])},
                                         {"region", region.attr()}, {"resource", Attr::string(name(resource))}}));
      }
      node.materialized = Attr::arrayOf(accesses);
      graph.nodes.push_back(std::move(node));
      continue;
    }
    std::vector<Effect> effects;
    bool modeled, recursive;
    operationEffects(op, effects, modeled, recursive);
    if (!modeled) continue;
    GraphNode node;
    node.source = op;
    node.nestedControl = !staticControl(op, function);
    bool allocates = false, frees = false;
    std::vector<Attr> accesses;
    for (const Effect &effect : effects) {
      unsigned bits = 0;
      if (effect.bits & Allocate) { bits = Allocate; allocates = true; }
      else if (effect.bits & Free) { bits = Free; frees = true; }
      else continue;
      if (!effect.value) throw CompileError("lifetime effect has no addressable resource");
      Value *resource = getBaseResource(effect.value);
      node.accesses.push_back({resource, bits, AccessRegion::whole()});
      accesses.push_back(Attr::dictOf({{"effects", effectList(bits)}, {"region", Attr::string("whole")},
                                       {"resource", Attr::string(name(resource))}}));
    }
    if (accesses.empty()) continue;
    node.id = unsigned(graph.nodes.size());
    node.kind = allocates && frees ? "lifetime" : allocates ? "alloc" : "free";
    node.materialized = Attr::arrayOf(accesses);
    graph.nodes.push_back(std::move(node));
  }
  if (std::none_of(graph.nodes.begin(), graph.nodes.end(), [](const GraphNode &n) { return n.kind == "dispatch"; }))
    return std::nullopt;

  std::unordered_map<const Op *, unsigned> nodeIds;
  for (const GraphNode &n : graph.nodes) nodeIds[n.source] = n.id;
  auto add = [&](unsigned from, unsigned to, EdgeReason reason) {
    if (from != to) graph.edges[{from, to}].push_back(std::move(reason));
  };

  // Explicit completion tokens and SSA producers (GraphAnalysis.cpp:436-458).
  for (const GraphNode &node : graph.nodes) {
    if (node.kind != "dispatch") continue;
    for (Value *token : dispatchDependencies(node.source)) {
      auto found = token->def ? nodeIds.find(token->def) : nodeIds.end();
      if (found == nodeIds.end()) throw CompileError(locationText(node.source) + ": completion dependency is not a graph node");
      add(found->second, node.id, {"explicit", "completion token", "", "", locationText(token->def), locationText(node.source)});
    }
    for (Value *argument : dispatchArguments(node.source)) {
      if (!argument->def) continue;
      auto found = nodeIds.find(argument->def);
      if (found != nodeIds.end())
        add(found->second, node.id, {"ssa", "dispatch argument", "", "", locationText(argument->def), locationText(node.source)});
    }
  }
  // Pairwise unknown barriers and conflicting accesses in program order (460-491).
  for (unsigned from = 0; from < graph.nodes.size(); ++from) {
    const GraphNode &a = graph.nodes[from];
    for (unsigned to = from + 1; to < graph.nodes.size(); ++to) {
      const GraphNode &b = graph.nodes[to];
      if (a.unknown || b.unknown)
        add(from, to, {"barrier", "unknown effect", "", "", locationText(a.source), locationText(b.source)});
      for (const BoundAccess &lhs : a.accesses) {
        for (const BoundAccess &rhs : b.accesses) {
          Alias alias = aliasWholeBuffers(lhs.resource, rhs.resource);
          if (alias == Alias::No || !hasConflictingAccesses(lhs.bits, rhs.bits)) continue;
          bool lifetime = ((lhs.bits | rhs.bits) & (Allocate | Free)) != 0;
          if (!lifetime && alias == Alias::Must && disjointRegions(lhs.region, rhs.region)) continue;
          std::string l = name(lhs.resource), r = name(rhs.resource);
          add(from, to, {lifetime ? "lifetime" : "memory", lifetime ? "resource lifetime" : "overlapping resource access",
                         l == r ? l : l + "~" + r, alias == Alias::Must ? "must" : "may", locationText(a.source),
                         locationText(b.source)});
        }
      }
    }
  }
  if (std::any_of(graph.nodes.begin(), graph.nodes.end(), [](const GraphNode &n) { return n.nestedControl; }))
    for (unsigned to = 1; to < graph.nodes.size(); ++to)
      add(to - 1, to, {"control", "nested control flow", "", "", locationText(graph.nodes[to - 1].source),
                       locationText(graph.nodes[to].source)});

  std::ostringstream dot;
  dot << "digraph \"" << graph.source << "\" {\n";
  for (const GraphNode &n : graph.nodes) {
    dot << "  n" << n.id << " [label=\"" << n.id << ": " << n.kind;
    if (!n.kernel.empty()) dot << " " << n.kernel;
    dot << "\"];\n";
  }
  for (const auto &[edge, reasons] : graph.edges)
    dot << "  n" << edge.first << " -> n" << edge.second << " [label=\"" << reasons.front().kind << "\"];\n";
  dot << "}\n";
  graph.dot = dot.str();

  // Storage-plan bridge (GraphAnalysis.cpp:143-288).
  constexpr std::size_t alignment = 256;
  std::unordered_map<const Value *, std::size_t> index;
  for (const GraphNode &node : graph.nodes) {
    if (node.kind != "dispatch") continue;
    const Attr *deviceAttr = node.source->attr("device");
    std::string device = deviceAttr ? deviceAttr->s : std::string();
    for (const BoundAccess &access : node.accesses) {
      Value *value = getBaseResource(access.resource);
      auto [it, inserted] = index.try_emplace(value, graph.resources.size());
      if (inserted) {
        PlannedResource info;
        info.name = name(value);
        info.device = device;
        info.addressSpace = value->type.memorySpace.empty() ? "global" : value->type.memorySpace;
        info.temporary = isAllocationValue(value);
        info.value = value;
        if (auto bytes = staticBytes(value)) info.bytes = *bytes;
        else if (info.temporary && graph.unavailableReason.empty())
          graph.unavailableReason = "temporary resource " + info.name + " requires a static identity-layout integer or float memref";
        graph.resources.push_back(std::move(info));
      }
      PlannedResource &info = graph.resources[it->second];
      if (info.device != device && graph.unavailableReason.empty())
        graph.unavailableReason = "resource " + info.name + " is used on multiple devices";
      if (info.users.empty() || info.users.back() != node.id) info.users.push_back(node.id);
    }
  }
  if (graph.unavailableReason.empty()) {
    std::vector<planning::Resource> plannerResources;
    for (std::size_t k = 0; k < graph.resources.size(); ++k) {
      const PlannedResource &r = graph.resources[k];
      if (!r.temporary) continue;
      auto ordinal = deviceOrdinal(r.device);
      if (!ordinal) { graph.unavailableReason = "only cuda:<ordinal>, rocm:<ordinal> or hip:<ordinal> devices are supported"; break; }
      plannerResources.push_back({r.name, r.bytes, alignment, r.addressSpace, *ordinal, planning::ResourceKind::Temporary,
                                  std::vector<planning::NodeId>(r.users.begin(), r.users.end())});
      graph.plannerToResource.push_back(k);
    }
    if (graph.unavailableReason.empty()) {
      std::vector<planning::GraphEdge> edges;
      for (const auto &[edge, _] : graph.edges) edges.push_back({edge.first, edge.second});
      auto planned = planning::MemoryPlanner(reuseStorage).tryPlan(graph.nodes.size(), edges, plannerResources);
      graph.reuseStorage = reuseStorage;
      if (planned) { graph.plan = *planned.value; graph.planned = true; }
      else graph.unavailableReason = planned.error;
    }
  }
  return graph;
}

// Argument descriptors of a dispatch node: what executable lowering will do with each argument
// (resource packing with a view's byte range, constant, or host scalar argN), so that an
// unsupported view or layout is visible in the graph before lowering rejects it.
static Attr argumentDescriptors(const Op *dispatch, const Op *function, Namer &name) {
  std::vector<Attr> out;
  std::vector<Value *> actuals = dispatchArguments(dispatch);
  for (size_t index = 0; index < actuals.size(); ++index) {
    Value *argument = actuals[index];
    std::vector<std::pair<std::string, Attr>> e = {{"index", Attr::integer(int64_t(index))},
                                                   {"type", Attr::typeAttr(argument->type)}};
    if (argument->type.isMemRef()) {
      e.push_back({"kind", Attr::string("resource")});
      e.push_back({"resource", Attr::string(name(argument))});
      std::string packing = "direct_pointer";
      if (getBaseResource(argument) != argument) {
        if (auto range = staticResourceRange(argument)) {
          e.push_back({"byte_offset", Attr::integer(range->offset)});
          e.push_back({"byte_length", Attr::integer(range->length)});
        } else {
          packing = "unsupported_view";
        }
      } else if (!argument->type.identityLayout || argument->type.unranked) {
        packing = "unsupported_layout";
      }
      e.push_back({"packing", Attr::string(packing)});
    } else if (argument->def) {
      if (const Attr *value = argument->def->attr("value")) {
        e.push_back({"kind", Attr::string("constant")});
        e.push_back({"value", *value});
      } else {
        e.push_back({"kind", Attr::string("unsupported")});
      }
    } else {
      e.push_back({"kind", Attr::string(argument->owner == function->entry() ? "scalar" : "unsupported")});
      e.push_back({"name", Attr::string("arg" + std::to_string(argument->index))});
    }
    out.push_back(Attr::dictOf(e));
  }
  return Attr::arrayOf(out);
}

static const Op *functionOf(const Op *op) {
  for (const Op *p = op ? op->parentOp() : nullptr; p; p = p->parentOp())
    if (p->name == "func.func") return p;
  return nullptr;
}

std::string Graph::print() const {
  std::ostringstream out;
  // Resource names as the lowering assigns them: allocations numbered by first use in node order.
  const Op *function = nodes.empty() ? nullptr : functionOf(nodes.front().source);
  std::optional<Namer> name;
  if (function) {
    name.emplace(function);
    for (const GraphNode &node : nodes)
      for (const BoundAccess &access : node.accesses) (*name)(access.resource);
  }
  std::vector<Attr> resourceAttrs;
  for (const PlannedResource &r : resources) {
    std::vector<std::pair<std::string, Attr>> e = {
        {"address_space", Attr::string(r.addressSpace)}, {"alignment", Attr::integer(256)},
        {"device", Attr::string(r.device)}, {"kind", Attr::string(r.temporary ? "temporary" : "external")},
        {"name", Attr::string(r.name)}};
    if (r.bytes) e.push_back({"bytes", Attr::integer(int64_t(r.bytes))});
    e.push_back({"users", Attr::denseI64(std::vector<int64_t>(r.users.begin(), r.users.end()))});
    resourceAttrs.push_back(Attr::dictOf(e));
  }
  Attr memoryPlan;
  if (!planned) {
    memoryPlan = Attr::dictOf({{"reason", Attr::string(unavailableReason)}, {"status", Attr::string("unavailable")}});
  } else {
    std::vector<Attr> heaps, assignments, decisions;
    for (const auto &h : plan.heaps)
      heaps.push_back(Attr::dictOf({{"address_space", Attr::string(h.addressSpace)}, {"alignment", Attr::integer(int64_t(h.alignment))},
                                    {"bytes", Attr::integer(int64_t(h.bytes))}, {"device", Attr::integer(h.device)}}));
    for (const auto &a : plan.assignments)
      assignments.push_back(Attr::dictOf({{"bytes", Attr::integer(int64_t(a.bytes))}, {"heap", Attr::integer(int64_t(a.heap))},
                                          {"offset", Attr::integer(int64_t(a.offset))},
                                          {"resource", Attr::string(resources[plannerToResource[a.resource]].name)},
                                          {"slot", Attr::integer(int64_t(a.slot))}}));
    for (const auto &d : plan.decisions) {
      std::vector<Attr> shares;
      for (auto prev : d.sharesWith) shares.push_back(Attr::string(resources[plannerToResource[prev]].name));
      decisions.push_back(Attr::dictOf({{"reason", Attr::string(d.reason)},
                                        {"resource", Attr::string(resources[plannerToResource[d.resource]].name)},
                                        {"shares_with", Attr::arrayOf(shares)}, {"slot", Attr::integer(int64_t(d.slot))}}));
    }
    memoryPlan = Attr::dictOf({{"assignments", Attr::arrayOf(assignments)}, {"baseline_bytes", Attr::integer(int64_t(plan.baselineBytes))},
                               {"decisions", Attr::arrayOf(decisions)}, {"heaps", Attr::arrayOf(heaps)},
                               {"planned_bytes", Attr::integer(int64_t(plan.plannedBytes))}, {"status", Attr::string("planned")}});
  }
  out << "  \"ckl.graph\"() <" << Attr::dictOf({{"dot", Attr::string(dot)}, {"name", Attr::string(source + ".graph")},
                                               {"source", Attr::symbol(source)}}).str() << "> ({\n";
  for (const GraphNode &n : nodes) {
    std::vector<std::pair<std::string, Attr>> props = {
        {"accesses", n.materialized}, {"id", Attr::integer(n.id)}, {"kind", Attr::string(n.kind)},
        {"ordering_scopes", Attr::arrayOf([&] { std::vector<Attr> v; for (auto &s : n.orderingScopes) v.push_back(Attr::string(s)); return v; }())},
        {"source", Attr::string(locationText(n.source))}, {"synchronizes", Attr::boolean(n.synchronizes)},
        {"unknown", Attr::boolean(n.unknown)}};
    if (!n.kernel.empty()) props.push_back({"kernel", Attr::symbol(n.kernel)});
    std::vector<std::pair<std::string, Attr>> extra = {
        {"ckl.execution_control", Attr::string(n.nestedControl ? "unsupported_control_flow" : "unconditional")}};
    if (n.kind == "dispatch") {
      const Op *op = n.source;
      for (const char *key : {"grid", "block"})
        if (const Attr *a = op->attr(key)) extra.push_back({std::string("ckl.launch_") + key, *a});
      if (const Attr *a = op->attr("shared_memory")) extra.push_back({"ckl.launch_shared_memory", *a});
      if (const Attr *a = op->attr("device")) extra.push_back({"ckl.launch_device", *a});
      if (const Attr *a = op->attr("implementation")) extra.push_back({"ckl.launch_implementation", *a});
      if (const Attr *a = op->attr("artifact") ? op->attr("artifact") : op->attr("implementation"))
        extra.push_back({"ckl.launch_artifact", *a});
      if (const Attr *a = op->attr("capabilities")) {
        extra.push_back({"ckl.launch_capabilities", *a});
        for (const Attr &c : a->array)
          if (c.s == "cuda.direct" || c.s == "rocm.bare_ptr") extra.push_back({"ckl.launch_abi", c});
      }
      if (name) extra.push_back({"ckl.arguments", argumentDescriptors(op, function, *name)});
    }
    out << "    \"ckl.graph_node\"() <" << Attr::dictOf(props).str() << "> " << Attr::dictOf(extra).str()
        << " : () -> ()\n";
  }
  for (const auto &[edge, reasons] : edges) {
    std::vector<Attr> rs;
    for (const EdgeReason &r : reasons) rs.push_back(r.attr());
    out << "    \"ckl.graph_edge\"() <" << Attr::dictOf({{"from", Attr::integer(edge.first)}, {"reasons", Attr::arrayOf(rs)},
                                                        {"to", Attr::integer(edge.second)}}).str()
        << "> : () -> ()\n";
  }
  out << "  }) " << Attr::dictOf({{"ckl.memory_plan", memoryPlan}, {"ckl.resources", Attr::arrayOf(resourceAttrs)}}).str()
      << " : () -> ()\n";
  return out.str();
}

// ====================================================================== transitive reduction
// lib/Analysis/GraphAlgorithms.cpp:10-46

std::map<unsigned, std::vector<unsigned>> reducedDispatchDependencies(const Graph &graph) {
  std::vector<planning::GraphEdge> edges;
  for (const auto &[edge, _] : graph.edges) edges.push_back({edge.first, edge.second});
  planning::Reachability reach(graph.nodes.size(), edges);
  std::vector<unsigned> dispatches;
  for (const GraphNode &n : graph.nodes) if (n.kind == "dispatch") dispatches.push_back(n.id);
  std::map<unsigned, std::vector<unsigned>> result;
  for (unsigned target : dispatches)
    for (unsigned candidate : dispatches) {
      if (candidate >= target || !reach.reaches(candidate, target)) continue;
      bool transitive = std::any_of(dispatches.begin(), dispatches.end(), [&](unsigned mid) {
        return candidate < mid && mid < target && reach.reaches(candidate, mid) && reach.reaches(mid, target);
      });
      if (!transitive) result[target].push_back(candidate);
    }
  return result;
}

// ====================================================================== executable plan
// lib/Transforms/ExecutablePlan.cpp:101-233, lib/Dialect/Exec/IR/CKLExecOps.cpp:35-192

Attr ExecArgument::attr() const {
  std::vector<std::pair<std::string, Attr>> e = {{"kind", Attr::string(kind)}, {"logical_index", Attr::integer(logicalIndex)},
                                                 {"slot", Attr::integer(slot)}, {"type", Attr::typeAttr(type)}};
  if (kind == "resource") {
    e.push_back({"resource", Attr::string(resource)});
    e.push_back({"packing", Attr::string(packing)});
    if (byteLength >= 0) {
      e.push_back({"byte_offset", Attr::integer(byteOffset)});
      e.push_back({"byte_length", Attr::integer(byteLength)});
    }
  } else if (kind == "scalar") {
    e.push_back({"name", Attr::string(name)});
  } else {
    e.push_back({"value", value});
  }
  return Attr::dictOf(e);
}

std::vector<uint8_t> constantBytes(const Attr &value, const Type &type) {
  unsigned width = Type::bitWidth(type.kind);
  if (!width || width % 8 || width > 64) throw CompileError("host lowering requires byte-sized scalars up to 64 bits");
  uint64_t bits = 0;
  if (value.kind == Attr::Int) bits = uint64_t(value.i);
  else if (value.kind == Attr::Float) {
    if (type.kind == Type::F32) { float f = float(value.f); uint32_t b; std::memcpy(&b, &f, 4); bits = b; }
    else std::memcpy(&bits, &value.f, 8);
  } else if (value.kind == Attr::Bool) bits = uint64_t(value.i);
  else throw CompileError("unsupported constant argument value");
  std::vector<uint8_t> out(width / 8);
  for (size_t k = 0; k < out.size(); ++k) out[k] = uint8_t(bits >> (8 * k));
  return out;
}

static std::string denseText(const std::vector<int64_t> &v) { return Attr::denseI64(v).str(); }

std::string ExecPlan::print() const {
  std::ostringstream out;
  out << "  \"ckl_exec.plan\"() <" << Attr::dictOf({{"backend", Attr::string(backend)}, {"name", Attr::string(name)},
                                                   {"source", Attr::symbol(source)}}).str() << "> ({\n";
  for (const ExecHeap &h : heaps)
    out << "    \"ckl_exec.heap\"() <" << Attr::dictOf({{"address_space", Attr::string(h.addressSpace)},
                                                       {"alignment", Attr::integer(h.alignment)}, {"bytes", Attr::integer(h.bytes)},
                                                       {"device", Attr::integer(h.device)}, {"id", Attr::integer(h.id)}}).str()
        << "> : () -> ()\n";
  for (const ExecResource &r : resources) {
    std::vector<std::pair<std::string, Attr>> e = {{"address_space", Attr::string(r.addressSpace)},
                                                   {"alignment", Attr::integer(r.alignment)},
                                                   {"device", Attr::string(r.device)}, {"kind", Attr::string(r.kind)},
                                                   {"name", Attr::string(r.name)}};
    if (r.bytes) e.push_back({"bytes", Attr::integer(r.bytes)});
    if (r.kind == "temporary") { e.push_back({"heap", Attr::integer(r.heap)}); e.push_back({"offset", Attr::integer(r.offset)}); }
    out << "    \"ckl_exec.resource\"() <" << Attr::dictOf(e).str() << "> : () -> ()\n";
  }
  for (const ExecHeap &h : workspaceHeaps)
    out << "    \"ckl_exec.workspace_heap\"() <" << Attr::dictOf({{"alignment", Attr::integer(h.alignment)},
                                                                 {"bytes", Attr::integer(h.bytes)},
                                                                 {"device", Attr::integer(h.device)},
                                                                 {"id", Attr::integer(h.id)}}).str()
        << "> : () -> ()\n";
  for (const ExecWorkspace &w : workspaces)
    out << "    \"ckl_exec.workspace\"() <" << Attr::dictOf({{"bytes", Attr::integer(w.bytes)}, {"heap", Attr::integer(w.heap)},
                                                            {"kernel", Attr::integer(w.kernel)}, {"name", Attr::string(w.name)},
                                                            {"offset", Attr::integer(w.offset)}, {"role", Attr::string(w.role)}}).str()
        << "> : () -> ()\n";
  for (const ExecKernel &k : kernels) {
    std::vector<Attr> args;
    for (const ExecArgument &a : k.arguments) args.push_back(a.attr());
    std::vector<std::pair<std::string, Attr>> e = {
        {"abi", Attr::string(k.abi)}, {"arguments", Attr::arrayOf(args)}, {"artifact", Attr::string(k.artifact)},
        {"block", Attr::denseI64(k.block)}, {"dependencies", Attr::denseI64(k.dependencies)}, {"device", Attr::string(k.device)},
        {"entry_point", Attr::string(k.function)}, {"grid", Attr::denseI64(k.grid)}, {"id", Attr::integer(k.id)},
        {"implementation", Attr::string(k.implementation)}, {"kernel", Attr::symbol(k.kernel)},
        {"logical_block", Attr::denseI64(k.logicalBlock)}, {"logical_grid", Attr::denseI64(k.logicalGrid)},
        {"shared_memory", Attr::integer(k.sharedMemory)}};
    if (!k.group.empty()) e.push_back({"group", Attr::string(k.group)});
    if (k.workspace) e.push_back({"workspace", Attr::integer(k.workspace)});
    if (k.partials >= 0) e.push_back({"partials", Attr::integer(k.partials)});
    out << "    \"ckl_exec.kernel\"() <" << Attr::dictOf(e).str() << "> : () -> ()\n";
  }
  out << "  }) : () -> ()\n";
  (void)denseText;
  return out.str();
}

void ExecPlan::verify() const {
  std::set<int64_t> heapIds, kernelIds;
  std::map<int64_t, int64_t> heapBytes;
  std::map<std::string, const ExecResource *> byName;
  for (const ExecHeap &h : heaps) {
    if (h.id < 0 || h.bytes <= 0) throw CompileError("'ckl_exec.heap' op requires a non-negative id and positive byte size");
    if (h.alignment <= 0 || (h.alignment & (h.alignment - 1))) throw CompileError("'ckl_exec.heap' op requires power-of-two alignment");
    if (!heapIds.insert(h.id).second) throw CompileError("'ckl_exec.heap' op has a duplicate heap id");
    heapBytes[h.id] = h.bytes;
  }
  for (const ExecResource &r : resources) {
    if (r.name.empty() || (r.kind != "external" && r.kind != "temporary"))
      throw CompileError("'ckl_exec.resource' op requires a name and external or temporary kind");
    if (!byName.emplace(r.name, &r).second) throw CompileError("'ckl_exec.resource' op has a duplicate resource name");
    if (r.kind == "temporary") {
      if (r.bytes <= 0 || r.heap < 0 || r.offset < 0)
        throw CompileError("'ckl_exec.resource' op temporary resource requires positive bytes and non-negative placement");
      if (!heapIds.count(r.heap)) throw CompileError("'ckl_exec.resource' op references an unknown heap");
      if (r.offset % r.alignment) throw CompileError("'ckl_exec.resource' op heap offset does not satisfy resource alignment");
      if (r.offset > heapBytes[r.heap] || r.bytes > heapBytes[r.heap] - r.offset)
        throw CompileError("'ckl_exec.resource' op placement exceeds its heap");
    }
  }
  if (workspaceHeaps.size() > 1) throw CompileError("'ckl_exec.workspace_heap' op may appear at most once");
  for (const ExecHeap &h : workspaceHeaps) {
    if (h.bytes <= 0 || h.alignment <= 0 || (h.alignment & (h.alignment - 1)) || !heapIds.insert(h.id).second)
      throw CompileError("'ckl_exec.workspace_heap' op requires a new heap id, positive bytes and power-of-two alignment");
    heapBytes[h.id] = h.bytes;
  }
  std::map<int64_t, std::map<std::string, const ExecWorkspace *>> roles;
  std::set<std::string> workspaceNames;
  for (const ExecWorkspace &w : workspaces) {
    if (!workspaceNames.insert(w.name).second) throw CompileError("'ckl_exec.workspace' op has a duplicate name");
    if (workspaceHeaps.empty() || w.heap != workspaceHeaps.front().id)
      throw CompileError("'ckl_exec.workspace' op must be placed in the workspace heap");
    if (w.role != "state" && w.role != "partials") throw CompileError("'ckl_exec.workspace' op role must be state or partials");
    if (w.bytes <= 0 || w.offset < 0 || w.offset % 256 || w.offset > heapBytes[w.heap] || w.bytes > heapBytes[w.heap] - w.offset)
      throw CompileError("'ckl_exec.workspace' op placement exceeds its heap");
    if (w.name.empty() || byName.count(w.name) || !roles[w.kernel].emplace(w.role, &w).second)
      throw CompileError("'ckl_exec.workspace' op requires a new name and one placement per kernel and role");
  }
  for (const auto &[kernel, _] : roles)
    if (std::none_of(kernels.begin(), kernels.end(), [&](const ExecKernel &k) { return k.id == kernel; }))
      throw CompileError("'ckl_exec.workspace' op references an unknown kernel");
  for (const ExecKernel &k : kernels) {
    if (!kernelIds.insert(k.id).second) throw CompileError("'ckl_exec.kernel' op has a duplicate kernel id");
    if (k.workspace < 0 || k.partials < -1) throw CompileError("'ckl_exec.kernel' op workspace sizes must be non-negative");
    auto placed = roles.find(k.id);
    auto bytesOf = [&](const char *role) -> int64_t {
      if (placed == roles.end() || !placed->second.count(role)) return 0;
      return placed->second.at(role)->bytes;
    };
    if (!workspaceHeaps.empty() && (bytesOf("state") != k.workspace || bytesOf("partials") != std::max<int64_t>(k.partials, 0)))
      throw CompileError("'ckl_exec.kernel' op workspace sizes do not match its placed workspaces");
    if (workspaceHeaps.empty() && k.partials > 0)
      throw CompileError("'ckl_exec.kernel' op with partial planes requires a workspace heap");
    if (k.implementation.empty() || k.artifact.empty() || k.abi.empty() || k.device.empty())
      throw CompileError("'ckl_exec.kernel' op requires implementation, artifact, ABI, and device identities");
    for (const auto *dims : {&k.grid, &k.block})
      if (dims->size() != 3 || std::any_of(dims->begin(), dims->end(), [](int64_t d) { return d <= 0; }))
        throw CompileError("'ckl_exec.kernel' op requires three positive launch dimensions");
    std::set<int64_t> seen;
    for (int64_t d : k.dependencies) {
      if (d < 0 || d >= k.id) throw CompileError("'ckl_exec.kernel' op dependencies must reference earlier kernel ids");
      if (!seen.insert(d).second) throw CompileError("'ckl_exec.kernel' op contains a duplicate dependency");
      if (!kernelIds.count(d)) throw CompileError("'ckl_exec.kernel' op references an unknown kernel dependency");
    }
    std::set<int64_t> slots;
    for (const ExecArgument &a : k.arguments) {
      if (!slots.insert(a.slot).second) throw CompileError("'ckl_exec.kernel' op contains a duplicate physical argument slot");
      if (a.kind == "resource") {
        auto it = byName.find(a.resource);
        if (it == byName.end()) throw CompileError("'ckl_exec.kernel' op argument references an unknown resource");
        if (k.abi == "rocm.bare_ptr" && a.packing != "bare_pointer")
          throw CompileError("'ckl_exec.kernel' op rocm.bare_ptr resource arguments require bare_pointer packing");
        if (k.abi == "cuda.direct" && a.packing != "direct_pointer")
          throw CompileError("'ckl_exec.kernel' op cuda.direct resource arguments require direct_pointer packing");
        if (a.byteLength >= 0) {
          // The range lies inside the resource, is as long as the argument's static identity-layout
          // memref, and starts on an element boundary.
          int64_t bound = it->second->bytes;
          const Type &t = a.type;
          int64_t element = t.isMemRef() ? int64_t(Type::bitWidth(t.element) / 8) : 0;
          bool typed = t.isMemRef() && t.hasStaticShape() && t.identityLayout && element > 0 &&
                       Type::bitWidth(t.element) % 8 == 0 && t.elementCount() * element == a.byteLength;
          if (a.byteOffset < 0 || a.byteLength <= 0 || a.byteOffset > bound || a.byteLength > bound - a.byteOffset ||
              !typed || a.byteOffset % element)
            throw CompileError("'ckl_exec.kernel' op invalid or out-of-bounds resource byte range");
        }
      } else if (a.kind == "scalar") {
        if (a.name.empty()) throw CompileError("'ckl_exec.kernel' op scalar argument requires a non-empty binding name");
      } else if (a.kind == "constant" || a.kind == "bytes") {
        if (a.bytes.empty()) throw CompileError("'ckl_exec.kernel' op constant argument requires a value");
      } else {
        throw CompileError("'ckl_exec.kernel' op contains an unsupported physical argument kind");
      }
    }
    for (int64_t s = 0; s < int64_t(k.arguments.size()); ++s)
      if (!slots.count(s)) throw CompileError("'ckl_exec.kernel' op physical argument slots must be contiguous");
  }
}

static std::vector<int64_t> dims3(const Attr *a) {
  if (!a) return {};
  std::vector<int64_t> out = a->dense;
  return out;
}

// Library workspaces (HIP addition, no reference counterpart): one workspace heap, numbered after
// the plan's heaps, so the temporaries' heaps and offsets stay those of the reference planner.
// State parts (zero page, completion counters) are laid out one after another at its start and
// never shared. Partial planes are placed by the storage planner with the temporaries' reuse
// setting, over the graph's nodes and edges; the users of a kernel's planes are the kernel and
// every later dispatch that accesses a resource the kernel writes: its readers, which add the
// planes themselves when the inferred graph defers the kernel's combine to them. (The graph's
// may-alias edges from a kernel to later writers of other external buffers order those writers
// after it, but they never read its planes.)
static void planWorkspaces(ExecPlan &plan, const Graph &graph) {
  constexpr std::size_t alignment = 256;
  // Readers of what a kernel writes: later dispatches that access the same base resource.
  auto readers = [&](std::size_t node) {
    std::vector<planning::NodeId> out;
    std::set<const Value *> written;
    for (const BoundAccess &a : graph.nodes.at(node).accesses)
      if (a.bits & Write) written.insert(getBaseResource(a.resource));
    for (std::size_t n = node + 1; n < graph.nodes.size(); ++n) {
      if (graph.nodes[n].kind != "dispatch") continue;
      for (const BoundAccess &a : graph.nodes[n].accesses)
        if (written.count(getBaseResource(a.resource))) { out.push_back(n); break; }
    }
    return out;
  };
  const int64_t heapId = int64_t(plan.heaps.size());
  int64_t state = 0;
  int device = -1;
  std::vector<planning::Resource> planes;
  std::vector<int64_t> owners;
  for (const ExecKernel &k : plan.kernels) {
    if (k.workspace < 0 || k.partials < -1) throw CompileError("library workspace sizes must be non-negative");
    if (!k.workspace && k.partials <= 0) continue;
    auto ordinal = deviceOrdinal(k.device);
    if (!ordinal || (device >= 0 && *ordinal != device))
      throw CompileError("library workspaces require one rocm:<ordinal> device");
    device = *ordinal;
    const std::string id = std::to_string(k.id);
    if (k.workspace) {
      plan.workspaces.push_back({"workspace" + id, "state", k.id, heapId, state, k.workspace});
      state += int64_t(planning::alignUp(std::size_t(k.workspace), alignment));
    }
    if (k.partials > 0) {
      std::vector<planning::NodeId> users{planning::NodeId(k.id)};
      for (planning::NodeId s : readers(std::size_t(k.id))) users.push_back(s);
      std::sort(users.begin(), users.end());
      users.erase(std::unique(users.begin(), users.end()), users.end());
      planes.push_back({"partials" + id, std::size_t(k.partials), alignment, "global", device,
                        planning::ResourceKind::Temporary, std::move(users)});
      owners.push_back(k.id);
    }
  }
  if (device < 0) return;
  int64_t bytes = state;
  if (!planes.empty()) {
    std::vector<planning::GraphEdge> edges;
    for (const auto &[edge, _] : graph.edges) edges.push_back({edge.first, edge.second});
    auto placed = planning::MemoryPlanner(graph.reuseStorage).tryPlan(graph.nodes.size(), edges, planes);
    if (!placed) throw CompileError("library workspace planning failed: " + placed.error);
    if (placed.value->heaps.size() != 1) throw CompileError("library workspace planes must form one heap");
    for (const planning::Assignment &a : placed.value->assignments)
      plan.workspaces.push_back({planes[a.resource].name, "partials", owners[a.resource], heapId,
                                 state + int64_t(a.offset), int64_t(planes[a.resource].bytes)});
    bytes = state + int64_t(placed.value->heaps.front().bytes);
  }
  plan.workspaceHeaps.push_back({heapId, bytes, int64_t(alignment), device, "global"});
}

ExecPlan lowerGraphToExec(const Module &module, const Op *function, const Graph &graph) {
  (void)module;
  if (!graph.planned) throw CompileError("executable lowering requires a successful static memory plan");
  for (const GraphNode &node : graph.nodes)
    if (node.nestedControl)
      throw CompileError("executable lowering does not support graph nodes nested in region or CFG control flow; "
                         "conditional and repeated execution must be represented explicitly before lowering");

  ExecPlan plan;
  plan.source = graph.source;
  plan.name = graph.source + ".graph.exec";
  if (Block *entry = function->entry())
    for (auto &arg : entry->args) plan.sourceArguments.push_back(arg->type);

  std::string backend;
  for (const GraphNode &node : graph.nodes) {
    if (node.kind != "dispatch") continue;
    const Attr *device = node.source->attr("device");
    if (!device) throw CompileError("executable lowering requires one known backend");
    std::string current = device->s.substr(0, device->s.find(':'));
    if (current.empty() || (!backend.empty() && current != backend)) throw CompileError("executable lowering requires one known backend");
    backend = current;
  }
  plan.backend = backend;
  auto reduced = reducedDispatchDependencies(graph);

  for (size_t k = 0; k < graph.plan.heaps.size(); ++k) {
    const auto &h = graph.plan.heaps[k];
    plan.heaps.push_back({int64_t(k), int64_t(h.bytes), int64_t(h.alignment), h.device, h.addressSpace});
  }
  std::map<std::string, const planning::Assignment *> assignments;
  for (const auto &a : graph.plan.assignments) assignments[graph.resources[graph.plannerToResource[a.resource]].name] = &a;
  for (const PlannedResource &r : graph.resources) {
    ExecResource out;
    out.name = r.name;
    out.kind = r.temporary ? "temporary" : "external";
    out.device = r.device;
    out.addressSpace = r.addressSpace;
    out.alignment = 256;
    out.bytes = int64_t(r.bytes);
    if (r.temporary) {
      auto found = assignments.find(r.name);
      if (found == assignments.end()) throw CompileError("temporary resource is missing a memory-plan assignment");
      out.heap = int64_t(found->second->heap);
      out.offset = int64_t(found->second->offset);
    } else if (!r.value->def && r.name.rfind("arg", 0) == 0) {
      out.argument = int64_t(r.value->index);
    }
    plan.resources.push_back(std::move(out));
  }

  Namer name(function);
  // Reproduce the namer's allocation numbering (first use in node order).
  for (const GraphNode &node : graph.nodes)
    for (const BoundAccess &access : node.accesses) name(access.resource);

  for (const GraphNode &node : graph.nodes) {
    if (node.kind != "dispatch") continue;
    const Op *op = node.source;
    ExecKernel k;
    k.id = node.id;
    k.kernel = node.kernel;
    const Attr *implementation = op->attr("implementation");
    const Attr *artifact = op->attr("artifact") ? op->attr("artifact") : implementation;
    const Attr *device = op->attr("device");
    const Attr *capabilities = op->attr("capabilities");
    std::string abi;
    if (capabilities)
      for (const Attr &c : capabilities->array)
        if (c.s == "cuda.direct" || c.s == "rocm.bare_ptr") abi = c.s;
    if (!implementation || !artifact || abi.empty() || !device || !op->attr("grid") || !op->attr("block") || !op->attr("shared_memory"))
      throw CompileError("executable lowering requires complete launch and ABI metadata");
    k.implementation = implementation->s;
    k.artifact = artifact->s;
    k.abi = abi;
    k.device = device->s;
    k.logicalGrid = dims3(op->attr("grid"));
    k.logicalBlock = dims3(op->attr("block"));
    k.sharedMemory = op->attr("shared_memory")->i;
    const Attr *entryPoint = op->attr("ckl.hip.entry_point");
    k.function = entryPoint ? entryPoint->s : node.kernel;
    k.grid = op->attr("ckl.hip.grid") ? dims3(op->attr("ckl.hip.grid")) : k.logicalGrid;
    k.block = op->attr("ckl.hip.block") ? dims3(op->attr("ckl.hip.block")) : k.logicalBlock;
    if (const Attr *shared = op->attr("ckl.hip.shared_memory")) k.sharedMemory = shared->i;
    if (const Attr *group = op->attr("ckl.hip.group")) k.group = group->s;
    if (const Attr *workspace = op->attr("ckl.hip.workspace")) k.workspace = workspace->i;
    if (const Attr *partials = op->attr("ckl.hip.partials")) k.partials = partials->i;

    std::vector<Value *> actuals = dispatchArguments(op);
    for (size_t slot = 0; slot < actuals.size(); ++slot) {
      Value *argument = actuals[slot];
      ExecArgument a;
      a.slot = a.logicalIndex = int64_t(slot);
      a.type = argument->type;
      if (argument->type.isMemRef()) {
        a.kind = "resource";
        a.resource = name(argument);
        Value *base = getBaseResource(argument);
        a.packing = "direct_pointer";
        if (base != argument) {
          if (auto range = staticResourceRange(argument)) { a.byteOffset = range->offset; a.byteLength = range->length; }
          else a.packing = "unsupported_view";
        } else if (!argument->type.identityLayout || argument->type.unranked) {
          a.packing = "unsupported_layout";
        }
        if (a.packing == "unsupported_view")
          throw CompileError("executable lowering does not support view/subview resource arguments in the direct-pointer ABI; "
                             "CKL backend lowering must preserve the view offset in physical argument packing");
        if (a.packing == "unsupported_layout")
          throw CompileError("executable lowering does not support non-identity or unranked resource layouts in the direct-pointer ABI");
        if (abi == "rocm.bare_ptr") a.packing = "bare_pointer";
      } else if (argument->def && argument->def->attr("value")) {
        a.kind = "constant";
        a.value = *argument->def->attr("value");
        a.bytes = constantBytes(a.value, a.type);
      } else if (!argument->def) {
        a.kind = "scalar";
        a.name = "arg" + std::to_string(argument->index);
        if (argument->owner != function->entry())
          throw CompileError("host lowering requires original argN bindings within the source signature");
      } else {
        throw CompileError("unsupported host argument binding");
      }
      k.arguments.push_back(std::move(a));
    }
    if (const Attr *constants = op->attr("ckl.hip.constants")) {
      for (const Attr &c : constants->array) {
        ExecArgument a;
        a.slot = a.logicalIndex = int64_t(k.arguments.size());
        a.kind = "constant";
        a.type = c.type;
        a.value = c;
        a.bytes = constantBytes(c, c.type);
        k.arguments.push_back(std::move(a));
      }
    }
    auto deps = reduced.find(node.id);
    if (deps != reduced.end()) k.dependencies.assign(deps->second.begin(), deps->second.end());
    plan.kernels.push_back(std::move(k));
  }
  planWorkspaces(plan, graph);
  plan.verify();
  return plan;
}

// ====================================================================== HIP preparation
// lib/Transforms/CudaKernels.cpp:20-153 (validation, artifact identity, dispatch metadata)

static bool numericScalar(const Type &t) {
  return t.kind == Type::I32 || t.kind == Type::I64 || t.kind == Type::F32 || t.kind == Type::F64;
}

std::string prepareHip(Module &module, const PrepareOptions &options) {
  unsigned count = 0;
  for (Op *function : module.functions()) {
    if (!function->attr("ckl.kernel")) continue;
    ++count;
    const Attr *results = function->attr("ckl.num_results");
    if (function->isDeclaration() || (results && results->i) || function->regions[0]->blocks.size() != 1)
      throw CompileError("HIP kernels require one defined entry block and no results");
    for (auto &arg : function->entry()->args) {
      Type t = arg->type;
      if (t.isMemRef()) {
        if (!t.hasStaticShape() || !t.identityLayout || !t.memorySpace.empty())
          throw CompileError("HIP direct ABI requires static identity-layout default-space memrefs");
        t = Type::scalar(t.element);
      }
      if (!numericScalar(t)) throw CompileError("HIP direct ABI supports only f32, f64, i32, and i64 arguments/elements");
    }
    bool supported = true;
    std::string bad;
    for (auto &op : function->entry()->ops)
      walkPreOrder(op.get(), [&](Op *o) {
        const std::string &n = o->name;
        bool ok = n == "ckl.load_element" || n == "ckl.store_element" || n == "ckl.thread_id" || n == "ckl.block_id" ||
                  n == "ckl.block_dim" || n == "ckl.grid_dim" || n == "ckl.global_id" || n == "func.return" || n == "scf.if" ||
                  n == "scf.for" || n == "scf.yield" || n.rfind("arith.", 0) == 0 || n == "math.exp" || n == "math.rsqrt";
        if (!ok && supported) { supported = false; bad = n; }
      });
    if (!supported)
      throw CompileError("unsupported operation '" + bad + "' in CKL HIP kernel; legacy whole-buffer operations have no device semantics");
  }
  if (!count) throw CompileError("HIP lowering requires at least one marked CKL kernel");

  Sha256 hash;
  hash.update("ckl.hip.v1;bare-ptr;index64;opt3;");
  hash.update(options.chip);
  hash.update(";");
  hash.update(options.features);
  for (Op *function : module.functions()) {
    if (!function->attr("ckl.kernel")) continue;
    auto summary = function->attrs.find("ckl.effect_summary");
    Attr saved;
    bool had = summary != function->attrs.end();
    if (had) { saved = summary->second; function->attrs.erase(summary); }
    hash.update(printOp(*function));
    if (had) function->attrs["ckl.effect_summary"] = saved;
  }
  std::string artifact = "ckl.hip." + hash.hex();

  const Attr *selection = module.op->attr("ckl.hip.selection");
  std::vector<Op *> dispatches;
  walkPreOrder(module.op.get(), [&](Op *o) { if (o->name == "ckl.dispatch") dispatches.push_back(o); });
  for (Op *dispatch : dispatches) {
    std::string symbol = symbolOf(dispatch, "kernel");
    Op *kernel = module.lookup(symbol);
    if (!kernel || !kernel->attr("ckl.kernel")) throw CompileError("HIP dispatch must reference a marked CKL kernel");
    const Attr *device = dispatch->attr("device");
    if (device && device->s != "unassigned:0" && device->s != "rocm:0")
      throw CompileError("initial CKL HIP compilation supports only logical device 0");
    const Attr *grid = dispatch->attr("grid");
    const Attr *block = dispatch->attr("block");
    if (!grid || !block || grid->dense.size() != 3 || block->dense.size() != 3)
      throw CompileError("'ckl.dispatch' op requires exactly three grid and block dimensions");
    for (int64_t d : grid->dense)
      if (d <= 0 || d > int64_t(UINT32_MAX)) throw CompileError("HIP grid dimension exceeds the physical launch ABI");
    uint64_t threads = 1;
    for (int64_t d : block->dense) {
      if (d <= 0 || d > 1024 || threads > 1024 / uint64_t(d)) throw CompileError("HIP block exceeds 1024 threads");
      threads *= uint64_t(d);
    }
    const Attr *shared = dispatch->attr("shared_memory");
    if (shared && shared->i > int64_t(UINT32_MAX)) throw CompileError("HIP shared-memory bytes exceed the physical launch ABI");
    dispatch->attrs["device"] = Attr::string("rocm:0");
    dispatch->attrs["capabilities"] = Attr::arrayOf({Attr::string("rocm.bare_ptr")});
    const Attr *chosen = selection ? selection->get(symbol) : nullptr;
    if (chosen) {
      const Attr *impl = chosen->get("implementation");
      const Attr *entry = chosen->get("entry_point");
      const Attr *art = chosen->get("artifact");
      if (!impl || !entry || !art) throw CompileError("library selection for " + symbol + " is incomplete");
      dispatch->attrs["artifact"] = *art;
      dispatch->attrs["implementation"] = *impl;
      dispatch->attrs["ckl.hip.entry_point"] = *entry;
      for (const char *key : {"grid", "block", "shared_memory", "constants", "group", "workspace", "partials"})
        if (const Attr *a = chosen->get(key)) dispatch->attrs[std::string("ckl.hip.") + key] = *a;
      if (const Attr *variants = chosen->get("variants")) {
        // Siblings: dispatches of this kernel in the same block whose first operand is the same
        // value (the inferred graph runs them as one shared-operand launch). The variant for the
        // most members not above their count replaces the launch, in every run mode alike.
        int64_t siblings = 0;
        for (auto &op : dispatch->parent->ops)
          if (op->name == "ckl.dispatch" && symbolOf(op.get(), "kernel") == symbol && !op->operands.empty() &&
              !dispatch->operands.empty() && op->operands[0] == dispatch->operands[0])
            ++siblings;
        const Attr *best = nullptr;
        int64_t bestMembers = 0;
        for (const Attr &v : variants->array) {
          const Attr *members = v.get("members");
          if (!members || members->kind != Attr::Int) throw CompileError("library selection variant for " + symbol + " is incomplete");
          if (members->i <= siblings && members->i > bestMembers) {
            best = &v;
            bestMembers = members->i;
          }
        }
        if (best) {
          if (const Attr *e = best->get("entry_point")) dispatch->attrs["ckl.hip.entry_point"] = *e;
          for (const char *key : {"grid", "block", "shared_memory", "constants", "workspace", "partials"})
            if (const Attr *a = best->get(key)) dispatch->attrs[std::string("ckl.hip.") + key] = *a;
        }
      }
    } else {
      dispatch->attrs["artifact"] = Attr::string(artifact);
      dispatch->attrs["implementation"] = Attr::string(artifact + "." + symbol);
    }
  }
  module.op->attrs["ckl.hip.artifact"] = Attr::string(artifact);
  module.op->attrs["ckl.hip.chip"] = Attr::string(options.chip);
  module.op->attrs["ckl.hip.features"] = Attr::string(options.features);
  return artifact;
}

} // namespace ckl
