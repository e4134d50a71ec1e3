// Guarded unary pointwise fusion (the reference's ckl-fuse-pointwise pass,
// lib/Transforms/PointwiseFusion.cpp:30-304), over this build's IR.
//
// Two adjacent dispatches (only allocations or constants between them) are merged into one
// kernel when both kernels are "guarded unary pointwise": one x index, one full bounds guard
// `i < N` (slt or ult) over rank-1 static buffers of N elements, exactly one input and one
// output buffer accessed at index i, a final store, and pure arithmetic without fast-math flags;
// when both launches have the same one-dimensional geometry, no shared memory and no explicit
// token dependencies; and when the producer's output is a temporary allocated in the host block
// whose only other uses are the consumer's input and one later free. The fused kernel keeps the
// intermediate in a register (rounded exactly as the materialised store would be: the device
// code generator never contracts across it), drops the temporary, and is named by a digest of its
// text. The module is marked `ckl.fusion.requires_disjoint`: fusing assumed the external buffers
// do not overlap, so binding falls back to the unfused program when they do.
#include "analysis.h"
#include "sha256.h"

#include <algorithm>
#include <optional>

namespace ckl {
namespace {

constexpr int64_t kSlt = 2, kUlt = 6;   // arith.cmpi predicate codes

struct Pointwise {
  Op *function = nullptr;
  Value *index = nullptr;   // the x global id
  Op *guard = nullptr;      // scf.if (i < N)
  Op *store = nullptr;      // the final ckl.store_element
  unsigned input = 0, output = 0;
  int64_t count = 0;
  int64_t predicate = 0;
};

bool entryArgument(const Op *function, const Value *value, unsigned &index) {
  if (!value || value->def || value->owner != function->entry()) return false;
  index = value->index;
  return true;
}

const Op *definingOp(const Value *value) { return value ? value->def : nullptr; }

// Dispatch operands: the kernel arguments, then explicit token dependencies (operandSegmentSizes).
size_t argumentCount(const Op *op) {
  const Attr *segments = op->attr("operandSegmentSizes");
  size_t count = segments && !segments->dense.empty() ? size_t(segments->dense[0]) : op->operands.size();
  return std::min(count, op->operands.size());
}
std::vector<Value *> dispatchArguments(const Op *op) {
  return std::vector<Value *>(op->operands.begin(), op->operands.begin() + std::ptrdiff_t(argumentCount(op)));
}
bool hasDependencies(const Op *op) { return argumentCount(op) < op->operands.size(); }

std::string symbolOf(const Op *op, const char *key) {
  const Attr *a = op->attr(key);
  return a && a->kind == Attr::Symbol && a->nested.empty() ? a->s : std::string();
}

bool hasFastMath(const Op &op) {
  const Attr *flags = op.attr("fastmath");
  if (!flags) return false;
  std::string text = flags->str();
  return text.find("none") == std::string::npos;
}

std::optional<Pointwise> recognize(Op *function) {
  if (!function || !function->attr("ckl.kernel") || function->isDeclaration() ||
      function->regions[0]->blocks.size() != 1)
    return {};
  if (const Attr *results = function->attr("ckl.num_results"); results && results->i) return {};
  Pointwise p;
  p.function = function;
  Block *entry = function->entry();
  unsigned buffers = 0;
  for (auto &arg : entry->args) {
    const Type &t = arg->type;
    if (!t.isMemRef()) continue;
    if (t.unranked || t.shape.size() != 1 || !t.hasStaticShape() || !t.identityLayout || !t.memorySpace.empty())
      return {};
    if (buffers && p.count != t.shape[0]) return {};
    p.count = t.shape[0];
    ++buffers;
  }
  if (buffers != 2 || p.count <= 0) return {};
  for (auto &op : entry->ops) {
    if (op->name == "ckl.global_id") {
      const Attr *axis = op->attr("axis");
      if (p.index || (axis && axis->i != 0)) return {};
      p.index = op->result();
    } else if (op->name == "scf.if") {
      if (p.guard || !op->results.empty() || op->regions.empty() || op->regions[0]->blocks.size() != 1) return {};
      for (size_t r = 1; r < op->regions.size(); ++r)
        for (auto &block : op->regions[r]->blocks)
          if (!block->ops.empty()) return {};
      p.guard = op.get();
    } else if (op->name != "arith.constant" && op->name != "arith.cmpi" && op->name != "func.return") {
      return {};
    }
  }
  if (!p.index || !p.guard || p.guard->operands.size() != 1) return {};
  const Op *compare = definingOp(p.guard->operands[0]);
  if (!compare || compare->name != "arith.cmpi" || compare->operands.size() != 2 || compare->operands[0] != p.index)
    return {};
  const Attr *predicate = compare->attr("predicate");
  if (!predicate || (predicate->i != kSlt && predicate->i != kUlt)) return {};
  const Op *bound = definingOp(compare->operands[1]);
  const Attr *value = bound && bound->name == "arith.constant" ? bound->attr("value") : nullptr;
  if (!value || value->kind != Attr::Int || value->i != p.count) return {};
  p.predicate = predicate->i;

  std::optional<unsigned> input;
  auto &body = p.guard->regions[0]->blocks[0]->ops;
  for (size_t k = 0; k < body.size(); ++k) {
    const Op &op = *body[k];
    if (op.name == "ckl.load_element") {
      unsigned arg = 0;
      if (op.operands.size() != 2 || !entryArgument(function, op.operands[0], arg) || op.operands[1] != p.index) return {};
      if (input && *input != arg) return {};
      input = arg;
    } else if (op.name == "ckl.store_element") {
      unsigned arg = 0;
      if (p.store || op.operands.size() != 3 || !entryArgument(function, op.operands[1], arg) ||
          op.operands[2] != p.index || k + 1 >= body.size() || body[k + 1]->name != "scf.yield")
        return {};
      p.store = body[k].get();
      p.output = arg;
    } else if (op.name == "scf.yield") {
      continue;
    } else if (op.name.rfind("arith.", 0) != 0 || !op.regions.empty()) {
      return {};
    }
    if (hasFastMath(op)) return {};
  }
  if (!input || !p.store || *input == p.output || entry->args[*input]->type != entry->args[p.output]->type) return {};
  p.input = *input;
  return p;
}

bool sameLaunch(const Op &a, const Op &b) {
  auto same = [&](const char *key) {
    const Attr *x = a.attr(key), *y = b.attr(key);
    return (!x && !y) || (x && y && *x == *y);
  };
  auto sharedBytes = [](const Op &op) { const Attr *s = op.attr("shared_memory"); return s ? s->i : 0; };
  auto unitY = [](const Attr *dims) { return dims && dims->dense.size() == 3 && dims->dense[1] == 1 && dims->dense[2] == 1; };
  return same("device") && same("grid") && same("block") && same("capabilities") && sharedBytes(a) == 0 &&
         sharedBytes(b) == 0 && unitY(a.attr("grid")) && unitY(a.attr("block")) && !hasDependencies(&a) &&
         !hasDependencies(&b);
}

// Every operand use of `value` under `root` (ops of nested regions included).
void collectUses(Op *root, const Value *value, std::vector<std::pair<Op *, size_t>> &uses) {
  walkPreOrder(root, [&](Op *op) {
    for (size_t k = 0; k < op->operands.size(); ++k)
      if (op->operands[k] == value) uses.emplace_back(op, k);
  });
}

size_t position(const Block *block, const Op *op) {
  for (size_t k = 0; k < block->ops.size(); ++k)
    if (block->ops[k].get() == op) return k;
  return block->ops.size();
}

void eraseOp(Block *block, const Op *op) {
  block->ops.erase(block->ops.begin() + std::ptrdiff_t(position(block, op)));
}

int64_t fusedSteps(const Op *function) {
  const Attr *steps = function->attr("ckl.fused_steps");
  return steps ? steps->i : 1;
}

bool fuse(Module &module, Op *host, Op *first, Op *second) {
  if (!sameLaunch(*first, *second)) return false;
  Block *block = host->entry();
  for (Op *dispatch : {first, second}) {
    std::vector<std::pair<Op *, size_t>> uses;
    for (auto &result : dispatch->results) collectUses(host, result.get(), uses);
    if (!uses.empty()) return false;   // an explicit token still orders something
  }
  auto producer = recognize(module.lookup(symbolOf(first, "kernel")));
  auto consumer = recognize(module.lookup(symbolOf(second, "kernel")));
  if (!producer || !consumer || producer->predicate != consumer->predicate || producer->count != consumer->count)
    return false;
  std::vector<Value *> firstArgs = dispatchArguments(first), secondArgs = dispatchArguments(second);
  if (producer->output >= firstArgs.size() || consumer->input >= secondArgs.size()) return false;
  Value *temporary = firstArgs[producer->output];
  Op *allocation = temporary->def;
  if (!allocation || allocation->name != "ckl.alloc" || allocation->parent != block || secondArgs[consumer->input] != temporary)
    return false;
  std::vector<std::pair<Op *, size_t>> uses;
  collectUses(host, temporary, uses);
  Op *release = nullptr;
  unsigned producers = 0, consumers = 0;
  for (auto &[op, operand] : uses) {
    if (op == first && operand == producer->output) ++producers;
    else if (op == second && operand == consumer->input) ++consumers;
    else if (op->name == "ckl.free" && !release && op->parent == block && position(block, second) < position(block, op))
      release = op;
    else
      return false;   // escapes, views, a second reader or writer
  }
  if (producers != 1 || consumers != 1 || !release) return false;

  // The fused signature keeps every binding except the temporary, equal actuals merged.
  std::vector<Value *> actuals;
  auto add = [&](Value *actual) {
    auto found = std::find(actuals.begin(), actuals.end(), actual);
    if (found != actuals.end()) return unsigned(found - actuals.begin());
    actuals.push_back(actual);
    return unsigned(actuals.size() - 1);
  };
  constexpr unsigned kDropped = ~0u;
  std::vector<unsigned> producerArgs, consumerArgs;
  for (size_t k = 0; k < firstArgs.size(); ++k) producerArgs.push_back(k == producer->output ? kDropped : add(firstArgs[k]));
  for (size_t k = 0; k < secondArgs.size(); ++k) consumerArgs.push_back(k == consumer->input ? kDropped : add(secondArgs[k]));
  // Equal input and output actuals would collapse the two-buffer form; keep the launches.
  if (actuals[producerArgs[producer->input]] == actuals[consumerArgs[consumer->output]]) return false;

  auto function = std::make_unique<Op>();
  function->name = "func.func";
  function->loc = producer->function->loc;
  function->attrs["sym_name"] = Attr::string("__ckl_fused");
  function->attrs["ckl.kernel"] = Attr::unit();
  function->attrs["ckl.num_results"] = Attr::integer(0);
  function->attrs["ckl.fused_steps"] = Attr::integer(fusedSteps(producer->function) + fusedSteps(consumer->function));
  Attr signature;
  signature.kind = Attr::TypeAttr;
  signature.type.kind = Type::Opaque;
  signature.type.text = "(";
  for (size_t k = 0; k < actuals.size(); ++k) signature.type.text += (k ? ", " : "") + actuals[k]->type.str();
  signature.type.text += ") -> ()";
  function->attrs["function_type"] = signature;
  auto region = std::make_unique<Region>();
  region->parent = function.get();
  auto entryBlock = std::make_unique<Block>();
  entryBlock->parent = region.get();
  for (size_t k = 0; k < actuals.size(); ++k) {
    auto arg = std::make_unique<Value>();
    arg->type = actuals[k]->type;
    arg->owner = entryBlock.get();
    arg->index = unsigned(k);
    entryBlock->args.push_back(std::move(arg));
  }
  Block *entry = entryBlock.get();
  region->blocks.push_back(std::move(entryBlock));
  function->regions.push_back(std::move(region));

  ValueMap pm, cm;
  Block *producerEntry = producer->function->entry(), *consumerEntry = consumer->function->entry();
  for (size_t k = 0; k < producerArgs.size(); ++k)
    if (producerArgs[k] != kDropped) pm[producerEntry->args[k].get()] = entry->args[producerArgs[k]].get();
  for (size_t k = 0; k < consumerArgs.size(); ++k)
    if (consumerArgs[k] != kDropped) cm[consumerEntry->args[k].get()] = entry->args[consumerArgs[k]].get();
  for (auto &op : producerEntry->ops)
    if (op.get() != producer->guard && op->name != "func.return") entry->ops.push_back(cloneOp(*op, entry, pm));
  cm[consumer->index] = pm.at(producer->index);
  for (auto &op : consumerEntry->ops)
    if (op.get() != consumer->guard && op->name != "func.return" && op->name != "ckl.global_id")
      entry->ops.push_back(cloneOp(*op, entry, cm));
  // The guard: the producer's body without its store, then the consumer's body reading the
  // producer's stored value instead of loading the temporary.
  std::unique_ptr<Op> guard = cloneOp(*producer->guard, entry, pm);
  Block *then = guard->regions[0]->blocks[0].get();
  then->ops.clear();
  std::unique_ptr<Op> yield;
  for (auto &op : producer->guard->regions[0]->blocks[0]->ops) {
    if (op->name == "scf.yield") { yield = cloneOp(*op, then, pm); continue; }
    if (op.get() == producer->store) continue;
    then->ops.push_back(cloneOp(*op, then, pm));
  }
  Value *intermediate = pm.at(producer->store->operands[0]);
  for (auto &op : consumer->guard->regions[0]->blocks[0]->ops) {
    if (op->name == "ckl.load_element") cm[op->result()] = intermediate;
    else if (op->name != "scf.yield") then->ops.push_back(cloneOp(*op, then, cm));
  }
  then->ops.push_back(std::move(yield));
  entry->ops.push_back(std::move(guard));
  for (auto &op : consumerEntry->ops)
    if (op->name == "func.return") { entry->ops.push_back(cloneOp(*op, entry, cm)); break; }

  std::string symbol = "kernel_fused_" + Sha256::of(printOp(*function)).substr(0, 24);
  std::string name = symbol;
  for (unsigned suffix = 0; module.lookup(name); ++suffix) name = symbol + "_" + std::to_string(suffix);
  function->attrs["sym_name"] = Attr::string(name);
  Block *moduleBody = module.body();
  function->parent = moduleBody;
  moduleBody->ops.push_back(std::move(function));

  ValueMap none;
  std::unique_ptr<Op> fused = cloneOp(*second, block, none);
  fused->operands = actuals;
  fused->attrs["operandSegmentSizes"] = Attr::denseI32({int64_t(actuals.size()), 0});
  fused->attrs["kernel"] = Attr::symbol(name);
  fused->attrs["implementation"] = Attr::string(name);
  fused->attrs.erase("artifact");
  size_t at = position(block, second);
  block->ops.insert(block->ops.begin() + std::ptrdiff_t(at), std::move(fused));
  eraseOp(block, first);
  eraseOp(block, second);
  eraseOp(block, release);
  eraseOp(block, allocation);
  return true;
}

bool referenced(const Module &module, const std::string &symbol) {
  bool found = false;
  walkPreOrder(module.op.get(), [&](Op *op) {
    for (const char *key : {"kernel", "callee"})
      if (symbolOf(op, key) == symbol) found = true;
  });
  return found;
}

} // namespace

bool fusePointwise(Module &module) {
  if (module.op->attr("ckl.hip.artifact")) throw CompileError("pointwise fusion must run before HIP preparation");
  bool changed = false, again = true;
  while (again) {
    again = false;
    for (Op *host : module.functions()) {
      if (host->attr("ckl.kernel") || host->isDeclaration() || host->regions[0]->blocks.size() != 1) continue;
      Op *previous = nullptr;
      for (auto &op : host->entry()->ops) {
        if (op->name == "ckl.dispatch") {
          if (previous && fuse(module, host, previous, op.get())) {
            again = changed = true;
            break;
          }
          previous = op.get();
        } else if (op->name != "ckl.alloc" && op->name != "arith.constant") {
          previous = nullptr;
        }
      }
      if (again) break;
    }
  }
  if (changed) {
    module.op->attrs["ckl.fusion.requires_disjoint"] = Attr::unit();
    Block *body = module.body();
    for (size_t k = 0; k < body->ops.size();) {
      Op *function = body->ops[k].get();
      function->attrs.erase("ckl.effect_summary");
      if (function->name == "func.func" && function->attr("ckl.kernel") && !referenced(module, function->symName()))
        body->ops.erase(body->ops.begin() + std::ptrdiff_t(k));
      else
        ++k;
    }
  }
  return changed;
}

} // namespace ckl
