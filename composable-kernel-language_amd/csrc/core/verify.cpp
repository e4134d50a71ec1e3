#include "verify.h"

#include <set>

namespace ckl {

namespace {

const std::set<std::string> kKnownDialects = {"builtin", "func", "arith", "math", "scf", "cf", "memref", "ckl", "ckl_exec",
                                               "ckl_host"};
const std::set<std::string> kCklOps = {
    "ckl.alloc", "ckl.free", "ckl.view", "ckl.subview", "ckl.load", "ckl.store", "ckl.load_element",
    "ckl.store_element", "ckl.atomic_rmw", "ckl.sync", "ckl.dispatch", "ckl.thread_id", "ckl.block_id",
    "ckl.block_dim", "ckl.grid_dim", "ckl.global_id", "ckl.graph", "ckl.graph_node", "ckl.graph_edge"};
const std::set<std::string> kExecOps = {"ckl_exec.plan", "ckl_exec.heap", "ckl_exec.resource", "ckl_exec.kernel",
                                         "ckl_exec.workspace_heap", "ckl_exec.workspace"};
const std::set<std::string> kHostOps = {"ckl_host.entry", "ckl_host.call"};
const std::set<std::string> kCallbacks = {"ckl_module", "ckl_heap", "ckl_resource", "ckl_kernel", "ckl_argument_resource",
                                          "ckl_argument_value", "ckl_workspace", "ckl_dependency", "ckl_commit"};
const std::set<std::string> kOrderings = {"relaxed", "acquire", "release", "acq_rel", "seq_cst"};
const std::set<std::string> kScopes = {"thread", "block", "device", "system"};

[[noreturn]] void fail(const Op *op, const std::string &message) {
  throw CompileError(sourcePosition(op) + "'" + op->name + "' op " + message);
}

std::string dialectOf(const std::string &name) {
  size_t dot = name.find('.');
  return dot == std::string::npos ? std::string() : name.substr(0, dot);
}

const Op *enclosingFunction(const Op *op) {
  for (const Op *p = op->parentOp(); p; p = p->parentOp())
    if (p->name == "func.func") return p;
  return nullptr;
}

bool isKernelFunction(const Op *function) {
  const Attr *marker = function ? function->attr("ckl.kernel") : nullptr;
  return marker && marker->kind == Attr::Unit;
}

bool numeric(Type::Kind k) {
  return k == Type::F16 || k == Type::F32 || k == Type::F64 || k == Type::I1 || k == Type::I8 || k == Type::I32 ||
         k == Type::I64 || k == Type::Index;
}

const std::string *stringAttr(const Op *op, const char *key) {
  const Attr *a = op->attr(key);
  return a && a->kind == Attr::String ? &a->s : nullptr;
}

std::optional<int64_t> intAttr(const Op *op, const char *key) {
  const Attr *a = op->attr(key);
  if (!a || a->kind != Attr::Int) return std::nullopt;
  return a->i;
}

std::optional<int64_t> constantIndex(const Value *v) {
  if (!v->def || v->def->name != "arith.constant") return std::nullopt;
  const Attr *a = v->def->attr("value");
  if (!a || a->kind != Attr::Int) return std::nullopt;
  return a->i;
}

// Byte size of a static identity-layout memref of byte-sized elements.
std::optional<int64_t> staticBytes(const Type &t) {
  if (!t.isMemRef() || !t.hasStaticShape() || !t.identityLayout) return std::nullopt;
  unsigned width = Type::bitWidth(t.element);
  if (!width || width % 8 || t.element == Type::Index) return std::nullopt;
  return t.elementCount() * int64_t(width / 8);
}

class Verifier {
public:
  Verifier(const Module &module, const VerifyOptions &options) : module(module), options(options) {}

  void run() {
    for (auto &op : module.body()->ops) visit(op.get());
  }

private:
  const Module &module;
  const VerifyOptions &options;

  void visit(const Op *op) {
    const std::string dialect = dialectOf(op->name);
    if (!kKnownDialects.count(dialect)) {
      if (!options.allowUnregisteredDialects)
        fail(op, "belongs to the unregistered dialect '" + dialect +
                     "'; pass --allow-unregistered-dialect to accept operations this build does not know");
    } else if (dialect == "ckl" && !kCklOps.count(op->name)) {
      fail(op, "is not an operation of the ckl dialect");
    } else if (dialect == "ckl_exec" && !kExecOps.count(op->name)) {
      fail(op, "is not an operation of the ckl_exec dialect");
    } else if (dialect == "ckl_host" && !kHostOps.count(op->name)) {
      fail(op, "is not an operation of the ckl_host dialect");
    }
    if (op->attr("ckl.kernel")) kernelAttribute(op);
    const std::string &n = op->name;
    if (n == "ckl.load" || n == "ckl.store") wholeAccess(op);
    else if (n == "ckl.load_element" || n == "ckl.store_element") elementAccess(op);
    else if (n == "ckl.thread_id" || n == "ckl.block_id" || n == "ckl.block_dim" || n == "ckl.grid_dim" || n == "ckl.global_id")
      deviceIndex(op);
    else if (n == "ckl.atomic_rmw") atomic(op);
    else if (n == "ckl.sync") sync(op);
    else if (n == "ckl.alloc") counts(op, 0, 1, true);
    else if (n == "ckl.free") counts(op, 1, 0, true);
    else if (n == "ckl.view") counts(op, 1, 1, true);
    else if (n == "ckl.subview") subview(op);
    else if (n == "ckl.dispatch") dispatch(op);
    else if (n == "ckl.graph") graph(op);
    else if (n == "ckl.graph_node" || n == "ckl.graph_edge") parent(op, "ckl.graph");
    else if (n == "ckl_exec.heap" || n == "ckl_exec.resource" || n == "ckl_exec.kernel" || n == "ckl_exec.workspace_heap" ||
             n == "ckl_exec.workspace")
      parent(op, "ckl_exec.plan");
    else if (n == "ckl_exec.plan") plan(op);
    else if (n == "ckl_host.entry") hostEntry(op);
    else if (n == "ckl_host.call") {
      parent(op, "ckl_host.entry");
      const std::string *callee = stringAttr(op, "callee");
      if (!callee || !kCallbacks.count(*callee)) fail(op, "names no host callback");
    }
    for (auto &region : op->regions)
      for (auto &block : region->blocks)
        for (auto &child : block->ops) visit(child.get());
  }

  // Operand and result counts; `memrefs` requires every memref-position operand/result to be one.
  void counts(const Op *op, size_t operands, size_t results, bool memrefs) {
    if (op->operands.size() != operands || op->results.size() != results)
      fail(op, "expects " + std::to_string(operands) + " operand(s) and " + std::to_string(results) + " result(s)");
    if (!memrefs) return;
    for (const Value *v : op->operands)
      if (!v->type.isMemRef()) fail(op, "requires memref operands");
    for (auto &r : op->results)
      if (!r->type.isMemRef()) fail(op, "requires a memref result");
  }

  void parent(const Op *op, const char *expected) {
    const Op *p = op->parentOp();
    if (!p || p->name != expected) fail(op, std::string("expects parent op '") + expected + "'");
  }

  void kernelAttribute(const Op *op) {
    const Attr *marker = op->attr("ckl.kernel");
    if (op->name != "func.func" || marker->kind != Attr::Unit) fail(op, "ckl.kernel requires a unit attribute on func.func");
    const Attr *results = op->attr("ckl.num_results");
    if (op->isDeclaration() || (results && results->i != 0)) fail(op, "ckl.kernel requires a defined function with no results");
    for (auto &arg : op->entry()->args) {
      const Type &t = arg->type;
      bool ok = t.isMemRef() ? !t.unranked && numeric(t.element) : numeric(t.kind);
      if (!ok) fail(op, "ckl.kernel arguments must be numeric scalars or ranked numeric memrefs");
    }
  }

  void kernelContext(const Op *op) {
    if (!isKernelFunction(enclosingFunction(op))) fail(op, "requires an enclosing func.func marked ckl.kernel");
  }

  void wholeAccess(const Op *op) {
    bool load = op->name == "ckl.load";
    counts(op, load ? 1 : 2, load ? 1 : 0, false);
    const Value *resource = op->operands[load ? 0 : 1];
    if (!resource->type.isMemRef()) fail(op, "requires a memref resource");
    const Type &value = load ? op->results[0]->type : op->operands[0]->type;
    if (value != Type::scalar(resource->type.element))
      fail(op, load ? "result type must match the resource element type" : "value type must match the resource element type");
  }

  void elementAccess(const Op *op) {
    bool load = op->name == "ckl.load_element";
    size_t first = load ? 1 : 2;
    if (op->operands.size() < first || op->results.size() != (load ? 1u : 0u))
      fail(op, load ? "expects a resource, its indices and one result" : "expects a value, a resource and its indices");
    kernelContext(op);
    const Type &buffer = op->operands[first - 1]->type;
    if (!buffer.isMemRef()) fail(op, "requires a memref resource");
    size_t indices = op->operands.size() - first;
    if (buffer.unranked || indices != buffer.shape.size()) fail(op, "requires one index per buffer dimension");
    const Type &value = load ? op->results[0]->type : op->operands[0]->type;
    if (value != Type::scalar(buffer.element)) fail(op, "value type must match the buffer element type");
    if (!numeric(buffer.element)) fail(op, "requires a numeric buffer element type");
    for (size_t axis = 0; axis < indices; ++axis) {
      const Value *index = op->operands[first + axis];
      if (index->type.kind != Type::Index) fail(op, "requires index-typed indices");
      auto constant = constantIndex(index);
      if (constant && (*constant < 0 || (buffer.shape[axis] >= 0 && *constant >= buffer.shape[axis])))
        fail(op, "constant index is out of bounds for dimension " + std::to_string(axis));
    }
  }

  void deviceIndex(const Op *op) {
    counts(op, 0, 1, false);
    kernelContext(op);
    auto axis = intAttr(op, "axis");
    if (!axis || *axis < 0 || *axis > 2) fail(op, "requires axis 0, 1, or 2");
    if (op->results[0]->type.kind != Type::Index) fail(op, "requires an index result");
  }

  void scope(const Op *op) {
    const std::string *s = stringAttr(op, "scope");
    if (!s || !kScopes.count(*s)) fail(op, "has unsupported ordering scope '" + (s ? *s : std::string()) + "'");
  }

  void atomic(const Op *op) {
    counts(op, 2, 1, false);
    const Type &buffer = op->operands[1]->type;
    if (!buffer.isMemRef()) fail(op, "requires a memref resource");
    Type element = Type::scalar(buffer.element);
    if (op->operands[0]->type != element || op->results[0]->type != element)
      fail(op, "value and result types must match the resource element type");
    const std::string *ordering = stringAttr(op, "ordering");
    if (!ordering || !kOrderings.count(*ordering))
      fail(op, "has unsupported atomic ordering '" + (ordering ? *ordering : std::string()) + "'");
    scope(op);
  }

  void sync(const Op *op) {
    if (!op->results.empty()) fail(op, "has no results");
    for (const Value *v : op->operands)
      if (!v->type.isMemRef()) fail(op, "requires memref operands");
    scope(op);
  }

  void subview(const Op *op) {
    counts(op, 1, 1, true);
    const Type &source = op->operands[0]->type, &result = op->results[0]->type;
    auto sourceBytes = staticBytes(source), resultBytes = staticBytes(result);
    if (!sourceBytes || !resultBytes || source.element != result.element || source.memorySpace != result.memorySpace)
      fail(op, "requires static contiguous source/result with matching element type and memory space");
    auto offset = intAttr(op, "offset");
    int64_t element = Type::bitWidth(source.element) / 8;
    if (!offset || *offset < 0 || *resultBytes <= 0 || *offset > *sourceBytes / element ||
        *resultBytes > *sourceBytes - *offset * element)
      fail(op, "subview is out of bounds or empty");
  }

  void dimensions(const Op *op, const char *key, const char *what) {
    const Attr *a = op->attr(key);
    if (!a || a->kind != Attr::DenseI64 || a->dense.size() != 3)
      fail(op, std::string("requires exactly three ") + what + " dimensions");
    for (int64_t d : a->dense)
      if (d <= 0) fail(op, std::string("requires positive ") + what + " dimensions");
  }

  void dispatch(const Op *op) {
    if (isKernelFunction(enclosingFunction(op))) fail(op, "cannot launch a kernel from a ckl.kernel body");
    dimensions(op, "grid", "grid");
    dimensions(op, "block", "block");
    auto shared = intAttr(op, "shared_memory");
    if (!shared) fail(op, "requires attribute 'shared_memory'");
    if (*shared < 0) fail(op, "requires non-negative shared memory");
    const std::string *implementation = stringAttr(op, "implementation");
    if (!implementation || implementation->empty()) fail(op, "requires a stable implementation identity");
    if (!stringAttr(op, "device")) fail(op, "requires attribute 'device'");
    const Attr *capabilities = op->attr("capabilities");
    if (!capabilities || capabilities->kind != Attr::Array) fail(op, "requires attribute 'capabilities'");
    for (const Attr &c : capabilities->array)
      if (c.kind != Attr::String) fail(op, "requires string capabilities");
    const Attr *segments = op->attr("operandSegmentSizes");
    if (!segments || segments->kind != Attr::DenseI32 || segments->dense.size() != 2 || segments->dense[0] < 0 ||
        segments->dense[1] < 0 || size_t(segments->dense[0] + segments->dense[1]) != op->operands.size())
      fail(op, "requires operandSegmentSizes with two entries that sum to its operand count");
    size_t arguments = size_t(segments->dense[0]);
    for (size_t k = arguments; k < op->operands.size(); ++k)
      if (op->operands[k]->type.kind != Type::Token) fail(op, "dependencies must be !ckl.token values");
    if (op->results.size() != 1 || op->results[0]->type.kind != Type::Token) fail(op, "returns one !ckl.token");
    const Attr *kernel = op->attr("kernel");
    if (!kernel || kernel->kind != Attr::Symbol) fail(op, "requires a kernel symbol");
    const Op *callee = kernel->nested.empty() ? module.lookup(kernel->s) : nullptr;
    if (!callee || callee->name != "func.func") fail(op, "references unknown kernel " + kernel->str());
    const Attr *results = callee->attr("ckl.num_results");
    if (results && results->i != 0) fail(op, "referenced kernel must have no results");
    std::vector<Type> formals;
    if (Block *entry = callee->entry()) {
      for (auto &arg : entry->args) formals.push_back(arg->type);
    } else if (const Attr *types = callee->attr("ckl.argument_types")) {
      for (const Attr &t : types->array) formals.push_back(t.type);
    }
    if (formals.size() != arguments)
      fail(op, "passes " + std::to_string(arguments) + " arguments to a kernel with " + std::to_string(formals.size()) +
                   " parameters");
    for (size_t k = 0; k < arguments; ++k)
      if (op->operands[k]->type != formals[k]) fail(op, "argument type does not match referenced kernel");
  }

  void graph(const Op *op) {
    const Attr *source = op->attr("source");
    const Op *function = source && source->kind == Attr::Symbol && source->nested.empty() ? module.lookup(source->s) : nullptr;
    if (!function || function->name != "func.func")
      fail(op, "references unknown source function " + (source ? source->str() : std::string("<none>")));
    if (op->regions.size() != 1 || op->regions[0]->blocks.size() != 1) fail(op, "requires a graph body block");
    std::set<int64_t> nodes;
    for (auto &child : op->regions[0]->blocks[0]->ops) {
      if (child->name == "ckl.graph_node") {
        auto id = intAttr(child.get(), "id");
        if (!id || !nodes.insert(*id).second) fail(child.get(), "has a duplicate node id");
      } else if (child->name != "ckl.graph_edge") {
        fail(child.get(), "is not a graph node or edge");
      }
    }
    for (auto &child : op->regions[0]->blocks[0]->ops) {
      if (child->name != "ckl.graph_edge") continue;
      auto from = intAttr(child.get(), "from"), to = intAttr(child.get(), "to");
      if (!from || !to || !nodes.count(*from) || !nodes.count(*to)) fail(child.get(), "references an unknown graph node");
      if (*from >= *to) fail(child.get(), "must preserve source program order");
      const Attr *reasons = child->attr("reasons");
      if (!reasons || reasons->kind != Attr::Array || reasons->array.empty())
        fail(child.get(), "requires at least one provenance reason");
    }
  }

  void plan(const Op *op);

  void hostEntry(const Op *op) {
    if (op->parentOp() != module.op.get()) fail(op, "must be at module level");
    if (op->regions.size() != 1 || op->regions[0]->blocks.size() != 1) fail(op, "requires a body block");
    const Attr *arguments = op->attr("arguments");
    if (!arguments || arguments->kind != Attr::Array || !stringAttr(op, "name") || !stringAttr(op, "source"))
      fail(op, "requires a name, a source and argument types");
    for (auto &child : op->regions[0]->blocks[0]->ops)
      if (child->name != "ckl_host.call") fail(child.get(), "is not a host callback");
  }
};

// ------------------------------------------------------------------ textual executable plans

const Attr &required(const Op *op, const char *key, Attr::Kind kind, const char *message) {
  const Attr *a = op->attr(key);
  if (!a || a->kind != kind) fail(op, message);
  return *a;
}

ExecArgument readArgument(const Op *kernel, const Attr &descriptor) {
  if (descriptor.kind != Attr::Dict) fail(kernel, "requires dictionary argument descriptors");
  const Attr *slot = descriptor.get("slot"), *logical = descriptor.get("logical_index");
  const Attr *kind = descriptor.get("kind"), *type = descriptor.get("type");
  if (!slot || slot->kind != Attr::Int || slot->i < 0 || !logical || logical->kind != Attr::Int || logical->i < 0 ||
      !kind || kind->kind != Attr::String || !type || type->kind != Attr::TypeAttr)
    fail(kernel, "argument descriptor requires non-negative slot and logical index plus a type");
  ExecArgument a;
  a.slot = slot->i;
  a.logicalIndex = logical->i;
  a.kind = kind->s;
  a.type = type->type;
  auto text = [&](const char *key) {
    const Attr *v = descriptor.get(key);
    return v && v->kind == Attr::String ? v->s : std::string();
  };
  if (a.kind == "resource") {
    a.resource = text("resource");
    a.packing = text("packing");
    const Attr *offset = descriptor.get("byte_offset"), *length = descriptor.get("byte_length");
    if (offset || length) {
      if (!offset || !length || offset->kind != Attr::Int || length->kind != Attr::Int)
        fail(kernel, "invalid or out-of-bounds resource byte range");
      a.byteOffset = offset->i;
      a.byteLength = length->i;
      if (a.byteLength < 0) fail(kernel, "invalid or out-of-bounds resource byte range");
    }
  } else if (a.kind == "scalar") {
    a.name = text("name");
  } else if (a.kind == "constant") {
    const Attr *value = descriptor.get("value");
    if (!value || (value->kind != Attr::Int && value->kind != Attr::Float) || value->type != a.type)
      fail(kernel, "constant argument requires a value matching its type");
    a.value = *value;
    try {
      a.bytes = constantBytes(*value, a.type);
    } catch (const CompileError &) {
      fail(kernel, "constant argument requires a byte-sized scalar type of at most 64 bits");
    }
  } else if (a.kind == "bytes") {
    const Attr *value = descriptor.get("value");
    const Type &t = a.type;
    if (!value || value->kind != Attr::DenseI8 || value->dense.empty() || t.kind != Type::Vector || t.shape.size() != 1 ||
        t.element != Type::I8 || int64_t(value->dense.size()) != t.shape[0])
      fail(kernel, "bytes argument requires a non-empty vector<Nxi8> type and N byte values");
    a.value = *value;
    for (int64_t b : value->dense) a.bytes.push_back(uint8_t(b));
  } else {
    fail(kernel, "contains an unsupported physical argument kind");
  }
  return a;
}

ExecPlan readPlan(const Module &module, const Op *op) {
  ExecPlan plan;
  const std::string *name = stringAttr(op, "name"), *backend = stringAttr(op, "backend");
  if (!name || !backend || name->empty() || backend->empty()) fail(op, "requires plan and backend identities");
  plan.name = *name;
  plan.backend = *backend;
  const Attr *source = op->attr("source");
  if (!source || source->kind != Attr::Symbol) fail(op, "requires a source function symbol");
  plan.source = source->s;
  if (const Op *function = source->nested.empty() ? module.lookup(source->s) : nullptr) {
    if (Block *entry = function->entry()) {
      for (auto &arg : entry->args) plan.sourceArguments.push_back(arg->type);
    } else if (const Attr *types = function->attr("ckl.argument_types")) {
      for (const Attr &t : types->array) plan.sourceArguments.push_back(t.type);
    }
  }
  if (op->regions.size() != 1 || op->regions[0]->blocks.size() != 1) fail(op, "requires a body block");
  for (auto &child : op->regions[0]->blocks[0]->ops) {
    const Op *c = child.get();
    if (c->name == "ckl_exec.heap") {
      ExecHeap h;
      h.id = required(c, "id", Attr::Int, "requires a non-negative id and positive byte size").i;
      h.bytes = required(c, "bytes", Attr::Int, "requires a non-negative id and positive byte size").i;
      h.alignment = required(c, "alignment", Attr::Int, "requires power-of-two alignment").i;
      h.device = required(c, "device", Attr::Int, "requires a non-negative device ordinal").i;
      if (h.device < 0) fail(c, "requires a non-negative device ordinal");
      h.addressSpace = stringAttr(c, "address_space") ? *stringAttr(c, "address_space") : "global";
      plan.heaps.push_back(h);
    } else if (c->name == "ckl_exec.resource") {
      ExecResource r;
      r.name = stringAttr(c, "name") ? *stringAttr(c, "name") : std::string();
      r.kind = stringAttr(c, "kind") ? *stringAttr(c, "kind") : std::string();
      r.device = stringAttr(c, "device") ? *stringAttr(c, "device") : std::string();
      r.addressSpace = stringAttr(c, "address_space") ? *stringAttr(c, "address_space") : "global";
      r.alignment = required(c, "alignment", Attr::Int, "requires power-of-two alignment").i;
      if (r.alignment <= 0 || (r.alignment & (r.alignment - 1))) fail(c, "requires power-of-two alignment");
      auto bytes = intAttr(c, "bytes"), heap = intAttr(c, "heap"), offset = intAttr(c, "offset");
      r.bytes = bytes ? *bytes : 0;
      if (r.kind == "temporary") {
        if (!bytes || !heap || !offset) fail(c, "temporary resource requires bytes, heap, and offset");
        r.heap = *heap;
        r.offset = *offset;
      } else if (heap || offset) {
        fail(c, "external resource cannot have a heap placement");
      } else if (r.name.size() > 3 && r.name.rfind("arg", 0) == 0 &&
                 r.name.find_first_not_of("0123456789", 3) == std::string::npos) {
        r.argument = std::stoll(r.name.substr(3));   // bound to host argument N, as the lowering names it
      }
      plan.resources.push_back(r);
    } else if (c->name == "ckl_exec.workspace_heap") {
      ExecHeap h;
      h.id = required(c, "id", Attr::Int, "requires an id and positive byte size").i;
      h.bytes = required(c, "bytes", Attr::Int, "requires an id and positive byte size").i;
      h.alignment = required(c, "alignment", Attr::Int, "requires power-of-two alignment").i;
      h.device = required(c, "device", Attr::Int, "requires a non-negative device ordinal").i;
      if (h.device < 0) fail(c, "requires a non-negative device ordinal");
      h.addressSpace = "global";
      plan.workspaceHeaps.push_back(h);
    } else if (c->name == "ckl_exec.workspace") {
      ExecWorkspace w;
      w.name = stringAttr(c, "name") ? *stringAttr(c, "name") : std::string();
      w.role = stringAttr(c, "role") ? *stringAttr(c, "role") : std::string();
      w.kernel = required(c, "kernel", Attr::Int, "requires kernel, heap, offset and bytes").i;
      w.heap = required(c, "heap", Attr::Int, "requires kernel, heap, offset and bytes").i;
      w.offset = required(c, "offset", Attr::Int, "requires kernel, heap, offset and bytes").i;
      w.bytes = required(c, "bytes", Attr::Int, "requires kernel, heap, offset and bytes").i;
      plan.workspaces.push_back(w);
    } else if (c->name == "ckl_exec.kernel") {
      ExecKernel k;
      k.id = required(c, "id", Attr::Int, "requires a non-negative id").i;
      if (k.id < 0) fail(c, "requires a non-negative id");
      const Attr *kernel = c->attr("kernel");
      if (kernel && kernel->kind == Attr::Symbol) {
        k.kernel = kernel->s;
        for (const std::string &n : kernel->nested) k.kernel += "::" + n;
      }
      for (auto [key, field] : {std::pair<const char *, std::string *>{"implementation", &k.implementation},
                                {"artifact", &k.artifact}, {"abi", &k.abi}, {"device", &k.device}})
        if (const std::string *v = stringAttr(c, key)) *field = *v;
      k.function = stringAttr(c, "entry_point") ? *stringAttr(c, "entry_point") : k.kernel;
      for (auto [key, what] : {std::pair<const char *, const char *>{"grid", "grid"}, {"block", "block"}}) {
        const Attr *dims = c->attr(key);
        if (!dims || dims->kind != Attr::DenseI64 || dims->dense.size() != 3)
          fail(c, std::string("requires exactly three ") + what + " dimensions");
        for (int64_t d : dims->dense)
          if (d <= 0) fail(c, std::string("requires positive ") + what + " dimensions");
      }
      k.grid = c->attr("grid")->dense;
      k.block = c->attr("block")->dense;
      k.logicalGrid = c->attr("logical_grid") ? c->attr("logical_grid")->dense : k.grid;
      k.logicalBlock = c->attr("logical_block") ? c->attr("logical_block")->dense : k.block;
      auto shared = intAttr(c, "shared_memory");
      if (!shared || *shared < 0) fail(c, "requires non-negative shared memory");
      k.sharedMemory = *shared;
      if (const std::string *group = stringAttr(c, "group")) k.group = *group;
      if (auto workspace = intAttr(c, "workspace")) k.workspace = *workspace;
      if (auto partials = intAttr(c, "partials")) k.partials = *partials;
      const Attr *dependencies = c->attr("dependencies");
      if (!dependencies || dependencies->kind != Attr::DenseI64) fail(c, "requires a dependencies array");
      k.dependencies = dependencies->dense;
      const Attr *arguments = c->attr("arguments");
      if (!arguments || arguments->kind != Attr::Array) fail(c, "requires dictionary argument descriptors");
      for (const Attr &descriptor : arguments->array) k.arguments.push_back(readArgument(c, descriptor));
      plan.kernels.push_back(std::move(k));
    } else {
      fail(c, "is not an executable-plan operation");
    }
  }
  try {
    plan.verify();
  } catch (const CompileError &error) {
    throw CompileError(sourcePosition(op) + error.what());
  }
  return plan;
}

void Verifier::plan(const Op *op) { readPlan(module, op); }

} // namespace

void verifyModule(const Module &module, const VerifyOptions &options) { Verifier(module, options).run(); }

std::vector<ExecPlan> readExecPlans(const Module &module) {
  std::vector<ExecPlan> plans;
  for (auto &op : module.body()->ops)
    if (op->name == "ckl_exec.plan") plans.push_back(readPlan(module, op.get()));
  return plans;
}

} // namespace ckl
