#include "compiler.h"
#include "verify.h"

#include "../runtime/callbacks.h"

#include <cstdio>
#include <set>
#include <sstream>

namespace ckl {

const Artifact *CompiledProgram::artifact(const std::string &identity) const {
  for (const Artifact &a : artifacts)
    if (a.identity == identity) return &a;
  return nullptr;
}

namespace {

std::string withPlan(const std::string &moduleText, const std::string &extra) {
  // Insert the extra top-level ops before the module's closing brace.
  size_t end = moduleText.rfind('}');
  if (end == std::string::npos) return moduleText + extra;
  return moduleText.substr(0, end) + extra + moduleText.substr(end);
}

std::string hexBytes(const void *data, size_t size) {
  std::string out;
  const uint8_t *p = static_cast<const uint8_t *>(data);
  char buf[4];
  for (size_t k = 0; k < size; ++k) {
    std::snprintf(buf, sizeof buf, k ? " %02X" : "%02X", p[k]);
    out += buf;
  }
  return out;
}

// Visitor over the host entry's call sequence (ExecToLLVM.cpp:35-117 order).
struct Sink {
  virtual ~Sink() = default;
  virtual void module(const Artifact &artifact) = 0;
  virtual void heap(uint64_t id, uint64_t bytes) = 0;
  virtual void resource(uint64_t id, uint64_t heap, uint64_t offset, int64_t argument) = 0;
  virtual void kernel(const ExecKernel &k) = 0;
  virtual void argumentResource(uint64_t id, uint64_t offset) = 0;
  virtual void argumentValue(const void *bytes, uint64_t size, const std::string &what) = 0;
  virtual void workspace(uint64_t bytes) = 0;
  virtual void dependency(uint64_t id) = 0;
  virtual void commit(uint64_t id) = 0;
};

using ArtifactLookup = std::function<const Artifact *(const std::string &identity)>;

void walkPlan(const ExecPlan &plan, const ArtifactLookup &artifacts, Sink &sink, void **values) {
  std::string current;
  auto select = [&](const std::string &identity) {
    if (identity == current) return;
    const Artifact *a = artifacts(identity);
    if (!a) throw CompileError("executable plan references an unavailable artifact " + identity);
    sink.module(*a);
    current = identity;
  };
  if (!plan.kernels.empty()) select(plan.kernels.front().artifact);
  for (const ExecHeap &h : plan.heaps) sink.heap(uint64_t(h.id), uint64_t(h.bytes));
  for (const ExecHeap &h : plan.workspaceHeaps) sink.heap(uint64_t(h.id), uint64_t(h.bytes));
  std::map<std::string, uint64_t> resourceIds;
  for (size_t k = 0; k < plan.resources.size(); ++k) {
    const ExecResource &r = plan.resources[k];
    resourceIds[r.name] = k;
    if (r.kind == "external") {
      if (r.argument < 0) throw CompileError("external resource " + r.name + " is not bound to a host argument");
      sink.resource(k, 0, 0, r.argument);
    } else {
      sink.resource(k, uint64_t(r.heap), uint64_t(r.offset), -1);
    }
  }
  // Library workspaces are heap placements like temporaries, numbered after the resources.
  std::map<std::pair<int64_t, std::string>, uint64_t> workspaceIds;
  for (const ExecWorkspace &w : plan.workspaces) {
    const uint64_t id = plan.resources.size() + workspaceIds.size();
    workspaceIds[{w.kernel, w.role}] = id;
    sink.resource(id, uint64_t(w.heap), uint64_t(w.offset), -1);
  }
  for (const ExecKernel &k : plan.kernels) {
    select(k.artifact);
    sink.kernel(k);
    std::vector<const ExecArgument *> slots;
    for (const ExecArgument &a : k.arguments) slots.push_back(&a);
    std::sort(slots.begin(), slots.end(), [](auto *a, auto *b) { return a->slot < b->slot; });
    for (const ExecArgument *a : slots) {
      if (a->kind == "resource") {
        sink.argumentResource(resourceIds.at(a->resource), a->byteLength >= 0 ? uint64_t(a->byteOffset) : 0);
      } else if (a->kind == "scalar") {
        unsigned index = unsigned(std::stoul(a->name.substr(3)));
        unsigned width = Type::bitWidth(a->type.kind);
        if (!width || width % 8 || width > 64) throw CompileError("host lowering requires byte-sized scalars up to 64 bits");
        sink.argumentValue(values ? values[index] : nullptr, width / 8, a->name);
      } else {
        sink.argumentValue(a->bytes.data(), a->bytes.size(), "");
      }
    }
    if (k.workspace < 0 || k.partials < -1) throw CompileError("library workspace size must be non-negative");
    // The workspace pointers follow the arguments: its state, then (kernels that take one) its
    // partial planes, or a null pointer when it has none. A plan without a workspace heap gives
    // the state as a private workspace (ckl_workspace).
    auto state = workspaceIds.find({k.id, "state"});
    if (state != workspaceIds.end()) sink.argumentResource(state->second, 0);
    else if (k.workspace) sink.workspace(uint64_t(k.workspace));
    if (k.partials >= 0) {
      auto planes = workspaceIds.find({k.id, "partials"});
      if (planes != workspaceIds.end()) {
        sink.argumentResource(planes->second, 0);
      } else {
        if (k.partials) throw CompileError("kernel " + std::to_string(k.id) + " has partial planes but no placement");
        const uint64_t null = 0;
        sink.argumentValue(&null, sizeof null, "");
      }
    }
    for (int64_t d : k.dependencies) sink.dependency(uint64_t(d));
    sink.commit(uint64_t(k.id));
  }
}

void walkEntry(const CompiledProgram &program, Sink &sink, void **values) {
  walkPlan(program.plan, [&](const std::string &identity) { return program.artifact(identity); }, sink, values);
}

struct CallbackSink : Sink {
  void *frame;
  void **values;
  CallbackSink(void *f, void **v) : frame(f), values(v) {}
  void module(const Artifact &a) override { ckl_module(frame, a.identity.c_str(), a.image->data(), a.image->size()); }
  void heap(uint64_t id, uint64_t bytes) override { ckl_heap(frame, id, bytes); }
  void resource(uint64_t id, uint64_t heap, uint64_t offset, int64_t argument) override {
    ckl_resource(frame, id, heap, offset, argument >= 0 ? values[argument] : nullptr);
  }
  void kernel(const ExecKernel &k) override {
    ckl_kernel(frame, k.function.c_str(), uint64_t(k.grid[0]), uint64_t(k.grid[1]), uint64_t(k.grid[2]),
               uint64_t(k.block[0]), uint64_t(k.block[1]), uint64_t(k.block[2]), uint64_t(k.sharedMemory));
  }
  void argumentResource(uint64_t id, uint64_t offset) override { ckl_argument_resource(frame, id, offset); }
  void argumentValue(const void *bytes, uint64_t size, const std::string &) override { ckl_argument_value(frame, bytes, size); }
  void workspace(uint64_t bytes) override { ckl_workspace(frame, bytes); }
  void dependency(uint64_t id) override { ckl_dependency(frame, id); }
  void commit(uint64_t id) override { ckl_commit(frame, id); }
};

struct TextSink : Sink {
  std::ostringstream out;
  void module(const Artifact &a) override {
    out << "ckl_module(\"" << a.identity << "\", " << (a.image ? a.image->size() : 0) << " bytes)\n";
  }
  void heap(uint64_t id, uint64_t bytes) override { out << "ckl_heap(" << id << ", " << bytes << ")\n"; }
  void resource(uint64_t id, uint64_t heap, uint64_t offset, int64_t argument) override {
    out << "ckl_resource(" << id << ", " << heap << ", " << offset << ", "
        << (argument >= 0 ? "arg" + std::to_string(argument) : std::string("null")) << ")\n";
  }
  void kernel(const ExecKernel &k) override {
    out << "ckl_kernel(\"" << k.function << "\", " << k.grid[0] << ", " << k.grid[1] << ", " << k.grid[2] << ", "
        << k.block[0] << ", " << k.block[1] << ", " << k.block[2] << ", " << k.sharedMemory << ")\n";
  }
  void argumentResource(uint64_t id, uint64_t offset) override {
    out << "ckl_argument_resource(" << id << ", " << offset << ")\n";
  }
  void argumentValue(const void *bytes, uint64_t size, const std::string &what) override {
    if (!what.empty()) out << "ckl_argument_value(" << what << ", " << size << ")\n";
    else out << "ckl_argument_value([" << hexBytes(bytes, size) << "], " << size << ")\n";
  }
  void workspace(uint64_t bytes) override { out << "ckl_workspace(" << bytes << ")\n"; }
  void dependency(uint64_t id) override { out << "ckl_dependency(" << id << ")\n"; }
  void commit(uint64_t id) override { out << "ckl_commit(" << id << ")\n"; }
};

// The host entry as IR: one "ckl_host.call" op per callback, in call order, inside a
// "ckl_host.entry" op that names the plan and the host signature. Constant argument bytes are
// kept exactly, as a string attribute (bytes outside printable ASCII print as \XX escapes).
struct HostIRSink : Sink {
  std::ostringstream out;
  void call(const char *callee, std::vector<std::pair<std::string, Attr>> fields) {
    fields.push_back({"callee", Attr::string(callee)});
    out << "    \"ckl_host.call\"() <" << Attr::dictOf(std::move(fields)).str() << "> : () -> ()\n";
  }
  static Attr u64(uint64_t v) { return Attr::integer(int64_t(v)); }
  void module(const Artifact &a) override { call("ckl_module", {{"artifact", Attr::string(a.identity)}}); }
  void heap(uint64_t id, uint64_t bytes) override { call("ckl_heap", {{"id", u64(id)}, {"bytes", u64(bytes)}}); }
  void resource(uint64_t id, uint64_t heap, uint64_t offset, int64_t argument) override {
    if (argument >= 0) call("ckl_resource", {{"id", u64(id)}, {"argument", Attr::integer(argument)}});
    else call("ckl_resource", {{"id", u64(id)}, {"heap", u64(heap)}, {"offset", u64(offset)}});
  }
  void kernel(const ExecKernel &k) override {
    call("ckl_kernel", {{"entry_point", Attr::string(k.function)}, {"grid", Attr::denseI64(k.grid)},
                        {"block", Attr::denseI64(k.block)}, {"shared_memory", Attr::integer(k.sharedMemory)}});
  }
  void argumentResource(uint64_t id, uint64_t offset) override {
    call("ckl_argument_resource", {{"resource", u64(id)}, {"offset", u64(offset)}});
  }
  void argumentValue(const void *bytes, uint64_t size, const std::string &what) override {
    if (!what.empty()) {
      call("ckl_argument_value", {{"argument", Attr::integer(std::stoll(what.substr(3)))}, {"size", u64(size)}});
    } else {
      const char *p = static_cast<const char *>(bytes);
      call("ckl_argument_value", {{"bytes", Attr::string(std::string(p, p + size))}, {"size", u64(size)}});
    }
  }
  void workspace(uint64_t bytes) override { call("ckl_workspace", {{"bytes", u64(bytes)}}); }
  void dependency(uint64_t id) override { call("ckl_dependency", {{"id", u64(id)}}); }
  void commit(uint64_t id) override { call("ckl_commit", {{"id", u64(id)}}); }
};

// Checks that `plan` is a complete single-device HIP handoff for the native host entry
// (the reference's host lowering, lib/Transforms/ExecToLLVM.cpp:122-190, requires the same of a
// CUDA plan) and returns the host entry IR.
std::string lowerPlanToHost(const Module &module, const ExecPlan &plan) {
  if (plan.backend != "rocm") throw CompileError("host lowering requires the rocm backend, not '" + plan.backend + "'");
  const Op *source = module.lookup(plan.source);
  const Attr *results = source ? source->attr("ckl.num_results") : nullptr;
  if (!source || source->name != "func.func" || (results && results->i != 0))
    throw CompileError("host lowering requires a source function declaration with no results");
  const std::vector<Type> &signature = plan.sourceArguments;
  auto bound = [&](const std::string &name) -> const Type * {
    if (name.size() <= 3 || name.rfind("arg", 0) != 0 || name.find_first_not_of("0123456789", 3) != std::string::npos)
      return nullptr;
    size_t index = std::stoul(name.substr(3));
    return index < signature.size() ? &signature[index] : nullptr;
  };
  for (const ExecResource &r : plan.resources) {
    if (r.device != "rocm:0") throw CompileError("host lowering requires rocm:0 resources, not '" + r.device + "'");
    if (r.kind != "external") continue;
    const Type *t = bound(r.name);
    if (!t) throw CompileError("host lowering requires external resources bound to original argN arguments");
    if (!t->isMemRef()) throw CompileError("external resource binding type does not match the source argument");
  }
  std::set<std::string> kernels;
  for (const ExecKernel &k : plan.kernels) {
    if (k.abi != "rocm.bare_ptr") throw CompileError("host lowering requires rocm.bare_ptr kernels, not '" + k.abi + "'");
    if (k.device != "rocm:0") throw CompileError("host lowering requires rocm:0 kernels, not '" + k.device + "'");
    kernels.insert(k.kernel.substr(0, k.kernel.find("::")));
    for (const ExecArgument &a : k.arguments) {
      if (a.kind != "scalar") continue;
      const Type *t = bound(a.name);
      if (!t) throw CompileError("host lowering requires original argN bindings within the source signature");
      if (*t != a.type) throw CompileError("scalar binding type does not match the source argument");
    }
  }
  // Device code is compiled separately: the host program holds the plan's source declaration
  // and the kernels it launches, and nothing else.
  for (auto &op : module.body()->ops) {
    bool expected = op->name == "ckl_exec.plan" ||
                    (op->name == "func.func" && (op->symName() == plan.source || kernels.count(op->symName())));
    if (!expected) throw CompileError(sourcePosition(op.get()) + "host lowering found an unexpected operation '" + op->name + "'");
  }
  HostIRSink sink;
  std::map<std::string, Artifact> stubs;
  walkPlan(plan, [&](const std::string &identity) {
    Artifact &a = stubs[identity];
    a.identity = identity;
    return &a;
  }, sink, nullptr);
  std::vector<Attr> arguments;
  for (const Type &t : signature) arguments.push_back(Attr::typeAttr(t));
  std::ostringstream out;
  out << "  \"ckl_host.entry\"() <" << Attr::dictOf({{"arguments", Attr::arrayOf(arguments)}, {"name", Attr::string(plan.name)},
                                                       {"source", Attr::string(plan.source)}}).str()
      << "> ({\n" << sink.out.str() << "  }) : () -> ()\n";
  return out.str();
}

std::string scalarName(const Type &t) {
  switch (t.kind) {
  case Type::I32: return "i32";
  case Type::I64: return "i64";
  case Type::F32: return "f32";
  case Type::F64: return "f64";
  default: return t.str();
  }
}

} // namespace

void replayPlan(const CompiledProgram &program, void *frame, void **values) {
  CallbackSink sink(frame, values);
  walkEntry(program, sink, values);
}

std::shared_ptr<CompiledProgram> compileProgram(const std::string &ir, const CompileOptions &options,
                                                const DeviceCompiler &deviceCompiler,
                                                const std::function<Artifact()> &libraryArtifact) {
  auto module = parseModule(ir);
  verifyModule(*module);
  if (module->op->attr("ckl.fusion.requires_disjoint"))
    throw CompileError("compile original source, not pre-fused guarded IR");
  bool fused = options.fusePointwise && fusePointwise(*module);
  std::string jitArtifact = prepareHip(*module, {options.chip, options.features});
  auto result = std::make_shared<CompiledProgram>();
  result->preparedIR = printModule(*module, true);

  auto executable = cloneModule(*module);
  auto summaries = deriveEffectSummaries(*executable, options.strict);
  std::optional<Graph> graph;
  Op *host = nullptr;
  for (Op *function : executable->functions()) {
    auto g = buildGraph(*executable, function, summaries, options.reuseStorage);
    if (!g) continue;
    if (graph) throw CompileError("compilation requires exactly one host program");
    graph = std::move(g);
    host = function;
  }
  if (!graph) throw CompileError("compilation requires exactly one host program");
  result->plan = lowerGraphToExec(*executable, host, *graph);
  result->executableIR = withPlan(printModule(*executable), result->plan.print());

  std::vector<std::string> jitKernels;
  bool usesLibrary = false;
  for (const ExecKernel &k : result->plan.kernels) {
    if (k.artifact == jitArtifact) {
      if (std::find(jitKernels.begin(), jitKernels.end(), k.kernel) == jitKernels.end()) jitKernels.push_back(k.kernel);
    } else {
      usesLibrary = true;
    }
  }
  // Artifacts in first-use order.
  for (const ExecKernel &k : result->plan.kernels) {
    if (result->artifact(k.artifact)) continue;
    if (k.artifact == jitArtifact) {
      if (!deviceCompiler) throw CompileError("kernel " + k.kernel + " has no library implementation and no device compiler is available");
      std::string source;
      Artifact a = deviceCompiler(*module, jitKernels, jitArtifact, source);
      result->deviceIR += source;
      result->artifacts.push_back(std::move(a));
    } else {
      Artifact lib = libraryArtifact ? libraryArtifact() : Artifact();
      if (lib.identity != k.artifact)
        throw CompileError("library artifact " + k.artifact + " does not match the loaded kernel library " + lib.identity);
      result->artifacts.push_back(std::move(lib));
    }
  }
  (void)usesLibrary;

  if (Block *entry = host->entry()) {
    for (auto &arg : entry->args) {
      if (arg->type.isMemRef()) {
        if (!arg->type.hasStaticShape()) throw CompileError("host buffers require static shapes");
        result->bufferBytes.push_back(uint64_t(arg->type.elementCount()) * (Type::bitWidth(arg->type.element) / 8));
        result->scalarTypes.push_back("");
      } else {
        result->bufferBytes.push_back(0);
        result->scalarTypes.push_back(scalarName(arg->type));
      }
    }
  }
  TextSink text;
  walkEntry(*result, text, nullptr);
  result->hostIR = text.out.str();
  if (fused) {
    CompileOptions unfused = options;
    unfused.fusePointwise = false;
    result->fallback = compileProgram(ir, unfused, deviceCompiler, libraryArtifact);
  }
  return result;
}

// ====================================================================== pass driver
std::string runPasses(const std::string &ir, const std::vector<std::string> &passes) {
  VerifyOptions verify;
  std::vector<std::string> pipeline;
  for (const std::string &spec : passes) {
    if (spec == "allow-unregistered-dialect") verify.allowUnregisteredDialects = true;
    else pipeline.push_back(spec);
  }
  auto module = parseModule(ir);
  verifyModule(*module, verify);
  std::vector<std::pair<Op *, Graph>> graphs;
  std::vector<ExecPlan> plans;
  std::map<const Op *, KernelSummary> summaries;
  for (const std::string &spec : pipeline) {
    std::string name = spec.substr(0, spec.find('{'));
    std::string options = spec.size() > name.size() ? spec.substr(name.size()) : std::string();
    auto has = [&](const char *option) { return options.find(option) != std::string::npos; };
    if (name == "summarize-effects") {
      summaries = deriveEffectSummaries(*module, !has("strict=false"));
    } else if (name == "build-graph") {
      graphs.clear();
      summaries = deriveEffectSummaries(*module, !has("strict=false"));
      for (Op *function : module->functions()) {
        auto g = buildGraph(*module, function, summaries, !has("reuse-storage=false"));
        if (g) graphs.emplace_back(function, std::move(*g));
      }
    } else if (name == "lower-graph-to-exec") {
      for (auto &[function, graph] : graphs) plans.push_back(lowerGraphToExec(*module, function, graph));
      graphs.clear();
    } else if (name == "prepare-hip") {
      prepareHip(*module, {});
    } else if (name == "fuse-pointwise") {
      if (fusePointwise(*module)) module->op->attrs["ckl.fusion.requires_disjoint"] = Attr::unit();
    } else if (name == "lower-exec-to-host") {
      // Plans written in the input and plans lowered earlier in this pipeline, in that order.
      if (&spec != &pipeline.back()) throw CompileError("lower-exec-to-host must be the last pass");
      if (!graphs.empty()) throw CompileError("host lowering requires graphs lowered to executable plans first");
      std::vector<ExecPlan> all = readExecPlans(*module);
      all.insert(all.end(), plans.begin(), plans.end());
      if (all.size() != 1) throw CompileError("host lowering requires exactly one executable plan");
      return "module {\n" + lowerPlanToHost(*module, all.front()) + "}\n";
    } else {
      throw CompileError("unknown pass '" + name + "'");
    }
  }
  std::string extra;
  for (auto &[_, graph] : graphs) extra += graph.print();
  for (auto &plan : plans) extra += plan.print();
  return withPlan(printModule(*module, true), extra);
}

} // namespace ckl
