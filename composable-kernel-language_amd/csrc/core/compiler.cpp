#include "compiler.h"

#include "../runtime/callbacks.h"

#include <cstdio>
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

void walkEntry(const CompiledProgram &program, Sink &sink, void **values) {
  const ExecPlan &plan = program.plan;
  std::string current;
  auto select = [&](const std::string &identity) {
    if (identity == current) return;
    const Artifact *a = program.artifact(identity);
    if (!a) throw CompileError("executable plan references an unavailable artifact " + identity);
    sink.module(*a);
    current = identity;
  };
  if (!plan.kernels.empty()) select(plan.kernels.front().artifact);
  for (const ExecHeap &h : plan.heaps) sink.heap(uint64_t(h.id), uint64_t(h.bytes));
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
    if (k.workspace < 0) throw CompileError("library workspace size must be non-negative");
    if (k.workspace) sink.workspace(uint64_t(k.workspace));
    for (int64_t d : k.dependencies) sink.dependency(uint64_t(d));
    sink.commit(uint64_t(k.id));
  }
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
  auto module = parseModule(ir);
  std::vector<std::pair<Op *, Graph>> graphs;
  std::vector<ExecPlan> plans;
  std::map<const Op *, KernelSummary> summaries;
  for (const std::string &spec : passes) {
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
