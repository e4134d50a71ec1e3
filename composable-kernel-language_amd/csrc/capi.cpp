// C ABI (include/ckl_hip.h) over the compiler pipeline and the HIP executor.
#include "../../include/ckl_hip.h"

#include "core/compiler.h"
#include "core/sha256.h"
#include "runtime/codegen.h"
#include "runtime/runtime.h"

#include <dlfcn.h>

#include <cstring>
#include <fstream>
#include <iterator>
#include <mutex>

struct ckl_program {
  std::shared_ptr<ckl::CompiledProgram> compiled;
  std::shared_ptr<ckl::rt::ProgramState> state;
};
struct ckl_device {
  std::shared_ptr<ckl::rt::Device> device;
};
struct ckl_buffer {
  std::shared_ptr<ckl::rt::Buffer> buffer;
};
struct ckl_invocation {
  std::shared_ptr<ckl::rt::Invocation> invocation;
};

namespace {

thread_local std::string lastError;

template <typename F> int guarded(F action) {
  try {
    lastError.clear();
    action();
    return CKL_OK;
  } catch (const std::invalid_argument &e) {
    lastError = e.what();
    return CKL_INVALID_ARGUMENT;
  } catch (const std::out_of_range &e) {
    lastError = e.what();
    return CKL_INVALID_ARGUMENT;
  } catch (const ckl::CompileError &e) {
    lastError = e.what();
    return CKL_COMPILE_ERROR;
  } catch (const ckl::IRError &e) {
    lastError = e.what();
    return CKL_COMPILE_ERROR;
  } catch (const std::exception &e) {
    lastError = e.what();
    return CKL_RUNTIME_ERROR;
  } catch (...) {
    lastError = "unknown native failure";
    return CKL_RUNTIME_ERROR;
  }
}

std::string libraryDirectory() {
  Dl_info info{};
  if (dladdr(reinterpret_cast<void *>(&ckl_abi_version), &info) && info.dli_fname) {
    std::string path = info.dli_fname;
    size_t slash = path.rfind('/');
    return slash == std::string::npos ? std::string(".") : path.substr(0, slash);
  }
  return ".";
}

const ckl::Artifact &libraryArtifact() {
  static ckl::Artifact artifact;
  static std::once_flag once;
  std::call_once(once, [] {
    const char *configured = std::getenv("CKL_KERNEL_LIBRARY");
    std::string path = configured ? configured : libraryDirectory() + "/ckl_kernels_gfx950.hsaco";
    std::ifstream input(path, std::ios::binary);
    if (!input) return;
    auto image = std::make_shared<std::vector<uint8_t>>(std::istreambuf_iterator<char>(input), std::istreambuf_iterator<char>());
    if (image->empty()) return;
    ckl::Sha256 hash;
    hash.update(image->data(), image->size());
    artifact.identity = "ckl.hip.library." + hash.hex().substr(0, 24);
    artifact.format = "rocm.hsaco";
    artifact.image = std::move(image);
  });
  return artifact;
}

void nativeEntry(void **packed) {
  void *frame = *static_cast<void **>(packed[0]);
  void **values = *static_cast<void ***>(packed[1]);
  auto *program = static_cast<const ckl::CompiledProgram *>(packed[2]);
  try {
    ckl::replayPlan(*program, frame, values);
  } catch (const std::exception &error) {
    auto *invocation = static_cast<ckl::rt::Invocation *>(frame);
    if (invocation->error.empty()) invocation->error = error.what();
  }
}

std::shared_ptr<ckl::rt::ProgramState> stateFor(const std::shared_ptr<ckl::CompiledProgram> &compiled) {
  auto state = std::make_shared<ckl::rt::ProgramState>();
  state->entry = &nativeEntry;
  state->entryContext = compiled.get();
  state->bufferBytes = compiled->bufferBytes;
  state->scalarTypes = compiled->scalarTypes;
  for (const ckl::ExecResource &r : compiled->plan.resources)
    state->resourceBytes.push_back(r.kind == "temporary" ? uint64_t(r.bytes) : 0);
  state->owner = compiled;
  if (compiled->fallback) state->aliasFallback = stateFor(compiled->fallback);
  return state;
}

template <typename T> void require(T *pointer, const char *what) {
  if (!pointer) throw std::invalid_argument(std::string(what) + " must not be null");
}

} // namespace

extern "C" {

int ckl_abi_version(void) { return 1; }
const char *ckl_last_error(void) { return lastError.c_str(); }
void ckl_string_free(char *text) { std::free(text); }

int ckl_compile(const char *ir, const ckl_compile_options *options, ckl_program **out) {
  return guarded([&] {
    require(ir, "ir");
    require(out, "out");
    ckl::CompileOptions o;
    if (options) {
      o.reuseStorage = options->reuse_storage != 0;
      o.fusePointwise = options->fuse_pointwise != 0;
      o.strict = options->strict != 0;
      if (options->chip) o.chip = options->chip;
    }
    auto compiled = ckl::compileProgram(ir, o, ckl::rt::compileDeviceCode, [] { return libraryArtifact(); });
    auto *program = new ckl_program{compiled, stateFor(compiled)};
    *out = program;
  });
}

int ckl_program_ir(ckl_program *program, int stage, const char **text, size_t *size) {
  return guarded([&] {
    require(program, "program");
    require(text, "text");
    if (!program->compiled) throw std::invalid_argument("program has no compiled IR");
    const std::string *s = nullptr;
    static const std::string empty;
    switch (stage) {
    case 0: s = &program->compiled->preparedIR; break;
    case 1: s = &program->compiled->executableIR; break;
    case 2: s = &program->compiled->deviceIR; break;
    case 3: s = &program->compiled->hostIR; break;
    case 4: s = program->compiled->fallback ? &program->compiled->fallback->hostIR : &empty; break;
    default: throw std::invalid_argument("invalid IR stage");
    }
    *text = s->c_str();
    if (size) *size = s->size();
  });
}

int ckl_program_signature(ckl_program *program, size_t *count, const uint64_t **bytes, const char *const **types) {
  return guarded([&] {
    require(program, "program");
    static thread_local std::vector<const char *> names;
    names.clear();
    for (const std::string &t : program->state->scalarTypes) names.push_back(t.c_str());
    if (count) *count = program->state->bufferBytes.size();
    if (bytes) *bytes = program->state->bufferBytes.data();
    if (types) *types = names.data();
  });
}

int ckl_program_from_entry(void (*entry)(void **), const uint64_t *bufferBytes, const char *const *scalarTypes,
                           size_t count, ckl_program *fallback, ckl_program **out) {
  return guarded([&] {
    require(out, "out");
    // NvidiaProgram's constructor check (lib/Runtime/NvidiaProgram.cpp:136-146): an entry and one
    // metadata entry per argument. Here each argument is also either a buffer (bytes > 0, no
    // scalar type) or a scalar of a type bind can pack, so a malformed signature fails now
    // rather than at every bind.
    if (!entry || (count && (!bufferBytes || !scalarTypes)))
      throw std::invalid_argument("invalid host entry or argument metadata");
    auto state = std::make_shared<ckl::rt::ProgramState>();
    state->entry = entry;
    for (size_t k = 0; k < count; ++k) {
      std::string type = scalarTypes[k] ? scalarTypes[k] : "";
      bool scalar = type == "i32" || type == "i64" || type == "f32" || type == "f64";
      if (bufferBytes[k] ? !type.empty() : !scalar)
        throw std::invalid_argument("invalid host entry or argument metadata: argument " + std::to_string(k) +
                                    " must be a buffer with a byte size or an i32/i64/f32/f64 scalar");
      state->bufferBytes.push_back(bufferBytes[k]);
      state->scalarTypes.push_back(type);
    }
    if (fallback) state->aliasFallback = fallback->state;
    *out = new ckl_program{nullptr, state};
  });
}

void ckl_program_release(ckl_program *program) { delete program; }

int ckl_opt(const char *ir, const char *passes, char **out) {
  return guarded([&] {
    require(ir, "ir");
    require(out, "out");
    std::vector<std::string> list;
    std::string all = passes ? passes : "";
    size_t start = 0;
    while (start <= all.size()) {
      size_t end = all.find(';', start);
      std::string item = all.substr(start, end == std::string::npos ? std::string::npos : end - start);
      if (!item.empty()) list.push_back(item);
      if (end == std::string::npos) break;
      start = end + 1;
    }
    std::string text = ckl::runPasses(ir, list);
    char *copy = static_cast<char *>(std::malloc(text.size() + 1));
    std::memcpy(copy, text.c_str(), text.size() + 1);
    *out = copy;
  });
}

int ckl_plan_storage(size_t nodeCount, const uint64_t *edges, size_t edgeCount, const ckl_storage_resource *resources,
                     size_t resourceCount, int reuseStorage, uint64_t *baseline, uint64_t *planned,
                     ckl_storage_assignment *out) {
  return guarded([&] {
    if (edgeCount && !edges) throw std::invalid_argument("edges must not be null");
    if (resourceCount && (!resources || !out)) throw std::invalid_argument("resources and out must not be null");
    std::vector<ckl::planning::GraphEdge> graph;
    for (size_t k = 0; k < edgeCount; ++k) graph.push_back({edges[2 * k], edges[2 * k + 1]});
    std::vector<ckl::planning::Resource> list;
    for (size_t k = 0; k < resourceCount; ++k) {
      const ckl_storage_resource &r = resources[k];
      ckl::planning::Resource res;
      res.name = "r" + std::to_string(k);
      res.bytes = r.bytes;
      res.alignment = r.alignment;
      res.device = r.device;
      res.addressSpace = r.address_space ? r.address_space : "global";
      if (r.kind < 0 || r.kind > 2) throw std::invalid_argument("resource kind must be 0, 1 or 2");
      res.kind = r.kind == 0 ? ckl::planning::ResourceKind::Temporary
                 : r.kind == 1 ? ckl::planning::ResourceKind::Persistent
                               : ckl::planning::ResourceKind::External;
      if (r.user_count && !r.users) throw std::invalid_argument("users must not be null");
      res.users.assign(r.users, r.users + r.user_count);
      list.push_back(std::move(res));
    }
    auto plan = ckl::planning::MemoryPlanner(reuseStorage != 0).plan(nodeCount, graph, list);
    if (baseline) *baseline = plan.baselineBytes;
    if (planned) *planned = plan.plannedBytes;
    const uint64_t none = ~uint64_t(0);
    for (size_t k = 0; k < resourceCount; ++k) out[k] = {none, none, none, none};
    for (const auto &a : plan.assignments) out[a.resource] = {a.heap, a.offset, a.slot, none};
    for (const auto &d : plan.decisions)
      if (!d.sharesWith.empty()) out[d.resource].shares_first = d.sharesWith.front();
  });
}

const char *ckl_library_identity(void) { return libraryArtifact().identity.c_str(); }

int ckl_device_count(void) { return ckl::rt::deviceCount(); }

int ckl_device_open(int ordinal, ckl_device **out) {
  return guarded([&] {
    require(out, "out");
    *out = new ckl_device{std::make_shared<ckl::rt::Device>(ordinal)};
  });
}

const char *ckl_device_name(ckl_device *device) { return device ? device->device->name.c_str() : ""; }
void ckl_device_release(ckl_device *device) { delete device; }

int ckl_buffer_alloc(ckl_device *device, uint64_t bytes, ckl_buffer **out) {
  return guarded([&] {
    require(device, "device");
    require(out, "out");
    *out = new ckl_buffer{ckl::rt::allocateBuffer(device->device, bytes)};
  });
}

int ckl_buffer_import(ckl_device *device, uint64_t address, uint64_t bytes, ckl_buffer **out) {
  return guarded([&] {
    require(device, "device");
    require(out, "out");
    *out = new ckl_buffer{ckl::rt::importBuffer(device->device, address, bytes)};
  });
}

int ckl_buffer_slice(ckl_buffer *buffer, uint64_t offset, uint64_t bytes, ckl_buffer **out) {
  return guarded([&] {
    require(buffer, "buffer");
    require(out, "out");
    *out = new ckl_buffer{ckl::rt::sliceBuffer(buffer->buffer, offset, bytes)};
  });
}

uint64_t ckl_buffer_address(ckl_buffer *buffer) { return buffer ? buffer->buffer->address() : 0; }
uint64_t ckl_buffer_nbytes(ckl_buffer *buffer) { return buffer ? buffer->buffer->bytes : 0; }

int ckl_buffer_copy_from_host(ckl_buffer *buffer, const void *data, uint64_t bytes) {
  return guarded([&] {
    require(buffer, "buffer");
    require(data, "data");
    buffer->buffer->copyFromHost(data, bytes);
  });
}

int ckl_buffer_copy_to_host(ckl_buffer *buffer, void *data, uint64_t bytes) {
  return guarded([&] {
    require(buffer, "buffer");
    require(data, "data");
    buffer->buffer->copyToHost(data, bytes);
  });
}

void ckl_buffer_release(ckl_buffer *buffer) { delete buffer; }

namespace {
std::vector<ckl::rt::Argument> convertArguments(const ckl_argument *arguments, size_t count) {
  if (count && !arguments) throw std::invalid_argument("arguments must not be null");
  std::vector<ckl::rt::Argument> args(count);
  for (size_t k = 0; k < count; ++k) {
    args[k].kind = arguments[k].kind;
    if (arguments[k].kind == CKL_ARG_BUFFER) {
      if (!arguments[k].buffer) throw std::invalid_argument("buffer argument must not be null");
      args[k].buffer = arguments[k].buffer->buffer;
    }
    args[k].integer = arguments[k].integer;
    args[k].real = arguments[k].real;
  }
  return args;
}
} // namespace

int ckl_bind(ckl_program *program, ckl_device *device, const ckl_argument *arguments, size_t count,
             ckl_invocation **out) {
  return guarded([&] {
    require(program, "program");
    require(device, "device");
    require(out, "out");
    *out = new ckl_invocation{ckl::rt::bind(program->state, device->device, convertArguments(arguments, count))};
  });
}

int ckl_bind_static(ckl_program *program, ckl_device *device, const ckl_argument *arguments, size_t count,
                    void *stream, ckl_invocation **out) {
  return guarded([&] {
    require(program, "program");
    require(device, "device");
    require(out, "out");
    if (count && !arguments) throw std::invalid_argument("arguments must not be null");
    std::vector<ckl::rt::Argument> args(count);
    for (size_t k = 0; k < count; ++k) {
      args[k].kind = arguments[k].kind;
      if (arguments[k].kind == CKL_ARG_BUFFER) {
        if (!arguments[k].buffer) throw std::invalid_argument("buffer argument must not be null");
        args[k].buffer = arguments[k].buffer->buffer;
      }
      args[k].integer = arguments[k].integer;
      args[k].real = arguments[k].real;
    }
    *out = new ckl_invocation{
        ckl::rt::bindStatic(program->state, device->device, args, static_cast<hipStream_t>(stream))};
  });
}

uint64_t ckl_static_scratch_bytes(void) { return CKL_STATIC_SCRATCH_BYTES; }

namespace {
// The ROCm tools extension's profiler control, looked up when first needed so that the library
// does not depend on it: rocprofv3 --selected-regions records only what runs between a resume and
// the following pause.
using RoctxControl = int (*)(uint64_t);
struct Roctx {
  RoctxControl pause = nullptr, resume = nullptr;
  Roctx() {
    for (const char *name : {"librocprofiler-sdk-roctx.so.1", "librocprofiler-sdk-roctx.so"}) {
      void *handle = dlopen(name, RTLD_NOW | RTLD_LOCAL);
      if (!handle) continue;
      pause = reinterpret_cast<RoctxControl>(dlsym(handle, "roctxProfilerPause"));
      resume = reinterpret_cast<RoctxControl>(dlsym(handle, "roctxProfilerResume"));
      if (pause && resume) return;
      pause = resume = nullptr;
    }
  }
};
} // namespace

int ckl_profiler_region(int active) {
  return guarded([&] {
    static Roctx roctx;
    if (!roctx.pause) throw std::runtime_error("the ROCm tools extension (librocprofiler-sdk-roctx) is not available");
    if ((active ? roctx.resume : roctx.pause)(0) != 0)
      throw std::runtime_error(active ? "roctxProfilerResume failed" : "roctxProfilerPause failed");
  });
}

int ckl_invocation_run(ckl_invocation *invocation, int mode, uint64_t batch) {
  return guarded([&] {
    require(invocation, "invocation");
    invocation->invocation->run(mode, batch);
  });
}

int ckl_invocation_benchmark(ckl_invocation *invocation, int mode, uint64_t iterations, uint64_t batch, double out[3]) {
  return guarded([&] {
    require(invocation, "invocation");
    require(out, "out");
    auto r = invocation->invocation->benchmark(mode, iterations, batch);
    out[0] = r[0];
    out[1] = r[1];
    out[2] = r[2];
  });
}

int ckl_invocations_run(ckl_invocation *const *invocations, size_t count, int mode, uint64_t iterations,
                        uint64_t batch, int serial, double out[2]) {
  return guarded([&] {
    require(invocations, "invocations");
    std::vector<ckl::rt::Invocation *> requests;
    for (size_t k = 0; k < count; ++k) {
      require(invocations[k], "invocation");
      requests.push_back(invocations[k]->invocation.get());
    }
    auto r = ckl::rt::runConcurrently(requests, mode, iterations, batch, serial != 0);
    if (out) {
      out[0] = r[0];
      out[1] = r[1];
    }
  });
}

int ckl_invocation_rebind(ckl_invocation *invocation, const ckl_argument *arguments, size_t count) {
  return guarded([&] {
    require(invocation, "invocation");
    invocation->invocation->rebind(convertArguments(arguments, count));
  });
}

int ckl_invocation_graph_instantiations(ckl_invocation *invocation, uint64_t *count) {
  return guarded([&] {
    require(invocation, "invocation");
    require(count, "count");
    *count = invocation->invocation->graphInstantiations();
  });
}

int ckl_invocation_memory(ckl_invocation *invocation, uint64_t out[3]) {
  return guarded([&] {
    require(invocation, "invocation");
    require(out, "out");
    const auto m = invocation->invocation->memory();
    for (int k = 0; k < 3; ++k) out[k] = m[k];
  });
}

uint64_t ckl_invocation_node_count(ckl_invocation *invocation) {
  return invocation ? invocation->invocation->nodeCount() : 0;
}

int ckl_invocation_launch_count(ckl_invocation *invocation, int mode, uint64_t batch, uint64_t *count) {
  return guarded([&] {
    require(invocation, "invocation");
    require(count, "count");
    *count = invocation->invocation->graphNodeCount(mode, batch);
  });
}

int ckl_invocation_edge_count(ckl_invocation *invocation, int mode, uint64_t batch, uint64_t *count) {
  return guarded([&] {
    require(invocation, "invocation");
    require(count, "count");
    *count = invocation->invocation->graphEdgeCount(mode, batch);
  });
}

int ckl_code_object_arguments(const void *image, uint64_t bytes, const char *kernel, uint32_t *offsets,
                              uint32_t *sizes, uint64_t capacity, uint64_t *count, uint32_t *segment_bytes) {
  return guarded([&] {
    require(image, "image");
    require(kernel, "kernel");
    require(count, "count");
    auto table = ckl::rt::readKernelSignatures(image, bytes);
    auto found = table.find(kernel);
    if (found == table.end()) throw std::invalid_argument(std::string("code object has no kernel ") + kernel);
    const auto &args = found->second.arguments;
    *count = args.size();
    for (size_t k = 0; k < args.size() && k < capacity; ++k) {
      if (offsets) offsets[k] = args[k].offset;
      if (sizes) sizes[k] = args[k].size;
    }
    if (segment_bytes) *segment_bytes = found->second.segmentBytes;
  });
}

int ckl_invocation_time_node(ckl_invocation *invocation, uint64_t index, uint64_t iterations, double *average_us) {
  return guarded([&] {
    require(invocation, "invocation");
    require(average_us, "average_us");
    *average_us = invocation->invocation->timeNode(index, iterations);
  });
}

const char *ckl_invocation_node_name(ckl_invocation *invocation, uint64_t index) {
  try {
    return invocation ? invocation->invocation->nodeName(index).c_str() : "";
  } catch (...) {
    return "";
  }
}

int ckl_invocation_unit_count(ckl_invocation *invocation, uint64_t *count) {
  return guarded([&] {
    require(invocation, "invocation");
    require(count, "count");
    *count = invocation->invocation->unitCount();
  });
}

int ckl_invocation_unit_name(ckl_invocation *invocation, uint64_t unit, const char **name) {
  return guarded([&] {
    require(invocation, "invocation");
    require(name, "name");
    *name = invocation->invocation->unitName(unit).c_str();
  });
}

int ckl_invocation_unit_members(ckl_invocation *invocation, uint64_t unit, uint64_t *members, uint64_t capacity,
                                uint64_t *count) {
  return guarded([&] {
    require(invocation, "invocation");
    require(count, "count");
    const auto &list = invocation->invocation->unitMembers(unit);
    *count = list.size();
    if (members)
      for (size_t k = 0; k < list.size() && k < capacity; ++k) members[k] = list[k];
  });
}

int ckl_invocation_time_unit(ckl_invocation *invocation, uint64_t unit, uint64_t iterations, double *average_us) {
  return guarded([&] {
    require(invocation, "invocation");
    require(average_us, "average_us");
    *average_us = invocation->invocation->timeUnit(unit, iterations);
  });
}

int ckl_invocation_profile_units(ckl_invocation *invocation, uint64_t repeats, double *durations_us, uint64_t capacity,
                                 uint64_t *count) {
  return guarded([&] {
    require(invocation, "invocation");
    require(count, "count");
    std::vector<double> d = invocation->invocation->profileUnits(repeats);
    *count = d.size();
    if (durations_us)
      for (size_t k = 0; k < d.size() && k < capacity; ++k) durations_us[k] = d[k];
  });
}

void ckl_invocation_release(ckl_invocation *invocation) { delete invocation; }

} // extern "C"
