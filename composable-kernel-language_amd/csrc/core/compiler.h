// Compilation pipeline: CKL IR text -> prepared module -> graph -> storage plan ->
// executable plan, plus the native host entry that replays the plan through the
// callback ABI at bind time.
//
// Reference pipeline: python/ckl/_jit.py:74-154 (fuse, prepare, build-graph,
// lower-graph-to-exec, device lowering, host lowering) and lib/Transforms/ExecToLLVM.cpp:25-120
// (the call sequence of the host entry). The host entry here is native code that walks the
// plan; it emits exactly the callback sequence ExecToLLVM would have compiled.
#pragma once

#include "analysis.h"

#include <functional>
#include <memory>
#include <string>
#include <vector>

namespace ckl {

struct CompileOptions {
  bool reuseStorage = true;
  bool fusePointwise = true;
  bool strict = true;
  std::string chip = "gfx950";
  std::string features = "";
};

struct Artifact {
  std::string identity;
  std::string format;            // "rocm.hsaco"
  std::shared_ptr<const std::vector<uint8_t>> image;
};

// Device code generation hook: returns the code object for the JIT-compiled kernels of a
// prepared module (empty image when the module has none), and the generated source.
using DeviceCompiler = std::function<Artifact(const Module &prepared, const std::vector<std::string> &kernels,
                                              const std::string &artifact, std::string &source)>;

struct CompiledProgram {
  std::string preparedIR, executableIR, deviceIR, hostIR;
  ExecPlan plan;
  std::vector<Artifact> artifacts;           // in first-use order
  std::vector<uint64_t> bufferBytes;         // per host argument (0 = scalar)
  std::vector<std::string> scalarTypes;      // per host argument ("" = buffer)
  std::shared_ptr<CompiledProgram> fallback; // unfused program for overlapping bindings
  const Artifact *artifact(const std::string &identity) const;
};

std::shared_ptr<CompiledProgram> compileProgram(const std::string &ir, const CompileOptions &options,
                                                const DeviceCompiler &deviceCompiler,
                                                const std::function<Artifact()> &libraryArtifact);

// Replays the plan as callback calls on `frame`; `values[k]` points at host argument k.
void replayPlan(const CompiledProgram &program, void *frame, void **values);

// ckl-opt style pass driver over textual IR (summarize-effects, build-graph,
// lower-graph-to-exec, prepare-hip, fuse-pointwise).
std::string runPasses(const std::string &ir, const std::vector<std::string> &passes);

} // namespace ckl
