// Device code generation for CKL kernels without a hand-written library implementation.
//
// The reference lowers kernel bodies through MLIR's GPU/NVVM pipeline to a CUBIN
// (lib/Transforms/CudaKernels.cpp:156-245, python/ckl/_jit.py:34-53). Here each prepared
// kernel body is translated to a gfx950 HIP kernel (one struct argument whose layout equals
// the runtime's packed argument block) and compiled in-process with hipRTC into a code object
// that the executor loads through hipModuleLoadData.
#pragma once

#include "../core/compiler.h"

namespace ckl::rt {

// Generated HIP source for `kernels` of a prepared module (no compilation).
std::string generateDeviceSource(const Module &prepared, const std::vector<std::string> &kernels);

// Generates and compiles; results are cached per artifact identity for the process lifetime.
Artifact compileDeviceCode(const Module &prepared, const std::vector<std::string> &kernels,
                           const std::string &artifact, std::string &source);

} // namespace ckl::rt
