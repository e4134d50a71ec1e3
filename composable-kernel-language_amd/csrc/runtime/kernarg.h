// Explicit kernel-argument layout read from a gfx950 code object.
//
// hipModuleLaunchKernel copies each explicit argument of a kernel from `kernelParams[i]` with
// the size the code object declares for it. The executor packs a CKL dispatch's arguments into
// one byte block (natural alignment, padded to 8; lib/Runtime/NvidiaProgram.cpp:86-100 packs the
// same way), so it must know, per kernel, where each explicit argument starts in that block and
// how large it is: a block shorter than the declared layout would make HIP read past it. This
// reader takes the AMDGPU metadata note (NT_AMDGPU_METADATA, a MessagePack map) out of the ELF
// code object (or out of the gfx950 entry of a clang offload bundle) and returns, for every
// kernel, its explicit arguments (value kinds other than `hidden_*`) in declaration order.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace ckl::rt {

struct KernelArgument {
  uint32_t offset = 0;
  uint32_t size = 0;
};

struct KernelSignature {
  std::vector<KernelArgument> arguments;   // explicit arguments, declaration order
  uint32_t segmentBytes = 0;               // .kernarg_segment_size (explicit + hidden)
  // End of the last explicit argument: the bytes a packed block must provide.
  uint32_t explicitBytes() const {
    uint32_t end = 0;
    for (const KernelArgument &a : arguments) end = a.offset + a.size > end ? a.offset + a.size : end;
    return end;
  }
};

// Kernel name (.name) -> signature. Throws std::invalid_argument when the image is neither an
// ELF code object nor an uncompressed offload bundle holding one, or its metadata is malformed.
std::map<std::string, KernelSignature> readKernelSignatures(const void *image, size_t bytes);

} // namespace ckl::rt
