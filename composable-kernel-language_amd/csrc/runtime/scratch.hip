// Static scratch arena (see scratch.h). Built by hipcc into libckl_hip.so so that the array is
// part of the library's own code object, which HIP loads on every device the process uses.
#include "scratch.h"

#include "../../../include/ckl_hip.h"

#include <array>
#include <mutex>
#include <stdexcept>
#include <string>

// The arena itself. In host code this name is only a handle for hipGetSymbolAddress: kernels
// receive the per-device address that call returns, never this symbol.
static __device__ __align__(256) unsigned char scratch[CKL_STATIC_SCRATCH_BYTES];

__global__ void __launch_bounds__(256) ckl_scratch_fill(uint4 *words, uint64_t count) {
  const uint4 zero = make_uint4(0u, 0u, 0u, 0u);
  for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += uint64_t(gridDim.x) * blockDim.x)
    words[i] = zero;
}

namespace ckl::rt {
namespace {

constexpr int kMaxDevices = 64;
std::mutex addressMutex;
std::array<uint64_t, kMaxDevices> addresses{};

void require(hipError_t status, const char *what) {
  if (status != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(status));
}

} // namespace

uint64_t staticScratchBytes() { return CKL_STATIC_SCRATCH_BYTES; }

uint64_t staticScratchAddress(int ordinal) {
  if (ordinal < 0 || ordinal >= kMaxDevices) throw std::invalid_argument("HIP device ordinal out of range for the static arena");
  std::lock_guard<std::mutex> lock(addressMutex);
  if (!addresses[size_t(ordinal)]) {
    require(hipSetDevice(ordinal), "hipSetDevice");
    void *pointer = nullptr;
    require(hipGetSymbolAddress(&pointer, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    if (!pointer) throw std::runtime_error("hipGetSymbolAddress returned no address for the static arena");
    addresses[size_t(ordinal)] = reinterpret_cast<uint64_t>(pointer);
  }
  return addresses[size_t(ordinal)];
}

void staticScratchClear(uint64_t address, uint64_t bytes, hipStream_t stream) {
  if (!bytes) return;
  if (address % 16 || bytes % 16) throw std::invalid_argument("static arena clears cover whole 16-byte words");
  const uint64_t words = bytes / 16;
  const unsigned blocks = unsigned(words / 256 + 1 < 1024 ? words / 256 + 1 : 1024);
  hipLaunchKernelGGL(ckl_scratch_fill, dim3(blocks), dim3(256), 0, stream, reinterpret_cast<uint4 *>(address), words);
  require(hipGetLastError(), "ckl_scratch_fill launch");
}

} // namespace ckl::rt
