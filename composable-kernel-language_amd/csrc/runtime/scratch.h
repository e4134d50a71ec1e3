// The static scratch arena of ckl_bind_static: device memory that exists for the life of the
// process on every GPU the library runs on, so that an invocation can be bound without any
// device allocation (include/ckl_hip.h, ckl_bind_static).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace ckl::rt {

// Capacity of the arena on each device (CKL_STATIC_SCRATCH_BYTES).
uint64_t staticScratchBytes();
// Device address of the arena on HIP device `ordinal`. The first call for an ordinal makes that
// device current and asks HIP for the address of the array on it (hipGetSymbolAddress); later
// calls return the recorded address. Throws std::runtime_error when HIP reports a failure.
uint64_t staticScratchAddress(int ordinal);
// Enqueues a kernel on `stream` that zero-fills [address, address + bytes) of an arena
// (both multiples of 16). No allocation, no memset node.
void staticScratchClear(uint64_t address, uint64_t bytes, hipStream_t stream);

} // namespace ckl::rt
