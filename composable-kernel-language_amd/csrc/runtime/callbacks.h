// Host-entry callback ABI (lib/Runtime/NvidiaProgram.cpp:60-108 for the reference's eight
// callbacks; ckl_module is the HIP addition that selects among several code objects, and
// ckl_workspace gives a library kernel its private zero-initialised device workspace).
// `frame` is the invocation under construction; errors are recorded in it, never thrown.
#pragma once

#include <cstdint>

extern "C" {
void ckl_begin(void *frame, const void *binary, uint64_t bytes);
void ckl_module(void *frame, const char *identity, const void *binary, uint64_t bytes);
void ckl_heap(void *frame, uint64_t id, uint64_t bytes);
void ckl_resource(void *frame, uint64_t id, uint64_t heap, uint64_t offset, void *external);
void ckl_kernel(void *frame, const char *name, uint64_t gx, uint64_t gy, uint64_t gz, uint64_t bx, uint64_t by,
                uint64_t bz, uint64_t shared);
void ckl_argument_resource(void *frame, uint64_t id, uint64_t offset);
void ckl_argument_value(void *frame, const void *bytes, uint64_t size);
void ckl_dependency(void *frame, uint64_t id);
void ckl_commit(void *frame, uint64_t id);
void ckl_workspace(void *frame, uint64_t bytes);
}
