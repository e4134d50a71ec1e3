/*
 * ckl_hip.h — C ABI of the MI355X (gfx950) CKL backend: compiler pipeline, HIP executor
 * and the host-entry callback protocol.
 *
 * This ABI replaces the reference's native boundary for the decode hot path:
 *   - the nanobind module `_ckl_native` (lib/Compiler/RuntimeBindings.cpp:56-105,
 *     lib/Compiler/NativeBindings.cpp:23-61) that python/ckl/cuda.py and python/ckl/_jit.py call;
 *   - the C++ program API (include/ckl/Runtime/NvidiaProgram.h:16-69);
 *   - the eight JIT->runtime callbacks (lib/Runtime/NvidiaProgram.cpp:60-108).
 * Plain pointers and sizes only. Every function returning int returns CKL_OK (0) on success;
 * on failure ckl_last_error() holds a thread-local message and the code tells the Python layer
 * which exception to raise (ValueError for CKL_INVALID_ARGUMENT, RuntimeError otherwise).
 */
#ifndef CKL_HIP_H
#define CKL_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  CKL_OK = 0,
  CKL_INVALID_ARGUMENT = 1, /* std::invalid_argument / out_of_range -> ValueError */
  CKL_RUNTIME_ERROR = 2,    /* HIP or runtime failure -> RuntimeError */
  CKL_COMPILE_ERROR = 3     /* IR, analysis or device compilation failure -> RuntimeError */
};

typedef struct ckl_program ckl_program;
typedef struct ckl_device ckl_device;
typedef struct ckl_buffer ckl_buffer;
typedef struct ckl_invocation ckl_invocation;

/* Version of this ABI; bumped on any incompatible change. */
int ckl_abi_version(void);
/* Message of the last failed call on this thread (empty when none). */
const char *ckl_last_error(void);
/* Releases strings returned through `char **` out-parameters. */
void ckl_string_free(char *text);

/* ---------------------------------------------------------------- compiler
 * Replaces python/ckl/_jit.py:74-154 (compile_program: fuse, prepare, build-graph,
 * lower-graph-to-exec, device and host lowering) and `make_program`
 * (lib/Compiler/RuntimeBindings.cpp:61-67). `ir` is CKL IR text as printed by the frontend. */
typedef struct {
  int reuse_storage;   /* graph-order temporary reuse (GraphAnalysis.cpp:610-612) */
  int fuse_pointwise;  /* guarded unary pointwise fusion (PointwiseFusion.cpp:260-304) */
  int strict;          /* reject operations without complete effect semantics */
  const char *chip;    /* "gfx950" */
} ckl_compile_options;

int ckl_compile(const char *ir, const ckl_compile_options *options, ckl_program **out);
/* IR views of CompiledProgram (python/ckl/cuda.py:189-208):
 * 0 prepared IR, 1 executable plan IR, 2 device code (generated HIP source),
 * 3 host entry call sequence, 4 host entry call sequence of the unfused fallback ("" if none).
 * The text is owned by the program. */
int ckl_program_ir(ckl_program *program, int stage, const char **text, size_t *size);
/* Host signature derived from the program (bufferBytes / scalarTypes of NvidiaProgram.h:44-48):
 * for argument k, bytes[k] > 0 for a buffer, else types[k] is "i32", "i64", "f32" or "f64". */
int ckl_program_signature(ckl_program *program, size_t *count, const uint64_t **bytes, const char *const **types);
/* A program whose plan is built by an external packed entry `entry(void*[]{&frame, &values})`
 * driving the callbacks below (NvidiaProgram::NvidiaProgram, NvidiaProgram.cpp:136-146). */
int ckl_program_from_entry(void (*entry)(void **), const uint64_t *buffer_bytes, const char *const *scalar_types,
                           size_t count, ckl_program *fallback, ckl_program **out);
void ckl_program_release(ckl_program *program);

/* ckl-opt style pass pipeline over IR text (tools/ckl-opt/ckl-opt.cpp:1-29): `passes` is a list
 * separated by ';', e.g. "build-graph{strict=false};lower-graph-to-exec". The input is verified
 * first; the item "allow-unregistered-dialect" lets operations of unknown dialects through. Passes:
 * summarize-effects, build-graph, lower-graph-to-exec, prepare-hip, fuse-pointwise and (last only)
 * lower-exec-to-host. On success *out holds the printed module (free with ckl_string_free). */
int ckl_opt(const char *ir, const char *passes, char **out);

/* Storage planner (MemoryPlanner::plan, lib/Core/MemoryPlanner.cpp:98-204 and
 * include/ckl/Core/MemoryPlanner.h:18-92) over an explicit graph: `edges` holds edge_count
 * (from, to) pairs. Resource kind: 0 temporary, 1 persistent, 2 external. For each resource k,
 * out[k] receives its heap, offset and slot (heap = UINT64_MAX for externals) and
 * shares_first the first earlier resident of its slot (UINT64_MAX when none). */
typedef struct {
  uint64_t bytes;
  uint64_t alignment;
  int device;
  int kind;
  const char *address_space;
  const uint64_t *users;
  size_t user_count;
} ckl_storage_resource;
typedef struct {
  uint64_t heap;
  uint64_t offset;
  uint64_t slot;
  uint64_t shares_first;
} ckl_storage_assignment;
int ckl_plan_storage(size_t node_count, const uint64_t *edges, size_t edge_count, const ckl_storage_resource *resources,
                     size_t resource_count, int reuse_storage, uint64_t *baseline_bytes, uint64_t *planned_bytes,
                     ckl_storage_assignment *out);

/* Explicit arguments of `kernel` as its gfx950 code object declares them (the AMDGPU metadata
 * note of an ELF code object or of the gfx950 entry of an offload bundle): up to `capacity`
 * offsets and sizes, their number in *count and the kernarg segment size (explicit + hidden) in
 * *segment_bytes. No reference counterpart: the executor checks every packed argument block
 * against this layout before a launch (CUDA's driver sizes a packed block itself), and tools
 * can inspect it. */
int ckl_code_object_arguments(const void *image, uint64_t bytes, const char *kernel, uint32_t *offsets,
                              uint32_t *sizes, uint64_t capacity, uint64_t *count, uint32_t *segment_bytes);

/* Identity of the hand-written gfx950 kernel library code object ("" when absent). */
const char *ckl_library_identity(void);

/* ---------------------------------------------------------------- runtime
 * Replaces `cuda_available`, `Device`, `Buffer`, `bind` and `Invocation`
 * (lib/Compiler/RuntimeBindings.cpp:18-105; python/ckl/cuda.py:93-300). */
int ckl_device_count(void);
int ckl_device_open(int ordinal, ckl_device **out);
const char *ckl_device_name(ckl_device *device);
void ckl_device_release(ckl_device *device);

int ckl_buffer_alloc(ckl_device *device, uint64_t bytes, ckl_buffer **out);
/* Borrows caller-owned device memory (Device.import_buffer, cuda.py:115-122). */
int ckl_buffer_import(ckl_device *device, uint64_t address, uint64_t bytes, ckl_buffer **out);
int ckl_buffer_slice(ckl_buffer *buffer, uint64_t offset, uint64_t bytes, ckl_buffer **out);
uint64_t ckl_buffer_address(ckl_buffer *buffer);
uint64_t ckl_buffer_nbytes(ckl_buffer *buffer);
/* Synchronous copies; complete before any later launch on any stream (cuda.py:154-164). */
int ckl_buffer_copy_from_host(ckl_buffer *buffer, const void *data, uint64_t bytes);
int ckl_buffer_copy_to_host(ckl_buffer *buffer, void *data, uint64_t bytes);
void ckl_buffer_release(ckl_buffer *buffer);

enum { CKL_ARG_BUFFER = 0, CKL_ARG_I32 = 1, CKL_ARG_I64 = 2, CKL_ARG_F32 = 3, CKL_ARG_F64 = 4 };
typedef struct {
  int kind;
  ckl_buffer *buffer;
  int64_t integer;
  double real;
} ckl_argument;

/* NvidiaProgram::bind (NvidiaProgram.cpp:156-215): packs arguments, selects the unfused
 * fallback when external byte ranges overlap, runs the host entry and returns the bound
 * invocation (one stream, one allocation per planned heap). */
int ckl_bind(ckl_program *program, ckl_device *device, const ckl_argument *arguments, size_t count,
             ckl_invocation **out);
/* No-allocation variant of ckl_bind. No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). It calls no hipMalloc/hipFree or other allocating routine:
 *  - planned heaps and library workspaces are carved from a static arena of
 *    CKL_STATIC_SCRATCH_BYTES per device (a file-scope device array of the library, held until
 *    the process ends); larger programs are refused with CKL_INVALID_ARGUMENT;
 *  - workspaces are cleared by a kernel enqueued on `stream` (a caller-owned hipStream_t, which
 *    the invocation launches on and never destroys);
 *  - every code object of the program must already be resident on the device (bind it once
 *    with ckl_bind); otherwise CKL_INVALID_ARGUMENT.
 * All static bindings on one device share that arena from its start: a later ckl_bind_static on
 * the device supersedes earlier ones (running a superseded invocation fails with
 * CKL_INVALID_ARGUMENT), and work of two static invocations that overlaps on one device races. */
#define CKL_STATIC_SCRATCH_BYTES (64ull << 20)
int ckl_bind_static(ckl_program *program, ckl_device *device, const ckl_argument *arguments, size_t count,
                    void *stream, ckl_invocation **out);
/* CKL_STATIC_SCRATCH_BYTES, for bindings that cannot read the macro. */
uint64_t ckl_static_scratch_bytes(void);

/* mode: 0 ordinary launches, 1 inferred graph, 2 single-stream capture (the reference's three,
 * lib/Runtime/NvidiaProgram.cpp:115-131), plus three variants of mode 1 with no reference
 * counterpart as separate modes: 3 one kernel node per dispatch with the reduced DAG's edges (the
 * reference's own inferred graph, lib/Runtime/NvidiaRuntime.cpp:391-433: branch concurrency
 * only), 4 mode 1's contracted and merged launches captured on one stream (contraction only) and
 * 5 the same launches issued on the invocation stream at every run, with no graph (for profilers,
 * and for plans of a few launches, where hipGraphLaunch's submission latency dominates).
 * Mode 1 is those contracted launches as an explicit graph with their DAG edges.
 * Synchronizes the invocation stream before returning. */
int ckl_invocation_run(ckl_invocation *invocation, int mode, uint64_t batch);
/* out[0] stream us/step, out[1] wall us/step, out[2] graph setup ms (NvidiaProgram.cpp:225-270). */
int ckl_invocation_benchmark(ckl_invocation *invocation, int mode, uint64_t iterations, uint64_t batch, double out[3]);
uint64_t ckl_invocation_node_count(ckl_invocation *invocation);
/* Rebind without re-instantiation (NvidiaGraphExecutable::updateKernel, lib/Runtime/
 * NvidiaRuntime.cpp:466-496, which updates one kernel node of an explicitly built graph): the
 * invocation's program on other buffers of the same sizes, scalars unchanged. Every resolved
 * argument address moves with its buffer; the cached explicit graphs (modes 1 and 3) whose units
 * keep their structure get their kernel nodes' parameters replaced in place
 * (hipGraphExecKernelNodeSetParams); captured graphs, and graphs whose chain decisions change with
 * the new addresses, are rebuilt at their next run. Refused (invalid argument) when a scalar
 * differs or the buffers overlap differently than at bind (fused vs unfused program). */
int ckl_invocation_rebind(ckl_invocation *invocation, const ckl_argument *arguments, size_t count);
/* Graph executables this invocation has instantiated so far (modes 1-4). */
int ckl_invocation_graph_instantiations(ckl_invocation *invocation, uint64_t *count);
/* Device memory of the binding (no reference counterpart; the reference reports heap bytes from
 * the plan text): out[0] bytes of the heaps the entry declared (ckl_heap: the plan's temporaries
 * and its library-workspace heap), placed together in one allocation cleared once at bind;
 * out[1] bytes of private workspaces (ckl_workspace); out[2] device allocations the bind made
 * (0 for ckl_bind_static). */
int ckl_invocation_memory(ckl_invocation *invocation, uint64_t out[3]);
/* Independent requests (replaces the thread-pool burst of benchmarks/decoder/experiment.py:53-70,
 * one native benchmark call per request thread): `iterations` runs of `batch` steps of each of
 * `count` distinct invocations of one device in `mode`, every invocation on its own stream, all
 * submitted from the calling thread; with `serial` 0 step k of every request is submitted before
 * step k+1 of any (the requests run side by side), otherwise each request completes before the
 * next starts. Returns after every stream has finished. out (may be NULL): [0] host wall us of
 * the burst, [1] its GPU span us (from an event every stream waits for to one that waits for
 * every stream). */
int ckl_invocations_run(ckl_invocation *const *invocations, size_t count, int mode, uint64_t iterations,
                        uint64_t batch, int serial, double out[2]);
/* Profiler region (replaces the CUDA profiler API range, cudaProfilerStart/Stop, that
 * benchmarks/decoder/experiment.py:121-130 opens around one measured burst): 1 resumes and 0
 * pauses collection through the ROCm tools extension (roctxProfilerResume/Pause), so
 * `rocprofv3 --selected-regions` records only the region. Fails if that library is absent. */
int ckl_profiler_region(int active);
/* Number of device launches (graph nodes) one execution of `batch` steps submits in `mode`. */
int ckl_invocation_launch_count(ckl_invocation *invocation, int mode, uint64_t batch, uint64_t *count);
/* Dependency edges of the explicit graph of `mode` (1 or 3; 0 for the other modes, whose
 * launches are ordered by the stream). No reference counterpart: reports the graph's shape. */
int ckl_invocation_edge_count(ckl_invocation *invocation, int mode, uint64_t batch, uint64_t *count);
/* Kernel-level timing for roofline measurement (no reference counterpart; the reference profiles
 * with nsys): plan node `index` (0 .. node_count-1, executable-plan order) is launched
 * `iterations` times back to back on the invocation stream between two HIP events; the average
 * duration in microseconds is returned. The node's effects are applied `iterations` times. */
int ckl_invocation_time_node(ckl_invocation *invocation, uint64_t index, uint64_t iterations, double *average_us);
/* Device entry point name of plan node `index` ("" when out of range). */
const char *ckl_invocation_node_name(ckl_invocation *invocation, uint64_t index);
/* The launches one inferred step (mode 1, batch 1) submits after chain contraction and sibling
 * grouping (no reference counterpart; measurement helpers like ckl_invocation_time_node):
 * their number, entry point name (valid while the invocation lives), the plan nodes each one
 * executes (up to `capacity` written to `members`, the total in *count), and the average
 * duration of launch `unit` issued `iterations` times back to back on the invocation stream. */
int ckl_invocation_unit_count(ckl_invocation *invocation, uint64_t *count);
int ckl_invocation_unit_name(ckl_invocation *invocation, uint64_t unit, const char **name);
int ckl_invocation_unit_members(ckl_invocation *invocation, uint64_t unit, uint64_t *members, uint64_t capacity,
                                uint64_t *count);
int ckl_invocation_time_unit(ckl_invocation *invocation, uint64_t unit, uint64_t iterations, double *average_us);
/* Durations of the inferred step's launches in sequence (operands as cold as in a graph replay):
 * every prefix of the launch chain (its first k launches, k = 0 .. count) is issued `repeats`
 * times between two HIP events, and launch k's duration is the difference of the median times
 * of prefixes k+1 and k (the events' cost cancels). The prefixes' effects are applied. Writes up
 * to `capacity` durations in microseconds; the launch count in *count. */
int ckl_invocation_profile_units(ckl_invocation *invocation, uint64_t repeats, double *durations_us, uint64_t capacity,
                                 uint64_t *count);
void ckl_invocation_release(ckl_invocation *invocation);

/* ---------------------------------------------------------------- host-entry callbacks
 * The reference's eight callbacks with identical signatures (NvidiaProgram.cpp:60-108) plus
 * ckl_module, which loads (once per device) and selects a named code object so one plan can
 * mix library kernels and JIT-compiled kernels, and ckl_workspace (below). Errors are recorded in `frame`; later
 * callbacks become no-ops and ckl_bind reports the first error. */
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
/* HIP addition (no reference counterpart): gives the pending kernel a private device workspace of
 * `bytes` bytes, zero-filled once at bind and owned by the invocation, and appends its address
 * as the next kernel argument. Compiled plans place their library kernels' workspaces in a
 * planned workspace heap instead (a ckl_heap after the temporaries' heaps, its placements
 * declared with ckl_resource and passed with ckl_argument_resource); this callback serves host
 * entries written by hand and plans without a workspace heap.
 * Every ckl_heap of one bind is placed in a single device allocation (ckl_bind_static: one range
 * of the static arena) when the entry first declares a resource, and that range is zero-filled
 * once, by one kernel on the invocation's stream. */
void ckl_workspace(void *frame, uint64_t bytes);

#ifdef __cplusplus
}
#endif

#endif /* CKL_HIP_H */
