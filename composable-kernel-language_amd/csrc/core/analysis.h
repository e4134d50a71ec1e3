// Effect summaries, the effect/alias-derived dependency graph, the storage-plan bridge and
// lowering to an executable plan.
//
// Reference counterparts (semantics kept, code written for this IR):
//   lib/Core/MemoryEffects.cpp          access bits, conflicts, base resources, regions
//   lib/Analysis/EffectAnalysis.cpp     interprocedural kernel effect summaries
//   lib/Analysis/GraphAnalysis.cpp      graph nodes, edges with reasons, memory plan bridge
//   lib/Analysis/GraphAlgorithms.cpp    transitive reduction among dispatch nodes
//   lib/Transforms/ExecutablePlan.cpp   heaps, resources and kernels of the executable plan
//   lib/Transforms/CudaKernels.cpp      kernel validation and artifact identity (HIP variant)
#pragma once

#include "ir.h"
#include "planner.h"

#include <map>
#include <set>
#include <string>
#include <vector>

namespace ckl {

enum AccessBits : unsigned { NoAccess = 0, Read = 1u, Write = 2u, Allocate = 4u, Free = 8u };

struct AccessRegion {
  enum Kind { Whole, Unknown, Interval } kind = Whole;
  int64_t offset = 0, length = 0;
  static AccessRegion whole() { return {}; }
  static AccessRegion unknown() { AccessRegion r; r.kind = Unknown; return r; }
  static AccessRegion interval(int64_t o, int64_t l) { AccessRegion r; r.kind = Interval; r.offset = o; r.length = l; return r; }
  Attr attr() const;
};

bool hasConflictingAccesses(unsigned lhs, unsigned rhs);
bool isAllocationValue(const Value *value);
Value *getBaseResource(Value *value);
enum class Alias { No, May, Must };
Alias aliasWholeBuffers(Value *lhs, Value *rhs);
// Static byte interval of a contiguous value relative to its base resource.
std::optional<AccessRegion> staticResourceRange(const Value *value);
AccessRegion composeAccessRegion(const Value *resource, const AccessRegion &relative);
std::optional<AccessRegion> mergeAccessRegions(const std::optional<AccessRegion> &lhs, const AccessRegion &rhs);
bool disjointRegions(const AccessRegion &lhs, const AccessRegion &rhs);

struct KernelSummary {
  std::vector<unsigned> effects;                         // per function argument
  std::vector<std::optional<AccessRegion>> regions;      // per function argument
  std::vector<std::string> orderingScopes;
  bool synchronizes = false;
  bool unknown = false;
};

struct CompileError : std::runtime_error {
  using std::runtime_error::runtime_error;
};

// Derives summaries for every function and attaches `ckl.effect_summary`.
// strict = reject operations without complete effect semantics.
std::map<const Op *, KernelSummary> deriveEffectSummaries(Module &module, bool strict);

// -------------------------------------------------------------------- graph
struct BoundAccess {
  Value *resource;
  unsigned bits;
  AccessRegion region;
};

struct GraphNode {
  unsigned id = 0;
  std::string kind;           // dispatch | alloc | free | lifetime
  Op *source = nullptr;
  std::string kernel;         // dispatch only
  std::vector<BoundAccess> accesses;
  Attr materialized;          // printed access list
  std::vector<std::string> orderingScopes;
  bool unknown = false, synchronizes = false, nestedControl = false;
};

struct EdgeReason {
  std::string kind, detail, resource, alias, from, to;
  Attr attr() const;
};

struct PlannedResource {
  std::string name, device, addressSpace;
  std::size_t bytes = 0;
  std::vector<unsigned> users;
  bool temporary = false;
  Value *value = nullptr;
};

struct Graph {
  std::string source;                                         // host function symbol
  std::vector<GraphNode> nodes;
  std::map<std::pair<unsigned, unsigned>, std::vector<EdgeReason>> edges;
  std::vector<PlannedResource> resources;
  bool planned = false;
  std::string unavailableReason;
  planning::MemoryPlan plan;                                  // valid when planned
  std::vector<std::size_t> plannerToResource;                 // planner resource id -> resources index
  bool reuseStorage = true;                                   // the storage-reuse setting of the plan
  std::string dot;
  std::string print() const;                                  // "ckl.graph" op text
};

// Builds the graph of one host function (nullopt when it contains no dispatch).
std::optional<Graph> buildGraph(Module &module, Op *function,
                                const std::map<const Op *, KernelSummary> &summaries, bool reuseStorage);

// Transitive reduction among dispatch nodes; graph node ids are kept.
std::map<unsigned, std::vector<unsigned>> reducedDispatchDependencies(const Graph &graph);

// -------------------------------------------------------------------- executable plan
struct ExecHeap {
  int64_t id, bytes, alignment, device;
  std::string addressSpace;
};

struct ExecResource {
  std::string name, kind, device, addressSpace;
  int64_t alignment = 256, bytes = 0;
  int64_t heap = -1, offset = -1;     // temporaries
  int64_t argument = -1;              // externals: host function argument number
};

struct ExecArgument {
  int64_t slot = 0, logicalIndex = 0;
  std::string kind;                   // resource | scalar | constant | bytes
  Type type;
  std::string resource;               // resource
  int64_t byteOffset = 0, byteLength = -1;
  std::string packing;
  std::string name;                   // scalar: "argN"
  std::vector<uint8_t> bytes;         // constant / bytes: little-endian payload
  Attr value;                         // constant / bytes: printed value
  Attr attr() const;
};

struct ExecKernel {
  int64_t id = 0;
  std::string kernel;                 // CKL kernel symbol
  std::string function;               // device entry point in the artifact
  std::string implementation, artifact, abi, device;
  std::vector<int64_t> grid, block;   // physical launch
  std::vector<int64_t> logicalGrid, logicalBlock;
  int64_t sharedMemory = 0;
  std::string group;                  // sibling-grouping family ("" = none)
  int64_t workspace = 0;              // library kernel: workspace state bytes (zero at every launch)
  int64_t partials = -1;              // library kernel: split-reduction plane bytes (-1: no such pointer)
  std::vector<ExecArgument> arguments;
  std::vector<int64_t> dependencies;
};

// Device memory a library kernel uses beyond its arguments (HIP addition, no reference
// counterpart), placed in the plan's workspace heap: role "state" (zero page and completion
// counters, read as zero at every launch: never shared) or "partials" (split-reduction planes,
// live from the kernel to its last reader: placed by the storage planner, so kernels whose
// planes are never live together share memory).
struct ExecWorkspace {
  std::string name, role;
  int64_t kernel = 0, heap = 0, offset = 0, bytes = 0;
};

struct ExecPlan {
  std::string name, source, backend;
  std::vector<Type> sourceArguments;
  std::vector<ExecHeap> heaps;
  std::vector<ExecResource> resources;
  std::vector<ExecHeap> workspaceHeaps;   // at most one; its id follows the heaps' ids
  std::vector<ExecWorkspace> workspaces;
  std::vector<ExecKernel> kernels;
  std::string print() const;          // "ckl_exec.plan" op text, one op per line
  void verify() const;                // throws CompileError
};

ExecPlan lowerGraphToExec(const Module &module, const Op *function, const Graph &graph);

// Little-endian bytes of an integer or float constant of a byte-sized scalar type of at most
// 64 bits, as the host passes it to a kernel argument slot.
std::vector<uint8_t> constantBytes(const Attr &value, const Type &type);

// -------------------------------------------------------------------- HIP preparation
struct PrepareOptions {
  std::string chip = "gfx950";
  std::string features = "";
};
// Validates kernels for the HIP direct ABI and assigns device, capabilities, artifact and
// implementation identities to every dispatch (CudaKernels.cpp:26-153, retargeted to HIP).
// Returns the artifact identity of the JIT-compiled kernel set.
std::string prepareHip(Module &module, const PrepareOptions &options);

// Guarded unary pointwise fusion through a single-use temporary (PointwiseFusion.cpp).
// Returns true when any chain was fused.
bool fusePointwise(Module &module);

} // namespace ckl
