// HIP executor for CKL executable plans on MI355X (gfx950).
//
// Replaces the reference's CUDA driver executor and program layer:
//   lib/Runtime/NvidiaRuntime.cpp:177-498   plans, repeat, ordinary launch, capture, explicit graphs
//   lib/Runtime/NvidiaProgram.cpp:13-294    callback ABI, bind, run, benchmark
//   lib/Runtime/HipRuntime.cpp:212-466      hipModule loading and kernel nodes
// Execution modes: 0 ordinary launches, 1 inferred graph (from the plan's dependency DAG),
// 2 single-stream capture of ordinary launches (the reference's three, NvidiaProgram.cpp:115-131),
// and two ablations of mode 1: 3 the reference's own inferred graph (one kernel node per dispatch
// with the reduced DAG's edges, NvidiaRuntime.cpp:391-433) and 4 mode 1's contracted launches
// captured on one stream in level order (no graph branches).
#pragma once

#include "callbacks.h"
#include "kernarg.h"

#include <hip/hip_runtime.h>

#include <array>
#include <atomic>
#include <cstdint>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

namespace ckl::rt {

void check(hipError_t status, const char *what);

enum Mode { kOrdinary = 0, kInferred = 1, kCapture = 2, kBranches = 3, kContractedCapture = 4, kInferredStream = 5 };

struct Device {
  explicit Device(int ordinal);
  ~Device();
  int ordinal;
  uint64_t id;
  std::string name;
  std::mutex moduleMutex;
  std::map<std::string, hipModule_t> modules;   // artifact identity -> loaded module
  // Explicit argument layout of every kernel of every loaded module (from its metadata note).
  std::map<hipFunction_t, KernelSignature> signatures;
  // Loads (once) the code object `identity`; with `allowLoad` false a module that is not yet
  // resident is an error instead (the no-allocation bind may not load code objects).
  hipModule_t load(const std::string &identity, const void *image, size_t bytes, bool allowLoad = true);
  // Layout of a kernel of a module loaded here; throws std::logic_error for an unknown function.
  const KernelSignature &signature(hipFunction_t function);
  void makeCurrent() const;
};

struct Buffer {
  std::shared_ptr<Device> device;
  std::shared_ptr<void> storage;   // owning allocation (null for imports)
  uint64_t base = 0;               // address of the underlying allocation/import
  uint64_t offset = 0;
  uint64_t bytes = 0;
  uint64_t address() const { return base + offset; }
  void copyFromHost(const void *data, uint64_t size) const;
  void copyToHost(void *data, uint64_t size) const;
};

std::shared_ptr<Buffer> allocateBuffer(std::shared_ptr<Device> device, uint64_t bytes);
std::shared_ptr<Buffer> importBuffer(std::shared_ptr<Device> device, uint64_t address, uint64_t bytes);
std::shared_ptr<Buffer> sliceBuffer(const std::shared_ptr<Buffer> &buffer, uint64_t offset, uint64_t bytes);

// One resolved kernel launch: function, geometry and the packed argument struct.
struct Launch {
  hipModule_t module = nullptr;             // code object the function comes from
  hipFunction_t function = nullptr;
  hipFunction_t groupFunction = nullptr;   // sibling-group entry point, when the artifact has one
  // Shared-operand entry points for 2 and 3 siblings (<name>_shared2, <name>_shared3).
  hipFunction_t sharedFunction[2] = {nullptr, nullptr};
  std::string name;
  unsigned grid[3] = {1, 1, 1};
  unsigned block[3] = {1, 1, 1};
  unsigned shared = 0;
  std::vector<uint8_t> arguments;           // kernarg bytes (natural alignment, padded to 8)
  // Where each explicit kernel argument starts in `arguments` (from the code object's metadata;
  // set by Invocation::prepare before the launch is issued or recorded).
  std::vector<uint32_t> paramOffsets;
  bool prepared = false;
  std::vector<size_t> slotOffsets;
  std::vector<size_t> slotSizes;
  std::vector<int64_t> slotResources;       // per slot: the plan resource it addresses, or -1
};

struct PlanNode {
  Launch launch;
  std::vector<size_t> dependencies;         // earlier plan nodes
};

struct Plan {
  std::vector<PlanNode> nodes;
  size_t addKernel(Launch launch, std::vector<size_t> dependencies);
  Plan repeat(size_t iterations) const;      // roots of iteration i+1 follow every leaf of i
};

// One launch of a graph mode and the plan nodes it executes (one for ordinary units, several
// for a contracted chain or a merged sibling group).
struct Unit {
  std::vector<size_t> members;
  Launch launch;
};

// Dependent dispatches the inferred graph runs as one launch of a kernel-library chain entry
// point (csrc/runtime/chains.cpp): `members` in dependency order, `launch` with the members'
// argument blocks back to back. Found on one iteration of the plan; `temporary[id]` tells
// whether plan resource `id` is a heap temporary (a buffer no caller can observe).
struct Chain {
  std::vector<size_t> members;                     // ascending plan indices
  Launch launch;
  std::vector<size_t> roles;                       // members in the chain block's order
  // Operands that may read a split linear's partial planes: {role, offset of the pointer in the
  // member's block, offset of its PartialSource in the chain block}.
  std::vector<std::array<size_t, 3>> deferrable;
};
// `refused` (optional) receives the members of every chain refused only because its buffers
// overlap in a way row-by-row execution would change.
std::vector<Chain> findChains(const Plan &plan, const std::vector<bool> &temporary,
                              std::vector<std::vector<size_t>> *refused = nullptr);
// Split linears whose every reader is a deferrable chain operand leave their combine to those
// chains: returns the patched linear launches (by plan index) and fills the chains' sources.
std::map<size_t, Launch> deferCombines(const Plan &plan, const std::vector<bool> &temporary, std::vector<Chain> &chains);
// Whether sibling launches of one entry point read the same operand the way its _shared<M> entry
// point requires (linears multiplying the same x with one shape and tiling).
bool sharesOperands(const std::vector<const Launch *> &members);
// Whether a library launch streams at least kStreamBytes of weights or cache (its <entry>_nt
// variant reads them with nontemporal loads).
bool streams(const Launch &launch);
// Looks up the _group and _shared<M> entry points of `entry` in the launch's module.
void bindVariants(Launch &launch, const std::string &entry);
// Checks the launch's packed block against the explicit arguments its code object declares for
// `launch.function` and records where each argument starts (std::invalid_argument on mismatch).
void prepareParams(Launch &launch, Device &device);

struct GraphExec {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  size_t nodeCount = 0;
  size_t edgeCount = 0;                        // dependency edges of an explicit graph
  std::vector<std::vector<uint8_t>> storage;   // kernarg blocks referenced during capture
  std::vector<Launch> launches;                // the units in graph order (every mode but 2)
  std::vector<std::vector<size_t>> members;    // plan nodes each of those launches executes
  std::vector<hipGraphNode_t> handles;         // kernel node of each unit (explicit graphs, modes 1 and 3)
  ~GraphExec();
};

struct ProgramState;

struct Argument {
  int kind = 0;                 // 0 buffer, 1 i32, 2 i64, 3 f32, 4 f64
  std::shared_ptr<Buffer> buffer;
  int64_t integer = 0;
  double real = 0;
};

// Invocation: a bound program with its stream, heaps, resolved plan and cached graphs.
struct Invocation {
  std::shared_ptr<ProgramState> program;
  std::shared_ptr<Device> device;
  hipStream_t stream = nullptr;
  std::vector<std::shared_ptr<Buffer>> heaps;
  std::vector<std::shared_ptr<Buffer>> buffers;     // keeps bound buffers alive
  std::vector<std::shared_ptr<Buffer>> workspaces;  // private library-kernel workspaces (zeroed at bind)
  std::vector<uint64_t> resources;
  std::vector<bool> temporaryResources;             // resource id -> placed in a heap
  std::vector<bool> externalResources;              // resource id -> a program argument's address
  Plan plan;
  hipModule_t module = nullptr;                     // current module during plan construction
  Launch pending;
  std::vector<size_t> dependencies;
  std::map<uint64_t, size_t> nodes;                 // graph node id -> plan node
  std::map<std::pair<int, uint64_t>, std::unique_ptr<GraphExec>> graphs;
  std::mutex runMutex;
  std::string error;

  // No-allocation binding (ckl_bind_static): heaps and workspaces are carved from the device's
  // static arena at [arenaBase, arenaBase + arenaLimit); `epoch` is the device's static-bind
  // count when this invocation was bound (a later static bind on the device supersedes it).
  bool staticArena = false;
  uint64_t arenaBase = 0, arenaUsed = 0, arenaLimit = 0, epoch = 0;
  bool ownsStream = true;
  bool arenaExceeded = false;                       // the static arena was too small (bind fails)
  uint64_t carve(uint64_t bytes);                   // 256-aligned arena range for `bytes`
  // Heaps declared (ckl_heap) and not yet placed: {id, bytes}. placeHeaps() puts all of them in
  // one allocation (or one static-arena range), cleared by one fill kernel on `stream`.
  std::vector<std::pair<uint64_t, uint64_t>> pendingHeaps;
  void placeHeaps();

  // The program arguments as bound: buffer addresses and scalar bytes; for each plan resource the
  // program argument it is (-1: a heap placement); the program that was asked for (the bound one
  // may be its unfused fallback). `bindingAddresses` is set while the host entry runs.
  std::shared_ptr<ProgramState> requested;
  std::vector<uint64_t> argumentAddresses, argumentScalars;
  std::vector<int64_t> resourceArgument;
  const uint64_t *bindingAddresses = nullptr;
  size_t bindingCount = 0;
  uint64_t instantiations = 0;                      // graph executables built for this invocation
  uint64_t allocations = 0;                         // device allocations the bind made

  Invocation(std::shared_ptr<ProgramState> program, std::shared_ptr<Device> device, hipStream_t external = nullptr);
  ~Invocation();
  void run(int mode, uint64_t batch);
  std::array<double, 3> benchmark(int mode, uint64_t iterations, uint64_t batch);
  // Rebinding without re-instantiation (NvidiaRuntime.cpp:466-496, updateKernel): the same
  // program on other buffers of the same sizes (scalars unchanged). The plan's resolved argument
  // addresses move; every cached explicit graph (modes 1 and 3) whose units keep their structure
  // has its kernel nodes' parameters replaced in place (hipGraphExecKernelNodeSetParams); captured
  // graphs and any graph whose units change are dropped and rebuilt at their next use.
  void rebind(const std::vector<Argument> &arguments);
  uint64_t graphInstantiations();
  // {heap bytes, other device memory the binding owns (private workspaces, moved temporaries),
  // device allocations made by the binding}.
  std::array<uint64_t, 3> memory() const;
  // Temporaries the inferred graph moved out of storage the plan shares (relocateForChains).
  std::shared_ptr<Buffer> relocation;
  bool relocationDecided = false;
  size_t nodeCount() const { return plan.nodes.size(); }
  size_t graphNodeCount(int mode, uint64_t batch);
  size_t graphEdgeCount(int mode, uint64_t batch);
  // Average duration (us) of plan node `index` launched `iterations` times back to back on the
  // invocation stream, bracketed by HIP events.
  double timeNode(size_t index, uint64_t iterations);
  const std::string &nodeName(size_t index) const { return plan.nodes.at(index).launch.name; }
  // The launches of one inferred (mode 1) step under the grouped policy: count, entry name, the
  // plan nodes each executes, and the average duration of one launched `iterations` times.
  size_t unitCount();
  const std::string &unitName(size_t unit);
  const std::vector<size_t> &unitMembers(size_t unit);
  double timeUnit(size_t unit, uint64_t iterations);
  // Per-launch durations of the inferred step in sequence (operands as cold as in a graph
  // replay): prefixes of the step's launch chain (the first k launches, k = 0 .. count) are
  // issued on the invocation stream between two HIP events, `repeats` times each; launch k's
  // duration is the difference of the median times of prefixes k+1 and k, so the events' own
  // cost cancels. The prefixes' effects are applied.
  std::vector<double> profileUnits(uint64_t repeats);

private:
  friend std::array<double, 2> runConcurrently(const std::vector<Invocation *> &, int, uint64_t, uint64_t, bool);
  void validate(int mode, uint64_t batch) const;
  void requireCurrent() const;                      // refuses a superseded static binding
  void relocateForChains();
  GraphExec &inferredUnits();
  double timeLaunch(const Launch &launch, uint64_t iterations);
  GraphExec &graphFor(int mode, uint64_t batch);
  std::vector<Unit> buildUnits(int mode, uint64_t batch, const Plan &repeated);
  void execute(int mode, uint64_t batch);
};

// Independent requests: `iterations` executions of `batch` steps of every invocation in `mode`,
// each on its own stream, submitted from this thread. Concurrent (`serial` false): step k of
// every request is submitted before step k+1 of any, so the requests' launches run side by side;
// serial: each request's executions complete before the next request starts. The invocations
// must be distinct and on one device. Returns {host wall us, GPU span us} of the whole burst: the
// span runs from an event that every stream waits for to one that waits for every stream.
std::array<double, 2> runConcurrently(const std::vector<Invocation *> &requests, int mode, uint64_t iterations,
                                      uint64_t batch, bool serial);

using Entry = void (*)(void **);

// Program: metadata for a packed host entry that builds the plan through the callback ABI.
struct ProgramState {
  Entry entry = nullptr;
  void *entryContext = nullptr;                     // native entries: the compiled plan
  std::vector<uint64_t> bufferBytes;
  std::vector<std::string> scalarTypes;
  // Bytes of each plan resource by host-entry resource id (temporaries; 0 where unknown: externals,
  // entries written by hand). The inferred graph moves a temporary only when its size is known.
  std::vector<uint64_t> resourceBytes;
  std::shared_ptr<ProgramState> aliasFallback;
  std::shared_ptr<void> owner;                      // keeps compiled state alive
};

std::shared_ptr<Invocation> bind(const std::shared_ptr<ProgramState> &program, std::shared_ptr<Device> device,
                                 const std::vector<Argument> &arguments);
// bind without any device allocation: heaps and library workspaces in the device's static arena
// (workspaces cleared by a kernel on `stream`), launches on the caller's `stream`, code objects
// already resident on the device. Supersedes every earlier static binding on that device.
std::shared_ptr<Invocation> bindStatic(const std::shared_ptr<ProgramState> &program, std::shared_ptr<Device> device,
                                       const std::vector<Argument> &arguments, hipStream_t stream);

int deviceCount();

} // namespace ckl::rt

