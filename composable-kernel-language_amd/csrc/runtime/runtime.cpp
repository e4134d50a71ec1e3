#include "runtime.h"
#include "scratch.h"
#include "../kernels/args.h"

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <set>
#include <stdexcept>

namespace ckl::rt {

void check(hipError_t status, const char *what) {
  if (status != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(status));
}

int deviceCount() {
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess) return 0;
  return count;
}


// ====================================================================== device and buffers
static std::atomic<uint64_t> nextDeviceId{0};

Device::Device(int ordinal_) : ordinal(ordinal_), id(nextDeviceId++) {
  int count = deviceCount();
  if (ordinal < 0 || ordinal >= count) throw std::invalid_argument("HIP device ordinal is not available");
  makeCurrent();
  hipDeviceProp_t props;
  check(hipGetDeviceProperties(&props, ordinal), "hipGetDeviceProperties");
  name = std::string(props.name[0] ? props.name : "AMD GPU") + " (" + props.gcnArchName + ")";
}

Device::~Device() {
  std::lock_guard<std::mutex> lock(moduleMutex);
  for (auto &[_, module] : modules) hipModuleUnload(module);
}

void Device::makeCurrent() const { check(hipSetDevice(ordinal), "hipSetDevice"); }

hipModule_t Device::load(const std::string &identity, const void *image, size_t bytes, bool allowLoad) {
  std::lock_guard<std::mutex> lock(moduleMutex);
  auto found = modules.find(identity);
  if (found != modules.end()) return found->second;
  if (!allowLoad)
    throw std::invalid_argument("code object " + identity + " is not resident on this device; a no-allocation bind "
                                "cannot load it (bind the program once with ckl_bind first)");
  if (!image || !bytes) throw std::invalid_argument("cannot load an empty code object");
  std::map<std::string, KernelSignature> layouts = readKernelSignatures(image, bytes);
  makeCurrent();
  hipModule_t module = nullptr;
  check(hipModuleLoadData(&module, image), "hipModuleLoadData");
  for (auto &[name, layout] : layouts) {
    hipFunction_t function = nullptr;
    if (hipModuleGetFunction(&function, module, name.c_str()) == hipSuccess) signatures[function] = std::move(layout);
    else (void)hipGetLastError();
  }
  modules[identity] = module;
  return module;
}

const KernelSignature &Device::signature(hipFunction_t function) {
  std::lock_guard<std::mutex> lock(moduleMutex);
  auto found = signatures.find(function);
  if (found == signatures.end()) throw std::logic_error("kernel function has no argument layout in its code object");
  return found->second;
}

void Buffer::copyFromHost(const void *data, uint64_t size) const {
  if (size != bytes) throw std::invalid_argument("host buffer byte count does not match device storage");
  device->makeCurrent();
  check(hipMemcpy(reinterpret_cast<void *>(address()), data, size, hipMemcpyHostToDevice), "hipMemcpy(H2D)");
  check(hipDeviceSynchronize(), "hipDeviceSynchronize");
}

void Buffer::copyToHost(void *data, uint64_t size) const {
  if (size != bytes) throw std::invalid_argument("destination must match device storage byte count");
  device->makeCurrent();
  check(hipDeviceSynchronize(), "hipDeviceSynchronize");
  check(hipMemcpy(data, reinterpret_cast<void *>(address()), size, hipMemcpyDeviceToHost), "hipMemcpy(D2H)");
}

std::shared_ptr<Buffer> allocateBuffer(std::shared_ptr<Device> device, uint64_t bytes) {
  if (!bytes) throw std::invalid_argument("HIP allocation size must be nonzero");
  device->makeCurrent();
  void *pointer = nullptr;
  check(hipMalloc(&pointer, bytes), "hipMalloc");
  auto buffer = std::make_shared<Buffer>();
  std::shared_ptr<Device> owner = device;
  buffer->storage = std::shared_ptr<void>(pointer, [owner](void *p) {
    owner->makeCurrent();
    hipFree(p);
  });
  buffer->device = std::move(device);
  buffer->base = reinterpret_cast<uint64_t>(pointer);
  buffer->bytes = bytes;
  return buffer;
}

std::shared_ptr<Buffer> importBuffer(std::shared_ptr<Device> device, uint64_t address, uint64_t bytes) {
  if (!address || !bytes) throw std::invalid_argument("imported HIP buffer requires an address and size");
  auto buffer = std::make_shared<Buffer>();
  buffer->device = std::move(device);
  buffer->base = address;
  buffer->bytes = bytes;
  return buffer;
}

std::shared_ptr<Buffer> sliceBuffer(const std::shared_ptr<Buffer> &parent, uint64_t offset, uint64_t bytes) {
  if (!bytes || offset > parent->bytes || bytes > parent->bytes - offset)
    throw std::out_of_range("HIP buffer slice exceeds its parent view");
  auto buffer = std::make_shared<Buffer>(*parent);
  buffer->offset = parent->offset + offset;
  buffer->bytes = bytes;
  return buffer;
}

// ====================================================================== plans
size_t Plan::addKernel(Launch launch, std::vector<size_t> deps) {
  if (!launch.function) throw std::invalid_argument("kernel plan node requires a resolved function");
  for (unsigned d : launch.grid) if (!d) throw std::invalid_argument("kernel plan node requires positive launch dimensions");
  for (unsigned d : launch.block) if (!d) throw std::invalid_argument("kernel plan node requires positive launch dimensions");
  size_t id = nodes.size();
  for (size_t d : deps)
    if (d >= id) throw std::invalid_argument("kernel dependencies must reference earlier plan nodes");
  nodes.push_back({std::move(launch), std::move(deps)});
  return id;
}

// ExecutionPlan::repeat semantics (lib/Core/ExecutionPlan.cpp:87-117).
Plan Plan::repeat(size_t iterations) const {
  if (!iterations) throw std::invalid_argument("HIP plan repeat count must be nonzero");
  if (nodes.empty()) throw std::invalid_argument("cannot repeat an empty HIP plan");
  std::vector<bool> hasSuccessor(nodes.size(), false);
  for (const PlanNode &n : nodes) for (size_t d : n.dependencies) hasSuccessor[d] = true;
  std::vector<size_t> leaves;
  for (size_t k = 0; k < nodes.size(); ++k) if (!hasSuccessor[k]) leaves.push_back(k);
  Plan out;
  for (size_t it = 0; it < iterations; ++it) {
    size_t offset = out.nodes.size();
    for (size_t k = 0; k < nodes.size(); ++k) {
      std::vector<size_t> deps;
      for (size_t d : nodes[k].dependencies) deps.push_back(offset + d);
      if (it && nodes[k].dependencies.empty())
        for (size_t leaf : leaves) deps.push_back(offset - nodes.size() + leaf);
      out.addKernel(nodes[k].launch, std::move(deps));
    }
  }
  return out;
}

GraphExec::~GraphExec() {
  if (exec) hipGraphExecDestroy(exec);
  if (graph) hipGraphDestroy(graph);
}

void prepareParams(Launch &launch, Device &device) {
  const KernelSignature &layout = device.signature(launch.function);
  const std::vector<KernelArgument> &args = layout.arguments;
  const size_t have = launch.arguments.size();
  auto mismatch = [&](const std::string &why) {
    return std::invalid_argument("argument block of kernel " + launch.name + " (" + std::to_string(have) +
                                 " bytes) does not match its code object's declared arguments: " + why);
  };
  launch.paramOffsets.clear();
  launch.prepared = false;
  if (args.empty()) {
    if (!launch.slotOffsets.empty()) throw mismatch("the kernel takes no arguments");
    launch.prepared = true;
    return;
  }
  if (args.size() == 1 && args[0].offset == 0) {
    // One argument (a struct of the packed fields, or a single field): HIP copies args[0].size
    // bytes from the block; the block is that many bytes plus the 8-byte padding of the packer.
    if (have < args[0].size || have - args[0].size >= 8)
      throw mismatch("one argument of " + std::to_string(args[0].size) + " bytes");
    launch.paramOffsets.push_back(0);
    launch.prepared = true;
    return;
  }
  if (launch.slotOffsets.size() != args.size() || launch.slotSizes.size() != args.size())
    throw mismatch(std::to_string(args.size()) + " arguments, " + std::to_string(launch.slotOffsets.size()) + " packed");
  for (size_t k = 0; k < args.size(); ++k) {
    if (launch.slotOffsets[k] != args[k].offset || launch.slotSizes[k] != args[k].size)
      throw mismatch("argument " + std::to_string(k) + " is " + std::to_string(args[k].size) + " bytes at offset " +
                     std::to_string(args[k].offset) + ", packed " + std::to_string(launch.slotSizes[k]) +
                     " bytes at offset " + std::to_string(launch.slotOffsets[k]));
    if (size_t(args[k].offset) + args[k].size > have) throw mismatch("argument " + std::to_string(k) + " past the block");
    launch.paramOffsets.push_back(args[k].offset);
  }
  launch.prepared = true;
}

void bindVariants(Launch &launch, const std::string &entry) {
  launch.groupFunction = nullptr;
  launch.sharedFunction[0] = launch.sharedFunction[1] = nullptr;
  hipFunction_t group = nullptr;
  if (hipModuleGetFunction(&group, launch.module, (entry + "_group").c_str()) == hipSuccess) launch.groupFunction = group;
  else (void)hipGetLastError();
  for (int m = 2; m <= 3; ++m) {
    hipFunction_t shared = nullptr;
    std::string sharedName = entry + "_shared" + std::to_string(m);
    if (hipModuleGetFunction(&shared, launch.module, sharedName.c_str()) == hipSuccess) launch.sharedFunction[m - 2] = shared;
    else (void)hipGetLastError();
  }
}

namespace {

constexpr size_t kMaxGroup = 4;

// hipModuleLaunchKernel reads explicit argument i from params[i] with the size the code object
// declares; Invocation::prepare has checked that `arguments` holds every one of them.
constexpr size_t kMaxParams = 64;

struct Params {
  void *at[kMaxParams] = {};
  Params(const Launch &launch, const uint8_t *block) {
    if (!launch.prepared || launch.paramOffsets.size() > kMaxParams)
      throw std::logic_error("launch " + launch.name + " has no prepared argument layout");
    for (size_t k = 0; k < launch.paramOffsets.size(); ++k) at[k] = const_cast<uint8_t *>(block + launch.paramOffsets[k]);
  }
};

void launchOne(const Launch &launch, hipStream_t stream) {
  Params params(launch, launch.arguments.data());
  check(hipModuleLaunchKernel(launch.function, launch.grid[0], launch.grid[1], launch.grid[2], launch.block[0],
                              launch.block[1], launch.block[2], launch.shared, stream, params.at, nullptr),
        "hipModuleLaunchKernel");
}

void launchOrdinary(const Plan &plan, hipStream_t stream) {
  for (const PlanNode &node : plan.nodes) launchOne(node.launch, stream);
}

// A unit of the inferred graph: one dispatch, a chain of dependent dispatches run by a chain
// entry point, or sibling units of one family executed by the family's group entry point (each
// member keeps its own grid range).

// Group<Args> block of sibling launches. A shared-operand launch (`shared`) runs one member's grid
// in which every workgroup serves all members; otherwise member m owns its own range of blocks.
Launch groupLaunch(const std::vector<const Launch *> &members, bool shared) {
  const Launch &first = *members[0];
  Launch out = first;
  out.function = shared ? first.sharedFunction[members.size() - 2] : first.groupFunction;
  out.groupFunction = nullptr;
  out.sharedFunction[0] = out.sharedFunction[1] = nullptr;
  out.name = first.name + (shared ? "_shared" + std::to_string(members.size()) : std::string("_group"));
  size_t stride = first.arguments.size();
  std::vector<uint8_t> blob(kMaxGroup * stride + 4 * (kMaxGroup + 1) + 4, 0);
  int32_t start = 0;
  std::vector<int32_t> starts;
  for (size_t k = 0; k < members.size(); ++k) {
    std::memcpy(blob.data() + k * stride, members[k]->arguments.data(), stride);
    starts.push_back(start);
    start += int32_t(members[k]->grid[0]);
  }
  starts.push_back(start);
  while (starts.size() < kMaxGroup + 1) starts.push_back(start);
  std::memcpy(blob.data() + kMaxGroup * stride, starts.data(), 4 * (kMaxGroup + 1));
  int32_t count = int32_t(members.size());
  std::memcpy(blob.data() + kMaxGroup * stride + 4 * (kMaxGroup + 1), &count, 4);
  blob.resize((blob.size() + 7) & ~size_t(7), 0);
  out.arguments = std::move(blob);
  out.grid[0] = shared ? first.grid[0] : unsigned(start);
  // A shared-operand linear passes the accumulators of up to kLinearEpilogueBytes worth of members
  // through LDS at once (linearEpilogueMembers, csrc/kernels/args.h); a member alone needs
  // `first.shared` bytes.
  if (shared && first.shared)
    out.shared = unsigned(std::min<size_t>(members.size(), std::max<size_t>(1, ckl::kernels::kLinearEpilogueBytes / first.shared)) * first.shared);
  return out;
}

// The inferred lowering: library chains are contracted into single units, units are levelled by
// their longest dependency path, and same-level units of one family become one group launch.
// `chains` and the patched launches `overrides` were found on one iteration of `iterations` (the
// plan's nodes repeat with that period).
std::vector<Unit> groupPlan(const Plan &plan, const std::vector<Chain> &found, const std::map<size_t, Launch> &overrides,
                            size_t iterations) {
  const size_t n = plan.nodes.size();
  const size_t period = n / iterations;
  std::vector<Chain> chains;
  for (size_t it = 0; it < iterations; ++it)
    for (const Chain &c : found) {
      Chain copy = c;
      for (size_t &m : copy.members) m += it * period;
      chains.push_back(std::move(copy));
    }
  std::vector<int> chainAt(n, -1);
  for (size_t c = 0; c < chains.size(); ++c) for (size_t m : chains[c].members) chainAt[m] = int(c);
  std::vector<size_t> unitOf(n);
  std::vector<Unit> base;
  for (size_t k = 0; k < n; ++k) {
    if (chainAt[k] >= 0) {
      const Chain &c = chains[size_t(chainAt[k])];
      if (c.members[0] != k) { unitOf[k] = unitOf[c.members[0]]; continue; }   // members ascend
      unitOf[k] = base.size();
      base.push_back({c.members, c.launch});
    } else {
      unitOf[k] = base.size();
      auto patched = overrides.find(k % period);
      base.push_back({{k}, patched != overrides.end() ? patched->second : plan.nodes[k].launch});
    }
  }
  const size_t units = base.size();
  std::vector<std::vector<size_t>> succ(units);
  std::vector<size_t> indegree(units, 0), level(units, 0);
  for (size_t k = 0; k < n; ++k)
    for (size_t d : plan.nodes[k].dependencies)
      if (unitOf[d] != unitOf[k]) { succ[unitOf[d]].push_back(unitOf[k]); ++indegree[unitOf[k]]; }
  std::vector<size_t> ready, order;
  for (size_t u = 0; u < units; ++u) if (!indegree[u]) ready.push_back(u);
  while (!ready.empty()) {
    size_t u = ready.back();
    ready.pop_back();
    order.push_back(u);
    for (size_t s : succ[u]) {
      level[s] = std::max(level[s], level[u] + 1);
      if (!--indegree[s]) ready.push_back(s);
    }
  }
  if (order.size() != units) throw std::logic_error("contracted inferred graph has a cycle");
  size_t maxLevel = 0;
  for (size_t u = 0; u < units; ++u) maxLevel = std::max(maxLevel, level[u]);
  std::vector<std::vector<size_t>> byLevel(maxLevel + 1);
  for (size_t u = 0; u < units; ++u) byLevel[level[u]].push_back(u);
  std::vector<Unit> out;
  for (const auto &members : byLevel) {
    std::vector<std::vector<size_t>> buckets;
    for (size_t u : members) {
      const Launch &l = base[u].launch;
      bool groupable = l.groupFunction && l.grid[1] == 1 && l.grid[2] == 1;
      bool placed = false;
      if (groupable)
        for (auto &bucket : buckets) {
          const Launch &b = base[bucket[0]].launch;
          if (bucket.size() < kMaxGroup && b.function == l.function && b.groupFunction &&
              std::equal(b.block, b.block + 3, l.block) && b.shared == l.shared &&
              b.arguments.size() == l.arguments.size() && b.grid[1] == 1 && b.grid[2] == 1) {
            bucket.push_back(u);
            placed = true;
            break;
          }
        }
      if (!placed) buckets.push_back({u});
    }
    for (auto &bucket : buckets) {
      if (bucket.size() == 1) {
        out.push_back(std::move(base[bucket[0]]));
        continue;
      }
      Unit g;
      std::vector<const Launch *> launches;
      for (size_t u : bucket) {
        g.members.insert(g.members.end(), base[u].members.begin(), base[u].members.end());
        launches.push_back(&base[u].launch);
      }
      const bool shared = launches.size() <= 3 && launches[0]->sharedFunction[launches.size() - 2] &&
                          sharesOperands(launches);
      g.launch = groupLaunch(launches, shared);
      out.push_back(std::move(g));
    }
  }
  return out;
}

std::unique_ptr<GraphExec> captureUnits(const std::vector<Launch> &launches, hipStream_t stream) {
  auto out = std::make_unique<GraphExec>();
  for (const Launch &l : launches) out->storage.push_back(l.arguments);
  check(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
  try {
    for (size_t k = 0; k < launches.size(); ++k) {
      const Launch &l = launches[k];
      Params params(l, out->storage[k].data());
      check(hipModuleLaunchKernel(l.function, l.grid[0], l.grid[1], l.grid[2], l.block[0], l.block[1], l.block[2],
                                  l.shared, stream, params.at, nullptr),
            "hipModuleLaunchKernel(capture)");
    }
  } catch (...) {
    hipGraph_t abandoned = nullptr;
    hipStreamEndCapture(stream, &abandoned);
    if (abandoned) hipGraphDestroy(abandoned);
    throw;
  }
  check(hipStreamEndCapture(stream, &out->graph), "hipStreamEndCapture");
  size_t count = 0;
  check(hipGraphGetNodes(out->graph, nullptr, &count), "hipGraphGetNodes");
  out->nodeCount = count;
  check(hipGraphInstantiate(&out->exec, out->graph, nullptr, nullptr, 0), "hipGraphInstantiate(captured)");
  return out;
}

// Explicit graph with one kernel node per unit and the units' dependency edges, transitively
// reduced at unit level (contracting chains and merging siblings can make plan edges redundant).
std::unique_ptr<GraphExec> explicitGraph(const Plan &plan, const std::vector<Unit> &units) {
  auto out = std::make_unique<GraphExec>();
  const size_t n = units.size();
  std::vector<size_t> unitOf(plan.nodes.size());
  for (size_t u = 0; u < n; ++u) for (size_t m : units[u].members) unitOf[m] = u;
  // Units arrive in a topological order (groupPlan levels them; one node per dispatch keeps plan
  // order), so every edge goes from a lower to a higher unit index.
  std::vector<std::vector<size_t>> preds(n);
  for (size_t u = 0; u < n; ++u) {
    for (size_t m : units[u].members)
      for (size_t d : plan.nodes[m].dependencies) {
        size_t du = unitOf[d];
        if (du == u) continue;
        if (du > u) throw std::logic_error("inferred graph units are not in topological order");
        preds[u].push_back(du);
      }
    std::sort(preds[u].begin(), preds[u].end());
    preds[u].erase(std::unique(preds[u].begin(), preds[u].end()), preds[u].end());
  }
  // reach[u]: the units in [u - span, u) that u depends on, directly or not, where span is the
  // longest distance from a unit to a predecessor. That window suffices: a predecessor p of u is
  // redundant when a later predecessor q reaches it, and then q - span <= u - span <= p < q. A
  // repeated plan's edges reach at most one step back, so the sets stay a few words long however
  // many steps one graph holds (dense sets would cost n^2/8 bytes).
  size_t span = 1;
  for (size_t u = 0; u < n; ++u)
    if (!preds[u].empty()) span = std::max(span, u - preds[u].front());
  const size_t words = span / 64 + 2;
  auto base = [&](size_t u) { return (u > span ? u - span : 0) / 64; };   // first word of u's window
  std::vector<uint64_t> reach(n * words, 0);
  std::vector<std::vector<size_t>> reduced(n);
  for (size_t u = 0; u < n; ++u) {
    uint64_t *mine = &reach[u * words];
    const size_t first = base(u);
    // A predecessor is kept when no later predecessor already reaches it (scan in descending order).
    for (auto it = preds[u].rbegin(); it != preds[u].rend(); ++it) {
      const size_t p = *it;
      uint64_t &word = mine[p / 64 - first];
      if (!(word >> (p % 64) & 1)) reduced[u].push_back(p);
      word |= uint64_t(1) << (p % 64);
      const uint64_t *theirs = &reach[p * words];
      const size_t from = base(p);                 // <= first: p's window starts no later than u's
      for (size_t w = first; w <= (p ? (p - 1) / 64 : 0) && w - from < words; ++w) mine[w - first] |= theirs[w - from];
    }
  }
  check(hipGraphCreate(&out->graph, 0), "hipGraphCreate");
  std::vector<hipGraphNode_t> handles(n);
  for (const Unit &u : units) out->storage.push_back(u.launch.arguments);
  for (size_t u = 0; u < n; ++u) {
    std::vector<hipGraphNode_t> deps;
    for (size_t p : reduced[u]) deps.push_back(handles[p]);
    const Launch &l = units[u].launch;
    Params params(l, out->storage[u].data());
    hipKernelNodeParams p{};
    p.func = reinterpret_cast<void *>(l.function);
    p.gridDim = dim3(l.grid[0], l.grid[1], l.grid[2]);
    p.blockDim = dim3(l.block[0], l.block[1], l.block[2]);
    p.sharedMemBytes = l.shared;
    p.kernelParams = params.at;
    check(hipGraphAddKernelNode(&handles[u], out->graph, deps.data(), deps.size(), &p), "hipGraphAddKernelNode");
    out->edgeCount += deps.size();
  }
  out->nodeCount = n;
  out->handles = handles;
  check(hipGraphInstantiate(&out->exec, out->graph, nullptr, nullptr, 0), "hipGraphInstantiate");
  return out;
}

} // namespace

// ====================================================================== invocation
Invocation::Invocation(std::shared_ptr<ProgramState> program_, std::shared_ptr<Device> device_, hipStream_t external)
    : program(std::move(program_)), device(std::move(device_)) {
  device->makeCurrent();
  if (external) {
    stream = external;
    ownsStream = false;
  } else {
    check(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "hipStreamCreateWithFlags");
  }
}

Invocation::~Invocation() {
  graphs.clear();
  if (stream) {
    device->makeCurrent();
    hipStreamSynchronize(stream);
    if (ownsStream) hipStreamDestroy(stream);
  }
}

void Invocation::placeHeaps() {
  if (pendingHeaps.empty()) return;
  uint64_t total = 0;
  std::vector<uint64_t> offsets;
  for (const auto &[id, bytes] : pendingHeaps) {
    offsets.push_back(total);
    total += (bytes + 255) & ~uint64_t(255);
  }
  device->makeCurrent();
  std::shared_ptr<Buffer> arena;
  if (staticArena) {
    arena = importBuffer(device, carve(total), total);
  } else {
    arena = allocateBuffer(device, total);
    ++allocations;
  }
  // Library workspaces keep state that must read zero (zero pages, completion counters); the
  // whole range is cleared once, before any launch of this invocation.
  staticScratchClear(arena->address(), total, stream);
  for (size_t k = 0; k < pendingHeaps.size(); ++k)
    heaps[pendingHeaps[k].first] = sliceBuffer(arena, offsets[k], pendingHeaps[k].second);
  pendingHeaps.clear();
}

uint64_t Invocation::carve(uint64_t bytes) {
  const uint64_t start = (arenaUsed + 255) & ~uint64_t(255);
  if (!bytes || start > arenaLimit || bytes > arenaLimit - start) {
    arenaExceeded = true;
    throw std::invalid_argument("the program needs more than the static arena's " + std::to_string(arenaLimit) +
                                " bytes (CKL_STATIC_SCRATCH_BYTES) of heaps and workspaces");
  }
  arenaUsed = start + bytes;
  return arenaBase + start;
}

namespace {
constexpr int kMaxStaticDevices = 64;
std::array<std::atomic<uint64_t>, kMaxStaticDevices> staticEpochs{};
} // namespace

void Invocation::requireCurrent() const {
  if (staticArena && staticEpochs[size_t(device->ordinal)].load() != epoch)
    throw std::invalid_argument("this invocation's static arena was taken over by a later ckl_bind_static on the same "
                                "device; bind it again");
}

void Invocation::validate(int mode, uint64_t batch) const {
  requireCurrent();
  if (mode < kOrdinary || mode > kInferredStream || !batch || plan.nodes.empty() ||
      batch > 1000000 / plan.nodes.size())
    throw std::invalid_argument("invalid execution mode or batch exceeds one million kernel nodes");
}

// The units of a graph mode: ordinary launches (modes 2 and 3: one per dispatch) or the inferred
// lowering (modes 1, 4 and 5: chains contracted, siblings of one family merged, units levelled by
// DAG depth).
std::vector<Unit> Invocation::buildUnits(int mode, uint64_t batch, const Plan &repeated) {
  std::vector<Unit> units;
  if (mode == kCapture || mode == kBranches) {
    for (size_t k = 0; k < repeated.nodes.size(); ++k) units.push_back({{k}, repeated.nodes[k].launch});
    return units;
  }
  if (!relocationDecided) {
    relocationDecided = true;
    relocateForChains();
    if (batch == 1) return buildUnits(mode, batch, plan);      // the repeated plan predates the move
    return buildUnits(mode, batch, plan.repeat(batch));
  }
  std::vector<Chain> chains = findChains(plan, temporaryResources);
  std::map<size_t, Launch> deferred = deferCombines(plan, temporaryResources, chains);
  units = groupPlan(repeated, chains, deferred, batch);
  for (Unit &u : units) prepareParams(u.launch, *device);
  return units;
}

GraphExec &Invocation::graphFor(int mode, uint64_t batch) {
  auto &slot = graphs[{mode, batch}];
  if (!slot) {
    Plan repeated = batch == 1 ? plan : plan.repeat(batch);
    std::vector<Unit> units = buildUnits(mode, batch, repeated);
    std::vector<Launch> launches;
    for (const Unit &u : units) launches.push_back(u.launch);
    // Mode 3 is the reference's inferred graph (one kernel node per dispatch, reduced DAG edges)
    // and mode 1 the units' DAG as an explicit graph; modes 2 and 4 capture their launch chain;
    // mode 5 keeps only the launch chain, issued on the stream at every execution.
    if (mode == kInferred || mode == kBranches) slot = explicitGraph(repeated, units);
    else if (mode == kCapture || mode == kContractedCapture) slot = captureUnits(launches, stream);
    else {
      slot = std::make_unique<GraphExec>();
      slot->nodeCount = launches.size();
    }
    if (mode != kInferredStream) ++instantiations;
    slot->launches = std::move(launches);
    for (Unit &u : units) slot->members.push_back(std::move(u.members));
  }
  return *slot;
}

void Invocation::execute(int mode, uint64_t batch) {
  device->makeCurrent();
  if (mode == kOrdinary) {
    for (uint64_t k = 0; k < batch; ++k) launchOrdinary(plan, stream);
    return;
  }
  GraphExec &graph = graphFor(mode, batch);
  if (mode == kInferredStream)
    for (const Launch &l : graph.launches) launchOne(l, stream);
  else
    check(hipGraphLaunch(graph.exec, stream), "hipGraphLaunch");
}

size_t Invocation::graphNodeCount(int mode, uint64_t batch) {
  std::lock_guard<std::mutex> lock(runMutex);
  validate(mode, batch);
  if (mode == kOrdinary) return plan.nodes.size() * batch;
  return graphFor(mode, batch).nodeCount;
}

size_t Invocation::graphEdgeCount(int mode, uint64_t batch) {
  std::lock_guard<std::mutex> lock(runMutex);
  validate(mode, batch);
  if (mode == kOrdinary) return 0;
  return graphFor(mode, batch).edgeCount;
}

void Invocation::run(int mode, uint64_t batch) {
  std::lock_guard<std::mutex> lock(runMutex);
  validate(mode, batch);
  execute(mode, batch);
  check(hipStreamSynchronize(stream), "hipStreamSynchronize");
}

std::array<double, 2> runConcurrently(const std::vector<Invocation *> &requests, int mode, uint64_t iterations,
                                      uint64_t batch, bool serial) {
  if (requests.empty() || !iterations) throw std::invalid_argument("no requests or no iterations");
  std::vector<Invocation *> order(requests);
  std::sort(order.begin(), order.end());
  if (std::adjacent_find(order.begin(), order.end()) != order.end())
    throw std::invalid_argument("an invocation appears twice among the requests");
  for (Invocation *r : order) {
    if (!r) throw std::invalid_argument("null invocation among the requests");
    if (r->device != order[0]->device) throw std::invalid_argument("requests on different devices");
  }
  // Locked in address order, so two bursts over overlapping sets cannot deadlock.
  std::vector<std::unique_lock<std::mutex>> locks;
  for (Invocation *r : order) locks.emplace_back(r->runMutex);
  for (Invocation *r : requests) r->validate(mode, batch);
  Device &device = *requests[0]->device;
  device.makeCurrent();
  for (Invocation *r : requests) {
    check(hipStreamSynchronize(r->stream), "hipStreamSynchronize");
    if (mode) r->graphFor(mode, batch);      // graphs built outside the timed burst
  }
  std::vector<hipEvent_t> events(requests.size() + 2, nullptr);
  auto release = [&] {
    for (hipEvent_t e : events)
      if (e) hipEventDestroy(e);
  };
  try {
    for (hipEvent_t &e : events) check(hipEventCreate(&e), "hipEventCreate");
    hipStream_t first = requests[0]->stream;
    using Clock = std::chrono::steady_clock;
    auto wall = Clock::now();
    check(hipEventRecord(events[0], first), "hipEventRecord");
    for (size_t k = 1; k < requests.size(); ++k)
      check(hipStreamWaitEvent(requests[k]->stream, events[0], 0), "hipStreamWaitEvent");
    if (serial) {
      for (size_t k = 0; k < requests.size(); ++k) {
        for (uint64_t i = 0; i < iterations; ++i) requests[k]->execute(mode, batch);
        check(hipStreamSynchronize(requests[k]->stream), "hipStreamSynchronize");
      }
    } else {
      for (uint64_t i = 0; i < iterations; ++i)
        for (Invocation *r : requests) r->execute(mode, batch);
    }
    for (size_t k = 1; k < requests.size(); ++k) {
      check(hipEventRecord(events[k + 1], requests[k]->stream), "hipEventRecord");
      check(hipStreamWaitEvent(first, events[k + 1], 0), "hipStreamWaitEvent");
    }
    check(hipEventRecord(events[1], first), "hipEventRecord");
    check(hipEventSynchronize(events[1]), "hipEventSynchronize");
    const double wallUs = std::chrono::duration<double, std::micro>(Clock::now() - wall).count();
    float elapsed = 0;
    check(hipEventElapsedTime(&elapsed, events[0], events[1]), "hipEventElapsedTime");
    for (Invocation *r : requests) check(hipStreamSynchronize(r->stream), "hipStreamSynchronize");
    release();
    return {wallUs, double(elapsed) * 1000.0};
  } catch (...) {
    release();
    throw;
  }
}

// The program arguments' device addresses (buffers, 0 for scalars) and scalar bytes, checked
// against the compiled signature; the buffers are appended to `keep`.
static void packArguments(const ProgramState &program, const Device *device, const std::vector<Argument> &arguments,
                          std::vector<uint64_t> &addresses, std::vector<uint64_t> &scalars,
                          std::vector<std::shared_ptr<Buffer>> &keep) {
  const size_t count = arguments.size();
  if (count != program.bufferBytes.size()) throw std::invalid_argument("incorrect program argument count");
  addresses.assign(count, 0);
  scalars.assign(count, 0);
  for (size_t k = 0; k < count; ++k) {
    const Argument &a = arguments[k];
    if (program.bufferBytes[k]) {
      if (a.kind != 0 || !a.buffer || a.buffer->device.get() != device || a.buffer->bytes < program.bufferBytes[k])
        throw std::invalid_argument("buffer device or size does not match compiled signature");
      addresses[k] = a.buffer->address();
      keep.push_back(a.buffer);
    } else {
      const std::string &type = program.scalarTypes[k];
      auto store = [&](auto value) { std::memcpy(&scalars[k], &value, sizeof(value)); };
      if (type == "i32" && a.kind == 1) store(int32_t(a.integer));
      else if (type == "i64" && a.kind == 2) store(int64_t(a.integer));
      else if (type == "f32" && a.kind == 3) store(float(a.real));
      else if (type == "f64" && a.kind == 4) store(double(a.real));
      else throw std::invalid_argument("argument type does not match compiled signature");
    }
  }
}

// Whether any two buffer arguments' byte ranges overlap (the fused program's fallback condition,
// lib/Runtime/NvidiaProgram.cpp:191-205).
static bool argumentsOverlap(const ProgramState &program, const std::vector<uint64_t> &addresses) {
  const size_t count = addresses.size();
  for (size_t i = 0; i < count; ++i)
    for (size_t j = i + 1; j < count; ++j) {
      if (!program.bufferBytes[i] || !program.bufferBytes[j]) continue;
      const bool overlap = addresses[i] <= addresses[j] ? addresses[j] - addresses[i] < program.bufferBytes[i]
                                                        : addresses[i] - addresses[j] < program.bufferBytes[j];
      if (overlap) return true;
    }
  return false;
}

static std::shared_ptr<Invocation> bindWith(const std::shared_ptr<ProgramState> &programIn, std::shared_ptr<Device> device,
                                            const std::vector<Argument> &arguments, bool arena, hipStream_t stream);

std::shared_ptr<Invocation> bind(const std::shared_ptr<ProgramState> &program, std::shared_ptr<Device> device,
                                 const std::vector<Argument> &arguments) {
  return bindWith(program, std::move(device), arguments, false, nullptr);
}

std::shared_ptr<Invocation> bindStatic(const std::shared_ptr<ProgramState> &program, std::shared_ptr<Device> device,
                                       const std::vector<Argument> &arguments, hipStream_t stream) {
  if (!device) throw std::invalid_argument("program binding requires a device");
  if (!stream) throw std::invalid_argument("a no-allocation bind needs the caller's stream");
  if (device->ordinal < 0 || device->ordinal >= kMaxStaticDevices)
    throw std::invalid_argument("HIP device ordinal out of range for the static arena");
  return bindWith(program, std::move(device), arguments, true, stream);
}

uint64_t Invocation::graphInstantiations() {
  std::lock_guard<std::mutex> lock(runMutex);
  return instantiations;
}

void Invocation::rebind(const std::vector<Argument> &arguments) {
  std::lock_guard<std::mutex> lock(runMutex);
  requireCurrent();
  if (!requested) throw std::invalid_argument("this invocation was not bound from program arguments");
  // A resource bound from an address the host entry did not take from the packed program
  // arguments cannot be followed to its new buffer.
  for (size_t id = 0; id < externalResources.size(); ++id)
    if (externalResources[id] && (id >= resourceArgument.size() || resourceArgument[id] < 0))
      throw std::invalid_argument("resource " + std::to_string(id) + " was bound from an address outside the packed "
                                  "program arguments, so a rebind cannot move it; bind again");
  std::vector<uint64_t> addresses, scalars;
  std::vector<std::shared_ptr<Buffer>> keep;
  packArguments(*requested, device.get(), arguments, addresses, scalars, keep);
  if (scalars != argumentScalars)
    throw std::invalid_argument("a rebind keeps the scalar arguments; bind again to change them");
  const bool fallback = requested->aliasFallback && argumentsOverlap(*requested, addresses);
  if ((fallback ? requested->aliasFallback : requested) != program)
    throw std::invalid_argument("the new buffers overlap differently (fused or unfused program); bind again");
  for (int64_t k : resourceArgument)
    if (k >= 0 && size_t(k) >= addresses.size()) throw std::logic_error("resource of an unknown argument");
  // Move every resolved argument address by its buffer's displacement.
  std::vector<uint64_t> delta(addresses.size());
  for (size_t k = 0; k < addresses.size(); ++k) delta[k] = addresses[k] - argumentAddresses[k];
  for (size_t id = 0; id < resourceArgument.size(); ++id)
    if (resourceArgument[id] >= 0) resources[id] += delta[size_t(resourceArgument[id])];
  for (PlanNode &node : plan.nodes) {
    Launch &l = node.launch;
    for (size_t s = 0; s < l.slotResources.size(); ++s) {
      const int64_t id = l.slotResources[s];
      if (id < 0 || size_t(id) >= resourceArgument.size() || resourceArgument[size_t(id)] < 0) continue;
      if (l.slotSizes[s] != 8) throw std::logic_error("an address slot is not 8 bytes");
      uint64_t value;
      std::memcpy(&value, l.arguments.data() + l.slotOffsets[s], 8);
      value += delta[size_t(resourceArgument[size_t(id)])];
      std::memcpy(l.arguments.data() + l.slotOffsets[s], &value, 8);
    }
  }
  argumentAddresses = addresses;
  buffers = std::move(keep);
  device->makeCurrent();
  check(hipStreamSynchronize(stream), "hipStreamSynchronize");
  // Explicit graphs: new unit launches from the moved plan; same structure -> update in place.
  for (auto it = graphs.begin(); it != graphs.end();) {
    const int mode = it->first.first;
    const uint64_t batch = it->first.second;
    GraphExec &g = *it->second;
    bool kept = false;
    if (mode == kInferredStream || ((mode == kInferred || mode == kBranches) && g.exec && g.handles.size() == g.launches.size())) {
      Plan repeated = batch == 1 ? plan : plan.repeat(batch);
      std::vector<Unit> units = buildUnits(mode, batch, repeated);
      bool same = units.size() == g.launches.size();
      for (size_t u = 0; same && u < units.size(); ++u) {
        const Launch &a = units[u].launch, &b = g.launches[u];
        same = a.function == b.function && a.shared == b.shared && units[u].members == g.members[u] &&
               std::equal(a.grid, a.grid + 3, b.grid) && std::equal(a.block, a.block + 3, b.block);
      }
      if (same) {
        if (mode != kInferredStream) {
          g.storage.resize(units.size());
          for (size_t u = 0; u < units.size(); ++u) {
            const Launch &l = units[u].launch;
            g.storage[u] = l.arguments;
            Params params(l, g.storage[u].data());
            hipKernelNodeParams p{};
            p.func = reinterpret_cast<void *>(l.function);
            p.gridDim = dim3(l.grid[0], l.grid[1], l.grid[2]);
            p.blockDim = dim3(l.block[0], l.block[1], l.block[2]);
            p.sharedMemBytes = l.shared;
            p.kernelParams = params.at;
            check(hipGraphExecKernelNodeSetParams(g.exec, g.handles[u], &p), "hipGraphExecKernelNodeSetParams");
          }
        }
        for (size_t u = 0; u < units.size(); ++u) g.launches[u] = std::move(units[u].launch);
        kept = true;
      }
    }
    if (kept) ++it;
    else it = graphs.erase(it);
  }
}

std::array<double, 3> Invocation::benchmark(int mode, uint64_t iterations, uint64_t batch) {
  if (!iterations) throw std::invalid_argument("benchmark iterations must be positive");
  std::lock_guard<std::mutex> lock(runMutex);
  validate(mode, batch);
  std::array<double, 3> result{};
  using Clock = std::chrono::steady_clock;
  device->makeCurrent();
  check(hipStreamSynchronize(stream), "hipStreamSynchronize");
  auto setup = Clock::now();
  if (mode) graphFor(mode, batch);
  result[2] = std::chrono::duration<double, std::milli>(Clock::now() - setup).count();
  hipEvent_t start = nullptr, stop = nullptr;
  check(hipEventCreate(&start), "hipEventCreate");
  try {
    check(hipEventCreate(&stop), "hipEventCreate");
    check(hipEventRecord(start, stream), "hipEventRecord");
    auto wall = Clock::now();
    for (uint64_t k = 0; k < iterations; ++k) execute(mode, batch);
    check(hipEventRecord(stop, stream), "hipEventRecord");
    check(hipEventSynchronize(stop), "hipEventSynchronize");
    auto wallStop = Clock::now();
    float elapsed = 0;
    check(hipEventElapsedTime(&elapsed, start, stop), "hipEventElapsedTime");
    result[0] = double(elapsed) * 1000.0 / double(iterations) / double(batch);
    result[1] = std::chrono::duration<double, std::micro>(wallStop - wall).count() / double(iterations) / double(batch);
  } catch (...) {
    hipEventDestroy(start);
    if (stop) hipEventDestroy(stop);
    throw;
  }
  hipEventDestroy(start);
  hipEventDestroy(stop);
  return result;
}

std::array<uint64_t, 3> Invocation::memory() const {
  std::array<uint64_t, 3> out{0, 0, allocations};
  for (const auto &h : heaps)
    if (h) out[0] += h->bytes;
  for (const auto &w : workspaces) out[1] += w->bytes;
  if (relocation) out[1] += relocation->bytes;
  return out;
}

// Storage reuse may put a dispatch's output where an input of the dispatch before it lived: dead
// in dispatch order, but live inside a chain that runs both dispatches as one launch, whose
// workgroups would then overwrite input rows other workgroups have not read yet. For the chains
// refused for that reason, the temporary of each overlapping pair that the plan uses later (the
// one placed into the other's dead storage) moves to a separate allocation of this invocation,
// provided a trial with the moved addresses shows more chains are then taken. Temporaries hold
// nothing from one execution to the next, so every run mode may use the moved addresses; the
// plan's heaps and offsets are unchanged. Static bindings allocate nothing and keep the plan.
void Invocation::relocateForChains() {
  const std::vector<uint64_t> &bytes = program->resourceBytes;
  if (staticArena || bytes.empty()) return;
  // Dispatches a set of chains saves (each chain runs its members as one launch).
  auto saved = [](const std::vector<Chain> &chains) {
    size_t out = 0;
    for (const Chain &c : chains) out += c.members.size() - 1;
    return out;
  };
  std::vector<std::vector<size_t>> refused;
  const size_t before = saved(findChains(plan, temporaryResources, &refused));
  if (refused.empty()) return;
  std::vector<size_t> first(resources.size(), plan.nodes.size());    // first plan node using each resource
  for (size_t k = plan.nodes.size(); k-- > 0;)
    for (int64_t id : plan.nodes[k].launch.slotResources)
      if (id >= 0 && size_t(id) < first.size()) first[size_t(id)] = k;
  auto movable = [&](int64_t id) {
    return id >= 0 && size_t(id) < bytes.size() && size_t(id) < temporaryResources.size() &&
           temporaryResources[size_t(id)] && bytes[size_t(id)] > 0;
  };
  std::set<int64_t> moved;
  for (const std::vector<size_t> &members : refused) {
    std::set<int64_t> ids;
    for (size_t m : members)
      for (int64_t id : plan.nodes[m].launch.slotResources)
        if (movable(id)) ids.insert(id);
    for (int64_t a : ids)
      for (int64_t b : ids) {
        if (a >= b || first[size_t(a)] == first[size_t(b)]) continue;
        const uint64_t a0 = resources[size_t(a)], b0 = resources[size_t(b)];
        if (a0 + bytes[size_t(a)] <= b0 || b0 + bytes[size_t(b)] <= a0) continue;
        moved.insert(first[size_t(a)] > first[size_t(b)] ? a : b);
      }
  }
  // The plan with `set` moved to consecutive 256-byte-aligned ranges from `base`.
  auto movedTo = [&](const std::set<int64_t> &set, uint64_t base, std::map<int64_t, uint64_t> *offsets) {
    std::map<int64_t, uint64_t> offset;
    uint64_t total = 0;
    for (int64_t id : set) {
      offset[id] = total;
      total += (bytes[size_t(id)] + 255) & ~uint64_t(255);
    }
    Plan out = plan;
    for (PlanNode &node : out.nodes) {
      Launch &l = node.launch;
      for (size_t s = 0; s < l.slotResources.size(); ++s) {
        auto it = offset.find(l.slotResources[s]);
        if (it == offset.end()) continue;
        if (l.slotSizes[s] != 8) throw std::logic_error("an address slot is not 8 bytes");
        uint64_t value;
        std::memcpy(&value, l.arguments.data() + l.slotOffsets[s], 8);
        value = value - resources[size_t(it->first)] + base + it->second;
        std::memcpy(l.arguments.data() + l.slotOffsets[s], &value, 8);
      }
    }
    if (offsets) *offsets = std::move(offset);
    return out;
  };
  // Trials only compare addresses: a base above every device address cannot overlap a buffer.
  const uint64_t trialBase = uint64_t(1) << 56;
  auto gain = [&](const std::set<int64_t> &set) { return saved(findChains(movedTo(set, trialBase, nullptr), temporaryResources)); };
  const size_t best = moved.empty() ? before : gain(moved);
  if (best <= before) return;
  // Keep only what the gain needs: drop each temporary whose move does not contribute.
  for (auto it = moved.begin(); it != moved.end();) {
    std::set<int64_t> fewer = moved;
    fewer.erase(*it);
    if (gain(fewer) >= best) it = moved.erase(it);
    else ++it;
  }
  std::map<int64_t, uint64_t> offset;
  uint64_t total = 0;
  for (int64_t id : moved) total += (bytes[size_t(id)] + 255) & ~uint64_t(255);
  if (const char *v = std::getenv("CKL_CHAIN_TRACE"); v && std::strcmp(v, "1") == 0) {
    std::fprintf(stderr, "[ckl chains] %zu chains refused for overlap; moving %zu temporaries (%llu bytes):", refused.size(),
                 moved.size(), (unsigned long long)total);
    for (int64_t id : moved) std::fprintf(stderr, " %lld", (long long)id);
    std::fprintf(stderr, "; dispatches saved %zu -> %zu\n", before, best);
  }
  relocation = allocateBuffer(device, total);
  ++allocations;
  plan = movedTo(moved, relocation->address(), &offset);
  for (const auto &[id, at] : offset) resources[size_t(id)] = relocation->address() + at;
}

double Invocation::timeNode(size_t index, uint64_t iterations) {
  std::lock_guard<std::mutex> lock(runMutex);
  requireCurrent();
  return timeLaunch(plan.nodes.at(index).launch, iterations);
}

GraphExec &Invocation::inferredUnits() {
  validate(kInferred, 1);
  return graphFor(kInferred, 1);
}

size_t Invocation::unitCount() {
  std::lock_guard<std::mutex> lock(runMutex);
  return inferredUnits().launches.size();
}

const std::string &Invocation::unitName(size_t unit) {
  std::lock_guard<std::mutex> lock(runMutex);
  return inferredUnits().launches.at(unit).name;
}

const std::vector<size_t> &Invocation::unitMembers(size_t unit) {
  std::lock_guard<std::mutex> lock(runMutex);
  return inferredUnits().members.at(unit);
}

double Invocation::timeUnit(size_t unit, uint64_t iterations) {
  std::lock_guard<std::mutex> lock(runMutex);
  return timeLaunch(inferredUnits().launches.at(unit), iterations);
}

std::vector<double> Invocation::profileUnits(uint64_t repeats) {
  if (!repeats) throw std::invalid_argument("repeats must be positive");
  std::lock_guard<std::mutex> lock(runMutex);
  GraphExec &units = inferredUnits();
  device->makeCurrent();
  const size_t n = units.launches.size();
  std::vector<std::vector<double>> prefix(n + 1);
  hipEvent_t start = nullptr, stop = nullptr;
  check(hipEventCreate(&start), "hipEventCreate");
  try {
    check(hipEventCreate(&stop), "hipEventCreate");
    for (uint64_t r = 0; r < repeats; ++r)
      for (size_t k = 0; k <= n; ++k) {
        check(hipStreamSynchronize(stream), "hipStreamSynchronize");
        check(hipEventRecord(start, stream), "hipEventRecord");
        for (size_t u = 0; u < k; ++u) launchOne(units.launches[u], stream);
        check(hipEventRecord(stop, stream), "hipEventRecord");
        check(hipEventSynchronize(stop), "hipEventSynchronize");
        float ms = 0;
        check(hipEventElapsedTime(&ms, start, stop), "hipEventElapsedTime");
        prefix[k].push_back(double(ms) * 1000.0);
      }
  } catch (...) {
    hipEventDestroy(start);
    if (stop) hipEventDestroy(stop);
    throw;
  }
  hipEventDestroy(start);
  hipEventDestroy(stop);
  std::vector<double> medians(n + 1);
  for (size_t k = 0; k <= n; ++k) {
    std::sort(prefix[k].begin(), prefix[k].end());
    medians[k] = prefix[k][prefix[k].size() / 2];
  }
  std::vector<double> out(n);
  for (size_t k = 0; k < n; ++k) out[k] = medians[k + 1] - medians[k];
  return out;
}

double Invocation::timeLaunch(const Launch &launch, uint64_t iterations) {
  if (!iterations) throw std::invalid_argument("iterations must be positive");
  device->makeCurrent();
  check(hipStreamSynchronize(stream), "hipStreamSynchronize");
  hipEvent_t start = nullptr, stop = nullptr;
  check(hipEventCreate(&start), "hipEventCreate");
  float elapsed = 0;
  try {
    check(hipEventCreate(&stop), "hipEventCreate");
    check(hipEventRecord(start, stream), "hipEventRecord");
    for (uint64_t k = 0; k < iterations; ++k) launchOne(launch, stream);
    check(hipEventRecord(stop, stream), "hipEventRecord");
    check(hipEventSynchronize(stop), "hipEventSynchronize");
    check(hipEventElapsedTime(&elapsed, start, stop), "hipEventElapsedTime");
  } catch (...) {
    hipEventDestroy(start);
    if (stop) hipEventDestroy(stop);
    throw;
  }
  hipEventDestroy(start);
  hipEventDestroy(stop);
  return double(elapsed) * 1000.0 / double(iterations);
}

// ====================================================================== callbacks
// The callback protocol of lib/Runtime/NvidiaProgram.cpp:48-108: exceptions never unwind
// through the entry; the first failure is recorded and later callbacks become no-ops.
template <typename F> static void callback(void *opaque, F action) {
  auto &frame = *static_cast<Invocation *>(opaque);
  if (!frame.error.empty()) return;
  try {
    action(frame);
  } catch (const std::exception &error) {
    frame.error = error.what();
    if (frame.error.empty()) frame.error = "callback failed";
  }
}

static void appendArgument(Launch &launch, const void *data, uint64_t size, int64_t resource = -1) {
  if (!data || !size) throw std::invalid_argument("physical kernel argument must not be empty");
  size_t align = (size == 1 || size == 2 || size == 4 || size == 8) ? size : 1;
  size_t offset = (launch.arguments.size() + align - 1) & ~(align - 1);
  launch.arguments.resize(offset + size, 0);
  std::memcpy(launch.arguments.data() + offset, data, size);
  launch.slotOffsets.push_back(offset);
  launch.slotSizes.push_back(size);
  launch.slotResources.push_back(resource);
}


static std::shared_ptr<Invocation> bindWith(const std::shared_ptr<ProgramState> &programIn, std::shared_ptr<Device> device,
                                            const std::vector<Argument> &arguments, bool arena, hipStream_t stream) {
  auto program = programIn;
  if (!device) throw std::invalid_argument("program binding requires a device");
  std::vector<uint64_t> addresses, scalars;
  std::vector<std::shared_ptr<Buffer>> buffers;
  packArguments(*program, device.get(), arguments, addresses, scalars, buffers);
  const size_t count = arguments.size();
  std::vector<void *> packed(count);
  for (size_t k = 0; k < count; ++k) packed[k] = program->bufferBytes[k] ? &addresses[k] : &scalars[k];
  // Fused programs fall back to their unfused form when external byte ranges overlap
  // (lib/Runtime/NvidiaProgram.cpp:191-205).
  if (program->aliasFallback && argumentsOverlap(*program, addresses)) program = program->aliasFallback;
  auto invocation = std::make_shared<Invocation>(program, device, stream);
  invocation->buffers = std::move(buffers);
  invocation->requested = programIn;
  invocation->argumentAddresses = addresses;
  invocation->argumentScalars = scalars;
  invocation->bindingAddresses = addresses.data();
  invocation->bindingCount = count;
  if (arena) {
    invocation->staticArena = true;
    invocation->arenaBase = staticScratchAddress(device->ordinal);
    invocation->arenaLimit = staticScratchBytes();
    // Every static bind on a device reuses the arena from its start: earlier ones are superseded.
    invocation->epoch = ++staticEpochs[size_t(device->ordinal)];
  }
  void *frame = invocation.get();
  void **values = packed.data();
  void *entryArguments[] = {&frame, &values, program->entryContext};
  program->entry(entryArguments);
  invocation->bindingAddresses = nullptr;
  // Heaps no resource asked for are placed as well (the binding's memory is its plan's).
  callback(invocation.get(), [](Invocation &f) { f.placeHeaps(); });
  if (!invocation->error.empty()) {
    // The reference reports callback failures as runtime errors; a program too large for the
    // static arena is the caller's argument error.
    if (invocation->arenaExceeded) throw std::invalid_argument(invocation->error);
    throw std::runtime_error(invocation->error);
  }
  return invocation;
}

} // namespace ckl::rt

using ckl::rt::Invocation;
using ckl::rt::Launch;

extern "C" void ckl_begin(void *frame, const void *binary, uint64_t bytes) {
  ckl_module(frame, "", binary, bytes);
}

extern "C" void ckl_module(void *frame, const char *identity, const void *binary, uint64_t bytes) {
  ckl::rt::callback(frame, [&](Invocation &f) {
    std::string key = identity && *identity ? identity : "program:" + std::to_string(reinterpret_cast<uintptr_t>(f.program.get()));
    f.module = f.device->load(key, binary, bytes, !f.staticArena);
  });
}

// Heaps are recorded and placed together, in one allocation (or one range of the static arena)
// cleared by one fill kernel, when the entry first needs an address (ckl::rt::placeHeaps).
extern "C" void ckl_heap(void *frame, uint64_t id, uint64_t bytes) {
  ckl::rt::callback(frame, [&](Invocation &f) {
    if (!bytes) throw std::invalid_argument("heaps must be non-empty");
    if (f.heaps.size() <= id) f.heaps.resize(id + 1);
    if (f.heaps[id] || std::any_of(f.pendingHeaps.begin(), f.pendingHeaps.end(), [&](auto &h) { return h.first == id; }))
      throw std::invalid_argument("heap " + std::to_string(id) + " declared twice");
    f.pendingHeaps.push_back({id, bytes});
  });
}

extern "C" void ckl_resource(void *frame, uint64_t id, uint64_t heap, uint64_t offset, void *external) {
  ckl::rt::callback(frame, [&](Invocation &f) {
    f.placeHeaps();
    if (f.resources.size() <= id) f.resources.resize(id + 1);
    if (f.temporaryResources.size() <= id) f.temporaryResources.resize(id + 1, false);
    if (f.resourceArgument.size() <= id) f.resourceArgument.resize(id + 1, -1);
    if (f.externalResources.size() <= id) f.externalResources.resize(id + 1, false);
    f.temporaryResources[id] = !external;
    f.externalResources[id] = external != nullptr;
    if (external) {
      f.resources[id] = *static_cast<uint64_t *>(external);
      // Which program argument the resource is: the entry passes the packed address's location.
      const uint64_t *at = static_cast<const uint64_t *>(external);
      if (f.bindingAddresses && at >= f.bindingAddresses && at < f.bindingAddresses + f.bindingCount)
        f.resourceArgument[id] = at - f.bindingAddresses;
    }
    else {
      const auto &h = f.heaps.at(heap);
      if (!h || offset > h->bytes) throw std::out_of_range("resource placement exceeds its heap");
      f.resources[id] = h->address() + offset;
    }
  });
}

extern "C" void ckl_kernel(void *frame, const char *name, uint64_t gx, uint64_t gy, uint64_t gz, uint64_t bx,
                           uint64_t by, uint64_t bz, uint64_t shared) {
  ckl::rt::callback(frame, [&](Invocation &f) {
    if (!f.module) throw std::invalid_argument("ckl_kernel requires a loaded module (ckl_begin)");
    Launch launch;
    launch.name = name;
    launch.module = f.module;
    ckl::rt::check(hipModuleGetFunction(&launch.function, f.module, name), "hipModuleGetFunction");
    ckl::rt::bindVariants(launch, name);
    uint64_t dims[6] = {gx, gy, gz, bx, by, bz};
    for (uint64_t d : dims)
      if (!d || d > 0xffffffffull) throw std::invalid_argument("kernel launch dimensions must be positive 32-bit values");
    launch.grid[0] = unsigned(gx); launch.grid[1] = unsigned(gy); launch.grid[2] = unsigned(gz);
    launch.block[0] = unsigned(bx); launch.block[1] = unsigned(by); launch.block[2] = unsigned(bz);
    launch.shared = unsigned(shared);
    f.pending = std::move(launch);
    f.dependencies.clear();
  });
}

extern "C" void ckl_argument_resource(void *frame, uint64_t id, uint64_t offset) {
  ckl::rt::callback(frame, [&](Invocation &f) {
    uint64_t address = f.resources.at(id) + offset;
    ckl::rt::appendArgument(f.pending, &address, sizeof address, int64_t(id));
  });
}

extern "C" void ckl_argument_value(void *frame, const void *bytes, uint64_t size) {
  ckl::rt::callback(frame, [&](Invocation &f) { ckl::rt::appendArgument(f.pending, bytes, size); });
}

extern "C" void ckl_workspace(void *frame, uint64_t bytes) {
  ckl::rt::callback(frame, [&](Invocation &f) {
    if (!bytes) throw std::invalid_argument("library workspace must be non-empty");
    std::shared_ptr<ckl::rt::Buffer> buffer;
    f.device->makeCurrent();
    if (f.staticArena) {
      // The arena keeps whatever the last user left: clear the workspace on the caller's stream.
      const uint64_t rounded = (bytes + 15) & ~uint64_t(15);
      buffer = ckl::rt::importBuffer(f.device, f.carve(rounded), rounded);
      ckl::rt::staticScratchClear(buffer->address(), rounded, f.stream);
    } else {
      buffer = ckl::rt::allocateBuffer(f.device, bytes);
      ++f.allocations;
      ckl::rt::check(hipMemset(reinterpret_cast<void *>(buffer->address()), 0, bytes), "hipMemset(workspace)");
      ckl::rt::check(hipDeviceSynchronize(), "hipDeviceSynchronize");
    }
    uint64_t address = buffer->address();
    ckl::rt::appendArgument(f.pending, &address, sizeof address);
    f.workspaces.push_back(std::move(buffer));
  });
}

extern "C" void ckl_dependency(void *frame, uint64_t id) {
  ckl::rt::callback(frame, [&](Invocation &f) { f.dependencies.push_back(f.nodes.at(id)); });
}

extern "C" void ckl_commit(void *frame, uint64_t id) {
  ckl::rt::callback(frame, [&](Invocation &f) {
    f.pending.arguments.resize((f.pending.arguments.size() + 7) & ~size_t(7), 0);
    if (f.pending.arguments.empty()) f.pending.arguments.resize(8, 0);
    // A library kernel whose streamed operand is large runs its nontemporal-load variant.
    if (f.pending.module && ckl::rt::streams(f.pending)) {
      hipFunction_t variant = nullptr;
      std::string nt = f.pending.name + "_nt";
      if (hipModuleGetFunction(&variant, f.pending.module, nt.c_str()) == hipSuccess) {
        f.pending.function = variant;
        ckl::rt::bindVariants(f.pending, nt);
      } else {
        (void)hipGetLastError();
      }
    }
    ckl::rt::prepareParams(f.pending, *f.device);
    f.nodes[id] = f.plan.addKernel(std::move(f.pending), std::move(f.dependencies));
    f.pending = Launch();
    f.dependencies.clear();
  });
}
