#include "planner.h"

#include <algorithm>
#include <limits>
#include <stdexcept>

namespace ckl::planning {

std::size_t alignUp(std::size_t value, std::size_t alignment) {
  if (!alignment || (alignment & (alignment - 1)))
    throw std::invalid_argument("resource alignment must be a nonzero power of two");
  if (value > std::numeric_limits<std::size_t>::max() - (alignment - 1))
    throw std::overflow_error("memory plan size overflow");
  return (value + alignment - 1) & ~(alignment - 1);
}

Reachability::Reachability(std::size_t nodeCount, const std::vector<GraphEdge> &edges)
    : nodes_(nodeCount), words_((nodeCount + 63) / 64) {
  if (nodeCount > (std::size_t(1) << 24))
    throw std::overflow_error("memory-planning graph is too large");
  rows_.assign(nodes_ * words_, 0);
  for (const GraphEdge &e : edges) {
    if (e.from >= nodeCount || e.to >= nodeCount)
      throw std::out_of_range("memory-planning edge references an unknown graph node");
    if (e.from == e.to)
      throw std::invalid_argument("memory-planning graph contains a self edge");
    rows_[e.from * words_ + (e.to >> 6)] |= uint64_t(1) << (e.to & 63);
  }
  // Warshall closure: for each intermediate `via`, every row that reaches `via` absorbs
  // the row of `via`.
  for (NodeId via = 0; via < nodes_; ++via) {
    const uint64_t *viaRow = &rows_[via * words_];
    for (NodeId from = 0; from < nodes_; ++from) {
      uint64_t *row = &rows_[from * words_];
      if ((row[via >> 6] >> (via & 63)) & 1u)
        for (std::size_t w = 0; w < words_; ++w) row[w] |= viaRow[w];
    }
  }
  for (NodeId n = 0; n < nodes_; ++n)
    if (reaches(n, n)) throw std::invalid_argument("memory-planning graph must be acyclic");
}

const Assignment *MemoryPlan::find(ResourceId resource) const {
  for (const Assignment &a : assignments)
    if (a.resource == resource) return &a;
  return nullptr;
}

namespace {

struct Slot {
  int device;
  std::string addressSpace;
  std::size_t bytes;
  std::size_t alignment;
  bool recyclable;
  std::vector<ResourceId> residents;
  std::size_t heap = 0;
  std::size_t offset = 0;
};

// Every use of `first` reaches every use of `second` (and none is shared).
bool ordered(const Reachability &r, const Resource &first, const Resource &second) {
  if (first.users.empty() || second.users.empty()) return false;
  for (NodeId a : first.users)
    for (NodeId b : second.users)
      if (a == b || !r.reaches(a, b)) return false;
  return true;
}

} // namespace

MemoryPlan MemoryPlanner::plan(std::size_t nodeCount, const std::vector<GraphEdge> &edges,
                               const std::vector<Resource> &resources) const {
  Reachability reach(nodeCount, edges);
  MemoryPlan result;
  std::vector<Slot> slots;
  const std::size_t none = std::numeric_limits<std::size_t>::max();
  std::vector<std::size_t> slotOf(resources.size(), none);

  for (ResourceId id = 0; id < resources.size(); ++id) {
    const Resource &res = resources[id];
    if (!res.bytes) throw std::invalid_argument("memory-planning resource size must be nonzero");
    alignUp(res.bytes, res.alignment);
    for (NodeId user : res.users)
      if (user >= nodeCount)
        throw std::out_of_range("memory-planning resource references an unknown graph node");
    if (res.kind == ResourceKind::Temporary && res.users.empty())
      throw std::invalid_argument("temporary memory-planning resource must have at least one user");
    if (res.kind == ResourceKind::External) continue;

    std::size_t dedicated = alignUp(res.bytes, res.alignment);
    if (result.baselineBytes > std::numeric_limits<std::size_t>::max() - dedicated)
      throw std::overflow_error("memory plan baseline size overflow");
    result.baselineBytes += dedicated;

    std::size_t chosen = none, growth = none;
    if (reuse_ && res.kind == ResourceKind::Temporary) {
      for (std::size_t k = 0; k < slots.size(); ++k) {
        const Slot &slot = slots[k];
        if (!slot.recyclable || slot.device != res.device || slot.addressSpace != res.addressSpace) continue;
        bool fits = std::all_of(slot.residents.begin(), slot.residents.end(), [&](ResourceId other) {
          return ordered(reach, res, resources[other]) || ordered(reach, resources[other], res);
        });
        if (!fits) continue;
        std::size_t g = std::max(slot.bytes, res.bytes) - slot.bytes;
        if (g < growth) { chosen = k; growth = g; }
      }
    }
    if (chosen == none) {
      chosen = slots.size();
      slots.push_back({res.device, res.addressSpace, res.bytes, res.alignment,
                       res.kind == ResourceKind::Temporary, {}});
    }
    Slot &slot = slots[chosen];
    std::vector<ResourceId> previous = slot.residents;
    slot.bytes = std::max(slot.bytes, res.bytes);
    slot.alignment = std::max(slot.alignment, res.alignment);
    slot.residents.push_back(id);
    slotOf[id] = chosen;
    std::string reason;
    if (!previous.empty()) reason = "all resource uses are ordered by existing graph edges";
    else if (res.kind == ResourceKind::Persistent) reason = "persistent resource gets dedicated storage";
    else reason = reuse_ ? "no compatible ordered lifetime" : "storage reuse disabled";
    result.decisions.push_back({id, chosen, std::move(previous), std::move(reason)});
  }

  for (Slot &slot : slots) {
    auto heap = std::find_if(result.heaps.begin(), result.heaps.end(), [&](const Heap &h) {
      return h.device == slot.device && h.addressSpace == slot.addressSpace;
    });
    if (heap == result.heaps.end()) {
      result.heaps.push_back({slot.device, slot.addressSpace, 0, slot.alignment});
      heap = std::prev(result.heaps.end());
    }
    slot.heap = std::size_t(heap - result.heaps.begin());
    heap->alignment = std::max(heap->alignment, slot.alignment);
    slot.offset = alignUp(heap->bytes, slot.alignment);
    if (slot.offset > std::numeric_limits<std::size_t>::max() - slot.bytes)
      throw std::overflow_error("memory plan heap size overflow");
    heap->bytes = slot.offset + slot.bytes;
  }
  for (Heap &heap : result.heaps) {
    heap.bytes = alignUp(heap.bytes, heap.alignment);
    if (result.plannedBytes > std::numeric_limits<std::size_t>::max() - heap.bytes)
      throw std::overflow_error("memory plan total size overflow");
    result.plannedBytes += heap.bytes;
  }
  for (ResourceId id = 0; id < resources.size(); ++id) {
    if (resources[id].kind == ResourceKind::External) continue;
    const Slot &slot = slots[slotOf[id]];
    result.assignments.push_back({id, slot.heap, slot.offset, resources[id].bytes, slotOf[id]});
  }
  return result;
}

MemoryPlanResult MemoryPlanner::tryPlan(std::size_t nodeCount, const std::vector<GraphEdge> &edges,
                                        const std::vector<Resource> &resources) const noexcept {
  try {
    return {plan(nodeCount, edges, resources), {}};
  } catch (const std::exception &error) {
    return {std::nullopt, error.what()};
  } catch (...) {
    return {std::nullopt, "unknown memory-planning failure"};
  }
}

} // namespace ckl::planning
