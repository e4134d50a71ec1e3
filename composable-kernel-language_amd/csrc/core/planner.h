// Graph-order storage planner: packs program temporaries into per-(device, address space)
// heaps, letting two temporaries share a slot only when graph reachability orders every use
// of one before every use of the other.
//
// Algorithm (the decisions must match the reference bit for bit, so its steps are kept):
// lib/Core/MemoryPlanner.cpp:98-204 and include/ckl/Core/MemoryPlanner.h:18-92.
//   * transitive closure of the node graph (MemoryPlanner.cpp:19-43),
//   * "A before B" iff every user of A reaches every user of B (45-55),
//   * a temporary may join a recyclable slot on the same device/space whose residents are all
//     ordered with it (75-88); among such slots the least byte growth wins, ties to the
//     lowest slot index (131-144),
//   * slots are laid out per heap in creation order at aligned offsets (171-188) and heaps are
//     rounded to their alignment (190-195).
#pragma once

#include <cstddef>
#include <cstdint>
#include <optional>
#include <string>
#include <vector>

namespace ckl::planning {

using NodeId = std::size_t;
using ResourceId = std::size_t;

struct GraphEdge {
  NodeId from;
  NodeId to;
};

enum class ResourceKind { Temporary, Persistent, External };

struct Resource {
  std::string name;
  std::size_t bytes = 0;
  std::size_t alignment = 1;
  std::string addressSpace = "global";
  int device = 0;
  ResourceKind kind = ResourceKind::Temporary;
  std::vector<NodeId> users;
};

struct Heap {
  int device = 0;
  std::string addressSpace;
  std::size_t bytes = 0;
  std::size_t alignment = 1;
};

struct Assignment {
  ResourceId resource = 0;
  std::size_t heap = 0;
  std::size_t offset = 0;
  std::size_t bytes = 0;
  std::size_t slot = 0;
};

struct ReuseDecision {
  ResourceId resource = 0;
  std::size_t slot = 0;
  std::vector<ResourceId> sharesWith;
  std::string reason;
};

struct MemoryPlan {
  std::size_t baselineBytes = 0;
  std::size_t plannedBytes = 0;
  std::vector<Heap> heaps;
  std::vector<Assignment> assignments;
  std::vector<ReuseDecision> decisions;
  const Assignment *find(ResourceId resource) const;
};

struct MemoryPlanResult {
  std::optional<MemoryPlan> value;
  std::string error;
  explicit operator bool() const { return value.has_value(); }
};

// Transitive closure over up to a few thousand nodes, stored as 64-bit row bitsets.
class Reachability {
public:
  Reachability(std::size_t nodeCount, const std::vector<GraphEdge> &edges);
  bool reaches(NodeId from, NodeId to) const {
    return (rows_[from * words_ + (to >> 6)] >> (to & 63)) & 1u;
  }
  std::size_t size() const { return nodes_; }

private:
  std::size_t nodes_, words_;
  std::vector<uint64_t> rows_;
};

class MemoryPlanner {
public:
  explicit MemoryPlanner(bool reuseStorage = true) : reuse_(reuseStorage) {}
  MemoryPlan plan(std::size_t nodeCount, const std::vector<GraphEdge> &edges,
                  const std::vector<Resource> &resources) const;
  MemoryPlanResult tryPlan(std::size_t nodeCount, const std::vector<GraphEdge> &edges,
                           const std::vector<Resource> &resources) const noexcept;

private:
  bool reuse_;
};

std::size_t alignUp(std::size_t value, std::size_t alignment);

} // namespace ckl::planning
