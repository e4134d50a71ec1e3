// Driver for the reference storage planner (TEST INFRASTRUCTURE; see oracle/__init__.py).
// Links the reference's own lib/Core/MemoryPlanner.cpp, compiled where it lies under
// /root/reference by oracle/Makefile, and prints its plan for a graph read from stdin:
//   nodes <N> reuse <0|1>
//   edge <from> <to>                                        (repeated)
//   resource <bytes> <alignment> <device> <kind 0|1|2> <user>...   (repeated, in order)
// Output: "baseline <B> planned <P>" then one "resource <k> <heap> <offset> <slot> <shares>"
// line per planned resource (shares = first earlier slot resident or -1); errors go to
// stdout as "error <message>".
#include "ckl/Core/MemoryPlanner.h"

#include <iostream>
#include <sstream>
#include <string>
#include <vector>

using namespace mlir::ckl::planning;

int main() {
  std::size_t nodes = 0;
  bool reuse = true;
  std::vector<GraphEdge> edges;
  std::vector<Resource> resources;
  std::string line;
  while (std::getline(std::cin, line)) {
    std::istringstream in(line);
    std::string tag;
    if (!(in >> tag)) continue;
    if (tag == "nodes") {
      std::string word;
      int r = 1;
      in >> nodes >> word >> r;
      reuse = r != 0;
    } else if (tag == "edge") {
      GraphEdge e{};
      in >> e.from >> e.to;
      edges.push_back(e);
    } else if (tag == "resource") {
      Resource res;
      int kind = 0;
      in >> res.bytes >> res.alignment >> res.device >> kind;
      res.kind = kind == 0 ? ResourceKind::Temporary : kind == 1 ? ResourceKind::Persistent : ResourceKind::External;
      res.name = "r" + std::to_string(resources.size());
      NodeId user;
      while (in >> user) res.users.push_back(user);
      resources.push_back(res);
    }
  }
  MemoryPlanResult result = MemoryPlanner(reuse).tryPlan(nodes, edges, resources);
  if (!result) {
    std::cout << "error " << result.error << "\n";
    return 0;
  }
  const MemoryPlan &plan = *result.value;
  std::cout << "baseline " << plan.baselineBytes << " planned " << plan.plannedBytes << "\n";
  for (const Assignment &a : plan.assignments) {
    long long shares = -1;
    for (const ReuseDecision &d : plan.decisions)
      if (d.resource == a.resource && !d.sharesWith.empty()) shares = (long long)d.sharesWith.front();
    std::cout << "resource " << a.resource << " " << a.heap << " " << a.offset << " " << a.slot << " " << shares << "\n";
  }
  return 0;
}
