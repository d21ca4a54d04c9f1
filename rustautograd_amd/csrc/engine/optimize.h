// Graph optimizer (reference src/optimize.rs) and the matrix-reassociation search that stands
// in for its equality-saturation pass (reference src/egraph.rs).
#pragma once
#include <optional>

#include "plan.h"

namespace rg {

enum class OptMode { None, Standard, SearchExact, SearchLinear, Search, Auto };
bool parse_opt_mode(const std::string& s, OptMode* out);

struct SearchStats {
  size_t iterations = 0, egraph_nodes = 0;
  double cost_before = 0, cost_after = 0;
};

struct OptStats {
  size_t nodes_before = 0, nodes_after = 0, folded = 0, simplified = 0, cse = 0, rematerialized = 0;
  bool searched = false, accepted = false;
  SearchStats search;
  Json json() const;
};

struct Optimized {
  Graph g;
  std::vector<uint32_t> outputs;
  OptStats stats;
};

// optimize_mode (optimize.rs:210-246). `device` enables the split of large full sums
// (optimize.rs:369-378) and selects the device cost model for the search.
Optimized optimize_mode(const Graph& g, const std::vector<uint32_t>& outputs, bool device, OptMode mode);

// Cost models of the search (egraph.rs:170-233).
enum class CostModel { Cpu, Device };
double graph_cost(CostModel m, const Graph& g, const std::vector<uint32_t>& outputs);

// Matrix-product reassociation over the simplified graph (egraph.rs:358-427, rule set Linear).
// Returns a rewritten graph when one is found, with statistics.
std::optional<std::pair<Graph, std::vector<uint32_t>>> matrix_search(const Graph& g, const std::vector<uint32_t>& outputs,
                                                                     CostModel model, OptMode mode, SearchStats* st);

}  // namespace rg
