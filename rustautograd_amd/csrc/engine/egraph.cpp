// Cost models and matrix-product reassociation.
//
// The reference runs equality saturation with the egg crate (src/egraph.rs:358-427, egg 0.11.0,
// not vendored) and extracts the cheapest tree under a cost model (egraph.rs:170-233). For the
// Linear rule set the rewrites that change cost are matrix-product reassociation, factoring and
// transpose flags (egraph.rs:147-152). This file restates the cost model and reaches the same
// optimum for the case the rule set exists for — chains of 2-D products — by dynamic
// programming over each maximal chain, the textbook matrix-chain order.
#include <cmath>
#include <functional>
#include <map>

#include "optimize.h"

namespace rg {

namespace {

struct Model {
  double per_op, per_element, per_flop, per_math_element, per_transpose_element;
};

// egraph.rs:184-185: CPU from M4 Pro measurements. The device model is MI355X: ~4 us per
// dispatch in a graph, HBM at ~5 TB/s effective (~0.0008 ns per fp32 element written), fp32
// MFMA at ~80 TFLOP/s sustained (~0.000025 ns per multiply-add).
Model model_of(CostModel m) {
  if (m == CostModel::Cpu) return {200.0, 0.06, 0.0015, 0.6, 1.4};
  return {4000.0, 0.0008, 0.000025, 0.0004, 0.0016};
}

double node_cost(const Model& c, const Op& op, const Shape& shape, const std::vector<Shape>& args) {
  double n = (double)numel(shape);
  double base = c.per_op + c.per_element * n;
  switch (op.kind) {
    case RG_OP_INPUT: case RG_OP_CONST: return 0.0;
    case RG_OP_RESHAPE: case RG_OP_STOP_GRADIENT: case RG_OP_OUTPUT: case RG_OP_CUSTOM: return 0.0;
    case RG_OP_MATMUL: {
      double k = args[0].empty() ? 1.0 : (double)args[0].back();
      return base + c.per_flop * n * k;
    }
    case RG_OP_MATMUL_T: {
      const Shape& a = args[0];
      double k = (double)(op.ta ? a[a.size() - 2] : a[a.size() - 1]);
      return base + c.per_flop * n * k;
    }
    case RG_OP_TRANSPOSE: return c.per_op + c.per_transpose_element * n;
    case RG_OP_EXP: case RG_OP_LOG: case RG_OP_SIN: case RG_OP_COS: case RG_OP_TANH:
      return base + c.per_math_element * n;
    case RG_OP_POW: return base + 16.0 * c.per_math_element * n;
    case RG_OP_DIV: case RG_OP_SQRT: return base + 0.2 * c.per_math_element * n;
    default: return base;
  }
}

}  // namespace

double graph_cost(CostModel m, const Graph& g, const std::vector<uint32_t>& outputs) {
  Model c = model_of(m);
  std::vector<bool> keep = g.reachable(outputs);
  double total = 0;
  for (size_t i = 0; i < g.nodes.size(); i++) {
    if (!keep[i]) continue;
    const Node& n = g.nodes[i];
    bool constant = !n.inputs.empty();
    std::vector<Shape> args;
    for (uint32_t x : n.inputs) {
      args.push_back(g.shape(x));
      constant = constant && g.nodes[x].op.kind == RG_OP_CONST;
    }
    total += constant ? 0.0 : node_cost(c, n.op, n.shape, args);
  }
  return total;
}

std::optional<std::pair<Graph, std::vector<uint32_t>>> matrix_search(const Graph& g, const std::vector<uint32_t>& outputs,
                                                                     CostModel model, OptMode mode, SearchStats* st) {
  st->cost_before = graph_cost(model, g, outputs);
  if (mode == OptMode::SearchExact) return std::nullopt;
  Model c = model_of(model);
  std::vector<bool> keep = g.reachable(outputs);
  // Uses of each node among kept nodes and outputs: only single-use inner products may be
  // reassociated, since a shared intermediate must stay materialized.
  std::vector<size_t> uses(g.nodes.size(), 0);
  for (size_t i = 0; i < g.nodes.size(); i++)
    if (keep[i])
      for (uint32_t x : g.nodes[i].inputs) uses[x]++;
  for (uint32_t o : outputs) uses[o]++;
  auto is_mm2 = [&](uint32_t id) {
    const Node& n = g.nodes[id];
    return n.op.kind == RG_OP_MATMUL && n.shape.size() == 2 && g.shape(n.inputs[0]).size() == 2 &&
           g.shape(n.inputs[1]).size() == 2 && n.dtype != DType::I32;
  };
  // Flattens a chain rooted at `id` into its factor list.
  std::function<void(uint32_t, bool, std::vector<uint32_t>&)> factors = [&](uint32_t id, bool root, std::vector<uint32_t>& out) {
    if (is_mm2(id) && (root || uses[id] == 1)) {
      factors(g.nodes[id].inputs[0], false, out);
      factors(g.nodes[id].inputs[1], false, out);
    } else {
      out.push_back(id);
    }
  };
  // A chain root: a 2-D product not itself an inner single-use factor of another product.
  std::vector<bool> inner(g.nodes.size(), false);
  for (size_t i = 0; i < g.nodes.size(); i++)
    if (keep[i] && is_mm2((uint32_t)i))
      for (uint32_t x : g.nodes[i].inputs)
        if (is_mm2(x) && uses[x] == 1) inner[x] = true;

  Graph h;
  std::vector<uint32_t> map(g.nodes.size(), UINT32_MAX);
  bool changed = false;
  size_t explored = 0;
  for (size_t i = 0; i < g.nodes.size(); i++) {
    const Node& n = g.nodes[i];
    h.cur_source = n.source;
    h.cur_origin = n.origin >= 0 ? 0 : -1;
    if (n.op.kind == RG_OP_INPUT) {
      map[i] = h.input(n.shape, n.dtype);
      h.nodes[map[i]].op = n.op;
      continue;
    }
    if (!keep[i] || inner[i]) continue;
    if (n.op.kind == RG_OP_CONST) {
      map[i] = h.constant(*n.op.t);
      continue;
    }
    if (is_mm2((uint32_t)i)) {
      std::vector<uint32_t> fs;
      factors((uint32_t)i, true, fs);
      if (fs.size() >= 3) {
        // dims[k] x dims[k+1] is factor k.
        size_t m = fs.size();
        std::vector<size_t> dims;
        dims.push_back(g.shape(fs[0])[0]);
        for (uint32_t f : fs) dims.push_back(g.shape(f)[1]);
        std::vector<std::vector<double>> best(m, std::vector<double>(m, 0.0));
        std::vector<std::vector<size_t>> split(m, std::vector<size_t>(m, 0));
        for (size_t len = 2; len <= m; len++) {
          for (size_t a = 0; a + len <= m; a++) {
            size_t b = a + len - 1;
            best[a][b] = INFINITY;
            for (size_t s = a; s < b; s++) {
              double out_n = (double)(dims[a] * dims[b + 1]);
              double cost = best[a][s] + best[s + 1][b] + c.per_op + c.per_element * out_n +
                            c.per_flop * out_n * (double)dims[s + 1];
              explored++;
              if (cost < best[a][b]) {
                best[a][b] = cost;
                split[a][b] = s;
              }
            }
          }
        }
        std::function<uint32_t(size_t, size_t)> emit = [&](size_t a, size_t b) -> uint32_t {
          if (a == b) return map[fs[a]];
          size_t s = split[a][b];
          uint32_t l = emit(a, s), r = emit(s + 1, b);
          return h.add(Op::make(RG_OP_MATMUL), {l, r});
        };
        // The original left-to-right or traced order, for comparison.
        map[i] = emit(0, m - 1);
        changed = true;
        continue;
      }
    }
    std::vector<uint32_t> ins;
    for (uint32_t x : n.inputs) ins.push_back(map[x]);
    map[i] = h.add(n.op, ins);
    h.nodes[map[i]].origin = n.origin >= 0 ? 0 : -1;
  }
  st->iterations = 1;
  st->egraph_nodes = explored;
  if (!changed) return std::nullopt;
  std::vector<uint32_t> out;
  for (uint32_t o : outputs) out.push_back(map[o]);
  st->cost_after = graph_cost(model, h, out);
  return std::make_pair(std::move(h), std::move(out));
}

}  // namespace rg
