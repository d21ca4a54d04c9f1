// Graph optimizer: single forward rewrite with identities, folding, broadcast elision,
// transpose flags, the device split of full sums and CSE, then rematerialization (followed, for
// device plans, by a merge of identical nodes).
// Follows the reference's src/optimize.rs:8-15 (constants), 42-77 (splat, identity),
// 79-166 (rematerialize), 172-285 (modes), 287-403 (simplify).
#include "optimize.h"

#include <unordered_map>

#include "backend.h"

namespace rg {

namespace {

constexpr size_t FOLD_LIMIT = 4096;
constexpr size_t CSE_CONST_LIMIT = 16;
// Device plans also merge equal constants up to this size (gradient seeds of ones, broadcast
// fills), so products and groups reading them merge too; the key spells out the constant's bytes.
constexpr size_t DEVICE_CSE_CONST_LIMIT = 4096;
constexpr size_t REMAT_MIN = 1 << 14;
constexpr size_t SPLIT_SUM_MIN = 4096;
constexpr double SEARCH_MIN_GAIN = 0.9;
// Above this peak of live intermediates, even expensive elementwise values are recomputed in the backward pass rather than kept (optimize.rs:79-84).
constexpr size_t COSTLY_REMAT_ABOVE_BYTES = size_t(2) << 30;

bool splat(const Graph& g, uint32_t id, double* value) {
  const Node& n = g.nodes[id];
  if (n.op.kind != RG_OP_CONST) return false;
  const Tensor& t = *n.op.t;
  if (t.n() == 0 || t.n() > FOLD_LIMIT) return false;
  double v0 = t.at(0);
  for (size_t i = 1; i < t.n(); i++)
    if (!(t.at(i) == v0)) return false;
  if (std::isnan(v0)) return false;  // NaN == NaN is false in the reference's comparison
  *value = v0;
  return true;
}

// A node already in the graph that computes the same value, if any. `x * 0` is left alone, since folding it to 0 would lose a NaN or Inf in x.
int64_t identity(const Graph& g, const Op& op, const std::vector<uint32_t>& ins, const Shape& shape) {
  auto same = [&](uint32_t id) { return g.shape(id) == shape; };
  auto is = [&](uint32_t id, double c) {
    double v;
    return splat(g, id, &v) && v == c;
  };
  switch (op.kind) {
    case RG_OP_STOP_GRADIENT: case RG_OP_CUSTOM: return ins[0];
    case RG_OP_ADD:
      if (is(ins[1], 0.0) && same(ins[0])) return ins[0];
      if (is(ins[0], 0.0) && same(ins[1])) return ins[1];
      return -1;
    case RG_OP_SUB: return is(ins[1], 0.0) && same(ins[0]) ? (int64_t)ins[0] : -1;
    case RG_OP_MUL:
      if (is(ins[1], 1.0) && same(ins[0])) return ins[0];
      if (is(ins[0], 1.0) && same(ins[1])) return ins[1];
      return -1;
    case RG_OP_DIV: return is(ins[1], 1.0) && same(ins[0]) ? (int64_t)ins[0] : -1;
    case RG_OP_POW: return is(ins[1], 1.0) && same(ins[0]) ? (int64_t)ins[0] : -1;
    case RG_OP_NEG:
      if (g.nodes[ins[0]].op.kind == RG_OP_NEG) return g.nodes[ins[0]].inputs[0];
      return -1;
    case RG_OP_RESHAPE: case RG_OP_BROADCAST_TO: return same(ins[0]) ? (int64_t)ins[0] : -1;
    case RG_OP_CAST: return op.dt == g.dtype(ins[0]) ? (int64_t)ins[0] : -1;
    case RG_OP_TRANSPOSE: {
      for (size_t i = 0; i < op.v.size(); i++)
        if (op.v[i] != i) return -1;
      return ins[0];
    }
    case RG_OP_SLICE: {
      // A slice of the whole value (every start 0, every stop the dimension) is the value.
      const Shape& in = g.shape(ins[0]);
      for (size_t i = 0; i < in.size(); i++)
        if (op.v[i] != 0 || op.w[i] != in[i]) return -1;
      return ins[0];
    }
    case RG_OP_TAKE: {
      // Constant indices 0, 1, ..., n - 1 along an axis of length n (a position table read at
      // arange(n)): every row in order, so the result is the table itself.
      const Node& idx = g.nodes[ins[1]];
      const Shape& in = g.shape(ins[0]);
      if (idx.op.kind != RG_OP_CONST || idx.shape.size() != 1 || op.a >= in.size() || idx.shape[0] != in[op.a]) return -1;
      for (size_t i = 0; i < idx.shape[0]; i++)
        if (idx.op.t->at(i) != (double)i) return -1;
      return same(ins[0]) ? (int64_t)ins[0] : -1;
    }
    default: return -1;
  }
}

// Elementwise ops cheap enough that redoing them later costs less than holding their result.
bool recomputable(const Op& op, bool costly_too) {
  bool elementwise = op.is_unary_elementwise() || op.is_binary_elementwise() || op.kind == RG_OP_WHERE;
  bool costly = op.kind == RG_OP_EXP || op.kind == RG_OP_LOG || op.kind == RG_OP_SIN || op.kind == RG_OP_COS ||
                op.kind == RG_OP_TANH || op.kind == RG_OP_SQRT;
  return elementwise && op.kind != RG_OP_POW && (costly_too || !costly);
}

struct Simplified {
  Graph g;
  std::vector<uint32_t> out;
  OptStats st;
  std::vector<bool> backward;
};

Simplified rematerialize(const Graph& g, const std::vector<uint32_t>& outputs, const std::vector<bool>& backward,
                         size_t min_n, bool costly_too, OptStats& st) {
  std::vector<bool> keep = g.reachable(outputs);
  auto large = [&](uint32_t id) { return g.nodes[id].n() >= min_n; };
  std::vector<bool> retained(g.nodes.size(), false);
  for (size_t i = 0; i < g.nodes.size(); i++)
    if (keep[i] && backward[i])
      for (uint32_t x : g.nodes[i].inputs)
        if (!backward[x]) retained[x] = true;
  std::vector<bool> remat(g.nodes.size(), false);
  for (size_t i = g.nodes.size(); i-- > 0;) {
    const Node& n = g.nodes[i];
    if (!retained[i] || backward[i] || !recomputable(n.op, costly_too) || !large((uint32_t)i)) continue;
    auto always_alive = [&](uint32_t x) { return g.nodes[x].op.kind == RG_OP_INPUT || g.nodes[x].op.kind == RG_OP_CONST; };
    std::vector<uint32_t> fresh;
    for (uint32_t x : n.inputs)
      if (large(x) && !retained[x] && !always_alive(x)) fresh.push_back(x);
    // Vec::dedup removes consecutive duplicates only.
    fresh.erase(std::unique(fresh.begin(), fresh.end()), fresh.end());
    if (fresh.size() <= 1) {
      remat[i] = true;
      retained[i] = false;
      for (uint32_t x : n.inputs) retained[x] = true;
    }
  }
  // Emit the graph again; a value that was not kept is recomputed just before its first backward reader.
  Simplified r;
  Graph& h = r.g;
  std::vector<uint32_t> map(g.nodes.size(), UINT32_MAX);
  std::vector<int64_t> clone(g.nodes.size(), -1);
  std::function<uint32_t(uint32_t)> value = [&](uint32_t i) -> uint32_t {
    if (!remat[i]) return map[i];
    if (clone[i] >= 0) return (uint32_t)clone[i];
    const Node& n = g.nodes[i];
    std::vector<uint32_t> ins;
    for (uint32_t x : n.inputs) ins.push_back(value(x));
    h.cur_source = n.source;
    uint32_t id = h.add(n.op, ins);
    clone[i] = id;
    st.rematerialized++;
    return id;
  };
  for (size_t i = 0; i < g.nodes.size(); i++) {
    const Node& n = g.nodes[i];
    if (n.op.kind == RG_OP_INPUT) {
      h.cur_source = n.source;
      map[i] = h.input(n.shape, n.dtype);
      h.nodes[map[i]].op = n.op;
      continue;
    }
    if (!keep[i]) continue;
    std::vector<uint32_t> ins;
    for (uint32_t x : n.inputs) ins.push_back(backward[i] ? value(x) : map[x]);
    h.cur_source = n.source;
    map[i] = n.op.kind == RG_OP_CONST ? h.constant(*n.op.t) : h.add(n.op, ins);
  }
  for (uint32_t o : outputs) r.out.push_back(map[o]);
  return r;
}

Simplified simplify(const Graph& g, const std::vector<uint32_t>& outputs, bool device, bool flip_transposes) {
  std::vector<bool> keep = g.reachable(outputs);
  Simplified r;
  for (bool k : keep) r.st.nodes_before += k;
  Graph& ng = r.g;
  std::vector<uint32_t> map(g.nodes.size(), UINT32_MAX);
  std::unordered_map<std::string, uint32_t> seen;
  auto& backward = r.backward;

  for (size_t i = 0; i < g.nodes.size(); i++) {
    const Node& node = g.nodes[i];
    ng.cur_source = node.source;
    ng.cur_origin = -1;
    if (node.op.kind == RG_OP_INPUT) {
      map[i] = ng.input(node.shape, node.dtype);
      ng.nodes[map[i]].op = node.op;
      backward.resize(ng.nodes.size(), false);
      continue;
    }
    if (!keep[i]) continue;
    std::vector<uint32_t> ins;
    for (uint32_t x : node.inputs) ins.push_back(map[x]);

    int64_t existing = identity(ng, node.op, ins, node.shape);
    if (existing >= 0) {
      map[i] = (uint32_t)existing;
      r.st.simplified++;
      continue;
    }
    Op op = node.op;
    double two;
    if (op.kind == RG_OP_POW && splat(ng, ins[1], &two) && two == 2.0 && ng.shape(ins[0]) == node.shape) {
      op = Op::make(RG_OP_MUL);
      ins = {ins[0], ins[0]};
      r.st.simplified++;
    }
    // Elementwise kernels read broadcast operands directly; an explicit broadcast copy is pure overhead.
    if (op.is_binary_elementwise()) {
      for (int k = 0; k < 2; k++) {
        const Node& n = ng.nodes[ins[k]];
        if (n.op.kind == RG_OP_BROADCAST_TO) {
          uint32_t source = n.inputs[0];
          uint32_t other = ins[1 - k];
          Shape b;
          if (broadcast_shapes(ng.shape(source), ng.shape(other), &b) && b == node.shape) {
            ins[k] = source;
            r.st.simplified++;
          }
        }
      }
    }
    // The product reads a transposed operand in place (the ta/tb flags); the transpose node then has no readers and dead-code elimination drops it.
    if (flip_transposes && op.kind == RG_OP_MATMUL) {
      auto flipped = [&](uint32_t id) -> int64_t {
        const Node& n = ng.nodes[id];
        if (n.op.kind != RG_OP_TRANSPOSE) return -1;
        const Shape& p = n.op.v;
        if (p.size() < 2) return -1;
        for (size_t j = 0; j < p.size(); j++) {
          bool ok = j + 2 < p.size() ? p[j] == j : j + p[j] == 2 * p.size() - 3;
          if (!ok) return -1;
        }
        return n.inputs[0];
      };
      int64_t fa = flipped(ins[0]), fb = flipped(ins[1]);
      if (fa >= 0 || fb >= 0) {
        op = Op::make(RG_OP_MATMUL_T);
        op.ta = fa >= 0;
        op.tb = fb >= 0;
        ins = {fa >= 0 ? (uint32_t)fa : ins[0], fb >= 0 ? (uint32_t)fb : ins[1]};
        r.st.simplified++;
      }
    }
    bool foldable = !op.is_control_flow() && op.kind != RG_OP_OUTPUT && !ins.empty() && node.n() <= FOLD_LIMIT;
    for (uint32_t x : ins) foldable = foldable && ng.nodes[x].op.kind == RG_OP_CONST;
    if (foldable) {
      Graph tmp;
      std::vector<uint32_t> ids;
      for (uint32_t x : ins) ids.push_back(tmp.constant(*ng.nodes[x].op.t));
      uint32_t id = tmp.add(op, ids);
      Tensor value = eval_on(eager_backend(), tmp, {id}, {})[0];
      op = Op::make(RG_OP_CONST);
      op.t = std::make_shared<const Tensor>(std::move(value));
      ins.clear();
      r.st.folded++;
    }
    if (op.kind == RG_OP_REDUCE && op.rk == RK::Sum) {
      Shape shape = ng.shape(ins[0]);
      if (device && shape.size() >= 2 && op.v.size() == shape.size() && node.n() == 1 &&
          ng.nodes[ins[0]].n() >= SPLIT_SUM_MIN && shape.back() > 1) {
        // With keepdims the row sums keep their axis, so the result has the original rank. The
        // reference drops it here (optimize.rs:372-375): a keepdims full sum then comes out one
        // rank short, and a later full sum of it fails shape inference. The values are the same.
        Op rows = Op::make(RG_OP_REDUCE);
        rows.rk = RK::Sum;
        rows.v = {shape.size() - 1};
        rows.keepdims = op.keepdims;
        uint32_t rid = ng.add(rows, {ins[0]});
        backward.resize(ng.nodes.size(), false);
        backward[rid] = node.origin >= 0;
        bool keepdims = op.keepdims;
        op = Op::make(RG_OP_REDUCE);
        op.rk = RK::Sum;
        for (size_t a = 0; a + 1 < shape.size(); a++) op.v.push_back(a);
        op.keepdims = keepdims;
        ins = {rid};
      }
    }
    bool big_const = op.kind == RG_OP_CONST && op.t->n() > (device ? DEVICE_CSE_CONST_LIMIT : CSE_CONST_LIMIT);
    std::string key;
    if (!big_const) {
      key = op.key() + "|";
      for (uint32_t x : ins) key += std::to_string(x) + ",";
      auto it = seen.find(key);
      if (it != seen.end()) {
        map[i] = it->second;
        r.st.cse++;
        continue;
      }
    }
    uint32_t id = op.kind == RG_OP_CONST ? ng.constant(*op.t) : ng.add(op, ins);
    ng.nodes[id].origin = node.origin;  // later passes only test whether it is set
    backward.resize(ng.nodes.size(), false);
    backward[id] = node.origin >= 0;
    if (!big_const) seen[key] = id;
    map[i] = id;
  }
  for (uint32_t o : outputs) r.out.push_back(map[o]);
  backward.resize(ng.nodes.size(), false);
  return r;
}

// A rematerialized value whose original also stays in the forward pass has a clone with the
// same inputs; level-order device plans compute both in the same group, so the clone only adds
// a second output of the same value. On the device, identical nodes are merged after
// rematerialization (the same keying as simplify's CSE).
Simplified merge_identical(const Graph& g, const std::vector<uint32_t>& outputs, OptStats& st) {
  std::vector<bool> keep = g.reachable(outputs);
  Simplified r;
  Graph& h = r.g;
  std::vector<uint32_t> map(g.nodes.size(), UINT32_MAX);
  std::unordered_map<std::string, uint32_t> seen;
  for (size_t i = 0; i < g.nodes.size(); i++) {
    const Node& n = g.nodes[i];
    h.cur_source = n.source;
    if (n.op.kind == RG_OP_INPUT) {
      map[i] = h.input(n.shape, n.dtype);
      h.nodes[map[i]].op = n.op;
      continue;
    }
    if (!keep[i]) continue;
    std::vector<uint32_t> ins;
    for (uint32_t x : n.inputs) ins.push_back(map[x]);
    const bool big_const = n.op.kind == RG_OP_CONST && n.op.t->n() > CSE_CONST_LIMIT;
    std::string key;
    if (!big_const) {
      key = n.op.key() + "|";
      for (uint32_t x : ins) key += std::to_string(x) + ",";
      auto it = seen.find(key);
      if (it != seen.end()) {
        map[i] = it->second;
        st.cse++;
        continue;
      }
    }
    map[i] = n.op.kind == RG_OP_CONST ? h.constant(*n.op.t) : h.add(n.op, ins);
    if (!big_const) seen[key] = map[i];
  }
  for (uint32_t o : outputs) r.out.push_back(map[o]);
  return r;
}

Optimized finish(const Simplified& s, OptStats st, bool device) {
  Simplified h = rematerialize(s.g, s.out, s.backward, REMAT_MIN, false, st);
  if (build_plan(h.g, h.out, true).peak_live_bytes > COSTLY_REMAT_ABOVE_BYTES) {
    st.rematerialized = 0;
    h = rematerialize(s.g, s.out, s.backward, REMAT_MIN, true, st);
  }
  if (device) h = merge_identical(h.g, h.out, st);
  size_t kept = 0;
  for (bool k : h.g.reachable(h.out)) kept += k;
  st.nodes_after = kept;
  return Optimized{std::move(h.g), std::move(h.out), st};
}

// Cheap pre-check: does the graph contain a chain or sum of products the search could rewrite (optimize.rs:259-281).
bool has_matrix_structure(const Graph& g, const std::vector<uint32_t>& outputs) {
  std::vector<bool> keep = g.reachable(outputs);
  auto is_product = [&](uint32_t id) {
    const Node* n = &g.nodes[id];
    if (n->op.kind == RG_OP_TRANSPOSE && n->op.v == Shape{1, 0}) n = &g.nodes[n->inputs[0]];
    return n->op.kind == RG_OP_MATMUL;
  };
  for (size_t i = 0; i < g.nodes.size(); i++) {
    if (!keep[i]) continue;
    const Node& n = g.nodes[i];
    if (n.op.kind == RG_OP_MATMUL) {
      for (uint32_t x : n.inputs)
        if (is_product(x)) return true;
    } else if (n.op.kind == RG_OP_ADD) {
      bool all = true;
      for (uint32_t x : n.inputs) all &= is_product(x);
      if (all) return true;
    }
  }
  return false;
}

size_t count_kept(const Graph& g, const std::vector<uint32_t>& out) {
  size_t k = 0;
  for (bool b : g.reachable(out)) k += b;
  return k;
}

}  // namespace

bool parse_opt_mode(const std::string& s, OptMode* out) {
  if (s == "none") *out = OptMode::None;
  else if (s == "standard") *out = OptMode::Standard;
  else if (s == "search-exact") *out = OptMode::SearchExact;
  else if (s == "search-linear") *out = OptMode::SearchLinear;
  else if (s == "search") *out = OptMode::Search;
  else if (s == "auto") *out = OptMode::Auto;
  else return false;
  return true;
}

Json OptStats::json() const {
  Json j = Json::obj();
  j["nodes_before"] = nodes_before;
  j["nodes_after"] = nodes_after;
  j["constants_folded"] = folded;
  j["algebraic_simplified"] = simplified;
  j["cse_merged"] = cse;
  j["rematerialized"] = rematerialized;
  if (searched) {
    Json s = Json::obj();
    s["accepted"] = accepted;
    s["iterations"] = search.iterations;
    s["egraph_nodes"] = search.egraph_nodes;
    s["cost_before"] = search.cost_before;
    s["cost_after"] = search.cost_after;
    j["search"] = s;
  } else {
    j["search"] = Json();
  }
  return j;
}

Optimized optimize_mode(const Graph& g, const std::vector<uint32_t>& outputs, bool device, OptMode mode) {
  if (mode == OptMode::None) {
    Optimized o{g, outputs, {}};
    o.stats.nodes_before = o.stats.nodes_after = count_kept(g, outputs);
    return o;
  }
  if (mode == OptMode::Search || mode == OptMode::SearchExact || mode == OptMode::SearchLinear) {
    Simplified baseline = simplify(g, outputs, device, true);
    Simplified first = simplify(g, outputs, false, false);
    if (mode == OptMode::SearchLinear && !has_matrix_structure(first.g, first.out)) {
      OptStats st = baseline.st;
      st.nodes_before = count_kept(g, outputs);
      return finish(baseline, st, device);
    }
    CostModel model = device ? CostModel::Device : CostModel::Cpu;
    SearchStats ss;
    auto found = matrix_search(first.g, first.out, model, mode, &ss);
    // Both graphs are compared after the same clean-up (constants folded, transposes turned into flags).
    ss.cost_before = graph_cost(model, baseline.g, baseline.out);
    std::optional<Simplified> candidate;
    if (found) candidate = simplify(found->first, found->second, device, true);
    double cost = candidate ? graph_cost(model, candidate->g, candidate->out) : ss.cost_before;
    ss.cost_after = cost;
    bool accepted = candidate && cost < ss.cost_before * SEARCH_MIN_GAIN;
    Simplified& chosen = accepted ? *candidate : baseline;
    OptStats st = chosen.st;
    st.nodes_before = count_kept(g, outputs);
    st.searched = true;
    st.accepted = accepted;
    st.search = ss;
    return finish(chosen, st, device);
  }
  Simplified s = simplify(g, outputs, device, true);
  return finish(s, s.st, device);
}

}  // namespace rg
