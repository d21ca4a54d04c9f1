// Planning: fusion schedules, group compilation, the slot allocator and plan serialization.
// Follows the reference's src/plan.rs:184-238 (Allocator), 240-309 (aliases, arg kinds,
// fusability, hoisting), 311-414 (greedy and level schedules), 416-457 (compile_group) and
// 466-634 (build_fused / build_with).
#include "plan.h"
#include "optimize.h"

#include <algorithm>
#include <cstring>
#include <iterator>
#include <map>
#include <queue>
#include <set>

namespace rg {

namespace {

struct Allocator {
  std::vector<std::pair<DType, size_t>> slots;
  std::vector<bool> pinned;
  std::vector<uint32_t> refs;
  std::vector<size_t> free;
  bool reuse = true;
  std::vector<size_t> held;
  size_t live = 0, peak = 0;

  size_t new_slot(DType d, size_t n, bool pin) {
    slots.push_back({d, n});
    pinned.push_back(pin);
    refs.push_back(1);
    held.push_back(0);
    return slots.size() - 1;
  }
  size_t alloc(DType d, size_t n, bool exact = false) {
    size_t s = pick(d, n, exact);
    held[s] = n * dsize(d);
    live += held[s];
    peak = std::max(peak, live);
    return s;
  }
  size_t pick(DType d, size_t n, bool exact) {
    // A plan output sized exactly for its state handoff gets a buffer of its own: reusing one
    // freed by an earlier step would order it after that step's readers, so the independent
    // updates at the end of a training step could not run side by side.
    if (exact) return new_slot(d, n, false);
    // Reusing a large buffer for a small value would keep the large one busy for as long as the small one lives.
    int64_t best = -1;
    for (size_t k = 0; k < free.size(); k++) {
      size_t s = free[k];
      bool fits = exact ? slots[s].second == n : slots[s].second >= n && slots[s].second <= std::max<size_t>(n, 1) * 4;
      if (slots[s].first == d && fits) {
        if (best < 0 || slots[s].second < slots[free[(size_t)best]].second) best = (int64_t)k;
      }
    }
    if (best >= 0) {
      size_t s = free[(size_t)best];
      free[(size_t)best] = free.back();  // swap_remove
      free.pop_back();
      refs[s] = 1;
      return s;
    }
    return new_slot(d, n, false);
  }
  void release(size_t s) {
    refs[s] -= 1;
    if (refs[s] == 0 && !pinned[s]) {
      live -= held[s];
      if (reuse) free.push_back(s);
    }
  }
};

bool is_alias(const Graph& g, size_t id) {
  const Node& n = g.nodes[id];
  switch (n.op.kind) {
    case RG_OP_RESHAPE: case RG_OP_STOP_GRADIENT: case RG_OP_CUSTOM: return true;
    case RG_OP_CAST: return n.op.dt == g.nodes[n.inputs[0]].dtype;
    default: return false;
  }
}

bool arg_kind(const Shape& s, const Shape& shape, rg_arg_kind* k, size_t* row) {
  size_t n = numel(s);
  if (s == shape) {
    *k = RG_ARG_FULL;
  } else if (n == 1) {
    *k = RG_ARG_SPLAT;
  } else if (!s.empty() && !shape.empty() && s.back() == shape.back() && n == s.back()) {
    *k = RG_ARG_ROW;
    *row = n;
  } else {
    return false;
  }
  return true;
}

// Approximate nanoseconds per element; only the CPU plan's threading threshold uses it (plan.rs:267-276).
double op_cost_ns(const Op& op) {
  switch (op.kind) {
    case RG_OP_EXP: case RG_OP_LOG: case RG_OP_SIN: case RG_OP_COS: case RG_OP_TANH: return 0.6;
    case RG_OP_POW: return 10.0;
    case RG_OP_DIV: case RG_OP_SQRT: return 0.2;
    default: return 0.06;
  }
}

bool is_elementwise(const Op& op) {
  return op.is_unary_elementwise() || op.is_binary_elementwise() || op.kind == RG_OP_WHERE;
}

bool fusable(const Graph& g, size_t id, bool device) {
  const Node& n = g.nodes[id];
  if (!is_elementwise(n.op) || n.dtype == DType::I32) return false;
  if (device) return true;
  rg_arg_kind k;
  size_t row;
  for (uint32_t x : n.inputs)
    if (!arg_kind(g.shape(x), n.shape, &k, &row)) return false;
  return true;
}

bool on_cpu_for_metal(const Op& op, DType dtype, size_t n, const std::vector<DType>& arg_dtypes) {
  bool wide = dtype == DType::F64 || std::find(arg_dtypes.begin(), arg_dtypes.end(), DType::F64) != arg_dtypes.end();
  bool small_int = dtype == DType::I32 && n <= 64 &&
                   std::all_of(arg_dtypes.begin(), arg_dtypes.end(), [](DType d) { return d == DType::I32; });
  return wide || small_int || op.kind == RG_OP_RAND_NORMAL || op.kind == RG_OP_KEY_SPLIT;
}

bool leaf(const Node& n) { return n.op.kind == RG_OP_INPUT || n.op.kind == RG_OP_CONST; }

std::vector<bool> hoisted(const Graph& g, const std::vector<bool>& keep) {
  std::vector<bool> up(g.nodes.size(), false);
  for (size_t i = 0; i < g.nodes.size(); i++) {
    const Node& n = g.nodes[i];
    if (!keep[i] || leaf(n)) continue;
    bool ready = true, all_up = true;
    std::vector<DType> dts;
    for (uint32_t x : n.inputs) {
      ready &= up[x] || leaf(g.nodes[x]);
      all_up &= up[x];
      dts.push_back(g.dtype(x));
    }
    up[i] = ready && (on_cpu_for_metal(n.op, n.dtype, n.n(), dts) || (is_alias(g, i) && all_up));
  }
  return up;
}

struct Item {
  bool group;
  size_t node;
  std::vector<size_t> members;
  bool rows = false;     // a row group (members in node order)
  int64_t attn = -1;     // an attention step: the region's index
  bool attn_bwd = false;  // its backward step
};

// BroadcastTo nodes whose every kept consumer is a device-fusable node, and which are not plan
// outputs: fused kernels read their source through a broadcast index instead.
std::vector<bool> absorbed_broadcasts(const Graph& g, const std::vector<bool>& keep, const std::vector<uint32_t>& outputs,
                                      const Fuse& cfg) {
  std::vector<bool> abs(g.nodes.size(), false);
  if (!cfg.device || !cfg.absorb_broadcasts) return abs;
  std::vector<bool> any_use(g.nodes.size(), false), bad(g.nodes.size(), false);
  for (size_t i = 0; i < g.nodes.size(); i++) {
    if (!keep[i]) continue;
    const Node& n = g.nodes[i];
    bool dev_fusable = fusable(g, i, true) && (cfg.fuse_f64 || n.dtype != DType::F64);
    for (uint32_t x : n.inputs) {
      any_use[x] = true;
      if (!dev_fusable) bad[x] = true;
    }
  }
  for (uint32_t o : outputs) bad[o] = true;
  for (size_t i = 0; i < g.nodes.size(); i++)
    abs[i] = keep[i] && g.nodes[i].op.kind == RG_OP_BROADCAST_TO && any_use[i] && !bad[i];
  return abs;
}

// Whether a node reads an input that is neither its own shape nor a scalar.
bool indexed_inputs(const Graph& g, size_t i) {
  for (uint32_t x : g.nodes[i].inputs) {
    rg_arg_kind k;
    size_t row;
    if (!arg_kind(g.shape(x), g.nodes[i].shape, &k, &row) || (k != RG_ARG_FULL && k != RG_ARG_SPLAT)) return true;
  }
  return false;
}

bool reads_absorbed(const Graph& g, const std::vector<size_t>& members, const std::vector<bool>& abs) {
  for (size_t m : members)
    for (uint32_t x : g.nodes[m].inputs)
      if (abs[x]) return true;
  return false;
}

size_t distinct_external(const Graph& g, const std::vector<size_t>& members, const Node& extra) {
  std::set<uint32_t> s;
  auto in = [&](uint32_t x) { return std::find(members.begin(), members.end(), (size_t)x) != members.end(); };
  for (size_t m : members)
    for (uint32_t x : g.nodes[m].inputs)
      if (!in(x)) s.insert(x);
  for (uint32_t x : extra.inputs)
    if (!in(x)) s.insert(x);
  return s.size();
}

// Tails: fusable values whose every user is a tail of the same shape and dtype, ending in plan
// outputs (e.g. an optimizer's per-parameter update chain). Computed users-first.
std::vector<bool> tails(const Graph& g, const std::vector<bool>& keep, const std::vector<uint32_t>& outputs, const std::vector<bool>& abs,
                        const std::function<bool(size_t)>& dev_fusable) {
  size_t total = g.nodes.size();
  std::vector<bool> is_out(total, false), tail(total, false), used(total, false);
  for (uint32_t o : outputs) is_out[o] = true;
  std::vector<std::vector<uint32_t>> users(total);
  for (size_t i = 0; i < total; i++)
    if (keep[i])
      for (uint32_t x : g.nodes[i].inputs) users[x].push_back((uint32_t)i);
  for (size_t i = total; i-- > 0;) {
    const Node& n = g.nodes[i];
    if (!keep[i] || abs[i] || is_alias(g, i) || !dev_fusable(i)) continue;
    if (!is_out[i] && users[i].empty()) continue;
    bool ok = true;
    for (uint32_t u : users[i])
      ok &= tail[u] && g.nodes[u].shape == n.shape && g.nodes[u].dtype == n.dtype;
    tail[i] = ok;
  }
  return tail;
}

// Longest rows a row-group kernel keeps in one wavefront's registers.
constexpr size_t ROW_MAX = 1024;

// A last-axis reduction with kept dimensions, the seed of a row group: [rows..., L] -> [rows..., 1].
bool row_reduce(const Graph& g, size_t i) {
  const Node& n = g.nodes[i];
  if (n.op.kind != RG_OP_REDUCE || !n.op.keepdims || n.dtype == DType::I32) return false;
  const Shape& s = g.shape(n.inputs[0]);
  return s.size() >= 2 && s.back() >= 2 && s.back() <= ROW_MAX && n.op.v.size() == 1 && n.op.v[0] == s.size() - 1;
}

// Row groups, grown greedily in node order. A node joins the most recent group it reads from
// when its shape fits the group (the full rows [P..., L] or the row values [P..., 1]; reductions
// by their input) and none of its inputs depends on the group through a non-member, which keeps
// every group a single schedulable unit. Groups without a reduction are dropped: plain fused
// groups serve them. Hoisted, tail and absorbed nodes never join.
std::vector<std::vector<size_t>> row_groups(const Graph& g, const std::vector<bool>& keep, const std::vector<bool>& abs,
                                            const std::vector<bool>& excluded, const std::function<bool(size_t)>& dev_fusable,
                                            size_t max_bindings) {
  size_t total = g.nodes.size();
  struct RG {
    Shape full, row;
    DType dtype;
    std::vector<size_t> members;
    std::set<uint32_t> external;
    bool reduces = false;
  };
  std::vector<RG> groups;
  std::vector<int64_t> gid(total, -1);
  std::vector<std::vector<int64_t>> taint(total);  // sorted ids of groups a non-member depends on
  auto tainted = [&](uint32_t x, int64_t k) { return std::binary_search(taint[x].begin(), taint[x].end(), k); };
  for (size_t i = 0; i < total; i++) {
    if (!keep[i] || leaf(g.nodes[i])) continue;
    const Node& n = g.nodes[i];
    bool member_ok = !excluded[i] && !abs[i] && !is_alias(g, i);
    bool red = member_ok && row_reduce(g, i);
    bool elem = member_ok && dev_fusable(i);
    int64_t chosen = -1;
    if (red || elem) {
      for (uint32_t x : n.inputs) {
        int64_t k = gid[x];
        if (k < 0 || k <= chosen) continue;
        const RG& G = groups[(size_t)k];
        bool fits = n.dtype == G.dtype && (red ? g.shape(n.inputs[0]) == G.full : (n.shape == G.full || n.shape == G.row));
        if (!fits) continue;
        bool clean = true;
        for (uint32_t y : n.inputs) clean &= !tainted(y, k);
        if (!clean) continue;
        std::set<uint32_t> ext = G.external;
        for (uint32_t y : n.inputs)
          if (gid[y] != k) ext.insert(y);
        if (ext.size() + G.members.size() + 1 > max_bindings) continue;
        chosen = k;
      }
      if (chosen < 0) {
        const Shape& full = red ? g.shape(n.inputs[0]) : n.shape;
        if (full.size() >= 2 && full.back() >= 2 && full.back() <= ROW_MAX && (red || n.shape == full)) {
          RG G;
          G.full = full;
          G.row = full;
          G.row.back() = 1;
          G.dtype = n.dtype;
          groups.push_back(std::move(G));
          chosen = (int64_t)groups.size() - 1;
        }
      }
    }
    if (chosen >= 0) {
      RG& G = groups[(size_t)chosen];
      G.members.push_back(i);
      G.reduces |= red;
      for (uint32_t y : n.inputs)
        if (gid[y] != chosen) G.external.insert(y);
      gid[i] = chosen;
    }
    std::vector<int64_t> t;
    for (uint32_t x : n.inputs) {
      t.insert(t.end(), taint[x].begin(), taint[x].end());
      if (gid[x] >= 0) t.push_back(gid[x]);
    }
    std::sort(t.begin(), t.end());
    t.erase(std::unique(t.begin(), t.end()), t.end());
    if (gid[i] >= 0) t.erase(std::remove(t.begin(), t.end(), gid[i]), t.end());
    taint[i] = std::move(t);
  }
  // Producers: an ungrouped row-compatible node whose every user is in one kept group, and whose
  // inputs do not depend on that group, joins it (e.g. a gradient scaled before its row group).
  // Users first, so chains of producers join too.
  std::vector<std::vector<uint32_t>> users(total);
  for (size_t i = 0; i < total; i++)
    if (keep[i])
      for (uint32_t x : g.nodes[i].inputs) users[x].push_back((uint32_t)i);
  auto kept = [&](int64_t k) { return k >= 0 && groups[(size_t)k].reduces && groups[(size_t)k].members.size() >= 2; };
  for (size_t i = total; i-- > 0;) {
    if (!keep[i] || leaf(g.nodes[i]) || kept(gid[i]) || users[i].empty()) continue;
    const Node& n = g.nodes[i];
    if (excluded[i] || abs[i] || is_alias(g, i) || !dev_fusable(i)) continue;
    int64_t k = gid[users[i][0]];
    if (!kept(k)) continue;
    bool ok = true;
    for (uint32_t u : users[i]) ok &= gid[u] == k;
    RG& G = groups[(size_t)k];
    ok = ok && n.dtype == G.dtype && (n.shape == G.full || n.shape == G.row);
    for (uint32_t y : n.inputs) ok = ok && !tainted(y, k);
    if (!ok || G.external.size() + G.members.size() + n.inputs.size() + 1 > max_bindings) continue;
    if (gid[i] >= 0) {  // leave its dropped group
      auto& old = groups[(size_t)gid[i]].members;
      old.erase(std::remove(old.begin(), old.end(), i), old.end());
    }
    G.members.insert(std::lower_bound(G.members.begin(), G.members.end(), i), i);
    G.external.erase((uint32_t)i);
    for (uint32_t y : n.inputs) G.external.insert(y);
    gid[i] = k;
  }
  // Column reductions: a reduction over every axis but the last of a value of a kept group's full
  // shape joins that group, folded from the rows the group walks anyway (e.g. a layer norm's
  // scale and shift gradients beside its input gradient). The value is a member, a value the
  // group reads, or an ungrouped elementwise node read only by such reductions that shares an
  // input with the group (it joins too). Nothing the group computes may depend on the reduction,
  // and no value it reads may depend on the group through a non-member.
  auto leading_reduce = [&](size_t i) {
    const Node& n = g.nodes[i];
    if (n.op.kind != RG_OP_REDUCE || n.dtype == DType::I32) return false;
    const Shape& s = g.shape(n.inputs[0]);
    if (s.size() < 2 || s.back() > (int64_t)ROW_MAX || n.op.v.size() + 1 != s.size()) return false;
    Shape ax = n.op.v;
    std::sort(ax.begin(), ax.end());
    for (size_t q = 0; q < ax.size(); q++)
      if (ax[q] != (int64_t)q) return false;
    return true;
  };
  auto reaches_group = [&](size_t from, int64_t k) {  // a member of group k depends on `from`
    size_t last = groups[(size_t)k].members.back();
    std::vector<size_t> stack = {from};
    std::set<size_t> seen;
    while (!stack.empty()) {
      size_t x = stack.back();
      stack.pop_back();
      for (uint32_t u : users[x]) {
        if (u > last || !seen.insert(u).second) continue;
        if (gid[u] == k) return true;
        stack.push_back(u);
      }
    }
    return false;
  };
  for (size_t i = 0; i < total; i++) {
    if (!keep[i] || gid[i] >= 0 || excluded[i] || abs[i] || !leading_reduce(i)) continue;
    const Node& n = g.nodes[i];
    const uint32_t x = n.inputs[0];
    const Shape& xs = g.shape(x);
    auto fits = [&](int64_t k) { return kept(k) && groups[(size_t)k].full == xs && groups[(size_t)k].dtype == n.dtype; };
    int64_t k = -1;
    bool pull = false;
    if (fits(gid[x])) {
      k = gid[x];
    } else {
      for (size_t q = 0; q < groups.size() && k < 0; q++)
        if (fits((int64_t)q) && groups[q].external.count(x) && !tainted(x, (int64_t)q)) k = (int64_t)q;
      const Node& xn = g.nodes[x];
      bool pullable = k < 0 && !kept(gid[x]) && keep[x] && !leaf(xn) && !excluded[x] && !abs[x] && !is_alias(g, x) && dev_fusable(x);
      for (uint32_t u : users[x]) pullable = pullable && leading_reduce(u) && g.shape(g.nodes[u].inputs[0]) == xs;
      for (size_t q = 0; q < groups.size() && pullable && k < 0; q++) {
        if (!fits((int64_t)q)) continue;
        bool ok = true, shared = false;
        for (uint32_t y : xn.inputs) {
          ok = ok && !tainted(y, (int64_t)q);
          shared = shared || gid[y] == (int64_t)q || groups[q].external.count(y);
        }
        if (ok && shared) {
          k = (int64_t)q;
          pull = true;
        }
      }
    }
    if (k < 0 || reaches_group(i, k)) continue;
    RG& G = groups[(size_t)k];
    std::set<uint32_t> ext = G.external;
    if (pull)
      for (uint32_t y : g.nodes[x].inputs)
        if (gid[y] != k) ext.insert(y);
    if (!pull && gid[x] != k) ext.insert(x);
    if (ext.size() + G.members.size() + 2 > max_bindings) continue;
    G.external = std::move(ext);
    if (pull) {
      if (gid[x] >= 0) {  // leave its dropped group
        auto& old = groups[(size_t)gid[x]].members;
        old.erase(std::remove(old.begin(), old.end(), (size_t)x), old.end());
      }
      G.members.insert(std::lower_bound(G.members.begin(), G.members.end(), (size_t)x), (size_t)x);
      gid[x] = k;
    }
    G.members.insert(std::lower_bound(G.members.begin(), G.members.end(), i), i);
    gid[i] = k;
  }
  std::vector<std::vector<size_t>> out;
  for (auto& G : groups)
    if (G.reduces && G.members.size() >= 2) out.push_back(G.members);
  return out;
}

// `keep`: the nodes to schedule; `keep_all`: every node the outputs reach in the graph, including
// the reshapes and transposes attention steps read through, which carry the row groups'
// dependence tracking.
std::vector<Item> schedule_levels(const Graph& g, const std::vector<bool>& keep, const std::vector<bool>& keep_all,
                                  const std::vector<uint32_t>& outputs, const Fuse& cfg, const std::vector<bool>& abs,
                                  const std::vector<int64_t>& claimed, const std::vector<std::vector<uint32_t>>& attn_inputs) {
  const size_t n_attn_units = attn_inputs.size();
  std::vector<bool> up = cfg.hoist ? hoisted(g, keep) : std::vector<bool>(g.nodes.size(), false);
  std::vector<Item> items;
  for (size_t i = 0; i < g.nodes.size(); i++)
    if (up[i]) items.push_back({false, i, {}});
  std::function<bool(size_t)> dev_fusable = [&](size_t i) {
    return fusable(g, i, true) && (cfg.fuse_f64 || g.nodes[i].dtype != DType::F64);
  };
  std::vector<bool> tail = cfg.sink_tails ? tails(g, keep, outputs, abs, dev_fusable) : std::vector<bool>(g.nodes.size(), false);
  const size_t total = g.nodes.size();
  for (size_t i = 0; i < total; i++) tail[i] = tail[i] && claimed[i] < 0;
  std::vector<std::vector<size_t>> rgs;
  std::vector<int64_t> rg_of(total, -1);
  if (cfg.row_groups) {
    std::vector<bool> excluded(total, false);
    for (size_t i = 0; i < total; i++) excluded[i] = up[i] || tail[i] || claimed[i] >= 0;
    rgs = row_groups(g, keep_all, abs, excluded, dev_fusable, cfg.max_bindings);
    for (size_t k = 0; k < rgs.size(); k++)
      for (size_t m : rgs[k]) rg_of[m] = (int64_t)k;
  }
  // Scheduling units in a topological order of the graph with each row group contracted to one
  // unit (unit total + k) and each attention step to one (unit total + rgs.size() + its index),
  // ties broken by node order.
  const size_t n_units = total + rgs.size() + n_attn_units;
  auto active = [&](size_t i) { return keep[i] && !up[i] && !leaf(g.nodes[i]); };
  auto unit_of = [&](size_t i) -> size_t {
    if (claimed[i] >= 0) return total + rgs.size() + (size_t)claimed[i];
    return rg_of[i] >= 0 ? total + (size_t)rg_of[i] : i;
  };
  std::vector<std::vector<size_t>> unit_users(n_units);
  std::vector<size_t> indeg(n_units, 0), first(n_units, SIZE_MAX);
  for (size_t i = 0; i < total; i++) {
    if (!active(i)) continue;
    size_t u = unit_of(i);
    first[u] = std::min(first[u], i);
    std::set<size_t> deps;
    for (uint32_t x : g.nodes[i].inputs)
      if (active(x) && unit_of(x) != u) deps.insert(unit_of(x));
    for (size_t d : deps) {
      unit_users[d].push_back(u);
      indeg[u]++;
    }
  }
  // An attention unit reads its operands through views of other values: those are its inputs.
  for (size_t k = 0; k < n_attn_units; k++) {
    size_t u = total + rgs.size() + k;
    if (first[u] == SIZE_MAX) continue;
    std::set<size_t> deps;
    for (uint32_t x : attn_inputs[k])
      if (active(x) && unit_of(x) != u) deps.insert(unit_of(x));
    for (size_t d : deps)
      if (std::find(unit_users[d].begin(), unit_users[d].end(), u) == unit_users[d].end()) {
        unit_users[d].push_back(u);
        indeg[u]++;
      }
  }
  std::priority_queue<std::pair<size_t, size_t>, std::vector<std::pair<size_t, size_t>>, std::greater<>> ready;
  for (size_t u = 0; u < n_units; u++)
    if (first[u] != SIZE_MAX && indeg[u] == 0) ready.push({first[u], u});
  std::vector<size_t> order;
  while (!ready.empty()) {
    size_t u = ready.top().second;
    ready.pop();
    order.push_back(u);
    for (size_t v : unit_users[u])
      if (--indeg[v] == 0) ready.push({first[v], v});
  }
  size_t n_real = 0;
  for (size_t u = 0; u < n_units; u++) n_real += first[u] != SIZE_MAX;
  if (order.size() != n_real) throw std::logic_error("planner: scheduling units depend on each other in a cycle");
  std::vector<size_t> sunk;
  std::vector<std::vector<size_t>> sunk_comps;
  std::vector<size_t> level(total, 0);
  // Members of each attention unit, in node order.
  std::vector<std::vector<size_t>> attn_members(n_attn_units);
  for (size_t i = 0; i < total; i++)
    if (claimed[i] >= 0) attn_members[(size_t)claimed[i]].push_back(i);
  std::vector<std::vector<size_t>> by_level;  // node ids, and total + k for unit k
  for (size_t u : order) {
    if (u >= total) {
      const auto& members = u < total + rgs.size() ? rgs[u - total] : attn_members[u - total - rgs.size()];
      size_t deepest = 0;
      for (size_t m : members)
        for (uint32_t x : g.nodes[m].inputs)
          if (unit_of(x) != u) deepest = std::max(deepest, level[x]);
      if (u >= total + rgs.size())
        for (uint32_t x : attn_inputs[u - total - rgs.size()]) deepest = std::max(deepest, level[x]);
      for (size_t m : members) level[m] = deepest + 1;
      if (by_level.size() <= deepest + 1) by_level.resize(deepest + 2);
      by_level[deepest + 1].push_back(u);
      continue;
    }
    size_t i = u;
    const Node& n = g.nodes[i];
    size_t deepest = 0;
    for (uint32_t x : n.inputs) deepest = std::max(deepest, level[x]);
    if (abs[i]) {
      level[i] = deepest;  // a view of its source: no kernel, no level of its own
      continue;
    }
    if (tail[i]) {
      sunk.push_back(i);  // placed in the final level below
      continue;
    }
    bool joins = dev_fusable(i) && deepest > 0;
    if (joins) {
      for (uint32_t x : n.inputs) {
        if (!(level[x] < deepest ||
              (dev_fusable(x) && rg_of[x] < 0 && g.nodes[x].shape == n.shape && g.nodes[x].dtype == n.dtype))) {
          joins = false;
          break;
        }
      }
    }
    level[i] = (is_alias(g, i) || joins) ? deepest : deepest + 1;
    if (by_level.size() <= level[i]) by_level.resize(level[i] + 1);
    by_level[level[i]].push_back(i);
  }
  // Tails read earlier levels or same-shape tails only, so one last level can hold them all;
  // node order keeps each producer ahead of its users within a group. The tails connected
  // through one another (an optimizer's moments and the parameter update they feed) are placed
  // together, component after component, so that a group holding part of a chain holds all of it
  // when the operand limit allows: no moment is written by one kernel and read back by the next.
  if (!sunk.empty()) {
    std::map<size_t, size_t> parent;
    std::function<size_t(size_t)> root = [&](size_t x) { return parent[x] == x ? x : parent[x] = root(parent[x]); };
    for (size_t i : sunk) parent[i] = i;
    for (size_t i : sunk)
      for (uint32_t x : g.nodes[i].inputs)
        if (parent.count(x)) parent[root(i)] = root(x);
    std::map<size_t, std::vector<size_t>> comps;  // keyed by each component's first node
    std::map<size_t, size_t> first_of;
    for (size_t i : sunk) {
      size_t r = root(i);
      if (!first_of.count(r)) first_of[r] = i;
      comps[first_of[r]].push_back(i);
    }
    std::vector<size_t> ordered;
    for (auto& [first_node, members] : comps) {
      ordered.insert(ordered.end(), members.begin(), members.end());
      sunk_comps.push_back(members);
    }
    by_level.push_back(ordered);
  }
  // Buffers a group of tails binds: its distinct external inputs and the members it writes out
  // (plan outputs, or values read outside the group).
  std::vector<bool> is_out(total, false);
  for (uint32_t o : outputs) is_out[o] = true;
  std::vector<std::vector<uint32_t>> users_of(total);
  if (!sunk.empty())
    for (size_t i = 0; i < total; i++)
      if (keep[i])
        for (uint32_t x : g.nodes[i].inputs) users_of[x].push_back((uint32_t)i);
  auto bindings = [&](const std::vector<size_t>& members) {
    std::set<size_t> in(members.begin(), members.end());
    std::set<uint32_t> ext;
    size_t written = 0;
    for (size_t m : members) {
      for (uint32_t x : g.nodes[m].inputs)
        if (!in.count(x)) ext.insert(x);
      bool out = is_out[m];
      for (uint32_t u : users_of[m]) out |= !in.count(u);
      written += out;
    }
    return ext.size() + written;
  };
  for (size_t lv = 0; lv < by_level.size(); lv++) {
    const auto& nodes = by_level[lv];
    std::vector<std::vector<size_t>> groups;
    std::vector<size_t> aliases, rows, attns;
    if (!sunk_comps.empty() && lv + 1 == by_level.size()) {
      // The tails, one group per component (one parameter's update chain, say): independent
      // chains stay separate kernels, which the runtime launches side by side, so each chain's
      // elements spread over the whole device instead of one thread walking every chain.
      std::vector<size_t> loose;
      for (const auto& comp : sunk_comps) {
        if (bindings(comp) <= cfg.max_bindings) groups.push_back(comp);
        else loose.insert(loose.end(), comp.begin(), comp.end());
      }
      for (size_t i : loose) {
        const Node& n = g.nodes[i];
        int64_t found = -1;
        for (size_t k = groups.size(); k-- > 0;)
          if (g.nodes[groups[k][0]].shape == n.shape && g.nodes[groups[k][0]].dtype == n.dtype) {
            found = (int64_t)k;
            break;
          }
        if (found >= 0 && distinct_external(g, groups[(size_t)found], n) + groups[(size_t)found].size() + 1 <= cfg.max_bindings)
          groups[(size_t)found].push_back(i);
        else
          groups.push_back({i});
      }
      for (auto& m : groups) {
        std::sort(m.begin(), m.end());
        if (m.size() >= 2 || reads_absorbed(g, m, abs) || (cfg.device && indexed_inputs(g, m[0]))) items.push_back({true, 0, m});
        else
          for (size_t x : m) items.push_back({false, x, {}});
      }
      continue;
    }
    for (size_t i : nodes) {
      if (i >= total + rgs.size()) {
        attns.push_back(i - total - rgs.size());
        continue;
      }
      if (i >= total) {
        rows.push_back(i - total);  // row groups read lower levels only: they follow the groups
        continue;
      }
      const Node& n = g.nodes[i];
      if (is_alias(g, i)) {
        aliases.push_back(i);  // its input is produced in this level: emit it after the level's groups
      } else if (dev_fusable(i)) {
        // Most recent open group of this shape and dtype; its members may feed the node.
        int64_t found = -1;
        for (size_t k = groups.size(); k-- > 0;) {
          const Node& f = g.nodes[groups[k][0]];
          if (f.shape == n.shape && f.dtype == n.dtype) {
            found = (int64_t)k;
            break;
          }
        }
        bool fits = found >= 0 &&
                    distinct_external(g, groups[(size_t)found], n) + groups[(size_t)found].size() + 1 <= cfg.max_bindings;
        if (found >= 0 && fits) groups[(size_t)found].push_back(i);
        else groups.push_back({i});
      } else {
        items.push_back({false, i, {}});
      }
    }
    for (auto& m : groups) {
      // A node reading an absorbed broadcast needs the fused kernel's broadcast indexing; one
      // reading a row vector or a broadcast runs faster as a generated kernel than through the
      // general strided instruction.
      if (m.size() >= 2 || reads_absorbed(g, m, abs) || (cfg.device && indexed_inputs(g, m[0]))) items.push_back({true, 0, m});
      else
        for (size_t x : m) items.push_back({false, x, {}});
    }
    for (size_t k : rows) items.push_back({true, 0, rgs[k], true});
    for (size_t k : attns) items.push_back({false, 0, {}, false, (int64_t)(k / 2), (k % 2) == 1});
    for (size_t a : aliases) items.push_back({false, a, {}});
  }
  return items;
}

// Greedy fusion with a single open group: an instruction that does not depend on the group is
// emitted ahead of it, and the first one reading a group member ends the group, so a group can
// never wait on its own output (plan.rs:311-350).
std::vector<Item> schedule(const Graph& g, const std::vector<bool>& keep, const std::vector<bool>& keep_all,
                           const std::vector<uint32_t>& outputs, const Fuse& cfg, const std::vector<bool>& abs,
                           const std::vector<int64_t>& claimed, const std::vector<std::vector<uint32_t>>& attn_inputs) {
  if (cfg.device && cfg.levels) return schedule_levels(g, keep, keep_all, outputs, cfg, abs, claimed, attn_inputs);
  std::vector<Item> items;
  std::vector<size_t> open;
  auto close = [&]() {
    double cost = 0;
    for (size_t m : open) cost += op_cost_ns(g.nodes[m].op) * (double)g.nodes[m].n();
    if ((open.size() >= (cfg.device ? 2u : 1u) || (!open.empty() && reads_absorbed(g, open, abs))) && cost >= cfg.parallel_ns) {
      items.push_back({true, 0, open});
    } else {
      for (size_t m : open) items.push_back({false, m, {}});
    }
    open.clear();
  };
  std::vector<bool> up = (cfg.device && cfg.hoist) ? hoisted(g, keep) : std::vector<bool>(g.nodes.size(), false);
  for (size_t i = 0; i < g.nodes.size(); i++)
    if (up[i]) items.push_back({false, i, {}});
  for (size_t i = 0; i < g.nodes.size(); i++) {
    const Node& n = g.nodes[i];
    if (!keep[i] || up[i] || leaf(n) || abs[i]) continue;
    if (fusable(g, i, cfg.device) && !(cfg.device && !cfg.fuse_f64 && n.dtype == DType::F64)) {
      bool same = open.empty() || (g.nodes[open[0]].shape == n.shape && g.nodes[open[0]].dtype == n.dtype);
      // Only device kernels bound their operand count; a CPU group's inputs need no count.
      if (!same || (cfg.device && distinct_external(g, open, n) + open.size() + 1 > cfg.max_bindings)) close();
      open.push_back(i);
    } else {
      bool reads = false;
      for (uint32_t x : n.inputs) reads |= std::find(open.begin(), open.end(), (size_t)x) != open.end();
      if (reads) close();
      items.push_back({false, i, {}});
    }
  }
  close();
  return items;
}

// Recomputation instead of storage. A group C that reads values X of an earlier group G walking
// the same elements (two fused groups of one shape, or two row groups over the same rows), where
// C is X's only other reader, recomputes X: the members of G that X depends on, back to values C
// reads anyway, are added to C (a node may then run in two kernels; a row group recomputes per-row
// reductions such as a layer norm's mean and variance). G stops writing what nobody else reads.
// Done when C reads no more full-size values than before (G then writes fewer), e.g. an
// activation's backward that would read every intermediate of its forward, or a layer norm's
// backward reading the centred input and the normalised values. Members stay sorted by node id.
void rematerialize(const Graph& g, const std::vector<bool>& keep, const std::vector<uint32_t>& outputs, std::vector<Item>& items,
                   size_t max_bindings) {
  const size_t total = g.nodes.size();
  std::vector<bool> is_out(total, false);
  for (uint32_t o : outputs) is_out[o] = true;
  std::vector<std::vector<uint32_t>> users(total);
  for (size_t i = 0; i < total; i++)
    if (keep[i])
      for (uint32_t x : g.nodes[i].inputs) users[x].push_back((uint32_t)i);
  std::vector<int64_t> item_of(total, -1);  // the group that first computes a node
  auto eligible = [&](const Item& it) { return it.group && it.attn < 0; };
  auto in = [](const std::vector<size_t>& v, size_t x) { return std::binary_search(v.begin(), v.end(), x); };
  // The shape a group walks: a row group's reduction input, a fused group's members' shape.
  auto walk_of = [&](const Item& it) -> Shape {
    if (it.rows)
      for (size_t m : it.members)
        if (g.nodes[m].op.kind == RG_OP_REDUCE) return g.shape(g.nodes[m].inputs[0]);
    return g.nodes[it.members[0]].shape;
  };
  auto last_axis_reduce = [&](size_t m) {
    const Node& n = g.nodes[m];
    return n.op.kind == RG_OP_REDUCE && n.op.v.size() == 1 && n.op.v[0] + 1 == (int64_t)g.shape(n.inputs[0]).size();
  };
  for (size_t ci = 0; ci < items.size(); ci++) {
    Item& C = items[ci];
    if (eligible(C)) {
      const Shape cf = walk_of(C);
      const size_t cn = numel(cf), rows = cf.empty() || cf.back() == 0 ? cn : cn / (size_t)cf.back();
      const DType cdt = g.nodes[C.members[0]].dtype;
      std::map<size_t, std::vector<uint32_t>> cand;  // producer group -> values C would recompute
      for (size_t u : C.members)
        for (uint32_t x : g.nodes[u].inputs) {
          if (in(C.members, x) || item_of[x] < 0 || is_out[x]) continue;
          const Item& G = items[(size_t)item_of[x]];
          const Node& n = g.nodes[x];
          // Same walk: a fused group's values from a fused group of its shape; a row group's full
          // or per-row values from a row group over the same rows.
          if (G.rows != C.rows || walk_of(G) != cf || n.dtype != cdt) continue;
          if (!(n.shape == cf || (C.rows && numel(n.shape) == rows && (n.op.kind != RG_OP_REDUCE || last_axis_reduce(x))))) continue;
          bool only = true;
          for (uint32_t w : users[x]) only &= in(G.members, w) || in(C.members, w);
          auto& v = cand[(size_t)item_of[x]];
          if (only && std::find(v.begin(), v.end(), x) == v.end()) v.push_back(x);
        }
      for (auto& [gi, xs] : cand) {
        const Item& G = items[gi];
        std::set<uint32_t> ext_c;
        for (size_t u : C.members)
          for (uint32_t y : g.nodes[u].inputs)
            if (!in(C.members, y)) ext_c.insert(y);
        // G's members that G writes whatever C does (read outside G and C, or plan outputs).
        auto written = [&](uint32_t y) {
          if (is_out[y]) return true;
          for (uint32_t w : users[y])
            if (!in(G.members, w) && !in(C.members, w)) return true;
          return false;
        };
        // X's ancestors within G, up to the values C reads anyway; with `stop`, also up to the
        // values G writes anyway, which C then reads instead of recomputing them from their own
        // inputs (a layer norm's backward reads the residual sum the forward stores rather than
        // the two values it adds).
        struct Option {
          std::vector<size_t> closure;
          std::set<uint32_t> fresh;
          size_t full = 0;
          bool ok = true;
        };
        auto option = [&](bool stop) {
          Option o;
          std::vector<uint32_t> stack(xs.begin(), xs.end());
          while (!stack.empty()) {
            uint32_t x = stack.back();
            stack.pop_back();
            if (std::find(o.closure.begin(), o.closure.end(), (size_t)x) != o.closure.end()) continue;
            o.closure.push_back(x);
            // Only reductions a row group folds per row may be recomputed.
            if (g.nodes[x].op.kind == RG_OP_REDUCE && !(C.rows && last_axis_reduce(x))) o.ok = false;
            for (uint32_t y : g.nodes[x].inputs) {
              const bool is_x = std::find(xs.begin(), xs.end(), y) != xs.end();
              if (in(G.members, y) && (!ext_c.count(y) || is_x) && (is_x || !stop || !written(y))) stack.push_back(y);
            }
          }
          std::sort(o.closure.begin(), o.closure.end());
          // Full-size values C would newly read.
          for (size_t m : o.closure)
            for (uint32_t y : g.nodes[m].inputs)
              if (!in(o.closure, y) && !in(C.members, y) && !ext_c.count(y)) o.fresh.insert(y);
          for (uint32_t y : o.fresh) o.full += numel(g.shape(y)) == cn;
          return o;
        };
        Option a = option(false), b = option(true);
        // The fewer full-size reads; on a tie the shorter recomputation.
        Option& best = (b.ok && (!a.ok || b.full < a.full || (b.full == a.full && b.closure.size() < a.closure.size()))) ? b : a;
        const std::vector<size_t>& closure = best.closure;
        // Full-size values C would newly read, against the full-size values it no longer reads
        // (and G no longer writes): a trade of equal reads still saves G's writes.
        size_t saved = 0;
        for (uint32_t x : xs) saved += numel(g.shape(x)) == cn;
        if (!best.ok || saved == 0 || best.full > saved || closure.size() > 64 ||
            ext_c.size() + best.fresh.size() + C.members.size() + closure.size() > max_bindings)
          continue;
        std::vector<size_t> merged;
        std::set_union(C.members.begin(), C.members.end(), closure.begin(), closure.end(), std::back_inserter(merged));
        C.members = std::move(merged);
      }
    }
    if (eligible(C))
      for (size_t m : C.members)
        if (item_of[m] < 0) item_of[m] = (int64_t)ci;
  }
}

Fused compile_group(const Graph& g, const std::vector<size_t>& members, const std::vector<size_t>& slot_of,
                    const std::vector<std::pair<size_t, size_t>>& out_slots, const std::vector<bool>& abs, bool rows) {
  const Node& first = g.nodes[members[0]];
  // A row group's shape is the full rows its reductions read; a fused group's is its members'.
  Shape shape = first.shape;
  if (rows)
    for (size_t m : members)
      if (g.nodes[m].op.kind == RG_OP_REDUCE) shape = g.shape(g.nodes[m].inputs[0]);
  Fused f;
  std::vector<std::pair<uint32_t, std::pair<bool, size_t>>> ext;  // (node, operand)
  size_t regs = 0;
  auto member = [&](uint32_t x) { return std::find(members.begin(), members.end(), (size_t)x) != members.end(); };
  for (size_t m : members) {
    for (uint32_t x : g.nodes[m].inputs) {
      bool seen = member(x);
      for (auto& e : ext) seen |= e.first == x;
      if (seen) continue;
      rg_arg_kind kind;
      size_t row = 0;
      // An absorbed broadcast is read from its source, whose slot it shares.
      const Shape& xs = abs[x] ? g.shape(g.nodes[x].inputs[0]) : g.shape(x);
      if (!arg_kind(xs, shape, &kind, &row)) kind = RG_ARG_BROADCAST;
      f.input_shapes.push_back(xs);
      std::pair<bool, size_t> operand;
      size_t reg = SIZE_MAX;
      if (kind == RG_ARG_FULL) {
        operand = {false, f.inputs.size()};
      } else {
        reg = regs++;
        operand = {true, reg};
      }
      f.inputs.push_back({slot_of[x], kind, row, reg});
      ext.push_back({x, operand});
    }
  }
  std::vector<size_t> reg_of(g.nodes.size(), SIZE_MAX);
  for (size_t m : members) {
    MicroOp mo;
    mo.op = g.nodes[m].op;
    for (uint32_t x : g.nodes[m].inputs) {
      bool found = false;
      for (auto& e : ext)
        if (e.first == x) {
          mo.args.push_back(e.second);
          found = true;
          break;
        }
      if (!found) mo.args.push_back({true, reg_of[x]});
    }
    reg_of[m] = regs;
    mo.reg = regs;
    f.ops.push_back(std::move(mo));
    regs++;
  }
  for (auto& [m, s] : out_slots) f.outputs.push_back({reg_of[m], s});
  f.dtype = first.dtype;
  f.n = numel(shape);
  f.regs = regs;
  f.shape = shape;
  f.row_len = rows ? shape.back() : 0;
  return f;
}

rg_mode binary_mode(const Op& op, const Shape& shape, const std::vector<Shape>& args) {
  if (!op.is_binary_elementwise()) return RG_MODE_SAME;
  const Shape &a = args[0], &b = args[1];
  auto one = [](const Shape& s) { return numel(s) == 1; };
  if (a == shape && b == shape) return RG_MODE_SAME;
  if (one(a) && b == shape) return RG_MODE_ASCALAR;
  if (a == shape && one(b)) return RG_MODE_BSCALAR;
  return RG_MODE_GENERAL;
}

Plan build_with(const Graph& g, const std::vector<uint32_t>& outputs, bool reuse, const Fuse* fuse) {
  std::vector<bool> keep = g.reachable(outputs);  // narrowed below when attention steps replace nodes
  const std::vector<bool> keep_all = keep;
  size_t total = g.nodes.size();
  std::vector<uint32_t> uses(total, 0);

  Allocator a;
  a.reuse = reuse;
  std::vector<size_t> value_slot(total, SIZE_MAX);
  Plan p;
  p.input_slots.assign(g.n_inputs, 0);
  p.input_ns.assign(g.n_inputs, 0);
  for (size_t i = 0; i < total; i++) {
    const Node& node = g.nodes[i];
    if (node.op.kind == RG_OP_INPUT) {
      size_t s = a.new_slot(node.dtype, node.n(), true);
      p.input_slots[node.op.a] = s;
      p.input_ns[node.op.a] = node.n();
      value_slot[i] = s;
    } else if (node.op.kind == RG_OP_CONST && keep[i]) {
      size_t s = a.new_slot(node.dtype, node.n(), true);
      p.consts.push_back({s, node.op.t});
      value_slot[i] = s;
    }
  }

  // Attention regions: members are computed by the fused steps, so their reads do not count;
  // each step reads its region's operands instead (the backward also O and the mask).
  std::vector<AttnRegion> regions;
  std::vector<int64_t> claimed(total, -1);  // attention unit: 2 * region (+ 1 for the backward)
  if (fuse && fuse->attention && fuse->device && fuse->levels) regions = match_attention(g, keep, outputs);
  // The operand views each step reads (q, k, v; the backward also O and dO), in that order,
  // then the mask.
  auto region_views = [&](const AttnRegion& r, bool bwd) {
    std::vector<AttnOperand> in = {r.in_q, r.in_k, r.in_v};
    if (bwd) {
      in.push_back(r.out_o);
      in.push_back(r.in_do);
    }
    return in;
  };
  auto region_inputs = [&](const AttnRegion& r, bool bwd) {
    std::vector<uint32_t> in;
    for (const AttnOperand& v : region_views(r, bwd)) in.push_back(v.node);
    if (r.mask >= 0) in.push_back((uint32_t)r.mask);
    return in;
  };
  for (size_t k = 0; k < regions.size(); k++) {
    const AttnRegion& r = regions[k];
    for (int b = 0; b < 2; b++)
      if (!b || r.has_bwd)
        for (uint32_t m : b ? r.bwd : r.fwd) claimed[m] = (int64_t)(2 * k + b);
  }
  if (!regions.empty()) {
    // Values only the replaced nodes read (e.g. the transposes that split the heads, now read
    // through views) are no longer computed.
    std::vector<bool> live(total, false);
    std::vector<uint32_t> stack(outputs.begin(), outputs.end());
    std::vector<bool> region_done(2 * regions.size(), false);
    while (!stack.empty()) {
      uint32_t x = stack.back();
      stack.pop_back();
      if (live[x]) continue;
      live[x] = true;
      if (claimed[x] >= 0) {
        size_t u = (size_t)claimed[x];
        if (region_done[u]) continue;
        region_done[u] = true;
        const AttnRegion& r = regions[u / 2];
        for (uint32_t y : region_inputs(r, u % 2)) stack.push_back(y);  // the backward's include the forward's O
        for (uint32_t m : u % 2 ? r.bwd : r.fwd) live[m] = true;
        continue;
      }
      for (uint32_t y : g.nodes[x].inputs) stack.push_back(y);
    }
    for (size_t i = 0; i < total; i++)
      if (claimed[i] < 0) keep[i] = keep[i] && live[i];
  }
  std::vector<size_t> stats_slot(regions.size(), SIZE_MAX);
  // One packed copy of each mask (node and broadcast shape), built by the first forward reading it.
  std::map<std::vector<int64_t>, size_t> mask_tables;

  std::vector<Item> items;
  std::vector<bool> abs = fuse ? absorbed_broadcasts(g, keep, outputs, *fuse) : std::vector<bool>(total, false);
  std::vector<bool> exact(total, false);
  if (fuse && fuse->exact_outputs)
    for (uint32_t o : outputs) exact[o] = true;
  if (fuse) {
    std::vector<std::vector<uint32_t>> attn_inputs(2 * regions.size());
    for (size_t k = 0; k < regions.size(); k++) {
      attn_inputs[2 * k] = region_inputs(regions[k], false);
      if (regions[k].has_bwd) attn_inputs[2 * k + 1] = region_inputs(regions[k], true);
    }
    items = schedule(g, keep, keep_all, outputs, *fuse, abs, claimed, attn_inputs);
  } else {
    for (size_t i = 0; i < total; i++)
      if (keep[i] && !leaf(g.nodes[i])) items.push_back({false, i, {}});
  }
  for (auto& item : items)
    if (item.group) std::sort(item.members.begin(), item.members.end());  // node order is topological
  if (fuse && fuse->remat) rematerialize(g, keep, outputs, items, fuse->max_bindings);

  // Reads of each value by later plan steps: a group's reads of its own members are registers,
  // an attention step reads its region's operands, an absorbed broadcast reads its source (as an
  // alias, on first use); plan outputs stay live past the last step.
  for (const auto& item : items) {
    if (item.attn >= 0) {
      for (uint32_t x : region_inputs(regions[(size_t)item.attn], item.attn_bwd)) uses[x]++;
    } else if (item.group) {
      for (size_t m : item.members)
        for (uint32_t x : g.nodes[m].inputs)
          if (!std::binary_search(item.members.begin(), item.members.end(), (size_t)x)) uses[x]++;
    } else {
      for (uint32_t x : g.nodes[item.node].inputs) uses[x]++;
    }
  }
  for (size_t i = 0; i < total; i++)
    if (keep[i] && abs[i] && claimed[i] < 0) uses[g.nodes[i].inputs[0]]++;
  for (uint32_t o : outputs) uses[o]++;

  for (auto& item : items) {
    if (item.attn >= 0) {
      const AttnRegion& r = regions[(size_t)item.attn];
      const bool bwd = item.attn_bwd;
      Step st;
      st.attn = true;
      Attn& at = st.att;
      at.backward = bwd;
      at.shape = attn_shape(r, g);
      at.div = r.div;
      at.fill = r.fill;
      std::vector<uint32_t> ins = region_inputs(r, bwd);
      at.mask_slot = r.mask >= 0 ? (int64_t)value_slot[(size_t)r.mask] : -1;
      auto view = [&](const AttnOperand& o) { return AttnView{value_slot[o.node], o.offset, o.sb, o.sh, o.st}; };
      for (const AttnOperand& o : region_views(r, bwd)) at.in.push_back(view(o));
      if (!bwd) stats_slot[(size_t)item.attn] = a.new_slot(DType::F32, attn_stats_words(r, g), true);
      at.stats_slot = stats_slot[(size_t)item.attn];
      if (r.mask >= 0) {
        const AttnShape& sh = at.shape;
        std::vector<int64_t> key = {(int64_t)r.mask, (int64_t)sh.bh, (int64_t)sh.heads, (int64_t)sh.tq, (int64_t)sh.tk};
        key.insert(key.end(), sh.mask_strides, sh.mask_strides + 4);
        auto it = mask_tables.find(key);
        if (it == mask_tables.end()) {
          it = mask_tables.emplace(key, a.new_slot(DType::F32, attn_mask_words(r, g), true)).first;
          at.build_mask_bits = true;  // items run in plan order: this is the first reader
        }
        at.mask_bits_slot = (int64_t)it->second;
      }
      for (uint32_t o : bwd ? r.bwd_out : r.fwd_out) {
        value_slot[o] = a.alloc(g.nodes[o].dtype, g.nodes[o].n(), exact[o]);
        p.naive_bytes += g.nodes[o].n() * dsize(g.nodes[o].dtype);
      }
      if (bwd)
        for (const AttnOperand* o : {&r.out_dq, &r.out_dk, &r.out_dv}) at.out.push_back(view(*o));
      else
        at.out.push_back(view(r.out_o));
      at.node = bwd ? r.dq : r.o;
      const auto share = attn_executed_share(r, g);
      at.executed = bwd ? share.second : share.first;
      p.steps.push_back(std::move(st));
      for (uint32_t x : ins)
        if (--uses[x] == 0) a.release(value_slot[x]);
      continue;
    }
    if (item.group) {
      const auto& members = item.members;
      // Absorbed broadcasts become aliases of their source on first use (as plan.rs:565-575).
      for (size_t m : members)
        for (uint32_t x : g.nodes[m].inputs)
          if (abs[x] && value_slot[x] == SIZE_MAX) {
            size_t src = g.nodes[x].inputs[0];
            size_t s = value_slot[src];
            a.refs[s]++;
            value_slot[x] = s;
            uses[src]--;
            if (uses[src] == 0) a.release(s);
          }
      std::vector<uint32_t> external;
      for (size_t m : members) {
        p.naive_bytes += g.nodes[m].n() * dsize(g.nodes[m].dtype);
        for (uint32_t x : g.nodes[m].inputs) {
          if (std::binary_search(members.begin(), members.end(), (size_t)x)) continue;
          uses[x]--;
          if (std::find(external.begin(), external.end(), x) == external.end()) external.push_back(x);
        }
      }
      // Output buffers are assigned before the step's inputs are released, so an output never lands on an input's buffer.
      std::vector<std::pair<size_t, size_t>> out_slots;
      for (size_t m : members) {
        if (uses[m] > 0) {
          size_t s = a.alloc(g.nodes[m].dtype, g.nodes[m].n(), exact[m]);
          value_slot[m] = s;
          out_slots.push_back({m, s});
        }
      }
      Step st;
      st.fused = true;
      st.group = compile_group(g, members, value_slot, out_slots, abs, item.rows);
      p.steps.push_back(std::move(st));
      for (uint32_t x : external)
        if (uses[x] == 0) a.release(value_slot[x]);
      continue;
    }
    size_t i = item.node;
    const Node& node = g.nodes[i];
    if (node.op.kind == RG_OP_OUTPUT) continue;
    if (is_alias(g, i)) {
      size_t x = node.inputs[0];
      size_t s = value_slot[x];
      a.refs[s]++;
      value_slot[i] = s;
      uses[x]--;
      if (uses[x] == 0) a.release(s);
      continue;
    }
    Instr in;
    for (uint32_t x : node.inputs) {
      in.arg_shapes.push_back(g.shape(x));
      in.args.push_back(value_slot[x]);
    }
    if (node.op.is_control_flow()) {
      // Results get slots before the inputs are released, so none lands on an input's buffer
      // (plan.rs:611-620); the bodies are planned like the program itself.
      for (uint32_t x : node.inputs) uses[x]--;
      for (size_t o = i + 1; o < total; o++) {
        const Node& on = g.nodes[o];
        if (keep[o] && on.op.kind == RG_OP_OUTPUT && on.inputs[0] == i) {
          const size_t sl = a.alloc(on.dtype, on.n(), exact[o]);
          value_slot[o] = sl;
          in.outs.push_back({on.op.a, sl});
          p.naive_bytes += on.n() * dsize(on.dtype);
        }
      }
      std::vector<uint32_t> dying;
      for (uint32_t x : node.inputs)
        if (uses[x] == 0 && std::find(dying.begin(), dying.end(), x) == dying.end()) dying.push_back(x);
      for (uint32_t x : dying) a.release(value_slot[x]);
      for (const Body* b : {node.op.body2.get(), node.op.body.get()}) {
        if (!b) continue;
        if (!fuse) {
          in.bodies.push_back(std::make_shared<const Plan>(build_with(b->graph, b->outputs, reuse, nullptr)));
        } else {
          Optimized ob = optimize_mode(b->graph, b->outputs, fuse->device, OptMode::Standard);
          in.bodies.push_back(std::make_shared<const Plan>(build_fused(ob.g, ob.outputs, *fuse)));
        }
      }
      if (node.op.kind == RG_OP_COND) std::reverse(in.bodies.begin(), in.bodies.end());  // then, else
      in.op = node.op;
      in.node = (uint32_t)i;
      in.dtype = node.dtype;
      in.dst = SIZE_MAX;
      in.shape = node.shape;
      in.n = 0;
      Step st;
      st.instr = std::move(in);
      p.steps.push_back(std::move(st));
      continue;
    }
    in.mode = binary_mode(node.op, node.shape, in.arg_shapes);
    for (uint32_t x : node.inputs) uses[x]--;
    std::vector<uint32_t> dying;
    for (uint32_t x : node.inputs)
      if (uses[x] == 0) dying.push_back(x);
    std::sort(dying.begin(), dying.end());
    dying.erase(std::unique(dying.begin(), dying.end()), dying.end());
    // An elementwise op may write over an argument of its own shape whose last reader it is.
    bool elementwise = node.op.is_unary_elementwise() || node.op.is_binary_elementwise();
    auto inplace = [&](uint32_t x) {
      return elementwise && in.mode != RG_MODE_GENERAL && g.shape(x) == node.shape && g.dtype(x) == node.dtype;
    };
    for (uint32_t x : dying)
      if (inplace(x)) a.release(value_slot[x]);
    size_t dst = a.alloc(node.dtype, node.n(), exact[i]);
    for (uint32_t x : dying)
      if (!inplace(x)) a.release(value_slot[x]);
    value_slot[i] = dst;
    p.naive_bytes += node.n() * dsize(node.dtype);
    in.op = node.op;
    in.node = (uint32_t)i;
    in.dtype = node.dtype;
    in.dst = dst;
    in.shape = node.shape;
    in.n = node.n();
    Step st;
    st.instr = std::move(in);
    p.steps.push_back(std::move(st));
  }
  for (uint32_t o : outputs) p.outputs.push_back({value_slot[o], g.shape(o), g.nodes[o].n()});
  p.reference = !reuse;
  p.slots = std::move(a.slots);
  p.pinned = std::move(a.pinned);
  p.peak_live_bytes = a.peak;
  return p;
}

}  // namespace

size_t Plan::planned_bytes() const {
  size_t b = 0;
  for (size_t s = 0; s < slots.size(); s++)
    if (!pinned[s]) b += dsize(slots[s].first) * slots[s].second;
  return b;
}

double Plan::gpu_cost_estimate(const Fuse& f) const {
  double c = 0;
  for (auto& s : steps) {
    double n = s.attn ? (double)(s.att.shape.bh * s.att.shape.tq * s.att.shape.hd * s.att.out.size())
                      : (double)(s.fused ? s.group.n * s.group.outputs.size() : s.instr.n);
    c += f.per_dispatch_ns + f.per_element_ns * n;
  }
  return c;
}

size_t Plan::n_fused() const {
  size_t k = 0;
  for (auto& s : steps) k += s.fused;
  return k;
}

size_t Plan::n_fused_ops() const {
  size_t k = 0;
  for (auto& s : steps)
    if (s.fused) k += s.group.ops.size();
  return k;
}

StepWork step_work(const Step& s, const StreamedFn& streamed) {
  StepWork w;
  if (s.attn) {
    const AttnShape& a = s.att.shape;
    const double ds = (double)dsize(s.att.dtype);
    // The products the step replaces: q k^T and P v forward; dO v^T, P^T dO, dS k and dS^T q backward.
    w.flops = (s.att.backward ? 4.0 : 2.0) * 2.0 * (double)a.bh * (double)a.tq * (double)a.tk * (double)a.hd;
    // Operands in order q, k, v (, O, dO) and O (or dq, dk, dv): key-length ones are k, v, dk, dv.
    auto rows = [&](size_t j, bool out) {
      const bool key = out ? (s.att.backward && j >= 1) : (j == 1 || j == 2);
      return (double)(key ? a.tk : a.tq);
    };
    for (size_t j = 0; j < s.att.in.size(); j++) w.bytes += rows(j, false) * (double)(a.bh * a.hd) * ds;
    for (size_t j = 0; j < s.att.out.size(); j++) w.bytes += rows(j, true) * (double)(a.bh * a.hd) * ds;
    w.executed_flops = w.flops * s.att.executed;
    w.compute = true;
    return w;
  }
  if (s.fused) {
    const Fused& f = s.group;
    const double ds = (double)dsize(f.dtype);
    std::vector<size_t> seen;
    for (size_t j = 0; j < f.inputs.size(); j++) {
      if (std::find(seen.begin(), seen.end(), f.inputs[j].slot) != seen.end()) continue;
      seen.push_back(f.inputs[j].slot);
      w.bytes += (double)numel(f.input_shapes[j]) * ds;
    }
    if (f.row_len == 0) {
      w.bytes += (double)(f.n * f.outputs.size()) * ds;
      return w;
    }
    // A row group: a register holds one value per row when it is read per row (a splat, or a
    // broadcast of a [rows..., 1] value), is a last-axis reduction, or is computed from such
    // registers alone; a reduction over the rows holds one value per column.
    const size_t L = f.row_len, rows = f.n / std::max<size_t>(L, 1), last = f.shape.size() - 1;
    std::vector<int> level(f.regs, 0);  // 0 full, 1 per row, 2 per column
    for (size_t j = 0; j < f.inputs.size(); j++) {
      const FusedIn& in = f.inputs[j];
      if (in.reg == SIZE_MAX) continue;
      const Shape& xs = f.input_shapes[j];
      level[in.reg] = in.kind == RG_ARG_SPLAT || (in.kind == RG_ARG_BROADCAST && (xs.empty() || xs.back() == 1)) ? 1 : 0;
    }
    for (auto& m : f.ops) {
      if (m.op.kind == RG_OP_REDUCE) {
        const bool over_last = std::find(m.op.v.begin(), m.op.v.end(), (int64_t)last) != m.op.v.end();
        level[m.reg] = over_last ? 1 : 2;
        continue;
      }
      bool per_row = true;
      for (auto& a : m.args) per_row = per_row && a.first && level[a.second] == 1;
      level[m.reg] = per_row ? 1 : 0;
    }
    for (auto& o : f.outputs) w.bytes += (double)(level[o.first] == 1 ? rows : level[o.first] == 2 ? L : f.n) * ds;
    return w;
  }
  const Instr& i = s.instr;
  const double ds = (double)dsize(i.dtype);
  double in_elems = 0;
  for (auto& a : i.arg_shapes) in_elems += (double)numel(a);
  switch (i.op.kind) {
    case RG_OP_MATMUL:
    case RG_OP_MATMUL_T: {
      // Dimensions as the backend lowers the product: a 2-D right operand with an untransposed
      // left one folds the left operand's batch dimensions into its rows.
      const bool ta = i.op.kind == RG_OP_MATMUL_T && i.op.ta, tb = i.op.kind == RG_OP_MATMUL_T && i.op.tb;
      const Shape &sa = i.arg_shapes[0], &sb = i.arg_shapes[1];
      const size_t ar = sa.size(), br = sb.size();
      uint64_t m = ar >= 2 ? (ta ? sa[ar - 1] : sa[ar - 2]) : 1;
      const uint64_t k = ar >= 2 ? (ta ? sa[ar - 2] : sa[ar - 1]) : (ar ? sa[0] : 1);
      const uint64_t n = br >= 2 ? (tb ? sb[br - 2] : sb[br - 1]) : 1;
      uint64_t batch = 1;
      Shape ba(sa.begin(), sa.begin() + (ar >= 2 ? ar - 2 : 0)), bb(sb.begin(), sb.begin() + (br >= 2 ? br - 2 : 0));
      if (bb.empty() && !ta) {
        m *= numel(ba);
      } else {
        const size_t r = std::max(ba.size(), bb.size());
        for (size_t q = 0; q < r; q++) {
          const size_t x = q < r - ba.size() ? 1 : ba[q - (r - ba.size())];
          const size_t y = q < r - bb.size() ? 1 : bb[q - (r - bb.size())];
          batch *= std::max(x, y);
        }
      }
      w.flops = 2.0 * (double)m * (double)n * (double)k * (double)batch;
      w.executed_flops = w.flops;
      w.bytes = (in_elems + (double)i.n) * ds;
      w.compute = i.dtype != DType::I32 && !(streamed && streamed(i.dtype, m, n, k, batch, ta, tb));
      return w;
    }
    case RG_OP_TAKE:
    case RG_OP_TAKE_ALONG:
      // The indices, and each gathered element read once and written once.
      w.bytes = (double)numel(i.arg_shapes[1]) * 4.0 + 2.0 * (double)i.n * ds;
      return w;
    case RG_OP_TAKE_GRAD:
    case RG_OP_TAKE_ALONG_GRAD:
      // The cotangent read, the indices, and the result written.
      w.bytes = ((double)numel(i.arg_shapes[0]) + (double)i.n) * ds + (double)numel(i.arg_shapes[1]) * 4.0;
      return w;
    default:
      w.bytes = (in_elems + (double)i.n) * ds;
      return w;
  }
}

Plan build_plan(const Graph& g, const std::vector<uint32_t>& outputs, bool reuse) {
  return build_with(g, outputs, reuse, nullptr);
}

namespace {

std::vector<size_t> step_reads(const Step& st) {
  std::vector<size_t> r;
  if (st.attn) {
    for (auto& v : st.att.in) r.push_back(v.slot);  // outputs are written whole (dq, dk, dv tile theirs)
    if (st.att.mask_slot >= 0) r.push_back((size_t)st.att.mask_slot);
    if (st.att.mask_bits_slot >= 0) r.push_back((size_t)st.att.mask_bits_slot);
    r.push_back(st.att.stats_slot);
  } else if (st.fused) {
    for (auto& in : st.group.inputs) r.push_back(in.slot);
  } else {
    r = st.instr.args;
  }
  return r;
}

std::vector<size_t> step_writes(const Step& st) {
  std::vector<size_t> w;
  if (st.attn) {
    for (auto& v : st.att.out) w.push_back(v.slot);
    w.push_back(st.att.stats_slot);
    if (st.att.mask_bits_slot >= 0) w.push_back((size_t)st.att.mask_bits_slot);
  } else if (st.fused) {
    for (auto& o : st.group.outputs) w.push_back(o.second);
  } else {
    w.push_back(st.instr.dst);
  }
  return w;
}

// Bias adds folded into products (device plans): a fused group whose only work is adding a
// per-column vector to the rows of the product just before it, the product's only reader, goes
// away; the vector becomes the product's third operand (include/rg_plan.h) and the product writes
// the group's output slot. The sum is the same fp32 addition of the finished product and the bias.
void fold_bias_into_products(Plan& p) {
  std::set<size_t> out_slots;
  for (auto& o : p.outputs) out_slots.insert(o.slot);
  for (size_t k = 0; k + 1 < p.steps.size(); k++) {
    Step& M = p.steps[k];
    const Step& F = p.steps[k + 1];
    if (M.fused || M.attn || F.attn || !F.fused || F.group.row_len != 0) continue;
    const Instr& mi = M.instr;
    if ((mi.op.kind != RG_OP_MATMUL && mi.op.kind != RG_OP_MATMUL_T) || mi.dtype != DType::F32 || mi.args.size() != 2 ||
        mi.shape.empty() || mi.n == 0)
      continue;
    const Fused& f = F.group;
    const size_t n = (size_t)mi.shape.back();
    if (f.dtype != DType::F32 || f.n != mi.n || f.ops.size() != 1 || f.ops[0].op.kind != RG_OP_ADD || f.inputs.size() != 2 ||
        f.outputs.size() != 1 || f.outputs[0].first != f.ops[0].reg)
      continue;
    int full = -1, row = -1;
    for (int j = 0; j < 2; j++) {
      const FusedIn& in = f.inputs[(size_t)j];
      if (in.kind == RG_ARG_FULL && in.slot == mi.dst) full = j;
      else if (in.kind == RG_ARG_ROW && in.row_len == n) row = j;
    }
    if (full < 0 || row < 0) continue;
    const size_t bias = f.inputs[(size_t)row].slot, out = f.outputs[0].second;
    // The group's output must not be an operand of the product, and the product's value must
    // have no other reader before its slot is written again.
    if (out == mi.args[0] || out == mi.args[1] || out == bias || bias == mi.dst || out_slots.count(mi.dst)) continue;
    bool sole = true;
    for (size_t j = k + 2; j < p.steps.size() && sole; j++) {
      auto r = step_reads(p.steps[j]);
      if (std::find(r.begin(), r.end(), mi.dst) != r.end()) sole = false;
      auto w = step_writes(p.steps[j]);
      if (std::find(w.begin(), w.end(), mi.dst) != w.end()) break;
    }
    if (!sole) continue;
    M.instr.args.push_back(bias);
    M.instr.arg_shapes.push_back(f.input_shapes[(size_t)row]);
    M.instr.dst = out;
    p.steps.erase(p.steps.begin() + (std::ptrdiff_t)(k + 1));
  }
}

}  // namespace

Plan build_fused(const Graph& g, const std::vector<uint32_t>& outputs, const Fuse& cfg) {
  Plan plan = build_with(g, outputs, true, &cfg);
  if (cfg.device && cfg.levels) {
    // Level order cuts dispatch dependencies but keeps values alive longer; keep the cheaper.
    Fuse greedy_cfg = cfg;
    greedy_cfg.levels = false;
    Plan greedy = build_with(g, outputs, true, &greedy_cfg);
    if (plan.peak_live_bytes > cfg.level_max_peak || greedy.gpu_cost_estimate(cfg) < plan.gpu_cost_estimate(cfg))
      plan = std::move(greedy);
  }
  if (cfg.device) fold_bias_into_products(plan);
  return plan;
}

static void put_op_attr(std::vector<int64_t>& a, const Op& op) {
  auto vec = [&](const Shape& s) {
    for (auto x : s) a.push_back((int64_t)x);
  };
  switch (op.kind) {
    case RG_OP_MATMUL_T: a.push_back(op.ta); a.push_back(op.tb); break;
    case RG_OP_REDUCE:
      a.push_back((int64_t)op.rk);
      a.push_back(op.keepdims);
      a.push_back((int64_t)op.v.size());
      vec(op.v);
      break;
    case RG_OP_TRANSPOSE: case RG_OP_BROADCAST_TO: case RG_OP_RESHAPE: case RG_OP_TAKE_ALONG_GRAD: vec(op.v); break;
    case RG_OP_SLICE: case RG_OP_PAD:
      a.push_back((int64_t)op.v.size());
      vec(op.v);
      vec(op.w);
      break;
    case RG_OP_CAST: a.push_back((int64_t)op.dt); break;
    case RG_OP_TAKE: case RG_OP_CONCAT: case RG_OP_KEY_SPLIT: case RG_OP_ARG_TOP_K: a.push_back((int64_t)op.a); break;
    case RG_OP_TAKE_GRAD: a.push_back((int64_t)op.a); vec(op.v); break;
    case RG_OP_RAND_UNIFORM: case RG_OP_RAND_NORMAL: a.push_back((int64_t)op.dt); vec(op.v); break;
    case RG_OP_CUMSUM: a.push_back(op.reverse); break;
    default: break;
  }
}

static void write_plan(const Plan& plan, std::vector<int64_t>* words, std::vector<uint8_t>* blob);

// Control flow: counts, the result slots, then each body's plan as a nested descriptor whose
// constants share the blob.
static void put_control_attr(std::vector<int64_t>& a, const Instr& in, std::vector<uint8_t>* blob) {
  const Op& op = in.op;
  if (op.kind == RG_OP_SCAN) {
    a.push_back((int64_t)op.n_carry);
    a.push_back((int64_t)op.n_x);
    a.push_back((int64_t)op.length);
    a.push_back(op.reverse ? 1 : 0);
  } else if (op.kind == RG_OP_WHILE) {
    a.push_back((int64_t)op.n_carry);
    a.push_back((int64_t)op.max_iter);
  }
  a.push_back((int64_t)in.outs.size());
  for (auto& [index, slot] : in.outs) {
    a.push_back((int64_t)index);
    a.push_back((int64_t)slot);
  }
  a.push_back((int64_t)in.bodies.size());
  for (auto& b : in.bodies) {
    std::vector<int64_t> sub;
    write_plan(*b, &sub, blob);
    a.push_back((int64_t)sub.size());
    a.insert(a.end(), sub.begin(), sub.end());
  }
}

void Plan::serialize(std::vector<int64_t>* words, std::vector<uint8_t>* blob) const {
  words->clear();
  blob->clear();
  write_plan(*this, words, blob);
}

static void write_plan(const Plan& plan, std::vector<int64_t>* words, std::vector<uint8_t>* blob) {
  const auto& slots = plan.slots;
  const auto& pinned = plan.pinned;
  const auto& consts = plan.consts;
  const auto& input_slots = plan.input_slots;
  const auto& input_ns = plan.input_ns;
  const auto& outputs = plan.outputs;
  const auto& steps = plan.steps;
  auto& w = *words;
  auto shape = [&](const Shape& s) {
    w.push_back((int64_t)s.size());
    for (auto d : s) w.push_back((int64_t)d);
  };
  w.push_back(RG_PLAN_MAGIC);
  w.push_back(RG_PLAN_VERSION);
  w.push_back((int64_t)slots.size());
  for (size_t s = 0; s < slots.size(); s++) {
    w.push_back((int64_t)slots[s].first);
    w.push_back((int64_t)slots[s].second);
    w.push_back(pinned[s] ? 1 : 0);
  }
  w.push_back((int64_t)consts.size());
  for (auto& [slot, t] : consts) {
    // 16-byte alignment keeps every constant readable as a vector.
    while (blob->size() % 16) blob->push_back(0);
    w.push_back((int64_t)slot);
    w.push_back((int64_t)t->n());
    w.push_back((int64_t)blob->size());
    blob->insert(blob->end(), t->data.begin(), t->data.end());
  }
  w.push_back((int64_t)input_slots.size());
  for (size_t k = 0; k < input_slots.size(); k++) {
    w.push_back((int64_t)input_slots[k]);
    w.push_back((int64_t)input_ns[k]);
  }
  w.push_back((int64_t)outputs.size());
  for (auto& o : outputs) {
    w.push_back((int64_t)o.slot);
    w.push_back((int64_t)o.n);
    shape(o.shape);
  }
  w.push_back((int64_t)steps.size());
  for (auto& st : steps) {
    if (st.attn) {
      const Attn& at = st.att;
      w.push_back(RG_STEP_ATTN);
      w.push_back((int64_t)at.dtype);
      w.push_back(at.backward ? 1 : 0);
      w.push_back((int64_t)at.shape.bh);
      w.push_back((int64_t)at.shape.heads);
      w.push_back((int64_t)at.shape.tq);
      w.push_back((int64_t)at.shape.tk);
      w.push_back((int64_t)at.shape.hd);
      int64_t bits;
      memcpy(&bits, &at.div, 8);
      w.push_back(bits);
      memcpy(&bits, &at.fill, 8);
      w.push_back(bits);
      w.push_back(at.mask_slot);
      for (int k = 0; k < 4; k++) w.push_back(at.shape.mask_strides[k]);
      w.push_back(at.mask_bits_slot);
      w.push_back(at.build_mask_bits ? 1 : 0);
      w.push_back((int64_t)at.stats_slot);
      auto views = [&](const std::vector<AttnView>& vs) {
        w.push_back((int64_t)vs.size());
        for (const AttnView& v : vs) {
          w.push_back((int64_t)v.slot);
          w.push_back(v.offset);
          w.push_back(v.sb);
          w.push_back(v.sh);
          w.push_back(v.st);
        }
      };
      views(at.in);
      views(at.out);
      w.push_back(at.node);
      continue;
    }
    if (!st.fused) {
      const Instr& in = st.instr;
      w.push_back(RG_STEP_INSTR);
      w.push_back(in.op.kind);
      w.push_back((int64_t)in.dtype);
      w.push_back((int64_t)in.dst);
      w.push_back((int64_t)in.n);
      w.push_back(in.mode);
      w.push_back(in.node);
      shape(in.shape);
      w.push_back((int64_t)in.args.size());
      for (size_t k = 0; k < in.args.size(); k++) {
        w.push_back((int64_t)in.args[k]);
        shape(in.arg_shapes[k]);
      }
      std::vector<int64_t> attr;
      if (in.op.is_control_flow()) put_control_attr(attr, in, blob);
      else put_op_attr(attr, in.op);
      w.push_back((int64_t)attr.size());
      w.insert(w.end(), attr.begin(), attr.end());
    } else {
      const Fused& f = st.group;
      const bool rows = f.row_len > 0;
      w.push_back(rows ? RG_STEP_ROWS : RG_STEP_FUSED);
      w.push_back((int64_t)f.dtype);
      w.push_back((int64_t)f.n);
      if (rows) w.push_back((int64_t)f.row_len);
      w.push_back((int64_t)f.regs);
      shape(f.shape);
      w.push_back((int64_t)f.inputs.size());
      for (size_t k = 0; k < f.inputs.size(); k++) {
        w.push_back((int64_t)f.inputs[k].slot);
        w.push_back(f.inputs[k].kind);
        w.push_back((int64_t)f.inputs[k].row_len);
        w.push_back(f.inputs[k].reg == SIZE_MAX ? -1 : (int64_t)f.inputs[k].reg);
        shape(f.input_shapes[k]);
      }
      w.push_back((int64_t)f.ops.size());
      for (auto& m : f.ops) {
        w.push_back(m.op.kind);
        w.push_back((int64_t)m.reg);
        if (rows) {
          // A reduction over the leading axes (a column reduction) is flagged with RG_ROWS_COLUMN.
          const bool col = m.op.kind == RG_OP_REDUCE &&
                           std::find(m.op.v.begin(), m.op.v.end(), (int64_t)f.shape.size() - 1) == m.op.v.end();
          w.push_back(m.op.kind == RG_OP_REDUCE ? (int64_t)m.op.rk + (col ? RG_ROWS_COLUMN : 0) : 0);
        }
        w.push_back((int64_t)m.args.size());
        for (auto& [is_reg, idx] : m.args) {
          w.push_back(is_reg ? 1 : 0);
          w.push_back((int64_t)idx);
        }
      }
      w.push_back((int64_t)f.outputs.size());
      for (auto& [r, s] : f.outputs) {
        w.push_back((int64_t)r);
        w.push_back((int64_t)s);
      }
    }
  }
}

}  // namespace rg
