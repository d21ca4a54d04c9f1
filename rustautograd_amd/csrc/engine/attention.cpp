// Attention regions for device plans: the subgraph of scaled, masked softmax attention and the
// reverse-mode subgraph the autodiff derives from it, each becoming one fused step
// (include/rg_plan.h RG_STEP_ATTN). No reference counterpart: rg plans these nodes one by one
// (src/plan.rs:311-414); the device planner keeps that plan for anything that does not match.
//
// Forward, as nn.MultiHeadAttention traces it (python/rg/nn.py:170-200 in the reference):
//
//   S = q k^T                       matmul_t(q, k; tb)       or matmul(q, transpose(k))
//   X = S / c                       div by a scalar constant (optional)
//   Y = where(mask, X, fill)        mask and fill broadcast to S's shape (optional)
//   m = max(Y, -1, keepdims)
//   E = exp(Y - m)
//   Z = sum(E, -1, keepdims)
//   P = E / Z
//   O = P v
//
// Backward, as the autodiff emits it for a cotangent dO of O (src/autodiff.rs rules for
// matmul, div, exp, sub, where):
//
//   dP = dO v^T;  dv = (E / Z)^T dO
//   dE = dP / Z + sum(-dP * E / (Z * Z), -1, keepdims);  dY = dE * E
//   dS = where(mask, dY, 0) / c;  dq = dS k;  dk = (q^T dS)^T  (or dS^T q)
//
// A region is claimed only when every intermediate is read by region nodes alone, so the fused
// steps replace the nodes exactly; O and dq, dk, dv stay ordinary values.
#include <algorithm>
#include <set>

#include "plan.h"

namespace rg {

namespace {

struct Matcher {
  const Graph& g;
  const std::vector<bool>& keep;
  std::vector<std::vector<uint32_t>> users;
  std::vector<bool> is_out;

  Matcher(const Graph& graph, const std::vector<bool>& k, const std::vector<uint32_t>& outputs) : g(graph), keep(k) {
    users.resize(g.nodes.size());
    is_out.assign(g.nodes.size(), false);
    for (size_t i = 0; i < g.nodes.size(); i++)
      if (keep[i])
        for (uint32_t x : g.nodes[i].inputs) users[x].push_back((uint32_t)i);
    for (uint32_t o : outputs) is_out[o] = true;
  }

  const Node& node(uint32_t i) const { return g.nodes[i]; }
  bool is(uint32_t i, rg_op k) const { return node(i).op.kind == k; }
  bool is_leaf(uint32_t i) const { return is(i, RG_OP_INPUT) || is(i, RG_OP_CONST); }

  bool scalar_const(uint32_t i, double* v) const {
    const Node& n = node(i);
    if (n.op.kind != RG_OP_CONST || n.n() != 1 || !n.op.t) return false;
    *v = n.op.t->at(0);
    return true;
  }
  // A scalar constant, one broadcast to `shape`, or a constant of `shape` with one value
  // throughout (a folded broadcast).
  bool scalar_or_bcast(uint32_t i, const Shape& shape, double* v) const {
    if (is(i, RG_OP_BROADCAST_TO) && node(i).shape == shape) return scalar_const(node(i).inputs[0], v);
    if (scalar_const(i, v)) return true;
    const Node& n = node(i);
    if (n.op.kind != RG_OP_CONST || !n.op.t || n.shape != shape || n.n() == 0) return false;
    const Tensor& t = *n.op.t;
    const double x = t.at(0);
    for (size_t j = 1; j < t.n(); j++)
      if (!(t.at(j) == x)) return false;
    *v = x;
    return true;
  }
  bool last_axis_reduce(uint32_t i, RK kind) const {
    const Node& n = node(i);
    if (n.op.kind != RG_OP_REDUCE || n.op.rk != kind || !n.op.keepdims || n.op.v.size() != 1) return false;
    return n.op.v[0] + 1 == g.shape(n.inputs[0]).size();
  }
  bool swap_last2(uint32_t i) const {
    const Node& n = node(i);
    if (n.op.kind != RG_OP_TRANSPOSE) return false;
    size_t r = n.op.v.size();
    if (r < 2) return false;
    for (size_t d = 0; d + 2 < r; d++)
      if (n.op.v[d] != d) return false;
    return n.op.v[r - 2] == r - 1 && n.op.v[r - 1] == r - 2;
  }
  bool matmul_t(uint32_t i, bool ta, bool tb) const {
    const Node& n = node(i);
    return n.op.kind == RG_OP_MATMUL_T && n.op.ta == ta && n.op.tb == tb;
  }
  // users(i) == want (as sets)
  bool users_are(uint32_t i, std::vector<uint32_t> want) const {
    std::vector<uint32_t> u = users[i];
    std::sort(u.begin(), u.end());
    u.erase(std::unique(u.begin(), u.end()), u.end());
    std::sort(want.begin(), want.end());
    want.erase(std::unique(want.begin(), want.end()), want.end());
    return u == want;
  }
  bool only_user(uint32_t i, uint32_t* out) const {
    std::set<uint32_t> u(users[i].begin(), users[i].end());
    if (u.size() != 1) return false;
    *out = *u.begin();
    return true;
  }
  // A binary node `kind` with inputs {a, x} in either order; returns x.
  bool commuted(uint32_t i, rg_op kind, uint32_t a, uint32_t* x) const {
    const Node& n = node(i);
    if (n.op.kind != kind || n.inputs.size() != 2) return false;
    if (n.inputs[0] == a) *x = n.inputs[1];
    else if (n.inputs[1] == a) *x = n.inputs[0];
    else return false;
    return true;
  }

  bool match_forward(uint32_t m, AttnRegion* r) const;
  bool match_backward(AttnRegion* r) const;
  bool closed(AttnRegion& r) const;
};

bool Matcher::match_forward(uint32_t m, AttnRegion* r) const {
  if (!last_axis_reduce(m, RK::Max)) return false;
  const uint32_t y = node(m).inputs[0];
  const Shape& ss = g.shape(y);
  if (ss.size() < 3 || node(y).dtype != DType::F32) return false;
  // m feeds D = Y - m only; D feeds E = exp(D) only.
  uint32_t d, e;
  if (!only_user(m, &d) || !is(d, RG_OP_SUB) || node(d).inputs[0] != y || node(d).inputs[1] != m) return false;
  if (!users_are(y, {m, d})) return false;
  if (!only_user(d, &e) || !is(e, RG_OP_EXP)) return false;
  // Z = sum(E) and P = E / Z among E's users.
  int64_t z = -1, p = -1;
  for (uint32_t u : users[e])
    if (last_axis_reduce(u, RK::Sum)) z = u;
  if (z < 0) return false;
  // O = P v (the backward may hold a second E / Z of its own).
  int64_t o = -1;
  for (uint32_t u : users[e]) {
    if (!is(u, RG_OP_DIV) || node(u).inputs[0] != e || node(u).inputs[1] != (uint32_t)z) continue;
    for (uint32_t w : users[u])
      if (is(w, RG_OP_MATMUL) && node(w).inputs[0] == u) {
        p = u;
        o = w;
      }
  }
  if (o < 0) return false;
  // Y = where(mask, X, fill) or X; X = S / c or S; S = q k^T.
  uint32_t x = y;
  r->fwd = {m, d, e, (uint32_t)z, (uint32_t)p, (uint32_t)o};
  r->mask = -1;
  if (is(y, RG_OP_WHERE)) {
    const uint32_t cond = node(y).inputs[0];
    x = node(y).inputs[1];
    const uint32_t fill = node(y).inputs[2];
    if (fill == x || cond == x || !scalar_or_bcast(fill, ss, &r->fill)) return false;
    if (!is_leaf(fill)) r->optional.push_back(fill);
    uint32_t src = cond;
    if (is(cond, RG_OP_BROADCAST_TO)) {
      src = node(cond).inputs[0];
      r->mask_bcast = cond;
      r->optional.push_back(cond);
    } else if (g.shape(cond) != ss) {
      return false;
    }
    while (is(src, RG_OP_BROADCAST_TO)) src = node(src).inputs[0];
    if (node(src).dtype != DType::F32) return false;
    r->mask = src;
    r->fwd.push_back(y);
    if (!users_are(x, {y})) return false;
  }
  uint32_t s = x;
  r->div = 1.0;
  r->scaled = false;
  if (is(x, RG_OP_DIV)) {
    if (!scalar_const(node(x).inputs[1], &r->div)) return false;
    s = node(x).inputs[0];
    r->scaled = true;
    r->fwd.push_back(x);
    if (!users_are(s, {x})) return false;
  }
  uint32_t q, k;
  if (matmul_t(s, false, true)) {
    q = node(s).inputs[0];
    k = node(s).inputs[1];
  } else if (is(s, RG_OP_MATMUL) && swap_last2(node(s).inputs[1])) {
    q = node(s).inputs[0];
    k = node(node(s).inputs[1]).inputs[0];
    r->optional.push_back(node(s).inputs[1]);
  } else {
    return false;
  }
  r->fwd.push_back(s);
  const uint32_t v = node((uint32_t)o).inputs[1];
  const Shape &qs = g.shape(q), &ks = g.shape(k), &vs = g.shape(v);
  const size_t rank = ss.size();
  if (qs.size() != rank || ks.size() != rank || vs.size() != rank) return false;
  for (size_t dd = 0; dd + 2 < rank; dd++)
    if (qs[dd] != ss[dd] || ks[dd] != ss[dd] || vs[dd] != ss[dd]) return false;
  if (ks[rank - 1] != qs[rank - 1] || vs[rank - 1] != qs[rank - 1] || vs[rank - 2] != ks[rank - 2]) return false;
  if (node(q).dtype != DType::F32 || node(k).dtype != DType::F32 || node(v).dtype != DType::F32) return false;
  // The steps read the operands' own buffers: broadcasts (possibly not materialized) are refused.
  if (is(q, RG_OP_BROADCAST_TO) || is(k, RG_OP_BROADCAST_TO) || is(v, RG_OP_BROADCAST_TO)) return false;
  r->q = q;
  r->k = k;
  r->v = v;
  r->o = (uint32_t)o;
  r->s = s;
  r->e = e;
  r->z = (uint32_t)z;
  r->p = (uint32_t)p;
  r->y = y;
  return true;
}

bool Matcher::match_backward(AttnRegion* r) const {
  const Shape& ss = g.shape(r->s);
  // dP = dO v^T.
  int64_t dp = -1;
  for (uint32_t u : users[r->v])
    if (matmul_t(u, false, true) && node(u).inputs[1] == r->v && g.shape(u) == ss) dp = u;
  if (dp < 0) return false;
  const uint32_t d_o = node((uint32_t)dp).inputs[0];
  // dv = P^T dO with P or a recomputed E / Z.
  int64_t dv = -1, pp = -1;
  for (uint32_t u : users[d_o]) {
    if (!matmul_t(u, true, false) || node(u).inputs[1] != d_o) continue;
    uint32_t a = node(u).inputs[0];
    if (a == r->p || (is(a, RG_OP_DIV) && node(a).inputs[0] == r->e && node(a).inputs[1] == r->z)) {
      dv = u;
      if (a != r->p) pp = a;
    }
  }
  if (dv < 0 || is(d_o, RG_OP_BROADCAST_TO)) return false;
  // dE = dP / Z + sum(-dP * E / (Z * Z)); dY = dE * E.
  uint32_t a = 0, b = 0;
  for (uint32_t u : users[(size_t)dp]) {
    if (is(u, RG_OP_DIV) && node(u).inputs[0] == (uint32_t)dp && node(u).inputs[1] == r->z) a = u;
    if (is(u, RG_OP_NEG)) b = u;
  }
  if (!a || !b || !users_are((uint32_t)dp, {a, b})) return false;
  uint32_t c, x;
  if (!only_user(b, &c) || !commuted(c, RG_OP_MUL, b, &x) || x != r->e) return false;
  uint32_t dd;
  if (!only_user(c, &dd) || !is(dd, RG_OP_DIV) || node(dd).inputs[0] != c) return false;
  const uint32_t zz = node(dd).inputs[1];
  if (!is(zz, RG_OP_MUL) || node(zz).inputs[0] != r->z || node(zz).inputs[1] != r->z || !users_are(zz, {dd})) return false;
  uint32_t sm, f, h;
  if (!only_user(dd, &sm) || !last_axis_reduce(sm, RK::Sum)) return false;
  if (!only_user(sm, &f) || !commuted(f, RG_OP_ADD, sm, &x) || x != a || !users_are(a, {f})) return false;
  if (!only_user(f, &h) || !commuted(h, RG_OP_MUL, f, &x) || x != r->e) return false;
  r->bwd = {(uint32_t)dp, (uint32_t)dv, a, b, c, dd, zz, sm, f, h};
  if (pp >= 0) {
    if (!users_are((uint32_t)pp, {(uint32_t)dv})) return false;
    r->bwd.push_back((uint32_t)pp);
  }
  // dX = where(mask, dY, 0); dS = dX / c; possibly once per reader when the zero operand is a
  // folded constant that common-subexpression elimination does not merge.
  std::vector<uint32_t> dss;
  if (r->mask >= 0) {
    for (uint32_t w : users[h]) {
      if (!is(w, RG_OP_WHERE) || node(w).inputs[1] != h) return false;
      const uint32_t cond = node(w).inputs[0];
      const uint32_t want = r->mask_bcast >= 0 ? (uint32_t)r->mask_bcast : (uint32_t)r->mask;
      double zero = 1.0;
      if (cond != want || !scalar_or_bcast(node(w).inputs[2], ss, &zero) || zero != 0.0) return false;
      if (!is_leaf(node(w).inputs[2])) r->optional.push_back(node(w).inputs[2]);
      r->bwd.push_back(w);
      dss.push_back(w);
    }
  } else {
    dss.push_back(h);
  }
  if (r->scaled) {
    for (uint32_t& w : dss) {
      double c2 = 0;
      uint32_t t;
      if (!only_user(w, &t) || !is(t, RG_OP_DIV) || node(t).inputs[0] != w || !scalar_const(node(t).inputs[1], &c2) || c2 != r->div)
        return false;
      r->bwd.push_back(t);
      w = t;
    }
  }
  auto is_ds = [&](uint32_t x) { return std::find(dss.begin(), dss.end(), x) != dss.end(); };
  // dq = dS k; dk = dS^T q, possibly as the transpose of q^T dS.
  std::set<uint32_t> readers;
  for (uint32_t x : dss) readers.insert(users[x].begin(), users[x].end());
  if (readers.size() != 2) return false;
  int64_t dq = -1, dk = -1;
  for (uint32_t u : readers) {
    const Node& n = node(u);
    if (matmul_t(u, false, true) && is_ds(n.inputs[0]) && swap_last2(n.inputs[1]) && node(n.inputs[1]).inputs[0] == r->k) {
      dq = u;
      r->optional.push_back(n.inputs[1]);
    } else if (is(u, RG_OP_MATMUL) && is_ds(n.inputs[0]) && n.inputs[1] == r->k) {
      dq = u;
    } else if (matmul_t(u, true, false) && n.inputs[0] == r->q && is_ds(n.inputs[1])) {
      uint32_t t;
      if (!only_user(u, &t) || !swap_last2(t)) return false;
      r->bwd.push_back(u);
      dk = t;
    } else if (matmul_t(u, true, false) && is_ds(n.inputs[0]) && n.inputs[1] == r->q) {
      dk = u;
    }
  }
  if (dq < 0 || dk < 0) return false;
  r->bwd.push_back((uint32_t)dq);
  r->bwd.push_back((uint32_t)dk);
  r->d_o = d_o;
  r->dq = (uint32_t)dq;
  r->dk = (uint32_t)dk;
  r->dv = (uint32_t)dv;
  r->has_bwd = true;
  return true;
}

// Claims the optional nodes (broadcasts of the mask and of constants, the transposed k) that
// members alone read; then every member other than the region's outputs must be read by members
// only and must not be a plan output.
bool Matcher::closed(AttnRegion& r) const {
  std::set<uint32_t> mem(r.fwd.begin(), r.fwd.end());
  mem.insert(r.bwd.begin(), r.bwd.end());
  if (mem.size() != r.fwd.size() + r.bwd.size()) return false;  // a node matched twice
  for (bool grew = true; grew;) {
    grew = false;
    for (uint32_t c : r.optional) {
      if (mem.count(c) || is_out[c]) continue;
      bool inner = !users[c].empty();
      for (uint32_t u : users[c]) inner &= mem.count(u) > 0;
      if (!inner) continue;
      mem.insert(c);
      r.fwd.push_back(c);  // read by no kernel: placed with the forward
      grew = true;
    }
  }
  std::set<uint32_t> outs = {r.o};
  if (r.has_bwd) outs.insert({r.dq, r.dk, r.dv});
  for (uint32_t m : mem) {
    if (!keep[m] || is_leaf(m)) return false;
    if (outs.count(m)) continue;
    if (is_out[m]) return false;
    for (uint32_t u : users[m])
      if (!mem.count(u)) return false;
  }
  return true;
}

}  // namespace

size_t attn_stats_words(const AttnRegion& r, const Graph& g) {
  AttnShape a = attn_shape(r, g);
  return 3 * a.bh * a.tq;
}

size_t attn_mask_words(const AttnRegion& r, const Graph& g) {
  if (r.mask < 0) return 0;
  AttnShape a = attn_shape(r, g);
  return a.mask_slices * (2 * a.tq * a.tk / 32 + a.tq);
}

// The device kernels work in 16 x 16 tiles of queries and keys. The forward skips a wave's key
// tile when none of its 16 rows sees a key of it, unless some row sees no key at all; the query
// pass walks the key tiles from the first to the last any of its rows sees, and the key pass the
// query tiles from the first to the last any of its keys is seen by, both only when every query
// row of the problem sees some key. Counted over the mask's distinct slices, as shares of all
// tiles; the backward's two passes each do two of its four products.
namespace {

// The value of a node computed from constants by structural operations only (slices, reshapes,
// broadcasts, transposes, casts), evaluated on the host; false for anything else.
bool host_value(const Graph& g, uint32_t id, std::vector<double>* out, int depth = 0) {
  const Node& n = g.nodes[id];
  const Op& op = n.op;
  if (depth > 16 || n.n() > (size_t)1 << 24) return false;
  if (op.kind == RG_OP_CONST) {
    out->resize(op.t->n());
    for (size_t i = 0; i < op.t->n(); i++) (*out)[i] = op.t->at(i);
    return true;
  }
  const bool structural = op.kind == RG_OP_RESHAPE || op.kind == RG_OP_STOP_GRADIENT || op.kind == RG_OP_CAST ||
                          op.kind == RG_OP_SLICE || op.kind == RG_OP_BROADCAST_TO || op.kind == RG_OP_TRANSPOSE;
  if (!structural || n.inputs.size() != 1) return false;
  std::vector<double> x;
  if (!host_value(g, n.inputs[0], &x, depth + 1)) return false;
  if (op.kind == RG_OP_RESHAPE || op.kind == RG_OP_STOP_GRADIENT || op.kind == RG_OP_CAST) {
    *out = std::move(x);
    return true;
  }
  const Shape& is = g.shape(n.inputs[0]);
  const Shape& os = g.shape(id);
  std::vector<size_t> ist(is.size(), 1);
  for (size_t d = is.size(); d-- > 1;) ist[d - 1] = ist[d] * is[d];
  out->assign(n.n(), 0.0);
  std::vector<size_t> idx(os.size(), 0);
  for (size_t e = 0; e < n.n(); e++) {
    size_t rem = e, src = 0;
    for (size_t d = os.size(); d-- > 0;) {
      idx[d] = rem % os[d];
      rem /= os[d];
    }
    if (op.kind == RG_OP_SLICE) {
      for (size_t d = 0; d < os.size(); d++) src += (idx[d] + (size_t)op.v[d]) * ist[d];
    } else if (op.kind == RG_OP_TRANSPOSE) {
      for (size_t d = 0; d < os.size(); d++) src += idx[d] * ist[(size_t)op.v[d]];
    } else {  // broadcast, right-aligned
      const size_t lead = os.size() - is.size();
      for (size_t d = 0; d < is.size(); d++) src += (is[d] == 1 ? 0 : idx[lead + d]) * ist[d];
    }
    (*out)[e] = x[src];
  }
  return true;
}

}  // namespace

std::pair<double, double> attn_executed_share(const AttnRegion& r, const Graph& g) {
  std::vector<double> mv;
  if (r.mask < 0 || !host_value(g, (uint32_t)r.mask, &mv)) return {1.0, 1.0};
  struct Values {
    const std::vector<double>& v;
    double at(size_t i) const { return v[i]; }
  } m{mv};
  const AttnShape a = attn_shape(r, g);
  const int64_t* st = a.mask_strides;
  const size_t T = 16, nq = (a.tq + T - 1) / T, nk = (a.tk + T - 1) / T;
  const size_t nb = st[0] ? a.bh / a.heads : 1, nh = st[1] ? a.heads : 1;
  double fwd = 0, qpass = 0, kpass = 0;
  for (size_t b = 0; b < nb; b++)
    for (size_t h = 0; h < nh; h++) {
      auto seen = [&](size_t q, size_t k) { return m.at((size_t)(b * st[0] + h * st[1] + q * st[2] + k * st[3])) != 0.0; };
      std::vector<char> row_sees(a.tq, 0);
      for (size_t q = 0; q < a.tq; q++)
        for (size_t k = 0; k < a.tk && !row_sees[q]; k++) row_sees[q] = seen(q, k);
      const bool all_rows = std::all_of(row_sees.begin(), row_sees.end(), [](char c) { return c != 0; });
      for (size_t qt = 0; qt < nq; qt++) {
        const size_t q0 = qt * T, q1 = std::min(a.tq, q0 + T);
        bool wave_rows = true;
        for (size_t q = q0; q < q1; q++) wave_rows = wave_rows && row_sees[q];
        size_t lo = nk, hi = 0, live = 0;
        for (size_t kt = 0; kt < nk; kt++) {
          bool any = false;
          for (size_t q = q0; q < q1 && !any; q++)
            for (size_t k = kt * T; k < std::min(a.tk, kt * T + T) && !any; k++) any = seen(q, k);
          if (any) {
            live++;
            lo = std::min(lo, kt);
            hi = kt + 1;
          }
        }
        fwd += wave_rows ? (double)live : (double)nk;
        qpass += all_rows ? (double)(hi > lo ? hi - lo : 0) : (double)nk;
      }
      for (size_t kt = 0; kt < nk; kt++) {
        size_t lo = nq, hi = 0;
        for (size_t qt = 0; qt < nq; qt++) {
          bool any = false;
          for (size_t q = qt * T; q < std::min(a.tq, qt * T + T) && !any; q++)
            for (size_t k = kt * T; k < std::min(a.tk, kt * T + T) && !any; k++) any = seen(q, k);
          if (any) {
            lo = std::min(lo, qt);
            hi = qt + 1;
          }
        }
        kpass += all_rows ? (double)(hi > lo ? hi - lo : 0) : (double)nq;
      }
    }
  const double tiles = (double)(nb * nh * nq * nk);
  return {fwd / tiles, (qpass + kpass) / (2.0 * tiles)};
}

AttnShape attn_shape(const AttnRegion& r, const Graph& g) {
  AttnShape a;
  const Shape& ss = g.shape(r.s);
  const size_t rank = ss.size();
  a.tq = ss[rank - 2];
  a.tk = ss[rank - 1];
  a.hd = g.shape(r.q)[rank - 1];
  a.bh = 1;
  for (size_t d = 0; d + 2 < rank; d++) a.bh *= ss[d];
  a.heads = rank >= 4 ? ss[rank - 3] : 1;
  if (rank == 3) a.heads = ss[0];
  if (r.mask >= 0) {
    // Strides of the mask source broadcast (right-aligned) to the scores' shape, over
    // (batch, heads, query, key) with the batch dimensions before the last three merged.
    const Shape& ms = g.shape((uint32_t)r.mask);
    std::vector<int64_t> st(rank, 0);
    int64_t run = 1;
    for (size_t j = ms.size(); j-- > 0;) {
      size_t d = rank - ms.size() + j;
      st[d] = ms[j] == 1 ? 0 : run;
      run *= (int64_t)ms[j];
    }
    a.mask_strides[2] = st[rank - 2];
    a.mask_strides[3] = st[rank - 1];
    a.mask_strides[1] = st[rank - 3];
    a.mask_strides[0] = rank >= 4 ? st[rank - 4] : 0;
    if (rank == 3) {  // one batch dimension: it plays the heads' role
      a.mask_strides[1] = st[0];
      a.mask_strides[0] = 0;
    }
    const size_t batches = a.bh / a.heads;
    a.mask_slices = (a.mask_strides[0] ? batches : 1) * (a.mask_strides[1] ? a.heads : 1);
  }
  return a;
}

namespace {

std::vector<int64_t> contiguous(const Shape& s) {
  std::vector<int64_t> st(s.size(), 1);
  for (size_t d = s.size(); d-- > 1;) st[d - 1] = st[d] * (int64_t)s[d];
  return st;
}

// Strides of a reshape of a strided view, when it needs no copy: groups of old dimensions that
// multiply to groups of new ones must be contiguous relative to each other.
bool reshape_strides(const Shape& os, const std::vector<int64_t>& ost, const Shape& ns, std::vector<int64_t>* nst) {
  std::vector<size_t> od;
  std::vector<int64_t> ostr;
  for (size_t i = 0; i < os.size(); i++)
    if (os[i] != 1) {
      od.push_back(os[i]);
      ostr.push_back(ost[i]);
    }
  nst->assign(ns.size(), 0);
  size_t oi = 0, ni = 0;
  while (ni < ns.size() && oi < od.size()) {
    if (ns[ni] == 1) {
      ni++;
      continue;
    }
    size_t np = ns[ni], op = od[oi], nj = ni + 1, oj = oi + 1;
    while (np != op) {
      if (np < op) {
        if (nj >= ns.size()) return false;
        np *= ns[nj++];
      } else {
        if (oj >= od.size()) return false;
        op *= od[oj++];
      }
    }
    for (size_t k = oi; k + 1 < oj; k++)
      if (ostr[k] != ostr[k + 1] * (int64_t)od[k + 1]) return false;
    int64_t st = ostr[oj - 1];
    for (size_t k = nj; k-- > ni;)
      if (ns[k] != 1) {
        (*nst)[k] = st;
        st *= (int64_t)ns[k];
      }
    ni = nj;
    oi = oj;
  }
  for (; ni < ns.size(); ni++)
    if (ns[ni] != 1) return false;
  return oi == od.size();
}

bool layout_op(const Node& n) {
  return n.op.kind == RG_OP_RESHAPE || n.op.kind == RG_OP_TRANSPOSE || n.op.kind == RG_OP_SLICE;
}

// The operand (b, h, t, d) strides of a [batch..., t, d] view, for the steps' (batch, heads)
// split of the problems: rank 3 puts every problem in the heads' place; ranks above 4 only
// when the leading batch dimensions merge.
bool operand_of(uint32_t node, int64_t offset, const Shape& shape, const std::vector<int64_t>& st, AttnOperand* out) {
  const size_t r = shape.size();
  if (r < 3 || st[r - 1] != 1) return false;
  AttnOperand o;
  o.node = node;
  o.offset = offset;
  o.st = st[r - 2];
  o.sh = st[r - 3];
  o.sb = 0;
  if (r >= 4) {
    o.sb = st[r - 4];
    for (size_t d = 0; d + 4 < r; d++)
      if (st[d] != st[d + 1] * (int64_t)shape[d + 1]) return false;
  }
  // 16-byte vectors along d.
  if (o.offset % 4 || o.st % 4 || o.sh % 4 || o.sb % 4) return false;
  *out = o;
  return true;
}

// Reads of node x: through unclaimed reshapes, transposes and slices back to the buffer of a
// materialized node. Falls back to x's own buffer.
AttnOperand read_view(const Graph& g, uint32_t x, const std::vector<bool>& claimed) {
  std::vector<uint32_t> chain;
  uint32_t cur = x;
  while (layout_op(g.nodes[cur]) && !claimed[cur]) {
    chain.push_back(cur);
    cur = g.nodes[cur].inputs[0];
  }
  AttnOperand own;
  operand_of(x, 0, g.shape(x), contiguous(g.shape(x)), &own);
  if (chain.empty() || g.nodes[cur].op.kind == RG_OP_BROADCAST_TO) return own;
  Shape shape = g.shape(cur);
  std::vector<int64_t> st = contiguous(shape);
  int64_t off = 0;
  for (size_t j = chain.size(); j-- > 0;) {
    const Node& n = g.nodes[chain[j]];
    if (n.op.kind == RG_OP_TRANSPOSE) {
      Shape s2(shape.size());
      std::vector<int64_t> t2(shape.size());
      for (size_t d = 0; d < shape.size(); d++) {
        s2[d] = shape[n.op.v[d]];
        t2[d] = st[n.op.v[d]];
      }
      shape = s2;
      st = t2;
    } else if (n.op.kind == RG_OP_SLICE) {
      for (size_t d = 0; d < shape.size(); d++) {
        off += (int64_t)n.op.v[d] * st[d];
        shape[d] = n.op.w[d] - n.op.v[d];
      }
    } else {
      std::vector<int64_t> t2;
      if (!reshape_strides(shape, st, n.shape, &t2)) return own;
      shape = n.shape;
      st = t2;
    }
  }
  AttnOperand v;
  return operand_of(cur, off, shape, st, &v) ? v : own;
}

// Results written straight into the layout their readers want. The forward writes O into the
// one transpose that alone reads it (the heads merged back). The backward writes dq, dk and dv
// into the transpose of their sum after each is padded into its slice of one tensor (the
// gradient of the slices that split q, k and v from one projection): the sum holds each value
// once, the zeros elsewhere add nothing. Nodes already claimed or returned by the program are
// not folded.
void fold_outputs(const Matcher& mt, const std::set<uint32_t>& taken, AttnRegion& r) {
  const Graph& g = mt.g;
  auto free_node = [&](uint32_t x) { return !taken.count(x) && !mt.is_out[x]; };
  operand_of(r.o, 0, g.shape(r.o), contiguous(g.shape(r.o)), &r.out_o);
  r.fwd_out = {r.o};
  uint32_t t;
  if (!mt.is_out[r.o] && mt.only_user(r.o, &t) && free_node(t) && mt.is(t, RG_OP_TRANSPOSE) &&
      g.nodes[t].op.v.back() == g.shape(t).size() - 1) {
    const Shape& ts = g.shape(t);
    std::vector<int64_t> ct = contiguous(ts), st(ts.size());
    for (size_t j = 0; j < ts.size(); j++) st[g.nodes[t].op.v[j]] = ct[j];
    AttnOperand w;
    if (operand_of(t, 0, g.shape(r.o), st, &w)) {
      r.out_o = w;
      r.fwd.push_back(t);
      r.fwd_out = {t};
    }
  }
  if (!r.has_bwd) return;
  const uint32_t grads[3] = {r.dq, r.dk, r.dv};
  AttnOperand* outs[3] = {&r.out_dq, &r.out_dk, &r.out_dv};
  for (int i = 0; i < 3; i++) operand_of(grads[i], 0, g.shape(grads[i]), contiguous(g.shape(grads[i])), outs[i]);
  r.bwd_out = {r.dq, r.dk, r.dv};
  // gradient -> reshape [1, ...] -> pad to [3, ...] at slice i.
  uint32_t re[3], pad[3], user[3];
  int64_t at[3];
  const Shape& gs = g.shape(r.dq);
  for (int i = 0; i < 3; i++) {
    if (mt.is_out[grads[i]] || g.shape(grads[i]) != gs) return;
    if (!mt.only_user(grads[i], &re[i]) || !free_node(re[i]) || !mt.is(re[i], RG_OP_RESHAPE)) return;
    if (!mt.only_user(re[i], &pad[i]) || !free_node(pad[i]) || !mt.is(pad[i], RG_OP_PAD)) return;
    const Shape& rs = g.shape(re[i]);
    const Node& pn = g.nodes[pad[i]];
    if (rs.size() != gs.size() + 1 || rs[0] != 1 || pn.op.w.size() != rs.size() || pn.op.w[0] != 3) return;
    for (size_t d = 1; d < rs.size(); d++)
      if (rs[d] != gs[d - 1] || pn.op.v[d] != 0 || pn.op.w[d] != rs[d]) return;
    at[i] = (int64_t)pn.op.v[0];
    if (!mt.only_user(pad[i], &user[i]) || !free_node(user[i]) || !mt.is(user[i], RG_OP_ADD)) return;
  }
  if (at[0] == at[1] || at[0] == at[2] || at[1] == at[2]) return;
  // Two adds: `inner` joins two pads, `outer` joins the third pad and `inner`.
  int64_t inner = -1;
  for (int i = 0; i < 3; i++)
    for (int j = i + 1; j < 3; j++)
      if (user[i] == user[j]) inner = user[i];
  if (inner < 0) return;
  uint32_t outer = 0;
  for (int i = 0; i < 3; i++)
    if (user[i] != (uint32_t)inner) outer = user[i];
  uint32_t u;
  if (!mt.only_user((uint32_t)inner, &u) || u != outer) return;
  // The sum, or the one transpose that alone reads it.
  uint32_t fin = outer;
  const Shape& ss = g.shape(outer);
  std::vector<int64_t> sst = contiguous(ss);  // strides of the [3, batch..., t, d] layout
  if (mt.only_user(outer, &u) && free_node(u) && !mt.is_out[outer] && mt.is(u, RG_OP_TRANSPOSE) &&
      g.nodes[u].op.v.back() == ss.size() - 1) {
    const Shape& ts = g.shape(u);
    std::vector<int64_t> ct = contiguous(ts);
    for (size_t j = 0; j < ts.size(); j++) sst[g.nodes[u].op.v[j]] = ct[j];
    fin = u;
  }
  std::vector<int64_t> gst(sst.begin() + 1, sst.end());
  AttnOperand w[3];
  for (int i = 0; i < 3; i++)
    if (!operand_of(fin, at[i] * sst[0], gs, gst, &w[i])) return;
  for (int i = 0; i < 3; i++) {
    *outs[i] = w[i];
    r.bwd.push_back(re[i]);
    r.bwd.push_back(pad[i]);
  }
  r.bwd.push_back((uint32_t)inner);
  r.bwd.push_back(outer);
  if (fin != outer) r.bwd.push_back(fin);
  r.bwd_out = {fin};
}

}  // namespace

std::vector<AttnRegion> match_attention(const Graph& g, const std::vector<bool>& keep, const std::vector<uint32_t>& outputs) {
  Matcher mt(g, keep, outputs);
  std::vector<AttnRegion> out;
  std::set<uint32_t> taken;
  for (size_t i = 0; i < g.nodes.size(); i++) {
    if (!keep[i]) continue;
    AttnRegion r;
    if (!mt.match_forward((uint32_t)i, &r)) continue;
    AttnRegion with_bwd = r;
    AttnRegion* pick = nullptr;
    if (mt.match_backward(&with_bwd) && mt.closed(with_bwd)) pick = &with_bwd;
    else if (mt.closed(r)) pick = &r;
    if (!pick) continue;
    AttnShape a = attn_shape(*pick, g);
    bool fits = (a.hd == 16 || a.hd == 32 || a.hd == 64) && a.tq % 32 == 0 && a.tk % 32 == 0 && a.tq <= RG_ATTN_MAX_T &&
                a.tk <= RG_ATTN_MAX_T && a.tq > 0 && a.tk > 0;
    const size_t rank = g.shape(pick->s).size();
    if (pick->mask >= 0 && (rank > 4 || g.shape((uint32_t)pick->mask).size() > rank)) fits = false;
    if (!fits) continue;
    bool clash = false;
    for (uint32_t m : pick->fwd) clash |= taken.count(m) > 0;
    for (uint32_t m : pick->bwd) clash |= taken.count(m) > 0;
    if (clash) continue;
    fold_outputs(mt, taken, *pick);
    taken.insert(pick->fwd.begin(), pick->fwd.end());
    taken.insert(pick->bwd.begin(), pick->bwd.end());
    out.push_back(*pick);
  }
  // Operand views, once every region's nodes are known: a walk stops at claimed nodes.
  std::vector<bool> claimed(g.nodes.size(), false);
  for (uint32_t m : taken) claimed[m] = true;
  for (auto& r : out) {
    r.in_q = read_view(g, r.q, claimed);
    r.in_k = read_view(g, r.k, claimed);
    r.in_v = read_view(g, r.v, claimed);
    if (r.has_bwd) r.in_do = read_view(g, r.d_o, claimed);
  }
  return out;
}

}  // namespace rg
