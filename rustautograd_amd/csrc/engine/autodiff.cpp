// Reverse-mode differentiation: VJP rules emitted as ordinary IR nodes, so grad-of-grad needs
// nothing extra. Follows the reference's src/autodiff.rs:6-16 (unbroadcast), 67-231 (control
// flow), 245-326 (grad) and 328-558 (per-op rules).
#include <algorithm>
#include <map>

#include "graph.h"

namespace rg {

namespace {

Op mk(rg_op k) { return Op::make(k); }

uint32_t reshape(Graph& g, uint32_t x, const Shape& s) {
  Op o = mk(RG_OP_RESHAPE);
  o.v = s;
  return g.add(o, {x});
}

// Reduces a cotangent of the broadcast shape to the operand's own shape by summing the broadcast axes (autodiff.rs:6-16).
uint32_t unbroadcast(Graph& g, uint32_t ct, Shape target) {  // by value: adding nodes moves g.nodes
  Shape shape = g.shape(ct);
  if (shape == target) return ct;
  size_t lead = shape.size() - target.size();
  Op r = mk(RG_OP_REDUCE);
  r.rk = RK::Sum;
  r.keepdims = true;
  for (size_t i = 0; i < shape.size(); i++)
    if (i < lead || (target[i - lead] == 1 && shape[i] != 1)) r.v.push_back(i);
  uint32_t summed = g.add(r, {ct});
  return reshape(g, summed, target);
}

bool blocks_gradient(const Op& op) {
  switch (op.kind) {
    case RG_OP_STOP_GRADIENT: case RG_OP_SIGN: case RG_OP_GT: case RG_OP_GE: case RG_OP_FLOOR:
    case RG_OP_ARGMAX: case RG_OP_RAND_UNIFORM: case RG_OP_RAND_NORMAL: case RG_OP_KEY_SPLIT:
    case RG_OP_PLACEHOLDER: case RG_OP_ARG_TOP_K:
      return true;
    default: return false;
  }
}

// Swap of the two innermost axes.
uint32_t swap_last(Graph& g, uint32_t v) {
  size_t r = g.shape(v).size();
  Op o = mk(RG_OP_TRANSPOSE);
  for (size_t i = 0; i < r; i++) o.v.push_back(i);
  std::swap(o.v[r - 2], o.v[r - 1]);
  return g.add(o, {v});
}

uint32_t bin(Graph& g, rg_op k, uint32_t a, uint32_t b) { return g.add(mk(k), {a, b}); }
uint32_t un(Graph& g, rg_op k, uint32_t a) { return g.add(mk(k), {a}); }

std::vector<std::pair<uint32_t, uint32_t>> vjp(Graph& g, size_t i, uint32_t ct, const std::vector<bool>& rel) {
  Node node = g.nodes[i];
  uint32_t me = (uint32_t)i;
  DType d = node.dtype;
  uint32_t x = node.inputs.empty() ? 0 : node.inputs[0];
  uint32_t y = node.inputs.size() > 1 ? node.inputs[1] : 0;
  std::vector<std::pair<uint32_t, uint32_t>> out;

  // Single-input ops: the local derivative multiplied into the incoming cotangent.
  int64_t factor = -1;
  switch (node.op.kind) {
    case RG_OP_EXP: factor = me; break;
    case RG_OP_COS: factor = un(g, RG_OP_NEG, un(g, RG_OP_SIN, x)); break;
    case RG_OP_SIN: factor = un(g, RG_OP_COS, x); break;
    case RG_OP_TANH: {
      uint32_t one = g.scalar(d, 1.0);
      uint32_t sq = bin(g, RG_OP_MUL, me, me);
      factor = bin(g, RG_OP_SUB, one, sq);
      break;
    }
    case RG_OP_ABS: factor = un(g, RG_OP_SIGN, x); break;
    default: break;
  }
  if (factor >= 0) {
    out.push_back({x, bin(g, RG_OP_MUL, ct, (uint32_t)factor)});
    return out;
  }

  switch (node.op.kind) {
    case RG_OP_INPUT: case RG_OP_CONST: case RG_OP_STOP_GRADIENT: case RG_OP_SIGN: case RG_OP_GT:
    case RG_OP_GE:
      break;
    case RG_OP_NEG: out.push_back({x, un(g, RG_OP_NEG, ct)}); break;
    case RG_OP_LOG: out.push_back({x, bin(g, RG_OP_DIV, ct, x)}); break;
    case RG_OP_SQRT: {
      uint32_t two = g.scalar(d, 2.0);
      uint32_t denom = bin(g, RG_OP_MUL, two, me);
      out.push_back({x, bin(g, RG_OP_DIV, ct, denom)});
      break;
    }
    case RG_OP_ADD: case RG_OP_SUB: case RG_OP_MUL: case RG_OP_DIV: case RG_OP_POW: case RG_OP_MAX:
    case RG_OP_MIN: {
      Shape sx = g.shape(x), sy = g.shape(y);
      rg_op k = node.op.kind;
      if (rel[x]) {
        uint32_t c;
        if (k == RG_OP_ADD || k == RG_OP_SUB) c = ct;
        else if (k == RG_OP_MUL) c = bin(g, RG_OP_MUL, ct, y);
        else if (k == RG_OP_DIV) c = bin(g, RG_OP_DIV, ct, y);
        else if (k == RG_OP_POW) {
          uint32_t one = g.scalar(d, 1.0);
          uint32_t e = bin(g, RG_OP_SUB, y, one);
          uint32_t p = bin(g, RG_OP_POW, x, e);
          uint32_t f = bin(g, RG_OP_MUL, y, p);
          c = bin(g, RG_OP_MUL, ct, f);
        } else {
          // On equality x receives all of it, as if the op were where(x >= y, x, y).
          uint32_t zero = g.scalar(d, 0.0);
          uint32_t m = k == RG_OP_MAX ? bin(g, RG_OP_GE, x, y) : bin(g, RG_OP_GE, y, x);
          c = g.add(mk(RG_OP_WHERE), {m, ct, zero});
        }
        out.push_back({x, unbroadcast(g, c, sx)});
      }
      if (rel[y]) {
        uint32_t c;
        if (k == RG_OP_ADD) c = ct;
        else if (k == RG_OP_SUB) c = un(g, RG_OP_NEG, ct);
        else if (k == RG_OP_MUL) c = bin(g, RG_OP_MUL, ct, x);
        else if (k == RG_OP_DIV) {
          uint32_t n = un(g, RG_OP_NEG, ct);
          uint32_t nx = bin(g, RG_OP_MUL, n, x);
          uint32_t yy = bin(g, RG_OP_MUL, y, y);
          c = bin(g, RG_OP_DIV, nx, yy);
        } else if (k == RG_OP_POW) {
          uint32_t l = un(g, RG_OP_LOG, x);
          uint32_t f = bin(g, RG_OP_MUL, me, l);
          c = bin(g, RG_OP_MUL, ct, f);
        } else {
          uint32_t zero = g.scalar(d, 0.0);
          uint32_t m = k == RG_OP_MAX ? bin(g, RG_OP_GE, x, y) : bin(g, RG_OP_GE, y, x);
          c = g.add(mk(RG_OP_WHERE), {m, zero, ct});
        }
        out.push_back({y, unbroadcast(g, c, sy)});
      }
      break;
    }
    case RG_OP_WHERE: {
      uint32_t zero = g.scalar(d, 0.0);
      uint32_t c = node.inputs[0], a = node.inputs[1], b = node.inputs[2];
      if (rel[a]) out.push_back({a, g.add(mk(RG_OP_WHERE), {c, ct, zero})});
      if (rel[b]) out.push_back({b, g.add(mk(RG_OP_WHERE), {c, zero, ct})});
      break;
    }
    case RG_OP_MATMUL: {
      // Vectors are lifted to matrices first, so the same formulas serve every operand rank and batching.
      Shape sa = g.shape(x), sb = g.shape(y);
      uint32_t a2 = sa.size() == 1 ? reshape(g, x, {1, sa[0]}) : x;
      uint32_t b2 = sb.size() == 1 ? reshape(g, y, {sb[0], 1}) : y;
      Shape cs = g.shape(ct);
      if (sb.size() == 1) cs.push_back(1);
      if (sa.size() == 1) cs.insert(cs.end() - 1, 1);
      uint32_t ct2 = reshape(g, ct, cs);
      if (rel[x]) {
        uint32_t by = swap_last(g, b2);
        uint32_t m = bin(g, RG_OP_MATMUL, ct2, by);
        Shape target = g.shape(a2);
        uint32_t c = unbroadcast(g, m, target);
        out.push_back({x, reshape(g, c, sa)});
      }
      if (rel[y]) {
        uint32_t c;
        if (sa.size() > 2 && sb.size() == 2) {
          // The right operand is one matrix for every batch: stacking the batch into rows makes
          // its gradient (the sum over batches) a single product, with no per-batch products to reduce.
          size_t k = sb[0], n = sb[1];
          size_t m_total = g.nodes[x].n() / k;
          uint32_t af = reshape(g, x, {m_total, k});
          uint32_t cf = reshape(g, ct2, {m_total, n});
          uint32_t ax = swap_last(g, af);
          c = bin(g, RG_OP_MATMUL, ax, cf);
        } else {
          uint32_t ax = swap_last(g, a2);
          uint32_t m = bin(g, RG_OP_MATMUL, ax, ct2);
          Shape target = g.shape(b2);
          c = unbroadcast(g, m, target);
        }
        out.push_back({y, reshape(g, c, sb)});
      }
      break;
    }
    case RG_OP_TAKE: {
      Op o = mk(RG_OP_TAKE_GRAD);
      o.a = node.op.a;
      o.v = g.shape(x);
      out.push_back({x, g.add(o, {ct, y})});
      break;
    }
    case RG_OP_TAKE_GRAD: {
      Op o = mk(RG_OP_TAKE);
      o.a = node.op.a;
      out.push_back({x, g.add(o, {ct, y})});
      break;
    }
    case RG_OP_TAKE_ALONG: {
      Op o = mk(RG_OP_TAKE_ALONG_GRAD);
      o.v = g.shape(x);
      out.push_back({x, g.add(o, {ct, y})});
      break;
    }
    case RG_OP_TAKE_ALONG_GRAD: out.push_back({x, g.add(mk(RG_OP_TAKE_ALONG), {ct, y})}); break;
    case RG_OP_CONCAT: {
      Shape shape = node.shape;
      size_t axis = node.op.a, at = 0;
      for (uint32_t input : node.inputs) {
        size_t len = g.shape(input)[axis];
        if (rel[input]) {
          Op o = mk(RG_OP_SLICE);
          o.v.assign(shape.size(), 0);
          o.w = shape;
          o.v[axis] = at;
          o.w[axis] = at + len;
          out.push_back({input, g.add(o, {ct})});
        }
        at += len;
      }
      break;
    }
    case RG_OP_CUSTOM: {
      // Copy the recorded rule's nodes, substituting the actual cotangent for its stand-in.
      std::map<uint32_t, uint32_t> memo{{node.op.placeholder, ct}};
      uint32_t last = node.op.placeholder;
      for (auto& r : node.op.rules) last = std::max(last, r.second);
      for (uint32_t id = node.op.placeholder + 1; id <= last; id++) {
        Node n = g.nodes[id];
        bool touches = false;
        for (uint32_t v : n.inputs)
          if (memo.count(v)) touches = true;
        if (touches) {
          std::vector<uint32_t> ins;
          for (uint32_t v : n.inputs) ins.push_back(memo.count(v) ? memo[v] : v);
          memo[id] = g.add(n.op, ins);
        }
      }
      for (auto& r : node.op.rules)
        if (rel[r.first]) out.push_back({r.first, memo.count(r.second) ? memo[r.second] : r.second});
      break;
    }
    case RG_OP_FLOOR: case RG_OP_ARGMAX: case RG_OP_RAND_UNIFORM: case RG_OP_RAND_NORMAL:
    case RG_OP_KEY_SPLIT: case RG_OP_PLACEHOLDER: case RG_OP_ARG_TOP_K: case RG_OP_OUTPUT:
      break;
    case RG_OP_CUMSUM: {
      Op o = mk(RG_OP_CUMSUM);
      o.reverse = !node.op.reverse;
      out.push_back({x, g.add(o, {ct})});
      break;
    }
    case RG_OP_REDUCE: {
      Shape in_shape = g.shape(x);
      Shape keep = in_shape;
      for (size_t a : node.op.v) keep[a] = 1;
      uint32_t ct_keep = reshape(g, ct, keep);
      uint32_t c;
      if (node.op.rk == RK::Sum) {
        Op b = mk(RG_OP_BROADCAST_TO);
        b.v = in_shape;
        c = g.add(b, {ct_keep});
      } else {
        // Equal maxima (minima) split the cotangent evenly among them.
        uint32_t m = reshape(g, me, keep);
        uint32_t mask = node.op.rk == RK::Max ? bin(g, RG_OP_GE, x, m) : bin(g, RG_OP_GE, m, x);
        Op s = mk(RG_OP_REDUCE);
        s.rk = RK::Sum;
        s.v = node.op.v;
        s.keepdims = true;
        uint32_t count = g.add(s, {mask});
        uint32_t share = bin(g, RG_OP_DIV, mask, count);
        c = bin(g, RG_OP_MUL, ct_keep, share);
      }
      out.push_back({x, c});
      break;
    }
    case RG_OP_RESHAPE: out.push_back({x, reshape(g, ct, g.shape(x))}); break;
    case RG_OP_TRANSPOSE: {
      Op o = mk(RG_OP_TRANSPOSE);
      o.v.assign(node.op.v.size(), 0);
      for (size_t k = 0; k < node.op.v.size(); k++) o.v[node.op.v[k]] = k;
      out.push_back({x, g.add(o, {ct})});
      break;
    }
    case RG_OP_BROADCAST_TO: out.push_back({x, unbroadcast(g, ct, g.shape(x))}); break;
    case RG_OP_SLICE: {
      Op o = mk(RG_OP_PAD);
      o.v = node.op.v;
      o.w = g.shape(x);
      out.push_back({x, g.add(o, {ct})});
      break;
    }
    case RG_OP_PAD: {
      Op o = mk(RG_OP_SLICE);
      o.v = node.op.v;
      const Shape& sx = g.shape(x);
      for (size_t k = 0; k < o.v.size(); k++) o.w.push_back(o.v[k] + sx[k]);
      out.push_back({x, g.add(o, {ct})});
      break;
    }
    case RG_OP_CAST: {
      Op o = mk(RG_OP_CAST);
      o.dt = g.dtype(x);
      out.push_back({x, g.add(o, {ct})});
      break;
    }
    default: {
      Json obs = Json::obj();
      obs["operation"] = node.op.name();
      throw DiagError{diag("GRAD_UNSUPPORTED", "error", g.node_json(me), obs, "no_vjp_rule_for_operation", "verified")};
    }
  }
  return out;
}

}  // namespace

namespace {

// ---- control flow ---------------------------------------------------------------------------

// A body's reverse pass as a graph of its own (autodiff.rs:22-59): the body's inputs, then one
// cotangent input per floating-point result; its results are the gradients of
// sum(result * cotangent) with respect to each floating-point input.
struct BodyVjp {
  Graph graph;
  std::vector<uint32_t> grads;      // per entry of float_in
  std::vector<size_t> float_in, float_out;
};

BodyVjp body_vjp(const Body& body) {
  BodyVjp v;
  v.graph = body.graph;
  Graph& g = v.graph;
  g.grads.clear();
  g.notes.clear();
  for (size_t k = 0; k < body.inputs.size(); k++)
    if (body.input_dtype(k) != DType::I32) v.float_in.push_back(k);
  for (size_t k = 0; k < body.outputs.size(); k++)
    if (body.output_dtype(k) != DType::I32) v.float_out.push_back(k);
  const DType d = v.float_in.empty() ? DType::F32 : body.input_dtype(v.float_in[0]);
  uint32_t total = g.scalar(d, 0.0);
  for (size_t k : v.float_out) {
    const uint32_t ct = g.input(body.output_shape(k), body.output_dtype(k));
    const uint32_t prod = bin(g, RG_OP_MUL, body.outputs[k], ct);
    Op r = mk(RG_OP_REDUCE);
    r.rk = RK::Sum;
    for (size_t a = 0; a < g.shape(prod).size(); a++) r.v.push_back(a);
    uint32_t sum = g.add(r, {prod});
    if (g.dtype(sum) != d) {
      Op c = mk(RG_OP_CAST);
      c.dt = d;
      sum = g.add(c, {sum});
    }
    total = bin(g, RG_OP_ADD, total, sum);
  }
  std::vector<uint32_t> wrts;
  for (size_t k : v.float_in) wrts.push_back(body.inputs[k]);
  v.grads = grad(g, total, wrts);
  g.grads.clear();
  g.notes.clear();
  return v;
}

uint32_t zeros(Graph& g, const Shape& s, DType d) { return g.constant(Tensor::full(d, s, 0.0)); }

Shape stacked(size_t len, const Shape& s) {
  Shape r{len};
  r.insert(r.end(), s.begin(), s.end());
  return r;
}

// An input node with a chosen index, appended to a body graph being rewired.
uint32_t numbered_input(Graph& g, size_t index, const Shape& s, DType d) {
  Node n;
  n.op = mk(RG_OP_INPUT);
  n.op.a = index;
  n.shape = s;
  n.dtype = d;
  g.nodes.push_back(std::move(n));
  g.n_inputs++;
  return (uint32_t)(g.nodes.size() - 1);
}

// Reverse rules of control flow (autodiff.rs:67-231). `cots` maps a result index of node `i` to
// its cotangent.
std::vector<std::pair<uint32_t, uint32_t>> vjp_control(Graph& g, size_t i, const std::map<size_t, uint32_t>& cots,
                                                       const std::vector<bool>& rel) {
  const Node node = g.nodes[i];
  std::vector<std::pair<uint32_t, uint32_t>> out;
  if (node.op.kind == RG_OP_WHILE) {
    Json obs = Json::obj();
    obs["alternative"] = "rg.scan with a fixed length";
    throw DiagError{diag("GRAD_THROUGH_WHILE", "error", g.node_json((uint32_t)i), obs, "iteration_count_is_a_runtime_value", "verified")};
  }
  if (node.op.kind == RG_OP_COND) {
    // The same cond over both branches' reverse passes, with the results' cotangents appended.
    BodyVjp t = body_vjp(*node.op.body), e = body_vjp(*node.op.body2);
    const Body& tb = *node.op.body;
    std::vector<uint32_t> ins = node.inputs;
    for (size_t k : t.float_out) {
      auto c = cots.find(k);
      ins.push_back(c != cots.end() ? c->second : zeros(g, tb.output_shape(k), tb.output_dtype(k)));
    }
    Op o = mk(RG_OP_COND);
    o.body = Body::make(std::move(t.graph), t.grads);
    o.body2 = Body::make(std::move(e.graph), e.grads);
    const uint32_t cn = g.add(o, ins);
    for (size_t j = 0; j < t.float_in.size(); j++) {
      const uint32_t target = node.inputs[t.float_in[j] + 1];
      if (rel[target]) out.push_back({target, g.output(cn, j, g.shape(target), g.dtype(target))});
    }
    return out;
  }
  // Scan: a scan in the opposite direction over the body's reverse pass.
  const Body& body = *node.op.body;
  const size_t c = node.op.n_carry, x = node.op.n_x, len = node.op.length;
  const size_t m = body.inputs.size() - c - x;
  const size_t n_y = body.outputs.size() - c;
  BodyVjp v = body_vjp(body);
  Graph& r = v.graph;
  std::vector<size_t> fc, fy, g_x, g_cap;
  for (size_t k : v.float_out) (k < c ? fc : fy).push_back(k);
  for (size_t j = 0; j < v.float_in.size(); j++) {
    if (v.float_in[j] >= c && v.float_in[j] < c + x) g_x.push_back(j);
    if (v.float_in[j] >= c + x) g_cap.push_back(j);
  }
  const size_t n_ct = fc.size(), n_acc = g_cap.size();
  // Cotangents of the stacked carries (second-order gradients) join each carry's gradient at its step.
  std::vector<size_t> hist;
  for (size_t k : fc)
    if (cots.count(c + n_y + k)) hist = fc;
  // The reverse scan's inputs: carries (carry cotangents, capture-gradient sums); xs (the carries
  // before each forward step, the forward xs, the ys' cotangents, the stacked carries'
  // cotangents); captures (the forward captures).
  const size_t n_orig = c + x + m;
  const size_t xs_at = n_ct + n_acc, caps_at = xs_at + c + x + fy.size() + hist.size();
  for (auto& n : r.nodes) {
    if (n.op.kind != RG_OP_INPUT) continue;
    const size_t k = n.op.a;
    if (k < c + x) n.op.a = xs_at + k;
    else if (k < n_orig) n.op.a = caps_at + (k - c - x);
    else if (k - n_orig < n_ct) n.op.a = k - n_orig;
    else n.op.a = xs_at + c + x + (k - n_orig - n_ct);
  }
  std::vector<uint32_t> acc_in;
  for (size_t a = 0; a < n_acc; a++) {
    const uint32_t gid = v.grads[g_cap[a]];
    acc_in.push_back(numbered_input(r, n_ct + a, r.shape(gid), r.dtype(gid)));
  }
  std::vector<uint32_t> outs;
  for (size_t k : fc) {
    const size_t j = (size_t)(std::find(v.float_in.begin(), v.float_in.end(), k) - v.float_in.begin());
    uint32_t gradient = v.grads[j];
    auto h = std::find(hist.begin(), hist.end(), k);
    if (h != hist.end()) {
      const uint32_t saved = numbered_input(r, xs_at + c + x + fy.size() + (size_t)(h - hist.begin()), r.shape(gradient), r.dtype(gradient));
      gradient = bin(r, RG_OP_ADD, gradient, saved);
    }
    outs.push_back(gradient);
  }
  for (size_t a = 0; a < n_acc; a++) outs.push_back(bin(r, RG_OP_ADD, acc_in[a], v.grads[g_cap[a]]));
  for (size_t j : g_x) outs.push_back(v.grads[j]);

  std::vector<uint32_t> ins;
  for (size_t k : fc) {
    auto ct = cots.find(k);
    ins.push_back(ct != cots.end() ? ct->second : zeros(g, body.output_shape(k), body.output_dtype(k)));
  }
  for (size_t j : g_cap) {
    const uint32_t target = node.inputs[v.float_in[j]];
    ins.push_back(zeros(g, g.shape(target), g.dtype(target)));
  }
  for (size_t k = 0; k < c; k++) ins.push_back(g.output((uint32_t)i, c + n_y + k, stacked(len, body.input_shape(k)), body.input_dtype(k)));
  ins.insert(ins.end(), node.inputs.begin() + c, node.inputs.begin() + c + x);
  for (size_t k : fy) {
    auto ct = cots.find(k);
    ins.push_back(ct != cots.end() ? ct->second : zeros(g, stacked(len, body.output_shape(k)), body.output_dtype(k)));
  }
  for (size_t k : hist) {
    auto ct = cots.find(c + n_y + k);
    ins.push_back(ct != cots.end() ? ct->second : zeros(g, stacked(len, body.input_shape(k)), body.input_dtype(k)));
  }
  ins.insert(ins.end(), node.inputs.begin() + c + x, node.inputs.end());
  Op o = mk(RG_OP_SCAN);
  o.body = Body::make(std::move(v.graph), outs);
  o.n_carry = n_ct + n_acc;
  o.n_x = c + x + fy.size() + hist.size();
  o.length = len;
  o.reverse = !node.op.reverse;
  const uint32_t back = g.add(o, ins);
  for (size_t a = 0; a < n_ct; a++) {
    const uint32_t target = node.inputs[fc[a]];
    if (rel[target]) out.push_back({target, g.output(back, a, g.shape(target), g.dtype(target))});
  }
  for (size_t a = 0; a < n_acc; a++) {
    const uint32_t target = node.inputs[v.float_in[g_cap[a]]];
    if (rel[target]) out.push_back({target, g.output(back, n_ct + a, g.shape(target), g.dtype(target))});
  }
  for (size_t a = 0; a < g_x.size(); a++) {
    const uint32_t target = node.inputs[v.float_in[g_x[a]]];
    if (rel[target]) out.push_back({target, g.output(back, n_ct + n_acc + a, g.shape(target), g.dtype(target))});
  }
  return out;
}

}  // namespace

std::vector<uint32_t> grad(Graph& g, uint32_t y, const std::vector<uint32_t>& wrts) {
  if (g.nodes[y].n() != 1) {
    Json obs = Json::obj();
    obs["output_shape"] = Json(g.shape(y));
    obs["required"] = "single element";
    throw DiagError{diag("GRAD_NON_SCALAR", "error", g.node_json(y), obs, "gradient_of_non_scalar_output", "verified")};
  }
  bool int_wrt = false;
  for (uint32_t w : wrts) int_wrt |= g.dtype(w) == DType::I32;
  if (g.dtype(y) == DType::I32 || int_wrt) {
    Json obs = Json::obj();
    obs["output_dtype"] = dname(g.dtype(y));
    Json ds = Json::arr();
    for (uint32_t w : wrts) ds.push(dname(g.dtype(w)));
    obs["wrt_dtypes"] = ds;
    throw DiagError{diag("GRAD_OF_INTEGER", "error", g.node_json(y), obs, "integers_are_not_differentiable", "verified")};
  }
  size_t end = y;
  auto saved_source = g.cur_source;
  int64_t saved_origin = g.cur_origin;

  std::vector<bool> rel(end + 1, false);
  for (size_t i = 0; i <= end; i++) {
    const Node& n = g.nodes[i];
    bool flows = false;
    if (n.op.kind == RG_OP_CUSTOM) {
      // Gradients flow through the user's rule only; the body it wraps is not differentiated.
      for (auto& r : n.op.rules) flows |= rel[r.first];
    } else if (!blocks_gradient(n.op)) {
      for (uint32_t x : n.inputs) flows |= rel[x];
    }
    bool is_wrt = std::find(wrts.begin(), wrts.end(), (uint32_t)i) != wrts.end();
    rel[i] = n.dtype != DType::I32 && (is_wrt || flows);
  }

  std::vector<int64_t> cot(end + 1, -1);
  if (rel[end]) cot[end] = g.constant(Tensor::full(g.dtype(y), g.shape(y), 1.0));
  for (size_t i = end + 1; i-- > 0;) {
    if (g.nodes[i].op.is_control_flow()) {
      if (!rel[i]) continue;
      // The node's results are its later RG_OP_OUTPUT readers, whose cotangents are complete.
      std::map<size_t, uint32_t> cots;
      for (size_t o = i + 1; o <= end; o++) {
        const Node& n = g.nodes[o];
        if (n.op.kind == RG_OP_OUTPUT && n.inputs[0] == i && cot[o] >= 0) cots[n.op.a] = (uint32_t)cot[o];
      }
      if (cots.empty()) continue;
      g.cur_source = g.nodes[i].source;
      g.cur_origin = (int64_t)i;
      for (auto& [input, c] : vjp_control(g, i, cots, rel))
        cot[input] = cot[input] >= 0 ? (int64_t)bin(g, RG_OP_ADD, (uint32_t)cot[input], c) : (int64_t)c;
      continue;
    }
    if (cot[i] < 0) continue;
    uint32_t ct = (uint32_t)cot[i];
    g.cur_source = g.nodes[i].source;
    g.cur_origin = (int64_t)i;
    for (auto& [input, c] : vjp(g, i, ct, rel)) {
      cot[input] = cot[input] >= 0 ? (int64_t)bin(g, RG_OP_ADD, (uint32_t)cot[input], c) : (int64_t)c;
    }
  }
  g.cur_source = saved_source;
  g.cur_origin = saved_origin;
  std::vector<uint32_t> out;
  for (uint32_t w : wrts) {
    int64_t found = w < cot.size() ? cot[w] : -1;
    uint32_t id;
    if (found >= 0) {
      id = (uint32_t)found;
    } else {
      Json obs = Json::obj();
      obs["output_node"] = (long long)y;
      obs["wrt_node"] = (long long)w;
      g.notes.push_back(diag("GRAD_DISCONNECTED", "warning", g.node_json(w), obs, "output_does_not_depend_on_input", "verified"));
      id = g.constant(Tensor::full(g.dtype(w), g.shape(w), 0.0));
    }
    g.grads.push_back({y, w, id});
    out.push_back(id);
  }
  return out;
}

}  // namespace rg
