// IR construction with arity, dtype and shape checks (reference src/graph.rs:316-522).
#include "graph.h"

#include <algorithm>
#include <cstdio>

namespace rg {

bool parse_dtype(const std::string& s, DType* out) {
  if (s == "float32" || s == "f32") *out = DType::F32;
  else if (s == "float64" || s == "f64") *out = DType::F64;
  else if (s == "int32" || s == "i32") *out = DType::I32;
  else return false;
  return true;
}

const char* Op::name() const {
  switch (kind) {
    case RG_OP_INPUT: return "input";
    case RG_OP_CONST: return "const";
    case RG_OP_NEG: return "neg";
    case RG_OP_EXP: return "exp";
    case RG_OP_LOG: return "log";
    case RG_OP_SQRT: return "sqrt";
    case RG_OP_SIN: return "sin";
    case RG_OP_COS: return "cos";
    case RG_OP_TANH: return "tanh";
    case RG_OP_ABS: return "abs";
    case RG_OP_SIGN: return "sign";
    case RG_OP_ADD: return "add";
    case RG_OP_SUB: return "sub";
    case RG_OP_MUL: return "mul";
    case RG_OP_DIV: return "div";
    case RG_OP_POW: return "pow";
    case RG_OP_MAX: return "maximum";
    case RG_OP_MIN: return "minimum";
    case RG_OP_GT: return "gt";
    case RG_OP_GE: return "ge";
    case RG_OP_WHERE: return "where";
    case RG_OP_MATMUL: return "matmul";
    case RG_OP_MATMUL_T: return "matmul_t";
    case RG_OP_REDUCE: return rk == RK::Sum ? "sum" : rk == RK::Max ? "max" : "min";
    case RG_OP_RESHAPE: return "reshape";
    case RG_OP_TRANSPOSE: return "transpose";
    case RG_OP_BROADCAST_TO: return "broadcast_to";
    case RG_OP_SLICE: return "slice";
    case RG_OP_PAD: return "pad";
    case RG_OP_CAST: return "cast";
    case RG_OP_STOP_GRADIENT: return "stop_gradient";
    case RG_OP_FLOOR: return "floor";
    case RG_OP_TAKE: return "take";
    case RG_OP_TAKE_ALONG: return "take_along";
    case RG_OP_TAKE_GRAD: return "take_grad";
    case RG_OP_TAKE_ALONG_GRAD: return "take_along_grad";
    case RG_OP_CONCAT: return "concat";
    case RG_OP_ARGMAX: return "argmax";
    case RG_OP_RAND_UNIFORM: return "random_uniform";
    case RG_OP_RAND_NORMAL: return "random_normal";
    case RG_OP_KEY_SPLIT: return "key_split";
    case RG_OP_ARG_TOP_K: return "arg_top_k";
    case RG_OP_CUMSUM: return "cumsum";
    case RG_OP_SCAN: return "scan";
    case RG_OP_WHILE: return "while_loop";
    case RG_OP_COND: return "cond";
    case RG_OP_OUTPUT: return "output";
    case RG_OP_PLACEHOLDER: return "placeholder";
    case RG_OP_CUSTOM: return "custom_vjp";
    default: return "unknown";
  }
}

bool Op::is_unary_elementwise() const {
  switch (kind) {
    case RG_OP_NEG: case RG_OP_EXP: case RG_OP_LOG: case RG_OP_SQRT: case RG_OP_SIN:
    case RG_OP_COS: case RG_OP_TANH: case RG_OP_ABS: case RG_OP_SIGN: case RG_OP_FLOOR:
      return true;
    default: return false;
  }
}

bool Op::is_binary_elementwise() const {
  switch (kind) {
    case RG_OP_ADD: case RG_OP_SUB: case RG_OP_MUL: case RG_OP_DIV: case RG_OP_POW:
    case RG_OP_MAX: case RG_OP_MIN: case RG_OP_GT: case RG_OP_GE:
      return true;
    default: return false;
  }
}

bool Op::int_ok() const {
  switch (kind) {
    case RG_OP_ADD: case RG_OP_SUB: case RG_OP_MUL: case RG_OP_GT: case RG_OP_GE: case RG_OP_WHERE:
    case RG_OP_RESHAPE: case RG_OP_TRANSPOSE: case RG_OP_BROADCAST_TO: case RG_OP_SLICE:
    case RG_OP_CONCAT: case RG_OP_TAKE: case RG_OP_TAKE_ALONG: case RG_OP_CAST:
    case RG_OP_STOP_GRADIENT: case RG_OP_CUMSUM:
      return true;
    default: return false;
  }
}

bool Op::is_nonsmooth() const {
  switch (kind) {
    case RG_OP_ABS: case RG_OP_SIGN: case RG_OP_FLOOR: case RG_OP_MAX: case RG_OP_MIN: case RG_OP_GT:
    case RG_OP_GE: case RG_OP_WHERE: case RG_OP_CUSTOM: case RG_OP_ARG_TOP_K: case RG_OP_COND:
      return true;
    case RG_OP_REDUCE: return rk != RK::Sum;
    default: return false;
  }
}

static void put_vec(std::string& k, const Shape& v) {
  k += '[';
  for (size_t i = 0; i < v.size(); i++) {
    if (i) k += ',';
    k += std::to_string(v[i]);
  }
  k += ']';
}

std::string Op::key() const {
  std::string k = name();
  k += '|';
  k += std::to_string((int)kind);
  k += ':' + std::to_string(a) + ':' + std::to_string(ta) + std::to_string(tb) + std::to_string(keepdims) +
       std::to_string(reverse) + ':' + std::to_string((int)dt) + ':';
  put_vec(k, v);
  put_vec(k, w);
  if (t) {
    k += ":T" + std::to_string((int)t->dtype);
    put_vec(k, t->shape);
    static const char* hex = "0123456789abcdef";
    for (uint8_t b : t->data) {
      k += hex[b >> 4];
      k += hex[b & 15];
    }
  }
  if (kind == RG_OP_CUSTOM) {
    k += ":C" + std::to_string(placeholder);
    for (auto& r : rules) k += "," + std::to_string(r.first) + "/" + std::to_string(r.second);
  }
  if (is_control_flow()) {
    char ids[64];
    snprintf(ids, sizeof ids, ":B%p,%p", (const void*)body.get(), (const void*)body2.get());
    k += ids;
    k += ":" + std::to_string(n_carry) + "," + std::to_string(n_x) + "," + std::to_string(length) + "," + std::to_string(max_iter);
  }
  return k;
}

Shape* broadcast_shapes(const Shape& a, const Shape& b, Shape* out) {
  size_t r = std::max(a.size(), b.size());
  out->assign(r, 0);
  for (size_t i = 0; i < r; i++) {
    size_t x = i < a.size() ? a[a.size() - 1 - i] : 1;
    size_t y = i < b.size() ? b[b.size() - 1 - i] : 1;
    if (x != y && x != 1 && y != 1) return nullptr;
    (*out)[r - 1 - i] = std::max(x, y);
  }
  return out;
}

static Json shape_json(const Shape& s) { return Json(s); }

Json Graph::node_json(uint32_t id) const {
  const Node& n = nodes[id];
  Json v = Json::obj();
  v["id"] = (long long)id;
  v["operation"] = n.op.name();
  v["source"] = n.source ? Json(*n.source) : Json();
  v["role"] = n.origin >= 0 ? "backward" : "forward";
  if (n.origin >= 0) {
    const Node& f = nodes[(size_t)n.origin];
    Json fw = Json::obj();
    fw["id"] = (long long)n.origin;
    fw["operation"] = f.op.name();
    fw["source"] = f.source ? Json(*f.source) : Json();
    v["forward_node"] = fw;
  }
  return v;
}

Json Graph::pending_json(const Op& op) const {
  Json v = Json::obj();
  v["id"] = Json();
  v["operation"] = op.name();
  v["source"] = cur_source ? Json(*cur_source) : Json();
  v["role"] = "forward";
  return v;
}

void Graph::static_err(const char* code, const Op& op, Json obs, const char* cause) const {
  throw DiagError{diag(code, "error", pending_json(op), std::move(obs), cause, "verified")};
}

uint32_t Graph::push(Op op, std::vector<uint32_t> inputs, Shape shape, DType dtype) {
  Node n;
  n.op = std::move(op);
  n.inputs = std::move(inputs);
  n.shape = std::move(shape);
  n.dtype = dtype;
  n.source = cur_source;
  n.origin = cur_origin;
  nodes.push_back(std::move(n));
  return (uint32_t)(nodes.size() - 1);
}

uint32_t Graph::input(const Shape& s, DType d) {
  Op o = Op::make(RG_OP_INPUT);
  o.a = n_inputs++;
  return push(o, {}, s, d);
}

uint32_t Graph::placeholder(const Shape& s, DType d) { return push(Op::make(RG_OP_PLACEHOLDER), {}, s, d); }

uint32_t Graph::constant(Tensor t) {
  Shape s = t.shape;
  DType d = t.dtype;
  Op o = Op::make(RG_OP_CONST);
  o.t = std::make_shared<const Tensor>(std::move(t));
  return push(o, {}, s, d);
}

uint32_t Graph::add(const Op& op, const std::vector<uint32_t>& inputs) {
  for (uint32_t i : inputs) {
    if (i >= nodes.size()) {
      Json obs = Json::obj();
      obs["input"] = (long long)i;
      static_err("INVALID_NODE_REF", op, obs, "unknown_node_id");
    }
  }
  size_t arity;
  switch (op.kind) {
    case RG_OP_INPUT: case RG_OP_CONST: case RG_OP_PLACEHOLDER: arity = 0; break;
    case RG_OP_WHERE: arity = 3; break;
    case RG_OP_MATMUL: case RG_OP_MATMUL_T: case RG_OP_TAKE: case RG_OP_TAKE_ALONG: case RG_OP_TAKE_GRAD:
    case RG_OP_TAKE_ALONG_GRAD:
      arity = 2; break;
    case RG_OP_CONCAT: arity = std::max<size_t>(inputs.size(), 1); break;
    default:
      if (op.is_control_flow()) arity = inputs.size();
      else if (op.is_binary_elementwise()) arity = 2;
      else arity = 1;
  }
  if (inputs.size() != arity) {
    Json obs = Json::obj();
    obs["expected"] = (long long)arity;
    obs["actual"] = (long long)inputs.size();
    static_err("ARITY_MISMATCH", op, obs, "wrong_input_count");
  }
  if (op.is_control_flow()) {
    check_control_flow(op, inputs);
    return push(op, inputs, {}, DType::F32);
  }
  if (op.kind == RG_OP_OUTPUT) {
    if (inputs.size() != 1 || !nodes[inputs[0]].op.is_control_flow()) {
      Json obs = Json::obj();
      obs["input"] = inputs.empty() ? Json() : Json(nodes[inputs[0]].op.name());
      static_err("INVALID_NODE_REF", op, obs, "output_reads_a_control_flow_node");
    }
    return push(op, inputs, op.v, op.dt);
  }

  std::vector<DType> dtypes;
  for (uint32_t i : inputs) dtypes.push_back(dtype(i));
  bool indexes = op.kind == RG_OP_TAKE || op.kind == RG_OP_TAKE_ALONG || op.kind == RG_OP_TAKE_GRAD ||
                 op.kind == RG_OP_TAKE_ALONG_GRAD;
  if (indexes && dtypes[1] != DType::I32) {
    Json obs = Json::obj();
    obs["index_dtype"] = dname(dtypes[1]);
    static_err("DTYPE_MISMATCH", op, obs, "index_must_be_int32");
  }
  bool random = op.kind == RG_OP_RAND_UNIFORM || op.kind == RG_OP_RAND_NORMAL || op.kind == RG_OP_KEY_SPLIT;
  if (random && (dtypes[0] != DType::I32 || shape(inputs[0]) != Shape{2})) {
    Json obs = Json::obj();
    obs["key_shape"] = shape_json(shape(inputs[0]));
    obs["key_dtype"] = dname(dtypes[0]);
    static_err("INVALID_KEY", op, obs, "key_must_be_int32_of_shape_2");
  }
  if (!indexes && !random && op.kind != RG_OP_CAST) {
    for (size_t k = 1; k < dtypes.size(); k++) {
      if (dtypes[k] != dtypes[k - 1]) {
        Json names = Json::arr();
        for (auto d : dtypes) names.push(dname(d));
        Json obs = Json::obj();
        obs["input_dtypes"] = names;
        static_err("DTYPE_MISMATCH", op, obs, "implicit_promotion_not_allowed");
      }
    }
  }
  if (!random && op.kind != RG_OP_ARGMAX && op.kind != RG_OP_ARG_TOP_K && !dtypes.empty() &&
      dtypes[0] == DType::I32 && !op.int_ok()) {
    Json obs = Json::obj();
    obs["dtype"] = "int32";
    static_err("UNSUPPORTED_DTYPE", op, obs, "operation_is_float_only_cast_first");
  }
  DType dt;
  switch (op.kind) {
    case RG_OP_CAST: dt = op.dt; break;
    case RG_OP_RAND_UNIFORM: case RG_OP_RAND_NORMAL: dt = op.dt; break;
    case RG_OP_KEY_SPLIT: case RG_OP_ARGMAX: case RG_OP_ARG_TOP_K: dt = DType::I32; break;
    default: dt = dtypes.empty() ? DType::F32 : dtypes[0];
  }
  std::vector<Shape> shapes;
  for (uint32_t i : inputs) shapes.push_back(nodes[i].shape);

  if (op.kind == RG_OP_WHERE) {
    // The condition is broadcast to the result shape up front, so the select itself only sees equal shapes (graph.rs:368-379).
    Shape target;
    bool ok = true;
    for (auto& s : shapes) {
      Shape out;
      if (!broadcast_shapes(target, s, &out)) {
        ok = false;
        break;
      }
      target = out;
    }
    if (!ok) {
      Json sh = Json::arr();
      for (auto& s : shapes) sh.push(shape_json(s));
      Json obs = Json::obj();
      obs["input_shapes"] = sh;
      static_err("SHAPE_MISMATCH", op, obs, "incompatible_broadcast");
    }
    std::vector<uint32_t> ids;
    for (size_t k = 0; k < inputs.size(); k++) {
      if (shapes[k] == target) ids.push_back(inputs[k]);
      else {
        Op b = Op::make(RG_OP_BROADCAST_TO);
        b.v = target;
        ids.push_back(add(b, {inputs[k]}));
      }
    }
    return push(op, ids, target, dt);
  }
  Shape s = infer(op, shapes);
  return push(op, inputs, s, dt);
}

Shape Graph::infer(const Op& op, const std::vector<Shape>& s) const {
  auto obs = Json::obj;
  if (op.is_unary_elementwise() || op.kind == RG_OP_CAST || op.kind == RG_OP_STOP_GRADIENT) return s[0];
  if (op.is_binary_elementwise()) {
    Shape out;
    if (!broadcast_shapes(s[0], s[1], &out)) {
      Json o = obs();
      o["lhs_shape"] = shape_json(s[0]);
      o["rhs_shape"] = shape_json(s[1]);
      static_err("SHAPE_MISMATCH", op, o, "incompatible_broadcast");
    }
    return out;
  }
  switch (op.kind) {
    case RG_OP_MATMUL: {
      const Shape &a = s[0], &b = s[1];
      if (a.empty() || b.empty()) {
        Json o = obs();
        o["lhs_shape"] = shape_json(a);
        o["rhs_shape"] = shape_json(b);
        o["minimum_rank"] = 1;
        static_err("UNSUPPORTED_RANK", op, o, "matmul_of_scalar");
      }
      size_t k_a = a.back();
      size_t k_b = b.size() >= 2 ? b[b.size() - 2] : b[0];
      if (k_a != k_b) {
        Json o = obs();
        o["lhs_shape"] = shape_json(a);
        o["rhs_shape"] = shape_json(b);
        o["lhs_inner"] = (long long)k_a;
        o["rhs_inner"] = (long long)k_b;
        static_err("SHAPE_MISMATCH", op, o, "matmul_inner_dimension_mismatch");
      }
      Shape ba(a.begin(), a.begin() + (a.size() >= 2 ? a.size() - 2 : 0));
      Shape bb(b.begin(), b.begin() + (b.size() >= 2 ? b.size() - 2 : 0));
      Shape out;
      if (!broadcast_shapes(ba, bb, &out)) {
        Json o = obs();
        o["lhs_shape"] = shape_json(a);
        o["rhs_shape"] = shape_json(b);
        static_err("SHAPE_MISMATCH", op, o, "matmul_batch_dimensions_incompatible");
      }
      if (a.size() >= 2) out.push_back(a[a.size() - 2]);
      if (b.size() >= 2) out.push_back(b.back());
      return out;
    }
    case RG_OP_MATMUL_T: {
      auto view = [](Shape t, bool flip) {
        if (flip) std::swap(t[t.size() - 2], t[t.size() - 1]);
        return t;
      };
      return infer(Op::make(RG_OP_MATMUL), {view(s[0], op.ta), view(s[1], op.tb)});
    }
    case RG_OP_TAKE: {
      size_t axis = op.a;
      if (axis >= s[0].size() || s[0][axis] == 0) {
        Json o = obs();
        o["shape"] = shape_json(s[0]);
        o["axis"] = (long long)axis;
        static_err("INVALID_AXIS", op, o, "axis_out_of_range_or_empty");
      }
      Shape out(s[0].begin(), s[0].begin() + axis);
      out.insert(out.end(), s[1].begin(), s[1].end());
      out.insert(out.end(), s[0].begin() + axis + 1, s[0].end());
      return out;
    }
    case RG_OP_TAKE_ALONG: {
      bool ok = !s[0].empty() && s[0].size() == s[1].size() &&
                std::equal(s[0].begin(), s[0].end() - 1, s[1].begin()) && s[0].back() > 0;
      if (!ok) {
        Json o = obs();
        o["values_shape"] = shape_json(s[0]);
        o["index_shape"] = shape_json(s[1]);
        static_err("SHAPE_MISMATCH", op, o, "take_along_requires_matching_batch_dimensions");
      }
      return s[1];
    }
    case RG_OP_TAKE_GRAD: case RG_OP_TAKE_ALONG_GRAD: return op.v;
    case RG_OP_CONCAT: {
      size_t axis = op.a, rank = s[0].size();
      bool ok = axis < rank;
      for (auto& t : s) {
        if (t.size() != rank) ok = false;
        else
          for (size_t d = 0; d < rank; d++)
            if (d != axis && t[d] != s[0][d]) ok = false;
      }
      if (!ok) {
        Json sh = Json::arr();
        for (auto& t : s) sh.push(shape_json(t));
        Json o = obs();
        o["input_shapes"] = sh;
        o["axis"] = (long long)axis;
        static_err("SHAPE_MISMATCH", op, o, "concat_shapes_differ_off_axis");
      }
      Shape out = s[0];
      out[axis] = 0;
      for (auto& t : s) out[axis] += t[axis];
      return out;
    }
    case RG_OP_ARG_TOP_K: {
      size_t v = s[0].empty() ? 0 : s[0].back();
      if (op.a == 0 || op.a > v) {
        Json o = obs();
        o["shape"] = shape_json(s[0]);
        o["k"] = (long long)op.a;
        static_err("INVALID_AXIS", op, o, "k_must_be_between_one_and_the_last_axis_size");
      }
      Shape out = s[0];
      out.back() = op.a;
      return out;
    }
    case RG_OP_CUMSUM: {
      if (s[0].empty()) {
        Json o = obs();
        o["shape"] = shape_json(s[0]);
        static_err("INVALID_AXIS", op, o, "cumsum_needs_at_least_one_axis");
      }
      return s[0];
    }
    case RG_OP_ARGMAX: {
      if (s[0].empty() || s[0].back() == 0) {
        Json o = obs();
        o["shape"] = shape_json(s[0]);
        static_err("INVALID_AXIS", op, o, "argmax_needs_a_nonempty_last_axis");
      }
      return Shape(s[0].begin(), s[0].end() - 1);
    }
    case RG_OP_RAND_UNIFORM: case RG_OP_RAND_NORMAL: return op.v;
    case RG_OP_KEY_SPLIT: return Shape{op.a, 2};
    case RG_OP_CUSTOM: return s[0];
    case RG_OP_REDUCE: {
      size_t r = s[0].size();
      std::vector<bool> seen(r, false);
      for (size_t a : op.v) {
        if (a >= r || seen[a]) {
          Json o = obs();
          o["shape"] = shape_json(s[0]);
          o["axes"] = shape_json(op.v);
          static_err("INVALID_AXIS", op, o, "axis_out_of_range_or_duplicate");
        }
        seen[a] = true;
      }
      for (size_t a : op.v)
        if (s[0][a] == 0) {
          Json o = obs();
          o["shape"] = shape_json(s[0]);
          o["axes"] = shape_json(op.v);
          static_err("INVALID_AXIS", op, o, "reduction_over_empty_axis");
        }
      Shape out;
      for (size_t i = 0; i < r; i++) {
        if (seen[i]) {
          if (op.keepdims) out.push_back(1);
        } else {
          out.push_back(s[0][i]);
        }
      }
      return out;
    }
    case RG_OP_RESHAPE: {
      if (numel(op.v) != numel(s[0])) {
        Json o = obs();
        o["input_shape"] = shape_json(s[0]);
        o["target_shape"] = shape_json(op.v);
        static_err("SHAPE_MISMATCH", op, o, "reshape_element_count_mismatch");
      }
      return op.v;
    }
    case RG_OP_TRANSPOSE: {
      Shape sorted = op.v;
      std::sort(sorted.begin(), sorted.end());
      bool ok = sorted.size() == s[0].size();
      for (size_t i = 0; ok && i < sorted.size(); i++) ok = sorted[i] == i;
      if (!ok) {
        Json o = obs();
        o["shape"] = shape_json(s[0]);
        o["perm"] = shape_json(op.v);
        static_err("INVALID_AXIS", op, o, "invalid_permutation");
      }
      Shape out;
      for (size_t p : op.v) out.push_back(s[0][p]);
      return out;
    }
    case RG_OP_BROADCAST_TO: {
      Shape out;
      if (!broadcast_shapes(s[0], op.v, &out) || out != op.v) {
        Json o = obs();
        o["input_shape"] = shape_json(s[0]);
        o["target_shape"] = shape_json(op.v);
        static_err("SHAPE_MISMATCH", op, o, "incompatible_broadcast");
      }
      return op.v;
    }
    case RG_OP_SLICE: {
      const Shape &st = op.v, &sp = op.w;
      bool ok = st.size() == s[0].size() && sp.size() == s[0].size();
      for (size_t i = 0; ok && i < s[0].size(); i++) ok = st[i] <= sp[i] && sp[i] <= s[0][i];
      if (!ok) {
        Json o = obs();
        o["shape"] = shape_json(s[0]);
        o["starts"] = shape_json(st);
        o["stops"] = shape_json(sp);
        static_err("INVALID_SLICE", op, o, "slice_out_of_bounds");
      }
      Shape out;
      for (size_t i = 0; i < s[0].size(); i++) out.push_back(sp[i] - st[i]);
      return out;
    }
    case RG_OP_PAD: {
      const Shape &st = op.v, &to = op.w;
      bool ok = st.size() == s[0].size() && to.size() == s[0].size();
      for (size_t i = 0; ok && i < s[0].size(); i++) ok = st[i] + s[0][i] <= to[i];
      if (!ok) {
        Json o = obs();
        o["shape"] = shape_json(s[0]);
        o["starts"] = shape_json(st);
        o["target_shape"] = shape_json(to);
        static_err("INVALID_SLICE", op, o, "pad_out_of_bounds");
      }
      return to;
    }
    default: {
      Json o = obs();
      o["operation"] = op.name();
      static_err("UNSUPPORTED_OPERATION", op, o, "operation_without_inputs_reached_inference");
    }
  }
}

// Inputs must match what the bodies were traced with (graph.rs:531-556). The frontend checks the
// structure first, so a mismatch here comes from a direct IR user; the bodies' own results are
// checked too, since the executors copy them into carries of the traced shapes.
void Graph::check_control_flow(const Op& op, const std::vector<uint32_t>& inputs) const {
  auto fail = [&](const Body* b, const std::vector<uint32_t>& args) {
    Json want = Json::arr(), have = Json::arr();
    if (b)
      for (size_t k = 0; k < b->inputs.size(); k++) want.push(Json(b->input_shape(k)));
    for (uint32_t a : args) have.push(Json(shape(a)));
    Json obs = Json::obj();
    obs["body_inputs"] = want;
    obs["given_inputs"] = have;
    static_err("CONTROL_FLOW_SHAPE_MISMATCH", op, obs, "inputs_differ_from_the_traced_body");
  };
  // Inputs [stacked_lo, stacked_hi) carry a leading axis of `length` over the body's input.
  auto expect = [&](const Body* b, const std::vector<uint32_t>& args, size_t stacked_lo, size_t stacked_hi, size_t length) {
    if (!b || b->inputs.size() != args.size()) fail(b, args);
    for (size_t k = 0; k < args.size(); k++) {
      const Shape& have = shape(args[k]);
      const Shape& want = b->input_shape(k);
      bool ok;
      if (k >= stacked_lo && k < stacked_hi) ok = !have.empty() && have[0] == length && Shape(have.begin() + 1, have.end()) == want;
      else ok = have == want;
      if (!ok || dtype(args[k]) != b->input_dtype(k)) fail(b, args);
    }
  };
  auto results_match = [&](const Body* b, size_t n, const Body* like, size_t offset) {
    if (b->outputs.size() < n) return false;
    for (size_t k = 0; k < n; k++)
      if (b->output_shape(k) != like->input_shape(offset + k) || b->output_dtype(k) != like->input_dtype(offset + k)) return false;
    return true;
  };
  switch (op.kind) {
    case RG_OP_SCAN:
      expect(op.body.get(), inputs, op.n_carry, op.n_carry + op.n_x, op.length);
      if (!results_match(op.body.get(), op.n_carry, op.body.get(), 0)) fail(op.body.get(), inputs);
      break;
    case RG_OP_WHILE: {
      expect(op.body2.get(), inputs, 0, 0, 0);
      expect(op.body.get(), inputs, 0, 0, 0);
      const Body* c = op.body2.get();
      const bool scalar = c->outputs.size() == 1 && (c->output_shape(0).empty() || c->output_shape(0) == Shape{1});
      if (!scalar || op.body->outputs.size() != op.n_carry || !results_match(op.body.get(), op.n_carry, op.body.get(), 0))
        fail(op.body.get(), inputs);
      break;
    }
    case RG_OP_COND: {
      if (inputs.empty() || numel(shape(inputs[0])) != 1) fail(op.body.get(), inputs);
      std::vector<uint32_t> args(inputs.begin() + 1, inputs.end());
      expect(op.body.get(), args, 0, 0, 0);
      expect(op.body2.get(), args, 0, 0, 0);
      const Body *t = op.body.get(), *e = op.body2.get();
      bool same = t->outputs.size() == e->outputs.size();
      for (size_t k = 0; same && k < t->outputs.size(); k++)
        same = t->output_shape(k) == e->output_shape(k) && t->output_dtype(k) == e->output_dtype(k);
      if (!same) fail(t, args);
      break;
    }
    default: break;
  }
}

uint32_t Graph::output(uint32_t node, size_t index, const Shape& s, DType d) {
  Op o = Op::make(RG_OP_OUTPUT);
  o.a = index;
  o.v = s;
  o.dt = d;
  return add(o, {node});
}

std::shared_ptr<const Body> Body::make(Graph g, std::vector<uint32_t> outputs) {
  auto b = std::make_shared<Body>();
  b->inputs.assign(g.n_inputs, UINT32_MAX);
  for (size_t id = 0; id < g.nodes.size(); id++)
    if (g.nodes[id].op.kind == RG_OP_INPUT && g.nodes[id].op.a < g.n_inputs) b->inputs[g.nodes[id].op.a] = (uint32_t)id;
  for (uint32_t id : b->inputs)
    if (id == UINT32_MAX) throw std::runtime_error("a control-flow body lacks one of its inputs");
  for (uint32_t o : outputs)
    if (o >= g.nodes.size()) throw std::runtime_error("a control-flow body returns an unknown node");
  b->graph = std::move(g);
  b->outputs = std::move(outputs);
  return b;
}

std::vector<bool> Graph::reachable(const std::vector<uint32_t>& outputs) const {
  std::vector<bool> keep(nodes.size(), false);
  for (uint32_t o : outputs) keep[o] = true;
  for (size_t i = nodes.size(); i-- > 0;)
    if (keep[i])
      for (uint32_t x : nodes[i].inputs) keep[x] = true;
  return keep;
}

Graph Graph::to_f64() const {
  Graph g = *this;
  for (auto& n : g.nodes) {
    if (n.op.body) n.op.body = Body::make(n.op.body->graph.to_f64(), n.op.body->outputs);
    if (n.op.body2) n.op.body2 = Body::make(n.op.body2->graph.to_f64(), n.op.body2->outputs);
    if (n.op.kind == RG_OP_OUTPUT && n.op.dt != DType::I32) n.op.dt = DType::F64;
    if (n.dtype == DType::I32) continue;
    n.dtype = DType::F64;
    switch (n.op.kind) {
      case RG_OP_CONST: {
        auto& t = *n.op.t;
        n.op.t = std::make_shared<const Tensor>(Tensor::from_f64(DType::F64, t.shape, t.to_f64()));
        break;
      }
      case RG_OP_CAST: case RG_OP_RAND_UNIFORM: case RG_OP_RAND_NORMAL: n.op.dt = DType::F64; break;
      default: break;
    }
  }
  return g;
}

}  // namespace rg
