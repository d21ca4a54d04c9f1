// Compile, validate and run: follows the reference's src/validate.rs:28-971. The executors are
// device backends (backend.h); the step loop is `run_loop` (validate.rs:289-363), delegated to
// the backend's device-resident loop when it has one.
#include "validate.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>

namespace rg {

namespace {

constexpr uint64_t VALIDATION_SEED = 0x9E3779B97F4A7C15ull;
constexpr size_t GRAD_CHECK_SAMPLES = 6;
constexpr double GRAD_CHECK_REL_TOL = 1e-4;
constexpr double GRAD_CHECK_ABS_TOL = 1e-7;
constexpr double PERTURBATION = 1e-3;
constexpr double EQUIVALENCE_TOL = 1e-7;
constexpr double DEVICE_TOL = 1e-2;
constexpr size_t MAX_ROOTS = 8;

using Clock = std::chrono::steady_clock;
double since(Clock::time_point t0) { return std::chrono::duration<double>(Clock::now() - t0).count(); }

// The shortest decimal form of an f32, so 92.7 reports as 92.7 (tensor.rs:271-273).
double json_f64(const Tensor& t, size_t i) {
  if (t.dtype != DType::F32) return t.at(i);
  float f;
  memcpy(&f, &t.data[i * 4], 4);
  if (!std::isfinite(f)) return f;
  char buf[48];
  auto r = std::to_chars(buf, buf + sizeof buf - 1, f);
  *r.ptr = 0;
  return strtod(buf, nullptr);
}

struct Stats {
  double min = INFINITY, max = -INFINITY;
  size_t nan = 0, inf = 0, zero = 0, n = 0;
  bool has_fraction = false;
  int64_t first_bad = -1;
};

Stats stats_of(const Tensor& t, size_t n) {
  Stats s;
  s.n = n;
  for (size_t i = 0; i < n; i++) {
    double f = json_f64(t, i);
    if (std::isnan(f)) s.nan++;
    else if (std::isinf(f)) s.inf++;
    else {
      s.min = std::min(s.min, f);
      s.max = std::max(s.max, f);
      s.zero += f == 0.0;
      s.has_fraction |= f != std::trunc(f);
      continue;
    }
    if (s.first_bad < 0) s.first_bad = (int64_t)i;
  }
  return s;
}

bool any_nonfinite(const Tensor& t) {
  if (t.dtype == DType::I32) return false;
  for (size_t i = 0; i < t.n(); i++)
    if (!std::isfinite(t.at(i))) return true;
  return false;
}

struct Classified {
  const char *code, *cause, *certainty;
};

// Classifies why an op turned finite inputs into a non-finite output (validate.rs:95-128).
Classified classify(const Instr& i, const std::vector<Stats>& args, const Stats& out) {
  switch (i.op.kind) {
    case RG_OP_EXP: return {"NUMERIC_OVERFLOW", "exponential_overflow", "verified"};
    case RG_OP_LOG:
      return args[0].min < 0.0 ? Classified{"DOMAIN_ERROR", "log_of_negative", "verified"}
                               : Classified{"DOMAIN_ERROR", "log_of_zero", "verified"};
    case RG_OP_SQRT: return {"DOMAIN_ERROR", "sqrt_of_negative", "verified"};
    case RG_OP_DIV:
      return args[1].zero > 0 ? Classified{"DIVIDE_BY_ZERO", "division_by_zero", "verified"}
                              : Classified{"NUMERIC_OVERFLOW", "division_overflow", "verified"};
    case RG_OP_POW: {
      const char* c = args[1].n == 1 ? "verified" : "suspected";
      if (args[0].min < 0.0 && args[1].has_fraction) return {"DOMAIN_ERROR", "negative_base_fractional_exponent", c};
      if (args[0].zero > 0 && args[1].min < 0.0) return {"DIVIDE_BY_ZERO", "zero_base_negative_exponent", c};
      return {"NUMERIC_OVERFLOW", "power_overflow", c};
    }
    case RG_OP_CAST: return {"NUMERIC_OVERFLOW", "cast_overflow", "verified"};
    case RG_OP_ADD: case RG_OP_SUB: case RG_OP_MUL: case RG_OP_REDUCE: case RG_OP_MATMUL:
      if (out.nan == 0) return {"NUMERIC_OVERFLOW", "arithmetic_overflow", "verified"};
      return {"NUMERIC_OVERFLOW", "overflow_then_cancellation", "suspected"};
    default: return {"NONFINITE_OUTPUT", "unknown", "unknown"};
  }
}

Tensor as_f64(const Tensor& t) { return t.dtype == DType::I32 ? t : Tensor::from_f64(DType::F64, t.shape, t.to_f64()); }

struct Rng {
  uint64_t s;
  uint64_t next() {
    s ^= s << 13;
    s ^= s >> 7;
    s ^= s << 17;
    return s;
  }
};

std::vector<Tensor> run_plan_once(Backend* b, const Plan& plan, const std::vector<Tensor>& inputs, size_t n_out) {
  DeviceProgram prog(b, plan);
  auto e = prog.exec();
  for (size_t k = 0; k < inputs.size(); k++) e->load(k, inputs[k]);
  e->step();
  if (auto f = e->failure()) throw DiagError{device_failure(b->name, *f)};
  std::vector<Tensor> out;
  for (size_t k = 0; k < n_out; k++) out.push_back(e->prefix(plan.outputs[k].slot, plan.outputs[k].n, plan.outputs[k].shape));
  return out;
}

Json check_status(const std::vector<Json>& d) {
  if (d.empty()) return "pass";
  for (auto& x : d)
    if (x.get("severity") && *x.get("severity") == "error") return "fail";
  return "warn";
}

bool is_error(const Json& d) { return d.get("severity") && *d.get("severity") == "error"; }

}  // namespace

bool parse_level(const std::string& s, Level* out) {
  if (s == "none") *out = Level::None;
  else if (s == "basic") *out = Level::Basic;
  else if (s == "standard") *out = Level::Standard;
  else if (s == "thorough") *out = Level::Thorough;
  else return false;
  return true;
}

Json device_failure(const std::string& device, const std::string& error) {
  Json obs = Json::obj();
  obs["device"] = device;
  obs["detail"] = error;
  return diag("DEVICE_EXECUTION_FAILED", "error", Json(), obs, "gpu_reported_a_failure", "verified");
}

void Compiled::check_inputs(const std::vector<Tensor>& inputs) const {
  std::vector<uint32_t> ids;
  for (size_t i = 0; i < raw.nodes.size(); i++)
    if (raw.nodes[i].op.kind == RG_OP_INPUT) ids.push_back((uint32_t)i);
  if (ids.size() != inputs.size()) {
    Json obs = Json::obj();
    obs["expected_inputs"] = ids.size();
    obs["actual_inputs"] = inputs.size();
    obs["recompile_required"] = true;
    throw DiagError{diag("INPUT_SIGNATURE_MISMATCH", "error", Json(), obs, "input_count_changed", "verified")};
  }
  for (size_t k = 0; k < ids.size(); k++) {
    const Node& node = raw.nodes[ids[k]];
    const Tensor& t = inputs[k];
    if (node.shape != t.shape || node.dtype != t.dtype) {
      Json obs = Json::obj();
      obs["input_index"] = k;
      obs["expected_shape"] = Json(node.shape);
      obs["actual_shape"] = Json(t.shape);
      obs["expected_dtype"] = dname(node.dtype);
      obs["actual_dtype"] = dname(t.dtype);
      obs["recompile_required"] = true;
      throw DiagError{diag("INPUT_SIGNATURE_MISMATCH", "error", raw.node_json(ids[k]), obs, "input_signature_changed", "verified")};
    }
  }
}

std::vector<Tensor> Compiled::try_call(const std::vector<Tensor>& inputs) const {
  std::unique_ptr<DeviceExec> e;
  try {
    e = program->exec();
  } catch (std::exception& ex) {
    throw DiagError{device_failure(device->name, ex.what())};
  }
  for (size_t k = 0; k < inputs.size(); k++) e->load(k, inputs[k]);
  e->step();
  if (auto f = e->failure()) throw DiagError{device_failure(device->name, *f)};
  std::vector<Tensor> out;
  for (auto& o : plan.outputs) out.push_back(e->prefix(o.slot, o.n, o.shape));
  return out;
}

std::vector<uint32_t> Compiled::raw_outputs() const {
  std::vector<uint32_t> all = outputs;
  for (auto& r : raw.grads) all.push_back(r.grad);
  return all;
}

namespace {

// Runs a plan of the traced graph one step at a time on the device, observing each instruction
// (validate.rs:132-230). Control-flow steps are interpreted here, each body iteration running as
// a program of its own, so findings inside a body name the body's node, with the iteration and
// nesting depth (validate.rs:143-153, 218-229), and a while loop stopped by its iteration limit is
// reported (validate.rs:224-229).
struct Observer {
  Compiled::Observed& o;
  Backend* device;
  std::map<const Plan*, std::unique_ptr<DeviceProgram>>& programs;
  std::vector<std::pair<const Body*, size_t>> scopes;

  Json node_json(const Graph& g, uint32_t id) const {
    Json v = g.node_json(id);
    if (!scopes.empty()) {
      Json cf = Json::obj();
      cf["iteration"] = (unsigned long long)scopes.back().second;
      cf["depth"] = (unsigned long long)scopes.size();
      v["control_flow"] = cf;
    }
    return v;
  }

  // A body's plan run once on `inputs`, inside scope (body, iteration).
  std::vector<Tensor> body(const Plan& plan, const Body& b, size_t iteration, const std::vector<Tensor>& inputs) {
    auto& prog = programs[&plan];
    if (!prog) prog = std::make_unique<DeviceProgram>(device, plan);
    scopes.push_back({&b, iteration});
    auto e = prog->exec();
    std::vector<Tensor> out = run(plan, b.graph, *e, inputs);
    scopes.pop_back();
    return out;
  }

  std::vector<Tensor> run(const Plan& plan, const Graph& g, DeviceExec& e, const std::vector<Tensor>& inputs) {
    std::vector<std::pair<size_t, const Tensor*>> loads;
    for (size_t k = 0; k < inputs.size(); k++) loads.push_back({k, &inputs[k]});
    e.load_all(loads);
    for (size_t si = 0; si < plan.steps.size(); si++) {
      const Instr& i = plan.steps[si].instr;
      if (i.op.is_control_flow()) {
        control(i, g, e);
        continue;
      }
      e.steps(si, si + 1);
      instr(i, g, e);
    }
    if (auto f = e.failure()) throw DiagError{device_failure(device->name, *f)};
    std::vector<Tensor> out;
    for (auto& po : plan.outputs) out.push_back(e.prefix(po.slot, po.n, po.shape));
    return out;
  }

  // plan.rs:737-831, with every body iteration observed.
  void control(const Instr& i, const Graph& g, DeviceExec& e) {
    std::vector<Tensor> args;
    for (size_t k = 0; k < i.args.size(); k++) args.push_back(e.prefix(i.args[k], numel(i.arg_shapes[k]), i.arg_shapes[k]));
    std::map<size_t, Tensor> result;
    const Op& op = i.op;
    if (op.kind == RG_OP_SCAN) {
      const Body& b = *op.body;
      const size_t c = op.n_carry, x = op.n_x, len = op.length, n_y = b.outputs.size() - c;
      std::vector<Tensor> carry(args.begin(), args.begin() + c);
      std::vector<Tensor> ys(n_y), before(c);
      for (size_t k = 0; k < n_y; k++) ys[k] = Tensor::full(b.output_dtype(k + c), stacked_shape(len, b.output_shape(k + c)), 0.0);
      for (size_t k = 0; k < c; k++) before[k] = Tensor::full(b.input_dtype(k), stacked_shape(len, b.input_shape(k)), 0.0);
      for (size_t step = 0; step < len; step++) {
        const size_t at = op.reverse ? len - 1 - step : step;
        std::vector<Tensor> in = carry;
        for (size_t k = c; k < c + x; k++) in.push_back(row_of(args[k], at, b.input_shape(k)));
        in.insert(in.end(), args.begin() + c + x, args.end());
        for (size_t k = 0; k < c; k++) put_row(before[k], at, carry[k]);
        std::vector<Tensor> out = body(*i.bodies[0], b, at, in);
        for (size_t k = 0; k < n_y; k++) put_row(ys[k], at, out[c + k]);
        carry.assign(out.begin(), out.begin() + c);
      }
      for (size_t k = 0; k < c; k++) result[k] = carry[k];
      for (size_t k = 0; k < n_y; k++) result[c + k] = ys[k];
      for (size_t k = 0; k < c; k++) result[c + n_y + k] = before[k];
    } else if (op.kind == RG_OP_WHILE) {
      const size_t c = op.n_carry;
      std::vector<Tensor> state(args.begin(), args.begin() + c), caps(args.begin() + c, args.end());
      size_t count = 0;
      for (;;) {
        std::vector<Tensor> in = state;
        in.insert(in.end(), caps.begin(), caps.end());
        if (body(*i.bodies[0], *op.body2, count, in)[0].at(0) == 0.0) break;
        if (count == op.max_iter) {
          Json obs = Json::obj();
          obs["max_iterations"] = (unsigned long long)op.max_iter;
          o.hard.push_back(diag("WHILE_LIMIT_REACHED", "error", node_json(g, i.node), obs, "condition_stayed_true_past_the_limit", "verified"));
          break;
        }
        std::vector<Tensor> out = body(*i.bodies[1], *op.body, count, in);
        state.assign(out.begin(), out.begin() + c);
        count++;
      }
      for (size_t k = 0; k < c; k++) result[k] = state[k];
      result[c] = Tensor::full(DType::I32, {}, (double)count);
    } else {
      const bool taken = args[0].at(0) != 0.0;
      std::vector<Tensor> in(args.begin() + 1, args.end());
      std::vector<Tensor> out = body(*i.bodies[taken ? 0 : 1], taken ? *op.body : *op.body2, 0, in);
      for (size_t k = 0; k < out.size(); k++) result[k] = out[k];
    }
    for (auto& [index, slot] : i.outs) e.write_prefix(slot, result.at(index));
  }

  static Shape stacked_shape(size_t len, const Shape& s) {
    Shape r{len};
    r.insert(r.end(), s.begin(), s.end());
    return r;
  }
  static Tensor row_of(const Tensor& t, size_t at, const Shape& shape) {
    Tensor r;
    r.shape = shape;
    r.dtype = t.dtype;
    const size_t bytes = numel(shape) * dsize(t.dtype);
    r.data.assign(t.data.begin() + at * bytes, t.data.begin() + (at + 1) * bytes);
    return r;
  }
  static void put_row(Tensor& t, size_t at, const Tensor& row) {
    std::copy(row.data.begin(), row.data.end(), t.data.begin() + at * row.data.size());
  }

  void instr(const Instr& i, const Graph& g, DeviceExec& e) {
    auto read_arg = [&](size_t k) { return e.prefix(i.args[k], numel(i.arg_shapes[k]), i.arg_shapes[k]); };
    // Index range check (validate.rs:148-161).
    if ((i.op.kind == RG_OP_TAKE || i.op.kind == RG_OP_TAKE_ALONG) && o.hard.size() < MAX_ROOTS) {
      size_t dim = i.op.kind == RG_OP_TAKE ? i.arg_shapes[0][i.op.a] : i.arg_shapes[0].back();
      size_t n = numel(i.arg_shapes[1]);
      Stats s = stats_of(read_arg(1), n);
      if (n > 0 && (s.min < 0.0 || s.max >= (double)dim)) {
        Json obs = Json::obj();
        obs["index_min"] = s.min;
        obs["index_max"] = s.max;
        obs["axis_size"] = dim;
        obs["behavior_at_runtime"] = "clamped";
        o.hard.push_back(diag("INDEX_OUT_OF_RANGE", "error", node_json(g, i.node), obs, "index_outside_axis", "verified"));
      }
    }
    if (i.dtype == DType::I32) return;
    Tensor dst = e.prefix(i.dst, i.n, i.shape);
    if (!any_nonfinite(dst)) return;
    std::vector<Stats> args;
    std::vector<Tensor> argv;
    bool propagated = false;
    for (size_t k = 0; k < i.args.size(); k++) {
      argv.push_back(read_arg(k));
      args.push_back(stats_of(argv.back(), argv.back().n()));
      propagated |= args.back().first_bad >= 0;
    }
    if (propagated) {
      o.propagated++;
      return;
    }
    if (o.roots.size() == MAX_ROOTS) return;
    Stats out = stats_of(dst, i.n);
    Classified c = classify(i, args, out);
    int64_t bad = out.first_bad;
    bool elementwise = i.op.is_unary_elementwise() || i.op.is_binary_elementwise();
    Json witness;
    if (elementwise && i.mode != RG_MODE_GENERAL) {
      witness = Json::obj();
      Json vals = Json::arr();
      for (size_t k = 0; k < argv.size(); k++)
        vals.push(num(json_f64(argv[k], argv[k].n() == i.n ? (size_t)bad : 0)));
      witness["index"] = (long long)bad;
      witness["inputs"] = vals;
      witness["output"] = num(json_f64(dst, (size_t)bad));
    }
    Json obs = Json::obj();
    obs["dtype"] = dname(i.dtype);
    Json ins = Json::arr();
    for (size_t k = 0; k < args.size(); k++) {
      Json a = Json::obj();
      a["shape"] = Json(i.arg_shapes[k]);
      a["min"] = num(args[k].min);
      a["max"] = num(args[k].max);
      a["contains_zero"] = args[k].zero > 0;
      ins.push(a);
    }
    obs["inputs"] = ins;
    obs["output_shape"] = Json(i.shape);
    obs["output_contains_inf"] = out.inf > 0;
    obs["output_contains_nan"] = out.nan > 0;
    obs["nonfinite_count"] = out.nan + out.inf;
    obs["witness"] = witness;
    if (args.size() == 1) {
      obs["input_max"] = num(args[0].max);
      obs["input_min"] = num(args[0].min);
      if (i.op.kind == RG_OP_EXP) obs["overflow_threshold"] = num(i.dtype == DType::F32 ? 88.722839 : 709.782712);
    }
    o.roots.push_back(diag(c.code, "error", node_json(g, i.node), obs, c.cause, c.certainty));
  }
};

}  // namespace

// Observes every node of the plan built from the traced graph as written (no optimization), so
// each finding carries the node id and source line the user traced (validate.rs:537-565,
// observer at 132-230). Runs on the compiled device, one step at a time.
Compiled::Observed Compiled::observed(const std::vector<Tensor>& inputs) {
  Observed o;
  std::vector<bool> keep = raw.reachable(raw_outputs());
  for (size_t id = 0; id < raw.nodes.size(); id++) {
    const Node& n = raw.nodes[id];
    const Tensor* t = nullptr;
    if (n.op.kind == RG_OP_INPUT) t = &inputs[n.op.a];
    else if (n.op.kind == RG_OP_CONST) t = n.op.t.get();
    if (!t || !keep[id] || t->is_finite()) continue;
    Stats s = stats_of(*t, t->n());
    Json obs = Json::obj();
    obs["dtype"] = dname(n.dtype);
    obs["shape"] = Json(n.shape);
    obs["contains_inf"] = s.inf > 0;
    obs["contains_nan"] = s.nan > 0;
    obs["nonfinite_count"] = s.nan + s.inf;
    obs["first_bad_index"] = s.first_bad >= 0 ? Json((long long)s.first_bad) : Json();
    o.roots.push_back(diag("NONFINITE_INPUT", "error", raw.node_json((uint32_t)id), obs, "nonfinite_value_supplied", "verified"));
  }
  if (!raw_program) raw_program = std::make_unique<DeviceProgram>(device, raw_plan);
  auto e = raw_program->exec();
  Observer ob{o, device, body_programs, {}};
  o.vals = ob.run(raw_plan, raw, *e, inputs);
  return o;
}

std::pair<Json, std::vector<Json>> Compiled::gradient_stats(const std::vector<Tensor>& vals) const {
  Json out = Json::arr();
  std::vector<Json> diags;
  for (size_t k = 0; k < raw.grads.size(); k++) {
    const GradRecord& r = raw.grads[k];
    std::vector<double> v = vals[outputs.size() + k].to_f64();
    if (v.empty()) continue;
    size_t zeros = 0;
    double sq = 0, max_abs = 0;
    for (double x : v) {
      zeros += x == 0.0;
      sq += x * x;
      if (std::fabs(x) > max_abs || std::isnan(x)) max_abs = std::fabs(x);
    }
    Json j = Json::obj();
    j["output_node"] = (long long)r.y;
    j["wrt_node"] = (long long)r.wrt;
    j["grad_node"] = (long long)r.grad;
    auto& src = raw.nodes[r.wrt].source;
    j["source"] = src ? Json(*src) : Json();
    j["norm"] = num(std::sqrt(sq));
    j["rms"] = num(std::sqrt(sq / (double)v.size()));
    j["max_abs"] = num(max_abs);
    j["zero_ratio"] = num((double)zeros / (double)v.size());
    out.push(j);
    bool is_const = raw.nodes[r.grad].op.kind == RG_OP_CONST;
    if (zeros == v.size() && !is_const) {
      Json obs = Json::obj();
      obs["wrt_node"] = (long long)r.wrt;
      obs["zero_ratio"] = 1.0;
      obs["elements"] = v.size();
      diags.push_back(diag("GRAD_ALL_ZERO", "warning", raw.node_json(r.grad), obs, "zero_gradient_at_sample", "suspected"));
    }
  }
  return {out, diags};
}

Json Compiled::check(const std::vector<Tensor>& inputs) {
  Observed o = observed(inputs);
  std::vector<size_t> bad_outputs;
  for (size_t k = 0; k < outputs.size(); k++)
    if (!o.vals[k].is_finite()) bad_outputs.push_back(k);
  if (bad_outputs.empty()) {
    for (auto& r : o.roots) {
      r["severity"] = "warning";
      r["status"] = "warning";
      r["masked"] = true;
    }
  }
  auto [grads, grad_diags] = gradient_stats(o.vals);
  const char* status = (!bad_outputs.empty() || !o.hard.empty()) ? "validation_failed"
                       : (!o.roots.empty() || !grad_diags.empty()) ? "warning" : "ok";
  size_t found = o.roots.size();
  Json diags = Json::arr();
  for (auto& r : o.roots) diags.push(r);
  for (auto& r : grad_diags) diags.push(r);
  for (auto& r : o.hard) diags.push(r);
  Json nf = Json::obj();
  nf["root_nodes"] = found;
  nf["propagated_nodes"] = o.propagated;
  nf["affected_outputs"] = Json(bad_outputs);
  Json j = Json::obj();
  j["status"] = status;
  j["nonfinite"] = nf;
  j["gradients"] = grads;
  j["diagnostics"] = diags;
  return j;
}

// The optimized, fused, buffer-reusing plan against the plain graph, both in f64
// (validate.rs:634-670). Both run on the compiled device.
Json Compiled::optimizer_check(const std::vector<Tensor>& examples) const {
  Graph shadow = raw.to_f64();
  std::vector<Tensor> inputs;
  for (auto& t : examples) inputs.push_back(as_f64(t));
  Optimized opt = optimize_mode(shadow, outputs, false, mode);
  std::vector<Tensor> fast = run_plan_once(device, build_fused(opt.g, opt.outputs, Fuse::cpu()), inputs, outputs.size());
  std::vector<Tensor> reference = run_plan_once(device, build_plan(shadow, outputs, false), inputs, outputs.size());
  double max_rel = 0;
  for (size_t k = 0; k < fast.size(); k++) {
    std::vector<double> va = fast[k].to_f64(), vb = reference[k].to_f64();
    double scale = 1e-30;
    for (double v : vb)
      if (std::isfinite(v)) scale = std::max(scale, std::fabs(v));
    for (size_t j = 0; j < va.size(); j++) {
      double x = va[j], y = vb[j];
      if (x == y || (std::isnan(x) && std::isnan(y))) continue;
      double rel = std::fabs(x - y) / scale;
      max_rel = std::isnan(rel) ? INFINITY : std::max(max_rel, rel);
      if (!(rel <= EQUIVALENCE_TOL)) {
        Json obs = Json::obj();
        obs["output_index"] = k;
        obs["element"] = j;
        obs["optimized"] = num(x);
        obs["reference"] = num(y);
        obs["relative_error"] = num(rel);
        obs["tolerance"] = EQUIVALENCE_TOL;
        obs["precision"] = "float64";
        throw DiagError{diag("OPTIMIZER_MISMATCH", "error", raw.node_json(outputs[k]), obs,
                             "optimized_plan_disagrees_with_reference", "verified")};
      }
    }
  }
  Json j = Json::obj();
  j["max_relative_error"] = num(max_rel);
  j["tolerance"] = EQUIVALENCE_TOL;
  j["precision"] = "float64";
  return j;
}

// Device results against the CPU reference executor in the program's own dtype
// (validate.rs:672-705). The CPU reference is the backend registered as "cpu".
std::pair<Json, std::vector<Json>> Compiled::device_check(const std::vector<Tensor>& examples) const {
  Backend* cpu = find_backend("cpu");
  if (!cpu) {
    Json j = Json::obj();
    j["skipped"] = "no_cpu_reference_backend";
    return {j, {}};
  }
  Optimized opt = optimize_mode(raw, outputs, false, mode);
  std::vector<Tensor> ref = run_plan_once(cpu, build_fused(opt.g, opt.outputs, Fuse::cpu()), examples, outputs.size());
  std::vector<Tensor> gpu;
  try {
    gpu = try_call(examples);
  } catch (DiagError& d) {
    Json j = Json::obj();
    j["skipped"] = "device_failed";
    return {j, {d.d}};
  }
  double max_rel = 0;
  std::vector<Json> diags;
  for (size_t k = 0; k < gpu.size(); k++) {
    std::vector<double> vg = gpu[k].to_f64(), vc = ref[k].to_f64();
    double scale = 1e-30;
    for (double v : vc)
      if (std::isfinite(v)) scale = std::max(scale, std::fabs(v));
    for (size_t j = 0; j < vg.size(); j++) {
      double x = vg[j], y = vc[j];
      if (x == y || (std::isnan(x) && std::isnan(y))) continue;
      double rel = std::fabs(x - y) / scale;
      if (std::isnan(rel)) rel = INFINITY;
      max_rel = std::max(max_rel, rel);
      if (rel > DEVICE_TOL && diags.empty()) {
        Json obs = Json::obj();
        obs["output_index"] = k;
        obs["element"] = j;
        obs[device->name] = num(x);
        obs["cpu"] = num(y);
        obs["relative_error"] = num(rel);
        obs["tolerance"] = DEVICE_TOL;
        diags.push_back(diag("DEVICE_MISMATCH", "warning", raw.node_json(outputs[k]), obs,
                             "device_result_differs_from_cpu", "suspected"));
      }
    }
  }
  Json j = Json::obj();
  j["max_relative_error"] = num(max_rel);
  j["tolerance"] = DEVICE_TOL;
  j["reference"] = cpu->name;
  return {j, diags};
}

// Central differences in f64 against every recorded gradient (validate.rs:707-772).
std::pair<Json, std::vector<Json>> Compiled::grad_check(const std::vector<Tensor>& examples) const {
  Graph shadow = raw.to_f64();
  std::vector<Tensor> inputs64;
  for (auto& t : examples) inputs64.push_back(as_f64(t));
  Rng rng{VALIDATION_SEED};
  size_t checked = 0;
  double max_rel = 0;
  Json skipped = Json::arr();
  std::vector<Json> diags;
  for (auto& r : raw.grads) {
    std::vector<bool> keep = raw.reachable({r.y});
    const Node& wn = raw.nodes[r.wrt];
    if (wn.op.kind != RG_OP_INPUT) {
      Json s = Json::obj();
      s["wrt_node"] = (long long)r.wrt;
      s["reason"] = "wrt_is_not_an_input";
      skipped.push(s);
      continue;
    }
    size_t k = wn.op.a;
    if (raw.nodes[r.grad].op.kind == RG_OP_CONST) {
      Json s = Json::obj();
      s["wrt_node"] = (long long)r.wrt;
      s["reason"] = "disconnected";
      skipped.push(s);
      continue;
    }
    bool suspect = false;
    for (size_t i = 0; i < raw.nodes.size(); i++)
      if (keep[i] && (raw.nodes[i].op.is_nonsmooth() || raw.nodes[i].op.kind == RG_OP_STOP_GRADIENT)) suspect = true;
    const char* certainty = suspect ? "suspected" : "verified";
    Plan analytic_plan = build_plan(shadow, {r.grad}, true);
    std::vector<double> analytic = run_plan_once(device, analytic_plan, inputs64, 1)[0].to_f64();
    Plan y_plan = build_plan(shadow, {r.y}, true);
    DeviceProgram yp(device, y_plan);
    auto yf = yp.exec();
    for (size_t j = 0; j < inputs64.size(); j++) yf->load(j, inputs64[j]);
    std::vector<double> base = inputs64[k].to_f64();
    Tensor probe = inputs64[k];
    for (size_t s = 0; s < std::min(GRAD_CHECK_SAMPLES, base.size()); s++) {
      size_t e = base.size() <= GRAD_CHECK_SAMPLES ? s : (size_t)(rng.next() % base.size());
      double h = 1e-6 * std::max(std::fabs(base[e]), 1.0);
      auto eval_at = [&](double x) {
        memcpy(&probe.data[e * 8], &x, 8);
        yf->load(k, probe);
        yf->step();
        return yf->scalar(y_plan.outputs[0].slot);
      };
      double up = eval_at(base[e] + h), down = eval_at(base[e] - h);
      memcpy(&probe.data[e * 8], &base[e], 8);
      double numeric = (up - down) / (2.0 * h);
      if (!std::isfinite(numeric) || !std::isfinite(analytic[e])) continue;
      checked++;
      double err = std::fabs(numeric - analytic[e]);
      double rel = err / std::max(std::max(std::fabs(numeric), std::fabs(analytic[e])), 1e-12);
      max_rel = std::max(max_rel, err <= GRAD_CHECK_ABS_TOL ? 0.0 : rel);
      if (err > GRAD_CHECK_ABS_TOL && rel > GRAD_CHECK_REL_TOL) {
        Json obs = Json::obj();
        obs["wrt_node"] = (long long)r.wrt;
        obs["element"] = e;
        obs["analytic"] = num(analytic[e]);
        obs["numeric"] = num(numeric);
        obs["relative_error"] = num(rel);
        obs["tolerance"] = GRAD_CHECK_REL_TOL;
        obs["finite_difference_h"] = h;
        obs["seed"] = (unsigned long long)VALIDATION_SEED;
        diags.push_back(diag("GRADIENT_MISMATCH", suspect ? "warning" : "error", raw.node_json(r.grad), obs,
                             "analytic_gradient_disagrees_with_finite_difference", certainty));
        break;
      }
    }
  }
  Json j = Json::obj();
  j["elements_checked"] = checked;
  j["max_relative_error"] = num(max_rel);
  j["skipped"] = skipped;
  return {j, diags};
}

Json Compiled::validate(const std::vector<Tensor>& examples) {
  Json checks = Json::arr();
  Json st = Json::obj();
  st["name"] = "static";
  st["status"] = "pass";
  st["detail"] = "shape and dtype inference passed during tracing";
  checks.push(st);
  std::vector<Json> diagnostics = raw.notes;
  Json gradients = Json::arr();
  if (level >= Level::Basic) {
    Json c = Json::obj();
    c["name"] = "test_run";
    try {
      auto out = try_call(examples);
      Json shapes = Json::arr();
      for (auto& t : out) shapes.push(Json(t.shape));
      c["status"] = "pass";
      c["output_shapes"] = shapes;
    } catch (DiagError& d) {
      c["status"] = "fail";
      diagnostics.push_back(d.d);
    }
    checks.push(c);
  }
  if (level >= Level::Standard) {
    bool ran = true;
    try {
      Json found = check(examples);
      std::vector<Json> ds = found.get("diagnostics")->items();
      Json c = Json::obj();
      c["name"] = "finite";
      c["status"] = check_status(ds);
      c["nonfinite"] = *found.get("nonfinite");
      checks.push(c);
      gradients = *found.get("gradients");
      diagnostics.insert(diagnostics.end(), ds.begin(), ds.end());
    } catch (DiagError& d) {
      ran = false;
      diagnostics.push_back(d.d);
    }
    Json c = Json::obj();
    c["name"] = "optimizer_equivalence";
    try {
      if (!ran) throw DiagError{Json()};
      c["detail"] = optimizer_check(examples);
      c["status"] = "pass";
    } catch (DiagError& d) {
      c["status"] = "fail";
      if (!d.d.is_null()) diagnostics.push_back(d.d);
    }
    checks.push(c);
    if (device->name != "cpu") {
      auto [info, ds] = device_check(examples);
      Json dc = Json::obj();
      dc["name"] = "device_equivalence";
      dc["status"] = info.get("skipped") ? Json("skipped") : check_status(ds);
      dc["detail"] = info;
      checks.push(dc);
      diagnostics.insert(diagnostics.end(), ds.begin(), ds.end());
      if (info.get("skipped") && *info.get("skipped") == "no_cpu_reference_backend") {
        // The product ships no CPU interpreter: say so instead of passing the gate silently.
        Json obs = Json::obj();
        obs["device"] = device->name;
        obs["available"] = Json(available_backends());
        diagnostics.push_back(diag("DEVICE_CHECK_SKIPPED", "warning", Json(), obs,
                                   "no_cpu_reference_backend_registered_device_results_unchecked", "verified"));
      }
    }
  }
  if (level >= Level::Thorough) {
    auto [info, ds] = grad_check(examples);
    Json c = Json::obj();
    c["name"] = "grad_check";
    c["status"] = check_status(ds);
    c["detail"] = info;
    checks.push(c);
    diagnostics.insert(diagnostics.end(), ds.begin(), ds.end());
    // Perturbation (validate.rs:774-797): a slightly moved input can expose what the sample hides.
    Rng rng{VALIDATION_SEED ^ 0xABCD};
    std::vector<Tensor> moved;
    for (auto& t : examples) {
      if (t.dtype == DType::I32) {
        moved.push_back(t);
        continue;
      }
      std::vector<double> v = t.to_f64();
      for (auto& x : v) x *= 1.0 + (rng.next() % 2 == 0 ? PERTURBATION : -PERTURBATION);
      moved.push_back(Tensor::from_f64(t.dtype, t.shape, v));
    }
    std::vector<Json> pd;
    for (auto d : observed(moved).roots) {
      d["severity"] = "warning";
      d["status"] = "warning";
      Json trig = Json::obj();
      trig["kind"] = "input_perturbation";
      trig["relative_magnitude"] = PERTURBATION;
      trig["seed"] = (unsigned long long)VALIDATION_SEED;
      d["trigger"] = trig;
      pd.push_back(d);
    }
    Json pc = Json::obj();
    pc["name"] = "input_perturbation";
    pc["status"] = check_status(pd);
    Json det = Json::obj();
    det["relative_magnitude"] = PERTURBATION;
    pc["detail"] = det;
    checks.push(pc);
    diagnostics.insert(diagnostics.end(), pd.begin(), pd.end());
  }
  bool err = false;
  for (auto& d : diagnostics) err |= is_error(d);
  Json r = Json::obj();
  r["status"] = err ? "validation_failed" : diagnostics.empty() ? "ok" : "warning";
  r["device"] = device->name;
  Json graph = Json::obj();
  graph["optimization"] = opt_stats.json();
  graph["steps"] = plan.steps.size();
  graph["fused_groups"] = plan.n_fused();
  graph["fused_ops"] = plan.n_fused_ops();
  r["graph"] = graph;
  Json mem = Json::obj();
  mem["intermediate_bytes_without_reuse"] = plan.naive_bytes;
  mem["intermediate_bytes_planned"] = plan.planned_bytes();
  mem["peak_live_bytes"] = plan.peak_live_bytes;
  r["memory"] = mem;
  r["checks"] = checks;
  r["gradients"] = gradients;
  Json ds = Json::arr();
  for (auto& d : diagnostics) ds.push(d);
  r["diagnostics"] = ds;
  Json repro = Json::obj();
  static const char* names[] = {"none", "basic", "standard", "thorough"};
  repro["level"] = names[(int)level];
  repro["seed"] = (unsigned long long)VALIDATION_SEED;
  r["repro"] = repro;
  return r;
}

StreamedFn Compiled::streamed_products() const {
  if (!device->gemm_streamed) return {};
  return [d = device](DType dt, uint64_t m, uint64_t n, uint64_t k, uint64_t batch, bool ta, bool tb) {
    return d->gemm_streamed((int32_t)dt, (int64_t)m, (int64_t)n, (int64_t)k, (int64_t)batch, ta, tb) != 0;
  };
}

Json Compiled::profile(const std::vector<Tensor>& inputs, size_t repeats) const {
  repeats = std::max<size_t>(repeats, 1);
  std::vector<double> seconds(plan.steps.size(), 0.0);
  Json breakdown;
  std::unique_ptr<DeviceExec> e;
  try {
    e = program->exec();
  } catch (std::exception& ex) {
    Json j = Json::obj();
    j["error"] = device_failure(device->name, ex.what());
    return j;
  }
  for (size_t k = 0; k < inputs.size(); k++) e->load(k, inputs[k]);
  if (device->exec_breakdown) {
    std::vector<char> buf(1 << 16);
    if (device->exec_breakdown(e->handle(), (int64_t)repeats, buf.data(), buf.size()) == 0) breakdown = Json(std::string(buf.data()));
  }
  for (size_t r = 0; r < repeats; r++) {
    if (device->exec_step_timed) {
      device->exec_step_timed(e->handle(), seconds.data());
    } else {
      for (size_t s = 0; s < plan.steps.size(); s++) {
        auto t0 = Clock::now();
        e->steps(s, s + 1);
        seconds[s] += since(t0);
      }
    }
  }
  // Each operation's algorithmic work (flops against the matrix-core peak, or bytes against HBM
  // bandwidth), as the device runs it, and the device's published peaks when it reports them.
  const StreamedFn streamed = streamed_products();
  double peaks[3] = {0, 0, 0};
  Json roofline = Json::obj();
  bool have_peaks = false;
  if (device->device_peaks) {
    char name[256] = {0};
    have_peaks = device->device_peaks(peaks, name, sizeof name) == 0;
    if (have_peaks) {
      roofline["device"] = std::string(name);
      roofline["hbm_gb_per_s"] = peaks[0];
      roofline["fp32_tflop_per_s"] = peaks[1];
      roofline["fp64_tflop_per_s"] = peaks[2];
    } else {
      roofline["unavailable"] = std::string(name);
    }
  } else {
    roofline["unavailable"] = "the backend reports no device peaks";
  }
  struct Row {
    double seconds = 0, flops = 0, executed_flops = 0, bytes = 0;
    size_t count = 0;
    bool compute = false, f64 = false;
  };
  std::map<std::string, Row> rows;
  auto shape_str = [](const Shape& s) {
    std::string o = "[";
    for (size_t i = 0; i < s.size(); i++) o += (i ? ", " : "") + std::to_string(s[i]);
    return o + "]";
  };
  // A fused group the device computes in a product's epilogue (step_runs_in pairs the two) is
  // counted in the product's row: its time (the combined kernel runs at one of the two steps) and
  // its bytes, with no launch or flops of its own.
  // Products the device launches together (one kernel at one of their steps) keep their own
  // rows; the kernel's time is shared between them in proportion to their flops.
  std::vector<size_t> row_of(plan.steps.size());
  std::vector<double> sec = seconds;
  auto plain = [&](size_t q) { return !plan.steps[q].fused && !plan.steps[q].attn; };
  auto product = [&](size_t q) {
    if (!plain(q)) return false;
    const std::string op = plan.steps[q].instr.op.name();
    return op == "matmul" || op == "matmul_t";
  };
  std::map<size_t, std::vector<size_t>> launched_with;  // launch step -> the products it computes
  for (size_t s = 0; s < plan.steps.size(); s++) row_of[s] = s;
  for (size_t s = 0; s < plan.steps.size(); s++) {
    const int64_t r = program->step_runs_in((int64_t)s);
    if (r < 0 || (size_t)r == s || (size_t)r >= plan.steps.size()) continue;
    if (product(s) && product((size_t)r)) {
      auto& g = launched_with[(size_t)r];
      if (g.empty()) g.push_back((size_t)r);
      g.push_back(s);
      continue;
    }
    // A group in a product's epilogue, or a column sum of its output: the product's row.
    size_t p = product(s) ? s : (size_t)r;
    if (!product(p))
      for (size_t q = 0; q < plan.steps.size(); q++)
        if (program->step_runs_in((int64_t)q) == r && product(q)) p = q;
    row_of[s] = row_of[(size_t)r] = p;
  }
  for (auto& [r, g] : launched_with) {
    double all = 0, flops = 0;
    for (size_t q : g) {
      all += sec[q];
      flops += step_work(plan.steps[q], streamed).flops;
    }
    for (size_t q : g) sec[q] = flops > 0 ? all * step_work(plan.steps[q], streamed).flops / flops : all / (double)g.size();
  }
  for (size_t s0 = 0; s0 < plan.steps.size(); s0++) {
    const size_t s = row_of[s0];
    const Step& st = plan.steps[s];
    std::string key;
    DType dt;
    if (st.attn) {
      key = std::string(st.att.backward ? "attention backward" : "attention") + " bh=" + std::to_string(st.att.shape.bh) +
            " t=" + std::to_string(st.att.shape.tq) + "x" + std::to_string(st.att.shape.tk) + " hd=" + std::to_string(st.att.shape.hd);
      dt = st.att.dtype;
    } else if (st.fused) {
      key = "fused[";
      for (size_t m = 0; m < st.group.ops.size(); m++) key += std::string(m ? "," : "") + st.group.ops[m].op.name();
      key += "] n=" + std::to_string(st.group.n);
      dt = st.group.dtype;
    } else {
      key = std::string(st.instr.op.name()) + " " + shape_str(st.instr.shape) + " <- [";
      for (size_t a = 0; a < st.instr.arg_shapes.size(); a++) key += (a ? ", " : "") + shape_str(st.instr.arg_shapes[a]);
      key += "]";
      dt = st.instr.dtype;
    }
    if (dt == DType::F64) key += " f64";
    const StepWork w = step_work(st, streamed);
    Row& r = rows[key];
    r.seconds += sec[s0];
    if (s0 != s) {  // the group in the product's epilogue
      r.bytes += step_work(plan.steps[s0], streamed).bytes;
      continue;
    }
    r.count++;
    r.flops += w.flops;
    r.executed_flops += w.executed_flops;
    r.bytes += w.bytes;
    r.compute = w.compute;
    r.f64 = dt == DType::F64;
  }
  double total = 0;
  for (double t : seconds) total += t;
  std::vector<std::pair<std::string, Row>> list(rows.begin(), rows.end());
  std::stable_sort(list.begin(), list.end(), [](auto& a, auto& b) { return a.second.seconds > b.second.seconds; });
  Json ops = Json::arr();
  double ideal = 0;  // seconds per pass if every operation ran at its peak
  for (auto& [k, v] : list) {
    Json o = Json::obj();
    o["operation"] = k;
    o["count"] = v.count;
    o["microseconds_per_run"] = v.seconds / (double)repeats * 1e6;
    o["share"] = total > 0 ? v.seconds / total : 0.0;
    o["bound"] = v.compute ? "mfma" : "hbm";
    o["flops_per_run"] = v.flops;
    if (v.compute && v.executed_flops != v.flops) o["executed_flops_per_run"] = v.executed_flops;
    o["bytes_per_run"] = v.bytes;
    const double per_run = v.seconds / (double)repeats;
    const double work = v.compute ? v.flops / 1e12 : v.bytes / 1e9;
    o["unit"] = v.compute ? "TFLOP/s" : "GB/s";
    if (per_run > 0) o["achieved"] = work / per_run;
    if (have_peaks) {
      const double peak = v.compute ? (v.f64 ? peaks[2] : peaks[1]) : peaks[0];
      o["peak"] = peak;
      if (per_run > 0) o["fraction_of_peak"] = work / per_run / peak;
      // Attention skips the tiles a mask hides: its rate over the products it executes.
      if (per_run > 0 && v.compute && v.executed_flops != v.flops) {
        o["executed_achieved"] = v.executed_flops / 1e12 / per_run;
        o["executed_fraction_of_peak"] = v.executed_flops / 1e12 / per_run / peak;
      }
      ideal += work / peak;
    }
    ops.push(o);
  }
  if (have_peaks && total > 0) {
    // The whole pass against the sum of its operations' roofline times.
    roofline["seconds_at_peak_per_run"] = ideal;
    roofline["fraction_of_peak"] = ideal / (total / (double)repeats);
  }
  Json j = Json::obj();
  j["repeats"] = repeats;
  j["microseconds_per_run"] = total / (double)repeats * 1e6;
  j["operations"] = ops;
  j["roofline"] = roofline;
  j["breakdown"] = breakdown;
  return j;
}

void Compiled::validate_spec(const RunSpec& spec) const {
  for (auto& [i, o] : spec.state) {
    uint32_t input = 0;
    for (size_t n = 0; n < raw.nodes.size(); n++)
      if (raw.nodes[n].op.kind == RG_OP_INPUT && raw.nodes[n].op.a == i) input = (uint32_t)n;
    uint32_t out = outputs[o];
    if (raw.shape(input) != raw.shape(out) || raw.dtype(input) != raw.dtype(out)) {
      Json obs = Json::obj();
      obs["input_index"] = i;
      obs["output_index"] = o;
      obs["input_shape"] = Json(raw.shape(input));
      obs["output_shape"] = Json(raw.shape(out));
      obs["input_dtype"] = dname(raw.dtype(input));
      obs["output_dtype"] = dname(raw.dtype(out));
      throw DiagError{diag("STATE_CONTRACT_VIOLATION", "error", raw.node_json(out), obs,
                           "returned_state_differs_from_input_state", "verified")};
    }
  }
}

// The hot loop (validate.rs:289-363).
RunOut Compiled::run(const RunSpec& spec, const std::vector<const Tensor*>& state, const std::vector<std::vector<Tensor>>& batches,
                     size_t steps) const {
  RunOut r;
  std::unique_ptr<DeviceExec> e;
  try {
    e = program->exec();
  } catch (std::exception& ex) {
    for (const Tensor* t : state) r.state.push_back(*t);
    r.history.assign(spec.history.size(), {});
    r.device_error = ex.what();
    return r;
  }
  const Plan& p = plan;
  auto load_batch = [&](const std::vector<Tensor>& b) {
    for (size_t k = 0; k < spec.data.size() && k < b.size(); k++) e->load(spec.data[k], b[k]);
  };
  {
    // The state (and a single batch) go over together, with one wait.
    std::vector<std::pair<size_t, const Tensor*>> first;
    for (size_t k = 0; k < spec.state.size() && k < state.size(); k++) first.push_back({spec.state[k].first, state[k]});
    if (batches.size() == 1)
      for (size_t k = 0; k < spec.data.size() && k < batches[0].size(); k++) first.push_back({spec.data[k], &batches[0][k]});
    e->load_all(first);
  }
  std::vector<bool> feeds_state(p.outputs.size(), false);
  if (spec.skip_state_outputs)
    for (auto& [i, o] : spec.state) feeds_state[o] = true;
  auto read_outputs = [&](auto slot_of) {
    std::vector<std::tuple<size_t, size_t, Shape>> reads;
    std::vector<size_t> at;
    r.outputs.assign(p.outputs.size(), Tensor{});
    for (size_t q = 0; q < p.outputs.size(); q++) {
      r.outputs[q].shape = p.outputs[q].shape;
      r.outputs[q].dtype = p.slots[p.outputs[q].slot].first;
      if (feeds_state[q]) continue;
      reads.push_back({slot_of(p.outputs[q].slot), p.outputs[q].n, p.outputs[q].shape});
      at.push_back(q);
    }
    auto got = e->prefix_all(reads);
    for (size_t j = 0; j < at.size(); j++) r.outputs[at[j]] = std::move(got[j]);
  };
  // Handoff by exchanging buffers where possible: the output slot must be unpinned, used by one state entry, and of the input's size; otherwise the values are copied.
  std::vector<size_t> out_slots;
  for (auto& [i, o] : spec.state) out_slots.push_back(p.outputs[o].slot);
  std::vector<std::pair<size_t, size_t>> swaps;
  std::vector<std::tuple<size_t, size_t, size_t>> copies;
  for (auto& [i, o] : spec.state) {
    size_t is = p.input_slots[i], os = p.outputs[o].slot;
    if (is == os) continue;
    size_t uses = std::count(out_slots.begin(), out_slots.end(), os);
    if (!p.pinned[os] && uses == 1 && p.slots[os].second == p.slots[is].second) swaps.push_back({is, os});
    else copies.push_back({is, os, p.outputs[o].n});
  }
  std::vector<size_t> hist_slots;
  for (size_t o : spec.history) hist_slots.push_back(p.outputs[o].slot);
  r.history.assign(hist_slots.size(), {});

  // Output slots overwritten by a copy lose their pre-handoff value; the device loop reads
  // outputs after the handoff, so such plans take the host loop.
  bool device_loop = device->exec_run != nullptr;
  for (auto& c : copies)
    for (auto& o : p.outputs)
      if (o.slot == std::get<0>(c)) device_loop = false;

  if (device_loop && steps > 0) {
    std::vector<int64_t> sw, cp, ds, hs;
    std::vector<uint64_t> db;
    for (auto& [a, b] : swaps) {
      sw.push_back((int64_t)a);
      sw.push_back((int64_t)b);
    }
    for (auto& [a, b, n] : copies) {
      cp.push_back((int64_t)a);
      cp.push_back((int64_t)b);
      cp.push_back((int64_t)n);
    }
    for (size_t d : spec.data) {
      size_t slot = p.input_slots[d];
      ds.push_back((int64_t)slot);
      db.push_back(p.input_ns[d] * dsize(p.slots[slot].first));
    }
    std::vector<const void*> bp;
    if (batches.size() > 1)
      for (auto& b : batches)
        for (size_t k = 0; k < spec.data.size(); k++) bp.push_back(b[k].data.data());
    for (size_t s : hist_slots) hs.push_back((int64_t)s);
    std::vector<double> hist(hist_slots.size() * steps, 0.0);
    rg_run_desc d{};
    d.n_swaps = (int64_t)swaps.size();
    d.swaps = sw.data();
    d.n_copies = (int64_t)copies.size();
    d.copies = cp.data();
    d.n_data = (int64_t)spec.data.size();
    d.data_slots = ds.data();
    d.data_bytes = db.data();
    d.n_batches = batches.size() > 1 ? (int64_t)batches.size() : 0;
    d.batches = bp.data();
    d.n_history = (int64_t)hist_slots.size();
    d.history_slots = hs.data();
    d.steps = (int64_t)steps;
    d.history = hist.data();
    rg_run_result res{};
    int rc = device->exec_run(e->handle(), &d, &res);
    r.steps = (size_t)res.done;
    r.seconds = res.seconds;
    r.nonfinite_step = res.nonfinite_step;
    for (size_t h = 0; h < hist_slots.size(); h++)
      r.history[h].assign(hist.begin() + (ptrdiff_t)(h * steps), hist.begin() + (ptrdiff_t)(h * steps + r.steps));
    if (rc != 0) {
      auto f = e->failure();
      r.device_error = f ? *f : std::string("device loop failed");
    }
    bool want_outputs = !r.device_error && r.steps > 0 && (r.steps == steps || r.nonfinite_step >= 0);
    if (want_outputs) {
      // After the handoff a swapped slot's pre-handoff value sits in its partner.
      read_outputs([&](size_t s) {
        for (auto& [a, b] : swaps) {
          if (s == b) return a;
          if (s == a) return b;
        }
        return s;
      });
    }
  } else {
    auto started = Clock::now();
    for (size_t k = 0; k < steps; k++) {
      if (batches.size() > 1) load_batch(batches[k % batches.size()]);
      e->step();
      if (auto f = e->failure()) {
        r.device_error = *f;
        break;
      }
      r.steps = k + 1;
      bool bad = false;
      for (size_t h = 0; h < hist_slots.size(); h++) {
        double v = e->scalar(hist_slots[h]);
        bad |= !std::isfinite(v);
        r.history[h].push_back(v);
      }
      if (bad) r.nonfinite_step = (int64_t)k;
      if (k + 1 == steps || bad) read_outputs([](size_t s) { return s; });
      std::vector<std::pair<size_t, Tensor>> temp;
      for (auto& [is, os, n] : copies) temp.push_back({is, e->prefix(os, n, {n})});
      for (auto& [is, os] : swaps) e->swap(is, os);
      for (auto& [is, t] : temp) e->write_prefix(is, t);
      if (bad) break;
    }
    r.seconds = since(started);
  }
  std::vector<std::tuple<size_t, size_t, Shape>> reads;
  for (auto& [i, o] : spec.state) reads.push_back({p.input_slots[i], p.input_ns[i], p.outputs[o].shape});
  r.state = e->prefix_all(reads);
  return r;
}

std::optional<std::tuple<size_t, size_t, std::vector<Tensor>>> Compiled::replay(const RunSpec& spec, const std::vector<Tensor>& state,
                                                                              const std::vector<std::vector<Tensor>>& batches,
                                                                              size_t steps) const {
  std::vector<Tensor> cur = state;
  for (size_t k = 0; k < steps; k++) {
    size_t b = batches.empty() ? 0 : k % batches.size();
    std::vector<std::vector<Tensor>> slice;
    if (!batches.empty()) slice.push_back(batches[b]);
    std::vector<const Tensor*> at;
    for (auto& t : cur) at.push_back(&t);
    RunOut out = run(spec, at, slice, 1);
    if (out.device_error) return std::nullopt;
    bool bad = false;
    for (auto& t : out.state) bad |= !t.is_finite();
    for (auto& t : out.outputs) bad |= !t.is_finite();
    if (bad) return std::make_tuple(k, b, cur);
    cur = std::move(out.state);
  }
  return std::nullopt;
}

namespace {

std::unique_ptr<Compiled> build(const Graph& raw, const std::vector<uint32_t>& outputs, const std::vector<Tensor>& examples,
                                Level level, Backend* device, OptMode mode) {
  auto c = std::make_unique<Compiled>();
  bool on_device = device->name != "cpu";
  Optimized opt = optimize_mode(raw, outputs, on_device, mode);
  c->plan = on_device ? build_fused(opt.g, opt.outputs, Fuse::hip()) : build_fused(opt.g, opt.outputs, Fuse::cpu());
  c->raw = raw;
  c->outputs = outputs;
  c->level = level;
  c->mode = mode;
  c->opt_stats = opt.stats;
  c->device = device;
  try {
    c->program = std::make_unique<DeviceProgram>(device, c->plan);
  } catch (std::exception& e) {
    Json obs = Json::obj();
    obs["device"] = device->name;
    obs["detail"] = e.what();
    throw DiagError{diag("DEVICE_UNAVAILABLE", "error", Json(), obs,
                         "device_memory_limit_or_kernel_compilation_failed", "verified")};
  }
  c->raw_plan = build_plan(c->raw, c->raw_outputs(), false);
  c->check_inputs(examples);
  c->report = c->validate(examples);
  return c;
}

bool has_equivalence_failure(const Json& report) {
  for (auto& d : report.get("diagnostics")->items())
    if (d.get("code") && *d.get("code") == "OPTIMIZER_MISMATCH") return true;
  return false;
}

}  // namespace

std::unique_ptr<Compiled> compile_mode(const Graph& raw, const std::vector<uint32_t>& outputs, const std::vector<Tensor>& examples,
                                       Level level, Backend* device, OptMode mode) {
  if (mode == OptMode::Auto) {
    // optimize="auto": time the standard and the rewritten plan on the examples and keep the faster (validate.rs:437-473).
    auto standard = build(raw, outputs, examples, Level::None, device, OptMode::Standard);
    auto searched = compile_mode(raw, outputs, examples, Level::Basic, device, OptMode::SearchLinear);
    bool rewritten = searched->opt_stats.searched && searched->opt_stats.accepted;
    bool use_search = false;
    Json timing;
    if (rewritten) {
      try {
        standard->try_call(examples);
        searched->try_call(examples);
        std::vector<double> ta, tb;
        auto started = Clock::now();
        for (int round = 0; round < 7; round++) {
          for (int k : {round % 2, 1 - round % 2}) {
            auto t0 = Clock::now();
            (k == 0 ? standard : searched)->try_call(examples);
            (k == 0 ? ta : tb).push_back(since(t0));
          }
          if (since(started) > 0.5) break;
        }
        std::sort(ta.begin(), ta.end());
        std::sort(tb.begin(), tb.end());
        double a = ta[ta.size() / 2], b = tb[tb.size() / 2];
        use_search = a / b >= 1.05;
        timing = Json::obj();
        timing["standard_seconds"] = a;
        timing["rewritten_seconds"] = b;
      } catch (DiagError&) {
      }
    }
    standard.reset();
    searched.reset();
    auto c = compile_mode(raw, outputs, examples, level, device, use_search ? OptMode::SearchLinear : OptMode::Standard);
    Json a = Json::obj();
    a["chosen"] = use_search ? "search-linear" : "standard";
    a["rewrite_proposed"] = rewritten;
    a["timing"] = timing;
    c->report["auto"] = a;
    return c;
  }
  auto c = build(raw, outputs, examples, level, device, mode);
  bool rewritten = c->opt_stats.searched && c->opt_stats.accepted;
  if (rewritten && has_equivalence_failure(c->report)) {
    Json rejected;
    for (auto& d : c->report.get("diagnostics")->items())
      if (d.get("code") && *d.get("code") == "OPTIMIZER_MISMATCH") {
        rejected = d;
        break;
      }
    c = build(raw, outputs, examples, level, device, OptMode::Standard);
    Json note = diag("REWRITE_REJECTED", "warning", *rejected.get("node"), *rejected.get("observation"),
                     "rewritten_program_failed_the_equivalence_check_standard_plan_used", "verified");
    c->report["diagnostics"].push(note);
    if (*c->report.get("status") == "ok") c->report["status"] = "warning";
  }
  return c;
}

}  // namespace rg
