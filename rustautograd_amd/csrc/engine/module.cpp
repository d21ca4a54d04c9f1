// Python bindings of the engine: the `_rg` module. Mirrors the reference's src/python.rs:1-303
// (Tensor, Graph, Compiled, compile, available_devices, DiagnosticError), plus
// `register_backend` to load device libraries.
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <chrono>
#include <thread>

#include "validate.h"

namespace py = pybind11;
using namespace rg;

namespace {

PyObject* g_diag_error = nullptr;

[[noreturn]] void raise_diag(const Json& d) { throw DiagError{d}; }

DType dtype_of(const std::string& s) {
  DType d;
  if (!parse_dtype(s, &d)) throw py::value_error("unsupported dtype " + s);
  return d;
}

struct PyTensor {
  Tensor t;
};

PyTensor make_tensor(py::bytes data, const std::vector<size_t>& shape, const std::string& dtype) {
  PyTensor p;
  p.t.dtype = dtype_of(dtype);
  p.t.shape = shape;
  std::string s = data;
  if (s.size() != numel(shape) * dsize(p.t.dtype))
    throw py::value_error(std::to_string(s.size()) + " bytes do not fit shape of " + dname(p.t.dtype));
  p.t.data.assign(s.begin(), s.end());
  return p;
}

template <class T>
T attr(const py::object& attrs, const char* key) {
  if (attrs.is_none() || !py::cast<py::dict>(attrs).contains(key)) throw py::value_error(std::string("missing attribute ") + key);
  try {
    return py::cast<T>(py::cast<py::dict>(attrs)[key]);
  } catch (py::cast_error&) {
    throw py::value_error(std::string("invalid attribute ") + key);
  }
}

Op parse_op(const std::string& name, const py::object& a) {
  static const std::map<std::string, rg_op> simple = {
      {"neg", RG_OP_NEG},   {"exp", RG_OP_EXP},       {"log", RG_OP_LOG},          {"sqrt", RG_OP_SQRT},
      {"sin", RG_OP_SIN},   {"cos", RG_OP_COS},       {"tanh", RG_OP_TANH},        {"abs", RG_OP_ABS},
      {"sign", RG_OP_SIGN}, {"add", RG_OP_ADD},       {"sub", RG_OP_SUB},          {"mul", RG_OP_MUL},
      {"div", RG_OP_DIV},   {"pow", RG_OP_POW},       {"maximum", RG_OP_MAX},      {"minimum", RG_OP_MIN},
      {"gt", RG_OP_GT},     {"ge", RG_OP_GE},         {"where", RG_OP_WHERE},      {"matmul", RG_OP_MATMUL},
      {"floor", RG_OP_FLOOR}, {"stop_gradient", RG_OP_STOP_GRADIENT}, {"take_along", RG_OP_TAKE_ALONG},
      {"argmax", RG_OP_ARGMAX}};
  auto it = simple.find(name);
  if (it != simple.end()) return Op::make(it->second);
  Op o;
  if (name == "sum" || name == "max" || name == "min") {
    o.kind = RG_OP_REDUCE;
    o.rk = name == "sum" ? RK::Sum : name == "max" ? RK::Max : RK::Min;
    o.v = attr<Shape>(a, "axes");
    o.keepdims = attr<bool>(a, "keepdims");
  } else if (name == "reshape") {
    o.kind = RG_OP_RESHAPE;
    o.v = attr<Shape>(a, "shape");
  } else if (name == "transpose") {
    o.kind = RG_OP_TRANSPOSE;
    o.v = attr<Shape>(a, "perm");
  } else if (name == "broadcast_to") {
    o.kind = RG_OP_BROADCAST_TO;
    o.v = attr<Shape>(a, "shape");
  } else if (name == "slice") {
    o.kind = RG_OP_SLICE;
    o.v = attr<Shape>(a, "starts");
    o.w = attr<Shape>(a, "stops");
  } else if (name == "pad") {
    o.kind = RG_OP_PAD;
    o.v = attr<Shape>(a, "starts");
    o.w = attr<Shape>(a, "shape");
  } else if (name == "cast") {
    o.kind = RG_OP_CAST;
    o.dt = dtype_of(attr<std::string>(a, "dtype"));
  } else if (name == "take") {
    o.kind = RG_OP_TAKE;
    o.a = attr<size_t>(a, "axis");
  } else if (name == "concat") {
    o.kind = RG_OP_CONCAT;
    o.a = attr<size_t>(a, "axis");
  } else if (name == "arg_top_k") {
    o.kind = RG_OP_ARG_TOP_K;
    o.a = attr<size_t>(a, "k");
  } else if (name == "cumsum") {
    o.kind = RG_OP_CUMSUM;
    o.reverse = attr<bool>(a, "reverse");
  } else if (name == "random_uniform" || name == "random_normal") {
    o.kind = name == "random_uniform" ? RG_OP_RAND_UNIFORM : RG_OP_RAND_NORMAL;
    o.v = attr<Shape>(a, "shape");
    o.dt = dtype_of(attr<std::string>(a, "dtype"));
  } else if (name == "key_split") {
    o.kind = RG_OP_KEY_SPLIT;
    o.a = attr<size_t>(a, "n");
  } else if (name == "take_grad") {
    o.kind = RG_OP_TAKE_GRAD;
    o.a = attr<size_t>(a, "axis");
    o.v = attr<Shape>(a, "shape");
  } else if (name == "take_along_grad") {
    o.kind = RG_OP_TAKE_ALONG_GRAD;
    o.v = attr<Shape>(a, "shape");
  } else {
    throw py::value_error("unknown op " + name);
  }
  return o;
}

struct PyGraph {
  Graph g;
  void set_source(const std::optional<std::string>& s) {
    g.cur_source = s ? std::make_shared<const std::string>(*s) : nullptr;
  }
};

struct PyCompiled {
  std::unique_ptr<Compiled> c;
};

std::vector<Tensor> tensors(const std::vector<PyTensor>& v) {
  std::vector<Tensor> out;
  for (auto& p : v) out.push_back(p.t);
  return out;
}

std::vector<PyTensor> wrap(std::vector<Tensor> v) {
  std::vector<PyTensor> out;
  for (auto& t : v) out.push_back(PyTensor{std::move(t)});
  return out;
}

}  // namespace

PYBIND11_MODULE(_rg, m) {
  g_diag_error = PyErr_NewException("rustautograd_amd._rg.DiagnosticError", PyExc_Exception, nullptr);
  m.add_object("DiagnosticError", py::handle(g_diag_error));
  py::register_exception_translator([](std::exception_ptr p) {
    try {
      if (p) std::rethrow_exception(p);
    } catch (const DiagError& d) {
      std::string text = d.d.dump();
      py::gil_scoped_acquire gil;
      py::object err = py::reinterpret_steal<py::object>(PyObject_CallFunction(g_diag_error, "s", text.c_str()));
      try {
        err.attr("diagnostic") = py::module_::import("json").attr("loads")(text);
      } catch (...) {
      }
      PyErr_SetObject(g_diag_error, err.ptr());
    }
  });

  py::class_<PyTensor>(m, "Tensor")
      .def(py::init(&make_tensor), py::arg("data"), py::arg("shape"), py::arg("dtype"))
      .def_property_readonly("shape", [](const PyTensor& t) { return t.t.shape; })
      .def_property_readonly("dtype", [](const PyTensor& t) { return std::string(dname(t.t.dtype)); })
      .def("is_finite", [](const PyTensor& t) { return t.t.is_finite(); })
      .def("tobytes", [](const PyTensor& t) { return py::bytes((const char*)t.t.data.data(), t.t.data.size()); });

  py::class_<PyGraph>(m, "Graph")
      .def(py::init<>())
      .def("input",
           [](PyGraph& g, const std::vector<size_t>& shape, const std::string& dtype, std::optional<std::string> source) {
             g.set_source(source);
             return g.g.input(shape, dtype_of(dtype));
           },
           py::arg("shape"), py::arg("dtype"), py::arg("source") = py::none())
      .def("constant",
           [](PyGraph& g, const PyTensor& t, std::optional<std::string> source) {
             g.set_source(source);
             return g.g.constant(t.t);
           },
           py::arg("t"), py::arg("source") = py::none())
      .def("op",
           [](PyGraph& g, const std::string& name, const std::vector<uint32_t>& inputs, py::object attrs,
              std::optional<std::string> source) {
             Op op = parse_op(name, attrs);
             g.set_source(source);
             return g.g.add(op, inputs);
           },
           py::arg("name"), py::arg("inputs"), py::arg("attrs") = py::none(), py::arg("source") = py::none())
      .def("grad",
           [](PyGraph& g, uint32_t y, const std::vector<uint32_t>& wrts, std::optional<std::string> source) {
             g.set_source(source);
             return grad(g.g, y, wrts);
           },
           py::arg("y"), py::arg("wrts"), py::arg("source") = py::none())
      // Control flow (python.rs:158-180): each body is a graph of its own, traced with inputs in
      // the order the node feeds them; a body's graph is copied into the node.
      .def("scan",
           [](PyGraph& g, const PyGraph& body, const std::vector<uint32_t>& body_outputs, size_t n_carry, size_t n_x, size_t length,
              const std::vector<uint32_t>& inputs, bool reverse, std::optional<std::string> source) {
             Op op = Op::make(RG_OP_SCAN);
             op.body = Body::make(body.g, body_outputs);
             op.n_carry = n_carry;
             op.n_x = n_x;
             op.length = length;
             op.reverse = reverse;
             g.set_source(source);
             return g.g.add(op, inputs);
           },
           py::arg("body"), py::arg("body_outputs"), py::arg("n_carry"), py::arg("n_x"), py::arg("length"), py::arg("inputs"),
           py::arg("reverse") = false, py::arg("source") = py::none())
      .def("while_loop",
           [](PyGraph& g, const PyGraph& cond, uint32_t cond_output, const PyGraph& body, const std::vector<uint32_t>& body_outputs,
              size_t n_carry, size_t max_iterations, const std::vector<uint32_t>& inputs, std::optional<std::string> source) {
             Op op = Op::make(RG_OP_WHILE);
             op.body2 = Body::make(cond.g, {cond_output});
             op.body = Body::make(body.g, body_outputs);
             op.n_carry = n_carry;
             op.max_iter = max_iterations;
             g.set_source(source);
             return g.g.add(op, inputs);
           },
           py::arg("cond"), py::arg("cond_output"), py::arg("body"), py::arg("body_outputs"), py::arg("n_carry"),
           py::arg("max_iterations"), py::arg("inputs"), py::arg("source") = py::none())
      .def("cond",
           [](PyGraph& g, const PyGraph& then_body, const std::vector<uint32_t>& then_outputs, const PyGraph& else_body,
              const std::vector<uint32_t>& else_outputs, const std::vector<uint32_t>& inputs, std::optional<std::string> source) {
             Op op = Op::make(RG_OP_COND);
             op.body = Body::make(then_body.g, then_outputs);
             op.body2 = Body::make(else_body.g, else_outputs);
             g.set_source(source);
             return g.g.add(op, inputs);
           },
           py::arg("then_body"), py::arg("then_outputs"), py::arg("else_body"), py::arg("else_outputs"), py::arg("inputs"),
           py::arg("source") = py::none())
      .def("output",
           [](PyGraph& g, uint32_t node, size_t index, const std::vector<size_t>& shape, const std::string& dtype,
              std::optional<std::string> source) {
             g.set_source(source);
             return g.g.output(node, index, shape, dtype_of(dtype));
           },
           py::arg("node"), py::arg("index"), py::arg("shape"), py::arg("dtype"), py::arg("source") = py::none())
      .def_property_readonly("n_inputs", [](const PyGraph& g) { return g.g.n_inputs; })
      .def("placeholder",
           [](PyGraph& g, const std::vector<size_t>& shape, const std::string& dtype) {
             return g.g.placeholder(shape, dtype_of(dtype));
           })
      .def("custom",
           [](PyGraph& g, uint32_t y, uint32_t placeholder, const std::vector<std::pair<uint32_t, uint32_t>>& rules,
              std::optional<std::string> source) {
             g.set_source(source);
             Op o = Op::make(RG_OP_CUSTOM);
             o.placeholder = placeholder;
             o.rules = rules;
             return g.g.add(o, {y});
           },
           py::arg("y"), py::arg("placeholder"), py::arg("rules"), py::arg("source") = py::none())
      .def("grad_records",
           [](const PyGraph& g) {
             std::vector<std::tuple<uint32_t, uint32_t, uint32_t>> out;
             for (auto& r : g.g.grads) out.push_back({r.y, r.wrt, r.grad});
             return out;
           })
      .def("shape", [](const PyGraph& g, uint32_t id) { return g.g.shape(id); })
      .def("dtype", [](const PyGraph& g, uint32_t id) { return std::string(dname(g.g.dtype(id))); })
      .def("__len__", [](const PyGraph& g) { return g.g.nodes.size(); })
      .def("eval", [](const PyGraph& g, const std::vector<uint32_t>& ids) {
        // Eager mode: a constant-only graph evaluated once on the eager backend.
        Backend* b = eager_backend();
        std::vector<Tensor> out;
        {
          py::gil_scoped_release nogil;
          out = eval_on(b, g.g, ids, {});
        }
        return wrap(std::move(out));
      });

  py::class_<PyCompiled>(m, "Compiled")
      .def_property_readonly("report_json", [](const PyCompiled& c) { return c.c->report.dump(); })
      .def_property_readonly("output_shapes",
                             [](const PyCompiled& c) {
                               std::vector<Shape> s;
                               for (auto& o : c.c->plan.outputs) s.push_back(o.shape);
                               return s;
                             })
      .def_property_readonly("device", [](const PyCompiled& c) { return c.c->device->name; })
      .def("plan_summary",
           [](const PyCompiled& c) {
             // Per-step description for measurement tools: kind, op, dtype, n, shapes.
             py::list out;
             const StreamedFn streamed = c.c->streamed_products();
             for (auto& s : c.c->plan.steps) {
               py::dict d;
               // Algorithmic work: flops priced against the matrix-core peak ("mfma"), or bytes
               // against HBM bandwidth ("hbm").
               const StepWork w = step_work(s, streamed);
               d["flops"] = w.flops;
               d["executed_flops"] = w.executed_flops;
               d["bytes"] = w.bytes;
               d["bound"] = w.compute ? "mfma" : "hbm";
               if (s.attn) {
                 const Attn& a = s.att;
                 d["kind"] = "attention";
                 d["backward"] = a.backward;
                 d["dtype"] = dname(a.dtype);
                 d["bh"] = a.shape.bh;
                 d["heads"] = a.shape.heads;
                 d["tq"] = a.shape.tq;
                 d["tk"] = a.shape.tk;
                 d["hd"] = a.shape.hd;
                 d["masked"] = a.mask_slot >= 0;
                 d["mask_bits_slot"] = a.mask_bits_slot;
                 d["builds_mask_bits"] = a.build_mask_bits;
                 d["n"] = a.shape.bh * a.shape.tq * a.shape.hd;
                 py::list ins, outs;
                 for (auto& v : a.in) ins.append(v.slot);
                 for (auto& v : a.out) outs.append(v.slot);
                 d["input_slots"] = ins;
                 d["output_slots"] = outs;
               } else if (s.fused) {
                 d["kind"] = "fused";
                 py::list ops;
                 for (auto& m : s.group.ops) ops.append(m.op.name());
                 d["ops"] = ops;
                 d["n"] = s.group.n;
                 d["dtype"] = dname(s.group.dtype);
                 d["inputs"] = s.group.input_shapes;
                 d["n_outputs"] = s.group.outputs.size();
                 d["row_len"] = s.group.row_len;  // > 0: a row group
                 size_t cols = 0;  // reductions over the rows (every axis but the last)
                 for (auto& m : s.group.ops)
                   cols += m.op.kind == RG_OP_REDUCE && std::find(m.op.v.begin(), m.op.v.end(), (int64_t)s.group.shape.size() - 1) == m.op.v.end();
                 d["column_reductions"] = cols;
                 static const char* kinds[] = {"full", "splat", "row", "broadcast"};
                 py::list in_kinds, in_slots, out_slots;
                 for (auto& in : s.group.inputs) {
                   in_kinds.append(kinds[in.kind]);
                   in_slots.append(in.slot);
                 }
                 for (auto& o : s.group.outputs) out_slots.append(o.second);
                 d["input_kinds"] = in_kinds;
                 d["input_slots"] = in_slots;
                 d["output_slots"] = out_slots;
               } else {
                 d["kind"] = "instr";
                 d["op"] = s.instr.op.name();
                 d["ta"] = s.instr.op.ta;
                 d["tb"] = s.instr.op.tb;
                 d["n"] = s.instr.n;
                 d["dtype"] = dname(s.instr.dtype);
                 d["shape"] = s.instr.shape;
                 d["arg_shapes"] = s.instr.arg_shapes;
                 d["dst"] = s.instr.dst;
                 d["args"] = s.instr.args;
               }
               out.append(d);
             }
             return out;
           })
      .def("plan_io",
           [](const PyCompiled& c) {
             // Slots of the plan's inputs and outputs, and every slot's (dtype, capacity, pinned).
             const Plan& p = c.c->plan;
             std::vector<size_t> outs;
             for (auto& o : p.outputs) outs.push_back(o.slot);
             std::vector<std::tuple<std::string, size_t, bool>> slots;
             for (size_t k = 0; k < p.slots.size(); k++) slots.push_back({dname(p.slots[k].first), p.slots[k].second, (bool)p.pinned[k]});
             return py::make_tuple(p.input_slots, outs, slots);
           })
      .def("step_times",
           [](const PyCompiled& c, const std::vector<PyTensor>& inputs, size_t repeats) {
             // Device seconds of each plan step, summed over `repeats` runs (metal.rs:690-698).
             auto in = tensors(inputs);
             c.c->check_inputs(in);
             std::vector<double> seconds(c.c->plan.steps.size(), 0.0);
             py::gil_scoped_release nogil;
             auto e = c.c->program->exec();
             for (size_t k = 0; k < in.size(); k++) e->load(k, in[k]);
             Backend* b = c.c->device;
             for (size_t r = 0; r < repeats; r++) {
               if (b->exec_step_timed) {
                 b->exec_step_timed(e->handle(), seconds.data());
               } else {
                 for (size_t s = 0; s < seconds.size(); s++) {
                   auto t0 = std::chrono::steady_clock::now();
                   e->steps(s, s + 1);
                   seconds[s] += std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
                 }
               }
             }
             if (auto f = e->failure()) raise_diag(device_failure(b->name, *f));
             return seconds;
           })
      .def("time_steps",
           [](const PyCompiled& c, const std::vector<PyTensor>& inputs, const std::vector<int64_t>& steps, size_t repeats) {
             // Device seconds of `repeats` back-to-back passes over the listed plan steps, after
             // one full step has filled every slot (rg_hip_exec_time_steps).
             Backend* b = c.c->device;
             if (!b->exec_time_steps) throw py::value_error("device " + b->name + " has no exec_time_steps");
             auto in = tensors(inputs);
             c.c->check_inputs(in);
             double seconds = 0.0;
             {
               py::gil_scoped_release nogil;
               auto e = c.c->program->exec();
               for (size_t k = 0; k < in.size(); k++) e->load(k, in[k]);
               e->steps(0, c.c->plan.steps.size());
               b->exec_time_steps(e->handle(), steps.data(), (int64_t)steps.size(), (int64_t)repeats, &seconds);
               if (auto f = e->failure()) raise_diag(device_failure(b->name, *f));
             }
             return seconds;
           })
      .def("call",
           [](const PyCompiled& c, const std::vector<PyTensor>& inputs) {
             auto in = tensors(inputs);
             c.c->check_inputs(in);
             std::vector<Tensor> out;
             {
               py::gil_scoped_release nogil;
               out = c.c->try_call(in);
             }
             return wrap(std::move(out));
           })
      .def("check",
           [](PyCompiled& c, const std::vector<PyTensor>& inputs) {
             auto in = tensors(inputs);
             c.c->check_inputs(in);
             py::gil_scoped_release nogil;
             return c.c->check(in).dump();
           })
      .def("profile",
           [](const PyCompiled& c, const std::vector<PyTensor>& inputs, size_t repeats) {
             auto in = tensors(inputs);
             c.c->check_inputs(in);
             py::gil_scoped_release nogil;
             return c.c->profile(in, repeats).dump();
           })
      .def("allocated_bytes", [](const PyCompiled& c) { return c.c->program->allocated_bytes(); })
      // Per plan step, the step whose kernel computes it (a product running a fused group in its
      // epilogue computes both; other steps compute themselves).
      .def("step_runs_in",
           [](const PyCompiled& c) {
             std::vector<int64_t> at;
             for (size_t k = 0; k < c.c->plan.steps.size(); k++) at.push_back(c.c->program->step_runs_in((int64_t)k));
             return at;
           })
      .def("inject_failure", [](const PyCompiled& c, int64_t after) { c.c->program->inject_failure(after); }, py::arg("after") = 0)
      .def("run",
           // The state arrives as pointers to the Python objects' tensors: a list of PyTensor by
           // value would be copied twice (tens of MB for a model's parameters and moments).
           [](const PyCompiled& c, const std::vector<std::pair<size_t, size_t>>& state_map, const std::vector<size_t>& data_inputs,
              const std::vector<size_t>& history, const std::vector<const PyTensor*>& state,
              const std::vector<std::vector<PyTensor>>& batches, size_t steps, bool skip_state_outputs) {
             RunSpec spec{state_map, data_inputs, history, skip_state_outputs};
             c.c->validate_spec(spec);
             std::vector<const Tensor*> st;
             for (const PyTensor* p : state) {
               if (!p) throw py::value_error("run: a state entry is None");
               st.push_back(&p->t);
             }
             std::vector<std::vector<Tensor>> bs;
             for (auto& b : batches) bs.push_back(tensors(b));
             RunOut out;
             {
               py::gil_scoped_release nogil;
               out = c.c->run(spec, st, bs, steps);
             }
             if (out.device_error) {
               Json d = device_failure(c.c->device->name, *out.device_error);
               d["observation"]["completed_steps"] = out.steps;
               raise_diag(d);
             }
             std::optional<size_t> bad;
             if (out.nonfinite_step >= 0) bad = (size_t)out.nonfinite_step;
             return py::make_tuple(wrap(out.state), wrap(out.outputs), out.history, out.steps, bad, out.seconds);
           },
           py::arg("state_map"), py::arg("data_inputs"), py::arg("history"), py::arg("state"), py::arg("batches"), py::arg("steps"),
           py::arg("skip_state_outputs") = false)
      .def("replay",
           [](const PyCompiled& c, const std::vector<std::pair<size_t, size_t>>& state_map, const std::vector<size_t>& data_inputs,
              const std::vector<size_t>& history, const std::vector<PyTensor>& state,
              const std::vector<std::vector<PyTensor>>& batches, size_t steps) -> py::object {
             RunSpec spec{state_map, data_inputs, history};
             auto st = tensors(state);
             std::vector<std::vector<Tensor>> bs;
             for (auto& b : batches) bs.push_back(tensors(b));
             std::optional<std::tuple<size_t, size_t, std::vector<Tensor>>> found;
             {
               py::gil_scoped_release nogil;
               found = c.c->replay(spec, st, bs, steps);
             }
             if (!found) return py::none();
             return py::make_tuple(std::get<0>(*found), std::get<1>(*found), wrap(std::get<2>(*found)));
           });

  m.def("compile", [](const PyGraph& graph, const std::vector<uint32_t>& outputs, const std::vector<PyTensor>& examples,
                      const std::string& level, const std::string& device, const std::string& optimize) {
    OptMode mode;
    if (!parse_opt_mode(optimize, &mode)) throw py::value_error("unknown optimize mode " + optimize);
    Backend* b = find_backend(device);
    if (!b) {
      Json obs = Json::obj();
      obs["device"] = device;
      obs["available"] = Json(available_backends());
      raise_diag(diag("DEVICE_UNAVAILABLE", "error", Json(), obs, "unknown_device", "verified"));
    }
    Level lv;
    if (!parse_level(level, &lv)) throw py::value_error("unknown validation level " + level);
    auto ex = tensors(examples);
    PyCompiled pc;
    {
      py::gil_scoped_release nogil;
      pc.c = compile_mode(graph.g, outputs, ex, lv, b, mode);
    }
    return pc;
  });
  m.def("available_devices", []() { return available_backends(); });
  // Whether every element of every tensor is finite, the tensors scanned on several threads (a
  // run's returned state: one scan per run instead of one per tensor).
  m.def("all_finite", [](const std::vector<const PyTensor*>& ts) {
    std::vector<const Tensor*> v;
    for (const PyTensor* p : ts)
      if (p) v.push_back(&p->t);
    py::gil_scoped_release nogil;
    const size_t threads = std::min<size_t>(8, std::max<size_t>(1, v.size()));
    std::vector<char> ok(threads, 1);
    std::vector<std::thread> pool;
    for (size_t t = 0; t < threads; t++)
      pool.emplace_back([&, t] {
        for (size_t k = t; k < v.size(); k += threads)
          if (!v[k]->is_finite()) ok[t] = 0;
      });
    for (auto& th : pool) th.join();
    return std::all_of(ok.begin(), ok.end(), [](char c) { return c != 0; });
  });
  m.def("plan_words", [](const PyGraph& graph, const std::vector<uint32_t>& outputs, const std::string& flavor, const std::string& optimize) {
    // The serialized plan a device would receive (include/rg_plan.h), without needing the device.
    OptMode mode;
    if (!parse_opt_mode(optimize, &mode)) throw py::value_error("unknown optimize mode " + optimize);
    bool dev = flavor != "cpu";
    Optimized opt = optimize_mode(graph.g, outputs, dev, mode);
    Plan plan = build_fused(opt.g, opt.outputs, dev ? Fuse::hip() : Fuse::cpu());
    std::vector<int64_t> words;
    std::vector<uint8_t> blob;
    plan.serialize(&words, &blob);
    return py::make_tuple(words, py::bytes((const char*)blob.data(), blob.size()));
  });
  m.def("matrix_search_products",
        [](const PyGraph& graph, const std::vector<uint32_t>& outputs, bool device) -> py::object {
          // The products (M, K, N) of the form the matrix search extracts, or None when it keeps
          // the traced form (egraph.rs:405-426). Test hook: compile applies its own acceptance.
          SearchStats st;
          auto found = matrix_search(graph.g, outputs, device ? CostModel::Device : CostModel::Cpu, OptMode::SearchLinear, &st);
          if (!found) return py::none();
          const Graph& h = found->first;
          std::vector<bool> keep = h.reachable(found->second);
          py::list out;
          for (size_t i = 0; i < h.nodes.size(); i++) {
            const Node& n = h.nodes[i];
            if (!keep[i] || n.op.kind != RG_OP_MATMUL) continue;
            const Shape& a = h.shape(n.inputs[0]);
            const Shape& b = h.shape(n.inputs[1]);
            out.append(py::make_tuple(a[0], a[1], b[1]));
          }
          return std::move(out);
        });
  m.def("register_backend", [](const std::string& name, const std::string& path, const std::string& prefix) {
    try {
      register_backend(name, path, prefix);
    } catch (std::runtime_error& e) {
      throw py::import_error(e.what());
    }
  });
}
