// rg's SSA IR: tensors, operations, nodes and the graph with shape/dtype inference.
// Restates the reference's src/tensor.rs:3-138 (dtypes, tensors) and src/graph.rs:41-522 (IR).
#pragma once
#include <algorithm>
#include <cstdint>
#include <cstring>
#include <memory>
#include <string>
#include <thread>
#include <vector>

#include "../../../include/rg_plan.h"
#include "json.h"

namespace rg {

enum class DType : int32_t { F32 = RG_F32, F64 = RG_F64, I32 = RG_I32 };
inline size_t dsize(DType d) { return d == DType::F64 ? 8 : 4; }
inline const char* dname(DType d) {
  return d == DType::F32 ? "float32" : d == DType::F64 ? "float64" : "int32";
}
bool parse_dtype(const std::string& s, DType* out);

using Shape = std::vector<size_t>;
inline size_t numel(const Shape& s) {
  size_t n = 1;
  for (auto d : s) n *= d;
  return n;
}

// Rust `as` from f64 to i32: truncates toward zero, saturates at the bounds, NaN gives 0
// (the reference's casts, src/plan.rs:1624-1642 and src/tensor.rs:87-93).
inline int32_t sat_i32(double x) {
  if (std::isnan(x)) return 0;
  if (x >= 2147483647.0) return INT32_MAX;
  if (x <= -2147483648.0) return INT32_MIN;
  return (int32_t)x;
}

// A row-major tensor with native-endian storage (src/tensor.rs:95-138).
struct Tensor {
  Shape shape;
  DType dtype = DType::F32;
  std::vector<uint8_t> data;
  size_t n() const { return data.size() / dsize(dtype); }
  double at(size_t i) const {
    switch (dtype) {
      case DType::F32: { float v; memcpy(&v, &data[i * 4], 4); return v; }
      case DType::F64: { double v; memcpy(&v, &data[i * 8], 8); return v; }
      default: { int32_t v; memcpy(&v, &data[i * 4], 4); return v; }
    }
  }
  std::vector<double> to_f64() const {
    std::vector<double> v(n());
    for (size_t i = 0; i < v.size(); i++) v[i] = at(i);
    return v;
  }
  static Tensor from_f64(DType d, const Shape& s, const std::vector<double>& v) {
    Tensor t;
    t.shape = s;
    t.dtype = d;
    t.data.resize(v.size() * dsize(d));
    for (size_t i = 0; i < v.size(); i++) {
      if (d == DType::F32) { float x = (float)v[i]; memcpy(&t.data[i * 4], &x, 4); }
      else if (d == DType::F64) memcpy(&t.data[i * 8], &v[i], 8);
      else { int32_t x = sat_i32(v[i]); memcpy(&t.data[i * 4], &x, 4); }
    }
    return t;
  }
  static Tensor full(DType d, const Shape& s, double x) {
    return from_f64(d, s, std::vector<double>(numel(s), x));
  }
  // Whether every element is finite: a scan of the exponent bits (all ones for inf and NaN), on
  // several threads for large tensors.
  bool is_finite() const {
    if (dtype != DType::F32 && dtype != DType::F64) return true;
    const size_t w = dsize(dtype), count = n();
    auto scan = [&](size_t lo, size_t hi) {
      bool bad = false;
      if (w == 4) {
        for (size_t i = lo; i < hi; i++) {
          uint32_t b;
          memcpy(&b, &data[i * 4], 4);
          bad |= (b & 0x7F800000u) == 0x7F800000u;
        }
      } else {
        for (size_t i = lo; i < hi; i++) {
          uint64_t b;
          memcpy(&b, &data[i * 8], 8);
          bad |= (b & 0x7FF0000000000000ull) == 0x7FF0000000000000ull;
        }
      }
      return !bad;
    };
    const size_t threads = std::min<size_t>(8, std::max<size_t>(1, count >> 20));
    if (threads <= 1) return scan(0, count);
    std::vector<char> ok(threads, 1);
    std::vector<std::thread> pool;
    for (size_t t = 1; t < threads; t++) pool.emplace_back([&, t] { ok[t] = scan(count * t / threads, count * (t + 1) / threads); });
    ok[0] = scan(0, count / threads);
    for (auto& th : pool) th.join();
    return std::all_of(ok.begin(), ok.end(), [](char c) { return c != 0; });
  }
};

enum class RK : int32_t { Sum = RG_REDUCE_SUM, Max = RG_REDUCE_MAX, Min = RG_REDUCE_MIN };

struct Body;

struct Op {
  rg_op kind = RG_OP_INPUT;
  size_t a = 0;  // Input index, Output index, Take/TakeGrad/Concat axis, KeySplit n, ArgTopK k
  bool ta = false, tb = false, keepdims = false, reverse = false;
  RK rk = RK::Sum;
  Shape v, w;  // axes / perm / target shape / starts ; stops / padded shape
  DType dt = DType::F32;  // Cast target, RandUniform/RandNormal dtype, Output dtype
  std::shared_ptr<const Tensor> t;  // Const
  uint32_t placeholder = 0;
  std::vector<std::pair<uint32_t, uint32_t>> rules;  // Custom
  // Control flow (graph.rs:101-107). Scan: `body` maps (carries, x slices, captures) to (carries,
  // ys) over `length` steps, from the last when `reverse`; its node's outputs by index are the
  // final carries, the stacked ys, then the stacked carries as they were before each step.
  // While: `body2` is the condition over (carries, captures), `body` the step; outputs are the
  // final carries, then the iteration count (int32), at most `max_iter`. Cond: input 0 is the
  // predicate and `body` / `body2` the branches over the remaining inputs; outputs are the taken
  // branch's. The node itself has shape [] and each result is an RG_OP_OUTPUT node reading it.
  std::shared_ptr<const Body> body, body2;
  size_t n_carry = 0, n_x = 0, length = 0, max_iter = 0;

  static Op make(rg_op k) {
    Op o;
    o.kind = k;
    return o;
  }
  const char* name() const;
  bool is_unary_elementwise() const;
  bool is_binary_elementwise() const;
  bool is_control_flow() const {
    return kind == RG_OP_SCAN || kind == RG_OP_WHILE || kind == RG_OP_COND;
  }
  bool int_ok() const;
  bool is_nonsmooth() const;
  // The identity of an operation with its attributes, for common-subexpression elimination.
  std::string key() const;
};

struct Node {
  Op op;
  std::vector<uint32_t> inputs;
  Shape shape;
  DType dtype = DType::F32;
  std::shared_ptr<const std::string> source;
  int64_t origin = -1;  // set on gradient nodes: which forward node's rule emitted them
  size_t n() const { return numel(shape); }
};

struct GradRecord {
  uint32_t y, wrt, grad;
};

Shape* broadcast_shapes(const Shape& a, const Shape& b, Shape* out);

class Graph {
 public:
  std::vector<Node> nodes;
  size_t n_inputs = 0;
  std::vector<GradRecord> grads;
  std::vector<Json> notes;
  std::shared_ptr<const std::string> cur_source;
  int64_t cur_origin = -1;

  uint32_t input(const Shape& s, DType d);
  uint32_t placeholder(const Shape& s, DType d);
  uint32_t constant(Tensor t);
  uint32_t scalar(DType d, double x) { return constant(Tensor::full(d, {}, x)); }
  const Shape& shape(uint32_t id) const { return nodes[id].shape; }
  DType dtype(uint32_t id) const { return nodes[id].dtype; }
  // Adds a node after arity, dtype and shape checks; throws DiagError with a structured diagnostic.
  uint32_t add(const Op& op, const std::vector<uint32_t>& inputs);
  std::vector<bool> reachable(const std::vector<uint32_t>& outputs) const;
  // The RG_OP_OUTPUT node reading result `index` of control-flow node `node`.
  uint32_t output(uint32_t node, size_t index, const Shape& shape, DType dtype);
  Graph to_f64() const;
  Json node_json(uint32_t id) const;

 private:
  uint32_t push(Op op, std::vector<uint32_t> inputs, Shape shape, DType dtype);
  Json pending_json(const Op& op) const;
  [[noreturn]] void static_err(const char* code, const Op& op, Json obs, const char* cause) const;
  Shape infer(const Op& op, const std::vector<Shape>& s) const;
  void check_control_flow(const Op& op, const std::vector<uint32_t>& inputs) const;
};

// A traced control-flow body (graph.rs:11-31): its own graph, whose inputs are numbered as the
// control-flow node feeds them, and the nodes it returns. Bodies are shared and immutable; a
// node's identity for common-subexpression elimination includes the body's address.
struct Body {
  Graph graph;
  std::vector<uint32_t> outputs;
  std::vector<uint32_t> inputs;  // node of each graph input, by input index
  static std::shared_ptr<const Body> make(Graph g, std::vector<uint32_t> outputs);
  const Shape& output_shape(size_t k) const { return graph.shape(outputs[k]); }
  DType output_dtype(size_t k) const { return graph.dtype(outputs[k]); }
  const Shape& input_shape(size_t k) const { return graph.shape(inputs[k]); }
  DType input_dtype(size_t k) const { return graph.dtype(inputs[k]); }
};

// Reverse-mode autodiff (src/autodiff.rs:245-326): adds the nodes computing the gradient of y with respect to each of `wrts`.
std::vector<uint32_t> grad(Graph& g, uint32_t y, const std::vector<uint32_t>& wrts);

}  // namespace rg
