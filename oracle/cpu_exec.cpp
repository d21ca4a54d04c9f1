// ORACLE — test infrastructure, not product code.
//
// A CPU restatement of rg's plan interpreter: the kernels of the reference's src/plan.rs
// (run_fused/run_block 892-970, binary/unary 1043-1141, structural 1289-1383, RNG 1391-1435,
// argmax 1437-1451, matmul 1453-1493, numeric 1495-1547, reduce 1549-1622, cast 1624-1642,
// arg_top_k 833-863, cumsum 865-885) over the Linux branch of src/tensor.rs (per-element libm
// calls 215-227, the naive i-p-j gemm 238-251). It executes the flat plan descriptor of
// include/rg_plan.h behind the same C ABI as the HIP backend, with the prefix `rg_cpu_`.
//
// Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load this library, as the
// parity checker and the CPU baseline. Build: oracle/build.sh (gcc, -ffp-contract=off, no fast
// math, so every float operation rounds exactly as the reference's does).
#include <omp.h>

#include <algorithm>
#include <array>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <numeric>
#include <string>
#include <vector>

#include "../include/rg_plan.h"

using namespace rgplan;

namespace {

constexpr size_t BLOCK = 256;               // plan.rs:7
constexpr size_t TASK = 16 * BLOCK;         // plan.rs:10
constexpr size_t PARALLEL_RANDOM = 1 << 15; // plan.rs:1393
constexpr size_t PARALLEL_COPY = 1 << 19;
constexpr size_t PARALLEL_SUM = 1 << 20;
constexpr size_t PARALLEL_MINMAX = 1 << 16;
constexpr size_t REDUCE_ROWS = 64;
constexpr size_t PARALLEL_FLOPS = 2000000;
// Row-parallel 2-D products (rg_cpu_set_row_parallel_gemm); the reference runs them serially.
bool g_row_parallel_gemm = false;
constexpr uint64_t GAMMA = 0x9E3779B97F4A7C15ull;
constexpr uint64_t GAMMA_SPLIT = 0xD1B54A32D192ED03ull;

using Sh = std::vector<int64_t>;
size_t prod(const Sh& s) {
  size_t n = 1;
  for (auto d : s) n *= (size_t)d;
  return n;
}

// Row-major strides (plan.rs:1155-1162).
std::vector<size_t> strides(const Sh& shape) {
  std::vector<size_t> out(shape.size(), 1);
  for (size_t i = shape.size(); i-- > 1;) out[i - 1] = out[i] * (size_t)shape[i];
  return out;
}

// Element strides of `shape` laid out against `rank` output dims from the right; a broadcast dim gets stride 0 (plan.rs:1164-1169).
std::vector<size_t> bstrides(const Sh& shape, size_t rank) {
  auto st = strides(shape);
  size_t lead = rank - shape.size();
  std::vector<size_t> out(rank, 0);
  for (size_t i = 0; i < rank; i++)
    out[i] = (i < lead || shape[i - lead] == 1) ? 0 : st[i - lead];
  return out;
}

// Walks every index of `shape` in row-major order, carrying one flat offset per operand (plan.rs:1171-1192).
template <size_t N, class F>
void walk(const Sh& shape, const std::vector<size_t>* st, F f) {
  size_t total = prod(shape);
  std::vector<size_t> idx(shape.size(), 0);
  size_t off[N] = {0};
  for (size_t t = 0; t < total; t++) {
    f(off);
    for (size_t d = shape.size(); d-- > 0;) {
      idx[d]++;
      for (size_t k = 0; k < N; k++) off[k] += st[k][d];
      if (idx[d] < (size_t)shape[d]) break;
      for (size_t k = 0; k < N; k++) off[k] -= st[k][d] * (size_t)shape[d];
      idx[d] = 0;
    }
  }
}

// (outer dims, row length) as split_rows (plan.rs:1146-1153).
void split_rows(const Sh& shape, Sh* outer, size_t* len) {
  if (shape.empty()) {
    *outer = shape;
    *len = 1;
  } else {
    *outer = Sh(shape.begin(), shape.end() - 1);
    *len = (size_t)shape.back();
  }
}

uint64_t mix(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

size_t clamp_index(int32_t ix, size_t dim) { return std::min((size_t)std::max(ix, 0), dim - 1); }

template <class T> T t_exp(T x);
template <> float t_exp(float x) { return expf(x); }
template <> double t_exp(double x) { return exp(x); }
template <class T> T t_log(T x);
template <> float t_log(float x) { return logf(x); }
template <> double t_log(double x) { return log(x); }
template <class T> T t_sin(T x);
template <> float t_sin(float x) { return sinf(x); }
template <> double t_sin(double x) { return sin(x); }
template <class T> T t_cos(T x);
template <> float t_cos(float x) { return cosf(x); }
template <> double t_cos(double x) { return cos(x); }
template <class T> T t_tanh(T x);
template <> float t_tanh(float x) { return tanhf(x); }
template <> double t_tanh(double x) { return tanh(x); }
template <class T> T t_pow(T x, T y);
template <> float t_pow(float x, float y) { return powf(x, y); }
template <> double t_pow(double x, double y) { return pow(x, y); }
template <class T> T t_sqrt(T x) { return std::sqrt(x); }
template <class T> T t_floor(T x) { return std::floor(x); }

template <class T> T nan_max(T a, T b) { return a > b ? a : (b >= a ? b : (T)NAN); }
template <class T> T nan_min(T a, T b) { return a < b ? a : (b <= a ? b : (T)NAN); }
template <class T> T sign(T x) { return x > 0 ? (T)1 : (x < 0 ? (T)-1 : x); }

template <class T>
T unary_op(int op, T x) {
  switch (op) {
    case RG_OP_NEG: return -x;
    case RG_OP_EXP: return t_exp(x);
    case RG_OP_LOG: return t_log(x);
    case RG_OP_SQRT: return t_sqrt(x);
    case RG_OP_SIN: return t_sin(x);
    case RG_OP_COS: return t_cos(x);
    case RG_OP_TANH: return t_tanh(x);
    case RG_OP_ABS: return std::fabs(x);
    case RG_OP_SIGN: return sign(x);
    case RG_OP_FLOOR: return t_floor(x);
  }
  return x;
}

template <class T>
T binary_op(int op, T a, T b) {
  switch (op) {
    case RG_OP_ADD: return a + b;
    case RG_OP_SUB: return a - b;
    case RG_OP_MUL: return a * b;
    case RG_OP_DIV: return a / b;
    case RG_OP_POW: return t_pow(a, b);
    case RG_OP_MAX: return nan_max(a, b);
    case RG_OP_MIN: return nan_min(a, b);
    case RG_OP_GT: return a > b ? (T)1 : (T)0;
    case RG_OP_GE: return a >= b ? (T)1 : (T)0;
  }
  return a;
}

int32_t int_op(int op, int32_t a, int32_t b) {
  switch (op) {
    case RG_OP_ADD: return (int32_t)((uint32_t)a + (uint32_t)b);
    case RG_OP_SUB: return (int32_t)((uint32_t)a - (uint32_t)b);
    case RG_OP_MUL: return (int32_t)((uint32_t)a * (uint32_t)b);
    case RG_OP_GT: return a > b;
    case RG_OP_GE: return a >= b;
  }
  return a;
}

bool is_unary(int op) {
  switch (op) {
    case RG_OP_NEG: case RG_OP_EXP: case RG_OP_LOG: case RG_OP_SQRT: case RG_OP_SIN: case RG_OP_COS:
    case RG_OP_TANH: case RG_OP_ABS: case RG_OP_SIGN: case RG_OP_FLOOR:
      return true;
  }
  return false;
}

bool is_binary(int op) {
  switch (op) {
    case RG_OP_ADD: case RG_OP_SUB: case RG_OP_MUL: case RG_OP_DIV: case RG_OP_POW: case RG_OP_MAX:
    case RG_OP_MIN: case RG_OP_GT: case RG_OP_GE:
      return true;
  }
  return false;
}

struct Buf {
  std::vector<uint8_t> bytes;
  template <class T> T* as() { return reinterpret_cast<T*>(bytes.data()); }
};

// Lane-wise accumulation: 8 lanes, lanes added in order, then the tail (plan.rs:1212-1230).
template <class T>
T fast_sum(const T* a, size_t n) {
  T acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  size_t full = n / 8 * 8;
  for (size_t i = 0; i < full; i += 8)
    for (size_t k = 0; k < 8; k++) acc[k] = acc[k] + a[i + k];
  T out = 0;
  for (size_t k = 0; k < 8; k++) out = out + acc[k];
  for (size_t i = full; i < n; i++) out = out + a[i];
  return out;
}

// tensor.rs:238-251: C (m x n) = A (m x k) times B (k x n), row-major, looping i, then p, then j, each term rounded on its own (no FMA).
template <class T>
void gemm(size_t m, size_t k, size_t n, const T* a, bool ta, const T* b, bool tb, T* out) {
  std::fill(out, out + m * n, (T)0);
  for (size_t i = 0; i < m; i++) {
    T* row = out + i * n;
    for (size_t p = 0; p < k; p++) {
      T x = ta ? a[p * m + i] : a[i * k + p];
      if (tb) {
        for (size_t j = 0; j < n; j++) row[j] = row[j] + x * b[j * k + p];
      } else {
        const T* bp = b + p * n;
        for (size_t j = 0; j < n; j++) row[j] = row[j] + x * bp[j];
      }
    }
  }
}

// Checker-only form of `gemm` (row-parallel mode): rows [r0, r1) of the product, with the
// right operand given as a contiguous k x n panel. Columns are taken 256 at a time and, for
// each p, every row of the block adds its term, so a B row segment is loaded once per block of
// rows; each output element still receives its terms in increasing p, one rounding per add
// and per multiply, exactly as `gemm` does: the results are bit-identical.
template <class T>
void gemm_rows_blocked(size_t m, size_t k, size_t n, const T* a, bool ta, const T* bk, T* out, size_t r0, size_t r1) {
  constexpr size_t JB = 256;
  for (size_t i = r0; i < r1; i++) std::fill(out + i * n, out + i * n + n, (T)0);
  for (size_t j0 = 0; j0 < n; j0 += JB) {
    size_t j1 = std::min(n, j0 + JB);
    for (size_t p = 0; p < k; p++) {
      const T* bp = bk + p * n;
      for (size_t i = r0; i < r1; i++) {
        T x = ta ? a[p * m + i] : a[i * k + p];
        T* row = out + i * n;
        for (size_t j = j0; j < j1; j++) row[j] = row[j] + x * bp[j];
      }
    }
  }
}

// The whole product on every thread, row blocks of 32 (checker-only; see gemm_rows_blocked).
template <class T>
void gemm_checker(size_t m, size_t k, size_t n, const T* a, bool ta, const T* b, bool tb, T* out) {
  std::vector<T> panel;
  const T* bk = b;
  if (tb) {
    panel.resize(k * n);
    for (size_t j = 0; j < n; j++)
      for (size_t p = 0; p < k; p++) panel[p * n + j] = b[j * k + p];
    bk = panel.data();
  }
  size_t blocks = (m + 31) / 32;
#pragma omp parallel for schedule(dynamic)
  for (size_t q = 0; q < blocks; q++) gemm_rows_blocked<T>(m, k, n, a, ta, bk, out, q * 32, std::min(m, q * 32 + 32));
}

struct Program;

struct Frame {
  std::vector<Buf> slots;
};

struct Exec {
  Program* prog;
  Frame frame;
  std::string failure;
};

// The control-flow attributes of a plan step (include/rg_plan.h): counts, result slots, and the
// bodies' plans, each with its own control-flow steps parsed.
struct Control;
struct PlanX {
  Plan plan;
  std::vector<std::unique_ptr<Control>> control;  // per step; null for every other step
};
struct Control {
  int op = 0;
  int64_t n_carry = 0, n_x = 0, length = 0, max_iter = 0;
  bool reverse = false;
  std::vector<std::pair<int64_t, int64_t>> outs;  // (result index, slot)
  std::vector<PlanX> bodies;                      // scan: body; while: condition, body; cond: then, else
};

void parse_control(PlanX& px);

PlanX load_plan(const int64_t* w, size_t n) {
  PlanX px;
  px.plan = parse(w, n);
  parse_control(px);
  return px;
}

void parse_control(PlanX& px) {
  px.control.resize(px.plan.steps.size());
  for (size_t k = 0; k < px.plan.steps.size(); k++) {
    const Step& st = px.plan.steps[k];
    if (st.kind != RG_STEP_INSTR || !is_control(st.instr.op)) continue;
    const ControlAttr a = parse_control(st.instr);
    auto c = std::make_unique<Control>();
    c->op = st.instr.op;
    c->n_carry = a.n_carry;
    c->n_x = a.n_x;
    c->length = a.length;
    c->max_iter = a.max_iterations;
    c->reverse = a.reverse;
    c->outs = a.results;
    for (auto [w, n] : a.bodies) c->bodies.push_back(load_plan(w, n));
    px.control[k] = std::move(c);
  }
}

struct Program {
  Plan plan;
  std::vector<std::unique_ptr<Control>> control;
  std::vector<uint8_t> blob;
  std::mutex mu;
  std::vector<Frame> pool;
  int64_t fail_in = -1;  // test hook: the step pass that fails next (0: the next one), or -1
  uint64_t allocated = 0;
};

template <class T>
void run_fused(const Fused& f, std::vector<Buf>& s) {
  std::vector<T*> outs;
  for (auto& o : f.outputs) outs.push_back(s[(size_t)o.second].as<T>());
  std::vector<const T*> ins;
  for (auto& in : f.inputs) ins.push_back(s[(size_t)in.slot].as<T>());
  size_t n = (size_t)f.n, rank = f.shape.size();
  // Broadcast inputs (device plans only): flat source index per output index.
  std::vector<std::vector<size_t>> bst(f.inputs.size());
  auto ds = strides(f.shape);
  for (size_t k = 0; k < f.inputs.size(); k++)
    if (f.inputs[k].kind == RG_ARG_BROADCAST) bst[k] = bstrides(f.inputs[k].shape, rank);
  size_t tasks = (n + TASK - 1) / TASK;
#pragma omp parallel
  {
    std::vector<T> temp((size_t)f.regs * BLOCK);
#pragma omp for schedule(static)
    for (size_t c = 0; c < tasks; c++) {
      size_t start = c * TASK, end = std::min(start + TASK, n);
      for (size_t b = start; b < end; b += BLOCK) {
        size_t len = std::min(BLOCK, end - b);
        for (size_t k = 0; k < f.inputs.size(); k++) {
          auto& in = f.inputs[k];
          T* r = temp.data() + (size_t)in.reg * BLOCK;
          if (in.kind == RG_ARG_SPLAT) {
            for (size_t j = 0; j < len; j++) r[j] = ins[k][0];
          } else if (in.kind == RG_ARG_ROW) {
            for (size_t j = 0; j < len; j++) r[j] = ins[k][(b + j) % (size_t)in.row_len];
          } else if (in.kind == RG_ARG_BROADCAST) {
            for (size_t j = 0; j < len; j++) {
              size_t idx = b + j, src = 0;
              for (size_t d = 0; d < rank; d++) src += (idx / ds[d]) % (size_t)f.shape[d] * bst[k][d];
              r[j] = ins[k][src];
            }
          }
        }
        for (auto& m : f.ops) {
          T* d = temp.data() + (size_t)m.reg * BLOCK;
          const T* a[3];
          for (size_t q = 0; q < m.args.size(); q++)
            a[q] = m.args[q].first ? temp.data() + (size_t)m.args[q].second * BLOCK : ins[(size_t)m.args[q].second] + b;
          if (m.op == RG_OP_WHERE) {
            for (size_t j = 0; j < len; j++) d[j] = a[0][j] != (T)0 ? a[1][j] : a[2][j];
          } else if (is_unary(m.op)) {
            for (size_t j = 0; j < len; j++) d[j] = unary_op<T>(m.op, a[0][j]);
          } else {
            for (size_t j = 0; j < len; j++) d[j] = binary_op<T>(m.op, a[0][j], a[1][j]);
          }
        }
        for (size_t k = 0; k < f.outputs.size(); k++)
          memcpy(outs[k] + b, temp.data() + (size_t)f.outputs[k].first * BLOCK, len * sizeof(T));
      }
    }
  }
}

template <class T>
void reduce(const Instr& i, std::vector<Buf>& s);

// A row group of a device plan (include/rg_plan.h RG_STEP_ROWS; no reference counterpart): each
// row computed on its own. Every register is held as a full row; a row-level register (per-row
// inputs, reductions, ops on row-level values) has the same value at every position and is
// stored as one value per row. Reductions fold the row in element order. A column reduction
// (RG_ROWS_COLUMN) collects its element-level operand for every row, then reduces it over the
// leading axes exactly as the standalone reduction instruction it replaces does.
template <class T>
void run_rows(const Fused& f, std::vector<Buf>& s) {
  const size_t L = (size_t)f.row_len, n = (size_t)f.n, rows = n / L, rank = f.shape.size();
  std::vector<bool> col_op(f.ops.size(), false), col_reg((size_t)f.regs, false);
  std::vector<Buf> col_src(f.ops.size());
  for (size_t q = 0; q < f.ops.size(); q++)
    if (f.ops[q].op == RG_OP_REDUCE && (f.ops[q].aux & RG_ROWS_COLUMN)) {
      col_op[q] = col_reg[(size_t)f.ops[q].reg] = true;
      col_src[q].bytes.resize(n * sizeof(T));
    }
  for (auto& m : f.ops)
    for (auto& a : m.args)
      if (a.first && col_reg[(size_t)a.second]) throw std::runtime_error("row group reads a column reduction");
  std::vector<bool> row_level((size_t)f.regs, false);
  std::vector<std::vector<size_t>> bst(f.inputs.size());
  auto ds = strides(f.shape);
  for (size_t k = 0; k < f.inputs.size(); k++) {
    auto& in = f.inputs[k];
    if (in.kind == RG_ARG_BROADCAST) bst[k] = bstrides(in.shape, rank);
    bool per_row = in.kind == RG_ARG_SPLAT || (in.kind == RG_ARG_BROADCAST && (in.shape.empty() || in.shape.back() == 1));
    if (in.reg >= 0) row_level[(size_t)in.reg] = per_row;
  }
  for (auto& m : f.ops) {
    bool r = true;
    for (auto& a : m.args) r = r && a.first && row_level[(size_t)a.second];
    row_level[(size_t)m.reg] = m.op == RG_OP_REDUCE || r;
  }
  std::vector<T*> outs;
  for (auto& o : f.outputs) outs.push_back(s[(size_t)o.second].as<T>());
  std::vector<const T*> ins;
  for (auto& in : f.inputs) ins.push_back(s[(size_t)in.slot].as<T>());
#pragma omp parallel
  {
    std::vector<T> reg((size_t)f.regs * L);
#pragma omp for schedule(static)
    for (size_t r = 0; r < rows; r++) {
      for (size_t k = 0; k < f.inputs.size(); k++) {
        auto& in = f.inputs[k];
        if (in.reg < 0) continue;
        T* d = reg.data() + (size_t)in.reg * L;
        for (size_t j = 0; j < L; j++) {
          size_t idx = r * L + j, src = 0;
          if (in.kind == RG_ARG_SPLAT) src = 0;
          else if (in.kind == RG_ARG_ROW) src = idx % (size_t)in.row_len;
          else
            for (size_t q = 0; q < rank; q++) src += (idx / ds[q]) % (size_t)f.shape[q] * bst[k][q];
          d[j] = ins[k][src];
        }
      }
      for (size_t oq = 0; oq < f.ops.size(); oq++) {
        const auto& m = f.ops[oq];
        T* d = reg.data() + (size_t)m.reg * L;
        const T* a[3];
        for (size_t q = 0; q < m.args.size(); q++)
          a[q] = m.args[q].first ? reg.data() + (size_t)m.args[q].second * L : ins[(size_t)m.args[q].second] + r * L;
        if (col_op[oq]) {
          memcpy(col_src[oq].as<T>() + r * L, a[0], L * sizeof(T));
        } else if (m.op == RG_OP_REDUCE) {
          T acc = a[0][0];
          for (size_t j = 1; j < L; j++)
            acc = m.aux == RG_REDUCE_SUM ? acc + a[0][j] : binary_op<T>(m.aux == RG_REDUCE_MAX ? RG_OP_MAX : RG_OP_MIN, acc, a[0][j]);
          for (size_t j = 0; j < L; j++) d[j] = acc;
        } else if (m.op == RG_OP_WHERE) {
          for (size_t j = 0; j < L; j++) d[j] = a[0][j] != (T)0 ? a[1][j] : a[2][j];
        } else if (is_unary(m.op)) {
          for (size_t j = 0; j < L; j++) d[j] = unary_op<T>(m.op, a[0][j]);
        } else {
          for (size_t j = 0; j < L; j++) d[j] = binary_op<T>(m.op, a[0][j], a[1][j]);
        }
      }
      for (size_t k = 0; k < f.outputs.size(); k++) {
        if (col_reg[(size_t)f.outputs[k].first]) continue;
        const T* v = reg.data() + (size_t)f.outputs[k].first * L;
        if (row_level[(size_t)f.outputs[k].first]) outs[k][r] = v[0];
        else memcpy(outs[k] + r * L, v, L * sizeof(T));
      }
    }
  }
  for (size_t q = 0; q < f.ops.size(); q++) {
    if (!col_op[q]) continue;
    Instr red;
    red.op = RG_OP_REDUCE;
    red.dtype = f.dtype;
    red.dst = 1;
    red.n = (int64_t)L;
    red.shape = {(int64_t)L};
    red.args = {Arg{0, f.shape}};
    red.attr = {f.ops[q].aux & ~(int64_t)RG_ROWS_COLUMN, 0, (int64_t)rank - 1};
    for (size_t ax = 0; ax + 1 < rank; ax++) red.attr.push_back((int64_t)ax);
    std::vector<Buf> tmp(2);
    tmp[0] = std::move(col_src[q]);
    tmp[1].bytes.resize(L * sizeof(T));
    reduce<T>(red, tmp);
    for (size_t k = 0; k < f.outputs.size(); k++)
      if (f.outputs[k].first == f.ops[q].reg) memcpy(outs[k], tmp[1].as<T>(), L * sizeof(T));
  }
}

template <class T, class F>
void binary(const Instr& i, std::vector<Buf>& s, F f) {
  size_t n = (size_t)i.n;
  T* dst = s[(size_t)i.dst].as<T>();
  const T* av = s[(size_t)i.args[0].slot].as<T>();
  const T* bv = s[(size_t)i.args[1].slot].as<T>();
  switch (i.mode) {
    case RG_MODE_SAME:
      for (size_t j = 0; j < n; j++) dst[j] = f(av[j], bv[j]);
      break;
    case RG_MODE_ASCALAR: {
      T c = av[0];
      for (size_t j = 0; j < n; j++) dst[j] = f(c, bv[j]);
      break;
    }
    case RG_MODE_BSCALAR: {
      T c = bv[0];
      for (size_t j = 0; j < n; j++) dst[j] = f(av[j], c);
      break;
    }
    default: {
      size_t rank = i.shape.size();
      std::vector<size_t> st[3] = {strides(i.shape), bstrides(i.args[0].shape, rank), bstrides(i.args[1].shape, rank)};
      Sh outer;
      size_t len;
      split_rows(i.shape, &outer, &len);
      size_t ra = rank ? st[1][rank - 1] : 0, rb = rank ? st[2][rank - 1] : 0;
      walk<3>(outer, st, [&](size_t* off) {
        T* row = dst + off[0];
        size_t p = off[1], q = off[2];
        for (size_t j = 0; j < len; j++) row[j] = f(av[p + (ra ? j : 0)], bv[q + (rb ? j : 0)]);
      });
    }
  }
}

// A product's optional third operand (device plans): a vector added to every row of the finished
// product, the fp32 addition the fused group it replaces would do (include/rg_plan.h).
template <class T>
void add_bias(const Instr& i, std::vector<Buf>& s) {
  if (i.args.size() != 3 || i.n == 0) return;
  const T* bias = s[(size_t)i.args[2].slot].template as<T>();
  T* dst = s[(size_t)i.dst].template as<T>();
  const size_t n = (size_t)i.shape.back();
  for (size_t e = 0; e < (size_t)i.n; e++) dst[e] = dst[e] + bias[e % n];
}

template <class T>
void matmul(const Instr& i, std::vector<Buf>& s, bool ta, bool tb) {
  const Sh &sa = i.args[0].shape, &sb = i.args[1].shape;
  const T* a = s[(size_t)i.args[0].slot].as<T>();
  const T* b = s[(size_t)i.args[1].slot].as<T>();
  T* dst = s[(size_t)i.dst].as<T>();
  size_t ar = sa.size(), br = sb.size();
  size_t m, k;
  if (ar >= 2 && !ta) {
    m = (size_t)sa[ar - 2];
    k = (size_t)sa[ar - 1];
  } else if (ar >= 2) {
    m = (size_t)sa[ar - 1];
    k = (size_t)sa[ar - 2];
  } else {
    m = 1;
    k = (size_t)sa[0];
  }
  size_t n = br >= 2 ? (size_t)(tb ? sb[br - 2] : sb[br - 1]) : 1;
  Sh ba(sa.begin(), sa.begin() + (ar >= 2 ? ar - 2 : 0)), bb(sb.begin(), sb.begin() + (br >= 2 ? br - 2 : 0));
  if (i.n == 0) return;
  if (bb.empty() && !ta) {
    // A 2-D right operand: the left operand's leading dims stack into rows of one matrix, so one gemm does it.
    size_t rows = prod(ba) * m;
    if (g_row_parallel_gemm && rows * k * n >= PARALLEL_FLOPS && rows >= 64) {
      // Checker-only speed-up (off by default, so the CPU baseline stays the reference's serial
      // loop): blocked rows on every thread, bit-identical to the serial call.
      gemm_checker<T>(rows, k, n, a, false, b, tb, dst);
      return;
    }
    gemm<T>(rows, k, n, a, false, b, tb, dst);
    return;
  }
  size_t r = std::max(ba.size(), bb.size());
  Sh batch(r);
  for (size_t q = 0; q < r; q++) {
    int64_t x = q < r - ba.size() ? 1 : ba[q - (r - ba.size())];
    int64_t y = q < r - bb.size() ? 1 : bb[q - (r - bb.size())];
    batch[q] = std::max(x, y);
  }
  size_t sz_a = m * k, sz_b = k * n, sz_o = m * n;
  std::vector<size_t> st[3] = {strides(batch), bstrides(ba, r), bstrides(bb, r)};
  for (auto& v : st[0]) v *= sz_o;
  for (auto& v : st[1]) v *= sz_a;
  for (auto& v : st[2]) v *= sz_b;
  std::vector<std::array<size_t, 3>> offs;
  walk<3>(batch, st, [&](size_t* off) { offs.push_back({off[0], off[1], off[2]}); });
  bool par = m * k * n * offs.size() >= PARALLEL_FLOPS;
  if (g_row_parallel_gemm && par && offs.size() < 8 && m >= 64) {
    // Few large products (the weight gradients): each one spread over the threads instead.
    for (auto& o : offs) gemm_checker<T>(m, k, n, a + o[1], ta, b + o[2], tb, dst + o[0]);
    return;
  }
#pragma omp parallel for schedule(static) if (par)
  for (size_t q = 0; q < offs.size(); q++) gemm<T>(m, k, n, a + offs[q][1], ta, b + offs[q][2], tb, dst + offs[q][0]);
}

template <class T>
void reduce(const Instr& i, std::vector<Buf>& s) {
  int kind = (int)i.attr[0];
  size_t n_axes = (size_t)i.attr[2];
  std::vector<size_t> axes(i.attr.begin() + 3, i.attr.begin() + 3 + (ptrdiff_t)n_axes);
  const T* a = s[(size_t)i.args[0].slot].as<T>();
  T* dst = s[(size_t)i.dst].as<T>();
  const Sh& in_shape = i.args[0].shape;
  size_t in_n = prod(in_shape), out_n = (size_t)i.n;
  if (kind == RG_REDUCE_SUM && axes.size() == in_shape.size()) {
    dst[0] = fast_sum(a, in_n);
    return;
  }
  Sh keep = in_shape;
  for (size_t ax : axes) keep[ax] = 1;
  auto out_st = strides(keep);
  for (size_t ax : axes) out_st[ax] = 0;
  auto in_st = strides(in_shape);
  Sh outer;
  size_t len;
  split_rows(in_shape, &outer, &len);
  bool last_reduced = !in_shape.empty() && out_st.back() == 0;
  auto combine = [kind](T acc, T x) {
    return kind == RG_REDUCE_SUM ? acc + x : kind == RG_REDUCE_MAX ? nan_max(acc, x) : nan_min(acc, x);
  };
  T init = kind == RG_REDUCE_SUM ? (T)0 : kind == RG_REDUCE_MAX ? (T)-INFINITY : (T)INFINITY;
  if (in_n >= (kind == RG_REDUCE_SUM ? PARALLEL_SUM : PARALLEL_MINMAX) && len > 0) {
    if (axes.size() == 1 && axes[0] == in_shape.size() - 1) {
      // One input row per output value.
#pragma omp parallel for schedule(static)
      for (size_t o = 0; o < out_n; o++) {
        const T* row = a + o * len;
        if (kind == RG_REDUCE_SUM) {
          dst[o] = fast_sum(row, len);
        } else {
          T acc = init;
          for (size_t j = 0; j < len; j++) acc = combine(acc, row[j]);
          dst[o] = acc;
        }
      }
      return;
    }
    bool has_last = std::find(axes.begin(), axes.end(), in_shape.size() - 1) != axes.end();
    if (axes.size() + 1 == in_shape.size() && !has_last) {
      // Only the last axis survives: partials over fixed 64-row chunks, combined in order.
      size_t rows = in_n / len, chunks = (rows + REDUCE_ROWS - 1) / REDUCE_ROWS;
      std::vector<T> parts(chunks * len, init);
#pragma omp parallel for schedule(static)
      for (size_t c = 0; c < chunks; c++) {
        T* part = parts.data() + c * len;
        for (size_t r = c * REDUCE_ROWS; r < std::min(rows, (c + 1) * REDUCE_ROWS); r++)
          for (size_t j = 0; j < len; j++) part[j] = combine(part[j], a[r * len + j]);
      }
      for (size_t j = 0; j < len; j++) dst[j] = init;
      for (size_t c = 0; c < chunks; c++)
        for (size_t j = 0; j < len; j++) dst[j] = combine(dst[j], parts[c * len + j]);
      return;
    }
  }
  for (size_t o = 0; o < out_n; o++) dst[o] = init;
  std::vector<size_t> st[2] = {in_st, out_st};
  walk<2>(outer, st, [&](size_t* off) {
    const T* row = a + off[0];
    size_t q = off[1];
    if (last_reduced && kind == RG_REDUCE_SUM) {
      dst[q] = dst[q] + fast_sum(row, len);
    } else if (last_reduced) {
      T acc = dst[q];
      for (size_t j = 0; j < len; j++) acc = combine(acc, row[j]);
      dst[q] = acc;
    } else {
      for (size_t j = 0; j < len; j++) dst[q + j] = combine(dst[q + j], row[j]);
    }
  });
}

template <class T>
void structural(const Instr& i, std::vector<Buf>& s) {
  T* dst = s[(size_t)i.dst].as<T>();
  const T* a = s[(size_t)i.args[0].slot].as<T>();
  size_t n = (size_t)i.n;
  auto ds = strides(i.shape);
  Sh outer;
  size_t len;
  switch (i.op) {
    case RG_OP_WHERE: {
      const T* x = s[(size_t)i.args[1].slot].as<T>();
      const T* y = s[(size_t)i.args[2].slot].as<T>();
      for (size_t j = 0; j < n; j++) dst[j] = a[j] != (T)0 ? x[j] : y[j];
      break;
    }
    case RG_OP_TRANSPOSE: {
      auto src = strides(i.args[0].shape);
      std::vector<size_t> mapped;
      for (auto p : i.attr) mapped.push_back(src[(size_t)p]);
      split_rows(i.shape, &outer, &len);
      size_t last = mapped.empty() ? 1 : mapped.back();
      std::vector<size_t> st[2] = {ds, mapped};
      std::vector<std::pair<size_t, size_t>> rows;
      walk<2>(outer, st, [&](size_t* off) { rows.push_back({off[0], off[1]}); });
#pragma omp parallel for schedule(static) if (n >= PARALLEL_COPY)
      for (size_t r = 0; r < rows.size(); r++)
        for (size_t j = 0; j < len; j++) dst[rows[r].first + j] = a[rows[r].second + j * last];
      break;
    }
    case RG_OP_BROADCAST_TO: {
      auto src = bstrides(i.args[0].shape, i.shape.size());
      split_rows(i.shape, &outer, &len);
      size_t last = src.empty() ? 0 : src.back();
      std::vector<size_t> st[2] = {ds, src};
      walk<2>(outer, st, [&](size_t* off) {
        for (size_t j = 0; j < len; j++) dst[off[0] + j] = last == 0 ? a[off[1]] : a[off[1] + j];
      });
      break;
    }
    case RG_OP_SLICE: {
      size_t r = (size_t)i.attr[0];
      auto src = strides(i.args[0].shape);
      size_t base = 0;
      for (size_t d = 0; d < r; d++) base += (size_t)i.attr[1 + d] * src[d];
      split_rows(i.shape, &outer, &len);
      std::vector<size_t> st[2] = {ds, src};
      walk<2>(outer, st, [&](size_t* off) { memcpy(dst + off[0], a + base + off[1], len * sizeof(T)); });
      break;
    }
    case RG_OP_PAD: {
      size_t r = (size_t)i.attr[0];
      std::fill(dst, dst + n, (T)0);
      auto src = strides(i.args[0].shape);
      size_t base = 0;
      for (size_t d = 0; d < r; d++) base += (size_t)i.attr[1 + d] * ds[d];
      split_rows(i.args[0].shape, &outer, &len);
      std::vector<size_t> st[2] = {ds, src};
      walk<2>(outer, st, [&](size_t* off) { memcpy(dst + base + off[0], a + off[1], len * sizeof(T)); });
      break;
    }
    case RG_OP_CONCAT: {
      size_t axis = (size_t)i.attr[0];
      size_t tail = 1, outer_n = 1;
      for (size_t d = axis + 1; d < i.shape.size(); d++) tail *= (size_t)i.shape[d];
      for (size_t d = 0; d < axis; d++) outer_n *= (size_t)i.shape[d];
      size_t at = 0;
      for (size_t o = 0; o < outer_n; o++)
        for (auto& arg : i.args) {
          size_t l = (size_t)arg.shape[axis] * tail;
          memcpy(dst + at, s[(size_t)arg.slot].as<T>() + o * l, l * sizeof(T));
          at += l;
        }
      break;
    }
    case RG_OP_TAKE: {
      size_t axis = (size_t)i.attr[0];
      const Sh& xs = i.args[0].shape;
      size_t block = 1, outer_n = 1;
      for (size_t d = axis + 1; d < xs.size(); d++) block *= (size_t)xs[d];
      for (size_t d = 0; d < axis; d++) outer_n *= (size_t)xs[d];
      size_t dim = (size_t)xs[axis], n_idx = prod(i.args[1].shape);
      const int32_t* idx = s[(size_t)i.args[1].slot].as<int32_t>();
      for (size_t o = 0; o < outer_n; o++)
        for (size_t j = 0; j < n_idx; j++)
          memcpy(dst + (o * n_idx + j) * block, a + (o * dim + clamp_index(idx[j], dim)) * block, block * sizeof(T));
      break;
    }
    case RG_OP_TAKE_ALONG: {
      size_t v = (size_t)i.args[0].shape.back(), k = (size_t)i.args[1].shape.back();
      const int32_t* idx = s[(size_t)i.args[1].slot].as<int32_t>();
      for (size_t j = 0; j < n; j++) dst[j] = a[(j / k) * v + clamp_index(idx[j], v)];
      break;
    }
  }
}

template <class T>
void numeric(const Instr& i, std::vector<Buf>& s) {
  T* dst = s[(size_t)i.dst].as<T>();
  size_t n = (size_t)i.n;
  switch (i.op) {
    case RG_OP_MATMUL: matmul<T>(i, s, false, false); add_bias<T>(i, s); break;
    case RG_OP_MATMUL_T: matmul<T>(i, s, i.attr[0] != 0, i.attr[1] != 0); add_bias<T>(i, s); break;
    case RG_OP_REDUCE: reduce<T>(i, s); break;
    case RG_OP_TAKE_GRAD: {
      size_t axis = (size_t)i.attr[0];
      Sh shape(i.attr.begin() + 1, i.attr.end());
      const T* ct = s[(size_t)i.args[0].slot].as<T>();
      size_t block = 1, outer_n = 1;
      for (size_t d = axis + 1; d < shape.size(); d++) block *= (size_t)shape[d];
      for (size_t d = 0; d < axis; d++) outer_n *= (size_t)shape[d];
      size_t dim = (size_t)shape[axis], n_idx = prod(i.args[1].shape);
      const int32_t* idx = s[(size_t)i.args[1].slot].as<int32_t>();
      std::fill(dst, dst + n, (T)0);
      for (size_t o = 0; o < outer_n; o++)
        for (size_t j = 0; j < n_idx; j++) {
          T* to = dst + (o * dim + clamp_index(idx[j], dim)) * block;
          const T* from = ct + (o * n_idx + j) * block;
          for (size_t q = 0; q < block; q++) to[q] = to[q] + from[q];
        }
      break;
    }
    case RG_OP_TAKE_ALONG_GRAD: {
      const T* ct = s[(size_t)i.args[0].slot].as<T>();
      size_t v = (size_t)i.attr.back();
      size_t k = (size_t)i.args[1].shape.back(), n_ct = prod(i.args[1].shape);
      const int32_t* idx = s[(size_t)i.args[1].slot].as<int32_t>();
      std::fill(dst, dst + n, (T)0);
      for (size_t j = 0; j < n_ct; j++) {
        size_t to = (j / k) * v + clamp_index(idx[j], v);
        dst[to] = dst[to] + ct[j];
      }
      break;
    }
    case RG_OP_RAND_UNIFORM: {
      const int32_t* kk = s[(size_t)i.args[0].slot].as<int32_t>();
      uint64_t key = ((uint64_t)(uint32_t)kk[0] << 32) | (uint64_t)(uint32_t)kk[1];
      int mant = sizeof(T) == 4 ? 24 : 53;
      double scale = std::ldexp(1.0, -mant);
#pragma omp parallel for schedule(static) if (n >= PARALLEL_RANDOM)
      for (size_t j = 0; j < n; j++)
        dst[j] = (T)((double)(mix(key + ((uint64_t)j + 1) * GAMMA) >> (64 - mant)) * scale);
      break;
    }
    case RG_OP_RAND_NORMAL: {
      const int32_t* kk = s[(size_t)i.args[0].slot].as<int32_t>();
      uint64_t key = ((uint64_t)(uint32_t)kk[0] << 32) | (uint64_t)(uint32_t)kk[1];
      auto unit = [key](uint64_t c) { return (double)(mix(key + c * GAMMA) >> 11) * std::ldexp(1.0, -53); };
      const double TAU = 6.283185307179586;
#pragma omp parallel for schedule(static) if (n >= PARALLEL_RANDOM)
      for (size_t j = 0; j < n; j++) {
        double u1 = 1.0 - unit(2 * (uint64_t)j + 1), u2 = unit(2 * (uint64_t)j + 2);
        dst[j] = (T)(std::sqrt(-2.0 * log(u1)) * cos(TAU * u2));
      }
      break;
    }
  }
}

template <class T>
void arg_top_k(const Instr& i, std::vector<Buf>& s) {
  size_t v = (size_t)i.args[0].shape.back(), k = (size_t)i.attr[0];
  const T* a = s[(size_t)i.args[0].slot].as<T>();
  int32_t* dst = s[(size_t)i.dst].as<int32_t>();
  size_t rows = prod(i.args[0].shape) / v;
  // Ordering used for the ranking: greater values rank first, equal values by position, NaN after everything (plan.rs:838-848).
  for (size_t r = 0; r < rows; r++) {
    const T* row = a + r * v;
    std::vector<int32_t> idx(v);
    std::iota(idx.begin(), idx.end(), 0);
    auto less = [row](int32_t x, int32_t y) {
      T p = row[x], q = row[y];
      bool pn = std::isnan(p), qn = std::isnan(q);
      if (pn || qn) {
        if (pn != qn) return qn;  // the non-NaN one first
        return x < y;
      }
      if (p != q) return p > q;
      return x < y;
    };
    std::stable_sort(idx.begin(), idx.end(), less);
    memcpy(dst + r * k, idx.data(), k * sizeof(int32_t));
  }
}

template <class T>
void cumsum(const Instr& i, std::vector<Buf>& s) {
  size_t v = (size_t)i.shape.back();
  if (v == 0) return;
  const T* a = s[(size_t)i.args[0].slot].as<T>();
  T* dst = s[(size_t)i.dst].as<T>();
  bool reverse = i.attr[0] != 0;
  for (size_t r = 0; r < (size_t)i.n / v; r++) {
    T acc = 0;
    if (reverse)
      for (size_t j = v; j-- > 0;) dst[r * v + j] = acc = acc + a[r * v + j];
    else
      for (size_t j = 0; j < v; j++) dst[r * v + j] = acc = acc + a[r * v + j];
  }
}

template <class T>
void argmax(const Instr& i, std::vector<Buf>& s) {
  size_t v = (size_t)i.args[0].shape.back();
  const T* a = s[(size_t)i.args[0].slot].as<T>();
  int32_t* dst = s[(size_t)i.dst].as<int32_t>();
  for (size_t o = 0; o < (size_t)i.n; o++) {
    const T* r = a + o * v;
    size_t best = 0;
    for (size_t j = 0; j < v; j++)
      if (r[j] > r[best]) best = j;
    dst[o] = (int32_t)best;
  }
}

int32_t sat_i32(double x) {
  if (std::isnan(x)) return 0;
  if (x >= 2147483647.0) return INT32_MAX;
  if (x <= -2147483648.0) return INT32_MIN;
  return (int32_t)x;
}

// Rust `as` conversions (plan.rs:1624-1642): float to int truncates and saturates, NaN is 0.
void cast(const Instr& i, int sd, std::vector<Buf>& s) {
  size_t n = (size_t)i.n;
  Buf& src = s[(size_t)i.args[0].slot];
  Buf& dst = s[(size_t)i.dst];
  int to = (int)i.attr[0];
  for (size_t j = 0; j < n; j++) {
    double x = sd == RG_F32 ? (double)src.as<float>()[j] : sd == RG_F64 ? src.as<double>()[j] : (double)src.as<int32_t>()[j];
    if (to == RG_F32) dst.as<float>()[j] = (float)x;  // one rounding, as the direct conversion
    else if (to == RG_F64) dst.as<double>()[j] = x;
    else dst.as<int32_t>()[j] = sat_i32(x);
  }
}



void key_split(const Instr& i, std::vector<Buf>& s) {
  const int32_t* kk = s[(size_t)i.args[0].slot].as<int32_t>();
  uint64_t key = ((uint64_t)(uint32_t)kk[0] << 32) | (uint64_t)(uint32_t)kk[1];
  int32_t* dst = s[(size_t)i.dst].as<int32_t>();
  for (size_t j = 0; j < (size_t)i.n / 2; j++) {
    uint64_t bits = mix(key + ((uint64_t)j + 1) * GAMMA_SPLIT);
    dst[2 * j] = (int32_t)(uint32_t)(bits >> 32);
    dst[2 * j + 1] = (int32_t)(uint32_t)bits;
  }
}

template <class T>
void step_float(const Instr& i, std::vector<Buf>& s) {
  if (is_unary(i.op)) {
    T* d = s[(size_t)i.dst].as<T>();
    const T* a = s[(size_t)i.args[0].slot].as<T>();
    for (size_t j = 0; j < (size_t)i.n; j++) d[j] = unary_op<T>(i.op, a[j]);
  } else if (is_binary(i.op)) {
    int op = i.op;
    binary<T>(i, s, [op](T a, T b) { return binary_op<T>(op, a, b); });
  } else if (i.op == RG_OP_CUMSUM) {
    cumsum<T>(i, s);
  } else if (i.op == RG_OP_WHERE || i.op == RG_OP_TRANSPOSE || i.op == RG_OP_BROADCAST_TO || i.op == RG_OP_SLICE ||
             i.op == RG_OP_PAD || i.op == RG_OP_CONCAT || i.op == RG_OP_TAKE || i.op == RG_OP_TAKE_ALONG) {
    structural<T>(i, s);
  } else {
    numeric<T>(i, s);
  }
}

void exec_instr(const Plan& p, const Instr& i, std::vector<Buf>& s) {
  int arg_dtype = i.args.empty() ? i.dtype : p.slots[(size_t)i.args[0].slot].dtype;
  switch (i.op) {
    case RG_OP_CAST: cast(i, arg_dtype, s); return;
    case RG_OP_KEY_SPLIT: key_split(i, s); return;
    case RG_OP_ARG_TOP_K:
      if (arg_dtype == RG_F32) arg_top_k<float>(i, s);
      else arg_top_k<double>(i, s);
      return;
    case RG_OP_ARGMAX:
      if (arg_dtype == RG_F32) argmax<float>(i, s);
      else argmax<double>(i, s);
      return;
    default: break;
  }
  if (i.dtype == RG_F32) step_float<float>(i, s);
  else if (i.dtype == RG_F64) step_float<double>(i, s);
  else {
    // Integer steps: wrapping arithmetic, comparisons, and the copying kernels (plan.rs:1272-1287).
    if (is_binary(i.op)) {
      int op = i.op;
      binary<int32_t>(i, s, [op](int32_t a, int32_t b) { return int_op(op, a, b); });
    } else if (i.op == RG_OP_CUMSUM) {
      // Wrapping addition, as i32's Add panics only in debug builds.
      size_t v = (size_t)i.shape.back();
      const int32_t* a = s[(size_t)i.args[0].slot].as<int32_t>();
      int32_t* d = s[(size_t)i.dst].as<int32_t>();
      bool reverse = i.attr[0] != 0;
      for (size_t r = 0; v && r < (size_t)i.n / v; r++) {
        uint32_t acc = 0;
        if (reverse)
          for (size_t j = v; j-- > 0;) d[r * v + j] = (int32_t)(acc += (uint32_t)a[r * v + j]);
        else
          for (size_t j = 0; j < v; j++) d[r * v + j] = (int32_t)(acc += (uint32_t)a[r * v + j]);
      }
    } else {
      structural<int32_t>(i, s);
    }
  }
}

// A fused attention step of a device plan (include/rg_plan.h RG_STEP_ATTN; no reference
// counterpart). Evaluated per (batch, head) problem with the same operations, in the same order,
// as the nodes the step replaces, so the result equals the unfused plan's bit for bit:
//   S = q k^T (matmul_t tb), Y = where(mask, S / div, fill), m = max_row(Y), E = exp(Y - m),
//   Z = sum_row(E) (plan.rs lane-wise row sum), P = E / Z, O = P v;
// backward: dP = dO v^T, dv = P^T dO, dY = (dP / Z + sum_row(-dP * E / (Z * Z))) * E,
//   dS = where(mask, dY, 0) / div, dq = dS k, dk = dS^T q
// (the autodiff's form of those nodes, rustautograd_amd/csrc/engine/attention.cpp).
void run_attention(const Attn& a, std::vector<Buf>& s) {
  const size_t tq = (size_t)a.tq, tk = (size_t)a.tk, hd = (size_t)a.hd, bh = (size_t)a.bh, heads = (size_t)a.heads;
  const float div = (float)a.div, fill = (float)a.fill;
  auto ptr = [&](int64_t slot) { return s[(size_t)slot].as<float>(); };
  const float* mask = a.mask_slot >= 0 ? ptr(a.mask_slot) : nullptr;
  // Operand views: row t of problem b at offset + (b / heads) sb + (b % heads) sh + t st.
  auto row = [&](const AttnView& v, size_t b, size_t t) {
    return ptr(v.slot) + v.offset + (int64_t)(b / heads) * v.sb + (int64_t)(b % heads) * v.sh + (int64_t)t * v.st;
  };
  auto gather = [&](const AttnView& v, size_t b, size_t t_n, std::vector<float>& out) {
    out.resize(t_n * hd);
    for (size_t t = 0; t < t_n; t++) memcpy(&out[t * hd], row(v, b, t), hd * sizeof(float));
  };
  auto scatter = [&](const AttnView& v, size_t b, size_t t_n, const std::vector<float>& in) {
    for (size_t t = 0; t < t_n; t++) memcpy(row(v, b, t), &in[t * hd], hd * sizeof(float));
  };
#pragma omp parallel for schedule(static)
  for (size_t b = 0; b < bh; b++) {
    std::vector<float> q, k, v;
    gather(a.in[0], b, tq, q);
    gather(a.in[1], b, tk, k);
    gather(a.in[2], b, tk, v);
    const float* mb = mask ? mask + (b / heads) * a.mask_strides[0] + (b % heads) * a.mask_strides[1] : nullptr;
    auto visible = [&](size_t i, size_t j) { return !mb || mb[(int64_t)i * a.mask_strides[2] + (int64_t)j * a.mask_strides[3]] != 0.0f; };
    std::vector<float> S(tq * tk), E(tq * tk), Z(tq), P(tq * tk);
    gemm<float>(tq, hd, tk, q.data(), false, k.data(), true, S.data());
    for (size_t i = 0; i < tq; i++) {
      float* y = &S[i * tk];
      float m = -INFINITY;
      for (size_t j = 0; j < tk; j++) {
        y[j] = visible(i, j) ? y[j] / div : fill;
        m = nan_max(m, y[j]);
      }
      for (size_t j = 0; j < tk; j++) E[i * tk + j] = t_exp(y[j] - m);
      Z[i] = fast_sum(&E[i * tk], tk);
      for (size_t j = 0; j < tk; j++) P[i * tk + j] = E[i * tk + j] / Z[i];
    }
    if (!a.backward) {
      std::vector<float> o(tq * hd);
      gemm<float>(tq, tk, hd, P.data(), false, v.data(), false, o.data());
      scatter(a.out[0], b, tq, o);
      continue;
    }
    std::vector<float> d_o, dP(tq * tk), dS(tq * tk), t(tk), dq(tq * hd), dk(tk * hd), dv(tk * hd);
    gather(a.in[4], b, tq, d_o);
    gemm<float>(tq, hd, tk, d_o.data(), false, v.data(), true, dP.data());
    gemm<float>(tk, tq, hd, P.data(), true, d_o.data(), false, dv.data());
    for (size_t i = 0; i < tq; i++) {
      const float z = Z[i], zz = z * z;
      for (size_t j = 0; j < tk; j++) t[j] = -dP[i * tk + j] * E[i * tk + j] / zz;
      const float e = fast_sum(t.data(), tk);
      for (size_t j = 0; j < tk; j++) {
        const float h = (dP[i * tk + j] / z + e) * E[i * tk + j];
        dS[i * tk + j] = (visible(i, j) ? h : 0.0f) / div;
      }
    }
    gemm<float>(tq, tk, hd, dS.data(), false, k.data(), false, dq.data());
    gemm<float>(tk, tq, hd, dS.data(), true, q.data(), false, dk.data());
    scatter(a.out[0], b, tq, dq);
    scatter(a.out[1], b, tk, dk);
    scatter(a.out[2], b, tk, dv);
  }
}

Frame frame_of(const Plan& plan, const std::vector<uint8_t>& blob) {
  Frame f;
  for (auto& s : plan.slots) f.slots.push_back(Buf{std::vector<uint8_t>(std::max<size_t>((size_t)s.cap * (size_t)dtype_size(s.dtype), 4), 0)});
  for (auto& c : plan.consts)
    memcpy(f.slots[(size_t)c.slot].bytes.data(), blob.data() + c.offset, (size_t)c.n * (size_t)dtype_size(plan.slots[(size_t)c.slot].dtype));
  return f;
}

void exec_plan_step(const Plan& plan, const std::vector<std::unique_ptr<Control>>& control, const std::vector<uint8_t>& blob,
                    std::vector<Buf>& slots, size_t k);

void exec_plan(const PlanX& px, const std::vector<uint8_t>& blob, Frame& f) {
  for (size_t k = 0; k < px.plan.steps.size(); k++) exec_plan_step(px.plan, px.control, blob, f.slots, k);
}

// Bytes of `n` elements of slot `slot` of `plan`.
size_t slot_bytes(const Plan& plan, int64_t slot, int64_t n) { return (size_t)n * (size_t)dtype_size(plan.slots[(size_t)slot].dtype); }

// Copies a body's carry results into its carry inputs, through a copy of all of them first, as
// one result may be another carry's input (plan.rs:730-735).
void feed_carry(const Plan& plan, Frame& f, size_t n_carry) {
  std::vector<std::vector<uint8_t>> next;
  for (size_t k = 0; k < n_carry; k++) {
    const auto& o = plan.outputs[k];
    const auto& b = f.slots[(size_t)o.slot].bytes;
    next.emplace_back(b.begin(), b.begin() + (ptrdiff_t)slot_bytes(plan, o.slot, o.n));
  }
  for (size_t k = 0; k < n_carry; k++) memcpy(f.slots[(size_t)plan.inputs[k].first].bytes.data(), next[k].data(), next[k].size());
}

// Control flow (plan.rs:737-831): the bodies' plans run on frames of their own, fed by copies.
void run_control(const Plan& plan, const Instr& in, const Control& c, const std::vector<uint8_t>& blob, std::vector<Buf>& s) {
  auto arg_bytes = [&](size_t k) { return s[(size_t)in.args[k].slot].bytes.data(); };
  auto load_inputs = [&](const PlanX& b, Frame& f, size_t first) {
    for (size_t k = 0; k + first < in.args.size(); k++)
      memcpy(f.slots[(size_t)b.plan.inputs[k].first].bytes.data(), arg_bytes(k + first),
             slot_bytes(b.plan, b.plan.inputs[k].first, b.plan.inputs[k].second));
  };
  if (c.op == RG_OP_SCAN) {
    const PlanX& b = c.bodies[0];
    const size_t nc = (size_t)c.n_carry, nx = (size_t)c.n_x, len = (size_t)c.length;
    const size_t n_y = b.plan.outputs.size() - nc;
    Frame f = frame_of(b.plan, blob);
    // Carries and captures once; the x slices every step.
    for (size_t k = 0; k < in.args.size(); k++)
      if (k < nc || k >= nc + nx)
        memcpy(f.slots[(size_t)b.plan.inputs[k].first].bytes.data(), arg_bytes(k),
               slot_bytes(b.plan, b.plan.inputs[k].first, b.plan.inputs[k].second));
    for (size_t step = 0; step < len; step++) {
      const size_t at = c.reverse ? len - 1 - step : step;
      for (size_t k = nc; k < nc + nx; k++) {
        const auto [slot, m] = b.plan.inputs[k];
        const size_t bytes = slot_bytes(b.plan, slot, m);
        memcpy(f.slots[(size_t)slot].bytes.data(), arg_bytes(k) + at * bytes, bytes);
      }
      for (auto& [index, dst] : c.outs)
        if ((size_t)index >= nc + n_y) {
          const auto [slot, m] = b.plan.inputs[(size_t)index - nc - n_y];
          const size_t bytes = slot_bytes(b.plan, slot, m);
          memcpy(s[(size_t)dst].bytes.data() + at * bytes, f.slots[(size_t)slot].bytes.data(), bytes);
        }
      exec_plan(b, blob, f);
      for (auto& [index, dst] : c.outs)
        if ((size_t)index >= nc && (size_t)index < nc + n_y) {
          const auto& o = b.plan.outputs[(size_t)index];
          const size_t bytes = slot_bytes(b.plan, o.slot, o.n);
          memcpy(s[(size_t)dst].bytes.data() + at * bytes, f.slots[(size_t)o.slot].bytes.data(), bytes);
        }
      feed_carry(b.plan, f, nc);
    }
    for (auto& [index, dst] : c.outs)
      if ((size_t)index < nc) {
        const auto [slot, m] = b.plan.inputs[(size_t)index];
        memcpy(s[(size_t)dst].bytes.data(), f.slots[(size_t)slot].bytes.data(), slot_bytes(b.plan, slot, m));
      }
  } else if (c.op == RG_OP_WHILE) {
    const PlanX &cp = c.bodies[0], &bp = c.bodies[1];
    const size_t nc = (size_t)c.n_carry;
    Frame cf = frame_of(cp.plan, blob), bf = frame_of(bp.plan, blob);
    load_inputs(cp, cf, 0);
    load_inputs(bp, bf, 0);
    int64_t count = 0;
    for (;;) {
      exec_plan(cp, blob, cf);
      const auto& o = cp.plan.outputs[0];
      const int d = cp.plan.slots[(size_t)o.slot].dtype;
      Buf& v = cf.slots[(size_t)o.slot];
      const double x = d == RG_F32 ? (double)v.as<float>()[0] : d == RG_F64 ? v.as<double>()[0] : (double)v.as<int32_t>()[0];
      if (x == 0.0 || count == c.max_iter) break;
      exec_plan(bp, blob, bf);
      feed_carry(bp.plan, bf, nc);
      for (size_t k = 0; k < nc; k++) {
        const auto [slot, m] = bp.plan.inputs[k];
        memcpy(cf.slots[(size_t)cp.plan.inputs[k].first].bytes.data(), bf.slots[(size_t)slot].bytes.data(), slot_bytes(bp.plan, slot, m));
      }
      count++;
    }
    for (auto& [index, dst] : c.outs) {
      if ((size_t)index < nc) {
        const auto [slot, m] = bp.plan.inputs[(size_t)index];
        memcpy(s[(size_t)dst].bytes.data(), bf.slots[(size_t)slot].bytes.data(), slot_bytes(bp.plan, slot, m));
      } else {
        s[(size_t)dst].as<int32_t>()[0] = (int32_t)count;
      }
    }
  } else {
    const int pd = plan.slots[(size_t)in.args[0].slot].dtype;
    Buf& pv = s[(size_t)in.args[0].slot];
    const double pred = pd == RG_F32 ? (double)pv.as<float>()[0] : pd == RG_F64 ? pv.as<double>()[0] : (double)pv.as<int32_t>()[0];
    const PlanX& b = c.bodies[pred != 0.0 ? 0 : 1];
    Frame f = frame_of(b.plan, blob);
    load_inputs(b, f, 1);
    exec_plan(b, blob, f);
    for (auto& [index, dst] : c.outs) {
      const auto& o = b.plan.outputs[(size_t)index];
      memcpy(s[(size_t)dst].bytes.data(), f.slots[(size_t)o.slot].bytes.data(), slot_bytes(b.plan, o.slot, o.n));
    }
  }
}

void exec_step(Program* p, Frame& f, size_t k) { exec_plan_step(p->plan, p->control, p->blob, f.slots, k); }

void exec_plan_step(const Plan& plan, const std::vector<std::unique_ptr<Control>>& control, const std::vector<uint8_t>& blob,
                    std::vector<Buf>& slots, size_t k) {
  const Step& st = plan.steps[k];
  if (control[k]) {
    run_control(plan, st.instr, *control[k], blob, slots);
  } else if (st.kind == RG_STEP_ATTN) {
    run_attention(st.attn, slots);
  } else if (st.kind == RG_STEP_ROWS) {
    if (st.fused.dtype == RG_F32) run_rows<float>(st.fused, slots);
    else run_rows<double>(st.fused, slots);
  } else if (st.kind == RG_STEP_FUSED) {
    if (st.fused.dtype == RG_F32) run_fused<float>(st.fused, slots);
    else run_fused<double>(st.fused, slots);
  } else {
    exec_instr(plan, st.instr, slots);
  }
}

Frame new_frame(Program* p) {
  Frame f;
  for (auto& s : p->plan.slots) f.slots.push_back(Buf{std::vector<uint8_t>(std::max<size_t>((size_t)s.cap * (size_t)dtype_size(s.dtype), 4), 0)});
  for (auto& c : p->plan.consts)
    memcpy(f.slots[(size_t)c.slot].bytes.data(), p->blob.data() + c.offset,
           (size_t)c.n * (size_t)dtype_size(p->plan.slots[(size_t)c.slot].dtype));
  return f;
}

void put_err(char* err, size_t len, const std::string& msg) {
  if (err && len) snprintf(err, len, "%s", msg.c_str());
}

}  // namespace

extern "C" {

int rg_cpu_available(void) { return 1; }

void* rg_cpu_program_new(const int64_t* words, size_t n_words, const void* blob, size_t blob_bytes, char* err, size_t err_len) {
  try {
    PlanX px = load_plan(words, n_words);
    auto* p = new Program;
    p->plan = std::move(px.plan);
    p->control = std::move(px.control);
    p->blob.assign((const uint8_t*)blob, (const uint8_t*)blob + blob_bytes);
    return p;
  } catch (std::exception& e) {
    put_err(err, err_len, e.what());
    return nullptr;
  }
}

void rg_cpu_program_free(void* program) { delete (Program*)program; }

uint64_t rg_cpu_program_allocated_bytes(void* program) {
  auto* p = (Program*)program;
  std::lock_guard<std::mutex> lock(p->mu);
  return p->allocated;
}

void rg_cpu_program_inject_failure(void* program) { ((Program*)program)->fail_in = 0; }

void rg_cpu_program_inject_failure_after(void* program, int64_t steps) { ((Program*)program)->fail_in = steps < 0 ? 0 : steps; }

void* rg_cpu_exec_new(void* program, char* err, size_t err_len) {
  auto* p = (Program*)program;
  auto* e = new Exec;
  e->prog = p;
  {
    std::lock_guard<std::mutex> lock(p->mu);
    if (!p->pool.empty()) {
      e->frame = std::move(p->pool.back());
      p->pool.pop_back();
      return e;
    }
  }
  try {
    e->frame = new_frame(p);
  } catch (std::exception& ex) {
    put_err(err, err_len, ex.what());
    delete e;
    return nullptr;
  }
  return e;
}

void rg_cpu_exec_free(void* exec) {
  auto* e = (Exec*)exec;
  {
    std::lock_guard<std::mutex> lock(e->prog->mu);
    e->prog->pool.push_back(std::move(e->frame));
  }
  delete e;
}

int rg_cpu_exec_write(void* exec, int64_t slot, const void* src, uint64_t bytes) {
  auto* e = (Exec*)exec;
  auto& b = e->frame.slots[(size_t)slot].bytes;
  if (bytes > b.size()) return -1;
  memcpy(b.data(), src, bytes);
  return 0;
}

int rg_cpu_exec_read(void* exec, int64_t slot, void* dst, uint64_t bytes) {
  auto* e = (Exec*)exec;
  auto& b = e->frame.slots[(size_t)slot].bytes;
  if (bytes > b.size()) return -1;
  memcpy(dst, b.data(), bytes);
  return 0;
}

int rg_cpu_exec_write_slots(void* exec, int64_t n, const int64_t* slots, const void* const* srcs, const uint64_t* bytes) {
  for (int64_t k = 0; k < n; k++)
    if (rg_cpu_exec_write(exec, slots[k], srcs[k], bytes[k]) != 0) return -1;
  return 0;
}

int rg_cpu_exec_read_slots(void* exec, int64_t n, const int64_t* slots, void* const* dsts, const uint64_t* bytes) {
  for (int64_t k = 0; k < n; k++)
    if (rg_cpu_exec_read(exec, slots[k], dsts[k], bytes[k]) != 0) return -1;
  return 0;
}

double rg_cpu_exec_scalar(void* exec, int64_t slot) {
  auto* e = (Exec*)exec;
  auto& b = e->frame.slots[(size_t)slot];
  int d = e->prog->plan.slots[(size_t)slot].dtype;
  return d == RG_F32 ? (double)b.as<float>()[0] : d == RG_F64 ? b.as<double>()[0] : (double)b.as<int32_t>()[0];
}

void rg_cpu_exec_swap(void* exec, int64_t a, int64_t b) {
  auto* e = (Exec*)exec;
  std::swap(e->frame.slots[(size_t)a], e->frame.slots[(size_t)b]);
}

void rg_cpu_exec_steps(void* exec, int64_t begin, int64_t end) {
  auto* e = (Exec*)exec;
  if (!e->failure.empty()) return;
  if (e->prog->fail_in == 0) {
    e->prog->fail_in = -1;
    e->failure = "injected failure";
    return;
  }
  if (e->prog->fail_in > 0) e->prog->fail_in--;
  for (int64_t k = begin; k < end; k++) exec_step(e->prog, e->frame, (size_t)k);
}

void rg_cpu_exec_step(void* exec) { rg_cpu_exec_steps(exec, 0, (int64_t)((Exec*)exec)->prog->plan.steps.size()); }

int rg_cpu_exec_failure(void* exec, char* buf, size_t len) {
  auto* e = (Exec*)exec;
  if (e->failure.empty()) return 0;
  put_err(buf, len, e->failure);
  return 1;
}

int rg_cpu_exec_step_timed(void* exec, double* seconds) {
  auto* e = (Exec*)exec;
  for (size_t k = 0; k < e->prog->plan.steps.size(); k++) {
    auto t0 = std::chrono::steady_clock::now();
    exec_step(e->prog, e->frame, k);
    seconds[k] += std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
  }
  return 0;
}

int rg_cpu_threads(void) { return omp_get_max_threads(); }
void rg_cpu_set_threads(int n) { omp_set_num_threads(n); }
void rg_cpu_set_row_parallel_gemm(int on) { g_row_parallel_gemm = on != 0; }

}  // extern "C"
