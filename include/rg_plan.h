/* rg plan descriptor: the flat, C-ABI form of rg's `Plan` (reference src/plan.rs:75-164).
 *
 * A device backend receives a plan as one array of int64 words plus one byte blob holding the
 * constant tensors. The words encode, in order:
 *
 *   header     RG_PLAN_MAGIC, RG_PLAN_VERSION
 *   slots      n_slots, then per slot: dtype, capacity (elements), pinned (0/1)
 *              (plan.rs:151-154: `slots`, `pinned`)
 *   consts     n_consts, then per const: slot, n (elements), byte offset into the blob
 *              (plan.rs:155 `consts`; values are row-major, native-endian, dtype sizes 4/8/4)
 *   inputs     n_inputs, then per input: slot, n                (plan.rs:156-157)
 *   outputs    n_outputs, then per output: slot, n, rank, dims  (plan.rs:142-147, 158)
 *   steps      n_steps, then per step a tagged record:
 *     RG_STEP_INSTR  op, dtype, dst, n, mode, node,
 *                    rank, dims (output shape),
 *                    n_args, per arg: slot, rank, dims,
 *                    n_attr, attr words (op specific, below)   (plan.rs:127-140 `Instr`)
 *     RG_STEP_FUSED  dtype, n, regs, rank, dims,
 *                    n_in, per input: slot, kind, row_len, reg, rank, dims,
 *                    n_ops, per micro-op: op, reg, n_args, per arg: is_reg, index,
 *                    n_out, per output: reg, slot                (plan.rs:85-111 `Fused`)
 *     RG_STEP_ROWS   dtype, n, row_len, regs, rank, dims,
 *                    n_in, per input: slot, kind, row_len, reg, rank, dims,
 *                    n_ops, per micro-op: op, reg, aux, n_args, per arg: is_reg, index,
 *                    n_out, per output: reg, slot
 *                    A row group (no reference counterpart; device plans only): `dims` is
 *                    [rows..., row_len], and each row is computed independently. A register
 *                    holds either a whole row (element level) or one value per row (row level:
 *                    per-row inputs, reductions, and ops on row-level values only). RG_OP_REDUCE
 *                    micro-ops reduce an element-level register over the row, `aux` being the
 *                    rg_reduce_kind. Inputs are read per element like a fused group's; a
 *                    Broadcast input whose last dimension is 1 is row level. Outputs of
 *                    row-level registers hold one value per row. An RG_OP_REDUCE whose `aux`
 *                    has RG_ROWS_COLUMN added reduces an element-level register over all the
 *                    rows instead (every axis but the last): its register is column level, one
 *                    value per position of the row, read by no other micro-op, and its outputs
 *                    hold row_len values.
 *     RG_STEP_ATTN   dtype, backward (0/1), bh, heads, tq, tk, hd, div (f64 bits), fill (f64 bits),
 *                    mask_slot (-1: none), mask strides (4 words), mask_bits_slot, build_bits (0/1),
 *                    stats_slot,
 *                    n_in, per in: slot, offset, sb, sh, st,  n_out, per out: the same,  node
 *                    Fused attention (no reference counterpart; device plans only) over bh
 *                    independent problems b * heads + h; row t, column d of an operand lies at
 *                    offset + b * sb + h * sh + t * st + d in its slot (so operands may be
 *                    slices and transposes of other values, and outputs may share a slot):
 *                      forward   in q, k, v        out O = softmax(where(mask, q k^T / div, fill)) v
 *                      backward  in q, k, v, O, dO out dq, dk, dv (the gradients of O's graph)
 *                    The softmax is over keys; the mask (f32, nonzero = visible) is read at
 *                    b * s0 + h * s1 + q * s2 + k * s3 for problem b * heads + h. The stats
 *                    slot holds 3 * bh * tq words of per-query statistics (written by the
 *                    forward, read by the backward). With a mask, mask_bits_slot holds
 *                    slices * (2 * tq * tk / 32 + tq) words of packed mask bits, slices being
 *                    (s0 ? bh / heads : 1) * (s1 ? heads : 1); the step with build_bits set
 *                    packs them, and later steps reading the same mask reuse them. Planned
 *                    only for hd in {16, 32, 64} and tq, tk multiples of 32 up to
 *                    RG_ATTN_MAX_T.
 *
 * Operands: MATMUL and MATMUL_T (f32, device plans) may carry a third argument, a vector of
 * the product's column count added to every row of the finished product (a bias add folded
 * into the product; no reference counterpart).
 *
 * Attribute words per op:
 *   MATMUL_T       ta, tb
 *   REDUCE         kind, keepdims, n_axes, axes...
 *   TRANSPOSE      perm...
 *   BROADCAST_TO   shape...            RESHAPE  shape...
 *   SLICE          rank, starts..., stops...
 *   PAD            rank, starts..., shape...
 *   CAST           target dtype
 *   TAKE           axis                TAKE_GRAD  axis, shape...
 *   TAKE_ALONG_GRAD shape...           CONCAT     axis
 *   RAND_UNIFORM / RAND_NORMAL  dtype, shape...
 *   KEY_SPLIT      n                   ARG_TOP_K  k          CUMSUM reverse
 *   SCAN           n_carry, n_x, length, reverse, RESULTS, BODIES
 *   WHILE          n_carry, max_iterations, RESULTS, BODIES
 *   COND           RESULTS, BODIES
 *     RESULTS      n_results, per result the program reads: result index, slot
 *     BODIES       n_bodies, per body: n_words, then a whole plan descriptor (header included)
 *                  whose constants lie in the same blob (scan: body; while: condition, body;
 *                  cond: then, else)
 *   Control flow (plan.rs:737-831): the step's `dst` is -1 and its results go to the listed
 *   slots. Scan runs its body `length` times (from the last position when `reverse`) over
 *   inputs (carries, one slice of each x, captures); its results by index are the final
 *   carries, the ys stacked along a new leading axis, then the carries as they were before each
 *   step, stacked. While runs its condition and, while that is nonzero and fewer than
 *   max_iterations steps ran, its body over (carries, captures); results are the final carries,
 *   then the step count (int32). Cond runs `then` when its first argument is nonzero, else
 *   `else`, over the remaining arguments; results are that body's outputs. A body's carry
 *   results are written back to its carry inputs after every step, all read before any is
 *   written.
 *
 * Slot buffers hold at least `capacity` elements (at least 4 bytes) and start zeroed; a value
 * is the row-major prefix of `n` elements of its slot.
 */
#ifndef RG_PLAN_H
#define RG_PLAN_H

#include <stddef.h>
#include <stdint.h>

#define RG_PLAN_MAGIC 0x4c50475244ll /* "DRGPL" */
#define RG_PLAN_VERSION 1

enum rg_dtype { RG_F32 = 0, RG_F64 = 1, RG_I32 = 2 };

/* Operation codes: the variants of `Op` (reference src/graph.rs:47-114) that can reach a plan. */
enum rg_op {
  RG_OP_INPUT = 0, RG_OP_CONST, RG_OP_NEG, RG_OP_EXP, RG_OP_LOG, RG_OP_SQRT, RG_OP_SIN, RG_OP_COS,
  RG_OP_TANH, RG_OP_ABS, RG_OP_SIGN, RG_OP_ADD, RG_OP_SUB, RG_OP_MUL, RG_OP_DIV, RG_OP_POW,
  RG_OP_MAX, RG_OP_MIN, RG_OP_GT, RG_OP_GE, RG_OP_WHERE, RG_OP_MATMUL, RG_OP_MATMUL_T,
  RG_OP_REDUCE, RG_OP_RESHAPE, RG_OP_TRANSPOSE, RG_OP_BROADCAST_TO, RG_OP_SLICE, RG_OP_PAD,
  RG_OP_CAST, RG_OP_STOP_GRADIENT, RG_OP_FLOOR, RG_OP_TAKE, RG_OP_TAKE_ALONG, RG_OP_TAKE_GRAD,
  RG_OP_TAKE_ALONG_GRAD, RG_OP_CONCAT, RG_OP_ARGMAX, RG_OP_RAND_UNIFORM, RG_OP_RAND_NORMAL,
  RG_OP_KEY_SPLIT, RG_OP_ARG_TOP_K, RG_OP_CUMSUM, RG_OP_SCAN, RG_OP_WHILE, RG_OP_COND,
  RG_OP_OUTPUT, RG_OP_PLACEHOLDER, RG_OP_CUSTOM, RG_OP_COUNT
};

enum rg_reduce_kind { RG_REDUCE_SUM = 0, RG_REDUCE_MAX = 1, RG_REDUCE_MIN = 2 };
/* Added to a row group's RG_OP_REDUCE `aux`: the reduction runs over the rows (a column reduction). */
#define RG_ROWS_COLUMN 4
/* Input kinds of a fused group (plan.rs:75-83). */
enum rg_arg_kind { RG_ARG_FULL = 0, RG_ARG_SPLAT = 1, RG_ARG_ROW = 2, RG_ARG_BROADCAST = 3 };
/* Binary broadcast modes of a single elementwise instruction (plan.rs:119-125). */
enum rg_mode { RG_MODE_SAME = 0, RG_MODE_ASCALAR = 1, RG_MODE_BSCALAR = 2, RG_MODE_GENERAL = 3 };
enum rg_step_kind { RG_STEP_INSTR = 0, RG_STEP_FUSED = 1, RG_STEP_ROWS = 2, RG_STEP_ATTN = 3 };
/* Longest query or key sequence of a fused attention step. */
#define RG_ATTN_MAX_T 256

#ifdef __cplusplus
#include <algorithm>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

namespace rgplan {

struct Arg {
  int64_t slot;
  std::vector<int64_t> shape;
};

struct Instr {
  int32_t op, dtype;
  int64_t dst, n, mode, node;
  std::vector<int64_t> shape;
  std::vector<Arg> args;
  std::vector<int64_t> attr;
};

struct FusedInput {
  int64_t slot, kind, row_len, reg;
  std::vector<int64_t> shape;
};

struct MicroOp {
  int32_t op;
  int64_t reg;
  int64_t aux = 0; /* RG_STEP_ROWS: the reduce kind of an RG_OP_REDUCE */
  std::vector<std::pair<int64_t, int64_t>> args; /* (is_reg, index) */
};

/* RG_STEP_FUSED, or RG_STEP_ROWS when row_len > 0. */
struct Fused {
  int32_t dtype;
  int64_t n, regs;
  int64_t row_len = 0;
  std::vector<int64_t> shape;
  std::vector<FusedInput> inputs;
  std::vector<MicroOp> ops;
  std::vector<std::pair<int64_t, int64_t>> outputs; /* (reg, slot) */
};

/* RG_STEP_ATTN */
struct AttnView {
  int64_t slot, offset, sb, sh, st;
};
struct Attn {
  int32_t dtype;
  bool backward;
  int64_t bh, heads, tq, tk, hd;
  double div, fill;
  int64_t mask_slot;
  int64_t mask_strides[4];
  int64_t mask_bits_slot;
  bool build_bits;
  int64_t stats_slot;
  std::vector<AttnView> in, out;
  int64_t node;
};

struct Step {
  int32_t kind;
  Instr instr;
  Fused fused;
  Attn attn;
};

struct Slot {
  int32_t dtype;
  int64_t cap;
  bool pinned;
};

struct Const {
  int64_t slot, n, offset;
};

struct Output {
  int64_t slot, n;
  std::vector<int64_t> shape;
};

struct Plan {
  std::vector<Slot> slots;
  std::vector<Const> consts;
  std::vector<std::pair<int64_t, int64_t>> inputs; /* (slot, n) */
  std::vector<Output> outputs;
  std::vector<Step> steps;
};

inline int64_t dtype_size(int32_t d) { return d == RG_F64 ? 8 : 4; }

/* Refuses a plan whose steps name slots it does not have or reach beyond a slot's capacity:
 * constants, inputs and outputs within their slots; every instruction argument's elements and
 * its `n` outputs within their slots; fused inputs by their read extent (Full n, Row row_len,
 * Splat 1, Broadcast the source size) and outputs by what they write; attention views by the
 * largest offset they touch, the statistics and the mask tables by their sizes. Called by
 * `parse`, so a backend never launches a kernel on a plan that would index past its buffers. */
inline void check_refs(const Plan& pl) {
  const int64_t ns = (int64_t)pl.slots.size();
  auto fail = [](const std::string& what) { throw std::runtime_error("plan descriptor: " + what); };
  auto prod_of = [](const std::vector<int64_t>& v) {
    int64_t n = 1;
    for (int64_t d : v) {
      if (d < 0) return (int64_t)-1;
      n *= d;
    }
    return n;
  };
  auto fits = [&](int64_t slot, int64_t n, const char* what) {
    if (slot < 0 || slot >= ns) fail(std::string(what) + " names slot " + std::to_string(slot) + " of " + std::to_string(ns));
    if (n < 0 || n > pl.slots[(size_t)slot].cap)
      fail(std::string(what) + " needs " + std::to_string(n) + " values of slot " + std::to_string(slot) + ", which holds " +
           std::to_string(pl.slots[(size_t)slot].cap));
  };
  for (const Slot& s : pl.slots)
    if ((s.dtype != RG_F32 && s.dtype != RG_F64 && s.dtype != RG_I32) || s.cap < 0) fail("a slot has a bad dtype or capacity");
  for (const Const& c : pl.consts) {
    fits(c.slot, c.n, "a constant");
    if (c.offset < 0) fail("a constant has a negative offset");
  }
  for (const auto& in : pl.inputs) fits(in.first, in.second, "an input");
  for (const Output& o : pl.outputs) {
    fits(o.slot, o.n, "an output");
    if (prod_of(o.shape) != o.n) fail("an output's shape does not hold its n values");
  }
  for (size_t k = 0; k < pl.steps.size(); k++) {
    const Step& st = pl.steps[k];
    const std::string at = "step " + std::to_string(k);
    if (st.kind == RG_STEP_INSTR) {
      const Instr& in = st.instr;
      if (in.dst != -1) fits(in.dst, in.n, (at + " output").c_str());
      for (const Arg& a : in.args)
        if (a.slot != -1) fits(a.slot, prod_of(a.shape), (at + " argument").c_str());
    } else if (st.kind == RG_STEP_FUSED || st.kind == RG_STEP_ROWS) {
      const Fused& f = st.fused;
      const int64_t rows = f.row_len > 0 ? f.n / f.row_len : 0;
      for (const FusedInput& fi : f.inputs) {
        int64_t extent = fi.kind == RG_ARG_FULL ? f.n : fi.kind == RG_ARG_ROW ? fi.row_len : fi.kind == RG_ARG_SPLAT ? 1 : prod_of(fi.shape);
        if (fi.kind < RG_ARG_FULL || fi.kind > RG_ARG_BROADCAST) fail(at + " has an input of unknown kind");
        fits(fi.slot, extent, (at + " input").c_str());
      }
      for (const auto& o : f.outputs)
        fits(o.second, f.row_len > 0 ? std::min(rows, f.row_len) : f.n, (at + " output").c_str());
    } else if (st.kind == RG_STEP_ATTN) {
      const Attn& a = st.attn;
      const int64_t batch = a.bh / a.heads;
      auto view = [&](const AttnView& v, int64_t t, const char* what) {
        if (v.offset < 0 || v.sb < 0 || v.sh < 0 || v.st < 0 || t <= 0 || a.hd <= 0) fail(at + " has a bad " + what + " view");
        fits(v.slot, v.offset + (batch - 1) * v.sb + (a.heads - 1) * v.sh + (t - 1) * v.st + a.hd, (at + " " + what).c_str());
      };
      const int64_t in_t[5] = {a.tq, a.tk, a.tk, a.tq, a.tq}, out_t[3] = {a.tq, a.tk, a.tk};
      for (size_t j = 0; j < a.in.size(); j++) view(a.in[j], in_t[j], "operand");
      for (size_t j = 0; j < a.out.size(); j++) view(a.out[j], a.backward ? out_t[j] : a.tq, "result");
      fits(a.stats_slot, 3 * a.bh * a.tq, (at + " statistics").c_str());
      if (a.mask_slot != -1) {
        const int64_t* m = a.mask_strides;
        if (m[0] < 0 || m[1] < 0 || m[2] < 0 || m[3] < 0) fail(at + " has a negative mask stride");
        fits(a.mask_slot, (batch - 1) * m[0] + (a.heads - 1) * m[1] + (a.tq - 1) * m[2] + (a.tk - 1) * m[3] + 1, (at + " mask").c_str());
        const int64_t slices = (m[0] ? batch : 1) * (m[1] ? a.heads : 1);
        fits(a.mask_bits_slot, slices * (2 * a.tq * a.tk / 32 + a.tq), (at + " mask bits").c_str());
      }
    }
  }
}

/* Parses the word array; throws std::runtime_error on a malformed descriptor. */
inline Plan parse(const int64_t* w, size_t nw) {
  size_t p = 0;
  auto next = [&]() -> int64_t {
    if (p >= nw) throw std::runtime_error("plan descriptor truncated");
    return w[p++];
  };
  auto vec = [&](int64_t n) {
    if (n < 0 || (size_t)n > nw) throw std::runtime_error("plan descriptor has a bad length");
    std::vector<int64_t> v((size_t)n);
    for (auto& x : v) x = next();
    return v;
  };
  if (next() != RG_PLAN_MAGIC) throw std::runtime_error("not an rg plan descriptor");
  if (next() != RG_PLAN_VERSION) throw std::runtime_error("unsupported plan descriptor version");
  Plan pl;
  int64_t ns = next();
  for (int64_t i = 0; i < ns; i++) {
    Slot s;
    s.dtype = (int32_t)next();
    s.cap = next();
    s.pinned = next() != 0;
    pl.slots.push_back(s);
  }
  int64_t nc = next();
  for (int64_t i = 0; i < nc; i++) {
    Const c;
    c.slot = next();
    c.n = next();
    c.offset = next();
    pl.consts.push_back(c);
  }
  int64_t ni = next();
  for (int64_t i = 0; i < ni; i++) {
    int64_t s = next();
    int64_t n = next();
    pl.inputs.push_back({s, n});
  }
  int64_t no = next();
  for (int64_t i = 0; i < no; i++) {
    Output o;
    o.slot = next();
    o.n = next();
    o.shape = vec(next());
    pl.outputs.push_back(o);
  }
  int64_t nst = next();
  for (int64_t i = 0; i < nst; i++) {
    Step st;
    st.kind = (int32_t)next();
    if (st.kind == RG_STEP_INSTR) {
      Instr& in = st.instr;
      in.op = (int32_t)next();
      in.dtype = (int32_t)next();
      in.dst = next();
      in.n = next();
      in.mode = next();
      in.node = next();
      in.shape = vec(next());
      int64_t na = next();
      for (int64_t a = 0; a < na; a++) {
        Arg arg;
        arg.slot = next();
        arg.shape = vec(next());
        in.args.push_back(arg);
      }
      in.attr = vec(next());
    } else if (st.kind == RG_STEP_FUSED || st.kind == RG_STEP_ROWS) {
      const bool rows = st.kind == RG_STEP_ROWS;
      Fused& f = st.fused;
      f.dtype = (int32_t)next();
      f.n = next();
      if (rows) {
        f.row_len = next();
        if (f.row_len <= 0) throw std::runtime_error("row group with an empty row");
      }
      f.regs = next();
      f.shape = vec(next());
      int64_t nin = next();
      for (int64_t a = 0; a < nin; a++) {
        FusedInput fi;
        fi.slot = next();
        fi.kind = next();
        fi.row_len = next();
        fi.reg = next();
        fi.shape = vec(next());
        f.inputs.push_back(fi);
      }
      int64_t nops = next();
      for (int64_t a = 0; a < nops; a++) {
        MicroOp m;
        m.op = (int32_t)next();
        m.reg = next();
        if (rows) m.aux = next();
        int64_t nargs = next();
        for (int64_t b = 0; b < nargs; b++) {
          int64_t is_reg = next();
          int64_t idx = next();
          m.args.push_back({is_reg, idx});
        }
        f.ops.push_back(m);
      }
      int64_t nout = next();
      for (int64_t a = 0; a < nout; a++) {
        int64_t r = next();
        int64_t s = next();
        f.outputs.push_back({r, s});
      }
    } else if (st.kind == RG_STEP_ATTN) {
      Attn& a = st.attn;
      a.dtype = (int32_t)next();
      a.backward = next() != 0;
      a.bh = next();
      a.heads = next();
      a.tq = next();
      a.tk = next();
      a.hd = next();
      int64_t bits = next();
      memcpy(&a.div, &bits, 8);
      bits = next();
      memcpy(&a.fill, &bits, 8);
      a.mask_slot = next();
      for (int k = 0; k < 4; k++) a.mask_strides[k] = next();
      a.mask_bits_slot = next();
      a.build_bits = next() != 0;
      a.stats_slot = next();
      for (int side = 0; side < 2; side++) {
        int64_t n = next();
        if (n < 0 || n > 8) throw std::runtime_error("malformed attention step");
        for (int64_t k = 0; k < n; k++) {
          AttnView v;
          v.slot = next();
          v.offset = next();
          v.sb = next();
          v.sh = next();
          v.st = next();
          (side ? a.out : a.in).push_back(v);
        }
      }
      a.node = next();
      if (a.in.size() != (a.backward ? 5u : 3u) || a.out.size() != (a.backward ? 3u : 1u) || a.bh <= 0 || a.heads <= 0 ||
          a.bh % a.heads != 0)
        throw std::runtime_error("malformed attention step");
    } else {
      throw std::runtime_error("unknown plan step kind");
    }
    pl.steps.push_back(std::move(st));
  }
  if (p != nw) throw std::runtime_error("plan descriptor has trailing words");
  check_refs(pl);
  return pl;
}

/* The attributes of a control-flow step (SCAN, WHILE, COND). Bodies point into the step's
 * attribute words; parse each with `parse`. */
struct ControlAttr {
  int64_t n_carry = 0, n_x = 0, length = 0, max_iterations = 0;
  bool reverse = false;
  std::vector<std::pair<int64_t, int64_t>> results; /* (result index, slot) */
  std::vector<std::pair<const int64_t*, size_t>> bodies;
};

inline bool is_control(int32_t op) { return op == RG_OP_SCAN || op == RG_OP_WHILE || op == RG_OP_COND; }

inline ControlAttr parse_control(const Instr& in) {
  const std::vector<int64_t>& a = in.attr;
  size_t q = 0;
  auto next = [&]() -> int64_t {
    if (q >= a.size()) throw std::runtime_error("control-flow attributes truncated");
    return a[q++];
  };
  ControlAttr c;
  if (in.op == RG_OP_SCAN) {
    c.n_carry = next();
    c.n_x = next();
    c.length = next();
    c.reverse = next() != 0;
  } else if (in.op == RG_OP_WHILE) {
    c.n_carry = next();
    c.max_iterations = next();
  }
  int64_t n = next();
  if (n < 0 || (size_t)n > a.size()) throw std::runtime_error("control-flow attributes have a bad length");
  for (int64_t j = 0; j < n; j++) {
    int64_t index = next();
    c.results.push_back({index, next()});
  }
  n = next();
  if (n < 0 || n > 2) throw std::runtime_error("control-flow step has a bad body count");
  for (int64_t j = 0; j < n; j++) {
    int64_t len = next();
    if (len < 0 || q + (size_t)len > a.size()) throw std::runtime_error("control-flow body truncated");
    c.bodies.push_back({a.data() + q, (size_t)len});
    q += (size_t)len;
  }
  const size_t want = in.op == RG_OP_SCAN ? 1 : 2;
  if (c.bodies.size() != want || c.n_carry < 0 || c.n_x < 0 || c.length < 0 || c.max_iterations < 0 ||
      (size_t)(c.n_carry + c.n_x) > in.args.size())
    throw std::runtime_error("control-flow step is malformed");
  return c;
}

}  // namespace rgplan
#endif /* __cplusplus */

#endif /* RG_PLAN_H */
