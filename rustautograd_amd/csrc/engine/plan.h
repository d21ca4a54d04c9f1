// Plan IR: fused groups and instructions over numbered slots, with buffer reuse.
// Restates the reference's src/plan.rs:12-27 (Fuse), 75-168 (types), 184-238 (allocator),
// 249-457 (scheduling and group compilation) and 462-655 (building).
#pragma once
#include <functional>
#include <memory>
#include <vector>

#include "graph.h"

namespace rg {

struct Fuse {
  // Estimated group cost at which a CPU group pays for the thread pool (plan.rs:14-18).
  double parallel_ns;
  // Compile groups to device kernels: chains of any cost (plan.rs:19).
  bool device;
  // Order device work by dependency level (plan.rs:21).
  bool levels;
  // Most buffers one fused kernel may bind. Metal binds about 31 (plan.rs:249-250); a HIP
  // kernel argument block holds far more, so the HIP flavour only caps code size.
  size_t max_bindings;
  // Schedule float64/small-integer bookkeeping first, as the Metal backend does for its CPU
  // fallback (plan.rs:283-309). The HIP backend has no CPU fallback and keeps natural order.
  bool hoist;
  // Whether float64 elementwise chains may form device groups (Metal cannot, plan.rs:381).
  bool fuse_f64;
  // Level order is refused above this peak of live intermediates (plan.rs:251, 475).
  size_t level_max_peak;
  // Cost model of `gpu_cost_estimate` (plan.rs:481-492).
  double per_dispatch_ns, per_element_ns;
  // A BroadcastTo read only by fusable nodes is not materialized: the consuming fused kernels
  // index its source directly (the reference materializes it, graph.rs:368-379, for Where).
  bool absorb_broadcasts;
  // Level order only: fusable chains that feed nothing but plan outputs (optimizer updates) run
  // in one final level, where chains of one shape share a kernel instead of one launch each.
  bool sink_tails;
  // Level order only: last-axis reductions and the fusable work around them on the same rows
  // (normalisation, softmax, their backward forms) form row groups, one kernel each.
  bool row_groups;
  // Plan outputs get buffers of exactly their size, so that a run loop can hand state over by
  // swapping buffers (validate.rs:303-318 swaps only equal-capacity slots) instead of copying.
  bool exact_outputs;
  // Level order only: scaled, masked softmax attention and its backward form become fused
  // attention steps (attention.cpp).
  bool attention;
  // A fused group recomputes elementwise values of an earlier group it alone reads instead of
  // reading them back from memory (plan.cpp rematerialize).
  bool remat;

  static Fuse cpu() { return {200000.0, false, false, 0, false, false, 0, 30000.0, 0.1, false, false, false, false, false, false}; }
  static Fuse metal() {
    return {0.0, true, true, 28, true, false, size_t(2) << 30, 30000.0, 0.1, false, false, false, false, false, false};
  }
  // MI355X: ~4 us per dispatch inside a captured graph, ~0.001 ns per fp32 element written at
  // HBM speed, and 288 GB of HBM so level order is capped far higher.
  static Fuse hip() { return {0.0, true, true, 64, false, true, size_t(64) << 30, 4000.0, 0.001, true, true, true, true, true, true}; }
};

// An attention region of the graph (attention.cpp): the nodes a fused forward step computes
// (`fwd`, with O = node `o` its one output) and, when the graph differentiates O, the nodes a
// fused backward step computes (`bwd`, outputs dq, dk, dv for the cotangent node `d_o`).
// One operand of an attention step: element (b, h, t, d) of a problem lies at
// offset + b sb + h sh + t st + d in the buffer of node `node` (d is contiguous).
struct AttnOperand {
  uint32_t node = 0;
  int64_t offset = 0, sb = 0, sh = 0, st = 0;
};
struct AttnRegion {
  uint32_t q = 0, k = 0, v = 0, o = 0, s = 0, e = 0, z = 0, p = 0, y = 0;
  int64_t mask = -1, mask_bcast = -1;  // the mask's source node and its broadcast
  double div = 1.0, fill = 0.0;        // Y = where(mask, S / div, fill)
  bool scaled = false;
  std::vector<uint32_t> fwd, bwd, optional;
  bool has_bwd = false;
  uint32_t d_o = 0, dq = 0, dk = 0, dv = 0;
  // Where the steps read their operands (through reshapes, transposes and slices of other
  // values) and write their results (into the one transpose that reads O, or into the transposed
  // sum of dq, dk and dv padded into one tensor); the nodes those results materialize.
  AttnOperand in_q, in_k, in_v, in_do, out_o, out_dq, out_dk, out_dv;
  std::vector<uint32_t> fwd_out, bwd_out;
};
// Problem sizes of a region: bh = batch * heads independent (tq x hd, tk x hd) problems, the
// mask's element strides over (batch, heads, query, key) and its number of distinct slices.
struct AttnShape {
  size_t bh = 1, heads = 1, tq = 0, tk = 0, hd = 0, mask_slices = 0;
  int64_t mask_strides[4] = {0, 0, 0, 0};
};
std::vector<AttnRegion> match_attention(const Graph& g, const std::vector<bool>& keep, const std::vector<uint32_t>& outputs);
AttnShape attn_shape(const AttnRegion& r, const Graph& g);
// 32-bit words of the statistics slot a region's steps share, and of the packed mask tables
// (include/rg_plan.h RG_STEP_ATTN).
size_t attn_stats_words(const AttnRegion& r, const Graph& g);
size_t attn_mask_words(const AttnRegion& r, const Graph& g);
// The share of the region's tile products the device kernels execute, forward and backward: they
// skip 16 x 16 tiles a constant mask hides (the rules of csrc/hip/attention.hip). 1 when there is
// no mask or the mask is not a constant (its hidden tiles are not known when planning).
std::pair<double, double> attn_executed_share(const AttnRegion& r, const Graph& g);

struct Plan;

struct Instr {
  Op op;
  uint32_t node = 0;
  DType dtype = DType::F32;
  size_t dst = 0;
  std::vector<size_t> args;
  Shape shape;
  std::vector<Shape> arg_shapes;
  size_t n = 0;
  rg_mode mode = RG_MODE_SAME;
  // Control flow (plan.rs:127-140 `outs`): the slot of each result the plan reads, as (result
  // index, slot), and the bodies' own plans (scan: body; while: condition, body; cond: then,
  // else). `dst` is unused (SIZE_MAX).
  std::vector<std::pair<size_t, size_t>> outs;
  std::vector<std::shared_ptr<const Plan>> bodies;
};

struct FusedIn {
  size_t slot;
  rg_arg_kind kind;
  size_t row_len;  // Row(L)
  size_t reg;      // register of non-Full inputs, SIZE_MAX for Full
};

struct MicroOp {
  Op op;
  size_t reg;
  std::vector<std::pair<bool, size_t>> args;  // (is register, index)
};

// A fused group (row_len 0), or a row group: every member has the group's shape [rows..., L] or
// the row shape [rows..., 1], and last-axis reductions may be members (include/rg_plan.h,
// RG_STEP_ROWS). Row groups exist in device plans only.
struct Fused {
  DType dtype = DType::F32;
  size_t n = 0;
  size_t row_len = 0;
  std::vector<FusedIn> inputs;
  std::vector<MicroOp> ops;
  std::vector<std::pair<size_t, size_t>> outputs;  // (register, slot); never aliases an input
  size_t regs = 0;
  Shape shape;
  std::vector<Shape> input_shapes;
};

// A fused attention step (include/rg_plan.h RG_STEP_ATTN; device plans only).
struct AttnView {
  size_t slot = 0;
  int64_t offset = 0, sb = 0, sh = 0, st = 0;
};
struct Attn {
  bool backward = false;
  DType dtype = DType::F32;
  AttnShape shape;
  double div = 1.0, fill = 0.0;
  int64_t mask_slot = -1;
  int64_t mask_bits_slot = -1;  // packed mask tables, shared by the steps of one mask
  bool build_mask_bits = false;  // this step packs them (the first forward that reads the mask)
  size_t stats_slot = 0;
  std::vector<AttnView> in, out;  // forward: q, k, v -> O; backward: q, k, v, O, dO -> dq, dk, dv
  uint32_t node = 0;              // the O node (forward) or the dq node (backward)
  double executed = 1.0;          // share of the tile products the kernels execute (attn_executed_share)
};

struct Step {
  bool fused = false;
  bool attn = false;
  Instr instr;
  Fused group;
  Attn att;
};

struct PlanOutput {
  size_t slot;
  Shape shape;
  size_t n;
};

struct Plan {
  std::vector<Step> steps;
  std::vector<std::pair<DType, size_t>> slots;
  std::vector<bool> pinned;
  std::vector<std::pair<size_t, std::shared_ptr<const Tensor>>> consts;
  std::vector<size_t> input_slots, input_ns;
  std::vector<PlanOutput> outputs;
  bool reference = false;
  size_t naive_bytes = 0;
  size_t peak_live_bytes = 0;

  size_t planned_bytes() const;
  double gpu_cost_estimate(const Fuse& f) const;
  size_t n_fused() const;
  size_t n_fused_ops() const;
  // The flat descriptor of include/rg_plan.h and its constant blob.
  void serialize(std::vector<int64_t>* words, std::vector<uint8_t>* blob) const;
};

// Algorithmic work of one step, the figure a roofline divides by its time: the flops of products
// (fused attention, and matrix products on matrix cores) priced against the matrix-core peak, and
// for every other step the bytes it must move at least (each distinct input read once, each output
// written once) priced against HBM bandwidth. `streamed` says whether the device runs a product
// of these dimensions through bandwidth-bound kernels (then it is priced by its bytes); when it is
// empty every floating-point product is priced by its flops.
struct StepWork {
  double flops = 0, bytes = 0;
  double executed_flops = 0;  // the flops the device executes: attention skips hidden tiles
  bool compute = false;       // priced by flops
};
using StreamedFn = std::function<bool(DType, uint64_t m, uint64_t n, uint64_t k, uint64_t batch, bool ta, bool tb)>;
StepWork step_work(const Step& s, const StreamedFn& streamed);

// Buffer assignment by last use, scanning steps in order; with reuse=false no buffer is shared (plan.rs:462-465).
Plan build_plan(const Graph& g, const std::vector<uint32_t>& outputs, bool reuse);
// Buffer reuse plus fused groups (plan.rs:466-479).
Plan build_fused(const Graph& g, const std::vector<uint32_t>& outputs, const Fuse& cfg);

}  // namespace rg
