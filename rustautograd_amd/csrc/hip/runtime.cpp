// The HIP executor behind include/rg_hip.h: lowers every plan step to a kernel launch, owns slot
// frames in HBM, latches device failures, and runs the step loop on the device with HIP graphs.
// Replaces the reference's MetalProgram / MetalExec (src/metal.rs:362-750).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <memory>
#include <mutex>
#include <set>
#include <sstream>
#include <stdexcept>
#include <string>
#include <thread>
#include <tuple>
#include <vector>

#include "../../../include/rg_hip.h"
#include "jit.h"
#include "kernels.h"
#include "noalloc.h"

using namespace rgplan;

namespace {

constexpr size_t ALIGN = 256;

std::string err_str(hipError_t e) { return std::string(hipGetErrorName(e)) + ": " + hipGetErrorString(e); }

#define HIP_OK(expr)                                                              \
  do {                                                                            \
    hipError_t e_ = (expr);                                                       \
    if (e_ != hipSuccess) throw std::runtime_error(std::string(#expr) + " -> " + err_str(e_)); \
  } while (0)

int esize(int dtype) { return dtype == RG_F64 ? 8 : 4; }

uint64_t prod(const std::vector<int64_t>& s) {
  uint64_t n = 1;
  for (auto d : s) n *= (uint64_t)d;
  return n;
}

// One launch of a plan step: (stream, slot pointer table, workspace).
using StepFn = std::function<void(hipStream_t, void* const*, void*)>;
// A product's launch arguments from the frame's slot table and workspace.
using GemmFill = std::function<rgk::GemmArgs(void* const*, void*)>;

// Device buffers and captured graphs of the step loop (rg_hip_exec_run), kept on the frame so
// that a later run with the same description only uploads its batches and resets the counter.
// `key` is the description (slot lists, sizes, batch count, chunk); `table` the two slot tables
// the state handoff alternates between, each with its graph.
// Device buffers one run of the step loop works in: the step counter, the history ring
// (`chunk` entries per recorded output), the cycled batches and the temporaries of the state
// copies.
struct RunBuffers {
  uint64_t* counter = nullptr;
  double* hist = nullptr;
  uint64_t chunk = 1;
  std::vector<void*> batch_bufs, temps;
};

struct RunCache {
  std::vector<int64_t> key;
  std::vector<void*> table[2];
  int n_graphs = 0;
  void* mem = nullptr;  // one allocation holding the run buffers and the snapshot
  uint64_t mem_bytes = 0;
  RunBuffers buf;
  std::vector<void*> snap;
  std::vector<int64_t> state_slots;
  std::vector<hipGraph_t> graphs;
  std::vector<hipGraphExec_t> execs;
  void clear_graphs() {
    for (auto g : execs) hipGraphExecDestroy(g);
    for (auto g : graphs) hipGraphDestroy(g);
    execs.clear();
    graphs.clear();
  }
  void release() {
    clear_graphs();
    if (mem) hipFree(mem);
    mem = nullptr;
    mem_bytes = 0;
    key.clear();
    buf = RunBuffers{};
    snap.clear();
    state_slots.clear();
  }
};

struct Frame {
  void* arena = nullptr;
  uint64_t bytes = 0;
  std::vector<void*> slot;
  void* workspace = nullptr;
  hipStream_t stream = nullptr;
  RunCache run;
  // Pinned host staging for the batched slot copies (rg_hip_exec_write_slots / read_slots), grown
  // on demand: the DMA engines read and write it directly, where pageable memory goes through the
  // runtime's own bounce buffer one slot at a time.
  void* stage = nullptr;
  uint64_t stage_bytes = 0;
};

struct Program {
  Plan plan;
  std::vector<uint8_t> blob;
  std::vector<StepFn> steps;
  std::vector<std::unique_ptr<rgjit::FusedKernel>> fused;
  // Per step: the product step whose kernel computes this fused group as its epilogue, or -1.
  std::vector<int64_t> epilogue_of;
  std::vector<bool> epilogue_sunk;  // per group step: the combined kernel runs at the group's step
  // Per step: for a product launched with others at another step (group_products), that step;
  // -1 otherwise.
  std::vector<int64_t> pair_of;
  // Per step: for a column sum computed by a product epilogue's kernel, the step it runs at; -1.
  std::vector<int64_t> absorbed_into;
  // Runs of consecutive small, independent fused groups launched as one kernel (merge_sets):
  // merged[m] replaces steps first..last when all of them run; merged_at[k] is the run starting
  // at step k, or -1. The single-step functions stay for partial ranges and per-step timing.
  struct Merged {
    size_t first, last;
    StepFn fn;
  };
  std::vector<Merged> merged;
  std::vector<int64_t> merged_at;
  // Column outputs of row groups and chunked leading-axis reductions: each kernel writes partial
  // rows into its own range of the fold area (after the workspace); the folds run together, one
  // launch, just before the first step that reads one of their outputs (folds_due[k]: the folds to
  // run before step k; k = number of steps: at the end).
  struct Fold {
    uint64_t offset;
    int64_t out_slot;
    uint32_t rows, k;
    int kind, dtype;
    bool wide = false;  // a sum over a few long rows (K-split partials): fold_wide
  };
  std::vector<Fold> folds;
  std::vector<std::vector<size_t>> folds_due;
  uint64_t fold_bytes = 0;
  uint64_t fold_base() const { return (workspace_bytes + 255) / 256 * 256; }
  std::vector<void*> device_tables;  // per-batch GEMM offset tables
  uint64_t workspace_bytes = 0;
  // Slot sizes: this program's own slots, then those of its control-flow bodies (body_slots).
  std::vector<uint64_t> slot_bytes;
  // Control-flow steps (include/rg_plan.h): each body is a program of its own whose slots follow
  // this program's in the frame's slot table, from `slot_base`, and whose workspace follows this
  // program's fold area, from `ws_offset`; `temp_offset` holds the step's staging copies of its
  // carries. Null for every other step.
  struct BodyProg {
    std::unique_ptr<Program> prog;
    size_t slot_base = 0;
    uint64_t ws_offset = 0;
  };
  struct Control {
    int op = 0;
    ControlAttr attr;
    std::vector<BodyProg> bodies;
    uint64_t temp_offset = 0;
    bool stage_carries = false;  // a carry result shares a buffer with another carry's input
  };
  std::vector<std::unique_ptr<Control>> control;
  uint64_t body_ws_bytes = 0;  // workspace for the bodies, after the fold area
  // A step waits for the device to decide what runs next (while, cond): never captured in a graph.
  bool host_sync = false;
  uint64_t ws_bytes() const { return fold_base() + (fold_bytes + 255) / 256 * 256 + body_ws_bytes; }
  std::mutex mu;
  std::vector<Frame*> pool;
  // Test hook: the plan step pass that fails next, counted from now (0: the next one), or -1.
  std::atomic<int64_t> fail_in{-1};
  int device = 0;
  ~Program() {
    for (auto* f : pool) {
      f->run.release();
      hipStreamDestroy(f->stream);
      hipFree(f->arena);
      if (f->stage) hipHostFree(f->stage);
      delete f;
    }
    for (void* p : device_tables) hipFree(p);
  }
};

struct Exec {
  Program* prog;
  Frame* frame;
  std::string failure;
};

void put(char* buf, size_t len, const std::string& s) {
  if (buf && len) snprintf(buf, len, "%s", s.c_str());
}

// ---- lowering of instructions --------------------------------------------------------------

void* P(void* const* slots, int64_t s) { return slots[s]; }

// The launch arguments of product `i` (empty for an empty product); `*base_out` gets them with
// null operand pointers, for decisions made at program build.
GemmFill gemm_fill(Program& prog, const Instr& i, bool ta, bool tb, rgk::GemmArgs* base_out) {
  const auto &sa = i.args[0].shape, &sb = i.args[1].shape;
  size_t ar = sa.size(), br = sb.size();
  uint64_t m, k;
  if (ar >= 2 && !ta) { m = sa[ar - 2]; k = sa[ar - 1]; }
  else if (ar >= 2) { m = sa[ar - 1]; k = sa[ar - 2]; }
  else { m = 1; k = sa[0]; }
  uint64_t n = br >= 2 ? (uint64_t)(tb ? sb[br - 2] : sb[br - 1]) : 1;
  std::vector<int64_t> ba(sa.begin(), sa.begin() + (ar >= 2 ? ar - 2 : 0)), bb(sb.begin(), sb.begin() + (br >= 2 ? br - 2 : 0));
  int dtype = i.dtype;
  int64_t as = i.args[0].slot, bs = i.args[1].slot, dst = i.dst;
  rgk::GemmArgs base{};
  base.dtype = dtype;
  base.ta = ta;
  base.tb = tb;
  base.n = n;
  base.k = k;
  if (bb.empty() && !ta) {
    // With a 2-D right operand and no transposed left one, the left operand's batch dims fold into its rows: one product (plan.rs:1471-1475).
    base.m = prod(ba) * m;
    base.batch = 1;
  } else {
    size_t r = std::max(ba.size(), bb.size());
    std::vector<int64_t> batch(r);
    for (size_t q = 0; q < r; q++) {
      int64_t x = q < r - ba.size() ? 1 : ba[q - (r - ba.size())];
      int64_t y = q < r - bb.size() ? 1 : bb[q - (r - bb.size())];
      batch[q] = std::max(x, y);
    }
    auto sa_st = rgk::bcast_strides(ba, r), sb_st = rgk::bcast_strides(bb, r);
    uint64_t count = prod(batch);
    std::vector<int64_t> ao(count), bo(count);
    std::vector<int64_t> idx(r, 0);
    for (uint64_t c = 0; c < count; c++) {
      int64_t x = 0, y = 0;
      for (size_t d = 0; d < r; d++) {
        x += idx[d] * sa_st[d];
        y += idx[d] * sb_st[d];
      }
      ao[c] = x * (int64_t)(m * k);
      bo[c] = y * (int64_t)(k * n);
      for (size_t d = r; d-- > 0;) {
        if (++idx[d] < batch[d]) break;
        idx[d] = 0;
      }
    }
    auto affine = [&](const std::vector<int64_t>& o, uint64_t* stride) {
      int64_t st = count > 1 ? o[1] - o[0] : 0;
      for (uint64_t c = 0; c < count; c++)
        if (o[c] != (int64_t)c * st || st < 0) return false;
      *stride = (uint64_t)st;
      return true;
    };
    base.m = m;
    base.batch = count;
    auto upload = [&](const std::vector<int64_t>& o) {
      void* d = nullptr;
      HIP_OK(hipMalloc(&d, o.size() * 8));
      HIP_OK(hipMemcpy(d, o.data(), o.size() * 8, hipMemcpyHostToDevice));
      prog.device_tables.push_back(d);
      return (const int64_t*)d;
    };
    auto all4 = [](const std::vector<int64_t>& o) {
      return std::all_of(o.begin(), o.end(), [](int64_t x) { return x % 4 == 0; });
    };
    if (!affine(ao, &base.a_stride)) {
      base.a_off = upload(ao);
      base.a_off4 = all4(ao);
    }
    if (!affine(bo, &base.b_stride)) {
      base.b_off = upload(bo);
      base.b_off4 = all4(bo);
    }
  }
  *base_out = base;
  if (i.n == 0) return GemmFill();
  // A third operand is a bias added to every row of the product (f32 plans only).
  const int64_t bias = i.args.size() == 3 ? i.args[2].slot : -1;
  if (bias >= 0 && (dtype != RG_F32 || i.args[2].shape.empty() || (uint64_t)i.args[2].shape.back() != n))
    throw std::runtime_error("product bias operand does not match the product's columns");
  const int splits = rgk::gemm_splits(dtype, base.m, base.n, base.k, base.batch, ta, tb);
  const uint64_t mn = base.m * base.n;
  if (splits > 1 && base.batch == 1 && mn % 4 == 0 && mn < (1ull << 32) && bias < 0) {
    // K-split partials go to the fold area; their sum joins the deferred folds (fold_wide).
    const uint64_t off = prog.fold_bytes;
    Program::Fold fd{off, dst, (uint32_t)splits, (uint32_t)mn, RG_REDUCE_SUM, dtype};
    fd.wide = true;
    prog.folds.push_back(fd);
    prog.fold_bytes += ((uint64_t)splits * mn * sizeof(float) + 255) / 256 * 256;
    base.defer_split = true;
    base.planned_splits = splits;
    *base_out = base;
    const Program* pp = &prog;
    return [base, as, bs, dst, off, pp](void* const* sl, void* wsp) {
      rgk::GemmArgs g = base;
      g.a = sl[as];
      g.b = sl[bs];
      g.c = sl[dst];
      g.workspace = (char*)wsp + pp->fold_base() + off;
      return g;
    };
  }
  uint64_t ws = rgk::gemm_workspace(dtype, base.m, base.n, base.k, base.batch, ta, tb);
  prog.workspace_bytes = std::max(prog.workspace_bytes, ws);
  base.workspace_bytes = ws;
  *base_out = base;
  return [base, as, bs, dst, bias](void* const* sl, void* wsp) {
    rgk::GemmArgs g = base;
    g.a = sl[as];
    g.b = sl[bs];
    g.c = sl[dst];
    g.bias = bias >= 0 ? sl[bias] : nullptr;
    g.workspace = wsp;
    return g;
  };
}

StepFn gemm_step(const GemmFill& fill) {
  if (!fill) return [](hipStream_t, void* const*, void*) {};
  return [fill](hipStream_t s, void* const* sl, void* wsp) { rgk::gemm(s, fill(sl, wsp)); };
}

StepFn lower_gemm(Program& prog, const Instr& i, bool ta, bool tb) {
  rgk::GemmArgs base{};
  return gemm_step(gemm_fill(prog, i, ta, tb, &base));
}

StepFn lower_reduce(Program& prog, const Instr& i) {
  int kind = (int)i.attr[0];
  size_t n_axes = (size_t)i.attr[2];
  std::vector<bool> red(i.args[0].shape.size(), false);
  for (size_t q = 0; q < n_axes; q++) red[(size_t)i.attr[3 + q]] = true;
  const auto& in = i.args[0].shape;
  // Canonical pattern: drop size-1 dims, merge neighbours with the same role.
  std::vector<std::pair<int64_t, bool>> pat;
  for (size_t d = 0; d < in.size(); d++) {
    if (in[d] == 1) continue;
    if (!pat.empty() && pat.back().second == red[d]) pat.back().first *= in[d];
    else pat.push_back({in[d], red[d]});
  }
  int dtype = i.dtype;
  int64_t a = i.args[0].slot, dst = i.dst;
  uint64_t out_n = (uint64_t)i.n;
  if (out_n == 0 || prod(in) == 0) return [](hipStream_t, void* const*, void*) {};
  if (pat.size() == 1 && pat[0].second) {  // full reduction
    uint64_t len = pat[0].first;
    constexpr uint64_t SEG = 1u << 16;
    if (len > (1u << 20) && len % SEG == 0) {
      // Partials of 2^16-element rows, then one row of partials.
      uint64_t parts = len / SEG;
      prog.workspace_bytes = std::max<uint64_t>(prog.workspace_bytes, parts * esize(dtype));
      return [=](hipStream_t s, void* const* sl, void* ws) {
        rgk::reduce_rows(s, dtype, kind, sl[a], ws, parts, SEG);
        rgk::reduce_rows(s, dtype, kind, ws, sl[dst], 1, parts);
      };
    }
    return [=](hipStream_t s, void* const* sl, void*) { rgk::reduce_rows(s, dtype, kind, sl[a], sl[dst], 1, len); };
  }
  if (pat.size() == 2 && !pat[0].second && pat[1].second) {  // [K, R]: rows
    uint64_t rows = pat[0].first, len = pat[1].first;
    return [=](hipStream_t s, void* const* sl, void*) { rgk::reduce_rows(s, dtype, kind, sl[a], sl[dst], rows, len); };
  }
  if ((pat.size() == 2 && pat[0].second && !pat[1].second) || (pat.size() == 3 && !pat[0].second && pat[1].second && !pat[2].second)) {
    uint64_t batch = pat.size() == 3 ? pat[0].first : 1;
    uint64_t r = pat[pat.size() - 2].first, k = pat.back().first;
    uint64_t chunks = rgk::reduce_cols_chunks(dtype, batch, r, k);
    if (chunks > 1 && batch == 1) {
      // The chunk partials go to the fold area and are folded with the other deferred folds.
      const uint64_t off = prog.fold_bytes;
      prog.folds.push_back({off, dst, (uint32_t)chunks, (uint32_t)k, kind, dtype});
      prog.fold_bytes += (chunks * k * esize(dtype) + 255) / 256 * 256;
      const Program* pp = &prog;
      return [=](hipStream_t s, void* const* sl, void* ws) {
        rgk::reduce_cols(s, dtype, kind, sl[a], nullptr, 1, r, k, (char*)ws + pp->fold_base() + off, chunks);
      };
    }
    if (chunks > 1) prog.workspace_bytes = std::max<uint64_t>(prog.workspace_bytes, batch * chunks * k * esize(dtype));
    return [=](hipStream_t s, void* const* sl, void* ws) { rgk::reduce_cols(s, dtype, kind, sl[a], sl[dst], batch, r, k, ws, chunks); };
  }
  // General: one thread per output over the reduced index space.
  std::vector<int64_t> keep_shape, red_shape, keep_st, red_st;
  auto st = rgk::row_strides(in);
  for (size_t d = 0; d < in.size(); d++) {
    if (red[d]) {
      red_shape.push_back(in[d]);
      red_st.push_back(st[d]);
    } else {
      keep_shape.push_back(in[d]);
      keep_st.push_back(st[d]);
    }
  }
  rgk::Strided outer = rgk::make_strided(keep_shape, {keep_st});
  rgk::Strided inner = rgk::make_strided(red_shape, {red_st});
  uint64_t red_n = prod(red_shape);
  return [=](hipStream_t s, void* const* sl, void*) { rgk::reduce_general(s, dtype, kind, sl[a], sl[dst], out_n, outer, inner, red_n); };
}

StepFn lower_instr(Program& prog, const Instr& i) {
  int dtype = i.dtype;
  int64_t dst = i.dst;
  uint64_t n = (uint64_t)i.n;
  auto arg = [&](size_t k) { return i.args[k].slot; };
  auto slot_dtype = [&](int64_t s) { return prog.plan.slots[(size_t)s].dtype; };
  switch (i.op) {
    case RG_OP_NEG: case RG_OP_EXP: case RG_OP_LOG: case RG_OP_SQRT: case RG_OP_SIN: case RG_OP_COS: case RG_OP_TANH:
    case RG_OP_ABS: case RG_OP_SIGN: case RG_OP_FLOOR: {
      int op = i.op;
      int64_t a = arg(0);
      return [=](hipStream_t s, void* const* sl, void*) { rgk::unary(s, dtype, op, sl[a], sl[dst], n); };
    }
    case RG_OP_ADD: case RG_OP_SUB: case RG_OP_MUL: case RG_OP_DIV: case RG_OP_POW: case RG_OP_MAX: case RG_OP_MIN:
    case RG_OP_GT: case RG_OP_GE: {
      int op = i.op;
      int64_t a = arg(0), b = arg(1);
      int mode = (int)i.mode;
      if (mode == RG_MODE_GENERAL) {
        size_t r = i.shape.size();
        rgk::Strided g = rgk::make_strided(i.shape, {rgk::bcast_strides(i.args[0].shape, r), rgk::bcast_strides(i.args[1].shape, r)});
        return [=](hipStream_t s, void* const* sl, void*) { rgk::binary(s, dtype, op, sl[a], sl[b], sl[dst], n, 3, &g); };
      }
      return [=](hipStream_t s, void* const* sl, void*) { rgk::binary(s, dtype, op, sl[a], sl[b], sl[dst], n, mode, nullptr); };
    }
    case RG_OP_WHERE: {
      int64_t c = arg(0), a = arg(1), b = arg(2);
      return [=](hipStream_t s, void* const* sl, void*) { rgk::where(s, esize(dtype), sl[c], sl[a], sl[b], sl[dst], n, dtype); };
    }
    case RG_OP_MATMUL: return lower_gemm(prog, i, false, false);
    case RG_OP_MATMUL_T: return lower_gemm(prog, i, i.attr[0] != 0, i.attr[1] != 0);
    case RG_OP_REDUCE: return lower_reduce(prog, i);
    case RG_OP_TRANSPOSE: case RG_OP_BROADCAST_TO: case RG_OP_SLICE: {
      int64_t a = arg(0);
      size_t r = i.shape.size();
      std::vector<int64_t> src;
      uint32_t base = 0;
      if (i.op == RG_OP_TRANSPOSE) {
        auto st = rgk::row_strides(i.args[0].shape);
        for (auto p : i.attr) src.push_back(st[(size_t)p]);
      } else if (i.op == RG_OP_BROADCAST_TO) {
        src = rgk::bcast_strides(i.args[0].shape, r);
      } else {
        src = rgk::row_strides(i.args[0].shape);
        for (size_t d = 0; d < r; d++) base += (uint32_t)(i.attr[1 + d] * src[d]);
      }
      rgk::Strided g = rgk::make_strided(i.shape, {src});
      g.base[0] = base;
      int es = esize(dtype);
      return [=](hipStream_t s, void* const* sl, void*) { rgk::gather(s, es, sl[a], sl[dst], n, g); };
    }
    case RG_OP_PAD: {
      int64_t a = arg(0);
      size_t r = (size_t)i.attr[0];
      std::vector<int64_t> starts(i.attr.begin() + 1, i.attr.begin() + 1 + (ptrdiff_t)r);
      auto out_shape = i.shape, in_shape = i.args[0].shape;
      int es = esize(dtype);
      return [=](hipStream_t s, void* const* sl, void*) { rgk::pad(s, es, sl[a], sl[dst], n, out_shape, starts, in_shape); };
    }
    case RG_OP_CONCAT: {
      size_t axis = (size_t)i.attr[0];
      uint64_t tail = 1, outer = 1;
      for (size_t d = axis + 1; d < i.shape.size(); d++) tail *= (uint64_t)i.shape[d];
      for (size_t d = 0; d < axis; d++) outer *= (uint64_t)i.shape[d];
      uint64_t total = (uint64_t)i.shape[axis] * tail, at = 0;
      std::vector<std::pair<int64_t, std::pair<uint64_t, uint64_t>>> pieces;
      for (auto& x : i.args) {
        uint64_t len = (uint64_t)x.shape[axis] * tail;
        pieces.push_back({x.slot, {len, at}});
        at += len;
      }
      int es = esize(dtype);
      return [=](hipStream_t s, void* const* sl, void*) {
        for (auto& p : pieces) rgk::concat_piece(s, es, sl[p.first], sl[dst], outer, p.second.first, total, p.second.second);
      };
    }
    case RG_OP_TAKE: {
      size_t axis = (size_t)i.attr[0];
      const auto& xs = i.args[0].shape;
      uint64_t block = 1;
      for (size_t d = axis + 1; d < xs.size(); d++) block *= (uint64_t)xs[d];
      uint64_t dim = (uint64_t)xs[axis], n_idx = prod(i.args[1].shape);
      int64_t a = arg(0), ix = arg(1);
      int es = esize(dtype);
      return [=](hipStream_t s, void* const* sl, void*) { rgk::take(s, es, sl[a], (const int32_t*)sl[ix], sl[dst], n, block, n_idx, dim); };
    }
    case RG_OP_TAKE_ALONG: {
      uint64_t v = (uint64_t)i.args[0].shape.back(), kk = (uint64_t)i.args[1].shape.back();
      int64_t a = arg(0), ix = arg(1);
      int es = esize(dtype);
      return [=](hipStream_t s, void* const* sl, void*) { rgk::take_along(s, es, sl[a], (const int32_t*)sl[ix], sl[dst], n, kk, v); };
    }
    case RG_OP_TAKE_GRAD: {
      size_t axis = (size_t)i.attr[0];
      std::vector<int64_t> shape(i.attr.begin() + 1, i.attr.end());
      uint64_t block = 1;
      for (size_t d = axis + 1; d < shape.size(); d++) block *= (uint64_t)shape[d];
      uint64_t dim = (uint64_t)shape[axis], n_idx = prod(i.args[1].shape);
      int64_t c = arg(0), ix = arg(1);
      return [=](hipStream_t s, void* const* sl, void*) { rgk::take_grad(s, dtype, sl[c], (const int32_t*)sl[ix], sl[dst], n, block, n_idx, dim); };
    }
    case RG_OP_TAKE_ALONG_GRAD: {
      uint64_t v = (uint64_t)i.attr.back(), kk = (uint64_t)i.args[1].shape.back();
      int64_t c = arg(0), ix = arg(1);
      return [=](hipStream_t s, void* const* sl, void*) { rgk::take_along_grad(s, dtype, sl[c], (const int32_t*)sl[ix], sl[dst], n, kk, v); };
    }
    case RG_OP_RAND_UNIFORM: {
      int64_t key = arg(0);
      return [=](hipStream_t s, void* const* sl, void*) { rgk::rand_uniform(s, dtype, (const int32_t*)sl[key], sl[dst], n); };
    }
    case RG_OP_RAND_NORMAL: {
      int64_t key = arg(0);
      return [=](hipStream_t s, void* const* sl, void*) { rgk::rand_normal(s, dtype, (const int32_t*)sl[key], sl[dst], n); };
    }
    case RG_OP_KEY_SPLIT: {
      int64_t key = arg(0);
      return [=](hipStream_t s, void* const* sl, void*) { rgk::key_split(s, (const int32_t*)sl[key], (int32_t*)sl[dst], n / 2); };
    }
    case RG_OP_CAST: {
      int64_t a = arg(0);
      int from = slot_dtype(a), to = (int)i.attr[0];
      return [=](hipStream_t s, void* const* sl, void*) { rgk::cast(s, from, to, sl[a], sl[dst], n); };
    }
    case RG_OP_ARGMAX: {
      int64_t a = arg(0);
      int from = slot_dtype(a);
      uint64_t v = (uint64_t)i.args[0].shape.back();
      return [=](hipStream_t s, void* const* sl, void*) { rgk::argmax(s, from, sl[a], (int32_t*)sl[dst], n, v); };
    }
    case RG_OP_ARG_TOP_K: {
      int64_t a = arg(0);
      int from = slot_dtype(a);
      uint64_t v = (uint64_t)i.args[0].shape.back(), kk = (uint64_t)i.attr[0];
      uint64_t rows = prod(i.args[0].shape) / std::max<uint64_t>(v, 1);
      return [=](hipStream_t s, void* const* sl, void*) { rgk::arg_top_k(s, from, sl[a], (int32_t*)sl[dst], rows, v, kk); };
    }
    case RG_OP_CUMSUM: {
      int64_t a = arg(0);
      uint64_t v = (uint64_t)i.shape.back();
      bool rev = i.attr[0] != 0;
      uint64_t rows = v ? n / v : 0;
      return [=](hipStream_t s, void* const* sl, void*) { rgk::cumsum(s, dtype, sl[a], sl[dst], rows, v, rev); };
    }
    default:
      throw std::runtime_error(std::string("operation ") + std::to_string(i.op) + " has no HIP kernel in this build");
  }
}

// A fused attention step (attention.hip). The statistics slot holds the per-query max, sum and
// rowsum(dO * O), then the packed mask bits.
StepFn lower_attention(Program& prog, const rgplan::Attn& at, int64_t col_off = -1) {
  if (!rgk::attention_supported(at.dtype, at.hd, at.tq, at.tk))
    throw std::runtime_error("attention step of unsupported shape (hd " + std::to_string(at.hd) + ", t " + std::to_string(at.tq) + "x" +
                             std::to_string(at.tk) + ")");
  rgk::AttnArgs base{};
  base.bh = (uint32_t)at.bh;
  base.heads = (uint32_t)at.heads;
  base.tq = (int)at.tq;
  base.tk = (int)at.tk;
  base.hd = (int)at.hd;
  base.div = (float)at.div;
  base.fill = (float)at.fill;
  for (int k = 0; k < 4; k++) base.mask_strides[k] = at.mask_strides[k];
  const uint64_t rows = (uint64_t)at.bh * at.tq;
  const auto& ss = prog.plan.slots[(size_t)at.stats_slot];
  if ((uint64_t)ss.cap < 3 * rows || esize(ss.dtype) != 4)
    throw std::runtime_error("attention statistics slot holds " + std::to_string(ss.cap) + " words, needs " + std::to_string(3 * rows));
  if (at.mask_slot >= 0) {
    rgk::AttnArgs t = base;
    t.mask = (const float*)1;
    const uint64_t need = rgk::attention_mask_words(t);
    const auto& ms = prog.plan.slots[(size_t)at.mask_bits_slot];
    if (at.mask_bits_slot < 0 || (uint64_t)ms.cap < need || esize(ms.dtype) != 4)
      throw std::runtime_error("attention mask table slot too small: needs " + std::to_string(need) + " words");
  }
  const int64_t bits_slot = at.mask_bits_slot;
  const bool build_bits = at.build_bits;
  const int64_t mask = at.mask_slot, stats = at.stats_slot;
  const std::vector<rgplan::AttnView> in = at.in, out = at.out;
  for (const auto* vs : {&in, &out})
    for (const auto& v : *vs)
      if (v.offset % 4 || v.sb % 4 || v.sh % 4 || v.st % 4 || esize(prog.plan.slots[(size_t)v.slot].dtype) != 4)
        throw std::runtime_error("attention operand view is not 16-byte aligned");
  const bool bwd = at.backward;
  const Program* pp = &prog;
  return [=](hipStream_t s, void* const* sl, void* wsp) {
    rgk::AttnArgs a = base;
    auto op = [&](const rgplan::AttnView& v) {
      return rgk::AttnOperand{(const float*)sl[v.slot] + v.offset, v.sb, v.sh, v.st};
    };
    a.q = op(in[0]);
    a.k = op(in[1]);
    a.v = op(in[2]);
    float* st = (float*)sl[stats];
    a.stat_m = st;
    a.stat_z = st + rows;
    a.stat_dd = st + 2 * rows;
    if (mask >= 0) {
      a.mask = (const float*)sl[mask];
      a.mask_bits = (uint32_t*)sl[bits_slot];
    }
    if (!bwd) {
      a.o = op(out[0]);
      rgk::attention_forward(s, a, build_bits);
    } else {
      a.o_in = op(in[3]);
      a.d_o = op(in[4]);
      a.dq = op(out[0]);
      a.dk = op(out[1]);
      a.dv = op(out[2]);
      if (col_off >= 0) {  // column sums of dq, dk, dv: partial rows in the fold area
        a.colp = (float*)((char*)wsp + pp->fold_base() + col_off);
        a.col_len = out[0].st;
        a.col_q = out[0].offset;
        a.col_k = out[1].offset;
        a.col_v = out[2].offset;
      }
      rgk::attention_backward(s, a);
    }
  };
}

// Horizontal fusion. Fused groups of at most MERGE_MAX_GRID blocks leave most of the 256 CUs idle
// and cost about a launch each (C4's AdamW updates: one group per parameter shape). Maximal runs
// of consecutive such groups that are independent (no group writes a slot another group of the
// run reads or writes; a group's own in-place update is fine) become one kernel, up to
// MERGE_MAX_ARGS pointer arguments.
constexpr uint32_t MERGE_MAX_GRID = 256;
constexpr size_t MERGE_MAX_ARGS = 240;

uint32_t fused_grid(const rgplan::Fused& f) {
  const uint64_t per = (uint64_t)rgjit::TPB * (f.dtype == RG_F64 ? 2 : 4);
  return (uint32_t)(((uint64_t)f.n + per - 1) / per);
}

std::vector<std::pair<size_t, size_t>> merge_sets(const Plan& plan) {
  std::vector<std::pair<size_t, size_t>> sets;
  auto small = [&](size_t k) {
    const Step& st = plan.steps[k];
    if (st.kind != RG_STEP_FUSED) return false;
    uint32_t g = fused_grid(st.fused);
    return g > 0 && g <= MERGE_MAX_GRID;
  };
  size_t k = 0;
  while (k < plan.steps.size()) {
    if (!small(k)) {
      k++;
      continue;
    }
    std::set<int64_t> reads, writes;
    size_t last = k;
    for (size_t j = k; j < plan.steps.size() && small(j); j++) {
      const auto& f = plan.steps[j].fused;
      std::set<int64_t> r, w;
      for (auto& in : f.inputs) r.insert(in.slot);
      for (auto& o : f.outputs) w.insert(o.second);
      // The merged kernel takes each distinct slot once.
      std::set<int64_t> all(reads);
      all.insert(writes.begin(), writes.end());
      all.insert(r.begin(), r.end());
      all.insert(w.begin(), w.end());
      bool clash = all.size() > MERGE_MAX_ARGS;
      for (int64_t x : w) clash |= reads.count(x) || writes.count(x);
      for (int64_t x : r) clash |= writes.count(x) > 0;
      if (clash) break;
      reads.insert(r.begin(), r.end());
      writes.insert(w.begin(), w.end());
      last = j;
    }
    if (last > k) sets.push_back({k, last});
    k = last + 1;
  }
  return sets;
}

// Slots a plan step reads.
std::vector<int64_t> step_reads(const Step& st) {
  std::vector<int64_t> r;
  if (st.kind == RG_STEP_FUSED || st.kind == RG_STEP_ROWS) {
    for (auto& in : st.fused.inputs) r.push_back(in.slot);
  } else if (st.kind == RG_STEP_ATTN) {
    for (auto& v : st.attn.in) r.push_back(v.slot);
    r.push_back(st.attn.mask_slot);
    r.push_back(st.attn.mask_bits_slot);
    r.push_back(st.attn.stats_slot);
  } else {
    for (auto& a : st.instr.args) r.push_back(a.slot);
  }
  return r;
}

bool has_slot(const std::vector<int64_t>& v, int64_t x) { return std::find(v.begin(), v.end(), x) != v.end(); }

bool flat_product(const Instr& i, uint64_t* m, uint64_t* n, uint64_t* k, bool* ta, bool* tb);

// Product `i` launched through `fk`, its kernel with group `f` as the epilogue (generate_gemm):
// the tile kernel's arguments, then the pointers of the epilogue (the product's output when
// `store_c`, else null; the group's inputs; its outputs), one kernel argument each.
StepFn lower_product_epilogue(const Instr& i, const rgplan::Fused& f, const rgjit::FusedKernel* fk, bool store_c, const Program* pp,
                              int64_t col_off) {
  uint64_t m, n, k;
  bool ta, tb;
  rgk::GemmTile t;
  if (!flat_product(i, &m, &n, &k, &ta, &tb) || !rgk::gemm_epilogue_tile(RG_F32, m, n, k, ta, tb, &t))
    throw std::runtime_error("product epilogue: the product no longer fits a single tile kernel");
  std::vector<int64_t> ptr_slots;
  ptr_slots.push_back(store_c ? i.dst : -1);
  for (auto& in : f.inputs) ptr_slots.push_back(in.slot);
  for (auto& o : f.outputs) ptr_slots.push_back(o.second);
  if (ptr_slots.size() > 128) throw std::runtime_error("product epilogue with more than 127 operands");
  const int64_t as = i.args[0].slot, bs = i.args[1].slot, bias = i.args.size() == 3 ? i.args[2].slot : -1;
  const int M = (int)m, N = (int)n, K = (int)k;
  return [fk, ptr_slots, as, bs, bias, t, M, N, K, pp, col_off](hipStream_t s, void* const* sl, void* ws) {
    const void* A = sl[as];
    const void* B = sl[bs];
    const void* bias_p = bias >= 0 ? sl[bias] : nullptr;
    int mm = M, nn = N, kk = K, splits = 1, kps = t.kps, swizzle = 1;
    const void* a_off = nullptr;
    const void* b_off = nullptr;
    uint64_t a_stride = 0, b_stride = 0;
    uint32_t tm = t.tm, tn = t.tn;
    void* ptrs[129];
    void* args[15 + 129] = {&A, &B, &mm, &nn, &kk, &a_off, &b_off, &a_stride, &b_stride, &splits, &kps, &bias_p, &tm, &tn, &swizzle};
    size_t q = 0;
    for (; q < ptr_slots.size(); q++) {
      ptrs[q] = ptr_slots[q] >= 0 ? sl[ptr_slots[q]] : nullptr;
      args[15 + q] = &ptrs[q];
    }
    if (col_off >= 0) {  // the column sums' partial rows, in the fold area
      ptrs[q] = (char*)ws + pp->fold_base() + col_off;
      args[15 + q] = &ptrs[q];
    }
    hipModuleLaunchKernel(fk->fn, tm * tn, 1, 1, fk->block, 1, 1, 0, s, args, nullptr);
  };
}

// Slots a plan step writes (control-flow steps are treated apart by their callers).
std::vector<int64_t> step_writes(const Step& st) {
  std::vector<int64_t> w;
  if (st.kind == RG_STEP_FUSED || st.kind == RG_STEP_ROWS) {
    for (auto& o : st.fused.outputs) w.push_back(o.second);
  } else if (st.kind == RG_STEP_ATTN) {
    for (auto& v : st.attn.out) w.push_back(v.slot);
    w.push_back(st.attn.stats_slot);
    if (st.attn.build_bits) w.push_back(st.attn.mask_bits_slot);
  } else if (st.instr.dst >= 0) {
    w.push_back(st.instr.dst);
  }
  return w;
}

// A product instruction as one unbatched M x N x K product (the left operand's batch dims folded
// into its rows where the right operand is 2-D, as lower_gemm does), or false.
bool flat_product(const Instr& i, uint64_t* m, uint64_t* n, uint64_t* k, bool* ta, bool* tb) {
  if (i.op == RG_OP_MATMUL) *ta = *tb = false;
  else if (i.op == RG_OP_MATMUL_T) *ta = i.attr[0] != 0, *tb = i.attr[1] != 0;
  else return false;
  if (i.args.size() < 2) return false;
  const auto &sa = i.args[0].shape, &sb = i.args[1].shape;
  if (sa.size() < 2 || sb.size() != 2) return false;
  const size_t ar = sa.size();
  if (*ta && ar != 2) return false;
  uint64_t lead = 1;
  for (size_t d = 0; d + 2 < ar; d++) lead *= (uint64_t)sa[d];
  *m = lead * (uint64_t)(*ta ? sa[ar - 1] : sa[ar - 2]);
  *k = (uint64_t)(*ta ? sa[ar - 2] : sa[ar - 1]);
  *n = (uint64_t)(*tb ? sb[0] : sb[1]);
  return true;
}

// Elementwise groups computed in the epilogue of the product they read (at[j] = k: plain fused
// group j reads product k's output and runs inside product k's kernel). Taken when product k is
// one unsplit fp32 MFMA tile product (gemm_epilogue_tile), group j walks its M x N outputs with
// Full, Row (length a multiple of 4) and Splat inputs and writes none of the product's operands
// (other blocks of the product still read them while the epilogue stores), and the combined
// kernel can run at one of the two steps without changing any value, with no control flow
// between them:
//  - at step k (`sunk` false) when nothing between them writes what the group reads, or reads or
//    writes what it writes;
//  - at step j (`sunk` true) when nothing between them writes the product's operands, or reads or
//    writes its output (a weight-gradient product between an input-gradient product and the
//    activation gradient that reads it, whose output reuses the slot the weight gradient reads).
// Groups small enough to be merged are left to the merged launches. The product's kernel also
// stores its own output when another step reads it. Only products of at least
// EPILOGUE_MIN_TILES tiles are taken: every block of a product ends its K loop at about the
// same time, and the epilogue's loads and stores then run with no products beside them unless a
// second round of blocks is still multiplying (measured on MI355X: C4's GELU forward and
// backward, 8192 x 1024 outputs in 1024 tiles, 1.7 % off the step; C2's activation gradient and
// its 2048 x 2048 AdamW update, 512 tiles each, 1.1 % slower fused). RG_HIP_EPILOGUE=0 turns
// this off; RG_HIP_EPILOGUE=all takes every product that qualifies otherwise.
constexpr uint64_t EPILOGUE_MIN_TILES = 1024;  // two rounds of two blocks on each of 256 CUs

// Whether product k's output is read by a step other than j (or by the host) before it is next
// written.
bool product_output_needed(const Plan& plan, size_t k, size_t j) {
  const int64_t c = plan.steps[k].instr.dst;
  for (size_t q = k + 1; q < plan.steps.size(); q++) {
    if (q != j && has_slot(step_reads(plan.steps[q]), c)) return true;
    if (has_slot(step_writes(plan.steps[q]), c)) return false;
  }
  for (auto& o : plan.outputs)
    if (o.slot == c) return true;
  return false;
}

struct Epilogues {
  std::vector<int64_t> at;  // per step: the product whose kernel computes this group, or -1
  std::vector<bool> sunk;   // per group step: the combined kernel runs at the group's step
  // Per group step: the column sum the combined kernel also computes (a later sum over every
  // axis but the last of one of the group's outputs), or -1; per step: the group whose kernel
  // computes this sum, or -1.
  std::vector<int64_t> sum_of, sum_in;
  std::vector<int> sum_out;  // per group step: which of the group's outputs the sum reads
};

// Whether step s is an f32 sum over every axis but the last of the value in `slot`, shaped
// [..., n] with `total` elements, into [1, ..., 1, n].
bool column_sum_of(const Step& st, int64_t slot, uint64_t total, uint64_t n) {
  if (st.kind != RG_STEP_INSTR || st.instr.op != RG_OP_REDUCE || st.instr.dtype != RG_F32 || st.instr.args.size() != 1) return false;
  const Instr& i = st.instr;
  const auto& in = i.args[0].shape;
  if (i.args[0].slot != slot || in.empty() || (uint64_t)in.back() != n || prod(in) != total || (int)i.attr[0] != RG_REDUCE_SUM) return false;
  const size_t n_axes = (size_t)i.attr[2];
  std::vector<bool> red(in.size(), false);
  for (size_t q = 0; q < n_axes; q++) red[(size_t)i.attr[3 + q]] = true;
  for (size_t d = 0; d + 1 < in.size(); d++)
    if (!red[d] && in[d] != 1) return false;
  return !red[in.size() - 1] && (uint64_t)i.n == n;
}

// The step q a few steps after attention backward step j that sums the three gradients' slot
// over every axis but the last (a bias gradient of the projection q, k and v come from), when the
// backward can write those sums itself: dq, dk and dv rows of one slot, L columns a row, the
// views' heads covering every column once, and shapes for which the backward writes column sums
// (rgk::attention_backward_column_sums). -1 otherwise, or with RG_HIP_EPILOGUE_SUMS=0.
int64_t attention_column_sum(const Plan& plan, size_t j) {
  const Step& sj = plan.steps[j];
  if (sj.kind != RG_STEP_ATTN || !sj.attn.backward || sj.attn.out.size() != 3 || sj.attn.dtype != RG_F32) return -1;
  const char* sums = getenv("RG_HIP_EPILOGUE_SUMS");
  if (sums && sums[0] == '0') return -1;
  const rgplan::Attn& at = sj.attn;
  rgk::AttnArgs a{};
  a.bh = (uint32_t)at.bh;
  a.heads = (uint32_t)at.heads;
  a.tq = (int)at.tq;
  a.tk = (int)at.tk;
  a.hd = (int)at.hd;
  if (at.heads <= 0 || !rgk::attention_backward_column_sums(a)) return -1;
  const int64_t slot = at.out[0].slot, L = at.out[0].st, B = at.bh / at.heads;
  std::vector<int> seen((size_t)std::max<int64_t>(L, 0), 0);
  for (const auto& v : at.out) {
    if (v.slot != slot || v.st != L || v.sb != at.tq * L || v.offset < 0) return -1;
    for (int64_t h = 0; h < at.heads; h++)
      for (int64_t c = 0; c < at.hd; c++) {
        const int64_t col = v.offset + h * v.sh + c;
        if (col < 0 || col >= L || seen[(size_t)col]++) return -1;
      }
  }
  for (int x : seen)
    if (!x) return -1;
  for (size_t q = j + 1; q < plan.steps.size() && q <= j + 4; q++) {
    const Step& sq = plan.steps[q];
    if (sq.kind == RG_STEP_INSTR && is_control(sq.instr.op)) return -1;
    if (column_sum_of(sq, slot, (uint64_t)(B * at.tq * L), (uint64_t)L)) {
      for (size_t r = j + 1; r < q; r++)
        if (has_slot(step_writes(plan.steps[r]), slot)) return -1;
      return (int64_t)q;
    }
  }
  return -1;
}


Epilogues find_epilogues(const Plan& plan) {
  const auto& steps = plan.steps;
  const size_t n = steps.size();
  Epilogues ep{std::vector<int64_t>(n, -1), std::vector<bool>(n, false), std::vector<int64_t>(n, -1), std::vector<int64_t>(n, -1),
               std::vector<int>(n, -1)};
  const char* env = getenv("RG_HIP_EPILOGUE");
  if (env && env[0] == '0') return ep;
  const bool every = env && std::string(env) == "all";
  std::vector<std::vector<int64_t>> reads(n), writes(n);
  for (size_t q = 0; q < n; q++) {
    reads[q] = step_reads(steps[q]);
    writes[q] = step_writes(steps[q]);
  }
  std::vector<bool> taken(n, false);
  for (size_t j = 0; j < n; j++) {
    const Step& sj = steps[j];
    if (sj.kind != RG_STEP_FUSED || sj.fused.row_len != 0 || sj.fused.dtype != RG_F32) continue;
    const rgplan::Fused& f = sj.fused;
    if (fused_grid(f) <= MERGE_MAX_GRID) continue;
    bool kinds_ok = true;
    for (auto& in : f.inputs)
      kinds_ok = kinds_ok && (in.kind == RG_ARG_FULL || in.kind == RG_ARG_SPLAT || (in.kind == RG_ARG_ROW && in.row_len % 4 == 0));
    if (!kinds_ok) continue;
    // The product: the latest earlier writer of one of the group's Full inputs.
    for (auto& in : f.inputs) {
      if (in.kind != RG_ARG_FULL) continue;
      int64_t k = -1;
      for (size_t q = j; q-- > 0;)
        if (has_slot(writes[q], in.slot)) {
          k = (int64_t)q;
          break;
        }
      if (k < 0 || taken[(size_t)k]) continue;
      const Step& sk = steps[(size_t)k];
      if (sk.kind != RG_STEP_INSTR || sk.instr.dtype != RG_F32 || sk.instr.dst != in.slot) continue;
      uint64_t m, nn, kk;
      bool ta, tb;
      rgk::GemmTile tile;
      if (!flat_product(sk.instr, &m, &nn, &kk, &ta, &tb) || (uint64_t)f.n != m * nn) continue;
      if (!rgk::gemm_epilogue_tile(RG_F32, m, nn, kk, ta, tb, &tile)) continue;
      if (!every && (uint64_t)tile.tm * tile.tn < EPILOGUE_MIN_TILES) continue;
      bool ok = true;
      for (auto& o : f.outputs)
        for (auto& a : sk.instr.args) ok = ok && o.second != a.slot;
      bool hoist = ok, sink = ok;
      for (size_t q = (size_t)k + 1; q < j && (hoist || sink); q++) {
        const Step& sq = steps[q];
        if (sq.kind == RG_STEP_INSTR && is_control(sq.instr.op)) hoist = sink = false;
        for (auto& x : f.inputs) hoist = hoist && !has_slot(writes[q], x.slot);
        for (auto& o : f.outputs) hoist = hoist && !has_slot(writes[q], o.second) && !has_slot(reads[q], o.second);
        for (auto& a : sk.instr.args) sink = sink && !has_slot(writes[q], a.slot);
        sink = sink && !has_slot(writes[q], sk.instr.dst) && !has_slot(reads[q], sk.instr.dst);
      }
      if (!hoist && !sink) continue;
      ep.at[j] = k;
      ep.sunk[j] = !hoist;
      taken[(size_t)k] = true;
      // A column sum of one of the group's outputs a few steps later, with nothing between the
      // group and it overwriting that output: computed by the combined kernel from the values
      // it stores, summed in registers (a K-contiguous B, whole 16x16-MFMA tiles: every output
      // goes through put4). RG_HIP_EPILOGUE_SUMS=0 leaves it to its own kernel.
      const char* sums = getenv("RG_HIP_EPILOGUE_SUMS");
      if ((sums && sums[0] == '0') || !tb || tile.ms != 16 || tile.mode != rgk::GEMM_WHOLE_TILES) break;
      for (size_t q = j + 1; q < n && q <= j + 4; q++) {
        if (steps[q].kind == RG_STEP_INSTR && is_control(steps[q].instr.op)) break;
        int out = -1;
        for (size_t o = 0; o < f.outputs.size(); o++)
          if (column_sum_of(steps[q], f.outputs[o].second, m * nn, nn)) out = (int)o;
        if (out >= 0) {
          bool clear = true;
          for (size_t r = j + 1; r < q; r++) clear = clear && !has_slot(writes[r], f.outputs[(size_t)out].second);
          if (clear) {
            ep.sum_of[j] = (int64_t)q;
            ep.sum_in[q] = (int64_t)j;
            ep.sum_out[j] = out;
          }
          break;
        }
      }
      break;
    }
  }
  return ep;
}

StepFn lower_control(Program& prog, size_t k);
void place_bodies(Program& prog);

// Source of product `pk`'s kernel with fused step `j` as its epilogue (kernel `prefix`rge`pk`).
// The product's own output is still stored (`*store_c`) when a later step or the host reads it
// before it is next written.
std::string epilogue_source(const Plan& plan, size_t j, int64_t pk, const std::string& prefix, bool* store_c, rgjit::FusedKernel* fk,
                            int col_sum) {
  const Instr& pi = plan.steps[(size_t)pk].instr;
  const int64_t c = pi.dst;
  const bool keep = product_output_needed(plan, (size_t)pk, j);
  *store_c = keep;
  uint64_t m, nn, kk;
  bool ta, tb;
  rgk::GemmTile t;
  if (!flat_product(pi, &m, &nn, &kk, &ta, &tb) || !rgk::gemm_epilogue_tile(RG_F32, m, nn, kk, ta, tb, &t))
    throw std::runtime_error("product epilogue: the product does not fit a single tile kernel");
  return rgjit::generate_gemm(plan.steps[j].fused, c, keep, rgjit::ProductTile{t.bm, t.bn, t.bk, t.wm, t.wn, t.ms, t.mode, ta, tb},
                              prefix + "rge" + std::to_string(pk), fk, col_sum);
}

// Independent products launched as one kernel (rgk::gemm_group): two adjacent plain products
// (no epilogue) k and k + 1, and with them, when it fits, the nearest earlier plain product j
// moved down to step k (nothing between j and k writes j's operands or reads or writes its
// output), or else the product k + 2 moved up to step k; then, for a plain product k left alone,
// the nearest earlier one left alone moved down to it the same way. No member reads or writes
// what another writes, and the launches group at program build (MFMA products of one tile shape
// and a sequence of operand layouts instantiated for groups, or streamed products of at most
// eight rows, any mix of the row, dot and outer-product kernels).
// Step k launches them all, the others nothing; at run time a group whose operands turn out not
// to fit (alignment) is launched as single kernels, at step k. The results are the single
// launches'. RG_HIP_PAIR=0 turns this off.
void group_products(Program& prog, const std::vector<GemmFill>& fills, const std::vector<rgk::GemmArgs>& base,
                    std::vector<size_t>& fold_producer) {
  const size_t n = prog.plan.steps.size();
  prog.pair_of.assign(n, -1);
  const char* env = getenv("RG_HIP_PAIR");
  if (env && env[0] == '0') return;
  std::vector<bool> used(n, false);
  auto independent = [&](const std::vector<size_t>& ks) {
    for (size_t x : ks)
      for (size_t y : ks) {
        if (x == y) continue;
        const Instr &a = prog.plan.steps[x].instr, &b = prog.plan.steps[y].instr;
        if (a.dst == b.dst) return false;
        for (auto& arg : b.args)
          if (arg.slot == a.dst) return false;
      }
    return true;
  };
  auto compatible = [&](const std::vector<size_t>& ks) {
    std::vector<rgk::GemmArgs> g;
    for (size_t x : ks) g.push_back(base[x]);
    return rgk::gemm_group(nullptr, g.data(), (int)g.size(), false);
  };
  // Whether product j can run at step k > j instead: nothing between them writes its operands or
  // reads or writes its output, and no control flow intervenes.
  auto movable = [&](size_t j, size_t k) {
    const Instr& pj = prog.plan.steps[j].instr;
    for (size_t q = j + 1; q < k; q++) {
      const Step& sq = prog.plan.steps[q];
      if (sq.kind == RG_STEP_INSTR && is_control(sq.instr.op)) return false;
      const auto w = step_writes(sq), r = step_reads(sq);
      for (auto& arg : pj.args)
        if (has_slot(w, arg.slot)) return false;
      if (has_slot(w, pj.dst) || has_slot(r, pj.dst)) return false;
    }
    return true;
  };
  // The nearest earlier plain product not yet grouped, within four steps of k, that can run at
  // step k with `with` (the group it would join, k included).
  auto earlier = [&](size_t k, const std::vector<size_t>& with) -> int64_t {
    for (size_t j = k; j-- > 0 && j + 4 >= k;) {
      if (prog.plan.steps[j].kind == RG_STEP_INSTR && is_control(prog.plan.steps[j].instr.op)) return -1;
      if (used[j] || !fills[j]) continue;
      std::vector<size_t> g = {j};
      g.insert(g.end(), with.begin(), with.end());
      if (movable(j, k) && independent(g) && compatible(g)) return (int64_t)j;
    }
    return -1;
  };
  auto launch_together = [&](const std::vector<size_t>& members, size_t k) {
    std::vector<GemmFill> f;
    for (size_t x : members) {
      f.push_back(fills[x]);
      used[x] = true;
      if (x != k) {
        prog.pair_of[x] = (int64_t)k;
        prog.steps[x] = [](hipStream_t, void* const*, void*) {};
        // Its K-split partials are written at step k now: their fold is due after it.
        for (auto& fp : fold_producer)
          if (fp == x) fp = k;
      }
    }
    prog.steps[k] = [f](hipStream_t s, void* const* sl, void* wsp) {
      rgk::GemmArgs g[3];
      for (size_t i = 0; i < f.size(); i++) g[i] = f[i](sl, wsp);
      if (!rgk::gemm_group(s, g, (int)f.size()))
        for (size_t i = 0; i < f.size(); i++) rgk::gemm(s, g[i]);
    };
  };
  for (size_t k = 0; k + 1 < n; k++) {
    if (!fills[k] || !fills[k + 1] || used[k] || used[k + 1]) continue;
    std::vector<size_t> members = {k, k + 1};
    if (!independent(members) || !compatible(members)) continue;
    const int64_t j = earlier(k, members);
    if (j >= 0) {
      members.insert(members.begin(), (size_t)j);
    } else if (k + 2 < n && fills[k + 2] && !used[k + 2]) {
      // Or the product after the pair, which then runs two steps early.
      std::vector<size_t> three = {k, k + 1, k + 2};
      if (independent(three) && compatible(three)) members = three;
    }
    launch_together(members, k);
  }
  for (size_t k = 0; k < n; k++) {
    if (!fills[k] || used[k]) continue;
    const int64_t j = earlier(k, {k});
    if (j >= 0) launch_together({(size_t)j, k}, k);
  }
}

void build_program(Program& prog) {
  std::vector<size_t> fold_producer;  // per fold: the step of the row group that writes its partials
  std::ostringstream src;
  std::vector<rgjit::FusedKernel*> kernels;
  const size_t n_steps = prog.plan.steps.size();
  const Epilogues ep = find_epilogues(prog.plan);
  prog.epilogue_of = ep.at;
  prog.epilogue_sunk = ep.sunk;
  prog.absorbed_into.assign(n_steps, -1);
  // Column sums the attention backward computes (attention_column_sum): per attention step, the
  // sum step; per sum step, the attention step.
  std::vector<int64_t> attn_sum_of(n_steps, -1), attn_sum_in(n_steps, -1);
  for (size_t j = 0; j < n_steps; j++) {
    const int64_t q = attention_column_sum(prog.plan, j);
    if (q >= 0 && ep.sum_in[(size_t)q] < 0) {
      attn_sum_of[j] = q;
      attn_sum_in[(size_t)q] = (int64_t)j;
    }
  }
  std::vector<int64_t> epilogue_at(n_steps, -1);  // product step -> the group it computes
  for (size_t j = 0; j < n_steps; j++)
    if (ep.at[j] >= 0) epilogue_at[(size_t)ep.at[j]] = (int64_t)j;
  std::vector<rgjit::FusedKernel*> kernel_of(n_steps, nullptr);
  std::vector<bool> store_c(n_steps, false);
  std::vector<GemmFill> gemm_fills(n_steps);
  std::vector<rgk::GemmArgs> gemm_base(n_steps);
  for (size_t k = 0; k < n_steps; k++) {
    const Step& st = prog.plan.steps[k];
    if (st.kind == RG_STEP_FUSED || st.kind == RG_STEP_ROWS) {
      auto fk = std::make_unique<rgjit::FusedKernel>();
      const int64_t pk = prog.epilogue_of[k];
      if (pk >= 0) {
        bool keep = false;
        src << epilogue_source(prog.plan, k, pk, "", &keep, fk.get(), ep.sum_out[k]);
        store_c[(size_t)pk] = keep;
      } else if (st.kind == RG_STEP_ROWS) {
        src << rgjit::generate_rows(st.fused, "rgr" + std::to_string(k), fk.get());
      } else {
        src << rgjit::generate(st.fused, "rgf" + std::to_string(k), fk.get());
      }
      kernel_of[k] = fk.get();
      kernels.push_back(fk.get());
      prog.fused.push_back(std::move(fk));
    }
  }
  const auto sets = merge_sets(prog.plan);
  std::vector<rgjit::FusedKernel*> merged_kernels;
  for (auto [first, last] : sets) {
    std::vector<const rgplan::Fused*> parts;
    for (size_t j = first; j <= last; j++) parts.push_back(&prog.plan.steps[j].fused);
    auto fk = std::make_unique<rgjit::FusedKernel>();
    src << rgjit::generate_merged(parts, "rgm" + std::to_string(first), fk.get());
    kernels.push_back(fk.get());
    merged_kernels.push_back(fk.get());
    prog.fused.push_back(std::move(fk));
  }
  rgjit::compile(src.str(), kernels);
  prog.merged_at.assign(prog.plan.steps.size(), -1);
  for (size_t m = 0; m < sets.size(); m++) {
    auto [first, last] = sets[m];
    std::vector<const rgplan::Fused*> parts;
    for (size_t j = first; j <= last; j++) parts.push_back(&prog.plan.steps[j].fused);
    const std::vector<int64_t> slots = rgjit::merged_slots(parts);
    rgjit::FusedKernel* fk = merged_kernels[m];
    prog.merged_at[first] = (int64_t)m;
    prog.merged.push_back({first, last, [fk, slots](hipStream_t s, void* const* sl, void*) {
                             void* ptrs[MERGE_MAX_ARGS];
                             void* args[MERGE_MAX_ARGS];
                             for (size_t j = 0; j < slots.size(); j++) {
                               ptrs[j] = sl[slots[j]];
                               args[j] = &ptrs[j];
                             }
                             hipModuleLaunchKernel(fk->fn, fk->grid, 1, 1, rgjit::TPB, 1, 1, 0, s, args, nullptr);
                           }});
  }
  size_t fi = 0;
  for (size_t k = 0; k < prog.plan.steps.size(); k++) {
    const Step& st = prog.plan.steps[k];
    // The combined kernel of product pk and group j, run at step k: with a column sum, its
    // partial rows (one per tile row) go to the fold area, folded like a reduction's.
    auto combined = [&](size_t pk, size_t j) {
      int64_t col_off = -1;
      if (ep.sum_of[j] >= 0) {
        const size_t q = (size_t)ep.sum_of[j];
        uint64_t m, nn, kk;
        bool ta, tb;
        rgk::GemmTile t;
        if (!flat_product(prog.plan.steps[pk].instr, &m, &nn, &kk, &ta, &tb) || !rgk::gemm_epilogue_tile(RG_F32, m, nn, kk, ta, tb, &t))
          throw std::runtime_error("product epilogue: the product no longer fits a single tile kernel");
        col_off = (int64_t)prog.fold_bytes;
        prog.folds.push_back({prog.fold_bytes, prog.plan.steps[q].instr.dst, t.tm, (uint32_t)nn, RG_REDUCE_SUM, RG_F32});
        fold_producer.push_back(k);
        prog.fold_bytes += ((uint64_t)t.tm * nn * 4 + 255) / 256 * 256;
        prog.absorbed_into[q] = (int64_t)k;
      }
      return lower_product_epilogue(prog.plan.steps[pk].instr, prog.plan.steps[j].fused, kernel_of[j], store_c[pk], &prog, col_off);
    };
    if ((st.kind == RG_STEP_FUSED || st.kind == RG_STEP_ROWS) && ep.at[k] >= 0) {
      // Computed by its product's kernel, run here when the product waits for this step.
      fi++;
      const size_t pk = (size_t)ep.at[k];
      if (ep.sunk[k]) prog.steps.push_back(combined(pk, k));
      else prog.steps.push_back([](hipStream_t, void* const*, void*) {});
      continue;
    }
    if (st.kind == RG_STEP_INSTR && epilogue_at[k] >= 0) {
      const size_t j = (size_t)epilogue_at[k];
      if (ep.sunk[j]) prog.steps.push_back([](hipStream_t, void* const*, void*) {});
      else prog.steps.push_back(combined(k, j));
      continue;
    }
    if (st.kind == RG_STEP_INSTR && (ep.sum_in[k] >= 0 || attn_sum_in[k] >= 0)) {
      // A column sum computed by the combined kernel of the group it reads, or by the attention
      // backward whose gradients it reads.
      prog.steps.push_back([](hipStream_t, void* const*, void*) {});
      continue;
    }
    if (st.kind == RG_STEP_FUSED || st.kind == RG_STEP_ROWS) {
      rgjit::FusedKernel* fk = prog.fused[fi++].get();
      std::vector<int64_t> ins, outs;
      for (auto& in : st.fused.inputs) ins.push_back(in.slot);
      for (auto& o : st.fused.outputs) outs.push_back(o.second);
      if (fk->grid == 0) {
        prog.steps.push_back([](hipStream_t, void* const*, void*) {});
        continue;
      }
      // Column outputs of a row group: partial rows in the fold area, folded later (folds_due).
      std::vector<uint64_t> col_off(outs.size(), UINT64_MAX);
      const int dtype = st.fused.dtype;
      for (size_t j = 0; j < outs.size() && !fk->col_kind.empty(); j++)
        if (fk->col_kind[j] >= 0) {
          col_off[j] = prog.fold_bytes;
          prog.folds.push_back({prog.fold_bytes, outs[j], fk->grid, fk->row_len, fk->col_kind[j], dtype});
          fold_producer.push_back(k);
          prog.fold_bytes += ((uint64_t)fk->grid * fk->row_len * esize(dtype) + 255) / 256 * 256;
        }
      if (ins.size() + outs.size() > 160) throw std::runtime_error("fused group with more than 160 operands");
      const Program* pp = &prog;
      prog.steps.push_back([fk, ins, outs, col_off, pp](hipStream_t s, void* const* sl, void* ws) {
        void* ptrs[160];
        void* args[160];
        size_t q = 0;
        for (auto x : ins) ptrs[q++] = sl[x];
        for (size_t j = 0; j < outs.size(); j++)
          ptrs[q++] = col_off[j] == UINT64_MAX ? sl[outs[j]] : (char*)ws + pp->fold_base() + col_off[j];
        for (size_t j = 0; j < q; j++) args[j] = &ptrs[j];
        hipModuleLaunchKernel(fk->fn, fk->grid, 1, 1, fk->block, 1, 1, 0, s, args, nullptr);
      });
    } else if (st.kind == RG_STEP_ATTN) {
      int64_t col_off = -1;
      if (attn_sum_of[k] >= 0) {
        const size_t q = (size_t)attn_sum_of[k];
        const uint64_t rows = (uint64_t)(st.attn.bh / st.attn.heads), len = (uint64_t)st.attn.out[0].st;
        col_off = (int64_t)prog.fold_bytes;
        prog.folds.push_back({prog.fold_bytes, prog.plan.steps[q].instr.dst, (uint32_t)rows, (uint32_t)len, RG_REDUCE_SUM, RG_F32});
        fold_producer.push_back(k);
        prog.fold_bytes += (rows * len * 4 + 255) / 256 * 256;
        prog.absorbed_into[q] = (int64_t)k;
      }
      prog.steps.push_back(lower_attention(prog, st.attn, col_off));
    } else if (is_control(st.instr.op)) {
      prog.steps.push_back(lower_control(prog, k));
    } else {
      const Instr& in = st.instr;
      if (in.op == RG_OP_MATMUL || in.op == RG_OP_MATMUL_T) {
        const bool ta = in.op == RG_OP_MATMUL_T && in.attr[0] != 0, tb = in.op == RG_OP_MATMUL_T && in.attr[1] != 0;
        gemm_fills[k] = gemm_fill(prog, in, ta, tb, &gemm_base[k]);
        prog.steps.push_back(gemm_step(gemm_fills[k]));
      } else {
        prog.steps.push_back(lower_instr(prog, in));
      }
      while (fold_producer.size() < prog.folds.size()) fold_producer.push_back(k);
    }
  }
  group_products(prog, gemm_fills, gemm_base, fold_producer);
  for (auto& s : prog.plan.slots) prog.slot_bytes.push_back(std::max<uint64_t>((uint64_t)s.cap * esize(s.dtype), 4));
  place_bodies(prog);
  // Each fold runs before the first later step reading its output, or right after its producer.
  const size_t n = prog.plan.steps.size();
  prog.folds_due.assign(n + 1, {});
  // A product and the group in its epilogue read their inputs at the step the combined kernel
  // runs at.
  auto reads_at = [&](size_t j) {
    std::vector<int64_t> r;
    // Products launched together read their operands at the step of the launch; a column sum
    // computed by a combined kernel reads nothing at its own step.
    if (prog.pair_of[j] >= 0 || prog.absorbed_into[j] >= 0) return r;
    bool grouped = false;
    for (size_t q = 0; q < n; q++)
      if (prog.pair_of[q] == (int64_t)j) {
        grouped = true;
        for (auto& a : prog.plan.steps[q].instr.args) r.push_back(a.slot);
      }
    if (grouped) {
      for (auto& a : prog.plan.steps[j].instr.args) r.push_back(a.slot);
      return r;
    }
    const bool combined_here = (ep.at[j] >= 0 && ep.sunk[j]) || (epilogue_at[j] >= 0 && !ep.sunk[(size_t)epilogue_at[j]]);
    const bool moved_away = (ep.at[j] >= 0 && !ep.sunk[j]) || (epilogue_at[j] >= 0 && ep.sunk[(size_t)epilogue_at[j]]);
    if (!moved_away && !combined_here) return step_reads(prog.plan.steps[j]);
    if (combined_here) {
      const size_t g = ep.at[j] >= 0 ? j : (size_t)epilogue_at[j];
      const size_t pk = (size_t)ep.at[g];
      for (auto& a : prog.plan.steps[pk].instr.args) r.push_back(a.slot);
      for (auto& in : prog.plan.steps[g].fused.inputs) r.push_back(in.slot);
    }
    return r;
  };
  for (size_t f = 0; f < prog.folds.size(); f++) {
    size_t due = fold_producer[f] + 1;
    for (size_t j = fold_producer[f] + 1; j < n; j++) {
      auto r = reads_at(j);
      if (std::find(r.begin(), r.end(), prog.folds[f].out_slot) != r.end()) {
        due = j;
        break;
      }
    }
    prog.folds_due[due].push_back(f);
  }
}

// Constants of a program and of its bodies (whose constants share the root program's blob).
void upload_consts(const Program& p, const std::vector<uint8_t>& blob, void* const* slots) {
  for (auto& c : p.plan.consts) {
    uint64_t bytes = (uint64_t)c.n * esize(p.plan.slots[(size_t)c.slot].dtype);
    if (c.offset < 0 || (uint64_t)c.offset + bytes > blob.size()) throw std::runtime_error("a constant lies outside the plan's blob");
    if (bytes) HIP_OK(hipMemcpy(slots[(size_t)c.slot], blob.data() + c.offset, bytes, hipMemcpyHostToDevice));
  }
  for (auto& ctl : p.control)
    if (ctl)
      for (auto& b : ctl->bodies) upload_consts(*b.prog, blob, slots + b.slot_base);
}

Frame* new_frame(Program& p) {
  auto* f = new Frame;
  uint64_t total = 0;
  std::vector<uint64_t> off;
  for (auto b : p.slot_bytes) {
    off.push_back(total);
    total += (b + ALIGN - 1) / ALIGN * ALIGN;
  }
  uint64_t ws_off = total;
  total += p.ws_bytes();
  total = std::max<uint64_t>(total, ALIGN);
  hipError_t e = hipMalloc(&f->arena, total);
  if (e != hipSuccess) {
    delete f;
    throw std::runtime_error("could not allocate a device frame of " + std::to_string(total) + " bytes: " + err_str(e));
  }
  f->bytes = total;
  HIP_OK(hipMemset(f->arena, 0, total));
  for (auto o : off) f->slot.push_back((char*)f->arena + o);
  f->workspace = (char*)f->arena + ws_off;
  HIP_OK(hipStreamCreateWithFlags(&f->stream, hipStreamNonBlocking));
  upload_consts(p, p.blob, f->slot.data());
  return f;
}

bool latch(Exec* e, hipError_t err, const char* what) {
  if (err == hipSuccess) return false;
  if (e->failure.empty()) e->failure = std::string(what) + ": " + err_str(err);
  return true;
}

// Runs the folds due before steps first..last: f32 ones together, FOLD_JOBS per launch.
void flush_folds(const Program& p, hipStream_t s, void* const* slots, void* ws, size_t first, size_t last) {
  if (p.folds.empty()) return;
  rgk::FoldJobs jobs;
  jobs.n = 0;
  uint32_t tiles = 0;
  rgk::WideFolds wide;
  wide.n = 0;
  uint32_t blocks = 0;
  char* base = (char*)ws + p.fold_base();
  for (size_t k = first; k <= last && k < p.folds_due.size(); k++)
    for (size_t f : p.folds_due[k]) {
      const auto& fd = p.folds[f];
      if (fd.wide) {
        wide.job[wide.n++] = {(const float*)(base + fd.offset), (float*)slots[fd.out_slot], fd.k, fd.rows, blocks};
        blocks += (fd.k + 1023) / 1024;
        if (wide.n == rgk::FOLD_JOBS) {
          rgk::fold_wide(s, wide, blocks);
          wide.n = 0;
          blocks = 0;
        }
        continue;
      }
      if (fd.dtype != RG_F32) {
        rgk::fold_rows(s, fd.dtype, fd.kind, base + fd.offset, slots[fd.out_slot], fd.rows, fd.k);
        continue;
      }
      jobs.job[jobs.n++] = {(const float*)(base + fd.offset), (float*)slots[fd.out_slot], fd.rows, fd.k, (uint32_t)fd.kind, tiles};
      tiles += (fd.k + 63) / 64;
      if (jobs.n == rgk::FOLD_JOBS) {
        rgk::fold_jobs(s, jobs, tiles);
        jobs.n = 0;
        tiles = 0;
      }
    }
  rgk::fold_jobs(s, jobs, tiles);
  rgk::fold_wide(s, wide, blocks);
}

// Enqueues plan steps begin..end-1, taking each merged run that lies wholly inside the range as
// its one kernel, and the folds due before each step.
void enqueue_range(const Program& p, hipStream_t s, void* const* slots, void* ws, size_t begin, size_t end) {
  for (size_t k = begin; k < end;) {
    int64_t m = p.merged_at.empty() ? -1 : p.merged_at[k];
    if (m >= 0 && p.merged[(size_t)m].last < end) {
      flush_folds(p, s, slots, ws, k, p.merged[(size_t)m].last);
      p.merged[(size_t)m].fn(s, slots, ws);
      k = p.merged[(size_t)m].last + 1;
    } else {
      flush_folds(p, s, slots, ws, k, k);
      p.steps[k](s, slots, ws);
      k++;
    }
  }
  if (end == p.steps.size()) flush_folds(p, s, slots, ws, end, end);
}

// Enqueues the listed steps in order, taking a merged run as its one kernel where the list holds
// all of its steps consecutively.
void enqueue_list(const Program& p, hipStream_t s, void* const* slots, void* ws, const int64_t* steps, size_t n) {
  for (size_t q = 0; q < n;) {
    size_t k = (size_t)steps[q];
    int64_t m = p.merged_at.empty() ? -1 : p.merged_at[k];
    if (m >= 0) {
      const auto& mr = p.merged[(size_t)m];
      size_t len = mr.last - mr.first + 1;
      bool whole = q + len <= n;
      for (size_t i = 0; whole && i < len; i++) whole = (size_t)steps[q + i] == k + i;
      if (whole) {
        flush_folds(p, s, slots, ws, mr.first, mr.last);
        mr.fn(s, slots, ws);
        q += len;
        continue;
      }
    }
    flush_folds(p, s, slots, ws, k, k);
    p.steps[k](s, slots, ws);
    q++;
  }
}

// ---- control flow (include/rg_plan.h SCAN / WHILE / COND; plan.rs:737-831) -------------------

// Copies gathered into batches of one launch each (rgk::copy_batch).
struct Copies {
  hipStream_t s;
  rgk::CopyJobs jobs{};
  void add(void* dst, const void* src, uint64_t bytes) {
    if (bytes == 0 || dst == src) return;
    if (jobs.n == rgk::COPY_JOBS) flush();
    jobs.dst[jobs.n] = (uint32_t*)dst;
    jobs.src[jobs.n] = (const uint32_t*)src;
    jobs.words[jobs.n] = bytes / 4;
    jobs.n++;
  }
  void flush() {
    rgk::copy_batch(s, jobs);
    jobs.n = 0;
  }
};

uint64_t input_bytes(const Program& p, size_t k) {
  const auto [slot, n] = p.plan.inputs[k];
  return (uint64_t)n * esize(p.plan.slots[(size_t)slot].dtype);
}

uint64_t output_bytes(const Program& p, size_t k) {
  const auto& o = p.plan.outputs[k];
  return (uint64_t)o.n * esize(p.plan.slots[(size_t)o.slot].dtype);
}

// Reads the first element of a slot as a double: a wait on the stream.
double read_scalar(hipStream_t s, const void* src, int dtype) {
  unsigned char raw[8] = {0};
  if (hipMemcpyAsync(raw, src, (size_t)esize(dtype), hipMemcpyDeviceToHost, s) != hipSuccess || hipStreamSynchronize(s) != hipSuccess)
    return 0.0;  // the failure surfaces at the caller's next wait
  if (dtype == RG_F32) {
    float v;
    memcpy(&v, raw, 4);
    return v;
  }
  if (dtype == RG_F64) {
    double v;
    memcpy(&v, raw, 8);
    return v;
  }
  int32_t v;
  memcpy(&v, raw, 4);
  return v;
}

// The body's carry results into its carry inputs, all read before any is written.
void feed_carry(hipStream_t s, const Program::Control& c, const Program& b, void* const* bs, void* ws) {
  Copies cp{s};
  const size_t nc = (size_t)c.attr.n_carry;
  if (!c.stage_carries) {
    for (size_t k = 0; k < nc; k++) cp.add(bs[(size_t)b.plan.inputs[k].first], bs[(size_t)b.plan.outputs[k].slot], input_bytes(b, k));
    cp.flush();
    return;
  }
  char* temp = (char*)ws + c.temp_offset;
  uint64_t at = 0;
  for (size_t k = 0; k < nc; k++) {
    cp.add(temp + at, bs[(size_t)b.plan.outputs[k].slot], input_bytes(b, k));
    at += (input_bytes(b, k) + ALIGN - 1) / ALIGN * ALIGN;
  }
  cp.flush();
  at = 0;
  for (size_t k = 0; k < nc; k++) {
    cp.add(bs[(size_t)b.plan.inputs[k].first], temp + at, input_bytes(b, k));
    at += (input_bytes(b, k) + ALIGN - 1) / ALIGN * ALIGN;
  }
  cp.flush();
}

void run_scan(hipStream_t s, const Program::Control& c, const Instr& in, void* const* sl, void* ws) {
  const Program::BodyProg& bp = c.bodies[0];
  const Program& b = *bp.prog;
  void* const* bs = sl + bp.slot_base;
  void* bws = (char*)ws + bp.ws_offset;
  const size_t nc = (size_t)c.attr.n_carry, nx = (size_t)c.attr.n_x, len = (size_t)c.attr.length;
  const size_t n_y = b.plan.outputs.size() - nc;
  Copies cp{s};
  // Carries and captures once; the x slices every step.
  for (size_t k = 0; k < in.args.size(); k++)
    if (k < nc || k >= nc + nx) cp.add(bs[(size_t)b.plan.inputs[k].first], sl[(size_t)in.args[k].slot], input_bytes(b, k));
  cp.flush();
  for (size_t step = 0; step < len; step++) {
    const size_t at = c.attr.reverse ? len - 1 - step : step;
    for (size_t k = nc; k < nc + nx; k++) {
      const uint64_t bytes = input_bytes(b, k);
      cp.add(bs[(size_t)b.plan.inputs[k].first], (char*)sl[(size_t)in.args[k].slot] + at * bytes, bytes);
    }
    for (auto [index, dst] : c.attr.results)
      if ((size_t)index >= nc + n_y) {
        const size_t k = (size_t)index - nc - n_y;
        const uint64_t bytes = input_bytes(b, k);
        cp.add((char*)sl[(size_t)dst] + at * bytes, bs[(size_t)b.plan.inputs[k].first], bytes);
      }
    cp.flush();
    enqueue_range(b, s, bs, bws, 0, b.steps.size());
    for (auto [index, dst] : c.attr.results)
      if ((size_t)index >= nc && (size_t)index < nc + n_y) {
        const uint64_t bytes = output_bytes(b, (size_t)index);
        cp.add((char*)sl[(size_t)dst] + at * bytes, bs[(size_t)b.plan.outputs[(size_t)index].slot], bytes);
      }
    cp.flush();
    feed_carry(s, c, b, bs, ws);
  }
  for (auto [index, dst] : c.attr.results)
    if ((size_t)index < nc) cp.add(sl[(size_t)dst], bs[(size_t)b.plan.inputs[(size_t)index].first], input_bytes(b, (size_t)index));
  cp.flush();
}

void run_while(hipStream_t s, const Program::Control& c, const Instr& in, void* const* sl, void* ws) {
  const Program &cb = *c.bodies[0].prog, &bb = *c.bodies[1].prog;
  void* const* cs = sl + c.bodies[0].slot_base;
  void* const* bs = sl + c.bodies[1].slot_base;
  void* cws = (char*)ws + c.bodies[0].ws_offset;
  void* bws = (char*)ws + c.bodies[1].ws_offset;
  const size_t nc = (size_t)c.attr.n_carry;
  Copies cp{s};
  for (size_t k = 0; k < in.args.size(); k++) {
    cp.add(cs[(size_t)cb.plan.inputs[k].first], sl[(size_t)in.args[k].slot], input_bytes(cb, k));
    cp.add(bs[(size_t)bb.plan.inputs[k].first], sl[(size_t)in.args[k].slot], input_bytes(bb, k));
  }
  cp.flush();
  const auto& co = cb.plan.outputs[0];
  int64_t count = 0;
  for (;;) {
    enqueue_range(cb, s, cs, cws, 0, cb.steps.size());
    if (read_scalar(s, cs[(size_t)co.slot], cb.plan.slots[(size_t)co.slot].dtype) == 0.0 || count == c.attr.max_iterations) break;
    enqueue_range(bb, s, bs, bws, 0, bb.steps.size());
    feed_carry(s, c, bb, bs, ws);
    for (size_t k = 0; k < nc; k++) cp.add(cs[(size_t)cb.plan.inputs[k].first], bs[(size_t)bb.plan.inputs[k].first], input_bytes(bb, k));
    cp.flush();
    count++;
  }
  for (auto [index, dst] : c.attr.results) {
    if ((size_t)index < nc) cp.add(sl[(size_t)dst], bs[(size_t)bb.plan.inputs[(size_t)index].first], input_bytes(bb, (size_t)index));
    else rgk::set_i32(s, (int32_t*)sl[(size_t)dst], (int32_t)count);
  }
  cp.flush();
}

void run_cond(hipStream_t s, const Program::Control& c, const Program& owner, const Instr& in, void* const* sl, void* ws) {
  const int pd = owner.plan.slots[(size_t)in.args[0].slot].dtype;
  const size_t j = read_scalar(s, sl[(size_t)in.args[0].slot], pd) != 0.0 ? 0 : 1;
  const Program& b = *c.bodies[j].prog;
  void* const* bs = sl + c.bodies[j].slot_base;
  Copies cp{s};
  for (size_t k = 1; k < in.args.size(); k++) cp.add(bs[(size_t)b.plan.inputs[k - 1].first], sl[(size_t)in.args[k].slot], input_bytes(b, k - 1));
  cp.flush();
  enqueue_range(b, s, bs, (char*)ws + c.bodies[j].ws_offset, 0, b.steps.size());
  for (auto [index, dst] : c.attr.results) cp.add(sl[(size_t)dst], bs[(size_t)b.plan.outputs[(size_t)index].slot], output_bytes(b, (size_t)index));
  cp.flush();
}

// Every slot fits the device and the kernels' 32-bit element indexing.
// The HIP source of every fused kernel of a plan and of its control-flow bodies (each body's
// kernels under their own prefix), as the runtime generates it; `count` kernels.
std::string plan_source(const Plan& root, int* count) {
  std::ostringstream src;
  std::function<void(const Plan&, const std::string&)> add = [&](const Plan& plan, const std::string& prefix) {
    const Epilogues eps = find_epilogues(plan);
    const std::vector<int64_t>& epi = eps.at;
    for (size_t k = 0; k < plan.steps.size(); k++) {
      const auto& st = plan.steps[k];
      if (st.kind == RG_STEP_INSTR && is_control(st.instr.op)) {
        const ControlAttr c = parse_control(st.instr);
        for (size_t j = 0; j < c.bodies.size(); j++)
          add(parse(c.bodies[j].first, c.bodies[j].second), prefix + "b" + std::to_string(k) + "_" + std::to_string(j) + "_");
        continue;
      }
      if (st.kind != RG_STEP_FUSED && st.kind != RG_STEP_ROWS) continue;
      rgjit::FusedKernel fk;
      bool keep;
      if (epi[k] >= 0) src << epilogue_source(plan, k, epi[k], prefix, &keep, &fk, eps.sum_out[k]);
      else if (st.kind == RG_STEP_ROWS) src << rgjit::generate_rows(st.fused, prefix + "rgr" + std::to_string(k), &fk);
      else src << rgjit::generate(st.fused, prefix + "rgf" + std::to_string(k), &fk);
      (*count)++;
    }
    for (auto [first, last] : merge_sets(plan)) {
      std::vector<const rgplan::Fused*> parts;
      for (size_t j = first; j <= last; j++) parts.push_back(&plan.steps[j].fused);
      rgjit::FusedKernel fk;
      src << rgjit::generate_merged(parts, prefix + "rgm" + std::to_string(first), &fk);
      (*count)++;
    }
  };
  add(root, "");
  return src.str();
}

void check_slots(const Plan& plan) {
  size_t free_b = 0, total = 0;
  HIP_OK(hipMemGetInfo(&free_b, &total));
  for (auto& s : plan.slots) {
    uint64_t bytes = (uint64_t)s.cap * esize(s.dtype);
    if (bytes > total)
      throw std::runtime_error("a " + std::string(s.dtype == RG_F64 ? "float64" : s.dtype == RG_F32 ? "float32" : "int32") + " buffer of " +
                               std::to_string(s.cap) + " elements exceeds this device's limit of " + std::to_string(total) + " bytes");
    if (s.cap >= (1ll << 31)) throw std::runtime_error("a buffer of " + std::to_string(s.cap) + " elements exceeds the 2^31 element index range");
  }
}


// A body's plan as a program of its own (kernels compiled, nested bodies placed).
std::unique_ptr<Program> body_program(const int64_t* w, size_t n, int device) {
  auto b = std::make_unique<Program>();
  b->plan = parse(w, n);
  b->device = device;
  check_slots(b->plan);
  build_program(*b);
  return b;
}

StepFn lower_control(Program& prog, size_t k) {
  const Instr& in = prog.plan.steps[k].instr;
  auto c = std::make_unique<Program::Control>();
  c->op = in.op;
  c->attr = parse_control(in);
  for (auto [w, n] : c->attr.bodies) {
    Program::BodyProg bp;
    bp.prog = body_program(w, n, prog.device);
    c->bodies.push_back(std::move(bp));
  }
  c->attr.bodies.clear();  // they pointed into the plan words
  // Check the body signatures against the step before anything runs.
  const size_t nc = (size_t)c->attr.n_carry;
  for (auto& bp : c->bodies) {
    const Plan& bpl = bp.prog->plan;
    const size_t want_in = c->op == RG_OP_COND ? in.args.size() - 1 : in.args.size();
    if (bpl.inputs.size() != want_in) throw std::runtime_error("control-flow body has the wrong number of inputs");
    prog.host_sync |= bp.prog->host_sync;
  }
  if (c->op != RG_OP_SCAN) prog.host_sync = true;
  for (auto [index, slot] : c->attr.results)
    if (index < 0 || slot < 0 || (size_t)slot >= prog.plan.slots.size()) throw std::runtime_error("control-flow result out of range");
  const Program& body = *c->bodies[c->op == RG_OP_WHILE ? 1 : 0].prog;
  if (c->op != RG_OP_COND) {
    if (body.plan.outputs.size() < nc || body.plan.inputs.size() < nc) throw std::runtime_error("control-flow body lacks its carries");
    // Staging when a carry result shares a buffer with the input of another carry.
    for (size_t a = 0; a < nc; a++)
      for (size_t q = 0; q < nc; q++)
        if (a != q && body.plan.outputs[a].slot == body.plan.inputs[q].first) c->stage_carries = true;
  }
  Program::Control* ctl = c.get();
  const Program* owner = &prog;
  if (prog.control.size() < prog.plan.steps.size()) prog.control.resize(prog.plan.steps.size());
  prog.control[k] = std::move(c);
  return [ctl, owner, k](hipStream_t s, void* const* sl, void* ws) {
    const Instr& ins = owner->plan.steps[k].instr;
    if (ctl->op == RG_OP_SCAN) run_scan(s, *ctl, ins, sl, ws);
    else if (ctl->op == RG_OP_WHILE) run_while(s, *ctl, ins, sl, ws);
    else run_cond(s, *ctl, *owner, ins, sl, ws);
  };
}

// Places the bodies' slots after this program's in the slot table, and their workspaces and the
// carry staging areas after this program's fold area.
void place_bodies(Program& prog) {
  uint64_t ws = 0;
  for (auto& c : prog.control) {
    if (!c) continue;
    if (c->stage_carries) {
      c->temp_offset = prog.fold_base() + (prog.fold_bytes + 255) / 256 * 256 + ws;
      const Program& body = *c->bodies[c->op == RG_OP_WHILE ? 1 : 0].prog;
      for (size_t k = 0; k < (size_t)c->attr.n_carry; k++) ws += (input_bytes(body, k) + ALIGN - 1) / ALIGN * ALIGN;
    }
    for (auto& b : c->bodies) {
      b.slot_base = prog.slot_bytes.size();
      prog.slot_bytes.insert(prog.slot_bytes.end(), b.prog->slot_bytes.begin(), b.prog->slot_bytes.end());
      b.ws_offset = prog.fold_base() + (prog.fold_bytes + 255) / 256 * 256 + ws;
      ws += (b.prog->ws_bytes() + ALIGN - 1) / ALIGN * ALIGN;
    }
  }
  prog.body_ws_bytes = ws;
}

// Consumes one pass of the failure countdown: true when this pass is the one that fails.
bool injected_now(Program* p) {
  int64_t f = p->fail_in.load();
  while (f >= 0 && !p->fail_in.compare_exchange_weak(f, f - 1)) {
  }
  return f == 0;
}

void run_steps(Exec* e, size_t begin, size_t end) {
  if (!e->failure.empty()) return;
  if (injected_now(e->prog)) {
    e->failure = "injected failure";
    return;
  }
  Frame* f = e->frame;
  try {
    enqueue_range(*e->prog, f->stream, f->slot.data(), f->workspace, begin, end);
  } catch (std::exception& ex) {
    e->failure = ex.what();
    return;
  }
  if (latch(e, hipGetLastError(), "kernel launch")) return;
  latch(e, hipStreamSynchronize(f->stream), "device execution");
}

double now() { return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count(); }

// Where a run's buffers lie in one block of device memory (offsets from its start).
struct RunLayout {
  uint64_t counter = 0, hist = 0, bytes = 0, chunk = 1;
  std::vector<uint64_t> batches, temps;
  RunBuffers place(void* base) const {
    RunBuffers b;
    b.counter = (uint64_t*)((char*)base + counter);
    b.hist = (double*)((char*)base + hist);
    b.chunk = chunk;
    for (auto o : batches) b.batch_bufs.push_back((char*)base + o);
    for (auto o : temps) b.temps.push_back((char*)base + o);
    return b;
  }
};

RunLayout run_layout(const Program& p, const rg_run_desc* d, uint64_t chunk) {
  RunLayout lay;
  lay.chunk = chunk;
  auto take = [&](uint64_t bytes) {
    uint64_t at = lay.bytes;
    lay.bytes += (std::max<uint64_t>(bytes, 1) + ALIGN - 1) / ALIGN * ALIGN;
    return at;
  };
  lay.counter = take(8);
  lay.hist = take((uint64_t)std::max<int64_t>(d->n_history, 1) * chunk * 8);
  for (int64_t j = 0; j < d->n_data && d->n_batches > 1; j++) lay.batches.push_back(take(d->data_bytes[j] * (uint64_t)d->n_batches));
  for (int64_t c = 0; c < d->n_copies; c++) lay.temps.push_back(take(p.slot_bytes[(size_t)d->copies[3 * c + 1]]));
  return lay;
}

// Copies the run's cycled batches into their device buffers (no wait).
void upload_batches(const rg_run_desc* d, const RunBuffers& b, hipStream_t s) {
  for (int64_t j = 0; j < (int64_t)b.batch_bufs.size(); j++)
    for (int64_t k = 0; k < d->n_batches; k++)
      HIP_OK(hipMemcpyAsync((char*)b.batch_bufs[(size_t)j] + d->data_bytes[j] * k, d->batches[k * d->n_data + j], d->data_bytes[j],
                            hipMemcpyHostToDevice, s));
}

// Everything one step of the loop enqueues under slot table `t`: batch loads, the plan, history
// records, the state copies into the next table `next` (every source read before any
// destination is written, validate.rs:349-355) and the step counter.
void enqueue_run_step(const Program& p, hipStream_t s, void* ws, const rg_run_desc* d, const RunBuffers& b, const std::vector<void*>& t,
                      const std::vector<void*>& next) {
  for (int64_t j = 0; j < (int64_t)b.batch_bufs.size(); j++)
    rgk::load_batch(s, t[(size_t)d->data_slots[j]], b.batch_bufs[(size_t)j], d->data_bytes[j], d->n_batches, b.counter);
  enqueue_range(p, s, t.data(), ws, 0, p.steps.size());
  for (int64_t h = 0; h < d->n_history; h++) {
    int64_t sl = d->history_slots[h];
    rgk::record_history(s, p.plan.slots[(size_t)sl].dtype, t[(size_t)sl], b.hist + h * b.chunk, b.counter, b.chunk);
  }
  // The state copies, batched: straight from each output into the next table's input when no
  // destination is also a source, else through the temporaries (all sources read first).
  bool overlap = false;
  for (int64_t c = 0; c < d->n_copies && !overlap; c++)
    for (int64_t q = 0; q < d->n_copies && !overlap; q++)
      overlap = next[(size_t)d->copies[3 * c]] == t[(size_t)d->copies[3 * q + 1]];
  Copies cp{s};
  for (int64_t c = 0; c < d->n_copies; c++) {
    int64_t is = d->copies[3 * c], os = d->copies[3 * c + 1], n = d->copies[3 * c + 2];
    cp.add(overlap ? b.temps[(size_t)c] : next[(size_t)is], t[(size_t)os], (uint64_t)n * esize(p.plan.slots[(size_t)os].dtype));
  }
  cp.flush();
  if (overlap) {
    for (int64_t c = 0; c < d->n_copies; c++) {
      int64_t is = d->copies[3 * c], os = d->copies[3 * c + 1], n = d->copies[3 * c + 2];
      cp.add(next[(size_t)is], b.temps[(size_t)c], (uint64_t)n * esize(p.plan.slots[(size_t)os].dtype));
    }
    cp.flush();
  }
  rgk::counter_inc(s, b.counter);
}

// The two slot tables a run alternates between: `start`, and `start` with every swap applied.
// Refuses a run description whose sizes or pointers do not fit this program before anything is
// copied or launched: every slot index in range; swapped slots pairwise disjoint, of one dtype
// and capacity; copies within both slots and of one dtype; data inputs within their slots, with
// a host pointer for every cycled batch; history slots holding at least one value and a history
// buffer to receive them. An empty string means the description is usable.
std::string check_run_desc(const Program& p, const rg_run_desc* d) {
  const int64_t n_slots = (int64_t)p.plan.slots.size();
  auto slot_ok = [&](int64_t s) { return s >= 0 && s < n_slots; };
  auto cap = [&](int64_t s) { return p.plan.slots[(size_t)s].cap; };
  auto dtype = [&](int64_t s) { return p.plan.slots[(size_t)s].dtype; };
  std::ostringstream why;
  if (!d) return "no run description";
  if (d->steps < 0 || d->n_swaps < 0 || d->n_copies < 0 || d->n_data < 0 || d->n_batches < 0 || d->n_history < 0)
    return "negative count in the run description";
  if ((d->n_swaps && !d->swaps) || (d->n_copies && !d->copies) || (d->n_data && (!d->data_slots || !d->data_bytes)) ||
      (d->n_history && !d->history_slots))
    return "a run description list is missing";
  std::vector<char> swapped((size_t)n_slots, 0);
  for (int64_t k = 0; k < d->n_swaps; k++) {
    int64_t a = d->swaps[2 * k], b = d->swaps[2 * k + 1];
    if (!slot_ok(a) || !slot_ok(b) || a == b) {
      why << "swap " << k << " names slots " << a << " and " << b << " of " << n_slots;
      return why.str();
    }
    if (swapped[(size_t)a] || swapped[(size_t)b]) {
      why << "slot " << (swapped[(size_t)a] ? a : b) << " is in two swaps";
      return why.str();
    }
    swapped[(size_t)a] = swapped[(size_t)b] = 1;
    if (dtype(a) != dtype(b) || cap(a) != cap(b) || p.slot_bytes[(size_t)a] != p.slot_bytes[(size_t)b]) {
      why << "swap " << k << ": slots " << a << " and " << b << " differ in dtype or capacity";
      return why.str();
    }
  }
  for (int64_t c = 0; c < d->n_copies; c++) {
    int64_t is = d->copies[3 * c], os = d->copies[3 * c + 1], n = d->copies[3 * c + 2];
    if (!slot_ok(is) || !slot_ok(os) || n < 0 || n > cap(is) || n > cap(os) || dtype(is) != dtype(os)) {
      why << "copy " << c << " of " << n << " values from slot " << os << " to slot " << is << " does not fit them";
      return why.str();
    }
  }
  for (int64_t j = 0; j < d->n_data; j++) {
    int64_t s = d->data_slots[j];
    if (!slot_ok(s) || d->data_bytes[j] > (uint64_t)cap(s) * (uint64_t)esize(dtype(s))) {
      why << "data input " << j << " (" << d->data_bytes[j] << " bytes) does not fit slot " << s;
      return why.str();
    }
    if (d->n_batches > 1) {
      if (!d->batches) return "cycled batches without batch pointers";
      for (int64_t b = 0; b < d->n_batches; b++)
        if (d->data_bytes[j] && !d->batches[b * d->n_data + j]) {
          why << "batch " << b << " has no host pointer for data input " << j;
          return why.str();
        }
    }
  }
  for (int64_t h = 0; h < d->n_history; h++) {
    int64_t s = d->history_slots[h];
    if (!slot_ok(s) || cap(s) < 1) {
      why << "history slot " << s << " holds no value";
      return why.str();
    }
  }
  if (d->n_history && d->steps && !d->history) return "history slots without a history buffer";
  return "";
}

void run_tables(const std::vector<void*>& start, const rg_run_desc* d, std::vector<void*> out[2]) {
  out[0] = start;
  out[1] = start;
  for (int64_t k = 0; k < d->n_swaps; k++) std::swap(out[1][(size_t)d->swaps[2 * k]], out[1][(size_t)d->swaps[2 * k + 1]]);
}

}  // namespace

extern "C" {

int rg_hip_available(void) {
  static int avail = [] {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return 0;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, 0) != hipSuccess) return 0;
    return strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
  }();
  return avail;
}

int rg_hip_gemm_streamed(int32_t dtype, int64_t m, int64_t n, int64_t k, int64_t batch, int32_t ta, int32_t tb) {
  if (m <= 0 || n <= 0 || k <= 0 || batch <= 0) return 0;
  return rgk::gemm_streamed(dtype, (uint64_t)m, (uint64_t)n, (uint64_t)k, (uint64_t)batch, ta != 0, tb != 0) ? 1 : 0;
}

int rg_hip_device_peaks(double* peaks, char* name, size_t len) {
  int dev = 0, n = 0;
  hipDeviceProp_t prop;
  if (hipGetDeviceCount(&n) != hipSuccess || n == 0 || hipGetDevice(&dev) != hipSuccess ||
      hipGetDeviceProperties(&prop, dev) != hipSuccess) {
    put(name, len, "no HIP device is visible");
    return 1;
  }
  // AMD's published dense figures: HBM3E at 8 TB/s; fp32 and fp64 matrix-core peaks.
  struct Part {
    const char* name;
    double hbm_gbs, fp32_tflops, fp64_tflops;
  };
  static const Part parts[] = {{"MI355X", 8000.0, 157.3, 78.6}, {"MI350X", 8000.0, 144.2, 72.1}};
  for (const Part& p : parts)
    if (strstr(prop.name, p.name)) {
      peaks[0] = p.hbm_gbs;
      peaks[1] = p.fp32_tflops;
      peaks[2] = p.fp64_tflops;
      put(name, len, std::string("AMD Instinct ") + p.name);
      return 0;
    }
  if (strncmp(prop.gcnArchName, "gfx950", 6) == 0 && prop.clockRate > 0) {
    // Another CDNA4 part: 256 fp32 (128 fp64) matrix flops per clock per CU at its peak clock.
    const double ghz = prop.clockRate / 1e6;
    peaks[0] = 8000.0;
    peaks[1] = 256.0 * prop.multiProcessorCount * ghz / 1000.0;
    peaks[2] = peaks[1] / 2.0;
    put(name, len, std::string(prop.name[0] ? prop.name : "gfx950") + ", " + std::to_string(prop.multiProcessorCount) + " CUs at " +
                       std::to_string(prop.clockRate / 1000) + " MHz (compute peaks from CU count and clock)");
    return 0;
  }
  put(name, len, std::string("no published peaks for ") + prop.name + " (" + prop.gcnArchName + ")");
  return 1;
}

uint64_t rg_hip_device_memory_bytes(void) {
  size_t free_b = 0, total = 0;
  if (hipMemGetInfo(&free_b, &total) != hipSuccess) return 0;
  return total;
}

void* rg_hip_program_new(const int64_t* words, size_t n_words, const void* blob, size_t blob_bytes, char* err, size_t err_len) {
  auto* p = new Program;
  try {
    if (!rg_hip_available()) throw std::runtime_error("no gfx950 device is visible to HIP");
    p->plan = parse(words, n_words);
    p->blob.assign((const uint8_t*)blob, (const uint8_t*)blob + blob_bytes);
    check_slots(p->plan);
    build_program(*p);
    return p;
  } catch (std::exception& e) {
    put(err, err_len, e.what());
    delete p;
    return nullptr;
  }
}

void rg_hip_program_free(void* program) { delete (Program*)program; }

// Generates and compiles every fused group of a plan for gfx950 without touching a device:
// the build-time check of the code generator. Returns the number of kernels, or -1.
int rg_hip_compile_check(const int64_t* words, size_t n_words, char* err, size_t err_len) {
  try {
    int count = 0;
    const std::string src = plan_source(parse(words, n_words), &count);
    if (count) rgjit::compile_code(src);
    return count;
  } catch (std::exception& e) {
    put(err, err_len, e.what());
    return -1;
  }
}

int rg_hip_kernel_source(const int64_t* words, size_t n_words, char* buf, size_t len) {
  try {
    int count = 0;
    const std::string src = plan_source(parse(words, n_words), &count);
    put(buf, len, src);
    return src.size() + 1 <= len ? count : -2;
  } catch (std::exception& e) {
    put(buf, len, e.what());
    return -1;
  }
}

uint64_t rg_hip_program_allocated_bytes(void* program) {
  (void)program;
  size_t free_b = 0, total = 0;
  if (hipMemGetInfo(&free_b, &total) != hipSuccess) return 0;
  return total - free_b;
}

int64_t rg_hip_program_step_runs_in(void* program, int64_t step) {
  const auto* p = (const Program*)program;
  if (step < 0 || (size_t)step >= p->plan.steps.size()) return -1;
  const size_t k = (size_t)step;
  if (p->pair_of[k] >= 0) return p->pair_of[k];
  if (p->absorbed_into[k] >= 0) return p->absorbed_into[k];
  if (p->epilogue_of[k] >= 0) return p->epilogue_sunk[k] ? step : p->epilogue_of[k];
  for (size_t j = 0; j < p->epilogue_of.size(); j++)
    if (p->epilogue_of[j] == step && p->epilogue_sunk[j]) return (int64_t)j;
  return step;
}

void rg_hip_program_inject_failure(void* program) { ((Program*)program)->fail_in = 0; }

void rg_hip_program_inject_failure_after(void* program, int64_t steps) { ((Program*)program)->fail_in = std::max<int64_t>(steps, 0); }

void* rg_hip_exec_new(void* program, char* err, size_t err_len) {
  auto* p = (Program*)program;
  auto* e = new Exec{p, nullptr, {}};
  {
    std::lock_guard<std::mutex> lock(p->mu);
    if (!p->pool.empty()) {
      e->frame = p->pool.back();
      p->pool.pop_back();
      return e;
    }
  }
  try {
    e->frame = new_frame(*p);
  } catch (std::exception& ex) {
    put(err, err_len, ex.what());
    delete e;
    return nullptr;
  }
  return e;
}

void rg_hip_exec_free(void* exec) {
  auto* e = (Exec*)exec;
  hipStreamSynchronize(e->frame->stream);
  {
    std::lock_guard<std::mutex> lock(e->prog->mu);
    e->prog->pool.push_back(e->frame);
  }
  delete e;
}

int rg_hip_exec_write(void* exec, int64_t slot, const void* src, uint64_t bytes) {
  auto* e = (Exec*)exec;
  if (slot < 0 || (size_t)slot >= e->frame->slot.size() || bytes > e->prog->slot_bytes[(size_t)slot]) return -1;
  if (!bytes) return 0;
  if (latch(e, hipMemcpyAsync(e->frame->slot[(size_t)slot], src, bytes, hipMemcpyHostToDevice, e->frame->stream), "write")) return -1;
  return latch(e, hipStreamSynchronize(e->frame->stream), "write") ? -1 : 0;
}

// Batches of slot copies at least this large go through the frame's pinned staging.
constexpr uint64_t STAGE_MIN_BYTES = 1ull << 20;

// Host copies of `pieces` (destination, source, bytes), the total split evenly over up to eight
// threads (at least 4 MiB each): one host thread copies well below the host's memory bandwidth.
void parallel_copy(const std::vector<std::tuple<char*, const char*, uint64_t>>& pieces) {
  uint64_t total = 0;
  for (auto& pc : pieces) total += std::get<2>(pc);
  const uint64_t hw = std::max(1u, std::thread::hardware_concurrency());
  const uint64_t nt = std::max<uint64_t>(1, std::min<uint64_t>(std::min<uint64_t>(8, hw), total >> 22));
  auto run = [&](uint64_t lo, uint64_t hi) {
    uint64_t at = 0;
    for (auto& [d, src, b] : pieces) {
      const uint64_t a = std::max(lo, at), end = std::min(hi, at + b);
      if (a < end) memcpy(d + (a - at), src + (a - at), end - a);
      at += b;
      if (at >= hi) break;
    }
  };
  std::vector<std::thread> threads;
  for (uint64_t t = 1; t < nt; t++) threads.emplace_back(run, total * t / nt, total * (t + 1) / nt);
  run(0, total / nt);
  for (auto& th : threads) th.join();
}

// Offsets of the copies' bytes in the staging (256-byte aligned each) and their total, or 0 when
// the batch is small or the staging cannot grow to it.
uint64_t stage_layout(Frame* f, int64_t n, const uint64_t* bytes, std::vector<uint64_t>* off) {
  uint64_t total = 0, payload = 0;
  for (int64_t k = 0; k < n; k++) {
    off->push_back(total);
    total += (bytes[k] + 255) / 256 * 256;
    payload += bytes[k];
  }
  if (payload < STAGE_MIN_BYTES) return 0;
  if (f->stage_bytes < total) {
    if (f->stage) hipHostFree(f->stage);
    f->stage = nullptr;
    f->stage_bytes = 0;
    if (hipHostMalloc(&f->stage, total, hipHostMallocDefault) != hipSuccess) {
      f->stage = nullptr;
      hipGetLastError();
      return 0;
    }
    f->stage_bytes = total;
  }
  return total;
}

int rg_hip_exec_write_slots(void* exec, int64_t n, const int64_t* slots, const void* const* srcs, const uint64_t* bytes) {
  auto* e = (Exec*)exec;
  Frame* f = e->frame;
  for (int64_t k = 0; k < n; k++)
    if (slots[k] < 0 || (size_t)slots[k] >= f->slot.size() || bytes[k] > e->prog->slot_bytes[(size_t)slots[k]]) return -1;
  std::vector<uint64_t> off;
  if (stage_layout(f, n, bytes, &off)) {
    // Into the pinned staging on several host threads, then one DMA per slot.
    std::vector<std::tuple<char*, const char*, uint64_t>> pieces;
    for (int64_t k = 0; k < n; k++) pieces.push_back({(char*)f->stage + off[(size_t)k], (const char*)srcs[k], bytes[k]});
    parallel_copy(pieces);
    for (int64_t k = 0; k < n; k++)
      if (bytes[k] && latch(e, hipMemcpyAsync(f->slot[(size_t)slots[k]], (char*)f->stage + off[(size_t)k], bytes[k], hipMemcpyHostToDevice, f->stream),
                            "write"))
        return -1;
    return latch(e, hipStreamSynchronize(f->stream), "write") ? -1 : 0;
  }
  for (int64_t k = 0; k < n; k++)
    if (bytes[k] && latch(e, hipMemcpyAsync(f->slot[(size_t)slots[k]], srcs[k], bytes[k], hipMemcpyHostToDevice, f->stream), "write"))
      return -1;
  return latch(e, hipStreamSynchronize(f->stream), "write") ? -1 : 0;
}

int rg_hip_exec_read_slots(void* exec, int64_t n, const int64_t* slots, void* const* dsts, const uint64_t* bytes) {
  auto* e = (Exec*)exec;
  Frame* f = e->frame;
  for (int64_t k = 0; k < n; k++)
    if (slots[k] < 0 || (size_t)slots[k] >= f->slot.size() || bytes[k] > e->prog->slot_bytes[(size_t)slots[k]]) return -1;
  std::vector<uint64_t> off;
  if (stage_layout(f, n, bytes, &off)) {
    // One DMA per slot into the pinned staging, then out of it on several host threads.
    for (int64_t k = 0; k < n; k++)
      if (bytes[k] && latch(e, hipMemcpyAsync((char*)f->stage + off[(size_t)k], f->slot[(size_t)slots[k]], bytes[k], hipMemcpyDeviceToHost, f->stream),
                            "read"))
        return -1;
    if (latch(e, hipStreamSynchronize(f->stream), "read")) return -1;
    std::vector<std::tuple<char*, const char*, uint64_t>> pieces;
    for (int64_t k = 0; k < n; k++) pieces.push_back({(char*)dsts[k], (const char*)f->stage + off[(size_t)k], bytes[k]});
    parallel_copy(pieces);
    return 0;
  }
  for (int64_t k = 0; k < n; k++)
    if (bytes[k] && latch(e, hipMemcpyAsync(dsts[k], f->slot[(size_t)slots[k]], bytes[k], hipMemcpyDeviceToHost, f->stream), "read"))
      return -1;
  return latch(e, hipStreamSynchronize(f->stream), "read") ? -1 : 0;
}

int rg_hip_exec_read(void* exec, int64_t slot, void* dst, uint64_t bytes) {
  auto* e = (Exec*)exec;
  if (slot < 0 || (size_t)slot >= e->frame->slot.size() || bytes > e->prog->slot_bytes[(size_t)slot]) return -1;
  if (!bytes) return 0;
  if (latch(e, hipMemcpyAsync(dst, e->frame->slot[(size_t)slot], bytes, hipMemcpyDeviceToHost, e->frame->stream), "read")) return -1;
  return latch(e, hipStreamSynchronize(e->frame->stream), "read") ? -1 : 0;
}

double rg_hip_exec_scalar(void* exec, int64_t slot) {
  auto* e = (Exec*)exec;
  int d = e->prog->plan.slots[(size_t)slot].dtype;
  uint8_t buf[8] = {0};
  if (rg_hip_exec_read(exec, slot, buf, esize(d)) != 0) return NAN;
  if (d == RG_F32) { float v; memcpy(&v, buf, 4); return v; }
  if (d == RG_F64) { double v; memcpy(&v, buf, 8); return v; }
  int32_t v;
  memcpy(&v, buf, 4);
  return v;
}

void rg_hip_exec_swap(void* exec, int64_t a, int64_t b) {
  auto* e = (Exec*)exec;
  std::swap(e->frame->slot[(size_t)a], e->frame->slot[(size_t)b]);
}

void rg_hip_exec_steps(void* exec, int64_t begin, int64_t end) { run_steps((Exec*)exec, (size_t)begin, (size_t)end); }

void rg_hip_exec_step(void* exec) { run_steps((Exec*)exec, 0, ((Exec*)exec)->prog->steps.size()); }

int rg_hip_exec_failure(void* exec, char* buf, size_t len) {
  auto* e = (Exec*)exec;
  if (e->failure.empty()) return 0;
  put(buf, len, e->failure);
  return 1;
}

int rg_hip_exec_step_timed(void* exec, double* seconds) {
  auto* e = (Exec*)exec;
  Frame* f = e->frame;
  size_t n = e->prog->steps.size();
  std::vector<hipEvent_t> ev(n + 1);
  for (auto& x : ev) hipEventCreate(&x);
  // The stream is held while every step and an event after each are enqueued, so the device
  // runs the steps back to back: the interval between consecutive events is then the step's
  // device time rather than host launch latency (metal.rs:690-698 times one command buffer per
  // step instead).
  rgk::hold_stream(f->stream, 3000.0 + 15.0 * (double)n);
  hipEventRecord(ev[0], f->stream);
  for (size_t k = 0; k < n; k++) {
    flush_folds(*e->prog, f->stream, f->slot.data(), f->workspace, k, k);
    e->prog->steps[k](f->stream, f->slot.data(), f->workspace);
    if (k + 1 == n) flush_folds(*e->prog, f->stream, f->slot.data(), f->workspace, n, n);
    hipEventRecord(ev[k + 1], f->stream);
  }
  if (!latch(e, hipEventSynchronize(ev[n]), "timed step")) {
    for (size_t k = 0; k < n; k++) {
      float ms = 0;
      hipEventElapsedTime(&ms, ev[k], ev[k + 1]);
      seconds[k] += ms * 1e-3;
    }
  }
  for (auto& x : ev) hipEventDestroy(x);
  return e->failure.empty() ? 0 : -1;
}

int rg_hip_exec_time_steps(void* exec, const int64_t* steps, int64_t n_steps, int64_t repeats, double* seconds) {
  auto* e = (Exec*)exec;
  Frame* f = e->frame;
  *seconds = 0.0;
  int64_t total = (int64_t)e->prog->steps.size();
  for (int64_t k = 0; k < n_steps; k++)
    if (steps[k] < 0 || steps[k] >= total) {
      latch(e, hipErrorInvalidValue, "time_steps: step index out of range");
      return -1;
    }
  if (n_steps == 0 || repeats <= 0) return 0;
  hipEvent_t a, b;
  hipEventCreate(&a);
  hipEventCreate(&b);
  // Hold the stream while the launches are enqueued, so the device never waits on the host.
  rgk::hold_stream(f->stream, 2000.0 + 4.0 * (double)(n_steps * repeats));
  hipEventRecord(a, f->stream);
  for (int64_t r = 0; r < repeats; r++) enqueue_list(*e->prog, f->stream, f->slot.data(), f->workspace, steps, (size_t)n_steps);
  hipEventRecord(b, f->stream);
  if (!latch(e, hipEventSynchronize(b), "time_steps")) {
    float ms = 0;
    hipEventElapsedTime(&ms, a, b);
    *seconds = ms * 1e-3;
  }
  hipEventDestroy(a);
  hipEventDestroy(b);
  return e->failure.empty() ? 0 : -1;
}

int rg_hip_exec_breakdown(void* exec, int64_t repeats, char* json, size_t len) {
  auto* e = (Exec*)exec;
  Frame* f = e->frame;
  repeats = std::max<int64_t>(repeats, 1);
  hipEvent_t a, b;
  hipEventCreate(&a);
  hipEventCreate(&b);
  double t0 = now();
  hipEventRecord(a, f->stream);
  for (int64_t r = 0; r < repeats && e->failure.empty(); r++)
    enqueue_range(*e->prog, f->stream, f->slot.data(), f->workspace, 0, e->prog->steps.size());
  hipEventRecord(b, f->stream);
  latch(e, hipEventSynchronize(b), "breakdown");
  double wall = now() - t0;
  float ms = 0;
  hipEventElapsedTime(&ms, a, b);
  hipEventDestroy(a);
  hipEventDestroy(b);
  size_t fused = 0;
  for (auto& st : e->prog->plan.steps) fused += st.kind == RG_STEP_FUSED || st.kind == RG_STEP_ROWS;
  std::ostringstream s;
  size_t launches = e->prog->steps.size();
  for (auto& m : e->prog->merged) launches -= m.last - m.first;
  s << "{\"wall_ms\":" << wall / repeats * 1e3 << ",\"gpu_ms\":" << ms / repeats << ",\"per_step\":{\"dispatches\":"
    << e->prog->steps.size() << ",\"fused_kernels\":" << fused << ",\"merged_launches\":" << e->prog->merged.size()
    << ",\"launches\":" << launches << ",\"cpu_steps\":0}}";
  put(json, len, s.str());
  return e->failure.empty() ? 0 : -1;
}

// The step loop on the device (validate.rs:289-363 semantics). Each step is a replay of one of
// two captured graphs: the swaps of the state handoff are disjoint pairs, so the slot table
// alternates between two permutations and each has its graph. Batches, history and the step
// counter live in device memory; history is read back once per chunk. Every chunk starts from a
// snapshot of the changing state slots: a non-finite value re-runs the chunk from it to stop
// exactly after the bad step's handoff, and a device failure puts the state back to the chunk
// start, so the state handed back always matches the completed steps. Graphs and buffers stay on
// the frame (RunCache) for the next run with the same description.
int rg_hip_exec_run(void* exec, const rg_run_desc* d, rg_run_result* out) {
  auto* e = (Exec*)exec;
  Program* p = e->prog;
  Frame* f = e->frame;
  out->done = 0;
  out->nonfinite_step = -1;
  out->seconds = 0;
  if (!e->failure.empty()) return -1;
  const std::string bad_desc = check_run_desc(*p, d);
  if (!bad_desc.empty()) {
    e->failure = "rg_hip_exec_run: " + bad_desc;
    return -1;
  }
  const int64_t fail_at = p->fail_in.exchange(-1);  // step index of an injected failure, or -1
  RunCache& rc = f->run;
  int result = 0;
  try {
    const int64_t steps = d->steps;
    const uint64_t chunk = d->n_history > 0 ? 64 : (uint64_t)std::max<int64_t>(steps, 1);
    const int n_graphs = d->n_swaps > 0 ? 2 : 1;
    // The run description: a cached run with the same one can be replayed as it is.
    std::vector<int64_t> key{d->n_swaps, d->n_copies, d->n_data, d->n_batches > 1 ? d->n_batches : 0, d->n_history, (int64_t)chunk};
    key.insert(key.end(), d->swaps, d->swaps + 2 * d->n_swaps);
    key.insert(key.end(), d->copies, d->copies + 3 * d->n_copies);
    key.insert(key.end(), d->data_slots, d->data_slots + d->n_data);
    for (int64_t j = 0; j < d->n_data; j++) key.push_back((int64_t)d->data_bytes[j]);
    key.insert(key.end(), d->history_slots, d->history_slots + d->n_history);
    auto tables_from = [&](const std::vector<void*>& start) { run_tables(start, d, rc.table); };
    if (rc.key != key) {
      rc.release();
      // One allocation: the run buffers, then the snapshot of the changing state slots.
      RunLayout lay = run_layout(*p, d, chunk);
      for (int64_t k = 0; k < d->n_swaps; k++) rc.state_slots.push_back(d->swaps[2 * k]);
      for (int64_t k = 0; k < d->n_copies; k++) rc.state_slots.push_back(d->copies[3 * k]);
      uint64_t total = lay.bytes;
      std::vector<uint64_t> snap_off;
      for (auto sl : rc.state_slots) {
        snap_off.push_back(total);
        total += (p->slot_bytes[(size_t)sl] + ALIGN - 1) / ALIGN * ALIGN;
      }
      HIP_OK(hipMalloc(&rc.mem, std::max<uint64_t>(total, ALIGN)));
      rc.mem_bytes = total;
      rc.buf = lay.place(rc.mem);
      for (auto o : snap_off) rc.snap.push_back((char*)rc.mem + o);
      rc.n_graphs = n_graphs;
      tables_from(f->slot);
      rc.key = key;
    } else if (f->slot != rc.table[0] && (n_graphs < 2 || f->slot != rc.table[1])) {
      // The frame's buffers were swapped outside a run: new tables, new graphs.
      rc.clear_graphs();
      tables_from(f->slot);
    }
    // Step k (counted from this run's start) runs under table (parity + k) % n_graphs.
    const int parity = f->slot == rc.table[0] ? 0 : 1;
    auto enqueue_step = [&](int g) { enqueue_run_step(*p, f->stream, f->workspace, d, rc.buf, rc.table[g], rc.table[(g + 1) % n_graphs]); };
    // Each slot table is captured once as a HIP graph and replayed; RG_HIP_GRAPHS=0 launches the
    // same kernels directly instead (for tools that do not follow graph launches).
    const char* env = getenv("RG_HIP_GRAPHS");
    const bool use_graphs = !(env && env[0] == '0') && !p->host_sync;
    if (use_graphs && rc.execs.empty()) {
      for (int g = 0; g < n_graphs; g++) {
        HIP_OK(hipStreamBeginCapture(f->stream, hipStreamCaptureModeThreadLocal));
        try {
          enqueue_step(g);
        } catch (...) {
          // End the capture before reporting, so the stream is usable again.
          hipGraph_t partial = nullptr;
          if (hipStreamEndCapture(f->stream, &partial) == hipSuccess && partial) hipGraphDestroy(partial);
          hipGetLastError();
          throw;
        }
        hipGraph_t graph;
        hipError_t ce = hipStreamEndCapture(f->stream, &graph);
        if (ce != hipSuccess) throw std::runtime_error("graph capture failed: " + err_str(ce));
        rc.graphs.push_back(graph);
        hipGraphExec_t ge;
        HIP_OK(hipGraphInstantiate(&ge, graph, nullptr, nullptr, 0));
        rc.execs.push_back(ge);
      }
    }
    upload_batches(d, rc.buf, f->stream);
    auto table_of = [&](int64_t k) { return (int)((parity + k) % n_graphs); };
    auto launch = [&](int64_t k) -> hipError_t {
      if (use_graphs) return hipGraphLaunch(rc.execs[(size_t)table_of(k)], f->stream);
      enqueue_step(table_of(k));
      return hipGetLastError();
    };
    // The changing state slots to or from the chunk's snapshot, COPY_JOBS slots per launch.
    auto snapshot = [&](int g, bool restore) {
      Copies cp{f->stream};
      for (size_t q = 0; q < rc.state_slots.size(); q++) {
        void* live = rc.table[g][(size_t)rc.state_slots[q]];
        uint64_t bytes = p->slot_bytes[(size_t)rc.state_slots[q]];
        cp.add(restore ? live : rc.snap[q], restore ? rc.snap[q] : live, bytes);
      }
      cp.flush();
    };
    HIP_OK(hipGetLastError());
    rgk::set_counter(f->stream, rc.buf.counter, 0);
    HIP_OK(hipStreamSynchronize(f->stream));
    double t0 = now();
    int64_t done = 0;
    std::vector<double> hbuf((size_t)std::max<int64_t>(d->n_history, 1) * chunk);
    while (done < steps) {
      int64_t c0 = done, c1 = std::min<int64_t>(steps, done + (int64_t)chunk);
      if (fail_at >= 0 && c0 >= fail_at) {
        // The injected failure: a device error before step c0, with every earlier step complete.
        e->failure = "injected failure";
        result = -1;
        break;
      }
      if (fail_at > c0) c1 = std::min<int64_t>(c1, fail_at);
      const int g0 = table_of(c0);
      snapshot(g0, false);
      bool failed = false;
      for (int64_t k = c0; k < c1 && !failed; k++) failed = latch(e, launch(k), "step launch");
      if (failed || latch(e, hipStreamSynchronize(f->stream), "device execution")) {
        // Back to the state before the chunk; if the device no longer runs copies, the state is
        // lost and the failure message stands for it.
        hipGetLastError();
        snapshot(g0, true);
        if (hipStreamSynchronize(f->stream) != hipSuccess) e->failure += " (state could not be restored)";
        result = -1;
        break;
      }
      int64_t bad = -1;
      if (d->n_history > 0) {
        HIP_OK(hipMemcpy(hbuf.data(), rc.buf.hist, (size_t)d->n_history * chunk * 8, hipMemcpyDeviceToHost));
        for (int64_t k = c0; k < c1 && bad < 0; k++)
          for (int64_t h = 0; h < d->n_history; h++)
            if (!std::isfinite(hbuf[(size_t)(h * chunk + (k - c0))])) bad = k;
        for (int64_t h = 0; h < d->n_history; h++)
          for (int64_t k = c0; k < (bad >= 0 ? bad + 1 : c1); k++) d->history[h * steps + k] = hbuf[(size_t)(h * chunk + (k - c0))];
      }
      if (bad >= 0) {
        // Back to the chunk start, then exactly through the bad step.
        snapshot(g0, true);
        rgk::set_counter(f->stream, rc.buf.counter, (uint64_t)c0);
        for (int64_t k = c0; k <= bad; k++) latch(e, launch(k), "step launch");
        if (latch(e, hipStreamSynchronize(f->stream), "device execution")) {
          result = -1;
          break;
        }
        done = bad + 1;
        out->nonfinite_step = bad;
        break;
      }
      done = c1;
    }
    out->seconds = now() - t0;
    out->done = done;
    // The frame's table reflects every handoff made.
    f->slot = rc.table[(size_t)table_of(done)];
  } catch (std::exception& ex) {
    if (e->failure.empty()) e->failure = ex.what();
    result = -1;
  }
  hipStreamSynchronize(f->stream);
  return result;
}

// The step loop with no allocation (include/rg_hip.h): the run's counter, history record, cycled
// batches and copy temporaries live in the static scratch array (noalloc.hip); the steps are
// launched directly (no graph is instantiated) and no snapshot is kept. With history, the loop
// waits after every step and reads the recorded values, so it stops exactly after the first
// step (and its handoff) that recorded a non-finite value, as rg_hip_exec_run does. A step
// counts as done only once a synchronization after it succeeded: without history that is the
// final one, so a device failure it reports leaves `done` at 0. The device's run lock is held for the
// whole call: overlapping calls on one GPU take turns.
int rg_hip_exec_run_noalloc(void* exec, const rg_run_desc* d, rg_run_result* out) {
  auto* e = (Exec*)exec;
  Program* p = e->prog;
  Frame* f = e->frame;
  out->done = 0;
  out->nonfinite_step = -1;
  out->seconds = 0;
  if (!e->failure.empty()) return -1;
  const std::string bad_desc = check_run_desc(*p, d);
  if (!bad_desc.empty()) {
    e->failure = "rg_hip_exec_run_noalloc: " + bad_desc;
    return -1;
  }
  const int64_t fail_at = p->fail_in.exchange(-1);
  std::string why;
  std::unique_lock<std::mutex> hold;
  void* base = rgk::noalloc_scratch(&why, &hold);
  if (!base) {
    e->failure = "rg_hip_exec_run_noalloc: " + why;
    return -1;
  }
  RunLayout lay = run_layout(*p, d, 1);
  if (lay.bytes > RG_NOALLOC_SCRATCH_BYTES) {
    e->failure = "rg_hip_exec_run_noalloc: this run needs " + std::to_string(lay.bytes) + " bytes of scratch (counter, history, " +
                 std::to_string(d->n_batches > 1 ? d->n_batches : 0) + " cycled batches, " + std::to_string(d->n_copies) +
                 " state copies); the static scratch holds " + std::to_string(RG_NOALLOC_SCRATCH_BYTES);
    return -1;
  }
  const RunBuffers b = lay.place(base);
  const int n_tables = d->n_swaps > 0 ? 2 : 1;
  std::vector<void*> table[2];
  run_tables(f->slot, d, table);
  int result = 0;
  int64_t enqueued = 0, done = 0;
  try {
    upload_batches(d, b, f->stream);
    rgk::set_counter(f->stream, b.counter, 0);
    HIP_OK(hipStreamSynchronize(f->stream));
    double t0 = now();
    std::vector<double> hbuf((size_t)std::max<int64_t>(d->n_history, 1));
    for (int64_t k = 0; k < d->steps; k++) {
      if (k == fail_at) {
        e->failure = "injected failure";
        result = -1;
        break;
      }
      enqueue_run_step(*p, f->stream, f->workspace, d, b, table[k % n_tables], table[(k + 1) % n_tables]);
      if (latch(e, hipGetLastError(), "step launch")) {
        result = -1;
        break;
      }
      enqueued = k + 1;
      if (d->n_history == 0) continue;
      // On the frame's stream: it does not synchronize with the null stream a plain hipMemcpy uses.
      if (latch(e, hipMemcpyAsync(hbuf.data(), b.hist, (size_t)d->n_history * 8, hipMemcpyDeviceToHost, f->stream), "history read") ||
          latch(e, hipStreamSynchronize(f->stream), "device execution")) {
        result = -1;
        break;
      }
      done = k + 1;
      bool bad = false;
      for (int64_t h = 0; h < d->n_history; h++) {
        d->history[h * d->steps + k] = hbuf[(size_t)h];
        bad |= !std::isfinite(hbuf[(size_t)h]);
      }
      if (bad) {
        out->nonfinite_step = k;
        break;
      }
    }
    // Without history, the steps launched are complete once this synchronization succeeds.
    if (latch(e, hipStreamSynchronize(f->stream), "device execution")) result = -1;
    else if (d->n_history == 0) done = enqueued;
    out->seconds = now() - t0;
  } catch (std::exception& ex) {
    if (e->failure.empty()) e->failure = ex.what();
    result = -1;
  }
  out->done = done;
  // The frame's table follows every handoff enqueued; after a failure the state is unspecified.
  f->slot = table[(size_t)(enqueued % n_tables)];
  hipStreamSynchronize(f->stream);
  return result;
}

}  // extern "C"
