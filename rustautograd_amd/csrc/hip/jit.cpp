#include "jit.h"

#include <hip/hiprtc.h>

#include <algorithm>
#include <cstdlib>
#include <map>
#include <memory>
#include <mutex>
#include <sstream>
#include <stdexcept>

#include "ops.h"

namespace rgjit {

// The text of gemm_mfma.h (generated at build time), for products compiled with an epilogue.
extern const char* const rg_gemm_mfma_source;

namespace {

std::vector<int64_t> row_strides(const std::vector<int64_t>& shape) {
  std::vector<int64_t> st(shape.size(), 1);
  for (size_t i = shape.size(); i-- > 1;) st[i - 1] = st[i] * shape[i];
  return st;
}

std::string expr(int op, const std::vector<std::string>& a) {
  switch (op) {
    case RG_OP_NEG: return "-" + a[0];
    case RG_OP_EXP: return "rg_exp(" + a[0] + ")";
    case RG_OP_LOG: return "rg_log(" + a[0] + ")";
    case RG_OP_SQRT: return "rg_sqrt(" + a[0] + ")";
    case RG_OP_SIN: return "rg_sin(" + a[0] + ")";
    case RG_OP_COS: return "rg_cos(" + a[0] + ")";
    case RG_OP_TANH: return "rg_tanh(" + a[0] + ")";
    case RG_OP_ABS: return "rg_abs(" + a[0] + ")";
    case RG_OP_SIGN: return "rg_sign(" + a[0] + ")";
    case RG_OP_FLOOR: return "rg_floor(" + a[0] + ")";
    case RG_OP_ADD: return a[0] + " + " + a[1];
    case RG_OP_SUB: return a[0] + " - " + a[1];
    case RG_OP_MUL: return a[0] + " * " + a[1];
    case RG_OP_DIV: return a[0] + " / " + a[1];
    case RG_OP_POW: return "rg_pow(" + a[0] + ", " + a[1] + ")";
    case RG_OP_MAX: return "rg_max(" + a[0] + ", " + a[1] + ")";
    case RG_OP_MIN: return "rg_min(" + a[0] + ", " + a[1] + ")";
    case RG_OP_GT: return "rg_gt(" + a[0] + ", " + a[1] + ")";
    case RG_OP_GE: return "rg_ge(" + a[0] + ", " + a[1] + ")";
    case RG_OP_WHERE: return "rg_where(" + a[0] + ", " + a[1] + ", " + a[2] + ")";
  }
  throw std::runtime_error("operation is not fusable");
}

}  // namespace

// A kernel walks its elements grid-stride with at most EW_BLOCKS blocks (16 per CU), so waves are
// long-lived; U vectors of V per thread per pass, all loaded before any is computed.
constexpr int EW_UNROLL = 1;
constexpr uint64_t EW_BLOCKS = 16 * 256;

std::string generate(const rgplan::Fused& f, const std::string& name, FusedKernel* k, bool device_fn) {
  const bool dbl = f.dtype == RG_F64;
  const char* T = dbl ? "double" : "float";
  const int V = dbl ? 2 : 4;
  const int U = EW_UNROLL;
  const uint64_t n = (uint64_t)f.n;
  const uint64_t chunk = (uint64_t)TPB * V * U;  // elements a block handles per pass
  const bool wide = n * 2 + chunk * 2 >= (1ull << 31);
  const char* I = wide ? "unsigned long long" : "unsigned int";
  k->name = name;
  k->vec = V * U;
  const uint64_t blocks = (n + chunk - 1) / chunk;
  k->grid = (uint32_t)(device_fn ? blocks : std::min<uint64_t>(blocks, EW_BLOCKS));

  std::ostringstream s;
  // Outputs that share a slot with an input are written in place, so no pointer is restrict.
  bool alias = false;
  for (auto& o : f.outputs)
    for (auto& in : f.inputs) alias |= in.slot == o.second;
  const char* R = alias ? "" : "__restrict__ ";
  if (device_fn) s << "static __device__ __forceinline__ void " << name << "(const unsigned int bid, ";
  else s << "extern \"C\" __global__ void __launch_bounds__(" << TPB << ") " << name << "(";
  for (size_t j = 0; j < f.inputs.size(); j++) s << (j ? ", " : "") << "const " << T << "* " << R << "in" << j;
  for (size_t j = 0; j < f.outputs.size(); j++) s << ", " << T << "* " << R << "out" << j;
  s << ") {\n";
  s << "  typedef " << I << " I;\n";
  s << "  const I n = " << n << "ull;\n";
  const char* VT = dbl ? "double2" : "float4";
  const char* lanes[4] = {"x", "y", "z", "w"};
  // Operand expressions per register and per Full input.
  std::vector<std::string> reg_expr((size_t)f.regs);
  auto rank = f.shape.size();
  auto ds = row_strides(f.shape);
  for (size_t j = 0; j < f.inputs.size(); j++) {
    const auto& in = f.inputs[j];
    if (in.kind == RG_ARG_SPLAT) {
      s << "  const " << T << " x" << j << "s = in" << j << "[0];\n";
      reg_expr[(size_t)in.reg] = "x" + std::to_string(j) + "s";
    } else if (in.reg >= 0) {
      reg_expr[(size_t)in.reg] = "x" + std::to_string(j) + "[u][v]";
    }
  }
  if (device_fn) s << "  {\n  const I blk = (I)bid * " << chunk << "u;\n";
  else s << "  for (I blk = (I)blockIdx.x * " << chunk << "u; blk < n; blk += (I)gridDim.x * " << chunk << "u) {\n";
  // Loads of every vector of the pass first.
  for (size_t j = 0; j < f.inputs.size(); j++)
    if (f.inputs[j].kind != RG_ARG_SPLAT) s << "  " << T << " x" << j << "[" << U << "][" << V << "];\n";
  s << "#pragma unroll\n  for (int u = 0; u < " << U << "; u++) {\n";
  s << "    const I i0 = blk + ((I)u * " << TPB << "u + (I)threadIdx.x) * " << V << "u;\n";
  s << "    if (i0 >= n) break;\n";
  s << "    const bool full = i0 + " << V << "u <= n;\n";
  for (size_t j = 0; j < f.inputs.size(); j++) {
    const auto& in = f.inputs[j];
    std::string x = "x" + std::to_string(j) + "[u]";
    if (in.kind == RG_ARG_SPLAT) continue;
    if (in.kind == RG_ARG_FULL) {
      s << "    if (full) { " << VT << " t = *(const " << VT << "*)(in" << j << " + i0);";
      for (int v = 0; v < V; v++) s << " " << x << "[" << v << "] = t." << lanes[v] << ";";
      s << " } else { for (int v = 0; v < " << V << "; v++) " << x << "[v] = i0 + v < n ? in" << j << "[i0 + v] : (" << T << ")0; }\n";
    } else if (in.kind == RG_ARG_ROW) {
      int64_t L = in.row_len;
      if (L % V == 0) {
        s << "    if (full) { " << VT << " t = *(const " << VT << "*)(in" << j << " + i0 % " << L << "u);";
        for (int v = 0; v < V; v++) s << " " << x << "[" << v << "] = t." << lanes[v] << ";";
        s << " } else { for (int v = 0; v < " << V << "; v++) " << x << "[v] = i0 + v < n ? in" << j << "[(i0 + v) % " << L
          << "u] : (" << T << ")0; }\n";
      } else {
        s << "    for (int v = 0; v < " << V << "; v++) " << x << "[v] = i0 + v < n ? in" << j << "[(i0 + v) % " << L << "u] : ("
          << T << ")0;\n";
      }
    } else {  // Broadcast: flat source index from the output coordinates
      const auto& is = in.shape;
      auto st = row_strides(is);
      size_t lead = rank - is.size();
      std::string idx;
      for (size_t d = 0; d < rank; d++) {
        int64_t bs = (d < lead || is[d - lead] == 1) ? 0 : st[d - lead];
        if (bs == 0 || f.shape[d] == 1) continue;
        std::string c = "(i / " + std::to_string(ds[d]) + "u)";
        if (d > 0) c = "(" + c + " % " + std::to_string(f.shape[d]) + "u)";
        if (!idx.empty()) idx += " + ";
        idx += c + " * " + std::to_string(bs) + "u";
      }
      if (idx.empty()) idx = "0u";
      s << "    for (int v = 0; v < " << V << "; v++) { I i = i0 + v; " << x << "[v] = i < n ? in" << j << "[" << idx << "] : (" << T
        << ")0; }\n";
    }
  }
  s << "  }\n";
  // Then the arithmetic and the stores, vector by vector.
  s << "#pragma unroll\n  for (int u = 0; u < " << U << "; u++) {\n";
  s << "    const I i0 = blk + ((I)u * " << TPB << "u + (I)threadIdx.x) * " << V << "u;\n";
  s << "    if (i0 >= n) break;\n";
  s << "    const bool full = i0 + " << V << "u <= n;\n";
  for (size_t j = 0; j < f.outputs.size(); j++) s << "    " << T << " o" << j << "[" << V << "];\n";
  s << "#pragma unroll\n    for (int v = 0; v < " << V << "; v++) {\n";
  for (auto& m : f.ops) {
    std::vector<std::string> args;
    for (auto& [is_reg, idx] : m.args) {
      if (is_reg) {
        const std::string& e = reg_expr[(size_t)idx];
        args.push_back(e.empty() ? "r" + std::to_string(idx) : e);
      } else {
        args.push_back("x" + std::to_string(idx) + "[u][v]");
      }
    }
    s << "      const " << T << " r" << m.reg << " = " << expr(m.op, args) << ";\n";
  }
  for (size_t j = 0; j < f.outputs.size(); j++) s << "      o" << j << "[v] = r" << f.outputs[j].first << ";\n";
  s << "    }\n";
  for (size_t j = 0; j < f.outputs.size(); j++) {
    s << "    if (full) { " << VT << " t;";
    for (int v = 0; v < V; v++) s << " t." << lanes[v] << " = o" << j << "[" << v << "];";
    s << " *(" << VT << "*)(out" << j << " + i0) = t; } else { for (int v = 0; v < " << V << "; v++) if (i0 + v < n) out" << j
      << "[i0 + v] = o" << j << "[v]; }\n";
  }
  s << "  }\n";
  s << "  }\n";
  s << "}\n";
  return s.str();
}

std::string generate_gemm(const rgplan::Fused& f, int64_t c_slot, bool store_c, const ProductTile& t, const std::string& name,
                          FusedKernel* k, int col_sum) {
  if (f.dtype != RG_F32) throw std::runtime_error("product epilogue: fp32 groups only");
  const std::string E = name + "_epi";
  // Column sums (col_sum >= 0): a K-contiguous B's transposed form, where each lane stores runs
  // of four columns, the same runs for every row (put4's slot: tile n across N, register group).
  const int slots = (t.bn / t.wn / t.ms) * (t.ms / 16) * (t.ms == 32 ? 4 : 1);
  if (col_sum >= 0 && (!t.tb || t.ms != 16)) throw std::runtime_error("product epilogue column sums: needs a K-contiguous B and 16x16 tiles");
  std::ostringstream s;
  s << "struct " << E << " {\n  float* c;\n";
  for (size_t j = 0; j < f.inputs.size(); j++) s << "  const float* in" << j << ";\n";
  for (size_t j = 0; j < f.outputs.size(); j++) s << "  float* out" << j << ";\n";
  if (col_sum >= 0) s << "  float4 colacc[" << slots << "];\n";
  s << "  __device__ __forceinline__ void begin(unsigned int, unsigned int) {}\n";
  // The group's value of element e + v for v < W, from the product's outputs `a`.
  auto body = [&](int W) {
    std::ostringstream b;
    std::vector<std::string> reg_expr((size_t)f.regs);
    std::vector<std::string> in_expr(f.inputs.size());
    for (size_t j = 0; j < f.inputs.size(); j++) {
      const auto& in = f.inputs[j];
      const std::string x = "x" + std::to_string(j);
      if (in.kind == RG_ARG_SPLAT) {
        b << "    const float " << x << "s = in" << j << "[0];\n";
        in_expr[j] = x + "s";
      } else if (in.kind == RG_ARG_FULL && in.slot == c_slot) {
        in_expr[j] = "a[v]";
      } else if (in.kind == RG_ARG_FULL || in.kind == RG_ARG_ROW) {
        const std::string at = in.kind == RG_ARG_FULL ? "e" : "(e % " + std::to_string(in.row_len) + "ull)";
        b << "    float " << x << "[" << W << "];\n";
        if (W == 4) b << "    { const float4 t = *(const float4*)(in" << j << " + " << at << "); " << x << "[0] = t.x; " << x << "[1] = t.y; " << x
                      << "[2] = t.z; " << x << "[3] = t.w; }\n";
        else if (W == 2) b << "    { const float2 t = *(const float2*)(in" << j << " + " << at << "); " << x << "[0] = t.x; " << x << "[1] = t.y; }\n";
        else b << "    " << x << "[0] = in" << j << "[" << at << "];\n";
        in_expr[j] = x + "[v]";
      } else {
        throw std::runtime_error("product epilogue: broadcast inputs are not supported");
      }
      if (in.reg >= 0) reg_expr[(size_t)in.reg] = in_expr[j];
    }
    for (size_t j = 0; j < f.outputs.size(); j++) b << "    float o" << j << "[" << W << "];\n";
    b << "#pragma unroll\n    for (int v = 0; v < " << W << "; v++) {\n";
    for (auto& m : f.ops) {
      std::vector<std::string> args;
      for (auto& [is_reg, idx] : m.args) {
        if (is_reg) {
          const std::string& e = reg_expr[(size_t)idx];
          args.push_back(e.empty() ? "r" + std::to_string(idx) : e);
        } else {
          args.push_back(in_expr[(size_t)idx]);
        }
      }
      b << "      const float r" << m.reg << " = " << expr(m.op, args) << ";\n";
    }
    for (size_t j = 0; j < f.outputs.size(); j++) b << "      o" << j << "[v] = r" << f.outputs[j].first << ";\n";
    b << "    }\n";
    for (size_t j = 0; j < f.outputs.size(); j++) {
      if (W == 4) b << "    *(float4*)(out" << j << " + e) = make_float4(o" << j << "[0], o" << j << "[1], o" << j << "[2], o" << j << "[3]);\n";
      else if (W == 2) b << "    *(float2*)(out" << j << " + e) = make_float2(o" << j << "[0], o" << j << "[1]);\n";
      else b << "    out" << j << "[e] = o" << j << "[0];\n";
    }
    return b.str();
  };
  s << "  __device__ __forceinline__ void put4(unsigned long long e, float4 acc, int slot) {\n";
  if (store_c) s << "    *(float4*)(c + e) = acc;\n";
  s << "    const float a[4] = {acc.x, acc.y, acc.z, acc.w};\n" << body(4);
  if (col_sum >= 0) {
    const std::string o = "o" + std::to_string(col_sum);
    s << "    colacc[slot] = make_float4(colacc[slot].x + " << o << "[0], colacc[slot].y + " << o << "[1], colacc[slot].z + " << o
      << "[2], colacc[slot].w + " << o << "[3]);\n";
  }
  s << "  }\n";
  s << "  __device__ __forceinline__ void put1(unsigned long long e, float acc) {\n";
  if (store_c) s << "    c[e] = acc;\n";
  s << "    const float a[1] = {acc};\n" << body(1) << "  }\n";
  s << "  __device__ __forceinline__ void put2(unsigned long long e, float2 acc) {\n";
  if (store_c) s << "    *(float2*)(c + e) = acc;\n";
  s << "    const float a[2] = {acc.x, acc.y};\n" << body(2) << "  }\n";
  s << "};\n";
  const int nt = 64 * t.wm * t.wn;
  // At least two waves per SIMD (at most 256 registers a wave, far above what the tile uses): with
  // that bound the compiler keeps the MFMA accumulators in ordinary VGPRs, as the precompiled
  // tiles are built (-amdgpu-mfma-vgpr-form), rather than copying them through AGPRs.
  // The epilogue's pointers arrive as kernel parameters, restrict-qualified when no output shares
  // a slot with an input or the product, so that the compiler may issue an output's loads before
  // the stores of the outputs before it.
  bool alias = false;
  for (auto& o : f.outputs) {
    alias |= o.second == c_slot;
    for (auto& in : f.inputs) alias |= in.slot == o.second;
  }
  const char* R = alias ? "" : "__restrict__ ";
  s << "extern \"C\" __global__ void __launch_bounds__(" << nt << ") __attribute__((amdgpu_waves_per_eu(2))) " << name
    << "(const float* __restrict__ A, const float* __restrict__ B, int M, int N, int K, const rgg::int64_t* a_off, const rgg::int64_t* b_off, "
       "rgg::uint64_t a_stride, rgg::uint64_t b_stride, int splits, int kps, const float* __restrict__ bias, rgg::uint32_t tiles_m, "
       "rgg::uint32_t tiles_n, int swizzle, float* "
    << R << "c";
  for (size_t j = 0; j < f.inputs.size(); j++) s << ", const float* " << R << "in" << j;
  for (size_t j = 0; j < f.outputs.size(); j++) s << ", float* " << R << "out" << j;
  if (col_sum >= 0) s << ", float* __restrict__ colp";
  s << ") {\n  " << E << " epi{c";
  for (size_t j = 0; j < f.inputs.size(); j++) s << ", in" << j;
  for (size_t j = 0; j < f.outputs.size(); j++) s << ", out" << j;
  s << "};\n";
  if (col_sum >= 0) s << "  for (int q = 0; q < " << slots << "; q++) epi.colacc[q] = make_float4(0.f, 0.f, 0.f, 0.f);\n";
  s << "  rgg::gemm_mfma_block<" << t.bm << ", " << t.bn << ", " << t.bk << ", " << t.wm << ", " << t.wn << ", " << (t.ta ? "true" : "false") << ", "
    << (t.tb ? "true" : "false") << ", " << t.mode << ", " << t.ms
    << ">(A, B, M, N, K, a_off, b_off, a_stride, b_stride, splits, kps, bias, tiles_m, tiles_n, swizzle, epi);\n";
  if (col_sum >= 0) {
    // The tile's column sums of output col_sum from the lanes' register sums (each lane summed
    // its rows in order): the 16 lanes holding the same columns combine by a fixed butterfly,
    // then the WM waves along M in order, through LDS; one partial row per tile row. Lane l of
    // wave (wm, wn) holds, in slot n, columns wn * WTN + 16 n + 4 (l / 16) .. + 3 of the tile.
    const int wtn = t.bn / t.wn;
    s << "  __shared__ float cs[" << t.wm << "][" << t.bn << "];\n";
    s << "  {\n    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, wmi = wave / " << t.wn << ", wni = wave % " << t.wn << ";\n";
    s << "    for (int q = 0; q < " << slots << "; q++) {\n";
    s << "      float4 v = epi.colacc[q];\n";
    s << "      for (int x = 1; x < 16; x <<= 1) {\n";
    s << "        v.x = v.x + __shfl_xor(v.x, x); v.y = v.y + __shfl_xor(v.y, x);\n";
    s << "        v.z = v.z + __shfl_xor(v.z, x); v.w = v.w + __shfl_xor(v.w, x);\n      }\n";
    s << "      if ((lane & 15) == 0) *(float4*)&cs[wmi][wni * " << wtn << " + 16 * q + 4 * (lane >> 4)] = v;\n    }\n  }\n";
    s << "  __syncthreads();\n";
    s << "  if (threadIdx.x < " << t.bn << ") {\n";
    s << "    const rgg::TileIndex ti = rgg::tile_of(blockIdx.x, gridDim.x, tiles_m, tiles_n, swizzle);\n";
    s << "    float v = cs[0][threadIdx.x];\n";
    s << "    for (int w = 1; w < " << t.wm << "; w++) v = v + cs[w][threadIdx.x];\n";
    s << "    colp[(rgg::uint64_t)ti.tm * N + ti.tn * " << t.bn << " + threadIdx.x] = v;\n  }\n";
  }
  s << "}\n";
  k->name = name;
  k->block = (uint32_t)nt;
  k->vec = 1;
  return s.str();
}

std::vector<int64_t> merged_slots(const std::vector<const rgplan::Fused*>& parts) {
  std::vector<int64_t> out;
  auto add = [&](int64_t slot) {
    if (std::find(out.begin(), out.end(), slot) == out.end()) out.push_back(slot);
  };
  for (const auto* f : parts) {
    for (auto& in : f->inputs) add(in.slot);
    for (auto& o : f->outputs) add(o.second);
  }
  return out;
}

std::string generate_merged(const std::vector<const rgplan::Fused*>& parts, const std::string& name, FusedKernel* k) {
  const std::vector<int64_t> slots = merged_slots(parts);
  std::ostringstream s, params, body;
  for (size_t q = 0; q < slots.size(); q++) {
    bool written = false, f64 = false;
    for (const auto* f : parts) {
      for (auto& o : f->outputs) written |= o.second == slots[q];
      for (auto& in : f->inputs) f64 |= in.slot == slots[q] && f->dtype == RG_F64;
      for (auto& o : f->outputs) f64 |= o.second == slots[q] && f->dtype == RG_F64;
    }
    params << (q ? ", " : "") << (written ? "" : "const ") << (f64 ? "double" : "float") << "* q" << q;
  }
  uint32_t start = 0;
  // Each branch reads only its part's pointers from the kernel argument segment. Passing the
  // named parameters instead has the compiler load all of them (up to MERGE_MAX_ARGS) at entry
  // and spill most to VGPR lanes, a prologue of hundreds of instructions in every block.
  body << "  const unsigned int b = blockIdx.x;\n";
  body << "  const __attribute__((address_space(4))) unsigned long long* ka = (const __attribute__((address_space(4))) unsigned long "
          "long*)__builtin_amdgcn_kernarg_segment_ptr();\n";
  auto arg = [&](int64_t slot, bool out, bool f64) {
    const size_t q = std::find(slots.begin(), slots.end(), slot) - slots.begin();
    return std::string("(") + (out ? "" : "const ") + (f64 ? "double" : "float") + "*)ka[" + std::to_string(q) + "]";
  };
  for (size_t j = 0; j < parts.size(); j++) {
    const rgplan::Fused& f = *parts[j];
    const std::string part = name + "_" + std::to_string(j);
    FusedKernel pk;
    s << generate(f, part, &pk, true);
    std::string call = part + "(b - " + std::to_string(start) + "u";
    for (auto& in : f.inputs) call += ", " + arg(in.slot, false, f.dtype == RG_F64);
    for (auto& o : f.outputs) call += ", " + arg(o.second, true, f.dtype == RG_F64);
    start += pk.grid;
    body << "  if (b < " << start << "u) { " << call << "); return; }\n";
  }
  k->name = name;
  k->grid = start;
  k->vec = 1;
  s << "extern \"C\" __global__ void __launch_bounds__(" << TPB << ") " << name << "(" << params.str() << ") {\n" << body.str() << "}\n";
  return s.str();
}

// A row group (RG_STEP_ROWS): one wavefront per row, each lane holding E elements of the row in
// registers (E = L/64 rounded up to the vector width), with V-wide coalesced loads and stores.
// Row-level values (per-row inputs, reductions) are one register per lane, equal across the
// wave; a reduction folds each lane's elements in order, then the 64 lanes by DPP exchanges and
// permlane swaps (no LDS; 4 % faster than a butterfly of LDS shuffles on C4's row groups), so
// every lane ends with the same result. (Issuing the next row's loads before the current row's
// arithmetic in the grid-stride column kernels measured 2 % slower.)
std::string generate_rows(const rgplan::Fused& f, const std::string& name, FusedKernel* k) {
  const bool dbl = f.dtype == RG_F64;
  const char* T = dbl ? "double" : "float";
  const int64_t L = f.row_len, rows = f.n / f.row_len;
  const int maxv = dbl ? 2 : 4;
  int V = 1;
  for (int v = maxv; v > 1; v /= 2)
    if (L % (64 * v) == 0) {
      V = v;
      break;
    }
  const int64_t E = (L + 64 * V - 1) / (64 * V) * V;
  const bool exact = L % (64 * V) == 0;
  const char* VT = dbl ? (V == 2 ? "double2" : "double") : (V == 4 ? "float4" : V == 2 ? "float2" : "float");
  const char* lanes[4] = {"x", "y", "z", "w"};
  k->name = name;
  k->vec = 1;
  k->grid = (uint32_t)((rows + 3) / 4);
  // Column reductions (RG_ROWS_COLUMN): the waves walk rows grid-stride, accumulating them.
  std::vector<bool> col_reg((size_t)f.regs, false);
  bool has_col = false;
  for (auto& m : f.ops)
    if (m.op == RG_OP_REDUCE && (m.aux & RG_ROWS_COLUMN)) col_reg[(size_t)m.reg] = has_col = true;
  k->col_kind.assign(f.outputs.size(), -1);
  k->row_len = (uint32_t)L;
  if (has_col) {
    k->grid = (uint32_t)std::min<int64_t>((rows + COL_WAVES - 1) / COL_WAVES, COL_BLOCKS);
    k->block = 64 * COL_WAVES;
    for (size_t j = 0; j < f.outputs.size(); j++)
      for (auto& m : f.ops)
        if (m.reg == f.outputs[j].first && col_reg[(size_t)m.reg]) k->col_kind[j] = (int)(m.aux & ~(int64_t)RG_ROWS_COLUMN);
  }

  // Levels: true for row-level registers.
  std::vector<int> level((size_t)f.regs, 0);
  auto ds = f.shape;
  const size_t rank = f.shape.size();
  auto per_row = [&](const rgplan::FusedInput& in) {
    return in.kind == RG_ARG_SPLAT || (in.kind == RG_ARG_BROADCAST && (in.shape.empty() || in.shape.back() == 1));
  };
  for (auto& in : f.inputs)
    if (in.reg >= 0) level[(size_t)in.reg] = per_row(in);
  for (auto& m : f.ops) {
    bool r = true;
    for (auto& a : m.args) r = r && a.first && level[(size_t)a.second];
    level[(size_t)m.reg] = m.op == RG_OP_REDUCE || r;
  }

  std::ostringstream s;
  bool alias = false;
  for (auto& o : f.outputs)
    for (auto& in : f.inputs) alias |= in.slot == o.second;
  const char* R = alias ? "" : "__restrict__ ";
  const int waves = has_col ? COL_WAVES : TPB / 64;
  s << "extern \"C\" __global__ void __launch_bounds__(" << 64 * waves << ") " << name << "(";
  for (size_t j = 0; j < f.inputs.size(); j++) s << (j ? ", " : "") << "const " << T << "* " << R << "in" << j;
  for (size_t j = 0; j < f.outputs.size(); j++) s << ", " << T << "* " << R << "out" << j;
  s << ") {\n";
  s << "  const unsigned lane = threadIdx.x & 63u;\n";
  auto col_init = [&](int64_t aux) {
    const int64_t kind = aux & ~(int64_t)RG_ROWS_COLUMN;
    return kind == RG_REDUCE_SUM ? std::string("0") : kind == RG_REDUCE_MAX ? std::string("-__builtin_huge_val()") : std::string("__builtin_huge_val()");
  };
  auto col_comb = [&](int64_t aux, const std::string& x, const std::string& y) {
    const int64_t kind = aux & ~(int64_t)RG_ROWS_COLUMN;
    return kind == RG_REDUCE_SUM ? x + " + " + y : std::string(kind == RG_REDUCE_MAX ? "rg_max(" : "rg_min(") + x + ", " + y + ")";
  };
  if (has_col) {
    for (auto& m : f.ops)
      if (col_reg[(size_t)m.reg])
        s << "  " << T << " c" << m.reg << "[" << E << "];\n  for (int e = 0; e < " << E << "; e++) c" << m.reg << "[e] = (" << T << ")"
          << col_init(m.aux) << ";\n";
    s << "  for (unsigned long long row = (unsigned long long)blockIdx.x * " << waves << "ull + (threadIdx.x >> 6); row < " << rows
      << "ull; row += (unsigned long long)gridDim.x * " << waves << "ull) {\n";
  } else {
    s << "  const unsigned long long row = (unsigned long long)blockIdx.x * 4ull + (threadIdx.x >> 6);\n";
    s << "  if (row >= " << rows << "ull) return;\n";
  }
  // Element e of this lane sits at column J(e) of the row.
  auto col = [&](int64_t e) {
    return std::to_string((e / V) * 64 * V + e % V) + "u + lane * " + std::to_string(V) + "u";
  };
  auto valid = [&](int64_t e) { return exact ? std::string("true") : "(" + col(e) + " < " + std::to_string(L) + "u)"; };
  // Offset of a broadcast input's row: coordinates of `row` over the leading dimensions.
  auto row_offset = [&](const std::vector<int64_t>& is) {
    size_t lead = rank - is.size();
    std::vector<int64_t> st(is.size(), 1);
    for (size_t i = is.size(); i-- > 1;) st[i - 1] = st[i] * is[i];
    std::string idx;
    int64_t inner = 1;  // product of the leading dimensions after d
    std::vector<int64_t> inner_of(rank, 1);
    for (size_t d = rank - 1; d-- > 0;) {
      inner_of[d] = inner;
      inner *= f.shape[d];
    }
    for (size_t d = 0; d + 1 < rank; d++) {
      int64_t bs = (d < lead || is[d - lead] == 1) ? 0 : st[d - lead];
      if (bs == 0 || f.shape[d] == 1) continue;
      std::string c = "(row / " + std::to_string(inner_of[d]) + "ull)";
      if (d > 0) c = "(" + c + " % " + std::to_string(f.shape[d]) + "ull)";
      if (!idx.empty()) idx += " + ";
      idx += c + " * " + std::to_string(bs) + "ull";
    }
    return idx.empty() ? std::string("0ull") : idx;
  };
  // Loads E elements of a row starting at pointer expression `base` into array `x`.
  auto load_row = [&](const std::string& x, const std::string& base) {
    s << "  " << T << " " << x << "[" << E << "];\n";
    if (V > 1) {
      for (int64_t c = 0; c < E / V; c++) {
        s << "  { const " << VT << " t = *(const " << VT << "*)(" << base << " + " << col(c * V) << ");";
        for (int v = 0; v < V; v++) s << " " << x << "[" << c * V + v << "] = t." << lanes[v] << ";";
        s << " }\n";
      }
    } else {
      for (int64_t e = 0; e < E; e++)
        s << "  " << x << "[" << e << "] = " << valid(e) << " ? " << base << "[" << col(e) << "] : (" << T << ")0;\n";
    }
  };
  std::vector<std::string> reg_name((size_t)f.regs);
  for (size_t j = 0; j < f.inputs.size(); j++) {
    const auto& in = f.inputs[j];
    std::string x = "x" + std::to_string(j), p = "in" + std::to_string(j);
    if (in.kind == RG_ARG_SPLAT) {
      s << "  const " << T << " " << x << " = " << p << "[0];\n";
    } else if (in.kind == RG_ARG_FULL) {
      load_row(x, "(" + p + " + row * " + std::to_string(L) + "ull)");
    } else if (in.kind == RG_ARG_ROW && in.row_len % L == 0) {
      int64_t reps = in.row_len / L;
      std::string base = reps == 1 ? p : "(" + p + " + (row % " + std::to_string(reps) + "ull) * " + std::to_string(L) + "ull)";
      load_row(x, base);
    } else if (in.kind == RG_ARG_ROW) {
      s << "  " << T << " " << x << "[" << E << "];\n";
      for (int64_t e = 0; e < E; e++)
        s << "  " << x << "[" << e << "] = " << valid(e) << " ? " << p << "[(row * " << L << "ull + " << col(e) << ") % " << in.row_len
          << "ull] : (" << T << ")0;\n";
    } else if (per_row(in)) {
      s << "  const " << T << " " << x << " = " << p << "[" << row_offset(in.shape) << "];\n";
    } else {  // a broadcast whose last dimension runs along the row: rows start at multiples of L
      std::string b = "b" + std::to_string(j);
      s << "  const unsigned long long " << b << " = " << row_offset(in.shape) << ";\n";
      load_row(x, "(" + p + " + " + b + ")");
    }
    if (in.reg >= 0) reg_name[(size_t)in.reg] = x;
  }
  auto operand = [&](const std::pair<int64_t, int64_t>& a, bool row_level, std::string* out_is_row) {
    std::string n = a.first ? (reg_name[(size_t)a.second].empty() ? "r" + std::to_string(a.second) : reg_name[(size_t)a.second])
                            : "x" + std::to_string(a.second);
    bool r = a.first && level[(size_t)a.second];
    (void)row_level;
    *out_is_row = r ? "1" : "0";
    return n;
  };
  for (auto& m : f.ops) {
    std::string rn = "r" + std::to_string(m.reg);
    if (col_reg[(size_t)m.reg]) {  // fold this row into the lane's column accumulators
      std::string is_row;
      std::string a = operand(m.args[0], false, &is_row);
      for (int64_t e = 0; e < E; e++) {
        std::string acc = "c" + std::to_string(m.reg) + "[" + std::to_string(e) + "]";
        // A row-level operand (a per-row or broadcast value) stands at every position of the row.
        std::string v = is_row == "1" ? a : a + "[" + std::to_string(e) + "]";
        if (exact) s << "  " << acc << " = " << col_comb(m.aux, acc, v) << ";\n";
        else s << "  if (" << valid(e) << ") " << acc << " = " << col_comb(m.aux, acc, v) << ";\n";
      }
      continue;
    }
    for (auto& a : m.args)
      if (a.first && col_reg[(size_t)a.second]) throw std::runtime_error("row group reads a column reduction");
    if (m.op == RG_OP_REDUCE) {
      std::string is_row;
      std::string a = operand(m.args[0], false, &is_row);
      const char* init = m.aux == RG_REDUCE_SUM ? "0" : m.aux == RG_REDUCE_MAX ? "-__builtin_huge_val()" : "__builtin_huge_val()";
      auto comb = [&](const std::string& x, const std::string& y) {
        return m.aux == RG_REDUCE_SUM ? x + " + " + y : std::string(m.aux == RG_REDUCE_MAX ? "rg_max(" : "rg_min(") + x + ", " + y + ")";
      };
      s << "  " << T << " " << rn << " = (" << T << ")" << init << ";\n";
      for (int64_t e = 0; e < E; e++) {
        // A row-level operand (a per-row or broadcast value) stands at every position of the row.
        std::string v = is_row == "1" ? a : a + "[" + std::to_string(e) + "]";
        if (exact) s << "  " << rn << " = " << comb(rn, v) << ";\n";
        else s << "  if (" << valid(e) << ") " << rn << " = " << comb(rn, v) << ";\n";
      }
      // The 64 lanes' partial values combined without LDS (rg_wave_sum and its kin, ops.h).
      s << "  " << rn << " = " << (m.aux == RG_REDUCE_SUM ? "rg_wave_sum(" : m.aux == RG_REDUCE_MAX ? "rg_wave_max(" : "rg_wave_min(") << rn
        << ");\n";
      continue;
    }
    if (level[(size_t)m.reg]) {
      std::vector<std::string> args;
      for (auto& a : m.args) {
        std::string r;
        args.push_back(operand(a, true, &r));
      }
      s << "  const " << T << " " << rn << " = " << expr(m.op, args) << ";\n";
      continue;
    }
    s << "  " << T << " " << rn << "[" << E << "];\n";
    s << "#pragma unroll\n  for (int e = 0; e < " << E << "; e++) " << rn << "[e] = ";
    std::vector<std::string> args;
    for (auto& a : m.args) {
      std::string r;
      std::string n = operand(a, false, &r);
      args.push_back(r == "1" || (!a.first && false) ? n : n + "[e]");
    }
    // Splat inputs are row level (a scalar); full inputs are element level.
    for (size_t q = 0; q < m.args.size(); q++) {
      const auto& a = m.args[q];
      if (!a.first) continue;
      if (level[(size_t)a.second]) args[q] = reg_name[(size_t)a.second].empty() ? "r" + std::to_string(a.second) : reg_name[(size_t)a.second];
    }
    s << expr(m.op, args) << ";\n";
  }
  for (size_t j = 0; j < f.outputs.size(); j++) {
    int64_t r = f.outputs[j].first;
    if (col_reg[(size_t)r]) continue;
    std::string rn = reg_name[(size_t)r].empty() ? "r" + std::to_string(r) : reg_name[(size_t)r];
    std::string o = "out" + std::to_string(j);
    if (level[(size_t)r]) {
      s << "  if (lane == 0) " << o << "[row] = " << rn << ";\n";
      continue;
    }
    std::string base = "(" + o + " + row * " + std::to_string(L) + "ull)";
    if (V > 1) {
      for (int64_t c = 0; c < E / V; c++) {
        s << "  { " << VT << " t;";
        for (int v = 0; v < V; v++) s << " t." << lanes[v] << " = " << rn << "[" << c * V + v << "];";
        s << " *(" << VT << "*)(" << base << " + " << col(c * V) << ") = t; }\n";
      }
    } else {
      for (int64_t e = 0; e < E; e++) s << "  if (" << valid(e) << ") " << base << "[" << col(e) << "] = " << rn << "[" << e << "];\n";
    }
  }
  if (has_col) {
    s << "  }\n";  // end of the row loop
    // The waves' accumulators, combined in wave order through LDS: one partial row per block.
    std::vector<size_t> cols;  // outputs that are column reductions
    for (size_t j = 0; j < f.outputs.size(); j++)
      if (col_reg[(size_t)f.outputs[j].first]) cols.push_back(j);
    auto aux_of = [&](size_t j) {
      int64_t aux = 0;
      for (auto& m : f.ops)
        if (m.reg == f.outputs[j].first) aux = m.aux;
      return aux;
    };
    auto stage = [&](size_t j, const std::string& dst) {
      const std::string c = "c" + std::to_string(f.outputs[j].first);
      for (int64_t e = 0; e < E; e++) {
        std::string w = "  " + dst + "[(threadIdx.x >> 6) * " + std::to_string(L) + "u + " + col(e) + "] = " + c + "[" + std::to_string(e) + "];\n";
        s << (exact ? w : "  if (" + valid(e) + ") " + w.substr(2));
      }
    };
    const uint64_t all_bytes = (uint64_t)cols.size() * waves * L * (dbl ? 8 : 4);
    if (cols.size() > 1 && all_bytes <= COL_LDS_BYTES) {
      // Every output's accumulators staged at once, then one thread per (output, column) adds
      // its column's wave values in wave order: one barrier, and the outputs' sums in parallel.
      s << "  __shared__ " << T << " cl[" << cols.size() << "][" << waves << " * " << L << "];\n";
      for (size_t i = 0; i < cols.size(); i++) stage(cols[i], "cl[" + std::to_string(i) + "]");
      s << "  __syncthreads();\n";
      s << "  for (unsigned q = threadIdx.x; q < " << cols.size() * L << "u; q += " << 64 * waves << "u) {\n";
      s << "    const unsigned o = q / " << L << "u, c = q % " << L << "u;\n";
      for (size_t i = 0; i < cols.size(); i++) {
        const int64_t aux = aux_of(cols[i]);
        const std::string cl = "cl[" + std::to_string(i) + "]";
        s << "    " << (i ? "else " : "") << "if (o == " << i << "u) {\n";
        s << "      " << T << " v = " << cl << "[c];\n";
        s << "      for (int w = 1; w < " << waves << "; w++) v = " << col_comb(aux, "v", cl + "[w * " + std::to_string(L) + "u + c]") << ";\n";
        s << "      out" << cols[i] << "[(unsigned long long)blockIdx.x * " << L << "ull + c] = v;\n";
        s << "    }\n";
      }
      s << "  }\n";
    } else {
      s << "  __shared__ " << T << " cl[" << waves << " * " << L << "];\n";
      for (size_t j : cols) {
        s << "  __syncthreads();\n";
        stage(j, "cl");
        s << "  __syncthreads();\n";
        s << "  for (unsigned q = threadIdx.x; q < " << L << "u; q += " << 64 * waves << "u) {\n";
        s << "    " << T << " v = cl[q];\n";
        s << "    for (int w = 1; w < " << waves << "; w++) v = " << col_comb(aux_of(j), "v", "cl[w * " + std::to_string(L) + "u + q]") << ";\n";
        s << "    out" << j << "[(unsigned long long)blockIdx.x * " << L << "ull + q] = v;\n";
        s << "  }\n";
      }
    }
  }
  s << "}\n";
  return s.str();
}

namespace {
std::mutex g_mu;
std::map<std::string, hipModule_t> g_modules;

}  // namespace

std::vector<char> compile_code(const std::string& body) {
  std::string src = std::string(rg_ops_source) + "\n";
  if (body.find("rgg::gemm_mfma_block") != std::string::npos) src += std::string(rg_gemm_mfma_source) + "\n";
  src += body;
  hiprtcProgram prog;
  if (hiprtcCreateProgram(&prog, src.c_str(), "rg_fused.hip", 0, nullptr, nullptr) != HIPRTC_SUCCESS)
    throw std::runtime_error("hiprtcCreateProgram failed");
  // The package's own flags (rustautograd_amd/build.py): no contraction, no fast math, denormals
  // kept, packed fp32 off. No -mllvm options: in a process that loaded another build of the code
  // object manager first (torch's), hiprtc runs that build's LLVM, and an option it does not know
  // ends the process.
  const char* opts[] = {"--offload-arch=gfx950", "-O3", "-ffp-contract=off", "-fno-fast-math", "-fno-gpu-flush-denormals-to-zero",
                        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};
  hiprtcResult r = hiprtcCompileProgram(prog, (int)(sizeof opts / sizeof opts[0]), opts);
  if (r != HIPRTC_SUCCESS) {
    size_t len = 0;
    hiprtcGetProgramLogSize(prog, &len);
    std::string log(len, '\0');
    if (len) hiprtcGetProgramLog(prog, &log[0]);
    hiprtcDestroyProgram(&prog);
    throw std::runtime_error("fused kernel compilation failed: " + log.substr(0, 1500));
  }
  size_t size = 0;
  hiprtcGetCodeSize(prog, &size);
  std::vector<char> code(size);
  hiprtcGetCode(prog, code.data());
  hiprtcDestroyProgram(&prog);
  return code;
}

namespace {
hipModule_t build_module(const std::string& body) {
  {
    std::lock_guard<std::mutex> lock(g_mu);
    auto it = g_modules.find(body);
    if (it != g_modules.end()) return it->second;
  }
  std::vector<char> code = compile_code(body);
  hipModule_t mod;
  hipError_t e = hipModuleLoadData(&mod, code.data());
  if (e != hipSuccess) throw std::runtime_error(std::string("hipModuleLoadData: ") + hipGetErrorString(e));
  std::lock_guard<std::mutex> lock(g_mu);
  g_modules[body] = mod;
  return mod;
}
}  // namespace

void compile(const std::string& source, std::vector<FusedKernel*>& kernels) {
  if (kernels.empty()) return;
  hipModule_t mod = build_module(source);
  for (auto* k : kernels) {
    hipError_t e = hipModuleGetFunction(&k->fn, mod, k->name.c_str());
    if (e != hipSuccess) throw std::runtime_error("kernel " + k->name + " missing from its module");
  }
}

}  // namespace rgjit
