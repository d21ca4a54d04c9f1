#include "jit.h"

#include <hip/hiprtc.h>

#include <map>
#include <memory>
#include <mutex>
#include <sstream>
#include <stdexcept>

#include "ops.h"

namespace rgjit {

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

std::string generate(const rgplan::Fused& f, const std::string& name, FusedKernel* k) {
  const bool dbl = f.dtype == RG_F64;
  const char* T = dbl ? "double" : "float";
  const int V = dbl ? 2 : 4;
  const uint64_t n = (uint64_t)f.n;
  const bool wide = n * 2 >= (1ull << 31);
  const char* I = wide ? "unsigned long long" : "unsigned int";
  k->name = name;
  k->vec = V;
  k->grid = (uint32_t)((n + (uint64_t)TPB * V - 1) / ((uint64_t)TPB * V));

  std::ostringstream s;
  // Outputs that share a slot with an input are written in place, so no pointer is restrict.
  bool alias = false;
  for (auto& o : f.outputs)
    for (auto& in : f.inputs) alias |= in.slot == o.second;
  const char* R = alias ? "" : "__restrict__ ";
  s << "extern \"C\" __global__ void __launch_bounds__(" << TPB << ") " << name << "(";
  for (size_t j = 0; j < f.inputs.size(); j++) s << (j ? ", " : "") << "const " << T << "* " << R << "in" << j;
  for (size_t j = 0; j < f.outputs.size(); j++) s << ", " << T << "* " << R << "out" << j;
  s << ") {\n";
  s << "  typedef " << I << " I;\n";
  s << "  const I n = " << n << "ull;\n";
  s << "  const I i0 = ((I)blockIdx.x * " << TPB << "u + (I)threadIdx.x) * " << V << "u;\n";
  s << "  if (i0 >= n) return;\n";
  s << "  const bool full = i0 + " << V << "u <= n;\n";
  const char* VT = dbl ? "double2" : "float4";
  const char* lanes[4] = {"x", "y", "z", "w"};
  // Operand expressions per register and per Full input.
  std::vector<std::string> reg_expr((size_t)f.regs);
  auto rank = f.shape.size();
  auto ds = row_strides(f.shape);
  for (size_t j = 0; j < f.inputs.size(); j++) {
    const auto& in = f.inputs[j];
    std::string x = "x" + std::to_string(j);
    if (in.kind == RG_ARG_SPLAT) {
      s << "  const " << T << " " << x << "s = in" << j << "[0];\n";
      reg_expr[(size_t)in.reg] = x + "s";
      continue;
    }
    s << "  " << T << " " << x << "[" << V << "];\n";
    if (in.reg >= 0) reg_expr[(size_t)in.reg] = x + "[v]";
    if (in.kind == RG_ARG_FULL) {
      s << "  if (full) { " << VT << " t = *(const " << VT << "*)(in" << j << " + i0);";
      for (int v = 0; v < V; v++) s << " " << x << "[" << v << "] = t." << lanes[v] << ";";
      s << " } else { for (int v = 0; v < " << V << "; v++) " << x << "[v] = i0 + v < n ? in" << j << "[i0 + v] : (" << T << ")0; }\n";
    } else if (in.kind == RG_ARG_ROW) {
      int64_t L = in.row_len;
      if (L % V == 0) {
        s << "  if (full) { " << VT << " t = *(const " << VT << "*)(in" << j << " + i0 % " << L << "u);";
        for (int v = 0; v < V; v++) s << " " << x << "[" << v << "] = t." << lanes[v] << ";";
        s << " } else { for (int v = 0; v < " << V << "; v++) " << x << "[v] = i0 + v < n ? in" << j << "[(i0 + v) % " << L
          << "u] : (" << T << ")0; }\n";
      } else {
        s << "  for (int v = 0; v < " << V << "; v++) " << x << "[v] = i0 + v < n ? in" << j << "[(i0 + v) % " << L << "u] : ("
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
      s << "  for (int v = 0; v < " << V << "; v++) { I i = i0 + v; " << x << "[v] = i < n ? in" << j << "[" << idx << "] : (" << T
        << ")0; }\n";
    }
  }
  for (size_t j = 0; j < f.outputs.size(); j++) s << "  " << T << " o" << j << "[" << V << "];\n";
  s << "#pragma unroll\n  for (int v = 0; v < " << V << "; v++) {\n";
  for (auto& m : f.ops) {
    std::vector<std::string> args;
    for (auto& [is_reg, idx] : m.args) {
      if (is_reg) {
        const std::string& e = reg_expr[(size_t)idx];
        args.push_back(e.empty() ? "r" + std::to_string(idx) : e);
      } else {
        args.push_back("x" + std::to_string(idx) + "[v]");
      }
    }
    s << "    const " << T << " r" << m.reg << " = " << expr(m.op, args) << ";\n";
  }
  for (size_t j = 0; j < f.outputs.size(); j++) s << "    o" << j << "[v] = r" << f.outputs[j].first << ";\n";
  s << "  }\n";
  for (size_t j = 0; j < f.outputs.size(); j++) {
    s << "  if (full) { " << VT << " t;";
    for (int v = 0; v < V; v++) s << " t." << lanes[v] << " = o" << j << "[" << v << "];";
    s << " *(" << VT << "*)(out" << j << " + i0) = t; } else { for (int v = 0; v < " << V << "; v++) if (i0 + v < n) out" << j
      << "[i0 + v] = o" << j << "[v]; }\n";
  }
  s << "}\n";
  return s.str();
}

namespace {
std::mutex g_mu;
std::map<std::string, hipModule_t> g_modules;

}  // namespace

std::vector<char> compile_code(const std::string& body) {
  std::string src = std::string(rg_ops_source) + "\n" + body;
  hiprtcProgram prog;
  if (hiprtcCreateProgram(&prog, src.c_str(), "rg_fused.hip", 0, nullptr, nullptr) != HIPRTC_SUCCESS)
    throw std::runtime_error("hiprtcCreateProgram failed");
  const char* opts[] = {"--offload-arch=gfx950", "-O3", "-ffp-contract=off", "-fno-fast-math",
                        "-fno-gpu-flush-denormals-to-zero", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};
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
