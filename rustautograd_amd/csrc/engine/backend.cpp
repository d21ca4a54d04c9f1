#include "backend.h"

#include <dlfcn.h>

#include <map>
#include <stdexcept>

namespace rg {

namespace {
std::mutex g_mu;
std::vector<std::unique_ptr<Backend>> g_backends;

template <class F>
void bind(Backend& b, F*& fn, const char* entry, bool required) {
  std::string sym = b.prefix + entry;
  fn = reinterpret_cast<F*>(dlsym(b.lib, sym.c_str()));
  if (!fn && required) throw std::runtime_error(b.path + " does not export " + sym);
}
}  // namespace

void register_backend(const std::string& name, const std::string& path, const std::string& prefix) {
  std::lock_guard<std::mutex> lock(g_mu);
  for (auto& b : g_backends)
    if (b->name == name) {
      if (b->path == path) return;
      throw std::runtime_error("backend " + name + " is already registered from " + b->path);
    }
  auto b = std::make_unique<Backend>();
  b->name = name;
  b->path = path;
  b->prefix = prefix;
  b->lib = dlopen(path.c_str(), RTLD_NOW | RTLD_LOCAL);
  if (!b->lib) throw std::runtime_error(std::string("cannot load ") + path + ": " + dlerror());
  bind(*b, b->available, "available", true);
  bind(*b, b->program_new, "program_new", true);
  bind(*b, b->program_free, "program_free", true);
  bind(*b, b->program_allocated_bytes, "program_allocated_bytes", true);
  bind(*b, b->program_inject_failure, "program_inject_failure", true);
  bind(*b, b->program_inject_failure_after, "program_inject_failure_after", false);
  bind(*b, b->program_step_runs_in, "program_step_runs_in", false);
  bind(*b, b->exec_new, "exec_new", true);
  bind(*b, b->exec_free, "exec_free", true);
  bind(*b, b->exec_write, "exec_write", true);
  bind(*b, b->exec_read, "exec_read", true);
  bind(*b, b->exec_write_slots, "exec_write_slots", false);
  bind(*b, b->exec_read_slots, "exec_read_slots", false);
  bind(*b, b->exec_scalar, "exec_scalar", true);
  bind(*b, b->exec_swap, "exec_swap", true);
  bind(*b, b->exec_step, "exec_step", true);
  bind(*b, b->exec_steps, "exec_steps", true);
  bind(*b, b->exec_failure, "exec_failure", true);
  bind(*b, b->exec_step_timed, "exec_step_timed", false);
  bind(*b, b->exec_breakdown, "exec_breakdown", false);
  bind(*b, b->exec_time_steps, "exec_time_steps", false);
  bind(*b, b->exec_run, "exec_run", false);
  bind(*b, b->gemm_streamed, "gemm_streamed", false);
  bind(*b, b->device_peaks, "device_peaks", false);
  g_backends.push_back(std::move(b));
}

Backend* find_backend(const std::string& name) {
  std::lock_guard<std::mutex> lock(g_mu);
  for (auto& b : g_backends)
    if (b->name == name && b->available()) return b.get();
  return nullptr;
}

std::vector<std::string> available_backends() {
  std::lock_guard<std::mutex> lock(g_mu);
  std::vector<std::string> out;
  for (auto& b : g_backends)
    if (b->available()) out.push_back(b->name);
  return out;
}

Backend* eager_backend() {
  if (Backend* b = find_backend("hip")) return b;
  {
    std::lock_guard<std::mutex> lock(g_mu);
    for (auto& b : g_backends)
      if (b->available()) return b.get();
  }
  Json obs = Json::obj();
  obs["device"] = "hip";
  obs["available"] = Json(available_backends());
  throw DiagError{diag("DEVICE_UNAVAILABLE", "error", Json(), obs, "no_device_backend_for_eager_evaluation", "verified")};
}

DeviceProgram::DeviceProgram(Backend* b, const Plan& plan) : b_(b), plan_(&plan) {
  std::vector<int64_t> words;
  std::vector<uint8_t> blob;
  plan.serialize(&words, &blob);
  char err[2048] = {0};
  p_ = b->program_new(words.data(), words.size(), blob.data(), blob.size(), err, sizeof err);
  if (!p_) throw std::runtime_error(err[0] ? err : "device program construction failed");
}

DeviceProgram::~DeviceProgram() {
  if (p_) b_->program_free(p_);
}

std::unique_ptr<DeviceExec> DeviceProgram::exec() const {
  char err[2048] = {0};
  void* e = b_->exec_new(p_, err, sizeof err);
  if (!e) throw std::runtime_error(err[0] ? err : "device frame allocation failed");
  return std::make_unique<DeviceExec>(b_, e, plan_);
}

void DeviceProgram::inject_failure(int64_t after) const {
  if (after > 0 && !b_->program_inject_failure_after) throw std::runtime_error(b_->name + " cannot delay an injected failure");
  if (after > 0) b_->program_inject_failure_after(p_, after);
  else b_->program_inject_failure(p_);
}

void DeviceExec::load_all(const std::vector<std::pair<size_t, const Tensor*>>& inputs) {
  if (!b_->exec_write_slots) {
    for (auto& [k, t] : inputs) load(k, *t);
    return;
  }
  std::vector<int64_t> slots;
  std::vector<const void*> srcs;
  std::vector<uint64_t> bytes;
  for (auto& [k, t] : inputs) {
    size_t slot = plan_->input_slots[k];
    slots.push_back((int64_t)slot);
    srcs.push_back(t->data.data());
    bytes.push_back(std::min<uint64_t>(plan_->input_ns[k] * dsize(plan_->slots[slot].first), t->data.size()));
  }
  b_->exec_write_slots(e_, (int64_t)slots.size(), slots.data(), srcs.data(), bytes.data());
}

std::vector<Tensor> DeviceExec::prefix_all(const std::vector<std::tuple<size_t, size_t, Shape>>& reads) const {
  std::vector<Tensor> out(reads.size());
  std::vector<int64_t> slots;
  std::vector<void*> dsts;
  std::vector<uint64_t> bytes;
  for (size_t q = 0; q < reads.size(); q++) {
    auto& [slot, n, shape] = reads[q];
    out[q].shape = shape;
    out[q].dtype = plan_->slots[slot].first;
    out[q].data.resize(n * dsize(out[q].dtype));
    slots.push_back((int64_t)slot);
    dsts.push_back(out[q].data.data());
    bytes.push_back(out[q].data.size());
  }
  if (b_->exec_read_slots) b_->exec_read_slots(e_, (int64_t)slots.size(), slots.data(), dsts.data(), bytes.data());
  else
    for (size_t q = 0; q < reads.size(); q++)
      if (bytes[q]) b_->exec_read(e_, slots[q], dsts[q], bytes[q]);
  return out;
}

void DeviceExec::load(size_t k, const Tensor& t) {
  size_t slot = plan_->input_slots[k];
  size_t bytes = plan_->input_ns[k] * dsize(plan_->slots[slot].first);
  b_->exec_write(e_, (int64_t)slot, t.data.data(), std::min(bytes, t.data.size()));
}

Tensor DeviceExec::prefix(size_t slot, size_t n, const Shape& shape) const {
  Tensor t;
  t.shape = shape;
  t.dtype = plan_->slots[slot].first;
  t.data.resize(n * dsize(t.dtype));
  if (n) b_->exec_read(e_, (int64_t)slot, t.data.data(), t.data.size());
  return t;
}

void DeviceExec::write_prefix(size_t slot, const Tensor& t) {
  if (!t.data.empty()) b_->exec_write(e_, (int64_t)slot, t.data.data(), t.data.size());
}

std::optional<std::string> DeviceExec::failure() const {
  char buf[2048] = {0};
  if (b_->exec_failure(e_, buf, sizeof buf)) return std::string(buf);
  return std::nullopt;
}

std::vector<Tensor> eval_on(Backend* b, const Graph& g, const std::vector<uint32_t>& outputs,
                            const std::vector<const Tensor*>& inputs) {
  Plan plan = build_plan(g, outputs, true);
  DeviceProgram prog(b, plan);
  auto e = prog.exec();
  for (size_t k = 0; k < inputs.size(); k++) e->load(k, *inputs[k]);
  e->step();
  if (auto f = e->failure()) {
    Json obs = Json::obj();
    obs["device"] = b->name;
    obs["detail"] = *f;
    throw DiagError{diag("DEVICE_EXECUTION_FAILED", "error", Json(), obs, "gpu_reported_a_failure", "verified")};
  }
  std::vector<Tensor> out;
  for (auto& o : plan.outputs) out.push_back(e->prefix(o.slot, o.n, o.shape));
  return out;
}

}  // namespace rg
