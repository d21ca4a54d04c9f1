// Device backends behind the C ABI of include/rg_hip.h, loaded at run time.
//
// The engine is written against this table exactly as the reference's `Compiled` is written
// against `Exec` (src/plan.rs:29-41). The product registers one backend, "hip" (librg_hip.so);
// a test harness may register a second library with the same ABI under another name.
#pragma once
#include <memory>
#include <mutex>
#include <optional>
#include <string>
#include <vector>

#include "../../../include/rg_hip.h"
#include "plan.h"

namespace rg {

struct Backend {
  std::string name, path, prefix;
  void* lib = nullptr;
  int (*available)() = nullptr;
  void* (*program_new)(const int64_t*, size_t, const void*, size_t, char*, size_t) = nullptr;
  void (*program_free)(void*) = nullptr;
  uint64_t (*program_allocated_bytes)(void*) = nullptr;
  void (*program_inject_failure)(void*) = nullptr;
  void (*program_inject_failure_after)(void*, int64_t) = nullptr;  // optional
  int64_t (*program_step_runs_in)(void*, int64_t) = nullptr;  // optional
  void* (*exec_new)(void*, char*, size_t) = nullptr;
  void (*exec_free)(void*) = nullptr;
  int (*exec_write)(void*, int64_t, const void*, uint64_t) = nullptr;
  int (*exec_read)(void*, int64_t, void*, uint64_t) = nullptr;
  int (*exec_write_slots)(void*, int64_t, const int64_t*, const void* const*, const uint64_t*) = nullptr;  // optional
  int (*exec_read_slots)(void*, int64_t, const int64_t*, void* const*, const uint64_t*) = nullptr;        // optional
  double (*exec_scalar)(void*, int64_t) = nullptr;
  void (*exec_swap)(void*, int64_t, int64_t) = nullptr;
  void (*exec_step)(void*) = nullptr;
  void (*exec_steps)(void*, int64_t, int64_t) = nullptr;
  int (*exec_failure)(void*, char*, size_t) = nullptr;
  int (*exec_step_timed)(void*, double*) = nullptr;  // optional
  int (*exec_breakdown)(void*, int64_t, char*, size_t) = nullptr;  // optional
  int (*exec_time_steps)(void*, const int64_t*, int64_t, int64_t, double*) = nullptr;  // optional
  int (*exec_run)(void*, const rg_run_desc*, rg_run_result*) = nullptr;  // optional
  int (*gemm_streamed)(int32_t, int64_t, int64_t, int64_t, int64_t, int32_t, int32_t) = nullptr;  // optional
  int (*device_peaks)(double*, char*, size_t) = nullptr;  // optional
};

// Loads `path` and resolves `<prefix><entry point>` for every ABI function; throws a message.
void register_backend(const std::string& name, const std::string& path, const std::string& prefix);
// The backend registered under `name` whose device is present, or nullptr.
Backend* find_backend(const std::string& name);
std::vector<std::string> available_backends();
// Where eager operations and constant folding run: "hip" when present, else the first other
// registered backend; throws DEVICE_UNAVAILABLE when there is none.
Backend* eager_backend();

class DeviceExec;

// A plan built into device kernels (`MetalProgram`).
class DeviceProgram {
 public:
  DeviceProgram(Backend* b, const Plan& plan);  // throws std::runtime_error with the device's message
  ~DeviceProgram();
  DeviceProgram(const DeviceProgram&) = delete;
  Backend* backend() const { return b_; }
  void* handle() const { return p_; }
  const Plan& plan() const { return *plan_; }
  std::unique_ptr<DeviceExec> exec() const;  // throws std::runtime_error
  // Test hooks (metal.rs:385-388, 525-529): device bytes held, and a failure after `after` passes.
  uint64_t allocated_bytes() const { return b_->program_allocated_bytes(p_); }
  void inject_failure(int64_t after) const;
  // The step whose kernel computes step `k` (itself when none), where the backend says.
  int64_t step_runs_in(int64_t k) const { return b_->program_step_runs_in ? b_->program_step_runs_in(p_, k) : k; }
 private:
  Backend* b_;
  void* p_ = nullptr;
  const Plan* plan_;
};

// One frame of slot buffers (`MetalExec`): the `Exec` trait over the C ABI.
class DeviceExec {
 public:
  DeviceExec(Backend* b, void* e, const Plan* plan) : b_(b), e_(e), plan_(plan) {}
  ~DeviceExec() { b_->exec_free(e_); }
  void load(size_t k, const Tensor& t);
  // `load` of several inputs (index, tensor), enqueued together with one wait.
  void load_all(const std::vector<std::pair<size_t, const Tensor*>>& inputs);
  void step() { b_->exec_step(e_); }
  void steps(size_t begin, size_t end) { b_->exec_steps(e_, (int64_t)begin, (int64_t)end); }
  void swap(size_t a, size_t c) { b_->exec_swap(e_, (int64_t)a, (int64_t)c); }
  Tensor prefix(size_t slot, size_t n, const Shape& shape) const;
  // `prefix` of several (slot, n, shape) at once, with one wait.
  std::vector<Tensor> prefix_all(const std::vector<std::tuple<size_t, size_t, Shape>>& reads) const;
  void write_prefix(size_t slot, const Tensor& t);
  double scalar(size_t slot) const { return b_->exec_scalar(e_, (int64_t)slot); }
  std::optional<std::string> failure() const;
  Backend* backend() const { return b_; }
  void* handle() const { return e_; }
 private:
  Backend* b_;
  void* e_;
  const Plan* plan_;
};

// Plans `g`, builds it on backend `b`, executes it once and returns the outputs (plan.rs:997-1006 `eval`).
std::vector<Tensor> eval_on(Backend* b, const Graph& g, const std::vector<uint32_t>& outputs,
                            const std::vector<const Tensor*>& inputs);

}  // namespace rg
