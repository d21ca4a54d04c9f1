// Compile, validate and run (reference src/validate.rs).
#pragma once
#include <map>
#include <memory>
#include <optional>

#include "backend.h"
#include "optimize.h"

namespace rg {

enum class Level { None = 0, Basic = 1, Standard = 2, Thorough = 3 };
bool parse_level(const std::string& s, Level* out);

struct RunSpec {
  std::vector<std::pair<size_t, size_t>> state;  // (input index, output index) fed back
  std::vector<size_t> data;                      // data input indices
  std::vector<size_t> history;                   // outputs whose single value is logged after each step
  // Outputs fed back into the state hold the same values as the final state: when set, `run`
  // does not read them a second time and leaves them empty (shape kept, no data).
  bool skip_state_outputs = false;
};

struct RunOut {
  std::vector<Tensor> state, outputs;
  std::vector<std::vector<double>> history;
  size_t steps = 0;
  int64_t nonfinite_step = -1;
  double seconds = 0;  // seconds spent stepping; loading state and setup are not counted
  std::optional<std::string> device_error;
};

class Compiled {
 public:
  Graph raw;
  std::vector<uint32_t> outputs;
  Plan plan, raw_plan;
  Json report;
  Level level = Level::None;
  OptMode mode = OptMode::Standard;
  OptStats opt_stats;
  Backend* device = nullptr;
  std::unique_ptr<DeviceProgram> program;
  std::unique_ptr<DeviceProgram> raw_program;  // built on first use by diagnostics
  // Programs of the control-flow bodies of `raw_plan`, which diagnostics run one iteration at a time.
  std::map<const Plan*, std::unique_ptr<DeviceProgram>> body_programs;

  void check_inputs(const std::vector<Tensor>& inputs) const;
  std::vector<Tensor> try_call(const std::vector<Tensor>& inputs) const;
  Json check(const std::vector<Tensor>& inputs);
  Json profile(const std::vector<Tensor>& inputs, size_t repeats) const;
  // How the device prices matrix products for step_work: which run on its streaming kernels.
  StreamedFn streamed_products() const;
  void validate_spec(const RunSpec& spec) const;
  // `state` is read in place (the run copies it to the device and returns the new state).
  RunOut run(const RunSpec& spec, const std::vector<const Tensor*>& state, const std::vector<std::vector<Tensor>>& batches,
             size_t steps) const;
  // Replays one step at a time until the state or an output goes non-finite; returns that step, its batch index and the state it started from.
  std::optional<std::tuple<size_t, size_t, std::vector<Tensor>>> replay(const RunSpec& spec, const std::vector<Tensor>& state,
                                                                       const std::vector<std::vector<Tensor>>& batches,
                                                                       size_t steps) const;
  Json validate(const std::vector<Tensor>& examples);
  std::vector<uint32_t> raw_outputs() const;

  // What the instrumented run of the traced graph found.
  struct Observed {
    std::vector<Json> roots, hard;
    size_t propagated = 0;
    std::vector<Tensor> vals;
  };

 private:
  Observed observed(const std::vector<Tensor>& inputs);
  std::pair<Json, std::vector<Json>> gradient_stats(const std::vector<Tensor>& vals) const;
  Json optimizer_check(const std::vector<Tensor>& examples) const;  // throws DiagError on mismatch
  std::pair<Json, std::vector<Json>> device_check(const std::vector<Tensor>& examples) const;
  std::pair<Json, std::vector<Json>> grad_check(const std::vector<Tensor>& examples) const;
};

// compile_mode (validate.rs:393-421): build, validate, and fall back to the standard plan when a
// rewrite fails the equivalence check.
std::unique_ptr<Compiled> compile_mode(const Graph& raw, const std::vector<uint32_t>& outputs,
                                       const std::vector<Tensor>& examples, Level level, Backend* device, OptMode mode);

Json device_failure(const std::string& device, const std::string& error);

}  // namespace rg
