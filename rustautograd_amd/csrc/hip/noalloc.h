// Static scratch memory for the run loop variant that allocates nothing (rg_hip_exec_run_noalloc).
#pragma once
#include <cstdint>
#include <mutex>
#include <string>

// Bytes of the static scratch array each GPU holds: the step counter, the history record, the
// cycled batches and the state-copy temporaries of one run must fit in it.
#define RG_NOALLOC_SCRATCH_BYTES (32ull << 20)

namespace rgk {
// The current device's address of the static scratch array (looked up on the first call per
// device, then cached), or nullptr with a message. `hold` receives that device's run lock, taken:
// the caller keeps it for as long as it uses the array, so calls on one GPU take turns.
void* noalloc_scratch(std::string* err, std::unique_lock<std::mutex>* hold);
}  // namespace rgk
