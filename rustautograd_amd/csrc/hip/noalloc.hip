// The static scratch memory of rg_hip_exec_run_noalloc: a file-scope device array, so that the
// entry point allocates nothing. Each GPU the library runs on holds its own copy, at its own
// address, until the process ends. Host code never uses the array's name as an address (on the
// host it is only a stand-in symbol): the device address comes from hipGetSymbolAddress, looked
// up once per device with that device current, and is what kernels receive.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "noalloc.h"

namespace {

static __device__ __align__(256) unsigned char scratch[RG_NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex g_mu;
void* g_ptr[MAX_DEVICES] = {};
// One lock per device, held by a run for its whole call: runs on one GPU share that GPU's array,
// so they take turns instead of overwriting each other's counter, history and temporaries.
std::mutex g_run_mu[MAX_DEVICES];

}  // namespace

namespace rgk {

void* noalloc_scratch(std::string* err, std::unique_lock<std::mutex>* hold) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= MAX_DEVICES) {
    *err = std::string("no current HIP device for the static scratch: ") + hipGetErrorString(e);
    return nullptr;
  }
  *hold = std::unique_lock<std::mutex>(g_run_mu[dev]);
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      *err = std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(e);
      return nullptr;
    }
    g_ptr[dev] = ptr;
  }
  return g_ptr[dev];
}

}  // namespace rgk
