// gdnr_status.hip -- the device word through which kernels report bounded
// waits that gave up (an LDS flag never raised), its host read-out and the
// waits' poll budget; the
// device array of the split replay entry point that allocates nothing; the
// compute-unit count of the current device.
//
// One word per device (a file-scope __device__ variable: every GPU that
// loads the library holds its own copy). Kernels add to it with a global
// atomic; the host reads and optionally clears it with gdnr_wait_timeouts().
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "gdnr_internal.h"

namespace gdnr {

__device__ uint32_t wait_status_word[1];

namespace {
constexpr int kMaxDevices = 64;
uint32_t* g_status_ptr[kMaxDevices] = {};
}  // namespace

uint32_t* status_word() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  if (!g_status_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(wait_status_word)) != hipSuccess) return nullptr;
    g_status_ptr[dev] = (uint32_t*)p;  // the same address on every call: a benign race between threads
  }
  return g_status_ptr[dev];
}

// The poll budget of the bounded waits, read by the launchers at each
// launch. Lowering it is a test of the give-up path: with 0 every wait
// gives up at once, the kernels still run to their end, and the waves whose
// waits gave up leave the checkpoint and its scales as they were.
namespace {
std::atomic<uint32_t> g_wait_polls{kWaitPolls};
}  // namespace
uint32_t wait_polls() { return g_wait_polls.load(std::memory_order_relaxed); }
uint32_t set_wait_polls(uint32_t polls) { return g_wait_polls.exchange(polls, std::memory_order_relaxed); }

int read_status(uint32_t* count, bool reset) {
  uint32_t* p = status_word();
  if (!p) return (int)hipErrorInvalidSymbol;
  hipError_t e = hipMemcpy(count, p, sizeof(uint32_t), hipMemcpyDeviceToHost);
  if (e == hipSuccess && reset) e = hipMemset(p, 0, sizeof(uint32_t));
  if (e == hipSuccess) e = hipDeviceSynchronize();
  return (int)e;
}

// The split replay's scratch for the entry point that allocates nothing. One
// array per GPU for the life of the process; host code reaches it through
// the address hipGetSymbolAddress returns on that GPU, never through the
// array's name (a host-side stand-in).
static __device__ __align__(256) uint8_t scratch[kSplitScratchBytes];
static uint8_t* g_scratch_ptr[kMaxDevices] = {};

uint8_t* split_scratch() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess) return nullptr;
    g_scratch_ptr[dev] = (uint8_t*)p;  // the same address on every call: a benign race between threads
  }
  return g_scratch_ptr[dev];
}

// compute units of the current device (cached per device; 256 if the query fails)
int device_cus() {
  static int cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cus[dev]) {
    int n = 0;
    cus[dev] = (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0) ? n : 256;
  }
  return cus[dev];
}

}  // namespace gdnr
