// Device scratch of the entry point that allocates nothing
// (ppk_decode_step_noalloc): a file-scope device array, so every GPU the
// library runs on holds its own copy from the first use until the process
// ends, and no call ever needs hipMalloc / hipFree for the attention
// workspace (partial records of rows that span several blocks).
//
// Host code never passes `scratch` itself to a kernel: on the host its name
// is only a stand-in for the symbol. The device address of each GPU's copy is
// looked up once per device (hipGetSymbolAddress, with that device current)
// and kept in a per-device table; every kernel argument, copy or fill uses
// that address.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "ppk_internal.hpp"

static __device__ __align__(256) unsigned char scratch[ppk::kScratchBytes];

namespace ppk {
namespace {

constexpr int kMaxDevices = 64;

struct ScratchTable {
  std::mutex mutex;
  bool looked_up[kMaxDevices] = {};
  void* address[kMaxDevices] = {};
  hipError_t status[kMaxDevices] = {};
};

ScratchTable& table() {
  static ScratchTable t;
  return t;
}

}  // namespace

void* scratch_lookup(int device) {
  require(device >= 0 && device < kMaxDevices, "HIP device ordinal beyond the scratch table");
  ScratchTable& t = table();
  std::lock_guard<std::mutex> lock(t.mutex);
  if (!t.looked_up[device]) {
    DeviceGuard guard(device);  // the lookup resolves the copy of the current device
    void* ptr = nullptr;
    const hipError_t st = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    t.status[device] = st;
    t.address[device] = st == hipSuccess ? ptr : nullptr;
    t.looked_up[device] = true;
  }
  if (t.status[device] != hipSuccess)
    throw PreconditionError(std::string("device scratch address lookup failed: ") +
                            hipGetErrorString(t.status[device]));
  return t.address[device];
}

}  // namespace ppk
