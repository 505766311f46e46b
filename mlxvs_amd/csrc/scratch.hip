// The fixed device scratch of the no-allocation entry point
// (mlxvs_brute_force_knn_device_noalloc): a file-scope device array each GPU
// the library runs on holds until the process ends, so that a call can find
// its workspace without hipMalloc (callers under graph capture, serving
// loops and harnesses that forbid allocation).
//
// In host code `scratch` names a host-side stand-in, not the device memory:
// its device address comes from hipGetSymbolAddress, called once per device
// with that device current, and only that address is handed to kernels.
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <stdexcept>
#include <string>

#include "knn_kernels.h"

namespace mlxvs::kern {
namespace {

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mutex;
std::map<int, void*> g_scratch_ptr;

}  // namespace

void* scratch_address() {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    throw std::runtime_error(std::string("[mlxvs] hipGetDevice: ") + hipGetErrorString(e));
  std::lock_guard<std::mutex> g(g_scratch_mutex);
  auto it = g_scratch_ptr.find(dev);
  if (it != g_scratch_ptr.end()) return it->second;
  void* p = nullptr;
  e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || p == nullptr)
    throw std::runtime_error(std::string("[mlxvs] hipGetSymbolAddress (scratch): ") +
                             hipGetErrorString(e));
  g_scratch_ptr[dev] = p;
  return p;
}

}  // namespace mlxvs::kern
