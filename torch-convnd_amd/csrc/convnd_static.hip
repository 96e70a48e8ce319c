// Device scratch of the allocation-free forward (convnd_hip_forward_noalloc): one file-scope
// array per GPU, and the kernel that writes the implicit GEMM's geometry tables into it.
//
// The array holds, for the call in flight, [geometry tables | staged input | packed weights]
// (the same regions convnd_hip_forward takes from its caller's workspace). Every GPU the
// library runs on keeps its copy until the process ends. Host code never passes the array's
// name to a kernel or a copy (on the host that name is only a stand-in for the symbol): it
// uses the device address hipGetSymbolAddress returns, looked up once per device with that
// device current.

#include <mutex>

#include "convnd_geometry.h"
#include "convnd_internal.h"

namespace convnd {
namespace {

__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

// One thread per table entry (grid-stride): the per-entry code the host builder runs.
__global__ __launch_bounds__(kThreads) void igemm_tables_kernel(IgemmArgs A, unsigned char* tab) {
  const long n = igemm_table_entries(A);
  for (long e = blockIdx.x * (long)kThreads + threadIdx.x; e < n; e += (long)gridDim.x * kThreads)
    igemm_table_entry(A, tab, e);
}

}  // namespace

hipError_t noalloc_scratch(void** ptr) {
  static std::mutex lock;
  static void* addresses[kMaxDevices] = {};
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return err;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> guard(lock);
  if (addresses[dev] == nullptr) {
    void* p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess) return err;
    addresses[dev] = p;
  }
  *ptr = addresses[dev];
  return hipSuccess;
}

hipError_t launch_igemm_tables(const IgemmArgs& a, void* tables, hipStream_t stream) {
  const long n = igemm_table_entries(a);
  if (n <= 0) return hipSuccess;
  const long blocks = (n + kThreads - 1) / kThreads;
  hipLaunchKernelGGL(igemm_tables_kernel, dim3(static_cast<unsigned>(blocks < 1024 ? blocks : 1024)),
                     dim3(kThreads), 0, stream, a, static_cast<unsigned char*>(tables));
  return hipGetLastError();
}

}  // namespace convnd
