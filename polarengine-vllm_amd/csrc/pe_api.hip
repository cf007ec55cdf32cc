// Host-side glue of the C ABI: status text, device queries, launch checks.

#include "pe_common.h"

#include <atomic>

namespace pe {

static std::atomic<int> g_cus[64];

int num_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int v = g_cus[dev].load(std::memory_order_relaxed);
  if (v > 0) return v;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  g_cus[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

int launch_status() {
  return hipGetLastError() == hipSuccess ? PE_OK : PE_ERR_LAUNCH;
}

}  // namespace pe

extern "C" const char* pe_status_string(int status) {
  switch (status) {
    case PE_OK: return "ok";
    case PE_ERR_NULL: return "a required pointer is NULL";
    case PE_ERR_DIMS: return "unsupported or inconsistent dimensions";
    case PE_ERR_BITS: return "unsupported bit width / codebook size";
    case PE_ERR_ALIGN: return "pointer or stride not 16-byte aligned";
    case PE_ERR_DTYPE: return "unsupported dtype or layout";
    case PE_ERR_WORKSPACE: return "workspace missing or too small";
    case PE_ERR_LAUNCH: return "kernel launch failed";
    case PE_ERR_DEVICE: return "device query failed";
    case PE_ERR_SCRATCH:
      return "the call needs more scratch than pe_linear_forward_noalloc holds "
             "(pe_linear_noalloc_max_bytes)";
    default: return "unknown status";
  }
}

extern "C" int pe_abi_version(void) { return 4; }
