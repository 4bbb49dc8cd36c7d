// trs_spmm_f16_noalloc: trs_spmm_f16 with its workspace (partial slots, staged hot rows) taken from
// a static device array instead of the caller, for callers that cannot allocate device memory
// (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  It
// launches the same kernels with the same arguments, so its output is bitwise equal to
// trs_spmm_f16's.
//
// The array `scratch` below is held by every GPU the library runs on, at its own address on each,
// until the process ends.  Host code never uses the array's name as a device address (in host code
// it only names a host-side stand-in): on the first call on a device, with that device current,
// hipGetSymbolAddress looks the address up, and that pointer -- kept per device -- is what the
// kernels receive.  All calls on one GPU share its array: calls that overlap on one GPU (several
// streams or threads at once) race and must be serialised by the caller.  Nothing needs clearing
// between calls: every partial slot a call's fixup kernel reads, and every staged row its task
// kernels read, was written earlier in that call.
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <string>

#include "trspmm.h"

namespace trs {
void set_error(const std::string& msg);
}

namespace {

constexpr int64_t kScratchBytes = TRS_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

std::mutex g_mu;
std::map<int, void*> g_scratch;   // device -> address of `scratch` on that device

int fail(int code, const std::string& msg) {
  trs::set_error(msg);
  return code;
}

// Address of `scratch` on the current device, looked up once per device.
int scratch_address(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return fail(TRS_EDEVICE, "trs_spmm_f16_noalloc: no HIP device available");
  }
  std::lock_guard<std::mutex> lock(g_mu);
  auto it = g_scratch.find(dev);
  if (it == g_scratch.end()) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      (void)hipGetLastError();
      return fail(TRS_EDEVICE, std::string("trs_spmm_f16_noalloc: hipGetSymbolAddress of the scratch array "
                                           "failed: ") + hipGetErrorString(e));
    }
    it = g_scratch.emplace(dev, ptr).first;
  }
  *out = it->second;
  return TRS_OK;
}

}  // namespace

extern "C" int trs_spmm_f16_noalloc(const trs_plan* p, const uint16_t* B, int64_t ldb, int32_t K, float* C,
                                    int64_t ldc, void* stream) {
  if (!p) return fail(TRS_EINVAL, "NULL plan");
  if (K < 0) return fail(TRS_EINVAL, "K must be non-negative");
  const int64_t need = trs_spmm_workspace_bytes(p, K);
  if (need > kScratchBytes)
    return fail(TRS_EINVAL, "trs_spmm_f16_noalloc: the plan's workspace needs " + std::to_string(need) +
                                " bytes at K = " + std::to_string(K) + ", more than the " +
                                std::to_string(kScratchBytes) +
                                "-byte scratch array holds; call trs_spmm_f16 with a workspace instead");
  void* ws = nullptr;
  if (need > 0) {
    const int rc = scratch_address(&ws);
    if (rc) return rc;
  }
  // trs_spmm_f16 checks the plan's device against the current one (whose scratch address this is)
  // before it launches anything
  return trs_spmm_f16(p, B, ldb, K, C, ldc, ws, need, stream);
}
