// vmi_sssd_scan_fwd_noalloc: the prefill scan of vmi_sssd_scan_fwd with its workspace taken
// from a fixed device array of this library instead of a caller-provided buffer, for callers
// that cannot allocate device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc).  It has no counterpart in the reference.
//
// The array `scratch` holds kScratchBytes on every GPU the library runs on, from the first
// use of the library's code object on that device until the process ends.  Its device
// address is looked up once per device (hipGetSymbolAddress, with that device current) and
// kept; the host never passes the array's name to a kernel.  Every call on one GPU shares
// that GPU's array: calls that overlap on one GPU (two streams, two host threads) race on
// it, so order them.  The scan's workspace needs no clearing: every part transform and
// segment start state it holds is written by the scan's first two passes before it is read.
#include <mutex>

#include "vmi_common.h"
#include "vmi_dispatch.h"

namespace {

constexpr size_t kScratchBytes = size_t(40) << 20;  // 40 MiB per GPU
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device (looked up on the first call there).
hipError_t scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (p == nullptr) return hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return hipSuccess;
}

bool valid_dtype(int dt) { return dt == VMI_F32 || dt == VMI_BF16 || dt == VMI_F16; }

}  // namespace

extern "C" int vmi_sssd_scan_fwd_noalloc(const void* q, const void* k, const void* v,
                                         const void* delta, int io_dtype, int delta_dtype,
                                         const float* psi_in, void* out, float* psi_out,
                                         int64_t B, int64_t T, int64_t H, int64_t D,
                                         void* stream) {
  if (!valid_dtype(io_dtype) || !valid_dtype(delta_dtype)) return VMI_ERR_INVALID_ARG;
  if (B < 0 || T < 0 || H < 0 || D < 1) return VMI_ERR_INVALID_ARG;
  if (D > 256) return VMI_ERR_UNSUPPORTED;
  if (B * H > INT32_MAX || B * T * H > INT32_MAX) return VMI_ERR_INVALID_ARG;
  if (psi_out == nullptr) return VMI_ERR_INVALID_ARG;
  if (T > 0 && (q == nullptr || k == nullptr || v == nullptr || delta == nullptr))
    return VMI_ERR_INVALID_ARG;
  const size_t state_bytes = static_cast<size_t>(B * H) * D * D * sizeof(float);
  if (psi_in != nullptr) {
    const char* a = reinterpret_cast<const char*>(psi_in);
    const char* b = reinterpret_cast<const char*>(psi_out);
    if (a < b + state_bytes && b < a + state_bytes) return VMI_ERR_ALIAS;
  }
  const size_t need = vmi::scan_workspace_bytes(B, T, H, D, io_dtype);
  if (need > kScratchBytes) return VMI_ERR_WORKSPACE;  // beyond the fixed array: use vmi_sssd_scan_fwd
  if (B == 0 || H == 0) return VMI_OK;
  void* ws = nullptr;
  if (need > 0) {
    const hipError_t e = scratch_address(&ws);
    if (e != hipSuccess) return vmi::hip_status(e);
  }
  return vmi::hip_status(vmi::dispatch_scan(q, k, v, delta, io_dtype, delta_dtype, psi_in, out,
                                            psi_out, static_cast<int>(B), static_cast<int>(T),
                                            static_cast<int>(H), static_cast<int>(D), ws, need,
                                            static_cast<hipStream_t>(stream)));
}
