// Kernel-family selection for the prefill scan.
#include "vmi_common.h"
#include "vmi_dispatch.h"

namespace vmi {

size_t scan_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t D, int io_dtype) {
  (void)B; (void)T; (void)H; (void)D; (void)io_dtype;
  return 0;
}

hipError_t dispatch_scan(const void* q, const void* k, const void* v, const void* delta,
                         int io_dtype, int delta_dtype, const float* psi_in, void* out,
                         float* psi_out, int B, int T, int H, int D, void* workspace,
                         size_t workspace_bytes, hipStream_t stream) {
  (void)workspace; (void)workspace_bytes;
  return launch_sssd_seq(q, k, v, delta, io_dtype, delta_dtype, psi_in, out, psi_out, B, T, H, D,
                         stream);
}

}  // namespace vmi
