// Kernel-family selection for the prefill scan:
//   bf16/fp16 I/O, head_dim 128, T >= 32  -> chunk-parallel MFMA scan (sssd_chunk.hip)
//   T == 1, head_dim 128 (any I/O dtype)   -> persistent single-step kernel (sssd_step.hip)
//   everything else (fp32 I/O, other head_dim, short T) -> token-sequential fp32
//   scan (sssd_seq.hip)
#include "vmi_common.h"
#include "vmi_dispatch.h"

namespace vmi {

size_t scan_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t D, int io_dtype) {
  return chunk_workspace_bytes(B, T, H, D, io_dtype);
}

hipError_t dispatch_scan(const void* q, const void* k, const void* v, const void* delta,
                         int io_dtype, int delta_dtype, const float* psi_in, void* out,
                         float* psi_out, int B, int T, int H, int D, void* workspace,
                         size_t workspace_bytes, hipStream_t stream) {
  (void)workspace_bytes;
  if (use_chunk_path(T, D, io_dtype))
    return launch_sssd_chunked(q, k, v, delta, io_dtype, delta_dtype, psi_in, out, psi_out, B, T,
                               H, workspace, stream);
  if (use_step128(T, D))
    return launch_sssd_step128(q, k, v, delta, io_dtype, delta_dtype, psi_in, out, psi_out,
                               B, H, stream);
  return launch_sssd_seq(q, k, v, delta, io_dtype, delta_dtype, psi_in, out, psi_out, B, T, H, D,
                         stream);
}

}  // namespace vmi
