// Internal launch functions shared between the kernel files and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace vmi {

// sssd_seq.hip: token-sequential fp32 scan, one workgroup per (b, h).
hipError_t launch_sssd_seq(const void* q, const void* k, const void* v, const void* delta,
                           int io_dtype, int delta_dtype, const float* psi_in, void* out,
                           float* psi_out, int B, int T, int H, int D, hipStream_t stream);

// sssd_step.hip: single-token step for head_dim 128 (persistent, loads of the next
// head overlap the update and store of the current one).  psi_in may equal psi_out.
bool use_step128(int64_t T, int64_t D);
hipError_t launch_sssd_step128(const void* q, const void* k, const void* v, const void* delta,
                               int io_dtype, int delta_dtype, const float* psi_in, void* out,
                               float* psi_out, int BH, hipStream_t stream);

// sssd_scan.hip: picks the kernel family for a prefill scan.
size_t scan_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t D, int io_dtype);
hipError_t dispatch_scan(const void* q, const void* k, const void* v, const void* delta,
                         int io_dtype, int delta_dtype, const float* psi_in, void* out,
                         float* psi_out, int B, int T, int H, int D, void* workspace,
                         size_t workspace_bytes, hipStream_t stream);

// sssd_chunk.hip: chunk-parallel MFMA scan (bf16/fp16 I/O, head_dim 128).
bool use_chunk_path(int64_t T, int64_t D, int io_dtype);
size_t chunk_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t D, int io_dtype);
hipError_t launch_sssd_chunked(const void* q, const void* k, const void* v, const void* delta,
                               int io_dtype, int delta_dtype, const float* psi_in, void* out,
                               float* psi_out, int B, int T, int H, void* workspace,
                               hipStream_t stream);

// cham_ns.hip: Newton-Schulz unitary retraction.
size_t ns_workspace_bytes(int64_t batch, int64_t n);
hipError_t launch_ns_retraction(const float* h_real, const float* h_imag, float* out_real,
                                float* out_imag, int batch, int n, int steps, void* workspace,
                                hipStream_t stream);

}  // namespace vmi
