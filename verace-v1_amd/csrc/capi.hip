// extern "C" entry points of libverace_sssd.so (declared in include/verace_sssd.h).
// Argument checking and dispatch only; the kernels live in sssd_*.hip / cham_*.hip.
#include <atomic>

#include "vmi_common.h"
#include "vmi_dispatch.h"

namespace {
thread_local int g_last_hip_error = 0;
constexpr int kMaxDevices = 64;
std::atomic<int> g_cu_count[kMaxDevices];  // 0: not queried yet
}  // namespace

namespace vmi {
int hip_status(hipError_t e) {
  if (e == hipSuccess) return VMI_OK;
  g_last_hip_error = static_cast<int>(e);
  return VMI_ERR_HIP;
}

hipError_t device_cu_count(int* cus) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev >= 0 && dev < kMaxDevices) {
    const int c = g_cu_count[dev].load(std::memory_order_relaxed);
    if (c > 0) {
      *cus = c;
      return hipSuccess;
    }
  }
  int c = 0;
  e = hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return e;
  if (dev >= 0 && dev < kMaxDevices) g_cu_count[dev].store(c, std::memory_order_relaxed);
  *cus = c;
  return hipSuccess;
}
}  // namespace vmi

namespace {

using vmi::hip_status;

bool valid_dtype(int dt) { return dt == VMI_F32 || dt == VMI_BF16 || dt == VMI_F16; }

bool ranges_overlap(const void* a, size_t abytes, const void* b, size_t bbytes) {
  const char* pa = static_cast<const char*>(a);
  const char* pb = static_cast<const char*>(b);
  return pa < pb + bbytes && pb < pa + abytes;
}

}  // namespace

extern "C" {

int vmi_version(void) { return 100; }

const char* vmi_status_string(int status) {
  switch (status) {
    case VMI_OK: return "ok";
    case VMI_ERR_INVALID_ARG: return "invalid argument";
    case VMI_ERR_UNSUPPORTED: return "unsupported head_dim/dtype combination";
    case VMI_ERR_WORKSPACE: return "workspace missing or too small";
    case VMI_ERR_ALIAS: return "forbidden aliasing between buffers";
    case VMI_ERR_HIP: return "HIP runtime error";
    case VMI_ERR_FULL: return "state cache layer full";
    default: return "unknown status";
  }
}

int vmi_last_hip_error(void) { return g_last_hip_error; }

int vmi_sssd_scan_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t D, int io_dtype,
                                  size_t* bytes) {
  if (bytes == nullptr || B < 0 || T < 0 || H < 0 || D < 1 || D > 256 || !valid_dtype(io_dtype))
    return VMI_ERR_INVALID_ARG;
  *bytes = vmi::scan_workspace_bytes(B, T, H, D, io_dtype);
  return VMI_OK;
}

int vmi_sssd_scan_fwd(const void* q, const void* k, const void* v, const void* delta,
                      int io_dtype, int delta_dtype, const float* psi_in, void* out,
                      float* psi_out, int64_t B, int64_t T, int64_t H, int64_t D, void* workspace,
                      size_t workspace_bytes, void* stream) {
  if (!valid_dtype(io_dtype) || !valid_dtype(delta_dtype)) return VMI_ERR_INVALID_ARG;
  if (B < 0 || T < 0 || H < 0 || D < 1) return VMI_ERR_INVALID_ARG;
  if (D > 256) return VMI_ERR_UNSUPPORTED;
  if (B * H > INT32_MAX || B * T * H > INT32_MAX) return VMI_ERR_INVALID_ARG;
  if (psi_out == nullptr) return VMI_ERR_INVALID_ARG;
  if (T > 0 && (q == nullptr || k == nullptr || v == nullptr || delta == nullptr))
    return VMI_ERR_INVALID_ARG;
  const size_t state_bytes = static_cast<size_t>(B * H) * D * D * sizeof(float);
  if (psi_in != nullptr && ranges_overlap(psi_in, state_bytes, psi_out, state_bytes))
    return VMI_ERR_ALIAS;
  const size_t need = vmi::scan_workspace_bytes(B, T, H, D, io_dtype);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) return VMI_ERR_WORKSPACE;
  if (B == 0 || H == 0) return VMI_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return hip_status(vmi::dispatch_scan(q, k, v, delta, io_dtype, delta_dtype, psi_in, out, psi_out,
                                       static_cast<int>(B), static_cast<int>(T),
                                       static_cast<int>(H), static_cast<int>(D), workspace,
                                       workspace_bytes, s));
}

int vmi_sssd_scan_bwd_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t D, size_t* bytes) {
  if (bytes == nullptr || B < 0 || T < 0 || H < 0 || D < 1) return VMI_ERR_INVALID_ARG;
  if (!vmi::sssd_bwd_supported(D)) return VMI_ERR_UNSUPPORTED;
  *bytes = vmi::use_bwd_chunk(T, D) ? vmi::sssd_bwd_chunk_workspace_bytes(B, T, H, D)
                                    : vmi::sssd_bwd_workspace_bytes(B, T, H, D);
  return VMI_OK;
}

int vmi_sssd_scan_bwd(const void* q, const void* k, const void* v, const void* delta,
                      int io_dtype, int delta_dtype, const float* psi_T, const void* d_out,
                      int d_out_dtype, const float* d_psi_T, void* dq, void* dk, void* dv,
                      void* d_delta, float* d_psi0, int64_t B, int64_t T, int64_t H, int64_t D,
                      void* workspace, size_t workspace_bytes, void* stream) {
  if (!valid_dtype(io_dtype) || !valid_dtype(delta_dtype) || !valid_dtype(d_out_dtype))
    return VMI_ERR_INVALID_ARG;
  if (B < 0 || T < 0 || H < 0 || D < 1) return VMI_ERR_INVALID_ARG;
  if (!vmi::sssd_bwd_supported(D)) return VMI_ERR_UNSUPPORTED;
  if (B * H > INT32_MAX || B * T * H > INT32_MAX) return VMI_ERR_INVALID_ARG;
  if (psi_T == nullptr) return VMI_ERR_INVALID_ARG;
  if (T > 0 && (q == nullptr || k == nullptr || v == nullptr || delta == nullptr ||
                d_out == nullptr || dq == nullptr || dk == nullptr || dv == nullptr ||
                d_delta == nullptr))
    return VMI_ERR_INVALID_ARG;
  const size_t state_bytes = static_cast<size_t>(B * H) * D * D * sizeof(float);
  if (d_psi0 != nullptr && (ranges_overlap(d_psi0, state_bytes, psi_T, state_bytes) ||
                            (d_psi_T != nullptr && ranges_overlap(d_psi0, state_bytes, d_psi_T, state_bytes))))
    return VMI_ERR_ALIAS;
  const bool chunked = vmi::use_bwd_chunk(T, D);
  const size_t need = chunked ? vmi::sssd_bwd_chunk_workspace_bytes(B, T, H, D)
                              : vmi::sssd_bwd_workspace_bytes(B, T, H, D);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) return VMI_ERR_WORKSPACE;
  if (B == 0 || H == 0) return VMI_OK;
  if (chunked)
    return hip_status(vmi::launch_sssd_bwd_chunk(q, k, v, delta, io_dtype, delta_dtype, psi_T,
                                                 d_out, d_out_dtype, d_psi_T, dq, dk, dv, d_delta,
                                                 d_psi0, static_cast<int>(B), static_cast<int>(T),
                                                 static_cast<int>(H), static_cast<int>(D),
                                                 workspace, static_cast<hipStream_t>(stream)));
  return hip_status(vmi::launch_sssd_bwd(q, k, v, delta, io_dtype, delta_dtype, psi_T, d_out,
                                         d_out_dtype, d_psi_T, dq, dk, dv, d_delta, d_psi0,
                                         static_cast<int>(B), static_cast<int>(T),
                                         static_cast<int>(H), static_cast<int>(D), workspace,
                                         static_cast<hipStream_t>(stream)));
}

int vmi_sssd_scan_fused_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t D, int io_dtype,
                                        size_t* bytes) {
  if (bytes == nullptr || B < 0 || T < 0 || H < 0 || D < 1 || !valid_dtype(io_dtype))
    return VMI_ERR_INVALID_ARG;
  if (!vmi::use_chunk_path(T, D, io_dtype)) return VMI_ERR_UNSUPPORTED;
  *bytes = vmi::chunk_workspace_bytes(B, T, H, D, io_dtype);
  return VMI_OK;
}

int vmi_sssd_scan_fused(const void* proj, int64_t proj_stride, int io_dtype, const uint8_t* mask,
                        const float* rms_weight, float rms_eps, const float* psi_in, void* out,
                        float* psi_out, int64_t B, int64_t T, int64_t H, int64_t D,
                        void* workspace, size_t workspace_bytes, void* stream) {
  if (!valid_dtype(io_dtype)) return VMI_ERR_INVALID_ARG;
  if (B < 0 || T < 0 || H < 0 || D < 1 || !(rms_eps >= 0.0f)) return VMI_ERR_INVALID_ARG;
  if (B * H > INT32_MAX || B * T > INT32_MAX) return VMI_ERR_INVALID_ARG;
  if (!vmi::use_chunk_path(T, D, io_dtype)) return VMI_ERR_UNSUPPORTED;
  if (proj == nullptr || out == nullptr || psi_out == nullptr) return VMI_ERR_INVALID_ARG;
  // 16-byte vector loads of every row: the row stride a multiple of 8 elements, the base aligned
  if (proj_stride < 3 * H * D + H || proj_stride % 8 != 0 ||
      reinterpret_cast<uintptr_t>(proj) % 16 != 0)
    return VMI_ERR_INVALID_ARG;
  const size_t state_bytes = static_cast<size_t>(B * H) * D * D * sizeof(float);
  if (psi_in != nullptr && ranges_overlap(psi_in, state_bytes, psi_out, state_bytes))
    return VMI_ERR_ALIAS;
  const size_t need = vmi::chunk_workspace_bytes(B, T, H, D, io_dtype);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) return VMI_ERR_WORKSPACE;
  if (B == 0 || H == 0) return VMI_OK;
  return hip_status(vmi::launch_sssd_chunked_fused(
      proj, proj_stride, io_dtype, mask, rms_weight, rms_eps, psi_in, out, psi_out, static_cast<int>(B),
      static_cast<int>(T), static_cast<int>(H), workspace, static_cast<hipStream_t>(stream)));
}

int vmi_sssd_step_inplace(const void* q, const void* k, const void* v, const void* delta,
                          int io_dtype, int delta_dtype, float* psi, void* out, int64_t B,
                          int64_t H, int64_t D, void* stream) {
  if (!valid_dtype(io_dtype) || !valid_dtype(delta_dtype)) return VMI_ERR_INVALID_ARG;
  if (B < 0 || H < 0 || D < 1) return VMI_ERR_INVALID_ARG;
  if (D > 256) return VMI_ERR_UNSUPPORTED;
  if (B * H > INT32_MAX) return VMI_ERR_INVALID_ARG;
  if (psi == nullptr || q == nullptr || k == nullptr || v == nullptr || delta == nullptr)
    return VMI_ERR_INVALID_ARG;
  if (B == 0 || H == 0) return VMI_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (vmi::use_step128(1, D))
    return hip_status(vmi::launch_sssd_step128(q, k, v, delta, io_dtype, delta_dtype, psi, out, psi,
                                               static_cast<int>(B),
                                               static_cast<int>(H), s));
  return hip_status(vmi::launch_sssd_seq(q, k, v, delta, io_dtype, delta_dtype, psi, out, psi,
                                         static_cast<int>(B), 1, static_cast<int>(H),
                                         static_cast<int>(D), s));
}

int vmi_sssd_step_fused(const void* proj, int64_t proj_stride, int io_dtype, const uint8_t* mask,
                        const float* rms_weight, float rms_eps, float* psi, void* out, int64_t B,
                        int64_t H, int64_t D, void* stream) {
  if (!valid_dtype(io_dtype)) return VMI_ERR_INVALID_ARG;
  if (B < 0 || H < 0 || D < 1 || !(rms_eps >= 0.0f)) return VMI_ERR_INVALID_ARG;
  if (!vmi::use_step128(1, D)) return VMI_ERR_UNSUPPORTED;
  if (B * H > INT32_MAX) return VMI_ERR_INVALID_ARG;
  if (proj == nullptr || psi == nullptr || proj_stride < 3 * H * D + H) return VMI_ERR_INVALID_ARG;
  if (B == 0 || H == 0) return VMI_OK;
  return hip_status(vmi::launch_sssd_step128_fused(proj, proj_stride, io_dtype, mask, rms_weight,
                                                   rms_eps, psi, out, static_cast<int>(B),
                                                   static_cast<int>(H),
                                                   static_cast<hipStream_t>(stream)));
}

int vmi_sssd_step_slots(const void* q, const void* k, const void* v, const void* delta,
                        int io_dtype, int delta_dtype, float* states, int64_t num_slots,
                        const int32_t* in_slot, const int32_t* out_slot, void* out, int64_t B,
                        int64_t H, int64_t D, void* stream) {
  if (!valid_dtype(io_dtype) || !valid_dtype(delta_dtype)) return VMI_ERR_INVALID_ARG;
  if (B < 0 || H < 0 || D < 1 || num_slots < 0) return VMI_ERR_INVALID_ARG;
  if (D > 256) return VMI_ERR_UNSUPPORTED;
  if (B * H > INT32_MAX || num_slots > INT32_MAX) return VMI_ERR_INVALID_ARG;
  if (B == 0 || H == 0) return VMI_OK;
  if (states == nullptr || in_slot == nullptr || out_slot == nullptr || out == nullptr ||
      q == nullptr || k == nullptr || v == nullptr || delta == nullptr)
    return VMI_ERR_INVALID_ARG;
  const vmi::StateMap map = {in_slot, out_slot, static_cast<int>(num_slots)};
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (vmi::use_step128(1, D))
    return hip_status(vmi::launch_sssd_step128(q, k, v, delta, io_dtype, delta_dtype, states, out,
                                               states, map, static_cast<int>(B),
                                               static_cast<int>(H), s));
  return hip_status(vmi::launch_sssd_seq(q, k, v, delta, io_dtype, delta_dtype, states, out,
                                         states, static_cast<int>(B), 1, static_cast<int>(H),
                                         static_cast<int>(D), s, map));
}

int vmi_cham_scan_workspace_bytes(int64_t B, int64_t T, int64_t h, size_t* bytes) {
  if (bytes == nullptr || B < 0 || T < 0 || h < 1) return VMI_ERR_INVALID_ARG;
  if (!vmi::cham_scan_supported(h)) return VMI_ERR_UNSUPPORTED;
  *bytes = vmi::cham_scan_workspace_bytes(B, T, h);
  return VMI_OK;
}

int vmi_cham_scan_fwd(const void* q, const void* k, const void* v, const void* gamma,
                      int io_dtype, int gamma_dtype, const float* h0_real, const float* h0_imag,
                      void* out, float* h_real_out, float* h_imag_out, int64_t B, int64_t T,
                      int64_t h, void* workspace, size_t workspace_bytes, void* stream) {
  if (!valid_dtype(io_dtype) || !valid_dtype(gamma_dtype)) return VMI_ERR_INVALID_ARG;
  if (B < 0 || T < 0 || h < 1 || B * T > INT32_MAX) return VMI_ERR_INVALID_ARG;
  if (!vmi::cham_scan_supported(h)) return VMI_ERR_UNSUPPORTED;
  // the per-token route above h = 1024: one item per grid row, 32-bit retraction indices
  if (h > vmi::kChamMaxDim && (B > 65535 || B * h * h > INT32_MAX)) return VMI_ERR_INVALID_ARG;
  if ((h0_real == nullptr) != (h0_imag == nullptr)) return VMI_ERR_INVALID_ARG;
  if (h_real_out == nullptr || h_imag_out == nullptr) return VMI_ERR_INVALID_ARG;
  if (T > 0 && (q == nullptr || k == nullptr || v == nullptr || gamma == nullptr || out == nullptr))
    return VMI_ERR_INVALID_ARG;
  const size_t state_bytes = static_cast<size_t>(B) * h * h * sizeof(float);
  if (h0_real != nullptr &&
      (ranges_overlap(h0_real, state_bytes, h_real_out, state_bytes) ||
       ranges_overlap(h0_real, state_bytes, h_imag_out, state_bytes) ||
       ranges_overlap(h0_imag, state_bytes, h_real_out, state_bytes) ||
       ranges_overlap(h0_imag, state_bytes, h_imag_out, state_bytes)))
    return VMI_ERR_ALIAS;
  const size_t need = vmi::cham_scan_workspace_bytes(B, T, h);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) return VMI_ERR_WORKSPACE;
  if (B == 0) return VMI_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return hip_status(vmi::launch_cham_scan(q, k, v, gamma, io_dtype, gamma_dtype, h0_real,
                                          h0_imag, out, h_real_out, h_imag_out,
                                          static_cast<int>(B), static_cast<int>(T),
                                          static_cast<int>(h), workspace, s));
}

int vmi_cham_scan_fused(const void* proj, int64_t proj_stride, int io_dtype, const uint8_t* mask,
                        void* out, float* h_real_out, float* h_imag_out, int64_t B, int64_t T,
                        int64_t h, void* workspace, size_t workspace_bytes, void* stream) {
  if (!valid_dtype(io_dtype)) return VMI_ERR_INVALID_ARG;
  if (B < 0 || T < 0 || h < 1 || B * T > INT32_MAX) return VMI_ERR_INVALID_ARG;
  if (!vmi::cham_fused_scan_supported(io_dtype, h)) return VMI_ERR_UNSUPPORTED;
  if (h_real_out == nullptr || h_imag_out == nullptr) return VMI_ERR_INVALID_ARG;
  // 16-byte vector loads of q rows and 8-byte loads of k, v rows: stride a multiple of 8
  // elements, the base and the output 16-byte aligned
  if (proj_stride < 3 * h + 1 || proj_stride % 8 != 0) return VMI_ERR_INVALID_ARG;
  if (T > 0 && (proj == nullptr || out == nullptr || reinterpret_cast<uintptr_t>(proj) % 16 != 0 ||
                reinterpret_cast<uintptr_t>(out) % 16 != 0))
    return VMI_ERR_INVALID_ARG;
  const size_t sb = static_cast<size_t>(B) * h * h * sizeof(float);
  if (B > 0 && ranges_overlap(h_real_out, sb, h_imag_out, sb)) return VMI_ERR_ALIAS;
  const size_t need = vmi::cham_scan_workspace_bytes(B, T, h);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) return VMI_ERR_WORKSPACE;
  if (B == 0) return VMI_OK;
  return hip_status(vmi::launch_cham_wide_fused(proj, proj_stride, io_dtype, mask, out, h_real_out,
                                                h_imag_out, static_cast<int>(B),
                                                static_cast<int>(T), static_cast<int>(h),
                                                workspace, static_cast<hipStream_t>(stream)));
}

int vmi_cham_step_workspace_bytes(int64_t B, int64_t h, size_t* bytes) {
  if (bytes == nullptr || B < 0 || h < 1) return VMI_ERR_INVALID_ARG;
  if (!vmi::cham_step_supported(h)) return VMI_ERR_UNSUPPORTED;
  *bytes = vmi::cham_step_workspace_bytes(B, h);
  return VMI_OK;
}

int vmi_cham_step_inplace(const void* q, const void* k, const void* v, const void* gamma,
                          int io_dtype, int gamma_dtype, float* h_real, float* h_imag,
                          float* r_real, float* r_imag, void* out, int64_t B, int64_t h,
                          void* workspace, size_t workspace_bytes, void* stream) {
  if (!valid_dtype(io_dtype) || !valid_dtype(gamma_dtype)) return VMI_ERR_INVALID_ARG;
  if (B < 0 || h < 1 || B > 65535) return VMI_ERR_INVALID_ARG;
  if (!vmi::cham_step_supported(h)) return VMI_ERR_UNSUPPORTED;
  if ((r_real == nullptr) != (r_imag == nullptr)) return VMI_ERR_INVALID_ARG;
  if (B > 0 && (q == nullptr || k == nullptr || v == nullptr || gamma == nullptr ||
                out == nullptr || h_real == nullptr || h_imag == nullptr))
    return VMI_ERR_INVALID_ARG;
  const size_t sb = static_cast<size_t>(B) * h * h * sizeof(float);
  if (B > 0 && ranges_overlap(h_real, sb, h_imag, sb)) return VMI_ERR_ALIAS;
  if (r_real != nullptr &&
      (ranges_overlap(r_real, sb, r_imag, sb) || ranges_overlap(r_real, sb, h_real, sb) ||
       ranges_overlap(r_real, sb, h_imag, sb) || ranges_overlap(r_imag, sb, h_real, sb) ||
       ranges_overlap(r_imag, sb, h_imag, sb)))
    return VMI_ERR_ALIAS;
  const size_t need = vmi::cham_step_workspace_bytes(B, h);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) return VMI_ERR_WORKSPACE;
  if (B == 0) return VMI_OK;
  return hip_status(vmi::launch_cham_step(q, k, v, gamma, io_dtype, gamma_dtype, h_real, h_imag,
                                          r_real, r_imag, out, static_cast<int>(B),
                                          static_cast<int>(h), workspace,
                                          static_cast<hipStream_t>(stream)));
}

int vmi_cham_step_fused(const void* proj, int64_t proj_stride, int io_dtype, const uint8_t* mask,
                        float* h_real, float* h_imag, float* r_real, float* r_imag, void* out,
                        int64_t B, int64_t h, void* workspace, size_t workspace_bytes,
                        void* stream) {
  if (!valid_dtype(io_dtype)) return VMI_ERR_INVALID_ARG;
  if (B < 0 || h < 1 || B > 65535) return VMI_ERR_INVALID_ARG;
  if (!vmi::cham_step_fused_supported(h)) return VMI_ERR_UNSUPPORTED;
  if ((r_real == nullptr) != (r_imag == nullptr)) return VMI_ERR_INVALID_ARG;
  if (proj_stride < 3 * h + 1) return VMI_ERR_INVALID_ARG;
  if (B > 0 && (proj == nullptr || out == nullptr || h_real == nullptr || h_imag == nullptr))
    return VMI_ERR_INVALID_ARG;
  const size_t sb = static_cast<size_t>(B) * h * h * sizeof(float);
  if (B > 0 && ranges_overlap(h_real, sb, h_imag, sb)) return VMI_ERR_ALIAS;
  if (r_real != nullptr &&
      (ranges_overlap(r_real, sb, r_imag, sb) || ranges_overlap(r_real, sb, h_real, sb) ||
       ranges_overlap(r_real, sb, h_imag, sb) || ranges_overlap(r_imag, sb, h_real, sb) ||
       ranges_overlap(r_imag, sb, h_imag, sb)))
    return VMI_ERR_ALIAS;
  const size_t need = vmi::cham_step_workspace_bytes(B, h);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) return VMI_ERR_WORKSPACE;
  if (B == 0) return VMI_OK;
  return hip_status(vmi::launch_cham_step_fused(proj, proj_stride, io_dtype, mask, h_real, h_imag,
                                                r_real, r_imag, out, static_cast<int>(B), workspace,
                                                static_cast<hipStream_t>(stream)));
}

int vmi_cham_ns_workspace_bytes(int64_t batch, int64_t n, size_t* bytes) {
  if (bytes == nullptr || batch < 0 || n < 1) return VMI_ERR_INVALID_ARG;
  *bytes = vmi::ns_workspace_bytes(batch, n);
  return VMI_OK;
}

int vmi_cham_ns_retraction(const float* h_real, const float* h_imag, float* out_real,
                           float* out_imag, int64_t batch, int64_t n, int steps, void* workspace,
                           size_t workspace_bytes, void* stream) {
  if (batch < 0 || n < 1 || steps < 0) return VMI_ERR_INVALID_ARG;
  if (batch * n * n > INT32_MAX) return VMI_ERR_INVALID_ARG;
  if (h_real == nullptr || h_imag == nullptr || out_real == nullptr || out_imag == nullptr)
    return VMI_ERR_INVALID_ARG;
  const size_t need = vmi::ns_workspace_bytes(batch, n);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) return VMI_ERR_WORKSPACE;
  if (batch == 0) return VMI_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return hip_status(vmi::launch_ns_retraction(h_real, h_imag, out_real, out_imag,
                                              static_cast<int>(batch), static_cast<int>(n), steps,
                                              workspace, s));
}

}  // extern "C"
