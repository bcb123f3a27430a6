// Internal launch functions shared between the kernel files and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace vmi {

// capi.hip: maps a HIP error to VMI_ERR_HIP and records it for vmi_last_hip_error().
int hip_status(hipError_t e);

// capi.hip: the compute-unit count of the current device, queried once per device and
// cached (launchers that size their grid by it make no runtime query per launch).
hipError_t device_cu_count(int* cus);

// Where the [D, D] state of head bh = b*H + h (batch item b, head h) lives, as an index
// into psi_in / psi_out in units of D*D floats:
//   DenseStates  index bh (the reference layout [B, H, D, D]);
//   StateMap     slots of a decode state cache: psi_in and psi_out are the same pool of
//                nslots slots of H states each, item b reads slot in_slot[b] and writes
//                slot out_slot[b] (device arrays);
//   SlotArgs     the same with the slot indexes carried in the kernel arguments (no
//                device array, no host-to-device copy; at most kMaxSlotArgs items).
// In the slotted maps an input index outside [0, nslots) (-1 by convention) starts from
// the identity and an output index outside it drops the state write.
struct DenseStates {
  static constexpr bool kSlotted = false;  // every index valid: no guard on the writes
  __device__ __forceinline__ int64_t in_index(int bh, int) const { return bh; }
  __device__ __forceinline__ int64_t out_index(int bh, int) const { return bh; }
  __device__ __forceinline__ bool skip(int) const { return false; }
};

// Dense states, and only the sequences whose flag word holds `tag` run (the others leave
// their outputs and states untouched): the fp32 recompute of the sequences a chunk scan
// found outside its accuracy envelope (rotation_outside_chunk_envelope).
struct FlaggedStates {
  static constexpr bool kSlotted = false;
  const uint32_t* flags;  // [B * H]
  uint32_t tag;
  __device__ __forceinline__ int64_t in_index(int bh, int) const { return bh; }
  __device__ __forceinline__ int64_t out_index(int bh, int) const { return bh; }
  __device__ __forceinline__ bool skip(int bh) const { return flags[bh] != tag; }
};

__device__ __forceinline__ int64_t slot_index(int s, int nslots, int bh, int H) {
  return (s >= 0 && s < nslots) ? static_cast<int64_t>(s) * H + bh % H : -1;
}

struct StateMap {
  static constexpr bool kSlotted = true;
  const int32_t* in_slot;
  const int32_t* out_slot;
  int nslots;
  __device__ __forceinline__ int64_t in_index(int bh, int H) const {
    return slot_index(in_slot[bh / H], nslots, bh, H);
  }
  __device__ __forceinline__ int64_t out_index(int bh, int H) const {
    return slot_index(out_slot[bh / H], nslots, bh, H);
  }
  __device__ __forceinline__ bool skip(int) const { return false; }
};

constexpr int kMaxSlotArgs = 256;
struct SlotArgs {
  static constexpr bool kSlotted = true;
  int32_t in_slot[kMaxSlotArgs];
  int32_t out_slot[kMaxSlotArgs];
  int nslots;
  __device__ __forceinline__ int64_t in_index(int bh, int H) const {
    return slot_index(in_slot[bh / H], nslots, bh, H);
  }
  __device__ __forceinline__ int64_t out_index(int bh, int H) const {
    return slot_index(out_slot[bh / H], nslots, bh, H);
  }
  __device__ __forceinline__ bool skip(int) const { return false; }
};

// sssd_seq.hip: token-sequential fp32 scan, one workgroup per (b, h).
hipError_t launch_sssd_seq(const void* q, const void* k, const void* v, const void* delta,
                           int io_dtype, int delta_dtype, const float* psi_in, void* out,
                           float* psi_out, int B, int T, int H, int D, hipStream_t stream);
hipError_t launch_sssd_seq(const void* q, const void* k, const void* v, const void* delta,
                           int io_dtype, int delta_dtype, const float* psi_in, void* out,
                           float* psi_out, int B, int T, int H, int D, hipStream_t stream,
                           const StateMap& map);
hipError_t launch_sssd_seq(const void* q, const void* k, const void* v, const void* delta,
                           int io_dtype, int delta_dtype, const float* psi_in, void* out,
                           float* psi_out, int B, int T, int H, int D, hipStream_t stream,
                           const SlotArgs& map);
hipError_t launch_sssd_seq(const void* q, const void* k, const void* v, const void* delta,
                           int io_dtype, int delta_dtype, const float* psi_in, void* out,
                           float* psi_out, int B, int T, int H, int D, hipStream_t stream,
                           const FlaggedStates& map);

// sssd_step.hip: single-token step for head_dim 128 (persistent, two workgroups per CU,
// heads in units of 64 columns whose loads run one unit ahead of the update and store).
// psi_in may equal psi_out;
// `map` places the states (dense, or slots of a decode state cache).
bool use_step128(int64_t T, int64_t D);
hipError_t launch_sssd_step128(const void* q, const void* k, const void* v, const void* delta,
                               int io_dtype, int delta_dtype, const float* psi_in, void* out,
                               float* psi_out, int B, int H, hipStream_t stream);
hipError_t launch_sssd_step128(const void* q, const void* k, const void* v, const void* delta,
                               int io_dtype, int delta_dtype, const float* psi_in, void* out,
                               float* psi_out, const StateMap& map, int B, int H,
                               hipStream_t stream);
hipError_t launch_sssd_step128(const void* q, const void* k, const void* v, const void* delta,
                               int io_dtype, int delta_dtype, const float* psi_in, void* out,
                               float* psi_out, const SlotArgs& map, int B, int H,
                               hipStream_t stream);

// The same step fused with the projections around it (head_dim 128, states in place):
// proj [B, stride] raw (x [W_q; W_k; W_v; W_delta]^T, one row per item); q, k, v normalised and
// delta = 0.1 sigmoid(.) * mask in the kernel; out = head_rmsnorm(o) when rms_w is given.
hipError_t launch_sssd_step128_fused(const void* proj, int64_t proj_stride, int io_dtype,
                                     const uint8_t* mask, const float* rms_w, float rms_eps,
                                     float* psi, void* out, int B, int H, hipStream_t stream);

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

// sssd_xsplit.hip: single-pass column-split scan (bf16/fp16 I/O, head_dim 128), four
// cooperating workgroups per sequence; taken by launch_sssd_chunked when use_xsplit holds.
bool use_xsplit(int64_t B, int64_t T, int64_t H, int64_t D, int io_dtype);
size_t xsplit_workspace_bytes(int64_t B, int64_t H);
hipError_t launch_sssd_xsplit(const void* q, const void* k, const void* v, const void* delta,
                              int io_dtype, int delta_dtype, const float* psi_in, void* out,
                              float* psi_out, int B, int T, int H, void* workspace,
                              uint32_t* flags, uint32_t ftag, hipStream_t stream);

// sssd_chunk.hip, fused projections: proj [B, T, 3HD + H] raw (x [W_q; W_k; W_v; W_delta]^T);
// q, k, v normalised and delta = 0.1 sigmoid(.) * mask in the kernel; out = head_rmsnorm(o)
// when rms_w is given (else o).  Needs use_chunk_path(T, 128, io_dtype).
hipError_t launch_sssd_chunked_fused(const void* proj, int64_t proj_stride, int io_dtype,
                                     const uint8_t* mask,
                                     const float* rms_w, float rms_eps, const float* psi_in,
                                     void* out, float* psi_out, int B, int T, int H,
                                     void* workspace, hipStream_t stream);

// cham_scan.hip: CHAM holographic scan (h <= 128 there, 128 < h <= kChamMaxDim routed to
// cham_wide.hip, larger h to the per-token steps of cham_step.hip): raw complex state with
// exact Cayley rank-2 updates, readout Re(NS_3(H_t) q_t).
constexpr int64_t kChamMaxDim = 1024;
bool cham_scan_supported(int64_t h);
size_t cham_scan_workspace_bytes(int64_t B, int64_t T, int64_t h);
hipError_t launch_cham_scan(const void* q, const void* k, const void* v, const void* gamma,
                            int io_dtype, int gamma_dtype, const float* h0r, const float* h0i,
                            void* out, float* hr_out, float* hi_out, int B, int T, int h,
                            void* workspace, hipStream_t stream);

// cham_step.hip: single-token CHAM step, states updated in place (cham_step_supported: h % 4
// == 0, h <= 4096); rr/ri (the readout state) may be null (then the readout uses H).
bool cham_step_supported(int64_t h);
size_t cham_step_workspace_bytes(int64_t B, int64_t h);
hipError_t launch_cham_step(const void* q, const void* k, const void* v, const void* gamma,
                            int io_dtype, int gamma_dtype, float* hr, float* hi, float* rr,
                            float* ri, void* out, int B, int h, void* workspace,
                            hipStream_t stream);

// The same fused with the projections before it (h = 1024, dense states): proj [B, stride] raw
// (x [W_q; W_k; W_v; W_gamma]^T, one row per item); v = silu(.), q, k, v normalised and gamma =
// 0.1 sigmoid(.) * mask in the kernel.  Workspace as cham_step_workspace_bytes(B, 1024).
bool cham_step_fused_supported(int64_t h);
hipError_t launch_cham_step_fused(const void* proj, int64_t proj_stride, int io_dtype,
                                  const uint8_t* mask, float* hr, float* hi, float* rr, float* ri,
                                  void* out, int B, void* workspace, hipStream_t stream);

// The same over the hologram pool of a decode state cache ([N, 2, h, h] per layer: slot s's
// real plane at pool + 2 s h^2, imaginary plane after it), in_slot / out_slot host arrays of
// B <= kMaxSlotArgs items (-1 in: the identity); no readout state (every cached hologram
// started from the identity, so NS_3(H) = H).
hipError_t launch_cham_step_slots(const void* q, const void* k, const void* v, const void* gamma,
                                  int io_dtype, int gamma_dtype, float* pool, const int32_t* in_slot,
                                  const int32_t* out_slot, void* out, int B, int h, void* workspace,
                                  hipStream_t stream);

// cham_step.hip: the holographic scan for kChamMaxDim < h (cham_step_supported), one step per
// token (H_0 copied to the outputs, R_0 = NS_3(H_0) in the workspace when H_0 is given).
size_t cham_step_scan_workspace_bytes(int64_t B, int64_t h);
hipError_t launch_cham_step_scan(const void* q, const void* k, const void* v, const void* gamma,
                                 int io_dtype, int gamma_dtype, const float* h0r,
                                 const float* h0i, void* out, float* hr_out, float* hi_out, int B,
                                 int T, int h, void* workspace, hipStream_t stream);

// cham_wide.hip: the same scan for 128 < h <= kChamMaxDim.
size_t cham_wide_workspace_bytes(int64_t B, int64_t T, int64_t h);
hipError_t launch_cham_wide(const void* q, const void* k, const void* v, const void* gamma,
                            int io_dtype, int gamma_dtype, const float* h0r, const float* h0i,
                            void* out, float* hr_out, float* hi_out, int B, int T, int h,
                            void* workspace, hipStream_t stream);

// cham_wide.hip: the scan fused with the projections before it (identity start, 16-bit I/O,
// 128 < h <= kChamMaxDim, h % 8 == 0): proj [B, T, stride] raw (x [W_q; W_k; W_v; W_gamma]^T;
// q at 0, k at h, v at 2h, the gamma logit at 3h; stride % 8 == 0, 16-byte aligned base);
// v = silu(v), q, k, v normalised and gamma = 0.1 sigmoid(.) * mask[b*T + t] in the kernels.
// Workspace as cham_scan_workspace_bytes.
bool cham_fused_scan_supported(int io_dtype, int64_t h);
hipError_t launch_cham_wide_fused(const void* proj, int64_t proj_stride, int io_dtype,
                                  const uint8_t* mask, void* out, float* hr_out, float* hi_out,
                                  int B, int T, int h, void* workspace, hipStream_t stream);

// cham_mfma.hip: the wide route's state carry on the matrix cores (16-bit k, v, h % 8 == 0,
// 16-byte aligned k, v; entries of k, v below 65504 in magnitude, as L2-normalised rows are).
bool cham_mfma_usable(int io_dtype, int h, const void* k, const void* v);
size_t cham_mfma_workspace_bytes(int64_t B, int64_t T, int64_t hp);  // hp: padded h
// identity start (no initial hologram): the whole scan, state carry with f16 snapshots in the
// `snap` buffer (cham_mfma_snap16_bytes) and the chunked readout into `out`; q and out 16-byte
// aligned besides cham_mfma_usable's conditions
size_t cham_mfma_snap16_bytes(int64_t B, int64_t T, int64_t hp);
hipError_t launch_cham_mfma_scan(const void* q, const void* k, const void* v, int io_dtype,
                                 const float* coef, void* snap, void* out, float* fr, float* fi,
                                 int B, int T, int h, int hp, void* ws, hipStream_t stream);
// the same from the stacked projection [B*T, stride] (fused: silu(v), normalised q, k, v; coef
// from the fused coefficient kernel, with the k and v norms in its floats 6 and 7)
hipError_t launch_cham_mfma_scan_fused(const void* proj, int64_t stride, int io_dtype,
                                       const float* coef, void* snap, void* out, float* fr,
                                       float* fi, int B, int T, int h, int hp, void* ws,
                                       hipStream_t stream);
hipError_t launch_cham_mfma_cols(const void* k, const void* v, int io_dtype, const float* coef,
                                 const float* i0r, const float* i0i, const float* i1r,
                                 const float* i1i, float* snap, float* fr, float* fi, int B,
                                 int T, int h, int hp, int nstates, int snap_on, int c2, void* ws,
                                 hipStream_t stream);

// sssd_bwd.hip: backward of the scan (dq, dk, dv, ddelta, dPsi_0 from dOut, dPsi_T), any
// head_dim up to 256 (the per-token reverse pass; padded to a multiple of 32 inside).
bool sssd_bwd_supported(int64_t D);
size_t sssd_bwd_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t D);
hipError_t launch_sssd_bwd(const void* q, const void* k, const void* v, const void* delta,
                           int io_dtype, int delta_dtype, const float* psi_T, const void* dout,
                           int dout_dtype, const float* dpsi_T, void* dq, void* dk, void* dv,
                           void* ddelta, float* dpsi0, int B, int T, int H, int D, void* ws,
                           hipStream_t stream);

// sssd_bwd_chunk.hip: the same backward in chunks of 16 tokens on the fp32 MFMA
// (used for T >= kBwdChunkMinT at head_dim 64 and 128; other head dims take sssd_bwd.hip).
constexpr int64_t kBwdChunkMinT = 32;
inline bool use_bwd_chunk(int64_t T, int64_t D) {
  return T >= kBwdChunkMinT && (D == 64 || D == 128);
}
size_t sssd_bwd_chunk_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t D);
hipError_t launch_sssd_bwd_chunk(const void* q, const void* k, const void* v, const void* delta,
                                 int io_dtype, int delta_dtype, const float* psi_T,
                                 const void* dout, int dout_dtype, const float* dpsi_T, void* dq,
                                 void* dk, void* dv, void* ddelta, float* dpsi0, int B, int T,
                                 int H, int D, void* ws, hipStream_t stream);

// cham_ns.hip: Newton-Schulz unitary retraction.
size_t ns_workspace_bytes(int64_t batch, int64_t n);
// cham_ns16.hip: the same retraction on the 16-bit matrix cores (f16 hi + lo operands) for
// n a multiple of 128; launch_ns_retraction takes it whenever ns16_usable(n).
bool ns16_usable(int64_t n);
size_t ns16_workspace_bytes(int64_t batch, int64_t n);
hipError_t launch_ns16_retraction(const float* h_real, const float* h_imag, float* out_real,
                                  float* out_imag, int batch, int n, int steps, void* workspace,
                                  hipStream_t stream);
hipError_t launch_ns_retraction(const float* h_real, const float* h_imag, float* out_real,
                                float* out_imag, int batch, int n, int steps, void* workspace,
                                hipStream_t stream);

}  // namespace vmi
