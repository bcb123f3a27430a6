/*
 * verace_sssd.h -- C ABI of the MI355X (gfx950) SSSD Cayley-scan library
 * (libverace_sssd.so, built from verace-v1_amd/csrc/).
 *
 * Every entry point takes plain device pointers, sizes and a HIP stream
 * (passed as void*, it is a hipStream_t; NULL = the null stream).  Nothing
 * here allocates device memory: scratch space is passed in by the caller and
 * sized with the matching *_workspace_bytes query and 16-byte aligned (as every
 * device allocation is; some kernels read it 16 bytes at a time).  Kernels are enqueued on
 * the given stream; no entry point synchronises the host.  The one piece of
 * mutable global state is the fixed scratch array of vmi_sssd_scan_fwd_noalloc
 * (one per GPU): calls of that entry point that overlap on one GPU race.  Every
 * other entry point is safe from several host threads as long as the calls
 * use disjoint output and workspace buffers.
 *
 * Math implemented (reference: verace_v1/modules/sssd_attention.py:144-182):
 *   X_t   = (delta_t / 2) * (k_t v_t^T - v_t k_t^T)
 *   R_t   = (I + X_t)^-1 (I - X_t)           (solve(right, left) order, :163-166)
 *   Psi_t = R_t Psi_{t-1},  Psi_0 = initial state (identity if NULL)
 *   o_t   = Psi_t q_t
 * R_t is applied in closed form (no solve): R = I + c(-X + X^2), c = 2/(1+m^2),
 * m^2 = (delta/2)^2 (|k|^2 |v|^2 - (k.v)^2), which is exact for any k, v and
 * equals I exactly at delta = 0.
 *
 * Layouts (all contiguous, row-major, identical to the reference launcher's
 * contract, verace_v1/serving/triton_kernels.py:612-627):
 *   q, k, v, out : [B, T, H, D]   dtype io_dtype (out takes q's dtype)
 *   delta        : [B, T, H]      dtype delta_dtype
 *   psi_in       : [B, H, D, D]   float32, NULL means identity
 *   psi_out      : [B, H, D, D]   float32
 */
#ifndef VERACE_SSSD_H
#define VERACE_SSSD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element type codes for io_dtype / delta_dtype. */
enum vmi_dtype {
  VMI_F32 = 0,
  VMI_BF16 = 1,
  VMI_F16 = 2
};

/* Status codes returned by every entry point (0 = success). */
enum vmi_status {
  VMI_OK = 0,
  VMI_ERR_INVALID_ARG = 1,     /* null pointer where one is required, bad size */
  VMI_ERR_UNSUPPORTED = 2,     /* head_dim / dtype combination not built */
  VMI_ERR_WORKSPACE = 3,       /* workspace missing or too small */
  VMI_ERR_ALIAS = 4,           /* forbidden aliasing between buffers */
  VMI_ERR_HIP = 5,             /* a HIP runtime call failed (see vmi_last_hip_error) */
  VMI_ERR_FULL = 6             /* a state cache layer has no free slot left */
};

/* Library version (major*10000 + minor*100 + patch). */
int vmi_version(void);

/* Human-readable text for a vmi_status value. */
const char* vmi_status_string(int status);

/* hipError_t of the last failing HIP call made by this thread inside the
 * library (0 if none). */
int vmi_last_hip_error(void);

/* Bytes of device workspace vmi_sssd_scan_fwd needs for this problem.
 * Replaces nothing in the reference (the Triton launcher allocates its
 * outputs itself); the caller allocates `*bytes` from its own allocator. */
int vmi_sssd_scan_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t D,
                                  int io_dtype, size_t* bytes);

/* Prefill scan over T tokens.
 * Replaces launch_sssd_triton_scan + sssd_cayley_scan_kernel
 * (verace_v1/serving/triton_kernels.py:603-636 and :41-144), whose results
 * must equal the eager path sssd_attention.py:144-181.
 *   psi_in   may be NULL (identity, triton_kernels.py:621-622); it is never
 *            written.  psi_out must not alias psi_in (the reference returns a
 *            fresh state, triton_kernels.py:627).
 *   out      may be NULL if only the final state is wanted.
 * Supported: io_dtype in {F32, BF16, F16}; delta_dtype in {F32, BF16, F16};
 * 1 <= D <= 256.  T = 0 copies psi_in (or identity) to psi_out.
 * Arithmetic: F32 I/O, D != 128 and T < 32 run in fp32 token by token.  BF16 / F16 I/O with
 * D = 128 and T >= 32 run the chunk-parallel scan, whose matrix-core operands (the state, W
 * and Z, once per 16-token chunk) are f16 with fp32 accumulation.  That holds the 2e-2
 * relative / 1e-4 norm-drift bars while every token's rotation
 * m = (delta/2) |k| |v| sin(angle(k, v)) stays <= 0.25 (measured to T = 65536); unit k, v
 * with delta <= 0.1 (the SSSD module's inputs) give m <= 0.05.  A
 * sequence with any token above m = 0.25 is detected on the device and recomputed in fp32
 * token by token within the same call (its result then equals the F32 path's on the same
 * values): no input leaves the bars, at the fp32 path's cost for such sequences. */
int vmi_sssd_scan_fwd(const void* q, const void* k, const void* v,
                      const void* delta, int io_dtype, int delta_dtype,
                      const float* psi_in, void* out, float* psi_out,
                      int64_t B, int64_t T, int64_t H, int64_t D,
                      void* workspace, size_t workspace_bytes, void* stream);

/* The same prefill scan with no workspace argument and no allocation: the scan's workspace
 * is a fixed 40 MiB device array of the library, one per GPU, held from the library's first
 * use on that GPU until the process ends (enough for every plan of the OP, FULL, LONG and DEC
 * shapes; plans needing more return VMI_ERR_WORKSPACE before anything is launched -- use
 * vmi_sssd_scan_fwd for them).  No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Calls on one GPU share its array, so calls that overlap on one
 * GPU (several streams or host threads) race: order them.  Arguments and results as
 * vmi_sssd_scan_fwd. */
int vmi_sssd_scan_fwd_noalloc(const void* q, const void* k, const void* v,
                              const void* delta, int io_dtype, int delta_dtype,
                              const float* psi_in, void* out, float* psi_out,
                              int64_t B, int64_t T, int64_t H, int64_t D, void* stream);

/* Prefill scan on the raw projections, with the steps either side of the scan fused:
 * replaces sssd_attention.py:114-126 (F.normalize of q, k, v; delta = 0.1 *
 * sigmoid(w_delta x) * active_mask) and :177 (head_rmsnorm) around the scan.
 *   proj   : [B, T, proj_stride] io_dtype, the output of one GEMM x [W_q; W_k; W_v;
 *            W_delta]^T (q, k, v of head h at columns h*D, H*D + h*D, 2*H*D + h*D,
 *            the delta logit at 3*H*D + h; proj_stride >= 3*H*D + H, a multiple of 8,
 *            proj 16-byte aligned), read once;
 *   mask   : [B, T] uint8 (nonzero = active) or NULL (all active);
 *   rms_weight : [D] float32 or NULL; out = rms_weight * o * rsqrt(mean_d(o^2) +
 *            rms_eps) (nn.RMSNorm; its default eps is torch.finfo(dtype).eps), or o when
 *            NULL;
 *   out    : [B, T, H, D] io_dtype; psi_in / psi_out as for vmi_sssd_scan_fwd.
 * q, k, v are scaled by 1 / max(|.|, 1e-12) in fp32 inside the kernel, and delta <= 0.1, so
 * every token rotates by m <= 0.05, inside the chunk scan's accuracy envelope (see
 * vmi_sssd_scan_fwd) without a check.  Supported:
 * io_dtype BF16 or F16, D = 128, T >= 32 (otherwise VMI_ERR_UNSUPPORTED: run the
 * unfused ops and vmi_sssd_scan_fwd).  Workspace from
 * vmi_sssd_scan_fused_workspace_bytes. */
int vmi_sssd_scan_fused_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t D,
                                        int io_dtype, size_t* bytes);
int vmi_sssd_scan_fused(const void* proj, int64_t proj_stride, int io_dtype, const uint8_t* mask,
                        const float* rms_weight, float rms_eps, const float* psi_in,
                        void* out, float* psi_out, int64_t B, int64_t T, int64_t H,
                        int64_t D, void* workspace, size_t workspace_bytes, void* stream);

/* One decode step (T = 1) with the state updated in place:
 *   psi <- R psi ;  out = psi q.
 * Replaces the reference's incremental forward at seq_len 1
 * (sssd_attention.py:103-182 called from acd_engine.py:116-121 and
 * hyper_generate.py:59-63), which returns a fresh state; the in-place form
 * is opt-in for callers that own the state (the reference never mutates
 * initial_state, so tree-search branches must pass a copy).
 * q, k, v, out: [B, 1, H, D]; delta: [B, 1, H]; psi: [B, H, D, D] float32. */
int vmi_sssd_step_inplace(const void* q, const void* k, const void* v,
                          const void* delta, int io_dtype, int delta_dtype,
                          float* psi, void* out,
                          int64_t B, int64_t H, int64_t D, void* stream);

/* vmi_sssd_step_inplace fused with the projections either side of it (as vmi_sssd_scan_fused
 * for the prefill): the decode step of the reference's forward at seq_len 1 from the
 * projections on (sssd_attention.py:114-126 before the scan, :177 after it, called from
 * acd_engine.py:116-121 and hyper_generate.py:59-63).
 *   proj : [B, proj_stride] io_dtype, row b = x_b [W_q; W_k; W_v; W_delta]^T raw (q of head h
 *          at h D, k at H D + h D, v at 2 H D + h D, the delta logit at 3 H D + h);
 *          proj_stride >= 3 H D + H;
 *   q, k, v are L2-normalised in the kernel (F.normalize, eps 1e-12) and
 *   delta = 0.1 sigmoid(logit) * mask[b] (mask: [B] uint8, null = every item active);
 *   psi : [B, H, D, D] float32, updated in place;
 *   out : [B, 1, H, D] io_dtype = head_rmsnorm(o) = o rsqrt(mean(o^2) + rms_eps) rms_weight
 *         when rms_weight ([D] float32) is given, else o.
 * D = 128 (otherwise VMI_ERR_UNSUPPORTED: run the unfused ops and vmi_sssd_step_inplace). */
int vmi_sssd_step_fused(const void* proj, int64_t proj_stride, int io_dtype, const uint8_t* mask,
                        const float* rms_weight, float rms_eps, float* psi, void* out,
                        int64_t B, int64_t H, int64_t D, void* stream);

/* One decode step over the slots of a state cache (copy-on-write decode):
 *   item b reads state slot in_slot[b] (or the identity when in_slot[b] == -1),
 *   writes R * state to slot out_slot[b], and out[b] = (R * state) q[b].
 * Replaces the per-item incremental forward of acd_engine.py:102-126 and the
 * branch fan-out of hyper_generate.py:97-121, which call sssd_attention.py:103-182
 * at seq_len 1 with a state taken from layer_states[l][i] and store the fresh
 * state back: here a branch reads its parent's slot and writes its own, so a
 * fork costs no copy.
 *   states: [num_slots, H, D, D] float32, one layer's pool (read and written);
 *   in_slot, out_slot: [B] int32 device arrays;
 *   q, k, v, out: [B, 1, H, D]; delta: [B, 1, H].
 * Out slots must be distinct, and an out slot may be read by no item other than
 * its own (in_slot[b] == out_slot[b] updates in place).  Indexes outside
 * [0, num_slots) read as the identity (in) or drop the state write (out). */
int vmi_sssd_step_slots(const void* q, const void* k, const void* v,
                        const void* delta, int io_dtype, int delta_dtype,
                        float* states, int64_t num_slots,
                        const int32_t* in_slot, const int32_t* out_slot, void* out,
                        int64_t B, int64_t H, int64_t D, void* stream);

/* ---- Decode state cache (copy-on-write branches) ---------------------------
 * Replaces the reference's per-item decode state threading: layer_states[l][i] =
 * (sssd_state, ...) lists stepped one item at a time (acd_engine.py:85-126) and
 * copied per tree-search branch (hyper_generate.py:97-121).  The caller allocates
 * the device pool [num_layers, num_slots, H, D, D] float32; the cache object (host
 * memory only) maps sequence handles to slots with reference counts:
 *   new      handles starting from the identity (no slot until first written);
 *   fork     handles sharing every layer's slot with a parent (no copy);
 *   step     one batched decode step of a layer: one launch (several above 256
 *            items); a sole holder is updated in place, a handle on a shared slot
 *            (or none) reads it and writes a fresh slot;
 *   plan     the same slot decisions without a launch (for whole-state writes,
 *            e.g. prefill results, which the caller copies into dst slots);
 *   slots    current slot of each handle (-1 = identity), for reads;
 *   release  drops handles; slots nobody holds return to their layer's free list.
 * Handle ids of released handles are reused.  Not thread-safe: one host thread per
 * cache; the steps of one cache must be ordered on one stream.  A failed step
 * (status != VMI_OK after planning) leaves the states of its handles undefined. */
typedef struct vmi_state_cache vmi_state_cache;
int vmi_state_cache_create(int64_t num_layers, int64_t num_slots, int64_t H, int64_t D,
                           float* pool, vmi_state_cache** cache);
int vmi_state_cache_destroy(vmi_state_cache* cache);
int vmi_state_cache_new(vmi_state_cache* cache, int64_t n, int64_t* handles);
int vmi_state_cache_fork(vmi_state_cache* cache, int64_t parent, int64_t n, int64_t* handles);
int vmi_state_cache_release(vmi_state_cache* cache, const int64_t* handles, int64_t n);
int vmi_state_cache_plan(vmi_state_cache* cache, int64_t layer, const int64_t* handles,
                         int64_t n, int32_t* src_slots, int32_t* dst_slots);
int vmi_state_cache_slots(vmi_state_cache* cache, int64_t layer, const int64_t* handles,
                          int64_t n, int32_t* slots);
int vmi_state_cache_refs(vmi_state_cache* cache, int64_t layer, int32_t* refs,
                         int64_t* free_slots);
/* q, k, v, out: [n, 1, H, D] io_dtype; delta: [n, 1, H]; item b continues handles[b]. */
int vmi_state_cache_step(vmi_state_cache* cache, int64_t layer, const int64_t* handles,
                         int64_t n, const void* q, const void* k, const void* v,
                         const void* delta, int io_dtype, int delta_dtype, void* out,
                         void* stream);

/* The CHAM half of the cached state: holo_pool [num_layers, num_slots, 2, h, h] float32 (the
 * caller's; slot s of layer l holds the raw hologram's real plane, then its imaginary plane)
 * becomes part of the cache, so a handle's (sssd_state, cham_hologram) tuple of
 * acd_engine.py:88-92 lives in one slot of each pool.  vmi_state_cache_cham_step runs the
 * in-place CHAM decode step (as vmi_cham_step_inplace) over the hologram slots with the slot
 * decisions of the layer's last vmi_state_cache_step: call it once, with the same handles in
 * the same order, after that layer's SSSD step (the CHAM sub-layer's inputs come from the
 * SSSD sub-layer's output, backbone.py:83-93).  Other handle lists, a second call for the
 * same step, and a call after a fork, a release or another plan of the layer in between
 * return VMI_ERR_INVALID_ARG.
 * A handle with no slot yet starts from the identity.  Every cached hologram is taken to have
 * started from the identity (unitary, so the readout NS_3(H) = H; write NS_3-retracted pairs
 * only if that holds).  q, k, v, out: [n, 1, h] io_dtype; gamma: [n] gamma_dtype; h % 4 == 0,
 * h <= 1024.  Workspace from vmi_state_cache_cham_workspace_bytes. */
int vmi_state_cache_attach_hologram(vmi_state_cache* cache, int64_t h, float* holo_pool);
int vmi_state_cache_cham_workspace_bytes(int64_t n, int64_t h, size_t* bytes);
int vmi_state_cache_cham_step(vmi_state_cache* cache, int64_t layer, const int64_t* handles,
                              int64_t n, const void* q, const void* k, const void* v,
                              const void* gamma, int io_dtype, int gamma_dtype, void* out,
                              void* workspace, size_t workspace_bytes, void* stream);

/* Backward of the scan (training).  Replaces the eager autograd through
 * sssd_attention.py:144-175 that the reference's training loop differentiates
 * (pretrain.py:164-195): given the forward's inputs, its final state psi_T
 * (vmi_sssd_scan_fwd's psi_out) and the gradients d_out = dL/dout [B,T,H,D]
 * (d_out_dtype) and d_psi_T = dL/dpsi_T [B,H,D,D] fp32 (NULL: zero), writes
 *   dq, dk, dv : [B,T,H,D] io_dtype;  d_delta : [B,T,H] delta_dtype;
 *   d_psi0     : [B,H,D,D] fp32 = dL/d initial_state (NULL: not needed).
 * The states are rebuilt in reverse from psi_T (every factor is exactly
 * orthogonal), so nothing but psi_T is kept from the forward.  1 <= D <= 256
 * (otherwise VMI_ERR_UNSUPPORTED): D = 64 and 128 with T >= 32 run the chunked
 * matrix-core backward, every other case the per-token reverse pass; workspace from
 * vmi_sssd_scan_bwd_workspace_bytes. */
int vmi_sssd_scan_bwd_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t D, size_t* bytes);
int vmi_sssd_scan_bwd(const void* q, const void* k, const void* v, const void* delta,
                      int io_dtype, int delta_dtype, const float* psi_T, const void* d_out,
                      int d_out_dtype, const float* d_psi_T, void* dq, void* dk, void* dv,
                      void* d_delta, float* d_psi0, int64_t B, int64_t T, int64_t H, int64_t D,
                      void* workspace, size_t workspace_bytes, void* stream);

/* CHAM holographic scan, holographic_dim h <= 1024, or h a multiple of 4 up to 4096:
 * replaces launch_cham_triton_update with its single-program kernel for h <= 128
 * (cham_holographic_scan_kernel, triton_kernels.py:151-306, :639-685) and its tiled route for
 * larger h (launch_cham_triton_tiled, :477-597), and the eager path of
 * ContinuousHolographicMemory.forward (cham_memory.py:167-238).
 *   H_t = U_t H_{t-1},  U_t = (I - i G_t/2)^-1 (I + i G_t/2),
 *   G_t = gamma_t (k_t v_t^T + v_t k_t^T)       (exact Cayley, closed rank-2 form)
 *   out_t = Re(NS_3(H_t) q_t)                   (3 Newton-Schulz steps, readout only)
 * H_0 = (h0_real, h0_imag) or the identity (both NULL); the raw, never retracted H_T
 * is written to (h_real_out, h_imag_out).
 *   q, k, v, out : [B, T, h] io_dtype;  gamma : [B, T] gamma_dtype;
 *   h0_*, h_*_out : [B, h, h] float32 (outputs must not overlap the inputs).
 * Above h = 1024 the scan runs one in-place step per token (the kernels of
 * vmi_cham_step_inplace on H and, when H_0 is given, on R = NS_3(H_0) held in the workspace):
 * O(T h^2) memory traffic, B <= 65535 and B h^2 <= 2^31 - 1; h > 4096 or h % 4 != 0 there:
 * VMI_ERR_UNSUPPORTED.  Workspace from vmi_cham_scan_workspace_bytes (for 128 < h <= 1024 it
 * holds a state snapshot per 64 tokens: about 2 B T h^2 / 64 floats; above 1024 the readout
 * state, the retraction's scratch and the step's partials).
 * Precondition of the 16-bit route for 128 < h <= 1024 (io_dtype BF16 or F16): every element
 * of k and v is below 65504 in magnitude, because the matrix-core carry converts them to f16
 * (exactly, inside that range).  A token with a larger element (bf16 values from 65536 up) is
 * taken as the identity, as a token with a non-finite element is.  The module's L2-normalised
 * k, v are at most 1; other callers with larger elements pass io_dtype F32, whose route takes
 * any finite value. */
int vmi_cham_scan_workspace_bytes(int64_t B, int64_t T, int64_t h, size_t* bytes);
int vmi_cham_scan_fwd(const void* q, const void* k, const void* v, const void* gamma,
                      int io_dtype, int gamma_dtype, const float* h0_real,
                      const float* h0_imag, void* out, float* h_real_out,
                      float* h_imag_out, int64_t B, int64_t T, int64_t h,
                      void* workspace, size_t workspace_bytes, void* stream);

/* One CHAM decode step (T = 1) with the holographic state updated in place:
 *   H <- U H  (U the exact Cayley factor of the token, as in vmi_cham_scan_fwd),
 *   R <- U R  when a readout state R is given,
 *   out = Re(NS_3(H') q) = Re(R' q)   (R = NS_3(H) is carried by the caller; NULL means H
 *                                      is unitary, e.g. it started from the identity, and
 *                                      then NS_3(H') = H').
 * Replaces the reference's incremental CHAM forward at seq_len 1 (cham_memory.py:117-238
 * with initial_hologram, called per token from acd_engine.py:116-121 and
 * hyper_generate.py:59-63), which returns a fresh raw state and retracts it for the readout;
 * the in-place form is opt-in for callers that own the state (as vmi_sssd_step_inplace).
 *   q, k, v, out : [B, 1, h] io_dtype;  gamma : [B] gamma_dtype;
 *   h_real, h_imag (and r_real, r_imag) : [B, h, h] float32, read and written, distinct.
 * h % 4 == 0 and h <= 4096 (otherwise VMI_ERR_UNSUPPORTED).  Workspace from
 * vmi_cham_step_workspace_bytes (per-block readout partials: B (h/16) h floats up to h = 1024,
 * B (h/4) h above). */
int vmi_cham_step_workspace_bytes(int64_t B, int64_t h, size_t* bytes);
int vmi_cham_step_inplace(const void* q, const void* k, const void* v, const void* gamma,
                          int io_dtype, int gamma_dtype, float* h_real, float* h_imag,
                          float* r_real, float* r_imag, void* out, int64_t B, int64_t h,
                          void* workspace, size_t workspace_bytes, void* stream);

/* vmi_cham_scan_fwd from the identity fused with the projections before it (the reference's
 * CHAM forward with no initial hologram, cham_memory.py:128-155 then :167-238, as the model's
 * prefill calls it):
 *   proj : [B, T, proj_stride] io_dtype (BF16 or F16), row (b, t) = x_{b,t} [W_q; W_k; W_v;
 *          W_gamma]^T raw (q at 0, k at h, v at 2h, the gamma logit at 3h); proj_stride >= 3h + 1
 *          and a multiple of 8; proj and out 16-byte aligned;
 *   in the kernels v = silu(v), q, k, v are L2-normalised (F.normalize, eps 1e-12) and
 *   gamma = 0.1 sigmoid(logit) * mask[b, t] (mask: [B, T] uint8, null = every token active);
 *   out : [B, T, h] io_dtype = Re(NS_3(H_t) q_t) (= Re(H_t q_t): H_t is unitary);
 *   h_real_out, h_imag_out : [B, h, h] float32, the raw final state.
 * 128 < h <= 1024 with h % 8 == 0 (otherwise VMI_ERR_UNSUPPORTED: run the unfused ops and
 * vmi_cham_scan_fwd).  Workspace from vmi_cham_scan_workspace_bytes. */
int vmi_cham_scan_fused(const void* proj, int64_t proj_stride, int io_dtype, const uint8_t* mask,
                        void* out, float* h_real_out, float* h_imag_out, int64_t B, int64_t T,
                        int64_t h, void* workspace, size_t workspace_bytes, void* stream);

/* vmi_cham_step_inplace fused with the projections before it: the CHAM decode step of the
 * reference's forward at seq_len 1 from the projections on (cham_memory.py:128-155 before the
 * scan, called per token from acd_engine.py:116-121 and hyper_generate.py:59-63).
 *   proj : [B, proj_stride] io_dtype, row b = x_b [W_q; W_k; W_v; W_gamma]^T raw (q at 0, k at
 *          h, v at 2h, the gamma logit at 3h); proj_stride >= 3h + 1;
 *   in the kernel v = silu(v), q, k, v are L2-normalised (F.normalize, eps 1e-12) and
 *   gamma = 0.1 sigmoid(logit) * mask[b] (mask: [B] uint8, null = every item active);
 *   h_real, h_imag (and r_real, r_imag): as vmi_cham_step_inplace, updated in place;
 *   out : [B, 1, h] io_dtype = Re(NS_3(H') q).
 * h = 1024 (otherwise VMI_ERR_UNSUPPORTED: run the unfused ops and vmi_cham_step_inplace).
 * Workspace from vmi_cham_step_workspace_bytes. */
int vmi_cham_step_fused(const void* proj, int64_t proj_stride, int io_dtype, const uint8_t* mask,
                        float* h_real, float* h_imag, float* r_real, float* r_imag, void* out,
                        int64_t B, int64_t h, void* workspace, size_t workspace_bytes,
                        void* stream);

/* Newton-Schulz unitary retraction of a batch of complex matrices
 * H = Hr + i Hi, `steps` iterations of H <- 0.5 H (3I - H^H H), both halves
 * of every iteration computed from the pre-update H.
 * Replaces newton_schulz_unitary_retraction / parallel_newton_schulz_retraction
 * (verace_v1/modules/cham_memory.py:21-51 and :296-315) and the in-kernel
 * NS loop of cham_holographic_scan_kernel (triton_kernels.py:280-292).
 *   h_real, h_imag : [batch, n, n] float32, read;
 *   out_real, out_imag : [batch, n, n] float32, written (may alias the inputs).
 * Needs vmi_cham_ns_workspace_bytes(batch, n) bytes of workspace. */
int vmi_cham_ns_workspace_bytes(int64_t batch, int64_t n, size_t* bytes);
int vmi_cham_ns_retraction(const float* h_real, const float* h_imag,
                           float* out_real, float* out_imag,
                           int64_t batch, int64_t n, int steps,
                           void* workspace, size_t workspace_bytes,
                           void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VERACE_SSSD_H */
