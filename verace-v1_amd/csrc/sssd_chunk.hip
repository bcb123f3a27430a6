// Chunk-parallel SSSD prefill scan on f16 MFMA (bf16 or fp16 I/O), head_dim 128.
//
// Math (reference recurrence sssd_attention.py:160-175, regrouped per chunk).
// For a chunk of C = 16 tokens starting from state S:
//   U = [k_0 v_0 k_1 v_1 ...]  (D x 32, rank row rho = 2t + {0: k, 1: v})
//   R_t = I + U_t M_t U_t^T with the closed-form 2x2 Cayley block M_t
//   G  = U^T U                                   (Gram, 32 x 32)
//   T~ = (I - L)^-1 blockdiag(M),  L_{t,i} = M_t G_{t,i} for i < t
//   W  = U^T S,  Z = T~ W                        (32 x D)
//   end state      S' = S + U Z
//   readout        O  = S Q + U (mask o (Z Q))   (D x 16), mask: token(rho) <= t
// T~ is computed in 8x8 blocks (4 tokens): diagonal blocks by forward
// substitution, off-diagonal blocks by T~_gh = T~_gg sum_{m=h}^{g-1} G_gm T~_mh.
//
// Precision: every MFMA accumulates in fp32.  U and q enter as f16 (exact for the
// L2-normalised inputs of this op); G, the Cayley blocks and T~ are fp32, and T~
// enters as an f16 hi + lo pair, so each chunk factor I + U T~ U^T is orthogonal to
// ~2^-22.  The state S (scaled by a power of two, see below), W and Z are rounded to
// f16 once per chunk (11-bit significand): the rounding errors are unbiased, so the
// state norm drifts as a random walk (~1e-6 over 65536 tokens, against 1e-4 allowed)
// and the state stays within ~3e-4 of the exact recurrence at that length.
//
// Workgroup = 12 waves for one (batch*head, segment):
//   waves 0-3 (consumers) each own a 32-column slab of the fp32 state, held in
//     MFMA accumulators for the whole segment; columns evolve independently, so
//     W, Z and the update need no cross-wave traffic.  With the readout every wave
//     also stashes its slab of S and Z (f16, transposed) in LDS.
//   waves 4-5 (readout, pass C only) compute, from the stashes of chunk c-1, 64
//     complete output rows each (transposing LDS loads, no reduction) while the
//     consumers work on chunk c.
//   the remaining 6 (pass C) or 8 (pass A) producer waves take chunks round-robin
//     (producer p owns chunks n = p mod NPW) and run each through NPW phases, one per
//     iteration, ahead of the consumers: loads of k/v/q/delta; Gram matrix on MFMA and
//     Cayley blocks; diagonal and off-diagonal 8x8 blocks of T~; the write of U, q
//     and T~ (f16 hi + lo) to LDS.  The producers are in different phases at any
//     time, so one chunk completes per iteration and no wave waits on another inside
//     an iteration; one LDS barrier per chunk hands the buffers over.  The readout
//     stashes are double-buffered by chunk parity, so the stash writes of chunk c need
//     no barrier against the readout of chunk c-1.
//
// Long sequences are split into segments processed by independent workgroups:
//   pass A (READOUT=false): the transforms of segments 0 .. S-2 from the identity,
//          spread over S workgroups per sequence (so it fills as many CUs as pass C):
//          each segment is covered by two parts, each part's transform is stored,
//   pass B (sssd_carry_kernel): start_s = (part 2 of s-1)(part 1 of s-1) start_{s-1},
//          column blocks in parallel workgroups, bf16x3 MFMA (fp32-faithful),
//   pass C (READOUT=true): every segment from its start state, with outputs.
//
// Fused mode (FUSED=true, vmi_sssd_scan_fused): the inputs are the raw projections
// [B, T, stride] of one GEMM x [W_q; W_k; W_v; W_delta]^T.  The producers normalise the
// k, v rows (norms from a Gram matrix of the raw rows, then one fp32 scaling and one f16
// rounding) and the q rows (sum of squares over a DPP row), and form delta = 0.1
// sigmoid(logit) * mask; the readout waves apply head RMSNorm, whose per-token mean
// square spans both readout waves: each keeps its rows of chunk c in registers for one
// iteration and stores them once both partial sums are in LDS.  The k/v normalisation
// takes the phase that otherwise converts k, v to f16.
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "vmi_common.h"
#include "vmi_dispatch.h"
#include "vmi_mfma.h"

namespace vmi {
namespace chunk {

constexpr int D = 128;
constexpr int C = 16;           // tokens per chunk
constexpr int R = 2 * C;        // rank rows per chunk
constexpr int NCW = 4;          // consumer waves
// 3 waves per SIMD (at most 168 VGPRs each).  Pass C: 4 consumers (the state), 2 readout
// waves and 6 producers; two readout waves of 64 rows each compute Z Q half as often as
// four of 32 rows and measured fastest.  Pass A (no readout): 4 consumers and 8
// producers, whose latency-bound phases are then split over a deeper pipeline.
template <bool READOUT> struct Cfg {
  static constexpr int NPW = READOUT ? 6 : 8;
  static constexpr int NRW = READOUT ? 2 : 0;  // readout waves (64 output rows each)
  static constexpr int NT = (NCW + NRW + NPW) * 64;
  static constexpr int NSCR = READOUT ? 3 : 8;  // producer scratch slots (chunk n % 3 / producer)
};
// LDS bank model (measured on gfx950): 64 banks of 4 B; a 64-bit access (also the
// transposing ds_read_b64_tr_b16 and each half of read2/write2_b64) is served in
// units of 32 lanes, a 128-bit access in units of 16 lanes, and a unit is conflict-free
// when its dwords fall in distinct banks.  Every layout below is conflict-free for all
// the accesses made to it (checked exhaustively against this model) while keeping each
// per-instruction offset additive, so addresses are one VGPR plus immediates.
//
// One chunk of inputs, token-major.  Rank row rho of U (= k_t for rho = 2t, v_t for
// rho = 2t + 1) lives in slot rho_slot(rho) (a fixed bit permutation of rho) with a
// pitch of 132 elements (264 B); the q rows follow with a pitch of 136 elements.
// Accesses: the producer's 16-B row writes, the W operand (32 rows rho, one column
// block), the transposing reads of U for the update (rows rho0 + 0..3, 32 columns)
// and for the readout (rows 4g + 0..3, 16 columns), and the readout's q reads.
constexpr int U_LD = D + 4;               // elements per U row slot
constexpr int Q_LD = D + 8;               // elements per q row
constexpr int Q_OFF = R * U_LD;           // q rows after the 32 U slots
constexpr int CHUNK_ELEMS = Q_OFF + C * Q_LD;
__host__ __device__ constexpr int rho_slot(int rho) {  // bits 0,1,2,3,4 -> 3,4,2,1,0
  return ((rho & 1) << 3) | ((rho & 2) << 3) | (rho & 4) | ((rho & 8) >> 2) | ((rho & 16) >> 4);
}
constexpr int T_LD = R + 4;     // floats per Gram row
constexpr int TT_LD = R + 4;    // elements per T~ hi/lo row (72 B: 32 rows in distinct banks)

// Readout stashes (shared by the consumer waves):
//   pst: chunk-start state, transposed: element (j, d) = Psi_s[d][j], row slot j_slot(j)
//   zst: Z transposed:                   element (j, rho) = Z[rho][j], row slot j_slot(j)
// with j_slot a bit permutation of the low 5 bits of j (rows j = 32w + l32 are written
// 8 bytes per lane; rows 32ks + 8pg + 4hh + 0..3 are read back with transposing loads).
constexpr int PST_LD = D + 4;   // 264 B
constexpr int ZST_LD = R + 4;   // 72 B
__host__ __device__ constexpr int j_slot(int j) {  // bits 0,1,2,3,4 -> 2,3,0,1,4 (j < 32)
  return ((j & 1) << 2) | ((j & 2) << 2) | ((j & 4) >> 2) | ((j & 8) >> 2) | (j & 16);
}

// Scratch of a producer wave from the Gram matrix to the off-diagonal blocks of one chunk.
struct PScratch {
  float gram[R * T_LD];         // Gram matrix G = U^T U (symmetric)
  float4 mcoef[C];              // (m00, m01, m10, m11) per token
  float drow[4][64];            // diagonal 8x8 blocks of T~, row-major [a*8 + c]
  float dcol[4][64];            // the same blocks, column-major [b*8 + c]
  float ocol[64];               // T~_10, column-major
  float orow[64];               // T~_32, row-major
  float sblk[2][64];            // S = G_10 T~_00 and G_32 T~_22, column-major
};

template <typename E, bool READOUT>
struct Smem {
  E tok[3][CHUNK_ELEMS];        // U rows and q rows of a chunk (3 chunks in flight)
  E tth[2][R * TT_LD];          // T~ = hi + lo (two 16-bit parts), row-major
  E ttpad[8];                   // puts ttl 4 banks after tth (conflict-light pair writes)
  E ttl[2][R * TT_LD];
  E pst[2][READOUT ? D * PST_LD : 1];  // readout stash (chunk parity): chunk-start state, transposed
  E zst[2][READOUT ? D * ZST_LD : 1];  // readout stash (chunk parity): Z, transposed
  PScratch pscr[Cfg<READOUT>::NSCR];   // producer scratch (chunk parity / producer wave)
  float smax[NCW];              // per consumer wave: max |start state| of its slab
  float rsum[READOUT ? 2 * Cfg<READOUT>::NRW * C : 1];  // fused RMSNorm: [chunk parity][readout wave][token]
};

struct Args {
  const void* q;
  const void* k;
  const void* v;
  const void* delta;
  int delta_dtype;
  const float* psi0;    // start of segment 0 ([BH][D][D]); null = identity
  const float* starts;  // start of segment s >= 1 at starts[(s-1)*BH + bh]; null = identity
  void* out;            // [B][T][H][D] (READOUT only)
  float* ends;          // see end_mode
  int end_mode;         // 0: pass A factors (see below); 1: ends[bh] for the last segment
  int T, H, BH;
  int seg_chunks;       // chunks per segment
  int nseg;             // segments per sequence
  // Pass A with npieces > 0: workgroup (bh, a) covers chunks [c_a, c_{a+1}) of the
  // first (nseg-1) * seg_chunks, c_a = a * that / npieces, and writes the transform of
  // every part between segment boundaries: factor 2s is the part of segment s before
  // the piece boundary inside it, factor 2s+1 the part after it (npieces = nseg puts
  // exactly one piece boundary inside every segment).  Factor f of sequence bh is at
  // ends[f * BH + bh].  With npieces = 0 the pieces are the segments, factor s = P_s.
  int npieces;
  // input layout: q/k/v element (t, d) of head h at q/k/v + (b*T + t)*in_stride + h*D + d,
  // delta of (t, h) at delta + (b*T + t)*dl_stride + h (the reference layout has
  // in_stride = H*D, dl_stride = H; the fused layout is the raw projection [B, T, 3HD + H])
  int64_t in_stride;
  int64_t dl_stride;
  // fused mode only (the FUSED kernels): q/k/v are normalised in the kernel, delta is the raw
  // logit (0.1 sigmoid(delta) * mask[b*T + t]; mask may be null), and with rms_w the output
  // is head_rmsnorm(o) = o * rsqrt(mean(o^2) + rms_eps) * rms_w
  const uint8_t* mask;
  const float* rms_w;
  float rms_eps;
  // pass C of the unfused scan: flags[bh] = tag when a token of sequence bh lies outside the
  // accuracy envelope (rotation_outside_chunk_envelope); null: no check
  uint32_t* flags;
  uint32_t tag;
};

// Workgroup barrier that orders LDS only.  __syncthreads() also waits for every
// outstanding global load (its release fence), which would stall the whole
// workgroup on the producers' prefetch of the chunk after next at every barrier.
// Only LDS carries data between waves here, so waiting for this wave's LDS
// operations (lgkmcnt(0)) before s_barrier is sufficient.  The empty asm
// statements keep the compiler from moving memory accesses across the barrier.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // vmcnt(63) expcnt(7) lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <typename E>
__device__ __forceinline__ typename mfma_t<E>::v4 lds4(const E* p) {
  return *reinterpret_cast<const typename mfma_t<E>::v4*>(p);
}
template <typename E>
__device__ __forceinline__ typename mfma_t<E>::v8 lds8(const E* p) {
  return *reinterpret_cast<const typename mfma_t<E>::v8*>(p);
}
// Two 8-byte reads issued as two ds_read_b64.  Plain loads would be fused by the compiler
// into ds_read2_b64, which gfx950 serves far slower for these operand patterns (measured with
// SQ_LDS_IDX_ACTIVE / SQ_LDS_BANK_CONFLICT: 16 LDS cycles per read2 of the W operand,
// half of them bank conflicts, against 2 + 2 for the two single reads); volatile LDS
// accesses are never fused.
template <typename E>
__device__ __forceinline__ typename mfma_t<E>::v4 lds4_single(const E* p) {
  typedef typename mfma_t<E>::v4 V4;
  typedef __attribute__((address_space(3))) const volatile V4 lds_v4;
  return *((lds_v4*)(p));
}
template <typename E>
__device__ __forceinline__ typename mfma_t<E>::v8 lds4x2(const E* p0, const E* p1) {
  typedef typename mfma_t<E>::v4 V4;
  typedef typename mfma_t<E>::v8 V8;
  return cat8<V4, V8>(lds4_single<E>(p0), lds4_single<E>(p1));
}

// Transposing LDS read (ds_read_b64_tr_b16).  Within each 16-lane group, lane 4i + r
// supplies the address of 4 consecutive 16-bit elements X[k0 + i][n0 + 4r .. 4r + 3]
// of a row-major block; lane n of the group receives X[k0 + 0..3][n0 + n], i.e. a
// 4-deep k-slice of column n (measured on gfx950).
template <typename E>
__device__ __forceinline__ typename mfma_t<E>::v4 lds_tr4(const E* p) {
  typedef short i16x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  const i16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
  return __builtin_bit_cast(typename mfma_t<E>::v4, r);
}
template <typename E>
__device__ __forceinline__ typename mfma_t<E>::v8 lds_tr4x2(const E* p0, const E* p1) {
  typedef typename mfma_t<E>::v4 V4;
  typedef typename mfma_t<E>::v8 V8;
  return cat8<V4, V8>(lds_tr4<E>(p0), lds_tr4<E>(p1));
}

// Eight 16-bit inputs (one uint4) as f16: bf16 -> f32 (a shift or a mask) -> f16 pairs
// (v_cvt_pk_f16_f32, round to nearest even).  Exact for |x| in [2^-14, 65504]; L2-normalised
// rows (|x| <= 1) lose at most 2^-25 absolute on entries below 2^-14.
template <typename IO> __device__ __forceinline__ uint4 to_f16x8(uint4 x);
template <> __device__ __forceinline__ uint4 to_f16x8<_Float16>(uint4 x) { return x; }
template <> __device__ __forceinline__ uint4 to_f16x8<__bf16>(uint4 x) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  auto cv = [](unsigned u) {
    h2 h;
    h[0] = static_cast<_Float16>(__uint_as_float(u << 16));
    h[1] = static_cast<_Float16>(__uint_as_float(u & 0xffff0000u));
    return __builtin_bit_cast(unsigned, h);
  };
  return make_uint4(cv(x.x), cv(x.y), cv(x.z), cv(x.w));
}

// The same with every value multiplied by s in fp32 first (one rounding to f16).
template <typename IO> __device__ __forceinline__ float lo16_f32(unsigned u);
template <typename IO> __device__ __forceinline__ float hi16_f32(unsigned u);
template <> __device__ __forceinline__ float lo16_f32<__bf16>(unsigned u) { return __uint_as_float(u << 16); }
template <> __device__ __forceinline__ float hi16_f32<__bf16>(unsigned u) {
  return __uint_as_float(u & 0xffff0000u);
}
template <> __device__ __forceinline__ float lo16_f32<_Float16>(unsigned u) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<unsigned short>(u)));
}
template <> __device__ __forceinline__ float hi16_f32<_Float16>(unsigned u) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<unsigned short>(u >> 16)));
}
template <typename IO> __device__ __forceinline__ uint4 to_f16x8_scaled(uint4 x, float s) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  auto cv = [s](unsigned u) {
    h2 h;
    h[0] = static_cast<_Float16>(lo16_f32<IO>(u) * s);
    h[1] = static_cast<_Float16>(hi16_f32<IO>(u) * s);
    return __builtin_bit_cast(unsigned, h);
  };
  return make_uint4(cv(x.x), cv(x.y), cv(x.z), cv(x.w));
}
// Sum over the 16 lanes of a DPP row (lanes 16i .. 16i+15): four DPP adds, no LDS.
template <int CTRL> __device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp_f32<0xB1>(x);   // quad_perm(1, 0, 3, 2)
  x += dpp_f32<0x4E>(x);   // quad_perm(2, 3, 0, 1)
  x += dpp_f32<0x141>(x);  // row_half_mirror: lane i <-> 7 - i within each half row
  x += dpp_f32<0x140>(x);  // row_mirror: lane i <-> 15 - i
  return x;
}

template <typename IO> __device__ __forceinline__ float sumsq8(uint4 x) {
  float acc = 0.f;
  const unsigned w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float a0 = lo16_f32<IO>(w[i]), a1 = hi16_f32<IO>(w[i]);
    acc = fmaf(a0, a0, acc);
    acc = fmaf(a1, a1, acc);
  }
  return acc;
}

template <typename IO, typename DT, bool READOUT, bool FUSED>
__global__ __launch_bounds__(Cfg<READOUT>::NT) void sssd_chunk_kernel(Args a) {
  constexpr int NPW = Cfg<READOUT>::NPW;
  constexpr int NRW = Cfg<READOUT>::NRW;
  constexpr int NT = Cfg<READOUT>::NT;
  typedef _Float16 E;  // MFMA operand type (inputs converted on the way into LDS)
  typedef mfma_t<E> MM;
  typedef typename MM::v8 V8;
  __shared__ Smem<E, READOUT> sm;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int l32 = lane & 31, g = lane >> 5;
  const int l16 = lane & 15, g4 = lane >> 4;

  const int bh = blockIdx.x;
  const int seg = blockIdx.y;
  const int b = bh / a.H, h = bh - (bh / a.H) * a.H;
  const int total_chunks = (a.T + C - 1) / C;
  int chunk0 = seg * a.seg_chunks;
  int nch = total_chunks - chunk0;
  if (nch > a.seg_chunks) nch = a.seg_chunks;
  int split = -1;  // pieces: chunk index (within the piece) where a segment starts
  if (!READOUT && a.npieces > 0) {
    const int64_t span = static_cast<int64_t>(a.nseg - 1) * a.seg_chunks;
    chunk0 = static_cast<int>(seg * span / a.npieces);
    nch = static_cast<int>((seg + 1) * span / a.npieces) - chunk0;
    const int bnd = (chunk0 + a.seg_chunks - 1) / a.seg_chunks * a.seg_chunks;
    if (bnd > chunk0 && bnd < chunk0 + nch) split = bnd - chunk0;
  }
  if (nch <= 0) return;  // uniform across the workgroup

  const int64_t DD = static_cast<int64_t>(D) * D;
  const int64_t tok_stride = a.in_stride;
  const int64_t tok_base = static_cast<int64_t>(b) * a.T * a.in_stride + static_cast<int64_t>(h) * D;
  const int64_t dl_base = static_cast<int64_t>(b) * a.T * a.dl_stride + h;
  const int64_t out_stride = static_cast<int64_t>(a.H) * D;
  const int64_t out_base = (static_cast<int64_t>(b) * a.T * a.H + h) * D;
  const IO* gq = static_cast<const IO*>(a.q);
  const IO* gk = static_cast<const IO*>(a.k);
  const IO* gv = static_cast<const IO*>(a.v);

  // zero T~ buffers (the strictly upper blocks are never written afterwards)
  for (int i = tid; i < 2 * R * TT_LD; i += NT) {
    (&sm.tth[0][0])[i] = E(0.0f);
    (&sm.ttl[0][0])[i] = E(0.0f);
  }

  // Consumers: start state slab (columns 32*wave + l32; tile rt holds rows
  // 32rt + 8(r/4) + 4g + r%4) and its largest magnitude, for the state scale below.
  f32x16 psi[4];
  const int col = 32 * wave + l32;
  if (wave < NCW) {
    const float* src = nullptr;
    if (READOUT && seg == 0)
      src = a.psi0 ? a.psi0 + bh * DD : nullptr;
    else if (READOUT && a.starts)
      src = a.starts + (static_cast<int64_t>(seg - 1) * a.BH + bh) * DD;
    if (src) {
#pragma unroll
      for (int rt = 0; rt < 4; ++rt)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          psi[rt][r] = src[(32 * rt + 8 * (r >> 2) + 4 * g + (r & 3)) * D + col];
    } else {
#pragma unroll
      for (int rt = 0; rt < 4; ++rt)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          psi[rt][r] = (32 * rt + 8 * (r >> 2) + 4 * g + (r & 3)) == col ? 1.f : 0.f;
    }
    float m = 0.f;
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int r = 0; r < 16; ++r) m = fmaxf(m, fabsf(psi[rt][r]));
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if (lane == 0) sm.smax[wave] = m;
  }
  __syncthreads();

  // ---------------------------------------------------------------- producers
  // Every wave runs iterations it = -NPW .. last with the same barriers.  Consumers
  // process chunk it in iteration it (and read out chunk it-1).  Producer p owns the
  // chunks n = p (mod NPW) and spends NPW iterations on each, one phase per iteration.
  // With 6 producers (pass C):
  //   it = n-6  phase 0: global loads of k, v, q, delta into registers
  //   it = n-5  phase 1: k, v to f16 (fused: normalised)
  //   it = n-4  phase 2: Gram matrix (MFMA), Cayley blocks
  //   it = n-3  phase 3: diagonal 8x8 blocks of T~, first off-diagonal step
  //   it = n-2  phase 4: the other off-diagonal blocks (the 16x16 block on MFMA)
  //   it = n-1  phase 5: k, v, q rows -> tok[n % 3], T~ (hi + lo) -> tt[n & 1]
  // with 8 (pass A) the diagonal blocks and the three off-diagonal steps take a phase each
  // (it = n-8 .. n-1), and the U rows go out with the 16x16 block (it = n-2: no readout
  // waves hold tok[n % 3] then).  tok[n % 3] last held chunk n-3, whose readout ended in
  // iteration n-2, and tt[n & 1] last held chunk n-2, so the write overwrites nothing still
  // in use.
  // The scratch of a chunk is pscr[n % 3] with 6 producers (used in iterations n-4 .. n-2;
  // chunk n+3, the next one to use it, starts its Gram in iteration n-1) and the
  // producer's own slot with 8.  Each phase is a short dependent chain, and NPW of them
  // are in flight per workgroup, so their latency stays off the consumers' critical path.
  struct Regs {
    uint4 kv[8];  // k/v in Gram-operand order: rho = l32, features 16ks + 8g + 0..7
    uint4 q[4];   // q: e = lane + 64m -> token e>>4, features 8*(e&15) + 0..7
    DT d;         // raw delta of token `lane` (lanes 0..15)
    uint8_t mk;   // fused mode: active-mask entry of token `lane`
  };

  // Branch-free loads: token indices are clamped to T-1 for the address and tokens
  // past the end are zeroed in phase 1, so no load is predicated.
  auto p_load = [&](Regs& r, int n) {
    const int t0 = (chunk0 + n) * C;
    const int tk = min(t0 + (l32 >> 1), a.T - 1);
    const IO* src = ((l32 & 1) ? gv : gk) + tok_base + tk * tok_stride + 8 * g;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) r.kv[ks] = *reinterpret_cast<const uint4*>(src + 16 * ks);
    if (READOUT) {  // q only feeds the readout
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int e = lane + 64 * m;
        const int tq = min(t0 + (e >> 4), a.T - 1);
        r.q[m] = *reinterpret_cast<const uint4*>(gq + tok_base + tq * tok_stride + 8 * (e & 15));
      }
    }
    const int td = min(t0 + (lane & (C - 1)), a.T - 1);
    r.d = static_cast<const DT*>(a.delta)[dl_base + static_cast<int64_t>(td) * a.dl_stride];
    if constexpr (FUSED) r.mk = a.mask ? a.mask[static_cast<int64_t>(b) * a.T + td] : 1;
  };

  auto dot8 = [](const float* x, const float* y) {
    const float4 x0 = *reinterpret_cast<const float4*>(x);
    const float4 x1 = *reinterpret_cast<const float4*>(x + 4);
    const float4 y0 = *reinterpret_cast<const float4*>(y);
    const float4 y1 = *reinterpret_cast<const float4*>(y + 4);
    float sacc = x0.x * y0.x;
    sacc = fmaf(x0.y, y0.y, sacc); sacc = fmaf(x0.z, y0.z, sacc); sacc = fmaf(x0.w, y0.w, sacc);
    sacc = fmaf(x1.x, y1.x, sacc); sacc = fmaf(x1.y, y1.y, sacc); sacc = fmaf(x1.z, y1.z, sacc);
    return fmaf(x1.w, y1.w, sacc);
  };

  // zero the tokens past the end; fused mode: normalise the k, v rows (to f16)
  auto p_prep = [&](Regs& r, int n) {
    const int t0 = (chunk0 + n) * C;
    if constexpr (!FUSED) {  // a phase before the Gram matrix
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) r.kv[ks] = to_f16x8<IO>(r.kv[ks]);
    }
    if (t0 + C > a.T) {  // last, partial chunk
      const uint4 z = make_uint4(0, 0, 0, 0);
      if (t0 + (l32 >> 1) >= a.T) {
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) r.kv[ks] = z;
      }
      if (READOUT) {
#pragma unroll
        for (int m = 0; m < 4; ++m)
          if (t0 + ((lane + 64 * m) >> 4) >= a.T) r.q[m] = z;
      }
      if (t0 + (lane & (C - 1)) >= a.T) r.d = DT{};
    }
    if constexpr (FUSED) {
      // raw k, v rows: their norms from the diagonal of the raw Gram matrix (MFMA on the
      // input type, fp32 accumulation), then each row scaled by 1 / max(|row|, 1e-12) in
      // fp32 and rounded once to f16 (F.normalize, sssd_attention.py:116-118)
      typedef mfma_t<IO> MR;
      f32x16 racc = {};
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        const typename MR::v8 x = __builtin_bit_cast(typename MR::v8, r.kv[ks]);
        racc = MR::mma32(x, x, racc);
      }
      // lane (l32, g) holds G[8(r/4) + 4g + r%4][l32]: the diagonal entry G[l32][l32] is
      // element r = 4(l32 >> 3) + (l32 & 3) of the half g = (l32 >> 2) & 1, and the other
      // half takes it from lane ^ 32
      const int ri = 4 * (l32 >> 3) + (l32 & 3);
      float dg = racc[0];
#pragma unroll
      for (int r2 = 1; r2 < 16; ++r2) dg = ri == r2 ? racc[r2] : dg;
      const float dx = __shfl_xor(dg, 32);
      const float nn = g == ((l32 >> 2) & 1) ? dg : dx;
      const float inv = rsqrtf(fmaxf(nn, 1e-24f));  // 1 / max(|row|, 1e-12)
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) r.kv[ks] = to_f16x8_scaled<IO>(r.kv[ks], inv);
    }
  };

  // U as f16 (what the consumers use); G = U^T U from the same values, so every chunk
  // factor I + U T~ U^T stays exactly consistent with its Gram matrix; Cayley blocks
  auto p_gram = [&](Regs& r, int n, PScratch& P) {
    const int t0 = (chunk0 + n) * C;
    f32x16 gacc = {};
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      const V8 x = *reinterpret_cast<const V8*>(&r.kv[ks]);
      gacc = MM::mma32(x, x, gacc);
    }
    // lane holds G[8(r/4) + 4g + r%4][l32]; G is symmetric, so store it as row l32
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4)
      *reinterpret_cast<float4*>(&P.gram[l32 * T_LD + 8 * q4 + 4 * g]) =
          make_float4(gacc[4 * q4], gacc[4 * q4 + 1], gacc[4 * q4 + 2], gacc[4 * q4 + 3]);
    wave_sync();
    bool ok = true, wide = false;
    if (lane < C) {
      const int t = lane;
      const float kk = P.gram[(2 * t) * T_LD + 2 * t];
      const float vv = P.gram[(2 * t + 1) * T_LD + 2 * t + 1];
      const float kv = P.gram[(2 * t) * T_LD + 2 * t + 1];
      float dl = io<DT>::to_f32(r.d);
      if constexpr (FUSED)  // delta = 0.1 sigmoid(w_delta x) * active_mask (sssd_attention.py:120-126)
        dl = (r.mk && t0 + t < a.T) ? 0.1f / (1.f + __expf(-dl)) : 0.f;
      const cayley2 M = cayley_guarded(dl, kk, vv, kv, ok);
      P.mcoef[t] = make_float4(M.m00, M.m01, M.m10, M.m11);
      // also every token the f16 operands cannot hold: a non-finite Gram entry comes from a
      // non-finite input (the fp32 kernel applies the same identity guard) or from a finite
      // 16-bit element above the f16 range (65504), which the fp32 kernel takes as it is
      if constexpr (READOUT && !FUSED) wide = !ok || rotation_outside_chunk_envelope(dl, kk, vv, kv);
    }
    if constexpr (READOUT && !FUSED) {
      // hand the sequence to the fp32 recompute (a plain store: every writer stores the tag)
      if (__ballot(wide) != 0 && lane == 0 && a.flags != nullptr) a.flags[bh] = a.tag;
    }
    // Tokens with a non-finite Cayley factor act as R = I (cayley_guarded): their U rows
    // are zeroed and the Gram matrix is recomputed, so no NaN/Inf reaches T~ or the
    // consumers.  The branch is uniform over the wave and taken only for such chunks.
    const uint64_t bad = __ballot(!ok);
    if (bad != 0) {
      if ((bad >> (l32 >> 1)) & 1) {
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) r.kv[ks] = make_uint4(0, 0, 0, 0);
      }
      f32x16 zacc = {};
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        const V8 x = *reinterpret_cast<const V8*>(&r.kv[ks]);
        zacc = MM::mma32(x, x, zacc);
      }
      wave_sync();  // every lane has read its diagonal entries
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4)
        *reinterpret_cast<float4*>(&P.gram[l32 * T_LD + 8 * q4 + 4 * g]) =
            make_float4(zacc[4 * q4], zacc[4 * q4 + 1], zacc[4 * q4 + 2], zacc[4 * q4 + 3]);
      wave_sync();
    }
  };

  // diagonal 8x8 blocks of T~ (4 tokens) by forward substitution, lane = (block gb, column c)
  auto p_diag = [&](PScratch& P) {
    if (lane < 32) {
      int ln = lane;
      asm volatile("" : "+v"(ln));  // lane constants recomputed here, not held across the loop
      const int gb = ln >> 3, c = ln & 7;
      float gblk[8][8];
#pragma unroll
      for (int rr = 0; rr < 8; ++rr) {
        const float4 g0 = *reinterpret_cast<const float4*>(&P.gram[(8 * gb + rr) * T_LD + 8 * gb]);
        const float4 g1 = *reinterpret_cast<const float4*>(&P.gram[(8 * gb + rr) * T_LD + 8 * gb + 4]);
        gblk[rr][0] = g0.x; gblk[rr][1] = g0.y; gblk[rr][2] = g0.z; gblk[rr][3] = g0.w;
        gblk[rr][4] = g1.x; gblk[rr][5] = g1.y; gblk[rr][6] = g1.z; gblk[rr][7] = g1.w;
      }
      float x[8];
#pragma unroll
      for (int t2 = 0; t2 < 4; ++t2) {
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int i = 0; i < 2 * t2; ++i) {
          s0 = fmaf(gblk[2 * t2][i], x[i], s0);
          s1 = fmaf(gblk[2 * t2 + 1][i], x[i], s1);
        }
        const float4 M = P.mcoef[4 * gb + t2];
        const float e0 = (c == 2 * t2 ? 1.f : 0.f) + s0;
        const float e1 = (c == 2 * t2 + 1 ? 1.f : 0.f) + s1;
        x[2 * t2] = fmaf(M.x, e0, M.y * e1);
        x[2 * t2 + 1] = fmaf(M.z, e0, M.w * e1);
      }
      *reinterpret_cast<float4*>(&P.dcol[gb][c * 8]) = make_float4(x[0], x[1], x[2], x[3]);
      *reinterpret_cast<float4*>(&P.dcol[gb][c * 8 + 4]) = make_float4(x[4], x[5], x[6], x[7]);
#pragma unroll
      for (int i = 0; i < 8; ++i) P.drow[gb][i * 8 + c] = x[i];
    }
  };

  // Off-diagonal blocks of T~, by composing the two 8-token halves.  With the 16x16
  // diagonal blocks A = T~[0:16, 0:16] and B = T~[16:32, 16:32] (each itself
  // [[T~_gg, 0], [T~_{g+1,g}, T~_{g+1,g+1}]] with T~_{g+1,g} = T~_{g+1,g+1} G_{g+1,g} T~_gg),
  // the lower-left block is T~[16:32, 0:16] = B G[16:32, 0:16] A.
  //   od_1a / od_1b: the 8x8 blocks T~_10 and T~_32 (lane = element (ea, eb); VALU dot
  //     products through LDS); tv[] receives this lane's element of the blocks 00, 11, 22,
  //     33, 10, 32.
  //   od_c: the 16x16 block by two 16x16x16 products on the fp32 MFMA (exact fp32
  //     products); cv[r] receives T~[16 + 4 g4 + r][l16].  k-slot s of lane group
  //     kg = lane >> 4 is k = 4 kg + s in both products, so the first product's result
  //     (lane (n, g4) holds rows 4 g4 + r of column n) is the second one's B operand as is.
  const int ea = lane >> 3, eb = lane & 7;
  auto od_1a = [&](PScratch& P, float* tv) {  // S for (1,0) and (3,2)
    const float* g1 = &P.gram[(8 + ea) * T_LD];
    const float* g3 = &P.gram[(24 + ea) * T_LD];
#pragma unroll
    for (int gb = 0; gb < 4; ++gb) tv[gb] = P.drow[gb][ea * 8 + eb];
    P.sblk[0][eb * 8 + ea] = dot8(g1, &P.dcol[0][eb * 8]);
    P.sblk[1][eb * 8 + ea] = dot8(g3 + 16, &P.dcol[2][eb * 8]);
  };
  auto od_1b = [&](PScratch& P, float* tv) {  // T~ (1,0) and (3,2)
    tv[4] = dot8(&P.drow[1][ea * 8], &P.sblk[0][eb * 8]);
    tv[5] = dot8(&P.drow[3][ea * 8], &P.sblk[1][eb * 8]);
    P.ocol[eb * 8 + ea] = tv[4];
    P.orow[ea * 8 + eb] = tv[5];
  };
  auto od_c = [&](PScratch& P, float* cv) {
    const int kg = g4;
    const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
    // X = G[16:32, 0:16] A: A operand G[16 + l16][4kg + s]; B operand A[4kg + s][l16]
    const f32x4 ga = *reinterpret_cast<const f32x4*>(&P.gram[(16 + l16) * T_LD + 4 * kg]);
    const float* bs = kg < 2 ? &P.dcol[0][(l16 & 7) * 8 + 4 * kg]
                             : (l16 < 8 ? &P.ocol[l16 * 8 + 4 * (kg - 2)]
                                        : &P.dcol[1][(l16 - 8) * 8 + 4 * (kg - 2)]);
    f32x4 bx = *reinterpret_cast<const f32x4*>(bs);
    if (kg < 2 && l16 >= 8) bx = z4;  // upper-right block of A is zero
    f32x4 X = z4;
#pragma unroll
    for (int si = 0; si < 4; ++si) X = __builtin_amdgcn_mfma_f32_16x16x4f32(ga[si], bx[si], X, 0, 0, 0);
    // T~[16:32, 0:16] = B X: A operand B[l16][4kg + s]; B operand X (as computed)
    const float* as = l16 < 8 ? &P.drow[2][l16 * 8 + 4 * (kg & 1)]
                              : (kg < 2 ? &P.orow[(l16 - 8) * 8 + 4 * kg]
                                        : &P.drow[3][(l16 - 8) * 8 + 4 * (kg - 2)]);
    f32x4 ax = *reinterpret_cast<const f32x4*>(as);
    if (l16 < 8 && kg >= 2) ax = z4;  // upper-right block of B is zero
    f32x4 Cc = z4;
#pragma unroll
    for (int si = 0; si < 4; ++si) Cc = __builtin_amdgcn_mfma_f32_16x16x4f32(ax[si], X[si], Cc, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < 4; ++r) cv[r] = Cc[r];
  };

  // the write: U and q rows, T~ (f16 hi + lo) for the consumers
  // q rows to f16; fused mode: normalised (token (lane + 64m) >> 4 spans 16 consecutive
  // lanes, one DPP row)
  auto p_qprep = [&](Regs& r) {
    if constexpr (READOUT) {
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        if constexpr (FUSED) {
          const float s2 = row16_sum(sumsq8<IO>(r.q[m]));
          r.q[m] = to_f16x8_scaled<IO>(r.q[m], rsqrtf(fmaxf(s2, 1e-24f)));
        } else {
          r.q[m] = to_f16x8<IO>(r.q[m]);
        }
      }
    }
  };

  // the write: U and q rows (p_write_rows), T~ as f16 hi + lo (p_write_tt) for the consumers
  auto p_write_rows = [&](Regs& r, int n) {
    E* tb = sm.tok[n % 3];
    // Each 16-byte piece as two ds_write_b64: rows are 8-byte aligned (264-byte pitch), and a
    // ds_write_b128 of this pattern measured 5x the LDS cycles of the two 8-byte writes.
    E* tdst = tb + rho_slot(l32) * U_LD;
    typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
    typedef __attribute__((address_space(3))) volatile u32x2 lds_u2;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      *((lds_u2*)(tdst + 16 * ks + 8 * g)) = u32x2{r.kv[ks].x, r.kv[ks].y};
      *((lds_u2*)(tdst + 16 * ks + 8 * g + 4)) = u32x2{r.kv[ks].z, r.kv[ks].w};
    }
    if (READOUT) {
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int e = lane + 64 * m;
        uint4 qh;
        if constexpr (FUSED) {
          const float s2 = row16_sum(sumsq8<IO>(r.q[m]));
          qh = to_f16x8_scaled<IO>(r.q[m], rsqrtf(fmaxf(s2, 1e-24f)));
        } else {
          qh = to_f16x8<IO>(r.q[m]);
        }
        *reinterpret_cast<uint4*>(tb + Q_OFF + (e >> 4) * Q_LD + 8 * (e & 15)) = qh;
      }
    }
  };
  auto p_write_tt = [&](int n, const float* tv, const float* cv) {
    // T~ as f16 hi + lo.  Lanes pair up (lane, lane ^ 1) on adjacent columns: the even
    // lane writes the two hi parts, the odd lane the two lo parts, as one 32-bit store
    // each (DPP quad_perm(1, 0, 3, 2) swaps the parts between the two lanes).
    const bool odd = lane & 1;
    uint32_t* const tw = reinterpret_cast<uint32_t*>(odd ? sm.ttl[n & 1] : sm.tth[n & 1]);
    auto put_pair = [&](float x, int row, int col_even) {
      // hi is the f16 rounding of the fp32 value x: the empty asm keeps the compiler from
      // folding the conversion into the FMA that produced x (one f16 rounding of the exact
      // product, which differs from this one in rare ties)
      asm("" : "+v"(x));
      const E hpart = static_cast<E>(x);
      const E lpart = static_cast<E>(x - static_cast<float>(hpart));
      const uint32_t hb = __builtin_bit_cast(uint16_t, hpart), lb = __builtin_bit_cast(uint16_t, lpart);
      const uint32_t recv = static_cast<uint32_t>(
          __builtin_amdgcn_mov_dpp(static_cast<int>(odd ? hb : lb), 0xB1, 0xF, 0xF, false));
      const uint32_t word = odd ? (recv | (lb << 16)) : (hb | (recv << 16));
      tw[(row * TT_LD + col_even) >> 1] = word;
    };
    // the 8x8 blocks 00, 11, 22, 33, 10, 32: element (ea, eb) of each
    const int brow[6] = {0, 1, 2, 3, 1, 3};
    const int bcol[6] = {0, 1, 2, 3, 0, 2};
#pragma unroll
    for (int i = 0; i < 6; ++i) put_pair(tv[i], 8 * brow[i] + ea, 8 * bcol[i] + (eb & ~1));
    // T~[16:32, 0:16]: rows 16 + 4 g4 + r of column l16
#pragma unroll
    for (int r = 0; r < 4; ++r) put_pair(cv[r], 16 + 4 * g4 + r, l16 & ~1);
  };
  auto p_write = [&](Regs& r, int n, const float* tv, const float* cv) {
    p_write_rows(r, n);
    p_write_tt(n, tv, cv);
  };

  // Every iteration ends with one workgroup barrier (A).
  const int last = READOUT ? nch : nch - 1;  // the readout of chunk c runs in iteration c+1
  if (wave >= NCW + NRW) {
    // ================================================ producers
    const int p = wave - NCW - NRW;
    Regs r;
    float tv[6], cv[4];
    // Chunk-major: producer p runs the phases of its chunks n = p, p + NPW, ... as
    // straight-line code, phase k of chunk n in iteration n - NPW + k; bare barriers
    // before its first chunk and after its last keep the count at one per iteration.
    int it = -NPW;
    for (; it < p - NPW; ++it) lds_barrier();  // (A)
    for (int n = p; n < nch; n += NPW) {
      PScratch& P = sm.pscr[NPW == 8 ? p : n % 3];
      if constexpr (NPW == 6) {
        // The diagonal-block and write phases run at a raised issue priority (they share
        // SIMDs with consumer and readout waves, which have slack).  Measured at OP against
        // no raised phase, and against raising the Gram phase or the 16x16 block's phase
        // as well: 1-3 % faster.
        p_load(r, n);
        lds_barrier();  // (A)
        p_prep(r, n);
        lds_barrier();  // (A)
        p_gram(r, n, P);
        lds_barrier();  // (A)
        __builtin_amdgcn_s_setprio(2);
        p_diag(P);
        wave_sync();
        od_1a(P, tv);
        __builtin_amdgcn_s_setprio(0);
        lds_barrier();  // (A)
        od_1b(P, tv);
        wave_sync();
        od_c(P, cv);
        lds_barrier();  // (A)
        __builtin_amdgcn_s_setprio(2);
        p_write(r, n, tv, cv);
        __builtin_amdgcn_s_setprio(0);
        lds_barrier();  // (A)
      } else {
        p_load(r, n);
        lds_barrier();  // (A)
        p_prep(r, n);
        lds_barrier();  // (A)
        p_gram(r, n, P);
        lds_barrier();  // (A)
        p_diag(P);
        lds_barrier();  // (A)
        od_1a(P, tv);
        lds_barrier();  // (A)
        od_1b(P, tv);
        lds_barrier();  // (A)
        od_c(P, cv);
        // no readout waves in this pass: tok[n % 3] (last used by the consumers of chunk n-3 in
        // iteration n-3) is free a phase early, which takes the U rows off the T~ write
        p_write_rows(r, n);
        lds_barrier();  // (A)
        p_write_tt(n, tv, cv);
        lds_barrier();  // (A)
      }
      it = n;
    }
    for (; it <= last; ++it) lds_barrier();  // (A)
    return;
  }

  // The state enters the MFMAs rounded to f16, so it is carried scaled by a power of
  // two s (exact) that puts its largest start entry in [1, 2): every column keeps its
  // norm under the orthogonal updates, so no later entry leaves the f16 range.  The
  // readout and the end state are multiplied back by 1/s.
  float sc = 1.f, inv_s = 1.f;
  {
    const float m = fmaxf(fmaxf(sm.smax[0], sm.smax[1]), fmaxf(sm.smax[2], sm.smax[3]));
    if (m > 0.f && m <= 3.0e38f) {
      int e;
      (void)frexpf(m, &e);  // m = f * 2^e, f in [0.5, 1)
      sc = ldexpf(1.f, 1 - e);
      inv_s = ldexpf(1.f, e - 1);
    }
  }
  const int pg = 2 * (g4 & 1) + (g4 >> 1);
  constexpr int PST_BUF = D * PST_LD, ZST_BUF = D * ZST_LD;

  if (READOUT && wave >= NCW) {
    // ================================================ readout waves
    // Readout of chunk c in iteration c+1 (after barrier (A) of iteration c, which ends
    // the consumers' stash writes of chunk c): readout wave w computes the output rows
    // d in [RWR w, RWR w + RWR) completely, so no cross-wave reduction is needed:
    //   O = S Q + U mask(Z Q)  restricted to those rows; S Q and Z Q contract over all
    //   128 state columns j (k-slot group g4 covers j = 32ks + 8pg + 0..7).
    // Offsets: U rows rho = 16hh + 4g4 + i, features RWR w + 16tl + 4r (transposing reads);
    // q token l16, features 32ks + 8pg; stash rows j = 32ks + 8pg + 4hh + (l16 >> 2),
    // where j_slot(8pg + 4hh + i) = j_slot(8pg + i) + hh (stashes of chunk c in buffer c & 1).
    constexpr int RWR = D / (NRW > 0 ? NRW : 1);  // output rows per readout wave
    constexpr int TL = RWR / 16;                    // 16-row output tiles per readout wave
    const int rw = wave - NCW;
    const int offO = rho_slot(4 * g4 + (l16 >> 2)) * U_LD + RWR * rw + 4 * (l16 & 3);
    const int offQ = Q_OFF + l16 * Q_LD + 8 * pg;
    const E* const pst_rd = sm.pst[0] + j_slot(8 * pg + (l16 >> 2)) * PST_LD + RWR * rw + 4 * (l16 & 3);
    const E* const zst_rd = sm.zst[0] + j_slot(8 * pg + (l16 >> 2)) * ZST_LD + 4 * (l16 & 3);
    // O of chunk c (rows of this wave, scaled state domain): lane (g4, t = l16) gets
    // O[RWR rw + 16 tl + 4 g4 + 0..3][t] in O[tl]
    auto readout_compute = [&](int c, f32x4* O) {
      const E* tb = sm.tok[c % 3];
      const E* const pst_c = pst_rd + (c & 1) * PST_BUF;
      const E* const zst_c = zst_rd + (c & 1) * ZST_BUF;
      f32x4 Y[2] = {};
#pragma unroll
      for (int tl = 0; tl < TL; ++tl) O[tl] = f32x4{};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const V8 bq = lds8<E>(tb + offQ + 32 * ks);
#pragma unroll
        for (int tl = 0; tl < TL; ++tl) {
          const E* p = pst_c + 32 * ks * PST_LD + 16 * tl;
          O[tl] = MM::mma16(lds_tr4x2<E>(p, p + PST_LD), bq, O[tl]);
        }
#pragma unroll
        for (int yy = 0; yy < 2; ++yy) {
          const E* p = zst_c + 32 * ks * ZST_LD + 16 * yy;
          Y[yy] = MM::mma16(lds_tr4x2<E>(p, p + ZST_LD), bq, Y[yy]);
        }
      }
      // Y lane (g4, t = l16) holds rho = 16yy + 4g4 + r: the B-operand layout of U mask(Y)
      V8 by;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        by[r] = static_cast<E>(((4 * g4 + r) >> 1) <= l16 ? Y[0][r] : 0.f);
        by[4 + r] = static_cast<E>(((16 + 4 * g4 + r) >> 1) <= l16 ? Y[1][r] : 0.f);
      }
#pragma unroll
      for (int tl = 0; tl < TL; ++tl)
        O[tl] = MM::mma16(lds_tr4x2<E>(tb + offO + 16 * tl, tb + offO + U_LD + 16 * tl), by, O[tl]);
    };
    // Stored through a buffer resource spanning chunk c's valid tokens: rows past the end
    // of the sequence fall outside it and the hardware drops them, so no branch is needed.
    // Element (row, t) is written as O * scale (* wr[tl][r] when given).
    auto store_out = [&](int c, const f32x4* O, float scale, const float (*wr)[4]) {
      const int t0 = (chunk0 + c) * C;
      const int nvalid = a.out ? min(C, a.T - t0) : 0;
      const __amdgpu_buffer_rsrc_t orsrc = __builtin_amdgcn_make_buffer_rsrc(
          static_cast<IO*>(a.out) + out_base + static_cast<int64_t>(t0) * out_stride, (short)0,
          nvalid * static_cast<int>(out_stride) * static_cast<int>(sizeof(IO)), 0x00020000);
      const int ooff = (l16 * static_cast<int>(out_stride) + RWR * rw + 4 * g4) * static_cast<int>(sizeof(IO));
#pragma unroll
      for (int tl = 0; tl < TL; ++tl) {
        typedef IO io4 __attribute__((ext_vector_type(4)));
        typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
        io4 o4;
#pragma unroll
        for (int r = 0; r < 4; ++r)
          o4[r] = static_cast<IO>(O[tl][r] * (wr ? scale * wr[tl][r] : scale));
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, o4), orsrc,
                                              ooff + 16 * tl * static_cast<int>(sizeof(IO)), 0, 0);
      }
    };
    if constexpr (!FUSED) {
      for (int it = -NPW; it <= last; ++it) {
        if (it >= 1) {  // it - 1 < nch since last = nch
          f32x4 O[TL];
          readout_compute(it - 1, O);
          store_out(it - 1, O, inv_s, nullptr);
        }
        lds_barrier();  // (A)
      }
      return;
    } else {
      // Fused head RMSNorm (sssd_attention.py:177-178, nn.RMSNorm over D): a token's
      // mean(o^2) sums over both readout waves' rows.  Each wave writes its partial sum
      // of chunk c to rsum[c & 1] in iteration c+1 and keeps O in registers; after the
      // next barrier both partials are visible and the chunk is scaled and stored.
      float wr[TL][4];
#pragma unroll
      for (int tl = 0; tl < TL; ++tl)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          wr[tl][r] = a.rms_w ? a.rms_w[RWR * rw + 16 * tl + 4 * g4 + r] : 1.f;
      f32x4 Op[TL];
      auto finalize = [&](int c, const f32x4* O) {
        float scale = inv_s;
        if (a.rms_w) {
          float s2 = 0.f;
#pragma unroll
          for (int w = 0; w < NRW; ++w) s2 += sm.rsum[((c & 1) * NRW + w) * C + l16];
          scale = inv_s * rsqrtf(s2 * inv_s * inv_s * (1.f / D) + a.rms_eps);
        }
        store_out(c, O, scale, wr);
      };
      for (int it = -NPW; it <= last; ++it) {
        if (it >= 1) {
          f32x4 O[TL];
          readout_compute(it - 1, O);
          float s2 = 0.f;
#pragma unroll
          for (int tl = 0; tl < TL; ++tl)
#pragma unroll
            for (int r = 0; r < 4; ++r) s2 = fmaf(O[tl][r], O[tl][r], s2);
          s2 += __shfl_xor(s2, 16);
          s2 += __shfl_xor(s2, 32);
          if (g4 == 0) sm.rsum[(((it - 1) & 1) * NRW + rw) * C + l16] = s2;
          if (it >= 2) finalize(it - 2, Op);
#pragma unroll
          for (int tl = 0; tl < TL; ++tl) Op[tl] = O[tl];
        }
        lds_barrier();  // (A)
      }
      if (last >= 1) finalize(last - 1, Op);
      return;
    }
  }

  // ================================================== consumers
#pragma unroll
  for (int rt = 0; rt < 4; ++rt) psi[rt] *= sc;

  // Per-lane element offsets into a chunk buffer (constant parts are added at the use).
  //   offW: W operand, U^T row rho = l32, features 32rt + 16ks + 4g + {0..3, 8..11}
  //   offU: update operand via transposing reads: rows rho = 16ks + 8hh + 4g + i,
  //         features 32rt + 16 (lane>>4 & 1) + 4r  ->  lane gets U[32rt + l32][rho..rho+3]
  // rho_slot is linear over disjoint bits, so +16ks / +8hh are +ks / +2hh slots.
  const int offW = rho_slot(l32) * U_LD + 4 * g;
  const int offU = rho_slot(4 * g + (l16 >> 2)) * U_LD + 16 * ((lane >> 4) & 1) + 4 * (l16 & 3);
  // readout stash rows written: j = col = 32 wave + l32 (buffer 0; chunk c uses buffer c & 1)
  E* const pst_wr = sm.pst[0] + (32 * wave + j_slot(l32)) * PST_LD + 4 * g;
  E* const zst_wr = sm.zst[0] + (32 * wave + j_slot(l32)) * ZST_LD + 4 * g;

  // One iteration; ACTIVE is compile-time so that the steady-state body is a single
  // basic block the scheduler can overlap freely.
  auto iteration = [&](int cc, auto active) {
    constexpr bool ACT = decltype(active)::value;
    const E* tb = sm.tok[ACT ? cc % 3 : 0];
    E* const pw = pst_wr + (cc & 1) * PST_BUF;  // this chunk's readout stashes
    E* const zw = zst_wr + (cc & 1) * ZST_BUF;
    V8 wu[4][2];  // W operands (ready since two iterations back)
    if constexpr (ACT) {
#pragma unroll
      for (int rt = 0; rt < 4; ++rt)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const E* p = tb + offW + 32 * rt + 16 * ks;
          wu[rt][ks] = lds4x2<E>(p, p + 8);
        }
    }

    // W = U^T Psi_slab  (32 x 32), the (scaled) state rounded once to f16; the same
    // f16 values go to the readout stash.
    V8 pb[4][2];
    f32x16 W = {};
    if constexpr (ACT) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) {
          float x[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) x[i] = psi[rt][8 * ks + i];
          pb[rt][ks] = round8<E>(x);
          W = MM::mma32(wu[rt][ks], pb[rt][ks], W);
        }
    }
    // T~ operands and the update operands (transposing reads of U): both buffers were
    // completed before earlier barriers.
    V8 ahi[2], alo[2], uu[2][4];
    if constexpr (ACT) {
      const int cb = cc & 1;  // T~ buffer
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const E* th = sm.tth[cb] + l32 * TT_LD + 16 * ks + 4 * g;
        const E* tl = sm.ttl[cb] + l32 * TT_LD + 16 * ks + 4 * g;
        ahi[ks] = lds4x2<E>(th, th + 8);
        alo[ks] = lds4x2<E>(tl, tl + 8);
      }
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) {
          const E* p = tb + offU + ks * U_LD + 32 * rt;
          uu[ks][rt] = lds_tr4x2<E>(p, p + 2 * U_LD);
        }
    }
    if constexpr (ACT) {
      if (READOUT) {
        // psi tile rt, ks, half hh holds rows 32rt + 16ks + 8hh + 4g + 0..3 of column col
#pragma unroll
        for (int rt = 0; rt < 4; ++rt)
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
            typedef typename MM::v4 V4;
            const V4 h0 = __builtin_shufflevector(pb[rt][ks], pb[rt][ks], 0, 1, 2, 3);
            const V4 h1 = __builtin_shufflevector(pb[rt][ks], pb[rt][ks], 4, 5, 6, 7);
            *reinterpret_cast<V4*>(pw + 32 * rt + 16 * ks) = h0;
            *reinterpret_cast<V4*>(pw + 32 * rt + 16 * ks + 8) = h1;
          }
      }

      // Z = T~ W with T~ = hi + lo (f16 pair) from the producers, W rounded once to f16
      f32x16 Z = {};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        float wv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) wv[i] = W[8 * ks + i];
        const V8 wb = round8<E>(wv);
        Z = MM::mma32(ahi[ks], wb, Z);
        Z = MM::mma32(alo[ks], wb, Z);
      }

      // Psi_slab += U Z;  Z tile ks holds rho = 16ks + 8hh + 4g + 0..3 of column col
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        float zv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) zv[i] = Z[8 * ks + i];
        const V8 zb = round8<E>(zv);
        if (READOUT) {
          typedef typename MM::v4 V4;
          *reinterpret_cast<V4*>(zw + 16 * ks) = __builtin_shufflevector(zb, zb, 0, 1, 2, 3);
          *reinterpret_cast<V4*>(zw + 16 * ks + 8) = __builtin_shufflevector(zb, zb, 4, 5, 6, 7);
        }
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) psi[rt] = MM::mma32(uu[ks][rt], zb, psi[rt]);
      }
    }
    lds_barrier();  // (A)
  };

  auto write_state = [&](float* dst) {
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        dst[(32 * rt + 8 * (r >> 2) + 4 * g + (r & 3)) * D + col] = psi[rt][r] * inv_s;
  };
  typedef std::integral_constant<bool, true> yes;
  typedef std::integral_constant<bool, false> no;
  for (int cc = -NPW; cc < 0; ++cc) iteration(cc, no{});
  if (READOUT) {
    for (int cc = 0; cc < nch; ++cc) iteration(cc, yes{});
    iteration(nch, no{});  // the readout waves' last iteration
    if (seg == a.nseg - 1) write_state(a.ends + bh * DD);
    return;
  }
  // pass A: factor slots of this workgroup's parts
  const int f0 = a.npieces > 0 ? (seg == 0 ? 0 : 2 * seg - 1) : seg;
  const int n1 = split > 0 ? split : nch;
  for (int cc = 0; cc < n1; ++cc) iteration(cc, yes{});
  if (split > 0) {  // a segment starts here: store the part so far, restart from I
    write_state(a.ends + (static_cast<int64_t>(f0) * a.BH + bh) * DD);
    int colx = col;
    asm volatile("" : "+v"(colx));  // keeps the identity pattern from being hoisted
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        psi[rt][r] = (32 * rt + 8 * (r >> 2) + 4 * g + (r & 3)) == colx ? 1.f : 0.f;
    for (int cc = split; cc < nch; ++cc) iteration(cc, yes{});
  }
  write_state(a.ends + (static_cast<int64_t>(split > 0 ? 2 * seg : f0) * a.BH + bh) * DD);
}

// The segment start states: X = psi0 (identity if null), then X <- F_f X for the pass A
// factors f = 0 .. nf-1 in order, storing start_s = X after every FSTRIDE-th factor
// (FSTRIDE = 1: F_f = P_f; 2: F_2s, F_2s+1 are the two parts of segment s).
// Left products act on the columns independently, so the chain of one sequence is
// split over CARRY_SPLIT workgroups of CARRY_COLS columns each (grid (BH, CARRY_SPLIT):
// with BH a multiple of 8 the blocks of one sequence share an XCD, hence its L2 copy of
// every factor).  Two roles per workgroup:
//   producer waves load factor f + 1 (coalesced float4, one product ahead) and stage it
//                  in LDS as a bf16 hi + lo pair (double-buffered) while
//   consumer waves multiply factor f into the running columns X (kept in LDS the same
//                  way, transposed): wave w produces rows 32w .. 32w+31 with bf16x3 MFMA
//                  (hi*hi + hi*lo + lo*hi, fp32-faithful), then writes them back to X.
// Both roles pass the same two LDS-only barriers per product.  (Staging on the same waves
// as the products, one buffer, two column blocks per sequence: 18.2 us at OP.)
constexpr int CARRY_SPLIT = 4;
constexpr int CARRY_COLS = D / CARRY_SPLIT;          // 32
constexpr int CARRY_CW = D / 32;                     // consumer waves (32 rows each)
constexpr int CARRY_PW = 8;                          // producer waves
constexpr int CARRY_NT = (CARRY_CW + CARRY_PW) * 64;
constexpr int CARRY_PT = CARRY_PW * 64;
constexpr int CP_LD = D + 8;   // bf16 per LDS row of a factor and of X^T (272 B)
constexpr int CARRY_F4 = D * D / 4 / CARRY_PT;      // float4 of a factor per producer thread
static_assert(CARRY_COLS == 32, "one 32-column MFMA tile per consumer wave");

template <int FSTRIDE>
__global__ __launch_bounds__(CARRY_NT) void sssd_carry_kernel(const float* psi0, const float* F,
                                                              float* starts, int BH, int nf) {
  static_assert(FSTRIDE == 1 || FSTRIDE == 2, "one or two factors per segment");
  typedef mfma_t<__bf16> MM;
  typedef MM::v8 V8;
  __shared__ __bf16 phi[2][D * CP_LD], plo[2][D * CP_LD];              // factor, row-major
  __shared__ __bf16 xhi[CARRY_COLS * CP_LD], xlo[CARRY_COLS * CP_LD];  // X^T: [n][k]
  const int bh = blockIdx.x, cb = blockIdx.y;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, g = lane >> 5;
  const int64_t DD = static_cast<int64_t>(D) * D;
  if (nf <= 0) return;  // uniform
  // producers: factor f + 1 is staged during product f, from registers loaded two
  // products ahead (two register buffers; every fetch and stage is issued, clamped to the
  // last factor past the end, so the waits count a fixed sequence of loads)
  const int pt = tid - CARRY_CW * 64;
  float4 pa[CARRY_F4], pb[CARRY_F4];
  auto fetch = [&](float4* pf, int f) {  // 0 <= f < nf
    const float4* src = reinterpret_cast<const float4*>(F + (static_cast<int64_t>(f) * BH + bh) * DD);
#pragma unroll
    for (int m = 0; m < CARRY_F4; ++m) pf[m] = src[pt + CARRY_PT * m];
  };
  auto stage = [&](const float4* pf, int buf) {  // 8-byte stores of hi and lo
    // not hoisted into the previous product's phase (it would wait for loads early)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int m = 0; m < CARRY_F4; ++m) {
      const int e = 4 * (pt + CARRY_PT * m);
      const int row = e / D, c0 = e - row * D;
      const float xv[4] = {pf[m].x, pf[m].y, pf[m].z, pf[m].w};
      bf16x4 h4, l4;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        h4[i] = static_cast<__bf16>(xv[i]);
        l4[i] = static_cast<__bf16>(xv[i] - static_cast<float>(h4[i]));
      }
      *reinterpret_cast<bf16x4*>(&phi[buf][row * CP_LD + c0]) = h4;
      *reinterpret_cast<bf16x4*>(&plo[buf][row * CP_LD + c0]) = l4;
    }
  };
  const bool producer = wave >= CARRY_CW;  // uniform per wave
  if (producer) {
    fetch(pa, 0);
    fetch(pb, nf > 1 ? 1 : 0);
  }
  // X = the block's columns of psi0, transposed (identity if null)
  if (psi0) {
    for (int e = tid; e < CARRY_COLS * D; e += CARRY_NT) {
      const int row = e / CARRY_COLS, n = e - row * CARRY_COLS;
      const float x = psi0[bh * DD + row * D + CARRY_COLS * cb + n];
      const __bf16 h = static_cast<__bf16>(x);
      xhi[n * CP_LD + row] = h;
      xlo[n * CP_LD + row] = static_cast<__bf16>(x - static_cast<float>(h));
    }
  } else {
    constexpr int WPR = CP_LD / 4;  // 8-byte words per X^T row (padding included)
    for (int w = tid; w < CARRY_COLS * WPR; w += CARRY_NT) {
      const int n = w / WPR, k0 = 4 * (w - n * WPR), diag = CARRY_COLS * cb + n;
      bf16x4 h4;
#pragma unroll
      for (int i = 0; i < 4; ++i) h4[i] = static_cast<__bf16>(k0 + i == diag ? 1.f : 0.f);
      *reinterpret_cast<bf16x4*>(&xhi[n * CP_LD + k0]) = h4;
      *reinterpret_cast<bf16x4*>(&xlo[n * CP_LD + k0]) = bf16x4{};
    }
  }
  if (producer) {
    stage(pa, 0);
    fetch(pa, nf > 2 ? 2 : nf - 1);
    lds_barrier();  // factor 0 staged, X complete
    int f = 0;
    for (; f + 1 < nf; f += 2) {
      // product f reads buffer 0: stage factor f+1 into buffer 1
      stage(pb, 1);
      fetch(pb, f + 3 < nf ? f + 3 : nf - 1);
      lds_barrier();  // product f has read its factor and X
      lds_barrier();  // X updated; factor f+1 staged
      // product f+1 reads buffer 1: stage factor f+2 (the last one again past the end)
      // into buffer 0, read by product f before the barrier above
      stage(pa, 0);
      fetch(pa, f + 4 < nf ? f + 4 : nf - 1);
      lds_barrier();
      lds_barrier();
    }
    if (f < nf) {  // odd nf: the last product stages nothing
      lds_barrier();
      lds_barrier();
    }
  } else {
    // consumers: X <- F_f X, rows 32 wave .. 32 wave + 31 of the block's columns
    lds_barrier();
    for (int f = 0; f < nf; ++f) {
      const int buf = f & 1;
      // A row = l32, B column = l32, k-slots 16ks + 8g + 0..7 in both operands; three
      // independent accumulator chains (hi hi, hi lo, lo hi) interleave in the MFMA pipe
      f32x16 Y = {}, Y1 = {}, Y2 = {};
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        const int ka = 16 * ks + 8 * g;
        const V8 ah = *reinterpret_cast<const V8*>(&phi[buf][(32 * wave + l32) * CP_LD + ka]);
        const V8 al = *reinterpret_cast<const V8*>(&plo[buf][(32 * wave + l32) * CP_LD + ka]);
        const V8 bh8 = *reinterpret_cast<const V8*>(&xhi[l32 * CP_LD + ka]);
        const V8 bl8 = *reinterpret_cast<const V8*>(&xlo[l32 * CP_LD + ka]);
        Y = MM::mma32(ah, bh8, Y);
        Y1 = MM::mma32(ah, bl8, Y1);
        Y2 = MM::mma32(al, bh8, Y2);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) Y[r] += Y1[r] + Y2[r];
      lds_barrier();  // every wave has read the factor and X before X is replaced
      // Y: lane (g, l32) holds rows 32 wave + 8(r/4) + 4g + r%4 of column l32
#pragma unroll
      for (int i = 0; i < 4; ++i) {  // rows 32 wave + 8i + 4g + 0..3: 4 consecutive k of X^T
        const int row0 = 32 * wave + 8 * i + 4 * g;
        bf16x4 h4, l4;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float y = Y[4 * i + r];
          h4[r] = static_cast<__bf16>(y);
          l4[r] = static_cast<__bf16>(y - static_cast<float>(h4[r]));
        }
        *reinterpret_cast<bf16x4*>(&xhi[l32 * CP_LD + row0]) = h4;
        *reinterpret_cast<bf16x4*>(&xlo[l32 * CP_LD + row0]) = l4;
      }
      if ((f + 1) % FSTRIDE == 0) {  // uniform: a segment start is complete
        float* dst = starts + (static_cast<int64_t>((f + 1) / FSTRIDE - 1) * BH + bh) * DD +
                     CARRY_COLS * cb + l32;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) dst[(32 * wave + 8 * i + 4 * g + r) * D] = Y[4 * i + r];
      }
      lds_barrier();  // X updated (and the next factor staged)
    }
  }
}

}  // namespace chunk

// ------------------------------------------------------------------ host side
namespace {

constexpr int kTargetWorkgroups = 256;  // one workgroup per CU (LDS-limited)

struct Plan {
  int nchunks, seg_chunks, nseg;
  int npieces;   // pass A workgroups per sequence (0: one per segment 0 .. nseg-2)
  int nfactors;  // pass A transforms per sequence
  int fstride;   // factors per segment
};

Plan make_plan(int64_t BH, int64_t T) {
  Plan p;
  p.nchunks = static_cast<int>((T + chunk::C - 1) / chunk::C);
  int64_t S = (kTargetWorkgroups + BH - 1) / BH;
  const int64_t max_by_len = p.nchunks / 4;  // keep >= 4 chunks per segment
  if (S > max_by_len) S = max_by_len;
  if (S < 1) S = 1;
  p.seg_chunks = static_cast<int>((p.nchunks + S - 1) / S);
  p.nseg = (p.nchunks + p.seg_chunks - 1) / p.seg_chunks;
  // Pass A covers segments 0 .. nseg-2.  Spread over nseg workgroups per sequence instead
  // of nseg-1 it fills as many CUs as pass C; every segment then holds exactly one piece
  // boundary (given seg_chunks >= 2 nseg) and contributes two factors to the carry.  That
  // saves seg_chunks / nseg chunk iterations of pass A (~1.4 us each) for nseg - 1 more
  // carry products (~2.8 us each), so pieces only pay while
  // seg_chunks > 2 nseg (nseg - 1) (OP: 64 > 24; the FULL shape, 16 chunks in 8
  // segments, and LONG, 256 in 16, take one workgroup per segment).
  if (p.nseg > 1 && p.seg_chunks >= 2 * p.nseg &&
      p.seg_chunks > 2 * p.nseg * (p.nseg - 1)) {
    p.npieces = p.nseg;
    p.nfactors = 2 * (p.nseg - 1);
    p.fstride = 2;
  } else {
    p.npieces = 0;
    p.nfactors = p.nseg - 1;
    p.fstride = 1;
  }
  return p;
}

bool chunk_path(int64_t T, int64_t D, int io_dtype) {
  return D == chunk::D && (io_dtype == VMI_BF16 || io_dtype == VMI_F16) && T >= 2 * chunk::C;
}

// The three launches of one scan; `a` carries the inputs (pointers, strides, fused-mode
// fields), the rest is filled in here.
template <typename IO, typename DT, bool FUSED>
hipError_t run_chunked_args(chunk::Args a, const float* psi_in, void* out, float* psi_out, int B,
                            int T, int H, void* workspace, hipStream_t stream) {
  const int BH = B * H;
  const Plan p = make_plan(BH, T);
  const int64_t DD = static_cast<int64_t>(chunk::D) * chunk::D;
  a.T = T; a.H = H; a.BH = BH;
  a.seg_chunks = p.seg_chunks;
  a.nseg = p.nseg;
  a.npieces = 0;
  // workspace: pass A factors, then the segment start states
  float* P = static_cast<float*>(workspace);
  float* starts = P ? P + static_cast<int64_t>(p.nfactors) * BH * DD : nullptr;
  if (p.nseg > 1) {
    chunk::Args pa = a;
    pa.psi0 = nullptr;
    pa.starts = nullptr;
    pa.out = nullptr;
    pa.ends = P;
    pa.end_mode = 0;
    pa.npieces = p.npieces;
    hipLaunchKernelGGL((chunk::sssd_chunk_kernel<IO, DT, false, FUSED>),
                       dim3(BH, p.npieces > 0 ? p.npieces : p.nseg - 1),
                       dim3(chunk::Cfg<false>::NT), 0, stream, pa);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (p.fstride == 2)
      hipLaunchKernelGGL(chunk::sssd_carry_kernel<2>, dim3(BH, chunk::CARRY_SPLIT),
                         dim3(chunk::CARRY_NT), 0, stream, psi_in, P, starts, BH, p.nfactors);
    else
      hipLaunchKernelGGL(chunk::sssd_carry_kernel<1>, dim3(BH, chunk::CARRY_SPLIT),
                         dim3(chunk::CARRY_NT), 0, stream, psi_in, P, starts, BH, p.nfactors);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  a.psi0 = psi_in;
  a.starts = p.nseg > 1 ? starts : nullptr;
  a.out = out;
  a.ends = psi_out;
  a.end_mode = 1;
  hipLaunchKernelGGL((chunk::sssd_chunk_kernel<IO, DT, true, FUSED>), dim3(BH, p.nseg),
                     dim3(chunk::Cfg<true>::NT), 0, stream, a);
  return hipGetLastError();
}

template <typename IO, typename DT>
hipError_t run_chunked(const void* q, const void* k, const void* v, const void* delta,
                       int delta_dtype, const float* psi_in, void* out, float* psi_out, int B,
                       int T, int H, void* workspace, uint32_t* flags, uint32_t tag,
                       hipStream_t stream) {
  chunk::Args a{};
  a.q = q; a.k = k; a.v = v; a.delta = delta; a.delta_dtype = delta_dtype;
  a.in_stride = static_cast<int64_t>(H) * chunk::D;
  a.dl_stride = H;
  a.flags = flags;
  a.tag = tag;
  return run_chunked_args<IO, DT, false>(a, psi_in, out, psi_out, B, T, H, workspace, stream);
}

// Raw projections proj [B, T, proj_stride] = x [W_q; W_k; W_v; W_delta]^T: q, k, v of head h
// at columns h*D, HD + h*D, 2HD + h*D, the delta logit at column 3HD + h.
template <typename IO>
hipError_t run_chunked_fused(const void* proj, int64_t proj_stride, const uint8_t* mask,
                             const float* rms_w,
                             float rms_eps, const float* psi_in, void* out, float* psi_out, int B,
                             int T, int H, void* workspace, hipStream_t stream) {
  const int64_t HD = static_cast<int64_t>(H) * chunk::D;
  const IO* base = static_cast<const IO*>(proj);
  chunk::Args a{};
  a.q = base; a.k = base + HD; a.v = base + 2 * HD; a.delta = base + 3 * HD;
  a.delta_dtype = std::is_same<IO, __bf16>::value ? VMI_BF16 : VMI_F16;
  a.in_stride = proj_stride;
  a.dl_stride = proj_stride;
  a.mask = mask;
  a.rms_w = rms_w;
  a.rms_eps = rms_eps;
  typedef typename std::conditional<std::is_same<IO, __bf16>::value, bf16_t, f16_t>::type DT;
  return run_chunked_args<IO, DT, true>(a, psi_in, out, psi_out, B, T, H, workspace, stream);
}

}  // namespace

namespace {

// Workspace of the unfused scan: the plan's own buffers (pass A factors and segment starts, or
// the column-split scan's rings), then one flag word per sequence at this offset.
size_t flags_offset(int64_t B, int64_t T, int64_t H, int64_t D, int io_dtype) {
  const Plan p = make_plan(B * H, T);
  size_t plan = p.nseg <= 1 ? 0
                            : static_cast<size_t>(p.nfactors + p.nseg - 1) * B * H * D * D *
                                  sizeof(float);
  // enough for either plan: the column-split scan is chosen at launch (use_xsplit)
  if (use_xsplit(B, T, H, D, io_dtype)) plan = std::max(plan, xsplit_workspace_bytes(B, H));
  return (plan + 255) & ~size_t(255);
}

// Tags of the envelope flags: a fresh nonzero value per scan, so flag words left in a reused
// workspace by earlier scans (or never written) do not match.
std::atomic<uint32_t> g_flag_tag{0x6a09e667u};
uint32_t next_flag_tag() {
  uint32_t t = ++g_flag_tag;
  if (t == 0) t = ++g_flag_tag;
  return t;
}

}  // namespace

size_t chunk_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t D, int io_dtype) {
  if (!chunk_path(T, D, io_dtype)) return 0;
  return flags_offset(B, T, H, D, io_dtype) + static_cast<size_t>(B * H) * sizeof(uint32_t);
}

bool use_chunk_path(int64_t T, int64_t D, int io_dtype) { return chunk_path(T, D, io_dtype); }

hipError_t launch_sssd_chunked_fused(const void* proj, int64_t proj_stride, int io_dtype,
                                     const uint8_t* mask,
                                     const float* rms_w, float rms_eps, const float* psi_in,
                                     void* out, float* psi_out, int B, int T, int H,
                                     void* workspace, hipStream_t stream) {
  if (io_dtype == VMI_BF16)
    return run_chunked_fused<__bf16>(proj, proj_stride, mask, rms_w, rms_eps, psi_in, out, psi_out, B, T, H,
                                     workspace, stream);
  return run_chunked_fused<_Float16>(proj, proj_stride, mask, rms_w, rms_eps, psi_in, out, psi_out, B, T, H,
                                     workspace, stream);
}

hipError_t launch_sssd_chunked(const void* q, const void* k, const void* v, const void* delta,
                               int io_dtype, int delta_dtype, const float* psi_in, void* out,
                               float* psi_out, int B, int T, int H, void* workspace,
                               hipStream_t stream) {
  // The f16-operand scan flags every sequence with a token outside its accuracy envelope
  // (rotation_outside_chunk_envelope); a second launch recomputes exactly those sequences in
  // fp32, token by token, from psi_in (which the scan leaves intact: it may not alias psi_out),
  // overwriting their outputs and final states.  Its other workgroups exit at once.
  uint32_t* flags = reinterpret_cast<uint32_t*>(static_cast<char*>(workspace) +
                                                flags_offset(B, T, H, chunk::D, io_dtype));
  const uint32_t tag = next_flag_tag();
  hipError_t e;
  if (use_xsplit(B, T, H, chunk::D, io_dtype) &&
      (delta_dtype == VMI_F32 || (reinterpret_cast<uintptr_t>(delta) & 3) == 0)) {
    e = launch_sssd_xsplit(q, k, v, delta, io_dtype, delta_dtype, psi_in, out, psi_out, B, T, H,
                           workspace, flags, tag, stream);
  } else {
#define VMI_RUN(E, DT) \
  e = run_chunked<E, DT>(q, k, v, delta, delta_dtype, psi_in, out, psi_out, B, T, H, workspace, \
                         flags, tag, stream)
    if (io_dtype == VMI_BF16) {
      if (delta_dtype == VMI_F32) VMI_RUN(__bf16, float);
      else if (delta_dtype == VMI_BF16) VMI_RUN(__bf16, bf16_t);
      else VMI_RUN(__bf16, f16_t);
    } else {
      if (delta_dtype == VMI_F32) VMI_RUN(_Float16, float);
      else if (delta_dtype == VMI_BF16) VMI_RUN(_Float16, bf16_t);
      else VMI_RUN(_Float16, f16_t);
    }
#undef VMI_RUN
  }
  if (e != hipSuccess) return e;
  return launch_sssd_seq(q, k, v, delta, io_dtype, delta_dtype, psi_in, out, psi_out, B, T, H,
                         chunk::D, stream, FlaggedStates{flags, tag});
}

}  // namespace vmi
