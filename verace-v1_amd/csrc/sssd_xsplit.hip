// Column-split SSSD prefill scan (bf16 or fp16 I/O, head_dim 128): one pass, no segment
// transforms.  Four workgroups per sequence (one "group") each own 32 of the 128 state
// columns for the whole sequence and run the chunked recurrence on them.  Left products
// act on the columns independently, so the state update needs nothing from the other
// workgroups; what they share is (a) each chunk's factor (U as f16 and T~), computed once
// by its owner workgroup (chunk n is owned by workgroup n mod 4) and handed to the group
// through a ring in global memory, and (b) the output, which sums over all 128 columns:
// every workgroup computes the partial output of its columns and the group reduces it
// (workgroup r sums output rows 32r .. 32r+31 of every chunk).  The four workgroups of a
// group run on one XCD (checked at start), so all of it stays in that XCD's L2.
//
// Math (reference recurrence sssd_attention.py:160-175, regrouped per chunk of C = 16
// tokens, as in sssd_chunk.hip): U = [k_0 v_0 k_1 v_1 ...] (D x 32), G = U^T U,
// T~ = (I - L)^-1 blockdiag(M) (L_{t,i} = M_t G_{t,i}, i < t), and for the state columns
// S of this workgroup:  W = U^T S,  Z = T~ W,  S' = S + U Z,
// partial readout O_g = S Q_g + U (mask o (Z Q_g)), Q_g the query entries of these columns.
//
// Workgroup = 6 waves (wave w runs on SIMD w mod 4):
//   0, 1  chain: 16 state columns each (8 MFMA 16x16x32 accumulators), per chunk W, Z and
//         the update; they stash the chunk-start state and Z (f16, transposed) in LDS
//   2     readout: partial output of chunk c-1 from the stashes; own rows to LDS, the other
//         three row blocks to the group's partial ring; loads q
//   3     producer: the chunk factors this workgroup owns, in 8 phases over 8 iterations
//         (two chunks in flight): loads, f16 conversion and Gram matrix on MFMA, Cayley
//         blocks, U rows to the ring, diagonal and off-diagonal blocks of T~, T~ (f16 hi + lo)
//         to the ring
//   4     loader: copies chunk n's ring image (U and T~, 14 KB) into LDS with direct
//         global->LDS loads three iterations ahead of its use
//   5     reducer: sums the four partials of its output rows and stores them
// All waves run the same iterations i = -LP .. N + LR + 1 with one LDS barrier each.
//
// Hand-offs between workgroups use per-workgroup progress counters in global memory
// (64-bit: call tag << 32 | count, so values left by other calls never match), written
// with device-scope stores after the data they cover has completed, and read with
// device-scope loads (which miss the CU's L1).  Each role loads the counters it needs one
// iteration ahead, and the leads below make them satisfied in steady state; a role whose
// counter is behind polls it (bounded: on timeout the call is marked failed, the wave stops
// waiting and the outputs it writes become NaN).  All waits point to earlier iterations of
// the other workgroups, which are resident at the same time (cooperative launch), so the
// grid always drains.
#include <atomic>
#include <type_traits>

#include "vmi_common.h"
#include "vmi_dispatch.h"
#include "vmi_mfma.h"

namespace vmi {
namespace xs {

typedef _Float16 E;
typedef mfma_t<E> MM;
typedef MM::v4 V4;
typedef MM::v8 V8;

constexpr int D = 128;
constexpr int C = 16;
constexpr int R = 2 * C;
constexpr int NG = 4;            // workgroups per sequence
constexpr int GC = D / NG;       // state columns per workgroup
constexpr int NWAVES = 8;
constexpr int NT = 64 * NWAVES;
constexpr int LDA = 3;           // the ring loader copies chunk n in iteration n - LDA
constexpr int NPH = 8;           // producer phases per chunk
constexpr int LP = 14;           // the producer starts chunk n in iteration n - LP
constexpr int NB = 5;            // LDS chunk buffers (chunks i-1 .. i+3 live in iteration i)
constexpr int NR = 12;           // ring slots per sequence (slot n mod NR)
constexpr int LQ = 3;            // the input loader copies q of chunk n in iteration n - LQ
constexpr int NQ = 5;            // LDS q slots
constexpr int LK = 4;            // ... and k, v, delta of owned chunk n in iteration n - LP - LK
constexpr int LRD = 4;           // the gatherer copies the partials of chunk i - LRD in iteration i
constexpr int NP = 6;            // partial-ring slots per sequence
constexpr int NOWN = 6;          // LDS slots for the readout's own row block
constexpr int I0 = -LP - LK;     // first iteration
static_assert(NPH == 2 * NG, "two owned chunks in flight per producer");
static_assert(NR % NG == 0, "a ring slot always has the same owner");

// Chunk image (ring slot and LDS buffer), f16 elements:
//   U row rho at rho_slot(rho) * U_LD, T~ hi rows at IMG_TH + row * TT_LD, T~ lo at IMG_TL.
constexpr int U_LD = D + 4;      // 264 B: rows rho_slot 0..31 fall 2 banks apart
constexpr int TT_LD = R + 8;     // 80 B
constexpr int IMG_TH = R * U_LD;
constexpr int IMG_TL = IMG_TH + R * TT_LD;
constexpr int IMG_ELEMS = IMG_TL + R * TT_LD;
constexpr int IMG_BYTES = 14 * 1024;  // multiple of the 1 KB one direct load instruction copies
constexpr int IMG_DMAS = IMG_BYTES / 1024;
static_assert(IMG_ELEMS * 2 <= IMG_BYTES, "chunk image");
// Readout stashes: rows j (state column within the workgroup) at slot jsig(j).
constexpr int PST_LD = D + 8;    // 272 B (68 dwords)
constexpr int ZST_LD = R + 8;    // 80 B
constexpr int T_LD = R + 4;      // fp32 Gram rows

// Bank model (gfx950): 64 banks of 4 B, 64-bit accesses served per 32 lanes.  The slot maps
// below make every operand read, transposing read and stash write conflict-free.
__host__ __device__ constexpr int rho_slot(int rho) {  // bits 0,1,2,3,4 -> 3,4,2,1,0
  return ((rho & 1) << 3) | ((rho & 2) << 3) | (rho & 4) | ((rho & 8) >> 2) | ((rho & 16) >> 4);
}
__host__ __device__ constexpr int jsig(int j) {  // bits 0,1,2,3,4 -> 1,2,3,0,4
  return (j & 16) | ((j & 7) << 1) | ((j >> 3) & 1);
}

// Per-sequence control block (256 B): 64-bit counters, tag << 32 | count.
enum { CTR_HELLO = 0, CTR_T = 4, CTR_R = 8, CTR_P = 12, CTR_D = 16, CTR_WORDS = 32 };
//   hello[g]: XCC id + 1 of workgroup g
//   tprog[g]: owned chunks < count have their ring image complete
//   rprog[g]: chunks < count have been copied out of the ring by workgroup g
//   pprog[g]: partial outputs of chunks < count written by workgroup g
//   dprog[g]: reductions of chunks < count done by workgroup g (its partial-ring reads)
constexpr int PART_BLOCK = 2048;              // one row block of one partial: 2 x 16x16 fp32
constexpr int PART_SLOT = NG * NG * PART_BLOCK;  // [dest row block][writer]

constexpr int DUMMY_BYTES = 16384;  // per workgroup: where stores of no chunk go
struct Layout {
  size_t ctrl, ring, part, dummy, total;
};
__host__ __device__ inline Layout layout(int BH) {
  Layout l;
  l.ctrl = 256;
  l.ring = (l.ctrl + static_cast<size_t>(BH) * CTR_WORDS * 8 + 1023) & ~static_cast<size_t>(1023);
  l.part = l.ring + static_cast<size_t>(BH) * NR * IMG_BYTES;
  l.dummy = l.part + static_cast<size_t>(BH) * NP * PART_SLOT;
  l.total = l.dummy + static_cast<size_t>(BH) * NG * DUMMY_BYTES;
  return l;
}

struct PScratch {
  float gram[R * T_LD];
  float4 mcoef[C];
  float drow[4][64];
  float dcol[4][64];
  float ocol[64];
  float orow[64];
  float sblk[2][64];
};

struct alignas(16) Smem {
  E cbuf[NB][IMG_BYTES / 2];       // ring images (U, T~) of chunks i-1 .. i+3
  E pst[2][R * PST_LD];            // readout stash: chunk-start state (f16, transposed)
  E zst[2][R * ZST_LD];            // readout stash: Z (f16, transposed)
  uint4 qs[NQ][64];                // q of this workgroup's columns as loaded (token l>>2)
  uint4 kvs[2][8][64];             // k, v of an owned chunk in Gram-operand order
  unsigned ds[2][64];              // delta of an owned chunk (token l & 15; 16-bit: word holding it)
  float4 own[NOWN][2][64];         // the readout's own row block of a chunk's partial output
  float4 pstage[3][6][64];         // the gatherer's copies of the other three partials
  PScratch pscr[2];
  float smax[2];
  int abort_flag;
};

struct Args {
  const void* q;
  const void* k;
  const void* v;
  const void* delta;
  int64_t in_stride;  // elements between tokens of q/k/v
  int64_t dl_stride;  // elements between tokens of delta
  const float* psi0;  // [BH][D][D], null = identity
  void* out;          // [B][T][H][D]
  float* psi_out;     // [BH][D][D]
  unsigned char* ws;  // workspace (layout())
  int T, H, BH, nch;
  unsigned tag;
  unsigned* flags;    // flags[bh] = ftag when a token lies outside the chunk envelope
  unsigned ftag;
};

// ------------------------------------------------------------------ small helpers
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
// s_waitcnt vmcnt(n) alone (expcnt 7 and lgkmcnt 15 mean no wait); n < 64 (bits 3:0, 15:14)
#define XS_VMCNT(n) __builtin_amdgcn_s_waitcnt(0x0F70 | ((n) & 15) | (((n) >> 4) << 14))

// Single 8-byte LDS reads (never fused into read2, which gfx950 serves slower here).
__device__ __forceinline__ V4 ld4(const E* p) {
  typedef __attribute__((address_space(3))) const volatile V4 lds_v4;
  return *((lds_v4*)(p));
}
__device__ __forceinline__ V8 ld4x2(const E* p0, const E* p1) { return cat8<V4, V8>(ld4(p0), ld4(p1)); }
// Transposing LDS read: within each 16-lane group, lane 4i + r addresses row k0 + i, columns
// n0 + 4r .. 4r+3 of a row-major block; lane n of the group receives rows k0 .. k0+3 of column
// n0 + n.
__device__ __forceinline__ V4 tr4(const E* p) {
  typedef short i16x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  return __builtin_bit_cast(V4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p)));
}
__device__ __forceinline__ V8 tr4x2(const E* p0, const E* p1) { return cat8<V4, V8>(tr4(p0), tr4(p1)); }
__device__ __forceinline__ void st4(E* p, V4 x) {
  typedef __attribute__((address_space(3))) volatile V4 lds_v4;
  *((lds_v4*)(p)) = x;
}
__device__ __forceinline__ V8 cvt8(const f32x4& a, const f32x4& b) {
  V8 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    r[i] = static_cast<E>(a[i]);
    r[4 + i] = static_cast<E>(b[i]);
  }
  return r;
}
__device__ __forceinline__ V4 lo4(V8 x) { return __builtin_shufflevector(x, x, 0, 1, 2, 3); }
__device__ __forceinline__ V4 hi4(V8 x) { return __builtin_shufflevector(x, x, 4, 5, 6, 7); }

// Eight 16-bit inputs (one uint4) as f16 (bf16 -> f32 -> f16, round to nearest even).
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

// Direct global -> LDS copies (global_load_lds): lane l's 16 (or 4) bytes land at LDS byte
// address lds + 16 l (4 l), M0 holding lds.  Issued through inline assembly: with the builtin
// (or with M0 in an asm clobber list) the compiler's wait insertion makes every LDS access of
// a wave that has any memory operation outstanding wait for all of them, which stalls the
// readout, reducer and producer waves on their own stores.  The copying waves wait for their
// copies with explicit vmcnt values.  SC1: device scope (misses the CU's L1, as data written
// by other workgroups requires).
__device__ __forceinline__ unsigned lds_addr(const void* p) {
  return static_cast<unsigned>(reinterpret_cast<uintptr_t>(
      (__attribute__((address_space(3))) const char*)(p)));
}
template <bool SC1>
__device__ __forceinline__ void dma16(const void* g, unsigned lds) {
  const unsigned m0v = __builtin_amdgcn_readfirstlane(lds);
  if constexpr (SC1)
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %1, off sc1" :: "{m0}"(m0v), "v"(g) : "memory");
  else
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %1, off" :: "{m0}"(m0v), "v"(g) : "memory");
}
__device__ __forceinline__ void dma4(const void* g, unsigned lds) {
  const unsigned m0v = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_nop 0\n\tglobal_load_lds_dword %1, off" :: "{m0}"(m0v), "v"(g) : "memory");
}

// Device-scope (sc1) counter accesses: they miss the CU's L1 and meet in the XCD's L2.
__device__ __forceinline__ unsigned long long ld_ctr(const unsigned long long* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_ctr(unsigned long long* p, unsigned long long v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool ctr_ok(unsigned long long v, unsigned tag, int need) {
  return static_cast<unsigned>(v >> 32) == tag && static_cast<int>(static_cast<unsigned>(v)) >= need;
}
__device__ __forceinline__ unsigned long long ctr_val(unsigned tag, int count) {
  return (static_cast<unsigned long long>(tag) << 32) | static_cast<unsigned>(count);
}

constexpr int kMaxPolls = 1 << 19;
// Polls until every lane l < nl has *p_l (its own counter) at tag with count >= need_l.
// Returns false if the call is already marked failed (this workgroup or another) or after
// kMaxPolls polls, in which case it marks the call failed.  Wave-uniform.
__device__ bool poll_ctrs(const unsigned long long* p, int need, bool active, unsigned tag,
                          unsigned long long* err, int* lds_abort) {
  if (__hip_atomic_load(lds_abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) return false;
  for (int it = 0; it < kMaxPolls; ++it) {
    bool ok = true;
    if (active) ok = ctr_ok(ld_ctr(p), tag, need);
    if (__builtin_amdgcn_ballot_w64(!ok) == 0) return true;
    if (static_cast<unsigned>(ld_ctr(err) >> 32) == tag) break;
    __builtin_amdgcn_s_sleep(8);
  }
  st_ctr(err, ctr_val(tag, 1));
  __hip_atomic_store(lds_abort, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  return false;
}

__device__ __forceinline__ float dot8(const float* x, const float* y) {
  const float4 x0 = *reinterpret_cast<const float4*>(x);
  const float4 x1 = *reinterpret_cast<const float4*>(x + 4);
  const float4 y0 = *reinterpret_cast<const float4*>(y);
  const float4 y1 = *reinterpret_cast<const float4*>(y + 4);
  float s = x0.x * y0.x;
  s = fmaf(x0.y, y0.y, s); s = fmaf(x0.z, y0.z, s); s = fmaf(x0.w, y0.w, s);
  s = fmaf(x1.x, y1.x, s); s = fmaf(x1.y, y1.y, s); s = fmaf(x1.z, y1.z, s);
  return fmaf(x1.w, y1.w, s);
}

// ------------------------------------------------------------------ the kernel
template <typename IO, typename DT>
__global__ __launch_bounds__(NT) void sssd_xsplit_kernel(Args a) {
  __shared__ Smem sm;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int l16 = lane & 15, g4 = lane >> 4;
  const int l32 = lane & 31, g2 = lane >> 5;

  // workgroup -> (sequence, column group): workgroups x, x+8, x+16, x+24 (same x mod 8)
  // form a group; dispatch places consecutive workgroups on consecutive XCDs
  const int wg = blockIdx.x;
  const int m = wg >> 3;
  const int bh = (m >> 2) * 8 + (wg & 7);
  const int g = m & 3;
  if (bh >= a.BH) return;  // padding of the grid to whole groups per XCD
  const int b = bh / a.H, h = bh - b * a.H;
  const int N = a.nch;
  const unsigned tag = a.tag;
  const Layout L = layout(a.BH);
  unsigned long long* const err = reinterpret_cast<unsigned long long*>(a.ws);
  unsigned long long* const ctr = reinterpret_cast<unsigned long long*>(a.ws + L.ctrl) + bh * CTR_WORDS;
  unsigned char* const ring = a.ws + L.ring + static_cast<size_t>(bh) * NR * IMG_BYTES;
  unsigned char* const part = a.ws + L.part + static_cast<size_t>(bh) * NP * PART_SLOT;
  const int64_t DD = static_cast<int64_t>(D) * D;

  if (tid == 0) sm.abort_flag = 0;
  // Group check: every member must run on the same XCD (they share data through its L2).
  if (wave == 0) {
    const unsigned xcc = __builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & 0xf;  // HW_REG_XCC_ID
    if (lane == 0) st_ctr(ctr + CTR_HELLO + g, ctr_val(tag, static_cast<int>(xcc) + 1));
    bool same = true;
    int it = 0;
    for (; it < kMaxPolls; ++it) {
      bool ok = true;
      if (lane < NG) {
        const unsigned long long v = ld_ctr(ctr + CTR_HELLO + lane);
        ok = static_cast<unsigned>(v >> 32) == tag;
        if (ok && static_cast<int>(static_cast<unsigned>(v)) != static_cast<int>(xcc) + 1) same = false;
      }
      if (__builtin_amdgcn_ballot_w64(!ok) == 0) break;
      __builtin_amdgcn_s_sleep(8);
    }
    const bool bad = it == kMaxPolls || __builtin_amdgcn_ballot_w64(!same) != 0;
    if (bad) {
      if (lane == 0) {
        st_ctr(err, ctr_val(tag, 2));
        sm.abort_flag = 1;
      }
    }
  }

  // chain waves: start slab (16 columns each) and its largest magnitude
  f32x4 psi[8];
  const int jl = 16 * wave + l16;  // chain waves: column within the workgroup
  const int jc = GC * g + jl;
  if (wave < 2) {
    if (a.psi0) {
      const float* src = a.psi0 + bh * DD + jc;
#pragma unroll
      for (int t = 0; t < 8; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) psi[t][r] = src[(16 * t + 4 * g4 + r) * D];
    } else {
#pragma unroll
      for (int t = 0; t < 8; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) psi[t][r] = (16 * t + 4 * g4 + r) == jc ? 1.f : 0.f;
    }
    float mx = 0.f;
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) mx = fmaxf(mx, fabsf(psi[t][r]));
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    if (lane == 0) sm.smax[wave] = mx;
  }
  __syncthreads();
  // The state enters the MFMAs as f16, so it is carried scaled by a power of two that puts
  // the largest start entry of this workgroup's columns in [1, 2); orthogonal updates keep
  // every column's norm, so no entry leaves the f16 range.  Outputs and the end state are
  // multiplied back by 1/s (each workgroup its own s: the partial outputs are unscaled
  // before the group adds them).
  float sc = 1.f, inv_s = 1.f;
  {
    const float mx = fmaxf(sm.smax[0], sm.smax[1]);
    if (mx > 0.f && mx <= 3.0e38f) {
      int e;
      (void)frexpf(mx, &e);
      sc = ldexpf(1.f, 1 - e);
      inv_s = ldexpf(1.f, e - 1);
    }
  }
  const int IEND = N + LRD + 1;  // the reducer consumes chunk N-1 in iteration N-1 + LRD + 2

  // ================================================================ chain waves
  if (wave < 2) {
#pragma unroll
    for (int t = 0; t < 8; ++t) psi[t] *= sc;
    const int offW = rho_slot(l16) * U_LD + 4 * g4;                      // + mt * U_LD (rho + 16)
    const int offT = IMG_TH + l16 * TT_LD + 4 * g4;                        // + 16 mt TT_LD
    const int offU = rho_slot(4 * g4 + (l16 >> 2)) * U_LD + 4 * (l16 & 3);  // + 16 t; + U_LD (rho + 16)
    const int offS = jsig(jl) * PST_LD + 4 * g4;
    const int offZ = jsig(jl) * ZST_LD + 4 * g4;
    for (int i = I0; i <= IEND; ++i) {
      if (i >= 0 && i < N) {
        const E* img = sm.cbuf[i % NB];
        V8 wa[2][4], th[2], tl[2], ut[8];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) {
            const E* p = img + offW + mt * U_LD + 32 * ks;
            wa[mt][ks] = ld4x2(p, p + 16);
          }
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          const E* p = img + offT + 16 * mt * TT_LD;
          th[mt] = ld4x2(p, p + 16);
          tl[mt] = ld4x2(p + (IMG_TL - IMG_TH), p + (IMG_TL - IMG_TH) + 16);
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const E* p = img + offU + 16 * t;
          ut[t] = tr4x2(p, p + U_LD);
        }
        // state as f16 (B operand: k-slots d = 32ks + 4g4 + s, 32ks + 16 + 4g4 + s) and stash
        V8 pb[4];
        E* const ps = sm.pst[i & 1] + offS;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          pb[ks] = cvt8(psi[2 * ks], psi[2 * ks + 1]);
          st4(ps + 32 * ks, lo4(pb[ks]));
          st4(ps + 32 * ks + 16, hi4(pb[ks]));
        }
        f32x4 W[2] = {};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
          for (int mt = 0; mt < 2; ++mt) W[mt] = MM::mma16(wa[mt][ks], pb[ks], W[mt]);
        const V8 wb = cvt8(W[0], W[1]);
        f32x4 Z[2];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          Z[mt] = MM::mma16(th[mt], wb, f32x4{});
          Z[mt] = MM::mma16(tl[mt], wb, Z[mt]);
        }
        const V8 zb = cvt8(Z[0], Z[1]);
        E* const zs = sm.zst[i & 1] + offZ;
        st4(zs, lo4(zb));
        st4(zs + 16, hi4(zb));
#pragma unroll
        for (int t = 0; t < 8; ++t) psi[t] = MM::mma16(ut[t], zb, psi[t]);
      }
      lds_barrier();
    }
    const float fin = sm.abort_flag ? __builtin_nanf("") : inv_s;
    float* dst = a.psi_out + bh * DD + jc;
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) dst[(16 * t + 4 * g4 + r) * D] = psi[t][r] * fin;
    return;
  }

  const int64_t tok_base = static_cast<int64_t>(b) * a.T * a.in_stride + static_cast<int64_t>(h) * D;
  const int64_t dl_base = static_cast<int64_t>(b) * a.T * a.dl_stride + h;
  unsigned char* const dummy = a.ws + L.dummy + static_cast<size_t>(bh * NG + g) * DUMMY_BYTES;

  // Memory waves issue the same operations in every iteration (operations that belong to no
  // chunk go to clamped sources, unused LDS slots or this workgroup's dummy area), so fixed
  // vmcnt values wait for exactly the operations meant.
  // ================================================================ readout wave
  if (wave == 2) {
    // per iteration: 6 partial stores, pprog store
    const int offP = jsig(4 * g4 + (l16 >> 2)) * PST_LD + 4 * (l16 & 3);  // + 16 tl; + 16 PST_LD
    const int offZ = jsig(4 * g4 + (l16 >> 2)) * ZST_LD + 4 * (l16 & 3);  // + 16 mt; + 16 ZST_LD
    const int offU = rho_slot(4 * g4 + (l16 >> 2)) * U_LD + 4 * (l16 & 3);  // + 16 tl; + U_LD
    // q B operand: token l16, features 4g4 + 0..3 and 16 + 4g4 + 0..3 of this workgroup's
    // 32 columns, in a qs slot at byte 64 t + 2 f
    const int offQ = 64 * l16 + 8 * g4;
    for (int i = I0; i <= IEND; ++i) {
      const int c = i - 1;  // chunk read out in this iteration
      const bool live = c >= 0 && c < N;
      // (the poller has checked, before the barrier that ended iteration i-1, that slot
      // c mod NP is free: the other three workgroups have reduced chunk c - NP)
      float4 o4[8];
      if (live) {
        const E* img = sm.cbuf[c % NB];
        const E* pst = sm.pst[c & 1];
        const E* zst = sm.zst[c & 1];
        const unsigned char* qsl = reinterpret_cast<const unsigned char*>(&sm.qs[c % NQ][0]);
        typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 qa = *reinterpret_cast<const u32x2*>(qsl + offQ);
        const u32x2 qb2 = *reinterpret_cast<const u32x2*>(qsl + offQ + 32);
        const uint4 qf = to_f16x8<IO>(make_uint4(qa.x, qa.y, qb2.x, qb2.y));
        const V8 bq = __builtin_bit_cast(V8, qf);
        f32x4 O[8], Y[2];
#pragma unroll
        for (int tl = 0; tl < 8; ++tl) {
          const E* p = pst + offP + 16 * tl;
          O[tl] = MM::mma16(tr4x2(p, p + 16 * PST_LD), bq, f32x4{});
        }
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          const E* p = zst + offZ + 16 * mt;
          Y[mt] = MM::mma16(tr4x2(p, p + 16 * ZST_LD), bq, f32x4{});
        }
        // Y lane (t = l16, g4) holds rho = 16mt + 4g4 + r: the B operand of U mask(Y)
        V8 by;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          by[r] = static_cast<E>(((4 * g4 + r) >> 1) <= l16 ? Y[0][r] : 0.f);
          by[4 + r] = static_cast<E>(((16 + 4 * g4 + r) >> 1) <= l16 ? Y[1][r] : 0.f);
        }
#pragma unroll
        for (int tl = 0; tl < 8; ++tl) {
          const E* p = img + offU + 16 * tl;
          O[tl] = MM::mma16(tr4x2(p, p + U_LD), by, O[tl]);
        }
#pragma unroll
        for (int tl = 0; tl < 8; ++tl) {
          const f32x4 o = O[tl] * inv_s;
          o4[tl] = make_float4(o[0], o[1], o[2], o[3]);
        }
      } else {
#pragma unroll
        for (int tl = 0; tl < 8; ++tl) o4[tl] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
      // own row block (rows 32g ..) to LDS, the other three to slot c mod NP, block
      // [dest rb][writer g].  One code path per g (uniform branch), so the row blocks are
      // compile-time indexes and every path issues the same six stores.
      unsigned char* const slot = live ? part + (c % NP) * PART_SLOT + g * PART_BLOCK + 32 * lane
                                       : dummy + 32 * lane;
#define XS_PUT(G)                                                                                \
  {                                                                                              \
    if (live) {                                                                                  \
      sm.own[c % NOWN][0][lane] = o4[2 * (G)];                                                   \
      sm.own[c % NOWN][1][lane] = o4[2 * (G) + 1];                                               \
    }                                                                                            \
    _Pragma("unroll") for (int rb = 0; rb < NG; ++rb) {                                          \
      if (rb == (G)) continue;                                                                   \
      const int k = rb - (rb > (G) ? 1 : 0);                                                     \
      float4* dst = reinterpret_cast<float4*>(slot + (live ? rb * NG * PART_BLOCK : k * PART_BLOCK)); \
      dst[0] = o4[2 * rb];                                                                       \
      dst[1] = o4[2 * rb + 1];                                                                   \
    }                                                                                            \
  }
      if (g == 0) XS_PUT(0)
      else if (g == 1) XS_PUT(1)
      else if (g == 2) XS_PUT(2)
      else XS_PUT(3)
#undef XS_PUT
      XS_VMCNT(7);  // the partial stores of iteration i-1 (chunk i-2) are complete
      st_ctr(ctr + CTR_P + g, ctr_val(tag, max(i - 1, 0)));  // chunks <= i-2 (all lanes)
      lds_barrier();
    }
    return;
  }

  // ================================================================ reducer wave
  if (wave == 5) {
    // Reducer: per iteration 2 output stores; reads only LDS (own block, the gatherer's
    // copies).  Poller: one load of the group's 16 counters per iteration (lane 4w + k:
    // counter k of workgroup w), checked before the barrier for every hand-off iteration
    // i+1 depends on, polling a counter that is behind.  No other wave loads a counter.
    IO* const gout = static_cast<IO*>(a.out);
    const int64_t out_row = static_cast<int64_t>(a.H) * D;
    const int cw = (lane >> 2) & 3, ck = lane & 3;  // ck: 0 tprog, 1 rprog, 2 pprog, 3 dprog
    const unsigned long long* const cptr = ctr + CTR_T + 4 * ck + cw;
    for (int i = I0; i <= IEND; ++i) {
      const unsigned long long cv = ld_ctr(cptr);
      const int cb = i - 2 - LRD;  // copied in iteration cb + LRD, complete at the barrier ending cb + LRD + 1
      const bool live = cb >= 0 && cb < N;
      float4 s[2];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        // fixed order over the four workgroups' partials (own block in its place)
        const float4 own = live ? sm.own[cb % NOWN][tt][lane] : make_float4(0.f, 0.f, 0.f, 0.f);
        const int sl = ((cb % 3) + 3) % 3;
        s[tt] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int w = 0; w < NG; ++w) {
          float4 x;
          if (w < NG - 1) {
            // staged block k = w - (w > g) holds writer w (w != g)
            const float4 st = sm.pstage[sl][2 * (w - (w > g ? 1 : 0)) + tt][lane];
            x = w == g ? own : st;
          } else {
            x = w == g ? own : sm.pstage[sl][2 * (NG - 2) + tt][lane];
          }
          s[tt].x += x.x; s[tt].y += x.y; s[tt].z += x.z; s[tt].w += x.w;
        }
      }
      const bool bad = sm.abort_flag != 0;
      const int t = cb * C + l16;
      const bool st_ok = live && t < a.T;
      IO* dst = st_ok ? gout + (static_cast<int64_t>(b) * a.T + t) * out_row + static_cast<int64_t>(h) * D +
                            GC * g + 4 * g4
                      : reinterpret_cast<IO*>(dummy + 16 * lane);
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        typedef IO io4 __attribute__((ext_vector_type(4)));
        io4 o;
        const float qn = __builtin_nanf("");
        o[0] = static_cast<IO>(bad ? qn : s[tt].x);
        o[1] = static_cast<IO>(bad ? qn : s[tt].y);
        o[2] = static_cast<IO>(bad ? qn : s[tt].z);
        o[3] = static_cast<IO>(bad ? qn : s[tt].w);
        *reinterpret_cast<io4*>(dst + (st_ok ? 16 * tt : 4 * tt)) = o;
      }
      // conditions of iteration i+1 (need <= 0: none)
      int need = 0;
      if (lane < 16) {
        if (ck == 0) {  // ring loader copies chunk nl: its owner has published it
          const int nl = i + 1 + LDA;
          if (nl >= 0 && nl < N && cw == (nl & 3)) need = nl + 1;
        } else if (ck == 1) {  // producer phase 3 of chunk nA: ring slot free in every workgroup
          const int pa = (i + 1 + LP - g + 64) & 3;
          const int nA = i + 1 + LP - pa;
          if (pa == 3 && nA >= 0 && nA < N) need = nA - NR + 1;
        } else if (ck == 2) {  // gatherer copies chunk ca: the other three have written it
          const int ca = i + 1 - LRD;
          if (ca >= 0 && ca < N && cw != g) need = ca + 1;
        } else {  // readout writes chunk c = i: the other three have reduced chunk c - NP
          if (i >= 0 && i < N && cw != g) need = i - NP + 1;
        }
      }
      XS_VMCNT(2);  // the counter load (the two output stores may remain in flight)
      const bool ok = need <= 0 || ctr_ok(cv, tag, need);
      if (__builtin_amdgcn_ballot_w64(!ok) != 0) poll_ctrs(cptr, need, need > 0, tag, err, &sm.abort_flag);
      lds_barrier();
    }
    return;
  }

  // ================================================================ gatherer wave
  if (wave == 7) {
    // per iteration: dprog store, 6 direct loads of partials (no loads into registers)
    for (int i = I0; i <= IEND; ++i) {
      XS_VMCNT(0);  // the copies of iteration i-1
      // the copies of chunk i-1-LRD (issued in iteration i-1) are complete: that slot of the
      // partial ring may be reused
      st_ctr(ctr + CTR_D + g, ctr_val(tag, max(i - LRD, 0)));  // chunks <= i-1-LRD (all lanes)
      // partials of chunk ca = i - LRD (the poller has checked that they are published)
      const int ca = i - LRD;
      const bool lca = ca >= 0 && ca < N;
      const int cs = lca ? ca : 0;
      const unsigned char* src = part + (cs % NP) * PART_SLOT + g * NG * PART_BLOCK + 32 * lane;
      const unsigned dst = lds_addr(&sm.pstage[((ca % 3) + 3) % 3][0][0]);
#pragma unroll
      for (int k = 0; k < NG - 1; ++k) {
        const int w = k + (k >= g ? 1 : 0);
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
          dma16<true>(src + w * PART_BLOCK + 16 * tt, dst + (2 * k + tt) * 1024);
      }
      lds_barrier();
    }
    return;
  }

  // ================================================================ ring loader wave
  if (wave == 4) {
    // per iteration: rprog store, IMG_DMAS direct loads of the ring image of chunk i + LDA
    const unsigned char* const src0 = ring + lane * 16;
    for (int i = I0; i <= IEND; ++i) {
      const int n = i + LDA;
      XS_VMCNT(IMG_DMAS + 1);  // the copy of chunk i+1 (issued in iteration i-2) is complete
      st_ctr(ctr + CTR_R + g, ctr_val(tag, max(i + 2, 0)));  // chunks <= i+1 in LDS (all lanes)
      const int ns = min(max(n, 0), N - 1);
      const unsigned char* src = src0 + (ns % NR) * IMG_BYTES;
      const unsigned dst = lds_addr(&sm.cbuf[((n % NB) + NB) % NB][0]);
#pragma unroll
      for (int kk = 0; kk < IMG_DMAS; ++kk) dma16<true>(src + kk * 1024, dst + kk * 1024);
      lds_barrier();
    }
    return;
  }

  // ================================================================ input loader wave
  if (wave == 6) {
    // per iteration: the q of chunk i + LQ (one direct load); in every fourth iteration also
    // k, v (8) and delta (1) of the owned chunk n = i + LP + LK, whose phase 0 runs in
    // iteration n - LP.  A wait at the start of iteration i for the operations of iteration
    // i-3 gives every copy three iterations.
    const IO* gq = static_cast<const IO*>(a.q);
    const IO* gk = static_cast<const IO*>(a.k);
    const IO* gv = static_cast<const IO*>(a.v);
    const int qt = lane >> 2, qp = lane & 3;
    const IO* const qsrc = gq + tok_base + GC * g + 8 * qp;
    // Gram-operand order: rank row rho = l32 (token rho >> 1, k or v), features 16ks + 8g2 + 0..7
    const IO* const kvsrc = ((l32 & 1) ? gv : gk) + tok_base + 8 * g2;
    const bool d16 = sizeof(DT) == 2;
    const unsigned char* const dsrc = static_cast<const unsigned char*>(a.delta);
    const int rk = (g - LP - LK + 64) & 3;  // iterations i = rk mod 4 copy k, v, delta
    auto ops = [&](int it) { return it < I0 ? 0 : (((it - rk + 64) & 3) == 0 ? 10 : 1); };
    for (int i = I0; i <= IEND; ++i) {
      const int wait = ops(i - 1) + ops(i - 2);
      if (wait == 2) XS_VMCNT(2);
      else if (wait == 11) XS_VMCNT(11);
      else if (wait == 1) XS_VMCNT(1);
      else if (wait == 10) XS_VMCNT(10);
      {
        const int nq = i + LQ;
        const int t = min(max(nq * C + qt, 0), a.T - 1);
        dma16<false>(qsrc + static_cast<int64_t>(t) * a.in_stride, lds_addr(&sm.qs[((nq % NQ) + NQ) % NQ][0]));
      }
      if (((i - rk + 64) & 3) == 0) {
        const int n = i + LP + LK;
        const int nc = min(max(n, 0), N - 1);
        const int tk = min(nc * C + (l32 >> 1), a.T - 1);
        const IO* src = kvsrc + static_cast<int64_t>(tk) * a.in_stride;
        const unsigned dst = lds_addr(&sm.kvs[(n >> 2) & 1][0][0]);
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) dma16<false>(src + 16 * ks, dst + ks * 1024);
        const int td = min(nc * C + l16, a.T - 1);
        const int64_t el = dl_base + static_cast<int64_t>(td) * a.dl_stride;
        // 16-bit delta: the aligned word holding it (an even head count keeps that word in
        // bounds); fp32: the element
        const unsigned char* dp = d16 ? dsrc + ((2 * el) & ~static_cast<int64_t>(3)) : dsrc + 4 * el;
        dma4(dp, lds_addr(&sm.ds[(n >> 2) & 1][0]));
      }
      lds_barrier();
    }
    return;
  }

  // ================================================================ producer wave (3)
  {
    struct Regs {
      uint4 kv[8];
      float d;
      f32x16 gacc;
    };
    Regs ra;                    // the chunk in phases 0-3
    float tv[6], cv[4];         // the chunk in phases 4-7
    const int ea = lane >> 3, eb = lane & 7;
    const bool dhi = sizeof(DT) == 2 && ((dl_base * 2) & 2);  // 16-bit delta in the word's upper half

    // phase 0: k, v rows (copied by the input loader) as f16 (zero past the end), delta, and the
    // Gram matrix on the MFMA
    auto p_gram = [&](int n) {
      const int sl = (n >> 2) & 1;
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) ra.kv[ks] = to_f16x8<IO>(sm.kvs[sl][ks][lane]);
      {
        const unsigned w = sm.ds[sl][l16];
        if constexpr (sizeof(DT) == 2) {
          const unsigned short hb = static_cast<unsigned short>(dhi ? (w >> 16) : (w & 0xffffu));
          DT dv;
          __builtin_memcpy(&dv, &hb, 2);
          ra.d = io<DT>::to_f32(dv);
        } else {
          ra.d = __uint_as_float(w);
        }
      }
      if (n * C + C > a.T && n * C + (l32 >> 1) >= a.T) {
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) ra.kv[ks] = make_uint4(0, 0, 0, 0);
      }
      f32x16 acc = {};
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        const V8 x = __builtin_bit_cast(V8, ra.kv[ks]);
        acc = MM::mma32(x, x, acc);
      }
      ra.gacc = acc;
    };
    // phase 1: Gram to scratch, Cayley blocks with the reference's non-finite guard
    auto p_cayley = [&](int n, PScratch& P) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4)
        *reinterpret_cast<float4*>(&P.gram[l32 * T_LD + 8 * q4 + 4 * g2]) =
            make_float4(ra.gacc[4 * q4], ra.gacc[4 * q4 + 1], ra.gacc[4 * q4 + 2], ra.gacc[4 * q4 + 3]);
      wave_sync();
      bool ok = true, wide = false;
      if (lane < C) {
        const int t = lane;
        const float kk = P.gram[(2 * t) * T_LD + 2 * t];
        const float vv = P.gram[(2 * t + 1) * T_LD + 2 * t + 1];
        const float kv = P.gram[(2 * t) * T_LD + 2 * t + 1];
        const float dl = n * C + t >= a.T ? 0.f : ra.d;
        const cayley2 M = cayley_guarded(dl, kk, vv, kv, ok);
        P.mcoef[t] = make_float4(M.m00, M.m01, M.m10, M.m11);
        wide = !ok || rotation_outside_chunk_envelope(dl, kk, vv, kv);  // as the segment scan
      }
      // hand the sequence to the fp32 recompute (a plain store: every writer stores the tag)
      if (__builtin_amdgcn_ballot_w64(wide) != 0 && lane == 0) a.flags[bh] = a.ftag;
      // a token whose factor is not finite acts as R = I: its rows are zeroed and the Gram
      // matrix recomputed (uniform branch, taken only for such chunks)
      const unsigned long long badm = __builtin_amdgcn_ballot_w64(!ok);
      if (badm != 0) {
        if ((badm >> (l32 >> 1)) & 1) {
#pragma unroll
          for (int ks = 0; ks < 8; ++ks) ra.kv[ks] = make_uint4(0, 0, 0, 0);
        }
        f32x16 z = {};
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
          const V8 x = __builtin_bit_cast(V8, ra.kv[ks]);
          z = MM::mma32(x, x, z);
        }
        wave_sync();
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4)
          *reinterpret_cast<float4*>(&P.gram[l32 * T_LD + 8 * q4 + 4 * g2]) =
              make_float4(z[4 * q4], z[4 * q4 + 1], z[4 * q4 + 2], z[4 * q4 + 3]);
      }
      wave_sync();
    };
    // phase 2: diagonal 8x8 blocks of T~ by forward substitution, lane = (block gb, column c)
    auto p_diag = [&](PScratch& P) {
      if (lane < 32) {
        const int gb = lane >> 3, c = lane & 7;
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
          for (int ii = 0; ii < 2 * t2; ++ii) {
            s0 = fmaf(gblk[2 * t2][ii], x[ii], s0);
            s1 = fmaf(gblk[2 * t2 + 1][ii], x[ii], s1);
          }
          const float4 Mc = P.mcoef[4 * gb + t2];
          const float e0 = (c == 2 * t2 ? 1.f : 0.f) + s0;
          const float e1 = (c == 2 * t2 + 1 ? 1.f : 0.f) + s1;
          x[2 * t2] = fmaf(Mc.x, e0, Mc.y * e1);
          x[2 * t2 + 1] = fmaf(Mc.z, e0, Mc.w * e1);
        }
        *reinterpret_cast<float4*>(&P.dcol[gb][c * 8]) = make_float4(x[0], x[1], x[2], x[3]);
        *reinterpret_cast<float4*>(&P.dcol[gb][c * 8 + 4]) = make_float4(x[4], x[5], x[6], x[7]);
#pragma unroll
        for (int ii = 0; ii < 8; ++ii) P.drow[gb][ii * 8 + c] = x[ii];
      }
    };
    // phase 3: U rows to the ring (the poller has checked that every workgroup has copied the
    // slot's previous chunk out)
    auto p_urows = [&](int n) {
      unsigned char* img = (n >= 0 && n < N) ? ring + (n % NR) * IMG_BYTES : dummy;
      typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
      u32x2* dst = reinterpret_cast<u32x2*>(img + 2 * (rho_slot(l32) * U_LD + 8 * g2));
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        dst[4 * ks] = u32x2{ra.kv[ks].x, ra.kv[ks].y};  // features 16ks + 8g2 + 0..3
        dst[4 * ks + 1] = u32x2{ra.kv[ks].z, ra.kv[ks].w};
      }
    };
    // Off-diagonal blocks (see sssd_chunk.hip): T~_10 = T~_11 G_10 T~_00 and T~_32 likewise
    // (VALU through LDS), then T~[16:32, 0:16] = B G[16:32, 0:16] A on the fp32 MFMA.
    auto od_1a = [&](PScratch& P) {
      const float* gg1 = &P.gram[(8 + ea) * T_LD];
      const float* gg3 = &P.gram[(24 + ea) * T_LD];
#pragma unroll
      for (int gb = 0; gb < 4; ++gb) tv[gb] = P.drow[gb][ea * 8 + eb];
      P.sblk[0][eb * 8 + ea] = dot8(gg1, &P.dcol[0][eb * 8]);
      P.sblk[1][eb * 8 + ea] = dot8(gg3 + 16, &P.dcol[2][eb * 8]);
    };
    auto od_1b = [&](PScratch& P) {
      tv[4] = dot8(&P.drow[1][ea * 8], &P.sblk[0][eb * 8]);
      tv[5] = dot8(&P.drow[3][ea * 8], &P.sblk[1][eb * 8]);
      P.ocol[eb * 8 + ea] = tv[4];
      P.orow[ea * 8 + eb] = tv[5];
    };
    auto od_c = [&](PScratch& P) {
      const int kg = g4;
      const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
      const f32x4 ga = *reinterpret_cast<const f32x4*>(&P.gram[(16 + l16) * T_LD + 4 * kg]);
      const float* bs = kg < 2 ? &P.dcol[0][(l16 & 7) * 8 + 4 * kg]
                               : (l16 < 8 ? &P.ocol[l16 * 8 + 4 * (kg - 2)]
                                          : &P.dcol[1][(l16 - 8) * 8 + 4 * (kg - 2)]);
      f32x4 bx = *reinterpret_cast<const f32x4*>(bs);
      if (kg < 2 && l16 >= 8) bx = z4;
      f32x4 X = z4;
#pragma unroll
      for (int si = 0; si < 4; ++si) X = __builtin_amdgcn_mfma_f32_16x16x4f32(ga[si], bx[si], X, 0, 0, 0);
      const float* as = l16 < 8 ? &P.drow[2][l16 * 8 + 4 * (kg & 1)]
                                : (kg < 2 ? &P.orow[(l16 - 8) * 8 + 4 * kg]
                                          : &P.drow[3][(l16 - 8) * 8 + 4 * (kg - 2)]);
      f32x4 ax = *reinterpret_cast<const f32x4*>(as);
      if (l16 < 8 && kg >= 2) ax = z4;
      f32x4 Cc = z4;
#pragma unroll
      for (int si = 0; si < 4; ++si) Cc = __builtin_amdgcn_mfma_f32_16x16x4f32(ax[si], X[si], Cc, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r) cv[r] = Cc[r];
    };
    // phase 7: T~ as f16 hi + lo into the ring image (lane pairs write 32-bit words: the even
    // lane the two hi parts, the odd lane the two lo parts) and the zero upper blocks
    auto p_tt = [&](int n) {
      unsigned char* img = (n >= 0 && n < N) ? ring + (n % NR) * IMG_BYTES : dummy;
      const bool odd = lane & 1;
      uint32_t* const tw = reinterpret_cast<uint32_t*>(img + 2 * (odd ? IMG_TL : IMG_TH));
      auto put_pair = [&](float x, int row, int col_even) {
        const E hp = static_cast<E>(x);
        const E lp = static_cast<E>(x - static_cast<float>(hp));
        const uint32_t hb = __builtin_bit_cast(uint16_t, hp), lb = __builtin_bit_cast(uint16_t, lp);
        const uint32_t recv = static_cast<uint32_t>(
            __builtin_amdgcn_mov_dpp(static_cast<int>(odd ? hb : lb), 0xB1, 0xF, 0xF, false));
        const uint32_t word = odd ? (recv | (lb << 16)) : (hb | (recv << 16));
        tw[(row * TT_LD + col_even) >> 1] = word;
      };
      const int brow[6] = {0, 1, 2, 3, 1, 3};
      const int bcol[6] = {0, 1, 2, 3, 0, 2};
#pragma unroll
      for (int ii = 0; ii < 6; ++ii) put_pair(tv[ii], 8 * brow[ii] + ea, 8 * bcol[ii] + (eb & ~1));
#pragma unroll
      for (int r = 0; r < 4; ++r) put_pair(cv[r], 16 + 4 * g4 + r, l16 & ~1);
      // upper blocks (a, b), b > a: 6 blocks x 8 rows x 4 words, hi and lo
      uint32_t* const th = reinterpret_cast<uint32_t*>(img + 2 * IMG_TH);
      uint32_t* const tlw = reinterpret_cast<uint32_t*>(img + 2 * IMG_TL);
      const int ubr[6] = {0, 0, 0, 1, 1, 2};
      const int ubc[6] = {1, 2, 3, 2, 3, 3};
#pragma unroll
      for (int kk = 0; kk < 3; ++kk) {
        const int w = lane + 64 * kk;  // 0 .. 191
        const int blk = w >> 5, row = (w >> 2) & 7, wd = w & 3;
        const int off = ((8 * ubr[blk] + row) * TT_LD + 8 * ubc[blk] + 2 * wd) >> 1;
        th[off] = 0u;
        tlw[off] = 0u;
      }
    };

    // chunk nA runs phases pa = 0..3 while chunk nB = nA - 4 runs phases pa + 4
    for (int i = I0; i <= IEND; ++i) {
      const int pa = (i + LP - g + 64) & 3;
      const int nA = i + LP - pa;
      const int nB = nA - 4;
      // Both chunks' work is issued without a validity branch (one basic block per phase, so the
      // two chains interleave); a chunk outside 0 .. N-1 works on its own scratch slot (the two
      // chunks in flight always use different ones) and stores into the dummy area.
      PScratch& PA = sm.pscr[(nA >> 2) & 1];
      PScratch& PB = sm.pscr[(nB >> 2) & 1];
      if (pa == 0) {
        p_gram(nA);
        od_1a(PB);
      } else if (pa == 1) {
        XS_VMCNT(0);  // the ring stores of chunk nA - 8 (phase 7 two iterations ago)
        if (nA - 8 >= 0 && nA - 8 < N) st_ctr(ctr + CTR_T + g, ctr_val(tag, nA - 8 + 1));
        p_cayley(nA, PA);
        od_1b(PB);
      } else if (pa == 2) {
        p_diag(PA);
        od_c(PB);
      } else {
        p_urows(nA);
        p_tt(nB);
      }
      lds_barrier();
    }
  }
}

}  // namespace xs

// ------------------------------------------------------------------ host side
namespace {

constexpr int kMaxDev = 64;
std::atomic<int> g_coop[kMaxDev];         // 0 unknown, 1 yes, -1 no
std::atomic<unsigned> g_tag{0x5eed0000u};

bool coop_supported() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return false;
  int c = g_coop[dev].load(std::memory_order_relaxed);
  if (c == 0) {
    int attr = 0;
    if (hipDeviceGetAttribute(&attr, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess) attr = 0;
    c = attr ? 1 : -1;
    g_coop[dev].store(c, std::memory_order_relaxed);
  }
  return c > 0;
}

int grid_for(int BH) { return 8 * ((BH + 7) / 8) * xs::NG; }

}  // namespace

// Opt-in (VMI_XSPLIT=1): measured on MI355X at B8 T4096 H8 this pass takes ~0.50 ms against
// ~0.18 ms for the segment plan of sssd_chunk.hip (its hand-offs wait on ~2000-cycle L2 round
// trips and each chunk's chain is LDS-bound at ~1100 cycles).  When enabled it needs the group
// to fill at least half of the device, enough chunks to amortise the pipeline's fill
// (N + 24 iterations for N chunks) and an even head count (16-bit delta is copied as the
// aligned 32-bit word holding it).
bool use_xsplit(int64_t B, int64_t T, int64_t H, int64_t D, int io_dtype) {
  if (D != xs::D || (io_dtype != VMI_BF16 && io_dtype != VMI_F16)) return false;
  if (T < 32 * xs::C || H % 2 != 0) return false;
  const char* env = getenv("VMI_XSPLIT");
  if (!env || env[0] != '1') return false;
  int cus = 0;
  if (device_cu_count(&cus) != hipSuccess) return false;
  const int64_t BH = B * H;
  const int64_t grid = grid_for(static_cast<int>(BH));
  if (grid > cus || 2 * grid < cus) return false;
  return coop_supported();
}

size_t xsplit_workspace_bytes(int64_t B, int64_t H) {
  return xs::layout(static_cast<int>(B * H)).total;
}

template <typename IO, typename DT>
static hipError_t run_xsplit(const void* q, const void* k, const void* v, const void* delta,
                             const float* psi_in, void* out, float* psi_out, int B, int T, int H,
                             void* workspace, uint32_t* flags, uint32_t ftag, hipStream_t stream) {
  xs::Args a{};
  a.flags = flags;
  a.ftag = ftag;
  a.q = q; a.k = k; a.v = v; a.delta = delta;
  a.in_stride = static_cast<int64_t>(H) * xs::D;
  a.dl_stride = H;
  a.psi0 = psi_in;
  a.out = out;
  a.psi_out = psi_out;
  a.ws = static_cast<unsigned char*>(workspace);
  a.T = T; a.H = H; a.BH = B * H;
  a.nch = (T + xs::C - 1) / xs::C;
  unsigned tag = g_tag.fetch_add(1, std::memory_order_relaxed) + 1;
  if (tag == 0) tag = g_tag.fetch_add(1, std::memory_order_relaxed) + 1;
  a.tag = tag;
  void* args[] = {&a};
  void (*kfn)(xs::Args) = xs::sssd_xsplit_kernel<IO, DT>;
  return hipLaunchCooperativeKernel(reinterpret_cast<const void*>(kfn), dim3(grid_for(a.BH)),
                                    dim3(xs::NT), args, 0, stream);
}

hipError_t launch_sssd_xsplit(const void* q, const void* k, const void* v, const void* delta,
                              int io_dtype, int delta_dtype, const float* psi_in, void* out,
                              float* psi_out, int B, int T, int H, void* workspace,
                              uint32_t* flags, uint32_t ftag, hipStream_t stream) {
#define VMI_RUN(E, DT) \
  return run_xsplit<E, DT>(q, k, v, delta, psi_in, out, psi_out, B, T, H, workspace, flags, ftag, \
                           stream)
  if (io_dtype == VMI_BF16) {
    if (delta_dtype == VMI_F32) VMI_RUN(__bf16, float);
    if (delta_dtype == VMI_BF16) VMI_RUN(__bf16, bf16_t);
    VMI_RUN(__bf16, f16_t);
  }
  if (delta_dtype == VMI_F32) VMI_RUN(_Float16, float);
  if (delta_dtype == VMI_BF16) VMI_RUN(_Float16, bf16_t);
  VMI_RUN(_Float16, f16_t);
#undef VMI_RUN
}

}  // namespace vmi
