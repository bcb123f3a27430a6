// Chunk-parallel SSSD prefill scan on bf16/fp16 MFMA, head_dim 128.
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
// Workgroup = 5 waves for one (batch*head, segment):
//   waves 0-3 (consumers) each own a 32-column slab of the fp32 state, held in
//     MFMA accumulators for the whole segment; columns evolve independently, so
//     W, Z and the update need no cross-wave traffic.  The readout is reduced
//     across waves through LDS.
//   waves 4-5 (producers) form a two-stage pipeline ahead of the consumers:
//     role 0 prefetches chunk n+1 into registers and, for chunk n, stages k/v/q
//     in LDS (token-major and feature-major), computes the Gram matrix on MFMA,
//     the Cayley blocks and the diagonal blocks of T~;
//     role 1 computes the off-diagonal blocks of T~ for chunk n-1 and writes the
//     complete T~ (as 16-bit hi + lo) for the consumers.
//   While the consumers process chunk c, role 1 works on c+1 and role 0 on c+2,
//   so no wave waits on another inside an iteration; one LDS barrier per chunk
//   (two with the readout) hands the buffers over.
//
// Long sequences are split into segments processed by independent workgroups:
//   pass A (READOUT=false): each segment s < S-1 from the identity -> its
//          transform P_s (the end state),
//   pass B (sssd_carry_kernel): start_s = P_{s-1} start_{s-1}, column blocks in
//          parallel, bf16x3 MFMA (fp32-faithful),
//   pass C (READOUT=true): every segment from its start state, with outputs.
#include "vmi_common.h"
#include "vmi_dispatch.h"
#include "vmi_mfma.h"

namespace vmi {
namespace chunk {

constexpr int D = 128;
constexpr int C = 16;           // tokens per chunk
constexpr int R = 2 * C;        // rank rows per chunk
constexpr int NCW = 4;          // consumer waves
constexpr int NPW = 2;          // producer waves
constexpr int NT = (NCW + NPW) * 64;
constexpr int TOK_LD = D + 8;   // elements per token-major row (272 B)
constexpr int UT_LD = R + 8;    // elements per feature-major row (80 B)
constexpr int T_LD = R + 4;     // floats per Gram row
constexpr int TT_LD = R + 8;    // elements per T~ hi/lo row (80 B)
constexpr int PS_LD = 32 + 8;   // elements per stash row (80 B)
constexpr int OP_LD = D + 4;    // floats per O-partial row

// Written by producer role 0 for chunk n, read by role 1 one iteration later.
struct Stage0 {
  float gram[R * T_LD];         // Gram matrix G = U^T U (symmetric)
  float4 mcoef[C];              // (m00, m01, m10, m11) per token
  float drow[4][64];            // diagonal 8x8 blocks of T~, row-major [a*8 + c]
  float dcol[4][64];            // the same blocks, column-major [b*8 + c]
};

// Private to producer role 1.
struct Stage1 {
  float ocol[3][64];            // T~_10, T~_21, T~_20, column-major
  float sblk[3][64];            // S = sum_m G_gm T~_mh, column-major
};

template <typename E>
struct Smem {
  E tok[3][3][C * TOK_LD];      // k, v, q of a chunk, token-major (3 chunks in flight)
  E ut[3][D * UT_LD];           // U feature-major: ut[d][rho]
  E tth[2][R * TT_LD];          // T~ = hi + lo (two 16-bit parts), row-major
  E ttl[2][R * TT_LD];
  Stage0 s0[2];
  Stage1 s1;
  E ps[NCW][D * PS_LD];         // per-wave: chunk-start state slab (row-major), then O partial
  E zs[NCW][R * PS_LD];         // per-wave: Z slab (row-major)
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
  int end_mode;         // 0: ends[s*BH + bh] for every segment; 1: ends[bh] for the last one
  int T, H, BH;
  int seg_chunks;       // chunks per segment
  int nseg;             // segments per sequence
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
template <typename E>
__device__ __forceinline__ typename mfma_t<E>::v8 lds4x2(const E* p0, const E* p1) {
  typedef typename mfma_t<E>::v4 V4;
  typedef typename mfma_t<E>::v8 V8;
  return cat8<V4, V8>(lds4<E>(p0), lds4<E>(p1));
}

template <typename E, typename DT, bool READOUT, bool PREC>
__global__ __launch_bounds__(NT) void sssd_chunk_kernel(Args a) {
  typedef mfma_t<E> MM;
  typedef typename MM::v8 V8;
  __shared__ Smem<E> sm;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int l32 = lane & 31, g = lane >> 5;
  const int l16 = lane & 15, g4 = lane >> 4;

  const int bh = blockIdx.x;
  const int seg = blockIdx.y;
  const int b = bh / a.H, h = bh - (bh / a.H) * a.H;
  const int total_chunks = (a.T + C - 1) / C;
  const int chunk0 = seg * a.seg_chunks;
  int nch = total_chunks - chunk0;
  if (nch > a.seg_chunks) nch = a.seg_chunks;
  if (nch <= 0) return;  // uniform across the workgroup

  const int64_t DD = static_cast<int64_t>(D) * D;
  const int64_t tok_stride = static_cast<int64_t>(a.H) * D;
  const int64_t tok_base = (static_cast<int64_t>(b) * a.T * a.H + h) * D;
  const int64_t dl_base = static_cast<int64_t>(b) * a.T * a.H + h;
  const E* gq = static_cast<const E*>(a.q);
  const E* gk = static_cast<const E*>(a.k);
  const E* gv = static_cast<const E*>(a.v);

  // zero T~ buffers (the strictly upper blocks are never written afterwards)
  for (int i = tid; i < 2 * R * TT_LD; i += NT) {
    (&sm.tth[0][0])[i] = E(0.0f);
    (&sm.ttl[0][0])[i] = E(0.0f);
  }
  __syncthreads();

  // ---------------------------------------------------------------- producers
  // Loop index it runs from -2 to nch-1 in every wave; consumers work on chunk it,
  // producer role 1 on chunk it+1, role 0 on chunk it+2.  Every wave executes one LDS
  // barrier per iteration (plus one more after the readout reduction).
  struct Regs {
    uint4 kv[8];  // k/v in Gram-operand order: rho = l32, features 16ks + 8g + 0..7
    uint4 q[4];   // q: e = lane + 64m -> token e>>4, features 8*(e&15) + 0..7
    DT d;         // raw delta of token `lane` (lanes 0..15)
  };

  // Branch-free loads: token indices are clamped to T-1 for the address and tokens
  // past the end are zeroed when staged (p_stage), so no load is predicated and the
  // destination registers need no initialisation while older loads are in flight.
  auto p_load = [&](Regs& r, int n) {
    const int t0 = (chunk0 + n) * C;
    const int tk = min(t0 + (l32 >> 1), a.T - 1);
    const E* src = ((l32 & 1) ? gv : gk) + tok_base + tk * tok_stride + 8 * g;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) r.kv[ks] = *reinterpret_cast<const uint4*>(src + 16 * ks);
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int e = lane + 64 * m;
      const int tq = min(t0 + (e >> 4), a.T - 1);
      r.q[m] = *reinterpret_cast<const uint4*>(gq + tok_base + tq * tok_stride + 8 * (e & 15));
    }
    const int td = min(t0 + (lane & (C - 1)), a.T - 1);
    r.d = static_cast<const DT*>(a.delta)[dl_base + static_cast<int64_t>(td) * a.H];
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

  // role 0, chunk n: stage inputs, Gram, Cayley blocks, diagonal blocks of T~
  auto p_stage = [&](const Regs& r_in, int n) {
    const int nb = n % 3;
    Stage0& P = sm.s0[n & 1];
    const int rho = l32;
    const int t0 = (chunk0 + n) * C;
    Regs r = r_in;
    if (t0 + C > a.T) {  // last, partial chunk: zero the tokens past the end
      const uint4 z = make_uint4(0, 0, 0, 0);
      if (t0 + (l32 >> 1) >= a.T) {
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) r.kv[ks] = z;
      }
#pragma unroll
      for (int m = 0; m < 4; ++m)
        if (t0 + ((lane + 64 * m) >> 4) >= a.T) r.q[m] = z;
      if (t0 + (lane & (C - 1)) >= a.T) r.d = DT{};
    }
    E* tdst = sm.tok[nb][rho & 1] + (rho >> 1) * TOK_LD;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      *reinterpret_cast<uint4*>(tdst + 16 * ks + 8 * g) = r.kv[ks];
      const V8 x = *reinterpret_cast<const V8*>(&r.kv[ks]);
#pragma unroll
      for (int i = 0; i < 8; ++i) sm.ut[nb][(16 * ks + 8 * g + i) * UT_LD + rho] = x[i];
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int e = lane + 64 * m;
      *reinterpret_cast<uint4*>(sm.tok[nb][2] + (e >> 4) * TOK_LD + 8 * (e & 15)) = r.q[m];
    }
    // Gram G = U^T U (A and B operands are the same registers)
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
    if (lane < C) {
      const int t = lane;
      const float kk = P.gram[(2 * t) * T_LD + 2 * t];
      const float vv = P.gram[(2 * t + 1) * T_LD + 2 * t + 1];
      const float kv = P.gram[(2 * t) * T_LD + 2 * t + 1];
      const cayley2 M = cayley_coeffs(io<DT>::to_f32(r.d), kk, vv, kv);
      P.mcoef[t] = make_float4(M.m00, M.m01, M.m10, M.m11);
    }
    wave_sync();
    // diagonal 8x8 blocks (4 tokens) by forward substitution, lane = (block gb, column c)
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

  // role 1, chunk n: off-diagonal blocks T~_{g,h} = T~_{g,g} S, S = sum_{m=h}^{g-1} G_{g,m} T~_{m,h};
  // writes all of T~ (hi + lo) for the consumers.  lane = element (ea, eb) of an 8x8 block.
  auto p_offdiag = [&](int n) {
    const Stage0& P = sm.s0[n & 1];
    Stage1& Q = sm.s1;
    E* tth = sm.tth[n & 1];
    E* ttl = sm.ttl[n & 1];
    auto tt_store = [&](int row, int col, float x) {
      const E hpart = static_cast<E>(x);
      tth[row * TT_LD + col] = hpart;
      ttl[row * TT_LD + col] = static_cast<E>(x - static_cast<float>(hpart));
    };
    const int ea = lane >> 3, eb = lane & 7;
    const float* g1 = &P.gram[(8 + ea) * T_LD];
    const float* g2 = &P.gram[(16 + ea) * T_LD];
    const float* g3 = &P.gram[(24 + ea) * T_LD];
#pragma unroll
    for (int gb = 0; gb < 4; ++gb) tt_store(8 * gb + ea, 8 * gb + eb, P.drow[gb][ea * 8 + eb]);
    // round 1: (1,0), (2,1), (3,2)
    Q.sblk[0][eb * 8 + ea] = dot8(g1, &P.dcol[0][eb * 8]);
    Q.sblk[1][eb * 8 + ea] = dot8(g2 + 8, &P.dcol[1][eb * 8]);
    Q.sblk[2][eb * 8 + ea] = dot8(g3 + 16, &P.dcol[2][eb * 8]);
    wave_sync();
    const float y10 = dot8(&P.drow[1][ea * 8], &Q.sblk[0][eb * 8]);
    const float y21 = dot8(&P.drow[2][ea * 8], &Q.sblk[1][eb * 8]);
    const float y32 = dot8(&P.drow[3][ea * 8], &Q.sblk[2][eb * 8]);
    tt_store(8 + ea, eb, y10);
    tt_store(16 + ea, 8 + eb, y21);
    tt_store(24 + ea, 16 + eb, y32);
    Q.ocol[0][eb * 8 + ea] = y10;
    Q.ocol[1][eb * 8 + ea] = y21;
    wave_sync();
    // round 2: (2,0), (3,1)
    Q.sblk[0][eb * 8 + ea] = dot8(g2, &P.dcol[0][eb * 8]) + dot8(g2 + 8, &Q.ocol[0][eb * 8]);
    Q.sblk[1][eb * 8 + ea] = dot8(g3 + 8, &P.dcol[1][eb * 8]) + dot8(g3 + 16, &Q.ocol[1][eb * 8]);
    wave_sync();
    const float y20 = dot8(&P.drow[2][ea * 8], &Q.sblk[0][eb * 8]);
    const float y31 = dot8(&P.drow[3][ea * 8], &Q.sblk[1][eb * 8]);
    tt_store(16 + ea, eb, y20);
    tt_store(24 + ea, 8 + eb, y31);
    Q.ocol[2][eb * 8 + ea] = y20;
    wave_sync();
    // round 3: (3,0)
    Q.sblk[2][eb * 8 + ea] = dot8(g3, &P.dcol[0][eb * 8]) + dot8(g3 + 8, &Q.ocol[0][eb * 8]) +
                             dot8(g3 + 16, &Q.ocol[2][eb * 8]);
    wave_sync();
    tt_store(24 + ea, eb, dot8(&P.drow[3][ea * 8], &Q.sblk[2][eb * 8]));
  };

  if (wave == NCW) {
    // ================================================ producer role 0
    Regs ra, rb;
    p_load(ra, 0);
    auto step0 = [&](const Regs& cur, Regs& nxt, int it) {
      const int n = it + 2;
      // issued unconditionally (clamped to the last chunk): a conditional prefetch
      // would make the compiler wait for it before using `cur`
      p_load(nxt, min(n + 1, nch - 1));
      if (n < nch) p_stage(cur, n);
      lds_barrier();
      if (READOUT && it >= 0) lds_barrier();
    };
    for (int it = -2; it < nch; it += 2) {
      step0(ra, rb, it);
      if (it + 1 < nch) step0(rb, ra, it + 1);
    }
    return;
  }
  if (wave == NCW + 1) {
    // ================================================ producer role 1
    for (int it = -2; it < nch; ++it) {
      const int n = it + 1;
      if (n >= 0 && n < nch) p_offdiag(n);
      lds_barrier();
      if (READOUT && it >= 0) lds_barrier();
    }
    return;
  }

  // ================================================== consumers
  f32x16 psi[4];  // slab columns 32*wave + l32, tile rt rows 32rt + 8(r/4) + 4g + r%4
  const int col = 32 * wave + l32;
  {
    const float* src = nullptr;
    if (seg == 0)
      src = a.psi0 ? a.psi0 + bh * DD : nullptr;
    else if (a.starts)
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
  }

  for (int cc = -2; cc < nch; ++cc) {
    const int cb = cc & 1;  // T~ buffer
    if (cc >= 0) {
      const int nb = cc % 3;
      const E* tk = sm.tok[nb][0];
      const E* tv = sm.tok[nb][1];
      const E* tq = sm.tok[nb][2];
      const E* ut = sm.ut[nb];
      
      // W = U^T Psi_slab  (32 x 32).  PREC: Psi split hi + lo (fp32-faithful);
      // otherwise Psi rounded once to 16 bits, and the rounded values double as the
      // readout stash below.
      f32x16 Wa = {}, Wb = {};  // two independent MFMA chains (row tiles 0-1 and 2-3)
      V8 pb[4][2];
      const E* urow = ((l32 & 1) ? tv : tk) + (l32 >> 1) * TOK_LD;
#pragma unroll
      for (int rt = 0; rt < 4; ++rt)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const int d0 = 32 * rt + 16 * ks + 4 * g;
          const V8 av = lds4x2<E>(urow + d0, urow + d0 + 8);
          float x[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) x[i] = psi[rt][8 * ks + i];
          f32x16& Wr = rt < 2 ? Wa : Wb;
          if (PREC) {
            V8 lo;
            split8<E>(x, pb[rt][ks], lo);
            Wr = MM::mma32(av, pb[rt][ks], Wr);
            Wr = MM::mma32(av, lo, Wr);
          } else {
            pb[rt][ks] = round8<E>(x);
            Wr = MM::mma32(av, pb[rt][ks], Wr);
          }
        }
      const f32x16 W = Wa + Wb;

      // Z = T~ W with T~ = hi + lo from the producers; PREC also splits W.
      f32x16 Z = {};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const E* th = sm.tth[cb] + l32 * TT_LD + 16 * ks + 4 * g;
        const E* tl = sm.ttl[cb] + l32 * TT_LD + 16 * ks + 4 * g;
        const V8 ahi = lds4x2<E>(th, th + 8);
        const V8 alo = lds4x2<E>(tl, tl + 8);
        float wv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) wv[i] = W[8 * ks + i];
        if (PREC) {
          V8 whi, wlo;
          split8<E>(wv, whi, wlo);
          Z = MM::mma32(ahi, whi, Z);
          Z = MM::mma32(ahi, wlo, Z);
          Z = MM::mma32(alo, whi, Z);
        } else {
          const V8 wb = round8<E>(wv);
          Z = MM::mma32(ahi, wb, Z);
          Z = MM::mma32(alo, wb, Z);
        }
      }

      if (READOUT) {
        E* ps = sm.ps[wave];
        E* zs = sm.zs[wave];
#pragma unroll
        for (int rt = 0; rt < 4; ++rt)
#pragma unroll
          for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int i = 0; i < 8; ++i)
              ps[(32 * rt + 16 * ks + 8 * (i >> 2) + 4 * g + (i & 3)) * PS_LD + l32] = pb[rt][ks][i];
#pragma unroll
        for (int r = 0; r < 16; ++r)
          zs[(8 * (r >> 2) + 4 * g + (r & 3)) * PS_LD + l32] = static_cast<E>(Z[r]);
        wave_sync();
        // O_w = S[:, slab] Q[slab, :] + U mask(Z[:, slab] Q[slab, :])   (128 x 16)
        const V8 bq = lds8<E>(tq + l16 * TOK_LD + 32 * wave + 8 * g4);
        f32x4 O[8];
#pragma unroll
        for (int it = 0; it < 8; ++it) {
          const f32x4 zero = {};
          O[it] = MM::mma16(lds8<E>(ps + (16 * it + l16) * PS_LD + 8 * g4), bq, zero);
        }
        const f32x4 zero = {};
        const f32x4 y0 = MM::mma16(lds8<E>(zs + l16 * PS_LD + 8 * g4), bq, zero);
        const f32x4 y1 = MM::mma16(lds8<E>(zs + (16 + l16) * PS_LD + 8 * g4), bq, zero);
        V8 by;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          by[r] = static_cast<E>(((4 * g4 + r) >> 1) <= l16 ? y0[r] : 0.f);
          by[4 + r] = static_cast<E>(((16 + 4 * g4 + r) >> 1) <= l16 ? y1[r] : 0.f);
        }
#pragma unroll
        for (int it = 0; it < 8; ++it) {
          const E* urow2 = ut + (16 * it + l16) * UT_LD;
          O[it] = MM::mma16(lds4x2<E>(urow2 + 4 * g4, urow2 + 16 + 4 * g4), by, O[it]);
        }
        wave_sync();  // every lane is done reading ps before it is reused for O
        float* op = reinterpret_cast<float*>(ps);
#pragma unroll
        for (int it = 0; it < 8; ++it)
          *reinterpret_cast<float4*>(&op[l16 * OP_LD + 16 * it + 4 * g4]) =
              make_float4(O[it][0], O[it][1], O[it][2], O[it][3]);
      }

      // Psi_slab += U Z
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        float zv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) zv[i] = Z[8 * ks + i];
        V8 zhi, zlo;
        if (PREC) split8<E>(zv, zhi, zlo);
        else zhi = round8<E>(zv);
#pragma unroll
        for (int rt = 0; rt < 4; ++rt) {
          const E* urow3 = ut + (32 * rt + l32) * UT_LD + 16 * ks + 4 * g;
          const V8 av = lds4x2<E>(urow3, urow3 + 8);
          psi[rt] = MM::mma32(av, zhi, psi[rt]);
          if (PREC) psi[rt] = MM::mma32(av, zlo, psi[rt]);
        }
      }
    }
    lds_barrier();  // (A)
    if (READOUT && cc >= 0) {
      if (tid < 256) {
        const int t = tid >> 4, fg = tid & 15;
        const int tok = (chunk0 + cc) * C + t;
        if (tok < a.T) {
          float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int w = 0; w < NCW; ++w) {
            const float* op = reinterpret_cast<const float*>(sm.ps[w]) + t * OP_LD + 8 * fg;
            const float4 x0 = *reinterpret_cast<const float4*>(op);
            const float4 x1 = *reinterpret_cast<const float4*>(op + 4);
            acc[0] += x0.x; acc[1] += x0.y; acc[2] += x0.z; acc[3] += x0.w;
            acc[4] += x1.x; acc[5] += x1.y; acc[6] += x1.z; acc[7] += x1.w;
          }
          V8 o8;
#pragma unroll
          for (int i = 0; i < 8; ++i) o8[i] = static_cast<E>(acc[i]);
          if (a.out != nullptr)
            *reinterpret_cast<V8*>(static_cast<E*>(a.out) + tok_base + tok * tok_stride + 8 * fg) = o8;
        }
      }
      lds_barrier();  // (B)
    }
  }

  // ---------------------------------------------------------------- end state
  {
    float* dst = nullptr;
    if (a.end_mode == 0) dst = a.ends + (static_cast<int64_t>(seg) * a.BH + bh) * DD;
    else if (seg == a.nseg - 1) dst = a.ends + bh * DD;
    if (dst) {
#pragma unroll
      for (int rt = 0; rt < 4; ++rt)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          dst[(32 * rt + 8 * (r >> 2) + 4 * g + (r & 3)) * D + col] = psi[rt][r];
    }
  }
}

// start_s = P_{s-1} start_{s-1}, s = 1 .. S-1, start_0 = psi0 (identity if null).
// One workgroup of 8 waves per (b, h); wave w owns the 16-column block w of the
// running start state (in MFMA accumulators).  Each P_{s-1} is staged once in LDS
// as a 16-bit hi + lo pair, shared by the 8 waves; the next P is prefetched into
// registers while the current product runs.  bf16x3 (hi*hi + hi*lo + lo*hi) keeps
// the chain fp32-faithful.
constexpr int CARRY_WAVES = D / 16;
constexpr int CARRY_NT = CARRY_WAVES * 64;
constexpr int CP_LD = D + 8;  // elements per staged P row (272 B)
constexpr int CARRY_F4 = D * D / 4 / CARRY_NT;  // float4 of P per thread

__global__ __launch_bounds__(CARRY_NT) void sssd_carry_kernel(const float* psi0, const float* P,
                                                              float* starts, int BH, int S) {
  typedef mfma_t<__bf16> MM;
  typedef MM::v8 V8;
  __shared__ __bf16 phi[D * CP_LD];
  __shared__ __bf16 plo[D * CP_LD];
  const int bh = blockIdx.x;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int l16 = lane & 15, g4 = lane >> 4;
  const int col = 16 * wave + l16;
  const int64_t DD = static_cast<int64_t>(D) * D;
  f32x4 X[8];  // X[16it + 4g4 + r][col]
#pragma unroll
  for (int it = 0; it < 8; ++it)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 16 * it + 4 * g4 + r;
      X[it][r] = psi0 ? psi0[bh * DD + row * D + col] : (row == col ? 1.f : 0.f);
    }
  float4 pf[CARRY_F4];  // this thread's share of the next P (element e = tid + NT*m)
  auto fetch = [&](int s) {
    const float4* src = reinterpret_cast<const float4*>(P + (static_cast<int64_t>(s - 1) * BH + bh) * DD);
#pragma unroll
    for (int m = 0; m < CARRY_F4; ++m) pf[m] = src[tid + CARRY_NT * m];
  };
  if (S > 1) fetch(1);
  for (int s = 1; s < S; ++s) {
    // stage P_{s-1} as hi + lo
#pragma unroll
    for (int m = 0; m < CARRY_F4; ++m) {
      const int e = 4 * (tid + CARRY_NT * m);
      const int row = e / D, c0 = e - row * D;
      const float xv[4] = {pf[m].x, pf[m].y, pf[m].z, pf[m].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const __bf16 hv = static_cast<__bf16>(xv[i]);
        phi[row * CP_LD + c0 + i] = hv;
        plo[row * CP_LD + c0 + i] = static_cast<__bf16>(xv[i] - static_cast<float>(hv));
      }
    }
    __syncthreads();
    if (s + 1 < S) fetch(s + 1);
    f32x4 Y[8];
#pragma unroll
    for (int it = 0; it < 8; ++it) Y[it] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      float xb[8];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        xb[r] = X[2 * ks][r];
        xb[4 + r] = X[2 * ks + 1][r];
      }
      V8 xhi, xlo;
      split8<__bf16>(xb, xhi, xlo);
#pragma unroll
      for (int it = 0; it < 8; ++it) {
        const int off = (16 * it + l16) * CP_LD + 32 * ks + 4 * g4;
        const V8 ahi = cat8<bf16x4, V8>(*reinterpret_cast<const bf16x4*>(&phi[off]),
                                         *reinterpret_cast<const bf16x4*>(&phi[off + 16]));
        const V8 alo = cat8<bf16x4, V8>(*reinterpret_cast<const bf16x4*>(&plo[off]),
                                         *reinterpret_cast<const bf16x4*>(&plo[off + 16]));
        Y[it] = MM::mma16(ahi, xhi, Y[it]);
        Y[it] = MM::mma16(ahi, xlo, Y[it]);
        Y[it] = MM::mma16(alo, xhi, Y[it]);
      }
    }
    float* dst = starts + (static_cast<int64_t>(s - 1) * BH + bh) * DD;
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      X[it] = Y[it];
#pragma unroll
      for (int r = 0; r < 4; ++r) dst[(16 * it + 4 * g4 + r) * D + col] = Y[it][r];
    }
    __syncthreads();  // the staged P is read by every wave before it is replaced
  }
}

}  // namespace chunk

// ------------------------------------------------------------------ host side
namespace {

constexpr int kTargetWorkgroups = 256;  // one 5-wave workgroup per CU (LDS-limited)

struct Plan {
  int nchunks, seg_chunks, nseg;
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
  return p;
}

bool chunk_path(int64_t T, int64_t D, int io_dtype) {
  return D == chunk::D && (io_dtype == VMI_BF16 || io_dtype == VMI_F16) && T >= 2 * chunk::C;
}

// PREC (the only variant dispatched): the state, W and Z enter the chunk GEMMs as
// hi + lo 16-bit pairs, so every product is fp32-faithful and the state norm is kept
// to ~1e-6 per 4096 tokens.  PREC=false rounds them to 16 bits once (about 6% faster
// at the OP shape, but its norm drift grows to ~4e-5 per 4096 tokens).
template <typename E, typename DT, bool PREC>
hipError_t run_chunked_p(const void* q, const void* k, const void* v, const void* delta,
                       int delta_dtype, const float* psi_in, void* out, float* psi_out, int B,
                       int T, int H, void* workspace, hipStream_t stream) {
  const int BH = B * H;
  const Plan p = make_plan(BH, T);
  const int64_t DD = static_cast<int64_t>(chunk::D) * chunk::D;
  chunk::Args a;
  a.q = q; a.k = k; a.v = v; a.delta = delta; a.delta_dtype = delta_dtype;
  a.T = T; a.H = H; a.BH = BH;
  a.seg_chunks = p.seg_chunks;
  a.nseg = p.nseg;
  float* P = static_cast<float*>(workspace);
  float* starts = P ? P + static_cast<int64_t>(p.nseg - 1) * BH * DD : nullptr;
  if (p.nseg > 1) {
    chunk::Args pa = a;
    pa.psi0 = nullptr;
    pa.starts = nullptr;
    pa.out = nullptr;
    pa.ends = P;
    pa.end_mode = 0;
    hipLaunchKernelGGL((chunk::sssd_chunk_kernel<E, DT, false, PREC>), dim3(BH, p.nseg - 1),
                       dim3(chunk::NT), 0, stream, pa);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(chunk::sssd_carry_kernel, dim3(BH), dim3(chunk::CARRY_NT), 0, stream,
                       psi_in, P, starts, BH, p.nseg);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  a.psi0 = psi_in;
  a.starts = p.nseg > 1 ? starts : nullptr;
  a.out = out;
  a.ends = psi_out;
  a.end_mode = 1;
  hipLaunchKernelGGL((chunk::sssd_chunk_kernel<E, DT, true, PREC>), dim3(BH, p.nseg), dim3(chunk::NT),
                     0, stream, a);
  return hipGetLastError();
}

template <typename E, typename DT>
hipError_t run_chunked(const void* q, const void* k, const void* v, const void* delta,
                       int delta_dtype, const float* psi_in, void* out, float* psi_out, int B,
                       int T, int H, void* workspace, hipStream_t stream) {
  return run_chunked_p<E, DT, true>(q, k, v, delta, delta_dtype, psi_in, out, psi_out, B, T, H,
                                    workspace, stream);
}

}  // namespace

size_t chunk_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t D, int io_dtype) {
  if (!chunk_path(T, D, io_dtype)) return 0;
  const Plan p = make_plan(B * H, T);
  if (p.nseg <= 1) return 0;
  return static_cast<size_t>(2) * (p.nseg - 1) * B * H * D * D * sizeof(float);
}

bool use_chunk_path(int64_t T, int64_t D, int io_dtype) { return chunk_path(T, D, io_dtype); }

hipError_t launch_sssd_chunked(const void* q, const void* k, const void* v, const void* delta,
                               int io_dtype, int delta_dtype, const float* psi_in, void* out,
                               float* psi_out, int B, int T, int H, void* workspace,
                               hipStream_t stream) {
#define VMI_RUN(E, DT) \
  return run_chunked<E, DT>(q, k, v, delta, delta_dtype, psi_in, out, psi_out, B, T, H, workspace, \
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
