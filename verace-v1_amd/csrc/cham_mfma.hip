// CHAM state carry on the matrix cores, for the wide route (128 < h <= 1024) with 16-bit
// k, v (reference: the h > 128 branch of launch_cham_triton_update, triton_kernels.py:639-685,
// and _cham_rank2_update_kernel, :477-597; parity target cham_memory.py:167-238).
//
// The per-token factor is U_t = I + W_t N_t W_t^T with W_t = [k_t v_t] real (h x 2) and N_t
// the complex 2 x 2 Cayley block (cham_common.h).  For a chunk of CT = 16 tokens, with
// Y = [W_1 .. W_16] (h x 32, real) and G = Y^T Y,
//   U_16 ... U_1 = I + Y T Y^T,   T = (I - L)^-1 blockdiag(N),  L_ti = N_t G_ti (i < t)
// (the same algebra as the SSSD chunk form, complex T).  A state column evolves on its own,
// so the chunk update of a block of columns H (h x 16, complex) is
//   W = Y^T H (real Y: one GEMM over [Re H | Im H]),  Z = T W (complex),  H += Y Z.
//
// Launches (before the readout kernels of cham_wide.hip, which read the snapshots written
// here exactly as they read the token-sequential kernel's):
//   1. cm_prep_kernel, one wave per (chunk, sequence): k, v converted to f16 (non-finite
//      elements zeroed) and stored in the column kernel's MFMA operand layout (each
//      16-feature block of the chunk's 32 rank rows as 64 lanes x 16 bytes, so every operand
//      load is a contiguous 1 KB), G on the MFMA from them, then T by
//      forward substitution over the 16 tokens (lane = column of T), stored as f16 hi + lo
//      parts of Re T and Im T.
//   2. cm_cols_kernel, workgroup (16 columns, sequence, state): 8 waves, wave w owns rows
//      [w RPW, (w+1) RPW) of the 16 complex columns as fp32 MFMA accumulators for the whole
//      call.  Per chunk: W partials (v_mfma_f32_32x32x16_f16, Y exact in f16, H as an f16
//      hi + lo pair, fp32 accumulation), an 8-way reduction through LDS, Z = T W on four waves
//      (16x16x32, hi/lo products), H += Y Z with Y read back through transposing LDS reads.
//
// Precision: k, v from bf16 / f16 are exact in f16 (bf16 values below 2^-14 round to f16
// subnormals, an absolute change below 2^-25; bf16 values from 2^16 up have no f16 value: their
// token is taken as the identity, like a token with a non-finite element, and the entry point
// documents |k|, |v| elements below 65504 as this route's precondition); H and W enter the products as f16 hi + lo
// pairs and T as an f16 hi + lo pair, so every product is fp32-faithful (~2^-21 relative)
// and the fp32 accumulators carry the state.  The state is carried scaled (TSCALE, SMAX
// below) so that the lo parts stay normal f16 numbers: measured against the fp64 closed form
// at h = 1024, T = 100 (bf16 inputs) the state is within 1e-7 relative.  Non-finite elements of k, v read as zero and
// their token has N = 0 (cham_common.h's guard), so the token's U is the identity.
#include "cham_common.h"
#include "vmi_dispatch.h"
#include "vmi_mfma.h"

namespace vmi {
namespace chamm {

typedef _Float16 E;
typedef mfma_t<E> MM;
typedef MM::v8 V8;
typedef MM::v4 V4;

constexpr int CT = 16;         // tokens per chunk
constexpr int RK = 2 * CT;     // rank rows per chunk (k_t, v_t)
constexpr int NWV = 8;         // waves per column workgroup
constexpr int NTH = NWV * 64;
constexpr int COLS = 16;       // complex state columns per workgroup
constexpr int NCF = 8;         // floats per token in the coefficient array (cham_wide.hip)
constexpr int TT_STRIDE = 4 * RK * RK;  // f16 per chunk: Re T hi, Re T lo, Im T hi, Im T lo
// T is stored scaled by TSCALE and the state carried scaled by a power of two that puts its
// largest start entry at most SMAX: the lo parts of the hi + lo pairs then stay in f16's normal
// range (below 2^-14 they would keep only 2^-24 absolute resolution).  Both are exact.
constexpr float TSCALE = 256.f;
constexpr float SMAX = 256.f;

// LDS row slot of rank row rho (bits 0,1,2,3,4 -> 3,4,2,1,0): with a 264-byte pitch both the
// 8-byte writes of a wave's Y rows and the transposing reads of the update operand fall in
// distinct banks (the slot map of the SSSD chunk scan, whose access patterns these are).
__host__ __device__ constexpr int rho_slot(int rho) {
  return ((rho & 1) << 3) | ((rho & 2) << 3) | (rho & 4) | ((rho & 8) >> 2) | ((rho & 16) >> 4);
}

// 16-bit values that have no finite f16 value, recognised by their magnitude bits: f16 Inf /
// NaN (0x7c00 and up), and for bf16 also the finite values from 2^16 (0x4780) up, which round
// to f16 Inf.  Such an element reads as zero, and its token is the identity (its coefficients
// are zeroed by wide_coef_kernel's matching test).
template <typename IO> struct bits16;
template <> struct bits16<f16_t> { static constexpr uint32_t LIMIT = 0x7c00u; };
template <> struct bits16<bf16_t> { static constexpr uint32_t LIMIT = 0x4780u; };

// mask with 0xffff in each 16-bit half of `w` that holds an f16-representable value, 0 elsewhere
template <typename IO> __device__ __forceinline__ uint32_t finite_mask(uint32_t w) {
  constexpr uint32_t L = bits16<IO>::LIMIT;
  const uint32_t lo = (w & 0x7fffu) >= L ? 0u : 0x0000ffffu;
  const uint32_t hi = ((w >> 16) & 0x7fffu) >= L ? 0u : 0xffff0000u;
  return lo | hi;
}

// 4 raw 16-bit inputs -> 4 f16 (bf16: exact conversion; f16: as is).  With `guard`,
// non-finite elements become 0 first.
template <typename IO> __device__ __forceinline__ V4 to_f16x4(uint2 raw, bool guard);
template <> __device__ __forceinline__ V4 to_f16x4<f16_t>(uint2 raw, bool guard) {
  if (guard) raw = make_uint2(raw.x & finite_mask<f16_t>(raw.x), raw.y & finite_mask<f16_t>(raw.y));
  return __builtin_bit_cast(V4, raw);
}
template <> __device__ __forceinline__ V4 to_f16x4<bf16_t>(uint2 raw, bool guard) {
  if (guard) raw = make_uint2(raw.x & finite_mask<bf16_t>(raw.x), raw.y & finite_mask<bf16_t>(raw.y));
  const float f[4] = {__uint_as_float(raw.x << 16), __uint_as_float(raw.x & 0xffff0000u),
                      __uint_as_float(raw.y << 16), __uint_as_float(raw.y & 0xffff0000u)};
  V4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = static_cast<E>(f[i]);
  return r;
}

// 4 raw 16-bit inputs -> fp32
template <typename IO> __device__ __forceinline__ void unpack4(uint2 raw, float* f);
template <> __device__ __forceinline__ void unpack4<bf16_t>(uint2 raw, float* f) {
  f[0] = __uint_as_float(raw.x << 16);
  f[1] = __uint_as_float(raw.x & 0xffff0000u);
  f[2] = __uint_as_float(raw.y << 16);
  f[3] = __uint_as_float(raw.y & 0xffff0000u);
}
template <> __device__ __forceinline__ void unpack4<f16_t>(uint2 raw, float* f) {
  const V4 h = __builtin_bit_cast(V4, raw);
#pragma unroll
  for (int i = 0; i < 4; ++i) f[i] = static_cast<float>(h[i]);
}

// fp32 -> (hi, lo) f16 pair (round to nearest): x = hi + lo to ~2^-22.  hi by a packed
// conversion per two values; lo = x - hi is exact in fp32 and is rounded to f16 by one
// mixed-precision FMA per value (x * 1.0 - hi, hi read as f16 from its half of the register).
__device__ __forceinline__ void split8p(const float* x, V8& hi, V8& lo) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const f2 xv = {x[2 * p], x[2 * p + 1]};
    const h2 hv = __builtin_convertvector(xv, h2);
    const uint32_t hb = __builtin_bit_cast(uint32_t, hv);
    uint32_t lb;
    asm("v_fma_mixlo_f16 %0, %1, 1.0, -%3 op_sel_hi:[0,0,1]\n\t"
        "v_fma_mixhi_f16 %0, %2, 1.0, -%3 op_sel:[0,0,1] op_sel_hi:[0,0,1]"
        : "=&v"(lb)
        : "v"(xv[0]), "v"(xv[1]), "v"(hb));
    const h2 lw = __builtin_bit_cast(h2, lb);
    hi[2 * p] = hv[0];
    hi[2 * p + 1] = hv[1];
    lo[2 * p] = lw[0];
    lo[2 * p + 1] = lw[1];
  }
}

// ---------------------------------------------------------------- 1: G and T per chunk
// FUSED: k and v are read from the stacked projection (passed as k; row b*T + t of `stride`
// elements: k at h, v at 2h), v through silu, both scaled by the norms the fused coefficient
// kernel stored (coef floats 6 and 7) and rounded by cham::fused_f16, as that kernel did for
// the Gram entries of its coefficients.
template <typename IO, bool FUSED = false>
__global__ __launch_bounds__(64) void cm_prep_kernel(const IO* __restrict__ k,
                                                     const IO* __restrict__ v,
                                                     const float* __restrict__ coef,
                                                     E* __restrict__ tt, E* __restrict__ yop,
                                                     int T, int h, int hp, int64_t stride = 0) {
  __shared__ float G[RK][RK + 1];
  __shared__ float Nc[CT][NCF];
  __shared__ float Tf[2][RK][RK + 1];
  const int lane = threadIdx.x, l32 = lane & 31, g = lane >> 5;
  const int m = blockIdx.x, b = blockIdx.y, nc = gridDim.x;
  const int t0 = m * CT;
  // Gram: lane (rho = l32, g) holds features 16 ks + 8 g + 0..7 of rank row rho
  const int tok = t0 + (l32 >> 1);
  const bool tok_ok = tok < T;
  const int64_t row = static_cast<int64_t>(b) * T + (tok_ok ? tok : 0);
  const IO* src = FUSED ? k + row * stride + ((l32 & 1) ? 2 * h : h) : ((l32 & 1) ? v : k) + row * h;
  const float scale = FUSED ? coef[row * NCF + 6 + (l32 & 1)] : 1.f;
  // operand block kb of this chunk: lane (rho, g) holds features 16 kb + 4 g + {0..3} and
  // 16 kb + 8 + 4 g + {0..3} of rank row rho (the K order of the column kernel's state tiles;
  // G sums over every feature, so any order serves it); blocks past h and tokens past T are 0
  E* dst = yop + (static_cast<int64_t>(b) * nc + m) * (hp / 16) * 512 + lane * 8;
  f32x16 acc = {};
  const int nks = (h + 15) / 16;  // the same trip counts in both half-waves (MFMA is wave-wide)
  for (int ks = 0; ks < hp / 16; ++ks) {
    const int f0 = 16 * ks + 4 * g, f1 = f0 + 8;  // h % 4 == 0: a piece is wholly in or out
    uint2 r0 = make_uint2(0, 0), r1 = make_uint2(0, 0);
    if (tok_ok && f0 < h) r0 = *reinterpret_cast<const uint2*>(src + f0);
    if (tok_ok && f1 < h) r1 = *reinterpret_cast<const uint2*>(src + f1);
    V8 x;
    if constexpr (FUSED) {
      float f[8];
      unpack4<IO>(r0, f);
      unpack4<IO>(r1, f + 4);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float y = (l32 & 1) ? cham::silu_f(f[i]) : f[i];
        x[i] = cham::fused_f16(y, scale);
      }
      if (!(tok_ok && f0 < h)) {
#pragma unroll
        for (int i = 0; i < 4; ++i) x[i] = static_cast<E>(0.f);
      }
      if (!(tok_ok && f1 < h)) {
#pragma unroll
        for (int i = 4; i < 8; ++i) x[i] = static_cast<E>(0.f);
      }
    } else {
      x = cat8<V4, V8>(to_f16x4<IO>(r0, true), to_f16x4<IO>(r1, true));
    }
    *reinterpret_cast<V8*>(dst + ks * 512) = x;
    if (ks < nks) acc = MM::mma32(x, x, acc);
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) G[8 * (r >> 2) + 4 * g + (r & 3)][l32] = acc[r];
  for (int e = lane; e < CT * NCF; e += 64) {
    const int t = e / NCF;
    Nc[t][e % NCF] = t0 + t < T ? coef[(static_cast<int64_t>(b) * T + t0 + t) * NCF + e % NCF] : 0.f;
  }
  __syncthreads();
  // T = (I - L)^-1 blockdiag(N): block row t = N_t (E_t + sum_{i<t} G_ti T_i); lane j < 32
  // computes column j (rows 0 .. 31, complex)
  if (lane < RK) {
    const int j = lane;
    float xr[RK], xi[RK];
#pragma unroll
    for (int t = 0; t < CT; ++t) {
      float a0r = j == 2 * t ? 1.f : 0.f, a1r = j == 2 * t + 1 ? 1.f : 0.f, a0i = 0.f, a1i = 0.f;
#pragma unroll
      for (int i = 0; i < 2 * t; ++i) {
        const float g0 = G[2 * t][i], g1 = G[2 * t + 1][i];
        a0r = fmaf(g0, xr[i], a0r);
        a0i = fmaf(g0, xi[i], a0i);
        a1r = fmaf(g1, xr[i], a1r);
        a1i = fmaf(g1, xi[i], a1i);
      }
      const float n11r = Nc[t][0], n11i = Nc[t][1], n12r = Nc[t][2], n12i = Nc[t][3];
      const float n22r = Nc[t][4], n22i = Nc[t][5];
      xr[2 * t] = n11r * a0r - n11i * a0i + n12r * a1r - n12i * a1i;
      xi[2 * t] = n11r * a0i + n11i * a0r + n12r * a1i + n12i * a1r;
      xr[2 * t + 1] = n12r * a0r - n12i * a0i + n22r * a1r - n22i * a1i;
      xi[2 * t + 1] = n12r * a0i + n12i * a0r + n22r * a1i + n22i * a1r;
    }
#pragma unroll
    for (int rr = 0; rr < RK; ++rr) {
      Tf[0][rr][j] = xr[rr];
      Tf[1][rr][j] = xi[rr];
    }
  }
  __syncthreads();
  // row-major hi / lo parts: lane = (part, row) writes the row's 32 values
  {
    const int part = lane >> 5, row = lane & 31;
    E* dh = tt + (static_cast<int64_t>(b) * nc + m) * TT_STRIDE + (2 * part) * RK * RK + row * RK;
    E* dl = dh + RK * RK;
#pragma unroll
    for (int q = 0; q < RK / 8; ++q) {
      V8 hi, lo;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float x = TSCALE * Tf[part][row][8 * q + i];
        hi[i] = static_cast<E>(x);
        lo[i] = static_cast<E>(x - static_cast<float>(hi[i]));
      }
      *reinterpret_cast<V8*>(dh + 8 * q) = hi;
      *reinterpret_cast<V8*>(dl + 8 * q) = lo;
    }
  }
}

// ---------------------------------------------------------------- 2: state columns
constexpr int Y_LD = 132;  // f16 per LDS row of a wave's Y block (128 rows + pad; 264 B)
constexpr int W_LD = 36;   // floats per row of the W partials / reduced W ([n][rho])
constexpr int Z_LD = 40;   // f16 per row of Z' ([n][rho])

template <int TPW>
struct alignas(16) ColsSmem {
  static constexpr int RPW = 32 * TPW;
  float wpart[NWV][32][W_LD];
  float wred[32][W_LD];
  E zh[32][Z_LD];
  E zl[32][Z_LD];
  E yt[NWV][RK][Y_LD];
};

// Workgroup (column block cb, sequence b, state z).  Lane (n = lane % 32, g = lane / 32)
// of wave w holds, in tile rt, rows w RPW + 32 rt + 8 (r/4) + 4 g + r%4 of MFMA column n:
// the real part of state column c0 + n for n < 16, the imaginary part of c0 + n - 16 else.
// Readout snapshots (the state at the start of every c2 tokens):
//   S16 = false: fp32 [B][nch][2][h][HP] as in cham_wide.hip;
//   S16 = true (identity start, every entry of the state at most 1 in magnitude): f16 in the
//   A-operand layout of cm_read_kernel, [B][nch][part][HP / 32][HP / 16][64][8]: block
//   (part, it, kb) lane (m, g) holds part's rows 32 it + m, columns
//   16 kb + 8 (i/4) + 4 g + i%4 (i < 8), so this workgroup writes the blocks kb = cb.
template <int TPW, bool S16>
__global__ __launch_bounds__(NTH) void cm_cols_kernel(
    const E* __restrict__ yop, const E* __restrict__ tt,
    const float* __restrict__ i0r, const float* __restrict__ i0i,
    const float* __restrict__ i1r, const float* __restrict__ i1i, void* __restrict__ snapv,
    float* __restrict__ fr, float* __restrict__ fi, int T, int h, int nstates, int snap_on,
    int c2) {
  constexpr int RPW = 32 * TPW, HP = NWV * RPW;
  __shared__ ColsSmem<TPW> sm;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, g = lane >> 5, l16 = lane & 15, g4 = lane >> 4;
  const int c0 = blockIdx.x * COLS, b = blockIdx.y, z = blockIdx.z;
  const int r0w = wave * RPW;
  const int nc = (T + CT - 1) / CT;
  const int nch = (T + c2 - 1) / c2;
  const int cpc = c2 / CT;  // chunks per readout chunk
  const int64_t hh = static_cast<int64_t>(h) * h;
  const int ncol = l32 & 15, part = l32 >> 4;
  const int col = c0 + ncol;
  const bool colok = col < h;

  // ---- initial state (row-major [h][h] planes through LDS column tiles, or the identity)
  f32x16 hs[TPW];
  {
    const float* ir = z == 0 ? i0r : i1r;
    const float* ii = z == 0 ? i0i : i1i;
    float* tile = &sm.wpart[0][0][0];  // [COLS][HP] floats of one plane (<= 64 KB)
    static_assert(sizeof(ColsSmem<TPW>) >= sizeof(float) * COLS * HP, "tile does not fit");
#pragma unroll
    for (int rt = 0; rt < TPW; ++rt) hs[rt] = f32x16{};
    for (int p = 0; p < 2; ++p) {
      const float* src = p == 0 ? ir : ii;
      if (src) {
        for (int e = tid; e < h * COLS; e += NTH) {
          const int r = e / COLS, cc = e % COLS;
          tile[cc * HP + r] = c0 + cc < h ? src[b * hh + static_cast<int64_t>(r) * h + c0 + cc] : 0.f;
        }
        __syncthreads();
        if (part == p) {
#pragma unroll
          for (int rt = 0; rt < TPW; ++rt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int row = r0w + 32 * rt + 8 * (r >> 2) + 4 * g + (r & 3);
              hs[rt][r] = row < h ? tile[ncol * HP + row] : 0.f;
            }
        }
        __syncthreads();
      } else if (p == 0) {  // identity
#pragma unroll
        for (int rt = 0; rt < TPW; ++rt)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int row = r0w + 32 * rt + 8 * (r >> 2) + 4 * g + (r & 3);
            hs[rt][r] = (part == 0 && colok && row == col) ? 1.f : 0.f;
          }
      }
    }
  }
  // state scale: a power of two putting the largest start entry at most SMAX (columns keep
  // their norms under the unitary factors, so no later entry grows past it)
  float ssc, inv_ssc;
  {
    float mx = 0.f;
#pragma unroll
    for (int rt = 0; rt < TPW; ++rt)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, fabsf(hs[rt][r]));
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    float* red = &sm.wred[0][0];
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = 0.f;
#pragma unroll
    for (int w = 0; w < NWV; ++w) mx = fmaxf(mx, red[w]);
    __syncthreads();
    int e = 0;
    if (mx > 0.f && mx <= 3.0e38f) (void)frexpf(mx / SMAX, &e);  // mx / SMAX in [2^(e-1), 2^e)
    ssc = ldexpf(1.f, -e);
    inv_ssc = ldexpf(1.f, e);
#pragma unroll
    for (int rt = 0; rt < TPW; ++rt) hs[rt] *= ssc;
  }
  const bool snaps = snap_on && z == nstates - 1;
  auto write_snap = [&](int n) {
    if (!snaps || !colok) return;
    float* d = static_cast<float*>(snapv) + ((static_cast<int64_t>(b) * nch + n) * 2 + part) * h * HP +
               static_cast<int64_t>(col) * HP;
#pragma unroll
    for (int rt = 0; rt < TPW; ++rt)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int row = r0w + 32 * rt + 8 * q + 4 * g;
        *reinterpret_cast<float4*>(d + row) =
            make_float4(hs[rt][4 * q] * inv_ssc, hs[rt][4 * q + 1] * inv_ssc,
                        hs[rt][4 * q + 2] * inv_ssc, hs[rt][4 * q + 3] * inv_ssc);
      }
  };

  // ---- Y of a chunk, as the A operand of W = Y^T H: lane (rho = l32, g), tile rt, K-step ks
  // holds rows r0w + 32 rt + 16 ks + 4 g + {0..3} and + 8 + {0..3} of rank row rho (k or v of
  // token t0 + rho / 2): operand block (r0w + 32 rt + 16 ks) / 16 of the prep kernel's layout,
  // one contiguous 16-byte piece per lane; loaded a chunk ahead.
  typedef V8 YBuf[TPW][2];
  typedef V8 TBuf[2][2];
  // tile rt of the next chunk's operands; the tiles are requested at four points of the chunk
  // (tile rt after barrier rt) so that the loads do not queue up behind each other
  auto load_y = [&](int m, YBuf& yraw, int rt) {
    if (rt >= TPW) return;
    const E* src = yop + (static_cast<int64_t>(b) * nc + (m < nc ? m : nc - 1)) * (HP / 16) * 512 +
                   (r0w / 16) * 512 + lane * 8;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) yraw[rt][ks] = *reinterpret_cast<const V8*>(src + (2 * rt + ks) * 512);
  };
  // update operand offsets (transposing reads of the wave's Y block): rows
  // rho = 16 ks + 8 hh + 4 g + i, local rows 32 rt + 16 (lane / 16 & 1) + 4 r
  E* const ytw = &sm.yt[wave][0][0];
  const int offU = rho_slot(4 * g + (l16 >> 2)) * Y_LD + 16 * ((lane >> 4) & 1) + 4 * (l16 & 3);
  E* const ywr = ytw + rho_slot(l32) * Y_LD + 4 * g;

  // f16 snapshot in operand layout: the wave's rows go through its own Y block in LDS (state
  // column n in place of rank row n) and come back transposed by the update's reads, so every
  // store is a contiguous 1 KB.  The wave's later Y writes follow these reads in its own LDS
  // queue, so they cannot overtake them.
  auto write_snap16 = [&](int n) {
#pragma unroll
    for (int rt = 0; rt < TPW; ++rt)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        V4 hv;
#pragma unroll
        for (int e = 0; e < 4; ++e) hv[e] = static_cast<E>(hs[rt][4 * q + e] * inv_ssc);
        *reinterpret_cast<V4*>(ywr + 32 * rt + 8 * q) = hv;
      }
    E* d = static_cast<E*>(snapv) + static_cast<int64_t>(b * nch + n) * 2 * (HP / 32) * (HP / 16) * 512 +
           (static_cast<int64_t>(r0w / 32) * (HP / 16) + blockIdx.x) * 512 + lane * 8;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)  // ks = part (columns 16 ks .. 16 ks + 15 of the block)
#pragma unroll
      for (int rt = 0; rt < TPW; ++rt) {
        typedef short i16x4 __attribute__((ext_vector_type(4)));
        typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
        const E* pp = ytw + offU + ks * Y_LD + 32 * rt;
        const V4 a0 = __builtin_bit_cast(V4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(pp)));
        const V4 a1 = __builtin_bit_cast(V4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(pp + 2 * Y_LD)));
        *reinterpret_cast<V8*>(d + (static_cast<int64_t>(ks) * (HP / 32) * (HP / 16) + rt * (HP / 16)) * 512) =
            cat8<V4, V8>(a0, a1);
      }
  };

  // T operands of the Z waves (A of [[Re T, -Im T], [Im T, Re T]], rows 16 (wave & 1) + l16 of
  // part wave / 2, K-steps kst = 0, 1, hi and lo), loaded a chunk ahead
  const int zpart = (wave >> 1) & 1;
  const int mrow = 16 * (wave & 1) + l16;
  auto load_t = [&](int m, TBuf& tnext) {
    if (wave >= 4) return;
    const E* tb = tt + (static_cast<int64_t>(b) * nc + (m < nc ? m : 0)) * TT_STRIDE;
#pragma unroll
    for (int kst = 0; kst < 2; ++kst) {
      // kst 0 -> (part 0: Re T, 1: Im T); kst 1 -> (part 0: -Im T, 1: Re T)
      const int mat = (zpart == 0) == (kst == 0) ? 0 : 2;  // 0: Re T, 2: Im T
      const E* ar = tb + mat * RK * RK + mrow * RK + 8 * g4;
      tnext[kst][0] = *reinterpret_cast<const V8*>(ar);
      tnext[kst][1] = *reinterpret_cast<const V8*>(ar + RK * RK);
    }
  };
  // one chunk; (yraw, tcur) hold its prefetched operands, (ynext, tnext) receive the next
  // chunk's (two buffer sets used alternately, so no register copies between iterations)
  auto chunk = [&](int m, YBuf& yraw, TBuf& tcur, YBuf& ynext, TBuf& tnext) {
    V8 ya[TPW][2];
#pragma unroll
    for (int rt = 0; rt < TPW; ++rt)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        ya[rt][ks] = yraw[rt][ks];
    // the snapshot stores go after this chunk's operands have arrived, so that waiting for
    // those loads never waits for the stores
    asm volatile("" ::: "memory");
    if (m % cpc == 0) {
      if constexpr (S16) {
        if (snaps) write_snap16(m / cpc);
      } else {
        write_snap(m / cpc);
      }
    }
    asm volatile("" ::: "memory");
    load_t(m + 1, tnext);
    load_y(m + 1, ynext, 0);
    // the wave's Y rows into LDS for the update's transposing reads
#pragma unroll
    for (int rt = 0; rt < TPW; ++rt)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        *reinterpret_cast<V4*>(ywr + 32 * rt + 16 * ks) = __builtin_shufflevector(ya[rt][ks], ya[rt][ks], 0, 1, 2, 3);
        *reinterpret_cast<V4*>(ywr + 32 * rt + 16 * ks + 8) = __builtin_shufflevector(ya[rt][ks], ya[rt][ks], 4, 5, 6, 7);
      }
    // W partial = Y^T H over this wave's rows (H as hi + lo)
    f32x16 wacc = {};
#pragma unroll
    for (int rt = 0; rt < TPW; ++rt)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        float x[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = hs[rt][8 * ks + i];
        V8 hhi, hlo;
        split8p(x, hhi, hlo);
        wacc = MM::mma32(ya[rt][ks], hhi, wacc);
        wacc = MM::mma32(ya[rt][ks], hlo, wacc);
      }
    // lane (n, g) holds W[8 (r/4) + 4 g + r%4][n]
#pragma unroll
    for (int q = 0; q < 4; ++q)
      *reinterpret_cast<float4*>(&sm.wpart[wave][l32][8 * q + 4 * g]) =
          make_float4(wacc[4 * q], wacc[4 * q + 1], wacc[4 * q + 2], wacc[4 * q + 3]);
    __syncthreads();
    load_y(m + 1, ynext, 1);
    // reduction: wave w sums columns n = 4w .. 4w + 3 (lane: n = 4w + lane / 16, rho pair 2 (lane % 16))
    {
      const int n = 4 * wave + (lane >> 4), rp = 2 * (lane & 15);
      float2 s = make_float2(0.f, 0.f);
#pragma unroll
      for (int w = 0; w < NWV; ++w) {
        const float2 x = *reinterpret_cast<const float2*>(&sm.wpart[w][n][rp]);
        s.x += x.x;
        s.y += x.y;
      }
      *reinterpret_cast<float2*>(&sm.wred[n][rp]) = s;
    }
    __syncthreads();
    load_y(m + 1, ynext, 2);
    // Z = T W on waves 0..3: [Zr; Zi] (64 x 16) = [[Tr, -Ti], [Ti, Tr]] (64 x 64) [Wr; Wi];
    // wave wz computes rows 16 wz .. 16 wz + 15 (part wz / 2, rho 16 (wz & 1) + ..)
    if (wave < 4) {
      const int wz = wave;
      f32x4 zacc = {};
#pragma unroll
      for (int kst = 0; kst < 2; ++kst) {
        const bool neg = zpart == 0 && kst == 1;
        V8 ahi = tcur[kst][0];
        V8 alo = tcur[kst][1];
        if (neg) {
          ahi = -ahi;
          alo = -alo;
        }
        // B: [Wr; Wi] rows 32 kst + 8 g4 + 0..7 of column c = l16
        const float* wsrc = &sm.wred[l16 + 16 * kst][8 * g4];
        const float4 w0 = *reinterpret_cast<const float4*>(wsrc);
        const float4 w1 = *reinterpret_cast<const float4*>(wsrc + 4);
        const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
        V8 bhi, blo;
        split8p(wv, bhi, blo);
        zacc = MM::mma16(ahi, bhi, zacc);
        zacc = MM::mma16(ahi, blo, zacc);
        zacc = MM::mma16(alo, bhi, zacc);
      }
      // lane (c = l16, g4): rows 16 wz + 4 g4 + r -> Z'[rho = 16 (wz & 1) + 4 g4 + r][n = c + 16 zpart]
      V4 zh4, zl4;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float zv = zacc[r] * (1.f / TSCALE);
        zh4[r] = static_cast<E>(zv);
        zl4[r] = static_cast<E>(zv - static_cast<float>(zh4[r]));
      }
      const int n = l16 + 16 * zpart, rho0 = 16 * (wz & 1) + 4 * g4;
      *reinterpret_cast<V4*>(&sm.zh[n][rho0]) = zh4;
      *reinterpret_cast<V4*>(&sm.zl[n][rho0]) = zl4;
    }
    __syncthreads();
    load_y(m + 1, ynext, 3);
    // H += Y Z': A = Y rows (transposing reads), B = Z' rows rho = 16 ks + 8 (i/4) + 4 g + i%4
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const E* zhp = &sm.zh[l32][16 * ks + 4 * g];
      const E* zlp = &sm.zl[l32][16 * ks + 4 * g];
      const V8 bh = cat8<V4, V8>(*reinterpret_cast<const V4*>(zhp), *reinterpret_cast<const V4*>(zhp + 8));
      const V8 bl = cat8<V4, V8>(*reinterpret_cast<const V4*>(zlp), *reinterpret_cast<const V4*>(zlp + 8));
#pragma unroll
      for (int rt = 0; rt < TPW; ++rt) {
        typedef short i16x4 __attribute__((ext_vector_type(4)));
        typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
        const E* p = ytw + offU + ks * Y_LD + 32 * rt;
        const V4 a0 = __builtin_bit_cast(V4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p)));
        const V4 a1 = __builtin_bit_cast(V4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p + 2 * Y_LD)));
        const V8 ay = cat8<V4, V8>(a0, a1);
        hs[rt] = MM::mma32(ay, bh, hs[rt]);
        hs[rt] = MM::mma32(ay, bl, hs[rt]);
      }
    }
    // no barrier here: yt is per wave, the next W partials are written after barriers 2 and 3
    // (every wave's reads of this chunk's partials are done by then), and the next Z' and W
    // reductions are written after the next barrier 1, which every wave reaches only once
    // its update has read this chunk's Z'
  };
  YBuf ya0, ya1;
  TBuf ta0, ta1;
#pragma unroll
  for (int rt = 0; rt < TPW; ++rt) load_y(0, ya0, rt);
  load_t(0, ta0);
  for (int m = 0; m < nc; m += 2) {
    chunk(m, ya0, ta0, ya1, ta1);
    if (m + 1 < nc) chunk(m + 1, ya1, ta1, ya0, ta0);
  }
  __syncthreads();  // the tile below overlays Z' and the Y blocks of the last update
  // ---- final raw state (z == 0): row-major planes through LDS column tiles
  if (z == 0) {
    float* tile = &sm.wpart[0][0][0];
    for (int p = 0; p < 2; ++p) {
      if (part == p) {
#pragma unroll
        for (int rt = 0; rt < TPW; ++rt)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int row = r0w + 32 * rt + 8 * (r >> 2) + 4 * g + (r & 3);
            tile[ncol * HP + row] = hs[rt][r] * inv_ssc;
          }
      }
      __syncthreads();
      float* dst = p == 0 ? fr : fi;
      for (int e = tid; e < h * COLS; e += NTH) {
        const int r = e / COLS, cc = e % COLS;
        if (c0 + cc < h) dst[b * hh + static_cast<int64_t>(r) * h + c0 + cc] = tile[cc * HP + r];
      }
      __syncthreads();
    }
  }
}

// ---------------------------------------------------------------- 3: readout from the identity
// With no initial hologram every readout state is H_t itself, a product of unitary factors, so
// its entries are at most 1 in magnitude and f16 snapshots of it lose only relative precision
// 2^-11 (the output is rounded to 16 bits anyway).  Workgroup = 32 consecutive tokens of one
// sequence (X = their readout vectors, rows of both parts as fp32 MFMA accumulators, laid out
// like the column kernel's state with tokens in place of columns):
//   0. q' = tau_t q_t in f16 (tau_t a power of two putting max |q_t| in [16, 32), so that X and
//      the products below stay far inside the f16 range) as B operands in LDS;
//   1. X = S q' with S the snapshot at the start of the token's 128-token block
//      (v_mfma_f32_32x32x16_f16; A operands stream from the snapshot, one 1 KB block per load);
//   2. for every 16-token chunk c of the block up to the group's last token: X += Y_c Z,
//      Z = mask(T_c Y_c^T X) (the chunk factor I + Y T Y^T of cm_cols_kernel; a token of chunk c
//      keeps the rank rows of tokens up to itself, a token of a later chunk all of them, a token
//      of an earlier chunk none), with single f16 operands;
//   3. rec_t = Re(x_t) / tau_t through LDS to contiguous rows of the output.
constexpr int RG = 32;    // tokens per readout workgroup
constexpr int C2M = 128;  // tokens per f16 snapshot
constexpr int WP_LD = 68; // floats per token row of the W partials ([wave][token][part, rho])

template <int TPW>
struct alignas(16) ReadSmem {
  static constexpr int HP = NWV * 32 * TPW;
  union {
    E qb[HP / 16][64][8];  // phase 1
    struct {
      float wpart[NWV][RG][WP_LD];
      float wred[RG][WP_LD];
      E zs[2][RG][Z_LD];
    } p2;                  // phase 2
    uint16_t ot[RG][HP + 8];  // phase 3
  } u;
  E yt[NWV][RK][Y_LD];
  float tau[RG];
};

template <typename IO> __device__ __forceinline__ void unpack8(uint4 r, float* f);
template <> __device__ __forceinline__ void unpack8<bf16_t>(uint4 r, float* f) {
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(w[i] << 16);
    f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}
template <> __device__ __forceinline__ void unpack8<f16_t>(uint4 r, float* f) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const h2 v = __builtin_bit_cast(h2, w[i]);
    f[2 * i] = static_cast<float>(v[0]);
    f[2 * i + 1] = static_cast<float>(v[1]);
  }
}
template <typename IO> __device__ __forceinline__ uint16_t pack_io(float x);
template <> __device__ __forceinline__ uint16_t pack_io<bf16_t>(float x) {
  // v_cvt_pk_bf16_f32: round to nearest even like f32_to_bf16, without its branch
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
}
template <> __device__ __forceinline__ uint16_t pack_io<f16_t>(float x) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
}

// FUSED: q is read from the stacked projection (row b*T + t of `stride` elements, q at 0) and
// L2-normalised here (F.normalize, eps 1e-12) before the power-of-two scaling.
template <typename IO, int TPW, bool FUSED = false>
__global__ __launch_bounds__(NTH) void cm_read_kernel(const IO* __restrict__ q,
                                                      const E* __restrict__ snap,
                                                      const E* __restrict__ yop,
                                                      const E* __restrict__ tt,
                                                      IO* __restrict__ out, int B, int T, int h,
                                                      int64_t stride = 0) {
  constexpr int RPW = 32 * TPW, HP = NWV * RPW, NKB = HP / 16;
  __shared__ ReadSmem<TPW> sm;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int l32 = lane & 31, g = lane >> 5, l16 = lane & 15, g4 = lane >> 4;
  // work item: consecutive items (the groups of one snapshot) on one XCD (workgroup i runs on
  // XCD i % 8), so the snapshot they share is read into that XCD's L2 once
  const int ngrp = (T + RG - 1) / RG, total = B * ngrp, per = (total + 7) / 8;
  const int item = (blockIdx.x % 8) * per + blockIdx.x / 8;
  if (item >= total) return;  // the whole workgroup
  const int b = item / ngrp, t0 = (item % ngrp) * RG;
  const int nc = (T + CT - 1) / CT, nsn = (T + C2M - 1) / C2M, sn = t0 / C2M;
  const int r0w = wave * RPW;

  // ---- 0: q' as B operands: block kb, lane (t, g) holds features 16 kb + 8 (i/4) + 4 g + i%4
  {
    constexpr int FPT = HP / 16, NP = FPT / 8;  // features and 8-element pieces per thread
    const int t = tid >> 4, s = tid & 15;       // 16 threads per token
    const int tok = t0 + t;
    const IO* src = q + (static_cast<int64_t>(b) * T + (tok < T ? tok : 0)) * (FUSED ? stride : h);
    float x[NP][8];
    float mx = 0.f, ss = 0.f;
#pragma unroll
    for (int u = 0; u < NP; ++u) {
      const int f = s * FPT + 8 * u;  // h % 8 == 0: a piece is wholly in or out
      const uint4 raw = (tok < T && f < h) ? *reinterpret_cast<const uint4*>(src + f) : make_uint4(0, 0, 0, 0);
      unpack8<IO>(raw, x[u]);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        mx = fmaxf(mx, fabsf(x[u][e]));
        if constexpr (FUSED) ss = fmaf(x[u][e], x[u][e], ss);
      }
    }
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) {
      mx = fmaxf(mx, __shfl_xor(mx, o));
      if constexpr (FUSED) ss += __shfl_xor(ss, o);
    }
    if constexpr (FUSED) {  // the token's 16 threads hold its whole row: normalise it
      const float nq = 1.f / fmaxf(sqrtf(ss), 1e-12f);
      mx *= nq;
#pragma unroll
      for (int u = 0; u < NP; ++u)
#pragma unroll
        for (int e = 0; e < 8; ++e) x[u][e] *= nq;
    }
    int ex = 5;
    if (mx > 0.f && mx <= 3.0e38f) {
      (void)frexpf(mx, &ex);  // mx in [2^(ex-1), 2^ex)
    }
    const float tau = ldexpf(1.f, 5 - ex);  // tau mx in [16, 32); 1 for zero / non-finite rows
    if (s == 0) sm.tau[t] = tau;
#pragma unroll
    for (int u = 0; u < NP; ++u) {
      const int f = s * FPT + 8 * u, kb = f >> 4, hf = (f >> 3) & 1;
      V4 lo, hi;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        lo[e] = static_cast<E>(x[u][e] * tau);
        hi[e] = static_cast<E>(x[u][4 + e] * tau);
      }
      *reinterpret_cast<V4*>(&sm.u.qb[kb][t][4 * hf]) = lo;
      *reinterpret_cast<V4*>(&sm.u.qb[kb][t + 32][4 * hf]) = hi;
    }
  }
  __syncthreads();

  // ---- 1: X = S q' over the column blocks kb of the snapshot (blocks past h were not written)
  f32x16 X[2][TPW];
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int rt = 0; rt < TPW; ++rt) X[p][rt] = f32x16{};
  {
    const int nkb = (h + 15) / 16;
    const E* sb = snap + static_cast<int64_t>(b * nsn + sn) * 2 * (HP / 32) * NKB * 512 +
                  static_cast<int64_t>(r0w / 32) * NKB * 512 + lane * 8;
    typedef V8 ABuf[2][TPW];
    auto load_a = [&](int kb, ABuf& a) {
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int rt = 0; rt < TPW; ++rt)
          a[p][rt] = *reinterpret_cast<const V8*>(sb + (static_cast<int64_t>(p * (HP / 32) + rt) * NKB + kb) * 512);
    };
    auto step = [&](int kb, ABuf& a) {
      const V8 bq = *reinterpret_cast<const V8*>(&sm.u.qb[kb][lane][0]);
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int rt = 0; rt < TPW; ++rt) X[p][rt] = MM::mma32(a[p][rt], bq, X[p][rt]);
    };
    ABuf a0, a1;
    load_a(0, a0);
    for (int kb = 0; kb < nkb; kb += 2) {
      if (kb + 1 < nkb) load_a(kb + 1, a1);
      step(kb, a0);
      if (kb + 1 < nkb) {
        if (kb + 2 < nkb) load_a(kb + 2, a0);
        step(kb + 1, a1);
      }
    }
  }
  __syncthreads();  // phase 2 overlays the B operands

  // ---- 2: the chunk factors of the block up to the group's last token
  E* const ytw = &sm.yt[wave][0][0];
  const int offU = rho_slot(4 * g + (l16 >> 2)) * Y_LD + 16 * ((lane >> 4) & 1) + 4 * (l16 & 3);
  E* const ywr = ytw + rho_slot(l32) * Y_LD + 4 * g;
  const int zpart = (wave >> 1) & 1, mrow = 16 * (wave & 1) + l16, ztok = 16 * (wave >> 2);
  const int cb = sn * (C2M / CT), ce = min(nc - 1, (t0 + RG - 1) / CT);
  V8 ya[TPW][2];
  V8 ta[2];
  auto load_y = [&](int c) {
    const E* src = yop + (static_cast<int64_t>(b) * nc + c) * NKB * 512 + (r0w / 16) * 512 + lane * 8;
#pragma unroll
    for (int rt = 0; rt < TPW; ++rt)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) ya[rt][ks] = *reinterpret_cast<const V8*>(src + (2 * rt + ks) * 512);
  };
  auto load_t = [&](int c) {  // hi parts of T's real form, rows mrow of part zpart
    const E* tb = tt + (static_cast<int64_t>(b) * nc + c) * TT_STRIDE;
#pragma unroll
    for (int kst = 0; kst < 2; ++kst) {
      const int mat = (zpart == 0) == (kst == 0) ? 0 : 2;  // 0: Re T, 2: Im T
      ta[kst] = *reinterpret_cast<const V8*>(tb + mat * RK * RK + mrow * RK + 8 * g4);
    }
  };
  load_y(cb);
  load_t(cb);
  for (int c = cb; c <= ce; ++c) {
    // Y rows into the wave's LDS block for the update's transposing reads
#pragma unroll
    for (int rt = 0; rt < TPW; ++rt)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        *reinterpret_cast<V4*>(ywr + 32 * rt + 16 * ks) = __builtin_shufflevector(ya[rt][ks], ya[rt][ks], 0, 1, 2, 3);
        *reinterpret_cast<V4*>(ywr + 32 * rt + 16 * ks + 8) = __builtin_shufflevector(ya[rt][ks], ya[rt][ks], 4, 5, 6, 7);
      }
    // W partials = Y^T X over this wave's rows, both parts
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      f32x16 wacc = {};
#pragma unroll
      for (int rt = 0; rt < TPW; ++rt)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          V8 xb;
#pragma unroll
          for (int i = 0; i < 8; ++i) xb[i] = static_cast<E>(X[p][rt][8 * ks + i]);
          wacc = MM::mma32(ya[rt][ks], xb, wacc);
        }
      // lane (t, g) holds W_p[8 (r/4) + 4 g + r%4][t]
#pragma unroll
      for (int qq = 0; qq < 4; ++qq)
        *reinterpret_cast<float4*>(&sm.u.p2.wpart[wave][l32][32 * p + 8 * qq + 4 * g]) =
            make_float4(wacc[4 * qq], wacc[4 * qq + 1], wacc[4 * qq + 2], wacc[4 * qq + 3]);
    }
    if (c < ce) load_y(c + 1);  // ya is in LDS and consumed: fetch the next chunk's
    __syncthreads();
    {  // reduction: thread -> token tid / 16, rows 4 (tid % 16) .. + 3
      const int t = tid >> 4, r4 = 4 * (tid & 15);
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int w = 0; w < NWV; ++w) {
        const float4 x = *reinterpret_cast<const float4*>(&sm.u.p2.wpart[w][t][r4]);
        acc.x += x.x;
        acc.y += x.y;
        acc.z += x.z;
        acc.w += x.w;
      }
      *reinterpret_cast<float4*>(&sm.u.p2.wred[t][r4]) = acc;
    }
    __syncthreads();
    {  // Z tile: rows (zpart, 16 (wave & 1) .. + 15), tokens ztok .. ztok + 15
      f32x4 zacc = {};
#pragma unroll
      for (int kst = 0; kst < 2; ++kst) {
        V8 a = ta[kst];
        if (zpart == 0 && kst == 1) a = -a;
        const float* wsrc = &sm.u.p2.wred[ztok + l16][32 * kst + 8 * g4];
        const float4 w0 = *reinterpret_cast<const float4*>(wsrc);
        const float4 w1 = *reinterpret_cast<const float4*>(wsrc + 4);
        const V8 bw = {static_cast<E>(w0.x), static_cast<E>(w0.y), static_cast<E>(w0.z), static_cast<E>(w0.w),
                       static_cast<E>(w1.x), static_cast<E>(w1.y), static_cast<E>(w1.z), static_cast<E>(w1.w)};
        zacc = MM::mma16(a, bw, zacc);
      }
      if (c < ce) load_t(c + 1);
      // lane (token ztok + l16, g4): rho = 16 (wave & 1) + 4 g4 + r
      const int tl = ztok + l16, tg = t0 + tl, ct = tg / CT;
      V4 zv;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int rho = 16 * (wave & 1) + 4 * g4 + r;
        const bool keep = ct > c || (ct == c && c * CT + (rho >> 1) <= tg);
        zv[r] = keep ? static_cast<E>(zacc[r] * (1.f / TSCALE)) : static_cast<E>(0.f);
      }
      *reinterpret_cast<V4*>(&sm.u.p2.zs[zpart][tl][16 * (wave & 1) + 4 * g4]) = zv;
    }
    __syncthreads();
    // X_p += Y Z_p: A = Y rows (transposing reads), B = Z_p rows rho = 16 ks + 8 (i/4) + 4 g + i%4
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      V8 ay[TPW];
#pragma unroll
      for (int rt = 0; rt < TPW; ++rt) {
        typedef short i16x4 __attribute__((ext_vector_type(4)));
        typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
        const E* pp = ytw + offU + ks * Y_LD + 32 * rt;
        const V4 a0 = __builtin_bit_cast(V4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(pp)));
        const V4 a1 = __builtin_bit_cast(V4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(pp + 2 * Y_LD)));
        ay[rt] = cat8<V4, V8>(a0, a1);
      }
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const E* zp = &sm.u.p2.zs[p][l32][16 * ks + 4 * g];
        const V8 bz = cat8<V4, V8>(*reinterpret_cast<const V4*>(zp), *reinterpret_cast<const V4*>(zp + 8));
#pragma unroll
        for (int rt = 0; rt < TPW; ++rt) X[p][rt] = MM::mma32(ay[rt], bz, X[p][rt]);
      }
    }
    // no barrier: the next partials / reduction / Z' are written after barriers that every
    // wave reaches only once it has finished reading this chunk's (as in cm_cols_kernel)
  }
  __syncthreads();  // the output rows overlay Z'

  // ---- 3: rec_t = Re(x_t) / tau_t, transposed through LDS to contiguous output rows
  {
    const float it = 1.f / sm.tau[l32];
#pragma unroll
    for (int rt = 0; rt < TPW; ++rt)
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const int row = r0w + 32 * rt + 8 * qq + 4 * g;
        uint2 pk;
        pk.x = static_cast<uint32_t>(pack_io<IO>(X[0][rt][4 * qq] * it)) |
               (static_cast<uint32_t>(pack_io<IO>(X[0][rt][4 * qq + 1] * it)) << 16);
        pk.y = static_cast<uint32_t>(pack_io<IO>(X[0][rt][4 * qq + 2] * it)) |
               (static_cast<uint32_t>(pack_io<IO>(X[0][rt][4 * qq + 3] * it)) << 16);
        *reinterpret_cast<uint2*>(&sm.u.ot[l32][row]) = pk;
      }
  }
  __syncthreads();
  {
    const int t = tid >> 4, s = tid & 15, tok = t0 + t;
    if (tok < T) {
      IO* dst = out + (static_cast<int64_t>(b) * T + tok) * h;
      for (int f = 8 * s; f < h; f += 128)
        *reinterpret_cast<uint4*>(dst + f) = *reinterpret_cast<const uint4*>(&sm.u.ot[t][f]);
    }
  }
}

template <typename IO, int TPW>
hipError_t launch_typed(const IO* k, const IO* v, const float* coef, const float* i0r,
                        const float* i0i, const float* i1r, const float* i1i, float* snap,
                        float* fr, float* fi, int B, int T, int h, int nstates, int snap_on,
                        int c2, void* ws, hipStream_t stream) {
  const int nc = (T + CT - 1) / CT;
  E* tt = static_cast<E*>(ws);
  E* yop = tt + static_cast<int64_t>(B) * nc * TT_STRIDE;  // [B][nc][HP / 16][64][8] f16
  if (nc > 0) {
    hipLaunchKernelGGL((cm_prep_kernel<IO>), dim3(nc, B), dim3(64), 0, stream, k, v, coef, tt, yop, T, h,
                       NWV * 32 * TPW);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((cm_cols_kernel<TPW, false>), dim3((h + COLS - 1) / COLS, B, nstates), dim3(NTH), 0,
                     stream, yop, tt, i0r, i0i, i1r, i1i, snap, fr, fi, T, h, nstates,
                     snap_on, c2);
  return hipGetLastError();
}

// identity start: state carry with f16 snapshots every C2M tokens, then the chunked readout
template <typename IO, int TPW>
hipError_t launch_scan16(const IO* q, const IO* k, const IO* v, const float* coef, void* snap,
                         IO* out, float* fr, float* fi, int B, int T, int h, void* ws,
                         hipStream_t stream, bool fused = false, int64_t stride = 0) {
  const int nc = (T + CT - 1) / CT;
  if (nc == 0) return hipSuccess;
  E* tt = static_cast<E*>(ws);
  E* yop = tt + static_cast<int64_t>(B) * nc * TT_STRIDE;
  if (fused)
    hipLaunchKernelGGL((cm_prep_kernel<IO, true>), dim3(nc, B), dim3(64), 0, stream, k, v, coef, tt,
                       yop, T, h, NWV * 32 * TPW, stride);
  else
    hipLaunchKernelGGL((cm_prep_kernel<IO>), dim3(nc, B), dim3(64), 0, stream, k, v, coef, tt, yop,
                       T, h, NWV * 32 * TPW, int64_t{0});
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((cm_cols_kernel<TPW, true>), dim3((h + COLS - 1) / COLS, B, 1), dim3(NTH), 0,
                     stream, yop, tt, nullptr, nullptr, nullptr, nullptr, snap, fr, fi, T, h, 1, 1,
                     C2M);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int total = B * ((T + RG - 1) / RG);
  if (fused)
    hipLaunchKernelGGL((cm_read_kernel<IO, TPW, true>), dim3(8 * ((total + 7) / 8)), dim3(NTH), 0,
                       stream, q, static_cast<const E*>(snap), yop, tt, out, B, T, h, stride);
  else
    hipLaunchKernelGGL((cm_read_kernel<IO, TPW>), dim3(8 * ((total + 7) / 8)), dim3(NTH), 0, stream,
                       q, static_cast<const E*>(snap), yop, tt, out, B, T, h, int64_t{0});
  return hipGetLastError();
}

}  // namespace chamm

// Workspace of the MFMA state carry (T per chunk, the f16 k and v of every chunk in operand
// layout, hp features each), in bytes; hp = 256, 512 or 1024, the padded height of the wide route.
size_t cham_mfma_workspace_bytes(int64_t B, int64_t T, int64_t hp) {
  const int64_t nc = (T + chamm::CT - 1) / chamm::CT;
  return static_cast<size_t>(B * nc * (chamm::TT_STRIDE + chamm::RK * hp)) * sizeof(_Float16) + 256;
}

size_t cham_mfma_snap16_bytes(int64_t B, int64_t T, int64_t hp) {
  return static_cast<size_t>(B * ((T + chamm::C2M - 1) / chamm::C2M) * 2 * hp * hp) * sizeof(_Float16);
}

hipError_t launch_cham_mfma_scan(const void* q, const void* k, const void* v, int io_dtype,
                                 const float* coef, void* snap, void* out, float* fr, float* fi,
                                 int B, int T, int h, int hp, void* ws, hipStream_t stream) {
#define VMI_CS(IO, TPW)                                                                          \
  return chamm::launch_scan16<IO, TPW>(static_cast<const IO*>(q), static_cast<const IO*>(k),      \
                                       static_cast<const IO*>(v), coef, snap, static_cast<IO*>(out), \
                                       fr, fi, B, T, h, ws, stream)
  if (io_dtype == VMI_BF16) {
    if (hp == 256) VMI_CS(bf16_t, 1);
    if (hp == 512) VMI_CS(bf16_t, 2);
    VMI_CS(bf16_t, 4);
  }
  if (hp == 256) VMI_CS(f16_t, 1);
  if (hp == 512) VMI_CS(f16_t, 2);
  VMI_CS(f16_t, 4);
#undef VMI_CS
}

hipError_t launch_cham_mfma_scan_fused(const void* proj, int64_t stride, int io_dtype,
                                       const float* coef, void* snap, void* out, float* fr,
                                       float* fi, int B, int T, int h, int hp, void* ws,
                                       hipStream_t stream) {
#define VMI_CS(IO, TPW)                                                                          \
  return chamm::launch_scan16<IO, TPW>(static_cast<const IO*>(proj), static_cast<const IO*>(proj), \
                                       static_cast<const IO*>(proj), coef, snap, static_cast<IO*>(out), \
                                       fr, fi, B, T, h, ws, stream, true, stride)
  if (io_dtype == VMI_BF16) {
    if (hp == 256) VMI_CS(bf16_t, 1);
    if (hp == 512) VMI_CS(bf16_t, 2);
    VMI_CS(bf16_t, 4);
  }
  if (hp == 256) VMI_CS(f16_t, 1);
  if (hp == 512) VMI_CS(f16_t, 2);
  VMI_CS(f16_t, 4);
#undef VMI_CS
}

bool cham_mfma_usable(int io_dtype, int h, const void* k, const void* v) {
  return (io_dtype == VMI_BF16 || io_dtype == VMI_F16) && h > 128 && h <= 1024 && h % 8 == 0 &&
         (reinterpret_cast<uintptr_t>(k) & 15) == 0 && (reinterpret_cast<uintptr_t>(v) & 15) == 0;
}

hipError_t launch_cham_mfma_cols(const void* k, const void* v, int io_dtype, const float* coef,
                                 const float* i0r, const float* i0i, const float* i1r,
                                 const float* i1i, float* snap, float* fr, float* fi, int B,
                                 int T, int h, int hp, int nstates, int snap_on, int c2, void* ws,
                                 hipStream_t stream) {
#define VMI_CM(IO, TPW)                                                                         \
  return chamm::launch_typed<IO, TPW>(static_cast<const IO*>(k), static_cast<const IO*>(v), coef, \
                                      i0r, i0i, i1r, i1i, snap, fr, fi, B, T, h, nstates, snap_on, \
                                      c2, ws, stream)
  if (io_dtype == VMI_BF16) {
    if (hp == 256) VMI_CM(bf16_t, 1);
    if (hp == 512) VMI_CM(bf16_t, 2);
    VMI_CM(bf16_t, 4);
  }
  if (hp == 256) VMI_CM(f16_t, 1);
  if (hp == 512) VMI_CM(f16_t, 2);
  VMI_CM(f16_t, 4);
#undef VMI_CM
}

}  // namespace vmi
