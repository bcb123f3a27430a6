// Newton-Schulz unitary retraction on the 16-bit matrix cores, n a multiple of 128
// (reference: verace_v1/modules/cham_memory.py:21-51, :296-315; the fp32-MFMA kernel of
// cham_ns.hip serves every other n).
//
// One iteration, every product taken from the pre-update H = Hr + i Hi:
//   Gram:   P = Hr^T Hr + Hi^T Hi,  Q = Hr^T Hi - Hi^T Hr;   Dr = 3I - P,  Di = -Q
//   update: Hr' = (Hr Dr - Hi Di) / 2,  Hi' = (Hr Di + Hi Dr) / 2
// Each line is ONE launch of a complex GEMM: a workgroup computes both the real and the
// imaginary 128 x 128 output tile from the same staged operand panels (four real products).
// Dr is symmetric and Di antisymmetric, so the Gram launch computes only the tiles on and
// above the diagonal and writes each one twice (itself and its mirror).
//
// Precision: every fp32 operand x enters as an f16 pair, x * 256 = hi + lo (hi = f16(256 x),
// lo = f16(256 x - hi)), and each real product is hi*hi + hi*lo + lo*hi on
// v_mfma_f32_32x32x16_f16 with fp32 accumulation: the dropped lo*lo term is ~2^-22 of the
// product, the same order as fp32 rounding.  The scale keeps lo in f16's normal range for
// entries down to 2^-11 (smaller entries keep 2^-32 absolute resolution) and hi finite for
// entries below 255; NS converges only for singular values below sqrt(3), so entries of H
// and D stay far inside that.
//
// Operand layout ("F layout"), written by the split kernel and by every GEMM's epilogue: the
// MFMA A-operand fragments of an n x n matrix X, fragment (mb, kb) = 64 lanes x 8 f16 where
// lane l holds X[32 mb + l%32][16 kb + 8 (l/32) + j], j = 0..7, stored [mb][kb][hi, lo][lane]
// (2 KB per fragment pair), so every fragment load is one contiguous 1 KB.  The B operand of
// X Y is the A-operand fragment of Y^T, so the Gram H^T H reads F(H^T) for both operands and
// the update H D reads F(H) and F(D^T).  The update's epilogue writes F(H') (next update) and
// F(H'^T) (next Gram), the Gram's F(D^T); the last update also writes fp32 H'.
//
// Workgroup: 4 waves, 128 x 128 output tile (wave (wr, wc) owns the 64 x 64 quarter: 2 x 2
// blocks of 32 x 32, real and imaginary accumulators = 128 fp32 per lane).  K runs in steps
// of 16 through a 4-stage ring of 32 KB LDS stages filled by LDS-direct loads
// (global_load_lds_dwordx4, one per 1 KB fragment, 8 per wave per step); one LDS barrier per
// step.  Per step a wave issues 48 MFMAs (4 blocks x 4 real products x 3 split terms).
#include "vmi_common.h"
#include "vmi_dispatch.h"
#include "vmi_mfma.h"

namespace vmi {
namespace ns16 {

typedef _Float16 E;
typedef mfma_t<E> MM;
typedef MM::v8 V8;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int TM = 128;            // output tile side
constexpr int NT = 256;            // 4 waves
constexpr int FRAG = 512;          // f16 per fragment (64 lanes x 8)
constexpr int NSTAGE = 4;
constexpr int STAGE_FRAGS = 32;    // A and B: 4 blocks x (re, im) x (hi, lo)
constexpr float SC = 256.f;        // operand scale
constexpr float INV_SC2 = 1.f / (SC * SC);
constexpr int EP_LD = TM + 4;      // epilogue tile pitch (floats)
constexpr size_t SMEM = static_cast<size_t>(NSTAGE) * STAGE_FRAGS * FRAG * sizeof(E);  // 128 KB
static_assert(SMEM >= static_cast<size_t>(TM) * EP_LD * sizeof(float), "epilogue tile fits");

// f16 offset of fragment (mb, kb), half hl, in an F array with nkb = n / 16 k-blocks
__device__ __forceinline__ int64_t frag_off(int mb, int kb, int hl, int nkb) {
  return ((static_cast<int64_t>(mb) * nkb + kb) * 2 + hl) * FRAG;
}

// x -> (hi, lo) f16 pairs of SC x, stored as the lane's 16 bytes of a fragment pair
__device__ __forceinline__ void split_store(const float* x, float sign, E* dst, int lane) {
  V8 hi, lo;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float y = sign * SC * x[j];
    const E h = static_cast<E>(y);
    hi[j] = h;
    lo[j] = static_cast<E>(y - static_cast<float>(h));
  }
  *reinterpret_cast<V8*>(dst + lane * 8) = hi;
  *reinterpret_cast<V8*>(dst + FRAG + lane * 8) = lo;
}

// ---------------------------------------------------------------- split of the input
// blockIdx.z: bit 0 = part (re / im), bit 1 = layout (F(H) / F(H^T)); one wave per fragment.
__global__ __launch_bounds__(NT) void ns16_split_kernel(const float* __restrict__ hr,
                                                        const float* __restrict__ hi, E* dr,
                                                        E* di, E* tr, E* ti, int n) {
  const int nkb = n / 16, nmb = n / 32;
  const int f = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (f >= nmb * nkb) return;
  const int mb = f / nkb, kb = f - (f / nkb) * nkb, lane = threadIdx.x & 63;
  const int part = blockIdx.z & 1, trans = blockIdx.z >> 1;
  const int64_t nn = static_cast<int64_t>(n) * n;
  const float* src = (part ? hi : hr) + blockIdx.y * nn;
  E* dst = (trans ? (part ? ti : tr) : (part ? di : dr)) + blockIdx.y * 2 * nn;
  const int row = 32 * mb + (lane & 31), k0 = 16 * kb + 8 * (lane >> 5);
  float x[8];
  if (!trans) {
    const float4 a = *reinterpret_cast<const float4*>(src + static_cast<int64_t>(row) * n + k0);
    const float4 b = *reinterpret_cast<const float4*>(src + static_cast<int64_t>(row) * n + k0 + 4);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = src[static_cast<int64_t>(k0 + j) * n + row];  // H^T[row][k]
  }
  split_store(x, 1.f, dst + frag_off(mb, kb, 0, nkb), lane);
}

// ---------------------------------------------------------------- the complex GEMM
struct Args {
  const E* ar;  // A operand F arrays (re, im), batch stride 2 n^2
  const E* ai;
  const E* br;  // B operand: F arrays of Y^T (re, im)
  const E* bi;
  E* o1r;       // GRAM: F(D^T);  update: F(H')
  E* o1i;
  E* o2r;       // update: F(H'^T)
  E* o2i;
  float* fr;    // last update: fp32 H' (re, im), batch stride n^2
  float* fi;
  int n, batch, tiles_side, ntiles, total;  // total: batch * ntiles rounded up to 8
};

__device__ __forceinline__ unsigned lds_addr(const void* p) {
  return static_cast<unsigned>(reinterpret_cast<uintptr_t>(
      (__attribute__((address_space(3))) const char*)(p)));
}
// 64 lanes x 16 bytes from global memory straight into LDS at m0 (the wave's base); M0 is
// passed as an asm operand so the compiler adds no waits of its own around LDS accesses.
__device__ __forceinline__ void dma16(const void* g, unsigned lds) {
  const unsigned m0v = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"{m0}"(m0v), "v"(g) : "memory");
}
// s_waitcnt vmcnt(n) alone (expcnt 7 and lgkmcnt 15 mean no wait)
#define NS16_VMCNT(n) __builtin_amdgcn_s_waitcnt(0x0F70 | ((n) & 15) | (((n) >> 4) << 14))
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ V8 lds_frag(const E* base, int lane) {
  typedef __attribute__((address_space(3))) const V8 lds_v8;
  return *((lds_v8*)(base + lane * 8));
}
__device__ __forceinline__ V8 negate(V8 x) {
  return __builtin_bit_cast(V8, __builtin_bit_cast(u32x4, x) ^ 0x80008000u);
}

template <bool GRAM, bool LAST>
__global__ __launch_bounds__(NT) void ns16_gemm_kernel(Args a) {
  __shared__ __align__(16) unsigned char smem[SMEM];
  E* st = reinterpret_cast<E*>(smem);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wr = wave >> 1, wc = wave & 1;
  const int n = a.n, nkb = n / 16, T = a.tiles_side;

  // XCD-aware order: workgroups dispatched to one XCD (g mod 8) take consecutive tiles, so
  // the tiles of one matrix share that XCD's L2 copy of their operand panels
  const int g = blockIdx.x;
  const int v = (g & 7) * (a.total >> 3) + (g >> 3);
  if (v >= a.ntiles * a.batch) return;  // padding (uniform over the workgroup)
  const int mat = v / a.ntiles;
  int t = v - mat * a.ntiles, bi, bj;
  if (GRAM) {  // tiles bi <= bj, row by row
    bi = 0;
    while (t >= T - bi) { t -= T - bi; ++bi; }
    bj = bi + t;
  } else {
    bi = t / T;
    bj = t - bi * T;
  }
  const int64_t nn = static_cast<int64_t>(n) * n;
  const int64_t moff = static_cast<int64_t>(mat) * 2 * nn;

  // stage layout (fragments): [A: blk 4][re/im][hi/lo], then [B: blk 4][re/im][hi/lo]
  const E* asrc[2] = {a.ar + moff, a.ai + moff};
  const E* bsrc[2] = {a.br + moff, a.bi + moff};
  auto issue = [&](int ks, int s) {
    E* sb = st + s * STAGE_FRAGS * FRAG;
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int hl = 0; hl < 2; ++hl) {
        dma16(asrc[p] + frag_off(4 * bi + wave, ks, hl, nkb) + lane * 8,
              lds_addr(sb + ((wave * 2 + p) * 2 + hl) * FRAG));
        dma16(bsrc[p] + frag_off(4 * bj + wave, ks, hl, nkb) + lane * 8,
              lds_addr(sb + (16 + (wave * 2 + p) * 2 + hl) * FRAG));
      }
  };

  f32x16 P[2][2], Q[2][2];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y) {
      P[x][y] = f32x16{};
      Q[x][y] = f32x16{};
    }

  const int nk = nkb;
#pragma unroll
  for (int s = 0; s < NSTAGE - 1; ++s)
    if (s < nk) issue(s, s);
  for (int ks = 0; ks < nk; ++ks) {
    // this wave's loads of step ks are done once at most those of the next two steps remain
    const int ahead = nk - 1 - ks;
    if (ahead >= 2) NS16_VMCNT(16);
    else if (ahead == 1) NS16_VMCNT(8);
    else NS16_VMCNT(0);
    lds_barrier();  // every wave's step-ks loads landed; every wave is done with step ks-1
    if (ks + NSTAGE - 1 < nk) issue(ks + NSTAGE - 1, (ks + NSTAGE - 1) % NSTAGE);
    const E* sb = st + (ks % NSTAGE) * STAGE_FRAGS * FRAG;
    V8 arh[2], arl[2], aih[2], ail[2], brh[2], brl[2], bih[2], bil[2];
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      const int blk = 2 * wr + x;
      arh[x] = lds_frag(sb + ((blk * 2 + 0) * 2 + 0) * FRAG, lane);
      arl[x] = lds_frag(sb + ((blk * 2 + 0) * 2 + 1) * FRAG, lane);
      aih[x] = lds_frag(sb + ((blk * 2 + 1) * 2 + 0) * FRAG, lane);
      ail[x] = lds_frag(sb + ((blk * 2 + 1) * 2 + 1) * FRAG, lane);
    }
#pragma unroll
    for (int y = 0; y < 2; ++y) {
      const int blk = 2 * wc + y;
      brh[y] = lds_frag(sb + (16 + (blk * 2 + 0) * 2 + 0) * FRAG, lane);
      brl[y] = lds_frag(sb + (16 + (blk * 2 + 0) * 2 + 1) * FRAG, lane);
      bih[y] = lds_frag(sb + (16 + (blk * 2 + 1) * 2 + 0) * FRAG, lane);
      bil[y] = lds_frag(sb + (16 + (blk * 2 + 1) * 2 + 1) * FRAG, lane);
    }
    // GRAM: P += Ar Br + Ai Bi, Q += Ar Bi - Ai Br;  update: P += Ar Br - Ai Bi, Q += Ar Bi + Ai Br
    V8 nih[2], nil[2];
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      nih[x] = negate(aih[x]);
      nil[x] = negate(ail[x]);
    }
#define NS16_TERM(ACC, XH, XL, YH, YL)                                 \
  _Pragma("unroll") for (int x = 0; x < 2; ++x)                         \
  _Pragma("unroll") for (int y = 0; y < 2; ++y)                         \
    ACC[x][y] = MM::mma32(XH[x], YH[y], ACC[x][y]);                     \
  _Pragma("unroll") for (int x = 0; x < 2; ++x)                         \
  _Pragma("unroll") for (int y = 0; y < 2; ++y)                         \
    ACC[x][y] = MM::mma32(XH[x], YL[y], ACC[x][y]);                     \
  _Pragma("unroll") for (int x = 0; x < 2; ++x)                         \
  _Pragma("unroll") for (int y = 0; y < 2; ++y)                         \
    ACC[x][y] = MM::mma32(XL[x], YH[y], ACC[x][y]);
    NS16_TERM(P, arh, arl, brh, brl)
    NS16_TERM(Q, arh, arl, bih, bil)
    if constexpr (GRAM) {
      NS16_TERM(P, aih, ail, bih, bil)
      NS16_TERM(Q, nih, nil, brh, brl)
    } else {
      NS16_TERM(P, nih, nil, bih, bil)
      NS16_TERM(Q, aih, ail, brh, brl)
    }
#undef NS16_TERM
  }

  // ---- epilogue: each output tile through LDS (pitch EP_LD floats), then F-layout writes
  lds_barrier();  // every wave is done reading the stages
  float* ep = reinterpret_cast<float*>(smem);
  const int g2 = lane >> 5, l32 = lane & 31;
#pragma unroll
  for (int part = 0; part < 2; ++part) {
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int y = 0; y < 2; ++y) {
        const f32x16& acc = part == 0 ? P[x][y] : Q[x][y];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = 64 * wr + 32 * x + 8 * (r >> 2) + 4 * g2 + (r & 3);
          const int col = 64 * wc + 32 * y + l32;
          float val;
          if constexpr (GRAM) {  // Dr = 3I - P, Di = -Q
            val = -acc[r] * INV_SC2;
            if (part == 0 && bi == bj && row == col) val += 3.f;
          } else {
            val = 0.5f * INV_SC2 * acc[r];
          }
          ep[row * EP_LD + col] = val;
        }
      }
    lds_barrier();
    E* o1 = (part == 0 ? a.o1r : a.o1i) + moff;
    // transposed write: F(C^T) blocks (mb over the tile's columns, kb over its rows); wave w
    // takes column block w.  GRAM: into F(D^T) at (4 bj + w, 8 bi + kbl); update: F(H'^T).
    {
      E* dstT = GRAM ? o1 : (part == 0 ? a.o2r : a.o2i) + moff;
#pragma unroll 2
      for (int kbl = 0; kbl < 8; ++kbl) {
        float xv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) xv[j] = ep[(16 * kbl + 8 * g2 + j) * EP_LD + 32 * wave + l32];
        split_store(xv, 1.f, dstT + frag_off(4 * bj + wave, 8 * bi + kbl, 0, nkb), lane);
      }
    }
    // direct write: F(C) blocks (mb over rows, kb over columns); wave w takes row block w.
    // GRAM: the mirror tile of F(D^T) (Dr symmetric: +, Di antisymmetric: -), off the diagonal
    // only; update: F(H').
    if (!GRAM || bi < bj) {
      const float sign = (GRAM && part == 1) ? -1.f : 1.f;
#pragma unroll 2
      for (int kbl = 0; kbl < 8; ++kbl) {
        const float* src = ep + (32 * wave + l32) * EP_LD + 16 * kbl + 8 * g2;
        float xv[8];
        const float4 p0 = *reinterpret_cast<const float4*>(src);
        const float4 p1 = *reinterpret_cast<const float4*>(src + 4);
        xv[0] = p0.x; xv[1] = p0.y; xv[2] = p0.z; xv[3] = p0.w;
        xv[4] = p1.x; xv[5] = p1.y; xv[6] = p1.z; xv[7] = p1.w;
        split_store(xv, sign, o1 + frag_off(4 * bi + wave, 8 * bj + kbl, 0, nkb), lane);
      }
    }
    if constexpr (LAST) {  // fp32 H' rows
      float* f = (part == 0 ? a.fr : a.fi) + static_cast<int64_t>(mat) * nn;
#pragma unroll 4
      for (int i = tid; i < TM * TM / 4; i += NT) {
        const int row = i / (TM / 4), c4 = i - row * (TM / 4);
        *reinterpret_cast<float4*>(f + static_cast<int64_t>(TM * bi + row) * n + TM * bj + 4 * c4) =
            *reinterpret_cast<const float4*>(ep + row * EP_LD + 4 * c4);
      }
    }
    lds_barrier();  // before the next part overwrites the tile
  }
}

}  // namespace ns16

bool ns16_usable(int64_t n) { return n >= ns16::TM && n % ns16::TM == 0 && n <= 4096; }

size_t ns16_workspace_bytes(int64_t batch, int64_t n) {
  // F(H) twice (ping-pong), F(H^T), F(D^T); each re + im, 2 n^2 f16 per part
  return static_cast<size_t>(8) * batch * 2 * n * n * sizeof(_Float16);
}

hipError_t launch_ns16_retraction(const float* h_real, const float* h_imag, float* out_real,
                                  float* out_imag, int batch, int n, int steps, void* workspace,
                                  hipStream_t stream) {
  using namespace ns16;
  const int64_t arr = static_cast<int64_t>(batch) * 2 * n * n;  // f16 per F array
  E* w = static_cast<E*>(workspace);
  E* hd[2][2] = {{w, w + arr}, {w + 2 * arr, w + 3 * arr}};  // [ping-pong][re, im]
  E* ht[2] = {w + 4 * arr, w + 5 * arr};
  E* dt[2] = {w + 6 * arr, w + 7 * arr};
  const int nfr = (n / 32) * (n / 16);
  hipLaunchKernelGGL(ns16_split_kernel, dim3((nfr + 3) / 4, batch, 4), dim3(NT), 0, stream,
                     h_real, h_imag, hd[0][0], hd[0][1], ht[0], ht[1], n);
  hipError_t e = hipGetLastError();
  const int T = n / TM;
  for (int s = 0; s < steps && e == hipSuccess; ++s) {
    const int cur = s & 1, nxt = cur ^ 1;
    Args g{};
    g.n = n;
    g.batch = batch;
    g.tiles_side = T;
    // Gram: A = B = F(H^T)
    g.ar = ht[0]; g.ai = ht[1]; g.br = ht[0]; g.bi = ht[1];
    g.o1r = dt[0]; g.o1i = dt[1];
    g.ntiles = T * (T + 1) / 2;
    g.total = (g.ntiles * batch + 7) / 8 * 8;
    hipLaunchKernelGGL((ns16_gemm_kernel<true, false>), dim3(g.total), dim3(NT), 0, stream, g);
    e = hipGetLastError();
    if (e != hipSuccess) break;
    // update: A = F(H), B = F(D^T); writes F(H') into the other buffer and F(H'^T) over F(H^T)
    Args u{};
    u.n = n;
    u.batch = batch;
    u.tiles_side = T;
    u.ar = hd[cur][0]; u.ai = hd[cur][1]; u.br = dt[0]; u.bi = dt[1];
    u.o1r = hd[nxt][0]; u.o1i = hd[nxt][1]; u.o2r = ht[0]; u.o2i = ht[1];
    u.fr = out_real; u.fi = out_imag;
    u.ntiles = T * T;
    u.total = (u.ntiles * batch + 7) / 8 * 8;
    if (s + 1 == steps)
      hipLaunchKernelGGL((ns16_gemm_kernel<false, true>), dim3(u.total), dim3(NT), 0, stream, u);
    else
      hipLaunchKernelGGL((ns16_gemm_kernel<false, false>), dim3(u.total), dim3(NT), 0, stream, u);
    e = hipGetLastError();
  }
  return e;
}

}  // namespace vmi
