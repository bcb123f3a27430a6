// Single-token CHAM step (decode) with the holographic state updated in place, for any
// holographic_dim h <= 1024.  Reference: the CHAM forward at seq_len 1
// (cham_memory.py:117-238) that the generator re-runs per token with the previous raw state
// as initial_hologram (hyper_generate.py:58-63, acd_engine.py:116-121); the reference returns
// a fresh state, this updates the caller's state in place (opt-in, like the SSSD step).
//
// Per item b (closed form as in cham_scan.hip): with the raw state H = Hr + i Hi,
//   a = k^T H,  b = v^T H             (complex row vectors: column sums over h rows)
//   H' = H + k (N11 a + N12 b) + v (N12 a + N22 b)
// and the readout rec = Re(NS_3(H') q).  Every factor is unitary, so NS_3(U H) = U NS_3(H):
// the readout state R = NS_3(H) evolves by the same update, R' = U R, and rec = Re(R' q) =
// Rr' q.  A caller whose H is unitary (a sequence that started from the identity) passes no
// R (then R = H); otherwise it carries R beside H (computed once by the Newton-Schulz
// retraction) and both are updated here.  That is O(h^2) per token instead of the 13
// applications of H^H H (or 28 dense h x h products) a fresh NS_3 per token takes.
//
// Bound: HBM (each state is read once and written once: 16 h^2 bytes per item and state,
// 8 flops per element).  Grid (h / 32 column blocks, B, number of states): columns evolve
// independently (a_j, b_j are sums over rows of column j), so a workgroup owns 32 columns of
// one state of one item (512 threads): thread (rg, cg) holds rows rg + (512 / (CB/4)) m and
// columns 4 cg .. 4 cg + 3 (float4; CB / 4 lanes cover a row piece of the block).  CB = 32
// (128-byte row pieces) up to h = 512, CB = 16 above (8 rows of both parts per thread: 64
// floats; 32 columns would need 128 and spill), and CB = 4 for 1024 < h <= 4096 (one float4
// column group, 512 row groups of 4 or 8 rows: the same 64 floats per thread, in 16-byte row
// pieces).  The readout sums over columns, so the readout-state workgroups write per-block
// partial sums of Rr' q; cham_step_finish_kernel adds them.  Token rows and gamma are read
// at item strides (ios, gs), so the holographic scan above h = 1024 runs this kernel once
// per token on the rows of its [B, T, h] inputs.
#include "cham_common.h"
#include "vmi_dispatch.h"

namespace vmi {
namespace chams {

using cham::NCoef;

constexpr int CB_MIN = 16;      // smallest column block up to h = 1024 (sizes the partials)
constexpr int CB_BIG = 4;       // column block above h = 2048 (8 from 1024 to 2048)
constexpr int H_BIG = 4096;     // largest h of the step kernels

// Where item b's state lives.  DenseItems: plane arrays [B, h, h] (real and imaginary
// separate).  SlotItems: the per-layer hologram pool of a decode state cache, slot s at
// pool + 2 s h^2 (real plane, then imaginary); item b reads slot in_slot[b] (-1: the
// identity) and writes slot out_slot[b] (copy-on-write when they differ), slots in the
// kernel arguments as for the SSSD step (vmi::SlotArgs).
struct DenseItems {
  static constexpr bool kSlotted = false;
};
struct SlotItems {
  static constexpr bool kSlotted = true;
  int32_t in_slot[kMaxSlotArgs];
  int32_t out_slot[kMaxSlotArgs];
};

struct ItemPtrs {
  const float* in_r;
  const float* in_i;
  float* out_r;
  float* out_i;
  bool identity;  // slotted item with no slot yet: the state is I (real), 0 (imaginary)
};
template <typename Map>
__device__ __forceinline__ ItemPtrs item_ptrs(const Map& map, float* re, float* im, int b,
                                              int64_t hh) {
  ItemPtrs p;
  if constexpr (Map::kSlotted) {
    const int si = map.in_slot[b], so = map.out_slot[b];
    p.identity = si < 0;
    p.in_r = re + 2 * static_cast<int64_t>(si < 0 ? 0 : si) * hh;
    p.in_i = p.in_r + hh;
    p.out_r = re + 2 * static_cast<int64_t>(so) * hh;
    p.out_i = p.out_r + hh;
  } else {
    (void)map;
    p.identity = false;
    p.in_r = p.out_r = re + static_cast<int64_t>(b) * hh;
    p.in_i = p.out_i = im + static_cast<int64_t>(b) * hh;
  }
  return p;
}
__device__ __forceinline__ float4 eye4(int r, int c0) {
  return make_float4(r == c0 ? 1.f : 0.f, r == c0 + 1 ? 1.f : 0.f, r == c0 + 2 ? 1.f : 0.f,
                     r == c0 + 3 ? 1.f : 0.f);
}

// EXACT: h == NT / 8 * RPT and h % 32 == 0, so every row and column of the block exists and
// the loads and stores need no guards (branches around them made the compiler serialise the
// loads and spill at 1024 threads).
// (h is then a compile-time constant, so every address is a base plus an immediate).
template <typename IO, typename GT, int NT, int CB, int RPT, bool EXACT, typename Map>
__global__ __launch_bounds__(NT) void cham_step_kernel(
    const IO* __restrict__ q, const IO* __restrict__ k, const IO* __restrict__ v,
    const GT* __restrict__ gamma, float* hr0, float* hi0, float* hr1, float* hi1,
    float* __restrict__ part, int h_arg, int nstates, const Map map, int64_t ios, int64_t gs) {
  constexpr int CGN = CB / 4;        // column groups of 4 columns (float4)
  const int h = EXACT ? NT / CGN * RPT : h_arg;
  constexpr int NRG = NT / CGN;  // row groups
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int cg = tid & (CGN - 1), rg = tid / CGN;
  // Below 32 columns, LG = 32 / CB blocks share each 128-byte line of a row.  Workgroups go to
  // the 8 XCDs round robin by linear id, so blocks x, x + 8, .. land on the same XCD (and L2):
  // they take the LG pieces of the same lines (column blocks LG c .. LG c + LG - 1).
  constexpr int LG = 32 / CB;
  const int bx = blockIdx.x;
  const int blk = (LG > 1 && gridDim.x % (8 * LG) == 0)
                      ? ((bx / (8 * LG)) * 8 + (bx & 7)) * LG + ((bx >> 3) % LG)
                      : bx;
  const int b = blockIdx.y, z = blockIdx.z;
  const int nblk = gridDim.x;
  const int c0 = blk * CB + 4 * cg;
  const bool readout = z == nstates - 1;
  float* __restrict__ sr = z == 0 ? hr0 : hr1;
  float* __restrict__ si = z == 0 ? hi0 : hi1;
  const int64_t hh = static_cast<int64_t>(h) * h;
  const int64_t tb = static_cast<int64_t>(b) * ios;  // this item's token row

  __shared__ float4 s_red[NT / 64][CB];  // per wave: (ar, ai, br, bi) of each column
  __shared__ float s_dot[NT / 64][3];

  // state rows rg + NRG m, columns c0 .. c0+3 (both parts); zero outside h.  Addresses are
  // the item's base (uniform) plus a 32-bit element offset (h^2 <= 2^20).
  float4 xr[RPT], xi[RPT];
  float kr[RPT], vr[RPT];
  const bool colok = c0 < h;  // h % 4 == 0 (checked by the host), so all four or none
  const ItemPtrs ip = item_ptrs(map, sr, si, b, hh);
  const IO* __restrict__ kb = k + tb;
  const IO* __restrict__ vb = v + tb;
  const int off0 = rg * h + c0;
#pragma unroll
  for (int m = 0; m < RPT; ++m) {
    const int r = rg + NRG * m;
    if (Map::kSlotted && ip.identity) {  // uniform over the workgroup
      xr[m] = (EXACT || (colok && r < h)) ? eye4(r, c0) : make_float4(0.f, 0.f, 0.f, 0.f);
      xi[m] = make_float4(0.f, 0.f, 0.f, 0.f);
      kr[m] = (EXACT || r < h) ? io<IO>::load(kb, r) : 0.f;
      vr[m] = (EXACT || r < h) ? io<IO>::load(vb, r) : 0.f;
    } else if constexpr (EXACT) {
      xr[m] = ld_stream4(ip.in_r + off0 + m * NRG * h);
      xi[m] = ld_stream4(ip.in_i + off0 + m * NRG * h);
      kr[m] = io<IO>::load(kb, r);
      vr[m] = io<IO>::load(vb, r);
    } else {
      xr[m] = make_float4(0.f, 0.f, 0.f, 0.f);
      xi[m] = xr[m];
      kr[m] = vr[m] = 0.f;
      if (r < h) {
        if (colok) {
          xr[m] = ld_stream4(ip.in_r + off0 + m * NRG * h);
          xi[m] = ld_stream4(ip.in_i + off0 + m * NRG * h);
        }
        kr[m] = io<IO>::load(kb, r);
        vr[m] = io<IO>::load(vb, r);
      }
    }
  }
  const float g = io<GT>::load(gamma, static_cast<int64_t>(b) * gs);
  float4 qc = make_float4(0.f, 0.f, 0.f, 0.f);
  if (readout && colok)
    qc = make_float4(io<IO>::load(q, tb + c0), io<IO>::load(q, tb + c0 + 1),
                     io<IO>::load(q, tb + c0 + 2), io<IO>::load(q, tb + c0 + 3));

  // Gram entries over all h rows (each row counted once: column group 0's lanes)
  float kk = 0.f, vv = 0.f, kv = 0.f;
  if (cg == 0) {
#pragma unroll
    for (int m = 0; m < RPT; ++m) {
      kk = fmaf(kr[m], kr[m], kk);
      vv = fmaf(vr[m], vr[m], vv);
      kv = fmaf(kr[m], vr[m], kv);
    }
  }
  // column partials a = k^T H, b = v^T H over this thread's rows
  float4 ar = make_float4(0.f, 0.f, 0.f, 0.f), ai = ar, br = ar, bi = ar;
#pragma unroll
  for (int m = 0; m < RPT; ++m) {
    ar.x = fmaf(kr[m], xr[m].x, ar.x); ar.y = fmaf(kr[m], xr[m].y, ar.y);
    ar.z = fmaf(kr[m], xr[m].z, ar.z); ar.w = fmaf(kr[m], xr[m].w, ar.w);
    ai.x = fmaf(kr[m], xi[m].x, ai.x); ai.y = fmaf(kr[m], xi[m].y, ai.y);
    ai.z = fmaf(kr[m], xi[m].z, ai.z); ai.w = fmaf(kr[m], xi[m].w, ai.w);
    br.x = fmaf(vr[m], xr[m].x, br.x); br.y = fmaf(vr[m], xr[m].y, br.y);
    br.z = fmaf(vr[m], xr[m].z, br.z); br.w = fmaf(vr[m], xr[m].w, br.w);
    bi.x = fmaf(vr[m], xi[m].x, bi.x); bi.y = fmaf(vr[m], xi[m].y, bi.y);
    bi.z = fmaf(vr[m], xi[m].z, bi.z); bi.w = fmaf(vr[m], xi[m].w, bi.w);
  }
  // sum over the wave's 8 row groups (lane bits 3..5), then over the waves in LDS
#pragma unroll
  for (int off = CGN; off <= 32; off <<= 1) {
    ar.x += __shfl_xor(ar.x, off); ar.y += __shfl_xor(ar.y, off);
    ar.z += __shfl_xor(ar.z, off); ar.w += __shfl_xor(ar.w, off);
    ai.x += __shfl_xor(ai.x, off); ai.y += __shfl_xor(ai.y, off);
    ai.z += __shfl_xor(ai.z, off); ai.w += __shfl_xor(ai.w, off);
    br.x += __shfl_xor(br.x, off); br.y += __shfl_xor(br.y, off);
    br.z += __shfl_xor(br.z, off); br.w += __shfl_xor(br.w, off);
    bi.x += __shfl_xor(bi.x, off); bi.y += __shfl_xor(bi.y, off);
    bi.z += __shfl_xor(bi.z, off); bi.w += __shfl_xor(bi.w, off);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    kk += __shfl_xor(kk, off);
    vv += __shfl_xor(vv, off);
    kv += __shfl_xor(kv, off);
  }
  if (lane < CGN) {  // columns 4cg + e: (ar, ai, br, bi)
    s_red[wave][4 * cg + 0] = make_float4(ar.x, ai.x, br.x, bi.x);
    s_red[wave][4 * cg + 1] = make_float4(ar.y, ai.y, br.y, bi.y);
    s_red[wave][4 * cg + 2] = make_float4(ar.z, ai.z, br.z, bi.z);
    s_red[wave][4 * cg + 3] = make_float4(ar.w, ai.w, br.w, bi.w);
  }
  if (lane == 0) {
    s_dot[wave][0] = kk; s_dot[wave][1] = vv; s_dot[wave][2] = kv;
  }
  __syncthreads();
  float4 A[4];  // (ar, ai, br, bi) of columns 4cg + e, summed over all rows
#pragma unroll
  for (int e = 0; e < 4; ++e) A[e] = s_red[0][4 * cg + e];
#pragma unroll
  for (int w = 1; w < NT / 64; ++w)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float4 x = s_red[w][4 * cg + e];
      A[e].x += x.x; A[e].y += x.y; A[e].z += x.z; A[e].w += x.w;
    }
  kk = s_dot[0][0]; vv = s_dot[0][1]; kv = s_dot[0][2];
#pragma unroll
  for (int w = 1; w < NT / 64; ++w) {
    kk += s_dot[w][0]; vv += s_dot[w][1]; kv += s_dot[w][2];
  }
  bool ok;
  const NCoef N = cham::cayley_n_guarded(g, kk, vv, kv, ok);
  if (!ok) {  // identity token: k, v read as zero (uniform over the workgroup)
#pragma unroll
    for (int m = 0; m < RPT; ++m) kr[m] = vr[m] = 0.f;
  }
  // C = N11 a + N12 b,  D = N12 a + N22 b (complex), per column
  float cr[4], ci[4], dr[4], di[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float4 s = A[e];  // (ar, ai, br, bi)
    cr[e] = N.n11r * s.x - N.n11i * s.y + N.n12r * s.z - N.n12i * s.w;
    ci[e] = N.n11r * s.y + N.n11i * s.x + N.n12r * s.w + N.n12i * s.z;
    dr[e] = N.n12r * s.x - N.n12i * s.y + N.n22r * s.z - N.n22i * s.w;
    di[e] = N.n12r * s.y + N.n12i * s.x + N.n22r * s.w + N.n22i * s.z;
    // identity token: the column sums were taken with the non-finite rows (NaN * 0 is NaN)
    if (!ok) cr[e] = ci[e] = dr[e] = di[e] = 0.f;
  }
  // update, store, readout partials
  float po[RPT];
#pragma unroll
  for (int m = 0; m < RPT; ++m) {
    const int r = rg + NRG * m;
    float4 yr = xr[m], yi = xi[m];
    yr.x = fmaf(kr[m], cr[0], fmaf(vr[m], dr[0], yr.x));
    yr.y = fmaf(kr[m], cr[1], fmaf(vr[m], dr[1], yr.y));
    yr.z = fmaf(kr[m], cr[2], fmaf(vr[m], dr[2], yr.z));
    yr.w = fmaf(kr[m], cr[3], fmaf(vr[m], dr[3], yr.w));
    yi.x = fmaf(kr[m], ci[0], fmaf(vr[m], di[0], yi.x));
    yi.y = fmaf(kr[m], ci[1], fmaf(vr[m], di[1], yi.y));
    yi.z = fmaf(kr[m], ci[2], fmaf(vr[m], di[2], yi.z));
    yi.w = fmaf(kr[m], ci[3], fmaf(vr[m], di[3], yi.w));
    if (EXACT || (colok && r < h)) {
      st_stream4(ip.out_r + off0 + m * NRG * h, yr);
      st_stream4(ip.out_i + off0 + m * NRG * h, yi);
    }
    po[m] = fmaf(yr.x, qc.x, fmaf(yr.y, qc.y, fmaf(yr.z, qc.z, yr.w * qc.w)));
  }
  if (readout) {
    // sum over the 8 column groups (lane bits 0..2): every lane of the group gets the row sum
#pragma unroll
    for (int m = 0; m < RPT; ++m) {
#pragma unroll
      for (int off = 1; off < CGN; off <<= 1) po[m] += __shfl_xor(po[m], off);
    }
    float* pp = part + (static_cast<int64_t>(b) * nblk + blk) * h;
#pragma unroll
    for (int m = 0; m < RPT; ++m) {
      const int r = rg + NRG * m;
      if (cg == (m & (CGN - 1)) && (EXACT || r < h)) pp[r] = po[m];
    }
  }
}

// h = 1024: 32-column blocks (full 128-byte row pieces) of 512 threads, 16 rows per thread.
// 16 rows of both parts (128 floats) do not fit in registers beside the rest, so rows
// rg + 64 m for m >= 8 pass through LDS (128 KiB per workgroup): loaded into registers,
// summed into the column partials, parked in LDS, and read back for the update.
// Fused mode (FUSED = true; reference cham_memory.py:128-155 at seq_len 1): q, k, v and the
// gamma logit of item b come from row b of the stacked projection proj = x [W_q; W_k; W_v;
// W_gamma]^T (passed as q; row stride `stride` elements): q at 0, k at h, v at 2h, the logit
// at 3h.  The kernel forms v = silu(v), normalises q, k, v (F.normalize: x / max(|x|, 1e-12),
// in fp32: the column sums are taken with the raw rows and scaled by the norms afterwards)
// and gamma = 0.1 sigmoid(logit) mask[b].
struct ChamFused {
  int64_t stride;
  const uint8_t* mask;  // per item (null: every item active)
};

template <typename IO, typename GT, typename Map, bool FUSED = false>
__global__ __launch_bounds__(512) void cham_step1024_kernel(
    const IO* __restrict__ q, const IO* __restrict__ k, const IO* __restrict__ v,
    const GT* __restrict__ gamma, float* hr0, float* hi0, float* hr1, float* hi1,
    float* __restrict__ part, int nstates, const Map map, ChamFused fz) {
  constexpr int NT = 512, H = 1024, CB = 32, CGN = 8, NRG = 64, RPT = 16, RR = 8;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int cg = tid & (CGN - 1), rg = tid / CGN;
  const int blk = blockIdx.x, b = blockIdx.y, z = blockIdx.z;
  const int nblk = gridDim.x;
  const int c0 = blk * CB + 4 * cg;
  const bool readout = z == nstates - 1;
  const ItemPtrs ip = item_ptrs(map, z == 0 ? hr0 : hr1, z == 0 ? hi0 : hi1, b,
                                static_cast<int64_t>(H) * H);
  const float* __restrict__ sr = ip.in_r;
  const float* __restrict__ si = ip.in_i;
  float* __restrict__ wr = ip.out_r;
  float* __restrict__ wi = ip.out_i;
  // item b's token row: q, k, v (fused: the three blocks of its projection row)
  const IO* __restrict__ qb = FUSED ? q + static_cast<int64_t>(b) * fz.stride
                                    : q + static_cast<int64_t>(b) * H;
  const IO* __restrict__ kb = FUSED ? qb + H : k + static_cast<int64_t>(b) * H;
  const IO* __restrict__ vb = FUSED ? qb + 2 * H : v + static_cast<int64_t>(b) * H;
  const int off0 = rg * H + c0;

  __shared__ float4 s_hold[RPT - RR][2][NT];  // rows m >= RR: real, imag
  __shared__ float4 s_red[NT / 64][CB];
  __shared__ float s_dot[NT / 64][4];

  float4 xr[RR], xi[RR];
  float kr[RPT], vr[RPT];
#pragma unroll
  for (int m = 0; m < RR; ++m) {
    if (Map::kSlotted && ip.identity) {
      xr[m] = eye4(rg + NRG * m, c0);
      xi[m] = make_float4(0.f, 0.f, 0.f, 0.f);
    } else {
      xr[m] = ld_stream4(sr + off0 + m * NRG * H);
      xi[m] = ld_stream4(si + off0 + m * NRG * H);
    }
  }
#pragma unroll
  for (int m = 0; m < RPT; ++m) {
    kr[m] = io<IO>::load(kb, rg + NRG * m);
    vr[m] = io<IO>::load(vb, rg + NRG * m);
  }
  float g;
  float qq = 0.f;  // fused: this thread's share of |q|^2 (entries tid and tid + 512)
  if constexpr (FUSED) {
    const float logit = io<IO>::load(qb, 3 * H);
    g = 0.1f / (1.f + expf(-logit)) * (fz.mask != nullptr ? static_cast<float>(fz.mask[b]) : 1.f);
    const float q0 = io<IO>::load(qb, tid), q1 = io<IO>::load(qb, tid + NT);
    qq = fmaf(q0, q0, q1 * q1);
  } else {
    g = io<GT>::load(gamma, b);
  }
  float4 qc = make_float4(0.f, 0.f, 0.f, 0.f);
  if (readout)
    qc = make_float4(io<IO>::load(qb, c0), io<IO>::load(qb, c0 + 1), io<IO>::load(qb, c0 + 2),
                     io<IO>::load(qb, c0 + 3));
  float4 ar = make_float4(0.f, 0.f, 0.f, 0.f), ai = ar, br = ar, bi = ar;
  auto acc = [&](float kx, float vx, const float4& yr, const float4& yi) {
    ar.x = fmaf(kx, yr.x, ar.x); ar.y = fmaf(kx, yr.y, ar.y);
    ar.z = fmaf(kx, yr.z, ar.z); ar.w = fmaf(kx, yr.w, ar.w);
    ai.x = fmaf(kx, yi.x, ai.x); ai.y = fmaf(kx, yi.y, ai.y);
    ai.z = fmaf(kx, yi.z, ai.z); ai.w = fmaf(kx, yi.w, ai.w);
    br.x = fmaf(vx, yr.x, br.x); br.y = fmaf(vx, yr.y, br.y);
    br.z = fmaf(vx, yr.z, br.z); br.w = fmaf(vx, yr.w, br.w);
    bi.x = fmaf(vx, yi.x, bi.x); bi.y = fmaf(vx, yi.y, bi.y);
    bi.z = fmaf(vx, yi.z, bi.z); bi.w = fmaf(vx, yi.w, bi.w);
  };
  __builtin_amdgcn_sched_barrier(0);
  {  // rows m >= RR: through registers into the partials and LDS
    float4 tr[RPT - RR], ti[RPT - RR];
#pragma unroll
    for (int m = RR; m < RPT; ++m) {
      if (Map::kSlotted && ip.identity) {
        tr[m - RR] = eye4(rg + NRG * m, c0);
        ti[m - RR] = make_float4(0.f, 0.f, 0.f, 0.f);
      } else {
        tr[m - RR] = ld_stream4(sr + off0 + m * NRG * H);
        ti[m - RR] = ld_stream4(si + off0 + m * NRG * H);
      }
    }
    if constexpr (FUSED) {  // silu, after the second batch of state loads is in flight
#pragma unroll
      for (int m = 0; m < RPT; ++m) vr[m] = vr[m] / (1.f + expf(-vr[m]));
    }
#pragma unroll
    for (int m = 0; m < RR; ++m) acc(kr[m], vr[m], xr[m], xi[m]);
#pragma unroll
    for (int m = RR; m < RPT; ++m) {
      acc(kr[m], vr[m], tr[m - RR], ti[m - RR]);
      s_hold[m - RR][0][tid] = tr[m - RR];
      s_hold[m - RR][1][tid] = ti[m - RR];
    }
  }
  float kk = 0.f, vv = 0.f, kv = 0.f;
  if (cg == 0) {
#pragma unroll
    for (int m = 0; m < RPT; ++m) {
      kk = fmaf(kr[m], kr[m], kk);
      vv = fmaf(vr[m], vr[m], vv);
      kv = fmaf(kr[m], vr[m], kv);
    }
  }
#pragma unroll
  for (int off = CGN; off <= 32; off <<= 1) {
    ar.x += __shfl_xor(ar.x, off); ar.y += __shfl_xor(ar.y, off);
    ar.z += __shfl_xor(ar.z, off); ar.w += __shfl_xor(ar.w, off);
    ai.x += __shfl_xor(ai.x, off); ai.y += __shfl_xor(ai.y, off);
    ai.z += __shfl_xor(ai.z, off); ai.w += __shfl_xor(ai.w, off);
    br.x += __shfl_xor(br.x, off); br.y += __shfl_xor(br.y, off);
    br.z += __shfl_xor(br.z, off); br.w += __shfl_xor(br.w, off);
    bi.x += __shfl_xor(bi.x, off); bi.y += __shfl_xor(bi.y, off);
    bi.z += __shfl_xor(bi.z, off); bi.w += __shfl_xor(bi.w, off);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    kk += __shfl_xor(kk, off);
    vv += __shfl_xor(vv, off);
    kv += __shfl_xor(kv, off);
    if constexpr (FUSED) qq += __shfl_xor(qq, off);
  }
  if (lane < CGN) {
    s_red[wave][4 * cg + 0] = make_float4(ar.x, ai.x, br.x, bi.x);
    s_red[wave][4 * cg + 1] = make_float4(ar.y, ai.y, br.y, bi.y);
    s_red[wave][4 * cg + 2] = make_float4(ar.z, ai.z, br.z, bi.z);
    s_red[wave][4 * cg + 3] = make_float4(ar.w, ai.w, br.w, bi.w);
  }
  if (lane == 0) {
    s_dot[wave][0] = kk; s_dot[wave][1] = vv; s_dot[wave][2] = kv; s_dot[wave][3] = qq;
  }
  __syncthreads();
  float4 A[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) A[e] = s_red[0][4 * cg + e];
#pragma unroll
  for (int w = 1; w < NT / 64; ++w)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float4 x = s_red[w][4 * cg + e];
      A[e].x += x.x; A[e].y += x.y; A[e].z += x.z; A[e].w += x.w;
    }
  kk = s_dot[0][0]; vv = s_dot[0][1]; kv = s_dot[0][2]; qq = s_dot[0][3];
#pragma unroll
  for (int w = 1; w < NT / 64; ++w) {
    kk += s_dot[w][0]; vv += s_dot[w][1]; kv += s_dot[w][2]; qq += s_dot[w][3];
  }
  float nk = 1.f, nv = 1.f;
  if constexpr (FUSED) {  // the sums of the normalised rows: scale by the norms
    nk = 1.f / fmaxf(sqrtf(kk), 1e-12f);
    nv = 1.f / fmaxf(sqrtf(vv), 1e-12f);
    const float nq = 1.f / fmaxf(sqrtf(qq), 1e-12f);
    kv = kv * nk * nv;
    kk = kk * nk * nk;
    vv = vv * nv * nv;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      A[e].x *= nk; A[e].y *= nk; A[e].z *= nv; A[e].w *= nv;
    }
    qc.x *= nq; qc.y *= nq; qc.z *= nq; qc.w *= nq;
  }
  bool ok;
  const NCoef N = cham::cayley_n_guarded(g, kk, vv, kv, ok);
  if (!ok) {
#pragma unroll
    for (int m = 0; m < RPT; ++m) kr[m] = vr[m] = 0.f;
  }
  float cr[4], ci[4], dr[4], di[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float4 s = A[e];
    cr[e] = N.n11r * s.x - N.n11i * s.y + N.n12r * s.z - N.n12i * s.w;
    ci[e] = N.n11r * s.y + N.n11i * s.x + N.n12r * s.w + N.n12i * s.z;
    dr[e] = N.n12r * s.x - N.n12i * s.y + N.n22r * s.z - N.n22i * s.w;
    di[e] = N.n12r * s.y + N.n12i * s.x + N.n22r * s.w + N.n22i * s.z;
    // identity token: the column sums were taken with the non-finite rows (NaN * 0 is NaN)
    if (!ok) cr[e] = ci[e] = dr[e] = di[e] = 0.f;
    if constexpr (FUSED) {  // H' = H + k^ c + v^ d with k^ = nk k, v^ = nv v: the raw rows
      cr[e] *= nk; ci[e] *= nk; dr[e] *= nv; di[e] *= nv;  // below, the norms folded in here
    }
  }
  float* pp = part + (static_cast<int64_t>(b) * nblk + blk) * H;
  auto upd = [&](int m, float4 yr, float4 yi) {
    yr.x = fmaf(kr[m], cr[0], fmaf(vr[m], dr[0], yr.x));
    yr.y = fmaf(kr[m], cr[1], fmaf(vr[m], dr[1], yr.y));
    yr.z = fmaf(kr[m], cr[2], fmaf(vr[m], dr[2], yr.z));
    yr.w = fmaf(kr[m], cr[3], fmaf(vr[m], dr[3], yr.w));
    yi.x = fmaf(kr[m], ci[0], fmaf(vr[m], di[0], yi.x));
    yi.y = fmaf(kr[m], ci[1], fmaf(vr[m], di[1], yi.y));
    yi.z = fmaf(kr[m], ci[2], fmaf(vr[m], di[2], yi.z));
    yi.w = fmaf(kr[m], ci[3], fmaf(vr[m], di[3], yi.w));
    st_stream4(wr + off0 + m * NRG * H, yr);
    st_stream4(wi + off0 + m * NRG * H, yi);
    if (readout) {  // this row's readout partial, summed over the 8 column groups
      float po = fmaf(yr.x, qc.x, fmaf(yr.y, qc.y, fmaf(yr.z, qc.z, yr.w * qc.w)));
#pragma unroll
      for (int off = 1; off < CGN; off <<= 1) po += __shfl_xor(po, off);
      if (cg == (m & (CGN - 1))) pp[rg + NRG * m] = po;
    }
  };
#pragma unroll
  for (int m = 0; m < RR; ++m) upd(m, xr[m], xi[m]);
  // keep the held rows' LDS reads after the register rows are stored (register pressure)
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int m = RR; m < RPT; ++m) upd(m, s_hold[m - RR][0][tid], s_hold[m - RR][1][tid]);
}

// out[b][i] = sum over the NB column blocks of the readout partials (io dtype), in block order.
// Four outputs per thread (16-byte loads; h % 4 == 0), 64 threads per workgroup; with NB
// (the block count, 32 at h = 1024) known, all NB loads of a thread are issued before the
// first add, so the partials cost one memory round trip (a runtime-length loop waited on
// each load: 9.2 us at B64 h1024).
template <typename IO, int NB>
__global__ __launch_bounds__(64) void cham_step_finish_kernel(const float* __restrict__ part,
                                                              IO* __restrict__ out, int h,
                                                              int nblk, int64_t os) {
  const int b = blockIdx.y;
  const int i = (blockIdx.x * 64 + threadIdx.x) * 4;
  if (i >= h) return;
  const float* pp = part + static_cast<int64_t>(b) * nblk * h + i;
  float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
  auto add = [&](const float4& x) { s.x += x.x; s.y += x.y; s.z += x.z; s.w += x.w; };
  (void)nblk;
  float4 x[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) x[j] = *reinterpret_cast<const float4*>(pp + static_cast<int64_t>(j) * h);
#pragma unroll
  for (int j = 0; j < NB; ++j) add(x[j]);
  IO* o = out + static_cast<int64_t>(b) * os + i;  // os: item stride of out (elements)
  io<IO>::store(o, 0, s.x);
  io<IO>::store(o, 1, s.y);
  io<IO>::store(o, 2, s.z);
  io<IO>::store(o, 3, s.w);
}

// The same for any block count: 1024 threads per 256 outputs, each of 16 thread slices sums
// its share of the blocks (16-byte loads, 8 in flight), then the slices are added in order
// through LDS (above h = 1024 there are up to 1024 blocks per output).
template <typename IO>
__global__ __launch_bounds__(1024) void cham_step_finish_sliced_kernel(
    const float* __restrict__ part, IO* __restrict__ out, int h, int nblk, int64_t os) {
  constexpr int NS = 16;
  __shared__ float4 acc[NS][64];
  const int b = blockIdx.y;
  const int og = threadIdx.x & 63, sl = threadIdx.x >> 6;
  const int i = (blockIdx.x * 64 + og) * 4;
  const int j0 = static_cast<int>(static_cast<int64_t>(nblk) * sl / NS);
  const int j1 = static_cast<int>(static_cast<int64_t>(nblk) * (sl + 1) / NS);
  float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
  if (i < h) {
    const float* pp = part + static_cast<int64_t>(b) * nblk * h + i;
    int j = j0;
    for (; j + 8 <= j1; j += 8) {
      float4 x[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) x[u] = *reinterpret_cast<const float4*>(pp + static_cast<int64_t>(j + u) * h);
#pragma unroll
      for (int u = 0; u < 8; ++u) { s.x += x[u].x; s.y += x[u].y; s.z += x[u].z; s.w += x[u].w; }
    }
    for (; j < j1; ++j) {
      const float4 x = *reinterpret_cast<const float4*>(pp + static_cast<int64_t>(j) * h);
      s.x += x.x; s.y += x.y; s.z += x.z; s.w += x.w;
    }
  }
  acc[sl][og] = s;
  __syncthreads();
  if (sl == 0 && i < h) {
    for (int u = 1; u < NS; ++u) {
      const float4 x = acc[u][og];
      s.x += x.x; s.y += x.y; s.z += x.z; s.w += x.w;
    }
    IO* o = out + static_cast<int64_t>(b) * os + i;
    io<IO>::store(o, 0, s.x);
    io<IO>::store(o, 1, s.y);
    io<IO>::store(o, 2, s.z);
    io<IO>::store(o, 3, s.w);
  }
}

template <typename IO>
hipError_t launch_finish(const float* part, void* out, int B, int h, int nblk, int64_t os,
                         hipStream_t stream) {
  const dim3 grid((h / 4 + 63) / 64, B);
  if (nblk == 32)
    hipLaunchKernelGGL((cham_step_finish_kernel<IO, 32>), grid, dim3(64), 0, stream, part,
                       static_cast<IO*>(out), h, nblk, os);
  else
    hipLaunchKernelGGL((cham_step_finish_sliced_kernel<IO>), grid, dim3(1024), 0, stream, part,
                       static_cast<IO*>(out), h, nblk, os);
  return hipGetLastError();
}

int step_block_cols(int h) {
  return h > 2048 ? CB_BIG : h > 1024 ? 8 : (h > 512 && h != 1024) ? 16 : 32;
}

// One step of B items.  Item b's q, k, v rows start at element b * ios of q, k, v, its gamma
// at b * gs, its output row at b * os of out (a single decode step: ios = os = h, gs = 1; a
// token of a [B, T, h] scan: ios = os = T h, gs = T, pointers offset to the token).
template <typename IO, typename GT, typename Map>
hipError_t launch_t(const void* q, const void* k, const void* v, const void* gamma, float* hr,
                    float* hi, float* rr, float* ri, void* out, int B, int h, float* part,
                    const Map& map, hipStream_t stream, int64_t ios, int64_t gs, int64_t os) {
  // h = 1024: the LDS-holding kernel with 32-column blocks (item strides h and 1 only); other h
  // above 512: 16-column blocks of 512 threads, 8 rows each (32 columns would need 16 rows per
  // thread and spill); above 1024: 4-column blocks, 4 or 8 rows per thread
  const int cb = step_block_cols(h);
  const int nblk = (h + cb - 1) / cb;
  const int nstates = rr ? 2 : 1;
  const dim3 grid(nblk, B, nstates);
  const IO* qq = static_cast<const IO*>(q);
  const IO* kq = static_cast<const IO*>(k);
  const IO* vq = static_cast<const IO*>(v);
  const GT* gg = static_cast<const GT*>(gamma);
#define VMI_CS(CB_, RPT_, EX_) \
  hipLaunchKernelGGL((cham_step_kernel<IO, GT, 512, CB_, RPT_, EX_, Map>), grid, dim3(512), 0, \
                     stream, qq, kq, vq, gg, hr, hi, rr, ri, part, h, nstates, map, ios, gs)

  if (h == 128) VMI_CS(32, 2, true);
  else if (h < 128) VMI_CS(32, 2, false);
  else if (h == 256) VMI_CS(32, 4, true);
  else if (h < 256) VMI_CS(32, 4, false);
  else if (h == 512) VMI_CS(32, 8, true);
  else if (h < 512) VMI_CS(32, 8, false);
  else if (h == 1024) {
    if (ios != h || gs != 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL((cham_step1024_kernel<IO, GT, Map>), grid, dim3(512), 0, stream, qq, kq, vq,
                       gg, hr, hi, rr, ri, part, nstates, map, ChamFused{});
  } else if (h < 1024) VMI_CS(16, 8, false);
  else if (h == 2048) VMI_CS(8, 8, true);
  else if (h < 2048) VMI_CS(8, 8, false);
  else if (h == H_BIG) VMI_CS(CB_BIG, 8, true);
  else VMI_CS(CB_BIG, 8, false);
#undef VMI_CS
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_finish<IO>(part, out, B, h, nblk, os, stream);
}

template <typename IO>
hipError_t launch_fused_t(const void* proj, int64_t stride, const uint8_t* mask, float* hr,
                         float* hi, float* rr, float* ri, void* out, int B, float* part,
                         hipStream_t stream) {
  constexpr int h = 1024, nblk = h / 32;
  const int nstates = rr ? 2 : 1;
  const IO* p = static_cast<const IO*>(proj);
  hipLaunchKernelGGL((cham_step1024_kernel<IO, IO, DenseItems, true>), dim3(nblk, B, nstates),
                     dim3(512), 0, stream, p, p, p, p, hr, hi, rr, ri, part, nstates,
                     DenseItems{}, ChamFused{stride, mask});
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_finish<IO>(part, out, B, h, nblk, h, stream);
}

}  // namespace chams

bool cham_step_fused_supported(int64_t h) { return h == 1024; }

hipError_t launch_cham_step_fused(const void* proj, int64_t proj_stride, int io_dtype,
                                  const uint8_t* mask, float* hr, float* hi, float* rr, float* ri,
                                  void* out, int B, void* workspace, hipStream_t stream) {
  float* part = static_cast<float*>(workspace);
  if (io_dtype == VMI_F32)
    return chams::launch_fused_t<float>(proj, proj_stride, mask, hr, hi, rr, ri, out, B, part,
                                        stream);
  if (io_dtype == VMI_BF16)
    return chams::launch_fused_t<bf16_t>(proj, proj_stride, mask, hr, hi, rr, ri, out, B, part,
                                         stream);
  return chams::launch_fused_t<f16_t>(proj, proj_stride, mask, hr, hi, rr, ri, out, B, part,
                                      stream);
}

size_t cham_step_workspace_bytes(int64_t B, int64_t h) {
  const int64_t cb = h > 2048 ? chams::CB_BIG : h > kChamMaxDim ? 8 : chams::CB_MIN;
  return static_cast<size_t>(B) * ((h + cb - 1) / cb) * h * sizeof(float);
}

bool cham_step_supported(int64_t h) {
  return h >= 1 && h % 4 == 0 && h <= chams::H_BIG;
}

template <typename Map>
hipError_t launch_cham_step_map(const void* q, const void* k, const void* v, const void* gamma,
                                int io_dtype, int gamma_dtype, float* hr, float* hi, float* rr,
                                float* ri, void* out, int B, int h, void* workspace, const Map& map,
                                hipStream_t stream, int64_t ios, int64_t gs, int64_t os) {
  float* part = static_cast<float*>(workspace);
#define VMI_GT(IO_)                                                                              \
  if (gamma_dtype == VMI_F32)                                                                  \
    return chams::launch_t<IO_, float, Map>(q, k, v, gamma, hr, hi, rr, ri, out, B, h, part, map, \
                                            stream, ios, gs, os);                              \
  if (gamma_dtype == VMI_BF16)                                                                 \
    return chams::launch_t<IO_, bf16_t, Map>(q, k, v, gamma, hr, hi, rr, ri, out, B, h, part, map, \
                                             stream, ios, gs, os);                             \
  return chams::launch_t<IO_, f16_t, Map>(q, k, v, gamma, hr, hi, rr, ri, out, B, h, part, map,   \
                                          stream, ios, gs, os);
  if (io_dtype == VMI_F32) { VMI_GT(float) }
  if (io_dtype == VMI_BF16) { VMI_GT(bf16_t) }
  VMI_GT(f16_t)
#undef VMI_GT
}

hipError_t launch_cham_step(const void* q, const void* k, const void* v, const void* gamma,
                            int io_dtype, int gamma_dtype, float* hr, float* hi, float* rr,
                            float* ri, void* out, int B, int h, void* workspace,
                            hipStream_t stream) {
  return launch_cham_step_map(q, k, v, gamma, io_dtype, gamma_dtype, hr, hi, rr, ri, out, B, h,
                              workspace, chams::DenseItems{}, stream, h, 1, h);
}

hipError_t launch_cham_step_slots(const void* q, const void* k, const void* v, const void* gamma,
                                  int io_dtype, int gamma_dtype, float* pool, const int32_t* in_slot,
                                  const int32_t* out_slot, void* out, int B, int h, void* workspace,
                                  hipStream_t stream) {
  chams::SlotItems map;
  for (int i = 0; i < B; ++i) {
    map.in_slot[i] = in_slot[i];
    map.out_slot[i] = out_slot[i];
  }
  return launch_cham_step_map(q, k, v, gamma, io_dtype, gamma_dtype, pool, pool, nullptr, nullptr,
                              out, B, h, workspace, map, stream, h, 1, h);
}

// ---------------------------------------------------------------------------------------------
// The holographic scan above h = 1024 (up to 4096, h % 4 == 0), where the chunked routes'
// register and LDS tiles end: the state starts as H_0 (or I) in the output buffers, the readout
// state R_0 = NS_3(H_0) (when H_0 is given) in the workspace, and every token is one step
// (the kernels above, one read and one write of each state per token) on its rows of the
// [B, T, h] inputs.  O(T h^2) memory traffic instead of the chunked routes' matrix-core
// products: a route for sizes the reference's own tiled fallback covers
// (launch_cham_triton_tiled, triton_kernels.py:477-597), not a fast path.
namespace chams {
__global__ __launch_bounds__(256) void eye_kernel(float* __restrict__ hr, float* __restrict__ hi,
                                                  int64_t n, int h) {
  const int64_t hh = static_cast<int64_t>(h) * h;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t e = i % hh;
    hr[i] = e / h == e % h ? 1.f : 0.f;
    hi[i] = 0.f;
  }
}
size_t elem_bytes(int dtype) { return dtype == VMI_F32 ? 4 : 2; }
size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }
}  // namespace chams

size_t cham_step_scan_workspace_bytes(int64_t B, int64_t h) {
  return chams::align256(cham_step_workspace_bytes(B, h)) +
         chams::align256(2 * static_cast<size_t>(B) * h * h * sizeof(float)) + ns_workspace_bytes(B, h);
}

hipError_t launch_cham_step_scan(const void* q, const void* k, const void* v, const void* gamma,
                                 int io_dtype, int gamma_dtype, const float* h0r,
                                 const float* h0i, void* out, float* hr_out, float* hi_out, int B,
                                 int T, int h, void* workspace, hipStream_t stream) {
  char* ws = static_cast<char*>(workspace);
  float* part = reinterpret_cast<float*>(ws);
  const int64_t hh = static_cast<int64_t>(h) * h;
  float* rr = reinterpret_cast<float*>(ws + chams::align256(cham_step_workspace_bytes(B, h)));
  float* ri = rr + B * hh;
  void* nsws = reinterpret_cast<char*>(rr) + chams::align256(2 * static_cast<size_t>(B) * hh * sizeof(float));
  const size_t sb = static_cast<size_t>(B) * hh * sizeof(float);
  hipError_t e;
  if (h0r != nullptr) {
    e = hipMemcpyAsync(hr_out, h0r, sb, hipMemcpyDeviceToDevice, stream);
    if (e == hipSuccess) e = hipMemcpyAsync(hi_out, h0i, sb, hipMemcpyDeviceToDevice, stream);
    if (e == hipSuccess) e = launch_ns_retraction(h0r, h0i, rr, ri, B, h, 3, nsws, stream);
  } else {
    hipLaunchKernelGGL(chams::eye_kernel, dim3(1024), dim3(256), 0, stream, hr_out, hi_out, B * hh, h);
    e = hipGetLastError();
  }
  if (e != hipSuccess) return e;
  const size_t ie = chams::elem_bytes(io_dtype), ge = chams::elem_bytes(gamma_dtype);
  const int64_t ts = static_cast<int64_t>(T) * h;  // item stride of q, k, v, out
  for (int t = 0; t < T; ++t) {
    const size_t o = static_cast<size_t>(t) * h * ie;
    e = launch_cham_step_map(static_cast<const char*>(q) + o, static_cast<const char*>(k) + o,
                             static_cast<const char*>(v) + o,
                             static_cast<const char*>(gamma) + static_cast<size_t>(t) * ge,
                             io_dtype, gamma_dtype, hr_out, hi_out, h0r ? rr : nullptr,
                             h0r ? ri : nullptr, static_cast<char*>(out) + o, B, h, part,
                             chams::DenseItems{}, stream, ts, T, ts);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace vmi
