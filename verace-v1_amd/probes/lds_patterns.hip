// LDS access-pattern microbenchmark for csrc/sssd_chunk.hip (measurement program, not part
// of the library).  Each kernel replays one LDS access pattern of sssd_chunk_kernel (the same
// offset formulas) NIT times in one wave per workgroup (four for the stash writes); run under
//   rocprofv3 --pmc SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE SQ_INSTS_LDS -- ./lds_patterns
// and divide the counters per kernel by SQ_INSTS_LDS to get LDS cycles (and bank-conflict
// cycles) per instruction of that pattern.  Build:
//   hipcc --offload-arch=gfx950 -O3 -std=c++17 -Xclang -target-feature -Xclang -packed-fp32-ops \
//         lds_patterns.hip -o lds_patterns
// All offsets stay inside `buf` (checked against BUF below for every pattern).
#include <hip/hip_runtime.h>
#include <cstdio>

typedef _Float16 E;
typedef E v4h __attribute__((ext_vector_type(4)));
typedef E v8h __attribute__((ext_vector_type(8)));
constexpr int D = 128, C = 16, R = 32;
constexpr int U_LD = D + 4, Q_LD = D + 8, Q_OFF = R * U_LD, CHUNK_ELEMS = Q_OFF + C * Q_LD;
constexpr int TT_LD = R + 4, PST_LD = D + 4, ZST_LD = R + 4;
constexpr int BUF = 17000;  // elements (>= 128 * PST_LD = 16896, >= CHUNK_ELEMS, >= 32 * TT_LD)
__host__ __device__ constexpr int rho_slot(int rho) {
  return ((rho & 1) << 3) | ((rho & 2) << 3) | (rho & 4) | ((rho & 8) >> 2) | ((rho & 16) >> 4);
}
__host__ __device__ constexpr int j_slot(int j) {
  return ((j & 1) << 2) | ((j & 2) << 2) | ((j & 4) >> 2) | ((j & 8) >> 2) | (j & 16);
}
constexpr int NIT = 2048;

__device__ __forceinline__ v4h rd4(const E* p) { return *reinterpret_cast<const v4h*>(p); }
__device__ __forceinline__ v4h tr4(const E* p) {
  typedef short i16x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  return __builtin_bit_cast(v4h, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p)));
}
__device__ __forceinline__ float fold(v4h x) { return (float)x[0] + (float)x[1] + (float)x[2] + (float)x[3]; }

#define PROLOGUE                                     \
  __shared__ E buf[BUF];                             \
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6; \
  const int l32 = lane & 31, g = lane >> 5, l16 = lane & 15, g4 = lane >> 4; \
  for (int i = threadIdx.x; i < BUF; i += blockDim.x) buf[i] = (E)(float)(i & 7); \
  __syncthreads();                                   \
  float acc = 0.f;                                   \
  (void)l32; (void)g; (void)l16; (void)g4; (void)wave;
#define EPILOGUE __syncthreads(); acc += (float)buf[(threadIdx.x * 37) % BUF]; out[blockIdx.x * blockDim.x + threadIdx.x] = acc;

// consumer W operand: rows rho = l32, features 32rt + 16ks + 4g (+8)
__global__ void k_consW(float* out) {
  PROLOGUE
  const int offW = rho_slot(l32) * U_LD + 4 * g;
  for (int it = 0; it < NIT; ++it) {
    const int rt = it & 3, ks = (it >> 2) & 1;
    const E* p = buf + offW + 32 * rt + 16 * ks;
    acc += fold(rd4(p)) + fold(rd4(p + 8));
    __builtin_amdgcn_s_waitcnt(0xC07F);
  }
  EPILOGUE
}
// consumer T~ operand
__global__ void k_consTT(float* out) {
  PROLOGUE
  for (int it = 0; it < NIT; ++it) {
    const int ks = it & 1;
    const E* th = buf + l32 * TT_LD + 16 * ks + 4 * g;
    acc += fold(rd4(th)) + fold(rd4(th + 8));
    __builtin_amdgcn_s_waitcnt(0xC07F);
  }
  EPILOGUE
}
// consumer update operand (transposing reads of U)
__global__ void k_consUU(float* out) {
  PROLOGUE
  const int offU = rho_slot(4 * g + (l16 >> 2)) * U_LD + 16 * ((lane >> 4) & 1) + 4 * (l16 & 3);
  for (int it = 0; it < NIT; ++it) {
    const int rt = it & 3, ks = (it >> 2) & 1;
    const E* p = buf + offU + ks * U_LD + 32 * rt;
    acc += fold(tr4(p)) + fold(tr4(p + 2 * U_LD));
    __builtin_amdgcn_s_waitcnt(0xC07F);
  }
  EPILOGUE
}
// consumer stash writes (4 waves)
__global__ void k_pstW(float* out) {
  PROLOGUE
  E* const pw = buf + (32 * wave + j_slot(l32)) * PST_LD + 4 * g;
  v4h x = {(E)1.f, (E)2.f, (E)3.f, (E)(float)lane};
  for (int it = 0; it < NIT; ++it) {
    const int rt = it & 3, ks = (it >> 2) & 1;
    *reinterpret_cast<v4h*>(pw + 32 * rt + 16 * ks) = x;
    *reinterpret_cast<v4h*>(pw + 32 * rt + 16 * ks + 8) = x;
    x[0] += (E)1.f;
    __builtin_amdgcn_s_waitcnt(0xC07F);
  }
  acc = (float)x[0];
  EPILOGUE
}
__global__ void k_zstW(float* out) {
  PROLOGUE
  E* const zw = buf + (32 * wave + j_slot(l32)) * ZST_LD + 4 * g;
  v4h x = {(E)1.f, (E)2.f, (E)3.f, (E)(float)lane};
  for (int it = 0; it < NIT; ++it) {
    const int ks = it & 1;
    *reinterpret_cast<v4h*>(zw + 16 * ks) = x;
    *reinterpret_cast<v4h*>(zw + 16 * ks + 8) = x;
    x[0] += (E)1.f;
    __builtin_amdgcn_s_waitcnt(0xC07F);
  }
  acc = (float)x[0];
  EPILOGUE
}
// readout (2 waves): stash reads, q, U
__global__ void k_rdPST(float* out) {
  PROLOGUE
  const int pg = 2 * (g4 & 1) + (g4 >> 1), rw = wave & 1;
  const E* pst_rd = buf + j_slot(8 * pg + (l16 >> 2)) * PST_LD + 64 * rw + 4 * (l16 & 3);
  for (int it = 0; it < NIT; ++it) {
    const int ks = it & 3, tl = (it >> 2) & 3;
    const E* p = pst_rd + 32 * ks * PST_LD + 16 * tl;
    acc += fold(tr4(p)) + fold(tr4(p + PST_LD));
    __builtin_amdgcn_s_waitcnt(0xC07F);
  }
  EPILOGUE
}
__global__ void k_rdZST(float* out) {
  PROLOGUE
  const int pg = 2 * (g4 & 1) + (g4 >> 1);
  const E* zst_rd = buf + j_slot(8 * pg + (l16 >> 2)) * ZST_LD + 4 * (l16 & 3);
  for (int it = 0; it < NIT; ++it) {
    const int ks = it & 3, yy = (it >> 2) & 1;
    const E* p = zst_rd + 32 * ks * ZST_LD + 16 * yy;
    acc += fold(tr4(p)) + fold(tr4(p + ZST_LD));
    __builtin_amdgcn_s_waitcnt(0xC07F);
  }
  EPILOGUE
}
__global__ void k_rdQ(float* out) {
  PROLOGUE
  const int pg = 2 * (g4 & 1) + (g4 >> 1);
  const int offQ = Q_OFF + l16 * Q_LD + 8 * pg;
  for (int it = 0; it < NIT; ++it) {
    const int ks = it & 3;
    const v8h x = *reinterpret_cast<const v8h*>(buf + offQ + 32 * ks);
    acc += (float)x[0] + (float)x[7];
    __builtin_amdgcn_s_waitcnt(0xC07F);
  }
  EPILOGUE
}
__global__ void k_rdU(float* out) {
  PROLOGUE
  const int rw = wave & 1;
  const int offO = rho_slot(4 * g4 + (l16 >> 2)) * U_LD + 64 * rw + 4 * (l16 & 3);
  for (int it = 0; it < NIT; ++it) {
    const int tl = it & 3;
    acc += fold(tr4(buf + offO + 16 * tl)) + fold(tr4(buf + offO + U_LD + 16 * tl));
    __builtin_amdgcn_s_waitcnt(0xC07F);
  }
  EPILOGUE
}
// producer writes of U rows and q rows (16 B per lane)
__global__ void k_prKV(float* out) {
  PROLOGUE
  E* tdst = buf + rho_slot(l32) * U_LD;
  uint4 x = make_uint4(lane, 1, 2, 3);
  for (int it = 0; it < NIT; ++it) {
    const int ks = it & 7;
    *reinterpret_cast<uint4*>(tdst + 16 * ks + 8 * g) = x;
    x.y += 1;
    __builtin_amdgcn_s_waitcnt(0xC07F);
  }
  acc = (float)x.y;
  EPILOGUE
}
__global__ void k_prQ(float* out) {
  PROLOGUE
  uint4 x = make_uint4(lane, 1, 2, 3);
  for (int it = 0; it < NIT; ++it) {
    const int m = it & 3, e = lane + 64 * m;
    *reinterpret_cast<uint4*>(buf + Q_OFF + (e >> 4) * Q_LD + 8 * (e & 15)) = x;
    x.y += 1;
    __builtin_amdgcn_s_waitcnt(0xC07F);
  }
  acc = (float)x.y;
  EPILOGUE
}
// producer T~ pair writes (32-bit): element (ea, eb) of the 8x8 blocks, then the 16x16 block
__global__ void k_prTT(float* out) {
  PROLOGUE
  const int ea = lane >> 3, eb = lane & 7;
  const bool odd = lane & 1;
  uint32_t* const tw = reinterpret_cast<uint32_t*>(odd ? buf + 32 * TT_LD + 8 : buf);
  const int brow[6] = {0, 1, 2, 3, 1, 3}, bcol[6] = {0, 1, 2, 3, 0, 2};
  uint32_t v = lane;
  for (int it = 0; it < NIT; ++it) {
    const int i = it % 10;
    int row, col;
    if (i < 6) { row = 8 * brow[i] + ea; col = 8 * bcol[i] + (eb & ~1); }
    else { row = 16 + 4 * g4 + (i - 6); col = l16 & ~1; }
    tw[(row * TT_LD + col) >> 1] = v;
    v += 3;
    __builtin_amdgcn_s_waitcnt(0xC07F);
  }
  acc = (float)v;
  EPILOGUE
}
// calibration: contiguous 64-bit reads (conflict-free) and a 2-way conflicting stride
__global__ void k_calFree(float* out) {
  PROLOGUE
  for (int it = 0; it < NIT; ++it) {
    acc += fold(rd4(buf + 4 * lane + 256 * (it & 7)));
    __builtin_amdgcn_s_waitcnt(0xC07F);
  }
  EPILOGUE
}
__global__ void k_cal2way(float* out) {
  PROLOGUE
  for (int it = 0; it < NIT; ++it) {
    // lanes l and l + 16 hit the same banks (offset 128 dwords apart) within each 32-lane unit
    acc += fold(rd4(buf + 4 * (lane & 15) + 256 * (lane >> 4) + 16 * (it & 7)));
    __builtin_amdgcn_s_waitcnt(0xC07F);
  }
  EPILOGUE
}


// ---- variants
// W operand as two separate ds_read_b64 (inline asm blocks the read2 merge)
__global__ void k_consW_sep(float* out) {
  PROLOGUE
  const int offW = rho_slot(l32) * U_LD + 4 * g;
  for (int it = 0; it < NIT; ++it) {
    const int rt = it & 3, ks = (it >> 2) & 1;
    const E* p = buf + offW + 32 * rt + 16 * ks;
    v4h a = rd4(p);
    asm volatile("" ::: "memory");
    v4h b = rd4(p + 8);
    acc += fold(a) + fold(b);
    __builtin_amdgcn_s_waitcnt(0xC07F);
  }
  EPILOGUE
}
// q-read pattern with pitch P: lane (l16, g4) reads row l16, cols 8 pg + 32 ks (16 B)
template <int P, int PERM>
__global__ void k_q(float* out) {
  PROLOGUE
  const int pg = PERM ? 2 * (g4 & 1) + (g4 >> 1) : g4;
  const int off = l16 * P + 8 * pg;
  for (int it = 0; it < NIT; ++it) {
    const int ks = it & 3;
    const v8h x = *reinterpret_cast<const v8h*>(buf + off + 32 * ks);
    acc += (float)x[0] + (float)x[7];
    __builtin_amdgcn_s_waitcnt(0xC07F);
  }
  EPILOGUE
}
// read2_b64 contiguous (lane * 16 B, halves 8 B apart) and b128 contiguous
__global__ void k_read2c(float* out) {
  PROLOGUE
  for (int it = 0; it < NIT; ++it) {
    const E* p = buf + 8 * lane + 512 * (it & 7);
    acc += fold(rd4(p)) + fold(rd4(p + 4));
    __builtin_amdgcn_s_waitcnt(0xC07F);
  }
  EPILOGUE
}
__global__ void k_b128c(float* out) {
  PROLOGUE
  for (int it = 0; it < NIT; ++it) {
    const v8h x = *reinterpret_cast<const v8h*>(buf + 8 * lane + 512 * (it & 7));
    acc += (float)x[0] + (float)x[7];
    __builtin_amdgcn_s_waitcnt(0xC07F);
  }
  EPILOGUE
}

// stash write as two separate b64 (no write2 merge)
__global__ void k_pstW_sep(float* out) {
  PROLOGUE
  E* const pw = buf + (32 * wave + j_slot(l32)) * PST_LD + 4 * g;
  v4h x = {(E)1.f, (E)2.f, (E)3.f, (E)(float)lane};
  for (int it = 0; it < NIT; ++it) {
    const int rt = it & 3, ks = (it >> 2) & 1;
    *reinterpret_cast<v4h*>(pw + 32 * rt + 16 * ks) = x;
    asm volatile("" ::: "memory");
    *reinterpret_cast<v4h*>(pw + 32 * rt + 16 * ks + 8) = x;
    x[0] += (E)1.f;
    __builtin_amdgcn_s_waitcnt(0xC07F);
  }
  acc = (float)x[0];
  EPILOGUE
}
__global__ void k_consTT_sep(float* out) {
  PROLOGUE
  for (int it = 0; it < NIT; ++it) {
    const int ks = it & 1;
    const E* th = buf + l32 * TT_LD + 16 * ks + 4 * g;
    v4h a = rd4(th);
    asm volatile("" ::: "memory");
    v4h b = rd4(th + 8);
    acc += fold(a) + fold(b);
    __builtin_amdgcn_s_waitcnt(0xC07F);
  }
  EPILOGUE
}

__global__ void k_kvW64(float* out) {
  PROLOGUE
  E* tdst = buf + rho_slot(l32) * U_LD;
  typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
    typedef __attribute__((address_space(3))) volatile u32x2 lds_u2;
  u32x2 x = {(unsigned)lane, 1u};
  for (int it = 0; it < NIT; ++it) {
    const int ks = it & 7;
    *((lds_u2*)(tdst + 16 * ks + 8 * g)) = x;
    *((lds_u2*)(tdst + 16 * ks + 8 * g + 4)) = x;
    x.y += 1;
    __builtin_amdgcn_s_waitcnt(0xC07F);
  }
  acc = (float)x.y;
  EPILOGUE
}
int main() {
  float* out;
  if (hipMalloc(&out, 256 * 256 * sizeof(float)) != hipSuccess) return 1;
  struct K { void (*f)(float*); int threads; const char* name; };
  K ks[] = {{k_calFree, 64, "calFree"},
            {k_cal2way, 64, "cal2way"},
            {k_consW, 64, "consW"},
            {k_consTT, 64, "consTT"},
            {k_consUU, 64, "consUU"},
            {k_pstW, 256, "pstW"},
            {k_zstW, 256, "zstW"},
            {k_rdPST, 128, "rdPST"},
            {k_rdZST, 64, "rdZST"},
            {k_rdQ, 64, "rdQ"},
            {k_rdU, 128, "rdU"},
            {k_prKV, 64, "prKV"},
            {k_prQ, 64, "prQ"},
            {k_prTT, 64, "prTT"},
            {k_consW_sep, 64, "consW_sep"},
            {k_read2c, 64, "read2c"},
            {k_b128c, 64, "b128c"},
            {k_q<144, 0>, 64, "q_P144_id"},
            {k_pstW_sep, 256, "pstW_sep"},
            {k_consTT_sep, 64, "consTT_sep"},
            {k_kvW64, 64, "kvW64"}};
  for (auto& k : ks) {
    hipLaunchKernelGGL(k.f, dim3(256), dim3(k.threads), 0, 0, out);
    if (hipDeviceSynchronize() != hipSuccess) { printf("fail %s\n", k.name); return 2; }
    printf("ran %s\n", k.name);
  }
  return 0;
}
