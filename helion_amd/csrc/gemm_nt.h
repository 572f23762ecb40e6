// Block-tiled GEMM core C = A * B^T for gfx950 with pluggable epilogues.
//
// Both operands are "K-contiguous": A is [M, K] and B is [N, K], row-major
// with leading dimensions lda / ldb (elements, multiples of 16 bytes), so
// every MFMA fragment is one 16-byte LDS read.  One workgroup = 4 wavefronts
// computes a kBM x kBN tile of C; wavefront w owns rows (w>>1)*128 .. +128 and
// columns (w&1)*64 .. +64, i.e. 4 x 2 tiles of 32 x 32.
//
// Accumulator layout (identical for the MFMA and the SIMT core, so epilogues
// are shared): acc[i][j][r] holds
//     C[m0 + wm*128 + 32*i + 8*(r/4) + 4*(lane/32) + r%4][n0 + wn*64 + 32*j + lane%32]
// which is the C layout of v_mfma_f32_32x32x16_{bf16,f16}.
//
// Pipeline: K is walked in tiles of 128 bytes per row (64 16-bit or 32 fp32
// elements), double-buffered in LDS (rows padded by 16 bytes against bank
// conflicts).  Global loads of tile k+1 are issued into registers before the
// MFMAs of tile k and written to the other LDS buffer afterwards, one barrier
// per K tile.  Out-of-range rows and the K tail read as zero.
#pragma once

#include "common.h"

namespace tri {
namespace gemm {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kBM = 256;
constexpr int kBN = 128;
constexpr int kThreads = 256;
constexpr int kMT = 4;  // 32-row MFMA tiles per wavefront
constexpr int kNT = 2;  // 32-column MFMA tiles per wavefront
constexpr int kRowBytes = 128;
constexpr int kPadBytes = 16;

template <typename T> constexpr int bk() { return kRowBytes / (int)sizeof(T); }
template <typename T> constexpr int ldl() { return (kRowBytes + kPadBytes) / (int)sizeof(T); }
template <typename T> constexpr int vec() { return 16 / (int)sizeof(T); }

template <typename T>
struct Smem {
  T a[2][kBM * ldl<T>()];
  T b[2][kBN * ldl<T>()];
};

struct Acc {
  f32x16 t[kMT][kNT];
};

// Registers holding one K tile of one operand between its global load and
// its LDS store: ROWS rows x 8 sixteen-byte vectors, spread over 256 lanes.
template <int ROWS>
struct Staging {
  uint4 v[ROWS * 8 / kThreads];
};

template <typename T, int ROWS>
__device__ __forceinline__ void load_tile(Staging<ROWS>& st, const T* __restrict__ base,
                                          int64_t ld, int64_t row0, int64_t n_rows, int64_t k0,
                                          int64_t K) {
  constexpr int VE = vec<T>();
#pragma unroll
  for (int i = 0; i < ROWS * 8 / kThreads; ++i) {
    const int idx = i * kThreads + threadIdx.x;
    const int64_t row = row0 + (idx >> 3);
    const int64_t k = k0 + (int64_t)(idx & 7) * VE;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (row < n_rows) {
      const T* p = base + row * ld + k;
      if (k + VE <= K) {
        v = *reinterpret_cast<const uint4*>(p);
      } else if (k < K) {
        Pack<T, VE> pk;
#pragma unroll
        for (int e = 0; e < VE; ++e) pk.v[e] = (k + e < K) ? p[e] : (T)0.f;
        v = __builtin_bit_cast(uint4, pk);
      }
    }
    st.v[i] = v;
  }
}

template <typename T, int ROWS>
__device__ __forceinline__ void store_tile(const Staging<ROWS>& st, T* lds) {
  constexpr int VE = vec<T>();
#pragma unroll
  for (int i = 0; i < ROWS * 8 / kThreads; ++i) {
    const int idx = i * kThreads + threadIdx.x;
    *reinterpret_cast<uint4*>(lds + (idx >> 3) * ldl<T>() + (idx & 7) * VE) = st.v[i];
  }
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// ---- per-K-tile compute: MFMA for 16-bit types, FMA for fp32 --------------
template <typename T> struct Core;

__device__ __forceinline__ f32x16 mma(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mma(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

template <typename T, typename V>
__device__ __forceinline__ void mfma_tile(Acc& acc, const T* As, const T* Bs, int wm, int wn) {
  const int lane = threadIdx.x & 63;
  const int l32 = lane & 31, g = lane >> 5;
  constexpr int LD = ldl<T>();
#pragma unroll
  for (int s = 0; s < bk<T>() / 16; ++s) {
    V a[kMT], b[kNT];
#pragma unroll
    for (int i = 0; i < kMT; ++i)
      a[i] = *reinterpret_cast<const V*>(As + (wm * 128 + 32 * i + l32) * LD + 16 * s + 8 * g);
#pragma unroll
    for (int j = 0; j < kNT; ++j)
      b[j] = *reinterpret_cast<const V*>(Bs + (wn * 64 + 32 * j + l32) * LD + 16 * s + 8 * g);
#pragma unroll
    for (int i = 0; i < kMT; ++i)
#pragma unroll
      for (int j = 0; j < kNT; ++j) acc.t[i][j] = mma(a[i], b[j], acc.t[i][j]);
  }
}

template <> struct Core<bf16_t> {
  static __device__ __forceinline__ void tile(Acc& acc, const bf16_t* As, const bf16_t* Bs,
                                              int wm, int wn) {
    mfma_tile<bf16_t, bf16x8>(acc, As, Bs, wm, wn);
  }
};
template <> struct Core<f16_t> {
  static __device__ __forceinline__ void tile(Acc& acc, const f16_t* As, const f16_t* Bs,
                                              int wm, int wn) {
    mfma_tile<f16_t, f16x8>(acc, As, Bs, wm, wn);
  }
};

// fp32: exact FMA arithmetic in the same accumulator layout.  Per 4-wide K
// step a lane reads one float4 per accumulated row group and per column.
template <> struct Core<float> {
  static __device__ __forceinline__ void tile(Acc& acc, const float* As, const float* Bs,
                                              int wm, int wn) {
    const int lane = threadIdx.x & 63;
    const int l32 = lane & 31, g = lane >> 5;
    constexpr int LD = ldl<float>();
#pragma unroll 1
    for (int k = 0; k < bk<float>(); k += 4) {
      float4 b[kNT];
#pragma unroll
      for (int j = 0; j < kNT; ++j)
        b[j] = *reinterpret_cast<const float4*>(Bs + (wn * 64 + 32 * j + l32) * LD + k);
#pragma unroll
      for (int i = 0; i < kMT; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = wm * 128 + 32 * i + 8 * (r >> 2) + 4 * g + (r & 3);
          const float4 a = *reinterpret_cast<const float4*>(As + m * LD + k);
#pragma unroll
          for (int j = 0; j < kNT; ++j) {
            float c = acc.t[i][j][r];
            c = fmaf(a.x, b[j].x, c);
            c = fmaf(a.y, b[j].y, c);
            c = fmaf(a.z, b[j].z, c);
            c = fmaf(a.w, b[j].w, c);
            acc.t[i][j][r] = c;
          }
        }
      }
    }
  }
};

// Tile coordinates of work item `w` of a tiles_m x tiles_n grid: groups of
// kGroupM row tiles are walked column by column so that the blocks resident
// on one XCD share A and B tiles in its L2.
constexpr int kGroupM = 4;
constexpr int kXcds = 8;

__device__ __forceinline__ void tile_of(int64_t bid, int64_t n_blocks, int tiles_m, int tiles_n,
                                        int& tm, int& tn) {
  // XCD-aware: block ids are dealt round-robin to the 8 XCDs; give each XCD a
  // contiguous range of work items.
  int64_t w = bid;
  if (n_blocks % kXcds == 0) w = (bid % kXcds) * (n_blocks / kXcds) + bid / kXcds;
  const int64_t per_group = (int64_t)kGroupM * tiles_n;
  const int64_t group = w / per_group;
  const int first_m = (int)(group * kGroupM);
  const int gsize = min(tiles_m - first_m, kGroupM);
  const int64_t in_group = w % per_group;
  tm = first_m + (int)(in_group % gsize);
  tn = (int)(in_group / gsize);
}

struct Problem {
  const void* a;
  const void* b;
  int64_t lda, ldb;
  int64_t M, N, K;
};

// Main loop: accumulate the (tm, tn) tile of A * B^T over all of K.
template <typename T>
__device__ __forceinline__ void mainloop(const Problem& p, int tm, int tn, Smem<T>& sm,
                                         Acc& acc) {
  const int wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const T* A = (const T*)p.a;
  const T* B = (const T*)p.b;
  const int64_t m0 = (int64_t)tm * kBM, n0 = (int64_t)tn * kBN;
  constexpr int BK = bk<T>();
#pragma unroll
  for (int i = 0; i < kMT; ++i)
#pragma unroll
    for (int j = 0; j < kNT; ++j) acc.t[i][j] = zero16();

  const int64_t nk = cdiv(p.K, BK);
  Staging<kBM> sa;
  Staging<kBN> sb;
  load_tile<T, kBM>(sa, A, p.lda, m0, p.M, 0, p.K);
  load_tile<T, kBN>(sb, B, p.ldb, n0, p.N, 0, p.K);
  store_tile<T, kBM>(sa, sm.a[0]);
  store_tile<T, kBN>(sb, sm.b[0]);
  __syncthreads();
  for (int64_t kt = 0; kt < nk; ++kt) {
    const int cur = (int)(kt & 1);
    const bool more = kt + 1 < nk;
    if (more) {
      load_tile<T, kBM>(sa, A, p.lda, m0, p.M, (kt + 1) * BK, p.K);
      load_tile<T, kBN>(sb, B, p.ldb, n0, p.N, (kt + 1) * BK, p.K);
    }
    Core<T>::tile(acc, sm.a[cur], sm.b[cur], wm, wn);
    if (more) {
      store_tile<T, kBM>(sa, sm.a[cur ^ 1]);
      store_tile<T, kBN>(sb, sm.b[cur ^ 1]);
    }
    __syncthreads();
  }
}

// Row of C held by accumulator element (i, r) of this lane, relative to the tile.
__device__ __forceinline__ int acc_row(int wm, int i, int r, int g) {
  return wm * 128 + 32 * i + 8 * (r >> 2) + 4 * g + (r & 3);
}
__device__ __forceinline__ int acc_col(int wn, int j, int l32) { return wn * 64 + 32 * j + l32; }

}  // namespace gemm
}  // namespace tri
