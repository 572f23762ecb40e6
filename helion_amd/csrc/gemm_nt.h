// Block-tiled GEMM core C = A * B^T for gfx950 with pluggable epilogues.
//
// Each operand is "K-contiguous" (A stored [M, K], B stored [N, K], row-major
// with leading dimension lda / ldb in elements, rows 16-byte aligned: every
// MFMA fragment is one 16-byte LDS read) or, for 16-bit types, selected per
// operand by the TA / TB template flags, "MN-contiguous" (A stored [K, M],
// B stored [K, N]: C = A^T B, A B, ... without transposed copies).  An
// MN-contiguous tile sits in LDS as BK k-rows of BM (BN) elements and its
// fragments come from pairs of ds_read_b64_tr_b16 transposing reads, which
// hand lane (m, g) the k values 8g .. 8g + 7 of column m, the same k order
// as the 16-byte reads, so the two layouts mix freely in one product.  Its
// m (n) extent is read in 8-element granules clamped to the last granule of
// round_up(M, 8) (round_up(N, 8)), so a stored row must hold that many
// elements.  A workgroup of WM x WN wavefronts
// computes a BM x BN tile of C; wavefront (wm, wn) owns the (BM/WM) x (BN/WN)
// sub-tile at (wm*BM/WM, wn*BN/WN), i.e. MT x NT tiles of 32 x 32.
//
// Accumulator layout (identical for the MFMA and the fp32 SIMT core, so the
// epilogues are shared): acc.t[i][j][r] holds
//     C[m0 + acc_row(wm, i, r, g)][n0 + acc_col(wn, j, lane % 32)],  g = lane / 32,
// the C layout of v_mfma_f32_32x32x16_{bf16,f16}.
//
// Pipeline: K is walked in tiles of RB bytes per row (64 or 128: 32 or 64
// 16-bit elements) through two LDS buffers.  Tiles are fetched with
// global_load_lds_dwordx4 (straight into LDS, no staging registers): lane i
// of an instruction fills bytes [16 i, 16 i + 16) of a 1 KiB run, which covers
// 1024 / RB rows; each lane picks which 16-byte granule it fetches so that the rows
// land XOR-swizzled (granule c of row r at slot c ^ swz_key(r)), and the MFMA
// fragment reads of consecutive rows hit distinct 16-byte bank groups.
// One barrier per K tile.  16-bit types run the cross-tile loop (xt_loop):
// the barrier that publishes tile kt + 1 sits before the MFMAs of tile kt's
// last 16-deep step and tile kt + 1's first fragments are read under them;
// fp32 (planned_loop) waits for tile kt, syncs, issues tile kt + 1 into the
// buffer read at step kt - 1, then computes.
// Rows past M (N) re-read the last valid row (their results are never
// stored); a partial last K tile is zero-filled through registers and done
// first, so the pipelined loop has no bounds checks.
#pragma once

#include "common.h"

namespace tri {
namespace gemm {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kXcds = 8;

// BM x BN tile, WM x WN wavefronts, STAGES LDS buffers of K tiles whose rows
// are RB bytes (64 or 128: 32 or 64 16-bit elements).
template <int BM_, int BN_, int WM_, int WN_, int STAGES_, int RB_ = 128>
struct Cfg {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, STAGES = STAGES_, RB = RB_;
  static constexpr int THREADS = WM * WN * 64;
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int MT = WTM / 32, NT = WTN / 32;
  static constexpr int GRAN = RB / 16;            // 16-byte granules per row
  static constexpr int DMA_ROWS = 1024 / RB;      // rows per global_load_lds (1 KiB)
  static constexpr int STAGE_BYTES = (BM + BN) * RB;
  static constexpr int SMEM_BYTES = STAGES * STAGE_BYTES;
  static constexpr int DMA_PER_WAVE = (BM + BN) / DMA_ROWS / (WM * WN);
  static_assert(RB == 64 || RB == 128, "row bytes");
  static_assert((BM + BN) % (DMA_ROWS * WM * WN) == 0, "rows must split evenly over the wavefronts");
  static_assert(BM % DMA_ROWS == 0 && WTM % 32 == 0 && WTN % 32 == 0, "32x32 MFMA tiles");
  static_assert(STAGES >= 2, "at least double buffering");
};

template <class C>
struct Acc {
  f32x16 t[C::MT][C::NT];
};

template <class C, typename T> constexpr int bk() { return C::RB / (int)sizeof(T); }
template <typename T> constexpr int vec() { return 16 / (int)sizeof(T); }

// XOR pattern of tile row r: a b128 read of the same granule of 8 consecutive
// rows (one 128-byte LDS cycle) or of 16 consecutive rows (one 256-byte
// cycle) touches every 16-byte bank group once.
template <class C>
__device__ __forceinline__ int swz_key(int r) {
  if constexpr (C::RB == 128) return (r & 7) ^ ((r >> 3) & 1);
  else return ((r >> 2) ^ (r >> 1)) & 3;
}
// Byte offset of 16-byte granule c of tile row r.
template <class C>
__device__ __forceinline__ int swz(int r, int c) { return r * C::RB + ((c ^ swz_key<C>(r)) << 4); }

// MN-contiguous tiles: k-row r of X columns, XR = X * 2 bytes.  Granule c
// of row r sits at slot c ^ tkey(r): the 4 rows x 4 granules one 32-lane
// cycle of a transposing read touches (rows 4j .. 4j + 3, granules 4q ..
// 4q + 3) land in 16 distinct 16-byte bank groups.
__device__ __forceinline__ int tkey(int r) { return (r & 3) << 2; }
template <int X>
__device__ __forceinline__ int tswz(int r, int c) { return r * (2 * X) + ((c ^ tkey(r)) << 4); }

// Fragment of an MN-contiguous tile of X columns: columns col0 .. col0 + 31
// (col0 a multiple of 32) as lane & 31, k = 16 S + 8 g .. + 7 (g = lane >> 5).
// One transposing read serves a 16-lane group: source lane s addresses k-row
// (s >> 2) at columns 4 (s & 3) .. + 3 of the group's 16 columns, and
// destination lane j receives the four k values of column j; two reads (k
// rows 8g .. 8g + 3 and 8g + 4 .. 8g + 7) make the 8 k values of a lane.
template <int X, class V>
__device__ __forceinline__ V frag_tr(const char* tile, int col0, int S) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  const int lane = threadIdx.x & 63;
  const int ts = lane & 15, th = (lane >> 4) & 1, g = lane >> 5;
  const int r1 = 16 * S + 8 * g + (ts >> 2);
  const int c = (col0 >> 3) + 2 * th + ((ts & 3) >> 1);
  const int sub = (ts & 1) * 8;
  const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4s*)(lds_addr(tile + tswz<X>(r1, c) + sub)));
  const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4s*)(lds_addr(tile + tswz<X>(r1 + 4, c) + sub)));
  // one whole-vector cast (element-wise assembly was miscompiled into broadcasts)
  return __builtin_bit_cast(V, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

template <class C>
__device__ __forceinline__ int acc_row(int wm, int i, int r, int g) {
  return wm * C::WTM + 32 * i + 8 * (r >> 2) + 4 * g + (r & 3);
}
template <class C>
__device__ __forceinline__ int acc_col(int wn, int j, int l32) {
  return wn * C::WTN + 32 * j + l32;
}

__device__ __forceinline__ int64_t imin(int64_t a, int64_t b) { return a < b ? a : b; }

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

struct Problem {
  const void* a;
  const void* b;
  int64_t lda, ldb;
  int64_t M, N, K;
};

// One operand of the partial last K tile, MN-contiguous: k-rows past K are
// zero, columns clamped like the DMA's.
template <class C, typename T, int X>
__device__ __forceinline__ void reg_tile_tr(char* tile, const void* base, int64_t ld, int64_t x0,
                                            int64_t xn, int64_t k0, int64_t K) {
  constexpr int VE = vec<T>(), XG = X / 8, BK = bk<C, T>();
  const int64_t last = ((xn + 7) & ~(int64_t)7) - 8;
  for (int idx = threadIdx.x; idx < BK * XG; idx += C::THREADS) {
    const int kr = idx / XG, c = idx % XG;
    Pack<T, VE> pk;
    if (k0 + kr < K) {
      pk = *reinterpret_cast<const Pack<T, VE>*>((const T*)base + (k0 + kr) * ld +
                                                 imin(x0 + c * VE, last));
    } else {
#pragma unroll
      for (int e = 0; e < VE; ++e) pk.v[e] = (T)0.f;
    }
    *reinterpret_cast<Pack<T, VE>*>(tile + tswz<X>(kr, c)) = pk;
  }
}

template <class C, typename T, bool TA = false, bool TB = false>
__device__ __forceinline__ void reg_tile(char* stage, const Problem& p, int64_t m0, int64_t n0,
                                         int64_t k0) {
  constexpr int VE = vec<T>();
  if constexpr (TA || TB) {
    if constexpr (TA) reg_tile_tr<C, T, C::BM>(stage, p.a, p.lda, m0, p.M, k0, p.K);
    if constexpr (TB) reg_tile_tr<C, T, C::BN>(stage + C::BM * C::RB, p.b, p.ldb, n0, p.N, k0, p.K);
    const int r0 = TA ? C::BM : 0, r1 = TB ? C::BM : C::BM + C::BN;  // K-contiguous rows left
    for (int idx = r0 * C::GRAN + threadIdx.x; idx < r1 * C::GRAN; idx += C::THREADS) {
      const int row = idx / C::GRAN, c = idx % C::GRAN;
      const T* src = row < C::BM ? (const T*)p.a + imin(m0 + row, p.M - 1) * p.lda
                                 : (const T*)p.b + imin(n0 + row - C::BM, p.N - 1) * p.ldb;
      const int64_t k = k0 + c * VE;
      Pack<T, VE> pk;
#pragma unroll
      for (int e = 0; e < VE; ++e) pk.v[e] = (k + e < p.K) ? src[k + e] : (T)0.f;
      *reinterpret_cast<Pack<T, VE>*>(stage + swz<C>(row, c)) = pk;
    }
    return;
  }
  for (int idx = threadIdx.x; idx < (C::BM + C::BN) * C::GRAN; idx += C::THREADS) {
    const int row = idx / C::GRAN, c = idx % C::GRAN;
    const T* src;
    if (row < C::BM) {
      src = (const T*)p.a + imin(m0 + row, p.M - 1) * p.lda;
    } else {
      src = (const T*)p.b + imin(n0 + row - C::BM, p.N - 1) * p.ldb;
    }
    const int64_t k = k0 + c * VE;
    Pack<T, VE> pk;
#pragma unroll
    for (int e = 0; e < VE; ++e) pk.v[e] = (k + e < p.K) ? src[k + e] : (T)0.f;
    *reinterpret_cast<Pack<T, VE>*>(stage + swz<C>(row, c)) = pk;
  }
}

// ---- per-K-tile compute: MFMA for 16-bit types, FMA for fp32 --------------
__device__ __forceinline__ f32x16 mma(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mma(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

template <typename T> struct FragOf;
template <> struct FragOf<bf16_t> { typedef bf16x8 V; };
template <> struct FragOf<f16_t> { typedef f16x8 V; };

// Compiler fence: no instruction is scheduled across it.
__device__ __forceinline__ void fence() { __builtin_amdgcn_sched_barrier(0); }

struct NoHook {
  template <int S> __device__ __forceinline__ void step() const {}
};

// 16-deep MFMA step S of a K tile and the ones after it; the fragment reads
// of step S + 1 are issued before the MFMAs of step S (explicit order,
// fenced against the scheduler: left alone, the compiler reuses one
// fragment buffer and waits on every read), and hook.step<S>() runs after
// step S's MFMAs are issued.
// A fragments (rows wm * WTM + 32 i ..) and B fragments (wn * WTN + 32 j ..)
// of 16-deep step S, from either tile layout.
template <class C, bool TA, class V>
__device__ __forceinline__ V frag_a(const char* As, int wm, int i, int S) {
  const int lane = threadIdx.x & 63;
  if constexpr (TA) return frag_tr<C::BM, V>(As, wm * C::WTM + 32 * i, S);
  else return *reinterpret_cast<const V*>(As + swz<C>(wm * C::WTM + 32 * i + (lane & 31), 2 * S + (lane >> 5)));
}
template <class C, bool TB, class V>
__device__ __forceinline__ V frag_b(const char* Bs, int wn, int j, int S) {
  const int lane = threadIdx.x & 63;
  if constexpr (TB) return frag_tr<C::BN, V>(Bs, wn * C::WTN + 32 * j, S);
  else return *reinterpret_cast<const V*>(Bs + swz<C>(wn * C::WTN + 32 * j + (lane & 31), 2 * S + (lane >> 5)));
}

template <class C, typename T, class Hook, int S, bool TA, bool TB, class V>
__device__ __forceinline__ void mma_steps(const char* As, const char* Bs, Acc<C>& acc, int wm,
                                          int wn, V (&a)[2][C::MT], V (&b)[2][C::NT],
                                          const Hook& hook) {
  constexpr int KS = C::RB / 32;
  if constexpr (S < KS) {
    if constexpr (S + 1 < KS) {
#pragma unroll
      for (int i = 0; i < C::MT; ++i) a[(S + 1) & 1][i] = frag_a<C, TA, V>(As, wm, i, S + 1);
#pragma unroll
      for (int j = 0; j < C::NT; ++j) b[(S + 1) & 1][j] = frag_b<C, TB, V>(Bs, wn, j, S + 1);
    }
    fence();
#pragma unroll
    for (int i = 0; i < C::MT; ++i)
#pragma unroll
      for (int j = 0; j < C::NT; ++j) acc.t[i][j] = mma(a[S & 1][i], b[S & 1][j], acc.t[i][j]);
    hook.template step<S>();
    fence();
    mma_steps<C, T, Hook, S + 1, TA, TB>(As, Bs, acc, wm, wn, a, b, hook);
  }
}

template <class C, class Hook, int S = 0>
__device__ __forceinline__ void all_steps(const Hook& hook) {
  if constexpr (S < C::RB / 32) {
    hook.template step<S>();
    all_steps<C, Hook, S + 1>(hook);
  }
}

// hook.step<s>() runs after the MFMAs of 16-deep step s are issued (the
// 2-stage loop issues the next tile's DMAs there, spread over the tile
// instead of in one burst while the MFMA pipe waits)
template <class C, typename T, class Hook = NoHook, bool TA = false, bool TB = false>
__device__ __forceinline__ void compute_tile(const char* stage, Acc<C>& acc, int wm, int wn,
                                             const Hook& hook = Hook()) {
  const char* As = stage;
  const char* Bs = stage + C::BM * C::RB;
  const int lane = threadIdx.x & 63;
  const int l32 = lane & 31, g = lane >> 5;
  static_assert(sizeof(T) == 2 || (!TA && !TB), "MN-contiguous operands: 16-bit types only");
  if constexpr (sizeof(T) == 2) {
    typedef typename FragOf<T>::V V;
    V a[2][C::MT], b[2][C::NT];
#pragma unroll
    for (int i = 0; i < C::MT; ++i) a[0][i] = frag_a<C, TA, V>(As, wm, i, 0);
#pragma unroll
    for (int j = 0; j < C::NT; ++j) b[0][j] = frag_b<C, TB, V>(Bs, wn, j, 0);
    fence();
    mma_steps<C, T, Hook, 0, TA, TB>(As, Bs, acc, wm, wn, a, b, hook);
  } else {
    all_steps<C>(hook);  // no MFMA steps to spread over: the hook's work up front
    // fp32: exact FMAs; one float4 (one granule) per row and per column per step
#pragma unroll 1
    for (int c = 0; c < C::GRAN; ++c) {
      float4 b[C::NT];
#pragma unroll
      for (int j = 0; j < C::NT; ++j)
        b[j] = *reinterpret_cast<const float4*>(Bs + swz<C>(wn * C::WTN + 32 * j + l32, c));
#pragma unroll
      for (int i = 0; i < C::MT; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float4 a = *reinterpret_cast<const float4*>(As + swz<C>(acc_row<C>(wm, i, r, g), c));
#pragma unroll
          for (int j = 0; j < C::NT; ++j) {
            float v = acc.t[i][j][r];
            v = fmaf(a.x, b[j].x, v);
            v = fmaf(a.y, b[j].y, v);
            v = fmaf(a.z, b[j].z, v);
            v = fmaf(a.w, b[j].w, v);
            acc.t[i][j][r] = v;
          }
        }
      }
    }
  }
}

// Tile coordinates of block `bid` of a tiles_m x tiles_n grid.  Block ids are
// dealt round-robin to the 8 XCDs; each XCD gets a contiguous range of work
// items, walked in groups of GROUP_M row tiles column by column so that the
// blocks resident on one XCD share A and B tiles in its L2.
// (groups of 2 or 8 row tiles measured 1-3% slower on config 4's linear-CE)
template <int GROUP_M = 4>
__device__ __forceinline__ void tile_of(int64_t bid, int64_t n_blocks, int tiles_m, int tiles_n,
                                        int& tm, int& tn) {
  int64_t w = bid;
  if (n_blocks % kXcds == 0) w = (bid % kXcds) * (n_blocks / kXcds) + bid / kXcds;
  const int64_t per_group = (int64_t)GROUP_M * tiles_n;
  const int64_t group = w / per_group;
  const int first_m = (int)(group * GROUP_M);
  const int gsize = min(tiles_m - first_m, GROUP_M);
  const int64_t in_group = w % per_group;
  tm = first_m + (int)(in_group % gsize);
  tn = (int)(in_group / gsize);
}

// DMA pattern of the fp32 loop (planned_loop): how many of a wavefront's
// DMAs follow each 16-deep step, as decimal digits read from the first step;
// 4400 (four after each of the first two steps) measured 3.5% faster than
// 2222 and 1.7% faster than 8000 on config 4's linear-CE in that loop's
// 16-bit form: the next tile's last DMAs have half a tile of MFMAs to land
// behind.
constexpr int kSpread = 4400;

// DMA plan of the 2-stage loop for one output tile: each of this
// wavefront's DMA_PER_WAVE runs (PA of A, then PB of B, as in dma_one) gets
// a per-lane byte offset computed once per tile from a wave-uniform operand
// base that advances by a fixed stride per K tile, so issuing a DMA in the
// loop costs scalar adds only (the per-DMA 64-bit address arithmetic and the
// generic-to-LDS pointer check it replaces cost ~20% of the GEMM's time).
// Offsets are 32-bit: K-contiguous operands need BM (BN) * ld * sizeof(T)
// < 4 GiB, MN-contiguous ones BK * ld * sizeof(T) < 4 GiB (host-checked).
template <class C, typename T, bool TR, int X>
__device__ __forceinline__ uint32_t run_voff(int run, int lane, int64_t ld, int64_t x0,
                                             int64_t xn) {
  constexpr int VE = vec<T>();
  if constexpr (!TR) {
    const int trow = run * C::DMA_ROWS + lane / C::GRAN;
    const int c = (lane % C::GRAN) ^ swz_key<C>(trow);
    const int64_t row = imin(trow, xn - 1 - x0);
    return (uint32_t)((row * ld + c * VE) * (int64_t)sizeof(T));
  } else {
    constexpr int XG = X / 8;
    const int krow = run * (64 / XG) + lane / XG;
    const int c = (lane % XG) ^ tkey(krow);
    const int64_t last = ((xn + 7) & ~(int64_t)7) - 8;
    const int64_t col = imin(x0 + c * VE, last) - x0;
    return (uint32_t)((krow * ld + col) * (int64_t)sizeof(T));
  }
}

template <class C, typename T, bool TA, bool TB>
struct DmaPlan {
  static constexpr int W = C::WM * C::WN;
  static constexpr int RUNS_A = C::BM / C::DMA_ROWS;
  static constexpr int PA = RUNS_A / W, PB = (C::BN / C::DMA_ROWS) / W;
  uint32_t voff[PA + PB];
  const char* base_a;
  const char* base_b;
  int64_t step_a, step_b;  // bytes per K tile
  uint32_t lds_a, lds_b;   // LDS byte address of this wavefront's first A / B run, stage 0

  __device__ __forceinline__ void init(const Problem& p, int64_t m0, int64_t n0, char* smem) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    constexpr int64_t BK = bk<C, T>(), ES = sizeof(T);
#pragma unroll
    for (int q = 0; q < PA; ++q) voff[q] = run_voff<C, T, TA, C::BM>(wave * PA + q, lane, p.lda, m0, p.M);
#pragma unroll
    for (int q = 0; q < PB; ++q) voff[PA + q] = run_voff<C, T, TB, C::BN>(wave * PB + q, lane, p.ldb, n0, p.N);
    base_a = (const char*)p.a + (TA ? m0 : m0 * p.lda) * ES;
    base_b = (const char*)p.b + (TB ? n0 : n0 * p.ldb) * ES;
    step_a = TA ? BK * p.lda * ES : BK * ES;
    step_b = TB ? BK * p.ldb * ES : BK * ES;
    const int ws = __builtin_amdgcn_readfirstlane(wave);
    const uint32_t l0 = __builtin_amdgcn_readfirstlane(lds_addr(smem));
    lds_a = l0 + (uint32_t)(ws * PA) * 1024u;
    lds_b = l0 + (uint32_t)(RUNS_A + ws * PB) * 1024u;
  }
  // A wave-uniform pointer in SGPRs: the compiler may compute base + kt *
  // step with vector instructions, and the DMA's scalar base operand needs
  // an SGPR pair (readfirstlane of a value already in SGPRs folds away).
  static __device__ __forceinline__ const char* in_sgprs(const char* p) {
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (const char*)(((uint64_t)hi << 32) | lo);
  }
  // DMA q of K tile kt into stage `stage`
  template <int Q>
  __device__ __forceinline__ void issue(int stage, int64_t kt) const {
    const uint32_t so = (uint32_t)stage * (uint32_t)C::STAGE_BYTES;
    if constexpr (Q < PA)
      dma16s(in_sgprs(base_a + kt * step_a), voff[Q], lds_a + so + Q * 1024u);
    else
      dma16s(in_sgprs(base_b + kt * step_b), voff[Q], lds_b + so + (Q - PA) * 1024u);
  }
  template <int Q, int Q1>
  __device__ __forceinline__ void issue_range(int stage, int64_t kt) const {
    if constexpr (Q < Q1) {
      issue<Q>(stage, kt);
      issue_range<Q + 1, Q1>(stage, kt);
    }
  }
};

// compute_tile hook of the planned loop: the DMAs of K tile kt after the
// steps the digits of PAT name.  Every wavefront follows one pattern: giving
// the second wavefront of each SIMD the opposite phase (DMAs after the last
// two steps) measured 37-57% slower.
constexpr int spread_digit2(int pat, int s, int ks) {
  for (int i = 0; i < ks - 1 - s; ++i) pat /= 10;
  return pat % 10;
}
template <class C>
constexpr int spread_first2(int pat, int s) {
  int q = 0;
  for (int i = 0; i < s; ++i) q += spread_digit2(pat, i, C::RB / 32);
  return q < C::DMA_PER_WAVE ? q : C::DMA_PER_WAVE;
}

template <class C, typename T, bool TA, bool TB, int PAT>
struct PlanSpread {
  const DmaPlan<C, T, TA, TB>* plan;
  int stage;
  int64_t kt;
  template <int S>
  __device__ __forceinline__ void step() const {
    constexpr int KS = C::RB / 32;
    constexpr int Q0 = spread_first2<C>(PAT, S);
    constexpr int Q1 = S + 1 == KS ? C::DMA_PER_WAVE : spread_first2<C>(PAT, S + 1);
    plan->template issue_range<Q0, Q1>(stage, kt);
  }
};

// The K loop of the planned 2-stage pipeline with DMA pattern PAT.
template <class C, typename T, bool TA, bool TB, int PAT>
__device__ __forceinline__ void planned_loop(const DmaPlan<C, T, TA, TB>& plan, char* smem,
                                             Acc<C>& acc, int wm, int wn, int64_t nfull) {
  for (int64_t kt = 0; kt + 1 < nfull; ++kt) {
    wait_vmcnt<0>();
    __syncthreads();
    const PlanSpread<C, T, TA, TB, PAT> spread{&plan, (int)((kt + 1) & 1), kt + 1};
    compute_tile<C, T, PlanSpread<C, T, TA, TB, PAT>, TA, TB>(
        smem + (int)(kt & 1) * C::STAGE_BYTES, acc, wm, wn, spread);
  }
}

// Cross-tile pipelined 2-stage loop.  The loop above starts every K tile
// with barrier -> step-0 fragment reads -> MFMAs, so all eight wavefronts
// wait out one LDS read latency per tile with the MFMA pipe empty.  Here the
// barrier that publishes tile kt + 1 sits before the MFMAs of tile kt's
// last 16-deep step, and tile kt + 1's step-0 fragments are read under
// those MFMAs.  Every wavefront has finished reading tile kt's stage when it
// passes that barrier (its last reads were issued a step earlier and
// lds_barrier waits for them), so the first half of its DMAs of
// tile kt + 2 go into that stage right after the last step's MFMAs, and the
// rest after the next tile's first step: the last DMAs of a tile then have
// two steps of MFMAs to land behind before the barrier waits for them, as in
// the loop above.
template <class C>
constexpr int xt_early() {
  return C::DMA_PER_WAVE / 2;
}

template <class C, bool TA, bool TB, class V>
__device__ __forceinline__ void read_step(const char* stage, int wm, int wn, int S, V (&a)[C::MT],
                                          V (&b)[C::NT]) {
  const char* As = stage;
  const char* Bs = stage + C::BM * C::RB;
#pragma unroll
  for (int i = 0; i < C::MT; ++i) a[i] = frag_a<C, TA, V>(As, wm, i, S);
#pragma unroll
  for (int j = 0; j < C::NT; ++j) b[j] = frag_b<C, TB, V>(Bs, wn, j, S);
}

// 16-deep step S (and the ones after it) of K tile kt, held in stage `cur`.
// NEXT: tile kt + 1 exists (published by the barrier before the last step,
// its step-0 fragments read under the last step's MFMAs, its remaining DMAs
// issued after step 0); NEXT2: tile kt + 2 exists (its first DMAs follow
// the last step's MFMAs, into stage `cur`).  Compile-time flags: a run-time
// branch around the barrier makes the compiler merge the LDS counters of
// both paths and wait for the next tile's reads before the last MFMAs.
template <class C, typename T, bool TA, bool TB, bool NEXT, bool NEXT2, int S = 0, class V>
__device__ __forceinline__ void xt_tile(const DmaPlan<C, T, TA, TB>& plan, char* smem, int cur,
                                        int64_t kt, Acc<C>& acc, int wm, int wn,
                                        V (&a)[2][C::MT], V (&b)[2][C::NT]) {
  constexpr int KS = C::RB / 32;
  constexpr int H = xt_early<C>();
  static_assert(KS % 2 == 0, "the next tile's step 0 lands in fragment buffer 0");
  if constexpr (S < KS) {
    if constexpr (S + 1 < KS) {
      read_step<C, TA, TB>(smem + cur * C::STAGE_BYTES, wm, wn, S + 1, a[(S + 1) & 1],
                           b[(S + 1) & 1]);
    } else if constexpr (NEXT) {
      wait_vmcnt<0>();
      lds_barrier();
      read_step<C, TA, TB>(smem + (cur ^ 1) * C::STAGE_BYTES, wm, wn, 0, a[0], b[0]);
    }
    fence();
#pragma unroll
    for (int i = 0; i < C::MT; ++i)
#pragma unroll
      for (int j = 0; j < C::NT; ++j) acc.t[i][j] = mma(a[S & 1][i], b[S & 1][j], acc.t[i][j]);
    if constexpr (S == 0 && NEXT) plan.template issue_range<H, C::DMA_PER_WAVE>(cur ^ 1, kt + 1);
    if constexpr (S + 1 == KS && NEXT2) plan.template issue_range<0, H>(cur, kt + 2);
    fence();
    xt_tile<C, T, TA, TB, NEXT, NEXT2, S + 1>(plan, smem, cur, kt, acc, wm, wn, a, b);
  }
}

// The cross-tile loop over nfull >= 1 full K tiles (the caller tests for
// none: an early return in here kept extra copies of the accumulators alive
// and spilled them).
template <class C, typename T, bool TA, bool TB>
__device__ __forceinline__ void xt_loop(const DmaPlan<C, T, TA, TB>& plan, char* smem,
                                        Acc<C>& acc, int wm, int wn, int64_t nfull) {
  typedef typename FragOf<T>::V V;
  constexpr int H = xt_early<C>();
  V a[2][C::MT], b[2][C::NT];
  plan.template issue_range<0, C::DMA_PER_WAVE>(0, 0);
  wait_vmcnt<0>();
  lds_barrier();
  read_step<C, TA, TB>(smem, wm, wn, 0, a[0], b[0]);
  if (nfull > 1) plan.template issue_range<0, H>(1, 1);
  fence();
  int64_t kt = 0;
  for (; kt + 2 < nfull; ++kt)
    xt_tile<C, T, TA, TB, true, true>(plan, smem, (int)(kt & 1), kt, acc, wm, wn, a, b);
  if (kt + 1 < nfull) {
    xt_tile<C, T, TA, TB, true, false>(plan, smem, (int)(kt & 1), kt, acc, wm, wn, a, b);
    ++kt;
  }
  xt_tile<C, T, TA, TB, false, false>(plan, smem, (int)(kt & 1), kt, acc, wm, wn, a, b);
}

// Accumulate the (tm, tn) tile of A * B^T over all of K (A, B in the
// layouts TA, TB select).  `smem` holds C::SMEM_BYTES of LDS (1 KiB aligned).
template <class C, typename T, bool TA = false, bool TB = false>
__device__ __forceinline__ void mainloop(const Problem& p, int tm, int tn, char* smem,
                                         Acc<C>& acc) {
  static_assert(C::STAGES == 2, "the 2-stage DMA loops");
  // the wavefront index stays a per-lane value here: it is part of every
  // fragment's LDS address, which then folds into one VGPR base plus
  // immediate offsets (a scalar index costs an add per read: -12% measured)
  const int wave = threadIdx.x >> 6;
  const int wm = wave / C::WN, wn = wave % C::WN;
  const int64_t m0 = (int64_t)tm * C::BM, n0 = (int64_t)tn * C::BN;
  constexpr int BK = bk<C, T>();
#pragma unroll
  for (int i = 0; i < C::MT; ++i)
#pragma unroll
    for (int j = 0; j < C::NT; ++j) acc.t[i][j] = zero16();

  const int64_t nfull = p.K / BK;
  if (p.K % BK != 0) {
    reg_tile<C, T, TA, TB>(smem, p, m0, n0, nfull * BK);
    __syncthreads();
    compute_tile<C, T, NoHook, TA, TB>(smem, acc, wm, wn);
    __syncthreads();
  }
  DmaPlan<C, T, TA, TB> plan;
  plan.init(p, m0, n0, smem);
  if constexpr (sizeof(T) == 2) {
    if (nfull > 0) xt_loop<C, T, TA, TB>(plan, smem, acc, wm, wn, nfull);
  } else {
    // branch-free steady state: wait for tile kt, sync, prefetch tile kt + 1
    // into the buffer read at step kt - 1, compute tile kt
    if (nfull > 0) plan.template issue_range<0, C::DMA_PER_WAVE>(0, 0);
    planned_loop<C, T, TA, TB, kSpread>(plan, smem, acc, wm, wn, nfull);
    if (nfull > 0) {
      wait_vmcnt<0>();
      __syncthreads();
      compute_tile<C, T, NoHook, TA, TB>(smem + (int)((nfull - 1) & 1) * C::STAGE_BYTES, acc, wm,
                                         wn);
    }
  }
  __syncthreads();
}

// Configurations: 16-bit types run 256 x 256 tiles on 8 wavefronts (2 per
// SIMD, 128 x 64 each), double-buffered 128-byte K rows; fp32 (exact SIMT
// arithmetic) runs 128 x 128 tiles on 4 wavefronts.
template <typename T> struct CfgOf { typedef Cfg<256, 256, 2, 4, 2, 128> type; };
template <> struct CfgOf<float> { typedef Cfg<128, 128, 2, 2, 2> type; };

}  // namespace gemm
}  // namespace tri
