// Fused linear + cross-entropy forward and backward for gfx950.
//
// Reference arithmetic: alkinun/helion tritium/ops/cross_entropy.py:219-293
// (forward: logits = hidden @ weight^T with fp32 accumulation, per-row
// lse = max + ln(sum exp(logit - max)), nll = lse - logit[target], mean) and
// 103-131 + 937-957 (backward: G = (softmax - onehot) * grad_out / count,
// dhidden = G @ weight, dweight = G^T @ hidden).  ignore_index follows
// torch's F.cross_entropy: ignored rows add nothing and the mean divides by
// the number of non-ignored rows.
//
// Forward -- the logits never reach HBM:
//   lce_fwd_kernel     S^T = W H^T tile by tile (gemm_nt.h core, vocab along
//                      the tile's rows, tokens along its columns); epilogue in
//                      registers: per (vocab block, token) max and sum of
//                      exp(logit - max), and the target logit (written by the
//                      one lane whose row is the target);
//   lce_fwd_rows       per token: combine the vocab-block partials online into
//                      lse, nll; per-block partial sums of nll and counts;
//   lce_fwd_finalize   one block: loss = sum(nll) / count in a fixed order.
// Backward (16-bit inputs), per vocab chunk of Vc rows (G of one chunk fits
// a 1 GiB workspace; nothing of size N x V is kept from the forward):
//   lce_g_kernel       recompute S^T for the chunk on the GEMM core, epilogue
//                      G = (exp(S - lse) - onehot) * grad_out / count (0 for
//                      ignored rows), written as G [N, Vc] in the input dtype;
//   dW_c = G^T H       GEMM with both operands MN-contiguous (G and H read in
//                      place through transposing LDS reads), the full token
//                      reduction inside one product, stored once;
//   dH (+)= G W_c      GEMM with W_c MN-contiguous, fp32 accumulation across
//                      chunks, rounded once after the last.
// All reductions are in a fixed order: results are bitwise reproducible.
#include <math.h>

#include <type_traits>

#include "common.h"
#include "gemm_nt.h"
#include "../../include/tritium_hip.h"

namespace tri {
namespace {

using gemm::Acc;
using gemm::acc_col;
using gemm::acc_row;
template <typename T> using CfgT = typename gemm::CfgOf<T>::type;
constexpr int kMaxBM = 256;  // largest row tile of any configuration

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kRowsBlock = 256;        // threads of lce_fwd_rows
constexpr int kRowsSplit = 8;          // threads per token in lce_fwd_rows
constexpr int64_t kGBudget = (int64_t)1 << 30;  // bytes of G for one vocabulary chunk

template <typename TT>
__device__ __forceinline__ int64_t load_target(const TT* t, int64_t n) {
  return (int64_t)t[n];
}

// raw bits of a 16-bit element, and back
template <typename T>
__device__ __forceinline__ uint16_t bits16(T x) {
  static_assert(sizeof(T) == 2, "16-bit type");
  return __builtin_bit_cast(uint16_t, x);
}
template <typename T>
__device__ __forceinline__ T from_bits16(uint16_t b) {
  static_assert(sizeof(T) == 2, "16-bit type");
  return __builtin_bit_cast(T, b);
}

// Four values rounded to the 16-bit type S, packed in 8 bytes.
template <typename S>
__device__ __forceinline__ uint2 pack4(const float* v) {
  uint2 pk;
  pk.x = (uint32_t)bits16(from_f32<S>(v[0])) | ((uint32_t)bits16(from_f32<S>(v[1])) << 16);
  pk.y = (uint32_t)bits16(from_f32<S>(v[2])) | ((uint32_t)bits16(from_f32<S>(v[3])) << 16);
  return pk;
}

// A 16-bit tile of 256 vocab rows x BN tokens, held by the lanes as 4
// consecutive vocab rows of one token, leaves for a token-major [N, ld]
// buffer through the (idle) LDS as whole 512-byte token rows; stored
// directly, every store instruction would touch 32 token rows.  Staging
// layout: the 8-byte slot s of token row r sits at slot s ^ (r & 63), so the
// 32 tokens of a half-wavefront write distinct banks.
__device__ __forceinline__ void stage_put4(char* tile, int tok, int vl, uint2 pk) {
  *reinterpret_cast<uint2*>(tile + tok * 512 + (((vl >> 2) ^ (tok & 63)) << 3)) = pk;
}

// Copy the staged tile out: 32 lanes per token row, 16 bytes (8 vocab
// entries) each; rows at or past N and vocab entries at or past Vc are not
// written.  The caller has passed a barrier since the last stage_put4.
template <int THREADS, int BN>
__device__ __forceinline__ void stage_out(const char* tile, uint16_t* out, int64_t ld, int64_t n0,
                                          int64_t v0, int64_t N, int64_t Vc) {
  constexpr int ITER = BN * 32 / THREADS;
#pragma unroll
  for (int it = 0; it < ITER; ++it) {
    const int idx = it * THREADS + threadIdx.x;
    const int row = idx >> 5, c = idx & 31;
    const int64_t n = n0 + row;
    const int64_t vb = v0 + 8 * c;
    // slots 2c and 2c + 1 sit in one 16-byte chunk, swapped for odd rows
    u32x4 v = *reinterpret_cast<const u32x4*>(tile + row * 512 + ((((2 * c) ^ (row & 63)) & ~1) << 3));
    if (row & 1) v = __builtin_shufflevector(v, v, 2, 3, 0, 1);
    if (n >= N || vb >= Vc) continue;
    uint16_t* dst = out + n * ld + vb;
    if (vb + 8 <= Vc) {
      st16(dst, v);
    } else {
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (vb + e < Vc) dst[e] = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
    }
  }
}

// ------------------------------------------------------------- forward ----
struct FwdArgs {
  const void* hidden;  // [N, D]
  const void* weight;  // [V, D]
  const void* target;  // [N] int32 / int64
  float* pmax;         // [tiles_v, N]
  float* psum;         // [tiles_v, N]
  float* tlogit;       // [N]
  int64_t N, D, V, ld;
  int tiles_v, tiles_n;
};

template <typename T, typename TT>
__global__ void __launch_bounds__(CfgT<T>::THREADS)
lce_fwd_kernel(FwdArgs a) {
  typedef CfgT<T> C;
  __shared__ __attribute__((aligned(1024))) char smem[C::SMEM_BYTES];
  __shared__ float red[C::WM][C::BN];
  int tm, tn;
  gemm::tile_of(blockIdx.x, gridDim.x, a.tiles_v, a.tiles_n, tm, tn);
  gemm::Problem p{a.weight, a.hidden, a.ld, a.ld, a.V, a.N, a.D};
  Acc<C> acc;
  gemm::mainloop<C, T>(p, tm, tn, smem, acc);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l32 = lane & 31, g = lane >> 5;
  const int wm = wave / C::WN, wn = wave % C::WN;
  const int64_t v0 = (int64_t)tm * C::BM, n0 = (int64_t)tn * C::BN;
  const TT* target = (const TT*)a.target;

  // every vocabulary row of an interior tile exists: no per-element check
  const bool full = v0 + C::BM <= a.V;
  float mx[C::NT];
#pragma unroll
  for (int j = 0; j < C::NT; ++j) {
    float m = -INFINITY;
    if (full) {
#pragma unroll
      for (int i = 0; i < C::MT; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) m = fmaxf(m, acc.t[i][j][r]);
    } else {
#pragma unroll
      for (int i = 0; i < C::MT; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (v0 + acc_row<C>(wm, i, r, g) < a.V) m = fmaxf(m, acc.t[i][j][r]);
    }
    m = fmaxf(m, __shfl_xor(m, 32, 64));
    if (g == 0) red[wm][acc_col<C>(wn, j, l32)] = m;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < C::NT; ++j) {
    const int col = acc_col<C>(wn, j, l32);
    float m = red[0][col];
#pragma unroll
    for (int k = 1; k < C::WM; ++k) m = fmaxf(m, red[k][col]);
    mx[j] = m;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < C::NT; ++j) {
    const int col = acc_col<C>(wn, j, l32);
    const int64_t n = n0 + col;
    const float ms = mx[j] * kLog2e;
    float s = 0.f;
    if (full) {
#pragma unroll
      for (int i = 0; i < C::MT; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) s += fast_exp2(acc.t[i][j][r] * kLog2e - ms);
    } else {
#pragma unroll
      for (int i = 0; i < C::MT; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (v0 + acc_row<C>(wm, i, r, g) < a.V) s += fast_exp2(acc.t[i][j][r] * kLog2e - ms);
    }
    s += __shfl_xor(s, 32, 64);
    if (g == 0) red[wm][col] = s;
    // the target logit: written by the single lane that holds its row
    if (n < a.N) {
      const int64_t t = load_target(target, n);
      const int64_t dt = t - v0 - wm * C::WTM;
      if (t < a.V && dt >= 0 && dt < C::WTM) {
#pragma unroll
        for (int i = 0; i < C::MT; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (acc_row<C>(0, i, r, g) == dt) a.tlogit[n] = acc.t[i][j][r];
      }
    }
  }
  __syncthreads();
  if (wm == 0 && g == 0) {
#pragma unroll
    for (int j = 0; j < C::NT; ++j) {
      const int col = acc_col<C>(wn, j, l32);
      const int64_t n = n0 + col;
      if (n < a.N) {
        float s = red[0][col];
#pragma unroll
        for (int k = 1; k < C::WM; ++k) s += red[k][col];
        a.pmax[(int64_t)tm * a.N + n] = mx[j];
        a.psum[(int64_t)tm * a.N + n] = s;
      }
    }
  }
}

__global__ void __launch_bounds__(256)
fill_f32(float* __restrict__ p, int64_t n, float value) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = value;
}

// Combine (max, sum) pairs: sum is relative to its max.
__device__ __forceinline__ void lse_merge(float& m, float& s, float m2, float s2) {
  const float mn = fmaxf(m, m2);
  if (mn == -INFINITY) return;
  s = s * fast_exp2((m - mn) * kLog2e) + s2 * fast_exp2((m2 - mn) * kLog2e);
  m = mn;
}

// kRowsSplit threads per token; the partial vocab blocks b = k, k+8, ... of
// one thread are merged online, then the 8 threads merge in a fixed order.
// Tokens run fastest across the lanes (thread t: token t % 32, part t / 32),
// so each load instruction reads 32 consecutive tokens of one vocab block
// (the partials are [vocab block][token]).
template <typename TT>
__global__ void __launch_bounds__(kRowsBlock)
lce_fwd_rows(const float* __restrict__ pmax, const float* __restrict__ psum,
             const float* __restrict__ tlogit, const TT* __restrict__ target,
             int64_t ignore_index, float* __restrict__ lse, double* __restrict__ block_nll,
             int* __restrict__ block_cnt, int64_t N, int tiles_v) {
  __shared__ float sm_m[kRowsBlock], sm_s[kRowsBlock];
  __shared__ double sm_nll[kRowsBlock / kRowsSplit];
  __shared__ int sm_cnt[kRowsBlock / kRowsSplit];
  constexpr int kTok = kRowsBlock / kRowsSplit;  // tokens per block
  const int tok = threadIdx.x % kTok, part = threadIdx.x / kTok;
  const int64_t n = (int64_t)blockIdx.x * (kRowsBlock / kRowsSplit) + tok;
  float m = -INFINITY, s = 0.f;
  if (n < N) {
    // eight blocks' partials loaded together, then merged in block order
    constexpr int kBatch = 8;
    for (int b0 = part; b0 < tiles_v; b0 += kRowsSplit * kBatch) {
      float bm[kBatch], bs[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int b = b0 + u * kRowsSplit;
        bm[u] = b < tiles_v ? pmax[(int64_t)b * N + n] : -INFINITY;
        bs[u] = b < tiles_v ? psum[(int64_t)b * N + n] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u)
        if (b0 + u * kRowsSplit < tiles_v) lse_merge(m, s, bm[u], bs[u]);
    }
  }
  sm_m[threadIdx.x] = m;
  sm_s[threadIdx.x] = s;
  __syncthreads();
  if (part == 0) {
    double nll = 0.0;
    int cnt = 0;
    if (n < N) {
      for (int k = 1; k < kRowsSplit; ++k) lse_merge(m, s, sm_m[tok + k * kTok], sm_s[tok + k * kTok]);
      const float l = m + logf(s);
      lse[n] = l;
      const int64_t t = load_target(target, n);
      if (t != ignore_index) {
        nll = (double)(l - tlogit[n]);
        cnt = 1;
      }
    }
    sm_nll[tok] = nll;
    sm_cnt[tok] = cnt;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double acc = 0.0;
    int cnt = 0;
    for (int k = 0; k < kRowsBlock / kRowsSplit; ++k) {
      acc += sm_nll[k];
      cnt += sm_cnt[k];
    }
    block_nll[blockIdx.x] = acc;
    block_cnt[blockIdx.x] = cnt;
  }
}

__global__ void __launch_bounds__(256)
lce_fwd_finalize(const double* __restrict__ block_nll, const int* __restrict__ block_cnt,
                 int n_blocks, float* __restrict__ loss, float* __restrict__ n_valid) {
  __shared__ double sn[256];
  __shared__ long long sc[256];
  double acc = 0.0;
  long long cnt = 0;
  for (int b = threadIdx.x; b < n_blocks; b += 256) {
    acc += block_nll[b];
    cnt += block_cnt[b];
  }
  sn[threadIdx.x] = acc;
  sc[threadIdx.x] = cnt;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (threadIdx.x < w) {
      sn[threadIdx.x] += sn[threadIdx.x + w];
      sc[threadIdx.x] += sc[threadIdx.x + w];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    // mean over non-ignored rows; no valid row gives 0/0 = NaN (torch semantics)
    loss[0] = (float)(sn[0] / (double)sc[0]);
    if (n_valid != nullptr) n_valid[0] = (float)sc[0];
  }
}

// ------------------------------------------------------------ backward ----
template <typename TT>
__global__ void __launch_bounds__(1024)
lce_count_valid(const TT* __restrict__ target, int64_t N, int64_t ignore_index,
                float* __restrict__ n_valid) {
  __shared__ int red[1024];
  int c = 0;
  for (int64_t n = threadIdx.x; n < N; n += 1024) c += (load_target(target, n) != ignore_index);
  red[threadIdx.x] = c;
  __syncthreads();
  for (int w = 512; w > 0; w >>= 1) {
    if (threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) n_valid[0] = (float)red[0];
}

struct GArgs {
  const void* hidden;   // [N, D]
  const void* weight;   // rows [vc0, vc0 + Vc) of [V, D]
  const void* target;   // [N]
  const float* lse;     // [N]
  const float* grad_out;
  const float* n_valid;
  void* gm;             // [N, ld_g]
  int64_t N, D, Vc, ld, ld_g, vc0, ignore_index;
  int tiles_v, tiles_n;
};

template <typename T, typename TT>
__global__ void __launch_bounds__(CfgT<T>::THREADS)
lce_g_kernel(GArgs a) {
  typedef CfgT<T> C;
  __shared__ __attribute__((aligned(1024))) char smem[C::SMEM_BYTES];
  int tm, tn;
  gemm::tile_of(blockIdx.x, gridDim.x, a.tiles_v, a.tiles_n, tm, tn);
  gemm::Problem p{a.weight, a.hidden, a.ld, a.ld, a.Vc, a.N, a.D};
  Acc<C> acc;
  gemm::mainloop<C, T>(p, tm, tn, smem, acc);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l32 = lane & 31, g = lane >> 5;
  const int wm = wave / C::WN, wn = wave % C::WN;
  const int64_t v0 = (int64_t)tm * C::BM, n0 = (int64_t)tn * C::BN;
  const float coef_all = a.grad_out[0] / a.n_valid[0];
  T* gm = (T*)a.gm;
  // G [N, Vc] is row-major by token while a lane holds 4 consecutive vocab
  // rows of one token: stored directly, every store instruction would touch
  // 32 token rows.  For 16-bit G the tile goes through the (now idle) LDS as
  // [token][vocab] and leaves as whole 512-byte token rows.  Staging layout:
  // the 8-byte slot s of token row r sits at slot s ^ (r & 63), so that the
  // 32 tokens of a half-wavefront write distinct banks.
  constexpr bool kStage = sizeof(T) == 2 && C::BM * 2 == 512 && C::BM * C::BN * 2 <= C::SMEM_BYTES;
  char* const tile = smem;
#pragma unroll
  for (int j = 0; j < C::NT; ++j) {
    const int tok = acc_col<C>(wn, j, l32);  // token inside the tile
    const int64_t n = n0 + tok;
    const bool nvalid = n < a.N;
    const float l2 = nvalid ? a.lse[n] * kLog2e : 0.f;
    const int64_t t = nvalid ? load_target((const TT*)a.target, n) : a.ignore_index;
    const float coef = (t == a.ignore_index) ? 0.f : coef_all;
    const int64_t tl = t - a.vc0;  // target row inside this chunk
    if constexpr (kStage) {
      // exp(S - lse) * coef everywhere, then the target entry rewritten as
      // (p - 1) * coef by the one lane holding it (a branch almost every
      // wavefront skips): the same arithmetic as forming each entry with
      // its one-hot term, without a 64-bit compare per entry
#pragma unroll
      for (int i = 0; i < C::MT; ++i)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          float gv[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) gv[e] = fast_exp2(acc.t[i][j][4 * rr + e] * kLog2e - l2) * coef;
          stage_put4(tile, tok, acc_row<C>(wm, i, 4 * rr, g), pack4<T>(gv));
        }
      const int64_t dt = tl - v0 - wm * C::WTM;  // target row inside this wavefront's rows
      if (dt >= 0 && dt < C::WTM) {
#pragma unroll
        for (int i = 0; i < C::MT; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (acc_row<C>(0, i, r, g) == dt) {
              const float gv = (fast_exp2(acc.t[i][j][r] * kLog2e - l2) - 1.f) * coef;
              const int vl = acc_row<C>(wm, i, r, g);
              *reinterpret_cast<uint16_t*>(tile + tok * 512 + (((vl >> 2) ^ (tok & 63)) << 3) +
                                           2 * (vl & 3)) = bits16(from_f32<T>(gv));
            }
      }
    } else {
#pragma unroll
      for (int i = 0; i < C::MT; ++i) {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int64_t vb = v0 + acc_row<C>(wm, i, 4 * rr, g);  // 4 consecutive vocab rows
          float gv[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float pr = fast_exp2(acc.t[i][j][4 * rr + e] * kLog2e - l2);
            gv[e] = (pr - (vb + e == tl ? 1.f : 0.f)) * coef;
          }
          if (!nvalid) continue;
          T* dst = gm + n * a.ld_g + vb;
          if (vb + 4 <= a.Vc) {
            store_f32<T, 4>(dst, gv);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (vb + e < a.Vc) dst[e] = from_f32<T>(gv[e]);
          }
        }
      }
    }
  }
  if constexpr (kStage) {
    __syncthreads();
    stage_out<C::THREADS, C::BN>(tile, (uint16_t*)gm, a.ld_g, n0, v0, a.N, a.Vc);
  }
}

// Plain GEMM: out[m, n] = (acc_in[m, n] if acc_in) + (A B^T)[m, n], A and B
// in the layouts TA, TB select (gemm_nt.h).
// With gridDim.y = S > 1 the reduction is split: split s takes K range
// [s ks, min((s + 1) ks, K)) and writes (and reads acc_in) at an offset of
// s * split_stride elements -- fp32 partials that a fixed-order sum finishes.
template <typename T, typename OT, bool TA, bool TB>
__global__ void __launch_bounds__(CfgT<T>::THREADS)
gemm_store_kernel(gemm::Problem p, const float* acc_in, OT* out, int64_t ldc, int tiles_m,
                  int tiles_n, int64_t ks, int64_t split_stride) {
  typedef CfgT<T> C;
  __shared__ __attribute__((aligned(1024))) char smem[C::SMEM_BYTES];
  int tm, tn;
  gemm::tile_of(blockIdx.x, gridDim.x, tiles_m, tiles_n, tm, tn);
  if (gridDim.y > 1) {
    const int64_t s = blockIdx.y, k0 = s * ks;
    p.K = gemm::imin(ks, p.K - k0);
    p.a = (const T*)p.a + (TA ? k0 * p.lda : k0);
    p.b = (const T*)p.b + (TB ? k0 * p.ldb : k0);
    out += s * split_stride;
    if (acc_in != nullptr) acc_in += s * split_stride;
  }
  Acc<C> acc;
  gemm::mainloop<C, T, TA, TB>(p, tm, tn, smem, acc);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l32 = lane & 31, g = lane >> 5;
  const int wm = wave / C::WN, wn = wave % C::WN;
  const int64_t m0 = (int64_t)tm * C::BM, n0 = (int64_t)tn * C::BN;
  if constexpr (C::WTM * C::BN * 4 <= C::SMEM_BYTES && C::BN % 128 == 0) {
    // Through the (now idle) LDS, one wavefront row of sub-tiles at a time:
    // the WTM x BN fp32 block of the wavefronts with wm == h is staged
    // row-major (columns XOR 32 on every other group of 4 rows, so the two
    // half-wavefronts of a store write distinct banks), then every thread
    // moves 4 consecutive columns: whole rows leave as 16-byte (fp32) or
    // 8-byte (16-bit) stores instead of one 2- or 4-byte store per element.
    float* st = reinterpret_cast<float*>(smem);
    const bool vec_ok = ldc % 4 == 0 && ((uintptr_t)out | (uintptr_t)acc_in) % 16 == 0;
    constexpr int RPI = C::THREADS * 4 / C::BN;  // rows per iteration
#pragma unroll 1
    for (int h = 0; h < C::WM; ++h) {
      if (wm == h) {
#pragma unroll
        for (int i = 0; i < C::MT; ++i)
#pragma unroll
          for (int j = 0; j < C::NT; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int row = acc_row<C>(0, i, r, g), col = acc_col<C>(wn, j, l32);
              st[row * C::BN + (col ^ (((row >> 2) & 1) << 5))] = acc.t[i][j][r];
            }
      }
      __syncthreads();
#pragma unroll 4
      for (int it = 0; it < C::WTM / RPI; ++it) {
        const int idx = it * C::THREADS + threadIdx.x;
        const int row = idx / (C::BN / 4), c = (idx % (C::BN / 4)) * 4;
        const int64_t m = m0 + h * C::WTM + row, n = n0 + c;
        if (m >= p.M || n >= p.N) continue;
        float4 v = *reinterpret_cast<const float4*>(st + row * C::BN + (c ^ (((row >> 2) & 1) << 5)));
        if (vec_ok && n + 4 <= p.N) {
          if (acc_in != nullptr) {
            const float4 a = *reinterpret_cast<const float4*>(acc_in + m * ldc + n);
            v.x += a.x; v.y += a.y; v.z += a.z; v.w += a.w;
          }
          const float f[4] = {v.x, v.y, v.z, v.w};
          store_f32<OT, 4>(out + m * ldc + n, f);
        } else {
          const float f[4] = {v.x, v.y, v.z, v.w};
          for (int e = 0; e < 4 && n + e < p.N; ++e)
            out[m * ldc + n + e] = from_f32<OT>(f[e] + (acc_in != nullptr ? acc_in[m * ldc + n + e] : 0.f));
        }
      }
      __syncthreads();
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < C::NT; ++j) {
    const int64_t n = n0 + acc_col<C>(wn, j, l32);
    if (n >= p.N) continue;
#pragma unroll
    for (int i = 0; i < C::MT; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t m = m0 + acc_row<C>(wm, i, r, g);
        if (m < p.M) {
          float v = acc.t[i][j][r];
          if (acc_in != nullptr) v += acc_in[m * ldc + n];
          out[m * ldc + n] = from_f32<OT>(v);
        }
      }
  }
}

// ----------------------------------------------------------- host side ----
int64_t round_up(int64_t x, int64_t m) { return cdiv(x, m) * m; }

struct FwdLayout {
  int tiles_v, tiles_n, rows_blocks;
  size_t pmax, psum, tlogit, bnll, bcnt, total;
};

FwdLayout fwd_layout(int64_t N, int64_t V, int bm, int bn) {
  FwdLayout L;
  L.tiles_v = (int)cdiv(V, bm);
  L.tiles_n = (int)cdiv(N, bn);
  L.rows_blocks = (int)cdiv(N, kRowsBlock / kRowsSplit);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += (size_t)round_up((int64_t)bytes, 256);
    return at;
  };
  L.pmax = take((size_t)L.tiles_v * N * 4);
  L.psum = take((size_t)L.tiles_v * N * 4);
  L.tlogit = take((size_t)N * 4);
  L.bnll = take((size_t)L.rows_blocks * 8);
  L.bcnt = take((size_t)L.rows_blocks * 4);
  L.total = off;
  return L;
}

// K splits for an M x N product over K: the smallest power of two (at most 8,
// at least 16 K tiles per split) whose grid fills the GPU twice; 1 for grids
// that already do (config 4's dH and dW).
template <typename T>
int split_count(int64_t M, int64_t N, int64_t K) {
  typedef CfgT<T> C;
  const int64_t tiles = cdiv(M, C::BM) * cdiv(N, C::BN), target = 2 * (int64_t)cu_count();
  int s = 1;
  while (s < 8 && tiles * s < target && K / (2 * s) >= 16 * gemm::bk<C, T>()) s *= 2;
  return s;
}

struct BwdLayout {
  int64_t chunk, n_chunks, ld_g;
  int sh, sw;  // K splits of the dH and dW products
  size_t n_valid, gm, dh_acc, dw_part, total;
};

// The backward's workspace: the count of valid rows, G of one vocabulary
// chunk [N, ld_g] (chunk rows chosen so that G fits kGBudget bytes, or
// chunk_rows rounded up to the row tile), the fp32 dH accumulator [sh, N, D]
// when there is more than one chunk or dH is split over K, and the fp32 dW
// partials [sw, chunk, D] when dW is split.
template <typename T>
BwdLayout bwd_layout(int64_t N, int64_t D, int64_t V, bool need_dh, bool need_dw,
                     int64_t chunk_rows) {
  const int esz = (int)sizeof(T);
  BwdLayout L;
  const int64_t vpad = round_up(V, kMaxBM);
  int64_t chunk = chunk_rows > 0 ? round_up(chunk_rows, kMaxBM)
                                 : (kGBudget / std::max<int64_t>(1, N * esz)) / kMaxBM * kMaxBM;
  // G rows are the K-contiguous A operand of dH: 256 of them must span less
  // than 4 GiB (32-bit DMA offsets of the GEMM core)
  chunk = std::max<int64_t>(kMaxBM, std::min<int64_t>({chunk, vpad, ((int64_t)1 << 23) - kMaxBM}));
  L.chunk = chunk;
  L.n_chunks = cdiv(V, chunk);
  L.ld_g = round_up(std::min<int64_t>(chunk, V), 8);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += (size_t)round_up((int64_t)bytes, 256);
    return at;
  };
  L.sh = need_dh ? split_count<T>(N, D, std::min(chunk, V)) : 1;
  L.sw = need_dw ? split_count<T>(std::min(chunk, V), D, N) : 1;
  L.n_valid = take(4);
  L.gm = take((size_t)N * L.ld_g * esz);
  L.dh_acc = (need_dh && (L.n_chunks > 1 || L.sh > 1)) ? take((size_t)L.sh * N * D * 4) : 0;
  L.dw_part = (need_dw && L.sw > 1) ? take((size_t)L.sw * std::min(chunk, V) * D * 4) : 0;
  L.total = off;
  return L;
}

int check_sizes(int64_t N, int64_t D, int64_t V, int dtype) {
  if (N < 0 || D <= 0 || V <= 0)
    return fail(TRI_EINVAL, "linear_ce: bad shape N=%lld D=%lld V=%lld", (long long)N,
                (long long)D, (long long)V);
  const int ve = dtype == kF32 ? 4 : 8;
  if (D % ve != 0)
    return fail(TRI_EINVAL, "linear_ce: hidden_size %lld must be a multiple of %d", (long long)D, ve);
  if (cdiv(V, 128) * cdiv(N, 128) >= ((int64_t)1 << 31) || N >= ((int64_t)1 << 31) ||
      cdiv(V, 64) > 65535 || cdiv(N, 64) > 65535)
    return fail(TRI_EINVAL, "linear_ce: problem too large");
  // the GEMM core's per-lane DMA offsets are 32-bit: 256 rows of hidden_size elements
  if (D >= ((int64_t)1 << 23))
    return fail(TRI_EINVAL, "linear_ce: hidden_size %lld must be below 2^23", (long long)D);
  return TRI_OK;
}

// out (+)= A B^T; with splits > 1, K is cut into `splits` ranges of whole K
// tiles, each writing fp32 partials at out + s * M * ldc (acc_in alike).
template <typename T, bool TA, bool TB>
int gemm_store(const gemm::Problem& p, const float* acc_in, void* out, bool out_f32, int64_t ldc,
               hipStream_t st, int splits = 1) {
  typedef CfgT<T> C;
  const int tiles_m = (int)cdiv(p.M, C::BM), tiles_n = (int)cdiv(p.N, C::BN);
  const unsigned blocks = (unsigned)((int64_t)tiles_m * tiles_n);
  const int64_t bkk = gemm::bk<C, T>();
  const int64_t ks = splits > 1 ? cdiv(cdiv(p.K, splits), bkk) * bkk : p.K;
  splits = splits > 1 ? (int)cdiv(p.K, ks) : 1;
  const dim3 grid(blocks, (unsigned)splits);
  const int64_t stride = p.M * ldc;
  if (out_f32)
    gemm_store_kernel<T, float, TA, TB><<<grid, C::THREADS, 0, st>>>(p, acc_in, (float*)out, ldc,
                                                                     tiles_m, tiles_n, ks, stride);
  else
    gemm_store_kernel<T, T, TA, TB><<<grid, C::THREADS, 0, st>>>(p, acc_in, (T*)out, ldc,
                                                                 tiles_m, tiles_n, ks, stride);
  return check_launch("linear_ce gemm");
}


template <typename T, typename TT>
int fwd_impl(const void* hidden, const void* weight, const void* target, int64_t ignore_index,
             float* loss, float* lse, float* n_valid, void* ws, size_t ws_bytes, int64_t N,
             int64_t D, int64_t V, hipStream_t st) {
  typedef CfgT<T> C;
  const FwdLayout L = fwd_layout(N, V, C::BM, C::BN);
  if (ws_bytes < L.total) return fail(TRI_EINVAL, "linear_ce forward: workspace too small");
  char* w = (char*)ws;
  FwdArgs a;
  a.hidden = hidden; a.weight = weight; a.target = target;
  a.pmax = (float*)(w + L.pmax);
  a.psum = (float*)(w + L.psum);
  a.tlogit = (float*)(w + L.tlogit);
  a.N = N; a.D = D; a.V = V; a.ld = D;
  a.tiles_v = L.tiles_v; a.tiles_n = L.tiles_n;
  // a target outside [0, V) that is not ignore_index leaves NaN here (-> NaN loss);
  // a fill kernel rather than a memset node, so the call can be graph-captured
  fill_f32<<<(unsigned)cdiv(N, 256), 256, 0, st>>>(a.tlogit, N, __builtin_nanf(""));
  if (int e = check_launch("linear_ce forward fill")) return e;
  lce_fwd_kernel<T, TT><<<(unsigned)((int64_t)L.tiles_v * L.tiles_n), C::THREADS, 0, st>>>(a);
  if (int e = check_launch("linear_ce forward gemm")) return e;
  lce_fwd_rows<TT><<<(unsigned)L.rows_blocks, kRowsBlock, 0, st>>>(
      a.pmax, a.psum, a.tlogit, (const TT*)target, ignore_index, lse, (double*)(w + L.bnll),
      (int*)(w + L.bcnt), N, L.tiles_v);
  if (int e = check_launch("linear_ce forward rows")) return e;
  lce_fwd_finalize<<<1, 256, 0, st>>>((const double*)(w + L.bnll), (const int*)(w + L.bcnt),
                                      L.rows_blocks, loss, n_valid);
  return check_launch("linear_ce forward finalize");
}

template <typename T, typename TT>
int bwd_impl(const float* grad_out, const void* hidden, const void* weight, const void* target,
             int64_t ignore_index, const float* lse, void* dhidden, void* dweight, void* ws,
             size_t ws_bytes, int64_t N, int64_t D, int64_t V, int64_t chunk_rows,
             hipStream_t st) {
  static_assert(sizeof(T) == 2, "16-bit backward (MN-contiguous GEMM operands)");
  const bool need_dh = dhidden != nullptr, need_dw = dweight != nullptr;
  if (!need_dh && !need_dw) return TRI_OK;
  const BwdLayout L = bwd_layout<T>(N, D, V, need_dh, need_dw, chunk_rows);
  if (ws_bytes < L.total) return fail(TRI_EINVAL, "linear_ce backward: workspace too small");
  char* w = (char*)ws;
  float* n_valid = (float*)(w + L.n_valid);
  lce_count_valid<TT><<<1, 1024, 0, st>>>((const TT*)target, N, ignore_index, n_valid);
  if (int e = check_launch("linear_ce count")) return e;
  T* gm = (T*)(w + L.gm);
  float* dh_acc = L.dh_acc ? (float*)(w + L.dh_acc) : nullptr;
  float* dw_part = L.dw_part ? (float*)(w + L.dw_part) : nullptr;
  for (int64_t c = 0; c < L.n_chunks; ++c) {
    const int64_t vc0 = c * L.chunk;
    const int64_t vc = std::min<int64_t>(L.chunk, V - vc0);
    GArgs ga;
    ga.hidden = hidden;
    ga.weight = (const T*)weight + vc0 * D;
    ga.target = target;
    ga.lse = lse;
    ga.grad_out = grad_out;
    ga.n_valid = n_valid;
    ga.gm = gm;
    ga.N = N; ga.D = D; ga.Vc = vc; ga.ld = D;
    ga.ld_g = L.ld_g; ga.vc0 = vc0; ga.ignore_index = ignore_index;
    ga.tiles_v = (int)cdiv(vc, CfgT<T>::BM);
    ga.tiles_n = (int)cdiv(N, CfgT<T>::BN);
    lce_g_kernel<T, TT><<<(unsigned)((int64_t)ga.tiles_v * ga.tiles_n), CfgT<T>::THREADS, 0, st>>>(ga);
    if (int e = check_launch("linear_ce gradient tile")) return e;
    const T* wc = (const T*)weight + vc0 * D;
    if (need_dw) {
      // dW[vc0 : vc0 + vc, :] = G^T H: A[v][n] = G[n][v] and B[d][n] = H[n][d],
      // both MN-contiguous; the token reduction in one product (or in sw
      // fp32 partials summed in order), rounded once
      gemm::Problem p{gm, hidden, L.ld_g, D, vc, D, N};
      T* dst = (T*)dweight + vc0 * D;
      if (L.sw == 1) {
        if (int e = gemm_store<T, true, true>(p, nullptr, dst, false, D, st)) return e;
      } else {
        if (int e = gemm_store<T, true, true>(p, nullptr, dw_part, true, D, st, L.sw)) return e;
        if (int e = tritium_sum_splits(dw_part, dst, L.sw, vc * D, std::is_same<T, bf16_t>::value ? kBF16 : kF16, st))
          return e;
      }
    }
    if (need_dh) {
      // dH[N, D] (+)= G W_c: A = G (K-contiguous), B[d][v] = W_c[v][d] (MN-contiguous);
      // with one chunk and no split straight into dH, else into sh fp32
      // accumulators (one per K split, each summed over the chunks in order)
      // that a fixed-order sum rounds once after the last chunk
      gemm::Problem p{gm, wc, L.ld_g, D, N, D, vc};
      const bool last = c + 1 == L.n_chunks;
      if (dh_acc == nullptr) {
        if (int e = gemm_store<T, false, true>(p, nullptr, dhidden, false, D, st)) return e;
      } else if (L.sh == 1 && last) {
        if (int e = gemm_store<T, false, true>(p, dh_acc, dhidden, false, D, st)) return e;
      } else {
        if (int e = gemm_store<T, false, true>(p, c > 0 ? dh_acc : nullptr, dh_acc, true, D, st, L.sh))
          return e;
        if (last) {
          if (int e = tritium_sum_splits(dh_acc, dhidden, L.sh, N * D, std::is_same<T, bf16_t>::value ? kBF16 : kF16, st))
            return e;
        }
      }
    }
  }
  return TRI_OK;
}

// G for vocabulary rows [v0, v0 + vc) only (no G^T), row stride ld_g.
template <typename T, typename TT>
int grad_logits_impl(const float* grad_out, const float* n_valid, const void* hidden,
                     const void* weight, const void* target, int64_t ignore_index,
                     const float* lse, void* g, int64_t ld_g, int64_t N, int64_t D, int64_t v0,
                     int64_t vc, hipStream_t st) {
  GArgs ga;
  ga.hidden = hidden;
  ga.weight = (const T*)weight + v0 * D;
  ga.target = target;
  ga.lse = lse;
  ga.grad_out = grad_out;
  ga.n_valid = n_valid;
  ga.gm = g;
  ga.N = N; ga.D = D; ga.Vc = vc; ga.ld = D;
  ga.ld_g = ld_g; ga.vc0 = v0; ga.ignore_index = ignore_index;
  ga.tiles_v = (int)cdiv(vc, CfgT<T>::BM);
  ga.tiles_n = (int)cdiv(N, CfgT<T>::BN);
  lce_g_kernel<T, TT><<<(unsigned)((int64_t)ga.tiles_v * ga.tiles_n), CfgT<T>::THREADS, 0, st>>>(ga);
  return check_launch("linear_ce gradient of the logits");
}

#define TRI_DISPATCH_TARGET(kind, TT, ...)                                         \
  do {                                                                             \
    if ((kind) == 1) { typedef int32_t TT; __VA_ARGS__; }                          \
    else if ((kind) == 2) { typedef int64_t TT; __VA_ARGS__; }                     \
    else return fail(TRI_EINVAL, "linear_ce: bad target kind %d", (int)(kind));    \
  } while (0)

}  // namespace
}  // namespace tri

using namespace tri;

extern "C" size_t tritium_linear_ce_fwd_workspace_size(int64_t n_rows, int64_t vocab, int dtype) {
  if (n_rows <= 0 || vocab <= 0) return 0;
  if (dtype == kF32) return fwd_layout(n_rows, vocab, CfgT<float>::BM, CfgT<float>::BN).total;
  return fwd_layout(n_rows, vocab, CfgT<bf16_t>::BM, CfgT<bf16_t>::BN).total;
}

extern "C" int tritium_linear_ce_fwd(const void* hidden, const void* weight, const void* target,
                                     int target_kind, int64_t ignore_index, float* loss,
                                     float* lse, float* n_valid, void* workspace,
                                     size_t workspace_bytes, int64_t n_rows, int64_t hidden_size,
                                     int64_t vocab, int dtype, void* stream) {
  if (int e = check_sizes(n_rows, hidden_size, vocab, dtype)) return e;
  if (n_rows == 0) return TRI_OK;
  if (!aligned16(hidden) || !aligned16(weight))
    return fail(TRI_EINVAL, "linear_ce: hidden and weight must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  TRI_DISPATCH_TARGET(target_kind, TT,
    TRI_DISPATCH_FLOAT(dtype, T,
      return fwd_impl<T, TT>(hidden, weight, target, ignore_index, loss, lse, n_valid, workspace,
                             workspace_bytes, n_rows, hidden_size, vocab, st)));
  return TRI_OK;
}

extern "C" size_t tritium_linear_ce_bwd_workspace_size(int64_t n_rows, int64_t hidden_size,
                                                       int64_t vocab, int dtype,
                                                       int need_dhidden, int need_dweight,
                                                       int64_t chunk_rows) {
  if (n_rows <= 0 || vocab <= 0 || hidden_size <= 0 || dtype == kF32) return 0;
  return bwd_layout<bf16_t>(n_rows, hidden_size, vocab, need_dhidden != 0, need_dweight != 0,
                            chunk_rows)
      .total;
}

extern "C" int tritium_linear_ce_bwd(const float* grad_out, const void* hidden, const void* weight,
                                     const void* target, int target_kind, int64_t ignore_index,
                                     const float* lse, void* dhidden, void* dweight,
                                     void* workspace, size_t workspace_bytes, int64_t n_rows,
                                     int64_t hidden_size, int64_t vocab, int64_t chunk_rows,
                                     int dtype, void* stream) {
  if (int e = check_sizes(n_rows, hidden_size, vocab, dtype)) return e;
  if (dtype == kF32) return fail(TRI_EINVAL, "linear_ce backward: 16-bit inputs only");
  if (n_rows == 0) return TRI_OK;
  if (!aligned16(hidden) || !aligned16(weight) || (dhidden && !aligned16(dhidden)) ||
      (dweight && !aligned16(dweight)) || !aligned16(workspace))
    return fail(TRI_EINVAL, "linear_ce: buffers must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  TRI_DISPATCH_TARGET(target_kind, TT,
    TRI_DISPATCH_FLOAT(dtype, T, if constexpr (sizeof(T) == 2) {
      return bwd_impl<T, TT>(grad_out, hidden, weight, target, ignore_index, lse, dhidden,
                             dweight, workspace, workspace_bytes, n_rows, hidden_size, vocab,
                             chunk_rows, st);
    }));
  return TRI_OK;
}

extern "C" int tritium_linear_ce_grad_logits(const float* grad_out, const float* n_valid,
                                             const void* hidden, const void* weight,
                                             const void* target, int target_kind,
                                             int64_t ignore_index, const float* lse, void* g,
                                             int64_t ld_g, int64_t n_rows, int64_t hidden_size,
                                             int64_t vocab, int64_t v0, int64_t vc, int dtype,
                                             void* stream) {
  if (int e = check_sizes(n_rows, hidden_size, vocab, dtype)) return e;
  if (v0 < 0 || vc < 0 || v0 + vc > vocab || ld_g < vc)
    return fail(TRI_EINVAL, "linear_ce grad_logits: bad chunk v0=%lld vc=%lld ld_g=%lld of vocab %lld",
                (long long)v0, (long long)vc, (long long)ld_g, (long long)vocab);
  if (n_rows == 0 || vc == 0) return TRI_OK;
  if (!aligned16(hidden) || !aligned16(weight) || !aligned16(g) || ld_g % 8 != 0)
    return fail(TRI_EINVAL, "linear_ce grad_logits: buffers must be 16-byte aligned, ld_g a multiple of 8");
  hipStream_t st = (hipStream_t)stream;
  TRI_DISPATCH_TARGET(target_kind, TT,
    TRI_DISPATCH_FLOAT(dtype, T,
      return grad_logits_impl<T, TT>(grad_out, n_valid, hidden, weight, target, ignore_index, lse,
                                     g, ld_g, n_rows, hidden_size, v0, vc, st)));
  return TRI_OK;
}
