// Embedding backward for gfx950, with the tied output head's weight gradient
// folded in.
//
// The reference's Embedding (alkinun/helion helion/nn.py:24-28) is a gather,
// weight[ids]; its backward is torch's scatter-add (a radix sort of the ids
// plus an indexing kernel) and, for a tied embedding, a separate add of the
// output head's weight gradient.  Here one kernel does both:
//
//   dw_out[v] = round(dw_in[v] + sum over tokens i with ids[i] == v, in token
//                     order, of dx[i])                  (fp32 sum, one rounding)
//
// The tokens are first bucketed by vocabulary row, stably: integer counts
// per (row, chunk of 1024 tokens), an exclusive scan of them, and a scatter
// in which each token's slot is its chunk's offset plus the number of
// earlier tokens of the chunk with the same id -- each row's tokens then lie
// together in token order (integer work only; the result does not depend on
// execution order).  Fixed windows of that list are then summed one
// wavefront each (emb_win_kernel, below: a run of one row inside a window
// is summed in token order and added to the row; a run that crosses windows
// leaves per-window fp32 parts that emb_merge_kernel adds in window order),
// out of place after dw_in is copied to dw_out.  Every row's sum is formed
// in an order fixed by the ids: results are bitwise reproducible, with no
// floating-point atomics and no sort.  Rows no token names are copied (or,
// in place, left alone); ids outside [0, vocab) contribute nothing.
#include "common.h"
#include "../../include/tritium_hip.h"

namespace tri {
namespace {

constexpr int kEmbThreads = 256;

template <typename TT>
__device__ __forceinline__ int64_t load_id(const TT* ids, int64_t i) {
  return (int64_t)ids[i];
}

// ---- bucketing: the tokens of every vocabulary row, in token order
// cnt[v * C + c] = tokens of chunk c (kEmbChunk tokens) whose id is v
constexpr int kEmbChunk = 1024;

template <typename TT>
__global__ void __launch_bounds__(kEmbChunk)
emb_count_kernel(const TT* __restrict__ ids, int64_t n_tok, int64_t vocab, int64_t C,
                 int* __restrict__ cnt) {
  const int64_t i = (int64_t)blockIdx.x * kEmbChunk + threadIdx.x;
  if (i >= n_tok) return;
  const int64_t id = load_id(ids, i);
  if (id < 0 || id >= vocab) return;
  atomicAdd(cnt + id * C + blockIdx.x, 1);  // integer counts: order-independent
}

// Exclusive scan of n ints in two levels: emb_scan_tiles turns each tile of
// kScanTile elements into its local exclusive prefix (coalesced loads, a
// wavefront-then-workgroup scan in LDS) and writes the tile's total;
// emb_scan_totals scans the totals in place in one workgroup.  The prefix of
// element x is then x's local prefix + totals[x / kScanTile].
constexpr int kScanTile = 1024;

__global__ void __launch_bounds__(kScanTile)
emb_scan_tiles(int* __restrict__ x, int64_t n, int* __restrict__ totals) {
  __shared__ int sh[kScanTile];
  const int t = threadIdx.x;
  const int64_t i = (int64_t)blockIdx.x * kScanTile + t;
  const int v = i < n ? x[i] : 0;
  sh[t] = v;
  __syncthreads();
  for (int off = 1; off < kScanTile; off <<= 1) {  // Hillis-Steele inclusive scan
    const int u = t >= off ? sh[t - off] : 0;
    __syncthreads();
    sh[t] += u;
    __syncthreads();
  }
  if (i < n) x[i] = sh[t] - v;
  if (t == kScanTile - 1) totals[blockIdx.x] = sh[t];
}

// exclusive scan of n tile totals by one workgroup, sequential per thread
// over contiguous segments of at most a few elements
__global__ void __launch_bounds__(kScanTile)
emb_scan_totals(int* __restrict__ totals, int64_t n) {
  __shared__ int part[kScanTile];
  const int t = threadIdx.x;
  const int64_t seg = cdiv(n, kScanTile), b0 = t * seg, b1 = min(n, b0 + seg);
  int s = 0;
  for (int64_t i = b0; i < b1; ++i) s += totals[i];
  part[t] = s;
  __syncthreads();
  for (int off = 1; off < kScanTile; off <<= 1) {
    const int u = t >= off ? part[t - off] : 0;
    __syncthreads();
    part[t] += u;
    __syncthreads();
  }
  int run = part[t] - s;
  for (int64_t i = b0; i < b1; ++i) {
    const int v = totals[i];
    totals[i] = run;
    run += v;
  }
  if (t == kScanTile - 1) totals[n] = part[t];  // the grand total
}

__device__ __forceinline__ int scanned(const int* off, const int* totals, int64_t x) {
  return off[x] + totals[x / kScanTile];
}

// list[off[v * C + c] + rank] = token index and rows[...] = v, rank = earlier
// tokens of chunk c with id v: each row's tokens end up contiguous and in
// token order.  A workgroup ranks kEmbThreads tokens against the ids of its
// chunk held in LDS.
template <typename TT>
__global__ void __launch_bounds__(kEmbThreads)
emb_scatter_kernel(const TT* __restrict__ ids, int64_t n_tok, int64_t vocab, int64_t C,
                   const int* __restrict__ off, const int* __restrict__ totals,
                   int* __restrict__ list, int* __restrict__ rows) {
  __shared__ int blk[kEmbChunk];
  const int t = threadIdx.x;
  const int64_t c = (int64_t)blockIdx.x * kEmbThreads / kEmbChunk;  // chunk of this workgroup
  const int64_t c0 = c * kEmbChunk;
  for (int u = t; u < kEmbChunk; u += kEmbThreads) {
    const int64_t j = c0 + u;
    int b = -1;
    if (j < n_tok) {
      const int64_t id = load_id(ids, j);
      if (id >= 0 && id < vocab) b = (int)id;
    }
    blk[u] = b;
  }
  __syncthreads();
  const int64_t i = (int64_t)blockIdx.x * kEmbThreads + t;
  const int me = (int)(i - c0);
  const int b = i < n_tok ? blk[me] : -1;
  if (b < 0) return;
  int rank = 0;
  for (int u = 0; u < me; ++u) rank += blk[u] == b;
  const int pos = scanned(off, totals, (int64_t)b * C + c) + rank;
  list[pos] = (int)i;
  rows[pos] = b;
}

// The bucketed list is cut into windows of kEmbWin positions, one wavefront
// each, so every wavefront sums about the same number of dx rows whatever
// the distribution of the ids (one id repeated over half the tokens still
// spreads over many wavefronts).  Window w covers positions [w W, w W + W):
// its wavefront walks them in order, summing each run of equal rows[] in
// token order in fp32 (dx rows loaded kEmbDepth positions ahead).  A run
// that lies inside the window is added to its row of dw and rounded once; a
// run that crosses a window boundary leaves this window's part as an fp32
// partial row in slot 2w (the run began in an earlier window) or 2w + 1 (it
// begins here and continues past the window) -- a window holds at most one
// of each -- and emb_merge_kernel, in the window where such a run ends,
// adds its parts in window order and rounds once.  The order of every sum
// depends on the ids only: results are bitwise reproducible.
//
// Columns: with VEC, lane l owns the 16-byte group l of each block of 64
// groups (every row, dx stride and pointer a multiple of 16 bytes); else
// columns c0 + l + 64 j, j < 16.  The partial rows use the same mapping.
constexpr int kEmbWin = 16;
constexpr int kEmbDepth = 4;

template <typename T, bool VEC>
struct EmbCols {
  static constexpr int L = VEC ? 16 / (int)sizeof(T) : 16;  // columns per lane per block
  static constexpr int BLK = kWave * L;                     // columns per block
  static __device__ __forceinline__ int64_t col(int64_t c0, int lane, int e) {
    return VEC ? c0 + (int64_t)lane * L + e : c0 + lane + (int64_t)kWave * e;
  }
  static __device__ __forceinline__ void load(const T* __restrict__ row, int64_t c0, int lane,
                                              int64_t dim, float (&x)[L]) {
    if constexpr (VEC) {
      if (col(c0, lane, 0) < dim) {
        const Pack<T, L> pk = *reinterpret_cast<const Pack<T, L>*>(row + col(c0, lane, 0));
#pragma unroll
        for (int e = 0; e < L; ++e) x[e] = to_f32(pk.v[e]);
      } else {
#pragma unroll
        for (int e = 0; e < L; ++e) x[e] = 0.f;
      }
    } else {
#pragma unroll
      for (int e = 0; e < L; ++e) x[e] = col(c0, lane, e) < dim ? to_f32(row[col(c0, lane, e)]) : 0.f;
    }
  }
  // row += acc, rounded once
  static __device__ __forceinline__ void add_round(T* row, int64_t c0, int lane, int64_t dim,
                                                   const float (&acc)[L]) {
    if constexpr (VEC) {
      if (col(c0, lane, 0) < dim) {
        Pack<T, L>* p = reinterpret_cast<Pack<T, L>*>(row + col(c0, lane, 0));
        Pack<T, L> pk = *p;
#pragma unroll
        for (int e = 0; e < L; ++e) pk.v[e] = from_f32<T>(to_f32(pk.v[e]) + acc[e]);
        *p = pk;
      }
    } else {
#pragma unroll
      for (int e = 0; e < L; ++e) {
        const int64_t c = col(c0, lane, e);
        if (c < dim) row[c] = from_f32<T>(to_f32(row[c]) + acc[e]);
      }
    }
  }
};

// rows[] of a window and of its two neighbours, and list[] of the window, in
// lanes (lane i: position k0 - 1 + i; -1 past either end), read back with
// readlane: one load each per wavefront.
struct EmbWinIds {
  int row_l, tok_l;
  __device__ __forceinline__ void load(const int* rows, const int* list, int64_t k0,
                                       int64_t n_list, int lane) {
    const int64_t k = k0 - 1 + lane;
    const bool in = k >= 0 && k < n_list && lane <= kEmbWin + 1;
    row_l = in ? rows[k] : -1;
    tok_l = in ? list[k] : 0;
  }
  __device__ __forceinline__ int row(int i) const { return __shfl(row_l, i + 1, kWave); }
  __device__ __forceinline__ int tok(int i) const { return __shfl(tok_l, i + 1, kWave); }
};

template <typename T, bool VEC>
__global__ void __launch_bounds__(kEmbThreads)
emb_win_kernel(const int* __restrict__ off, const int* __restrict__ totals, int64_t B, int64_t C,
               const int* __restrict__ list, const int* __restrict__ rows,
               const T* __restrict__ dx, int64_t ld_dx, T* dw, int64_t dim,
               float* __restrict__ part) {
  typedef EmbCols<T, VEC> E;
  constexpr int W = kEmbThreads / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t w = (int64_t)blockIdx.x * W + (threadIdx.x >> 6);
  // the list holds only the tokens whose id is in range: its length is the
  // scan's grand total, not the token count
  const int64_t n_list = scanned(off, totals, B * C);
  const int64_t k0 = w * kEmbWin;
  if (k0 >= n_list) return;
  const int n = (int)min((int64_t)kEmbWin, n_list - k0);
  EmbWinIds ids;
  ids.load(rows, list, k0, n_list, lane);
  const int before = ids.row(-1), after = ids.row(n);  // -1 past the list's ends
  for (int64_t c0 = 0; c0 < dim; c0 += E::BLK) {
    float ring[kEmbDepth][E::L], acc[E::L];
#pragma unroll
    for (int d = 0; d < kEmbDepth; ++d)
      if (d < n) E::load(dx + (int64_t)ids.tok(d) * ld_dx, c0, lane, dim, ring[d]);
#pragma unroll
    for (int e = 0; e < E::L; ++e) acc[e] = 0.f;
    int run0 = 0;
    for (int i0 = 0; i0 < n; i0 += kEmbDepth) {
#pragma unroll
      for (int d = 0; d < kEmbDepth; ++d) {
        const int i = i0 + d;
        if (i < n) {
#pragma unroll
          for (int e = 0; e < E::L; ++e) acc[e] += ring[d][e];
          if (i + kEmbDepth < n)
            E::load(dx + (int64_t)ids.tok(i + kEmbDepth) * ld_dx, c0, lane, dim, ring[d]);
          const int v = ids.row(i);
          const bool last = i + 1 == n;
          const int next = last ? after : ids.row(i + 1);
          if (last || next != v) {  // the window's part of the run [run0, i] of row v is complete
            const bool begins_here = run0 > 0 || before != v;
            const bool ends_here = next != v;
            if (begins_here && ends_here) {
              E::add_round(dw + (int64_t)v * dim, c0, lane, dim, acc);
            } else {
              float* pr = part + (2 * w + (begins_here ? 1 : 0)) * dim;
#pragma unroll
              for (int e = 0; e < E::L; ++e) {
                const int64_t c = E::col(c0, lane, e);
                if (c < dim) pr[c] = acc[e];
              }
            }
#pragma unroll
            for (int e = 0; e < E::L; ++e) acc[e] = 0.f;
            run0 = i + 1;
          }
        }
      }
    }
  }
}

// One wavefront per window w: if the run at the window's first position began
// in an earlier window and ends in this one, add its parts -- slot 2 w0 + 1
// of its first window w0, then slot 2 w' of each later window up to w -- in
// that order, and add the sum to its row of dw (one rounding).
template <typename T, bool VEC>
__global__ void __launch_bounds__(kEmbThreads)
emb_merge_kernel(const int* __restrict__ off, const int* __restrict__ totals, int64_t B,
                 int64_t C, const int* __restrict__ list, const int* __restrict__ rows, T* dw,
                 int64_t dim, const float* __restrict__ part) {
  typedef EmbCols<T, VEC> E;
  constexpr int W = kEmbThreads / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t w = (int64_t)blockIdx.x * W + (threadIdx.x >> 6);
  const int64_t n_list = scanned(off, totals, B * C);
  const int64_t k0 = w * kEmbWin;
  if (k0 >= n_list || k0 == 0) return;
  const int n = (int)min((int64_t)kEmbWin, n_list - k0);
  EmbWinIds ids;
  ids.load(rows, list, k0, n_list, lane);
  const int v = ids.row(0);
  if (ids.row(-1) != v) return;                       // the run begins in this window
  if (ids.row(n - 1) == v && ids.row(n) == v) return;  // it continues past the window
  const int64_t w0 = (int64_t)scanned(off, totals, (int64_t)v * C) / kEmbWin;
  for (int64_t c0 = 0; c0 < dim; c0 += E::BLK) {
    float acc[E::L], x[kEmbDepth][E::L];
#pragma unroll
    for (int e = 0; e < E::L; ++e) acc[e] = 0.f;
    auto slot = [&](int64_t ww) { return part + (ww == w0 ? 2 * ww + 1 : 2 * ww) * dim; };
    for (int64_t ww = w0; ww <= w; ww += kEmbDepth) {
#pragma unroll
      for (int d = 0; d < kEmbDepth; ++d) {  // the loads of up to kEmbDepth slots together
        const float* pr = slot(ww + d);
#pragma unroll
        for (int e = 0; e < E::L; ++e) {
          const int64_t c = E::col(c0, lane, e);
          x[d][e] = ww + d <= w && c < dim ? pr[c] : 0.f;
        }
      }
#pragma unroll
      for (int d = 0; d < kEmbDepth; ++d)
#pragma unroll
        for (int e = 0; e < E::L; ++e) acc[e] += x[d][e];
    }
    E::add_round(dw + (int64_t)v * dim, c0, lane, dim, acc);
  }
}

// dst = src, 16 bytes per thread where both are 16-byte aligned
__global__ void __launch_bounds__(kEmbThreads)
emb_copy_kernel(const char* __restrict__ src, char* __restrict__ dst, int64_t bytes) {
  const int64_t i = ((int64_t)blockIdx.x * kEmbThreads + threadIdx.x) * 16;
  if (i + 16 <= bytes) {
    st16(dst + i, ld16(src + i));
  } else {
    for (int64_t b = i; b < bytes; ++b) dst[b] = src[b];
  }
}

__global__ void __launch_bounds__(kEmbThreads)
emb_zero_kernel(int* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * kEmbThreads + threadIdx.x;
  if (i < n) p[i] = 0;
}

struct EmbLayout {
  int64_t B, C, tiles, windows;
  size_t off, totals, list, rows, part, total;
};

// workspace: off [B * C + 1] counts / local prefixes, totals [tiles + 1],
// list [n_tok] token indices and rows [n_tok] their ids (one bucket per
// vocabulary row), part [2 * windows, dim] fp32 partial rows
EmbLayout emb_layout(int64_t n_tok, int64_t vocab, int64_t dim) {
  EmbLayout L;
  L.B = vocab;
  L.C = std::max<int64_t>(1, cdiv(n_tok, kEmbChunk));
  L.tiles = cdiv(L.B * L.C + 1, kScanTile);
  L.windows = std::max<int64_t>(1, cdiv(n_tok, kEmbWin));
  auto up = [](int64_t b) { return (size_t)cdiv(b, 256) * 256; };
  L.off = 0;
  L.totals = up((L.B * L.C + 1) * 4);
  L.list = L.totals + up((L.tiles + 1) * 4);
  L.rows = L.list + up(std::max<int64_t>(1, n_tok) * 4);
  L.part = L.rows + up(std::max<int64_t>(1, n_tok) * 4);
  L.total = L.part + up(2 * L.windows * dim * 4);
  return L;
}

}  // namespace
}  // namespace tri

using namespace tri;

extern "C" size_t tritium_embedding_bwd_workspace_size(int64_t n_tokens, int64_t vocab,
                                                       int64_t dim) {
  if (n_tokens < 0 || vocab <= 0 || dim <= 0) return 0;
  return emb_layout(n_tokens, vocab, dim).total;
}

extern "C" int tritium_embedding_bwd(const void* ids, int id_kind, int64_t n_tokens,
                                     const void* dx, int64_t ld_dx, const void* dw_in,
                                     void* dw_out, int64_t vocab, int64_t dim, void* workspace,
                                     size_t workspace_bytes, int dtype, void* stream) {
  if (n_tokens < 0 || vocab <= 0 || dim <= 0 || ld_dx < dim)
    return fail(TRI_EINVAL, "embedding backward: bad sizes n_tokens=%lld vocab=%lld dim=%lld ld_dx=%lld",
                (long long)n_tokens, (long long)vocab, (long long)dim, (long long)ld_dx);
  if (id_kind != 1 && id_kind != 2)
    return fail(TRI_EINVAL, "embedding backward: bad id kind %d", id_kind);
  if (dtype != kF32 && dtype != kF16 && dtype != kBF16)
    return fail(TRI_EINVAL, "unsupported dtype code %d", dtype);
  if (n_tokens >= ((int64_t)1 << 31) || vocab >= ((int64_t)1 << 31))
    return fail(TRI_EINVAL, "embedding backward: token count and vocab must be below 2^31");
  const EmbLayout L = emb_layout(n_tokens, vocab, dim);
  if (L.B * L.C + 1 >= ((int64_t)1 << 31))
    return fail(TRI_EINVAL, "embedding backward: problem too large");
  if (workspace == nullptr || workspace_bytes < L.total)
    return fail(TRI_EINVAL, "embedding backward: workspace of %zu bytes needed", L.total);
  int* off = (int*)((char*)workspace + L.off);
  int* totals = (int*)((char*)workspace + L.totals);
  int* list = (int*)((char*)workspace + L.list);
  int* rows = (int*)((char*)workspace + L.rows);
  const int64_t n_off = L.B * L.C + 1;
  hipStream_t st = (hipStream_t)stream;
  // counts cleared by a kernel (no memset node: the call can be graph-captured)
  emb_zero_kernel<<<(unsigned)cdiv(n_off, kEmbThreads), kEmbThreads, 0, st>>>(off, n_off);
  if (int e = check_launch("embedding backward zero")) return e;
  // counts, the two-level scan (always: with no token every block's range
  // is then empty), and the stable scatter
  if (n_tokens > 0) {
    if (id_kind == 1)
      emb_count_kernel<int32_t><<<(unsigned)L.C, kEmbChunk, 0, st>>>(
          (const int32_t*)ids, n_tokens, vocab, L.C, off);
    else
      emb_count_kernel<int64_t><<<(unsigned)L.C, kEmbChunk, 0, st>>>(
          (const int64_t*)ids, n_tokens, vocab, L.C, off);
  }
  emb_scan_tiles<<<(unsigned)L.tiles, kScanTile, 0, st>>>(off, n_off, totals);
  emb_scan_totals<<<1, kScanTile, 0, st>>>(totals, L.tiles);
  if (n_tokens > 0) {
    const unsigned sb = (unsigned)cdiv(n_tokens, kEmbThreads);
    if (id_kind == 1)
      emb_scatter_kernel<int32_t><<<sb, kEmbThreads, 0, st>>>(
          (const int32_t*)ids, n_tokens, vocab, L.C, off, totals, list, rows);
    else
      emb_scatter_kernel<int64_t><<<sb, kEmbThreads, 0, st>>>(
          (const int64_t*)ids, n_tokens, vocab, L.C, off, totals, list, rows);
  }
  if (int e = check_launch("embedding backward bucketing")) return e;
  if (dw_in != dw_out) {
    // out of place: copy, then add into the copy
    const int64_t bytes = vocab * dim * dtype_size(dtype);
    if (aligned16(dw_in) && aligned16(dw_out)) {
      emb_copy_kernel<<<(unsigned)cdiv(cdiv(bytes, 16), kEmbThreads), kEmbThreads, 0, st>>>(
          (const char*)dw_in, (char*)dw_out, bytes);
    } else {
      hipError_t err = hipMemcpyAsync(dw_out, dw_in, (size_t)bytes, hipMemcpyDeviceToDevice, st);
      if (err != hipSuccess) return fail(TRI_ELAUNCH, "embedding backward copy: %s", hipGetErrorString(err));
    }
    if (int e = check_launch("embedding backward copy")) return e;
  }
  if (n_tokens == 0) return TRI_OK;
  float* part = (float*)((char*)workspace + L.part);
  const unsigned blocks = (unsigned)cdiv(L.windows, kEmbThreads / kWave);
  const int esz = dtype_size(dtype);
  const bool vec = aligned16(dx) && aligned16(dw_out) && (dim * esz) % 16 == 0 &&
                   (ld_dx * esz) % 16 == 0;
#define EMB_LAUNCH(VEC)                                                                        \
  TRI_DISPATCH_FLOAT(dtype, T, {                                                               \
    emb_win_kernel<T, VEC><<<blocks, kEmbThreads, 0, st>>>(off, totals, L.B, L.C, list, rows,   \
                                                           (const T*)dx, ld_dx, (T*)dw_out,     \
                                                           dim, part);                          \
    if (int e = check_launch("embedding backward")) return e;                                  \
    emb_merge_kernel<T, VEC><<<blocks, kEmbThreads, 0, st>>>(off, totals, L.B, L.C, list, rows, \
                                                             (T*)dw_out, dim, part);            \
  })
  if (vec) EMB_LAUNCH(true);
  else EMB_LAUNCH(false);
#undef EMB_LAUNCH
  return check_launch("embedding backward (merge)");
}
