// Cross-entropy on materialised logits for gfx950.
//
// Reference arithmetic: alkinun/helion tritium/ops/cross_entropy.py:36-68
// (forward: per row lse = log(sum(exp(x - max))) + max in fp32, nll = lse -
// x[target], loss = mean(nll)) and 71-100 (backward: dlogits = (exp(x - lse) -
// onehot(target)) * grad_out / n_rows, stored in the logits dtype).
//
// Both kernels stream the logits once with 16-byte nontemporal accesses.
// Forward: each lane keeps a running (max, sum of exp) over its vectors,
// rescaling the sum once per vector when the max grows; the lanes of a row
// then merge their pairs with cross-lane shuffles (and LDS across the
// wavefronts of a block when a whole block shares one row).  Rows shorter
// than kWideRow get one wavefront each, longer ones a 256-lane block, so both
// small vocabularies with many rows and one long row fill the machine; a few
// long rows are cut into spans over more blocks (ce_span_kernel).  The per-row
// nll values are summed by one wavefront in a fixed order (the reference
// accumulates them with atomics), so the loss is deterministic.  A one-launch
// form (the last block to finish forms the loss behind an arrival counter)
// was measured slower: its agent-scope release and acquire fences cost more
// on this 8-XCD part than the second launch.
#include "common.h"
#include "../../include/tritium_hip.h"

namespace tri {
namespace {

constexpr int kBlock = 256;
constexpr int64_t kWideRow = 8192;        // rows at least this long get a whole block
constexpr int64_t kBwdChunk = 256 * 8 * 4;  // elements of one row per backward block
constexpr int kInFlight = 8;              // 16-byte loads in flight per lane (forward)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// exp(x - m) in base 2 on pre-scaled values: a = x * log2(e), mb = m * log2(e)
__device__ __forceinline__ float exp_shift(float a, float mb) { return fast_exp2(a - mb); }

// Merge (m2, s2) into (m, s): both sums are relative to their own max (in
// log2 units); an all -inf side contributes nothing.
__device__ __forceinline__ void merge_ms(float& m, float& s, float m2, float s2) {
  const float mx = fmaxf(m, m2);
  if (mx == -INFINITY) return;
  s = (m == -INFINITY ? 0.0f : s * fast_exp2(m - mx)) + (m2 == -INFINITY ? 0.0f : s2 * fast_exp2(m2 - mx));
  m = mx;
}

template <typename TT>
__device__ __forceinline__ int64_t target_at(const void* t, int64_t row) {
  return (int64_t)static_cast<const TT*>(t)[row];
}

// One row's (max, sum) in log2 units for the lanes [lane, lane + LANES, ...).
template <typename T, int LANES>
__device__ __forceinline__ void row_ms(const T* __restrict__ x, int64_t V, bool vec_ok, int lane,
                                       float& m, float& s) {
  constexpr int VEC = 16 / sizeof(T);
  m = -INFINITY;
  s = 0.0f;
  int64_t tail = 0;
  // fold one raw 16-byte vector into (m, s)
  auto fold = [&](u32x4 raw) {
    float f[VEC];
    unpack<T>(raw, f);
    float vm = -INFINITY;
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      f[i] *= kLog2e;
      vm = fmaxf(vm, f[i]);
    }
    if (vm > m) {
      s = (m == -INFINITY) ? 0.0f : s * fast_exp2(m - vm);
      m = vm;
    }
    if (m != -INFINITY) {
#pragma unroll
      for (int i = 0; i < VEC; ++i) s += exp_shift(f[i], m);
    }
  };
  if (vec_ok) {
    const int64_t nv = V / VEC;
    // up to kInFlight loads issued together: the fold's branch on the running
    // max would otherwise serialise one memory round trip per vector
    for (int64_t iv = lane; iv < nv; iv += kInFlight * LANES) {
      u32x4 raw[kInFlight];
#pragma unroll
      for (int u = 0; u < kInFlight; ++u)
        if (iv + u * LANES < nv) raw[u] = ld16_nt(x + (iv + u * LANES) * VEC);
#pragma unroll
      for (int u = 0; u < kInFlight; ++u)
        if (iv + u * LANES < nv) fold(raw[u]);
    }
    tail = nv * VEC;
  }
  for (int64_t i = tail + lane; i < V; i += LANES) {
    const float a = to_f32(x[i]) * kLog2e;
    if (a > m) {
      s = (m == -INFINITY) ? 0.0f : s * fast_exp2(m - a);
      m = a;
    }
    if (m != -INFINITY) s += exp_shift(a, m);
  }
}

__device__ __forceinline__ void wave_merge(float& m, float& s) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float m2 = __shfl_xor(m, off, kWave);
    const float s2 = __shfl_xor(s, off, kWave);
    merge_ms(m, s, m2, s2);
  }
}

// LANES = 64: one wavefront per row, 4 rows per block; LANES = 256: one row per block.
template <typename T, typename TT, int LANES>
__global__ void __launch_bounds__(kBlock)
ce_fwd_kernel(const T* __restrict__ logits, const void* __restrict__ target, float* __restrict__ lse,
              float* __restrict__ nll, int64_t n_rows, int64_t V, int vec_ok) {
  constexpr int kRowsPerBlock = kBlock / LANES;
  const int lane = threadIdx.x % LANES;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + threadIdx.x / LANES;
  float m = -INFINITY, s = 0.0f;
  if (row < n_rows) row_ms<T, LANES>(logits + row * V, V, vec_ok != 0, lane, m, s);
  wave_merge(m, s);
  if constexpr (LANES > kWave) {
    __shared__ float sm[kBlock / kWave], ss[kBlock / kWave];
    const int w = threadIdx.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0) {
      sm[w] = m;
      ss[w] = s;
    }
    __syncthreads();
    m = sm[0];
    s = ss[0];
#pragma unroll
    for (int i = 1; i < kBlock / kWave; ++i) merge_ms(m, s, sm[i], ss[i]);
  }
  if (lane == 0 && row < n_rows) {
    // natural-log logsumexp: (m + log2 s) * ln 2
    const float l = (m + __log2f(s)) * kLn2;
    lse[row] = l;
    const int64_t t = target_at<TT>(target, row);
    // an out-of-range target has no logit: its nll (and so the loss) is NaN
    nll[row] = (t >= 0 && t < V) ? l - to_f32(logits[row * V + t]) : __builtin_nanf("");
  }
}

// sum over the 64 lanes of fp64 partials; lane 0's total is formed in a fixed order
__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// loss = sum(nll) / n_rows by one wavefront, summed in a fixed order (fp64
// partials: lane l takes rows l, l + 64, ...).  A single wavefront needs no
// barrier, which keeps this tail launch short (4.0 -> 3.6 us at 128 rows).
__global__ void __launch_bounds__(kWave)
ce_mean_kernel(const float* __restrict__ nll, int64_t n_rows, float* __restrict__ loss) {
  double acc = 0.0;
  int64_t i = threadIdx.x;
  for (; i + 3 * kWave < n_rows; i += 4 * kWave) {
    const float a = nll[i], b = nll[i + kWave], c = nll[i + 2 * kWave], d = nll[i + 3 * kWave];
    acc += (double)a;
    acc += (double)b;
    acc += (double)c;
    acc += (double)d;
  }
  for (; i < n_rows; i += kWave) acc += (double)nll[i];
  acc = wave_sum_f64(acc);
  if (threadIdx.x == 0) loss[0] = (float)(acc / (double)n_rows);
}

// Few long rows (fewer rows than the GPU has room for blocks): each row is
// cut into `chunks` spans of `span` elements (a multiple of 8), one 256-lane
// block per span writes the span's (max, sum) in log2 units; ce_finish_kernel
// merges a row's spans in span order.  A single block per row would leave
// most compute units idle and stream each row through one of them.
template <typename T>
__global__ void __launch_bounds__(kBlock)
ce_span_kernel(const T* __restrict__ logits, float2* __restrict__ part, int64_t V, int64_t span,
               int chunks, int vec_ok) {
  const int64_t row = blockIdx.x / chunks;
  const int c = (int)(blockIdx.x - row * chunks);
  const int64_t c0 = (int64_t)c * span;
  const int64_t len = min(span, V - c0);
  float m = -INFINITY, s = 0.0f;
  row_ms<T, kBlock>(logits + row * V + c0, len, vec_ok != 0, threadIdx.x, m, s);
  wave_merge(m, s);
  __shared__ float sm[kBlock / kWave], ss[kBlock / kWave];
  const int w = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) {
    sm[w] = m;
    ss[w] = s;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    m = sm[0];
    s = ss[0];
#pragma unroll
    for (int i = 1; i < kBlock / kWave; ++i) merge_ms(m, s, sm[i], ss[i]);
    part[blockIdx.x] = make_float2(m, s);
  }
}

// One wavefront: lane l finishes rows l, l + 64, ... (the spans merged in
// order, lse, nll) and the loss is their mean in a fixed order (fp64).
template <typename T, typename TT>
__global__ void __launch_bounds__(kWave)
ce_finish_kernel(const T* __restrict__ logits, const void* __restrict__ target,
                 const float2* __restrict__ part, float* __restrict__ lse, float* __restrict__ loss,
                 int64_t n_rows, int64_t V, int chunks) {
  double acc = 0.0;
  for (int64_t row = threadIdx.x; row < n_rows; row += kWave) {
    const int64_t t = target_at<TT>(target, row);
    const float xt = (t >= 0 && t < V) ? to_f32(logits[row * V + t]) : 0.0f;
    float m = -INFINITY, s = 0.0f;
    for (int c = 0; c < chunks; ++c) {
      const float2 p = part[row * chunks + c];
      merge_ms(m, s, p.x, p.y);
    }
    const float l = (m + __log2f(s)) * kLn2;
    lse[row] = l;
    acc += (t >= 0 && t < V) ? (double)(l - xt) : (double)__builtin_nanf("");
  }
  acc = wave_sum_f64(acc);
  if (threadIdx.x == 0) loss[0] = (float)(acc / (double)n_rows);
}

// Span split of the forward: (chunks, span) with chunks = 1 for the per-row
// kernels.  Rows of at least 2 kMinSpan elements are split when there are
// fewer rows than two blocks per compute unit, into spans of at least
// kMinSpan elements, enough of them to give every compute unit two blocks.
constexpr int64_t kMinSpan = 4096;
void span_split(int64_t n_rows, int64_t V, int& chunks, int64_t& span) {
  chunks = 1;
  span = V;
  const int64_t want = 2 * (int64_t)cu_count();
  if (V < 2 * kMinSpan || n_rows >= want) return;
  const int64_t c = std::min<int64_t>(V / kMinSpan, cdiv(want, n_rows));
  span = cdiv(cdiv(V, c), 8) * 8;
  chunks = (int)cdiv(V, span);
}

// dlogits for one kBwdChunk-element span of one row per block.
template <typename T, typename TT>
__global__ void __launch_bounds__(kBlock)
ce_bwd_kernel(const float* __restrict__ grad_out, const T* __restrict__ logits,
              const void* __restrict__ target, const float* __restrict__ lse, T* __restrict__ dlogits,
              int64_t V, int64_t chunks_per_row, float inv_den, int vec_ok) {
  constexpr int VEC = 16 / sizeof(T);
  const int64_t row = blockIdx.x / chunks_per_row;
  const int64_t c0 = (blockIdx.x - row * chunks_per_row) * kBwdChunk;
  const int64_t c1 = min(c0 + kBwdChunk, V);
  const float scale = grad_out[0] * inv_den;
  const float lb = lse[row] * kLog2e;
  const int64_t t = target_at<TT>(target, row);
  const T* x = logits + row * V;
  T* d = dlogits + row * V;
  int64_t tail = c0;
  if (vec_ok) {
    const int64_t v_end = c0 + ((c1 - c0) / VEC) * VEC;
    for (int64_t e = c0 + (int64_t)threadIdx.x * VEC; e < v_end; e += (int64_t)kBlock * VEC) {
      float f[VEC];
      unpack<T>(ld16_nt(x + e), f);
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        const float p = fast_exp2(f[i] * kLog2e - lb);
        f[i] = (p - (e + i == t ? 1.0f : 0.0f)) * scale;
      }
      st16_nt(d + e, pack<T>(f));
    }
    tail = v_end;
  }
  for (int64_t e = tail + threadIdx.x; e < c1; e += kBlock) {
    const float p = fast_exp2(to_f32(x[e]) * kLog2e - lb);
    d[e] = from_f32<T>((p - (e == t ? 1.0f : 0.0f)) * scale);
  }
}

#define TRI_DISPATCH_INDEX(kind, TT, ...)                                           \
  do {                                                                              \
    if ((kind) == 1) { typedef int32_t TT; __VA_ARGS__; }                           \
    else if ((kind) == 2) { typedef int64_t TT; __VA_ARGS__; }                      \
    else return fail(TRI_EINVAL, "cross_entropy: bad target kind %d", (int)(kind)); \
  } while (0)

bool rows_vec_ok(const void* p, int64_t V, int dtype) {
  return aligned16(p) && ((V * dtype_size(dtype)) % 16) == 0;
}

}  // namespace
}  // namespace tri

using namespace tri;

extern "C" size_t tritium_cross_entropy_fwd_workspace_size(int64_t n_rows, int64_t vocab, int dtype) {
  (void)dtype;
  if (n_rows <= 0 || vocab <= 0) return 0;
  int chunks;
  int64_t span;
  span_split(n_rows, vocab, chunks, span);
  return chunks > 1 ? (size_t)(n_rows * chunks) * sizeof(float2) : (size_t)n_rows * sizeof(float);
}

extern "C" int tritium_cross_entropy_fwd_ws(const void* logits, const void* target,
                                            int target_kind, float* loss, float* lse, void* work,
                                            size_t work_bytes, int64_t n_rows, int64_t vocab,
                                            int dtype, void* stream) {
  if (n_rows < 0 || vocab <= 0) return fail(TRI_EINVAL, "cross_entropy: bad sizes");
  if (n_rows >= ((int64_t)1 << 31)) return fail(TRI_EINVAL, "cross_entropy: too many rows");
  hipStream_t st = (hipStream_t)stream;
  if (n_rows == 0) return TRI_OK;
  const size_t need = tritium_cross_entropy_fwd_workspace_size(n_rows, vocab, dtype);
  if (work == nullptr || work_bytes < need)
    return fail(TRI_EINVAL, "cross_entropy: workspace of %zu bytes, %zu needed", work_bytes, need);
  if ((reinterpret_cast<uintptr_t>(work) & 7u) != 0)
    return fail(TRI_EINVAL, "cross_entropy: workspace must be 8-byte aligned");
  const int vec_ok = rows_vec_ok(logits, vocab, dtype);
  int chunks;
  int64_t span;
  span_split(n_rows, vocab, chunks, span);
  if (chunks > 1) {
    float2* part = reinterpret_cast<float2*>(work);
    TRI_DISPATCH_INDEX(target_kind, TT,
      TRI_DISPATCH_FLOAT(dtype, T, {
        ce_span_kernel<T><<<(unsigned)(n_rows * chunks), kBlock, 0, st>>>(
            (const T*)logits, part, vocab, span, chunks, vec_ok);
        if (int e = check_launch("cross_entropy_fwd")) return e;
        ce_finish_kernel<T, TT><<<1, kWave, 0, st>>>((const T*)logits, target, part, lse, loss,
                                                   n_rows, vocab, chunks);
      }));
    return check_launch("cross_entropy_finish");
  }
  float* nll = reinterpret_cast<float*>(work);
  TRI_DISPATCH_INDEX(target_kind, TT,
    TRI_DISPATCH_FLOAT(dtype, T, {
      if (vocab >= kWideRow) {
        ce_fwd_kernel<T, TT, kBlock><<<(unsigned)n_rows, kBlock, 0, st>>>(
            (const T*)logits, target, lse, nll, n_rows, vocab, vec_ok);
      } else {
        ce_fwd_kernel<T, TT, kWave><<<(unsigned)cdiv(n_rows, kBlock / kWave), kBlock, 0, st>>>(
            (const T*)logits, target, lse, nll, n_rows, vocab, vec_ok);
      }
    }));
  if (int e = check_launch("cross_entropy_fwd")) return e;
  ce_mean_kernel<<<1, kWave, 0, st>>>(nll, n_rows, loss);
  return check_launch("cross_entropy_mean");
}

extern "C" int tritium_cross_entropy_bwd(const float* grad_out, const void* logits,
                                         const void* target, int target_kind, const float* lse,
                                         void* dlogits, int64_t n_rows, int64_t vocab,
                                         double grad_denominator, int dtype, void* stream) {
  if (n_rows < 0 || vocab <= 0) return fail(TRI_EINVAL, "cross_entropy: bad sizes");
  if (n_rows == 0) return TRI_OK;
  const int64_t chunks = cdiv(vocab, kBwdChunk);
  if (n_rows * chunks > 0x7fffffffLL) return fail(TRI_EINVAL, "cross_entropy: grid too large");
  const int vec_ok = rows_vec_ok(logits, vocab, dtype) && rows_vec_ok(dlogits, vocab, dtype);
  const float inv_den = (float)(1.0 / grad_denominator);
  hipStream_t st = (hipStream_t)stream;
  TRI_DISPATCH_INDEX(target_kind, TT,
    TRI_DISPATCH_FLOAT(dtype, T,
      ce_bwd_kernel<T, TT><<<(unsigned)(n_rows * chunks), kBlock, 0, st>>>(
          grad_out, (const T*)logits, target, lse, (T*)dlogits, vocab, chunks, inv_den, vec_ok)));
  return check_launch("cross_entropy_bwd");
}
