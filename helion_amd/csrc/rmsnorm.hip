// RMSNorm / residual-RMSNorm forward and backward for gfx950.
//
// Reference arithmetic: alkinun/helion tritium/ops/rmsnorm.py:45-51 (forward),
// 72-83 (residual forward), 121-129 (dx), 253 + 279 + 439 (dweight).
//
// Fast path (row length a multiple of one 16-byte vector, all pointers 16-byte
// aligned, row fits in registers): TPR lanes (a whole number of wavefronts)
// own one row; every lane keeps NV 16-byte vectors of the row in registers, so
// x / dy are read from HBM exactly once.  Row sums are wavefront butterflies
// plus one LDS exchange when a row spans several wavefronts.
//
// dweight is deterministic: each block accumulates sum(dy*x*rstd) over its own
// contiguous run of rows in registers (fp64 for fp32 inputs, fp32 otherwise),
// writes one partial row, and a second kernel adds the partial rows in a fixed
// order and casts to the weight dtype.  No atomics anywhere.
//
// Streaming path (anything else): one 256-lane block per row, two passes over
// the row, column-parallel dweight partials.
#include "common.h"
#include "../../include/tritium_hip.h"

namespace tri {
namespace {

// Fast-path backward grid = dweight partial rows (1024 or 2048 measured
// slower, with a longer reduction).
constexpr int kMaxPartialRows = 512;
constexpr int kGenericBlock = 256;
constexpr int kStage1Rows = 128;       // streaming-path rows per dweight partial

template <int TPR>
constexpr int block_of() { return TPR < 256 ? 256 : TPR; }

// dweight accumulates in double for fp32 inputs (a column sum over thousands
// of rows must stay within 1e-5 of the exact sum) and in fp32 for 16-bit
// inputs, whose tolerance is far wider.
template <typename T> struct DwAcc { typedef float type; };
template <> struct DwAcc<float> { typedef double type; };

// Sum a pair of values over the TPR lanes owning one row.  Every lane of the
// block must call this the same number of times (it may hold barriers).
template <int TPR>
__device__ __forceinline__ void row_sum2(float& a, float& b, float2* red) {
  a = wave_sum(a);
  b = wave_sum(b);
  if constexpr (TPR > kWave) {
    constexpr int WPR = TPR / kWave;
    const int wave = threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    __syncthreads();
    if (lane == 0) red[wave] = make_float2(a, b);
    __syncthreads();
    const int first = (wave / WPR) * WPR;
    float sa = 0.f, sb = 0.f;
#pragma unroll
    for (int i = 0; i < WPR; ++i) {
      float2 t = red[first + i];
      sa += t.x;
      sb += t.y;
    }
    a = sa;
    b = sb;
  }
}

// ---------------------------------------------------------------- forward --
// Persistent rows: row group g of block b takes rows b * RPB + g, then
// advances by gridDim.x * RPB.  The weight is read once per lane; the next
// row's raw vectors are loaded while the current row is reduced; x / residual
// are read and y / residual_out written with the nontemporal hint.
template <typename T, int TPR, int NV>
__global__ void __launch_bounds__(block_of<TPR>())
rmsnorm_fwd_kernel(const T* __restrict__ x, const T* __restrict__ res,
                   const T* __restrict__ w, T* __restrict__ y, T* __restrict__ z,
                   float* __restrict__ rstd, int64_t n_rows, int hidden, float eps) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int RPB = block_of<TPR>() / TPR;
  __shared__ float2 red[block_of<TPR>() / kWave];
  const int g = threadIdx.x / TPR;
  const int lt = threadIdx.x % TPR;
  const int nvec = hidden / VEC;
  const int64_t first = (int64_t)blockIdx.x * RPB;
  const int64_t stride = (int64_t)gridDim.x * RPB;
  const int64_t iters = first < n_rows ? cdiv(n_rows - first, stride) : 0;  // block-uniform

  u32x4 wr[NV], xr[NV], rr[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int vi = lt + j * TPR;
    wr[j] = vi < nvec ? ld16(w + (int64_t)vi * VEC) : u32x4{0u, 0u, 0u, 0u};
    xr[j] = rr[j] = u32x4{0u, 0u, 0u, 0u};
  }
  auto fetch = [&](int64_t row) {
    if (row >= n_rows) return;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int vi = lt + j * TPR;
      if (vi < nvec) {
        xr[j] = ld16_nt(x + row * hidden + (int64_t)vi * VEC);
        if (res != nullptr) rr[j] = ld16_nt(res + row * hidden + (int64_t)vi * VEC);
      }
    }
  };
  fetch(first + g);
  for (int64_t it = 0; it < iters; ++it) {
    const int64_t row = first + g + it * stride;
    const bool active = row < n_rows;
    float v[NV][VEC];
    float ss = 0.f, unused = 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      unpack<T>(xr[j], v[j]);
      if (res != nullptr) {
        float r[VEC];
        unpack<T>(rr[j], r);
#pragma unroll
        for (int i = 0; i < VEC; ++i) v[j][i] += r[i];
      }
#pragma unroll
      for (int i = 0; i < VEC; ++i) ss += v[j][i] * v[j][i];
    }
    fetch(row + stride);
    row_sum2<TPR>(ss, unused, red);
    const float rs = 1.0f / sqrtf(ss / (float)hidden + eps);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int vi = lt + j * TPR;
      if (active && vi < nvec) {
        float wv[VEC], o[VEC];
        unpack<T>(wr[j], wv);
#pragma unroll
        for (int i = 0; i < VEC; ++i) o[i] = v[j][i] * rs * wv[i];
        st16_nt(y + row * hidden + (int64_t)vi * VEC, pack<T>(o));
        if (z != nullptr) st16_nt(z + row * hidden + (int64_t)vi * VEC, pack<T>(v[j]));
      }
    }
    if (active && lt == 0) rstd[row] = rs;
  }
}

// --------------------------------------------------------------- backward --
// dx for the rows of this block (persistent, as the forward) and, when
// dw_partial != null, one dweight partial row per block: the row groups
// accumulate sum(dy * x * rstd) over their rows in registers and are added
// through LDS in a fixed order.  Raw x / dy of the next row stream in while
// the current row is reduced.
template <typename T, int TPR, int NV>
__global__ void __launch_bounds__(block_of<TPR>())
rmsnorm_bwd_kernel(const T* __restrict__ dy, const T* __restrict__ x,
                   const T* __restrict__ w, const float* __restrict__ rstd_in,
                   const T* __restrict__ dres, T* __restrict__ dx,
                   typename DwAcc<T>::type* __restrict__ dw_partial, int64_t n_rows, int hidden,
                   float eps) {
  typedef typename DwAcc<T>::type A;
  constexpr int VEC = 16 / sizeof(T);
  constexpr int RPB = block_of<TPR>() / TPR;
  constexpr int SLOT = TPR * NV * VEC;
  __shared__ float2 red[block_of<TPR>() / kWave];
  __shared__ A dw_lds[(RPB > 1 ? RPB - 1 : 1) * SLOT];
  const int g = threadIdx.x / TPR;
  const int lt = threadIdx.x % TPR;
  const int nvec = hidden / VEC;
  const float inv_h = 1.0f / (float)hidden;
  const int64_t first = (int64_t)blockIdx.x * RPB;
  const int64_t stride = (int64_t)gridDim.x * RPB;
  const int64_t iters = first < n_rows ? cdiv(n_rows - first, stride) : 0;  // block-uniform

  u32x4 wr[NV], xr[NV], gr[NV], xn[NV], gn[NV];
  A acc[NV][VEC];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int vi = lt + j * TPR;
    wr[j] = vi < nvec ? ld16(w + (int64_t)vi * VEC) : u32x4{0u, 0u, 0u, 0u};
    xr[j] = gr[j] = xn[j] = gn[j] = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < VEC; ++i) acc[j][i] = 0;
  }
  float rs_next = 0.f;
  auto fetch = [&](int64_t row, u32x4 (&xb)[NV], u32x4 (&gb)[NV], float& rsb) {
    if (row >= n_rows) return;
    // all of a lane's x vectors, then its dy vectors (config 2: 69.8 -> 68.7
    // us against the two of each vector together)
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int vi = lt + j * TPR;
      if (vi < nvec) xb[j] = ld16_nt(x + row * hidden + (int64_t)vi * VEC);
    }
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int vi = lt + j * TPR;
      if (vi < nvec) gb[j] = ld16_nt(dy + row * hidden + (int64_t)vi * VEC);
    }
    if (rstd_in != nullptr) rsb = rstd_in[row];
  };
  fetch(first + g, xr, gr, rs_next);
  for (int64_t it = 0; it < iters; ++it) {
    const int64_t row = first + g + it * stride;
    const bool active = row < n_rows;
    float rs = rs_next;
    float ss = 0.f, c = 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      float xv[VEC], gv[VEC], wv[VEC];
      unpack<T>(xr[j], xv);
      unpack<T>(gr[j], gv);
      unpack<T>(wr[j], wv);
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        ss += xv[i] * xv[i];
        c += gv[i] * wv[i] * xv[i];
      }
    }
    fetch(row + stride, xn, gn, rs_next);
    u32x4 rr[NV];
    if (dres != nullptr && active) {
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int vi = lt + j * TPR;
        if (vi < nvec) rr[j] = ld16_nt(dres + row * hidden + (int64_t)vi * VEC);
      }
    }
    row_sum2<TPR>(ss, c, red);
    if (rstd_in == nullptr) rs = 1.0f / sqrtf(ss * inv_h + eps);
    const float k3 = rs * rs * rs * inv_h;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int vi = lt + j * TPR;
      if (active && vi < nvec) {
        float xv[VEC], gv[VEC], wv[VEC], o[VEC];
        unpack<T>(xr[j], xv);
        unpack<T>(gr[j], gv);
        unpack<T>(wr[j], wv);
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          o[i] = rs * (gv[i] * wv[i]) - k3 * xv[i] * c;
          acc[j][i] += (A)gv[i] * (A)xv[i] * (A)rs;
        }
        if (dres != nullptr) {
          float r[VEC];
          unpack<T>(rr[j], r);
#pragma unroll
          for (int i = 0; i < VEC; ++i) o[i] += r[i];
        }
        st16_nt(dx + row * hidden + (int64_t)vi * VEC, pack<T>(o));
      }
    }
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      xr[j] = xn[j];
      gr[j] = gn[j];
    }
  }

  if (dw_partial == nullptr) return;
  if constexpr (RPB > 1) {
    if (g > 0) {
#pragma unroll
      for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int i = 0; i < VEC; ++i)
          dw_lds[(g - 1) * SLOT + (j * TPR + lt) * VEC + i] = acc[j][i];
    }
    __syncthreads();
    if (g > 0) return;
#pragma unroll
    for (int s = 0; s < RPB - 1; ++s)
#pragma unroll
      for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int i = 0; i < VEC; ++i) acc[j][i] += dw_lds[s * SLOT + (j * TPR + lt) * VEC + i];
  }
  A* out = dw_partial + (int64_t)blockIdx.x * hidden;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int vi = lt + j * TPR;
    if (vi < nvec) {
      *reinterpret_cast<Pack<A, VEC>*>(out + (int64_t)vi * VEC) =
          *reinterpret_cast<const Pack<A, VEC>*>(acc[j]);
    }
  }
}

// Column sums of partial rows, in two levels with a fixed order: level 1
// (grid = column blocks x row groups) adds kDwGroup consecutive partial rows
// per column; level 2 adds the group sums and casts to the weight dtype.
constexpr int kDwGroup = 8;

// The loads of a group are independent (issued together); the adds run in
// row order, so the result does not depend on timing.
template <typename A>
__global__ void __launch_bounds__(256)
dw_sum_groups_kernel(const A* __restrict__ partial, int64_t n_part, int hidden,
                     A* __restrict__ sums) {
  const int col = blockIdx.x * 256 + threadIdx.x;
  if (col >= hidden) return;
  const int64_t p0 = (int64_t)blockIdx.y * kDwGroup;
  A v[kDwGroup];
#pragma unroll
  for (int i = 0; i < kDwGroup; ++i) v[i] = p0 + i < n_part ? partial[(p0 + i) * hidden + col] : 0;
  A s = 0;
#pragma unroll
  for (int i = 0; i < kDwGroup; ++i) s += v[i];
  sums[(int64_t)blockIdx.y * hidden + col] = s;
}

template <typename T, typename A>
__global__ void __launch_bounds__(256)
dw_finish_kernel(const A* __restrict__ sums, int64_t n_groups, int hidden, T* __restrict__ dw) {
  const int col = blockIdx.x * 256 + threadIdx.x;
  if (col >= hidden) return;
  A s = 0;
  int64_t p = 0;
  for (; p + 8 <= n_groups; p += 8) {
    A v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = sums[(p + i) * hidden + col];
#pragma unroll
    for (int i = 0; i < 8; ++i) s += v[i];
  }
  for (; p < n_groups; ++p) s += sums[p * hidden + col];
  dw[col] = from_f32<T>((float)s);
}

// Column sums of the partial rows in one launch (hidden a multiple of the
// 16-byte vector): block b owns kDwCg 16-byte column groups (128 bytes of
// every partial row, so no two blocks fetch one cache line); thread t takes
// the column group t % kDwCg of rows s, s + kDwSlices, s + 2 kDwSlices, ...
// (s = t / kDwCg, rows added in increasing order, eight loads in flight),
// and the kDwSlices slice sums of each column are added through LDS in two
// fixed-order levels (a quarter of the slices each, then the 4 group sums).
// The order depends on n_part and hidden only, so dweight is deterministic.
// Replaces two launches (group sums, then their sum) whose launch and tail
// time was most of the reduction's 9 us at 512 partial rows.
constexpr int kDwCg = 8;                  // 16-byte column groups per block
constexpr int kDwSlices = 256 / kDwCg;    // row slices (32)

template <typename T, typename A>
__global__ void __launch_bounds__(256)
dw_reduce_kernel(const A* __restrict__ partial, int64_t n_part, int hidden, T* __restrict__ dw) {
  constexpr int VA = 16 / (int)sizeof(A);
  constexpr int COLS = kDwCg * VA;
  constexpr int U = 8;
  __shared__ A red[kDwSlices][COLS];
  __shared__ A red2[4][COLS];
  const int cg = threadIdx.x % kDwCg, s = threadIdx.x / kDwCg;
  const int c0 = blockIdx.x * COLS + cg * VA;
  A acc[VA];
#pragma unroll
  for (int i = 0; i < VA; ++i) acc[i] = 0;
  if (c0 < hidden) {
    int64_t p = s;
    for (; p + (U - 1) * kDwSlices < n_part; p += U * kDwSlices) {
      Pack<A, VA> v[U];
#pragma unroll
      for (int u = 0; u < U; ++u)
        v[u] = *reinterpret_cast<const Pack<A, VA>*>(partial + (p + u * kDwSlices) * hidden + c0);
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int i = 0; i < VA; ++i) acc[i] += v[u].v[i];
    }
    for (; p < n_part; p += kDwSlices) {
      const Pack<A, VA> v = *reinterpret_cast<const Pack<A, VA>*>(partial + p * hidden + c0);
#pragma unroll
      for (int i = 0; i < VA; ++i) acc[i] += v.v[i];
    }
  }
#pragma unroll
  for (int i = 0; i < VA; ++i) red[s][cg * VA + i] = acc[i];
  __syncthreads();
  if (threadIdx.x < 4 * COLS) {
    const int col = threadIdx.x % COLS, q = threadIdx.x / COLS;
    A t = 0;
#pragma unroll
    for (int k = 0; k < kDwSlices / 4; ++k) t += red[q * (kDwSlices / 4) + k][col];
    red2[q][col] = t;
  }
  __syncthreads();
  if (threadIdx.x < COLS) {
    const int col = blockIdx.x * COLS + threadIdx.x;
    const A t = (red2[0][threadIdx.x] + red2[1][threadIdx.x]) +
                (red2[2][threadIdx.x] + red2[3][threadIdx.x]);
    if (col < hidden) dw[col] = from_f32<T>((float)t);
  }
}

// Column sum of n_part partial rows into dw: one launch when hidden is a
// multiple of the 16-byte vector, else two levels through `sums`
// (cdiv(n_part, kDwGroup) rows).
template <typename T, typename A>
int dw_reduce(const A* partial, int64_t n_part, int hidden, A* sums, T* dw, hipStream_t stream) {
  constexpr int VA = 16 / (int)sizeof(A);
  if (hidden % VA == 0 && aligned16(partial)) {
    dw_reduce_kernel<T, A><<<(unsigned)cdiv(hidden, kDwCg * VA), 256, 0, stream>>>(
        partial, n_part, hidden, dw);
    return check_launch("rmsnorm dweight reduce");
  }
  const int64_t n_groups = cdiv(n_part, kDwGroup);
  dw_sum_groups_kernel<A><<<dim3((unsigned)cdiv(hidden, 256), (unsigned)n_groups), 256, 0,
                            stream>>>(partial, n_part, hidden, sums);
  if (int e = check_launch("rmsnorm dweight reduce (groups)")) return e;
  dw_finish_kernel<T, A><<<(unsigned)cdiv(hidden, 256), 256, 0, stream>>>(sums, n_groups, hidden,
                                                                          dw);
  return check_launch("rmsnorm dweight reduce");
}

// -------------------------------------------------------- streaming path --
template <typename T>
__global__ void __launch_bounds__(kGenericBlock)
rmsnorm_fwd_generic_kernel(const T* __restrict__ x, const T* __restrict__ res,
                           const T* __restrict__ w, T* __restrict__ y, T* __restrict__ z,
                           float* __restrict__ rstd, int hidden, float eps) {
  __shared__ float2 red[kGenericBlock / kWave];
  const int64_t base = (int64_t)blockIdx.x * hidden;
  float ss = 0.f, unused = 0.f;
  for (int c = threadIdx.x; c < hidden; c += kGenericBlock) {
    float v = to_f32(x[base + c]);
    if (res != nullptr) v += to_f32(res[base + c]);
    ss += v * v;
  }
  row_sum2<kGenericBlock>(ss, unused, red);
  const float rs = 1.0f / sqrtf(ss / (float)hidden + eps);
  for (int c = threadIdx.x; c < hidden; c += kGenericBlock) {
    float v = to_f32(x[base + c]);
    if (res != nullptr) v += to_f32(res[base + c]);
    y[base + c] = from_f32<T>(v * rs * to_f32(w[c]));
    if (z != nullptr) z[base + c] = from_f32<T>(v);
  }
  if (threadIdx.x == 0) rstd[blockIdx.x] = rs;
}

template <typename T>
__global__ void __launch_bounds__(kGenericBlock)
rmsnorm_bwd_generic_kernel(const T* __restrict__ dy, const T* __restrict__ x,
                           const T* __restrict__ w, const float* __restrict__ rstd_in,
                           const T* __restrict__ dres, T* __restrict__ dx,
                           float* __restrict__ rstd_used, int hidden, float eps) {
  __shared__ float2 red[kGenericBlock / kWave];
  const int64_t row = blockIdx.x;
  const int64_t base = row * hidden;
  float ss = 0.f, c = 0.f;
  for (int i = threadIdx.x; i < hidden; i += kGenericBlock) {
    const float xv = to_f32(x[base + i]);
    ss += xv * xv;
    c += to_f32(dy[base + i]) * to_f32(w[i]) * xv;
  }
  row_sum2<kGenericBlock>(ss, c, red);
  const float inv_h = 1.0f / (float)hidden;
  const float rs = rstd_in != nullptr ? rstd_in[row] : 1.0f / sqrtf(ss * inv_h + eps);
  const float k3 = rs * rs * rs * inv_h;
  for (int i = threadIdx.x; i < hidden; i += kGenericBlock) {
    const float xv = to_f32(x[base + i]);
    float o = rs * (to_f32(dy[base + i]) * to_f32(w[i])) - k3 * xv * c;
    if (dres != nullptr) o += to_f32(dres[base + i]);
    dx[base + i] = from_f32<T>(o);
  }
  if (threadIdx.x == 0) rstd_used[row] = rs;
}

// partial[rb][col] = sum over rows of block rb of dy*x*rstd (column parallel).
template <typename T>
__global__ void __launch_bounds__(kGenericBlock)
dw_stage1_kernel(const T* __restrict__ dy, const T* __restrict__ x,
                 const float* __restrict__ rstd, typename DwAcc<T>::type* __restrict__ partial,
                 int64_t n_rows, int hidden) {
  typedef typename DwAcc<T>::type A;
  const int col = blockIdx.y * kGenericBlock + threadIdx.x;
  if (col >= hidden) return;
  const int64_t r0 = (int64_t)blockIdx.x * kStage1Rows;
  const int64_t r1 = min(r0 + kStage1Rows, n_rows);
  A s = 0;
  for (int64_t r = r0; r < r1; ++r) {
    s += (A)to_f32(dy[r * hidden + col]) * (A)to_f32(x[r * hidden + col]) * (A)rstd[r];
  }
  partial[(int64_t)blockIdx.x * hidden + col] = s;
}

// ------------------------------------------------------------ host side --
struct FastCfg {
  int tpr = 0;  // 0: no register-resident config fits
  int nv = 0;
};

// Smallest row width (in lanes) whose NV <= max_nv vectors per lane cover the row.
FastCfg pick_fast(int64_t hidden, int vec, int max_nv) {
  FastCfg cfg;
  if (hidden % vec != 0) return cfg;
  const int64_t nvec = hidden / vec;
  for (int tpr = 64; tpr <= 1024; tpr *= 2) {
    const int64_t need = cdiv(nvec, tpr);
    if (need <= max_nv) {
      int nv = 1;
      while (nv < need) nv *= 2;
      cfg.tpr = tpr;
      cfg.nv = nv;
      return cfg;
    }
  }
  return cfg;
}

#define TRI_FAST_SWITCH(cfg, LAUNCH)                                         \
  switch (cfg.tpr * 100 + cfg.nv) {                                          \
    case 6401: LAUNCH(64, 1); break;    case 6402: LAUNCH(64, 2); break;     \
    case 6404: LAUNCH(64, 4); break;    case 6408: LAUNCH(64, 8); break;     \
    case 12801: LAUNCH(128, 1); break;  case 12802: LAUNCH(128, 2); break;   \
    case 12804: LAUNCH(128, 4); break;  case 12808: LAUNCH(128, 8); break;   \
    case 25601: LAUNCH(256, 1); break;  case 25602: LAUNCH(256, 2); break;   \
    case 25604: LAUNCH(256, 4); break;  case 25608: LAUNCH(256, 8); break;   \
    case 51201: LAUNCH(512, 1); break;  case 51202: LAUNCH(512, 2); break;   \
    case 51204: LAUNCH(512, 4); break;  case 51208: LAUNCH(512, 8); break;   \
    case 102401: LAUNCH(1024, 1); break; case 102402: LAUNCH(1024, 2); break; \
    case 102404: LAUNCH(1024, 4); break; case 102408: LAUNCH(1024, 8); break; \
    default: return fail(TRI_EINVAL, "rmsnorm: no kernel for tpr=%d nv=%d", cfg.tpr, cfg.nv); \
  }

// Forward: one vector per lane (rows of up to 1024 vectors on the fast
// path), a persistent grid of 8192 workgroups (2 rows each at config 2; 1024
// to 4096 workgroups or two vectors per lane measured slower); backward: up
// to 4 vectors per lane.
constexpr int kFwdMaxNV = 1;
constexpr int64_t kFwdBlocks = 8192;
constexpr int kBwdMaxNV = 4;

template <typename T>
int fwd_impl(const void* x, const void* res, const void* w, void* y, void* z, float* rstd,
             int64_t n_rows, int64_t hidden, float eps, hipStream_t stream) {
  constexpr int VEC = 16 / sizeof(T);
  const bool aligned = aligned16(x) && aligned16(w) && aligned16(y) &&
                       (res == nullptr || aligned16(res)) && (z == nullptr || aligned16(z));
  FastCfg cfg = aligned ? pick_fast(hidden, VEC, kFwdMaxNV) : FastCfg{};
  if (cfg.tpr != 0) {
    const int rpb = (cfg.tpr < 256 ? 256 : cfg.tpr) / cfg.tpr;
    const dim3 grid((unsigned)std::min<int64_t>(cdiv(n_rows, rpb), kFwdBlocks));
#define LAUNCH(TPR, NV)                                                                  \
  rmsnorm_fwd_kernel<T, TPR, NV><<<grid, block_of<TPR>(), 0, stream>>>(                  \
      (const T*)x, (const T*)res, (const T*)w, (T*)y, (T*)z, rstd, n_rows, (int)hidden, eps)
    TRI_FAST_SWITCH(cfg, LAUNCH)
#undef LAUNCH
  } else {
    rmsnorm_fwd_generic_kernel<T><<<(unsigned)n_rows, kGenericBlock, 0, stream>>>(
        (const T*)x, (const T*)res, (const T*)w, (T*)y, (T*)z, rstd, (int)hidden, eps);
  }
  return check_launch("rmsnorm forward");
}

int64_t fast_bwd_blocks(int64_t n_rows, int rpb) {
  return std::min<int64_t>(cdiv(n_rows, rpb), kMaxPartialRows);
}

// Workspace of the dweight reduction: partial rows, then their group sums.
template <typename A>
int64_t dw_ws_bytes(int64_t n_part, int64_t hidden) {
  return (n_part + cdiv(n_part, kDwGroup)) * hidden * (int64_t)sizeof(A);
}

template <typename T>
int bwd_impl(const void* dy, const void* x, const void* w, const float* rstd, const void* dres,
             void* dx, void* dw, void* ws, size_t ws_bytes, int64_t n_rows, int64_t hidden,
             float eps, hipStream_t stream) {
  typedef typename DwAcc<T>::type A;
  constexpr int VEC = 16 / sizeof(T);
  const bool aligned = aligned16(dy) && aligned16(x) && aligned16(w) && aligned16(dx) &&
                       (dres == nullptr || aligned16(dres)) && aligned16(ws);
  FastCfg cfg = aligned ? pick_fast(hidden, VEC, kBwdMaxNV) : FastCfg{};
  if (cfg.tpr != 0) {
    const int rpb = (cfg.tpr < 256 ? 256 : cfg.tpr) / cfg.tpr;
    const int64_t n_part = fast_bwd_blocks(n_rows, rpb);
    A* partial = dw != nullptr ? (A*)ws : nullptr;
    if (dw != nullptr && (size_t)dw_ws_bytes<A>(n_part, hidden) > ws_bytes)
      return fail(TRI_EINVAL, "rmsnorm backward: workspace too small");
#define LAUNCH(TPR, NV)                                                                   \
  rmsnorm_bwd_kernel<T, TPR, NV><<<(unsigned)n_part, block_of<TPR>(), 0, stream>>>(        \
      (const T*)dy, (const T*)x, (const T*)w, rstd, (const T*)dres, (T*)dx, partial, n_rows, \
      (int)hidden, eps)
    TRI_FAST_SWITCH(cfg, LAUNCH)
#undef LAUNCH
    if (int e = check_launch("rmsnorm backward")) return e;
    if (dw != nullptr)
      return dw_reduce<T, A>(partial, n_part, (int)hidden, partial + n_part * hidden, (T*)dw,
                             stream);
    return TRI_OK;
  }
  // streaming path: workspace = rstd_used[n_rows] then partial[row_blocks][hidden]
  const int64_t rstd_bytes = cdiv(n_rows * 4, 256) * 256;
  const int64_t n_rb = cdiv(n_rows, kStage1Rows);
  if ((size_t)(rstd_bytes + dw_ws_bytes<A>(n_rb, hidden)) > ws_bytes)
    return fail(TRI_EINVAL, "rmsnorm backward: workspace too small");
  float* rstd_used = (float*)ws;
  A* partial = (A*)((char*)ws + rstd_bytes);
  rmsnorm_bwd_generic_kernel<T><<<(unsigned)n_rows, kGenericBlock, 0, stream>>>(
      (const T*)dy, (const T*)x, (const T*)w, rstd, (const T*)dres, (T*)dx, rstd_used,
      (int)hidden, eps);
  if (int e = check_launch("rmsnorm backward (streaming)")) return e;
  if (dw == nullptr) return TRI_OK;
  dw_stage1_kernel<T><<<dim3((unsigned)n_rb, (unsigned)cdiv(hidden, kGenericBlock)),
                        kGenericBlock, 0, stream>>>((const T*)dy, (const T*)x, rstd_used,
                                                    partial, n_rows, (int)hidden);
  if (int e = check_launch("rmsnorm dweight stage1")) return e;
  return dw_reduce<T, A>(partial, n_rb, (int)hidden, partial + n_rb * hidden, (T*)dw, stream);
}

int check_shape(int64_t n_rows, int64_t hidden) {
  if (n_rows < 0 || hidden <= 0 || hidden > (int64_t)1 << 30 || n_rows > ((int64_t)1 << 31) - 1)
    return fail(TRI_EINVAL, "rmsnorm: unsupported shape n_rows=%lld hidden=%lld",
                (long long)n_rows, (long long)hidden);
  return TRI_OK;
}

}  // namespace
}  // namespace tri

using namespace tri;

extern "C" int tritium_rmsnorm_fwd(const void* x, const void* residual, const void* weight,
                                   void* y, void* residual_out, float* rstd, int64_t n_rows,
                                   int64_t hidden, float eps, int dtype, void* stream) {
  if (int e = check_shape(n_rows, hidden)) return e;
  if ((residual == nullptr) != (residual_out == nullptr))
    return fail(TRI_EINVAL, "rmsnorm: residual and residual_out must be given together");
  if (n_rows == 0) return TRI_OK;
  TRI_DISPATCH_FLOAT(dtype, T,
                     return fwd_impl<T>(x, residual, weight, y, residual_out, rstd, n_rows,
                                        hidden, eps, (hipStream_t)stream));
  return TRI_OK;
}

extern "C" size_t tritium_rmsnorm_bwd_workspace_size(int64_t n_rows, int64_t hidden) {
  if (n_rows <= 0 || hidden <= 0) return 0;
  const int64_t fast = dw_ws_bytes<double>(kMaxPartialRows, hidden);
  const int64_t streaming =
      cdiv(n_rows * 4, 256) * 256 + dw_ws_bytes<double>(cdiv(n_rows, kStage1Rows), hidden);
  return (size_t)std::max(fast, streaming);
}

extern "C" int tritium_rmsnorm_bwd(const void* dy, const void* x, const void* weight,
                                   const float* rstd, const void* dresidual, void* dx,
                                   void* dweight, void* workspace, size_t workspace_bytes,
                                   int64_t n_rows, int64_t hidden, float eps, int dtype,
                                   void* stream) {
  if (int e = check_shape(n_rows, hidden)) return e;
  if (n_rows == 0) return TRI_OK;
  TRI_DISPATCH_FLOAT(dtype, T,
                     return bwd_impl<T>(dy, x, weight, rstd, dresidual, dx, dweight, workspace,
                                        workspace_bytes, n_rows, hidden, eps,
                                        (hipStream_t)stream));
  return TRI_OK;
}
