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

constexpr int kMaxPartialRows = 512;   // fast-path dweight partial rows
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
  const int64_t row = (int64_t)blockIdx.x * RPB + g;
  const bool active = row < n_rows;
  const int nvec = hidden / VEC;
  const int64_t base = row * (int64_t)hidden;

  float v[NV][VEC];
  float ss = 0.f, unused = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int vi = lt + j * TPR;
    if (active && vi < nvec) {
      load_f32<T, VEC>(x + base + (int64_t)vi * VEC, v[j]);
      if (res != nullptr) {
        float r[VEC];
        load_f32<T, VEC>(res + base + (int64_t)vi * VEC, r);
#pragma unroll
        for (int i = 0; i < VEC; ++i) v[j][i] += r[i];
      }
#pragma unroll
      for (int i = 0; i < VEC; ++i) ss += v[j][i] * v[j][i];
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) v[j][i] = 0.f;
    }
  }
  row_sum2<TPR>(ss, unused, red);
  const float rs = 1.0f / sqrtf(ss / (float)hidden + eps);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int vi = lt + j * TPR;
    if (active && vi < nvec) {
      float wv[VEC], o[VEC];
      load_f32<T, VEC>(w + (int64_t)vi * VEC, wv);
#pragma unroll
      for (int i = 0; i < VEC; ++i) o[i] = v[j][i] * rs * wv[i];
      store_f32<T, VEC>(y + base + (int64_t)vi * VEC, o);
      if (z != nullptr) store_f32<T, VEC>(z + base + (int64_t)vi * VEC, v[j]);
    }
  }
  if (active && lt == 0) rstd[row] = rs;
}

// --------------------------------------------------------------- backward --
// dx for rows [blockIdx.x*rows_per_block, ...) and, when dw_partial != null,
// one dweight partial row per block.
template <typename T, int TPR, int NV>
__global__ void __launch_bounds__(block_of<TPR>())
rmsnorm_bwd_kernel(const T* __restrict__ dy, const T* __restrict__ x,
                   const T* __restrict__ w, const float* __restrict__ rstd_in,
                   const T* __restrict__ dres, T* __restrict__ dx,
                   typename DwAcc<T>::type* __restrict__ dw_partial, int64_t n_rows, int hidden,
                   float eps, int64_t rows_per_block) {
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

  float wv[NV][VEC];
  A acc[NV][VEC];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int vi = lt + j * TPR;
    if (vi < nvec) {
      load_f32<T, VEC>(w + (int64_t)vi * VEC, wv[j]);
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) wv[j][i] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < VEC; ++i) acc[j][i] = 0;
  }

  const int64_t row0 = (int64_t)blockIdx.x * rows_per_block;
  const int64_t row_end = min(row0 + rows_per_block, n_rows);
  const int64_t iters = cdiv(rows_per_block, RPB);
  for (int64_t it = 0; it < iters; ++it) {
    const int64_t row = row0 + it * RPB + g;
    const bool active = row < row_end;
    const int64_t base = row * (int64_t)hidden;
    float xv[NV][VEC], gv[NV][VEC];
    float ss = 0.f, c = 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int vi = lt + j * TPR;
      if (active && vi < nvec) {
        load_f32<T, VEC>(x + base + (int64_t)vi * VEC, xv[j]);
        load_f32<T, VEC>(dy + base + (int64_t)vi * VEC, gv[j]);
      } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) xv[j][i] = gv[j][i] = 0.f;
      }
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        ss += xv[j][i] * xv[j][i];
        c += gv[j][i] * wv[j][i] * xv[j][i];
      }
    }
    row_sum2<TPR>(ss, c, red);
    float rs;
    if (rstd_in != nullptr) {
      rs = active ? rstd_in[row] : 0.f;
    } else {
      rs = 1.0f / sqrtf(ss * inv_h + eps);
    }
    const float k3 = rs * rs * rs * inv_h;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int vi = lt + j * TPR;
      if (active && vi < nvec) {
        float o[VEC];
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          o[i] = rs * (gv[j][i] * wv[j][i]) - k3 * xv[j][i] * c;
          acc[j][i] += (A)gv[j][i] * (A)xv[j][i] * (A)rs;
        }
        if (dres != nullptr) {
          float r[VEC];
          load_f32<T, VEC>(dres + base + (int64_t)vi * VEC, r);
#pragma unroll
          for (int i = 0; i < VEC; ++i) o[i] += r[i];
        }
        store_f32<T, VEC>(dx + base + (int64_t)vi * VEC, o);
      }
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

// Sum `n_part` fp32 partial rows into dweight (cast to the weight dtype).
// Block: 64 columns x 4 wavefronts; wavefront k adds rows k, k+4, ... and the
// four column sums are then added in a fixed order.
template <typename T, typename A>
__global__ void __launch_bounds__(256)
dw_reduce_kernel(const A* __restrict__ partial, int64_t n_part, int hidden,
                 T* __restrict__ dw) {
  __shared__ A red[4][kWave];
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int col = blockIdx.x * kWave + lane;
  A s = 0;
  if (col < hidden) {
    for (int64_t p = wave; p < n_part; p += 4) s += partial[p * hidden + col];
  }
  red[wave][lane] = s;
  __syncthreads();
  if (wave == 0 && col < hidden) {
    dw[col] = from_f32<T>((float)(((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane]));
  }
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

constexpr int kFwdMaxNV = 8;
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
    const dim3 grid((unsigned)cdiv(n_rows, rpb));
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
    const int64_t blocks = fast_bwd_blocks(n_rows, rpb);
    const int64_t rows_per_block = cdiv(n_rows, blocks);
    const int64_t n_part = cdiv(n_rows, rows_per_block);
    A* partial = dw != nullptr ? (A*)ws : nullptr;
    if (dw != nullptr && (size_t)(n_part * hidden * sizeof(A)) > ws_bytes)
      return fail(TRI_EINVAL, "rmsnorm backward: workspace too small");
#define LAUNCH(TPR, NV)                                                                   \
  rmsnorm_bwd_kernel<T, TPR, NV><<<(unsigned)n_part, block_of<TPR>(), 0, stream>>>(        \
      (const T*)dy, (const T*)x, (const T*)w, rstd, (const T*)dres, (T*)dx, partial, n_rows, \
      (int)hidden, eps, rows_per_block)
    TRI_FAST_SWITCH(cfg, LAUNCH)
#undef LAUNCH
    if (int e = check_launch("rmsnorm backward")) return e;
    if (dw != nullptr) {
      dw_reduce_kernel<T, A><<<(unsigned)cdiv(hidden, kWave), 256, 0, stream>>>(
          partial, n_part, (int)hidden, (T*)dw);
      return check_launch("rmsnorm dweight reduce");
    }
    return TRI_OK;
  }
  // streaming path: workspace = rstd_used[n_rows] then partial[row_blocks][hidden]
  const int64_t rstd_bytes = cdiv(n_rows * 4, 256) * 256;
  const int64_t n_rb = cdiv(n_rows, kStage1Rows);
  if ((size_t)(rstd_bytes + n_rb * hidden * sizeof(A)) > ws_bytes)
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
  dw_reduce_kernel<T, A><<<(unsigned)cdiv(hidden, kWave), 256, 0, stream>>>(partial, n_rb,
                                                                         (int)hidden, (T*)dw);
  return check_launch("rmsnorm dweight reduce");
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
  const int64_t fast = kMaxPartialRows * hidden * 8;
  const int64_t streaming = cdiv(n_rows * 4, 256) * 256 + cdiv(n_rows, kStage1Rows) * hidden * 8;
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
