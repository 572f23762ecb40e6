// SwiGLU forward and backward for gfx950.
//
// Reference arithmetic: alkinun/helion tritium/ops/swiglu.py:32-35 (forward)
// and 51-58 (backward), all in fp32 with the result stored in the input dtype.
//
// Pure streaming kernels: each lane moves U 16-byte vectors per operand, the
// U loads of a lane are issued before any math so a wavefront keeps
// U * (#operands) * 1 KiB in flight; a block covers one contiguous
// kBlock * U * VEC element span, so every access is fully coalesced.  Every
// operand is touched once: loads and stores carry the nontemporal hint.
#include "common.h"
#include "../../include/tritium_hip.h"

#include <initializer_list>

namespace tri {
namespace {

// One wavefront per workgroup, one vector per lane per operand: config-2
// fwd+bwd 463-464 -> 448-449 us on one box with two vectors per lane (64
// lanes with four vectors: 456.5; 128 lanes: 465-466), then 447-449 ->
// 444-445 us with one (another box, alternating runs).
constexpr int kBlock = 64;
constexpr int kUnroll = 1;
// A lane issues its loads operand by operand (all U vectors of x, then of
// gate, ...) and its stores likewise, rather than the operands of one vector
// together (config 2 fwd+bwd 473-475 -> 471 us with 256-lane workgroups).

__device__ __forceinline__ float sigmoid_f32(float x) { return 1.0f / (1.0f + __expf(-x)); }

template <typename T, int VEC, int U>
__global__ void __launch_bounds__(kBlock)
swiglu_fwd_kernel(const T* __restrict__ x, const T* __restrict__ g, T* __restrict__ out,
                  int64_t n) {
  const int64_t nvec = n / VEC;
  const int64_t first = (int64_t)blockIdx.x * kBlock * U + threadIdx.x;
  float xv[U][VEC], gv[U][VEC];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t iv = first + (int64_t)u * kBlock;
    if (iv < nvec) load_stream<T, VEC>(x + iv * VEC, xv[u]);
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t iv = first + (int64_t)u * kBlock;
    if (iv < nvec) load_stream<T, VEC>(g + iv * VEC, gv[u]);
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t iv = first + (int64_t)u * kBlock;
    if (iv < nvec) {
      float o[VEC];
#pragma unroll
      for (int i = 0; i < VEC; ++i) o[i] = xv[u][i] * sigmoid_f32(xv[u][i]) * gv[u][i];
      store_stream<T, VEC>(out + iv * VEC, o);
    }
  }
  if (VEC > 1 && blockIdx.x == gridDim.x - 1) {
    for (int64_t e = nvec * VEC + threadIdx.x; e < n; e += kBlock) {
      const float a = to_f32(x[e]);
      out[e] = from_f32<T>(a * sigmoid_f32(a) * to_f32(g[e]));
    }
  }
}

template <typename T, int VEC, int U>
__global__ void __launch_bounds__(kBlock)
swiglu_bwd_kernel(const T* __restrict__ dy, const T* __restrict__ x, const T* __restrict__ g,
                  T* __restrict__ dx, T* __restrict__ dg, int64_t n) {
  const int64_t nvec = n / VEC;
  const int64_t first = (int64_t)blockIdx.x * kBlock * U + threadIdx.x;
  float dv[U][VEC], xv[U][VEC], gv[U][VEC];
  const T* src[3] = {dy, x, g};
  float (*dst[3])[VEC] = {dv, xv, gv};
#pragma unroll
  for (int o = 0; o < 3; ++o)
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t iv = first + (int64_t)u * kBlock;
      if (iv < nvec) load_stream<T, VEC>(src[o] + iv * VEC, dst[o][u]);
    }
  // gradients in place: dv becomes dx, xv becomes dgate
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      const float s = sigmoid_f32(xv[u][i]);
      const float silu = xv[u][i] * s;
      const float dsilu = s * (1.0f + xv[u][i] * (1.0f - s));
      const float d = dv[u][i];
      dv[u][i] = d * gv[u][i] * dsilu;
      xv[u][i] = d * silu;
    }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t iv = first + (int64_t)u * kBlock;
    if (iv < nvec) store_stream<T, VEC>(dx + iv * VEC, dv[u]);
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t iv = first + (int64_t)u * kBlock;
    if (iv < nvec) store_stream<T, VEC>(dg + iv * VEC, xv[u]);
  }
  if (VEC > 1 && blockIdx.x == gridDim.x - 1) {
    for (int64_t e = nvec * VEC + threadIdx.x; e < n; e += kBlock) {
      const float a = to_f32(x[e]), d = to_f32(dy[e]), gg = to_f32(g[e]);
      const float s = sigmoid_f32(a);
      dx[e] = from_f32<T>(d * gg * (s * (1.0f + a * (1.0f - s))));
      dg[e] = from_f32<T>(d * (a * s));
    }
  }
}

// Row-strided variants: n_rows rows of n_cols elements; x and gate rows at
// stride ld_in, dy rows at ld_dy, outputs at ld_out (elements) -- e.g. x and
// gate as the two halves of each row of a fused [tokens, 2 * d_ff]
// projection, and the gradients written back into the same layout.  A
// workgroup covers up to kBlock * kRowU vectors of one row (the row index is
// one scalar division per workgroup).  One vector per lane per operand: at
// the GPT block's [16384, 2 x 3072] forward 55.5 -> 48.0 us and backward
// 83.2 -> 75.8 us against two (same box, alternating runs).
constexpr int kRowU = 1;

template <typename T, int VEC>
__global__ void __launch_bounds__(kBlock)
swiglu_rows_fwd_kernel(const T* __restrict__ x, const T* __restrict__ g, T* __restrict__ out,
                       int64_t n_cols, int64_t ld_in, int64_t ld_out, int64_t chunks) {
  const int64_t row = blockIdx.x / chunks;
  const int64_t c0 = (blockIdx.x - row * chunks) * (int64_t)kBlock * kRowU * VEC;
  const T* xr = x + row * ld_in;
  const T* gr = g + row * ld_in;
  T* orow = out + row * ld_out;
  float xv[kRowU][VEC], gv[kRowU][VEC];
#pragma unroll
  for (int u = 0; u < kRowU; ++u) {
    const int64_t c = c0 + ((int64_t)u * kBlock + threadIdx.x) * VEC;
    if (c < n_cols) {
      load_stream<T, VEC>(xr + c, xv[u]);
      load_stream<T, VEC>(gr + c, gv[u]);
    }
  }
#pragma unroll
  for (int u = 0; u < kRowU; ++u) {
    const int64_t c = c0 + ((int64_t)u * kBlock + threadIdx.x) * VEC;
    if (c < n_cols) {
      float o[VEC];
#pragma unroll
      for (int i = 0; i < VEC; ++i) o[i] = xv[u][i] * sigmoid_f32(xv[u][i]) * gv[u][i];
      store_stream<T, VEC>(orow + c, o);
    }
  }
}

template <typename T, int VEC>
__global__ void __launch_bounds__(kBlock)
swiglu_rows_bwd_kernel(const T* __restrict__ dy, const T* __restrict__ x, const T* __restrict__ g,
                       T* __restrict__ dx, T* __restrict__ dg, int64_t n_cols, int64_t ld_dy,
                       int64_t ld_in, int64_t ld_out, int64_t chunks) {
  const int64_t row = blockIdx.x / chunks;
  const int64_t c0 = (blockIdx.x - row * chunks) * (int64_t)kBlock * kRowU * VEC;
  const T* dyr = dy + row * ld_dy;
  const T* xr = x + row * ld_in;
  const T* gr = g + row * ld_in;
  float dv[kRowU][VEC], xv[kRowU][VEC], gv[kRowU][VEC];
#pragma unroll
  for (int u = 0; u < kRowU; ++u) {
    const int64_t c = c0 + ((int64_t)u * kBlock + threadIdx.x) * VEC;
    if (c < n_cols) {
      load_stream<T, VEC>(dyr + c, dv[u]);
      load_stream<T, VEC>(xr + c, xv[u]);
      load_stream<T, VEC>(gr + c, gv[u]);
    }
  }
#pragma unroll
  for (int u = 0; u < kRowU; ++u) {
    const int64_t c = c0 + ((int64_t)u * kBlock + threadIdx.x) * VEC;
    if (c < n_cols) {
      float ox[VEC], og[VEC];
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        const float s = sigmoid_f32(xv[u][i]);
        const float silu = xv[u][i] * s;
        const float dsilu = s * (1.0f + xv[u][i] * (1.0f - s));
        ox[i] = dv[u][i] * gv[u][i] * dsilu;
        og[i] = dv[u][i] * silu;
      }
      store_stream<T, VEC>(dx + row * ld_out + c, ox);
      store_stream<T, VEC>(dg + row * ld_out + c, og);
    }
  }
}

// VEC-element vectors when every row start stays 16-byte aligned and no
// vector straddles a row end.
template <typename T>
bool rows_vec_ok(std::initializer_list<const void*> ptrs, std::initializer_list<int64_t> lds,
                 int64_t n_cols) {
  constexpr int VEC = 16 / sizeof(T);
  for (const void* p : ptrs)
    if (!aligned16(p)) return false;
  for (int64_t ld : lds)
    if (ld % VEC) return false;
  return n_cols % VEC == 0;
}

template <int VEC>
int64_t row_chunks(int64_t n_cols) { return cdiv(n_cols, (int64_t)kBlock * kRowU * VEC); }

int check_rows(int64_t n_rows, int64_t n_cols, std::initializer_list<int64_t> lds) {
  if (n_rows < 0 || n_cols < 0)
    return fail(TRI_EINVAL, "swiglu_rows: bad shape %lld x %lld", (long long)n_rows,
                (long long)n_cols);
  for (int64_t ld : lds)
    if (ld < n_cols)
      return fail(TRI_EINVAL, "swiglu_rows: row stride %lld below %lld columns", (long long)ld,
                  (long long)n_cols);
  if (n_rows * cdiv(std::max<int64_t>(n_cols, 1), kBlock * kRowU) >= ((int64_t)1 << 31))
    return fail(TRI_EINVAL, "swiglu_rows: grid too large");
  return TRI_OK;
}

template <int VEC>
unsigned grid_for(int64_t n) {
  const int64_t nvec = n / VEC;
  return (unsigned)std::max<int64_t>(1, cdiv(nvec, (int64_t)kBlock * kUnroll));
}

template <typename T>
int fwd_impl(const void* x, const void* g, void* out, int64_t n, hipStream_t s) {
  constexpr int VEC = 16 / sizeof(T);
  if (aligned16(x) && aligned16(g) && aligned16(out)) {
    swiglu_fwd_kernel<T, VEC, kUnroll><<<grid_for<VEC>(n), kBlock, 0, s>>>(
        (const T*)x, (const T*)g, (T*)out, n);
  } else {
    swiglu_fwd_kernel<T, 1, kUnroll><<<grid_for<1>(n), kBlock, 0, s>>>(
        (const T*)x, (const T*)g, (T*)out, n);
  }
  return check_launch("swiglu forward");
}

template <typename T>
int bwd_impl(const void* dy, const void* x, const void* g, void* dx, void* dg, int64_t n,
             hipStream_t s) {
  constexpr int VEC = 16 / sizeof(T);
  if (aligned16(dy) && aligned16(x) && aligned16(g) && aligned16(dx) && aligned16(dg)) {
    swiglu_bwd_kernel<T, VEC, kUnroll><<<grid_for<VEC>(n), kBlock, 0, s>>>(
        (const T*)dy, (const T*)x, (const T*)g, (T*)dx, (T*)dg, n);
  } else {
    swiglu_bwd_kernel<T, 1, kUnroll><<<grid_for<1>(n), kBlock, 0, s>>>(
        (const T*)dy, (const T*)x, (const T*)g, (T*)dx, (T*)dg, n);
  }
  return check_launch("swiglu backward");
}

int check_n(int64_t n) {
  if (n < 0 || n / ((int64_t)kBlock * kUnroll) >= ((int64_t)1 << 31))
    return fail(TRI_EINVAL, "swiglu: unsupported element count %lld", (long long)n);
  return TRI_OK;
}

}  // namespace
}  // namespace tri

using namespace tri;

extern "C" int tritium_swiglu_fwd(const void* x, const void* gate, void* out, int64_t n,
                                  int dtype, void* stream) {
  if (int e = check_n(n)) return e;
  if (n == 0) return TRI_OK;
  TRI_DISPATCH_FLOAT(dtype, T, return fwd_impl<T>(x, gate, out, n, (hipStream_t)stream));
  return TRI_OK;
}

extern "C" int tritium_swiglu_bwd(const void* dy, const void* x, const void* gate, void* dx,
                                  void* dgate, int64_t n, int dtype, void* stream) {
  if (int e = check_n(n)) return e;
  if (n == 0) return TRI_OK;
  TRI_DISPATCH_FLOAT(dtype, T,
                     return bwd_impl<T>(dy, x, gate, dx, dgate, n, (hipStream_t)stream));
  return TRI_OK;
}

extern "C" int tritium_swiglu_rows_fwd(const void* x, const void* gate, void* out, int64_t n_rows,
                                       int64_t n_cols, int64_t ld_in, int64_t ld_out, int dtype,
                                       void* stream) {
  if (int e = check_rows(n_rows, n_cols, {ld_in, ld_out})) return e;
  if (n_rows == 0 || n_cols == 0) return TRI_OK;
  hipStream_t st = (hipStream_t)stream;
  TRI_DISPATCH_FLOAT(dtype, T, {
    constexpr int VEC = 16 / sizeof(T);
    if (rows_vec_ok<T>({x, gate, out}, {ld_in, ld_out}, n_cols)) {
      const int64_t ch = row_chunks<VEC>(n_cols);
      swiglu_rows_fwd_kernel<T, VEC><<<(unsigned)(n_rows * ch), kBlock, 0, st>>>(
          (const T*)x, (const T*)gate, (T*)out, n_cols, ld_in, ld_out, ch);
    } else {
      const int64_t ch = row_chunks<1>(n_cols);
      swiglu_rows_fwd_kernel<T, 1><<<(unsigned)(n_rows * ch), kBlock, 0, st>>>(
          (const T*)x, (const T*)gate, (T*)out, n_cols, ld_in, ld_out, ch);
    }
  });
  return check_launch("swiglu_rows forward");
}

extern "C" int tritium_swiglu_rows_bwd(const void* dy, const void* x, const void* gate, void* dx,
                                       void* dgate, int64_t n_rows, int64_t n_cols, int64_t ld_dy,
                                       int64_t ld_in, int64_t ld_out, int dtype, void* stream) {
  if (int e = check_rows(n_rows, n_cols, {ld_dy, ld_in, ld_out})) return e;
  if (n_rows == 0 || n_cols == 0) return TRI_OK;
  hipStream_t st = (hipStream_t)stream;
  TRI_DISPATCH_FLOAT(dtype, T, {
    constexpr int VEC = 16 / sizeof(T);
    if (rows_vec_ok<T>({dy, x, gate, dx, dgate}, {ld_dy, ld_in, ld_out}, n_cols)) {
      const int64_t ch = row_chunks<VEC>(n_cols);
      swiglu_rows_bwd_kernel<T, VEC><<<(unsigned)(n_rows * ch), kBlock, 0, st>>>(
          (const T*)dy, (const T*)x, (const T*)gate, (T*)dx, (T*)dgate, n_cols, ld_dy, ld_in,
          ld_out, ch);
    } else {
      const int64_t ch = row_chunks<1>(n_cols);
      swiglu_rows_bwd_kernel<T, 1><<<(unsigned)(n_rows * ch), kBlock, 0, st>>>(
          (const T*)dy, (const T*)x, (const T*)gate, (T*)dx, (T*)dgate, n_cols, ld_dy, ld_in,
          ld_out, ch);
    }
  });
  return check_launch("swiglu_rows backward");
}
