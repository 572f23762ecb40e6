// Sum of split-K partial products, rounded once into the output dtype.
//
// A weight gradient dW = dY^T X over many token rows is computed as s batched
// GEMMs over token slices with fp32 outputs (the short-and-wide product gets
// the parallelism a single GEMM lacks); this kernel finishes it in one pass:
// dst[i] = (T)(src[0][i] + src[1][i] + ... + src[s-1][i]), summed in fp32 in
// slice order, 16-byte nontemporal loads, 4 outputs per lane.  It replaces a
// framework reduction followed by a separate cast (two passes over the output).
#include "common.h"
#include "../../include/tritium_hip.h"

namespace tri {
namespace {

// 64-lane workgroups (the GPT step's split sums 22.9 -> 20.2 us on average
// against 256 lanes, same box)
constexpr int kBlock = 64;

template <typename T>
__global__ void __launch_bounds__(kBlock)
sum_splits_kernel(const float* __restrict__ src, T* __restrict__ dst, int64_t n_splits, int64_t n,
                  int vec_ok) {
  const int64_t i = ((int64_t)blockIdx.x * kBlock + threadIdx.x) * 4;
  if (i >= n) return;
  if (vec_ok && i + 4 <= n) {
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
    for (int64_t s = 0; s < n_splits; ++s) {
      float f[4];
      unpack<float>(ld16_nt(src + s * n + i), f);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] += f[e];
    }
    store_f32<T, 4>(dst + i, acc);
    return;
  }
  for (int64_t j = i; j < i + 4 && j < n; ++j) {
    float acc = 0.f;
    for (int64_t s = 0; s < n_splits; ++s) acc += src[s * n + j];
    dst[j] = from_f32<T>(acc);
  }
}

}  // namespace
}  // namespace tri

using namespace tri;

extern "C" int tritium_sum_splits(const float* src, void* dst, int64_t n_splits, int64_t n,
                                  int dtype, void* stream) {
  if (n_splits <= 0 || n < 0) return fail(TRI_EINVAL, "sum_splits: bad sizes");
  if (n == 0) return TRI_OK;
  const int vec_ok = aligned16(src) && n % 4 == 0 && ((uintptr_t)dst % (4 * dtype_size(dtype))) == 0;
  const int64_t blocks = cdiv(cdiv(n, 4), kBlock);
  if (blocks > 0x7fffffffLL) return fail(TRI_EINVAL, "sum_splits: too many elements");
  hipStream_t st = (hipStream_t)stream;
  TRI_DISPATCH_FLOAT(dtype, T,
    sum_splits_kernel<T><<<(unsigned)blocks, kBlock, 0, st>>>(src, (T*)dst, n_splits, n, vec_ok));
  return check_launch("sum_splits");
}
