// HBM streaming probes for bench.py --stream-probe: the practical ceilings the
// row kernels' bandwidth is judged against.  Every pattern streams 16-byte
// vectors with the nontemporal hint (as the row kernels do), U = 4 vectors
// per lane in flight, a persistent grid of `blocks` 256-lane workgroups:
//   0  read only            (reads n vectors of a)
//   1  copy                 (a -> b)
//   2  fill                 (writes n vectors of b)
//   3  AdamW-shaped update  (reads p, g, m, v; writes p, m, v in place)
// Measurement only: no operator of the library depends on it.
#include "common.h"
#include "../../include/tritium_hip.h"

namespace tri {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
constexpr int kU = 4;

__device__ __forceinline__ f4 ldn(const f4* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ void stn(f4* p, f4 v) { __builtin_nontemporal_store(v, p); }

__global__ void __launch_bounds__(256) probe_read(const f4* __restrict__ a, int64_t n, float* sink) {
  int64_t i = (int64_t)blockIdx.x * 256 * kU + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * 256 * kU;
  f4 s = {0.f, 0.f, 0.f, 0.f};
  for (; i + 256 * (kU - 1) < n; i += stride) {
    f4 v[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) v[u] = ldn(a + i + 256 * u);
#pragma unroll
    for (int u = 0; u < kU; ++u) s += v[u];
  }
  // keeps the loads; a real sum of this value never happens for the probe's data
  if (s.x + s.y + s.z + s.w == 1.2345e30f) sink[threadIdx.x] = s.x;
}

__global__ void __launch_bounds__(256) probe_copy(const f4* __restrict__ a, f4* __restrict__ b, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * 256 * kU + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * 256 * kU;
  for (; i + 256 * (kU - 1) < n; i += stride) {
    f4 v[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) v[u] = ldn(a + i + 256 * u);
#pragma unroll
    for (int u = 0; u < kU; ++u) stn(b + i + 256 * u, v[u]);
  }
}

__global__ void __launch_bounds__(256) probe_fill(f4* __restrict__ b, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * 256 * kU + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * 256 * kU;
  const f4 z = {1.f, 2.f, 3.f, 4.f};
  for (; i + 256 * (kU - 1) < n; i += stride) {
#pragma unroll
    for (int u = 0; u < kU; ++u) stn(b + i + 256 * u, z);
  }
}

__global__ void __launch_bounds__(256) probe_update(f4* __restrict__ p, const f4* __restrict__ g,
                                                    f4* __restrict__ m, f4* __restrict__ v, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * 256 * kU + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * 256 * kU;
  for (; i + 256 * (kU - 1) < n; i += stride) {
    f4 a[kU], b[kU], c[kU], d[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      a[u] = ldn(p + i + 256 * u);
      b[u] = ldn(g + i + 256 * u);
      c[u] = ldn(m + i + 256 * u);
      d[u] = ldn(v + i + 256 * u);
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      c[u] = 0.9f * c[u] + 0.1f * b[u];
      d[u] = 0.95f * d[u] + 0.05f * b[u] * b[u];
      a[u] = a[u] - 1e-3f * c[u] / (d[u] + 1e-8f);
      stn(p + i + 256 * u, a[u]);
      stn(m + i + 256 * u, c[u]);
      stn(v + i + 256 * u, d[u]);
    }
  }
}

}  // namespace
}  // namespace tri

using namespace tri;

extern "C" int tritium_stream_probe(int pattern, void* a, void* b, void* c, void* d,
                                    int64_t n_vec4, int blocks, void* stream) {
  if (pattern < 0 || pattern > 3 || n_vec4 < 0 || blocks <= 0 || blocks > (1 << 20))
    return fail(TRI_EINVAL, "stream probe: bad pattern %d, n_vec4 %lld or blocks %d", pattern,
                (long long)n_vec4, blocks);
  if (a == nullptr || (pattern != 2 && b == nullptr) ||
      (pattern == 3 && (c == nullptr || d == nullptr)))
    return fail(TRI_EINVAL, "stream probe: missing buffer for pattern %d", pattern);
  hipStream_t st = (hipStream_t)stream;
  switch (pattern) {
    case 0: probe_read<<<blocks, 256, 0, st>>>((const f4*)a, n_vec4, (float*)b); break;
    case 1: probe_copy<<<blocks, 256, 0, st>>>((const f4*)a, (f4*)b, n_vec4); break;
    case 2: probe_fill<<<blocks, 256, 0, st>>>((f4*)a, n_vec4); break;
    default: probe_update<<<blocks, 256, 0, st>>>((f4*)a, (const f4*)b, (f4*)c, (f4*)d, n_vec4); break;
  }
  return check_launch("stream probe");
}
