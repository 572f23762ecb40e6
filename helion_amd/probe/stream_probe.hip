// HBM streaming probes: the practical ceilings that the row kernels'
// bandwidth is judged against.  Built into its own library,
// libtritium_probe.so, which only `bench.py --stream-probe` loads; no
// operator depends on it and the product library does not contain it.
//
// Every pattern streams 16-byte vectors with the nontemporal hint, as the
// row kernels do.  Persistent patterns run `blocks` 256-lane workgroups that
// stride over the array with kU = 4 vectors per lane in flight (the vectors a
// lane's last full group does not cover are handled one per lane after the
// loop); grid-covering patterns launch one 256-lane workgroup per 256 vectors,
// one vector per lane, and ignore `blocks`:
//   0  read only, persistent             (reads a; b is a 1 KB sink)
//   1  copy a -> b, persistent
//   2  fill a, persistent
//   3  AdamW-shaped update, persistent   (reads a, b, c, d; writes a, c, d)
//   4  read only, grid-covering          (reads a; b is a 1 KB sink)
//   5  copy a -> b, grid-covering
//   6  fill a, grid-covering
//   7  two streams read, one written, grid-covering (a + b -> c): the
//      access shape of the RMSNorm backward (x, dy -> dx) and SwiGLU forward
//   8  AdamW-shaped update, grid-covering: `blocks` is the workgroup size (64
//      or 256 lanes), each lane one 16-byte vector of each of a, b, c, d
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
constexpr int kU = 4;
constexpr int kBlock = 256;

char g_err[256];

__device__ __forceinline__ f4 ldn(const f4* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ void stn(f4* p, f4 v) { __builtin_nontemporal_store(v, p); }

// Persistent loops: full groups of kU vectors per lane while the whole group
// is in range, then the remainder one vector per lane.
__global__ void __launch_bounds__(kBlock) probe_read(const f4* __restrict__ a, int64_t n,
                                                     float* sink) {
  int64_t i = (int64_t)blockIdx.x * kBlock * kU + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * kBlock * kU;
  f4 s = {0.f, 0.f, 0.f, 0.f};
  for (; i + kBlock * (kU - 1) < n; i += stride) {
    f4 v[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) v[u] = ldn(a + i + kBlock * u);
#pragma unroll
    for (int u = 0; u < kU; ++u) s += v[u];
  }
  for (int u = 0; u < kU; ++u)
    if (i + kBlock * u < n) s += ldn(a + i + kBlock * u);
  // keeps the loads; the probe's data never sums to this value
  if (s.x + s.y + s.z + s.w == 1.2345e30f) sink[threadIdx.x] = s.x;
}

__global__ void __launch_bounds__(kBlock) probe_copy(const f4* __restrict__ a, f4* __restrict__ b,
                                                     int64_t n) {
  int64_t i = (int64_t)blockIdx.x * kBlock * kU + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * kBlock * kU;
  for (; i + kBlock * (kU - 1) < n; i += stride) {
    f4 v[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) v[u] = ldn(a + i + kBlock * u);
#pragma unroll
    for (int u = 0; u < kU; ++u) stn(b + i + kBlock * u, v[u]);
  }
  for (int u = 0; u < kU; ++u)
    if (i + kBlock * u < n) stn(b + i + kBlock * u, ldn(a + i + kBlock * u));
}

__global__ void __launch_bounds__(kBlock) probe_fill(f4* __restrict__ a, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * kBlock * kU + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * kBlock * kU;
  const f4 z = {1.f, 2.f, 3.f, 4.f};
  for (; i + kBlock * (kU - 1) < n; i += stride) {
#pragma unroll
    for (int u = 0; u < kU; ++u) stn(a + i + kBlock * u, z);
  }
  for (int u = 0; u < kU; ++u)
    if (i + kBlock * u < n) stn(a + i + kBlock * u, z);
}

__device__ __forceinline__ void adamw_like(f4& p, f4 g, f4& m, f4& v) {
  m = 0.9f * m + 0.1f * g;
  v = 0.95f * v + 0.05f * g * g;
  p = p - 1e-3f * m / (v + 1e-8f);
}

__global__ void __launch_bounds__(kBlock) probe_update(f4* __restrict__ p, const f4* __restrict__ g,
                                                       f4* __restrict__ m, f4* __restrict__ v,
                                                       int64_t n) {
  int64_t i = (int64_t)blockIdx.x * kBlock * kU + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * kBlock * kU;
  for (; i + kBlock * (kU - 1) < n; i += stride) {
    f4 a[kU], b[kU], c[kU], d[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      a[u] = ldn(p + i + kBlock * u);
      b[u] = ldn(g + i + kBlock * u);
      c[u] = ldn(m + i + kBlock * u);
      d[u] = ldn(v + i + kBlock * u);
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      adamw_like(a[u], b[u], c[u], d[u]);
      stn(p + i + kBlock * u, a[u]);
      stn(m + i + kBlock * u, c[u]);
      stn(v + i + kBlock * u, d[u]);
    }
  }
  for (int u = 0; u < kU; ++u) {
    const int64_t j = i + kBlock * u;
    if (j >= n) continue;
    f4 a = ldn(p + j), c = ldn(m + j), d = ldn(v + j);
    adamw_like(a, ldn(g + j), c, d);
    stn(p + j, a);
    stn(m + j, c);
    stn(v + j, d);
  }
}

__global__ void __launch_bounds__(kBlock) cover_read(const f4* __restrict__ a, int64_t n,
                                                     float* sink) {
  const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= n) return;
  const f4 s = ldn(a + i);
  if (s.x + s.y + s.z + s.w == 1.2345e30f) sink[threadIdx.x] = s.x;
}

__global__ void __launch_bounds__(kBlock) cover_copy(const f4* __restrict__ a, f4* __restrict__ b,
                                                     int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i < n) stn(b + i, ldn(a + i));
}

__global__ void __launch_bounds__(kBlock) cover_fill(f4* __restrict__ a, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const f4 z = {1.f, 2.f, 3.f, 4.f};
  if (i < n) stn(a + i, z);
}

__global__ void __launch_bounds__(kBlock) cover_2r1w(const f4* __restrict__ a,
                                                     const f4* __restrict__ b,
                                                     f4* __restrict__ c, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i < n) stn(c + i, ldn(a + i) + ldn(b + i));
}

template <int L>
__global__ void __launch_bounds__(L) cover_update(f4* __restrict__ p, const f4* __restrict__ g,
                                                  f4* __restrict__ m, f4* __restrict__ v,
                                                  int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * L + threadIdx.x;
  if (i >= n) return;
  f4 a = ldn(p + i);
  const f4 b = ldn(g + i);
  f4 c = ldn(m + i), d = ldn(v + i);
  adamw_like(a, b, c, d);
  stn(m + i, c);
  stn(v + i, d);
  stn(p + i, a);
}

}  // namespace

extern "C" const char* tritium_probe_last_error() { return g_err; }

// Returns 0, or 1 with tritium_probe_last_error() set.  Buffers of n_vec4
// 16-byte vectors each, 16-byte aligned, on the current device.
extern "C" int tritium_stream_probe(int pattern, void* a, void* b, void* c, void* d,
                                    int64_t n_vec4, int blocks, void* stream) {
  if (pattern < 0 || pattern > 8 || n_vec4 < 0 || blocks <= 0 || blocks > (1 << 20) ||
      (pattern == 8 && blocks != 64 && blocks != 256)) {
    snprintf(g_err, sizeof(g_err), "stream probe: bad pattern %d, n_vec4 %lld or blocks %d",
             pattern, (long long)n_vec4, blocks);
    return 1;
  }
  const bool need_b = pattern != 2 && pattern != 6;
  const bool need_cd = pattern == 3 || pattern == 8;
  if (a == nullptr || (need_b && b == nullptr) || (need_cd && d == nullptr) ||
      ((need_cd || pattern == 7) && c == nullptr)) {
    snprintf(g_err, sizeof(g_err), "stream probe: missing buffer for pattern %d", pattern);
    return 1;
  }
  hipStream_t st = (hipStream_t)stream;
  const int lanes = pattern == 8 ? blocks : kBlock;
  const int64_t cover = (n_vec4 + lanes - 1) / lanes;
  if (pattern >= 4 && (cover == 0 || cover > 0x7fffffffLL)) {
    snprintf(g_err, sizeof(g_err), "stream probe: %lld vectors do not fit one grid",
             (long long)n_vec4);
    return 1;
  }
  switch (pattern) {
    case 0: probe_read<<<blocks, kBlock, 0, st>>>((const f4*)a, n_vec4, (float*)b); break;
    case 1: probe_copy<<<blocks, kBlock, 0, st>>>((const f4*)a, (f4*)b, n_vec4); break;
    case 2: probe_fill<<<blocks, kBlock, 0, st>>>((f4*)a, n_vec4); break;
    case 3:
      probe_update<<<blocks, kBlock, 0, st>>>((f4*)a, (const f4*)b, (f4*)c, (f4*)d, n_vec4);
      break;
    case 4: cover_read<<<(unsigned)cover, kBlock, 0, st>>>((const f4*)a, n_vec4, (float*)b); break;
    case 5: cover_copy<<<(unsigned)cover, kBlock, 0, st>>>((const f4*)a, (f4*)b, n_vec4); break;
    case 6: cover_fill<<<(unsigned)cover, kBlock, 0, st>>>((f4*)a, n_vec4); break;
    case 7:
      cover_2r1w<<<(unsigned)cover, kBlock, 0, st>>>((const f4*)a, (const f4*)b, (f4*)c, n_vec4);
      break;
    default:
      if (blocks == 64)
        cover_update<64><<<(unsigned)cover, 64, 0, st>>>((f4*)a, (const f4*)b, (f4*)c, (f4*)d, n_vec4);
      else
        cover_update<256><<<(unsigned)cover, 256, 0, st>>>((f4*)a, (const f4*)b, (f4*)c, (f4*)d, n_vec4);
      break;
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    snprintf(g_err, sizeof(g_err), "stream probe: %s", hipGetErrorString(e));
    return 1;
  }
  return 0;
}
