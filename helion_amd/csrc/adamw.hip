// Fused AdamW for gfx950: one tensor per launch, or a whole parameter list in
// ONE launch driven by a device-side descriptor table.
//
// Reference arithmetic: alkinun/helion tritium/ops/adamw.py:40-54 -- fp32
// moments, decoupled weight decay on the pre-update parameter, then
// p -= (lr / bc1) * m / (sqrt(v / bc2) + eps); bias corrections come from
// the host (adamw.py:133-134).
//
// Each block updates one CHUNK of one tensor with 16-byte accesses (4 fp32 or
// 8 fp16/bf16 parameters per access).  28 bytes move per fp32 parameter
// (read p, g, m, v; write p, m, v) -- the whole step is one HBM pass, every
// access streamed with the nontemporal hint.
//
// Multi-tensor table (int64, kDescWords per tensor, built by the host):
//   [param_ptr, grad_ptr, exp_avg_ptr, exp_avg_sq_ptr, numel, flags,
//    first_chunk]
// flags = dtype code | (1 << 8 if all four pointers are 16-byte aligned).
// first_chunk is the exclusive prefix sum of per-tensor chunk counts; block b
// finds its tensor as the length of the prefix of rows with first_chunk <= b
// (find_tensor).
#include "common.h"
#include "../../include/tritium_hip.h"

namespace tri {
namespace {

// One wavefront per workgroup: config-2 update 612-618 -> 586-595 us against
// 256 lanes (128: 607-617, 512: 620-623, 1024: 651-653), on the same boxes.
constexpr int kBlock = 64;
// 256 elements per workgroup, one group of 4 per lane (one 16-byte vector
// of each fp32 stream): config-2 update 561-565 us against 579-581 us with
// 512 (two groups per lane), same box, alternating runs -- the access shape
// of the fastest AdamW-shaped streaming probe (a grid of 64-lane workgroups,
// one vector per lane per array).
constexpr int64_t kChunk = 256;
// The mixed-precision kernel (four fp32 and two 16-bit streams per element)
// takes one group of 4 elements per lane, 256 elements per workgroup, as
// the fp32 kernel, loads and stores stream by stream: 715-718 us for the
// GPT step's 151.9 M parameters against 848 us for four steps of 8
// elements (two 16-byte vectors per fp32 stream) per lane; two groups per
// lane 719-735 us, four 712-738, eight 741-744 (same boxes).
constexpr int64_t kChunkMixed = (int64_t)kBlock * 4;  // 256 elements

struct Hyper {
  float lr, beta1, beta2, eps, weight_decay, bc1, bc2;
};

__device__ __forceinline__ void adam_update(float& p, float g, float& m, float& v,
                                            const Hyper& h, float lr_wd, float step_size) {
  m = h.beta1 * m + (1.0f - h.beta1) * g;
  v = h.beta2 * v + (1.0f - h.beta2) * g * g;
  p = p - lr_wd * p;
  const float denom = sqrtf(v / h.bc2) + h.eps;
  p = p - step_size * m / denom;
}

// Four consecutive elements of T as fp32, and back: one 16-byte access for
// fp32, 8 bytes for 16-bit types, both with the nontemporal hint.
template <typename T>
__device__ __forceinline__ void load4_nt(const T* __restrict__ p, float (&f)[4]) {
  if constexpr (sizeof(T) == 4) {
    unpack<float>(ld16_nt(p), f);
  } else {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 u = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
    const Pack<T, 4> pk = __builtin_bit_cast(Pack<T, 4>, u);
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = to_f32(pk.v[i]);
  }
}
template <typename T>
__device__ __forceinline__ void store4_nt(T* __restrict__ p, const float (&f)[4]) {
  if constexpr (sizeof(T) == 4) {
    st16_nt(p, pack<float>(f));
  } else {
    Pack<T, 4> pk;
#pragma unroll
    for (int i = 0; i < 4; ++i) pk.v[i] = from_f32<T>(f[i]);
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    __builtin_nontemporal_store(__builtin_bit_cast(u32x2, pk), reinterpret_cast<u32x2*>(p));
  }
}

// Update elements [start, start + kChunk) of one tensor (clipped to n).
// With 16-byte aligned tensors each lane owns NS = kChunk / (4 kBlock) groups
// of 4 consecutive elements (one at 256 elements per workgroup), kBlock
// groups apart, and issues its loads stream by stream (its
// p groups, then g, m, v) and its stores likewise (m, v, p); elements past
// the last whole group of 4 go one per lane.
template <typename T>
__device__ __forceinline__ void adam_chunk(T* __restrict__ p, const T* __restrict__ g,
                                           float* __restrict__ m, float* __restrict__ v,
                                           int64_t n, int64_t start, bool vec_ok,
                                           const Hyper& h) {
  const float lr_wd = h.lr * h.weight_decay;
  const float step_size = h.lr / h.bc1;
  const int64_t end = min(start + kChunk, n);
  int64_t tail = start;
  if (vec_ok) {
    constexpr int NS = (int)(kChunk / (4 * kBlock));
    static_assert(NS * 4 * kBlock == kChunk, "chunk = whole groups of 4 per lane");
    const int64_t vec_end = start + ((end - start) / 4) * 4;
    float pv[NS][4] = {}, gv[NS][4] = {}, mv[NS][4] = {}, vv[NS][4] = {};  // lanes past the end compute on zeros
    auto elem = [&](int u) { return start + ((int64_t)u * kBlock + threadIdx.x) * 4; };
#pragma unroll
    for (int u = 0; u < NS; ++u)
      if (elem(u) < vec_end) load4_nt<T>(p + elem(u), pv[u]);
#pragma unroll
    for (int u = 0; u < NS; ++u)
      if (elem(u) < vec_end) load4_nt<T>(g + elem(u), gv[u]);
#pragma unroll
    for (int u = 0; u < NS; ++u)
      if (elem(u) < vec_end) load4_nt<float>(m + elem(u), mv[u]);
#pragma unroll
    for (int u = 0; u < NS; ++u)
      if (elem(u) < vec_end) load4_nt<float>(v + elem(u), vv[u]);
#pragma unroll
    for (int u = 0; u < NS; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) adam_update(pv[u][i], gv[u][i], mv[u][i], vv[u][i], h, lr_wd, step_size);
#pragma unroll
    for (int u = 0; u < NS; ++u)
      if (elem(u) < vec_end) store4_nt<float>(m + elem(u), mv[u]);
#pragma unroll
    for (int u = 0; u < NS; ++u)
      if (elem(u) < vec_end) store4_nt<float>(v + elem(u), vv[u]);
#pragma unroll
    for (int u = 0; u < NS; ++u)
      if (elem(u) < vec_end) store4_nt<T>(p + elem(u), pv[u]);
    tail = vec_end;
  }
  for (int64_t e = tail + threadIdx.x; e < end; e += kBlock) {
    float pp = to_f32(p[e]), mm = m[e], vv2 = v[e];
    adam_update(pp, to_f32(g[e]), mm, vv2, h, lr_wd, step_size);
    m[e] = mm;
    v[e] = vv2;
    p[e] = from_f32<T>(pp);
  }
}

template <typename T>
__global__ void __launch_bounds__(kBlock)
adamw_single_kernel(T* __restrict__ p, const T* __restrict__ g, float* __restrict__ m,
                    float* __restrict__ v, int64_t n, int vec_ok, Hyper h) {
  adam_chunk<T>(p, g, m, v, n, (int64_t)blockIdx.x * kChunk, vec_ok != 0, h);
}

constexpr int kDescWords = 7;

// The tensor of block b: the last table row whose first_chunk (word 6) is
// <= b.  first_chunk does not decrease, so the rows that pass form a prefix
// and its length is the count of passing rows: each lane tests four rows per
// round, the loads issued together, where a binary search would chain
// log2(n) dependent loads before the block's first data load.
__device__ __forceinline__ int find_tensor(const int64_t* __restrict__ table, int words, int n,
                                           int64_t b) {
  const int lane = threadIdx.x & 63;
  int count = 0;
  for (int base = 0; base < n; base += 4 * 64) {
    bool le[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int i = base + k * 64 + lane;
      le[k] = i < n && table[(int64_t)i * words + 6] <= b;
    }
    int c = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) c += __popcll(__ballot(le[k]));
    count += c;
    if (c < 4 * 64) break;  // the prefix ended in this round
  }
  return __builtin_amdgcn_readfirstlane(count - 1);
}

__global__ void __launch_bounds__(kBlock)
adamw_multi_kernel(const int64_t* __restrict__ table, int n_tensors, Hyper h) {
  const int64_t b = blockIdx.x;
  const int64_t* d = table + (int64_t)find_tensor(table, kDescWords, n_tensors, b) * kDescWords;
  const int64_t n = d[4];
  const int flags = (int)d[5];
  const int64_t start = (b - d[6]) * kChunk;
  if (start >= n) return;
  const bool vec_ok = (flags >> 8) & 1;
  switch (flags & 0xff) {
    case kF32:
      adam_chunk<float>((float*)d[0], (const float*)d[1], (float*)d[2], (float*)d[3], n, start, vec_ok, h);
      break;
    case kF16:
      adam_chunk<f16_t>((f16_t*)d[0], (const f16_t*)d[1], (float*)d[2], (float*)d[3], n, start, vec_ok, h);
      break;
    case kBF16:
      adam_chunk<bf16_t>((bf16_t*)d[0], (const bf16_t*)d[1], (float*)d[2], (float*)d[3], n, start, vec_ok, h);
      break;
    default:
      break;
  }
}

// Mixed precision: fp32 parameters and moments, 16-bit gradients (read as
// they are), and optionally a 16-bit copy of each updated parameter (the
// working weights of a mixed-precision model) written in the same pass --
// 28 bytes per parameter, where widening the gradients first and rounding
// the weights afterwards would add 12.  Groups of 4 elements per lane: one
// 16-byte vector of each fp32 stream, 8 bytes of each 16-bit stream.
template <typename TG>
__device__ __forceinline__ void adam_chunk_mixed(float* __restrict__ p, const TG* __restrict__ g,
                                                 float* __restrict__ m, float* __restrict__ v,
                                                 TG* __restrict__ shadow, int64_t n, int64_t start,
                                                 bool vec_ok, const Hyper& h) {
  static_assert(sizeof(TG) == 2, "16-bit gradients");
  const float lr_wd = h.lr * h.weight_decay;
  const float step_size = h.lr / h.bc1;
  const int64_t end = min(start + kChunkMixed, n);
  int64_t tail = start;
  if (vec_ok) {
    constexpr int NS = (int)(kChunkMixed / (4 * kBlock));
    const int64_t vec_end = start + ((end - start) / 4) * 4;
    float pv[NS][4] = {}, gv[NS][4] = {}, mv[NS][4] = {}, vv[NS][4] = {};  // lanes past the end compute on zeros
    auto elem = [&](int u) { return start + ((int64_t)u * kBlock + threadIdx.x) * 4; };
#pragma unroll
    for (int u = 0; u < NS; ++u)
      if (elem(u) < vec_end) load4_nt<float>(p + elem(u), pv[u]);
#pragma unroll
    for (int u = 0; u < NS; ++u)
      if (elem(u) < vec_end) load4_nt<TG>(g + elem(u), gv[u]);
#pragma unroll
    for (int u = 0; u < NS; ++u)
      if (elem(u) < vec_end) load4_nt<float>(m + elem(u), mv[u]);
#pragma unroll
    for (int u = 0; u < NS; ++u)
      if (elem(u) < vec_end) load4_nt<float>(v + elem(u), vv[u]);
#pragma unroll
    for (int u = 0; u < NS; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) adam_update(pv[u][i], gv[u][i], mv[u][i], vv[u][i], h, lr_wd, step_size);
#pragma unroll
    for (int u = 0; u < NS; ++u)
      if (elem(u) < vec_end) store4_nt<float>(m + elem(u), mv[u]);
#pragma unroll
    for (int u = 0; u < NS; ++u)
      if (elem(u) < vec_end) store4_nt<float>(v + elem(u), vv[u]);
#pragma unroll
    for (int u = 0; u < NS; ++u)
      if (elem(u) < vec_end) store4_nt<float>(p + elem(u), pv[u]);
    if (shadow != nullptr) {
#pragma unroll
      for (int u = 0; u < NS; ++u)
        if (elem(u) < vec_end) store4_nt<TG>(shadow + elem(u), pv[u]);
    }
    tail = vec_end;
  }
  for (int64_t e = tail + threadIdx.x; e < end; e += kBlock) {
    float pp = p[e], mm = m[e], vv2 = v[e];
    adam_update(pp, to_f32(g[e]), mm, vv2, h, lr_wd, step_size);
    m[e] = mm;
    v[e] = vv2;
    p[e] = pp;
    if (shadow != nullptr) shadow[e] = from_f32<TG>(pp);
  }
}

// Table rows of kMixedWords int64: [param, grad, exp_avg, exp_avg_sq, numel,
// flags (bit 0: every pointer 16-byte aligned), first_chunk, shadow or 0].
constexpr int kMixedWords = 8;

template <typename TG>
__global__ void __launch_bounds__(kBlock)
adamw_mixed_kernel(const int64_t* __restrict__ table, int n_tensors, Hyper h) {
  const int64_t b = blockIdx.x;
  const int64_t* d = table + (int64_t)find_tensor(table, kMixedWords, n_tensors, b) * kMixedWords;
  const int64_t n = d[4];
  const int64_t start = (b - d[6]) * kChunkMixed;
  if (start >= n) return;
  adam_chunk_mixed<TG>((float*)d[0], (const TG*)d[1], (float*)d[2], (float*)d[3], (TG*)d[7], n,
                       start, (d[5] & 1) != 0, h);
}

Hyper make_hyper(float lr, float beta1, float beta2, float eps, float wd, double bc1, double bc2) {
  return Hyper{lr, beta1, beta2, eps, wd, (float)bc1, (float)bc2};
}

}  // namespace
}  // namespace tri

using namespace tri;

extern "C" int64_t tritium_adamw_chunk_elements(void) { return kChunk; }
extern "C" int64_t tritium_adamw_mixed_chunk_elements(void) { return kChunkMixed; }

extern "C" int tritium_adamw_step(void* param, const void* grad, float* exp_avg, float* exp_avg_sq,
                                  int64_t n, float lr, float beta1, float beta2, float eps,
                                  float weight_decay, double bias_correction1,
                                  double bias_correction2, int dtype, void* stream) {
  if (n < 0) return fail(TRI_EINVAL, "adamw: negative numel");
  if (n == 0) return TRI_OK;
  const Hyper h = make_hyper(lr, beta1, beta2, eps, weight_decay, bias_correction1, bias_correction2);
  const int vec_ok = aligned16(param) && aligned16(grad) && aligned16(exp_avg) && aligned16(exp_avg_sq);
  const int64_t blocks = cdiv(n, kChunk);
  if (blocks >= ((int64_t)1 << 31)) return fail(TRI_EINVAL, "adamw: tensor too large");
  TRI_DISPATCH_FLOAT(dtype, T,
    adamw_single_kernel<T><<<(unsigned)blocks, kBlock, 0, (hipStream_t)stream>>>(
        (T*)param, (const T*)grad, exp_avg, exp_avg_sq, n, vec_ok, h));
  return check_launch("adamw step");
}

extern "C" int tritium_adamw_step_multi(const int64_t* table, int n_tensors, int64_t total_chunks,
                                        float lr, float beta1, float beta2, float eps,
                                        float weight_decay, double bias_correction1,
                                        double bias_correction2, void* stream) {
  if (n_tensors < 0 || total_chunks < 0) return fail(TRI_EINVAL, "adamw multi: bad table size");
  if (n_tensors == 0 || total_chunks == 0) return TRI_OK;
  if (total_chunks >= ((int64_t)1 << 31)) return fail(TRI_EINVAL, "adamw multi: too many chunks");
  const Hyper h = make_hyper(lr, beta1, beta2, eps, weight_decay, bias_correction1, bias_correction2);
  adamw_multi_kernel<<<(unsigned)total_chunks, kBlock, 0, (hipStream_t)stream>>>(table, n_tensors, h);
  return check_launch("adamw multi-tensor step");
}

extern "C" int tritium_adamw_step_mixed(const int64_t* table, int n_tensors, int64_t total_chunks,
                                        float lr, float beta1, float beta2, float eps,
                                        float weight_decay, double bias_correction1,
                                        double bias_correction2, int grad_dtype, void* stream) {
  if (n_tensors < 0 || total_chunks < 0) return fail(TRI_EINVAL, "adamw mixed: bad table size");
  if (n_tensors == 0 || total_chunks == 0) return TRI_OK;
  if (total_chunks >= ((int64_t)1 << 31)) return fail(TRI_EINVAL, "adamw mixed: too many chunks");
  const Hyper h = make_hyper(lr, beta1, beta2, eps, weight_decay, bias_correction1, bias_correction2);
  hipStream_t st = (hipStream_t)stream;
  if (grad_dtype == kBF16) {
    adamw_mixed_kernel<bf16_t><<<(unsigned)total_chunks, kBlock, 0, st>>>(table, n_tensors, h);
  } else if (grad_dtype == kF16) {
    adamw_mixed_kernel<f16_t><<<(unsigned)total_chunks, kBlock, 0, st>>>(table, n_tensors, h);
  } else {
    return fail(TRI_EINVAL, "adamw mixed: gradients must be 16-bit (dtype code %d)", grad_dtype);
  }
  return check_launch("adamw mixed-precision step");
}
