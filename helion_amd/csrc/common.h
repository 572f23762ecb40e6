// Shared device helpers and C-ABI error plumbing for libtritium_hip.so.
//
// Everything here is written for gfx950 (CDNA4): 64-lane wavefronts,
// 16-byte global vector accesses, hardware bf16 conversion.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <algorithm>
#include <type_traits>

namespace tri {

// dtype codes shared with the Python boundary (helion_amd/_lib.py).
enum DType : int { kF32 = 0, kF16 = 1, kBF16 = 2 };

typedef __bf16 bf16_t;
typedef _Float16 f16_t;

constexpr int kWave = 64;

// N elements of T moved as one aligned access (16 bytes for N*sizeof(T)==16).
template <typename T, int N>
struct __attribute__((aligned(sizeof(T) * N))) Pack {
  T v[N];
};

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(f16_t x) { return (float)x; }
__device__ __forceinline__ float to_f32(bf16_t x) { return (float)x; }

template <typename T>
__device__ __forceinline__ T from_f32(float x) {
  return (T)x;  // round-to-nearest-even (v_cvt_pk_bf16_f32 / v_cvt_f16_f32)
}

template <typename T, int N>
__device__ __forceinline__ void load_f32(const T* __restrict__ p, float (&out)[N]) {
  Pack<T, N> pk = *reinterpret_cast<const Pack<T, N>*>(p);
#pragma unroll
  for (int i = 0; i < N; ++i) out[i] = to_f32(pk.v[i]);
}

template <typename T, int N>
__device__ __forceinline__ void store_f32(T* __restrict__ p, const float (&in)[N]) {
  Pack<T, N> pk;
#pragma unroll
  for (int i = 0; i < N; ++i) pk.v[i] = from_f32<T>(in[i]);
  *reinterpret_cast<Pack<T, N>*>(p) = pk;
}

// ---- 16-byte raw vectors ----------------------------------------------------
// A row is streamed as raw 16-byte vectors (8 x 16-bit or 4 x fp32) and
// unpacked to fp32 only where it is used, so a prefetched row costs 4 VGPRs
// per vector.  *_nt accesses carry the nontemporal hint: data read or
// written once streams past the caches (measured on MI355X: a copy reaches
// about 6.1 TB/s this way against 5.5 TB/s with ordinary stores).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ u32x4 ld16_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }
__device__ __forceinline__ void st16_nt(void* p, u32x4 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

// fp32 values of one raw vector of T (16 / sizeof(T) elements).
template <typename T>
__device__ __forceinline__ void unpack(u32x4 u, float (&f)[16 / sizeof(T)]) {
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = __uint_as_float(u[i]);
  } else if constexpr (std::is_same<T, bf16_t>::value) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // bf16 -> fp32 is exact: the high half of the word
      f[2 * i] = __uint_as_float(u[i] << 16);
      f[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
    }
  } else {
    const Pack<T, 8> p = __builtin_bit_cast(Pack<T, 8>, u);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = (float)p.v[i];
  }
}

// Round fp32 values to T (nearest-even) and pack them into one raw vector.
template <typename T>
__device__ __forceinline__ u32x4 pack(const float (&f)[16 / sizeof(T)]) {
  Pack<T, 16 / sizeof(T)> p;
#pragma unroll
  for (int i = 0; i < 16 / (int)sizeof(T); ++i) p.v[i] = from_f32<T>(f[i]);
  return __builtin_bit_cast(u32x4, p);
}

// VEC elements at p as fp32 / stored from fp32; a 16-byte vector (the aligned
// fast paths) streams with the nontemporal hint, anything else is a plain
// access.
template <typename T, int VEC>
__device__ __forceinline__ void load_stream(const T* __restrict__ p, float (&f)[VEC]) {
  if constexpr (VEC * sizeof(T) == 16) unpack<T>(ld16_nt(p), f);
  else load_f32<T, VEC>(p, f);
}
template <typename T, int VEC>
__device__ __forceinline__ void store_stream(T* __restrict__ p, const float (&f)[VEC]) {
  if constexpr (VEC * sizeof(T) == 16) st16_nt(p, pack<T>(f));
  else store_f32<T, VEC>(p, f);
}

// Butterfly sum over the 64 lanes of a wavefront; every lane gets the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// Index of the calling wavefront in its workgroup, as a wave-uniform
// (scalar) value: conditions built from it become scalar branches instead
// of per-lane exec masking.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

// 2^x as one v_exp_f32.  exp2f() wraps it in a range reduction (compare,
// two selects, add, ldexp) that keeps results below 2^-126 exact; softmax
// weights that small are negligible, and exp2(-inf) = 0 either way.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// One RoPE pair (a, b) at angle (c = cos, s = sin): (a c - b s, b c + a s);
// the inverse rotation passes -s.  Shared by the RoPE kernels and the
// attention kernels that rotate q on load, so that both round alike: the
// fused multiply-adds are spelled out, since the compiler's own contraction
// of a * c - b * s may pick either product depending on the surrounding code,
// and the fp32 results are materialised, since a 16-bit conversion that
// follows could otherwise be folded into a mixed-precision fma that rounds
// once (v_fma_mix*) where the other kernel rounds to fp32 first.
__device__ __forceinline__ void rope_pair(float a, float b, float c, float s, float& oa, float& ob) {
  oa = fmaf(a, c, -(b * s));
  ob = fmaf(b, c, a * s);
  asm volatile("" : "+v"(oa), "+v"(ob));
}

__host__ __device__ constexpr inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---- global -> LDS DMA -----------------------------------------------------
typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(lds_void*)p;
}

// One global_load_lds_dwordx4: lane i's 16 bytes at `g` land at LDS byte
// lds + 16 i (lds must be wave-uniform).  Issued through inline assembly on
// purpose: the compiler models a pending LDS DMA by turning every later
// LDS-read wait into lgkmcnt(0), which serialises fragment reads with the
// MFMAs they should overlap (the hardware counts the DMA in vmcnt only).
// Callers wait for it explicitly (wait_vmcnt before the barrier that
// publishes the tile); VMEM operations the compiler does not see can only
// make its own in-order vmcnt waits stricter.
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds)
               : "memory", "m0");
}

// dma16 with a wave-uniform 64-bit base and a 32-bit per-lane byte offset
// (the scalar-base addressing form: no 64-bit address arithmetic per lane).
__device__ __forceinline__ void dma16s(const void* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "s"(lds)
               : "memory", "m0");
}

// Same with 4 bytes per lane: lane i's dword lands at LDS byte lds + 4 i.
__device__ __forceinline__ void dma4(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(lds)
               : "memory", "m0");
}

// s_waitcnt with vmcnt = N and the other counters unconstrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Workgroup barrier for LDS hand-offs between wavefronts.  __syncthreads
// compiles to s_waitcnt vmcnt(0) lgkmcnt(0) + s_barrier, which also drains
// every global load in flight -- a prefetch DMA into another LDS stage
// included.  This one waits for the wavefront's own LDS operations only
// (its LDS writes are then visible, its LDS reads done), so prefetches stay
// in flight across it; a DMA'd tile is published as before, by wait_vmcnt
// ahead of the barrier.  The memory clobber keeps the compiler from moving
// LDS accesses across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int dtype_size(int dtype) { return dtype == kF32 ? 4 : 2; }

// Compute units of the current device (cached per device; 256 on MI355X),
// for launch-shape decisions.
inline int cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// ---- error plumbing (defined in capi.hip) ---------------------------------
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Returns 0, or records the pending launch error of the calling thread.
int check_launch(const char* what);

}  // namespace tri

// Error codes returned by every extern "C" entry point.
#define TRI_OK 0
#define TRI_EINVAL 1   // argument rejected by the library
#define TRI_ELAUNCH 2  // HIP runtime reported an error

// Dispatch a runtime dtype code to a storage type `T` inside `body`.
#define TRI_DISPATCH_FLOAT(dtype, T, ...)                                \
  do {                                                                   \
    switch (dtype) {                                                     \
      case ::tri::kF32: { typedef float T; __VA_ARGS__; } break;         \
      case ::tri::kF16: { typedef ::tri::f16_t T; __VA_ARGS__; } break;  \
      case ::tri::kBF16: { typedef ::tri::bf16_t T; __VA_ARGS__; } break; \
      default: return ::tri::fail(TRI_EINVAL, "unsupported dtype code %d", (int)(dtype)); \
    }                                                                    \
  } while (0)
