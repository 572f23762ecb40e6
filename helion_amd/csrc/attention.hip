// Scaled dot-product attention (causal or not, GQA, q_len != kv_len) for gfx950.
//
// Reference arithmetic: alkinun/helion tritium/ops/attention.py:69-141
// (forward: scale = head_dim^-0.5 applied to q.k, top-left causal mask
// q_pos >= kv_pos, online softmax, lse = m + ln l) and 399-629 (backward:
// P = exp(s - lse), dP = dO v^T, D_i = rowsum(P dP), dS = P (dP - D_i),
// dV = P^T dO, dQ = dS k * scale, dK = dS^T q * scale).
//
// bf16 / fp16 inputs with head_dim in {16, 32, 64, 128} run on the MFMA path
// (v_mfma_f32_32x32x16_{bf16,f16}, fp32 accumulation):
//
//  forward   a wavefront computes S^T = K Q^T for its 32 query rows against a
//            64-row K/V tile staged in LDS (K and V rows by DMA, XOR-swizzled),
//            so each lane owns ONE query column: the online-softmax max needs a
//            single lane^32 exchange and P^T feeds the next MFMA
//            (O^T = V^T P^T) straight from registers, V^T by transposing LDS
//            reads.  attn_fwd_v2: 4 wavefronts = 128 query rows per workgroup;
//            attn_fwd_pp (head_dim 128, large grids): 8 wavefronts in two
//            groups on opposite MFMA / softmax phases, two 256-row query tiles
//            per workgroup.
//  backward  (1) Q-parallel dQ kernel, which also writes delta = rowsum(dO * O);
//            (2) KV-parallel dK/dV kernel: wavefront pairs own 32 kv rows (K
//            or V fragments in registers), sweep the query tiles that can see
//            them in opposite phases, and accumulate dV^T and dK^T in registers
//            (GQA: all query heads of the group), written once in the output
//            dtype.  No atomics: results are bitwise deterministic.
//            With a dS workspace (head_dim 128, no RoPE): delta first, then
//            the dK/dV kernel storing every dS tile it forms (2 bytes per
//            visible pair), then dQ = dS K * scale from the stored tiles --
//            no second S and dP, at the price of the dS traffic.
//
// fp32 inputs (and head_dim outside the MFMA set, up to 1024) run on a SIMT
// path: one wavefront per row, exact fp32 arithmetic.
//
// Workgroup order is XCD-aware: the 8 XCDs receive workgroups round-robin, so
// block ids are remapped to give every XCD a contiguous range of
// (batch, head)s (their K/V stay in that XCD's L2), heaviest causal tiles
// first.
#include <math.h>

#include <atomic>
#include <mutex>
#include <type_traits>

#include "common.h"
#include "../../include/tritium_hip.h"

namespace tri {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int kXcds = 8;

template <typename T> struct Mfma;
template <> struct Mfma<bf16_t> {
  typedef bf16x8_t V;
  static __device__ __forceinline__ f32x16 mma(V a, V b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mfma<f16_t> {
  typedef f16x8_t V;
  static __device__ __forceinline__ f32x16 mma(V a, V b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

// 8 consecutive elements (16 bytes, 16-byte aligned).
template <typename T>
__device__ __forceinline__ typename Mfma<T>::V ld8(const T* p) {
  return *reinterpret_cast<const typename Mfma<T>::V*>(p);
}

// Elements p0[0..3] followed by p1[0..3] (two 8-byte aligned reads).
template <typename T>
__device__ __forceinline__ typename Mfma<T>::V ld4x2(const T* p0, const T* p1) {
  const uint2 a = *reinterpret_cast<const uint2*>(p0);
  const uint2 b = *reinterpret_cast<const uint2*>(p1);
  uint4 u;
  u.x = a.x; u.y = a.y; u.z = b.x; u.w = b.y;
  return __builtin_bit_cast(typename Mfma<T>::V, u);
}

template <typename T>
__device__ __forceinline__ typename Mfma<T>::V zero8() {
  return __builtin_bit_cast(typename Mfma<T>::V, make_uint4(0, 0, 0, 0));
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// Masks of a 32 x 32 MFMA accumulator whose element r lies at row offset
// c(r) = 8 (r / 4) + 4 g + r % 4 of its 32-row block (g = lane / 32).  The
// caller folds every lane-dependent term of the bound into one integer, so
// each element costs one compare against the constant 8 (r / 4) + r % 4 and
// one select (a per-element row index and two tests cost four VALU and two
// scalar ops).
// mask_above: element r -> -inf when c(r) - 4 g > lim.
__device__ __forceinline__ void mask_above(f32x16& s, int lim) {
#pragma unroll
  for (int r = 0; r < 16; ++r) s[r] = 8 * (r >> 2) + (r & 3) > lim ? -INFINITY : s[r];
}
// mask_outside: element r -> -inf unless lo <= c(r) - 4 g < hi (one
// unsigned compare of c - 4 g - lo against the span).
__device__ __forceinline__ void mask_outside(f32x16& s, int lo, int hi) {
  const uint32_t span = hi > lo ? (uint32_t)(hi - lo) : 0u;
#pragma unroll
  for (int r = 0; r < 16; ++r)
    s[r] = (uint32_t)(8 * (r >> 2) + (r & 3) - lo) >= span ? -INFINITY : s[r];
}

// Max of a value over lanes l and l ^ 32 without an LDS round trip
// (ds_bpermute waits on every outstanding LDS read): v_permlane32_swap hands
// each half-wave the other's copy.
__device__ __forceinline__ float xor32_max(float x) {
  const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                   false);
  return fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
}

// Scheduling fence: the compiler keeps every instruction on its side.
__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }

// Pin a loop-carried value to AGPRs (pin_agpr) or VGPRs (pin_vgpr) at the
// top of each iteration.  Without it the register allocator may home an
// MFMA accumulator in the other register file and copy it into and out of
// the MFMA's registers every iteration.  Emits no instruction.
template <typename X>
__device__ __forceinline__ void pin_agpr(X& x) { asm volatile("" : "+a"(x)); }
template <typename X>
__device__ __forceinline__ void pin_vgpr(X& x) { asm volatile("" : "+v"(x)); }

// Workgroup id -> work id such that each XCD (block id mod 8) processes a
// contiguous range of work ids.
__device__ __forceinline__ int xcd_remap(int bid, int n) {
  if (n % kXcds != 0) return bid;
  return (bid % kXcds) * (n / kXcds) + bid / kXcds;
}

// Work item w (from xcd_remap, n = n_slices * n_tiles items) -> its slice
// (batch * head) and tile rank.  Under a causal mask the tiles of a slice
// differ in length, rank 0 the longest.  When each XCD's range of w holds
// whole slices, the XCD takes its slices in groups of `group` and each
// group's tiles rank by rank (the longest of the group first), so the short
// tiles fill the tail instead of a slice's longest tile starting last: for 8
// tiles of 2 .. 16 steps on 64 workgroup slots a dispatch-order simulation
// gives 28 steps of makespan with the whole XCD as one group against 36
// slice by slice (ideal 27).  A small group keeps fewer slices' operands in
// the XCD's L2 at a time.  Otherwise slice by slice, longest tile first.
__device__ __forceinline__ void lpt_item(int w, int n, int n_slices, int n_tiles, bool causal,
                                         int group, int& slice, int& rank) {
  if (causal && n % kXcds == 0 && n_slices % kXcds == 0) {
    const int spx = n_slices / kXcds, per = n / kXcds;  // per = spx * n_tiles
    const int gs = min(group, spx);
    const int x = w / per, local = w - x * per;
    const int grp = local / (gs * n_tiles), within = local - grp * gs * n_tiles;
    const int gsz = min(gs, spx - grp * gs);  // the last group may be smaller
    rank = within / gsz;
    slice = x * spx + grp * gs + (within - rank * gsz);
  } else {
    slice = w / n_tiles;
    rank = w - slice * n_tiles;
  }
}

// RoPE applied to q as it is loaded (cos == nullptr: q is used as given).
// Non-interleaved halves: element i pairs with i + D/2 at table column i of
// the row's position; tables [max_pos, D/2] float32; the position of query
// row t of batch b is pos[b * Tq + t] (kind 1 int32, 2 int64) or t (kind 0).
struct RopeQ {
  const float* cos; const float* sin; const void* pos;
  int kind;
  int64_t max_pos;
};

struct FwdArgs {
  const void* q; const void* k; const void* v; void* o; float* lse;
  int64_t sq_b, sq_h, sq_s, sk_b, sk_h, sk_s, sv_b, sv_h, sv_s, so_b, so_h, so_s;
  int B, H, Hkv, Tq, Tkv, n_tiles, causal;
  float scale;  // head_dim ** -0.5
  RopeQ rope;
};

struct BwdArgs {
  const void* q; const void* k; const void* v; const void* o; const void* dout;
  const float* lse; float* delta; void* dq; void* dk; void* dv;
  int64_t sq_b, sq_h, sq_s, sk_b, sk_h, sk_s, sv_b, sv_h, sv_s, so_b, so_h, so_s;
  int64_t sdo_b, sdo_h, sdo_s, sdq_b, sdq_h, sdq_s, sdk_b, sdk_h, sdk_s, sdv_b, sdv_h, sdv_s;
  int B, H, Hkv, Tq, Tkv, n_tiles, causal;
  float scale;
  RopeQ rope;
  void* q_rot;  // with rope: [B, H, Tq, D] rotated q, written by the dQ kernel for dK/dV
  void* ds;       // stored-dS path: the dS chunks (ds_row below), else nullptr
  int64_t ds_bh;  // elements per (batch, query head) in ds
};

// Stored-dS layout.  Per (batch, query head) a run of ds_bh 16-bit elements
// holds 64 x 64 chunks: those of query tile qt (rows 64 qt ..) are the kv
// tiles j = 0 .. n_j(qt) - 1 in order from chunk ds_row(qt) on, with
// n_j = min(qt + 1, n_kvt) under the causal mask (kv row <= query row) and
// n_kvt without.  A chunk holds [64 kv rows][64 columns] as 16-byte granules
// (8 columns of a row): granule c of row r at element
// 2048 (r >> 5) + 512 (c & 3) + 8 (32 (c >> 2) + (r & 31)), i.e. in the
// order in which the dK/dV kernel's wavefront pair holds the tile (row
// r & 31 its lane's kv row, c >> 2 the lane half g, c & 3 the operand t), so
// each of its four 16-byte stores per lane writes 1 KiB contiguous; column
// 8 c + e holds query row 16 (c & 3) + 8 (e >> 2) + 4 (c >> 2) + (e & 3) of
// the tile.
__host__ __device__ __forceinline__ int64_t ds_row(int causal, int qt, int n_kvt) {
  if (!causal) return (int64_t)qt * n_kvt;
  if (qt <= n_kvt) return (int64_t)qt * (qt + 1) / 2;
  return (int64_t)n_kvt * (n_kvt + 1) / 2 + (int64_t)(qt - n_kvt) * n_kvt;
}

// Query row (within its tile) of chunk column c.
__device__ __forceinline__ int ds_col_row(int c) {
  const int gr = c >> 3, e = c & 7;
  return 16 * (gr & 3) + 8 * (e >> 2) + 4 * (gr >> 2) + (e & 3);
}

// Position of query row t of batch b under r, and whether the tables hold it.
__device__ __forceinline__ bool rope_position(const RopeQ& r, int b, int Tq, int t, int64_t& pos) {
  const int64_t token = (int64_t)b * Tq + t;
  pos = r.kind == 1 ? (int64_t)((const int32_t*)r.pos)[token]
                    : r.kind == 2 ? ((const int64_t*)r.pos)[token] : (int64_t)t;
  return pos >= 0 && pos < r.max_pos;
}

// Rotate a lane's q fragment in place: qf[st] holds elements 16 st + 8 g ..
// + 7 of one row, so the pairs (i, i + D/2) are qf[st][j], qf[st + KS/2][j].
// Rounded to T as the RoPE kernel rounds its output; NaN outside the tables.
template <typename T, int D>
__device__ __forceinline__ void rope_q_frag(typename Mfma<T>::V (&qf)[D / 16], const RopeQ& r,
                                            int64_t pos, bool valid, int g) {
  constexpr int H2 = D / 32, HALF = D / 2;
  const float nan = __builtin_nanf("");
#pragma unroll
  for (int st = 0; st < H2; ++st) {
    float c[8] = {}, s[8] = {};
    if (valid) {
      const float* cr = r.cos + pos * HALF + 16 * st + 8 * g;
      const float* sr = r.sin + pos * HALF + 16 * st + 8 * g;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        c[j] = cr[j];
        s[j] = sr[j];
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float oa, ob;
      rope_pair((float)qf[st][j], (float)qf[st + H2][j], c[j], s[j], oa, ob);
      qf[st][j] = (T)(valid ? oa : nan);
      qf[st + H2][j] = (T)(valid ? ob : nan);
    }
  }
}

// Transposed LDS tiles are [d][64] with no padding: the 8-byte unit u (4
// elements) of row d sits at slot u ^ tr_key(d).  A 32-lane 8-byte read of
// 32 consecutive rows at one u, and a write of rows 8 apart, both touch
// every bank pair once (tr_key is a bijection on any 16 even or odd rows).
__device__ __forceinline__ int tr_key(int d) { return ((d >> 1) ^ (d >> 3)) & 15; }
__device__ __forceinline__ int tr_off(int d, int u) { return d * 64 + ((u ^ tr_key(d)) << 2); }

// A ROWS x D tile of T (row stride `ld` elements in global memory, rows >=
// valid_rows read as zero), copied in two halves so that the global loads
// of the next tile are in flight while the current one is multiplied:
// fetch() issues the loads into registers (each thread 4 rows x 8 columns,
// four 16-byte loads), put_rm() writes the tile row-major (row stride RLD)
// and put_tr() transposed (a tr_off() tile, 8-byte writes).
template <typename T, int ROWS, int D>
struct TileRegs {
  static constexpr int CH = D / 8;
  static constexpr int ITEMS = (ROWS / 4) * CH;
  static constexpr int PER_THREAD = (ITEMS + 255) / 256;
  Pack<T, 8> v[PER_THREAD][4];

  __device__ __forceinline__ void fetch(const T* __restrict__ g, int64_t ld, int valid_rows) {
#pragma unroll
    for (int q = 0; q < PER_THREAD; ++q) {
      const int it = q * 256 + threadIdx.x;
      const int r4 = it / CH, cc = it % CH;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = r4 * 4 + i;
        if (it < ITEMS && r < valid_rows) {
          v[q][i] = *reinterpret_cast<const Pack<T, 8>*>(g + (int64_t)r * ld + cc * 8);
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) v[q][i].v[j] = (T)0.f;
        }
      }
    }
  }

  template <int RLD>
  __device__ __forceinline__ void put_rm(T* rm) const {
#pragma unroll
    for (int q = 0; q < PER_THREAD; ++q) {
      const int it = q * 256 + threadIdx.x;
      if (it >= ITEMS) continue;
      const int r4 = it / CH, cc = it % CH;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *reinterpret_cast<Pack<T, 8>*>(rm + (r4 * 4 + i) * RLD + cc * 8) = v[q][i];
    }
  }

  // Transposed copy into a tr_off() tile (ROWS must be 64).  A lane writes
  // its 8 rows in an order keyed on r4's parity, so the two halves of a
  // 32-lane write cycle land in opposite bank halves.
  __device__ __forceinline__ void put_tr(T* tr) const {
    static_assert(ROWS == 64, "transposed tiles are 64 wide");
#pragma unroll
    for (int q = 0; q < PER_THREAD; ++q) {
      const int it = q * 256 + threadIdx.x;
      if (it >= ITEMS) continue;
      const int r4 = it / CH, cc = it % CH;
      const bool odd = (r4 & 1) != 0;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        // row j = k ^ odd, selected between two compile-time register indices
        Pack<T, 4> col;
#pragma unroll
        for (int i = 0; i < 4; ++i) col.v[i] = odd ? v[q][i].v[k ^ 1] : v[q][i].v[k];
        *reinterpret_cast<Pack<T, 4>*>(tr + tr_off(cc * 8 + (k ^ (int)odd), r4)) = col;
      }
    }
  }
};

// Zero rows [D, DP) of a transposed LDS tile (head_dim < 32 pads to 32).
template <typename T, int D, int DP, int TLD>
__device__ __forceinline__ void zero_pad_rows(T* tr) {
  for (int i = threadIdx.x; i < (DP - D) * TLD; i += 256) tr[D * TLD + i] = (T)0.f;
}

// Store 4 consecutive values (one C-fragment quad) as 4 elements of T.
template <typename T>
__device__ __forceinline__ void store4(T* p, float a, float b, float c, float d) {
  Pack<T, 4> pk;
  pk.v[0] = (T)a; pk.v[1] = (T)b; pk.v[2] = (T)c; pk.v[3] = (T)d;
  *reinterpret_cast<Pack<T, 4>*>(p) = pk;
}

// ------------------------------------------------------------ MFMA forward --
constexpr int kFwdBM = 128;
constexpr int kFwdBN = 64;

template <typename T, int D>
__global__ void __launch_bounds__(256)
attn_fwd_mfma(FwdArgs a) {
  typedef Mfma<T> M;
  typedef typename M::V V;
  constexpr int KS = D / 16;
  constexpr int DP = D < 32 ? 32 : D;
  constexpr int MT = DP / 32;
  constexpr int KLD = D + 8;
  constexpr int VLD = kFwdBN;  // transposed V: tr_off() layout
  __shared__ __attribute__((aligned(16))) T K_sb[2][kFwdBN * KLD];
  __shared__ __attribute__((aligned(16))) T Vt_sb[2][DP * VLD];

  const int lane = threadIdx.x & 63, wave = wave_id();
  const int l32 = lane & 31, g = lane >> 5;
  const int w = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = w / a.n_tiles;
  const int qt = a.n_tiles - 1 - (w % a.n_tiles);
  const int b = bh / a.H, h = bh % a.H;
  const int hk = h / (a.H / a.Hkv);
  const T* qp = (const T*)a.q + b * a.sq_b + h * a.sq_h;
  const T* kp = (const T*)a.k + b * a.sk_b + hk * a.sk_h;
  const T* vp = (const T*)a.v + b * a.sv_b + hk * a.sv_h;
  T* op = (T*)a.o + b * a.so_b + h * a.so_h;
  const int q0 = qt * kFwdBM;
  const int qw0 = q0 + wave * 32;
  const int qrow = qw0 + l32;
  const bool qvalid = qrow < a.Tq;
  const float sl2 = a.scale * kLog2e;

  if (D < DP) {
    zero_pad_rows<T, D, DP, VLD>(Vt_sb[0]);
    zero_pad_rows<T, D, DP, VLD>(Vt_sb[1]);
  }

  V qf[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s)
    qf[s] = qvalid ? ld8(qp + (int64_t)qrow * a.sq_s + 16 * s + 8 * g) : zero8<T>();

  f32x16 o[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) o[mt] = zero16();
  float m = -INFINITY, l = 0.f;

  const int kv_end = a.causal ? min(a.Tkv, q0 + kFwdBM) : a.Tkv;
  // double-buffered: the loads of K/V tile i+1 are in flight during tile i
  TileRegs<T, kFwdBN, D> kr, vr;
  if (kv_end > 0) {
    kr.fetch(kp, a.sk_s, min(kFwdBN, a.Tkv));
    vr.fetch(vp, a.sv_s, min(kFwdBN, a.Tkv));
  }
  for (int kv0 = 0, it = 0; kv0 < kv_end; kv0 += kFwdBN, ++it) {
    T* K_s = K_sb[it & 1];
    T* Vt_s = Vt_sb[it & 1];
    kr.template put_rm<KLD>(K_s);
    vr.put_tr(Vt_s);
    __syncthreads();
    if (kv0 + kFwdBN < kv_end) {
      const int nxt = kv0 + kFwdBN;
      kr.fetch(kp + (int64_t)nxt * a.sk_s, a.sk_s, min(kFwdBN, a.Tkv - nxt));
      vr.fetch(vp + (int64_t)nxt * a.sv_s, a.sv_s, min(kFwdBN, a.Tkv - nxt));
    }

    f32x16 s[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      s[u] = zero16();
#pragma unroll
      for (int st = 0; st < KS; ++st) {
        const V kf = ld8(K_s + (32 * u + l32) * KLD + 16 * st + 8 * g);
        s[u] = M::mma(kf, qf[st], s[u]);
      }
    }
    // s[u][r] = S^T[kv0 + 32u + 8(r/4) + 4g + r%4][qrow]
    const bool need_mask = (kv0 + kFwdBN > a.Tkv) || (a.causal && kv0 + kFwdBN - 1 > qw0);
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float x = s[u][r] * sl2;
        if (need_mask) {
          const int kv = kv0 + 32 * u + 8 * (r >> 2) + 4 * g + (r & 3);
          if (kv >= a.Tkv || (a.causal && kv > qrow)) x = -INFINITY;
        }
        s[u][r] = x;
        mx = fmaxf(mx, x);
      }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = fast_exp2(m - m_use);
    m = m_new;
    float rs = 0.f;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = fast_exp2(s[u][r] - m_use);
        s[u][r] = p;
        rs += p;
      }
    }
    l = l * alpha + rs;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[mt][r] *= alpha;

#pragma unroll
    for (int t = 0; t < kFwdBN / 16; ++t) {
      V pb;
#pragma unroll
      for (int j = 0; j < 8; ++j) pb[j] = (T)s[t >> 1][8 * (t & 1) + j];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int row = 32 * mt + l32;
        o[mt] = M::mma(ld4x2<T>(Vt_s + tr_off(row, 4 * t + g), Vt_s + tr_off(row, 4 * t + 2 + g)),
                       pb, o[mt]);
      }
    }
  }

  const float lt = l + __shfl_xor(l, 32, 64);
  const float inv = lt > 0.f ? 1.0f / lt : 0.f;
  if (qvalid) {
    T* orow = op + (int64_t)qrow * a.so_s;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int d0 = 32 * mt + 8 * rr + 4 * g;
        if (d0 < D)
          store4<T>(orow + d0, o[mt][4 * rr] * inv, o[mt][4 * rr + 1] * inv,
                    o[mt][4 * rr + 2] * inv, o[mt][4 * rr + 3] * inv);
      }
    }
    if (g == 0) a.lse[(int64_t)bh * a.Tq + qrow] = (m + log2f(lt)) * kLn2;
  }
}

// ------------------------------- 64-row tiles in LDS, head_dim 64 and 128 --
// The head_dim 64/128 kernels stage 64-row tiles of K/V (forward, dQ) or
// Q/dO (dK/dV) in LDS by direct global->LDS DMA, row-major, double-buffered,
// and read them two ways: as MFMA A operands along rows (16-byte reads of 32 rows)
// and transposed (ds_read_b64_tr_b16: the A operand of X^T, m = column of
// X, k = 16 rows of X).  The 16-byte granule c of row r sits at slot
// c ^ key(r); key makes both reads bank-conflict free:
//   * 16 consecutive rows at one granule hit 16 distinct 16-byte bank groups
//     (256-byte rows: key is a bijection of r & 15; 128-byte rows: of
//     (r >> 1) & 7, rows of opposite parity already use opposite halves);
//   * 4 consecutive rows x 4 consecutive granules (one 32-lane cycle of a
//     transposing read) land in 16 distinct groups (bits 3:2 of the key,
//     bit 2 for 128-byte rows, differ between rows of one parity).
template <int D>
struct BTile {
  static_assert(D == 64 || D == 128 || D == 256, "head_dim");
  static constexpr int RB = 2 * D;              // bytes per row
  static constexpr int GR = RB / 16;            // granules per row
  static constexpr int BYTES = 64 * RB;         // one 64-row tile
  static constexpr int DMA_ROWS = 1024 / RB;    // rows per wave-wide DMA
  static constexpr int DMAS = BYTES / 1024;     // wave-wide DMAs per tile
  static __device__ __forceinline__ int key(int r) {
    if constexpr (GR >= 16) return ((r & 3) << 2) | ((r >> 2) & 3);
    else return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
  }
  static __device__ __forceinline__ int off(int r, int c) { return r * RB + ((c ^ key(r)) << 4); }
};

// DMA two 64-row tiles (x rows r0.. of x and y, rows clamped to n_rows - 1)
// into dst and dst + BYTES, spread over the WAVES wavefronts.
template <typename T, int D, int WAVES>
__device__ __forceinline__ void bt_dma2(char* dst, const T* x, int64_t sx, const T* y, int64_t sy,
                                        int r0, int n_rows) {
  typedef BTile<D> P;
  constexpr int PER = 2 * P::DMAS / WAVES;
  static_assert(PER * WAVES == 2 * P::DMAS, "DMA split");
  const int lane = threadIdx.x & 63, wave = wave_id();
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int grp = wave * PER + i;
    const bool second = grp >= P::DMAS;
    const int part = grp % P::DMAS;
    const int trow = part * P::DMA_ROWS + lane / P::GR;
    const int row = min(r0 + trow, n_rows - 1);
    const int c = (lane % P::GR) ^ P::key(trow);
    const T* src = (second ? y + (int64_t)row * sy : x + (int64_t)row * sx) + c * 8;
    dma16(src, __builtin_amdgcn_readfirstlane(lds_addr(dst + (second ? P::BYTES : 0) + part * 1024)));
  }
}

// bt_dma2 for the steady state: each lane's byte offsets from a tile's first
// row are computed once (init), a full tile then costs one scalar base per
// tensor and no per-lane address arithmetic; a tile that reaches past
// n_rows falls back to bt_dma2's clamped rows.
template <typename T, int D, int WAVES>
struct BtDma {
  typedef BTile<D> P;
  static constexpr int PER = 2 * P::DMAS / WAVES;
  uint32_t off[PER];
  bool fast;
  __device__ __forceinline__ void init(int64_t sx, int64_t sy) {
    const int lane = threadIdx.x & 63, wave = wave_id();
    fast = (int64_t)64 * (sx > sy ? sx : sy) * (int64_t)sizeof(T) < ((int64_t)1 << 31);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int grp = wave * PER + i;
      const int trow = (grp % P::DMAS) * P::DMA_ROWS + lane / P::GR;
      const int c = (lane % P::GR) ^ P::key(trow);
      off[i] = fast ? (uint32_t)((trow * (grp >= P::DMAS ? sy : sx) + c * 8) * (int64_t)sizeof(T)) : 0u;
    }
  }
  __device__ __forceinline__ void issue(char* dst, const T* x, int64_t sx, const T* y, int64_t sy,
                                        int r0, int n_rows) const {
    if (fast && r0 + 64 <= n_rows) {
      const int wave = wave_id();
      const T* bx = x + (int64_t)r0 * sx;
      const T* by = y + (int64_t)r0 * sy;
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int grp = wave * PER + i;
        const bool second = grp >= P::DMAS;
        dma16s(second ? by : bx, off[i],
               __builtin_amdgcn_readfirstlane(
                   lds_addr(dst + (second ? P::BYTES : 0) + (grp % P::DMAS) * 1024)));
      }
    } else {
      bt_dma2<T, D, WAVES>(dst, x, sx, y, sy, r0, n_rows);
    }
  }
};

// One 64-row tile (rows r0.. of x, clamped to n_rows - 1) by DMA, spread
// over WAVES wavefronts (wavefront index taken relative to wave0).  A full
// tile uses per-lane byte offsets computed once (init); a tile that reaches
// past n_rows recomputes them with the rows clamped, from a lane index the
// compiler cannot hoist out of the caller's loop (hoisted, that path's
// per-lane addresses would hold registers for the whole loop).
template <typename T, int D, int WAVES>
struct BtDma1 {
  typedef BTile<D> P;
  static constexpr int PER = P::DMAS / WAVES;
  static_assert(PER * WAVES == P::DMAS, "DMA split");
  uint32_t off[PER];
  int wv;
  bool fast;
  // byte offset of this lane's 16 bytes of DMA i from row r0, rows past
  // r0 + lim clamped to r0 + lim
  static __device__ __forceinline__ uint32_t offset(int lane, int wv, int i, int64_t sx, int lim) {
    const int trow = (wv * PER + i) * P::DMA_ROWS + lane / P::GR;
    const int c = (lane % P::GR) ^ P::key(trow);
    return (uint32_t)((min(trow, lim) * sx + c * 8) * (int64_t)sizeof(T));
  }
  __device__ __forceinline__ void init(int64_t sx, int wave0) {
    const int lane = threadIdx.x & 63;
    wv = wave_id() - wave0;
    fast = (int64_t)64 * sx * (int64_t)sizeof(T) < ((int64_t)1 << 31);
#pragma unroll
    for (int i = 0; i < PER; ++i) off[i] = fast ? offset(lane, wv, i, sx, 63) : 0u;
  }
  __device__ __forceinline__ void issue(char* dst, const T* x, int64_t sx, int r0, int n_rows) const {
    issue_at(dst, x + (int64_t)r0 * sx, sx, n_rows - r0);
  }
  // DMA i of this wavefront's share of a full tile from bx (init's offsets)
  __device__ __forceinline__ void issue_one(char* dst, const T* bx, int i) const {
    dma16s(bx, off[i], __builtin_amdgcn_readfirstlane(lds_addr(dst + (wv * PER + i) * 1024)));
  }
  // the tile whose first row is bx, with rows_left rows from bx on
  __device__ __forceinline__ void issue_at(char* dst, const T* bx, int64_t sx, int rows_left) const {
    if (fast && rows_left >= 64) {
#pragma unroll
      for (int i = 0; i < PER; ++i)
        dma16s(bx, off[i], __builtin_amdgcn_readfirstlane(lds_addr(dst + (wv * PER + i) * 1024)));
      return;
    }
    int lane;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lane));
    if (fast) {
#pragma unroll
      for (int i = 0; i < PER; ++i)
        dma16s(bx, offset(lane, wv, i, sx, rows_left - 1),
               __builtin_amdgcn_readfirstlane(lds_addr(dst + (wv * PER + i) * 1024)));
    } else {
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int trow = (wv * PER + i) * P::DMA_ROWS + lane / P::GR;
        const int row = min(trow, rows_left - 1);
        const int c = (lane % P::GR) ^ P::key(trow);
        dma16(bx + (int64_t)row * sx + c * 8,
              __builtin_amdgcn_readfirstlane(lds_addr(dst + (wv * PER + i) * 1024)));
      }
    }
  }
};

// A operand from rows rb + (lane & 31), columns 16 st + 8 (lane >> 5) .. +7.
template <typename T, int D>
__device__ __forceinline__ typename Mfma<T>::V bt_row(const char* tile, int rb, int st) {
  const int lane = threadIdx.x & 63;
  return *reinterpret_cast<const typename Mfma<T>::V*>(
      tile + BTile<D>::off(rb + (lane & 31), 2 * st + (lane >> 5)));
}

// A operand of X^T: m = column 32 mt + (lane & 31) of X, k = rows
// rb + 4g + {0..3} then rb + 8 + 4g + {0..3} (g = lane >> 5), rb a multiple
// of 16.  In each 16-lane group, source lane s addresses row (s >> 2) at
// column 4 (s & 3) of the group's 16 columns; the transposing read hands
// destination lane j the four rows of column j.
template <typename T, int D>
__device__ __forceinline__ typename Mfma<T>::V bt_tr(const char* tile, int rb, int mt) {
  typedef BTile<D> P;
  typedef short v4s __attribute__((ext_vector_type(4)));
  const int lane = threadIdx.x & 63;
  const int ts = lane & 15, th = (lane >> 4) & 1, g = lane >> 5;
  const int r1 = rb + 4 * g + (ts >> 2), r2 = r1 + 8;
  const int c = 4 * mt + 2 * th + ((ts & 3) >> 1);
  const int sub = (ts & 1) * 8;
  const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4s*)(lds_addr(tile + P::off(r1, c) + sub)));
  const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4s*)(lds_addr(tile + P::off(r2, c) + sub)));
  // one whole-vector cast: assembling the operand element by element from
  // the two results was miscompiled into broadcasts of their first element
  return __builtin_bit_cast(typename Mfma<T>::V,
                            __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// bt_row / bt_tr with the per-lane byte offsets computed once: the swizzle
// key of row r depends on r mod 16 only, so a row block rb (a multiple of
// 16) adds rb * RB, which the reads take as an immediate offset.  Without
// this the compiler keeps one address per distinct read (about 50 registers
// for D = 128) and spills them.
template <typename T, int D>
struct BtOffs {
  typedef BTile<D> P;
  typedef typename Mfma<T>::V V;
  static constexpr int KS = D / 16, MT = D / 32;
  uint32_t row[KS];    // bt_row(tile, 0, st)
  uint32_t tr[MT][2];  // bt_tr(tile, 0, mt): rows 4g + {0..3} and 8 + 4g + {0..3}
  __device__ __forceinline__ void init() {
    const int lane = threadIdx.x & 63;
    const int ts = lane & 15, th = (lane >> 4) & 1, g = lane >> 5;
#pragma unroll
    for (int st = 0; st < KS; ++st) row[st] = (uint32_t)P::off(lane & 31, 2 * st + g);
    const int r1 = 4 * g + (ts >> 2);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int c = 4 * mt + 2 * th + ((ts & 3) >> 1);
      tr[mt][0] = (uint32_t)(P::off(r1, c) + (ts & 1) * 8);
      tr[mt][1] = (uint32_t)(P::off(r1 + 8, c) + (ts & 1) * 8);
    }
  }
  __device__ __forceinline__ V rd_row(const char* tile, int rb, int st) const {
    return *reinterpret_cast<const V*>(tile + row[st] + rb * P::RB);
  }
  __device__ __forceinline__ V rd_tr(const char* tile, int rb, int mt) const {
    return rd_tr(tr_base(tile), rb, mt);
  }
  // The lane's transposing-read addresses in one tile (its 32-bit LDS
  // address plus the lane offsets), computed once per tile and made opaque:
  // the row block then goes into each read's immediate offset.  Left to
  // itself the compiler reassociates tile + (offset + row block), keeps the
  // 4 D / 16 sums of the last two in registers for the whole kernel and
  // spends one or two VALU ops per read rebasing them.
  struct TrBase {
    uint32_t v[MT][2];
  };
  __device__ __forceinline__ TrBase tr_base(const char* tile) const {
    TrBase r;
    const uint32_t t = lds_addr(tile);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        uint32_t x = t + tr[mt][k];
        asm("" : "+v"(x));
        r.v[mt][k] = x;
      }
    }
    return r;
  }
  __device__ __forceinline__ V rd_tr(const TrBase& bs, int rb, int mt) const {
    typedef short v4s __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) v4s lds_v4s;
    const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_v4s*)(uintptr_t)(bs.v[mt][0] + (uint32_t)(rb * P::RB)));
    const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_v4s*)(uintptr_t)(bs.v[mt][1] + (uint32_t)(rb * P::RB)));
    return __builtin_bit_cast(V, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  }
};



// ------------------------------------------------- MFMA forward, v2 (DMA) --
// One workgroup = 8 wavefronts = 256 query rows of one (batch, head); each
// wavefront owns 32 query rows (Q in registers) and computes, per 64-row K/V
// tile, S^T = K Q^T (K fragments: 16-byte LDS reads) and O^T += V^T P^T
// (V^T fragments: ds_read_b64_tr_b16 transposing reads of the row-major V
// tile, P^T straight from the S^T accumulators).  K and V tiles arrive by
// global_load_lds_dwordx4 into two LDS stages (the next tile streams in
// while the current one is multiplied); rows are XOR-swizzled per tile so
// that both the 16-byte K reads and the transposing V reads are conflict-free.
constexpr int kF2Waves = 4;
constexpr int kF2BM = 32 * kF2Waves;  // query rows per workgroup
constexpr int kF2BN = 64;             // K/V rows per tile
// MFMA operands in flight ahead of use (8 measured within 2% at head_dim 64)
constexpr int kRing = 4;
// K/V tiles in the LDS ring (3 measured 9% slower at the GPT block's shape)
constexpr int kF2Stages = 2;

template <typename T, int D>
__global__ void __launch_bounds__(64 * kF2Waves, D > 128 ? 1 : 8 / kF2Waves)  // 2 wavefronts per SIMD (1 at D = 256)
attn_fwd_v2(FwdArgs a) {
  typedef Mfma<T> M;
  typedef typename M::V V;
  typedef BTile<D> P;
  constexpr int KS = D / 16;
  constexpr int MT = D / 32;
  constexpr int STAGE = 2 * P::BYTES;  // K, V
  __shared__ __attribute__((aligned(1024))) char smem[kF2Stages * STAGE];

  const int lane = threadIdx.x & 63, wave = wave_id();
  const int l32 = lane & 31, g = lane >> 5;
  int bh, rank;
  lpt_item(xcd_remap(blockIdx.x, gridDim.x), gridDim.x, a.B * a.H, a.n_tiles, a.causal, a.B * a.H,
           bh, rank);
  const int qt = a.n_tiles - 1 - rank;  // rank 0: the most kv tiles
  const int b = bh / a.H, h = bh % a.H;
  const int hk = h / (a.H / a.Hkv);
  const T* qp = (const T*)a.q + b * a.sq_b + h * a.sq_h;
  const T* kp = (const T*)a.k + b * a.sk_b + hk * a.sk_h;
  const T* vp = (const T*)a.v + b * a.sv_b + hk * a.sv_h;
  T* op = (T*)a.o + b * a.so_b + h * a.so_h;
  const int q0 = qt * kF2BM;
  const int qw0 = q0 + wave * 32;
  const int qrow = qw0 + l32;
  const bool qvalid = qrow < a.Tq;
  const float sl2 = a.scale * kLog2e;

  V qf[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s)
    qf[s] = qvalid ? ld8(qp + (int64_t)qrow * a.sq_s + 16 * s + 8 * g) : zero8<T>();
  if (a.rope.cos != nullptr && qvalid) {
    int64_t pos;
    const bool ok = rope_position(a.rope, b, a.Tq, qrow, pos);
    rope_q_frag<T, D>(qf, a.rope, pos, ok, g);
  }

  f32x16 o[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) o[mt] = zero16();
  float m = -INFINITY, l = 0.f;
  float nm = 0.f;  // -m, or 0 while m is -inf (exp2 of a masked score is then 0)

  const int kv_end = a.causal ? min(a.Tkv, q0 + kF2BM) : a.Tkv;
  const int n_kv = (int)cdiv(kv_end, kF2BN);
  // kF2Stages-deep ring: tile it + kF2Stages - 1 streams in while tile it
  // is multiplied, so a tile has kF2Stages - 1 tiles of compute to land
  BtDma<T, D, kF2Waves> dma;
  dma.init(a.sk_s, a.sv_s);
#pragma unroll
  for (int j = 0; j < kF2Stages - 1; ++j)
    if (j < n_kv) dma.issue(smem + j * STAGE, kp, a.sk_s, vp, a.sv_s, j * kF2BN, a.Tkv);
  for (int it = 0; it < n_kv; ++it) {
    const int kv0 = it * kF2BN;
    // tile it has landed once at most the DMAs of the kF2Stages - 2 younger
    // tiles (issued in order, counted in order) are outstanding
    if (it + kF2Stages - 2 < n_kv) wait_vmcnt<(kF2Stages - 2) * BtDma<T, D, kF2Waves>::PER>();
    else wait_vmcnt<0>();
    __syncthreads();
    if (it + kF2Stages - 1 < n_kv)
      dma.issue(smem + ((it + kF2Stages - 1) % kF2Stages) * STAGE, kp, a.sk_s, vp, a.sv_s,
                kv0 + (kF2Stages - 1) * kF2BN, a.Tkv);
    const char* Ks = smem + (it % kF2Stages) * STAGE;
    const char* Vs = Ks + P::BYTES;
    if (a.causal && kv0 > qw0 + 31) continue;  // this wavefront's rows see none of the tile

    // S^T = K Q^T: MFMA i = 2 st + u (the two 32-row halves interleaved);
    // each K fragment is read kRing MFMAs before its use, and the fences
    // keep the compiler from pulling reads back next to their MFMAs
    auto kread = [&](int i) { return bt_row<T, D>(Ks, 32 * (i & 1), i >> 1); };
    f32x16 s[2] = {zero16(), zero16()};
    V kb[kRing];
#pragma unroll
    for (int i = 0; i < kRing; ++i) kb[i] = kread(i);
    // the MFMA chains run at raised wave priority, so the SIMD's arbiter
    // issues them ahead of the other wavefront's softmax (1.8% at head_dim 64)
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int i = 0; i < 2 * KS; ++i) {
      sched_fence();
      s[i & 1] = M::mma(kb[i % kRing], qf[i >> 1], s[i & 1]);
      if (i + kRing < 2 * KS) kb[i % kRing] = kread(i + kRing);
    }
    sched_fence();
    __builtin_amdgcn_s_setprio(0);
    // V^T fragments for the first O^T MFMAs, in flight during the softmax
    auto vread = [&](int i) { return bt_tr<T, D>(Vs, 16 * (i / MT), i % MT); };  // MFMA i = MT t + mt
    V vb[kRing];
#pragma unroll
    for (int i = 0; i < kRing; ++i) vb[i] = vread(i);
    // s[u][r] = S^T[kv0 + 32u + 8(r/4) + 4g + r%4][qrow]; masked when that
    // kv row is >= Tkv or (causal) > qrow
    const bool need_mask = (kv0 + kF2BN > a.Tkv) || (a.causal && kv0 + kF2BN - 1 > qw0);
    if (need_mask) {
      const int lim = (a.causal ? min(a.Tkv - 1, qrow) : a.Tkv - 1) - kv0 - 4 * g;
      mask_above(s[0], lim);
      mask_above(s[1], lim - 32);
    }
    // row max of the raw scores (the scale is positive), in log2 units
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[u][r]);
    mx = xor32_max(mx) * sl2;
    // Lazy rescaling: the reference point m of o and l only moves when some
    // row's max exceeds it by more than 8 (so every p <= 2^8); o / l and
    // lse = m + log2 l do not depend on which m is used.
    if (__builtin_amdgcn_ballot_w64(mx > m + 8.f) != 0) {
      const float m_new = fmaxf(m, mx);
      const float alpha = m_new == -INFINITY ? 1.f : fast_exp2(m - m_new);
      m = m_new;
      nm = m == -INFINITY ? 0.f : -m;
      l *= alpha;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[mt][r] *= alpha;
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = fast_exp2(fmaf(s[u][r], sl2, nm));
        s[u][r] = p;
        l += p;
      }
    }

    // O^T += V^T P^T: MFMA i = MT t + mt, kv rows 16t + 4g + {0..3} and
    // 16t + 8 + 4g + {0..3} (the P^T operand order of the S^T accumulator)
    V pb;
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int i = 0; i < (kF2BN / 16) * MT; ++i) {
      const int t = i / MT, mt = i % MT;
      sched_fence();
      if (mt == 0) {
#pragma unroll
        for (int j = 0; j < 8; ++j) pb[j] = (T)s[t >> 1][8 * (t & 1) + j];
      }
      o[mt] = M::mma(vb[i % kRing], pb, o[mt]);
      if (i + kRing < (kF2BN / 16) * MT) vb[i % kRing] = vread(i + kRing);
    }
    sched_fence();
    __builtin_amdgcn_s_setprio(0);
  }

  const float lt = l + __shfl_xor(l, 32, 64);
  const float inv = lt > 0.f ? 1.0f / lt : 0.f;
  if (qvalid) {
    T* orow = op + (int64_t)qrow * a.so_s;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int d0 = 32 * mt + 8 * rr + 4 * g;
        store4<T>(orow + d0, o[mt][4 * rr] * inv, o[mt][4 * rr + 1] * inv,
                  o[mt][4 * rr + 2] * inv, o[mt][4 * rr + 3] * inv);
      }
    }
    if (g == 0) a.lse[(int64_t)bh * a.Tq + qrow] = (m + log2f(lt)) * kLn2;
  }
}

// ------------------------------------------ MFMA forward, ping-pong (8 waves) --
// attn_fwd_v2's tile step is an MFMA stretch (S^T, then O^T) and a VALU
// stretch (mask, max, exp2, row sums, bf16 packing) of about the same length,
// and every wavefront of a workgroup runs the same stretch at the same time,
// so the MFMA pipe idles through the softmax.  Here one workgroup = 8
// wavefronts in two groups of 4; SIMD s hosts wavefront s of group 0 and
// wavefront s + 4 of group 1, and a half-step barrier keeps the groups in
// opposite phases: while one group multiplies (O^T += V_{j-1}^T P_{j-1}^T,
// then S_j^T = K_j Q^T), the other runs the softmax of its S_j^T.  P_j waits
// in registers (bf16 operands) for the group's next MFMA phase.  The
// multiplying group raises its wave priority so its MFMAs issue as soon as
// the pipe frees and the softmax fills the gaps.
//
// K/V tiles stream through a 4-stage LDS ring with two iterations of lead,
// issued from the softmax phases (group 0 the K tiles, group 1 the V tiles);
// the half-step barriers wait for LDS operations only, so the DMAs stay in
// flight across them.  Each wavefront owns 32 query rows; the two groups
// take alternate 32-row blocks so that near the causal diagonal both stop
// within a tile of each other.
constexpr int kPPWaves = 8;
constexpr int kPPBM = 32 * kPPWaves;  // query rows per workgroup
constexpr int kPPStages = 4;          // tile j + 2 streams in during iteration j

// MFMA phase of the ping-pong forward: O^T += V^T P^T over the previous
// tile (DPV; MFMA i = MT t + mt, t the 16-row slice of the tile), then
// S^T = K Q^T over the current one (DS; MFMA i = 2 st + u, u the 32-row
// half of the tile).  Operands stream through one kRing-deep ring that runs
// on from the first chain into the second; with DPV the caller has already
// read the first kRing V^T operands into it (before the phase barrier).
template <typename T, int D>
__device__ __forceinline__ void pp_mfma(bool dpv, bool ds, const char* Vs, const char* Ks,
                                        const BtOffs<T, D>& fo,
                                        const typename Mfma<T>::V (&qf)[D / 16],
                                        const typename Mfma<T>::V (&pb)[4],
                                        typename Mfma<T>::V (&rb)[kRing], f32x16 (&s)[2],
                                        f32x16 (&o)[D / 32]) {
  typedef Mfma<T> M;
  constexpr int MT = D / 32, NP = 4 * MT, NS = 2 * (D / 16);
  static_assert(NP % kRing == 0 && NS >= kRing, "ring");
  auto kread = [&](int i) { return fo.rd_row(Ks, 32 * (i & 1), i >> 1); };
  const typename BtOffs<T, D>::TrBase vb = fo.tr_base(Vs);
  auto vread = [&](int i) { return fo.rd_tr(vb, 16 * (i / MT), i % MT); };
  if (dpv) {
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      sched_fence();
      o[i % MT] = M::mma(rb[i % kRing], pb[i / MT], o[i % MT]);
      if (i + kRing < NP) rb[i % kRing] = vread(i + kRing);
      else if (ds) rb[i % kRing] = kread(i + kRing - NP);
    }
  } else if (ds) {
#pragma unroll
    for (int i = 0; i < kRing; ++i) rb[i] = kread(i);
  }
  if (ds) {
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      sched_fence();
      s[i & 1] = M::mma(rb[i % kRing], qf[i >> 1], i < 2 ? zero16() : s[i & 1]);
      if (i + kRing < NS) rb[i % kRing] = kread(i + kRing);
    }
  }
  sched_fence();
}

template <typename T, int D>
__global__ void __launch_bounds__(64 * kPPWaves, 1)  // 2 wavefronts per SIMD
attn_fwd_pp(FwdArgs a) {
  typedef Mfma<T> M;
  typedef typename M::V V;
  typedef BTile<D> P;
  typedef BtDma1<T, D, 4> Dma;  // group 0 streams the K tiles, group 1 the V tiles
  constexpr int KS = D / 16;
  constexpr int MT = D / 32;
  constexpr int STAGE = 2 * P::BYTES;  // K, V
  __shared__ __attribute__((aligned(1024))) char smem[kPPStages * STAGE];

  const int lane = threadIdx.x & 63, wave = wave_id();
  const int l32 = lane & 31, g = lane >> 5;
  const int grp = wave >> 2;
  const int rblk = 2 * (wave & 3) + grp;
  // a workgroup runs the query tiles n - 1 - i and i (n = a.n_tiles): with
  // the causal mask every workgroup then has the same number of K/V tiles
  const int n_items = (a.n_tiles + 1) / 2;
  const int w = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = w / n_items;
  const int pi = w % n_items;
  const int b = bh / a.H, h = bh % a.H;
  const int hk = h / (a.H / a.Hkv);
  const T* qp = (const T*)a.q + b * a.sq_b + h * a.sq_h;
  const T* kp = (const T*)a.k + b * a.sk_b + hk * a.sk_h;
  const T* vp = (const T*)a.v + b * a.sv_b + hk * a.sv_h;
  T* op = (T*)a.o + b * a.so_b + h * a.so_h;
  const float sl2 = a.scale * kLog2e;
  // tile t of this group's tensor -> its slot in stage t % kPPStages
  const T* xp = grp ? vp : kp;
  const int64_t sx = grp ? a.sv_s : a.sk_s;
  char* const slot0 = smem + grp * P::BYTES;
  Dma dma;
  dma.init(sx, 4 * grp);
  BtOffs<T, D> fo;
  fo.init();

  for (int item = 0; item < 2; ++item) {
    const int qt = item == 0 ? a.n_tiles - 1 - pi : pi;
    if (item == 1 && qt == a.n_tiles - 1 - pi) break;  // odd tile count: the middle tile runs alone
    const int q0 = qt * kPPBM;
    const int qw0 = q0 + 32 * rblk;
    const int qrow = qw0 + l32;
    const bool qvalid = qrow < a.Tq;

    V qf[KS];
#pragma unroll
    for (int st = 0; st < KS; ++st)
      qf[st] = qvalid ? ld8(qp + (int64_t)qrow * a.sq_s + 16 * st + 8 * g) : zero8<T>();
    if (a.rope.cos != nullptr && qvalid) {
      int64_t pos;
      const bool ok = rope_position(a.rope, b, a.Tq, qrow, pos);
      rope_q_frag<T, D>(qf, a.rope, pos, ok, g);
    }
    f32x16 o[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) o[mt] = zero16();
    V pb[4], rb[kRing];
    float m = -INFINITY, l = 0.f;

    // tiles of the workgroup, and of this wavefront (rows past Tq need none)
    const int kv_end = a.causal ? min(a.Tkv, q0 + kPPBM) : a.Tkv;
    const int n_kv = (int)cdiv(kv_end, 64);
    const int kv_end_w = qw0 >= a.Tq ? 0 : (a.causal ? min(a.Tkv, qw0 + 32) : a.Tkv);
    const int n_w = (int)cdiv(kv_end_w, 64);

    // (the previous item's last LDS reads finished before its final barrier)
    if (n_kv > 0) dma.issue(slot0, xp, sx, 0, a.Tkv);
    if (n_kv > 1) dma.issue(slot0 + STAGE, xp, sx, 64, a.Tkv);
    if (n_kv > 1) wait_vmcnt<Dma::PER>();
    else wait_vmcnt<0>();
    lds_barrier();

    // Every wavefront runs MFMA(0), softmax(0), MFMA(1), ... with a barrier
    // after each phase; group 1 starts one barrier later, so the two groups
    // are always in opposite phases: global half-step 2j + grp is this
    // group's MFMA(j) -- O^T += V_{j-1}^T P_{j-1}^T (1 <= j <= n_w), then
    // S_j^T = K_j Q^T (j < n_w) -- and 2j + 1 + grp its softmax(j).
    // The DMAs are issued in the softmax phases, whose VALU work hides them:
    // group 0 loads K_{j+2} in half-step 2j + 1 (K_{j-2}'s slot, last read
    // in 2j - 3) and has K_{j+1} landed by its end (first read in 2j + 2);
    // group 1 loads V_{j+2} in 2j + 2 (V_{j-2}'s slot, last read in 2j - 1)
    // and has V_{j+1} landed by its end (first read in 2j + 4).  V_j, read
    // ahead at the end of softmax(j), landed by the end of half-step 2j.
    if (grp == 1) lds_barrier();
    for (int j = 0; j <= n_kv; ++j) {
      f32x16 s[2];
      __builtin_amdgcn_s_setprio(1);
      pp_mfma<T, D>(j >= 1 && j <= n_w, j < n_w,
                    smem + ((j + kPPStages - 1) % kPPStages) * STAGE + P::BYTES,
                    smem + (j % kPPStages) * STAGE, fo, qf, pb, rb, s, o);
      __builtin_amdgcn_s_setprio(0);
      lds_barrier();

      if (j + 2 < n_kv) dma.issue(slot0 + ((j + 2) % kPPStages) * STAGE, xp, sx, (j + 2) * 64, a.Tkv);
      if (j < n_w) {
        const int kv0 = 64 * j;
        // s[u][r] = S^T[kv0 + 32u + 8(r/4) + 4g + r%4][qrow]
        if ((kv0 + 64 > a.Tkv) || (a.causal && kv0 + 63 > qw0)) {
          const int lim = (a.causal ? min(a.Tkv - 1, qrow) : a.Tkv - 1) - kv0 - 4 * g;
          mask_above(s[0], lim);
          mask_above(s[1], lim - 32);
        }
        // row max and (below) row sum as 4 independent chains: a lone
        // wavefront's VALU stream would otherwise wait out each dependent step
        float mq[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          mq[c] = fmaxf(s[c >> 1][8 * (c & 1)], s[c >> 1][8 * (c & 1) + 1]);
#pragma unroll
          for (int r = 2; r < 8; ++r) mq[c] = fmaxf(mq[c], s[c >> 1][8 * (c & 1) + r]);
        }
        float mx = fmaxf(fmaxf(mq[0], mq[1]), fmaxf(mq[2], mq[3]));
        // the other half of this query row's scores sit in lane ^ 32
        mx = xor32_max(mx) * sl2;
        // lazy rescaling, as in attn_fwd_v2: the reference point m moves
        // only when a row's max exceeds it by more than 8 (every p <= 2^8)
        if (__builtin_amdgcn_ballot_w64(mx > m + 8.f) != 0) {
          const float m_new = fmaxf(m, mx);
          const float alpha = m_new == -INFINITY ? 1.f : fast_exp2(m - m_new);
          m = m_new;
          l *= alpha;
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[mt][r] *= alpha;
        }
        const float nm = m == -INFINITY ? 0.f : -m;
        // P^T operands: slice t holds kv rows 16t + 4g + {0..3}, 16t + 8 + 4g + {0..3}
        float ls[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
#pragma unroll
          for (int jj = 0; jj < 8; ++jj) {
            const float p = fast_exp2(fmaf(s[t >> 1][8 * (t & 1) + jj], sl2, nm));
            ls[jj & 3] += p;
            pb[t][jj] = (T)p;
          }
        }
        l += (ls[0] + ls[1]) + (ls[2] + ls[3]);
        // first V^T operands of MFMA(j + 1), read ahead of its barrier
        const auto vn = fo.tr_base(smem + (j % kPPStages) * STAGE + P::BYTES);
#pragma unroll
        for (int i = 0; i < kRing; ++i) rb[i] = fo.rd_tr(vn, 16 * (i / MT), i % MT);
      }
      // publish tile j + 1 (tile j + 2's DMAs may stay in flight)
      if (j + 2 < n_kv) wait_vmcnt<Dma::PER>();
      else wait_vmcnt<0>();
      lds_barrier();
    }
    if (grp == 0) lds_barrier();

    const float lt = l + __shfl_xor(l, 32, 64);
    const float inv = lt > 0.f ? 1.0f / lt : 0.f;
    if (qvalid) {
      T* orow = op + (int64_t)qrow * a.so_s;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int d0 = 32 * mt + 8 * rr + 4 * g;
          store4<T>(orow + d0, o[mt][4 * rr] * inv, o[mt][4 * rr + 1] * inv,
                    o[mt][4 * rr + 2] * inv, o[mt][4 * rr + 3] * inv);
        }
      }
      if (g == 0) a.lse[(int64_t)bh * a.Tq + qrow] = (m + log2f(lt)) * kLn2;
    }
  }
}

// ------------------------------------------------------ backward: delta --
// delta[bh][q] = sum_d dO[q][d] * O[q][d] (fp32).  One wavefront per row.
template <typename T>
__global__ void __launch_bounds__(256)
attn_bwd_delta(BwdArgs a, int D) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t n_rows = (int64_t)a.B * a.H * a.Tq;
  if (row >= n_rows) return;
  const int q = (int)(row % a.Tq);
  const int64_t bh = row / a.Tq;
  const int b = (int)(bh / a.H), h = (int)(bh % a.H);
  const T* o = (const T*)a.o + b * a.so_b + h * a.so_h + (int64_t)q * a.so_s;
  const T* d = (const T*)a.dout + b * a.sdo_b + h * a.sdo_h + (int64_t)q * a.sdo_s;
  float s = 0.f;
  for (int i = lane; i < D; i += 64) s += to_f32(o[i]) * to_f32(d[i]);
  s = wave_sum(s);
  if (lane == 0) a.delta[row] = s;
}

// ------------------------------------------------- MFMA backward: dK, dV --
constexpr int kDkvBN = 128;  // kv rows per workgroup (32 per wavefront)
constexpr int kDkvBM = 64;   // query rows per step

template <typename T, int D>
__global__ void __launch_bounds__(256)
attn_bwd_dkdv_mfma(BwdArgs a) {
  typedef Mfma<T> M;
  typedef typename M::V V;
  constexpr int KS = D / 16;
  constexpr int DP = D < 32 ? 32 : D;
  constexpr int MT = DP / 32;
  constexpr int QLD = D + 8;
  constexpr int TLD = kDkvBM;  // transposed Q, dO: tr_off() layout
  __shared__ __attribute__((aligned(16))) T Q_sb[2][kDkvBM * QLD];
  __shared__ __attribute__((aligned(16))) T dO_sb[2][kDkvBM * QLD];
  __shared__ __attribute__((aligned(16))) T Qt_sb[2][DP * TLD];
  __shared__ __attribute__((aligned(16))) T dOt_sb[2][DP * TLD];
  __shared__ float lse_sb[2][kDkvBM], delta_sb[2][kDkvBM];

  const int lane = threadIdx.x & 63, wave = wave_id();
  const int l32 = lane & 31, g = lane >> 5;
  const int w = xcd_remap(blockIdx.x, gridDim.x);
  const int bhk = w / a.n_tiles;
  const int kt = a.n_tiles - 1 - (w % a.n_tiles);  // heaviest (fewest visible queries) last
  const int b = bhk / a.Hkv, hk = bhk % a.Hkv;
  const int group = a.H / a.Hkv;
  const int kv0 = kt * kDkvBN;
  const int kvw = kv0 + wave * 32 + l32;  // this lane's kv row (MFMA column)
  const bool kvvalid = kvw < a.Tkv;
  const T* kp = (const T*)a.k + b * a.sk_b + hk * a.sk_h;
  const T* vp = (const T*)a.v + b * a.sv_b + hk * a.sv_h;
  const float sl2 = a.scale * kLog2e;

  if (D < DP) {
#pragma unroll
    for (int b2 = 0; b2 < 2; ++b2) {
      zero_pad_rows<T, D, DP, TLD>(Qt_sb[b2]);
      zero_pad_rows<T, D, DP, TLD>(dOt_sb[b2]);
    }
  }

  V kf[KS], vf[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    kf[s] = kvvalid ? ld8(kp + (int64_t)kvw * a.sk_s + 16 * s + 8 * g) : zero8<T>();
    vf[s] = kvvalid ? ld8(vp + (int64_t)kvw * a.sv_s + 16 * s + 8 * g) : zero8<T>();
  }
  f32x16 dv[MT], dk[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    dv[mt] = zero16();
    dk[mt] = zero16();
  }

  const int q_begin = a.causal ? (kv0 / kDkvBM) * kDkvBM : 0;
  const int n_q = a.Tq > q_begin ? (int)cdiv(a.Tq - q_begin, kDkvBM) : 0;
  const int n_steps = n_q * group;  // (query head of the group, query tile) pairs
  // double-buffered: the loads of step i+1 are in flight during step i
  TileRegs<T, kDkvBM, D> q_regs, do_regs;
  float lse_r = INFINITY, del_r = 0.f;
  auto fetch = [&](int step) {
    const int hq = hk * group + step / n_q;
    const int q0 = q_begin + (step % n_q) * kDkvBM;
    const int valid = min(kDkvBM, a.Tq - q0);
    const T* qp = (const T*)a.q + b * a.sq_b + hq * a.sq_h + (int64_t)q0 * a.sq_s;
    const T* dop = (const T*)a.dout + b * a.sdo_b + hq * a.sdo_h + (int64_t)q0 * a.sdo_s;
    q_regs.fetch(qp, a.sq_s, valid);
    do_regs.fetch(dop, a.sdo_s, valid);
    if (threadIdx.x < kDkvBM) {
      const int qq = q0 + threadIdx.x;
      const int64_t row = ((int64_t)b * a.H + hq) * a.Tq + qq;
      lse_r = qq < a.Tq ? a.lse[row] * kLog2e : INFINITY;
      del_r = qq < a.Tq ? a.delta[row] : 0.f;
    }
  };
  if (n_steps > 0) fetch(0);
  for (int step = 0; step < n_steps; ++step) {
    const int q0 = q_begin + (step % n_q) * kDkvBM;
    const int buf = step & 1;
    T* Q_s = Q_sb[buf];
    T* dO_s = dO_sb[buf];
    T* Qt_s = Qt_sb[buf];
    T* dOt_s = dOt_sb[buf];
    float* lse_s = lse_sb[buf];
    float* delta_s = delta_sb[buf];
    {
      q_regs.template put_rm<QLD>(Q_s);
      q_regs.put_tr(Qt_s);
      do_regs.template put_rm<QLD>(dO_s);
      do_regs.put_tr(dOt_s);
      if (threadIdx.x < kDkvBM) {
        lse_s[threadIdx.x] = lse_r;
        delta_s[threadIdx.x] = del_r;
      }
      __syncthreads();
      if (step + 1 < n_steps) fetch(step + 1);
      if (a.causal && q0 + kDkvBM - 1 < kv0 + wave * 32) continue;  // wave fully masked

#pragma unroll
      for (int mq = 0; mq < kDkvBM / 32; ++mq) {
        f32x16 s = zero16(), dp = zero16();
#pragma unroll
        for (int st = 0; st < KS; ++st) {
          const V qa = ld8(Q_s + (32 * mq + l32) * QLD + 16 * st + 8 * g);
          s = M::mma(qa, kf[st], s);
          const V da = ld8(dO_s + (32 * mq + l32) * QLD + 16 * st + 8 * g);
          dp = M::mma(da, vf[st], dp);
        }
        // s[r] = S[q0 + 32mq + 8(r/4) + 4g + r%4][kvw]
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int qi = 32 * mq + 8 * (r >> 2) + 4 * g + (r & 3);
          float p = fast_exp2(s[r] * sl2 - lse_s[qi]);
          if (!kvvalid || (a.causal && kvw > q0 + qi)) p = 0.f;
          s[r] = p;
          dp[r] = p * (dp[r] - delta_s[qi]);
        }
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          V pb, db;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            pb[j] = (T)s[8 * t + j];
            db[j] = (T)dp[8 * t + j];
          }
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const int row = 32 * mt + l32, u = 8 * mq + 4 * t + g;
            dv[mt] = M::mma(ld4x2<T>(dOt_s + tr_off(row, u), dOt_s + tr_off(row, u + 2)), pb,
                            dv[mt]);
            dk[mt] = M::mma(ld4x2<T>(Qt_s + tr_off(row, u), Qt_s + tr_off(row, u + 2)), db,
                            dk[mt]);
          }
        }
      }
    }
  }

  if (kvvalid) {
    T* dkr = (T*)a.dk + b * a.sdk_b + hk * a.sdk_h + (int64_t)kvw * a.sdk_s;
    T* dvr = (T*)a.dv + b * a.sdv_b + hk * a.sdv_h + (int64_t)kvw * a.sdv_s;
    const float sc = a.scale;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int d0 = 32 * mt + 8 * rr + 4 * g;
        if (d0 < D) {
          store4<T>(dkr + d0, dk[mt][4 * rr] * sc, dk[mt][4 * rr + 1] * sc,
                    dk[mt][4 * rr + 2] * sc, dk[mt][4 * rr + 3] * sc);
          store4<T>(dvr + d0, dv[mt][4 * rr], dv[mt][4 * rr + 1], dv[mt][4 * rr + 2],
                    dv[mt][4 * rr + 3]);
        }
      }
    }
  }
}

// ----------------------------------------------------- MFMA backward: dQ --
constexpr int kDqBM = 128;  // query rows per workgroup (32 per wavefront)
constexpr int kDqBN = 64;   // kv rows per step

template <typename T, int D>
__global__ void __launch_bounds__(256)
attn_bwd_dq_mfma(BwdArgs a) {
  typedef Mfma<T> M;
  typedef typename M::V V;
  constexpr int KS = D / 16;
  constexpr int DP = D < 32 ? 32 : D;
  constexpr int MT = DP / 32;
  constexpr int KLD = D + 8;
  constexpr int TLD = kDqBN;  // transposed K: tr_off() layout
  __shared__ __attribute__((aligned(16))) T K_sb[2][kDqBN * KLD];
  __shared__ __attribute__((aligned(16))) T V_sb[2][kDqBN * KLD];
  __shared__ __attribute__((aligned(16))) T Kt_sb[2][DP * TLD];

  const int lane = threadIdx.x & 63, wave = wave_id();
  const int l32 = lane & 31, g = lane >> 5;
  const int w = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = w / a.n_tiles;
  const int qt = a.n_tiles - 1 - (w % a.n_tiles);
  const int b = bh / a.H, h = bh % a.H;
  const int hk = h / (a.H / a.Hkv);
  const T* qp = (const T*)a.q + b * a.sq_b + h * a.sq_h;
  const T* dop = (const T*)a.dout + b * a.sdo_b + h * a.sdo_h;
  const T* kp = (const T*)a.k + b * a.sk_b + hk * a.sk_h;
  const T* vp = (const T*)a.v + b * a.sv_b + hk * a.sv_h;
  const int q0 = qt * kDqBM;
  const int qw0 = q0 + wave * 32;
  const int qrow = qw0 + l32;
  const bool qvalid = qrow < a.Tq;
  const float sl2 = a.scale * kLog2e;

  if (D < DP) {
    zero_pad_rows<T, D, DP, TLD>(Kt_sb[0]);
    zero_pad_rows<T, D, DP, TLD>(Kt_sb[1]);
  }

  V qf[KS], df[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    qf[s] = qvalid ? ld8(qp + (int64_t)qrow * a.sq_s + 16 * s + 8 * g) : zero8<T>();
    df[s] = qvalid ? ld8(dop + (int64_t)qrow * a.sdo_s + 16 * s + 8 * g) : zero8<T>();
  }
  const float lse2 = qvalid ? a.lse[(int64_t)bh * a.Tq + qrow] * kLog2e : INFINITY;
  const float dl = qvalid ? a.delta[(int64_t)bh * a.Tq + qrow] : 0.f;

  f32x16 dq[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) dq[mt] = zero16();

  const int kv_end = a.causal ? min(a.Tkv, q0 + kDqBM) : a.Tkv;
  // double-buffered: the loads of K/V tile i+1 are in flight during tile i
  TileRegs<T, kDqBN, D> k_regs, v_regs;
  if (kv_end > 0) {
    k_regs.fetch(kp, a.sk_s, min(kDqBN, a.Tkv));
    v_regs.fetch(vp, a.sv_s, min(kDqBN, a.Tkv));
  }
  for (int kv0 = 0, it = 0; kv0 < kv_end; kv0 += kDqBN, ++it) {
    T* K_s = K_sb[it & 1];
    T* V_s = V_sb[it & 1];
    T* Kt_s = Kt_sb[it & 1];
    k_regs.template put_rm<KLD>(K_s);
    k_regs.put_tr(Kt_s);
    v_regs.template put_rm<KLD>(V_s);
    __syncthreads();
    if (kv0 + kDqBN < kv_end) {
      const int nxt = kv0 + kDqBN;
      k_regs.fetch(kp + (int64_t)nxt * a.sk_s, a.sk_s, min(kDqBN, a.Tkv - nxt));
      v_regs.fetch(vp + (int64_t)nxt * a.sv_s, a.sv_s, min(kDqBN, a.Tkv - nxt));
    }
    if (a.causal && kv0 > qw0 + 31) continue;  // wave fully masked

    f32x16 ds[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      f32x16 s = zero16(), dp = zero16();
#pragma unroll
      for (int st = 0; st < KS; ++st) {
        s = M::mma(ld8(K_s + (32 * u + l32) * KLD + 16 * st + 8 * g), qf[st], s);
        dp = M::mma(ld8(V_s + (32 * u + l32) * KLD + 16 * st + 8 * g), df[st], dp);
      }
      // s[r] = S^T[kv0 + 32u + 8(r/4) + 4g + r%4][qrow]
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kv = kv0 + 32 * u + 8 * (r >> 2) + 4 * g + (r & 3);
        float p = fast_exp2(s[r] * sl2 - lse2);
        if (kv >= a.Tkv || (a.causal && kv > qrow)) p = 0.f;
        ds[u][r] = p * (dp[r] - dl);
      }
    }
#pragma unroll
    for (int t = 0; t < kDqBN / 16; ++t) {
      V db;
#pragma unroll
      for (int j = 0; j < 8; ++j) db[j] = (T)ds[t >> 1][8 * (t & 1) + j];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int row = 32 * mt + l32;
        dq[mt] = M::mma(ld4x2<T>(Kt_s + tr_off(row, 4 * t + g), Kt_s + tr_off(row, 4 * t + 2 + g)),
                        db, dq[mt]);
      }
    }
  }

  if (qvalid) {
    T* dqr = (T*)a.dq + b * a.sdq_b + h * a.sdq_h + (int64_t)qrow * a.sdq_s;
    const float sc = a.scale;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int d0 = 32 * mt + 8 * rr + 4 * g;
        if (d0 < D)
          store4<T>(dqr + d0, dq[mt][4 * rr] * sc, dq[mt][4 * rr + 1] * sc,
                    dq[mt][4 * rr + 2] * sc, dq[mt][4 * rr + 3] * sc);
      }
    }
  }
}


// dK, dV: a workgroup owns 32 * WAVES kv rows of one (batch, kv head), a
// wavefront 32 of them (K, V fragments in registers, lane = kv row), and
// sweeps the 64-row query tiles of every query head of the GQA group that
// can see them: S = Q K^T and dP = dO V^T from row reads of the Q / dO
// tiles, dV^T += dO^T P and dK^T += Q^T dS from transposing reads.
template <typename T, int D, int WAVES, int PASS = 0>
__global__ void __launch_bounds__(64 * WAVES, D == 64 ? 8 / WAVES : 1)
attn_bwd_dkdv_v2(BwdArgs a) {
  // PASS 0: dK and dV; 1: dV alone; 2: dK alone (head_dim 256, where the K
  // and V fragments and both accumulators of 32 kv rows would not fit one
  // wavefront's 512 registers: two launches, S formed in each)
  constexpr bool DO_DV = PASS != 2, DO_DK = PASS != 1;
  typedef Mfma<T> M;
  typedef typename M::V V;
  typedef BTile<D> P;
  constexpr int KS = D / 16;
  constexpr int MT = D / 32;
  constexpr int BN = 32 * WAVES;
  constexpr int STAGE = 2 * P::BYTES + 512;  // Q, dO, lse[64], delta[64]
  static_assert(WAVES >= 2 && BN % 64 == 0, "waves");
  __shared__ __attribute__((aligned(1024))) char smem[2 * STAGE];

  const int lane = threadIdx.x & 63, wave = wave_id();
  const int l32 = lane & 31, g = lane >> 5;
  int bhk, kt;  // kt = 0 sees the most queries: heaviest first
  lpt_item(xcd_remap(blockIdx.x, gridDim.x), gridDim.x, a.B * a.Hkv, a.n_tiles, a.causal,
           a.B * a.Hkv, bhk, kt);
  const int b = bhk / a.Hkv, hk = bhk % a.Hkv;
  const int group = a.H / a.Hkv;
  const int kv0 = kt * BN;
  const int kvb = kv0 + wave * 32;
  const int kvw = kvb + l32;  // this lane's kv row (MFMA column)
  const bool kvvalid = kvw < a.Tkv;
  const T* kp = (const T*)a.k + b * a.sk_b + hk * a.sk_h;
  const T* vp = (const T*)a.v + b * a.sv_b + hk * a.sv_h;
  const float sl2 = a.scale * kLog2e;

  V kf[KS], vf[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    kf[s] = kvvalid ? ld8(kp + (int64_t)kvw * a.sk_s + 16 * s + 8 * g) : zero8<T>();
    vf[s] = kvvalid && DO_DK ? ld8(vp + (int64_t)kvw * a.sv_s + 16 * s + 8 * g) : zero8<T>();
  }
  f32x16 dv[MT], dk[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    dv[mt] = zero16();
    dk[mt] = zero16();
  }

  const int q_begin = a.causal ? kv0 : 0;  // top-left causal: rows < kv0 see none
  const int n_q = a.Tq > q_begin ? (int)cdiv(a.Tq - q_begin, 64) : 0;
  const int n_steps = n_q * group;  // (query head of the group, query tile) pairs
  BtDma<T, D, WAVES> dma;
  dma.init(a.sq_s, a.sdo_s);
  auto issue = [&](int step, char* stage) {
    const int hq = hk * group + step / n_q;
    const int q0 = q_begin + (step % n_q) * 64;
    const T* qp = (const T*)a.q + b * a.sq_b + hq * a.sq_h;
    const T* dop = (const T*)a.dout + b * a.sdo_b + hq * a.sdo_h;
    dma.issue(stage, qp, a.sq_s, dop, a.sdo_s, q0, a.Tq);
    const int64_t row = ((int64_t)b * a.H + hq) * a.Tq + min(q0 + lane, a.Tq - 1);
    if (wave == 0) dma4(a.lse + row, __builtin_amdgcn_readfirstlane(lds_addr(stage + 2 * P::BYTES)));
    if (wave == 1)
      dma4(a.delta + row, __builtin_amdgcn_readfirstlane(lds_addr(stage + 2 * P::BYTES + 256)));
  };
  if (n_steps > 0) issue(0, smem);
  for (int step = 0; step < n_steps; ++step) {
    // 4 wavefronts: 512 registers, accumulators and K/V fragments in AGPRs
    // (MFMA operands), VGPRs left to the softmax; 8 wavefronts: 256, VGPRs
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if constexpr (WAVES <= 4 && D != 64) {
        if constexpr (DO_DV) pin_agpr(dv[mt]);
        if constexpr (DO_DK) pin_agpr(dk[mt]);
      } else {
        if constexpr (DO_DV) pin_vgpr(dv[mt]);
        if constexpr (DO_DK) pin_vgpr(dk[mt]);
      }
    }
    if constexpr (WAVES <= 4 && D != 64) {
#pragma unroll
      for (int st = 0; st < KS; ++st) {
        pin_agpr(kf[st]);
        if constexpr (DO_DK) pin_agpr(vf[st]);
      }
    }
    wait_vmcnt<0>();
    // wavefront 0 DMA'd this stage's lse and has just waited for it: it turns
    // the 64 values into log2 units before the barrier publishes the stage
    // (one multiply per query row instead of one per score)
    if (wave == 0) {
      float* l2 = reinterpret_cast<float*>(smem + (step & 1) * STAGE + 2 * P::BYTES);
      l2[lane] *= kLog2e;
    }
    __syncthreads();
    if (step + 1 < n_steps) issue(step + 1, smem + ((step + 1) & 1) * STAGE);
    const int q0 = q_begin + (step % n_q) * 64;
    if (a.causal && q0 + 63 < kvb) continue;  // this wavefront's kv rows see none of the tile
    const char* Qs = smem + (step & 1) * STAGE;
    const char* dOs = Qs + P::BYTES;
    const float* lse_s = reinterpret_cast<const float*>(Qs + 2 * P::BYTES);
    const float* del_s = lse_s + 64;
    const bool need_mask = (a.causal && q0 < kvb + 31) || q0 + 64 > a.Tq;

#pragma unroll
    for (int mq = 0; mq < 2; ++mq) {
      f32x16 s = zero16(), dp = zero16();
      // MFMA chains at raised wave priority (5.5% at head_dim 64; the dQ
      // kernel, measured the same way, did not gain and runs without)
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int st = 0; st < KS; ++st) {
        s = M::mma(bt_row<T, D>(Qs, 32 * mq, st), kf[st], s);
        if constexpr (DO_DK) dp = M::mma(bt_row<T, D>(dOs, 32 * mq, st), vf[st], dp);
      }
      __builtin_amdgcn_s_setprio(0);
      // phases are fenced so that no more than one phase's LDS fragments
      // are live at a time (the wavefront's registers hold K, V, dK, dV)
      // s[r] = S[q0 + 32mq + 8(r/4) + 4g + r%4][kvw]; masked scores -> -inf (p = 0):
      // query rows >= Tq or (causal) < kvw
      if (need_mask) {
        const int base = q0 + 32 * mq + 4 * g;
        mask_outside(s, a.causal ? kvw - base : -64, a.Tq - base);
      }
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int qi = 32 * mq + 8 * rr + 4 * g;
        const float4 L = *reinterpret_cast<const float4*>(lse_s + qi);
        const float4 Dl = *reinterpret_cast<const float4*>(del_s + qi);
        const float lv[4] = {L.x, L.y, L.z, L.w};  // log2 units
        const float dlv[4] = {Dl.x, Dl.y, Dl.z, Dl.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = 4 * rr + j;
          const float p = fast_exp2(fmaf(s[r], sl2, -lv[j]));
          s[r] = p;
          dp[r] = p * (dp[r] - dlv[j]);
        }
      }
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        V pb, db;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          pb[j] = (T)s[8 * t + j];
          db[j] = (T)dp[8 * t + j];
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          if constexpr (DO_DV) dv[mt] = M::mma(bt_tr<T, D>(dOs, 32 * mq + 16 * t, mt), pb, dv[mt]);
          if constexpr (DO_DK) dk[mt] = M::mma(bt_tr<T, D>(Qs, 32 * mq + 16 * t, mt), db, dk[mt]);
        }
      }
      __builtin_amdgcn_s_setprio(0);
    }
  }

  if (kvvalid) {
    T* dkr = (T*)a.dk + b * a.sdk_b + hk * a.sdk_h + (int64_t)kvw * a.sdk_s;
    T* dvr = (T*)a.dv + b * a.sdv_b + hk * a.sdv_h + (int64_t)kvw * a.sdv_s;
    const float sc = a.scale;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int d0 = 32 * mt + 8 * rr + 4 * g;
        if constexpr (DO_DK)
          store4<T>(dkr + d0, dk[mt][4 * rr] * sc, dk[mt][4 * rr + 1] * sc,
                    dk[mt][4 * rr + 2] * sc, dk[mt][4 * rr + 3] * sc);
        if constexpr (DO_DV)
          store4<T>(dvr + d0, dv[mt][4 * rr], dv[mt][4 * rr + 1], dv[mt][4 * rr + 2],
                    dv[mt][4 * rr + 3]);
      }
    }
  }
}

// dK, dV with wavefront pairs: a workgroup owns 128 kv rows of one
// (batch, kv head); wavefronts p and p + 4 (same SIMD) share kv rows
// 32p .. 32p + 31, role A (p: K fragments, dV accumulators) and role B
// (p + 4: V fragments, dK accumulators) -- one set of fragments and
// accumulators each, so two wavefronts fit per SIMD -- in opposite phases,
// so that one's VALU work runs under the other's MFMAs.  With tile s the
// s-th (query head, 64-row query tile) step, half-step 2s and 2s + 1 are
//   2s      A: dV^T += dO_{s-1}^T P_{s-1};  S_s = Q_s K^T          (MFMA)
//           B: dS_{s-1} = P_{s-1} (dP_{s-1} - D), P from A via LDS  (VALU)
//   2s + 1  A: P_s = exp(S_s * scale - lse), to LDS and registers  (VALU)
//           B: dK^T += Q_{s-1}^T dS_{s-1};  dP_s = dO_s V^T        (MFMA)
// Tiles stream through a 3-stage LDS ring, each role loading from its VALU
// phases: B loads Q, lse and D of tile s + 1 in half-step 2s (the stage of
// tile s - 2, last read in 2s - 1) and has them landed by the end of 2s + 1
// (Q first read in 2s + 2); A loads dO of tile s + 1 in 2s + 1 and has it
// landed by the end of 2s + 2 (first read in 2s + 3).
// DS: role B also stores each dS tile (cast to T, as the dK MFMAs take it)
// in the stored-dS layout, for attn_bwd_dq_ds; zero in kv rows >= Tkv.
constexpr int kPairWaves = 8;
constexpr int kPairBN = 128;
constexpr int kDkvPPStages = 3;
constexpr int kDkvRing = 8;  // MFMA operands in flight ahead of use

template <int D>
struct PairLds {
  static constexpr int STAGE = 2 * BTile<D>::BYTES + 512;  // Q, dO, lse[64], delta[64]
  static constexpr int XCH = 2 * 4 * 64 * 16;  // per pair: 2 query halves x [4][64 lanes][4 fp32]
};

// The work of one (batch * kv head, kv tile) item; smem and xch_all are the
// workgroup's LDS (PairLds sizes).
template <typename T, int D, bool DS>
__device__ __forceinline__ void dkdv_pair_item(const BwdArgs& a, char* smem, char* xch_all,
                                               int bhk, int kt) {
  typedef Mfma<T> M;
  typedef typename M::V V;
  typedef BTile<D> P;
  constexpr int KS = D / 16;
  constexpr int MT = D / 32;
  constexpr int STAGE = PairLds<D>::STAGE;
  constexpr int XCH = PairLds<D>::XCH;

  const int lane = threadIdx.x & 63, wave = wave_id();
  const int l32 = lane & 31, g = lane >> 5;
  const int pair = wave & 3;
  const bool role_b = wave >= 4;  // wave-uniform
  const int b = bhk / a.Hkv, hk = bhk % a.Hkv;
  const int group = a.H / a.Hkv;
  const int kv0 = kt * kPairBN;
  const int kvb = kv0 + pair * 32;
  const int kvw = kvb + l32;
  const bool kvvalid = kvw < a.Tkv;
  const float sl2 = a.scale * kLog2e;
  char* xch = xch_all + pair * XCH;

  // A: K rows, B: V rows of this lane's kv row
  const T* fp = role_b ? (const T*)a.v + b * a.sv_b + hk * a.sv_h + (int64_t)kvw * a.sv_s
                       : (const T*)a.k + b * a.sk_b + hk * a.sk_h + (int64_t)kvw * a.sk_s;
  V frag[KS];
#pragma unroll
  for (int st = 0; st < KS; ++st) frag[st] = kvvalid ? ld8(fp + 16 * st + 8 * g) : zero8<T>();
  f32x16 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = zero16();

  const int q_begin = a.causal ? kv0 : 0;
  const int n_q = a.Tq > q_begin ? (int)cdiv(a.Tq - q_begin, 64) : 0;
  const int n_steps = n_q * group;
  const int q_end = q_begin + 64 * n_q;
  BtOffs<T, D> fo;
  fo.init();
  typedef typename BtOffs<T, D>::TrBase TrBase;
  // Role A streams every tile: Q and dO (a quarter of each per wavefront,
  // issued between the MFMAs of its MFMA phase, whose issue slots are
  // mostly free), lse (wavefront 0) and D (wavefront 1).  Steps run over the
  // query tiles from the last one down (then the next query head), so that
  // the workgroups of one kv head, started together, read the same tiles at
  // about the same time.  The tile the next issue loads is advanced one step
  // per issue: the loop divides by nothing.
  BtDma1<T, D, 4> dq_dma, do_dma;
  dq_dma.init(a.sq_s, 0);
  do_dma.init(a.sdo_s, 0);
  constexpr int PER = BtDma1<T, D, 4>::PER;
  const int q_last = q_end - 64;
  const int hq0 = hk * group;
  const T* q_head = (const T*)a.q + b * a.sq_b + hq0 * a.sq_h;
  const T* do_head = (const T*)a.dout + b * a.sdo_b + hq0 * a.sdo_h;
  const T* q_src = q_head + (int64_t)q_last * a.sq_s;
  const T* do_src = do_head + (int64_t)q_last * a.sdo_s;
  const float* lse_h = a.lse + ((int64_t)b * a.H + hq0) * a.Tq;
  const float* del_h = a.delta + ((int64_t)b * a.H + hq0) * a.Tq;
  int ld_q0 = q_last, ld_stage = 0;
  // a full tile whose DMAs take the per-lane offsets of init (else clamped rows)
  auto ld_fast = [&]() { return dq_dma.fast && do_dma.fast && ld_q0 + 64 <= a.Tq; };
  auto issue_stats = [&]() {
    char* st = smem + ld_stage * STAGE;
    const int r = min(ld_q0 + lane, a.Tq - 1);
    if (wave == 0) dma4(lse_h + r, __builtin_amdgcn_readfirstlane(lds_addr(st + 2 * P::BYTES)));
    if (wave == 1) dma4(del_h + r, __builtin_amdgcn_readfirstlane(lds_addr(st + 2 * P::BYTES + 256)));
  };
  // DMA k of this wavefront's share of the tile: k < PER of Q, then of dO
  auto issue_part = [&](int k) {
    char* st = smem + ld_stage * STAGE;
    if (k < PER) dq_dma.issue_one(st, q_src, k);
    else do_dma.issue_one(st + P::BYTES, do_src, k - PER);
  };
  auto issue_all = [&]() {
    char* st = smem + ld_stage * STAGE;
    issue_stats();
    dq_dma.issue_at(st, q_src, a.sq_s, a.Tq - ld_q0);
    do_dma.issue_at(st + P::BYTES, do_src, a.sdo_s, a.Tq - ld_q0);
  };
  auto advance = [&]() {
    ld_stage = ld_stage == kDkvPPStages - 1 ? 0 : ld_stage + 1;
    if (ld_q0 == q_begin) {
      ld_q0 = q_last;
      q_head += a.sq_h;
      do_head += a.sdo_h;
      q_src = q_head + (int64_t)q_last * a.sq_s;
      do_src = do_head + (int64_t)q_last * a.sdo_s;
      lse_h += a.Tq;
      del_h += a.Tq;
    } else {
      ld_q0 -= 64;
      q_src -= 64 * a.sq_s;
      do_src -= 64 * a.sdo_s;
    }
  };
  // pair-uniform: the query tile from q0 has rows at or past this pair's kv rows
  auto active = [&](int q0) { return !(a.causal && q0 + 63 < kvb); };

  // MFMA phase: acc^T += T2^T op over the previous tile (MFMA i = MT t + mt,
  // t the 16-row slice), then x[mq] = T1 frag^T over the current one (MFMA
  // i = 2 st + mq).  One kRing-deep operand ring runs from the first chain
  // into the second; the caller has read the first kDkvRing T2 operands into
  // it already (before the phase barrier).
  constexpr int N2 = 4 * MT, N1 = 2 * KS, NPART = 2 * PER;
  static_assert(N2 % kDkvRing == 0 && N1 >= kDkvRing, "operand ring");
  static_assert(2 * NPART <= N2 && 2 * NPART <= N1, "DMA slots");
  V ring[kDkvRing];
  auto pre_tr = [&](const TrBase& b2) {
#pragma unroll
    for (int i = 0; i < kDkvRing; ++i) ring[i] = fo.rd_tr(b2, 16 * (i / MT), i % MT);
  };
  // the first chain: acc^T += T2^T op, the ring then running on into the
  // first T1 operands (read even when T1 is not multiplied after: a branch
  // per MFMA costs more than the unused reads of a resident tile); with
  // inter the next tile's DMAs go out after its odd MFMAs
  auto tr_chain = [&](bool inter, const TrBase& b2, const char* T1, const V (&op)[4]) {
#pragma unroll
    for (int i = 0; i < N2; ++i) {
      sched_fence();
      acc[i % MT] = M::mma(ring[i % kDkvRing], op[i / MT], acc[i % MT]);
      const int n = i + kDkvRing;
      if (n < N2) ring[i % kDkvRing] = fo.rd_tr(b2, 16 * (n / MT), n % MT);
      else ring[i % kDkvRing] = fo.rd_row(T1, 32 * ((n - N2) & 1), (n - N2) >> 1);
      if ((i & 1) && i < 2 * NPART && inter) issue_part(i >> 1);
    }
  };
  auto rows_chain = [&](const char* T1, f32x16 (&x)[2]) {
#pragma unroll
    for (int i = 0; i < N1; ++i) {
      sched_fence();
      x[i & 1] = M::mma(ring[i % kDkvRing], frag[i >> 1], i < 2 ? zero16() : x[i & 1]);
      const int n = i + kDkvRing;
      if (n < N1) ring[i % kDkvRing] = fo.rd_row(T1, 32 * (n & 1), n >> 1);
    }
  };
  // dtr: tr_chain (the ring pre-read by the caller), drows: rows_chain;
  // inter: the next tile's DMAs interleaved with tr_chain (needs dtr)
  auto mfma_phase = [&](bool dtr, bool drows, bool inter, const TrBase& b2, const char* T1,
                        const V (&op)[4], f32x16 (&x)[2]) {
    if (dtr) {
      tr_chain(inter, b2, T1, op);
    } else {
#pragma unroll
      for (int i = 0; i < kDkvRing; ++i) ring[i] = fo.rd_row(T1, 32 * (i & 1), i >> 1);
    }
    if (drows) rows_chain(T1, x);
    sched_fence();
  };

  // (role A's wavefronts only: the DMA offsets of init cover a tile with
  // wavefronts 0..3)
  if (n_steps > 0 && !role_b) {
    issue_all();
    advance();
  }
  wait_vmcnt<0>();
  lds_barrier();
  f32x16 x[2];
  V op[4];  // MFMA operand: slice t = 2 mq + u holds query rows 16t + 4g + {0..3}, 16t + 8 + 4g + {0..3}
  // per step s: q0 of s and s - 1, the LDS stage of s (s - 1 is the stage before it)
  int q0c = q_last, q0p = q_last, sc = 0;
  if (!role_b) {
    for (int s = 0; s <= n_steps; ++s) {
      const int sp = sc == 0 ? kDkvPPStages - 1 : sc - 1;
      char* const stc = smem + sc * STAGE;
      const bool cur = s < n_steps && active(q0c), prev = s >= 1 && active(q0p);
      // half-step 2s: dV^T += dO_{s-1}^T P_{s-1}, S_s = Q_s K^T (the first dO
      // operands were read ahead, at the end of half-step 2s - 1), and the
      // DMAs of tile s + 1 (into the stage of tile s - 2, whose last reads
      // were in half-step 2s - 1)
      const bool nxt = s + 1 < n_steps;
      const bool inter = nxt && prev && ld_fast();
      if (nxt && !inter) issue_all();
      if (inter) issue_stats();
      __builtin_amdgcn_s_setprio(1);
      mfma_phase(prev, cur, inter, fo.tr_base(smem + sp * STAGE + P::BYTES), stc, op, x);
      __builtin_amdgcn_s_setprio(0);
      if (nxt) advance();
      lds_barrier();
      // half-step 2s + 1: P_s (lse_s scaled by log2 e in half-step 2s)
      if (cur) {
        const float* lse_s = reinterpret_cast<const float*>(stc + 2 * P::BYTES);
        const bool need_mask = (a.causal && q0c < kvb + 31) || q0c + 64 > a.Tq;
#pragma unroll
        for (int mq = 0; mq < 2; ++mq) {
          // x[mq][r] = S[q0 + 32mq + 8(r/4) + 4g + r%4][kvw]; masked scores -> -inf (P = 0):
          // query rows >= Tq or (causal) < kvw
          if (need_mask) {
            const int base = q0c + 32 * mq + 4 * g;
            mask_outside(x[mq], a.causal ? kvw - base : -64, a.Tq - base);
          }
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) {
            const float4 L = *reinterpret_cast<const float4*>(lse_s + 32 * mq + 8 * rr + 4 * g);
            const float lv[4] = {L.x, L.y, L.z, L.w};
            float4 pv;
            float* pf = reinterpret_cast<float*>(&pv);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const float p = fast_exp2(fmaf(x[mq][4 * rr + j], sl2, -lv[j]));
              pf[j] = p;
              op[2 * mq + (rr >> 1)][4 * (rr & 1) + j] = (T)p;
            }
            *reinterpret_cast<float4*>(xch + ((mq * 4 + rr) * 64 + lane) * 16) = pv;
          }
        }
        // dO_s landed long ago: the first dV operands of half-step 2s + 2
        // are read here, under the barrier wait
        pre_tr(fo.tr_base(stc + P::BYTES));
      }
      wait_vmcnt<0>();  // tile s + 1 (issued in half-step 2s)
      lds_barrier();
      q0p = q0c;
      q0c = q0c == q_begin ? q_last : q0c - 64;
      sc = sc == kDkvPPStages - 1 ? 0 : sc + 1;
    }
  } else {
    // stored dS: the pair's chunk column, its row there, whether it exists
    // (n_kvt columns) and whether the pair has rows past Tkv (pair-uniform)
    const int n_kvt = (a.Tkv + 63) >> 6;
    const int ds_j = kvb >> 6;
    const bool ds_on = DS && ds_j < n_kvt, ds_tail = kvb + 32 > a.Tkv;
    T* const ds_lane = DS ? (T*)a.ds + ((kvb >> 5) & 1) * 2048 + lane * 8 : nullptr;
    int hc = 0, hp = 0;  // query head (from hq0) of steps s and s - 1
    for (int s = 0; s <= n_steps; ++s) {
      const int sp = sc == 0 ? kDkvPPStages - 1 : sc - 1;
      char* const stc = smem + sc * STAGE;
      char* const stp = smem + sp * STAGE;
      const bool cur = s < n_steps && active(q0c), prev = s >= 1 && active(q0p);
      // half-step 2s: dS_{s-1}; lse_s (landed at the end of half-step
      // 2s - 1) to log2 units for role A's exponentials, one value a lane
      if (wave == 4 && s < n_steps) {
        float* l = reinterpret_cast<float*>(stc + 2 * P::BYTES);
        l[lane] *= kLog2e;
      }
      const TrBase qb = fo.tr_base(stp);
      if (prev) {
        const float* del_s = reinterpret_cast<const float*>(stp + 2 * P::BYTES + 256);
#pragma unroll
        for (int mq = 0; mq < 2; ++mq) {
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) {
            const float4 pv = *reinterpret_cast<const float4*>(xch + ((mq * 4 + rr) * 64 + lane) * 16);
            const float4 Dl = *reinterpret_cast<const float4*>(del_s + 32 * mq + 8 * rr + 4 * g);
            const float pp[4] = {pv.x, pv.y, pv.z, pv.w}, dd[4] = {Dl.x, Dl.y, Dl.z, Dl.w};
#pragma unroll
            for (int j = 0; j < 4; ++j)
              op[2 * mq + (rr >> 1)][4 * (rr & 1) + j] = (T)(pp[j] * (x[mq][4 * rr + j] - dd[j]));
          }
        }
        // the first dK operands (Q_{s-1}^T) of the coming MFMA phase
        pre_tr(qb);
        // the stored dS, behind those reads (1.6% faster than ahead of them)
        if constexpr (DS) {
          if (ds_on) {
            T* dst = ds_lane + ((int64_t)(b * a.H + hq0 + hp) * a.ds_bh +
                                (ds_row(a.causal, q0p >> 6, n_kvt) + ds_j) * 4096);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              u32x4 u = __builtin_bit_cast(u32x4, op[t]);
              if (ds_tail && !kvvalid) u = u32x4{0u, 0u, 0u, 0u};
              __builtin_nontemporal_store(u, reinterpret_cast<u32x4*>(dst + 512 * t));
            }
          }
        }
      }
      lds_barrier();
      // half-step 2s + 1: dK^T += Q_{s-1}^T dS_{s-1}, dP_s = dO_s V^T
      __builtin_amdgcn_s_setprio(1);
      mfma_phase(prev, cur, false, qb, stc + P::BYTES, op, x);
      __builtin_amdgcn_s_setprio(0);
      lds_barrier();
      q0p = q0c;
      hp = hc;
      hc += q0c == q_begin;
      q0c = q0c == q_begin ? q_last : q0c - 64;
      sc = sc == kDkvPPStages - 1 ? 0 : sc + 1;
    }
  }

  if (kvvalid) {
    T* out = role_b ? (T*)a.dk + b * a.sdk_b + hk * a.sdk_h + (int64_t)kvw * a.sdk_s
                    : (T*)a.dv + b * a.sdv_b + hk * a.sdv_h + (int64_t)kvw * a.sdv_s;
    const float sc = role_b ? a.scale : 1.0f;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int d0 = 32 * mt + 8 * rr + 4 * g;
        store4<T>(out + d0, acc[mt][4 * rr] * sc, acc[mt][4 * rr + 1] * sc,
                  acc[mt][4 * rr + 2] * sc, acc[mt][4 * rr + 3] * sc);
      }
    }
  }
}

// dK, dV (and with DS the stored dS) over (batch * kv head, kv tile) items.
// PERSIST: one workgroup per compute unit walks a fixed list of items
// instead of one workgroup per item (a workgroup's turnaround on its compute
// unit measured about 8 us, 10% of the config-3 kernel at 16 items per CU).
// Each XCD (workgroups b with b % 8 == x) owns a contiguous eighth of the
// (batch, kv head)s, so their Q / dO tiles stay in that XCD's L2.  Its
// workgroups take the XCD's kv-tile pairs (t, n - 1 - t) round-robin, head by
// head: under the causal mask every pair carries the same number of steps,
// whatever the ratio of kv tiles to workgroups (taking single tiles
// round-robin balanced only with as many workgroups per XCD as kv tiles: at
// [8, 32, 2048, 128], 16 tiles per head for 32 workgroups, each workgroup
// kept one tile index and the kernel ran 1.17-1.36 ms against 1.43-1.65 ms
// for the twice larger [4, 32, 4096, 128]).
template <typename T, int D, bool DS, bool PERSIST>
__global__ void __launch_bounds__(64 * kPairWaves, 1)  // 2 wavefronts per SIMD
attn_bwd_dkdv_pair(BwdArgs a) {
  __shared__ __attribute__((aligned(1024))) char smem[kDkvPPStages * PairLds<D>::STAGE];
  __shared__ __attribute__((aligned(16))) char xch_all[4 * PairLds<D>::XCH];
  if constexpr (PERSIST) {
    const int per = a.B * a.Hkv / kXcds;  // the host checks divisibility
    const int slots = (int)gridDim.x / kXcds;
    const int x = (int)blockIdx.x % kXcds, slot = (int)blockIdx.x / kXcds;
    const int n_pairs = (a.n_tiles + 1) / 2;  // per head; odd n: the middle tile alone
    const int n_work = per * n_pairs;
    for (int w = slot; w < n_work; w += slots) {
      const int j = w / n_pairs, t0 = w % n_pairs, t1 = a.n_tiles - 1 - t0;
      dkdv_pair_item<T, D, DS>(a, smem, xch_all, x * per + j, t0);
      lds_barrier();  // every wavefront is done with the LDS before the next item's DMAs
      if (t1 != t0) {
        dkdv_pair_item<T, D, DS>(a, smem, xch_all, x * per + j, t1);
        lds_barrier();
      }
    }
  } else {
    int bhk, kt;  // kt = 0 sees the most queries: heaviest first
    lpt_item(xcd_remap(blockIdx.x, gridDim.x), gridDim.x, a.B * a.Hkv, a.n_tiles, a.causal,
             a.B * a.Hkv, bhk, kt);
    dkdv_pair_item<T, D, DS>(a, smem, xch_all, bhk, kt);
  }
}

// dQ of one query row from its MFMA accumulators (element d = 32 mt + 8 rr +
// 4 g + j at dq[mt][4 rr + j]): scaled, with RoPE the inverse rotation (the
// gradient of the unrotated q; d pairs with d + D/2 in dq[mt + MT/2]; NaN for
// a position outside the tables), rounded once and stored.
template <typename T, int D>
__device__ __forceinline__ void store_dq_row(f32x16 (&dq)[D / 32], T* dqr, float sc,
                                             const RopeQ& rp, bool rope, int64_t rpos,
                                             bool rpos_ok, int g) {
  constexpr int MT = D / 32;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int r = 0; r < 16; ++r) dq[mt][r] *= sc;
  if (rope) {
    const float nan = __builtin_nanf("");
#pragma unroll
    for (int mt = 0; mt < MT / 2; ++mt) {
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int d0 = 32 * mt + 8 * rr + 4 * g;
        float c[4] = {}, s[4] = {};
        if (rpos_ok) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            c[j] = rp.cos[rpos * (D / 2) + d0 + j];
            s[j] = rp.sin[rpos * (D / 2) + d0 + j];
          }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float oa, ob;
          rope_pair(dq[mt][4 * rr + j], dq[mt + MT / 2][4 * rr + j], c[j], -s[j], oa, ob);
          dq[mt][4 * rr + j] = rpos_ok ? oa : nan;
          dq[mt + MT / 2][4 * rr + j] = rpos_ok ? ob : nan;
        }
      }
    }
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int d0 = 32 * mt + 8 * rr + 4 * g;
      store4<T>(dqr + d0, dq[mt][4 * rr], dq[mt][4 * rr + 1], dq[mt][4 * rr + 2],
                dq[mt][4 * rr + 3]);
    }
  }
}

// dQ: a workgroup owns 32 * WAVES query rows of one (batch, head), a
// wavefront 32 of them (Q, dO fragments in registers, lane = query row),
// and sweeps the 64-row K/V tiles it can see: S^T = K Q^T and
// dP^T = V dO^T from row reads, dQ^T += K^T dS^T from transposing reads.
template <typename T, int D, int WAVES>
__global__ void __launch_bounds__(64 * WAVES, D > 128 ? 1 : 8 / WAVES)  // 2 wavefronts per SIMD (1 at D = 256)
attn_bwd_dq_v2(BwdArgs a) {
  typedef Mfma<T> M;
  typedef typename M::V V;
  typedef BTile<D> P;
  constexpr int KS = D / 16;
  constexpr int MT = D / 32;
  constexpr int BM = 32 * WAVES;
  constexpr int STAGE = 2 * P::BYTES;  // K, V
  __shared__ __attribute__((aligned(1024))) char smem[2 * STAGE];

  const int lane = threadIdx.x & 63, wave = wave_id();
  const int l32 = lane & 31, g = lane >> 5;
  int bh, rank;
  lpt_item(xcd_remap(blockIdx.x, gridDim.x), gridDim.x, a.B * a.H, a.n_tiles, a.causal, a.B * a.H,
           bh, rank);
  const int qt = a.n_tiles - 1 - rank;  // rank 0: the most kv tiles
  const int b = bh / a.H, h = bh % a.H;
  const int hk = h / (a.H / a.Hkv);
  const T* qp = (const T*)a.q + b * a.sq_b + h * a.sq_h;
  const T* dop = (const T*)a.dout + b * a.sdo_b + h * a.sdo_h;
  const T* kp = (const T*)a.k + b * a.sk_b + hk * a.sk_h;
  const T* vp = (const T*)a.v + b * a.sv_b + hk * a.sv_h;
  const int q0 = qt * BM;
  const int qw0 = q0 + wave * 32;
  const int qrow = qw0 + l32;
  const bool qvalid = qrow < a.Tq;
  const float sl2 = a.scale * kLog2e;

  V qf[KS], df[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    qf[s] = qvalid ? ld8(qp + (int64_t)qrow * a.sq_s + 16 * s + 8 * g) : zero8<T>();
    df[s] = qvalid ? ld8(dop + (int64_t)qrow * a.sdo_s + 16 * s + 8 * g) : zero8<T>();
  }
  // with RoPE: rotate q on load, and hand the rotated rows to the dK/dV kernel
  const bool rope = a.rope.cos != nullptr;
  int64_t rpos = 0;
  bool rpos_ok = false;
  if (rope && qvalid) {
    rpos_ok = rope_position(a.rope, b, a.Tq, qrow, rpos);
    rope_q_frag<T, D>(qf, a.rope, rpos, rpos_ok, g);
    T* qr = (T*)a.q_rot + ((int64_t)bh * a.Tq + qrow) * D;
#pragma unroll
    for (int s = 0; s < KS; ++s) *reinterpret_cast<V*>(qr + 16 * s + 8 * g) = qf[s];
  }
  const float lse2 = qvalid ? a.lse[(int64_t)bh * a.Tq + qrow] * kLog2e : INFINITY;
  // delta = rowsum(dO * O) for this lane's query row (the two lanes of a row
  // hold alternate 8-column halves); written out for the dK/dV kernel
  float dl = 0.f;
  if (qvalid) {
    const T* orow = (const T*)a.o + b * a.so_b + h * a.so_h + (int64_t)qrow * a.so_s;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const V of = ld8(orow + 16 * s + 8 * g);
#pragma unroll
      for (int j = 0; j < 8; ++j) dl += (float)df[s][j] * (float)of[j];
    }
  }
  dl += __shfl_xor(dl, 32, 64);
  if (qvalid && g == 0) a.delta[(int64_t)bh * a.Tq + qrow] = dl;

  f32x16 dq[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) dq[mt] = zero16();

  const int kv_end = a.causal ? min(a.Tkv, q0 + BM) : a.Tkv;
  const int n_kv = (int)cdiv(kv_end, 64);
  BtDma<T, D, WAVES> dma;
  dma.init(a.sk_s, a.sv_s);
  if (n_kv > 0) dma.issue(smem, kp, a.sk_s, vp, a.sv_s, 0, a.Tkv);
  for (int it = 0; it < n_kv; ++it) {
    const int kv0 = it * 64;
    // accumulators in VGPRs (the softmax needs the rest); at head_dim 256
    // they take the AGPRs, beside Q and dO in VGPRs
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if constexpr (D > 128) pin_agpr(dq[mt]);
      else pin_vgpr(dq[mt]);
    }
    wait_vmcnt<0>();
    __syncthreads();
    if (it + 1 < n_kv)
      dma.issue(smem + ((it + 1) & 1) * STAGE, kp, a.sk_s, vp, a.sv_s, kv0 + 64, a.Tkv);
    if (a.causal && kv0 > qw0 + 31) continue;  // this wavefront's rows see none of the tile
    const char* Ks = smem + (it & 1) * STAGE;
    const char* Vs = Ks + P::BYTES;
    const bool need_mask = kv0 + 64 > a.Tkv || (a.causal && kv0 + 63 > qw0);

    V dsb[4];  // dS^T rounded to T as formed: operand t holds rows 16t + 4g + {0..3}, 16t + 8 + ...
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      f32x16 s = zero16(), dp = zero16();
#pragma unroll
      for (int st = 0; st < KS; ++st) {
        s = M::mma(bt_row<T, D>(Ks, 32 * u, st), qf[st], s);
        dp = M::mma(bt_row<T, D>(Vs, 32 * u, st), df[st], dp);
      }
      // s[r] = S^T[kv0 + 32u + 8(r/4) + 4g + r%4][qrow]; masked scores -> -inf (p = 0):
      // kv rows >= Tkv or (causal) > qrow
      if (need_mask)
        mask_above(s, (a.causal ? min(a.Tkv - 1, qrow) : a.Tkv - 1) - kv0 - 32 * u - 4 * g);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = fast_exp2(fmaf(s[r], sl2, -lse2));
        dsb[2 * u + (r >> 3)][r & 7] = (T)(p * (dp[r] - dl));
      }
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) dq[mt] = M::mma(bt_tr<T, D>(Ks, 16 * t, mt), dsb[t], dq[mt]);
    }
  }

  if (qvalid)
    store_dq_row<T, D>(dq, (T*)a.dq + b * a.sdq_b + h * a.sdq_h + (int64_t)qrow * a.sdq_s, a.scale,
                       a.rope, rope, rpos, rpos_ok, g);
}

// --------------------------------------------- backward: stored-dS path --
// With a dS workspace the dK/dV kernel stores the dS tiles it forms and dQ =
// scale * dS K becomes a product over them, instead of a dQ kernel that forms
// S and dP a second time (the recomputing backward executes 14 D flops per
// visible (query, key) pair, this one the algorithmic 10 D, plus a 2-byte
// store and load of dS per pair).  delta then comes from its own kernel,
// ahead of dK/dV.

// delta[bh][q] = sum_d dO[q][d] * O[q][d] (fp32): D / 8 lanes a row, one
// 16-byte granule of each tensor per lane, shuffle-reduced (1.3x faster than
// two lanes a row); with RoPE also the rotated q rows (q_rot, [B, H, Tq, D])
// that the dK/dV kernel reads, rotated as rope_q_frag rotates them (lane
// sub's granule pairs with lane sub ^ (D / 16)'s, D / 2 columns away).
template <typename T, int D>
__global__ void __launch_bounds__(256)
attn_bwd_delta_v(BwdArgs a) {
  typedef typename Mfma<T>::V V;
  constexpr int LPR = D / 8, RPB = 256 / LPR, HALF = D / 2;
  const int sub = threadIdx.x % LPR;
  const int64_t n_rows = (int64_t)a.B * a.H * a.Tq;
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / LPR;
  const bool valid = row < n_rows;
  const int64_t r = valid ? row : n_rows - 1;  // every lane takes part in the shuffles
  const int q = (int)(r % a.Tq);
  const int64_t bh = r / a.Tq;
  const int b = (int)(bh / a.H), h = (int)(bh % a.H);
  const V ov = ld8((const T*)a.o + b * a.so_b + h * a.so_h + (int64_t)q * a.so_s + 8 * sub);
  const V dv = ld8((const T*)a.dout + b * a.sdo_b + h * a.sdo_h + (int64_t)q * a.sdo_s + 8 * sub);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) s = fmaf((float)ov[j], (float)dv[j], s);
#pragma unroll
  for (int m = LPR / 2; m >= 1; m >>= 1) s += __shfl_xor(s, m, 64);
  if (valid && sub == 0) a.delta[row] = s;
  if (a.rope.cos != nullptr) {
    const V qv = ld8((const T*)a.q + b * a.sq_b + h * a.sq_h + (int64_t)q * a.sq_s + 8 * sub);
    const u32x4 mine = __builtin_bit_cast(u32x4, qv);
    u32x4 other;
#pragma unroll
    for (int k = 0; k < 4; ++k) other[k] = __shfl_xor(mine[k], LPR / 2, 64);
    const V qo = __builtin_bit_cast(V, other);
    int64_t pos = 0;
    const bool ok = rope_position(a.rope, b, a.Tq, q, pos);
    const bool lo = sub < LPR / 2;
    const int col = 8 * (sub & (LPR / 2 - 1));  // table column of the lane's first element
    const float nan = __builtin_nanf("");
    V out;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float c = ok ? a.rope.cos[pos * HALF + col + j] : 0.f;
      const float sn = ok ? a.rope.sin[pos * HALF + col + j] : 0.f;
      float oa, ob;
      rope_pair((float)(lo ? qv[j] : qo[j]), (float)(lo ? qo[j] : qv[j]), c, sn, oa, ob);
      out[j] = (T)(ok ? (lo ? oa : ob) : nan);
    }
    if (valid) *reinterpret_cast<V*>((T*)a.q_rot + row * D + 8 * sub) = out;
  }
}

// dQ from the stored dS: a workgroup owns query tiles 4 qb .. 4 qb + 3 of one
// (batch, head) and sweeps the kv tiles they see; per kv tile, K [64][D] and
// the four dS chunks arrive by DMA in a 3-stage LDS ring (one K tile per four
// chunks: the sweep moves 1.5 bytes through the CU per byte of dS), and
// wavefront w accumulates dQ^T over all D for chunk columns 32 (w & 1) .. + 31
// of query tile 4 qb + (w >> 1): A = K^T and B = dS^T, both from transposing
// reads (k = kv rows).
constexpr int kDsWaves = 8;
constexpr int kDsTiles = 4;  // query tiles per workgroup
constexpr int kDsStages = 3;  // 2 measured 0.670 against 0.545 ms at config 3

template <typename T, int D>
__global__ void __launch_bounds__(64 * kDsWaves, 1)
attn_bwd_dq_ds(BwdArgs a) {
  typedef Mfma<T> M;
  typedef typename M::V V;
  typedef BTile<D> PK;
  typedef BTile<64> PS;
  constexpr int MT = D / 32;
  constexpr int STAGE = PK::BYTES + kDsTiles * PS::BYTES;
  __shared__ __attribute__((aligned(1024))) char smem[kDsStages * STAGE];
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int l32 = lane & 31, g = lane >> 5;
  // causal: the longest sweeps first across four (batch, head)s at a time per
  // XCD -- config 3: 560 us one at a time (a long tail), 519 us two, 491-512
  // four or eight, 537 all sixteen of the XCD's (K falls out of its L2)
  int bh, rank;
  lpt_item(xcd_remap(blockIdx.x, gridDim.x), gridDim.x, a.B * a.H, a.n_tiles, a.causal, 4, bh, rank);
  const int qb = a.n_tiles - 1 - rank;
  const int b = bh / a.H, h = bh % a.H, hk = h / (a.H / a.Hkv);
  const int n_qt = (a.Tq + 63) >> 6, n_kvt = (a.Tkv + 63) >> 6;
  const int qt0 = kDsTiles * qb;
  const int last = min(qt0 + kDsTiles, n_qt) - 1;  // the workgroup's last query tile
  const int sel = wave >> 1, mq = wave & 1;
  const int qt = qt0 + sel;
  // kv tiles in a query tile's row of chunks, the sweep's, this wavefront's
  auto n_j = [&](int q) { return a.causal ? min(q + 1, n_kvt) : n_kvt; };
  const int n_kv = n_j(last);
  const int my_kv = qt > last ? 0 : n_j(qt);
  const T* kb = (const T*)a.k + b * a.sk_b + hk * a.sk_h;
  const T* dsb = (const T*)a.ds + (int64_t)bh * a.ds_bh;
  BtOffs<T, D> ko;
  ko.init();
  // B operand: transposing-read offsets of this wavefront's 32 chunk columns
  // (BtOffs' table indexed by the run-time mq would be moved to LDS)
  uint32_t so[2];
  {
    const int ts = lane & 15, th = (lane >> 4) & 1, r1 = 4 * g + (ts >> 2);
#pragma unroll
    for (int k = 0; k < 2; ++k)
      so[k] = PS::off(r1 + 8 * k, 4 * mq + 2 * th + ((ts & 3) >> 1)) + (ts & 1) * 8;
  }
  BtDma1<T, D, kDsWaves> kdma;
  kdma.init(a.sk_s, 0);
  // chunk DMA: this wavefront fills LDS rows 8 wave .. + 7 of each chunk
  // tile, lane -> row 8 wave + lane / 8, granule (lane % 8) ^ key(row)
  static_assert(PS::DMAS == kDsWaves, "one DMA per wavefront per chunk");
  uint32_t soff;
  {
    const int r = 8 * wave + (lane >> 3), c = (lane & 7) ^ PS::key(r);
    soff = (uint32_t)(2 * (2048 * (r >> 5) + 512 * (c & 3) + 8 * (32 * (c >> 2) + (r & 31))));
  }
  constexpr int PERW = BtDma1<T, D, kDsWaves>::PER + kDsTiles;  // DMAs per wavefront per tile
  // kv tile j: K, and chunk (q, j) of each query tile q, clamped to the
  // tile's row (a tile past the workgroup's last, or a chunk past its row
  // under the causal mask, is loaded but not multiplied)
  auto issue = [&](int j) {
    char* st = smem + (j % kDsStages) * STAGE;
    kdma.issue_at(st, kb + (int64_t)(64 * j) * a.sk_s, a.sk_s, a.Tkv - 64 * j);
#pragma unroll
    for (int k = 0; k < kDsTiles; ++k) {
      const int q = min(qt0 + k, last);
      const T* src = dsb + (ds_row(a.causal, q, n_kvt) + min(j, n_j(q) - 1)) * 4096;
      dma16s(src, soff,
             __builtin_amdgcn_readfirstlane(lds_addr(st + PK::BYTES + k * PS::BYTES + wave * 1024)));
    }
  };
  typedef short v4s __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) v4s lds_v4s;
  f32x16 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = zero16();
#pragma unroll
  for (int j = 0; j < kDsStages - 1; ++j)
    if (j < n_kv) issue(j);
  for (int j = 0; j < n_kv; ++j) {
    // tile j landed (the later tiles issued so far stay in flight)
    if (j + kDsStages - 2 < n_kv) wait_vmcnt<(kDsStages - 2) * PERW>();
    else wait_vmcnt<0>();
    lds_barrier();  // ... for every wavefront; tile j - 1's stage is free
    if (j + kDsStages - 1 < n_kv) issue(j + kDsStages - 1);
    if (j < my_kv) {
      const char* st = smem + (j % kDsStages) * STAGE;
      const auto kbs = ko.tr_base(st);
      uint32_t sx[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        sx[k] = lds_addr(st + PK::BYTES + sel * PS::BYTES) + so[k];
        asm("" : "+v"(sx[k]));
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_v4s*)(uintptr_t)(sx[0] + (uint32_t)(16 * t * PS::RB)));
        const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_v4s*)(uintptr_t)(sx[1] + (uint32_t)(16 * t * PS::RB)));
        const V bs = __builtin_bit_cast(V, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt] = M::mma(ko.rd_tr(kbs, 16 * t, mt), bs, acc[mt]);
      }
    }
  }
  if (qt <= last) {
    const int qr = 64 * qt + ds_col_row(32 * mq + l32);
    if (qr < a.Tq) {
      const bool rope = a.rope.cos != nullptr;
      int64_t rpos = 0;
      const bool rpos_ok = rope && rope_position(a.rope, b, a.Tq, qr, rpos);
      store_dq_row<T, D>(acc, (T*)a.dq + b * a.sdq_b + h * a.sdq_h + (int64_t)qr * a.sdq_s,
                         a.scale, a.rope, rope, rpos, rpos_ok, g);
    }
  }
}

// ------------------------------------------------------ decode (q_len 1) --
// One query row per (batch, head) against a K/V cache: memory-bound, and a
// grid of B * H one-row tiles leaves most of the GPU idle.  A workgroup owns
// one (batch, kv head) and one chunk of the key sequence and serves every
// query head of the GQA group from the same K/V reads; D / 8 lanes hold one
// 16-byte slice each of a key row, so a wavefront walks 64 / (D / 8) keys
// per step.  Each lane group keeps an online softmax state (m, l, o over its
// slice of dims, log2 units, rescaled only when a score exceeds m by more
// than 8) per query head; the groups of a wavefront merge through cross-lane
// shuffles, the wavefronts through LDS, and each workgroup writes its chunk's
// unnormalised (m, l, o) per head to a workspace that attn_decode_combine
// merges over the chunks (o = sum o_c 2^(m_c - M) / sum l_c 2^(m_c - M)).
constexpr int kDecWaves = 4;
constexpr int kDecMinChunk = 256;        // keys per chunk at least
// workgroups to aim for: 512 against 2048 (graph replays, same box) took
// [8, 32, 8, 8192, 128] 58.3 -> 53.6-54.4 us and [8, 32, 32, 4096, 128]
// 89.6 -> 87.7 us, [16, 12, 12, 1024, 64] 15.0 -> 15.5 us; 256 was slower
constexpr int kDecTargetBlocks = 512;
constexpr int kDecUnroll = 4;            // key rows in flight per lane
constexpr int kDecMaxSplits = 256;       // chunks per (batch, head) at most

struct DecArgs {
  const void* q; const void* k; const void* v; void* o; float* lse; float* part;
  int64_t sq_b, sq_h, sk_b, sk_h, sk_s, sv_b, sv_h, sv_s, so_b, so_h;
  int B, H, Hkv, Tkv, n_splits, chunk;
  float sl2;  // scale * log2(e)
};

int dec_splits(int64_t B, int64_t Hkv, int64_t Tkv) {
  const int64_t want = cdiv(kDecTargetBlocks, std::max<int64_t>(1, B * Hkv));
  const int64_t most = std::min<int64_t>(kDecMaxSplits, std::max<int64_t>(1, cdiv(Tkv, kDecMinChunk)));
  return (int)std::max<int64_t>(1, std::min(want, most));
}

// Sum over each aligned group of N lanes (N = 8 or 16, inside one 16-lane
// DPP row) with DPP moves: two quad permutations (xor 1, xor 2), then the
// half-row and row mirrors -- four VALU adds, where __shfl_xor would make
// four dependent LDS permute round trips.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                               0xF, 0xF, false));
}
template <int N>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(N == 8 || N == 16, "lane group of 8 or 16");
  v += dpp_mov<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v += dpp_mov<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v += dpp_mov<0x141>(v);  // row_half_mirror: lane i of 8 <- lane 7 - i
  if constexpr (N == 16) v += dpp_mov<0x140>(v);  // row_mirror: lane i of 16 <- lane 15 - i
  return v;
}

// (m, l, o) <- merge of two online-softmax states over disjoint keys
template <int N>
__device__ __forceinline__ void dec_merge(float& m, float& l, float (&o)[N], float m2, float l2,
                                          const float (&o2)[N]) {
  const float mx = fmaxf(m, m2);
  if (mx == -INFINITY) return;  // both empty
  const float c1 = fast_exp2(m - mx), c2 = fast_exp2(m2 - mx);
  l = l * c1 + l2 * c2;
#pragma unroll
  for (int i = 0; i < N; ++i) o[i] = o[i] * c1 + o2[i] * c2;
  m = mx;
}

template <typename T, int D, int G>
__global__ void __launch_bounds__(64 * kDecWaves)
attn_decode_kernel(DecArgs a) {
  constexpr int LPK = D / 8;     // lanes per key row
  constexpr int KPW = 64 / LPK;  // keys per wavefront step
  __shared__ float sm[kDecWaves][G], sl[kDecWaves][G], so[kDecWaves][G][D];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane / LPK, part = lane % LPK;
  int bid = blockIdx.x;
  const int split = bid % a.n_splits;
  bid /= a.n_splits;
  const int hk = bid % a.Hkv, b = bid / a.Hkv;
  const int group = a.H / a.Hkv;
  const int kv0 = split * a.chunk;
  const int kv1 = min(a.Tkv, kv0 + a.chunk);

  float qv[G][8], m[G], l[G], o[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[g][i] = 0.f;
    if (g < group) {
      float f[8];
      unpack<T>(ld16((const T*)a.q + b * a.sq_b + (int64_t)(hk * group + g) * a.sq_h + part * 8), f);
#pragma unroll
      for (int i = 0; i < 8; ++i) qv[g][i] = f[i] * a.sl2;
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) qv[g][i] = 0.f;
    }
  }
  const T* kb = (const T*)a.k + b * a.sk_b + hk * a.sk_h + part * 8;
  const T* vb = (const T*)a.v + b * a.sv_b + hk * a.sv_h + part * 8;
  // kDecUnroll key rows per lane are loaded before any is used (memory-level
  // parallelism for a latency-bound stream); the LPK lanes of a key row share
  // its bounds, so the shuffles below only combine lanes active together
  constexpr int kStride = kDecWaves * KPW;
  for (int kv = kv0 + wave * KPW + sub; kv < kv1; kv += kDecUnroll * kStride) {
    u32x4 kr[kDecUnroll], vr[kDecUnroll];
#pragma unroll
    for (int u = 0; u < kDecUnroll; ++u) {
      const int ku = kv + u * kStride;
      if (ku < kv1) {
        kr[u] = ld16_nt(kb + (int64_t)ku * a.sk_s);
        vr[u] = ld16_nt(vb + (int64_t)ku * a.sv_s);
      }
    }
#pragma unroll
    for (int u = 0; u < kDecUnroll; ++u) {
      if (kv + u * kStride >= kv1) break;
      float kf[8], vf[8];
      unpack<T>(kr[u], kf);
      unpack<T>(vr[u], vf);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) s = fmaf(qv[g][i], kf[i], s);
        s = group_sum<LPK>(s);
        if (s > m[g] + 8.f) {
          const float c = fast_exp2(m[g] - s);
          l[g] *= c;
#pragma unroll
          for (int i = 0; i < 8; ++i) o[g][i] *= c;
          m[g] = s;
        }
        const float p = fast_exp2(s - m[g]);
        l[g] += p;
#pragma unroll
        for (int i = 0; i < 8; ++i) o[g][i] = fmaf(p, vf[i], o[g][i]);
      }
    }
  }
  // merge the KPW key slots of the wavefront (lanes part, part + LPK, ...)
#pragma unroll
  for (int off = LPK; off < kWave; off <<= 1) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float o2[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) o2[i] = __shfl_xor(o[g][i], off, kWave);
      const float m2 = __shfl_xor(m[g], off, kWave), l2 = __shfl_xor(l[g], off, kWave);
      dec_merge<8>(m[g], l[g], o[g], m2, l2, o2);
    }
  }
  if (sub == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (part == 0) {
        sm[wave][g] = m[g];
        sl[wave][g] = l[g];
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) so[wave][g][part * 8 + i] = o[g][i];
    }
  }
  __syncthreads();
  // merge the wavefronts; thread d < D owns dimension d of every head
  for (int g = 0; g < group && g < G; ++g) {
    if (threadIdx.x < D) {
      float mm = sm[0][g], ll = sl[0][g], oo[1] = {so[0][g][threadIdx.x]};
#pragma unroll
      for (int w = 1; w < kDecWaves; ++w) {
        const float o2[1] = {so[w][g][threadIdx.x]};
        dec_merge<1>(mm, ll, oo, sm[w][g], sl[w][g], o2);
      }
      if (a.n_splits == 1) {
        // one chunk holds the whole cache: o and lse directly, as the
        // combine kernel would form them from this one partial (its weight
        // 2^(m - m) = 1), so no second launch
        const int hq = hk * group + g;
        T* orow = (T*)a.o + b * a.so_b + hq * a.so_h;
        orow[threadIdx.x] = from_f32<T>(ll > 0.f ? oo[0] / ll : 0.f);
        if (threadIdx.x == 0) a.lse[(int64_t)b * a.H + hq] = (mm + log2f(ll)) * kLn2;
      } else {
        float* dst = a.part + (((int64_t)b * a.H + hk * group + g) * a.n_splits + split) * (D + 2);
        dst[2 + threadIdx.x] = oo[0];
        if (threadIdx.x == 0) {
          dst[0] = mm;
          dst[1] = ll;
        }
      }
    }
  }
}

// o[b, h] and lse[b, h] from the chunks' (m, l, o): the chunk maxima and
// weights 2^(m_c - M) are formed by strided threads and reduced through LDS
// (independent loads, not a serial walk over the chunks); thread d then sums
// dimension d of every chunk's o with the weights, loads unrolled.
template <typename T, int D>
__global__ void __launch_bounds__(D)
attn_decode_combine(DecArgs a) {
  constexpr int NW = D / kWave;
  __shared__ float wgt[kDecMaxSplits];
  __shared__ float red[2][NW];
  const int bh = blockIdx.x;
  const int b = bh / a.H, h = bh % a.H;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const float* src = a.part + (int64_t)bh * a.n_splits * (D + 2);
  float mx = -INFINITY;
  for (int c = threadIdx.x; c < a.n_splits; c += D) mx = fmaxf(mx, src[c * (D + 2)]);
  mx = wave_max(mx);
  if (lane == 0) red[0][wave] = mx;
  __syncthreads();
  mx = red[0][0];
#pragma unroll
  for (int w = 1; w < NW; ++w) mx = fmaxf(mx, red[0][w]);
  float ls = 0.f;
  for (int c = threadIdx.x; c < a.n_splits; c += D) {
    const float mc = src[c * (D + 2)];
    const float w = mc == -INFINITY ? 0.f : fast_exp2(mc - mx);  // a chunk without keys
    wgt[c] = w;
    ls += src[c * (D + 2) + 1] * w;
  }
  ls = wave_sum(ls);
  if (lane == 0) red[1][wave] = ls;
  __syncthreads();
  float l = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) l += red[1][w];
  float od = 0.f;
#pragma unroll 8
  for (int c = 0; c < a.n_splits; ++c) od += src[c * (D + 2) + 2 + threadIdx.x] * wgt[c];
  T* orow = (T*)a.o + b * a.so_b + h * a.so_h;
  orow[threadIdx.x] = from_f32<T>(l > 0.f ? od / l : 0.f);
  if (threadIdx.x == 0) a.lse[bh] = (mx + log2f(l)) * kLn2;
}

// --------------------------------------------------------------- SIMT path --
// One wavefront per row; lane i owns head-dim entries i, i+64, ...
constexpr int kSimtMaxPerLane = 16;  // head_dim <= 1024

template <typename T, int PL>
__global__ void __launch_bounds__(64)
attn_fwd_simt(FwdArgs a, int D) {
  const int lane = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int qrow = (int)(row % a.Tq);
  const int64_t bh = row / a.Tq;
  const int b = (int)(bh / a.H), h = (int)(bh % a.H);
  const int hk = h / (a.H / a.Hkv);
  const T* qp = (const T*)a.q + b * a.sq_b + h * a.sq_h + (int64_t)qrow * a.sq_s;
  const T* kp = (const T*)a.k + b * a.sk_b + hk * a.sk_h;
  const T* vp = (const T*)a.v + b * a.sv_b + hk * a.sv_h;
  float qv[PL], acc[PL];
#pragma unroll
  for (int j = 0; j < PL; ++j) {
    const int d = lane + 64 * j;
    qv[j] = d < D ? to_f32(qp[d]) : 0.f;
    acc[j] = 0.f;
  }
  float m = -INFINITY, l = 0.f;
  const int kv_end = a.causal ? min(a.Tkv, qrow + 1) : a.Tkv;
  for (int kv = 0; kv < kv_end; ++kv) {
    const T* kr = kp + (int64_t)kv * a.sk_s;
    float part = 0.f;
#pragma unroll
    for (int j = 0; j < PL; ++j) {
      const int d = lane + 64 * j;
      if (d < D) part += qv[j] * to_f32(kr[d]);
    }
    const float s = wave_sum(part) * a.scale;
    const float m_new = fmaxf(m, s);
    const float alpha = expf(m - m_new);
    const float p = expf(s - m_new);
    l = l * alpha + p;
    m = m_new;
    const T* vr = vp + (int64_t)kv * a.sv_s;
#pragma unroll
    for (int j = 0; j < PL; ++j) {
      const int d = lane + 64 * j;
      acc[j] = acc[j] * alpha + (d < D ? p * to_f32(vr[d]) : 0.f);
    }
  }
  const float inv = l > 0.f ? 1.0f / l : 0.f;
  T* orow = (T*)a.o + b * a.so_b + h * a.so_h + (int64_t)qrow * a.so_s;
#pragma unroll
  for (int j = 0; j < PL; ++j) {
    const int d = lane + 64 * j;
    if (d < D) orow[d] = from_f32<T>(acc[j] * inv);
  }
  if (lane == 0) a.lse[row] = m + logf(l);
}

template <typename T, int PL>
__global__ void __launch_bounds__(64)
attn_bwd_dq_simt(BwdArgs a, int D) {
  const int lane = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int qrow = (int)(row % a.Tq);
  const int64_t bh = row / a.Tq;
  const int b = (int)(bh / a.H), h = (int)(bh % a.H);
  const int hk = h / (a.H / a.Hkv);
  const T* qp = (const T*)a.q + b * a.sq_b + h * a.sq_h + (int64_t)qrow * a.sq_s;
  const T* dp_ = (const T*)a.dout + b * a.sdo_b + h * a.sdo_h + (int64_t)qrow * a.sdo_s;
  const T* kp = (const T*)a.k + b * a.sk_b + hk * a.sk_h;
  const T* vp = (const T*)a.v + b * a.sv_b + hk * a.sv_h;
  const float lse = a.lse[row], dl = a.delta[row];
  float qv[PL], dov[PL], acc[PL];
#pragma unroll
  for (int j = 0; j < PL; ++j) {
    const int d = lane + 64 * j;
    qv[j] = d < D ? to_f32(qp[d]) : 0.f;
    dov[j] = d < D ? to_f32(dp_[d]) : 0.f;
    acc[j] = 0.f;
  }
  const int kv_end = a.causal ? min(a.Tkv, qrow + 1) : a.Tkv;
  for (int kv = 0; kv < kv_end; ++kv) {
    const T* kr = kp + (int64_t)kv * a.sk_s;
    const T* vr = vp + (int64_t)kv * a.sv_s;
    float ps = 0.f, pd = 0.f;
#pragma unroll
    for (int j = 0; j < PL; ++j) {
      const int d = lane + 64 * j;
      if (d < D) {
        ps += qv[j] * to_f32(kr[d]);
        pd += dov[j] * to_f32(vr[d]);
      }
    }
    const float p = expf(wave_sum(ps) * a.scale - lse);
    const float ds = p * (wave_sum(pd) - dl);
#pragma unroll
    for (int j = 0; j < PL; ++j) {
      const int d = lane + 64 * j;
      if (d < D) acc[j] += ds * to_f32(kr[d]);
    }
  }
  T* out = (T*)a.dq + b * a.sdq_b + h * a.sdq_h + (int64_t)qrow * a.sdq_s;
#pragma unroll
  for (int j = 0; j < PL; ++j) {
    const int d = lane + 64 * j;
    if (d < D) out[d] = from_f32<T>(acc[j] * a.scale);
  }
}

template <typename T, int PL>
__global__ void __launch_bounds__(64)
attn_bwd_dkdv_simt(BwdArgs a, int D) {
  const int lane = threadIdx.x;
  const int64_t row = blockIdx.x;  // over B * Hkv * Tkv
  const int kv = (int)(row % a.Tkv);
  const int64_t bhk = row / a.Tkv;
  const int b = (int)(bhk / a.Hkv), hk = (int)(bhk % a.Hkv);
  const int group = a.H / a.Hkv;
  const T* kr = (const T*)a.k + b * a.sk_b + hk * a.sk_h + (int64_t)kv * a.sk_s;
  const T* vr = (const T*)a.v + b * a.sv_b + hk * a.sv_h + (int64_t)kv * a.sv_s;
  float kv_k[PL], kv_v[PL], dk[PL], dv[PL];
#pragma unroll
  for (int j = 0; j < PL; ++j) {
    const int d = lane + 64 * j;
    kv_k[j] = d < D ? to_f32(kr[d]) : 0.f;
    kv_v[j] = d < D ? to_f32(vr[d]) : 0.f;
    dk[j] = dv[j] = 0.f;
  }
  for (int hq = hk * group; hq < (hk + 1) * group; ++hq) {
    const T* qp = (const T*)a.q + b * a.sq_b + hq * a.sq_h;
    const T* dop = (const T*)a.dout + b * a.sdo_b + hq * a.sdo_h;
    const int64_t rbase = ((int64_t)b * a.H + hq) * a.Tq;
    for (int q = a.causal ? kv : 0; q < a.Tq; ++q) {
      const T* qr = qp + (int64_t)q * a.sq_s;
      const T* dr = dop + (int64_t)q * a.sdo_s;
      float ps = 0.f, pd = 0.f;
#pragma unroll
      for (int j = 0; j < PL; ++j) {
        const int d = lane + 64 * j;
        if (d < D) {
          ps += to_f32(qr[d]) * kv_k[j];
          pd += to_f32(dr[d]) * kv_v[j];
        }
      }
      const float p = expf(wave_sum(ps) * a.scale - a.lse[rbase + q]);
      const float ds = p * (wave_sum(pd) - a.delta[rbase + q]);
#pragma unroll
      for (int j = 0; j < PL; ++j) {
        const int d = lane + 64 * j;
        if (d < D) {
          dv[j] += p * to_f32(dr[d]);
          dk[j] += ds * to_f32(qr[d]);
        }
      }
    }
  }
  T* dko = (T*)a.dk + b * a.sdk_b + hk * a.sdk_h + (int64_t)kv * a.sdk_s;
  T* dvo = (T*)a.dv + b * a.sdv_b + hk * a.sdv_h + (int64_t)kv * a.sdv_s;
#pragma unroll
  for (int j = 0; j < PL; ++j) {
    const int d = lane + 64 * j;
    if (d < D) {
      dko[d] = from_f32<T>(dk[j] * a.scale);
      dvo[d] = from_f32<T>(dv[j]);
    }
  }
}

// ------------------------------------------------------------- host side --
bool mfma_head_dim(int64_t d) { return d == 16 || d == 32 || d == 64 || d == 128 || d == 256; }

int simt_per_lane(int64_t d) {
  int pl = 1;
  while (pl * 64 < d) pl *= 2;
  return pl;
}

#define TRI_SIMT_SWITCH(pl, LAUNCH)                                   \
  switch (pl) {                                                       \
    case 1: LAUNCH(1); break;  case 2: LAUNCH(2); break;              \
    case 4: LAUNCH(4); break;  case 8: LAUNCH(8); break;              \
    case 16: LAUNCH(16); break;                                       \
    default: return fail(TRI_EINVAL, "attention: head_dim too large"); \
  }

#define TRI_HEAD_DIM_SWITCH(d, LAUNCH)                                \
  switch (d) {                                                        \
    case 16: LAUNCH(16); break;  case 32: LAUNCH(32); break;          \
    case 64: LAUNCH(64); break;  case 128: LAUNCH(128); break;        \
    default: return fail(TRI_EINVAL, "attention: no MFMA kernel for head_dim %d", (int)d); \
  }

template <typename T>
int fwd_mfma(const FwdArgs& a, int64_t D, hipStream_t st) {
  // The ping-pong kernel (one 8-wavefront workgroup per CU, two 256-row
  // query tiles each) measured faster than attn_fwd_v2 only for D = 128
  // with at least 4 workgroups per CU; with fewer the CUs run out of
  // workgroups, and for D = 64 its MFMA phase is too short to hide the
  // softmax.
  if (D == 128) {
    FwdArgs x = a;
    x.n_tiles = (int)cdiv(a.Tq, kPPBM);
    const int64_t blocks = (int64_t)((x.n_tiles + 1) / 2) * a.B * a.H;  // tile pairs
    if (blocks >= 4 * (int64_t)cu_count()) {
      attn_fwd_pp<T, 128><<<(unsigned)blocks, 64 * kPPWaves, 0, st>>>(x);
      return check_launch("attention forward (mfma)");
    }
  }
  if (D == 64 || D == 128 || D == 256) {
    FwdArgs x = a;
    x.n_tiles = (int)cdiv(a.Tq, kF2BM);
    const int64_t blocks = (int64_t)x.n_tiles * a.B * a.H;
    if (D == 256)
      attn_fwd_v2<T, 256><<<(unsigned)blocks, 64 * kF2Waves, 0, st>>>(x);
    else if (D == 128)
      attn_fwd_v2<T, 128><<<(unsigned)blocks, 64 * kF2Waves, 0, st>>>(x);
    else
      attn_fwd_v2<T, 64><<<(unsigned)blocks, 64 * kF2Waves, 0, st>>>(x);
    return check_launch("attention forward (mfma)");
  }
  FwdArgs x = a;
  x.n_tiles = (int)cdiv(a.Tq, kFwdBM);
  const int64_t blocks = (int64_t)x.n_tiles * a.B * a.H;
#define LAUNCH(DD) attn_fwd_mfma<T, DD><<<(unsigned)blocks, 256, 0, st>>>(x)
  TRI_HEAD_DIM_SWITCH(D, LAUNCH)
#undef LAUNCH
  return check_launch("attention forward (mfma)");
}

template <typename T>
int fwd_simt(const FwdArgs& a, int64_t D, hipStream_t st) {
  const int64_t rows = (int64_t)a.B * a.H * a.Tq;
#define LAUNCH(PL) attn_fwd_simt<T, PL><<<(unsigned)rows, 64, 0, st>>>(a, (int)D)
  TRI_SIMT_SWITCH(simt_per_lane(D), LAUNCH)
#undef LAUNCH
  return check_launch("attention forward (simt)");
}

// Wavefronts per workgroup of the one-role dK/dV and the dQ kernels (8
// measured no faster at the GPT block's shape; dQ 7% slower).
constexpr int kDkvWaves = 4, kDqWaves = 4;

// The dK/dV pair kernel over x.n_tiles kv tiles of every (batch, kv head):
// persistent (one workgroup per compute unit) when the (batch, kv head)s
// split evenly over the XCDs and there are at least two items per compute
// unit, else one workgroup per item.
template <typename T, int D, bool DS>
int launch_dkdv_pair(const BwdArgs& x, hipStream_t st) {
  const int64_t n_bhk = (int64_t)x.B * x.Hkv;
  const int64_t items = n_bhk * x.n_tiles;
  const int cus = cu_count();
  if (n_bhk % kXcds == 0 && cus % kXcds == 0 && items >= 2 * (int64_t)cus)
    attn_bwd_dkdv_pair<T, D, DS, true><<<(unsigned)cus, 64 * kPairWaves, 0, st>>>(x);
  else
    attn_bwd_dkdv_pair<T, D, DS, false><<<(unsigned)items, 64 * kPairWaves, 0, st>>>(x);
  return check_launch(DS ? "attention backward (dk/dv storing ds)"
                         : "attention backward (dk/dv, mfma pairs)");
}

// Stored-dS path (head_dim 128): delta (and with RoPE the rotated q), then
// dK/dV storing dS, then dQ from the stored dS.  (At head_dim 64 the
// recompute costs half as much and the stored path measured slower: GPT
// config-5 layer 0.319 against 0.297 ms.)
template <typename T, int D>
int bwd_ds(const BwdArgs& a, hipStream_t st) {
  BwdArgs x = a;
  const int64_t rows = (int64_t)a.B * a.H * a.Tq;
  attn_bwd_delta_v<T, D><<<(unsigned)cdiv(rows, 256 / (D / 8)), 256, 0, st>>>(x);
  if (int e = check_launch("attention backward (delta)")) return e;
  if (a.rope.cos != nullptr) {  // dK/dV take the rotated q
    x.q = a.q_rot;
    x.sq_s = D;
    x.sq_h = (int64_t)a.Tq * D;
    x.sq_b = (int64_t)a.H * a.Tq * D;
  }
  static_assert(D == 128, "stored-dS backward: head_dim 128");
  x.n_tiles = (int)cdiv(a.Tkv, kPairBN);
  if (int e = launch_dkdv_pair<T, D, true>(x, st)) return e;
  x.q = a.q;  // dQ from dS reads K and dS only; the row strides of q stay the caller's
  x.sq_s = a.sq_s;
  x.sq_h = a.sq_h;
  x.sq_b = a.sq_b;
  x.n_tiles = (int)cdiv(cdiv(a.Tq, 64), kDsTiles);
  const int64_t q_blocks = (int64_t)x.n_tiles * a.B * a.H;
  attn_bwd_dq_ds<T, D><<<(unsigned)q_blocks, 64 * kDsWaves, 0, st>>>(x);
  return check_launch("attention backward (dq from stored ds)");
}

// dQ first: it also computes delta, which the dK/dV kernel reads.
template <typename T, int D>
int bwd_v2(const BwdArgs& a, hipStream_t st) {
  constexpr int WK = kDkvWaves, WQ = kDqWaves;
  if constexpr (D == 128) {
    if (a.ds != nullptr) return bwd_ds<T, D>(a, st);
  }
  BwdArgs x = a;
  x.n_tiles = (int)cdiv(a.Tq, 32 * WQ);
  const int64_t q_blocks = (int64_t)x.n_tiles * a.B * a.H;
  attn_bwd_dq_v2<T, D, WQ><<<(unsigned)q_blocks, 64 * WQ, 0, st>>>(x);
  if (int e = check_launch("attention backward (dq, mfma)")) return e;
  if (a.rope.cos != nullptr) {  // dK/dV take the rotated q the dQ kernel wrote
    x.q = a.q_rot;
    x.sq_s = D;
    x.sq_h = (int64_t)a.Tq * D;
    x.sq_b = (int64_t)a.H * a.Tq * D;
  }
  // head_dim 128: wavefront pairs; head_dim 64 has half the MFMAs per tile
  // for the same VALU work, and one wavefront doing both roles with its
  // K and V fragments (attn_bwd_dkdv_v2) measured faster there (0.27 vs
  // 0.30 ms at [16, 12, 1024, 64], 1.35 vs 1.60 ms at [4, 32, 4096, 64])
  if constexpr (D == 128) {
    x.n_tiles = (int)cdiv(a.Tkv, kPairBN);
    return launch_dkdv_pair<T, D, false>(x, st);
  }
  x.n_tiles = (int)cdiv(a.Tkv, 32 * WK);
  const int64_t kv_blocks = (int64_t)x.n_tiles * a.B * a.Hkv;
  if constexpr (D == 256) {  // dV, then dK: one pass does not fit the registers
    attn_bwd_dkdv_v2<T, D, WK, 1><<<(unsigned)kv_blocks, 64 * WK, 0, st>>>(x);
    if (int e = check_launch("attention backward (dv, mfma)")) return e;
    attn_bwd_dkdv_v2<T, D, WK, 2><<<(unsigned)kv_blocks, 64 * WK, 0, st>>>(x);
    return check_launch("attention backward (dk, mfma)");
  } else {
    attn_bwd_dkdv_v2<T, D, WK><<<(unsigned)kv_blocks, 64 * WK, 0, st>>>(x);
    return check_launch("attention backward (dk/dv, mfma)");
  }
}

template <typename T>
int bwd_mfma(const BwdArgs& a, int64_t D, hipStream_t st) {
  BwdArgs x = a;
  x.n_tiles = (int)cdiv(a.Tkv, kDkvBN);
  const int64_t kv_blocks = (int64_t)x.n_tiles * a.B * a.Hkv;
#define LAUNCH(DD) attn_bwd_dkdv_mfma<T, DD><<<(unsigned)kv_blocks, 256, 0, st>>>(x)
  TRI_HEAD_DIM_SWITCH(D, LAUNCH)
#undef LAUNCH
  if (int e = check_launch("attention backward (dk/dv, mfma)")) return e;
  x.n_tiles = (int)cdiv(a.Tq, kDqBM);
  const int64_t q_blocks = (int64_t)x.n_tiles * a.B * a.H;
#define LAUNCH(DD) attn_bwd_dq_mfma<T, DD><<<(unsigned)q_blocks, 256, 0, st>>>(x)
  TRI_HEAD_DIM_SWITCH(D, LAUNCH)
#undef LAUNCH
  return check_launch("attention backward (dq, mfma)");
}

template <typename T>
int bwd_impl(const BwdArgs& a, int64_t D, bool mfma, hipStream_t st) {
  if constexpr (!std::is_same<T, float>::value) {
    if (mfma && D == 256) return bwd_v2<T, 256>(a, st);
    if (mfma && D == 128) return bwd_v2<T, 128>(a, st);
    if (mfma && D == 64) return bwd_v2<T, 64>(a, st);
  }
  const int64_t rows = (int64_t)a.B * a.H * a.Tq;
  attn_bwd_delta<T><<<(unsigned)cdiv(rows, 4), 256, 0, st>>>(a, (int)D);
  if (int e = check_launch("attention backward (delta)")) return e;
  if constexpr (!std::is_same<T, float>::value) {
    if (mfma) return bwd_mfma<T>(a, D, st);
  }
  const int64_t kv_rows = (int64_t)a.B * a.Hkv * a.Tkv;
  const int pl = simt_per_lane(D);
#define LAUNCH(PL) attn_bwd_dq_simt<T, PL><<<(unsigned)rows, 64, 0, st>>>(a, (int)D)
  TRI_SIMT_SWITCH(pl, LAUNCH)
#undef LAUNCH
  if (int e = check_launch("attention backward (dq, simt)")) return e;
#define LAUNCH(PL) attn_bwd_dkdv_simt<T, PL><<<(unsigned)kv_rows, 64, 0, st>>>(a, (int)D)
  TRI_SIMT_SWITCH(pl, LAUNCH)
#undef LAUNCH
  return check_launch("attention backward (dk/dv, simt)");
}

// Row strides must keep 16-byte alignment of every row for the MFMA path.
bool rows_aligned(const void* p, int64_t sb, int64_t sh, int64_t ss) {
  return aligned16(p) && sb % 8 == 0 && sh % 8 == 0 && ss % 8 == 0;
}

int check_dims(int64_t B, int64_t H, int64_t Hkv, int64_t Tq, int64_t Tkv, int64_t D) {
  if (B < 0 || H <= 0 || Hkv <= 0 || H % Hkv != 0 || Tq < 0 || Tkv < 0 || D <= 0)
    return fail(TRI_EINVAL, "attention: bad shape B=%lld H=%lld Hkv=%lld Tq=%lld Tkv=%lld D=%lld",
                (long long)B, (long long)H, (long long)Hkv, (long long)Tq, (long long)Tkv,
                (long long)D);
  if (D > 64 * kSimtMaxPerLane)
    return fail(TRI_EINVAL, "attention: head_dim %lld exceeds %d", (long long)D,
                64 * kSimtMaxPerLane);
  if (B * H * Tq >= ((int64_t)1 << 31) || B * Hkv * Tkv >= ((int64_t)1 << 31) ||
      Tq >= ((int64_t)1 << 30) || Tkv >= ((int64_t)1 << 30))
    return fail(TRI_EINVAL, "attention: problem too large");
  return TRI_OK;
}

}  // namespace
}  // namespace tri

using namespace tri;

namespace {

// tritium_attention_fwd / _fwd_rope: rope.cos == nullptr leaves q as given
int attention_fwd(const void* q, const void* k, const void* v, void* o, float* lse, int64_t B,
                  int64_t H, int64_t Hkv, int64_t Tq, int64_t Tkv, int64_t D,
                  const int64_t* strides, int causal, int dtype, const RopeQ& rope,
                  void* stream) {
  if (int e = check_dims(B, H, Hkv, Tq, Tkv, D)) return e;
  if (B == 0 || Tq == 0) return TRI_OK;
  FwdArgs a;
  a.q = q; a.k = k; a.v = v; a.o = o; a.lse = lse;
  a.sq_b = strides[0]; a.sq_h = strides[1]; a.sq_s = strides[2];
  a.sk_b = strides[3]; a.sk_h = strides[4]; a.sk_s = strides[5];
  a.sv_b = strides[6]; a.sv_h = strides[7]; a.sv_s = strides[8];
  a.so_b = strides[9]; a.so_h = strides[10]; a.so_s = strides[11];
  a.B = (int)B; a.H = (int)H; a.Hkv = (int)Hkv; a.Tq = (int)Tq; a.Tkv = (int)Tkv;
  a.causal = causal != 0;
  a.n_tiles = 0;
  a.scale = (float)(1.0 / sqrt((double)D));
  a.rope = rope;
  hipStream_t st = (hipStream_t)stream;
  const bool mfma = dtype != kF32 && mfma_head_dim(D) &&
                    rows_aligned(q, a.sq_b, a.sq_h, a.sq_s) &&
                    rows_aligned(k, a.sk_b, a.sk_h, a.sk_s) &&
                    rows_aligned(v, a.sv_b, a.sv_h, a.sv_s) && aligned16(o) &&
                    a.so_s % 4 == 0 && a.so_b % 4 == 0 && a.so_h % 4 == 0;
  if (rope.cos != nullptr && !(mfma && (D == 64 || D == 128)))
    return fail(TRI_EINVAL, "attention with rope: needs 16-bit q/k/v with head_dim 64 or 128 and "
                "16-byte aligned rows (dtype %d, head_dim %lld)", dtype, (long long)D);
  if (mfma) {
    if (dtype == kBF16) return fwd_mfma<bf16_t>(a, D, st);
    return fwd_mfma<f16_t>(a, D, st);
  }
  TRI_DISPATCH_FLOAT(dtype, T, return fwd_simt<T>(a, D, st));
  return TRI_OK;
}

// Bytes of the stored-dS workspace (0: the shape does not take that path).
size_t ds_workspace_bytes(int64_t B, int64_t H, int64_t Tq, int64_t Tkv, int64_t D, int causal,
                          int dtype) {
  if (dtype == kF32 || D != 128 || B <= 0 || H <= 0 || Tq <= 0 || Tkv <= 0) return 0;
  if (Tq >= ((int64_t)1 << 30) || Tkv >= ((int64_t)1 << 30)) return 0;
  const int64_t per_bh = ds_row(causal != 0, (int)cdiv(Tq, 64), (int)cdiv(Tkv, 64)) * 4096;
  return (size_t)(B * H) * (size_t)per_bh * 2;
}

int attention_bwd(const void* dout, const void* q, const void* k, const void* v, const void* o,
                  const float* lse, void* dq, void* dk, void* dv, float* delta, int64_t B,
                  int64_t H, int64_t Hkv, int64_t Tq, int64_t Tkv, int64_t D,
                  const int64_t* strides, int causal, int dtype, const RopeQ& rope, void* q_rot,
                  void* ds_ws, size_t ds_bytes, void* stream) {
  if (int e = check_dims(B, H, Hkv, Tq, Tkv, D)) return e;
  if (B == 0 || Tq == 0 || Tkv == 0) return TRI_OK;
  BwdArgs a;
  a.q = q; a.k = k; a.v = v; a.o = o; a.dout = dout; a.lse = lse; a.delta = delta;
  a.dq = dq; a.dk = dk; a.dv = dv;
  a.sq_b = strides[0]; a.sq_h = strides[1]; a.sq_s = strides[2];
  a.sk_b = strides[3]; a.sk_h = strides[4]; a.sk_s = strides[5];
  a.sv_b = strides[6]; a.sv_h = strides[7]; a.sv_s = strides[8];
  a.so_b = strides[9]; a.so_h = strides[10]; a.so_s = strides[11];
  a.sdo_b = strides[12]; a.sdo_h = strides[13]; a.sdo_s = strides[14];
  a.sdq_b = strides[15]; a.sdq_h = strides[16]; a.sdq_s = strides[17];
  a.sdk_b = strides[18]; a.sdk_h = strides[19]; a.sdk_s = strides[20];
  a.sdv_b = strides[21]; a.sdv_h = strides[22]; a.sdv_s = strides[23];
  a.B = (int)B; a.H = (int)H; a.Hkv = (int)Hkv; a.Tq = (int)Tq; a.Tkv = (int)Tkv;
  a.causal = causal != 0;
  a.n_tiles = 0;
  a.scale = (float)(1.0 / sqrt((double)D));
  a.rope = rope;
  a.q_rot = q_rot;
  a.ds = nullptr;
  a.ds_bh = 0;
  const bool out_ok = [&] {
    const int64_t* s = strides + 15;
    for (int i = 0; i < 9; ++i)
      if (s[i] % 4 != 0) return false;
    return aligned16(dq) && aligned16(dk) && aligned16(dv);
  }();
  const bool mfma = dtype != kF32 && mfma_head_dim(D) &&
                    rows_aligned(q, a.sq_b, a.sq_h, a.sq_s) &&
                    rows_aligned(k, a.sk_b, a.sk_h, a.sk_s) &&
                    rows_aligned(v, a.sv_b, a.sv_h, a.sv_s) &&
                    rows_aligned(dout, a.sdo_b, a.sdo_h, a.sdo_s) &&
                    rows_aligned(o, a.so_b, a.so_h, a.so_s) && out_ok;
  hipStream_t st = (hipStream_t)stream;
  if (rope.cos != nullptr) {
    if (!(mfma && (D == 64 || D == 128)))
      return fail(TRI_EINVAL, "attention backward with rope: needs 16-bit tensors with head_dim "
                  "64 or 128 and 16-byte aligned rows (dtype %d, head_dim %lld)", dtype,
                  (long long)D);
    if (q_rot == nullptr || !aligned16(q_rot))
      return fail(TRI_EINVAL, "attention backward with rope: q_rot workspace missing or unaligned");
  }
  if (ds_ws != nullptr && mfma) {
    const size_t need = ds_workspace_bytes(B, H, Tq, Tkv, D, causal, dtype);
    if (need > 0) {
      if (ds_bytes < need || !aligned16(ds_ws))
        return fail(TRI_EINVAL, "attention backward: dS workspace of %zu bytes (need %zu, "
                    "16-byte aligned)", ds_bytes, need);
      a.ds = ds_ws;
      a.ds_bh = (int64_t)(need / 2 / (size_t)(B * H));
    }
  }
  TRI_DISPATCH_FLOAT(dtype, T, return bwd_impl<T>(a, D, mfma, st));
  return TRI_OK;
}

int rope_tables(const float* cos_table, const float* sin_table, const void* position_ids,
                int position_kind, int64_t max_position, RopeQ& r) {
  if (cos_table == nullptr || sin_table == nullptr || max_position < 0 || position_kind < 0 ||
      position_kind > 2 || (position_kind != 0 && position_ids == nullptr))
    return fail(TRI_EINVAL, "attention rope: bad tables or position_ids (kind %d)", position_kind);
  r.cos = cos_table;
  r.sin = sin_table;
  r.pos = position_ids;
  r.kind = position_kind;
  r.max_pos = max_position;
  return TRI_OK;
}

}  // namespace

extern "C" int tritium_attention_fwd(const void* q, const void* k, const void* v, void* o,
                                     float* lse, int64_t B, int64_t H, int64_t Hkv, int64_t Tq,
                                     int64_t Tkv, int64_t D, const int64_t* strides, int causal,
                                     int dtype, void* stream) {
  return attention_fwd(q, k, v, o, lse, B, H, Hkv, Tq, Tkv, D, strides, causal, dtype, RopeQ{},
                       stream);
}

extern "C" int tritium_attention_bwd(const void* dout, const void* q, const void* k,
                                     const void* v, const void* o, const float* lse, void* dq,
                                     void* dk, void* dv, float* delta, int64_t B, int64_t H,
                                     int64_t Hkv, int64_t Tq, int64_t Tkv, int64_t D,
                                     const int64_t* strides, int causal, int dtype,
                                     void* stream) {
  return attention_bwd(dout, q, k, v, o, lse, dq, dk, dv, delta, B, H, Hkv, Tq, Tkv, D, strides,
                       causal, dtype, RopeQ{}, nullptr, nullptr, 0, stream);
}

extern "C" size_t tritium_attention_bwd_workspace_size(int64_t B, int64_t H, int64_t Tq,
                                                       int64_t Tkv, int64_t D, int causal,
                                                       int dtype) {
  return ds_workspace_bytes(B, H, Tq, Tkv, D, causal, dtype);
}

extern "C" int tritium_attention_bwd_ws(const void* dout, const void* q, const void* k,
                                        const void* v, const void* o, const float* lse, void* dq,
                                        void* dk, void* dv, float* delta, void* workspace,
                                        size_t workspace_bytes, int64_t B, int64_t H, int64_t Hkv,
                                        int64_t Tq, int64_t Tkv, int64_t D,
                                        const int64_t* strides, int causal, int dtype,
                                        void* stream) {
  return attention_bwd(dout, q, k, v, o, lse, dq, dk, dv, delta, B, H, Hkv, Tq, Tkv, D, strides,
                       causal, dtype, RopeQ{}, nullptr, workspace, workspace_bytes, stream);
}

extern "C" int tritium_attention_fwd_rope(const void* q, const void* k, const void* v, void* o,
                                          float* lse, int64_t B, int64_t H, int64_t Hkv,
                                          int64_t Tq, int64_t Tkv, int64_t D,
                                          const int64_t* strides, int causal, int dtype,
                                          const float* cos_table, const float* sin_table,
                                          const void* position_ids, int position_kind,
                                          int64_t max_position, void* stream) {
  RopeQ r{};
  if (int e = rope_tables(cos_table, sin_table, position_ids, position_kind, max_position, r))
    return e;
  return attention_fwd(q, k, v, o, lse, B, H, Hkv, Tq, Tkv, D, strides, causal, dtype, r, stream);
}

extern "C" int tritium_attention_bwd_rope(const void* dout, const void* q, const void* k,
                                          const void* v, const void* o, const float* lse,
                                          void* dq, void* dk, void* dv, float* delta,
                                          void* q_rot, int64_t B, int64_t H, int64_t Hkv,
                                          int64_t Tq, int64_t Tkv, int64_t D,
                                          const int64_t* strides, int causal, int dtype,
                                          const float* cos_table, const float* sin_table,
                                          const void* position_ids, int position_kind,
                                          int64_t max_position, void* stream) {
  RopeQ r{};
  if (int e = rope_tables(cos_table, sin_table, position_ids, position_kind, max_position, r))
    return e;
  return attention_bwd(dout, q, k, v, o, lse, dq, dk, dv, delta, B, H, Hkv, Tq, Tkv, D, strides,
                       causal, dtype, r, q_rot, nullptr, 0, stream);
}

extern "C" int tritium_attention_bwd_rope_ws(
    const void* dout, const void* q, const void* k, const void* v, const void* o,
    const float* lse, void* dq, void* dk, void* dv, float* delta, void* q_rot, void* workspace,
    size_t workspace_bytes, int64_t B, int64_t H, int64_t Hkv, int64_t Tq, int64_t Tkv, int64_t D,
    const int64_t* strides, int causal, int dtype, const float* cos_table,
    const float* sin_table, const void* position_ids, int position_kind, int64_t max_position,
    void* stream) {
  RopeQ r{};
  if (int e = rope_tables(cos_table, sin_table, position_ids, position_kind, max_position, r))
    return e;
  return attention_bwd(dout, q, k, v, o, lse, dq, dk, dv, delta, B, H, Hkv, Tq, Tkv, D, strides,
                       causal, dtype, r, q_rot, workspace, workspace_bytes, stream);
}

extern "C" size_t tritium_attention_decode_workspace_size(int64_t B, int64_t H, int64_t Hkv,
                                                          int64_t Tkv, int64_t D) {
  if (B <= 0 || H <= 0 || Hkv <= 0 || Tkv <= 0 || D <= 0) return 0;
  return (size_t)B * H * dec_splits(B, Hkv, Tkv) * (D + 2) * sizeof(float);
}

namespace {

int decode_launch(const void* q, const void* k, const void* v, void* o, float* lse,
                  void* workspace, size_t workspace_bytes, int64_t B, int64_t H, int64_t Hkv,
                  int64_t Tkv, int64_t D, const int64_t* strides, int dtype, void* stream) {
  if (int e = check_dims(B, H, Hkv, 1, Tkv, D)) return e;
  if (B == 0) return TRI_OK;
  if (Tkv < 1) return fail(TRI_EINVAL, "attention decode: needs at least one key");
  if (dtype == kF32 || (D != 64 && D != 128))
    return fail(TRI_EINVAL, "attention decode: 16-bit inputs with head_dim 64 or 128 only");
  const int64_t group = H / Hkv;
  if (group > 8) return fail(TRI_EINVAL, "attention decode: at most 8 query heads per kv head");
  DecArgs a;
  a.q = q; a.k = k; a.v = v; a.o = o; a.lse = lse; a.part = (float*)workspace;
  a.sq_b = strides[0]; a.sq_h = strides[1];
  a.sk_b = strides[3]; a.sk_h = strides[4]; a.sk_s = strides[5];
  a.sv_b = strides[6]; a.sv_h = strides[7]; a.sv_s = strides[8];
  a.so_b = strides[9]; a.so_h = strides[10];
  if (!aligned16(q) || a.sq_b % 8 || a.sq_h % 8 || !rows_aligned(k, a.sk_b, a.sk_h, a.sk_s) ||
      !rows_aligned(v, a.sv_b, a.sv_h, a.sv_s))
    return fail(TRI_EINVAL, "attention decode: q, k, v rows must be 16-byte aligned");
  a.B = (int)B; a.H = (int)H; a.Hkv = (int)Hkv; a.Tkv = (int)Tkv;
  a.n_splits = dec_splits(B, Hkv, Tkv);
  const int step = kDecWaves * (64 / (int)(D / 8));
  a.chunk = (int)(cdiv(cdiv(Tkv, a.n_splits), step) * step);
  a.sl2 = (float)(1.0 / sqrt((double)D)) * kLog2e;
  const size_t need = (size_t)B * H * a.n_splits * (D + 2) * sizeof(float);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(TRI_EINVAL, "attention decode: workspace of %zu bytes needed", need);
  const int64_t blocks = B * Hkv * a.n_splits;
  if (blocks >= ((int64_t)1 << 31)) return fail(TRI_EINVAL, "attention decode: grid too large");
  hipStream_t st = (hipStream_t)stream;
#define TRI_DEC_LAUNCH(TT, DD, GG) \
  attn_decode_kernel<TT, DD, GG><<<(unsigned)blocks, 64 * kDecWaves, 0, st>>>(a)
#define TRI_DEC_GROUPS(TT, DD)                        \
  do {                                                \
    if (group == 1) TRI_DEC_LAUNCH(TT, DD, 1);        \
    else if (group == 2) TRI_DEC_LAUNCH(TT, DD, 2);   \
    else if (group <= 4) TRI_DEC_LAUNCH(TT, DD, 4);   \
    else TRI_DEC_LAUNCH(TT, DD, 8);                   \
  } while (0)
  if (dtype == kBF16) {
    if (D == 64) TRI_DEC_GROUPS(bf16_t, 64); else TRI_DEC_GROUPS(bf16_t, 128);
  } else {
    if (D == 64) TRI_DEC_GROUPS(f16_t, 64); else TRI_DEC_GROUPS(f16_t, 128);
  }
#undef TRI_DEC_GROUPS
#undef TRI_DEC_LAUNCH
  if (int e = check_launch("attention decode")) return e;
  if (a.n_splits == 1) return TRI_OK;  // the decode kernel wrote o and lse
  if (dtype == kBF16) {
    if (D == 64) attn_decode_combine<bf16_t, 64><<<(unsigned)(B * H), 64, 0, st>>>(a);
    else attn_decode_combine<bf16_t, 128><<<(unsigned)(B * H), 128, 0, st>>>(a);
  } else {
    if (D == 64) attn_decode_combine<f16_t, 64><<<(unsigned)(B * H), 64, 0, st>>>(a);
    else attn_decode_combine<f16_t, 128><<<(unsigned)(B * H), 128, 0, st>>>(a);
  }
  return check_launch("attention decode combine");
}

}  // namespace

// Scratch of the no-allocation decode entry: the chunks' partial (m, l, o)
// rows, one copy per GPU, resident until the process ends.  Every partial
// row a call reads was written by the same call's first kernel, so nothing
// has to be cleared between calls.  On the host, `scratch` names a host-side
// stand-in; kernels get the device address from hipGetSymbolAddress.
constexpr size_t kDecScratchBytes = size_t(32) << 20;
static __device__ __align__(256) float scratch[kDecScratchBytes / sizeof(float)];

namespace {

constexpr int kMaxDevices = 64;
std::atomic<float*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// The device address of `scratch` on the current device, looked up once per
// device (with that device current) and kept.  `stream` must belong to the
// current device, or the kernels would run on another GPU than the address.
int decode_scratch(void* stream, float** out) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess)
    return fail(TRI_ELAUNCH, "attention decode (no-alloc): hipGetDevice: %s", hipGetErrorString(err));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(TRI_EINVAL, "attention decode (no-alloc): device %d beyond %d", dev, kMaxDevices);
  if (stream != nullptr) {
    int sdev = dev;
    err = hipStreamGetDevice((hipStream_t)stream, &sdev);
    if (err != hipSuccess)
      return fail(TRI_ELAUNCH, "attention decode (no-alloc): hipStreamGetDevice: %s",
                  hipGetErrorString(err));
    if (sdev != dev)
      return fail(TRI_EINVAL,
                  "attention decode (no-alloc): the stream belongs to device %d but device %d is current",
                  sdev, dev);
  }
  float* ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (ptr == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    ptr = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (ptr == nullptr) {
      void* p = nullptr;
      err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (err != hipSuccess || p == nullptr)
        return fail(TRI_ELAUNCH, "attention decode (no-alloc): hipGetSymbolAddress: %s",
                    hipGetErrorString(err));
      ptr = (float*)p;
      g_scratch_ptr[dev].store(ptr, std::memory_order_release);
    }
  }
  *out = ptr;
  return TRI_OK;
}

}  // namespace

extern "C" int tritium_attention_decode(const void* q, const void* k, const void* v, void* o,
                                        float* lse, void* workspace, size_t workspace_bytes,
                                        int64_t B, int64_t H, int64_t Hkv, int64_t Tkv, int64_t D,
                                        const int64_t* strides, int dtype, void* stream) {
  return decode_launch(q, k, v, o, lse, workspace, workspace_bytes, B, H, Hkv, Tkv, D, strides,
                       dtype, stream);
}

extern "C" size_t tritium_attention_decode_noalloc_max_bytes(void) { return kDecScratchBytes; }

extern "C" int tritium_attention_decode_noalloc(const void* q, const void* k, const void* v,
                                                void* o, float* lse, int64_t B, int64_t H,
                                                int64_t Hkv, int64_t Tkv, int64_t D,
                                                const int64_t* strides, int dtype, void* stream) {
  if (int e = check_dims(B, H, Hkv, 1, Tkv, D)) return e;
  if (B == 0) return TRI_OK;
  const size_t need = tritium_attention_decode_workspace_size(B, H, Hkv, Tkv, D);
  if (need > kDecScratchBytes)
    return fail(TRI_EINVAL,
                "attention decode (no-alloc): %zu bytes of partials needed, more than its %zu-byte "
                "scratch; use tritium_attention_decode with a workspace",
                need, kDecScratchBytes);
  float* part = nullptr;
  if (int e = decode_scratch(stream, &part)) return e;
  return decode_launch(q, k, v, o, lse, part, kDecScratchBytes, B, H, Hkv, Tkv, D, strides, dtype,
                       stream);
}
