// Rotary position embedding (forward rotation and its inverse) for gfx950.
//
// Reference arithmetic: alkinun/helion tritium/ops/rope.py:42-90.  The
// position of token t is position_ids[t] + offset, or t + offset; pairs are
// (x[i], x[i+half]) or, interleaved, (x[2i], x[2i+1]); forward
// (a*c - b*s, b*c + a*s), inverse (a*c + b*s, b*c - a*s); fp32 math, result
// stored in the input dtype.
//
// One lane rotates P pairs of q AND the same P pairs of k for one
// (token, head): the cos/sin values it loads serve both tensors, and the 32+
// lanes of a token that read the same cos/sin row hit in L1.  q/k accesses
// are 16-byte vectors when the layout allows it, streamed with the
// nontemporal hint (each element is read and written once).
//
// A position outside [0, max_position) has no table row; the kernel then
// writes NaN for that token instead of reading out of bounds.
//
// Token rows of the inputs and of the outputs each have their own stride
// (elements; heads are adjacent inside a row), so q and k can be read in
// place from a fused [tokens, 3, heads, head_dim] projection and the inverse
// rotation written back into the matching gradient rows.
#include "common.h"
#include "../../include/tritium_hip.h"

namespace tri {
namespace {

constexpr int kBlock = 256;

template <typename T, typename CT, int P>
__global__ void __launch_bounds__(kBlock)
rope_kernel(const T* q, const T* k, const CT* __restrict__ cos_t,
            const CT* __restrict__ sin_t, const void* __restrict__ pos_ids, int pos_kind,
            T* q_out, T* k_out, uint32_t n_items, uint32_t items_per_head, uint32_t n_heads,
            int head_dim, int64_t max_pos, int64_t offset, int interleaved, int inverse,
            int64_t in_ts, int64_t out_ts) {
  const uint32_t item = blockIdx.x * kBlock + threadIdx.x;
  if (item >= n_items) return;
  const uint32_t th = item / items_per_head;
  const uint32_t chunk = item - th * items_per_head;
  const uint32_t token = th / n_heads;
  const int half = head_dim >> 1;

  int64_t pos;
  if (pos_kind == 1) {
    pos = (int64_t)((const int32_t*)pos_ids)[token] + offset;
  } else if (pos_kind == 2) {
    pos = ((const int64_t*)pos_ids)[token] + offset;
  } else {
    pos = (int64_t)token + offset;
  }
  const int64_t hoff = (int64_t)(th - token * n_heads) * head_dim;
  const int64_t base = (int64_t)token * in_ts + hoff;   // q, k
  const int64_t obase = (int64_t)token * out_ts + hoff;  // q_out, k_out
  const bool valid = pos >= 0 && pos < max_pos;

  // The P pairs this lane owns start at pair index p0 (cos/sin column p0).
  const int p0 = (int)chunk * P;
  float c[P] = {}, s[P] = {};
  if (valid) {
    load_f32<CT, P>(cos_t + pos * half + p0, c);
    load_f32<CT, P>(sin_t + pos * half + p0, s);
    if (inverse) {
#pragma unroll
      for (int i = 0; i < P; ++i) s[i] = -s[i];
    }
  }
  const float nan = __builtin_nanf("");

  // q == nullptr: k only (a caller that rotates q elsewhere); qa, qb stay 0
  const bool has_q = q != nullptr;
  if (!interleaved) {
    float qa[P] = {}, qb[P] = {}, ka[P], kb[P];
    if (has_q) {
      load_stream<T, P>(q + base + p0, qa);
      load_stream<T, P>(q + base + half + p0, qb);
    }
    load_stream<T, P>(k + base + p0, ka);
    load_stream<T, P>(k + base + half + p0, kb);
    float oqa[P], oqb[P], oka[P], okb[P];
#pragma unroll
    for (int i = 0; i < P; ++i) {
      rope_pair(qa[i], qb[i], c[i], s[i], oqa[i], oqb[i]);
      rope_pair(ka[i], kb[i], c[i], s[i], oka[i], okb[i]);
      if (!valid) oqa[i] = oqb[i] = oka[i] = okb[i] = nan;
    }
    if (has_q) {
      store_stream<T, P>(q_out + obase + p0, oqa);
      store_stream<T, P>(q_out + obase + half + p0, oqb);
    }
    store_stream<T, P>(k_out + obase + p0, oka);
    store_stream<T, P>(k_out + obase + half + p0, okb);
  } else {
    // elements [2*p0, 2*p0 + 2P) hold P adjacent (a, b) pairs
    float qv[2 * P] = {}, kv[2 * P];
    if (has_q) {
      load_stream<T, P>(q + base + 2 * p0, *reinterpret_cast<float(*)[P]>(qv));
      load_stream<T, P>(q + base + 2 * p0 + P, *reinterpret_cast<float(*)[P]>(qv + P));
    }
    load_stream<T, P>(k + base + 2 * p0, *reinterpret_cast<float(*)[P]>(kv));
    load_stream<T, P>(k + base + 2 * p0 + P, *reinterpret_cast<float(*)[P]>(kv + P));
    float oq[2 * P], ok[2 * P];
#pragma unroll
    for (int i = 0; i < P; ++i) {
      rope_pair(qv[2 * i], qv[2 * i + 1], c[i], s[i], oq[2 * i], oq[2 * i + 1]);
      rope_pair(kv[2 * i], kv[2 * i + 1], c[i], s[i], ok[2 * i], ok[2 * i + 1]);
      if (!valid) oq[2 * i] = oq[2 * i + 1] = ok[2 * i] = ok[2 * i + 1] = nan;
    }
    if (has_q) {
      store_stream<T, P>(q_out + obase + 2 * p0, *reinterpret_cast<float(*)[P]>(oq));
      store_stream<T, P>(q_out + obase + 2 * p0 + P, *reinterpret_cast<float(*)[P]>(oq + P));
    }
    store_stream<T, P>(k_out + obase + 2 * p0, *reinterpret_cast<float(*)[P]>(ok));
    store_stream<T, P>(k_out + obase + 2 * p0 + P, *reinterpret_cast<float(*)[P]>(ok + P));
  }
}

template <typename T, typename CT, int P>
int launch(const void* q, const void* k, const void* cs, const void* sn, const void* pos,
           int pos_kind, void* qo, void* ko, int64_t n_tokens, int64_t n_heads, int64_t head_dim,
           int64_t max_pos, int64_t offset, int interleaved, int inverse, int64_t in_ts,
           int64_t out_ts, hipStream_t stream) {
  const int64_t items_per_head = (head_dim / 2) / P;
  const int64_t n_items = n_tokens * n_heads * items_per_head;
  if (n_items >= ((int64_t)1 << 32) - kBlock)
    return fail(TRI_EINVAL, "rope: too many elements (%lld rotation items)", (long long)n_items);
  rope_kernel<T, CT, P><<<(unsigned)cdiv(n_items, kBlock), kBlock, 0, stream>>>(
      (const T*)q, (const T*)k, (const CT*)cs, (const CT*)sn, pos, pos_kind, (T*)qo, (T*)ko,
      (uint32_t)n_items, (uint32_t)items_per_head, (uint32_t)n_heads, (int)head_dim, max_pos,
      offset, interleaved, inverse, in_ts, out_ts);
  return check_launch("rope");
}

template <typename T, typename CT>
int dispatch_pairs(const void* q, const void* k, const void* cs, const void* sn, const void* pos,
                   int pos_kind, void* qo, void* ko, int64_t n_tokens, int64_t n_heads,
                   int64_t head_dim, int64_t max_pos, int64_t offset, int interleaved,
                   int inverse, int64_t in_ts, int64_t out_ts, hipStream_t stream) {
  // P pairs per lane: 16-byte q/k vectors when every access stays aligned.
  constexpr int PV = 16 / sizeof(T);
  const int64_t half = head_dim / 2;
  const bool ptr_ok = aligned16(q) && aligned16(k) && aligned16(qo) && aligned16(ko) &&
                      in_ts % PV == 0 && out_ts % PV == 0;
  // split layout: offsets p0 and half+p0 (elements) must be multiples of PV, cos/sin
  // offsets pos*half+p0 multiples of PV (CT) -> half % PV == 0 covers all of them.
  // interleaved: offsets 2*p0 and 2*p0+P must be multiples of P -> half % PV == 0.
  const bool tbl_ok = ((uintptr_t)cs % (sizeof(CT) * PV) == 0) &&
                      ((uintptr_t)sn % (sizeof(CT) * PV) == 0);
  if (ptr_ok && tbl_ok && half % PV == 0) {
    return launch<T, CT, PV>(q, k, cs, sn, pos, pos_kind, qo, ko, n_tokens, n_heads, head_dim,
                             max_pos, offset, interleaved, inverse, in_ts, out_ts, stream);
  }
  return launch<T, CT, 1>(q, k, cs, sn, pos, pos_kind, qo, ko, n_tokens, n_heads, head_dim,
                          max_pos, offset, interleaved, inverse, in_ts, out_ts, stream);
}

}  // namespace
}  // namespace tri

using namespace tri;

extern "C" int tritium_rope_strided(const void* q, const void* k, const void* cos_table,
                                    const void* sin_table, const void* position_ids,
                                    int position_kind, void* q_out, void* k_out, int64_t n_tokens,
                                    int64_t n_heads, int64_t head_dim, int64_t max_position,
                                    int64_t position_offset, int interleaved, int inverse,
                                    int64_t in_token_stride, int64_t out_token_stride, int dtype,
                                    int table_dtype, void* stream) {
  if (n_tokens < 0 || n_heads <= 0 || head_dim <= 0 || (head_dim & 1) || max_position < 0)
    return fail(TRI_EINVAL, "rope: bad shape tokens=%lld heads=%lld head_dim=%lld",
                (long long)n_tokens, (long long)n_heads, (long long)head_dim);
  if (in_token_stride < n_heads * head_dim || out_token_stride < n_heads * head_dim)
    return fail(TRI_EINVAL, "rope: token strides %lld/%lld below heads*head_dim %lld",
                (long long)in_token_stride, (long long)out_token_stride,
                (long long)(n_heads * head_dim));
  if (position_kind < 0 || position_kind > 2 || (position_kind != 0 && position_ids == nullptr))
    return fail(TRI_EINVAL, "rope: bad position_ids kind %d", position_kind);
  if ((q == nullptr) != (q_out == nullptr) || k == nullptr || k_out == nullptr)
    return fail(TRI_EINVAL, "rope: k and k_out are required; q and q_out are both given or both null");
  if (n_tokens == 0) return TRI_OK;
  hipStream_t s = (hipStream_t)stream;
  TRI_DISPATCH_FLOAT(dtype, T,
    TRI_DISPATCH_FLOAT(table_dtype, CT,
      return dispatch_pairs<T, CT>(q, k, cos_table, sin_table, position_ids, position_kind,
                                   q_out, k_out, n_tokens, n_heads, head_dim, max_position,
                                   position_offset, interleaved, inverse, in_token_stride,
                                   out_token_stride, s)));
  return TRI_OK;
}

extern "C" int tritium_rope(const void* q, const void* k, const void* cos_table,
                            const void* sin_table, const void* position_ids, int position_kind,
                            void* q_out, void* k_out, int64_t n_tokens, int64_t n_heads,
                            int64_t head_dim, int64_t max_position, int64_t position_offset,
                            int interleaved, int inverse, int dtype, int table_dtype,
                            void* stream) {
  return tritium_rope_strided(q, k, cos_table, sin_table, position_ids, position_kind, q_out,
                              k_out, n_tokens, n_heads, head_dim, max_position, position_offset,
                              interleaved, inverse, n_heads * head_dim, n_heads * head_dim, dtype,
                              table_dtype, stream);
}
