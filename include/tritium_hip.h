/*
 * tritium_hip.h -- C ABI of libtritium_hip.so, the gfx950 (MI355X) kernel
 * library behind the Python `helion_amd` package (a drop-in for the
 * reference's `tritium.ops` layer, alkinun/helion tritium/ops/).
 *
 * Conventions for every entry point:
 *   - all tensor arguments are raw device pointers to densely packed,
 *     row-major data unless a stride argument says otherwise;
 *   - `dtype` codes: 0 = float32, 1 = float16, 2 = bfloat16;
 *   - `stream` is a hipStream_t (torch.cuda.current_stream().cuda_stream);
 *     every call only enqueues work on it and never synchronises;
 *   - the library never allocates device memory: outputs and workspaces come
 *     from the caller (torch's caching allocator on the Python side);
 *   - return value 0 = success, 1 = argument rejected, 2 = HIP launch error;
 *     tritium_last_error() then returns a message (thread-local).
 */
#ifndef TRITIUM_HIP_H_
#define TRITIUM_HIP_H_

#include <stddef.h>
#include <stdint.h>

#define TRITIUM_HIP_ABI_VERSION 1

#ifdef __cplusplus
extern "C" {
#endif

/* ---- library -------------------------------------------------------------
 * Replaces tritium/_compat.py:1-34 (the Triton build shim applied at import):
 * the loader checks these before any kernel call. */
const char* tritium_last_error(void);
int tritium_abi_version(void);
int tritium_runtime_version(void);

/* ---- RMSNorm ---------------------------------------------------------------
 * Forward of tritium.rmsnorm / tritium.residual_rmsnorm
 * (tritium/ops/rmsnorm.py:29-51 `_rmsnorm_forward_kernel`, 54-83
 * `_residual_rmsnorm_forward_kernel`, host side 325-349 and 749-778).
 * x, residual, y, residual_out: [n_rows, hidden] in `dtype`; weight: [hidden]
 * in `dtype`; rstd: [n_rows] float32.  residual and residual_out are both
 * NULL (plain RMSNorm) or both set (y = rmsnorm(x + residual),
 * residual_out = x + residual). */
int tritium_rmsnorm_fwd(const void* x, const void* residual, const void* weight, void* y,
                        void* residual_out, float* rstd, int64_t n_rows, int64_t hidden,
                        float eps, int dtype, void* stream);

/* Workspace bytes tritium_rmsnorm_bwd may use for these sizes. */
size_t tritium_rmsnorm_bwd_workspace_size(int64_t n_rows, int64_t hidden);

/* Backward of RMSNorm (tritium/ops/rmsnorm.py:105-280 kernels, host
 * `_rmsnorm_backward_with_rstd` 519-574, standalone `rmsnorm_backward`
 * 577-613 and the residual backward 700-734).
 * rstd == NULL recomputes it from x (standalone rmsnorm_backward);
 * dresidual != NULL is added to dx (residual backward, fused add);
 * dweight == NULL skips dweight, else it receives [hidden] in `dtype`,
 * reduced deterministically through `workspace`. */
int tritium_rmsnorm_bwd(const void* dy, const void* x, const void* weight, const float* rstd,
                        const void* dresidual, void* dx, void* dweight, void* workspace,
                        size_t workspace_bytes, int64_t n_rows, int64_t hidden, float eps,
                        int dtype, void* stream);

/* ---- RoPE ------------------------------------------------------------------
 * tritium.rope / tritium.rope_ and the RoPE backward (tritium/ops/rope.py:24-90
 * `_rope_kernel`, host 201-291, autograd 294-360).
 * q, k, q_out, k_out: [n_tokens, n_heads, head_dim] in `dtype` (q_out may equal
 * q and k_out may equal k: in-place); cos/sin tables: [max_position,
 * head_dim/2] in `table_dtype`; position_kind 0 = none (position = token),
 * 1 = int32 ids, 2 = int64 ids; inverse != 0 applies the inverse rotation
 * (the backward).  A position outside [0, max_position) yields NaN outputs
 * for that token. */
int tritium_rope(const void* q, const void* k, const void* cos_table, const void* sin_table,
                 const void* position_ids, int position_kind, void* q_out, void* k_out,
                 int64_t n_tokens, int64_t n_heads, int64_t head_dim, int64_t max_position,
                 int64_t position_offset, int interleaved, int inverse, int dtype,
                 int table_dtype, void* stream);

/* tritium_rope with its own token-row strides (elements) for the inputs q, k
 * and for the outputs q_out, k_out; heads stay adjacent inside a row
 * (tritium_rope is this with both strides n_heads * head_dim).  No counterpart
 * in the reference, whose rope requires contiguous q and k (rope.py:192-195):
 * it lets a caller rotate q and k in place inside a fused
 * [tokens, 3, heads, head_dim] q/k/v projection (token stride
 * 3 * heads * head_dim), and write the backward's inverse rotation straight
 * into the fused gradient.  q and q_out may both be null: k alone is rotated
 * (for a caller whose attention rotates q on load). */
int tritium_rope_strided(const void* q, const void* k, const void* cos_table,
                         const void* sin_table, const void* position_ids, int position_kind,
                         void* q_out, void* k_out, int64_t n_tokens, int64_t n_heads,
                         int64_t head_dim, int64_t max_position, int64_t position_offset,
                         int interleaved, int inverse, int64_t in_token_stride,
                         int64_t out_token_stride, int dtype, int table_dtype, void* stream);

/* ---- SwiGLU ----------------------------------------------------------------
 * tritium.swiglu forward (tritium/ops/swiglu.py:21-35 `_swiglu_forward_kernel`,
 * host 61-73): out = silu(x) * gate over n elements. */
int tritium_swiglu_fwd(const void* x, const void* gate, void* out, int64_t n, int dtype,
                       void* stream);

/* tritium.swiglu_backward (tritium/ops/swiglu.py:38-58 `_swiglu_backward_kernel`,
 * host 76-100). */
int tritium_swiglu_bwd(const void* dy, const void* x, const void* gate, void* dx, void* dgate,
                       int64_t n, int dtype, void* stream);

/* SwiGLU over n_rows rows of n_cols elements with row strides (elements): x
 * and gate rows at ld_in, out rows at ld_out; the backward reads dy rows at
 * ld_dy and writes dx, dgate rows at ld_out.  Same arithmetic as
 * tritium_swiglu_fwd/_bwd.  No counterpart in the reference (its swiglu takes
 * two separate tensors, swiglu.py:61-100): it lets a caller keep the gate and
 * up projections as the two halves of one fused [tokens, 2 * d_ff] GEMM
 * output and receive their gradients in the same layout. */
int tritium_swiglu_rows_fwd(const void* x, const void* gate, void* out, int64_t n_rows,
                            int64_t n_cols, int64_t ld_in, int64_t ld_out, int dtype,
                            void* stream);
int tritium_swiglu_rows_bwd(const void* dy, const void* x, const void* gate, void* dx,
                            void* dgate, int64_t n_rows, int64_t n_cols, int64_t ld_dy,
                            int64_t ld_in, int64_t ld_out, int dtype, void* stream);

/* ---- AdamW -----------------------------------------------------------------
 * tritium.adamw_step (tritium/ops/adamw.py:20-54 `_adamw_step_kernel`, host
 * 113-151): in-place update of one parameter tensor (param/grad in `dtype`,
 * exp_avg/exp_avg_sq float32).  Bias corrections 1 - beta**step come from the
 * caller (adamw.py:133-134). */
int tritium_adamw_step(void* param, const void* grad, float* exp_avg, float* exp_avg_sq,
                       int64_t n, float lr, float beta1, float beta2, float eps,
                       float weight_decay, double bias_correction1, double bias_correction2,
                       int dtype, void* stream);

/* Elements one block of the multi-tensor kernel updates. */
int64_t tritium_adamw_chunk_elements(void);
/* Elements one block of the mixed-precision multi-tensor kernel updates. */
int64_t tritium_adamw_mixed_chunk_elements(void);

/* Multi-tensor AdamW in ONE launch (replaces the per-parameter loop of
 * helion.AdamW.step, helion/optim.py:50-70, each iteration of which calls
 * adamw.py:113-151).  `table` is a DEVICE array of n_tensors * 7 int64:
 * [param, grad, exp_avg, exp_avg_sq, numel, flags, first_chunk] where
 * flags = dtype | (16-byte-aligned << 8) and first_chunk is the exclusive
 * prefix sum of ceil(numel / tritium_adamw_chunk_elements()). */
int tritium_adamw_step_multi(const int64_t* table, int n_tensors, int64_t total_chunks,
                             float lr, float beta1, float beta2, float eps, float weight_decay,
                             double bias_correction1, double bias_correction2, void* stream);

/* Mixed-precision multi-tensor AdamW, one launch: fp32 params and moments,
 * 16-bit gradients (grad_dtype 1 = fp16, 2 = bf16) read as they are, and an
 * optional 16-bit copy of each updated parameter written in the same pass.
 * Arithmetic per element as tritium_adamw_step on the widened gradient.
 * table: device int64 rows of 8 words [param, grad, exp_avg, exp_avg_sq,
 * numel, flags (bit 0: all pointers 16-byte aligned), first_chunk, shadow or
 * 0], first_chunk the prefix sum of ceil(numel / tritium_adamw_mixed_chunk_elements()).
 * No counterpart in the reference (whose adamw_step requires grad and param
 * of one dtype, adamw.py:86-90): it serves a training step whose weights are
 * 16-bit copies of fp32 masters, which would otherwise widen every gradient
 * and re-round every weight in two extra passes. */
int tritium_adamw_step_mixed(const int64_t* table, int n_tensors, int64_t total_chunks, float lr,
                             float beta1, float beta2, float eps, float weight_decay,
                             double bias_correction1, double bias_correction2, int grad_dtype,
                             void* stream);

/* ---- attention -------------------------------------------------------------
 * Forward of tritium.attention (tritium/ops/attention.py:31-141
 * `_attention_forward_kernel`, 144-217 decode kernel, host 284-396).
 * q: [B, H, Tq, D], k/v: [B, Hkv, Tkv, D], o: like q, all in `dtype` with a
 * unit head_dim stride and element strides strides[0..11] =
 * {q_b, q_h, q_s, k_b, k_h, k_s, v_b, v_h, v_s, o_b, o_h, o_s} (host array).
 * lse: [B, H, Tq] float32, natural-log logsumexp of the scaled scores.
 * causal != 0 applies the top-left mask q_pos >= kv_pos; scale = D^-0.5.
 * bf16/fp16 with D in {16, 32, 64, 128, 256} run on MFMA, anything else on
 * the SIMT path (D <= 1024).  (At D = 256 the backward's dK/dV runs as two
 * launches, dV then dK, each forming S again: the fragments and accumulators
 * of one pass would not fit a wavefront's registers.) */
int tritium_attention_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                          int64_t B, int64_t H, int64_t Hkv, int64_t Tq, int64_t Tkv, int64_t D,
                          const int64_t* strides, int causal, int dtype, void* stream);

/* Backward of tritium.attention (tritium/ops/attention.py:399-629 kernels,
 * host `_attention_backward_impl` 632-702).  strides[0..23] = q, k, v, o,
 * dout, dq, dk, dv (batch, head, seq each); dq/dk/dv are written in `dtype`
 * with their own strides (no atomics); delta: [B*H*Tq] float32 workspace. */
int tritium_attention_bwd(const void* dout, const void* q, const void* k, const void* v,
                          const void* o, const float* lse, void* dq, void* dk, void* dv,
                          float* delta, int64_t B, int64_t H, int64_t Hkv, int64_t Tq,
                          int64_t Tkv, int64_t D, const int64_t* strides, int causal, int dtype,
                          void* stream);

/* Bytes of the dS workspace that tritium_attention_bwd_ws (and _bwd_rope_ws)
 * take for these arguments, 0 when the shape does not use one (head_dim other
 * than 128, float32).  It grows with Tq * Tkv: B * H * (causal ? about
 * n(n+1)/2 : n_q n_kv) 8 KiB chunks, n = Tq / 64 (2.2 GB at B 4, H 32,
 * Tq = Tkv = 4096, causal). */
size_t tritium_attention_bwd_workspace_size(int64_t B, int64_t H, int64_t Tq, int64_t Tkv,
                                            int64_t D, int causal, int dtype);

/* tritium_attention_bwd (same reference interface, attention.py:632-702) with
 * a dS workspace of tritium_attention_bwd_workspace_size bytes (16-byte
 * aligned; a smaller one is TRI_EINVAL): for head_dim 128 the dK/dV kernel
 * then stores dS and dQ is formed from it, instead of a dQ kernel that
 * recomputes S and dP.  Where the size is 0, or the tensors take the SIMT
 * path, the workspace is not used. */
int tritium_attention_bwd_ws(const void* dout, const void* q, const void* k, const void* v,
                             const void* o, const float* lse, void* dq, void* dk, void* dv,
                             float* delta, void* workspace, size_t workspace_bytes, int64_t B,
                             int64_t H, int64_t Hkv, int64_t Tq, int64_t Tkv, int64_t D,
                             const int64_t* strides, int causal, int dtype, void* stream);

/* tritium_attention_fwd with RoPE applied to q as each row is loaded: q holds
 * the unrotated rows, k the rotated ones (tritium_rope_strided with a null q
 * rotates k alone).  No counterpart in the reference, which rotates q and k
 * into new tensors right before attention (helion/nn.py:196-220): this is
 * that sequence for q without the rotated copy in memory.  The rotation is
 * tritium_rope's (non-interleaved halves, rounded to `dtype`): cos_table /
 * sin_table [max_position, D/2] float32; the position of query row t of
 * batch b is position_ids[b * Tq + t] (position_kind 1: int32, 2: int64) or
 * t (position_kind 0); positions outside [0, max_position) give NaN rows.
 * 16-bit tensors with D in {64, 128} and 16-byte aligned rows only
 * (TRI_EINVAL otherwise). */
int tritium_attention_fwd_rope(const void* q, const void* k, const void* v, void* o, float* lse,
                               int64_t B, int64_t H, int64_t Hkv, int64_t Tq, int64_t Tkv,
                               int64_t D, const int64_t* strides, int causal, int dtype,
                               const float* cos_table, const float* sin_table,
                               const void* position_ids, int position_kind,
                               int64_t max_position, void* stream);

/* Backward of tritium_attention_fwd_rope (no counterpart in the reference;
 * see above): q unrotated as in the forward, dq the gradient of the
 * unrotated q (the inverse rotation applied before the store).  q_rot:
 * [B, H, Tq, D] contiguous workspace in `dtype`, 16-byte aligned, which the
 * dQ kernel fills with the rotated q for the dK/dV kernel. */
int tritium_attention_bwd_rope(const void* dout, const void* q, const void* k, const void* v,
                               const void* o, const float* lse, void* dq, void* dk, void* dv,
                               float* delta, void* q_rot, int64_t B, int64_t H, int64_t Hkv,
                               int64_t Tq, int64_t Tkv, int64_t D, const int64_t* strides,
                               int causal, int dtype, const float* cos_table,
                               const float* sin_table, const void* position_ids,
                               int position_kind, int64_t max_position, void* stream);

/* tritium_attention_bwd_rope with the dS workspace of tritium_attention_bwd_ws
 * (no counterpart in the reference, as tritium_attention_fwd_rope): the
 * rotated q for the dK/dV kernel is then written by the kernel that computes
 * delta, and the dQ kernel applies the inverse rotation as it stores. */
int tritium_attention_bwd_rope_ws(const void* dout, const void* q, const void* k, const void* v,
                                  const void* o, const float* lse, void* dq, void* dk, void* dv,
                                  float* delta, void* q_rot, void* workspace,
                                  size_t workspace_bytes, int64_t B, int64_t H, int64_t Hkv,
                                  int64_t Tq, int64_t Tkv, int64_t D, const int64_t* strides,
                                  int causal, int dtype, const float* cos_table,
                                  const float* sin_table, const void* position_ids,
                                  int position_kind, int64_t max_position, void* stream);

/* The attention forward for one query row per (batch, head) against a K/V
 * cache (the reference's decode branch, attention.py:144-217, 354-396:
 * q_len = 1, no causal mask, strided cache slices): same outputs as
 * tritium_attention_fwd (o in q's layout, natural-log lse [B, H]) for 16-bit
 * inputs with head_dim 64 or 128 and at most 8 query heads per kv head.
 * The key sequence is split into chunks over extra workgroups whose partial
 * (m, l, o) go to `workspace` (tritium_attention_decode_workspace_size bytes)
 * and are merged by a second kernel.  strides as for tritium_attention_fwd
 * (the query and output sequence strides are unused). */
size_t tritium_attention_decode_workspace_size(int64_t B, int64_t H, int64_t Hkv, int64_t Tkv,
                                               int64_t D);
int tritium_attention_decode(const void* q, const void* k, const void* v, void* o, float* lse,
                             void* workspace, size_t workspace_bytes, int64_t B, int64_t H,
                             int64_t Hkv, int64_t Tkv, int64_t D, const int64_t* strides,
                             int dtype, void* stream);

/* tritium_attention_decode without a workspace argument and without any
 * allocation: no counterpart in the reference.  It is for callers that cannot
 * allocate device memory -- code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc.  The partial (m, l, o) rows go to a
 * scratch array that the library holds on each GPU it runs on until the
 * process ends (tritium_attention_decode_noalloc_max_bytes() bytes = 32 MiB);
 * a call whose partials would need more (the workspace size that
 * tritium_attention_decode_workspace_size returns for the same arguments) is
 * rejected with TRI_EINVAL.  Results are bitwise those of
 * tritium_attention_decode.  The scratch is looked up once per device, with
 * that device current; `stream` must belong to the current device.  Every
 * call on one GPU shares that GPU's scratch: calls that overlap on one GPU
 * (on different streams, or from several threads) race. */
size_t tritium_attention_decode_noalloc_max_bytes(void);
int tritium_attention_decode_noalloc(const void* q, const void* k, const void* v, void* o,
                                     float* lse, int64_t B, int64_t H, int64_t Hkv, int64_t Tkv,
                                     int64_t D, const int64_t* strides, int dtype, void* stream);

/* ---- fused linear + cross-entropy ---------------------------------------------
 * Forward of tritium.linear_cross_entropy (tritium/ops/cross_entropy.py:134-293
 * kernels, host `_linear_cross_entropy_forward` 563-640, autograd 663-705),
 * plus torch's ignore_index (absent from the reference).
 * hidden: [n_rows, hidden_size], weight: [vocab, hidden_size] in `dtype`,
 * 16-byte aligned, hidden_size a multiple of 8 (16-bit) or 4 (fp32);
 * target: [n_rows] int32 (target_kind 1) or int64 (2).  Writes loss[0] = mean
 * over rows whose target != ignore_index of lse - logit[target] (NaN when no
 * row counts), lse: [n_rows] float32 (natural log), n_valid[0] (may be NULL) =
 * that row count as float.  The logits are never written to memory. */
size_t tritium_linear_ce_fwd_workspace_size(int64_t n_rows, int64_t vocab, int dtype);
int tritium_linear_ce_fwd(const void* hidden, const void* weight, const void* target,
                          int target_kind, int64_t ignore_index, float* loss, float* lse,
                          float* n_valid, void* workspace, size_t workspace_bytes,
                          int64_t n_rows, int64_t hidden_size, int64_t vocab, int dtype,
                          void* stream);

/* Backward: tritium.linear_cross_entropy_backward (tritium/ops/cross_entropy.py:863-959),
 * 16-bit dtypes.  grad_out: device float32 scalar; lse from the forward.
 * dhidden: [n_rows, hidden_size], dweight: [vocab, hidden_size], both in
 * `dtype`; either may be NULL (not computed).  Per vocabulary chunk of
 * chunk_rows rows (0 = automatic: the chunk's gradient of the logits fills at
 * most 1 GiB), the logits are recomputed on the library's MFMA GEMM core and
 * turned into that gradient G [n_rows, chunk] in the workspace; dweight's rows
 * = G^T hidden and dhidden += G weight_chunk run on the same core, reading
 * G, hidden and weight in place (no transposed copies).  dhidden accumulates
 * in fp32 in the workspace when there is more than one chunk.  Workspace:
 * tritium_linear_ce_bwd_workspace_size bytes (0 for float32, rejected). */
size_t tritium_linear_ce_bwd_workspace_size(int64_t n_rows, int64_t hidden_size, int64_t vocab,
                                            int dtype, int need_dhidden, int need_dweight,
                                            int64_t chunk_rows);
int tritium_linear_ce_bwd(const float* grad_out, const void* hidden, const void* weight,
                          const void* target, int target_kind, int64_t ignore_index,
                          const float* lse, void* dhidden, void* dweight, void* workspace,
                          size_t workspace_bytes, int64_t n_rows, int64_t hidden_size,
                          int64_t vocab, int64_t chunk_rows, int dtype, void* stream);

/* Gradient of the logits for one vocabulary chunk, the fused part of
 * linear_cross_entropy_backward (reference cross_entropy.py:928-946: the
 * per-chunk F.linear + in-place CE kernel; its mm/addmm at 947-957 are plain
 * GEMMs the caller runs on these rows): for vocabulary rows [v0, v0 + vc),
 *   g[n, j] = (exp(hidden[n] . weight[v0 + j] - lse[n]) - [target[n] == v0 + j])
 *             * grad_out / n_valid,   0 for rows whose target == ignore_index,
 * written to g [n_rows, vc] with row stride ld_g (a multiple of 8) in
 * `dtype`; the logits themselves exist only in registers.  grad_out and
 * n_valid (the number of non-ignored targets) are device floats. */
int tritium_linear_ce_grad_logits(const float* grad_out, const float* n_valid, const void* hidden,
                                  const void* weight, const void* target, int target_kind,
                                  int64_t ignore_index, const float* lse, void* g, int64_t ld_g,
                                  int64_t n_rows, int64_t hidden_size, int64_t vocab, int64_t v0,
                                  int64_t vc, int dtype, void* stream);

/* ---- Embedding backward with a tied output head ---------------------------
 * No tritium.ops counterpart: replaces torch's backward of the gather in the
 * reference's Embedding (helion/nn.py:24-28, weight[ids]; torch sorts the ids
 * and scatter-adds) and, for an embedding tied to the output head
 * (examples/common.py), the separate add of the head's weight gradient:
 *   dw_out[v] = dw_in[v] + sum over tokens i with ids[i] == v of dx[i]
 * summed in fp32 in token order and rounded once (bitwise deterministic: the
 * tokens are bucketed by vocabulary row with integer counts, and each row
 * sums its tokens in order; no floating-point atomics).  ids:
 * [n_tokens] int32 (id_kind 1) or int64 (2); dx: [n_tokens, dim] with row
 * stride ld_dx; dw_in, dw_out: [vocab, dim] contiguous, all in `dtype`.
 * dw_out may be dw_in (rows no id names are then left as they are).  Ids
 * outside [0, vocab) contribute nothing.  A row's tokens are summed in
 * windows of 16 positions of the bucketed list and the windows' parts added
 * in order, so a heavily repeated id (padding, end of text) spreads over many
 * wavefronts.  workspace: tritium_embedding_bwd_workspace_size bytes,
 * cleared by the call itself where it needs to be: 4 bytes per (vocabulary
 * row, 1024-token chunk) of counts -- 4 * vocab * ceil(n_tokens / 1024),
 * which grows with both (0.8 MB at vocab 50304 and 16K tokens, 512 MB at a
 * 128K vocabulary and 1M tokens) -- plus 8 bytes per token for the bucketed
 * list and dim * n_tokens / 2 bytes of fp32 window parts. */
size_t tritium_embedding_bwd_workspace_size(int64_t n_tokens, int64_t vocab, int64_t dim);
int tritium_embedding_bwd(const void* ids, int id_kind, int64_t n_tokens, const void* dx,
                          int64_t ld_dx, const void* dw_in, void* dw_out, int64_t vocab,
                          int64_t dim, void* workspace, size_t workspace_bytes, int dtype,
                          void* stream);

/* ---- Split-K finish -------------------------------------------------------
 * dst[i] = (dtype)(src[0 * n + i] + src[1 * n + i] + ... + src[(n_splits - 1) * n + i]),
 * summed in fp32 in split order, for src [n_splits, n] float32 (the fp32
 * outputs of a GEMM split over its reduction dimension) and dst [n] in
 * `dtype`.  No reference counterpart: the training harness's weight
 * gradients use it (the reference computes them with one matmul per weight,
 * tritium/ops/matmul.py:311-333). */
int tritium_sum_splits(const float* src, void* dst, int64_t n_splits, int64_t n, int dtype,
                       void* stream);

/* ---- Cross-entropy on materialised logits ----------------------------------
 * tritium.cross_entropy forward (tritium/ops/cross_entropy.py:36-68
 * `_cross_entropy_forward_kernel`, host 534-561): for logits [n_rows, vocab]
 * in `dtype` (row-major, contiguous) and int32 (target_kind 1) or int64 (2)
 * targets, lse[row] = logsumexp(logits[row]) in fp32, nll[row] = lse[row] -
 * logits[row, target[row]] (NaN for a target outside [0, vocab)), and
 * loss[0] = mean(nll) summed in a fixed order.  `work` is caller-provided
 * scratch (8-byte aligned) of `work_bytes` bytes, at least
 * tritium_cross_entropy_fwd_workspace_size(n_rows, vocab, dtype): the n_rows
 * nll values, or, for fewer rows than the GPU has room for blocks of long
 * rows, a (max, sum) pair per span of each row.  A smaller or misaligned
 * buffer is rejected with TRI_EINVAL before anything is launched. */
int tritium_cross_entropy_fwd_ws(const void* logits, const void* target, int target_kind,
                                 float* loss, float* lse, void* work, size_t work_bytes,
                                 int64_t n_rows, int64_t vocab, int dtype, void* stream);
size_t tritium_cross_entropy_fwd_workspace_size(int64_t n_rows, int64_t vocab, int dtype);

/* tritium.cross_entropy_backward (cross_entropy.py:71-100
 * `_cross_entropy_backward_kernel`, host 728-799): dlogits = (exp(logits -
 * lse) - onehot(target)) * grad_out[0] / grad_denominator in `dtype`
 * (grad_out a device float; the reference's denominator is n_rows). */
int tritium_cross_entropy_bwd(const float* grad_out, const void* logits, const void* target,
                              int target_kind, const float* lse, void* dlogits, int64_t n_rows,
                              int64_t vocab, double grad_denominator, int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TRITIUM_HIP_H_ */
