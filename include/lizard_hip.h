/*
 * lizard_hip.h -- C ABI of the MI355X (gfx950) Lizard attention hot path.
 *
 * Library: lizard_reproduction_amd/_lib/liblizard_hip.so (hipcc --offload-arch=gfx950).
 *
 * Conventions for every entry point:
 *   - tensors are device pointers to contiguous row-major buffers;
 *     [BH, L, X] means batch*heads rows of length*X elements, the layout of a
 *     contiguous torch tensor of shape [B, H, L, X];
 *   - "bf16" buffers hold bfloat16, "f32" buffers float;
 *   - the library never allocates device memory: outputs, saved tensors and
 *     workspaces are owned by the caller (the reference's autograd Functions
 *     own theirs the same way, src/kernels/gla.py:221-225, swa.py:144-146);
 *   - work is enqueued on `stream` (a hipStream_t; NULL = default stream) and
 *     the call returns without synchronising;
 *   - return value 0 = success; otherwise an error code, with a message
 *     available from lz_last_error() on the calling thread.
 *   - extents: one (batch, head) slab of fp32 rows, length x max(F, D) x 4
 *     bytes, stays under 2 GiB, and batch*heads*length under 2^31 - 2^20; the
 *     kernels address slabs with 32-bit offsets, and larger calls are refused.
 *
 * The reference (mahdikhashan/lizard-reproduction) is pure Python + Triton; the
 * functions below replace its Triton launches.  Each comment names the
 * reference code the entry point stands in for.
 */
#ifndef LIZARD_HIP_H
#define LIZARD_HIP_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LZ_ABI_VERSION 15

/*
 * gate_mode of the GLA entry points: a combination of
 *   LZ_GATE_PER_HEAD  the gate is [B, H, L] (one per head); without it [B, L]
 *                     (one per token, shared by the heads), the reference's
 *                     two layouts (src/kernels/gla.py:259-263)
 *   LZ_GATE_LOGIT     the gate buffer holds the logit z, and the kernels use
 *                     log_gamma = logsigmoid(z), the reference layer's
 *                     F.logsigmoid (src/lizard_attention.py:92); the gate
 *                     gradient they write is then d/dz = d log_gamma *
 *                     sigmoid(-z).  Without it the buffer holds log_gamma.
 *   LZ_GLA_NO_REUSE   a hint: nothing reads fq, fk and v again soon (no
 *                     backward follows this forward), so the forward walk may
 *                     load them nontemporally.  Used by lz_gla_fwd,
 *                     lz_gla_prefill and lz_gla_fwd_noalloc (for one segment
 *                     per row and kv_heads == heads), ignored by the other
 *                     GLA entry points; the results are the same bits with or
 *                     without it.  No counterpart in the reference (a cache
 *                     policy of this build's loads).
 * Other bits are refused.
 */
#define LZ_GATE_PER_HEAD 1
#define LZ_GATE_LOGIT 2
#define LZ_GLA_NO_REUSE 4

/* Largest feature (nf) and value (nd) dim the GLA entry points take. */
#define LZ_GLA_MAX_DIM 4096
/* Most sink logits (n_meta) the SWA entry points take. */
#define LZ_SWA_MAX_META 65536

/* ABI version of the loaded library (LZ_ABI_VERSION). */
int lz_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* lz_last_error(void);

/* Workspace bytes lz_gla_fwd needs for these sizes (0 when B*H alone fills the GPU). */
size_t lz_gla_fwd_workspace_bytes(int batch, int heads, int length, int nf, int nd,
                                  int gate_mode, int chunk);

/*
 * GLA forward.  Replaces kernels.gla's forward: the gate cumsum and head
 * expand (src/kernels/gla.py:259-263) and the two launches of _GLA.forward,
 * _gla_fwd_h + _gla_fwd_o (src/kernels/gla.py:213-234).
 *   fq          bf16 [BH, L, nf]      feature-mapped queries
 *   fk          bf16 [B*kv_heads, L, nf]  feature-mapped keys
 *   v           bf16 [B*kv_heads, L, nd]
 *   kv_heads    heads of fk and v (divides heads): query head h reads kv head
 *               h / (heads / kv_heads), grouped-query attention without
 *               materialised copies; kv_heads = heads is the reference's layout
 *   log_gamma   f32  [B, L], or [B, H, L] with LZ_GATE_PER_HEAD in gate_mode;
 *               log of the gate (<= 0), NOT its cumsum, or with LZ_GATE_LOGIT
 *               the gate's logit z (log_gamma = logsigmoid(z))
 *   y           bf16 [BH, L, nd]      output
 *   chunk       tiling hint of the reference API (power of two >= 16); the
 *               kernels always walk 64-token chunks, results are
 *               chunk-independent up to rounding
 *   workspace   device buffer of lz_gla_fwd_workspace_bytes() bytes (may be
 *               NULL when that is 0): per-segment states when the sequence is
 *               split into segments to fill the GPU
 * Sizes: any nf, nd up to LZ_GLA_MAX_DIM, as the reference's kernels loop
 * over feature blocks (src/kernels/gla.py:74,154,171).  The walks take
 * nf <= 256, nd <= 128 (nd <= 64 when nf > 128) directly; past that the
 * library runs them on value tiles (exact) and, for nf > 256, on feature
 * tiles whose unnormalised numerators and denominators it sums before the
 * division (the bf16 weights a rounded per tile), with the workspace size
 * that lz_gla_fwd_workspace_bytes reports.
 * Nothing is saved for the backward: lz_gla_bwd recomputes what it needs, so
 * the output is the same with and without autograd (tests/test_kernels.py:102-107).
 */
int lz_gla_fwd(const void* fq, const void* fk, const void* v, const float* log_gamma, void* y,
               int batch, int heads, int kv_heads, int length, int nf, int nd, int gate_mode,
               int chunk, void* workspace, size_t workspace_bytes, void* stream);

/*
 * GLA forward that allocates nothing and takes no workspace.  No counterpart
 * in the reference: it is for callers that cannot allocate device memory
 * (tight serving loops, harnesses that forbid hipMalloc).  Capturing it into
 * a HIP graph is untested: the one capture this library's path ever ran (a
 * whole fwd+bwd through the Python API) crashed the host process in the
 * runtime's capture end, and that crash has no known cause, so capture is
 * not recommended.  Same arguments, result and kernels as lz_gla_fwd without the
 * workspace, at the walks' own sizes (nf <= 256, nd <= 128, nd <= 64 when
 * nf > 128): the per-segment states that lz_gla_fwd keeps in
 * its workspace (when B*H alone cannot fill the GPU) live in a static device
 * array of LZ_GLA_FWD_NOALLOC_MAX_BYTES per GPU, held until the process
 * ends.  That covers every size the forward takes on a whole MI355X; sizes
 * whose states would not fit are refused with an error.  Every call on one
 * GPU shares that GPU's array: calls that overlap on one GPU (on different
 * streams, or from different threads) race and must be serialised by the
 * caller.  Nothing in the array needs to start at zero: each call writes
 * every state it reads.
 */
#define LZ_GLA_FWD_NOALLOC_MAX_BYTES (66u << 20)
int lz_gla_fwd_noalloc(const void* fq, const void* fk, const void* v, const float* log_gamma,
                       void* y, int batch, int heads, int kv_heads, int length, int nf, int nd,
                       int gate_mode, int chunk, void* stream);

/*
 * Set-up of lz_gla_fwd_noalloc on the current device, once per device: the
 * device address of its static array (hipGetSymbolAddress), and the LDS
 * limits (hipFuncSetAttribute) of every kernel it can launch.  No
 * counterpart in the reference.  lz_gla_fwd_noalloc makes the same set-up on
 * its first call on a device.  After it, a call of lz_gla_fwd_noalloc still
 * makes these runtime calls besides its kernel launches: hipGetDevice (to
 * find the device's array and set-up), the device attribute queries of its
 * first call on a device (CU and XCD counts), and hipGetLastError after the
 * launches.  Returns 0 or an error code (lz_last_error).
 */
int lz_init(void);

/*
 * GLA prefill: lz_gla_fwd that also writes the recurrent state after the last
 * token, for decoding.  No counterpart in the reference (it has no decode
 * path); the state is that of its recurrent form (tests/test_lizard.py:41-52):
 *   S_L = sum_t (prod_{s>t} gamma_s) fk_t v_t^T,  z_L = sum_t (prod_{s>t} gamma_s) fk_t
 *   state  f32 [B, H, nf*nd + nf]: S row-major [nf][nd], then z [nf]
 * Other arguments as lz_gla_fwd (same workspace), at the walks' own sizes:
 * nf <= 256, nd <= 128, nd <= 64 when nf > 128.
 */
int lz_gla_prefill(const void* fq, const void* fk, const void* v, const float* log_gamma,
                   void* y, float* state, int batch, int heads, int kv_heads, int length, int nf,
                   int nd, int gate_mode, int chunk, void* workspace, size_t workspace_bytes,
                   void* stream);

/*
 * GLA forward with the feature map of q formed inside the walk.  Replaces
 * hedgehog(q, phi_q) (src/lizard_attention.py:9-11, 85) followed by
 * kernels.gla's forward (src/kernels/gla.py:213-263), for a layer's
 * forward without autograd (inference, prefill): fq is never written to
 * memory; each chunk's fq = [softmax(q Wq^T), softmax(-q Wq^T)] is formed
 * from the q rows and Wq in the walk, with the arithmetic of
 * lz_layer_prologue_fwd (bf16 products, fp32 softmax, bf16 result).
 *   q          bf16 [B, L, heads, head_dim]  (the q_proj output, not RoPE'd)
 *   wq         bf16 [feature_dim, head_dim]  (phi_q.weight)
 *   fk         bf16 [B, kv_heads, L, 2 feature_dim]  (lz_layer_prologue_fwd's fk)
 *   v          bf16 [B, kv_heads, L, head_dim]
 *   y          bf16 [B, heads, L, head_dim]
 *   state      f32 [B, heads, nf*nd + nf] (nf = 2 feature_dim, nd = head_dim): the
 *              recurrent state after the last token as lz_gla_prefill writes it,
 *              or NULL
 * Other arguments as lz_gla_fwd, whose workspace (lz_gla_fwd_workspace_bytes
 * with nf = 2 feature_dim, nd = head_dim) this takes.  Sizes: head_dim 64,
 * feature_dim 128 (the config of Llama-3.2-1B with the reference's default
 * feature_dim); a batch row of q under 2 GiB.
 */
int lz_gla_fwd_phi(const void* q, const void* wq, const void* fk, const void* v,
                   const float* log_gamma, void* y, float* state, int batch, int heads,
                   int kv_heads, int length, int head_dim, int feature_dim, int gate_mode,
                   int chunk, void* workspace, size_t workspace_bytes, void* stream);

/*
 * GLA decode step: one new token per (b, h) on the recurrent form
 * (tests/test_lizard.py:41-52), state updated in place:
 *   S <- gamma S + fk v^T,  z <- gamma z + fk,  y = fq S / max(fq . z, FLT_MIN)
 *   fq  bf16 [B, H, nf];  fk  bf16 [B, kv_heads, nf];  v  bf16 [B, kv_heads, nd]
 *   (query head h reads kv head h / (heads / kv_heads));  y  bf16 [B, H, nd]
 *   log_gamma  f32 [B], or [B, H] with LZ_GATE_PER_HEAD;  gamma = exp(log_gamma)
 *              (with LZ_GATE_LOGIT the logit z: log_gamma = logsigmoid(z))
 *   state  f32 [B, H, nf*nd + nf] as written by lz_gla_prefill (zeros: empty prefix)
 * Sizes as lz_gla_prefill.
 */
int lz_gla_decode_step(const void* fq, const void* fk, const void* v, const float* log_gamma,
                       float* state, void* y, int batch, int heads, int kv_heads, int nf, int nd,
                       int gate_mode, void* stream);

/* Workspace bytes lz_gla_bwd needs for these sizes. */
size_t lz_gla_bwd_workspace_bytes(int batch, int heads, int length, int nf, int nd,
                                  int gate_mode, int chunk);

/*
 * GLA backward.  Replaces _GLA.backward (src/kernels/gla.py:236-256): delta,
 * _gla_bwd_dh, _gla_bwd_dqkv, the dg reduction, and the autograd steps of
 * the gate path (expand-sum over heads, reverse cumsum, gla.py:260-262).
 *   dy            bf16 [BH, L, nd]      upstream gradient
 *   dfq, dfk      [BH, L, nf], dv [BH, L, nd]: bf16 if grad_bf16 else f32; per
 *                 query head also when kv_heads < heads (each query head's
 *                 share; their sum over a group is the kv head's gradient)
 *   dlog_gamma    f32, same shape as log_gamma (with LZ_GATE_LOGIT: the gradient of
 *                 the logit z, d log_gamma * sigmoid(-z))
 *   fwd_workspace the workspace lz_gla_fwd used for these inputs, if the caller
 *                 kept it (it then holds the segment state records, scanned
 *                 into the state entering each segment or, for at most 4
 *                 segments, left for the walks to combine, and the backward
 *                 skips recomputing them); may be NULL
 * The other arguments are those of lz_gla_fwd, with its sizes.
 */
int lz_gla_bwd(const void* fq, const void* fk, const void* v, const float* log_gamma,
               const void* dy, void* dfq, void* dfk, void* dv, float* dlog_gamma, int grad_bf16,
               int batch, int heads, int kv_heads, int length, int nf, int nd, int gate_mode,
               int chunk, const void* fwd_workspace, size_t fwd_workspace_bytes, void* workspace,
               size_t workspace_bytes, void* stream);

/*
 * SWA forward.  Replaces _SWA.forward / _swa_fwd (src/kernels/swa.py:136-156,
 * 19-59).
 *   q           bf16 [BH, L, dim]  (RoPE already applied)
 *   k, v        bf16 [B*kv_heads, L, dim]  (RoPE applied to k); kv_heads divides
 *               heads, query head h reads kv head h / (heads / kv_heads)
 *   meta        f32 [n_meta] sink logits (n_meta may be 0; at most LZ_SWA_MAX_META)
 *   y           bf16 [BH, L, dim] output
 *   lse         f32 [BH, L] log of each row's softmax denominator (saved for backward)
 *   window      keys i-window < t <= i;  scale  usually 1/sqrt(dim)
 * Supported sizes: dim <= 256.
 */
int lz_swa_fwd(const void* q, const void* k, const void* v, const float* meta, int n_meta,
               void* y, float* lse, int batch, int heads, int kv_heads, int length, int dim,
               int window, float scale, void* stream);

/*
 * SWA decode step: the forward's output row for one new query per (b, h), at
 * absolute position pos, against a ring-buffered window cache.  No counterpart
 * in the reference (it has no decode path); the row is that of _swa_fwd
 * (src/kernels/swa.py:19-59) at i = pos:
 *   q         bf16 [B, H, dim]  (RoPE at position pos applied)
 *   k_cache, v_cache  bf16 [B, kv_heads, window, dim]; position p (RoPE applied
 *             to k) in slot p % window; the caller writes position pos there
 *             first, so slots of positions max(0, pos-window+1) .. pos are read
 *   meta      f32 [n_meta] sink logits;  y  bf16 [B, H, dim]
 *   window    at most 8192;  dim <= 256;  pos >= 0
 */
int lz_swa_decode_step(const void* q, const void* k_cache, const void* v_cache,
                       const float* meta, int n_meta, void* y, int batch, int heads, int kv_heads,
                       int window, int dim, int pos, float scale, void* stream);

/* Workspace bytes lz_swa_bwd needs for these sizes. */
size_t lz_swa_bwd_workspace_bytes(int batch, int heads, int length, int dim, int n_meta);

/*
 * SWA backward.  Replaces _SWA.backward (src/kernels/swa.py:158-179): delta,
 * _swa_bwd_q, _swa_bwd_kv and the dmeta reduction.  delta_i = dy_i . y_i is
 * formed in fp32 as sum_t p_it (dy_i . v_t) from the recomputed
 * probabilities (the reference takes it from the bf16 output, swa.py:164),
 * so the forward saves only lse.
 *   lse         from lz_swa_fwd;  dy  bf16 [BH, L, dim]
 *   dq, dk, dv  [BH, L, dim]: bf16 if grad_bf16 else f32 (dk, dv per query head,
 *               as lz_gla_bwd's dfk, dv)
 *   dmeta       f32 [n_meta] (untouched when n_meta == 0)
 */
int lz_swa_bwd(const void* q, const void* k, const void* v, const float* meta, int n_meta,
               const float* lse, const void* dy, void* dq, void* dk, void* dv, float* dmeta,
               int grad_bf16, int batch, int heads, int kv_heads, int length, int dim, int window,
               float scale, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Layer prologue, forward.  Replaces the torch ops of LizardAttention.forward
 * between the projections and the kernel calls (src/lizard_attention.py:73-88):
 * split + repeat_interleave of q/k/v, the fp32 promotion, hedgehog(q, phi_q),
 * hedgehog(k, phi_k) (:9-11) and apply_rotary_pos_emb (:88), plus the kernels'
 * bf16 casts (src/kernels/gla.py:217, swa.py:139).
 *   q           [B, L, heads, head_dim]     (the q_proj output)
 *   k, v        [B, L, kv_heads, head_dim]  (k_proj, v_proj outputs)
 *   wq, wk      [feature_dim, head_dim]     (phi_q.weight, phi_k.weight)
 *   cos, sin    [B, L, head_dim] if cos_batched else [L, head_dim]
 *   all of them bf16 if dtype_bf16 else f32.
 *   fq          bf16 [B, heads, L, 2 feature_dim]: [softmax(q Wq^T), softmax(-q Wq^T)],
 *               or NULL: then the q rows are only rotated (qr), for lz_gla_fwd_phi,
 *               which forms their feature map itself
 *   fk          bf16 [B, kv_heads, L, 2 feature_dim]: the same of k with Wk
 *   qr          bf16 [B, heads, L, head_dim]: rotate_half RoPE of q
 *   kr, v_out   bf16 [B, kv_heads, L, head_dim]: RoPE of k; v
 *   The k-side operands stay per kv head: lz_gla_* and lz_swa_* read them with
 *   kv_heads < heads, which replaces the reference's repeat_interleave without
 *   writing its copies.
 * Supported sizes: head_dim 32, 64 or 128; feature_dim a multiple of 4, at most
 * 128 (64 when head_dim is 128 and dtype_bf16 is 0).
 */
int lz_layer_prologue_fwd(const void* q, const void* k, const void* v, const void* wq,
                          const void* wk, const void* cos, const void* sin, int cos_batched,
                          void* fq, void* fk, void* qr, void* kr, void* v_out, int dtype_bf16,
                          int batch, int length, int heads, int kv_heads, int head_dim,
                          int feature_dim, void* stream);

/* Workspace bytes lz_layer_prologue_bwd needs for these sizes. */
size_t lz_layer_prologue_bwd_workspace_bytes(int batch, int length, int heads, int kv_heads,
                                             int head_dim, int feature_dim);

/*
 * Layer prologue, backward: what autograd does for the same ops.
 *   dfq, dfk         bf16 [B, heads, L, 2 feature_dim]  (gradients of fq, and of fk per
 *                    query head, as lz_gla_bwd writes them)
 *   dqr, dkr, dv     bf16 [B, heads, L, head_dim]       (gradients of qr, kr, v_out per
 *                    query head, as lz_swa_bwd / lz_gla_bwd write them)
 *   dv2              NULL or a second bf16 gradient of v_out, added to dv in
 *                    fp32 (v_out feeds both attention branches)
 *   dq               [B, L, heads, head_dim];  dk, dv_out [B, L, kv_heads, head_dim]
 *                    (summed over each kv head's query heads), bf16 if dtype_bf16 else f32
 *   dwq, dwk         f32 [feature_dim, head_dim]  (summed over every row, deterministically)
 * q, k, wq, wk, cos, sin as given to lz_layer_prologue_fwd.
 */
int lz_layer_prologue_bwd(const void* q, const void* k, const void* wq, const void* wk,
                          const void* cos, const void* sin, int cos_batched, const void* dfq,
                          const void* dfk, const void* dqr, const void* dkr, const void* dv,
                          const void* dv2, void* dq, void* dk, void* dv_out, float* dwq,
                          float* dwk,
                          int dtype_bf16, int batch, int length, int heads, int kv_heads,
                          int head_dim, int feature_dim, void* workspace, size_t workspace_bytes,
                          void* stream);

/*
 * Layer epilogue, forward.  Replaces y = y_gla.to(dtype) + alpha * y_swa.to(dtype)
 * and y.to(x.dtype).transpose(1, 2).flatten(2) (src/lizard_attention.py:94-97).
 *   y_gla, y_swa  bf16 [B, heads, L, head_dim];  alpha  f32 [1] (device)
 *   out           [B, L, heads * head_dim], bf16 if out_bf16 else f32
 * head_dim a multiple of 8.
 */
int lz_layer_combine_fwd(const void* y_gla, const void* y_swa, const float* alpha, void* out,
                         int out_bf16, int batch, int heads, int length, int head_dim,
                         void* stream);

/* Workspace bytes lz_layer_combine_bwd needs. */
size_t lz_layer_combine_bwd_workspace_bytes(void);

/*
 * Layer epilogue, backward: dy_gla = bf16(dout), dy_swa = bf16(alpha dout)
 * (bf16 [B, heads, L, head_dim]) and dalpha = sum(dout * y_swa) (f32 [1],
 * summed in a fixed order).  dout as `out` of lz_layer_combine_fwd.
 */
int lz_layer_combine_bwd(const void* dout, const void* y_swa, const float* alpha, void* dy_gla,
                         void* dy_swa, float* dalpha, int out_bf16, int batch, int heads,
                         int length, int head_dim, void* workspace, size_t workspace_bytes,
                         void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LIZARD_HIP_H */
