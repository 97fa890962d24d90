/*
 * evograd_hip.h — C ABI of libevograd_hip.so, the gfx950 (MI355X) kernels behind
 * evograd's autograd-pair hot path.
 *
 * The reference (akumdam2/evograd) has no native code: each operator's pair is a
 * Python module exposing
 *     <op>_forward_with_saved(*declared args) -> (y, saved)
 *     <op>_backward_from_saved(dy, saved, **scalar inactive args) -> grads
 * found by src/evograd/opdecl/bind.py:28-47 (lookup_pair) and called by
 * src/evograd/opdecl/verify.py:118-143 and src/evograd/bench/harness.py:216-349.
 * Every entry point below is one kernel launch sequence that such a module calls.
 * The citation on each names the reference computation it replaces.
 *
 * Conventions (all entry points):
 *   - Pointers are device pointers to contiguous row-major tensors. The caller
 *     owns every buffer: outputs, saved state and workspace are allocated by the
 *     caller (in the Python modules: torch.empty on the caching allocator).
 *     The library never allocates, frees or synchronises.
 *   - Work is enqueued asynchronously on `stream` (a hipStream_t; NULL is the
 *     legacy default stream).
 *   - Return 0 on success. A non-zero return means nothing was launched (or the
 *     launch itself failed); eg_last_error() then describes why. The message
 *     buffer is thread-local.
 *   - `dtype` is one of eg_dtype. Reductions always accumulate in fp32.
 *   - Results are deterministic: no atomics; every reduction has a fixed order.
 */
#ifndef EVOGRAD_HIP_H
#define EVOGRAD_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  EG_F32 = 0,
  EG_F16 = 1,
  EG_BF16 = 2,
} eg_dtype;

/* ABI version of this header; bumped on any signature change. */
int eg_abi_version(void);

/* Description of the last failure on the calling thread ("" if none). */
const char* eg_last_error(void);

/* Measurement hook; no counterpart in the reference (its harness times with
 * torch.cuda.Event around whole calls, src/evograd/bench/harness.py:173-213).
 * Arms the calling thread's next kernel launches: the `index`-th launch (0-based,
 * in launch order, counted from the next entry-point call on and across the calls
 * that follow it) is made with hipExtLaunchKernelGGL so the dispatch records
 * `start_event` / `stop_event` (hipEvent_t, created with timing) at that kernel's
 * start and end. The arm lasts until that launch or the next eg_time_kernel. For
 * callers that time one kernel of a multi-kernel entry point or of a short
 * sequence of calls (bench.py); results are unchanged. */
int eg_time_kernel(void* start_event, void* stop_event, int index);

/* 1 when the launch armed by eg_time_kernel has not run yet (its events hold
 * nothing of this arm), 0 when it has; drops the arm either way. */
int eg_time_kernel_missed(void);

/* Name of the kernel the calling thread's last eg_time_kernel arm launched ("" until
 * that launch has happened). */
const char* eg_time_kernel_label(void);

/* ---------------------------------------------------------------- softmax
 * Replaces softmax_forward_ref (src/evograd/ops/level1/softmax/forward_ref.py:6-7):
 *   y = softmax(x.float(), dim=-1).to(x.dtype), x and y [rows, cols].
 * Saved state is y itself. */
int eg_softmax_fwd(const void* x, void* y, int64_t rows, int64_t cols, int dtype,
                   void* stream);

/* Replaces the autograd backward of softmax_forward_ref, declared at
 * src/evograd/ops/level1/softmax/__init__.py:78:
 *   dx = y * (dy - sum(dy * y, -1)), accumulated in fp32. */
int eg_softmax_bwd(const void* y, const void* dy, void* dx, int64_t rows, int64_t cols,
                   int dtype, void* stream);

/* ---------------------------------------------------------------- rmsnorm
 * Replaces rmsnorm_forward_ref (src/evograd/ops/level1/rmsnorm/forward_ref.py:6-21):
 *   rstd = rsqrt(mean(x^2, -1) + eps); y = ((x * rstd) * weight).to(x.dtype)
 * x, y [rows, hidden] (dtype); weight [hidden] (dtype); rstd [rows] fp32 (saved). */
int eg_rmsnorm_fwd(const void* x, const void* weight, void* y, float* rstd, int64_t rows,
                   int64_t hidden, float eps, int dtype, void* stream);

/* Bytes of fp32 workspace eg_rmsnorm_bwd needs for its per-block dweight partials. */
size_t eg_rmsnorm_workspace_bytes(int64_t rows, int64_t hidden);

/* Replaces the autograd backward of rmsnorm_forward_ref, declared at
 * src/evograd/ops/level1/rmsnorm/__init__.py:85-86:
 *   xhat = x * rstd, g = dy * weight
 *   dx = (g - xhat * mean(g * xhat, -1)) * rstd
 *   dweight = sum_rows(dy * xhat)   (two stages: per-block partials, fixed-order sum) */
int eg_rmsnorm_bwd(const void* dy, const void* x, const void* weight, const float* rstd,
                   void* dx, void* dweight, void* workspace, int64_t rows, int64_t hidden,
                   int dtype, void* stream);

/* The same backward as eg_rmsnorm_bwd (src/evograd/ops/level1/rmsnorm/__init__.py:
 * 85-86) in one launch and with no workspace, for few rows (the reference's small
 * regime, under 4096 tokens: src/evograd/opdecl/models.py:306): column workgroups
 * sum dweight = sum_rows(dy * x * rstd) directly in a fixed order while row
 * workgroups form dx. dy and x are read twice: faster than eg_rmsnorm_bwd up to
 * about 512 rows (bf16, hidden 1024-8192), slower from about 768 rows on. */
int eg_rmsnorm_bwd_small(const void* dy, const void* x, const void* weight, const float* rstd,
                         void* dx, void* dweight, int64_t rows, int64_t hidden, int dtype,
                         void* stream);

/* Size of the device-resident scratch array behind eg_rmsnorm_bwd_noalloc (16 MiB
 * per GPU: the [G, hidden] fp32 partial rows for hidden up to 8192). */
#define EG_NOALLOC_SCRATCH_BYTES (16 * 1024 * 1024)

/* No counterpart in the reference: for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid it).
 * eg_rmsnorm_bwd without the workspace argument: the partial rows live in a
 * library-owned device array of EG_NOALLOC_SCRATCH_BYTES per GPU, so the call
 * allocates nothing. Sizes whose partial rows exceed it (eg_rmsnorm_workspace_bytes
 * > EG_NOALLOC_SCRATCH_BYTES) are refused with an error. `stream` must belong to
 * the current device. Calls that overlap on one GPU share the array and race. */
int eg_rmsnorm_bwd_noalloc(const void* dy, const void* x, const void* weight,
                           const float* rstd, void* dx, void* dweight, int64_t rows,
                           int64_t hidden, int dtype, void* stream);

/* ----------------------------------------------------- fused_add_rms_norm
 * Replaces fused_add_rms_norm_forward_ref
 * (src/evograd/ops/level2/fused_add_rms_norm/forward_ref.py:6-16):
 *   s = x + r; rstd = rsqrt(mean(s^2, -1) + eps); out = (s * rstd) * weight
 * s is formed in fp32 and never stored; x, r, out [rows, hidden] (dtype), weight
 * [hidden], rstd [rows] fp32 (saved with x and r). */
int eg_fused_add_rmsnorm_fwd(const void* x, const void* r, const void* weight, void* out,
                             float* rstd, int64_t rows, int64_t hidden, float eps, int dtype,
                             void* stream);

/* Replaces the autograd backward declared at
 * src/evograd/ops/level2/fused_add_rms_norm/__init__.py:103-106: with s = x + r
 * formed again from the inputs, shat = s * rstd, g = dout * weight,
 *   ds = (g - shat * mean(g * shat, -1)) * rstd   (= dx = dr, written once to ds)
 *   dweight = sum_rows(dout * shat)               (two stages, fixed order)
 * Workspace: eg_rmsnorm_workspace_bytes(rows, hidden). */
int eg_fused_add_rmsnorm_bwd(const void* dout, const void* x, const void* r,
                             const void* weight, const float* rstd, void* ds, void* dweight,
                             void* workspace, int64_t rows, int64_t hidden, int dtype,
                             void* stream);

/* -------------------------------------------------------------- layernorm
 * Replaces layernorm_forward_ref (src/evograd/ops/level1/layernorm/forward_ref.py:6-23):
 *   mean = mean(x, -1); var = mean((x - mean)^2, -1); rstd = rsqrt(var + eps)
 *   y = ((x - mean) * rstd * weight + bias).to(x.dtype)
 * mean, rstd [rows] fp32 are saved. */
int eg_layernorm_fwd(const void* x, const void* weight, const void* bias, void* y,
                     float* mean, float* rstd, int64_t rows, int64_t hidden, float eps,
                     int dtype, void* stream);

/* Bytes of fp32 workspace eg_layernorm_bwd needs (dweight and dbias partials). */
size_t eg_layernorm_workspace_bytes(int64_t rows, int64_t hidden);

/* Replaces the autograd backward of layernorm_forward_ref
 * (src/evograd/ops/level1/layernorm/__init__.py:124-171 declares dx, dweight, dbias):
 *   xhat = (x - mean) * rstd, g = dy * weight
 *   dx = rstd * (g - mean(g, -1) - xhat * mean(g * xhat, -1))
 *   dweight = sum_rows(dy * xhat), dbias = sum_rows(dy)   (two-stage, fixed order) */
int eg_layernorm_bwd(const void* dy, const void* x, const void* weight, const float* mean,
                     const float* rstd, void* dx, void* dweight, void* dbias,
                     void* workspace, int64_t rows, int64_t hidden, int dtype,
                     void* stream);

/* eg_layernorm_bwd in one launch with no workspace, for few rows (as
 * eg_rmsnorm_bwd_small): dweight = sum_rows(dy * xhat), dbias = sum_rows(dy) summed
 * per column in a fixed order, dx per row. */
int eg_layernorm_bwd_small(const void* dy, const void* x, const void* weight, const float* mean,
                           const float* rstd, void* dx, void* dweight, void* dbias,
                           int64_t rows, int64_t hidden, int dtype, void* stream);

/* ----------------------------------------------------------------- swiglu
 * Replaces swiglu_forward_ref (src/evograd/ops/level1/swiglu/forward_ref.py:6-9):
 *   c = silu(a.float()).to(a.dtype) * b    (the silu is rounded to dtype first)
 * a, b, c hold n elements. */
int eg_swiglu_fwd(const void* a, const void* b, void* c, int64_t n, int dtype,
                  void* stream);

/* Replaces the autograd backward declared at
 * src/evograd/ops/level1/swiglu/__init__.py:70-73, sigmoid recomputed from a:
 *   s = sigmoid(a); db = dc * a * s; da = dc * b * (s + a * s * (1 - s))
 * da may alias a and db may alias b (backward_may_overwrite, :96): each element
 * is read before it is written, by the same thread. */
int eg_swiglu_bwd(const void* dc, const void* a, const void* b, void* da, void* db,
                  int64_t n, int dtype, void* stream);

/* ------------------------------------------------------------------- rope
 * Replaces rope_forward_ref (src/evograd/ops/level1/rope/forward_ref.py:28-47),
 * half-rotated layout, for up to two tensors in one launch (q and k of a GQA layer):
 *   y = x * cos + rotate_half(x) * sin, rotate_half(x) = [-x2, x1], in fp32.
 * q [batch, heads_q, tokens, head_dim], k [batch, heads_k, tokens, head_dim]
 * (k, k_out may be NULL with heads_k = 0); cos, sin [tokens, head_dim] of
 * table_dtype (EG_F32 or the same dtype as q). `inverse` = 1 applies the
 * transpose rotation (sin negated): the backward declared at
 * src/evograd/ops/level1/rope/__init__.py:124-130. Out-of-place only. */
int eg_rope(const void* q, const void* k, void* q_out, void* k_out, const void* cos,
            const void* sin, int64_t batch, int64_t heads_q, int64_t heads_k,
            int64_t tokens, int64_t head_dim, int dtype, int table_dtype, int inverse,
            void* stream);

/* ------------------------------------------------------ causal attention
 * Replaces F.scaled_dot_product_attention(q, k, v, is_causal=True) as used by
 * src/evograd/ops/level3/llama3_decoder_layer/forward_ref.py:107:
 *   o = softmax(q k^T * scale + causal mask) v
 * q, k, v, o [batch, heads, seq, head_dim]; lse [batch, heads, seq] fp32 = logsumexp
 * of the scaled, masked scores (saved). bf16/fp16 at head_dim 64 or 128 run on MFMA;
 * fp32, and any other even head_dim up to 128, on plain fp32 arithmetic (the shapes
 * of the decoder layer's correctness gate,
 * src/evograd/ops/level3/llama3_decoder_layer/__init__.py:55-65). */
int eg_attn_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                int64_t batch, int64_t heads, int64_t seq, int64_t head_dim, float scale,
                int dtype, void* stream);

/* Grouped-query attention: q, o [batch, heads, seq, head_dim]; k, v [batch,
 * kv_heads, seq, head_dim] with heads a multiple of kv_heads. Query head h attends
 * with kv head h / (heads / kv_heads): the repeat_interleave of k and v at
 * src/evograd/ops/level3/llama3_decoder_layer/forward_ref.py:101-105 followed by
 * the SDPA call at :107, without materialising the repeated tensors.
 * eg_attn_fwd is this with kv_heads = heads. */
int eg_attn_gqa_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                    int64_t batch, int64_t heads, int64_t kv_heads, int64_t seq,
                    int64_t head_dim, float scale, int dtype, void* stream);

/* Bytes of workspace eg_attn_gqa_bwd needs: delta = rowsum(do * o), fp32 [batch,
 * heads, seq] (heads = query heads), rounded up to 256 bytes; then, for shapes with
 * fewer than 1024 (kv head, 128-key block) pairs, where the dK/dV walk over the
 * query tiles is split into parts (at most 8, a choice of the shape alone), the
 * parts' fp32 sums: 2 x parts x batch x kv_heads x seq x head_dim x 4 bytes.
 * eg_attn_workspace_bytes (for eg_attn_bwd) is this with kv_heads = heads. */
size_t eg_attn_gqa_workspace_bytes(int64_t batch, int64_t heads, int64_t kv_heads,
                                   int64_t seq, int64_t head_dim);
size_t eg_attn_workspace_bytes(int64_t batch, int64_t heads, int64_t seq,
                               int64_t head_dim);

/* Backward of the above: P is recomputed from q, k and lse; produces dq, dk, dv
 * of q's dtype. */
int eg_attn_bwd(const void* dout, const void* q, const void* k, const void* v,
                const void* o, const float* lse, void* dq, void* dk, void* dv,
                void* workspace, int64_t batch, int64_t heads, int64_t seq,
                int64_t head_dim, float scale, int dtype, void* stream);

/* Backward of eg_attn_gqa_fwd: dq [batch, heads, seq, head_dim]; dk, dv [batch,
 * kv_heads, seq, head_dim], each the sum over the heads/kv_heads query heads that
 * share the kv head (the gradient of the repeat_interleave), accumulated in fp32
 * in a fixed order. Workspace: eg_attn_gqa_workspace_bytes. */
int eg_attn_gqa_bwd(const void* dout, const void* q, const void* k, const void* v,
                    const void* o, const float* lse, void* dq, void* dk, void* dv,
                    void* workspace, int64_t batch, int64_t heads, int64_t kv_heads,
                    int64_t seq, int64_t head_dim, float scale, int dtype, void* stream);

/* ------------------------------------- RoPE(q, k) -> grouped causal attention
 * Replaces the attention half of the Llama-3 decoder layer,
 * src/evograd/ops/level3/llama3_decoder_layer/forward_ref.py:93-107:
 *   q_r = rope(q), k_r = rope(k)   (rotate-half, fp32 tables, rounded to dtype)
 *   o = causal attention of q_r against k_r, v repeated over each query group
 * q, o, dout, dq [batch, heads, seq, head_dim]; k, v, dk, dv [batch, kv_heads,
 * seq, head_dim]; cos, sin fp32 [seq, head_dim] (duplicated halves); lse fp32
 * [batch, heads, seq] of the rotated scores. The backward takes the pre-rotation
 * q, k and rotates them again: the saved state holds no rotated copy. dq and dk
 * are the gradients of the pre-rotation q and k.
 * Workspace: the backward's holds q_r, k_r (dtype), then what eg_attn_gqa_bwd's
 * workspace holds (delta, and the split dK/dV walk's sums for shapes that split it)
 * (eg_llama3_attn_workspace_bytes); the forward's needs only batch * kv_heads
 * * seq * head_dim elements of dtype (its rotated keys). */
size_t eg_llama3_attn_workspace_bytes(int64_t batch, int64_t heads, int64_t kv_heads,
                                      int64_t seq, int64_t head_dim);
int eg_llama3_attn_fwd(const void* q, const void* k, const void* v, const float* cos,
                       const float* sin, void* o, float* lse, void* workspace, int64_t batch,
                       int64_t heads, int64_t kv_heads, int64_t seq, int64_t head_dim,
                       float scale, int dtype, void* stream);
int eg_llama3_attn_bwd(const void* dout, const void* q, const void* k, const void* v,
                       const void* o, const float* lse, const float* cos, const float* sin,
                       void* dq, void* dk, void* dv, void* workspace, int64_t batch,
                       int64_t heads, int64_t kv_heads, int64_t seq, int64_t head_dim,
                       float scale, int dtype, void* stream);

/* ---------------------------------------------------------- cross entropy
 * Replaces cross_entropy_forward_ref
 * (src/evograd/ops/level1/cross_entropy/forward_ref.py:6-12):
 *   loss = F.cross_entropy(logits.float(), target, reduction="mean",
 *                          ignore_index=ignore_index).to(logits.dtype)
 * logits [rows, cols] (dtype); target [rows] int64; loss one element (dtype).
 * Saved: lse [rows] fp32 (logsumexp of each row) and n_valid, one fp32 (the
 * number of rows whose target != ignore_index). A target outside [0, cols) that
 * is not ignore_index makes the loss NaN. rows == 0 gives NaN (0/0), as torch.
 * Workspace: eg_cross_entropy_workspace_bytes(rows). */
int eg_cross_entropy_fwd(const void* logits, const int64_t* target, void* loss, float* lse,
                         float* n_valid, void* workspace, int64_t rows, int64_t cols,
                         int64_t ignore_index, int dtype, void* stream);

/* Bytes of workspace eg_cross_entropy_fwd needs: one fp32 row loss per row. */
size_t eg_cross_entropy_workspace_bytes(int64_t rows);

/* Backward of eg_cross_entropy_fwd, the rule declared at
 * src/evograd/ops/level1/cross_entropy/__init__.py:91-94:
 *   dlogits = dloss * (softmax(logits) - onehot(target)) / n_valid,
 * zero on rows whose target is ignore_index. dloss is one element (dtype) in
 * device memory; dlogits [rows, cols] (dtype). */
int eg_cross_entropy_bwd(const void* dloss, const void* logits, const int64_t* target,
                         const float* lse, const float* n_valid, void* dlogits, int64_t rows,
                         int64_t cols, int64_t ignore_index, int dtype, void* stream);

/* Mean of per-row losses: loss = sum(rowloss[r] over rows with target[r] !=
 * ignore_index) / n_valid, written in loss_dtype; n_valid (one fp32) is the count.
 * Ignored rows must hold rowloss 0 (as eg_cross_entropy_fwd writes them). The reduction
 * of cross_entropy_forward_ref (src/evograd/ops/level1/cross_entropy/forward_ref.py:9-11)
 * over rows whose losses were produced chunk by chunk. */
int eg_cross_entropy_mean(const int64_t* target, const float* rowloss, void* loss,
                          float* n_valid, int64_t rows, int64_t ignore_index, int loss_dtype,
                          void* stream);

/* --------------------------------------------- fused linear cross entropy
 * Replaces fused_linear_cross_entropy_forward_ref
 * (src/evograd/ops/level2/fused_linear_cross_entropy/forward_ref.py:23-35) and
 * forms its gradient (declared at fused_linear_cross_entropy/__init__.py:91-152)
 * in the same pass, one chunk of rows at a time, every product on this library's
 * MFMA kernels:
 *   logits_c = x_c @ weight.T (fp32 accumulation; 16-bit inputs: the softmax terms
 *            are formed in the product's epilogue and no fp32 logits are stored;
 *            fp32 inputs: one chunk of fp32 logits)
 *   loss = mean over rows with target != ignore_index of lse - logits[target] (fp32)
 *   dl_c = softmax(logits_c) - onehot(target) (dtype; zero on ignored rows)
 *   dx_c = dl_c @ weight; dweight = sum over chunks of dl_c.T @ x_c (16-bit inputs
 *            over several chunks: summed in an fp32 [vocab, hidden] buffer of the
 *            workspace and rounded once; fp32 inputs: summed in dweight)
 *   n_valid = the number of counted rows (fp32)
 * Neither the logits nor dl of all rows exist at once: the workspace
 * (eg_flce_workspace_bytes, same chunk_rows and dtype) holds dl of one chunk, the
 * softmax group statistics of one chunk (16-bit) or one chunk of fp32 logits
 * (fp32), two fp32 values per row and, for 16-bit inputs over more than one
 * chunk, the fp32 dweight sum. chunk_rows <= 0 takes the default: as many rows as
 * 1 GiB of dl allows.
 * x [rows, hidden], weight [vocab, hidden], dx, dweight as their inputs (dtype);
 * target int64 [rows]; a target outside [0, vocab) that is not ignore_index
 * gives NaN. 16-bit inputs need hidden % 64 == 0. The backward scales dx and
 * dweight by dloss / n_valid (eg_scale_copy). */
size_t eg_flce_workspace_bytes(int64_t rows, int64_t hidden, int64_t vocab, int64_t chunk_rows,
                               int dtype);
int eg_flce_fwd(const void* x, const void* weight, const int64_t* target, float* loss, void* dx,
                void* dweight, float* n_valid, void* workspace, int64_t rows, int64_t hidden,
                int64_t vocab, int64_t ignore_index, int64_t chunk_rows, int dtype,
                void* stream);

/* dst[i] = src[i] * mul[0] / div[0] for n elements, with conversion from src_dtype
 * to dst_dtype; mul (of mul_dtype) and div (fp32) are device scalars and either
 * may be NULL (factor 1); a zero *div gives factor 0. Applies dloss / n_valid to the fused linear cross
 * entropy's saved gradients (the chain rule of
 * src/evograd/ops/level2/fused_linear_cross_entropy/__init__.py:116-123). */
int eg_scale_copy(const void* src, int src_dtype, void* dst, int dst_dtype, int64_t n,
                  const void* mul, int mul_dtype, const float* div, void* stream);

/* ------------------------------------------------------------ dense product
 * The products inside fused_linear_cross_entropy (the logits x @ weight.T of
 * src/evograd/ops/level2/fused_linear_cross_entropy/forward_ref.py:23-35 and the
 * dx = dlogits @ weight, dweight = dlogits.T @ x of its gradient) and inside the
 * Llama-3 decoder layer (the F.linear projections and residual adds of
 * src/evograd/ops/level3/llama3_decoder_layer/forward_ref.py:91-117 and their
 * gradients), on MFMA:
 *   c[m][n] = r[m][n] + sum_k a(m, k) b(k, n)   (fp32 accumulation; bf16/fp16
 *             operands on MFMA, fp32 operands on a plain tiled path; r may be NULL
 *             for none, and r == c with ldr == ldc accumulates in place)
 * a_k_contiguous: a(m, k) = a[m * lda + k], else a[k * lda + m];
 * b_k_contiguous: b(k, n) = b[n * ldb + k], else b[k * ldb + n];
 * c [m][ldc] and r [m][ldr] in c_dtype (EG_F32 or dtype); r is added in fp32
 * before c is rounded. A 16-bit k-contiguous operand needs k % 64 == 0, or, when the
 * other operand is k-major, a row stride of at least k rounded up to 64 whose columns
 * past k hold finite values (zeros); strides are multiples of 8 elements and a, b are
 * 16-byte aligned.
 * Products with at most half as many output tiles (256 x 256) as an MI355X has CUs
 * split k over workgroups when `workspace` holds at least
 * eg_gemm_workspace_bytes(m, n, k, dtype) bytes (else, or with workspace NULL, they
 * run unsplit): each k range writes an fp32 partial, and a second pass sums them in
 * a fixed order, adds r and rounds c once. So do the tiles of a last wave that is at most half full (more than 256
 * tiles). The split depends on the shape only, so results are bitwise repeatable. */
size_t eg_gemm_workspace_bytes(int64_t m, int64_t n, int64_t k, int dtype);
int eg_gemm(const void* a, const void* b, void* c, const void* r, int64_t m, int64_t n,
            int64_t k, int64_t lda, int64_t ldb, int64_t ldc, int64_t ldr, int a_k_contiguous,
            int b_k_contiguous, int dtype, int c_dtype, void* workspace, size_t workspace_bytes,
            void* stream);

/* eg_gemm over operands that are concatenations of up to 4 buffers along one
 * dimension (no counterpart call in the reference; it runs several of the decoder
 * layer's F.linear calls of forward_ref.py:89-91 and :115-116, and their gradients,
 * as one product): seg_dim 1 (M), 2 (N) or 3 (K); seg_sizes[i] is segment i's extent
 * along it (all but the last a multiple of 256 for M and N, of 64 for K; they add up
 * to m, n or k). a_segs, b_segs, c_segs (arrays of nseg pointers, or NULL for an
 * operand that is the single buffer a, b or c) point at the first element of each
 * segment of the operands the dimension indexes: along M, rows of A (columns of a
 * k-major A) and rows of C; along N, B's rows (columns of a k-major B) and C's
 * columns; along K, A and B. Segments of one operand share its row stride. No
 * residual; workspace as for eg_gemm (eg_gemm_workspace_bytes of the whole shape). */
int eg_gemm_segmented(const void* a, const void* b, void* c, int64_t m, int64_t n, int64_t k,
                      int64_t lda, int64_t ldb, int64_t ldc, int a_k_contiguous,
                      int b_k_contiguous, int seg_dim, int nseg, const int64_t* seg_sizes,
                      const void* const* a_segs, const void* const* b_segs, void* const* c_segs,
                      int dtype, int c_dtype, void* workspace, size_t workspace_bytes,
                      void* stream);

/* ---------------------------------------------- decoder layer: layout, adds
 * The steps of the Llama-3 decoder layer
 * (src/evograd/ops/level3/llama3_decoder_layer/forward_ref.py:91-117) between its
 * products (eg_gemm), norms (eg_rmsnorm_*) and attention (eg_attn_gqa_*).
 *
 * eg_split_heads: src [batch * tokens, ld] (each token row holds heads x head_dim
 * values from column 0) -> dst [batch, heads, tokens, head_dim]: the
 * .view(batch, tokens, heads, head_dim).transpose(1, 2) of :94-96. rope = 1 also
 * applies _apply_rope (:43-47, :98-99): y = x cos + [-x2, x1] sin in fp32, cast
 * back, with cos, sin [tokens, head_dim] of table_dtype (EG_F32 or dtype); rope = 0
 * copies (tables may be NULL).
 * eg_merge_heads: the inverse layout change, src [batch, heads, tokens, head_dim] ->
 * dst [batch * tokens, ld] (attn.transpose(1, 2).reshape(...) of :109); rope = 2
 * applies the rotation's transpose dx = dy cos + [dy2, -dy1] sin on the way (the
 * gradient of the rotated q and k), rope = 0 copies. Columns of dst past
 * heads x head_dim are not written. */
int eg_split_heads(const void* src, void* dst, const void* cos, const void* sin, int64_t batch,
                   int64_t tokens, int64_t heads, int64_t head_dim, int64_t ld, int rope,
                   int table_dtype, int dtype, void* stream);
int eg_merge_heads(const void* src, void* dst, const void* cos, const void* sin, int64_t batch,
                   int64_t tokens, int64_t heads, int64_t head_dim, int64_t ld, int rope,
                   int table_dtype, int dtype, void* stream);

/* eg_split_heads / eg_merge_heads for the q, k and v of one fused projection in one
 * launch (the [q | k | v] output of the layer's single product over Wq, Wk, Wv):
 * each token row of src (split) or dst (merge) [batch * tokens, ld] holds heads_q
 * query heads, then heads_kv key heads, then heads_kv value heads of head_dim
 * from column 0; q is [batch, heads_q, tokens, head_dim], k and v
 * [batch, heads_kv, tokens, head_dim]. rope (0, 1 or 2 as above) applies to the
 * query and key heads; value heads are copied. */
int eg_split_qkv_heads(const void* src, void* q, void* k, void* v, const void* cos,
                       const void* sin, int64_t batch, int64_t tokens, int64_t heads_q,
                       int64_t heads_kv, int64_t head_dim, int64_t ld, int rope, int table_dtype,
                       int dtype, void* stream);
int eg_merge_qkv_heads(const void* q, const void* k, const void* v, void* dst, const void* cos,
                       const void* sin, int64_t batch, int64_t tokens, int64_t heads_q,
                       int64_t heads_kv, int64_t head_dim, int64_t ld, int rope, int table_dtype,
                       int dtype, void* stream);

/* c = a + b over n elements (fp32 sum, one rounding): where a residual
 * connection's gradient meets a norm's (forward_ref.py:110 and :117, backward). */
int eg_add(const void* a, const void* b, void* c, int64_t n, int dtype, void* stream);

/* out = (silu(gate.float()) * up.float()).to(dtype) over n elements, one rounding:
 * the MLP activation of forward_ref.py:115-116 (unlike the level-1 SwiGLU, which
 * rounds silu first). Its backward is eg_swiglu_bwd's formula. */
int eg_silu_mul(const void* gate, const void* up, void* out, int64_t n, int dtype, void* stream);

/* ---- measurement aid (no counterpart in the reference) ---------------------
 * Sustained bf16 MFMA rate, for reading the roofline fractions of the MFMA-bound
 * kernels (bench.py reports it beside the published peak): `workgroups` 256-thread
 * workgroups (pass the CU count: one per CU, one wave per SIMD) each run `iters`
 * iterations of 64 v_mfma_f32_32x32x16_bf16 per wave from registers, on operands
 * taken from `operands` (32 KiB, 16-byte aligned, random bf16 values: the clock
 * the device holds depends on how much the operand bits toggle). Work:
 * workgroups x 4 x iters x 64 x 32768 FLOP. `out` receives workgroups x 256 floats
 * (checksums that keep the work live). */
int eg_probe_mfma_bf16(const void* operands, float* out, int workgroups, int iters, void* stream);

/* Measurement aid (no counterpart in the reference): the same 64 x 32768 FLOP per
 * wave and iteration as eg_probe_mfma_bf16, in one of four loops, for the ceilings
 * bench.py reports beside the MFMA-bound kernels' fractions:
 *   kind 0: eg_probe_mfma_bf16's loop (32 x 32 x 16 from registers, one wave per
 *           SIMD: pass the CU count as `workgroups`);
 *   kind 1: 128 v_mfma_f32_16x16x32_bf16 from registers (pass twice the CU count:
 *           two waves per SIMD);
 *   kind 2: 64 v_mfma_f32_32x32x16_bf16 each fed one ds_read_b128 of the operands
 *           staged in LDS, 1 KiB per wave and MFMA as in the attention kernels
 *           (twice the CU count);
 *   kind 3: kind 2 plus one v_exp_f32 per MFMA (the softmax's exponentials).
 * Operands, out and the checksums as for eg_probe_mfma_bf16. */
int eg_probe_mfma_mix(int kind, const void* operands, float* out, int workgroups, int iters,
                      void* stream);

#ifdef __cplusplus
}
#endif

#endif /* EVOGRAD_HIP_H */
