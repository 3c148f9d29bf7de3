/*
 * femtohip.h — C ABI of the MI355X (gfx950) kernels behind the fused
 * activation-checkpointed Llama decoder layer.
 *
 * The reference path this library replaces is one checkpointed
 * `LlamaDecoderLayer` call: the `checkpoint_fn` hook of
 * femtotron/training/activation_ckpt.py:25-26,78-86 (invoked per layer from
 * femtotron/model/llama_partial_model.py:205-215), which by default runs
 * torch.utils.checkpoint.checkpoint around the Hugging Face layer
 * (transformers 5.15.0, models/llama/modeling_llama.py:284-325).  The reference
 * has no native code of its own; each entry point below names the aten op
 * chain of that layer it stands in for.
 *
 * Conventions
 *   - Every pointer is a device pointer owned by the caller; the library never
 *     allocates or frees device memory.  Scratch space is passed in as a
 *     `workspace` whose size the matching *_workspace_size() call returns.
 *   - Tensors are row-major.  `ld*` arguments are row strides in elements.
 *   - Calls are asynchronous on `stream` (a hipStream_t; 0 = null stream)
 *     and never synchronise the host.
 *   - Return value: FH_OK (0) or an FH_ERR_* code; fh_last_error() then holds
 *     a message for the calling thread.  Nothing aborts the process.
 *   - Thread-safe: the library's own global state is the per-thread error
 *     string, per-device values looked up once under std::call_once (compute
 *     unit count, the scratch address below), and one device buffer: the
 *     file-scope scratch array of fh_rmsnorm_bwd_noalloc, shared by every
 *     call of that entry point on a device, so calls of it that overlap on
 *     one device (two host threads, or two streams) race on its contents.
 *     Every other entry point works only on the caller's buffers.
 */
#ifndef FEMTOHIP_H_
#define FEMTOHIP_H_

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FH_ABI_VERSION 6

typedef enum fh_dtype {
  FH_BF16 = 0, /* bfloat16 storage, fp32 arithmetic */
  FH_F32 = 1   /* float32 storage and arithmetic     */
} fh_dtype;

enum {
  FH_OK = 0,
  FH_ERR_INVALID = 1,     /* bad shape / stride / alignment / dtype */
  FH_ERR_LAUNCH = 2,      /* hipLaunchKernel (or a HIP call) failed  */
  FH_ERR_UNSUPPORTED = 3  /* valid but not implemented configuration */
};

/* Library ABI version (FH_ABI_VERSION of the build). */
int fh_abi_version(void);

/* Message describing the last failing call on this thread ("" if none). */
const char* fh_last_error(void);

/* ------------------------------------------------------------------ RMSNorm
 * Replaces LlamaRMSNorm.forward (modeling_llama.py:62-67):
 *   y = w * to_dtype(x_f32 * rsqrt(mean(x_f32^2) + eps))
 * x, y: [rows, cols]; w: [cols].  rstd (nullable): fp32 [rows] receives
 * rsqrt(mean(x^2)+eps).  cols % 8 == 0, cols <= 8192, 16-byte aligned rows.
 */
int fh_rmsnorm_fwd(fh_dtype dt, const void* x, const void* w, void* y,
                   float* rstd, int64_t rows, int64_t cols, float eps,
                   hipStream_t stream);

/* Residual add followed by RMSNorm: the `residual + hidden_states` at
 * modeling_llama.py:317 feeding post_attention_layernorm (:320).
 *   h = to_dtype(x + a);  y = rmsnorm(h) as above.
 * h may alias neither x nor a.  rstd nullable.
 */
int fh_add_rmsnorm_fwd(fh_dtype dt, const void* x, const void* a,
                       const void* w, void* h, void* y, float* rstd,
                       int64_t rows, int64_t cols, float eps,
                       hipStream_t stream);

/* Bytes of fp32 workspace fh_rmsnorm_bwd needs for (rows, cols). */
size_t fh_rmsnorm_bwd_workspace_size(int64_t rows, int64_t cols);

/* Backward of LlamaRMSNorm (autograd of modeling_llama.py:62-67), fused with
 * the residual-branch gradient of the add at modeling_llama.py:317/323:
 *   dn  = to_dtype(dy * w)
 *   dx  = to_dtype(r * (dn - n * mean(dn * n)) + dres)   (n = x*r, r = rstd)
 *   dw  = sum_rows dy * to_dtype(n)
 * rstd nullable (recomputed from x and eps); dres nullable (no residual).
 * dw: [cols] in dtype dt, overwritten.  workspace: see above, 16-byte
 * aligned like every other pointer (the partial rows are read as float4).
 */
int fh_rmsnorm_bwd(fh_dtype dt, const void* dy, const void* x, const void* w,
                   const float* rstd, const void* dres, void* dx, void* dw,
                   void* workspace, int64_t rows, int64_t cols, float eps,
                   hipStream_t stream);

/* fh_rmsnorm_bwd without a workspace argument.  No counterpart in the
 * reference (whose RMSNorm backward is autograd over aten ops): it is for
 * callers that cannot allocate device memory -- code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc.  Same arguments,
 * results (bit for bit) and errors as fh_rmsnorm_bwd; the fp32 partial rows go
 * to a scratch array the library holds in device memory, one per device
 * (fh_rmsnorm_bwd_noalloc_max_workspace() bytes, 16.8 MB, enough for every
 * valid rows x cols since cols <= 8192), kept until the process ends.  Calls
 * no allocating routine.  All calls on one device share that scratch: calls
 * that may overlap on one device (different streams, or different host
 * threads, without ordering between them) race and must be serialised by the
 * caller.  The first call on each device looks up the scratch's device
 * address (hipGetSymbolAddress) once.
 */
size_t fh_rmsnorm_bwd_noalloc_max_workspace(void);
int fh_rmsnorm_bwd_noalloc(fh_dtype dt, const void* dy, const void* x, const void* w,
                           const float* rstd, const void* dres, void* dx, void* dw,
                           int64_t rows, int64_t cols, float eps, hipStream_t stream);

/* --------------------------------------------------------------------- RoPE
 * In-place rotate-half rotary embedding, replacing apply_rotary_pos_emb +
 * rotate_half (modeling_llama.py:130-160) for q and k together:
 *   out[i]      = x[i]*cos[i]      - x[i+d/2]*sin[i]
 *   out[i+d/2]  = x[i+d/2]*cos[i+d/2] + x[i]*sin[i+d/2]        (i < d/2)
 * with the same bf16 rounding points as the reference (each product, then
 * the sum).  qk: [tokens, ld]; heads 0..n_heads-1 at columns h*head_dim.
 * Token t is (batch t / seq_len, position t % seq_len).  cos/sin:
 * [seq_len, head_dim] (cos_per_token == 0, i.e. shape [1,S,hd]) or
 * [tokens, head_dim] (cos_per_token != 0, shape [B,S,hd]).
 * head_dim % 16 == 0.
 */
int fh_rope_fwd(fh_dtype dt, void* qk, int64_t ld, int64_t tokens,
                int64_t seq_len, int64_t n_heads, int64_t head_dim,
                const void* cos, const void* sin, int cos_per_token,
                hipStream_t stream);

/* Backward of fh_rope_fwd (rotation by the transposed matrix), in place on
 * the gradient buffer with the same layout arguments. */
int fh_rope_bwd(fh_dtype dt, void* dqk, int64_t ld, int64_t tokens,
                int64_t seq_len, int64_t n_heads, int64_t head_dim,
                const void* cos, const void* sin, int cos_per_token,
                hipStream_t stream);

/* ------------------------------------------------------------------- SwiGLU
 * Replaces `act_fn(gate_proj(x)) * up_proj(x)` (modeling_llama.py:174-176,
 * act_fn = SiLU, activations.py:93-103):  p = to_dtype(to_dtype(silu(g)) * u)
 * g, u: [rows, cols] with row stride ld_gu; p: row stride ld_p.
 * cols % 8 == 0.
 */
int fh_swiglu_fwd(fh_dtype dt, const void* g, const void* u, int64_t ld_gu,
                  void* p, int64_t ld_p, int64_t rows, int64_t cols,
                  hipStream_t stream);

/* Backward of fh_swiglu_fwd:
 *   du = dp * to_dtype(silu(g))
 *   dg = to_dtype(dp*u) * sig(g) * (1 + g*(1 - sig(g)))
 * dg, du share row stride ld_dgu (they may be the two halves of one buffer).
 * p (optional, may be NULL; row stride ld_p): also writes the forward's
 * product p = to_dtype(to_dtype(silu(g)) * u), bit for bit what fh_swiglu_fwd
 * writes, for a recompute that stops before the product (the down
 * projection's weight gradient reads it after this call).  p may be dp itself
 * (same ld), which this call then overwrites; no other overlap.
 */
int fh_swiglu_bwd(fh_dtype dt, const void* dp, int64_t ld_dp, const void* g,
                  const void* u, int64_t ld_gu, void* dg, void* du,
                  int64_t ld_dgu, void* p, int64_t ld_p, int64_t rows,
                  int64_t cols, hipStream_t stream);

/* Elementwise residual add out = to_dtype(a + b) over n elements
 * (modeling_llama.py:323).  n % 8 == 0; out may alias a or b. */
int fh_add(fh_dtype dt, const void* a, const void* b, void* out, int64_t n,
           hipStream_t stream);

/* out = to_dtype(x * scale[0]) over n elements, scale a device fp32 scalar:
 * the chain rule of a saved gradient times the incoming gradient of a scalar
 * loss, `(g_saved * grad).to(dtype)` in torch (the fused loss head's backward;
 * the reference's loss backward is autograd over aten ops, model/llama.py:91-111).
 * n % 8 == 0; out may alias x. */
int fh_scale(fh_dtype dt, const void* x, void* out, int64_t n, const float* scale,
             hipStream_t stream);

/* ---------------------------------------------------------------- attention
 * Causal GQA softmax attention, replacing F.scaled_dot_product_attention(
 * q, k, v, is_causal=True, enable_gqa=True, scale) as called from
 * sdpa_attention_forward (transformers integrations/sdpa_attention.py:79-166)
 * by LlamaAttention (modeling_llama.py:235-281), forward and backward.
 * Token-major layouts: row t = b*seq_len + s; query head h occupies columns
 * h*head_dim.. of q/o/dout/dq (row strides ldq, ldo, ...), kv head j columns
 * j*head_dim.. of k/v/dk/dv; q head h reads kv head h / (n_heads/n_kv_heads).
 * head_dim in {32, 64, 128}; strides multiples of 8 and < 2^24; 16-byte
 * aligned bases.
 * FH_BF16 runs on MFMA (fp32 softmax/accumulation); FH_F32 in fp32 FMA.
 * lse: fp32 [batch, n_heads, seq_len], natural-log row log-sum-exp of the
 * scaled scores (nullable in the forward).
 */
int fh_attn_fwd(fh_dtype dt, const void* q, int64_t ldq, const void* k, int64_t ldk,
                const void* v, int64_t ldv, void* o, int64_t ldo, float* lse,
                int64_t batch, int64_t seq_len, int64_t n_heads, int64_t n_kv_heads,
                int64_t head_dim, float scale, hipStream_t stream);

/* fh_attn_fwd with the RoPE forward applied to q as it is loaded: the result
 * equals, bit for bit, fh_rope_fwd over q's n_heads heads followed by
 * fh_attn_fwd (apply_rotary_pos_emb then SDPA, modeling_llama.py:130-160,
 * 256-271).  k must arrive rotated (fh_rope_fwd over the kv heads); q is read
 * unrotated.  q_out (nullable; may be q itself with ldqo == ldq) receives the
 * rotated q, which the backward reads.  cos/sin as in fh_rope_fwd (same dtype,
 * [seq_len, head_dim] or, with cos_per_token != 0, [batch*seq_len, head_dim]),
 * 16-byte aligned.
 */
int fh_attn_fwd_rope(fh_dtype dt, const void* q, int64_t ldq, const void* k, int64_t ldk,
                     const void* v, int64_t ldv, void* o, int64_t ldo, float* lse, void* q_out,
                     int64_t ldqo, int64_t batch, int64_t seq_len, int64_t n_heads,
                     int64_t n_kv_heads, int64_t head_dim, float scale, const void* cos,
                     const void* sin, int cos_per_token, hipStream_t stream);

/* Bytes of workspace fh_attn_bwd needs (per query, fp32: rowsum(dO*O) and the
 * lse in log2 units). */
size_t fh_attn_bwd_workspace_size(int64_t batch, int64_t seq_len, int64_t n_heads);

/* Gradients of fh_attn_fwd given o, lse and dout: writes dq, dk, dv (each
 * fully overwritten; the kv-head gradients already summed over the query
 * heads sharing them). */
int fh_attn_bwd(fh_dtype dt, const void* q, int64_t ldq, const void* k, int64_t ldk,
                const void* v, int64_t ldv, const void* o, int64_t ldo,
                const void* dout, int64_t lddo, const float* lse, void* dq,
                int64_t lddq, void* dk, int64_t lddk, void* dv, int64_t lddv,
                void* workspace, int64_t batch, int64_t seq_len, int64_t n_heads,
                int64_t n_kv_heads, int64_t head_dim, float scale, hipStream_t stream);

/* fh_attn_bwd with the RoPE backward fused into the dq and dk stores: the
 * result equals, bit for bit, fh_attn_bwd followed by fh_rope_bwd over dq's
 * n_heads heads and over dk's n_kv_heads heads, i.e. the gradients with
 * respect to the projections' outputs before apply_rotary_pos_emb
 * (modeling_llama.py:130-160, 256).  cos/sin as in fh_rope_fwd (same dtype as
 * the gradients, [seq_len, head_dim] or, with cos_per_token != 0,
 * [batch*seq_len, head_dim]), 16-byte aligned.
 */
int fh_attn_bwd_rope(fh_dtype dt, const void* q, int64_t ldq, const void* k, int64_t ldk,
                     const void* v, int64_t ldv, const void* o, int64_t ldo,
                     const void* dout, int64_t lddo, const float* lse, void* dq,
                     int64_t lddq, void* dk, int64_t lddk, void* dv, int64_t lddv,
                     void* workspace, int64_t batch, int64_t seq_len, int64_t n_heads,
                     int64_t n_kv_heads, int64_t head_dim, float scale, const void* cos,
                     const void* sin, int cos_per_token, hipStream_t stream);

/* ------------------------------------------------------------------------
 * Causal-LM cross-entropy, forward and gradient in one pass, in place.
 * Replaces, for one chunk of rows of the logits, the loss head of
 * femtotron/model/llama.py:104-111 and femtotron/model/base.py:24-31:
 *   F.cross_entropy(logits.float().view(-1, V), labels.view(-1), ignore_index=-100)
 * (mean over the rows whose label is not ignore_index) and its autograd
 * gradient (softmax(x) - onehot(label)) / n_valid, rounded to the logits dtype
 * as the backward of .float() does.  The next-token shift is the caller's
 * (labels[b, s] = input label at s+1, ignore_index at each sequence's end).
 *
 * logits: [rows, vocab] row stride ld (FH_BF16 or FH_F32), overwritten with the
 *         gradient; labels: int64 [rows] device; inv_count: device fp32 scalar
 *         1/n_valid; loss_rows: fp32 [rows] = logsumexp(x_r) - x_r[label_r]
 *         (0 for ignored rows; NaN, with a NaN gradient row, for a label
 *         outside [0, vocab)).  The loss is sum(loss_rows) * inv_count.
 * fp32 log-sum-exp; deterministic (fixed-order reductions).
 */
int fh_ce_fwd_bwd(fh_dtype dt, void* logits, int64_t ld, const int64_t* labels, int64_t rows,
                  int64_t vocab, int64_t ignore_index, const float* inv_count, float* loss_rows,
                  hipStream_t stream);

/* ------------------------------------------------------------------------
 * Mixed-precision AdamW step with global gradient-norm clipping.
 * Replaces femtotron/training/mixed_precision_manager.py:318-331 (step():
 * master.grad = param.grad.float(); ClipGradNorm of grad_transform.py:13-63;
 * torch.optim.AdamW on the fp32 masters, femtotron/scripts/train.py:264-276; param.copy_(master),
 * param_group.py:82-87) for every tensor of one device in two passes over the
 * gradients.  table: device array of n_tensors FhAdamTensor; chunk_start:
 * device int64 [n_tensors + 1], chunk_start[i] = sum over j < i of
 * ceil(numel_j / 2048), chunk_start[n] = total_chunks.  All pointers 16-byte
 * aligned; param/grad in dt (FH_BF16 or FH_F32), the rest fp32.
 * hyper: the betas and eps.  Per tensor: decay = 1 - lr * wd and the bias
 * corrections of the tensor's own step count t (torch.optim.AdamW counts steps
 * per parameter, skipping parameters without a gradient): step_size =
 * lr / (1 - beta1^t), bias_correction2_sqrt = sqrt(1 - beta2^t).
 * max_grad_norm <= 0 disables clipping.  workspace: fh_adamw_workspace_size
 * bytes; after the call it holds, at float index total_chunks, the clipping
 * coefficient and then the gradient norm (before clipping).
 */
typedef struct {
  void* param;            /* model-dtype parameter (receives the cast master) */
  const void* grad;       /* model-dtype gradient */
  float* master;          /* fp32 master weights */
  float* exp_avg;         /* fp32 first moment */
  float* exp_avg_sq;      /* fp32 second moment */
  int64_t numel;
  float decay;                  /* 1 - lr * weight_decay of this tensor's group */
  float step_size;              /* lr / (1 - beta1^t), t = this tensor's step */
  float bias_correction2_sqrt;  /* sqrt(1 - beta2^t), > 0 */
  float reserved;
} FhAdamTensor;

typedef struct {
  float one_minus_beta1;
  float beta2;
  float one_minus_beta2;
  float eps;
} FhAdamHyper;

size_t fh_adamw_workspace_size(int64_t total_chunks);
int fh_adamw_step(fh_dtype dt, const FhAdamTensor* table, const int64_t* chunk_start,
                  int n_tensors, int64_t total_chunks, FhAdamHyper hyper, float max_grad_norm,
                  void* workspace, hipStream_t stream);

/* ------------------------------------------------------------------------
 * Token embedding of the first pipeline stage
 * (femtotron/model/llama_partial_model.py:181-184): nn.Embedding, replaced at
 * TP = 1 by VocabParallelEmbedding (femtotron/parallel/tensor_parallel/
 * embedding.py:57-79: ids outside [0, vocab) give zero rows).
 *
 * fh_embedding_fwd: out[t, :] = weight[ids[t], :] for 0 <= ids[t] < vocab,
 * zeros otherwise.  weight [vocab, hidden], out [n_tokens, hidden] (contiguous,
 * FH_BF16 or FH_F32, 16-byte aligned, hidden % 8 == 0); ids int64 on the device.
 */
int fh_embedding_fwd(fh_dtype dt, const void* weight, const int64_t* ids, void* out,
                     int64_t n_tokens, int64_t vocab, int64_t hidden, hipStream_t stream);

/* Bytes of workspace fh_embedding_bwd needs. */
size_t fh_embedding_bwd_workspace_size(int64_t n_tokens, int64_t vocab);

/* Backward of the lookup (F.embedding's weight gradient, the reference's
 * scatter-add): dweight[v, :] = sum over tokens t with ids[t] == v of
 * dy[t, :], accumulated in fp32 in ascending t and rounded once; every row of
 * dweight [vocab, hidden] is written (zeros for ids no token uses).  Tokens
 * whose id is outside [0, vocab) or equals padding_idx (nn.Embedding's; pass
 * -1 for none) contribute nothing.  Deterministic: a stable radix sort of the
 * ids, no floating-point atomics; n_tokens, vocab < 2^31.
 */
int fh_embedding_bwd(fh_dtype dt, const void* dy, const int64_t* ids, void* dweight,
                     int64_t n_tokens, int64_t vocab, int64_t hidden, int64_t padding_idx,
                     void* workspace, hipStream_t stream);

/* ------------------------------------------------------------------------
 * GEMMs of the layer's seven projections, the F.linear of femtotron's
 * Column/RowParallelLinear at one rank (femtotron/parallel/tensor_parallel/
 * linear.py:66-80 forward, :194-214; HF nn.Linear) in its three layouts:
 *   FH_GEMM_NT  C[m,n] = sum_k A[m,k] B[n,k]   A [m,k], B [n,k]   y = x W^T
 *   FH_GEMM_NN  C[m,n] = sum_k A[m,k] B[k,n]   A [m,k], B [k,n]   dx = dy W
 *   FH_GEMM_TN  C[m,n] = sum_k A[k,m] B[k,n]   A [k,m], B [k,n]   dW = dy^T x
 * bf16, row-major with leading dims lda/ldb/ldc (elements); fp32 accumulation,
 * C rounded to bf16 once, as torch's bf16 matmul does.  If `residual` (bf16
 * [m, n], row stride ldr) is given, C = to_bf16(residual + to_bf16(A.B)): the
 * projection output rounded, then the residual add `hidden_states = residual +
 * hidden_states` of modeling_llama.py:323 fused into the epilogue with its own
 * rounding.  `residual` may be C itself (same ldc), any other overlap is not
 * allowed.  With residual == C this is the accumulating epilogue (alpha =
 * beta = 1) of gradient accumulation: FH_GEMM_TN into an existing bf16 weight
 * gradient gives C = to_bf16(C + to_bf16(dY^T X)), bit for bit autograd's
 * `param.grad += new_grad` after the GEMM rounded new_grad (the in-place
 * accumulation of femtotron/training/grad_accumulator.py:24-36 with
 * grad_acc_dtype None).
 * Requirements: k % 64 == 0; n % 8 == 0 (and m % 8 == 0 for FH_GEMM_TN);
 * lda, ldb, ldc and ldr multiples of 8 (< 2^26 for lda, ldb); A, B, C and the
 * residual 16-byte aligned; m, n, k < 2^30.
 * When the output has few 256 x 256 tiles the k range is split into slices
 * whose fp32 partial sums go to `workspace` (fh_gemm_bf16_workspace_size bytes;
 * 0 = none needed) and are added in slice order; when its tiles leave the
 * last round of CUs partly idle, each CU instead takes an equal share of the
 * k-steps and the tiles split between CUs are summed from fp32 segments in
 * `workspace` in k order.  Either way results are bitwise deterministic (the
 * form depends only on m, n, k and the device's CU count).
 */
typedef enum fh_gemm_op {
  FH_GEMM_NT = 0,
  FH_GEMM_NN = 1,
  FH_GEMM_TN = 2
} fh_gemm_op;

size_t fh_gemm_bf16_workspace_size(int op, int64_t m, int64_t n, int64_t k);
int fh_gemm_bf16(int op, const void* a, int64_t lda, const void* b, int64_t ldb, void* c,
                 int64_t ldc, const void* residual, int64_t ldr, int64_t m, int64_t n,
                 int64_t k, void* workspace, hipStream_t stream);

/* Up to three GEMMs of one layout and one k in one launch: problem i is
 * fh_gemm_bf16(op, a, lda, b, ldb, c, ldc, residual, ldr, m, n, k) of its
 * fields, with the same roundings, requirements and residual rules.  The
 * layer's weight gradients that read the same tokens (k = tokens: q/k/v, o and
 * down, each with few output tiles) run together this way
 * (femtotron/parallel/tensor_parallel/linear.py:66-80, 194-214 backward,
 * accumulated as fh_gemm_bf16's residual == C).  When the problems' tiles
 * together fill more than one round of the CUs they share one launch in the
 * stream form (every CU an equal share of the group's k-steps, problem by
 * problem; split tiles summed in k order from fp32 segments in `workspace`);
 * otherwise each runs as its own fh_gemm_bf16 call.  Bitwise deterministic
 * (the form depends only on the problems' sizes, k and the CU count); a
 * problem's result may differ in the last bit from its own fh_gemm_bf16 call,
 * whose form may split k differently.  The problems' outputs must not overlap
 * each other's operands or outputs.  The reference runs each of these
 * weight-gradient matmuls on its own.
 */
typedef struct fh_gemm_problem {
  const void* a;
  int64_t lda;
  const void* b;
  int64_t ldb;
  void* c;
  int64_t ldc;
  const void* residual;
  int64_t ldr;
  int64_t m;
  int64_t n;
} fh_gemm_problem;

/* Workspace bytes for fh_gemm_bf16_grouped (reads the problems' m and n only;
 * 0 for invalid sizes or when none is needed). */
size_t fh_gemm_bf16_grouped_workspace_size(int op, int count, const fh_gemm_problem* problems, int64_t k);
int fh_gemm_bf16_grouped(int op, int count, const fh_gemm_problem* problems, int64_t k, void* workspace,
                         hipStream_t stream);

/* The q/k/v projection with the rotary embedding in its epilogue: C = A B^T
 * (FH_GEMM_NT, no residual) and then, on columns [0, rot_cols) of C (the q and
 * k heads of head_dim columns each), the rotation of fh_rope_fwd -- bit for
 * bit fh_gemm_bf16 followed by fh_rope_fwd(FH_BF16, c, ldc, m, seq_len,
 * rot_cols / head_dim, head_dim, cos, sin, cos_per_token), i.e.
 * apply_rotary_pos_emb(q_proj(x), k_proj(x)) of modeling_llama.py:130-160,
 * 253-256.  Rows of C are tokens (row t at position t % seq_len; m a multiple
 * of seq_len unless cos_per_token).  head_dim in {32, 64, 128}; rot_cols a
 * multiple of head_dim, at most n; cos/sin bf16 [seq_len or m, head_dim],
 * 16-byte aligned.  K is never split: no workspace.
 */
int fh_gemm_bf16_rope(const void* a, int64_t lda, const void* b, int64_t ldb, void* c,
                      int64_t ldc, int64_t m, int64_t n, int64_t k, int64_t rot_cols,
                      int64_t head_dim, int64_t seq_len, const void* cos, const void* sin,
                      int cos_per_token, hipStream_t stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* FEMTOHIP_H_ */
