/*
 * cobra_amd -- C ABI of the MI355X (gfx950) attention-sublayer forward.
 *
 * The reference (dalberrt/COBRA-GPU-Kernel) is a single Python file whose GPU
 * path is five Triton kernels behind Python launchers; it has no native ABI.
 * Each entry point below replaces one of those launchers (cited as
 * torch_transformer_benchmark.py:LINE, "TTB"), so a host that used the
 * reference's ops can bind these symbols instead (ctypes / cffi / any FFI).
 *
 * Conventions shared by every entry point:
 *   - all tensors are device pointers to row-major, densely packed buffers,
 *     16-byte aligned; the caller allocates every buffer (outputs included);
 *   - dtype codes: COBRA_F16 (IEEE half), COBRA_F32, and COBRA_BF16 (bfloat16)
 *     where an entry point says so;
 *   - `stream` is a hipStream_t (NULL = legacy default stream).  Work is only
 *     enqueued: nothing allocates, frees or synchronises, so every call may be
 *     captured into a hipGraph;
 *   - the return value is a hipError_t code: 0 on success, non-zero when the
 *     arguments are rejected (nothing is enqueued then) or the launch failed.
 *     cobra_error_string() names it.  No C++ exception crosses the ABI;
 *   - a call with no rows (M, rows, batch or seq_len 0) checks its shape and dtype
 *     arguments and returns 0 without reading any pointer or enqueueing work, so
 *     empty tensors (whose data pointers may be NULL) pass through.
 */
#ifndef COBRA_AMD_H
#define COBRA_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define COBRA_ABI_VERSION 11

enum { COBRA_F16 = 0, COBRA_F32 = 1, COBRA_BF16 = 2 };

/*
 * Epilogue / row-mask flags (bit set), applied in this order.  A row mask is
 * one byte per row: 0 = padded row, any other value = valid row.
 *   COBRA_EPI_GELU        v = gelu(v), exact erf form, after the bias
 *                         (the reference GEMM's GELU, TTB:326-328);
 *   COBRA_EPI_MASK_BRANCH padded rows: v = 0 before the residual add (the
 *                         attention output's masked_fill, TTB:121-122);
 *   COBRA_EPI_MASK_RESID  padded rows: (v + resid) * 0, also the stored
 *                         residual (the reference's MASK_RESID, TTB:346-348, 511-516);
 *   COBRA_EPI_MASK_OUT    padded rows: LayerNorm output * 0 (MASK_OUT, TTB:533-534).
 */
enum {
  COBRA_EPI_GELU = 1,
  COBRA_EPI_MASK_BRANCH = 2,
  COBRA_EPI_MASK_RESID = 4,
  COBRA_EPI_MASK_OUT = 8
};

/* ABI version of the loaded library (COBRA_ABI_VERSION it was built with). */
int cobra_version(void);

/* Human-readable name of a code returned by any entry point. */
const char* cobra_error_string(int code);

/*
 * Row LayerNorm with optional residual branch and row mask:
 *     r = x + branch (branch optional);  r *= m (COBRA_EPI_MASK_RESID);
 *     resid_out = r (optional, fp32);
 *     y = (r - mean(r)) * rsqrt(var(r) + eps) * gamma + beta     (biased var)
 *     y *= m (COBRA_EPI_MASK_OUT)
 * x, branch, y: [rows, d]; x and y in any of the three dtypes, branch COBRA_F16 or
 * COBRA_F32; gamma, beta: [d] fp32; row_mask: [rows] bytes
 * (required when mask_flags != 0; only the two flags above are accepted).
 * d <= 4096; pointers aligned to their element size (widths that are multiples of
 * 8 on 16-byte aligned buffers take the vector kernels).  Replaces _tl_add_ln /
 * _add_ln_kernel (TTB:539-569, 491-535).
 */
int cobra_ln_fwd(const void* x, int x_dtype, const void* branch, int branch_dtype, const float* gamma,
                 const float* beta, const uint8_t* row_mask, int mask_flags, float* resid_out, void* y, int y_dtype,
                 int64_t rows, int64_t d, float eps, void* stream);

/*
 * cobra_ln_fwd over the first d columns of row-strided buffers: row i of x, branch,
 * resid_out and y starts ldx, ldb, ldr, ldy elements after row i - 1 (each >= d; 0
 * means d).  With ldy > d, columns d .. ldy-1 of y are written as 0, so y is a
 * zero-padded operand for a GEMM whose K is a multiple of 8.  The statistics and the
 * output cover exactly the d true columns: the counterpart of _add_ln_kernel's masked
 * BLOCK_N columns (TTB:491-535), which normalises rows of any width; this build's
 * stack uses it for d_model / ffn_dim / head_dim that are not multiples of 8.
 * Element alignment suffices.
 */
int cobra_ln_fwd_strided(const void* x, int x_dtype, int64_t ldx, const void* branch, int branch_dtype, int64_t ldb,
                         const float* gamma, const float* beta, const uint8_t* row_mask, int mask_flags,
                         float* resid_out, int64_t ldr, void* y, int y_dtype, int64_t ldy, int64_t rows, int64_t d,
                         float eps, void* stream);

/*
 * Projection GEMM with fused epilogue:
 *     v = a . w^T + bias;  then the epi flags GELU, MASK_BRANCH;  v += resid;
 *     then MASK_RESID;  c = v
 * a: [M, K] and w: [N, K] (nn.Linear weight layout) in ab_dtype, COBRA_F16 or
 * COBRA_BF16 (v_mfma_f32_32x32x16_bf16); bias: [N] fp32 (optional), resid: [M, N]
 * (optional), row_mask: [M] bytes (required by the mask flags), c: [M, N] in
 * c_dtype.  resid and c are COBRA_F16 / COBRA_F32 with fp16 operands, COBRA_BF16 /
 * COBRA_F32 with bf16 operands.  fp32 accumulate and epilogue.
 * K % 8 == 0; COBRA_EPI_MASK_OUT is rejected (no LayerNorm here).  Replaces
 * _tl_linear / _gemm_kernel (TTB:355-381, 283-353).
 */
int cobra_linear_fwd(const void* a, const void* w, int ab_dtype, const float* bias, const void* resid, int resid_dtype,
                     const uint8_t* row_mask, int epi, void* c, int c_dtype, int64_t M, int64_t N, int64_t K,
                     void* stream);

/*
 * Projection GEMM + residual + LayerNorm over whole rows:
 *     r = a . w^T + bias (GELU, MASK_BRANCH) + resid (MASK_RESID);
 *     resid_out = r (optional, fp32);  y = LayerNorm(r) * gamma + beta (MASK_OUT)
 * Shapes as cobra_linear_fwd with fp16 operands; requires N <= 128 (one workgroup owns
 * a row) and N % 8 == 0.  Replaces _tl_linear_ln / _gemm_ln_kernel (TTB:465-488, 394-463).
 */
int cobra_linear_ln_fwd(const void* a, const void* w, const float* bias, const void* resid, int resid_dtype,
                        const uint8_t* row_mask, int epi, float* resid_out, const float* gamma, const float* beta,
                        void* y, int y_dtype, int64_t M, int64_t N, int64_t K, float eps, void* stream);

/*
 * LayerNorm fused into the prologue of the projection that consumes it:
 *     h = (x - mean) * rsqrt(var + eps) * gamma + beta   per row (biased var);
 *     c = h . w^T + bias                                  (h never stored)
 * x: [M, d] in x_dtype with d = 64 or 128 (one k-tile per row); gamma, beta:
 * [d] fp32; w: [N, d] fp16 with N <= 3 d (a QKV projection); bias: [N] fp32
 * (optional); c: [M, N] fp16.  N % 8 == 0.  Replaces the pair _tl_add_ln -> F.linear of the reference's
 * layer-0 / pre-attention path (TTB:1216-1234) with one kernel.
 */
int cobra_ln_linear_fwd(const void* x, int x_dtype, const float* gamma, const float* beta, const void* w,
                        const float* bias, void* c, int64_t M, int64_t N, int64_t d, float eps, void* stream);

/*
 * Token mask -> packed key bits for cobra_attn_fwd:
 *     mask: [batch, seq_len] bytes (0 = padded token);
 *     key_bits: [batch][ceil(seq_len / 64)] uint64, 8-byte aligned; bit j of
 *     word w is set iff token 64 w + j exists and is valid.
 * The reference builds an additive -inf bias from the mask for SDPA instead
 * (TTB:1207-1213); the bits are 1/32 of that tensor's size.
 */
int cobra_mask_bits(const uint8_t* mask, uint64_t* key_bits, int64_t batch, int64_t seq_len, void* stream);

/*
 * Multi-head attention on a packed projection buffer:
 *     qkv: [batch*seq_len, 3*D] in dtype (COBRA_F16 or COBRA_BF16) with column
 *          blocks q | k | v, each split into `heads` contiguous slices of head_dim
 *          (D = heads*head_dim);
 *     ctx: [batch*seq_len, D] in dtype, ctx_i = softmax((q_i k^T) * scale) v per head
 *          (fp32 scores and softmax; the probabilities rounded to dtype for the P.V
 *          product, as the reference's fp16 kernel does).
 * causal != 0 masks keys j > i; key_bits (optional, from cobra_mask_bits)
 * masks padded keys (TTB:106-109).  A query left with no valid key gets a
 * zero row (the reference's softmax would give NaN there; the sublayer zeroes
 * such rows anyway).  head_dim % 8 == 0, head_dim <= 256.
 * Replaces _tl_attn / _attn_kernel (TTB:828-854, 572-649; causal only there)
 * and the SDPA call used for non-causal and masked attention (TTB:1240-1253).
 */
int cobra_attn_fwd(const void* qkv, void* ctx, int dtype, const uint64_t* key_bits, int64_t batch, int64_t seq_len,
                   int64_t heads, int64_t head_dim, float scale, int causal, void* stream);

/*
 * Fused QKV projection + multi-head attention on a normalised activation:
 *     q | k | v = h . w_qkv^T + b_qkv   (rounded to fp16)
 *     ctx = MHA(q, k, v)                (as cobra_attn_fwd: scale, causal, key_bits)
 * h: [batch*seq_len, D] fp16 (D = heads*head_dim); w_qkv: [3*D, D] fp16 (rows:
 * q_proj, k_proj, v_proj weights); b_qkv: [3*D] fp32 (optional); ctx: [batch*seq_len, D]
 * fp16.  head_dim % 8 == 0, head_dim <= 256.  For head_dim 256 with seq_len <= 128 it is
 * one launch -- the projection inside the attention kernel, one workgroup per (sequence,
 * head), q / k / v never in memory -- cobra_qkv_attn_workspace_bytes() returns 0 (the
 * workspace may be null) and ctx must not overlap h.  Otherwise two launches (the
 * projection GEMM into the workspace, cobra_qkv_attn_workspace_bytes() bytes, then the
 * attention).  Replaces _tl_qkvattn / _qkvattn_kernel (TTB:761-785, 654-741), which is
 * causal only, takes the transposed weight [D, 3D] and is used when one query block
 * covers the sequence (TTB:1030-1071).
 */
int64_t cobra_qkv_attn_workspace_bytes(int64_t batch, int64_t seq_len, int64_t heads, int64_t head_dim);
int cobra_qkv_attn_fwd(const void* h, const void* w_qkv, const float* b_qkv, void* ctx, const uint64_t* key_bits,
                       void* workspace, int64_t workspace_bytes, int64_t batch, int64_t seq_len, int64_t heads,
                       int64_t head_dim, float scale, int causal, void* stream);

/* Execution plans of cobra_layer_fwd. */
enum {
  COBRA_PLAN_FUSED = 0,  /* one kernel for the whole sublayer, no workspace */
  COBRA_PLAN_STAGED = 1, /* LN1, QKV GEMM, attention, out-proj GEMM (+LN) through a workspace */
  COBRA_PLAN_PADDED = 2  /* the staged plan on zero-padded copies: head_dim or d_model not a multiple of 8 */
};

/*
 * Which plan cobra_layer_fwd runs for this shape and activation dtype, or -1
 * if the shape (or x_dtype) is not supported (d_model % heads != 0, head_dim >
 * 256, d_model > 4096).  PADDED covers every head_dim or d_model that is not a
 * multiple of 8 (the reference zero-pads head_dim to HD_PAD inside its attention
 * kernel, TTB:578, 763-765, and masks its GEMM loads).  FUSED covers seq_len <= 128 with
 * d_model 128 (head_dim 32 or 64), 64 (32, 64) or 96 (32), with or without a
 * token mask; and, for fp16 activations while batch * ceil(seq_len / 32) <= 2 x
 * the device's compute units, d_model 128 at head_dim 8 or 128.  bf16 activations
 * (x_dtype COBRA_BF16) take STAGED (or PADDED): LN1, the QKV GEMM, the attention and
 * the out-projection with bf16 operands.  `masked` (a token
 * mask will be passed) only changes the STAGED plan's workspace.  Host-only: no
 * device work.  The reference's counterpart is the gate set of
 * UserOptimizedTransformer._prepare (TTB:1030-1071), which also looks at the
 * dtype (TTB:952-996).
 */
int cobra_layer_plan(int64_t batch, int64_t seq_len, int64_t d_model, int64_t heads, int masked, int x_dtype);

/* Device workspace (bytes) cobra_layer_fwd needs for this shape (0 for FUSED). */
int64_t cobra_layer_workspace_bytes(int64_t batch, int64_t seq_len, int64_t d_model, int64_t heads, int masked,
                                    int x_dtype);

/*
 * The whole attention sublayer (TTB:141-142 with TTB:88-123):
 *     h = LN1(x);  [q|k|v] = h . w_qkv^T + b_qkv;  c = MHA(q, k, v)
 *     r = x + (c . w_o^T + b_o);   y = LN2(r)
 * valid_mask (optional): [batch, seq_len] bytes, 0 = padded token.  Padded
 * keys are masked in the attention (TTB:106-109) and padded rows get a zero
 * attention output, r = x (TTB:121-122); the workspace must then be sized
 * with masked = 1.
 * x, y: [batch*seq_len, d_model] in x_dtype (COBRA_F16, COBRA_F32 or COBRA_BF16);
 * w_qkv: [3*d_model, d_model] (rows: q_proj, k_proj, v_proj weights, in that order)
 * and w_o: [d_model, d_model] in fp16, or in bf16 when x_dtype is COBRA_BF16;
 * b_qkv: [3*d_model], b_o and the LayerNorm parameters fp32.  With bf16
 * activations h, q, k, v, the probabilities and the context are bf16 MFMA operands
 * and r = x + branch is formed in fp32.
 * ln1_w and ln1_b may both be NULL: LN1 without elementwise affine, for a
 * caller that has folded it into the projection (w_qkv . diag(ln1_w) and
 * b_qkv + w_qkv . ln1_b), which spares the kernels those reads; exactly one
 * of them NULL is rejected.  resid_out (optional): r in fp32.  workspace: cobra_layer_workspace_bytes()
 * bytes (may be NULL when that is 0).  One launch for the FUSED plan.
 * Replaces the attention half of UserOptimizedTransformer._run_fused
 * (TTB:1216-1268), which is what its CUDA graph replays (TTB:1331-1360).
 */
int cobra_layer_fwd(const void* x, int x_dtype, const uint8_t* valid_mask, const void* w_qkv, const float* b_qkv,
                    const void* w_o, const float* b_o, const float* ln1_w, const float* ln1_b, const float* ln2_w,
                    const float* ln2_b, void* y, float* resid_out, void* workspace, int64_t workspace_bytes,
                    int64_t batch, int64_t seq_len, int64_t d_model, int64_t heads, int causal, float eps,
                    void* stream);

/*
 * A prepared cobra_layer_fwd: everything but the activations and the stream is
 * validated and bound once, so a steady-state forward crosses the ABI with six
 * arguments.  cobra_layer_bind returns NULL for arguments cobra_layer_fwd would
 * reject (workspace sized for `masked`); the handle is host memory only, owns
 * none of the buffers it names, and is released with cobra_layer_unbind.
 * cobra_layer_run(h, x, valid_mask, y, resid_out, stream) equals
 * cobra_layer_fwd with the bound arguments; valid_mask must be NULL unless the
 * handle was bound with masked = 1.  The counterpart of the reference's
 * per-signature _prepare followed by a graph replay per forward
 * (TTB:948-1081, 1331-1360).
 */
typedef struct cobra_layer_launch cobra_layer_launch;
cobra_layer_launch* cobra_layer_bind(int x_dtype, int masked, const void* w_qkv, const float* b_qkv, const void* w_o,
                                     const float* b_o, const float* ln1_w, const float* ln1_b, const float* ln2_w,
                                     const float* ln2_b, void* workspace, int64_t workspace_bytes, int64_t batch,
                                     int64_t seq_len, int64_t d_model, int64_t heads, int causal, float eps);
int cobra_layer_run(const cobra_layer_launch* h, const void* x, const uint8_t* valid_mask, void* y, float* resid_out,
                    void* stream);
void cobra_layer_unbind(cobra_layer_launch* h);

/*
 * Size of the device scratch that cobra_layer_fwd_noalloc uses in place of a
 * workspace: 128 MiB, one copy per GPU the library runs on, held until the
 * process ends.
 */
#define COBRA_NOALLOC_MAX_BYTES (128ll << 20)

/*
 * cobra_layer_fwd without a workspace argument, for callers that cannot
 * allocate device memory (code under hipGraph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  It has no counterpart in the reference.
 * Same arguments, plans and results as cobra_layer_fwd (bit for bit); the
 * STAGED plan's intermediates go to a file-scope device array of
 * COBRA_NOALLOC_MAX_BYTES instead of a caller-provided workspace.  Nothing is
 * allocated or freed, here or in any callee.
 *   - Shapes whose cobra_layer_workspace_bytes() exceeds COBRA_NOALLOC_MAX_BYTES
 *     are rejected with hipErrorInvalidValue before anything is enqueued (at
 *     d_model 128, S 1024 up to 128 sequences fit, 127 with a token mask; at
 *     d_model 1024, S 128 up to 85).  The FUSED plan needs no scratch at all.
 *   - `stream` must belong to the current device (the array is per device).
 *   - Every call on one GPU shares that GPU's array, and nothing in it
 *     outlives a call: calls that overlap on one GPU (two streams, two host
 *     threads) race.  Calls on one stream are ordered and safe.
 */
int cobra_layer_fwd_noalloc(const void* x, int x_dtype, const uint8_t* valid_mask, const void* w_qkv,
                            const float* b_qkv, const void* w_o, const float* b_o, const float* ln1_w,
                            const float* ln1_b, const float* ln2_w, const float* ln2_b, void* y, float* resid_out,
                            int64_t batch, int64_t seq_len, int64_t d_model, int64_t heads, int causal, float eps,
                            void* stream);

/*
 * One whole transformer block of the reference's fused stack in one launch
 * (replaces the loop body of _run_fused, torch_transformer_benchmark.py:1216-1267,
 * fuse_ln branch: _tl_attn / _tl_qkvattn, _tl_linear_ln, _tl_linear(gelu),
 * _tl_linear_ln):
 *   r1  = r + mask_branch(attention(h) W_o^T + b_o)      (fp32)
 *   h2  = LN2(r1)                                        (fp16)
 *   f   = gelu(h2 W1^T + b1)                             (fp16, exact erf GELU)
 *   r2  = (r1 + f W2^T + b2) * row_valid                 (fp32 -> r_out)
 *   out = LNn(r2) [* row_valid if mask_out]              (out_dtype)
 * h = norm1(r) in fp16 (the previous block's epilogue, or a LayerNorm of the
 * model input for block 0); r fp32.  LNn is the next block's norm1, or
 * final_norm for the last block (then mask_out = 1 with a token mask, and
 * out_dtype the model's).  Weights: w_qkv [3D, D] (q | k | v rows), w_o [D, D],
 * w1 [F, D], w2 [D, F] fp16; biases and LayerNorm parameters fp32.
 * r_out may equal r (in place); out must not overlap h, r or r_out, and r_out
 * must not overlap h.  Shapes: cobra_block_plan() >= 0 (d_model 128,
 * ffn_dim 128, seq_len <= 128, head_dim 8 / 32 / 64 / 128).  No workspace.
 */
int cobra_block_fwd(const void* h, const float* r, const uint8_t* valid_mask, const void* w_qkv, const float* b_qkv,
                    const void* w_o, const float* b_o, const float* ln2_w, const float* ln2_b, const void* w1,
                    const float* b1, const void* w2, const float* b2, const float* lnn_w, const float* lnn_b,
                    float* r_out, void* out, int out_dtype, int mask_out, int64_t batch, int64_t seq_len,
                    int64_t d_model, int64_t heads, int64_t ffn_dim, int causal, float eps, void* stream);

/*
 * Whether cobra_block_fwd takes a shape: -1 no; 0 yes, but composing the
 * per-op entry points is expected to be faster (more than two rounds of
 * workgroups: every workgroup recomputes its sequence's K and V); 1 yes and
 * preferred.  (The reference gates its fused paths by shape the same way,
 * torch_transformer_benchmark.py:1030-1071.)
 */
int cobra_block_plan(int64_t batch, int64_t seq_len, int64_t d_model, int64_t heads, int64_t ffn_dim);

#ifdef __cplusplus
}
#endif

#endif /* COBRA_AMD_H */
