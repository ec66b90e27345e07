/*
 * bdh_hip.h - C ABI of the MI355X (gfx950) BDH strict-tril attention library.
 *
 * The op: out[b,h,i,:] = sum_{j<i} <Q[b,h,i,:], K[b,h,j,:]> * V[b,hv,j,:]
 * (tril(Q K^T, -1) V: no softmax, no 1/sqrt(d), diagonal excluded), with BDH's
 * RoPE (adjacent-pair rotation, phase = frac(pos * freq)) optionally fused into
 * the operand loads.
 *
 * Conventions
 *  - Every tensor is a 4-D strided view (bdh_tensor4): element strides, the
 *    last dimension must have stride 1 (when its size is > 1).  Other strides
 *    are honoured, so permuted views and capacity-strided cache views are
 *    passed without copies.  V may broadcast over heads (size[1] == 1).
 *  - dtype is BDH_F32 or BDH_BF16.  Arithmetic follows the q/k dtype: bf16
 *    operands use bf16 MFMA with fp32 accumulation, fp32 operands use fp32
 *    MFMA.  Outputs are cast to their own dtype on store.
 *  - The library never allocates device memory.  Entry points that need
 *    scratch take a caller-provided workspace whose size comes from the
 *    matching *_workspace() query.
 *  - Work is enqueued on `stream` (a hipStream_t); calls are asynchronous.
 *  - Return value: BDH_OK (0) or an error code; bdh_error_string() names it.
 *    Shape/dtype/stride errors are detected before anything is launched.
 */
#ifndef BDH_HIP_H_
#define BDH_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { BDH_F32 = 0, BDH_BF16 = 1 };

enum {
  BDH_OK = 0,
  BDH_ERR_SHAPE = 1,     /* inconsistent sizes between operands            */
  BDH_ERR_DTYPE = 2,     /* unsupported dtype or dtype combination         */
  BDH_ERR_STRIDE = 3,    /* last dimension not unit-stride                 */
  BDH_ERR_WORKSPACE = 4, /* workspace missing or smaller than required     */
  BDH_ERR_LAUNCH = 5,    /* the HIP runtime rejected a kernel launch       */
  BDH_ERR_ARG = 6,       /* other invalid argument (NULL pointer, range)   */
  BDH_ERR_ALIAS = 7,     /* an output overlaps an input it must not alias  */
  BDH_ERR_SCRATCH = 8    /* larger than the no-allocation scratch holds    */
};

typedef struct bdh_tensor4 {
  void* data;
  int64_t size[4];
  int64_t stride[4]; /* in elements */
  int32_t dtype;     /* BDH_F32 | BDH_BF16 */
  int32_t reserved;
} bdh_tensor4;

typedef void* bdh_stream; /* hipStream_t */

/* Library version string and error names. */
const char* bdh_version(void);
const char* bdh_error_string(int code);

/*
 * Cold strict-tril score x V.
 * Replaces tril_score_v (reference csrc/tril_attn_bind.cpp:3-12, dispatching to
 * tril_score_v_cuda, csrc/tril_attn_cuda.cu:251-339; Python wrapper
 * kernels/cuda_attn.py:391-414).
 * q, k: (B,H,T,Dk) same dtype; v: (B,1|H,T,Dv); out: (B,H,T,Dv).
 */
size_t bdh_tril_score_v_workspace(int64_t B, int64_t H, int64_t T, int64_t Dk,
                                  int64_t Dv, int32_t qk_dtype);
int bdh_tril_score_v(const bdh_tensor4* q, const bdh_tensor4* k,
                     const bdh_tensor4* v, const bdh_tensor4* out,
                     void* workspace, size_t workspace_bytes, bdh_stream stream);

/*
 * Cold BDH attention with RoPE fused into the operand loads: Q = K = RoPE(x).
 * Replaces the pair bdh.py:405 (self.rope(...) -> kernels/rope.py:220-240)
 * followed by bdh.py:412 (bdh_attn(QR, QR, V), kernels/attention_dispatch.py:
 * 263-308).  freqs: N fp32 values (bdh.py:41-49 layout, pairs share a value);
 * positions are rope_start + t.  qr_out (optional, may be NULL): also store
 * RoPE(x) there, in its own dtype (the KR cache slot, bdh.py:1000-1016).
 */
int bdh_tril_rope_score_v(const bdh_tensor4* x, const bdh_tensor4* v,
                          const bdh_tensor4* out, const float* freqs,
                          int64_t rope_start, const bdh_tensor4* qr_out,
                          void* workspace, size_t workspace_bytes,
                          bdh_stream stream);

/*
 * Queries at an offset (chunked prefill): T new rows after `past` cached rows.
 * out[b,h,i,:] = sum_{j < past+i} <q[b,h,i,:], k[b,h,j,:]> v[b,hv,j,:].
 * Replaces the reference's multi-token step with a cache, which recomputes
 * the whole strict-tril attention over past||new and keeps the last T rows
 * (bdh.py:446-461: bdh_attn(QR_all, QR_all, V_all)[..., S:, :]); here only
 * the score tiles that reach a new row are computed.
 * q: (B,H,T,Dk); k: (B,H,past+T,Dk) (rows past.. are the new keys); v:
 * (B,1|H,past+T,Dv); out: (B,H,T,Dv).  q and k share a dtype.  past == 0 is
 * bdh_tril_score_v.
 */
size_t bdh_tril_score_v_past_workspace(int64_t B, int64_t H, int64_t T,
                                       int64_t past, int64_t Dk, int64_t Dv,
                                       int32_t qk_dtype);
int bdh_tril_score_v_past(const bdh_tensor4* q, const bdh_tensor4* k,
                          const bdh_tensor4* v, const bdh_tensor4* out,
                          int64_t past, void* workspace, size_t workspace_bytes,
                          bdh_stream stream);

/*
 * Decode against the packed past: out = (q K_past^T) V_past (all past keys
 * valid; the new token never attends to itself).
 * Replaces tril_decode (reference csrc/tril_attn_bind.cpp:14-23 ->
 * csrc/tril_attn_cuda.cu:544-661; kernels/cuda_attn.py:490-502) and the eager
 * decode of kernels/attention.py:193-219.
 * q: (B,H,Tq,Dk); k_past: (B,H,S,Dk) (capacity-strided views allowed);
 * v_past: (B,1|H,S,Dv); out: (B,H,Tq,Dv).  q and the cache may have different
 * dtypes (e.g. fp32 compute over a bf16 cache).
 */
size_t bdh_tril_decode_workspace(int64_t B, int64_t H, int64_t Tq, int64_t S,
                                 int64_t Dk, int64_t Dv);
int bdh_tril_decode(const bdh_tensor4* q, const bdh_tensor4* k_past,
                    const bdh_tensor4* v_past, const bdh_tensor4* out,
                    void* workspace, size_t workspace_bytes, bdh_stream stream);

/*
 * Decode that allocates nothing and takes no workspace.  It has no
 * counterpart in the reference: it is for callers that cannot call hipMalloc
 * or hand in a workspace (code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation).  Same operands, kernels and results as
 * bdh_tril_decode.  The partial sums go to a library-owned device array of
 * BDH_NOALLOC_SCRATCH_BYTES per GPU (each GPU the library runs on holds one
 * until the process ends); inputs whose partials exceed it return
 * BDH_ERR_SCRATCH.  The partials take B*H*Tq * Dv * 4 bytes per chunk of past
 * keys: 64-key chunks on both streaming kernels (q and key rows 16-byte
 * aligned, and Dk a multiple of 2048 for bf16 q over bf16 keys, or of 256 /
 * 512 for fp32 / bf16 keys under the fp32-arithmetic kernel), 32-key chunks on
 * the generic kernel (any other operands).  C3's B*H = 256, Dv = 256 fits
 * S <= 4096 on the streaming kernels.  The current device must be
 * the tensors' device.  Every call on one GPU shares that GPU's array: calls
 * that overlap in time on one GPU (other streams, other threads) race and must
 * be serialised by the caller.
 */
#define BDH_NOALLOC_SCRATCH_BYTES (16u << 20)
int bdh_tril_decode_noalloc(const bdh_tensor4* q, const bdh_tensor4* k_past,
                            const bdh_tensor4* v_past, const bdh_tensor4* out,
                            bdh_stream stream);

/*
 * RoPE apply: out = rotate(v, cos, sin) over adjacent pairs.
 * Replaces eager_rope_rotate / rope_rotate_t1 / rope_rotate_paired
 * (reference kernels/rope.py:174-240) behind bdh_rope_rotate and
 * bdh_rope_rotate_paired (kernels/rope_dispatch.py:64-99).
 * cos, sin: views broadcastable to v (stride 0 on broadcast dims), last dim N.
 * Same rounding as the reference: fp32 v -> fp32 products and add; bf16 v ->
 * each product rounded to bf16, then a bf16 add.  out may have another dtype.
 * backward != 0 applies the transpose rotation (kernels/rope.py:543-556).
 */
int bdh_rope_rotate(const bdh_tensor4* v, const bdh_tensor4* cos,
                    const bdh_tensor4* sin, const bdh_tensor4* out,
                    int32_t backward, bdh_stream stream);

/*
 * Analytic backward of out = tril(q k^T, -1) v.
 * Replaces analytic_tril_attn_backward[_blocked] (reference
 * kernels/attention_bwd.py:45-181) as used by StrictTrilAttnFn and
 * StrictTrilSelfAttnFn (:218-291).
 * k == NULL means self attention (k is q): dq receives dq + dk (the merged
 * gradient of attention_bwd.py:284-291) and dk must be NULL.
 * dv has v's shape; with broadcast v the head gradients are summed.
 */
size_t bdh_tril_score_v_bwd_workspace(int64_t B, int64_t H, int64_t Hv,
                                      int64_t T, int64_t Dk, int64_t Dv,
                                      int32_t qk_dtype);
int bdh_tril_score_v_bwd(const bdh_tensor4* q, const bdh_tensor4* k,
                         const bdh_tensor4* v, const bdh_tensor4* dout,
                         const bdh_tensor4* dq, const bdh_tensor4* dk,
                         const bdh_tensor4* dv, void* workspace,
                         size_t workspace_bytes, bdh_stream stream);

/*
 * Self-attention backward from saved scores: the save-S side of the
 * reference's save-or-recompute choice.  Its default autograd path
 * (tril_(-1) then matmul, kernels/attention.py:27-40) keeps S for the
 * backward; analytic_tril_attn_backward (kernels/attention_bwd.py:45-83)
 * recomputes it.
 * bdh_tril_score_v_keeps_scores returns 1 when bdh_tril_score_v(x, x, v, ...)
 * on these views runs the bf16 MFMA path, whose workspace then starts with the
 * score tiles of tril(x x^T, -1) (*scores_bytes bytes); else 0.
 * bdh_tril_score_v_bwd_saved computes the gradients of bdh_tril_score_v_bwd
 * with k == NULL (dx = merged dq + dk, dv) from that workspace, passed as
 * `scores`, instead of recomputing the tiles.  x must be the forward's x,
 * unchanged since; other views give BDH_ERR_ARG.
 */
int bdh_tril_score_v_keeps_scores(const bdh_tensor4* x, const bdh_tensor4* v,
                                  size_t* scores_bytes);
size_t bdh_tril_score_v_bwd_saved_workspace(int64_t B, int64_t H, int64_t Hv,
                                            int64_t T, int64_t N, int64_t Dv,
                                            int32_t x_dtype);
int bdh_tril_score_v_bwd_saved(const bdh_tensor4* x, const bdh_tensor4* v,
                               const bdh_tensor4* dout, const bdh_tensor4* dx,
                               const bdh_tensor4* dv, const void* scores,
                               size_t scores_bytes, void* workspace,
                               size_t workspace_bytes, bdh_stream stream);

/*
 * Backward of bdh_tril_rope_score_v: dx = RoPE^-1((dS + dS^T) RoPE(x)) and
 * dv = sum_h M_h^T dout_h, M = tril(RoPE(x) RoPE(x)^T, -1).
 * Replaces the autograd chain of bdh.py:405-412 under BDH_ATTN_AUTOGRAD
 * (StrictTrilSelfAttnFn, kernels/attention_bwd.py:259-291, then the RoPE
 * backward of kernels/rope.py:543-556).
 */
size_t bdh_tril_rope_score_v_bwd_workspace(int64_t B, int64_t H, int64_t Hv,
                                           int64_t T, int64_t N, int64_t Dv,
                                           int32_t x_dtype);
int bdh_tril_rope_score_v_bwd(const bdh_tensor4* x, const bdh_tensor4* v,
                              const bdh_tensor4* dout, const float* freqs,
                              int64_t rope_start, const bdh_tensor4* dx,
                              const bdh_tensor4* dv, void* workspace,
                              size_t workspace_bytes, bdh_stream stream);

/*
 * The same gradients from the score tiles the forward kept (the save-S side
 * of the reference's choice, as bdh_tril_score_v_bwd_saved; the reference's
 * default autograd keeps S, attention_bwd.py:259-291).
 * bdh_tril_rope_score_v_keeps_scores returns 1 when bdh_tril_rope_score_v(x, v,
 * out, freqs, rope_start, NULL, ...) on these views runs the bf16 MFMA path
 * and leaves its score tiles in its workspace, of which the backward needs
 * the first *scores_bytes; else 0.  bdh_tril_rope_score_v_bwd_saved takes
 * that workspace as `scores` (x, v, freqs and rope_start those of the
 * forward, x unchanged since) and recomputes no score tile: dv from the kept
 * tiles, dx as above with x rotated (absolute positions) as the dQ product
 * stages it, so R(x) is never written.  Other views
 * give BDH_ERR_ARG.  bf16 x, dout and v; D a multiple of 64 up to 256.
 */
int bdh_tril_rope_score_v_keeps_scores(const bdh_tensor4* x, const bdh_tensor4* v,
                                       size_t* scores_bytes);
size_t bdh_tril_rope_score_v_bwd_saved_workspace(int64_t B, int64_t H, int64_t Hv,
                                                 int64_t T, int64_t N, int64_t Dv,
                                                 int32_t x_dtype);
int bdh_tril_rope_score_v_bwd_saved(const bdh_tensor4* x, const bdh_tensor4* v,
                                    const bdh_tensor4* dout, const float* freqs,
                                    int64_t rope_start, const bdh_tensor4* dx,
                                    const bdh_tensor4* dv, const void* scores,
                                    size_t scores_bytes, void* workspace,
                                    size_t workspace_bytes, bdh_stream stream);

/*
 * Consumer of the attention in the BDH layer: out = x * max(y, 0), elementwise.
 * Replaces the ReLU of encoder_v's output (bdh.py:914-925, `_bias_relu_`) and
 * the sparse product of _mlp_merge (bdh.py:927-945, `x_bthn * y_bthn`) in one
 * pass.  x, y, out: 4-D views of equal sizes, each in its own dtype, so y can
 * be the head-major (nh, B, T, N) output of a batched GEMM viewed as
 * (B, T, nh, N).  The product is formed in fp32 and rounded once to out's
 * dtype; NaN in y propagates as in torch's relu.
 */
int bdh_relu_mul(const bdh_tensor4* x, const bdh_tensor4* y, const bdh_tensor4* out,
                 bdh_stream stream);

/*
 * encoder_v GEMM with the gated product fused into its epilogue, bf16:
 *   out[b,t,h,n] = x[b,t,h,n] * max(sum_k y[b,h,t,k] * wt[0,h,n,k], 0)
 * Replaces `_encoder_v_relu` (bdh.py:914-925, einsum("bhtd,hdn->bthn") +
 * ReLU) followed by the `x_bthn * y_bthn` of _mlp_merge (bdh.py:927-945); the
 * GEMM's output never reaches HBM.  y: (B, nh, T, K), the LayerNorm of the
 * attention output; wt: (1, nh, N, K), encoder_v transposed; x, out:
 * (B, T, nh, N).  K a multiple of 32, N of 8, rows 16-byte aligned; one
 * head's view of y and of wt spans at most 4 GiB (else BDH_ERR_SHAPE).  The
 * GEMM result is rounded to bf16 after the ReLU, then multiplied by x.  K =
 * 256 with N a multiple of 64, and K = 512 with N a multiple of 32, run on the
 * streaming kernel (one workgroup per head and 256 tokens); other shapes on a
 * tile kernel.  Both give the same bits.
 */
int bdh_gated_gemm(const bdh_tensor4* y, const bdh_tensor4* wt, const bdh_tensor4* x,
                   const bdh_tensor4* out, bdh_stream stream);

/*
 * The same GEMM without the gate, the encoder with its ReLU:
 *   out[b,t,h,n] = max(sum_k y[b,h,t,k] * wt[0,h,n,k], 0)          (bf16)
 * Replaces `_encoder_relu` (bdh.py:861-912: x @ encoder per head, ReLU) for the
 * prefill: y (B, nh, T, K), the layer input, with a head stride of 0 when all
 * heads share it; wt (1, nh, N, K), the encoder transposed; out (B, T, nh, N).
 * Same sizes, strides, limits and kernels as bdh_gated_gemm.
 */
int bdh_relu_gemm(const bdh_tensor4* y, const bdh_tensor4* wt, const bdh_tensor4* out, bdh_stream stream);

/*
 * The gated product chained into the decoder product, bf16 operands, fp32
 * accumulation:
 *   out[b,t,0,:] = sum_h sum_n x[b,t,h,n] * max(sum_k y[b,h,t,k] * wt[0,h,n,k], 0)
 *                  * dec[0,0,h*N+n,:]
 * Replaces `_encoder_v_relu` (bdh.py:914-925) and the whole of _mlp_merge
 * (bdh.py:927-945: `x_bthn * y_bthn`, then F.linear with the decoder) for the
 * prefill; the product x * relu(...) never reaches memory.  y: (B, nh, T, K),
 * the LayerNorm of the attention output; wt: (1, nh, N, K), encoder_v
 * transposed; x: (B, T, nh, N); dec: (1, 1, nh*N, D), the decoder; out:
 * (B, T, 1, D), bf16 or fp32, rows evenly spaced.  K = D = 256, N a multiple
 * of 32, rows 16-byte aligned; one head's rows of wt and of dec span at most
 * 4 GiB (else BDH_ERR_SHAPE).  Each product x * relu(...) is rounded to bf16
 * once.  The workspace holds the heads' fp32 partial outputs (nh * B*T * D
 * floats), summed in head order.
 */
size_t bdh_gated_decoder_workspace(int64_t nh, int64_t M);
int bdh_gated_decoder(const bdh_tensor4* y, const bdh_tensor4* wt, const bdh_tensor4* x,
                      const bdh_tensor4* dec, const bdh_tensor4* out, void* workspace,
                      size_t workspace_bytes, bdh_stream stream);

/*
 * Few-row GEMM with split K, bf16 operands, fp32 accumulation:
 *   out (1, 1, M, D) = a (1, 1, M, K) @ b (1, 1, K, D)
 * For the decoder product of a decode step (bdh.py:927-945, `_mlp_merge`'s
 * F.linear with M = batch rows, K = nh*N, D = n_embd), where a library GEMM
 * walks the whole K with a few tiles.  out is bf16 or fp32.  The workspace
 * holds the fp32 partial sums of the K splits: it must be 4-byte aligned
 * (else BDH_ERR_WORKSPACE); a 16-byte aligned one takes the vectorized split
 * reduction.
 */
size_t bdh_small_gemm_workspace(int64_t M, int64_t K, int64_t D);
int bdh_small_gemm(const bdh_tensor4* a, const bdh_tensor4* b, const bdh_tensor4* out,
                   void* workspace, size_t workspace_bytes, bdh_stream stream);

/*
 * LayerNorm over the last dim (no affine, eps 1e-5, fp32 arithmetic) of the
 * rows of 4-D views: out = LN(y), or with x (not NULL) out = LN(x + LN(y)).
 * Replaces the model's _ln (reference bdh.py:565-574, F.layer_norm without
 * weights) and _residual_ln (bdh.py:731-750, LN(x + LN(y_mlp))) in one pass.
 * x, y, out: one shape, each f32 or bf16 (out rounded once); D = size[3] a
 * multiple of 64, at most 1024, with D/64 a power of two.
 */
int bdh_layer_norm_rows(const bdh_tensor4* x, const bdh_tensor4* y,
                        const bdh_tensor4* out, bdh_stream stream);

/*
 * bdh_layer_norm_rows that also writes the result rounded once to bf16 into
 * out_bf16 (one shape with y, bf16, any strides, overlapping no other
 * operand).  The model's bf16 forward feeds the next layer's encoder and
 * attention V (bdh.py:396-413, 861-912, under autocast both take the residual
 * stream in bf16) from it without a cast pass; a decode step writes it
 * straight into the KV cache's V slot.  The two outputs hold the same values:
 * out_bf16 equals out converted to bf16 (round to nearest even).
 */
int bdh_layer_norm_rows2(const bdh_tensor4* x, const bdh_tensor4* y,
                         const bdh_tensor4* out, const bdh_tensor4* out_bf16,
                         bdh_stream stream);

/*
 * Per-kernel timing (measurement support; no counterpart in the reference).
 * While enabled, every kernel the library launches is bracketed by HIP events
 * on its stream.  bdh_profile_collect() waits for the recorded events and
 * returns up to `max` (name, milliseconds) records, then clears the log.
 * The events leave each kernel's duration as it is, but the runtime then
 * starts a launch only after the previous one has ended (several
 * microseconds between kernels), so time whole steps with profiling off.
 */
void bdh_profile_enable(int32_t on);
int bdh_profile_collect(char* names, int32_t name_len, float* ms, int32_t max);

#ifdef __cplusplus
}
#endif

#endif /* BDH_HIP_H_ */
