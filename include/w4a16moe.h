/*
 * w4a16moe.h -- C ABI of the MI355X (gfx950) W4A16 mixture-of-experts library
 * (libw4a16moe.so, built from hybridagent_amd/csrc).
 *
 * Replaces the W4A16 MoE hot path of HybridAgent, hybrid_agent/quantization.py
 * and the router block of hybrid_agent/backends.py.  Every entry point:
 *   - takes raw device pointers, sizes and a hipStream_t passed as void*
 *     (NULL = the default stream);
 *   - validates its arguments on the host before touching the GPU and returns
 *     a W4A16_* status (0 = success);
 *   - never allocates: scratch memory is a caller-provided workspace whose
 *     size the matching *_workspace_bytes() function returns;
 *   - is asynchronous on the given stream, performs no host synchronisation
 *     and keeps no global mutable state (re-entrant across streams/threads).
 *
 * Data layout (compressed-tensors pack-quantized, quantization.py:1-5,132-137,
 * 153-159, 191-218):
 *   packed weights  int32 [.., N, K/8]; word j of row n holds w[n, 8j+i] for
 *                   i = 0..7 in bits 4i..4i+3 as q + 8 (q in [-8, 7]);
 *   scales          bf16  [.., N, ceil(K/G)]; group g covers columns
 *                   g*G .. min(K, (g+1)*G) - 1 (the last group may be partial);
 *   activations     bf16, row-major, rows of length K;
 *   bf16 values are passed as uint16_t bit patterns.
 * Constraints: K % 32 == 0 for every reduction length, G a power of two
 * >= 32, pointers 16-byte aligned, E <= 512, top_k <= 32.
 */
#ifndef W4A16MOE_H
#define W4A16MOE_H

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define W4A16_API __attribute__((visibility("default")))
#else
#define W4A16_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

enum w4a16_status {
  W4A16_OK = 0,
  W4A16_ERR_NULL = 1,      /* a required pointer is NULL */
  W4A16_ERR_SHAPE = 2,     /* a size is out of range or inconsistent */
  W4A16_ERR_GROUP = 3,     /* unsupported group size */
  W4A16_ERR_ALIGN = 4,     /* a pointer is not 16-byte aligned */
  W4A16_ERR_WORKSPACE = 5, /* workspace missing or too small */
  W4A16_ERR_LAUNCH = 6     /* a HIP launch failed */
};

/* (major << 16) | (minor << 8) | patch */
W4A16_API int w4a16moe_version(void);

/* Static description of a status code. */
W4A16_API const char* w4a16moe_status_string(int status);

/* dequantize_int4_packed(packed, scale, shifts)  -- quantization.py:132-137
 * out[r, k] = bf16_RNE(q[r, k] * scale[r, k / G]), bit-identical to the
 * reference's bf16 dequant.  rows = product of the leading dims.          */
W4A16_API int w4a16_dequantize(const int32_t* packed, const uint16_t* scale, uint16_t* out, int64_t rows,
                     int64_t K, int64_t group_size, void* stream);

/* Linear4Bit.forward  -- quantization.py:171-175
 * y[M, N] = x[M, K] @ dequant(W)^T (+ bias[N]), fp32 accumulation, bf16 out.
 * bias may be NULL.                                                        */
W4A16_API size_t w4a16_linear_workspace_bytes(int64_t M, int64_t K, int64_t group_size);
W4A16_API int w4a16_linear(const uint16_t* x, const int32_t* w_packed, const uint16_t* w_scale,
                 const uint16_t* bias, uint16_t* y, int64_t M, int64_t N, int64_t K,
                 int64_t group_size, void* workspace, size_t workspace_bytes, void* stream);

/* Residual add + RMSNorm of the MoE input in the latent harness (config 4):
 * RMSNorm -- transformers/models/gemma4/modeling_gemma4.py:197-215 (fp32
 * x * rsqrt(mean(x^2) + eps) * weight, back to bf16); the add is the
 * harness's h <- h + MoE(...).
 *   x      = bf16(h + delta)       written to h_out; delta NULL: x = h and
 *                                  h_out is not written (may be NULL)
 *   y      = bf16((x * rsqrt(mean(x^2) + eps)) * weight)
 * h, delta, h_out, y [M, H] bf16; weight [H] bf16.  H % 8 == 0, H <= 8192;
 * 16-byte aligned pointers.  No workspace.                                  */
W4A16_API int w4a16_add_rms_norm(const uint16_t* h, const uint16_t* delta, const uint16_t* weight,
                       uint16_t* h_out, uint16_t* y, int64_t M, int64_t H, float eps,
                       void* stream);

/* HybridLink latent map -- hybridlink.py:17-28 (HybridLink.forward; the
 * latent loop applies it to the last hidden state, engine.py:381-390):
 *   a   = LayerNorm(h; ln1_w, ln1_b)                     (pre_ln)
 *   g   = bf16(GELU_erf(bf16(a p1_w^T + p1_b)))          (proj1, act)
 *   r   = bf16(h + bf16(g p2_w^T + p2_b))                (proj2, residual)
 *   out = LayerNorm(r; ln2_w, ln2_b)                     (post_ln)
 * LayerNorm: fp32 mean and variance, (x - mean) * rsqrt(var + eps) * w + b,
 * bf16 out (nn.LayerNorm, eps = 1e-5 in the reference module).
 * h, out [B, H] bf16; ln*_w, ln*_b, p*_b [H] bf16; p1_w, p2_w [H, H] bf16
 * (nn.Linear layout, out x in).  H % 32 == 0, H <= 8192; 16-byte aligned
 * h, out, weights, LayerNorm parameters and workspace.                     */
W4A16_API size_t w4a16_hybridlink_workspace_bytes(int64_t B, int64_t H);
W4A16_API int w4a16_hybridlink(const uint16_t* h, const uint16_t* ln1_w, const uint16_t* ln1_b,
                     const uint16_t* p1_w, const uint16_t* p1_b, const uint16_t* p2_w,
                     const uint16_t* p2_b, const uint16_t* ln2_w, const uint16_t* ln2_b,
                     uint16_t* out, int64_t B, int64_t H, float eps, void* workspace,
                     size_t workspace_bytes, void* stream);

/* Router  -- backends.py:111-117 (HF Gemma4TextRouter.forward,
 * transformers/models/gemma4/modeling_gemma4.py:1335-1356):
 *   r       = bf16(bf16(rms_norm(hidden) * router_scale) * scalar_root)
 *   logits  = bf16(r @ proj_w^T)                     (fp32 accumulation)
 *   p       = softmax(logits) in fp32
 *   topk_idx, topk_w = top_k of p (value desc, then lower index), renormalised
 *   topk_w *= per_expert_scale[topk_idx]
 * hidden [M, H], router_scale [H], proj_w [E, H], per_expert_scale [E] bf16;
 * logits_out [M, E] bf16 may be NULL; topk_idx int64 [M, top_k];
 * topk_w float32 [M, top_k].                                               */
W4A16_API size_t moe_router_workspace_bytes(int64_t M, int64_t H, int64_t E);
W4A16_API int moe_router_topk(const uint16_t* hidden, const uint16_t* router_scale, float scalar_root,
                    const uint16_t* proj_w, const uint16_t* per_expert_scale, float eps,
                    int64_t M, int64_t H, int64_t E, int64_t top_k, uint16_t* logits_out,
                    int64_t* topk_idx, float* topk_w, void* workspace, size_t workspace_bytes,
                    void* stream);

/* Softmax / top-k / renormalise / per-expert scale from given bf16 logits
 * [M, E]  -- backends.py:114-117.                                          */
W4A16_API int moe_topk_from_logits(const uint16_t* logits, const uint16_t* per_expert_scale, int64_t M,
                         int64_t E, int64_t top_k, int64_t* topk_idx, float* topk_w,
                         void* stream);

/* Token -> expert grouping  -- quantization.py:266-276 (implicit order of
 * torch.where over one_hot(top_k_index).permute(2,1,0)[e]).
 * sorted_pos int32 [M*top_k]: rows t*top_k + j of the token-major
 * flattening, grouped by ascending expert, k-slot-major / token-minor inside
 * each expert; expert_offsets int32 [E+1]: segment bounds.  Indices outside
 * [0, E) are skipped (the reference's "expert_idx == num_experts" rows).   */
W4A16_API size_t moe_sort_workspace_bytes(int64_t M, int64_t top_k, int64_t E);
W4A16_API int moe_sort_permute(const int64_t* topk_idx, int64_t M, int64_t top_k, int64_t E,
                     int32_t* sorted_pos, int32_t* expert_offsets, void* workspace,
                     size_t workspace_bytes, void* stream);

/* Gemma4TextExperts4Bit.forward / fused_triton_4bit_moe_forward
 *   -- quantization.py:88-129, 225-240
 * out[M, H] = sum_j bf16(topk_w[t,j]) * down_e(gelu_tanh(gate_e(x)) * up_e(x))
 * with e = topk_idx[t, j], bf16 rounding at the reference's points.
 * hidden [M, H] bf16; topk_idx int64 [M, top_k]; topk_w float32 [M, top_k];
 * gu_packed int32 [E, 2I, H/8] (gate rows 0..I-1, up rows I..2I-1);
 * gu_scale bf16 [E, 2I, ceil(H/G)]; dn_packed int32 [E, H, I/8];
 * dn_scale bf16 [E, H, ceil(I/G)].  Slots whose index is outside [0, E)
 * contribute nothing.  moe_forward = moe_plan + moe_gate_up + moe_down +
 * moe_combine on one workspace.                                            */
W4A16_API size_t moe_workspace_bytes(int64_t M, int64_t top_k, int64_t E, int64_t H, int64_t I);
W4A16_API int moe_forward(const uint16_t* hidden, const int64_t* topk_idx, const float* topk_w,
                const int32_t* gu_packed, const uint16_t* gu_scale, const int32_t* dn_packed,
                const uint16_t* dn_scale, uint16_t* out, int64_t M, int64_t top_k, int64_t E,
                int64_t H, int64_t I, int64_t group_size, void* workspace,
                size_t workspace_bytes, void* stream);

/* moe_forward without a workspace and without allocating -- no counterpart
 * in the reference.  For callers that cannot allocate device memory at call
 * time (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Same arguments and results as moe_forward minus the
 * workspace: the scratch is a file-scope device array of
 * W4A16_STATIC_SCRATCH_BYTES per GPU, which each GPU the library runs on
 * holds until the process ends; its address is looked up once per device,
 * on the first call there.  Sizes whose moe_workspace_bytes() exceeds the
 * array are rejected with W4A16_ERR_SHAPE (16 MiB covers every decode size,
 * M <= 256, at the Gemma-4-26B-A4B shape).  The stream must belong to the
 * current device (W4A16_ERR_LAUNCH otherwise).  Every call on a GPU shares
 * that GPU's array: calls that overlap on one GPU (other streams, other
 * threads) race.  Nothing in the array needs to start at zero; it keeps the
 * last call's contents.                                                    */
#define W4A16_STATIC_SCRATCH_BYTES ((size_t)16 << 20)
W4A16_API int moe_forward_static(const uint16_t* hidden, const int64_t* topk_idx, const float* topk_w,
                       const int32_t* gu_packed, const uint16_t* gu_scale, const int32_t* dn_packed,
                       const uint16_t* dn_scale, uint16_t* out, int64_t M, int64_t top_k,
                       int64_t E, int64_t H, int64_t I, int64_t group_size, void* stream);

/* The four stages of moe_forward, for callers that schedule or time them
 * separately.  They share one workspace of moe_workspace_bytes(M, top_k, E,
 * H, I) bytes that carries the routing plan and the intermediate
 * activations from stage to stage; call them in this order, on one stream,
 * with identical sizes.
 *   moe_plan      expert sort of topk_idx (quantization.py:266-276) and the
 *                 activation staging for the expert GEMMs;
 *   moe_gate_up   grouped gate_up GEMM with the gated GELU fused
 *                 (first Triton launch + glue, quantization.py:112-120);
 *   moe_down      grouped down GEMM (second launch, quantization.py:122-127);
 *   moe_combine   weighted top-k sum into out (quantization.py:128-129).    */
W4A16_API int moe_plan(const uint16_t* hidden, const int64_t* topk_idx, int64_t M, int64_t top_k,
             int64_t E, int64_t H, int64_t I, int64_t group_size, void* workspace,
             size_t workspace_bytes, void* stream);
W4A16_API int moe_gate_up(const uint16_t* hidden, const int32_t* gu_packed, const uint16_t* gu_scale, int64_t M, int64_t top_k,
                int64_t E, int64_t H, int64_t I, int64_t group_size, void* workspace,
                size_t workspace_bytes, void* stream);
W4A16_API int moe_down(const int32_t* dn_packed, const uint16_t* dn_scale, int64_t M, int64_t top_k,
             int64_t E, int64_t H, int64_t I, int64_t group_size, void* workspace,
             size_t workspace_bytes, void* stream);
W4A16_API int moe_combine(const int64_t* topk_idx, const float* topk_w, uint16_t* out, int64_t M,
                int64_t top_k, int64_t E, int64_t H, int64_t I, void* workspace,
                size_t workspace_bytes, void* stream);

/* Router + experts in one call: the MoE half of _ffn_moe_4bit_step
 *   -- backends.py:111-122
 * router_in [M, H] feeds the router (moe_router_topk semantics), hidden
 * [M, H] feeds the experts (moe_forward semantics); they may alias.  Writes
 * out [M, H] and the routing topk_idx [M, top_k] / topk_w [M, top_k].     */
W4A16_API size_t moe_layer_workspace_bytes(int64_t M, int64_t top_k, int64_t E, int64_t H, int64_t I);
W4A16_API int moe_layer_forward(const uint16_t* router_in, const uint16_t* router_scale, float scalar_root,
                      const uint16_t* proj_w, const uint16_t* per_expert_scale, float eps,
                      const uint16_t* hidden, const int32_t* gu_packed, const uint16_t* gu_scale,
                      const int32_t* dn_packed, const uint16_t* dn_scale, uint16_t* out,
                      int64_t* topk_idx, float* topk_w, int64_t M, int64_t top_k, int64_t E,
                      int64_t H, int64_t I, int64_t group_size, void* workspace,
                      size_t workspace_bytes, void* stream);

/* Tiled weight copies: load-time copies of an expert stack's packed weights
 * (the layout the checkpoint loader writes, quantization.py:325-430) in the
 * order a kernel reads them, so each of its load instructions reads one
 * contiguous KiB instead of 16 or 32 bytes of many rows.  The reference keeps
 * one layout; these copies are extra (their own buffers; the packed tensors
 * are left as they are and still serve every path).  Kinds:
 *   W4A16_TILED_GATE_UP_DECODE / _DOWN_DECODE
 *       the decode streamers' copies of gate_up_packed / down_packed, for
 *       group size 128 (an even group count per row) or 32 / 64; at 32 and
 *       64 the copy also holds the rows' group scales (taken from `scale`),
 *       laid out so each lane loads the scales of its own weight chunks in
 *       one 16-byte read beside them;
 *   W4A16_TILED_GATE_UP_PREFILL / _DOWN_PREFILL
 *       the exact-form prefill GEMM's copies (any group size; `scale` unused).
 *   w4a16_tiled_bytes  bytes of a copy of `kind` for (E, H, I, group_size),
 *                      0 where the kernel that reads it has no tiled form;
 *   w4a16_tile         writes it (W4A16_ERR_SHAPE where the bytes are 0,
 *                      W4A16_ERR_WORKSPACE when tiled_bytes is short).
 * A w4a16_tiled_experts names the copies of one expert stack and the shape
 * they were made for; the *_tiled entry points below take one (NULL: none)
 * and check it before any launch: E, H, I and group_size must equal the
 * call's (else W4A16_ERR_SHAPE), every non-NULL copy must exist for that
 * shape (W4A16_ERR_SHAPE) and hold at least w4a16_tiled_bytes() bytes
 * (W4A16_ERR_WORKSPACE), 16-byte aligned (W4A16_ERR_ALIGN).  A NULL copy
 * leaves its kernel on the packed tensors; each copy serves the kernels that
 * read it where they run (decode or prefill sizes).  Results are
 * bit-identical to the untiled calls.
 *   moe_gate_up_tiled, moe_down_tiled    the stage calls (moe_gate_up, moe_down);
 *   moe_forward_tiled                    moe_forward (fused_triton_4bit_moe_forward,
 *                                        quantization.py:88-129);
 *   moe_layer_forward_tiled              moe_layer_forward (backends.py:111-122);
 *   moe_ffn_block_forward_tiled          moe_ffn_block_forward (backends.py:77-126).  */
enum w4a16_tiled_kind {
  W4A16_TILED_GATE_UP_DECODE = 0,
  W4A16_TILED_DOWN_DECODE = 1,
  W4A16_TILED_GATE_UP_PREFILL = 2,
  W4A16_TILED_DOWN_PREFILL = 3
};
typedef struct w4a16_tiled_experts {
  int64_t E, H, I, group_size;      /* the expert stack the copies were made from */
  const int32_t* gu_decode;  size_t gu_decode_bytes;   /* W4A16_TILED_GATE_UP_DECODE or NULL */
  const int32_t* dn_decode;  size_t dn_decode_bytes;   /* W4A16_TILED_DOWN_DECODE or NULL */
  const int32_t* gu_prefill; size_t gu_prefill_bytes;  /* W4A16_TILED_GATE_UP_PREFILL or NULL */
  const int32_t* dn_prefill; size_t dn_prefill_bytes;  /* W4A16_TILED_DOWN_PREFILL or NULL */
} w4a16_tiled_experts;
W4A16_API size_t w4a16_tiled_bytes(int kind, int64_t E, int64_t H, int64_t I, int64_t group_size);
W4A16_API int w4a16_tile(int kind, const int32_t* packed, const uint16_t* scale, int64_t E, int64_t H, int64_t I,
                         int64_t group_size, int32_t* tiled, size_t tiled_bytes, void* stream);
W4A16_API int moe_gate_up_tiled(const uint16_t* hidden, const int32_t* gu_packed, const uint16_t* gu_scale,
                                const w4a16_tiled_experts* tiled, int64_t M, int64_t top_k, int64_t E, int64_t H,
                                int64_t I, int64_t group_size, void* workspace, size_t workspace_bytes,
                                void* stream);
W4A16_API int moe_down_tiled(const int32_t* dn_packed, const uint16_t* dn_scale, const w4a16_tiled_experts* tiled,
                             int64_t M, int64_t top_k, int64_t E, int64_t H, int64_t I, int64_t group_size,
                             void* workspace, size_t workspace_bytes, void* stream);
W4A16_API int moe_forward_tiled(const uint16_t* hidden, const int64_t* topk_idx, const float* topk_w,
                                const int32_t* gu_packed, const uint16_t* gu_scale, const int32_t* dn_packed,
                                const uint16_t* dn_scale, const w4a16_tiled_experts* tiled, uint16_t* out,
                                int64_t M, int64_t top_k, int64_t E, int64_t H, int64_t I, int64_t group_size,
                                void* workspace, size_t workspace_bytes, void* stream);
W4A16_API int moe_layer_forward_tiled(const uint16_t* router_in, const uint16_t* router_scale,
                                      float scalar_root, const uint16_t* proj_w,
                                      const uint16_t* per_expert_scale, float eps, const uint16_t* hidden,
                                      const int32_t* gu_packed, const uint16_t* gu_scale,
                                      const int32_t* dn_packed, const uint16_t* dn_scale,
                                      const w4a16_tiled_experts* tiled, uint16_t* out, int64_t* topk_idx,
                                      float* topk_w, int64_t M, int64_t top_k, int64_t E, int64_t H,
                                      int64_t I, int64_t group_size, void* workspace,
                                      size_t workspace_bytes, void* stream);

/* The latent harness's layer step (configs[4], the latent loop's MoE
 * stack: h <- h + MoE(RMSNorm(h)) per layer, the RMSNorm of
 * modeling_gemma4.py:197-215, the router lines of backends.py:111-122):
 * moe_layer_forward
 * on router_in = h and hidden = RMSNorm(h) (tiled: NULL or the copies, as for
 * moe_layer_forward_tiled), then the residual add and the next layer's norm
 *   h_out = bf16(h + out),  y_out = bf16((h_out * rsqrt(mean(h_out^2) + norm_eps)) * norm_w)
 * -- bit for bit moe_layer_forward followed by w4a16_add_rms_norm(h, out,
 * norm_w) -- with the combine, the add and the norm in one launch where the
 * layer combines in a launch of its own (more than 32 routed rows, top_k <= 8).
 * No function of the reference matches it: it fuses the harness's residual
 * add and norm around moe_layer_forward.  norm_w [H], h_out, y_out [M, H]
 * bf16, 16-byte aligned; H <= 8192; workspace as for moe_layer_forward.    */
W4A16_API int moe_layer_forward_add_norm(const uint16_t* router_in, const uint16_t* router_scale,
                                         float scalar_root, const uint16_t* proj_w,
                                         const uint16_t* per_expert_scale, float eps, const uint16_t* hidden,
                                         const int32_t* gu_packed, const uint16_t* gu_scale,
                                         const int32_t* dn_packed, const uint16_t* dn_scale,
                                         const w4a16_tiled_experts* tiled, uint16_t* out, int64_t* topk_idx,
                                         float* topk_w, const uint16_t* norm_w, float norm_eps, uint16_t* h_out,
                                         uint16_t* y_out, int64_t M, int64_t top_k, int64_t E, int64_t H,
                                         int64_t I, int64_t group_size, void* workspace,
                                         size_t workspace_bytes, void* stream);

/* The BF16 experts (unquantised Gemma4TextExperts weights) on the same
 * routing machinery: _bf16_experts_fast_forward  -- backends.py:209-283
 * (installed on every BF16 experts module by patch_bf16_experts_fastpath,
 * backends.py:286-298):
 *   out[t] = sum_j bf16(topk_w[t,j]) * down_e(gelu_tanh(gate_e(x)) * up_e(x)),
 * e = topk_idx[t, j], bf16 rounding after every op.
 * hidden [M, H] bf16; gate_up_proj [E, 2I, H] bf16 (gate rows first);
 * down_proj [E, H, I] bf16; topk as for moe_forward; slots outside [0, E)
 * contribute nothing.  Workspace: moe_bf16_experts_workspace_bytes().    */
W4A16_API size_t moe_bf16_experts_workspace_bytes(int64_t M, int64_t top_k, int64_t E, int64_t H,
                                                  int64_t I);
W4A16_API int moe_bf16_experts_forward(const uint16_t* hidden, const int64_t* topk_idx,
                             const float* topk_w, const uint16_t* gate_up_proj,
                             const uint16_t* down_proj, uint16_t* out, int64_t M, int64_t top_k,
                             int64_t E, int64_t H, int64_t I, void* workspace,
                             size_t workspace_bytes, void* stream);

/* The post-attention FFN block of a Gemma-4 MoE decoder layer,
 * _ffn_moe_4bit_step  -- backends.py:77-126 (installed per layer by
 * patch_compiled_ffn_4bit, backends.py:132-201):
 *   h      = rms_norm(attn_out) * post_attn_ln_w;  res = residual + h
 *   h_ff   = rms_norm(res) * pre_ff_ln_w
 *   h_mlp  = down(gelu_tanh(gate(h_ff)) * up(h_ff))        (shared bf16 MLP)
 *   h_1    = rms_norm(h_mlp) * post_ff_ln1_w
 *   router on res (moe_router_topk semantics), experts on
 *   h2_in  = rms_norm(res) * pre_ff_ln2_w (moe_forward semantics)
 *   h_2    = rms_norm(moe_out) * post_ff_ln2_w
 *   h_comb = rms_norm(h_1 + h_2) * post_ff_ln_w
 *   out    = (res + h_comb) * layer_scalar
 * bf16 rounding after every op (the eager torch ops' rounding points).
 * residual, attn_out, out [M, H] bf16; the norm weights [H] bf16;
 * mlp_gate_w, mlp_up_w [Im, H], mlp_down_w [H, Im] bf16 (nn.Linear layout);
 * router and expert tensors as for moe_layer_forward; layer_scalar: one bf16
 * value in device memory.  H % 32 == 0, H <= 8192, Im % 32 == 0.          */
W4A16_API size_t moe_ffn_block_workspace_bytes(int64_t M, int64_t top_k, int64_t E, int64_t H,
                                               int64_t I, int64_t Im);
W4A16_API int moe_ffn_block_forward(const uint16_t* residual, const uint16_t* attn_out,
                          const uint16_t* post_attn_ln_w, const uint16_t* pre_ff_ln_w,
                          const uint16_t* mlp_gate_w, const uint16_t* mlp_up_w,
                          const uint16_t* mlp_down_w, const uint16_t* post_ff_ln1_w,
                          const uint16_t* router_scale, float router_scalar_root,
                          const uint16_t* router_proj_w, const uint16_t* router_per_expert_scale,
                          const uint16_t* pre_ff_ln2_w, const int32_t* gu_packed,
                          const uint16_t* gu_scale, const int32_t* dn_packed,
                          const uint16_t* dn_scale, const uint16_t* post_ff_ln2_w,
                          const uint16_t* post_ff_ln_w, const uint16_t* layer_scalar, float eps,
                          uint16_t* out, int64_t M, int64_t top_k, int64_t E, int64_t H, int64_t I,
                          int64_t Im, int64_t group_size, void* workspace, size_t workspace_bytes,
                          void* stream);
/* moe_ffn_block_forward with the experts' tiled weight copies (see
 * w4a16_tiled_experts above; NULL: none).                                  */
W4A16_API int moe_ffn_block_forward_tiled(
    const uint16_t* residual, const uint16_t* attn_out, const uint16_t* post_attn_ln_w, const uint16_t* pre_ff_ln_w,
    const uint16_t* mlp_gate_w, const uint16_t* mlp_up_w, const uint16_t* mlp_down_w, const uint16_t* post_ff_ln1_w,
    const uint16_t* router_scale, float router_scalar_root, const uint16_t* router_proj_w,
    const uint16_t* router_per_expert_scale, const uint16_t* pre_ff_ln2_w, const int32_t* gu_packed,
    const uint16_t* gu_scale, const int32_t* dn_packed, const uint16_t* dn_scale, const w4a16_tiled_experts* tiled,
    const uint16_t* post_ff_ln2_w, const uint16_t* post_ff_ln_w, const uint16_t* layer_scalar, float eps,
    uint16_t* out, int64_t M, int64_t top_k, int64_t E, int64_t H, int64_t I, int64_t Im, int64_t group_size,
    void* workspace, size_t workspace_bytes, void* stream);
/* Where moe_ffn_block_forward[_tiled] leaves, in its workspace, the routing
 * its router step took (backends.py:111-117): top_k_index int64 [M, top_k]
 * at byte *idx_offset and top_k_weights float32 [M, top_k] at *w_offset,
 * valid after the call until the workspace is reused.  The reference's
 * compiled block keeps them internal; this lets a caller (or a test) read
 * the routing each output row used.                                        */
W4A16_API int moe_ffn_block_routing_offsets(int64_t M, int64_t top_k, int64_t E, int64_t H, int64_t I,
                                            int64_t Im, size_t* idx_offset, size_t* w_offset);

#ifdef __cplusplus
}
#endif

#endif /* W4A16MOE_H */
