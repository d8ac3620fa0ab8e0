/*
 * xk_moe.h — C ABI of the MI355X (gfx950 / CDNA4) quantized fused-MoE library
 * (libxk_moe.so).
 *
 * Every entry point takes raw device pointers, 64-bit sizes and the HIP stream to
 * launch on. The caller owns every buffer: inputs, outputs and the scratch
 * workspace (sized by the matching *_workspace_bytes query). The library never
 * allocates or frees device memory and never synchronises the stream.
 * Entry points are re-entrant; concurrent calls on different streams must use
 * different workspaces.
 *
 * Return value: XK_OK (0) on success, otherwise an XK_ERR_* code; the message
 * for the last failure on the calling thread is returned by xk_last_error().
 *
 * Dtype codes (XK_DT_*) describe activations / outputs. Weights use the fixed
 * formats of the reference op specs:
 *   INT4 W4A16 : packed int32 [E, N, K/8], 8 uint4b8 nibbles per word, low nibble
 *                = lowest k; value = (nibble - 8) * scale; scale bf16 [E, N, K/g].
 *   MXFP4      : uint8 [E, rows, K/2], two e2m1 nibbles per byte, low nibble = even
 *                k; scale uint8 e8m0 [E, rows, K/32], value = e2m1 * 2^(byte-127),
 *                byte 0xFF decodes as 0.
 *
 * Reference interfaces replaced (paths relative to the xkernels checkout):
 *   xk_moe_align_block_size  -> src/xkernels/ops/moe/align.py:34-70
 *                               (oracle w4a16.py:53-101, EP remap w4a16.py:104-155)
 *   xk_moe_sum_reduce        -> src/xkernels/ops/moe/sum_reduce.py:45-58
 *                               (oracle sum_reduce.py:20-39)
 *   xk_moe_int4_w4a16        -> src/xkernels/ops/moe/interface.py:19-83
 *                               (oracle reference.py:22-70)
 *   xk_moe_mxfp4             -> src/xkernels/ops/moe/mxfp4_interface.py:22-100
 *                               (oracle mxfp4_reference.py:28-112)
 *   stage entry points       -> the launch steps inside
 *                               triton/moe_int4_kernel.py:438-577 and
 *                               triton/moe_mxfp4_kernel.py:487-568
 */
#ifndef XK_MOE_H
#define XK_MOE_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define XK_OK 0
#define XK_ERR_INVALID 1   /* bad argument: shape, dtype, null pointer, size */
#define XK_ERR_WORKSPACE 2 /* workspace too small */
#define XK_ERR_LAUNCH 3    /* hipGetLastError reported a launch failure */

#define XK_DT_BF16 0
#define XK_DT_FP32 1
#define XK_DT_FP16 2 /* accepted by xk_moe_topk_softmax only */
#define XK_DT_NONE (-1) /* "no tensor" for optional weights */

/* int4 `flags` arguments: pass 0. Every dequantised weight is rounded to bf16
 * before the contraction, as the reference does. Bits 8 and 9 are test-only
 * kernel choices used by this library's GPU tests (force the prefill tile
 * kernel / the decode stream kernel where the shapes allow both); a fused call
 * given them returns XK_ERR_INVALID when the partial planes the forced kernel
 * writes do not fit the workspace sized by xk_moe_int4_w4a16_workspace_bytes.
 * Every other bit is rejected (XK_ERR_INVALID). */

/* Message of the last failed call on this thread ("" if none). */
const char* xk_last_error(void);

/* ABI version (major * 100 + minor). */
int xk_abi_version(void);

/* ---------------------------------------------------------------------------
 * moe_align_block_size — align.py:34-70 / w4a16.py:53-101.
 *
 * Groups the flattened token-slots t = m*top_k + j of topk_ids by expert in
 * ascending slot order (a stable sort), pads each expert's run to a multiple of
 * block_size with pad id = numel, and emits one expert id per block.
 *   sorted_token_ids [max_pad]   max_pad = numel + (num_experts+1)*(block_size-1)
 *   expert_ids       [max_blocks] max_blocks = ceil(max_pad / block_size); blocks
 *                    past num_tokens_post_padded hold 0 (the truncate=False form;
 *                    the truncated view is a prefix of it)
 *   num_tokens_post_padded [1]
 *   expert_offsets   [num_experts+1] padded exclusive prefix in slots (nullable)
 * expert_map (nullable, [num_global_experts]) remaps global ids to local rows;
 * -1 drops the slot (w4a16.py:104-155). Ids outside [0, num_experts) after the
 * remap are counted nowhere and never placed (w4a16.py:74-88).
 * ------------------------------------------------------------------------- */
int64_t xk_moe_align_workspace_bytes(int64_t numel, int32_t num_experts);
int xk_moe_align_block_size(const int32_t* topk_ids, int64_t numel,
                            int32_t num_experts, int32_t block_size,
                            const int32_t* expert_map, int32_t num_global_experts,
                            int32_t* sorted_token_ids, int32_t* expert_ids,
                            int32_t* num_tokens_post_padded,
                            int32_t* expert_offsets,
                            void* workspace, int64_t workspace_bytes,
                            hipStream_t stream);

/* ---------------------------------------------------------------------------
 * moe_sum_reduce — sum_reduce.py:20-39.
 *   out[m, h] = routed_scaling_factor * sum_k w[m, k] * y[m, k, h]
 * accumulated in fp32, written in y's dtype. w may be NULL (plain sum).
 * y [M, top_k, H] and w [M, top_k] are contiguous.
 * ------------------------------------------------------------------------- */
int xk_moe_sum_reduce(const void* y, int32_t y_dtype, int64_t M, int64_t top_k,
                      int64_t H, const void* w, int32_t w_dtype,
                      float routed_scaling_factor, void* out,
                      hipStream_t stream);

/* ---------------------------------------------------------------------------
 * fused_moe_int4_w4a16 — interface.py:19-83 / reference.py:22-70.
 *   out[m] = sum_j [w[m,j]] * (A[m] @ W[e_j]^T),  e_j = topk_ids[m, j]
 * A [M, K] bf16|fp32, out [M, N] in A's dtype, topk_w fp32 [M, top_k].
 * expert_map (nullable) selects this rank's experts; the result is then the
 * rank's partial output. Runs align -> grouped GEMM -> weighted combine.
 * ------------------------------------------------------------------------- */
int64_t xk_moe_int4_w4a16_workspace_bytes(int64_t M, int64_t top_k, int64_t E,
                                          int64_t N, int64_t K);
/* The workspace for calls with an expert map over num_global_experts experts
 * (>= the above). With an expert map the kernel choice counts the slots
 * expected on the E local experts (M*top_k*E/num_global_experts, the rows per
 * expert of the dense call) when the workspace holds that choice's partial
 * planes, as one of this size does; otherwise every slot counts. The result is
 * the same contraction either way (fp32 summation order aside). No
 * counterpart in the reference (it has no workspace query). */
int64_t xk_moe_int4_w4a16_ep_workspace_bytes(int64_t M, int64_t top_k, int64_t E,
                                             int64_t N, int64_t K,
                                             int32_t num_global_experts);
int xk_moe_int4_w4a16(const void* A, int32_t a_dtype, int64_t M, int64_t K,
                      const int32_t* packed, const uint16_t* scale, int64_t E,
                      int64_t N, int32_t group_size, const int32_t* topk_ids,
                      const float* topk_w, int64_t top_k,
                      const int32_t* expert_map, int32_t num_global_experts,
                      int32_t mul_routed_weight, int32_t flags, void* out,
                      void* workspace, int64_t workspace_bytes, hipStream_t stream);

/* No counterpart in the reference. xk_moe_int4_w4a16 for callers that cannot
 * allocate device memory (code under HIP graph capture that must not call
 * hipMalloc, tight serving loops, harnesses that forbid allocation): same
 * arguments without the workspace; the scratch is a fixed device array of
 * xk_moe_int4_w4a16_noalloc_max_bytes() bytes (64 MiB) inside the library,
 * one per GPU, held until the process ends. A call whose
 * xk_moe_int4_w4a16_workspace_bytes(...) exceeds it fails with XK_ERR_INVALID.
 * Every call on one GPU uses the same array: calls that overlap on a GPU (two
 * streams, two host threads) race; calls ordered on one stream do not. */
int64_t xk_moe_int4_w4a16_noalloc_max_bytes(void);
int xk_moe_int4_w4a16_noalloc(const void* A, int32_t a_dtype, int64_t M, int64_t K,
                              const int32_t* packed, const uint16_t* scale, int64_t E,
                              int64_t N, int32_t group_size, const int32_t* topk_ids,
                              const float* topk_w, int64_t top_k,
                              const int32_t* expert_map, int32_t num_global_experts,
                              int32_t mul_routed_weight, int32_t flags, void* out,
                              hipStream_t stream);

/* Stage entry point: only the grouped INT4 GEMM (the reference's
 * _fused_moe_int4_kernel launch, moe_int4_kernel.py:78-272). Consumes the
 * align outputs built with block_size = xk_moe_int4_block_size(M, top_k, E)
 * (expert_offsets are multiples of that block size) and writes un-weighted
 * fp32 per-slot rows for every routed slot (rows of dropped slots are left
 * untouched). The decode kernel splits K: slot_out is [parts, numel, N] with
 * parts = xk_moe_int4_gemm_parts(...) for the same arguments; every plane
 * holds one K slice's partial rows and xk_moe_topk_combine(..., nparts =
 * parts) sums them. The prefill tile kernel keeps a tile queue of
 * xk_moe_int4_gemm_workspace_bytes(...) bytes in the workspace (one workspace
 * per concurrently running call); with a NULL or smaller workspace it deals
 * its tiles statically. The other kernels use no workspace. A, packed and scale
 * must be 16-byte aligned for the MFMA kernels. In the decode regime
 * (xk_moe_int4_gemm_parts(...) > 1 or M * top_k small against E, at most 4096
 * routed slots) sorted_token_ids and expert_offsets may both be NULL: the
 * kernel then routes the slots from topk_ids / expert_map itself (the fused
 * call does this and skips the align). Used by benchmarks to time the GEMM
 * alone. */
int32_t xk_moe_int4_block_size(int64_t M, int64_t top_k, int64_t E);
/* Which grouped-GEMM kernel a fused call with these shapes runs: 0 the scalar
 * kernel (shapes the MFMA kernels do not take, including activations or one
 * expert's packed weights of 2^31 bytes or more; the fused call runs a batch
 * whose activations reach 2^31 bytes as token chunks, each with the choice for
 * its own M), 1 the decode weight-streaming
 * kernel, 2 the prefill MFMA tile kernel. num_global_experts: the expert map's
 * size for an expert-parallel call with a workspace of
 * xk_moe_int4_w4a16_ep_workspace_bytes, else 0. No counterpart in the
 * reference (its Triton launcher has no such query); for tests and tooling. */
int32_t xk_moe_int4_kernel(int64_t M, int64_t top_k, int64_t E, int64_t N,
                           int64_t K, int32_t a_dtype, int32_t group_size,
                           int32_t flags, int32_t num_global_experts);
int32_t xk_moe_int4_gemm_parts(int64_t M, int64_t top_k, int64_t E, int64_t N, int64_t K,
                               int32_t a_dtype, int32_t group_size, int32_t flags);
int64_t xk_moe_int4_gemm_workspace_bytes(int64_t M, int64_t K);
int xk_moe_int4_w4a16_gemm(const void* A, int32_t a_dtype, int64_t M, int64_t K,
                           const int32_t* packed, const uint16_t* scale,
                           int64_t E, int64_t N, int32_t group_size,
                           const int32_t* topk_ids, int64_t top_k,
                           const int32_t* expert_map, int32_t num_global_experts,
                           const int32_t* sorted_token_ids,
                           const int32_t* expert_offsets, float* slot_out,
                           int32_t flags, void* workspace, int64_t workspace_bytes,
                           hipStream_t stream);

/* Stage entry point: the weighted top-k combine of per-slot fp32 rows,
 *   out[m, n] = sum_j valid(m,j) * [w[m,j]] * sum_p slot_out[p, m*top_k + j, n]
 * where valid drops slots whose expert is not local (expert_map) or out of
 * range; out in out_dtype. */
int xk_moe_topk_combine(const float* slot_out, int64_t M, int64_t top_k,
                        int64_t N, const float* topk_w, int32_t mul_routed_weight,
                        const int32_t* topk_ids, int32_t num_local_experts,
                        const int32_t* expert_map, int32_t num_global_experts,
                        void* out, int32_t out_dtype, int32_t nparts,
                        hipStream_t stream);

/* ---------------------------------------------------------------------------
 * topk_softmax — topk_softmax.py:33-120 (the router that produces topk_ids /
 * topk_w for the MoE calls). probs = softmax(fp32(gating[m, :])) over all E
 * experts; the k largest in descending probability, ties broken by ascending
 * expert id; with renormalize the selected weights are divided by their sum.
 * gating [M, E] bf16 | fp32 | fp16 contiguous; topk_weights fp32 [M, k],
 * topk_ids int32 [M, k]. 1 <= k <= E (rows of more than 2048 experts take a
 * streaming kernel: k passes over the row).
 * ------------------------------------------------------------------------- */
int xk_moe_topk_softmax(const void* gating_output, int32_t dtype, int64_t M, int64_t E,
                        int64_t topk, int32_t renormalize, float* topk_weights,
                        int32_t* topk_ids, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * fused_moe_mxfp4 — mxfp4_interface.py:22-100 / mxfp4_reference.py:28-112.
 * Per routed (m, e): gu = bf16(A[m]) @ w13[e]^T (+b13[e]); g, u = halves;
 * act = bf16(silu(min(g, L)) * clamp(u, -L, L)); down = act @ w2[e]^T (+b2[e]);
 * out[m] += [w] * down. swiglu_limit <= 0 disables the clamp.
 * A [M, hidden] bf16|fp32; w13 [E, 2*ispp, hidden/2] u8; w13_scale
 * [E, 2*ispp, hidden/32] u8; w2 [E, hidden, ispp/2] u8; w2_scale
 * [E, hidden, ispp/32] u8; b13 [E, 2*ispp] bf16 | NULL; b2 [E, hidden] bf16 |
 * NULL; out [M, hidden] in A's dtype.
 * ------------------------------------------------------------------------- */
int64_t xk_moe_mxfp4_workspace_bytes(int64_t M, int64_t top_k, int64_t E,
                                     int64_t hidden, int64_t ispp);
int xk_moe_mxfp4(const void* A, int32_t a_dtype, int64_t M, int64_t hidden,
                 const uint8_t* w13, const uint8_t* w13_scale, const uint8_t* w2,
                 const uint8_t* w2_scale, int64_t E, int64_t ispp,
                 const uint16_t* b13, const uint16_t* b2, float swiglu_limit,
                 int32_t group_size, const int32_t* topk_ids, const float* topk_w,
                 int64_t top_k, const int32_t* expert_map,
                 int32_t num_global_experts, int32_t mul_routed_weight, void* out,
                 void* workspace, int64_t workspace_bytes, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* XK_MOE_H */
