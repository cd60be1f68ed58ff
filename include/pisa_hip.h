/*
 * pisa_hip.h -- C ABI of the MI355X (gfx950) attention hot path.
 *
 * One shared library (libpisa_hip.so) exports these entry points.  Every
 * argument is a plain pointer, integer, float or a POD struct; no framework
 * type crosses the boundary.  Device pointers are HIP device addresses, the
 * stream is a hipStream_t passed as void*, and every call only enqueues work
 * on that stream (no host synchronisation, no allocation: callers pass the
 * workspace sized by the matching *_workspace_bytes function).
 *
 * Every entry point returns PISA_OK (0) or a PISA_ERR_* code; a human readable
 * description of the last failure on the calling thread is available from
 * pisa_hip_last_error().  Validation failures never launch a kernel.
 * Problem sizes: every entry point takes B*H <= 65535 and at most 2^24 - 1
 * 64-token blocks over all heads (B*H*ceil(T/64), for dense attention both
 * Tq and Tk); larger problems return PISA_ERR_UNSUPPORTED and the
 * *_workspace_bytes functions return 0 for them.
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   native/rdna35_pisa_ck/csrc/bindings.cpp:34-83          pybind module _C
 *   native/rdna35_pisa_ck/rdna35_pisa_ck/__init__.py:233-433 forward / forward_spatial_bhtd
 *   rdna35_block_attention/generic_pisa.py:141-232        generic_pisa_attention
 *   rdna35_block_attention/triton_kernel.py:166-244       Triton full / fixed-block kernels
 *   rdna35_block_attention/pisa_kernel.py:90-131          Triton PISA statistics
 */
#ifndef PISA_HIP_H
#define PISA_HIP_H

#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define PISA_HIP_EXPORT __attribute__((visibility("default")))
#else
#define PISA_HIP_EXPORT
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define PISA_HIP_API_VERSION 1
#define PISA_BLOCK_SIZE 64

/* ---- status codes ------------------------------------------------------ */
#define PISA_OK 0
#define PISA_ERR_INVALID_ARGUMENT 1
#define PISA_ERR_UNSUPPORTED 2
#define PISA_ERR_WORKSPACE 3
#define PISA_ERR_LAUNCH 4
#define PISA_ERR_DEVICE 5

/* ---- element types ----------------------------------------------------- */
#define PISA_DTYPE_BF16 0
#define PISA_DTYPE_F16 1
#define PISA_DTYPE_F32 2

/* ---- PISA statistics modes --------------------------------------------- */
/* plain block means, each element pre-scaled by 1/len before accumulation
 * (pisa_kernels.cu:130-164, block_stats_kernel)                              */
#define PISA_STATS_MEANS 0
/* HYD: sum-then-scale means, key covariance centred in fp32
 * (pisa_kernels.cu:167-244, block_stats_hyd_kernel)                          */
#define PISA_STATS_HYD 1
/* generic: centred keys rounded to the input dtype before the product
 * (pisa_kernel.py:49-84, _pisa_block_stats_kernel)                          */
#define PISA_STATS_GENERIC 2
/* OR-ed into pisa_hip_block_stats' stats_mode (HYD or GENERIC, out_dtype
 * PISA_DTYPE_F32): v_means receives the fp32 per-block value sums instead of
 * the means, the v_sums output of pisa_prepare_triton (pisa_kernel.py:74,78) */
#define PISA_STATS_FLAG_VALUE_SUMS 0x100

/* ---- routing modes ----------------------------------------------------- */
/* HYD: r = s * (bf16(qbar) . bf16(kbar)) + ln(h_norm + 1e-5)
 * (native/rdna35_pisa_ck/rdna35_pisa_ck/__init__.py:258-264)                */
#define PISA_ROUTE_HYD 0
/* centroid: r = s * (qbar_f32 . kbar_f32)   (generic_pisa.py:303-315)        */
#define PISA_ROUTE_CENTROID 1

/* No sink block (the reference encodes None as -2, __init__.py:403). */
#define PISA_NO_SINK (-2)

/*
 * A [B, H, T, D] tensor view whose head_dim stride is 1.  Strides are in
 * elements.  Row (b, h, t) starts at data + b*batch_stride + h*head_stride
 * + t*token_stride.  This covers contiguous [B,H,T,D], BHTD views of
 * [B,T,H,D] storage (the Anima layout), flat [BH,T,D] (batch=BH, heads=1)
 * and strided views into a fused [B,T,3,H,D] projection (MiniMax-H3).
 */
typedef struct pisa_view {
    void* data;
    int64_t batch_stride;
    int64_t head_stride;
    int64_t token_stride;
} pisa_view;

/*
 * Token order of the PISA blocks.  frames == 0: block b holds tokens
 * [64b, 64b+64) (identity order).  frames > 0: tokens are raster ordered on a
 * frames x height x width grid (height, width multiples of 8) and block b of
 * frame f is the 8x8 spatial tile number b (row-major over tiles) of that
 * frame, its 64 tokens in row-major order inside the tile.  This is the order
 * produced by pack_spatial_qkv_kernel (pisa_kernels.cu:55-64,247-272) for
 * frames=1, height=width=96, and by _pack_video_blocks (generic_pisa.py:37-52).
 */
typedef struct pisa_token_grid {
    int32_t frames;
    int32_t height;
    int32_t width;
} pisa_token_grid;

/*
 * Attention mask of fixed-block attention (fixed_block_attention_ref's
 * `mask`, reference.py:114-156 slicing, :186-195 use), already broadcast to
 * [B, H, T, T]: element (b, h, i, j) is at data + b*batch_stride +
 * h*head_stride + i*query_stride + j*key_stride (elements; a stride of 0
 * broadcasts), with h < heads.  Only the block-diagonal entries are read.
 *   PISA_MASK_BOOL      1-byte values, the score is kept where nonzero
 *   PISA_MASK_ADD_F32 / _F16 / _BF16   added to the scaled score
 */
#define PISA_MASK_NONE 0
#define PISA_MASK_BOOL 1
#define PISA_MASK_ADD_F32 2
#define PISA_MASK_ADD_F16 3
#define PISA_MASK_ADD_BF16 4
typedef struct pisa_mask {
    const void* data;
    int32_t kind;
    int32_t heads;
    int64_t batch_stride;
    int64_t head_stride;
    int64_t query_stride;
    int64_t key_stride;
} pisa_mask;

/* ---- library metadata -------------------------------------------------- */

/* API revision of this header (the reference checks api==6, pisa_attention.py:470). */
PISA_HIP_EXPORT int pisa_hip_api_version(void);

/* Static description of the status code. */
PISA_HIP_EXPORT const char* pisa_hip_status_string(int status);

/* Description of the last failure on the calling thread ("" if none). */
PISA_HIP_EXPORT const char* pisa_hip_last_error(void);

/* Writes "key=value;..." build information into buffer (NUL terminated).
 * Replaces build_info in bindings.cpp:70-82. Returns PISA_ERR_INVALID_ARGUMENT
 * when capacity is too small. */
PISA_HIP_EXPORT int pisa_hip_build_info(char* buffer, int64_t capacity);

/* ---- PISA forward (subsystems 1-4 fused into three launches) ----------- */

/* Bytes of workspace pisa_hip_forward needs for this problem. */
PISA_HIP_EXPORT int64_t pisa_hip_forward_workspace_bytes(int32_t batch, int32_t heads, int32_t tokens,
                                         int32_t head_dim, int32_t exact_blocks);

/*
 * PISA block-sparse self attention, output written through `out`.
 * Replaces rdna35_pisa_ck._forward_impl (__init__.py:233-316) including its
 * spatial variant (_forward_spatial_bhtd_op, __init__.py:344-365, with the
 * fused epilogue of pisa_kernels.cu:296-340) and generic_pisa_attention
 * (generic_pisa.py:141-232).
 *   head_dim       128, or any multiple of 8 up to 256 with PISA_STATS_GENERIC and
 *                  PISA_ROUTE_CENTROID (first_order at any of them: the Triton
 *                  statistics of generic_pisa.py:128-138 form H_sum at every width)
 *   stats_mode     PISA_STATS_HYD or PISA_STATS_GENERIC
 *   route_mode     PISA_ROUTE_HYD or PISA_ROUTE_CENTROID
 *   first_order    1 adds C = s/T * q . bf16(H_sum) weighted by the tail mass
 *   exact_blocks   0 <= exact_blocks < ceil(T/64)  (the caller routes == N to
 *                  attn_hip_dense_forward, as the reference routes it to SDPA)
 *   sink_block     PISA_NO_SINK, 0 or -1
 *   grid           token order of q/k/v/out (out uses the same order)
 *   debug_indices  nullable int32 [B*H, N, exact_blocks] selected key blocks
 *   debug_scores   nullable float [B*H, N, N] routing scores
 */
PISA_HIP_EXPORT int pisa_hip_forward(int32_t dtype, int32_t batch, int32_t heads, int32_t tokens, int32_t head_dim,
                     pisa_view q, pisa_view k, pisa_view v, pisa_view out, pisa_token_grid grid,
                     int32_t exact_blocks, float scale, int32_t sink_block,
                     int32_t stats_mode, int32_t route_mode, int32_t first_order,
                     int32_t* debug_indices, float* debug_scores,
                     void* workspace, int64_t workspace_bytes, void* stream);

/*
 * pisa_hip_forward in two stages sharing one workspace:
 *   pisa_hip_prepare  statistics, H_sum reduction, routing and top-k (3 launches)
 *   pisa_hip_attend   exact tiles + tail + correction + merge (1 launch)
 * attend reads what prepare left in the workspace, so the pair must use the
 * same arguments and workspace, in that order on one stream; prepare + attend
 * is exactly pisa_hip_forward.  Callers that re-attend with unchanged
 * statistics, and profilers that time the attention kernel alone, use these.
 * The reference computes the same stages inside _forward_impl
 * (__init__.py:254-298).
 */
PISA_HIP_EXPORT int pisa_hip_prepare(int32_t dtype, int32_t batch, int32_t heads, int32_t tokens, int32_t head_dim,
                     pisa_view q, pisa_view k, pisa_view v, pisa_view out, pisa_token_grid grid,
                     int32_t exact_blocks, float scale, int32_t sink_block,
                     int32_t stats_mode, int32_t route_mode, int32_t first_order,
                     void* workspace, int64_t workspace_bytes, void* stream);
PISA_HIP_EXPORT int pisa_hip_attend(int32_t dtype, int32_t batch, int32_t heads, int32_t tokens, int32_t head_dim,
                    pisa_view q, pisa_view k, pisa_view v, pisa_view out, pisa_token_grid grid,
                    int32_t exact_blocks, float scale, int32_t sink_block,
                    int32_t stats_mode, int32_t route_mode, int32_t first_order,
                    void* workspace, int64_t workspace_bytes, void* stream);

/*
 * pisa_hip_forward without a caller workspace and without any allocation.
 * This entry point has no counterpart in the reference: it exists for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, hosts that forbid hipMalloc).  The workspace is a static
 * device array of PISA_NOALLOC_SCRATCH_BYTES (192 MiB) inside the library,
 * one per GPU, held until the process ends.  The array belongs to the
 * library's code object, so every process that loads libpisa_hip.so holds
 * these 192 MiB on every GPU it uses the library on, whether or not it ever
 * calls this entry point.  A problem whose
 * pisa_hip_forward_workspace_bytes exceeds it is refused with
 * PISA_ERR_WORKSPACE before anything is launched (the Anima profile
 * B=2 H=16 T=9216 needs 187.3-189.4 MiB, at any exact-block count; the
 * array is sized for it and no larger).  No debug outputs.  Every call on one GPU
 * uses that GPU's one array: calls that overlap on one GPU (two streams, two
 * host threads) race and must be serialised by the caller; calls in one
 * stream are ordered and safe.  Nothing in the array needs to start at zero
 * (every stage writes what it later reads), so no clearing is enqueued.
 * Arguments as pisa_hip_forward.
 */
#define PISA_NOALLOC_SCRATCH_BYTES (192LL << 20)
PISA_HIP_EXPORT int pisa_hip_forward_noalloc(int32_t dtype, int32_t batch, int32_t heads, int32_t tokens,
                             int32_t head_dim, pisa_view q, pisa_view k, pisa_view v, pisa_view out,
                             pisa_token_grid grid, int32_t exact_blocks, float scale, int32_t sink_block,
                             int32_t stats_mode, int32_t route_mode, int32_t first_order, void* stream);

/* ---- subsystem 1: block statistics ------------------------------------- */

PISA_HIP_EXPORT int64_t pisa_hip_block_stats_workspace_bytes(int32_t batch, int32_t heads, int32_t tokens,
                                             int32_t head_dim);

/*
 * Per-64-token-block statistics.  Replaces _C.block_stats / _C.block_stats_hyd
 * (bindings.cpp:36-47, pisa_kernels.cu:563-635) and pisa_prepare_triton
 * (pisa_kernel.py:90-131).
 *   q_centroids  [BH,N,D] in out_dtype (dtype or PISA_DTYPE_F32)
 *   k_centroids  [BH,N,D] float32
 *   v_means      [BH,N,D] in out_dtype
 *   h_sum        [BH,D,D] float32, nullable for PISA_STATS_MEANS
 *   h_norm       [BH,N]   float32 ||H_b||_F, nullable for PISA_STATS_MEANS and, at head
 *                dims other than 128, for PISA_STATS_GENERIC (formed when given)
 *   head_dim     128 or any multiple of 8 up to 256, in every mode: _C.block_stats_hyd
 *                takes 0 < D <= 256 (pisa_kernels.cu:603), pisa_prepare_triton any
 *                width up to 256; other widths return PISA_ERR_UNSUPPORTED
 * H_sum and h_norm are reduced deterministically (no floating-point atomics).
 */
PISA_HIP_EXPORT int pisa_hip_block_stats(int32_t dtype, int32_t out_dtype, int32_t batch, int32_t heads,
                         int32_t tokens, int32_t head_dim, pisa_view q, pisa_view k, pisa_view v,
                         pisa_token_grid grid, int32_t stats_mode,
                         void* q_centroids, float* k_centroids, void* v_means,
                         float* h_sum, float* h_norm,
                         void* workspace, int64_t workspace_bytes, void* stream);

/* ---- subsystem 2: routing score + per-query-block top-k ----------------- */

/*
 * r[bh,i,j] = scale * dot(qc[bh,i], kc[bh,j]) (+ ln(h_norm[bh,j] + 1e-5) when
 * h_norm != NULL); r[..., sink] = +inf; selects the exact_blocks largest per
 * row with ties to the lowest index and writes them ascending.  round_bf16=1
 * rounds both centroids to bf16 before the fp32 dot (HYD,
 * __init__.py:255-259).  Replaces the bmm/topk/sort sequence of
 * __init__.py:258-264 and generic_pisa.py:303-315.
 *   qc, kc      float32 [BH, N, D]
 *   indices     int32   [BH, N, exact_blocks]
 *   scores      nullable float32 [BH, N, N]
 */
PISA_HIP_EXPORT int pisa_hip_route_topk(int32_t batch_heads, int32_t blocks, int32_t head_dim,
                        const float* qc, const float* kc, const float* h_norm,
                        int32_t round_bf16, float scale, int32_t sink_block, int32_t exact_blocks,
                        int32_t* indices, float* scores, void* stream);

/* ---- spatial layout helpers --------------------------------------------- */

/* Raster [B,H,T,D] views -> block-major [B*H, T, D] contiguous.
 * Replaces _C.pack_spatial_qkv (bindings.cpp:48-53, pisa_kernels.cu:638-676). */
PISA_HIP_EXPORT int pisa_hip_pack_spatial_qkv(int32_t dtype, int32_t batch, int32_t heads, int32_t tokens,
                              int32_t head_dim, pisa_view q, pisa_view k, pisa_view v,
                              pisa_token_grid grid, void* packed_q, void* packed_k,
                              void* packed_v, void* stream);

/* Block-major [B*H, T, D] -> raster [B, T, H*D].
 * Replaces _C.unpack_spatial_output (bindings.cpp:54-59, pisa_kernels.cu:679-707). */
PISA_HIP_EXPORT int pisa_hip_unpack_spatial_output(int32_t dtype, int32_t batch, int32_t heads, int32_t tokens,
                                   int32_t head_dim, const void* packed, pisa_token_grid grid,
                                   void* raster, void* stream);

/* out = bf16(O_e*exp(L_e-L) + (O_a + C)*exp(L_a-L)), L = logaddexp(L_e, L_a),
 * stored raster [B, T, H*D].  Replaces _C.fuse_spatial_epilogue
 * (bindings.cpp:60-69, pisa_kernels.cu:710-773). */
PISA_HIP_EXPORT int pisa_hip_fuse_spatial_epilogue(int32_t dtype, int32_t batch, int32_t heads, int32_t tokens,
                                   int32_t head_dim, const void* exact_output,
                                   const float* exact_lse, const void* approximate_output,
                                   const float* approximate_lse, const float* correction,
                                   pisa_token_grid grid, void* out, void* stream);

/* ---- exact attention ----------------------------------------------------- */

PISA_HIP_EXPORT int64_t attn_hip_dense_workspace_bytes(int32_t batch, int32_t heads, int32_t kv_tokens,
                                       int32_t head_dim);

/*
 * Exact non-causal softmax attention, online softmax in fp32 on bf16/fp16
 * MFMA.  q/out have q_tokens rows, k/v kv_tokens rows (cross attention
 * allowed); any strides (unit head_dim stride).  head_dim a multiple of 8
 * up to 256 (the reference's Triton kernel takes 64 and 128).
 * Replaces full_attention_triton_bh (triton_kernel.py:113-197) and the dense
 * SDPA fallbacks of __init__.py:251-252.
 */
PISA_HIP_EXPORT int attn_hip_dense_forward(int32_t dtype, int32_t batch, int32_t heads, int32_t q_tokens,
                           int32_t kv_tokens, int32_t head_dim, pisa_view q, pisa_view k,
                           pisa_view v, pisa_view out, float scale,
                           void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Fixed block-diagonal attention: each block of block_size tokens attends
 * only to itself (causal optional).  dtype bf16/fp16/fp32, head_dim 32, 64
 * or 128, block_size 64.  Replaces fixed_block_attention_triton_bh
 * (triton_kernel.py:53-100,200-244); semantics of fixed_block_attention_ref
 * (reference.py:159-200).
 */
PISA_HIP_EXPORT int attn_hip_fixed_block_forward(int32_t dtype, int32_t batch, int32_t heads, int32_t tokens,
                                 int32_t head_dim, int32_t block_size, pisa_view q, pisa_view k,
                                 pisa_view v, pisa_view out, float scale, int32_t causal,
                                 void* stream);

/*
 * attn_hip_fixed_block_forward with an attention mask (the masked calls the
 * reference sends to its eager block loop, dispatch.py:50-79 ->
 * fixed_block_attention_ref, reference.py:186-195): causal masking first,
 * then the bool mask (-inf where false) or the additive mask; a row whose
 * keys are all masked gives NaN, as torch.softmax does.
 */
PISA_HIP_EXPORT int attn_hip_fixed_block_forward_masked(int32_t dtype, int32_t batch, int32_t heads, int32_t tokens,
                                        int32_t head_dim, int32_t block_size, pisa_view q, pisa_view k,
                                        pisa_view v, pisa_view out, float scale, int32_t causal,
                                        pisa_mask mask, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PISA_HIP_H */
