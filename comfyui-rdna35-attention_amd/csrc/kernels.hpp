// Argument blocks and launchers of the gfx950 kernels (one translation unit
// per subsystem; api.hip validates arguments and calls the launchers).
#pragma once

#include "common.hpp"

namespace pisa {

constexpr int kMaxRouteBlocks = 1024;  // routing row length held in LDS

struct StatsArgs {
    View q, k, v;
    TokenMap map;
    int tokens, blocks, chunk_blocks, chunks;
    // API outputs
    void* qc_out;   // [BH][N][D] (f32 when qc_f32)
    int qc_f32;
    float* kc_out;  // [BH][N][D] (nullable at head dim 128)
    void* vm_out;   // [BH][N][D] (f32 when vm_f32; nullable)
    int vm_f32;
    int vm_sums;    // nonzero: vm_out (f32) receives the per-block value sums instead of the means
    float* hnorm_out;  // [BH][N] (nullable)
    float* hpart;      // [BH][chunks][D][D] (HYD / GENERIC)
    // attention operands (nullable)
    float* qc_route;   // [BH][N][D] f32 means for routing
    int qc_route_round;  // nonzero: the routing q_bar is the dtype-rounded mean (generic routing on HYD statistics)
    void* kp_blocks;   // [BH][N] packed key blocks (kfrag_elem order)
    void* vp_blocks;   // [BH][N] packed value blocks (vfrag_elem order)
    void* kbar_pad;    // [BH][npad/64] packed key chunks of dtype k_bar
    void* vbar_t_pad;  // [BH][npad/64] packed value chunks of dtype v_bar
    int npad;
    int head_dim;      // real head dim D (outputs are [.][.][D]; packed tables use the padded width)
};

// Sums the per-chunk partials in chunk order; writes H_sum (fp32), the
// transposed dtype copy used by the first-order correction, and zeroes the
// padding of the centroid tables.
struct ReduceArgs {
    const float* hpart;
    int chunks;
    float* hsum;       // [BH][hsum_dim][hsum_dim] (nullable): the first hsum_dim rows and columns
    int hsum_dim;      // 0: the reduction's width
    void* ht;          // [BH] packed D x D, element (c, r) = dtype(H_sum[r][c]) (nullable)
    void* kbar_pad;    // nullable
    void* vbar_t_pad;  // nullable
    int blocks, npad;
    // head dims other than 128: per-block tile sums of squares of H_b
    // ([BH][N][tiles], from stats_cov_kernel) and ||H_b||_F out (both nullable)
    const float* normpart;
    float* hnorm;
};

// One 32x32 tile (tile = (D/32) * row tile + column tile) of the H_sum
// reduction of head bh at width D, by 256 threads: the per-chunk partials are
// added in chunk order (the sum does not depend on how the loads are
// batched), H_sum is written in fp32 and its transpose as packed dtype
// fragments (both optional).  `tile_lds` is a 32 x 33 float array; the call
// ends with a barrier, so it can be called again on the same array.  The
// partials are read once, with the non-temporal hint (C4 prepare -0.7 us).
template <typename T, int D = 128>
__device__ inline void reduce_h_tile(const ReduceArgs& a, int bh, int tile, float (*tile_lds)[33], int t) {
    const int tr = tile / (D / 32);  // 32-row tile index
    const int tc = tile % (D / 32);  // 32-col tile index
    const float* src = a.hpart + (int64_t)bh * a.chunks * D * D;
    float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    int64_t off[4];
#pragma unroll
    for (int it = 0; it < 4; ++it) off[it] = (int64_t)(tr * 32 + it * 8 + (t >> 5)) * D + tc * 32 + (t & 31);
    constexpr int kBatch = 8;
    for (int ch0 = 0; ch0 < a.chunks; ch0 += kBatch) {
        float x[kBatch][4];
#pragma unroll
        for (int u = 0; u < kBatch; ++u)
#pragma unroll
            for (int it = 0; it < 4; ++it)
                x[u][it] = __builtin_nontemporal_load(&src[(int64_t)min(ch0 + u, a.chunks - 1) * D * D + off[it]]);  // unconditional
#pragma unroll
        for (int u = 0; u < kBatch; ++u)
#pragma unroll
            for (int it = 0; it < 4; ++it)
                if (ch0 + u < a.chunks) s[it] += x[u][it];
    }
    const int hd = a.hsum_dim > 0 ? a.hsum_dim : D;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int r = tr * 32 + it * 8 + (t >> 5);
        const int c = tc * 32 + (t & 31);
        if (a.hsum && r < hd && c < hd) a.hsum[((int64_t)bh * hd + r) * hd + c] = s[it];
        tile_lds[it * 8 + (t >> 5)][t & 31] = s[it];
    }
    __syncthreads();
    if (a.ht) {
        T* ht = static_cast<T*>(a.ht) + (int64_t)bh * D * D;
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            const int lr = it * 8 + (t >> 5);  // output row = H column
            const int lc = t & 31;
            ht[kfrag_elem(tc * 32 + lr, tr * 32 + lc, D)] = from_f32<T>(tile_lds[lc][lr]);
        }
    }
    __syncthreads();
}

// Zeroes the packed centroids past the last block of head bh (their scores
// are masked to -inf, and a zero value keeps 0 * value finite in the PV
// product); any number of threads, t = thread index, `stride` threads.
template <typename T>
__device__ inline void zero_centroid_pad(const ReduceArgs& a, int bh, int t, int stride = 256) {
    constexpr int D = 128;
    const int pad = a.npad - a.blocks;
    const int64_t head_base = (int64_t)bh * a.npad * D;
    for (int i = t; i < pad * D; i += stride) {
        const int j = a.blocks + i / D;
        const int d = i - (i / D) * D;
        const int64_t base = head_base + (int64_t)(j & ~63) * D;
        if (a.kbar_pad) static_cast<T*>(a.kbar_pad)[base + kfrag_elem(j & 63, d, D)] = T(0.0f);
        if (a.vbar_t_pad) static_cast<T*>(a.vbar_t_pad)[base + vfrag_elem(j & 63, d)] = T(0.0f);
    }
}

struct RouteArgs {
    const float* qc;     // [BH][N][D]
    const float* kc;     // [BH][N][D]
    const float* hnorm;  // [BH][N] or null
    int rows, blocks, head_dim, round_bf16, sink, k;
    float scale;
    int32_t* idx;        // [BH][N][k]
    float* scores;       // [BH][N][N] or null
    uint32_t* selmask;   // [BH][N][mask_words] or null
    int mask_words;
    // HYD at head dim 128 with bf16 inputs: the bf16 means the statistics kernel
    // wrote (q_bar row-major, k_bar as packed 64-centroid chunks), which equal
    // the bf16 rounding of qc / kc; scored on bf16 MFMA when both are set
    const bf16_t* qc_bf16;   // [BH][N][128] or null
    const bf16_t* kc_pack;   // [BH][npad/64] packed chunks or null
    int npad;
};

struct AttnArgs {
    View q;
    OutView o;
    const char* kp;   // [BH][kv_blocks] packed key blocks (kfrag_elem order)
    const char* vp;   // [BH][kv_blocks] packed value blocks (vfrag_elem order)
    TokenMap qmap;
    int q_tokens, kv_tokens, q_blocks, kv_blocks;
    float scale_log2;  // softmax scale * log2(e)
    float inv_scale_log2;  // 1 / scale_log2 (centroid biases in score units)
    // sparse exact chunks
    const int32_t* idx;  // [BH][q_blocks][exact]
    int exact;
    // tail chunks
    const char* kbar;        // [BH][npad/64] packed key chunks (centroids as keys)
    const char* vbar_t;      // [BH][npad/64] packed value chunks
    const uint32_t* selmask; // [BH][q_blocks][mask_words]
    int mask_words, npad, centroids;
    float last_len_log2;     // log2(length of the last block)
    // first-order correction
    const char* ht;          // [BH] packed D x D (kfrag_elem), element (c, r) = H_sum[r][c]
    float corr_scale;        // s / T
    int head_dim;            // real head dim (<= the kernel's padded width)
    // set by the launcher: query blocks of the grid, and blocks per XCD run as
    // two one-tile halves in the last round (0: no split)
    int q_blocks_total, split_r;
};

struct LayoutArgs {
    View in[3];
    char* out[3];
    int ntensors;
    TokenMap map;
    int tokens, head_dim, heads;
};

int launch_stats(int dtype, int mode, const StatsArgs& a, int bh_count, hipStream_t stream);
// H_sum partials at a padded head dim other than 128 (the statistics kernel
// forms them at 128): H_b = (K_b - k_bar_b)^T V_b summed over each chunk of
// chunk_blocks blocks, one wave per (head, chunk, 32x32 tile of H); centred
// keys rounded to the dtype (generic) or kept at fp32 accuracy (hyd).  kmean
// holds the fp32 block means of K that the means kernel wrote
// ([BH][N][head_dim]).
struct CovArgs {
    View k, v;
    TokenMap map;
    int tokens, blocks, head_dim, chunk_blocks, chunks;
    const float* kmean;
    float* hpart;     // [BH][chunks][Dp][Dp]
    float* normpart;  // [BH][N][(Dp/32)^2] tile sums of squares of H_b (nullable)
};
int launch_stats_cov(int dtype, int padded, const CovArgs& a, int bh_count, hipStream_t stream, bool hyd);
// Chunk-order sum of launch_stats_cov's partials into dtype(H_sum)^T packed at
// the padded width (ReduceArgs.ht; hsum optional).
int launch_cov_reduce(int dtype, int padded, const ReduceArgs& a, int bh_count, hipStream_t stream);
int launch_stats_reduce(int dtype, const ReduceArgs& a, int bh_count, hipStream_t stream);
int launch_route(const RouteArgs& a, hipStream_t stream);
// Routing with the H_sum reduction of head dim 128 (stats_reduce_kernel's work,
// `r`) done by the routing workgroups of each head before they score.
int launch_route_reduce(int dtype, const RouteArgs& a, const ReduceArgs& r, hipStream_t stream);
// Block means at padded width `padded` (a.head_dim < 128 or > 128): sum / len,
// or sum * (1/len) for the HYD statistics (`hyd`).
int launch_stats_means(int dtype, int padded, const StatsArgs& a, int bh_count, hipStream_t stream, bool hyd);
// `padded` = padded_head_dim(a.head_dim); dense (sparse = tail = false) or PISA (both true).
int launch_attention(int dtype, int padded, bool sparse, bool tail, const AttnArgs& a, int bh_count,
                     hipStream_t stream);
// Packed key / value blocks of width `padded` (dims >= head_dim and rows >= kv_tokens are zero);
// block j row r is token map(64 j + r).
int launch_kv_pack(int dtype, int padded, int head_dim, const View& k, const View& v, TokenMap map, int kv_tokens,
                   int kv_blocks, int bh_count, char* kp, char* vp, hipStream_t stream);
// Fixed-block attention mask, broadcast to [B][heads][T][T] by element strides.
struct MaskView {
    const char* data;
    int kind;  // PISA_MASK_*
    int heads;
    int64_t sb, sh, sq, sk;
};
int launch_fixed_block(int dtype, int head_dim, const View& q, const View& k, const View& v, const OutView& o,
                       int tokens, int bh_count, float scale, int causal, const MaskView& mask, hipStream_t stream);
int launch_pack(int dtype, const LayoutArgs& a, int bh_count, hipStream_t stream);
int launch_unpack(int dtype, const char* packed, char* out, TokenMap map, int tokens, int head_dim, int heads,
                  int bh_count, hipStream_t stream);
int launch_merge(int dtype, const char* exact, const float* exact_lse, const char* approx, const float* approx_lse,
                 const float* corr, char* out, TokenMap map, int tokens, int head_dim, int heads, int bh_count,
                 hipStream_t stream);

}  // namespace pisa
