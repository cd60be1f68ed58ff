// HYD routing scores and per-query-block top-k selection.
//
// One 256-thread workgroup owns 8 routing rows (query blocks i) of one
// (batch, head): each wave scores 2 rows against every key block j.  Lane l
// holds the candidates j = l, l+64, ... of both rows, so one key-centroid
// value read from LDS feeds 2 fused multiply-adds.  The key centroids are
// staged in LDS transposed ([d][j]) from the row-major [N][D] table with
// coalesced loads: when the routing inputs are bf16-rounded (HYD) and the
// table fits, all of it at once as bf16 pairs (one load phase); otherwise 16
// dimensions at a time in fp32, the next slice loaded while the current one
// is consumed.  Scores are fp32 dot products accumulated in dimension order
// (inputs rounded to bf16 first for HYD), times the scale, plus the HYD bias
// ln(h_norm + 1e-5) and the sink override (+inf).
//
// With head dim 128 the same launch also carries the H_sum reduction
// (reduce_h_tile): workgroups past the routing ones each sum two 32x32 tiles,
// running beside the latency-bound routing workgroups instead of in a launch
// of their own.
//
// Selection per row is a radix select on a total order of fp32 (NaN largest,
// -0 == +0): 32 ballot rounds find the k-th largest key T; keys above T are
// selected, and keys equal to T are taken in ascending block order until k
// are chosen - i.e. the k largest scores with ties to the lowest index,
// independent of scheduling, so the selection is reproducible bit for bit.
// Indices are written in ascending order, with the selection bit mask the
// attention tail uses.
//
// Semantics: native/rdna35_pisa_ck/rdna35_pisa_ck/__init__.py:258-269 (HYD:
// bf16 centroids, fp32 products, + ln(h_norm + 1e-5), sink = +inf, topk then
// ascending sort) and generic_pisa.py:303-317 (fp32 centroids, no bias).
#include "kernels.hpp"

namespace pisa {

constexpr int kRouteWaves = 4;
constexpr int kRouteRows = 2;                    // rows per wave
constexpr int kRouteGroup = kRouteWaves * kRouteRows;
constexpr int kRouteDims = 16;                   // dims staged per pass (sliced path)
constexpr size_t kRouteWholeLds = 64 * 1024;     // largest whole bf16-pair table staged at once

__device__ __forceinline__ uint32_t order_key(float x) {
    uint32_t b = __float_as_uint(x);
    if (x != x) return 0xFFFFFFFFu;       // NaN above +inf
    if (b == 0x80000000u) b = 0u;         // -0 == +0
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float round_bf16(float x) { return static_cast<float>(static_cast<bf16_t>(x)); }
__device__ __forceinline__ uint32_t bf16_bits(float x) {
    return __builtin_bit_cast(uint16_t, static_cast<bf16_t>(x));
}

// WHOLE: bf16-pair table of all D dims staged once (requires round_bf16, even
// D and the table size check of the launcher); otherwise 16-dim fp32 slices.
// T is the dtype of the H_sum copy written by the fused reduction.
template <int PL, bool WHOLE, typename T>  // candidates per lane: N <= 64 * PL
__global__ __launch_bounds__(64 * kRouteWaves) void route_topk_kernel(RouteArgs a, ReduceArgs r, int fuse_reduce) {
    // Dynamic LDS: the query rows of the workgroup ([wave][row][D] fp32), then
    // the staged key centroids (row stride `stride` words).
    extern __shared__ __attribute__((aligned(16))) float route_lds[];
    __shared__ float red_tile[32][33];
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int N = a.blocks;
    const int D = a.head_dim;
    const int groups = (N + kRouteGroup - 1) / kRouteGroup;
    const int route_wgs = (a.rows / N) * groups;
    if ((int)blockIdx.x >= route_wgs) {
        // H_sum reduction workgroups (fuse_reduce): two 32x32 tiles each
        const int id = blockIdx.x - route_wgs;
        const int rbh = id >> 3;
        reduce_h_tile<T>(r, rbh, 2 * (id & 7), red_tile, t);
        reduce_h_tile<T>(r, rbh, 2 * (id & 7) + 1, red_tile, t);
        if ((id & 7) == 0) zero_centroid_pad<T>(r, rbh, t);
        return;
    }
    const int bh = blockIdx.x / groups;
    const int g = blockIdx.x - bh * groups;
    const int i0 = g * kRouteGroup + wave * kRouteRows;
    float* qrows = route_lds + wave * kRouteRows * D;  // this wave's rows
    float* kt = route_lds + kRouteWaves * kRouteRows * D;
    // odd word stride: the transposed staging stores of consecutive threads
    // (2 rows apart) spread over 16 banks
    const int stride = WHOLE ? (N | 1) : N + 4;

    // query centroids of this wave's rows (rows past N mirror row N-1)
#pragma unroll
    for (int rr = 0; rr < kRouteRows; ++rr) {
        const float* q = a.qc + ((int64_t)bh * N + min(i0 + rr, N - 1)) * D;
        for (int d = lane; d < D; d += 64) qrows[rr * D + d] = a.round_bf16 ? round_bf16(q[d]) : q[d];
    }

    float acc[kRouteRows][PL];
#pragma unroll
    for (int rr = 0; rr < kRouteRows; ++rr)
#pragma unroll
        for (int u = 0; u < PL; ++u) acc[rr][u] = 0.0f;
    const float* kbase = a.kc + (int64_t)bh * N * D;

    if constexpr (WHOLE) {
        // word (dp, j) = bf16(kc[j][2dp]) | bf16(kc[j][2dp+1]) << 16; thread
        // piece id covers key j = id / (D/4), dims 4 * (id % (D/4)) .. +3;
        // loads are issued in batches of 24 per thread (one batch at C4)
        uint32_t* kw = reinterpret_cast<uint32_t*>(kt);
        const int per_row = D / 4;
        const int pieces = N * per_row;
        constexpr int kBatch = 24;
        for (int id0 = 0; id0 < pieces; id0 += kBatch * 64 * kRouteWaves) {
            f32x4 buf[kBatch];
#pragma unroll
            for (int s = 0; s < kBatch; ++s) {
                const int id = id0 + t + s * 64 * kRouteWaves;
                f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
                if (id < pieces) v = *reinterpret_cast<const f32x4*>(kbase + (int64_t)id * 4);
                buf[s] = v;
            }
#pragma unroll
            for (int s = 0; s < kBatch; ++s) {
                const int id = id0 + t + s * 64 * kRouteWaves;
                if (id < pieces) {
                    const int j = id / per_row;
                    const int dp = 2 * (id - j * per_row);
                    kw[dp * stride + j] = bf16_bits(buf[s][0]) | (bf16_bits(buf[s][1]) << 16);
                    kw[(dp + 1) * stride + j] = bf16_bits(buf[s][2]) | (bf16_bits(buf[s][3]) << 16);
                }
            }
        }
        __syncthreads();
        for (int d = 0; d < D; d += 4) {
            f32x4 qv[kRouteRows];
#pragma unroll
            for (int rr = 0; rr < kRouteRows; ++rr) qv[rr] = *reinterpret_cast<const f32x4*>(&qrows[rr * D + d]);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                float k0[PL], k1[PL];
#pragma unroll
                for (int u = 0; u < PL; ++u) {
                    const uint32_t w = kw[(d / 2 + h) * stride + min(lane + 64 * u, N - 1)];
                    k0[u] = __uint_as_float(w << 16);
                    k1[u] = __uint_as_float(w & 0xFFFF0000u);
                }
#pragma unroll
                for (int rr = 0; rr < kRouteRows; ++rr)
#pragma unroll
                    for (int u = 0; u < PL; ++u) {
                        acc[rr][u] = fmaf(qv[rr][2 * h], k0[u], acc[rr][u]);
                        acc[rr][u] = fmaf(qv[rr][2 * h + 1], k1[u], acc[rr][u]);
                    }
            }
        }
    } else {
        // Each thread stages up to kStage float4 pieces (key j, 4 dims) per
        // slice; the pieces of slice c+1 are loaded while slice c is consumed.
        constexpr int kStage = PL * 64 * (kRouteDims / 4) / (64 * kRouteWaves);  // N <= 64 * PL
        const int pieces = N * (kRouteDims / 4);
        auto fetch = [&](int d0, f32x4 (&buf)[kStage]) {
#pragma unroll
            for (int s = 0; s < kStage; ++s) {
                const int id = t + s * 64 * kRouteWaves;
                const int j = id >> 2;
                const int dq = (id & 3) * 4;
                f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
                if (id < pieces && d0 + dq < D) v = *reinterpret_cast<const f32x4*>(kbase + (int64_t)j * D + d0 + dq);
                buf[s] = v;
            }
        };
        f32x4 buf[kStage];
        fetch(0, buf);
        for (int d0 = 0; d0 < D; d0 += kRouteDims) {
            __syncthreads();  // previous slice fully consumed (and qrows written)
#pragma unroll
            for (int s = 0; s < kStage; ++s) {
                const int id = t + s * 64 * kRouteWaves;
                if (id < pieces) {
                    const int j = id >> 2;
                    const int dq = (id & 3) * 4;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        kt[(dq + e) * stride + j] = a.round_bf16 ? round_bf16(buf[s][e]) : buf[s][e];
                }
            }
            __syncthreads();
            if (d0 + kRouteDims < D) fetch(d0 + kRouteDims, buf);
            const int dn = min(kRouteDims, D - d0);
            for (int d = 0; d < dn; d += 4) {
                f32x4 qv[kRouteRows];
#pragma unroll
                for (int rr = 0; rr < kRouteRows; ++rr)
                    qv[rr] = *reinterpret_cast<const f32x4*>(&qrows[rr * D + d0 + d]);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float kv[PL];
#pragma unroll
                    for (int u = 0; u < PL; ++u) kv[u] = kt[(d + e) * stride + min(lane + 64 * u, N - 1)];
#pragma unroll
                    for (int rr = 0; rr < kRouteRows; ++rr)
#pragma unroll
                        for (int u = 0; u < PL; ++u) acc[rr][u] = fmaf(qv[rr][e], kv[u], acc[rr][u]);
                }
            }
        }
    }

    // ---- scores: scale, HYD bias, sink
    const int sink_j = a.sink == PISA_NO_SINK ? -1 : (a.sink < 0 ? N + a.sink : a.sink);
    float bias[PL];
#pragma unroll
    for (int u = 0; u < PL; ++u) {
        const int j = lane + 64 * u;
        bias[u] = (a.hnorm && j < N) ? logf(a.hnorm[(int64_t)bh * N + j] + 1e-5f) : 0.0f;
    }
    const uint64_t lt_mask = (1ull << lane) - 1ull;
    uint32_t key[kRouteRows][PL];
#pragma unroll
    for (int rr = 0; rr < kRouteRows; ++rr) {
        const int i = i0 + rr;
#pragma unroll
        for (int u = 0; u < PL; ++u) {
            const int j = lane + 64 * u;
            float sc = acc[rr][u] * a.scale + bias[u];
            if (j == sink_j) sc = __builtin_inff();
            key[rr][u] = j < N ? order_key(sc) : 0u;  // padding below every real key
            if (a.scores && j < N && i < N) a.scores[((int64_t)bh * N + i) * N + j] = sc;
        }
    }
    const int k = a.k;
    if (k <= 0) {  // nothing selected: the tail keeps every block
#pragma unroll
        for (int rr = 0; rr < kRouteRows; ++rr) {
            const int i = i0 + rr;
            if (a.selmask && i < N)
                for (int w = lane; w < a.mask_words; w += 64) a.selmask[((int64_t)bh * N + i) * a.mask_words + w] = 0u;
        }
        return;
    }
    // k-th largest key of each row: largest T with #{key >= T} >= k; the rows'
    // bit-by-bit searches are independent and run interleaved (rows past N
    // mirror row N-1 and are not stored)
    uint32_t T_k[kRouteRows];
#pragma unroll
    for (int rr = 0; rr < kRouteRows; ++rr) T_k[rr] = 0u;
    for (int b = 31; b >= 0; --b) {
#pragma unroll
        for (int rr = 0; rr < kRouteRows; ++rr) {
            const uint32_t cand = T_k[rr] | (1u << b);
            int cnt = 0;
#pragma unroll
            for (int u = 0; u < PL; ++u) cnt += __popcll(__ballot(key[rr][u] >= cand));
            if (cnt >= k) T_k[rr] = cand;
        }
    }
#pragma unroll
    for (int rr = 0; rr < kRouteRows; ++rr) {
        const int i = i0 + rr;
        if (i >= N) break;  // wave-uniform
        int gt = 0;
#pragma unroll
        for (int u = 0; u < PL; ++u) gt += __popcll(__ballot(key[rr][u] > T_k[rr]));
        int ties_left = k - gt;  // keys equal to T_k still to take, lowest index first
        int32_t* out_idx = a.idx + ((int64_t)bh * N + i) * k;
        uint32_t* mask = a.selmask ? a.selmask + ((int64_t)bh * N + i) * a.mask_words : nullptr;
        int before = 0;
#pragma unroll
        for (int u = 0; u < PL; ++u) {
            const uint64_t tie = __ballot(key[rr][u] == T_k[rr]);
            const int tie_rank = __popcll(tie & lt_mask);
            const bool sel = key[rr][u] > T_k[rr] || (key[rr][u] == T_k[rr] && tie_rank < ties_left);
            ties_left -= min(ties_left, __popcll(tie));
            const uint64_t bal = __ballot(sel);
            if (sel) out_idx[before + __popcll(bal & lt_mask)] = lane + 64 * u;
            if (mask && lane == 0) {
                if (2 * u < a.mask_words) mask[2 * u] = static_cast<uint32_t>(bal);
                if (2 * u + 1 < a.mask_words) mask[2 * u + 1] = static_cast<uint32_t>(bal >> 32);
            }
            before += __popcll(bal);
        }
    }
}

// Whole-table staging: bf16-rounded inputs, even D, and the pair table of
// D/2 rows x (N | 1) words within kRouteWholeLds.
static bool route_whole(const RouteArgs& a) {
    return a.round_bf16 && a.head_dim % 2 == 0 &&
           (size_t)(a.head_dim / 2) * (size_t)(a.blocks | 1) * 4 <= kRouteWholeLds;
}

template <int PL, typename T>
static void launch_route_pl(const RouteArgs& a, const ReduceArgs& r, int fuse, hipStream_t stream) {
    const int groups = (a.blocks + kRouteGroup - 1) / kRouteGroup;
    const int bh_count = a.rows / a.blocks;
    const dim3 grid(bh_count * groups + (fuse ? bh_count * 8 : 0));  // routing, then reduction workgroups
    const size_t q_lds = (size_t)kRouteGroup * a.head_dim * sizeof(float);
    if (route_whole(a)) {
        const size_t lds = q_lds + (size_t)(a.head_dim / 2) * (size_t)(a.blocks | 1) * 4;
        hipLaunchKernelGGL((route_topk_kernel<PL, true, T>), grid, dim3(64 * kRouteWaves), lds, stream, a, r, fuse);
    } else {
        const size_t lds = q_lds + (size_t)kRouteDims * (a.blocks + 4) * sizeof(float);
        hipLaunchKernelGGL((route_topk_kernel<PL, false, T>), grid, dim3(64 * kRouteWaves), lds, stream, a, r, fuse);
    }
}

template <typename T>
static void launch_route_t(const RouteArgs& a, const ReduceArgs& r, int fuse, hipStream_t stream) {
    const int pl = (a.blocks + 63) / 64;
    if (pl <= 1) launch_route_pl<1, T>(a, r, fuse, stream);
    else if (pl <= 2) launch_route_pl<2, T>(a, r, fuse, stream);
    else if (pl <= 3) launch_route_pl<3, T>(a, r, fuse, stream);
    else if (pl <= 4) launch_route_pl<4, T>(a, r, fuse, stream);
    else if (pl <= 8) launch_route_pl<8, T>(a, r, fuse, stream);
    else launch_route_pl<16, T>(a, r, fuse, stream);
}

int launch_route(const RouteArgs& a, hipStream_t stream) {
    ReduceArgs none{};
    launch_route_t<bf16_t>(a, none, 0, stream);
    return pisa_host::check_launch("route_topk_kernel");
}

int launch_route_reduce(int dtype, const RouteArgs& a, const ReduceArgs& r, hipStream_t stream) {
    if (a.head_dim != 128) return pisa_host::fail(PISA_ERR_UNSUPPORTED, "fused H_sum reduction needs head dim 128");
    if (dtype == PISA_DTYPE_BF16) launch_route_t<bf16_t>(a, r, 1, stream);
    else launch_route_t<f16_t>(a, r, 1, stream);
    return pisa_host::check_launch("route_topk_kernel");
}

}  // namespace pisa
