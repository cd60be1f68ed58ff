// HYD routing scores and per-query-block top-k selection.
//
// One 256-thread workgroup owns 16 routing rows (query blocks i) of one
// (batch, head): each wave scores 4 rows against every key block j.  Lane l
// holds the candidates j = l, l+64, ... of all 4 rows, so one key-centroid
// value read from LDS feeds 4 fused multiply-adds.  The key centroids are
// staged through LDS 16 dimensions at a time, transposed ([d][j]), from the
// row-major [N][D] table with coalesced loads.  Scores are fp32 dot products
// (inputs rounded to bf16 first for HYD), times the scale, plus the HYD bias
// ln(h_norm + 1e-5) and the sink override (+inf).
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
constexpr int kRouteRows = 4;                    // rows per wave
constexpr int kRouteGroup = kRouteWaves * kRouteRows;
constexpr int kRouteDims = 16;                   // dims staged per pass

__device__ __forceinline__ uint32_t order_key(float x) {
    uint32_t b = __float_as_uint(x);
    if (x != x) return 0xFFFFFFFFu;       // NaN above +inf
    if (b == 0x80000000u) b = 0u;         // -0 == +0
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float round_bf16(float x) { return static_cast<float>(static_cast<bf16_t>(x)); }

template <int PL>  // candidates per lane: N <= 64 * PL
__global__ __launch_bounds__(64 * kRouteWaves) void route_topk_kernel(RouteArgs a) {
    // kt: key centroids of the current 16-dim chunk, transposed ([d][j], row
    // stride N + 4 floats); sized at launch from N.
    extern __shared__ __attribute__((aligned(16))) float route_lds[];
    __shared__ __attribute__((aligned(16))) float qrows[kRouteWaves][kRouteRows][256];
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int N = a.blocks;
    const int D = a.head_dim;
    const int stride = N + 4;
    float* kt = route_lds;
    const int groups = (N + kRouteGroup - 1) / kRouteGroup;
    const int bh = blockIdx.x / groups;
    const int i0 = (blockIdx.x - bh * groups) * kRouteGroup + wave * kRouteRows;

    // query centroids of this wave's rows (rows past N mirror row N-1)
#pragma unroll
    for (int r = 0; r < kRouteRows; ++r) {
        const float* q = a.qc + ((int64_t)bh * N + min(i0 + r, N - 1)) * D;
        for (int d = lane; d < D; d += 64) qrows[wave][r][d] = a.round_bf16 ? round_bf16(q[d]) : q[d];
    }

    float acc[kRouteRows][PL];
#pragma unroll
    for (int r = 0; r < kRouteRows; ++r)
#pragma unroll
        for (int u = 0; u < PL; ++u) acc[r][u] = 0.0f;

    // Each thread stages up to kStage float4 pieces (key j, 4 dims) per chunk;
    // the pieces of chunk c+1 are loaded while chunk c is consumed.
    constexpr int kStage = PL * 64 * (kRouteDims / 4) / (64 * kRouteWaves);  // N <= 64 * PL
    const int pieces = N * (kRouteDims / 4);
    const float* kbase = a.kc + (int64_t)bh * N * D;
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
        __syncthreads();  // previous chunk fully consumed (and qrows written)
#pragma unroll
        for (int s = 0; s < kStage; ++s) {
            const int id = t + s * 64 * kRouteWaves;
            if (id < pieces) {
                const int j = id >> 2;
                const int dq = (id & 3) * 4;
#pragma unroll
                for (int e = 0; e < 4; ++e) kt[(dq + e) * stride + j] = a.round_bf16 ? round_bf16(buf[s][e]) : buf[s][e];
            }
        }
        __syncthreads();
        if (d0 + kRouteDims < D) fetch(d0 + kRouteDims, buf);
        const int dn = min(kRouteDims, D - d0);
        for (int d = 0; d < dn; d += 4) {
            f32x4 qv[kRouteRows];
#pragma unroll
            for (int r = 0; r < kRouteRows; ++r) qv[r] = *reinterpret_cast<const f32x4*>(&qrows[wave][r][d0 + d]);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float kv[PL];
#pragma unroll
                for (int u = 0; u < PL; ++u) kv[u] = kt[(d + e) * stride + min(lane + 64 * u, N - 1)];
#pragma unroll
                for (int r = 0; r < kRouteRows; ++r)
#pragma unroll
                    for (int u = 0; u < PL; ++u) acc[r][u] = fmaf(qv[r][e], kv[u], acc[r][u]);
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
#pragma unroll
    for (int r = 0; r < kRouteRows; ++r) {
        const int i = i0 + r;
        if (i >= N) break;  // wave-uniform; no barrier below
        uint32_t key[PL];
#pragma unroll
        for (int u = 0; u < PL; ++u) {
            const int j = lane + 64 * u;
            float sc = acc[r][u] * a.scale + bias[u];
            if (j == sink_j) sc = __builtin_inff();
            key[u] = j < N ? order_key(sc) : 0u;  // padding below every real key
            if (a.scores && j < N) a.scores[((int64_t)bh * N + i) * N + j] = sc;
        }
        const int k = a.k;
        uint32_t* mask = a.selmask ? a.selmask + ((int64_t)bh * N + i) * a.mask_words : nullptr;
        if (k <= 0) {  // nothing selected: the tail keeps every block
            if (mask)
                for (int w = lane; w < a.mask_words; w += 64) mask[w] = 0u;
            continue;
        }
        // k-th largest key: largest T with #{key >= T} >= k
        uint32_t T = 0u;
        for (int b = 31; b >= 0; --b) {
            const uint32_t cand = T | (1u << b);
            int cnt = 0;
#pragma unroll
            for (int u = 0; u < PL; ++u) cnt += __popcll(__ballot(key[u] >= cand));
            if (cnt >= k) T = cand;
        }
        int gt = 0;
#pragma unroll
        for (int u = 0; u < PL; ++u) gt += __popcll(__ballot(key[u] > T));
        int ties_left = k - gt;  // keys equal to T still to take, lowest index first
        int32_t* out_idx = a.idx + ((int64_t)bh * N + i) * k;
        int before = 0;
#pragma unroll
        for (int u = 0; u < PL; ++u) {
            const uint64_t tie = __ballot(key[u] == T);
            const int tie_rank = __popcll(tie & lt_mask);
            const bool sel = key[u] > T || (key[u] == T && tie_rank < ties_left);
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

template <int PL>
static void launch_route_pl(const RouteArgs& a, hipStream_t stream) {
    const int groups = (a.blocks + kRouteGroup - 1) / kRouteGroup;
    const int bh_count = a.rows / a.blocks;
    const size_t lds = (size_t)kRouteDims * (a.blocks + 4) * sizeof(float);
    hipLaunchKernelGGL((route_topk_kernel<PL>), dim3(bh_count * groups), dim3(64 * kRouteWaves), lds, stream, a);
}

int launch_route(const RouteArgs& a, hipStream_t stream) {
    const int pl = (a.blocks + 63) / 64;
    if (pl <= 1) launch_route_pl<1>(a, stream);
    else if (pl <= 2) launch_route_pl<2>(a, stream);
    else if (pl <= 3) launch_route_pl<3>(a, stream);
    else if (pl <= 4) launch_route_pl<4>(a, stream);
    else if (pl <= 8) launch_route_pl<8>(a, stream);
    else launch_route_pl<16>(a, stream);
    return pisa_host::check_launch("route_topk_kernel");
}

}  // namespace pisa
