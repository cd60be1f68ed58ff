// Subsystem 2: HYD routing scores and per-query-block top-k selection.
//
// One wavefront owns one routing row (bh, query block i).  Lane l scores the
// candidate key blocks j = l, l+64, ... with a sequential fp32 dot product
// (order d = 0..D-1, fused multiply-add), adds the HYD bias ln(h_norm + 1e-5)
// and the sink override, stages the row in LDS and ranks every candidate
// against the whole row:
//     rank(j) = #{j' : key(j') > key(j)} + #{j' < j : key(j') == key(j)}
// where key() is a total order on fp32 (NaN largest, -0 == +0).  Candidates
// with rank < k are selected - the k largest scores, ties to the lowest index
// - and written in ascending index order using wave ballots.  The result does
// not depend on scheduling, so the selection is reproducible bit for bit.
//
// Semantics: native/rdna35_pisa_ck/rdna35_pisa_ck/__init__.py:258-269 (HYD:
// bf16 centroids, fp32 products, + ln(h_norm + 1e-5), sink = +inf, topk then
// ascending sort) and generic_pisa.py:303-317 (fp32 centroids, no bias).
#include "kernels.hpp"

namespace pisa {

constexpr int kRouteWaves = 4;


__device__ __forceinline__ uint32_t order_key(float x) {
    uint32_t b = __float_as_uint(x);
    if (x != x) return 0xFFFFFFFFu;       // NaN above +inf
    if (b == 0x80000000u) b = 0u;         // -0 == +0
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float round_bf16(float x) { return static_cast<float>(static_cast<bf16_t>(x)); }

__global__ __launch_bounds__(64 * kRouteWaves) void route_topk_kernel(RouteArgs a) {
    __shared__ float row_scores[kRouteWaves][kMaxRouteBlocks];
    __shared__ float qrow[kRouteWaves][256];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int row_raw = blockIdx.x * kRouteWaves + wave;
    const bool active = row_raw < a.rows;
    const int row = active ? row_raw : a.rows - 1;  // inactive waves mirror a valid row, write nothing
    const int bh = row / a.blocks;
    const int i = row - bh * a.blocks;
    const int D = a.head_dim;
    const int N = a.blocks;

    const float* q = a.qc + ((int64_t)bh * N + i) * D;
    for (int d = lane; d < D; d += 64) {
        const float x = q[d];
        qrow[wave][d] = a.round_bf16 ? round_bf16(x) : x;
    }
    __syncthreads();

    float* sc = row_scores[wave];
    const float* kbase = a.kc + (int64_t)bh * N * D;
    for (int j = lane; j < N; j += 64) {
        const float* kr = kbase + (int64_t)j * D;
        float acc = 0.0f;
        for (int d = 0; d < D; d += 4) {
            const f32x4 kv = *reinterpret_cast<const f32x4*>(kr + d);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float kx = a.round_bf16 ? round_bf16(kv[e]) : kv[e];
                acc = fmaf(qrow[wave][d + e], kx, acc);
            }
        }
        float r = acc * a.scale;
        if (a.hnorm) r += logf(a.hnorm[(int64_t)bh * N + j] + 1e-5f);
        sc[j] = r;
    }
    __syncthreads();
    if (a.sink != PISA_NO_SINK && lane == 0) sc[a.sink < 0 ? N + a.sink : a.sink] = __builtin_inff();
    __syncthreads();
    if (!active) return;  // every barrier of the kernel is above this line

    if (a.scores) {
        float* out = a.scores + ((int64_t)bh * N + i) * N;
        for (int j = lane; j < N; j += 64) out[j] = sc[j];
    }

    // ---- rank every candidate held by this lane against the whole row
    constexpr int kMaxPerLane = kMaxRouteBlocks / 64;
    uint32_t mykey[kMaxPerLane];
    int rank[kMaxPerLane];
    const int per_lane = (N + 63) >> 6;
#pragma unroll
    for (int u = 0; u < kMaxPerLane; ++u) {
        const int j = lane + 64 * u;
        mykey[u] = (u < per_lane && j < N) ? order_key(sc[j]) : 0u;
        rank[u] = 0;
    }
    for (int jp = 0; jp < N; ++jp) {
        const uint32_t kp = order_key(sc[jp]);
#pragma unroll
        for (int u = 0; u < kMaxPerLane; ++u) {
            if (u < per_lane) {
                const int j = lane + 64 * u;
                rank[u] += (kp > mykey[u]) || (kp == mykey[u] && jp < j);
            }
        }
    }

    // ---- ascending output positions from ballots
    int32_t* out_idx = a.idx + ((int64_t)bh * N + i) * a.k;
    int before = 0;
#pragma unroll
    for (int u = 0; u < kMaxPerLane; ++u) {
        if (u < per_lane) {
            const int j = lane + 64 * u;
            const bool sel = j < N && rank[u] < a.k;
            const uint64_t bal = __ballot(sel);
            if (sel) {
                const int pos = before + __popcll(bal & ((1ull << lane) - 1ull));
                out_idx[pos] = j;
            }
            if (a.selmask && lane == 0) {
                uint32_t* m = a.selmask + ((int64_t)bh * N + i) * a.mask_words;
                if (2 * u < a.mask_words) m[2 * u] = static_cast<uint32_t>(bal);
                if (2 * u + 1 < a.mask_words) m[2 * u + 1] = static_cast<uint32_t>(bal >> 32);
            }
            before += __popcll(bal);
        }
    }
}

int launch_route(const RouteArgs& a, hipStream_t stream) {
    const int wgs = (a.rows + kRouteWaves - 1) / kRouteWaves;
    hipLaunchKernelGGL(route_topk_kernel, dim3(wgs), dim3(64 * kRouteWaves), 0, stream, a);
    return pisa_host::check_launch("route_topk_kernel");
}

}  // namespace pisa
