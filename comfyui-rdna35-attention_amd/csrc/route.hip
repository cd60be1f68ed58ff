// HYD and centroid routing scores and per-query-block top-k selection.
//
// One 256-thread workgroup owns 16 (or 8) routing rows (query blocks i) of one
// (batch, head).  Scores S[i][j] = q_i . k_j for every key block j are 16 x 16
// tiles of MFMA written to LDS: for HYD with bf16 inputs the bf16 means the
// statistics kernel wrote (which equal the bf16 rounding of the fp32 means) on
// v_mfma_f32_16x16x32_bf16, otherwise the fp32 means on v_mfma_f32_16x16x4_f32
// (rounded to bf16 first for HYD); every product is exact and only the fp32
// summation order is the hardware's.  Then each wave selects 4 (or 2) rows:
// lane l holds the candidates j = l, l+64, ... of a row (scale, HYD bias
// ln(h_norm + 1e-5), sink override +inf).  The launch is a chain of dependent
// loads, products and ballot rounds per workgroup; when 16-row workgroups
// would leave the CUs with fewer than two each, 8-row workgroups (half of
// each score tile unused) halve the selection and store part of that chain.
//
// With head dim 128 the same launch also carries the H_sum reduction
// (reduce_h_tile): workgroups past the routing ones each sum two 32x32 tiles,
// running beside the routing workgroups instead of in a launch of their own.
//
// Selection per row is a radix select on a total order of fp32 (NaN largest,
// -0 == +0): 32 ballot rounds find the k-th largest key T; keys above T are
// selected, and keys equal to T are taken in ascending block order until k
// are chosen - i.e. the k largest scores with ties to the lowest index,
// independent of scheduling, so the selection is reproducible bit for bit.
// A wave's rows are searched together, with no branch between them, until
// every row's prefix has exactly k keys at or above it.  Indices are written in
// ascending order, with the selection bit mask the attention tail uses (lane w
// writing word w).  h_norm is loaded before the scores are formed.
//
// Semantics: native/rdna35_pisa_ck/rdna35_pisa_ck/__init__.py:258-269 (HYD:
// bf16 centroids, fp32 products, + ln(h_norm + 1e-5), sink = +inf, topk then
// ascending sort) and generic_pisa.py:303-317 (fp32 centroids, no bias).
#include "kernels.hpp"

namespace pisa {

constexpr int kRouteWaves = 4;
constexpr int kScoreRows = 16;  // rows of a score tile (rows of the 16x16 MFMA tiles)

__device__ __forceinline__ uint32_t order_key(float x) {
    uint32_t b = __float_as_uint(x);
    if (x != x) return 0xFFFFFFFFu;       // NaN above +inf
    if (b == 0x80000000u) b = 0u;         // -0 == +0
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float round_bf16(float x) { return static_cast<float>(static_cast<bf16_t>(x)); }

// fp32 16x16x4 MFMA: A[m][k] = a of lane (k = lane / 16, m = lane % 16),
// B[k][n] = b of lane (k = lane / 16, n = lane % 16); lane l holds D[4(l/16) + v][l % 16].
__device__ __forceinline__ f32x4 mfma16_f32(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// One 256-thread workgroup owns TILE (16 or 8) routing rows of one head.
// Scores: each wave takes every 4th 16-candidate tile and forms the 16 x 16
// tile S[i][j] = sum_d q_i[d] k_j[d] with fp32 16x16x4 MFMAs (the four lane
// groups take interleaved groups of 4 dims, so each lane loads aligned 16-byte
// pieces of one query row and one key row, the next 16 steps' pieces in
// flight while the current ones are multiplied); products of the
// (bf16-rounded for HYD) fp32 inputs are exact, sums are fp32.  The tile goes
// to LDS (rows past TILE are formed and not used).  Selection: wave w takes
// rows TILE/4 w .. TILE/4 (w+1) - 1 together, lane l reading candidates l,
// l+64, ... of a row from LDS.  T: dtype of the H_sum copy of the fused
// reduction workgroups.
template <int PL, int TILE, typename T>  // candidates per lane in the selection: N <= 64 * PL
__global__ __launch_bounds__(64 * kRouteWaves) void route_topk_kernel(RouteArgs a, ReduceArgs r, int fuse_reduce) {
    static_assert(TILE == 16 || TILE == 8, "routing rows per workgroup");
    constexpr int kRouteTile = TILE;
    constexpr int kRouteRows = TILE / kRouteWaves;  // rows selected together per wave
    extern __shared__ __attribute__((aligned(16))) float s_lds[];  // [kScoreRows][N + 1]
    __shared__ float red_tile[32][33];
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int kg = lane >> 4;   // k group of the 16x16x4 operands
    const int c16 = lane & 15;  // row (A) / candidate (B) of the operands
    const int N = a.blocks;
    const int D = a.head_dim;
    const int row_tiles = (N + kRouteTile - 1) / kRouteTile;
    const int route_wgs = (a.rows / N) * row_tiles;
    if ((int)blockIdx.x >= route_wgs) {
        // H_sum reduction workgroups (fuse_reduce): two 32x32 tiles each
        const int id = blockIdx.x - route_wgs;
        const int rbh = id >> 3;
        reduce_h_tile<T>(r, rbh, 2 * (id & 7), red_tile, t);
        reduce_h_tile<T>(r, rbh, 2 * (id & 7) + 1, red_tile, t);
        if ((id & 7) == 0) zero_centroid_pad<T>(r, rbh, t);
        return;
    }
    const int bh = blockIdx.x / row_tiles;
    const int i0 = (blockIdx.x - bh * row_tiles) * kRouteTile;
    const int stride = N + 1;
    const bool rnd = a.round_bf16 != 0;
    // h_norm of the candidates l, l+64, ... (HYD bias), loaded before the
    // scores so its latency hides behind them; indices clamped into the row
    // (candidates past N get key 0 whatever their bias)
    const bool has_h = a.hnorm != nullptr;
    float hn[PL];
#pragma unroll
    for (int u = 0; u < PL; ++u) hn[u] = has_h ? a.hnorm[(int64_t)bh * N + min(lane + 64 * u, N - 1)] : 0.0f;

    // ---- scores of rows i0 .. i0+15 against every candidate tile.  K step s
    // of lane group g multiplies dim 16(s/4) + 4g + s%4 when D is a multiple
    // of 16 (one aligned 16-byte load per 4 steps), else dim 4s + g (scalar
    // loads); dims past D are zero.  Steps go 16 at a time ("pieces"), the
    // operands of piece x+1 loaded while piece x is multiplied.
    const int cand_tiles = (N + 15) / 16;
    const bool wide = D % 16 == 0;
    const int ksteps = wide ? D / 4 : (D + 3) / 4;
    const int per_tile = (ksteps + 15) / 16;
    const int my_tiles = cand_tiles > wave ? (cand_tiles - wave + kRouteWaves - 1) / kRouteWaves : 0;
    const int pieces = my_tiles * per_tile;
    const float* qrow = a.qc + ((int64_t)bh * N + min(i0 + c16, N - 1)) * D;
    const float* kbase = a.kc + (int64_t)bh * N * D;
    // The loads are unconditional (addresses clamped into the row), so the
    // compiler's wait counts stay exact and the next pieces' loads really stay
    // in flight; dims past D are zeroed where the operands are used (mask_piece,
    // only when D is not a multiple of 64).
    auto fetch = [&](int x, float (&qa)[16], float (&kb)[16]) {
        const int ct = wave + kRouteWaves * (x / per_tile);
        const int s0 = 16 * (x % per_tile);
        const float* krow = kbase + (int64_t)min(ct * 16 + c16, N - 1) * D;
        if (wide) {
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const int d = min(16 * (s0 / 4 + p) + 4 * kg, D - 4);
                const f32x4 xq = *reinterpret_cast<const f32x4*>(qrow + d);
                const f32x4 xk = *reinterpret_cast<const f32x4*>(krow + d);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    qa[4 * p + e] = xq[e];
                    kb[4 * p + e] = xk[e];
                }
            }
        } else {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int d = min(4 * (s0 + e) + kg, D - 1);
                qa[e] = qrow[d];
                kb[e] = krow[d];
            }
        }
    };
    const bool need_mask = D % 64 != 0;
    auto mask_piece = [&](int x, float (&q)[16], float (&k)[16]) {
        const int s0 = 16 * (x % per_tile);
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int d = wide ? 16 * (s0 / 4 + e / 4) + 4 * kg + (e & 3) : 4 * (s0 + e) + kg;
            if (d >= D) {
                q[e] = 0.0f;
                k[e] = 0.0f;
            }
        }
    };
    float qa[2][16], kb[2][16];
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    auto piece = [&](int x, float (&q)[16], float (&k)[16]) {
        if (need_mask) mask_piece(x, q, k);
#pragma unroll
        for (int e = 0; e < 16; ++e) acc = mfma16_f32(rnd ? round_bf16(q[e]) : q[e], rnd ? round_bf16(k[e]) : k[e], acc);
        if (x % per_tile == per_tile - 1) {  // tile done: acc[v] = S[i0 + 4 kg + v][ct * 16 + c16]
            const int j = (wave + kRouteWaves * (x / per_tile)) * 16 + c16;
            if (j < N) {
#pragma unroll
                for (int v = 0; v < 4; ++v) s_lds[(4 * kg + v) * stride + j] = acc[v];
            }
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[v] = 0.0f;
        }
    };
    if (a.qc_bf16 && a.kc_pack && D == 128) {
        // bf16 means (HYD, bf16 inputs): 16x16x32 bf16 MFMA, lane (kg, c16)
        // holding dims 32s + 8kg .. +7 of query row i0 + c16 (A) and of centroid
        // ct*16 + c16 (B) for step s; products are exact, sums fp32.  All loads
        // are unconditional (rows clamped; tiles past the wave's are formed but
        // not stored), so the next tile's loads stay in flight while one tile is
        // multiplied.
        const bf16_t* qr = a.qc_bf16 + ((int64_t)bh * N + min(i0 + c16, N - 1)) * 128 + 8 * kg;
        bf16x8 qf[4], kt[2][4];
#pragma unroll
        for (int st = 0; st < 4; ++st) qf[st] = *reinterpret_cast<const bf16x8*>(qr + 32 * st);
        auto load_tile = [&](int m, bf16x8 (&kf)[4]) {
            const int j = min((wave + kRouteWaves * min(m, my_tiles - 1)) * 16 + c16, N - 1);
            const bf16_t* kr = a.kc_pack + ((int64_t)bh * a.npad + (j & ~63)) * 128;
#pragma unroll
            for (int st = 0; st < 4; ++st)
                kf[st] = *reinterpret_cast<const bf16x8*>(kr + kfrag_elem(j & 63, 32 * st + 8 * kg, 128));
        };
        auto tile = [&](int m, const bf16x8 (&kf)[4]) {
            f32x4 c4 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int st = 0; st < 4; ++st) c4 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qf[st], kf[st], c4, 0, 0, 0);
            const int j = (wave + kRouteWaves * m) * 16 + c16;
            if (j < N) {
#pragma unroll
                for (int v = 0; v < 4; ++v) s_lds[(4 * kg + v) * stride + j] = c4[v];
            }
        };
        if (my_tiles > 0) {
            load_tile(0, kt[0]);
            for (int m = 0; m < my_tiles; m += 2) {
                load_tile(m + 1, kt[1]);
                tile(m, kt[0]);
                load_tile(m + 2, kt[0]);
                tile(m + 1, kt[1]);
            }
        }
    } else {
    if (pieces > 0) {
        // every step loads and multiplies (a piece index past the wave's last
        // re-loads it; its tile lies past N and is not stored), so the count of
        // loads after each operand's load is fixed and the waits stay exact
        fetch(0, qa[0], kb[0]);
        for (int x = 0; x < pieces; x += 2) {
            fetch(min(x + 1, pieces - 1), qa[1], kb[1]);
            piece(x, qa[0], kb[0]);
            fetch(min(x + 2, pieces - 1), qa[0], kb[0]);
            piece(x + 1, qa[1], kb[1]);
        }
    }
    }
    float bias[PL];
#pragma unroll
    for (int u = 0; u < PL; ++u) bias[u] = has_h ? logf(hn[u] + 1e-5f) : 0.0f;
    __syncthreads();

    // ---- scale, HYD bias, sink; selection of rows 4 wave .. 4 wave + 3
    const int sink_j = a.sink == PISA_NO_SINK ? -1 : (a.sink < 0 ? N + a.sink : a.sink);
    const uint64_t lt_mask = (1ull << lane) - 1ull;
    const int k = a.k;
    {
        const int r0 = kRouteRows * wave;  // local rows r0 .. r0 + kRouteRows - 1
        uint32_t key[kRouteRows][PL];
#pragma unroll
        for (int rr = 0; rr < kRouteRows; ++rr) {
            const int i = i0 + r0 + rr;
#pragma unroll
            for (int u = 0; u < PL; ++u) {
                const int j = lane + 64 * u;
                float sc = (j < N ? s_lds[(r0 + rr) * stride + j] : 0.0f) * a.scale + bias[u];
                if (j == sink_j) sc = __builtin_inff();
                key[rr][u] = j < N ? order_key(sc) : 0u;  // padding below every real key
                if (a.scores && j < N && i < N) a.scores[((int64_t)bh * N + i) * N + j] = sc;
            }
        }
        if (k <= 0) {  // nothing selected: the tail keeps every block
#pragma unroll
            for (int rr = 0; rr < kRouteRows; ++rr) {
                const int i = i0 + r0 + rr;
                if (a.selmask && i < N)
                    for (int w = lane; w < a.mask_words; w += 64)
                        a.selmask[((int64_t)bh * N + i) * a.mask_words + w] = 0u;
            }
            return;
        }
        // k-th largest key of each row: largest T with #{key >= T} >= k, found
        // bit by bit for the four rows together, without branches between them.
        // Once a row's prefix has exactly k keys at or above it, those k keys
        // are its k largest and every later step keeps #{key >= T} == k (a
        // candidate is taken only when its count is >= k, and it is <= k), so
        // the rows still searched after that select the same set; the search
        // ends when every row has reached that point (or after bit 0).
        uint32_t T_k[kRouteRows];
        bool done[kRouteRows];
#pragma unroll
        for (int rr = 0; rr < kRouteRows; ++rr) {
            T_k[rr] = 0u;
            done[rr] = false;
        }
        for (int b = 31; b >= 0; --b) {
            bool all_done = true;
#pragma unroll
            for (int rr = 0; rr < kRouteRows; ++rr) {
                const uint32_t cand = T_k[rr] | (1u << b);
                int cnt = 0;
#pragma unroll
                for (int u = 0; u < PL; ++u) cnt += __popcll(__ballot(key[rr][u] >= cand));
                T_k[rr] = cnt >= k ? cand : T_k[rr];
                done[rr] = done[rr] || cnt == k;
                all_done = all_done && done[rr];
            }
            if (all_done) break;
        }
#pragma unroll
        for (int rr = 0; rr < kRouteRows; ++rr) {
            const int i = i0 + r0 + rr;
            if (i >= N) break;  // wave-uniform
            int gt = 0;
#pragma unroll
            for (int u = 0; u < PL; ++u) gt += __popcll(__ballot(key[rr][u] > T_k[rr]));
            int ties_left = k - gt;  // keys equal to T_k still to take, lowest index first
            int32_t* out_idx = a.idx + ((int64_t)bh * N + i) * k;
            int before = 0;
            uint32_t word = 0u;  // mask word `lane` of the row
#pragma unroll
            for (int u = 0; u < PL; ++u) {
                const uint64_t tie = __ballot(key[rr][u] == T_k[rr]);
                const int tie_rank = __popcll(tie & lt_mask);
                const bool sel = key[rr][u] > T_k[rr] || (key[rr][u] == T_k[rr] && tie_rank < ties_left);
                ties_left -= min(ties_left, static_cast<int>(__popcll(tie)));
                const uint64_t bal = __ballot(sel);
                if (sel) out_idx[before + __popcll(bal & lt_mask)] = lane + 64 * u;
                word = lane == 2 * u ? static_cast<uint32_t>(bal) : word;
                word = lane == 2 * u + 1 ? static_cast<uint32_t>(bal >> 32) : word;
                before += __popcll(bal);
            }
            if (a.selmask && lane < a.mask_words) a.selmask[((int64_t)bh * N + i) * a.mask_words + lane] = word;
        }
    }
}

template <int PL, int TILE, typename T>
static int launch_route_pl(const RouteArgs& a, const ReduceArgs& r, int fuse, hipStream_t stream) {
    const int row_tiles = (a.blocks + TILE - 1) / TILE;
    const int bh_count = a.rows / a.blocks;
    const dim3 grid(bh_count * row_tiles + (fuse ? bh_count * 8 : 0));  // routing, then reduction workgroups
    // dynamic LDS: 16 score rows of N + 1 floats (65.6 KB at N = 1024, beside
    // 4.2 KB of static LDS); gfx950 has 160 KB per workgroup, checked here
    const size_t lds = (size_t)kScoreRows * (a.blocks + 1) * sizeof(float);
    static const int lds_limit = [] {
        int dev = 0, bytes = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&bytes, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
            return 0;
        return bytes;
    }();
    const size_t static_lds = sizeof(float) * 32 * 33;
    if (lds_limit <= 0 || lds + static_lds > (size_t)lds_limit)
        return pisa_host::fail(PISA_ERR_UNSUPPORTED, "routing over %d blocks needs %zu bytes of LDS, device allows %d",
                               a.blocks, lds + static_lds, lds_limit);
    hipLaunchKernelGGL((route_topk_kernel<PL, TILE, T>), grid, dim3(64 * kRouteWaves), lds, stream, a, r, fuse);
    return PISA_OK;
}

// 8-row workgroups when 16-row ones would give the CUs fewer than two each
// (C4: 288 workgroups of 16 rows on 256 CUs; prepare 105.9 -> 103.5 us), and
// only up to 256 candidates: every workgroup forms the score
// tiles of all N candidates, so at C5 (N = 512, 1280 workgroups of 16 rows)
// halving the rows per workgroup doubles that work and the launch is 65 us
// slower.
template <typename T>
static int launch_route_t(const RouteArgs& a, const ReduceArgs& r, int fuse, hipStream_t stream) {
    static const int cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return 0;
        return n;
    }();
    const int pl = (a.blocks + 63) / 64;
    const int64_t wgs16 = (int64_t)(a.rows / a.blocks) * ((a.blocks + 15) / 16);
    const bool rows8 = pl <= 4 && wgs16 < 2 * (int64_t)cus;
    if (pl <= 1) return rows8 ? launch_route_pl<1, 8, T>(a, r, fuse, stream) : launch_route_pl<1, 16, T>(a, r, fuse, stream);
    if (pl <= 2) return rows8 ? launch_route_pl<2, 8, T>(a, r, fuse, stream) : launch_route_pl<2, 16, T>(a, r, fuse, stream);
    if (pl <= 3) return rows8 ? launch_route_pl<3, 8, T>(a, r, fuse, stream) : launch_route_pl<3, 16, T>(a, r, fuse, stream);
    if (pl <= 4) return rows8 ? launch_route_pl<4, 8, T>(a, r, fuse, stream) : launch_route_pl<4, 16, T>(a, r, fuse, stream);
    if (pl <= 8) return launch_route_pl<8, 16, T>(a, r, fuse, stream);
    return launch_route_pl<16, 16, T>(a, r, fuse, stream);
}

int launch_route(const RouteArgs& a, hipStream_t stream) {
    ReduceArgs none{};
    if (int rc = launch_route_t<bf16_t>(a, none, 0, stream)) return rc;
    return pisa_host::check_launch("route_topk_kernel");
}

int launch_route_reduce(int dtype, const RouteArgs& a, const ReduceArgs& r, hipStream_t stream) {
    if (a.head_dim != 128) return pisa_host::fail(PISA_ERR_UNSUPPORTED, "fused H_sum reduction needs head dim 128");
    const int rc = dtype == PISA_DTYPE_BF16 ? launch_route_t<bf16_t>(a, r, 1, stream) : launch_route_t<f16_t>(a, r, 1, stream);
    if (rc) return rc;
    return pisa_host::check_launch("route_topk_kernel");
}

}  // namespace pisa
