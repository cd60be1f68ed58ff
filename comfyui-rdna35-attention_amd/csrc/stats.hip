// Per-64-token-block statistics on gfx950.
//
// One 256-thread workgroup owns `chunk_blocks` consecutive key blocks of one
// (batch, head).  For every block it
//   * reads the 64 query/key/value rows once (16-byte loads, token order from
//     the grid map, so raster spatial/video layouts need no packing pass),
//   * reduces the column sums (lane shuffles + one LDS exchange) into the
//     block means q_bar, k_bar, v_bar,
//   * centres the keys in fp32, splits them into a pair hi + lo of the input
//     dtype (kSplitScale) and stages hi, lo and V transposed in LDS,
//   * computes H_b = (K - k_bar)^T V with 32x32x16 MFMAs (hi and lo passes,
//     fp32 accumulation), its Frobenius norm, and accumulates H_b into a
//     per-workgroup partial of H_sum held in the MFMA accumulators,
//   * writes the key and value block packed as attention-kernel operand
//     fragments (kfrag_elem / vfrag_elem; both staged in LDS so every wave
//     store is one contiguous 1 KB fragment) and the packed centroid chunks
//     used by the tail.
// The partial H_sum of each workgroup is written once; stats_reduce_kernel
// sums the partials in a fixed order, so H_sum is deterministic (the
// reference accumulates it with float atomicAdd, pisa_kernels.cu:227).
//
// Semantics follow block_stats_hyd_kernel (pisa_kernels.cu:167-244: means are
// sum-then-scale, keys centred in fp32), block_stats_kernel
// (pisa_kernels.cu:130-164: every element pre-scaled by 1/len) and the Triton
// statistics (pisa_kernel.py:49-84: centred keys rounded to the input dtype).
#include "kernels.hpp"

namespace pisa {

constexpr int kStatsThreads = 256;

// The HYD statistics centre the keys in fp32 and carry each centred value c as
// a pair hi + lo of the input dtype for the MFMA.  |c| <= 2 * max|k| exceeds
// fp16's range for keys near it, so fp16 pairs carry c / 2 and the fp32 products
// are doubled after the MFMA; scaling by a power of two is exact, so the
// results equal those of the unscaled pair wherever it does not overflow
// (bf16 has fp32's range and no scale).
template <typename T> struct SplitScale { static constexpr float value = 1.0f; };
template <> struct SplitScale<f16_t> { static constexpr float value = 0.5f; };
constexpr int kLdsRow = kBlock + 8;  // padded LDS row (elements) of a transposed block
constexpr int kKRow = 128 + 8;       // padded LDS row (elements) of a raw key row

// Element (row d, token position p) of a transposed block in LDS.  The 16-byte
// chunks of a row are XOR-swizzled by (d / 8) % 8: the staging writes (rows 8
// apart across lanes) and the operand reads (32 consecutive rows) then hit at
// most 2 lanes per bank, against 8 for the plain padded layout.
__device__ __forceinline__ int stage_off(int d, int p) {
    return d * kLdsRow + ((((p >> 3) ^ (d >> 3)) & 7) << 3) + (p & 7);
}


template <typename T, int MODE>
__global__ __launch_bounds__(kStatsThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void stats_kernel(StatsArgs a) {
    constexpr int D = 128;
    typedef typename Elem<T>::vec8 vec8;
    __shared__ __attribute__((aligned(16))) T lds_hi[D * kLdsRow];
    __shared__ __attribute__((aligned(16))) T lds_lo[D * kLdsRow];
    __shared__ __attribute__((aligned(16))) T lds_v[D * kLdsRow];
    __shared__ __attribute__((aligned(16))) T lds_k[kBlock * kKRow];  // raw key rows of the block
    __shared__ float red[3][4][D];
    __shared__ float kmean[D];
    __shared__ float norm_part[4];

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int half = lane >> 5;
    const int col = lane & 31;
    const int c16 = t & 15;        // dims c16*8 .. c16*8+7
    const int rq = t >> 4;         // tokens rq*4 .. rq*4+3 of the block
    const int bh = blockIdx.x / a.chunks;
    const int chunk = blockIdx.x - bh * a.chunks;
    const int first = chunk * a.chunk_blocks;
    const int last = min(a.blocks, first + a.chunk_blocks);
    constexpr bool kCov = MODE != PISA_STATS_MEANS;

    f32x16 hp[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int v = 0; v < 16; ++v) hp[nt][v] = 0.0f;

    // Issues the loads of 4 rows x 8 dims of q, k, v of block b (rows past the
    // end of a short last block read a valid row; mask_block zeroes them once
    // the loads are used, so issuing the loads does not wait for them).  The
    // key and value rows are read with the non-temporal hint: nothing reads
    // them again (the attention kernel reads the packed tables written here,
    // which then stay in the caches; C4 prepare 102.8 -> 92.7 us, call
    // 360.2 -> 351.4 us, same box), while the query rows, which the attention
    // kernel reads again, are ordinary loads.
    auto load_block = [&](int b, vec8 (&qv)[4], vec8 (&kv)[4], vec8 (&vv)[4]) {
        const int start = b * kBlock;
        const int len = min(kBlock, a.tokens - start);
        const int64_t off = (c16 * 8) * (int64_t)sizeof(T);
        // raster token of row r = block_base(b) + intra_offset(r): the map's
        // divisions run once per block (wave-uniform), not once per row
        const int base = a.map.block_base(b);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int tok = rq * 4 + r;
            const int raster = base + a.map.intra_offset(min(tok, len - 1));
            qv[r] = load8<vec8>(a.q.data + a.q.row(bh, raster) * sizeof(T) + off);
            kv[r] = load8_nt<vec8>(a.k.data + a.k.row(bh, raster) * sizeof(T) + off);
            vv[r] = load8_nt<vec8>(a.v.data + a.v.row(bh, raster) * sizeof(T) + off);
        }
    };
    auto mask_block = [&](int len, vec8 (&qv)[4], vec8 (&kv)[4], vec8 (&vv)[4]) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (rq * 4 + r >= len)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    qv[r][e] = T(0.0f);
                    kv[r][e] = T(0.0f);
                    vv[r][e] = T(0.0f);
                }
    };

    // Two workgroups share each CU (at most 256 registers per lane), so one
    // workgroup's loads overlap the other's reductions and MFMAs; within a
    // workgroup the next block's rows are loaded once this block is staged in
    // LDS, beside the H_b MFMAs and the packed value stores.
    vec8 qv[4], kv[4], vv[4];
    if (first < last) load_block(first, qv, kv, vv);
    for (int b = first; b < last; ++b) {
        // per-thread indices re-derived every block: LDS and store addresses
        // are recomputed where used instead of held in registers across the loop
        int t_opaque = threadIdx.x;
        asm volatile("" : "+v"(t_opaque));
        const int t = t_opaque;
        const int lane = t & 63;
        const int wave = t >> 6;
        const int half = lane >> 5;
        const int col = lane & 31;
        const int c16 = t & 15;
        const int rq = t >> 4;
        const int start = b * kBlock;
        const int len = min(kBlock, a.tokens - start);
        const float inv_len = 1.0f / static_cast<float>(len);
        mask_block(len, qv, kv, vv);
        // ---- raw key rows to LDS (rows past a short block are zero); they are
        // written out as packed key fragments after the next barrier, one
        // contiguous 1 KB fragment per wave store
        if (a.kp_blocks) {
#pragma unroll
            for (int r = 0; r < 4; ++r) *reinterpret_cast<vec8*>(&lds_k[(rq * 4 + r) * kKRow + c16 * 8]) = kv[r];
        }

        // ---- column sums over this thread's 4 rows, then over the block
        float sq[8], sk[8], sv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float xq = 0.0f, xk = 0.0f, xv = 0.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if (MODE == PISA_STATS_MEANS) {
                    xq += to_f32(qv[r][e]) * inv_len;
                    xk += to_f32(kv[r][e]) * inv_len;
                    xv += to_f32(vv[r][e]) * inv_len;
                } else {
                    xq += to_f32(qv[r][e]);
                    xk += to_f32(kv[r][e]);
                    xv += to_f32(vv[r][e]);
                }
            }
            xq = add_xor32(add_xor16(xq));
            xk = add_xor32(add_xor16(xk));
            xv = add_xor32(add_xor16(xv));
            sq[e] = xq;
            sk[e] = xk;
            sv[e] = xv;
        }
        if (lane < 16) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                red[0][wave][c16 * 8 + e] = sq[e];
                red[1][wave][c16 * 8 + e] = sk[e];
                red[2][wave][c16 * 8 + e] = sv[e];
            }
        }
        __syncthreads();
        if (a.kp_blocks) {
            // packed key block for the attention kernel: element id*8.. of the
            // block is fragment f = id / 64 (rows 32(f/8).., dims 16(f%8)..),
            // lane L = id % 64 (row 32(f/8) + L%32, dims + 8(L/32)) (kfrag_elem)
            T* dst = static_cast<T*>(a.kp_blocks) + ((int64_t)bh * a.blocks + b) * D * kBlock;
#pragma unroll
            for (int it = 0; it < 4; ++it) {
                const int id = it * kStatsThreads + t;
                const int f = id >> 6;
                const int L = id & 63;
                const int key = (f >> 3) * 32 + (L & 31);
                const int d = (f & 7) * 16 + (L >> 5) * 8;
                store8(dst + id * 8, *reinterpret_cast<const vec8*>(&lds_k[key * kKRow + d]));
            }
        }
        if (t < D) {
            const int d = t;
            float mq = ((red[0][0][d] + red[0][1][d]) + red[0][2][d]) + red[0][3][d];
            float mk = ((red[1][0][d] + red[1][1][d]) + red[1][2][d]) + red[1][3][d];
            float mv = ((red[2][0][d] + red[2][1][d]) + red[2][2][d]) + red[2][3][d];
            const float v_sum = mv;  // the sum itself in HYD / GENERIC mode (pisa_kernel.py:74,78)
            if (MODE == PISA_STATS_HYD) {
                mq *= inv_len;
                mk *= inv_len;
                mv *= inv_len;
            } else if (MODE == PISA_STATS_GENERIC) {
                const float fl = static_cast<float>(len);
                mq /= fl;
                mk /= fl;
                mv /= fl;
            }
            kmean[d] = mk;
            const int64_t o = ((int64_t)bh * a.blocks + b) * D + d;
            if (a.qc_f32) static_cast<float*>(a.qc_out)[o] = mq;
            else static_cast<T*>(a.qc_out)[o] = from_f32<T>(mq);
            // (the fused forward routes bf16 HYD on the bf16 means and the packed
            // centroid chunks, and passes null for the outputs nothing reads)
            if (a.kc_out) a.kc_out[o] = mk;
            if (!a.vm_out) {
            } else if (a.vm_f32) {
                static_cast<float*>(a.vm_out)[o] = (MODE != PISA_STATS_MEANS && a.vm_sums) ? v_sum : mv;
            } else {
                static_cast<T*>(a.vm_out)[o] = from_f32<T>(mv);
            }
            if (a.qc_route) a.qc_route[o] = a.qc_route_round ? to_f32(from_f32<T>(mq)) : mq;
            const int64_t chunk_base = ((int64_t)bh * a.npad + (b & ~63)) * D;  // packed 64-centroid chunk
            if (a.kbar_pad) static_cast<T*>(a.kbar_pad)[chunk_base + kfrag_elem(b & 63, d, D)] = from_f32<T>(mk);
            if (a.vbar_t_pad) static_cast<T*>(a.vbar_t_pad)[chunk_base + vfrag_elem(b & 63, d)] = from_f32<T>(mv);
        }
        if (!kCov) {
            if (b + 1 < last) load_block(b + 1, qv, kv, vv);
            __syncthreads();
            continue;
        }
        __syncthreads();

        // ---- centre keys, stage hi / lo / V transposed (swap23 token order)
        const int p0 = swap23(rq * 4);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int d = c16 * 8 + e;
            const float km = kmean[d];
            T hi[4], lo[4], vt[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const bool valid = rq * 4 + r < len;
                const float c = valid ? to_f32(kv[r][e]) - km : 0.0f;
                const float cs = MODE == PISA_STATS_HYD ? c * SplitScale<T>::value : c;
                hi[r] = from_f32<T>(cs);
                lo[r] = (MODE == PISA_STATS_HYD) ? from_f32<T>(cs - to_f32(hi[r])) : T(0.0f);
                vt[r] = vv[r][e];
            }
            typedef T vec4 __attribute__((ext_vector_type(4)));
            vec4 h4 = {hi[0], hi[1], hi[2], hi[3]};
            vec4 l4 = {lo[0], lo[1], lo[2], lo[3]};
            vec4 v4 = {vt[0], vt[1], vt[2], vt[3]};
            *reinterpret_cast<vec4*>(&lds_hi[stage_off(d, p0)]) = h4;
            if (MODE == PISA_STATS_HYD) *reinterpret_cast<vec4*>(&lds_lo[stage_off(d, p0)]) = l4;
            *reinterpret_cast<vec4*>(&lds_v[stage_off(d, p0)]) = v4;
        }
        // the rows of this block are staged: the next block's loads fly during
        // the H_b MFMAs and the packed value stores
        __builtin_amdgcn_sched_barrier(0);
        if (b + 1 < last) load_block(b + 1, qv, kv, vv);
        __syncthreads();

        // ---- H_b tile rows [32*wave, 32*wave+32) x all 128 columns, one
        // 32-column tile at a time (16 accumulators live; the row operands
        // of the four 16-token steps are read once)
        vec8 ah[4], al[4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const int pos = ks * 16 + half * 8;
            ah[ks] = *reinterpret_cast<const vec8*>(&lds_hi[stage_off(wave * 32 + col, pos)]);
            if (MODE == PISA_STATS_HYD) al[ks] = *reinterpret_cast<const vec8*>(&lds_lo[stage_off(wave * 32 + col, pos)]);
        }
        float ss = 0.0f;
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
            f32x16 hb;
#pragma unroll
            for (int v = 0; v < 16; ++v) hb[v] = 0.0f;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const vec8 bv = *reinterpret_cast<const vec8*>(&lds_v[stage_off(nt * 32 + col, ks * 16 + half * 8)]);
                hb = mfma32(ah[ks], bv, hb);
                if (MODE == PISA_STATS_HYD) hb = mfma32(al[ks], bv, hb);
            }
            if (MODE == PISA_STATS_HYD && SplitScale<T>::value != 1.0f)
#pragma unroll
                for (int v = 0; v < 16; ++v) hb[v] *= 1.0f / SplitScale<T>::value;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                ss += hb[v] * hb[v];
                hp[nt][v] += hb[v];
            }
            // one 32-column tile at a time: keeps the accumulators of a single
            // tile live beside the next block's loads
            __builtin_amdgcn_sched_barrier(0);
        }
        ss = wave_sum(ss);
        if (lane == 0) norm_part[wave] = ss;

        // ---- packed value block for the attention kernel
        if (a.vp_blocks) {
            // value fragment f = 4md + ks, lane (half, col): V^T row 32md + col,
            // swap23 positions 16ks + 8half .. +7 (lds_v is stored in that order)
            T* dst = static_cast<T*>(a.vp_blocks) + ((int64_t)bh * a.blocks + b) * D * kBlock;
#pragma unroll
            for (int it = 0; it < 4; ++it) {
                const int id = it * kStatsThreads + t;
                const int f = id >> 6;
                const int L = id & 63;
                const int row = (f >> 2) * 32 + (L & 31);
                const int pos = (f & 3) * 16 + (L >> 5) * 8;
                store8(dst + id * 8, *reinterpret_cast<const vec8*>(&lds_v[stage_off(row, pos)]));
            }
        }
        __syncthreads();
        if (t == 0 && a.hnorm_out)
            a.hnorm_out[(int64_t)bh * a.blocks + b] =
                sqrtf(((norm_part[0] + norm_part[1]) + norm_part[2]) + norm_part[3]);
    }

    if (kCov) {
        float* dst = a.hpart + ((int64_t)bh * a.chunks + chunk) * D * D;
#pragma unroll
        for (int nt = 0; nt < 4; ++nt)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int r = wave * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
                dst[r * D + nt * 32 + col] = hp[nt][v];
            }
    }
}


template <typename T>
__global__ __launch_bounds__(256) void stats_reduce_kernel(ReduceArgs a) {
    __shared__ float tile[32][33];
    reduce_h_tile<T>(a, blockIdx.y, blockIdx.x, tile, threadIdx.x);
    if (blockIdx.x == 0) zero_centroid_pad<T>(a, blockIdx.y, threadIdx.x);
}

// Eight elements d0 .. d0+7 of a row (d0 < head_dim): one 16-byte load when
// head_dim is a multiple of 8 (rows and pieces 16-byte aligned), else element
// loads with the dims past head_dim read as zero (rows of an odd width are
// only element aligned).
template <typename T, typename vec8>
__device__ __forceinline__ vec8 load_piece(const char* row, int d0, int head_dim) {
    if (head_dim % 8 == 0) return load8<vec8>(row + d0 * (int64_t)sizeof(T));
    vec8 x;
    const T* r = reinterpret_cast<const T*>(row);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = d0 + e < head_dim ? r[d0 + e] : T(0.0f);
    return x;
}

// Block means at head dims other than 128 (H_sum and the H_b norms, when
// asked for, come from stats_cov_kernel below): one 256-thread workgroup per
// (batch*head, block).
// Thread (row group rr, piece pc) sums the 8 dims pc*8.. of rows rr, rr+R, ..
// in fp32; an LDS pass adds the R row groups in order.  Means are sum / len
// for the generic statistics (generic_pisa.py:128-132, pisa_kernel.py:72-77)
// and sum * fp32(1/len) for the HYD statistics (pisa_kernels.cu:207-209).
// Writes the [BH][N][D] means and, for the attention kernel, the packed
// centroid chunks at the padded width DP (zero in dims >= D and for the
// centroids past the last block).
template <typename T, int DP, bool HYD>
__global__ __launch_bounds__(256) void stats_means_kernel(StatsArgs a) {
    typedef typename Elem<T>::vec8 vec8;
    constexpr int P = DP / 8;    // 16-byte pieces per row
    constexpr int R = 256 / P;   // rows per pass
    constexpr int kPasses = (kBlock + R - 1) / R;
    __shared__ float red[3][R][DP];
    const int t = threadIdx.x;
    const int bh = blockIdx.x / a.blocks;
    const int b = blockIdx.x - bh * a.blocks;
    const int start = b * kBlock;
    const int len = min(kBlock, a.tokens - start);
    const int pc = t % P;
    const int rr = t / P;
    const bool mapped = t < R * P;
    const int base = a.map.block_base(b);  // raster token of row r: base + intra_offset(r)
    float sq[8], sk[8], sv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) sq[e] = sk[e] = sv[e] = 0.0f;
    if (mapped && pc * 8 < a.head_dim) {
#pragma unroll
        for (int pass = 0; pass < kPasses; ++pass) {
            const int r = pass * R + rr;
            if (r < len) {
                const int raster = base + a.map.intra_offset(r);
                const vec8 x = load_piece<T, vec8>(a.q.data + a.q.row(bh, raster) * sizeof(T), pc * 8, a.head_dim);
                const vec8 y = load_piece<T, vec8>(a.k.data + a.k.row(bh, raster) * sizeof(T), pc * 8, a.head_dim);
                const vec8 z = load_piece<T, vec8>(a.v.data + a.v.row(bh, raster) * sizeof(T), pc * 8, a.head_dim);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    sq[e] += to_f32(x[e]);
                    sk[e] += to_f32(y[e]);
                    sv[e] += to_f32(z[e]);
                }
            }
        }
    }
    if (mapped) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            red[0][rr][pc * 8 + e] = sq[e];
            red[1][rr][pc * 8 + e] = sk[e];
            red[2][rr][pc * 8 + e] = sv[e];
        }
    }
    __syncthreads();
    if (t >= DP) return;
    const int d = t;
    float mq = 0.0f, mk = 0.0f, mv = 0.0f;
    for (int i = 0; i < R; ++i) {
        mq += red[0][i][d];
        mk += red[1][i][d];
        mv += red[2][i][d];
    }
    const float v_sum = mv;  // pisa_kernel.py:74,78 returns the fp32 sum itself
    const float fl = static_cast<float>(len);
    if (HYD) {
        const float inv_len = 1.0f / fl;
        mq *= inv_len;
        mk *= inv_len;
        mv *= inv_len;
    } else {
        mq /= fl;
        mk /= fl;
        mv /= fl;
    }
    const bool live = d < a.head_dim;
    if (live) {
        const int64_t o = ((int64_t)bh * a.blocks + b) * a.head_dim + d;
        if (a.qc_f32) static_cast<float*>(a.qc_out)[o] = mq;
        else static_cast<T*>(a.qc_out)[o] = from_f32<T>(mq);
        a.kc_out[o] = mk;  // the covariance kernel centres on these
        if (!a.vm_out) {
        } else if (a.vm_f32) {
            static_cast<float*>(a.vm_out)[o] = a.vm_sums ? v_sum : mv;
        } else {
            static_cast<T*>(a.vm_out)[o] = from_f32<T>(mv);
        }
        if (a.qc_route) a.qc_route[o] = mq;
    }
    if (!a.kbar_pad) return;  // the standalone statistics entry point wants no packed centroids
    const int64_t head_base = (int64_t)bh * a.npad * DP;
    T* kbar = static_cast<T*>(a.kbar_pad);
    T* vbar = static_cast<T*>(a.vbar_t_pad);
    const int64_t chunk_base = head_base + (int64_t)(b & ~63) * DP;
    kbar[chunk_base + kfrag_elem(b & 63, d, DP)] = live ? from_f32<T>(mk) : T(0.0f);
    vbar[chunk_base + vfrag_elem(b & 63, d)] = live ? from_f32<T>(mv) : T(0.0f);
    if (b == a.blocks - 1) {
        // centroids past the last block: masked to -inf in the tail, zero here
        // so that 0 * value stays finite in the PV product
        for (int j = a.blocks; j < a.npad; ++j) {
            const int64_t base = head_base + (int64_t)(j & ~63) * DP;
            kbar[base + kfrag_elem(j & 63, d, DP)] = T(0.0f);
            vbar[base + vfrag_elem(j & 63, d)] = T(0.0f);
        }
    }
}

template <typename T, bool HYD>
int launch_stats_means_t(int padded, const StatsArgs& a, int bh_count, hipStream_t stream) {
    const dim3 grid(bh_count * a.blocks);
    switch (padded) {
        case 64: hipLaunchKernelGGL((stats_means_kernel<T, 64, HYD>), grid, dim3(256), 0, stream, a); break;
        case 96: hipLaunchKernelGGL((stats_means_kernel<T, 96, HYD>), grid, dim3(256), 0, stream, a); break;
        case 128: hipLaunchKernelGGL((stats_means_kernel<T, 128, HYD>), grid, dim3(256), 0, stream, a); break;  // 104..120
        case 160: hipLaunchKernelGGL((stats_means_kernel<T, 160, HYD>), grid, dim3(256), 0, stream, a); break;
        case 192: hipLaunchKernelGGL((stats_means_kernel<T, 192, HYD>), grid, dim3(256), 0, stream, a); break;
        case 256: hipLaunchKernelGGL((stats_means_kernel<T, 256, HYD>), grid, dim3(256), 0, stream, a); break;
        default: return pisa_host::fail(PISA_ERR_UNSUPPORTED, "block means: padded head dim %d", padded);
    }
    return pisa_host::check_launch("stats_means_kernel");
}

int launch_stats_means(int dtype, int padded, const StatsArgs& a, int bh_count, hipStream_t stream, bool hyd) {
    if (dtype == PISA_DTYPE_BF16)
        return hyd ? launch_stats_means_t<bf16_t, true>(padded, a, bh_count, stream)
                   : launch_stats_means_t<bf16_t, false>(padded, a, bh_count, stream);
    return hyd ? launch_stats_means_t<f16_t, true>(padded, a, bh_count, stream)
               : launch_stats_means_t<f16_t, false>(padded, a, bh_count, stream);
}

// H_sum partials (and H_b norms) at head dims other than 128, one wave per
// (head, chunk of blocks, 32x32 tile (tr, tc) of H).  For each block it reads
// the block's 32 key dims of row slice tr and 32 value dims of column slice tc
// (16-byte pieces, token order from the grid map), centres the keys on the
// fp32 block means of the means kernel, stages both slices transposed in LDS
// (dim-major, 4 consecutive tokens per 8-byte write) and forms the tile
// H_b[32tr + i][32tc + j] with 32x32x16 MFMAs (tokens as the contraction),
// which it adds to the chunk's partial.
//   HYD = false: the Triton statistics every head dim up to 256 takes
//     (pisa_kernel.py:71-84): centred keys rounded to the input dtype.
//   HYD = true: block_stats_hyd_kernel (pisa_kernels.cu:214-243): keys
//     centred in fp32, carried as a dtype pair hi + lo (hi = dtype(c s),
//     lo = dtype(c s - hi), s = SplitScale) with one MFMA pass each.
// When normpart is set, the wave also writes the tile's sum of squares of
// H_b for every block ([BH][N][tiles]); cov_reduce_kernel adds the tiles in
// order into ||H_b||_F.  Rows past a short last block contribute zero, as
// their zero values make them contribute in the reference.  The partial of
// each chunk is written once (no float atomics; the reference adds with
// atomicAdd / tl.atomic_add).
template <typename T, int DP, bool HYD>
__global__ __launch_bounds__(64) void stats_cov_kernel(CovArgs a) {
    typedef typename Elem<T>::vec8 vec8;
    typedef T vec4 __attribute__((ext_vector_type(4)));
    constexpr int TD = DP / 32;
    constexpr int kRowT = kBlock + 8;  // padded LDS row (tokens) of a transposed slice
    __shared__ __attribute__((aligned(16))) T kts[32 * kRowT];
    __shared__ __attribute__((aligned(16))) T kts_lo[HYD ? 32 * kRowT : 8];
    __shared__ __attribute__((aligned(16))) T vts[32 * kRowT];
    const int lane = threadIdx.x;
    const int tile = blockIdx.x % (TD * TD);
    const int rest = blockIdx.x / (TD * TD);
    const int chunk = rest % a.chunks;
    const int bh = rest / a.chunks;
    const int tr = tile / TD;
    const int tc = tile % TD;
    const int first = chunk * a.chunk_blocks;
    const int last = min(a.blocks, first + a.chunk_blocks);
    const int pc = lane & 3;    // 8-dim piece of the slices
    const int q4 = lane >> 2;   // tokens 4 q4 .. 4 q4 + 3
    const int dk = 32 * tr + 8 * pc;
    const int dv = 32 * tc + 8 * pc;
    const bool kdims = dk < a.head_dim;  // dims past head_dim read as zero (load_piece)
    const bool vdims = dv < a.head_dim;
    const int col = lane & 31;
    const int half = lane >> 5;
    f32x16 acc;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
    for (int b = first; b < last; ++b) {
        const int len = min(kBlock, a.tokens - b * kBlock);
        const int base = a.map.block_base(b);
        float mean[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
            mean[e] = dk + e < a.head_dim ? a.kmean[((int64_t)bh * a.blocks + b) * a.head_dim + dk + e] : 0.0f;
        vec8 kx[4], vx[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int raster = base + a.map.intra_offset(min(4 * q4 + r, len - 1));
            if (kdims) kx[r] = load_piece<T, vec8>(a.k.data + a.k.row(bh, raster) * (int64_t)sizeof(T), dk, a.head_dim);
            if (vdims) vx[r] = load_piece<T, vec8>(a.v.data + a.v.row(bh, raster) * (int64_t)sizeof(T), dv, a.head_dim);
        }
        // the previous block's operand reads by other lanes come before these
        // stores (one wave: the barrier orders its LDS accesses, at no cost)
        __syncthreads();
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            vec4 ck, cl, cv;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const bool valid = 4 * q4 + r < len;
                const float c0 = (valid && kdims) ? to_f32(kx[r][e]) - mean[e] : 0.0f;
                const float c = HYD ? c0 * SplitScale<T>::value : c0;
                ck[r] = from_f32<T>(c);
                if (HYD) cl[r] = from_f32<T>(c - to_f32(ck[r]));
                cv[r] = (valid && vdims) ? vx[r][e] : T(0.0f);
            }
            *reinterpret_cast<vec4*>(&kts[(8 * pc + e) * kRowT + 4 * q4]) = ck;
            if (HYD) *reinterpret_cast<vec4*>(&kts_lo[(8 * pc + e) * kRowT + 4 * q4]) = cl;
            *reinterpret_cast<vec4*>(&vts[(8 * pc + e) * kRowT + 4 * q4]) = cv;
        }
        // the slices written by every lane are read below
        __syncthreads();
        f32x16 hb;
#pragma unroll
        for (int v = 0; v < 16; ++v) hb[v] = 0.0f;
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            const vec8 ka = *reinterpret_cast<const vec8*>(&kts[col * kRowT + 16 * st + 8 * half]);
            const vec8 vb = *reinterpret_cast<const vec8*>(&vts[col * kRowT + 16 * st + 8 * half]);
            hb = mfma32(ka, vb, hb);
            if (HYD) {
                const vec8 kl = *reinterpret_cast<const vec8*>(&kts_lo[col * kRowT + 16 * st + 8 * half]);
                hb = mfma32(kl, vb, hb);
            }
        }
        if (HYD && SplitScale<T>::value != 1.0f)
#pragma unroll
            for (int v = 0; v < 16; ++v) hb[v] *= 1.0f / SplitScale<T>::value;
        float ss = 0.0f;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            acc[v] += hb[v];
            ss += hb[v] * hb[v];
        }
        if (a.normpart) {
            ss = wave_sum(ss);
            if (lane == 0) a.normpart[((int64_t)bh * a.blocks + b) * (TD * TD) + tile] = ss;
        }
    }
    float* dst = a.hpart + ((int64_t)bh * a.chunks + chunk) * DP * DP;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int row = 32 * tr + 8 * (v >> 2) + 4 * half + (v & 3);
        dst[row * DP + 32 * tc + col] = acc[v];
    }
}

// Chunk-order sum of the partials (one 32x32 tile of H_sum per workgroup);
// the tile-0 workgroup of each head also adds every block's tile sums of
// squares in tile order into ||H_b||_F when asked for.
template <typename T, int DP>
__global__ __launch_bounds__(256) void cov_reduce_kernel(ReduceArgs a) {
    __shared__ float tile[32][33];
    const int bh = blockIdx.y;
    reduce_h_tile<T, DP>(a, bh, blockIdx.x, tile, threadIdx.x);
    if (blockIdx.x == 0 && a.hnorm) {
        constexpr int kTiles = (DP / 32) * (DP / 32);
        for (int b = threadIdx.x; b < a.blocks; b += 256) {
            const float* src = a.normpart + ((int64_t)bh * a.blocks + b) * kTiles;
            float ss = 0.0f;
#pragma unroll 8
            for (int i = 0; i < kTiles; ++i) ss += src[i];
            a.hnorm[(int64_t)bh * a.blocks + b] = sqrtf(ss);
        }
    }
}

template <typename T, int DP>
static void launch_cov_dp(const CovArgs& a, const ReduceArgs* r, bool hyd, int bh_count, hipStream_t stream) {
    constexpr int tiles = (DP / 32) * (DP / 32);
    const dim3 grid(bh_count * a.chunks * tiles);
    if (r) hipLaunchKernelGGL((cov_reduce_kernel<T, DP>), dim3(tiles, bh_count), dim3(256), 0, stream, *r);
    else if (hyd) hipLaunchKernelGGL((stats_cov_kernel<T, DP, true>), grid, dim3(64), 0, stream, a);
    else hipLaunchKernelGGL((stats_cov_kernel<T, DP, false>), grid, dim3(64), 0, stream, a);
}

template <typename T>
static int launch_cov_t(int padded, const CovArgs& a, const ReduceArgs* r, bool hyd, int bh_count,
                        hipStream_t stream) {
    switch (padded) {
        case 64: launch_cov_dp<T, 64>(a, r, hyd, bh_count, stream); break;
        case 96: launch_cov_dp<T, 96>(a, r, hyd, bh_count, stream); break;
        case 128: launch_cov_dp<T, 128>(a, r, hyd, bh_count, stream); break;  // head dims 104..120
        case 160: launch_cov_dp<T, 160>(a, r, hyd, bh_count, stream); break;
        case 192: launch_cov_dp<T, 192>(a, r, hyd, bh_count, stream); break;
        case 256: launch_cov_dp<T, 256>(a, r, hyd, bh_count, stream); break;
        default: return pisa_host::fail(PISA_ERR_UNSUPPORTED, "H_sum: padded head dim %d", padded);
    }
    return pisa_host::check_launch(r ? "cov_reduce_kernel" : "stats_cov_kernel");
}

int launch_stats_cov(int dtype, int padded, const CovArgs& a, int bh_count, hipStream_t stream, bool hyd) {
    if (dtype == PISA_DTYPE_BF16) return launch_cov_t<bf16_t>(padded, a, nullptr, hyd, bh_count, stream);
    return launch_cov_t<f16_t>(padded, a, nullptr, hyd, bh_count, stream);
}

int launch_cov_reduce(int dtype, int padded, const ReduceArgs& r, int bh_count, hipStream_t stream) {
    const CovArgs none{};
    if (dtype == PISA_DTYPE_BF16) return launch_cov_t<bf16_t>(padded, none, &r, false, bh_count, stream);
    return launch_cov_t<f16_t>(padded, none, &r, false, bh_count, stream);
}

template <typename T, int MODE>
int launch_stats_t(const StatsArgs& a, int bh_count, hipStream_t stream) {
    hipLaunchKernelGGL((stats_kernel<T, MODE>), dim3(bh_count * a.chunks), dim3(kStatsThreads), 0,
                       stream, a);
    return pisa_host::check_launch("stats_kernel");
}

int launch_stats(int dtype, int mode, const StatsArgs& a, int bh_count, hipStream_t stream) {
    if (dtype == PISA_DTYPE_BF16) {
        if (mode == PISA_STATS_MEANS) return launch_stats_t<bf16_t, PISA_STATS_MEANS>(a, bh_count, stream);
        if (mode == PISA_STATS_HYD) return launch_stats_t<bf16_t, PISA_STATS_HYD>(a, bh_count, stream);
        return launch_stats_t<bf16_t, PISA_STATS_GENERIC>(a, bh_count, stream);
    }
    if (mode == PISA_STATS_MEANS) return launch_stats_t<f16_t, PISA_STATS_MEANS>(a, bh_count, stream);
    if (mode == PISA_STATS_HYD) return launch_stats_t<f16_t, PISA_STATS_HYD>(a, bh_count, stream);
    return launch_stats_t<f16_t, PISA_STATS_GENERIC>(a, bh_count, stream);
}

int launch_stats_reduce(int dtype, const ReduceArgs& a, int bh_count, hipStream_t stream) {
    if (dtype == PISA_DTYPE_BF16)
        hipLaunchKernelGGL(stats_reduce_kernel<bf16_t>, dim3(16, bh_count), dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL(stats_reduce_kernel<f16_t>, dim3(16, bh_count), dim3(256), 0, stream, a);
    return pisa_host::check_launch("stats_reduce_kernel");
}

}  // namespace pisa
