// Fixed block-diagonal attention: every 64-token block attends only to itself.
//
// Four kernels.  bf16/fp16 calls without a mask run fixed_block_mfma_kernel
// (matrix cores, the reference's Triton semantics, below); fp32 calls without
// a mask run fixed_block_f32x3_kernel (head dims 32, 64: fp32 products from
// exact three-part bf16 splits on the bf16 matrix cores) or
// fixed_block_f32_mfma_kernel (head dim 128: fp32 matrix cores).  Masked
// calls and rows that are not 16-byte aligned - the calls the reference sends
// to its eager fp32 loop - run fixed_block_kernel:
//
// One 256-thread workgroup per (block, batch*head).  The block's Q, K and V
// (64 x D) are staged in LDS as fp32; thread (rt, kt) = (t/16, t%16) owns the
// score rows {rt + 16i} x keys {kt + 16i'} (i, i' < 4), so every LDS read of a
// 16-lane group touches 16 consecutive padded rows (conflict free) or
// broadcasts.  The softmax is computed in fp32 (row max and sum over the 16
// lanes of a row group by shuffles), the normalised probabilities go back to
// LDS and the same lanes form O = P V for dims {kt + 16j}.
//
// All arithmetic is fp32 whatever the storage type, as in
// fixed_block_attention_ref (reference.py:179-198: fp32 scores, softmax, fp32
// P @ V, cast to the input dtype).  Keys past the end of a partial last block
// are excluded and `causal` masks keys after the query inside the block
// (reference.py:186-188, triton_kernel.py:86-89); an attention mask then
// removes keys (bool, false -> -inf) or adds to the scaled scores
// (reference.py:190-195).  A row with every key masked gives NaN, the value
// torch.softmax returns for it.
#include <type_traits>

#include "kernels.hpp"

namespace pisa {

template <typename T> __device__ __forceinline__ float ld(const char* p) { return to_f32(*reinterpret_cast<const T*>(p)); }

// Score after the attention mask entry at element offset `off`.
__device__ __forceinline__ float apply_mask(const MaskView& m, int64_t off, float s) {
    switch (m.kind) {
        case PISA_MASK_BOOL: return m.data[off] ? s : -__builtin_inff();
        case PISA_MASK_ADD_F32: return s + reinterpret_cast<const float*>(m.data)[off];
        case PISA_MASK_ADD_F16: return s + to_f32(reinterpret_cast<const f16_t*>(m.data)[off]);
        case PISA_MASK_ADD_BF16: return s + to_f32(reinterpret_cast<const bf16_t*>(m.data)[off]);
        default: return s;
    }
}

template <typename T, int D>
__global__ __launch_bounds__(256) void fixed_block_kernel(View q, View k, View v, OutView o, int tokens,
                                                          int nblocks, float scale, int causal, MaskView mask) {
    constexpr int kRow = D + 4;
    constexpr int kPRow = 68;
    __shared__ __attribute__((aligned(16))) float qs[64 * kRow];
    __shared__ __attribute__((aligned(16))) float ps[64 * kPRow];
    __shared__ __attribute__((aligned(16))) float ks[64 * kRow];
    __shared__ __attribute__((aligned(16))) float vs[64 * kRow];
    const int t = threadIdx.x;
    const int bh = blockIdx.x / nblocks;
    const int blk = blockIdx.x - bh * nblocks;
    const int start = blk * 64;
    const int len = min(64, tokens - start);

    // ---- stage the block (zero rows beyond len)
    for (int e = t; e < 64 * D; e += 256) {
        const int r = e / D;
        const int d = e - r * D;
        float xq = 0.0f, xk = 0.0f, xv = 0.0f;
        if (r < len) {
            xq = ld<T>(q.data + (q.row(bh, start + r) + d) * sizeof(T));
            xk = ld<T>(k.data + (k.row(bh, start + r) + d) * sizeof(T));
            xv = ld<T>(v.data + (v.row(bh, start + r) + d) * sizeof(T));
        }
        qs[r * kRow + d] = xq;
        ks[r * kRow + d] = xk;
        vs[r * kRow + d] = xv;
    }
    __syncthreads();

    const int rt = t >> 4;
    const int kt = t & 15;
    float s[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) s[i][j] = 0.0f;
    for (int d = 0; d < D; d += 4) {
        f32x4 qa[4], kb[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            qa[i] = *reinterpret_cast<const f32x4*>(&qs[(rt + 16 * i) * kRow + d]);
            kb[i] = *reinterpret_cast<const f32x4*>(&ks[(kt + 16 * i) * kRow + d]);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) s[i][j] = fmaf(qa[i][e], kb[j][e], s[i][j]);
    }

    // mask element (b, h, start + row, start + key) of this workgroup's rows
    int64_t mask_base = 0;
    if (mask.kind != PISA_MASK_NONE) {
        const int mb = bh / mask.heads;
        const int mh = bh - mb * mask.heads;
        mask_base = mb * mask.sb + mh * mask.sh + (int64_t)start * (mask.sq + mask.sk);
    }
    float p[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = rt + 16 * i;
        float mx = -__builtin_inff();
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int key = kt + 16 * j;
            const bool dead = key >= len || row >= len || (causal && key > row);
            s[i][j] = dead ? -__builtin_inff() : s[i][j] * scale;
            if (!dead && mask.kind != PISA_MASK_NONE)
                s[i][j] = apply_mask(mask, mask_base + row * mask.sq + key * mask.sk, s[i][j]);
            mx = fmaxf(mx, s[i][j]);
        }
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
        const float m_use = (mx == -__builtin_inff()) ? 0.0f : mx;
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            p[i][j] = expf(s[i][j] - m_use);
            sum += p[i][j];
        }
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) sum += __shfl_xor(sum, off);
        const float inv = sum > 0.0f ? 1.0f / sum : __builtin_nanf("");  // all keys masked
#pragma unroll
        for (int j = 0; j < 4; ++j) p[i][j] *= inv;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) ps[(rt + 16 * i) * kPRow + kt + 16 * j] = p[i][j];
    __syncthreads();

    constexpr int kDims = D / 16;
    float acc[4][kDims];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int c = 0; c < kDims; ++c) acc[i][c] = 0.0f;
    for (int key = 0; key < 64; ++key) {
        float pv[4], vv[kDims];
#pragma unroll
        for (int i = 0; i < 4; ++i) pv[i] = ps[(rt + 16 * i) * kPRow + key];
#pragma unroll
        for (int c = 0; c < kDims; ++c) vv[c] = vs[key * kRow + kt + 16 * c];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int c = 0; c < kDims; ++c) acc[i][c] = fmaf(pv[i], vv[c], acc[i][c]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = rt + 16 * i;
        if (row >= len) continue;
        T* dst = reinterpret_cast<T*>(o.data + o.row(bh, start + row) * (int64_t)sizeof(T));
#pragma unroll
        for (int c = 0; c < kDims; ++c) dst[kt + 16 * c] = from_f32<T>(acc[i][c]);
    }
}

// bf16 / fp16 without a mask: one wavefront per block on 32x32x16 MFMA, the
// semantics of the reference's Triton kernel (triton_kernel.py:53-100): scores
// with fp32 accumulation, softmax in fp32, probabilities normalised and then
// rounded to the input dtype, P @ V with fp32 accumulation, rounded output.
//
// Nothing is staged in LDS, so the occupancy is set by registers alone.  The
// products are formed transposed as in the attention kernels (S^T = K Q^T,
// O^T = V^T P^T): a query is a lane column and the probabilities feed the
// second MFMA from their accumulator registers.  The Q and K operands are 16
// bytes of one row per lane (rows 32x + col, dims 16t + 8half .. +7), read
// straight from the rows.  The V^T operand needs 8 keys of one dim per lane;
// the dims of an output tile are assigned so that a lane reads MD = D/32
// consecutive dims of a key row with one load (output tile md holds dims
// MD*i + md of accumulator row i), one load instruction covers two whole key
// rows, and the operand of tile md takes element md of 8 such loads.
template <typename T, int D>
__global__ __launch_bounds__(64) void fixed_block_mfma_kernel(View q, View k, View v, OutView o, int tokens,
                                                               int nblocks, float scale_log2, int causal) {
    typedef typename Elem<T>::vec8 vec8;
    constexpr int KT = D / 16;  // 16-deep k-steps of the score product
    constexpr int MD = D / 32;  // output dim tiles; dims a lane reads per key row
    typedef T vecmd __attribute__((ext_vector_type(MD)));
    const int lane = threadIdx.x;
    const int half = lane >> 5;
    const int col = lane & 31;
    const int bh = blockIdx.x / nblocks;
    const int start = (blockIdx.x - bh * nblocks) * 64;
    const int len = min(64, tokens - start);
    auto at = [&](const View& x, int r) {  // row r of the block, clamped to the last real row
        return x.data + x.row(bh, start + min(r, len - 1)) * (int64_t)sizeof(T);
    };

    // ---- S^T[key][query] for key tiles mt and query tiles nt
    // requested k-step by k-step, the order the products consume them
    vec8 kf[2][KT], qf[2][KT];
    const char* krow[2] = {at(k, col), at(k, 32 + col)};
    const char* qrow[2] = {at(q, col), at(q, 32 + col)};
#pragma unroll
    for (int t = 0; t < KT; ++t)
#pragma unroll
        for (int x = 0; x < 2; ++x) {
            kf[x][t] = load8<vec8>(krow[x] + (16 * t + 8 * half) * sizeof(T));
            qf[x][t] = load8<vec8>(qrow[x] + (16 * t + 8 * half) * sizeof(T));
        }
    // every Q and K request is issued before the first product (the
    // scheduler would otherwise issue each just before its use, one memory
    // round trip at a time), and the V requests right after the products
    __builtin_amdgcn_sched_barrier(0);
    f32x16 s[2][2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int e = 0; e < 16; ++e) s[mt][nt][e] = 0.0f;
#pragma unroll
    for (int t = 0; t < KT; ++t)
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) s[mt][nt] = mfma32(kf[mt][t], qf[nt][t], s[mt][nt]);

    // ---- value rows: key 32mt + 16ss + 4half + 8(e/4) + e%4 (the key of
    // probability element e of k-step (mt, ss) in this lane), dims MD*col ..
    // Keys past the block's length read its last row and get probability 0.
    // The loads are unconditional: behind a branch, the compiler's wait
    // counts would wait for every earlier load before each of them.
    vecmd vr[2][2][8];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int ss = 0; ss < 2; ++ss)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int key = 32 * mt + 16 * ss + 4 * half + 8 * (e >> 2) + (e & 3);
                vr[mt][ss][e] = *reinterpret_cast<const vecmd*>(at(v, key) + MD * col * sizeof(T));
            }

    __builtin_amdgcn_sched_barrier(0);

    // ---- masking and the softmax of query column (nt, col), in log2 units:
    // accumulator e of tile mt is key 32mt + 8(e/4) + 4half + e%4
    vec8 pf[2][2][2];  // [nt][mt][ss]: 8 probabilities, elements 8ss .. 8ss+7 of tile mt
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const int query = 32 * nt + col;
        float mx = -__builtin_inff();
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int key = 32 * mt + 8 * (e >> 2) + 4 * half + (e & 3);
                const bool dead = key >= len || (causal && key > query);
                s[mt][nt][e] = dead ? -__builtin_inff() : s[mt][nt][e] * scale_log2;
                mx = fmaxf(mx, s[mt][nt][e]);
            }
        mx = max_xor32(mx);
        const float m_use = mx == -__builtin_inff() ? 0.0f : mx;
        float sum = 0.0f;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                s[mt][nt][e] = __builtin_amdgcn_exp2f(s[mt][nt][e] - m_use);
                sum += s[mt][nt][e];
            }
        sum = add_xor32(sum);
        const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;  // rows past len: never stored
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int ss = 0; ss < 2; ++ss)
#pragma unroll
                for (int e = 0; e < 8; ++e) pf[nt][mt][ss][e] = from_f32<T>(s[mt][nt][ss * 8 + e] * inv);
    }

    // ---- O^T[dim][query] = sum_key V^T[dim][key] P^T[key][query]; row i of tile md is dim MD*i + md
    f32x16 acc[MD][2];
#pragma unroll
    for (int md = 0; md < MD; ++md)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[md][nt][e] = 0.0f;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int ss = 0; ss < 2; ++ss)
#pragma unroll
            for (int md = 0; md < MD; ++md) {
                vec8 vf;
#pragma unroll
                for (int e = 0; e < 8; ++e) vf[e] = vr[mt][ss][e][md];
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) acc[md][nt] = mfma32(vf, pf[nt][mt][ss], acc[md][nt]);
            }

    // ---- store: accumulator e of every tile is row i = 8(e/4) + 4half + e%4,
    // i.e. dims MD*i .. MD*i + MD-1 of query 32nt + col across the MD tiles
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const int query = 32 * nt + col;
        if (query >= len) continue;
        char* dst = o.data + o.row(bh, start + query) * (int64_t)sizeof(T);
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int i = 8 * (e >> 2) + 4 * half + (e & 3);
            vecmd x;
#pragma unroll
            for (int md = 0; md < MD; ++md) x[md] = from_f32<T>(acc[md][nt][e]);
            *reinterpret_cast<vecmd*>(dst + MD * i * sizeof(T)) = x;
        }
    }
}

// fp32 without a mask: four waves per block on v_mfma_f32_16x16x4_f32 (fp32
// operands, fp32 accumulation), the arithmetic of fixed_block_kernel above
// (fp32 scores, softmax with expf, fp32 P @ V).  Wave w owns queries
// 16w .. 16w+15 (a lane column c = lane % 16, lane group g = lane / 16).
//   S^T = K Q^T: k-step t = 4s + e contracts dim 16s + 4g + e in lane group g,
//     so each lane reads its K and Q rows as float4 pieces (dims 16s + 4g ..);
//     accumulator r of key tile n is key 16n + 4g + r of query 16w + c.
//   O^T = V^T P^T: k-step (n, r) contracts key 16n + 4g + r, exactly the
//     probability the lane holds in accumulator r of key tile n.  Row i of
//     output tile m is dim VW*i + m (VW = D/16), so a lane reads VW
//     consecutive dims of a key row with one load and, at the end, holds the
//     4*VW consecutive dims 4*VW*g .. of its query.
// The block's K and V rows are loaded once per workgroup (wave w reads rows
// 16w .. 16w+15 of both) and staged in LDS with padded rows, from where every
// wave reads its operands: with each wave loading all 64 rows itself, the four
// waves moved four times the K/V bytes through the CU's memory path (C1:
// 13.4 -> 11.3 us).  Q rows are read by their own wave.  Rows past the block's
// length are read clamped to its last row (unconditional loads, so the
// compiler's wait counts stay partial) and get probability 0 (keys) or are not
// stored (queries).
template <int D>
__global__ __launch_bounds__(256) void fixed_block_f32_mfma_kernel(View q, View k, View v, OutView o, int tokens,
                                                                   int nblocks, float scale, int causal) {
    constexpr int S4 = D / 16;  // float4 pieces of a Q or K row per lane
    constexpr int VW = D / 16;  // V dims per lane per key row = output dim tiles
    constexpr int kRowF = D + 4;  // padded LDS row (floats)
    __shared__ __attribute__((aligned(16))) float ks[64 * kRowF];
    __shared__ __attribute__((aligned(16))) float vs[64 * kRowF];
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int c = lane & 15;
    const int g = lane >> 4;
    const int bh = blockIdx.x / nblocks;
    const int start = (blockIdx.x - bh * nblocks) * 64;
    const int len = min(64, tokens - start);
    auto at = [&](const View& x, int r) {
        return reinterpret_cast<const float*>(x.data) + x.row(bh, start + min(r, len - 1));
    };

    f32x4 qv[S4], kv[4][S4];
    {
        const float* qr = at(q, 16 * w + c);
#pragma unroll
        for (int s4 = 0; s4 < S4; ++s4) qv[s4] = *reinterpret_cast<const f32x4*>(qr + 16 * s4 + 4 * g);
    }
    float vv[4][4][VW];
    {
        // staging: lane l of wave w loads dims D/4 (l%4) .. of row 16w + l/4 of K and V
        constexpr int P = D / 16;  // float4 pieces per lane
        const int row = 16 * w + (lane >> 2);
        const int d0 = (lane & 3) * (D / 4);
        const float* kr = at(k, row) + d0;
        const float* vr = at(v, row) + d0;
        f32x4 xk[P], xv[P];
#pragma unroll
        for (int p = 0; p < P; ++p) {
            xk[p] = *reinterpret_cast<const f32x4*>(kr + 4 * p);
            xv[p] = *reinterpret_cast<const f32x4*>(vr + 4 * p);
        }
#pragma unroll
        for (int p = 0; p < P; ++p) {
            *reinterpret_cast<f32x4*>(&ks[row * kRowF + d0 + 4 * p]) = xk[p];
            *reinterpret_cast<f32x4*>(&vs[row * kRowF + d0 + 4 * p]) = xv[p];
        }
    }
    __syncthreads();
#pragma unroll
    for (int n = 0; n < 4; ++n)
#pragma unroll
        for (int s4 = 0; s4 < S4; ++s4)
            kv[n][s4] = *reinterpret_cast<const f32x4*>(&ks[(16 * n + c) * kRowF + 16 * s4 + 4 * g]);
#pragma unroll
    for (int n = 0; n < 4; ++n)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int key = 16 * n + 4 * g + r;
#pragma unroll
            for (int m = 0; m < VW; ++m) vv[n][r][m] = vs[key * kRowF + VW * c + m];
        }
    // all operand reads issued before the first product at D <= 64 (at D = 128
    // the operands held at once would cost occupancy)
    if constexpr (D <= 64) __builtin_amdgcn_sched_barrier(0);
    // key tile by key tile, in the order the operands were read: the products
    // of a tile wait only for its own reads
    f32x4 sacc[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) {
        sacc[n] = f32x4(0.0f);
#pragma unroll
        for (int s4 = 0; s4 < S4; ++s4)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                sacc[n] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[n][s4][e], qv[s4][e], sacc[n], 0, 0, 0);
    }

    // softmax of query column 16w + c: its 64 keys are 16 accumulators in each of the lanes c, c+16, c+32, c+48
    const int query = 16 * w + c;
    float mx = -__builtin_inff();
#pragma unroll
    for (int n = 0; n < 4; ++n)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int key = 16 * n + 4 * g + r;
            const bool dead = key >= len || (causal && key > query);
            sacc[n][r] = dead ? -__builtin_inff() : sacc[n][r] * scale;
            mx = fmaxf(mx, sacc[n][r]);
        }
    {
        const float2 p16 = pair_xor16(mx);
        mx = max_xor32(fmaxf(p16.x, p16.y));
    }
    const float m_use = (mx == -__builtin_inff()) ? 0.0f : mx;
    float sum = 0.0f;
#pragma unroll
    for (int n = 0; n < 4; ++n)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            sacc[n][r] = expf(sacc[n][r] - m_use);
            sum += sacc[n][r];
        }
    sum = add_xor32(add_xor16(sum));
    const float inv = sum > 0.0f ? 1.0f / sum : __builtin_nanf("");  // all keys masked
#pragma unroll
    for (int n = 0; n < 4; ++n)
#pragma unroll
        for (int r = 0; r < 4; ++r) sacc[n][r] *= inv;

    f32x4 oacc[VW];
#pragma unroll
    for (int m = 0; m < VW; ++m) oacc[m] = f32x4(0.0f);
#pragma unroll
    for (int n = 0; n < 4; ++n)
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int m = 0; m < VW; ++m)
                oacc[m] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[n][r][m], sacc[n][r], oacc[m], 0, 0, 0);

    if (query >= len) return;
    // dims 4*VW*g + VW*r + m hold oacc[m][r]: 4*VW consecutive floats
    float* dst = reinterpret_cast<float*>(o.data) + o.row(bh, start + query) + 4 * VW * g;
#pragma unroll
    for (int f = 0; f < 4 * VW; f += 4) {
        f32x4 x;
#pragma unroll
        for (int j = 0; j < 4; ++j) x[j] = oacc[(f + j) % VW][(f + j) / VW];
        *reinterpret_cast<f32x4*>(dst + f) = x;
    }
}

// e^x for x <= 0 in fp32: 2^(x log2 e) on v_exp_f32, with the rounding error of
// the product (an fma) and the low part of log2 e carried into a first-order
// factor (its neglected square is below 1e-10 for x >= -100); -inf gives 0.
// Four full-rate instructions and one exponential where expf's range handling
// takes about a dozen (C1 9.43 -> 9.06 us, same error against float64).
__device__ __forceinline__ float exp_nonpos(float x) {
    const float hi = x * kLog2e;
    const float lo = fmaf(x, kLog2e, -hi) + x * 1.925963e-8f;  // log2(e) - fp32(log2(e)) = 1.925963e-8
    const float e = __builtin_amdgcn_exp2f(hi) * fmaf(lo, 0.69314718f, 1.0f);
    return x == -__builtin_inff() ? 0.0f : e;
}

// fp32 fixed-block attention on the bf16 matrix cores (head dims 32 and 64;
// at 128 its LDS tables would leave one workgroup per CU, and
// fixed_block_f32_mfma_kernel above measured faster).  Every fp32 operand x
// is split into three bf16 parts by truncation, x = hi + mid + lo (hi = x with
// the low 16 bits cleared, mid likewise of x - hi, lo = the rest, which has at
// most 8 significant bits: exact for |x| >= 2^-110, below which lo is an fp32
// denormal and its bf16 part loses at most 2^-133), and a product a.b is formed from the
// six terms whose weight is at least 2^-16 of a_hi.b_hi (mm, hl, lh, hm, mh,
// hh, smallest first), accumulated in fp32 by v_mfma_f32_16x16x32_bf16: six
// products at sixteen times the fp32 matrix rate.  The dropped terms (ml, lm,
// ll) weigh at most 2^-24 of a_hi.b_hi, about one fp32 rounding.
// Wave w owns queries 16w .. 16w+15 (lane column c = lane % 16, lane group
// g = lane / 16), as in fixed_block_f32_mfma_kernel:
//   S^T = K Q^T: k-step s contracts dims 32s + 8g .. +7 in lane group g; the
//     key parts are staged in LDS row-major, the query parts split in
//     registers; accumulator r of key tile n is key 16n + 4g + r.
//   O^T = V^T P^T: k-step j contracts keys 32j .. 32j+31, lane group g taking
//     keys 32j + 4g + (0..3) and 32j + 16 + 4g + (0..3) - exactly the
//     probabilities the lane holds in key tiles 2j and 2j + 1 - so the value
//     parts are staged transposed with the keys of each 32-key step in that
//     order (slot of key kk: 8 (kk/4 % 4) + 4 (kk/16) + kk % 4).
template <int D>
__global__ __launch_bounds__(256) void fixed_block_f32x3_kernel(View q, View k, View v, OutView o, int tokens,
                                                                int nblocks, float scale, int causal) {
    typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
    constexpr int KS = D / 32;      // 32-dim k-steps of the score products
    constexpr int MT = D / 16;      // 16-dim output tiles
    constexpr int kKRow = D + 8;    // LDS row of a key part (bf16)
    constexpr int kVRow = 64 + 8;   // LDS row of a transposed value part (bf16)
    constexpr int DG = D / 4;       // 4-dim groups of a row
    constexpr int TILES = 16 * DG;  // 4 keys x 4 dims staging tiles of the block
    __shared__ __attribute__((aligned(16))) __bf16 kp[3][64 * kKRow];
    __shared__ __attribute__((aligned(16))) __bf16 vp[3][D * kVRow];
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int w = t >> 6;
    const int c = lane & 15;
    const int g = lane >> 4;
    const int bh = blockIdx.x / nblocks;
    const int start = (blockIdx.x - bh * nblocks) * 64;
    const int len = min(64, tokens - start);
    auto at = [&](const View& x, int r) {
        return reinterpret_cast<const float*>(x.data) + x.row(bh, start + min(r, len - 1));
    };
    // exact three-way split by truncation
    auto split = [](float x, float& h, float& m, float& l) {
        h = __uint_as_float(__float_as_uint(x) & 0xffff0000u);
        const float r = x - h;
        m = __uint_as_float(__float_as_uint(r) & 0xffff0000u);
        l = r - m;
    };
    auto bf = [](float x) { return __builtin_bit_cast(__bf16, (unsigned short)(__float_as_uint(x) >> 16)); };

    // ---- staging: thread t stages 4 keys x 4 dims tiles (key group kg, dim group dg)
    for (int tile = t; tile < TILES; tile += 256) {
        const int kg = tile / DG;
        const int dg = tile - kg * DG;
        f32x4 xk[4], xv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            xk[r] = *reinterpret_cast<const f32x4*>(at(k, 4 * kg + r) + 4 * dg);
            xv[r] = *reinterpret_cast<const f32x4*>(at(v, 4 * kg + r) + 4 * dg);
        }
        // key parts row-major: 4 dims of each of the 4 keys
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            __bf16 ph[4], pm[4], pl[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float h, m, l;
                split(xk[r][e], h, m, l);
                ph[e] = bf(h); pm[e] = bf(m); pl[e] = bf(l);
            }
            const int off = (4 * kg + r) * kKRow + 4 * dg;
            typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
            *reinterpret_cast<bf16x4*>(&kp[0][off]) = bf16x4{ph[0], ph[1], ph[2], ph[3]};
            *reinterpret_cast<bf16x4*>(&kp[1][off]) = bf16x4{pm[0], pm[1], pm[2], pm[3]};
            *reinterpret_cast<bf16x4*>(&kp[2][off]) = bf16x4{pl[0], pl[1], pl[2], pl[3]};
        }
        // value parts transposed: 4 keys of each of the 4 dims, at the slots of
        // keys 4kg .. 4kg+3 (consecutive)
        const int kk = (4 * kg) & 31;
        const int slot = ((4 * kg) & ~31) + 8 * ((kk >> 2) & 3) + 4 * (kk >> 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            __bf16 ph[4], pm[4], pl[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float h, m, l;
                split(xv[r][e], h, m, l);
                ph[r] = bf(h); pm[r] = bf(m); pl[r] = bf(l);
            }
            const int off = (4 * dg + e) * kVRow + slot;
            typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
            *reinterpret_cast<bf16x4*>(&vp[0][off]) = bf16x4{ph[0], ph[1], ph[2], ph[3]};
            *reinterpret_cast<bf16x4*>(&vp[1][off]) = bf16x4{pm[0], pm[1], pm[2], pm[3]};
            *reinterpret_cast<bf16x4*>(&vp[2][off]) = bf16x4{pl[0], pl[1], pl[2], pl[3]};
        }
    }
    // ---- query parts: lane (c, g) holds dims 32s + 8g .. +7 of query 16w + c
    bf16x8 qh[KS], qm[KS], ql[KS];
    {
        const float* qr = at(q, 16 * w + c);
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const f32x4 a = *reinterpret_cast<const f32x4*>(qr + 32 * s + 8 * g);
            const f32x4 b = *reinterpret_cast<const f32x4*>(qr + 32 * s + 8 * g + 4);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                float h, m, l;
                split(e < 4 ? a[e] : b[e - 4], h, m, l);
                qh[s][e] = bf(h); qm[s][e] = bf(m); ql[s][e] = bf(l);
            }
        }
    }
    __syncthreads();

    auto kfrag = [&](int part, int n, int s) {
        return *reinterpret_cast<const bf16x8*>(&kp[part][(16 * n + c) * kKRow + 32 * s + 8 * g]);
    };
    f32x4 sacc[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) {
        sacc[n] = f32x4(0.0f);
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const bf16x8 kh = kfrag(0, n, s), km = kfrag(1, n, s), kl = kfrag(2, n, s);
            sacc[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(km, qm[s], sacc[n], 0, 0, 0);
            sacc[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh, ql[s], sacc[n], 0, 0, 0);
            sacc[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kl, qh[s], sacc[n], 0, 0, 0);
            sacc[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh, qm[s], sacc[n], 0, 0, 0);
            sacc[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(km, qh[s], sacc[n], 0, 0, 0);
            sacc[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh, qh[s], sacc[n], 0, 0, 0);
        }
    }

    // softmax of query column 16w + c (as fixed_block_f32_mfma_kernel)
    const int query = 16 * w + c;
    float mx = -__builtin_inff();
#pragma unroll
    for (int n = 0; n < 4; ++n)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int key = 16 * n + 4 * g + r;
            const bool dead = key >= len || (causal && key > query);
            sacc[n][r] = dead ? -__builtin_inff() : sacc[n][r] * scale;
            mx = fmaxf(mx, sacc[n][r]);
        }
    {
        const float2 p16 = pair_xor16(mx);
        mx = max_xor32(fmaxf(p16.x, p16.y));
    }
    const float m_use = (mx == -__builtin_inff()) ? 0.0f : mx;
    float sum = 0.0f;
#pragma unroll
    for (int n = 0; n < 4; ++n)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            sacc[n][r] = exp_nonpos(sacc[n][r] - m_use);
            sum += sacc[n][r];
        }
    sum = add_xor32(add_xor16(sum));
    const float inv = sum > 0.0f ? 1.0f / sum : __builtin_nanf("");
    // probability parts: k-step j takes key tiles 2j (slots 0-3) and 2j+1 (slots 4-7)
    bf16x8 ph[2], pm[2], pl[2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float h, m, l;
            split(sacc[2 * j + (e >> 2)][e & 3] * inv, h, m, l);
            ph[j][e] = bf(h); pm[j][e] = bf(m); pl[j][e] = bf(l);
        }
    auto vfrag = [&](int part, int mt, int j) {
        return *reinterpret_cast<const bf16x8*>(&vp[part][(16 * mt + c) * kVRow + 32 * j + 8 * g]);
    };
    f32x4 oacc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        oacc[mt] = f32x4(0.0f);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const bf16x8 vh = vfrag(0, mt, j), vm = vfrag(1, mt, j), vl = vfrag(2, mt, j);
            oacc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vm, pm[j], oacc[mt], 0, 0, 0);
            oacc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vh, pl[j], oacc[mt], 0, 0, 0);
            oacc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vl, ph[j], oacc[mt], 0, 0, 0);
            oacc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vh, pm[j], oacc[mt], 0, 0, 0);
            oacc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vm, ph[j], oacc[mt], 0, 0, 0);
            oacc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vh, ph[j], oacc[mt], 0, 0, 0);
        }
    }
    if (query >= len) return;
    // accumulator r of output tile mt is dim 16mt + 4g + r of query 16w + c
    float* dst = reinterpret_cast<float*>(o.data) + o.row(bh, start + query);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) *reinterpret_cast<f32x4*>(dst + 16 * mt + 4 * g) = oacc[mt];
}

template <typename T, int D>
static void launch_fixed_mfma(const View& q, const View& k, const View& v, const OutView& o, int tokens, int nblocks,
                              int bh_count, float scale, int causal, hipStream_t stream) {
    hipLaunchKernelGGL((fixed_block_mfma_kernel<T, D>), dim3(bh_count * nblocks), dim3(64), 0, stream, q, k, v, o,
                       tokens, nblocks, scale * kLog2e, causal);
}

template <int D>
static void launch_fixed_f32_mfma(const View& q, const View& k, const View& v, const OutView& o, int tokens,
                                  int nblocks, int bh_count, float scale, int causal, hipStream_t stream) {
    if constexpr (D <= 64)
        hipLaunchKernelGGL((fixed_block_f32x3_kernel<D>), dim3(bh_count * nblocks), dim3(256), 0, stream, q, k, v, o,
                           tokens, nblocks, scale, causal);
    else
        hipLaunchKernelGGL((fixed_block_f32_mfma_kernel<D>), dim3(bh_count * nblocks), dim3(256), 0, stream, q, k, v,
                           o, tokens, nblocks, scale, causal);
}

template <typename T>
int launch_fixed_t(int head_dim, const View& q, const View& k, const View& v, const OutView& o, int tokens,
                   int bh_count, float scale, int causal, const MaskView& mask, hipStream_t stream) {
    const int nblocks = (tokens + 63) / 64;
    const dim3 grid(bh_count * nblocks);
    auto aligned = [](const char* p, int64_t sb, int64_t sh, int64_t st, int bytes) {
        const int64_t unit = bytes / (int64_t)sizeof(T);
        return reinterpret_cast<uintptr_t>(p) % bytes == 0 && sb % unit == 0 && sh % unit == 0 && st % unit == 0;
    };
    // 16-byte row loads and stores need 16-byte aligned rows (the output of
    // the 16-bit kernel: 2 * head_dim / 32 bytes per store)
    const int out_bytes = std::is_same<T, float>::value ? 16 : 2 * head_dim / 32;
    const bool rows16 = aligned(q.data, q.sb, q.sh, q.st, 16) && aligned(k.data, k.sb, k.sh, k.st, 16) &&
                        aligned(v.data, v.sb, v.sh, v.st, 16) && aligned(o.data, o.sb, o.sh, o.st, out_bytes);
    if constexpr (std::is_same<T, float>::value) {
        if (mask.kind == PISA_MASK_NONE && rows16) {
            if (head_dim == 32) launch_fixed_f32_mfma<32>(q, k, v, o, tokens, nblocks, bh_count, scale, causal, stream);
            else if (head_dim == 64) launch_fixed_f32_mfma<64>(q, k, v, o, tokens, nblocks, bh_count, scale, causal, stream);
            else launch_fixed_f32_mfma<128>(q, k, v, o, tokens, nblocks, bh_count, scale, causal, stream);
            return pisa_host::check_launch("fixed_block_f32 kernel");
        }
    } else {
        if (mask.kind == PISA_MASK_NONE && rows16) {  // the reference's Triton path: no mask (dispatch.py:50-79)
            if (head_dim == 32) launch_fixed_mfma<T, 32>(q, k, v, o, tokens, nblocks, bh_count, scale, causal, stream);
            else if (head_dim == 64) launch_fixed_mfma<T, 64>(q, k, v, o, tokens, nblocks, bh_count, scale, causal, stream);
            else launch_fixed_mfma<T, 128>(q, k, v, o, tokens, nblocks, bh_count, scale, causal, stream);
            return pisa_host::check_launch("fixed_block_mfma_kernel");
        }
    }
    if (head_dim == 32)
        hipLaunchKernelGGL((fixed_block_kernel<T, 32>), grid, dim3(256), 0, stream, q, k, v, o, tokens, nblocks, scale,
                           causal, mask);
    else if (head_dim == 64)
        hipLaunchKernelGGL((fixed_block_kernel<T, 64>), grid, dim3(256), 0, stream, q, k, v, o, tokens, nblocks, scale,
                           causal, mask);
    else
        hipLaunchKernelGGL((fixed_block_kernel<T, 128>), grid, dim3(256), 0, stream, q, k, v, o, tokens, nblocks, scale,
                           causal, mask);
    return pisa_host::check_launch("fixed_block_kernel");
}

int launch_fixed_block(int dtype, int head_dim, const View& q, const View& k, const View& v, const OutView& o,
                       int tokens, int bh_count, float scale, int causal, const MaskView& mask, hipStream_t stream) {
    if (dtype == PISA_DTYPE_BF16)
        return launch_fixed_t<bf16_t>(head_dim, q, k, v, o, tokens, bh_count, scale, causal, mask, stream);
    if (dtype == PISA_DTYPE_F16)
        return launch_fixed_t<f16_t>(head_dim, q, k, v, o, tokens, bh_count, scale, causal, mask, stream);
    return launch_fixed_t<float>(head_dim, q, k, v, o, tokens, bh_count, scale, causal, mask, stream);
}

}  // namespace pisa
