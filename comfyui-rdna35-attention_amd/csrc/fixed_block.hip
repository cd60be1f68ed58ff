// Fixed block-diagonal attention: every 64-token block attends only to itself.
//
// Two kernels.  bf16/fp16 calls without a mask run fixed_block_mfma_kernel
// (matrix cores, the reference's Triton semantics, below).  fp32 calls and
// masked calls - the ones the reference sends to its eager fp32 loop - run
// fixed_block_kernel:
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
// The block is staged in LDS - Q and K row-major, V transposed with its key
// index in swap23 order - and the products are formed transposed as in the
// attention kernels (S^T = K Q^T, O^T = V^T P^T), so a query is a lane column
// and the probabilities feed the second MFMA from their accumulator registers.
template <typename T, int D>
__global__ __launch_bounds__(64) void fixed_block_mfma_kernel(View q, View k, View v, OutView o, int tokens,
                                                               int nblocks, float scale_log2, int causal) {
    typedef typename Elem<T>::vec8 vec8;
    constexpr int KT = D / 16;      // 16-deep k-steps of the score product
    constexpr int MD = D / 32;      // 32-dim tiles of the output
    constexpr int P = D / 8;        // 16-byte pieces per row
    constexpr int kRow = D + 8;     // padded row (elements) of the row-major Q and K tiles
    constexpr int kVtRow = 64 + 8;  // padded row (elements) of the transposed V tile
    __shared__ __attribute__((aligned(16))) T q_lds[64 * kRow];
    __shared__ __attribute__((aligned(16))) T k_lds[64 * kRow];
    __shared__ __attribute__((aligned(16))) T vt_lds[D * kVtRow];
    const int lane = threadIdx.x;
    const int half = lane >> 5;
    const int col = lane & 31;
    const int bh = blockIdx.x / nblocks;
    const int start = (blockIdx.x - bh * nblocks) * 64;
    const int len = min(64, tokens - start);

    // ---- stage: piece id = row * P + pc (rows past len are zero)
    for (int id = lane; id < 64 * P; id += 64) {
        const int r = id / P;
        const int pc = id - r * P;
        const int tok = start + min(r, len - 1);
        vec8 xq = load8<vec8>(q.data + (q.row(bh, tok) + pc * 8) * (int64_t)sizeof(T));
        vec8 xk = load8<vec8>(k.data + (k.row(bh, tok) + pc * 8) * (int64_t)sizeof(T));
        vec8 xv = load8<vec8>(v.data + (v.row(bh, tok) + pc * 8) * (int64_t)sizeof(T));
        if (r >= len) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                xq[e] = T(0.0f);
                xk[e] = T(0.0f);
                xv[e] = T(0.0f);
            }
        }
        store8(&q_lds[r * kRow + pc * 8], xq);
        store8(&k_lds[r * kRow + pc * 8], xk);
        const int pos = swap23(r);
#pragma unroll
        for (int e = 0; e < 8; ++e) {  // rotated by the piece, so the 16 lanes of a row hit 16 banks
            const int ee = (e + pc) & 7;
            vt_lds[(pc * 8 + ee) * kVtRow + pos] = xv[ee];
        }
    }
    __syncthreads();

    // ---- S^T[key][query] for key tiles mt and query tiles nt
    f32x16 s[2][2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int e = 0; e < 16; ++e) s[mt][nt][e] = 0.0f;
#pragma unroll
    for (int t = 0; t < KT; ++t) {
        vec8 kf[2], qf[2];
#pragma unroll
        for (int x = 0; x < 2; ++x) {
            kf[x] = *reinterpret_cast<const vec8*>(&k_lds[(32 * x + col) * kRow + 16 * t + 8 * half]);
            qf[x] = *reinterpret_cast<const vec8*>(&q_lds[(32 * x + col) * kRow + 16 * t + 8 * half]);
        }
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) s[mt][nt] = mfma32(kf[mt], qf[nt], s[mt][nt]);
    }

    // ---- masking and the softmax of query column (nt, col), in log2 units:
    // accumulator v of tile mt is key 32mt + 8(v/4) + 4half + v%4
    typename Elem<T>::vec8 pf[2][2][2];  // [nt][mt][ss]: 8 probabilities, keys 16ss.. of tile mt in swap23 order
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

    // ---- O^T[dim][query] = sum_key V^T[dim][key] P^T[key][query]
    f32x16 acc[MD][2];
#pragma unroll
    for (int md = 0; md < MD; ++md)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[md][nt][e] = 0.0f;
#pragma unroll
    for (int md = 0; md < MD; ++md)
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int ss = 0; ss < 2; ++ss) {
                const vec8 vf = *reinterpret_cast<const vec8*>(
                    &vt_lds[(32 * md + col) * kVtRow + 32 * mt + 16 * ss + 8 * half]);
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) acc[md][nt] = mfma32(vf, pf[nt][mt][ss], acc[md][nt]);
            }

    // ---- store: accumulator v of tile md is dim 32md + 8(v/4) + 4half + v%4 of query 32nt + col
    typedef T vec4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const int query = 32 * nt + col;
        if (query >= len) continue;
        char* dst = o.data + o.row(bh, start + query) * (int64_t)sizeof(T);
#pragma unroll
        for (int md = 0; md < MD; ++md)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                vec4 x;
#pragma unroll
                for (int e = 0; e < 4; ++e) x[e] = from_f32<T>(acc[md][nt][4 * g + e]);
                *reinterpret_cast<vec4*>(dst + (32 * md + 8 * g + 4 * half) * sizeof(T)) = x;
            }
    }
}

template <typename T, int D>
static void launch_fixed_mfma(const View& q, const View& k, const View& v, const OutView& o, int tokens, int nblocks,
                              int bh_count, float scale, int causal, hipStream_t stream) {
    hipLaunchKernelGGL((fixed_block_mfma_kernel<T, D>), dim3(bh_count * nblocks), dim3(64), 0, stream, q, k, v, o,
                       tokens, nblocks, scale * kLog2e, causal);
}

template <typename T>
int launch_fixed_t(int head_dim, const View& q, const View& k, const View& v, const OutView& o, int tokens,
                   int bh_count, float scale, int causal, const MaskView& mask, hipStream_t stream) {
    const int nblocks = (tokens + 63) / 64;
    const dim3 grid(bh_count * nblocks);
    if constexpr (!std::is_same<T, float>::value) {
        // 16-byte row loads and 8-byte output stores need aligned rows
        auto aligned = [](const char* p, int64_t sb, int64_t sh, int64_t st, int bytes) {
            const int64_t unit = bytes / (int64_t)sizeof(T);
            return reinterpret_cast<uintptr_t>(p) % bytes == 0 && sb % unit == 0 && sh % unit == 0 && st % unit == 0;
        };
        const bool rows16 = aligned(q.data, q.sb, q.sh, q.st, 16) && aligned(k.data, k.sb, k.sh, k.st, 16) &&
                            aligned(v.data, v.sb, v.sh, v.st, 16) && aligned(o.data, o.sb, o.sh, o.st, 8);
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
