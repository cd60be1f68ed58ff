// Fixed block-diagonal attention: every 64-token block attends only to itself.
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

template <typename T>
int launch_fixed_t(int head_dim, const View& q, const View& k, const View& v, const OutView& o, int tokens,
                   int bh_count, float scale, int causal, const MaskView& mask, hipStream_t stream) {
    const int nblocks = (tokens + 63) / 64;
    const dim3 grid(bh_count * nblocks);
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
