// Subsystems 3 and 4: exact attention on bf16/fp16 MFMA with the PISA tail,
// first-order correction and merge fused into the epilogue.
//
// One wavefront owns one 64-row query block (all four SIMDs of a CU run
// independent query blocks, 1 wave per SIMD, up to 512 registers each).  The
// wave keeps its query block in registers for the whole kernel and walks a
// list of 64-key chunks:
//   1. exact chunks: the key blocks the router selected (sparse) or every key
//      block (dense), K rows read straight from the caller's layout and the
//      transposed value block from the V^T table;
//   2. tail chunks (PISA only): the block centroids k_bar (dtype) as keys with
//      score bias ln(len_j), -inf for selected blocks, v_bar as values;
// accumulating one online softmax in fp32.  Scores are computed transposed,
//     S^T[key][query] = sum_d K[key][d] Q[query][d]          (32x32x16 MFMA)
// so that a query is a lane column: row maxima need one lane exchange, and
// the probabilities feed the second MFMA from their accumulator registers:
//     O^T[dim][query] += sum_key V^T[dim][key] P^T[key][query].
// The tail mass l_tail is tracked next to the total mass l, and the epilogue
// writes   out = O / l + C * l_tail / l,   C = s/T * q . dtype(H_sum),
// i.e. the LSE-weighted merge of the exact and tail softmaxes
// (__init__.py:310-316, fused kernel pisa_kernels.cu:296-340) and the
// first-order correction (__init__.py:281-282) in one pass, stored through the
// output view (raster order for the spatial layouts).
//
// Reference semantics: exact tile __init__.py:127-137,286-298; tail
// __init__.py:139-164 (score_mod: selected -> -inf, else + ln(len)); dense
// online softmax triton_kernel.py:113-160.
#include "kernels.hpp"

namespace pisa {


template <typename T, int D>
struct Wave {
    typedef typename Elem<T>::vec8 vec8;
    static constexpr int KT = D / 16;   // contraction steps over head_dim
    static constexpr int MD = D / 32;   // 32-row tiles of head_dim
};

// ---- one 64-key chunk: S^T = K Q^T, online softmax update, O^T += V^T P^T.
// `s` holds the raw scores on entry.  kind: 0 exact full chunk, 1 exact chunk
// with key bound, 2 tail chunk.
template <typename T, int D>
__device__ __forceinline__ void softmax_update(f32x16 (&s)[2][2], float (&m)[2], float (&l)[2],
                                               float (&lt)[2], f32x16 (&o)[D / 32][2], bool tail) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        float mx = -__builtin_inff();
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[mt][nt][v]);
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m[nt], mx);
        const float m_use = (m_new == -__builtin_inff()) ? 0.0f : m_new;
        const float alpha = __builtin_amdgcn_exp2f(m[nt] - m_use);
        m[nt] = m_new;
        float rs = 0.0f;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const float p = __builtin_amdgcn_exp2f(s[mt][nt][v] - m_use);
                s[mt][nt][v] = p;
                rs += p;
            }
        l[nt] = l[nt] * alpha + rs;
        lt[nt] = lt[nt] * alpha + (tail ? rs : 0.0f);
#pragma unroll
        for (int md = 0; md < D / 32; ++md)
#pragma unroll
            for (int v = 0; v < 16; ++v) o[md][nt][v] *= alpha;
    }
}

template <typename T, int D>
__device__ __forceinline__ void pv_update(const f32x16 (&p)[2][2],
                                          const typename Elem<T>::vec8 (&vf)[D / 32][4],
                                          f32x16 (&o)[D / 32][2]) {
    typedef typename Elem<T>::vec8 vec8;
    vec8 pf[2][4];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int ss = 0; ss < 2; ++ss)
#pragma unroll
                for (int j = 0; j < 8; ++j) pf[nt][mt * 2 + ss][j] = from_f32<T>(p[mt][nt][ss * 8 + j]);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int md = 0; md < D / 32; ++md)
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) o[md][nt] = mfma32(vf[md][ks], pf[nt][ks], o[md][nt]);
}

template <typename T, int D, bool SPARSE, bool TAIL>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(1, 1)))
void attention_kernel(AttnArgs a) {
    typedef typename Elem<T>::vec8 vec8;
    constexpr int KT = D / 16;
    constexpr int MD = D / 32;
    // Query fragments live in LDS, lane-private (lane l owns bytes [16l, 16l+16)
    // of every 1 KB row), so reads are conflict free and need no barrier.
    __shared__ __attribute__((aligned(16))) vec8 qs[2 * KT][64];
    const int lane = threadIdx.x;
    const int half = lane >> 5;
    const int col = lane & 31;
    const int work = xcd_remap(blockIdx.x, gridDim.x);
    const int bh = work / a.q_blocks;
    const int qb = work - bh * a.q_blocks;

    // ---- query block: qs[nt*KT+t][lane] = Q[qb*64+nt*32+col][t*16+half*8 .. +7]
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const int qrow = qb * kBlock + nt * 32 + col;
        const bool valid = qrow < a.q_tokens;
        const char* base = a.q.data + a.q.row(bh, a.qmap(valid ? qrow : 0)) * (int64_t)sizeof(T);
#pragma unroll
        for (int t = 0; t < KT; ++t) {
            vec8 x;
            if (valid) x = load8<vec8>(base + (t * 16 + half * 8) * sizeof(T));
            else
#pragma unroll
                for (int e = 0; e < 8; ++e) x[e] = T(0.0f);
            qs[nt * KT + t][lane] = x;
        }
    }

    f32x16 o[MD][2];
#pragma unroll
    for (int md = 0; md < MD; ++md)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int v = 0; v < 16; ++v) o[md][nt][v] = 0.0f;
    float m[2] = {-__builtin_inff(), -__builtin_inff()};
    float l[2] = {0.0f, 0.0f};
    float lt[2] = {0.0f, 0.0f};

    auto scores = [&](const vec8 (&kf)[2][KT], f32x16 (&s)[2][2]) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                for (int v = 0; v < 16; ++v) s[mt][nt][v] = 0.0f;
#pragma unroll
        for (int t = 0; t < KT; ++t) {
            const vec8 q0 = qs[t][lane];
            const vec8 q1 = qs[KT + t][lane];
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                s[mt][0] = mfma32(kf[mt][t], q0, s[mt][0]);
                s[mt][1] = mfma32(kf[mt][t], q1, s[mt][1]);
            }
        }
    };

    // ---- exact chunks
    const int n_exact = SPARSE ? a.exact : a.kv_blocks;
    const int32_t* my_idx = SPARSE ? a.idx + ((int64_t)bh * a.q_blocks + qb) * a.exact : nullptr;
    const char* vt_base = a.vt + (int64_t)bh * a.kv_blocks * D * kBlock * sizeof(T);

    auto load_k = [&](vec8 (&kf)[2][KT], int j) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            const int key = j * kBlock + mt * 32 + col;
            const bool valid = key < a.kv_tokens;
            const char* base = a.k.data + a.k.row(bh, a.kmap(valid ? key : 0)) * (int64_t)sizeof(T);
#pragma unroll
            for (int t = 0; t < KT; ++t) {
                if (valid) kf[mt][t] = load8<vec8>(base + (t * 16 + half * 8) * sizeof(T));
                else
#pragma unroll
                    for (int e = 0; e < 8; ++e) kf[mt][t][e] = T(0.0f);
            }
        }
    };

    vec8 kf[2][KT];
    if (n_exact > 0) load_k(kf, SPARSE ? my_idx[0] : 0);
    for (int n = 0; n < n_exact; ++n) {
        // Compiler barrier: keeps the query fragments in LDS instead of letting
        // them be hoisted into (and exhaust) the register file.
        asm volatile("" ::: "memory");
        const int j = SPARSE ? my_idx[n] : n;
        vec8 vf[MD][4];
        const char* vb = vt_base + (int64_t)j * D * kBlock * sizeof(T);
#pragma unroll
        for (int md = 0; md < MD; ++md)
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
                vf[md][ks] = load8<vec8>(vb + ((md * 32 + col) * kBlock + ks * 16 + half * 8) * sizeof(T));

        f32x16 s[2][2];
        scores(kf, s);
        const bool bounded = (j + 1) * kBlock > a.kv_tokens;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int key = j * kBlock + mt * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
                    const float x = s[mt][nt][v] * a.scale_log2;
                    s[mt][nt][v] = (bounded && key >= a.kv_tokens) ? -__builtin_inff() : x;
                }
        softmax_update<T, D>(s, m, l, lt, o, false);
        if (n + 1 < n_exact) load_k(kf, SPARSE ? my_idx[n + 1] : n + 1);
        pv_update<T, D>(s, vf, o);
    }

    // ---- tail chunks over the block centroids
    if (TAIL) {
        const uint32_t* mask = a.selmask + ((int64_t)bh * a.q_blocks + qb) * a.mask_words;
        const char* kbar = a.kbar + (int64_t)bh * a.npad * D * sizeof(T);
        const char* vbt = a.vbar_t + (int64_t)bh * D * a.npad * sizeof(T);
        for (int c = 0; c < a.npad / kBlock; ++c) {
            asm volatile("" ::: "memory");
            vec8 cf[2][KT];
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int t = 0; t < KT; ++t)
                    cf[mt][t] = load8<vec8>(kbar + ((int64_t)(c * kBlock + mt * 32 + col) * D + t * 16 + half * 8) * sizeof(T));
            vec8 vf[MD][4];
#pragma unroll
            for (int md = 0; md < MD; ++md)
#pragma unroll
                for (int ks = 0; ks < 4; ++ks)
                    vf[md][ks] = load8<vec8>(vbt + ((int64_t)(md * 32 + col) * a.npad + c * kBlock + ks * 16 + half * 8) * sizeof(T));
            f32x16 s[2][2];
            scores(cf, s);
            // centroid jc = 64c + 32mt + bit lives in selection word 2c + mt (wave uniform)
            uint32_t words[2];
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) words[mt] = (2 * c + mt < a.mask_words) ? mask[2 * c + mt] : 0u;
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int bit = 8 * (v >> 2) + 4 * half + (v & 3);
                    const int jc = c * kBlock + mt * 32 + bit;
                    const bool dead = jc >= a.centroids || ((words[mt] >> bit) & 1u);
                    const float bias = (jc == a.centroids - 1) ? a.last_len_log2 : 6.0f;  // log2(64)
#pragma unroll
                    for (int nt = 0; nt < 2; ++nt) {
                        const float x = s[mt][nt][v] * a.scale_log2 + bias;
                        s[mt][nt][v] = dead ? -__builtin_inff() : x;
                    }
                }
            softmax_update<T, D>(s, m, l, lt, o, true);
            pv_update<T, D>(s, vf, o);
        }
    }

    // ---- epilogue: normalise, add the first-order correction one 32-dim
    // tile at a time (keeps only 32 extra accumulators live), store
    float inv[2], wa[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const float lf = l[nt] + __shfl_xor(l[nt], 32);
        const float ltf = lt[nt] + __shfl_xor(lt[nt], 32);
        inv[nt] = 1.0f / lf;
        wa[nt] = ltf * inv[nt] * a.corr_scale;
    }
    const bool first_order = TAIL && a.ht != nullptr;
    const char* ht = first_order ? a.ht + (int64_t)bh * D * D * sizeof(T) : nullptr;
    char* obase[2];
    bool ovalid[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const int qrow = qb * kBlock + nt * 32 + col;
        ovalid[nt] = qrow < a.q_tokens;
        obase[nt] = a.o.data + a.o.row(bh, a.qmap(ovalid[nt] ? qrow : 0)) * (int64_t)sizeof(T);
    }
    typedef T vec4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int md = 0; md < MD; ++md) {
        asm volatile("" ::: "memory");
        f32x16 corr[2];
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int v = 0; v < 16; ++v) corr[nt][v] = 0.0f;
        if (first_order) {
#pragma unroll
            for (int t = 0; t < KT; ++t) {
                const vec8 hf = load8<vec8>(ht + ((md * 32 + col) * D + t * 16 + half * 8) * sizeof(T));
                corr[0] = mfma32(hf, qs[t][lane], corr[0]);
                corr[1] = mfma32(hf, qs[KT + t][lane], corr[1]);
            }
        }
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            if (!ovalid[nt]) continue;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                vec4 out;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float x = o[md][nt][4 * g + e] * inv[nt];
                    if (first_order) x += corr[nt][4 * g + e] * wa[nt];
                    out[e] = from_f32<T>(x);
                }
                *reinterpret_cast<vec4*>(obase[nt] + (md * 32 + 8 * g + 4 * half) * sizeof(T)) = out;
            }
        }
    }
}

// ---- transposed V blocks for dense attention: [BH][nblk][D][64], swap23 keys
template <typename T, int D>
__global__ __launch_bounds__(256) void vt_pack_kernel(View v, int kv_tokens, int kv_blocks, char* vt) {
    typedef typename Elem<T>::vec8 vec8;
    typedef T vec4 __attribute__((ext_vector_type(4)));
    constexpr int kRow = kBlock + 8;
    __shared__ __attribute__((aligned(16))) T lds[D * kRow];
    const int t = threadIdx.x;
    const int bh = blockIdx.x / kv_blocks;
    const int j = blockIdx.x - bh * kv_blocks;
    constexpr int kChunks = D / 8;            // 16-byte pieces per row
    constexpr int kRowsPerPass = 256 / kChunks;
    const int c = t % kChunks;
    const int r0 = t / kChunks;
    for (int r = r0 * 4; r < kBlock; r += kRowsPerPass * 4) {
        vec8 x[4];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const int key = j * kBlock + r + rr;
            if (key < kv_tokens) x[rr] = load8<vec8>(v.data + (v.row(bh, key) + c * 8) * sizeof(T));
            else
#pragma unroll
                for (int e = 0; e < 8; ++e) x[rr][e] = T(0.0f);
        }
        const int p = swap23(r);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            vec4 w = {x[0][e], x[1][e], x[2][e], x[3][e]};
            *reinterpret_cast<vec4*>(&lds[(c * 8 + e) * kRow + p]) = w;
        }
    }
    __syncthreads();
    T* dst = reinterpret_cast<T*>(vt) + ((int64_t)bh * kv_blocks + j) * D * kBlock;
    for (int id = t; id < D * 8; id += 256) {
        const int d = id >> 3;
        const int pc = id & 7;
        store8(dst + d * kBlock + pc * 8, *reinterpret_cast<const vec8*>(&lds[d * kRow + pc * 8]));
    }
}

template <typename T, int D, bool SPARSE, bool TAIL>
int launch_attention_t(const AttnArgs& a, int bh_count, hipStream_t stream) {
    const int waves = bh_count * a.q_blocks;
    hipLaunchKernelGGL((attention_kernel<T, D, SPARSE, TAIL>), dim3(waves), dim3(64), 0, stream, a);
    return pisa_host::check_launch("attention_kernel");
}

int launch_attention(int dtype, int head_dim, bool sparse, bool tail, const AttnArgs& a, int bh_count,
                     hipStream_t stream) {
    if (dtype == PISA_DTYPE_BF16) {
        if (head_dim == 128) {
            if (sparse) return tail ? launch_attention_t<bf16_t, 128, true, true>(a, bh_count, stream)
                                    : launch_attention_t<bf16_t, 128, true, false>(a, bh_count, stream);
            return tail ? launch_attention_t<bf16_t, 128, false, true>(a, bh_count, stream)
                        : launch_attention_t<bf16_t, 128, false, false>(a, bh_count, stream);
        }
        return launch_attention_t<bf16_t, 64, false, false>(a, bh_count, stream);
    }
    if (head_dim == 128) {
        if (sparse) return tail ? launch_attention_t<f16_t, 128, true, true>(a, bh_count, stream)
                                : launch_attention_t<f16_t, 128, true, false>(a, bh_count, stream);
        return tail ? launch_attention_t<f16_t, 128, false, true>(a, bh_count, stream)
                    : launch_attention_t<f16_t, 128, false, false>(a, bh_count, stream);
    }
    return launch_attention_t<f16_t, 64, false, false>(a, bh_count, stream);
}

int launch_vt_pack(int dtype, int head_dim, const View& v, int kv_tokens, int kv_blocks, int bh_count,
                   char* vt, hipStream_t stream) {
    const dim3 grid(bh_count * kv_blocks);
    if (dtype == PISA_DTYPE_BF16) {
        if (head_dim == 128) hipLaunchKernelGGL((vt_pack_kernel<bf16_t, 128>), grid, dim3(256), 0, stream, v, kv_tokens, kv_blocks, vt);
        else hipLaunchKernelGGL((vt_pack_kernel<bf16_t, 64>), grid, dim3(256), 0, stream, v, kv_tokens, kv_blocks, vt);
    } else {
        if (head_dim == 128) hipLaunchKernelGGL((vt_pack_kernel<f16_t, 128>), grid, dim3(256), 0, stream, v, kv_tokens, kv_blocks, vt);
        else hipLaunchKernelGGL((vt_pack_kernel<f16_t, 64>), grid, dim3(256), 0, stream, v, kv_tokens, kv_blocks, vt);
    }
    return pisa_host::check_launch("vt_pack_kernel");
}

}  // namespace pisa
