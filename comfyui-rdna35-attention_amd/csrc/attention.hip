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

constexpr float kLazyRescale = 8.0f;  // log2 headroom before the running max is moved

// Online-softmax update of one 64-key chunk held transposed in `s`
// (s[mt][nt][v] = score of key 32mt + 8(v/4) + 4half + v%4, query 32nt + col).
// `c` converts raw scores to the log2 domain (c = scale*log2(e) for exact
// chunks, 1 for tail chunks whose scores are pre-converted).  The running max
// only moves when a column's chunk max exceeds it by kLazyRescale, so the
// O rescale (128 accumulators) runs on the first chunk and rarely after;
// probabilities are then bounded by 2^kLazyRescale, well inside bf16/fp32.
template <typename T, int D>
__device__ __forceinline__ void softmax_update(f32x16 (&s)[2][2], float (&m)[2], float (&l)[2], float (&lt)[2],
                                               f32x16 (&o)[D / 32][2], float c, bool tail) {
    float mx[2];
    bool need[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        float x = -__builtin_inff();
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int v = 0; v < 16; ++v) x = fmaxf(x, s[mt][nt][v]);
        x = fmaxf(x, __shfl_xor(x, 32));
        mx[nt] = x * c;
        need[nt] = mx[nt] > m[nt] + kLazyRescale;
    }
    if (__any(need[0] || need[1])) {
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            const float alpha = need[nt] ? __builtin_amdgcn_exp2f(m[nt] - mx[nt]) : 1.0f;
            m[nt] = need[nt] ? mx[nt] : m[nt];
            l[nt] *= alpha;
            lt[nt] *= alpha;
#pragma unroll
            for (int md = 0; md < D / 32; ++md)
#pragma unroll
                for (int v = 0; v < 16; ++v) o[md][nt][v] *= alpha;
        }
    }
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const float neg_m = (m[nt] == -__builtin_inff()) ? 0.0f : -m[nt];
        float rs = 0.0f;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const float p = __builtin_amdgcn_exp2f(fmaf(s[mt][nt][v], c, neg_m));
                s[mt][nt][v] = p;
                rs += p;
            }
        l[nt] += rs;
        if (tail) lt[nt] += rs;
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
    const float c = a.scale_log2;

    // Token of row r of block j is block_base(j) + intra_offset(r): the lane
    // offsets are fixed, the block base is one scalar computation per block.
    const int q_off[2] = {a.qmap.intra_offset(col), a.qmap.intra_offset(32 + col)};
    const int k_off[2] = {a.kmap.intra_offset(col), a.kmap.intra_offset(32 + col)};
    const char* q_head = a.q.data + a.q.row(bh, 0) * (int64_t)sizeof(T) + half * 16;
    const char* k_head = a.k.data + a.k.row(bh, 0) * (int64_t)sizeof(T) + half * 16;

    // ---- query block: qs[nt*KT+t][lane] = Q[qb*64+nt*32+col][t*16+half*8 .. +7]
    {
        const int base = a.qmap.block_base(qb);
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            const int tok = min(base + q_off[nt], a.q_tokens - 1);  // rows past the end are never stored
            const char* p = q_head + (int64_t)tok * a.q.st * (int64_t)sizeof(T);
#pragma unroll
            for (int t = 0; t < KT; ++t) qs[nt * KT + t][lane] = load8<vec8>(p + t * 32);
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

    // Keys past the end of the sequence read the last row (a valid address);
    // their scores are masked below and their V^T columns are zero.
    auto load_k = [&](vec8 (&kf)[2][KT], int j) {
        const int base = a.kmap.block_base(j);
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            const int tok = min(base + k_off[mt], a.kv_tokens - 1);
            const char* p = k_head + (int64_t)tok * a.k.st * (int64_t)sizeof(T);
#pragma unroll
            for (int t = 0; t < KT; ++t) kf[mt][t] = load8<vec8>(p + t * 32);
        }
    };

    // ---- exact chunks
    const int n_exact = SPARSE ? a.exact : a.kv_blocks;
    const int32_t* my_idx = SPARSE ? a.idx + ((int64_t)bh * a.q_blocks + qb) * a.exact : nullptr;
    const char* vt_base = a.vt + (int64_t)bh * a.kv_blocks * D * kBlock * sizeof(T) +
                          ((int64_t)col * kBlock + half * 8) * sizeof(T);

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
                vf[md][ks] = load8<vec8>(vb + (md * 32 * kBlock + ks * 16) * sizeof(T));

        f32x16 s[2][2];
        scores(kf, s);
        if (n + 1 < n_exact) load_k(kf, SPARSE ? my_idx[n + 1] : n + 1);

        if ((j + 1) * kBlock > a.kv_tokens) {  // wave-uniform: only a short last block
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int key = j * kBlock + mt * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
                    if (key >= a.kv_tokens) {
                        s[mt][0][v] = -__builtin_inff();
                        s[mt][1][v] = -__builtin_inff();
                    }
                }
        }
        softmax_update<T, D>(s, m, l, lt, o, c, false);
        pv_update<T, D>(s, vf, o);
    }

    // ---- tail chunks over the block centroids
    if (TAIL) {
        const uint32_t* mask = a.selmask + ((int64_t)bh * a.q_blocks + qb) * a.mask_words;
        const char* kbar = a.kbar + ((int64_t)bh * a.npad * D + half * 8) * sizeof(T);
        const char* vbt = a.vbar_t + ((int64_t)bh * D * a.npad + (int64_t)col * a.npad + half * 8) * sizeof(T);
        for (int cb = 0; cb < a.npad / kBlock; ++cb) {
            asm volatile("" ::: "memory");
            vec8 cf[2][KT];
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int t = 0; t < KT; ++t)
                    cf[mt][t] = load8<vec8>(kbar + ((int64_t)(cb * kBlock + mt * 32 + col) * D + t * 16) * sizeof(T));
            vec8 vf[MD][4];
#pragma unroll
            for (int md = 0; md < MD; ++md)
#pragma unroll
                for (int ks = 0; ks < 4; ++ks)
                    vf[md][ks] = load8<vec8>(vbt + ((int64_t)md * 32 * a.npad + cb * kBlock + ks * 16) * sizeof(T));
            f32x16 s[2][2];
            scores(cf, s);
            // centroid jc = 64cb + 32mt + bit lives in selection word 2cb + mt (wave uniform)
            uint32_t words[2];
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) words[mt] = (2 * cb + mt < a.mask_words) ? mask[2 * cb + mt] : 0u;
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int bit = 8 * (v >> 2) + 4 * half + (v & 3);
                    const int jc = cb * kBlock + mt * 32 + bit;
                    const bool dead = jc >= a.centroids || ((words[mt] >> bit) & 1u);
                    const float bias = (jc == a.centroids - 1) ? a.last_len_log2 : 6.0f;  // log2(64)
#pragma unroll
                    for (int nt = 0; nt < 2; ++nt)
                        s[mt][nt][v] = dead ? -__builtin_inff() : fmaf(s[mt][nt][v], c, bias);
                }
            softmax_update<T, D>(s, m, l, lt, o, 1.0f, true);
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
    const char* ht = first_order ? a.ht + ((int64_t)bh * D * D + (int64_t)col * D + half * 8) * sizeof(T) : nullptr;
    char* obase[2];
    bool ovalid[2];
    {
        const int base = a.qmap.block_base(qb);
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            const int tok = base + q_off[nt];
            ovalid[nt] = tok < a.q_tokens;
            obase[nt] = a.o.data + a.o.row(bh, ovalid[nt] ? tok : 0) * (int64_t)sizeof(T);
        }
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
                const vec8 hf = load8<vec8>(ht + (md * 32 * D + t * 16) * sizeof(T));
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
