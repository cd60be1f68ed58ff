// Exact attention on bf16/fp16 MFMA with the PISA tail, first-order
// correction and merge fused into the epilogue.
//
// One wavefront owns one 64-row query block (all four SIMDs of a CU run
// independent query blocks, 1 wave per SIMD, up to 512 registers each; at
// padded head dims above 128 two waves split the block into 32-row halves).
// At head dim 128 the waves are persistent (attention_persistent_kernel) and
// copy the next block's first operands to LDS while the current one runs.
// The wave keeps its query rows in registers for the whole kernel and walks
// one list of 64-key chunks, with the operands of chunk c+1 in flight while
// chunk c is computed:
//   1. exact chunks: the key blocks the router selected (sparse) or every key
//      block (dense);
//   2. tail chunks (PISA only): the block centroids k_bar (dtype) as keys with
//      score bias ln(len_j), -inf for selected blocks, v_bar as values;
// accumulating one online softmax in fp32.  Every chunk is read from a packed
// table (kfrag_elem / vfrag_elem order: one coalesced 1 KB load per MFMA
// operand fragment) written by the statistics kernel or kv_pack_kernel.
// Scores are computed transposed,
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
#include <type_traits>

#include "kernels.hpp"

namespace pisa {

constexpr float kLazyRescale = 8.0f;  // log2 headroom before the running max is moved

// Sum of the 8 elements of a packed operand, fp32 accumulation (v_dot2 with ones).
__device__ __forceinline__ float sum8(bf16x8 x, float acc) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(x, x, 0, 1), one, acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(x, x, 2, 3), one, acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(x, x, 4, 5), one, acc, false);
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(x, x, 6, 7), one, acc, false);
}
__device__ __forceinline__ float sum8(f16x8 x, float acc) {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
    acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(x, x, 0, 1), one, acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(x, x, 2, 3), one, acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(x, x, 4, 5), one, acc, false);
    return __builtin_amdgcn_fdot2(__builtin_shufflevector(x, x, 6, 7), one, acc, false);
}

// The chunk loop works on 32-key half chunks.  One straight-line region per
// half h issues the 16 score MFMAs of half h+1 interleaved with the
// exponentials of half h, then the 16 PV MFMAs of half h interleaved with the
// operand loads of the next chunk and with the masking and column maxima of
// half h+1 (whose scores are ready by then); only the rare running-max move
// branches, after the region.  VALU, memory and MFMA work of the one wave on
// the SIMD thus overlap.

// Column maxima of half-chunk scores s[nt] (s[nt][v] = score of key
// 8(v/4) + 4half + v%4 of the half, query tile nt, column col) in log2 units
// (`c` converts the scores to them).  IEEE `maximum` (NaN-propagating) is
// v_maximum3_f32, two scores per instruction with no canonicalising of the
// MFMA results that fmaxf needs first (12 fewer VALU instructions per half
// chunk at NT = 2).  A NaN score makes its column's output NaN either way: its
// probability is NaN whatever the running max is.
// With two tiles, one swap of the lanes' partial maxima leaves lanes 0-31 with
// both halves' values of tile 0 and lanes 32-63 with those of tile 1; their
// maximum, swapped with itself, gives every lane both column maxima.
template <int NT>
__device__ __forceinline__ void half_max(const f32x16 (&s)[NT], float c, float (&mx)[NT]) {
    float x[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        x[nt] = s[nt][0];
#pragma unroll
        for (int v = 1; v < 16; ++v) x[nt] = __builtin_elementwise_maximum(x[nt], s[nt][v]);
    }
    if constexpr (NT == 2) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x[0]), __float_as_uint(x[1]), false, false);
        const float both = __builtin_elementwise_maximum(__uint_as_float(r[0]), __uint_as_float(r[1]));
        const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(both), __float_as_uint(both), false, false);
        mx[0] = __uint_as_float(b[0]) * c;
        mx[1] = __uint_as_float(b[1]) * c;
    } else {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const float2 p = pair_xor32(x[nt]);
            mx[nt] = __builtin_elementwise_maximum(p.x, p.y) * c;
        }
    }
}

// Running-max update from the column maxima mx of the next half.  The running
// max only moves when a column's max exceeds it by kLazyRescale, so the O
// rescale runs on the first half chunk and rarely after; probabilities stay
// below 2^kLazyRescale.  `enable` false (scores past the last chunk) leaves
// the state unchanged.  The running max m of a column is held as the two
// values the per-half code uses, both set only when m moves: nm = -m (0 while
// m = -inf: the exponent offset of the probabilities) and mth = m +
// kLazyRescale (the threshold, -inf while m = -inf).  -nm is m exactly, so
// every decision is the one m itself would give, and so is the factor
// 2^(m - mx) < 2^-kLazyRescale of a finite m; while m = -inf, l and O are
// still zero, and min(., 0) keeps the factor finite (no 0 * inf).
template <int NT, int MD>
__device__ __forceinline__ void rescale_to(const float (&mx)[NT], bool enable, float (&nm)[NT], float (&mth)[NT],
                                          float (&l)[NT], float (&lt)[NT], f32x16 (&o)[MD][NT]) {
    bool need[NT];
    bool any_need = false;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        need[nt] = enable && mx[nt] > mth[nt];
        any_need = any_need || need[nt];
    }
    if (__any(any_need)) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const float alpha = need[nt] ? __builtin_amdgcn_exp2f(fminf(-nm[nt] - mx[nt], 0.0f)) : 1.0f;
            nm[nt] = need[nt] ? -mx[nt] : nm[nt];
            mth[nt] = need[nt] ? mx[nt] + kLazyRescale : mth[nt];
            l[nt] *= alpha;
            lt[nt] *= alpha;
#pragma unroll
            for (int md = 0; md < MD; ++md)
#pragma unroll
                for (int v = 0; v < 16; ++v) o[md][nt][v] *= alpha;
        }
    }
}

// Probabilities of a half chunk as packed PV operands pf[nt][ss] (keys
// 16ss .. 16ss+15 of the half in swap23 order, which is the accumulator row
// order), and their masses: l (and lt for tail chunks) sum the rounded
// probabilities the PV product uses, so every output row's weights sum to 1.
// Exact chunks accumulate straight into l; tail chunks form the half's sum
// first, which goes to both l and lt.
template <typename T, int NT>
__device__ __forceinline__ void probs_half(const f32x16 (&s)[NT], float c, const float (&nm)[NT], float (&l)[NT],
                                           float (&lt)[NT], bool tail, typename Elem<T>::vec8 (&pf)[NT][2]) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const float neg_m = nm[nt];
        float rs = tail ? 0.0f : l[nt];
#pragma unroll
        for (int ss = 0; ss < 2; ++ss) {
            typename Elem<T>::vec8 p;
#pragma unroll
            for (int e = 0; e < 8; ++e) p[e] = from_f32<T>(__builtin_amdgcn_exp2f(fmaf(s[nt][ss * 8 + e], c, neg_m)));
            pf[nt][ss] = p;
            rs = sum8(p, rs);
        }
        l[nt] = tail ? l[nt] + rs : rs;
        lt[nt] = tail ? lt[nt] + rs : lt[nt];
    }
}

// The block a persistent wave runs next (nt = 0: none): its query rows (and,
// in the dense kernel, its first chunk) are copied to the wave's LDS while the
// current block runs.
// Chunk-step kinds of the attention loop (see check_half / chunk_step).
constexpr int kStepGeneral = 0, kStepExact = 1, kStepTail = 2;

struct NextBlock {
    int bh, qb, sub, nt;
};
typedef __attribute__((address_space(3))) char lds_char;

// Direct-to-LDS copy of 16 bytes per lane: lane l's 16 bytes at gptr land at
// LDS byte address lds_base + 16 l.  Written as inline asm so that the
// compiler's memory-counter bookkeeping does not model it (it would fall back
// to full waits in the chunk loop); its counts then include fewer operations
// than are in flight, which only makes its waits stricter, and the callers
// order the copy with explicit waits.
// M0 (the LDS base of the copy) is reserved by the compiler, which warns about
// clobbering it; no other code in these kernels uses M0.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_copy16(const void* gptr, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :
                 : "v"(gptr), "s"(lds_base)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

// D is the padded head dim (padded_head_dim); a.head_dim <= D is the real
// one.  A wave holds NT 32-row query tiles of query block qb of head bh, rows
// 32(sub + nt) + col: both tiles of the 64-row block (NT = 2, sub = 0) up to
// D = 128, or one tile (NT = 1, sub = 0 or 1, two waves per block) above,
// where the accumulators and operands of 64 rows would not fit the 512
// registers, and for the split blocks of the last round (attention_kernel).
template <typename T, int D, int NT, bool SPARSE, bool TAIL, bool PERSIST = false>
__device__ __forceinline__ void attention_block(const AttnArgs& a, int bh, int qb, int sub,
                                                const int32_t* __restrict__ sel,
                                                const uint32_t* __restrict__ selmask,
                                                lds_char* lds = nullptr, bool from_lds = false,
                                                NextBlock next = NextBlock{0, 0, 0, 0}) {
    static_assert(D % 32 == 0 && D <= 256, "padded head dim");
    static_assert(NT == 1 || (NT == 2 && D <= 128), "query tiles per wave");
    typedef typename Elem<T>::vec8 vec8;
    constexpr int KT = D / 16;
    constexpr int MD = D / 32;
    constexpr int64_t kBlockBytes = (int64_t)D * kBlock * sizeof(T);
    int lane_id = threadIdx.x;
    // a persistent wave re-derives its lane terms per block rather than holding
    // every lane-dependent offset in registers across blocks
    if constexpr (PERSIST) asm volatile("" : "+v"(lane_id));
    const int lane = lane_id;
    const int half = lane >> 5;
    const int col = lane & 31;
    const float c = a.scale_log2;
    const bool all_dims = a.head_dim >= D;  // else dims past the real head dim read as zero

    // Token of row r of block j is block_base(j) + intra_offset(r); this
    // wave's rows are 32(sub + nt) + col.
    int q_off[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) q_off[nt] = a.qmap.intra_offset(32 * (sub + nt) + col);

    // ---- query rows: qreg[nt][t] = Q[row nt][t*16+half*8 .. +7] (zero past
    // the real head dim), kept in registers for the whole kernel.  At D = 256
    // (QLDS) the fragments go to this wave's LDS (`lds`, 16 KB, fragment t at
    // byte 1024 t, lane l's 16 bytes at 16 l) and each score MFMA reads its
    // fragment there: with 64 registers of query fragments the kernel needs
    // more than 512 registers and spills, and the register allocator has
    // rebuilt a spilled fragment wrongly inside the chunk loop (one of its four
    // dwords taken from the previous iteration's scores).
    constexpr bool QLDS = D > 192 && !PERSIST;
    vec8 qreg[NT][KT];
    auto q_lds = [&](int t) {
        return reinterpret_cast<__attribute__((address_space(3))) u32x4*>(lds + t * 1024 + lane * 16);
    };
    if (PERSIST && from_lds) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int t = 0; t < KT; ++t)
                qreg[nt][t] = __builtin_bit_cast(
                    vec8, *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(
                              lds + (nt * KT + t) * 1024 + lane * 16));
    } else {
        const char* q_head = a.q.data + a.q.row(bh, 0) * (int64_t)sizeof(T) + half * 16;
        const int base = a.qmap.block_base(qb);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const int tok = min(base + q_off[nt], a.q_tokens - 1);  // rows past the end are never stored
            const char* p = q_head + (int64_t)tok * a.q.st * (int64_t)sizeof(T);
#pragma unroll
            for (int t = 0; t < KT; ++t) {
                if (all_dims || t * 16 + half * 8 < a.head_dim) {
                    qreg[nt][t] = load8<vec8>(p + t * 32);
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) qreg[nt][t][e] = T(0.0f);
                }
                if constexpr (QLDS) *q_lds(t) = __builtin_bit_cast(u32x4, qreg[nt][t]);
            }
        }
    }
    // query fragment t of tile nt for the score MFMAs; `qoff` is this lane's
    // byte offset lane * 16, passed through an empty asm once per half chunk so
    // that the LDS reads stay inside the chunk loop (hoisted out of it, they
    // would hold the fragments in registers again)
    auto qfrag = [&](int nt, int t, uint32_t qoff) -> vec8 {
        if constexpr (QLDS)
            return __builtin_bit_cast(
                vec8, *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(lds + t * 1024 + qoff));
        return qreg[nt][t];
    };
    // Pins the query fragments to AGPRs (an empty asm with an "a" operand):
    // the architectural VGPRs hold O, S and P, and leaving the choice to the
    // register allocator makes it copy fragments between the two files.
    // MFMA reads its B operand from AGPRs directly.
    auto pin_q = [&]() {
        if constexpr (QLDS) return;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int t = 0; t < KT; ++t) {
                f32x4 x = __builtin_bit_cast(f32x4, qreg[nt][t]);
                asm volatile("" : "+a"(x));
                qreg[nt][t] = __builtin_bit_cast(vec8, x);
            }
    };

    f32x16 o[MD][NT];
#pragma unroll
    for (int md = 0; md < MD; ++md)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int v = 0; v < 16; ++v) o[md][nt][v] = 0.0f;
    float nm[NT], mth[NT], l[NT], lt[NT];  // running max as -m and m + kLazyRescale (rescale_to)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        nm[nt] = 0.0f;
        mth[nt] = -__builtin_inff();
        l[nt] = 0.0f;
        lt[nt] = 0.0f;
    }

    // ---- chunk list: [0, n_exact) exact blocks, [n_exact, n_chunks) centroid chunks
    const int n_exact = SPARSE ? a.exact : a.kv_blocks;
    const int n_chunks = n_exact + (TAIL ? a.npad / kBlock : 0);
    const int32_t* my_idx = SPARSE ? sel + ((int64_t)bh * a.q_blocks + qb) * a.exact : nullptr;
    const uint32_t* my_mask = TAIL ? selmask + ((int64_t)bh * a.q_blocks + qb) * a.mask_words : nullptr;
    // Packed tables of this head as buffer resources: a chunk is addressed by a
    // wave-uniform byte offset (scalar arithmetic), the lane part is a fixed
    // vector offset, and reads past a table return zero.
    constexpr int kRawFlags = 0x00020000;  // untyped 32-bit data format
    const int tab_bytes = a.kv_blocks * (int)kBlockBytes;
    const __amdgpu_buffer_rsrc_t kp_rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.kp + (int64_t)bh * a.kv_blocks * kBlockBytes), (short)0, tab_bytes, kRawFlags);
    const __amdgpu_buffer_rsrc_t vp_rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.vp + (int64_t)bh * a.kv_blocks * kBlockBytes), (short)0, tab_bytes, kRawFlags);
    const int cen_bytes = TAIL ? a.npad * D * (int)sizeof(T) : 0;
    const __amdgpu_buffer_rsrc_t kc_rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(TAIL ? a.kbar + (int64_t)bh * a.npad * D * sizeof(T) : a.kp), (short)0, cen_bytes, kRawFlags);
    const __amdgpu_buffer_rsrc_t vc_rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(TAIL ? a.vbar_t + (int64_t)bh * a.npad * D * sizeof(T) : a.vp), (short)0, cen_bytes, kRawFlags);
    const int lane_off = lane * 16;
    // The first-order correction needs the packed D x D matrix (fragment md*KT
    // + t: rows 32md.., columns 16t..): the last iteration loads its first two
    // 32-row tiles into kf and, up to D = 128, the rest into vf, in place of the
    // next chunk; above 128 (more fragments than kf and vf hold) the epilogue
    // loads the tiles from the third on, one ahead of their products.
    const bool first_order = TAIL && a.ht != nullptr;
    const __amdgpu_buffer_rsrc_t ht_rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(first_order ? a.ht + (int64_t)bh * D * D * sizeof(T) : a.kp), (short)0,
        first_order ? D * D * (int)sizeof(T) : 0, kRawFlags);
    // Copies the next block's query rows (fragment nt*KT + t at 1 KB each) to
    // this wave's LDS, and in the dense kernel (kCopyChunk) also the key
    // fragments of its first chunk (LDS + 16 KB) and the value fragments of that
    // chunk's first half (LDS + 32 KB).  The query rows come from the raster
    // layout in HBM; a sparse block's first chunk is usually an L2 hit, and
    // each copy waits for room in the CU's memory queue, so copying it made
    // the sparse kernel slower (dense blocks all start at the same chunk, which
    // gains from the copy a little).
    constexpr bool kCopyChunk = !SPARSE;
    auto prefetch_next = [&]() {
        if (!PERSIST || next.nt == 0) return;
        __builtin_amdgcn_s_waitcnt(kWaitLgkm0);  // this block's LDS reads have landed
        const uint32_t lds_addr = (uint32_t)(uintptr_t)lds;
        const char* nq = a.q.data + a.q.row(next.bh, 0) * (int64_t)sizeof(T) + half * 16;
        const int nbase = a.qmap.block_base(next.qb);
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            if (nt < next.nt) {
                const int tok = min(nbase + a.qmap.intra_offset(32 * (next.sub + nt) + col), a.q_tokens - 1);
                const char* p = nq + (int64_t)tok * a.q.st * (int64_t)sizeof(T);
#pragma unroll
                for (int t = 0; t < KT; ++t) lds_copy16(p + t * 32, lds_addr + (nt * KT + t) * 1024);
            }
        }
        if (kCopyChunk && n_chunks > 0) {
            const char* src = a.kp + (int64_t)next.bh * a.kv_blocks * kBlockBytes + lane_off;
#pragma unroll
            for (int f = 0; f < 2 * KT; ++f) lds_copy16(src + f * 1024, lds_addr + 16384 + f * 1024);
            const char* vsrc = a.vp + (int64_t)next.bh * a.kv_blocks * kBlockBytes + lane_off;
#pragma unroll
            for (int md = 0; md < MD; ++md)
#pragma unroll
                for (int ss = 0; ss < 2; ++ss)
                    lds_copy16(vsrc + (md * 4 + ss) * 1024, lds_addr + 32768 + (md * 2 + ss) * 1024);
        }
    };

    // Chunks past the end re-read the last one, so every iteration issues the
    // same loads (their results are never used).
    auto is_tail = [&](int x) { return TAIL && min(x, n_chunks - 1) >= n_exact; };
    auto table_row = [&](int x) -> int {  // block id, or centroid chunk id for tail chunks
        x = min(x, n_chunks - 1);
        if (TAIL && x >= n_exact) return x - n_exact;
        return SPARSE ? my_idx[x] : x;
    };
    struct Src {
        __amdgpu_buffer_rsrc_t rs;
        int off;  // wave-uniform byte offset of the chunk
    };
    auto kptr = [&](int x, int row) { return Src{is_tail(x) ? kc_rs : kp_rs, row * (int)kBlockBytes}; };
    auto vptr = [&](int x, int row) { return Src{is_tail(x) ? vc_rs : vp_rs, row * (int)kBlockBytes}; };
    // fragment `frag` of a chunk: the 4 KB-aligned part of its offset is scalar
    // (wave-uniform, read from the first lane so that the compiler never treats
    // it as a per-lane value), the rest (< 4 KB) a constant on the lane offset
    // that the load's immediate offset field carries, so four consecutive
    // fragments share one scalar offset
    auto ld_frag = [&](const Src& p, int frag) -> vec8 {
        const int soff = __builtin_amdgcn_readfirstlane(p.off + (frag >> 2) * 4096);
        return __builtin_bit_cast(vec8,
                                  __builtin_amdgcn_raw_buffer_load_b128(p.rs, lane_off + (frag & 3) * 1024, soff, 0));
    };

    vec8 kf[2][KT];   // kf[mt]: key fragments of the next half chunk that uses them
    vec8 vf[MD][4];   // value fragments; [.][0..1] first half, [.][2..3] second half
    auto load_k_half = [&](vec8 (&k)[KT], const Src& p, int mt) {
#pragma unroll
        for (int t = 0; t < KT; ++t) k[t] = ld_frag(p, mt * KT + t);
    };
    auto load_v_half = [&](const Src& p, int mt) {
#pragma unroll
        for (int md = 0; md < MD; ++md)
#pragma unroll
            for (int ss = 0; ss < 2; ++ss) vf[md][2 * mt + ss] = ld_frag(p, md * 4 + 2 * mt + ss);
    };
    // Centroid chunks of bf16 problems get their score bias from the matrix
    // core: one more MFMA per query tile adds A x B with A's first two
    // contraction slots holding the key's bias / c as a bf16 hi + lo pair
    // (bias_frag: 16 significant bits, relative error below 2^-16) and B's
    // holding ones, so the softmax of a centroid half is the exact blocks' one
    // (scores times c in the exponent's fma).  fp16 keeps the VALU transform
    // (transform_tail): bias / c can exceed fp16's range at small softmax
    // scales.
    constexpr bool kBiasMfma = TAIL && std::is_same<T, bf16_t>::value;
    const vec8 ones_frag = [&] {
        vec8 x;
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = T((half == 0 && e < 2) ? 1.0f : 0.0f);
        return x;
    }();
    auto scores_half = [&](const vec8 (&k)[KT], f32x16 (&s)[NT], const vec8* bias = nullptr) {
        uint32_t qoff = lane * 16;
        if constexpr (QLDS) asm volatile("" : "+v"(qoff));
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int v = 0; v < 16; ++v) s[nt][v] = 0.0f;
#pragma unroll
        for (int t = 0; t < KT; ++t)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) s[nt] = mfma32(k[t], qfrag(nt, t, qoff), s[nt]);
        if (kBiasMfma && bias)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) s[nt] = mfma32(*bias, ones_frag, s[nt]);
    };
    auto pv_half = [&](int mt, const vec8 (&pf)[NT][2]) {
#pragma unroll
        for (int ss = 0; ss < 2; ++ss)
#pragma unroll
            for (int md = 0; md < MD; ++md)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) o[md][nt] = mfma32(vf[md][2 * mt + ss], pf[nt][ss], o[md][nt]);
    };
    // Whether half chunks of chunk x (table row `row`) need transform_half: tail
    // chunks whose bias is not added by the matrix core, and a short last key
    // block (wave-uniform).
    auto special = [&](int x, int row) { return (!kBiasMfma && is_tail(x)) || (row + 1) * kBlock > a.kv_tokens; };
    // A operand of the bias MFMA of half mt of chunk x (table row `row`):
    // lane (0, col) holds the bias of centroid 64 row + 32 mt + col divided by
    // c, as bf16 hi and lo; every other slot is zero (all of them for an exact
    // chunk).  Selected blocks and padding get -inf (hi), others log2(len).
    auto bias_frag = [&](int x, int row, int mt) -> vec8 {
        vec8 f;
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = T(0.0f);
        if (!is_tail(x) || half != 0) return f;
        const int base = row * kBlock + mt * 32;
        const uint32_t word = (2 * row + mt < a.mask_words) ? my_mask[2 * row + mt] : 0u;
        const int j = base + col;
        const bool dead = ((word >> col) & 1u) != 0u || j >= a.centroids;
        const float b = (j == a.centroids - 1 ? a.last_len_log2 : 6.0f) * a.inv_scale_log2;
        const T hi = from_f32<T>(b);
        f[0] = dead ? T(-__builtin_inff()) : hi;
        f[1] = dead ? T(0.0f) : from_f32<T>(b - to_f32(hi));
        return f;
    };
    // Tail bias of half mt of the centroid chunk in table row `row`; the
    // scores come out in log2 units (returns the factor 1).
    auto transform_tail = [&](int row, int mt, f32x16 (&s)[NT]) -> float {
        // centroid jc = base + bit (base = 64row + 32mt): selected blocks and
        // padding -> -inf, others + log2(len_jc) (scores moved to log2 units
        // here).  One bias per accumulator row, shared by the query tiles: the
        // dead bits of the half (selection word | padding) are one scalar word,
        // shifted to this lane's rows once.
        const int base = row * kBlock + mt * 32;
        const uint32_t word = (2 * row + mt < a.mask_words) ? my_mask[2 * row + mt] : 0u;
        const int rem = a.centroids - base;  // live centroids of the half are bits 0 .. rem-1
        const uint32_t live = rem >= 32 ? 0xffffffffu : (rem <= 0 ? 0u : (1u << rem) - 1u);
        const uint32_t lane_dead = (word | ~live) >> (4 * half);
        float bias[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int b = 8 * (v >> 2) + (v & 3);
            const int dead = (int)(lane_dead << (31 - b)) >> 31;  // 0 or -1
            bias[v] = __builtin_bit_cast(float, (dead & (int)0xff800000u) | (~dead & 0x40c00000));  // -inf or 6 = log2(64)
        }
        if (rem >= 1 && rem <= 32) {  // the half holds the last centroid (bit rem - 1), whose block may be short
#pragma unroll
            for (int v = 0; v < 16; ++v)
                if (8 * (v >> 2) + 4 * half + (v & 3) == rem - 1 && bias[v] == 6.0f) bias[v] = a.last_len_log2;
        }
#pragma unroll
        for (int v = 0; v < 16; ++v)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) s[nt][v] = fmaf(s[nt][v], c, bias[v]);
        return 1.0f;
    };
    // Masks / tail bias of half mt of chunk x (row = its table row); returns
    // the factor that converts the resulting scores to log2 units.
    auto transform_half = [&](int x, int row, int mt, f32x16 (&s)[NT]) -> float {
        if (!is_tail(x)) {
            if ((row + 1) * kBlock > a.kv_tokens) {  // wave-uniform: only a short last block
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int key = row * kBlock + mt * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
                    if (key >= a.kv_tokens)
#pragma unroll
                        for (int nt = 0; nt < NT; ++nt) s[nt][v] = -__builtin_inff();
                }
            }
            return c;
        }
        if constexpr (kBiasMfma) return c;
        return transform_tail(row, mt, s);
    };

    // Column maxima of half mt of chunk x, then the running-max update.  The
    // common half (exact, full block) takes no branch before its maxima, so
    // they are computed in the region of the preceding PV MFMAs; tail chunks
    // and a short last block are transformed and re-maxed on a side path.
    // `kind` (a constant in each inlined copy): kStepExact, chunk x is known to
    // be an exact full block, so there is no side path at all (with one, the
    // scores are copied to the registers the two paths merge into, every
    // half); kStepTail, x is known to be a centroid chunk, transformed
    // unconditionally and maxed once; kStepGeneral tests.
    auto check_half = [&](int x, int row, int mt, f32x16 (&s)[NT], bool enable, int kind) -> float {
        float mx[NT];
        float f = c;
        if (kind == kStepTail && kBiasMfma) {
            half_max<NT>(s, c, mx);
        } else if (kind == kStepTail) {
            f = transform_tail(row, mt, s);
            half_max<NT>(s, f, mx);
        } else {
            half_max<NT>(s, c, mx);
            if (kind == kStepGeneral && special(x, row)) {
                f = transform_half(x, row, mt, s);
                half_max<NT>(s, f, mx);
            }
        }
        rescale_to<NT, MD>(mx, enable, nm, mth, l, lt, o);
        return f;
    };

    f32x16 sa[NT], sb[NT];  // scores of the first / second half of the current chunk
    float ca = c;           // factor to log2 units of the (transformed) scores in sa
    int row0 = 0, row1 = 0;
    if (n_chunks > 0) {
        row0 = table_row(0);
        row1 = table_row(1);
        const Src k0 = kptr(0, row0);
        const Src v0 = vptr(0, row0);
        // The loop sits inside this block: entered only after the query loads
        // have landed (the first scores use them), the compiler's wait counts
        // at the loop head cover just the chunk loads in flight.  The loads
        // after the first scores go out in the loop's order (K half 1, V half
        // 0, next K half 0, V half 1).
        if (kCopyChunk && PERSIST && from_lds) {
#pragma unroll
            for (int f = 0; f < 2 * KT; ++f)
                kf[f / KT][f % KT] = __builtin_bit_cast(
                    vec8, *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(
                              lds + 16384 + f * 1024 + lane * 16));
#pragma unroll
            for (int md = 0; md < MD; ++md)
#pragma unroll
                for (int ss = 0; ss < 2; ++ss)
                    vf[md][ss] = __builtin_bit_cast(
                        vec8, *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(
                                  lds + 32768 + (md * 2 + ss) * 1024 + lane * 16));
        } else {
            load_k_half(kf[0], k0, 0);
            load_k_half(kf[1], k0, 1);
            load_v_half(v0, 0);
        }
        pin_q();
        {
            const vec8 bf0 = kBiasMfma ? bias_frag(0, row0, 0) : ones_frag;
            scores_half(kf[0], sa, (kBiasMfma && is_tail(0)) ? &bf0 : nullptr);
        }
        load_k_half(kf[0], kptr(1, row1), 0);
        load_v_half(v0, 1);
        ca = check_half(0, row0, 0, sa, true, kStepGeneral);
        // One chunk step: half 0 of chunk cc (scores in sa) beside the scores of
        // half 1, then half 1 beside the scores of the next chunk's half 0.  The
        // last step (`last`, a constant in each inlined copy) has no next chunk:
        // those scores are dead code, and its loads bring the packed H_sum^T
        // fragments of the correction instead.
        // `kind`: kStepExact, chunks cc, cc + 1 and cc + 2 are exact blocks and
        // cc, cc + 1 full ones (no tail or short-block tests, direct table
        // rows); kStepTail, chunks cc and cc + 1 are centroid chunks (as is
        // cc + 2, or the last one re-read).
        auto chunk_step = [&](int cc, bool last, bool half0_only, int kind) __attribute__((always_inline)) {
            const bool exact_k = kind == kStepExact, tail_k = kind == kStepTail;
            const int row2 = exact_k ? (SPARSE ? my_idx[cc + 2] : cc + 2) : table_row(cc + 2);
            const bool tail = tail_k || (!exact_k && is_tail(cc));
            const Src kn = (first_order && last) ? Src{ht_rs, 0}
                           : exact_k ? Src{kp_rs, row1 * (int)kBlockBytes}
                           : tail_k  ? Src{kc_rs, row1 * (int)kBlockBytes} : kptr(cc + 1, row1);
            const Src vn = (first_order && last) ? Src{ht_rs, 2 * KT * 1024}
                           : exact_k ? Src{vp_rs, row1 * (int)kBlockBytes}
                           : tail_k  ? Src{vc_rs, row1 * (int)kBlockBytes} : vptr(cc + 1, row1);
            const Src kn2 = (first_order && last) ? Src{ht_rs, 0}
                            : exact_k ? Src{kp_rs, row2 * (int)kBlockBytes}
                            : tail_k  ? Src{kc_rs, row2 * (int)kBlockBytes} : kptr(cc + 2, row2);
            vec8 pf[NT][2];

            // ---- first half: scores in sa (issued, masked and max-checked one half earlier)
            if (!half0_only) {
                // only centroid chunks carry the bias MFMA
                const vec8 bf1 = (kBiasMfma && !exact_k) ? bias_frag(cc, row0, 1) : ones_frag;
                scores_half(kf[1], sb, (kBiasMfma && (tail_k || (!exact_k && is_tail(cc)))) ? &bf1 : nullptr);
            }
            probs_half<T, NT>(sa, ca, nm, l, lt, tail, pf);
            load_k_half(kf[1], kn, 1);
            pv_half(0, pf);
            load_v_half(vn, 0);
            const float cb = half0_only ? c : check_half(cc, row0, 1, sb, true, kind);

            // ---- second half: scores in sb; also scores the next chunk's first half
            if (!last) {
                const vec8 bf0 = (kBiasMfma && !exact_k) ? bias_frag(cc + 1, row1, 0) : ones_frag;
                scores_half(kf[0], sa, (kBiasMfma && (tail_k || (!exact_k && is_tail(cc + 1)))) ? &bf0 : nullptr);
            }
            if (!half0_only) probs_half<T, NT>(sb, cb, nm, l, lt, tail, pf);
            load_k_half(kf[0], kn2, 0);
            if (!half0_only) pv_half(1, pf);
            load_v_half(vn, 1);
            if (!last) ca = check_half(cc + 1, row1, 0, sa, true, kind);
            row0 = row1;
            row1 = row2;
        };
        // Exact chunks before the last two are full blocks (the selection is
        // ascending, so a short last key block can only be the last exact
        // chunk) and are followed by exact chunks: they take the plain exact
        // step.  The last two exact chunks take the general step, and centroid
        // chunks followed by centroid chunks the centroid step.
        int cc = 0;
        for (; cc + 3 <= n_exact; ++cc) chunk_step(cc, false, false, kStepExact);
        for (; cc + 1 < n_chunks && (!TAIL || cc < n_exact); ++cc) chunk_step(cc, false, false, kStepGeneral);
        if constexpr (TAIL)
            for (; cc + 1 < n_chunks; ++cc) chunk_step(cc, false, false, kStepTail);
        // The last chunk.  A centroid chunk whose second half holds only
        // padding (centroids past the last block: C4's 144 centroids end 16 keys
        // into their third chunk) skips that half's scores, softmax and PV
        // (they would add exactly zero to l, l_tail and O); its loads still go
        // out, unconditionally, so no register keeps two values across a branch.
        const int cl = n_chunks - 1;
        chunk_step(cl, true, TAIL && is_tail(cl) && table_row(cl) * kBlock + 32 >= a.centroids, kStepGeneral);
    }

    // The copies of the next block's query rows go out here,
    // after an explicit wait for this block's last loads (the correction's
    // fragments, needed next anyway): the copies are hidden from the compiler's
    // counters, so every wait issued after them also waits for them.  Issued in
    // the prologue, they held the block's first chunk waits; here they land
    // during the correction and the stores, which wait for nothing.
    if constexpr (PERSIST) {
        __builtin_amdgcn_s_waitcnt(kWaitVm0);
        prefetch_next();
    }

    // ---- epilogue: normalise, add the first-order correction one 32-dim
    // tile at a time (keeps only 32 extra accumulators live), store the real
    // head dims
    float inv[NT], wa[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const float lf = add_xor32(l[nt]);
        const float ltf = add_xor32(lt[nt]);
        inv[nt] = 1.0f / lf;
        wa[nt] = ltf * inv[nt] * a.corr_scale;
    }
    char* obase[NT];
    bool ovalid[NT];
    {
        const int base = a.qmap.block_base(qb);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const int tok = base + q_off[nt];
            ovalid[nt] = tok < a.q_tokens;
            obase[nt] = a.o.data + a.o.row(bh, ovalid[nt] ? tok : 0) * (int64_t)sizeof(T);
        }
    }
    typedef T vec4 __attribute__((ext_vector_type(4)));
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    // 16-byte stores when every output row start is 16-byte aligned (8-byte
    // ones otherwise)
    const bool st16 = (reinterpret_cast<uintptr_t>(a.o.data) % 16 == 0) &&
                      ((a.o.sb | a.o.sh | a.o.st) * (int64_t)sizeof(T)) % 16 == 0;
#pragma unroll
    for (int md = 0; md < MD; ++md) {
        f32x16 corr[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int v = 0; v < 16; ++v) corr[nt][v] = 0.0f;
        if (first_order) {
            // packed D x D matrix fragment (md, t): rows 32md.., columns 16t..
            // (kfrag_elem), in kf (md < 2) and up to D = 128 in vf (md >= 2)
            // since the last iteration; above 128 tile md + 1 is loaded into
            // kf[(md + 1) % 2] here (tile md - 1 used it last)
            if constexpr (D > 128)
                if (md + 1 < MD && md + 1 >= 2) load_k_half(kf[(md + 1) & 1], Src{ht_rs, 0}, md + 1);
            uint32_t qoff = lane * 16;
            if constexpr (QLDS) asm volatile("" : "+v"(qoff));
#pragma unroll
            for (int t = 0; t < KT; ++t) {
                const vec8 hf = (D > 128 || md < 2) ? kf[md & 1][t] : vf[(md >= 2 ? md - 2 : 0) * 2 + t / 4][t % 4];
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) corr[nt] = mfma32(hf, qfrag(nt, t, qoff), corr[nt]);
            }
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            if (!ovalid[nt]) continue;  // lanes l and l + 32 (one query) take the same branch
            // w[g]: the 4 outputs of accumulator group g packed, dims 8g + 4half ..
            u32x2 w[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                vec4 out;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float x = o[md][nt][4 * g + e] * inv[nt];
                    if (first_order) x += corr[nt][4 * g + e] * wa[nt];
                    out[e] = from_f32<T>(x);
                }
                w[g] = __builtin_bit_cast(u32x2, out);
            }
            if (st16) {
                // one lane-half swap per dword of groups 2p and 2p + 1 leaves lanes
                // 0-31 with dims 8(2p) .. +7 of their query and lanes 32-63 with
                // dims 8(2p + 1) .. +7: one 16-byte store each
#pragma unroll
                for (int p = 0; p < 2; ++p) {
                    u32x4 x16;
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const auto r = __builtin_amdgcn_permlane32_swap(w[2 * p][j], w[2 * p + 1][j], false, false);
                        x16[j] = r[0];
                        x16[2 + j] = r[1];
                    }
                    const int d = md * 32 + 8 * (2 * p + half);
                    if (all_dims || d < a.head_dim) *reinterpret_cast<u32x4*>(obase[nt] + d * sizeof(T)) = x16;
                }
            } else {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int d = md * 32 + 8 * g + 4 * half;
                    if (all_dims || d < a.head_dim) *reinterpret_cast<u32x2*>(obase[nt] + d * sizeof(T)) = w[g];
                }
            }
        }
    }
    // A persistent wave waits here until its stores are acknowledged and the
    // copies for the next block have landed: the next block then reads its LDS
    // safely and starts with no writes in flight (the compiler counts pending
    // reads exactly only when no writes are pending alongside them).
    if constexpr (PERSIST) __builtin_amdgcn_s_waitcnt(kWaitVm0);
}

// One wavefront per work item.  Work items are query blocks (64 rows, NT = 2)
// up to D = 128 and 32-row halves of query blocks (NT = 1) above.  Consecutive
// work items run on the same XCD (xcd_remap), keeping a head's packed K/V in
// that XCD's L2.
//
// Split last round (a.split_r > 0, D = 128): a grid of B query blocks on S
// wave slots (one wave per SIMD) runs in ceil(B / S) rounds, and a last round
// of r = B mod S blocks leaves S - r SIMDs idle for a whole block time.  With
// 2r <= S the last r blocks of every XCD instead run as 2r one-tile waves
// (NT = 1, ~0.6 of a block's time each) that fill the XCD's SIMDs.  Each XCD
// takes a contiguous range of qx = B / 8 blocks: its first qx - r work items
// are whole blocks, the following 2r the halves of the rest, dispatched last.
template <typename T, int D, bool SPARSE, bool TAIL>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(1, 1)))
void attention_kernel(AttnArgs a, const int32_t* __restrict__ sel, const uint32_t* __restrict__ selmask) {
    // sel/selmask are a.idx/a.selmask passed as restrict-qualified arguments: the
    // kernel never writes them, so their wave-uniform reads become scalar loads.
    if constexpr (D == 128) {
        if (a.split_r > 0) {
            const int xcd = blockIdx.x & 7;
            const int local = blockIdx.x >> 3;
            const int qx = a.q_blocks_total >> 3;
            const int full = qx - a.split_r;
            if (local < full) {
                const int blk = xcd * qx + local;
                const int bh = blk / a.q_blocks;
                attention_block<T, D, 2, SPARSE, TAIL>(a, bh, blk - bh * a.q_blocks, 0, sel, selmask);
            } else {
                const int h = local - full;
                const int blk = xcd * qx + full + (h >> 1);
                const int bh = blk / a.q_blocks;
                attention_block<T, D, 1, SPARSE, TAIL>(a, bh, blk - bh * a.q_blocks, h & 1, sel, selmask);
            }
            return;
        }
    }
    constexpr int NT = D <= 128 ? 2 : 1;  // 32-row query tiles per wave
    constexpr int SUBS = 2 / NT;          // waves per 64-row query block
    const int work = xcd_remap(blockIdx.x, gridDim.x);
    const int block_work = work / SUBS;
    const int bh = block_work / a.q_blocks;
    lds_char* qbuf = nullptr;
    if constexpr (D > 192) {  // the query fragments of the wave (attention_block, QLDS)
        __shared__ __attribute__((aligned(1024))) char q_lds[D / 16 * 1024];
        qbuf = (lds_char*)q_lds;
    }
    attention_block<T, D, NT, SPARSE, TAIL>(a, bh, block_work - bh * a.q_blocks, work - block_work * SUBS, sel,
                                            selmask, qbuf);
}

// Persistent variant (D = 128, head dim 128, a grid that splits evenly into the
// 8 XCDs): one wave per SIMD for the whole launch.  Slot j of XCD x (S
// slots per XCD, qx = B / 8 blocks per XCD) runs blocks x*qx + j + S*it for
// it < F = qx / S, then its share of the r = qx mod S blocks left: one-tile
// halves of block x*qx + F*S + j/2 when 2r <= S (as attention_kernel's split),
// else whole block x*qx + F*S + j for j < r.  While a block runs, the next
// block's query rows (and in the dense kernel its first chunk) are copied to
// the wave's LDS (16 KB, dense 40 KB per wave; direct-to-LDS loads), so its
// prologue reads them from LDS instead of waiting on HBM.
template <typename T, bool SPARSE, bool TAIL>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(1, 1)))
void attention_persistent_kernel(AttnArgs a, const int32_t* __restrict__ sel, const uint32_t* __restrict__ selmask) {
    constexpr int D = 128;
    __shared__ __attribute__((aligned(1024))) char lds_buf[(SPARSE ? 16 : 40) * 1024];
    lds_char* const lds = (lds_char*)lds_buf;
    const int xcd = blockIdx.x & 7;
    const int j = blockIdx.x >> 3;
    const int S = gridDim.x >> 3;
    const int qx = a.q_blocks_total >> 3;
    const int F = qx / S;
    const int r = qx - F * S;
    const bool split = 2 * r <= S;
    const int n_items = F + ((split ? j < 2 * r : j < r) ? 1 : 0);
    auto item = [&](int it) -> NextBlock {
        if (it >= n_items) return NextBlock{0, 0, 0, 0};
        int blk = xcd * qx + F * S + j, sub = 0, nt = 2;
        if (it < F) {
            blk = xcd * qx + j + S * it;
        } else if (split) {
            blk = xcd * qx + F * S + (j >> 1);
            sub = j & 1;
            nt = 1;
        }
        const int bh = blk / a.q_blocks;
        return NextBlock{bh, blk - bh * a.q_blocks, sub, nt};
    };
    NextBlock cur = item(0);
    for (int it = 0; it < n_items; ++it) {
        const NextBlock nxt = item(it + 1);
        if (cur.nt == 2)
            attention_block<T, D, 2, SPARSE, TAIL, true>(a, cur.bh, cur.qb, 0, sel, selmask, lds, it > 0, nxt);
        else
            attention_block<T, D, 1, SPARSE, TAIL, true>(a, cur.bh, cur.qb, cur.sub, sel, selmask, lds, it > 0, nxt);
        cur = nxt;
    }
}

// ---- packed key and value blocks (kfrag_elem / vfrag_elem order at the
// padded width D; dims >= d_real and rows >= kv_tokens are zero; block j
// row r is token map(64 j + r)).  One workgroup per block: 64 rows x D of K
// and V are read with 16-byte loads (4 rows per thread), the key fragments are
// written straight from registers and the value block is transposed through
// LDS.
template <typename T, int D>
__global__ __launch_bounds__(256) void kv_pack_kernel(View k, View v, TokenMap map, int kv_tokens, int kv_blocks,
                                                      int d_real, char* kp, char* vp) {
    typedef typename Elem<T>::vec8 vec8;
    typedef T vec4 __attribute__((ext_vector_type(4)));
    constexpr int kRow = kBlock + 8;
    __shared__ __attribute__((aligned(16))) T lds[D * kRow];
    const int t = threadIdx.x;
    const int bh = blockIdx.x / kv_blocks;
    const int j = blockIdx.x - bh * kv_blocks;
    constexpr int kPieces = D / 8;            // 16-byte pieces per row
    constexpr int kRowsPerPass = 256 / kPieces;
    const int pc = t % kPieces;
    const int r0 = t / kPieces;
    const bool live_d = pc * 8 < d_real;      // d_real is a multiple of 8
    T* kdst = reinterpret_cast<T*>(kp) + ((int64_t)bh * kv_blocks + j) * D * kBlock;
    T* vdst = reinterpret_cast<T*>(vp) + ((int64_t)bh * kv_blocks + j) * D * kBlock;
    const int base = map.block_base(j);          // raster token of row r: base + intra_offset(r)
    const int last = kv_tokens - 1 - j * kBlock;  // rows past the end read the last token
    for (int r = r0 * 4; r < kBlock; r += kRowsPerPass * 4) {
        // the 8 loads of the 4 rows go out together and unconditionally (rows
        // past kv_tokens re-read the last token, dims past d_real the first
        // piece; both are zeroed at use), so no load waits behind another
        vec8 kx[4], x[4];
        bool live[4];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const int key = j * kBlock + r + rr;
            live[rr] = key < kv_tokens && live_d;
            const int tok = base + map.intra_offset(min(r + rr, last));
            const int dc = live_d ? pc * 8 : 0;
            kx[rr] = load8<vec8>(k.data + (k.row(bh, tok) + dc) * sizeof(T));
            x[rr] = load8<vec8>(v.data + (v.row(bh, tok) + dc) * sizeof(T));
        }
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            if (!live[rr]) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    kx[rr][e] = T(0.0f);
                    x[rr][e] = T(0.0f);
                }
            }
            store8(kdst + kfrag_elem(r + rr, pc * 8, D), kx[rr]);
        }
        const int p = swap23(r);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            vec4 w = {x[0][e], x[1][e], x[2][e], x[3][e]};
            *reinterpret_cast<vec4*>(&lds[(pc * 8 + e) * kRow + p]) = w;
        }
    }
    __syncthreads();
    // value fragment f = 4md + ks, lane (half, col): row 32md + col, positions 16ks + 8half
    for (int id = t; id < D * 8; id += 256) {
        const int f = id >> 6;
        const int L = id & 63;
        const int row = (f >> 2) * 32 + (L & 31);
        const int pos = (f & 3) * 16 + (L >> 5) * 8;
        store8(vdst + id * 8, *reinterpret_cast<const vec8*>(&lds[row * kRow + pos]));
    }
}

// Wave slots per XCD at one wave per SIMD (0 if the device does not split
// evenly into 8 XCDs).
static int xcd_slots() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus % 8 != 0)
        return 0;
    return cus / 8 * 4;
}

template <typename T, int D, bool SPARSE, bool TAIL>
int launch_attention_t(const AttnArgs& a_in, int bh_count, hipStream_t stream) {
    constexpr int kSubs = D <= 128 ? 1 : 2;  // waves per query block
    AttnArgs a = a_in;
    a.q_blocks_total = bh_count * a.q_blocks;
    a.split_r = 0;
    if constexpr (D == 128) {
        static const int pslots = xcd_slots();
        if (a.head_dim == D && a.q_blocks_total % 8 == 0 && pslots > 0) {
            hipLaunchKernelGGL((attention_persistent_kernel<T, SPARSE, TAIL>), dim3(8 * pslots), dim3(64), 0, stream,
                               a, a.idx, a.selmask);
            return pisa_host::check_launch("attention_persistent_kernel");
        }
    }
    int waves = a.q_blocks_total * kSubs;
    if (D == 128 && a.q_blocks_total % 8 == 0) {
        static const int slots = xcd_slots();
        const int r = slots > 0 ? (a.q_blocks_total / 8) % slots : 0;
        if (r > 0 && 2 * r <= slots) {
            a.split_r = r;
            waves = a.q_blocks_total + 8 * r;
        }
    }
    hipLaunchKernelGGL((attention_kernel<T, D, SPARSE, TAIL>), dim3(waves), dim3(64), 0, stream, a, a.idx, a.selmask);
    return pisa_host::check_launch("attention_kernel");
}

// The dense launchers (SPARSE = TAIL = false) are compiled in a translation
// unit of their own, attention_dense.hip (this file with PISA_ATTENTION_DENSE
// defined), under the max-memory-clause machine scheduler: it serves the dense
// chunk loop better and the sparse one worse.  This file without the macro
// holds the sparse kernels, the dispatcher and the packing kernel.
#define PISA_DENSE_INSTANCES(X) \
    X(bf16_t, 64) X(bf16_t, 96) X(bf16_t, 128) X(bf16_t, 160) X(bf16_t, 192) X(bf16_t, 256) \
    X(f16_t, 64) X(f16_t, 96) X(f16_t, 128) X(f16_t, 160) X(f16_t, 192) X(f16_t, 256)
#ifdef PISA_ATTENTION_DENSE
#define PISA_DENSE_INSTANCE(T, D) template int launch_attention_t<T, D, false, false>(const AttnArgs&, int, hipStream_t);
PISA_DENSE_INSTANCES(PISA_DENSE_INSTANCE)
#undef PISA_DENSE_INSTANCE
#else
#define PISA_DENSE_EXTERN(T, D) \
    extern template int launch_attention_t<T, D, false, false>(const AttnArgs&, int, hipStream_t);
PISA_DENSE_INSTANCES(PISA_DENSE_EXTERN)
#undef PISA_DENSE_EXTERN

template <typename T, int D>
int launch_attention_d(bool sparse, bool tail, const AttnArgs& a, int bh_count, hipStream_t stream) {
    if (sparse && tail) return launch_attention_t<T, D, true, true>(a, bh_count, stream);
    if (!sparse && !tail) return launch_attention_t<T, D, false, false>(a, bh_count, stream);
    return pisa_host::fail(PISA_ERR_UNSUPPORTED, "attention kernel: sparse and tail go together");
}

template <typename T>
int launch_attention_dt(int padded, bool sparse, bool tail, const AttnArgs& a, int bh_count, hipStream_t stream) {
    switch (padded) {
        case 64: return launch_attention_d<T, 64>(sparse, tail, a, bh_count, stream);
        case 96: return launch_attention_d<T, 96>(sparse, tail, a, bh_count, stream);
        case 128: return launch_attention_d<T, 128>(sparse, tail, a, bh_count, stream);
        case 160: return launch_attention_d<T, 160>(sparse, tail, a, bh_count, stream);
        case 192: return launch_attention_d<T, 192>(sparse, tail, a, bh_count, stream);
        case 256: return launch_attention_d<T, 256>(sparse, tail, a, bh_count, stream);
        default: return pisa_host::fail(PISA_ERR_UNSUPPORTED, "attention kernel: padded head dim %d", padded);
    }
}

int launch_attention(int dtype, int padded, bool sparse, bool tail, const AttnArgs& a, int bh_count,
                     hipStream_t stream) {
    if (dtype == PISA_DTYPE_BF16) return launch_attention_dt<bf16_t>(padded, sparse, tail, a, bh_count, stream);
    return launch_attention_dt<f16_t>(padded, sparse, tail, a, bh_count, stream);
}

template <typename T>
int launch_kv_pack_t(int padded, int head_dim, const View& k, const View& v, TokenMap map, int kv_tokens,
                     int kv_blocks, int bh_count, char* kp, char* vp, hipStream_t stream) {
    const dim3 grid(bh_count * kv_blocks);
#define PISA_KV_PACK(DP)                                                                                     \
    case DP:                                                                                                 \
        hipLaunchKernelGGL((kv_pack_kernel<T, DP>), grid, dim3(256), 0, stream, k, v, map, kv_tokens, kv_blocks, \
                           head_dim, kp, vp);                                                                \
        break;
    switch (padded) {
        PISA_KV_PACK(64)
        PISA_KV_PACK(96)
        PISA_KV_PACK(128)
        PISA_KV_PACK(160)
        PISA_KV_PACK(192)
        PISA_KV_PACK(256)
        default: return pisa_host::fail(PISA_ERR_UNSUPPORTED, "kv pack: padded head dim %d", padded);
    }
#undef PISA_KV_PACK
    return pisa_host::check_launch("kv_pack_kernel");
}

int launch_kv_pack(int dtype, int padded, int head_dim, const View& k, const View& v, TokenMap map, int kv_tokens,
                   int kv_blocks, int bh_count, char* kp, char* vp, hipStream_t stream) {
    if (dtype == PISA_DTYPE_BF16)
        return launch_kv_pack_t<bf16_t>(padded, head_dim, k, v, map, kv_tokens, kv_blocks, bh_count, kp, vp, stream);
    return launch_kv_pack_t<f16_t>(padded, head_dim, k, v, map, kv_tokens, kv_blocks, bh_count, kp, vp, stream);
}
#endif  // PISA_ATTENTION_DENSE

}  // namespace pisa
