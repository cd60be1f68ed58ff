// Shared device/host helpers for the gfx950 attention kernels.
//
// Conventions used by every kernel in this library:
//   * a wavefront is 64 lanes; `lane = threadIdx.x & 63`, `half = lane >> 5`,
//     `col = lane & 31` are the coordinates of the 32x32 MFMA layouts;
//   * v_mfma_f32_32x32x16_{bf16,f16}: lane (half, col) supplies 8 operand
//     values A[col][slot] / B[slot][col] for the 16-deep contraction slots
//     half*8 .. half*8+7, and receives accumulator values
//       D[row = 8*(v/4) + 4*half + (v%4)][col],  v = 0..15;
//   * value blocks are stored as V^T operand fragments with the key index
//     bit-permuted by swap23(), so that a lane's 8 accumulator rows of one
//     MFMA output (probabilities) are the B operand of the next MFMA.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pisa_hip.h"

namespace pisa {

typedef __bf16 bf16_t;
typedef _Float16 f16_t;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kBlock = PISA_BLOCK_SIZE;  // tokens per PISA block
// s_waitcnt immediates (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4,
// lgkmcnt 11:8) for the explicit waits around the direct-to-LDS copies, which
// the compiler's counters do not model.  tests/test_build_guards.py checks
// that the assembler prints them as the single waits named here.
constexpr int kWaitLgkm0 = 0xC07F;  // s_waitcnt lgkmcnt(0) (vmcnt, expcnt at their maximum)
constexpr int kWaitVm0 = 0x0F70;    // s_waitcnt vmcnt(0) (lgkmcnt, expcnt at their maximum)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ---------------------------------------------------------------- element types
template <typename T> struct Elem;
template <> struct Elem<bf16_t> {
    typedef bf16x8 vec8;
    static constexpr int dtype = PISA_DTYPE_BF16;
};
template <> struct Elem<f16_t> {
    typedef f16x8 vec8;
    static constexpr int dtype = PISA_DTYPE_F16;
};

__device__ __forceinline__ float to_f32(bf16_t x) { return static_cast<float>(x); }
__device__ __forceinline__ float to_f32(f16_t x) { return static_cast<float>(x); }
__device__ __forceinline__ float to_f32(float x) { return x; }

template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ bf16_t from_f32<bf16_t>(float x) { return static_cast<bf16_t>(x); }
template <> __device__ __forceinline__ f16_t from_f32<f16_t>(float x) { return static_cast<f16_t>(x); }
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }

// 32x32x16 MFMA on 8-element operands, fp32 accumulation.
__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// 16-byte global load / store of 8 elements.
template <typename V> __device__ __forceinline__ V load8(const void* p) {
    u32x4 raw = *reinterpret_cast<const u32x4*>(p);
    return __builtin_bit_cast(V, raw);
}
// The same load with the non-temporal hint, for rows a kernel reads once and
// no later launch reads again: they then do not displace from the L2 and the
// last-level cache the data that later launches do re-read.
template <typename V> __device__ __forceinline__ V load8_nt(const void* p) {
    return __builtin_bit_cast(V, __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p)));
}
template <typename V> __device__ __forceinline__ void store8(void* p, V v) {
    *reinterpret_cast<u32x4*>(p) = __builtin_bit_cast(u32x4, v);
}

// Cross-lane exchanges without the LDS crossbar.  v_permlane32_swap swaps the
// upper 32 lanes of one register with the lower 32 lanes of another, so
// applied to two copies of x it yields {x[l], x[l ^ 32]} in every lane
// (in some order); v_permlane16_swap does the same for 16-lane rows,
// {x[l], x[l ^ 16]}.  Sums and maxima of the pair are order independent.
__device__ __forceinline__ float2 pair_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float2 pair_xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float add_xor32(float x) { const float2 p = pair_xor32(x); return p.x + p.y; }
__device__ __forceinline__ float add_xor16(float x) { const float2 p = pair_xor16(x); return p.x + p.y; }
__device__ __forceinline__ float max_xor32(float x) { const float2 p = pair_xor32(x); return fmaxf(p.x, p.y); }

__device__ __forceinline__ float wave_sum(float x) {
    x = add_xor32(x);
    x = add_xor16(x);
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) x += __shfl_xor(x, o);
    return x;
}

// Bits 2 and 3 of a key index swapped: the storage position of key `k`
// inside a transposed key block (self inverse).
__host__ __device__ __forceinline__ int swap23(int k) {
    return (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1);
}

// ---------------------------------------------------------------- packed blocks
// A 64-key block (or a 64-centroid chunk, or a D x D matrix read as D/32
// "key" tiles) is stored as MFMA operand fragments of 64 lanes x 16 bytes,
// each fragment contiguous, so the attention kernel reads one fragment with a
// single fully coalesced 1 KB load (a row-major block would touch 32 cache
// lines per load instruction, 32 bytes of each).
//   key fragment (mt, t), t < D/16:  lane (half, col) holds
//       K[32mt + col][16t + 8half .. +7]                 -> kfrag_elem
//   value fragment (md, ks), ks < 4: lane (half, col) holds the keys at
//       positions 16ks + 8half .. +7 of the swap23 order of V[.][32md + col]
//                                                        -> vfrag_elem
// Both return the element offset inside the block (block size 64 * D).
__host__ __device__ __forceinline__ int kfrag_elem(int key, int d, int D) {
    return ((((key >> 5) * (D >> 4) + (d >> 4)) * 64 + ((d >> 3) & 1) * 32 + (key & 31)) << 3) + (d & 7);
}
__host__ __device__ __forceinline__ int vfrag_elem(int key, int d) {
    const int p = (key & ~12) | ((key & 4) << 1) | ((key & 8) >> 1);  // swap23(key)
    return ((((d >> 5) * 4 + (p >> 4)) * 64 + ((p >> 3) & 1) * 32 + (d & 31)) << 3) + (p & 7);
}

// Head dims other than 128 (generic path, dense attention) run on kernels
// instantiated for a padded width: the packed tables hold zeros in dims
// [D, Dp), queries are loaded as zero there and outputs are not stored.
// Returns 0 for unsupported D (D must be a multiple of 8, at most 256).
__host__ __device__ inline int padded_head_dim(int d) {
    if (d <= 0 || d % 8 || d > 256) return 0;
    if (d <= 64) return 64;
    if (d <= 96) return 96;
    if (d <= 128) return 128;
    if (d <= 160) return 160;
    if (d <= 192) return 192;
    return 256;
}

// ---------------------------------------------------------------- views
struct View {
    const char* data;  // byte pointer
    int64_t sb, sh, st;  // element strides
    int heads;
    __device__ __forceinline__ int64_t row(int bh, int64_t token) const {
        const int b = bh / heads;
        const int h = bh - b * heads;
        return b * sb + h * sh + token * st;
    }
};

struct OutView {
    char* data;
    int64_t sb, sh, st;
    int heads;
    __device__ __forceinline__ int64_t row(int bh, int64_t token) const {
        const int b = bh / heads;
        const int h = bh - b * heads;
        return b * sb + h * sh + token * st;
    }
};

// Block-major position -> raster token (see pisa_token_grid in pisa_hip.h).
struct TokenMap {
    int frame_tokens;   // 0: identity
    int width;
    int tiles_per_row;
    __device__ __forceinline__ int operator()(int o) const {
        if (frame_tokens == 0) return o;
        const int f = o / frame_tokens;
        const int w = o - f * frame_tokens;
        const int tile = w >> 6;
        const int intra = w & 63;
        const int tr = tile / tiles_per_row;
        const int tc = tile - tr * tiles_per_row;
        return f * frame_tokens + ((tr << 3) + (intra >> 3)) * width + (tc << 3) + (intra & 7);
    }
    // token(64j + r) == block_base(j) + intra_offset(r) for 0 <= r < 64
    __device__ __forceinline__ int block_base(int j) const {
        if (frame_tokens == 0) return j << 6;
        const int blocks_per_frame = frame_tokens >> 6;
        const int f = j / blocks_per_frame;
        const int tile = j - f * blocks_per_frame;
        const int tr = tile / tiles_per_row;
        const int tc = tile - tr * tiles_per_row;
        return f * frame_tokens + (tr << 3) * width + (tc << 3);
    }
    __device__ __forceinline__ int intra_offset(int r) const {
        return frame_tokens == 0 ? r : (r >> 3) * width + (r & 7);
    }
};

inline TokenMap make_token_map(const pisa_token_grid& g) {
    TokenMap m;
    if (g.frames <= 0) {
        m.frame_tokens = 0;
        m.width = 0;
        m.tiles_per_row = 0;
    } else {
        m.frame_tokens = g.height * g.width;
        m.width = g.width;
        m.tiles_per_row = g.width / 8;
    }
    return m;
}

// Wavefront -> logical work index so that consecutive logical indices land on
// the same XCD (workgroups are dispatched round robin over the 8 XCDs).
__device__ __forceinline__ int xcd_remap(int wg, int total) {
    const int xcd = wg & 7;
    const int local = wg >> 3;
    const int base = total >> 3;
    const int rem = total & 7;
    return xcd * base + (xcd < rem ? xcd : rem) + local;
}

}  // namespace pisa

// ---------------------------------------------------------------- host side
namespace pisa_host {
void set_error(const char* fmt, ...);
int fail(int status, const char* fmt, ...);
int check_launch(const char* what);
bool valid_dtype(int dtype);
}  // namespace pisa_host
