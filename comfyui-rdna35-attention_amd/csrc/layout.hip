// Bandwidth-bound layout kernels: spatial/video tile packing, the inverse
// permutation, and the standalone LSE merge epilogue.  Each thread moves one
// 16-byte vector (8 elements of one token row); a 256-thread workgroup covers
// 256 / (D/8) consecutive block-major tokens of one (batch, head).
//
// pack   : packed[bh][o][:] = x[b][h][raster(o)][:]      (pisa_kernels.cu:247-272)
// unpack : out[b][raster(o)][h][:] = packed[bh][o][:]    (pisa_kernels.cu:275-293)
// merge  : out[b][raster(o)][h][:] = dtype(O_e*w_e + O_a*w_a + C*w_a) with
//          w_x = exp(L_x - logaddexp(L_e, L_a))           (pisa_kernels.cu:296-340)
//
// pack and merge read their 16-bit rows with the non-temporal hint (each row
// is read once; measured same-box with fresh inputs each call: pack 88.1 ->
// 68.6 us, merge 71.9 -> 63.5 us at the C4 shape); unpack's reads and merge's
// fp32 correction reads measured faster without it.
#include "kernels.hpp"

namespace pisa {


template <typename T>
__global__ __launch_bounds__(256) void pack_kernel(LayoutArgs a) {
    typedef typename Elem<T>::vec8 vec8;
    const int per_token = a.head_dim / 8;
    const int tokens_per_wg = 256 / per_token;
    const int wgs_per_bh = (a.tokens + tokens_per_wg - 1) / tokens_per_wg;
    const int bh = blockIdx.x / wgs_per_bh;
    const int o = (blockIdx.x - bh * wgs_per_bh) * tokens_per_wg + threadIdx.x / per_token;
    const int c = threadIdx.x % per_token;
    if (o >= a.tokens || threadIdx.x >= tokens_per_wg * per_token) return;
    const int raster = a.map(o);
    for (int x = 0; x < a.ntensors; ++x) {
        const vec8 val = load8_nt<vec8>(a.in[x].data + (a.in[x].row(bh, raster) + c * 8) * sizeof(T));
        store8(a.out[x] + (((int64_t)bh * a.tokens + o) * a.head_dim + c * 8) * sizeof(T), val);
    }
}

template <typename T>
__global__ __launch_bounds__(256) void unpack_kernel(const char* packed, char* raster_out, TokenMap map, int tokens,
                                                     int head_dim, int heads) {
    typedef typename Elem<T>::vec8 vec8;
    const int per_token = head_dim / 8;
    const int tokens_per_wg = 256 / per_token;
    const int wgs_per_bh = (tokens + tokens_per_wg - 1) / tokens_per_wg;
    const int bh = blockIdx.x / wgs_per_bh;
    const int o = (blockIdx.x - bh * wgs_per_bh) * tokens_per_wg + threadIdx.x / per_token;
    const int c = threadIdx.x % per_token;
    if (o >= tokens || threadIdx.x >= tokens_per_wg * per_token) return;
    const int b = bh / heads;
    const int h = bh - b * heads;
    const int raster = map(o);
    const vec8 val = load8<vec8>(packed + (((int64_t)bh * tokens + o) * head_dim + c * 8) * sizeof(T));
    store8(raster_out + ((((int64_t)b * tokens + raster) * heads + h) * head_dim + c * 8) * sizeof(T), val);
}

template <typename T>
__global__ __launch_bounds__(256) void merge_kernel(const char* exact, const float* exact_lse, const char* approx,
                                                    const float* approx_lse, const float* corr, char* raster_out,
                                                    TokenMap map, int tokens, int head_dim, int heads) {
    typedef typename Elem<T>::vec8 vec8;
    const int per_token = head_dim / 8;
    const int tokens_per_wg = 256 / per_token;
    const int wgs_per_bh = (tokens + tokens_per_wg - 1) / tokens_per_wg;
    const int bh = blockIdx.x / wgs_per_bh;
    const int o = (blockIdx.x - bh * wgs_per_bh) * tokens_per_wg + threadIdx.x / per_token;
    const int c = threadIdx.x % per_token;
    if (o >= tokens || threadIdx.x >= tokens_per_wg * per_token) return;
    const int b = bh / heads;
    const int h = bh - b * heads;
    const int64_t row = (int64_t)bh * tokens + o;
    const float le = exact_lse[row];
    const float la = approx_lse[row];
    const float mx = fmaxf(le, la);
    const float total = mx + logf(expf(le - mx) + expf(la - mx));
    const float we = expf(le - total);
    const float wa = expf(la - total);
    const int64_t off = row * head_dim + c * 8;
    const vec8 xe = load8_nt<vec8>(exact + off * sizeof(T));
    const vec8 xa = load8_nt<vec8>(approx + off * sizeof(T));
    const f32x4 c0 = *reinterpret_cast<const f32x4*>(corr + off);
    const f32x4 c1 = *reinterpret_cast<const f32x4*>(corr + off + 4);
    vec8 res;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float ce = e < 4 ? c0[e] : c1[e - 4];
        res[e] = from_f32<T>(to_f32(xe[e]) * we + to_f32(xa[e]) * wa + ce * wa);
    }
    store8(raster_out + ((((int64_t)b * tokens + map(o)) * heads + h) * head_dim + c * 8) * sizeof(T), res);
}

static int layout_grid(int bh_count, int tokens, int head_dim) {
    const int per_token = head_dim / 8;
    const int tokens_per_wg = 256 / per_token;
    return bh_count * ((tokens + tokens_per_wg - 1) / tokens_per_wg);
}

int launch_pack(int dtype, const LayoutArgs& a, int bh_count, hipStream_t stream) {
    const dim3 grid(layout_grid(bh_count, a.tokens, a.head_dim));
    if (dtype == PISA_DTYPE_BF16) hipLaunchKernelGGL(pack_kernel<bf16_t>, grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL(pack_kernel<f16_t>, grid, dim3(256), 0, stream, a);
    return pisa_host::check_launch("pack_kernel");
}

int launch_unpack(int dtype, const char* packed, char* out, TokenMap map, int tokens, int head_dim, int heads,
                  int bh_count, hipStream_t stream) {
    const dim3 grid(layout_grid(bh_count, tokens, head_dim));
    if (dtype == PISA_DTYPE_BF16)
        hipLaunchKernelGGL(unpack_kernel<bf16_t>, grid, dim3(256), 0, stream, packed, out, map, tokens, head_dim, heads);
    else
        hipLaunchKernelGGL(unpack_kernel<f16_t>, grid, dim3(256), 0, stream, packed, out, map, tokens, head_dim, heads);
    return pisa_host::check_launch("unpack_kernel");
}

int launch_merge(int dtype, const char* exact, const float* exact_lse, const char* approx, const float* approx_lse,
                 const float* corr, char* out, TokenMap map, int tokens, int head_dim, int heads, int bh_count,
                 hipStream_t stream) {
    const dim3 grid(layout_grid(bh_count, tokens, head_dim));
    if (dtype == PISA_DTYPE_BF16)
        hipLaunchKernelGGL(merge_kernel<bf16_t>, grid, dim3(256), 0, stream, exact, exact_lse, approx, approx_lse, corr,
                           out, map, tokens, head_dim, heads);
    else
        hipLaunchKernelGGL(merge_kernel<f16_t>, grid, dim3(256), 0, stream, exact, exact_lse, approx, approx_lse, corr,
                           out, map, tokens, head_dim, heads);
    return pisa_host::check_launch("merge_kernel");
}

}  // namespace pisa
