// extern "C" entry points of libpisa_hip.so (declared in include/pisa_hip.h):
// argument validation, workspace carving and kernel orchestration.  Nothing
// here allocates device memory or synchronises: every call enqueues its
// kernels on the caller's stream and returns.
#include <stdarg.h>
#include <algorithm>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <string>


#include "kernels.hpp"

namespace pisa_host {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
}

int fail(int status, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return status;
}

int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(PISA_ERR_LAUNCH, "%s launch failed: %s", what, hipGetErrorString(e));
    return PISA_OK;
}

bool valid_dtype(int dtype) { return dtype == PISA_DTYPE_BF16 || dtype == PISA_DTYPE_F16; }

static int elem_size(int dtype) { return dtype == PISA_DTYPE_F32 ? 4 : 2; }

// The library ships gfx950 code objects only; refuse other devices with a
// clear message instead of a launch failure.
static int check_device() {
    static std::mutex mu;
    static int cached[64];
    static bool init = false;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(PISA_ERR_DEVICE, "hipGetDevice failed");
    if (dev < 0 || dev >= 64) return fail(PISA_ERR_DEVICE, "device index %d out of range", dev);
    std::lock_guard<std::mutex> lock(mu);
    if (!init) {
        for (int i = 0; i < 64; ++i) cached[i] = -1;
        init = true;
    }
    if (cached[dev] < 0) {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, dev) != hipSuccess)
            return fail(PISA_ERR_DEVICE, "hipGetDeviceProperties failed for device %d", dev);
        cached[dev] = strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
        if (!cached[dev]) {
            set_error("device %d is %s; this library is built for gfx950 only", dev, prop.gcnArchName);
            return PISA_ERR_DEVICE;
        }
    }
    if (!cached[dev]) return fail(PISA_ERR_DEVICE, "device %d is not gfx950; this library is built for gfx950 only", dev);
    return PISA_OK;
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

static int check_view(const char* name, const pisa_view& v, int esize, bool vec16) {
    if (!v.data) return fail(PISA_ERR_INVALID_ARGUMENT, "%s is null", name);
    if (vec16) {
        if (!aligned16(v.data)) return fail(PISA_ERR_INVALID_ARGUMENT, "%s must be 16-byte aligned", name);
        const int64_t unit = 16 / esize;
        if (v.batch_stride % unit || v.head_stride % unit || v.token_stride % unit)
            return fail(PISA_ERR_INVALID_ARGUMENT, "%s strides must be multiples of %lld elements", name, (long long)unit);
    }
    return PISA_OK;
}

// Launch sizes: the block grids are 1-D with at most 256 threads per
// workgroup (so below 2^24 workgroups the thread count stays under 2^32) and
// the H_sum reductions run one grid row per head (at most 65535 rows).
constexpr int64_t kMaxBatchHeads = 65535;
constexpr int64_t kMaxGridBlocks = (int64_t(1) << 24) - 1;

static bool sizes_fit(int32_t batch, int32_t heads, int32_t tokens) {
    const int64_t bh = (int64_t)batch * heads;
    return bh <= kMaxBatchHeads && bh * (((int64_t)tokens + pisa::kBlock - 1) / pisa::kBlock) <= kMaxGridBlocks;
}

static int check_sizes(const char* what, int32_t batch, int32_t heads, int32_t tokens) {
    if (sizes_fit(batch, heads, tokens)) return PISA_OK;
    return fail(PISA_ERR_UNSUPPORTED, "%s supports B*H <= %lld and B*H*ceil(T/64) <= %lld blocks, got B=%d H=%d T=%d",
                what, (long long)kMaxBatchHeads, (long long)kMaxGridBlocks, batch, heads, tokens);
}

static int check_grid(const pisa_token_grid& g, int tokens) {
    if (g.frames <= 0) return PISA_OK;
    if (g.height <= 0 || g.width <= 0 || g.height % 8 || g.width % 8)
        return fail(PISA_ERR_INVALID_ARGUMENT, "token grid height/width must be positive multiples of 8");
    if ((int64_t)g.frames * g.height * g.width != tokens)
        return fail(PISA_ERR_INVALID_ARGUMENT, "token grid %dx%dx%d does not match %d tokens", g.frames, g.height,
                    g.width, tokens);
    return PISA_OK;
}

static pisa::View to_view(const pisa_view& v, int heads) {
    pisa::View r;
    r.data = static_cast<const char*>(v.data);
    r.sb = v.batch_stride;
    r.sh = v.head_stride;
    r.st = v.token_stride;
    r.heads = heads;
    return r;
}

static pisa::OutView to_out(const pisa_view& v, int heads) {
    pisa::OutView r;
    r.data = static_cast<char*>(v.data);
    r.sb = v.batch_stride;
    r.sh = v.head_stride;
    r.st = v.token_stride;
    r.heads = heads;
    return r;
}

// ---- workspace carving
struct Carver {
    char* base;
    int64_t off = 0;
    explicit Carver(void* b) : base(static_cast<char*>(b)) {}
    template <typename P> P* take(int64_t bytes) {
        P* p = base ? reinterpret_cast<P*>(base + off) : nullptr;
        off += (bytes + 255) & ~int64_t(255);
        return p;
    }
};

struct StatsPlan {
    int blocks, npad, chunks, chunk_blocks, mask_words;
};

// The statistics grid is bh x chunks workgroups of chunk_blocks consecutive
// blocks; two workgroups fit a CU (LDS), so 512 run at once.  The chunking
// minimises (rounds of 512 workgroups) x (blocks of a workgroup + its start-up,
// about three blocks' time): a grid of 520 workgroups would run its last 8 as
// a second round of a whole workgroup's time (C5: 40 heads x 13 chunks of 40
// blocks; 12 chunks of 43 fit one round).
static StatsPlan plan_stats(int bh, int tokens) {
    constexpr int kSlots = 512;
    constexpr int kStartBlocks = 3;
    StatsPlan p;
    p.blocks = (tokens + pisa::kBlock - 1) / pisa::kBlock;
    p.npad = (p.blocks + 63) / 64 * 64;
    p.chunk_blocks = p.blocks;
    p.chunks = 1;
    int64_t best = -1;
    for (int c = 1; c <= p.blocks && c <= 1024; ++c) {
        const int cb = (p.blocks + c - 1) / c;
        const int cc = (p.blocks + cb - 1) / cb;
        const int64_t rounds = ((int64_t)bh * cc + kSlots - 1) / kSlots;
        const int64_t cost = rounds * (cb + kStartBlocks);
        if (best < 0 || cost < best) {
            best = cost;
            p.chunk_blocks = cb;
            p.chunks = cc;
        }
    }
    p.mask_words = (p.blocks + 31) / 32;
    return p;
}

struct ForwardBuffers {
    void* qc;
    float* qc_route;
    float* kc;
    void* vm;
    float* hnorm;
    float* hpart;
    void* kp;
    void* vp;
    void* kbar_pad;
    void* vbar_t_pad;
    void* ht;
    int32_t* idx;
    uint32_t* selmask;
    int64_t total;
};

// Chunks of the H_sum partials at head dims other than 128 (stats_cov_kernel:
// one wave per (head, chunk, 32x32 tile of H)): about 2048 waves, at most 16
// chunks per head.
static void plan_cov(int bh, int blocks, int padded, int* chunks, int* chunk_blocks) {
    const int per_chunk = bh * (padded / 32) * (padded / 32);
    const int c = std::max(1, std::min((2048 + per_chunk - 1) / per_chunk, std::min(blocks, 16)));
    *chunk_blocks = (blocks + c - 1) / c;
    *chunks = (blocks + *chunk_blocks - 1) / *chunk_blocks;
}

// Means and routing buffers have the real head dim; the packed tables the
// attention kernel reads have the padded one.  The H_sum partials and the
// packed H_sum^T have width 128 at head dim 128 (chunks of the statistics
// kernel) and the padded width otherwise (chunks of plan_cov).
static ForwardBuffers carve_forward(void* ws, int bh, int tokens, int head_dim, int exact, int esize) {
    const StatsPlan p = plan_stats(bh, tokens);
    const int padded = pisa::padded_head_dim(head_dim) ? pisa::padded_head_dim(head_dim) : head_dim;
    const int cov_dim = head_dim == 128 ? head_dim : padded;
    int cov_chunks = p.chunks, cov_chunk_blocks = p.chunk_blocks;
    if (head_dim != 128) plan_cov(bh, p.blocks, padded, &cov_chunks, &cov_chunk_blocks);
    const int64_t nd = (int64_t)bh * p.blocks * head_dim;
    const int64_t ndp = (int64_t)bh * p.blocks * padded;
    Carver c(ws);
    ForwardBuffers f;
    f.qc = c.take<void>(nd * esize);
    f.qc_route = c.take<float>(nd * 4);
    f.kc = c.take<float>(nd * 4);
    f.vm = c.take<void>(nd * esize);
    f.hnorm = c.take<float>((int64_t)bh * p.blocks * 4);
    f.hpart = c.take<float>((int64_t)bh * cov_chunks * cov_dim * cov_dim * 4);
    f.kp = c.take<void>(ndp * pisa::kBlock * esize);
    f.vp = c.take<void>(ndp * pisa::kBlock * esize);
    f.kbar_pad = c.take<void>((int64_t)bh * p.npad * padded * esize);
    f.vbar_t_pad = c.take<void>((int64_t)bh * p.npad * padded * esize);
    f.ht = c.take<void>((int64_t)bh * cov_dim * cov_dim * esize);
    f.idx = c.take<int32_t>((int64_t)bh * p.blocks * (exact > 0 ? exact : 1) * 4);
    f.selmask = c.take<uint32_t>((int64_t)bh * p.blocks * p.mask_words * 4);
    f.total = c.off;
    return f;
}

static bool workspace_ok(void* ws, int64_t have, int64_t need) { return need == 0 || (ws && have >= need && aligned16(ws)); }

}  // namespace pisa_host

using namespace pisa_host;

extern "C" {

int pisa_hip_api_version(void) { return PISA_HIP_API_VERSION; }

const char* pisa_hip_status_string(int status) {
    switch (status) {
        case PISA_OK: return "ok";
        case PISA_ERR_INVALID_ARGUMENT: return "invalid argument";
        case PISA_ERR_UNSUPPORTED: return "unsupported configuration";
        case PISA_ERR_WORKSPACE: return "workspace too small";
        case PISA_ERR_LAUNCH: return "kernel launch failed";
        case PISA_ERR_DEVICE: return "unsupported device";
        default: return "unknown status";
    }
}

const char* pisa_hip_last_error(void) { return g_last_error.c_str(); }

int pisa_hip_build_info(char* buffer, int64_t capacity) {
    char info[512];
    const int n = snprintf(info, sizeof(info),
                           "api=%d;architecture=gfx950;implementation=hip_mfma_fused_pisa;"
                           "hip_build_version=%d.%d.%d;block_size=%d;head_dim=128;max_blocks=%d",
                           PISA_HIP_API_VERSION, HIP_VERSION_MAJOR, HIP_VERSION_MINOR, HIP_VERSION_PATCH,
                           PISA_BLOCK_SIZE, pisa::kMaxRouteBlocks);
    if (!buffer || capacity <= n) return fail(PISA_ERR_INVALID_ARGUMENT, "build_info buffer too small");
    memcpy(buffer, info, n + 1);
    return PISA_OK;
}

int64_t pisa_hip_forward_workspace_bytes(int32_t batch, int32_t heads, int32_t tokens, int32_t head_dim,
                                         int32_t exact_blocks) {
    if (batch <= 0 || heads <= 0 || tokens <= 0 || head_dim <= 0 || !sizes_fit(batch, heads, tokens)) return 0;
    return carve_forward(nullptr, batch * heads, tokens, head_dim, exact_blocks, 2).total;
}

}  // extern "C"

namespace pisa_host {

// Validation shared by the three PISA entry points; fills the plan on success.
static int validate_forward(int32_t dtype, int32_t batch, int32_t heads, int32_t tokens, int32_t head_dim,
                            const pisa_view& q, const pisa_view& k, const pisa_view& v, const pisa_view& out,
                            const pisa_token_grid& grid, int32_t exact_blocks, float scale, int32_t sink_block,
                            int32_t stats_mode, int32_t route_mode, int32_t first_order, void* workspace,
                            int64_t workspace_bytes, StatsPlan* plan) {
    if (!valid_dtype(dtype)) return fail(PISA_ERR_UNSUPPORTED, "PISA forward supports bf16 and fp16 only");
    if (batch <= 0 || heads <= 0 || tokens <= 0)
        return fail(PISA_ERR_INVALID_ARGUMENT, "PISA forward requires B>0, H>0, T>0");
    int rc;
    if ((rc = check_sizes("PISA forward", batch, heads, tokens))) return rc;
    if (head_dim != 128) {
        // other head dims take the Triton statistics (generic_pisa.py:128-138,
        // pisa_kernel.py:90-130: any head dim up to 256, H_sum included) and
        // centroid routing (no HYD bias, so no H_b norms)
        if (!pisa::padded_head_dim(head_dim))
            return fail(PISA_ERR_UNSUPPORTED, "PISA forward supports head_dim a multiple of 8 up to 256, got %d",
                        head_dim);
        if (stats_mode != PISA_STATS_GENERIC || route_mode != PISA_ROUTE_CENTROID)
            return fail(PISA_ERR_UNSUPPORTED, "head_dim %d requires GENERIC statistics and CENTROID routing", head_dim);
    }
    const int bh = batch * heads;
    const StatsPlan p = plan_stats(bh, tokens);
    if (p.blocks > pisa::kMaxRouteBlocks)
        return fail(PISA_ERR_UNSUPPORTED, "PISA forward supports at most %d blocks, got %d", pisa::kMaxRouteBlocks, p.blocks);
    if (exact_blocks < 0 || exact_blocks >= p.blocks)
        return fail(PISA_ERR_INVALID_ARGUMENT, "exact_blocks must be in [0,%d) for the sparse path, got %d", p.blocks,
                    exact_blocks);
    if (sink_block != PISA_NO_SINK && sink_block != 0 && sink_block != -1)
        return fail(PISA_ERR_INVALID_ARGUMENT, "sink_block must be None, -1, or 0");
    if (sink_block != PISA_NO_SINK && exact_blocks == 0)
        return fail(PISA_ERR_INVALID_ARGUMENT, "sink_block requires at least one exact block");
    if (!(scale > 0.0f) || scale == __builtin_inff()) return fail(PISA_ERR_INVALID_ARGUMENT, "scale must be positive and finite");
    if (stats_mode != PISA_STATS_HYD && stats_mode != PISA_STATS_GENERIC)
        return fail(PISA_ERR_INVALID_ARGUMENT, "stats_mode must be HYD or GENERIC");
    if (route_mode != PISA_ROUTE_HYD && route_mode != PISA_ROUTE_CENTROID)
        return fail(PISA_ERR_INVALID_ARGUMENT, "route_mode must be HYD or CENTROID");
    if ((rc = check_grid(grid, tokens)) || (rc = check_view("q", q, 2, true)) || (rc = check_view("k", k, 2, true)) ||
        (rc = check_view("v", v, 2, true)) || (rc = check_view("out", out, 2, false)))
        return rc;
    if (out.token_stride % 4 || out.head_stride % 4 || out.batch_stride % 4 || (reinterpret_cast<uintptr_t>(out.data) & 7))
        return fail(PISA_ERR_INVALID_ARGUMENT, "out must be 8-byte aligned with strides multiple of 4 elements");
    const ForwardBuffers need = carve_forward(nullptr, bh, tokens, head_dim, exact_blocks, 2);
    if (!workspace_ok(workspace, workspace_bytes, need.total))
        return fail(PISA_ERR_WORKSPACE, "workspace of %lld bytes (16-byte aligned) required, got %lld",
                    (long long)need.total, (long long)workspace_bytes);
    if ((rc = check_device())) return rc;
    *plan = p;
    return PISA_OK;
}

static int route_impl(const ForwardBuffers& w, int32_t head_dim, int32_t exact_blocks, float scale,
                      int32_t sink_block, int32_t route_mode, int32_t* debug_indices, float* debug_scores,
                      const StatsPlan& p, int bh, hipStream_t st, int32_t dtype = 0,
                      const pisa::ReduceArgs* fused_reduce = nullptr);

static int prepare_impl(int32_t dtype, int32_t heads, int32_t tokens, int32_t head_dim, const pisa_view& q,
                        const pisa_view& k, const pisa_view& v, const pisa_token_grid& grid, int32_t exact_blocks,
                        float scale, int32_t sink_block, int32_t stats_mode, int32_t route_mode, int32_t first_order,
                        int32_t* debug_indices, float* debug_scores, void* workspace, const StatsPlan& p, int bh,
                        hipStream_t st) {
    const ForwardBuffers w = carve_forward(workspace, bh, tokens, head_dim, exact_blocks, 2);
    pisa::StatsArgs sa;
    memset(&sa, 0, sizeof(sa));
    sa.q = to_view(q, heads);
    sa.k = to_view(k, heads);
    sa.v = to_view(v, heads);
    sa.map = pisa::make_token_map(grid);
    sa.tokens = tokens;
    sa.blocks = p.blocks;
    sa.chunk_blocks = p.chunk_blocks;
    sa.chunks = p.chunks;
    sa.qc_out = w.qc;
    sa.qc_f32 = 0;
    // bf16 HYD routing at head dim 128 reads the bf16 means and the packed
    // centroid chunks (route_impl), so the fp32 routing means are not written;
    // the dtype value means are never read by the forward (the tail reads the
    // packed value chunks)
    const bool bf16_route = head_dim == 128 && dtype == PISA_DTYPE_BF16 && route_mode == PISA_ROUTE_HYD;
    sa.kc_out = bf16_route ? nullptr : w.kc;
    sa.vm_out = nullptr;
    sa.vm_f32 = 0;
    sa.hnorm_out = w.hnorm;
    sa.hpart = w.hpart;
    sa.qc_route = bf16_route ? nullptr : w.qc_route;
    // generic routing on HYD statistics multiplies the dtype-rounded q_bar with
    // the fp32 k_bar (generic_pisa.py:120-126,172-173: block_stats_hyd returns
    // q_bar in the input dtype, routed as q_bar.float())
    sa.qc_route_round = (stats_mode == PISA_STATS_HYD && route_mode == PISA_ROUTE_CENTROID) ? 1 : 0;
    sa.kp_blocks = w.kp;
    sa.vp_blocks = w.vp;
    sa.kbar_pad = w.kbar_pad;
    sa.vbar_t_pad = w.vbar_t_pad;
    sa.npad = p.npad;
    sa.head_dim = head_dim;
    int rc;
    if (head_dim != 128) {
        const int padded = pisa::padded_head_dim(head_dim);
        if ((rc = pisa::launch_stats_means(dtype, padded, sa, bh, st, false))) return rc;
        if ((rc = pisa::launch_kv_pack(dtype, padded, head_dim, sa.k, sa.v, sa.map, tokens, p.blocks, bh,
                                       static_cast<char*>(w.kp), static_cast<char*>(w.vp), st)))
            return rc;
        if (first_order) {
            // H_sum of the Triton statistics (pisa_kernel.py:80-84) from the
            // block means just written, then dtype(H_sum)^T for the correction
            pisa::CovArgs ca{};
            ca.k = sa.k;
            ca.v = sa.v;
            ca.map = sa.map;
            ca.tokens = tokens;
            ca.blocks = p.blocks;
            ca.head_dim = head_dim;
            plan_cov(bh, p.blocks, padded, &ca.chunks, &ca.chunk_blocks);
            ca.kmean = w.kc;
            ca.hpart = w.hpart;
            if ((rc = pisa::launch_stats_cov(dtype, padded, ca, bh, st, false))) return rc;
            pisa::ReduceArgs cr{};
            cr.hpart = w.hpart;
            cr.chunks = ca.chunks;
            cr.ht = w.ht;
            cr.blocks = p.blocks;
            cr.npad = p.npad;
            if ((rc = pisa::launch_cov_reduce(dtype, padded, cr, bh, st))) return rc;
        }
        return route_impl(w, head_dim, exact_blocks, scale, sink_block, route_mode, debug_indices, debug_scores, p, bh,
                          st);
    }
    if ((rc = pisa::launch_stats(dtype, stats_mode, sa, bh, st))) return rc;

    pisa::ReduceArgs ra{};
    ra.hpart = w.hpart;
    ra.chunks = p.chunks;
    ra.hsum = nullptr;
    ra.ht = first_order ? w.ht : nullptr;
    ra.kbar_pad = w.kbar_pad;
    ra.vbar_t_pad = w.vbar_t_pad;
    ra.blocks = p.blocks;
    ra.npad = p.npad;
    // the routing workgroups also sum the H_sum partials (one launch)
    return route_impl(w, head_dim, exact_blocks, scale, sink_block, route_mode, debug_indices, debug_scores, p, bh, st,
                      dtype, &ra);
}

static int route_impl(const ForwardBuffers& w, int32_t head_dim, int32_t exact_blocks, float scale,
                      int32_t sink_block, int32_t route_mode, int32_t* debug_indices, float* debug_scores,
                      const StatsPlan& p, int bh, hipStream_t st, int32_t dtype,
                      const pisa::ReduceArgs* fused_reduce) {
    int rc;
    pisa::RouteArgs ro;
    ro.qc = w.qc_route;
    ro.kc = w.kc;
    ro.hnorm = route_mode == PISA_ROUTE_HYD ? w.hnorm : nullptr;
    ro.rows = bh * p.blocks;
    ro.blocks = p.blocks;
    ro.head_dim = head_dim;
    ro.round_bf16 = route_mode == PISA_ROUTE_HYD ? 1 : 0;
    ro.sink = sink_block;
    ro.k = exact_blocks;
    ro.scale = scale;
    ro.idx = w.idx;
    ro.scores = debug_scores;
    ro.selmask = w.selmask;
    ro.mask_words = p.mask_words;
    const bool bf16_means = fused_reduce && route_mode == PISA_ROUTE_HYD && dtype == PISA_DTYPE_BF16 && head_dim == 128;
    ro.qc_bf16 = bf16_means ? static_cast<const pisa::bf16_t*>(w.qc) : nullptr;
    ro.kc_pack = bf16_means ? static_cast<const pisa::bf16_t*>(w.kbar_pad) : nullptr;
    ro.npad = p.npad;
    if (fused_reduce) rc = pisa::launch_route_reduce(dtype, ro, *fused_reduce, st);
    else rc = pisa::launch_route(ro, st);
    if (rc) return rc;
    if (debug_indices && exact_blocks > 0) {
        if (hipMemcpyAsync(debug_indices, w.idx, (size_t)bh * p.blocks * exact_blocks * 4, hipMemcpyDeviceToDevice, st) !=
            hipSuccess)
            return fail(PISA_ERR_LAUNCH, "copy of debug indices failed");
    }
    return PISA_OK;
}

static int attend_impl(int32_t dtype, int32_t heads, int32_t tokens, int32_t head_dim, const pisa_view& q,
                       const pisa_view& k, const pisa_view& out, const pisa_token_grid& grid, int32_t exact_blocks,
                       float scale, int32_t first_order, void* workspace, const StatsPlan& p, int bh, hipStream_t st) {
    const ForwardBuffers w = carve_forward(workspace, bh, tokens, head_dim, exact_blocks, 2);
    const pisa::TokenMap map = pisa::make_token_map(grid);
    pisa::AttnArgs aa;
    aa.q = to_view(q, heads);
    aa.o = to_out(out, heads);
    aa.kp = static_cast<const char*>(w.kp);
    aa.vp = static_cast<const char*>(w.vp);
    aa.qmap = map;
    aa.q_tokens = tokens;
    aa.kv_tokens = tokens;
    aa.q_blocks = p.blocks;
    aa.kv_blocks = p.blocks;
    aa.scale_log2 = scale * pisa::kLog2e;
    aa.inv_scale_log2 = 1.0f / aa.scale_log2;
    aa.idx = w.idx;
    aa.exact = exact_blocks;
    aa.kbar = static_cast<const char*>(w.kbar_pad);
    aa.vbar_t = static_cast<const char*>(w.vbar_t_pad);
    aa.selmask = w.selmask;
    aa.mask_words = p.mask_words;
    aa.npad = p.npad;
    aa.centroids = p.blocks;
    const int last_len = tokens - (p.blocks - 1) * pisa::kBlock;
    aa.last_len_log2 = log2f(static_cast<float>(last_len));
    aa.ht = first_order ? static_cast<const char*>(w.ht) : nullptr;
    aa.corr_scale = scale / static_cast<float>(tokens);
    aa.head_dim = head_dim;
    return pisa::launch_attention(dtype, pisa::padded_head_dim(head_dim), true, true, aa, bh, st);
}

}  // namespace pisa_host

extern "C" {

int pisa_hip_forward(int32_t dtype, int32_t batch, int32_t heads, int32_t tokens, int32_t head_dim, pisa_view q,
                     pisa_view k, pisa_view v, pisa_view out, pisa_token_grid grid, int32_t exact_blocks, float scale,
                     int32_t sink_block, int32_t stats_mode, int32_t route_mode, int32_t first_order,
                     int32_t* debug_indices, float* debug_scores, void* workspace, int64_t workspace_bytes,
                     void* stream) {
    StatsPlan p;
    int rc = validate_forward(dtype, batch, heads, tokens, head_dim, q, k, v, out, grid, exact_blocks, scale,
                              sink_block, stats_mode, route_mode, first_order, workspace, workspace_bytes, &p);
    if (rc) return rc;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int bh = batch * heads;
    if ((rc = prepare_impl(dtype, heads, tokens, head_dim, q, k, v, grid, exact_blocks, scale, sink_block, stats_mode,
                           route_mode, first_order, debug_indices, debug_scores, workspace, p, bh, st)))
        return rc;
    return attend_impl(dtype, heads, tokens, head_dim, q, k, out, grid, exact_blocks, scale, first_order, workspace, p,
                       bh, st);
}

int pisa_hip_prepare(int32_t dtype, int32_t batch, int32_t heads, int32_t tokens, int32_t head_dim, pisa_view q,
                     pisa_view k, pisa_view v, pisa_view out, pisa_token_grid grid, int32_t exact_blocks, float scale,
                     int32_t sink_block, int32_t stats_mode, int32_t route_mode, int32_t first_order,
                     void* workspace, int64_t workspace_bytes, void* stream) {
    StatsPlan p;
    int rc = validate_forward(dtype, batch, heads, tokens, head_dim, q, k, v, out, grid, exact_blocks, scale,
                              sink_block, stats_mode, route_mode, first_order, workspace, workspace_bytes, &p);
    if (rc) return rc;
    return prepare_impl(dtype, heads, tokens, head_dim, q, k, v, grid, exact_blocks, scale, sink_block, stats_mode,
                        route_mode, first_order, nullptr, nullptr, workspace, p, batch * heads,
                        static_cast<hipStream_t>(stream));
}

int pisa_hip_attend(int32_t dtype, int32_t batch, int32_t heads, int32_t tokens, int32_t head_dim, pisa_view q,
                    pisa_view k, pisa_view v, pisa_view out, pisa_token_grid grid, int32_t exact_blocks, float scale,
                    int32_t sink_block, int32_t stats_mode, int32_t route_mode, int32_t first_order,
                    void* workspace, int64_t workspace_bytes, void* stream) {
    StatsPlan p;
    int rc = validate_forward(dtype, batch, heads, tokens, head_dim, q, k, v, out, grid, exact_blocks, scale,
                              sink_block, stats_mode, route_mode, first_order, workspace, workspace_bytes, &p);
    if (rc) return rc;
    return attend_impl(dtype, heads, tokens, head_dim, q, k, out, grid, exact_blocks, scale, first_order, workspace, p,
                       batch * heads, static_cast<hipStream_t>(stream));
}

// ---- allocation-free forward (pisa_hip_forward_noalloc) -----------------
// Callers that cannot allocate (code under HIP graph capture, tight serving
// loops, hosts that forbid hipMalloc) run the PISA forward in this file-scope
// device array instead of a caller workspace.  Every GPU the library runs on
// holds its own copy (PISA_NOALLOC_SCRATCH_BYTES) until the process ends.  Its
// device address is looked up once per device with hipGetSymbolAddress; host
// code never uses the array's name as an address (on the host it is only a
// stand-in for the symbol).
static __device__ __align__(256) unsigned char scratch[PISA_NOALLOC_SCRATCH_BYTES];

}  // extern "C"

namespace pisa_host {

static int scratch_address(void** out) {
    static std::mutex mu;
    static void* per_device[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(PISA_ERR_DEVICE, "hipGetDevice failed");
    if (dev < 0 || dev >= 64) return fail(PISA_ERR_DEVICE, "device index %d out of range", dev);
    std::lock_guard<std::mutex> lock(mu);
    if (!per_device[dev]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            return fail(PISA_ERR_DEVICE, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                        hipGetErrorString(e));
        per_device[dev] = ptr;
    }
    *out = per_device[dev];
    return PISA_OK;
}

}  // namespace pisa_host

extern "C" {

int pisa_hip_forward_noalloc(int32_t dtype, int32_t batch, int32_t heads, int32_t tokens, int32_t head_dim,
                             pisa_view q, pisa_view k, pisa_view v, pisa_view out, pisa_token_grid grid,
                             int32_t exact_blocks, float scale, int32_t sink_block, int32_t stats_mode,
                             int32_t route_mode, int32_t first_order, void* stream) {
    // the size check comes first, so an oversized problem never touches the device
    const int64_t need = pisa_hip_forward_workspace_bytes(batch, heads, tokens, head_dim, exact_blocks);
    if (need > PISA_NOALLOC_SCRATCH_BYTES)
        return fail(PISA_ERR_WORKSPACE,
                    "pisa_hip_forward_noalloc: this problem needs %lld bytes of scratch, the static scratch holds %lld "
                    "(use pisa_hip_forward with a caller workspace)",
                    (long long)need, (long long)PISA_NOALLOC_SCRATCH_BYTES);
    if (!valid_dtype(dtype)) return fail(PISA_ERR_UNSUPPORTED, "PISA forward supports bf16 and fp16 only");
    void* ws = nullptr;
    int rc;
    if ((rc = check_device()) || (rc = scratch_address(&ws))) return rc;
    return pisa_hip_forward(dtype, batch, heads, tokens, head_dim, q, k, v, out, grid, exact_blocks, scale,
                            sink_block, stats_mode, route_mode, first_order, nullptr, nullptr, ws,
                            PISA_NOALLOC_SCRATCH_BYTES, stream);
}

// Head dims other than 128: the H_sum partials of plan_cov's chunks, then the
// per-block tile sums of squares of H_b that the norms are reduced from.
static int64_t cov_partial_bytes(int bh, int blocks, int padded) {
    int chunks, chunk_blocks;
    plan_cov(bh, blocks, padded, &chunks, &chunk_blocks);
    return ((int64_t)bh * chunks * padded * padded * 4 + 255) / 256 * 256;
}

// Padded width of the block statistics off head dim 128: any 0 < D <= 256
// (dims past D are zero), 0 otherwise.
static int stats_padded_dim(int head_dim) {
    return head_dim > 0 && head_dim <= 256 ? pisa::padded_head_dim((head_dim + 7) & ~7) : 0;
}

int64_t pisa_hip_block_stats_workspace_bytes(int32_t batch, int32_t heads, int32_t tokens, int32_t head_dim) {
    if (batch <= 0 || heads <= 0 || tokens <= 0 || head_dim <= 0 || !sizes_fit(batch, heads, tokens)) return 0;
    const StatsPlan p = plan_stats(batch * heads, tokens);
    if (head_dim == 128) return (int64_t)batch * heads * p.chunks * head_dim * head_dim * 4;
    const int padded = stats_padded_dim(head_dim);
    if (!padded) return 0;
    const int tiles = (padded / 32) * (padded / 32);
    return cov_partial_bytes(batch * heads, p.blocks, padded) + (int64_t)batch * heads * p.blocks * tiles * 4;
}

int pisa_hip_block_stats(int32_t dtype, int32_t out_dtype, int32_t batch, int32_t heads, int32_t tokens,
                         int32_t head_dim, pisa_view q, pisa_view k, pisa_view v, pisa_token_grid grid,
                         int32_t stats_mode, void* q_centroids, float* k_centroids, void* v_means, float* h_sum,
                         float* h_norm, void* workspace, int64_t workspace_bytes, void* stream) {
    if (!valid_dtype(dtype)) return fail(PISA_ERR_UNSUPPORTED, "block statistics support bf16 and fp16 only");
    if (out_dtype != dtype && out_dtype != PISA_DTYPE_F32)
        return fail(PISA_ERR_INVALID_ARGUMENT, "out_dtype must equal dtype or be float32");
    if (batch <= 0 || heads <= 0 || tokens <= 0) return fail(PISA_ERR_INVALID_ARGUMENT, "requires B>0, H>0, T>0");
    int rc;
    if ((rc = check_sizes("block statistics", batch, heads, tokens))) return rc;
    const bool value_sums = (stats_mode & PISA_STATS_FLAG_VALUE_SUMS) != 0;
    stats_mode &= ~PISA_STATS_FLAG_VALUE_SUMS;
    if (stats_mode != PISA_STATS_MEANS && stats_mode != PISA_STATS_HYD && stats_mode != PISA_STATS_GENERIC)
        return fail(PISA_ERR_INVALID_ARGUMENT, "unknown stats_mode %d", stats_mode);
    if (value_sums && (stats_mode == PISA_STATS_MEANS || out_dtype != PISA_DTYPE_F32))
        return fail(PISA_ERR_INVALID_ARGUMENT, "value sums need HYD or GENERIC statistics and float32 outputs");
    // head dims other than 128: the HYD statistics (block_stats_hyd takes any
    // 0 < D <= 256, pisa_kernels.cu:605) and the Triton statistics
    // (pisa_kernel.py:90-130, any width up to 256, padded)
    const int padded = head_dim == 128 ? 128 : stats_padded_dim(head_dim);
    if (!padded) return fail(PISA_ERR_UNSUPPORTED, "block statistics support 0 < head_dim <= 256, got %d", head_dim);
    if (!q_centroids || !k_centroids || !v_means) return fail(PISA_ERR_INVALID_ARGUMENT, "centroid outputs are required");
    const bool cov = stats_mode != PISA_STATS_MEANS;
    // h_norm: required for HYD; optional for GENERIC off 128 (the Triton
    // statistics form no norms), required at 128 where the kernel writes them
    if (cov && (!h_sum || (!h_norm && (stats_mode == PISA_STATS_HYD || head_dim == 128))))
        return fail(PISA_ERR_INVALID_ARGUMENT, "h_sum and h_norm are required");
    // 16-byte row loads at widths that are multiples of 8; element loads otherwise
    const bool rows16 = head_dim % 8 == 0;
    if ((rc = check_grid(grid, tokens)) || (rc = check_view("q", q, 2, rows16)) ||
        (rc = check_view("k", k, 2, rows16)) || (rc = check_view("v", v, 2, rows16)))
        return rc;
    const int bh = batch * heads;
    const StatsPlan p = plan_stats(bh, tokens);
    const int64_t need = cov ? pisa_hip_block_stats_workspace_bytes(batch, heads, tokens, head_dim) : 0;
    if (!workspace_ok(workspace, workspace_bytes, need))
        return fail(PISA_ERR_WORKSPACE, "workspace of %lld bytes required, got %lld", (long long)need,
                    (long long)workspace_bytes);
    if ((rc = check_device())) return rc;
    hipStream_t st = static_cast<hipStream_t>(stream);
    pisa::StatsArgs sa;
    memset(&sa, 0, sizeof(sa));
    sa.q = to_view(q, heads);
    sa.k = to_view(k, heads);
    sa.v = to_view(v, heads);
    sa.map = pisa::make_token_map(grid);
    sa.tokens = tokens;
    sa.blocks = p.blocks;
    sa.chunk_blocks = p.chunk_blocks;
    sa.chunks = p.chunks;
    sa.qc_out = q_centroids;
    sa.qc_f32 = out_dtype == PISA_DTYPE_F32;
    sa.kc_out = k_centroids;
    sa.vm_out = v_means;
    sa.vm_f32 = out_dtype == PISA_DTYPE_F32;
    sa.vm_sums = value_sums ? 1 : 0;
    sa.hnorm_out = cov ? h_norm : nullptr;
    sa.hpart = cov ? static_cast<float*>(workspace) : nullptr;
    sa.npad = p.npad;
    sa.head_dim = head_dim;
    if (head_dim != 128) {
        const bool hyd = stats_mode == PISA_STATS_HYD;
        if ((rc = pisa::launch_stats_means(dtype, padded, sa, bh, st, hyd))) return rc;
        if (!cov) return PISA_OK;
        pisa::CovArgs ca{};
        ca.k = sa.k;
        ca.v = sa.v;
        ca.map = sa.map;
        ca.tokens = tokens;
        ca.blocks = p.blocks;
        ca.head_dim = head_dim;
        plan_cov(bh, p.blocks, padded, &ca.chunks, &ca.chunk_blocks);
        ca.kmean = k_centroids;
        ca.hpart = static_cast<float*>(workspace);
        ca.normpart = h_norm ? reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                                        cov_partial_bytes(bh, p.blocks, padded))
                             : nullptr;
        if ((rc = pisa::launch_stats_cov(dtype, padded, ca, bh, st, hyd))) return rc;
        pisa::ReduceArgs cr{};
        cr.hpart = ca.hpart;
        cr.chunks = ca.chunks;
        cr.hsum = h_sum;
        cr.hsum_dim = head_dim;
        cr.blocks = p.blocks;
        cr.npad = p.npad;
        cr.normpart = ca.normpart;
        cr.hnorm = h_norm;
        return pisa::launch_cov_reduce(dtype, padded, cr, bh, st);
    }
    if ((rc = pisa::launch_stats(dtype, stats_mode, sa, bh, st))) return rc;
    if (!cov) return PISA_OK;
    pisa::ReduceArgs ra;
    memset(&ra, 0, sizeof(ra));
    ra.hpart = static_cast<float*>(workspace);
    ra.chunks = p.chunks;
    ra.hsum = h_sum;
    ra.blocks = p.blocks;
    ra.npad = p.npad;
    return pisa::launch_stats_reduce(dtype, ra, bh, st);
}

int pisa_hip_route_topk(int32_t batch_heads, int32_t blocks, int32_t head_dim, const float* qc, const float* kc,
                        const float* h_norm, int32_t round_bf16, float scale, int32_t sink_block, int32_t exact_blocks,
                        int32_t* indices, float* scores, void* stream) {
    if (batch_heads <= 0 || blocks <= 0) return fail(PISA_ERR_INVALID_ARGUMENT, "requires BH>0 and blocks>0");
    if (blocks > pisa::kMaxRouteBlocks) return fail(PISA_ERR_UNSUPPORTED, "at most %d blocks", pisa::kMaxRouteBlocks);
    int rc;
    if ((rc = check_sizes("routing", 1, batch_heads, blocks * pisa::kBlock))) return rc;
    if (head_dim <= 0 || head_dim > 256 || head_dim % 4)
        return fail(PISA_ERR_UNSUPPORTED, "head_dim must be a multiple of 4 in (0, 256]");
    if (exact_blocks < 0 || exact_blocks > blocks) return fail(PISA_ERR_INVALID_ARGUMENT, "exact_blocks out of range");
    if (sink_block != PISA_NO_SINK && sink_block != 0 && sink_block != -1)
        return fail(PISA_ERR_INVALID_ARGUMENT, "sink_block must be None, -1, or 0");
    if (!qc || !kc || (!indices && exact_blocks > 0)) return fail(PISA_ERR_INVALID_ARGUMENT, "null pointer argument");
    if (!aligned16(kc)) return fail(PISA_ERR_INVALID_ARGUMENT, "kc must be 16-byte aligned");
    if ((rc = check_device())) return rc;
    pisa::RouteArgs ro;
    ro.qc = qc;
    ro.kc = kc;
    ro.hnorm = h_norm;
    ro.rows = batch_heads * blocks;
    ro.blocks = blocks;
    ro.head_dim = head_dim;
    ro.round_bf16 = round_bf16 ? 1 : 0;
    ro.sink = sink_block;
    ro.k = exact_blocks;
    ro.scale = scale;
    ro.idx = indices;
    ro.scores = scores;
    ro.selmask = nullptr;
    ro.mask_words = 0;
    ro.qc_bf16 = nullptr;
    ro.kc_pack = nullptr;
    ro.npad = 0;
    return pisa::launch_route(ro, static_cast<hipStream_t>(stream));
}

int pisa_hip_pack_spatial_qkv(int32_t dtype, int32_t batch, int32_t heads, int32_t tokens, int32_t head_dim,
                              pisa_view q, pisa_view k, pisa_view v, pisa_token_grid grid, void* packed_q,
                              void* packed_k, void* packed_v, void* stream) {
    if (!valid_dtype(dtype)) return fail(PISA_ERR_UNSUPPORTED, "pack supports bf16 and fp16 only");
    if (batch <= 0 || heads <= 0 || tokens <= 0) return fail(PISA_ERR_INVALID_ARGUMENT, "requires B>0, H>0, T>0");
    if (head_dim <= 0 || head_dim % 8 || head_dim > 2048)
        return fail(PISA_ERR_UNSUPPORTED, "head_dim must be a multiple of 8 (<= 2048)");
    int rc;
    if ((rc = check_sizes("spatial layout", batch, heads, tokens))) return rc;
    if ((rc = check_grid(grid, tokens)) || (rc = check_view("q", q, 2, true)) || (rc = check_view("k", k, 2, true)) ||
        (rc = check_view("v", v, 2, true)))
        return rc;
    if (!packed_q || !packed_k || !packed_v || !aligned16(packed_q) || !aligned16(packed_k) || !aligned16(packed_v))
        return fail(PISA_ERR_INVALID_ARGUMENT, "packed outputs must be non-null and 16-byte aligned");
    if ((rc = check_device())) return rc;
    pisa::LayoutArgs la;
    la.in[0] = to_view(q, heads);
    la.in[1] = to_view(k, heads);
    la.in[2] = to_view(v, heads);
    la.out[0] = static_cast<char*>(packed_q);
    la.out[1] = static_cast<char*>(packed_k);
    la.out[2] = static_cast<char*>(packed_v);
    la.ntensors = 3;
    la.map = pisa::make_token_map(grid);
    la.tokens = tokens;
    la.head_dim = head_dim;
    la.heads = heads;
    return pisa::launch_pack(dtype, la, batch * heads, static_cast<hipStream_t>(stream));
}

int pisa_hip_unpack_spatial_output(int32_t dtype, int32_t batch, int32_t heads, int32_t tokens, int32_t head_dim,
                                   const void* packed, pisa_token_grid grid, void* raster, void* stream) {
    if (!valid_dtype(dtype)) return fail(PISA_ERR_UNSUPPORTED, "unpack supports bf16 and fp16 only");
    if (batch <= 0 || heads <= 0 || tokens <= 0) return fail(PISA_ERR_INVALID_ARGUMENT, "requires B>0, H>0, T>0");
    if (head_dim <= 0 || head_dim % 8 || head_dim > 2048)
        return fail(PISA_ERR_UNSUPPORTED, "head_dim must be a multiple of 8 (<= 2048)");
    int rc;
    if ((rc = check_sizes("spatial layout", batch, heads, tokens))) return rc;
    if ((rc = check_grid(grid, tokens))) return rc;
    if (!packed || !raster || !aligned16(packed) || !aligned16(raster))
        return fail(PISA_ERR_INVALID_ARGUMENT, "packed and raster must be non-null and 16-byte aligned");
    if ((rc = check_device())) return rc;
    return pisa::launch_unpack(dtype, static_cast<const char*>(packed), static_cast<char*>(raster),
                               pisa::make_token_map(grid), tokens, head_dim, heads, batch * heads,
                               static_cast<hipStream_t>(stream));
}

int pisa_hip_fuse_spatial_epilogue(int32_t dtype, int32_t batch, int32_t heads, int32_t tokens, int32_t head_dim,
                                   const void* exact_output, const float* exact_lse, const void* approximate_output,
                                   const float* approximate_lse, const float* correction, pisa_token_grid grid,
                                   void* out, void* stream) {
    if (!valid_dtype(dtype)) return fail(PISA_ERR_UNSUPPORTED, "epilogue supports bf16 and fp16 only");
    if (batch <= 0 || heads <= 0 || tokens <= 0) return fail(PISA_ERR_INVALID_ARGUMENT, "requires B>0, H>0, T>0");
    if (head_dim <= 0 || head_dim % 8 || head_dim > 2048)
        return fail(PISA_ERR_UNSUPPORTED, "head_dim must be a multiple of 8 (<= 2048)");
    int rc;
    if ((rc = check_sizes("spatial layout", batch, heads, tokens))) return rc;
    if ((rc = check_grid(grid, tokens))) return rc;
    if (!exact_output || !exact_lse || !approximate_output || !approximate_lse || !correction || !out)
        return fail(PISA_ERR_INVALID_ARGUMENT, "null pointer argument");
    if (!aligned16(exact_output) || !aligned16(approximate_output) || !aligned16(correction) || !aligned16(out))
        return fail(PISA_ERR_INVALID_ARGUMENT, "outputs and correction must be 16-byte aligned");
    if ((rc = check_device())) return rc;
    return pisa::launch_merge(dtype, static_cast<const char*>(exact_output), exact_lse,
                              static_cast<const char*>(approximate_output), approximate_lse, correction,
                              static_cast<char*>(out), pisa::make_token_map(grid), tokens, head_dim, heads,
                              batch * heads, static_cast<hipStream_t>(stream));
}

int64_t attn_hip_dense_workspace_bytes(int32_t batch, int32_t heads, int32_t kv_tokens, int32_t head_dim) {
    if (batch <= 0 || heads <= 0 || kv_tokens <= 0 || head_dim <= 0 || !sizes_fit(batch, heads, kv_tokens)) return 0;
    const int64_t blocks = (kv_tokens + pisa::kBlock - 1) / pisa::kBlock;
    const int padded = pisa::padded_head_dim(head_dim) ? pisa::padded_head_dim(head_dim) : head_dim;
    return 2 * (int64_t)batch * heads * blocks * padded * pisa::kBlock * 2;  // packed K and V blocks
}

int attn_hip_dense_forward(int32_t dtype, int32_t batch, int32_t heads, int32_t q_tokens, int32_t kv_tokens,
                           int32_t head_dim, pisa_view q, pisa_view k, pisa_view v, pisa_view out, float scale,
                           void* workspace, int64_t workspace_bytes, void* stream) {
    if (!valid_dtype(dtype)) return fail(PISA_ERR_UNSUPPORTED, "dense attention supports bf16 and fp16 only");
    if (batch <= 0 || heads <= 0 || q_tokens <= 0 || kv_tokens <= 0)
        return fail(PISA_ERR_INVALID_ARGUMENT, "requires B>0, H>0, Tq>0, Tk>0");
    int rc;
    if ((rc = check_sizes("dense attention", batch, heads, q_tokens)) ||
        (rc = check_sizes("dense attention", batch, heads, kv_tokens)))
        return rc;
    const int padded = pisa::padded_head_dim(head_dim);
    if (!padded)
        return fail(PISA_ERR_UNSUPPORTED, "dense attention supports head_dim a multiple of 8 up to 256, got %d",
                    head_dim);
    if (!(scale > 0.0f) || scale == __builtin_inff()) return fail(PISA_ERR_INVALID_ARGUMENT, "scale must be positive and finite");
    // the attention kernel addresses one head's packed key (value) table with
    // 32-bit byte offsets in a buffer resource
    const int64_t head_table_bytes = ((int64_t)kv_tokens + pisa::kBlock - 1) / pisa::kBlock * pisa::kBlock * padded * 2;
    if (head_table_bytes > INT32_MAX)
        return fail(PISA_ERR_UNSUPPORTED, "dense attention: Tk=%d at head_dim %d needs %lld bytes of packed keys per head, "
                    "above 2 GiB", kv_tokens, head_dim, (long long)head_table_bytes);
    if ((rc = check_view("q", q, 2, true)) || (rc = check_view("k", k, 2, true)) || (rc = check_view("v", v, 2, true)) ||
        (rc = check_view("out", out, 2, false)))
        return rc;
    if (out.token_stride % 4 || out.head_stride % 4 || out.batch_stride % 4 || (reinterpret_cast<uintptr_t>(out.data) & 7))
        return fail(PISA_ERR_INVALID_ARGUMENT, "out must be 8-byte aligned with strides multiple of 4 elements");
    const int64_t need = attn_hip_dense_workspace_bytes(batch, heads, kv_tokens, head_dim);
    if (!workspace_ok(workspace, workspace_bytes, need))
        return fail(PISA_ERR_WORKSPACE, "workspace of %lld bytes required, got %lld", (long long)need,
                    (long long)workspace_bytes);
    if ((rc = check_device())) return rc;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int bh = batch * heads;
    const int kv_blocks = (kv_tokens + pisa::kBlock - 1) / pisa::kBlock;
    const int64_t table_bytes = need / 2;
    char* kp = static_cast<char*>(workspace);
    char* vp = kp + table_bytes;
    if ((rc = pisa::launch_kv_pack(dtype, padded, head_dim, to_view(k, heads), to_view(v, heads),
                                   pisa::TokenMap{0, 0, 0}, kv_tokens, kv_blocks, bh, kp, vp, st)))
        return rc;
    pisa::AttnArgs aa;
    memset(&aa, 0, sizeof(aa));
    aa.q = to_view(q, heads);
    aa.o = to_out(out, heads);
    aa.kp = kp;
    aa.vp = vp;
    aa.qmap = pisa::TokenMap{0, 0, 0};
    aa.q_tokens = q_tokens;
    aa.kv_tokens = kv_tokens;
    aa.q_blocks = (q_tokens + pisa::kBlock - 1) / pisa::kBlock;
    aa.kv_blocks = kv_blocks;
    aa.scale_log2 = scale * pisa::kLog2e;
    aa.inv_scale_log2 = 1.0f / aa.scale_log2;
    aa.head_dim = head_dim;
    return pisa::launch_attention(dtype, padded, false, false, aa, bh, st);
}

int attn_hip_fixed_block_forward_masked(int32_t dtype, int32_t batch, int32_t heads, int32_t tokens,
                                        int32_t head_dim, int32_t block_size, pisa_view q, pisa_view k, pisa_view v,
                                        pisa_view out, float scale, int32_t causal, pisa_mask mask, void* stream) {
    if (dtype != PISA_DTYPE_BF16 && dtype != PISA_DTYPE_F16 && dtype != PISA_DTYPE_F32)
        return fail(PISA_ERR_UNSUPPORTED, "fixed-block attention supports bf16, fp16 and fp32");
    if (batch <= 0 || heads <= 0 || tokens <= 0) return fail(PISA_ERR_INVALID_ARGUMENT, "requires B>0, H>0, T>0");
    if (block_size != 64) return fail(PISA_ERR_UNSUPPORTED, "fixed-block attention supports block_size=64 only");
    int rc;
    if ((rc = check_sizes("fixed-block attention", batch, heads, tokens))) return rc;
    if (head_dim != 32 && head_dim != 64 && head_dim != 128)
        return fail(PISA_ERR_UNSUPPORTED, "fixed-block attention supports head_dim 32/64/128, got %d", head_dim);
    if (!(scale == scale) || scale == __builtin_inff() || scale == -__builtin_inff())
        return fail(PISA_ERR_INVALID_ARGUMENT, "scale must be finite");
    if (mask.kind < PISA_MASK_NONE || mask.kind > PISA_MASK_ADD_BF16)
        return fail(PISA_ERR_INVALID_ARGUMENT, "unknown mask kind %d", mask.kind);
    if (mask.kind != PISA_MASK_NONE) {
        const int esize = mask.kind == PISA_MASK_BOOL ? 1 : mask.kind == PISA_MASK_ADD_F32 ? 4 : 2;
        if (!mask.data || (reinterpret_cast<uintptr_t>(mask.data) & (esize - 1)))
            return fail(PISA_ERR_INVALID_ARGUMENT, "mask data must be non-null and aligned to its element size");
        if (mask.heads <= 0 || batch * heads % mask.heads)
            return fail(PISA_ERR_INVALID_ARGUMENT, "mask heads %d must divide B*H=%d", mask.heads, batch * heads);
    }
    const int es = elem_size(dtype);
    if ((rc = check_view("q", q, es, false)) || (rc = check_view("k", k, es, false)) ||
        (rc = check_view("v", v, es, false)) || (rc = check_view("out", out, es, false)))
        return rc;
    if ((rc = check_device())) return rc;
    pisa::MaskView mv;
    mv.data = static_cast<const char*>(mask.data);
    mv.kind = mask.kind;
    mv.heads = mask.kind != PISA_MASK_NONE ? mask.heads : 1;
    mv.sb = mask.batch_stride;
    mv.sh = mask.head_stride;
    mv.sq = mask.query_stride;
    mv.sk = mask.key_stride;
    return pisa::launch_fixed_block(dtype, head_dim, to_view(q, heads), to_view(k, heads), to_view(v, heads),
                                    to_out(out, heads), tokens, batch * heads, scale, causal ? 1 : 0, mv,
                                    static_cast<hipStream_t>(stream));
}

int attn_hip_fixed_block_forward(int32_t dtype, int32_t batch, int32_t heads, int32_t tokens, int32_t head_dim,
                                 int32_t block_size, pisa_view q, pisa_view k, pisa_view v, pisa_view out, float scale,
                                 int32_t causal, void* stream) {
    pisa_mask none;
    memset(&none, 0, sizeof(none));
    return attn_hip_fixed_block_forward_masked(dtype, batch, heads, tokens, head_dim, block_size, q, k, v, out, scale,
                                               causal, none, stream);
}

}  // extern "C"
