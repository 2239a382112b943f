// Context, arena and host<->device copies of libom_hip.so.
#include "om_internal.hpp"

#include <cstring>
#include <mutex>

namespace {
std::mutex g_null_ctx_mu;
std::string g_null_ctx_err;  // message for failures before a context exists
}  // namespace

namespace om {

om_status fail(om_ctx *ctx, om_status code, const char *fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (ctx) {
        ctx->err = buf;
    } else {
        std::lock_guard<std::mutex> g(g_null_ctx_mu);
        g_null_ctx_err = buf;
    }
    return code;
}

om_status check_hip(om_ctx *ctx, hipError_t e, const char *what) {
    if (e == hipSuccess) return OM_OK;
    return fail(ctx, e == hipErrorOutOfMemory ? OM_E_OOM : OM_E_DEVICE, "%s: %s", what, hipGetErrorString(e));
}

static om_status grow(om_ctx *ctx, float *&buf, uint64_t &have, uint64_t bytes, float **out, const char *what) {
    if (bytes <= have) {
        *out = buf;
        return OM_OK;
    }
    // No kernel may still use the old buffer.
    om_status s = check_hip(ctx, hipStreamSynchronize(ctx->stream), "scratch sync");
    if (s) return s;
    if (buf) (void)hipFree(buf);
    buf = nullptr;
    have = 0;
    uint64_t want = bytes < (64ull << 20) ? (64ull << 20) : bytes + (bytes >> 2);
    s = check_hip(ctx, hipMalloc(&buf, want), what);
    if (s) return s;
    have = want;
    *out = buf;
    return OM_OK;
}
om_status scratch(om_ctx *ctx, uint64_t bytes, float **out) {
    return grow(ctx, ctx->scratch, ctx->scratch_bytes, bytes, out, "scratch alloc");
}
om_status scratch2(om_ctx *ctx, uint64_t bytes, float **out) {
    return grow(ctx, ctx->scratch2, ctx->scratch2_bytes, bytes, out, "scratch alloc");
}

}  // namespace om

static om_status add_slab(om_ctx *ctx, om_region &r, uint64_t bytes) {
    om_slab s;
    hipError_t e = hipMalloc(&s.base, bytes);
    if (e != hipSuccess) return om::check_hip(ctx, e, "arena slab");
    s.size = bytes;
    r.slabs.push_back(s);
    return OM_OK;
}

extern "C" {

int om_abi_version(void) { return 100; }

om_status om_ctx_create(int device, om_ctx **out) {
    if (!out) return om::fail(nullptr, OM_E_ARG, "om_ctx_create: out is NULL");
    *out = nullptr;
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count == 0)
        return om::fail(nullptr, OM_E_DEVICE, "om_ctx_create: no HIP device (%s)", hipGetErrorString(e));
    if (device < 0 || device >= count) return om::fail(nullptr, OM_E_ARG, "om_ctx_create: device %d of %d", device, count);
    e = hipSetDevice(device);
    if (e != hipSuccess) return om::fail(nullptr, OM_E_DEVICE, "hipSetDevice: %s", hipGetErrorString(e));
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) == hipSuccess && std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return om::fail(nullptr, OM_E_DEVICE, "om_ctx_create: device %d is %s; this library is built for gfx950 only",
                        device, prop.gcnArchName);
    om_ctx *ctx = new om_ctx();
    ctx->device = device;
    ctx->num_cus = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
    // Default priority stream (never a prioritised one).
    e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete ctx;
        return om::fail(nullptr, OM_E_DEVICE, "hipStreamCreate: %s", hipGetErrorString(e));
    }
    ctx->region[0].default_slab = 64ull << 20;
    ctx->region[1].default_slab = 256ull << 20;
    // A failed lookup leaves only om_layernorm_bwd_noalloc unusable (it reports the error); everything else works.
    (void)om::noalloc_init(ctx);
    ctx->err.clear();
    *out = ctx;
    return OM_OK;
}

om_status om_ctx_destroy(om_ctx *ctx) {
    OM_CHECK_CTX(ctx);
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    for (auto &r : ctx->region)
        for (auto &s : r.slabs) (void)hipFree(s.base);
    if (ctx->scratch) (void)hipFree(ctx->scratch);
    if (ctx->scratch2) (void)hipFree(ctx->scratch2);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return OM_OK;
}

om_status om_ctx_sync(om_ctx *ctx) {
    OM_CHECK_CTX(ctx);
    return om::check_hip(ctx, hipStreamSynchronize(ctx->stream), "om_ctx_sync");
}

const char *om_last_error(om_ctx *ctx) {
    if (!ctx) {
        std::lock_guard<std::mutex> g(g_null_ctx_mu);
        return g_null_ctx_err.c_str();
    }
    return ctx->err.c_str();
}

void *om_ctx_stream(om_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

om_status om_arena_reserve(om_ctx *ctx, uint64_t persistent_bytes, uint64_t step_bytes) {
    OM_CHECK_CTX(ctx);
    uint64_t want[2] = {persistent_bytes, step_bytes};
    for (int i = 0; i < 2; i++) {
        om_region &r = ctx->region[i];
        if (want[i] == 0) continue;
        uint64_t have = 0;
        for (auto &s : r.slabs) have += s.size;
        if (have >= want[i]) continue;
        om_status st = add_slab(ctx, r, want[i] - have);
        if (st) return st;
    }
    return OM_OK;
}

om_status om_alloc(om_ctx *ctx, int region, uint64_t bytes, void **out) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, out && (region == 0 || region == 1), "om_alloc: bad region %d or NULL out", region);
    *out = nullptr;
    om_region &r = ctx->region[region];
    uint64_t need = (bytes + 255) & ~uint64_t(255);
    if (need == 0) need = 256;
    while (true) {
        if (r.cur < r.slabs.size()) {
            om_slab &s = r.slabs[r.cur];
            if (r.off + need <= s.size) {
                *out = s.base + r.off;
                r.off += need;
                r.used += need;
                return OM_OK;
            }
            if (r.cur + 1 < r.slabs.size()) {  // next slab already exists: move on
                r.cur++;
                r.off = 0;
                continue;
            }
        }
        uint64_t sz = need > r.default_slab ? need : r.default_slab;
        om_status st = add_slab(ctx, r, sz);
        if (st) return om::fail(ctx, OM_E_OOM, "om_alloc: %llu bytes in region %d: %s", (unsigned long long)bytes,
                                region, ctx->err.c_str());
        r.cur = r.slabs.size() - 1;
        r.off = 0;
    }
}

om_status om_step_reset(om_ctx *ctx) {
    OM_CHECK_CTX(ctx);
    om_region &r = ctx->region[OM_REGION_STEP];
    r.cur = 0;
    r.off = 0;
    r.used = 0;
    return OM_OK;
}

om_status om_arena_stats(om_ctx *ctx, int region, uint64_t *used, uint64_t *reserved) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, region == 0 || region == 1, "om_arena_stats: bad region %d", region);
    uint64_t have = 0;
    for (auto &s : ctx->region[region].slabs) have += s.size;
    if (used) *used = ctx->region[region].used;
    if (reserved) *reserved = have;
    return OM_OK;
}

om_status om_upload(om_ctx *ctx, void *dst, const void *src, uint64_t bytes) {
    OM_CHECK_CTX(ctx);
    if (bytes == 0) return OM_OK;
    OM_REQUIRE(ctx, dst && src, "om_upload: NULL pointer");
    // Pageable host memory: the copy is staged by the runtime and completes before the call returns.
    return om::check_hip(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream), "om_upload");
}

om_status om_download(om_ctx *ctx, void *dst, const void *src, uint64_t bytes) {
    OM_CHECK_CTX(ctx);
    if (bytes == 0) return OM_OK;
    OM_REQUIRE(ctx, dst && src, "om_download: NULL pointer");
    om_status s = om::check_hip(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream), "om_download");
    if (s) return s;
    return om::check_hip(ctx, hipStreamSynchronize(ctx->stream), "om_download sync");
}

om_status om_copy(om_ctx *ctx, void *dst, const void *src, uint64_t bytes) {
    OM_CHECK_CTX(ctx);
    if (bytes == 0) return OM_OK;
    OM_REQUIRE(ctx, dst && src, "om_copy: NULL pointer");
    return om::check_hip(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream), "om_copy");
}

}  // extern "C"

__global__ void k_fill(float *__restrict__ d, float v, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) d[i] = v;
}
__global__ void k_zero_bytes(unsigned char *__restrict__ d, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) d[i] = 0;
}

extern "C" om_status om_fill(om_ctx *ctx, float *dst, float value, int64_t n) {
    OM_CHECK_CTX(ctx);
    if (n <= 0) return OM_OK;
    OM_REQUIRE(ctx, dst, "om_fill: NULL pointer");
    hipLaunchKernelGGL(k_fill, dim3(om::grid1d(n, 256, 8192)), dim3(256), 0, ctx->stream, dst, value, n);
    return OM_LAUNCH_CHECK(ctx, "om_fill");
}

extern "C" om_status om_zero(om_ctx *ctx, void *dst, uint64_t bytes) {
    OM_CHECK_CTX(ctx);
    if (bytes == 0) return OM_OK;
    OM_REQUIRE(ctx, dst, "om_zero: NULL pointer");
    if ((bytes & 3) == 0 && ((uintptr_t)dst & 3) == 0) return om_fill(ctx, (float *)dst, 0.0f, (int64_t)(bytes >> 2));
    hipLaunchKernelGGL(k_zero_bytes, dim3(om::grid1d((int64_t)bytes, 256, 8192)), dim3(256), 0, ctx->stream,
                       (unsigned char *)dst, (int64_t)bytes);
    return OM_LAUNCH_CHECK(ctx, "om_zero");
}
