// Context, arena and host<->device copies of libom_hip.so.
#include "om_internal.hpp"

#include <atomic>
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

om_status refuse_in_capture(om_ctx *ctx, const char *what) {
    if (!ctx->cap) return OM_OK;
    return fail(ctx, OM_E_STATE, "%s: not possible inside a step-graph capture (it would wait for the device or read "
                "host memory when the graph runs)", what);
}

static om_status grow(om_ctx *ctx, float *&buf, uint64_t &have, uint64_t bytes, float **out, const char *what) {
    if (bytes <= have) {
        *out = buf;
        return OM_OK;
    }
    // Growth synchronises the stream, which a capture cannot hold; a step run once outside the capture has grown it.
    if (om_status s = refuse_in_capture(ctx, "context scratch growth")) return s;
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
    om_status s = grow(ctx, ctx->scratch, ctx->scratch_bytes, bytes, out, "scratch alloc");
    return s ? s : poison(ctx, *out, bytes);
}
om_status scratch2(om_ctx *ctx, uint64_t bytes, float **out) {
    om_status s = grow(ctx, ctx->scratch2, ctx->scratch2_bytes, bytes, out, "scratch alloc");
    return s ? s : poison(ctx, *out, bytes);
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

constexpr int kProbeMax = 1024;
int om::probe_begin(om_ctx *ctx) {
    if (!ctx->probe_on || ctx->cap || ctx->probe_n >= kProbeMax) return -1;
    const int i = ctx->probe_n;
    while ((int)ctx->probe_ev.size() < 2 * (i + 1)) {
        hipEvent_t e;
        if (hipEventCreate(&e) != hipSuccess) return -1;
        ctx->probe_ev.push_back(e);
    }
    if (hipEventRecord(ctx->probe_ev[2 * i], ctx->stream) != hipSuccess) return -1;
    return i;
}
void om::probe_end(om_ctx *ctx, int slot) {
    if (slot < 0 || slot != ctx->probe_n) return;
    if (hipEventRecord(ctx->probe_ev[2 * slot + 1], ctx->stream) == hipSuccess) ctx->probe_n++;
}

extern "C" {

int om_abi_version(void) { return 105; }
int om_build_checked(void) {
#ifdef OM_CHECKED
    return 1;
#else
    return 0;
#endif
}

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
    if (ctx->cap) (void)om_graph_capture_abort(ctx);
    (void)hipStreamSynchronize(ctx->stream);
    om::noalloc_release(ctx);  // the stream is idle: no launch of this context still uses its slot
    for (auto &r : ctx->region)
        for (auto &s : r.slabs) (void)hipFree(s.base);
    if (ctx->scratch) (void)hipFree(ctx->scratch);
    if (ctx->scratch2) (void)hipFree(ctx->scratch2);
    for (hipEvent_t e : ctx->probe_ev) (void)hipEventDestroy(e);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return OM_OK;
}

om_status om_ctx_set_gelu(om_ctx *ctx, int mode) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, mode == OM_GELU_FAST || mode == OM_GELU_REFERENCE,
               "om_ctx_set_gelu: mode must be OM_GELU_FAST or OM_GELU_REFERENCE");
    ctx->gelu_mode = mode;
    return OM_OK;
}

om_status om_ctx_probe(om_ctx *ctx, int on) {
    OM_CHECK_CTX(ctx);
    if (on) ctx->probe_n = 0;
    ctx->probe_on = on != 0;
    return OM_OK;
}

om_status om_ctx_probe_read(om_ctx *ctx, int *calls, double *mean_ms) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, calls && mean_ms, "om_ctx_probe_read: NULL output");
    if (om_status s = om::refuse_in_capture(ctx, "om_ctx_probe_read")) return s;
    if (om_status s = om::check_hip(ctx, hipStreamSynchronize(ctx->stream), "om_ctx_probe_read")) return s;
    double sum = 0.0;
    for (int i = 0; i < ctx->probe_n; i++) {
        float ms = 0.0f;
        if (om_status s = om::check_hip(ctx, hipEventElapsedTime(&ms, ctx->probe_ev[2 * i], ctx->probe_ev[2 * i + 1]),
                                        "om_ctx_probe_read"))
            return s;
        sum += ms;
    }
    *calls = ctx->probe_n;
    *mean_ms = ctx->probe_n ? sum / ctx->probe_n : 0.0;
    return OM_OK;
}

om_status om_ctx_sync(om_ctx *ctx) {
    OM_CHECK_CTX(ctx);
    if (om_status s = om::refuse_in_capture(ctx, "om_ctx_sync")) return s;
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
    if (r.limit && r.used + need > r.limit)
        return om::fail(ctx, OM_E_OOM, "om_alloc: %llu bytes in region %d: over the limit of %llu bytes set by "
                        "om_arena_set_limit (%llu in use)", (unsigned long long)bytes, region,
                        (unsigned long long)r.limit, (unsigned long long)r.used);
    while (true) {
        if (r.cur < r.slabs.size()) {
            om_slab &s = r.slabs[r.cur];
            if (r.off + need <= s.size) {
                *out = s.base + r.off;
                r.off += need;
                r.used += need;
                return om::poison(ctx, *out, need);
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

om_status om_arena_set_limit(om_ctx *ctx, int region, uint64_t bytes) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, region == 0 || region == 1, "om_arena_set_limit: bad region %d", region);
    ctx->region[region].limit = bytes;
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
    if (om_status s = om::refuse_in_capture(ctx, "om_upload")) return s;
    // Pageable host memory: the copy is staged by the runtime and completes before the call returns.
    return om::check_hip(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream), "om_upload");
}

om_status om_download(om_ctx *ctx, void *dst, const void *src, uint64_t bytes) {
    OM_CHECK_CTX(ctx);
    if (bytes == 0) return OM_OK;
    OM_REQUIRE(ctx, dst && src, "om_download: NULL pointer");
    if (om_status s = om::refuse_in_capture(ctx, "om_download")) return s;
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
    OM_LDS_POISON();
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) d[i] = v;
}
__global__ void k_fill_bits(unsigned *__restrict__ d, unsigned v, int64_t n) {
    OM_LDS_POISON();
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) d[i] = v;
}
__global__ void k_zero_bytes(unsigned char *__restrict__ d, int64_t n) {
    OM_LDS_POISON();
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) d[i] = 0;
}

om_status om::poison(om_ctx *ctx, void *p, uint64_t bytes) {
#ifdef OM_CHECKED
    const int64_t n = (int64_t)(bytes / 4);  // allocations and scratch are 256-byte aligned: whole words
    if (n > 0)
        hipLaunchKernelGGL(k_fill_bits, dim3(om::grid1d(n, 256, 8192)), dim3(256), 0, ctx->stream,
                           static_cast<unsigned *>(p), 0xFFFFFFFFu, n);
    return OM_LAUNCH_CHECK(ctx, "checked-build poison fill");
#else
    (void)ctx;
    (void)p;
    (void)bytes;
    return OM_OK;
#endif
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

// ------------------------------------------------------------------------------------------------ step graphs
namespace {

// The graph's first node: copies the values the host wrote for this launch into device memory for the later nodes,
// then tells the host the entry may be overwritten (the launch number into the ack word). The entry is read as two
// 16-byte loads (one PCIe round trip; the memory is fine-grained, so nothing is cached on the way), and the ack is
// stored only after both have returned (s_waitcnt on every counter), so the host never overwrites an entry that is
// still being read. No system-scope fence: the later nodes read `dev` in stream order, and the host needs only the
// ack word itself.
__global__ void k_step_begin(const om_step_block *entry, om_step_block *dev, uint64_t *ack) {
    OM_LDS_POISON();
    if (threadIdx.x != 0) return;
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 *src = reinterpret_cast<const u32x4 *>(entry);
    const u32x4 lo = __builtin_nontemporal_load(src), hi = __builtin_nontemporal_load(src + 1);
    u32x4 *dst = reinterpret_cast<u32x4 *>(dev);
    dst[0] = lo;
    dst[1] = hi;
    __builtin_amdgcn_s_waitcnt(0);
    const uint64_t id = (uint64_t)hi.z | ((uint64_t)hi.w << 32);  // om_step_block::id
    __hip_atomic_store(ack, id, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

om_step_block *entry_of(om_graph *g) { return reinterpret_cast<om_step_block *>(g->host); }
volatile uint64_t *ack_of(om_graph *g) { return reinterpret_cast<volatile uint64_t *>(g->host + sizeof(om_step_block)); }

void free_graph(om_graph *g) {
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    if (g->dev) (void)hipFree(g->dev);
    if (g->host) (void)hipHostFree(g->host);
    delete g;
}

}  // namespace

extern "C" {

om_status om_graph_capture_begin(om_ctx *ctx) {
    OM_CHECK_CTX(ctx);
    if (ctx->cap) return om::fail(ctx, OM_E_STATE, "om_graph_capture_begin: a capture is already running");
    om_graph *g = new om_graph;
    g->ctx = ctx;
    // Fine-grained (coherent) pinned memory: the first node reads what the host wrote just before the launch, and
    // the host polls the ack the node writes, with no cache in between.
    hipError_t e = hipHostMalloc((void **)&g->host, 64, hipHostMallocCoherent);
    if (e == hipSuccess) e = hipMalloc((void **)&g->dev, sizeof(om_step_block));
    if (e != hipSuccess) {
        free_graph(g);
        return om::check_hip(ctx, e, "om_graph_capture_begin");
    }
    std::memset(g->host, 0, 64);
    e = hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeRelaxed);
    if (e != hipSuccess) {
        free_graph(g);
        return om::check_hip(ctx, e, "om_graph_capture_begin");
    }
    ctx->cap = g;
    hipLaunchKernelGGL(k_step_begin, dim3(1), dim3(64), 0, ctx->stream, (const om_step_block *)g->host, g->dev,
                       (uint64_t *)(g->host + sizeof(om_step_block)));
    om_status s = OM_LAUNCH_CHECK(ctx, "om_graph_capture_begin");
    if (s) {
        std::string msg = ctx->err;
        (void)om_graph_capture_abort(ctx);
        ctx->err = msg;
    }
    return s;
}

om_status om_graph_capture_abort(om_ctx *ctx) {
    OM_CHECK_CTX(ctx);
    om_graph *g = ctx->cap;
    if (!g) return OM_OK;
    ctx->cap = nullptr;
    hipGraph_t partial = nullptr;
    (void)hipStreamEndCapture(ctx->stream, &partial);
    if (partial) (void)hipGraphDestroy(partial);
    (void)hipGetLastError();
    free_graph(g);
    return OM_OK;
}

om_status om_graph_capture_end(om_ctx *ctx, om_graph **out) {
    OM_CHECK_CTX(ctx);
    if (!ctx->cap) return om::fail(ctx, OM_E_STATE, "om_graph_capture_end: no capture is running");
    if (!out) {
        (void)om_graph_capture_abort(ctx);
        return om::fail(ctx, OM_E_ARG, "om_graph_capture_end: out is NULL");
    }
    *out = nullptr;
    om_graph *g = ctx->cap;
    ctx->cap = nullptr;
    hipError_t e = hipStreamEndCapture(ctx->stream, &g->graph);
    if (e == hipSuccess) e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        free_graph(g);
        return om::check_hip(ctx, e, "om_graph_capture_end");
    }
    *out = g;
    return OM_OK;
}

om_status om_graph_launch(om_graph *g, const om_step_values *v) {
    if (!g || !v) return OM_E_ARG;
    om_ctx *ctx = g->ctx;
    if (ctx->cap) return om::fail(ctx, OM_E_STATE, "om_graph_launch: a capture is running on the stream");
    // The entry is reused: the previous launch's first node must have read it (it normally has: the host waited for
    // that launch's loss, which comes later in the graph).
    for (uint64_t n = 1; *ack_of(g) != g->launches; n++) {
        if (n % 256) continue;
        hipError_t e = hipStreamQuery(ctx->stream);
        if (e == hipErrorNotReady) continue;
        if (e != hipSuccess) return om::check_hip(ctx, e, "om_graph_launch");
        if (*ack_of(g) != g->launches) return om::fail(ctx, OM_E_DEVICE, "om_graph_launch: the previous launch did not start");
    }
    uint64_t seq = 0;
    if (g->rb) {
        // The readback's previous post (eager or graph) must have landed before its buffer is written again.
        char *dst;
        uint64_t *seq_at;
        const uint64_t *seq_dev;
        om_status s = om::readback_target(ctx, g->rb, g->rb_bytes, &dst, &seq_at, &seq, &seq_dev);
        if (s) return s;
    }
    om_step_block *entry = entry_of(g);
    entry->lr = v->lr;
    entry->step_size = v->step_size;
    entry->sqrt_bc2 = v->sqrt_bc2;
    entry->pad = 0.0f;
    entry->seq = seq;
    entry->id = g->launches + 1;
    std::atomic_thread_fence(std::memory_order_seq_cst);
    om_status s = om::check_hip(ctx, hipGraphLaunch(g->exec, ctx->stream), "om_graph_launch");
    if (s) return s;
    g->launches++;
    if (g->rb) om::readback_posted(g->rb, seq, g->rb_bytes);
    return OM_OK;
}

om_status om_graph_destroy(om_graph *g) {
    if (!g) return OM_OK;
    om_status s = om::check_hip(g->ctx, hipStreamSynchronize(g->ctx->stream), "om_graph_destroy");
    free_graph(g);
    return s;
}

}  // extern "C"
