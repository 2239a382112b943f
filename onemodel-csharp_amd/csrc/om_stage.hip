// Host data staging: batches travel from the producer to HBM through a ring of pinned host slots, uploaded on a
// copy stream while the previous step computes.
//
// A slot is a pinned host buffer (hipHostMalloc) and a device buffer of the same size. The producer fills the host
// side in place (om_stager_begin hands out the pointer once the slot's previous upload has read it), om_stager_commit
// queues the upload on the copy stream behind the event that marks the slot's previous device copy consumed, the
// step makes the context's stream wait for the upload (om_stager_acquire) and marks the device copy consumed after
// its last launch (om_stager_release). Upload k+1 then runs on the DMA engines under step k. Both streams have the
// default priority.
#include <atomic>
#include <cstring>

#include "om_internal.hpp"

struct om_stager {
    om_ctx *ctx = nullptr;
    uint64_t slot_bytes = 0;
    int slots = 0;
    int next = 0;
    hipStream_t copy = nullptr;
    std::vector<char *> host;
    std::vector<char *> dev;
    std::vector<hipEvent_t> uploaded, consumed;
    std::vector<char> upload_pending, consume_pending, begun, in_use;
};

namespace {

om_status destroy(om_stager *s) {
    om_status st = OM_OK;
    if (s->copy && hipStreamSynchronize(s->copy) != hipSuccess) st = OM_E_DEVICE;
    if (s->ctx && s->ctx->stream && hipStreamSynchronize(s->ctx->stream) != hipSuccess) st = OM_E_DEVICE;
    for (char *p : s->host)
        if (p) (void)hipHostFree(p);
    for (char *p : s->dev)
        if (p) (void)hipFree(p);
    for (hipEvent_t e : s->uploaded)
        if (e) (void)hipEventDestroy(e);
    for (hipEvent_t e : s->consumed)
        if (e) (void)hipEventDestroy(e);
    if (s->copy) (void)hipStreamDestroy(s->copy);
    delete s;
    return st;
}

bool valid_slot(const om_stager *s, int slot) { return s && slot >= 0 && slot < s->slots; }

}  // namespace

extern "C" {

om_status om_stager_create(om_ctx *ctx, uint64_t slot_bytes, int slots, om_stager **out) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, out, "om_stager_create: out is NULL");
    *out = nullptr;
    OM_REQUIRE(ctx, slot_bytes > 0 && slots >= 2 && slots <= 64, "om_stager_create: need slot_bytes > 0 and 2..64 slots");
    om_stager *s = new om_stager;
    s->ctx = ctx;
    s->slot_bytes = slot_bytes;
    s->slots = slots;
    s->host.assign(slots, nullptr);
    s->dev.assign(slots, nullptr);
    s->uploaded.assign(slots, nullptr);
    s->consumed.assign(slots, nullptr);
    s->upload_pending.assign(slots, 0);
    s->consume_pending.assign(slots, 0);
    s->begun.assign(slots, 0);
    s->in_use.assign(slots, 0);
    hipError_t e = hipStreamCreateWithFlags(&s->copy, hipStreamNonBlocking);
    for (int i = 0; e == hipSuccess && i < slots; i++) {
        e = hipHostMalloc((void **)&s->host[i], slot_bytes, hipHostMallocDefault);
        if (e == hipSuccess) e = hipMalloc((void **)&s->dev[i], slot_bytes);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&s->uploaded[i], hipEventDisableTiming);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&s->consumed[i], hipEventDisableTiming);
    }
    if (e != hipSuccess) {
        destroy(s);
        return om::check_hip(ctx, e, "om_stager_create");
    }
    *out = s;
    return OM_OK;
}

om_status om_stager_destroy(om_stager *s) {
    if (!s) return OM_OK;
    return destroy(s);
}

uint64_t om_stager_slot_bytes(const om_stager *s) { return s ? s->slot_bytes : 0; }

om_status om_stager_begin(om_stager *s, void **host, int *slot) {
    if (!s) return OM_E_ARG;
    om_ctx *ctx = s->ctx;
    OM_REQUIRE(ctx, host && slot, "om_stager_begin: NULL output");
    const int k = s->next;
    OM_REQUIRE(ctx, !s->begun[k], "om_stager_begin: slot %d is still being filled (commit it first)", k);
    if (s->in_use[k])
        return om::fail(ctx, OM_E_STATE, "om_stager_begin: all %d slots hold batches not yet released", s->slots);
    // The pinned buffer is free once its previous upload has read it.
    if (s->upload_pending[k]) {
        om_status st = om::check_hip(ctx, hipEventSynchronize(s->uploaded[k]), "om_stager_begin wait");
        if (st) return st;
        s->upload_pending[k] = 0;
    }
    s->begun[k] = 1;
    s->next = (k + 1) % s->slots;
    *host = s->host[k];
    *slot = k;
    return OM_OK;
}

om_status om_stager_commit(om_stager *s, int slot, uint64_t bytes, void **device) {
    if (!valid_slot(s, slot)) return OM_E_ARG;
    om_ctx *ctx = s->ctx;
    OM_REQUIRE(ctx, s->begun[slot], "om_stager_commit: slot %d was not begun", slot);
    OM_REQUIRE(ctx, bytes <= s->slot_bytes, "om_stager_commit: %llu bytes exceed the slot size %llu",
               (unsigned long long)bytes, (unsigned long long)s->slot_bytes);
    // The device buffer is free once the step that read it has finished.
    if (s->consume_pending[slot]) {
        om_status st = om::check_hip(ctx, hipStreamWaitEvent(s->copy, s->consumed[slot], 0), "om_stager_commit wait");
        if (st) return st;
        s->consume_pending[slot] = 0;
    }
    if (bytes) {
        om_status st = om::check_hip(
            ctx, hipMemcpyAsync(s->dev[slot], s->host[slot], bytes, hipMemcpyHostToDevice, s->copy), "om_stager_commit");
        if (st) return st;
    }
    om_status st = om::check_hip(ctx, hipEventRecord(s->uploaded[slot], s->copy), "om_stager_commit record");
    if (st) return st;
    s->upload_pending[slot] = 1;
    s->begun[slot] = 0;
    s->in_use[slot] = 1;
    if (device) *device = s->dev[slot];
    return OM_OK;
}

om_status om_stager_acquire(om_stager *s, int slot) {
    if (!valid_slot(s, slot)) return OM_E_ARG;
    if (om_status st = om::refuse_in_capture(s->ctx, "om_stager_acquire")) return st;
    return om::check_hip(s->ctx, hipStreamWaitEvent(s->ctx->stream, s->uploaded[slot], 0), "om_stager_acquire");
}

om_status om_stager_release(om_stager *s, int slot) {
    if (!valid_slot(s, slot)) return OM_E_ARG;
    om_ctx *ctx = s->ctx;
    if (om_status st = om::refuse_in_capture(ctx, "om_stager_release")) return st;
    om_status st = om::check_hip(ctx, hipEventRecord(s->consumed[slot], ctx->stream), "om_stager_release");
    if (st) return st;
    s->consume_pending[slot] = 1;
    s->in_use[slot] = 0;
    return OM_OK;
}

}  // extern "C"

// Readback: a pinned host buffer that a one-workgroup kernel on the context's stream writes a device value into,
// through the buffer's device mapping, followed by a sequence number. The host polls that number instead of
// waiting on an event: an event's marker on the stream makes the queue drain before the next launch, which left the
// device idle for several microseconds in the middle of every training step. Launches queued after the post keep
// running while the host returns with the value.
struct om_readback {
    om_ctx *ctx = nullptr;
    uint64_t bytes = 0;
    char *host = nullptr;      // [data, rounded up to 8 bytes][uint64 sequence]
    char *host_dev = nullptr;  // the same buffer as the device addresses it
    uint64_t seq = 0;          // sequence number of the last post
    uint64_t posted = 0;       // bytes of the last post, 0 before the first
};

namespace {

constexpr uint64_t kReadbackMax = 64 << 10;

// Copies n bytes to dst, then, once every thread's stores have completed, writes seq after the data. The stores are
// system-scope write-through stores (global_store sc0 sc1) into the fine-grained host buffer and each thread waits
// for its own before the barrier, so the sequence number cannot overtake the data; no L2 write-back or invalidate
// is needed, which a system-scope fence would do to the whole L2 of the workgroup's XCD in the middle of a step.
// Inside a step graph the number is read from seq_dev when the kernel runs.
__global__ void __launch_bounds__(256) k_readback(char *__restrict__ dst, const char *__restrict__ src, uint64_t n,
                                                  uint64_t *seq_at, uint64_t seq, const uint64_t *seq_dev) {
    OM_LDS_POISON();
    for (uint64_t i = threadIdx.x; i < n; i += 256)
        __hip_atomic_store(dst + i, src[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0)
        __hip_atomic_store(seq_at, seq_dev ? *seq_dev : seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

volatile uint64_t *seq_host(const om_readback *r) {
    return reinterpret_cast<volatile uint64_t *>(r->host + (r->bytes + 7) / 8 * 8);
}

// Waits until the last post's sequence number has landed. Every 256 polls it asks the stream: an error is reported,
// and a stream that has finished everything must have written the number.
om_status await(om_readback *r) {
    om_ctx *ctx = r->ctx;
    for (uint64_t n = 1; *seq_host(r) != r->seq; n++) {
        if (n % 256) continue;
        hipError_t e = hipStreamQuery(ctx->stream);
        if (e == hipErrorNotReady) continue;
        if (e != hipSuccess) return om::check_hip(ctx, e, "om_readback_wait");
        if (*seq_host(r) != r->seq) return om::fail(ctx, OM_E_DEVICE, "om_readback_wait: the copy did not land");
    }
    std::atomic_thread_fence(std::memory_order_acquire);
    return OM_OK;
}

}  // namespace

namespace om {

om_status readback_target(om_ctx *ctx, om_readback *r, uint64_t bytes, char **dst, uint64_t **seq_at, uint64_t *seq,
                          const uint64_t **seq_dev) {
    OM_REQUIRE(ctx, r && r->ctx == ctx, "readback post: the readback belongs to another context");
    OM_REQUIRE(ctx, bytes > 0 && bytes <= r->bytes, "readback post: need 1 .. %llu bytes", (unsigned long long)r->bytes);
    *seq_dev = nullptr;
    if (om_graph *g = ctx->cap) {
        // Recorded into a step graph: each launch of the graph posts, with the number om_graph_launch assigns.
        if (g->rb && g->rb != r)
            return om::fail(ctx, OM_E_STATE, "readback post: a step graph holds one readback, this is a second one");
        g->rb = r;
        g->rb_bytes = bytes;
        *dst = r->host_dev;
        *seq_at = reinterpret_cast<uint64_t *>(r->host_dev + (r->bytes + 7) / 8 * 8);
        *seq = 0;
        *seq_dev = &g->dev->seq;
        return OM_OK;
    }
    // The pinned buffer may still be the target of the previous post.
    if (r->posted) {
        om_status st = await(r);
        if (st) return st;
    }
    *dst = r->host_dev;
    *seq_at = reinterpret_cast<uint64_t *>(r->host_dev + (r->bytes + 7) / 8 * 8);
    *seq = r->seq + 1;
    return OM_OK;
}

void readback_posted(om_readback *r, uint64_t seq, uint64_t bytes) {
    if (r->ctx->cap) return;  // recorded, not run: om_graph_launch advances the readback
    r->seq = seq;
    r->posted = bytes;
}

}  // namespace om

extern "C" {

om_status om_readback_create(om_ctx *ctx, uint64_t bytes, om_readback **out) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, out, "om_readback_create: out is NULL");
    *out = nullptr;
    OM_REQUIRE(ctx, bytes > 0 && bytes <= kReadbackMax, "om_readback_create: need 1 .. 64 KiB, got %llu",
               (unsigned long long)bytes);
    om_readback *r = new om_readback;
    r->ctx = ctx;
    r->bytes = bytes;
    const uint64_t total = (bytes + 7) / 8 * 8 + sizeof(uint64_t);
    // Fine-grained: the device's write-through stores land in host memory without a cache flush.
    hipError_t e = hipHostMalloc((void **)&r->host, total, hipHostMallocCoherent);
    if (e == hipSuccess) e = hipHostGetDevicePointer((void **)&r->host_dev, r->host, 0);
    if (e != hipSuccess) {
        if (r->host) (void)hipHostFree(r->host);
        delete r;
        return om::check_hip(ctx, e, "om_readback_create");
    }
    memset(r->host, 0, total);
    *out = r;
    return OM_OK;
}

om_status om_readback_destroy(om_readback *r) {
    if (!r) return OM_OK;
    om_status st = OM_OK;
    if (r->posted && hipStreamSynchronize(r->ctx->stream) != hipSuccess) st = OM_E_DEVICE;
    (void)hipHostFree(r->host);
    delete r;
    return st;
}

om_status om_readback_post(om_readback *r, const void *src, uint64_t bytes) {
    if (!r) return OM_E_ARG;
    om_ctx *ctx = r->ctx;
    OM_REQUIRE(ctx, src, "om_readback_post: NULL source");
    char *dst;
    uint64_t *seq_at, seq;
    const uint64_t *seq_dev;
    om_status st = om::readback_target(ctx, r, bytes, &dst, &seq_at, &seq, &seq_dev);
    if (st) return st;
    hipLaunchKernelGGL(k_readback, dim3(1), dim3(256), 0, ctx->stream, dst, static_cast<const char *>(src), bytes,
                       seq_at, seq, seq_dev);
    st = OM_LAUNCH_CHECK(ctx, "om_readback_post");
    if (st) return st;
    om::readback_posted(r, seq, bytes);
    return OM_OK;
}

om_status om_readback_wait(om_readback *r, void *dst, uint64_t bytes) {
    if (!r) return OM_E_ARG;
    om_ctx *ctx = r->ctx;
    if (!r->posted) return om::fail(ctx, OM_E_STATE, "om_readback_wait: nothing was posted");
    OM_REQUIRE(ctx, dst && bytes <= r->posted, "om_readback_wait: need a destination and at most %llu bytes",
               (unsigned long long)r->posted);
    om_status st = await(r);
    if (st) return st;
    memcpy(dst, r->host, bytes);
    return OM_OK;
}

}  // extern "C"
