// Runtime under the matmul path: device context, one HIP stream, a caching allocator, events,
// thread-local errors and the shape-keyed launch profiler.
//
// Replaces, for a discrete-HBM GPU, IronTensor's MetalContext singleton (src/device.rs:10-71), the
// CommandBatch sync/async modes (src/command_batch.rs:166-391) and per-op MTLBuffer allocation
// (src/tensor.rs:63-88, src/ops/kernel.rs:70-80).
#include <cstdio>
#include <cstring>
#include <string>

#include "internal.hpp"

namespace it {

static thread_local std::string g_last_error;

it_status fail(it_status st, const std::string &msg) {
    g_last_error = msg;
    return st;
}

it_status fail_hip(hipError_t err, const char *what) {
    std::string msg = std::string(what) + ": " + hipGetErrorName(err) + " (" +
                      hipGetErrorString(err) + ")";
    if (err == hipErrorOutOfMemory || err == hipErrorMemoryAllocation)
        return fail(IT_ERR_OOM, msg);
    if (err == hipErrorNoDevice || err == hipErrorInvalidDevice) return fail(IT_ERR_NO_DEVICE, msg);
    return fail(IT_ERR_HIP, msg);
}

void clear_error() { g_last_error.clear(); }

it_status sync_all(it_context *ctx) {
    IT_HIP_TRY(hipStreamSynchronize(ctx->main_stream));
    IT_HIP_TRY(hipStreamSynchronize(ctx->side_stream));
    return IT_OK;
}

it_status join_side(it_context *ctx) {
    if (!ctx->side_pending) return IT_OK;
    IT_HIP_TRY(hipEventRecord(ctx->join_ev, ctx->side_stream));
    IT_HIP_TRY(hipStreamWaitEvent(ctx->main_stream, ctx->join_ev, 0));
    ctx->side_pending = false;
    return IT_OK;
}

static it_status grow(it_context *ctx, void *&buf, size_t &have, size_t bytes, void **out) {
    if (have < bytes && ctx->capturing)
        return fail(IT_ERR_INVALID, "scratch of " + std::to_string(bytes) +
                                        " bytes needed during graph capture: run the work once before capturing");
    if (have < bytes) {
        if (buf) {
            if (!ctx->graphs.empty()) {
                // A live graph may have been captured with this block: keep it until the last
                // graph is destroyed.
                ctx->retired.emplace_back(buf, have);
            } else {
                if (const it_status st_ = sync_all(ctx); st_ != IT_OK) return st_;
                IT_HIP_TRY(hipFree(buf));
            }
            buf = nullptr;
            have = 0;
        }
        size_t want = bytes < (size_t(64) << 20) ? (size_t(64) << 20) : bytes;
        IT_HIP_TRY(hipMalloc(&buf, want));
        have = want;
    }
    *out = buf;
    return IT_OK;
}

it_status ensure_scratch(it_context *ctx, size_t bytes, void **out) {
    return grow(ctx, ctx->scratch[ctx->cur], ctx->scratch_bytes[ctx->cur], bytes, out);
}

it_status ensure_attn_scratch(it_context *ctx, size_t bytes, void **out) {
    return grow(ctx, ctx->attn_scratch[ctx->cur], ctx->attn_scratch_bytes[ctx->cur], bytes, out);
}

it_status ensure_counters(it_context *ctx, int **out) {
    int *&f = ctx->counters[ctx->cur];
    if (!f) {
        if (ctx->capturing)
            return fail(IT_ERR_INVALID, "arrival counters needed during graph capture: run the work once before capturing");
        IT_HIP_TRY(hipMalloc(&f, COUNTERS * sizeof(int)));
        // Synchronous zero fill at allocation (never inside a captured graph).
        hipError_t e = hipMemset(f, 0, COUNTERS * sizeof(int));
        if (e == hipSuccess) e = hipDeviceSynchronize();
        if (e != hipSuccess) {
            (void)hipFree(f);
            f = nullptr;
            return fail_hip(e, "zeroing the arrival counters");
        }
    }
    *out = f;
    return IT_OK;
}

static hipEvent_t pool_event(it_context *ctx) {
    if (!ctx->event_pool.empty()) {
        hipEvent_t e = ctx->event_pool.back();
        ctx->event_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

void profile_begin(it_context *ctx, const std::string &, hipEvent_t *start_out) {
    *start_out = nullptr;
    if (!ctx->profiling || ctx->capturing) return;
    hipEvent_t e = pool_event(ctx);
    if (e && hipEventRecord(e, ctx->stream) == hipSuccess) *start_out = e;
}

void profile_end(it_context *ctx, const std::string &key, hipEvent_t start) {
    if (!ctx->profiling || !start) return;
    hipEvent_t e = pool_event(ctx);
    if (!e || hipEventRecord(e, ctx->stream) != hipSuccess) {
        ctx->event_pool.push_back(start);
        return;
    }
    ctx->pending.push_back(ProfileRecord{key, start, e});
}

static it_status profile_drain(it_context *ctx) {
    if (ctx->pending.empty()) return IT_OK;
    if (const it_status st_ = sync_all(ctx); st_ != IT_OK) return st_;
    for (auto &r : ctx->pending) {
        float ms = 0.f;
        IT_HIP_TRY(hipEventElapsedTime(&ms, r.start, r.stop));
        auto &st = ctx->stats[r.key];
        st.calls += 1;
        st.total_ms += ms;
        ctx->event_pool.push_back(r.start);
        ctx->event_pool.push_back(r.stop);
    }
    ctx->pending.clear();
    return IT_OK;
}

}  // namespace it

using it::fail;

extern "C" {

const char *it_last_error(void) { return it::g_last_error.c_str(); }

const char *it_status_string(it_status s) {
    switch (s) {
    case IT_OK: return "ok";
    case IT_ERR_INNER_DIM: return "inner dimensions don't match";
    case IT_ERR_SHAPE: return "shape mismatch";
    case IT_ERR_PRECISION: return "precision mismatch";
    case IT_ERR_DIMS: return "unsupported dimensions";
    case IT_ERR_INVALID: return "invalid value";
    case IT_ERR_NULL: return "null pointer";
    case IT_ERR_OOM: return "out of device memory";
    case IT_ERR_NO_DEVICE: return "no HIP device";
    case IT_ERR_HIP: return "HIP runtime error";
    case IT_ERR_NOT_READY: return "not ready";
    }
    return "unknown status";
}

int it_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

it_status it_init(int device, it_context **out_ctx) {
    if (!out_ctx) return fail(IT_ERR_NULL, "it_init: out_ctx is NULL");
    *out_ctx = nullptr;
    int n = it_device_count();
    if (n <= 0) return fail(IT_ERR_NO_DEVICE, "it_init: no HIP device found");
    if (device < 0 || device >= n)
        return fail(IT_ERR_NO_DEVICE, "it_init: device ordinal " + std::to_string(device) +
                                          " out of range (" + std::to_string(n) + " devices)");
    IT_HIP_TRY(hipSetDevice(device));
    if (const it_status st = it::noalloc_init(device); st != IT_OK) return st;
    hipDeviceProp_t prop;
    IT_HIP_TRY(hipGetDeviceProperties(&prop, device));
    auto *ctx = new it_context();
    ctx->device = device;
    ctx->num_cus = prop.multiProcessorCount;
    ctx->clock_khz = prop.clockRate;
    std::snprintf(ctx->name, sizeof(ctx->name), "%s", prop.gcnArchName);
    // Default priority only: streams of mixed priority are avoided on purpose.
    hipError_t e = hipStreamCreateWithFlags(&ctx->main_stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&ctx->side_stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&ctx->fork_ev, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&ctx->join_ev, hipEventDisableTiming);
    if (e != hipSuccess) {
        if (ctx->main_stream) (void)hipStreamDestroy(ctx->main_stream);
        if (ctx->side_stream) (void)hipStreamDestroy(ctx->side_stream);
        if (ctx->fork_ev) (void)hipEventDestroy(ctx->fork_ev);
        delete ctx;
        return it::fail_hip(e, "stream/event creation");
    }
    ctx->stream = ctx->main_stream;
    *out_ctx = ctx;
    it::clear_error();
    return IT_OK;
}

it_status it_shutdown(it_context *ctx) {
    if (!ctx) return fail(IT_ERR_NULL, "it_shutdown: ctx is NULL");
    (void)hipSetDevice(ctx->device);
    (void)it::sync_all(ctx);
    for (auto &r : ctx->pending) {
        (void)hipEventDestroy(r.start);
        (void)hipEventDestroy(r.stop);
    }
    for (auto e : ctx->event_pool) (void)hipEventDestroy(e);
    for (auto &kv : ctx->cache) (void)hipFree(kv.second);
    for (auto &kv : ctx->live) (void)hipFree(kv.first);
    for (auto &kv : ctx->rope_tables) (void)hipFree(kv.second);
    for (it_graph *g : ctx->graphs) g->ctx = nullptr;  // graphs may still be destroyed afterwards
    for (auto &r : ctx->retired) (void)hipFree(r.first);
    for (int i = 0; i < 2; ++i) {
        if (ctx->scratch[i]) (void)hipFree(ctx->scratch[i]);
        if (ctx->attn_scratch[i]) (void)hipFree(ctx->attn_scratch[i]);
        if (ctx->counters[i]) (void)hipFree(ctx->counters[i]);
    }
    (void)hipEventDestroy(ctx->fork_ev);
    (void)hipEventDestroy(ctx->join_ev);
    (void)hipStreamDestroy(ctx->main_stream);
    (void)hipStreamDestroy(ctx->side_stream);
    delete ctx;
    return IT_OK;
}

it_status it_device_info(it_context *ctx, char *name, size_t name_len, int *num_cus,
                         int *clock_khz) {
    if (!ctx) return fail(IT_ERR_NULL, "it_device_info: ctx is NULL");
    if (name && name_len) std::snprintf(name, name_len, "%s", ctx->name);
    if (num_cus) *num_cus = ctx->num_cus;
    if (clock_khz) *clock_khz = ctx->clock_khz;
    return IT_OK;
}

it_status it_malloc(it_context *ctx, size_t bytes, void **out_ptr) {
    if (!ctx || !out_ptr) return fail(IT_ERR_NULL, "it_malloc: NULL argument");
    *out_ptr = nullptr;
    // Round to 256 B so cached blocks are reusable across nearby sizes and every block is aligned
    // for 128-bit loads.
    size_t sz = bytes == 0 ? 256 : ((bytes + 255) / 256) * 256;
    auto it = ctx->cache.find(sz);
    void *p = nullptr;
    if (it != ctx->cache.end()) {
        p = it->second;
        ctx->cache.erase(it);
    } else {
        if (ctx->capturing)
            return fail(IT_ERR_INVALID, "it_malloc: no cached block of " + std::to_string(sz) +
                                            " bytes during graph capture");
        hipError_t e = hipMalloc(&p, sz);
        if (e != hipSuccess) {
            // Release the cache once and retry before giving up.
            (void)it::sync_all(ctx);
            for (auto &kv : ctx->cache) (void)hipFree(kv.second);
            ctx->cache.clear();
            (void)hipGetLastError();
            e = hipMalloc(&p, sz);
            if (e != hipSuccess)
                return fail(IT_ERR_OOM, "it_malloc: failed to allocate " + std::to_string(sz) +
                                            " bytes: " + hipGetErrorString(e));
        }
    }
    ctx->live[p] = sz;
    ctx->bytes_live += sz;
    *out_ptr = p;
    return IT_OK;
}

it_status it_free(it_context *ctx, void *ptr) {
    if (!ctx) return fail(IT_ERR_NULL, "it_free: ctx is NULL");
    if (!ptr) return IT_OK;
    auto it = ctx->live.find(ptr);
    if (it == ctx->live.end()) return fail(IT_ERR_INVALID, "it_free: pointer not from it_malloc");
    // The block may be reused by the next main-stream allocation: order that after pending side work.
    if (const it_status st_ = it::join_side(ctx); st_ != IT_OK) return st_;
    ctx->bytes_live -= it->second;
    ctx->cache.emplace(it->second, ptr);
    ctx->live.erase(it);
    return IT_OK;
}

size_t it_mem_allocated(it_context *ctx) { return ctx ? ctx->bytes_live : 0; }

size_t it_mem_scratch(it_context *ctx) {
    if (!ctx) return 0;
    size_t total = 0;
    for (int i = 0; i < 2; ++i) total += ctx->scratch_bytes[i] + ctx->attn_scratch_bytes[i];
    for (auto &r : ctx->retired) total += r.second;
    return total;
}

it_status it_empty_cache(it_context *ctx) {
    if (!ctx) return fail(IT_ERR_NULL, "it_empty_cache: ctx is NULL");
    if (const it_status st_ = it::sync_all(ctx); st_ != IT_OK) return st_;
    for (auto &kv : ctx->cache) IT_HIP_TRY(hipFree(kv.second));
    ctx->cache.clear();
    return IT_OK;
}

it_status it_memcpy_h2d(it_context *ctx, void *dst, const void *src, size_t bytes) {
    if (!ctx || (!dst && bytes) || (!src && bytes)) return fail(IT_ERR_NULL, "it_memcpy_h2d: NULL");
    if (!bytes) return IT_OK;
    IT_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    // Pageable host memory: the copy has consumed `src` only once the stream reaches it.
    IT_HIP_TRY(hipStreamSynchronize(ctx->stream));
    return IT_OK;
}

it_status it_memcpy_d2h(it_context *ctx, void *dst, const void *src, size_t bytes) {
    if (!ctx || (!dst && bytes) || (!src && bytes)) return fail(IT_ERR_NULL, "it_memcpy_d2h: NULL");
    if (!bytes) return IT_OK;
    // Results may come from either stream: read after both.
    if (const it_status st_ = it::join_side(ctx); st_ != IT_OK) return st_;
    IT_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->main_stream));
    IT_HIP_TRY(hipStreamSynchronize(ctx->main_stream));
    return IT_OK;
}

it_status it_memcpy_d2d(it_context *ctx, void *dst, const void *src, size_t bytes) {
    if (!ctx || (!dst && bytes) || (!src && bytes)) return fail(IT_ERR_NULL, "it_memcpy_d2d: NULL");
    if (!bytes) return IT_OK;
    IT_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
    return IT_OK;
}

it_status it_zero(it_context *ctx, void *dst, size_t bytes) {
    if (!ctx || (!dst && bytes)) return fail(IT_ERR_NULL, "it_zero: NULL");
    if (!bytes) return IT_OK;
    return it::launch_zero(ctx->stream, dst, bytes);
}

it_status it_stream_sync(it_context *ctx) {
    if (!ctx) return fail(IT_ERR_NULL, "it_stream_sync: ctx is NULL");
    if (const it_status st_ = it::join_side(ctx); st_ != IT_OK) return st_;
    return it::sync_all(ctx);
}

it_status it_side_begin(it_context *ctx) {
    if (!ctx) return fail(IT_ERR_NULL, "it_side_begin: ctx is NULL");
    if (ctx->cur != 0) return fail(IT_ERR_INVALID, "it_side_begin: already on the side stream");
    IT_HIP_TRY(hipEventRecord(ctx->fork_ev, ctx->main_stream));
    IT_HIP_TRY(hipStreamWaitEvent(ctx->side_stream, ctx->fork_ev, 0));
    ctx->cur = 1;
    ctx->stream = ctx->side_stream;
    ctx->side_pending = true;
    return IT_OK;
}

it_status it_side_end(it_context *ctx) {
    if (!ctx) return fail(IT_ERR_NULL, "it_side_end: ctx is NULL");
    if (ctx->cur != 1) return fail(IT_ERR_INVALID, "it_side_end: not on the side stream");
    ctx->cur = 0;
    ctx->stream = ctx->main_stream;
    return IT_OK;
}

it_status it_side_join(it_context *ctx) {
    if (!ctx) return fail(IT_ERR_NULL, "it_side_join: ctx is NULL");
    if (ctx->cur != 0) return fail(IT_ERR_INVALID, "it_side_join: call it_side_end first");
    return it::join_side(ctx);
}

void *it_stream(it_context *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

it_status it_event_create(it_context *ctx, it_event **out_ev) {
    if (!ctx || !out_ev) return fail(IT_ERR_NULL, "it_event_create: NULL argument");
    auto *ev = new it_event();
    hipError_t e = hipEventCreate(&ev->ev);
    if (e != hipSuccess) {
        delete ev;
        return it::fail_hip(e, "hipEventCreate");
    }
    *out_ev = ev;
    return IT_OK;
}

it_status it_event_record(it_context *ctx, it_event *ev) {
    if (!ctx || !ev) return fail(IT_ERR_NULL, "it_event_record: NULL argument");
    IT_HIP_TRY(hipEventRecord(ev->ev, ctx->stream));
    return IT_OK;
}

it_status it_event_query(it_event *ev) {
    if (!ev) return fail(IT_ERR_NULL, "it_event_query: NULL event");
    hipError_t e = hipEventQuery(ev->ev);
    if (e == hipSuccess) return IT_OK;
    if (e == hipErrorNotReady) return IT_ERR_NOT_READY;
    return it::fail_hip(e, "hipEventQuery");
}

it_status it_event_sync(it_event *ev) {
    if (!ev) return fail(IT_ERR_NULL, "it_event_sync: NULL event");
    IT_HIP_TRY(hipEventSynchronize(ev->ev));
    return IT_OK;
}

it_status it_event_elapsed_ms(it_event *start, it_event *end, float *ms) {
    if (!start || !end || !ms) return fail(IT_ERR_NULL, "it_event_elapsed_ms: NULL argument");
    IT_HIP_TRY(hipEventElapsedTime(ms, start->ev, end->ev));
    return IT_OK;
}

it_status it_event_destroy(it_event *ev) {
    if (!ev) return IT_OK;
    (void)hipEventDestroy(ev->ev);
    delete ev;
    return IT_OK;
}

it_status it_capture_begin(it_context *ctx) {
    if (!ctx) return fail(IT_ERR_NULL, "it_capture_begin: ctx is NULL");
    if (ctx->capturing) return fail(IT_ERR_INVALID, "it_capture_begin: already capturing");
    if (ctx->cur != 0) return fail(IT_ERR_INVALID, "it_capture_begin: call it_side_end first");
    // Side work issued before the capture must not become a dependency of the graph.
    if (ctx->side_pending) IT_HIP_TRY(hipStreamSynchronize(ctx->side_stream));
    ctx->side_pending = false;
    IT_HIP_TRY(hipStreamBeginCapture(ctx->main_stream, hipStreamCaptureModeThreadLocal));
    ctx->capturing = true;
    return IT_OK;
}

it_status it_capture_end(it_context *ctx, it_graph **out_graph) {
    if (!ctx || !out_graph) return fail(IT_ERR_NULL, "it_capture_end: NULL argument");
    if (!ctx->capturing) return fail(IT_ERR_INVALID, "it_capture_end: not capturing");
    *out_graph = nullptr;
    if (ctx->cur != 0) {
        ctx->cur = 0;
        ctx->stream = ctx->main_stream;
    }
    // The side stream rejoins the main stream inside the capture (a forked stream must).
    const it_status js = it::join_side(ctx);
    ctx->capturing = false;
    auto *g = new it_graph();
    hipError_t e = hipStreamEndCapture(ctx->main_stream, &g->graph);
    if (js != IT_OK && e == hipSuccess) e = hipErrorInvalidValue;
    if (e == hipSuccess) e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        if (g->graph) (void)hipGraphDestroy(g->graph);
        delete g;
        return it::fail_hip(e, "hipStreamEndCapture/hipGraphInstantiate");
    }
    g->ctx = ctx;
    ctx->graphs.insert(g);
    *out_graph = g;
    return IT_OK;
}

it_status it_graph_launch(it_context *ctx, it_graph *graph) {
    if (!ctx || !graph) return fail(IT_ERR_NULL, "it_graph_launch: NULL argument");
    // The graph's buffers (scratch included) belong to the context that captured it.
    if (graph->ctx != ctx) return fail(IT_ERR_INVALID, "it_graph_launch: graph was captured on another context");
    IT_HIP_TRY(hipGraphLaunch(graph->exec, ctx->main_stream));
    return IT_OK;
}

it_status it_graph_destroy(it_graph *graph) {
    if (!graph) return IT_OK;
    it_context *ctx = graph->ctx;
    it_status st = IT_OK;
    if (ctx) {
        // A replay may still be running: the graph's resources go once the streams have drained.
        (void)hipSetDevice(ctx->device);
        st = it::sync_all(ctx);
        ctx->graphs.erase(graph);
    }
    if (graph->exec) (void)hipGraphExecDestroy(graph->exec);
    if (graph->graph) (void)hipGraphDestroy(graph->graph);
    delete graph;
    if (ctx && ctx->graphs.empty() && st == IT_OK) {
        for (auto &r : ctx->retired) (void)hipFree(r.first);
        ctx->retired.clear();
    }
    return st;
}

it_status it_profiler_enable(it_context *ctx, int enable) {
    if (!ctx) return fail(IT_ERR_NULL, "it_profiler_enable: ctx is NULL");
    ctx->profiling = enable != 0;
    return IT_OK;
}

it_status it_profiler_reset(it_context *ctx) {
    if (!ctx) return fail(IT_ERR_NULL, "it_profiler_reset: ctx is NULL");
    it_status st = it::profile_drain(ctx);
    ctx->stats.clear();
    return st;
}

it_status it_profiler_report(it_context *ctx, char *buf, size_t buf_len, size_t *needed) {
    if (!ctx) return fail(IT_ERR_NULL, "it_profiler_report: ctx is NULL");
    it_status st = it::profile_drain(ctx);
    if (st != IT_OK) return st;
    std::string out = "{";
    bool first = true;
    for (auto &kv : ctx->stats) {
        char tmp[128];
        std::snprintf(tmp, sizeof(tmp), "{\"calls\": %lld, \"total_ms\": %.6f}",
                      (long long)kv.second.calls, kv.second.total_ms);
        if (!first) out += ", ";
        first = false;
        out += "\"" + kv.first + "\": " + tmp;
    }
    out += "}";
    if (needed) *needed = out.size() + 1;
    if (!buf || buf_len < out.size() + 1)
        return fail(IT_ERR_INVALID, "it_profiler_report: buffer too small");
    std::memcpy(buf, out.c_str(), out.size() + 1);
    return IT_OK;
}

}  // extern "C"

namespace {

// The GEMMs of one profiler key "gemm_<dtype>_<AB>_<plan>|<tag>[M,N,K](+[M,N,K])*x<batch> s<splits>"
// (or gemv_...): layout letters and shapes; false for other kernels (attention, training ops).
struct KeyGemm {
    bool ta, tb;
    long long m, n, k;
};

bool parse_gemm_key(const std::string &key, std::vector<KeyGemm> &out) {
    out.clear();
    if (key.rfind("gemm_", 0) != 0 && key.rfind("gemv_", 0) != 0) return false;
    const size_t u1 = key.find('_'), u2 = key.find('_', u1 + 1);
    if (u2 == std::string::npos || u2 + 2 >= key.size()) return false;
    const char a = key[u2 + 1], b = key[u2 + 2];
    const size_t bar = key.find('|');
    if (bar == std::string::npos) return false;
    size_t pos = key.find('[', bar);
    while (pos != std::string::npos) {
        KeyGemm g{a == 'T', b == 'T', 0, 0, 0};
        if (std::sscanf(key.c_str() + pos, "[%lld,%lld,%lld]", &g.m, &g.n, &g.k) != 3) return false;
        out.push_back(g);
        const size_t close = key.find(']', pos);
        if (close == std::string::npos || close + 1 >= key.size() || key[close + 1] != '+') break;
        pos = close + 2;
    }
    return !out.empty();
}

}  // namespace

extern "C" {

it_status it_profiler_report_shapes(it_context *ctx, char *buf, size_t buf_len, size_t *needed) {
    if (!ctx) return fail(IT_ERR_NULL, "it_profiler_report_shapes: ctx is NULL");
    it_status st = it::profile_drain(ctx);
    if (st != IT_OK) return st;
    std::map<std::string, it::ProfileStat> shapes;
    std::vector<KeyGemm> gs;
    for (auto &kv : ctx->stats) {
        if (!parse_gemm_key(kv.first, gs)) continue;
        double flops = 0.0;
        for (const KeyGemm &g : gs) flops += (double)g.m * g.n * g.k;
        for (const KeyGemm &g : gs) {
            // The stored operands as the reference names them: A [M,K] or, transposed, [K,M]^T;
            // B [K,N] or [N,K]^T (src/ops/mps_gemm.rs:22-30,421-422).
            const long long a0 = g.ta ? g.k : g.m, a1 = g.ta ? g.m : g.k;
            const long long b0 = g.tb ? g.n : g.k, b1 = g.tb ? g.k : g.n;
            const std::string shape = "[" + std::to_string(a0) + "," + std::to_string(a1) + "]" + (g.ta ? "^T" : "") +
                                      "x[" + std::to_string(b0) + "," + std::to_string(b1) + "]" + (g.tb ? "^T" : "");
            auto &d = shapes[shape];
            d.calls += kv.second.calls;
            d.total_ms += flops > 0.0 ? kv.second.total_ms * ((double)g.m * g.n * g.k / flops)
                                      : kv.second.total_ms / (double)gs.size();
        }
    }
    std::string out = "{";
    bool first = true;
    for (auto &kv : shapes) {
        char tmp[128];
        std::snprintf(tmp, sizeof(tmp), "{\"count\": %lld, \"total_ms\": %.6f}", (long long)kv.second.calls,
                      kv.second.total_ms);
        if (!first) out += ", ";
        first = false;
        out += "\"" + kv.first + "\": " + tmp;
    }
    out += "}";
    if (needed) *needed = out.size() + 1;
    if (!buf || buf_len < out.size() + 1)
        return fail(IT_ERR_INVALID, "it_profiler_report_shapes: buffer too small");
    std::memcpy(buf, out.c_str(), out.size() + 1);
    return IT_OK;
}

}  // extern "C"
