// tnhip runtime: errors, probe, counters, device memory, streams, events and
// the per-(device, stream) workspace.
//
// The error/refusal convention follows torchnative's err.rs:11-28 (refusals
// are NotImplementedError naming the reason; runtime failures RuntimeError),
// the probe/counter shape follows device.rs:1671-1708 and vulkan.rs:2138-2268.
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <utility>
#include <vector>
#include <algorithm>

#include "tn_common.h"

namespace tn {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

tn_status fail(tn_status code, const std::string& msg) {
    g_last_error = msg;
    if (code == TN_ENOTIMPL) counters().refusals.fetch_add(1);
    return code;
}

tn_status hip_fail(hipError_t e, const char* what) {
    char buf[512];
    std::snprintf(buf, sizeof buf, "tnhip: HIP error %d (%s) in %s", (int)e, hipGetErrorString(e), what);
    return fail(TN_EHIP, buf);
}

Counters& counters() {
    static Counters c;
    return c;
}

namespace {
// A stream's scratch. A graph captured from a stream keeps the addresses it
// saw, so once a stream has been captured a buffer outgrown by a later,
// larger call is retired (kept) rather than freed, and all of them go with
// tn_stream_destroy; growth at least doubles, so the retired ones total less
// than the live one. A stream never captured (the default stream cannot be)
// frees the outgrown buffer at once, after a synchronisation.
struct Workspace {
    void* ptr = nullptr;
    size_t bytes = 0;
    uint32_t* tickets = nullptr;  // zeroed counters, returned to zero by their users
    size_t ntickets = 0;
    std::vector<void*> retired;
    size_t retired_bytes = 0;
    bool captured = false;  // a capture has begun on this stream
    std::string refused;    // a call refused while the stream was capturing
};
std::mutex g_ws_mu;
std::map<std::pair<int, hipStream_t>, Workspace> g_ws;

// Growth allocates, which a stream under graph capture must not do (and a
// graph could not replay): refused by name. The refusal is also recorded, so
// that ending the capture fails instead of returning a graph that lacks the
// refused launch.
tn_status refuse_if_capturing(Workspace& w, hipStream_t stream, const char* what) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    TN_HIP(hipStreamIsCapturing(stream, &cs));
    if (cs != hipStreamCaptureStatusNone) {
        const std::string msg = std::string("tnhip: this call needs more ") + what +
                                " than the stream holds, and a stream under graph capture cannot allocate; make "
                                "the same call (or a larger one) once before capturing";
        if (w.refused.empty()) w.refused = msg;
        return fail(TN_EINVAL, msg);
    }
    return TN_OK;
}

// An outgrown buffer: kept for the stream's graphs, or freed at once when the
// stream has never been captured.
tn_status retire(Workspace& w, hipStream_t stream, void* old, size_t bytes) {
    if (!old) return TN_OK;
    if (w.captured) {
        w.retired.push_back(old);
        w.retired_bytes += bytes;
        return TN_OK;
    }
    TN_HIP(hipStreamSynchronize(stream));  // kernels already queued may still read it
    TN_HIP(hipFree(old));
    counters().workspace_bytes.fetch_sub(bytes);
    return TN_OK;
}
}  // namespace

tn_status workspace(hipStream_t stream, size_t bytes, void** out) {
    int dev = 0;
    TN_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(g_ws_mu);
    Workspace& w = g_ws[{dev, stream}];
    if (w.bytes < bytes) {
        TN_TRY(refuse_if_capturing(w, stream, "workspace"));
        size_t want = std::max(bytes, std::max((size_t)1 << 20, 2 * w.bytes));
        want = (want + 4095) & ~(size_t)4095;
        void* p = nullptr;
        TN_HIP(hipMalloc(&p, want));
        TN_TRY(retire(w, stream, w.ptr, w.bytes));
        w.ptr = p;
        w.bytes = want;
        counters().workspace_bytes.fetch_add(want);
    }
    *out = w.ptr;
    return TN_OK;
}

tn_status tickets(hipStream_t stream, size_t n, uint32_t** out) {
    int dev = 0;
    TN_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(g_ws_mu);
    Workspace& w = g_ws[{dev, stream}];
    if (w.ntickets < n) {
        TN_TRY(refuse_if_capturing(w, stream, "ticket counters"));
        size_t want = std::max(n, std::max((size_t)4096, 2 * w.ntickets));
        want = (want + 4095) & ~(size_t)4095;
        uint32_t* p = nullptr;
        TN_HIP(hipMalloc(reinterpret_cast<void**>(&p), want * 4));
        // zeroed once, ahead of the first kernel on this stream that takes a ticket
        TN_HIP(hipMemsetAsync(p, 0, want * 4, stream));
        TN_TRY(retire(w, stream, w.tickets, w.ntickets * 4));
        w.tickets = p;
        w.ntickets = want;
        counters().workspace_bytes.fetch_add(want * 4);
    }
    *out = w.tickets;
    return TN_OK;
}

namespace {
struct OccKey {
    int dev;
    const void* kernel;
    int block;
    size_t lds;
    bool operator<(const OccKey& o) const {
        if (dev != o.dev) return dev < o.dev;
        if (kernel != o.kernel) return kernel < o.kernel;
        if (block != o.block) return block < o.block;
        return lds < o.lds;
    }
};
std::mutex g_occ_mu;
std::map<OccKey, int> g_occ;
}  // namespace

tn_status resident_workgroups(const void* kernel, int block, size_t lds, int* out) {
    int dev = 0;
    TN_HIP(hipGetDevice(&dev));
    const OccKey key{dev, kernel, block, lds};
    {
        std::lock_guard<std::mutex> lock(g_occ_mu);
        auto it = g_occ.find(key);
        if (it != g_occ.end()) {
            *out = it->second;
            return TN_OK;
        }
    }
    int per_cu = 0, cus = 0;
    TN_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block, lds));
    TN_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    const int n = (per_cu > 0 ? per_cu : 1) * (cus > 0 ? cus : 1);
    std::lock_guard<std::mutex> lock(g_occ_mu);
    g_occ[key] = n;
    *out = n;
    return TN_OK;
}

}  // namespace tn

using namespace tn;

extern "C" {

const char* tn_last_error(void) { return g_last_error.c_str(); }

int tn_abi_version(void) { return TN_ABI_VERSION; }

const char* tn_ops(void) {
    return "torch._C._quantize(q4_0),torch._C._dequantize(q4_0),torch._C._quantized_linear(q4_0),"
           "torch._C._quantize(q8_0),torch._C._dequantize(q8_0),torch._C._quantized_linear(q8_0),"
           "torch._C._quantize(q4_k),torch._C._dequantize(q4_k),torch._C._quantized_linear(q4_k),"
           "torch._C._quantize(f32|f16|bf16),torch._C._dequantize(f32|f16|bf16),"
           "torch._C._quantized_linear(f32|f16|bf16),aten.linear.default,"
           "torch._C._quantized_to,torch._C._quantized_blob,"
           "aten._scaled_dot_product_flash_attention_for_cpu.default,sdpa_decode,"
           "aten.embedding.default,rms_norm,rotary_embedding,silu_mul,aten.add.Tensor,aten.argmax.default,"
           "kv_append,q4_0_linear_decode,llama_decode_step,llama_prefill";
}

tn_status tn_probe(char* buf, size_t len) {
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0)
        return fail(TN_ENOTIMPL, e != hipSuccess
                                     ? std::string("tnhip: no_driver: hipGetDeviceCount failed: ") + hipGetErrorString(e)
                                     : std::string("tnhip: no_device: the HIP runtime sees no GPU"));
    int dev = 0;
    TN_HIP(hipGetDevice(&dev));
    hipDeviceProp_t p;
    TN_HIP(hipGetDeviceProperties(&p, dev));
    if (std::strncmp(p.gcnArchName, "gfx950", 6) != 0)
        return fail(TN_ENOTIMPL, std::string("tnhip: wrong_arch: this library is built for gfx950 (MI355X), "
                                             "the current device is ") + p.gcnArchName);
    if (buf && len) {
        std::snprintf(buf, len, "name=%s;arch=%s;cus=%d;hbm_bytes=%zu;clock_khz=%d;devices=%d;device=%d",
                      p.name, p.gcnArchName, p.multiProcessorCount, (size_t)p.totalGlobalMem, p.clockRate, n,
                      dev);
    }
    return TN_OK;
}

tn_status tn_counters(tn_counters_t* out) {
    if (!out) return fail(TN_EVALUE, "tn_counters: null output");
    Counters& c = counters();
    out->dispatches = c.dispatches.load();
    out->bytes_uploaded = c.bytes_uploaded.load();
    out->host_downloads = c.host_downloads.load();
    out->bytes_downloaded = c.bytes_downloaded.load();
    out->refusals = c.refusals.load();
    out->workspace_bytes = c.workspace_bytes.load();
    return TN_OK;
}

tn_status tn_counters_reset(void) {
    Counters& c = counters();
    c.dispatches = 0;
    c.bytes_uploaded = 0;
    c.host_downloads = 0;
    c.bytes_downloaded = 0;
    c.refusals = 0;
    return TN_OK;
}

tn_status tn_device_count(int* n) {
    hipError_t e = hipGetDeviceCount(n);
    if (e == hipErrorNoDevice) {
        *n = 0;
        return TN_OK;
    }
    TN_HIP(e);
    return TN_OK;
}

tn_status tn_set_device(int ordinal) {
    TN_HIP(hipSetDevice(ordinal));
    return TN_OK;
}

tn_status tn_get_device(int* ordinal) {
    TN_HIP(hipGetDevice(ordinal));
    return TN_OK;
}

tn_status tn_malloc(void** ptr, size_t bytes) {
    if (!ptr) return fail(TN_EVALUE, "tn_malloc: null output");
    *ptr = nullptr;
    if (bytes == 0) return TN_OK;
    TN_HIP(hipMalloc(ptr, bytes));
    return TN_OK;
}

tn_status tn_free(void* ptr) {
    if (ptr) TN_HIP(hipFree(ptr));
    return TN_OK;
}

tn_status tn_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream) {
    if (!bytes) return TN_OK;
    TN_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream));
    TN_HIP(hipStreamSynchronize((hipStream_t)stream));  // the host buffer may be freed on return
    counters().bytes_uploaded.fetch_add(bytes);
    return TN_OK;
}

tn_status tn_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream) {
    counters().host_downloads.fetch_add(1);
    if (!bytes) return TN_OK;
    TN_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream));
    TN_HIP(hipStreamSynchronize((hipStream_t)stream));
    counters().bytes_downloaded.fetch_add(bytes);
    return TN_OK;
}

tn_status tn_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream) {
    if (!bytes) return TN_OK;
    TN_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream));
    return TN_OK;
}

tn_status tn_memset(void* dst, int value, size_t bytes, void* stream) {
    if (!bytes) return TN_OK;
    TN_HIP(hipMemsetAsync(dst, value, bytes, (hipStream_t)stream));
    return TN_OK;
}

tn_status tn_stream_create(void** stream) {
    hipStream_t s;
    TN_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *stream = s;
    return TN_OK;
}

tn_status tn_stream_destroy(void* stream) {
    if (stream) {
        {
            int dev = 0;
            TN_HIP(hipGetDevice(&dev));
            std::lock_guard<std::mutex> lock(g_ws_mu);
            auto it = g_ws.find({dev, (hipStream_t)stream});
            if (it != g_ws.end()) {
                TN_HIP(hipStreamSynchronize((hipStream_t)stream));
                if (it->second.ptr) {
                    TN_HIP(hipFree(it->second.ptr));
                    counters().workspace_bytes.fetch_sub(it->second.bytes);
                }
                if (it->second.tickets) {
                    TN_HIP(hipFree(it->second.tickets));
                    counters().workspace_bytes.fetch_sub(it->second.ntickets * 4);
                }
                for (void* r : it->second.retired) TN_HIP(hipFree(r));
                counters().workspace_bytes.fetch_sub(it->second.retired_bytes);
                g_ws.erase(it);
            }
        }
        TN_HIP(hipStreamDestroy((hipStream_t)stream));
    }
    return TN_OK;
}

tn_status tn_stream_begin_capture(void* stream) {
    if (!stream) return fail(TN_EVALUE, "tn_stream_begin_capture: the default stream cannot be captured");
    {
        int dev = 0;
        TN_HIP(hipGetDevice(&dev));
        std::lock_guard<std::mutex> lock(g_ws_mu);
        Workspace& w = g_ws[{dev, (hipStream_t)stream}];
        w.captured = true;  // from now on outgrown buffers are kept for the graph
        w.refused.clear();
    }
    TN_HIP(hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal));
    return TN_OK;
}

tn_status tn_stream_end_capture(void* stream, void** graph) {
    if (!graph) return fail(TN_EVALUE, "tn_stream_end_capture: null output");
    *graph = nullptr;
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture((hipStream_t)stream, &g);
    std::string refused;
    {
        int dev = 0;
        TN_HIP(hipGetDevice(&dev));
        std::lock_guard<std::mutex> lock(g_ws_mu);
        auto it = g_ws.find({dev, (hipStream_t)stream});
        if (it != g_ws.end()) refused.swap(it->second.refused);
    }
    if (e != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        return hip_fail(e, "hipStreamEndCapture");
    }
    // a call refused during the capture is missing from the graph: no graph
    if (!refused.empty()) {
        if (g) (void)hipGraphDestroy(g);
        return fail(TN_EINVAL, "tn_stream_end_capture: a call was refused during the capture, so the graph would "
                               "lack its launch; no graph was made. The refusal: " + refused);
    }
    hipGraphExec_t exec = nullptr;
    const hipError_t ei = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (ei != hipSuccess) return hip_fail(ei, "hipGraphInstantiate");
    *graph = exec;
    return TN_OK;
}

tn_status tn_stream_synchronize(void* stream) {
    TN_HIP(hipStreamSynchronize((hipStream_t)stream));
    return TN_OK;
}

tn_status tn_device_synchronize(void) {
    TN_HIP(hipDeviceSynchronize());
    return TN_OK;
}

tn_status tn_event_create(void** event) {
    hipEvent_t e;
    TN_HIP(hipEventCreate(&e));
    *event = e;
    return TN_OK;
}

tn_status tn_event_destroy(void* event) {
    if (event) TN_HIP(hipEventDestroy((hipEvent_t)event));
    return TN_OK;
}

tn_status tn_event_record(void* event, void* stream) {
    TN_HIP(hipEventRecord((hipEvent_t)event, (hipStream_t)stream));
    return TN_OK;
}

tn_status tn_event_synchronize(void* event) {
    TN_HIP(hipEventSynchronize((hipEvent_t)event));
    return TN_OK;
}

tn_status tn_event_elapsed_ms(float* ms, void* start, void* end) {
    TN_HIP(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)end));
    return TN_OK;
}

}  // extern "C"
