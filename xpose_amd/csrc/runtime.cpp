// C-ABI plumbing: errors, device set-up, memory, streams and events. This is
// the part of the reference's runtime core (Context / Buffer / Fence,
// include/vulkore/{context,buffer,sync}.hpp) the decode path needs, reduced
// to thin HIP calls.
#include "xp_internal.hpp"
#include "xp_launch.hpp"

#include <cstdio>
#include <cstring>
#include <functional>
#include <mutex>
#include <vector>

namespace xp {

namespace {
thread_local char g_err[1024] = "";
std::mutex g_scratch_mu;
std::vector<DeviceScratch*> g_scratch;  // indexed by device, never freed
}  // namespace

int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

void clear_error() { g_err[0] = '\0'; }

DeviceScratch* scratch() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        set_error(XP_E_HIP, "scratch: hipGetDevice failed");
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (dev >= int(g_scratch.size())) g_scratch.resize(dev + 1, nullptr);
    if (!g_scratch[dev]) {
        auto* s = new DeviceScratch;
        s->device = dev;
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, dev) == hipSuccess) s->n_cu = p.multiProcessorCount;
        g_scratch[dev] = s;
    }
    return g_scratch[dev];
}

bool ensure_partial(DeviceScratch* s, size_t floats) {
    if (s->partial_floats >= floats) return true;
    // The old buffer may still be read by queued work; drain before freeing.
    if (s->partial) {
        if (hipDeviceSynchronize() != hipSuccess || hipFree(s->partial) != hipSuccess) {
            set_error(XP_E_HIP, "scratch: could not release partial buffer");
            return false;
        }
        s->partial = nullptr;
        s->partial_floats = 0;
    }
    size_t n = floats < (1u << 20) ? (1u << 20) : floats;
    if (hipMalloc(&s->partial, n * sizeof(float)) != hipSuccess) {
        s->partial = nullptr;
        set_error(XP_E_NOMEM, "scratch: hipMalloc(%zu floats) failed", n);
        return false;
    }
    s->partial_floats = n;
    return true;
}

bool ensure_tickets(DeviceScratch* s, size_t n) {
    if (s->n_tickets >= n) return true;
    if (s->tickets) {
        if (hipDeviceSynchronize() != hipSuccess || hipFree(s->tickets) != hipSuccess) {
            set_error(XP_E_HIP, "scratch: could not release ticket buffer");
            return false;
        }
        s->tickets = nullptr;
        s->n_tickets = 0;
    }
    size_t m = n < 65536 ? 65536 : n;
    if (hipMalloc(&s->tickets, m * sizeof(uint32_t)) != hipSuccess) {
        s->tickets = nullptr;
        set_error(XP_E_NOMEM, "scratch: hipMalloc(%zu tickets) failed", m);
        return false;
    }
    // Tickets must start at zero; every kernel that takes one returns it to
    // zero before it exits.
    if (hipMemset(s->tickets, 0, m * sizeof(uint32_t)) != hipSuccess ||
        hipDeviceSynchronize() != hipSuccess) {
        set_error(XP_E_HIP, "scratch: zeroing tickets failed");
        return false;
    }
    s->n_tickets = m;
    return true;
}

bool ensure_attn_x(DeviceScratch* s, size_t floats, size_t words) {
    if (s->attn_x_floats >= floats && s->attn_state_words >= words) return true;
    if (s->attn_x || s->attn_state) {
        if (hipDeviceSynchronize() != hipSuccess || hipFree(s->attn_x) != hipSuccess ||
            hipFree(s->attn_state) != hipSuccess) {
            set_error(XP_E_HIP, "scratch: could not release attention exchange buffers");
            return false;
        }
        s->attn_x = nullptr;
        s->attn_state = nullptr;
        s->attn_x_floats = s->attn_state_words = 0;
    }
    if (hipMalloc(&s->attn_x, floats * sizeof(float)) != hipSuccess ||
        hipMalloc(&s->attn_state, words * sizeof(uint32_t)) != hipSuccess ||
        hipMemset(s->attn_x, 0, floats * sizeof(float)) != hipSuccess ||
        hipMemset(s->attn_state, 0, words * sizeof(uint32_t)) != hipSuccess ||
        hipDeviceSynchronize() != hipSuccess) {
        set_error(XP_E_NOMEM, "scratch: attention exchange buffers (%zu floats) failed", floats);
        return false;
    }
    s->attn_x_floats = floats;
    s->attn_state_words = words;
    return true;
}

int graph_batch_timed(const std::function<int(hipStream_t)>& record, uint32_t reps, hipStream_t replay,
                      float* best_ms) {
    hipStream_t cap = nullptr;
    XP_HIP(hipStreamCreateWithFlags(&cap, hipStreamNonBlocking));
    hipGraph_t g = nullptr;
    hipGraphExec_t ge = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = XP_OK;
    if (hipStreamBeginCapture(cap, hipStreamCaptureModeThreadLocal) != hipSuccess) {
        rc = set_error(XP_E_HIP, "graph_batch_timed: hipStreamBeginCapture failed");
    } else {
        rc = record(cap);
        const hipError_t ee = hipStreamEndCapture(cap, &g);
        if (rc == XP_OK && ee != hipSuccess)
            rc = set_error(XP_E_HIP, "graph_batch_timed: hipStreamEndCapture -> %s", hipGetErrorString(ee));
    }
    if (rc == XP_OK && hipGraphInstantiate(&ge, g, nullptr, nullptr, 0) != hipSuccess)
        rc = set_error(XP_E_HIP, "graph_batch_timed: hipGraphInstantiate failed");
    if (rc == XP_OK && (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess))
        rc = set_error(XP_E_HIP, "graph_batch_timed: hipEventCreate failed");
    // one untimed replay, then `reps` replays each between two events
    if (rc == XP_OK && hipGraphLaunch(ge, replay) != hipSuccess)
        rc = set_error(XP_E_HIP, "graph_batch_timed: hipGraphLaunch failed");
    if (rc == XP_OK && hipStreamSynchronize(replay) != hipSuccess)
        rc = set_error(XP_E_HIP, "graph_batch_timed: sync failed");
    float best = 1e30f;
    for (uint32_t r = 0; r < reps && rc == XP_OK; ++r) {
        float ms = 0.0f;
        if (hipEventRecord(e0, replay) != hipSuccess || hipGraphLaunch(ge, replay) != hipSuccess ||
            hipEventRecord(e1, replay) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
            hipEventElapsedTime(&ms, e0, e1) != hipSuccess)
            rc = set_error(XP_E_HIP, "graph_batch_timed: replay %u failed", r);
        else if (ms < best)
            best = ms;
    }
    if (rc == XP_OK) *best_ms = best;
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (ge) (void)hipGraphExecDestroy(ge);
    if (g) (void)hipGraphDestroy(g);
    (void)hipStreamDestroy(cap);
    return rc;
}

}  // namespace xp

using namespace xp;

extern "C" {

const char* xp_last_error(void) { return g_err; }
const char* xp_version(void) { return "xpose-amd 0.1 (gfx950)"; }

int xp_init(int dev) {
    clear_error();
    int n = 0;
    XP_HIP(hipGetDeviceCount(&n));
    XP_REQUIRE(dev >= 0 && dev < n, "device %d out of range (%d devices)", dev, n);
    XP_HIP(hipSetDevice(dev));
    DeviceScratch* s = scratch();
    if (!s) return XP_E_HIP;
    if (!ensure_tickets(s, 65536)) return XP_E_NOMEM;
    if (!ensure_partial(s, 1u << 20)) return XP_E_NOMEM;
    MvNoAlloc na{};
    return mv_noalloc_setup(nullptr, true, &na);
}

int xp_device_info(char* name, size_t cap, int* n_cu, size_t* hbm_bytes, char* arch,
                   size_t arch_cap) {
    int dev = 0;
    XP_HIP(hipGetDevice(&dev));
    hipDeviceProp_t p;
    XP_HIP(hipGetDeviceProperties(&p, dev));
    if (name && cap) {
        std::strncpy(name, p.name, cap - 1);
        name[cap - 1] = '\0';
    }
    if (arch && arch_cap) {
        std::strncpy(arch, p.gcnArchName, arch_cap - 1);
        arch[arch_cap - 1] = '\0';
    }
    if (n_cu) *n_cu = p.multiProcessorCount;
    if (hbm_bytes) *hbm_bytes = p.totalGlobalMem;
    return XP_OK;
}

int xp_malloc(void** dptr, size_t bytes) {
    XP_REQUIRE(dptr != nullptr, "dptr is null");
    *dptr = nullptr;
    if (bytes == 0) return XP_OK;
    hipError_t e = hipMalloc(dptr, bytes);
    if (e != hipSuccess) {
        *dptr = nullptr;
        return set_error(XP_E_NOMEM, "xp_malloc: hipMalloc(%zu) -> %s", bytes,
                         hipGetErrorString(e));
    }
    return XP_OK;
}

int xp_free(void* dptr) {
    if (dptr) XP_HIP(hipFree(dptr));
    return XP_OK;
}

int xp_memcpy_htod(void* dst, const void* src, size_t bytes) {
    if (!bytes) return XP_OK;
    XP_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return XP_OK;
}

int xp_memcpy_dtoh(void* dst, const void* src, size_t bytes) {
    if (!bytes) return XP_OK;
    XP_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return XP_OK;
}

int xp_memcpy_dtod(void* dst, const void* src, size_t bytes) {
    if (!bytes) return XP_OK;
    XP_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice));
    return XP_OK;
}

int xp_memset(void* dst, int value, size_t bytes) {
    if (!bytes) return XP_OK;
    XP_HIP(hipMemset(dst, value, bytes));
    return XP_OK;
}

int xp_synchronize(void) {
    XP_HIP(hipDeviceSynchronize());
    return XP_OK;
}

int xp_stream_create(xp_stream* s) {
    XP_REQUIRE(s != nullptr, "s is null");
    hipStream_t h = nullptr;
    // Default priority only: streams of mixed priorities are not used here.
    XP_HIP(hipStreamCreateWithFlags(&h, hipStreamNonBlocking));
    *s = reinterpret_cast<xp_stream>(h);
    return XP_OK;
}

int xp_stream_destroy(xp_stream s) {
    if (s) XP_HIP(hipStreamDestroy(as_stream(s)));
    return XP_OK;
}

int xp_stream_synchronize(xp_stream s) {
    XP_HIP(hipStreamSynchronize(as_stream(s)));
    return XP_OK;
}

int xp_event_create(xp_event* e) {
    XP_REQUIRE(e != nullptr, "e is null");
    hipEvent_t h = nullptr;
    XP_HIP(hipEventCreate(&h));
    *e = reinterpret_cast<xp_event>(h);
    return XP_OK;
}

int xp_event_destroy(xp_event e) {
    if (e) XP_HIP(hipEventDestroy(reinterpret_cast<hipEvent_t>(e)));
    return XP_OK;
}

int xp_event_record(xp_event e, xp_stream s) {
    XP_HIP(hipEventRecord(reinterpret_cast<hipEvent_t>(e), as_stream(s)));
    return XP_OK;
}

int xp_event_elapsed_ms(xp_event a, xp_event b, float* ms) {
    XP_REQUIRE(ms != nullptr, "ms is null");
    XP_HIP(hipEventSynchronize(reinterpret_cast<hipEvent_t>(b)));
    XP_HIP(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(a),
                               reinterpret_cast<hipEvent_t>(b)));
    return XP_OK;
}

}  // extern "C"
