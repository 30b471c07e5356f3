// Host-side internals shared by every translation unit of libxpose: error
// state, HIP call checking, argument checks and the per-device scratch the
// kernels use (split-k tickets and partial sums). Nothing here crosses the
// C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <functional>
#include <string>

#include "../../include/xpose.h"

namespace xp {

// Formats the message into the thread's error slot and returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// Per-device scratch. Allocated once by xp_init (or lazily by the first
// entry point that needs it) and kept until process exit.
struct DeviceScratch {
    int       device       = -1;
    int       n_cu         = 0;
    uint32_t* tickets      = nullptr;  // split-k arrival counters, all zero at rest
    size_t    n_tickets    = 0;
    float*    partial      = nullptr;  // split-k / split-span partial sums
    size_t    partial_floats = 0;
    // Decode attention's exchange mode (its own, zeroed: its records carry
    // launch tags that no other data may imitate, and its epoch words persist)
    float*    attn_x       = nullptr;
    size_t    attn_x_floats = 0;
    uint32_t* attn_state   = nullptr;
    size_t    attn_state_words = 0;
};

// Returns the scratch of the current device, creating it on first use.
// nullptr (with the error set) if allocation fails.
DeviceScratch* scratch();
// Grows the partial buffer to at least `floats`; returns false on failure.
bool ensure_partial(DeviceScratch* s, size_t floats);
bool ensure_tickets(DeviceScratch* s, size_t n);
// The attention exchange buffers, zeroed when (re)allocated.
bool ensure_attn_x(DeviceScratch* s, size_t floats, size_t words);

inline hipStream_t as_stream(xp_stream s) { return reinterpret_cast<hipStream_t>(s); }

// Measurement in the form of a decode step's submission: `record` enqueues a
// batch of launches on the stream it is given, which is captured into one
// HIP graph; the graph is replayed once untimed and then `reps` times on
// `replay`, each replay between two events. *best_ms = the fastest replay.
// `record` must not allocate, synchronise or enqueue memsets.
int graph_batch_timed(const std::function<int(hipStream_t)>& record, uint32_t reps, hipStream_t replay,
                      float* best_ms);

}  // namespace xp

// Evaluates a HIP call; on failure records "<where>: <call> -> <hip error>"
// and returns XP_E_HIP from the enclosing function.
#define XP_HIP(call)                                                           \
    do {                                                                       \
        hipError_t _e = (call);                                                \
        if (_e != hipSuccess)                                                  \
            return ::xp::set_error(XP_E_HIP, "%s: %s -> %s", __func__, #call,  \
                                   hipGetErrorString(_e));                     \
    } while (0)

// Argument check: returns XP_E_ARG naming the entry point and the condition.
#define XP_REQUIRE(cond, ...)                                                  \
    do {                                                                       \
        if (!(cond)) {                                                         \
            std::string _m = std::string(__func__) + ": ";                     \
            char _b[256];                                                      \
            std::snprintf(_b, sizeof _b, __VA_ARGS__);                         \
            return ::xp::set_error(XP_E_ARG, "%s%s", _m.c_str(), _b);          \
        }                                                                      \
    } while (0)

// Checks the launch that was just made.
#define XP_LAUNCHED()                                                          \
    do {                                                                       \
        hipError_t _e = hipGetLastError();                                     \
        if (_e != hipSuccess)                                                  \
            return ::xp::set_error(XP_E_HIP, "%s: kernel launch -> %s",        \
                                   __func__, hipGetErrorString(_e));           \
    } while (0)
