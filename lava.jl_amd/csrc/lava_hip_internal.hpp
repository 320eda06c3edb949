// lava_hip_internal.hpp -- status handling shared by the entry points.
#pragma once
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>

#include <functional>

#include "lava_hip.h"

namespace lava {

// Thread-local message behind lava_hip_last_error().
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();
int hip_fail(hipError_t e, const char* what);
// Launch check: the error (if any) hipGetLastError reports for the launch just made; a launch
// that succeeded is appended to the thread's kernel log (lava_hip_kernel_log).
int check_launch(const char* kernel);
// The kernel choice pinned for a family (LAVA_HIP_FAMILY_*) by lava_hip_set_kernel_override; 0 = automatic.
int kernel_override(int family);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// The library's workspace for `stream` on the current device: grown to at least `bytes` (a
// grown buffer is retired, not freed), then launch(buffer) runs under the lock that orders its
// users, so calls from several threads use it one after another in stream order.  The first
// STREAM_WS_RESERVED bytes hold the W8A16 split-K arrival counters, which every call leaves at
// zero; other users write only past them.
constexpr size_t STREAM_WS_RESERVED = 4096;
// A call on a stream that is capturing a graph does not allocate: it must fit the workspace the
// stream already has (the buffer is then kept until the process ends, since the graph holds
// its address).
int with_stream_workspace(size_t bytes, void* stream, const std::function<int(void*)>& launch);
// The most workspace a call on `stream` may plan for: unlimited (SIZE_MAX) unless the stream is
// capturing a graph, then the size of the buffer it already has (0 if none).
size_t stream_workspace_cap(void* stream);

// Frees the workspaces kept for `stream` (called by lava_hip_stream_destroy once the stream
// has drained).
void w8a16_release_stream(void* stream);

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

}  // namespace lava

#define LAVA_REQUIRE(cond, code, ...)      \
    do {                                   \
        if (!(cond)) {                     \
            ::lava::set_error(__VA_ARGS__); \
            return (code);                 \
        }                                  \
    } while (0)

#define LAVA_ARG(cond, ...) LAVA_REQUIRE(cond, LAVA_HIP_ERR_INVALID_ARG, __VA_ARGS__)

#define LAVA_HIP_TRY(expr)                                      \
    do {                                                        \
        hipError_t _lava_e = (expr);                            \
        if (_lava_e != hipSuccess) return ::lava::hip_fail(_lava_e, #expr); \
    } while (0)

#define LAVA_LAUNCH_CHECK(name)                    \
    do {                                           \
        int _lava_rc = ::lava::check_launch(name); \
        if (_lava_rc != LAVA_HIP_OK) return _lava_rc; \
    } while (0)
