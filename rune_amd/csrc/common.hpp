// Shared host/device utilities of the RUNE HIP library.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/rune_hip.h"

namespace rune {

// Error carrying a RUNE_ERR_* code; converted at the C boundary.
struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string &m) : std::runtime_error(m), code(c) {}
};

void set_last_error(const std::string &msg);

#define RUNE_HIP_CHECK(expr)                                                          \
    do {                                                                              \
        hipError_t _e = (expr);                                                       \
        if (_e != hipSuccess)                                                         \
            throw ::rune::Error(RUNE_ERR_HIP, std::string(#expr) + ": " +             \
                                                  hipGetErrorString(_e));             \
    } while (0)

#define RUNE_REQUIRE(cond, code, msg)                                                 \
    do {                                                                              \
        if (!(cond)) throw ::rune::Error((code), (msg));                              \
    } while (0)

// Runs f and converts exceptions into return codes + thread-local message.
template <class F>
int guarded(F &&f) {
    try {
        f();
        return RUNE_OK;
    } catch (const Error &e) {
        set_last_error(e.what());
        return e.code;
    } catch (const std::exception &e) {
        set_last_error(e.what());
        return RUNE_ERR_ARGUMENT;
    }
}

// Growable device buffer owned by a handle.  Capacity only grows; contents
// are not preserved across growth.
struct DeviceBuffer {
    void *ptr = nullptr;
    size_t bytes = 0;
    DeviceBuffer() = default;
    DeviceBuffer(const DeviceBuffer &) = delete;
    DeviceBuffer &operator=(const DeviceBuffer &) = delete;
    ~DeviceBuffer() { release(); }
    void release() {
        if (ptr) (void)hipFree(ptr);
        ptr = nullptr;
        bytes = 0;
    }
    void reserve(size_t need) {
        if (need <= bytes) return;
        release();
        size_t grow = need + need / 4 + 256;
        RUNE_HIP_CHECK(hipMalloc(&ptr, grow));
        bytes = grow;
    }
    template <class T>
    T *as() const { return static_cast<T *>(ptr); }
};

// A few words of pinned host memory that kernels store into directly (small
// readbacks need no copy then); allocated on first use.
struct PinnedWords {
    int32_t *ptr = nullptr;
    PinnedWords() = default;
    PinnedWords(const PinnedWords &) = delete;
    PinnedWords &operator=(const PinnedWords &) = delete;
    ~PinnedWords() {
        if (ptr) (void)hipHostFree(ptr);
    }
    int32_t *get() {
        if (!ptr) {
            void *p = nullptr;
            RUNE_HIP_CHECK(hipHostMalloc(&p, 64, hipHostMallocCoherent));
            ptr = static_cast<int32_t *>(p);
        }
        return ptr;
    }
    int32_t read(int k) const { return static_cast<volatile int32_t *>(ptr)[k]; }
};

// Bump allocator over one DeviceBuffer: plan sizes first, then carve.
struct Arena {
    std::vector<size_t> sizes;
    size_t total = 0;
    static size_t align(size_t x) { return (x + 255) & ~size_t(255); }
    size_t add(size_t bytes) {
        size_t off = total;
        total += align(bytes);
        return off;
    }
};

inline int ceil_div(int64_t a, int64_t b) { return int((a + b - 1) / b); }

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace rune
