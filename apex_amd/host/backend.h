// The engine's GPU interface, as src/backend/backend.h:9-63 declares it: opaque buffers,
// positional kernel arguments, threadgroup grids, and an in-order queue with sync().
// Kept identical in names and signatures so engine code written against the reference
// interface builds unchanged against apex::HipBackend (hip_backend.h).
#pragma once
#include <cstddef>
#include <cstdint>
#include <initializer_list>

namespace apex {

struct Buffer; // defined by each backend (hip_backend.h for HIP)

// One kernel argument: a buffer (plus byte offset) or a small value whose bytes are
// copied when the launch is queued, so temporaries are fine (backend.h:15-29).
struct Arg {
    Buffer *buffer = nullptr;
    size_t offset = 0;
    const void *bytes = nullptr;
    size_t size = 0;

    static Arg buf(Buffer *b, size_t offset = 0) { return {b, offset, nullptr, 0}; }
    template <class T> static Arg val(const T &v) { return {nullptr, 0, &v, sizeof(T)}; }
};

// Grid (in threadgroups) or threadgroup shape, 1D to 3D (backend.h:31-37).
struct Dim3 {
    uint32_t x = 1, y = 1, z = 1;
    Dim3(uint32_t x_, uint32_t y_ = 1, uint32_t z_ = 1) : x(x_), y(y_), z(z_) {}
    uint32_t total() const { return x * y * z; }
};

class Backend {
  public:
    virtual ~Backend() = default;
    // GPU-visible view of caller memory (backend.h:43-44).
    virtual Buffer *wrapNoCopy(void *cpu_ptr, size_t bytes) = 0;
    // Fresh memory reachable from the CPU (contents) and the GPU (backend.h:46-47).
    virtual Buffer *allocate(size_t bytes, const char *category) = 0;
    // CPU pointer to the buffer's bytes (backend.h:49-50).
    virtual void *contents(Buffer *buffer) = 0;
    // Free a buffer (backend.h:52-53).
    virtual void release(Buffer *buffer) = 0;
    // Queue one kernel launch (backend.h:55-60).
    virtual void run(const char *kernel, std::initializer_list<Arg> args, Dim3 threadgroups,
                     Dim3 threads_per_group) = 0;
    // Submit queued work and wait for it (backend.h:62-63).
    virtual void sync() = 0;
};

} // namespace apex
