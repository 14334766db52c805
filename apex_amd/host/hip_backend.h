// apex::HipBackend: the Backend interface (backend.h) on an AMD GPU, over the C ABI of
// include/apex_hip.h.  It takes the place of src/backend/metal_backend.h /
// metal_backend.cpp; engine code (src/ops.h callers) switches backends by constructing
// a HipBackend instead of a MetalBackend.
//
// Memory model: the reference's buffers are unified (CPU and GPU share the bytes).
// Here every buffer is device memory with a host mirror managed by the C ABI:
// contents() returns the mirror (downloading it if a kernel wrote the buffer since),
// and the next run() that reads the buffer uploads the mirror first.  A pointer from
// contents() stays valid until release(); write through it before run(), read
// through it after sync() -- exactly the reference tests' pattern
// (src/tests/dense_mlp.cpp:97-109).
//
// Errors become std::runtime_error carrying the C ABI's message, as the Metal backend
// throws (metal_backend.cpp:18-34, 61-76, 91-93, 117-119, 169-171).  Not thread-safe:
// one host thread drives one backend, which owns one in-order stream.
#pragma once
#include <cstddef>
#include <cstdint>
#include <string>

#include "apex_hip.h"
#include "backend.h"

namespace apex {

struct Buffer {
    apex_hip_buffer *handle = nullptr;
    size_t length = 0;
    std::string category; // MemoryTracker category of an allocated buffer
    bool tracked = false; // allocated (tracked) or wrapped (not tracked)
};

class HipBackend : public Backend {
  public:
    explicit HipBackend(int device = 0);
    ~HipBackend() override;

    Buffer *wrapNoCopy(void *cpu_ptr, size_t bytes) override;
    Buffer *allocate(size_t bytes, const char *category) override;
    void *contents(Buffer *buffer) override;
    void release(Buffer *buffer) override;
    void run(const char *kernel, std::initializer_list<Arg> args, Dim3 threadgroups,
             Dim3 threads_per_group) override;
    void sync() override;

    // GPU name for benchmark output (metal_backend.h:29-30).
    const char *deviceName() const { return name_.c_str(); }
    // Device address of a buffer (for the direct entry points of apex_hip.h).
    void *devicePtr(Buffer *buffer) const;
    // The backend's stream (hipStream_t), for interop with other HIP code.
    void *stream() const;
    // Stream bytes [file_offset, file_offset + bytes) of a file into the buffer at
    // `offset` (pread into pinned staging overlapped with host-to-device copies); returns
    // when they are on the device.  Where the reference maps a packed file and wraps the
    // mapping (src/tests/dense_mlp.cpp:24-30), a discrete GPU loads it once.
    void loadFile(Buffer *buffer, size_t offset, const std::string &path, uint64_t file_offset,
                  uint64_t bytes);

    HipBackend(const HipBackend &) = delete;
    HipBackend &operator=(const HipBackend &) = delete;

  private:
    apex_hip_backend *b_ = nullptr;
    std::string name_;
};

} // namespace apex
