// apex::HipBackend over the C ABI (include/apex_hip.h).  Host-only C++: it includes no
// HIP headers and links only libapex_hip.so.
#include "hip_backend.h"

#include <stdexcept>
#include <vector>

#include "profiling.h"

namespace apex {
namespace {

void check(int rc, const char *what) {
    if (rc != APEX_HIP_OK)
        throw std::runtime_error(std::string(what) + ": " + apex_hip_last_error());
}

} // namespace

HipBackend::HipBackend(int device) {
    check(apex_hip_backend_create(device, &b_), "HipBackend");
    char name[256] = {};
    if (apex_hip_device_name(b_, name, sizeof(name)) == APEX_HIP_OK)
        name_ = name;
}

HipBackend::~HipBackend() {
    if (b_)
        apex_hip_backend_destroy(b_);
}

Buffer *HipBackend::wrapNoCopy(void *cpu_ptr, size_t bytes) {
    apex_hip_buffer *h = nullptr;
    check(apex_hip_wrap_no_copy(b_, cpu_ptr, bytes, &h), "wrapNoCopy");
    return new Buffer{h, bytes, "", false};
}

Buffer *HipBackend::allocate(size_t bytes, const char *category) {
    apex_hip_buffer *h = nullptr;
    check(apex_hip_allocate(b_, bytes, category, &h), "allocate");
    const std::string cat = category ? category : "";
    MemoryTracker::get().add(cat, bytes);
    return new Buffer{h, bytes, cat, true};
}

void *HipBackend::contents(Buffer *buffer) {
    if (!buffer)
        throw std::runtime_error("contents: null buffer");
    void *p = nullptr;
    check(apex_hip_contents(b_, buffer->handle, &p), "contents");
    return p;
}

void HipBackend::release(Buffer *buffer) {
    if (!buffer)
        return;
    if (buffer->tracked) // wrapped buffers are not tracked
        MemoryTracker::get().remove(buffer->category, buffer->length);
    check(apex_hip_release(b_, buffer->handle), "release");
    delete buffer;
}

void HipBackend::run(const char *kernel, std::initializer_list<Arg> args, Dim3 threadgroups,
                     Dim3 threads_per_group) {
    std::vector<apex_hip_arg> a;
    a.reserve(args.size());
    for (const Arg &x : args)
        a.push_back({x.buffer ? x.buffer->handle : nullptr, x.offset, x.bytes, x.size});
    const apex_hip_dim3 g{threadgroups.x, threadgroups.y, threadgroups.z};
    const apex_hip_dim3 t{threads_per_group.x, threads_per_group.y, threads_per_group.z};
    check(apex_hip_run(b_, kernel, a.data(), a.size(), g, t), kernel ? kernel : "run");
}

void HipBackend::sync() {
    Timer t("gpu_sync");
    check(apex_hip_sync(b_), "sync");
}

void HipBackend::loadFile(Buffer *buffer, size_t offset, const std::string &path,
                          uint64_t file_offset, uint64_t bytes) {
    check(apex_hip_load_file(b_, buffer ? buffer->handle : nullptr, offset, path.c_str(),
                             file_offset, bytes),
          "loadFile");
}

void *HipBackend::devicePtr(Buffer *buffer) const {
    void *p = nullptr;
    check(apex_hip_buffer_device_ptr(buffer->handle, &p), "devicePtr");
    return p;
}

void *HipBackend::stream() const { return apex_hip_backend_stream(b_); }

} // namespace apex
