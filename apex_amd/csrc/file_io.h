// Packed weight files -> device memory through pinned staging buffers (file_io.cpp).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

namespace apex_hip {

struct FileRange {
    uint64_t offset; // in the file
    uint64_t bytes;
    void *dst;       // device destination
};

struct FileCopyStatus {
    uint64_t bytes = 0;
    std::string error; // empty on success
};

// Copy each range of the file into its device destination, reading chunk_bytes at a
// time into a ring of n_buffers pinned buffers while earlier chunks' copies run on
// `stream`.  Returns once every copy has completed.
FileCopyStatus copy_file_ranges(const char *path, const FileRange *ranges, size_t n_ranges,
                                uint64_t chunk_bytes, uint32_t n_buffers, hipStream_t stream);

} // namespace apex_hip
