// Streaming packed weight files into device memory (the layer_NN.bin / core.bin files
// of tools/repack.py:180-257, read by the reference through mmap, src/file.h:27-73).
//
// The reference's memory is unified, so it maps a file and lets the GPU read the pages.
// Here device memory is separate: bytes move disk -> pinned host -> HBM.  A ring of
// pinned buffers overlaps the two legs: while buffer i's host-to-device copy runs on
// the stream, the next buffer is filled with pread; a buffer is refilled only after the
// event recorded behind its copy has completed.
#include "apex_hip.h"

#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>
#include <string>
#include <vector>

#include "file_io.h"

namespace apex_hip {

namespace {

struct Ring {
    std::vector<void *> host;
    std::vector<hipEvent_t> done;
    ~Ring() {
        for (hipEvent_t e : done)
            if (e)
                (void)hipEventDestroy(e);
        for (void *p : host)
            if (p)
                (void)hipHostFree(p);
    }
};

// pread until `len` bytes arrive (short reads are legal); false on error or EOF.
bool read_full(int fd, void *dst, uint64_t len, uint64_t off, std::string &err) {
    auto *p = static_cast<char *>(dst);
    while (len > 0) {
        const ssize_t n = pread(fd, p, len, (off_t)off);
        if (n < 0) {
            if (errno == EINTR)
                continue;
            err = std::string("read failed: ") + std::strerror(errno);
            return false;
        }
        if (n == 0) {
            err = "unexpected end of file";
            return false;
        }
        p += n;
        off += (uint64_t)n;
        len -= (uint64_t)n;
    }
    return true;
}

} // namespace

FileCopyStatus copy_file_ranges(const char *path, const FileRange *ranges, size_t n_ranges,
                                uint64_t chunk_bytes, uint32_t n_buffers, hipStream_t stream) {
    FileCopyStatus st;
    if (n_buffers == 0 || chunk_bytes == 0) {
        st.error = "chunk size and buffer count must be positive";
        return st;
    }
    const int fd = open(path, O_RDONLY);
    if (fd < 0) {
        st.error = std::string("cannot open ") + path + ": " + std::strerror(errno);
        return st;
    }
    struct stat sb {};
    if (fstat(fd, &sb) != 0) {
        st.error = std::string("cannot stat ") + path;
        close(fd);
        return st;
    }
    for (size_t r = 0; r < n_ranges; ++r)
        if (ranges[r].offset + ranges[r].bytes > (uint64_t)sb.st_size) {
            st.error = std::string("range past the end of ") + path;
            close(fd);
            return st;
        }
    Ring ring;
    ring.host.assign(n_buffers, nullptr);
    ring.done.assign(n_buffers, nullptr);
    for (uint32_t i = 0; i < n_buffers; ++i) {
        if (hipHostMalloc(&ring.host[i], chunk_bytes, hipHostMallocDefault) != hipSuccess ||
            hipEventCreateWithFlags(&ring.done[i], hipEventDisableTiming) != hipSuccess) {
            st.error = "cannot allocate pinned staging buffers";
            close(fd);
            return st;
        }
    }
    std::vector<bool> in_use(n_buffers, false);
    uint32_t next = 0;
    for (size_t r = 0; r < n_ranges && st.error.empty(); ++r) {
        const FileRange &fr = ranges[r];
        for (uint64_t done = 0; done < fr.bytes;) {
            const uint64_t len = fr.bytes - done < chunk_bytes ? fr.bytes - done : chunk_bytes;
            const uint32_t b = next;
            next = (next + 1) % n_buffers;
            if (in_use[b] && hipEventSynchronize(ring.done[b]) != hipSuccess) {
                st.error = "device copy failed";
                break;
            }
            if (!read_full(fd, ring.host[b], len, fr.offset + done, st.error))
                break;
            if (hipMemcpyAsync(static_cast<char *>(fr.dst) + done, ring.host[b], len,
                               hipMemcpyHostToDevice, stream) != hipSuccess ||
                hipEventRecord(ring.done[b], stream) != hipSuccess) {
                st.error = "cannot queue a host-to-device copy";
                break;
            }
            in_use[b] = true;
            done += len;
            st.bytes += len;
        }
    }
    // every staging buffer must be idle before it is freed
    for (uint32_t i = 0; i < n_buffers; ++i)
        if (in_use[i] && hipEventSynchronize(ring.done[i]) != hipSuccess && st.error.empty())
            st.error = "device copy failed";
    close(fd);
    return st;
}

} // namespace apex_hip
