// Streaming packed weight files into device memory (the layer_NN.bin / core.bin files
// of tools/repack.py:180-257, read by the reference through mmap, src/file.h:27-73).
//
// The reference's memory is unified, so it maps a file and lets the GPU read the pages.
// Here device memory is separate: bytes move disk -> pinned host -> HBM.  Reader
// threads (one per two staging buffers) take the file's chunks from a shared counter;
// each fills one of its pinned buffers with pread while its other buffer's
// host-to-device copy runs on the stream, and refills a buffer only after the event
// recorded behind its copy has completed.  One reader's pread runs at about one core's
// copy rate from the page cache (24 GB/s measured), below what the copy engines take.
#include "apex_hip.h"

#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cerrno>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "file_io.h"

namespace apex_hip {

namespace {

// Pinned staging buffers and their events, kept for the process: pinning tens of MB
// costs milliseconds, as much as streaming a layer file.  Rebuilt when a call asks for
// another shape; one call at a time holds it.
struct Ring {
    std::vector<void *> host;
    std::vector<hipEvent_t> done;
    uint64_t chunk = 0;
    int device = -1;
    void release() {
        for (hipEvent_t e : done)
            if (e)
                (void)hipEventDestroy(e);
        for (void *p : host)
            if (p)
                (void)hipHostFree(p);
        host.clear();
        done.clear();
        chunk = 0;
        device = -1;
    }
    bool fits(uint64_t c, uint32_t n, int dev) const {
        return chunk == c && host.size() == n && device == dev;
    }
};

std::mutex g_ring_mu;
Ring g_ring;

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
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) {
        st.error = "no current device";
        close(fd);
        return st;
    }
    std::lock_guard<std::mutex> ring_lock(g_ring_mu);
    Ring &ring = g_ring;
    if (!ring.fits(chunk_bytes, n_buffers, device)) {
        ring.release();
        ring.host.assign(n_buffers, nullptr);
        ring.done.assign(n_buffers, nullptr);
        for (uint32_t i = 0; i < n_buffers; ++i) {
            if (hipHostMalloc(&ring.host[i], chunk_bytes, hipHostMallocDefault) != hipSuccess ||
                hipEventCreateWithFlags(&ring.done[i], hipEventDisableTiming) != hipSuccess) {
                ring.release();
                st.error = "cannot allocate pinned staging buffers";
                close(fd);
                return st;
            }
        }
        ring.chunk = chunk_bytes;
        ring.device = device;
    }
    // the chunks of every range, in file order
    struct Chunk {
        uint64_t off, len;
        char *dst;
    };
    std::vector<Chunk> chunks;
    for (size_t r = 0; r < n_ranges; ++r)
        for (uint64_t done = 0; done < ranges[r].bytes; done += chunk_bytes)
            chunks.push_back({ranges[r].offset + done, std::min(chunk_bytes, ranges[r].bytes - done),
                              static_cast<char *>(ranges[r].dst) + done});
    constexpr uint32_t kMaxReaders = 8;
    const uint32_t readers = std::max(1u, std::min(kMaxReaders, n_buffers / 2));
    const uint32_t per = n_buffers / readers; // buffers of each reader
    std::vector<char> in_use(n_buffers, 0);
    std::atomic<size_t> next{0};
    std::atomic<uint64_t> bytes{0};
    std::atomic<bool> failed{false};
    std::mutex err_mu;
    auto fail = [&](const std::string &why) {
        std::lock_guard<std::mutex> lock(err_mu);
        if (st.error.empty())
            st.error = why;
        failed = true;
    };
    auto reader = [&](uint32_t r) {
        if (r > 0 && hipSetDevice(device) != hipSuccess) // a new thread starts on device 0
            return fail("cannot select the device in a reader thread");
        for (uint32_t k = 0; !failed; ++k) {
            const size_t i = next.fetch_add(1);
            if (i >= chunks.size())
                return;
            const Chunk &c = chunks[i];
            const uint32_t b = r * per + k % per;
            if (in_use[b] && hipEventSynchronize(ring.done[b]) != hipSuccess)
                return fail("device copy failed");
            std::string why;
            if (!read_full(fd, ring.host[b], c.len, c.off, why))
                return fail(why);
            if (hipMemcpyAsync(c.dst, ring.host[b], c.len, hipMemcpyHostToDevice, stream) !=
                    hipSuccess ||
                hipEventRecord(ring.done[b], stream) != hipSuccess)
                return fail("cannot queue a host-to-device copy");
            in_use[b] = 1;
            bytes += c.len;
        }
    };
    std::vector<std::thread> pool;
    try {
        for (uint32_t r = 1; r < readers; ++r)
            pool.emplace_back(reader, r);
    } catch (const std::exception &) {
        fail("cannot start reader threads");
    }
    reader(0);
    for (std::thread &t : pool)
        t.join();
    st.bytes = bytes;
    // every staging buffer must be idle before it is freed
    for (uint32_t i = 0; i < n_buffers; ++i)
        if (in_use[i] && hipEventSynchronize(ring.done[i]) != hipSuccess && st.error.empty())
            st.error = "device copy failed";
    close(fd);
    return st;
}

} // namespace apex_hip
