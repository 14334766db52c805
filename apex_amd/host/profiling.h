// Memory and time accounting used by the backend, in the roles of the reference's
// src/profiling/memory.h (allocations by category) and src/profiling/timer.h
// (named phases, e.g. "gpu_sync").  Linux/ROCm version: device allocations are
// counted by category; the process view comes from /proc/self/status.
#pragma once
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <fstream>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

namespace apex {

// Device bytes held by the engine, per category ("core_weights", "expert_slots", ...).
class MemoryTracker {
  public:
    static MemoryTracker &get() {
        static MemoryTracker t;
        return t;
    }
    void add(const std::string &category, uint64_t bytes) {
        std::lock_guard<std::mutex> lock(mu_);
        by_category_[category] += bytes;
        total_ += bytes;
        if (total_ > peak_)
            peak_ = total_;
    }
    void remove(const std::string &category, uint64_t bytes) {
        std::lock_guard<std::mutex> lock(mu_);
        uint64_t &c = by_category_[category];
        c = c >= bytes ? c - bytes : 0;
        total_ = total_ >= bytes ? total_ - bytes : 0;
    }
    uint64_t total() {
        std::lock_guard<std::mutex> lock(mu_);
        return total_;
    }
    uint64_t peak() {
        std::lock_guard<std::mutex> lock(mu_);
        return peak_;
    }
    uint64_t category(const std::string &c) {
        std::lock_guard<std::mutex> lock(mu_);
        auto it = by_category_.find(c);
        return it == by_category_.end() ? 0 : it->second;
    }
    // Resident set size of the process in bytes (0 if unavailable).
    static uint64_t process_rss() {
        std::ifstream f("/proc/self/status");
        std::string key;
        while (f >> key) {
            if (key == "VmRSS:") {
                uint64_t kb = 0;
                f >> kb;
                return kb * 1024;
            }
            std::getline(f, key);
        }
        return 0;
    }
    void print(FILE *out = stderr) {
        std::lock_guard<std::mutex> lock(mu_);
        std::fprintf(out, "%-20s %14s\n", "category", "device MiB");
        for (const auto &[name, bytes] : by_category_)
            std::fprintf(out, "%-20s %14.2f\n", name.c_str(), bytes / 1048576.0);
        std::fprintf(out, "%-20s %14.2f (peak %.2f)\n", "total", total_ / 1048576.0,
                     peak_ / 1048576.0);
    }

  private:
    std::mutex mu_;
    std::map<std::string, uint64_t> by_category_;
    uint64_t total_ = 0, peak_ = 0;
};

// Wall-clock accounting per named phase ("gpu_sync" around Backend::sync, "mmap",
// ...).  Timer scopes report into the process-wide Profile; phases keep the order in
// which they first appeared.  Durations are kept as integer nanoseconds, so sums do
// not drift however many calls a phase collects.
class Profile {
  public:
    struct Phase {
        uint64_t count = 0;
        uint64_t total_ns = 0;
        uint64_t shortest_ns = UINT64_MAX;
        uint64_t longest_ns = 0;
        double mean_ms() const { return count ? total_ns / 1e6 / count : 0.0; }
    };

    static Profile &get() {
        static Profile p;
        return p;
    }
    // One call of `phase` that took `ms` milliseconds.
    void add(const std::string &phase, double ms) {
        const uint64_t ns = ms > 0.0 ? (uint64_t)(ms * 1e6 + 0.5) : 0;
        std::lock_guard<std::mutex> lock(mu_);
        Phase &p = slot(phase);
        p.count += 1;
        p.total_ns += ns;
        p.shortest_ns = ns < p.shortest_ns ? ns : p.shortest_ns;
        p.longest_ns = ns > p.longest_ns ? ns : p.longest_ns;
    }
    // A copy of one phase's record (all zero if it never ran).
    Phase phase(const std::string &name) {
        std::lock_guard<std::mutex> lock(mu_);
        for (const auto &e : phases_)
            if (e.first == name)
                return e.second;
        return Phase{};
    }
    void reset() {
        std::lock_guard<std::mutex> lock(mu_);
        phases_.clear();
    }
    // One line per phase: calls, total, mean, shortest and longest call.
    void print(FILE *out = stderr) {
        std::lock_guard<std::mutex> lock(mu_);
        for (const auto &[name, p] : phases_)
            std::fprintf(out, "[time] %s: %llu call%s, %.3f ms in all, %.3f ms each (%.3f .. %.3f)\n",
                         name.c_str(), (unsigned long long)p.count, p.count == 1 ? "" : "s",
                         p.total_ns / 1e6, p.mean_ms(), p.shortest_ns / 1e6, p.longest_ns / 1e6);
    }

  private:
    Phase &slot(const std::string &name) {
        for (auto &e : phases_)
            if (e.first == name)
                return e.second;
        phases_.emplace_back(name, Phase{});
        return phases_.back().second;
    }
    std::mutex mu_;
    std::vector<std::pair<std::string, Phase>> phases_;
};

// Times the enclosing scope: on destruction the elapsed steady-clock time is added
// to Profile::get() under the timer's phase name.
class Timer {
  public:
    explicit Timer(std::string phase) : phase_(std::move(phase)), t0_(Clock::now()) {}
    Timer(const Timer &) = delete;
    Timer &operator=(const Timer &) = delete;
    ~Timer() { Profile::get().add(phase_, elapsed_ms()); }
    double elapsed_ms() const {
        return std::chrono::duration<double, std::milli>(Clock::now() - t0_).count();
    }

  private:
    using Clock = std::chrono::steady_clock;
    std::string phase_;
    Clock::time_point t0_;
};

} // namespace apex
