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

struct PhaseStats {
    double total_ms = 0.0, max_ms = 0.0;
    long calls = 0;
};

// Accumulated wall time per named phase.
class Profile {
  public:
    static Profile &get() {
        static Profile p;
        return p;
    }
    void add(const std::string &phase, double ms) {
        std::lock_guard<std::mutex> lock(mu_);
        PhaseStats &s = stats_[phase];
        s.total_ms += ms;
        s.calls++;
        if (ms > s.max_ms)
            s.max_ms = ms;
    }
    PhaseStats stats(const std::string &phase) {
        std::lock_guard<std::mutex> lock(mu_);
        return stats_[phase];
    }
    void reset() {
        std::lock_guard<std::mutex> lock(mu_);
        stats_.clear();
    }
    void print(FILE *out = stderr) {
        std::lock_guard<std::mutex> lock(mu_);
        std::fprintf(out, "%-24s %10s %8s %10s %10s\n", "phase", "total ms", "calls", "avg ms",
                     "max ms");
        for (const auto &[name, s] : stats_)
            std::fprintf(out, "%-24s %10.2f %8ld %10.3f %10.3f\n", name.c_str(), s.total_ms,
                         s.calls, s.total_ms / s.calls, s.max_ms);
    }

  private:
    std::mutex mu_;
    std::map<std::string, PhaseStats> stats_;
};

// Scope timer: adds the elapsed time to Profile under its name when destroyed.
class Timer {
  public:
    explicit Timer(std::string name)
        : name_(std::move(name)), start_(std::chrono::steady_clock::now()) {}
    Timer(const Timer &) = delete;
    Timer &operator=(const Timer &) = delete;
    ~Timer() {
        const auto end = std::chrono::steady_clock::now();
        Profile::get().add(name_, std::chrono::duration<double, std::milli>(end - start_).count());
    }

  private:
    std::string name_;
    std::chrono::steady_clock::time_point start_;
};

} // namespace apex
