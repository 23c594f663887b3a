// Per-kernel event timing behind dsalt_timing_enable / dsalt_timing_report.
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/dsalt_amd.h"
#include "timing.h"

namespace dsalt {
namespace {

struct Pending {
    std::string name;
    hipEvent_t a, b;
};

std::atomic<bool> g_on{false};
std::mutex g_mu;
std::vector<Pending> g_pending;
std::vector<hipEvent_t> g_pool;
std::map<std::string, std::pair<long, double>> g_acc;
thread_local int t_open = -1;  // index in g_pending of this thread's open record

hipEvent_t take_event() {
    if (!g_pool.empty()) {
        hipEvent_t e = g_pool.back();
        g_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

}  // namespace

bool timing_enabled() { return g_on.load(std::memory_order_relaxed); }

void timing_begin(const char* name, hipStream_t stream) {
    std::lock_guard<std::mutex> lk(g_mu);
    Pending p;
    p.name = name;
    p.a = take_event();
    p.b = take_event();
    if (!p.a || !p.b) return;
    if (hipEventRecord(p.a, stream) != hipSuccess) return;  // this launch goes untimed
    g_pending.push_back(p);
    t_open = (int)g_pending.size() - 1;
}

void timing_end(hipStream_t stream) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (t_open < 0 || t_open >= (int)g_pending.size()) return;
    if (hipEventRecord(g_pending[t_open].b, stream) != hipSuccess)
        g_pending.erase(g_pending.begin() + t_open);  // no end mark: drop the launch from the report
    t_open = -1;
}

}  // namespace dsalt

extern "C" {

int dsalt_timing_enable(int enable) {
    std::lock_guard<std::mutex> lk(dsalt::g_mu);
    dsalt::g_on.store(enable != 0);
    return DSALT_OK;
}

int dsalt_timing_report(char* buf, size_t len) {
    std::lock_guard<std::mutex> lk(dsalt::g_mu);
    for (auto& p : dsalt::g_pending) {
        float ms = 0.f;
        if (hipEventSynchronize(p.b) == hipSuccess && hipEventElapsedTime(&ms, p.a, p.b) == hipSuccess) {
            auto& e = dsalt::g_acc[p.name];
            e.first += 1;
            e.second += ms;
        }
        dsalt::g_pool.push_back(p.a);
        dsalt::g_pool.push_back(p.b);
    }
    dsalt::g_pending.clear();
    std::string out;
    char line[256];
    for (auto& kv : dsalt::g_acc) {
        snprintf(line, sizeof(line), "%s %ld %.6f\n", kv.first.c_str(), kv.second.first, kv.second.second);
        out += line;
    }
    dsalt::g_acc.clear();
    if (buf && len) {
        size_t n = out.size() < len - 1 ? out.size() : len - 1;
        memcpy(buf, out.data(), n);
        buf[n] = 0;
    }
    return (int)out.size();
}

}  // extern "C"
