// Optional per-kernel timing with HIP events on the launching stream (off by default).
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "common.h"

namespace hm {
namespace {

struct Span {
    std::string name;
    hipEvent_t begin, end;
};

std::mutex g_mu;
bool g_on = false;
std::vector<Span> g_pending;
std::vector<hipEvent_t> g_pool;
std::map<std::string, std::pair<double, int64_t>> g_totals;
std::string g_open;
hipEvent_t g_open_event = nullptr;

hipEvent_t get_event() {
    if (!g_pool.empty()) {
        hipEvent_t e = g_pool.back();
        g_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

void collect_locked() {
    for (auto& s : g_pending) {
        float ms = 0.0f;
        if (hipEventSynchronize(s.end) == hipSuccess && hipEventElapsedTime(&ms, s.begin, s.end) == hipSuccess) {
            auto& t = g_totals[s.name];
            t.first += ms;
            t.second += 1;
        }
        g_pool.push_back(s.begin);
        g_pool.push_back(s.end);
    }
    g_pending.clear();
}

}  // namespace

// launches of an allocation-free entry point record no timing events (events are created on demand)
thread_local int g_quiet = 0;
ProfileOff::ProfileOff() { ++g_quiet; }
ProfileOff::~ProfileOff() { --g_quiet; }

// profiling() gates host-side readbacks for the timing report: never inside an allocation-free call, which must
// not synchronise its stream (a caller may be capturing it into a graph)
bool profiling() { return g_on && !g_quiet; }

void prof_begin(hipStream_t st, const char* name) {
    if (!g_on || g_quiet) return;
    std::lock_guard<std::mutex> lock(g_mu);
    g_open = name;
    g_open_event = get_event();
    if (g_open_event) (void)hipEventRecord(g_open_event, st);
}

void prof_end(hipStream_t st) {
    if (!g_on || g_quiet) return;
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_open_event) return;
    hipEvent_t e = get_event();
    if (!e) return;
    (void)hipEventRecord(e, st);
    g_pending.push_back(Span{g_open, g_open_event, e});
    g_open_event = nullptr;
}

void prof_count(const char* name, int64_t count) {
    if (!g_on || g_quiet) return;
    std::lock_guard<std::mutex> lock(g_mu);
    g_totals[name].second += count;
}

}  // namespace hm

extern "C" void hm_profile_enable(int on) {
    std::lock_guard<std::mutex> lock(hm::g_mu);
    hm::g_on = on != 0;
}

extern "C" void hm_profile_reset(void) {
    std::lock_guard<std::mutex> lock(hm::g_mu);
    hm::collect_locked();
    hm::g_totals.clear();
}

extern "C" int hm_profile_query(const char* name, double* total_ms, int64_t* launches) {
    std::lock_guard<std::mutex> lock(hm::g_mu);
    hm::collect_locked();
    auto it = hm::g_totals.find(name ? name : "");
    if (total_ms) *total_ms = it == hm::g_totals.end() ? 0.0 : it->second.first;
    if (launches) *launches = it == hm::g_totals.end() ? 0 : it->second.second;
    return HM_OK;
}
