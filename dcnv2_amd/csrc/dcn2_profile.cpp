// Opt-in per-stage timing with HIP events on the caller's stream
// (dcn2_profile_enable / dcn2_profile_read in include/dcnv2_amd.h).
#include <hip/hip_runtime.h>

#include <vector>

#include "../../include/dcnv2_amd.h"
#include "dcn2_profile.h"

namespace dcn2 {

namespace {
struct Pending {
    hipEvent_t start, stop;
};
struct ProfState {
    bool on = false;
    std::vector<Pending> pending[DCN2_STAGE_COUNT];
    std::vector<hipEvent_t> pool;
    Pending open[DCN2_STAGE_COUNT];
    bool is_open[DCN2_STAGE_COUNT] = {};
};
thread_local ProfState g_prof;

hipEvent_t take_event() {
    if (!g_prof.pool.empty()) {
        hipEvent_t e = g_prof.pool.back();
        g_prof.pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}
}  // namespace

void prof_begin(int stage, hipStream_t s) {
    if (!g_prof.on || stage < 0 || stage >= DCN2_STAGE_COUNT) return;
    Pending p{take_event(), take_event()};
    if (!p.start || !p.stop) return;
    hipEventRecord(p.start, s);
    g_prof.open[stage] = p;
    g_prof.is_open[stage] = true;
}

void prof_end(int stage, hipStream_t s) {
    if (!g_prof.on || stage < 0 || stage >= DCN2_STAGE_COUNT || !g_prof.is_open[stage]) return;
    Pending p = g_prof.open[stage];
    hipEventRecord(p.stop, s);
    g_prof.pending[stage].push_back(p);
    g_prof.is_open[stage] = false;
}

}  // namespace dcn2

using namespace dcn2;

extern "C" {

int dcn2_profile_enable(int on) {
    g_prof.on = on != 0;
    return DCN2_OK;
}

int dcn2_profile_read(int stage, double *total_ms, int *launches) {
    if (stage < 0 || stage >= DCN2_STAGE_COUNT) return DCN2_EINVAL;
    double sum = 0.0;
    int n = 0;
    for (Pending &p : g_prof.pending[stage]) {
        float ms = 0.0f;
        if (hipEventSynchronize(p.stop) == hipSuccess &&
            hipEventElapsedTime(&ms, p.start, p.stop) == hipSuccess) {
            sum += ms;
            ++n;
        }
        g_prof.pool.push_back(p.start);
        g_prof.pool.push_back(p.stop);
    }
    g_prof.pending[stage].clear();
    if (total_ms) *total_ms = sum;
    if (launches) *launches = n;
    return DCN2_OK;
}

}  // extern "C"
