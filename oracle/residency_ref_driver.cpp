// residency_ref_driver.cpp -- test infrastructure: a C entry layer over the
// reference's MoEResidencyTracker (src/layers/moe_residency.{h,cpp}), compiled
// together with that unmodified source into oracle/_ref/libresidency_ref.so by
// oracle/Makefile.  The tests drive it with the same dispatch sequences as
// libqmoe's tracker and compare cold counts, resident sets and frequencies.
#include <algorithm>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>

#include "moe_residency.h"

namespace {
thread_local std::string g_err;
}

extern "C" {

const char* ref_res_last_error() { return g_err.c_str(); }

void* ref_res_create(int n_experts, int resident_k) {
    try {
        return new MoEResidencyTracker(n_experts, resident_k);
    } catch (const std::exception& e) {
        g_err = e.what();
        return nullptr;
    }
}

void ref_res_destroy(void* t) { delete static_cast<MoEResidencyTracker*>(t); }

// 0 on success, 1 when the tracker threw (message in ref_res_last_error)
int ref_res_record(void* t, int expert_id) {
    try {
        static_cast<MoEResidencyTracker*>(t)->record_dispatch(expert_id);
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return 1;
    }
}

uint64_t ref_res_cold(const void* t) { return static_cast<const MoEResidencyTracker*>(t)->cold_dispatch_count(); }

int ref_res_is_resident(const void* t, int expert_id) {
    return static_cast<const MoEResidencyTracker*>(t)->is_resident(expert_id) ? 1 : 0;
}

int ref_res_resident_set(const void* t, int* out, int cap) {
    const auto& r = static_cast<const MoEResidencyTracker*>(t)->resident_set();
    for (int i = 0; i < (int)r.size() && i < cap; ++i) out[i] = r[(size_t)i];
    return (int)r.size();
}

void ref_res_frequencies(const void* t, uint64_t* out, int cap) {
    const auto& f = static_cast<const MoEResidencyTracker*>(t)->frequencies();
    std::memcpy(out, f.data(), sizeof(uint64_t) * (size_t)std::min<size_t>(f.size(), (size_t)cap));
}

void ref_res_reset(void* t) { static_cast<MoEResidencyTracker*>(t)->reset(); }

}  // extern "C"
