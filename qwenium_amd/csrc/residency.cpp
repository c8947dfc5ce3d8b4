// residency.cpp -- expert-dispatch telemetry on the host: per-expert dispatch
// frequencies, the resident set (the resident_k most dispatched experts) and
// the count of "cold" dispatches (to an expert outside the resident set at the
// moment of dispatch).
//
// Behaviour restated from the reference (src/layers/moe_residency.cpp:8-82,
// src/layers/moe_residency.h:1-70, src/telemetry/metrics.h:13-17):
//   - resident_k is clamped to n_experts; n_experts <= 0 or resident_k <= 0
//     is an error (same messages);
//   - a dispatch checks residency BEFORE counting itself, then the resident
//     set is refreshed; ids outside [0, n_experts) are an error;
//   - the resident set is the first resident_k experts of the ids 0..E-1
//     partially sorted by descending frequency, keeping those with frequency
//     > 0, in that order;
//   - reset() zeroes everything.
// Equal frequencies: the C++ standard leaves partial_sort's order of equivalent
// elements open, and the reference's cold counts depend on it (which of two
// tied experts stays resident).  The selection therefore runs the same
// standard-library partial_sort over ascending ids with the same "frequency
// greater" order, so both agree bit for bit when built against the same
// standard library.  The per-expert residency flags make is_resident O(1).
//
// record_counts is the batched feed from the device histogram that the
// routing's count sort accumulates (qmoe_layer_set_expert_counts): a batch of
// dispatches is cold by the resident set at the batch's start, then the set is
// refreshed once.  For a batch of one dispatch it equals record.
#include <algorithm>
#include <cstdint>
#include <numeric>
#include <string>
#include <vector>

#include "qmoe.h"
#include "qmoe_internal.h"

struct qmoe_residency {
    int n_experts = 0;
    int resident_k = 0;
    std::vector<uint64_t> freq;
    std::vector<int32_t> resident;  // the resident set, in selection order
    std::vector<uint8_t> is_res;    // [n_experts] membership of `resident`
    std::vector<int32_t> order;     // selection scratch
    uint64_t cold = 0;

    void refresh() {
        for (int32_t e : resident) is_res[(size_t)e] = 0;
        resident.clear();
        std::iota(order.begin(), order.end(), 0);
        const uint64_t* f = freq.data();
        std::partial_sort(order.begin(), order.begin() + resident_k, order.end(),
                          [f](int32_t a, int32_t b) { return f[a] > f[b]; });
        for (int i = 0; i < resident_k; ++i) {
            const int32_t e = order[(size_t)i];
            if (f[e] == 0) continue;
            resident.push_back(e);
            is_res[(size_t)e] = 1;
        }
    }
};

namespace {

int range_error(int e, int n) {
    return qmoe::set_error(QMOE_ERR_VALUE, "moe_residency: record_dispatch: expert_id=" + std::to_string(e) +
                                               " out of range [0, " + std::to_string(n) + ")");
}

}  // namespace

extern "C" {

int qmoe_residency_create(int32_t n_experts, int32_t resident_k, qmoe_residency** out) {
    qmoe::clear_error();
    if (!out) return qmoe::set_error(QMOE_ERR_NULL, "qmoe: out expected non-null, got null");
    *out = nullptr;
    if (n_experts <= 0)
        return qmoe::set_error(QMOE_ERR_VALUE, "moe_residency: n_experts must be > 0; got " + std::to_string(n_experts));
    if (resident_k <= 0)
        return qmoe::set_error(QMOE_ERR_VALUE, "moe_residency: resident_k must be > 0; got " + std::to_string(resident_k));
    auto r = new qmoe_residency();
    r->n_experts = n_experts;
    r->resident_k = std::min(resident_k, n_experts);
    r->freq.assign((size_t)n_experts, 0);
    r->is_res.assign((size_t)n_experts, 0);
    r->order.resize((size_t)n_experts);
    r->resident.reserve((size_t)r->resident_k);
    *out = r;
    return QMOE_OK;
}

void qmoe_residency_destroy(qmoe_residency* r) { delete r; }

int qmoe_residency_record(qmoe_residency* r, const int32_t* expert_ids, int64_t n) {
    qmoe::clear_error();
    if (!r) return qmoe::set_error(QMOE_ERR_NULL, "qmoe: tracker expected non-null, got null");
    if (n > 0 && !expert_ids) return qmoe::set_error(QMOE_ERR_NULL, "qmoe: expert_ids expected non-null, got null");
    for (int64_t i = 0; i < n; ++i) {
        const int e = expert_ids[i];
        if (e < 0 || e >= r->n_experts) return range_error(e, r->n_experts);
        if (!r->is_res[(size_t)e]) ++r->cold;
        ++r->freq[(size_t)e];
        r->refresh();
    }
    return QMOE_OK;
}

int qmoe_residency_record_counts(qmoe_residency* r, const uint64_t* counts, int32_t n) {
    qmoe::clear_error();
    if (!r || !counts) return qmoe::set_error(QMOE_ERR_NULL, "qmoe: tracker and counts expected non-null, got null");
    if (n != r->n_experts)
        return qmoe::set_error(QMOE_ERR_SHAPE, "moe_residency: counts expected " + std::to_string(r->n_experts) +
                                                   " entries, got " + std::to_string(n));
    uint64_t total = 0;
    for (int e = 0; e < n; ++e) {
        if (!r->is_res[(size_t)e]) r->cold += counts[e];
        r->freq[(size_t)e] += counts[e];
        total += counts[e];
    }
    if (total) r->refresh();
    return QMOE_OK;
}

int qmoe_residency_is_resident(const qmoe_residency* r, int32_t expert_id) {
    if (!r || expert_id < 0 || expert_id >= r->n_experts) return 0;
    return r->is_res[(size_t)expert_id] ? 1 : 0;
}

int qmoe_residency_metrics(const qmoe_residency* r, qmoe_moe_metrics* out) {
    qmoe::clear_error();
    if (!r || !out) return qmoe::set_error(QMOE_ERR_NULL, "qmoe: tracker and out expected non-null, got null");
    out->cold_dispatch_count = r->cold;
    return QMOE_OK;
}

int32_t qmoe_residency_resident_set(const qmoe_residency* r, int32_t* out, int32_t cap) {
    if (!r) return 0;
    const int32_t n = (int32_t)r->resident.size();
    for (int32_t i = 0; out && i < std::min(n, cap); ++i) out[i] = r->resident[(size_t)i];
    return n;
}

int qmoe_residency_frequencies(const qmoe_residency* r, uint64_t* out, int32_t cap) {
    qmoe::clear_error();
    if (!r || !out) return qmoe::set_error(QMOE_ERR_NULL, "qmoe: tracker and out expected non-null, got null");
    if (cap < r->n_experts)
        return qmoe::set_error(QMOE_ERR_CAPACITY, "qmoe: out expected room for " + std::to_string(r->n_experts) +
                                                      " counts, got " + std::to_string(cap));
    std::copy(r->freq.begin(), r->freq.end(), out);
    return QMOE_OK;
}

void qmoe_residency_reset(qmoe_residency* r) {
    if (!r) return;
    std::fill(r->freq.begin(), r->freq.end(), 0);
    std::fill(r->is_res.begin(), r->is_res.end(), 0);
    r->resident.clear();
    r->cold = 0;
}

}  // extern "C"
