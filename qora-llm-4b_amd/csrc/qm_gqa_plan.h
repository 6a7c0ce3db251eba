// qm_gqa_plan.h -- host-side row-block order for the GQA causal prefill
// attention's per-group queues (plain C++, no device code; shared by the
// runtime and its CPU test).
#pragma once
#include <stdint.h>

#include <algorithm>
#include <vector>

#include "qm_kernel_args.h"

namespace qm_plan {
// Row-block order of the attention's per-group queues.  Each kv group's
// blocks go to whichever of its `bins` workgroups draws next, so the order
// decides how the causal triangle's unequal blocks pack.  Block tb (rows
// 48 tb .. 48 tb + 47) costs its 64-key tiles plus about eight tiles' worth
// of q preparation and epilogue (per-workgroup stamps at 8192 tokens: ~2.5 us
// per tile, 14-20 us per block).  Longest first packs some lengths badly: at
// 8192 tokens (171 blocks over 64 workgroups) the busiest workgroup gets 12%
// more than the mean.  The plan packs the blocks by best-fit decreasing (each block
// into the fullest workgroup it fits, under the smallest capacity, raised in
// 0.25% steps from the mean, at which all fit) and lists them by planned
// start time, longest first among equal starts: at equal speeds the queue
// then reproduces the packing, and it still adapts when workgroups run at
// different speeds.
inline double gqp_block_cost(int32_t tb, int32_t S) {
    const int32_t rows_end = std::min(48 * tb + 48, S);
    return static_cast<double>((rows_end + 63) / 64) + 8.0;
}

// Finish time of the last of `bins` workgroups that draw the blocks in this
// order, each drawing as it finishes (all at equal speed).
inline double gqp_makespan(const std::vector<int32_t>& order, int32_t S, int32_t bins) {
    std::vector<double> t(static_cast<size_t>(bins), 0.0);
    for (int32_t tb : order) {
        auto it = std::min_element(t.begin(), t.end());
        *it += gqp_block_cost(tb, S);
    }
    return *std::max_element(t.begin(), t.end());
}

inline std::vector<int32_t> gqp_packed_order(int32_t S, int32_t bins) {
    const int32_t nblk = (S + 47) / 48;
    double total = 0.0;
    for (int32_t tb = 0; tb < nblk; ++tb) total += gqp_block_cost(tb, S);
    std::vector<std::vector<int32_t>> bin;
    for (int step = 0;; ++step) {
        const double cap = total / bins * (1.0 + 0.0025 * step) + 1e-9;
        bin.assign(static_cast<size_t>(bins), {});
        std::vector<double> load(static_cast<size_t>(bins), 0.0);
        bool ok = true;
        for (int32_t tb = nblk - 1; tb >= 0 && ok; --tb) {   // longest first
            const double c = gqp_block_cost(tb, S);
            int best = -1;
            for (int i = 0; i < bins; ++i)
                if (load[i] + c <= cap && (best < 0 || load[i] > load[best])) best = i;
            if (best < 0) ok = false;
            else { bin[best].push_back(tb); load[best] += c; }
        }
        if (ok) break;
    }
    struct Entry { double start, cost; int32_t tb; };
    std::vector<Entry> e;
    for (const auto& b : bin) {
        double t = 0.0;
        for (int32_t tb : b) {                  // already longest first
            e.push_back({t, gqp_block_cost(tb, S), tb});
            t += gqp_block_cost(tb, S);
        }
    }
    std::stable_sort(e.begin(), e.end(), [](const Entry& x, const Entry& y) {
        return x.start != y.start ? x.start < y.start : x.cost > y.cost;
    });
    std::vector<int32_t> order;
    for (const auto& x : e) order.push_back(x.tb);
    return order;
}

// Write the queue order for seq_len S over `bins` workgroups per group into
// order[0 .. nblk) and return 1, or return 0 for longest first.
// mode 0: the packed order where the queue simulation puts longest first at
// least 5% behind it; 1: longest first; 2: the packed order whenever the
// blocks outnumber the workgroups and fit the table.
inline int32_t gqp_set_order(uint16_t* order, int32_t S, int32_t bins, int64_t mode) {
    const int32_t nblk = (S + 47) / 48;
    if (mode == 1 || nblk <= bins || nblk > QM_GQA_PREFILL_ORDER_MAX) return 0;
    const std::vector<int32_t> packed = gqp_packed_order(S, bins);
    if (mode == 0) {
        std::vector<int32_t> longest(static_cast<size_t>(nblk));
        for (int32_t n = 0; n < nblk; ++n) longest[n] = nblk - 1 - n;
        if (gqp_makespan(longest, S, bins) < 1.05 * gqp_makespan(packed, S, bins)) return 0;
    }
    // every block exactly once, or the longest-first order stays
    std::vector<char> seen(static_cast<size_t>(nblk), 0);
    if (static_cast<int32_t>(packed.size()) != nblk) return 0;
    for (int32_t tb : packed) {
        if (tb < 0 || tb >= nblk || seen[tb]) return 0;
        seen[tb] = 1;
    }
    for (int32_t n = 0; n < nblk; ++n) order[n] = static_cast<uint16_t>(packed[n]);
    return 1;
}
}  // namespace qm_plan
