// CPU checks of the GQA prefill attention's row-block order
// (qora-llm-4b_amd/csrc/qm_gqa_plan.h): every order hands out each block once,
// the list-scheduling model matches hand-worked and brute-force cases, and the
// automatic choice takes the packed order only where longest first is at
// least 5% behind it.
#include <cstdio>
#include <cstdlib>

#include "qm_gqa_plan.h"

using namespace qm_plan;

static int failures = 0;
#define CHECK(c)                                                                   \
    do {                                                                           \
        if (!(c)) {                                                                \
            std::printf("FAILED %s:%d: %s\n", __FILE__, __LINE__, #c);           \
            ++failures;                                                            \
        }                                                                          \
    } while (0)

static std::vector<int32_t> longest_first(int32_t nblk) {
    std::vector<int32_t> v;
    for (int32_t n = 0; n < nblk; ++n) v.push_back(nblk - 1 - n);
    return v;
}

static double mean_load(int32_t S, int32_t bins) {
    double t = 0.0;
    for (int32_t tb = 0; tb < (S + 47) / 48; ++tb) t += gqp_block_cost(tb, S);
    return t / bins;
}

// smallest makespan over every assignment of the blocks to the bins
static double brute_force(int32_t S, int32_t bins) {
    const int32_t nblk = (S + 47) / 48;
    long total = 1;
    for (int32_t i = 0; i < nblk; ++i) total *= bins;
    double best = 1e30;
    for (long a = 0; a < total; ++a) {
        std::vector<double> l(static_cast<size_t>(bins), 0.0);
        long x = a;
        for (int32_t i = 0; i < nblk; ++i, x /= bins) l[x % bins] += gqp_block_cost(i, S);
        best = std::min(best, *std::max_element(l.begin(), l.end()));
    }
    return best;
}

int main() {
    // block costs: 64-key tiles up to the block's last row, plus 8
    CHECK(gqp_block_cost(0, 8192) == 1 + 8);
    CHECK(gqp_block_cost(1, 8192) == 2 + 8);
    CHECK(gqp_block_cost(2, 8192) == 3 + 8 && gqp_block_cost(3, 8192) == 3 + 8);
    CHECK(gqp_block_cost(170, 8192) == 128 + 8);     // rows 8160..8191, the last one partial
    CHECK(gqp_block_cost(4, 218) == 4 + 8);          // rows 192..217

    // hand-worked: S = 218, 5 blocks of costs 9, 10, 11, 11, 12 over 2 workgroups.
    // Longest first: 12 | 11, then 11 -> the second (22), 10 -> the first (22),
    // 9 -> the first (31).  The best split is {9, 10, 11} | {11, 12} = 30.
    CHECK(gqp_makespan(longest_first(5), 218, 2) == 31);
    CHECK(brute_force(218, 2) == 30);
    CHECK(gqp_makespan(gqp_packed_order(218, 2), 218, 2) == 30);

    // tiny cases against brute force: the order the automatic mode picks is
    // never behind longest first, and within 10% of the best assignment
    for (int32_t S = 100; S <= 48 * 11; S += 29)
        for (int32_t bins = 2; bins <= 3; ++bins) {
            const int32_t nblk = (S + 47) / 48;
            if (nblk <= bins) continue;
            std::vector<uint16_t> order(QM_GQA_PREFILL_ORDER_MAX);
            const int32_t used = gqp_set_order(order.data(), S, bins, 0);
            std::vector<int32_t> chosen = longest_first(nblk);
            if (used) chosen.assign(order.begin(), order.begin() + nblk);
            const double m = gqp_makespan(chosen, S, bins);
            CHECK(m <= gqp_makespan(longest_first(nblk), S, bins));
            CHECK(m <= 1.10 * brute_force(S, bins));
        }

    // every forced order is a permutation of the blocks; longest first is
    // the fallback where the table cannot hold them or they do not outnumber
    // the workgroups
    for (int32_t S : {1, 47, 48, 49, 1000, 3000, 3072, 4096, 5000, 8191, 8192, 8193, 12000, 16384, 32768,
                      49152, 49153, 65536})
        for (int32_t bins : {16, 32, 64}) {
            const int32_t nblk = (S + 47) / 48;
            const int32_t b = std::max(1, std::min(bins, nblk));
            std::vector<uint16_t> order(QM_GQA_PREFILL_ORDER_MAX, 0xffff);
            CHECK(gqp_set_order(order.data(), S, b, 1) == 0);
            const int32_t used = gqp_set_order(order.data(), S, b, 2);
            CHECK(used == (nblk > b && nblk <= QM_GQA_PREFILL_ORDER_MAX ? 1 : 0));
            if (used) {
                std::vector<int> seen(static_cast<size_t>(nblk), 0);
                for (int32_t n = 0; n < nblk; ++n) {
                    CHECK(order[n] < nblk);
                    if (order[n] < nblk) ++seen[order[n]];
                }
                CHECK(std::all_of(seen.begin(), seen.end(), [](int k) { return k == 1; }));
            }
        }

    // 8192 tokens over 64 workgroups per group: longest first leaves the
    // busiest 12% over the mean, the packed order within 1%, and the
    // automatic mode takes it; at the other measured lengths longest first
    // is within 5% and stays
    {
        const double mean = mean_load(8192, 64);
        std::vector<uint16_t> order(QM_GQA_PREFILL_ORDER_MAX);
        CHECK(gqp_makespan(longest_first(171), 8192, 64) >= 1.10 * mean);
        CHECK(gqp_makespan(gqp_packed_order(8192, 64), 8192, 64) <= 1.01 * mean);
        CHECK(gqp_set_order(order.data(), 8192, 64, 0) == 1);
        for (int32_t S : {4096, 6000, 12000, 16384, 32768})
            CHECK(gqp_set_order(order.data(), S, std::min(64, (S + 47) / 48), 0) == 0);
    }

    if (failures) {
        std::printf("%d checks failed\n", failures);
        return 1;
    }
    std::printf("all checks passed\n");
    return 0;
}
