// Host-side drive of the plan builders, router and diagnostics under
// AddressSanitizer / UndefinedBehaviorSanitizer (compiled and run by
// tests/test_host_sanitize.py; no GPU).  Every array of every tile layout the
// host builder makes is exported, and invalid inputs must return an error.
#include <cstdio>
#include <cstdlib>
#include <algorithm>
#include <random>
#include <vector>

#include "ra_spmm.h"

namespace {

int failures = 0;
#define EXPECT(cond)                                                              \
    do {                                                                          \
        if (!(cond)) {                                                            \
            std::fprintf(stderr, "EXPECT failed at line %d: %s\n", __LINE__, #cond); \
            ++failures;                                                           \
        }                                                                         \
    } while (0)

struct Csr {
    int M, K;
    std::vector<int32_t> rowptr, colind;
    std::vector<float> vals;
};

// Random CSR with empty rows, duplicate (row, column) entries and a few hub rows.
Csr random_csr(std::mt19937& rng, int M, int K, int avg, int hub) {
    Csr a{M, K, {0}, {}, {}};
    std::uniform_int_distribution<int> col(0, K - 1);
    std::uniform_real_distribution<float> val(-2.f, 2.f);
    for (int r = 0; r < M; ++r) {
        int d = static_cast<int>(rng() % (2 * avg + 1));
        if (r % 17 == 0) d = 0;
        if (r % 97 == 5) d = hub;
        std::vector<int32_t> cols;
        for (int i = 0; i < d; ++i) cols.push_back(col(rng));
        if (d > 1) cols.push_back(cols[0]);  // a duplicate
        std::sort(cols.begin(), cols.end());
        for (int32_t c : cols) {
            a.colind.push_back(c);
            a.vals.push_back(val(rng));
        }
        a.rowptr.push_back(static_cast<int32_t>(a.colind.size()));
    }
    return a;
}

void drive(const Csr& a) {
    const char* names[] = {"block_offsets", "atox", "win_rows", "vals", "seg_window", "seg_bbegin",
                           "seg_bend", "seg_slot", "split_windows", "split_offsets"};
    for (int kind = 0; kind < 3; ++kind) {
        for (int dtype : {RA_DTYPE_F16, RA_DTYPE_BF16}) {
            ra_tile_host* h = nullptr;
            EXPECT(ra_tile_host_build(kind, a.rowptr.data(), a.colind.data(), a.vals.data(), a.M, a.K, 64, dtype,
                                      &h) == RA_OK);
            ra_tile_info info;
            EXPECT(ra_tile_host_get_info(h, &info) == RA_OK);
            for (const char* n : names) {
                int64_t count = -1;
                EXPECT(ra_tile_host_export(h, n, nullptr, &count) == RA_OK && count >= 0);
                std::vector<char> buf(static_cast<size_t>(count) * 4 + 4);
                EXPECT(ra_tile_host_export(h, n, buf.data(), &count) == RA_OK);
            }
            ra_tile_host_destroy(h);
        }
    }
    ra_features f;
    EXPECT(ra_features_host(a.rowptr.data(), a.M, a.K, 128, &f) == RA_OK);
    for (int portfolio : {RA_PORTFOLIO_MAIN, RA_PORTFOLIO_FULL})
        for (int table : {RA_TABLE_REFERENCE, RA_TABLE_MI355X}) {
            ra_route r;
            EXPECT(ra_route_dispatch(&f, portfolio, table, &r) == RA_OK);
        }
    ra_diag_features d;
    EXPECT(ra_analyze_matrix(a.rowptr.data(), a.colind.data(), a.M, a.K, 128, &d) == RA_OK);
}

}  // namespace

int main() {
    std::mt19937 rng(12345);
    drive(random_csr(rng, 1, 1, 1, 1));
    drive(random_csr(rng, 300, 200, 5, 150));
    drive(random_csr(rng, 2000, 5000, 12, 3000));
    drive(random_csr(rng, 64, 70000, 40, 9000));
    // Invalid inputs return a status, never touch memory out of bounds.
    std::vector<int32_t> bad_rp = {0, 3, 1, 4}, ci = {0, 1, 2, 3};
    std::vector<float> v = {1, 2, 3, 4};
    ra_tile_host* h = nullptr;
    EXPECT(ra_tile_host_build(0, bad_rp.data(), ci.data(), v.data(), 3, 4, 64, RA_DTYPE_F16, &h) != RA_OK);
    std::vector<int32_t> rp = {0, 2, 4}, bad_ci = {0, 9, 1, 2};
    EXPECT(ra_tile_host_build(0, rp.data(), bad_ci.data(), v.data(), 2, 4, 64, RA_DTYPE_F16, &h) != RA_OK);
    ra_features f;
    EXPECT(ra_features_host(bad_rp.data(), 3, 4, 64, &f) != RA_OK);
    ra_route r;
    EXPECT(ra_route_dispatch(nullptr, 0, 0, &r) != RA_OK);
    std::printf("host sanitize driver: %d failures\n", failures);
    return failures == 0 ? 0 : 1;
}
