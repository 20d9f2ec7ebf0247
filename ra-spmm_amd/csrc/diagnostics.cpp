// diagnostics.cpp — the diagnostic ("FULL") feature extractor.
//
// Structural statistics the reference reports through analyze_matrix and its
// FULL-portfolio plans (router/router_features.cpp:113-432).  None of them
// feeds the deployed seven-rule decision, which reads only M, d, CV and N.
// The statistics, thresholds and score weights are the reference's (they are
// the interface: a caller compares them across builds); the code is
// organised around four passes over host CSR arrays:
//   1. rows: lengths, column span, centroid and a 64-bucket column signature
//   2. 16x16 tiles: nnz per nonempty tile (sorted keys instead of a hash map;
//      the fills are sorted before use, so the statistics are identical)
//   3. locality: Jaccard similarity of signatures of adjacent rows, in the
//      natural order and in a (centroid bucket, span, -length) order
//   4. 16-row windows: compactness, similarity, density and irregularity scores
// Compiled with -ffp-contract=off so the float expressions round as written.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <numeric>
#include <vector>

#include "../../include/ra_spmm.h"
#include "ra_internal.hpp"

namespace {

constexpr int kTile = 16;          // tile edge of the fill statistics
constexpr int kBuckets = 64;       // signature buckets over the column range
constexpr int kWindow = 16;        // rows per scoring window
constexpr float kTcFill = 0.25f;   // tile fill of a tensor-core candidate

struct RowSig {
    int32_t len = 0, lo = 0, hi = 0;
    float centroid = 0.f;
    uint64_t sig = 0;
};

float clamp01(float x) { return std::max(0.f, std::min(1.f, x)); }
float ratio_or_zero(float num, float den) { return std::fabs(den) > 1e-6f ? num / den : 0.f; }

template <typename T>
float mean_of(const std::vector<T>& v) {
    if (v.empty()) return 0.f;
    double s = 0.0;
    for (T x : v) s += static_cast<double>(x);
    return static_cast<float>(s / static_cast<double>(v.size()));
}

float jaccard(uint64_t a, uint64_t b) {
    const int u = __builtin_popcountll(a | b);
    return u == 0 ? 0.f : static_cast<float>(__builtin_popcountll(a & b)) / static_cast<float>(u);
}

}  // namespace

extern "C" ra_status ra_analyze_matrix(const int32_t* rowptr, const int32_t* colind, int32_t M, int32_t K,
                                       int32_t N, ra_diag_features* out) {
    if (!out) return ra::fail(RA_ERR_INVALID_ARGUMENT, "analyze: out is NULL");
    std::memset(out, 0, sizeof(*out));
    if (M > 0 && !rowptr) return ra::fail(RA_ERR_INVALID_ARGUMENT, "analyze: rowptr is NULL");
    if (M <= 0 || K <= 0) return RA_OK;
    ra_diag_features& f = *out;
    const int64_t nnz = rowptr[M];
    f.M = M;
    f.K = K;
    f.N = N;
    f.nnz = nnz;
    if (nnz <= 0) return RA_OK;
    if (!colind) return ra::fail(RA_ERR_INVALID_ARGUMENT, "analyze: colind is NULL");
    for (int32_t r = 0; r < M; ++r)
        if (rowptr[r + 1] < rowptr[r]) return ra::fail(RA_ERR_INVALID_ARGUMENT, "analyze: rowptr not monotone");

    // 1. Rows.
    std::vector<RowSig> rows(M);
    double sum_len = 0.0;
    int32_t max_len = 0;
    for (int32_t r = 0; r < M; ++r) {
        const int32_t b = rowptr[r], e = rowptr[r + 1];
        RowSig& x = rows[r];
        x.len = e - b;
        sum_len += x.len;
        max_len = std::max(max_len, x.len);
        if (x.len > 0) {
            x.lo = colind[b];
            x.hi = colind[e - 1];
        }
        double csum = 0.0;
        for (int32_t p = b; p < e; ++p) {
            const int64_t c = colind[p];
            if (c < 0 || c >= K) return ra::fail(RA_ERR_INVALID_ARGUMENT, "analyze: column index out of range");
            csum += static_cast<double>(c);
            x.sig |= uint64_t{1} << std::min<int64_t>(kBuckets - 1, c * kBuckets / K);
        }
        x.centroid = x.len > 0 ? static_cast<float>(csum / x.len) : 0.f;
    }
    const double avg = sum_len / M;
    double dev2 = 0.0;
    int64_t dense_rows = 0, long_rows = 0, long_nnz = 0;
    const double long_at = std::max(32.0, 2.0 * avg);
    std::vector<int32_t> lens(M);
    for (int32_t r = 0; r < M; ++r) {
        const int32_t len = rows[r].len;
        lens[r] = len;
        dev2 += (len - avg) * (len - avg);
        dense_rows += len > 2.0 * avg;
        if (len >= long_at) {
            ++long_rows;
            long_nnz += len;
        }
    }
    const double sd = std::sqrt(dev2 / M);
    std::partial_sort(lens.begin(), lens.begin() + std::min<int32_t>(5, M), lens.end(), std::greater<int32_t>());
    int64_t top5 = 0;
    for (int i = 0; i < std::min<int32_t>(5, M); ++i) top5 += lens[i];
    const float fM = static_cast<float>(M), fnnz = static_cast<float>(nnz);
    f.avg_nnz_per_row = static_cast<float>(avg);
    f.std_nnz_per_row = static_cast<float>(sd);
    f.degree_cv = avg > 1e-6 ? static_cast<float>(sd / avg) : 0.f;
    f.max_to_mean_ratio = avg > 1e-6 ? static_cast<float>(max_len / avg) : 0.f;
    f.frac_dense_rows = static_cast<float>(dense_rows) / fM;
    f.skew_ratio = f.max_to_mean_ratio;
    f.long_row_fraction = static_cast<float>(long_rows) / fM;
    f.long_row_nnz_fraction = static_cast<float>(long_nnz) / fnnz;
    f.top_1_row_nnz_fraction = static_cast<float>(lens[0]) / fnnz;
    f.top_5_row_nnz_fraction = static_cast<float>(top5) / fnnz;

    // 2. Tiles: one key per nonzero, sorted, run lengths = nnz per tile.
    const int64_t tiles_c = (K + kTile - 1) / kTile, tiles_r = (M + kTile - 1) / kTile;
    std::vector<int64_t> keys;
    keys.reserve(nnz);
    for (int32_t r = 0; r < M; ++r)
        for (int32_t p = rowptr[r]; p < rowptr[r + 1]; ++p)
            keys.push_back((int64_t)(r / kTile) * tiles_c + colind[p] / kTile);
    std::sort(keys.begin(), keys.end());
    std::vector<float> fills;
    int64_t cand_nnz = 0;
    int32_t cand_tiles = 0;
    for (size_t i = 0; i < keys.size();) {
        size_t j = i;
        while (j < keys.size() && keys[j] == keys[i]) ++j;
        const float fill = static_cast<float>(j - i) / static_cast<float>(kTile * kTile);
        fills.push_back(fill);
        if (fill >= kTcFill) {
            cand_nnz += static_cast<int64_t>(j - i);
            ++cand_tiles;
        }
        i = j;
    }
    std::sort(fills.begin(), fills.end());
    const float fill_mean = mean_of(fills);
    double fill_var = 0.0;
    for (float x : fills) fill_var += (static_cast<double>(x) - fill_mean) * (static_cast<double>(x) - fill_mean);
    const size_t nt = fills.size();
    f.tile_fill_mean = fill_mean;
    f.tile_fill_median = fills[nt / 2];
    f.tile_fill_p90 = fills[std::min(nt - 1, nt * 9 / 10)];
    f.tile_fill_max = fills.back();
    f.tile_fill_variance = static_cast<float>(fill_var / static_cast<double>(nt));
    f.tile_occupancy = static_cast<float>(nt) / static_cast<float>(std::max<int64_t>(1, tiles_r * tiles_c));
    f.actual_nnz_coverage = static_cast<float>(cand_nnz) / fnnz;
    f.avg_nnz_per_tile = fnnz / static_cast<float>(nt);
    f.tc_candidate_tiles = cand_tiles;
    f.tc_candidate_ratio = static_cast<float>(cand_tiles) / static_cast<float>(nt);

    // 3. Locality of adjacent rows, natural and reordered.
    auto adjacent_mean = [&](auto row_at) {
        std::vector<float> sims;
        sims.reserve(M);
        for (int32_t i = 1; i < M; ++i) {
            const RowSig &a = rows[row_at(i - 1)], &b = rows[row_at(i)];
            if (a.len > 0 && b.len > 0) sims.push_back(jaccard(a.sig, b.sig));
        }
        return mean_of(sims);
    };
    f.local_row_similarity_proxy = adjacent_mean([](int32_t i) { return i; });
    std::vector<int32_t> order(M);
    std::iota(order.begin(), order.end(), 0);
    const float fK = static_cast<float>(K);
    std::stable_sort(order.begin(), order.end(), [&](int32_t a, int32_t b) {
        const RowSig &x = rows[a], &y = rows[b];
        const int bx = static_cast<int>(x.centroid * 16.f / fK), by = static_cast<int>(y.centroid * 16.f / fK);
        if (bx != by) return bx < by;
        const int sx = x.len > 0 ? x.hi - x.lo + 1 : K, sy = y.len > 0 ? y.hi - y.lo + 1 : K;
        if (sx != sy) return sx < sy;
        return x.len > y.len;
    });
    f.reordered_locality_proxy = adjacent_mean([&](int32_t i) { return order[i]; });

    // 4. 16-row windows.
    std::vector<float> w_compact, w_sim, w_irreg;
    int64_t tc_nnz = 0, cuda_nnz = 0;
    int32_t irregular = 0;
    for (int32_t base = 0; base < M; base += kWindow) {
        const int32_t end = std::min(M, base + kWindow), h = end - base;
        int64_t wnnz = 0, wlong = 0;
        int32_t lo = K, hi = -1, wmax = 0, sim_n = 0;
        float sim_sum = 0.f;
        for (int32_t r = base; r < end; ++r) {
            const RowSig& x = rows[r];
            wnnz += x.len;
            wmax = std::max(wmax, x.len);
            if (x.len > 0) {
                lo = std::min(lo, x.lo);
                hi = std::max(hi, x.hi);
            }
            if (r > base && rows[r - 1].len > 0 && x.len > 0) {
                sim_sum += jaccard(rows[r - 1].sig, x.sig);
                ++sim_n;
            }
        }
        const float avg_len = static_cast<float>(wnnz) / static_cast<float>(std::max(1, h));
        const float long_len = std::max(32.f, 2.5f * avg_len);
        for (int32_t r = base; r < end; ++r)
            if (static_cast<float>(rows[r].len) >= long_len) wlong += rows[r].len;
        const int32_t span = hi >= lo ? hi - lo + 1 : K;
        const float compact = static_cast<float>(wnnz) / static_cast<float>(std::max(1, h * std::max(1, span)));
        const float sim = sim_n > 0 ? sim_sum / static_cast<float>(sim_n) : 0.f;
        const int32_t span16 = std::max(16, (span + 15) / 16 * 16);
        const float density = static_cast<float>(wnnz) / static_cast<float>(std::max(16, h * span16));
        const float compact_n = clamp01(compact * 6.f);
        const float density_n = clamp01(density * 10.f);
        const float uniform_n = clamp01(1.f - ratio_or_zero(static_cast<float>(wmax), 4.f * avg_len + 1.f));
        const float long_mass = ratio_or_zero(static_cast<float>(wlong), static_cast<float>(std::max<int64_t>(1, wnnz)));
        w_compact.push_back(compact);
        w_sim.push_back(sim);
        const float tc_score = 0.35f * compact_n + 0.30f * sim + 0.20f * density_n + 0.15f * uniform_n;
        const float irr_score = 0.40f * long_mass +
                                0.25f * clamp01(ratio_or_zero(static_cast<float>(wmax), avg_len + 1.f) / 6.f) +
                                0.20f * (1.f - compact_n) + 0.15f * (1.f - sim);
        w_irreg.push_back(irr_score);
        if (avg_len >= 8.f && tc_score >= 0.55f && irr_score < 0.45f) tc_nnz += wnnz;
        if (irr_score >= 0.50f || long_mass >= 0.20f) {
            cuda_nnz += wnnz;
            ++irregular;
        }
    }
    f.row_window_colspan_compactness = mean_of(w_compact);
    const float sim_mean = mean_of(w_sim), irr_mean = mean_of(w_irreg);

    // Composite proxies.
    f.tc_synergy_proxy = 0.35f * clamp01(f.tile_fill_mean / 0.20f) + 0.25f * f.tc_candidate_ratio +
                         0.20f * f.reordered_locality_proxy + 0.20f * f.row_window_colspan_compactness;
    f.locality_gain_proxy = clamp01(f.reordered_locality_proxy - f.local_row_similarity_proxy);
    const float ordered = clamp01(f.local_row_similarity_proxy * clamp01(f.row_window_colspan_compactness * 2.f));
    f.locality_selectivity_proxy = clamp01(f.locality_gain_proxy * (1.f - ordered));
    f.road_likeness_proxy = clamp01(f.local_row_similarity_proxy * clamp01(1.f - f.degree_cv / 0.35f) *
                                    clamp01(1.f - f.avg_nnz_per_row / 24.f) *
                                    clamp01(f.row_window_colspan_compactness / 0.25f));
    const float skew_branch = 0.45f * clamp01((f.skew_ratio - 2.0f) / 6.0f) + 0.30f * f.long_row_nnz_fraction +
                              0.15f * clamp01(f.top_1_row_nnz_fraction / 0.0020f) +
                              0.10f * clamp01(f.top_5_row_nnz_fraction / 0.0100f);
    const float n_scale = clamp01((static_cast<float>(N) - 128.f) / 384.f);
    const float dense_branch = clamp01(f.avg_nnz_per_row / 192.f) * (0.35f + 0.65f * n_scale);
    f.row_split_affinity_proxy = clamp01(std::max(skew_branch, dense_branch));
    f.estimated_tc_partition_ratio = clamp01(static_cast<float>(tc_nnz) / fnnz);
    f.estimated_cuda_partition_ratio = clamp01(static_cast<float>(cuda_nnz) / fnnz);
    f.irregular_window_fraction =
        static_cast<float>(irregular) / static_cast<float>(std::max(1, (M + kWindow - 1) / kWindow));
    const float tcr = f.estimated_tc_partition_ratio, cur = f.estimated_cuda_partition_ratio;
    const float balance = ratio_or_zero(2.f * std::min(tcr, cur), tcr + cur + 1e-6f);
    f.mixedness_proxy = clamp01(balance * clamp01((tcr + cur) / 0.60f));
    f.tc_granularity_proxy = 0.55f * clamp01(f.avg_nnz_per_row / 64.f) +
                             0.45f * clamp01((1.f - f.long_row_fraction) + 0.5f * f.locality_selectivity_proxy);
    f.redundancy_risk_proxy = clamp01(0.45f * f.long_row_nnz_fraction +
                                      0.30f * (1.f - f.row_window_colspan_compactness) +
                                      0.15f * (1.f - sim_mean) + 0.10f * irr_mean);
    return RA_OK;
}
