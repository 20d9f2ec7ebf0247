// router.cpp — routing features (shared finalisation) and the seven-rule router.
//
// Compiled with -ffp-contract=off: every floating-point step below must be the
// same IEEE operation sequence as the Python mirror (ra_spmm/router.py), so
// the two make bit-identical decisions.
//
// Reference: compute_production_router_features, router/router_features.cpp:79-111;
//            compute_production_router_features_gpu, router/router_features_cuda.cu:51-92;
//            route_dispatch deployed block, router/router_dispatch.cpp:979-1110;
//            compute_feasible, router/router_dispatch.cpp:107-464.
#include <cmath>
#include <cstring>

#include "ra_internal.hpp"

namespace {

// Threshold table of the rule tree.  Field names follow the rule they gate.
struct RouterTable {
    float cv_extreme;        // rule 1: cv >= -> ZERO_OVERHEAD_CSR
    float cv_uniform;        // rule 2: cv <
    float d_ultralow;        //   d <
    int   n_ultralow_csr;    //   N <= -> CSR_DIRECT
    float cv_comm_lo;        //   cv >=
    float d_comm;            //   d <
    int   n_comm_csr;        //   N <= -> CSR_DIRECT
    float cv_skewed;         // rule 3: cv >=
    int   m_skewed_large;    //   M >= -> COMMUNITY_TC else SEGMENT_HYBRID
    float d_dense;           // rule 4: d >=
    int   m_small;           // rule 5: M <
    float d_small_dense;     //   d >=
    int   n_small_narrow;    //   N < -> CUSPARSE (baseline CSR)
    int   n_small_mid;       //   N < -> SEGMENT_HYBRID
    float d_heavy;           // rule 6: d >=
    float cv_heavy;          //   cv >=
    float d_web;             // rule 7: d <
    float cv_web_lo;         //   cv in [lo, hi]
    float cv_web_hi;
    int   m_web;             //   M >=
    float cv_gate_csr;       // tile gated: cv < -> CSR_DIRECT else ZERO_OVERHEAD_CSR
    double plan_s_per_nnz;   // tile gate: est build seconds per nnz (d*M)
    double plan_budget_s;    //   withheld above this
    float d_fp32_route;      // precision: d < -> FP32 route
    int   m_fp32_small;      //   or (M <= and
    float d_fp32_small;      //       d <)
    // MI355X-only knobs (inert in the reference table).
    int   fp32_route_csr;    // FP32-route picks go to the CSR family instead
    float zo_min_cv;         // CSR_DIRECT picks with cv >= this go to ZERO_OVERHEAD_CSR
    int   n_uniform_csr;     // rule 2, remaining uniform graphs: N <= -> CSR_DIRECT
    int   skewed_path;       // rule 3: path, or -1 for the split on M
    int   small_dense_path;  // rule 5: path, or -1 for the split on N
    int   heavy_path;        // rule 6 path
    int   web_path;          // rule 7 path
    int   web_fp32;          //   rule 7 forces the FP32 route
    float fp32_small_max_cv; // the small-graph FP32 condition applies only when cv <
};

// Published thresholds (router/router_dispatch.cpp:1004-1094, ra_router_eval.py:37-124).
constexpr RouterTable kReference = {
    5.0f, 0.7f, 4.5f, 256, 0.2f, 7.0f, 128, 3.0f, 250000, 40.0f, 20000, 25.0f, 96, 256,
    25.0f, 1.8f, 9.0f, 1.10f, 1.45f, 250000, 1.5f, 2e-8, 20.0, 5.0f, 25000, 9.0f,
    0, 1e30f, 0, -1, -1, RA_PATH_COMMUNITY_TC, RA_PATH_COMMUNITY_TC, 1, 1e30f};

// MI355X calibration.  The structure of the tree is unchanged; each knob is
// set from one measured sweep on gfx950 (bench.py --sweep regimes,C1,...,C5
// at N = 64, 128, 256, 512: 27 graphs, 108 points, at least one graph in every
// branch of the tree; router_eval.py scores a table against it).  On that
// sweep this table picks the fastest path on 67 of 108 points (the reference
// table: 38) at a router/oracle geomean of 0.943 (0.865):
//  - tile gate: the device tile build runs at 1.0-1.9e-10 s per nnz, plus
//    ~3e-10 s per nnz to upload a host CSR, so the estimate is 1e-9 s per nnz
//    with the same 20 s budget;
//  - FP32-route tile picks go to the CSR family, which needs no plan (the
//    FP32 tile route runs the same CSR kernels on the plan's stored values);
//  - a CSR_DIRECT pick on skewed rows (cv >= 1.5) goes to ZERO_OVERHEAD_CSR
//    (one lane group per hub row is 6.6x slower on config 2);
//  - rule 2, uniform graphs of d >= 7 at N <= 64 go to CSR_DIRECT (faster on
//    2 of the 3 such graphs);
//  - rules 3, 5 and 6 pick SEGMENT_HYBRID: the fastest path on 26 of the 32
//    points of those regions and within 19% on the rest (rule 5's guardrail
//    pick, the baseline kernel, was 5-6x slower; rule 6's COMMUNITY_TC 1.5x
//    slower on a graph with local columns; rule 3's split on M gave
//    COMMUNITY_TC to large graphs, where it was 0-40% slower);
//  - rule 7 picks TC_DIRECT without forcing the FP32 route (fastest on 5 of
//    8 points; COMMUNITY_TC on the FP32 route meant CSR_DIRECT here, 1.45-1.5x
//    slower at N = 64), and the small-graph FP32 condition (M <= 25000,
//    d < 9) holds only for uniform rows (cv < 0.7): on a small graph of cv 1
//    the 16-bit tiles beat CSR_DIRECT 1.3-1.7x.
//  Rule 1 keeps the reference's pick, ZERO_OVERHEAD_CSR (the exact fp32
//  path), although the 16-bit COMMUNITY_TC is 1.3-1.7x faster there and
//  passes the harness's gate: the rule carries the fp32 benchmark configs 2
//  and 5, and the bf16x3 split that would keep ~2^-16 accuracy measured
//  slower than ZERO_OVERHEAD_CSR.
constexpr RouterTable kMI355X = {
    5.0f, 0.7f, 4.5f, 256, 0.2f, 7.0f, 128, 3.0f, 250000, 40.0f, 20000, 25.0f, 96, 256,
    25.0f, 1.8f, 9.0f, 1.10f, 1.45f, 250000, 1.5f, 1e-9, 20.0, 5.0f, 25000, 9.0f,
    1, 1.5f, 64, RA_PATH_SEGMENT_HYBRID, RA_PATH_SEGMENT_HYBRID, RA_PATH_SEGMENT_HYBRID,
    RA_PATH_TC_DIRECT, 0, 0.7f};

// Decision reason of a rule whose path comes from the table: "<path>_<rule>".
const char* table_reason(int p, int rule) {
    static const char* const kReasons[4][5] = {
        // CSR_DIRECT, ZERO_OVERHEAD_CSR, TC_DIRECT, COMMUNITY_TC, SEGMENT_HYBRID
        {"csr_direct_skewed", "zero_overhead_skewed", "tc_direct_skewed", "community_tc_skewed",
         "segment_hybrid_skewed"},
        {"csr_direct_small_dense", "zero_overhead_small_dense", "tc_direct_small_dense",
         "community_tc_small_dense", "segment_hybrid_small_dense_allN"},
        {"csr_direct_heavy_mixed", "zero_overhead_heavy_mixed", "tc_direct_heavy_mixed",
         "community_tc_heavy_mixed", "segment_hybrid_heavy_mixed"},
        {"csr_direct_web_locality", "zero_overhead_web_locality", "tc_direct_web_locality",
         "community_tc_web_locality", "segment_hybrid_web_locality"}};
    const int r = rule == 3 ? 0 : rule == 5 ? 1 : rule == 6 ? 2 : 3;
    switch (p) {
        case RA_PATH_CSR_DIRECT: return kReasons[r][0];
        case RA_PATH_ZERO_OVERHEAD_CSR: return kReasons[r][1];
        case RA_PATH_TC_DIRECT: return kReasons[r][2];
        case RA_PATH_COMMUNITY_TC: return kReasons[r][3];
        case RA_PATH_SEGMENT_HYBRID: return kReasons[r][4];
        default: return "table_path";
    }
}

bool tile_family(int p) {
    return p == RA_PATH_TC_DIRECT || p == RA_PATH_COMMUNITY_TC || p == RA_PATH_SEGMENT_HYBRID;
}

bool in_main_portfolio(int p) {
    // router/router_dispatch.cpp:50-72
    switch (p) {
        case RA_PATH_CSR_DIRECT: case RA_PATH_ROW_SPLIT_CUDA: case RA_PATH_TC_REORDERED:
        case RA_PATH_HYBRID_TC_CUDA: case RA_PATH_CUSPARSE: case RA_PATH_RODE_ENHANCED:
        case RA_PATH_VECTORIZED_COARSE: case RA_PATH_LOCALITY_TILED: case RA_PATH_TC_DIRECT:
        case RA_PATH_COMMUNITY_TC: case RA_PATH_ZERO_OVERHEAD_CSR: case RA_PATH_SEGMENT_HYBRID:
            return true;
        default:
            return false;
    }
}

// Kernels this engine implements.  Legacy/ablation paths of the reference are
// reported infeasible (they are not built on MI355X).
bool implemented(int p) {
    return p == RA_PATH_CSR_DIRECT || p == RA_PATH_CUSPARSE || p == RA_PATH_TC_DIRECT ||
           p == RA_PATH_COMMUNITY_TC || p == RA_PATH_ZERO_OVERHEAD_CSR ||
           p == RA_PATH_SEGMENT_HYBRID;
}

}  // namespace

extern "C" {

ra_status ra_features_from_moments(int32_t M, int32_t K, int32_t N, int64_t nnz,
                                   int64_t sum_deg_sq, int32_t max_deg, int64_t empty_rows,
                                   ra_features* out) {
    if (!out) return ra::fail(RA_ERR_INVALID_ARGUMENT, "features: out is NULL");
    std::memset(out, 0, sizeof(*out));
    out->M = M;
    out->K = K;
    out->N = N;
    // No features for an empty shape (router/router_features_cuda.cu:57-59).
    if (M <= 0 || K <= 0) return RA_OK;
    out->nnz = nnz;
    out->sum_deg_sq = sum_deg_sq;
    out->max_deg = max_deg;
    out->empty_rows = empty_rows;
    // Moment form of router/router_features_cuda.cu:83-91 on exact integers.
    const double avg = static_cast<double>(nnz) / static_cast<double>(M);
    double var = static_cast<double>(sum_deg_sq) / static_cast<double>(M) - avg * avg;
    if (var < 0.0) var = 0.0;
    const double std_dev = std::sqrt(var);
    out->avg = avg;
    out->std_dev = std_dev;
    out->avg_nnz_per_row = static_cast<float>(avg);
    out->std_nnz_per_row = static_cast<float>(std_dev);
    out->degree_cv = (avg > 1e-6) ? static_cast<float>(std_dev / avg) : 0.0f;
    out->max_to_mean_ratio = (avg > 1e-6) ? static_cast<float>(max_deg / avg) : 0.0f;
    return RA_OK;
}

ra_status ra_features_host(const int32_t* h_rowptr, int32_t M, int32_t K, int32_t N,
                           ra_features* out) {
    if (!out) return ra::fail(RA_ERR_INVALID_ARGUMENT, "features: out is NULL");
    if (!h_rowptr && M > 0) return ra::fail(RA_ERR_INVALID_ARGUMENT, "features: rowptr is NULL");
    if (M < 0) return ra::fail(RA_ERR_INVALID_ARGUMENT, "features: M < 0");
    std::memset(out, 0, sizeof(*out));
    out->M = M;
    out->K = K;
    out->N = N;
    // Two-pass form of router/router_features.cpp:79-111: no features for an
    // empty shape (:86-88); avg only when nnz <= 0 (:94-96); otherwise
    // sigma^2 = sum (d - avg)^2 / M, summed in ascending row order.
    if (M == 0 || K <= 0) return RA_OK;
    int64_t s2 = 0, empty = 0;
    int32_t mx = 0;
    for (int32_t r = 0; r < M; ++r) {
        const int64_t d = static_cast<int64_t>(h_rowptr[r + 1]) - h_rowptr[r];
        if (d < 0) return ra::fail(RA_ERR_INVALID_ARGUMENT, "features: rowptr not monotone");
        s2 += d * d;
        if (d > mx) mx = static_cast<int32_t>(d);
        empty += (d == 0);
    }
    const int64_t nnz = static_cast<int64_t>(h_rowptr[M]) - h_rowptr[0];
    out->nnz = nnz;
    out->sum_deg_sq = s2;
    out->max_deg = mx;
    out->empty_rows = empty;
    const double avg = static_cast<double>(nnz) / static_cast<double>(M);
    out->avg = avg;
    out->avg_nnz_per_row = static_cast<float>(avg);
    if (nnz <= 0) return RA_OK;
    double dev2 = 0.0;
    for (int32_t r = 0; r < M; ++r) {
        const double delta = static_cast<double>(h_rowptr[r + 1] - h_rowptr[r]) - avg;
        dev2 += delta * delta;
    }
    const double std_dev = std::sqrt(dev2 / static_cast<double>(M));
    out->std_dev = std_dev;
    out->std_nnz_per_row = static_cast<float>(std_dev);
    out->degree_cv = (avg > 1e-6) ? static_cast<float>(std_dev / avg) : 0.0f;
    out->max_to_mean_ratio = (avg > 1e-6) ? static_cast<float>(mx / avg) : 0.0f;
    return RA_OK;
}

ra_status ra_route_dispatch(const ra_features* f, int32_t portfolio, int32_t table,
                            ra_route* out) {
    if (!f || !out) return ra::fail(RA_ERR_INVALID_ARGUMENT, "route: NULL argument");
    if (table != RA_TABLE_REFERENCE && table != RA_TABLE_MI355X)
        return ra::fail(RA_ERR_INVALID_ARGUMENT, "route: unknown threshold table");
    const RouterTable& T = (table == RA_TABLE_REFERENCE) ? kReference : kMI355X;
    std::memset(out, 0, sizeof(*out));

    const float d = f->avg_nnz_per_row;
    const float cv = f->degree_cv;
    const int N = f->N;
    const int M = f->M;

    // Feasibility (router/router_dispatch.cpp:107-464 restricted to the MAIN
    // production features): tile families need N >= 16.
    for (int p = 0; p < RA_PATH_COUNT; ++p) {
        bool ok = true;
        int8_t code = RA_REJECT_CHOSEN;
        if (portfolio == RA_PORTFOLIO_MAIN && !in_main_portfolio(p)) {
            ok = false;
            code = RA_REJECT_NOT_IN_PORTFOLIO;
        } else if (!implemented(p)) {
            ok = false;
            code = RA_REJECT_NOT_FEASIBLE;
        } else if (tile_family(p) && N < 16) {
            ok = false;
            code = RA_REJECT_MARGIN_TOO_SMALL;
        }
        out->feasible[p] = ok ? 1 : 0;
        out->rejection_code[p] = code;
    }

    int choice = out->feasible[RA_PATH_TC_DIRECT] ? RA_PATH_TC_DIRECT : RA_PATH_CSR_DIRECT;
    const char* reason = out->feasible[RA_PATH_TC_DIRECT] ? "tc_direct_default_winner"
                                                           : "csr_direct_tc_direct_infeasible";
    float risk = 0.05f;
    bool fp32_route = false;
    int rule = 0;

    // Preprocessing-aware tile gate (router/router_dispatch.cpp:1006-1013).
    const double est_plan_s = T.plan_s_per_nnz * static_cast<double>(d) * static_cast<double>(M);
    const bool tile_ok = out->feasible[RA_PATH_TC_DIRECT] && est_plan_s <= T.plan_budget_s;

    auto csr_by_skew = [&](const char* csr_reason, const char* zo_reason) {
        if (cv < T.cv_gate_csr) {
            choice = RA_PATH_CSR_DIRECT;
            reason = csr_reason;
            risk = 0.05f;
        } else {
            choice = RA_PATH_ZERO_OVERHEAD_CSR;
            reason = zo_reason;
            risk = 0.06f;
        }
    };
    auto pick_tile = [&](int p, const char* why, bool force_fp32) {
        if (tile_ok && out->feasible[p]) {
            const bool want_fp32 =
                force_fp32 || (d < T.d_fp32_route || (M <= T.m_fp32_small && d < T.d_fp32_small &&
                                                      cv < T.fp32_small_max_cv));
            if (want_fp32 && T.fp32_route_csr) {
                csr_by_skew("csr_direct_over_fp32_tile", "zero_overhead_over_fp32_tile");
                return;
            }
            choice = p;
            reason = why;
            risk = 0.06f;
            fp32_route = want_fp32;
        } else {
            csr_by_skew("csr_direct_tile_gated", "zero_overhead_tile_gated");
        }
    };

    // A rule's path from the table: a tile family goes through the tile gate
    // and the precision rule, a CSR family is taken as is.
    auto pick_table = [&](int p, const char* why) {
        if (tile_family(p)) {
            pick_tile(p, why, false);
        } else {
            choice = p;
            reason = why;
            risk = p == RA_PATH_ZERO_OVERHEAD_CSR ? 0.06f : 0.05f;
        }
    };

    if (cv >= T.cv_extreme) {
        rule = 1;
        choice = RA_PATH_ZERO_OVERHEAD_CSR;
        reason = "zero_overhead_extreme_skew";
        risk = 0.06f;
    } else if (cv < T.cv_uniform) {
        rule = 2;
        if (d < T.d_ultralow) {
            if (N <= T.n_ultralow_csr) {
                choice = RA_PATH_CSR_DIRECT;
                reason = "csr_direct_uniform_ultralow_d";
                risk = 0.05f;
            } else {
                pick_tile(RA_PATH_TC_DIRECT, "tc_direct_uniform_wideN", false);
            }
        } else if (cv >= T.cv_comm_lo && d < T.d_comm) {
            if (N <= T.n_comm_csr) {
                choice = RA_PATH_CSR_DIRECT;
                reason = "csr_direct_synth_community";
                risk = 0.05f;
            } else {
                pick_tile(RA_PATH_TC_DIRECT, "tc_direct_community_wideN", true);
            }
        } else if (N <= T.n_uniform_csr) {
            choice = RA_PATH_CSR_DIRECT;
            reason = "csr_direct_uniform_narrowN";
            risk = 0.05f;
        } else {
            pick_tile(RA_PATH_TC_DIRECT, "tc_direct_uniform", false);
        }
    } else if (cv >= T.cv_skewed) {
        rule = 3;
        if (T.skewed_path >= 0) {
            pick_table(T.skewed_path, table_reason(T.skewed_path, 3));
        } else if (M >= T.m_skewed_large) {
            pick_tile(RA_PATH_COMMUNITY_TC, "community_tc_skewed_large", false);
        } else {
            pick_tile(RA_PATH_SEGMENT_HYBRID, "segment_hybrid_skewed_medium", false);
        }
    } else if (d >= T.d_dense) {
        rule = 4;
        pick_tile(RA_PATH_COMMUNITY_TC, "community_tc_dense_rows", false);
    } else if (M < T.m_small && d >= T.d_small_dense) {
        rule = 5;
        if (T.small_dense_path >= 0) {
            pick_table(T.small_dense_path, table_reason(T.small_dense_path, 5));
        } else if (N < T.n_small_narrow) {
            choice = RA_PATH_CUSPARSE;
            reason = "cusparse_small_dense_narrowN";
            risk = 0.05f;
        } else if (N < T.n_small_mid) {
            pick_tile(RA_PATH_SEGMENT_HYBRID, "segment_hybrid_small_dense", false);
        } else {
            pick_tile(RA_PATH_COMMUNITY_TC, "community_tc_small_dense_wideN", false);
        }
    } else if (d >= T.d_heavy && cv >= T.cv_heavy) {
        rule = 6;
        pick_table(T.heavy_path, table_reason(T.heavy_path, 6));
    } else if (d < T.d_web && cv >= T.cv_web_lo && cv <= T.cv_web_hi && M >= T.m_web) {
        rule = 7;
        if (tile_family(T.web_path)) pick_tile(T.web_path, table_reason(T.web_path, 7), T.web_fp32 != 0);
        else pick_table(T.web_path, table_reason(T.web_path, 7));
    } else {
        rule = 8;
        pick_tile(RA_PATH_TC_DIRECT, "tc_direct_default", false);
    }

    // MI355X: a CSR_DIRECT pick on a skewed row distribution serialises hubs
    // on one lane group; the hub-chunked kernel is the safe CSR choice.
    if (choice == RA_PATH_CSR_DIRECT && cv >= T.zo_min_cv) {
        choice = RA_PATH_ZERO_OVERHEAD_CSR;
        reason = "zero_overhead_skewed_csr";
        risk = 0.06f;
    }

    out->chosen_path = choice;
    out->use_tf32 = (tile_family(choice) && fp32_route) ? 1 : 0;
    out->rule = rule;
    out->tile_ok = tile_ok ? 1 : 0;
    out->estimated_risk = risk;
    out->est_plan_s = est_plan_s;
    std::strncpy(out->decision_reason, reason, sizeof(out->decision_reason) - 1);
    // Every other feasible path lost to the chosen one
    // (router/router_dispatch.cpp:960-966 / mark_choice :482-499).
    for (int p = 0; p < RA_PATH_COUNT; ++p) {
        if (out->feasible[p] && p != choice) out->rejection_code[p] = RA_REJECT_NOT_STRONG_ENOUGH;
    }
    out->rejection_code[choice] = RA_REJECT_CHOSEN;
    return RA_OK;
}

}  // extern "C"
