// torch_binding.cpp — the `ra_spmm` extension surface over the C ABI.
//
// Mirrors the deployed subset of the reference pybind module
// (bindings/ra_bindings.cpp:2318-2899): same function names, keyword names,
// argument meaning, plan classes and RuntimeError behaviour.  Everything here
// is marshalling: tensor checks, C allocation, plan ownership and dicts.  All
// compute goes through include/ra_spmm.h; launches use the current torch
// stream (the reference used the legacy default stream for its CSR kernels and
// the current stream for its tile kernels, bindings/ra_bindings.cpp:2164).
#include <torch/extension.h>
#include <c10/hip/HIPStream.h>

#include <ATen/Parallel.h>
#include <hip/hip_runtime_api.h>

#include <chrono>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>

#include "../../include/ra_spmm.h"

namespace {

ra_stream_t current_stream() {
    return reinterpret_cast<ra_stream_t>(c10::hip::getCurrentHIPStream().stream());
}

void check(ra_status s, const char* what) {
    TORCH_CHECK(s == RA_OK, what, " failed: ", ra_status_string(s), ": ", ra_last_error());
}

// bindings/ra_bindings.cpp:288-306
void check_gpu_tensor(const torch::Tensor& t, const char* name) {
    TORCH_CHECK(t.is_cuda(), name, " must be a CUDA tensor");
    TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
}
void check_dense_float(const torch::Tensor& t, const char* name) {
    check_gpu_tensor(t, name);
    TORCH_CHECK(t.scalar_type() == torch::kFloat32, name, " must be float32");
    TORCH_CHECK(t.dim() == 2, name, " must be 2-D");
}
void check_csr(const torch::Tensor& rowptr, const torch::Tensor& colind, const torch::Tensor& vals) {
    check_gpu_tensor(rowptr, "rowptr");
    check_gpu_tensor(colind, "colind");
    check_gpu_tensor(vals, "vals");
    TORCH_CHECK(rowptr.scalar_type() == torch::kInt32, "rowptr must be int32");
    TORCH_CHECK(colind.scalar_type() == torch::kInt32, "colind must be int32");
    TORCH_CHECK(vals.scalar_type() == torch::kFloat32, "vals must be float32");
    TORCH_CHECK(rowptr.dim() == 1 && rowptr.numel() >= 1, "rowptr must be 1-D with M+1 entries");
}
void check_same_device(const torch::Tensor& a, const torch::Tensor& b) {
    TORCH_CHECK(a.device() == b.device(), "tensors must be on the same device");
}
// Plans hold device memory of the GPU they were built on.
void check_plan_device(int plan_device, const torch::Tensor& B) {
    TORCH_CHECK(B.device().index() == plan_device, "the plan was built on cuda:", plan_device, ", B is on ",
                B.device());
}

// Host tensor -> new device tensor of `dtype` on the current stream.  Pageable
// tensors of 1 MiB and more go through two pinned 16 MiB staging buffers: the
// (multi-threaded) host copy of chunk i+1 overlaps the DMA of chunk i, which
// moves 128 MB in ~2.7 ms against ~4.9 ms for a plain pageable copy.  The
// staging buffers are allocated once per process and shared by all devices;
// each buffer is reused only after the copy that last read it (on whichever
// device) has completed.  The source may be freed as soon as this returns.
torch::Tensor upload(const torch::Tensor& t, torch::ScalarType dtype, const torch::Device& dev) {
    if (t.is_cuda()) return t.to(dev, dtype).contiguous();
    const torch::Tensor h = t.contiguous().to(dtype);
    constexpr int64_t kStage = int64_t{16} << 20;
    const int64_t bytes = h.numel() * static_cast<int64_t>(h.element_size());
    if (bytes < (int64_t{1} << 20)) return h.to(dev);
    auto out = torch::empty(h.sizes(), h.options().device(dev));
    static std::mutex mu;
    static void* stage[2] = {nullptr, nullptr};
    static hipEvent_t done[64][2] = {};
    static int last_dev[2] = {-1, -1};  // device whose copy last read each buffer
    std::lock_guard<std::mutex> lock(mu);
    const int di = dev.index();
    TORCH_CHECK(di >= 0 && di < 64, "upload: device index out of range");
    for (int k = 0; k < 2; ++k) {
        if (!stage[k]) TORCH_CHECK(hipHostMalloc(&stage[k], kStage, hipHostMallocNonCoherent) == hipSuccess,
                                   "upload: pinned staging allocation failed");
        if (!done[di][k])
            TORCH_CHECK(hipEventCreateWithFlags(&done[di][k], hipEventDisableTiming) == hipSuccess,
                        "upload: event creation failed");
    }
    hipStream_t st = c10::hip::getCurrentHIPStream(di).stream();
    const char* src = static_cast<const char*>(h.data_ptr());
    char* dst = static_cast<char*>(out.data_ptr());
    int k = 0;
    for (int64_t off = 0; off < bytes; off += kStage, k ^= 1) {
        const int64_t len = std::min(kStage, bytes - off);
        if (last_dev[k] >= 0)
            TORCH_CHECK(hipEventSynchronize(done[last_dev[k]][k]) == hipSuccess, "upload: staging wait failed");
        char* buf = static_cast<char*>(stage[k]);
        torch::from_blob(buf, {len}, torch::TensorOptions().dtype(torch::kUInt8))
            .copy_(torch::from_blob(const_cast<char*>(src) + off, {len}, torch::TensorOptions().dtype(torch::kUInt8)));
        TORCH_CHECK(hipMemcpyAsync(dst + off, buf, len, hipMemcpyHostToDevice, st) == hipSuccess,
                    "upload: copy failed");
        TORCH_CHECK(hipEventRecord(done[di][k], st) == hipSuccess, "upload: event record failed");
        last_dev[k] = di;
    }
    return out;
}

torch::Tensor host_i32(const torch::Tensor& t) { return t.cpu().contiguous().to(torch::kInt32); }
torch::Tensor host_f32(const torch::Tensor& t) { return t.cpu().contiguous().to(torch::kFloat32); }

// ------------------------------------------------------------ CSR_DIRECT
torch::Tensor spmm_csr_direct(torch::Tensor rowptr, torch::Tensor colind, torch::Tensor vals,
                              torch::Tensor B) {
    check_csr(rowptr, colind, vals);
    check_dense_float(B, "B");
    check_same_device(rowptr, B);
    const c10::DeviceGuard guard(B.device());
    const int M = static_cast<int>(rowptr.size(0)) - 1;
    const int K = static_cast<int>(B.size(0));
    const int N = static_cast<int>(B.size(1));
    auto C = torch::empty({M, N}, B.options());
    check(ra_spmm_csr_direct(rowptr.data_ptr<int32_t>(), colind.data_ptr<int32_t>(),
                             vals.data_ptr<float>(), B.data_ptr<float>(), C.data_ptr<float>(), M,
                             K, N, colind.numel(), current_stream()),
          "spmm_csr_direct");
    return C;
}

// --------------------------------------------------- baseline (guardrail)
torch::Tensor spmm_csr_baseline(torch::Tensor rowptr, torch::Tensor colind, torch::Tensor vals,
                                torch::Tensor B) {
    check_csr(rowptr, colind, vals);
    check_dense_float(B, "B");
    check_same_device(rowptr, B);
    const c10::DeviceGuard guard(B.device());
    const int M = static_cast<int>(rowptr.size(0)) - 1;
    const int K = static_cast<int>(B.size(0));
    const int N = static_cast<int>(B.size(1));
    auto C = torch::empty({M, N}, B.options());
    check(ra_spmm_csr_baseline(rowptr.data_ptr<int32_t>(), colind.data_ptr<int32_t>(),
                               vals.data_ptr<float>(), B.data_ptr<float>(), C.data_ptr<float>(),
                               M, K, N, colind.numel(), current_stream()),
          "spmm_csr_baseline");
    return C;
}

// Precision-matched baseline on fp16 A values and fp16 B (already converted by
// the caller; spmm_cusparse_fp16 in ra_spmm/dispatch.py converts first).
torch::Tensor spmm_csr_baseline_f16(torch::Tensor rowptr, torch::Tensor colind, torch::Tensor vals_h,
                                    torch::Tensor B_h) {
    check_gpu_tensor(rowptr, "rowptr");
    check_gpu_tensor(colind, "colind");
    check_gpu_tensor(vals_h, "vals");
    check_gpu_tensor(B_h, "B");
    TORCH_CHECK(rowptr.scalar_type() == torch::kInt32 && colind.scalar_type() == torch::kInt32,
                "rowptr/colind must be int32");
    TORCH_CHECK(vals_h.scalar_type() == torch::kFloat16 && B_h.scalar_type() == torch::kFloat16,
                "vals and B must be float16");
    TORCH_CHECK(rowptr.dim() == 1 && rowptr.numel() >= 1 && B_h.dim() == 2, "bad shapes");
    check_same_device(rowptr, B_h);
    const c10::DeviceGuard guard(B_h.device());
    const int M = static_cast<int>(rowptr.size(0)) - 1;
    const int K = static_cast<int>(B_h.size(0));
    const int N = static_cast<int>(B_h.size(1));
    auto C = torch::empty({M, N}, B_h.options().dtype(torch::kFloat32));
    check(ra_spmm_csr_baseline_f16(rowptr.data_ptr<int32_t>(), colind.data_ptr<int32_t>(),
                                   static_cast<const uint16_t*>(vals_h.data_ptr()),
                                   static_cast<const uint16_t*>(B_h.data_ptr()), C.data_ptr<float>(), M, K, N,
                                   colind.numel(), current_stream()),
          "spmm_csr_baseline_f16");
    return C;
}

// Reusable guardrail plan: keeps the CSR tensors and owns its output, like the
// reference CuSparsePlanWrapper (bindings/ra_bindings.cpp:620-631, 1025-1037):
// run_cusparse_plan writes into and returns the same C every call.
struct BaselinePlan {
    torch::Tensor rowptr, colind, vals, C;
    int64_t K = 0, N = 0;
};

std::shared_ptr<BaselinePlan> make_cusparse_plan(torch::Tensor rowptr, torch::Tensor colind,
                                                 torch::Tensor vals, torch::Tensor B) {
    check_csr(rowptr, colind, vals);
    check_dense_float(B, "B");
    check_same_device(rowptr, B);
    auto p = std::make_shared<BaselinePlan>();
    p->rowptr = rowptr;
    p->colind = colind;
    p->vals = vals;
    p->K = B.size(0);
    p->N = B.size(1);
    p->C = torch::zeros({rowptr.size(0) - 1, B.size(1)}, B.options());
    return p;
}

torch::Tensor run_cusparse_plan(std::shared_ptr<BaselinePlan> p, torch::Tensor B) {
    TORCH_CHECK(p, "Invalid cuSPARSE plan");
    check_dense_float(B, "B");
    TORCH_CHECK(B.size(0) == p->K && B.size(1) == p->N, "cuSPARSE plan expects B shape [", p->K,
                ", ", p->N, "], got [", B.size(0), ", ", B.size(1), "]");
    check_same_device(p->C, B);
    const c10::DeviceGuard guard(B.device());
    const int M = static_cast<int>(p->rowptr.size(0)) - 1;
    check(ra_spmm_csr_baseline(p->rowptr.data_ptr<int32_t>(), p->colind.data_ptr<int32_t>(),
                               p->vals.data_ptr<float>(), B.data_ptr<float>(),
                               p->C.data_ptr<float>(), M, static_cast<int>(p->K),
                               static_cast<int>(p->N), p->colind.numel(), current_stream()),
          "run_cusparse_plan");
    return p->C;
}

// ------------------------------------------------------------- features
ra_features features_of(const torch::Tensor& rowptr, int M, int K, int N, const char** backend) {
    ra_features f{};
    TORCH_CHECK(rowptr.numel() >= M + 1, "rowptr has fewer than M+1 entries");
    if (rowptr.is_cuda()) {
        TORCH_CHECK(rowptr.scalar_type() == torch::kInt32 && rowptr.is_contiguous(),
                    "device rowptr must be contiguous int32");
        const c10::DeviceGuard guard(rowptr.device());
        check(ra_features_device(rowptr.data_ptr<int32_t>(), M, K, N, current_stream(), &f),
              "features");
        *backend = "cuda_rowptr_moments";
    } else {
        auto rp = host_i32(rowptr);
        check(ra_features_host(rp.data_ptr<int32_t>(), M, K, N, &f), "features");
        *backend = "cpu_rowptr";  // bindings/ra_bindings.cpp:1726
    }
    return f;
}

int parse_table(const std::string& table) {
    if (table == "mi355x" || table == "MI355X") return RA_TABLE_MI355X;
    if (table == "reference" || table == "REFERENCE") return RA_TABLE_REFERENCE;
    TORCH_CHECK(false, "unknown router table '", table, "' (expected 'mi355x' or 'reference')");
    return -1;
}

pybind11::dict features_to_dict(const ra_features& f) {
    pybind11::dict d;
    d["M"] = f.M;
    d["K"] = f.K;
    d["N"] = f.N;
    d["nnz"] = f.nnz;
    d["sum_deg_sq"] = f.sum_deg_sq;
    d["max_deg"] = f.max_deg;
    d["empty_rows"] = f.empty_rows;
    d["avg"] = f.avg;
    d["std"] = f.std_dev;
    d["avg_nnz_per_row"] = f.avg_nnz_per_row;
    d["std_nnz_per_row"] = f.std_nnz_per_row;
    d["degree_cv"] = f.degree_cv;
    d["max_to_mean_ratio"] = f.max_to_mean_ratio;
    return d;
}

// Python strings of the plan dict, made once: a dict of 15 paths built from
// C strings costs ~5 us per routing call, most of it in string creation.
// Deliberately leaked, so no destructor runs after the interpreter is gone.
struct DictStrings {
    pybind11::str path[RA_PATH_COUNT];
    pybind11::str reject[RA_REJECT_UNKNOWN + 1];
    pybind11::str detail[RA_PATH_COUNT][3];  // N < 16, not built, not in portfolio
    pybind11::str empty;
    DictStrings() : empty("") {
        for (int p = 0; p < RA_PATH_COUNT; ++p) {
            const std::string name = ra_path_name(p);
            path[p] = pybind11::str(name);
            detail[p][0] = pybind11::str("N < 16");
            detail[p][1] = pybind11::str("not built for MI355X");
            detail[p][2] = pybind11::str(name + " not in selected portfolio");
        }
        for (int c = 0; c <= RA_REJECT_UNKNOWN; ++c) reject[c] = pybind11::str(ra_reject_name(c));
    }
};
const DictStrings& dict_strings() {
    static const DictStrings* s = new DictStrings();
    return *s;
}

// bindings/ra_bindings.cpp:634-718 (plan_to_dict) + :1717-1753 (make_router_plan_fn)
pybind11::dict route_to_dict(const ra_features& f, const ra_route& r, float ms) {
    const DictStrings& S = dict_strings();
    pybind11::dict d;
    d["chosen_path"] = S.path[r.chosen_path];
    d["use_tf32"] = static_cast<bool>(r.use_tf32);
    d["chosen_path_int"] = r.chosen_path;
    d["decision_reason"] = std::string(r.decision_reason);
    d["matched_rule"] = r.rule;
    d["estimated_risk"] = r.estimated_risk;
    d["planning_time_ms"] = ms;
    d["gate_margin_raw"] = 0.0f;
    d["gate_margin_norm"] = 0.0f;
    d["est_plan_s"] = r.est_plan_s;
    d["tile_ok"] = static_cast<bool>(r.tile_ok);
    d["path_count"] = static_cast<int>(RA_PATH_COUNT);
    pybind11::list names(static_cast<size_t>(RA_PATH_COUNT)), feas(static_cast<size_t>(RA_PATH_COUNT));
    pybind11::dict by_path, codes, details;
    for (int p = 0; p < RA_PATH_COUNT; ++p) {
        const pybind11::str& name = S.path[p];
        const bool ok = r.feasible[p] != 0;
        names[p] = name;
        feas[p] = pybind11::bool_(ok);
        by_path[name] = pybind11::bool_(ok);
        const int code = r.rejection_code[p];
        codes[name] = S.reject[(code < 0 || code > RA_REJECT_UNKNOWN) ? RA_REJECT_UNKNOWN : code];
        details[name] = code == RA_REJECT_MARGIN_TOO_SMALL  ? S.detail[p][0]
                        : code == RA_REJECT_NOT_FEASIBLE     ? S.detail[p][1]
                        : code == RA_REJECT_NOT_IN_PORTFOLIO ? S.detail[p][2]
                                                             : S.empty;
    }
    d["path_names"] = names;
    d["feasible"] = feas;
    d["feasible_by_path"] = by_path;
    d["rejection_codes"] = codes;
    d["rejection_details"] = details;
    pybind11::dict fv = features_to_dict(f);
    d["feature_values"] = fv;
    pybind11::dict scores;  // diagnostic-only in the reference (router_scores.cpp)
    for (const char* k : {"csr_direct", "csr_adaptive", "staged_reuse", "tc_sparse",
                          "row_split_cuda", "tc_reordered", "hybrid_tc_cuda", "cusparse"})
        scores[k] = 0.0f;
    d["scores"] = scores;
    return d;
}

// analyze_matrix_fn, bindings/ra_bindings.cpp:1993-2049 (host copy of the CSR).
ra_diag_features diag_of(torch::Tensor rowptr, torch::Tensor colind, int M, int K, int N) {
    auto rp = host_i32(rowptr);
    auto ci = host_i32(colind);
    TORCH_CHECK(rp.numel() >= M + 1, "rowptr has fewer than M+1 entries");
    ra_diag_features g{};
    check(ra_analyze_matrix(rp.data_ptr<int32_t>(), ci.numel() ? ci.data_ptr<int32_t>() : nullptr, M, K, N, &g),
          "analyze_matrix");
    return g;
}

void diag_into(pybind11::dict& d, const ra_diag_features& g) {
    d["avg_nnz_per_row"] = g.avg_nnz_per_row;
    d["std_nnz_per_row"] = g.std_nnz_per_row;
    d["degree_cv"] = g.degree_cv;
    d["max_to_mean_ratio"] = g.max_to_mean_ratio;
    d["frac_dense_rows"] = g.frac_dense_rows;
    d["skew_ratio"] = g.skew_ratio;
    d["long_row_fraction"] = g.long_row_fraction;
    d["long_row_nnz_fraction"] = g.long_row_nnz_fraction;
    d["top_1_row_nnz_fraction"] = g.top_1_row_nnz_fraction;
    d["top_5_row_nnz_fraction"] = g.top_5_row_nnz_fraction;
    d["tile_fill_mean"] = g.tile_fill_mean;
    d["tile_fill_median"] = g.tile_fill_median;
    d["tile_fill_p90"] = g.tile_fill_p90;
    d["tile_fill_max"] = g.tile_fill_max;
    d["tile_fill_variance"] = g.tile_fill_variance;
    d["tile_occupancy"] = g.tile_occupancy;
    d["actual_nnz_coverage"] = g.actual_nnz_coverage;
    d["avg_nnz_per_tile"] = g.avg_nnz_per_tile;
    d["row_window_colspan_compactness"] = g.row_window_colspan_compactness;
    d["local_row_similarity_proxy"] = g.local_row_similarity_proxy;
    d["reordered_locality_proxy"] = g.reordered_locality_proxy;
    d["locality_gain_proxy"] = g.locality_gain_proxy;
    d["locality_selectivity_proxy"] = g.locality_selectivity_proxy;
    d["road_likeness_proxy"] = g.road_likeness_proxy;
    d["row_split_affinity_proxy"] = g.row_split_affinity_proxy;
    d["mixedness_proxy"] = g.mixedness_proxy;
    d["tc_candidate_ratio"] = g.tc_candidate_ratio;
    d["tc_synergy_proxy"] = g.tc_synergy_proxy;
    d["estimated_tc_partition_ratio"] = g.estimated_tc_partition_ratio;
    d["estimated_cuda_partition_ratio"] = g.estimated_cuda_partition_ratio;
    d["irregular_window_fraction"] = g.irregular_window_fraction;
    d["tc_granularity_proxy"] = g.tc_granularity_proxy;
    d["redundancy_risk_proxy"] = g.redundancy_risk_proxy;
    d["tc_candidate_tiles"] = g.tc_candidate_tiles;
}

pybind11::dict analyze_matrix(torch::Tensor rowptr, torch::Tensor colind, int M, int K, int N) {
    const ra_diag_features g = diag_of(rowptr, colind, M, K, N);
    pybind11::dict d;
    diag_into(d, g);
    d["nnz"] = g.nnz;
    return d;
}

pybind11::dict make_router_plan(torch::Tensor rowptr, torch::Tensor colind, torch::Tensor vals,
                                int M, int K, int N, std::string portfolio, std::string table) {
    const auto t0 = std::chrono::high_resolution_clock::now();
    const int port = (portfolio == "FULL") ? RA_PORTFOLIO_FULL : RA_PORTFOLIO_MAIN;
    const char* backend = "";
    ra_features f = features_of(rowptr, M, K, N, &backend);
    ra_route r{};
    check(ra_route_dispatch(&f, port, parse_table(table), &r), "route_dispatch");
    const auto t1 = std::chrono::high_resolution_clock::now();
    pybind11::dict d =
        route_to_dict(f, r, std::chrono::duration<float, std::milli>(t1 - t0).count());
    d["feature_backend"] = backend;
    d["router_table"] = table;
    if (port == RA_PORTFOLIO_FULL) {
        // FULL plans carry the diagnostic features (router_dispatch.cpp:1123-1125);
        // the decision above read only M, d, CV and N, which they share.
        d["feature_set"] = "full";
        pybind11::dict fv = d["feature_values"];
        diag_into(fv, diag_of(rowptr, colind, M, K, N));
        d["planning_time_ms"] =
            std::chrono::duration<float, std::milli>(std::chrono::high_resolution_clock::now() - t0).count();
    } else {
        d["feature_set"] = "production_4";
    }
    (void)vals;
    return d;
}

pybind11::dict compute_features(torch::Tensor rowptr, int M, int K, int N) {
    const char* backend = "";
    ra_features f = features_of(rowptr, M, K, N, &backend);
    pybind11::dict d = features_to_dict(f);
    d["feature_backend"] = backend;
    return d;
}

pybind11::dict route_features(int M, int K, int N, int64_t nnz, int64_t sum_deg_sq, int max_deg,
                              int64_t empty_rows, std::string portfolio, std::string table) {
    ra_features f{};
    check(ra_features_from_moments(M, K, N, nnz, sum_deg_sq, max_deg, empty_rows, &f), "features");
    ra_route r{};
    check(ra_route_dispatch(&f, portfolio == "FULL" ? RA_PORTFOLIO_FULL : RA_PORTFOLIO_MAIN,
                            parse_table(table), &r),
          "route_dispatch");
    pybind11::dict d = route_to_dict(f, r, 0.f);
    d["router_table"] = table;
    return d;
}

// --------------------------------------------------- ZERO_OVERHEAD_CSR
struct ZOPlan {
    ra_zo_plan* plan = nullptr;
    ra_zo_info info{};
    bool valid = false;
    int device = -1;
    ~ZOPlan() { ra_zo_plan_destroy(plan); }
};

// build: "auto"/"gpu" bin on the device (a host rowptr is uploaded first),
// "host" runs the host binning loop.  Both give identical lists.
std::shared_ptr<ZOPlan> make_zero_overhead_plan(torch::Tensor rowptr_cpu, int M, int K,
                                                const std::string& build) {
    TORCH_CHECK(build == "auto" || build == "gpu" || build == "host",
                "build must be 'auto', 'gpu' or 'host'");
    TORCH_CHECK(rowptr_cpu.numel() >= M + 1, "rowptr has fewer than M+1 entries");
    auto w = std::make_shared<ZOPlan>();
    if (build == "host") {
        auto rp = host_i32(rowptr_cpu);
        w->device = c10::hip::current_device();
        check(ra_zo_plan_create(rp.data_ptr<int32_t>(), M, K, &w->plan), "make_zero_overhead_plan");
    } else {
        const auto dev = rowptr_cpu.is_cuda() ? rowptr_cpu.device()
                                              : torch::Device(torch::kCUDA, c10::hip::current_device());
        const c10::DeviceGuard guard(dev);
        w->device = dev.index();
        auto rp = upload(rowptr_cpu, torch::kInt32, dev);
        check(ra_zo_plan_create_device(rp.data_ptr<int32_t>(), M, K, current_stream(), &w->plan),
              "make_zero_overhead_plan");
    }
    check(ra_zo_plan_get_info(w->plan, &w->info), "zero_overhead info");
    w->valid = true;
    return w;
}

torch::Tensor run_zero_overhead_plan(std::shared_ptr<ZOPlan> w, torch::Tensor rowptr,
                                     torch::Tensor colind, torch::Tensor vals, torch::Tensor B) {
    check_gpu_tensor(rowptr, "rowptr");
    check_gpu_tensor(colind, "colind");
    check_gpu_tensor(vals, "vals");
    check_dense_float(B, "B");
    TORCH_CHECK(w && w->valid, "Invalid ZeroOverhead plan");
    TORCH_CHECK(B.size(0) >= w->info.K, "B has ", B.size(0), " rows; the plan was built for K = ", w->info.K);
    TORCH_CHECK(rowptr.numel() == w->info.M + 1, "rowptr has ", rowptr.numel(), " entries; the plan was built for M = ",
                w->info.M);
    TORCH_CHECK(rowptr.scalar_type() == torch::kInt32 && colind.scalar_type() == torch::kInt32 &&
                    vals.scalar_type() == torch::kFloat32,
                "rowptr/colind must be int32 and vals float32");
    check_same_device(rowptr, B);
    check_plan_device(w->device, B);
    const c10::DeviceGuard guard(B.device());
    const int M = w->info.M;
    const int N = static_cast<int>(B.size(1));
    auto C = torch::empty({M, N}, B.options());
    check(ra_zo_plan_run(w->plan, rowptr.data_ptr<int32_t>(), colind.data_ptr<int32_t>(),
                         vals.data_ptr<float>(), B.data_ptr<float>(), C.data_ptr<float>(), N,
                         current_stream()),
          "run_zero_overhead_plan");
    return C;
}

// Stage-timing hook: writes into a caller-provided C (see ra_zo_plan_run_stage).
void run_zero_overhead_plan_stage(std::shared_ptr<ZOPlan> w, torch::Tensor rowptr,
                                  torch::Tensor colind, torch::Tensor vals, torch::Tensor B,
                                  torch::Tensor C, int stage) {
    TORCH_CHECK(w && w->valid, "Invalid ZeroOverhead plan");
    check_csr(rowptr, colind, vals);
    check_dense_float(B, "B");
    check_dense_float(C, "C");
    check_same_device(rowptr, B);
    check_same_device(C, B);
    check_plan_device(w->device, B);
    const c10::DeviceGuard guard(B.device());
    TORCH_CHECK(B.size(0) >= w->info.K, "B has ", B.size(0), " rows; the plan was built for K = ", w->info.K);
    TORCH_CHECK(rowptr.numel() == w->info.M + 1, "rowptr does not match the plan's M");
    TORCH_CHECK(C.size(0) == w->info.M && C.size(1) == B.size(1), "C must be [M, N]");
    check(ra_zo_plan_run_stage(w->plan, rowptr.data_ptr<int32_t>(), colind.data_ptr<int32_t>(),
                               vals.data_ptr<float>(), B.data_ptr<float>(), C.data_ptr<float>(),
                               static_cast<int>(B.size(1)), stage, current_stream()),
          "run_zero_overhead_plan_stage");
}

// --------------------------------------------------------- tile family
struct TilePlan {
    ra_tile_plan* plan = nullptr;
    ra_tile_info info{};
    bool valid = false;
    int device = -1;
    ~TilePlan() { ra_tile_plan_destroy(plan); }
};

int parse_value_dtype(const std::string& s) {
    if (s == "fp16" || s == "float16" || s == "half") return RA_DTYPE_F16;
    if (s == "bf16" || s == "bfloat16") return RA_DTYPE_BF16;
    TORCH_CHECK(false, "value_dtype must be 'fp16' or 'bf16', got '", s, "'");
    return -1;
}

// build: "auto" (device build; host tensors are uploaded first), "gpu", or
// "host" (the host C++ builder).  Both produce the same plan bit for bit.
std::shared_ptr<TilePlan> make_tile_plan(int kind, torch::Tensor rowptr_cpu, torch::Tensor colind_cpu,
                                         torch::Tensor vals_cpu, int M, int K, int N,
                                         const std::string& value_dtype, const std::string& build,
                                         int rows_per_window, const char* what) {
    TORCH_CHECK(build != "host" || rows_per_window == 0 || rows_per_window == 8,
                "the host builder makes 8-row windows only");
    TORCH_CHECK(build == "auto" || build == "gpu" || build == "host",
                "build must be 'auto', 'gpu' or 'host'");
    TORCH_CHECK(rowptr_cpu.numel() >= M + 1, "rowptr has fewer than M+1 entries");
    auto w = std::make_shared<TilePlan>();
    const int vd = parse_value_dtype(value_dtype);
    if (build == "host") {
        auto rp = host_i32(rowptr_cpu);
        auto ci = host_i32(colind_cpu);
        auto vl = host_f32(vals_cpu);
        w->device = c10::hip::current_device();
        check(ra_tile_plan_create(kind, rp.data_ptr<int32_t>(), ci.data_ptr<int32_t>(),
                                  vl.data_ptr<float>(), M, K, N, vd, &w->plan),
              what);
    } else {
        const auto dev = rowptr_cpu.is_cuda() ? rowptr_cpu.device()
                                              : torch::Device(torch::kCUDA, c10::hip::current_device());
        const c10::DeviceGuard guard(dev);
        w->device = dev.index();
        auto rp = upload(rowptr_cpu, torch::kInt32, dev);
        auto ci = upload(colind_cpu, torch::kInt32, dev);
        auto vl = upload(vals_cpu, torch::kFloat32, dev);
        check(ra_tile_plan_create_device(kind, rp.data_ptr<int32_t>(), ci.data_ptr<int32_t>(),
                                         vl.data_ptr<float>(), M, K, N, vd, rows_per_window,
                                         current_stream(), &w->plan),
              what);
    }
    check(ra_tile_plan_get_info(w->plan, &w->info), "tile info");
    w->valid = true;
    return w;
}

torch::Tensor run_tile_plan(const std::shared_ptr<TilePlan>& w, const torch::Tensor& B, int route,
                            const char* what) {
    TORCH_CHECK(w && w->valid, "Invalid tile plan");
    check_gpu_tensor(B, "B");
    TORCH_CHECK(B.dim() == 2, "B must be 2-D");
    TORCH_CHECK(B.size(0) >= w->info.K, "B has ", B.size(0), " rows; the plan was built for K = ", w->info.K);
    check_plan_device(w->device, B);
    const c10::DeviceGuard guard(B.device());
    const int M = w->info.M;
    const int N = static_cast<int>(B.size(1));
    auto C = torch::empty({M, N}, B.options().dtype(torch::kFloat32));
    if (B.scalar_type() == torch::kFloat32) {
        check(ra_tile_plan_run(w->plan, B.data_ptr<float>(), C.data_ptr<float>(), N, route,
                               current_stream()),
              what);
    } else {
        TORCH_CHECK(B.scalar_type() == torch::kFloat16 || B.scalar_type() == torch::kBFloat16,
                    "B must be float32, float16 or bfloat16");
        TORCH_CHECK(N % 8 == 0, "fp16/bf16 B needs N % 8 == 0 (pass float32 B otherwise)");
        check(ra_tile_plan_run_lowp(w->plan, B.data_ptr(), N,
                                    B.scalar_type() == torch::kFloat16 ? RA_DTYPE_F16 : RA_DTYPE_BF16,
                                    C.data_ptr<float>(), N, current_stream()),
              what);
    }
    return C;
}

int half_route(const TilePlan& w) {
    // The low-precision route follows the plan's stored value type.
    return w.info.value_dtype == RA_DTYPE_BF16 ? RA_TILE_ROUTE_BF16 : RA_TILE_ROUTE_F16;
}

void bind_tile_props(pybind11::class_<TilePlan, std::shared_ptr<TilePlan>>& c) {
    c.def_property_readonly("valid", [](const TilePlan& w) { return w.valid; })
        .def_property_readonly("active", [](const TilePlan& w) { return w.info.active != 0; })
        .def_property_readonly("M", [](const TilePlan& w) { return w.info.M; })
        .def_property_readonly("K", [](const TilePlan& w) { return w.info.K; })
        .def_property_readonly("nnz", [](const TilePlan& w) { return w.info.nnz; })
        .def_property_readonly("num_windows", [](const TilePlan& w) { return w.info.num_windows; })
        .def_property_readonly("num_tc_tiles", [](const TilePlan& w) { return w.info.num_blocks; })
        .def_property_readonly("num_vectors", [](const TilePlan& w) { return w.info.num_vectors; })
        .def_property_readonly("avg_tc_tile_density",
                               [](const TilePlan& w) { return w.info.avg_tile_density; })
        .def_property_readonly("plan_bytes", [](const TilePlan& w) { return w.info.plan_bytes; })
        .def_property_readonly("build_ms", [](const TilePlan& w) { return w.info.build_ms; })
        .def_property_readonly("value_scale_log2", [](const TilePlan& w) { return w.info.value_scale_log2; })
        .def_property_readonly("max_window_blocks", [](const TilePlan& w) { return w.info.max_window_blocks; })
        .def_property_readonly("num_blocks", [](const TilePlan& w) { return w.info.num_blocks; })
        .def_property_readonly("num_split_segs", [](const TilePlan& w) { return w.info.num_split_segs; })
        .def_property_readonly("rows_per_window", [](const TilePlan& w) { return w.info.rows_per_window; })
        .def_property_readonly("col_parts", [](const TilePlan& w) { return w.info.col_parts; });
}

}  // namespace

PYBIND11_MODULE(_C, m) {
    m.doc() = "MI355X-native regime-aware SpMM (ra_spmm) — HIP kernels for gfx950";

    m.def("spmm_csr_direct", &spmm_csr_direct, "CSR_DIRECT SpMM (lane group per row, wave64)",
          pybind11::arg("rowptr"), pybind11::arg("colind"), pybind11::arg("vals"),
          pybind11::arg("B"));
    m.def("spmm_csr_baseline", &spmm_csr_baseline,
          "Regime-free baseline CSR SpMM (one wavefront per row)", pybind11::arg("rowptr"),
          pybind11::arg("colind"), pybind11::arg("vals"), pybind11::arg("B"));

    // Guardrail names of the reference, served by the baseline CSR kernel.
    m.def("spmm_csr_baseline_f16", &spmm_csr_baseline_f16,
          "Precision-matched baseline CSR kernel: fp16 vals and B (float16 tensors), fp32 accumulate and C",
          pybind11::arg("rowptr"), pybind11::arg("colind"), pybind11::arg("vals"), pybind11::arg("B"));
    m.def("spmm_cusparse", &spmm_csr_baseline,
          "Guardrail SpMM (served by the hand-written baseline CSR kernel)",
          pybind11::arg("rowptr"), pybind11::arg("colind"), pybind11::arg("vals"),
          pybind11::arg("B"));
    pybind11::class_<BaselinePlan, std::shared_ptr<BaselinePlan>>(m, "CuSparsePlan")
        .def_property_readonly("algorithm",
                               [](const BaselinePlan&) { return std::string("RA_BASELINE_CSR_WAVE_PER_ROW"); });
    m.def("make_cusparse_plan", &make_cusparse_plan, "Reusable guardrail plan (owns C)",
          pybind11::arg("rowptr"), pybind11::arg("colind"), pybind11::arg("vals"),
          pybind11::arg("B"));
    m.def("run_cusparse_plan", &run_cusparse_plan, "Run a reusable guardrail plan",
          pybind11::arg("plan"), pybind11::arg("B"));

    m.def("make_router_plan", &make_router_plan,
          "Four-feature MAIN router plan (features on the GPU when rowptr is a device tensor)",
          pybind11::arg("rowptr"), pybind11::arg("colind"), pybind11::arg("vals"),
          pybind11::arg("M"), pybind11::arg("K"), pybind11::arg("N"),
          pybind11::arg("portfolio") = "MAIN", pybind11::arg("table") = "mi355x");
    m.def("upload", [](torch::Tensor t) {
              return upload(t, t.scalar_type(), torch::Device(torch::kCUDA, c10::hip::current_device()));
          }, "Host tensor to the current device through the pipelined pinned staging used by the plan builders",
          pybind11::arg("tensor"));
    m.def("compute_features", &compute_features, "Production routing features of a rowptr",
          pybind11::arg("rowptr"), pybind11::arg("M"), pybind11::arg("K"), pybind11::arg("N"));
    m.def("route_features", &route_features,
          "Route from exact integer moments (CPU only; no tensors)", pybind11::arg("M"),
          pybind11::arg("K"), pybind11::arg("N"), pybind11::arg("nnz"), pybind11::arg("sum_deg_sq"),
          pybind11::arg("max_deg"), pybind11::arg("empty_rows"), pybind11::arg("portfolio") = "MAIN",
          pybind11::arg("table") = "mi355x");

    pybind11::class_<ZOPlan, std::shared_ptr<ZOPlan>>(m, "RAZeroOverheadPlan")
        .def_property_readonly("valid", [](const ZOPlan& w) { return w.valid; })
        .def_property_readonly("M", [](const ZOPlan& w) { return w.info.M; })
        .def_property_readonly("K", [](const ZOPlan& w) { return w.info.K; })
        .def_property_readonly("num_tiny", [](const ZOPlan& w) { return w.info.num_tiny; })
        .def_property_readonly("num_short", [](const ZOPlan& w) { return w.info.num_short; })
        .def_property_readonly("num_medium", [](const ZOPlan& w) { return w.info.num_medium; })
        .def_property_readonly("num_long", [](const ZOPlan& w) { return w.info.num_long; })
        .def_property_readonly("num_empty", [](const ZOPlan& w) { return w.info.num_empty; })
        .def_property_readonly("num_chunks", [](const ZOPlan& w) { return w.info.num_chunks; })
        .def_property_readonly("num_split_rows", [](const ZOPlan& w) { return w.info.num_split_rows; })
        .def_property_readonly("max_long_chunks", [](const ZOPlan& w) { return w.info.max_long_chunks; })
        .def_property_readonly("num_split_chunks", [](const ZOPlan& w) { return w.info.num_split_chunks; })
        .def_property_readonly("plan_bytes", [](const ZOPlan& w) { return w.info.plan_bytes; });
    m.def("make_zero_overhead_plan", &make_zero_overhead_plan,
          "Build the ZERO_OVERHEAD_CSR plan (degree-binned dispatch; device binning by default)",
          pybind11::arg("rowptr_cpu"), pybind11::arg("M"), pybind11::arg("K"),
          pybind11::arg("build") = "auto");
    m.def("export_zero_overhead_plan",
          [](std::shared_ptr<ZOPlan> w, std::string name) {
              TORCH_CHECK(w && w->valid, "Invalid ZeroOverhead plan");
              int64_t n = 0;
              check(ra_zo_plan_export(w->plan, name.c_str(), nullptr, &n), "export_zero_overhead_plan");
              auto t = torch::empty({n}, torch::TensorOptions().dtype(torch::kInt32));
              check(ra_zo_plan_export(w->plan, name.c_str(), t.data_ptr<int32_t>(), &n),
                    "export_zero_overhead_plan");
              return t;
          },
          "Copy a plan list to the host (short_rows, chunk_rows, chunk_starts, chunk_slot, "
          "split_rows, split_off)",
          pybind11::arg("plan"), pybind11::arg("name"));
    m.def("run_zero_overhead_plan", &run_zero_overhead_plan, "Run ZERO_OVERHEAD_CSR SpMM",
          pybind11::arg("plan"), pybind11::arg("rowptr"), pybind11::arg("colind"),
          pybind11::arg("vals"), pybind11::arg("B"));

    m.def("run_zero_overhead_plan_stage", &run_zero_overhead_plan_stage,
          "Run one ZERO_OVERHEAD_CSR launch stage into C (1 = fused kernel, 2 = merge, 0 = both)",
          pybind11::arg("plan"), pybind11::arg("rowptr"), pybind11::arg("colind"),
          pybind11::arg("vals"), pybind11::arg("B"), pybind11::arg("C"), pybind11::arg("stage"));

    auto tc = pybind11::class_<TilePlan, std::shared_ptr<TilePlan>>(m, "RATilePlan");
    bind_tile_props(tc);
    tc.def_property_readonly("num_groups", [](const TilePlan& w) { return w.info.num_windows; })
        .def_property_readonly("num_communities", [](const TilePlan& w) { return w.info.num_windows; })
        .def_property_readonly("num_tc_groups", [](const TilePlan& w) { return w.info.num_windows; })
        .def_property_readonly("num_segments", [](const TilePlan& w) { return w.info.num_segments; })
        .def_property_readonly("num_split_windows", [](const TilePlan& w) { return w.info.num_split_windows; })
        .def_property_readonly("num_fp32_rows", [](const TilePlan&) { return 0; })
        .def_property_readonly("fp32_group_fraction", [](const TilePlan&) { return 0.0f; })
        .def_property_readonly("intra_community_nnz_fraction",
                               [](const TilePlan& w) { return w.info.avg_tile_density; })
        .def_property_readonly("tc_nnz_fraction", [](const TilePlan&) { return 1.0f; })
        .def_property_readonly("cuda_nnz_fraction", [](const TilePlan&) { return 0.0f; })
        .def_property_readonly("kind", [](const TilePlan& w) { return w.info.kind; });
    // The reference exposes one class per family; they share one layout here.
    m.attr("RATcDirectPlan") = tc;
    m.attr("RACommunityTCPlan") = tc;
    m.attr("RASegmentHybridPlan") = tc;

    struct Fam {
        const char* make;
        const char* run;
        const char* run32;
        int kind;
    };
    for (const Fam& f : {Fam{"make_tc_direct_plan", "run_tc_direct_plan", "run_tc_direct_plan_tf32",
                             RA_TILE_TC_DIRECT},
                         Fam{"make_community_tc_plan", "run_community_tc_plan",
                             "run_community_tc_plan_tf32", RA_TILE_COMMUNITY_TC},
                         Fam{"make_segment_hybrid_plan", "run_segment_hybrid_plan",
                             "run_segment_hybrid_plan_tf32", RA_TILE_SEGMENT_HYBRID}}) {
        const int kind = f.kind;
        const std::string make_name = f.make;
        m.def(f.make,
              [kind, make_name](torch::Tensor rp, torch::Tensor ci, torch::Tensor vl, int M, int K,
                                int N, std::string value_dtype, std::string build, int rows_per_window) {
                  return make_tile_plan(kind, rp, ci, vl, M, K, N, value_dtype, build, rows_per_window,
                                        make_name.c_str());
              },
              "Build the tile plan (device build by default; build='host' for the host builder; "
              "rows_per_window 0 = chosen from the matrix, 8 = the reference's windows, 16/32 = tall)",
              pybind11::arg("rowptr_cpu"), pybind11::arg("colind_cpu"), pybind11::arg("vals_cpu"),
              pybind11::arg("M"), pybind11::arg("K"), pybind11::arg("N"),
              pybind11::arg("value_dtype") = "fp16", pybind11::arg("build") = "auto",
              pybind11::arg("rows_per_window") = 0);
        if (kind == RA_TILE_SEGMENT_HYBRID) {
            // run_segment_hybrid_plan(plan, colind, vals, B): colind/vals are kept
            // for ABI compatibility, as in tc/ra_segment_hybrid.cu:546-551.
            m.def(f.run,
                  [](std::shared_ptr<TilePlan> w, torch::Tensor, torch::Tensor, torch::Tensor B) {
                      return run_tile_plan(w, B, half_route(*w),
                                           "run_segment_hybrid_plan");
                  },
                  "Run on the FP16/BF16 MFMA route", pybind11::arg("plan"), pybind11::arg("colind"),
                  pybind11::arg("vals"), pybind11::arg("B"));
            m.def(f.run32,
                  [](std::shared_ptr<TilePlan> w, torch::Tensor, torch::Tensor, torch::Tensor B) {
                      return run_tile_plan(w, B, RA_TILE_ROUTE_FP32, "run_segment_hybrid_plan_tf32");
                  },
                  "Run on the FP32-FMA route (replaces the TF32 path)", pybind11::arg("plan"),
                  pybind11::arg("colind"), pybind11::arg("vals"), pybind11::arg("B"));
        } else {
            const std::string rn = f.run, rn32 = f.run32;
            m.def(f.run,
                  [rn](std::shared_ptr<TilePlan> w, torch::Tensor B) {
                      return run_tile_plan(w, B, half_route(*w),
                                           rn.c_str());
                  },
                  "Run on the FP16/BF16 MFMA route", pybind11::arg("plan"), pybind11::arg("B"));
            m.def(f.run32,
                  [rn32](std::shared_ptr<TilePlan> w, torch::Tensor B) {
                      return run_tile_plan(w, B, RA_TILE_ROUTE_FP32, rn32.c_str());
                  },
                  "Run on the FP32-FMA route (replaces the TF32 path)", pybind11::arg("plan"),
                  pybind11::arg("B"));
        }
    }
    m.def("export_tile_plan",
          [](std::shared_ptr<TilePlan> w, std::string name) {
              TORCH_CHECK(w && w->valid, "Invalid tile plan");
              int64_t n = 0;
              check(ra_tile_plan_export(w->plan, name.c_str(), nullptr, &n), "export_tile_plan");
              auto t = torch::empty({n}, torch::TensorOptions().dtype(name == "vals" ? torch::kInt16 : torch::kInt32));
              check(ra_tile_plan_export(w->plan, name.c_str(), t.data_ptr(), &n), "export_tile_plan");
              return t;
          },
          "Copy a plan array to the host (block_offsets, atox, win_rows, vals, seg_*, split_*)",
          pybind11::arg("plan"), pybind11::arg("name"));
    m.def("run_tile_plan_route",
          [](std::shared_ptr<TilePlan> w, torch::Tensor B, std::string route) {
              int r = RA_TILE_ROUTE_F16;
              if (route == "bf16") r = RA_TILE_ROUTE_BF16;
              else if (route == "fp32") r = RA_TILE_ROUTE_FP32;
              else TORCH_CHECK(route == "fp16", "route must be fp16, bf16 or fp32");
              return run_tile_plan(w, B, r, "run_tile_plan_route");
          },
          "Run a tile plan on an explicit route", pybind11::arg("plan"), pybind11::arg("B"),
          pybind11::arg("route"));

    m.def("analyze_matrix", &analyze_matrix,
          "Diagnostic structural features of a CSR matrix (host computation)", pybind11::arg("rowptr"),
          pybind11::arg("colind"), pybind11::arg("M"), pybind11::arg("K"), pybind11::arg("N"));
    m.def("abi_version", &ra_abi_version);
}
