// tile_build.cpp — host build of the tile format (windows of 8 rows, 8x1
// vectors, blocks of 8 vectors), parallel over window ranges.
//
// Reference algorithm (same windows, vectors, blocks and splits; own code):
//   build_ra_tc_direct_plan_impl   tc/ra_tc_direct.cu:627-780 (natural order)
//   make_ra_community_tc_plan      tc/ra_community_tc.cu:320-471 (rows stable-
//                                  sorted by (leading column or INT_MAX, row))
//   make_ra_segment_hybrid_plan    tc/ra_segment_hybrid.cu:470-498 (windows of
//                                  more than 64 blocks split into <=64-block segments)
// Differences, on purpose: duplicate (row, column) entries are summed before
// rounding (the reference would store both into one slot); vector padding is
// -1 so kernels skip it instead of gathering B row 0.
#include <algorithm>
#include <chrono>
#include <climits>
#include <cmath>
#include <cstring>
#include <numeric>

#include "half_convert.hpp"
#include "ra_internal.hpp"
#include "tile_format.hpp"

namespace ra {

uint16_t f32_to_f16_rne(float f) { return half_rne_bits(f); }
uint16_t f32_to_bf16_rne(float f) { return bf16_rne_bits(f); }

int32_t f16_value_scale_log2(float max_abs) {
    if (!(max_abs > 0.f) || !std::isfinite(max_abs)) return 0;
    const int e = std::ilogb(max_abs);           // max_abs in [2^e, 2^(e+1))
    int s = 13 - e;                               // -> [2^13, 2^14)
    if (s > 24) s = 24;
    if (s < -24) s = -24;
    return s;
}

namespace {

struct WindowRange {
    std::vector<int32_t> blocks;  // per window in the range
    std::vector<int32_t> atox;
    std::vector<uint16_t> vals;
    int64_t nnz = 0, vectors = 0;
};

struct Entry {
    uint64_t key;  // (column << 3) | slot
    int64_t p;     // CSR position: deterministic order for duplicates
    bool operator<(const Entry& o) const { return key < o.key || (key == o.key && p < o.p); }
};

}  // namespace

ra_status tile_host_build(int32_t kind, const int32_t* rowptr, const int32_t* colind,
                          const float* vals, int32_t M, int32_t K, int32_t N, int32_t value_dtype,
                          ra_tile_host& out) {
    const auto t0 = std::chrono::steady_clock::now();
    if (kind < RA_TILE_TC_DIRECT || kind > RA_TILE_SEGMENT_HYBRID)
        return fail(RA_ERR_INVALID_ARGUMENT, "tile: unknown kind");
    if (value_dtype != RA_DTYPE_F16 && value_dtype != RA_DTYPE_BF16)
        return fail(RA_ERR_INVALID_ARGUMENT, "tile: value_dtype must be F16 or BF16");
    if (M < 0 || K < 0) return fail(RA_ERR_INVALID_ARGUMENT, "tile: negative dimension");
    if (M > 0 && !rowptr) return fail(RA_ERR_INVALID_ARGUMENT, "tile: rowptr is NULL");
    out = ra_tile_host{};
    out.kind = kind;
    out.M = M;
    out.K = K;
    out.N = N;
    out.value_dtype = value_dtype;
    // Plans are inactive below the MFMA minimum width (tc/ra_tc_direct.cu:644-646).
    if (M == 0 || K == 0 || N < 16) return RA_OK;
    for (int32_t r = 0; r < M; ++r)
        if (rowptr[r + 1] < rowptr[r]) return fail(RA_ERR_INVALID_ARGUMENT, "tile: rowptr not monotone");
    const int64_t total = static_cast<int64_t>(rowptr[M]) - rowptr[0];
    if (total > 0 && (!colind || !vals)) return fail(RA_ERR_INVALID_ARGUMENT, "tile: colind/vals NULL");
    for (int64_t p = rowptr[0]; p < rowptr[M]; ++p)
        if (colind[p] < 0 || colind[p] >= K) return fail(RA_ERR_INVALID_ARGUMENT, "tile: column index out of range");

    const int32_t W = (M + kTileWindow - 1) / kTileWindow;
    out.win_rows.assign(static_cast<size_t>(W) * kTileWindow, -1);
    if (kind == RA_TILE_COMMUNITY_TC) {
        // Leading-neighbour order; (key, row) pairs are unique, so any sort
        // gives the stable order of tc/ra_community_tc.cu:338-343.
        std::vector<uint64_t> keyed(M);
        parallel_for(M, 1 << 16, [&](int64_t b, int64_t e) {
            for (int64_t r = b; r < e; ++r) {
                const uint32_t lead = rowptr[r] < rowptr[r + 1] ? static_cast<uint32_t>(colind[rowptr[r]])
                                                                : static_cast<uint32_t>(INT_MAX);
                keyed[r] = (static_cast<uint64_t>(lead) << 32) | static_cast<uint32_t>(r);
            }
        });
        std::sort(keyed.begin(), keyed.end());
        for (int32_t i = 0; i < M; ++i) out.win_rows[i] = static_cast<int32_t>(keyed[i] & 0xFFFFFFFFu);
    } else {
        std::iota(out.win_rows.begin(), out.win_rows.begin() + M, 0);
    }

    const bool bf16 = value_dtype == RA_DTYPE_BF16;
    if (!bf16) {
        float mx = 0.f;
        for (int64_t p = rowptr[0]; p < rowptr[M]; ++p) mx = std::max(mx, std::fabs(vals[p]));
        out.value_scale_log2 = f16_value_scale_log2(mx);
    }
    const float vscale = std::ldexp(1.0f, out.value_scale_log2);
    constexpr int64_t kWinPerTask = 256;
    const int64_t ntasks = (W + kWinPerTask - 1) / kWinPerTask;
    std::vector<WindowRange> parts(ntasks);
    parallel_for(ntasks, 1, [&](int64_t tb, int64_t te) {
        std::vector<Entry> ent;
        std::vector<float> acc;
        for (int64_t t = tb; t < te; ++t) {
            WindowRange& part = parts[t];
            const int64_t w0 = t * kWinPerTask, w1 = std::min<int64_t>(W, w0 + kWinPerTask);
            part.blocks.assign(w1 - w0, 0);
            for (int64_t w = w0; w < w1; ++w) {
                ent.clear();
                for (int slot = 0; slot < kTileWindow; ++slot) {
                    const int32_t r = out.win_rows[w * kTileWindow + slot];
                    if (r < 0) continue;
                    for (int64_t p = rowptr[r]; p < rowptr[r + 1]; ++p)
                        ent.push_back({(static_cast<uint64_t>(colind[p]) << 3) | static_cast<uint64_t>(slot), p});
                }
                if (ent.empty()) continue;
                std::sort(ent.begin(), ent.end());
                // Distinct columns -> vectors; duplicate (col, slot) summed in CSR order.
                int64_t nvec = 0;
                uint64_t prev_col = UINT64_MAX;
                for (const Entry& e : ent) {
                    if ((e.key >> 3) != prev_col) {
                        ++nvec;
                        prev_col = e.key >> 3;
                    }
                }
                const int32_t nblk = static_cast<int32_t>((nvec + kTileVec - 1) / kTileVec);
                part.blocks[w - w0] = nblk;
                part.vectors += nvec;
                const size_t abase = part.atox.size(), vbase = part.vals.size();
                part.atox.resize(abase + static_cast<size_t>(nblk) * kTileVec, -1);
                part.vals.resize(vbase + static_cast<size_t>(nblk) * kTileVec * kTileWindow, 0);
                acc.assign(static_cast<size_t>(nblk) * kTileVec * kTileWindow, 0.f);
                int64_t v = -1;
                prev_col = UINT64_MAX;
                uint64_t prev_key = UINT64_MAX;
                for (const Entry& e : ent) {
                    const uint64_t col = e.key >> 3;
                    const int slot = static_cast<int>(e.key & 7u);
                    if (col != prev_col) {
                        ++v;
                        prev_col = col;
                        part.atox[abase + v] = static_cast<int32_t>(col);
                    }
                    const size_t idx = static_cast<size_t>(v / kTileVec) * 64 + slot * kTileVec + (v % kTileVec);
                    acc[idx] += vals[e.p];
                    if (e.key != prev_key) ++part.nnz;
                    prev_key = e.key;
                }
                for (size_t i = 0; i < acc.size(); ++i)
                    part.vals[vbase + i] = bf16 ? f32_to_bf16_rne(acc[i]) : f32_to_f16_rne(acc[i] * vscale);
            }
        }
    });

    out.block_offsets.assign(static_cast<size_t>(W) + 1, 0);
    std::vector<int64_t> task_block0(ntasks + 1, 0);
    for (int64_t t = 0; t < ntasks; ++t) {
        const int64_t w0 = t * kWinPerTask;
        int64_t acc = task_block0[t];
        for (size_t i = 0; i < parts[t].blocks.size(); ++i) {
            out.block_offsets[w0 + i] = static_cast<int32_t>(acc);
            acc += parts[t].blocks[i];
            out.max_window_blocks = std::max(out.max_window_blocks, parts[t].blocks[i]);
        }
        task_block0[t + 1] = acc;
        out.nnz += parts[t].nnz;
        out.num_vectors += parts[t].vectors;
    }
    const int64_t total_blocks = task_block0[ntasks];
    if (total_blocks > INT32_MAX / 64) return fail(RA_ERR_UNSUPPORTED, "tile: too many blocks for int32 offsets");
    out.block_offsets[W] = static_cast<int32_t>(total_blocks);
    out.atox.resize(static_cast<size_t>(total_blocks) * kTileVec);
    out.vals.resize(static_cast<size_t>(total_blocks) * kTileVec * kTileWindow);
    parallel_for(ntasks, 1, [&](int64_t tb, int64_t te) {
        for (int64_t t = tb; t < te; ++t) {
            std::copy(parts[t].atox.begin(), parts[t].atox.end(),
                      out.atox.begin() + task_block0[t] * kTileVec);
            std::copy(parts[t].vals.begin(), parts[t].vals.end(),
                      out.vals.begin() + task_block0[t] * kTileVec * kTileWindow);
        }
    });

    {
        // tc/ra_segment_hybrid.cu:470-498: windows of more than `limit` blocks
        // are split into consecutive <= limit-block segments with private
        // partial slots, merged in ascending slot order.
        const int32_t limit = kind == RA_TILE_SEGMENT_HYBRID ? kTileSegBlocks : kTileDirectSplitBlocks;
        out.split_offsets.push_back(0);
        int32_t slots = 0;
        for (int32_t w = 0; w < W; ++w) {
            const int32_t b0 = out.block_offsets[w], b1 = out.block_offsets[w + 1];
            if (b1 - b0 <= limit) {
                out.seg_window.push_back(static_cast<int32_t>(static_cast<uint32_t>(w) | kTileSoleFlag));
                out.seg_bbegin.push_back(b0);
                out.seg_bend.push_back(b1);
                out.seg_slot.push_back(-1);
            } else {
                out.split_windows.push_back(w);
                for (int32_t b = b0; b < b1; b += limit) {
                    out.seg_window.push_back(w);
                    out.seg_bbegin.push_back(b);
                    out.seg_bend.push_back(std::min(b + limit, b1));
                    out.seg_slot.push_back(slots++);
                }
                out.split_offsets.push_back(slots);
            }
        }
    }
    out.active = true;
    out.build_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    return RA_OK;
}

}  // namespace ra

extern "C" {

ra_status ra_tile_host_build(int32_t kind, const int32_t* h_rowptr, const int32_t* h_colind,
                             const float* h_vals, int32_t M, int32_t K, int32_t N,
                             int32_t value_dtype, ra_tile_host** out) {
    if (!out) return ra::fail(RA_ERR_INVALID_ARGUMENT, "tile: out is NULL");
    *out = nullptr;
    auto h = new (std::nothrow) ra_tile_host();
    if (!h) return ra::fail(RA_ERR_OUT_OF_MEMORY, "tile: host allocation");
    ra_status s;
    try {
        s = ra::tile_host_build(kind, h_rowptr, h_colind, h_vals, M, K, N, value_dtype, *h);
    } catch (const std::bad_alloc&) {
        s = ra::fail(RA_ERR_OUT_OF_MEMORY, "tile: host build out of memory");
    }
    if (s != RA_OK) {
        delete h;
        return s;
    }
    *out = h;
    return RA_OK;
}

ra_status ra_tile_host_get_info(const ra_tile_host* h, ra_tile_info* info) {
    if (!h || !info) return ra::fail(RA_ERR_INVALID_ARGUMENT, "tile: NULL argument");
    std::memset(info, 0, sizeof(*info));
    info->kind = h->kind;
    info->M = h->M;
    info->K = h->K;
    info->active = h->active ? 1 : 0;
    info->num_windows = h->active ? static_cast<int32_t>(h->block_offsets.size() - 1) : 0;
    info->num_blocks = h->active ? h->block_offsets.back() : 0;
    info->num_segments = static_cast<int32_t>(h->seg_window.size());
    info->num_split_windows = static_cast<int32_t>(h->split_windows.size());
    info->num_split_segs = h->split_offsets.empty() ? 0 : h->split_offsets.back();
    info->max_window_blocks = h->max_window_blocks;
    info->nnz = h->nnz;
    info->num_vectors = h->num_vectors;
    info->plan_bytes = static_cast<int64_t>(
        4 * (h->win_rows.size() + h->block_offsets.size() + h->atox.size() + h->seg_window.size() +
             h->seg_bbegin.size() + h->seg_bend.size() + h->seg_slot.size() +
             h->split_windows.size() + h->split_offsets.size()) +
        2 * h->vals.size());
    info->avg_tile_density =
        info->num_blocks > 0 ? static_cast<float>(static_cast<double>(h->nnz) / (64.0 * info->num_blocks)) : 0.f;
    info->value_dtype = h->value_dtype;
    info->value_scale_log2 = h->value_scale_log2;
    info->rows_per_window = ra::kTileWindow;
    info->col_parts = 1;
    info->build_ms = h->build_ms;
    return RA_OK;
}

ra_status ra_tile_host_export(const ra_tile_host* h, const char* name, void* dst, int64_t* count) {
    if (!h || !name || !count) return ra::fail(RA_ERR_INVALID_ARGUMENT, "tile export: NULL argument");
    const std::vector<int32_t>* iv = nullptr;
    const std::string n(name);
    if (n == "vals") {
        *count = static_cast<int64_t>(h->vals.size());
        if (dst && !h->vals.empty()) std::memcpy(dst, h->vals.data(), h->vals.size() * 2);
        return RA_OK;
    }
    if (n == "block_offsets") iv = &h->block_offsets;
    else if (n == "atox") iv = &h->atox;
    else if (n == "win_rows") iv = &h->win_rows;
    else if (n == "seg_window") iv = &h->seg_window;
    else if (n == "seg_bbegin") iv = &h->seg_bbegin;
    else if (n == "seg_bend") iv = &h->seg_bend;
    else if (n == "seg_slot") iv = &h->seg_slot;
    else if (n == "split_windows") iv = &h->split_windows;
    else if (n == "split_offsets") iv = &h->split_offsets;
    else return ra::fail(RA_ERR_INVALID_ARGUMENT, "tile export: unknown array '" + n + "'");
    *count = static_cast<int64_t>(iv->size());
    if (dst && !iv->empty()) std::memcpy(dst, iv->data(), iv->size() * 4);
    return RA_OK;
}

void ra_tile_host_destroy(ra_tile_host* h) { delete h; }

}  // extern "C"
