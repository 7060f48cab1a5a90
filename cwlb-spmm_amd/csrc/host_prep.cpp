// Host preprocessing of the CWLB-SpMM path: degree reordering, cost-weighted
// task partitioning, segment-size selection and the cost file.  Plain
// C++17, compiled with -ffp-contract=off so the partition's double
// arithmetic is the IEEE sequence the reference executes.
#include <algorithm>
#include <cerrno>
#include <climits>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <iomanip>
#include <string>
#include <thread>
#include <utility>
#include <vector>

#include "cwlb.h"

namespace cwlb {
cwlb_status fail(cwlb_status st, const std::string& msg);
}

namespace {

// ---------------------------------------------------------------------------
// Threads for the host reordering: up to 16 (the host share of one GPU),
// about one per 256K rows + nonzeros, at least one.
constexpr int32_t kDenseDegrees = 1 << 16;

int reorder_threads(int32_t n_rows, int64_t nnz)
{
    const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
    const int64_t by_size = (static_cast<int64_t>(n_rows) + nnz) / (1 << 18) + 1;
    return static_cast<int>(std::min<int64_t>({static_cast<int64_t>(hw), 16, by_size}));
}

// fn(t) for t in [0, T): on T - 1 new threads and the caller's.
template <class Fn>
void parallel_for(int T, Fn fn)
{
    std::vector<std::thread> pool;
    pool.reserve(static_cast<size_t>(T > 0 ? T - 1 : 0));
    for (int t = 1; t < T; ++t) pool.emplace_back(fn, t);
    fn(0);
    for (std::thread& th : pool) th.join();
}

// ---------------------------------------------------------------------------
// Cost-weighted partition (reference src/utils.cpp:832-1021).
//
// Rows are visited in reordered order.  A row whose full weight
// wCL*deg + Cs fits the capacity is packed into the open task; a heavier row
// is cut into segments of at most S nonzeros (weight wCL*nnz + Ca), where S
// is recovered from the capacity.  The deg % S remainder of a long row may
// ride at the end of the task before it ("current prefix", :879-912), and
// the last segment of a long row may take the remainder of the next long
// row ("next prefix", :915-939).  Ties and comparisons are exactly the
// reference's, in double.
class Partitioner {
public:
    Partitioner(const int32_t* rp, int32_t n, const cwlb_cost_params& c, double cap)
        : rp_(rp), n_(n), wcl_(c.C_compute_ns + c.C_load_ns), cs_(c.C_store_ns),
          ca_(c.C_atomic_ns), cap_(cap)
    {
        // std::max(1e-30, wCL) keeps 1e-30 unless wCL is larger (NaN -> 1e-30).
        const double denom = (1e-30 < wcl_) ? wcl_ : 1e-30;
        const double x = std::floor((cap_ - ca_) / denom);
        // static_cast<int> as x86-64 executes it (out of range / NaN -> INT_MIN).
        int s = INT_MIN;
        if (x == x && x < 2147483648.0 && x > -2147483649.0) s = static_cast<int>(x);
        seg_ = std::max(1, s);
    }

    std::vector<cwlb_task> run()
    {
        if (n_ <= 0) return {};
        int row = 0;
        while (row < n_) {
            const int deg = degree(row);
            const double wr = full_weight(row);
            if (wr <= cap_) {
                if (load_ == 0.0 || load_ + wr <= cap_) {
                    load_ += wr;
                    ++row;
                } else {
                    close(row, 0);
                    open_at(row, 0);
                }
                continue;
            }
            split_long_row(row, deg);
            ++row;
        }
        if (load_ > 0.0 || start_ < n_) emit(start_, n_, off0_, 0);
        return std::move(out_);
    }

private:
    int degree(int r) const { return rp_[r + 1] - rp_[r]; }
    double full_weight(int r) const { return wcl_ * static_cast<double>(degree(r)) + cs_; }
    double seg_weight(int nnz) const { return wcl_ * static_cast<double>(nnz) + ca_; }

    void emit(int s, int e, int fo, int last)
    {
        if (s < e) out_.push_back(cwlb_task{s, e, fo, last});
    }
    // Emits the open task [start_, end_row) whose last row ends at `last`.
    void close(int end_row, int last) { emit(start_, end_row, off0_, last); }
    void open_at(int row, int off)
    {
        start_ = row;
        off0_ = off;
        load_ = 0.0;
    }

    void split_long_row(int row, int deg)
    {
        const bool prefix_taken = (load_ == 0.0 && start_ == row && off0_ > 0);
        int off = prefix_taken ? off0_ : 0;
        int remaining = deg - off;
        if (remaining <= 0) {
            open_at(row + 1, 0);
            return;
        }
        if (!prefix_taken && !(load_ <= 0.0)) {
            // Ride the deg % S remainder at the end of the open task.
            const int r = deg % seg_;
            if (r == 0 || r >= deg) {
                close(row, 0);
                open_at(row, 0);
            } else if (seg_weight(r) <= cap_ - load_) {
                close(row + 1, r);
                open_at(row, r);
                remaining -= r;
                off += r;
            } else {
                close(row, 0);
                open_at(row, 0);
            }
        }
        while (remaining > 0) {
            const int take = std::min(remaining, seg_);
            load_ += seg_weight(take);
            remaining -= take;
            off += take;
            if (remaining > 0) {
                close(row + 1, off);
                open_at(row, off);
            } else if (!take_next_prefix(row)) {
                close(row + 1, 0);
                open_at(row + 1, 0);
            }
        }
    }

    // The last segment of `row` takes the deg % S remainder of the next row
    // when that row is long and the remainder fits.
    bool take_next_prefix(int row)
    {
        if (load_ >= cap_) return false;
        const int nr = row + 1;
        if (nr >= n_) return false;
        const int nd = degree(nr);
        if (full_weight(nr) <= cap_) return false;
        const int r2 = nd % seg_;
        if (r2 == 0 || r2 >= nd) return false;
        if (seg_weight(r2) > cap_ - load_) return false;
        close(nr + 1, r2);
        open_at(nr, r2);
        return true;
    }

    const int32_t* rp_;
    int32_t n_;
    double wcl_, cs_, ca_, cap_;
    int seg_ = 1;
    int start_ = 0;    // first row of the open task
    int off0_ = 0;     // nonzero offset of the open task's first row
    double load_ = 0.0;
    std::vector<cwlb_task> out_;
};

}  // namespace

extern "C" {

cwlb_status cwlb_partition(const int32_t* row_ptr, int32_t n_rows, const cwlb_cost_params* costs,
                           double capacity_weight, cwlb_task* out, int64_t capacity_tasks,
                           int64_t* n_tasks)
{
    if (!costs || !n_tasks) return cwlb::fail(CWLB_INVALID_ARG, "cwlb_partition: null argument");
    if (n_rows > 0 && !row_ptr)
        return cwlb::fail(CWLB_INVALID_ARG, "cwlb_partition: null row_ptr");
    std::vector<cwlb_task> tasks;
    try {
        tasks = Partitioner(row_ptr, n_rows, *costs, capacity_weight).run();
    } catch (const std::bad_alloc&) {
        return cwlb::fail(CWLB_OOM, "cwlb_partition: out of host memory");
    }
    *n_tasks = static_cast<int64_t>(tasks.size());
    if (static_cast<int64_t>(tasks.size()) > capacity_tasks || (!out && !tasks.empty()))
        return cwlb::fail(CWLB_INSUFFICIENT, "cwlb_partition: output buffer too small");
    if (!tasks.empty()) std::memcpy(out, tasks.data(), tasks.size() * sizeof(cwlb_task));
    return CWLB_OK;
}

// Degree reordering (reference main.cpp:197-278): a stable counting sort by
// degree gives the (degree, original id) order of the reference comparator.
// It runs on up to 16 threads over contiguous row chunks (per-chunk
// histograms, then positions in chunk order, so equal degrees keep
// ascending ids), as the reference's oneDPL/TBB sort runs on all cores.
cwlb_status cwlb_reorder_by_degree(int32_t n_rows, int64_t nnz, const int32_t* row_ptr,
                                   const int32_t* col_idx, const float* val, int32_t* origin,
                                   int32_t* row_ptr_out, int32_t* col_idx_out, float* val_out)
{
    if (n_rows < 0 || nnz < 0 || nnz > INT32_MAX)
        return cwlb::fail(CWLB_INVALID_ARG, "cwlb_reorder_by_degree: bad sizes");
    if (n_rows == 0) {
        if (row_ptr_out) row_ptr_out[0] = 0;
        return CWLB_OK;
    }
    if (!row_ptr || !origin || !row_ptr_out || (nnz > 0 && (!col_idx || !val || !col_idx_out ||
                                                            !val_out)))
        return cwlb::fail(CWLB_INVALID_ARG, "cwlb_reorder_by_degree: null pointer");
    const int T = reorder_threads(n_rows, nnz);
    const auto lo = [&](int t) { return static_cast<int32_t>(static_cast<int64_t>(n_rows) * t / T); };

    // 1. Validation and per-thread histograms of the degrees below
    //    kDenseDegrees; heavier rows are rare (at most nnz / kDenseDegrees)
    //    and are ordered separately.
    std::vector<std::vector<int64_t>> hist(static_cast<size_t>(T));
    std::vector<std::vector<std::pair<int32_t, int32_t>>> heavy(static_cast<size_t>(T));
    std::vector<int32_t> maxdeg(static_cast<size_t>(T), 0);
    std::vector<char> bad(static_cast<size_t>(T), 0);
    parallel_for(T, [&](int t) {
        std::vector<int64_t>& h = hist[static_cast<size_t>(t)];
        int32_t m = 0;
        for (int32_t i = lo(t); i < lo(t + 1); ++i) {
            const int32_t d = row_ptr[i + 1] - row_ptr[i];
            if (d < 0 || row_ptr[i] < 0 || row_ptr[i + 1] > nnz) {
                bad[static_cast<size_t>(t)] = 1;
                return;
            }
            m = std::max(m, d);
            if (d < kDenseDegrees) {
                if (static_cast<size_t>(d) >= h.size()) h.resize(static_cast<size_t>(d) + 1, 0);
                ++h[static_cast<size_t>(d)];
            }
        }
        maxdeg[static_cast<size_t>(t)] = m;
    });
    if (std::any_of(bad.begin(), bad.end(), [](char c) { return c != 0; }))
        return cwlb::fail(CWLB_INVALID_ARG, "cwlb_reorder_by_degree: row_ptr not a CSR offset array");
    const int32_t dmax = *std::max_element(maxdeg.begin(), maxdeg.end());
    const size_t D = static_cast<size_t>(std::min<int32_t>(dmax, kDenseDegrees - 1)) + 1;

    // 2. Stable positions: degree d, thread t starts after every row of a
    //    smaller degree and every row of degree d in an earlier chunk.
    std::vector<std::vector<int64_t>> pos(static_cast<size_t>(T), std::vector<int64_t>(D, 0));
    int64_t running = 0;
    for (size_t d = 0; d < D; ++d)
        for (int t = 0; t < T; ++t) {
            pos[static_cast<size_t>(t)][d] = running;
            const std::vector<int64_t>& h = hist[static_cast<size_t>(t)];
            running += d < h.size() ? h[d] : 0;
        }
    const int64_t n_light = running;

    // 3. Scatter of the row ids.
    parallel_for(T, [&](int t) {
        std::vector<int64_t>& p = pos[static_cast<size_t>(t)];
        for (int32_t i = lo(t); i < lo(t + 1); ++i) {
            const int32_t d = row_ptr[i + 1] - row_ptr[i];
            if (d < kDenseDegrees) origin[p[static_cast<size_t>(d)]++] = i;
            else heavy[static_cast<size_t>(t)].emplace_back(d, i);
        }
    });
    // Heavy rows in (degree, id) order after all lighter ones; the chunks
    // are in id order, so a stable sort by degree gives it.
    std::vector<std::pair<int32_t, int32_t>> all_heavy;
    for (const auto& v : heavy) all_heavy.insert(all_heavy.end(), v.begin(), v.end());
    std::stable_sort(all_heavy.begin(), all_heavy.end(),
                     [](const auto& x, const auto& y) { return x.first < y.first; });
    for (size_t k = 0; k < all_heavy.size(); ++k)
        origin[n_light + static_cast<int64_t>(k)] = all_heavy[k].second;

    // 4. Offsets: inclusive scan of the sorted degrees, chunk sums first.
    std::vector<int64_t> part(static_cast<size_t>(T) + 1, 0);
    parallel_for(T, [&](int t) {
        int64_t acc = 0;
        for (int32_t r = lo(t); r < lo(t + 1); ++r) acc += row_ptr[origin[r] + 1] - row_ptr[origin[r]];
        part[static_cast<size_t>(t) + 1] = acc;
    });
    for (int t = 0; t < T; ++t) part[static_cast<size_t>(t) + 1] += part[static_cast<size_t>(t)];
    if (part[static_cast<size_t>(T)] != nnz)
        return cwlb::fail(CWLB_RUNTIME_ERROR,
                          "DPL CPU degree reordering produced an inconsistent NNZ count.");
    row_ptr_out[0] = 0;
    parallel_for(T, [&](int t) {
        int64_t acc = part[static_cast<size_t>(t)];
        for (int32_t r = lo(t); r < lo(t + 1); ++r) {
            acc += row_ptr[origin[r] + 1] - row_ptr[origin[r]];
            row_ptr_out[r + 1] = static_cast<int32_t>(acc);
        }
    });

    // 5. Row copies, each row keeping its entry order.  The degrees ascend,
    //    so the chunks are cut at equal shares of the nonzeros, not rows.
    const auto nz_lo = [&](int t) {
        const int64_t target = nnz * t / T;
        return static_cast<int32_t>(
            std::lower_bound(row_ptr_out, row_ptr_out + n_rows, target) - row_ptr_out);
    };
    parallel_for(T, [&](int t) {
        const int32_t end = t + 1 == T ? n_rows : nz_lo(t + 1);
        for (int32_t r = t == 0 ? 0 : nz_lo(t); r < end; ++r) {
            const int32_t o = origin[r];
            const int32_t len = row_ptr[o + 1] - row_ptr[o];
            if (len == 0) continue;  // the arrays may be null when nnz == 0
            std::memcpy(col_idx_out + row_ptr_out[r], col_idx + row_ptr[o],
                        sizeof(int32_t) * static_cast<size_t>(len));
            std::memcpy(val_out + row_ptr_out[r], val + row_ptr[o],
                        sizeof(float) * static_cast<size_t>(len));
        }
    });
    return CWLB_OK;
}

// capacity_from_s (reference main.cpp:281-292).
double cwlb_capacity_from_s(int32_t s, const cwlb_cost_params* costs)
{
    const double edge = costs->C_compute_ns + costs->C_load_ns;
    const int32_t cs = std::max(1, s);
    if (edge <= 0.0) return std::max(0.0, costs->C_atomic_ns);
    return std::max(0.0, costs->C_atomic_ns + edge * static_cast<double>(cs));
}

// wave_based_s (reference main.cpp:295-321).
cwlb_status cwlb_wave_based_s(int64_t nnz, int64_t row_ptr_len, int32_t compute_units,
                              int32_t wave, int32_t* s_out)
{
    if (compute_units <= 0 || wave <= 0)
        return cwlb::fail(CWLB_INVALID_ARG, "compute_units and wave must be positive.");
    if (row_ptr_len == 0) {
        *s_out = 1;
        return CWLB_OK;
    }
    const uint64_t n = static_cast<uint64_t>(nnz);
    const uint64_t den = static_cast<uint64_t>(compute_units) * static_cast<uint64_t>(wave);
    uint64_t s = (n + den - 1) / den;
    s = std::max<uint64_t>(1, s);
    s = std::min<uint64_t>(s, static_cast<uint64_t>(INT32_MAX));
    *s_out = static_cast<int32_t>(s);
    return CWLB_OK;
}

// recommended_candidate_w (reference main.cpp:87-95).
void cwlb_recommended_candidate_w(uint64_t nnz, int32_t out3[3])
{
    struct Row {
        uint64_t below;
        int32_t w[3];
    };
    static const Row table[] = {
        {100000ULL, {64, 32, 16}},       {500000ULL, {128, 64, 32}},
        {1000000ULL, {256, 128, 64}},    {5000000ULL, {512, 256, 128}},
        {10000000ULL, {1024, 512, 256}}, {50000000ULL, {4096, 2048, 1024}},
    };
    for (const Row& r : table) {
        if (nnz < r.below) {
            std::copy(r.w, r.w + 3, out3);
            return;
        }
    }
    out3[0] = 8192;
    out3[1] = 4096;
    out3[2] = 2048;
}

// candidate_search_bounds (reference main.cpp:109-127).
cwlb_status cwlb_candidate_search_bounds(const int32_t v[3], int64_t best, int32_t* lower,
                                         int32_t* upper)
{
    if (best < 0 || best >= 3 || v[0] <= 0 || v[1] < v[0] || v[2] < v[1])
        return cwlb::fail(CWLB_INVALID_ARG, "Invalid ordered candidate values or best index.");
    int64_t lo = v[0], hi = v[2];
    if (best == 0) {
        lo = 2LL * v[0] - v[1];
        hi = v[1];
    } else if (best == 2) {
        lo = v[1];
        hi = 2LL * v[2] - v[1];
    }
    *lower = static_cast<int32_t>(std::max<int64_t>(1, lo));
    *upper = static_cast<int32_t>(std::min<int64_t>(INT32_MAX, hi));
    return CWLB_OK;
}

constexpr int64_t kMaxSearchPoints = 10000;

// candidate_search_by_count (reference main.cpp:130-148).
cwlb_status cwlb_candidate_search_by_count(int32_t lower, int32_t upper, int32_t requested,
                                           int32_t* out, int64_t capacity, int64_t* count)
{
    if (lower <= 0 || upper < lower || requested <= 0)
        return cwlb::fail(CWLB_INVALID_ARG, "Invalid search interval or point count.");
    const int64_t width = static_cast<int64_t>(upper) - lower;
    const int64_t n = std::min<int64_t>(requested, width + 1);
    if (n > kMaxSearchPoints)
        return cwlb::fail(CWLB_INVALID_ARG, "Search plan exceeds 10000 points; reduce the count.");
    *count = n;
    if (n > capacity || !out) return cwlb::fail(CWLB_INSUFFICIENT, "search: buffer too small");
    if (n == 1) {
        out[0] = static_cast<int32_t>(lower + width / 2);
        return CWLB_OK;
    }
    for (int64_t i = 0; i < n; ++i)
        out[i] = static_cast<int32_t>(lower + (width * i + (n - 1) / 2) / (n - 1));
    return CWLB_OK;
}

// candidate_search_by_step (reference main.cpp:151-167).
cwlb_status cwlb_candidate_search_by_step(int32_t lower, int32_t upper, int32_t step,
                                          int32_t* out, int64_t capacity, int64_t* count)
{
    if (lower <= 0 || upper < lower || step <= 0)
        return cwlb::fail(CWLB_INVALID_ARG, "Invalid search interval or step.");
    const int64_t width = static_cast<int64_t>(upper) - lower;
    const int64_t n = width / step + 1 + (width % step != 0);
    if (n > kMaxSearchPoints)
        return cwlb::fail(CWLB_INVALID_ARG, "Search plan exceeds 10000 points; increase the step.");
    *count = n;
    if (n > capacity || !out) return cwlb::fail(CWLB_INSUFFICIENT, "search: buffer too small");
    int64_t i = 0;
    for (int64_t v = lower; v <= upper; v += step) out[i++] = static_cast<int32_t>(v);
    if (out[i - 1] != upper) out[i++] = upper;
    return CWLB_OK;
}

// save_costs_one_per_line (reference utils.cpp:1024-1075).
cwlb_status cwlb_save_costs(const cwlb_cost_params* p, const char* filepath, int append,
                            int precision)
{
    namespace fs = std::filesystem;
    if (!p || !filepath || !*filepath) return cwlb::fail(CWLB_IO_ERROR, "cost file: empty path");
    std::error_code ec;
    const fs::path path(filepath);
    if (path.has_parent_path()) {
        const fs::path dir = path.parent_path();
        if (fs::exists(dir, ec) && !fs::is_directory(dir, ec))
            return cwlb::fail(CWLB_IO_ERROR, "cost file: parent path is not a directory");
        if (!fs::exists(dir, ec)) {
            if (!fs::create_directories(dir, ec) && ec)
                return cwlb::fail(CWLB_IO_ERROR, "cost file: cannot create parent directory");
        }
    }
    std::ofstream ofs(path, std::ios::out | (append ? std::ios::app : std::ios::trunc));
    if (!ofs.is_open()) return cwlb::fail(CWLB_IO_ERROR, "cost file: cannot open for writing");
    ofs << std::fixed << std::setprecision(precision) << p->C_compute_ns << "\n"
        << p->C_load_ns << "\n"
        << p->C_store_ns << "\n"
        << p->C_atomic_ns << "\n";
    if (!ofs.good()) return cwlb::fail(CWLB_IO_ERROR, "cost file: write failed");
    return CWLB_OK;
}

// read_costs_one_per_line (reference utils.cpp:1077-1092).
cwlb_status cwlb_read_costs(cwlb_cost_params* out, const char* filepath)
{
    if (!out || !filepath) return cwlb::fail(CWLB_IO_ERROR, "cost file: null argument");
    std::ifstream ifs(filepath);
    if (!ifs.is_open()) return cwlb::fail(CWLB_IO_ERROR, std::string("cannot open cost file: ") + filepath);
    double v[4];
    for (double& x : v)
        if (!(ifs >> x)) return cwlb::fail(CWLB_IO_ERROR, std::string("malformed cost file: ") + filepath);
    out->C_compute_ns = v[0];
    out->C_load_ns = v[1];
    out->C_store_ns = v[2];
    out->C_atomic_ns = v[3];
    return CWLB_OK;
}

}  // extern "C"
