// Seeded synthetic workloads for the mean-aggregation SpMM: graphs as CSR
// (rows are sources, columns sorted and deduplicated within a row, unit edge
// values) and dense features in U[-1, 1).
//
// Every random draw comes from a counter-based generator (a splitmix64
// finaliser over seed, stream and counter), so the output does not depend on
// the thread count or schedule.  The reference ships no generators; it reads
// datasets from disk (data.cpp:18-118) and draws features with mt19937
// (main.cpp:324-336).  These generators make the synthetic configurations
// that the SpMM is measured and checked on.
#include <omp.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <vector>

namespace {

inline uint64_t mix64(uint64_t z)
{
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

inline uint64_t draw(uint64_t seed, uint64_t stream, uint64_t ctr)
{
    return mix64(mix64(seed ^ (stream * 0xD6E8FEB86659FD93ull)) + ctr);
}

// Uniform in [0, 1) with 53 random bits.
inline double u01(uint64_t x) { return static_cast<double>(x >> 11) * 0x1.0p-53; }

// Uniform in (0, 1]: safe for log().
inline double u01_open0(uint64_t x)
{
    return (static_cast<double>(x >> 11) + 1.0) * 0x1.0p-53;
}

struct EdgeList {
    std::vector<int32_t> src, dst;
};

}  // namespace

extern "C" {

struct synth_csr {
    int32_t n;
    int64_t nnz;
    int32_t* row_ptr;
    int32_t* col_idx;
};

void synth_free(synth_csr* g)
{
    std::free(g->row_ptr);
    std::free(g->col_idx);
    g->row_ptr = nullptr;
    g->col_idx = nullptr;
    g->n = 0;
    g->nnz = 0;
}

}  // extern "C"

namespace {

// Builds a CSR from an edge list: bucket by source, then sort and
// deduplicate each row.  Deterministic: rows are sorted after the parallel
// scatter.  Returns 0, or -1 when nnz would not fit int32.
int edges_to_csr(int32_t n, const EdgeList& e, synth_csr* out)
{
    const int64_t m = static_cast<int64_t>(e.src.size());
    std::vector<int64_t> cnt(static_cast<size_t>(n) + 1, 0);
    {
        std::vector<std::atomic<int64_t>> c(static_cast<size_t>(n));
        for (auto& x : c) x.store(0, std::memory_order_relaxed);
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < m; ++i)
            c[e.src[i]].fetch_add(1, std::memory_order_relaxed);
        for (int32_t i = 0; i < n; ++i) cnt[i + 1] = cnt[i] + c[i].load();
    }
    std::vector<int32_t> bucket(static_cast<size_t>(m));
    {
        std::vector<std::atomic<int64_t>> cur(static_cast<size_t>(n));
        for (int32_t i = 0; i < n; ++i) cur[i].store(cnt[i], std::memory_order_relaxed);
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < m; ++i) {
            int64_t p = cur[e.src[i]].fetch_add(1, std::memory_order_relaxed);
            bucket[p] = e.dst[i];
        }
    }
    std::vector<int64_t> deg(static_cast<size_t>(n) + 1, 0);
#pragma omp parallel for schedule(dynamic, 1024)
    for (int32_t r = 0; r < n; ++r) {
        int32_t* b = bucket.data() + cnt[r];
        int32_t* en = bucket.data() + cnt[r + 1];
        std::sort(b, en);
        deg[r + 1] = std::unique(b, en) - b;
    }
    for (int32_t r = 0; r < n; ++r) deg[r + 1] += deg[r];
    if (deg[n] > INT32_MAX) return -1;
    out->n = n;
    out->nnz = deg[n];
    out->row_ptr = static_cast<int32_t*>(std::malloc(sizeof(int32_t) * (static_cast<size_t>(n) + 1)));
    out->col_idx = static_cast<int32_t*>(std::malloc(sizeof(int32_t) * std::max<int64_t>(1, deg[n])));
    if (!out->row_ptr || !out->col_idx) return -2;
    for (int32_t r = 0; r <= n; ++r) out->row_ptr[r] = static_cast<int32_t>(deg[r]);
#pragma omp parallel for schedule(dynamic, 1024)
    for (int32_t r = 0; r < n; ++r)
        std::memcpy(out->col_idx + deg[r], bucket.data() + cnt[r],
                    sizeof(int32_t) * static_cast<size_t>(deg[r + 1] - deg[r]));
    return 0;
}

// Per-row generator run twice: a counting pass and a filling pass with the
// same draws.  gen(row, emit) calls emit(col) in ascending column order.
template <class Gen>
int rowwise_csr(int32_t n, Gen gen, synth_csr* out)
{
    std::vector<int64_t> rp(static_cast<size_t>(n) + 1, 0);
#pragma omp parallel for schedule(dynamic, 256)
    for (int32_t r = 0; r < n; ++r) {
        int64_t c = 0;
        gen(r, [&](int32_t) { ++c; });
        rp[r + 1] = c;
    }
    for (int32_t r = 0; r < n; ++r) rp[r + 1] += rp[r];
    if (rp[n] > INT32_MAX) return -1;
    out->n = n;
    out->nnz = rp[n];
    out->row_ptr = static_cast<int32_t*>(std::malloc(sizeof(int32_t) * (static_cast<size_t>(n) + 1)));
    out->col_idx = static_cast<int32_t*>(std::malloc(sizeof(int32_t) * std::max<int64_t>(1, rp[n])));
    if (!out->row_ptr || !out->col_idx) return -2;
    for (int32_t r = 0; r <= n; ++r) out->row_ptr[r] = static_cast<int32_t>(rp[r]);
#pragma omp parallel for schedule(dynamic, 256)
    for (int32_t r = 0; r < n; ++r) {
        int32_t* p = out->col_idx + rp[r];
        gen(r, [&](int32_t c) { *p++ = c; });
    }
    return 0;
}

// Visits the positions of Bernoulli(p) successes in [0, len) in ascending
// order by geometric skipping; ctr is advanced per draw.
template <class F>
void bernoulli_positions(int64_t len, double p, uint64_t seed, uint64_t stream,
                         uint64_t& ctr, F f)
{
    if (p <= 0.0 || len <= 0) return;
    if (p >= 1.0) {
        for (int64_t i = 0; i < len; ++i) f(i);
        return;
    }
    const double lq = std::log1p(-p);
    int64_t pos = -1;
    for (;;) {
        const double u = u01_open0(draw(seed, stream, ctr++));
        const double skip = std::floor(std::log(u) / lq);
        if (skip >= static_cast<double>(len)) return;
        pos += 1 + static_cast<int64_t>(skip);
        if (pos >= len) return;
        f(pos);
    }
}

}  // namespace

extern "C" {

// Erdos-Renyi: row i includes each column j != i independently with
// probability avg_deg / (n - 1).  exact_pairs != 0 draws one value per pair
// (O(n^2), used for small n); otherwise geometric skipping.
int synth_erdos_renyi(int32_t n, double avg_deg, uint64_t seed, int exact_pairs, synth_csr* out)
{
    if (n <= 0) return -3;
    const double p = n > 1 ? avg_deg / static_cast<double>(n - 1) : 0.0;
    if (exact_pairs) {
        const uint64_t thr = p >= 1.0 ? UINT64_MAX
                                      : static_cast<uint64_t>(std::ldexp(p, 64));
        return rowwise_csr(n, [&](int32_t r, auto emit) {
            for (int32_t j = 0; j < n; ++j) {
                if (j == r) continue;
                if (draw(seed, static_cast<uint64_t>(r), static_cast<uint64_t>(j)) < thr) emit(j);
            }
        }, out);
    }
    return rowwise_csr(n, [&](int32_t r, auto emit) {
        uint64_t ctr = 0;
        bernoulli_positions(n - 1, p, seed, static_cast<uint64_t>(r), ctr, [&](int64_t i) {
            emit(static_cast<int32_t>(i < r ? i : i + 1));
        });
    }, out);
}

// Chung-Lu: weights w_i = (i+1)^(-1/(gamma-1)) scaled so that the expected
// out-degree sums to avg_deg * n, with every weight capped at max_deg (the
// uncapped weights are rescaled until the total holds).  avg_deg * n
// (source, destination) pairs are drawn with both ends ~ w; duplicates are
// removed.
int synth_chung_lu(int32_t n, double avg_deg, double gamma, double max_deg, uint64_t seed,
                   synth_csr* out)
{
    if (n <= 0 || gamma <= 1.0) return -3;
    std::vector<double> base(static_cast<size_t>(n)), w(static_cast<size_t>(n));
    const double ex = -1.0 / (gamma - 1.0);
    for (int32_t i = 0; i < n; ++i) base[i] = std::pow(static_cast<double>(i) + 1.0, ex);
    const double total = avg_deg * static_cast<double>(n);
    // Weights decrease with i, so the capped set is a prefix [0, k).
    int32_t k = 0;
    double scale = 0.0;
    for (int it = 0; it < 64; ++it) {
        double rest = 0.0;
        for (int32_t i = k; i < n; ++i) rest += base[i];
        scale = (total - max_deg * k) / rest;
        int32_t k2 = k;
        while (k2 < n && base[k2] * scale > max_deg) ++k2;
        if (k2 == k) break;
        k = k2;
    }
    for (int32_t i = 0; i < n; ++i) w[i] = i < k ? max_deg : base[i] * scale;
    std::vector<double> cdf(static_cast<size_t>(n));
    double acc = 0.0;
    for (int32_t i = 0; i < n; ++i) {
        acc += w[i];
        cdf[i] = acc;
    }
    const int64_t m = static_cast<int64_t>(std::llround(total));
    EdgeList e;
    e.src.resize(static_cast<size_t>(m));
    e.dst.resize(static_cast<size_t>(m));
    auto pick = [&](uint64_t x) {
        const double t = u01(x) * acc;
        int32_t i = static_cast<int32_t>(std::upper_bound(cdf.begin(), cdf.end(), t) - cdf.begin());
        return i < n ? i : n - 1;
    };
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < m; ++i) {
        e.src[i] = pick(draw(seed, 1, static_cast<uint64_t>(i)));
        e.dst[i] = pick(draw(seed, 2, static_cast<uint64_t>(i)));
    }
    return edges_to_csr(n, e, out);
}

// Stochastic block model: n_blocks equal blocks; row i links to each other
// node of its own block with probability p_in and to each node of another
// block with probability p_out (no self-loops).
int synth_sbm(int32_t n, int32_t n_blocks, double p_in, double p_out, uint64_t seed,
              synth_csr* out)
{
    if (n <= 0 || n_blocks <= 0 || n % n_blocks != 0) return -3;
    const int32_t bs = n / n_blocks;
    return rowwise_csr(n, [&](int32_t r, auto emit) {
        uint64_t ctr = 0;
        const int32_t rb = r / bs;
        for (int32_t b = 0; b < n_blocks; ++b) {
            const int32_t base = b * bs;
            if (b == rb) {
                const int32_t self = r - base;
                bernoulli_positions(bs - 1, p_in, seed, static_cast<uint64_t>(r), ctr,
                                    [&](int64_t i) {
                                        emit(base + static_cast<int32_t>(i < self ? i : i + 1));
                                    });
            } else {
                bernoulli_positions(bs, p_out, seed, static_cast<uint64_t>(r), ctr,
                                    [&](int64_t i) { emit(base + static_cast<int32_t>(i)); });
            }
        }
    }, out);
}

// R-MAT: `edges` samples over 2^scale nodes; at each level the quadrant is
// (0,0) with probability a, (0,1) with b, (1,0) with c, (1,1) otherwise.
// Node ids are relabelled by a seeded random permutation when relabel != 0
// (otherwise the hubs cluster at id 0); duplicates are removed, self-loops
// kept.
int synth_rmat(int32_t scale, int64_t edges, double a, double b, double c, uint64_t seed,
               int relabel, synth_csr* out)
{
    if (scale <= 0 || scale > 30 || edges < 0) return -3;
    const int32_t n = 1 << scale;
    EdgeList e;
    e.src.resize(static_cast<size_t>(edges));
    e.dst.resize(static_cast<size_t>(edges));
    const double ab = a + b, abc = a + b + c;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < edges; ++i) {
        int32_t s = 0, d = 0;
        for (int32_t l = 0; l < scale; ++l) {
            const double u = u01(draw(seed, static_cast<uint64_t>(l) + 16, static_cast<uint64_t>(i)));
            int32_t sb = 0, db = 0;
            if (u < a) {
            } else if (u < ab) {
                db = 1;
            } else if (u < abc) {
                sb = 1;
            } else {
                sb = 1;
                db = 1;
            }
            s = (s << 1) | sb;
            d = (d << 1) | db;
        }
        e.src[i] = s;
        e.dst[i] = d;
    }
    if (relabel) {
        std::vector<int32_t> perm(static_cast<size_t>(n));
        for (int32_t i = 0; i < n; ++i) perm[i] = i;
        for (int32_t i = n - 1; i > 0; --i) {
            const uint64_t x = draw(seed, 3, static_cast<uint64_t>(i));
            const int32_t j = static_cast<int32_t>(x % static_cast<uint64_t>(i + 1));
            std::swap(perm[i], perm[j]);
        }
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < edges; ++i) {
            e.src[i] = perm[e.src[i]];
            e.dst[i] = perm[e.dst[i]];
        }
    }
    return edges_to_csr(n, e, out);
}

// 2D mesh with shortcuts: a side x side lattice (node y*side + x); each of
// the four directed lattice edges of a node is kept with probability
// p_keep; `shortcuts` extra (source, destination) pairs are drawn
// uniformly.  Duplicates are removed.
int synth_mesh(int32_t side, double p_keep, int64_t shortcuts, uint64_t seed, synth_csr* out)
{
    if (side <= 0) return -3;
    const int64_t n64 = static_cast<int64_t>(side) * side;
    if (n64 > INT32_MAX) return -3;
    const int32_t n = static_cast<int32_t>(n64);
    const uint64_t thr = p_keep >= 1.0 ? UINT64_MAX
                                       : static_cast<uint64_t>(std::ldexp(p_keep, 64));
    // Count lattice edges per node, then fill.
    std::vector<uint8_t> keep(static_cast<size_t>(n));
#pragma omp parallel for schedule(static)
    for (int32_t v = 0; v < n; ++v) {
        const int32_t y = v / side, x = v % side;
        uint8_t mask = 0;
        const bool ok[4] = {y > 0, y + 1 < side, x > 0, x + 1 < side};
        for (int dir = 0; dir < 4; ++dir)
            if (ok[dir] && draw(seed, 4, static_cast<uint64_t>(v) * 4 + dir) < thr) mask |= 1u << dir;
        keep[v] = mask;
    }
    int64_t lattice = 0;
    for (int32_t v = 0; v < n; ++v) lattice += __builtin_popcount(keep[v]);
    EdgeList e;
    e.src.resize(static_cast<size_t>(lattice + shortcuts));
    e.dst.resize(static_cast<size_t>(lattice + shortcuts));
    std::vector<int64_t> off(static_cast<size_t>(n) + 1, 0);
    for (int32_t v = 0; v < n; ++v) off[v + 1] = off[v] + __builtin_popcount(keep[v]);
#pragma omp parallel for schedule(static)
    for (int32_t v = 0; v < n; ++v) {
        int64_t p = off[v];
        const int32_t nb[4] = {v - side, v + side, v - 1, v + 1};
        for (int dir = 0; dir < 4; ++dir)
            if (keep[v] & (1u << dir)) {
                e.src[p] = v;
                e.dst[p] = nb[dir];
                ++p;
            }
    }
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < shortcuts; ++i) {
        e.src[lattice + i] = static_cast<int32_t>(draw(seed, 5, static_cast<uint64_t>(i)) % static_cast<uint64_t>(n));
        e.dst[lattice + i] = static_cast<int32_t>(draw(seed, 6, static_cast<uint64_t>(i)) % static_cast<uint64_t>(n));
    }
    return edges_to_csr(n, e, out);
}

// Features in U[-1, 1): value(idx) for idx = row * K + k is
// (int(top 24 bits of mix64(mix64(seed) + idx)) - 2^23) * 2^-23, exact in
// float.  The device generator in libcwlb computes the same bits.
void synth_features(int64_t rows, int32_t K, uint64_t seed, float* out)
{
    const uint64_t s = mix64(seed);
    const int64_t total = rows * static_cast<int64_t>(K);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < total; ++i) {
        const uint64_t x = mix64(s + static_cast<uint64_t>(i));
        const int32_t u = static_cast<int32_t>(x >> 40);
        out[i] = static_cast<float>(u - 8388608) * 0x1.0p-23f;
    }
}

int synth_max_threads(void) { return omp_get_max_threads(); }

}  // extern "C"
