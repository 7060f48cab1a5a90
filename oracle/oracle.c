/*
 * oracle.c -- CPU restatement of CWLB-SpMM's FP32 mean-aggregation path.
 *
 * TEST INFRASTRUCTURE ONLY: tests/, the smoke check of __graft_entry__ and
 * the cpu_baseline leg of bench.py load it.  The
 * product path (libcwlb.so) never links, loads or calls it.
 *
 * Each function names the reference file:line it restates.  How each one is
 * pinned (reference extract, closed forms, hand-derived known answers,
 * brute force) is stated next to it; nothing here is "parity unpinned".
 *
 * Build: oracle/Makefile (gcc, -O2, -ffp-contract=off so that double
 * arithmetic in the partitioner is plain IEEE; fmaf() is the correctly
 * rounded libm/hardware fma).
 */
#include <limits.h>
#include <math.h>
#include <stdatomic.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* A deliberately planted mistake, used only by tests that show the checks
 * catch it (0 = faithful restatement).  1: next-row prefix absorption
 * disabled; 2: current-row prefix absorption disabled; 3: strict '<' in the
 * packing rule; 4: divide by chunk length instead of full degree;
 * 5: reorder ties broken by descending id; 7: atomic calibration divides
 * by the group target instead of the rounded-up writer groups. */
static int g_mutation = 0;
void oracle_set_mutation(int m) { g_mutation = m; }

/* ------------------------------------------------------------------------
 * Degree reordering: main.cpp:197-278 (sortCSRByDegreeDPLCPU).
 * Rows sorted by (degree, original id) ascending (main.cpp:229-238); offsets
 * are the inclusive scan of sorted degrees (main.cpp:247-253); each row's
 * entries are copied in their original order (main.cpp:257-272).  The
 * comparator is a strict total order, so any correct sort gives this
 * permutation; a stable counting sort by degree is used here.
 * Pinned by: numpy stable argsort (closed form) in tests.
 * Returns 0, or -1 when ColInd/Value sizes disagree with RowOffset.
 * ---------------------------------------------------------------------- */
int oracle_reorder_by_degree(int n, const int *rp, const int *ci,
                             const float *val, int *origin, int *rp_out,
                             int *ci_out, float *val_out)
{
    if (n <= 0) {
        if (rp_out) rp_out[0] = 0;
        return 0;
    }
    int maxdeg = 0;
    for (int i = 0; i < n; ++i) {
        int d = rp[i + 1] - rp[i];
        if (d > maxdeg) maxdeg = d;
    }
    long *start = (long *)calloc((size_t)maxdeg + 2, sizeof(long));
    if (!start) return -2;
    for (int i = 0; i < n; ++i) start[rp[i + 1] - rp[i] + 1]++;
    for (int d = 0; d <= maxdeg; ++d) start[d + 1] += start[d];
    if (g_mutation == 5) {
        for (int i = n - 1; i >= 0; --i) origin[start[rp[i + 1] - rp[i]]++] = i;
    } else {
        for (int i = 0; i < n; ++i) origin[start[rp[i + 1] - rp[i]]++] = i;
    }
    free(start);
    rp_out[0] = 0;
    for (int r = 0; r < n; ++r) {
        int o = origin[r];
        rp_out[r + 1] = rp_out[r] + (rp[o + 1] - rp[o]);
    }
    for (int r = 0; r < n; ++r) {
        int o = origin[r];
        int len = rp[o + 1] - rp[o];
        memcpy(ci_out + rp_out[r], ci + rp[o], (size_t)len * sizeof(int));
        memcpy(val_out + rp_out[r], val + rp[o], (size_t)len * sizeof(float));
    }
    if (rp_out[n] != rp[n]) return -1;
    return 0;
}

/* ------------------------------------------------------------------------
 * Cost-weighted task partitioning: utils.cpp:832-1021.
 * full row weight wCL*deg + Cs (utils.cpp:850-852); segment weight
 * wCL*nnz + Ca (utils.cpp:854-856); S recovered from the capacity
 * (utils.cpp:859-864); greedy packing (utils.cpp:946-958); current-row
 * prefix absorption (utils.cpp:879-912); next-row prefix absorption
 * (utils.cpp:915-939); splitting (utils.cpp:960-1012); flush
 * (utils.cpp:1016-1018).  Sequential IEEE double, same operation order.
 * Pinned by: the reference extract (oracle/_ref), the hand-derived known
 * answers and the tiling invariants in tests.
 * Writes up to out_cap tasks (4 ints each) and returns the task count.
 * ---------------------------------------------------------------------- */
typedef struct {
    int *buf;
    long cap;
    long n;
} task_sink;

static void emit(task_sink *t, int s, int e, int fo, int last)
{
    if (s < e) {
        if (t->n < t->cap) {
            t->buf[4 * t->n + 0] = s;
            t->buf[4 * t->n + 1] = e;
            t->buf[4 * t->n + 2] = fo;
            t->buf[4 * t->n + 3] = last;
        }
        t->n++;
    }
}

/* static_cast<int>(double) as x86-64 executes it: out-of-range and NaN
 * inputs give INT_MIN (cvttsd2si). */
static int trunc_to_int_x86(double x)
{
    if (x != x) return INT_MIN;
    if (x >= 2147483648.0 || x <= -2147483649.0) return INT_MIN;
    return (int)x;
}

typedef struct {
    const int *rp;
    int n;
    double wCL, Cs, Ca, cap;
    int S;
    int g_start, first_off;
    double acc;
    task_sink *sink;
} part_state;

static double full_w(const part_state *p, int r)
{
    return p->wCL * (double)(p->rp[r + 1] - p->rp[r]) + p->Cs;
}

static double chunk_w(const part_state *p, int nnz)
{
    return p->wCL * (double)nnz + p->Ca;
}

static void absorb_current_prefix(part_state *p, int row_deg, int row_idx,
                                  int *remaining, int *off)
{
    if (p->acc <= 0.0) return;
    int r = row_deg % p->S;
    if (g_mutation == 2) r = 0;
    if (r == 0 || r >= row_deg) {
        emit(p->sink, p->g_start, row_idx, p->first_off, 0);
        p->g_start = row_idx;
        p->first_off = 0;
        p->acc = 0.0;
        return;
    }
    double w = chunk_w(p, r);
    double rem = p->cap - p->acc;
    if (w <= rem) {
        emit(p->sink, p->g_start, row_idx + 1, p->first_off, r);
        p->g_start = row_idx;
        p->first_off = r;
        p->acc = 0.0;
        *remaining -= r;
        *off += r;
    } else {
        emit(p->sink, p->g_start, row_idx, p->first_off, 0);
        p->g_start = row_idx;
        p->first_off = 0;
        p->acc = 0.0;
    }
}

static int absorb_next_prefix(part_state *p, int cur_row)
{
    if (g_mutation == 1) return 0;
    if (p->acc >= p->cap) return 0;
    if (cur_row + 1 >= p->n) return 0;
    int nr = cur_row + 1;
    int nd = p->rp[nr + 1] - p->rp[nr];
    if (full_w(p, nr) <= p->cap) return 0;
    int r2 = nd % p->S;
    if (r2 == 0 || r2 >= nd) return 0;
    double w = chunk_w(p, r2);
    double rem = p->cap - p->acc;
    if (w > rem) return 0;
    emit(p->sink, p->g_start, nr + 1, p->first_off, r2);
    p->g_start = nr;
    p->first_off = r2;
    p->acc = 0.0;
    return 1;
}

long oracle_partition(const int *rp, long rp_len, double Cc, double Cl,
                      double Cs, double Ca, double capacity, int *out,
                      long out_cap)
{
    task_sink sink = {out, out_cap, 0};
    int n = (int)(rp_len - 1);
    if (n <= 0) return 0;
    part_state p;
    p.rp = rp;
    p.n = n;
    p.wCL = Cc + Cl;
    p.Cs = Cs;
    p.Ca = Ca;
    p.cap = capacity;
    {
        double denom = p.wCL > 1e-30 ? p.wCL : 1e-30;
        int s = trunc_to_int_x86(floor((capacity - Ca) / denom));
        p.S = s > 1 ? s : 1;
    }
    p.g_start = 0;
    p.first_off = 0;
    p.acc = 0.0;
    p.sink = &sink;

    int row = 0;
    while (row < n) {
        int deg = rp[row + 1] - rp[row];
        double wr = full_w(&p, row);
        int fits = (g_mutation == 3) ? (wr < capacity) : (wr <= capacity);
        if (fits) {
            int pack = (g_mutation == 3) ? (p.acc + wr < capacity)
                                         : (p.acc + wr <= capacity);
            if (p.acc == 0.0 || pack) {
                p.acc += wr;
                ++row;
                continue;
            }
            emit(&sink, p.g_start, row, p.first_off, 0);
            p.g_start = row;
            p.first_off = 0;
            p.acc = 0.0;
            continue;
        }
        int off = 0;
        int has_prefix = (p.acc == 0.0 && p.g_start == row && p.first_off > 0);
        if (has_prefix) off = p.first_off;
        int remaining = deg - off;
        if (remaining <= 0) {
            p.g_start = row + 1;
            p.first_off = 0;
            p.acc = 0.0;
            ++row;
            continue;
        }
        if (!has_prefix) absorb_current_prefix(&p, deg, row, &remaining, &off);
        while (remaining > 0) {
            int take = remaining < p.S ? remaining : p.S;
            double w = chunk_w(&p, take);
            p.acc += w;
            remaining -= take;
            off += take;
            if (remaining > 0) {
                emit(&sink, p.g_start, row + 1, p.first_off, off);
                p.g_start = row;
                p.first_off = off;
                p.acc = 0.0;
                continue;
            }
            if (!absorb_next_prefix(&p, row)) {
                emit(&sink, p.g_start, row + 1, p.first_off, 0);
                p.g_start = row + 1;
                p.first_off = 0;
                p.acc = 0.0;
            }
        }
        ++row;
    }
    if (p.acc > 0.0 || p.g_start < n) emit(&sink, p.g_start, n, p.first_off, 0);
    return sink.n;
}

/* ------------------------------------------------------------------------
 * Segment-size selection: main.cpp:87-95, 109-167, 281-321.
 * Pinned by: the reference extract and README.md:289,306-310,342-345,369-376.
 * ---------------------------------------------------------------------- */
double oracle_capacity_from_s(int s, double Cc, double Cl, double Cs, double Ca)
{
    (void)Cs;
    double edge = Cc + Cl;
    int cs = s > 1 ? s : 1;
    if (edge <= 0.0) return Ca > 0.0 ? Ca : 0.0;
    double c = Ca + edge * (double)cs;
    return c > 0.0 ? c : 0.0;
}

/* Returns S, or -1 for non-positive compute_units / wave (the reference
 * throws invalid_argument). rp_len == 0 means an empty RowOffset. */
int oracle_wave_based_s(unsigned long long nnz, long rp_len, int cu, int wave)
{
    if (cu <= 0 || wave <= 0) return -1;
    if (rp_len == 0) return 1;
    unsigned long long den = (unsigned long long)cu * (unsigned long long)wave;
    unsigned long long s = (nnz + den - 1) / den;
    if (s < 1) s = 1;
    if (s > (unsigned long long)INT_MAX) s = INT_MAX;
    return (int)s;
}

void oracle_recommended_candidate_w(unsigned long long nnz, int *w3)
{
    static const unsigned long long lim[6] = {100000ULL, 500000ULL, 1000000ULL,
                                              5000000ULL, 10000000ULL,
                                              50000000ULL};
    static const int first[7] = {64, 128, 256, 512, 1024, 4096, 8192};
    int i = 0;
    while (i < 6 && nnz >= lim[i]) ++i;
    w3[0] = first[i];
    w3[1] = first[i] / 2;
    w3[2] = first[i] / 4;
}

int oracle_candidate_search_bounds(const int *v, long best, int *lo, int *hi)
{
    if (best < 0 || best >= 3 || v[0] <= 0 || v[1] < v[0] || v[2] < v[1])
        return 1;
    long long lower = v[0], upper = v[2];
    if (best == 0) {
        lower = 2LL * v[0] - v[1];
        upper = v[1];
    } else if (best == 2) {
        lower = v[1];
        upper = 2LL * v[2] - v[1];
    }
    if (lower < 1) lower = 1;
    if (upper > INT_MAX) upper = INT_MAX;
    *lo = (int)lower;
    *hi = (int)upper;
    return 0;
}

#define ORACLE_MAX_SEARCH_POINTS 10000

long oracle_candidate_search_by_count(int lo, int hi, int req, int *out,
                                      long cap, int *err)
{
    *err = 0;
    if (lo <= 0 || hi < lo || req <= 0) {
        *err = 1;
        return 0;
    }
    long long width = (long long)hi - lo;
    long long count = req < width + 1 ? req : width + 1;
    if (count > ORACLE_MAX_SEARCH_POINTS) {
        *err = 1;
        return 0;
    }
    if (count == 1) {
        if (cap > 0) out[0] = (int)(lo + width / 2);
        return 1;
    }
    for (long long i = 0; i < count; ++i) {
        long long off = (width * i + (count - 1) / 2) / (count - 1);
        if (i < cap) out[i] = (int)(lo + off);
    }
    return (long)count;
}

long oracle_candidate_search_by_step(int lo, int hi, int step, int *out,
                                     long cap, int *err)
{
    *err = 0;
    if (lo <= 0 || hi < lo || step <= 0) {
        *err = 1;
        return 0;
    }
    long long width = (long long)hi - lo;
    long long count = width / step + 1 + (width % step != 0);
    if (count > ORACLE_MAX_SEARCH_POINTS) {
        *err = 1;
        return 0;
    }
    long n = 0;
    long long last = lo;
    for (long long v = lo; v <= hi; v += step) {
        if (n < cap) out[n] = (int)v;
        last = v;
        ++n;
    }
    if (last != hi) {
        if (n < cap) out[n] = hi;
        ++n;
    }
    return n;
}

/* ------------------------------------------------------------------------
 * Mean aggregation, reference value order: parallelMatrix.cpp:148-236.
 * For each task in order, each row chunk [begin,end) (clamps :169-176):
 * acc_k = fma(val, H[col][k], acc) in CSR order (:207-211), acc /= deg
 * (:219), then C[origin[r]][k] = acc for a full row (:223-225) or += acc
 * for a partial one (:226-234; sequential task order is one legal order of
 * the reference's relaxed atomics).  C starts at zero (:112); rows with
 * deg <= 0 are skipped (:167).  K == 0 or no tasks leave C zero (:80-83,
 * :101-104).
 * Pinned by: the fp64 closed form C[o] = (A H)[o] / deg, scipy, brute-force
 * dense products for tiny graphs, and exact special cases (deg-1 rows,
 * all-ones H, K = 1) in tests.
 * ---------------------------------------------------------------------- */
static void row_chunk(const int *rp, int r, int row_s, int row_e, int fo,
                      int last, int *b, int *e, int *deg)
{
    int d = rp[r + 1] - rp[r];
    int begin = (r == row_s) ? fo : 0;
    int end = d;
    if (r == row_e - 1 && last > 0) end = last;
    if (begin < 0) begin = 0;
    if (begin > d) begin = d;
    if (end < begin) end = begin;
    if (end > d) end = d;
    *b = begin;
    *e = end;
    *deg = d;
}

void oracle_spmm_mean_f32(int n_rows, const int *rp, const int *ci,
                          const float *val, const int *origin, const float *H,
                          int K, const int *tasks, long n_tasks, float *C)
{
    memset(C, 0, (size_t)n_rows * (size_t)(K > 0 ? K : 0) * sizeof(float));
    if (K <= 0) return;
    float *acc = (float *)malloc((size_t)K * sizeof(float));
    for (long t = 0; t < n_tasks; ++t) {
        int rs = tasks[4 * t], re = tasks[4 * t + 1];
        int fo = tasks[4 * t + 2], ln = tasks[4 * t + 3];
        for (int r = rs; r < re; ++r) {
            int b, e, d;
            row_chunk(rp, r, rs, re, fo, ln, &b, &e, &d);
            if (d <= 0 || b >= e) continue;
            for (int k = 0; k < K; ++k) acc[k] = 0.0f;
            for (int j = rp[r] + b; j < rp[r] + e; ++j) {
                const float *h = H + (size_t)ci[j] * (size_t)K;
                float a = val[j];
                for (int k = 0; k < K; ++k) acc[k] = fmaf(a, h[k], acc[k]);
            }
            float div = (g_mutation == 4) ? (float)(e - b) : (float)d;
            float *c = C + (size_t)origin[r] * (size_t)K;
            if (b == 0 && e == d) {
                for (int k = 0; k < K; ++k) c[k] = acc[k] / div;
            } else {
                for (int k = 0; k < K; ++k) c[k] += acc[k] / div;
            }
        }
    }
    free(acc);
}

/* Closed form in double from the ORIGINAL (unreordered) CSR:
 * C[i][k] = sum_j val_ij H[col_ij][k] / deg(i), 0 when deg(i) == 0.
 * Independent of the permutation and the partition. */
void oracle_spmm_mean_f64(int n, const int *rp, const int *ci,
                          const float *val, const float *H, int K, double *C)
{
    for (int i = 0; i < n; ++i) {
        double *c = C + (size_t)i * (size_t)K;
        for (int k = 0; k < K; ++k) c[k] = 0.0;
        int d = rp[i + 1] - rp[i];
        if (d <= 0) continue;
        for (int j = rp[i]; j < rp[i + 1]; ++j) {
            const float *h = H + (size_t)ci[j] * (size_t)K;
            double a = (double)val[j];
            for (int k = 0; k < K; ++k) c[k] += a * (double)h[k];
        }
        for (int k = 0; k < K; ++k) c[k] /= (double)d;
    }
}

/* ------------------------------------------------------------------------
 * CPU baseline: the reference kernel's semantics (parallelMatrix.cpp:148-236)
 * restated with OpenMP: one task per loop iteration, dynamic schedule, per
 * feature fma in CSR order, IEEE divide, direct store for full rows and a
 * CAS-loop float atomic add for partial rows.  C must be zero on entry.
 * Timed by bench.py as the reported CPU figure; checked against
 * oracle_spmm_mean_f32 in tests.
 * ---------------------------------------------------------------------- */
static inline void atomic_add_f32(float *addr, float v)
{
    _Atomic uint32_t *p = (_Atomic uint32_t *)addr;
    uint32_t old = atomic_load_explicit(p, memory_order_relaxed);
    for (;;) {
        float f;
        memcpy(&f, &old, sizeof f);
        f += v;
        uint32_t nw;
        memcpy(&nw, &f, sizeof nw);
        if (atomic_compare_exchange_weak_explicit(p, &old, nw,
                                                  memory_order_relaxed,
                                                  memory_order_relaxed))
            return;
    }
}

__attribute__((target_clones("arch=haswell", "default")))
void oracle_spmm_mean_f32_omp(int n_rows, const int *rp, const int *ci,
                              const float *val, const int *origin,
                              const float *H, int K, const int *tasks,
                              long n_tasks, float *C, int threads)
{
    (void)n_rows;
    if (K <= 0) return;
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#else
    (void)threads;
#endif
#pragma omp parallel
    {
        float *acc = (float *)malloc((size_t)K * sizeof(float));
#pragma omp for schedule(dynamic, 16)
        for (long t = 0; t < n_tasks; ++t) {
            int rs = tasks[4 * t], re = tasks[4 * t + 1];
            int fo = tasks[4 * t + 2], ln = tasks[4 * t + 3];
            for (int r = rs; r < re; ++r) {
                int b, e, d;
                row_chunk(rp, r, rs, re, fo, ln, &b, &e, &d);
                if (d <= 0 || b >= e) continue;
                for (int k = 0; k < K; ++k) acc[k] = 0.0f;
                for (int j = rp[r] + b; j < rp[r] + e; ++j) {
                    const float *h = H + (size_t)ci[j] * (size_t)K;
                    float a = val[j];
                    for (int k = 0; k < K; ++k) acc[k] = fmaf(a, h[k], acc[k]);
                }
                float fd = (float)d;
                float *c = C + (size_t)origin[r] * (size_t)K;
                if (b == 0 && e == d) {
                    for (int k = 0; k < K; ++k) c[k] = acc[k] / fd;
                } else {
                    for (int k = 0; k < K; ++k) atomic_add_f32(&c[k], acc[k] / fd);
                }
            }
        }
        free(acc);
    }
}

int oracle_max_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------------
 * Calibration normalisation: utils.cpp:419-421 (compute), 522-524 (load),
 * 583-585 (store): C = ((mean_ms * 1e6) / WI) / K * 10, i.e. ns per op per
 * work-item x 10; utils.cpp:597-640 and 791-806 (atomic): K_block =
 * min(K, 128) rounded down to a multiple of 32 (32 when that is 0), writer
 * groups = the smallest multiple of `writers` (>= 1) that reaches
 * ceil(WI / 128) (at least `writers`), ops = groups * K_block,
 * C_atomic = (mean_ms * 1e6) / ops * 10.  ms[] = compute, load, store,
 * atomic mean launch times; out[] the four coefficients; ops[] the divisors.
 * Pinned by hand-derived known answers in tests (exact binary fractions).
 * ---------------------------------------------------------------------- */
void oracle_cost_coefficients(const double *ms, int K, int WI, int writers,
                              double *out, long long *ops)
{
    for (int i = 0; i < 3; ++i) {
        double per_wi = (ms[i] * 1e6) / (double)WI;
        out[i] = per_wi / (double)K * 10;
        ops[i] = (long long)WI * K;
    }
    int gpr = writers > 1 ? writers : 1;
    int kb = K < 128 ? K : 128;
    kb = (kb / 32) * 32;
    if (kb <= 0) kb = 32;
    int target = (WI + 127) / 128;
    if (target < 1) target = 1;
    int G = target / gpr;
    if (G < 1) G = 1;
    long long groups = (long long)G * gpr;
    while (groups < target) {
        ++G;
        groups = (long long)G * gpr;
    }
    if (g_mutation == 7) groups = target;
    double n_ops = (double)groups * (double)kb;
    out[3] = (ms[3] * 1.0e6) / n_ops * 10.0;
    ops[3] = groups * kb;
}

/* ------------------------------------------------------------------------
 * Cost file: utils.cpp:1024-1092.  Four lines, compute/load/store/atomic,
 * std::fixed with `precision` decimals; truncating (or appending) write;
 * the parent directory is created; a parent path that is a file fails.
 * Reading takes four whitespace-separated doubles.
 * Pinned by: the reference extract (byte-identical files) in tests.
 * ---------------------------------------------------------------------- */
int oracle_format_costs(const double *c4, int precision, char *buf, long cap)
{
    int n = snprintf(buf, (size_t)cap, "%.*f\n%.*f\n%.*f\n%.*f\n", precision,
                     c4[0], precision, c4[1], precision, c4[2], precision,
                     c4[3]);
    return n;
}

int oracle_parse_costs(const char *text, double *c4)
{
    char *end = NULL;
    const char *p = text;
    for (int i = 0; i < 4; ++i) {
        double v = strtod(p, &end);
        if (end == p) return 0;
        c4[i] = v;
        p = end;
    }
    return 1;
}
