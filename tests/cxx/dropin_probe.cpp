// Test driver of the C++17 drop-in layer (include/config.h, Matrix.h,
// utils.h, parallelMatrix.h, data.h, cwlb_driver.h): each subcommand calls
// the drop-in functions on inputs read from raw little-endian files and
// writes their outputs the same way, so that the Python tests can compare
// them with the oracle.  Exceptions are reported on stdout as
//     EXC <kind> <message>
// with exit status 3 (kind: invalid_argument, runtime_error, overflow_error,
// out_of_range, bad_alloc, other).
//
// Subcommands (files are raw arrays; "csr" = int64 n, int64 nnz,
// int32 rp[n+1], int32 ci[nnz], float val[nnz]; "order" = int64 n,
// int64 nnz, int32 origin[n], int32 rp[n+1], int32 ci[nnz], float val[nnz]):
//   reorder-cpu CSR OUT_ORDER          sortCSRByDegreeDPLCPU
//   reorder-gpu CSR OUT_ORDER          sortCSRByDegree_HIP on device 0
//   partition ORDER CC CL CS CA S OUT  capacity_from_s + costWeightedTaskPartitioning
//                                      (OUT: float64 capacity, int32 tasks[T][4])
//   spmm ORDER H ROWS K TASKS OUT      spmmKernel or, for K > 1024,
//                                      spmmKernelLargeKFallback (prints time)
//   spmm-large ORDER H ROWS K TASKS OUT   spmmKernelLargeKFallback
//   run-single-s ORDER H ROWS K CC CL CS CA S OUT   run_single_s (prints average, schedule)
//   load DIR NAME                      loadDatasetToCSR from working directory DIR
//                                      (prints V E, then offsets and columns)
//   features ROWS COLS OUT             deterministic_features
//   dense2csr ROWS COLS DENSE OUT_CSR  CSR(const RowMajorMatrixXf&)
//   validate A B CSR DENSE ROWS COLS DROWS TOL   validate_custom_csr_result
//   select NNZ RP_LEN CU WAVE          wave_based_s, recommended_candidate_w
//   search LO HI MODE N                candidate_search_by_count / _by_step
//   bounds V0 V1 V2 BEST               candidate_search_bounds
//   posarg TEXT                        positive_search_argument
//   costs-save PATH APPEND PREC CC CL CS CA / costs-read PATH
//   device                             cwlb::Device properties
//   partition-gpu ORDER CC CL CS CA S OUT    costWeightedTaskPartitioning_HIP
//   partition-emul ORDER CC CL CS CA S OUT   the GPU partition's algorithm
//                                      (fresh-node transitions, pointer doubling,
//                                      chain expansion) run on the host
#include <climits>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <iostream>
#include <iterator>
#include <new>
#include <stdexcept>
#include <string>
#include <unistd.h>
#include <vector>

#include "cwlb_driver.h"
#include "data.h"
#include "partition_sim.h"
#include "parallelMatrix.h"
#include "utils.h"

namespace {

std::vector<char> read_file(const std::string& path)
{
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("probe: cannot open " + path);
    return std::vector<char>(std::istreambuf_iterator<char>(f), {});
}

struct Reader {
    std::vector<char> buf;
    std::size_t pos = 0;
    template <class T>
    std::vector<T> take(std::size_t n)
    {
        if (pos + n * sizeof(T) > buf.size()) throw std::runtime_error("probe: short input file");
        std::vector<T> v(n);
        if (n) std::copy(buf.data() + pos, buf.data() + pos + n * sizeof(T), reinterpret_cast<char*>(v.data()));
        pos += n * sizeof(T);
        return v;
    }
    int64_t i64() { return take<int64_t>(1)[0]; }
};

struct Writer {
    std::ofstream f;
    explicit Writer(const std::string& p) : f(p, std::ios::binary)
    {
        if (!f) throw std::runtime_error("probe: cannot write " + p);
    }
    template <class T>
    void put(const std::vector<T>& v)
    {
        f.write(reinterpret_cast<const char*>(v.data()), static_cast<std::streamsize>(v.size() * sizeof(T)));
    }
    template <class T>
    void one(T x)
    {
        f.write(reinterpret_cast<const char*>(&x), sizeof x);
    }
};

CSR read_csr(const std::string& path)
{
    Reader r{read_file(path)};
    const int64_t n = r.i64(), nnz = r.i64();
    CSR c;
    c.RowOffset = r.take<int>(static_cast<std::size_t>(n + 1));
    c.ColInd = r.take<int>(static_cast<std::size_t>(nnz));
    c.Value = r.take<float>(static_cast<std::size_t>(nnz));
    return c;
}

CSR_Order read_order(const std::string& path)
{
    Reader r{read_file(path)};
    const int64_t n = r.i64(), nnz = r.i64();
    CSR_Order c;
    c.Origin_local = r.take<int>(static_cast<std::size_t>(n));
    c.RowOffset = r.take<int>(static_cast<std::size_t>(n + 1));
    c.ColInd = r.take<int>(static_cast<std::size_t>(nnz));
    c.Value = r.take<float>(static_cast<std::size_t>(nnz));
    return c;
}

void write_order(const std::string& path, const CSR_Order& c)
{
    Writer w(path);
    w.one<int64_t>(static_cast<int64_t>(c.Origin_local.size()));
    w.one<int64_t>(static_cast<int64_t>(c.ColInd.size()));
    w.put(c.Origin_local);
    w.put(c.RowOffset);
    w.put(c.ColInd);
    w.put(c.Value);
}

Defined::RowMajorMatrixXf read_dense(const std::string& path, long rows, long cols)
{
    Reader r{read_file(path)};
    Defined::RowMajorMatrixXf m(rows, cols);
    const std::vector<float> v = r.take<float>(static_cast<std::size_t>(rows * cols));
    std::copy(v.begin(), v.end(), m.data());
    return m;
}

void write_dense(const std::string& path, const Defined::RowMajorMatrixXf& m)
{
    Writer w(path);
    w.f.write(reinterpret_cast<const char*>(m.data()), static_cast<std::streamsize>(m.size() * sizeof(float)));
}

std::vector<ParallelDataWeighted> read_tasks(const std::string& path)
{
    Reader r{read_file(path)};
    const std::vector<int> flat = r.take<int>(r.buf.size() / sizeof(int));
    std::vector<ParallelDataWeighted> t(flat.size() / 4);
    for (std::size_t i = 0; i < t.size(); ++i)
        t[i] = ParallelDataWeighted{flat[4 * i], flat[4 * i + 1], flat[4 * i + 2], flat[4 * i + 3]};
    return t;
}

SpmmCostParams costs_from(char** a)
{
    SpmmCostParams c;
    c.C_compute_ns = std::stod(a[0]);
    c.C_load_ns = std::stod(a[1]);
    c.C_store_ns = std::stod(a[2]);
    c.C_atomic_ns = std::stod(a[3]);
    return c;
}

// The GPU partition's steps (csrc/partition.hip) executed sequentially with
// the same per-node simulation, so the decomposition and the doubling are
// checked on the host.
std::vector<ParallelDataWeighted> partition_emulated(const std::vector<int>& rp,
                                                     const SpmmCostParams& c, double cap)
{
    namespace P = cwlb::part;
    const int n = static_cast<int>(rp.size()) - 1;
    std::vector<ParallelDataWeighted> out;
    if (n <= 0) return out;
    P::PartParams p{};
    p.rp = rp.data();
    p.n = n;
    p.wcl = c.C_compute_ns + c.C_load_ns;
    p.cs = c.C_store_ns;
    p.ca = c.C_atomic_ns;
    p.cap = cap;
    const double denom = (1e-30 < p.wcl) ? p.wcl : 1e-30;
    const double x = std::floor((cap - p.ca) / denom);
    int s = INT_MIN;
    if (x == x && x < 2147483648.0 && x > -2147483649.0) s = static_cast<int>(x);
    p.S = std::max(1, s);
    if (!(p.cs > 0.0) || !(p.wcl >= 0.0) || !std::isfinite(cap) || cap / p.cs > 65536.0)
        throw std::invalid_argument("partition-emul: unsupported costs");
    p.max_scan = static_cast<long long>(cap / p.cs * (1.0 + 1e-6)) + 4;
    std::vector<int> long_idx(static_cast<std::size_t>(n), -1), long_row;
    for (int r = 0; r < n; ++r)
        if (!(P::full_w(p, r) <= cap)) {
            long_idx[static_cast<std::size_t>(r)] = static_cast<int>(long_row.size());
            long_row.push_back(r);
        }
    p.long_row = long_row.data();
    p.long_idx = long_idx.data();
    const long long V = n + 1 + static_cast<long long>(long_row.size());
    std::vector<std::vector<int>> J(1, std::vector<int>(static_cast<std::size_t>(V)));
    std::vector<int> cnt(static_cast<std::size_t>(V));
    for (long long v = 0; v < V; ++v) {
        P::Emitter em{nullptr, 0};
        int overrun = 0;
        J[0][static_cast<std::size_t>(v)] = P::simulate(p, static_cast<int>(v), em, &overrun);
        cnt[static_cast<std::size_t>(v)] = static_cast<int>(em.count);
        if (overrun) throw std::runtime_error("partition-emul: scan overrun");
    }
    // As on the GPU: L levels with 2^(L-1) >= V, then the first level whose
    // jump from A(0) reaches the end (which L levels must contain).
    int L = 1;
    while ((1LL << (L - 1)) < V) ++L;
    while (static_cast<int>(J.size()) < L) {
        const std::vector<int>& a = J.back();
        std::vector<int> b(a.size());
        for (std::size_t v = 0; v < a.size(); ++v) b[v] = a[static_cast<std::size_t>(a[v])];
        J.push_back(std::move(b));
    }
    int levels = 0;
    for (int k = 0; k < L && levels == 0; ++k)
        if (J[static_cast<std::size_t>(k)][0] == n) levels = k + 1;
    if (levels == 0) throw std::runtime_error("partition-emul: chain too long");
    J.resize(static_cast<std::size_t>(levels));
    const long long len = 1LL << (J.size() - 1);
    std::vector<int> chain(static_cast<std::size_t>(len), 0);
    for (int j = static_cast<int>(J.size()) - 2; j >= 0; --j) {
        const long long half = 1LL << j;
        for (long long pos = 0; pos < len; pos += 2 * half)
            chain[static_cast<std::size_t>(pos + half)] =
                J[static_cast<std::size_t>(j)][static_cast<std::size_t>(chain[static_cast<std::size_t>(pos)])];
    }
    long long total = 0;
    std::vector<long long> off(static_cast<std::size_t>(len));
    for (long long i = 0; i < len; ++i) {
        off[static_cast<std::size_t>(i)] = total;
        const int v = chain[static_cast<std::size_t>(i)];
        if (v != n) total += cnt[static_cast<std::size_t>(v)];
    }
    std::vector<cwlb_task> tasks(static_cast<std::size_t>(total));
    for (long long i = 0; i < len; ++i) {
        const int v = chain[static_cast<std::size_t>(i)];
        if (v == n) continue;
        P::Emitter em{tasks.data() + off[static_cast<std::size_t>(i)], 0};
        int overrun = 0;
        (void)P::simulate(p, v, em, &overrun);
        if (em.count != cnt[static_cast<std::size_t>(v)])
            throw std::runtime_error("partition-emul: emitted and counted tasks differ");
    }
    for (const cwlb_task& t : tasks)
        out.push_back(ParallelDataWeighted{t.row_start, t.row_end, t.first_row_offset, t.last_row_nnz});
    return out;
}

int run(int argc, char** argv)
{
    if (argc < 2) throw std::invalid_argument("probe: no subcommand");
    const std::string cmd = argv[1];
    auto need = [&](int n) {
        if (argc != n + 2) throw std::invalid_argument("probe: " + cmd + " takes " + std::to_string(n) + " arguments");
    };
    std::cout.precision(9);
    if (cmd == "reorder-cpu" || cmd == "reorder-gpu") {
        need(2);
        const CSR csr = read_csr(argv[2]);
        if (cmd == "reorder-cpu") {
            write_order(argv[3], sortCSRByDegreeDPLCPU(csr));
        } else {
            cwlb::Device q(0);
            write_order(argv[3], sortCSRByDegree_HIP(csr, q));
        }
    } else if (cmd == "partition") {
        need(7);
        const CSR_Order o = read_order(argv[2]);
        const SpmmCostParams c = costs_from(argv + 3);
        const double cap = capacity_from_s(std::stoi(argv[7]), c);
        const std::vector<ParallelDataWeighted> t = costWeightedTaskPartitioning(o, c, cap);
        Writer w(argv[8]);
        w.one(cap);
        w.put(t);
    } else if (cmd == "partition-gpu") {
        need(7);
        const CSR_Order o = read_order(argv[2]);
        const SpmmCostParams c = costs_from(argv + 3);
        const double cap = capacity_from_s(std::stoi(argv[7]), c);
        cwlb::Device q(0);
        const std::vector<ParallelDataWeighted> t = costWeightedTaskPartitioning_HIP(o, c, cap, q);
        Writer w(argv[8]);
        w.one(cap);
        w.put(t);
    } else if (cmd == "partition-emul") {
        need(7);
        const CSR_Order o = read_order(argv[2]);
        const SpmmCostParams c = costs_from(argv + 3);
        const double cap = capacity_from_s(std::stoi(argv[7]), c);
        const std::vector<ParallelDataWeighted> t = partition_emulated(o.RowOffset, c, cap);
        Writer w(argv[8]);
        w.one(cap);
        w.put(t);
    } else if (cmd == "spmm" || cmd == "spmm-large") {
        need(6);
        const CSR_Order o = read_order(argv[2]);
        const Defined::RowMajorMatrixXf H = read_dense(argv[3], std::stol(argv[4]), std::stol(argv[5]));
        const std::vector<ParallelDataWeighted> t = read_tasks(argv[6]);
        cwlb::Device q(0);
        double time = -1.0;
        const int K = static_cast<int>(H.cols());
        const bool large = cmd == "spmm-large";
        const Defined::RowMajorMatrixXf C = large ? spmmKernelLargeKFallback(q, o, H, K, K, t, time)
                                                  : spmmKernel(q, o, H, K, K, t, time);
        std::cout << "time " << time << " rows " << C.rows() << " cols " << C.cols() << "\n";
        write_dense(argv[7], C);
    } else if (cmd == "run-single-s") {
        need(10);
        const CSR_Order o = read_order(argv[2]);
        const Defined::RowMajorMatrixXf H = read_dense(argv[3], std::stol(argv[4]), std::stol(argv[5]));
        const SpmmCostParams c = costs_from(argv + 6);
        cwlb::Device q(0);
        const SingleSResult r = run_single_s(q, o, H, static_cast<int>(H.cols()), c, std::stoi(argv[10]), true);
        std::cout << "average " << r.average_us << " tasks " << r.task_count << " samples "
                  << r.timed_samples_us.size() << " capacity " << r.capacity << " schedule "
                  << r.schedule[0] << ',' << r.schedule[1] << ',' << r.schedule[2] << ','
                  << r.schedule[3] << " hints " << r.cache_hint_bytes << " occupancy "
                  << r.waves_per_simd << " phases " << r.column_phases << " tiling "
                  << r.lane_tiling << "\n";
        write_dense(argv[11], r.output);
    } else if (cmd == "load") {
        need(2);
        if (chdir(argv[2]) != 0) throw std::runtime_error("probe: chdir failed");
        int V = -1, E = -1;
        const CSR c = loadDatasetToCSR(argv[3], V, E);
        std::cout << "V " << V << " E " << E << "\nrp";
        for (int x : c.RowOffset) std::cout << ' ' << x;
        std::cout << "\nci";
        for (int x : c.ColInd) std::cout << ' ' << x;
        std::cout << "\nval";
        for (float x : c.Value) std::cout << ' ' << x;
        std::cout << "\n";
    } else if (cmd == "features") {
        need(3);
        write_dense(argv[4], deterministic_features(std::stoi(argv[2]), std::stoi(argv[3])));
    } else if (cmd == "dense2csr") {
        need(4);
        const CSR c(read_dense(argv[4], std::stol(argv[2]), std::stol(argv[3])));
        Writer w(argv[5]);
        w.one<int64_t>(static_cast<int64_t>(c.RowOffset.size()) - 1);
        w.one<int64_t>(static_cast<int64_t>(c.ColInd.size()));
        w.put(c.RowOffset);
        w.put(c.ColInd);
        w.put(c.Value);
    } else if (cmd == "validate") {
        need(8);
        const long rows = std::stol(argv[6]), cols = std::stol(argv[7]), drows = std::stol(argv[8]);
        const auto A = read_dense(argv[2], rows, cols);
        const auto B = read_dense(argv[3], rows, cols);
        const CSR csr = read_csr(argv[4]);
        const auto D = read_dense(argv[5], drows, cols);
        const bool ok = validate_custom_csr_result(A, B, csr, D, std::stof(argv[9]));
        std::cout << "RESULT " << (ok ? "pass" : "fail") << "\n";
    } else if (cmd == "select") {
        need(4);
        CSR_Order o;
        o.RowOffset.assign(static_cast<std::size_t>(std::stoll(argv[3])), 0);
        if (!o.RowOffset.empty()) o.RowOffset.back() = std::stoi(argv[2]);
        const auto w = recommended_candidate_w(std::stoull(argv[2]));
        std::cout << "w " << w[0] << ' ' << w[1] << ' ' << w[2] << "\n";
        const int sel = wave_based_s(o, std::stoi(argv[4]), std::stoi(argv[5]));
        std::cout << "s " << sel << "\n";
    } else if (cmd == "search") {
        need(4);
        const std::string mode = argv[4];
        const std::vector<int> v =
            mode == "count" ? candidate_search_by_count(std::stoi(argv[2]), std::stoi(argv[3]), std::stoi(argv[5]))
                            : candidate_search_by_step(std::stoi(argv[2]), std::stoi(argv[3]), std::stoi(argv[5]));
        std::cout << "grid";
        for (int x : v) std::cout << ' ' << x;
        std::cout << "\n";
    } else if (cmd == "bounds") {
        need(4);
        const auto b = candidate_search_bounds({std::stoi(argv[2]), std::stoi(argv[3]), std::stoi(argv[4])},
                                               static_cast<std::size_t>(std::stoull(argv[5])));
        std::cout << "bounds " << b.first << ' ' << b.second << "\n";
    } else if (cmd == "posarg") {
        need(1);
        const int v = positive_search_argument(argv[2]);
        std::cout << "value " << v << "\n";
    } else if (cmd == "costs-save") {
        need(7);
        const bool ok = save_costs_one_per_line(costs_from(argv + 5), argv[2], std::stoi(argv[3]) != 0,
                                                std::stoi(argv[4]));
        std::cout << "saved " << ok << "\n";
    } else if (cmd == "costs-read") {
        need(1);
        SpmmCostParams c;
        c.K = 7;
        const bool ok = read_costs_one_per_line(c, argv[2]);
        std::cout << "read " << ok << ' ' << c.C_compute_ns << ' ' << c.C_load_ns << ' ' << c.C_store_ns
                  << ' ' << c.C_atomic_ns << " K " << c.K << "\n";
    } else if (cmd == "device") {
        need(0);
        cwlb::Device q(0);
        std::cout << "cu " << q.max_compute_units() << " wg " << q.max_work_group_size() << " wave "
                  << q.wavefront_size() << " lds " << q.local_mem_size() << " arch " << q.arch() << "\n";
    } else {
        throw std::invalid_argument("probe: unknown subcommand " + cmd);
    }
    return 0;
}

}  // namespace

int main(int argc, char** argv)
{
    try {
        return run(argc, argv);
    } catch (const std::invalid_argument& e) {
        std::cout << "EXC invalid_argument " << e.what() << "\n";
    } catch (const std::overflow_error& e) {
        std::cout << "EXC overflow_error " << e.what() << "\n";
    } catch (const std::out_of_range& e) {
        std::cout << "EXC out_of_range " << e.what() << "\n";
    } catch (const std::runtime_error& e) {
        std::cout << "EXC runtime_error " << e.what() << "\n";
    } catch (const std::bad_alloc& e) {
        std::cout << "EXC bad_alloc " << e.what() << "\n";
    } catch (const std::exception& e) {
        std::cout << "EXC other " << e.what() << "\n";
    }
    return 3;
}
