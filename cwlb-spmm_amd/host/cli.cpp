// The cwlb-spmm and costWrite command lines (reference main.cpp:431-741,
// weightCost.cpp:11-77): same arguments, prompts, output lines, results
// file blocks and exit codes.  Device: HIP device 0 (select another with
// HIP_VISIBLE_DEVICES), in place of the reference's SYCL GPU selector.
#include <cmath>
#include <cstdint>
#include <fstream>
#include <iomanip>
#include <iostream>
#include <limits>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "cwlb_driver.h"
#include "data.h"

namespace {

constexpr const char* S_SEARCH_RESULT_PATH = "../resources/results.txt";

enum class Mode { WaveW, DirectS, SRange, Candidates, CandidateSearch };

struct Args {
    std::string dataset;
    int K = 0;
    Mode mode = Mode::WaveW;
    int value = 0;       // w (WaveW), S (DirectS) or S_begin (SRange)
    int s_max = 0;
    int s_step = 0;
    int search_count = 6;
    int search_step = 0;
};

void usage()
{
    std::cerr << "Usage:\n"
              << "  ./cwlb-spmm [dataset] [K] [wave]\n"
              << "  ./cwlb-spmm [dataset] [K] --S [S]\n"
              << "  ./cwlb-spmm [dataset] [K] --candidates\n"
              << "  ./cwlb-spmm [dataset] [K] --candidate-search [count=6]\n"
              << "  ./cwlb-spmm [dataset] [K] --candidate-search --step [step]\n"
              << "  ./cwlb-spmm [dataset] [K] [S_begin] [S_max] [S_step]\n";
}

// Argument forms of main.cpp:445-506; throws std::invalid_argument (or
// std::stoi's exceptions) for a malformed command line.
Args parse(int argc, char* argv[])
{
    Args a;
    a.dataset = argv[1];
    a.K = std::stoi(argv[2]);
    const std::string third = argv[3];
    if (third == "--candidate-search") {
        a.mode = Mode::CandidateSearch;
        if (argc == 5) {
            a.search_count = positive_search_argument(argv[4]);
        } else if (argc == 6 && std::string(argv[4]) == "--step") {
            a.search_step = positive_search_argument(argv[5]);
        } else if (argc != 4) {
            throw std::invalid_argument(
                "Use --candidate-search [count] or --candidate-search --step step.");
        }
    } else if (argc == 4) {
        if (third == "--candidates") a.mode = Mode::Candidates;
        else a.value = std::stoi(third);
    } else if (argc == 5 && third == "--S") {
        a.mode = Mode::DirectS;
        a.value = std::stoi(argv[4]);
    } else if (argc == 6) {
        a.mode = Mode::SRange;
        a.value = std::stoi(third);
        a.s_max = std::stoi(argv[4]);
        a.s_step = std::stoi(argv[5]);
    } else {
        throw std::invalid_argument("The five-argument form must use --S.");
    }
    const bool candidates = a.mode == Mode::Candidates || a.mode == Mode::CandidateSearch;
    if (a.K <= 0 || (!candidates && a.value <= 0))
        throw std::invalid_argument("K and the hyperparameter must be positive.");
    if (candidates && (WARMUPCOUNT < 0 || LOOPCOUNT <= WARMUPCOUNT))
        throw std::invalid_argument("Candidate timing requires 0 <= WARMUPCOUNT < LOOPCOUNT.");
    if (a.mode == Mode::SRange && (a.s_max <= 0 || a.s_step <= 0))
        throw std::invalid_argument("S_begin, S_max and S_step must be positive.");
    if (a.mode == Mode::SRange && a.value > a.s_max)
        throw std::invalid_argument("S_begin must not be greater than S_max.");
    return a;
}

struct Candidate {
    int number = 0;
    int wave = 0;
    int s = 0;
    double average_us = 0.0;
};

struct Session {
    const Args& a;
    cwlb::Device& q;
    const CSR_Order& csr;
    const Defined::RowMajorMatrixXf& features;
    const SpmmCostParams& costs;
    int V = 0;
    int E = 0;

    SingleSResult run(int s, bool keep_samples) const
    {
        return run_single_s(q, csr, features, a.K, costs, s, keep_samples);
    }
    void print(const SingleSResult& r) const { print_single_s_result(a.dataset, V, E, costs, r); }
};

void print_samples(const char* tag, const std::string& id, const SingleSResult& r)
{
    std::cout << tag << '\t' << id;
    for (double x : r.timed_samples_us) std::cout << '\t' << x;
    std::cout << '\n';
}

// --candidates and --candidate-search (main.cpp:534-656).
int candidates_mode(const Session& ss)
{
    const Args& a = ss.a;
    const int cu = ss.q.max_compute_units();
    const std::uint64_t nnz =
        ss.csr.RowOffset.empty() ? 0ULL : static_cast<std::uint64_t>(ss.csr.RowOffset.back());
    const std::array<int, 3> waves = recommended_candidate_w(nnz);
    std::cout << "[Candidates] dataset=" << a.dataset << " K=" << a.K << " NNZ=" << nnz
              << " compute_units=" << cu << " warmup_launches=" << WARMUPCOUNT
              << " timed_launches=" << LOOPCOUNT - WARMUPCOUNT << '\n';
    std::vector<Candidate> cands;
    std::size_t best = 0;
    for (std::size_t i = 0; i < waves.size(); ++i) {
        const int s = wave_based_s(ss.csr, cu, waves[i]);
        std::cout << "[Candidates] running S" << i + 1 << " w=" << waves[i] << " S=" << s << '\n';
        const SingleSResult r = ss.run(s, true);
        if (!std::isfinite(r.average_us) || r.average_us <= 0.0)
            throw std::runtime_error("Invalid candidate kernel time.");
        ss.print(r);
        print_samples("candidate_samples_us", "S" + std::to_string(i + 1), r);
        cands.push_back(Candidate{static_cast<int>(i + 1), waves[i], s, r.average_us});
        if (r.average_us < cands[best].average_us) best = i;
    }
    std::cout << "\n=== Candidate summary (SpMM kernel time, us) ===\n"
              << "candidate\tw\tS\tSpMM_time_us\n";
    for (const Candidate& c : cands)
        std::cout << 'S' << c.number << '\t' << c.wave << '\t' << c.s << '\t' << c.average_us
                  << '\n';
    const Candidate& b = cands[best];
    std::cout << "Best among the three measured candidates: S" << b.number << " (w=" << b.wave
              << ", S=" << b.s << "), SpMM time=" << b.average_us << " us\n"
              << "best_candidate=S" << b.number << " best_S=" << b.s
              << " best_kernel_time_us=" << b.average_us << '\n';
    if (a.mode != Mode::CandidateSearch) return 0;

    const std::array<int, 3> initial = {cands[0].s, cands[1].s, cands[2].s};
    const std::pair<int, int> bounds = candidate_search_bounds(initial, best);
    const std::vector<int> plan =
        a.search_step > 0 ? candidate_search_by_step(bounds.first, bounds.second, a.search_step)
                          : candidate_search_by_count(bounds.first, bounds.second, a.search_count);
    std::cout << "[Search plan] lower=" << bounds.first << " upper=" << bounds.second;
    if (a.search_step > 0) std::cout << " manual_step=" << a.search_step;
    else std::cout << " requested_count=" << a.search_count;
    std::cout << " actual_count=" << plan.size() << '\n' << "[Search plan] S values:";
    for (int s : plan) std::cout << ' ' << s;
    std::cout << '\n';
    if (!confirm_candidate_search()) {
        std::cout << "Search cancelled; results.txt unchanged.\n";
        return 0;
    }
    Candidate overall = b;
    std::string source = "initial_candidate_S" + std::to_string(b.number);
    std::vector<Candidate> found;
    for (std::size_t i = 0; i < plan.size(); ++i) {
        std::cout << "[Search] running P" << i + 1 << " S=" << plan[i] << '\n';
        const SingleSResult r = ss.run(plan[i], true);
        if (!std::isfinite(r.average_us) || r.average_us <= 0.0)
            throw std::runtime_error("Invalid search kernel time.");
        ss.print(r);
        print_samples("search_samples_us", "P" + std::to_string(i + 1), r);
        found.push_back(Candidate{static_cast<int>(i + 1), 0, plan[i], r.average_us});
        if (r.average_us < overall.average_us) {
            overall = found.back();
            source = "search_P" + std::to_string(i + 1);
        }
    }
    // Written only after confirmation and completion, both phases together.
    std::ostringstream block;
    block << std::fixed << std::setprecision(6) << "cwlb-spmm-candidates\t" << a.dataset << '\t'
          << a.K << '\n';
    for (const Candidate& c : cands) block << c.s << '\t' << c.average_us << '\n';
    block << "cwlb-spmm-candidate-search\t" << a.dataset << '\t' << a.K << '\n';
    for (const Candidate& c : found) block << c.s << '\t' << c.average_us << '\n';
    std::ofstream out(S_SEARCH_RESULT_PATH, std::ios::out | std::ios::app);
    if (!out)
        throw std::runtime_error("Cannot append search results to " +
                                 std::string(S_SEARCH_RESULT_PATH));
    out << block.str();
    out.flush();
    if (!out) throw std::runtime_error("Failed to save candidate-search results.");
    std::cout << "\n=== Search summary (SpMM kernel time, us) ===\n"
              << "point\tS\tSpMM_time_us\n";
    for (const Candidate& c : found)
        std::cout << 'P' << c.number << '\t' << c.s << '\t' << c.average_us << '\n';
    std::cout << "Best among all evaluated initial/search configurations: S=" << overall.s
              << ", SpMM time=" << overall.average_us << " us\n"
              << "final_best_S=" << overall.s
              << " final_best_kernel_time_us=" << overall.average_us << " source=" << source
              << '\n'
              << "Results appended to " << S_SEARCH_RESULT_PATH << '\n';
    return 0;
}

// S_begin S_max S_step (main.cpp:657-711).
int range_mode(const Session& ss)
{
    const Args& a = ss.a;
    std::ofstream out(S_SEARCH_RESULT_PATH, std::ios::out | std::ios::app);
    if (!out.is_open())
        throw std::runtime_error("Cannot open S search result file: " +
                                 std::string(S_SEARCH_RESULT_PATH));
    out << "cwlb-spmm\t" << a.dataset << '\t' << a.K << '\n';
    out << std::fixed << std::setprecision(6);
    out.flush();
    int best_s = 0;
    double best_us = std::numeric_limits<double>::infinity();
    for (std::int64_t s = a.value; s <= a.s_max; s += a.s_step) {
        const SingleSResult r = ss.run(static_cast<int>(s), false);
        ss.print(r);
        out << r.s << '\t' << r.average_us << '\n';
        out.flush();
        if (!out)
            throw std::runtime_error("Failed to append S search result file: " +
                                     std::string(S_SEARCH_RESULT_PATH));
        if (r.average_us < best_us) {
            best_s = r.s;
            best_us = r.average_us;
        }
    }
    std::cout << std::fixed << std::setprecision(6) << "best_S=" << best_s
              << " best_kernel_time_us=" << best_us << '\n';
    return 0;
}

}  // namespace

int cwlb_spmm_main(int argc, char* argv[])
{
    if (argc != 4 && argc != 5 && argc != 6) {
        usage();
        return 1;
    }
    try {
        const Args a = parse(argc, argv);
        int V = 0, E = 0;
        const CSR adjacency = loadDatasetToCSR(a.dataset, V, E);
        cwlb::Device q(0);
        SpmmCostParams costs;
        if (!read_costs_one_per_line(costs))
            throw std::runtime_error("Cannot read microbenchmark cost file: " + COSTFILEPATH +
                                     ". Run ./costWrite first.");
        const Defined::RowMajorMatrixXf features = deterministic_features(V, a.K);
        const CSR_Order sorted = sortCSRByDegreeDPLCPU(adjacency);
        const Session ss{a, q, sorted, features, costs, V, E};
        if (a.mode == Mode::Candidates || a.mode == Mode::CandidateSearch)
            return candidates_mode(ss);
        if (a.mode == Mode::SRange) return range_mode(ss);
        int s = a.value;
        if (a.mode == Mode::WaveW) s = wave_based_s(sorted, q.max_compute_units(), a.value);
        ss.print(ss.run(s, false));
    } catch (const std::exception& e) {
        std::cerr << e.what() << '\n';
        return 1;
    }
    return 0;
}

int cost_write_main(int argc, char* argv[])
{
    try {
        int K = 128, repeat = 500, WI = 131072, load_MB = 512, writers = 8;
        if (argc != 1 && argc != 6) {
            std::cerr << "Usage:\n"
                      << "  ./costWrite\n"
                      << "  ./costWrite [K] [repeat] [WI] [load_MB] [atomic_writers]\n";
            return 1;
        }
        if (argc == 6) {
            K = std::stoi(argv[1]);
            repeat = std::stoi(argv[2]);
            WI = std::stoi(argv[3]);
            load_MB = std::stoi(argv[4]);
            writers = std::stoi(argv[5]);
        }
        if (K <= 0 || repeat <= 0 || WI <= 0 || load_MB <= 0 || writers <= 0)
            throw std::invalid_argument("All microbenchmark parameters must be positive.");
        cwlb::Device q(0);
        const SpmmCostParams c = measure_spmm_costs(q, K, repeat, WI, load_MB, writers);
        std::cout << "device: " << q.name() << '\n'
                  << "C_compute_ns: " << c.C_compute_ns << '\n'
                  << "C_load_ns: " << c.C_load_ns << '\n'
                  << "C_store_ns: " << c.C_store_ns << '\n'
                  << "C_atomic_ns: " << c.C_atomic_ns << '\n';
        if (!save_costs_one_per_line(c))
            throw std::runtime_error("Failed to write microbenchmark cost file: " + COSTFILEPATH);
        std::cout << "Saved cost parameters to: " << COSTFILEPATH << '\n';
    } catch (const std::exception& e) {
        std::cerr << e.what() << '\n';
        return 1;
    }
    return 0;
}
