// Column phases of the feature-row gathers.
//
// When the feature matrix is larger than the 256 MB Infinity Cache and the
// columns of each row are spread over all of it (block models, uniform
// random graphs), the gathers of all waves in flight range over the whole
// matrix and miss the caches.  An aggregation in P column phases runs the
// task list P times, launch p gathering only the nonzeros of band p: while
// every wave works in one band, the feature rows read are 1/P of the matrix,
// which the caches hold.
//
// The bands interleave the columns, band(c) = c mod P.  Contiguous bands
// ([p * h_rows / P, (p + 1) * h_rows / P)) give each phase the same share of
// the matrix but not of the work when communities occupy ranges of ids: a
// row then has most of its nonzeros in the one band that holds its
// community, and every phase ends on the waves that hold such rows (the
// 240k-row block model: 34.7 ms in 16 contiguous phases, 27.7 ms when the
// bands interleave the blocks).  With interleaved bands a row's nonzeros of
// band p are not contiguous in CSR order, so each phased call first writes a
// copy of the column and value arrays in which every row's nonzeros are
// stably sorted by band, and the row bounds of the bands,
//     B_p(r) = row_ptr[r] + #{ j in row r : band(col_idx[j]) < p },
// B_0(r) = row_ptr[r], B_P(r) = row_ptr[r + 1]; launch p reads the copy's
// range [B_p(r), B_{p+1}(r)) of each row.  The copy is rewritten by every
// call, so arrays the caller rewrites in place are always read as they are.
#include <algorithm>

#include "internal.h"

namespace cwlb {
namespace {

constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / 64;

// The band of a column: c mod P; a column outside [0, h_rows) is put in
// band 0 (the aggregation reports it).
__device__ __forceinline__ int band_of(int c, long long h_rows, int P)
{
    return (c < 0 || c >= h_rows) ? 0 : c % P;
}

// Lanes of one band: with one ballot per bit of the band numbers (bits
// ballots, nb of them), the lanes whose band equals `band` are those that
// agree with it on every bit.  mine: the lanes of this lane's band; lane_q:
// the lanes of band `lane` (lane q's own band q), for the per-band counts.
__device__ __forceinline__ void band_masks(int band, int nb, unsigned long long& mine,
                                           unsigned long long& lane_q)
{
    const int lane = threadIdx.x & 63;
    mine = ~0ull;
    lane_q = ~0ull;
    for (int b = 0; b < nb; ++b) {
        const unsigned long long bb = __ballot((band >> b) & 1);
        mine &= ((band >> b) & 1) ? bb : ~bb;
        lane_q &= ((lane >> b) & 1) ? bb : ~bb;
    }
}

// One wave per row (grid-stride), in batches of kBatch chunks of 64
// nonzeros whose loads are all issued before any is used.
//   * Counting pass: per chunk, the bit-sliced band masks above (one ballot
//     per bit of P, not one per band); lane q keeps band q's count in the
//     row, and for a row of one batch (at most 64 * kBatch nonzeros) also
//     band q's count before each chunk, while each lane keeps its nonzero's
//     rank among the chunk's nonzeros of its band.  The bounds B_q(r), q in
//     [1, P), are an exclusive scan of the counts.
//   * A row of one batch keeps its columns and values in registers: each
//     goes to its band's start + the band's count before its chunk + its
//     rank (one shuffle per chunk), into the wave's LDS buffer, and the row
//     is written out with coalesced stores.
//   * A longer row is read again and scattered straight to memory, each
//     nonzero to its band's next free slot (the band masks and one shuffle
//     per chunk; lane q holds band q's next free position).
// A row whose offsets leave [0, nnz] or decrease gets bounds 0 and no copy
// (the aggregation skips and reports it).  Row positions are 64-bit: a row
// may end within 64 of 2^31.
constexpr int kBatch = 8;

__global__ void __launch_bounds__(kBlock)
band_sort(const int* __restrict__ rp, const int* __restrict__ ci, const float* __restrict__ val,
          int n_rows, long long nnz, long long h_rows, int P, int* __restrict__ bounds,
          int* __restrict__ ci_out, float* __restrict__ val_out, int* __restrict__ chain_word)
{
    // The aggregation's not-a-chain word starts each phased call cleared
    // (the clearing pass that runs next sets it for a list that is no chain).
    if (chain_word && blockIdx.x == 0 && threadIdx.x == 0) *chain_word = 0;
    __shared__ int s_col[kWavesPerBlock][64 * kBatch];
    __shared__ float s_val[kWavesPerBlock][64 * kBatch];
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const unsigned long long below = (1ull << lane) - 1ull;  // lanes before this one
    const int nb = 32 - __clz(P);  // bits of 0..P (P marks lanes past the row)
    const long long waves = static_cast<long long>(gridDim.x) * kWavesPerBlock;
    for (long long r = static_cast<long long>(blockIdx.x) * kWavesPerBlock + wv; r < n_rows;
         r += waves) {
        const int p0 = rp[r];
        const int p1 = rp[r + 1];
        const bool ok = p0 >= 0 && p1 >= p0 && static_cast<long long>(p1) <= nnz;
        const bool copy = ok && ci_out;
        const bool one_batch = static_cast<long long>(p1) - p0 <= 64 * kBatch;
        int tot = 0;           // lane q: band q's nonzeros in the row
        int before[kBatch];    // lane q: band q's nonzeros before chunk k
        int rank[kBatch];      // this lane's rank in its band within chunk k
        int c[kBatch];
        float v[kBatch];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) before[k] = rank[k] = 0;
        if (ok) {
            for (long long b0 = p0; b0 < p1; b0 += 64 * kBatch) {
#pragma unroll
                for (int k = 0; k < kBatch; ++k) {
                    const long long j = b0 + 64 * k + lane;
                    c[k] = j < p1 ? ci[j] : 0;
                    if (copy) v[k] = j < p1 ? val[j] : 0.0f;
                }
#pragma unroll
                for (int k = 0; k < kBatch; ++k) {
                    const long long j = b0 + 64 * k + lane;
                    const int band = j < p1 ? band_of(c[k], h_rows, P) : P;
                    before[k] = tot;
                    unsigned long long mine, lane_q;
                    band_masks(band, nb, mine, lane_q);
                    rank[k] = __popcll(mine & below);
                    if (lane < P) tot += __popcll(lane_q);
                }
            }
        }
        // Band q starts at p0 + the counts of the bands below q.
        int start = tot;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int t = __shfl_up(start, off);
            if (lane >= off) start += t;
        }
        start = p0 + start - tot;
        if (bounds && lane >= 1 && lane < P)
            bounds[static_cast<long long>(lane - 1) * n_rows + r] = ok ? start : 0;
        if (!copy) continue;
        if (one_batch) {
#pragma unroll
            for (int k = 0; k < kBatch; ++k) {
                const int j = 64 * k + lane;
                const int band = j < p1 - p0 ? band_of(c[k], h_rows, P) : 0;
                const int dst = __shfl(start + before[k], band) + rank[k];
                if (j < p1 - p0) {
                    s_col[wv][dst - p0] = c[k];
                    s_val[wv][dst - p0] = v[k];
                }
            }
            // The wave's LDS writes above are complete before its reads
            // (wave-ordered LDS); the fences keep the compiler from moving
            // accesses across, here and before the next row's writes.
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            const int len = p1 - p0;
#pragma unroll
            for (int k = 0; k < kBatch; ++k) {
                const int i = 64 * k + lane;
                if (i < len) {
                    ci_out[static_cast<long long>(p0) + i] = s_col[wv][i];
                    val_out[static_cast<long long>(p0) + i] = s_val[wv][i];
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            continue;
        }
        int next = start;  // lane q: band q's next free position
        for (long long b0 = p0; b0 < p1; b0 += 64 * kBatch) {
#pragma unroll
            for (int k = 0; k < kBatch; ++k) {
                const long long j = b0 + 64 * k + lane;
                c[k] = j < p1 ? ci[j] : 0;
                v[k] = j < p1 ? val[j] : 0.0f;
            }
#pragma unroll
            for (int k = 0; k < kBatch; ++k) {
                const long long j = b0 + 64 * k + lane;
                const bool in = j < p1;
                const int band = in ? band_of(c[k], h_rows, P) : P;
                unsigned long long mine, lane_q;
                band_masks(band, nb, mine, lane_q);
                const int dst = __shfl(next, band) + __popcll(mine & below);
                if (lane < P) next += __popcll(lane_q);
                if (in) {
                    ci_out[dst] = c[k];
                    val_out[dst] = v[k];
                }
            }
        }
    }
}

unsigned band_grid(int n_rows)
{
    return static_cast<unsigned>(std::min<long long>(
        (static_cast<long long>(n_rows) + kWavesPerBlock - 1) / kWavesPerBlock, 65536));
}

// Grows a context-owned phase buffer.  Once a captured graph has used the
// phase buffers, a buffer that must grow is retired (freed by
// cwlb_ctx_destroy) instead of freed: the graph keeps its address.
template <class T>
cwlb_status grow(cwlb_ctx* ctx, T** p, long long* cap, long long want)
{
    if (*p && want <= *cap) return CWLB_OK;
    if (*p) {
        if (ctx->phases_captured) ctx->retired.push_back(*p);
        else CWLB_HIP_TRY(hipFree(*p));
    }
    *p = nullptr;
    *cap = 0;
    CWLB_HIP_TRY(hipMalloc(reinterpret_cast<void**>(p), sizeof(T) * static_cast<size_t>(want)));
    *cap = want;
    return CWLB_OK;
}

}  // namespace

cwlb_status launch_band_sort(hipStream_t st, const int32_t* row_ptr, const int32_t* col_idx,
                             const float* val, int32_t n_rows, int64_t nnz, int64_t h_rows,
                             int phases, int32_t* bounds, int32_t* col_out, float* val_out,
                             int32_t* chain_word)
{
    if (n_rows <= 0 || phases < 2) return CWLB_OK;
    hipLaunchKernelGGL(band_sort, dim3(band_grid(n_rows)), dim3(kBlock), 0, st, row_ptr, col_idx,
                       val, n_rows, static_cast<long long>(nnz), static_cast<long long>(h_rows),
                       phases, bounds, col_out, val_out, chain_word);
    CWLB_LAUNCH_CHECK("band_sort");
    return CWLB_OK;
}

cwlb_status prepare_column_phases(cwlb_ctx* ctx, const SpmmArgs& a, int phases, bool may_build,
                                  PhaseArrays* out)
{
    *out = PhaseArrays{};
    if (phases < 2 || a.n_rows <= 0 || a.h_rows <= 0) return CWLB_OK;
    const long long want_b = static_cast<long long>(phases - 1) * a.n_rows;
    const long long want_e = std::max<long long>(a.nnz, 1);
    if (!may_build) {
        // Under capture nothing is allocated: the buffers must already be
        // large enough (an earlier eager call made them so).
        if (!ctx->d_phase_bounds || want_b > ctx->phase_cap || !ctx->d_band_col ||
            want_e > ctx->band_cap_col || !ctx->d_band_val || want_e > ctx->band_cap_val)
            return CWLB_OK;
        ctx->phases_captured = true;
    } else {
        cwlb_status s = grow(ctx, &ctx->d_phase_bounds, &ctx->phase_cap, want_b);
        if (s == CWLB_OK) s = grow(ctx, &ctx->d_band_col, &ctx->band_cap_col, want_e);
        if (s == CWLB_OK) s = grow(ctx, &ctx->d_band_val, &ctx->band_cap_val, want_e);
        if (s != CWLB_OK) return s;
    }
    out->bounds = ctx->d_phase_bounds;
    out->col = ctx->d_band_col;
    out->val = ctx->d_band_val;
    return CWLB_OK;
}

}  // namespace cwlb
