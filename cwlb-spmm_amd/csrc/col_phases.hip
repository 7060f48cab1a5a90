// Column phases of the feature-row gathers.
//
// When the feature matrix is larger than the 256 MB Infinity Cache and the
// columns of each row are spread over all of it (block models, uniform
// random graphs), the gathers of all waves in flight range over the whole
// matrix and miss the caches.  An aggregation in P column phases runs the
// task list P times, launch p gathering only the nonzeros whose column lies
// in band p = [p * h_rows / P, (p + 1) * h_rows / P): while every wave works
// in one band, the feature rows read span 1/P of the matrix, which the
// caches hold.  A row's nonzeros of band p are one contiguous range of its
// CSR range when its columns are sorted; its bounds are
//     B_p(r) = row_ptr[r] + #{ j in row r : band(col_idx[j]) < p },
// B_0(r) = row_ptr[r] and B_P(r) = row_ptr[r + 1].  They split the row
// exactly for any column order (unsorted rows only lose the locality), and
// the aggregation clamps them into the row, so bounds built for other
// contents of the arrays can only cost speed.  The P - 1 interior bounds
// are kept on the context, P - 1 arrays of n_rows ints, and rebuilt when
// the row or column array, n_rows, nnz, h_rows or P changes.
#include <algorithm>

#include "internal.h"

namespace cwlb {
namespace {

constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / 64;

// One wave per row (grid-stride): lane q in [1, P) counts the row's
// nonzeros of bands below q, 64 nonzeros per step, and writes B_q(r).
// Columns outside [0, h_rows) count in the first or last band (the
// aggregation reports them); a row whose offsets leave [0, nnz] or decrease
// gets bounds 0 (the aggregation skips and reports it).
__global__ void __launch_bounds__(kBlock)
phase_bounds(const int* __restrict__ rp, const int* __restrict__ ci, int n_rows, long long nnz,
             long long h_rows, int P, int* __restrict__ out)
{
    const int lane = threadIdx.x & 63;
    const long long waves = static_cast<long long>(gridDim.x) * kWavesPerBlock;
    for (long long r = static_cast<long long>(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6);
         r < n_rows; r += waves) {
        const int p0 = rp[r];
        const int p1 = rp[r + 1];
        const bool ok = p0 >= 0 && p1 >= p0 && static_cast<long long>(p1) <= nnz;
        int cnt = 0;
        if (ok) {
            // (64-bit steps: a row may end within 64 of 2^31)
            for (long long j0 = p0; j0 < p1; j0 += 64) {
                const long long j = j0 + lane;
                int band = P;  // past the row: below no bound
                if (j < p1) {
                    const int c = ci[j];
                    band = c < 0 ? 0
                                 : c >= h_rows ? P - 1
                                               : static_cast<int>(static_cast<long long>(c) * P /
                                                                  h_rows);
                }
                for (int q = 1; q < P; ++q) {
                    const unsigned long long m = __ballot(band < q);
                    if (lane == q) cnt += __popcll(m);
                }
            }
        }
        if (lane >= 1 && lane < P)
            out[static_cast<long long>(lane - 1) * n_rows + r] = ok ? p0 + cnt : 0;
    }
}

}  // namespace

cwlb_status launch_phase_bounds(hipStream_t st, const int32_t* row_ptr, const int32_t* col_idx,
                                int32_t n_rows, int64_t nnz, int64_t h_rows, int phases,
                                int32_t* out)
{
    if (n_rows <= 0 || phases < 2) return CWLB_OK;
    const long long blocks = std::min<long long>(
        (static_cast<long long>(n_rows) + kWavesPerBlock - 1) / kWavesPerBlock, 65536);
    hipLaunchKernelGGL(phase_bounds, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, st,
                       row_ptr, col_idx, n_rows, static_cast<long long>(nnz),
                       static_cast<long long>(h_rows), phases, out);
    CWLB_LAUNCH_CHECK("phase_bounds");
    return CWLB_OK;
}

cwlb_status build_column_phases(cwlb_ctx* ctx, const SpmmArgs& a, int phases, bool may_build,
                                const int** bounds)
{
    *bounds = nullptr;
    if (phases < 2 || a.n_rows <= 0 || a.h_rows <= 0) return CWLB_OK;
    if (ctx->phase_rp == a.row_ptr && ctx->phase_col == a.col_idx &&
        ctx->phase_n_rows == a.n_rows && ctx->phase_nnz == a.nnz &&
        ctx->phase_h_rows == a.h_rows && ctx->phase_P == phases) {
        *bounds = ctx->d_phase_bounds;
        if (!may_build) ctx->phases_captured = true;
        return CWLB_OK;
    }
    if (!may_build) return CWLB_OK;
    ctx->phase_rp = nullptr;  // invalid until rebuilt
    if (ctx->phases_captured) {
        // A captured graph reads these bounds: keep them until
        // cwlb_ctx_destroy.
        if (ctx->d_phase_bounds) ctx->retired.push_back(ctx->d_phase_bounds);
        ctx->d_phase_bounds = nullptr;
        ctx->phase_cap = 0;
        ctx->phases_captured = false;
    }
    const long long want = static_cast<long long>(phases - 1) * a.n_rows;
    if (!ctx->d_phase_bounds || want > ctx->phase_cap) {
        if (ctx->d_phase_bounds) CWLB_HIP_TRY(hipFree(ctx->d_phase_bounds));
        ctx->d_phase_bounds = nullptr;
        ctx->phase_cap = 0;
        CWLB_HIP_TRY(hipMalloc(reinterpret_cast<void**>(&ctx->d_phase_bounds),
                               sizeof(int) * static_cast<size_t>(want)));
        ctx->phase_cap = want;
    }
    const cwlb_status s = launch_phase_bounds(ctx->stream, a.row_ptr, a.col_idx, a.n_rows, a.nnz,
                                              a.h_rows, phases, ctx->d_phase_bounds);
    if (s != CWLB_OK) return s;
    // The bounds are complete before any stream can use them (the context's
    // stream may be switched before the next call).
    CWLB_HIP_TRY(hipStreamSynchronize(ctx->stream));
    ctx->phase_rp = a.row_ptr;
    ctx->phase_col = a.col_idx;
    ctx->phase_n_rows = a.n_rows;
    ctx->phase_nnz = a.nnz;
    ctx->phase_h_rows = a.h_rows;
    ctx->phase_P = phases;
    *bounds = ctx->d_phase_bounds;
    return CWLB_OK;
}

}  // namespace cwlb
