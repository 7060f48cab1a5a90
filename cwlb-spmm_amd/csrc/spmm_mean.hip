// FP32 mean-aggregation SpMM over a cost-weighted task list, for gfx950.
//
// Semantics follow spmmKernel (reference src/parallelMatrix.cpp:148-236):
// every task is a half-open range of reordered rows whose first row starts
// at first_row_offset and whose last row ends at last_row_nnz (0 = full
// degree); for each row chunk the kernel forms
//     acc[k] = sum_j val[j] * H[col[j]][k]   (fma, CSR order per lane)
// divides by the FULL degree, then stores C[origin[r]] for a full row or
// adds atomically for a partial one.  Rows of degree 0 are written as zeros
// unless C holds zeros there already (the call clears C, or the caller says
// an earlier clear did): the reference leaves its host-zeroed C untouched
// there.
//
// Mapping to CDNA4 (64-lane waves):
//   * a wave executes a run of M consecutive tasks (M = 1 reproduces the
//     reference's one task per work-group).  Inside the run it executes
//     "segments": maximal stretches of consecutive tasks in which each task
//     starts exactly where the previous one ended.  A segment is itself a
//     task (row_start and first_row_offset of its first task, row_end and
//     last_row_nnz of its last), so a row split only between tasks of one
//     segment is reduced in registers and stored instead of being added
//     atomically chunk by chunk.  The partition's task lists tile the
//     nonzeros in order, so there a segment is the whole run (or a 64-task
//     window of it); a shuffled list, one with gaps or malformed tasks
//     falls apart into one-task segments, the reference's semantics;
//   * a row slice of Ks = K / SL floats is covered by a "slot" of G lanes,
//     each lane holding R vectors of VEC floats (128-bit loads when
//     K % 4 == 0); a wave has NS = 64 / G slots.  By default G is the
//     smallest power of two that holds the slice (R = 1); packed slots
//     (G lanes of 3 or 5 vectors, see pick_tiling) cover slices of other
//     widths with fewer idle lanes.  With SL > 1 the feature
//     slices are spread over the XCDs (work-groups are dispatched to the 8
//     XCDs round-robin), so each XCD's L2 caches one slice of the hot
//     feature rows and holds SL times as many of them;
//   * short rows run row-per-slot, RU rows per slot at a time, each row
//     summed sequentially in CSR order (bit-identical to the reference's
//     per-work-item loop);
//   * a long chunk runs on all slots at once, UL nonzeros in flight per
//     slot, followed by a shuffle reduction across slots;
//   * the occupancy variant (O6) keeps UL <= 2, which lets slots of 4 to 16
//     lanes fit 80 VGPRs: 6 waves per SIMD instead of 5, for graphs of
//     short rows, where waves in flight set the speed;
//   * column phases (PH, csrc/col_phases.hip): the launch is repeated once
//     per band of columns (c mod P) over a copy of the CSR sorted by band
//     within each row, so that the feature rows all waves gather at a time
//     fit the caches; on a chain of tasks each run owns whole rows, stored
//     in the first phase and added to without atomics in the others;
//   * column indices and values are fetched with coalesced streaming loads:
//     64 at a time for a long chunk, handed to the slots with cross-lane
//     shuffles; for a group of short rows, the group's whole contiguous
//     range (up to 256 nonzeros) at once, into a per-wave LDS window, so no
//     row waits on an index load before its feature-row loads.  C is written
//     with streaming stores.
// Split rows are cleared by zero_split_rows before the main kernel: a row
// that a segment leaves open is cleared by the task whose chunk of it starts
// at nonzero 0.
#include "internal.h"

#include <algorithm>

namespace cwlb {
namespace {

// The aggregation kernel runs one wave per work-group: its waves never
// synchronise, and a work-group's slot frees as soon as its wave ends (with
// 4-wave groups a slot waits for the slowest of four runs; measured 1-wave
// groups: mesh 2.4%, block model 0.9%, R-MAT 0.4% faster).  The clearing
// and fill kernels use 256-thread groups.
constexpr int kWaves = 1;
constexpr int kBlock = 64 * kWaves;
constexpr int kAuxBlock = 256;
// A launch holds fewer than 2^32 work-items.
constexpr long long kMaxGridBlocks = (1ll << 32) / kBlock - 8;

typedef float f2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));

template <int VEC>
struct VecT;
template <>
struct VecT<1> {
    using T = float;
};
template <>
struct VecT<2> {
    using T = f2;
};
template <>
struct VecT<4> {
    using T = f4;
};


template <int VEC>
__device__ __forceinline__ typename VecT<VEC>::T vzero()
{
    return typename VecT<VEC>::T(0.0f);
}

template <int VEC>
__device__ __forceinline__ typename VecT<VEC>::T vload(const float* p)
{
    return *reinterpret_cast<const typename VecT<VEC>::T*>(p);
}

template <int VEC>
__device__ __forceinline__ void vstore(float* p, typename VecT<VEC>::T v)
{
    *reinterpret_cast<typename VecT<VEC>::T*>(p) = v;
}

// Streaming (non-temporal) store: C is written once and not re-read.
template <int VEC>
__device__ __forceinline__ void vstore_nt(float* p, typename VecT<VEC>::T v)
{
    __builtin_nontemporal_store(v, reinterpret_cast<typename VecT<VEC>::T*>(p));
}

// Feature-row gathers under cache-policy hints: a raw buffer resource over
// H (byte offsets below 4 GiB, bounds-checked by the hardware), and one
// 16-byte load whose policy is non-temporal for a cold column.  The policy
// is an immediate of the load instruction, so the two loads stay distinct.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t feature_rsrc(const float* H, long long h_rows,
                                                               int ld)
{
    const unsigned long long bytes = static_cast<unsigned long long>(h_rows) * ld * 4ull;
    return __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(H), 0,
        bytes > 0xFFFFFFFFull ? 0xFFFFFFFFu : static_cast<unsigned>(bytes), 0x00020000);
}

__device__ __forceinline__ f4 gather_hinted(__amdgpu_buffer_rsrc_t r, unsigned byte_off, bool cold)
{
    if (cold) return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 2));
    return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
}

// Bit 31 of a staged column index carries the cold hint of its nonzero
// (valid column indices are below 2^31; a negative, invalid one becomes
// INT_MAX, which the column bounds check still rejects).
__device__ __forceinline__ int with_hint(int col, const unsigned long long* __restrict__ hints,
                                         long long j)
{
    const unsigned cold = static_cast<unsigned>((hints[j >> 6] >> (j & 63)) & 1ull);
    const unsigned c = col < 0 ? 0x7fffffffu : static_cast<unsigned>(col);
    return static_cast<int>(c | (cold << 31));
}

__device__ __forceinline__ float vfma(float a, float h, float c) { return __builtin_fmaf(a, h, c); }
__device__ __forceinline__ f2 vfma(float a, f2 h, f2 c)
{
    f2 r;
    r.x = __builtin_fmaf(a, h.x, c.x);
    r.y = __builtin_fmaf(a, h.y, c.y);
    return r;
}
__device__ __forceinline__ f4 vfma(float a, f4 h, f4 c)
{
    f4 r;
    r.x = __builtin_fmaf(a, h.x, c.x);
    r.y = __builtin_fmaf(a, h.y, c.y);
    r.z = __builtin_fmaf(a, h.z, c.z);
    r.w = __builtin_fmaf(a, h.w, c.w);
    return r;
}

__device__ __forceinline__ float vdiv(float v, float d) { return v / d; }
__device__ __forceinline__ f2 vdiv(f2 v, float d)
{
    f2 r;
    r.x = v.x / d;
    r.y = v.y / d;
    return r;
}
__device__ __forceinline__ f4 vdiv(f4 v, float d)
{
    f4 r;
    r.x = v.x / d;
    r.y = v.y / d;
    r.z = v.z / d;
    r.w = v.w / d;
    return r;
}

__device__ __forceinline__ float vshfl_xor(float v, int m) { return __shfl_xor(v, m); }
__device__ __forceinline__ f2 vshfl_xor(f2 v, int m)
{
    f2 r;
    r.x = __shfl_xor(v.x, m);
    r.y = __shfl_xor(v.y, m);
    return r;
}
__device__ __forceinline__ f4 vshfl_xor(f4 v, int m)
{
    f4 r;
    r.x = __shfl_xor(v.x, m);
    r.y = __shfl_xor(v.y, m);
    r.z = __shfl_xor(v.z, m);
    r.w = __shfl_xor(v.w, m);
    return r;
}

__device__ __forceinline__ void vatomic_add(float* p, float v) { unsafeAtomicAdd(p, v); }
__device__ __forceinline__ void vatomic_add(float* p, f2 v)
{
    unsafeAtomicAdd(p, v.x);
    unsafeAtomicAdd(p + 1, v.y);
}
__device__ __forceinline__ void vatomic_add(float* p, f4 v)
{
    unsafeAtomicAdd(p, v.x);
    unsafeAtomicAdd(p + 1, v.y);
    unsafeAtomicAdd(p + 2, v.z);
    unsafeAtomicAdd(p + 3, v.w);
}

// How a finished chunk reaches C: 0 stored, 1 added by a plain
// read-modify-write (a row one segment owns, after the first column
// phase), 2 added atomically (a row split between segments).
template <bool PH, class Ch>
__device__ __forceinline__ int write_mode(bool ph, bool first, const Ch& c)
{
    if constexpr (PH) {
        if (ph) return c.own ? (first ? 0 : 1) : 2;
    }
    return (c.b == 0 && c.e == c.d) ? 0 : 2;
}

template <int VEC>
__device__ __forceinline__ void write_row(float* p, typename VecT<VEC>::T v, int how)
{
    if (how == 0)
        vstore_nt<VEC>(p, v);
    else if (how == 1)
        vstore_nt<VEC>(p, vload<VEC>(p) + v);
    else
        vatomic_add(p, v);
}

__device__ __forceinline__ int wave_max(int v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = max(v, __shfl_xor(v, off));
    return v;
}

// Nonzero range of row r inside task (rs, re, fo, ln), with the reference's
// clamps (parallelMatrix.cpp:164-176).  Rows of degree 0 have an empty
// chunk.  A row whose offsets leave [0, nnz] or decrease gets d = -1 and an
// empty chunk: no load can leave the arrays, and the caller reports it.
struct Chunk {
    int base;  // row_ptr[r]
    int b;     // chunk begin within the row
    int e;     // chunk end within the row
    int d;     // full degree (-1: malformed offsets)
    int own;   // column phases only: the task covers the whole row
};

__device__ __forceinline__ Chunk row_chunk(const int* __restrict__ rp, int r, int rs, int re,
                                           int fo, int ln, long long nnz)
{
    Chunk c;
    const int p0 = rp[r];
    const int p1 = rp[r + 1];
    c.base = p0;
    c.b = 0;
    c.e = 0;
    if (p0 < 0 || p1 < p0 || static_cast<long long>(p1) > nnz) {
        c.d = -1;
        return c;
    }
    c.d = p1 - p0;
    if (c.d == 0) return c;
    int b = (r == rs) ? fo : 0;
    int e = c.d;
    if (r == re - 1 && ln > 0) e = ln;
    b = min(max(b, 0), c.d);
    e = min(max(e, b), c.d);
    c.b = b;
    c.e = e;
    return c;
}

// Row r's chunk under column phases.  With ph (the task list is a chain,
// see zero_split_rows) the chunk is cut to the row's nonzeros of this
// phase, [pb[r], pe[r]) -- the row's start for the first phase (pb null),
// its end for the last (pe null) -- with the bounds clamped into the row,
// so any non-decreasing bounds split the row exactly.  own records, before
// the cut, whether the task covers the whole row: such a row belongs to
// this one segment in every phase.
template <bool PH>
__device__ __forceinline__ Chunk task_chunk(const int* __restrict__ rp, int r, int rs, int re,
                                            int fo, int ln, long long nnz, bool ph,
                                            const int* __restrict__ pb,
                                            const int* __restrict__ pe)
{
    if constexpr (!PH) {
        return row_chunk(rp, r, rs, re, fo, ln, nnz);
    } else {
        int lo_abs = 0, hi_abs = 0;
        if (ph && pb) lo_abs = pb[r];
        if (ph && pe) hi_abs = pe[r];
        Chunk c = row_chunk(rp, r, rs, re, fo, ln, nnz);
        c.own = c.d > 0 && c.b == 0 && c.e == c.d;
        if (ph && c.d > 0) {
            const int lo = pb ? min(max(lo_abs - c.base, 0), c.d) : 0;
            const int hi = pe ? min(max(hi_abs - c.base, lo), c.d) : c.d;
            c.b = max(c.b, lo);
            c.e = max(min(c.e, hi), c.b);
        }
        return c;
    }
}

constexpr int cmin(int a, int b) { return a < b ? a : b; }

// x, opaque to the optimiser.  Lane-derived values (lane ids, shuffle
// sources) computed from it inside a loop stay there: hoisted to the kernel
// entry they would each hold a VGPR for the whole kernel, which costs the
// aggregation kernel a wave per SIMD (4 instead of 5 at K = 32 and 64).
__device__ __forceinline__ int fresh(int x)
{
    asm volatile("" : "+v"(x));
    return x;
}

// ------------------------------------------------------------ segments
// A task is well formed when its rows lie in [0, n_rows), it has at least
// one row, its offsets are non-negative, and a one-row task with an end
// offset ends after it starts.
__device__ __forceinline__ bool task_well_formed(const cwlb_task& t, int n_rows)
{
    return t.row_start >= 0 && t.row_start < t.row_end && t.row_end <= n_rows &&
           t.first_row_offset >= 0 && t.last_row_nnz >= 0 &&
           (t.row_end - t.row_start > 1 || t.last_row_nnz == 0 ||
            t.first_row_offset < t.last_row_nnz);
}

// b starts exactly where a ends: on the row after a's last row when a ends
// on a row boundary (last_row_nnz == 0), else inside a's last row at a's
// end offset.
__device__ __forceinline__ bool continues(const cwlb_task& a, const cwlb_task& b)
{
    return a.last_row_nnz == 0
               ? (b.row_start == a.row_end && b.first_row_offset == 0)
               : (b.row_start == a.row_end - 1 && b.first_row_offset == a.last_row_nnz);
}

// Whether task cur, at position in_run inside its run of M tasks (prev is
// the task before it), starts a segment: at every 64-task window of a run
// (the run's first task included), and wherever either task is malformed or
// cur does not continue prev.  The aggregation kernel and the split-row
// clearing pass use this same rule.
__device__ __forceinline__ bool segment_break(const cwlb_task& prev, const cwlb_task& cur,
                                              long long in_run, int n_rows)
{
    return (in_run & 63) == 0 || !task_well_formed(prev, n_rows) ||
           !task_well_formed(cur, n_rows) || !continues(prev, cur);
}

__device__ __forceinline__ cwlb_task shfl_up_task(const cwlb_task& t)
{
    cwlb_task p;
    p.row_start = __shfl_up(t.row_start, 1);
    p.row_end = __shfl_up(t.row_end, 1);
    p.first_row_offset = __shfl_up(t.first_row_offset, 1);
    p.last_row_nnz = __shfl_up(t.last_row_nnz, 1);
    return p;
}

// Block b runs on XCD b % 8; slice = XCD % SL.  The P = 8 / SL XCDs of one
// slice share its run blocks [0, n_blocks), either interleaved (XCD q of the
// slice takes blocks q, q + P, q + 2P, ...) or contiguous (XCD q takes
// blocks [q * chunk, (q + 1) * chunk), chunk = ceil(n_blocks / P)), so that
// each XCD's L2 sees one stretch of the run order.  Both are bijections from
// the launched grid onto a superset of [0, n_blocks).
template <int SL>
__device__ __forceinline__ void block_slice(int& slice, long long& jb, long long chunk)
{
    constexpr int P = 8 / SL;
    const int bx = blockIdx.x;
    const int xcd = bx & 7;
    slice = xcd % SL;
    const int q = xcd / SL;
    jb = chunk > 0 ? static_cast<long long>(q) * chunk + (bx >> 3)
                   : static_cast<long long>(bx >> 3) * P + q;
}

// PH: one launch of a column-phased call (pb, pe: this phase's row bounds
// in ci_b / val_b, the copy of ci / val with each row's nonzeros sorted by
// band; first: the first phase; seq: the call's sequence number; status[1]
// == seq marks a task list that is not a chain, which then runs in one pass
// over ci / val in the first launch and not at all in the others).
// write_empty: rows without nonzeros are stored as zeros; 0 leaves them to
// the caller's clearing, as the reference's kernel never writes them.
template <int VEC, int G, int R, int U, int SL, bool HN, bool O6, bool PH>
__global__ void __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(O6 ? 6 : 1)))
spmm_mean_runs(const int* __restrict__ rp, const int* __restrict__ ci,
               const float* __restrict__ val, const int* __restrict__ origin, int n_rows,
               long long nnz, const float* __restrict__ H, long long h_rows, int ld,
               const cwlb_task* __restrict__ tasks, long long n_tasks, int M, long long n_runs,
               long long n_blocks, long long chunk, const int* __restrict__ run_order,
               const unsigned long long* __restrict__ hints, float* __restrict__ C,
               int* __restrict__ status, const int* __restrict__ pb,
               const int* __restrict__ pe, const int* __restrict__ ci_b,
               const float* __restrict__ val_b, int first_phase, int seq, int write_empty)
{
    static_assert(!HN || VEC == 4, "hinted gathers move 16 bytes per lane");
    using V = typename VecT<VEC>::T;
    constexpr int NS = 64 / G;                     // row slots per wave
    constexpr int RU = cmin(cmin(U, 4), G);        // rows per slot (short rows)
    constexpr int GROUP = NS * RU;                 // rows per short-row group (<= 64)
    // nonzeros per slot per step (long rows)
    constexpr int UL = O6 ? cmin(cmin(U, G), 2) : cmin(U, G);
    constexpr int STEP = NS * UL;                  // nonzeros per wave step (<= 64)
    constexpr int kLong = GROUP > 2 ? GROUP : 2;   // chunk length that runs on all slots
    // A short-row group holds at most GROUP * (kLong - 1) nonzeros.  When
    // that can exceed 64, a group's nonzeros (up to kStage, the group is cut
    // there) go through a per-wave LDS window; otherwise through one
    // 64-entry register window.  Either way no row waits on a column-index
    // load before its feature-row loads.
    constexpr int kMaxGroupNnz = GROUP * (kLong - 1);
    constexpr int kStage = kMaxGroupNnz > 64 ? cmin(kMaxGroupNnz, 256) : 0;
    constexpr int kWin = kStage > 0 ? kStage : 64;  // nonzeros of one group
    __shared__ int s_col[kWaves * (kStage > 0 ? kStage : 1)];
    __shared__ float s_val[kWaves * (kStage > 0 ? kStage : 1)];

    const int lane = threadIdx.x & 63;
    const int slot = lane / G;
    const int sub = lane - slot * G;
    int slice;
    long long jb;
    block_slice<SL>(slice, jb, chunk);
    if (jb >= n_blocks) return;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const long long pos = jb * kWaves + wv;
    if (pos >= n_runs) return;
    // Column phases apply to chains only: rows whose whole range one
    // segment covers are then stored in the first phase and added to,
    // without atomics, in the others.
    bool ph = false;
    const bool first = !PH || first_phase != 0;
    if constexpr (PH) {
        ph = __builtin_amdgcn_readfirstlane(status[1]) != seq;
        if (!ph && !first) return;
    }
    int* __restrict__ wcol = s_col + wv * (kStage > 0 ? kStage : 1);
    float* __restrict__ wval = s_val + wv * (kStage > 0 ? kStage : 1);
    // run_order (optional) is a permutation of [0, n_runs): runs execute in
    // that order instead of task order.
    const long long run = run_order ? static_cast<long long>(run_order[pos]) : pos;

    // This slice's vectors [f0, f0 + F) of the row's ld / VEC: whole
    // vectors, as even as the row allows (sizes differ by at most one).
    const int FT = ld / VEC;
    const int f0 = slice * FT / SL;
    const int F = (slice + 1) * FT / SL - f0;
    const float* __restrict__ Hs = H + f0 * VEC;
    float* __restrict__ Cs = C + f0 * VEC;
    const int npass = (F + G * R - 1) / (G * R);
    int bad = 0;
    // Hinted gathers: byte offset of feature vector f of column c's slice.
    __amdgpu_buffer_rsrc_t hrsrc;
    if constexpr (HN) hrsrc = feature_rsrc(H, h_rows, ld);
    const unsigned slice_bytes = static_cast<unsigned>(f0 * VEC) * 4u;

    // One segment: task (rs, re, fo, ln) over the column and value arrays
    // cx / vx; banded: the rows are whole rows of a chain, read band by band
    // from the sorted copy under column phases.
    auto run_segment = [&](const int rs, const int re, const int fo, const int ln,
                           const int* __restrict__ cx, const float* __restrict__ vx,
                           const bool banded) {
        const bool bph = PH && ph && banded;
        const int rlo = max(rs, 0);
        const int rhi = min(re, n_rows);
        for (int pass = 0; pass < npass; ++pass) {
            const int fl = pass * G * R + sub;  // first vector element of this lane
            int r = rlo;
            while (r < rhi) {
                // With groups of 32 or more short rows, each lane of the first
                // GROUP reads its row's chunk before the long/short decision,
                // which takes lane 0's (row r): the group's offsets and row
                // r's arrive in one memory round trip (measured on the 16M-row
                // mesh: 1.7-3.5% faster).  Smaller groups read row r's chunk
                // alone first (faster on R-MAT, whose runs hold long rows).
                constexpr bool kEarly = GROUP >= 32;
                const int lane_g = fresh(threadIdx.x & 63);
                const int rr = r + lane_g;
                const bool mine = lane_g < GROUP && rr < rhi;
                Chunk my = {0, 0, 0, 0};
                Chunk c0;
                if constexpr (kEarly) {
                    if (mine) my = task_chunk<PH>(rp, rr, rs, re, fo, ln, nnz, bph, pb, pe);
                    c0.base = __builtin_amdgcn_readfirstlane(my.base);
                    c0.b = __builtin_amdgcn_readfirstlane(my.b);
                    c0.e = __builtin_amdgcn_readfirstlane(my.e);
                    c0.d = __builtin_amdgcn_readfirstlane(my.d);
                    if constexpr (PH) c0.own = __builtin_amdgcn_readfirstlane(my.own);
                } else {
                    c0 = task_chunk<PH>(rp, r, rs, re, fo, ln, nnz, bph, pb, pe);
                }
                const int len0 = c0.e - c0.b;
                if (len0 >= kLong) {
                    // ---------------- long chunk: all slots on one row
                    V acc[R];
#pragma unroll
                    for (int q = 0; q < R; ++q) acc[q] = vzero<VEC>();
                    // (an unsigned step: a chunk may end within 64 of 2^31)
                    for (unsigned uw = c0.b; uw < static_cast<unsigned>(c0.e); uw += 64u) {
                        const int w0 = static_cast<int>(uw);
                        const int wn = min(64, c0.e - w0);
                        const int lane = fresh(threadIdx.x & 63);
                        int colw = 0;
                        float valw = 0.0f;
                        if (lane < wn) {
                            colw = __builtin_nontemporal_load(cx + c0.base + w0 + lane);
                            valw = __builtin_nontemporal_load(vx + c0.base + w0 + lane);
                            if constexpr (HN) colw = with_hint(colw, hints, c0.base + w0 + lane);
                        }
                        for (int k0 = 0; k0 < wn; k0 += STEP) {
                            int cc[UL];
                            float a[UL];
                            bool ok[UL];
                            bool cold[UL];
                            const int sl = fresh(slot);
#pragma unroll
                            for (int u = 0; u < UL; ++u) {
                                const int jj = k0 + u * NS + sl;
                                cc[u] = __shfl(colw, jj & 63);
                                a[u] = __shfl(valw, jj & 63);
                                cold[u] = HN && cc[u] < 0;
                                if constexpr (HN) cc[u] &= 0x7fffffff;
                                ok[u] = jj < wn;
                                if (ok[u] && static_cast<unsigned long long>(cc[u]) >=
                                                 static_cast<unsigned long long>(h_rows)) {
                                    ok[u] = false;
                                    bad |= 1;
                                }
                            }
                            V h[UL][R];
#pragma unroll
                            for (int u = 0; u < UL; ++u) {
                                const float* hrow = Hs + static_cast<size_t>(cc[u]) * ld;
#pragma unroll
                                for (int q = 0; q < R; ++q) {
                                    const int f = fl + G * q;
                                    if constexpr (HN)
                                        h[u][q] = (ok[u] && f < F)
                                                      ? gather_hinted(hrsrc,
                                                                      static_cast<unsigned>(cc[u]) * ld * 4u +
                                                                          slice_bytes + f * 16u,
                                                                      cold[u])
                                                      : vzero<VEC>();
                                    else
                                        h[u][q] = (ok[u] && f < F) ? vload<VEC>(hrow + f * VEC)
                                                                   : vzero<VEC>();
                                }
                            }
#pragma unroll
                            for (int u = 0; u < UL; ++u) {
                                if (ok[u]) {
#pragma unroll
                                    for (int q = 0; q < R; ++q) acc[q] = vfma(a[u], h[u][q], acc[q]);
                                }
                            }
                        }
                    }
#pragma unroll
                    for (int off = G; off < 64; off <<= 1) {
#pragma unroll
                        for (int q = 0; q < R; ++q) acc[q] = acc[q] + vshfl_xor(acc[q], off);
                    }
                    const int o = origin[r];
                    if (static_cast<unsigned>(o) >= static_cast<unsigned>(n_rows)) {
                        bad |= 2;
                    } else if (slot == 0) {
                        float* crow = Cs + static_cast<size_t>(o) * ld;
                        const float fd = static_cast<float>(c0.d);
                        const int how = write_mode<PH>(bph, first, c0);
#pragma unroll
                        for (int q = 0; q < R; ++q) {
                            const int f = fl + G * q;
                            if (f < F) write_row<VEC>(crow + f * VEC, vdiv(acc[q], fd), how);
                        }
                    }
                    ++r;
                    continue;
                }

                // ---------------- short rows: one row per slot, RU rows per slot
                const int lane = lane_g;
                if constexpr (!kEarly) {
                    if (mine) my = task_chunk<PH>(rp, rr, rs, re, fo, ln, nnz, bph, pb, pe);
                }
                const int mylen = my.e - my.b;
                // The group: the leading rows that are short, start where the
                // previous row's chunk ends (always, for a non-decreasing
                // row_ptr) and end within kWin nonzeros of the group's start.
                // The first row always qualifies (its chunk is shorter than
                // kLong <= kWin), so every group makes progress, and the
                // group's nonzeros are the contiguous range [gs, gs + gn).
                const int mys = my.base + my.b;
                const int mye = my.base + my.e;
                const int gs = c0.base + c0.b;
                const int prev_end = __shfl_up(mye, 1);
                const bool fits = mine && mylen < kLong && (lane == 0 || mys == prev_end) &&
                                  mye - gs <= kWin;
                const unsigned long long stop = __ballot(!fits);
                int cnt = min(GROUP, rhi - r);
                if (stop) cnt = min(cnt, static_cast<int>(__ffsll(static_cast<long long>(stop))) - 1);
                const int myo = (mine && lane < cnt) ? origin[rr] : 0;
                const int ge = __shfl(mye, cnt - 1);
                const int gn = (gs >= 0 && static_cast<long long>(ge) <= nnz) ? ge - gs : 0;
                int colw = 0;
                float valw = 0.0f;
                if constexpr (kStage > 0) {
                    // The previous group's reads of this wave's window are done
                    // (wave-ordered LDS); the fences keep the compiler from
                    // moving accesses across the exchange.
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                    __builtin_amdgcn_wave_barrier();
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                    // All loads first, then the LDS writes: one memory round trip.
                    constexpr int NT = (kStage + 63) / 64;
                    int lc[NT];
                    float lv[NT];
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        const int i = lane + 64 * t;
                        lc[t] = i < gn ? __builtin_nontemporal_load(cx + gs + i) : 0;
                        lv[t] = i < gn ? __builtin_nontemporal_load(vx + gs + i) : 0.0f;
                        if constexpr (HN)
                            if (i < gn) lc[t] = with_hint(lc[t], hints, gs + i);
                    }
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        const int i = lane + 64 * t;
                        if (i < gn) {
                            wcol[i] = lc[t];
                            wval[i] = lv[t];
                        }
                    }
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                    __builtin_amdgcn_wave_barrier();
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                } else if (lane < gn) {
                    colw = __builtin_nontemporal_load(cx + gs + lane);
                    valw = __builtin_nontemporal_load(vx + gs + lane);
                    if constexpr (HN) colw = with_hint(colw, hints, gs + lane);
                }
                V acc[RU][R];
                int pos[RU];
                int len[RU];
                int maxlen = 0;
#pragma unroll
                for (int u = 0; u < RU; ++u) {
                    const int gi = u * NS + fresh(slot);
                    pos[u] = __shfl(mys - gs, gi);  // window position of the chunk
                    len[u] = __shfl(mylen, gi);
                    if (gi >= cnt) len[u] = 0;
                    maxlen = max(maxlen, len[u]);
#pragma unroll
                    for (int q = 0; q < R; ++q) acc[u][q] = vzero<VEC>();
                }
                const int jmax = wave_max(maxlen);
                for (int j = 0; j < jmax; ++j) {
                    int cc[RU];
                    float a[RU];
                    bool ok[RU];
                    bool cold[RU];
#pragma unroll
                    for (int u = 0; u < RU; ++u) {
                        ok[u] = j < len[u];
                        const int src = pos[u] + j;  // in [0, gn) whenever ok[u]
                        if constexpr (kStage > 0) {
                            cc[u] = wcol[ok[u] ? src : 0];
                            a[u] = wval[ok[u] ? src : 0];
                        } else {
                            cc[u] = __shfl(colw, src & 63);
                            a[u] = __shfl(valw, src & 63);
                        }
                        cold[u] = HN && cc[u] < 0;
                        if constexpr (HN) cc[u] &= 0x7fffffff;
                        if (ok[u] && static_cast<unsigned long long>(cc[u]) >=
                                         static_cast<unsigned long long>(h_rows)) {
                            ok[u] = false;
                            bad |= 1;
                        }
                    }
                    V h[RU][R];
#pragma unroll
                    for (int u = 0; u < RU; ++u) {
                        const float* hrow = Hs + static_cast<size_t>(cc[u]) * ld;
#pragma unroll
                        for (int q = 0; q < R; ++q) {
                            const int f = fl + G * q;
                            if constexpr (HN)
                                h[u][q] = (ok[u] && f < F)
                                              ? gather_hinted(hrsrc,
                                                              static_cast<unsigned>(cc[u]) * ld * 4u +
                                                                  slice_bytes + f * 16u,
                                                              cold[u])
                                              : vzero<VEC>();
                            else
                                h[u][q] = (ok[u] && f < F) ? vload<VEC>(hrow + f * VEC) : vzero<VEC>();
                        }
                    }
#pragma unroll
                    for (int u = 0; u < RU; ++u) {
                        if (ok[u]) {
#pragma unroll
                            for (int q = 0; q < R; ++q) acc[u][q] = vfma(a[u], h[u][q], acc[u][q]);
                        }
                    }
                }
#pragma unroll
                for (int u = 0; u < RU; ++u) {
                    const int gi = u * NS + fresh(slot);
                    const int o = __shfl(myo, gi);
                    Chunk cu;
                    cu.d = __shfl(my.d, gi);
                    cu.b = __shfl(my.b, gi);
                    cu.e = __shfl(my.e, gi);
                    if constexpr (PH) cu.own = __shfl(my.own, gi);
                    if (gi < cnt) {
                        if (cu.d < 0) {
                            bad |= 4;
                            continue;
                        }
                        if (static_cast<unsigned>(o) >= static_cast<unsigned>(n_rows)) {
                            bad |= 2;
                            continue;
                        }
                        float* crow = Cs + static_cast<size_t>(o) * ld;
                        if (cu.d == 0) {
                            if (first && write_empty) {
#pragma unroll
                                for (int q = 0; q < R; ++q) {
                                    const int f = fl + G * q;
                                    if (f < F) vstore_nt<VEC>(crow + f * VEC, vzero<VEC>());
                                }
                            }
                        } else if (cu.e > cu.b || (bph && first && cu.own)) {
                            // (an owned row with no nonzero in the first phase
                            // is stored as zeros all the same)
                            const float fd = static_cast<float>(cu.d);
                            const int how = write_mode<PH>(bph, first, cu);
#pragma unroll
                            for (int q = 0; q < R; ++q) {
                                const int f = fl + G * q;
                                if (f < F) write_row<VEC>(crow + f * VEC, vdiv(acc[u][q], fd), how);
                            }
                        }
                    }
                }
                r += cnt;
            }
        }
    };

    // The run's tasks, 64 at a time: the window's segment starts by ballot
    // (one coalesced load of the window), then the segments in order, each
    // reading its first and last task.
    const long long t0 = run * M;
    const int cnt = static_cast<int>(min(static_cast<long long>(M), n_tasks - t0));
    if constexpr (PH) {
        if (ph) {
            // A chain under column phases: the run takes, whole, every row
            // whose first nonzero lies in its tasks -- from its first task's
            // row (the next row when that task continues a row begun
            // earlier) to its last task's row, completed -- so each row has
            // one wave and no atomics.  The chain's ends keep their offsets:
            // the first task's start, and the last task's end in its row.
            const cwlb_task a = tasks[t0];
            const cwlb_task z = tasks[t0 + cnt - 1];
            const cwlb_task zl = tasks[n_tasks - 1];
            const bool head = t0 == 0;
            const int rs = (head || a.first_row_offset == 0) ? a.row_start : a.row_start + 1;
            const int re = z.row_end;
            const int fo = head ? a.first_row_offset : 0;
            const int ln = re == zl.row_end ? zl.last_row_nnz : 0;
            if (rs < re) {
                // Task offsets index the caller's order of a row's nonzeros:
                // the rows the chain covers only in part (its first row when
                // it starts inside it, its last when it ends at an offset)
                // are summed whole from ci / val in the first phase; the
                // others band by band from the sorted copy.
                const int bs = rs + (fo > 0 ? 1 : 0);
                const int be = max(bs, re - (ln > 0 ? 1 : 0));
                for (int piece = 0; piece < 3; ++piece) {
                    int s = bs, e = be, pfo = 0, pln = 0;
                    bool banded = true;
                    if (piece == 1) {  // the first row, from offset fo
                        if (!first || fo == 0) continue;
                        s = rs;
                        e = rs + 1;
                        pfo = fo;
                        pln = (ln > 0 && re == rs + 1) ? ln : 0;
                        banded = false;
                    } else if (piece == 2) {  // the last row, up to offset ln
                        if (!first || ln == 0 || (fo > 0 && re == rs + 1)) continue;
                        s = re - 1;
                        e = re;
                        pln = ln;
                        banded = false;
                    }
                    if (s < e)
                        run_segment(s, e, pfo, pln, banded ? ci_b : ci, banded ? val_b : val,
                                    banded);
                }
            }
            if (bad) atomicOr(status, bad);
            return;
        }
    }
    for (int w = 0; w < cnt; w += 64) {
        const int wn = min(64, cnt - w);
        const long long tw = t0 + w;
        unsigned long long rest;
        {
            // Lane i compares task i of the window with task i - 1 (both
            // loaded by the lane itself: a cross-lane shuffle here would keep
            // a lane-id register alive through the whole kernel).
            const int lane = fresh(threadIdx.x & 63);
            bool brk = lane == 0;
            if (lane > 0 && lane < wn)
                brk = segment_break(tasks[tw + lane - 1], tasks[tw + lane], w + lane, n_rows);
            rest = __ballot(lane < wn && brk);
        }
        do {
            const int s0 = __builtin_ctzll(rest);
            rest &= rest - 1;
            const int e0 = rest ? __builtin_ctzll(rest) : wn;
            const cwlb_task a = tasks[tw + s0];
            const cwlb_task z = tasks[tw + e0 - 1];
            run_segment(a.row_start, z.row_end, a.first_row_offset, z.last_row_nnz, ci, val,
                        false);
        } while (rest);
    }
    if (bad) atomicOr(status, bad);
}

// Clears the C rows that receive atomic partial sums.  One lane per task,
// with the segment rule of the aggregation kernel.  Only a task's last row
// can be left open (its chunk starts at nonzero 0 and stops before the
// row's end; a first row that is not also the last always runs to the row's
// end).  The row is completed inside the segment, and later stored whole,
// when the following tasks continue it (no segment start in between) up to
// one whose chunk reaches the row's end; otherwise every segment adds a part
// of it atomically and it is cleared here.  The look-ahead counts a task as
// reaching the row's end when it has more rows or ends on a row boundary
// (a one-row task with last_row_nnz >= deg reaches it too but is passed
// over, which can only clear more), and stops at the wave's last lane: a
// row it cannot follow further is cleared, which costs only a store when
// the row is later stored whole.  So only the tasks that open a row read
// row offsets.  The wave clears the marked rows with coalesced stores.
// Block 0 also resets the status word.  For a column-phased call (seq > 0)
// the pass also checks that the list is a chain -- every task well formed
// and continuing its predecessor, so that no two tasks share a nonzero and
// a row covered whole by one segment is touched by no other -- and
// otherwise writes seq into status[1] (the call's band sort, which runs
// just before, cleared it; seq is never 0).
template <int VEC>
__global__ void __launch_bounds__(kAuxBlock)
zero_split_rows(const int* __restrict__ rp, const int* __restrict__ origin, int n_rows,
                long long nnz, const cwlb_task* __restrict__ tasks, long long n_tasks, int M,
                int K, float* __restrict__ C, int* __restrict__ status, int seq)
{
    const int lane = threadIdx.x & 63;
    const long long t = static_cast<long long>(blockIdx.x) * kAuxBlock + threadIdx.x;
    if (blockIdx.x == 0 && threadIdx.x == 0) *status = 0;
    cwlb_task cur{0, 0, 0, 0};
    if (t < n_tasks) cur = tasks[t];
    cwlb_task prev = shfl_up_task(cur);
    if (lane == 0 && t > 0 && t < n_tasks) prev = tasks[t - 1];
    bool brk = true;    // task t starts a segment (lanes past the end count as starts)
    bool ends = false;  // task t's chunk of its first row reaches that row's end
    int o = -1;         // original id of the row task t leaves open
    bool unlinked = false;  // task t breaks the chain
    if (t < n_tasks) {
        brk = segment_break(prev, cur, t % M, n_rows);
        unlinked = !task_well_formed(cur, n_rows) ||
                   (t > 0 && (!task_well_formed(prev, n_rows) || !continues(prev, cur)));
        const int rs = cur.row_start, re = cur.row_end;
        const int fo = cur.first_row_offset, ln = cur.last_row_nnz;
        int r = -1;  // the candidate row
        if (task_well_formed(cur, n_rows)) {
            ends = re - rs > 1 || ln == 0;
            if (ln > 0 && (re - rs > 1 || fo == 0)) r = re - 1;
        } else if (max(rs, 0) < min(re, n_rows)) {
            r = min(re, n_rows) - 1;  // clamped rows, as the kernel executes them
        }
        if (r >= 0) {
            const Chunk z = row_chunk(rp, r, rs, re, fo, ln, nnz);
            if (z.d > 0 && z.b == 0 && z.e > 0 && z.e < z.d) o = origin[r];
        }
        if (o >= n_rows) o = -1;
    }
    if (seq > 0 && __ballot(unlinked) != 0ull && lane == 0) status[1] = seq;
    const unsigned long long mb = __ballot(brk);
    const unsigned long long me = __ballot(ends);
    if (o >= 0 && lane < 63) {
        const unsigned long long ahead = (mb | me) >> (lane + 1);
        if (ahead) {
            const int u = lane + 1 + __builtin_ctzll(ahead);
            if (!((mb >> u) & 1ull)) o = -1;  // completed inside the segment
        }
    }
    const int F = K / VEC;
    unsigned long long m = __ballot(o >= 0);
    while (m) {
        const int src = __ffsll(static_cast<long long>(m)) - 1;
        m &= m - 1;
        const int row = __shfl(o, src);
        float* crow = C + static_cast<size_t>(row) * K;
        for (int f = lane; f < F; f += 64) vstore<VEC>(crow + f * VEC, vzero<VEC>());
    }
}

// Clears n floats (graph-capture safe, unlike a memset node): 16-byte
// stores from the first 16-byte boundary, single floats before it and after
// the last whole vector.
__global__ void __launch_bounds__(kAuxBlock) fill_zero(float* __restrict__ p, long long n,
                                                    int* __restrict__ status)
{
    if (blockIdx.x == 0 && threadIdx.x == 0 && status) *status = 0;
    const long long gid = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    const long long stride = static_cast<long long>(gridDim.x) * blockDim.x;
    const unsigned long long addr = reinterpret_cast<unsigned long long>(p);
    long long head = (addr & 3ull) ? n : static_cast<long long>(((16ull - (addr & 15ull)) & 15ull) >> 2);
    head = head < n ? head : n;
    for (long long i = gid; i < head; i += stride) p[i] = 0.0f;
    const long long n4 = (n - head) / 4;
    f4* p4 = reinterpret_cast<f4*>(p + head);
    for (long long i = gid; i < n4; i += stride) p4[i] = f4(0.0f);
    for (long long i = head + n4 * 4 + gid; i < n; i += stride) p[i] = 0.0f;
}

__device__ __forceinline__ unsigned long long mix64(unsigned long long z)
{
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__global__ void __launch_bounds__(kAuxBlock)
fill_features(float* __restrict__ H, long long total, unsigned long long s)
{
    const long long stride = static_cast<long long>(gridDim.x) * blockDim.x;
    for (long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += stride) {
        const unsigned long long x = mix64(s + static_cast<unsigned long long>(i));
        const int u = static_cast<int>(x >> 40);
        H[i] = static_cast<float>(u - 8388608) * 0x1.0p-23f;
    }
}

unsigned long long host_mix64(unsigned long long z)
{
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Launch geometry of one call: M tasks per wave, SL feature slices.
struct Plan {
    int vec;
    int sl;
    int M;
    long long runs;
    long long blocks;      // run blocks per slice
    long long chunk;       // run blocks per XCD when contiguous, else 0
    long long grid;        // launched blocks
    bool ordered;          // runs execute sorted by output row id
    bool o6;               // the 6-waves-per-SIMD variant
    bool packed;           // packed slots (G lanes x R vectors, see pick_tiling)
    int G;                 // lanes per slot of the launch
    int R;                 // vectors per lane and pass of the launch
    const int* order;      // that order (device), set at launch
    const unsigned long long* hints;  // cold-column bits (device) or null
    int phases;            // column phases (1 = none)
    // The launch's phase: its row bounds (null = the row's own start / end),
    // whether it is the first, and the call's sequence number.
    const int* pb;
    const int* pe;
    const int* cb;    // the band-sorted copy of the columns
    const float* vb;  // and of the values
    int first;
    int seq;
    int write_empty;  // store rows without nonzeros (as zeros)
};

// Launches one instantiation; returns its resident waves per CU at most
// (from its register and LDS use, queried once per instantiation).
template <int VEC, int G, int R, int SL, bool HN = false, bool O6 = false, bool PH = false>
int launch_main(hipStream_t st, const SpmmArgs& a, const Plan& p, int* status)
{
    constexpr int U = (R == 1) ? 8 : (R == 2) ? 4 : (R <= 4) ? 2 : 1;
    static const int waves_per_cu = [] {
        int blocks = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &blocks,
                reinterpret_cast<const void*>(&spmm_mean_runs<VEC, G, R, U, SL, HN, O6, PH>),
                kBlock, 0) != hipSuccess)
            blocks = 0;
        return blocks * kWaves;
    }();
    hipLaunchKernelGGL((spmm_mean_runs<VEC, G, R, U, SL, HN, O6, PH>),
                       dim3(static_cast<unsigned>(p.grid)), dim3(kBlock), 0, st, a.row_ptr,
                       a.col_idx, a.val, a.origin, a.n_rows, static_cast<long long>(a.nnz), a.H,
                       static_cast<long long>(a.h_rows), a.K, a.tasks,
                       static_cast<long long>(a.n_tasks), p.M, p.runs, p.blocks, p.chunk, p.order,
                       p.hints, a.C, status, p.pb, p.pe, p.cb, p.vb, p.first, p.seq,
                       p.write_empty);
    return waves_per_cu;
}

// Column phases: 16-byte lanes, one vector per lane, no hints, the
// standard kernel.
template <int SL>
int dispatch_phased(hipStream_t st, const SpmmArgs& a, const Plan& p, int* status, int G)
{
    switch (G) {
    case 1: return launch_main<4, 1, 1, SL, false, false, true>(st, a, p, status);
    case 2: return launch_main<4, 2, 1, SL, false, false, true>(st, a, p, status);
    case 4: return launch_main<4, 4, 1, SL, false, false, true>(st, a, p, status);
    case 8: return launch_main<4, 8, 1, SL, false, false, true>(st, a, p, status);
    case 16: return launch_main<4, 16, 1, SL, false, false, true>(st, a, p, status);
    case 32: return launch_main<4, 32, 1, SL, false, false, true>(st, a, p, status);
    default: return launch_main<4, 64, 1, SL, false, false, true>(st, a, p, status);
    }
}

// Feature slices of one lane group (one vector per lane) under cache hints.
template <int VEC, int SL>
int dispatch_hinted(hipStream_t st, const SpmmArgs& a, const Plan& p, int* status, int G)
{
    switch (G) {
    case 1: return launch_main<VEC, 1, 1, SL, true>(st, a, p, status);
    case 2: return launch_main<VEC, 2, 1, SL, true>(st, a, p, status);
    case 4: return launch_main<VEC, 4, 1, SL, true>(st, a, p, status);
    case 8: return launch_main<VEC, 8, 1, SL, true>(st, a, p, status);
    case 16: return launch_main<VEC, 16, 1, SL, true>(st, a, p, status);
    case 32: return launch_main<VEC, 32, 1, SL, true>(st, a, p, status);
    default: return launch_main<VEC, 64, 1, SL, true>(st, a, p, status);
    }
}

// The occupancy variant: slots of 4, 8 or 16 lanes of 16 bytes.
template <int SL, bool HN>
int dispatch_o6(hipStream_t st, const SpmmArgs& a, const Plan& p, int* status, int G)
{
    switch (G) {
    case 4: return launch_main<4, 4, 1, SL, HN, true>(st, a, p, status);
    case 8: return launch_main<4, 8, 1, SL, HN, true>(st, a, p, status);
    default: return launch_main<4, 16, 1, SL, HN, true>(st, a, p, status);
    }
}

// Packed slots (16-byte lanes): G lanes of R = 3 or 5 vectors each, for the
// slices those cover with fewer idle lanes than one vector per lane in a
// power-of-two slot.  Slices of at most 64 vectors (all variants) use
// G x R in {4x3, 4x5, 8x3, 8x5, 16x3}; wider ones (plain kernel only) also
// 16x5, 32x3 and 32x5 (64x3 and 64x5 are the SL = 1 wide tilings).
template <int SL, bool HN, bool PH>
int dispatch_packed(hipStream_t st, const SpmmArgs& a, const Plan& p, int* status)
{
    switch (p.G * 10 + p.R) {
    case 43: return launch_main<4, 4, 3, SL, HN, false, PH>(st, a, p, status);
    case 45: return launch_main<4, 4, 5, SL, HN, false, PH>(st, a, p, status);
    case 83: return launch_main<4, 8, 3, SL, HN, false, PH>(st, a, p, status);
    case 85: return launch_main<4, 8, 5, SL, HN, false, PH>(st, a, p, status);
    default: return launch_main<4, 16, 3, SL, HN, false, PH>(st, a, p, status);
    }
}

template <int SL>
int dispatch_packed_wide(hipStream_t st, const SpmmArgs& a, const Plan& p, int* status)
{
    switch (p.G * 10 + p.R) {
    case 165: return launch_main<4, 16, 5, SL>(st, a, p, status);
    case 323: return launch_main<4, 32, 3, SL>(st, a, p, status);
    case 325: return launch_main<4, 32, 5, SL>(st, a, p, status);
    case 643: return launch_main<4, 64, 3, SL>(st, a, p, status);
    case 645: return launch_main<4, 64, 5, SL>(st, a, p, status);
    default: return dispatch_packed<SL, false, false>(st, a, p, status);
    }
}

template <int VEC, int SL>
int dispatch_width(hipStream_t st, const SpmmArgs& a, const Plan& p, int* status)
{
    const int F = (a.K / VEC + SL - 1) / SL;  // vectors of the widest slice
    if constexpr (VEC == 4) {
        if (p.packed) {
            if (p.phases > 1) return dispatch_packed<SL, false, true>(st, a, p, status);
            if (p.hints) return dispatch_packed<SL, true, false>(st, a, p, status);
            return dispatch_packed_wide<SL>(st, a, p, status);
        }
    }
    if (F <= 64) {
        int G = 1;
        while (G < F) G <<= 1;
        if constexpr (VEC == 4) {
            if (p.phases > 1) return dispatch_phased<SL>(st, a, p, status, G);
            if (p.o6 && G >= 4 && G <= 16) {
                if (p.hints) return dispatch_o6<SL, true>(st, a, p, status, G);
                return dispatch_o6<SL, false>(st, a, p, status, G);
            }
            if (p.hints) return dispatch_hinted<VEC, SL>(st, a, p, status, G);
        }
        switch (G) {
        case 1: return launch_main<VEC, 1, 1, SL>(st, a, p, status);
        case 2: return launch_main<VEC, 2, 1, SL>(st, a, p, status);
        case 4: return launch_main<VEC, 4, 1, SL>(st, a, p, status);
        case 8: return launch_main<VEC, 8, 1, SL>(st, a, p, status);
        case 16: return launch_main<VEC, 16, 1, SL>(st, a, p, status);
        case 32: return launch_main<VEC, 32, 1, SL>(st, a, p, status);
        default: return launch_main<VEC, 64, 1, SL>(st, a, p, status);
        }
    }
    if constexpr (SL != 1) {
        // Wider slices than one wave: the kernel loops over feature passes.
        return launch_main<VEC, 64, 1, SL>(st, a, p, status);
    } else {
        const int R = std::min((F + 63) / 64, 8);
        switch (R) {
        case 2: return launch_main<VEC, 64, 2, 1>(st, a, p, status);
        case 3: return launch_main<VEC, 64, 3, 1>(st, a, p, status);
        case 4: return launch_main<VEC, 64, 4, 1>(st, a, p, status);
        case 5: return launch_main<VEC, 64, 5, 1>(st, a, p, status);
        case 6: return launch_main<VEC, 64, 6, 1>(st, a, p, status);
        case 7: return launch_main<VEC, 64, 7, 1>(st, a, p, status);
        default: return launch_main<VEC, 64, 8, 1>(st, a, p, status);
        }
    }
}

template <int VEC>
int dispatch_main(hipStream_t st, const SpmmArgs& a, const Plan& p, int* status)
{
    if (p.sl == 8) return dispatch_width<VEC, 8>(st, a, p, status);
    if (p.sl == 4) return dispatch_width<VEC, 4>(st, a, p, status);
    if (p.sl == 2) return dispatch_width<VEC, 2>(st, a, p, status);
    return dispatch_width<VEC, 1>(st, a, p, status);
}

template <int VEC>
void launch_zero(hipStream_t st, const SpmmArgs& a, const Plan& p, int* status)
{
    const long long blocks = (a.n_tasks + kAuxBlock - 1) / kAuxBlock;
    hipLaunchKernelGGL(zero_split_rows<VEC>, dim3(static_cast<unsigned>(blocks)), dim3(kAuxBlock), 0,
                       st, a.row_ptr, a.origin, a.n_rows, static_cast<long long>(a.nnz), a.tasks,
                       static_cast<long long>(a.n_tasks), p.M, a.K, a.C, status,
                       p.phases > 1 ? p.seq : 0);
}

int pick_vec(const SpmmArgs& a)
{
    const auto h = reinterpret_cast<uintptr_t>(a.H);
    const auto c = reinterpret_cast<uintptr_t>(a.C);
    if (a.K % 4 == 0 && h % 16 == 0 && c % 16 == 0) return 4;
    if (a.K % 2 == 0 && h % 8 == 0 && c % 8 == 0) return 2;
    return 1;
}

// The slot tiling of a slice of F vectors: G lanes per slot, R vectors per
// lane and pass, ceil(F / (G R)) passes over the row's nonzeros.
// Power-of-two slots: G the smallest power of two >= F with R = 1
// (F <= 64); wider slices G = 64 and, without feature slices,
// R = ceil(F / 64) up to 8.  Packed slots: for F <= 64, of those and the
// one-pass G x R in {4x3, 4x5, 8x3, 8x5, 16x3}, the fewest vector loads per
// nonzero (G R: the fewest idle lanes), the smaller R on a tie; for wider
// slices, of those and 16x5, 32x3, 32x5, 64x3 and 64x5, the fewest passes
// (each pass reads the row's indices again), then the fewest loads, then
// the smaller R.  wide: slices above 64 vectors may use the wide tilings
// (not under hints or column phases).
void pick_tiling(int F, int SL, bool packed, bool wide, int* G_out, int* R_out)
{
    int G = 64, R = 1;
    if (F <= 64) {
        G = 1;
        while (G < F) G <<= 1;
    } else if (SL == 1) {
        R = std::min((F + 63) / 64, 8);
    }
    if (packed) {
        auto passes = [F](int g, int r) { return (F + g * r - 1) / (g * r); };
        auto better = [&](int g, int r) {
            const long long c = static_cast<long long>(passes(g, r)) * g * r;
            const long long c0 = static_cast<long long>(passes(G, R)) * G * R;
            if (passes(g, r) != passes(G, R)) return passes(g, r) < passes(G, R);
            if (c != c0) return c < c0;
            return r < R;
        };
        const int narrow[5][2] = {{4, 3}, {4, 5}, {8, 3}, {8, 5}, {16, 3}};
        const int wide_t[5][2] = {{16, 5}, {32, 3}, {32, 5}, {64, 3}, {64, 5}};
        if (F <= 64) {
            for (const auto& t : narrow)
                if (t[0] * t[1] >= F && better(t[0], t[1])) {
                    G = t[0];
                    R = t[1];
                }
        } else if (wide) {
            for (const auto& t : wide_t)
                if ((t[0] < 64 || SL == 1) && better(t[0], t[1])) {
                    G = t[0];
                    R = t[1];
                }
        }
    }
    *G_out = G;
    *R_out = R;
}

// Automatic schedule (the context's settings override each choice):
//   * feature slices across XCDs only when the feature matrix is well beyond
//     what the 256 MB Infinity Cache holds (>= 512 MB): then each XCD's L2
//     caching a slice of the hot rows pays; below that, slicing only
//     multiplies the per-row work (measured: Chung-Lu K=64, H = 256 MB, 10%
//     slower with 2 slices).  Slices of 32 to 128 floats are best: 2 slices
//     up to K = 256, 4 slices up to K = 512 (measured on R-MAT, H = 2 to
//     8.6 GB: K=128 2 slices 1.4% faster than 4, K=256 3.5% faster; K=512
//     4 slices 2% faster than 2; K=192 2 slices 18% faster than 1);
//   * tasks per wave M: the largest M that keeps at least 64 waves per CU
//     (runs x slices) and at most ~256 rows per run (long runs of short rows
//     serialise latency: the 16M-row mesh is 9% faster at 4 tasks per wave
//     than at 16), clamped to [1, 64].
Plan make_plan(const cwlb_ctx* ctx, const SpmmArgs& a, bool per_task)
{
    Plan p{};
    p.vec = pick_vec(a);
    p.M = 1;
    p.sl = 1;
    if (!per_task) {
        const long long h_bytes = a.h_rows * static_cast<long long>(a.K) * 4;
        if (ctx->sched_slices > 0) {
            p.sl = ctx->sched_slices;
        } else if (h_bytes >= (512ll << 20)) {
            if (a.K % 64 == 0 && a.K >= 64 && a.K <= 256) p.sl = 2;
            else if (a.K % 128 == 0 && a.K > 256 && a.K <= 512) p.sl = 4;
        }
        if (p.vec != 4 || a.K / 4 < p.sl) p.sl = 1;
        if (ctx->sched_tasks_per_wave > 0) {
            p.M = ctx->sched_tasks_per_wave;
        } else {
            const long long waves = static_cast<long long>(std::max(ctx->compute_units, 1)) * 64;
            const long long m_par = a.n_tasks * p.sl / waves;
            const long long m_rows = a.n_rows > 0 ? 256 * a.n_tasks / a.n_rows : 64;
            p.M = static_cast<int>(std::max<long long>(1, std::min({m_par, m_rows, 64ll})));
        }
    }
    const bool contiguous = !per_task && ctx->sched_xcd == 2;
    for (;;) {
        p.runs = (a.n_tasks + p.M - 1) / p.M;
        p.blocks = (p.runs + kWaves - 1) / kWaves;
        if (contiguous) {
            const long long P = 8 / p.sl;
            p.chunk = (p.blocks + P - 1) / P;
            p.grid = p.chunk * 8;
        } else {
            p.chunk = 0;
            p.grid = p.sl == 1 ? p.blocks : (p.blocks * p.sl + 7) / 8 * 8;
        }
        // An automatic run length grows until the grid fits one launch.
        if (p.grid <= kMaxGridBlocks || per_task || ctx->sched_tasks_per_wave > 0) break;
        p.M *= 2;
    }
    p.ordered = !per_task && ctx->sched_order == 2 && p.runs > 1;
    // The occupancy variant exists for 16-byte lanes and slots of 4 to 16
    // lanes (more than 8 and at most 64 floats per feature slice).
    const int f4 = (a.K / 4 + p.sl - 1) / p.sl;  // vectors of the widest slice
    p.o6 = !per_task && ctx->sched_occupancy == 6 && p.vec == 4 && f4 > 2 && f4 <= 16;
    p.order = nullptr;
    p.hints = nullptr;
    // Column phases: 16-byte lanes and at most 64 vectors per slice; they
    // replace the occupancy variant and the cache hints.
    p.phases = 1;
    if (!per_task && ctx->sched_phases > 1 && p.vec == 4 && f4 <= 64 && a.h_rows > 0) {
        p.phases = ctx->sched_phases;
        p.o6 = false;
    }
    p.pb = nullptr;
    p.pe = nullptr;
    p.cb = nullptr;
    p.vb = nullptr;
    p.first = 1;
    p.seq = 0;
    p.write_empty = 1;
    // Packed slots: 16-byte lanes, not with the occupancy variant or one
    // task per wave.  The tiling is settled at launch (hints and phases
    // restrict it).
    p.packed = !per_task && ctx->sched_tiling == 2 && p.vec == 4 && !p.o6;
    p.G = 0;
    p.R = 0;
    return p;
}

}  // namespace

cwlb_status launch_spmm_mean(cwlb_ctx* ctx, const SpmmArgs& a, bool zero_all, bool per_task,
                             bool keep_empty, bool record_events)
{
    hipStream_t st = ctx->stream;
    (void)hipGetLastError();  // report only the launches below
    Plan p = make_plan(ctx, a, per_task);
    // Rows without nonzeros hold zeros already when this call clears C, or
    // when the caller says an earlier one did.
    p.write_empty = zero_all || keep_empty ? 0 : 1;
    if (a.n_tasks > kMaxGridBlocks * kBlock && a.K > 0)
        return fail(CWLB_UNSUPPORTED, "spmm: more than 2^32 tasks");
    if (p.grid > kMaxGridBlocks && a.n_tasks > 0 && a.K > 0)
        return fail(CWLB_UNSUPPORTED,
                    "spmm: too many runs for one launch (more than 2^32 work-items); use more "
                    "tasks per wave (cwlb_ctx_set_schedule) or a larger S");
    // Under graph capture the run order and the cache hints are only reused,
    // never built (building allocates and synchronises); without them the
    // launch runs in task order with the normal cache policy, which gives
    // the same results.
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    CWLB_HIP_TRY(hipStreamIsCapturing(st, &capture));
    const bool may_build = capture == hipStreamCaptureStatusNone;
    const bool work = a.n_tasks > 0 && a.K > 0;
    // Column phases: the context's buffers for the band sort (under capture
    // only when an earlier call sized them; without them the call runs in
    // one pass, with the same result).
    PhaseArrays ph_arr;
    if (p.phases > 1 && work) {
        const cwlb_status s = prepare_column_phases(ctx, a, p.phases, may_build, &ph_arr);
        if (s != CWLB_OK) return s;
    }
    if (!ph_arr.bounds) p.phases = 1;
    if (p.phases > 1) {
        ctx->phase_seq = ctx->phase_seq >= 0x7fffffff ? 1 : ctx->phase_seq + 1;
        p.seq = ctx->phase_seq;
    }
    // Cache hints: 16-byte lanes, one vector per lane and slice, and the
    // feature matrix addressable by 32-bit byte offsets.
    if (!per_task && p.phases == 1 && ctx->sched_hot_bytes > 0 && p.vec == 4 && a.n_tasks > 0 && a.K > 0 &&
        (a.K / 4 + p.sl - 1) / p.sl <= 64 &&
        static_cast<unsigned long long>(a.h_rows) * a.K * 4ull <= 0xFFFFFFFFull) {
        const long long hot_rows = ctx->sched_hot_bytes / (4ll * a.K);
        const cwlb_status s = build_cache_hints(ctx, a, hot_rows, may_build, &p.hints);
        if (s != CWLB_OK) return s;
    }
    ctx->last_call_hinted = p.hints != nullptr;
    if (p.ordered && a.n_tasks > 0 && a.K > 0) {
        const cwlb_status s = build_run_order(ctx, a, p.M, p.runs, may_build, &p.order);
        if (s != CWLB_OK) return s;
    }
    if (record_events) CWLB_HIP_TRY(hipEventRecord(ctx->ev[0], st));
    const long long total = static_cast<long long>(a.n_rows) * a.K;
    if (zero_all) {
        const long long want = (total / 4 + kAuxBlock - 1) / kAuxBlock;
        const unsigned blocks =
            static_cast<unsigned>(std::max<long long>(1, std::min<long long>(want, 65536)));
        hipLaunchKernelGGL(fill_zero, dim3(blocks), dim3(kAuxBlock), 0, st, a.C,
                           std::max<long long>(total, 0), ctx->d_status);
    }
    ctx->last_launch.tasks_per_wave = p.M;
    ctx->last_launch.feature_slices = p.sl;
    ctx->last_launch.run_order = p.order ? 2 : 1;
    ctx->last_launch.xcd_blocks = p.chunk > 0 ? 2 : 1;
    ctx->last_launch.cache_hints = p.hints ? 1 : 0;
    ctx->last_launch.vector_width = p.vec;
    ctx->last_launch.waves_per_simd = p.o6 ? 6 : 0;
    ctx->last_launch.grid_blocks = a.n_tasks > 0 && a.K > 0 ? p.grid : 0;
    ctx->last_launch.max_waves_per_cu = 0;
    ctx->last_launch.column_phases = p.phases;
    {
        const int F = (a.K / p.vec + p.sl - 1) / p.sl;
        pick_tiling(F, p.sl, p.packed, !p.hints && p.phases == 1, &p.G, &p.R);
        // A packed pick that is no different launches the standard tilings.
        int G1 = 0, R1 = 0;
        pick_tiling(F, p.sl, false, false, &G1, &R1);
        if (p.G == G1 && p.R == R1) p.packed = false;
        ctx->last_call_packed = p.packed && work;
        ctx->last_launch.slot_lanes = p.G;
        ctx->last_launch.lane_vectors = p.R;
    }
    // A phased call sorts each row's nonzeros by band into the context's
    // copy, and always runs the clearing pass: it also checks the chain.
    if (p.phases > 1) {
        const cwlb_status s =
            launch_band_sort(st, a.row_ptr, a.col_idx, a.val, a.n_rows, a.nnz, a.h_rows,
                             p.phases, ph_arr.bounds, ph_arr.col, ph_arr.val, ctx->d_status + 1);
        if (s != CWLB_OK) return s;
    }
    if ((!zero_all || p.phases > 1) && work) {
        if (p.vec == 4) launch_zero<4>(st, a, p, ctx->d_status);
        else if (p.vec == 2) launch_zero<2>(st, a, p, ctx->d_status);
        else launch_zero<1>(st, a, p, ctx->d_status);
    } else if (!zero_all) {
        hipLaunchKernelGGL(fill_zero, dim3(1), dim3(kAuxBlock), 0, st, a.C, 0LL, ctx->d_status);
    }
    CWLB_HIP_TRY(hipGetLastError());
    if (record_events) CWLB_HIP_TRY(hipEventRecord(ctx->ev[1], st));
    if (work) {
        int waves = 0;
        p.cb = ph_arr.col;
        p.vb = ph_arr.val;
        for (int ph = 0; ph < p.phases; ++ph) {
            // Phase ph reads the bounds ph - 1 and ph of the P - 1 stored
            // per row (the row's own start and end at the outer phases).
            const long long n = a.n_rows;
            p.pb = ph > 0 ? ph_arr.bounds + (ph - 1) * n : nullptr;
            p.pe = ph < p.phases - 1 ? ph_arr.bounds + ph * n : nullptr;
            p.first = ph == 0;
            if (p.vec == 4) waves = dispatch_main<4>(st, a, p, ctx->d_status);
            else if (p.vec == 2) waves = dispatch_main<2>(st, a, p, ctx->d_status);
            else waves = dispatch_main<1>(st, a, p, ctx->d_status);
            CWLB_HIP_TRY(hipGetLastError());
        }
        ctx->last_launch.max_waves_per_cu = waves;
    }
    if (record_events) CWLB_HIP_TRY(hipEventRecord(ctx->ev[2], st));
    return CWLB_OK;
}

cwlb_status launch_fill_features(cwlb_ctx* ctx, float* H, int64_t rows, int32_t K, uint64_t seed)
{
    const long long total = static_cast<long long>(rows) * K;
    if (total <= 0) return CWLB_OK;
    const unsigned blocks =
        static_cast<unsigned>(std::min<long long>((total + kAuxBlock - 1) / kAuxBlock, 65536));
    hipLaunchKernelGGL(fill_features, dim3(blocks), dim3(kAuxBlock), 0, ctx->stream, H, total,
                       host_mix64(seed));
    CWLB_HIP_TRY(hipGetLastError());
    return CWLB_OK;
}

}  // namespace cwlb
