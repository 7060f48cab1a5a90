// The GPU partition's per-node simulation (csrc/partition.hip), kept in a
// header so that the same code also builds for the host, where the tests
// check the decomposition of the host partition into fresh-node transitions.
// Compile without floating-point contraction: the double operations must be
// the host partition's, one rounding each.
#pragma once

#include <cstdint>

#include "cwlb.h"

#if defined(__HIPCC__)
#define CWLB_HD __host__ __device__
#else
#define CWLB_HD
#endif

#if defined(__clang__)
#pragma clang fp contract(off)
#endif

namespace cwlb {
namespace part {

struct PartParams {
    const int* rp;
    const int* long_row;  // long row of compact index c
    const int* long_idx;  // compact index of long row r, or -1
    int n;
    int S;
    double wcl, cs, ca, cap;
    long long max_scan;
};

CWLB_HD inline int degree(const PartParams& p, int r) { return p.rp[r + 1] - p.rp[r]; }
CWLB_HD inline double full_w(const PartParams& p, int r)
{
    return p.wcl * static_cast<double>(degree(p, r)) + p.cs;
}
CWLB_HD inline double chunk_w(const PartParams& p, int k)
{
    return p.wcl * static_cast<double>(k) + p.ca;
}

struct Emitter {
    cwlb_task* out;  // null: count only
    long long count;
    CWLB_HD void emit(int s, int e, int fo, int last)
    {
        if (s < e) {
            if (out) out[count] = cwlb_task{s, e, fo, last};
            ++count;
        }
    }
};

// Simulates the host state machine from fresh node x to the next fresh
// node (returned), emitting the tasks closed on the way.  *overrun is set
// when a short-row scan exceeds its bound (the caller then fails the call).
CWLB_HD inline int simulate(const PartParams& p, int x, Emitter& em, int* overrun)
{
    const int n = p.n;
    const int S = p.S;
    int L, g, fo, off, remaining;
    double acc = 0.0;
    if (x <= n) {
        // ---- A(x): pack whole rows.
        if (x == n) return n;
        int row = x;
        g = x;
        fo = 0;
        long long steps = 0;
        for (;;) {
            if (row == n) {
                if (acc > 0.0 || g < n) em.emit(g, n, fo, 0);
                return n;
            }
            if (++steps > p.max_scan) {
                *overrun = 1;
                return n;
            }
            const double wr = full_w(p, row);
            if (!(wr <= p.cap)) break;  // long row
            if (acc == 0.0 || acc + wr <= p.cap) {
                acc += wr;
                ++row;
                continue;
            }
            em.emit(g, row, fo, 0);
            return row;
        }
        L = row;
        const int deg = degree(p, L);
        off = 0;
        remaining = deg;
        if (remaining <= 0) return L + 1;  // the host drops the open task here
        // Ride the deg % S prefix at the end of the open task.
        if (!(acc <= 0.0)) {
            const int r = deg % S;
            if (r == 0 || r >= deg) {
                em.emit(g, L, fo, 0);
                g = L;
                fo = 0;
                acc = 0.0;
            } else if (chunk_w(p, r) <= p.cap - acc) {
                em.emit(g, L + 1, fo, r);
                g = L;
                fo = r;
                acc = 0.0;
                remaining -= r;
                off += r;
            } else {
                em.emit(g, L, fo, 0);
                g = L;
                fo = 0;
                acc = 0.0;
            }
        }
    } else {
        // ---- B(L): the prefix of L already belongs to the previous task.
        L = p.long_row[x - n - 1];
        const int deg = degree(p, L);
        g = L;
        fo = deg % S;
        off = fo;
        remaining = deg - off;
        if (remaining <= 0) return L + 1;
    }
    // ---- Segments of at most S nonzeros: every segment but the last closes
    // a task; the last one's load decides the next-prefix absorption.
    const int nseg = (remaining - 1) / S + 1;
    const int last = remaining - (nseg - 1) * S;
    if (nseg > 1) {
        if (em.out) {
            for (int i = 0; i < nseg - 1; ++i) {
                off += S;
                em.emit(g, L + 1, fo, off);
                g = L;
                fo = off;
            }
        } else {
            em.count += nseg - 1;
            off += (nseg - 1) * S;
            g = L;
            fo = off;
        }
        acc = 0.0;
    }
    acc += chunk_w(p, last);
    // Next long row's prefix at the end of this row's last segment.
    if (!(acc >= p.cap) && L + 1 < n) {
        const int nr = L + 1;
        if (!(full_w(p, nr) <= p.cap)) {
            const int nd = degree(p, nr);
            const int r2 = nd % S;
            if (r2 != 0 && r2 < nd && !(chunk_w(p, r2) > p.cap - acc)) {
                em.emit(g, nr + 1, fo, r2);
                return n + 1 + p.long_idx[nr];
            }
        }
    }
    em.emit(g, L + 1, fo, 0);
    return L + 1;
}

}  // namespace part
}  // namespace cwlb
