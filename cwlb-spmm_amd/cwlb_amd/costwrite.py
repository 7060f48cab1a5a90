"""costWrite: calibrates the operation costs on the GPU and saves the cost
file (reference weightCost.cpp:11-77).

    python -m cwlb_amd.costwrite [K repeat WI load_MB atomic_writers] [--out PATH]

Defaults 128 500 131072 512 8; the file has four lines (compute, load,
store, atomic) with six decimals.
"""
import argparse
import sys

from . import capi


def main(argv=None):
    ap = argparse.ArgumentParser(prog="costWrite")
    ap.add_argument("params", nargs="*", type=int)
    ap.add_argument("--out", default="../resources/spmm_costs.txt")
    ap.add_argument("--device", type=int, default=0)
    a = ap.parse_args(argv)
    if len(a.params) not in (0, 5):
        print("Usage:\n  costWrite\n  costWrite [K] [repeat] [WI] [load_MB] [atomic_writers]",
              file=sys.stderr)
        return 1
    K, repeat, WI, load_MB, writers = a.params or [128, 500, 131072, 512, 8]
    try:
        ctx = capi.Context(a.device)
        c = ctx.calibrate(K, repeat, WI, load_MB, writers)
        print(f"device: {ctx.info().name.decode()}")
        print(f"C_compute_ns: {c.C_compute_ns:.6f}")
        print(f"C_load_ns: {c.C_load_ns:.6f}")
        print(f"C_store_ns: {c.C_store_ns:.6f}")
        print(f"C_atomic_ns: {c.C_atomic_ns:.6f}")
        capi.save_costs(c.tuple4(), a.out)
        print(f"Saved cost parameters to: {a.out}")
    except capi.CwlbError as e:
        print(str(e), file=sys.stderr)
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
