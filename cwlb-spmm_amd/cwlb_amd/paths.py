"""Locations of the built libraries and executables (in-tree builds)."""
import os

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REPO_DIR = os.path.dirname(PKG_DIR)
LIB_DIR = os.path.join(PKG_DIR, "lib")
BIN_DIR = os.path.join(PKG_DIR, "bin")
INCLUDE_DIR = os.path.join(REPO_DIR, "include")
# The cost coefficients calibrated on gfx950 (costWrite format).
COST_FILE = os.path.join(PKG_DIR, "resources", "spmm_costs_gfx950.txt")
