// costWrite: operation-cost calibration (reference weightCost.cpp).
#include "cwlb_driver.h"

int main(int argc, char* argv[]) { return cost_write_main(argc, argv); }
