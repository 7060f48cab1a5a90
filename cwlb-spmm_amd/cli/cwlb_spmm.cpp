// cwlb-spmm: the CWLB-SpMM benchmark driver (reference main.cpp).
#include "cwlb_driver.h"

int main(int argc, char* argv[]) { return cwlb_spmm_main(argc, argv); }
