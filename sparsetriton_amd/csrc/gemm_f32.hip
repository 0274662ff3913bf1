// Instantiates the gather-GEMM / weight-gradient launchers for float.
#include "gemm_kernels.h"

ST_GEMM_OPS(, float)
