// Instantiates the gather-GEMM / weight-gradient launchers for _Float16.
#include "gemm_kernels.h"

ST_GEMM_OPS(, _Float16)
