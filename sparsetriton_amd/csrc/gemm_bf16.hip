// Instantiates the gather-GEMM / weight-gradient launchers for __bf16.
#include "gemm_kernels.h"

ST_GEMM_OPS(, __bf16)
