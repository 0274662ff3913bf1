// Measurement helper: the sustained dense bf16 MFMA rate of the chip it runs
// on, against which the gather-GEMM and weight-gradient rates are read beside
// the spec-sheet peak.  Every wave runs kPeakChains independent chains of
// v_mfma_f32_16x16x32_bf16 on register operands (no memory traffic inside the
// loop), so the MFMA pipes never wait on a result; each thread's sum is stored
// at the end.
#include "common.h"
#include "mfma.h"

namespace st {

constexpr int kPeakChains = 8;

// One chain's MFMA with its accumulator tied to one VGPR quad: written through the compiler
// builtin, the loop-carried accumulators were shuffled between AGPR tuples every iteration
// (copies and wait states between the MFMAs), which measured half the rate.
#define ST_PEAK_MFMA(c) asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b))

__global__ __launch_bounds__(256) void mfma_peak_kernel(int iters, float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  v8bf a, b;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    a[e] = (__bf16)(0.001f * (float)(lane + e));
    b[e] = (__bf16)(0.002f * (float)(lane - e));
  }
  v4f c0 = {0.f, 0.f, 0.f, 0.f}, c1 = c0, c2 = c0, c3 = c0, c4 = c0, c5 = c0, c6 = c0, c7 = c0;
  static_assert(kPeakChains == 8, "eight chains below");
  for (int i = 0; i < iters; ++i) {
    ST_PEAK_MFMA(c0);
    ST_PEAK_MFMA(c1);
    ST_PEAK_MFMA(c2);
    ST_PEAK_MFMA(c3);
    ST_PEAK_MFMA(c4);
    ST_PEAK_MFMA(c5);
    ST_PEAK_MFMA(c6);
    ST_PEAK_MFMA(c7);
  }
  const v4f s = c0 + c1 + c2 + c3 + c4 + c5 + c6 + c7;
  out[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = s[0] + s[1] + s[2] + s[3];
}
#undef ST_PEAK_MFMA

}  // namespace st

extern "C" int st_mfma_peak(int iters, int blocks, float* out, int64_t* flops, st_stream_t stream) {
  if (iters < 1 || blocks < 1 || !out || !flops) return ST_ERR_ARG;
  // 4 waves a workgroup, kPeakChains MFMAs of 16 x 16 x 32 (2 * 8192 flops) per wave and iteration
  *flops = (int64_t)blocks * 4 * iters * st::kPeakChains * 2 * 16 * 16 * 32;
  st::mfma_peak_kernel<<<(unsigned)blocks, 256, 0, stream>>>(iters, out);
  ST_CHECK_LAUNCH();
  return ST_OK;
}
