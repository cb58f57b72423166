// Weighted SwiGLU as standalone kernels (the unfused megatron surface).
//
//   h[m, f] = silu(g) * u * p[m],  g = y1[m, f], u = y1[m, F + f]
// and its backward
//   dy1[m, f]     = dh * p * u * sig(g) * (1 + g * (1 - sig(g)))
//   dy1[m, F + f] = dh * p * silu(g)
//   dp[m]         = sum_f dh * silu(g) * u
// (megatron weighted_bias_swiglu_impl / weighted_swiglu_back, restated in
// src/art/megatron/compile_workarounds.py:73-106; gate columns first, :85).
// The fused layer computes the same in the FC1 / FC2-dgrad epilogues; these
// serve the module-level path (grouped FC1 -> SwiGLU -> grouped FC2).
// bf16 in and out, fp32 arithmetic, one rounding per output.
#include "common.h"

namespace art {

// one thread per 8 columns of one row
__global__ __launch_bounds__(256) void weighted_swiglu_kernel(const U4 *__restrict__ y1,
                                                              const float *__restrict__ prob,
                                                              int64_t M, int F8,
                                                              U4 *__restrict__ h) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M * F8) return;
  const int64_t m = i / F8;
  const int c = (int)(i - m * F8);
  float g[8], u[8], o[8];
  unpack8(y1[m * 2 * F8 + c], g);
  unpack8(y1[m * 2 * F8 + F8 + c], u);
  const float p = prob ? prob[m] : 1.0f;
#pragma unroll
  for (int t = 0; t < 8; ++t) o[t] = silu_f(g[t]) * u[t] * p;
  h[m * F8 + c] = pack8(o);
}

// one wavefront per row (the dp reduction runs over the row's F columns)
__global__ __launch_bounds__(256) void weighted_swiglu_back_kernel(
    const U4 *__restrict__ dh, const U4 *__restrict__ y1, const float *__restrict__ prob,
    int64_t M, int F8, U4 *__restrict__ dy1, float *__restrict__ dprob) {
  const int lane = threadIdx.x & 63;
  const int64_t m = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (m >= M) return;
  const float p = prob ? prob[m] : 1.0f;
  float dp = 0.0f;
  for (int c = lane; c < F8; c += kWave) {
    float d[8], g[8], u[8], dg[8], du[8];
    unpack8(dh[m * F8 + c], d);
    unpack8(y1[m * 2 * F8 + c], g);
    unpack8(y1[m * 2 * F8 + F8 + c], u);
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const float sg = sigmoid_f(g[t]);
      const float si = g[t] * sg;
      dg[t] = d[t] * p * u[t] * sg * (1.0f + g[t] * (1.0f - sg));
      du[t] = d[t] * p * si;
      dp += d[t] * si * u[t];
    }
    dy1[m * 2 * F8 + c] = pack8(dg);
    dy1[m * 2 * F8 + F8 + c] = pack8(du);
  }
  dp = wave_sum(dp);
  if (lane == 0 && dprob) dprob[m] = dp;
}

}  // namespace art

using namespace art;

extern "C" int art_moe_weighted_swiglu(const void *y1, const float *prob, int64_t M, int32_t F,
                                       void *h, void *stream) {
  clear_error();
  ART_REQUIRE(M >= 0 && F > 0 && F % 8 == 0, "weighted_swiglu: need F a positive multiple of 8");
  if (M == 0) return ART_MOE_OK;
  ART_REQUIRE(y1 && h, "weighted_swiglu: null pointer");
  ART_REQUIRE(((uintptr_t)y1 & 15) == 0 && ((uintptr_t)h & 15) == 0,
              "weighted_swiglu: operands must be 16-byte aligned");
  const int64_t n = M * (F / 8);
  weighted_swiglu_kernel<<<dim3((unsigned)((n + 255) / 256)), 256, 0, as_stream(stream)>>>(
      (const U4 *)y1, prob, M, F / 8, (U4 *)h);
  return check_launch("weighted_swiglu");
}

extern "C" int art_moe_weighted_swiglu_back(const void *dh, const void *y1, const float *prob,
                                            int64_t M, int32_t F, void *dy1, float *dprob,
                                            void *stream) {
  clear_error();
  ART_REQUIRE(M >= 0 && F > 0 && F % 8 == 0,
              "weighted_swiglu_back: need F a positive multiple of 8");
  if (M == 0) return ART_MOE_OK;
  ART_REQUIRE(dh && y1 && dy1, "weighted_swiglu_back: null pointer");
  ART_REQUIRE(((uintptr_t)dh & 15) == 0 && ((uintptr_t)y1 & 15) == 0 && ((uintptr_t)dy1 & 15) == 0,
              "weighted_swiglu_back: operands must be 16-byte aligned");
  weighted_swiglu_back_kernel<<<dim3((unsigned)((M + 3) / 4)), 256, 0, as_stream(stream)>>>(
      (const U4 *)dh, (const U4 *)y1, prob, M, F / 8, (U4 *)dy1, dprob);
  return check_launch("weighted_swiglu_back");
}
