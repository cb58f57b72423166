// Shared device/host helpers of libart_moe (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include <string>

#include "art_moe.h"

namespace art {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;

// ------------------------------------------------------------ host errors
void set_error(const char *fmt, ...);
void clear_error();

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

// Returns ART_MOE_OK, or ART_MOE_ERR_HIP with the message recorded.
int check_launch(const char *what);

int device_cu_count();

#define ART_REQUIRE(cond, ...)                  \
  do {                                          \
    if (!(cond)) {                              \
      ::art::set_error(__VA_ARGS__);            \
      return ART_MOE_ERR_INVALID_ARG;           \
    }                                           \
  } while (0)

// ------------------------------------------------------------ device helpers
__device__ __forceinline__ float bf16_to_f(bf16 v) { return (float)v; }
__device__ __forceinline__ bf16 f_to_bf16(float v) { return (bf16)v; }

// sigmoid through v_rcp_f32 (within 1 ulp) instead of a correctly rounded divide: the
// divide's scale / refine / fixup sequence was half of the SwiGLU epilogues' vector
// instructions, and the difference stays far below the bf16 rounding of every output.
// Limits match the divide: g -> +inf gives 1 (silu g), g -> -inf gives 0 (silu -0), NaN
// stays NaN.
__device__ __forceinline__ float sigmoid_f(float g) {
  return __builtin_amdgcn_rcpf(1.0f + __expf(-g));
}
__device__ __forceinline__ float silu_f(float g) { return g * sigmoid_f(g); }

__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// 16-byte vector of 8 bf16 held as 4 dwords.
struct alignas(16) U4 {
  uint32_t x, y, z, w;
};

__device__ __forceinline__ void unpack8(const U4 &u, float *f) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(w[i] << 16);
    f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

__device__ __forceinline__ uint32_t pack2(float a, float b) {
  bf16 x = (bf16)a, y = (bf16)b;
  uint16_t ux = __builtin_bit_cast(uint16_t, x), uy = __builtin_bit_cast(uint16_t, y);
  return (uint32_t)ux | ((uint32_t)uy << 16);
}

__device__ __forceinline__ U4 pack8(const float *f) {
  U4 u;
  u.x = pack2(f[0], f[1]);
  u.y = pack2(f[2], f[3]);
  u.z = pack2(f[4], f[5]);
  u.w = pack2(f[6], f[7]);
  return u;
}

}  // namespace art
