// Segmented "TN" products: LoRA weight gradients with fp32 accumulation.
//
//   out[e][p][q] (+)= alpha * sum_{m in segment e} Lm[lrow(m), p] * R[rrow(m), q]
//
// This is the varlen-K GEMM of the reference's grouped LoRA backward
// (src/art/megatron/kernels/cute_grouped_lora_quack.py:301-334, 411-431):
// grad_A[e] = x_e^T (s dy_e B_e^T) and grad_B[e] = s (x_e A_e)^T dy_e, where the
// reduction runs over the rows (tokens) of expert e's segment.
//
// One workgroup owns an output tile BP x BQ of one expert and walks the whole
// segment in steps of 64 rows, so each output element is produced by one
// fixed-order fp32 sum (deterministic; no atomics).  Rows are staged in LDS
// in their natural (row-major) layout; the MFMA operands need 8 consecutive
// rows per lane, which are gathered with 16-bit LDS reads.  The row stride is
// padded by 2 elements so that the four 16-lane groups of a wavefront, which
// read rows 8 apart, land on disjoint bank sets.
// MFMA: v_mfma_f32_16x16x32_bf16 (P and Q tiles in multiples of 16, so LoRA
// ranks of 16 waste nothing).
#include "common.h"

namespace art {

struct WArgs {
  const bf16 *l;
  int64_t ldl;
  const int32_t *l_rows;
  const bf16 *r;
  int64_t ldr;
  const int32_t *r_rows;
  const int32_t *seg;
  int E, P, Q;
  float alpha;
  void *out;
  int64_t o_es, o_sp, o_sq;
  void *out2;  // columns q >= q_split land here (column q - q_split)
  int q_split;
  int64_t o2_es, o2_sp, o2_sq;
  int mode;  // ART_MOE_WGRAD_STORE / _ACCUMULATE / _STORE_BF16
};

template <int BP, int BQ>
__global__ __launch_bounds__(256) void wgrad_tn_kernel(const WArgs a) {
  constexpr int BKM = 64;
  constexpr int LDL = BP + 2, LDR = BQ + 2;
  constexpr int TMW = BP / 64, TNW = BQ / 16;  // 16x16 blocks per wave (4 waves split P)
  static_assert(TMW >= 1 && TNW >= 1, "tile");
  __shared__ __attribute__((aligned(16))) bf16 sL[BKM * LDL];
  __shared__ __attribute__((aligned(16))) bf16 sR[BKM * LDR];

  const int e = blockIdx.x;
  const int p0 = blockIdx.y * BP, q0 = blockIdx.z * BQ;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l16 = lane & 15, g4 = lane >> 4;
  const int m_begin = a.seg[e], m_end = a.seg[e + 1];

  f32x4 acc[TMW][TNW];
#pragma unroll
  for (int i = 0; i < TMW; ++i)
#pragma unroll
    for (int j = 0; j < TNW; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[i][j][v] = 0.0f;

  for (int mb = m_begin; mb < m_end; mb += BKM) {
    for (int c = tid; c < BKM * BP / 8; c += 256) {
      const int row = c / (BP / 8), pc = c - row * (BP / 8);
      const int m = mb + row, pp = p0 + pc * 8;
      U4 v = U4{0u, 0u, 0u, 0u};
      if (m < m_end && pp < a.P) {
        const int64_t src = a.l_rows ? (int64_t)a.l_rows[m] : (int64_t)m;
        v = *(const U4 *)(a.l + src * a.ldl + pp);
      }
      uint32_t *d = (uint32_t *)&sL[row * LDL + pc * 8];
      d[0] = v.x; d[1] = v.y; d[2] = v.z; d[3] = v.w;
    }
    for (int c = tid; c < BKM * BQ / 8; c += 256) {
      const int row = c / (BQ / 8), qc = c - row * (BQ / 8);
      const int m = mb + row, qq = q0 + qc * 8;
      U4 v = U4{0u, 0u, 0u, 0u};
      if (m < m_end && qq < a.Q) {
        const int64_t src = a.r_rows ? (int64_t)a.r_rows[m] : (int64_t)m;
        v = *(const U4 *)(a.r + src * a.ldr + qq);
      }
      uint32_t *d = (uint32_t *)&sR[row * LDR + qc * 8];
      d[0] = v.x; d[1] = v.y; d[2] = v.z; d[3] = v.w;
    }
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < BKM / 32; ++ks) {
      const int rbase = ks * 32 + g4 * 8;
      bf16x8 af[TMW], bfv[TNW];
#pragma unroll
      for (int i = 0; i < TMW; ++i) {
        const int pc = wave * (BP / 4) + i * 16 + l16;
#pragma unroll
        for (int t = 0; t < 8; ++t) af[i][t] = sL[(rbase + t) * LDL + pc];
      }
#pragma unroll
      for (int j = 0; j < TNW; ++j) {
        const int qc = j * 16 + l16;
#pragma unroll
        for (int t = 0; t < 8; ++t) bfv[j][t] = sR[(rbase + t) * LDR + qc];
      }
#pragma unroll
      for (int i = 0; i < TMW; ++i)
#pragma unroll
        for (int j = 0; j < TNW; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfv[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }

  // Accumulator element v of a 16x16 block: row 4*(lane/16) + v, column lane%16.
#pragma unroll
  for (int i = 0; i < TMW; ++i)
#pragma unroll
    for (int j = 0; j < TNW; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int pp = p0 + wave * (BP / 4) + i * 16 + g4 * 4 + v;
        const int qq = q0 + j * 16 + l16;
        if (pp < a.P && qq < a.Q) {
          const bool second = a.out2 != nullptr && qq >= a.q_split;
          void *base = second ? a.out2 : a.out;
          const int64_t off = second
              ? (int64_t)e * a.o2_es + (int64_t)pp * a.o2_sp + (int64_t)(qq - a.q_split) * a.o2_sq
              : (int64_t)e * a.o_es + (int64_t)pp * a.o_sp + (int64_t)qq * a.o_sq;
          const float val = a.alpha * acc[i][j][v];
          if (a.mode == ART_MOE_WGRAD_STORE_BF16) {
            ((bf16 *)base)[off] = (bf16)val;
          } else {
            float *o = (float *)base + off;
            *o = a.mode == ART_MOE_WGRAD_ACCUMULATE ? *o + val : val;
          }
        }
      }
}

template <int BP, int BQ>
static int launch_wgrad(const WArgs &a, hipStream_t s) {
  const dim3 grid((unsigned)a.E, (unsigned)((a.P + BP - 1) / BP), (unsigned)((a.Q + BQ - 1) / BQ));
  wgrad_tn_kernel<BP, BQ><<<grid, 256, 0, s>>>(a);
  return check_launch("grouped_wgrad");
}

}  // namespace art

using namespace art;

extern "C" int art_moe_grouped_wgrad(const void *lm, int64_t ldl, const int32_t *l_rows,
                                     const void *r, int64_t ldr, const int32_t *r_rows,
                                     const int32_t *seg, int32_t E, int32_t P, int32_t Q,
                                     float alpha, void *out, int64_t o_es, int64_t o_ps,
                                     int64_t o_qs, void *out2, int32_t q_split, int64_t o2_es,
                                     int64_t o2_ps, int64_t o2_qs, int32_t mode, void *stream) {
  clear_error();
  ART_REQUIRE(E >= 1 && E <= 65535, "grouped_wgrad: need 1 <= E <= 65535 (E=%d)", E);
  ART_REQUIRE(P > 0 && Q > 0 && P % 8 == 0 && Q % 8 == 0,
              "grouped_wgrad: P and Q must be positive multiples of 8 (P=%d Q=%d)", P, Q);
  ART_REQUIRE(ldl % 8 == 0 && ldr % 8 == 0, "grouped_wgrad: row strides must be multiples of 8");
  ART_REQUIRE(lm && r && seg && out, "grouped_wgrad: null pointer");
  ART_REQUIRE(mode == ART_MOE_WGRAD_STORE || mode == ART_MOE_WGRAD_ACCUMULATE ||
                  mode == ART_MOE_WGRAD_STORE_BF16,
              "grouped_wgrad: unknown mode %d", mode);
  ART_REQUIRE(((uintptr_t)lm & 15) == 0 && ((uintptr_t)r & 15) == 0,
              "grouped_wgrad: operands must be 16-byte aligned");
  WArgs a{};
  a.l = (const bf16 *)lm; a.ldl = ldl; a.l_rows = l_rows;
  a.r = (const bf16 *)r; a.ldr = ldr; a.r_rows = r_rows;
  a.seg = seg; a.E = E; a.P = P; a.Q = Q; a.alpha = alpha;
  ART_REQUIRE(!out2 || (q_split > 0 && q_split < Q),
              "grouped_wgrad: split output needs 0 < q_split < Q (q_split=%d Q=%d)", q_split, Q);
  a.out = out; a.o_es = o_es; a.o_sp = o_ps; a.o_sq = o_qs; a.mode = mode;
  a.out2 = out2; a.q_split = out2 ? q_split : Q;
  a.o2_es = o2_es; a.o2_sp = o2_ps; a.o2_sq = o2_qs;
  hipStream_t s = as_stream(stream);
  if (Q <= 16) return launch_wgrad<128, 16>(a, s);
  if (Q <= 32) return launch_wgrad<128, 32>(a, s);
  if (Q <= 64) return launch_wgrad<128, 64>(a, s);
  return launch_wgrad<128, 128>(a, s);
}
