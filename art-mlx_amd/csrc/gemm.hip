// Grouped bf16 MFMA GEMMs over ragged expert segments (gfx950).
//
// One kernel template serves every dense product of the layer:
//   C[m, n] = alpha * ( sum_c A[row(m), c] B[e][n, c] + sum_j Tl[m, j] L[e][n, j] )
// for the rows m of expert e's segment.  Both operands are "K-contiguous"
// (NT form), so every MFMA operand is one 16-byte LDS read per lane.  The
// LoRA product (x A) B is folded in as extra K-steps (the "K-extension"):
// after the K loop over the base weight the same accumulators keep going over
// the rank dimension with Tl = x A (or the data-gradient intermediate) and
// L = the LoRA factor laid out [E][N][kt].  The base + adapter add of the
// reference (src/art/megatron/lora.py:1529, 1571) therefore costs no pass.
//
// Scheduling: persistent workgroups walk a tile list (expert-major row
// tiles x column tiles) read from the device segment table, so no host sync
// on tokens_per_expert is needed and zero-token experts produce no tiles.  The
// workgroup -> tile order is remapped so that each of the 8 XCDs works on a
// contiguous run of tiles (shared A rows / expert weights stay in its L2).
//
// Tiles: BM x BN per workgroup, BK = 64, WM x WN wavefronts, each wave owning
// (BM/WM) x (BN/WN) in 32x32 blocks of v_mfma_f32_32x32x16_bf16.  LDS holds
// two stages of A and B; 16-byte chunks are XOR-swizzled by row so that both
// the global->LDS stores and the MFMA operand reads are bank-conflict free.
// Global loads of stage k+1 are issued before the MFMAs of stage k.
#include "common.h"

namespace art {

enum { EPI_STORE = 0, EPI_SWIGLU_FWD = 1, EPI_SWIGLU_BWD = 2 };

struct NTArgs {
  const bf16 *a;
  int64_t lda;
  const int32_t *a_rows;
  const bf16 *b;
  int64_t ldb;
  int64_t b_es;
  const bf16 *t;
  int64_t ldt;
  const bf16 *l;
  int64_t ldl;
  int64_t l_es;
  int kt;
  const int32_t *seg_off;   // [E+1]
  const int32_t *tile_off;  // [E+1] for this BM
  int E;
  int N;  // logical columns (2F for the SwiGLU forward)
  int K;
  float alpha;
  void *c;
  int64_t ldc;
  int c_fp32;
  // SwiGLU
  int F;
  const float *prob;
  bf16 *y1;      // fwd out [M][2F]
  bf16 *h;       // fwd out [M][F]
  const bf16 *y1_in;  // bwd in [M][2F]
  bf16 *dy1;     // bwd out [M][2F]
  float *dp_part;  // bwd out [n_tiles][M]
  int64_t M;
};

__device__ __forceinline__ int swz(int row, int chunk) { return (chunk ^ (row & 7)) * 8; }

template <int BM, int BN, int WM, int WN, int EPI>
__global__ __launch_bounds__(WM *WN * 64) void gemm_nt_kernel(const NTArgs p) {
  constexpr int BK = 64;
  constexpr int NT = WM * WN * 64;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  constexpr int CA = BM * 8 / NT, CB = BN * 8 / NT;  // 16-byte chunks per thread
  static_assert(TM >= 1 && TN >= 1 && CA >= 1 && CB >= 1, "tile config");
  static_assert(EPI != EPI_SWIGLU_FWD || (TN % 2 == 0), "SwiGLU forward pairs gate/up blocks");
  static_assert(NT % 8 == 0, "threads");

  __shared__ __attribute__((aligned(16))) bf16 sA[2][BM * BK];
  __shared__ __attribute__((aligned(16))) bf16 sB[2][BN * BK];
  __shared__ float sRed[EPI == EPI_SWIGLU_BWD ? WN * BM : 1];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int lrow = lane & 31, lk = lane >> 5;
  const int n_tiles = (p.N + BN - 1) / BN;
  const int total = p.tile_off[p.E] * n_tiles;
  const int nb = gridDim.x;
  const int lb = (nb % 8 == 0) ? ((blockIdx.x & 7) * (nb >> 3) + (blockIdx.x >> 3)) : blockIdx.x;
  const int nk_main = (p.K + BK - 1) / BK;
  const int nk = nk_main + (p.kt + BK - 1) / BK;
  const int chunk = tid & 7;

  for (int tile = lb; tile < total; tile += nb) {
    const int mt = tile / n_tiles, nt = tile - mt * n_tiles;
    int lo = 0, hi = p.E;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (p.tile_off[mid] <= mt) lo = mid; else hi = mid;
    }
    const int e = lo;
    const int m0 = p.seg_off[e] + (mt - p.tile_off[e]) * BM;
    const int m_end = p.seg_off[e + 1];

    // Row pointers of this thread's A / Tl chunks and B / L chunks.
    const bf16 *aptr[CA];
    const bf16 *tptr[CA];
#pragma unroll
    for (int i = 0; i < CA; ++i) {
      const int r = (tid >> 3) + i * (NT / 8);
      const int m = m0 + r;
      if (m < m_end) {
        const int64_t src = p.a_rows ? (int64_t)p.a_rows[m] : (int64_t)m;
        aptr[i] = p.a + src * p.lda;
        tptr[i] = p.t ? p.t + (int64_t)m * p.ldt : nullptr;
      } else {
        aptr[i] = nullptr;
        tptr[i] = nullptr;
      }
    }
    const bf16 *bptr[CB];
    const bf16 *lptr[CB];
#pragma unroll
    for (int i = 0; i < CB; ++i) {
      const int r = (tid >> 3) + i * (NT / 8);
      int n = nt * BN + r;
      bool ok = n < p.N;
      if (EPI == EPI_SWIGLU_FWD) {
        // logical 32-column blocks alternate gate / up of the same columns
        const int blk = r >> 5, within = r & 31;
        n = ((blk & 1) ? p.F : 0) + nt * (BN / 2) + (blk >> 1) * 32 + within;
        ok = (nt * (BN / 2) + (blk >> 1) * 32 + within) < p.F;
      }
      bptr[i] = ok ? p.b + (int64_t)e * p.b_es + (int64_t)n * p.ldb : nullptr;
      lptr[i] = (ok && p.l) ? p.l + (int64_t)e * p.l_es + (int64_t)n * p.ldl : nullptr;
    }

    U4 ra[CA], rb[CB];
    auto gload = [&](int ks) {
      const bool main = ks < nk_main;
      const int k0 = (main ? ks : ks - nk_main) * BK + chunk * 8;
      const int klim = main ? p.K : p.kt;
#pragma unroll
      for (int i = 0; i < CA; ++i) {
        const bf16 *s = main ? aptr[i] : tptr[i];
        if (s && k0 < klim) ra[i] = *(const U4 *)(s + k0);
        else ra[i] = U4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int i = 0; i < CB; ++i) {
        const bf16 *s = main ? bptr[i] : lptr[i];
        if (s && k0 < klim) rb[i] = *(const U4 *)(s + k0);
        else rb[i] = U4{0u, 0u, 0u, 0u};
      }
    };
    auto lstore = [&](int st) {
#pragma unroll
      for (int i = 0; i < CA; ++i) {
        const int r = (tid >> 3) + i * (NT / 8);
        *(U4 *)&sA[st][r * BK + swz(r, chunk)] = ra[i];
      }
#pragma unroll
      for (int i = 0; i < CB; ++i) {
        const int r = (tid >> 3) + i * (NT / 8);
        *(U4 *)&sB[st][r * BK + swz(r, chunk)] = rb[i];
      }
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    __syncthreads();  // previous tile's readers of stage 0 are done
    gload(0);
    lstore(0);
    __syncthreads();
    for (int ks = 0; ks < nk; ++ks) {
      const int st = ks & 1;
      if (ks + 1 < nk) gload(ks + 1);
#pragma unroll
      for (int kk = 0; kk < BK / 16; ++kk) {
        bf16x8 af[TM], bfv[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          const int r = wm * WTM + i * 32 + lrow;
          af[i] = *(const bf16x8 *)&sA[st][r * BK + swz(r, kk * 2 + lk)];
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int r = wn * WTN + j * 32 + lrow;
          bfv[j] = *(const bf16x8 *)&sB[st][r * BK + swz(r, kk * 2 + lk)];
        }
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfv[j], acc[i][j], 0, 0, 0);
      }
      if (ks + 1 < nk) lstore(st ^ 1);
      __syncthreads();
    }

    // ------------------------------------------------------------ epilogue
    // Accumulator element v of block (i, j) sits at row
    // 8*(v/4) + 4*(lane/32) + v%4 and column lane%32 of the 32x32 block.
    if (EPI == EPI_STORE) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int n = nt * BN + wn * WTN + j * 32 + lrow;
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int m = m0 + wm * WTM + i * 32 + 8 * (v >> 2) + 4 * lk + (v & 3);
            if (m < m_end && n < p.N) {
              const float val = p.alpha * acc[i][j][v];
              if (p.c_fp32) ((float *)p.c)[(int64_t)m * p.ldc + n] = val;
              else ((bf16 *)p.c)[(int64_t)m * p.ldc + n] = (bf16)val;
            }
          }
        }
    } else if (EPI == EPI_SWIGLU_FWD) {
      const int F = p.F;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int jp = 0; jp < TN / 2; ++jp) {
          const int f = nt * (BN / 2) + ((wn * TN) / 2 + jp) * 32 + lrow;
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int m = m0 + wm * WTM + i * 32 + 8 * (v >> 2) + 4 * lk + (v & 3);
            if (m < m_end && f < F) {
              const bf16 gb = (bf16)(p.alpha * acc[i][2 * jp][v]);
              const bf16 ub = (bf16)(p.alpha * acc[i][2 * jp + 1][v]);
              const float g = (float)gb, u = (float)ub;
              bf16 *yr = p.y1 + (int64_t)m * (2 * F);
              yr[f] = gb;
              yr[F + f] = ub;
              p.h[(int64_t)m * F + f] = (bf16)(silu_f(g) * u * p.prob[m]);
            }
          }
        }
    } else {  // EPI_SWIGLU_BWD
      const int F = p.F;
      float rs[TM][16];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) rs[i][v] = 0.0f;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int f = nt * BN + wn * WTN + j * 32 + lrow;
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int m = m0 + wm * WTM + i * 32 + 8 * (v >> 2) + 4 * lk + (v & 3);
            if (m < m_end && f < F) {
              const float dh = p.alpha * acc[i][j][v];
              const bf16 *yr = p.y1_in + (int64_t)m * (2 * F);
              const float g = (float)yr[f], u = (float)yr[F + f];
              const float pr = p.prob[m];
              const float sg = sigmoid_f(g);
              const float sl = g * sg;
              const float dhp = dh * pr;
              bf16 *dr = p.dy1 + (int64_t)m * (2 * F);
              dr[f] = (bf16)(dhp * u * sg * (1.0f + g * (1.0f - sg)));
              dr[F + f] = (bf16)(dhp * sl);
              rs[i][v] += dh * sl * u;
            }
          }
        }
      // Sum over the 32 columns each half-wave holds, then over the WN waves.
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          float s = rs[i][v];
#pragma unroll
          for (int o = 1; o < 32; o <<= 1) s += __shfl_xor(s, o, kWave);
          rs[i][v] = s;
        }
      if (lrow == 0) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int v = 0; v < 16; ++v)
            sRed[wn * BM + wm * WTM + i * 32 + 8 * (v >> 2) + 4 * lk + (v & 3)] = rs[i][v];
      }
      __syncthreads();
      for (int r = tid; r < BM; r += NT) {
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < WN; ++w) s += sRed[w * BM + r];
        const int m = m0 + r;
        if (m < m_end) p.dp_part[(int64_t)nt * p.M + m] = s;
      }
    }
  }
}

template <int BM, int BN, int WM, int WN, int EPI>
static int launch_nt(const NTArgs &a, const int32_t *seg, int64_t M, hipStream_t s,
                     const char *what) {
  constexpr int bmi = BM == 32 ? 0 : BM == 64 ? 1 : BM == 128 ? 2 : 3;
  static_assert(BM == 32 || BM == 64 || BM == 128 || BM == 256, "BM must be 32<<b");
  NTArgs p = a;
  p.seg_off = seg;
  p.tile_off = seg + (1 + bmi) * (a.E + 1);
  const int n_tiles = (a.N + BN - 1) / BN;
  const int64_t max_tiles = ((M + BM - 1) / BM + a.E) * (int64_t)n_tiles;
  int64_t grid = (int64_t)device_cu_count() * 2;
  if (grid > max_tiles) grid = max_tiles;
  if (grid >= 8) grid &= ~(int64_t)7;
  if (grid < 1) grid = 1;
  gemm_nt_kernel<BM, BN, WM, WN, EPI><<<dim3((unsigned)grid), WM * WN * 64, 0, s>>>(p);
  return check_launch(what);
}

}  // namespace art

using namespace art;

static bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

// Shared argument checks: every 16-byte operand chunk must be aligned, so
// base pointers are 16-byte aligned and leading dimensions multiples of 8.
static int check_common(const void *a, int64_t lda, const void *b, int64_t ldb,
                        const int32_t *seg, int32_t E, int64_t M, int32_t K, int32_t kt,
                        const void *tl, int64_t ldt, const void *l, int64_t ldl,
                        const char *who) {
  ART_REQUIRE(E >= 1 && E <= 1024, "%s: need 1 <= E <= 1024 (E=%d)", who, E);
  ART_REQUIRE(M >= 0 && M < INT32_MAX, "%s: M out of range", who);
  ART_REQUIRE(K > 0 && K % 8 == 0, "%s: K must be a positive multiple of 8 (K=%d)", who, K);
  ART_REQUIRE(kt >= 0 && kt % 16 == 0, "%s: LoRA kt must be a multiple of 16 (kt=%d)", who, kt);
  ART_REQUIRE(a && b && seg, "%s: null pointer", who);
  ART_REQUIRE(lda >= K && lda % 8 == 0 && ldb >= K && ldb % 8 == 0,
              "%s: leading dimensions must be >= K and multiples of 8 (lda=%lld ldb=%lld)", who,
              (long long)lda, (long long)ldb);
  ART_REQUIRE(aligned16(a) && aligned16(b), "%s: A and B must be 16-byte aligned", who);
  if (kt) {
    ART_REQUIRE(tl && l, "%s: kt > 0 needs tl and l", who);
    ART_REQUIRE(ldt >= kt && ldt % 8 == 0 && ldl >= kt && ldl % 8 == 0,
                "%s: LoRA leading dimensions must be >= kt and multiples of 8", who);
    ART_REQUIRE(aligned16(tl) && aligned16(l), "%s: LoRA operands must be 16-byte aligned", who);
  }
  return ART_MOE_OK;
}

extern "C" int art_moe_grouped_gemm(const void *a, int64_t lda, const int32_t *a_rows,
                                    const void *b, int64_t ldb, int64_t b_estride,
                                    const void *tl, int64_t ldt, const void *l, int64_t ldl,
                                    int64_t l_estride, int32_t kt, const int32_t *seg, int32_t E,
                                    int64_t M, int32_t N, int32_t K, float alpha, void *c,
                                    int64_t ldc, int32_t c_fp32, void *stream) {
  clear_error();
  int rc = check_common(a, lda, b, ldb, seg, E, M, K, kt, tl, ldt, l, ldl, "grouped_gemm");
  if (rc) return rc;
  ART_REQUIRE(N > 0 && c, "grouped_gemm: need N > 0 and an output");
  if (M == 0) return ART_MOE_OK;
  NTArgs p{};
  p.a = (const bf16 *)a; p.lda = lda; p.a_rows = a_rows;
  p.b = (const bf16 *)b; p.ldb = ldb; p.b_es = b_estride;
  p.t = kt ? (const bf16 *)tl : nullptr; p.ldt = ldt;
  p.l = kt ? (const bf16 *)l : nullptr; p.ldl = ldl; p.l_es = l_estride; p.kt = kt;
  p.E = E; p.N = N; p.K = K; p.alpha = alpha; p.c = c; p.ldc = ldc; p.c_fp32 = c_fp32; p.M = M;
  hipStream_t s = as_stream(stream);
  if (N <= 32) return launch_nt<128, 32, 4, 1, EPI_STORE>(p, seg, M, s, "grouped_gemm/n32");
  if (N <= 64) return launch_nt<128, 64, 4, 1, EPI_STORE>(p, seg, M, s, "grouped_gemm/n64");
  return launch_nt<128, 128, 2, 2, EPI_STORE>(p, seg, M, s, "grouped_gemm/n128");
}

extern "C" int art_moe_fc1_swiglu(const void *a, int64_t lda, const int32_t *a_rows,
                                  const void *w1, const void *tl, int64_t ldt, const void *l1,
                                  int32_t kt, const int32_t *seg, int32_t E, int64_t M, int32_t F,
                                  int32_t K, const float *row_prob, void *y1, void *h,
                                  void *stream) {
  clear_error();
  int rc = check_common(a, lda, w1, K, seg, E, M, K, kt, tl, ldt, l1, kt, "fc1_swiglu");
  if (rc) return rc;
  ART_REQUIRE(F > 0 && F % 64 == 0, "fc1_swiglu: F must be a positive multiple of 64 (F=%d)", F);
  ART_REQUIRE(row_prob && y1 && h, "fc1_swiglu: null pointer");
  if (M == 0) return ART_MOE_OK;
  NTArgs p{};
  p.a = (const bf16 *)a; p.lda = lda; p.a_rows = a_rows;
  p.b = (const bf16 *)w1; p.ldb = K; p.b_es = (int64_t)2 * F * K;
  p.t = kt ? (const bf16 *)tl : nullptr; p.ldt = ldt;
  p.l = kt ? (const bf16 *)l1 : nullptr; p.ldl = kt; p.l_es = (int64_t)2 * F * kt; p.kt = kt;
  p.E = E; p.N = 2 * F; p.K = K; p.alpha = 1.0f; p.F = F; p.prob = row_prob;
  p.y1 = (bf16 *)y1; p.h = (bf16 *)h; p.M = M;
  return launch_nt<128, 128, 2, 2, EPI_SWIGLU_FWD>(p, seg, M, as_stream(stream), "fc1_swiglu");
}

extern "C" int art_moe_dgrad_swiglu_parts(int32_t F) { return F > 0 ? (F + 127) / 128 : 0; }

extern "C" int art_moe_fc2_dgrad_swiglu(const void *a, int64_t lda, const int32_t *a_rows,
                                        const void *w2t, const void *tl, int64_t ldt,
                                        const void *l2, int32_t kt, const int32_t *seg, int32_t E,
                                        int64_t M, int32_t F, int32_t K, const void *y1,
                                        const float *row_prob, void *dy1, float *dp_part,
                                        void *stream) {
  clear_error();
  int rc = check_common(a, lda, w2t, K, seg, E, M, K, kt, tl, ldt, l2, kt, "fc2_dgrad_swiglu");
  if (rc) return rc;
  ART_REQUIRE(F > 0 && F % 8 == 0, "fc2_dgrad_swiglu: F must be a positive multiple of 8 (F=%d)", F);
  ART_REQUIRE(y1 && row_prob && dy1 && dp_part, "fc2_dgrad_swiglu: null pointer");
  if (M == 0) return ART_MOE_OK;
  NTArgs p{};
  p.a = (const bf16 *)a; p.lda = lda; p.a_rows = a_rows;
  p.b = (const bf16 *)w2t; p.ldb = K; p.b_es = (int64_t)F * K;
  p.t = kt ? (const bf16 *)tl : nullptr; p.ldt = ldt;
  p.l = kt ? (const bf16 *)l2 : nullptr; p.ldl = kt; p.l_es = (int64_t)F * kt; p.kt = kt;
  p.E = E; p.N = F; p.K = K; p.alpha = 1.0f; p.F = F; p.prob = row_prob;
  p.y1_in = (const bf16 *)y1; p.dy1 = (bf16 *)dy1; p.dp_part = dp_part; p.M = M;
  return launch_nt<128, 128, 2, 2, EPI_SWIGLU_BWD>(p, seg, M, as_stream(stream),
                                                   "fc2_dgrad_swiglu");
}
