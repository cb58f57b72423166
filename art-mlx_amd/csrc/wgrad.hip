// Segmented "TN" products: LoRA weight gradients with fp32 accumulation.
//
//   out[e][p][q] (+)= alpha * sum_{m in segment e} Lm[lrow(m), p] * R[rrow(m), q]
//
// This is the varlen-K GEMM of the reference's grouped LoRA backward
// (src/art/megatron/kernels/cute_grouped_lora_quack.py:301-334, 411-431):
// grad_A[e] = x_e^T (s dy_e B_e^T) and grad_B[e] = s (x_e A_e)^T dy_e, where the
// reduction runs over the rows (tokens) of expert e's segment.
//
// Work split: a segment is cut into chunks of kWgChunkRows rows (the segment
// table's last tile row counts them per expert); one workgroup owns one
// 128 x BQ output tile of one chunk.  A chunk that is its expert's only one
// writes the output directly; chunks of longer segments write fp32 partial
// tiles to the caller's workspace and a second kernel sums them in chunk
// order.  Every output element is therefore one fixed-order fp32 sum
// (deterministic, no atomics) while a heavily loaded expert (replayed Zipf
// routes) is spread over several workgroups.
//
// Main loop per 64-row step: the next step's rows are loaded into registers
// (16-byte loads, gathered through the row maps) while the MFMAs consume the
// current step from LDS.  The MFMA operands need 8 consecutive rows per lane,
// so rows are transposed on the way into LDS: two rows (m, m+1) are packed
// into 32-bit words at [p][m] (row pitch 128 bytes = 64 rows m), and operand
// fragments are single 16-byte LDS reads.  The 16-byte slot of a chunk is
// XOR-swizzled with bits of the row index so that the 16 lanes of an operand
// read cover all 64 banks and the transposing writes conflict at most 2-way.
// MFMA: v_mfma_f32_16x16x32_bf16 (ranks of 16 waste nothing).
#include "common.h"

namespace art {

constexpr int kWgBK = 64;          // segment rows per main-loop step
constexpr int kWgBP = 128;         // P extent of a workgroup tile
constexpr int kWgChunkRows = ART_MOE_WGRAD_CHUNK;  // rows per chunk: BM of the segment table's last tile row
constexpr int kWgChunkSegRow = ART_MOE_SEG_NBM;  // that row's index in the table

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
  int mode;    // ART_MOE_WGRAD_STORE / _ACCUMULATE / _STORE_BF16
  float *ws;   // partial tiles of multi-chunk experts
  int n_pt, n_qt;
};

// Byte offset in an LDS operand tile of the 16-byte chunk c (rows m = 8c..8c+7)
// of row `row` (a p or q index).
__device__ __forceinline__ int wg_off(int row, int c) {
  return row * 128 + ((c ^ ((row >> 1) ^ (row >> 4)) & 7) << 4);
}

__device__ __forceinline__ void wg_store(const WArgs &a, int e, int p, int q, float acc) {
  const bool second = a.out2 != nullptr && q >= a.q_split;
  void *base = second ? a.out2 : a.out;
  const int64_t off = second
      ? (int64_t)e * a.o2_es + (int64_t)p * a.o2_sp + (int64_t)(q - a.q_split) * a.o2_sq
      : (int64_t)e * a.o_es + (int64_t)p * a.o_sp + (int64_t)q * a.o_sq;
  const float val = a.alpha * acc;
  if (a.mode == ART_MOE_WGRAD_STORE_BF16) {
    ((bf16 *)base)[off] = (bf16)val;
  } else {
    float *o = (float *)base + off;
    *o = a.mode == ART_MOE_WGRAD_ACCUMULATE ? *o + val : val;
  }
}

// 32-bit word holding element j of row m (low half) and of row m+1 (high half)
__device__ __forceinline__ uint32_t pair_word(const U4 &a, const U4 &b, int j) {
  const uint32_t wa = j < 2 ? a.x : j < 4 ? a.y : j < 6 ? a.z : a.w;
  const uint32_t wb = j < 2 ? b.x : j < 4 ? b.y : j < 6 ? b.z : b.w;
  return (j & 1) ? ((wa >> 16) | (wb & 0xffff0000u)) : ((wa & 0xffffu) | (wb << 16));
}

// Rows [mb, mb+64) x columns [c0, c0 + 8*NC) of a row-major operand: NPAIR
// (row pair, 8-column chunk) items per thread, consecutive threads on
// consecutive chunks of a row (coalesced).
template <int NC, int NPAIR>
__device__ __forceinline__ void wg_load(U4 (&v)[NPAIR][2], const bf16 *base, int64_t ld,
                                        const int32_t *rows, int mb, int m_end, int c0, int ncols) {
#pragma unroll
  for (int i = 0; i < NPAIR; ++i) {
    const int id = (int)threadIdx.x + 256 * i;
    const int cc = id % NC, rp = id / NC;
    const int col = c0 + cc * 8;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int m = mb + 2 * rp + h;
      v[i][h] = U4{0u, 0u, 0u, 0u};
      if (rp < kWgBK / 2 && m < m_end && col < ncols) {
        const int64_t src = rows ? (int64_t)rows[m] : (int64_t)m;
        v[i][h] = *(const U4 *)(base + src * ld + col);
      }
    }
  }
}

template <int NC, int NPAIR>
__device__ __forceinline__ void wg_stash(const U4 (&v)[NPAIR][2], char *lds) {
#pragma unroll
  for (int i = 0; i < NPAIR; ++i) {
    const int id = (int)threadIdx.x + 256 * i;
    const int cc = id % NC, rp = id / NC;
    if (rp >= kWgBK / 2) continue;
    const int mm = 2 * rp;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      *(uint32_t *)(lds + wg_off(cc * 8 + j, mm >> 3) + ((mm & 7) << 1)) =
          pair_word(v[i][0], v[i][1], j);
  }
}

// WP x WQ waves; each wave owns TP x TQ blocks of 16x16 outputs.
template <int BQ, int WP, int WQ, int TP, int TQ>
__global__ __launch_bounds__(256) void wgrad_kernel(const WArgs a) {
  static_assert(WP * WQ == 4 && WP * TP * 16 == kWgBP && WQ * TQ * 16 == BQ, "tile");
  constexpr int NCL = kWgBP / 8, NCR = BQ / 8;                    // 8-column chunks per row
  constexpr int NPL = (NCL * kWgBK / 2 + 255) / 256;              // pair items per thread
  constexpr int NPR = (NCR * kWgBK / 2 + 255) / 256;
  constexpr int BUF = (kWgBP + BQ) * 128;                         // bytes per LDS buffer
  __shared__ __attribute__((aligned(16))) char lds[2 * BUF];

  // 1-D grid, XCD-aware: workgroups are dispatched round-robin over the 8
  // XCDs, so the tiles of chunk c all go to XCD c % 8, back to back, and
  // share its L2 for the chunk's rows.
  const int xcd = blockIdx.x & 7, j = blockIdx.x >> 3;
  const int per_chunk = a.n_pt * a.n_qt;
  const int c = (j / per_chunk) * 8 + xcd;
  const int tile = j - (j / per_chunk) * per_chunk;
  const int ty = tile % a.n_pt, tz = tile / a.n_pt;
  const int32_t *cpre = a.seg + kWgChunkSegRow * (a.E + 1);
  if (c >= cpre[a.E]) return;  // workgroup-uniform
  int lo = 0, hi = a.E - 1;    // expert of chunk c: the last e with cpre[e] <= c
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (cpre[mid] <= c) lo = mid; else hi = mid - 1;
  }
  const int e = lo;
  const int nce = cpre[e + 1] - cpre[e];
  const int m0 = a.seg[e] + (c - cpre[e]) * kWgChunkRows;
  const int m1 = min(a.seg[e + 1], m0 + kWgChunkRows);
  const int p0 = ty * kWgBP, q0 = tz * BQ;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wp = wave % WP, wq = wave / WP;
  const int l16 = lane & 15, g4 = lane >> 4;

  f32x4 acc[TP][TQ];
#pragma unroll
  for (int i = 0; i < TP; ++i)
#pragma unroll
    for (int j = 0; j < TQ; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[i][j][v] = 0.0f;

  U4 vl[NPL][2], vr[NPR][2];
  const int nk = (m1 - m0 + kWgBK - 1) / kWgBK;
  wg_load<NCL, NPL>(vl, a.l, a.ldl, a.l_rows, m0, m1, p0, a.P);
  wg_load<NCR, NPR>(vr, a.r, a.ldr, a.r_rows, m0, m1, q0, a.Q);
  wg_stash<NCL, NPL>(vl, lds);
  wg_stash<NCR, NPR>(vr, lds + kWgBP * 128);
  __syncthreads();
  for (int ks = 0; ks < nk; ++ks) {
    const bool more = ks + 1 < nk;
    if (more) {  // next step's rows in flight during this step's MFMAs
      const int mb = m0 + (ks + 1) * kWgBK;
      wg_load<NCL, NPL>(vl, a.l, a.ldl, a.l_rows, mb, m1, p0, a.P);
      wg_load<NCR, NPR>(vr, a.r, a.ldr, a.r_rows, mb, m1, q0, a.Q);
    }
    const char *bl = lds + (ks & 1) * BUF;
    const char *br = bl + kWgBP * 128;
#pragma unroll
    for (int kk = 0; kk < kWgBK / 32; ++kk) {
      const int cidx = kk * 4 + g4;  // lanes 16g..16g+15 take rows m = 32kk + 8g .. +7
      bf16x8 af[TP], bq[TQ];
#pragma unroll
      for (int i = 0; i < TP; ++i)
        af[i] = *(const bf16x8 *)(bl + wg_off(wp * TP * 16 + i * 16 + l16, cidx));
#pragma unroll
      for (int j = 0; j < TQ; ++j)
        bq[j] = *(const bf16x8 *)(br + wg_off(wq * TQ * 16 + j * 16 + l16, cidx));
#pragma unroll
      for (int i = 0; i < TP; ++i)
#pragma unroll
        for (int j = 0; j < TQ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bq[j], acc[i][j], 0, 0, 0);
    }
    if (more) {  // the other buffer: its last readers passed the previous barrier
      char *nb = lds + ((ks + 1) & 1) * BUF;
      wg_stash<NCL, NPL>(vl, nb);
      wg_stash<NCR, NPR>(vr, nb + kWgBP * 128);
    }
    __syncthreads();
  }

  // Accumulator element v of a 16x16 block: row 4*(lane/16) + v, column lane%16.
  // (a multi-chunk expert without workspace means M understated the rows:
  // the host sized nothing for it, so nothing is written)
  if (nce != 1 && a.ws == nullptr) return;
  float *part = nce == 1 ? nullptr
      : a.ws + (((size_t)c * a.n_pt + ty) * a.n_qt + tz) * (size_t)(kWgBP * BQ);
#pragma unroll
  for (int i = 0; i < TP; ++i)
#pragma unroll
    for (int j = 0; j < TQ; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int pl = wp * TP * 16 + i * 16 + g4 * 4 + v;
        const int ql = wq * TQ * 16 + j * 16 + l16;
        if (part) {
          part[pl * BQ + ql] = acc[i][j][v];
        } else if (p0 + pl < a.P && q0 + ql < a.Q) {
          wg_store(a, e, p0 + pl, q0 + ql, acc[i][j][v]);
        }
      }
}

// Outputs of the experts without exactly one chunk: their chunk partials
// summed in chunk order (no chunk: zero).  One workgroup per (expert, tile).
template <int BQ>
__global__ __launch_bounds__(256) void wgrad_reduce_kernel(const WArgs a) {
  const int e = blockIdx.x;
  const int32_t *cpre = a.seg + kWgChunkSegRow * (a.E + 1);
  const int c0 = cpre[e], nce = cpre[e + 1] - c0;
  if (nce == 1 || (nce == 0 && a.mode == ART_MOE_WGRAD_ACCUMULATE)) return;
  if (nce > 1 && a.ws == nullptr) return;
  const int p0 = blockIdx.y * kWgBP, q0 = blockIdx.z * BQ;
  for (int t = threadIdx.x; t < kWgBP * BQ; t += 256) {
    const int pl = t / BQ, ql = t - pl * BQ;
    if (p0 + pl >= a.P || q0 + ql >= a.Q) continue;
    // partials of 8 chunks are loaded before they are added (same chunk order
    // as a plain loop: the sum is identical, the loads overlap)
    const size_t cstride = (size_t)a.n_pt * a.n_qt * (kWgBP * BQ);
    const float *src = a.ws + (((size_t)c0 * a.n_pt + blockIdx.y) * a.n_qt + blockIdx.z) *
                                  (size_t)(kWgBP * BQ) + t;
    float s = 0.0f;
    for (int cb = 0; cb < nce; cb += 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = cb + u < nce ? src[(size_t)(cb + u) * cstride] : 0.0f;
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (cb + u < nce) s += v[u];
    }
    wg_store(a, e, p0 + pl, q0 + ql, s);
  }
}

static int wgrad_bq(int Q) { return Q <= 16 ? 16 : Q <= 32 ? 32 : Q <= 64 ? 64 : 128; }

static int64_t wgrad_max_chunks(int64_t M, int E) {
  return (M + kWgChunkRows - 1) / kWgChunkRows + E;
}

template <int BQ, int WP, int WQ, int TP, int TQ>
static int launch_wgrad(WArgs a, int64_t M, hipStream_t s) {
  a.n_pt = (a.P + kWgBP - 1) / kWgBP;
  a.n_qt = (a.Q + BQ - 1) / BQ;
  if (M > 0) {
    const int64_t groups = (wgrad_max_chunks(M, a.E) + 7) / 8;  // chunk groups of 8 (one per XCD)
    const int64_t blocks = groups * 8 * a.n_pt * a.n_qt;
    ART_REQUIRE(blocks < (int64_t)1 << 31, "grouped_wgrad: too many tiles");
    wgrad_kernel<BQ, WP, WQ, TP, TQ><<<dim3((unsigned)blocks), 256, 0, s>>>(a);
    if (int rc = check_launch("grouped_wgrad")) return rc;
  }
  wgrad_reduce_kernel<BQ><<<dim3((unsigned)a.E, a.n_pt, a.n_qt), 256, 0, s>>>(a);
  return check_launch("grouped_wgrad reduce");
}

}  // namespace art

using namespace art;

extern "C" size_t art_moe_wgrad_workspace_bytes(int64_t M, int32_t E, int32_t P, int32_t Q) {
  if (M <= kWgChunkRows || E <= 0 || P <= 0 || Q <= 0) return 0;  // no segment spans two chunks
  const int bq = wgrad_bq(Q);
  return (size_t)wgrad_max_chunks(M, E) * ((P + kWgBP - 1) / kWgBP) * ((Q + bq - 1) / bq) *
         kWgBP * bq * sizeof(float);
}

extern "C" int art_moe_grouped_wgrad(const void *lm, int64_t ldl, const int32_t *l_rows,
                                     const void *r, int64_t ldr, const int32_t *r_rows,
                                     const int32_t *seg, int32_t E, int64_t M, int32_t P,
                                     int32_t Q, float alpha, void *out, int64_t o_es,
                                     int64_t o_ps, int64_t o_qs, void *out2, int32_t q_split,
                                     int64_t o2_es, int64_t o2_ps, int64_t o2_qs, int32_t mode,
                                     void *workspace, size_t workspace_bytes, void *stream) {
  clear_error();
  ART_REQUIRE(E >= 1 && E <= 65535, "grouped_wgrad: need 1 <= E <= 65535 (E=%d)", E);
  ART_REQUIRE(M >= 0 && M < (int64_t)1 << 31, "grouped_wgrad: need 0 <= M < 2^31");
  ART_REQUIRE(P > 0 && Q > 0 && P % 8 == 0 && Q % 8 == 0,
              "grouped_wgrad: P and Q must be positive multiples of 8 (P=%d Q=%d)", P, Q);
  ART_REQUIRE(ldl % 8 == 0 && ldr % 8 == 0, "grouped_wgrad: row strides must be multiples of 8");
  ART_REQUIRE(lm && r && seg && out, "grouped_wgrad: null pointer");
  ART_REQUIRE(((uintptr_t)lm & 15) == 0 && ((uintptr_t)r & 15) == 0,
              "grouped_wgrad: operands must be 16-byte aligned");
  ART_REQUIRE(mode == ART_MOE_WGRAD_STORE || mode == ART_MOE_WGRAD_ACCUMULATE ||
                  mode == ART_MOE_WGRAD_STORE_BF16,
              "grouped_wgrad: unknown mode %d", mode);
  ART_REQUIRE(!out2 || (q_split > 0 && q_split < Q),
              "grouped_wgrad: split output needs 0 < q_split < Q (q_split=%d Q=%d)", q_split, Q);
  const size_t need = art_moe_wgrad_workspace_bytes(M, E, P, Q);
  ART_REQUIRE(workspace_bytes >= need && (need == 0 || workspace),
              "grouped_wgrad: needs a workspace of %zu bytes (art_moe_wgrad_workspace_bytes)",
              need);
  WArgs a{};
  a.l = (const bf16 *)lm; a.ldl = ldl; a.l_rows = l_rows;
  a.r = (const bf16 *)r; a.ldr = ldr; a.r_rows = r_rows;
  a.seg = seg; a.E = E; a.P = P; a.Q = Q; a.alpha = alpha;
  a.out = out; a.o_es = o_es; a.o_sp = o_ps; a.o_sq = o_qs; a.mode = mode;
  a.out2 = out2; a.q_split = out2 ? q_split : Q;
  a.o2_es = o2_es; a.o2_sp = o2_ps; a.o2_sq = o2_qs;
  a.ws = (float *)workspace;
  hipStream_t s = as_stream(stream);
  switch (wgrad_bq(Q)) {
    case 16: return launch_wgrad<16, 4, 1, 2, 1>(a, M, s);
    case 32: return launch_wgrad<32, 4, 1, 2, 2>(a, M, s);
    case 64: return launch_wgrad<64, 2, 2, 4, 2>(a, M, s);
    default: return launch_wgrad<128, 2, 2, 4, 4>(a, M, s);
  }
}
