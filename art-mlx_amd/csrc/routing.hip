// Routing, dispatch plan, permute and combine kernels (bandwidth-bound family).
//
// Reference semantics (paths under the reference tree):
//   top-k softmax routing   megatron TopKRouter.routing, contract in
//                           tests/unit/test_moe_routing_replay.py:181-205,
//                           restated in src/art/megatron/dsv4/layer.py:139-191
//   routing replay          RouterReplay.get_replay_topk (fake at
//                           tests/unit/test_moe_routing_replay.py:149-161)
//   dispatch order          expert-major, token-ascending (megatron permute
//                           with routing map; canonical order enforced at
//                           tests/integration/megatron/routing_replay/trace.py:181-232)
//   combine                 megatron moe_utils.unpermute (scatter-add of the k
//                           expert rows of each token), signature at
//                           src/art/megatron/runtime/bridge_runtime.py:870-879
#include <math.h>

#include "common.h"

namespace art {

// ---------------------------------------------------------------- top-k
// Total order used for selection: NaN above every number, -0.0 == +0.0, and
// among equal values the lower expert id first.  order_key maps a float to an
// unsigned key that compares like the float; the 64-bit candidate key packs
// (order_key << 32) | ~expert so that one unsigned max picks value then id.
__device__ __forceinline__ uint32_t order_key(float f) {
  if (f != f) return 0xFFFFFFFFu;
  uint32_t u = __float_as_uint(f);
  if ((u << 1) == 0) u = 0;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float key_value(uint32_t key) {
  if (key == 0xFFFFFFFFu) return __uint_as_float(0x7fc00000u);
  uint32_t u = (key & 0x80000000u) ? (key & 0x7fffffffu) : ~key;
  return __uint_as_float(u);
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int o) {
  uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
  lo = __shfl_xor(lo, o, kWave);
  hi = __shfl_xor(hi, o, kWave);
  return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint64_t shfl_u64(uint64_t v, int src) {
  uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
  lo = __shfl(lo, src, kWave);
  hi = __shfl(hi, src, kWave);
  return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// One wavefront per token row; lane l holds experts l, l+64, ... (EPL of them).
template <int EPL>
__global__ __launch_bounds__(256) void topk_softmax_kernel(
    const float *__restrict__ logits, int64_t T, int E, int k,
    int32_t *__restrict__ idx, float *__restrict__ w) {
  const int lane = lane_id();
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const float *row = logits + t * (int64_t)E;
  uint64_t cand[EPL];
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int e = lane + kWave * i;
    cand[i] = (e < E) ? (((uint64_t)order_key(row[e]) << 32) | (uint32_t)(~(uint32_t)e)) : 0ull;
  }
  uint64_t mine = 0;
  for (int j = 0; j < k; ++j) {
    uint64_t best = 0;
#pragma unroll
    for (int i = 0; i < EPL; ++i) best = cand[i] > best ? cand[i] : best;
    uint64_t wbest = best;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      uint64_t other = shfl_xor_u64(wbest, o);
      wbest = other > wbest ? other : wbest;
    }
    // Keys are unique (they embed the id), so exactly one lane owns wbest.
#pragma unroll
    for (int i = 0; i < EPL; ++i)
      if (cand[i] == wbest) cand[i] = 0ull;
    if (lane == j) mine = wbest;
  }
  const bool act = lane < k;
  const float v = act ? key_value((uint32_t)(mine >> 32)) : 0.0f;
  const float vmax = __shfl(v, 0, kWave);  // first winner is the maximum
  const float ex = act ? expf(v - vmax) : 0.0f;
  const float s = wave_sum(ex);
  if (act) {
    idx[t * k + lane] = (int32_t)(~(uint32_t)mine);
    w[t * k + lane] = ex / s;
  }
}

// Replay: lane j < k of the token's wave takes target[t, j].
// The target row of token t is target[t, :] (int64), or, with a row map,
// table[rows[t], :] (int32 [n_rows, k]) for rows[t] >= 0 and
// extra[-rows[t] - 1, :] (int32 [n_extra, k]) for rows[t] < 0; a row map
// entry outside both tables rejects all k ids of the token.
__global__ __launch_bounds__(256) void replay_kernel(
    const float *__restrict__ logits, const int64_t *__restrict__ target,
    const int32_t *__restrict__ table, int64_t n_rows, const int32_t *__restrict__ extra,
    int64_t n_extra, const int32_t *__restrict__ rows,
    int64_t T, int E, int k, int32_t *__restrict__ idx, float *__restrict__ w,
    int32_t *__restrict__ status) {
  const int lane = lane_id();
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const bool act = lane < k;
  int64_t e = -1;
  if (act) {
    if (rows) {
      const int64_t r = rows[t];
      if (r >= 0) e = r < n_rows ? (int64_t)table[r * k + lane] : -1;
      else e = -r <= n_extra ? (int64_t)extra[(-r - 1) * k + lane] : -1;
    } else {
      e = target[t * k + lane];
    }
  }
  bool valid = act && e >= 0 && e < E;
  // Repeated id in a row: every later occurrence is rejected.
  for (int j = 0; j < k; ++j) {
    const int64_t ej = (int64_t)shfl_u64((uint64_t)e, j);
    if (j < lane && ej == e) valid = false;
  }
  const float v = valid ? logits[t * (int64_t)E + e] : -INFINITY;
  const float vmax = wave_max(valid ? v : -INFINITY);
  const float ex = valid ? expf(v - vmax) : 0.0f;
  const float s = wave_sum(ex);
  if (act) {
    idx[t * k + lane] = valid ? (int32_t)e : -1;
    w[t * k + lane] = valid ? ex / s : 0.0f;
    if (!valid) atomicAdd(status, 1);
  }
}

// ------------------------------------------------------------ dispatch plan
// Tokens are cut into chunks of 64 (one wavefront each).  For every chunk c
// and expert e the plan keeps the 64-bit set of chunk lanes routed to e; the
// permuted row of (t, e) is then
//   seg[e] + sum_{c' < c} popcount(mask[c'][e]) + popcount(mask[c][e] & lanes_below(t))
// which is exactly the stable expert-major / token-ascending order.
__global__ __launch_bounds__(256) void plan_count_kernel(
    const int32_t *__restrict__ idx, int64_t T, int E, int k,
    uint64_t *__restrict__ masks, int32_t *__restrict__ chunk_cnt,
    int32_t *__restrict__ status) {
  extern __shared__ uint64_t lds_mask[];  // [4][E]
  const int wv = threadIdx.x >> 6, lane = lane_id();
  const int64_t nchunks = (T + 63) >> 6;
  const int64_t chunk = (int64_t)blockIdx.x * 4 + wv;
  uint64_t *m = lds_mask + wv * E;
  for (int e = lane; e < E; e += kWave) m[e] = 0ull;
  __syncthreads();
  const int64_t t = chunk * 64 + lane;
  if (chunk < nchunks && t < T) {
    const uint64_t bit = 1ull << lane;
    for (int j = 0; j < k; ++j) {
      const int e = idx[t * k + j];
      if (e < 0 || e >= E) {
        atomicAdd(status, 1);
        continue;
      }
      const uint64_t old = atomicOr((unsigned long long *)&m[e], (unsigned long long)bit);
      if (old & bit) atomicAdd(status, 1);
    }
  }
  __syncthreads();
  if (chunk < nchunks) {
    for (int e = lane; e < E; e += kWave) {
      masks[chunk * E + e] = m[e];
      chunk_cnt[chunk * E + e] = __popcll(m[e]);
    }
  }
}

// Block-wide exclusive scan of one int per thread (blockDim.x <= 1024).
__device__ int block_exclusive_scan(int v, int *total) {
  __shared__ int wsum[16];
  const int lane = lane_id(), wv = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
  int incl = v;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int y = __shfl_up(incl, o, kWave);
    if (lane >= o) incl += y;
  }
  __syncthreads();
  if (lane == kWave - 1) wsum[wv] = incl;
  __syncthreads();
  int base = 0, tot = 0;
  for (int i = 0; i < nw; ++i) {
    if (i < wv) base += wsum[i];
    tot += wsum[i];
  }
  *total = tot;
  return base + incl - v;
}

// One workgroup per expert: exclusive scan of its per-chunk counts.
__global__ __launch_bounds__(256) void plan_scan_kernel(
    const int32_t *__restrict__ chunk_cnt, int64_t nchunks, int E,
    int32_t *__restrict__ chunk_base, int32_t *__restrict__ counts) {
  const int e = blockIdx.x;
  const int64_t per = (nchunks + blockDim.x - 1) / blockDim.x;
  const int64_t c0 = threadIdx.x * per;
  const int64_t c1 = c0 + per < nchunks ? c0 + per : nchunks;
  int s = 0;
  for (int64_t c = c0; c < c1; ++c) s += chunk_cnt[c * E + e];
  int total;
  int run = block_exclusive_scan(s, &total);
  for (int64_t c = c0; c < c1; ++c) {
    chunk_base[c * E + e] = run;
    run += chunk_cnt[c * E + e];
  }
  if (threadIdx.x == 0) counts[e] = total;
}

// Segment table from counts: row offsets plus row-tile prefixes for BM = 64*b.
template <typename CT>
__global__ __launch_bounds__(1024) void segments_kernel(const CT *__restrict__ counts, int E,
                                                        int32_t *__restrict__ seg) {
  const int e = threadIdx.x;
  const int c = e < E ? (int)counts[e] : 0;
#pragma unroll
  for (int b = 0; b <= ART_MOE_SEG_NBM; ++b) {
    int v;
    if (b == 0) {
      v = c;
    } else {
      // row-tile heights 64, 128, 192, 256 and the 2048-row wgrad chunk
      const int bm = b == ART_MOE_SEG_NBM ? ART_MOE_WGRAD_CHUNK : 64 * b;
      v = (c + bm - 1) / bm;
    }
    int total;
    const int ex = block_exclusive_scan(v, &total);
    if (e < E) seg[b * (E + 1) + e] = ex;
    if (e == 0) seg[b * (E + 1) + E] = total;
  }
}

__global__ __launch_bounds__(256) void plan_scatter_kernel(
    const int32_t *__restrict__ idx, const float *__restrict__ w, int64_t T, int E, int k,
    const uint64_t *__restrict__ masks, const int32_t *__restrict__ chunk_base,
    const int32_t *__restrict__ seg, int32_t *__restrict__ dest,
    int32_t *__restrict__ row_token, float *__restrict__ row_prob) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= T * k) return;
  // Rows past the last segment (one per rejected or repeated id) belong to no
  // expert; they map to token 0 with probability 0, so a consumer that walks
  // all T*k rows (the fp8 row quantiser) gathers in-bounds rows.  No (t, e)
  // pair scatters there: every pos below is < seg[E].
  if (i >= seg[E]) {
    row_token[i] = 0;
    if (row_prob) row_prob[i] = 0.0f;
  }
  const int64_t t = i / k;
  const int j = (int)(i - t * k);
  const int e = idx[i];
  bool ok = e >= 0 && e < E;
  for (int jj = 0; jj < j; ++jj)
    if (idx[t * k + jj] == e) ok = false;
  if (!ok) {
    dest[i] = -1;
    return;
  }
  const int64_t c = t >> 6;
  const int lane = (int)(t & 63);
  const uint64_t m = masks[c * E + e];
  const uint64_t below = lane ? (m & ((1ull << lane) - 1ull)) : 0ull;
  const int pos = seg[e] + chunk_base[c * E + e] + __popcll(below);
  dest[i] = pos;
  row_token[pos] = (int32_t)t;
  if (row_prob) row_prob[pos] = w[i];
}

// ---------------------------------------------------------- permute / combine
// One wavefront per token; rows move as 16-byte chunks of 8 bf16.  A token's
// destination slots are read 64 at a time (one per lane) and broadcast.
__global__ __launch_bounds__(256) void permute_kernel(const U4 *__restrict__ x,
                                                      const int32_t *__restrict__ dest,
                                                      int64_t T, int k, int H8,
                                                      U4 *__restrict__ xp) {
  const int lane = lane_id();
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const int my_dest = lane < k ? dest[t * k + lane] : -1;
  const U4 *src = x + t * H8;
  for (int c0 = 0; c0 < H8; c0 += 4 * kWave) {
    U4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = c0 + u * kWave + lane;
      if (c < H8) v[u] = src[c];
    }
    for (int j0 = 0; j0 < k; j0 += kWave) {
      const int md = j0 == 0 ? my_dest : (j0 + lane < k ? dest[t * k + j0 + lane] : -1);
      const int kb = k - j0 < kWave ? k - j0 : kWave;
      for (int j = 0; j < kb; ++j) {
        const int d = __shfl(md, j, kWave);
        if (d < 0) continue;
        U4 *dst = xp + (int64_t)d * H8;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int c = c0 + u * kWave + lane;
          if (c < H8) dst[c] = v[u];
        }
      }
    }
  }
}

constexpr int kMaxK = 32;        // top-k of the router kernels
constexpr int kMaxSlots = 1024;  // slots per token of permute / combine (capacity layouts: E)

__global__ __launch_bounds__(256) void combine_kernel(
    const U4 *__restrict__ yp, const int32_t *__restrict__ dest, const float *__restrict__ wgt,
    const float *__restrict__ dl, const int32_t *__restrict__ idx, const U4 *__restrict__ w_r,
    const U4 *__restrict__ addend, int64_t T, int k, int H8, int n_chunks, U4 *__restrict__ y) {
  const int lane = lane_id();
  // One wavefront per (token, 64-lane chunk of the row): short waves that
  // keep many rows in flight and leave no long tail when the grid is a
  // fraction of a round over the resident waves.
  const int64_t wv = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t t = wv / n_chunks;
  if (t >= T) return;
  const int c0 = (int)(wv - t * n_chunks) * kWave;
  const bool act = lane < k;
  const int my_e = (act && w_r) ? idx[t * k + lane] : -1;     // w_r: k <= 32
  const float my_dl = (act && w_r) ? dl[t * k + lane] : 0.0f;
  // Every lane of the wavefront runs the slot loops (uniform), so the slot
  // broadcasts below always read active lanes.  Slots go in blocks of 8
  // whose row loads are all issued before the first is accumulated (8 loads
  // in flight per lane instead of a chain of k); the accumulation order
  // stays slot-ascending.  Slot j >= k reads lane j's inactive dest (-1).
  {
    const int c = c0 + lane;
    const bool on = c < H8;
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
    for (int j0 = 0; j0 < k; j0 += kWave) {      // slots 64 at a time, one per lane
      const int kb = k - j0 < kWave ? k - j0 : kWave;
      const bool a = lane < kb;
      const int my_dest = a ? dest[t * k + j0 + lane] : -1;
      const float my_w = (a && wgt) ? wgt[t * k + j0 + lane] : 1.0f;
      for (int jb = 0; jb < kb; jb += 8) {
        U4 v[8];
        int dj[8];
        float wj[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          dj[u] = __shfl(my_dest, jb + u, kWave);
          wj[u] = __shfl(my_w, jb + u, kWave);
          v[u] = (dj[u] >= 0 && on) ? yp[(int64_t)dj[u] * H8 + c] : U4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          if (dj[u] < 0) continue;
          float f[8];
          unpack8(v[u], f);
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[i] += wj[u] * f[i];
        }
      }
    }
    if (w_r) {
      for (int jb = 0; jb < k; jb += 8) {
        U4 v[8];
        int ej[8];
        float lj[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          ej[u] = __shfl(my_e, jb + u, kWave);
          lj[u] = __shfl(my_dl, jb + u, kWave);
          v[u] = (ej[u] >= 0 && on) ? w_r[(int64_t)ej[u] * H8 + c] : U4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          if (ej[u] < 0) continue;
          float f[8];
          unpack8(v[u], f);
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[i] += lj[u] * f[i];
        }
      }
    }
    if (addend && on) {
      float f[8];
      unpack8(addend[t * H8 + c], f);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] += f[i];
    }
    if (on) y[t * H8 + c] = pack8(acc);
  }
}

// ---------------------------------------------------------- router LoRA
// logits[t, :] += scale * t_r[t, :] B over 64-token tiles.  LDS holds the
// tile's t_r transposed, [rank][token] with a 68-float row (16-byte aligned,
// and the transposing writes spread over 16 banks), and one 64-column chunk of
// B as fp32 [rank][64]: dynamic size (68 + 64) * rp floats, rp = the rank
// padded to 4.  Wave w owns tokens 16w .. 16w+15 of the tile and lane l column
// l of the chunk; per rank step it reads its 16 tokens' t_r values as four
// broadcast float4s and one B value, four rank steps' reads issued together.
constexpr int kLoraTileTokens = 64, kLoraCols = 64, kLoraMaxRank = 256, kLoraTrRow = 68;

__global__ __launch_bounds__(256) void router_lora_apply_kernel(
    const float *__restrict__ t_r, int64_t T, int r, const bf16 *__restrict__ b, int E,
    float scale, float *__restrict__ logits, bf16 *__restrict__ t_bf16) {
  extern __shared__ __attribute__((aligned(16))) float lora_s[];
  const int lane = lane_id(), wave = threadIdx.x >> 6;
  const int64_t t0 = (int64_t)blockIdx.x * kLoraTileTokens;
  const int nt = (int)(T - t0 < kLoraTileTokens ? T - t0 : kLoraTileTokens);
  const int rp = (r + 3) & ~3;  // rank padded to 4 (zeros)
  float *tr_s = lora_s, *b_s = lora_s + kLoraTrRow * rp;
  for (int i = lane; i < rp; i += kWave) {  // lanes along the rank, 16 token rows per wave
    float v[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) {  // loads first, so all 16 are in flight together
      const int u = wave + 4 * q;
      v[q] = (u < nt && i < r) ? t_r[(t0 + u) * r + i] : 0.0f;
    }
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int u = wave + 4 * q;
      tr_s[i * kLoraTrRow + u] = v[q];
      if (t_bf16 && u < nt && i < r) t_bf16[(t0 + u) * r + i] = (bf16)v[q];
    }
  }
  const float *trw = tr_s + wave * 16;
  for (int e0 = 0; e0 < E; e0 += kLoraCols) {
    __syncthreads();  // tr_s written / the previous chunk of b_s consumed
    for (int i0 = wave; i0 < rp; i0 += 4 * 8) {  // rank rows, lanes along the columns
      float v[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int i = i0 + 4 * q;
        v[q] = (i < r && e0 + lane < E) ? (float)b[(int64_t)i * E + e0 + lane] : 0.0f;
      }
#pragma unroll
      for (int q = 0; q < 8; ++q)
        if (i0 + 4 * q < rp) b_s[(i0 + 4 * q) * kLoraCols + lane] = v[q];
    }
    __syncthreads();
    float acc[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) acc[u] = 0.0f;
    for (int i = 0; i < rp; i += 4) {
      float bv[4];
      float4 tv[4][4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        bv[c] = b_s[(i + c) * kLoraCols + lane];
#pragma unroll
        for (int q = 0; q < 4; ++q) tv[c][q] = *(const float4 *)(trw + (i + c) * kLoraTrRow + 4 * q);
      }
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          acc[4 * q + 0] += tv[c][q].x * bv[c];
          acc[4 * q + 1] += tv[c][q].y * bv[c];
          acc[4 * q + 2] += tv[c][q].z * bv[c];
          acc[4 * q + 3] += tv[c][q].w * bv[c];
        }
    }
    const int e = e0 + lane;
    if (e < E) {
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int tu = wave * 16 + u;
        if (tu < nt) logits[(t0 + tu) * E + e] += scale * acc[u];
      }
    }
  }
}

// B^T staged in LDS ([E][r] bf16) once per block; each wavefront walks its
// tokens in batches of 64 / k, whose ids and weights one load brings in (lane
// l holds slot l % k of the batch's token l / k): lane i of g sums the k
// selected columns of B, and the dense bf16 dlogits row is written with lanes
// over E.
constexpr int kLoraGradTokens = 64;  // tokens per workgroup (16 per wavefront)

__global__ __launch_bounds__(256) void router_lora_grad_kernel(
    const float *__restrict__ dl, const int32_t *__restrict__ idx, int64_t T, int k,
    const bf16 *__restrict__ b, int r, int E, float scale, bf16 *__restrict__ g,
    bf16 *__restrict__ dlog) {
  extern __shared__ bf16 bt[];  // [E][r + 2]: the padded row spreads the transposing writes
  const int rs = r + 2;
  const int lane = lane_id(), wave = threadIdx.x >> 6;
  for (int e = lane; e < E; e += kWave)
    for (int i0 = wave; i0 < r; i0 += 4 * 8) {  // 8 loads in flight per lane
      bf16 v[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int i = i0 + 4 * q;
        v[q] = i < r ? b[(int64_t)i * E + e] : (bf16)0.0f;
      }
#pragma unroll
      for (int q = 0; q < 8; ++q)
        if (i0 + 4 * q < r) bt[e * rs + i0 + 4 * q] = v[q];
    }
  __syncthreads();
  const int64_t tb = (int64_t)blockIdx.x * kLoraGradTokens + wave * (kLoraGradTokens / 4);
  const int64_t te = tb + kLoraGradTokens / 4 < T ? tb + kLoraGradTokens / 4 : T;
  const int per = kWave / k;  // tokens per batch (k <= 32: at least 2)
  for (int64_t t0 = tb; t0 < te; t0 += per) {
    const int nb = (int)(te - t0 < per ? te - t0 : per);
    const bool act = lane < nb * k;
    const int my_e = act ? idx[t0 * k + lane] : -1;
    const float my_dl = act ? dl[t0 * k + lane] : 0.0f;
    for (int u = 0; u < nb; ++u) {
      const int64_t t = t0 + u;
      for (int i0 = 0; i0 < r; i0 += kWave) {
        const int i = i0 + lane;
        const int ic = i < r ? i : r - 1;
        float acc = 0.0f;
        for (int j0 = 0; j0 < k; j0 += 8) {  // 8 slots' LDS reads in flight together
          float lj[8], bv[8];
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            const int j = j0 + q < k ? j0 + q : k - 1;
            const int e = __shfl(my_e, u * k + j, kWave);
            lj[q] = (j0 + q < k && e >= 0) ? __shfl(my_dl, u * k + j, kWave) : 0.0f;
            bv[q] = (float)bt[(e >= 0 ? e : 0) * rs + ic];
          }
#pragma unroll
          for (int q = 0; q < 8; ++q) acc += lj[q] * bv[q];
        }
        if (i < r) g[t * r + i] = (bf16)(scale * acc);
      }
      for (int e0 = 0; e0 < E; e0 += kWave) {
        const int e = e0 + lane;
        float v = 0.0f;
        for (int j = 0; j < k; ++j) {
          const int ej = __shfl(my_e, u * k + j, kWave);
          const float lj = __shfl(my_dl, u * k + j, kWave);
          if (ej == e) v += lj;
        }
        if (e < E) dlog[t * E + e] = (bf16)v;
      }
    }
  }
}

// dl[t,j] = w_j * (dw_j - sum_i w_i dw_i), dw_j = sum_p dp_part[p][dest[t,j]].
__global__ __launch_bounds__(256) void router_backward_kernel(
    const float *__restrict__ dp_part, int n_part, int64_t M, const int32_t *__restrict__ dest,
    const float *__restrict__ w, const int32_t *__restrict__ idx, int64_t T, int E, int k,
    float *__restrict__ dl, float *__restrict__ dlogits) {
  const int lane = lane_id();
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const bool act = lane < k;
  const int d = act ? dest[t * k + lane] : -1;
  float dw = 0.0f;
  if (d >= 0)
    for (int p = 0; p < n_part; ++p) dw += dp_part[(int64_t)p * M + d];
  const float wj = (act && d >= 0) ? w[t * k + lane] : 0.0f;
  const float s = wave_sum(wj * dw);
  const float g = wj * (dw - s);
  if (act) dl[t * k + lane] = g;
  if (dlogits) {
    const int my_e = (act && d >= 0) ? idx[t * k + lane] : -1;
    int ej[kMaxK];
    float gj[kMaxK];
#pragma unroll
    for (int j = 0; j < kMaxK; ++j) {
      ej[j] = __shfl(my_e, j, kWave);
      gj[j] = __shfl(g, j, kWave);
    }
    for (int e = lane; e < E; e += kWave) {
      float v = 0.0f;
#pragma unroll
      for (int j = 0; j < kMaxK; ++j)
        if (j < k && ej[j] == e) v = gj[j];
      dlogits[t * (int64_t)E + e] = v;
    }
  }
}

// ------------------------------------------------------------ transpose
__global__ __launch_bounds__(256) void transpose_kernel(const bf16 *__restrict__ src, int R, int C,
                                                        int64_t s_es, int64_t s_ld,
                                                        bf16 *__restrict__ dst, int64_t d_es,
                                                        int64_t d_ld, float scale) {
  __shared__ float tile[32][33];
  const int e = blockIdx.z;
  const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
  const bf16 *s = src + e * s_es;
  bf16 *d = dst + e * d_es;
  for (int i = ty; i < 32; i += 8) {
    const int r = r0 + i, c = c0 + tx;
    tile[i][tx] = (r < R && c < C) ? (float)s[(int64_t)r * s_ld + c] : 0.0f;
  }
  __syncthreads();
  for (int i = ty; i < 32; i += 8) {
    const int c = c0 + i, r = r0 + tx;
    if (r < R && c < C) d[(int64_t)c * d_ld + r] = (bf16)(scale * tile[tx][i]);
  }
}

// ---------------------------------------------------------------- pack
struct PackArgs {
  art_moe_pack_desc d[ART_MOE_PACK_MAX];
  int32_t tile_start[ART_MOE_PACK_MAX + 1];  // prefix of tiles over descriptors
  int32_t tc_log2[ART_MOE_PACK_MAX];         // tile = (4096 >> tc_log2) x (1 << tc_log2)
  int32_t vec_read[ART_MOE_PACK_MAX];        // 16-byte source loads allowed
  int32_t vec_write[ART_MOE_PACK_MAX];       // 16-byte destination stores allowed
  int n;
};

constexpr int kPackTile = 4096;  // elements per workgroup tile

// Tile width: the destination's row length rounded up to a power of two in
// [16, 256], capped at 64 when the block is also tall (square-ish copies),
// so that rank-sized dimensions (16..64) fill whole tiles.
static int pack_tc_log2(int R, int C) {
  int l = 4;
  while (l < 8 && (1 << l) < C) ++l;
  if (R >= 64 && l > 6) l = 6;
  return l;
}

// One workgroup per tile of one expert; each thread moves two runs of 8
// elements.  Source runs follow the source's fast index (the one with stride
// 1 when there is one: coalesced for plain and transposed reads alike), are
// parked in LDS as fp32 (row pitch TC+1), and leave as 8-element runs along
// destination rows.  Runs are 16-byte accesses where the host found strides
// and alignment to allow it and the run is whole; element accesses otherwise.
// 16-bit element access of pack_kernel: bfloat16, or IEEE half with F16.
template <bool F16>
__device__ __forceinline__ float ld16(const bf16 *p) {
  if constexpr (F16) return (float)*(const _Float16 *)p;
  else return (float)*p;
}
template <bool F16>
__device__ __forceinline__ void st16(bf16 *p, float v) {
  if constexpr (F16) *(_Float16 *)p = (_Float16)v;
  else *p = (bf16)v;
}
template <bool F16>
__device__ __forceinline__ void unpack8t(const U4 &u, float *f) {
  if constexpr (F16) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] & 0xffffu));
      f[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] >> 16));
    }
  } else {
    unpack8(u, f);
  }
}
template <bool F16>
__device__ __forceinline__ U4 pack8t(const float *f) {
  if constexpr (F16) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f[2 * i]) |
             ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f[2 * i + 1]) << 16);
    return U4{w[0], w[1], w[2], w[3]};
  } else {
    return pack8(f);
  }
}

template <bool F16>
__global__ __launch_bounds__(256) void pack_kernel(const PackArgs a) {
  __shared__ float tile[kPackTile + 256];
  const int b = blockIdx.x;
  int k = 0;
  while (k + 1 < a.n && a.tile_start[k + 1] <= b) ++k;
  const art_moe_pack_desc &d = a.d[k];
  const int tcl = a.tc_log2[k];
  const int TC = 1 << tcl, TR = kPackTile >> tcl, pitch = TC + 1;
  const int lb = b - a.tile_start[k];
  const int tcn = (d.C + TC - 1) / TC, per_e = ((d.R + TR - 1) / TR) * tcn;
  const int e = lb / per_e, rem = lb - e * per_e;
  const int r0 = (rem / tcn) * TR, c0 = (rem % tcn) * TC;
  const bool cfast = d.s_cs == 1;
  const int64_t fstride = cfast ? d.s_cs : d.s_rs;
  const int f8l = (cfast ? tcl : 12 - tcl) - 3;  // log2(runs per fast line)
  const int fast_lim = cfast ? d.src_c : d.src_r, slow_lim = cfast ? d.src_r : d.src_c;
  const bool vr = a.vec_read[k] != 0, vw = a.vec_write[k] != 0;
  const bf16 *src = (const bf16 *)d.src + (int64_t)e * d.s_es;

  float v[2][8];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int u = j * 256 + (int)threadIdx.x;
    const int f0 = (u & ((1 << f8l) - 1)) * 8, sl = u >> f8l;
    const int rb = r0 + (cfast ? sl : f0), cb = c0 + (cfast ? f0 : sl);
    const int fa = cfast ? cb : rb, sa = cfast ? rb : cb;
    const bf16 *p = src + (int64_t)rb * d.s_rs + (int64_t)cb * d.s_cs;
    if (sa < slow_lim && vr && fa + 8 <= fast_lim) {
      unpack8t<F16>(*(const U4 *)p, v[j]);
#pragma unroll
      for (int t = 0; t < 8; ++t) v[j][t] *= d.scale;
    } else {
#pragma unroll
      for (int t = 0; t < 8; ++t)
        v[j][t] = (sa < slow_lim && fa + t < fast_lim) ? d.scale * ld16<F16>(p + t * fstride) : 0.0f;
    }
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int u = j * 256 + (int)threadIdx.x;
    const int f0 = (u & ((1 << f8l) - 1)) * 8, sl = u >> f8l;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int rr = cfast ? sl : f0 + t, cc = cfast ? f0 + t : sl;
      tile[rr * pitch + cc] = v[j][t];
    }
  }
  __syncthreads();
  bf16 *dst = (bf16 *)d.dst + (int64_t)e * d.d_es;
  const int c8l = tcl - 3;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int u = j * 256 + (int)threadIdx.x;
    const int cc0 = (u & ((1 << c8l) - 1)) * 8, rr = u >> c8l;
    const int r = r0 + rr, c = c0 + cc0;
    if (r >= d.R) continue;
    float w[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) w[t] = tile[rr * pitch + cc0 + t];
    bf16 *q = dst + (int64_t)r * d.d_rs + c;
    if (vw && c + 8 <= d.C) {
      *(U4 *)q = pack8t<F16>(w);
    } else {
#pragma unroll
      for (int t = 0; t < 8; ++t)
        if (c + t < d.C) st16<F16>(q + t, w[t]);
    }
  }
}

}  // namespace art

using namespace art;

// ================================================================ C ABI
extern "C" int art_moe_router_topk(const float *logits, int64_t T, int32_t E, int32_t k,
                                   int32_t *idx, float *w, void *stream) {
  clear_error();
  ART_REQUIRE(T >= 0 && E >= 1 && E <= 1024, "router_topk: need T >= 0 and 1 <= E <= 1024 (T=%lld E=%d)", (long long)T, E);
  ART_REQUIRE(k >= 1 && k <= E && k <= kMaxK, "router_topk: need 1 <= k <= min(E, 32) (k=%d)", k);
  if (T == 0) return ART_MOE_OK;
  ART_REQUIRE(logits && idx && w, "router_topk: null pointer");
  const dim3 grid((unsigned)((T + 3) / 4));
  hipStream_t s = as_stream(stream);
  const int epl = (E + 63) / 64;
  if (epl <= 1) topk_softmax_kernel<1><<<grid, 256, 0, s>>>(logits, T, E, k, idx, w);
  else if (epl <= 2) topk_softmax_kernel<2><<<grid, 256, 0, s>>>(logits, T, E, k, idx, w);
  else if (epl <= 4) topk_softmax_kernel<4><<<grid, 256, 0, s>>>(logits, T, E, k, idx, w);
  else if (epl <= 8) topk_softmax_kernel<8><<<grid, 256, 0, s>>>(logits, T, E, k, idx, w);
  else topk_softmax_kernel<16><<<grid, 256, 0, s>>>(logits, T, E, k, idx, w);
  return check_launch("router_topk");
}

extern "C" int art_moe_router_replay(const float *logits, const int64_t *target, int64_t T,
                                     int32_t E, int32_t k, int32_t *idx, float *w,
                                     int32_t *status, void *stream) {
  clear_error();
  ART_REQUIRE(T >= 0 && E >= 1, "router_replay: need T >= 0 and E >= 1");
  ART_REQUIRE(k >= 1 && k <= E && k <= kMaxK, "router_replay: need 1 <= k <= min(E, 32) (k=%d)", k);
  if (T == 0) return ART_MOE_OK;
  ART_REQUIRE(logits && target && idx && w && status, "router_replay: null pointer");
  replay_kernel<<<dim3((unsigned)((T + 3) / 4)), 256, 0, as_stream(stream)>>>(
      logits, target, nullptr, 0, nullptr, 0, nullptr, T, E, k, idx, w, status);
  return check_launch("router_replay");
}

extern "C" int art_moe_router_replay_rows(const float *logits, const int32_t *table,
                                          int64_t n_rows, const int32_t *extra, int64_t n_extra,
                                          const int32_t *rows, int64_t T, int32_t E, int32_t k,
                                          int32_t *idx, float *w, int32_t *status, void *stream) {
  clear_error();
  ART_REQUIRE(T >= 0 && n_rows >= 0 && n_extra >= 0 && E >= 1,
              "router_replay_rows: need T, n_rows, n_extra >= 0 and E >= 1");
  ART_REQUIRE(k >= 1 && k <= E && k <= kMaxK, "router_replay_rows: need 1 <= k <= min(E, 32) (k=%d)",
              k);
  if (T == 0) return ART_MOE_OK;
  ART_REQUIRE(logits && rows && idx && w && status && (table || n_rows == 0) &&
                  (extra || n_extra == 0),
              "router_replay_rows: null pointer");
  replay_kernel<<<dim3((unsigned)((T + 3) / 4)), 256, 0, as_stream(stream)>>>(
      logits, nullptr, table, n_rows, extra, n_extra, rows, T, E, k, idx, w, status);
  return check_launch("router_replay_rows");
}

extern "C" int art_moe_router_backward(const float *dp_part, int32_t n_part, int64_t M,
                                       const int32_t *dest, const float *w, const int32_t *idx,
                                       int64_t T, int32_t E, int32_t k, float *dl, float *dlogits,
                                       void *stream) {
  clear_error();
  ART_REQUIRE(T >= 0 && E >= 1 && k >= 1 && k <= kMaxK && n_part >= 0,
              "router_backward: bad sizes (T=%lld E=%d k=%d n_part=%d)", (long long)T, E, k, n_part);
  if (T == 0) return ART_MOE_OK;
  ART_REQUIRE(dest && w && dl && (n_part == 0 || dp_part) && (!dlogits || idx),
              "router_backward: null pointer");
  router_backward_kernel<<<dim3((unsigned)((T + 3) / 4)), 256, 0, as_stream(stream)>>>(
      dp_part, n_part, M, dest, w, idx, T, E, k, dl, dlogits);
  return check_launch("router_backward");
}

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

extern "C" size_t art_moe_plan_workspace_bytes(int64_t T, int32_t E) {
  if (T < 0 || E < 1) return 0;
  const size_t nch = (size_t)((T + 63) / 64);
  return align256(nch * E * sizeof(uint64_t)) + 2 * align256(nch * E * sizeof(int32_t));
}

extern "C" int art_moe_dispatch_plan(const int32_t *idx, const float *w, int64_t T, int32_t E,
                                     int32_t k, int32_t *counts, int32_t *seg, int32_t *dest,
                                     int32_t *row_token, float *row_prob, int32_t *status,
                                     void *workspace, size_t workspace_bytes, void *stream) {
  clear_error();
  ART_REQUIRE(T >= 0 && E >= 1 && E <= 1024, "dispatch_plan: need 1 <= E <= 1024 (E=%d)", E);
  ART_REQUIRE(k >= 1 && k <= E && k <= kMaxK, "dispatch_plan: need 1 <= k <= min(E, 32) (k=%d)", k);
  ART_REQUIRE(T * (int64_t)k < (int64_t)INT32_MAX, "dispatch_plan: T*k must fit int32");
  ART_REQUIRE(counts && seg && status, "dispatch_plan: null pointer");
  const size_t need = art_moe_plan_workspace_bytes(T, E);
  ART_REQUIRE(workspace_bytes >= need, "dispatch_plan: workspace %zu < %zu bytes", workspace_bytes, need);
  hipStream_t s = as_stream(stream);
  const int64_t nch = (T + 63) / 64;
  char *ws = (char *)workspace;
  uint64_t *masks = (uint64_t *)ws;
  int32_t *ccnt = (int32_t *)(ws + align256(nch * E * sizeof(uint64_t)));
  int32_t *cbase = (int32_t *)((char *)ccnt + align256(nch * E * sizeof(int32_t)));
  if (T > 0) {
    ART_REQUIRE(idx && dest && row_token && (!row_prob || w), "dispatch_plan: null pointer");
    plan_count_kernel<<<dim3((unsigned)((nch + 3) / 4)), 256, 4 * E * sizeof(uint64_t), s>>>(
        idx, T, E, k, masks, ccnt, status);
    int rc = check_launch("dispatch_plan/count");
    if (rc) return rc;
    plan_scan_kernel<<<dim3(E), 256, 0, s>>>(ccnt, nch, E, cbase, counts);
    rc = check_launch("dispatch_plan/scan");
    if (rc) return rc;
    segments_kernel<int32_t><<<1, 1024, 0, s>>>(counts, E, seg);
    rc = check_launch("dispatch_plan/segments");
    if (rc) return rc;
    const int64_t n = T * k;
    plan_scatter_kernel<<<dim3((unsigned)((n + 255) / 256)), 256, 0, s>>>(
        idx, w, T, E, k, masks, cbase, seg, dest, row_token, row_prob);
    return check_launch("dispatch_plan/scatter");
  }
  // T == 0: all experts empty.
  plan_scan_kernel<<<dim3(E), 256, 0, s>>>(ccnt, 0, E, cbase, counts);
  int rc = check_launch("dispatch_plan/scan");
  if (rc) return rc;
  segments_kernel<int32_t><<<1, 1024, 0, s>>>(counts, E, seg);
  return check_launch("dispatch_plan/segments");
}

extern "C" int art_moe_segments_from_counts(const int64_t *counts, int32_t E, int32_t *seg,
                                            void *stream) {
  clear_error();
  ART_REQUIRE(E >= 1 && E <= 1024, "segments_from_counts: need 1 <= E <= 1024 (E=%d)", E);
  ART_REQUIRE(counts && seg, "segments_from_counts: null pointer");
  segments_kernel<int64_t><<<1, 1024, 0, as_stream(stream)>>>(counts, E, seg);
  return check_launch("segments_from_counts");
}

extern "C" int art_moe_permute(const void *x, const int32_t *dest, int64_t T, int32_t k,
                               int32_t H, void *x_perm, void *stream) {
  clear_error();
  ART_REQUIRE(T >= 0 && k >= 1 && k <= kMaxSlots && H > 0 && H % 8 == 0,
              "permute: need H %% 8 == 0 and 1 <= k <= 1024 (H=%d k=%d)", H, k);
  if (T == 0) return ART_MOE_OK;
  ART_REQUIRE(x && dest && x_perm, "permute: null pointer");
  permute_kernel<<<dim3((unsigned)((T + 3) / 4)), 256, 0, as_stream(stream)>>>(
      (const U4 *)x, dest, T, k, H / 8, (U4 *)x_perm);
  return check_launch("permute");
}

extern "C" int art_moe_combine(const void *y_perm, const int32_t *dest, const float *wgt,
                               const float *dl, const int32_t *idx, const void *w_r,
                               const void *addend, int64_t T, int32_t k, int32_t H, void *y,
                               void *stream) {
  clear_error();
  ART_REQUIRE(T >= 0 && k >= 1 && k <= kMaxSlots && H > 0 && H % 8 == 0,
              "combine: need H %% 8 == 0 and 1 <= k <= 1024 (H=%d k=%d)", H, k);
  ART_REQUIRE(!w_r || k <= kMaxK, "combine: the router-gradient term needs k <= 32 (k=%d)", k);
  if (T == 0) return ART_MOE_OK;
  ART_REQUIRE(y_perm && dest && y && (!w_r || (dl && idx)), "combine: null pointer");
  const int n_chunks = (H / 8 + kWave - 1) / kWave;
  const int64_t blocks = (T * n_chunks + 3) / 4;
  ART_REQUIRE(blocks < ((int64_t)1 << 31), "combine: T * H too large (T=%lld H=%d)", (long long)T, H);
  combine_kernel<<<dim3((unsigned)blocks), 256, 0, as_stream(stream)>>>(
      (const U4 *)y_perm, dest, wgt, dl, idx, (const U4 *)w_r, (const U4 *)addend, T, k, H / 8,
      n_chunks, (U4 *)y);
  return check_launch("combine");
}

extern "C" int art_moe_router_lora_apply(const float *t_r, int64_t T, int32_t r, const void *b,
                                         int32_t E, float scale, float *logits, void *t_bf16,
                                         void *stream) {
  clear_error();
  ART_REQUIRE(T >= 0 && r >= 1 && E >= 1, "router_lora_apply: need T >= 0, r >= 1, E >= 1");
  if (T == 0) return ART_MOE_OK;
  ART_REQUIRE(t_r && b && logits, "router_lora_apply: null pointer");
  ART_REQUIRE(r <= kLoraMaxRank, "router_lora_apply: rank must be <= %d (r=%d)", kLoraMaxRank, r);
  const size_t lds = (size_t)(kLoraTrRow + kLoraCols) * ((r + 3) & ~3) * sizeof(float);
  router_lora_apply_kernel<<<dim3((unsigned)((T + kLoraTileTokens - 1) / kLoraTileTokens)), 256, lds,
                             as_stream(stream)>>>(t_r, T, r, (const bf16 *)b, E, scale, logits,
                                                  (bf16 *)t_bf16);
  return check_launch("router_lora_apply");
}

extern "C" int art_moe_router_lora_grad(const float *dl, const int32_t *idx, int64_t T, int32_t k,
                                        const void *b, int32_t r, int32_t E, float scale, void *g,
                                        void *dlog, void *stream) {
  clear_error();
  ART_REQUIRE(T >= 0 && k >= 1 && k <= kMaxK && r >= 1 && E >= 1,
              "router_lora_grad: need 1 <= k <= 32, r >= 1, E >= 1 (k=%d r=%d E=%d)", k, r, E);
  ART_REQUIRE((int64_t)(r + 2) * E <= 65536,
              "router_lora_grad: (r + 2) * E must be <= 65536 (r=%d E=%d)", r, E);
  if (T == 0) return ART_MOE_OK;
  ART_REQUIRE(dl && idx && b && g && dlog, "router_lora_grad: null pointer");
  const size_t lds = (size_t)(r + 2) * E * sizeof(bf16);
  router_lora_grad_kernel<<<dim3((unsigned)((T + kLoraGradTokens - 1) / kLoraGradTokens)), 256, lds,
                            as_stream(stream)>>>(dl, idx, T, k, (const bf16 *)b, r, E, scale,
                                                 (bf16 *)g, (bf16 *)dlog);
  return check_launch("router_lora_grad");
}

extern "C" int art_moe_transpose(const void *src, int32_t E, int32_t R, int32_t C, int64_t s_es,
                                 int64_t s_ld, void *dst, int64_t d_es, int64_t d_ld, float scale,
                                 void *stream) {
  clear_error();
  ART_REQUIRE(E >= 0 && R >= 0 && C >= 0, "transpose: negative size");
  if (E == 0 || R == 0 || C == 0) return ART_MOE_OK;
  ART_REQUIRE(src && dst, "transpose: null pointer");
  ART_REQUIRE(E <= 65535, "transpose: E too large");
  const dim3 grid((unsigned)((C + 31) / 32), (unsigned)((R + 31) / 32), (unsigned)E);
  transpose_kernel<<<grid, 256, 0, as_stream(stream)>>>((const bf16 *)src, R, C, s_es, s_ld,
                                                        (bf16 *)dst, d_es, d_ld, scale);
  return check_launch("transpose");
}

extern "C" int art_moe_pack(const art_moe_pack_desc *descs, int32_t n, void *stream) {
  return art_moe_pack_typed(descs, n, 0, stream);
}

extern "C" int art_moe_pack_typed(const art_moe_pack_desc *descs, int32_t n, int32_t f16,
                                  void *stream) {
  clear_error();
  ART_REQUIRE(n >= 0 && n <= ART_MOE_PACK_MAX, "pack: need 0 <= n <= %d (n=%d)", ART_MOE_PACK_MAX, n);
  if (n == 0) return ART_MOE_OK;
  ART_REQUIRE(descs, "pack: null descriptor array");
  PackArgs a{};
  a.n = n;
  a.tile_start[0] = 0;
  int64_t tiles = 0;
  for (int k = 0; k < n; ++k) {
    const art_moe_pack_desc &d = descs[k];
    ART_REQUIRE(d.E >= 0 && d.R >= 0 && d.C >= 0 && d.src_r >= 0 && d.src_c >= 0,
                "pack: negative extent in descriptor %d", k);
    ART_REQUIRE(d.dst || (int64_t)d.E * d.R * d.C == 0, "pack: null destination in descriptor %d", k);
    ART_REQUIRE(d.src || d.src_r == 0 || d.src_c == 0 || (int64_t)d.E * d.R * d.C == 0,
                "pack: null source in descriptor %d", k);
    a.d[k] = d;
    const int tcl = pack_tc_log2(d.R, d.C);
    const int TC = 1 << tcl, TR = kPackTile >> tcl;
    a.tc_log2[k] = tcl;
    const bool cfast = d.s_cs == 1;
    const int64_t slow_stride = cfast ? d.s_rs : d.s_cs;
    a.vec_read[k] = ((cfast || d.s_rs == 1) && ((uintptr_t)d.src & 15) == 0 && d.s_es % 8 == 0 &&
                     slow_stride % 8 == 0) ? 1 : 0;
    a.vec_write[k] = (((uintptr_t)d.dst & 15) == 0 && d.d_es % 8 == 0 && d.d_rs % 8 == 0) ? 1 : 0;
    tiles += (int64_t)d.E * ((d.R + TR - 1) / TR) * ((d.C + TC - 1) / TC);
    ART_REQUIRE(tiles < (int64_t)1 << 31, "pack: too many tiles");
    a.tile_start[k + 1] = (int32_t)tiles;
  }
  if (tiles == 0) return ART_MOE_OK;
  if (f16) pack_kernel<true><<<dim3((unsigned)tiles), 256, 0, as_stream(stream)>>>(a);
  else pack_kernel<false><<<dim3((unsigned)tiles), 256, 0, as_stream(stream)>>>(a);
  return check_launch("pack");
}
