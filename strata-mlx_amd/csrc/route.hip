// The router and the MoE block's end: the router's product in float32, its top-k with the routing weights, the
// combine of the experts' outputs with the shared expert, and the prompt's pairs laid out in tiles of one expert.
#include <type_traits>

#include "decode.h"
#include "launch.h"
#include "xmv.h"

namespace sh {

// ---- router product: W (E x d, fp16 or bf16) times a window of T <= 8 tokens, float32 sums
// (strata_mlx/fused.py:334-390). One wave a row; each token's sum taken in the same order whatever the window.
template <typename WT, typename XT>
__global__ __launch_bounds__(256) void k_router_matvec(const WT* __restrict__ w, const XT* __restrict__ x, int T,
                                                       float* __restrict__ out, int rows, int cols) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const WT* row = w + (int64_t)r * cols;
  float acc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) acc[t] = 0.0f;
  for (int c = lane; c < cols; c += 64) {
    float wv = to_f32(row[c]);
#pragma unroll
    for (int t = 0; t < 8; ++t)
      if (t < T) acc[t] = fmaf(wv, to_f32(x[(int64_t)t * cols + c]), acc[t]);
  }
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    if (t < T) {
      float v = acc[t];
      for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
      if (lane == 0) out[(int64_t)t * rows + r] = v;
    }
  }
}

// ---- top-k: the indices of the k largest logits of a row, largest first, ties to the lower index
// (strata_mlx/fused.py:400-418), and optionally the softmax of the chosen logits (fused.py:491).
//
// One wave a row. A logit and its index make one 64-bit key that orders as (value, -index): the largest key is the
// largest value and, among equal values, the lowest index (-0 and +0 equal, as the reference's float comparisons
// have them). The wave's largest key is found on DPP (xmv.h).
__device__ __forceinline__ uint64_t topk_key(float v, int i) {
  uint32_t u = __float_as_uint(v);
  u = u == 0x80000000u ? 0u : u;                     // -0 as +0
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);  // float order as unsigned order
  return ((uint64_t)u << 32) | (uint32_t)(0x7fffffff - i);
}
__device__ __forceinline__ float key_value(uint64_t k) {
  uint32_t u = (uint32_t)(k >> 32);
  u = (u & 0x80000000u) ? (u & 0x7fffffffu) : ~u;
  return __uint_as_float(u);
}
__device__ __forceinline__ int key_index(uint64_t k) { return 0x7fffffff - (int)(uint32_t)k; }

template <typename LT, int VPL>
__global__ __launch_bounds__(256) void k_top_k(const LT* __restrict__ logits, int rows, int n, int k,
                                               int32_t* __restrict__ idx, float* __restrict__ weights) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const LT* l = logits + (int64_t)row * n;
  uint64_t key[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    int j = i * 64 + lane;
    key[i] = j < n ? topk_key(to_f32(l[j]), j) : 0;  // 0: below every real key
  }
  float top = 0.0f, sum = 0.0f, chosen[VPL];  // chosen[r / 64] at lane r % 64: exp of the r-th largest
#pragma unroll
  for (int i = 0; i < VPL; ++i) chosen[i] = 0.0f;
  for (int r = 0; r < k; ++r) {
    uint64_t best = 0;
#pragma unroll
    for (int i = 0; i < VPL; ++i) best = key[i] > best ? key[i] : best;
    best = wave_max_u64(best);
    int who = key_index(best);
    float v = key_value(best);
    if (r == 0) top = v;
    float e = expf(v - top);
    sum += e;
#pragma unroll
    for (int i = 0; i < VPL; ++i)
      if (r == i * 64 + lane) chosen[i] = e;
    if (lane == 0) idx[(int64_t)row * k + r] = who;
#pragma unroll
    for (int i = 0; i < VPL; ++i)
      if (i * 64 + lane == who) key[i] = 0;
  }
  if (weights) {
#pragma unroll
    for (int i = 0; i < VPL; ++i)
      if (i * 64 + lane < k) weights[(int64_t)row * k + i * 64 + lane] = chosen[i] / sum;
  }
}

// ---- the end of the MoE block (strata_mlx/fused.py:448-481):
// out = OutT(sum_k y_k w_k) + OutT(OutT(sigmoid(g)) * s), the experts added as 8 rows j taking k = j, j + 8, ...
// then the rows in order, every product rounded before it is added.
template <typename XT>
__global__ __launch_bounds__(256) void k_moe_combine(const XT* __restrict__ y, const float* __restrict__ w,
                                                     const XT* __restrict__ g, const XT* __restrict__ s,
                                                     XT* __restrict__ out, int K, int D) {
#pragma clang fp contract(off)
  const int i = blockIdx.x * 256 + threadIdx.x;
  const int t = blockIdx.y;
  if (i >= D) return;
  float acc = 0.0f;
  for (int j = 0; j < 8 && j < K; ++j) {
    float part = 0.0f;
    for (int kk = j; kk < K; kk += 8) {
      float prod = to_f32(y[((int64_t)t * K + kk) * D + i]) * w[(int64_t)t * K + kk];
      part = prod + part;
    }
    acc = j == 0 ? part : part + acc;
  }
  XT routed = from_f32<XT>(acc);
  XT gate = from_f32<XT>(1.0f / (1.0f + expf(-to_f32(g[t]))));
  XT shared = from_f32<XT>(to_f32(gate) * to_f32(s[(int64_t)t * D + i]));
  out[(int64_t)t * D + i] = from_f32<XT>(to_f32(routed) + to_f32(shared));
}

// ---- tiles_of (strata_mlx/blocks.py:539-563): the pairs of a prompt chunk in tiles of 16 slots, each tile one
// expert's; pairs of an expert keep their order. Two kernels: the count of each expert, then the placement.
constexpr int TOKENS_TILE = 16;

__global__ __launch_bounds__(1024) void k_tile_counts(const int32_t* __restrict__ flat, int pairs, int experts,
                                                      int32_t* __restrict__ counts) {
  extern __shared__ int32_t c[];
  for (int e = threadIdx.x; e < experts; e += 1024) c[e] = 0;
  __syncthreads();
  for (int p0 = threadIdx.x; p0 < pairs; p0 += 8 * 1024) {  // eight loads in flight a thread
    int v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = p0 + 1024 * i < pairs ? flat[p0 + 1024 * i] : -1;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (v[i] >= 0 && v[i] < experts) atomicAdd(&c[v[i]], 1);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < experts; e += 1024) counts[e] = c[e];
}

// One block an expert (and one more for the tiles no pair fills), 16 waves. The pairs go by in batches of
// 16 x 1024: wave w scans its run of 1024 consecutive pairs of the batch, 16 a lane, once into bit masks of the
// pairs that are this expert's; their counts, summed over the earlier waves, place each wave's run; the masks'
// ballots rank the pairs within it. Pairs of the expert keep their order.
constexpr int PLACE_NT = 1024, PLACE_PER = 16;

__device__ __forceinline__ int place_block_sum(int v, int32_t* s_w) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d);
  if (lane == 0) s_w[wv] = v;
  __syncthreads();
  int total = 0;
#pragma unroll
  for (int w = 0; w < PLACE_NT / 64; ++w) total += s_w[w];
  __syncthreads();
  return total;
}

__global__ __launch_bounds__(PLACE_NT) void k_tile_place(const int32_t* __restrict__ flat, int pairs, int k,
                                                         int experts, const int32_t* __restrict__ counts, int most,
                                                         int32_t* __restrict__ tile_expert,
                                                         int32_t* __restrict__ token, int32_t* __restrict__ where) {
  __shared__ int32_t s_w[PLACE_NT / 64];
  const int e = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const uint64_t below = (1ull << lane) - 1ull;
  // tiles of the experts before this one, and all tiles (the tail block needs the total)
  int before = 0, all = 0;
  for (int j = tid; j < experts; j += PLACE_NT) {
    const int t = (counts[j] + TOKENS_TILE - 1) / TOKENS_TILE;
    all += t;
    if (j < e) before += t;
  }
  before = place_block_sum(before, s_w);
  all = place_block_sum(all, s_w);
  if (e == experts) {  // the tiles no pair fills: no expert, token 0
    for (int t = all + tid; t < most; t += PLACE_NT) {
      tile_expert[t] = experts;
      for (int j = 0; j < TOKENS_TILE; ++j) token[t * TOKENS_TILE + j] = 0;
    }
    return;
  }
  const int count = counts[e], tiles = (count + TOKENS_TILE - 1) / TOKENS_TILE;
  for (int t = tid; t < tiles; t += PLACE_NT) tile_expert[before + t] = e;
  for (int j = count + tid; j < tiles * TOKENS_TILE; j += PLACE_NT) token[before * TOKENS_TILE + j] = 0;
  constexpr int RUN = 64 * PLACE_PER, BATCH = RUN * (PLACE_NT / 64);
  int seen = 0;
  for (int b0 = 0; b0 < pairs; b0 += BATCH) {
    const int p0 = b0 + wv * RUN + lane;  // the lane's pair of slot i: p0 + 64 i
    int v[PLACE_PER];
#pragma unroll
    for (int i = 0; i < PLACE_PER; ++i) v[i] = p0 + 64 * i < pairs ? flat[p0 + 64 * i] : -1;
    uint32_t bits = 0;
    int n = 0;
#pragma unroll
    for (int i = 0; i < PLACE_PER; ++i) {
      const bool mine = v[i] == e;
      bits |= (uint32_t)mine << i;
      n += __popcll(__ballot(mine));
    }
    if (lane == 0) s_w[wv] = n;
    __syncthreads();
    int off = seen, total = 0;
#pragma unroll
    for (int w = 0; w < PLACE_NT / 64; ++w) {
      const int c = s_w[w];
      off += w < wv ? c : 0;
      total += c;
    }
    __syncthreads();  // s_w is read by all before the next batch writes it
    int run = before * TOKENS_TILE + off;
#pragma unroll
    for (int i = 0; i < PLACE_PER; ++i) {
      const bool mine = (bits >> i) & 1u;
      const uint64_t m = __ballot(mine);
      if (mine) {
        const int p = p0 + 64 * i, slot = run + __popcll(m & below);
        token[slot] = p / k;
        where[p] = slot;
      }
      run += __popcll(m);
    }
    seen += total;
  }
}

}  // namespace sh

using namespace sh;

extern "C" {

int sh_router_matvec(const void* w, int w_dtype, int64_t rows, int64_t cols, const void* x, int x_dtype,
                     int64_t tokens, float* out, void* stream) {
  if (tokens <= 0 || rows <= 0) return OK;
  if (tokens > 8) return fail(E_SHAPE, "router_matvec: %lld tokens (a window is at most 8)", (long long)tokens);
  if (cols <= 0 || cols > (1 << 24)) return fail(E_SHAPE, "router_matvec: %lld columns", (long long)cols);
  if (!w || !x || !out) return fail(E_ARG, "router_matvec: null pointer");
  return with_half_dtype(w_dtype, [&](auto* wp) {
    using WT = std::remove_pointer_t<decltype(wp)>;
    return with_dtype(x_dtype, [&](auto* xp) {
      using XT = std::remove_pointer_t<decltype(xp)>;
      hipLaunchKernelGGL((k_router_matvec<WT, XT>), dim3((unsigned)((rows + 3) / 4)), dim3(256), 0,
                         (hipStream_t)stream, (const WT*)w, (const XT*)x, (int)tokens, out, (int)rows, (int)cols);
      return check_launch("router_matvec");
    });
  });
}

int sh_top_k(const void* logits, int dtype, int64_t rows, int64_t n, int64_t k, int32_t* idx, float* weights,
             void* stream) {
  if (rows <= 0) return OK;
  if (n <= 0 || n > 2048) return fail(E_SHAPE, "top_k: rows of %lld logits (at most 2048)", (long long)n);
  if (k <= 0 || k > n) return fail(E_SHAPE, "top_k: k = %lld of %lld", (long long)k, (long long)n);
  if (!logits || !idx) return fail(E_ARG, "top_k: null pointer");
  int vpl = (int)((n + 63) / 64);
  vpl = vpl <= 1 ? 1 : vpl <= 2 ? 2 : vpl <= 4 ? 4 : vpl <= 8 ? 8 : vpl <= 16 ? 16 : 32;
  return with_dtype(dtype, [&](auto* lp) {
    using LT = std::remove_pointer_t<decltype(lp)>;
    dim3 grid((unsigned)((rows + 3) / 4));
    auto go = [&](auto v) {
      constexpr int V = decltype(v)::value;
      hipLaunchKernelGGL((k_top_k<LT, V>), grid, dim3(256), 0, (hipStream_t)stream, (const LT*)logits, (int)rows,
                         (int)n, (int)k, idx, weights);
      return check_launch("top_k");
    };
    switch (vpl) {
      case 1: return go(kind_c<1>{});
      case 2: return go(kind_c<2>{});
      case 4: return go(kind_c<4>{});
      case 8: return go(kind_c<8>{});
      case 16: return go(kind_c<16>{});
      default: return go(kind_c<32>{});
    }
  });
}

int sh_moe_combine(const void* y, const float* w, const void* g, const void* s, int dtype, int64_t tokens, int64_t k,
                   int64_t d, void* out, void* stream) {
  if (tokens <= 0) return OK;
  if (tokens > 65535 || k <= 0 || d <= 0) return fail(E_SHAPE, "moe_combine: shape (%lld, %lld, %lld)",
                                                     (long long)tokens, (long long)k, (long long)d);
  if (!y || !w || !g || !s || !out) return fail(E_ARG, "moe_combine: null pointer");
  return with_dtype(dtype, [&](auto* tp) {
    using XT = std::remove_pointer_t<decltype(tp)>;
    dim3 grid((unsigned)((d + 255) / 256), (unsigned)tokens);
    hipLaunchKernelGGL((k_moe_combine<XT>), grid, dim3(256), 0, (hipStream_t)stream, (const XT*)y, w, (const XT*)g,
                       (const XT*)s, (XT*)out, (int)k, (int)d);
    return check_launch("moe_combine");
  });
}

// workspace: experts int32 counts
size_t sh_tiles_workspace(int64_t experts) { return (size_t)(experts > 0 ? experts : 0) * 4; }

int64_t sh_tiles_most(int64_t pairs, int64_t experts) {
  return pairs / TOKENS_TILE + (experts < pairs ? experts : pairs);
}

int sh_tiles_of(const int32_t* flat, int64_t pairs, int64_t k, int64_t experts, int32_t* tile_expert, int32_t* token,
                int32_t* where, void* workspace, size_t workspace_bytes, void* stream) {
  if (pairs <= 0) return OK;
  if (k <= 0 || pairs % k) return fail(E_SHAPE, "tiles_of: %lld pairs in rows of %lld", (long long)pairs, (long long)k);
  if (experts <= 0 || experts > 16384) return fail(E_SHAPE, "tiles_of: %lld experts (at most 16384)", (long long)experts);
  if (pairs > (1 << 26)) return fail(E_SHAPE, "tiles_of: %lld pairs", (long long)pairs);
  if (!flat || !tile_expert || !token || !where) return fail(E_ARG, "tiles_of: null pointer");
  if (!workspace || workspace_bytes < sh_tiles_workspace(experts))
    return fail(E_WORKSPACE, "tiles_of: workspace of %zu bytes, %zu needed", workspace_bytes, sh_tiles_workspace(experts));
  int64_t most = sh_tiles_most(pairs, experts);
  int32_t* counts = (int32_t*)workspace;
  hipLaunchKernelGGL(k_tile_counts, dim3(1), dim3(1024), (size_t)experts * 4, (hipStream_t)stream, flat, (int)pairs,
                     (int)experts, counts);
  int st = check_launch("tiles_of");
  if (st) return st;
  hipLaunchKernelGGL(k_tile_place, dim3((unsigned)experts + 1), dim3(PLACE_NT), 0, (hipStream_t)stream, flat, (int)pairs,
                     (int)k, (int)experts, counts, (int)most, tile_expert, token, where);
  return check_launch("tiles_of");
}

}  // extern "C"
