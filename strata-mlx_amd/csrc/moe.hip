// One MoE block's decode step for a window of B <= 16 tokens, in three kernels — the path of strata-mlx's
// `_Routed.__call__` (strata_mlx/fused.py:484-497) with its routed experts through switch_glu's bf16 branch
// (strata_mlx/blocks.py:819-829) and its end in `moe_combine` (fused.py:448-481):
//
//   route     one block: each token's top-k of the router logits (largest first, ties to the lower index), the
//             softmax of the chosen logits, the shared expert's gate logit x . w_g, the (token, expert) pairs grouped
//             by expert (first occurrence order; the shared expert one more group of all B tokens), and the hidden
//             states written in the layout gate/up's decode reads
//   gate_up   a block = 16 rows of gate and of up of one group's expert, for the group's tokens; the epilogue rounds
//             gate and up to the activation type, takes swiglu with mlx-lm's roundings and writes it in the layout
//             down's decode reads
//   down      a block = 16 rows of down of every group, chunks of groups double-buffered in LDS, a wave a group; each
//             pair's outputs rounded to the activation type stay in LDS for the combine:
//             OutT(sum_k y_k w_k) + OutT(OutT(sigmoid(g)) * s)
//
// Only weights go through LDS: the activations each kernel multiplies were written by the kernel before in the
// order its MFMA fragments take them, and are read straight from memory (L2). Grids are sized by the most groups
// there could be (B*k + 1); blocks past the groups the route found leave at once, so nothing waits on the host.
#include <atomic>
#include <cassert>
#include <mutex>

#include "launch.h"
#include "regmac.h"
#include "xmv.h"

namespace sh {

constexpr int MOE_MAX_TOKENS = 16;
constexpr int MOE_MAX_PAIRS = 160;  // tokens * k
constexpr int MOE_MAX_D = 8192;     // d_model

// experts a multiple of 64 whose count of 64s is a power of two up to 32 (the route's keys a lane holds)
inline bool vpl_bad(int64_t experts) {
  const int64_t v = experts / 64;
  return experts % 64 || v < 1 || v > 32 || (v & (v - 1));
}

// the workspace, carved from one caller buffer: the control words first, at the same offsets whatever the shape
// (the one-launch layer needs them at zero when it starts, and its last block leaves them at zero, so a workspace
// used for several shapes in turn keeps them), then the shape's arrays
struct MoeWs {
  int32_t* n_groups;  // [1]
  int32_t* g_expert;  // [G]: expert, or `experts` for the shared expert
  int32_t* g_ntok;    // [G]
  int32_t* g_pair;    // [G][16]: pair t*k + j, or B*k + t for the shared expert's token t
  int32_t* idx;       // [B][k]
  float* w;           // [B][k]
  float* gsh;         // [B]: the shared expert's gate logit, rounded to the activation type
  uint8_t* xp;        // [B][D]: the hidden states staged for gate/up's kind (xmv.h stage_index)
  uint8_t* h;         // [B*k + B][F]: swiglu(gate, up), staged for down's kind (natural order in the two-kernel path)
  float* y;           // [B*k + B][D]: each pair's down outputs, rounded to the activation type (the common shape)
  // counters, each in a 256-byte line of its own (CTR_STRIDE words apart): agent-scope atomics on one line are
  // done one after another, about 10 ns each, so hundreds of blocks counting on one line would wait microseconds.
  // The one-launch layer's come in two sets, used by calls in turn: `par` names the set a call uses, and the call's
  // last block to draw a ticket clears the other set for the next call and switches `par` to it.
  int32_t* cnt;       // [D / 64]: the tail's finished items a row tile when it combines, zero between calls
  int32_t* par;       // [1]: one-launch layer: the set of counters the next call uses (0 or 1)
  int32_t* ticket;    // [1]: one-launch layer: tickets drawn, zero between calls
  int32_t* gdone;     // [2][G]: one-launch layer: gate / up items done a group
  int32_t* gall;      // [2]: one-launch layer: groups complete
  int32_t* gflag;     // [2][8]: one-launch layer: every group complete (eight copies: the down blocks poll by eighths)
  int32_t* err;       // [1]: set (and left set) if a wait gave up or the counters were not at zero
};
constexpr int MOE_CNT_WORDS = MOE_MAX_D / 64 + 1;
constexpr int CTR_STRIDE = 64;

constexpr size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }
// the control words' bytes at the head of every workspace
constexpr size_t MOE_HEAD_BYTES = align256(4 * CTR_STRIDE * MOE_CNT_WORDS) + 2 * 256 +
                                  align256(4 * CTR_STRIDE * 2 * (MOE_MAX_PAIRS + 1)) + align256(4 * CTR_STRIDE * 2) +
                                  align256(4 * CTR_STRIDE * 2 * 8) + 256;

static size_t moe_carve(MoeWs* ws, uint8_t* base, int64_t B, int64_t k, int64_t D, int64_t F, int es) {
  const int64_t G = B * k + 1, P = B * k + B;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    uint8_t* p = base ? base + off : nullptr;
    off = align256(off + bytes);
    return p;
  };
  MoeWs w;
  w.cnt = (int32_t*)take((size_t)4 * CTR_STRIDE * MOE_CNT_WORDS);
  w.par = (int32_t*)take(4);
  w.ticket = (int32_t*)take(4);
  w.gdone = (int32_t*)take((size_t)4 * CTR_STRIDE * 2 * (MOE_MAX_PAIRS + 1));
  w.gall = (int32_t*)take((size_t)4 * CTR_STRIDE * 2);
  w.gflag = (int32_t*)take((size_t)4 * CTR_STRIDE * 2 * 8);
  w.err = (int32_t*)take(4);
  assert(off == MOE_HEAD_BYTES);
  w.n_groups = (int32_t*)take(4);
  w.g_expert = (int32_t*)take(4 * G);
  w.g_ntok = (int32_t*)take(4 * G);
  w.g_pair = (int32_t*)take(4 * 16 * G);
  w.idx = (int32_t*)take(4 * B * k);
  w.w = (float*)take(4 * B * k);
  w.gsh = (float*)take(4 * B);
  w.xp = take((size_t)B * D * es);
  w.h = take((size_t)P * F * es);
  w.y = (float*)take((size_t)P * D * 4);
  if (ws) *ws = w;
  return off;
}

// ---- route

// Route keys: a logit in an order-preserving unsigned form above the complement of its index, so the largest key
// is the largest logit and, among equal logits, the lowest index (-0 taken as +0: equal, as float comparisons have
// them). 16-bit logits make 32-bit keys; float32 64-bit.
template <typename LT> struct RouteKey {
  using type = uint32_t;
  __device__ static __forceinline__ uint32_t make(LT v, int i) {
    uint32_t b = __builtin_bit_cast(uint16_t, v);
    b = b == 0x8000u ? 0u : b;
    b = (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
    return (b << 16) | (0xffffu - (uint32_t)i);
  }
  __device__ static __forceinline__ int index(uint32_t k) { return 0xffff - (int)(k & 0xffffu); }
  __device__ static __forceinline__ float value(uint32_t k) {
    const uint32_t o = k >> 16;
    return to_f32(__builtin_bit_cast(LT, (uint16_t)((o & 0x8000u) ? (o & 0x7fffu) : (~o & 0xffffu))));
  }
  __device__ static __forceinline__ uint32_t wave_max(uint32_t k) { return wave_max_u32(k); }
};
template <> struct RouteKey<float> {
  using type = uint64_t;
  __device__ static __forceinline__ uint64_t make(float v, int i) {
    uint32_t b = __float_as_uint(v);
    b = b == 0x80000000u ? 0u : b;
    b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)b << 32) | (0xffffffffu - (uint32_t)i);
  }
  __device__ static __forceinline__ int index(uint64_t k) { return (int)(0xffffffffu - (uint32_t)k); }
  __device__ static __forceinline__ float value(uint64_t k) {
    const uint32_t o = (uint32_t)(k >> 32);
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
  }
  __device__ static __forceinline__ uint64_t wave_max(uint64_t k) { return wave_max_u64(k); }
};

// One token's top-k by selection instead of k rounds of arg-max: the k-th largest value found bit by bit from the
// top over the value half of the keys (a candidate stays if at least k keys are at or above it: a ballot and a
// popcount a slot and bit); the keys above that value, and of the keys equal to it the lowest indices, as many as
// k still wants; then the k chosen ranked among themselves. Key slot i of lane l is index i * 64 + l; keys are
// unique, the larger chosen first (RouteKey: the value above the index's complement). Leaves the chosen keys in
// descending order in sorted[0, k) (LDS, the wave's own; scratch the same size).
template <typename RK, int VPL>
__device__ __forceinline__ void select_k(const typename RK::type (&key)[VPL], int K, typename RK::type* scratch,
                                         typename RK::type* sorted) {
  using key_t = typename RK::type;
  constexpr int BITS = 8 * (int)sizeof(key_t), IBITS = BITS / 2;  // the low half holds the index
  const int lane = threadIdx.x & 63;
  const uint64_t below = (1ull << lane) - 1ull;
  auto count_ge = [&](key_t c) {
    int n = 0;
#pragma unroll
    for (int i = 0; i < VPL; ++i) n += __popcll(__ballot(key[i] >= c));
    return n;
  };
  key_t lo = 0;  // the k-th largest value, its index half zero
  for (int bit = BITS - 1; bit >= IBITS; --bit) {
    const key_t cand = lo | ((key_t)1 << bit);
    if (count_ge(cand) >= K) lo = cand;
  }
  const key_t hi = lo + ((key_t)1 << IBITS);  // keys at or above: a larger value (hi wraps to 0 only for the
  int need = K - (hi ? count_ge(hi) : 0);     // largest value, which nothing exceeds)
  int base = 0;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {  // index order: slot i, then lane
    const bool above = hi && key[i] >= hi;
    const bool equal = key[i] >= lo && !above;
    const uint64_t me = __ballot(equal);
    const bool sel = above || (equal && __popcll(me & below) < need);
    need -= min(need, __popcll(me));
    const uint64_t m = __ballot(sel);
    if (sel) scratch[base + __popcll(m & below)] = key[i];
    base += __popcll(m);
  }
  __builtin_amdgcn_wave_barrier();
  if (lane < K) {
    const key_t mine = scratch[lane];
    int rank = 0;
    for (int j = 0; j < K; ++j) rank += scratch[j] > mine;
    sorted[rank] = mine;
  }
  __builtin_amdgcn_wave_barrier();
}

// select_k over the wave's VPL keys a lane, narrowed first: the k-th largest value among the lanes' maxima bounds
// the k-th largest key from below (those k maxima are k keys at or above it), so only the keys at or above that
// value can be chosen; when at most 64 are, they go one a lane (in index order) and select_k runs on one slot.
// cand: LDS, 64 keys, the wave's own.
template <typename RK, int VPL>
__device__ __forceinline__ void wave_top_k(const typename RK::type (&key)[VPL], int K, typename RK::type* cand,
                                           typename RK::type* scratch, typename RK::type* sorted) {
  using key_t = typename RK::type;
  constexpr int BITS = 8 * (int)sizeof(key_t), IBITS = BITS / 2;
  const int lane = threadIdx.x & 63;
  const uint64_t below = (1ull << lane) - 1ull;
  key_t mx = key[0];
#pragma unroll
  for (int i = 1; i < VPL; ++i) mx = key[i] > mx ? key[i] : mx;
  key_t lo = 0;
  for (int bit = BITS - 1; bit >= IBITS; --bit) {
    const key_t c = lo | ((key_t)1 << bit);
    if (__popcll(__ballot(mx >= c)) >= K) lo = c;
  }
  int n = 0;
  uint64_t sel[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    sel[i] = __ballot(key[i] >= lo);
    n += __popcll(sel[i]);
  }
  if (n > 64) {  // many keys tied at the bound: the whole set
    select_k<RK, VPL>(key, K, scratch, sorted);
    return;
  }
  int base = 0;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    if (key[i] >= lo) cand[base + __popcll(sel[i] & below)] = key[i];
    base += __popcll(sel[i]);
  }
  __builtin_amdgcn_wave_barrier();
  const key_t one[1] = {lane < n ? cand[lane] : (key_t)0};  // key 0 is no real key and is never chosen (n >= k)
  select_k<RK, 1>(one, K, scratch, sorted);
}

template <int KIND, typename XT, typename LT, int VPL>
__global__ __launch_bounds__(256) void k_moe_route(const LT* __restrict__ logits, const XT* __restrict__ x,
                                                   const XT* __restrict__ wg, int B, int E, int K, int D, MoeWs ws) {
  using RK = RouteKey<LT>;
  using key_t = typename RK::type;
  __shared__ int s_idx[MOE_MAX_PAIRS];
  __shared__ int s_first[MOE_MAX_PAIRS], s_gid[MOE_MAX_PAIRS], s_rank[MOE_MAX_PAIRS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  for (int t = wave; t < B; t += 4) {
    // every load of the token first: its logits, its hidden state and the shared gate's weights (16-byte vectors)
    key_t key[VPL];
#pragma unroll
    for (int i = 0; i < VPL; ++i) key[i] = RK::make(logits[(int64_t)t * E + i * 64 + lane], i * 64 + lane);
    u32x4 xv[MOE_MAX_D / 512], wv[MOE_MAX_D / 512];
#pragma unroll
    for (int j = 0; j < MOE_MAX_D / 512; ++j) {
      const int c8 = lane + 64 * j;
      if (c8 < D / 8) {
        xv[j] = *(const u32x4*)(x + (int64_t)t * D + 8 * c8);
        wv[j] = *(const u32x4*)(wg + 8 * c8);
      }
    }
    float top = 0.0f, sum = 0.0f, my_e = 0.0f;
    int my_idx = 0;
    for (int r = 0; r < K; ++r) {
      key_t best = key[0];
#pragma unroll
      for (int i = 1; i < VPL; ++i) best = key[i] > best ? key[i] : best;
      best = RK::wave_max(best);  // the same in every lane
      const int who = RK::index(best);
      const float v = RK::value(best);
      if (r == 0) top = v;
      const float e = expf(v - top);
      sum += e;
      if (lane == r) {
        my_e = e;
        my_idx = who;
        s_idx[t * K + r] = who;
      }
#pragma unroll
      for (int i = 0; i < VPL; ++i)
        if (key[i] == best) key[i] = 0;
    }
    if (lane < K) {
      ws.w[t * K + lane] = my_e / sum;
      ws.idx[t * K + lane] = my_idx;
    }
    // the shared expert's gate logit, rounded to the activation type (a Linear(d, 1) in mlx-lm); and the hidden
    // state in the order gate/up's MFMA fragments take it
    float acc = 0.0f;
    XT* xp = (XT*)ws.xp + (int64_t)t * D;
#pragma unroll
    for (int j = 0; j < MOE_MAX_D / 512; ++j) {
      const int c8 = lane + 64 * j;
      if (c8 < D / 8) {
        const XT* a = (const XT*)&xv[j];
        const XT* b = (const XT*)&wv[j];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          acc = fmaf(to_f32(a[e]), to_f32(b[e]), acc);
          float scale;
          const int at = stage_index<KIND, XT>(8 * c8 + e, scale);
          xp[at] = from_f32<XT>(to_f32(a[e]) * scale);
        }
      }
    }
    acc = wave_sum(acc);
    if (lane == 0) ws.gsh[t] = to_f32(from_f32<XT>(acc));
  }
  __syncthreads();

  // pairs grouped by expert, groups in order of first occurrence
  const int P = B * K;
  if (tid < P) {
    const int e = s_idx[tid];
    int first = tid, rank = 0;
    for (int q = 0; q < tid; ++q)
      if (s_idx[q] == e) {
        rank += 1;
        first = q < first ? q : first;
      }
    s_first[tid] = first;
    s_rank[tid] = rank;
  }
  __syncthreads();
  if (tid < P && s_first[tid] == tid) {
    int gid = 0;
    for (int q = 0; q < tid; ++q) gid += s_first[q] == q;
    s_gid[tid] = gid;
  }
  __syncthreads();
  if (tid < P) {
    const int gid = s_gid[s_first[tid]];
    ws.g_pair[gid * 16 + s_rank[tid]] = tid;
    if (s_rank[tid] == 0) {
      int count = 1;
      for (int q = tid + 1; q < P; ++q) count += s_first[q] == tid;
      ws.g_expert[gid] = s_idx[tid];
      ws.g_ntok[gid] = count;
    }
  }
  if (tid == 0) {
    int groups = 0;
    for (int q = 0; q < P; ++q) groups += s_first[q] == q;
    ws.g_expert[groups] = E;  // the shared expert: every token
    ws.g_ntok[groups] = B;
    for (int t = 0; t < B; ++t) ws.g_pair[groups * 16 + t] = P + t;
    *ws.n_groups = groups + 1;
  }
}

template <int KIND> constexpr int moe_tab_bytes() { return KIND == IQ3_S ? IQ3S_SIGNED_BYTES : 0; }

// ---- gate and up, SwiGLU in the epilogue

template <int KIND, int KIND_DOWN, typename XT, int TPG>
__global__ __launch_bounds__(256) void k_moe_gate_up(const uint8_t* __restrict__ gate, const uint8_t* __restrict__ up,
                                                     const uint8_t* __restrict__ sh_gate, const uint8_t* __restrict__ sh_up,
                                                     int E, int K, int B, int D, int F,
                                                     const uint8_t* __restrict__ signed_tab, MoeWs ws) {
  using MT = XT;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row0 = blockIdx.x * 16, gy = blockIdx.y;
  __shared__ int s_groups, s_n, s_e, s_pair[16];
  __shared__ float s_red[2][4][64][TPG];
  extern __shared__ u32x4 dyn[];
  uint8_t* tab = (uint8_t*)dyn;
  const int64_t rb = row_bytes_dev(KIND, D);
  uint8_t* wg = tab + moe_tab_bytes<KIND>();
  uint8_t* wu = wg + 16 * rb + 16;
  // the group, in one trip: every field read by a thread of its own (entries past the groups are unused)
  if (tid == 0) s_groups = *ws.n_groups;
  if (tid == 1) s_e = ws.g_expert[gy];
  if (tid == 2) s_n = ws.g_ntok[gy];
  if (tid >= 16 && tid < 32) s_pair[tid - 16] = ws.g_pair[gy * 16 + tid - 16];
  __syncthreads();
  if (gy >= s_groups) return;
  const int n_tok = s_n, e = s_e;
  const int64_t ebytes = (int64_t)F * rb;
  const uint8_t* g_src = (e == E ? sh_gate : gate + (int64_t)e * ebytes) + (int64_t)row0 * rb;
  const uint8_t* u_src = (e == E ? sh_up : up + (int64_t)e * ebytes) + (int64_t)row0 * rb;
  ByteStage<8> wst(wg, g_src, (int)(16 * rb), wu, u_src, (int)(16 * rb));
  for (int p = 0; p < wst.passes(256); ++p) {
    wst.load(p, tid, 256);
    wst.store(p, tid, 256);
  }
  if constexpr (KIND == IQ3_S) {
    ByteStage<8> tst(tab, signed_tab, IQ3S_SIGNED_BYTES, nullptr, nullptr, 0);
    for (int p = 0; p < tst.passes(256); ++p) {
      tst.load(p, tid, 256);
      tst.store(p, tid, 256);
    }
  }
  __syncthreads();
  // this wave's quarter of the columns, the A fragments straight from the staged hidden states
  const int mt = lane_token<TPG>();
  const bool real = mt < n_tok;
  const int p = s_pair[real ? mt : 0];
  const MT* xg = (const MT*)ws.xp + (int64_t)(p < B * K ? p / K : p - B * K) * D;
  float acc[2][TPG];
#pragma unroll
  for (int i = 0; i < TPG; ++i) acc[0][i] = acc[1][i] = 0.0f;
  const uint8_t* tiles[2] = {wg + lead_of(g_src), wu + lead_of(u_src)};
  // the row's scale groups split four ways, the parts differing by at most one group (a row of fewer than four
  // groups leaves some waves none)
  const int ng = D / scale_group<KIND>();
  tile_mac_global<KIND, MT, TPG, frag_chunk<KIND>(), 2>(tiles, (int)rb, xg, real, wave * ng / 4, (wave + 1) * ng / 4,
                                                         (const uint32_t*)tab, acc);
#pragma unroll
  for (int i = 0; i < TPG; ++i) {
    s_red[0][wave][lane][i] = acc[0][i];
    s_red[1][wave][lane][i] = acc[1][i];
  }
  __syncthreads();
  if (wave == 0) {
    const int g = lane >> 4, n = lane & 15;
    float scale;
    const int at = stage_index<KIND_DOWN, XT>(row0 + n, scale);
#pragma unroll
    for (int i = 0; i < TPG; ++i) {
      const int t = g * TPG + i;
      if (t < n_tok) {
        const XT gv = from_f32<XT>(s_red[0][0][lane][i] + s_red[0][1][lane][i] + s_red[0][2][lane][i] + s_red[0][3][lane][i]);
        const XT uv = from_f32<XT>(s_red[1][0][lane][i] + s_red[1][1][lane][i] + s_red[1][2][lane][i] + s_red[1][3][lane][i]);
        ((XT*)ws.h)[(int64_t)s_pair[t] * F + at] = from_f32<XT>(to_f32(swiglu_one(gv, uv)) * scale);
      }
    }
  }
}

// ---- the common shape (512 experts, d_model 2048, expert width 512): three kernels
//
// front    route, gate and up with SwiGLU. A block of 8 waves routes the whole window itself (a wave a token: its
//          top-k of the 512 logits), so no kernel boundary stands between the choice and the expert products, then
//          streams a run of the items (group g, row tile r: 16 rows of gate and 16 of up of the group's expert)
//          within one group. The groups are the chosen experts in ascending order, then the shared expert. Items
//          go through an LDS ring filled by direct loads, NBUF - 1 in flight while one is multiplied; wave q
//          multiplies the 16 rows of gate and of up over column eighth q with the group's activation fragments in
//          registers (loaded as they are: the Q2_0 decode shifts each code down itself). The epilogue rounds gate
//          and up to the activation type and writes swiglu(gate, up) per pair, in natural order. Block 0 also
//          writes the choice, its weights and the groups' experts; block 1 the shared expert's gate logits.
// tail     down. Its blocks stream runs of the items (group g, 64 rows of down of g's expert; wave (r, h) 16 rows
//          over column half h) within one group through an LDS ring as the front does, writing each pair's
//          outputs, rounded to the activation type, to the workspace.
// combine  a thread an output (token, row): the routed outputs weighted in the reference's order, the shared
//          expert gated.

constexpr int FRONT_E = 512, FRONT_D = 2048, FRONT_F = 512;
constexpr int FRONT_WAVES = 8;
constexpr int TAIL_COMBINE_UPTO = 4;  // tokens up to which the tail combines in-kernel
// the same bound as set at run time (sh_moe_set_tail_combine): 0 sends every window to the combine kernel
static std::atomic<int> g_tail_combine_upto{TAIL_COMBINE_UPTO};
// whether the common shape's step runs as one launch (sh_moe_set_one_launch). Off, and it cannot be switched on:
// the one-launch layer (k_moe_layer) made an illegal memory access at 2 tokens (Q2_0, float16). The cause found
// since (its direct loads read a base address that v_readfirstlane had just written, inside the hazard window that
// lds_dma16 now waits out) is fixed, but the fix has not run on a GPU: until it has, every window takes the two
// launches.
static std::atomic<int> g_one_launch{0};

// the pairs of group expert e in token order, into this wave's wp[0, n): pair t * K + j of each token t choosing e
// (a token chooses an expert at most once), or every token's shared pair P + t for the shared expert (e == E)
__device__ __forceinline__ int group_pairs(int e, int E, const int* s_idx, int B, int K, int* wp) {
  const int lane = threadIdx.x & 63;
  int n = 0;
  if (e < E) {  // the pairs in order (so by token): a lane a pair, three reads at once
    int hit[(MOE_MAX_PAIRS + 63) / 64];
#pragma unroll
    for (int c = 0; c < (MOE_MAX_PAIRS + 63) / 64; ++c) {
      const int p = c * 64 + lane;
      hit[c] = p < B * K && s_idx[p] == e;
    }
#pragma unroll
    for (int c = 0; c < (MOE_MAX_PAIRS + 63) / 64; ++c) {
      const uint64_t m = __ballot(hit[c]);
      if (hit[c]) wp[n + __popcll(m & ((1ull << lane) - 1ull))] = c * 64 + lane;
      n += __popcll(m);
    }
  } else {
    n = B;
    if (lane < B) wp[lane] = B * K + lane;
  }
  __builtin_amdgcn_wave_barrier();
  return n;
}

// block `bid` of `nblk`'s run of items: chunk c of group g's TILES items, chunks of `per` items, per the least that
// leaves a block for every chunk (at least one block a group). Returns false for a block past the chunks.
template <int TILES>
__device__ __forceinline__ bool group_chunk(int groups, int nblk, int bid, int& g, int& first, int& last) {
  int per = max(1, (groups * TILES + nblk - 1) / nblk);
  while (per < TILES && groups * ((TILES + per - 1) / per) > nblk) ++per;
  const int cpg = (TILES + per - 1) / per;
  g = bid / cpg;
  const int c = bid - g * cpg;
  first = g * TILES + c * per;
  last = g * TILES + min(TILES, (c + 1) * per);
  return g < groups;
}

// an item in LDS: 16 rows of gate then 16 of up at a padded stride, as 16-byte chunks; wave w loads the runs of 64
// chunks w, w + 8, ... (the last run's chunks past the item re-read its last chunk into the slot's tail)
template <int KIND> struct FrontItem {
  static constexpr int RB = (int)row_bytes_dev(KIND, FRONT_D);
  static constexpr int RSTRIDE = padded_stride(RB);
  static constexpr int CPR = RSTRIDE / 16, CPR_SRC = RB / 16;
  static constexpr int CHUNKS = 2 * 16 * CPR, RUNS = (CHUNKS + 63) / 64;
  static constexpr int SLOT = RUNS * 1024;
  static constexpr int LOADS = (RUNS + FRONT_WAVES - 1) / FRONT_WAVES;  // of the waves with the most
  static_assert(RB % 16 == 0 && RUNS >= FRONT_WAVES, "front item layout");
};

struct FrontPlan {
  int nbuf;      // ring slots
  int ring_off;  // after the IQ3_S table
  int red_off;   // [2][2][7][64][TPG] floats: gate's and up's partial sums of waves 1..7, the last two items
};

// ---- the route of a window, in every block that needs it

// the route's LDS: the chosen experts and weights of every pair, the flags of the chosen experts, selection scratch
template <typename LT> struct RouteLds {
  using key_t = typename RouteKey<LT>::type;
  int idx[MOE_MAX_PAIRS];
  float wt[MOE_MAX_PAIRS];
  uint32_t flag[FRONT_E / 32];
  key_t tk[FRONT_WAVES][2][16];
  key_t cand[FRONT_WAVES][64];
  float ev[FRONT_WAVES][16];
};

// the groups after the route, as every wave holds them: lane l's flag word (experts 32l .. 32l + 31) and the
// inclusive count of chosen experts up to it; `total` chosen experts, `groups` = total + 1 (the shared expert last)
struct RouteGroups {
  uint32_t word;
  int incl, total, groups;
};

// 1. each token's top-k of the logits and the softmax of the chosen (a wave a token, its logits loaded first); the
// chosen experts flagged as they are found. 2. the groups: the chosen experts in ascending order, then the shared
// expert, counted by each wave from the flags. Ends past a block barrier.
template <typename LT>
__device__ __forceinline__ RouteGroups moe_route(const LT* __restrict__ logits, int K, int B, RouteLds<LT>& r) {
  using RK = RouteKey<LT>;
  using key_t = typename RK::type;
  constexpr int E = FRONT_E, VPL = E / 64, WORDS = E / 32;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  if (tid < WORDS) r.flag[tid] = 0u;
  {
    key_t key[2][VPL];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int t = wave + FRONT_WAVES * u;
      if (t < B) {
#pragma unroll
        for (int i = 0; i < VPL; ++i) key[u][i] = RK::make(logits[(int64_t)t * E + i * 64 + lane], i * 64 + lane);
      }
    }
    lds_sync();  // the flags cleared (the loads stay in flight)
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int t = wave + FRONT_WAVES * u;
      if (t >= B) break;
      wave_top_k<RK, VPL>(key[u], K, r.cand[wave], r.tk[wave][0], r.tk[wave][1]);
      // the softmax of the chosen in rank order, as the reference sums it
      const key_t* sorted = r.tk[wave][1];
      const float top = RK::value(sorted[0]);
      if (lane < K) r.ev[wave][lane] = expf(RK::value(sorted[lane]) - top);
      __builtin_amdgcn_wave_barrier();
      float sum = 0.0f;
      for (int q = 0; q < K; ++q) sum += r.ev[wave][q];
      if (lane < K) {
        const int e = RK::index(sorted[lane]);
        r.idx[t * K + lane] = e;
        r.wt[t * K + lane] = r.ev[wave][lane] / sum;
        atomicOr(&r.flag[e >> 5], 1u << (e & 31));
      }
      __builtin_amdgcn_wave_barrier();
    }
  }
  __syncthreads();
  RouteGroups g;
  g.word = lane < WORDS ? r.flag[lane] : 0u;
  const int cnt = __popc(g.word);
  int incl = cnt;
#pragma unroll
  for (int o = 1; o < WORDS; o <<= 1) {
    const int v = __shfl_up(incl, o);
    if (lane >= o) incl += v;
  }
  g.incl = incl;
  g.total = __shfl(incl, WORDS - 1);
  g.groups = g.total + 1;
  return g;
}

// the expert of group g (wave-uniform): the (g - before)-th flag of the word holding it; E for the shared group
__device__ __forceinline__ int group_expert(const RouteGroups& rg, int g) {
  constexpr int WORDS = FRONT_E / 32;
  const int lane = threadIdx.x & 63;
  if (g >= rg.total) return FRONT_E;
  const int at = __builtin_amdgcn_readfirstlane(__ffsll((unsigned long long)__ballot(lane < WORDS && rg.incl > g)) - 1);
  uint32_t w = __builtin_amdgcn_readfirstlane((uint32_t)__shfl((int)rg.word, at));
  for (int k = g - (__shfl(rg.incl, at) - __popc(w)); k > 0; --k) w &= w - 1u;
  return at * 32 + __ffs(w) - 1;
}

// the route's results for the caller and the combine kernel (one block writes them): the choice, its weights, the
// groups' experts, the group count; and clears the down's row-tile counters (two-kernel form)
template <typename LT>
__device__ __forceinline__ void route_publish(const RouteGroups& rg, const RouteLds<LT>& r, int P, MoeWs ws,
                                              bool clear_counters) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (tid < P) {
    ws.idx[tid] = r.idx[tid];
    ws.w[tid] = r.wt[tid];
  }
  if (wave == 0) {
    int pos = rg.incl - __popc(rg.word);
    for (uint32_t w = rg.word; w; w &= w - 1u) ws.g_expert[pos++] = lane * 32 + __ffs(w) - 1;
    if (lane == 0) ws.g_expert[rg.total] = FRONT_E;
  }
  if (clear_counters && tid < FRONT_D / 64) ws.cnt[tid * CTR_STRIDE] = 0;  // the tail's row-tile counters
  if (tid == 0) *ws.n_groups = rg.groups;
}

// the shared expert's gate logit of each token, rounded to the activation type, into gsh (a wave a token)
template <typename XT>
__device__ __forceinline__ void shared_gate_logits(const XT* __restrict__ x, const XT* __restrict__ wgt, int B,
                                                   float* gsh) {
  constexpr int D = FRONT_D;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int t = wave; t < B; t += FRONT_WAVES) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < D / 512; ++j) {
      const u32x4 xv = *(const u32x4*)(x + (int64_t)t * D + 8 * (lane + 64 * j));
      const u32x4 wv = *(const u32x4*)(wgt + 8 * (lane + 64 * j));
      const XT* a = (const XT*)&xv;
      const XT* b = (const XT*)&wv;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc = fmaf(to_f32(a[i]), to_f32(b[i]), acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) gsh[t] = to_f32(from_f32<XT>(acc));
  }
}

// ---- gate / up items of a block's run: part of one group's 16-row items. `signal` (one-launch layer): 0, or one
// more than the counter set to count the block's items into when its rows of h are out.

template <int KIND, typename XT, typename LT, int TPG>
__device__ __forceinline__ void front_items(int bid, int nblk, const RouteGroups& rg, const RouteLds<LT>& r,
                                            const uint8_t* __restrict__ gate, const uint8_t* __restrict__ up,
                                            const uint8_t* __restrict__ sh_gate, const uint8_t* __restrict__ sh_up,
                                            const XT* __restrict__ x, int K, int B, const FrontPlan& fp, MoeWs ws,
                                            int signal, int (*s_wp)[16]) {
  using MT = XT;
  constexpr int E = FRONT_E, D = FRONT_D, F = FRONT_F, TILES = F / 16;
  constexpr int NT = FRONT_WAVES * 64;
  constexpr int GPER = KIND == Q2_0 ? D / 64 / FRONT_WAVES : D / 32 / FRONT_WAVES;  // a wave's eighth of the groups
  using IT = FrontItem<KIND>;
  constexpr int RB = IT::RB;
  extern __shared__ u32x4 dyn[];
  uint8_t* lds = (uint8_t*)dyn;
  const uint32_t lds_base = SH_LDS_ADDR(dyn);
  float* red = (float*)(lds + fp.red_off);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kq = wave;
  const int P = B * K;

  int g0, first, last;
  if (!group_chunk<TILES>(rg.groups, nblk, bid, g0, first, last)) return;  // block-uniform
  const int e0 = group_expert(rg, g0);

  // this thread's chunks of an item: matrix (0 gate, 1 up) and byte offset from the item's first row; the slot's
  // tail past the two matrices re-reads up's last chunk. Each wave waits on its own count of loads.
  const int loads = (IT::RUNS - wave + FRONT_WAVES - 1) / FRONT_WAVES;
  int pre_off[IT::LOADS];
  bool pre_up[IT::LOADS];
#pragma unroll
  for (int j = 0; j < IT::LOADS; ++j) {
    const int s = (j * FRONT_WAVES + wave) * 64 + lane;
    const int m = s / (16 * IT::CPR), rem = s - m * 16 * IT::CPR;
    const int row = rem / IT::CPR, kk = rem - row * IT::CPR;
    pre_up[j] = m >= 1;
    pre_off[j] = m >= 2 ? 15 * RB + 16 * (IT::CPR_SRC - 1) : row * RB + 16 * min(kk, IT::CPR_SRC - 1);
  }
  const int64_t ebytes = (int64_t)F * RB;
  const uint8_t* gate_e = e0 == E ? sh_gate : gate + (int64_t)e0 * ebytes;
  const uint8_t* up_e = e0 == E ? sh_up : up + (int64_t)e0 * ebytes;
  auto issue = [&](int item) {
    const int rr = item - g0 * TILES;
    const uint8_t* gs = gate_e + (int64_t)rr * 16 * RB;
    const uint8_t* us = up_e + (int64_t)rr * 16 * RB;
    const uint32_t buf = lds_base + fp.ring_off + (item % fp.nbuf) * IT::SLOT + wave * 1024;
#pragma unroll
    for (int j = 0; j < IT::LOADS; ++j)
      if (j < loads) lds_dma16p((pre_up[j] ? us : gs) + pre_off[j], buf + j * (NT * 16));
  };
  // the group's tokens and their activation loads, then the ring's first items: both in flight at once
  const int n_tok = group_pairs(e0, E, r.idx, B, K, s_wp[wave]);
  XRaw<KIND, GPER> xraw;
  {
    int mt = lane_token<TPG>();
    mt = mt < n_tok ? mt : 0;
    const int pp = s_wp[wave][mt];
    x_issue<KIND, XT, GPER>(xraw, x + (int64_t)(pp < P ? pp / K : pp - P) * D, kq * GPER);
  }
  for (int k = 0; k < fp.nbuf - 1 && first + k < last; ++k) issue(first + k);
  XRegs<KIND, TPG, GPER> X;
  x_finish<KIND, XT, TPG, GPER>(X, xraw);

  const DecodeRegs kr = decode_regs<KIND, MT>();
  const int wcol = KIND == Q2_0 ? kq * GPER * 18 : (kq * GPER / 8) * 110;  // the wave's first group in a row
  constexpr int RED = 7 * 64 * TPG;  // up's partial sums after gate's
  // An item's results are reduced and stored at the start of the next item, after its barrier, which also makes
  // the other waves' partial sums (double-buffered) visible: one barrier an item. The stores go before the next
  // loads are issued (a store counts on vmcnt like a load).
  float pg[TPG], pu[TPG];
  int hrow = -1, pbuf = 0;
  auto finish = [&]() {
    if (wave == 0 && hrow >= 0) {
      const int q = lane >> 4;
      const float* rd = red + pbuf * 2 * RED + lane * TPG;
#pragma unroll
      for (int t = 0; t < TPG; ++t) {
        float gs = pg[t], us = pu[t];
#pragma unroll
        for (int w = 0; w < FRONT_WAVES - 1; ++w) {
          gs += rd[w * 64 * TPG + t];
          us += rd[RED + w * 64 * TPG + t];
        }
        const int tt = q * TPG + t;
        if (tt >= n_tok) continue;
        XT* at = (XT*)ws.h + (int64_t)s_wp[0][tt] * F + hrow;
        const XT hv = swiglu_one(from_f32<XT>(gs), from_f32<XT>(us));
        if (signal)
          st_agent<XT>(at, hv);
        else
          *at = hv;
      }
    }
  };
  for (int item = first; item < last; ++item) {
    const int ahead = min(fp.nbuf - 2, last - 1 - item);  // items issued after this one
    wait_vmcnt(ahead * loads);
    lds_sync();  // this item is in LDS for every wave; every wave is done with the item before
    finish();
    if (item + fp.nbuf - 1 < last) issue(item + fp.nbuf - 1);
    const int rr = item - g0 * TILES;
    float acc_g[TPG], acc_u[TPG];
#pragma unroll
    for (int t = 0; t < TPG; ++t) acc_g[t] = acc_u[t] = 0.0f;
    const uint8_t* row0 = lds + fp.ring_off + (item % fp.nbuf) * IT::SLOT + wcol;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    item_mac<KIND, MT, TPG, GPER, true>(row0, IT::RSTRIDE, X, (const uint32_t*)lds, kr, acc_g);
    item_mac<KIND, MT, TPG, GPER, true>(row0 + 16 * IT::RSTRIDE, IT::RSTRIDE, X, (const uint32_t*)lds, kr, acc_u);
    pbuf = item & 1;
    if (wave > 0) {
      float* rw = red + pbuf * 2 * RED;
#pragma unroll
      for (int t = 0; t < TPG; ++t) {
        rw[((wave - 1) * 64 + lane) * TPG + t] = acc_g[t];
        rw[RED + ((wave - 1) * 64 + lane) * TPG + t] = acc_u[t];
      }
    } else {
#pragma unroll
      for (int t = 0; t < TPG; ++t) {
        pg[t] = acc_g[t];
        pu[t] = acc_u[t];
      }
      hrow = rr * 16 + (lane & 15);
    }
  }
  lds_sync();
  finish();
  if (signal && wave == 0) {
    // this run's rows of h (wave 0's agent-scope stores) are complete: counted into the group's; the block that
    // completes a group counts the group, and the one that completes the last group raises the flags
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (lane == 0) {
      const int set = signal - 1, n = last - first;
      if (__hip_atomic_fetch_add(&ws.gdone[(set * (MOE_MAX_PAIRS + 1) + g0) * CTR_STRIDE], n, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT) + n == TILES &&
          __hip_atomic_fetch_add(&ws.gall[set * CTR_STRIDE], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
              rg.groups - 1) {
        for (int c = 0; c < 8; ++c)
          __hip_atomic_store(&ws.gflag[(set * 8 + c) * CTR_STRIDE], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

template <int KIND, typename XT, typename LT, int TPG>
__global__ __launch_bounds__(FRONT_WAVES * 64) void k_moe_front(
    const uint8_t* __restrict__ gate, const uint8_t* __restrict__ up, const uint8_t* __restrict__ sh_gate,
    const uint8_t* __restrict__ sh_up, const LT* __restrict__ logits, const XT* __restrict__ x,
    const XT* __restrict__ wgt, int K, int B, FrontPlan fp, const uint8_t* __restrict__ signed_tab, MoeWs ws) {
  constexpr int NT = FRONT_WAVES * 64;
  __shared__ RouteLds<LT> r;
  __shared__ int s_wp[FRONT_WAVES][16];
  extern __shared__ u32x4 dyn[];
  const uint32_t lds_base = SH_LDS_ADDR(dyn);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // the IQ3_S table first: it does not wait on the choice (2048 chunks, four a thread)
  if constexpr (KIND == IQ3_S) {
#pragma unroll
    for (int i = 0; i < IQ3S_SIGNED_BYTES / 16 / NT; ++i) {
      const int c0 = wave * 64 + i * NT;
      lds_dma16(signed_tab, 16 * (c0 + lane), lds_base + 16 * c0);
    }
  }
  const RouteGroups rg = moe_route<LT>(logits, K, B, r);
  if (blockIdx.x == 0) route_publish<LT>(rg, r, B * K, ws, true);
  if (blockIdx.x == 1 % gridDim.x) shared_gate_logits<XT>(x, wgt, B, ws.gsh);
  front_items<KIND, XT, LT, TPG>(blockIdx.x, gridDim.x, rg, r, gate, up, sh_gate, sh_up, x, K, B, fp, ws, 0,
                                 s_wp);
}

// the combine (strata_mlx/fused.py:448-462) of output (token t, row): experts in 8 rows j taking k = j, j + 8, ...,
// each product rounded as the reference rounds it, then the shared expert gated (its gate logit gsh). y(p) and w(p)
// read pair p's output and routing weight.
template <typename XT, typename YF, typename WF>
__device__ __forceinline__ void combine_one(int t, int row, int K, int B, float gsh, XT* out, YF&& y, WF&& w) {
#pragma clang fp contract(off)
  constexpr int D = FRONT_D;
  float yk[16], wk[16];  // k <= 16
#pragma unroll
  for (int kk = 0; kk < 16; ++kk) {
    yk[kk] = kk < K ? y(t * K + kk) : 0.0f;
    wk[kk] = kk < K ? w(t * K + kk) : 0.0f;
  }
  const float ys = y(B * K + t);
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if (j < K) {
      float part = 0.0f;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int kk = j + 8 * i;
        if (kk < K) {
          const float prod = yk[kk] * wk[kk];
          part = prod + part;
        }
      }
      acc = j == 0 ? part : part + acc;
    }
  }
  const XT routed = from_f32<XT>(acc);
  const XT gate = from_f32<XT>(1.0f / (1.0f + expf(-gsh)));
  const XT shared = from_f32<XT>(to_f32(gate) * ys);
  out[(int64_t)t * D + row] = from_f32<XT>(to_f32(routed) + to_f32(shared));
}

// an item of the tail: 64 rows of down (wave (r, h): rows 16r.. of column half h), 16-byte chunks copied as they
// lie (the rows of a Q2_0 / IQ3_S expert of width 512 are 144 / 220 bytes: 16 rows at that stride fall in distinct
// or two-way shared bank windows); wave w loads the runs of 64 chunks w, w + 8, ...
template <int KIND> struct TailItem {
  static constexpr int RB = (int)row_bytes_dev(KIND, FRONT_F);
  static constexpr int ROWS = 64, TILES = FRONT_D / ROWS;
  static constexpr int CHUNKS = ROWS * RB / 16, RUNS = (CHUNKS + 63) / 64;
  static constexpr int SLOT = RUNS * 1024;
  static constexpr int LOADS = (RUNS + FRONT_WAVES - 1) / FRONT_WAVES;
  static_assert(ROWS * RB % 16 == 0 && RUNS >= FRONT_WAVES && FRONT_WAVES == 8, "tail item layout");
};

struct TailPlan {
  int nbuf;      // ring slots
  int ring_off;  // after the IQ3_S table
  int red_off;   // [2][4][64][TPG] floats: the second column half's sums of the last two items
};

// Spins a block may make on a count another block raises before it gives up and flags the workspace (a guard
// against a hang, never reached when every block runs: the counts it waits on are raised by blocks that wait on
// nothing)
constexpr int MOE_MAX_SPINS = 1 << 20;

// ---- down items of a block's run: part of one group's 64-row items, each pair's outputs rounded to the activation
// type; with `combine`, the block completing a row tile's count combines the tile. `gexp(g)` is group g's expert;
// w(p) the routing weight of pair p, gsh[t] token t's shared gate logit.
template <int KIND, typename XT, int TPG, typename GE, typename WF>
__device__ __forceinline__ void tail_items(int bid, int nblk, int groups, const int* s_idx, GE&& gexp, WF&& wsrc,
                                           const float* gsh, const uint8_t* __restrict__ down,
                                           const uint8_t* __restrict__ sh_down, int K, int B, const TailPlan& tp,
                                           MoeWs ws, int combine, XT* __restrict__ out, int (*s_wp)[16]) {
#pragma clang fp contract(off)
  using MT = XT;
  using IT = TailItem<KIND>;
  constexpr int E = FRONT_E, D = FRONT_D, F = FRONT_F, NT = FRONT_WAVES * 64, TILES = IT::TILES;
  constexpr int GPER = KIND == Q2_0 ? F / 64 / 2 : F / 32 / 2;  // a wave's half of the columns
  constexpr int RB = IT::RB;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rg = wave & 3, kh = wave >> 2;
  const int wcol = KIND == Q2_0 ? kh * GPER * 18 : kh * 110;
  __shared__ int s_ncomb;
  __shared__ int s_comb[TILES];  // the row tiles this block completes (its run's items are distinct tiles)
  extern __shared__ u32x4 dyn[];
  uint8_t* lds = (uint8_t*)dyn;
  const uint32_t lds_base = SH_LDS_ADDR(dyn);
  float* red = (float*)(lds + tp.red_off);

  int g0, first, last;  // this block's run of items: part of one group's
  if (!group_chunk<TILES>(groups, nblk, bid, g0, first, last)) return;  // block-uniform
  if (tid == 0) s_ncomb = 0;

  const int loads = (IT::RUNS - wave + FRONT_WAVES - 1) / FRONT_WAVES;
  int pre_off[IT::LOADS];
#pragma unroll
  for (int j = 0; j < IT::LOADS; ++j) pre_off[j] = 16 * min((j * FRONT_WAVES + wave) * 64 + lane, IT::CHUNKS - 1);
  const int e0 = gexp(g0);
  const uint8_t* down_e = e0 == E ? sh_down : down + (int64_t)e0 * D * RB;
  auto issue = [&](int item) {
    const uint8_t* src = down_e + (int64_t)(item - g0 * TILES) * IT::ROWS * RB;
    const uint32_t buf = lds_base + tp.ring_off + (item % tp.nbuf) * IT::SLOT + wave * 1024;
#pragma unroll
    for (int j = 0; j < IT::LOADS; ++j)
      if (j < loads) lds_dma16(src, pre_off[j], buf + j * (NT * 16));
  };
  const int n_tok = group_pairs(e0, E, s_idx, B, K, s_wp[wave]);
  XRaw<KIND, GPER> xraw;
  {
    // the group's tokens and their loads of h, then the ring's first items: both in flight at once
    int mt = lane_token<TPG>();
    mt = mt < n_tok ? mt : 0;
    x_issue<KIND, XT, GPER>(xraw, (const XT*)ws.h + (int64_t)s_wp[wave][mt] * F, kh * GPER);
    for (int k = 0; k < tp.nbuf - 1 && first + k < last; ++k) issue(first + k);
  }
  XRegs<KIND, TPG, GPER> X;
  x_finish<KIND, XT, TPG, GPER>(X, xraw);

  const DecodeRegs kr = decode_regs<KIND, MT>();
  // Each pair's outputs, rounded to the activation type, reduced and stored at the start of the next item, after
  // its barrier, which also makes the other column half's sums (double-buffered) visible: one barrier an item.
  // With the combine in this kernel they go out as device-scope stores for the block that combines them.
  float pacc[TPG];
  int yrow = -1, pbuf = 0;
  auto store_y = [&]() {
    if (kh == 0 && yrow >= 0) {
      const int q = lane >> 4;
      const float* rd = red + (pbuf * 4 * 64 + rg * 64 + lane) * TPG;
#pragma unroll
      for (int t = 0; t < TPG; ++t) {
        const int tt = q * TPG + t;
        if (tt >= n_tok) continue;
        float* at = ws.y + (int64_t)s_wp[wave][tt] * D + yrow;
        const float v = to_f32(from_f32<XT>(pacc[t] + rd[t]));
        if (combine)
          __hip_atomic_store(at, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else
          *at = v;
      }
    }
  };
  for (int item = first; item < last; ++item) {
    const int ahead = min(tp.nbuf - 2, last - 1 - item);
    wait_vmcnt(ahead * loads);
    lds_sync();
    store_y();
    if (item + tp.nbuf - 1 < last) issue(item + tp.nbuf - 1);
    const int tile = item - g0 * TILES;
    float acc[TPG];
#pragma unroll
    for (int t = 0; t < TPG; ++t) acc[t] = 0.0f;
    const uint8_t* row0 = lds + tp.ring_off + (item % tp.nbuf) * IT::SLOT + rg * 16 * RB + wcol;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    item_mac<KIND, MT, TPG, GPER, true>(row0, RB, X, (const uint32_t*)lds, kr, acc);
    pbuf = item & 1;
    if (kh == 1) {
#pragma unroll
      for (int t = 0; t < TPG; ++t) red[(pbuf * 4 * 64 + rg * 64 + lane) * TPG + t] = acc[t];
    } else {
#pragma unroll
      for (int t = 0; t < TPG; ++t) pacc[t] = acc[t];
      yrow = tile * IT::ROWS + rg * 16 + (lane & 15);
    }
  }
  lds_sync();
  store_y();
  if (!combine) return;
  // Count this block's items into their row tiles' counters once every output of them is out; the block that
  // completes a tile's count combines the tile and clears the counter. The hand-off is release / acquire at agent
  // scope: the block's outputs are ordered before its counts by one release fence (after the barrier that joins
  // every wave's stores), and a combining block's reads after its counts by one acquire fence. The outputs
  // themselves are agent-scope stores and loads, so neither fence has much to write back or invalidate.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid < last - first) {
    const int tile = (first + tid) % TILES;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    if (__hip_atomic_fetch_add(&ws.cnt[tile * CTR_STRIDE], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
        groups - 1)
      s_comb[atomicAdd(&s_ncomb, 1)] = tile;
  }
  __syncthreads();
  const int ncomb = s_ncomb;
  if (ncomb == 0) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  for (int qv = tid; qv < ncomb * B * IT::ROWS; qv += NT) {
    const int c = qv / (B * IT::ROWS), rest = qv - c * (B * IT::ROWS);
    const int t = rest / IT::ROWS, row = s_comb[c] * IT::ROWS + rest % IT::ROWS;
    combine_one<XT>(t, row, K, B, gsh[t], out, [&](int p) {
      return __hip_atomic_load(ws.y + (int64_t)p * D + row, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }, wsrc);
  }
  if (tid < ncomb)
    __hip_atomic_store(&ws.cnt[s_comb[tid] * CTR_STRIDE], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int KIND, typename XT, int TPG>
__global__ __launch_bounds__(FRONT_WAVES * 64) void k_moe_tail(const uint8_t* __restrict__ down,
                                                               const uint8_t* __restrict__ sh_down, int K, int B,
                                                               TailPlan tp, const uint8_t* __restrict__ signed_tab,
                                                               MoeWs ws, int combine, XT* __restrict__ out) {
  constexpr int NT = FRONT_WAVES * 64;
  const int P = B * K;
  __shared__ int s_groups;
  __shared__ int s_idx[MOE_MAX_PAIRS], s_gexp[MOE_MAX_PAIRS + 1];
  __shared__ float s_w[MOE_MAX_PAIRS], s_gsh[MOE_MAX_TOKENS];
  __shared__ int s_wp[FRONT_WAVES][16];
  extern __shared__ u32x4 dyn[];
  const uint32_t lds_base = SH_LDS_ADDR(dyn);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // the IQ3_S table (it waits on nothing), then the front's choice and groups in one trip
  if constexpr (KIND == IQ3_S) {
#pragma unroll
    for (int i = 0; i < IQ3S_SIGNED_BYTES / 16 / NT; ++i) {
      const int c0 = wave * 64 + i * NT;
      lds_dma16(signed_tab, 16 * (c0 + lane), lds_base + 16 * c0);
    }
  }
  if (tid == 0) s_groups = *ws.n_groups;
  if (tid < P) {
    s_idx[tid] = ws.idx[tid];
    s_w[tid] = ws.w[tid];
  }
  if (tid <= P) s_gexp[tid] = ws.g_expert[tid];  // entries past the groups are never read
  if (tid < B) s_gsh[tid] = ws.gsh[tid];
  __syncthreads();  // (also waits for the table)
  tail_items<KIND, XT, TPG>(blockIdx.x, gridDim.x, s_groups, s_idx,
                            [&](int g) { return __builtin_amdgcn_readfirstlane(s_gexp[g]); },
                            [&](int p) { return s_w[p]; }, s_gsh, down, sh_down, K, B, tp, ws, combine, out,
                            s_wp);
}

// ---- the whole layer in one launch, for windows of few groups (the common shape, Q2_0). SWITCHED OFF (nothing
// reaches it: sh_moe_set_one_launch refuses to switch it on): at 2 tokens of float16 it made an illegal memory
// access, from direct loads issued inside the wait-state window after v_readfirstlane wrote their base (lds_dma16
// now waits it out); it stays off until that fix has run on a GPU. Every block routes the
// window; then its ticket, taken in the order blocks start, makes it a gate / up block (the first `nfront`) or a
// down block. A down block owns 16 rows of the output for every group: its waves load those rows of their groups'
// down weights at once (a wave the groups w, w + 8, w + 16, two at a time), wait until every group's gate / up is
// out, read the groups' h rows, and combine the 16 rows in LDS. The blocks a down block waits on hold lower
// tickets, so they started before it and wait on nothing: no order of dispatch or residency can make the wait
// circular. The counters come in two sets used by calls in turn; every block reads which before it draws its
// ticket, and the block that draws the last ticket clears the other set and switches to it for the next call.
constexpr int LAYER_GROUPS = 3 * FRONT_WAVES;  // groups a window may have for the one launch
constexpr int LAYER_PAIRS = 48;                // pairs and shared tokens (B * k + B) it may have
constexpr int LAYER_ROWS = 16;                 // output rows a down block owns

template <int KIND> struct RowSlot {  // a group's 16 rows of down weights in LDS, as they lie
  static constexpr int RB = (int)row_bytes_dev(KIND, FRONT_F);
  static constexpr int CHUNKS = LAYER_ROWS * RB / 16, LOADS = (CHUNKS + 63) / 64, SLOT = LOADS * 1024;
};

template <int KIND, typename XT, typename LT, int TPG>
__global__ __launch_bounds__(FRONT_WAVES * 64) void k_moe_layer(
    const uint8_t* __restrict__ gate, const uint8_t* __restrict__ up, const uint8_t* __restrict__ down,
    const uint8_t* __restrict__ sh_gate, const uint8_t* __restrict__ sh_up, const uint8_t* __restrict__ sh_down,
    const LT* __restrict__ logits, const XT* __restrict__ x, const XT* __restrict__ wgt, int K, int B, FrontPlan fp,
    int row_off, int nfront, MoeWs ws, XT* __restrict__ out) {
  static_assert(KIND == Q2_0, "the one-launch layer is written for Q2_0 gate, up and down");
  using MT = XT;
  using RS = RowSlot<KIND>;
  constexpr int E = FRONT_E, D = FRONT_D, F = FRONT_F, NT = FRONT_WAVES * 64, GPER = F / 64;
  constexpr int TW = FRONT_WAVES - 1;  // the ticket's wave: past the route's tokens for windows of few groups
  __shared__ RouteLds<LT> r;
  __shared__ int s_ticket, s_set;
  __shared__ float s_gsh[MOE_MAX_TOKENS];
  __shared__ int s_wp[LAYER_GROUPS][16];  // gate / up: a wave's group's pairs; down: each group's
  __shared__ float s_y[LAYER_PAIRS][LAYER_ROWS];
  extern __shared__ u32x4 dyn[];
  uint8_t* lds = (uint8_t*)dyn;
  const uint32_t lds_base = SH_LDS_ADDR(dyn);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // the counter set, read before the ticket is drawn; the ticket's value is used after the route (its wave issues
  // no loads meanwhile, so nothing waits on the atomic until then)
  int set = 0, ticket = 0;
  if (tid == TW * 64) {
    set = __hip_atomic_load(ws.par, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    ticket = __hip_atomic_fetch_add(ws.ticket, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  const RouteGroups rg = moe_route<LT>(logits, K, B, r);
  if (tid == TW * 64) {
    s_ticket = ticket;
    s_set = set;
  }
  lds_sync();
  ticket = s_ticket;
  set = s_set;
  if (ticket < 0 || ticket >= (int)gridDim.x || (set & ~1)) {  // counters not at zero: no work, nothing read past them
    if (tid == 0) __hip_atomic_store(ws.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  if (ticket == (int)gridDim.x - 1) {  // every block has read the set and drawn its ticket
    const int other = set ^ 1;
    for (int i = tid; i < MOE_MAX_PAIRS + 1; i += NT)
      __hip_atomic_store(&ws.gdone[(other * (MOE_MAX_PAIRS + 1) + i) * CTR_STRIDE], 0, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    if (tid < 8)
      __hip_atomic_store(&ws.gflag[(other * 8 + tid) * CTR_STRIDE], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (tid == 0) {
      __hip_atomic_store(&ws.gall[other * CTR_STRIDE], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(ws.ticket, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(ws.par, other, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if (ticket < nfront) {
    if (ticket == 0) {
      route_publish<LT>(rg, r, B * K, ws, false);
      shared_gate_logits<XT>(x, wgt, B, ws.gsh);
    }
    front_items<KIND, XT, LT, TPG>(ticket, nfront, rg, r, gate, up, sh_gate, sh_up, x, K, B, fp, ws, set + 1, s_wp);
    return;
  }
  const int rt = ticket - nfront;  // block-uniform
  if (rt >= D / LAYER_ROWS) return;
  const int row0 = rt * LAYER_ROWS, groups = rg.groups;
  const int ng = groups > wave ? (groups - wave + FRONT_WAVES - 1) / FRONT_WAVES : 0;  // this wave's groups
  auto slot = [&](int j) { return row_off + (2 * wave + (j & 1)) * RS::SLOT; };
  auto issue = [&](int j) {
    const int e = group_expert(rg, wave + FRONT_WAVES * j);
    const uint8_t* src = (e == E ? sh_down : down + (int64_t)e * D * RS::RB) + (int64_t)row0 * RS::RB;
#pragma unroll
    for (int c = 0; c < RS::LOADS; ++c)
      lds_dma16(src, 16 * min(c * 64 + lane, RS::CHUNKS - 1), lds_base + slot(j) + c * 1024);
  };
  for (int j = 0; j < ng && j < 2; ++j) issue(j);
  int n_tok[3];
  for (int j = 0; j < 3; ++j)
    n_tok[j] = j < ng ? group_pairs(group_expert(rg, wave + FRONT_WAVES * j), E, r.idx, B, K,
                                    s_wp[wave + FRONT_WAVES * j])
                      : 0;
  shared_gate_logits<XT>(x, wgt, B, s_gsh);
  if (tid == 0) {  // every group's h is out once this block's eighth of the flags is up
    const int32_t* flag = ws.gflag + (set * 8 + (rt & 7)) * CTR_STRIDE;
    int spins = 0;
    while (__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0) {
      __builtin_amdgcn_s_sleep(1);
      if (++spins > MOE_MAX_SPINS) {
        __hip_atomic_store(ws.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
    }
  }
  lds_sync();  // (the slots' loads stay in flight)
  const DecodeRegs kr = decode_regs<KIND, MT>();
  for (int j = 0; j < ng; ++j) {
    const int* wp = s_wp[wave + FRONT_WAVES * j];
    int mt = lane_token<TPG>();
    mt = mt < n_tok[j] ? mt : 0;
    XRaw<KIND, GPER> xraw;
    x_issue_agent<KIND, XT, GPER>(xraw, (const XT*)ws.h, wp[mt], F, 0);
    XRegs<KIND, TPG, GPER> X;
    x_finish<KIND, XT, TPG, GPER>(X, xraw);
    wait_vmcnt(0);  // the slot's rows, loaded before h
    float acc[TPG];
#pragma unroll
    for (int t = 0; t < TPG; ++t) acc[t] = 0.0f;
    item_mac<KIND, MT, TPG, GPER, true>(lds + slot(j), RS::RB, X, nullptr, kr, acc);
    const int q = lane >> 4, n = lane & 15;
#pragma unroll
    for (int t = 0; t < TPG; ++t) {
      const int tt = q * TPG + t;
      if (tt < n_tok[j]) s_y[wp[tt]][n] = to_f32(from_f32<XT>(acc[t]));
    }
    if (j == 0 && ng > 2) {  // the third group into the first one's slot, once this wave has read it
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      issue(2);
    }
  }
  lds_sync();
  if (tid < B * LAYER_ROWS) {
    const int t = tid / LAYER_ROWS, n = tid % LAYER_ROWS;
    combine_one<XT>(t, row0 + n, K, B, s_gsh[t], out, [&](int p) { return s_y[p][n]; },
                    [&](int p) { return r.wt[p]; });
  }
}

// The tail for a window of few groups (at most 16: one token's k experts and the shared one), Q2_0: a block is 16
// rows of down, a wave a group (all 512 columns; its 16 rows' bytes by direct loads into the wave's own LDS slot,
// its tokens' activations in registers, all issued at once), each pair's 16 outputs rounded into LDS, then the
// combine of those 16 rows for every token in LDS: no partial outputs through memory and no third launch.
constexpr int TAIL1_WAVES = 16;

template <typename XT, int TPG>
__global__ __launch_bounds__(TAIL1_WAVES * 64) void k_moe_tail1(const uint8_t* __restrict__ down,
                                                                 const uint8_t* __restrict__ sh_down, int K, int B,
                                                                 MoeWs ws, XT* __restrict__ out) {
  using MT = XT;
  constexpr int E = FRONT_E, D = FRONT_D, F = FRONT_F;
  constexpr int GPER = F / 64;                           // a wave's 16 rows whole: 8 Q2_0 blocks
  constexpr int RB = (int)row_bytes_dev(Q2_0, F);       // 144 bytes: 16 rows at that stride in distinct banks
  constexpr int CHUNKS = 16 * RB / 16, LOADS = (CHUNKS + 63) / 64, SLOT = LOADS * 1024;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int row0 = blockIdx.x * 16;
  const int P = B * K;
  __shared__ int s_groups, s_idx[16], s_gexp[TAIL1_WAVES], s_wp[TAIL1_WAVES][16];
  __shared__ float s_w[16], s_gsh[MOE_MAX_TOKENS];
  __shared__ float s_y[MOE_MAX_TOKENS * 2][16];  // [pair][row]: P + B <= 32 when the groups are at most 16
  extern __shared__ u32x4 dyn[];
  uint8_t* lds = (uint8_t*)dyn;
  const uint32_t lds_base = SH_LDS_ADDR(dyn);

  if (tid == 0) s_groups = *ws.n_groups;
  if (tid < P) {
    s_idx[tid] = ws.idx[tid];
    s_w[tid] = ws.w[tid];
  }
  if (tid < TAIL1_WAVES) s_gexp[tid] = ws.g_expert[min(tid, P)];  // entries past the groups are never read
  if (tid < B) s_gsh[tid] = ws.gsh[tid];
  __syncthreads();
  const int groups = s_groups;
  if (wave < groups) {
    const int e = __builtin_amdgcn_readfirstlane(s_gexp[wave]);
    const uint8_t* src = (e == E ? sh_down : down + (int64_t)e * D * RB) + (int64_t)row0 * RB;
    const uint32_t buf = lds_base + wave * SLOT;
#pragma unroll
    for (int j = 0; j < LOADS; ++j) lds_dma16(src, 16 * min(j * 64 + lane, CHUNKS - 1), buf + j * 1024);
    const int n_tok = group_pairs(e, E, s_idx, B, K, s_wp[wave]);
    int mt = lane_token<TPG>();
    mt = mt < n_tok ? mt : 0;
    XRegs<Q2_0, TPG, GPER> X;
    load_x_row<Q2_0, XT, TPG, GPER, true>(X, (const XT*)ws.h + (int64_t)s_wp[wave][mt] * F, 0);
    const DecodeRegs kr = decode_regs<Q2_0, MT>();
    wait_vmcnt(0);
    float acc[TPG];
#pragma unroll
    for (int t = 0; t < TPG; ++t) acc[t] = 0.0f;
    item_mac<Q2_0, MT, TPG, GPER, true>(lds + wave * SLOT, RB, X, nullptr, kr, acc);
    const int q = lane >> 4, n = lane & 15;
#pragma unroll
    for (int t = 0; t < TPG; ++t) {
      const int tt = q * TPG + t;
      if (tt < n_tok) s_y[s_wp[wave][tt]][n] = to_f32(from_f32<XT>(acc[t]));
    }
  }
  __syncthreads();
  if (tid < B * 16) {
    const int t = tid >> 4, n = tid & 15;
    combine_one<XT>(t, row0 + n, K, B, s_gsh[t], out, [&](int p) { return s_y[p][n]; },
                    [&](int p) { return s_w[p]; });
  }
}

// the combine as a kernel of its own after the tail, a thread an output
template <typename XT>
__global__ __launch_bounds__(256) void k_moe_combine(int K, int B, MoeWs ws, XT* __restrict__ out) {
  const int row = blockIdx.x * 256 + threadIdx.x;
  combine_one<XT>(blockIdx.y, row, K, B, ws.gsh[blockIdx.y], out, [&](int p) { return ws.y[(int64_t)p * FRONT_D + row]; },
                  [&](int p) { return ws.w[p]; });
}

// ---- down and the combine: a block is 16 output rows of every group's expert
//
// The groups go through in chunks of cg <= DOWN_CHUNK_G (as many as LDS holds twice), their weight slices
// double-buffered in LDS: the next chunk's loads
// are in flight while this chunk multiplies. A wave takes every fourth group of a chunk; each pair's 16 outputs,
// rounded to the activation type, stay in LDS for the combine at the end.

constexpr int DOWN_CHUNK_G = 16;

// DOWN_CHUNK_G byte ranges of n bytes (16 rows of an expert) from their own sources to LDS slots of `slot` bytes
// (alignment kept modulo 16, edge chunks byte by byte): 16 threads a range, a pass of U chunks each.
template <int U> struct SliceStage {
  const uint8_t* const* src;
  uint8_t* dst;
  int n, nr, slot;
  u32x4 v[U];
  bool full[U];

  __device__ __forceinline__ SliceStage(uint8_t* dst_, const uint8_t* const* src_, int nr_, int n_, int slot_)
      : src(src_), dst(dst_), n(n_), nr(nr_), slot(slot_) {}
  __device__ __forceinline__ int chunks() const { return (15 + n + 15) >> 4; }
  __device__ __forceinline__ int passes() const { return (chunks() + 16 * U - 1) / (16 * U); }
  __device__ __forceinline__ void load(int pass, int tid) {
    const int r = tid >> 4, j = tid & 15;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int cc = (pass * U + u) * 16 + j;
      full[u] = false;
      if (r < nr && cc < chunks()) {
        const uint8_t* s = src[r];
        const uint8_t* p = (const uint8_t*)(((uintptr_t)s & ~(uintptr_t)15) + 16 * (uintptr_t)cc);
        if (p >= s && p + 16 <= s + n) {
          v[u] = *(const u32x4*)p;
          full[u] = true;
        }
      }
    }
  }
  __device__ __forceinline__ void store(int pass, int tid) {
    const int r = tid >> 4, j = tid & 15;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int cc = (pass * U + u) * 16 + j;
      if (r >= nr || cc >= chunks()) continue;
      const uint8_t* s = src[r];
      const uint8_t* p = (const uint8_t*)(((uintptr_t)s & ~(uintptr_t)15) + 16 * (uintptr_t)cc);
      uint8_t* d = dst + r * slot + 16 * cc;
      if (full[u]) {
        *(u32x4*)d = v[u];
      } else {
        for (int b = 0; b < 16; ++b)
          if (p + b >= s && p + b < s + n) d[b] = p[b];
      }
    }
  }
};

template <int KIND, typename XT, int TPG>
__global__ __launch_bounds__(256) void k_moe_down(const uint8_t* __restrict__ down, const uint8_t* __restrict__ sh_down,
                                                  int E, int K, int B, int D, int F, int cg,
                                                  const uint8_t* __restrict__ signed_tab, MoeWs ws, XT* __restrict__ out) {
#pragma clang fp contract(off)
  using MT = XT;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row0 = blockIdx.x * 16;
  const int P = B * K, G = P + 1;
  __shared__ int s_groups, s_e[MOE_MAX_PAIRS + 1], s_n[MOE_MAX_PAIRS + 1], s_pair[MOE_MAX_PAIRS + 1][16];
  __shared__ float s_w[MOE_MAX_PAIRS], s_gsh[MOE_MAX_TOKENS];
  __shared__ float s_y[MOE_MAX_PAIRS + MOE_MAX_TOKENS][16];
  __shared__ const uint8_t* s_src[2][DOWN_CHUNK_G];
  extern __shared__ u32x4 dyn[];
  uint8_t* tab = (uint8_t*)dyn;
  const int64_t rb = row_bytes_dev(KIND, F);
  const int slot = (int)(((15 + 16 * rb + 15) >> 4) << 4);
  uint8_t* buf[2] = {tab + moe_tab_bytes<KIND>(), tab + moe_tab_bytes<KIND>() + cg * slot};

  // the whole group table, the routing weights and the shared gate in one trip
  if (tid == 0) s_groups = *ws.n_groups;
  if (tid < B) s_gsh[tid] = ws.gsh[tid];
  copy_to_lds<1>(s_e, ws.g_expert, G, tid, 256);
  copy_to_lds<1>(s_n, ws.g_ntok, G, tid, 256);
  copy_to_lds<1>(s_w, ws.w, P, tid, 256);
  copy_to_lds<11>(&s_pair[0][0], ws.g_pair, G * 16, tid, 256);
  if constexpr (KIND == IQ3_S) {
    ByteStage<8> tst(tab, signed_tab, IQ3S_SIGNED_BYTES, nullptr, nullptr, 0);
    for (int p = 0; p < tst.passes(256); ++p) {
      tst.load(p, tid, 256);
      tst.store(p, tid, 256);
    }
  }
  __syncthreads();
  const int groups = s_groups;
  const int chunks = (groups + cg - 1) / cg;
  auto sources = [&](int c) {
    const int g0 = c * cg;
    if (tid < cg && g0 + tid < groups) {
      const int e = s_e[g0 + tid];
      s_src[c & 1][tid] = (e == E ? sh_down : down + (int64_t)e * D * rb) + (int64_t)row0 * rb;
    }
  };
  sources(0);
  __syncthreads();
  SliceStage<10> st(buf[0], s_src[0], min(cg, groups), (int)(16 * rb), slot);
  for (int p = 0; p < st.passes(); ++p) {
    st.load(p, tid);
    st.store(p, tid);
  }
  if (chunks > 1) sources(1);
  __syncthreads();
  for (int c = 0; c < chunks; ++c) {
    // the next chunk's loads go out before this chunk multiplies
    const bool more = c + 1 < chunks;
    SliceStage<10> nx(buf[(c + 1) & 1], s_src[(c + 1) & 1], more ? min(cg, groups - (c + 1) * cg) : 0,
                      (int)(16 * rb), slot);
    const int single = nx.passes() == 1;
    if (more && single) nx.load(0, tid);
    const int g0 = c * cg, gn = min(cg, groups - g0);
    for (int li = wave; li < gn; li += 4) {
      const int gi = g0 + li;
      const int n_tok = s_n[gi];
      const int mt = lane_token<TPG>();
      const bool real = mt < n_tok;
      const MT* xg = (const MT*)ws.h + (int64_t)s_pair[gi][real ? mt : 0] * F;
      float acc[1][TPG];
#pragma unroll
      for (int i = 0; i < TPG; ++i) acc[0][i] = 0.0f;
      const uint8_t* tiles[1] = {buf[c & 1] + li * slot + lead_of(s_src[c & 1][li])};
      tile_mac_global<KIND, MT, TPG, frag_chunk<KIND>(), 1>(tiles, (int)rb, xg, real, 0, F / scale_group<KIND>(),
                                                            (const uint32_t*)tab, acc);
      const int g = lane >> 4, n = lane & 15;
#pragma unroll
      for (int i = 0; i < TPG; ++i) {
        const int t = g * TPG + i;
        if (t < n_tok) s_y[s_pair[gi][t]][n] = to_f32(from_f32<XT>(acc[0][i]));
      }
    }
    if (more) {
      if (single) {
        nx.store(0, tid);
      } else {
        for (int p = 0; p < nx.passes(); ++p) {
          nx.load(p, tid);
          nx.store(p, tid);
        }
      }
    }
    __syncthreads();
    if (c + 2 < chunks) sources(c + 2);
    __syncthreads();
  }
  // the combine (strata_mlx/fused.py:448-462): experts in 8 rows j taking k = j, j + 8, ..., each product rounded
  if (tid < B * 16) {
    const int t = tid >> 4, n = tid & 15;
    float acc = 0.0f;
    for (int j = 0; j < 8 && j < K; ++j) {
      float part = 0.0f;
      for (int kk = j; kk < K; kk += 8) {
        const float prod = s_y[t * K + kk][n] * s_w[t * K + kk];
        part = prod + part;
      }
      acc = j == 0 ? part : part + acc;
    }
    const XT routed = from_f32<XT>(acc);
    const XT gate = from_f32<XT>(1.0f / (1.0f + expf(-s_gsh[t])));
    const XT shared = from_f32<XT>(to_f32(gate) * s_y[P + t][n]);
    out[(int64_t)t * D + row0 + n] = from_f32<XT>(to_f32(routed) + to_f32(shared));
  }
}

template <int KIND, int KIND_DOWN, typename XT, typename LT, int TPG>
static int launch_moe(const uint8_t* gate, const uint8_t* up, const uint8_t* down, int64_t E, const uint8_t* sg,
                      const uint8_t* su, const uint8_t* sd, const XT* wg, const uint8_t* tables, const LT* logits,
                      const XT* x, int64_t B, int64_t K, int64_t D, int64_t F, XT* out, const MoeWs& ws,
                      hipStream_t stream, int phases) {
  const uint8_t* stab = tables ? tables + TAB_IQ3S_SIGNED : nullptr;
  int st = OK;
  if (phases & 32) {  // the whole layer in one launch (windows of few groups, Q2_0), else the two launches
    if constexpr (KIND == Q2_0 && KIND_DOWN == Q2_0) {
      const int64_t groups_most = std::min<int64_t>(B * K, E) + 1;
      if (groups_most <= LAYER_GROUPS && B * K + B <= LAYER_PAIRS) {
        using IF = FrontItem<KIND>;
        using RS = RowSlot<KIND_DOWN>;
        auto kern = k_moe_layer<KIND, XT, LT, TPG>;
        const int nt = FRONT_WAVES * 64;
        const size_t fixed = static_lds(kern);
        const size_t red_f = (size_t)2 * 2 * 7 * 64 * TPG * 4;
        const size_t rows = (size_t)2 * FRONT_WAVES * RS::SLOT;  // the down blocks' slots
        FrontPlan fp;
        fp.ring_off = 0;
        // direct loads land below 128 KiB; a shallower ring where that makes room for two blocks a CU
        fp.nbuf = 3;
        while (fp.nbuf > 2 && ((size_t)fp.nbuf * IF::SLOT > 128 * 1024 ||
                               fixed + (size_t)fp.nbuf * IF::SLOT + red_f > LDS_BYTES ||
                               (fixed + (size_t)fp.nbuf * IF::SLOT + red_f > LDS_BYTES / 2 &&
                                fixed + (size_t)(fp.nbuf - 1) * IF::SLOT + red_f <= LDS_BYTES / 2)))
          --fp.nbuf;
        fp.red_off = fp.nbuf * IF::SLOT;
        const size_t lds = std::max((size_t)fp.red_off + red_f, rows);
        if ((size_t)fp.red_off > 128 * 1024 || rows > 128 * 1024 || lds + fixed > LDS_BYTES)
          return fail(E_UNSUPPORTED, "moe_decode: %zu bytes of LDS for the one-launch layer", lds);
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, nt, lds) != hipSuccess || per_cu < 1)
          per_cu = 1;
        // the down blocks first (a block a 16-row slice of the output), the gate / up blocks what is left of the
        // blocks that fit at once, up to a block an item
        const int64_t ndown = FRONT_D / LAYER_ROWS, fit = (int64_t)device_cus() * per_cu;
        const int64_t nfront = std::min<int64_t>(groups_most * (FRONT_F / 16), fit - ndown);
        if (nfront >= groups_most) {
          hipLaunchKernelGGL(kern, dim3((unsigned)(nfront + ndown)), dim3(nt), lds, stream, gate, up, down, sg, su, sd,
                             logits, x, wg, (int)K, (int)B, fp, 0, (int)nfront, ws, out);
          return check_launch("moe_decode layer");
        }
      }
    }
    phases = 8 | 16;
  }
  if (phases & 8) {  // front: route, gate and up (the common shape)
    using IT = FrontItem<KIND>;
    FrontPlan fp;
    const int nt = FRONT_WAVES * 64;
    fp.ring_off = moe_tab_bytes<KIND>();
    const size_t red = (size_t)2 * 2 * 7 * 64 * TPG * 4;
    auto kern = k_moe_front<KIND, XT, LT, TPG>;
    const size_t fixed = static_lds(kern);
    // direct loads land below 128 KiB
    fp.nbuf = 3;
    while (fp.nbuf > 2 && ((size_t)fp.ring_off + (size_t)fp.nbuf * IT::SLOT > 128 * 1024 ||
                           fixed + fp.ring_off + (size_t)fp.nbuf * IT::SLOT + red > LDS_BYTES))
      --fp.nbuf;
    fp.red_off = fp.ring_off + fp.nbuf * IT::SLOT;
    const size_t lds = (size_t)fp.red_off + red;
    if ((size_t)fp.ring_off + (size_t)fp.nbuf * IT::SLOT > 128 * 1024 || lds + fixed > LDS_BYTES)
      return fail(E_UNSUPPORTED, "moe_decode: %zu bytes of LDS for the front", lds);
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, nt, lds) != hipSuccess || per_cu < 1) per_cu = 1;
    const int64_t most = (std::min<int64_t>(B * K, E) + 1) * (FRONT_F / 16);
    const int64_t grid = std::min<int64_t>(most, (int64_t)device_cus() * per_cu);
    if (grid < std::min<int64_t>(B * K, E) + 1)  // a block at least for each group
      return fail(E_UNSUPPORTED, "moe_decode: %lld blocks for the front", (long long)grid);
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(nt), lds, stream, gate, up, sg, su, logits, x, wg, (int)K,
                       (int)B, fp, stab, ws);
    st = check_launch("moe_decode front");
    if (st) return st;
  }
  if (phases & 16) {  // tail: down and the combine (the common shape)
    using IT = TailItem<KIND_DOWN>;
    TailPlan tp;
    tp.ring_off = moe_tab_bytes<KIND_DOWN>();
    auto kern = k_moe_tail<KIND_DOWN, XT, TPG>;
    const size_t fixed = static_lds(kern);
    const size_t red = (size_t)2 * 4 * 64 * TPG * 4;
    tp.nbuf = 4;
    while (tp.nbuf > 2 && ((size_t)tp.ring_off + (size_t)tp.nbuf * IT::SLOT > 128 * 1024 ||
                           fixed + tp.ring_off + (size_t)tp.nbuf * IT::SLOT + red > LDS_BYTES))
      --tp.nbuf;
    tp.red_off = tp.ring_off + tp.nbuf * IT::SLOT;
    const size_t lds = (size_t)tp.red_off + red;
    if ((size_t)tp.red_off > 128 * 1024 || lds + fixed > LDS_BYTES)
      return fail(E_UNSUPPORTED, "moe_decode: %zu bytes of LDS for the tail", lds);
    const int nt = FRONT_WAVES * 64;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, nt, lds) != hipSuccess || per_cu < 1) per_cu = 1;
    const int64_t most = (std::min<int64_t>(B * K, E) + 1) * IT::TILES;
    const int64_t grid = std::min<int64_t>(most, (int64_t)device_cus() * per_cu);
    if (grid < std::min<int64_t>(B * K, E) + 1)  // a block at least for each group (a block's items are then at
      return fail(E_UNSUPPORTED, "moe_decode: %lld blocks for the tail", (long long)grid);  // most TILES)
    // a few tokens: the tail's last block of a row tile combines it (no third launch); more: a combine kernel
    // (the tiles' last blocks would each combine several tiles, serially)
    const int combine = B <= g_tail_combine_upto.load(std::memory_order_relaxed);
    if constexpr (KIND_DOWN == Q2_0) {
      if (std::min<int64_t>(B * K, E) + 1 <= TAIL1_WAVES) {  // few groups: a block a 16-row tile, a wave a group
        constexpr int LOADS = (16 * (int)row_bytes_dev(Q2_0, FRONT_F) / 16 + 63) / 64;
        const size_t lds1 = (size_t)TAIL1_WAVES * LOADS * 1024;
        hipLaunchKernelGGL((k_moe_tail1<XT, TPG>), dim3(FRONT_D / 16), dim3(TAIL1_WAVES * 64), lds1, stream, down, sd,
                           (int)K, (int)B, ws, out);
        return check_launch("moe_decode tail");
      }
    }
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(nt), lds, stream, down, sd, (int)K, (int)B, tp, stab, ws,
                       combine, out);
    st = check_launch("moe_decode tail");
    if (st) return st;
    if (!combine) {
      hipLaunchKernelGGL(k_moe_combine<XT>, dim3((unsigned)(FRONT_D / 256), (unsigned)B), dim3(256), 0, stream,
                         (int)K, (int)B, ws, out);
      st = check_launch("moe_decode combine");
      if (st) return st;
    }
  }
  if (phases & 1) {
    auto route = [&](auto vc) {
      constexpr int V = decltype(vc)::value;
      hipLaunchKernelGGL((k_moe_route<KIND, XT, LT, V>), dim3(1), dim3(256), 0, stream, logits, x, wg, (int)B, (int)E,
                         (int)K, (int)D, ws);
      return check_launch("moe_decode route");
    };
    const int vpl = (int)(E / 64);
    st = vpl == 1 ? route(kind_c<1>{}) : vpl == 2 ? route(kind_c<2>{}) : vpl == 4 ? route(kind_c<4>{})
       : vpl == 8 ? route(kind_c<8>{}) : vpl == 16 ? route(kind_c<16>{}) : route(kind_c<32>{});
    if (st) return st;
  }
  if (phases & 2) {
    const size_t lds = (size_t)moe_tab_bytes<KIND>() + 2 * (16 * row_bytes(KIND, D) + 16);
    auto kern = k_moe_gate_up<KIND, KIND_DOWN, XT, TPG>;
    if (lds + static_lds(kern) > LDS_BYTES) return fail(E_UNSUPPORTED, "moe_decode: %zu bytes of LDS", lds);
    hipLaunchKernelGGL(kern, dim3((unsigned)(F / 16), (unsigned)(B * K + 1)), dim3(256), lds, stream, gate, up, sg,
                       su, (int)E, (int)K, (int)B, (int)D, (int)F, stab, ws);
    st = check_launch("moe_decode gate_up");
    if (st) return st;
  }
  if (phases & 4) {
    const int64_t rbd = row_bytes(KIND_DOWN, F);
    const size_t slot = (size_t)(((15 + 16 * rbd + 15) >> 4) << 4);
    // as many groups a chunk as two chunks' slices fit beside the kernel's own LDS
    auto kern = k_moe_down<KIND_DOWN, XT, TPG>;
    const size_t used = static_lds(kern) + (size_t)moe_tab_bytes<KIND_DOWN>();
    const size_t room = used < LDS_BYTES ? LDS_BYTES - used : 0;
    const int cg = (int)std::min<size_t>(DOWN_CHUNK_G, room / (2 * slot));
    if (cg < 1) return fail(E_UNSUPPORTED, "moe_decode: down rows of %lld bytes", (long long)rbd);
    const size_t lds = (size_t)moe_tab_bytes<KIND_DOWN>() + 2 * (size_t)cg * slot;
    hipLaunchKernelGGL(kern, dim3((unsigned)(D / 16)), dim3(256), lds, stream, down, sd, (int)E, (int)K, (int)B,
                       (int)D, (int)F, cg, stab, ws, out);
    st = check_launch("moe_decode down");
  }
  return st;
}

}  // namespace sh

using namespace sh;

namespace {

int moe_decode(int phases, int kind, int kind_down, const void* gate, const void* up, const void* down,
                      int64_t experts, const void* shared_gate, const void* shared_up, const void* shared_down,
                      const void* shared_gate_w, const void* tables, const void* logits, int logits_dtype,
                      const void* x, int dtype, int64_t tokens, int64_t k, int64_t d_model, int64_t d_ff, void* out,
                      int32_t* idx_out, float* w_out, void* workspace, size_t workspace_bytes, void* stream) {
  if (tokens <= 0) return OK;
  if (tokens > MOE_MAX_TOKENS || tokens * k > MOE_MAX_PAIRS || k <= 0 || k > 16)
    return fail(E_SHAPE, "moe_decode: %lld tokens of %lld experts (at most %d tokens, %d pairs)", (long long)tokens,
                (long long)k, MOE_MAX_TOKENS, MOE_MAX_PAIRS);
  if (experts <= 0 || vpl_bad(experts) || k > experts)
    return fail(E_SHAPE, "moe_decode: %lld experts (64 times a power of two, at most 2048)", (long long)experts);
  // widths: whole blocks of the kinds that read them (gate / up rows of d_model, down rows of d_ff: 64 weights a
  // Q2_0 block, 256 an IQ3_S one), d_ff in 16-row tiles of gate / up (the reference model's 2560 / 640 with Q2_0 down)
  if (d_model <= 0 || d_ff <= 0 || d_model > MOE_MAX_D || d_model % (kind == IQ3_S ? 256 : 64) ||
      d_ff % (kind_down == IQ3_S ? 256 : 64))
    return fail(E_SHAPE, "moe_decode: widths %lld / %lld (whole blocks of their kinds, d_model at most %d)",
                (long long)d_model, (long long)d_ff, MOE_MAX_D);
  if (!mfma_kind_host(kind) || !mfma_kind_host(kind_down))
    return fail(E_UNSUPPORTED, "moe_decode: kinds %d / %d (the fused step takes Q2_0 and IQ3_S)", kind, kind_down);
  if (!gate || !up || !down || !shared_gate || !shared_up || !shared_down || !shared_gate_w || !logits || !x || !out)
    return fail(E_ARG, "moe_decode: null pointer");
  if ((kind == IQ3_S || kind_down == IQ3_S) && !tables) return fail(E_ARG, "moe_decode: IQ3_S needs the tables");
  const size_t need = moe_carve(nullptr, nullptr, tokens, k, d_model, d_ff, dtype_size(dtype));
  if (!workspace || workspace_bytes < need)
    return fail(E_WORKSPACE, "moe_decode: workspace of %zu bytes, %zu needed", workspace_bytes, need);
  MoeWs ws;
  moe_carve(&ws, (uint8_t*)workspace, tokens, k, d_model, d_ff, dtype_size(dtype));
  // the common shape takes two kernels: route, gate and up (phase bit 8), down and the combine (16); the others
  // the three-kernel path
  const bool aligned = ((uintptr_t)gate | (uintptr_t)up | (uintptr_t)down | (uintptr_t)shared_gate |
                        (uintptr_t)shared_up | (uintptr_t)shared_down | (uintptr_t)x | (uintptr_t)shared_gate_w) % 16 == 0;
  if (experts == FRONT_E && d_model == FRONT_D && d_ff == FRONT_F && aligned) {
    // the whole step in one launch, or (kernel by kernel, or with the one-launch form off) front then tail
    if (phases == 7 && g_one_launch.load(std::memory_order_relaxed))
      phases = 32;
    else
      phases = (phases & 3 ? 8 : 0) | (phases & 4 ? 16 : 0);
  }
  const int tpg = tokens <= 4 ? 1 : tokens <= 8 ? 2 : 4;
  if (logits_dtype != F32 && logits_dtype != dtype)
    return fail(E_DTYPE, "moe_decode: logits of dtype %d with activations of %d (float32 or the same)", logits_dtype, dtype);
  int st = with_half_dtype(dtype, [&](auto* tp) {
    using XT = std::remove_pointer_t<decltype(tp)>;
    auto go = [&](auto kc, auto kd, auto tc) {
      constexpr int K1 = decltype(kc)::value, K2 = decltype(kd)::value, T = decltype(tc)::value;
      if (logits_dtype == F32)
        return launch_moe<K1, K2, XT, float, T>((const uint8_t*)gate, (const uint8_t*)up, (const uint8_t*)down, experts,
                                                (const uint8_t*)shared_gate, (const uint8_t*)shared_up,
                                                (const uint8_t*)shared_down, (const XT*)shared_gate_w,
                                                (const uint8_t*)tables, (const float*)logits, (const XT*)x, tokens, k,
                                                d_model, d_ff, (XT*)out, ws, (hipStream_t)stream, phases);
      return launch_moe<K1, K2, XT, XT, T>((const uint8_t*)gate, (const uint8_t*)up, (const uint8_t*)down, experts,
                                       (const uint8_t*)shared_gate, (const uint8_t*)shared_up,
                                       (const uint8_t*)shared_down, (const XT*)shared_gate_w, (const uint8_t*)tables,
                                       (const XT*)logits, (const XT*)x, tokens, k, d_model, d_ff, (XT*)out, ws,
                                       (hipStream_t)stream, phases);
    };
    auto by_t = [&](auto kc, auto kd) {
      return tpg == 1 ? go(kc, kd, kind_c<1>{}) : tpg == 2 ? go(kc, kd, kind_c<2>{}) : go(kc, kd, kind_c<4>{});
    };
    auto by_down = [&](auto kc) {
      return kind_down == Q2_0 ? by_t(kc, kind_c<Q2_0>{}) : by_t(kc, kind_c<IQ3_S>{});
    };
    return kind == Q2_0 ? by_down(kind_c<Q2_0>{}) : by_down(kind_c<IQ3_S>{});
  });
  if (st) return st;
  if (!(phases & (9 | 32))) return OK;  // the choice comes from the route, the front or the one-launch layer
  if (idx_out && hipMemcpyAsync(idx_out, ws.idx, 4 * tokens * k, hipMemcpyDeviceToDevice, (hipStream_t)stream) != hipSuccess)
    return fail(E_HIP, "moe_decode: copy of the choice failed");
  if (w_out && hipMemcpyAsync(w_out, ws.w, 4 * tokens * k, hipMemcpyDeviceToDevice, (hipStream_t)stream) != hipSuccess)
    return fail(E_HIP, "moe_decode: copy of the weights failed");
  return OK;
}

// ---- the entry point that allocates nothing: its workspace is this file's device array, one copy a GPU

constexpr size_t MOE_SCRATCH_BYTES = (size_t)8 << 20;
static __device__ __align__(256) uint8_t scratch[MOE_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_at[MAX_DEVICES];  // the array's device address on each GPU, found once a GPU

__global__ void k_clear_words(int32_t* p, int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) p[i] = 0;
}

// the current device's copy of `scratch`: its address comes from the runtime (the array's name in host code is a
// stand-in, not a device address), looked up the first time a device calls and kept for it; that first call also
// clears the control words at its head on `stream` (every call after leaves them at zero)
static int scratch_of(void** at, hipStream_t stream) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES)
    return fail(E_HIP, "moe_decode_noalloc: no current device (%d)", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_at[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(E_HIP, "moe_decode_noalloc: address of the scratch array on device %d: %s", dev,
                  hipGetErrorString(e));
    hipLaunchKernelGGL(k_clear_words, dim3(1), dim3(256), 0, stream, (int32_t*)p, (int)(MOE_HEAD_BYTES / 4));
    const int st = check_launch("moe_decode_noalloc clear");
    if (st) return st;
    g_scratch_at[dev] = p;
  }
  *at = g_scratch_at[dev];
  return OK;
}

}  // namespace

extern "C" {

size_t sh_moe_scratch_bytes(void) { return MOE_SCRATCH_BYTES; }

int sh_moe_decode_noalloc(int kind, int kind_down, const void* gate, const void* up, const void* down,
                          int64_t experts, const void* shared_gate, const void* shared_up, const void* shared_down,
                          const void* shared_gate_w, const void* tables, const void* logits, int logits_dtype,
                          const void* x, int dtype, int64_t tokens, int64_t k, int64_t d_model, int64_t d_ff,
                          void* out, int32_t* idx_out, float* w_out, void* stream) {
  if (tokens > 0 && k > 0 && d_model > 0 && d_ff > 0) {
    const size_t need = moe_carve(nullptr, nullptr, tokens, k, d_model, d_ff, dtype_size(dtype));
    if (need > MOE_SCRATCH_BYTES)
      return fail(E_WORKSPACE, "moe_decode_noalloc: %lld tokens x %lld experts at d_model %lld, d_ff %lld need %zu "
                  "bytes of scratch; the library's array holds %zu", (long long)tokens, (long long)k,
                  (long long)d_model, (long long)d_ff, need, MOE_SCRATCH_BYTES);
  }
  if (tokens <= 0) return OK;
  void* ws = nullptr;
  const int st = scratch_of(&ws, (hipStream_t)stream);
  if (st) return st;
  return moe_decode(7, kind, kind_down, gate, up, down, experts, shared_gate, shared_up, shared_down, shared_gate_w,
                    tables, logits, logits_dtype, x, dtype, tokens, k, d_model, d_ff, out, idx_out, w_out, ws,
                    MOE_SCRATCH_BYTES, stream);
}

size_t sh_moe_workspace(int64_t tokens, int64_t k, int64_t d_model, int64_t d_ff, int dtype) {
  if (tokens <= 0 || k <= 0 || d_model <= 0 || d_ff <= 0) return 0;
  return moe_carve(nullptr, nullptr, tokens, k, d_model, d_ff, dtype_size(dtype));
}

int sh_moe_decode(int kind, int kind_down, const void* gate, const void* up, const void* down, int64_t experts,
                  const void* shared_gate, const void* shared_up, const void* shared_down, const void* shared_gate_w,
                  const void* tables, const void* logits, int logits_dtype, const void* x, int dtype, int64_t tokens,
                  int64_t k, int64_t d_model, int64_t d_ff, void* out, int32_t* idx_out, float* w_out, void* workspace,
                  size_t workspace_bytes, void* stream) {
  return moe_decode(7, kind, kind_down, gate, up, down, experts, shared_gate, shared_up, shared_down, shared_gate_w,
                    tables, logits, logits_dtype, x, dtype, tokens, k, d_model, d_ff, out, idx_out, w_out, workspace,
                    workspace_bytes, stream);
}

int sh_moe_set_one_launch(int on) {
  if (on)
    return fail(E_UNSUPPORTED, "moe_set_one_launch: the one-launch layer is switched off (an illegal memory access at "
                "2 tokens; its cause is fixed but the fix has not run on a GPU)");
  return g_one_launch.exchange(0);
}

int sh_moe_set_tail_combine(int upto) {
  if (upto < 0 || upto > MOE_MAX_TOKENS)
    return fail(E_ARG, "moe_set_tail_combine: %d tokens (0 to %d)", upto, MOE_MAX_TOKENS);
  return g_tail_combine_upto.exchange(upto);
}

int sh_moe_decode_phase(int phase, int kind, int kind_down, const void* gate, const void* up, const void* down,
                        int64_t experts, const void* shared_gate, const void* shared_up, const void* shared_down,
                        const void* shared_gate_w, const void* tables, const void* logits, int logits_dtype,
                        const void* x, int dtype, int64_t tokens, int64_t k, int64_t d_model, int64_t d_ff, void* out,
                        void* workspace, size_t workspace_bytes, void* stream) {
  if (phase < 0 || phase > 2) return fail(E_ARG, "moe_decode_phase: phase %d (0 route, 1 gate_up, 2 down)", phase);
  return moe_decode(1 << phase, kind, kind_down, gate, up, down, experts, shared_gate, shared_up, shared_down,
                    shared_gate_w, tables, logits, logits_dtype, x, dtype, tokens, k, d_model, d_ff, out, nullptr,
                    nullptr, workspace, workspace_bytes, stream);
}

}  // extern "C"
