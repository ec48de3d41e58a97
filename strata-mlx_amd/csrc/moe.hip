// One MoE block's decode step for a window of B <= 16 tokens, in three kernels — the path of strata-mlx's
// `_Routed.__call__` (strata_mlx/fused.py:484-497) with its routed experts through switch_glu's bf16 branch
// (strata_mlx/blocks.py:819-829) and its end in `moe_combine` (fused.py:448-481):
//
//   route     one block: each token's top-k of the router logits (largest first, ties to the lower index), the
//             softmax of the chosen logits, the shared expert's gate logit x . w_g, and the (token, expert) pairs
//             grouped by expert (first occurrence order), the shared expert as one more group of all B tokens
//   gate_up   a block = 16 rows of gate and of up of one group's expert, for the group's tokens; its epilogue
//             rounds gate and up to the activation type and writes swiglu(gate, up) with mlx-lm's roundings
//   down      a block = 16 rows of down, a wave a group; y rounded to the activation type; the last block to finish
//             a row tile (an atomic count) combines: OutT(sum_k y_k w_k) + OutT(OutT(sigmoid(g)) * s)
//
// Grids are sized by the most groups there could be (B*k + 1); blocks past the groups the route found leave at once,
// so nothing waits on the host. Expert blocks are read straight from the GGUF stacks (xmv.h).
#include "launch.h"
#include "xmv.h"

namespace sh {

constexpr int MOE_MAX_TOKENS = 16;
constexpr int MOE_MAX_PAIRS = 256;  // tokens * k

// the workspace, carved from one caller buffer
struct MoeWs {
  int32_t* n_groups;  // [1]
  int32_t* g_expert;  // [G]: expert, or `experts` for the shared expert
  int32_t* g_ntok;    // [G]
  int32_t* g_pair;    // [G][16]: pair t*k + j, or B*k + t for the shared expert's token t
  int32_t* idx;       // [B][k]
  float* w;           // [B][k]
  float* gsh;         // [B]: the shared expert's gate logit, rounded to the activation type
  int32_t* counter;   // [D / 16]: blocks of down done with a row tile
  uint8_t* h;         // [B*k + B][F] activation type
  uint8_t* y;         // [B*k + B][D] activation type
};

static inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

static size_t moe_carve(MoeWs* ws, uint8_t* base, int64_t B, int64_t k, int64_t D, int64_t F, int es) {
  const int64_t G = B * k + 1, P = B * k + B;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    uint8_t* p = base ? base + off : nullptr;
    off = align256(off + bytes);
    return p;
  };
  MoeWs w;
  w.n_groups = (int32_t*)take(4);
  w.g_expert = (int32_t*)take(4 * G);
  w.g_ntok = (int32_t*)take(4 * G);
  w.g_pair = (int32_t*)take(4 * 16 * G);
  w.idx = (int32_t*)take(4 * B * k);
  w.w = (float*)take(4 * B * k);
  w.gsh = (float*)take(4 * B);
  w.counter = (int32_t*)take(4 * (D / 16));
  w.h = take((size_t)P * F * es);
  w.y = take((size_t)P * D * es);
  if (ws) *ws = w;
  return off;
}

// ---- route

// Route keys: a logit in an order-preserving unsigned form above the complement of its index, so the largest key
// is the largest logit and, among equal logits, the lowest index. 16-bit logits make 32-bit keys; float32 64-bit.
template <typename LT> struct RouteKey {
  using type = uint32_t;
  __device__ static __forceinline__ uint32_t make(LT v, int i) {
    uint32_t b = __builtin_bit_cast(uint16_t, v);
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

template <typename XT, typename LT>
__global__ __launch_bounds__(256) void k_moe_route(const LT* __restrict__ logits, const XT* __restrict__ x,
                                                   const XT* __restrict__ wg, int B, int E, int K, int D, MoeWs ws) {
  using RK = RouteKey<LT>;
  using key_t = typename RK::type;
  __shared__ int s_idx[MOE_MAX_PAIRS];
  __shared__ int s_first[MOE_MAX_PAIRS], s_gid[MOE_MAX_PAIRS], s_rank[MOE_MAX_PAIRS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int vpl = E >> 6;  // E a multiple of 64, at most 2048
  for (int i = tid; i < D / 16; i += 256) ws.counter[i] = 0;

  for (int t = wave; t < B; t += 4) {
    key_t key[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) key[i] = i < vpl ? RK::make(logits[(int64_t)t * E + i * 64 + lane], i * 64 + lane) : 0;
    float top = 0.0f, sum = 0.0f, my_e = 0.0f;
    int my_idx = 0;
    for (int r = 0; r < K; ++r) {
      key_t best = 0;
#pragma unroll
      for (int i = 0; i < 32; ++i) best = key[i] > best ? key[i] : best;
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
      for (int i = 0; i < 32; ++i)
        if (key[i] == best) key[i] = 0;
    }
    if (lane < K) {
      ws.w[t * K + lane] = my_e / sum;
      ws.idx[t * K + lane] = my_idx;
    }
    // the shared expert's gate logit, rounded to the activation type (a Linear(d, 1) in mlx-lm)
    float acc = 0.0f;
    for (int c = lane; c < D; c += 64) acc = fmaf(to_f32(x[(int64_t)t * D + c]), to_f32(wg[c]), acc);
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
    if (s_rank[tid] == 0) ws.g_expert[gid] = s_idx[tid];
  }
  __syncthreads();
  if (tid < P && s_first[tid] == tid) {
    int count = 0;
    for (int q = 0; q < P; ++q) count += s_first[q] == tid;
    ws.g_ntok[s_gid[tid]] = count;
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

// ---- gate and up, SwiGLU in the epilogue


template <int KIND> constexpr int moe_tab_bytes() { return KIND == IQ3_S ? IQ3S_SIGNED_BYTES : 0; }

template <int KIND, typename XT, int TPG>
__global__ __launch_bounds__(256) void k_moe_gate_up(const uint8_t* __restrict__ gate, const uint8_t* __restrict__ up,
                                                     const uint8_t* __restrict__ sh_gate, const uint8_t* __restrict__ sh_up,
                                                     int E, int K, int B, int D, int F, const XT* __restrict__ x,
                                                     const uint8_t* __restrict__ signed_tab, MoeWs ws) {
  constexpr int NT = 4 * TPG;
  using MT = XT;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row0 = blockIdx.x * 16, gy = blockIdx.y;
  __shared__ int s_n, s_e, s_pair[NT];
  __shared__ const XT* s_xrow[NT];
  __shared__ float s_red[2][4][64][TPG];
  extern __shared__ u32x4 dyn[];
  uint8_t* tab = (uint8_t*)dyn;
  MT* xs = (MT*)(tab + moe_tab_bytes<KIND>());
  const int64_t rb = row_bytes_dev(KIND, D);
  uint8_t* wg = (uint8_t*)(xs + NT * D);
  uint8_t* wu = wg + 16 * rb + 16;
  if (tid == 0) {
    const int groups = *ws.n_groups;
    s_n = gy < groups ? ws.g_ntok[gy] : 0;
    s_e = gy < groups ? ws.g_expert[gy] : 0;
  }
  __syncthreads();
  const int n_tok = s_n, e = s_e;
  if (n_tok == 0) return;
  if (tid < n_tok) {
    const int p = ws.g_pair[gy * 16 + tid];
    s_pair[tid] = p;
    s_xrow[tid] = x + (int64_t)(p < B * K ? p / K : p - B * K) * D;
  }
  __syncthreads();
  const int64_t ebytes = (int64_t)F * rb;
  const uint8_t* g_src = (e == E ? sh_gate : gate + (int64_t)e * ebytes) + (int64_t)row0 * rb;
  const uint8_t* u_src = (e == E ? sh_up : up + (int64_t)e * ebytes) + (int64_t)row0 * rb;
  ByteStage<4> wst(wg, g_src, (int)(16 * rb), wu, u_src, (int)(16 * rb));
  XStage<KIND, XT, MT, 4> xst(xs, s_xrow, n_tok, D);
  wst.load(0, tid, 256);
  xst.load(0, tid, 256);
  wst.store(0, tid, 256);
  xst.store(0, tid, 256);
  for (int p = 1; p < wst.passes(256); ++p) {
    wst.load(p, tid, 256);
    wst.store(p, tid, 256);
  }
  for (int p = 1; p < xst.passes(256); ++p) {
    xst.load(p, tid, 256);
    xst.store(p, tid, 256);
  }
  if constexpr (KIND == IQ3_S) {
    ByteStage<4> tst(tab, signed_tab, IQ3S_SIGNED_BYTES, nullptr, nullptr, 0);
    for (int p = 0; p < tst.passes(256); ++p) {
      tst.load(p, tid, 256);
      tst.store(p, tid, 256);
    }
  }
  __syncthreads();
  float ag[TPG], au[TPG];
#pragma unroll
  for (int i = 0; i < TPG; ++i) ag[i] = au[i] = 0.0f;
  const int per = D / scale_group<KIND>() / 4;
  tile_mac<KIND, MT, TPG>(wg + lead_of(g_src), (int)rb, xs, D, n_tok, wave * per, (wave + 1) * per, (const uint32_t*)tab, ag);
  tile_mac<KIND, MT, TPG>(wu + lead_of(u_src), (int)rb, xs, D, n_tok, wave * per, (wave + 1) * per, (const uint32_t*)tab, au);
#pragma unroll
  for (int i = 0; i < TPG; ++i) {
    s_red[0][wave][lane][i] = ag[i];
    s_red[1][wave][lane][i] = au[i];
  }
  __syncthreads();
  if (wave == 0) {
    const int g = lane >> 4, n = lane & 15;
#pragma unroll
    for (int i = 0; i < TPG; ++i) {
      const int t = g * TPG + i;
      if (t < n_tok) {
        const XT gv = from_f32<XT>(s_red[0][0][lane][i] + s_red[0][1][lane][i] + s_red[0][2][lane][i] + s_red[0][3][lane][i]);
        const XT uv = from_f32<XT>(s_red[1][0][lane][i] + s_red[1][1][lane][i] + s_red[1][2][lane][i] + s_red[1][3][lane][i]);
        ((XT*)ws.h)[(int64_t)s_pair[t] * F + row0 + n] = swiglu_one(gv, uv);
      }
    }
  }
}

// ---- down, a wave a group, and the combine by the last block of a row tile

constexpr int DOWN_GROUPS = 4;

template <int KIND, typename XT, int TPG>
__global__ __launch_bounds__(256) void k_moe_down(const uint8_t* __restrict__ down, const uint8_t* __restrict__ sh_down,
                                                  int E, int K, int B, int D, int F,
                                                  const uint8_t* __restrict__ signed_tab, MoeWs ws, XT* __restrict__ out) {
#pragma clang fp contract(off)
  constexpr int NT = 4 * TPG;
  using MT = XT;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row0 = blockIdx.x * 16, by = blockIdx.y;
  __shared__ int s_groups, s_n[DOWN_GROUPS], s_e[DOWN_GROUPS], s_pair[DOWN_GROUPS][NT], s_last;
  __shared__ const XT* s_xrow[DOWN_GROUPS][NT];
  extern __shared__ u32x4 dyn[];
  uint8_t* tab = (uint8_t*)dyn;
  const int64_t rb = row_bytes_dev(KIND, F);
  const size_t wave_bytes = (size_t)NT * F * sizeof(MT) + ((16 * rb + 16 + 15) & ~(int64_t)15);
  uint8_t* mine = tab + moe_tab_bytes<KIND>() + wave * wave_bytes;
  MT* xs = (MT*)mine;
  uint8_t* wt = mine + (size_t)NT * F * sizeof(MT);
  if (tid == 0) s_groups = *ws.n_groups;
  __syncthreads();
  const int groups = s_groups;
  const int first = by * DOWN_GROUPS;
  if (first >= groups) return;
  if (tid < DOWN_GROUPS) {
    const int gi = first + tid;
    s_n[tid] = gi < groups ? ws.g_ntok[gi] : 0;
    s_e[tid] = gi < groups ? ws.g_expert[gi] : 0;
  }
  __syncthreads();
  if (tid < DOWN_GROUPS * NT) {
    const int w = tid / NT, t = tid % NT;
    if (t < s_n[w]) {
      const int p = ws.g_pair[(first + w) * 16 + t];
      s_pair[w][t] = p;
      s_xrow[w][t] = (const XT*)ws.h + (int64_t)p * F;
    }
  }
  __syncthreads();
  const int n_tok = s_n[wave], e = s_e[wave];
  const uint8_t* src = (e == E ? sh_down : down + (int64_t)e * D * rb) + (int64_t)row0 * rb;
  ByteStage<4> wst(wt, src, n_tok ? (int)(16 * rb) : 0, nullptr, nullptr, 0);
  XStage<KIND, XT, MT, 8> xst(xs, s_xrow[wave], n_tok, F);
  wst.load(0, lane, 64);
  xst.load(0, lane, 64);
  wst.store(0, lane, 64);
  xst.store(0, lane, 64);
  for (int p = 1; p < wst.passes(64); ++p) {
    wst.load(p, lane, 64);
    wst.store(p, lane, 64);
  }
  for (int p = 1; p < xst.passes(64); ++p) {
    xst.load(p, lane, 64);
    xst.store(p, lane, 64);
  }
  if constexpr (KIND == IQ3_S) {
    ByteStage<4> tst(tab, signed_tab, IQ3S_SIGNED_BYTES, nullptr, nullptr, 0);
    for (int p = 0; p < tst.passes(256); ++p) {
      tst.load(p, tid, 256);
      tst.store(p, tid, 256);
    }
  }
  __syncthreads();
  if (n_tok) {
    float acc[TPG];
#pragma unroll
    for (int i = 0; i < TPG; ++i) acc[i] = 0.0f;
    tile_mac<KIND, MT, TPG>(wt + lead_of(src), (int)rb, xs, F, n_tok, 0, F / scale_group<KIND>(), (const uint32_t*)tab, acc);
    const int g = lane >> 4, n = lane & 15;
#pragma unroll
    for (int i = 0; i < TPG; ++i) {
      const int t = g * TPG + i;
      if (t < n_tok) ((XT*)ws.y)[(int64_t)s_pair[wave][t] * D + row0 + n] = from_f32<XT>(acc[i]);
    }
  }
  // the last block of this row tile to finish combines it
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const int batches = (groups + DOWN_GROUPS - 1) / DOWN_GROUPS;
    s_last = atomicAdd(&ws.counter[blockIdx.x], 1) == batches - 1;
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  if (tid == 0) ws.counter[blockIdx.x] = 0;
  if (tid < B * 16) {
    const int t = tid >> 4, n = tid & 15, col = row0 + n;
    const XT* y = (const XT*)ws.y;
    float acc = 0.0f;
    for (int j = 0; j < 8 && j < K; ++j) {
      float part = 0.0f;
      for (int kk = j; kk < K; kk += 8) {
        const float prod = to_f32(y[(int64_t)(t * K + kk) * D + col]) * ws.w[t * K + kk];
        part = prod + part;
      }
      acc = j == 0 ? part : part + acc;
    }
    const XT routed = from_f32<XT>(acc);
    const XT gate = from_f32<XT>(1.0f / (1.0f + expf(-ws.gsh[t])));
    const XT shared = from_f32<XT>(to_f32(gate) * to_f32(y[(int64_t)(B * K + t) * D + col]));
    out[(int64_t)t * D + col] = from_f32<XT>(to_f32(routed) + to_f32(shared));
  }
}

template <int KIND, int KIND_DOWN, typename XT, typename LT, int TPG>
static int launch_moe(const uint8_t* gate, const uint8_t* up, const uint8_t* down, int64_t E, const uint8_t* sg,
                      const uint8_t* su, const uint8_t* sd, const XT* wg, const uint8_t* tables, const LT* logits,
                      const XT* x, int64_t B, int64_t K, int64_t D, int64_t F, XT* out, const MoeWs& ws,
                      hipStream_t stream, int phases) {
  constexpr int NT = 4 * TPG;
  const uint8_t* stab = tables ? tables + TAB_IQ3S_SIGNED : nullptr;
  int st = OK;
  if (phases & 1) {
    hipLaunchKernelGGL((k_moe_route<XT, LT>), dim3(1), dim3(256), 0, stream, logits, x, wg, (int)B, (int)E, (int)K, (int)D, ws);
    st = check_launch("moe_decode route");
    if (st) return st;
  }
  if (!(phases & 2)) goto down_phase;
  {
  const size_t lds_gu = (size_t)moe_tab_bytes<KIND>() + (size_t)NT * D * sizeof(XT) + 2 * (16 * row_bytes(KIND, D) + 16);
  hipLaunchKernelGGL((k_moe_gate_up<KIND, XT, TPG>), dim3((unsigned)(F / 16), (unsigned)(B * K + 1)), dim3(256), lds_gu,
                     stream, gate, up, sg, su, (int)E, (int)K, (int)B, (int)D, (int)F, x, stab, ws);
  st = check_launch("moe_decode gate_up");
  if (st) return st;
  }
down_phase:
  if (!(phases & 4)) return OK;
  {
  const size_t wave_bytes = (size_t)NT * F * sizeof(XT) + ((16 * row_bytes(KIND_DOWN, F) + 16 + 15) & ~(int64_t)15);
  const size_t lds_d = (size_t)moe_tab_bytes<KIND_DOWN>() + 4 * wave_bytes;
  const unsigned batches = (unsigned)((B * K + 1 + DOWN_GROUPS - 1) / DOWN_GROUPS);
  hipLaunchKernelGGL((k_moe_down<KIND_DOWN, XT, TPG>), dim3((unsigned)(D / 16), batches), dim3(256), lds_d, stream, down,
                     sd, (int)E, (int)K, (int)B, (int)D, (int)F, stab, ws, out);
  return check_launch("moe_decode down");
  }
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
  if (experts <= 0 || experts % 64 || experts > 2048 || k > experts)
    return fail(E_SHAPE, "moe_decode: %lld experts (a multiple of 64, at most 2048)", (long long)experts);
  if (d_model % 256 || d_ff % 256 || d_model <= 0 || d_ff <= 0)
    return fail(E_SHAPE, "moe_decode: widths %lld / %lld (multiples of 256)", (long long)d_model, (long long)d_ff);
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
  if (!(phases & 1)) return OK;
  if (idx_out && hipMemcpyAsync(idx_out, ws.idx, 4 * tokens * k, hipMemcpyDeviceToDevice, (hipStream_t)stream) != hipSuccess)
    return fail(E_HIP, "moe_decode: copy of the choice failed");
  if (w_out && hipMemcpyAsync(w_out, ws.w, 4 * tokens * k, hipMemcpyDeviceToDevice, (hipStream_t)stream) != hipSuccess)
    return fail(E_HIP, "moe_decode: copy of the weights failed");
  return OK;
}

}  // namespace

extern "C" {

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
