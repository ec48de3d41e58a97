// Expert matvec on MFMA: out[pair, r] = W[idx[pair], r, :] . x[pair / share] for bf16 / fp16 activations, the
// decode path of strata-mlx's BlockSwitchLinear (strata_mlx/blocks.py:196-220, 407-436) rebuilt for CDNA4.
//
// A block of 256 threads takes 16 rows of one expert for the tokens that chose it: pairs sharing an expert are
// grouped in the block itself (up to 128 pairs), so an expert's blocks are read once for every verify token that
// chose it. The 16 rows' bytes, the tokens' activations and (IQ3_S) the signed codebook are staged to LDS with every
// load issued before any store; the 4 waves split the columns and decode straight into MFMA operands (xmv.h).
#include "launch.h"
#include "xmv.h"

namespace sh {

constexpr int XMV_GROUPED_UPTO = 128;  // pairs grouped by expert inside each block; beyond, a block is a pair

struct XmvGroup {
  int chunk, expert, n_tok, zero;
  int xrow[16], orow[16];
};

template <int KIND> constexpr int xmv_tab_bytes() { return KIND == IQ3_S ? IQ3S_SIGNED_BYTES : 0; }

template <int KIND, typename XT, int TPG>
__global__ __launch_bounds__(256) void k_xmv(const uint8_t* __restrict__ blocks, int64_t expert_bytes, int n_experts,
                                             int rows, int cols, int64_t rbytes, const int32_t* __restrict__ idx,
                                             int pairs, const XT* __restrict__ x, int share, XT* __restrict__ out,
                                             const uint8_t* __restrict__ signed_tab) {
  constexpr int NT = 4 * TPG;
  using MT = XT;  // the MFMA element type is the activations' own
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row0 = blockIdx.x * 16;
  const int gy = blockIdx.y;

  __shared__ XmvGroup grp;
  __shared__ int s_e[XMV_GROUPED_UPTO], s_rank[XMV_GROUPED_UPTO], s_chunks[XMV_GROUPED_UPTO];
  __shared__ const XT* s_xrow[NT];
  __shared__ float s_red[4][64][TPG];
  extern __shared__ u32x4 dyn[];
  // dynamic LDS: [signed table][staged x: NT tokens x cols][weights: 16 rows + 16 bytes]
  uint8_t* tab = (uint8_t*)dyn;
  MT* xs = (MT*)((uint8_t*)dyn + xmv_tab_bytes<KIND>());
  uint8_t* wt = (uint8_t*)xs + (size_t)NT * cols * sizeof(MT);

  // 1. which expert and tokens this block serves
  if (pairs <= XMV_GROUPED_UPTO) {
    if (tid < pairs) {
      int e = idx[tid];
      s_e[tid] = (e >= 0 && e < n_experts) ? e : -1;
    }
    __syncthreads();
    if (tid < pairs) {
      int e = s_e[tid], rank = 0, count = 0;
      for (int q = 0; q < pairs; ++q) {
        int same = s_e[q] == e;
        count += same;
        rank += same && q < tid;
      }
      s_rank[tid] = rank;
      s_chunks[tid] = rank == 0 ? (count + NT - 1) / NT : 0;
    }
    __syncthreads();
    if (tid < pairs && s_chunks[tid]) {
      int base = 0;
      for (int q = 0; q < tid; ++q) base += s_chunks[q];
      if (gy >= base && gy < base + s_chunks[tid]) {
        grp.expert = s_e[tid];
        grp.zero = s_e[tid] < 0;
        grp.n_tok = 0;
        grp.chunk = gy - base;  // which NT pairs of this expert's
      }
    }
    if (tid == 0) {
      int g = 0;
      for (int q = 0; q < pairs; ++q) g += s_chunks[q];
      if (gy >= g) grp.expert = -2;  // beyond the groups there are
    }
    __syncthreads();
    if (grp.expert == -2) return;
    if (tid < pairs && s_e[tid] == grp.expert && s_rank[tid] / NT == grp.chunk) {
      int t = s_rank[tid] % NT;
      grp.xrow[t] = tid / share;
      grp.orow[t] = tid;
      atomicAdd(&grp.n_tok, 1);
    }
    __syncthreads();
  } else {
    if (tid == 0) {
      int e = idx[gy];
      grp.zero = !(e >= 0 && e < n_experts);
      grp.expert = grp.zero ? 0 : e;
      grp.n_tok = 1;
      grp.xrow[0] = gy / share;
      grp.orow[0] = gy;
    }
    __syncthreads();
  }
  const int n_tok = grp.n_tok;
  const int rows_here = min(16, rows - row0);
  if (grp.zero) {
    for (int i = tid; i < n_tok * rows_here; i += 256)
      out[(int64_t)grp.orow[i / rows_here] * rows + row0 + i % rows_here] = from_f32<XT>(0.0f);
    return;
  }
  if (tid < n_tok) s_xrow[tid] = x + (int64_t)grp.xrow[tid] * cols;
  __syncthreads();

  // 2. the rows' bytes, the table and the activations to LDS: all loads out before any store
  const uint8_t* src = blocks + (int64_t)grp.expert * expert_bytes + (int64_t)row0 * rbytes;
  ByteStage<4> wst(wt, src, (int)(rows_here * rbytes), tab, signed_tab, xmv_tab_bytes<KIND>());
  XStage<KIND, XT, MT, 4> xst(xs, s_xrow, n_tok, cols);
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
  __syncthreads();

  // 3. this wave's quarter of the columns
  float acc[TPG];
#pragma unroll
  for (int i = 0; i < TPG; ++i) acc[i] = 0.0f;
  const int per = cols / scale_group<KIND>() / 4;
  tile_mac<KIND, MT, TPG>(wt + lead_of(src), (int)rbytes, xs, cols, n_tok, wave * per, (wave + 1) * per,
                          (const uint32_t*)tab, acc);

  // 4. the waves' column quarters summed, one lane a (row, token)
#pragma unroll
  for (int i = 0; i < TPG; ++i) s_red[wave][lane][i] = acc[i];
  __syncthreads();
  if (wave == 0) {
    const int g = lane >> 4, n = lane & 15;
#pragma unroll
    for (int i = 0; i < TPG; ++i) {
      float total = s_red[0][lane][i] + s_red[1][lane][i] + s_red[2][lane][i] + s_red[3][lane][i];
      const int t = g * TPG + i;
      if (t < n_tok && n < rows_here) out[(int64_t)grp.orow[t] * rows + row0 + n] = from_f32<XT>(total);
    }
  }
}

// the kinds and shapes the MFMA path takes
inline bool xmv_takes(int kind, int64_t cols, int dt) {
  if (dt != BF16 && dt != F16) return false;
  if (kind == Q2_0) return cols % 256 == 0;
  if (kind == IQ3_S) return cols % 256 == 0;  // runs split evenly over the 4 waves
  return false;
}

template <int KIND, typename XT, int TPG>
static int launch_xmv(const uint8_t* blocks, const uint8_t* tables, int64_t n_experts, int64_t rows, int64_t cols,
                      const int32_t* idx, int64_t pairs, const XT* x, int64_t share, XT* out, hipStream_t stream) {
  size_t lds = (size_t)xmv_tab_bytes<KIND>() + (size_t)4 * TPG * cols * sizeof(XT) + 16 * row_bytes(KIND, cols) + 16;
  if (lds > 160 * 1024) return fail(E_UNSUPPORTED, "switch_matvec: %zu bytes of LDS for rows of %lld", lds, (long long)cols);
  dim3 grid((unsigned)((rows + 15) / 16), (unsigned)pairs);
  hipLaunchKernelGGL((k_xmv<KIND, XT, TPG>), grid, dim3(256), lds, stream, blocks, rows * row_bytes(KIND, cols),
                     (int)n_experts, (int)rows, (int)cols, row_bytes(KIND, cols), idx, (int)pairs, x, (int)share, out,
                     tables ? tables + TAB_IQ3S_SIGNED : nullptr);
  return check_launch("switch_matvec");
}

}  // namespace sh

using namespace sh;

extern "C" int sh_switch_matvec_generic(int kind, const void* blocks, const void* const* expert_ptrs, const void* tables,
                                        int64_t n_experts, int64_t rows, int64_t cols, const int32_t* idx,
                                        int64_t pairs, const void* x, int x_dtype, int64_t share, void* out,
                                        void* stream);

extern "C" {

size_t sh_switch_workspace(int kind, int64_t rows, int64_t cols, int64_t pairs, int x_dtype) { return 0; }

int sh_switch_matvec(int kind, const void* blocks, const void* tables, int64_t n_experts, int64_t rows, int64_t cols,
                     const int32_t* idx, int64_t pairs, const void* x, int x_dtype, int64_t share, void* out,
                     void* workspace, size_t workspace_bytes, void* stream) {
  int st = check_rows(kind, rows, cols, "switch_matvec");
  if (st) return st;
  if (pairs <= 0) return OK;
  if (pairs > 65535) return fail(E_SHAPE, "switch_matvec: %lld pairs (at most 65535 a call)", (long long)pairs);
  if (share <= 0) return fail(E_ARG, "switch_matvec: share %lld", (long long)share);
  if (!blocks || !idx || !x || !out || (needs_tables(kind) && !tables)) return fail(E_ARG, "switch_matvec: null pointer");
  if (!xmv_takes(kind, cols, x_dtype))
    return sh_switch_matvec_generic(kind, blocks, nullptr, tables, n_experts, rows, cols, idx, pairs, x, x_dtype, share,
                                    out, stream);
  // tokens a group holds: 4, 8 or 16, by how many pairs could share an expert
  int64_t most_per_expert = pairs <= XMV_GROUPED_UPTO ? pairs : 1;
  int tpg = most_per_expert <= 4 ? 1 : most_per_expert <= 8 ? 2 : 4;
  return with_half_dtype(x_dtype, [&](auto* tp) {
    using XT = std::remove_pointer_t<decltype(tp)>;
    auto go = [&](auto kc, auto tc) {
      constexpr int K = decltype(kc)::value, T = decltype(tc)::value;
      return launch_xmv<K, XT, T>((const uint8_t*)blocks, (const uint8_t*)tables, n_experts, rows, cols, idx, pairs,
                                  (const XT*)x, share, (XT*)out, (hipStream_t)stream);
    };
    auto by_tpg = [&](auto kc) {
      return tpg == 1 ? go(kc, kind_c<1>{}) : tpg == 2 ? go(kc, kind_c<2>{}) : go(kc, kind_c<4>{});
    };
    return kind == Q2_0 ? by_tpg(kind_c<Q2_0>{}) : by_tpg(kind_c<IQ3_S>{});
  });
}

}  // extern "C"
