// Streaming matvec over a stack of matrices: out[m][t] = W_m . x[m][t] for n_mats matrices of GGUF blocks and up to
// 16 tokens each, bf16 / fp16 activations — strata-mlx's window matvec (strata_mlx/blocks.py:351-394: one layer, a
// window of T <= 8 tokens, each run unpacked once for all of them) taken over many matrices in one launch, the form
// in which a decode pass streams its weights.
//
// A persistent grid; an item is IR = 16 * WAVES / KW rows of one matrix (WAVES / KW waves take 16 rows each, KW
// waves split the columns) and a block takes a contiguous run of items. A block stages its matrix's activations in
// LDS in the order the MFMA fragments take them, with the sums the magic-number decode's offsets add (XStageCorr),
// again only when the matrix changes. The next item's weight bytes (and activations, at a change of matrix) are
// loaded into registers while this item multiplies from LDS, then stored over it: one LDS buffer, the registers the
// second. Two shapes: streaming (64-row items) for many matrices, and 16-row items split four ways for few.
#include <type_traits>

#include "launch.h"
#include "xmv.h"

namespace sh {

template <int KIND, typename XT, int TPG, int WAVES, int KW, int UW, int UX>
__global__ __launch_bounds__(WAVES * 64) void k_stack_mv(const uint8_t* __restrict__ blocks, int64_t mat_bytes,
                                                         int rows, int cols, int64_t rbytes, const XT* __restrict__ x,
                                                         int tokens, XT* __restrict__ out,
                                                         const uint8_t* __restrict__ signed_tab, int n_items) {
  using MT = XT;
  constexpr int NT = WAVES * 64, RG = WAVES / KW, IR = 16 * RG;
  constexpr int TAB = KIND == IQ3_S ? IQ3S_SIGNED_BYTES : 0;
  __shared__ float s_red[KW][RG][64][TPG];
  extern __shared__ u32x4 dyn[];
  const int ngroups = cols / scale_group<KIND>();
  uint8_t* tab = (uint8_t*)dyn;
  MT* xs = (MT*)(tab + TAB);
  float* corr = (float*)(xs + (size_t)tokens * cols);
  uint8_t* wt = (uint8_t*)(corr + ((tokens * ngroups + 3) & ~3));
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rg = wave % RG, kh = wave / RG;
  const int items_per_mat = (rows + IR - 1) / IR;
  const int gper = ngroups / KW;

  const int per = (n_items + gridDim.x - 1) / gridDim.x;
  const int first = blockIdx.x * per, last = min(n_items, first + per);
  if (first >= last) return;
  auto src_of = [&](int item, int& nbytes) {
    const int m = item / items_per_mat, r0 = (item - m * items_per_mat) * IR;
    nbytes = (int)(min(IR, rows - r0) * rbytes);
    return blocks + (int64_t)m * mat_bytes + (int64_t)r0 * rbytes;
  };
  int nb;
  const uint8_t* src = src_of(first, nb);
  int m = first / items_per_mat;
  {
    ByteStage<UW> st(wt, src, nb, tab, signed_tab, TAB);
    XStageCorr<KIND, XT, MT, UX> xst(xs, corr, x + (int64_t)m * tokens * cols, tokens, cols);
    st.load(0, tid, NT);
    xst.load(0, tid, NT);
    st.store(0, tid, NT);
    xst.store(0, tid, NT);
    for (int p = 1; p < st.passes(NT); ++p) {
      st.load(p, tid, NT);
      st.store(p, tid, NT);
    }
    for (int p = 1; p < xst.passes(NT); ++p) {
      xst.load(p, tid, NT);
      xst.store(p, tid, NT);
    }
  }
  __syncthreads();
  for (int item = first; item < last; ++item) {
    const bool more = item + 1 < last;
    int nb_next = 0;
    const uint8_t* src_next = more ? src_of(item + 1, nb_next) : src;
    const int m_next = more ? (item + 1) / items_per_mat : m;
    ByteStage<UW> nw(wt, src_next, nb_next, nullptr, nullptr, 0);
    XStageCorr<KIND, XT, MT, UX> nxs(xs, corr, x + (int64_t)m_next * tokens * cols, m_next != m ? tokens : 0, cols);
    const bool w1 = nw.passes(NT) <= 1, x1 = nxs.passes(NT) <= 1;
    if (w1) nw.load(0, tid, NT);  // in flight while this item multiplies
    if (x1) nxs.load(0, tid, NT);

    const int r0 = (item - m * items_per_mat) * IR;
    const int rows_here = min(IR, rows - r0);
    float acc[TPG];
#pragma unroll
    for (int t = 0; t < TPG; ++t) acc[t] = 0.0f;
    if (rg * 16 < rows_here)
      tile_mac_lds<KIND, MT, TPG>(wt + lead_of(src) + (size_t)rg * 16 * rbytes, (int)rbytes, xs, corr, cols, ngroups,
                                  tokens, kh * gper, (kh + 1) * gper, (const uint32_t*)tab, acc);
    if constexpr (KW > 1) {
#pragma unroll
      for (int t = 0; t < TPG; ++t) s_red[kh][rg][lane][t] = acc[t];
    }
    __syncthreads();  // every wave is done with this item's bytes (and has left its partial sums)
    if (kh == 0 && rg * 16 < rows_here) {
      const int g = lane >> 4, n = lane & 15;
#pragma unroll
      for (int t = 0; t < TPG; ++t) {
        float total = acc[t];
        if constexpr (KW > 1) {
#pragma unroll
          for (int k2 = 1; k2 < KW; ++k2) total += s_red[k2][rg][lane][t];
        }
        const int tok = g * TPG + t, row = r0 + rg * 16 + n;
        if (tok < tokens && row < rows) out[((int64_t)m * tokens + tok) * rows + row] = from_f32<XT>(total);
      }
    }
    if (more) {
      if (w1) {
        nw.store(0, tid, NT);
      } else {
        for (int p = 0; p < nw.passes(NT); ++p) {
          nw.load(p, tid, NT);
          nw.store(p, tid, NT);
        }
      }
      if (x1) {
        nxs.store(0, tid, NT);
      } else {
        for (int p = 0; p < nxs.passes(NT); ++p) {
          nxs.load(p, tid, NT);
          nxs.store(p, tid, NT);
        }
      }
    }
    src = src_next;
    m = m_next;
    __syncthreads();
  }
}

// launch shapes: waves a block, waves splitting the columns, 16-byte weight loads a thread, activation vectors a thread
template <int KIND, bool STREAM, int TPG> struct StackShape;
template <int TPG> struct StackShape<Q2_0, true, TPG> { static constexpr int WAVES = 4, KW = 1, UW = 10, UX = 4 * TPG; };
template <int TPG> struct StackShape<Q2_0, false, TPG> { static constexpr int WAVES = 4, KW = 4, UW = 3, UX = 4 * TPG; };
template <int TPG> struct StackShape<IQ3_S, true, TPG> { static constexpr int WAVES = 8, KW = 2, UW = 8, UX = 2 * TPG; };
template <int TPG> struct StackShape<IQ3_S, false, TPG> { static constexpr int WAVES = 4, KW = 4, UW = 4, UX = 4 * TPG; };

static int device_cus() {
  static int cus = 0;
  if (!cus) {
    int dev = 0;
    (void)hipGetDevice(&dev);
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (cus <= 0) cus = 256;
  }
  return cus;
}

template <int KIND, bool STREAM, typename XT, int TPG>
static int launch_stack(const uint8_t* blocks, const uint8_t* tables, int64_t n_mats, int64_t rows, int64_t cols,
                        const XT* x, int64_t tokens, XT* out, hipStream_t stream) {
  using S = StackShape<KIND, STREAM, TPG>;
  constexpr int IR = 16 * S::WAVES / S::KW;
  const int64_t rb = row_bytes(KIND, cols);
  const int64_t ngroups = cols / (KIND == Q2_0 ? 64 : 32);
  const int64_t items = n_mats * ((rows + IR - 1) / IR);
  const size_t lds = (size_t)(KIND == IQ3_S ? IQ3S_SIGNED_BYTES : 0) + (size_t)tokens * cols * sizeof(XT) +
                     (size_t)((tokens * ngroups + 3) & ~3) * 4 + (size_t)IR * rb + 16;
  if (lds > 160 * 1024) return fail(E_UNSUPPORTED, "stack_matvec: %zu bytes of LDS", lds);
  auto kern = k_stack_mv<KIND, XT, TPG, S::WAVES, S::KW, S::UW, S::UX>;
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, S::WAVES * 64, lds) != hipSuccess || per_cu < 1)
    per_cu = 1;
  const int64_t grid = std::min<int64_t>(items, (int64_t)device_cus() * per_cu);
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(S::WAVES * 64), lds, stream, blocks, rows * rb, (int)rows,
                     (int)cols, rb, x, (int)tokens, out, tables ? tables + TAB_IQ3S_SIGNED : nullptr, (int)items);
  return check_launch("stack_matvec");
}

}  // namespace sh

using namespace sh;

extern "C" {

size_t sh_stack_workspace(int kind, int64_t n_mats, int64_t rows, int64_t cols, int64_t tokens, int x_dtype) {
  return 0;
}

int sh_stack_matvec(int kind, const void* blocks, const void* tables, int64_t n_mats, int64_t rows, int64_t cols,
                    const void* x, int x_dtype, int64_t tokens, void* out, void* workspace, size_t workspace_bytes,
                    void* stream) {
  int st = check_rows(kind, rows, cols, "stack_matvec");
  if (st) return st;
  if (n_mats <= 0 || tokens <= 0) return OK;
  if (tokens > 16) return fail(E_SHAPE, "stack_matvec: %lld tokens a matrix (at most 16)", (long long)tokens);
  if (n_mats * ((rows + 15) / 16) > (1ll << 31) - 1)
    return fail(E_SHAPE, "stack_matvec: %lld matrices too many", (long long)n_mats);
  if (!mfma_kind_host(kind) || (x_dtype != BF16 && x_dtype != F16) || cols % 256)
    return fail(E_UNSUPPORTED, "stack_matvec: kind %d, dtype %d, %lld columns (Q2_0 / IQ3_S, bf16 / fp16, columns a "
                "multiple of 256)", kind, x_dtype, (long long)cols);
  if (!blocks || !x || !out || (kind == IQ3_S && !tables)) return fail(E_ARG, "stack_matvec: null pointer");
  const int tpg = tokens <= 4 ? 1 : tokens <= 8 ? 2 : 4;
  // many items to go round: 64-row items streamed; few: 16-row items with the columns split four ways
  const bool stream_shape = n_mats * ((rows + 63) / 64) >= 2 * (int64_t)device_cus();
  return with_half_dtype(x_dtype, [&](auto* tp) {
    using XT = std::remove_pointer_t<decltype(tp)>;
    auto go = [&](auto kc, auto sc, auto tc) {
      constexpr int K = decltype(kc)::value, T = decltype(tc)::value;
      constexpr bool S = decltype(sc)::value != 0;
      return launch_stack<K, S, XT, T>((const uint8_t*)blocks, (const uint8_t*)tables, n_mats, rows, cols,
                                       (const XT*)x, tokens, (XT*)out, (hipStream_t)stream);
    };
    auto by_t = [&](auto kc, auto sc) {
      return tpg == 1 ? go(kc, sc, kind_c<1>{}) : tpg == 2 ? go(kc, sc, kind_c<2>{}) : go(kc, sc, kind_c<4>{});
    };
    auto by_s = [&](auto kc) { return stream_shape ? by_t(kc, kind_c<1>{}) : by_t(kc, kind_c<0>{}); };
    return kind == Q2_0 ? by_s(kind_c<Q2_0>{}) : by_s(kind_c<IQ3_S>{});
  });
}

}  // extern "C"
