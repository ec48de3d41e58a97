// Streaming matvec over a stack of matrices: out[m][t] = W_m . x[m][t] for n_mats matrices of GGUF blocks and up to
// 16 tokens each, bf16 / fp16 activations — strata-mlx's window matvec (strata_mlx/blocks.py:351-394: one layer, a
// window of T <= 8 tokens, each run unpacked once for all of them) taken over many matrices in one launch, the form
// in which a decode pass streams its weights.
//
// A block is RG x KW waves: RG row groups of 16 rows, the columns split KW ways, each wave owning GPER scale groups
// of every row it multiplies. An item is IR = 16 * RG rows of one matrix; a block takes a contiguous run of items
// and keeps NBUF of them in an LDS ring, filled by direct 16-byte loads into LDS (no registers, no stores), so
// NBUF - 1 items are in flight while one is multiplied. Rows sit in LDS at a stride padded (when a row is whole
// 16-byte chunks) so the 16 rows a wave reads fall in distinct banks.
//
// A wave's activation fragments for its columns, and minus the sums the magic-number decode's offsets add, live in
// registers, loaded from global memory once per matrix: the multiply reads only weight bytes from LDS (three 16-bit
// reads a Q2_0 block), fully unrolled over the wave's GPER groups. An IQ3_S block also holds the 32 KiB table of
// signed grid entries in LDS.
#include <type_traits>

#include "launch.h"
#include "regmac.h"
#include "xmv.h"

namespace sh {

constexpr int STACK_LMAX = 6;  // direct loads a thread an item, at most

// one launch's shape, shared by host and device through the kernel arguments
struct StackPlan {
  int rows, cols, tokens, ngroups;
  int64_t rbytes, mat_bytes;
  int items, items_per_mat, rstride, padded, loads, nbuf;  // loads: direct loads a thread an item
  int rg, kw, nw;                                          // row groups, column splits, waves (rg * kw)
  int ring_off, buf_bytes, red_off;                        // LDS byte offsets and sizes
};

template <int KIND, typename XT, int TPG, int GPER, int NWMAX, int RW>
__global__ __launch_bounds__(NWMAX * 64) void k_stack_mv(const uint8_t* __restrict__ blocks, StackPlan P,
                                                        const XT* __restrict__ x, XT* __restrict__ out,
                                                        const uint8_t* __restrict__ signed_tab) {
  using MT = XT;
  extern __shared__ u32x4 dyn[];
  uint8_t* lds = (uint8_t*)dyn;
  const uint32_t lds_base = SH_LDS_ADDR(dyn);
  // [2][kw - 1][rg][64][TPG] (RW 2: the splits after the first; the first's wave adds them to its own) or
  // [2][kw][rg][64][TPG] (RW 1: every split; the entries' sums shared out over all waves): the column splits'
  // partial sums of the last two items, read a barrier later
  float* red = (float*)(lds + P.red_off);
  const int red_sz = (RW == 1 ? P.kw : P.kw - 1) * P.rg * 64 * TPG;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // RW 1: wave (r, h) multiplies row group r over column split h; RW 2: wave h both row groups over split h (one
  // set of activation registers for two row groups: fewer registers a row, more waves a SIMD)
  const int rg0 = RW == 1 ? wave % P.rg : 0, kh = RW == 1 ? wave / P.rg : wave;
  const int nt = 64 * P.nw, IR = 16 * P.rg;
  const int wcol = KIND == Q2_0 ? kh * GPER * 18 : (kh * GPER / 8) * 110;  // the wave's first group in a row

  const int per = (P.items + gridDim.x - 1) / gridDim.x;
  const int first = blockIdx.x * per, last = min(P.items, first + per);
  if (first >= last) return;

  // this thread's slot of each of its loads, as a byte offset from the item's first byte (padded layout) or
  // from the 16-byte chunk holding it (packed layout); clamped to the item's last chunk at issue
  int pre[STACK_LMAX];
  const int cpr = P.rstride >> 4, cpr_src = (int)(P.rbytes >> 4);
#pragma unroll
  for (int j = 0; j < STACK_LMAX; ++j) {
    const int s = (j * P.nw + wave) * 64 + lane;
    if (P.padded) {
      const int row = s / cpr, kk = s - row * cpr;
      pre[j] = row * (int)P.rbytes + 16 * min(kk, cpr_src - 1);
    } else {
      pre[j] = 16 * s;
    }
  }
  auto src_of = [&](int item) {
    const int m = item / P.items_per_mat, r0 = (item - m * P.items_per_mat) * IR;
    return blocks + (int64_t)m * P.mat_bytes + (int64_t)r0 * P.rbytes;
  };
  auto issue = [&](int item) {
    const int m = item / P.items_per_mat, r0 = (item - m * P.items_per_mat) * IR;
    const int nb = min(IR, P.rows - r0) * (int)P.rbytes;
    const uint8_t* src = src_of(item);
    const uint8_t* base = P.padded ? src : (const uint8_t*)((uintptr_t)src & ~(uintptr_t)15);
    const int lastc = P.padded ? nb - 16 : ((lead_of(src) + nb - 1) & ~15);
    const uint32_t buf = lds_base + P.ring_off + (item % P.nbuf) * P.buf_bytes + wave * 1024;
#pragma unroll
    for (int j = 0; j < STACK_LMAX; ++j)
      if (j < P.loads) lds_dma16(base, min(pre[j], lastc), buf + j * (nt * 16));
  };

  // the IQ3_S table (whole waves of 64 chunks; a last wave's chunks past the table repeat its last chunk into
  // the ring's first bytes, before the ring is filled), then the ring's first NBUF - 1 items
  if constexpr (KIND == IQ3_S) {
    constexpr int CH = IQ3S_SIGNED_BYTES / 16;
    for (int c0 = wave * 64; c0 < CH; c0 += nt) lds_dma16(signed_tab, 16 * min(c0 + lane, CH - 1), lds_base + 16 * c0);
    wait_vmcnt(0);
  }
  for (int k = 0; k < P.nbuf - 1 && first + k < last; ++k) issue(first + k);

  const DecodeRegs kr = decode_regs<KIND, MT>();
  XRegs<KIND, TPG, GPER> X;
  // An item's results are reduced and stored at the start of the next item, after its barrier (which also makes the
  // other column splits' partial sums visible: one barrier an item) and before its loads are issued (a store counts
  // on vmcnt like a load: issued after an item's loads, the wait for the item before them would wait for part of
  // them too).
  float pend[RW][TPG];
  int64_t pend_at[RW];  // the element of the last item's results for this lane's first token, or -1: none
#pragma unroll
  for (int r = 0; r < RW; ++r) pend_at[r] = -1;
  int pend_buf = 0;
  int fin_m = -1, fin_r0 = 0;  // RW 1: the item whose results are pending, its matrix and first row
  auto finish = [&]() {
    const float* rb = red + pend_buf * red_sz;
    if constexpr (RW == 1) {  // entry e = (row group, lane, token slot) of the item's rg x 64 x TPG: thread e's
      if (fin_m < 0) return;
      const int entries = P.rg * 64 * TPG;
      for (int e = threadIdx.x; e < entries; e += nt) {
        const int t = e % TPG, l = (e / TPG) & 63, r = e / (64 * TPG);
        const int row = fin_r0 + r * 16 + (l & 15), tok = (l >> 4) * TPG + t;
        float total = rb[e];
        for (int k2 = 1; k2 < P.kw; ++k2) total += rb[k2 * entries + e];
        if (tok < P.tokens && row < P.rows) out[((int64_t)fin_m * P.tokens + tok) * P.rows + row] = from_f32<XT>(total);
      }
      return;
    }
    const int g = lane >> 4;
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      if (pend_at[r] < 0) continue;
#pragma unroll
      for (int t = 0; t < TPG; ++t) {
        float total = pend[r][t];
        for (int k2 = 1; k2 < P.kw; ++k2) total += rb[(((k2 - 1) * P.rg + rg0 + r) * 64 + lane) * TPG + t];
        if (g * TPG + t < P.tokens) out[pend_at[r] + (int64_t)t * P.rows] = from_f32<XT>(total);
      }
    }
  };
  int m = -1;
  for (int item = first; item < last; ++item) {
    const int ahead = min(P.nbuf - 2, last - 1 - item);  // items issued after this one
    wait_vmcnt(ahead * P.loads);
    lds_sync();  // this item is in LDS for every wave; every wave is done with the item before
    finish();
    if (item + P.nbuf - 1 < last) issue(item + P.nbuf - 1);
    const int mi = item / P.items_per_mat;
    if (mi != m) {  // a new matrix: this wave's activation fragments and offset sums
      m = mi;
      load_x<KIND, XT, TPG, GPER>(X, x + (int64_t)m * P.tokens * P.cols, P.cols, P.tokens, kh * GPER);
    }
    const int r0 = (item - m * P.items_per_mat) * IR;
    const int rows_here = min(IR, P.rows - r0);
    float acc[RW][TPG];
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
      for (int t = 0; t < TPG; ++t) acc[r][t] = 0.0f;
    const uint8_t* row0 = lds + P.ring_off + (item % P.nbuf) * P.buf_bytes + (P.padded ? 0 : lead_of(src_of(item)));
    // nothing of the LDS / scalar-load counter pending (scalar loads return out of order: with one pending the
    // multiply's reads could only be waited for all at once)
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int r = 0; r < RW; ++r)
      if ((rg0 + r) * 16 < rows_here)
        item_mac<KIND, MT, TPG, GPER>(row0 + (size_t)(rg0 + r) * 16 * P.rstride + wcol, P.rstride, X,
                                      (const uint32_t*)lds, kr, acc[r]);
    if (RW == 1 || kh > 0) {
      const int k0 = RW == 1 ? kh : kh - 1;
#pragma unroll
      for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int t = 0; t < TPG; ++t)
          red[(item & 1) * red_sz + ((k0 * P.rg + rg0 + r) * 64 + lane) * TPG + t] = acc[r][t];
    }
    if constexpr (RW == 1) {
      fin_m = m, fin_r0 = r0, pend_buf = item & 1;
      continue;
    }
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      pend_at[r] = -1;
      const int row = r0 + (rg0 + r) * 16 + (lane & 15);
      if (kh == 0 && (rg0 + r) * 16 < rows_here && row < P.rows) {
#pragma unroll
        for (int t = 0; t < TPG; ++t) pend[r][t] = acc[r][t];
        pend_at[r] = ((int64_t)m * P.tokens + (lane >> 4) * TPG) * P.rows + row;
      }
    }
    pend_buf = item & 1;
  }
  lds_sync();
  finish();
  wait_vmcnt(0);
}

template <int KIND, typename XT, int TPG, int GPER, int RW>
static int launch_stack(const uint8_t* blocks, const uint8_t* tables, int64_t n_mats, int64_t rows, int64_t cols,
                        const XT* x, int64_t tokens, XT* out, bool few, hipStream_t stream) {
  StackPlan P;
  P.rows = (int)rows;
  P.cols = (int)cols;
  P.tokens = (int)tokens;
  P.ngroups = (int)(cols / scale_group<KIND>());
  P.kw = P.ngroups / GPER;
  P.rg = RW == 2 ? 2 : few ? 1 : std::max(1, (KIND == Q2_0 ? 8 : 16) / P.kw);
  P.nw = RW == 2 ? P.kw : P.rg * P.kw;
  const int IR = 16 * P.rg, nt = 64 * P.nw;
  P.rbytes = row_bytes(KIND, cols);
  P.mat_bytes = rows * P.rbytes;
  P.items_per_mat = (int)((rows + IR - 1) / IR);
  P.items = (int)(n_mats * P.items_per_mat);
  row_layout(P.rbytes, ((uintptr_t)blocks & 15) == 0, P.rstride, P.padded);
  const int64_t item_bytes = P.padded ? (int64_t)IR * P.rstride : IR * P.rbytes + 15;
  P.loads = (int)((item_bytes + 16 * nt - 1) / (16 * nt));
  if (P.loads > STACK_LMAX || P.nw > 16)
    return fail(E_UNSUPPORTED, "stack_matvec: rows of %lld bytes", (long long)P.rbytes);
  P.buf_bytes = P.loads * 16 * nt;
  P.ring_off = KIND == IQ3_S ? IQ3S_SIGNED_BYTES : 0;
  const size_t red = (size_t)2 * (RW == 1 ? P.kw : P.kw - 1) * P.rg * 64 * TPG * 4, tail = 128;
  const size_t cap = 160 * 1024;
  // direct loads into LDS land below 128 KiB: the table and the ring stay under it
  const size_t dma_limit = 128 * 1024;
  // the deepest ring (up to six items) that leaves room for two blocks a CU, else the deepest for one
  auto fits = [&](int nb, size_t limit) {
    return (size_t)P.ring_off + (size_t)nb * P.buf_bytes + red + tail <= limit &&
           (size_t)P.ring_off + (size_t)nb * P.buf_bytes <= dma_limit;
  };
  P.nbuf = 0;
  for (int nb = 6; nb >= 3 && !P.nbuf; --nb)
    if (fits(nb, cap / 2)) P.nbuf = nb;
  for (int nb = 6; nb >= 2 && !P.nbuf; --nb)
    if (fits(nb, cap)) P.nbuf = nb;
  if (!P.nbuf)
    return fail(E_UNSUPPORTED, "stack_matvec: no ring of %d-byte items fits in LDS below the 128 KiB direct-load range",
                P.buf_bytes);
  P.red_off = P.ring_off + P.nbuf * P.buf_bytes;
  const size_t lds = (size_t)P.red_off + red + tail;
  if (lds > cap) return fail(E_UNSUPPORTED, "stack_matvec: %zu bytes of LDS", lds);
  auto run = [&](auto kern) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, nt, lds) != hipSuccess || per_cu < 1) per_cu = 1;
    const int64_t grid = few ? P.items : std::min<int64_t>(P.items, (int64_t)device_cus() * per_cu);
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(nt), lds, stream, blocks, P, x, out,
                       tables ? tables + TAB_IQ3S_SIGNED : nullptr);
    return check_launch("stack_matvec");
  };
  return P.nw <= 8 ? run(k_stack_mv<KIND, XT, TPG, GPER, 8, RW>) : run(k_stack_mv<KIND, XT, TPG, GPER, 16, RW>);
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
  if (n_mats * ((rows + 15) / 16) > (1ll << 31) - 1 || rows * row_bytes(kind, cols) > (1ll << 31) - 1)
    return fail(E_SHAPE, "stack_matvec: %lld matrices of %lld x %lld too many", (long long)n_mats, (long long)rows,
                (long long)cols);
  if (!mfma_kind_host(kind) || (x_dtype != BF16 && x_dtype != F16) || cols % 256)
    return fail(E_UNSUPPORTED, "stack_matvec: kind %d, dtype %d, %lld columns (Q2_0 / IQ3_S, bf16 / fp16, columns a "
                "multiple of 256)", kind, x_dtype, (long long)cols);
  if (!blocks || !x || !out || (kind == IQ3_S && !tables)) return fail(E_ARG, "stack_matvec: null pointer");
  if (((uintptr_t)x & 15) || (tables && ((uintptr_t)tables & 15)))
    return fail(E_ARG, "stack_matvec: activations and tables must be 16-byte aligned");
  // a wave's columns: GPER scale groups (8 or 4 Q2_0 blocks, 16 or 8 IQ3_S runs), at most 16 waves across a row
  const int64_t ngroups = cols / (kind == Q2_0 ? 64 : 32);
  // Streaming Q2_0 for up to 4 tokens: 8 column splits of 4 groups, each wave both row groups of a 32-row item (one
  // set of activation registers: two blocks a CU), when that covers a row in at most 8 waves. Otherwise a wave a
  // row group: Q2_0 8 (else 4) groups a wave in 8-wave blocks; IQ3_S 8 (else 16) groups a wave in blocks of up to
  // 16 waves (its table lookups want more waves a SIMD). Measured on the 3072 x 2048 stream.
  const int64_t small = 4;
  const bool rw2_shape = kind == Q2_0 && tokens <= 4 && ngroups % small == 0 && ngroups / small <= 8;
  const int gper1 = kind == Q2_0 ? (ngroups % 8 == 0 ? 8 : 4) : (ngroups % 8 == 0 && ngroups / 8 <= 16 ? 8 : 16);
  if (ngroups / gper1 > 16)
    return fail(E_UNSUPPORTED, "stack_matvec: %lld columns (at most %d)", (long long)cols,
                16 * gper1 * (kind == Q2_0 ? 64 : 32));
  const int tpg = tokens <= 4 ? 1 : tokens <= 8 ? 2 : 4;
  // few items to go round the CUs: one row group a block, one item a block
  const int64_t kw1 = ngroups / gper1, ir = rw2_shape ? 32 : 16 * std::max<int64_t>(1, (kind == Q2_0 ? 8 : 16) / kw1);
  const bool few = n_mats * ((rows + ir - 1) / ir) < 2 * (int64_t)device_cus();
  const bool rw2 = rw2_shape && !few;
  const int gper = rw2 ? (int)small : gper1;
  return with_half_dtype(x_dtype, [&](auto* tp) {
    using XT = std::remove_pointer_t<decltype(tp)>;
    auto go = [&](auto kc, auto gc, auto tc) {
      constexpr int K = decltype(kc)::value, G = decltype(gc)::value, T = decltype(tc)::value;
      if (rw2)
        return launch_stack<K, XT, T, G, 2>((const uint8_t*)blocks, (const uint8_t*)tables, n_mats, rows, cols,
                                            (const XT*)x, tokens, (XT*)out, few, (hipStream_t)stream);
      return launch_stack<K, XT, T, G, 1>((const uint8_t*)blocks, (const uint8_t*)tables, n_mats, rows, cols,
                                          (const XT*)x, tokens, (XT*)out, few, (hipStream_t)stream);
    };
    auto by_t = [&](auto kc, auto gc) {
      return tpg == 1 ? go(kc, gc, kind_c<1>{}) : tpg == 2 ? go(kc, gc, kind_c<2>{}) : go(kc, gc, kind_c<4>{});
    };
    if (kind == Q2_0) return gper == 8 ? by_t(kind_c<Q2_0>{}, kind_c<8>{}) : by_t(kind_c<Q2_0>{}, kind_c<4>{});
    return gper == 16 ? by_t(kind_c<IQ3_S>{}, kind_c<16>{}) : by_t(kind_c<IQ3_S>{}, kind_c<8>{});
  });
}

}  // extern "C"
