// Prompt path: the grouped expert GEMM over pairs laid out in tiles of 16, each tile one expert's
// (strata_mlx/blocks.py:465-536, `tile_matmul`): out[p] = W[expert of p's tile] . a[p], the weights dequantized
// and rounded to a's type, float32 sums, rows of tiles that name no expert left as they were.
//
// A block takes TG consecutive tiles and RB rows of the output. Within its tiles, each run of one expert is done
// together: the run's RB rows of blocks come into LDS once (contiguous bytes of the stack, 16-byte loads); chunk by
// chunk of KCH columns the block dequantizes them into LDS (rounded to bf16 / fp16, as the reference rounds them;
// IQ3_S from a table of signed grid entries, Q2_0 as d * (c - 1), one fma a weight, exact before the rounding),
// two buffers in turn, while the waves whose tiles are in the run multiply the previous chunk (16 pairs against RB
// rows) on 16x16x32 MFMA, fp32 accumulators in registers, activation fragments straight from global memory. LDS
// rows of a chunk are XOR-swizzled by 16-byte chunk so the MFMA operand reads fall in distinct banks.
#include <atomic>
#include <type_traits>

#include "launch.h"
#include "xmv.h"

namespace sh {

constexpr int TILE_TOKENS = 16, TG = 8, RB = 64, KCH = 256;

// the tables a kind's dequantization reads in LDS, and their size: IQ3_S the 32 KiB signed table, others as
// stage_tables lays them out
template <int KIND> constexpr int tile_tab_bytes() { return KIND == IQ3_S ? IQ3S_SIGNED_BYTES : (KIND == Q2_0 || KIND == Q3_K) ? 0 : LDS_TAB_MAX; }

// two floats rounded to nearest even in XT, packed (lo in the low half): one v_cvt_pk a pair
template <typename XT> __device__ __forceinline__ uint32_t pack_rne(float lo, float hi) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef XT x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){lo, hi}, x2));
}

// run `n` (32 weights) of a row of blocks in LDS, dequantized and rounded to XT, as 16 XT values in 4 u32x4 each
// (the run's weights 8c .. 8c + 7 in w[c])
template <int KIND, typename XT>
__device__ __forceinline__ void dequant_run(const uint8_t* row, int n, const uint8_t* tab, u32x4* w) {
  float f[32];
  if constexpr (KIND == IQ3_S) {
    const uint8_t* b = row + (n >> 3) * 110;
    const int ib = n & 7;
    const float db = half_bits(*(const uint16_t*)b) * (float)(1 + 2 * (((uint32_t)b[106 + ib / 2] >> (4 * (ib & 1))) & 15u));
    const float nb16 = -16.0f * db;
    const uint32_t qh = b[66 + ib];
    const uint32_t s01 = *(const uint16_t*)(b + 74 + 4 * ib), s23 = *(const uint16_t*)(b + 76 + 4 * ib);
    const uint32_t sg = s01 | (s23 << 16);
    const uint32_t* stab = (const uint32_t*)tab;
#pragma unroll
    for (int l = 0; l < 8; ++l) {
      const uint32_t q = b[2 + 8 * ib + l];
      const uint32_t e = stab[q | (((qh >> l) & 1u) << 8) | (((sg >> (4 * l)) & 15u) << 9)];  // bytes 16 +- v
#pragma unroll
      for (int j = 0; j < 4; ++j) f[4 * l + j] = fmaf(db, (float)((e >> (8 * j)) & 0xffu), nb16);  // db * v, exact
    }
  } else if constexpr (KIND == Q2_0) {
    const uint8_t* b = row + (n >> 1) * 18;
    const float d = half_bits(*(const uint16_t*)b);
    const uint8_t* q = b + 2 + 8 * (n & 1);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t c = q[i];
#pragma unroll
      for (int j = 0; j < 4; ++j) f[4 * i + j] = fmaf(d, (float)((c >> (2 * j)) & 3u), -d);  // d * (c - 1), exact
    }
  } else {
    unpack32<KIND>(row, n, f, tab);
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    uint32_t p[4];
#pragma unroll
    for (int h = 0; h < 4; ++h) p[h] = pack_rne<XT>(f[8 * c + 2 * h], f[8 * c + 2 * h + 1]);
    w[c] = u32x4{p[0], p[1], p[2], p[3]};
  }
}

// A block: TG tiles x RB rows; per run of one expert within its tiles, the run's rows of blocks come into LDS
// once, then chunk after chunk of KCH columns is dequantized into one of two LDS buffers while the waves whose
// tiles are in the run multiply the other on 16x16x32 MFMA.
template <int KIND, typename XT>
__global__ __launch_bounds__(TG * 64) void k_tile_matmul(const uint8_t* __restrict__ blocks,
                                                         const uint8_t* __restrict__ tables, int experts, int rows,
                                                         int cols, int64_t rbytes, const XT* __restrict__ a,
                                                         int n_tiles, const int32_t* __restrict__ tile_expert,
                                                         float* __restrict__ out) {
  constexpr int CH = KCH / 8, SW = 15, NT = TG * 64, TAB = tile_tab_bytes<KIND>();
  constexpr int UNITS = RB * (KCH / 32);  // (row, run) pairs of a chunk: one a thread
  static_assert(UNITS == NT, "one run a thread a chunk");
  extern __shared__ u32x4 dyn[];
  uint8_t* tab = (uint8_t*)dyn;
  XT* wl = (XT*)((uint8_t*)dyn + TAB);         // two [RB][KCH] buffers of the dequantized chunk
  uint8_t* raw = (uint8_t*)(wl + 2 * RB * KCH);  // the run's RB rows of blocks, as stored
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, n = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int t0 = blockIdx.x * TG, r0 = blockIdx.y * RB;
  const int nt = min(TG, n_tiles - t0);
  const int slab = RB * (int)rbytes;  // bytes of the run's rows: contiguous in the stack
  const int nch = (cols + KCH - 1) / KCH;  // the last chunk may be partial: whole runs of 32 past the row are zeros

  if constexpr (KIND == IQ3_S) {
    for (int i = tid; i < IQ3S_SIGNED_BYTES / 16; i += NT) ((u32x4*)tab)[i] = ((const u32x4*)(tables + TAB_IQ3S_SIGNED))[i];
  } else if constexpr (TAB > 0) {
    stage_tables<KIND>(tab, tables);
  }
  int ex[TG];
#pragma unroll
  for (int i = 0; i < TG; ++i) {
    const int e = i < nt ? tile_expert[t0 + i] : experts;
    ex[i] = (e >= 0 && e < experts) ? e : experts;  // a tile naming no expert is skipped
  }
  // this thread's (row, run) of every chunk, and where its 4 dequantized 16-byte pieces go
  const int ur = tid / (KCH / 32), urun = tid - ur * (KCH / 32);

  for (int ta = 0; ta < nt;) {
    const int e = ex[ta];
    int tb = ta + 1;
    while (tb < nt && ex[tb] == e) ++tb;
    if (e >= experts) {
      ta = tb;
      continue;
    }
    const bool mine = wave >= ta && wave < tb;
    __syncthreads();  // the previous run is done with the slab and the buffers
    {
      const uint8_t* src = blocks + ((int64_t)e * rows + r0) * rbytes;
      const int n16 = slab >> 4;
      for (int base = 0; base < n16; base += 4 * NT) {
        u32x4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int i = base + u * NT + tid;
          if (i < n16) v[u] = *(const u32x4*)(src + 16 * (int64_t)i);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int i = base + u * NT + tid;
          if (i < n16) *(u32x4*)(raw + 16 * i) = v[u];
        }
      }
    }
    __syncthreads();
    auto dequant = [&](int c, int buf) {
      u32x4 w[4] = {};
      const int run = c * (KCH / 32) + urun;
      if (run * 32 < cols) dequant_run<KIND, XT>(raw + ur * (int)rbytes, run, tab, w);
      XT* dst = wl + buf * RB * KCH + ur * KCH;
#pragma unroll
      for (int q = 0; q < 4; ++q) *(u32x4*)(dst + 8 * ((4 * urun + q) ^ (ur & SW))) = w[q];
    };
    dequant(0, 0);
    f32x4 acc[RB / 16];
#pragma unroll
    for (int nb = 0; nb < RB / 16; ++nb) acc[nb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const XT* arow = a + ((int64_t)(t0 + wave) * TILE_TOKENS + n) * cols;  // the lane's A row (its tile's token n)
    for (int c = 0; c < nch; ++c) {
      u32x4 af[KCH / 32];
      if (mine) {
#pragma unroll
        for (int ks = 0; ks < KCH / 32; ++ks)
          af[ks] = c * KCH + ks * 32 < cols ? *(const u32x4*)(arow + c * KCH + ks * 32 + 8 * g) : u32x4{0u, 0u, 0u, 0u};
      }
      __syncthreads();  // chunk c is in buffer c & 1; chunk c - 1's readers are done with the other
      if (c + 1 < nch) dequant(c + 1, (c + 1) & 1);
      if (mine) {
        const XT* wb = wl + (c & 1) * RB * KCH;
#pragma unroll
        for (int ks = 0; ks < KCH / 32; ++ks) {
#pragma unroll
          for (int nb = 0; nb < RB / 16; ++nb) {
            const int r = nb * 16 + n;
            const u32x4 bf = *(const u32x4*)(wb + r * KCH + 8 * ((4 * ks + g) ^ (r & SW)));
            acc[nb] = mfma<XT>(af[ks], bf, acc[nb]);
          }
        }
      }
    }
    if (mine) {
      const int64_t p0 = ((int64_t)t0 + wave) * TILE_TOKENS;
#pragma unroll
      for (int nb = 0; nb < RB / 16; ++nb)
#pragma unroll
        for (int i = 0; i < 4; ++i) out[(p0 + 4 * g + i) * rows + r0 + nb * 16 + n] = acc[nb][i];
    }
    ta = tb;
  }
}

template <int KIND, typename XT>
static int launch_tiles(const uint8_t* blocks, const uint8_t* tables, int64_t experts, int64_t rows, int64_t cols,
                        const XT* a, int64_t n_tiles, const int32_t* tile_expert, float* out, hipStream_t stream) {
  const int64_t rb = row_bytes(KIND, cols);
  const dim3 grid((unsigned)((n_tiles + TG - 1) / TG), (unsigned)(rows / RB));
  const size_t lds = tile_tab_bytes<KIND>() + 2 * (size_t)RB * KCH * sizeof(XT) + (size_t)RB * rb;
  if (lds > 160 * 1024)
    return fail(E_UNSUPPORTED, "tile_matmul: rows of %lld bytes (%zu bytes of LDS)", (long long)rb, lds);
  hipLaunchKernelGGL((k_tile_matmul<KIND, XT>), grid, dim3(TG * 64), lds, stream, blocks, tables, (int)experts,
                     (int)rows, (int)cols, rb, a, (int)n_tiles, tile_expert, out);
  return check_launch("tile_matmul");
}


// ---- the streaming form (Q2_0 and IQ3_S, columns in chunks of 256, the last possibly partial, rows in blocks of 64)
//
// Persistent blocks, one a CU. A block first lays its window of tiles out in units: a unit is at most TS_TGU
// consecutive tiles of one expert, a run of one expert's tiles cut every TS_TGU tiles from its start; tiles that
// name no expert make no unit. Every block computes the same list, then takes the items (unit, block of 64 rows)
// blockIdx.x, blockIdx.x + gridDim.x, ... All its items' chunks form one stream. Waves 0-7 (producers) bring chunk
// after chunk of 256 columns of the item's 64 rows of blocks into an LDS ring by direct loads, TS_LEAD chunks
// ahead, and dequantize each into one of two bf16 / fp16 buffers; waves 8-15 (consumers) multiply the other
// buffer on MFMA, all 64 rows against one tile each, their activation fragments loaded two steps ahead. Only consumers issue ordinary loads, so the
// compiler's waits for them never wait on the ring's loads. A step is one barrier: producers have landed chunk
// q + 1 and dequantize it while consumers multiply chunk q.
//
// Modes: TS_PLAIN is tile_matmul (a in slot order, float32 rows of the slots out); TS_GLU takes a token's row of
// x for each slot, runs gate and up (32 rows of each an item) and writes silu(g) * u rounded to x's type in slot
// order; TS_DOWN takes those rows and writes each pair's row, rounded to x's type, where the slot's pair is.
// TS_DOWN_S is TS_DOWN with a short unit's tiles shared among consumers, its activation fragments loaded one step
// ahead into one register buffer instead of two steps ahead into two (the registers the sharing needs).
enum { TS_PLAIN = 0, TS_GLU = 1, TS_DOWN = 2, TS_DOWN_S = 3 };
constexpr int TS_KCH = 256, TS_RBV = 64, TS_TGU = 8, TS_NR = 6, TS_LEAD = 5, TS_NT = 1024;
constexpr int TS_WT = 3 * TS_NT;                      // tiles of a window: three a thread in the layout
constexpr int TS_PPR = 8;                             // 16-byte pieces a row's chunk may cover
constexpr int TS_SLOT = TS_RBV * TS_PPR * 16;         // bytes of a ring slot: one piece a producer lane
constexpr int TS_BUF = TS_RBV * TS_KCH;               // elements of a dequantized chunk
static_assert(TS_NR >= TS_LEAD + 1, "a ring slot is reloaded only after a barrier past its dequantization");
static_assert(TS_WT <= 4096 && TS_TGU < 16, "a unit packs its first tile in 12 bits and its length in 4");
static_assert(TS_SLOT == 512 * 16 && TS_RBV * (TS_KCH / 32) == 512, "a piece and a run of 32 a producer lane");

struct TileStreamArgs {
  const uint8_t* w0;           // the stack (gate for TS_GLU)
  const uint8_t* w1;           // up (TS_GLU)
  const uint8_t* tables;       // the codebook blob (IQ3_S: its signed table)
  const void* a;               // TS_PLAIN / TS_DOWN: (slots, cols); TS_GLU: x (tokens, cols)
  const int32_t* token;        // TS_GLU: the row of x of each slot
  const int32_t* pair;         // TS_DOWN: the output row of each slot, or -1
  const int32_t* tile_expert;  // (n_tiles,)
  void* out;
  int64_t n_src;               // TS_GLU: rows of x (tokens are clamped into them); TS_DOWN: output rows (pairs)
  int experts, rows, cols, rbytes, n_tiles;
  int tile0;                   // the first tile of this launch's window of at most TS_WT tiles
  int share;                   // short units' tiles shared among consumer waves (sh_tiles_set_share)
};

template <int KIND> __host__ __device__ constexpr int ts_chunk_bytes() { return TS_KCH / wpb(KIND) * bpb(KIND); }
template <int KIND> __host__ __device__ constexpr int ts_tab_bytes() { return KIND == IQ3_S ? IQ3S_SIGNED_BYTES : 0; }
// LDS: [table][ring][two dequantized chunks][tile experts of the window][units of the window][scan scratch]
template <int KIND, typename XT> __host__ __device__ constexpr int ts_lds_bytes() {
  return ts_tab_bytes<KIND>() + TS_NR * TS_SLOT + 2 * TS_BUF * (int)sizeof(XT) + TS_WT * 2 + TS_WT * 2 + 64;
}

// a position in a block's stream: chunk c of item (unit u, row block rb), and the unit's first tile, length and
// expert; advanced chunk by chunk without divisions
struct TsCursor {
  int q, c, u, rb, start, len, e;
};

// exclusive scan over the block (MAX: running maximum, identity -1; else running sum), and the total
// x, which the compiler cannot see through: values computed from it in a loop stay in the loop
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

template <bool MAX> __device__ __forceinline__ int ts_block_scan(int v, int* scr, int& total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int inc = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(inc, d);
    if (lane >= d) inc = MAX ? max(inc, o) : inc + o;
  }
  if (lane == 63) scr[wave] = inc;
  __syncthreads();
  int pre = MAX ? -1 : 0, tot = MAX ? -1 : 0;
#pragma unroll
  for (int w = 0; w < TS_NT / 64; ++w) {
    const int s = scr[w];
    if (w < wave) pre = MAX ? max(pre, s) : pre + s;
    tot = MAX ? max(tot, s) : tot + s;
  }
  __syncthreads();
  int ex = __shfl_up(inc, 1);
  if (lane == 0) ex = MAX ? -1 : 0;
  total = tot;
  return MAX ? max(pre, ex) : pre + ex;
}

template <int KIND, typename XT, int MODE>
__global__ __launch_bounds__(TS_NT) void k_tile_stream(TileStreamArgs g) {
  constexpr int CB = ts_chunk_bytes<KIND>(), TAB = ts_tab_bytes<KIND>(), TPT = TS_WT / TS_NT;
  constexpr int VR = MODE == TS_GLU ? TS_RBV / 2 : TS_RBV;  // rows of one stack an item
  constexpr bool DOWN = MODE == TS_DOWN || MODE == TS_DOWN_S;
  constexpr int ABUF = MODE == TS_DOWN_S ? 1 : 2;  // activation fragment buffers: steps loaded ahead
  static_assert(CB + 15 <= TS_PPR * 16, "a row's chunk fits its ring row");
  extern __shared__ u32x4 dyn[];
  uint8_t* lds = (uint8_t*)dyn;
  uint8_t* tab = lds;
  uint8_t* ring = lds + TAB;
  XT* wl = (XT*)(ring + TS_NR * TS_SLOT);
  int16_t* s_te = (int16_t*)(wl + 2 * TS_BUF);  // expert of each tile of the window, -1 for none
  uint16_t* s_unit = (uint16_t*)(s_te + TS_WT);
  int* s_scr = (int*)(s_unit + TS_WT);
  const uint32_t ring_lds = SH_LDS_ADDR(dyn) + TAB;

  const int tid = threadIdx.x, lane = tid & 63, n = lane & 15, gq = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // the last chunk may be partial (Q2_0 rows of 64-column blocks): its bytes past the row are not loaded, its runs
  // past the row dequantize to zeros and its activations past the row are zeros
  const int nch = (g.cols + TS_KCH - 1) / TS_KCH, rblk = g.rows / VR;
  const int64_t rbytes = g.rbytes;

  if constexpr (KIND == IQ3_S) {  // the signed table, once a block
    const uint8_t* src = g.tables + TAB_IQ3S_SIGNED;
    constexpr int PIECES = IQ3S_SIGNED_BYTES / 16;
#pragma unroll
    for (int i = 0; i < (PIECES + TS_NT - 1) / TS_NT; ++i)
      if (i * TS_NT + wave * 64 < PIECES)  // whole waves: PIECES is a multiple of 64
        lds_dma16(src, (uint32_t)((i * TS_NT + tid) * 16), SH_LDS_ADDR(dyn) + (uint32_t)((i * TS_NT + wave * 64) * 16));
  }

  {
    // ---- the window's units (one window a launch: a loop around both roles would let the compiler's waits
    // for one role's loads reach into the other's code)
    const int w0 = g.tile0, nwin = min(TS_WT, g.n_tiles - w0);
    for (int i = tid; i < TS_WT; i += TS_NT) {
      const int e = i < nwin ? g.tile_expert[w0 + i] : -1;
      s_te[i] = (int16_t)((e >= 0 && e < g.experts) ? e : -1);
    }
    __syncthreads();
    int ex[TPT], rsl[TPT];
    int carry = -1;
#pragma unroll
    for (int j = 0; j < TPT; ++j) {
      const int i = TPT * tid + j;
      ex[j] = s_te[i];
      if (i == 0 || ex[j] != s_te[i - 1]) carry = i;  // a run of one expert (or of none) starts here
      rsl[j] = carry;
    }
    int ignore;
    const int carry_in = ts_block_scan<true>(carry, s_scr, ignore);
    int cnt = 0;
    bool seg[TPT], unit[TPT];
#pragma unroll
    for (int j = 0; j < TPT; ++j) {
      const int i = TPT * tid + j, r = rsl[j] >= 0 ? rsl[j] : carry_in;
      seg[j] = (i - r) % TS_TGU == 0;
      unit[j] = seg[j] && ex[j] >= 0 && i < nwin;
      cnt += unit[j];
    }
    uint8_t* s_seg = (uint8_t*)wl;  // segment starts, in the first dequantization buffer until the stream
#pragma unroll
    for (int j = 0; j < TPT; ++j) s_seg[TPT * tid + j] = seg[j];
    int n_units;
    int pos = ts_block_scan<false>(cnt, s_scr, n_units);  // (its barriers publish s_seg)
#pragma unroll
    for (int j = 0; j < TPT; ++j) {
      const int i = TPT * tid + j;
      if (unit[j]) {
        int len = 1;
        while (len < TS_TGU && i + len < nwin && !s_seg[i + len]) ++len;
        s_unit[pos++] = (uint16_t)(i | (len << 12));
      }
    }
    __syncthreads();

    // ---- the stream of this block's items' chunks
    const int n_items = n_units * rblk;
    const int my_items = n_items > (int)blockIdx.x ? (n_items - 1 - (int)blockIdx.x) / (int)gridDim.x + 1 : 0;
    const int Q = my_items * nch;
    if (Q == 0) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no load into LDS outlives the block
      return;
    }
    const int G = (int)gridDim.x, gdiv = G / rblk, gmod = G - gdiv * rblk;
    auto cur_fill = [&](TsCursor& k) {
      const int uu = s_unit[k.u];
      k.start = w0 + (uu & 4095);
      k.len = uu >> 12;
      k.e = s_te[uu & 4095];
    };
    auto cur_at = [&](int q) {
      TsCursor k;
      k.q = q;
      const int kk = q / nch, item = (int)blockIdx.x + kk * G;
      k.c = q - kk * nch;
      k.u = item / rblk;
      k.rb = item - k.u * rblk;
      k.start = k.len = k.e = 0;
      if (q < Q) cur_fill(k);
      return k;
    };
    auto cur_next = [&](TsCursor& k) {
      ++k.q;
      if (++k.c == nch) {
        k.c = 0;
        k.rb += gmod;
        k.u += gdiv;
        if (k.rb >= rblk) k.rb -= rblk, ++k.u;
        if (k.q < Q) cur_fill(k);
      }
    };

    if (wave < 8) {
      // ---- producers: the ring and the dequantization; lane (row v, piece / run j), the row's first byte in
      // the item of each cursor recomputed only when the cursor enters an item
      const int v = tid >> 3, j = tid & 7;
      auto row_base = [&](const TsCursor& s) {
        const uint8_t* stack = g.w0;
        int r = s.rb * VR + v;
        if constexpr (MODE == TS_GLU) {
          stack = v < VR ? g.w0 : g.w1;
          r = s.rb * VR + (v & (VR - 1));
        }
        return stack + ((int64_t)s.e * g.rows + r) * rbytes;
      };
      TsCursor ci = cur_at(0), cd = cur_at(0);  // the next chunk to load, the next to dequantize
      const uint8_t* ibase = row_base(ci);
      const uint8_t* dbase = ibase;
      int islot = 0, dslot = 0;  // their ring slots
      auto issue = [&]() {  // chunk ci.q into ring slot islot: piece j of row v
        const uint8_t* src = ibase + ci.c * CB;
        const int lead = (int)((uintptr_t)src & 15);
        const int cb = min(CB, (int)rbytes - ci.c * CB);  // the chunk's bytes in the row
        if (16 * j < lead + cb) lds_dma16p(src - lead + 16 * j, ring_lds + (uint32_t)(islot * TS_SLOT + wave * 1024));
        islot = islot + 1 == TS_NR ? 0 : islot + 1;
        cur_next(ci);
        if (ci.c == 0 && ci.q < Q) ibase = row_base(ci);
      };
      auto dequant = [&]() {  // chunk cd.q into buffer cd.q & 1: run j of row v
        const uint8_t* src = dbase + cd.c * CB;
        const uint8_t* raw = ring + dslot * TS_SLOT + v * (TS_PPR * 16) + ((uintptr_t)src & 15);
        u32x4 w[4] = {};
        if (cd.c * TS_KCH + 32 * j < g.cols) dequant_run<KIND, XT>(raw, j, tab, w);
        XT* dst = wl + (cd.q & 1) * TS_BUF + v * TS_KCH;
#pragma unroll
        for (int h = 0; h < 4; ++h) *(u32x4*)(dst + 8 * ((4 * j + h) ^ (v & 15))) = w[h];
        dslot = dslot + 1 == TS_NR ? 0 : dslot + 1;
        cur_next(cd);
        if (cd.c == 0 && cd.q < Q) dbase = row_base(cd);
      };
      const int lead0 = min(TS_LEAD, Q);
      for (int q = 0; q < lead0; ++q) issue();
      if constexpr (KIND == IQ3_S) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // (the table, and the lead)
      wait_vmcnt(lead0 - 1);
      lds_sync();
      dequant();
      for (int q = 0; q < Q; ++q) {
        if (ci.q < Q) {  // ci.q == q + TS_LEAD: the steady state, TS_LEAD - 1 loads after chunk q + 1's
          issue();
          static_assert(TS_LEAD - 1 == 4, "the immediate below");
          asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
        } else if (q + 1 < Q) {
          wait_vmcnt(Q - 1 - (q + 1));
        }
        lds_sync();
        if (cd.q < Q) dequant();  // cd.q == q + 1
      }
    } else {
      // ---- consumers: the 64 rows (four fragments of 16) against the unit's tiles. A unit of 5-8 tiles gives
      // consumer cw tile cw and all four fragments; a shorter unit shares each tile among wpt waves (2 or 4: up to
      // 8 waves busy), wave cw taking tile cw / wpt and fragments fg, fg + wpt, ... (fg = cw % wpt: for TS_GLU a
      // gate fragment and the up fragment two on, so wpt <= 2). The activation fragments of the wave's tile for
      // chunk q are in af[q & 1], loaded two steps ahead (the loop is unrolled by two: the buffers stay registers)
      const int cw = wave - 8;
      auto wpt_of = [&](int len) {  // (TS_DOWN: one wave a tile; its registers are at the limit already)
        constexpr int MAXW = MODE == TS_PLAIN || MODE == TS_DOWN_S ? 4 : MODE == TS_GLU ? 2 : 1;
        return !g.share ? 1 : len <= 2 ? MAXW : len <= 4 ? min(2, MAXW) : 1;
      };
      auto tile_of = [&](int len) { return cw / wpt_of(len); };
      const XT* a = (const XT*)g.a;
      f32x4 acc[4];
      int pr[4] = {0, 0, 0, 0};  // TS_DOWN: the output rows of the lane's four slots in the current item
      u32x4 af[ABUF][TS_KCH / 32];
      const XT* arow = a;
#pragma unroll
      for (int f = 0; f < 4; ++f) acc[f] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      TsCursor cs = cur_at(0), cl = cur_at(0);  // the chunk to multiply, the next to load fragments of
      // TS_GLU: the token of the lane's slot in the item the loading cursor enters next, loaded an item ahead
      auto item_after = [&](TsCursor k) {  // chunk 0 of the item after k's (k at a chunk 0)
        k.q += nch;
        k.rb += gmod;
        k.u += gdiv;
        if (k.rb >= rblk) k.rb -= rblk, ++k.u;
        if (k.q < Q) cur_fill(k);
        return k;
      };
      auto token_of = [&](const TsCursor& k) {
        int t = 0;
        const int tl = tile_of(k.len);
        if (k.q < Q && tl < k.len) t = g.token[(int64_t)(k.start + tl) * TILE_TOKENS + (lane & 15)];
        return t;
      };
      int tok_next = 0;
      if constexpr (MODE == TS_GLU) tok_next = token_of(cl);
      auto load_a = [&](const TsCursor& s, auto bc) {  // chunk s.q's fragments of the lane's row into af[bc]
        constexpr int BUF = decltype(bc)::value;
        const int ln = opaque(lane), n = ln & 15, gq = ln >> 4;
        const int tl = tile_of(s.len);
        if (s.c == 0) {  // a new item: the row of the lane's slot
          int64_t row = (int64_t)(s.start + tl) * TILE_TOKENS + n;
          if constexpr (MODE == TS_GLU) {
            row = min(max((int64_t)tok_next, (int64_t)0), g.n_src - 1);
            tok_next = token_of(item_after(s));
          }
          arow = a + row * g.cols;
        }
        if (tl < s.len) {
          const int left = g.cols - s.c * TS_KCH;  // columns of the row from this chunk on
#pragma unroll
          for (int ks = 0; ks < TS_KCH / 32; ++ks)
            af[BUF][ks] = ks * 32 < left ? *(const u32x4*)(arow + s.c * TS_KCH + ks * 32 + 8 * gq)
                                         : u32x4{0u, 0u, 0u, 0u};
        } else {  // (defined on every path: the fragments are not live across the epilogue)
#pragma unroll
          for (int ks = 0; ks < TS_KCH / 32; ++ks) af[BUF][ks] = u32x4{0u, 0u, 0u, 0u};
        }
      };
      auto step = [&](auto bc) {
        constexpr int BUF = decltype(bc)::value;
        const TsCursor& s = cs;
        const int q = s.q;
        lds_sync();
        const XT* wb = wl + (q & 1) * TS_BUF;
        // the wave's tile and fragments as constants of the path (a fragment count known at compile time keeps
        // the accumulators and operands in registers)
        auto multiply = [&](auto wc) {
          constexpr int WPT = decltype(wc)::value, NF = 4 / WPT;
          const int tl = cw / WPT, fg = cw - tl * WPT;
          if (tl >= s.len) return;
          const int ln = opaque(lane), n = ln & 15, gq = ln >> 4;
          auto read_b = [&](int ks, u32x4* b) {
#pragma unroll
            for (int j = 0; j < NF; ++j) {
              const int r = 16 * (fg + WPT * j) + n;
              b[j] = *(const u32x4*)(wb + r * TS_KCH + 8 * ((4 * ks + gq) ^ (r & 15)));
            }
          };
          u32x4 b[2][NF];  // the fragments of k-step ks + 1 are read while those of ks multiply
          read_b(0, b[0]);
#pragma unroll
          for (int ks = 0; ks < TS_KCH / 32; ++ks) {
            if (ks + 1 < TS_KCH / 32) read_b(ks + 1, b[(ks + 1) & 1]);
            __builtin_amdgcn_sched_barrier(0);  // (the scheduler would sink the reads to their MFMAs)
#pragma unroll
            for (int j = 0; j < NF; ++j) acc[j] = mfma<XT>(af[BUF][ks], b[ks & 1][j], acc[j]);
          }
          const int64_t slot0 = (int64_t)(s.start + tl) * TILE_TOKENS + 4 * gq;
          if constexpr (DOWN) {  // the slots' output rows, at the item's first chunk
            if (s.c == 0) {
#pragma unroll
              for (int i = 0; i < 4; ++i) pr[i] = g.pair[slot0 + i];
            }
          }
          if (s.c == nch - 1) {  // the item's rows are done
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              if constexpr (MODE == TS_PLAIN) {
                float* o = (float*)g.out + (slot0 + i) * g.rows + s.rb * VR + n;
#pragma unroll
                for (int j = 0; j < NF; ++j) o[16 * (fg + WPT * j)] = acc[j][i];
              } else if constexpr (MODE == TS_GLU) {  // gate fragment j, its up fragment j + NF / 2
                XT* o = (XT*)g.out + (slot0 + i) * g.rows + s.rb * VR + n;
#pragma unroll
                for (int j = 0; j < NF / 2; ++j) {
                  const float gt = acc[j][i], up = acc[j + NF / 2][i];
                  o[16 * (fg + WPT * j)] = from_f32<XT>(gt / (1.0f + expf(-gt)) * up);
                }
              } else {
                const int p = pr[i];
                if (p >= 0 && p < g.n_src) {
                  XT* o = (XT*)g.out + (int64_t)p * g.rows + s.rb * VR + n;
#pragma unroll
                  for (int j = 0; j < NF; ++j) o[16 * (fg + WPT * j)] = from_f32<XT>(acc[j][i]);
                }
              }
            }
#pragma unroll
            for (int f = 0; f < 4; ++f) acc[f] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
          }
        };
        if constexpr (MODE == TS_DOWN) {  // (TS_DOWN_S takes the shared forms below)
          multiply(std::integral_constant<int, 1>{});
        } else {
          const int wpt = wpt_of(s.len);
          if (wpt == 1)
            multiply(std::integral_constant<int, 1>{});
          else if (MODE == TS_GLU || wpt == 2)
            multiply(std::integral_constant<int, 2>{});
          else
            multiply(std::integral_constant<int, (MODE == TS_GLU ? 2 : 4)>{});
        }
        __builtin_amdgcn_sched_barrier(0);  // chunk q + 2's fragments load after chunk q's are consumed
        cur_next(cs);
        if (cl.q < Q) {  // cl.q == q + ABUF
          load_a(cl, bc);
          cur_next(cl);
        }
      };
      using B0 = std::integral_constant<int, 0>;
      using B1 = std::integral_constant<int, 1>;
      load_a(cl, B0{});
      cur_next(cl);
      if constexpr (ABUF == 2) {
        if (Q > 1) {
          load_a(cl, B1{});
          cur_next(cl);
        }
      }
      if constexpr (KIND == IQ3_S) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // (the table)
      lds_sync();
      int q = 0;
      if constexpr (ABUF == 2) {
        for (; q + 1 < Q; q += 2) {
          step(B0{});
          step(B1{});
        }
        if (q < Q) step(B0{});
      } else {
        for (; q < Q; ++q) step(B0{});
      }
      // nothing of the consumers' left in flight where the compiler joins the roles' paths: its waits in the
      // producers' code would count against their ring loads
      __builtin_amdgcn_s_waitcnt(0);
    }
  }
}

// whether the stream kernels share a short unit's tiles among consumer waves (on unless switched off, for
// measuring the two forms against each other)
static std::atomic<int> g_share{1};

template <int KIND, typename XT, int MODE>
static int launch_stream(const TileStreamArgs& g, hipStream_t stream, const char* what) {
  constexpr size_t lds = ts_lds_bytes<KIND, XT>();
  static_assert(lds <= 160 * 1024, "the stream's LDS fits a CU");
  auto kern = k_tile_stream<KIND, XT, MODE>;
  if (lds + static_lds(kern) > LDS_BYTES) return fail(E_UNSUPPORTED, "%s: %zu bytes of LDS", what, lds);
  if (g.experts > 32767) return fail(E_UNSUPPORTED, "%s: %d experts (at most 32767)", what, g.experts);
  for (int w0 = 0; w0 < g.n_tiles; w0 += TS_WT) {
    TileStreamArgs gw = g;
    gw.tile0 = w0;
    gw.share = g_share.load(std::memory_order_relaxed);
    hipLaunchKernelGGL(kern, dim3((unsigned)device_cus()), dim3(TS_NT), lds, stream, gw);
    const int st = check_launch(what);
    if (st) return st;
  }
  return OK;
}

}  // namespace sh

using namespace sh;

extern "C" {

int sh_tile_matmul(int kind, const void* blocks, const void* tables, int64_t experts, int64_t rows, int64_t cols,
                   const void* a, int a_dtype, int64_t pairs, const int32_t* tile_expert, float* out, void* stream) {
  int st = check_rows(kind, rows, cols, "tile_matmul");
  if (st) return st;
  if (pairs <= 0) return OK;
  if (rows % RB || cols % 64) return fail(E_SHAPE, "tile_matmul: %lld x %lld is not in tiles of %d x 64",
                                          (long long)rows, (long long)cols, RB);
  if (pairs % TILE_TOKENS) return fail(E_SHAPE, "tile_matmul: %lld pairs are not whole tiles of 16", (long long)pairs);
  if (a_dtype != BF16 && a_dtype != F16)
    return fail(E_UNSUPPORTED, "tile_matmul: activations of dtype %d (bfloat16 or float16)", a_dtype);
  const bool needs_tables = kind != Q2_0 && kind != Q3_K;
  if (!blocks || !a || !tile_expert || !out || (needs_tables && !tables))
    return fail(E_ARG, "tile_matmul: null pointer");
  if (((uintptr_t)a & 15) || ((uintptr_t)blocks & 15))
    return fail(E_ARG, "tile_matmul: activations and blocks must be 16-byte aligned");
  const int64_t n_tiles = pairs / TILE_TOKENS;
  if (kind == IQ3_S || kind == Q2_0) {
    TileStreamArgs g{};
    g.w0 = (const uint8_t*)blocks;
    g.tables = (const uint8_t*)tables;
    g.a = a;
    g.tile_expert = tile_expert;
    g.out = out;
    g.experts = (int)experts, g.rows = (int)rows, g.cols = (int)cols, g.rbytes = (int)row_bytes(kind, cols);
    g.n_tiles = (int)n_tiles;
    return with_half_dtype(a_dtype, [&](auto* tp) {
      using XT = std::remove_pointer_t<decltype(tp)>;
      return kind == IQ3_S ? launch_stream<IQ3_S, XT, TS_PLAIN>(g, (hipStream_t)stream, "tile_matmul")
                           : launch_stream<Q2_0, XT, TS_PLAIN>(g, (hipStream_t)stream, "tile_matmul");
    });
  }
  return with_kind(kind, [&](auto kc) {
    constexpr int K = decltype(kc)::value;
    return with_half_dtype(a_dtype, [&](auto* tp) {
      using XT = std::remove_pointer_t<decltype(tp)>;
      return launch_tiles<K, XT>((const uint8_t*)blocks, (const uint8_t*)tables, experts, rows, cols, (const XT*)a,
                                 n_tiles, tile_expert, out, (hipStream_t)stream);
    });
  });
}

}  // extern "C"

extern "C" {

int sh_tile_glu(int kind, const void* gate, const void* up, const void* tables, int64_t experts, int64_t rows,
                int64_t cols, const void* x, int x_dtype, int64_t tokens, const int32_t* token, int64_t slots,
                const int32_t* tile_expert, void* h, void* stream) {
  int st = check_rows(kind, rows, cols, "tile_glu");
  if (st) return st;
  if (slots <= 0) return OK;
  if (kind != IQ3_S && kind != Q2_0) return fail(E_UNSUPPORTED, "tile_glu: kind %d (Q2_0 or IQ3_S)", kind);
  if (rows % (TS_RBV / 2) || cols % 64)
    return fail(E_UNSUPPORTED, "tile_glu: %lld x %lld is not in blocks of %d x 64", (long long)rows, (long long)cols,
                TS_RBV / 2);
  if (slots % TILE_TOKENS) return fail(E_SHAPE, "tile_glu: %lld slots are not whole tiles of 16", (long long)slots);
  if (slots / TILE_TOKENS > (1 << 26) || tokens <= 0)
    return fail(E_SHAPE, "tile_glu: %lld slots of %lld tokens", (long long)slots, (long long)tokens);
  if (!gate || !up || (kind == IQ3_S && !tables) || !x || !token || !tile_expert || !h)
    return fail(E_ARG, "tile_glu: null pointer");
  if (((uintptr_t)x & 15) || ((uintptr_t)gate & 15) || ((uintptr_t)up & 15))
    return fail(E_ARG, "tile_glu: activations and blocks must be 16-byte aligned");
  TileStreamArgs g{};
  g.w0 = (const uint8_t*)gate, g.w1 = (const uint8_t*)up, g.tables = (const uint8_t*)tables;
  g.a = x, g.token = token, g.tile_expert = tile_expert, g.out = h;
  g.experts = (int)experts, g.rows = (int)rows, g.cols = (int)cols, g.rbytes = (int)row_bytes(kind, cols);
  g.n_tiles = (int)(slots / TILE_TOKENS), g.n_src = tokens;
  return with_half_dtype(x_dtype, [&](auto* tp) {
    using XT = std::remove_pointer_t<decltype(tp)>;
    return kind == IQ3_S ? launch_stream<IQ3_S, XT, TS_GLU>(g, (hipStream_t)stream, "tile_glu")
                         : launch_stream<Q2_0, XT, TS_GLU>(g, (hipStream_t)stream, "tile_glu");
  });
}

int sh_tiles_set_share(int on) { return g_share.exchange(on ? 1 : 0); }

int sh_tile_down(int kind, const void* down, const void* tables, int64_t experts, int64_t rows, int64_t cols,
                 const void* h, int h_dtype, int64_t slots, const int32_t* tile_expert, const int32_t* pair,
                 int64_t pairs, void* out, void* stream) {
  int st = check_rows(kind, rows, cols, "tile_down");
  if (st) return st;
  if (slots <= 0 || pairs <= 0) return OK;
  if (kind != IQ3_S && kind != Q2_0) return fail(E_UNSUPPORTED, "tile_down: kind %d (Q2_0 or IQ3_S)", kind);
  if (rows % TS_RBV || cols % 64)
    return fail(E_UNSUPPORTED, "tile_down: %lld x %lld is not in blocks of %d x 64", (long long)rows,
                (long long)cols, TS_RBV);
  if (slots % TILE_TOKENS) return fail(E_SHAPE, "tile_down: %lld slots are not whole tiles of 16", (long long)slots);
  if (slots / TILE_TOKENS > (1 << 26)) return fail(E_SHAPE, "tile_down: %lld slots", (long long)slots);
  if (!down || (kind == IQ3_S && !tables) || !h || !tile_expert || !pair || !out)
    return fail(E_ARG, "tile_down: null pointer");
  if (((uintptr_t)h & 15) || ((uintptr_t)down & 15))
    return fail(E_ARG, "tile_down: activations and blocks must be 16-byte aligned");
  TileStreamArgs g{};
  g.w0 = (const uint8_t*)down, g.tables = (const uint8_t*)tables;
  g.a = h, g.pair = pair, g.tile_expert = tile_expert, g.out = out;
  g.experts = (int)experts, g.rows = (int)rows, g.cols = (int)cols, g.rbytes = (int)row_bytes(kind, cols);
  g.n_tiles = (int)(slots / TILE_TOKENS), g.n_src = pairs;
  return with_half_dtype(h_dtype, [&](auto* tp) {
    using XT = std::remove_pointer_t<decltype(tp)>;
    if (g_share.load(std::memory_order_relaxed))
      return kind == IQ3_S ? launch_stream<IQ3_S, XT, TS_DOWN_S>(g, (hipStream_t)stream, "tile_down")
                           : launch_stream<Q2_0, XT, TS_DOWN_S>(g, (hipStream_t)stream, "tile_down");
    return kind == IQ3_S ? launch_stream<IQ3_S, XT, TS_DOWN>(g, (hipStream_t)stream, "tile_down")
                         : launch_stream<Q2_0, XT, TS_DOWN>(g, (hipStream_t)stream, "tile_down");
  });
}

}  // extern "C"
