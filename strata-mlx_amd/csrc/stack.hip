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

// ---- Q2_0 stacks for 1 to 4 tokens (taken for 1 and 2), streamed by independent waves (rows a multiple of 16,
// columns of 512).
// A block's waves share nothing per item: each wave streams its own tasks (a row tile of 32 rows, or 16 when the
// matrix's rows are not a multiple of 32, x 8 blocks: 512 columns, 144 bytes a row) through its own LDS ring of
// direct loads and waits only on its own loads, so a wave's multiply overlaps the other waves' memory time with
// no barrier between them; each activation fragment read from LDS serves the tile's row groups. The block's row
// tiles (a contiguous range of the stack) are taken in units of one matrix: at a unit's start the block meets,
// turns the matrix's activations into the MFMA fragments (each value scaled by the unit of the mask that decodes
// its code) and the offset sums in LDS, and meets again; within a unit wave w takes row tiles w, w + 4, ..., all
// K-chunks of one before the next. Outputs wait in LDS and are stored when the block is done.
constexpr int SQ_WAVES = 4, SQ_KC = 8;  // waves a block; Q2_0 blocks (64 columns each) a K-chunk
// a task: RT row groups (16 RT rows) x SQ_KC blocks, 144 bytes a row, read as 9 RT 16-byte chunks a row group
template <int RT> constexpr int sq_slot() { return RT * 16 * 144; }
template <int RT> constexpr int sq_ni() { return (RT * 144 + 63) / 64; }  // direct loads a task
template <int RT> constexpr int sq_ns() { return RT == 1 ? 4 : 3; }      // ring slots a wave

struct SqPlan {
  int rows, cols, tokens, ng, nkc;  // ng: 64-column groups a row; nkc: K-chunks a row
  int64_t rbytes, mat_bytes;
  int rgm;         // row tiles (16 RT rows) a matrix
  int total, rg0;  // row tiles of the stack (< 2^31); the launch's first
  int per;         // row tiles a block
  int xs_off, nc_off, pt_off, out_off, ring_off;  // LDS byte offsets
};

template <typename XT, int RT>
__global__ __launch_bounds__(SQ_WAVES * 64) void k_stack_q2(const uint8_t* __restrict__ blocks, SqPlan P,
                                                            const XT* __restrict__ x, XT* __restrict__ out) {
  using MT = XT;
  constexpr int SQ_SLOT = sq_slot<RT>(), SQ_NI = sq_ni<RT>(), SQ_NS = sq_ns<RT>(), TR = 16 * RT;
  extern __shared__ u32x4 dyn[];
  uint8_t* lds = (uint8_t*)dyn;
  const uint32_t lds_base = SH_LDS_ADDR(dyn);
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, n = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int A = P.rg0 + (int)blockIdx.x * P.per, Bend = min(P.total, A + P.per);
  if (A >= Bend) return;
  u32x4* xs = (u32x4*)(lds + P.xs_off);   // [token][group][fragment a / b][lane group], tokens xst apart
  const int xst = P.ng * 8 + 1;           // (a token's fragments one 16-byte entry more: distinct banks)
  float* ncs = (float*)(lds + P.nc_off);  // [group][token]: minus the offsets' sum
  float* pt = (float*)(lds + P.pt_off);   // [token][group][lane group]: the sum's four parts
  XT* obuf = (XT*)(lds + P.out_off);      // [row tile - A][token][16 RT rows]
  const uint32_t ring = lds_base + P.ring_off + wave * SQ_NS * SQ_SLOT;
  const uint8_t* ringp = lds + P.ring_off + wave * SQ_NS * SQ_SLOT;

  // the lane's chunks of a task: chunk 64 i + lane = 16-byte piece c % 9 of row c / 9 (rows 144 bytes apart in
  // the ring: their 16-bit reads fall in distinct banks)
  uint32_t coff[SQ_NI];
#pragma unroll
  for (int i = 0; i < SQ_NI; ++i) {
    const int c = min(64 * i + lane, TR * 9 - 1);
    coff[i] = (uint32_t)((c / 9) * P.rbytes + 16 * (c % 9));
  }
  // a wave's tasks: (row tile, K-chunk), units in order, row tiles w, w + 4, ... of each, K-chunks in order
  struct Cur {
    int rg, ue, m, kc;  // the row tile (-1: no more), its unit's end and matrix, the K-chunk
  };
  const int m_first = A / P.rgm;
  auto settle = [&](Cur& c, int us, int m) {  // the first unit from us (of matrix m) holding a row tile of the wave
    c.m = m;
    c.ue = min(Bend, (m + 1) * P.rgm);
    while (us < Bend && us + wave >= c.ue) {
      us = c.ue;
      c.ue = min(Bend, (++c.m + 1) * P.rgm);
    }
    c.rg = us < Bend ? us + wave : -1;
    c.kc = 0;
  };
  auto next = [&](Cur& c) {
    if (++c.kc < P.nkc) return;
    c.kc = 0;
    c.rg += SQ_WAVES;
    if (c.rg >= c.ue) settle(c, c.ue, c.m + 1);
  };
  auto issue = [&](const Cur& c, int slot) {
    const int r0 = (c.rg - c.m * P.rgm) * TR;
    const uint8_t* src = blocks + (int64_t)c.m * P.mat_bytes + (int64_t)r0 * P.rbytes + c.kc * (SQ_KC * 18);
    const uint32_t dst = ring + slot * SQ_SLOT;
#pragma unroll
    for (int i = 0; i < SQ_NI - 1; ++i) lds_dma16(src, coff[i], dst + 1024 * i);
    if (lane < TR * 9 - 64 * (SQ_NI - 1)) lds_dma16(src, coff[SQ_NI - 1], dst + 1024 * (SQ_NI - 1));
  };

  Cur ci, cc;
  settle(ci, A, m_first);
  cc = ci;
  int n_issued = 0, n_done = 0;
  for (int k = 0; k < SQ_NS - 1 && ci.rg >= 0; ++k) {
    issue(ci, n_issued % SQ_NS);
    ++n_issued;
    next(ci);
  }
  const DecodeRegs kr = decode_regs<Q2_0, MT>();
  const int tok_n = (n & 3) == 0 && (n >> 2) < P.tokens ? n >> 2 : 0;  // the lane's A-row token (TPG 1 layout)
  const int tok_g = min(g, P.tokens - 1);                             // its D-row 4g's token
  float acc[RT];
#pragma unroll
  for (int r = 0; r < RT; ++r) acc[r] = 0.0f;
  for (int us = A, m = m_first; us < Bend; ++m) {
    const int ue = min(Bend, (m + 1) * P.rgm);
    __syncthreads();  // every wave is done with the last unit's fragments
    for (int e = tid; e < P.tokens * P.ng * 4; e += SQ_WAVES * 64) {
      const int t = e / (P.ng * 4), j = (e >> 2) % P.ng, gg = e & 3;
      const XT* xr = x + ((int64_t)m * P.tokens + t) * P.cols + j * 64;
      const u32x4 v0 = *(const u32x4*)(xr + 8 * gg), v1 = *(const u32x4*)(xr + 32 + 8 * gg);
      const XT* h0 = (const XT*)&v0;
      const XT* h1 = (const XT*)&v1;
      float p = 0.0f;
      uint32_t w[2][4];
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const float inv = 1.0f / q2_unit<MT>(jj);  // a power of two: exact
          const MT s0 = from_f32<MT>(to_f32(h0[4 * a + jj]) * inv);
          const MT s1 = from_f32<MT>(to_f32(h1[4 * a + jj]) * inv);
          p += (Magic<MT>::BASE + q2_unit<MT>(jj)) * (to_f32(s0) + to_f32(s1));
          w[a][jj] = (uint32_t)__builtin_bit_cast(uint16_t, s0) | ((uint32_t)__builtin_bit_cast(uint16_t, s1) << 16);
        }
      xs[t * xst + (j * 2 + 0) * 4 + gg] = u32x4{w[0][0], w[0][1], w[0][2], w[0][3]};
      xs[t * xst + (j * 2 + 1) * 4 + gg] = u32x4{w[1][0], w[1][1], w[1][2], w[1][3]};
      pt[(t * P.ng + j) * 4 + gg] = p;
    }
    __syncthreads();
    for (int e = tid; e < P.tokens * P.ng; e += SQ_WAVES * 64) {
      const float* q = pt + e * 4;
      ncs[(e % P.ng) * P.tokens + e / P.ng] = -((q[0] + q[1]) + (q[2] + q[3]));
    }
    __syncthreads();
    for (; cc.rg >= 0 && cc.rg < ue; next(cc)) {
      // the slot this issue refills was read by the task before: its reads are back
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (ci.rg >= 0) {
        issue(ci, n_issued % SQ_NS);
        ++n_issued;
        next(ci);
      }
      if (n_issued - 1 - n_done == SQ_NS - 1)  // the steady state: the other slots' loads in flight
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(SQ_NI * (SQ_NS - 1)) : "memory");
      else
        wait_vmcnt(SQ_NI * (n_issued - 1 - n_done));
      const uint8_t* slot = ringp + (n_done % SQ_NS) * SQ_SLOT + n * (SQ_KC * 18);
      const int gb = cc.kc * SQ_KC;
      uint32_t w0[RT][SQ_KC], w1[RT][SQ_KC], dh[RT][SQ_KC];
      u32x4 xa[SQ_KC], xb[SQ_KC];
      float nc[SQ_KC];
#pragma unroll
      for (int j = 0; j < SQ_KC; ++j) {
#pragma unroll
        for (int r = 0; r < RT; ++r) {
          const uint8_t* b = slot + r * 16 * (SQ_KC * 18) + j * 18;
          w0[r][j] = *(const uint16_t*)(b + 2 + 2 * g);
          w1[r][j] = *(const uint16_t*)(b + 10 + 2 * g);
          dh[r][j] = *(const uint16_t*)b;
        }
        xa[j] = xs[tok_n * xst + ((gb + j) * 2 + 0) * 4 + g];
        xb[j] = xs[tok_n * xst + ((gb + j) * 2 + 1) * 4 + g];
        nc[j] = ncs[(gb + j) * P.tokens + tok_g];
      }
#pragma unroll
      for (int j = 0; j < SQ_KC; ++j)
#pragma unroll
      for (int r = 0; r < RT; ++r) {
        const uint32_t W = w0[r][j] | (w1[r][j] << 16), W8 = W >> 8;
        u32x4 fa, fb;
        fa.x = (W & kr.m0) | kr.magic;
        fa.y = (W & kr.m1) | kr.magic;
        fa.z = (W & kr.m2) | kr.magic;
        fb.x = (W8 & kr.m0) | kr.magic;
        fb.y = (W8 & kr.m1) | kr.magic;
        fb.z = (W8 & kr.m2) | kr.magic;
        if constexpr (std::is_same_v<MT, bf16>) {  // bit 7 of a bf16 half is exponent: code 3 shifted down
          fa.w = ((W >> 6) & kr.m0) | kr.magic;
          fb.w = ((W >> 14) & kr.m0) | kr.magic;
        } else {
          fa.w = (W & (kr.m2 << 2)) | kr.magic;
          fb.w = (W8 & (kr.m2 << 2)) | kr.magic;
        }
        f32x4 D = mfma<MT>(xa[j], fa, f32x4{0.0f, 0.0f, 0.0f, 0.0f});
        D = mfma<MT>(xb[j], fb, D);
        acc[r] = fmaf(half_bits(dh[r][j]), D[0] + nc[j], acc[r]);
      }
      if (cc.kc == P.nkc - 1) {  // the row tile is done: lane (g, n) holds token g's row 16 r + n
#pragma unroll
        for (int r = 0; r < RT; ++r) {
          if (g < P.tokens) obuf[((cc.rg - A) * P.tokens + g) * TR + 16 * r + n] = from_f32<XT>(acc[r]);
          acc[r] = 0.0f;
        }
      }
      ++n_done;
    }
    us = ue;
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  const int nout = (Bend - A) * P.tokens * TR;
  for (int e = tid; e < nout; e += SQ_WAVES * 64) {
    const int rg = A + e / (P.tokens * TR);
    const int t = (e / TR) % P.tokens;
    const int m = rg / P.rgm, row = (rg - m * P.rgm) * TR + e % TR;
    out[((int64_t)m * P.tokens + t) * P.rows + row] = obuf[e];
  }
}

template <typename XT, int RT>
static int launch_stack_q2(const uint8_t* blocks, int64_t n_mats, int64_t rows, int64_t cols, const XT* x,
                           int64_t tokens, XT* out, hipStream_t stream, bool dry) {
  constexpr int TR = 16 * RT;
  constexpr size_t ring = (size_t)SQ_WAVES * sq_ns<RT>() * sq_slot<RT>();
  SqPlan P{};
  P.rows = (int)rows;
  P.cols = (int)cols;
  P.tokens = (int)tokens;
  P.ng = (int)(cols / 64);
  P.nkc = (int)(cols / (64 * SQ_KC));
  P.rbytes = row_bytes(Q2_0, cols);
  P.mat_bytes = rows * P.rbytes;
  P.rgm = (int)(rows / TR);
  P.total = (int)(n_mats * P.rgm);
  const size_t xs = (size_t)tokens * (P.ng * 8 + 1) * 16, nc = (size_t)P.ng * tokens * 4, pt = (size_t)tokens * P.ng * 16;
  const size_t out_cap = 16 * 1024;  // outputs a block holds at most
  const int per_cap = (int)(out_cap / (tokens * TR * sizeof(XT)));
  P.xs_off = 0;
  P.nc_off = (int)xs;
  P.pt_off = (int)(xs + nc);
  const size_t fixed = xs + nc + pt;
  const int cus = device_cus();
  // blocks a CU: as many as LDS holds (up to 4), the outputs sized for the launch's share
  int per_cu = 4, per = 0;
  size_t lds = 0;
  for (; per_cu >= 1; --per_cu) {
    per = (int)std::min<int64_t>(per_cap, (P.total + (int64_t)cus * per_cu - 1) / ((int64_t)cus * per_cu));
    const size_t ob = ((size_t)per * tokens * TR * sizeof(XT) + 15) & ~(size_t)15;
    lds = ((fixed + 15) & ~(size_t)15) + ob + ring;
    if ((size_t)per_cu * lds <= 160 * 1024) break;
  }
  if (per_cu < 1) return fail(E_UNSUPPORTED, "stack_matvec: %zu bytes of LDS", lds);
  P.per = per;
  P.out_off = (int)((fixed + 15) & ~(size_t)15);
  P.ring_off = (int)(lds - ring);
  if (lds > 128 * 1024)
    return fail(E_UNSUPPORTED, "stack_matvec: ring past the direct-load range");
  if (dry) return OK;
  const int64_t grid = (int64_t)cus * per_cu, window = grid * per;
  for (int64_t r = 0; r < P.total; r += window) {
    P.rg0 = (int)r;
    const int64_t nb = std::min<int64_t>(grid, (P.total - r + per - 1) / per);
    hipLaunchKernelGGL((k_stack_q2<XT, RT>), dim3((unsigned)nb), dim3(SQ_WAVES * 64), lds, stream, blocks, P, x, out);
    const int st = check_launch("stack_matvec");
    if (st) return st;
  }
  return OK;
}

template <int KIND, typename XT, int TPG, int GPER, int RW>
static int launch_stack(const uint8_t* blocks, const uint8_t* tables, int64_t n_mats, int64_t rows, int64_t cols,
                        const XT* x, int64_t tokens, XT* out, bool few, hipStream_t stream, bool dry) {
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
  if (dry) return OK;
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

}  // extern "C"

// The stack matvec's checks and plan, then its launches (dry: the checks and the plan only, nothing launched).
static int stack_matvec(bool dry, int kind, const void* blocks, const void* tables, int64_t n_mats, int64_t rows,
                        int64_t cols, const void* x, int x_dtype, int64_t tokens, void* out, void* stream) {
  int st = check_rows(kind, rows, cols, "stack_matvec");
  if (st) return st;
  if (n_mats <= 0 || tokens <= 0) return OK;
  if (tokens > 16) return fail(E_SHAPE, "stack_matvec: %lld tokens a matrix (at most 16)", (long long)tokens);
  if (n_mats * ((rows + 15) / 16) > (1ll << 31) - 1 || rows * row_bytes(kind, cols) > (1ll << 31) - 1)
    return fail(E_SHAPE, "stack_matvec: %lld matrices of %lld x %lld too many", (long long)n_mats, (long long)rows,
                (long long)cols);
  // the other kinds, float32 activations and rows the MFMA decode does not tile: the streaming kernel of exact
  // weights and float32 sums (stream.hip), which refuses what it does not take
  if (!mfma_kind_host(kind) || (x_dtype != BF16 && x_dtype != F16) || cols % 256)
    return stream_matvec(dry, kind, blocks, tables, n_mats, rows, cols, x, x_dtype, tokens, out, stream);
  if (!blocks || !x || (!out && !dry) || (kind == IQ3_S && !tables)) return fail(E_ARG, "stack_matvec: null pointer");
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
  // the groups split evenly over the waves: IQ3_S rows past 4096 columns (16 runs a wave) in whole 512s
  if (ngroups / gper1 > 16 || ngroups % gper1)
    return fail(E_UNSUPPORTED, "stack_matvec: %lld columns (at most %d%s)", (long long)cols,
                16 * gper1 * (kind == Q2_0 ? 64 : 32), kind == IQ3_S ? ", past 4096 a multiple of 512" : "");
  const int tpg = tokens <= 4 ? 1 : tokens <= 8 ? 2 : 4;
  // few items to go round the CUs: one row group a block, one item a block
  const int64_t kw1 = ngroups / gper1, ir = rw2_shape ? 32 : 16 * std::max<int64_t>(1, (kind == Q2_0 ? 8 : 16) / kw1);
  const bool few = n_mats * ((rows + ir - 1) / ir) < 2 * (int64_t)device_cus();
  const bool rw2 = rw2_shape && !few;
  const int gper = rw2 ? (int)small : gper1;
  // Q2_0 for 1 or 2 tokens, whole row groups and 512-column chunks, many row groups: the wave-streamed kernel
  // (measured on the 3072 x 2048 stream: 4.1 against 3.3 TB/s at one token, even at four)
  const bool q2_stream = kind == Q2_0 && tokens <= 2 && rows % 16 == 0 && cols % 512 == 0 &&
                         ((uintptr_t)blocks & 15) == 0 && n_mats * (rows / 16) >= 4 * (int64_t)device_cus() &&
                         n_mats * (rows / 16) < (1ll << 31);
  return with_half_dtype(x_dtype, [&](auto* tp) {
    using XT = std::remove_pointer_t<decltype(tp)>;
    if (q2_stream && rows % 32 == 0)
      return launch_stack_q2<XT, 2>((const uint8_t*)blocks, n_mats, rows, cols, (const XT*)x, tokens, (XT*)out,
                                    (hipStream_t)stream, dry);
    if (q2_stream)
      return launch_stack_q2<XT, 1>((const uint8_t*)blocks, n_mats, rows, cols, (const XT*)x, tokens, (XT*)out,
                                    (hipStream_t)stream, dry);
    auto go = [&](auto kc, auto gc, auto tc) {
      constexpr int K = decltype(kc)::value, G = decltype(gc)::value, T = decltype(tc)::value;
      if (rw2)
        return launch_stack<K, XT, T, G, 2>((const uint8_t*)blocks, (const uint8_t*)tables, n_mats, rows, cols,
                                            (const XT*)x, tokens, (XT*)out, few, (hipStream_t)stream, dry);
      return launch_stack<K, XT, T, G, 1>((const uint8_t*)blocks, (const uint8_t*)tables, n_mats, rows, cols,
                                          (const XT*)x, tokens, (XT*)out, few, (hipStream_t)stream, dry);
    };
    auto by_t = [&](auto kc, auto gc) {
      return tpg == 1 ? go(kc, gc, kind_c<1>{}) : tpg == 2 ? go(kc, gc, kind_c<2>{}) : go(kc, gc, kind_c<4>{});
    };
    if (kind == Q2_0) return gper == 8 ? by_t(kind_c<Q2_0>{}, kind_c<8>{}) : by_t(kind_c<Q2_0>{}, kind_c<4>{});
    return gper == 16 ? by_t(kind_c<IQ3_S>{}, kind_c<16>{}) : by_t(kind_c<IQ3_S>{}, kind_c<8>{});
  });
}

extern "C" {

int sh_stack_matvec(int kind, const void* blocks, const void* tables, int64_t n_mats, int64_t rows, int64_t cols,
                    const void* x, int x_dtype, int64_t tokens, void* out, void* workspace, size_t workspace_bytes,
                    void* stream) {
  return stack_matvec(false, kind, blocks, tables, n_mats, rows, cols, x, x_dtype, tokens, out, stream);
}

int sh_stack_takes(int kind, const void* blocks, const void* tables, int64_t n_mats, int64_t rows, int64_t cols,
                   const void* x, int x_dtype, int64_t tokens) {
  return stack_matvec(true, kind, blocks, tables, n_mats, rows, cols, x, x_dtype, tokens, nullptr, nullptr) == OK;
}

}  // extern "C"
