// Decode attention over a paged KV cache, split over the context, GQA: the query heads that share a KV head are
// that head's query rows — strata-mlx's `_gathered` (strata_mlx/attention.py:144-165), which attends each query to
// its cell list with the group of query heads as the rows of one SDPA, taken to a page table: position p of the
// context is cell table[p / 16] * 16 + p % 16. The window's B queries are the last B positions; query t sees
// positions 0 .. ctx - B + t (the causal mask among drafts, attention.py:118-129). The same kernel also takes
// `_gathered`'s own form: a list of cells per query, each with a validity flag (attention.py:132-141).
//
// Split-K: block (split, unit, row group) runs the online softmax over its run of 16-position tiles for up to 64
// query rows and leaves (max, sum, unnormalised output) in a workspace; a second kernel merges the splits.
//
// Per tile, on MFMA (16x16x32 bf16/f16 for scores, 16x16x16 for the values):
//   S^T = K Q^T: K (16 positions x D) is the A operand read from LDS, Q^T the B operand held in registers, so a
//        lane (g, n) holds the scores of positions 4g..4g+3 for query row n;
//   O += P V:    that is exactly the A operand layout of P for 16x16x16 (row n, positions 4g..4g+3); V (16 x D)
//        is the B operand, read from LDS; O[row 4g + i][dim n] accumulates in registers, 16 dims a tile.
// The block's tiles come into LDS by direct 16-byte loads (no registers), two steps of tiles in flight, every
// destination below 128 KiB. Rows of K and V are not padded: chunk c of position r sits at chunk c ^ (r % 16) of
// its row, so the 16 positions a K read touches, and the 4 rows a V read touches, fall in distinct banks.
#include <type_traits>

#include "launch.h"
#include "xmv.h"

namespace sh {

struct AttnArgs {
  const void* q;             // (n_q, hq, D)
  const void* k;             // paged: (pages, hkv, 16, D); cells: (hkv, kv_len, D)
  const void* v;
  const int32_t* table;      // paged: physical page of each tile of 16 positions; cells: (n_q, ctx) cell ids
  const uint8_t* real;       // cells: (n_q, ctx) validity; paged: null
  float* ws;                 // the workspace: wm, wl [splits][units][rows] max and sum; wo the outputs, as the
  float *wm, *wl, *wo;       // lanes hold them: [splits][units][zgroups][4 row tiles][D / 16][64 lanes][4 rows]
  void* out;                 // (n_q, hq, D)
  int n_q, hq, hkv, ctx;     // ctx: paged context length, or cells a query
  int64_t kv_len;            // cells: rows of one KV head; paged: pages in the pool
  int tiles, tiles_per_split, splits, units, rows;  // rows: query rows of a unit (paged n_q * group, cells group)
  float scale_log2;          // scale * log2(e)
  const void* gate;          // optional output gate: out = out * sigmoid(gate), gate element (query t, head h, dim d)
  int64_t gate_ts, gate_hs;  // at gate[t * gate_ts + h * gate_hs + d]
  const int32_t* cell_pages;  // cells over a paged pool: cell c at page cell_pages[c / 16], slot c % 16 (else null)
  int64_t cell_npages;
};

constexpr int ATT_WAVES = 4, ATT_NT = 256;
constexpr int ATT_DMA_LIMIT = 128 * 1024;             // direct loads into LDS land below this address
template <int D> constexpr int att_part_insts() { return 16 * D / 8 / 64; }  // a tile's K or V: 16 rows of D
template <int D> constexpr int att_part_bytes() { return 16 * D * 2; }

template <typename XT> __device__ __forceinline__ f32x4 mfma16x16x16(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1,
                                                                     f32x4 c) {
  typedef short s4 __attribute__((ext_vector_type(4)));
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  const uint64_t a = (uint64_t)a0 | ((uint64_t)a1 << 32), b = (uint64_t)b0 | ((uint64_t)b1 << 32);
  if constexpr (std::is_same_v<XT, bf16>)
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s4, a), __builtin_bit_cast(s4, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(h4, a), __builtin_bit_cast(h4, b), c, 0, 0, 0);
}

typedef short v4i16 __attribute__((ext_vector_type(4)));

template <typename XT> __device__ __forceinline__ uint32_t pack_pair(float lo, float hi) {
  return (uint32_t)__builtin_bit_cast(uint16_t, from_f32<XT>(lo)) |
         ((uint32_t)__builtin_bit_cast(uint16_t, from_f32<XT>(hi)) << 16);
}

// Block: 4 waves; RT4 row tiles of 16 rows (1, 2 or 4) x PL = 4 / RT4 tile phases. A step stages PL tiles; wave
// (rt, ph) multiplies row tile rt against the step's tile ph.
template <typename XT, int D, bool CELLS>
__global__ __launch_bounds__(ATT_NT, 3) void k_attn_split(AttnArgs a) {  // (3 blocks a CU by registers)
  constexpr int NC = D / 32, NDT = D / 16, PI = att_part_insts<D>(), NCH = D / 8;  // NCH: chunks a row
  constexpr int PB = att_part_bytes<D>(), RS = D * 2;  // bytes a staged row
  extern __shared__ u32x4 dyn[];
  const uint32_t lds_base = SH_LDS_ADDR(dyn);
  const uint8_t* lds = (const uint8_t*)dyn;
  const int lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int split = blockIdx.x, unit = blockIdx.y, zrow = blockIdx.z * 64;
  const int group = a.hq / a.hkv;
  const int h = CELLS ? unit % a.hkv : unit;
  const int qcell = CELLS ? unit / a.hkv : 0;  // cells form: the unit's one query
  const int rows_here = min(64, a.rows - zrow);
  const int RT = (rows_here + 15) / 16, RT4 = RT <= 1 ? 1 : RT <= 2 ? 2 : 4, PL = ATT_WAVES / RT4;
  const int rt = wave % RT4, ph = wave / RT4;
  const int t0 = split * a.tiles_per_split, t1 = min(a.tiles, t0 + a.tiles_per_split);
  const int steps = (t1 - t0 + PL - 1) / PL;
  const int step_bytes = 2 * PL * PB;  // K and V of PL tiles

  // ---- this wave's direct loads of a step: instruction q of the step's 2 * PL * PI is wave q % 4's
  const int n_inst = 2 * PL * PI;
  const int my_insts = (n_inst - wave + ATT_WAVES - 1) / ATT_WAVES;
  const XT* kb = (const XT*)a.k;
  const XT* vb = (const XT*)a.v;
  // the split's page ids (paged) or cell ids and flags (cells), staged in LDS once: the loads of a step then
  // wait on no global read
  int32_t* tab = (int32_t*)(lds + 2 * step_bytes);
  uint8_t* flags = (uint8_t*)(tab + (CELLS ? 16 : 1) * a.tiles_per_split);
  {
    const int n = CELLS ? min(16 * (t1 - t0), a.ctx - 16 * t0) : t1 - t0;
    const int32_t* src = CELLS ? a.table + (int64_t)qcell * a.ctx + 16 * t0 : a.table + t0;
    // ids outside the pool are clamped into it: a bad table gives wrong numbers, never a load outside K and V
    const int hi = (int)(a.kv_len - 1);
    for (int i = threadIdx.x; i < n; i += ATT_NT) {
      int id = min(max(src[i], 0), hi);
      if (CELLS && a.cell_pages) {  // the cell's row in the pool less its head's 16 rows: page * hkv * 16 + slot
        const int64_t pg = min(max((int64_t)a.cell_pages[id >> 4], (int64_t)0), a.cell_npages - 1);
        id = (int)(pg * a.hkv * 16 + (id & 15));
      }
      tab[i] = id;
    }
    if constexpr (CELLS) {
      const uint8_t* rs = a.real + (int64_t)qcell * a.ctx + 16 * t0;
      for (int i = threadIdx.x; i < 16 * (t1 - t0); i += ATT_NT) flags[i] = i < n ? rs[i] : 0;
    }
    lds_sync();
  }
  auto row_off = [&](int tile, int tok) -> int64_t {  // elements from the K / V base to a tile position's row
    if constexpr (CELLS) {
      const int i = min((tile - t0) * 16 + tok, a.ctx - 16 * t0 - 1);
      return ((int64_t)h * (a.cell_pages ? 16 : a.kv_len) + tab[i]) * D;
    } else {
      const int64_t phys = tab[tile - t0];
      return ((phys * a.hkv + h) * 16 + tok) * D;
    }
  };
  auto issue = [&](int step) {
    const uint32_t buf = lds_base + (step & 1) * step_bytes;
    for (int q = wave; q < n_inst; q += ATT_WAVES) {
      const int part = q / PI, j = q - part * PI;  // part: tile ph' = part / 2, K (0) or V (1)
      const int tile = min(t0 + step * PL + part / 2, t1 - 1);
      const int s = j * 64 + lane;                          // slot: chunk s % NCH of row s / NCH
      const int tok = s / NCH, piece = (s % NCH) ^ (tok & 15);  // the chunk that slot holds
      const int64_t off = (row_off(tile, tok) + 8 * piece) * (int64_t)sizeof(XT);
      lds_dma16(part & 1 ? (const void*)vb : (const void*)kb, (uint32_t)off, buf + part * PB + j * 1024);
    }
  };

  // ---- Q^T fragments (B operand of S^T = K Q^T): lane (g, n) holds row n's dims c*32 + 8g .. +7
  const int r_local = 16 * rt + n;                     // the lane's B column: its query row within the block
  const int row = zrow + min(r_local, rows_here - 1);  // padding rows repeat the last real one (never stored)
  const int qt = CELLS ? qcell : row / group, qh = h * group + (CELLS ? row : row % group);
  const XT* qrow = (const XT*)a.q + ((int64_t)qt * a.hq + qh) * D;
  u32x4 qf[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) qf[c] = *(const u32x4*)(qrow + c * 32 + 8 * g);
  // the last position the lane's query row may see (paged: causal among the window's queries)
  const int vis_last = CELLS ? a.ctx - 1 : a.ctx - a.n_q + qt;

  float m_run = -INFINITY, l_run = 0.0f;  // for query row n (replicated over g)
  f32x4 O[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) O[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  if (steps > 0) issue(0);
  for (int st = 0; st < steps; ++st) {
    const bool more = st + 1 < steps;
    if (more) issue(st + 1);
    wait_vmcnt(more ? my_insts : 0);
    lds_sync();
    const int tile = t0 + st * PL + ph;
    if (rt < RT && tile < t1) {
      const uint8_t* kt = lds + (st & 1) * step_bytes + (2 * ph) * PB;
      const uint8_t* vt = kt + PB;
      // scores of positions 4g..4g+3 for row n
      f32x4 S = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const u32x4 kf = *(const u32x4*)(kt + n * RS + 16 * ((4 * c + g) ^ n));
        S = mfma<XT>(kf, qf[c], S);
      }
      float sv[4], mx = -INFINITY;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int pos = tile * 16 + 4 * g + i;
        bool ok;
        if constexpr (CELLS) ok = flags[pos - 16 * t0] != 0;
        else ok = pos < a.ctx && pos <= vis_last;
        sv[i] = ok ? S[i] * a.scale_log2 : -INFINITY;
        mx = fmaxf(mx, sv[i]);
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m_run, mx);
      const float base = m_new == -INFINITY ? 0.0f : m_new;  // a row with nothing visible yet stays at zero
      const float alpha = exp2f(m_run - base);
      float p[4], ps = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p[i] = exp2f(sv[i] - base);
        ps += p[i];
      }
      ps += __shfl_xor(ps, 16);
      ps += __shfl_xor(ps, 32);
      l_run = l_run * alpha + ps;
      m_run = m_new;
      // O rows are 4g + i: their factors sit with the lanes whose column is that row
      if (__any(alpha != 1.0f)) {
        float ar[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) ar[i] = __shfl(alpha, 4 * g + i);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
          for (int i = 0; i < 4; ++i) O[dt][i] *= ar[i];
      }
      const uint32_t pa0 = pack_pair<XT>(p[0], p[1]), pa1 = pack_pair<XT>(p[2], p[3]);
      // V fragments by transposing LDS reads: within each 16-lane group, lane i receives element i % 4 of the
      // 8-byte pieces named by lanes i / 4 + 4m (m = 0..3). Lane (g, n) names row 4g + n / 4, dims
      // 16 dt + 4 (n % 4) .. + 3, so it receives V[4g + m][16 dt + n], m = 0..3: the B operand of O += P V.
      const int vr = 4 * g + (n >> 2), vq = n & 3;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const int cv = 2 * dt + (vq >> 1);  // the 16-byte chunk of dims 16 dt + 4 vq
        const uint8_t* vp = vt + vr * RS + 16 * (cv ^ (vr & 15)) + 8 * (vq & 1);
        const v4i16 vv = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16*)vp);
        const uint32_t b0 = (uint32_t)(uint16_t)vv[0] | ((uint32_t)(uint16_t)vv[1] << 16);
        const uint32_t b1 = (uint32_t)(uint16_t)vv[2] | ((uint32_t)(uint16_t)vv[3] << 16);
        O[dt] = mfma16x16x16<XT>(pa0, pa1, b0, b1, O[dt]);
      }
    }
    lds_sync();  // every wave is done with this step's buffer before the step after next fills it
  }

  // ---- merge the PL phases of each row tile in LDS, then the first phase's wave writes the split's partial
  // [ph][rt][64 lanes]: m, l; then O as [ph][rt][dim tile][64 lanes] of the lanes' four accumulators (16-byte
  // stores and loads, consecutive across lanes: no bank conflicts)
  float* red = (float*)dyn;
  f32x4* redo = (f32x4*)(red + 2 * ATT_WAVES * 64);
  if (PL > 1) {
    red[(ph * RT4 + rt) * 64 + lane] = m_run;
    red[ATT_WAVES * 64 + (ph * RT4 + rt) * 64 + lane] = l_run;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) redo[((ph * RT4 + rt) * NDT + dt) * 64 + lane] = O[dt];
    lds_sync();
    if (ph == 0) {
      // lane (g, n): its column row n for m, l; O rows 4g + i
      float m_all = m_run;
      for (int p2 = 1; p2 < PL; ++p2) m_all = fmaxf(m_all, red[(p2 * RT4 + rt) * 64 + lane]);
      const float base = m_all == -INFINITY ? 0.0f : m_all;
      float l_all = 0.0f;
      for (int p2 = 0; p2 < PL; ++p2)
        l_all += red[ATT_WAVES * 64 + (p2 * RT4 + rt) * 64 + lane] * exp2f(red[(p2 * RT4 + rt) * 64 + lane] - base);
      // O rows 4g + i: phase by phase (the first is this wave's own), all NDT reads of a phase in flight at once
      float bq[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) bq[i] = __shfl(base, 4 * g + i);
      for (int p2 = 0; p2 < PL; ++p2) {
        float fr[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) fr[i] = exp2f(red[(p2 * RT4 + rt) * 64 + 4 * g + i] - bq[i]);
        if (p2 == 0) {
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              float o = 0.0f;
              o += O[dt][i] * fr[i];
              O[dt][i] = o;
            }
        } else {
          f32x4 v[NDT];
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) v[dt] = redo[((p2 * RT4 + rt) * NDT + dt) * 64 + lane];
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int i = 0; i < 4; ++i) O[dt][i] += v[dt][i] * fr[i];
        }
      }
      m_run = m_all;
      l_run = l_all;
    }
  }
  if (ph == 0 && rt < RT) {
    const int64_t su = (int64_t)split * a.units + unit;
    if (g == 0 && r_local < rows_here) {  // lane's column row: max and sum
      a.wm[su * a.rows + zrow + r_local] = m_run;
      a.wl[su * a.rows + zrow + r_local] = l_run;
    }
    // the outputs as the lanes hold them (rows 4g + i of the row tile, dim 16 dt + n): a 16-byte store a dim tile
    f32x4* wo = (f32x4*)a.wo + ((su * gridDim.z + blockIdx.z) * 4 + rt) * NDT * 64;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) wo[dt * 64 + lane] = O[dt];
  }
}

// merge the splits of 4 rows x 16 dims (block (dim tile, row quad, unit x row group)):
// out = sum_s O_s 2^(m_s - m) / sum_s l_s 2^(m_s - m); a row that sees no position (every cell masked) gives zeros.
// Its time is memory latency and the misses one CU keeps in flight, so the merge spreads over many small blocks
// (a row quad's 64 floats of a dim tile: 256 consecutive bytes a split, a coalesced read a wave) and each thread keeps
// many loads in flight. The block's 16 waves share the splits: wave w sums its sixteenth, in split order, and the
// 16 sums add in wave order. Its first chunk of partial outputs is on the way while the block turns the 4 rows'
// maxima and sums of every split (4 a thread, in one round) into factors in LDS. C, the loads of a chunk, is 8 when
// that holds a sixteenth of the splits, else 16 (two chunks in flight).
constexpr int ATT_MAX_SPLITS = 1024;
constexpr int ATT_MERGE_NT = 1024;

template <typename XT, int D, bool CELLS, int C>
__global__ __launch_bounds__(ATT_MERGE_NT) void k_attn_merge(AttnArgs a) {
  extern __shared__ float fac[];  // [splits][4] maxima, then factors; then [splits][4] sums
  __shared__ float s_red[2][16], s_inv[4];
  __shared__ float s_part[16][64];
  static_assert(ATT_MAX_SPLITS <= 4 * 256, "one round of 4 loads a thread covers the splits");
  constexpr int NDT = D / 16;
  const int tid = threadIdx.x;
  const int zgroups = CELLS ? 1 : (a.rows + 63) / 64;
  const int dt = blockIdx.x, quad = blockIdx.y, unit = blockIdx.z / zgroups, zg = blockIdx.z % zgroups;
  const int row0 = zg * 64 + 4 * quad;
  if (row0 >= a.rows) return;  // the last row group's padding quads (the whole block)
  const int S = a.splits;
  float* sums = fac + S * 4;
  // wave w, lane t: element t of the quad's 64 floats (row row0 + t % 4, dim 16 dt + t / 4), splits [w Q, w Q + Q)
  const int w = tid >> 6, t = tid & 63, Q = (S + 15) / 16, s_lo = w * Q;
  const int64_t ostride = (int64_t)a.units * zgroups * 4 * NDT * 256;  // floats a split
  const float* od = a.wo + ((((int64_t)unit * zgroups + zg) * 4 + (quad >> 2)) * NDT + dt) * 256 + 64 * (quad & 3) + t;
  float v[C], w2[C];
#pragma unroll
  for (int c = 0; c < C; ++c) v[c] = od[(int64_t)min(s_lo + c, S - 1) * ostride];
  {
    const int r = tid >> 8, j = tid & 255, row = row0 + r;  // 4 waves a row
    const bool real = row < a.rows;
    float m = -INFINITY;
    if (real) {
      const int64_t stride = (int64_t)a.units * a.rows;
      const float* m0 = a.wm + (int64_t)unit * a.rows + row;
      const float* l0 = a.wl + (int64_t)unit * a.rows + row;
      float mv[4], lv[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int s2 = min(256 * c + j, S - 1);
        mv[c] = m0[s2 * stride];
        lv[c] = l0[s2 * stride];
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int s2 = 256 * c + j;
        if (s2 < S) {
          fac[s2 * 4 + r] = mv[c];
          sums[s2 * 4 + r] = lv[c];
          m = fmaxf(m, mv[c]);
        }
      }
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((tid & 63) == 0) s_red[0][w] = m;
    __syncthreads();
    m = fmaxf(fmaxf(s_red[0][4 * r], s_red[0][4 * r + 1]), fmaxf(s_red[0][4 * r + 2], s_red[0][4 * r + 3]));
    const float base = m == -INFINITY ? 0.0f : m;
    float l = 0.0f;
    for (int s2 = j; s2 < S; s2 += 256) {
      float f = 0.0f;
      if (real) {
        f = exp2f(fac[s2 * 4 + r] - base);
        l += sums[s2 * 4 + r] * f;
      }
      fac[s2 * 4 + r] = f;
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) l += __shfl_xor(l, o);
    if ((tid & 63) == 0) s_red[1][w] = l;
  }
  __syncthreads();
  if (tid < 4) {
    const float l = ((s_red[1][4 * tid] + s_red[1][4 * tid + 1]) + s_red[1][4 * tid + 2]) + s_red[1][4 * tid + 3];
    s_inv[tid] = l > 0.0f ? 1.0f / l : 0.0f;
  }
  const int rq = t & 3, s_hi = min(s_lo + Q, S), nch = (Q + C - 1) / C;
  float acc = 0.0f;
  for (int k = 0; k < nch; k += 2) {
    if (k + 1 < nch) {
#pragma unroll
      for (int c = 0; c < C; ++c) w2[c] = od[(int64_t)min(s_lo + (k + 1) * C + c, S - 1) * ostride];
    }
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int s2 = s_lo + k * C + c;
      const float sum = acc + v[c] * fac[min(s2, S - 1) * 4 + rq];
      acc = s2 < s_hi ? sum : acc;
    }
    if (k + 1 >= nch) break;
    if (k + 2 < nch) {
#pragma unroll
      for (int c = 0; c < C; ++c) v[c] = od[(int64_t)min(s_lo + (k + 2) * C + c, S - 1) * ostride];
    }
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int s2 = s_lo + (k + 1) * C + c;
      const float sum = acc + w2[c] * fac[min(s2, S - 1) * 4 + rq];
      acc = s2 < s_hi ? sum : acc;
    }
  }
  s_part[w][t] = acc;
  __syncthreads();
  const int row = row0 + rq;
  if (w == 0 && row < a.rows) {
#pragma unroll
    for (int u = 1; u < 16; ++u) acc += s_part[u][t];
    const int group = a.hq / a.hkv;
    const int h = CELLS ? unit % a.hkv : unit;
    const int qt = CELLS ? unit / a.hkv : row / group, qh = h * group + (CELLS ? row : row % group);
    const int dim = 16 * dt + (t >> 2);
    XT o = from_f32<XT>(acc * s_inv[rq]);
    if (a.gate) {  // attention.py:261: out * sigmoid(gate), the sigmoid and the product each rounded to the type
      const float g = to_f32(((const XT*)a.gate)[qt * a.gate_ts + qh * a.gate_hs + dim]);
      o = from_f32<XT>(to_f32(o) * to_f32(from_f32<XT>(1.0f / (1.0f + expf(-g)))));
    }
    ((XT*)a.out)[((int64_t)qt * a.hq + qh) * D + dim] = o;
  }
}

static int attn_cus() {
  static int cus = 0;
  if (!cus) {
    int dev = 0;
    (void)hipGetDevice(&dev);
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (cus <= 0) cus = 256;
  }
  return cus;
}

// splits of the context: one round of blocks over the chip (as many a CU as LDS holds), at least one step of
// tiles a split (`min_tiles`), at most ATT_MAX_SPLITS splits
static void plan_splits(AttnArgs& a, int zgroups, int min_tiles, int per_cu) {
  const int64_t want = (int64_t)per_cu * attn_cus();
  const int64_t per_unit = std::max<int64_t>(1, want / ((int64_t)a.units * zgroups));
  int64_t tps = std::max<int64_t>(min_tiles, (a.tiles + per_unit - 1) / per_unit);
  tps = std::max<int64_t>(tps, (a.tiles + ATT_MAX_SPLITS - 1) / ATT_MAX_SPLITS);
  a.tiles_per_split = (int)tps;
  a.splits = (int)((a.tiles + tps - 1) / tps);
}

static int att_phases(int rows_here) {
  const int RT = (rows_here + 15) / 16, RT4 = RT <= 1 ? 1 : RT <= 2 ? 2 : 4;
  return ATT_WAVES / RT4;
}

template <int D, bool CELLS> static size_t attn_lds(int rows_here, int tiles_per_split) {
  const int PL = att_phases(rows_here);
  const size_t stage = 2 * (size_t)(2 * PL * att_part_bytes<D>());
  const size_t tabs = CELLS ? (size_t)tiles_per_split * 16 * 5 : (size_t)tiles_per_split * 4;
  const size_t merge = PL > 1 ? sizeof(float) * (2 * ATT_WAVES * 64 + (size_t)ATT_WAVES * D * 16) : 0;
  return std::max(stage + ((tabs + 15) & ~(size_t)15), merge);
}

// tiles a split at least: a step of tiles, and enough that its partial outputs (rows x D floats) stay near a
// quarter of its K and V (16 positions x D x 2 x 2 bytes a tile)
static int att_min_tiles(int rows) { return std::max(att_phases(std::min(64, rows)), (std::min(64, rows) + 7) / 8); }

// blocks a CU by LDS (the stage and the phase merge; the tables taken at 4 KiB) and by registers (the split
// kernel's occupancy at that LDS, asked of the runtime for one representative instantiation a head size, so that
// workspace sizing and launch plan alike)
static int att_blocks_per_cu(int rows_here, int D) {
  const int PL = att_phases(rows_here);
  const size_t stage = 2 * (size_t)(2 * PL * 16 * D * 2) + 4096;
  const size_t merge = PL > 1 ? sizeof(float) * (2 * ATT_WAVES * 64 + (size_t)ATT_WAVES * D * 16) : 0;
  const size_t lds = std::max(stage, merge);
  int by_regs = 0;
  const hipError_t e = D == 256 ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&by_regs, k_attn_split<bf16, 256, false>,
                                                                             ATT_NT, lds)
                                : hipOccupancyMaxActiveBlocksPerMultiprocessor(&by_regs, k_attn_split<bf16, 128, false>,
                                                                             ATT_NT, lds);
  if (e != hipSuccess || by_regs < 1) by_regs = 1;
  return (int)std::max<size_t>(1, std::min<size_t>({8, 160 * 1024 / lds, (size_t)by_regs}));
}

template <typename XT, int D, bool CELLS> static int launch_attn(AttnArgs a, hipStream_t stream) {
  const int zgroups = CELLS ? 1 : (a.rows + 63) / 64;
  plan_splits(a, zgroups, att_min_tiles(a.rows), att_blocks_per_cu(std::min(64, a.rows), D));
  // the last row group may have fewer rows, more tile phases and so a larger stage
  const size_t lds = std::max(attn_lds<D, CELLS>(std::min(64, a.rows), a.tiles_per_split),
                              attn_lds<D, CELLS>(a.rows - 64 * (zgroups - 1), a.tiles_per_split));
  static_assert(2 * 2 * ATT_WAVES * att_part_bytes<D>() <= ATT_DMA_LIMIT, "the stage fits under the load limit");
  if (lds > 160 * 1024) return fail(E_UNSUPPORTED, "attention: %zu bytes of LDS", lds);
  hipLaunchKernelGGL((k_attn_split<XT, D, CELLS>), dim3(a.splits, a.units, zgroups), dim3(ATT_NT), lds, stream, a);
  int st = check_launch("attention split");
  if (st) return st;
  const int quads = (std::min(64, a.rows) + 3) / 4;  // row quads of a row group (the last group may hold fewer)
  const dim3 mgrid(D / 16, quads, a.units * zgroups);
  const size_t mlds = (size_t)a.splits * 2 * 4 * sizeof(float);
  if ((a.splits + 15) / 16 <= 8)
    hipLaunchKernelGGL((k_attn_merge<XT, D, CELLS, 8>), mgrid, dim3(ATT_MERGE_NT), mlds, stream, a);
  else
    hipLaunchKernelGGL((k_attn_merge<XT, D, CELLS, 16>), mgrid, dim3(ATT_MERGE_NT), mlds, stream, a);
  return check_launch("attention merge");
}

// the workspace: max and sum a (split, unit, row), then the outputs (16-byte aligned) in the lanes' layout
static size_t attn_ws_carve(AttnArgs* a_out, float* base, int units, int rows, int tiles, int zgroups, int D) {
  AttnArgs a{};
  a.units = units;
  a.tiles = tiles;
  plan_splits(a, zgroups, att_min_tiles(rows), att_blocks_per_cu(std::min(64, rows), D));
  const size_t ml = ((size_t)a.splits * units * rows + 3) & ~(size_t)3;  // floats, a multiple of 4
  if (a_out) {
    a_out->wm = base;
    a_out->wl = base + ml;
    a_out->wo = base + 2 * ml;
  }
  return (2 * ml + (size_t)a.splits * units * zgroups * 4 * D * 16) * sizeof(float);
}

}  // namespace sh

using namespace sh;

extern "C" {

size_t sh_paged_attn_workspace(int64_t n_q, int64_t hq, int64_t hkv, int64_t head_dim, int64_t ctx_len) {
  if (n_q <= 0 || hkv <= 0 || hq % hkv || ctx_len <= 0) return 0;
  const int rows = (int)(n_q * (hq / hkv));
  return attn_ws_carve(nullptr, nullptr, (int)hkv, rows, (int)((ctx_len + 15) / 16), (rows + 63) / 64,
                       (int)head_dim);
}

}  // extern "C"

namespace {

int paged_attn(const void* q, const void* k_pages, const void* v_pages, const int32_t* page_table, int64_t n_pages,
               int64_t ctx_len, int64_t n_q, int64_t hq, int64_t hkv, int64_t head_dim, float scale, int dtype,
               const void* gate, int64_t gate_ts, int64_t gate_hs, void* out, void* workspace, size_t workspace_bytes,
               void* stream) {
  if (n_q <= 0) return OK;
  if (hkv <= 0 || hq <= 0 || hq % hkv) return fail(E_SHAPE, "paged_attn: %lld query heads over %lld KV heads",
                                                   (long long)hq, (long long)hkv);
  if (head_dim != 256 && head_dim != 128) return fail(E_UNSUPPORTED, "paged_attn: head_dim %lld (128 or 256)",
                                                      (long long)head_dim);
  if (ctx_len <= 0 || n_q > ctx_len) return fail(E_SHAPE, "paged_attn: %lld queries in a context of %lld",
                                                 (long long)n_q, (long long)ctx_len);
  if (n_pages < (ctx_len + 15) / 16) return fail(E_SHAPE, "paged_attn: %lld pages for %lld positions",
                                                 (long long)n_pages, (long long)ctx_len);
  if (n_pages * hkv * 16 * head_dim * 2 > (int64_t)UINT32_MAX)
    return fail(E_UNSUPPORTED, "paged_attn: a K or V pool of more than 4 GiB");
  if (!q || !k_pages || !v_pages || !page_table || !out) return fail(E_ARG, "paged_attn: null pointer");
  if (((uintptr_t)q | (uintptr_t)k_pages | (uintptr_t)v_pages) & 15)
    return fail(E_ARG, "paged_attn: q, k and v must be 16-byte aligned");
  const size_t need = sh_paged_attn_workspace(n_q, hq, hkv, head_dim, ctx_len);
  if (!workspace || workspace_bytes < need)
    return fail(E_WORKSPACE, "paged_attn: workspace of %zu bytes, %zu needed", workspace_bytes, need);
  AttnArgs a{};
  a.q = q;
  a.k = k_pages;
  a.v = v_pages;
  a.table = page_table;
  a.real = nullptr;
  a.kv_len = n_pages;
  a.ws = (float*)workspace;
  a.out = out;
  a.n_q = (int)n_q;
  a.hq = (int)hq;
  a.hkv = (int)hkv;
  a.ctx = (int)ctx_len;
  a.tiles = (int)((ctx_len + 15) / 16);
  a.units = (int)hkv;
  a.rows = (int)(n_q * (hq / hkv));
  a.scale_log2 = scale * 1.4426950408889634f;
  a.gate = gate, a.gate_ts = gate_ts, a.gate_hs = gate_hs;
  attn_ws_carve(&a, (float*)workspace, a.units, a.rows, a.tiles, (a.rows + 63) / 64, (int)head_dim);
  return with_half_dtype(dtype, [&](auto* tp) {
    using XT = std::remove_pointer_t<decltype(tp)>;
    return head_dim == 256 ? launch_attn<XT, 256, false>(a, (hipStream_t)stream)
                           : launch_attn<XT, 128, false>(a, (hipStream_t)stream);
  });
}

}  // namespace

extern "C" {

int sh_paged_attn(const void* q, const void* k_pages, const void* v_pages, const int32_t* page_table, int64_t n_pages,
                  int64_t ctx_len, int64_t n_q, int64_t hq, int64_t hkv, int64_t head_dim, float scale, int dtype,
                  void* out, void* workspace, size_t workspace_bytes, void* stream) {
  return paged_attn(q, k_pages, v_pages, page_table, n_pages, ctx_len, n_q, hq, hkv, head_dim, scale, dtype, nullptr,
                    0, 0, out, workspace, workspace_bytes, stream);
}

int sh_paged_attn_gated(const void* q, const void* k_pages, const void* v_pages, const int32_t* page_table,
                        int64_t n_pages, int64_t ctx_len, int64_t n_q, int64_t hq, int64_t hkv, int64_t head_dim,
                        float scale, int dtype, const void* gate, int64_t gate_token_stride, int64_t gate_head_stride,
                        void* out, void* workspace, size_t workspace_bytes, void* stream) {
  if (n_q > 0 && !gate) return fail(E_ARG, "paged_attn_gated: null gate");
  return paged_attn(q, k_pages, v_pages, page_table, n_pages, ctx_len, n_q, hq, hkv, head_dim, scale, dtype, gate,
                    gate_token_stride, gate_head_stride, out, workspace, workspace_bytes, stream);
}

size_t sh_cells_attn_workspace(int64_t n_q, int64_t hq, int64_t hkv, int64_t head_dim, int64_t cells) {
  if (n_q <= 0 || hkv <= 0 || hq % hkv || cells <= 0) return 0;
  return attn_ws_carve(nullptr, nullptr, (int)(n_q * hkv), (int)(hq / hkv), (int)((cells + 15) / 16), 1,
                       (int)head_dim);
}

}  // extern "C"

namespace {

int cells_attn(const void* q, const void* k, const void* v, int64_t kv_len, const int32_t* cells,
               const uint8_t* real, int64_t n_cells, int64_t n_q, int64_t hq, int64_t hkv, int64_t head_dim,
               float scale, int dtype, const int32_t* page_table, int64_t n_pages, const void* gate, int64_t gate_ts,
               int64_t gate_hs, void* out, void* workspace, size_t workspace_bytes, void* stream) {
  if (n_q <= 0) return OK;
  if (hkv <= 0 || hq <= 0 || hq % hkv) return fail(E_SHAPE, "cells_attn: %lld query heads over %lld KV heads",
                                                   (long long)hq, (long long)hkv);
  if (hq / hkv > 64) return fail(E_UNSUPPORTED, "cells_attn: %lld query heads a KV head (at most 64)",
                                 (long long)(hq / hkv));
  if (head_dim != 256 && head_dim != 128) return fail(E_UNSUPPORTED, "cells_attn: head_dim %lld (128 or 256)",
                                                      (long long)head_dim);
  if (n_cells <= 0 || kv_len <= 0) return fail(E_SHAPE, "cells_attn: %lld cells of %lld", (long long)n_cells,
                                                (long long)kv_len);
  if (hkv * kv_len * head_dim * 2 > (int64_t)UINT32_MAX)
    return fail(E_UNSUPPORTED, "cells_attn: a K or V cache of more than 4 GiB");
  if (!q || !k || !v || !cells || !real || !out) return fail(E_ARG, "cells_attn: null pointer");
  if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v) & 15)
    return fail(E_ARG, "cells_attn: q, k and v must be 16-byte aligned");
  const size_t need = sh_cells_attn_workspace(n_q, hq, hkv, head_dim, n_cells);
  if (!workspace || workspace_bytes < need)
    return fail(E_WORKSPACE, "cells_attn: workspace of %zu bytes, %zu needed", workspace_bytes, need);
  AttnArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.table = cells;
  a.real = real;
  a.ws = (float*)workspace;
  a.out = out;
  a.n_q = (int)n_q;
  a.hq = (int)hq;
  a.hkv = (int)hkv;
  a.ctx = (int)n_cells;
  a.kv_len = kv_len;
  a.tiles = (int)((n_cells + 15) / 16);
  a.units = (int)(n_q * hkv);
  a.rows = (int)(hq / hkv);
  a.scale_log2 = scale * 1.4426950408889634f;
  a.gate = gate, a.gate_ts = gate_ts, a.gate_hs = gate_hs;
  a.cell_pages = page_table, a.cell_npages = n_pages;
  attn_ws_carve(&a, (float*)workspace, a.units, a.rows, a.tiles, 1, (int)head_dim);
  return with_half_dtype(dtype, [&](auto* tp) {
    using XT = std::remove_pointer_t<decltype(tp)>;
    return head_dim == 256 ? launch_attn<XT, 256, true>(a, (hipStream_t)stream)
                           : launch_attn<XT, 128, true>(a, (hipStream_t)stream);
  });
}

}  // namespace

extern "C" {

int sh_cells_attn(const void* q, const void* k, const void* v, int64_t kv_len, const int32_t* cells,
                  const uint8_t* real, int64_t n_cells, int64_t n_q, int64_t hq, int64_t hkv, int64_t head_dim,
                  float scale, int dtype, void* out, void* workspace, size_t workspace_bytes, void* stream) {
  return cells_attn(q, k, v, kv_len, cells, real, n_cells, n_q, hq, hkv, head_dim, scale, dtype, nullptr, 0,
                    nullptr, 0, 0, out, workspace, workspace_bytes, stream);
}

int sh_cells_attn_paged(const void* q, const void* k_pages, const void* v_pages, const int32_t* page_table,
                        int64_t n_pages, const int32_t* cells, const uint8_t* real, int64_t n_cells, int64_t n_q,
                        int64_t hq, int64_t hkv, int64_t head_dim, float scale, int dtype, const void* gate,
                        int64_t gate_token_stride, int64_t gate_head_stride, void* out, void* workspace,
                        size_t workspace_bytes, void* stream) {
  if (n_q > 0 && (!page_table || n_pages <= 0)) return fail(E_ARG, "cells_attn_paged: no page table");
  if (n_pages * hkv * 16 * head_dim * 2 > (int64_t)UINT32_MAX)
    return fail(E_UNSUPPORTED, "cells_attn_paged: a K or V pool of more than 4 GiB");
  return cells_attn(q, k_pages, v_pages, n_pages * 16, cells, real, n_cells, n_q, hq, hkv, head_dim, scale, dtype,
                    page_table, n_pages, gate, gate_token_stride, gate_head_stride, out, workspace, workspace_bytes,
                    stream);
}

}  // extern "C"
