// Expert matvec on MFMA: out[pair, r] = W[idx[pair], r, :] . x[pair / share] for bf16 / fp16 activations, the
// decode path of strata-mlx's BlockSwitchLinear (strata_mlx/blocks.py:196-220, 407-436) rebuilt for CDNA4.
//
// Work: a block of 256 threads takes 16 rows of one expert for the tokens that chose it (pairs sharing an expert
// are grouped in the block itself, so an expert's blocks are read once for every verify token that chose it).
// The 16 rows' bytes are staged to LDS with 16-byte loads; the 4 waves split the columns, each decoding its
// share from LDS straight into MFMA operands:
//
//   D[token][row] += x[token][k] * q[k][row]      v_mfma_f32_16x16x32_{bf16,f16}
//
// with the weights as the B operand, so a lane's accumulators are for the row it decoded (row = lane % 16) and the
// block scale it decoded applies to them directly. Tokens sit at M-rows 4 * (t / TPG) + t % TPG, so only TPG of a
// lane's four accumulators are real and the scale costs TPG fmas a group.
//
// Decode without multiplies: a code is ORed into the mantissa of a constant ("magic") — for bf16 0x4300 | c is
// 128 + c — so a pair of weights is one v_and_or. Codes sitting higher in a byte are masked in place (value
// 128 + U*c) and their activation staged as x / U (exact: a power of two). The constant offsets are removed by a
// correction MFMA against a constant operand, chained as the accumulator input:
//   Q2_0:  q = 128 + U c  (bf16) or 1024 + U c (fp16),  correction -(BASE + U)   ->  sum (c - 1) x
//   IQ3_S: q = 144 + v    (bf16) or 1040 + v  (fp16),   v = +-grid from a 32 KiB LDS table of signed entries,
//          correction -144 / -1040                     ->  sum v x
// Every product is exact in float32; the offsets cost precision only in the float32 accumulation (relative error
// about 1e-6 of a block's sum for bf16), far inside the 1e-2 bf16 tolerance.
#include <type_traits>

#include "decode.h"
#include "launch.h"

namespace sh {

constexpr int XMV_GROUPED_UPTO = 128;  // pairs grouped by expert inside each block; beyond, a block is a pair

template <typename MT> struct Magic;
template <> struct Magic<bf16> {
  static constexpr uint32_t M2 = 0x43004300u;  // two bf16 128.0
  static constexpr uint32_t HI = 0x43u;        // high byte of a bf16 128 + b
  static constexpr float BASE = 128.0f;
};
template <> struct Magic<f16> {
  static constexpr uint32_t M2 = 0x64006400u;  // two fp16 1024.0
  static constexpr uint32_t HI = 0x64u;
  static constexpr float BASE = 1024.0f;
};

template <typename MT> __device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (std::is_same_v<MT, bf16>)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
}

template <typename MT> __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  uint16_t a = __builtin_bit_cast(uint16_t, (MT)lo), b = __builtin_bit_cast(uint16_t, (MT)hi);
  return (uint32_t)a | ((uint32_t)b << 16);
}

// ---- Q2_0 (64 weights, 18 bytes: fp16 d, then 16 code bytes, byte i holding weights 4i..4i+3)
//
// Lane group g = lane / 16 of the wave decodes code bytes 2g, 2g+1, 8+2g, 9+2g of each block for its row: the
// dword W = b[2+2g] | b[3+2g] << 8 | b[10+2g] << 16 | b[11+2g] << 24. Block-local weight
// k = 32h + 8g + 4a + j (h: low/high half of W, a: MFMA a or b, j: code within the byte) goes to slot 2j + h of
// MFMA a. U_j is the scale of the in-place mask of code j.
template <typename MT> __device__ __forceinline__ float q2_unit(int j) {
  if constexpr (std::is_same_v<MT, bf16>) return j == 1 ? 4.0f : j == 2 ? 16.0f : 1.0f;  // bits 6-7 shifted down
  else return j == 1 ? 4.0f : j == 2 ? 16.0f : j == 3 ? 64.0f : 1.0f;
}

template <typename MT> __device__ __forceinline__ void q2_decode(uint32_t W, u32x4& fa, u32x4& fb) {
  constexpr uint32_t M = Magic<MT>::M2;
  const uint32_t W8 = W >> 8;
  fa.x = (W & 0x00030003u) | M;
  fa.y = (W & 0x000C000Cu) | M;
  fa.z = (W & 0x00300030u) | M;
  fb.x = (W8 & 0x00030003u) | M;
  fb.y = (W8 & 0x000C000Cu) | M;
  fb.z = (W8 & 0x00300030u) | M;
  if constexpr (std::is_same_v<MT, bf16>) {  // bit 7 of a bf16 half is exponent: code 3 shifted to bits 0-1
    fa.w = ((W >> 6) & 0x00030003u) | M;
    fb.w = ((W >> 14) & 0x00030003u) | M;
  } else {
    fa.w = (W & 0x00C000C0u) | M;
    fb.w = (W8 & 0x00C000C0u) | M;
  }
}

// the correction operand: slot 2j + h holds -(BASE + U_j)
template <typename MT> __device__ __forceinline__ u32x4 q2_correction() {
  u32x4 c;
  c.x = pack2<MT>(-(Magic<MT>::BASE + q2_unit<MT>(0)), -(Magic<MT>::BASE + q2_unit<MT>(0)));
  c.y = pack2<MT>(-(Magic<MT>::BASE + q2_unit<MT>(1)), -(Magic<MT>::BASE + q2_unit<MT>(1)));
  c.z = pack2<MT>(-(Magic<MT>::BASE + q2_unit<MT>(2)), -(Magic<MT>::BASE + q2_unit<MT>(2)));
  c.w = pack2<MT>(-(Magic<MT>::BASE + q2_unit<MT>(3)), -(Magic<MT>::BASE + q2_unit<MT>(3)));
  return c;
}

// where activation k of a Q2_0 block goes in the staged layout: fragment (a, g), slot 2j + h; and its scale 1/U
__device__ __forceinline__ int q2_stage_pos(int kk, int& j) {
  int h = kk >> 5, g = (kk >> 3) & 3, a = (kk >> 2) & 1;
  j = kk & 3;
  return ((a * 4 + g) * 8) + 2 * j + h;  // in elements within the block's 64
}

// ---- IQ3_S signed table: entry (grid index | sign nibble << 9) -> four bytes 16 +- grid value
constexpr int IQ3S_SIGNED_BYTES = 8192 * 4;

// ---- the kernel

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
  __shared__ float s_red[4][64][TPG];
  extern __shared__ u32x4 dyn[];
  // dynamic LDS: [table][staged x: NT tokens x cols][weights: 16 rows + 16 bytes]
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

  // 2. the 16 rows' bytes to LDS, at the same address modulo 16 as in memory
  const uint8_t* src = blocks + (int64_t)grp.expert * expert_bytes + (int64_t)row0 * rbytes;
  const int64_t nbytes = (int64_t)rows_here * rbytes;
  const uintptr_t a0 = (uintptr_t)src & ~(uintptr_t)15;
  const int lead = (int)((uintptr_t)src - a0);
  const int chunks = (int)((lead + nbytes + 15) >> 4);
  for (int c = tid; c < chunks; c += 256) {
    const uint8_t* p = (const uint8_t*)(a0 + 16 * (uintptr_t)c);
    if (p >= src && p + 16 <= src + nbytes) {
      ((u32x4*)wt)[c] = *(const u32x4*)p;
    } else {
      for (int b = 0; b < 16; ++b)
        if (p + b >= src && p + b < src + nbytes) wt[16 * c + b] = p[b];
    }
  }
  const uint8_t* wrow0 = wt + lead;

  // 3. the table (IQ3_S) and the tokens' activations in the layout the decode wants
  if constexpr (KIND == IQ3_S) {
    for (int i = tid; i < IQ3S_SIGNED_BYTES / 16; i += 256) ((u32x4*)tab)[i] = ((const u32x4*)signed_tab)[i];
  }
  for (int i = tid; i < n_tok * cols; i += 256) {
    int t = i / cols, k = i - t * cols;
    float v = to_f32(x[(int64_t)grp.xrow[t] * cols + k]);
    if constexpr (KIND == Q2_0) {
      int j, blk = k >> 6;
      int pos = q2_stage_pos(k & 63, j);
      xs[(size_t)t * cols + blk * 64 + pos] = (MT)(v / q2_unit<MT>(j));
    } else {
      xs[(size_t)t * cols + k] = (MT)v;
    }
  }
  __syncthreads();

  // 4. this wave's quarter of the columns
  const int g = lane >> 4, n = lane & 15;
  const int m = n;  // A operand row this lane supplies
  const int mt = (m & 3) < TPG ? (m >> 2) * TPG + (m & 3) : NT;  // token of A row m, NT if padding
  const bool real = mt < n_tok;
  const uint8_t* wrow = wrow0 + (size_t)n * rbytes;  // this lane's weight row (rows beyond rows_here: stale LDS)
  float acc[TPG];
#pragma unroll
  for (int i = 0; i < TPG; ++i) acc[i] = 0.0f;
  const f32x4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
  const u32x4 zfrag = {0u, 0u, 0u, 0u};

  if constexpr (KIND == Q2_0) {
    const int nblk = cols >> 6, per_wave = nblk >> 2;
    const u32x4 corr = q2_correction<MT>();
    const MT* xt = xs + (size_t)(real ? mt : 0) * cols;
    for (int bi = 0; bi < per_wave; ++bi) {
      const int blk = wave * per_wave + bi;
      const uint8_t* b = wrow + blk * 18;
      const uint32_t W = (uint32_t)*(const uint16_t*)(b + 2 + 2 * g) | ((uint32_t)*(const uint16_t*)(b + 10 + 2 * g) << 16);
      const float d = half_bits(*(const uint16_t*)b);
      u32x4 fa, fb;
      q2_decode<MT>(W, fa, fb);
      u32x4 xa = real ? *(const u32x4*)(xt + blk * 64 + g * 8) : zfrag;
      u32x4 xb = real ? *(const u32x4*)(xt + blk * 64 + 32 + g * 8) : zfrag;
      f32x4 D = mfma<MT>(xa, corr, zero4);
      D = mfma<MT>(xb, corr, D);
      D = mfma<MT>(xa, fa, D);
      D = mfma<MT>(xb, fb, D);
#pragma unroll
      for (int i = 0; i < TPG; ++i) acc[i] = fmaf(d, D[i], acc[i]);
    }
  } else if constexpr (KIND == IQ3_S) {
    const int runs = cols >> 5, per_wave = runs >> 2;
    const float cval = -(Magic<MT>::BASE + 16.0f);
    const uint32_t c2 = pack2<MT>(cval, cval);
    const u32x4 corr = {c2, c2, c2, c2};
    const MT* xt = xs + (size_t)(real ? mt : 0) * cols;
    const uint32_t* stab = (const uint32_t*)tab;
    constexpr uint32_t HI = Magic<MT>::HI;
    const uint32_t hi4 = HI * 0x01010101u;
    for (int ri = 0; ri < per_wave; ++ri) {
      const int run = wave * per_wave + ri;
      const uint8_t* b = wrow + (run >> 3) * 110;
      const int ib = run & 7;
      const float db = half_bits(*(const uint16_t*)b) * (float)(1 + 2 * (((uint32_t)b[106 + ib / 2] >> (4 * (ib & 1))) & 15u));
      const uint32_t q2 = *(const uint16_t*)(b + 2 + 8 * ib + 2 * g);
      const uint32_t qh = (uint32_t)b[66 + ib] >> (2 * g);
      const uint32_t sg = b[74 + 4 * ib + g];
      const uint32_t i0 = (q2 & 0xffu) | ((qh & 1u) << 8) | ((sg & 15u) << 9);
      const uint32_t i1 = (q2 >> 8) | ((qh & 2u) << 7) | ((sg >> 4) << 9);
      const uint32_t e0 = stab[i0], e1 = stab[i1];
      u32x4 fw;
      fw.x = __builtin_amdgcn_perm(hi4, e0, 0x04010400u);
      fw.y = __builtin_amdgcn_perm(hi4, e0, 0x04030402u);
      fw.z = __builtin_amdgcn_perm(hi4, e1, 0x04010400u);
      fw.w = __builtin_amdgcn_perm(hi4, e1, 0x04030402u);
      u32x4 xa = real ? *(const u32x4*)(xt + run * 32 + g * 8) : zfrag;
      f32x4 D = mfma<MT>(xa, corr, zero4);
      D = mfma<MT>(xa, fw, D);
#pragma unroll
      for (int i = 0; i < TPG; ++i) acc[i] = fmaf(db, D[i], acc[i]);
    }
  }

  // 5. the waves' column quarters summed, one lane a (row, token)
#pragma unroll
  for (int i = 0; i < TPG; ++i) s_red[wave][lane][i] = acc[i];
  __syncthreads();
  if (wave == 0) {
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
