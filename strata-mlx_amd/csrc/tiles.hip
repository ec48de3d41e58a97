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
#include <type_traits>

#include "launch.h"
#include "xmv.h"

namespace sh {

constexpr int TILE_TOKENS = 16, TG = 8, RB = 64, KCH = 256;

// the tables a kind's dequantization reads in LDS, and their size: IQ3_S the 32 KiB signed table, others as
// stage_tables lays them out
template <int KIND> constexpr int tile_tab_bytes() { return KIND == IQ3_S ? IQ3S_SIGNED_BYTES : (KIND == Q2_0 || KIND == Q3_K) ? 0 : LDS_TAB_MAX; }

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
    for (int h = 0; h < 4; ++h)
      p[h] = (uint32_t)__builtin_bit_cast(uint16_t, from_f32<XT>(f[8 * c + 2 * h])) |
             ((uint32_t)__builtin_bit_cast(uint16_t, from_f32<XT>(f[8 * c + 2 * h + 1])) << 16);
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
  const int nch = cols / KCH;

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
      u32x4 w[4];
      dequant_run<KIND, XT>(raw + ur * (int)rbytes, c * (KCH / 32) + urun, tab, w);
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
        for (int ks = 0; ks < KCH / 32; ++ks) af[ks] = *(const u32x4*)(arow + c * KCH + ks * 32 + 8 * g);
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
  if (cols % KCH) return fail(E_UNSUPPORTED, "tile_matmul: %lld columns (a multiple of %d)", (long long)cols, KCH);
  if (pairs % TILE_TOKENS) return fail(E_SHAPE, "tile_matmul: %lld pairs are not whole tiles of 16", (long long)pairs);
  if (a_dtype != BF16 && a_dtype != F16)
    return fail(E_UNSUPPORTED, "tile_matmul: activations of dtype %d (bfloat16 or float16)", a_dtype);
  const bool needs_tables = kind != Q2_0 && kind != Q3_K;
  if (!blocks || !a || !tile_expert || !out || (needs_tables && !tables))
    return fail(E_ARG, "tile_matmul: null pointer");
  if (((uintptr_t)a & 15) || ((uintptr_t)blocks & 15))
    return fail(E_ARG, "tile_matmul: activations and blocks must be 16-byte aligned");
  const int64_t n_tiles = pairs / TILE_TOKENS;
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
