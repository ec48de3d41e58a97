// Prompt path: the grouped expert GEMM over pairs laid out in tiles of 16, each tile one expert's
// (strata_mlx/blocks.py:465-536, `tile_matmul`): out[p] = W[expert of p's tile] . a[p], the weights dequantized
// and rounded to a's type, float32 sums, rows of tiles that name no expert left as they were.
//
// A block takes TG consecutive tiles and RB rows of the output. Within its tiles, each run of one expert is done
// together: per chunk of KC columns the block dequantizes the expert's RB x KC weights once into LDS (rounded to
// bf16 / fp16, as the reference rounds them) and stages the run's activation rows beside them; then wave w
// multiplies its tile (16 pairs) against the RB rows on 16x16x32 MFMA, fp32 accumulators in registers. LDS rows
// are XOR-swizzled by 16-byte chunk so the MFMA operand reads fall in distinct banks.
#include <type_traits>

#include "launch.h"
#include "xmv.h"

namespace sh {

constexpr int TILE_TOKENS = 16, TG = 4, RB = 64;

template <int KIND, typename XT, int KC>
__global__ __launch_bounds__(TG * 64) void k_tile_matmul(const uint8_t* __restrict__ blocks,
                                                         const uint8_t* __restrict__ tables, int experts, int rows,
                                                         int cols, int64_t rbytes, const XT* __restrict__ a,
                                                         int n_tiles, const int32_t* __restrict__ tile_expert,
                                                         float* __restrict__ out) {
  constexpr int CH = KC / 8;                            // 16-byte chunks of a staged row
  constexpr int SW = CH < 16 ? CH - 1 : 15;             // swizzle mask
  extern __shared__ u32x4 dyn[];
  uint8_t* tab = (uint8_t*)dyn;
  XT* wl = (XT*)((uint8_t*)dyn + LDS_TAB_MAX);          // [RB][KC]
  XT* al = wl + RB * KC;                                // [TG * 16][KC]
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, n = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int t0 = blockIdx.x * TG, r0 = blockIdx.y * RB;
  const int nt = min(TG, n_tiles - t0);

  stage_tables<KIND>(tab, tables);
  int ex[TG];
#pragma unroll
  for (int i = 0; i < TG; ++i) {
    const int e = i < nt ? tile_expert[t0 + i] : experts;
    ex[i] = (e >= 0 && e < experts) ? e : experts;  // a tile naming no expert is skipped
  }
  __syncthreads();

  for (int ta = 0; ta < nt;) {
    const int e = ex[ta];
    int tb = ta + 1;
    while (tb < nt && ex[tb] == e) ++tb;
    if (e >= experts) {
      ta = tb;
      continue;
    }
    const bool mine = wave >= ta && wave < tb;
    f32x4 acc[RB / 16];
#pragma unroll
    for (int nb = 0; nb < RB / 16; ++nb) acc[nb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const uint8_t* wexp = blocks + ((int64_t)e * rows + r0) * rbytes;
    const int tokens = (tb - ta) * TILE_TOKENS;
    for (int k0 = 0; k0 < cols; k0 += KC) {
      __syncthreads();  // the previous chunk's readers are done
      // the expert's RB x KC weights: one run of 32 a thread at a time, rounded to XT
      for (int u = tid; u < RB * (KC / 32); u += TG * 64) {
        const int r = u / (KC / 32), run = u - r * (KC / 32);
        float w[32];
        unpack32<KIND>(wexp + (int64_t)r * rbytes, (k0 >> 5) + run, w, tab);
        XT* dst = wl + r * KC;
#pragma unroll
        for (int c = 0; c < 4; ++c) {  // chunk 4 run + c of row r
          uint32_t p[4];
#pragma unroll
          for (int h = 0; h < 4; ++h)
            p[h] = (uint32_t)__builtin_bit_cast(uint16_t, from_f32<XT>(w[8 * c + 2 * h])) |
                   ((uint32_t)__builtin_bit_cast(uint16_t, from_f32<XT>(w[8 * c + 2 * h + 1])) << 16);
          *(u32x4*)(dst + 8 * ((4 * run + c) ^ (r & SW))) = u32x4{p[0], p[1], p[2], p[3]};
        }
      }
      // the run's activation rows
      for (int u = tid; u < tokens * CH; u += TG * 64) {
        const int t = u / CH, c = u - t * CH;
        const int lt = ta * TILE_TOKENS + t;  // row within the block's tiles
        const u32x4 v = *(const u32x4*)(a + ((int64_t)t0 * TILE_TOKENS + lt) * cols + k0 + 8 * c);
        *(u32x4*)(al + lt * KC + 8 * (c ^ (lt & SW))) = v;
      }
      __syncthreads();
      if (mine) {
        const int lt = wave * TILE_TOKENS + n;  // the lane's A row: token n of the wave's tile
#pragma unroll
        for (int ks = 0; ks < KC / 32; ++ks) {
          const u32x4 af = *(const u32x4*)(al + lt * KC + 8 * ((4 * ks + g) ^ (lt & SW)));
#pragma unroll
          for (int nb = 0; nb < RB / 16; ++nb) {
            const int r = nb * 16 + n;
            const u32x4 bf = *(const u32x4*)(wl + r * KC + 8 * ((4 * ks + g) ^ (r & SW)));
            acc[nb] = mfma<XT>(af, bf, acc[nb]);
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
  if (cols % 256 == 0) {
    constexpr int KC = 256;
    const size_t lds = LDS_TAB_MAX + (size_t)(RB + TG * TILE_TOKENS) * KC * sizeof(XT);
    hipLaunchKernelGGL((k_tile_matmul<KIND, XT, KC>), grid, dim3(TG * 64), lds, stream, blocks, tables, (int)experts,
                       (int)rows, (int)cols, rb, a, (int)n_tiles, tile_expert, out);
  } else {
    constexpr int KC = 64;
    const size_t lds = LDS_TAB_MAX + (size_t)(RB + TG * TILE_TOKENS) * KC * sizeof(XT);
    hipLaunchKernelGGL((k_tile_matmul<KIND, XT, KC>), grid, dim3(TG * 64), lds, stream, blocks, tables, (int)experts,
                       (int)rows, (int)cols, rb, a, (int)n_tiles, tile_expert, out);
  }
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
  if (pairs % TILE_TOKENS) return fail(E_SHAPE, "tile_matmul: %lld pairs are not whole tiles of 16", (long long)pairs);
  if (a_dtype != BF16 && a_dtype != F16)
    return fail(E_UNSUPPORTED, "tile_matmul: activations of dtype %d (bfloat16 or float16)", a_dtype);
  const bool needs_tables = kind != Q2_0 && kind != Q3_K;
  if (!blocks || !a || !tile_expert || !out || (needs_tables && !tables))
    return fail(E_ARG, "tile_matmul: null pointer");
  if (((uintptr_t)a & 15)) return fail(E_ARG, "tile_matmul: activations must be 16-byte aligned");
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
