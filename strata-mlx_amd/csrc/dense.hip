// Dense Q6_K layers held as three parts (strata_mlx/dense.py:109-167, ScaledLinear): w[r][c] = code[r][c] *
// scale[r][c / 16] * d[r][c / d_step], codes and scales int8, d float16.
//
// The window product reads the three parts (1.07 bytes a weight) once for every token of the window: the window's
// activations are staged in LDS once a block; four lanes share a row, each taking a 16-byte run of codes (one
// scale group) at a time, so a wave covers 16 rows with 64 consecutive bytes of each and reads the activations of
// a group as one broadcast from LDS. Per group the lane sums code * x in float32, then adds scale * d times that
// sum; the four lanes' sums meet by two lane exchanges. HBM-bound for a token or two, VALU-bound at eight.
#include <algorithm>

#include "launch.h"

namespace sh {

constexpr int SC_LANES = 4;                  // lanes a row
constexpr int SC_ROWS = 64 / SC_LANES;       // rows a wave
constexpr int SC_WAVES = 4;                  // waves a block
constexpr int SC_MAX_TOKENS = 8;

__device__ __forceinline__ float half_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

template <typename XT, int T>
__global__ __launch_bounds__(SC_WAVES * 64) void k_scaled_matvec(const int8_t* __restrict__ codes,
                                                                   const int8_t* __restrict__ scales,
                                                                   const uint16_t* __restrict__ d, int rows, int cols,
                                                                   int d_step, const XT* __restrict__ x,
                                                                   XT* __restrict__ out) {
  extern __shared__ float xs[];  // [T][cols] as float
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int i = tid; i < T * cols; i += SC_WAVES * 64) xs[i] = to_f32(x[i]);
  __syncthreads();
  const int part = lane & (SC_LANES - 1), groups = cols / 16, dpr = cols / d_step;
  for (int r0 = (blockIdx.x * SC_WAVES + wave) * SC_ROWS; r0 < rows; r0 += gridDim.x * SC_WAVES * SC_ROWS) {
    const int r = r0 + lane / SC_LANES;
    float acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = 0.0f;
    if (r < rows) {
      const int8_t* crow = codes + (int64_t)r * cols;
      const int8_t* srow = scales + (int64_t)r * groups;
      const uint16_t* drow = d + (int64_t)r * dpr;
      for (int g = part; g < groups; g += SC_LANES) {
        const u32x4 cv = *(const u32x4*)(crow + 16 * g);
        const float s = (float)srow[g] * half_to_f32(drow[16 * g / d_step]);
        float c[16];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t w = cv[i];
#pragma unroll
          for (int b = 0; b < 4; ++b) c[4 * i + b] = (float)(int8_t)(w >> (8 * b));
        }
#pragma unroll
        for (int t = 0; t < T; ++t) {
          const float* xg = xs + t * cols + 16 * g;
          float a = 0.0f;
#pragma unroll
          for (int i = 0; i < 16; ++i) a = fmaf(c[i], xg[i], a);
          acc[t] = fmaf(s, a, acc[t]);
        }
      }
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
      float v = acc[t];
      v += __shfl_xor(v, 1);
      v += __shfl_xor(v, 2);
      if (part == 0 && r < rows) out[(int64_t)t * rows + r] = from_f32<XT>(v);
    }
  }
}

// every weight as a float of OutT: a thread the 16 weights of one scale (dense.py:72-82)
template <typename OT>
__global__ __launch_bounds__(256) void k_scaled_floats(const int8_t* __restrict__ codes,
                                                        const int8_t* __restrict__ scales,
                                                        const uint16_t* __restrict__ d, int rows, int cols,
                                                        int d_step, OT* __restrict__ out) {
  const int64_t gi = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int groups = cols / 16;
  if (gi >= (int64_t)rows * groups) return;
  const int64_t r = gi / groups;
  const int g = (int)(gi - r * groups);
  const float s = half_to_f32(d[r * (cols / d_step) + 16 * g / d_step]) * (float)scales[gi];
  const int8_t* c = codes + r * cols + 16 * g;
  OT* o = out + r * cols + 16 * g;
#pragma unroll
  for (int i = 0; i < 16; ++i) o[i] = from_f32<OT>(s * (float)c[i]);
}

static int check_scaled(int64_t rows, int64_t cols, int64_t d_step, const char* what) {
  if (rows <= 0 || cols <= 0 || cols % 256 || rows % 4)
    return fail(E_SHAPE, "%s: a layer of %lld x %lld (rows by 4, columns by 256)", what, (long long)rows,
                (long long)cols);
  if (d_step <= 0 || d_step % 16 || cols % d_step)
    return fail(E_SHAPE, "%s: a d to %lld weights of %lld", what, (long long)d_step, (long long)cols);
  if (rows > (1ll << 30) || cols > (1ll << 20)) return fail(E_SHAPE, "%s: shape too large", what);
  return OK;
}

}  // namespace sh

using namespace sh;

extern "C" {

int sh_scaled_matvec(const int8_t* codes, const int8_t* scales, const uint16_t* d, int64_t rows, int64_t cols,
                     int64_t d_step, const void* x, int x_dtype, int64_t tokens, void* out, void* stream) {
  int st = check_scaled(rows, cols, d_step, "scaled_matvec");
  if (st) return st;
  if (tokens <= 0) return OK;
  if (tokens > SC_MAX_TOKENS)
    return fail(E_SHAPE, "scaled_matvec: %lld tokens (a window is at most %d)", (long long)tokens, SC_MAX_TOKENS);
  if (!codes || !scales || !d || !x || !out) return fail(E_ARG, "scaled_matvec: null pointer");
  if ((uintptr_t)codes & 15) return fail(E_ARG, "scaled_matvec: codes must be 16-byte aligned");
  const size_t lds = (size_t)tokens * cols * 4;
  if (lds > 128 * 1024) return fail(E_UNSUPPORTED, "scaled_matvec: %lld tokens of %lld inputs", (long long)tokens,
                                    (long long)cols);
  const int64_t per_block = SC_WAVES * SC_ROWS;
  const unsigned grid = (unsigned)std::min<int64_t>((rows + per_block - 1) / per_block, 4 * device_cus());
  return with_dtype(x_dtype, [&](auto* tp) {
    using XT = std::remove_pointer_t<decltype(tp)>;
    auto go = [&](auto tc) {
      constexpr int T = decltype(tc)::value;
      hipLaunchKernelGGL((k_scaled_matvec<XT, T>), dim3(grid), dim3(SC_WAVES * 64), lds, (hipStream_t)stream, codes,
                         scales, d, (int)rows, (int)cols, (int)d_step, (const XT*)x, (XT*)out);
      return check_launch("scaled_matvec");
    };
    switch (tokens) {
      case 1: return go(kind_c<1>{});
      case 2: return go(kind_c<2>{});
      case 3: return go(kind_c<3>{});
      case 4: return go(kind_c<4>{});
      case 5: return go(kind_c<5>{});
      case 6: return go(kind_c<6>{});
      case 7: return go(kind_c<7>{});
      default: return go(kind_c<8>{});
    }
  });
}

int sh_scaled_floats(const int8_t* codes, const int8_t* scales, const uint16_t* d, int64_t rows, int64_t cols,
                     int64_t d_step, void* out, int out_dtype, void* stream) {
  int st = check_scaled(rows, cols, d_step, "scaled_floats");
  if (st) return st;
  if (!codes || !scales || !d || !out) return fail(E_ARG, "scaled_floats: null pointer");
  const int64_t n = rows * (cols / 16);
  if ((n + 255) / 256 > 0x7fffffff) return fail(E_SHAPE, "scaled_floats: %lld weights", (long long)(rows * cols));
  return with_dtype(out_dtype, [&](auto* tp) {
    using OT = std::remove_pointer_t<decltype(tp)>;
    hipLaunchKernelGGL((k_scaled_floats<OT>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       codes, scales, d, (int)rows, (int)cols, (int)d_step, (OT*)out);
    return check_launch("scaled_floats");
  });
}

}  // extern "C"
