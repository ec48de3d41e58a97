// The hyper-connection read between two blocks, with the write of the block before folded in (strata_mlx/fused.py:
// 46-131 and 281-323, FusedResidual): for each token of a window, the HC residual streams of D each are
// h_s = before_s + out * inject_in_s (the new residual), normalized a stream at a time; a low-rank gate over all of
// them (down, R rows, and the HC inject rows) and its SiLU; the up projection's sigmoid gates mix the streams into the
// block's input, and 2 sigmoid of the inject rows says how strongly the block's output goes back into each stream.
//
// Four launches, each reading its weights once for the whole window (HBM-bound: down and up are R x HC D each):
//   norm   a block a (stream, token): residual in the activation type, normed in float32 (workspace)
//   down   split over 1024-column slices: a block stages the slice of every token's normed in LDS once and its 8
//          waves take a row each (8 weights a lane a step, 16-byte loads); one float a (token, row, slice)
//   gate   a thread a (token, row): the slices added in order, / HC, then z sigmoid(z) or 2 sigmoid(z)
//   up     4 lanes a row of `up` (a stream's column), the low-rank activations in LDS; the row's sum by two lane
//          exchanges, its gate on normed, then a column's streams added in order and / HC
// Every token's sums are taken in the same order whatever the window, so a token gets the same bits alone or in a
// window.
#include <algorithm>

#include "launch.h"
#include "xmv.h"

namespace sh {

constexpr int HC_MAX_TOKENS = 16;
constexpr int HC_SLICE = 1024;      // columns of a down slice
constexpr int HC_DOWN_WAVES = 8;    // rows a down block
constexpr int HC_UP_LANES = 4;      // lanes a row of up
constexpr int HC_UP_THREADS = 256;

template <typename WT> struct W8 {  // eight consecutive weights as float (16-byte loads)
  __device__ __forceinline__ static void load(const WT* p, float (&w)[8]) {
    if constexpr (sizeof(WT) == 2) {
      const u32x4 v = *(const u32x4*)p;
      const WT* e = (const WT*)&v;
#pragma unroll
      for (int i = 0; i < 8; ++i) w[i] = to_f32(e[i]);
    } else {
      const f32x4 a = *(const f32x4*)p, b = *(const f32x4*)(p + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        w[i] = a[i];
        w[4 + i] = b[i];
      }
    }
  }
};

template <typename XT>
__global__ __launch_bounds__(256) void k_hc_norm(const XT* __restrict__ before, const XT* __restrict__ out,
                                                 const XT* __restrict__ inject_in, const float* __restrict__ norm,
                                                 int hc, int D, float eps, XT* __restrict__ residual,
                                                 float* __restrict__ normed) {
  __shared__ float red[4];
  const int s = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
  const int64_t HD = (int64_t)hc * D;
  const float back = to_f32(inject_in[t * hc + s]);
  const XT* b = before + t * HD + (int64_t)s * D;
  const XT* o = out + (int64_t)t * D;
  float sq = 0.0f;
  for (int i = tid; i < D; i += 256) {
    const float h = to_f32(b[i]) + to_f32(o[i]) * back;
    sq += h * h;
  }
  sq = wave_sum(sq);
  if ((tid & 63) == 0) red[tid >> 6] = sq;
  __syncthreads();
  const float scale = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)D + eps);
  XT* r = residual + t * HD + (int64_t)s * D;
  float* nd = normed + t * HD + (int64_t)s * D;
  const float* w = norm + (int64_t)s * D;
  for (int i = tid; i < D; i += 256) {
    const float h = to_f32(b[i]) + to_f32(o[i]) * back;
    r[i] = from_f32<XT>(h);
    nd[i] = h * scale * w[i];
  }
}

template <typename WT>
__global__ __launch_bounds__(HC_DOWN_WAVES * 64) void k_hc_down(const float* __restrict__ normed,
                                                                const WT* __restrict__ down,
                                                                const WT* __restrict__ inject_w, int R, int NR, int HD,
                                                                int tokens, int nslices, float* __restrict__ part) {
  extern __shared__ float xs[];  // [tokens][HC_SLICE]: the slice of every token's normed
  const int slice = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int k0 = slice * HC_SLICE, klen = min(HC_SLICE, HD - k0);
  for (int i = tid; i < tokens * klen; i += HC_DOWN_WAVES * 64) {
    const int t = i / klen, k = i - t * klen;
    xs[t * HC_SLICE + k] = normed[(int64_t)t * HD + k0 + k];
  }
  __syncthreads();
  const int row = blockIdx.x * HC_DOWN_WAVES + wave;
  if (row >= NR) return;  // wave-uniform, past the block's last barrier
  const WT* w = (row < R ? down + (int64_t)row * HD : inject_w + (int64_t)(row - R) * HD) + k0;
  float acc[HC_MAX_TOKENS];
#pragma unroll
  for (int t = 0; t < HC_MAX_TOKENS; ++t) acc[t] = 0.0f;
  for (int k = lane * 8; k < klen; k += 512) {
    float wv[8];
    W8<WT>::load(w + k, wv);
#pragma unroll
    for (int t = 0; t < HC_MAX_TOKENS; ++t) {
      if (t < tokens) {
        const float* x = xs + t * HC_SLICE + k;
        float a = acc[t];
#pragma unroll
        for (int i = 0; i < 8; ++i) a = fmaf(wv[i], x[i], a);
        acc[t] = a;
      }
    }
  }
#pragma unroll
  for (int t = 0; t < HC_MAX_TOKENS; ++t) {
    if (t < tokens) {
      const float v = wave_sum(acc[t]);
      if (lane == 0) part[((int64_t)t * NR + row) * nslices + slice] = v;
    }
  }
}

template <typename XT>
__global__ __launch_bounds__(256) void k_hc_gate(const float* __restrict__ part, int R, int NR, int nslices,
                                                 int tokens, int hc, float* __restrict__ low,
                                                 XT* __restrict__ inject) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= tokens * NR) return;
  const int t = i / NR, j = i - t * NR;
  const float* p = part + ((int64_t)t * NR + j) * nslices;
  float total = 0.0f;
  for (int s = 0; s < nslices; ++s) total += p[s];
  total /= (float)hc;
  const float gate = 1.0f / (1.0f + expf(-total));
  if (j < R)
    low[t * R + j] = total * gate;
  else
    inject[t * (NR - R) + (j - R)] = from_f32<XT>(2.0f * gate);
}

template <typename XT, typename WT>
__global__ __launch_bounds__(HC_UP_THREADS) void k_hc_up(const float* __restrict__ normed, const WT* __restrict__ up,
                                                         const float* __restrict__ low, int hc, int D, int R,
                                                         int tokens, XT* __restrict__ mixed) {
  extern __shared__ float lds[];  // low [tokens][R], then vals [cols a block * hc][tokens]
  constexpr int ROWS = HC_UP_THREADS / HC_UP_LANES;  // rows of up a block
  const int tid = threadIdx.x, cpb = ROWS / hc;
  float* lows = lds;
  float* vals = lds + tokens * R;
  for (int i = tid; i < tokens * R; i += HC_UP_THREADS) lows[i] = low[i];
  __syncthreads();
  const int rb = tid / HC_UP_LANES, part = tid % HC_UP_LANES;
  const int cc = rb / hc, s = rb - cc * hc;
  const int c = blockIdx.x * cpb + cc;
  const bool live = c < D;
  const int per = R / HC_UP_LANES;
  const WT* w = up + ((int64_t)s * D + (live ? c : 0)) * R + part * per;
  const float* lw = lows + part * per;
  float acc[HC_MAX_TOKENS];
#pragma unroll
  for (int t = 0; t < HC_MAX_TOKENS; ++t) acc[t] = 0.0f;
  for (int r = 0; r < per; r += 8) {
    float wv[8];
    W8<WT>::load(w + r, wv);
#pragma unroll
    for (int t = 0; t < HC_MAX_TOKENS; ++t) {
      if (t < tokens) {
        const float* x = lw + t * R + r;
        float a = acc[t];
#pragma unroll
        for (int i = 0; i < 8; ++i) a = fmaf(wv[i], x[i], a);
        acc[t] = a;
      }
    }
  }
  const int64_t HD = (int64_t)hc * D;
#pragma unroll
  for (int t = 0; t < HC_MAX_TOKENS; ++t) {
    if (t < tokens) {
      float g = acc[t];
      g += __shfl_xor(g, 1);  // the row's four lanes are consecutive in the wave
      g += __shfl_xor(g, 2);
      if (part == 0 && live) vals[rb * tokens + t] = normed[t * HD + (int64_t)s * D + c] / (1.0f + expf(-g));
    }
  }
  __syncthreads();
  for (int i = tid; i < cpb * tokens; i += HC_UP_THREADS) {
    const int c2 = i / tokens, t = i - c2 * tokens, col = blockIdx.x * cpb + c2;
    if (col >= D) continue;
    float m = 0.0f;
    for (int k = 0; k < hc; ++k) m += vals[(c2 * hc + k) * tokens + t];
    mixed[(int64_t)t * D + col] = from_f32<XT>(m / (float)hc);
  }
}

struct HcWs {
  float *normed, *part, *low;
};

static size_t hc_carve(HcWs* ws, uint8_t* base, int64_t T, int64_t hc, int64_t d, int64_t R, int64_t n_inject) {
  const int64_t HD = hc * d, NR = R + n_inject, nslices = (HD + HC_SLICE - 1) / HC_SLICE;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    uint8_t* p = base ? base + off : nullptr;
    off = (off + bytes + 255) & ~(size_t)255;
    return p;
  };
  HcWs w;
  w.normed = (float*)take((size_t)4 * T * HD);
  w.part = (float*)take((size_t)4 * T * NR * nslices);
  w.low = (float*)take((size_t)4 * T * R);
  if (ws) *ws = w;
  return off;
}

static int hc_check(int64_t T, int64_t hc, int64_t d, int64_t R, int64_t n_inject) {
  if (T < 1 || T > HC_MAX_TOKENS)
    return fail(E_SHAPE, "hc_residual: %lld tokens (1 to %d a call)", (long long)T, HC_MAX_TOKENS);
  if (hc < 1 || hc > 8 || (hc & (hc - 1)))
    return fail(E_SHAPE, "hc_residual: %lld streams (1, 2, 4 or 8)", (long long)hc);
  if (d < 64 || d % 64 || hc * d > (1 << 20))
    return fail(E_SHAPE, "hc_residual: streams of %lld (a multiple of 64)", (long long)d);
  if (R < 32 || R > 512 || R % 32) return fail(E_SHAPE, "hc_residual: rank %lld (32 to 512, a multiple of 32)", (long long)R);
  if (n_inject != 0 && n_inject != hc)
    return fail(E_SHAPE, "hc_residual: %lld inject rows for %lld streams (0 or the streams)", (long long)n_inject,
                (long long)hc);
  return OK;
}

template <typename XT, typename WT>
static int hc_launch(const XT* before, const XT* out, const XT* inject_in, const float* norm, const WT* down,
                     const WT* up, const WT* inject_w, int T, int hc, int d, int R, int n_inject, float eps,
                     XT* residual, XT* mixed, XT* inject, const HcWs& ws, hipStream_t stream) {
  const int HD = hc * d, NR = R + n_inject, nslices = (HD + HC_SLICE - 1) / HC_SLICE;
  hipLaunchKernelGGL(k_hc_norm<XT>, dim3(hc, T), dim3(256), 0, stream, before, out, inject_in, norm, hc, d, eps,
                     residual, ws.normed);
  int st = check_launch("hc_residual norm");
  if (st) return st;
  const size_t down_lds = (size_t)4 * T * HC_SLICE;
  if (down_lds + static_lds(k_hc_down<WT>) > LDS_BYTES) return fail(E_UNSUPPORTED, "hc_residual: LDS of down");
  hipLaunchKernelGGL(k_hc_down<WT>, dim3((NR + HC_DOWN_WAVES - 1) / HC_DOWN_WAVES, nslices), dim3(HC_DOWN_WAVES * 64),
                     down_lds, stream, ws.normed, down, n_inject ? inject_w : down, R, NR, HD, T, nslices, ws.part);
  st = check_launch("hc_residual down");
  if (st) return st;
  hipLaunchKernelGGL(k_hc_gate<XT>, dim3((T * NR + 255) / 256), dim3(256), 0, stream, ws.part, R, NR, nslices, T, hc,
                     ws.low, inject);
  st = check_launch("hc_residual gate");
  if (st) return st;
  const int cpb = HC_UP_THREADS / HC_UP_LANES / hc;
  const size_t up_lds = (size_t)4 * T * (R + cpb * hc);
  if (up_lds + static_lds(k_hc_up<XT, WT>) > LDS_BYTES) return fail(E_UNSUPPORTED, "hc_residual: LDS of up");
  hipLaunchKernelGGL((k_hc_up<XT, WT>), dim3((d + cpb - 1) / cpb), dim3(HC_UP_THREADS), up_lds, stream, ws.normed,
                     up, ws.low, hc, d, R, T, mixed);
  return check_launch("hc_residual up");
}

}  // namespace sh

using namespace sh;

extern "C" {

size_t sh_hc_workspace(int64_t tokens, int64_t hc, int64_t d, int64_t rank, int64_t n_inject) {
  if (tokens <= 0 || hc <= 0 || d <= 0 || rank <= 0 || n_inject < 0) return 0;
  return hc_carve(nullptr, nullptr, tokens, hc, d, rank, n_inject);
}

int sh_hc_residual(const void* before, const void* out, const void* inject_in, int dtype, const void* norm,
                   const void* down, const void* up, const void* inject_w, int w_dtype, int64_t tokens, int64_t hc,
                   int64_t d, int64_t rank, int64_t n_inject, float eps, void* residual, void* mixed, void* inject,
                   void* workspace, size_t workspace_bytes, void* stream) {
  int st = hc_check(tokens, hc, d, rank, n_inject);
  if (st) return st;
  if (!before || !out || !inject_in || !norm || !down || !up || !residual || !mixed ||
      (n_inject && (!inject_w || !inject)))
    return fail(E_ARG, "hc_residual: null pointer");
  if (((uintptr_t)down | (uintptr_t)up | (uintptr_t)(n_inject ? inject_w : down)) % 16)
    return fail(E_ARG, "hc_residual: weights must be 16-byte aligned");
  const size_t need = hc_carve(nullptr, nullptr, tokens, hc, d, rank, n_inject);
  if (!workspace || workspace_bytes < need)
    return fail(E_WORKSPACE, "hc_residual: workspace of %zu bytes, %zu needed", workspace_bytes, need);
  HcWs ws;
  hc_carve(&ws, (uint8_t*)workspace, tokens, hc, d, rank, n_inject);
  return with_dtype(dtype, [&](auto* xp) {
    using XT = std::remove_pointer_t<decltype(xp)>;
    return with_dtype(w_dtype, [&](auto* wp) {
      using WT = std::remove_pointer_t<decltype(wp)>;
      return hc_launch<XT, WT>((const XT*)before, (const XT*)out, (const XT*)inject_in, (const float*)norm,
                               (const WT*)down, (const WT*)up, (const WT*)inject_w, (int)tokens, (int)hc, (int)d,
                               (int)rank, (int)n_inject, eps, (XT*)residual, (XT*)mixed, (XT*)inject, ws,
                               (hipStream_t)stream);
    });
  });
}

}  // extern "C"
