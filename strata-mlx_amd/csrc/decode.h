// Exact decoding of GGUF blocks: the n-th run of 32 weights of a row as float32.
//
// One function per block type, following the block layouts strata-mlx's kernels read
// (strata_mlx/blocks.py:57-194, helpers 40-54; second texts strata_mlx/gguf.py:182-276). Every weight is an fp16
// scale times small integer or dyadic factors of at most 23 significant bits in all, so these float32 values are
// exact and equal to the oracle's bit for bit.
//
// `row` is the first byte of a row (global or LDS); `tab` points at the kernel's LDS table (small table in bytes
// 0..127, grid from LDS_GRID).
#pragma once

#include "common.h"

namespace sh {

__device__ __forceinline__ uint32_t rd16(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }
__device__ __forceinline__ uint32_t rd32(const uint8_t* p) { return rd16(p) | (rd16(p + 2) << 16); }
__device__ __forceinline__ float half_bits(uint32_t h) { return (float)__builtin_bit_cast(f16, (uint16_t)h); }
__device__ __forceinline__ float half_at(const uint8_t* p) { return half_bits(rd16(p)); }

// the k-th of a Q3_K block's sixteen 6-bit scales, less 32 (low four bits in bytes 0..7, high two in 8..11)
__device__ __forceinline__ float q3k_scale(const uint8_t* s, int k) {
  int p = k & 3, word = k >> 2;
  uint32_t low = word < 2 ? (s[4 * word + p] & 15u) : (uint32_t)(s[4 * (word - 2) + p] >> 4);
  uint32_t high = ((uint32_t)s[8 + p] >> (2 * word)) & 3u;
  return (float)((int)(low | (high << 4)) - 32);
}

template <int KIND> __device__ __forceinline__ void unpack32(const uint8_t* row, int n, float* w, const uint8_t* tab);

template <> __device__ __forceinline__ void unpack32<Q2_0>(const uint8_t* row, int n, float* w, const uint8_t*) {
  const uint8_t* b = row + (n >> 1) * 18;
  const uint8_t* q = b + 2 + 8 * (n & 1);
  float d = half_at(b);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    uint32_t c = q[i];
#pragma unroll
    for (int j = 0; j < 4; ++j) w[4 * i + j] = d * ((float)((c >> (2 * j)) & 3u) - 1.0f);
  }
}

template <> __device__ __forceinline__ void unpack32<IQ4_NL>(const uint8_t* row, int n, float* w, const uint8_t* tab) {
  const uint8_t* b = row + n * 18;
  const int8_t* kv = (const int8_t*)tab;
  float d = half_at(b);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    uint32_t q = b[2 + i];
    w[i] = d * (float)kv[q & 15];
    w[16 + i] = d * (float)kv[q >> 4];
  }
}

template <> __device__ __forceinline__ void unpack32<IQ4_XS>(const uint8_t* row, int n, float* w, const uint8_t* tab) {
  const uint8_t* b = row + (n >> 3) * 136;
  int ib = n & 7;
  const int8_t* kv = (const int8_t*)tab;
  uint32_t ls = (((uint32_t)b[4 + ib / 2] >> (4 * (ib & 1))) & 15u) | (((rd16(b + 2) >> (2 * ib)) & 3u) << 4);
  float d = half_at(b) * ((float)ls - 32.0f);
  const uint8_t* q = b + 8 + 16 * ib;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    w[i] = d * (float)kv[q[i] & 15];
    w[16 + i] = d * (float)kv[q[i] >> 4];
  }
}

template <> __device__ __forceinline__ void unpack32<IQ3_S>(const uint8_t* row, int n, float* w, const uint8_t* tab) {
  const uint8_t* b = row + (n >> 3) * 110;
  int ib = n & 7;
  float d = half_at(b) * (float)(1 + 2 * (((uint32_t)b[106 + ib / 2] >> (4 * (ib & 1))) & 15u));
  uint32_t high = b[66 + ib];
#pragma unroll
  for (int l = 0; l < 8; ++l) {
    const uint8_t* g = tab + LDS_GRID + 4 * ((uint32_t)b[2 + 8 * ib + l] | (((high >> l) & 1u) << 8));
    uint32_t sign = (uint32_t)b[74 + 4 * ib + l / 2] >> (4 * (l & 1));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v = d * (float)g[j];
      w[4 * l + j] = ((sign >> j) & 1u) ? -v : v;
    }
  }
}

template <> __device__ __forceinline__ void unpack32<IQ3_XXS>(const uint8_t* row, int n, float* w, const uint8_t* tab) {
  const uint8_t* b = row + (n >> 3) * 98;
  int ib = n & 7;
  uint32_t aux = rd32(b + 66 + 4 * ib);
  float d = half_at(b) * (0.5f + (float)(aux >> 28)) * 0.5f;
#pragma unroll
  for (int l = 0; l < 8; ++l) {
    const uint8_t* g = tab + LDS_GRID + 4 * (uint32_t)b[2 + 8 * ib + l];
    uint32_t sign = (uint32_t)tab[(aux >> (7 * (l / 2))) & 127u] >> (4 * (l & 1));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v = d * (float)g[j];
      w[4 * l + j] = ((sign >> j) & 1u) ? -v : v;
    }
  }
}

template <> __device__ __forceinline__ void unpack32<IQ2_S>(const uint8_t* row, int n, float* w, const uint8_t* tab) {
  const uint8_t* b = row + (n >> 3) * 82;
  int ib = n & 7;
  float d = half_at(b) * 0.25f;
  uint32_t high = b[66 + ib], scales = b[74 + ib];
#pragma unroll
  for (int l = 0; l < 4; ++l) {
    const uint8_t* g = tab + LDS_GRID + 8 * ((uint32_t)b[2 + 4 * ib + l] | (((high >> (2 * l)) & 3u) << 8));
    uint32_t sign = b[34 + 4 * ib + l];
    float dl = d * (0.5f + (float)(l < 2 ? (scales & 15u) : (scales >> 4)));
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float v = dl * (float)g[j];
      w[8 * l + j] = ((sign >> j) & 1u) ? -v : v;
    }
  }
}

template <> __device__ __forceinline__ void unpack32<IQ2_XS>(const uint8_t* row, int n, float* w, const uint8_t* tab) {
  const uint8_t* b = row + (n >> 3) * 74;
  int ib = n & 7;
  float d = half_at(b) * 0.25f;
  uint32_t scales = b[66 + ib];
#pragma unroll
  for (int l = 0; l < 4; ++l) {
    uint32_t q = rd16(b + 2 + 2 * (4 * ib + l));
    const uint8_t* g = tab + LDS_GRID + 8 * (q & 511u);
    uint32_t sign = tab[q >> 9];
    float dl = d * (0.5f + (float)(l < 2 ? (scales & 15u) : (scales >> 4)));
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float v = dl * (float)g[j];
      w[8 * l + j] = ((sign >> j) & 1u) ? -v : v;
    }
  }
}

template <> __device__ __forceinline__ void unpack32<IQ2_XXS>(const uint8_t* row, int n, float* w, const uint8_t* tab) {
  const uint8_t* b = row + (n >> 3) * 66;
  const uint8_t* q = b + 2 + 8 * (n & 7);
  uint32_t aux = rd32(q + 4);
  float d = half_at(b) * (0.5f + (float)(aux >> 28)) * 0.25f;
#pragma unroll
  for (int l = 0; l < 4; ++l) {
    const uint8_t* g = tab + LDS_GRID + 8 * (uint32_t)q[l];
    uint32_t sign = tab[(aux >> (7 * l)) & 127u];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float v = d * (float)g[j];
      w[8 * l + j] = ((sign >> j) & 1u) ? -v : v;
    }
  }
}

template <> __device__ __forceinline__ void unpack32<Q3_K>(const uint8_t* row, int n, float* w, const uint8_t*) {
  const uint8_t* b = row + (n >> 3) * 110;
  int r = n & 7;
  const uint8_t* q = b + 32 + 32 * (r >> 2);
  int shift = 2 * (r & 3);
  float d = half_at(b + 108);
  float s0 = d * q3k_scale(b + 96, 2 * r), s1 = d * q3k_scale(b + 96, 2 * r + 1);
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    int v = (int)(((uint32_t)q[i] >> shift) & 3u) - ((((uint32_t)b[i] >> r) & 1u) ? 0 : 4);
    w[i] = (i < 16 ? s0 : s1) * (float)v;
  }
}

template <> __device__ __forceinline__ void unpack32<IQ1_M>(const uint8_t* row, int n, float* w, const uint8_t* tab) {
  const uint8_t* b = row + (n >> 3) * 56;
  int ib = n & 7;
  uint32_t packed = (rd16(b + 48) >> 12) | ((rd16(b + 50) >> 8) & 0x00f0u) | ((rd16(b + 52) >> 4) & 0x0f00u)
                  | (rd16(b + 54) & 0xf000u);
  float d = half_bits(packed);
  uint32_t scales = rd16(b + 48 + 2 * (ib / 2)) >> (6 * (ib & 1));
#pragma unroll
  for (int l = 0; l < 4; ++l) {
    uint32_t high = ((uint32_t)b[32 + 2 * ib + l / 2] >> (4 * (l & 1))) & 15u;
    const uint8_t* g = tab + LDS_GRID + 8 * ((uint32_t)b[4 * ib + l] | ((high & 7u) << 8));
    float dl = d * (float)(2 * ((scales >> (3 * (l / 2))) & 7u) + 1);
    float delta = (high & 8u) ? -1.125f : -0.875f;
#pragma unroll
    for (int j = 0; j < 8; ++j) w[8 * l + j] = dl * ((float)g[j] + delta);
  }
}

// float32 dot of a run's 32 weights with 32 activations, in order (the generic kernels' sum of a run)
template <typename XT> __device__ __forceinline__ float dot32(const float* w, const XT* x) {
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < 32; ++j) s = fmaf(w[j], to_f32(x[j]), s);
  return s;
}

// the sum over the P lanes (a power of two, an aligned group of a wave) that share a row, as a butterfly
__device__ __forceinline__ float lanes_sum(float v, int P) {
  for (int o = P >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// silu(g) * u as the reference rounds it: sigmoid in float32 rounded to the activations' type, then g * sigma
// and * u each rounded to that type (strata_mlx/blocks.py:222-237).
template <typename XT> __device__ __forceinline__ XT swiglu_one(XT g, XT u) {
  const float gf = to_f32(g);
  const float y = 1.0f / (1.0f + expf(fabsf(gf)));
  const XT sig = from_f32<XT>(gf < 0.0f ? y : 1.0f - y);
  const XT a = from_f32<XT>(gf * to_f32(sig));
  return from_f32<XT>(to_f32(a) * to_f32(u));
}

// Copy the tables KIND reads from the blob in global memory to `lds` (small table at 0, grid at LDS_GRID).
// Every thread of the block takes part; a barrier must follow before use.
template <int KIND> __device__ __forceinline__ void stage_tables(uint8_t* lds, const uint8_t* blob) {
  constexpr int so = small_offset(KIND), sb = small_bytes(KIND), go = grid_offset(KIND), gb = grid_bytes(KIND);
  const int t = threadIdx.x + threadIdx.y * blockDim.x, nt = blockDim.x * blockDim.y;
  if constexpr (sb > 0) {
    for (int i = t; i < sb / 4; i += nt) ((uint32_t*)lds)[i] = ((const uint32_t*)(blob + so))[i];
  }
  if constexpr (gb > 0) {
    for (int i = t; i < gb / 16; i += nt) ((u32x4*)(lds + LDS_GRID))[i] = ((const u32x4*)(blob + go))[i];
  }
}

}  // namespace sh
