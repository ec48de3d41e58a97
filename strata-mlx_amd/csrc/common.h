// Shared definitions of the strata-hip library: block types, dtypes, codebook table layout, number formats,
// MFMA operand types and the error channel of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sh {

// GGUF block types on the path (strata_mlx/blocks.py:36-38); values are the C ABI's SH_KIND_* codes.
enum Kind : int {
  Q2_0 = 0, IQ4_NL = 1, IQ4_XS = 2, IQ3_S = 3, IQ3_XXS = 4, IQ2_S = 5, IQ2_XS = 6, IQ2_XXS = 7, IQ1_M = 8,
  Q3_K = 9, N_KINDS = 10
};

// Activation / output element types (the C ABI's SH_DTYPE_* codes).
enum DType : int { F32 = 0, F16 = 1, BF16 = 2 };

// weights per block, bytes per block
__host__ __device__ constexpr int wpb(int k) {
  return k == Q2_0 ? 64 : k == IQ4_NL ? 32 : 256;
}
__host__ __device__ constexpr int bpb(int k) {
  return k == Q2_0 ? 18 : k == IQ4_NL ? 18 : k == IQ4_XS ? 136 : k == IQ3_S ? 110 : k == IQ3_XXS ? 98
       : k == IQ2_S ? 82 : k == IQ2_XS ? 74 : k == IQ2_XXS ? 66 : k == IQ1_M ? 56 : 110;
}

__host__ __device__ constexpr int64_t row_bytes_dev(int k, int64_t cols) { return cols / wpb(k) * bpb(k); }

// the LDS stride of rows of rbytes (a multiple of 16): padded by 16-byte chunks so 16 consecutive rows start in
// distinct 4-bank windows of the 64 banks
__host__ __device__ constexpr int padded_stride(int rbytes) {
  for (int pad = 0; pad <= 48; pad += 16) {
    const int dw = (rbytes + pad) / 4;
    bool distinct = true;
    for (int a = 0; a < 16 && distinct; ++a)
      for (int b = a + 1; b < 16 && distinct; ++b) distinct = ((a * dw) % 64) / 4 != ((b * dw) % 64) / 4;
    if (distinct) return rbytes + pad;
  }
  return rbytes + 16;
}

// Codebook blob: every table one kernel may need, at fixed 16-byte aligned offsets. The blob is device memory
// the caller uploads once; kernels that need a table copy it to LDS.
constexpr int TAB_KVALUES = 0;       // int8 [16]        IQ4_NL / IQ4_XS values (strata_mlx/gguf.py:34)
constexpr int TAB_KSIGNS = 16;       // uint8 [128]      7 sign bits -> 8 (IQ3_XXS, IQ2_XS, IQ2_XXS)
constexpr int TAB_IQ3S = 144;        // uint8 [512][4]
constexpr int TAB_IQ3XXS = 2192;     // uint8 [256][4]
constexpr int TAB_IQ2S = 3216;       // uint8 [1024][8]
constexpr int TAB_IQ2XS = 11408;     // uint8 [512][8]
constexpr int TAB_IQ2XXS = 15504;    // uint8 [256][8]
constexpr int TAB_IQ1 = 17552;       // uint8 [2048][8]  grid -1/0/1 stored as 0/1/2
constexpr int TAB_IQ3S_SIGNED = 33936;  // uint8 [8192][4] derived: entry (index | signs << 9), bytes 16 +- value
constexpr int TAB_BYTES = 66704;

// The tables a kind reads, as a kernel holds them in LDS: the small table (kvalues or ksigns) in the first 128
// bytes, the kind's grid from byte 128 on.
__host__ __device__ constexpr int small_offset(int k) {
  return k == IQ4_NL || k == IQ4_XS ? TAB_KVALUES : (k == IQ3_XXS || k == IQ2_XS || k == IQ2_XXS) ? TAB_KSIGNS : -1;
}
__host__ __device__ constexpr int small_bytes(int k) {
  return k == IQ4_NL || k == IQ4_XS ? 16 : (k == IQ3_XXS || k == IQ2_XS || k == IQ2_XXS) ? 128 : 0;
}
__host__ __device__ constexpr int grid_offset(int k) {
  return k == IQ3_S ? TAB_IQ3S : k == IQ3_XXS ? TAB_IQ3XXS : k == IQ2_S ? TAB_IQ2S : k == IQ2_XS ? TAB_IQ2XS
       : k == IQ2_XXS ? TAB_IQ2XXS : k == IQ1_M ? TAB_IQ1 : -1;
}
__host__ __device__ constexpr int grid_bytes(int k) {
  return k == IQ3_S ? 2048 : k == IQ3_XXS ? 1024 : k == IQ2_S ? 8192 : k == IQ2_XS ? 4096 : k == IQ2_XXS ? 2048
       : k == IQ1_M ? 16384 : 0;
}
constexpr int LDS_GRID = 128;                 // where the grid starts in a kernel's LDS table
constexpr int LDS_TAB_MAX = 128 + 16384;      // the largest LDS table (IQ1_M)
__host__ __device__ constexpr int lds_tab_bytes(int k) { return grid_bytes(k) ? LDS_GRID + grid_bytes(k) : 128; }

// ---- number formats

typedef __bf16 bf16;
typedef _Float16 f16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <typename T> __device__ __forceinline__ float to_f32(T v) { return (float)v; }
template <typename T> __device__ __forceinline__ T from_f32(float v) { return (T)v; }  // round to nearest even

// Activation element type <-> DType code
template <typename T> struct dtype_of;
template <> struct dtype_of<float> { static constexpr int value = F32; };
template <> struct dtype_of<f16> { static constexpr int value = F16; };
template <> struct dtype_of<bf16> { static constexpr int value = BF16; };

__host__ __device__ constexpr int dtype_size(int dt) { return dt == F32 ? 4 : 2; }

// ---- error channel of the C ABI (errors.cpp)

enum Status : int {
  OK = 0, E_ARG = -1, E_SHAPE = -2, E_KIND = -3, E_DTYPE = -4, E_HIP = -5, E_WORKSPACE = -6, E_UNSUPPORTED = -7
};
int fail(int status, const char* fmt, ...);
int check_launch(const char* what);

}  // namespace sh
