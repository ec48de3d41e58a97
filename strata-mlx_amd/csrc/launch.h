// Host-side helpers: turning the C ABI's runtime kind / dtype codes into template instantiations, and shape checks.
#pragma once

#include <type_traits>

#include "common.h"

namespace sh {

template <int V> using kind_c = std::integral_constant<int, V>;

// f(kind_c<K>{}) for the runtime kind; E_KIND for an unknown one
template <typename F> int with_kind(int kind, F&& f) {
  switch (kind) {
    case Q2_0: return f(kind_c<Q2_0>{});
    case IQ4_NL: return f(kind_c<IQ4_NL>{});
    case IQ4_XS: return f(kind_c<IQ4_XS>{});
    case IQ3_S: return f(kind_c<IQ3_S>{});
    case IQ3_XXS: return f(kind_c<IQ3_XXS>{});
    case IQ2_S: return f(kind_c<IQ2_S>{});
    case IQ2_XS: return f(kind_c<IQ2_XS>{});
    case IQ2_XXS: return f(kind_c<IQ2_XXS>{});
    case IQ1_M: return f(kind_c<IQ1_M>{});
    case Q3_K: return f(kind_c<Q3_K>{});
  }
  return fail(E_KIND, "unknown block kind %d", kind);
}

// f((T*)nullptr) with T the element type of the runtime dtype
template <typename F> int with_dtype(int dt, F&& f) {
  switch (dt) {
    case F32: return f((float*)nullptr);
    case F16: return f((f16*)nullptr);
    case BF16: return f((bf16*)nullptr);
  }
  return fail(E_DTYPE, "unknown dtype %d", dt);
}

template <typename F> int with_half_dtype(int dt, F&& f) {
  switch (dt) {
    case F16: return f((f16*)nullptr);
    case BF16: return f((bf16*)nullptr);
  }
  return fail(E_DTYPE, "dtype %d: float16 or bfloat16 expected", dt);
}

// checks shared by the block-product entry points: rows of `cols` weights end on a block
inline int check_rows(int kind, int64_t rows, int64_t cols, const char* what) {
  if (kind < 0 || kind >= N_KINDS) return fail(E_KIND, "%s: unknown block kind %d", what, kind);
  if (rows <= 0 || cols <= 0) return fail(E_SHAPE, "%s: empty shape %lld x %lld", what, (long long)rows, (long long)cols);
  if (cols % wpb(kind))
    return fail(E_SHAPE, "%s: rows of %lld weights do not end on a block of %d", what, (long long)cols, wpb(kind));
  if (cols % 32) return fail(E_SHAPE, "%s: rows of %lld weights are not runs of 32", what, (long long)cols);
  if (rows > (1ll << 30) || cols > (1ll << 24)) return fail(E_SHAPE, "%s: shape too large", what);
  return OK;
}

inline int64_t row_bytes(int kind, int64_t cols) { return cols / wpb(kind) * bpb(kind); }

inline bool mfma_kind_host(int kind) { return kind == Q2_0 || kind == IQ3_S; }

inline int needs_tables(int kind) { return grid_bytes(kind) > 0 || small_bytes(kind) > 0; }

// lanes that share a row in the generic kernels: a power of two, at most a wave, at most the row's runs
inline int lanes_per_row(int64_t runs) {
  int p = 1;
  while (p < 64 && 2 * p <= runs) p *= 2;
  return p;
}

// LDS a workgroup may hold on gfx950, and the static LDS a kernel declares: a launch asking for more than the
// sum fits is refused by the queue (an invalid allocation that ends the process), so launches check it first
constexpr size_t LDS_BYTES = 160 * 1024;
template <typename K> inline size_t static_lds(K* kern) {
  hipFuncAttributes attr;
  if (hipFuncGetAttributes(&attr, (const void*)kern) != hipSuccess) return LDS_BYTES;
  return attr.sharedSizeBytes;
}

// compute units of the current device
inline int device_cus() {
  static int cus = 0;
  if (!cus) {
    int dev = 0;
    (void)hipGetDevice(&dev);
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (cus <= 0) cus = 256;
  }
  return cus;
}

// the LDS row stride of rows of rbytes: padded by 16-byte chunks so 16 consecutive rows start in distinct
// 4-bank windows of the 64 banks, where the row is whole chunks and the blocks are 16-byte aligned
inline void row_layout(int64_t rbytes, bool aligned, int& rstride, int& padded) {
  padded = 0;
  rstride = (int)rbytes;
  if (rbytes % 16 || !aligned) return;
  rstride = padded_stride((int)rbytes);
  padded = 1;
}

// the streaming matvec of every kind (stream.hip): out[m][t] = W_m . x[m][t] for n_mats matrices and 1-8 tokens,
// or (idx) out[m] = W[idx[m]] . x[m / share] for n_mats pairs over a stack of n_experts, or (experts) the same with
// pair m's blocks at experts[m]; exact weights and float32 sums; E_UNSUPPORTED where it does not take the arguments
// (dry: checks and plan only)
int stream_matvec(bool dry, int kind, const void* blocks, const void* tables, int64_t n_mats, int64_t rows,
                  int64_t cols, const void* x, int x_dtype, int64_t tokens, void* out, void* stream,
                  const int32_t* idx = nullptr, int64_t n_experts = 0, int64_t share = 1,
                  const void* const* experts = nullptr);
// dequantize (stream.hip) rows of `cols` weights to out_dtype by coalesced 16-byte loads and stores; E_UNSUPPORTED
// where it does not take the tensor
int dequant_stream(int kind, const void* blocks, const void* tables, int64_t rows, int64_t cols, void* out,
                   int out_dtype, void* stream);

}  // namespace sh
