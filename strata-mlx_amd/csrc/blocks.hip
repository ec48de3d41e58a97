// Block products for every GGUF type, exact float32 weights: dequantize, the gather matvec of a stack of experts,
// the same with a buffer per pair, a window of tokens through one layer, and down taking silu(gate) * up itself.
//
// These kernels decode each run of 32 weights to exact float32 (decode.h) and take float32 sums: they serve every
// type and every activation type, and float32 activations. The bf16/fp16 decode path of Q2_0 and IQ3_S goes
// through the MFMA kernels of expert.hip instead.
//
// Launch shape: 256 threads; P lanes (a power of two up to 64) share a row and split its runs, sums meet by
// __shfl_xor within the P lanes.
#include "decode.h"
#include "launch.h"

namespace sh {

template <int KIND, typename OT>
__global__ __launch_bounds__(256) void k_dequant(const uint8_t* __restrict__ blocks, const uint8_t* __restrict__ tabs,
                                                 OT* __restrict__ out, int64_t total_runs, int runs, int64_t rbytes) {
  __shared__ u32x4 tab4[lds_tab_bytes(KIND) / 16];
  uint8_t* tab = (uint8_t*)tab4;
  stage_tables<KIND>(tab, tabs);
  __syncthreads();
  int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (g >= total_runs) return;
  int64_t r = g / runs;
  int n = (int)(g % runs);
  float w[32];
  unpack32<KIND>(blocks + r * rbytes, n, w, tab);
  OT* o = out + r * (int64_t)runs * 32 + 32 * n;
#pragma unroll
  for (int j = 0; j < 32; ++j) o[j] = from_f32<OT>(w[j]);
}

// out[pair, r] = W[expert of pair] . x[pair / share]; the expert's blocks are `experts[pair]` when given, else
// blocks + idx[pair] * expert_bytes. A pair naming no expert (idx outside [0, n_experts)) gets zeros.
template <int KIND, typename XT>
__global__ __launch_bounds__(256) void k_switch_matvec(const uint8_t* __restrict__ blocks,
                                                       const uint8_t* const* __restrict__ experts,
                                                       const int32_t* __restrict__ idx, int n_experts,
                                                       int64_t expert_bytes, const XT* __restrict__ x, int share,
                                                       XT* __restrict__ out, int rows, int cols, int64_t rbytes, int P,
                                                       const uint8_t* __restrict__ tabs) {
  __shared__ u32x4 tab4[lds_tab_bytes(KIND) / 16];
  uint8_t* tab = (uint8_t*)tab4;
  stage_tables<KIND>(tab, tabs);
  __syncthreads();
  const int pair = blockIdx.y;
  const int part = threadIdx.x & (P - 1);
  const int r = blockIdx.x * (256 / P) + threadIdx.x / P;
  if (r >= rows) return;
  const uint8_t* base;
  if (experts) {
    base = experts[pair];
  } else {
    int e = idx[pair];
    if (e < 0 || e >= n_experts) {
      if (part == 0) out[(int64_t)pair * rows + r] = from_f32<XT>(0.0f);
      return;
    }
    base = blocks + (int64_t)e * expert_bytes;
  }
  const uint8_t* row = base + (int64_t)r * rbytes;
  const XT* xr = x + (int64_t)(pair / share) * cols;
  float w[32], sum = 0.0f;
  for (int n = part; n < cols / 32; n += P) {
    unpack32<KIND>(row, n, w, tab);
    sum += dot32(w, xr + 32 * n);
  }
  sum = lanes_sum(sum, P);
  if (part == 0) out[(int64_t)pair * rows + r] = from_f32<XT>(sum);
}

// out[t, r] = W . x[t] for one layer and a window of T <= 8 tokens; each run unpacked once for all of them, and a
// token's sum taken in the same order whatever the window (strata_mlx/blocks.py:351-394).
template <int KIND, typename XT>
__global__ __launch_bounds__(256) void k_window_matvec(const uint8_t* __restrict__ blocks, const XT* __restrict__ x,
                                                       int T, XT* __restrict__ out, int rows, int cols, int64_t rbytes,
                                                       int P, const uint8_t* __restrict__ tabs) {
  __shared__ u32x4 tab4[lds_tab_bytes(KIND) / 16];
  uint8_t* tab = (uint8_t*)tab4;
  stage_tables<KIND>(tab, tabs);
  __syncthreads();
  const int part = threadIdx.x & (P - 1);
  const int r = blockIdx.x * (256 / P) + threadIdx.x / P;
  if (r >= rows) return;
  const uint8_t* row = blocks + (int64_t)r * rbytes;
  float w[32], sum[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) sum[t] = 0.0f;
  for (int n = part; n < cols / 32; n += P) {
    unpack32<KIND>(row, n, w, tab);
#pragma unroll
    for (int t = 0; t < 8; ++t)
      if (t < T) sum[t] += dot32(w, x + (int64_t)t * cols + 32 * n);
  }
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    if (t < T) {
      float total = lanes_sum(sum[t], P);
      if (part == 0) out[(int64_t)t * rows + r] = from_f32<XT>(total);
    }
  }
}


// out[pair, r] = W[idx[pair]] . swiglu(gate[pair], up[pair]); the inner activations live in LDS
template <int KIND, typename XT>
__global__ __launch_bounds__(256) void k_matvec_glu(const uint8_t* __restrict__ blocks, const int32_t* __restrict__ idx,
                                                    int n_experts, int64_t expert_bytes, const XT* __restrict__ gate,
                                                    const XT* __restrict__ up, XT* __restrict__ out, int rows, int cols,
                                                    int64_t rbytes, int P, const uint8_t* __restrict__ tabs) {
  __shared__ u32x4 tab4[lds_tab_bytes(KIND) / 16];
  extern __shared__ u32x4 dyn[];
  uint8_t* tab = (uint8_t*)tab4;
  XT* xs = (XT*)dyn;
  stage_tables<KIND>(tab, tabs);
  const int pair = blockIdx.y;
  for (int c = threadIdx.x; c < cols; c += 256)
    xs[c] = swiglu_one(gate[(int64_t)pair * cols + c], up[(int64_t)pair * cols + c]);
  __syncthreads();
  const int part = threadIdx.x & (P - 1);
  const int r = blockIdx.x * (256 / P) + threadIdx.x / P;
  if (r >= rows) return;
  int e = idx[pair];
  if (e < 0 || e >= n_experts) {
    if (part == 0) out[(int64_t)pair * rows + r] = from_f32<XT>(0.0f);
    return;
  }
  const uint8_t* row = blocks + (int64_t)e * expert_bytes + (int64_t)r * rbytes;
  float w[32], sum = 0.0f;
  for (int n = part; n < cols / 32; n += P) {
    unpack32<KIND>(row, n, w, tab);
    sum += dot32(w, xs + 32 * n);
  }
  sum = lanes_sum(sum, P);
  if (part == 0) out[(int64_t)pair * rows + r] = from_f32<XT>(sum);
}

// ---- Q2_0 table of sums (strata_mlx/blocks.py:579-771): for every two inputs (a, b), the 16 sums
// (c0 - 1) a + (c1 - 1) b two codes make of them, in the activations' type; a row is then two lookups a code byte.

template <typename XT>
__global__ __launch_bounds__(256) void k_lookup_table(const XT* __restrict__ x, XT* __restrict__ table, int cols) {
  int g = blockIdx.x * 256 + threadIdx.x;
  int n = blockIdx.y;
  if (g >= cols / 2) return;
  float a = to_f32(x[(int64_t)n * cols + 2 * g]), b = to_f32(x[(int64_t)n * cols + 2 * g + 1]);
  XT* t = table + ((int64_t)n * (cols / 2) + g) * 16;
#pragma unroll
  for (int c = 0; c < 16; ++c) t[c] = from_f32<XT>(((float)(c & 3) - 1.0f) * a + ((float)(c >> 2) - 1.0f) * b);
}

__device__ __forceinline__ float silu_f32(float g) { return g / (1.0f + expf(-g)); }

template <typename XT>
__global__ __launch_bounds__(256) void k_lookup_table_glu(const XT* __restrict__ gate, const XT* __restrict__ up,
                                                          XT* __restrict__ table, int cols) {
  int g = blockIdx.x * 256 + threadIdx.x;
  int n = blockIdx.y;
  if (g >= cols / 2) return;
  int64_t at = (int64_t)n * cols + 2 * g;
  float a = silu_f32(to_f32(gate[at])) * to_f32(up[at]);
  float b = silu_f32(to_f32(gate[at + 1])) * to_f32(up[at + 1]);
  XT* t = table + ((int64_t)n * (cols / 2) + g) * 16;
#pragma unroll
  for (int c = 0; c < 16; ++c) t[c] = from_f32<XT>(((float)(c & 3) - 1.0f) * a + ((float)(c >> 2) - 1.0f) * b);
}

// one row's sum over runs n = part, part + P, ... by two lookups a code byte, the block's scale applied per run
template <typename TT>
__device__ __forceinline__ float lookup_row(const uint8_t* row, const TT* t_, int cols, int part, int P) {
  float sum = 0.0f;
  for (int n = part; n < cols / 32; n += P) {
    const uint8_t* b = row + (n >> 1) * 18;
    const uint8_t* q = b + 2 + 8 * (n & 1);
    const TT* t = t_ + 256 * n;
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      uint32_t c = q[i];
      s += to_f32(t[32 * i + (c & 15)]) + to_f32(t[32 * i + 16 + (c >> 4)]);
    }
    sum += half_at(b) * s;
  }
  return lanes_sum(sum, P);
}

template <typename XT>
__global__ __launch_bounds__(256) void k_lookup_matvec(const uint8_t* __restrict__ blocks, const int32_t* __restrict__ idx,
                                                       int n_experts, int64_t expert_bytes, const XT* __restrict__ table,
                                                       int share, XT* __restrict__ out, int rows, int cols, int P) {
  const int pair = blockIdx.y;
  const int part = threadIdx.x & (P - 1);
  const int r = blockIdx.x * (256 / P) + threadIdx.x / P;
  if (r >= rows) return;
  int e = idx[pair];
  if (e < 0 || e >= n_experts) {
    if (part == 0) out[(int64_t)pair * rows + r] = from_f32<XT>(0.0f);
    return;
  }
  const uint8_t* row = blocks + (int64_t)e * expert_bytes + (int64_t)r * (cols / 64 * 18);
  float total = lookup_row(row, table + (int64_t)(pair / share) * (cols / 2) * 16, cols, part, P);
  if (part == 0) out[(int64_t)pair * rows + r] = from_f32<XT>(total);
}

// down with the table of silu(gate) * up built in LDS by each block (a block is one pair's rows): the same table
// and the same bits as k_lookup_table_glu then k_lookup_matvec with one row to each pair.
template <typename XT>
__global__ __launch_bounds__(256) void k_lookup_down_glu(const uint8_t* __restrict__ blocks, const int32_t* __restrict__ idx,
                                                         int n_experts, int64_t expert_bytes, const XT* __restrict__ gate,
                                                         const XT* __restrict__ up, XT* __restrict__ out, int rows,
                                                         int cols, int P) {
  extern __shared__ u32x4 dyn[];
  XT* tab = (XT*)dyn;
  const int pair = blockIdx.y;
  for (int g = threadIdx.x; g < cols / 2; g += 256) {
    int64_t at = (int64_t)pair * cols + 2 * g;
    float a = silu_f32(to_f32(gate[at])) * to_f32(up[at]);
    float b = silu_f32(to_f32(gate[at + 1])) * to_f32(up[at + 1]);
#pragma unroll
    for (int c = 0; c < 16; ++c)
      tab[g * 16 + c] = from_f32<XT>(((float)(c & 3) - 1.0f) * a + ((float)(c >> 2) - 1.0f) * b);
  }
  __syncthreads();
  const int part = threadIdx.x & (P - 1);
  const int r = blockIdx.x * (256 / P) + threadIdx.x / P;
  if (r >= rows) return;
  int e = idx[pair];
  if (e < 0 || e >= n_experts) {
    if (part == 0) out[(int64_t)pair * rows + r] = from_f32<XT>(0.0f);
    return;
  }
  const uint8_t* row = blocks + (int64_t)e * expert_bytes + (int64_t)r * (cols / 64 * 18);
  float total = lookup_row(row, tab, cols, part, P);
  if (part == 0) out[(int64_t)pair * rows + r] = from_f32<XT>(total);
}

// the lanes a row gets in the table-of-sums kernels: as many as leave each at least four runs, at most 16,
// fewer when there are many pairs (strata_mlx/blocks.py:682-686 keeps the same idea)
static int lookup_lanes(int64_t cols, int64_t pairs) {
  int64_t runs = cols / 32;
  int p = 1;
  while (p < 16 && runs % (2 * p) == 0 && runs / (2 * p) >= 4) p *= 2;
  if (pairs > 20 && p > 4) p = 4;
  return p;
}

}  // namespace sh

using namespace sh;

extern "C" {

int sh_dequantize(int kind, const void* blocks, const void* tables, int64_t n_mats, int64_t rows, int64_t cols,
                  void* out, int out_dtype, void* stream) {
  int st = check_rows(kind, rows, cols, "dequantize");
  if (st) return st;
  if (n_mats <= 0) return fail(E_SHAPE, "dequantize: %lld matrices", (long long)n_mats);
  if (!blocks || !out || (needs_tables(kind) && !tables)) return fail(E_ARG, "dequantize: null pointer");
  if (out_dtype != F32 && out_dtype != F16 && out_dtype != BF16) return fail(E_DTYPE, "unknown dtype %d", out_dtype);
  // coalesced loads and stores where the stream takes the tensor, else a run a thread
  st = dequant_stream(kind, blocks, tables, n_mats * rows, cols, out, out_dtype, stream);
  if (st != E_UNSUPPORTED) return st;
  int64_t total = n_mats * rows * (cols / 32);
  return with_kind(kind, [&](auto kc) {
    constexpr int K = decltype(kc)::value;
    return with_dtype(out_dtype, [&](auto* tp) {
      using OT = std::remove_pointer_t<decltype(tp)>;
      hipLaunchKernelGGL((k_dequant<K, OT>), dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                         (const uint8_t*)blocks, (const uint8_t*)tables, (OT*)out, total, (int)(cols / 32),
                         row_bytes(K, cols));
      return check_launch("dequantize");
    });
  });
}

int sh_switch_matvec_generic(int kind, const void* blocks, const void* const* expert_ptrs, const void* tables,
                             int64_t n_experts, int64_t rows, int64_t cols, const int32_t* idx, int64_t pairs,
                             const void* x, int x_dtype, int64_t share, void* out, void* stream) {
  int st = check_rows(kind, rows, cols, "switch_matvec");
  if (st) return st;
  if (pairs <= 0) return OK;
  if (pairs > 65535) return fail(E_SHAPE, "switch_matvec: %lld pairs (at most 65535 a call)", (long long)pairs);
  if (share <= 0) return fail(E_ARG, "switch_matvec: share %lld", (long long)share);
  if ((!blocks && !expert_ptrs) || (!expert_ptrs && !idx) || !x || !out || (needs_tables(kind) && !tables))
    return fail(E_ARG, "switch_matvec: null pointer");
  // the exact-weight stream over the pairs where it takes them, else a block a few rows a pair
  st = stream_matvec(false, kind, blocks, tables, pairs, rows, cols, x, x_dtype, 1, out, stream,
                     expert_ptrs ? nullptr : idx, n_experts, share, expert_ptrs);
  if (st != E_UNSUPPORTED) return st;
  int P = lanes_per_row(cols / 32);
  return with_kind(kind, [&](auto kc) {
    constexpr int K = decltype(kc)::value;
    return with_dtype(x_dtype, [&](auto* tp) {
      using XT = std::remove_pointer_t<decltype(tp)>;
      dim3 grid((unsigned)((rows + 256 / P - 1) / (256 / P)), (unsigned)pairs);
      hipLaunchKernelGGL((k_switch_matvec<K, XT>), grid, dim3(256), 0, (hipStream_t)stream, (const uint8_t*)blocks,
                         (const uint8_t* const*)expert_ptrs, idx, (int)n_experts, rows * row_bytes(K, cols),
                         (const XT*)x, (int)share, (XT*)out, (int)rows, (int)cols, row_bytes(K, cols), P,
                         (const uint8_t*)tables);
      return check_launch("switch_matvec");
    });
  });
}

int sh_matvec_separate(int kind, const void* const* expert_ptrs, const void* tables, int64_t rows, int64_t cols,
                       int64_t pairs, const void* x, int x_dtype, int64_t share, void* out, void* stream) {
  if (!expert_ptrs) return fail(E_ARG, "matvec_separate: null expert pointer list");
  return sh_switch_matvec_generic(kind, nullptr, expert_ptrs, tables, pairs, rows, cols, nullptr, pairs, x, x_dtype,
                                  share, out, stream);
}

int sh_window_matvec(int kind, const void* blocks, const void* tables, int64_t rows, int64_t cols, const void* x,
                     int x_dtype, int64_t tokens, void* out, void* stream) {
  int st = check_rows(kind, rows, cols, "window_matvec");
  if (st) return st;
  if (tokens <= 0) return OK;
  if (tokens > 8) return fail(E_SHAPE, "window_matvec: %lld tokens (a window is at most 8)", (long long)tokens);
  if (!blocks || !x || !out || (needs_tables(kind) && !tables)) return fail(E_ARG, "window_matvec: null pointer");
  // the exact-weight stream where it takes the layer, else a block a few rows
  st = stream_matvec(false, kind, blocks, tables, 1, rows, cols, x, x_dtype, tokens, out, stream);
  if (st != E_UNSUPPORTED) return st;
  int P = lanes_per_row(cols / 32);
  return with_kind(kind, [&](auto kc) {
    constexpr int K = decltype(kc)::value;
    return with_dtype(x_dtype, [&](auto* tp) {
      using XT = std::remove_pointer_t<decltype(tp)>;
      dim3 grid((unsigned)((rows + 256 / P - 1) / (256 / P)));
      hipLaunchKernelGGL((k_window_matvec<K, XT>), grid, dim3(256), 0, (hipStream_t)stream, (const uint8_t*)blocks,
                         (const XT*)x, (int)tokens, (XT*)out, (int)rows, (int)cols, row_bytes(K, cols), P,
                         (const uint8_t*)tables);
      return check_launch("window_matvec");
    });
  });
}

int sh_matvec_glu(int kind, const void* blocks, const void* tables, int64_t n_experts, int64_t rows, int64_t cols,
                  const int32_t* idx, int64_t pairs, const void* gate, const void* up, int dtype, void* out,
                  void* stream) {
  int st = check_rows(kind, rows, cols, "matvec_glu");
  if (st) return st;
  if (pairs <= 0) return OK;
  if (pairs > 65535) return fail(E_SHAPE, "matvec_glu: %lld pairs (at most 65535 a call)", (long long)pairs);
  if (cols * dtype_size(dtype) > 65536) return fail(E_SHAPE, "matvec_glu: inner width %lld too wide", (long long)cols);
  if (!blocks || !idx || !gate || !up || !out || (needs_tables(kind) && !tables))
    return fail(E_ARG, "matvec_glu: null pointer");
  int P = lanes_per_row(cols / 32);
  return with_kind(kind, [&](auto kc) {
    constexpr int K = decltype(kc)::value;
    return with_dtype(dtype, [&](auto* tp) {
      using XT = std::remove_pointer_t<decltype(tp)>;
      dim3 grid((unsigned)((rows + 256 / P - 1) / (256 / P)), (unsigned)pairs);
      size_t lds = ((size_t)cols * sizeof(XT) + 15) / 16 * 16;
      hipLaunchKernelGGL((k_matvec_glu<K, XT>), grid, dim3(256), lds, (hipStream_t)stream, (const uint8_t*)blocks, idx,
                         (int)n_experts, rows * row_bytes(K, cols), (const XT*)gate, (const XT*)up, (XT*)out,
                         (int)rows, (int)cols, row_bytes(K, cols), P, (const uint8_t*)tables);
      return check_launch("matvec_glu");
    });
  });
}

int sh_lookup_table(const void* x, int dtype, int64_t n, int64_t cols, void* table, void* stream) {
  if (n <= 0) return OK;
  if (cols <= 0 || cols % 64) return fail(E_SHAPE, "lookup_table: %lld inputs (Q2_0 rows are blocks of 64)", (long long)cols);
  if (!x || !table) return fail(E_ARG, "lookup_table: null pointer");
  return with_dtype(dtype, [&](auto* tp) {
    using XT = std::remove_pointer_t<decltype(tp)>;
    dim3 grid((unsigned)((cols / 2 + 255) / 256), (unsigned)n);
    hipLaunchKernelGGL((k_lookup_table<XT>), grid, dim3(256), 0, (hipStream_t)stream, (const XT*)x, (XT*)table, (int)cols);
    return check_launch("lookup_table");
  });
}

int sh_lookup_table_glu(const void* gate, const void* up, int dtype, int64_t n, int64_t cols, void* table,
                        void* stream) {
  if (n <= 0) return OK;
  if (cols <= 0 || cols % 64) return fail(E_SHAPE, "lookup_table_glu: %lld inputs", (long long)cols);
  if (!gate || !up || !table) return fail(E_ARG, "lookup_table_glu: null pointer");
  return with_dtype(dtype, [&](auto* tp) {
    using XT = std::remove_pointer_t<decltype(tp)>;
    dim3 grid((unsigned)((cols / 2 + 255) / 256), (unsigned)n);
    hipLaunchKernelGGL((k_lookup_table_glu<XT>), grid, dim3(256), 0, (hipStream_t)stream, (const XT*)gate,
                       (const XT*)up, (XT*)table, (int)cols);
    return check_launch("lookup_table_glu");
  });
}

int sh_lookup_matvec(const void* blocks, int64_t n_experts, int64_t rows, int64_t cols, const int32_t* idx,
                     int64_t pairs, const void* table, int dtype, int64_t share, void* out, void* stream) {
  int st = check_rows(Q2_0, rows, cols, "lookup_matvec");
  if (st) return st;
  if (pairs <= 0) return OK;
  if (pairs > 65535 || share <= 0) return fail(E_SHAPE, "lookup_matvec: %lld pairs, share %lld", (long long)pairs, (long long)share);
  if (!blocks || !idx || !table || !out) return fail(E_ARG, "lookup_matvec: null pointer");
  int P = lookup_lanes(cols, pairs);
  return with_dtype(dtype, [&](auto* tp) {
    using XT = std::remove_pointer_t<decltype(tp)>;
    dim3 grid((unsigned)((rows + 256 / P - 1) / (256 / P)), (unsigned)pairs);
    hipLaunchKernelGGL((k_lookup_matvec<XT>), grid, dim3(256), 0, (hipStream_t)stream, (const uint8_t*)blocks, idx,
                       (int)n_experts, rows * row_bytes(Q2_0, cols), (const XT*)table, (int)share, (XT*)out,
                       (int)rows, (int)cols, P);
    return check_launch("lookup_matvec");
  });
}

int sh_lookup_down_glu(const void* blocks, int64_t n_experts, int64_t rows, int64_t cols, const int32_t* idx,
                       int64_t pairs, const void* gate, const void* up, int dtype, void* out, void* stream) {
  int st = check_rows(Q2_0, rows, cols, "lookup_down_glu");
  if (st) return st;
  if (pairs <= 0) return OK;
  if (pairs > 65535) return fail(E_SHAPE, "lookup_down_glu: %lld pairs", (long long)pairs);
  if (!blocks || !idx || !gate || !up || !out) return fail(E_ARG, "lookup_down_glu: null pointer");
  size_t lds = (size_t)cols / 2 * 16 * dtype_size(dtype);
  if (lds > 65536) return fail(E_UNSUPPORTED, "lookup_down_glu: a table of %lld inputs does not fit LDS", (long long)cols);
  int P = lookup_lanes(cols, pairs);
  return with_dtype(dtype, [&](auto* tp) {
    using XT = std::remove_pointer_t<decltype(tp)>;
    dim3 grid((unsigned)((rows + 256 / P - 1) / (256 / P)), (unsigned)pairs);
    hipLaunchKernelGGL((k_lookup_down_glu<XT>), grid, dim3(256), lds, (hipStream_t)stream, (const uint8_t*)blocks, idx,
                       (int)n_experts, rows * row_bytes(Q2_0, cols), (const XT*)gate, (const XT*)up, (XT*)out,
                       (int)rows, (int)cols, P);
    return check_launch("lookup_down_glu");
  });
}

}  // extern "C"
