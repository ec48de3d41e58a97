// The rest of a decode layer's attention around the attend step (strata_mlx/attention.py:228-261): the queries'
// and keys' norm and rotary position (`qk_rope`, attention.py:183-222) and the append of a window's keys and values
// to the paged cache (`cache.update_and_fetch`, attention.py:251). Both are small and memory-bound: a wave a
// (token, head) row for the norm and rope, a 16-byte piece a thread for the append.
#include <algorithm>

#include "launch.h"

namespace sh {

constexpr int QR_MAX_D = 512;

// q or k of a window: each head's rms norm with its weight, then rope on the first `rot` dims, every step rounded
// to the activations' type as the reference's kernel computes in it: normed = w * T(x * inv); a = T(v c), b =
// T(o s), v = T(a + b) with o the rotated partner (-x[j + rot/2] below rot/2, x[j - rot/2] above). A wave a row.
template <typename T, int E>
__global__ __launch_bounds__(64) void k_qk_rope(const T* __restrict__ x, int heads, int tokens, int stride,
                                                 const T* __restrict__ w, float eps, const T* __restrict__ cosv,
                                                 const T* __restrict__ sinv, int rot, T* __restrict__ out,
                                                 int heads_first) {
  constexpr int D = 64 * E;
  __shared__ float normed[D];
  const int lane = threadIdx.x, h = blockIdx.x, t = blockIdx.y;
  const T* row = x + ((int64_t)t * heads + h) * stride;
  float xs[E];
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < E; ++i) {
    xs[i] = to_f32(row[lane * E + i]);
    acc = fmaf(xs[i], xs[i], acc);
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) acc += __shfl_xor(acc, o);
  const float inv = 1.0f / sqrtf(acc / (float)D + eps);
#pragma unroll
  for (int i = 0; i < E; ++i) {
    const int j = lane * E + i;
    normed[j] = to_f32(from_f32<T>(to_f32(w[j]) * to_f32(from_f32<T>(xs[i] * inv))));
  }
  __syncthreads();
  T* o = out + (heads_first ? ((int64_t)h * tokens + t) : ((int64_t)t * heads + h)) * D;
#pragma unroll
  for (int i = 0; i < E; ++i) {
    const int j = lane * E + i;
    float v = normed[j];
    if (j < rot) {
      const float c = to_f32(cosv[(int64_t)t * rot + j]), s = to_f32(sinv[(int64_t)t * rot + j]);
      const float other = j < rot / 2 ? -normed[j + rot / 2] : normed[j - rot / 2];
      const float a = to_f32(from_f32<T>(v * c)), b = to_f32(from_f32<T>(other * s));
      v = a + b;
    }
    o[j] = from_f32<T>(v);
  }
}

// the window's keys and values (n_new, hkv, D) into their pages: position pos0 + i of KV head h goes to page
// table[(pos0 + i) / 16], slot (pos0 + i) % 16 of the pool (n_pages, hkv, 16, D). A page id outside the pool is
// not written.
__global__ __launch_bounds__(256) void k_kv_append(const u32x4* __restrict__ k, const u32x4* __restrict__ v,
                                                    int64_t pieces, int hkv, int per_row, u32x4* __restrict__ kp,
                                                    u32x4* __restrict__ vp, const int32_t* __restrict__ table,
                                                    int64_t n_pages, int64_t pos0) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < pieces; i += (int64_t)gridDim.x * 256) {
    const int64_t rowi = i / per_row;  // (token, head) row
    const int c = (int)(i - rowi * per_row);
    const int64_t tok = rowi / hkv;
    const int h = (int)(rowi - tok * hkv);
    const int64_t pos = pos0 + tok;
    const int64_t page = table[pos / 16];
    if (page < 0 || page >= n_pages) continue;
    const int64_t at = ((page * hkv + h) * 16 + pos % 16) * per_row + c;
    kp[at] = k[i];
    vp[at] = v[i];
  }
}

}  // namespace sh

using namespace sh;

extern "C" {

int sh_qk_rope(const void* x, int dtype, int64_t tokens, int64_t heads, int64_t head_dim, int64_t stride,
               const void* weight, float eps, const void* cos, const void* sin, int64_t rot, void* out, int heads_first,
               void* stream) {
  if (tokens <= 0 || heads <= 0) return OK;
  if (head_dim % 64 || head_dim <= 0 || head_dim > QR_MAX_D)
    return fail(E_UNSUPPORTED, "qk_rope: head_dim %lld (a multiple of 64, at most %d)", (long long)head_dim, QR_MAX_D);
  if (stride < head_dim || rot < 0 || rot > head_dim || rot % 2)
    return fail(E_SHAPE, "qk_rope: stride %lld, rot %lld for heads of %lld", (long long)stride, (long long)rot,
                (long long)head_dim);
  if (heads > 65535 || tokens > 65535) return fail(E_SHAPE, "qk_rope: %lld heads x %lld tokens", (long long)heads,
                                                   (long long)tokens);
  if (!x || !weight || !out || (rot && (!cos || !sin))) return fail(E_ARG, "qk_rope: null pointer");
  return with_dtype(dtype, [&](auto* tp) {
    using T = std::remove_pointer_t<decltype(tp)>;
    auto go = [&](auto ec) {
      constexpr int E = decltype(ec)::value;
      hipLaunchKernelGGL((k_qk_rope<T, E>), dim3((unsigned)heads, (unsigned)tokens), dim3(64), 0, (hipStream_t)stream,
                         (const T*)x, (int)heads, (int)tokens, (int)stride, (const T*)weight, eps, (const T*)cos,
                         (const T*)sin, (int)rot, (T*)out, heads_first);
      return check_launch("qk_rope");
    };
    switch (head_dim / 64) {
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

int sh_kv_append(const void* k, const void* v, int64_t n_new, int64_t hkv, int64_t head_dim, int dtype, void* k_pages,
                 void* v_pages, const int32_t* page_table, int64_t table_pages, int64_t n_pages, int64_t pos0,
                 void* stream) {
  if (n_new <= 0) return OK;
  if (hkv <= 0 || head_dim <= 0 || (head_dim * dtype_size(dtype)) % 16 || pos0 < 0 || n_pages <= 0)
    return fail(E_SHAPE, "kv_append: %lld KV heads of %lld at position %lld", (long long)hkv, (long long)head_dim,
                (long long)pos0);
  if (table_pages <= 0 || pos0 + n_new > table_pages * 16)
    return fail(E_SHAPE, "kv_append: positions %lld .. %lld past a page table of %lld pages", (long long)pos0,
                (long long)(pos0 + n_new - 1), (long long)table_pages);
  if (dtype != F16 && dtype != BF16 && dtype != F32) return fail(E_DTYPE, "kv_append: dtype %d", dtype);
  if (!k || !v || !k_pages || !v_pages || !page_table) return fail(E_ARG, "kv_append: null pointer");
  if (((uintptr_t)k | (uintptr_t)v | (uintptr_t)k_pages | (uintptr_t)v_pages) & 15)
    return fail(E_ARG, "kv_append: keys, values and pages must be 16-byte aligned");
  const int per_row = (int)(head_dim * dtype_size(dtype) / 16);
  const int64_t pieces = n_new * hkv * per_row;
  const unsigned grid = (unsigned)std::min<int64_t>((pieces + 255) / 256, 4 * device_cus());
  hipLaunchKernelGGL(k_kv_append, dim3(grid), dim3(256), 0, (hipStream_t)stream, (const u32x4*)k, (const u32x4*)v,
                     pieces, (int)hkv, per_row, (u32x4*)k_pages, (u32x4*)v_pages, page_table, n_pages, pos0);
  return check_launch("kv_append");
}

}  // extern "C"
