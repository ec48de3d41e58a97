// The HIP device environment the library's kernels are written against, restated for the host so that the kernels
// themselves run on the CPU: test infrastructure only (tests/hostrun/build.py compiles strata-mlx_amd/csrc with it
// into a separate library the tests call; the package never loads it).
//
// Execution model. A launch runs its workgroups one after another. Inside a workgroup every thread is a fiber with a
// stack of its own; a fiber runs until it reaches a point where the hardware would make it wait for other threads:
// a workgroup barrier, or a cross-lane operation of its wave (DPP, ballot, shuffles, readfirstlane, MFMA, the
// transposing LDS read). A cross-lane operation completes when every live lane of the wave has reached it, from the
// values all of them brought, as the wave's single instruction would. LDS is a buffer of the launch's dynamic size,
// filled with a garbage pattern before each workgroup; loads into LDS complete at once. Global memory is host
// memory. What this model cannot show: timing, the memory model across workgroups running at once, wait states.
#pragma once

#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <functional>
#include <type_traits>

#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define __launch_bounds__(...)
#define __restrict__ __restrict
#define __align__(n) __attribute__((aligned(n)))
#define __shared__ static

#ifndef __HIP_MEMORY_SCOPE_AGENT
#define __HIP_MEMORY_SCOPE_WAVEFRONT 2
#define __HIP_MEMORY_SCOPE_WORKGROUP 3
#define __HIP_MEMORY_SCOPE_AGENT 4
#define __HIP_MEMORY_SCOPE_SYSTEM 5
#endif

struct dim3 {
  uint32_t x, y, z;
  constexpr dim3(uint32_t x_ = 1, uint32_t y_ = 1, uint32_t z_ = 1) : x(x_), y(y_), z(z_) {}
};

namespace hostrun {

struct Idx3 {
  uint32_t x, y, z;
};

struct Wave {
  uint64_t live = 0;     // lanes that have not returned
  uint64_t arrived = 0;  // lanes waiting at the pending operation
  const void* site = nullptr;
  void (*pending)(Wave&, const void*) = nullptr;
  const void* pending_fn = nullptr;
  alignas(16) unsigned char in[64][64];
  alignas(16) unsigned char out[64][64];
};

enum State : int { READY = 0, WAITING = 1, DONE = 2 };

struct Fiber {
  void* sp = nullptr;
  char* stack = nullptr;
  Idx3 tid{0, 0, 0};
  int flat = 0, lane = 0;
  Wave* wave = nullptr;
  State state = READY;
  bool at_barrier = false;
};

extern Fiber* cur;
extern Idx3 block_idx, block_dim, grid_dim;

[[noreturn]] void die(const char* fmt, ...);
void yield();                   // back to the scheduler (the fiber has set its state)
void complete(Wave& w);         // run the pending operation, release its lanes
void barrier();                 // __syncthreads / s_barrier
unsigned char* lds_base();      // the workgroup's dynamic LDS
size_t lds_size();
uint32_t lds_addr(const void* p);  // LDS byte address of a pointer into the dynamic LDS
void load_lds(const void* src, uint32_t m0);  // one lane's 16 bytes of a direct load into LDS
void launch(const char* name, dim3 grid, dim3 block, size_t shmem, const std::function<void()>& body);

template <class F> struct SiteTag {
  static constexpr char tag = 0;
};

template <class In, class Out, class F> void run_op(Wave& w, const void* fnp) {
  const F& fn = *(const F*)fnp;
  In in[64];
  Out out[64];
  for (int l = 0; l < 64; ++l) memcpy((void*)&in[l], w.in[l], sizeof(In));
  memset((void*)out, 0, sizeof out);
  fn(in, out, w.live);
  for (int l = 0; l < 64; ++l) memcpy(w.out[l], (const void*)&out[l], sizeof(Out));
}

// one cross-lane operation: each lane brings `v`; fn(in[64], out[64], live) computes every lane's result once all
// live lanes have arrived. fn may only use values of its lanes' inputs (captures must be the same in every lane).
template <class In, class Out, class F> inline Out wave_op(const In& v, const F& fn) {
  static_assert(sizeof(In) <= 64 && sizeof(Out) <= 64, "wave operands of at most 64 bytes");
  Fiber* f = cur;
  Wave& w = *f->wave;
  memcpy(w.in[f->lane], (const void*)&v, sizeof(In));
  const void* site = &SiteTag<F>::tag;
  if (w.arrived == 0) {
    w.site = site;
    w.pending = &run_op<In, Out, F>;
    w.pending_fn = &fn;
  } else if (w.site != site) {
    die("lanes of one wave at different cross-lane operations (divergent control flow)");
  }
  w.arrived |= 1ull << f->lane;
  if (w.arrived == w.live) {
    complete(w);
  } else {
    f->state = WAITING;
    yield();
  }
  Out r;
  memcpy((void*)&r, w.out[f->lane], sizeof(Out));
  return r;
}

// a value the kernel holds wave-uniform by contract, taken from the lane itself
template <class T> inline T lane_value(T v) { return v; }

inline int first_lane(uint64_t live) { return live ? __builtin_ctzll(live) : 0; }

template <class T> struct Pair {
  T a;
  int b;
};

template <int KPL> struct MfmaIn {
  unsigned char a[KPL * 2], b[KPL * 2];
  float c[4];
};
struct F4 {
  float v[4];
};

inline float hostrun_half(uint16_t h, bool bf) {
  if (bf) {
    const uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
  }
  _Float16 v;
  memcpy(&v, &h, 2);
  return (float)v;
}

// D = C + A B for one 16 x 16 tile of a wave, K = 4 KPL: lane l holds A[l % 16][k] and B[k][l % 16] for
// k = KPL (l / 16) .. + KPL - 1, and D[4 (l / 16) + r][l % 16], r = 0..3. The products of 16-bit values are exact
// in float32; the sums here are float32 in k order (the hardware's order and roundings of its sums differ at the
// last bits).
template <int KPL, bool BF> inline F4 mfma(const MfmaIn<KPL>& in) {
  return wave_op<MfmaIn<KPL>, F4>(in, [](const MfmaIn<KPL>* x, F4* d, uint64_t live) {
    if (live != ~0ull) die("an MFMA with lanes that have returned");
    constexpr int K = 4 * KPL;
    float A[16][K], B[16][K], C[16][16];  // B by column
    for (int l = 0; l < 64; ++l) {
      uint16_t ha[KPL], hb[KPL];
      memcpy(ha, x[l].a, sizeof ha);
      memcpy(hb, x[l].b, sizeof hb);
      for (int j = 0; j < KPL; ++j) {
        A[l % 16][KPL * (l / 16) + j] = hostrun_half(ha[j], BF);
        B[l % 16][KPL * (l / 16) + j] = hostrun_half(hb[j], BF);
      }
      for (int r = 0; r < 4; ++r) C[4 * (l / 16) + r][l % 16] = x[l].c[r];
    }
    for (int m = 0; m < 16; ++m)
      for (int n = 0; n < 16; ++n) {
        float s = 0.0f;
        for (int k = 0; k < K; ++k) s = fmaf(A[m][k], B[n][k], s);
        C[m][n] += s;
      }
    for (int l = 0; l < 64; ++l)
      for (int r = 0; r < 4; ++r) d[l].v[r] = C[4 * (l / 16) + r][l % 16];
  });
}

// DPP source lane of `lane` for the controls the kernels use; -1 where the control reads no lane
inline int dpp_source(int lane, int ctrl) {
  const int row = lane & ~15, in_row = lane & 15;
  if (ctrl <= 0xff) return (lane & ~3) | ((ctrl >> (2 * (lane & 3))) & 3);  // quad_perm
  if (ctrl >= 0x101 && ctrl <= 0x10f) {                                    // row_shl
    const int n = ctrl & 15;
    return in_row + n < 16 ? lane + n : -1;
  }
  if (ctrl >= 0x111 && ctrl <= 0x11f) {  // row_shr
    const int n = ctrl & 15;
    return in_row >= n ? lane - n : -1;
  }
  if (ctrl >= 0x121 && ctrl <= 0x12f) return row + ((in_row - (ctrl & 15)) & 15);  // row_ror
  if (ctrl == 0x130) return lane < 63 ? lane + 1 : -1;                            // wave_shl:1
  if (ctrl == 0x134) return (lane + 1) & 63;                                      // wave_rol:1
  if (ctrl == 0x138) return lane > 0 ? lane - 1 : -1;                             // wave_shr:1
  if (ctrl == 0x13c) return (lane + 63) & 63;                                     // wave_ror:1
  if (ctrl == 0x140) return row + 15 - in_row;                                    // row_mirror
  if (ctrl == 0x141) return (lane & ~7) + 7 - (lane & 7);                         // row_half_mirror
  if (ctrl == 0x142) return row >= 16 ? row - 1 : -1;                             // row_bcast:15
  if (ctrl == 0x143) return row >= 32 ? 31 : -1;                                  // row_bcast:31
  die("DPP control 0x%x", ctrl);
}

}  // namespace hostrun

#define threadIdx (::hostrun::cur->tid)
#define blockIdx (::hostrun::block_idx)
#define blockDim (::hostrun::block_dim)
#define gridDim (::hostrun::grid_dim)

// ---- cross-lane operations

template <class T> inline T __shfl(T v, int src, int width = 64) {
  using P = hostrun::Pair<T>;
  return hostrun::wave_op<P, T>(P{v, src}, [](const P* in, T* out, uint64_t) {
    for (int l = 0; l < 64; ++l) {
      // HIP: index = src + (lane & ~(width - 1)), read modulo the wave
      out[l] = in[(in[l].b + (l & ~63)) & 63].a;
    }
  });
}
template <class T> inline T __shfl_xor(T v, int mask, int width = 64) {
  using P = hostrun::Pair<T>;
  return hostrun::wave_op<P, T>(P{v, mask}, [](const P* in, T* out, uint64_t) {
    for (int l = 0; l < 64; ++l) {
      const int i = l ^ in[l].b;
      out[l] = in[i >= 64 ? l : i].a;
    }
  });
}
template <class T> inline T __shfl_up(T v, unsigned delta, int width = 64) {
  using P = hostrun::Pair<T>;
  return hostrun::wave_op<P, T>(P{v, (int)delta}, [](const P* in, T* out, uint64_t) {
    for (int l = 0; l < 64; ++l) {
      const int i = l - in[l].b;
      out[l] = in[i < 0 ? l : i].a;
    }
  });
}
inline unsigned long long __ballot(int pred) {
  return hostrun::wave_op<int, unsigned long long>(pred, [](const int* in, unsigned long long* out, uint64_t live) {
    unsigned long long m = 0;
    for (int l = 0; l < 64; ++l)
      if (((live >> l) & 1) && in[l]) m |= 1ull << l;
    for (int l = 0; l < 64; ++l) out[l] = m;
  });
}
inline int __any(int pred) { return __ballot(pred) != 0; }
inline int __all(int pred) {
  return hostrun::wave_op<int, int>(pred, [](const int* in, int* out, uint64_t live) {
    int all = 1;
    for (int l = 0; l < 64; ++l)
      if (((live >> l) & 1) && !in[l]) all = 0;
    for (int l = 0; l < 64; ++l) out[l] = all;
  });
}
template <class T> inline T __builtin_amdgcn_readfirstlane(T v) {
  return hostrun::wave_op<T, T>(v, [](const T* in, T* out, uint64_t live) {
    const T x = in[hostrun::first_lane(live)];
    for (int l = 0; l < 64; ++l) out[l] = x;
  });
}
template <class T> inline T __builtin_amdgcn_readlane(T v, int lane) {
  using P = hostrun::Pair<T>;
  return hostrun::wave_op<P, T>(P{v, lane}, [](const P* in, T* out, uint64_t live) {
    const T x = in[in[hostrun::first_lane(live)].b & 63].a;
    for (int l = 0; l < 64; ++l) out[l] = x;
  });
}
template <class T>
inline T __builtin_amdgcn_update_dpp(T old, T src, int ctrl, int row_mask, int bank_mask, bool bound_ctrl) {
  static_assert(sizeof(T) == 4, "32-bit DPP moves");
  struct In {
    T old, src;
    int ctrl, row_mask, bank_mask, bound;
  };
  return hostrun::wave_op<In, T>(In{old, src, ctrl, row_mask, bank_mask, bound_ctrl ? 1 : 0},
                                 [](const In* in, T* out, uint64_t live) {
                                   for (int l = 0; l < 64; ++l) {
                                     const In& me = in[l];
                                     const bool on = ((me.row_mask >> (l >> 4)) & 1) &&
                                                     ((me.bank_mask >> ((l & 15) >> 2)) & 1);
                                     const int s = hostrun::dpp_source(l, me.ctrl);
                                     if (!on)
                                       out[l] = me.old;
                                     else if (s < 0 || !((live >> s) & 1))
                                       out[l] = me.bound ? T{} : me.old;
                                     else
                                       out[l] = in[s].src;
                                   }
                                 });
}
inline void __builtin_amdgcn_wave_barrier() {
  hostrun::wave_op<int, int>(0, [](const int*, int*, uint64_t) {});
}
inline void __syncthreads() { hostrun::barrier(); }
inline void __builtin_amdgcn_s_barrier() { hostrun::barrier(); }
inline void __builtin_amdgcn_sched_barrier(int) {}
inline void __builtin_amdgcn_s_waitcnt(int) {}
inline void __builtin_amdgcn_s_sleep(int) { hostrun::die("s_sleep: a wait on another workgroup cannot end here"); }
#define __builtin_amdgcn_fence(order, scope) ((void)0)

template <class V, class C> inline C __builtin_amdgcn_mfma_f32_16x16x32_bf16(V a, V b, C c, int, int, int) {
  static_assert(sizeof(V) == 16, "8 bfloat16 a lane");
  hostrun::MfmaIn<8> in;
  memcpy(in.a, &a, 16);
  memcpy(in.b, &b, 16);
  memcpy(in.c, &c, 16);
  const hostrun::F4 d = hostrun::mfma<8, true>(in);
  C r;
  memcpy(&r, d.v, 16);
  return r;
}
template <class V, class C> inline C __builtin_amdgcn_mfma_f32_16x16x32_f16(V a, V b, C c, int, int, int) {
  static_assert(sizeof(V) == 16, "8 float16 a lane");
  hostrun::MfmaIn<8> in;
  memcpy(in.a, &a, 16);
  memcpy(in.b, &b, 16);
  memcpy(in.c, &c, 16);
  const hostrun::F4 d = hostrun::mfma<8, false>(in);
  C r;
  memcpy(&r, d.v, 16);
  return r;
}
template <class V, class C> inline C __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(V a, V b, C c, int, int, int) {
  static_assert(sizeof(V) == 8, "4 bfloat16 a lane");
  hostrun::MfmaIn<4> in;
  memcpy(in.a, &a, 8);
  memcpy(in.b, &b, 8);
  memcpy(in.c, &c, 16);
  const hostrun::F4 d = hostrun::mfma<4, true>(in);
  C r;
  memcpy(&r, d.v, 16);
  return r;
}
template <class V, class C> inline C __builtin_amdgcn_mfma_f32_16x16x16f16(V a, V b, C c, int, int, int) {
  static_assert(sizeof(V) == 8, "4 float16 a lane");
  hostrun::MfmaIn<4> in;
  memcpy(in.a, &a, 8);
  memcpy(in.b, &b, 8);
  memcpy(in.c, &c, 16);
  const hostrun::F4 d = hostrun::mfma<4, false>(in);
  C r;
  memcpy(&r, d.v, 16);
  return r;
}

typedef short hostrun_v4i16 __attribute__((ext_vector_type(4)));
// gfx950's transposing LDS read of 16-bit elements: within each 16-lane group, lane i receives element i % 4 of the
// 8-byte pieces named by lanes i / 4 + 4 m of the group, m = 0..3
template <class P> inline hostrun_v4i16 __builtin_amdgcn_ds_read_tr16_b64_v4i16(P p) {
  struct In {
    uint64_t piece;
  };
  uint64_t piece;
  memcpy(&piece, (const void*)p, 8);
  struct Out {
    int16_t e[4];
  };
  const Out o = hostrun::wave_op<In, Out>(In{piece}, [](const In* in, Out* out, uint64_t) {
    for (int l = 0; l < 64; ++l) {
      const int g = l & ~15, i = l & 15;
      for (int m = 0; m < 4; ++m) out[l].e[m] = (int16_t)(in[g + i / 4 + 4 * m].piece >> (16 * (i % 4)));
    }
  });
  hostrun_v4i16 r;
  for (int m = 0; m < 4; ++m) r[m] = o.e[m];
  return r;
}

// ---- per-lane operations

inline uint32_t __builtin_amdgcn_perm(uint32_t s0, uint32_t s1, uint32_t sel) {
  const uint64_t d = ((uint64_t)s0 << 32) | s1;
  uint32_t r = 0;
  for (int i = 0; i < 4; ++i) {
    const uint32_t s = (sel >> (8 * i)) & 0xff;
    uint32_t b;
    if (s >= 13)
      b = 0xff;
    else if (s == 12)
      b = 0;
    else if (s >= 8)
      b = ((d >> (16 * (s - 8) + 15)) & 1) ? 0xff : 0;
    else
      b = (uint32_t)(d >> (8 * s)) & 0xff;
    r |= b << (8 * i);
  }
  return r;
}

struct hostrun_rsrc {
  const char* base;
};
typedef hostrun_rsrc __amdgpu_buffer_rsrc_t;
inline __amdgpu_buffer_rsrc_t __builtin_amdgcn_make_buffer_rsrc(void* base, short, int, int) {
  return hostrun_rsrc{(const char*)base};
}
typedef uint32_t hostrun_u32x4 __attribute__((ext_vector_type(4)));
inline hostrun_u32x4 __builtin_amdgcn_raw_buffer_load_b128(__amdgpu_buffer_rsrc_t r, int voff, int soff, int) {
  hostrun_u32x4 v;
  memcpy(&v, r.base + (int64_t)voff + soff, 16);
  return v;
}

#define HOSTRUN_MINMAX(T)                             \
  inline T min(T a, T b) { return a < b ? a : b; } \
  inline T max(T a, T b) { return a < b ? b : a; }
HOSTRUN_MINMAX(int)
HOSTRUN_MINMAX(unsigned)
HOSTRUN_MINMAX(long)
HOSTRUN_MINMAX(unsigned long)
HOSTRUN_MINMAX(long long)
HOSTRUN_MINMAX(unsigned long long)
HOSTRUN_MINMAX(float)
HOSTRUN_MINMAX(double)
#undef HOSTRUN_MINMAX

inline int __popc(unsigned v) { return __builtin_popcount(v); }
inline int __popcll(unsigned long long v) { return __builtin_popcountll(v); }
inline int __ffs(int v) { return __builtin_ffs(v); }
inline int __ffsll(long long v) { return __builtin_ffsll(v); }
inline int __ffsll(unsigned long long v) { return __builtin_ffsll((long long)v); }
inline float __uint_as_float(unsigned v) { return __builtin_bit_cast(float, v); }
inline unsigned __float_as_uint(float v) { return __builtin_bit_cast(unsigned, v); }

// __hip_atomic_* are the compiler's own builtins on every target; HIP's atomicAdd / atomicOr over them
template <class T> inline T atomicAdd(T* p, T v) {
  T old, next;
  __atomic_load(p, &old, __ATOMIC_SEQ_CST);
  do {
    next = old + v;
  } while (!__atomic_compare_exchange(p, &old, &next, false, __ATOMIC_SEQ_CST, __ATOMIC_SEQ_CST));
  return old;
}
template <class T> inline T atomicOr(T* p, T v) { return __atomic_fetch_or(p, v, __ATOMIC_SEQ_CST); }

// ---- the host API the library calls

typedef struct hostrun_stream* hipStream_t;
typedef int hipError_t;
constexpr hipError_t hipSuccess = 0;
enum hipMemcpyKind { hipMemcpyHostToHost = 0, hipMemcpyHostToDevice, hipMemcpyDeviceToHost, hipMemcpyDeviceToDevice,
                     hipMemcpyDefault };
enum hipDeviceAttribute_t { hipDeviceAttributeMultiprocessorCount = 1 };
struct hipFuncAttributes {
  size_t sharedSizeBytes = 0;
};

hipError_t hipGetLastError();
const char* hipGetErrorString(hipError_t);
hipError_t hipGetDevice(int* dev);
hipError_t hipDeviceGetAttribute(int* v, hipDeviceAttribute_t a, int dev);
hipError_t hipMemcpyAsync(void* dst, const void* src, size_t n, hipMemcpyKind, hipStream_t);
hipError_t hipMemsetAsync(void* dst, int v, size_t n, hipStream_t);
hipError_t hipFuncGetAttributes(hipFuncAttributes* a, const void* f);
int hostrun_occupancy(int threads, size_t shmem);
template <class K> inline hipError_t hipOccupancyMaxActiveBlocksPerMultiprocessor(int* n, K, int threads, size_t shmem) {
  *n = hostrun_occupancy(threads, shmem);
  return hipSuccess;
}
inline hipError_t hipGetSymbolAddress(void** p, const void* symbol) {
  *p = const_cast<void*>(symbol);
  return hipSuccess;
}
#define HIP_SYMBOL(s) ((const void*)&(s))

#define hipLaunchKernelGGL(K, G, B, S, ST, ...) \
  ::hostrun::launch(#K, dim3(G), dim3(B), (size_t)(S), [=]() { K(__VA_ARGS__); })
