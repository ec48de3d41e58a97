// Device building blocks of the MFMA expert products (expert.hip, moe.hip): magic-number decode of Q2_0 and IQ3_S
// codes into MFMA operands, staging of weights and activations to LDS with every load issued before any store, the
// per-tile multiply-accumulate, and wave reductions on DPP.
//
//   D[token][row] += x[token][k] * q[k][row]      v_mfma_f32_16x16x32_{bf16,f16}
//
// The weights are the B operand, so a lane's accumulators are for the row it decoded (row = lane % 16) and the block
// scale it decoded applies to them directly. Tokens sit at M-rows 4 * (t / TPG) + t % TPG: only TPG of a lane's four
// accumulators are real, and the scale costs TPG fmas a scale group.
//
// Decode without multiplies: a code is ORed into the mantissa of a constant ("magic") — for bf16 0x4300 | c is
// 128 + c — so a pair of weights is one v_and_or. Codes sitting higher in a byte are masked in place (value
// 128 + U*c) and their activation staged as x / U (exact: a power of two). The constant offsets are removed by a
// correction MFMA against a constant operand, chained as the accumulator input:
//   Q2_0:  q = 128 + U c  (bf16) or 1024 + U c (fp16),  correction -(BASE + U)   ->  sum (c - 1) x
//   IQ3_S: q = 144 + v    (bf16) or 1040 + v  (fp16),   v = +-grid from a 32 KiB LDS table of signed entries,
//          correction -144 / -1040                     ->  sum v x
// Every product is exact in float32; the offsets cost precision only in the float32 accumulation (about 1e-6 of a
// block's sum for bf16), far inside the 1e-2 bf16 tolerance.
#pragma once

#include <type_traits>

#include "decode.h"

namespace sh {

template <typename MT> struct Magic;
template <> struct Magic<bf16> {
  static constexpr uint32_t M2 = 0x43004300u;  // two bf16 128.0
  static constexpr uint32_t HI = 0x43u;        // high byte of a bf16 128 + b
  static constexpr float BASE = 128.0f;
};
template <> struct Magic<f16> {
  static constexpr uint32_t M2 = 0x64006400u;  // two fp16 1024.0
  static constexpr uint32_t HI = 0x64u;
  static constexpr float BASE = 1024.0f;
};

template <typename MT> __device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (std::is_same_v<MT, bf16>)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
}

template <typename MT> __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  uint16_t a = __builtin_bit_cast(uint16_t, (MT)lo), b = __builtin_bit_cast(uint16_t, (MT)hi);
  return (uint32_t)a | ((uint32_t)b << 16);
}

// ---- Q2_0 (64 weights, 18 bytes: fp16 d, then 16 code bytes, byte i holding weights 4i..4i+3)
//
// Lane group g = lane / 16 of the wave decodes code bytes 2g, 2g+1, 8+2g, 9+2g of each block for its row: the
// dword W = b[2+2g] | b[3+2g] << 8 | b[10+2g] << 16 | b[11+2g] << 24. Block-local weight
// k = 32h + 8g + 4a + j (h: low/high half of W, a: MFMA a or b, j: code within the byte) goes to slot 2j + h of
// MFMA a. U_j is the scale of the in-place mask of code j.
template <typename MT> __host__ __device__ constexpr float q2_unit(int j) {
  if constexpr (std::is_same_v<MT, bf16>) return j == 1 ? 4.0f : j == 2 ? 16.0f : 1.0f;  // bits 6-7 shifted down
  else return j == 1 ? 4.0f : j == 2 ? 16.0f : j == 3 ? 64.0f : 1.0f;
}

template <typename MT> __device__ __forceinline__ void q2_decode(uint32_t W, u32x4& fa, u32x4& fb) {
  constexpr uint32_t M = Magic<MT>::M2;
  const uint32_t W8 = W >> 8;
  fa.x = (W & 0x00030003u) | M;
  fa.y = (W & 0x000C000Cu) | M;
  fa.z = (W & 0x00300030u) | M;
  fb.x = (W8 & 0x00030003u) | M;
  fb.y = (W8 & 0x000C000Cu) | M;
  fb.z = (W8 & 0x00300030u) | M;
  if constexpr (std::is_same_v<MT, bf16>) {  // bit 7 of a bf16 half is exponent: code 3 shifted to bits 0-1
    fa.w = ((W >> 6) & 0x00030003u) | M;
    fb.w = ((W >> 14) & 0x00030003u) | M;
  } else {
    fa.w = (W & 0x00C000C0u) | M;
    fb.w = (W8 & 0x00C000C0u) | M;
  }
}

// the correction operand: slot 2j + h holds -(BASE + U_j)
template <typename MT> __device__ __forceinline__ u32x4 q2_correction() {
  u32x4 c;
  c.x = pack2<MT>(-(Magic<MT>::BASE + q2_unit<MT>(0)), -(Magic<MT>::BASE + q2_unit<MT>(0)));
  c.y = pack2<MT>(-(Magic<MT>::BASE + q2_unit<MT>(1)), -(Magic<MT>::BASE + q2_unit<MT>(1)));
  c.z = pack2<MT>(-(Magic<MT>::BASE + q2_unit<MT>(2)), -(Magic<MT>::BASE + q2_unit<MT>(2)));
  c.w = pack2<MT>(-(Magic<MT>::BASE + q2_unit<MT>(3)), -(Magic<MT>::BASE + q2_unit<MT>(3)));
  return c;
}

// the staged position (within the block's 64) of activation kk of a Q2_0 block: fragment (a, g), slot 2j + h
__device__ __forceinline__ int q2_stage_pos(int kk, int& j) {
  int h = kk >> 5, g = (kk >> 3) & 3, a = (kk >> 2) & 1;
  j = kk & 3;
  return ((a * 4 + g) * 8) + 2 * j + h;
}

constexpr int IQ3S_SIGNED_BYTES = 8192 * 4;  // entry (grid index | sign nibble << 9) -> four bytes 16 +- value

// ---- staging: every load of a thread's share issued before any of its stores (one memory round trip)

__device__ __forceinline__ int lead_of(const void* p) { return (int)((uintptr_t)p & 15); }

// ---- direct loads into LDS (gfx950 global_load_lds_dwordx4): lane l of the wave writes the 16 bytes at
// base + off_l to LDS address lds + 16 * l; base and lds (an LDS byte address, lds_addr of the block's LDS array
// plus an offset) are the same for every lane of the wave. The load counts in vmcnt like
// any other; readers wait with wait_vmcnt and meet at lds_sync. Issued from inline assembly: the compiler's wait
// insertion, which would count such a load as pending on the LDS counter too and then wait for every LDS read at
// once, does not see it (its own waits on younger loads stay correct: the counter drains in order).
//
// The wait states the hardware needs before such a load are in the assembly itself, since the compiler inserts none
// for an inline-assembly instruction: a VMEM instruction reading an SGPR that a VALU instruction wrote needs 5 (the
// base, when the compiler computed it in vector registers, is moved to SGPRs by v_readfirstlane just before), and
// an LDS direct load needs 1 after M0 is written (the compiler writes M0 just before). Without them the load can
// take a stale base or LDS address: the two kernels that issued loads in that state ended in illegal memory
// accesses.
__device__ __forceinline__ void lds_dma16(const void* base, uint32_t off, uint32_t lds) {
  // the base is wave-uniform by contract: read from the first lane, it is a scalar operand whatever the compiler
  // could prove
  const uint64_t b = (uint64_t)(uintptr_t)base;
  const uint64_t sb = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) << 32) |
                      (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
  asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"((const void*)(uintptr_t)sb),
               "{m0}"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}
// the same with a full address a lane (sources in different tensors within one wave's load): no SGPR operand, the
// wait state after M0's write
__device__ __forceinline__ void lds_dma16p(const void* src, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}
// the LDS byte address of a __shared__ array (cast on the array itself: no null check of a generic pointer)
#define SH_LDS_ADDR(arr) ((uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)(arr))

// ---- data handed from block to block inside one launch: stores and loads with the agent-scope coherence bit (sc1),
// which the chip keeps coherent across its XCDs' L2s as it keeps agent-scope atomics (they compile to the same
// accesses). A writer's stores are complete once its vmcnt drains, so it waits for them and then counts; a reader
// issues its loads after it has seen the count. No cache is written back or invalidated on either side: an
// agent-scope fence would do both, over the whole L2 of its XCD, and a launch of hundreds of blocks that each fence
// spends tens of microseconds on them.
template <typename T> __device__ __forceinline__ void st_agent(T* p, T v) {
  static_assert(sizeof(T) == 2 || sizeof(T) == 4, "st_agent: 16- or 32-bit values");
  using U = std::conditional_t<sizeof(T) == 2, uint16_t, uint32_t>;
  U bits;
  __builtin_memcpy(&bits, &v, sizeof(T));
  __hip_atomic_store((U*)p, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// 16 bytes at base + off (base wave-uniform, off < 2^31), read at agent scope
__device__ __forceinline__ u32x4 ld_agent16(const void* base, uint32_t off) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7fffffff, 0x00020000);
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 16 /* sc1 */);
}

// at most n of this wave's memory loads still in flight (n wave-uniform; values above 63 wait for none)
__device__ __forceinline__ void wait_vmcnt(int n) {
#define SH_VMCNT_CASE(k) \
  case k: asm volatile("s_waitcnt vmcnt(" #k ")" ::: "memory"); break;
#define SH_VMCNT_8(k) SH_VMCNT_CASE(k) SH_VMCNT_CASE(k + 1) SH_VMCNT_CASE(k + 2) SH_VMCNT_CASE(k + 3) \
  SH_VMCNT_CASE(k + 4) SH_VMCNT_CASE(k + 5) SH_VMCNT_CASE(k + 6) SH_VMCNT_CASE(k + 7)
  switch (n) {
    SH_VMCNT_8(0) SH_VMCNT_8(8) SH_VMCNT_8(16) SH_VMCNT_8(24) SH_VMCNT_8(32) SH_VMCNT_8(40) SH_VMCNT_8(48)
    SH_VMCNT_8(56)
    default: break;
  }
#undef SH_VMCNT_8
#undef SH_VMCNT_CASE
}

// every wave's LDS stores done and visible to the block; loads into LDS still in flight stay in flight (a
// __syncthreads would wait for them)
__device__ __forceinline__ void lds_sync() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Up to two byte ranges to LDS, range i at dst_i + (src_i & 15) (alignment kept modulo 16), 16-byte chunks; edge
// chunks byte by byte. A pass covers UNROLL * nthreads chunks: load(pass) then store(pass).
template <int UNROLL> struct ByteStage {
  const uint8_t *s0, *s1;
  uint8_t *d0, *d1;
  uintptr_t a0, a1;
  int n0, n1, c0, total;
  u32x4 v[UNROLL];
  bool full[UNROLL];

  __device__ __forceinline__ ByteStage(uint8_t* dst0, const uint8_t* src0, int nb0, uint8_t* dst1, const uint8_t* src1,
                                       int nb1)
      : s0(src0), s1(src1), d0(dst0), d1(dst1), n0(nb0), n1(nb1) {
    a0 = (uintptr_t)src0 & ~(uintptr_t)15;
    a1 = (uintptr_t)src1 & ~(uintptr_t)15;
    c0 = nb0 > 0 ? ((int)((uintptr_t)src0 - a0) + nb0 + 15) >> 4 : 0;
    int c1 = nb1 > 0 ? ((int)((uintptr_t)src1 - a1) + nb1 + 15) >> 4 : 0;
    total = c0 + c1;
  }
  __device__ __forceinline__ int passes(int nthreads) const { return (total + UNROLL * nthreads - 1) / (UNROLL * nthreads); }
  __device__ __forceinline__ const uint8_t* chunk(int c, const uint8_t*& s, int& n, uint8_t*& d) const {
    const bool first = c < c0;
    const int cc = first ? c : c - c0;
    s = first ? s0 : s1;
    n = first ? n0 : n1;
    d = (first ? d0 : d1) + 16 * cc;
    return (const uint8_t*)((first ? a0 : a1) + 16 * (uintptr_t)cc);
  }
  __device__ __forceinline__ void load(int pass, int tid, int nthreads) {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int c = (pass * UNROLL + u) * nthreads + tid;
      full[u] = false;
      if (c < total) {
        const uint8_t* s;
        int n;
        uint8_t* d;
        const uint8_t* p = chunk(c, s, n, d);
        if (p >= s && p + 16 <= s + n) {
          v[u] = *(const u32x4*)p;
          full[u] = true;
        }
      }
    }
  }
  __device__ __forceinline__ void store(int pass, int tid, int nthreads) {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int c = (pass * UNROLL + u) * nthreads + tid;
      if (c >= total) continue;
      const uint8_t* s;
      int n;
      uint8_t* d;
      const uint8_t* p = chunk(c, s, n, d);
      if (full[u]) {
        *(u32x4*)d = v[u];
      } else {
        for (int b = 0; b < 16; ++b)
          if (p + b >= s && p + b < s + n) d[b] = p[b];
      }
    }
  }
};

// n_tok activation rows (row t at xrow[t], `cols` 16-bit values, 16-byte aligned) into LDS `xs` (row t at
// xs + t * cols, MT) in the layout KIND's decode reads: Q2_0 permuted and scaled by 1 / U per slot, IQ3_S as they
// are. A pass covers UNROLL * nthreads vectors of 8: load(pass) then store(pass).
template <int KIND, typename XT, typename MT, int UNROLL> struct XStage {
  static_assert(sizeof(XT) == 2, "16-bit activations");
  const XT* const* xrow;
  MT* xs;
  int cols, per_row, total;
  u32x4 v[UNROLL];

  __device__ __forceinline__ XStage(MT* xs_, const XT* const* xrow_, int n_tok, int cols_)
      : xrow(xrow_), xs(xs_), cols(cols_), per_row(cols_ >> 3), total(n_tok * (cols_ >> 3)) {}
  __device__ __forceinline__ int passes(int nthreads) const { return (total + UNROLL * nthreads - 1) / (UNROLL * nthreads); }
  __device__ __forceinline__ void load(int pass, int tid, int nthreads) {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int i = (pass * UNROLL + u) * nthreads + tid;
      if (i < total) {
        const int t = i / per_row, c8 = i - t * per_row;
        v[u] = *(const u32x4*)(xrow[t] + 8 * c8);
      }
    }
  }
  __device__ __forceinline__ void store(int pass, int tid, int nthreads) {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int i = (pass * UNROLL + u) * nthreads + tid;
      if (i >= total) continue;
      const int t = i / per_row, c8 = i - t * per_row;
      MT* dst = xs + (size_t)t * cols;
      if constexpr (KIND == Q2_0) {
        const int k0 = 8 * c8, blk = k0 >> 6;
        const XT* vals = (const XT*)&v[u];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          int j, pos = q2_stage_pos((k0 + e) & 63, j);
          const float scale = 1.0f / q2_unit<MT>(j);  // a power of two: exact
          dst[blk * 64 + pos] = (MT)(to_f32(vals[e]) * scale);
        }
      } else {
        *(u32x4*)(dst + 8 * c8) = v[u];
      }
    }
  }
};

// n values from global memory to LDS, every load of a thread's share issued before its stores
template <int U, typename T>
__device__ __forceinline__ void copy_to_lds(T* dst, const T* src, int n, int tid, int nthreads) {
  for (int base = 0; base < n; base += U * nthreads) {
    T v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = base + u * nthreads + tid;
      if (i < n) v[u] = src[i];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = base + u * nthreads + tid;
      if (i < n) dst[i] = v[u];
    }
  }
}

// the token of the A row a lane supplies (4 * TPG if a padding row)
template <int TPG> __device__ __forceinline__ int lane_token() {
  const int n = threadIdx.x & 15;
  return (n & 3) < TPG ? (n >> 2) * TPG + (n & 3) : 4 * TPG;
}

// XStage that also leaves, per scale group of each row, minus the sum the magic-number decode's constant offsets
// add (Q2_0: sum_k (BASE + U_k) xs_k; IQ3_S: sum_k (BASE + 16) x_k) at corr[t * ngroups + group]: the eight (Q2_0) or
// four (IQ3_S) threads of a group hold consecutive vectors and meet by __shfl_xor. nthreads % 64 == 0.
template <int KIND, typename XT, typename MT, int UNROLL> struct XStageCorr {
  static_assert(sizeof(XT) == 2, "16-bit activations");
  const XT* base;
  MT* xs;
  float* corr;
  int cols, per_row, total;
  u32x4 v[UNROLL];

  // row t of the activations at base + t * cols
  __device__ __forceinline__ XStageCorr(MT* xs_, float* corr_, const XT* base_, int n_tok, int cols_)
      : base(base_), xs(xs_), corr(corr_), cols(cols_), per_row(cols_ >> 3), total(n_tok * (cols_ >> 3)) {}
  __device__ __forceinline__ int passes(int nthreads) const { return (total + UNROLL * nthreads - 1) / (UNROLL * nthreads); }
  __device__ __forceinline__ void load(int pass, int tid, int nthreads) {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int i = (pass * UNROLL + u) * nthreads + tid;
      if (i < total) {
        v[u] = *(const u32x4*)(base + 8 * (int64_t)i);  // rows are contiguous: vector i of the block
      }
    }
  }
  __device__ __forceinline__ void store(int pass, int tid, int nthreads) {
    constexpr int SG = KIND == Q2_0 ? 64 : 32, LANES = SG / 8;
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int i = (pass * UNROLL + u) * nthreads + tid;  // i and its group's other vectors: consecutive threads
      float part = 0.0f;
      if (i < total) {
        const int t = i / per_row, c8 = i - t * per_row;
        MT* dst = xs + (size_t)t * cols;
        const XT* vals = (const XT*)&v[u];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int k = 8 * c8 + e;
          if constexpr (KIND == Q2_0) {
            int j;
            const int pos = q2_stage_pos(k & 63, j);
            const MT staged = from_f32<MT>(to_f32(vals[e]) * (1.0f / q2_unit<MT>(j)));
            dst[(k & ~63) + pos] = staged;
            part += (Magic<MT>::BASE + q2_unit<MT>(j)) * to_f32(staged);
          } else {
            dst[k] = vals[e];
            part += (Magic<MT>::BASE + 16.0f) * to_f32(vals[e]);
          }
        }
      }
#pragma unroll
      for (int o = LANES >> 1; o > 0; o >>= 1) part += __shfl_xor(part, o);
      if (i < total && (tid & (LANES - 1)) == 0) {
        const int t = i / per_row, c8 = i - t * per_row;
        corr[t * (cols / SG) + (8 * c8) / SG] = -part;
      }
    }
  }
};

// ---- the tile multiply-accumulate: this wave's share of a 16-row tile's columns, for the block's tokens
//
// wrow0: LDS address of row 0 of the tile (row n at wrow0 + n * rbytes); xs: staged activations (token t at
// xs + t * cols); the wave takes scale groups [g_begin, g_end) (Q2_0 blocks of 64, IQ3_S runs of 32).
template <int KIND, typename MT, int TPG>
__device__ __forceinline__ void tile_mac(const uint8_t* wrow0, int rbytes, const MT* xs, int cols, int n_tok,
                                         int g_begin, int g_end, const uint32_t* stab, float* acc) {
  const int lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
  const int mt = (n & 3) < TPG ? (n >> 2) * TPG + (n & 3) : 4 * TPG;  // token of A row n
  const bool real = mt < n_tok;
  const uint8_t* wrow = wrow0 + (size_t)n * rbytes;
  const MT* xt = xs + (size_t)(real ? mt : 0) * cols;
  const f32x4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
  const u32x4 zfrag = {0u, 0u, 0u, 0u};
  if constexpr (KIND == Q2_0) {
    const u32x4 corr = q2_correction<MT>();
    for (int blk = g_begin; blk < g_end; ++blk) {
      const uint8_t* b = wrow + blk * 18;
      const uint32_t W = (uint32_t)*(const uint16_t*)(b + 2 + 2 * g) | ((uint32_t)*(const uint16_t*)(b + 10 + 2 * g) << 16);
      const float d = half_bits(*(const uint16_t*)b);
      u32x4 fa, fb;
      q2_decode<MT>(W, fa, fb);
      u32x4 xa = real ? *(const u32x4*)(xt + blk * 64 + g * 8) : zfrag;
      u32x4 xb = real ? *(const u32x4*)(xt + blk * 64 + 32 + g * 8) : zfrag;
      f32x4 D = mfma<MT>(xa, corr, zero4);
      D = mfma<MT>(xb, corr, D);
      D = mfma<MT>(xa, fa, D);
      D = mfma<MT>(xb, fb, D);
#pragma unroll
      for (int i = 0; i < TPG; ++i) acc[i] = fmaf(d, D[i], acc[i]);
    }
  } else if constexpr (KIND == IQ3_S) {
    const float cval = -(Magic<MT>::BASE + 16.0f);
    const uint32_t c2 = pack2<MT>(cval, cval);
    const u32x4 corr = {c2, c2, c2, c2};
    constexpr uint32_t hi4 = Magic<MT>::HI * 0x01010101u;
    for (int run = g_begin; run < g_end; ++run) {
      const uint8_t* b = wrow + (run >> 3) * 110;
      const int ib = run & 7;
      const float db = half_bits(*(const uint16_t*)b) * (float)(1 + 2 * (((uint32_t)b[106 + ib / 2] >> (4 * (ib & 1))) & 15u));
      const uint32_t q2 = *(const uint16_t*)(b + 2 + 8 * ib + 2 * g);
      const uint32_t qh = (uint32_t)b[66 + ib] >> (2 * g);
      const uint32_t sg = b[74 + 4 * ib + g];
      const uint32_t i0 = (q2 & 0xffu) | ((qh & 1u) << 8) | ((sg & 15u) << 9);
      const uint32_t i1 = (q2 >> 8) | ((qh & 2u) << 7) | ((sg >> 4) << 9);
      const uint32_t e0 = stab[i0], e1 = stab[i1];
      u32x4 fw;
      fw.x = __builtin_amdgcn_perm(hi4, e0, 0x04010400u);
      fw.y = __builtin_amdgcn_perm(hi4, e0, 0x04030402u);
      fw.z = __builtin_amdgcn_perm(hi4, e1, 0x04010400u);
      fw.w = __builtin_amdgcn_perm(hi4, e1, 0x04030402u);
      u32x4 xa = real ? *(const u32x4*)(xt + run * 32 + g * 8) : zfrag;
      f32x4 D = mfma<MT>(xa, corr, zero4);
      D = mfma<MT>(xa, fw, D);
#pragma unroll
      for (int i = 0; i < TPG; ++i) acc[i] = fmaf(db, D[i], acc[i]);
    }
  }
}

// Where activation k of a row goes in KIND's staged layout, and the factor it is staged with (a power of two):
// Q2_0 permuted and scaled per slot, IQ3_S as it is. A producer that writes its output this way (the route's x,
// gate/up's inner activations) lets the next kernel load its MFMA A fragments straight from memory.
template <int KIND, typename MT> __device__ __forceinline__ int stage_index(int k, float& scale) {
  if constexpr (KIND == Q2_0) {
    int j;
    const int pos = q2_stage_pos(k & 63, j);
    scale = 1.0f / q2_unit<MT>(j);
    return (k & ~63) + pos;
  } else {
    scale = 1.0f;
    return k;
  }
}

// NW weight tiles (16 rows each, row n of tile w at wrow0[w] + n * rbytes, in LDS) against one token's staged row in
// memory (xg, global: L2-resident), CH scale groups at a time: every fragment load of a chunk is issued before its
// MFMAs, and each fragment serves all NW tiles. acc[w][TPG] accumulates tile w.
template <int KIND, typename MT, int TPG, int CH, int NW>
__device__ __forceinline__ void tile_mac_global(const uint8_t* const* wrow0, int rbytes, const MT* xg, bool real,
                                                int g_begin, int g_end, const uint32_t* stab, float (*acc)[TPG]) {
  constexpr int PER = KIND == Q2_0 ? 2 : 1;  // fragments a scale group
  const int lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
  const f32x4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int c0 = g_begin; c0 < g_end; c0 += CH) {
    const int cn = min(CH, g_end - c0);
    u32x4 fr[CH * PER];
#pragma unroll
    for (int i = 0; i < CH * PER; ++i) {
      fr[i] = u32x4{0u, 0u, 0u, 0u};
      if (real && i < cn * PER) {
        const int sg = c0 + i / PER;
        const int at = KIND == Q2_0 ? sg * 64 + (i % PER) * 32 + g * 8 : sg * 32 + g * 8;
        fr[i] = *(const u32x4*)(xg + at);
      }
    }
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const uint8_t* wrow = wrow0[w] + (size_t)n * rbytes;
      if constexpr (KIND == Q2_0) {
        const u32x4 corr = q2_correction<MT>();
#pragma unroll
        for (int i = 0; i < CH; ++i) {
          if (i < cn) {
            const uint8_t* b = wrow + (c0 + i) * 18;
            const uint32_t W = (uint32_t)*(const uint16_t*)(b + 2 + 2 * g) | ((uint32_t)*(const uint16_t*)(b + 10 + 2 * g) << 16);
            const float d = half_bits(*(const uint16_t*)b);
            u32x4 fa, fb;
            q2_decode<MT>(W, fa, fb);
            f32x4 D = mfma<MT>(fr[2 * i], corr, zero4);
            D = mfma<MT>(fr[2 * i + 1], corr, D);
            D = mfma<MT>(fr[2 * i], fa, D);
            D = mfma<MT>(fr[2 * i + 1], fb, D);
#pragma unroll
            for (int t = 0; t < TPG; ++t) acc[w][t] = fmaf(d, D[t], acc[w][t]);
          }
        }
      } else {
        const float cval = -(Magic<MT>::BASE + 16.0f);
        const uint32_t c2 = pack2<MT>(cval, cval);
        const u32x4 corr = {c2, c2, c2, c2};
        constexpr uint32_t hi4 = Magic<MT>::HI * 0x01010101u;
#pragma unroll
        for (int i = 0; i < CH; ++i) {
          if (i < cn) {
            const int run = c0 + i;
            const uint8_t* b = wrow + (run >> 3) * 110;
            const int ib = run & 7;
            const float db = half_bits(*(const uint16_t*)b) * (float)(1 + 2 * (((uint32_t)b[106 + ib / 2] >> (4 * (ib & 1))) & 15u));
            const uint32_t q2 = *(const uint16_t*)(b + 2 + 8 * ib + 2 * g);
            const uint32_t qh = (uint32_t)b[66 + ib] >> (2 * g);
            const uint32_t sg = b[74 + 4 * ib + g];
            const uint32_t e0 = stab[(q2 & 0xffu) | ((qh & 1u) << 8) | ((sg & 15u) << 9)];
            const uint32_t e1 = stab[(q2 >> 8) | ((qh & 2u) << 7) | ((sg >> 4) << 9)];
            u32x4 fw;
            fw.x = __builtin_amdgcn_perm(hi4, e0, 0x04010400u);
            fw.y = __builtin_amdgcn_perm(hi4, e0, 0x04030402u);
            fw.z = __builtin_amdgcn_perm(hi4, e1, 0x04010400u);
            fw.w = __builtin_amdgcn_perm(hi4, e1, 0x04030402u);
            f32x4 D = mfma<MT>(fr[i], corr, zero4);
            D = mfma<MT>(fr[i], fw, D);
#pragma unroll
            for (int t = 0; t < TPG; ++t) acc[w][t] = fmaf(db, D[t], acc[w][t]);
          }
        }
      }
    }
  }
}

// NW weight tiles against one token row of staged activations (xg, in memory) whose offsets' sums were computed
// with the staging (corr: token t's sums at corr_rows + t * ngroups): the accumulator starts at minus the sum, so a
// Q2_0 block takes 2 MFMAs and an IQ3_S run 1. D rows hold tokens g * TPG + t (t < TPG), real below n_tok.
template <int KIND, typename MT, int TPG, int CH, int NW>
__device__ __forceinline__ void tile_mac_staged(const uint8_t* const* wrow0, int rbytes, const MT* xg, bool areal,
                                                const float* corr_rows, int ngroups, int n_tok, int g_begin, int g_end,
                                                const uint32_t* stab, float (*acc)[TPG]) {
  constexpr int PER = KIND == Q2_0 ? 2 : 1;  // fragments a scale group
  const int lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
  for (int c0 = g_begin; c0 < g_end; c0 += CH) {
    const int cn = min(CH, g_end - c0);
    u32x4 fr[CH * PER];
    f32x4 cinit[CH];
#pragma unroll
    for (int i = 0; i < CH * PER; ++i) {
      fr[i] = u32x4{0u, 0u, 0u, 0u};
      if (areal && i < cn * PER) {
        const int sg = c0 + i / PER;
        const int at = KIND == Q2_0 ? sg * 64 + (i % PER) * 32 + g * 8 : sg * 32 + g * 8;
        fr[i] = *(const u32x4*)(xg + at);
      }
    }
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      cinit[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int t = 0; t < TPG; ++t) {
        const int tok = g * TPG + t;
        if (i < cn && tok < n_tok) cinit[i][t] = -corr_rows[(int64_t)tok * ngroups + c0 + i];
      }
    }
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const uint8_t* wrow = wrow0[w] + (size_t)n * rbytes;
      if constexpr (KIND == Q2_0) {
#pragma unroll
        for (int i = 0; i < CH; ++i) {
          if (i < cn) {
            const uint8_t* b = wrow + (c0 + i) * 18;
            const uint32_t W = (uint32_t)*(const uint16_t*)(b + 2 + 2 * g) | ((uint32_t)*(const uint16_t*)(b + 10 + 2 * g) << 16);
            const float d = half_bits(*(const uint16_t*)b);
            u32x4 fa, fb;
            q2_decode<MT>(W, fa, fb);
            f32x4 D = mfma<MT>(fr[2 * i], fa, cinit[i]);
            D = mfma<MT>(fr[2 * i + 1], fb, D);
#pragma unroll
            for (int t = 0; t < TPG; ++t) acc[w][t] = fmaf(d, D[t], acc[w][t]);
          }
        }
      } else {
        constexpr uint32_t hi4 = Magic<MT>::HI * 0x01010101u;
#pragma unroll
        for (int i = 0; i < CH; ++i) {
          if (i < cn) {
            const int run = c0 + i;
            const uint8_t* b = wrow + (run >> 3) * 110;
            const int ib = run & 7;
            const float db = half_bits(*(const uint16_t*)b) * (float)(1 + 2 * (((uint32_t)b[106 + ib / 2] >> (4 * (ib & 1))) & 15u));
            const uint32_t q2 = *(const uint16_t*)(b + 2 + 8 * ib + 2 * g);
            const uint32_t qh = (uint32_t)b[66 + ib] >> (2 * g);
            const uint32_t sg = b[74 + 4 * ib + g];
            const uint32_t e0 = stab[(q2 & 0xffu) | ((qh & 1u) << 8) | ((sg & 15u) << 9)];
            const uint32_t e1 = stab[(q2 >> 8) | ((qh & 2u) << 7) | ((sg >> 4) << 9)];
            u32x4 fw;
            fw.x = __builtin_amdgcn_perm(hi4, e0, 0x04010400u);
            fw.y = __builtin_amdgcn_perm(hi4, e0, 0x04030402u);
            fw.z = __builtin_amdgcn_perm(hi4, e1, 0x04010400u);
            fw.w = __builtin_amdgcn_perm(hi4, e1, 0x04030402u);
            const f32x4 D = mfma<MT>(fr[i], fw, cinit[i]);
#pragma unroll
            for (int t = 0; t < TPG; ++t) acc[w][t] = fmaf(db, D[t], acc[w][t]);
          }
        }
      }
    }
  }
}

// scale groups a chunk of tile_mac_global takes (16 fragments)
template <int KIND> __host__ __device__ constexpr int frag_chunk() { return KIND == Q2_0 ? 8 : 16; }

// scale groups of a row (Q2_0 blocks of 64 weights, IQ3_S runs of 32)
template <int KIND> __host__ __device__ constexpr int scale_group() { return KIND == Q2_0 ? 64 : 32; }

template <int KIND> __host__ __device__ constexpr bool mfma_kind() { return KIND == Q2_0 || KIND == IQ3_S; }

// ---- wave reductions on DPP (no LDS round trip): the result is valid in lane 63, broadcast by readlane

__device__ __forceinline__ uint32_t dpp_max_step(uint32_t v, uint32_t moved) { return v > moved ? v : moved; }

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = dpp_max_step(v, __builtin_amdgcn_update_dpp(v, v, 0xb1, 0xf, 0xf, false));   // quad_perm [1,0,3,2]
  v = dpp_max_step(v, __builtin_amdgcn_update_dpp(v, v, 0x4e, 0xf, 0xf, false));   // quad_perm [2,3,0,1]
  v = dpp_max_step(v, __builtin_amdgcn_update_dpp(v, v, 0x141, 0xf, 0xf, false));  // row_half_mirror
  v = dpp_max_step(v, __builtin_amdgcn_update_dpp(v, v, 0x140, 0xf, 0xf, false));  // row_mirror
  v = dpp_max_step(v, __builtin_amdgcn_update_dpp(v, v, 0x142, 0xa, 0xf, false));  // row_bcast:15
  v = dpp_max_step(v, __builtin_amdgcn_update_dpp(v, v, 0x143, 0xc, 0xf, false));  // row_bcast:31
  return __builtin_amdgcn_readlane(v, 63);
}

template <int CTRL, int ROW_MASK> __device__ __forceinline__ uint64_t dpp_max64(uint64_t v) {
  const uint32_t hi = (uint32_t)(v >> 32), lo = (uint32_t)v;
  const uint32_t ohi = __builtin_amdgcn_update_dpp(hi, hi, CTRL, ROW_MASK, 0xf, false);
  const uint32_t olo = __builtin_amdgcn_update_dpp(lo, lo, CTRL, ROW_MASK, 0xf, false);
  const uint64_t o = ((uint64_t)ohi << 32) | olo;
  return o > v ? o : v;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  v = dpp_max64<0xb1, 0xf>(v);
  v = dpp_max64<0x4e, 0xf>(v);
  v = dpp_max64<0x141, 0xf>(v);
  v = dpp_max64<0x140, 0xf>(v);
  v = dpp_max64<0x142, 0xa>(v);
  v = dpp_max64<0x143, 0xc>(v);
  const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(v >> 32), 63), lo = __builtin_amdgcn_readlane((uint32_t)v, 63);
  return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ float wave_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, 0.0f), __builtin_bit_cast(int, v), 0xb1, 0xf, 0xf, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, 0.0f), __builtin_bit_cast(int, v), 0x4e, 0xf, 0xf, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, 0.0f), __builtin_bit_cast(int, v), 0x141, 0xf, 0xf, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, 0.0f), __builtin_bit_cast(int, v), 0x140, 0xf, 0xf, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, 0.0f), __builtin_bit_cast(int, v), 0x142, 0xa, 0xf, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, 0.0f), __builtin_bit_cast(int, v), 0x143, 0xc, 0xf, false));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

}  // namespace sh
