// Streaming matvec of every block kind with float32 sums of exact weights: out[m][t] = W_m . x[m][t] for a stack
// of n_mats matrices and up to 8 tokens each (one matrix is strata-mlx's window matvec, strata_mlx/blocks.py:
// 351-394: a window of T <= 8 tokens, each run unpacked once for all of them). Serves float32 activations and the
// kinds the MFMA kernels do not decode, for one layer (sh_window_matvec) and for a stack (sh_stack_matvec).
//
// Arithmetic: the generic kernels' own (blocks.hip k_window_matvec): P lanes share a row, lane `part` takes the
// runs part, part + P, ... in order, each run's 32 weights decoded exactly (decode.h unpack32) and dotted with the
// token's 32 activations in order, the P lanes' sums met by a butterfly: their bits for the codebook kinds. The
// kinds with a scale a run (or half run) take it, and the offset, out of the sums, with roundings of the same size:
// Q2_0 d (sum q x - sum x) (q the codes 0..3 converted a byte at a time, sum x the run's activations summed once a
// matrix): two VALU instructions a weight and a token instead of four; IQ4_NL / IQ4_XS dl sum kv[q] x; Q3_K
// s (sum (q + 4h) x - 4 sum x) a half run. Where the bytes come from differs too:
//   - persistent blocks of 256 threads each take a contiguous run of items (tile_rows rows of one matrix); an
//     item's bytes, contiguous in the stack, are read with 16-byte loads (all 256 threads, consecutive chunks:
//     fully coalesced) into registers while the item before is multiplied, then written to LDS;
//   - the activations of a block's current matrix sit in LDS as they are (the element type), a run of 32 at a
//     stride padded by 16 bytes, so the lanes of a wave reading 64 different runs with 16-byte reads fall in
//     distinct banks; each activation is read from LDS, never again from memory;
//   - the kind's codebook tables are in LDS (static).
#include <algorithm>
#include <type_traits>

#include "decode.h"
#include "launch.h"

namespace sh {

constexpr int SM_NT = 256;                          // threads a block
constexpr int SM_LOADS = 4;                         // 16-byte loads a thread an item, at most
constexpr int SM_TILE = SM_LOADS * SM_NT * 16;      // LDS bytes of an item's buffer (16 KiB)
constexpr int SM_X_MAX = 96 * 1024;                 // LDS bytes the activations of a matrix may take

// one launch's shape, shared by host and device through the kernel arguments
struct StreamPlan {
  int rows, cols, tokens, runs, P, rp;  // rp = 256 / P rows a pass of the block
  int64_t rbytes, mat_bytes;
  int tile_rows, items_per_mat;
  int64_t items, per;                   // items of the stack; a block's
  int x_stride, x_bytes, xsum_bytes;    // LDS bytes a run of activations; of a matrix's; of its runs' sums
  int loads;                            // 16-byte loads a thread an item
};

// Q2_0's code values (0..3) of a run as floats, in weight order: weight 4i + j is bits 2j, 2j + 1 of code byte i.
// Four bytes are masked at once a code position and each byte converted as it stands (the empty statement keeps
// the compiler from folding mask and byte into a bit-field extract a weight).
__device__ __forceinline__ void q2_codes(const uint8_t* q, float* c) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t word = rd32(q + 4 * h);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t m = (word >> (2 * j)) & 0x03030303u;
      asm("" : "+v"(m));
#pragma unroll
      for (int i = 0; i < 4; ++i) c[4 * (4 * h + i) + j] = (float)((m >> (8 * i)) & 0xffu);
    }
  }
}

// float32 dot of a run's 32 weights with 32 activations read from LDS as 16-byte vectors (dot32's order)
template <typename XT> __device__ __forceinline__ float dot32_lds(const float* w, const uint8_t* xr) {
  constexpr int NV = 32 * (int)sizeof(XT) / 16;
  u32x4 v[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) v[i] = *(const u32x4*)(xr + 16 * i);
  return dot32<XT>(w, (const XT*)v);
}

// the same as two dots of 16 (the run's halves), each in order
template <typename XT> __device__ __forceinline__ void dot32h_lds(const float* w, const uint8_t* xr, float& a0,
                                                                  float& a1) {
  constexpr int NV = 32 * (int)sizeof(XT) / 16;
  u32x4 v[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) v[i] = *(const u32x4*)(xr + 16 * i);
  const XT* x = (const XT*)v;
  a0 = 0.0f, a1 = 0.0f;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    a0 = fmaf(w[j], to_f32(x[j]), a0);
    a1 = fmaf(w[16 + j], to_f32(x[16 + j]), a1);
  }
}

// activations a sum of the staging covers, for the kinds whose runs subtract an offset times them: Q2_0 a run,
// Q3_K half a run (one scale each); 0: none
template <int KIND> constexpr int stream_sum_group() { return KIND == Q2_0 ? 32 : KIND == Q3_K ? 16 : 0; }

// Matrix m is the stack's m-th with activations x[m]; or, for pairs (one token each, activations x[m / share]),
// expert idx[m] of the stack (a pair naming no expert, outside [0, n_experts), gets zeros) or the buffer
// experts[m]. An expert buffer need not start on 16 bytes: its first chunk is read from the 16 bytes holding its
// first byte, inside the allocation it lies in (allocations start on 256 bytes).
template <int KIND, typename XT, int TM>
__global__ __launch_bounds__(SM_NT) void k_stream_mv(const uint8_t* __restrict__ blocks, StreamPlan S,
                                                     const XT* __restrict__ x, XT* __restrict__ out,
                                                     const uint8_t* __restrict__ tabs, const int32_t* __restrict__ idx,
                                                     int n_experts, int share,
                                                     const uint8_t* const* __restrict__ experts) {
  __shared__ u32x4 tab4[lds_tab_bytes(KIND) / 16];
  extern __shared__ u32x4 dyn[];
  uint8_t* tab = (uint8_t*)tab4;
  uint8_t* xl = (uint8_t*)dyn;              // the current matrix's activations: [token][run], x_stride bytes a run
  float* xsum = (float*)((uint8_t*)dyn + S.x_bytes);  // sums of activations [token][run][32 / SUMG]
  uint8_t* tl = (uint8_t*)dyn + S.x_bytes + S.xsum_bytes;  // the item's bytes from the 16-byte chunk holding its first
  const int tid = threadIdx.x;
  const int64_t first = (int64_t)blockIdx.x * S.per, last = min(S.items, first + S.per);
  if (first >= last) return;  // the whole block
  stage_tables<KIND>(tab, tabs);

  // an item: rows [r0, r0 + nr) of matrix m, bytes [a, a + nr * rbytes) read from a16 = a rounded down to 16
  // (inside the stack: the stack starts 16-byte aligned): `nfull` whole chunks by 16-byte loads, the `ntail`
  // bytes after them one a thread
  struct Span {
    int64_t m;
    int r0, nr, lead, nfull, ntail;
    bool valid;  // the matrix exists (a pair's expert in range): else no loads, zeros out
    const uint8_t* a16;
  };
  auto span = [&](int64_t item) {
    Span s;
    s.m = item / S.items_per_mat;
    s.r0 = (int)(item - s.m * S.items_per_mat) * S.tile_rows;
    s.nr = min(S.tile_rows, S.rows - s.r0);
    int64_t mat = s.m;
    s.valid = true;
    if (idx) {
      const int e = idx[s.m];
      s.valid = e >= 0 && e < n_experts;
      mat = s.valid ? e : 0;
    }
    if (experts) {
      const uint8_t* a = experts[s.m] + (int64_t)s.r0 * S.rbytes;
      s.a16 = (const uint8_t*)((uintptr_t)a & ~(uintptr_t)15);
      s.lead = (int)(a - s.a16);
    } else {
      const int64_t off = mat * S.mat_bytes + (int64_t)s.r0 * S.rbytes;
      s.a16 = blocks + (off & ~(int64_t)15);  // from the kernel argument: global loads
      s.lead = (int)(off & 15);
    }
    const int n = s.valid ? s.lead + s.nr * (int)S.rbytes : 0;
    s.nfull = n >> 4;
    s.ntail = n & 15;
    return s;
  };
  u32x4 stg[SM_LOADS];
  uint32_t stail = 0;
  auto issue = [&](const Span& s) {
#pragma unroll
    for (int j = 0; j < SM_LOADS; ++j) {
      const int c = j * SM_NT + tid;
      if (j < S.loads && c < s.nfull) stg[j] = *(const u32x4*)(s.a16 + 16 * c);
    }
    if (tid < s.ntail) stail = s.a16[16 * s.nfull + tid];
  };
  auto commit = [&](const Span& s) {
#pragma unroll
    for (int j = 0; j < SM_LOADS; ++j) {
      const int c = j * SM_NT + tid;
      if (j < S.loads && c < s.nfull) *(u32x4*)(tl + 16 * c) = stg[j];
    }
    if (tid < s.ntail) tl[16 * s.nfull + tid] = (uint8_t)stail;
  };
  // matrix m's activations into LDS: x[m] is [tokens][cols], so 16-byte vector v lies in run (t * runs + n)
  auto stage_x = [&](int64_t m) {
    constexpr int RB = 32 * (int)sizeof(XT), SUMG = stream_sum_group<KIND>();
    const uint8_t* xs = (const uint8_t*)(x + m / share * S.tokens * S.cols);
    const int nv = S.tokens * S.cols * (int)sizeof(XT) / 16;
    for (int v0 = 0; v0 < nv; v0 += SM_NT) {  // every lane the same rounds (the sums' lane exchanges)
      const int v = v0 + tid;
      const bool in = v < nv;
      const int tr = (16 * v) / RB, o = 16 * v - tr * RB;
      u32x4 xv = {0u, 0u, 0u, 0u};
      if (in) {
        xv = *(const u32x4*)(xs + 16 * v);
        *(u32x4*)(xl + tr * S.x_stride + o) = xv;
      }
      if constexpr (SUMG > 0) {
        // the sums of SUMG activations (a run, or half one): each lane its vector's elements in order, then the
        // group's NL lanes (consecutive, an aligned group: nv is whole runs) by a butterfly
        constexpr int NE = 16 / (int)sizeof(XT), NL = SUMG / NE;
        const XT* e = (const XT*)&xv;
        float p = 0.0f;
#pragma unroll
        for (int i = 0; i < NE; ++i) p += to_f32(e[i]);
#pragma unroll
        for (int o2 = NL / 2; o2 > 0; o2 >>= 1) p += __shfl_xor(p, o2);
        if (in && v % NL == 0) xsum[v / NL] = p;
      }
    }
  };

  const int part = tid & (S.P - 1), rin = tid / S.P;
  int64_t cur = -1;
  issue(span(first));
  for (int64_t item = first; item < last; ++item) {
    const Span s = span(item);
    __syncthreads();  // every wave is done with the item before (and with its activations)
    commit(s);
    if (s.m != cur) {
      stage_x(s.m);
      cur = s.m;
    }
    if (item + 1 < last) issue(span(item + 1));  // in flight while this item is multiplied
    __syncthreads();
    for (int r0 = 0; r0 < s.nr; r0 += S.rp) {  // passes: every lane the same (the sums' lane exchanges)
      const int r = r0 + rin;
      const bool act = r < s.nr && s.valid;  // the P lanes of a row alike
      const uint8_t* row = tl + s.lead + (int64_t)r * S.rbytes;
      float w[32], sum[TM];
#pragma unroll
      for (int t = 0; t < TM; ++t) sum[t] = 0.0f;
      for (int n = act ? part : S.runs; n < S.runs; n += S.P) {
        if constexpr (KIND == Q2_0) {  // d (sum q x - sum x): the scale and the offset once a run
          const uint8_t* b = row + (n >> 1) * 18;
          const float d = half_at(b);
          q2_codes(b + 2 + 8 * (n & 1), w);
#pragma unroll
          for (int t = 0; t < TM; ++t)
            if (t < S.tokens)
              sum[t] += d * (dot32_lds<XT>(w, xl + (t * S.runs + n) * S.x_stride) - xsum[t * S.runs + n]);
        } else if constexpr (KIND == IQ4_NL || KIND == IQ4_XS) {  // the scale once a run: dl sum kv[q] x
          const uint8_t* q;
          float dl;
          if constexpr (KIND == IQ4_NL) {
            q = row + n * 18 + 2;
            dl = half_at(q - 2);
          } else {
            const uint8_t* b = row + (n >> 3) * 136;
            const int ib = n & 7;
            const uint32_t ls = (((uint32_t)b[4 + ib / 2] >> (4 * (ib & 1))) & 15u) | (((rd16(b + 2) >> (2 * ib)) & 3u) << 4);
            dl = half_at(b) * ((float)ls - 32.0f);
            q = b + 8 + 16 * ib;
          }
          const int8_t* kv = (const int8_t*)tab;
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const uint32_t c = q[i];
            w[i] = (float)kv[c & 15];
            w[16 + i] = (float)kv[c >> 4];
          }
#pragma unroll
          for (int t = 0; t < TM; ++t)
            if (t < S.tokens) sum[t] += dl * dot32_lds<XT>(w, xl + (t * S.runs + n) * S.x_stride);
        } else if constexpr (KIND == Q3_K) {  // two scales of 16: s (sum (q + 4h) x - 4 sum x) each
          const uint8_t* b = row + (n >> 3) * 110;
          const int r = n & 7, shift = 2 * (r & 3);
          const uint8_t* q = b + 32 + 32 * (r >> 2);
          const float d = half_at(b + 108);
          const float s0 = d * q3k_scale(b + 96, 2 * r), s1 = d * q3k_scale(b + 96, 2 * r + 1);
#pragma unroll
          for (int k = 0; k < 8; ++k) {  // weights 4k .. 4k + 3: (q >> shift & 3) | (h >> r & 1) << 2, 0..7
            uint32_t m = ((rd32(q + 4 * k) >> shift) & 0x03030303u) | (((rd32(b + 4 * k) >> r) & 0x01010101u) << 2);
            asm("" : "+v"(m));
#pragma unroll
            for (int i = 0; i < 4; ++i) w[4 * k + i] = (float)((m >> (8 * i)) & 0xffu);
          }
#pragma unroll
          for (int t = 0; t < TM; ++t) {
            if (t < S.tokens) {
              float a0, a1;
              dot32h_lds<XT>(w, xl + (t * S.runs + n) * S.x_stride, a0, a1);
              const float* xs2 = xsum + 2 * (t * S.runs + n);
              sum[t] += s0 * (a0 - 4.0f * xs2[0]) + s1 * (a1 - 4.0f * xs2[1]);
            }
          }
        } else {
          unpack32<KIND>(row, n, w, tab);
#pragma unroll
          for (int t = 0; t < TM; ++t)
            if (t < S.tokens) sum[t] += dot32_lds<XT>(w, xl + (t * S.runs + n) * S.x_stride);
        }
      }
#pragma unroll
      for (int t = 0; t < TM; ++t) {
        if (t < S.tokens) {
          const float total = lanes_sum(sum[t], S.P);
          if (r < s.nr && part == 0) out[(s.m * S.tokens + t) * S.rows + s.r0 + r] = from_f32<XT>(total);
        }
      }
    }
  }
}

// The plan for n_mats matrices of rows x cols of `kind` and `tokens` activations of `x_dtype`; E_UNSUPPORTED where
// the kernel does not take them (the callers then take another kernel or refuse).
static int stream_plan(int kind, int x_dtype, const void* blocks, const void* x, int64_t n_mats, int64_t rows,
                       int64_t cols, int64_t tokens, StreamPlan& S) {
  if (tokens < 1 || tokens > 8) return fail(E_UNSUPPORTED, "stream matvec: %lld tokens (1 to 8)", (long long)tokens);
  if (((uintptr_t)blocks & 15) || ((uintptr_t)x & 15))  // (blocks NULL: pairs bringing their own buffers)
    return fail(E_UNSUPPORTED, "stream matvec: blocks and activations must be 16-byte aligned");
  const int64_t runs = cols / 32, rb = row_bytes(kind, cols), xs = 32 * dtype_size(x_dtype) + 16;
  if (tokens * runs * xs > SM_X_MAX)
    return fail(E_UNSUPPORTED, "stream matvec: %lld tokens of %lld activations do not fit LDS", (long long)tokens,
                (long long)cols);
  const int P = lanes_per_row(runs), rp = SM_NT / P;
  const int64_t fit = (SM_TILE - 32) / rb / rp * rp;  // rows an item's buffer holds, whole passes
  if (fit < rp) return fail(E_UNSUPPORTED, "stream matvec: rows of %lld bytes too long", (long long)rb);
  if (n_mats * rows * rb > (1ll << 62) || rows > (1 << 30))
    return fail(E_SHAPE, "stream matvec: stack too large");
  // items small enough that a single matrix spreads over the CUs twice, at most what the buffer holds
  const int64_t want = std::max<int64_t>(rp, n_mats * rows / (2 * device_cus()) / rp * rp);
  S.rows = (int)rows, S.cols = (int)cols, S.tokens = (int)tokens, S.runs = (int)runs, S.P = P, S.rp = rp;
  S.rbytes = rb, S.mat_bytes = rows * rb;
  S.tile_rows = (int)std::min(fit, want);
  S.items_per_mat = (int)((rows + S.tile_rows - 1) / S.tile_rows);
  S.items = n_mats * S.items_per_mat;
  S.x_stride = (int)xs, S.x_bytes = (int)(tokens * runs * xs);
  const int sums = kind == Q2_0 ? 1 : kind == Q3_K ? 2 : 0;  // a run's (stream_sum_group)
  S.xsum_bytes = (int)((tokens * runs * sums * 4 + 15) & ~15ll);
  const int64_t nmax = (15 + (int64_t)S.tile_rows * rb) / 16;  // whole chunks of an item, at most
  S.loads = (int)((nmax + SM_NT - 1) / SM_NT);
  return OK;
}

template <int KIND, typename XT, int TM>
static int launch_stream(const StreamPlan& S0, const uint8_t* blocks, const uint8_t* tabs, const XT* x, XT* out,
                         hipStream_t stream, bool dry, const int32_t* idx, int n_experts, int share,
                         const uint8_t* const* experts) {
  StreamPlan S = S0;
  auto kern = k_stream_mv<KIND, XT, TM>;
  const size_t dyn_lds = (size_t)S.x_bytes + S.xsum_bytes + SM_TILE;
  const size_t lds = dyn_lds + static_lds(kern);
  if (lds > LDS_BYTES) return fail(E_UNSUPPORTED, "stream matvec: %zu bytes of LDS", lds);
  if (dry) return OK;
  const int64_t bpc = std::max<int64_t>(1, std::min<int64_t>(8, (int64_t)LDS_BYTES / (int64_t)lds));
  const int64_t cap = (int64_t)device_cus() * bpc;
  S.per = (S.items + cap - 1) / cap;
  const int64_t grid = (S.items + S.per - 1) / S.per;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(SM_NT), dyn_lds, stream, blocks, S, x, out, tabs, idx,
                     n_experts, share, experts);
  return check_launch("stream matvec");
}

// the streaming matvec's checks, plan and launch (dry: checks and plan only); E_UNSUPPORTED where it does not take
// the arguments. With idx, the n_mats "matrices" are pairs: pair m multiplies expert idx[m] of the stack's
// n_experts by x[m / share] (one token a pair).
int stream_matvec(bool dry, int kind, const void* blocks, const void* tables, int64_t n_mats, int64_t rows,
                  int64_t cols, const void* x, int x_dtype, int64_t tokens, void* out, void* stream,
                  const int32_t* idx, int64_t n_experts, int64_t share, const void* const* experts) {
  int st = check_rows(kind, rows, cols, "stream matvec");
  if (st) return st;
  if ((!blocks && !experts) || !x || (!out && !dry) || (needs_tables(kind) && !tables))
    return fail(E_ARG, "stream matvec: null pointer");
  if ((idx || experts) && (tokens != 1 || share < 1 || n_experts < 0 || n_experts > (1ll << 31) - 1))
    return fail(E_UNSUPPORTED, "stream matvec: pairs of %lld tokens, share %lld", (long long)tokens,
                (long long)share);
  StreamPlan S;
  st = stream_plan(kind, x_dtype, blocks, x, n_mats, rows, cols, tokens, S);
  if (st) return st;
  return with_kind(kind, [&](auto kc) {
    constexpr int K = decltype(kc)::value;
    return with_dtype(x_dtype, [&](auto* tp) {
      using XT = std::remove_pointer_t<decltype(tp)>;
      if (tokens == 1)
        return launch_stream<K, XT, 1>(S, (const uint8_t*)blocks, (const uint8_t*)tables, (const XT*)x, (XT*)out,
                                       (hipStream_t)stream, dry, idx, (int)n_experts, (int)share,
                                       (const uint8_t* const*)experts);
      return launch_stream<K, XT, 8>(S, (const uint8_t*)blocks, (const uint8_t*)tables, (const XT*)x, (XT*)out,
                                     (hipStream_t)stream, dry, idx, (int)n_experts, (int)share,
                                       (const uint8_t* const*)experts);
    });
  });
}

// ---- dequantize: every weight of a tensor of rows as a float of OutT (strata_mlx/blocks.py:397-404), the same
// memory path: an item's rows come in as 16-byte loads into LDS (the next item's into registers meanwhile), each
// lane decodes runs of 32 from LDS (unpack32, the generic kernel's values) into an LDS output tile at a padded run
// stride (16-byte writes in distinct banks), and the tile, contiguous in the output, leaves as consecutive
// 16-byte stores of all 256 threads.

constexpr int DQ_OUT = 32 * 1024;  // LDS bytes of an item's output rows (before padding)

struct DequantPlan {
  int64_t rows;  // rows of the whole tensor
  int cols, runs, tile_rows, loads;
  int64_t rbytes, items, per;
  int in_bytes;  // LDS bytes of the input buffer
};

template <int KIND, typename OT>
__global__ __launch_bounds__(SM_NT) void k_dequant_stream(const uint8_t* __restrict__ blocks, DequantPlan S,
                                                          OT* __restrict__ out, const uint8_t* __restrict__ tabs) {
  constexpr int RUN = 32 * (int)sizeof(OT), RSTR = RUN + 16, CPR = RUN / 16;  // a run's output bytes, stride, chunks
  __shared__ u32x4 tab4[lds_tab_bytes(KIND) / 16];
  extern __shared__ u32x4 dyn[];
  uint8_t* tab = (uint8_t*)tab4;
  uint8_t* tl = (uint8_t*)dyn;                // the item's bytes from the 16-byte chunk holding its first
  uint8_t* ol = (uint8_t*)dyn + S.in_bytes;   // its output runs, RSTR bytes apart
  const int tid = threadIdx.x;
  const int64_t first = (int64_t)blockIdx.x * S.per, last = min(S.items, first + S.per);
  if (first >= last) return;  // the whole block
  stage_tables<KIND>(tab, tabs);
  struct Span {
    int64_t r0;
    int nr, lead, nfull, ntail;
    const uint8_t* a16;
  };
  auto span = [&](int64_t item) {
    Span s;
    s.r0 = item * S.tile_rows;
    s.nr = (int)min((int64_t)S.tile_rows, S.rows - s.r0);
    const int64_t off = s.r0 * S.rbytes;
    s.a16 = blocks + (off & ~(int64_t)15);
    s.lead = (int)(off & 15);
    const int n = s.lead + s.nr * (int)S.rbytes;
    s.nfull = n >> 4;
    s.ntail = n & 15;
    return s;
  };
  u32x4 stg[SM_LOADS];
  uint32_t stail = 0;
  auto issue = [&](const Span& s) {
#pragma unroll
    for (int j = 0; j < SM_LOADS; ++j) {
      const int c = j * SM_NT + tid;
      if (j < S.loads && c < s.nfull) stg[j] = *(const u32x4*)(s.a16 + 16 * c);
    }
    if (tid < s.ntail) stail = s.a16[16 * s.nfull + tid];
  };
  issue(span(first));
  for (int64_t item = first; item < last; ++item) {
    const Span s = span(item);
    __syncthreads();  // every wave is done with the item before (its input and output tiles)
#pragma unroll
    for (int j = 0; j < SM_LOADS; ++j) {
      const int c = j * SM_NT + tid;
      if (j < S.loads && c < s.nfull) *(u32x4*)(tl + 16 * c) = stg[j];
    }
    if (tid < s.ntail) tl[16 * s.nfull + tid] = (uint8_t)stail;
    if (item + 1 < last) issue(span(item + 1));
    __syncthreads();
    const int nruns = s.nr * S.runs;
    for (int q = tid; q < nruns; q += SM_NT) {
      const int r = q / S.runs, n = q - r * S.runs;
      float w[32];
      unpack32<KIND>(tl + s.lead + (int64_t)r * S.rbytes, n, w, tab);
      OT o[32];
#pragma unroll
      for (int j = 0; j < 32; ++j) o[j] = from_f32<OT>(w[j]);
#pragma unroll
      for (int c = 0; c < CPR; ++c) *(u32x4*)(ol + q * RSTR + 16 * c) = ((const u32x4*)o)[c];
    }
    __syncthreads();
    uint8_t* dst = (uint8_t*)(out + s.r0 * S.cols);
    const int nch = nruns * CPR;
    for (int c = tid; c < nch; c += SM_NT) {
      const int q = c / CPR;
      *(u32x4*)(dst + 16 * c) = *(const u32x4*)(ol + q * RSTR + 16 * (c - q * CPR));
    }
  }
}

// dequantize by the stream: E_UNSUPPORTED where it does not take the tensor (the caller takes the generic kernel)
int dequant_stream(int kind, const void* blocks, const void* tables, int64_t rows, int64_t cols, void* out,
                   int out_dtype, void* stream) {
  if (((uintptr_t)blocks & 15) || ((uintptr_t)out & 15))
    return fail(E_UNSUPPORTED, "dequantize stream: blocks and output must be 16-byte aligned");
  const int64_t rb = row_bytes(kind, cols), ob = cols * dtype_size(out_dtype);
  const int64_t fit = std::min<int64_t>((SM_TILE - 32) / rb, DQ_OUT / ob);
  if (fit < 1) return fail(E_UNSUPPORTED, "dequantize stream: rows of %lld weights too long", (long long)cols);
  DequantPlan S;
  S.rows = rows, S.cols = (int)cols, S.runs = (int)(cols / 32), S.rbytes = rb;
  S.tile_rows = (int)std::min(fit, std::max<int64_t>(1, rows / (2 * device_cus())));
  S.items = (rows + S.tile_rows - 1) / S.tile_rows;
  S.loads = (int)(((15 + (int64_t)S.tile_rows * rb) / 16 + SM_NT - 1) / SM_NT);
  S.in_bytes = SM_TILE;
  return with_kind(kind, [&](auto kc) {
    constexpr int K = decltype(kc)::value;
    return with_dtype(out_dtype, [&](auto* tp) {
      using OT = std::remove_pointer_t<decltype(tp)>;
      auto kern = k_dequant_stream<K, OT>;
      const size_t dyn_lds = (size_t)SM_TILE + (size_t)S.tile_rows * S.runs * (32 * sizeof(OT) + 16);
      const size_t lds = dyn_lds + static_lds(kern);
      if (lds > LDS_BYTES) return fail(E_UNSUPPORTED, "dequantize stream: %zu bytes of LDS", lds);
      const int64_t bpc = std::max<int64_t>(1, std::min<int64_t>(8, (int64_t)LDS_BYTES / (int64_t)lds));
      const int64_t cap = (int64_t)device_cus() * bpc;
      DequantPlan P = S;
      P.per = (S.items + cap - 1) / cap;
      const int64_t grid = (S.items + P.per - 1) / P.per;
      hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(SM_NT), dyn_lds, (hipStream_t)stream, (const uint8_t*)blocks,
                         P, (OT*)out, (const uint8_t*)tables);
      return check_launch("dequantize");
    });
  });
}

}  // namespace sh
