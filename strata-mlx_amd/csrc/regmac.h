// Register-resident activations for the MFMA decode of Q2_0 / IQ3_S rows staged in LDS: a wave's activation
// fragments for its scale groups, and minus the sums the magic-number decode's offsets add, are loaded once (per
// matrix, per group of tokens) into registers; the multiply then reads only weight bytes from LDS. Used by the
// streaming stack matvec (stack.hip) and the fused MoE decode (moe.hip).
#pragma once

#include <type_traits>

#include "xmv.h"

namespace sh {

// Loop-invariant decode constants held in VGPRs: a gfx9 VOP3 instruction takes no literal, so with the masks and
// the magic in registers each pair of Q2_0 weights is one v_and_or_b32.
struct DecodeRegs {
  uint32_t m0, m1, m2, magic;
};
__device__ __forceinline__ uint32_t vreg(uint32_t c) {
  uint32_t r;
  asm("v_mov_b32 %0, %1" : "=v"(r) : "s"(c));
  return r;
}
template <int KIND, typename MT> __device__ __forceinline__ DecodeRegs decode_regs() {
  DecodeRegs r;
  if constexpr (KIND == Q2_0) {
    r.m0 = vreg(0x00030003u);
    r.m1 = vreg(0x000C000Cu);
    r.m2 = vreg(0x00300030u);
    r.magic = vreg(Magic<MT>::M2);
  } else {
    r.m0 = r.m1 = r.m2 = 0;
    r.magic = vreg(Magic<MT>::HI * 0x01010101u);
  }
  return r;
}

// a wave's activation fragments for its GPER scale groups (A operand: lane (g, n) holds row n = its token's
// fragment g), and minus the offsets' sums for the TPG tokens of its D-rows
template <int KIND, int TPG, int GPER> struct XRegs {
  u32x4 xa[GPER];
  u32x4 xb[KIND == Q2_0 ? GPER : 1];
  float nc[GPER][TPG];
};

// A wave's activation row loads for its GPER scale groups as they lie (lane g: Q2_0 values 8g..8g+7 and
// 32+8g..32+8g+7 of each block, IQ3_S values 8g..8g+7 of each run), issued by x_issue and turned into XRegs by
// x_finish: a caller can put other loads in flight between the two.
template <int KIND, int GPER> struct XRaw {
  u32x4 v[GPER][KIND == Q2_0 ? 2 : 1];
};

template <int KIND, typename XT, int GPER>
__device__ __forceinline__ void x_issue(XRaw<KIND, GPER>& R, const XT* xr, int gbase) {
  const int g = (threadIdx.x & 63) >> 4;
#pragma unroll
  for (int j = 0; j < GPER; ++j) {
    if constexpr (KIND == Q2_0) {
      R.v[j][0] = *(const u32x4*)(xr + (gbase + j) * 64 + 8 * g);
      R.v[j][1] = *(const u32x4*)(xr + (gbase + j) * 64 + 32 + 8 * g);
    } else {
      R.v[j][0] = *(const u32x4*)(xr + (gbase + j) * 32 + 8 * g);
    }
  }
}

// the same loads of row `row` of `base` (row length `len`) written by other blocks of the launch (ld_agent16)
template <int KIND, typename XT, int GPER>
__device__ __forceinline__ void x_issue_agent(XRaw<KIND, GPER>& R, const XT* base, int row, int len, int gbase) {
  const int g = (threadIdx.x & 63) >> 4;
  const uint32_t r0 = (uint32_t)row * len * sizeof(XT);
#pragma unroll
  for (int j = 0; j < GPER; ++j) {
    if constexpr (KIND == Q2_0) {
      R.v[j][0] = ld_agent16(base, r0 + ((gbase + j) * 64 + 8 * g) * sizeof(XT));
      R.v[j][1] = ld_agent16(base, r0 + ((gbase + j) * 64 + 32 + 8 * g) * sizeof(XT));
    } else {
      R.v[j][0] = ld_agent16(base, r0 + ((gbase + j) * 32 + 8 * g) * sizeof(XT));
    }
  }
}

// minus each group's offset sum for the TPG tokens of the lane's D-rows: the lane's share, added over the four
// lanes of a row (xor 16, 32), then fetched from a lane whose A-row is the wanted token (lane 4g + t holds token
// g * TPG + t)
template <int TPG, int GPER>
__device__ __forceinline__ void x_sums(float (&nc)[GPER][TPG], const float (&part)[GPER]) {
  const int g = (threadIdx.x & 63) >> 4;
#pragma unroll
  for (int j = 0; j < GPER; ++j) {
    float p = part[j];
    p += __shfl_xor(p, 16);
    p += __shfl_xor(p, 32);
#pragma unroll
    for (int t = 0; t < TPG; ++t) nc[j][t] = -__shfl(p, 4 * g + t);
  }
}

// XRegs from raw loads, activations as they are: Q2_0 lane g's fragment a takes block-local weights
// k = 32h + 8g + 4a + j (j < 4, h < 2) into slot 2j + h (for item_mac's RAW decode, which shifts each code down to
// bit 0); IQ3_S the run's values 8g..8g+7
template <int KIND, typename XT, int TPG, int GPER>
__device__ __forceinline__ void x_finish(XRegs<KIND, TPG, GPER>& X, const XRaw<KIND, GPER>& R) {
  using MT = XT;
  float part[GPER];
#pragma unroll
  for (int j = 0; j < GPER; ++j) {
    if constexpr (KIND == Q2_0) {
      // slot 2j + h of fragment a: x[32h + 8g + 4a + j], so each dword pairs a half of v[j][0] with the same half
      // of v[j][1]
      const uint32_t a0[4] = {R.v[j][0].x, R.v[j][0].y, R.v[j][0].z, R.v[j][0].w};
      const uint32_t a1[4] = {R.v[j][1].x, R.v[j][1].y, R.v[j][1].z, R.v[j][1].w};
      X.xa[j] = u32x4{__builtin_amdgcn_perm(a1[0], a0[0], 0x05040100u), __builtin_amdgcn_perm(a1[0], a0[0], 0x07060302u),
                      __builtin_amdgcn_perm(a1[1], a0[1], 0x05040100u), __builtin_amdgcn_perm(a1[1], a0[1], 0x07060302u)};
      X.xb[j] = u32x4{__builtin_amdgcn_perm(a1[2], a0[2], 0x05040100u), __builtin_amdgcn_perm(a1[2], a0[2], 0x07060302u),
                      __builtin_amdgcn_perm(a1[3], a0[3], 0x05040100u), __builtin_amdgcn_perm(a1[3], a0[3], 0x07060302u)};
      const XT* h0 = (const XT*)&R.v[j][0];
      const XT* h1 = (const XT*)&R.v[j][1];
      float p = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) p += to_f32(h0[i]) + to_f32(h1[i]);
      part[j] = (Magic<MT>::BASE + 1.0f) * p;
    } else {
      X.xa[j] = R.v[j][0];
      const XT* e = (const XT*)&R.v[j][0];
      float p = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) p += to_f32(e[i]);
      part[j] = (Magic<MT>::BASE + 16.0f) * p;
    }
  }
  x_sums<TPG, GPER>(X.nc, part);
}

// XRegs for scale groups [gbase, gbase + GPER) of the lane's activation row xr (the row of its A-row token).
// Q2_0: lane g's fragment a takes block-local weights k = 32h + 8g + 4a + j (j < 4, h < 2) into slot 2j + h, scaled
// by 1 / U_j (the in-place mask's unit), as XStage stages them, or as they are with RAW (x_finish); IQ3_S: values
// 8g..8g+7 of the run as they are.
template <int KIND, typename XT, int TPG, int GPER, bool RAW = false>
__device__ __forceinline__ void load_x_row(XRegs<KIND, TPG, GPER>& X, const XT* xr, int gbase) {
  using MT = XT;
  if constexpr (KIND != Q2_0 || RAW) {
    XRaw<KIND, GPER> R;
    x_issue<KIND, XT, GPER>(R, xr, gbase);
    x_finish<KIND, XT, TPG, GPER>(X, R);
  } else {
    const int lane = threadIdx.x & 63, g = lane >> 4;
    float part[GPER];
    u32x4 v[GPER][2];
#pragma unroll
    for (int j = 0; j < GPER; ++j) {
      v[j][0] = *(const u32x4*)(xr + (gbase + j) * 64 + 8 * g);
      v[j][1] = *(const u32x4*)(xr + (gbase + j) * 64 + 32 + 8 * g);
    }
#pragma unroll
    for (int j = 0; j < GPER; ++j) {
      const XT* h0 = (const XT*)&v[j][0];
      const XT* h1 = (const XT*)&v[j][1];
      float p = 0.0f;
      uint32_t w[2][4];
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const float inv = 1.0f / q2_unit<MT>(jj);  // a power of two: exact
          const MT s0 = from_f32<MT>(to_f32(h0[4 * a + jj]) * inv);
          const MT s1 = from_f32<MT>(to_f32(h1[4 * a + jj]) * inv);
          p += (Magic<MT>::BASE + q2_unit<MT>(jj)) * (to_f32(s0) + to_f32(s1));
          w[a][jj] = (uint32_t)__builtin_bit_cast(uint16_t, s0) | ((uint32_t)__builtin_bit_cast(uint16_t, s1) << 16);
        }
      X.xa[j] = u32x4{w[0][0], w[0][1], w[0][2], w[0][3]};
      X.xb[j] = u32x4{w[1][0], w[1][1], w[1][2], w[1][3]};
      part[j] = p;
    }
    x_sums<TPG, GPER>(X.nc, part);
  }
}

// load_x_row for a matrix's n_tok tokens at xm + t * cols; padding A-rows read token 0
template <int KIND, typename XT, int TPG, int GPER>
__device__ __forceinline__ void load_x(XRegs<KIND, TPG, GPER>& X, const XT* xm, int cols, int n_tok, int gbase) {
  int mt = lane_token<TPG>();
  mt = mt < n_tok ? mt : 0;
  load_x_row<KIND, XT, TPG, GPER>(X, xm + (size_t)mt * cols, gbase);
}

// one wave's item: its 16 rows (row n at wrow0 + n * rstride, already advanced to the wave's first group) x its
// GPER groups. All LDS reads are issued up front; a group's scale is applied to its accumulator chain (two
// chains, in turn) after the other chain's MFMAs. The D-rows past TPG are padding rows: their accumulators keep
// whatever the chain left and are never used. RAW (Q2_0): every code shifted down to bits 0-1 before its mask, for
// activations as they are (load_x_row's RAW form).
template <int KIND, typename MT, int TPG, int GPER, bool RAW = false>
__device__ __forceinline__ void item_mac(const uint8_t* wrow0, int rstride, const XRegs<KIND, TPG, GPER>& X,
                                         const uint32_t* stab, const DecodeRegs& k, float* acc) {
  const int lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
  const uint8_t* wrow = wrow0 + (size_t)n * rstride;
  uint32_t w0[GPER], w1[GPER], dh[GPER], sc[GPER];
  if constexpr (KIND == Q2_0) {
#pragma unroll
    for (int j = 0; j < GPER; ++j) {
      const uint8_t* b = wrow + j * 18;
      w0[j] = *(const uint16_t*)(b + 2 + 2 * g);
      w1[j] = *(const uint16_t*)(b + 10 + 2 * g);
      dh[j] = *(const uint16_t*)b;
    }
  } else {
    static_assert(KIND != IQ3_S || GPER % 8 == 0, "IQ3_S: whole superblocks a wave");
    // a superblock's header once: its eight high-bit bytes as two words, its four scale bytes as one
    uint32_t q2[GPER], sg[GPER], qd[GPER / 4];
#pragma unroll
    for (int j = 0; j < GPER; ++j) {
      const uint8_t* b = wrow + (j >> 3) * 110;
      const int ib = j & 7;
      q2[j] = *(const uint16_t*)(b + 2 + 8 * ib + 2 * g);
      sg[j] = b[74 + 4 * ib + g];
      if (ib % 4 == 0)
        qd[j / 4] = (uint32_t)b[66 + ib] | ((uint32_t)b[67 + ib] << 8) | ((uint32_t)b[68 + ib] << 16) |
                    ((uint32_t)b[69 + ib] << 24);
      if (ib == 0) {
        dh[j] = *(const uint16_t*)b;
        sc[j] = (uint32_t)b[106] | ((uint32_t)b[107] << 8) | ((uint32_t)b[108] << 16) | ((uint32_t)b[109] << 24);
      }
    }
    // The two grid indices of run j, (low byte | high bit << 8 | sign nibble << 9), built side by side as the two
    // halves of one word: the high bits of four runs spread to bit 0 of a byte each (E: the first index's, O: the
    // second's), a byte permute picks run j's pair, the sign nibbles go to bits 1-4 of their bytes, and a second
    // permute interleaves those bytes with the low bytes.
#pragma unroll
    for (int j4 = 0; j4 < GPER / 4; ++j4) {
      const uint32_t qs = qd[j4] >> (2 * g);
      const uint32_t E = qs & 0x01010101u, O = (qs >> 1) & 0x01010101u;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = 4 * j4 + r;
        const uint32_t hr = __builtin_amdgcn_perm(O, E, 0x0c0c0000u | ((uint32_t)(4 + r) << 8) | (uint32_t)r);
        const uint32_t t = (((sg[j] << 1) | (sg[j] << 5)) & 0x1e1eu) | hr;
        const uint32_t w = __builtin_amdgcn_perm(t, q2[j], 0x05010400u);
        w0[j] = stab[w & 0xffffu];
        w1[j] = stab[w >> 16];
      }
    }
  }
  f32x4 D[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
  float dprev = 0.0f;
#pragma unroll
  for (int j = 0; j < GPER; ++j) {
    f32x4& Dj = D[j & 1];
#pragma unroll
    for (int t = 0; t < TPG; ++t) Dj[t] = X.nc[j][t];
    if constexpr (KIND == Q2_0 && RAW) {
      const uint32_t W = w0[j] | (w1[j] << 16);
      u32x4 fa, fb;
      fa.x = (W & k.m0) | k.magic;
      fa.y = ((W >> 2) & k.m0) | k.magic;
      fa.z = ((W >> 4) & k.m0) | k.magic;
      fa.w = ((W >> 6) & k.m0) | k.magic;
      fb.x = ((W >> 8) & k.m0) | k.magic;
      fb.y = ((W >> 10) & k.m0) | k.magic;
      fb.z = ((W >> 12) & k.m0) | k.magic;
      fb.w = ((W >> 14) & k.m0) | k.magic;
      Dj = mfma<MT>(X.xa[j], fa, Dj);
      Dj = mfma<MT>(X.xb[j], fb, Dj);
    } else if constexpr (KIND == Q2_0) {
      const uint32_t W = w0[j] | (w1[j] << 16), W8 = W >> 8;
      u32x4 fa, fb;
      fa.x = (W & k.m0) | k.magic;
      fa.y = (W & k.m1) | k.magic;
      fa.z = (W & k.m2) | k.magic;
      fb.x = (W8 & k.m0) | k.magic;
      fb.y = (W8 & k.m1) | k.magic;
      fb.z = (W8 & k.m2) | k.magic;
      if constexpr (std::is_same_v<MT, bf16>) {  // bit 7 of a bf16 half is exponent: code 3 shifted down
        fa.w = ((W >> 6) & k.m0) | k.magic;
        fb.w = ((W >> 14) & k.m0) | k.magic;
      } else {
        fa.w = (W & (k.m2 << 2)) | k.magic;
        fb.w = (W8 & (k.m2 << 2)) | k.magic;
      }
      Dj = mfma<MT>(X.xa[j], fa, Dj);
      Dj = mfma<MT>(X.xb[j], fb, Dj);
    } else {
      u32x4 fw;
      fw.x = __builtin_amdgcn_perm(k.magic, w0[j], 0x04010400u);
      fw.y = __builtin_amdgcn_perm(k.magic, w0[j], 0x04030402u);
      fw.z = __builtin_amdgcn_perm(k.magic, w1[j], 0x04010400u);
      fw.w = __builtin_amdgcn_perm(k.magic, w1[j], 0x04030402u);
      Dj = mfma<MT>(X.xa[j], fw, Dj);
    }
    if (j > 0) {  // the previous group, on the other chain
#pragma unroll
      for (int t = 0; t < TPG; ++t) acc[t] = fmaf(dprev, D[(j - 1) & 1][t], acc[t]);
    }
    if constexpr (KIND == Q2_0) {
      dprev = half_bits(dh[j]);
    } else {
      // 1 + 2 x the run's scale nibble: the superblock's four scale bytes turned into those values for the even
      // runs (low nibbles) and the odd runs (high nibbles), a byte each
      const int ib = j & 7;
      const uint32_t s4 = sc[j & ~7];
      const uint32_t odd = ib & 1 ? (s4 >> 3) & 0x1e1e1e1eu : (s4 << 1) & 0x1e1e1e1eu;
      dprev = half_bits(dh[j & ~7]) * (float)(((odd | 0x01010101u) >> (8 * (ib >> 1))) & 0xffu);
    }
  }
#pragma unroll
  for (int t = 0; t < TPG; ++t) acc[t] = fmaf(dprev, D[(GPER - 1) & 1][t], acc[t]);
}

}  // namespace sh
