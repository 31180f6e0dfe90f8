// Lane-per-block decode arithmetic shared by the decode GEMV kernels (mxa_gemv_lpb.hip,
// mxa_gemv_flow.hip): lane i of a wave computes one whole packed 256-value block, read from LDS,
// against the Q8_K activations of up to MAXM rows (float activations for IQ4_XS), giving one
// float block value per activation row. The per-row fold of those values in block order is the
// oracle's fused steps, so every kernel built on this equals the oracle bit for bit (IQ4_XS:
// within tolerance, one summation order in every kernel).
#pragma once

#include "mxa_device.hpp"

#pragma clang fp contract(off)

namespace mxa {
namespace {

constexpr int kWaveLanes = 64;
constexpr int kActPad = 16;  // LDS bytes of padding after each staged 256-value activation block

typedef __attribute__((address_space(3))) void lds_void;

template <int TYPE>
struct Lpb;

// Block arithmetic on float activations for the K-quants and Q8_0 (the fp32-activation GEMV: x is
// not quantized to Q8_K): the type ids with this flag added.
constexpr int kF32Act = 0x100;
constexpr int T_Q8_0_F = T_Q8_0 | kF32Act, T_Q4_K_F = T_Q4_K | kF32Act, T_Q6_K_F = T_Q6_K | kF32Act;

// How a block type's activations sit in LDS: Q8_K (256 int8 + padding; bsums and the scale
// separately), or floats (256 fp32 + padding) for IQ4_XS and the fp32-activation types, which
// also keep the sixteen sums of 16 consecutive activations after the floats.
template <int TYPE>
struct ActTraits {
  static constexpr bool kFloat = TYPE == T_IQ4_XS || (TYPE & kF32Act) != 0;
  static constexpr bool kSums = (TYPE & kF32Act) != 0;
  static constexpr int kBlk = kFloat ? QK * 4 + (kSums ? 64 : 0) + kActPad : QK + kActPad;
};

// NW dwords of LDS from byte `off` of the 4-byte aligned `base` (off 2-byte aligned at worst).
// LDS addresses stay base + integer offset in every kernel using these: an LDS pointer that passes
// through an integer cast becomes a flat pointer, and flat loads are counted by vmcnt too.
template <int NW>
__device__ __forceinline__ void lds_words(const uint8_t* base, int off, uint32_t* w) {
  const uint32_t* p = (const uint32_t*)(base + (off & ~3));
  const uint32_t sh = (uint32_t)(off & 3);
  uint32_t raw[NW + 1];
#pragma unroll
  for (int i = 0; i < NW + 1; ++i) raw[i] = p[i];
#pragma unroll
  for (int i = 0; i < NW; ++i) w[i] = __builtin_amdgcn_alignbyte(raw[i + 1], raw[i], sh);
}

// Activations of one 256-value block of row m in LDS: q8 values, 16 bsums (or 256 floats, and for
// the fp32-activation types the sums of their 16 runs of 16).
struct ActBlock {
  const int8_t* q;
  const int16_t* bsums;
  float d;
  const float* x;
  __device__ i32x4a4 q16(int off) const { return *(const i32x4a4*)(q + off); }  // q8[off .. off + 15]
  __device__ u32x4a4 bs8(int h) const { return *(const u32x4a4*)(bsums + 8 * h); }  // bsums 8h .. 8h + 7
  __device__ uint32_t bs2(int j) const { return *(const uint32_t*)(bsums + 2 * j); }  // bsums 2j, 2j + 1
  __device__ float4 x4(int off) const { return *(const float4*)(x + off); }
  __device__ float4 s4(int c) const { return *(const float4*)(x + QK + 4 * c); }  // sums 4c .. 4c + 3
  __device__ float s1(int j) const { return x[QK + j]; }                           // sum j
};

// The same block held in registers (one activation row): the arrays are only ever indexed with
// constants once the compute loops are unrolled.
struct ActRegs {
  i32x4a4 q[16];
  u32x4a4 bs[2];
  __device__ i32x4a4 q16(int off) const { return q[off >> 4]; }
  __device__ u32x4a4 bs8(int h) const { return bs[h]; }
  __device__ uint32_t bs2(int j) const { return bs[j >> 2][j & 3]; }
  __device__ float4 x4(int) const { return float4{0.0f, 0.0f, 0.0f, 0.0f}; }
};

template <>
struct Lpb<T_Q4_K> {
  static constexpr int kBytes = 144;
  static constexpr bool kHasD = false;
  // value: fmaf(d, sumi, -(dmin * summ))   (mx_dot_k_ssse3.c:150-154)
  template <int MAXM, class A>
  __device__ static void compute(const uint8_t* wb, int off, const A* a, int M, float* V, float& D) {
    const uint8_t* blk = wb + off;  // 4-byte aligned
    const u32x4a4 h = *(const u32x4a4*)blk;
    uint32_t q[32];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const u32x4a4 v = *(const u32x4a4*)(blk + 16 + 16 * i);
      q[4 * i] = v.x, q[4 * i + 1] = v.y, q[4 * i + 2] = v.z, q[4 * i + 3] = v.w;
    }
    const float d = half_to_float(h.x), dmin = half_to_float(h.x >> 16);
    const K4Scales s = k4_scales(h.y, h.z, h.w);
#pragma unroll
    for (int m = 0; m < MAXM; ++m) {
      if (m < M) {
        // X[sb]: sum of the 32 activations of sub-block sb (its two 16-value bsums)
        const u32x4a4 b0 = a[m].bs8(0), b1 = a[m].bs8(1);
        const uint32_t bw[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
        int X[8];
#pragma unroll
        for (int sb = 0; sb < 8; ++sb) X[sb] = (int)(int16_t)(bw[sb] & 0xFFFFu) + (int)(int16_t)(bw[sb] >> 16);
        // High nibbles h as signed bytes 16 h - 128 ((w & 0xF0) ^ 0x80, one bit operation):
        // sum(h * x) = (sum((16 h - 128) * x) + 128 X) / 16, exactly. 16 * sumi stays below 2^29.
        int sumi16 = 0, summ = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          int lo = 0, hs = 0;
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            const i32x4a4 xl = a[m].q16(64 * c + 16 * i);
            const i32x4a4 xh = a[m].q16(64 * c + 32 + 16 * i);
            const int xlv[4] = {xl.x, xl.y, xl.z, xl.w}, xhv[4] = {xh.x, xh.y, xh.z, xh.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              const uint32_t w = q[8 * c + 4 * i + k];
              lo = sdot4(w & 0x0F0F0F0Fu, (uint32_t)xlv[k], lo);
              hs = sdot4((w & 0xF0F0F0F0u) ^ 0x80808080u, (uint32_t)xhv[k], hs);
            }
          }
          // 24-bit multiplies (full rate): |lo| < 2^16, |hs + 128 X| < 2^20, scales < 64
          sumi16 += 16 * __mul24((int)k4_pick(s.sc_lo, s.sc_hi, 2 * c), lo) +
                    __mul24((int)k4_pick(s.sc_lo, s.sc_hi, 2 * c + 1), hs + 128 * X[2 * c + 1]);
        }
        const int sumi = sumi16 >> 4;  // exact: a multiple of 16
#pragma unroll
        for (int sb = 0; sb < 8; ++sb) summ += (int)k4_pick(s.mn_lo, s.mn_hi, sb) * X[sb];
        V[m] = fmaf(d, (float)sumi, -(dmin * (float)summ));
      }
    }
    D = 0.0f;
  }
  __device__ static float fold(float acc, float xd, float v, float) { return fmaf(xd, v, acc); }
};

template <>
struct Lpb<T_Q6_K> {
  static constexpr int kBytes = 210;
  static constexpr bool kHasD = true;
  // value: sumi = sum_s sc_s * sum((u - 32) * q8); fold (y.d * d) * sumi   (mx_dot_k_ssse3.c:167-209)
  template <int MAXM, class A>
  __device__ static void compute(const uint8_t* wb, int off, const A* a, int M, float* V, float& D) {
    uint32_t w[53];  // bytes 0..211: ql 0..127, qh 128..191, scales 192..207, d 208..209
    lds_words<53>(wb, off, w);
    int sumi[MAXM];
#pragma unroll
    for (int m = 0; m < MAXM; ++m) sumi[m] = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        uint32_t U[8];  // codes u = q + 32 of elements 128h + 32g + 4i .. +3
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t l = w[16 * h + ((g & 1) ? 8 : 0) + i], qh = w[32 + 8 * h + i];
          U[i] = g == 0 ? q6_codes<0>(l, qh) : g == 1 ? q6_codes<1>(l, qh)
               : g == 2 ? q6_codes<2>(l, qh) : q6_codes<3>(l, qh);
        }
#pragma unroll
        for (int m = 0; m < MAXM; ++m) {
          if (m < M) {
            const uint32_t bwd = a[m].bs2(4 * h + g);
#pragma unroll
            for (int half16 = 0; half16 < 2; ++half16) {  // sub-block 8h + 2g + half16
              const i32x4a4 x = a[m].q16(128 * h + 32 * g + 16 * half16);
              int sdot = 0;
              sdot = sdot4(U[4 * half16 + 0], (uint32_t)x.x, sdot);
              sdot = sdot4(U[4 * half16 + 1], (uint32_t)x.y, sdot);
              sdot = sdot4(U[4 * half16 + 2], (uint32_t)x.z, sdot);
              sdot = sdot4(U[4 * half16 + 3], (uint32_t)x.w, sdot);
              const int sbi = 8 * h + 2 * g + half16;
              const int sc = (int)(int8_t)(uint8_t)(w[48 + (sbi >> 2)] >> (8 * (sbi & 3)));
              const int bs = half16 ? (int)(int16_t)(bwd >> 16) : (int)(int16_t)(bwd & 0xFFFFu);
              sumi[m] += __mul24(sc, sdot - 32 * bs);  // |sc| < 2^7, |sdot - 32 bs| < 2^18
            }
          }
        }
      }
#pragma unroll
    for (int m = 0; m < MAXM; ++m) V[m] = (float)sumi[m];
    D = half_to_float(w[52]);
  }
  __device__ static float fold(float acc, float xd, float v, float d) { return fmaf(xd * d, v, acc); }
};

template <>
struct Lpb<T_Q8_0> {
  static constexpr int kBytes = 272;  // eight 34-byte blocks
  static constexpr bool kHasD = false;
  // value: block_sum = sum_k d_k * sum(qs * q8) in k order (mx_dot_q8_0.c:8-18)
  template <int MAXM, class A>
  __device__ static void compute(const uint8_t* wb, int off, const A* a, int M, float* V, float& D) {
    const uint8_t* blk = wb + off;  // 4-byte aligned
    float bs[MAXM];
#pragma unroll
    for (int m = 0; m < MAXM; ++m) bs[m] = 0.0f;
#pragma unroll
    for (int pr = 0; pr < 4; ++pr) {  // pairs of 34-byte blocks: 68 bytes, 17 words
      uint32_t w[17];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const u32x4a4 v = *(const u32x4a4*)(blk + 68 * pr + 16 * i);
        w[4 * i] = v.x, w[4 * i + 1] = v.y, w[4 * i + 2] = v.z, w[4 * i + 3] = v.w;
      }
      w[16] = *(const uint32_t*)(blk + 68 * pr + 64);
#pragma unroll
      for (int e = 0; e < 2; ++e) {  // block k = 2pr + e: d then 32 qs
        const int k = 2 * pr + e;
        const float dk = e == 0 ? half_to_float(w[0]) : half_to_float(w[8] >> 16);
        uint32_t qs[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          qs[i] = e == 0 ? __builtin_amdgcn_alignbyte(w[i + 1], w[i], 2) : w[9 + i];
#pragma unroll
        for (int m = 0; m < MAXM; ++m) {
          if (m < M) {
            const i32x4a4 x0 = a[m].q16(32 * k);
            const i32x4a4 x1 = a[m].q16(32 * k + 16);
            int p = 0;
            p = sdot4(qs[0], (uint32_t)x0.x, p);
            p = sdot4(qs[1], (uint32_t)x0.y, p);
            p = sdot4(qs[2], (uint32_t)x0.z, p);
            p = sdot4(qs[3], (uint32_t)x0.w, p);
            p = sdot4(qs[4], (uint32_t)x1.x, p);
            p = sdot4(qs[5], (uint32_t)x1.y, p);
            p = sdot4(qs[6], (uint32_t)x1.z, p);
            p = sdot4(qs[7], (uint32_t)x1.w, p);
            bs[m] = fmaf(dk, (float)p, bs[m]);
          }
        }
      }
    }
#pragma unroll
    for (int m = 0; m < MAXM; ++m) V[m] = bs[m];
    D = 0.0f;
  }
  __device__ static float fold(float acc, float xd, float v, float) { return fmaf(xd, v, acc); }
};

template <>
struct Lpb<T_IQ4_XS> {
  static constexpr int kBytes = 136;
  static constexpr bool kHasD = false;
  // value: sum over sub-blocks of dl * sum(x * grid) (mx_dot_f32.c:42-55 up to float order), in
  // the order every IQ4_XS kernel here uses, so a token's result does not depend on the batch:
  // p = sequential fmaf over a sub-block's 16 low-nibble / 16 high-nibble elements four at a
  // time, quarters fmaf(dl1, p1, dl0 * p0), block (q0 + q1) + (q2 + q3), rows sum blocks in order
  template <int MAXM, class A>
  __device__ static void compute(const uint8_t* wb, int off, const A* a, int M, float* V, float& D) {
    const uint8_t* blk = wb + off;  // 4-byte aligned
    uint32_t w[34];
#pragma unroll
    for (int i = 0; i < 17; ++i) {
      const u32x2a4 v = *(const u32x2a4*)(blk + 8 * i);
      w[2 * i] = v.x, w[2 * i + 1] = v.y;
    }
    const float d = half_to_float(w[0]);
    const uint32_t sh = w[0] >> 16, sl = w[1];
    float dl[8];
#pragma unroll
    for (int ib = 0; ib < 8; ++ib) {
      const int ls = (int)(((sl >> (4 * ib)) & 15u) | (((sh >> (2 * ib)) & 3u) << 4));
      dl[ib] = d * (float)(ls - 32);
    }
#pragma unroll
    for (int m = 0; m < MAXM; ++m) {
      if (m < M) {
        float L[4];  // 64-element quarters: fmaf(dl[2j+1], p[2j+1], dl[2j] * p[2j])
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float p[2];
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            const int ib = 2 * j + t;
            p[t] = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const uint32_t qw = w[2 + 4 * ib + i];
              const uint32_t gl = iq4_lookup4(qw & 0x0F0F0F0Fu), gh = iq4_lookup4((qw >> 4) & 0x0F0F0F0Fu);
              const float4 xl = a[m].x4(32 * ib + 4 * i);
              const float4 xh = a[m].x4(32 * ib + 16 + 4 * i);
              p[t] = fmaf(xl.x, sbyte_f<0>(gl), p[t]);
              p[t] = fmaf(xl.y, sbyte_f<1>(gl), p[t]);
              p[t] = fmaf(xl.z, sbyte_f<2>(gl), p[t]);
              p[t] = fmaf(xl.w, sbyte_f<3>(gl), p[t]);
              p[t] = fmaf(xh.x, sbyte_f<0>(gh), p[t]);
              p[t] = fmaf(xh.y, sbyte_f<1>(gh), p[t]);
              p[t] = fmaf(xh.z, sbyte_f<2>(gh), p[t]);
              p[t] = fmaf(xh.w, sbyte_f<3>(gh), p[t]);
            }
          }
          L[j] = fmaf(dl[2 * j + 1], p[1], dl[2 * j] * p[0]);
        }
        V[m] = (L[0] + L[1]) + (L[2] + L[3]);
      }
    }
    D = 0.0f;
  }
  __device__ static float fold(float acc, float, float v, float) { return acc + v; }
};


// ------------------------------------------------------------------ fp32 activations
// The decode GEMV on float activations for the K-quants and Q8_0, the device counterpart of the
// reference's fp32-activation GEMVs (app/gguf/dequant/quantized_gemv.py:51-180,
// quantized_gemv_legacy.py:167-194): every weight value is d * sc * q (minus dmin * m for Q4_K) in
// float and meets an unquantized activation. A sub-block's terms factor as
// (d * sc) * sum(x * q) - (dmin * m) * sum(x): the codes q become floats exactly (one conversion
// per value), sum(x * q) is a chain of fmaf over the sub-block in element order, and sum(x) comes
// from the sums of 16 activations staged with them (the same for every row). The block value
// sums its sub-block terms pairwise; rows add block values in order. Float rounding differs from
// the reference's fastmath order; results are held to the float64 product within tolerance.

template <int K>
__device__ __forceinline__ float ubyte_f(uint32_t w) {
  return (float)((w >> (8 * K)) & 0xFFu);
}

// p + x . (four unsigned bytes of w as floats), in element order
__device__ __forceinline__ float dot4_f(float4 x, uint32_t w, float p) {
  p = fmaf(x.x, ubyte_f<0>(w), p);
  p = fmaf(x.y, ubyte_f<1>(w), p);
  p = fmaf(x.z, ubyte_f<2>(w), p);
  return fmaf(x.w, ubyte_f<3>(w), p);
}

template <>
struct Lpb<T_Q4_K_F> {
  static constexpr int kBytes = 144;
  static constexpr bool kHasD = false;
  // sub-block sb: (d * sc_sb) * sum(x * q) - (dmin * m_sb) * sum(x); high nibbles are taken as
  // 16 q (one bit operation), whose exact factor 1/16 goes into their scale. The block's codes
  // are read 32 bytes (two sub-blocks) at a time and met by every row before the next 32: with
  // the whole block held across rows, two or more rows spill at the pipelined kernel's budget.
  template <int MAXM, class A>
  __device__ static void compute(const uint8_t* wb, int off, const A* a, int M, float* V, float& D) {
    const uint8_t* blk = wb + off;  // 4-byte aligned
    const u32x4a4 h = *(const u32x4a4*)blk;
    const float d = half_to_float(h.x), dmin = half_to_float(h.x >> 16);
    const K4Scales s = k4_scales(h.y, h.z, h.w);
    float t[MAXM][8];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      uint32_t q[8];
      const u32x4a4 v0 = *(const u32x4a4*)(blk + 16 + 32 * c);
      const u32x4a4 v1 = *(const u32x4a4*)(blk + 32 + 32 * c);
      q[0] = v0.x, q[1] = v0.y, q[2] = v0.z, q[3] = v0.w;
      q[4] = v1.x, q[5] = v1.y, q[6] = v1.z, q[7] = v1.w;
      const float d1 = d * (float)k4_pick(s.sc_lo, s.sc_hi, 2 * c);
      const float m1 = dmin * (float)k4_pick(s.mn_lo, s.mn_hi, 2 * c);
      const float d2 = (d * (float)k4_pick(s.sc_lo, s.sc_hi, 2 * c + 1)) * 0.0625f;
      const float m2 = dmin * (float)k4_pick(s.mn_lo, s.mn_hi, 2 * c + 1);
#pragma unroll
      for (int m = 0; m < MAXM; ++m) {
        if (m < M) {
          float plo = 0.0f, phi = 0.0f;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            plo = dot4_f(a[m].x4(64 * c + 4 * i), q[i] & 0x0F0F0F0Fu, plo);
            phi = dot4_f(a[m].x4(64 * c + 32 + 4 * i), q[i] & 0xF0F0F0F0u, phi);
          }
          const float4 sx = a[m].s4(c);  // sums of elements 64c .. 64c + 63, 16 at a time
          t[m][2 * c] = fmaf(d1, plo, -(m1 * (sx.x + sx.y)));
          t[m][2 * c + 1] = fmaf(d2, phi, -(m2 * (sx.z + sx.w)));
        }
      }
    }
#pragma unroll
    for (int m = 0; m < MAXM; ++m)
      if (m < M)
        V[m] = ((t[m][0] + t[m][1]) + (t[m][2] + t[m][3])) + ((t[m][4] + t[m][5]) + (t[m][6] + t[m][7]));
    D = 0.0f;
  }
  __device__ static float fold(float acc, float, float v, float) { return acc + v; }
};

template <>
struct Lpb<T_Q6_K_F> {
  static constexpr int kBytes = 210;
  static constexpr bool kHasD = false;
  // sub-block sb of 16: (d * sc_sb) * (sum(x * u) - 32 sum(x)), u = q + 32 the stored code
  template <int MAXM, class A>
  __device__ static void compute(const uint8_t* wb, int off, const A* a, int M, float* V, float& D) {
    uint32_t w[53];  // bytes 0..211: ql 0..127, qh 128..191, scales 192..207, d 208..209
    lds_words<53>(wb, off, w);
    const float d = half_to_float(w[52]);
    float r[MAXM][8];  // sums of sub-block pairs 2i, 2i + 1
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        uint32_t U[8];  // codes of elements 128h + 32g + 4i .. +3
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t l = w[16 * h + ((g & 1) ? 8 : 0) + i], qh = w[32 + 8 * h + i];
          U[i] = g == 0 ? q6_codes<0>(l, qh) : g == 1 ? q6_codes<1>(l, qh)
               : g == 2 ? q6_codes<2>(l, qh) : q6_codes<3>(l, qh);
        }
        const int sb = 8 * h + 2 * g;  // sub-blocks sb, sb + 1
        const float dsc0 = d * (float)(int)(int8_t)(uint8_t)(w[48 + (sb >> 2)] >> (8 * (sb & 3)));
        const float dsc1 = d * (float)(int)(int8_t)(uint8_t)(w[48 + (sb >> 2)] >> (8 * (sb & 3) + 8));
#pragma unroll
        for (int m = 0; m < MAXM; ++m) {
          if (m < M) {
            float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              p0 = dot4_f(a[m].x4(128 * h + 32 * g + 4 * i), U[i], p0);
              p1 = dot4_f(a[m].x4(128 * h + 32 * g + 16 + 4 * i), U[4 + i], p1);
            }
            r[m][4 * h + g] = dsc0 * fmaf(-32.0f, a[m].s1(sb), p0) + dsc1 * fmaf(-32.0f, a[m].s1(sb + 1), p1);
          }
        }
      }
#pragma unroll
    for (int m = 0; m < MAXM; ++m)
      if (m < M) V[m] = ((r[m][0] + r[m][1]) + (r[m][2] + r[m][3])) + ((r[m][4] + r[m][5]) + (r[m][6] + r[m][7]));
    D = 0.0f;
  }
  __device__ static float fold(float acc, float, float v, float) { return acc + v; }
};

template <>
struct Lpb<T_Q8_0_F> {
  static constexpr int kBytes = 272;  // eight 34-byte blocks
  static constexpr bool kHasD = false;
  // block k of 32: d_k * (sum(x * (q + 128)) - 128 sum(x)), the signed codes taken as unsigned
  // bytes q + 128 (one bit operation)
  template <int MAXM, class A>
  __device__ static void compute(const uint8_t* wb, int off, const A* a, int M, float* V, float& D) {
    const uint8_t* blk = wb + off;  // 4-byte aligned
    float t[MAXM][8];
#pragma unroll
    for (int pr = 0; pr < 4; ++pr) {  // pairs of 34-byte blocks: 68 bytes, 17 words
      uint32_t w[17];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const u32x4a4 v = *(const u32x4a4*)(blk + 68 * pr + 16 * i);
        w[4 * i] = v.x, w[4 * i + 1] = v.y, w[4 * i + 2] = v.z, w[4 * i + 3] = v.w;
      }
      w[16] = *(const uint32_t*)(blk + 68 * pr + 64);
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int k = 2 * pr + e;
        const float dk = e == 0 ? half_to_float(w[0]) : half_to_float(w[8] >> 16);
        uint32_t qs[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          qs[i] = (e == 0 ? __builtin_amdgcn_alignbyte(w[i + 1], w[i], 2) : w[9 + i]) ^ 0x80808080u;
#pragma unroll
        for (int m = 0; m < MAXM; ++m) {
          if (m < M) {
            float p = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) p = dot4_f(a[m].x4(32 * k + 4 * i), qs[i], p);
            t[m][k] = dk * fmaf(-128.0f, a[m].s1(2 * k) + a[m].s1(2 * k + 1), p);
          }
        }
      }
    }
#pragma unroll
    for (int m = 0; m < MAXM; ++m)
      if (m < M) V[m] = ((t[m][0] + t[m][1]) + (t[m][2] + t[m][3])) + ((t[m][4] + t[m][5]) + (t[m][6] + t[m][7]));
    D = 0.0f;
  }
  __device__ static float fold(float acc, float, float v, float) { return acc + v; }
};

}  // namespace
}  // namespace mxa
