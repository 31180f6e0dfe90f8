// Matrix-core operand builders for packed weight tiles (Q4_K / Q6_K / Q8_0), shared by the
// batched kernels.
//
// Operands of v_mfma_i32_16x16x64_i8: A (16 activation rows m x 64 k), B (64 k x 16 weight rows n)
// built in registers from the packed bytes. Lane l supplies row (l % 16) and k-group g = l / 16 of
// both; its output holds n = l % 16 and m = 4 g + i (i < 4). The k-group / MFMA t assignment of the
// 256 values of a block differs per type and is chosen so that every lane-group slice of an MFMA
// lies inside one scale sub-block:
//   Q4_K  (8 sub-blocks of 32): lane group g, MFMA t: elements 64 g + 16 t + (0..15). The scale is
//         folded into B exactly as two int8 planes, (sc >> 3) * u and (sc & 7) * u (both <= 105),
//         8 * plane_hi + plane_lo; the min term sum(min * bsums) is one fp16 MFMA (exact).
//   Q6_K  (16 sub-blocks of 16): lane group g (half h = g / 2, quarter q = g % 2), MFMA t: elements
//         128 h + 32 t + 16 q + (0..15) = sub-block 8 h + 2 t + q. A lane group then reads 16
//         bytes of qh and 2 x 16 of ql that no other lane group reads. B is the unsigned code u =
//         q + 32 (<= 63); masking B to one lane group per MFMA gives each sub-block's integer dot,
//         scaled by its signed 8-bit scale in integer arithmetic; the -32 * sum(sc * bsums) term is
//         one fp16 MFMA of bsums (|.| <= 2032) against the scales, exact.
//   Q8_0  (8 blocks of 32): lane group g, MFMA t: elements 64 g + 16 t + (0..15), i.e. Q8_0 block
//         2 g + t / 2; B is the int8 quants as stored, masked to one lane group per MFMA pair.
//
// Numerics: integer block dots are exact; the fp32 steps and their order are the CPU oracle's
// (app/native/src/mx_dot_k_ssse3.c:150-154, 200-206; mx_dot_q8_0.c:8-18).
#pragma once

#include "mxa_device.hpp"

#pragma clang fp contract(off)

namespace mxa {
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // 16-byte aligned (LDS reads)

__device__ __forceinline__ i32x4 as_i32x4(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  return i32x4{(int)a, (int)b, (int)c, (int)d};
}

// Each byte of u times s (s * byte <= 255, so no carry crosses a byte): v_pk_mul_lo_u16.
__device__ __forceinline__ uint32_t mul_bytes(uint32_t u, uint32_t s) {
  const u16x2 a = __builtin_bit_cast(u16x2, u);
  const u16x2 b = {(uint16_t)s, (uint16_t)s};
  return __builtin_bit_cast(uint32_t, a * b);
}

// Four Q8_K bsums (int16, |.| <= 2032) as fp16, exactly.
__device__ __forceinline__ f16x4 bsums_f16x4(const int16_t* p) {
  const u32x2a4 v = ld8((const uint8_t*)p);
  return f16x4{(_Float16)(float)(int16_t)(v.x & 0xFFFFu), (_Float16)(float)(int16_t)(v.x >> 16),
               (_Float16)(float)(int16_t)(v.y & 0xFFFFu), (_Float16)(float)(int16_t)(v.y >> 16)};
}

// The lane-group mask of a B operand, built where it is used. `fresh` hides the operand from
// common-subexpression elimination, so a caller that feeds one weight tile to many activation
// tiles rebuilds the 16 masked operands per tile instead of keeping them all live.
template <bool kFresh>
__device__ __forceinline__ i32x4 masked_b(u32x4a4 v, bool on) {
  if constexpr (kFresh) asm volatile("" : "+v"(v));
  return as_i32x4(on ? v.x : 0u, on ? v.y : 0u, on ? v.z : 0u, on ? v.w : 0u);
}

// Activation chunk in LDS: q8 rows, bsums (as fp16) and scales of 16 * MT rows x kCB blocks.
struct ActTile {
  const int8_t* q;        // row r at q + r * qs, block bb at + bb * QK
  const _Float16* bs;     // row r at bs + r * bst, block bb at + bb * 16
  int qs, bst;            // row strides (bytes, halves)
};

// Every type provides: W (a lane's bytes of one weight tile's block) and load(); P = prep(W, g),
// the B operands of that tile and block; F = frag(A, bb, mt, ln, g), the A operands of activation
// tile mt (shared by all weight tiles of the wave); value(P, F, g, sink), which calls
// sink(e, v, d) with the block value of m = 4 g + e of the tile, n = lane % 16; and fold(acc, xd,
// v, d), the oracle's fold step.

// ---------------------------------------------------------------------------------------- Q4_K
struct TileQ4 {
  struct W {
    u32x4a4 hdr, qa, qb;
  };
  struct P {
    i32x4 bh[4], bl[4];  // planes of MFMA t: (sc >> 3) * u and (sc & 7) * u
    f16x4 bmin;
    float d, dmin;
  };
  struct F {
    i32x4 a[4];
    f16x4 bs;
  };
  __device__ static W load(const uint8_t* row, int b, int g) {
    const uint8_t* blk = row + (size_t)b * 144;
    W L;
    L.hdr = ld16_stream(blk);
    L.qa = ld16_stream(blk + 16 + 32 * g);
    L.qb = ld16_stream(blk + 32 + 32 * g);
    return L;
  }
  // The same bytes from a copy of the block at buf + off in LDS (off 4-byte aligned).
  __device__ __forceinline__ static W load_lds(const uint8_t* buf, int off, int g) {
    W L;
    L.hdr = ld16(buf + off);
    L.qa = ld16(buf + off + 16 + 32 * g);
    L.qb = ld16(buf + off + 32 + 32 * g);
    return L;
  }
  // A operands of activation row m, block b, from the Q8_K activations in global memory.
  __device__ __forceinline__ static F frag_g(const Act& act, int m, int b, int g) {
    F f;
    const int8_t* arow = act.q + (size_t)m * act.k + (size_t)b * QK + 64 * g;
#pragma unroll
    for (int t = 0; t < 4; ++t) f.a[t] = __builtin_bit_cast(i32x4, ld16s(arow + 16 * t));
    f.bs = bsums_f16x4(act.bsums + ((size_t)m * act.nb + b) * 16 + 4 * g);
    return f;
  }
  __device__ static float fold(float acc, float xd, float v, float) { return fmaf(xd, v, acc); }
  __device__ static P prep(const W& L, int g) {
    P p;
    p.d = half_to_float(L.hdr.x);
    p.dmin = half_to_float(L.hdr.x >> 16);
    const K4Scales s = k4_scales(L.hdr.y, L.hdr.z, L.hdr.w);
    const uint32_t sc0 = k4_pick(s.sc_lo, s.sc_hi, 2 * g), sc1 = k4_pick(s.sc_lo, s.sc_hi, 2 * g + 1);
    const uint32_t mn0 = k4_pick(s.mn_lo, s.mn_hi, 2 * g), mn1 = k4_pick(s.mn_lo, s.mn_hi, 2 * g + 1);
    const uint32_t q[8] = {L.qa.x, L.qa.y, L.qa.z, L.qa.w, L.qb.x, L.qb.y, L.qb.z, L.qb.w};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint32_t sh = (t < 2 ? sc0 : sc1) >> 3, sl = (t < 2 ? sc0 : sc1) & 7;
      uint32_t u[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        u[i] = t == 0 ? q[i] & 0x0F0F0F0Fu : t == 1 ? q[4 + i] & 0x0F0F0F0Fu
             : t == 2 ? (q[i] >> 4) & 0x0F0F0F0Fu : (q[4 + i] >> 4) & 0x0F0F0F0Fu;
      p.bh[t] = as_i32x4(mul_bytes(u[0], sh), mul_bytes(u[1], sh), mul_bytes(u[2], sh), mul_bytes(u[3], sh));
      p.bl[t] = as_i32x4(mul_bytes(u[0], sl), mul_bytes(u[1], sl), mul_bytes(u[2], sl), mul_bytes(u[3], sl));
    }
    const _Float16 m0 = (_Float16)(float)mn0, m1 = (_Float16)(float)mn1;
    p.bmin = f16x4{m0, m0, m1, m1};
    return p;
  }
  __device__ static F frag(const ActTile& A, int bb, int mt, int ln, int g) {
    F f;
    const int8_t* arow = A.q + (16 * mt + ln) * A.qs + bb * QK + 64 * g;
#pragma unroll
    for (int t = 0; t < 4; ++t) f.a[t] = __builtin_bit_cast(i32x4, *(const u32x4*)(arow + 16 * t));
    f.bs = *(const f16x4*)(A.bs + (16 * mt + ln) * A.bst + bb * 16 + 4 * g);
    return f;
  }
  template <bool kFresh = false, class S>
  __device__ static void value(const P& p, const F& f, int, S&& sink) {
    // the two planes accumulate in independent chains (half the dependent MFMA latency); the
    // integer result 8 * sh + sl is the same exact sum
    i32x4 sh = {0, 0, 0, 0}, sl = {0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      sh = __builtin_amdgcn_mfma_i32_16x16x64_i8(f.a[t], p.bh[t], sh, 0, 0, 0);
      sl = __builtin_amdgcn_mfma_i32_16x16x64_i8(f.a[t], p.bl[t], sl, 0, 0, 0);
    }
    const i32x4 sum = sh * 8 + sl;
    // summ = sum over the 16 bsums of min_{s/2} * bsum: A = bsums (k = 4g..4g+3), B = mins
    const f32x4 summ = __builtin_amdgcn_mfma_f32_16x16x16f16(f.bs, p.bmin, f32x4{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) sink(i, fmaf(p.d, (float)sum[i], -(p.dmin * summ[i])), 0.0f);
  }
  // value() already issues its MFMAs in two independent chains
  template <class S>
  __device__ static void value_wide(const P& p, const F& f, int g, S&& sink) {
    value(p, f, g, static_cast<S&&>(sink));
  }
};

// ---------------------------------------------------------------------------------------- Q6_K
struct TileQ6 {
  struct W {
    u32x4a4 qla, qlb, qh, sc;  // ql[64h + 16q ..], ql[64h + 32 + 16q ..], qh[32h + 16q ..], scales
    uint32_t d;
  };
  struct P {
    u32x4a4 bu[4];  // codes u of MFMA t (elements 128 h + 32 t + 16 q + j)
    int scv[4][4];  // scale of the sub-block of (MFMA t, lane group g2), row n
    f16x4 bsc;      // scales 4 g .. 4 g + 3 of row n (the bsums term)
    float d;
  };
  struct F {
    i32x4 a[4];
    f16x4 bs;
  };
  // 16 bytes at p, 2-byte aligned at worst (210-byte blocks): dword loads + v_alignbyte. The fifth
  // dword is read only when p is not 4-byte aligned, so no byte past p + 15 is touched.
  __device__ static u32x4a4 ld16_a2(const uint8_t* p) {
    const uintptr_t a = (uintptr_t)p;
    const uint8_t* base = (const uint8_t*)(a & ~(uintptr_t)3);
    const uint32_t sh = (uint32_t)(a & 3);
    const u32x4a4 v = ld16_stream(base);
    const uint32_t e = sh ? __builtin_nontemporal_load((const uint32_t*)(base + 16)) : 0u;
    return u32x4a4{__builtin_amdgcn_alignbyte(v.y, v.x, sh), __builtin_amdgcn_alignbyte(v.z, v.y, sh),
                   __builtin_amdgcn_alignbyte(v.w, v.z, sh), __builtin_amdgcn_alignbyte(e, v.w, sh)};
  }
  __device__ static W load(const uint8_t* row, int b, int g) {
    const uint8_t* blk = row + (size_t)b * 210;
    const int h = g >> 1, q = g & 1;
    W L;
    L.qla = ld16_a2(blk + 64 * h + 16 * q);
    L.qlb = ld16_a2(blk + 64 * h + 32 + 16 * q);
    L.qh = ld16_a2(blk + 128 + 32 * h + 16 * q);
    L.sc = ld16_a2(blk + 192);
    L.d = (uint32_t)*(const uint16_t*)(blk + 208);
    return L;
  }
  // ld16_a2 on a copy in LDS: 16 bytes at buf + off, off even.
  __device__ __forceinline__ static u32x4a4 lds16_a2(const uint8_t* buf, int off) {
    const int base = off & ~3;
    const uint32_t sh = (uint32_t)(off & 3);
    const u32x4a4 v = ld16(buf + base);
    const uint32_t e = sh ? ld4(buf + base + 16) : 0u;
    return u32x4a4{__builtin_amdgcn_alignbyte(v.y, v.x, sh), __builtin_amdgcn_alignbyte(v.z, v.y, sh),
                   __builtin_amdgcn_alignbyte(v.w, v.z, sh), __builtin_amdgcn_alignbyte(e, v.w, sh)};
  }
  // The same bytes from a copy of the block at buf + off in LDS (off even).
  __device__ __forceinline__ static W load_lds(const uint8_t* buf, int off, int g) {
    const int h = g >> 1, q = g & 1;
    W L;
    L.qla = lds16_a2(buf, off + 64 * h + 16 * q);
    L.qlb = lds16_a2(buf, off + 64 * h + 32 + 16 * q);
    L.qh = lds16_a2(buf, off + 128 + 32 * h + 16 * q);
    L.sc = lds16_a2(buf, off + 192);
    L.d = (uint32_t)*(const uint16_t*)(buf + off + 208);
    return L;
  }
  // A operands of activation row m, block b, from the Q8_K activations in global memory.
  __device__ __forceinline__ static F frag_g(const Act& act, int m, int b, int g) {
    F f;
    const int8_t* arow = act.q + (size_t)m * act.k + (size_t)b * QK + 128 * (g >> 1) + 16 * (g & 1);
#pragma unroll
    for (int t = 0; t < 4; ++t) f.a[t] = __builtin_bit_cast(i32x4, ld16s(arow + 32 * t));
    f.bs = bsums_f16x4(act.bsums + ((size_t)m * act.nb + b) * 16 + 4 * g);
    return f;
  }
  // block value sumi (as float) with the block's d; fold (xd * d) * sumi (mx_dot_k_ssse3.c:200-206)
  __device__ static float fold(float acc, float xd, float v, float d) { return fmaf(xd * d, v, acc); }
  __device__ static P prep(const W& L, int g) {
    P p;
    p.d = half_to_float(L.d);
    const uint32_t la[4] = {L.qla.x, L.qla.y, L.qla.z, L.qla.w};
    const uint32_t lb[4] = {L.qlb.x, L.qlb.y, L.qlb.z, L.qlb.w};
    const uint32_t hh[4] = {L.qh.x, L.qh.y, L.qh.z, L.qh.w};
    const uint32_t scw[4] = {L.sc.x, L.sc.y, L.sc.z, L.sc.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p.bu[0][i] = q6_codes<0>(la[i], hh[i]);
      p.bu[1][i] = q6_codes<1>(lb[i], hh[i]);
      p.bu[2][i] = q6_codes<2>(la[i], hh[i]);
      p.bu[3][i] = q6_codes<3>(lb[i], hh[i]);
    }
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int g2 = 0; g2 < 4; ++g2) {
        const int sub = 8 * (g2 >> 1) + 2 * t + (g2 & 1);
        p.scv[t][g2] = (int)(int8_t)(uint8_t)(scw[sub >> 2] >> (8 * (sub & 3)));
      }
    const uint32_t sw = scw[g];
    p.bsc = f16x4{(_Float16)(float)(int8_t)(sw & 0xFF), (_Float16)(float)(int8_t)((sw >> 8) & 0xFF),
                  (_Float16)(float)(int8_t)((sw >> 16) & 0xFF), (_Float16)(float)(int8_t)(sw >> 24)};
    return p;
  }
  __device__ static F frag(const ActTile& A, int bb, int mt, int ln, int g) {
    F f;
    const int8_t* arow = A.q + (16 * mt + ln) * A.qs + bb * QK + 128 * (g >> 1) + 16 * (g & 1);
#pragma unroll
    for (int t = 0; t < 4; ++t) f.a[t] = __builtin_bit_cast(i32x4, *(const u32x4*)(arow + 32 * t));
    f.bs = *(const f16x4*)(A.bs + (16 * mt + ln) * A.bst + bb * 16 + 4 * g);
    return f;
  }
  template <bool kFresh = false, class S>
  __device__ static void value(const P& p, const F& f, int g, S&& sink) {
    int sumi[4] = {0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int g2 = 0; g2 < 4; ++g2) {
        const bool on = g == g2;  // B restricted to lane group g2: one sub-block's dot
        const i32x4 b = masked_b<kFresh>(p.bu[t], on);
        const i32x4 D = __builtin_amdgcn_mfma_i32_16x16x64_i8(f.a[t], b, i32x4{0, 0, 0, 0}, 0, 0, 0);
        // |D| <= 16 * 63 * 127 < 2^17, |sc| <= 128: 24-bit products
#pragma unroll
        for (int i = 0; i < 4; ++i) sumi[i] += __mul24(p.scv[t][g2], D[i]);
      }
    // C = sum over the 16 sub-blocks of bsums(m) * sc(n), exact (|C| < 2^22)
    const f32x4 C = __builtin_amdgcn_mfma_f32_16x16x16f16(f.bs, p.bsc, f32x4{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) sink(i, (float)(sumi[i] - 32 * (int)C[i]), p.d);
  }
  // value() with the 16 sub-block MFMAs issued into results of their own before any is scaled, so
  // that they overlap instead of each waiting out its predecessor's latency (64 more VGPRs live:
  // for kernels with one activation tile); the same exact integer sum
  template <class S>
  __device__ static void value_wide(const P& p, const F& f, int g, S&& sink) {
    i32x4 D[4][4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int g2 = 0; g2 < 4; ++g2)
        D[t][g2] = __builtin_amdgcn_mfma_i32_16x16x64_i8(f.a[t], masked_b<false>(p.bu[t], g == g2),
                                                          i32x4{0, 0, 0, 0}, 0, 0, 0);
    const f32x4 C = __builtin_amdgcn_mfma_f32_16x16x16f16(f.bs, p.bsc, f32x4{0, 0, 0, 0}, 0, 0, 0);
    int sumi[4] = {0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int g2 = 0; g2 < 4; ++g2)
#pragma unroll
        for (int i = 0; i < 4; ++i) sumi[i] += __mul24(p.scv[t][g2], D[t][g2][i]);
#pragma unroll
    for (int i = 0; i < 4; ++i) sink(i, (float)(sumi[i] - 32 * (int)C[i]), p.d);
  }
};

// ------------------------------------------------------------------------- Q6_K, 32-deep MFMAs
// Q6_K on v_mfma_i32_16x16x32_i8 (A 16 x 32, B 32 x 16, a lane holding 8 k-values) with the block's
// elements in natural order: chunk c (MFMA k = 32 c .. 32 c + 31) gives lane group g elements
// 32 c + 8 g + (0..7), so lane groups {0, 1} hold sub-block 2 c and {2, 3} sub-block 2 c + 1.
// Zeroing one operand outside one pair of lane groups gives a sub-block's integer dot, in 16 MFMAs
// of half the depth. The zeroing sits in the A operands: F holds a lane's activation bytes twice,
// once per lane-group pair, the copy of the other pair zero, so a kernel whose waves keep their A
// operands across weight tiles builds the masks once per operand instead of selecting 32 B dwords
// per block and tile (the B codes go to the MFMAs unmasked). Element
// 32 c + 8 g + j (half h = c / 4, quarter r = c % 4, l = 8 g + j) is ql[64 h + l + 32 (r & 1)]'s
// low (r < 2) or high nibble with qh[32 h + l]'s bits 2 r .. 2 r + 1 above (kquants.py:138-159),
// so a lane reads four 8-byte runs of ql and two of qh. The integer block sum equals TileQ6's.
struct TileQ6s {
  struct W {
    u32x2a4 ql[2][2];  // ql[64 h + 32 q + 8 g ..] for half h, q = r & 1
    u32x2a4 qh[2];     // qh[32 h + 8 g ..]
    u32x4a4 sc;        // the row's 16 scales
    uint32_t d;
  };
  struct P {
    u32x2a4 bu[8];  // codes u of chunk c
    uint32_t scw[4];
    f16x4 bsc;  // scales 4 g .. 4 g + 3 (the bsums term)
    float d;
  };
  struct F {
    long a[2][8];  // activations 32 c + 8 g .. + 7 of row ln in a[g / 2][c]; a[1 - g / 2][c] = 0
    f16x4 bs;
  };
  // 8 bytes at buf + off in LDS, off even (2-byte-aligned blocks): dword reads + v_alignbyte.
  __device__ __forceinline__ static u32x2a4 lds8_a2(const uint8_t* buf, int off) {
    const int base = off & ~3;
    const uint32_t sh = (uint32_t)(off & 3);
    const u32x2a4 v = *(const u32x2a4*)(buf + base);
    const uint32_t e = sh ? *(const uint32_t*)(buf + base + 8) : 0u;
    return u32x2a4{__builtin_amdgcn_alignbyte(v.y, v.x, sh), __builtin_amdgcn_alignbyte(e, v.y, sh)};
  }
  __device__ __forceinline__ static W load_lds(const uint8_t* buf, int off, int g) {
    W L;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int q = 0; q < 2; ++q) L.ql[h][q] = lds8_a2(buf, off + 64 * h + 32 * q + 8 * g);
      L.qh[h] = lds8_a2(buf, off + 128 + 32 * h + 8 * g);
    }
    L.sc = TileQ6::lds16_a2(buf, off + 192);
    L.d = (uint32_t)*(const uint16_t*)(buf + off + 208);
    return L;
  }
  __device__ static float fold(float acc, float xd, float v, float d) { return fmaf(xd * d, v, acc); }
  __device__ static P prep(const W& L, int g) {
    P p;
    p.d = half_to_float(L.d);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int h = c >> 2, r = c & 3;
      const u32x2a4 lo = L.ql[h][r & 1], hi = L.qh[h];
      const uint32_t ls = 4 * (r >> 1), hs = 2 * r;
      p.bu[c] = u32x2a4{((lo.x >> ls) & 0x0F0F0F0Fu) | (((hi.x >> hs) & 0x03030303u) << 4),
                        ((lo.y >> ls) & 0x0F0F0F0Fu) | (((hi.y >> hs) & 0x03030303u) << 4)};
    }
    p.scw[0] = L.sc.x, p.scw[1] = L.sc.y, p.scw[2] = L.sc.z, p.scw[3] = L.sc.w;
    const uint32_t sw = g == 0 ? L.sc.x : g == 1 ? L.sc.y : g == 2 ? L.sc.z : L.sc.w;  // no indexing
    p.bsc = f16x4{(_Float16)(float)(int8_t)(sw & 0xFF), (_Float16)(float)(int8_t)((sw >> 8) & 0xFF),
                  (_Float16)(float)(int8_t)((sw >> 16) & 0xFF), (_Float16)(float)(int8_t)(sw >> 24)};
    return p;
  }
  // the 16 sub-block dots (chunk c, lane-group pair u: sub-block 2 c + u) issued before any is
  // scaled; C = sum over the sub-blocks of bsums(m) * sc(n), exact
  template <class S>
  __device__ static void value_wide(const P& p, const F& f, int g, S&& sink) {
    i32x4 D[8][2];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const long b = (long)(((uint64_t)p.bu[c].y << 32) | p.bu[c].x);
#pragma unroll
      for (int u = 0; u < 2; ++u)
        D[c][u] = __builtin_amdgcn_mfma_i32_16x16x32_i8(f.a[u][c], b, i32x4{0, 0, 0, 0}, 0, 0, 0);
    }
    const f32x4 C = __builtin_amdgcn_mfma_f32_16x16x16f16(f.bs, p.bsc, f32x4{0, 0, 0, 0}, 0, 0, 0);
    int sumi[4] = {0, 0, 0, 0};
#pragma unroll
    for (int c = 0; c < 8; ++c)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int s = 2 * c + u;
        const int sc = (int)(int8_t)(uint8_t)(p.scw[s >> 2] >> (8 * (s & 3)));
#pragma unroll
        for (int i = 0; i < 4; ++i) sumi[i] += __mul24(sc, D[c][u][i]);
      }
#pragma unroll
    for (int i = 0; i < 4; ++i) sink(i, (float)(sumi[i] - 32 * (int)C[i]), p.d);
  }
};

// ---------------------------------------------------------------------------------------- Q8_0
struct TileQ8 {
  struct W {
    uint32_t w[17];  // bytes 68 g .. 68 g + 67 of the 272-byte group: blocks 2 g and 2 g + 1
  };
  struct P {
    u32x4a4 qb[4];  // quants of MFMA t: block 2 g + t / 2, elements 16 (t % 2) ..
    float dk[8];    // d of the 8 blocks of row n
  };
  struct F {
    i32x4 a[4];
  };
  __device__ static W load(const uint8_t* row, int b, int g) {
    const uint8_t* p = row + (size_t)b * 272 + 68 * g;  // 4-byte aligned
    W L;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4a4 v = ld16_stream(p + 16 * i);
      L.w[4 * i] = v.x, L.w[4 * i + 1] = v.y, L.w[4 * i + 2] = v.z, L.w[4 * i + 3] = v.w;
    }
    L.w[16] = __builtin_nontemporal_load((const uint32_t*)(p + 64));
    return L;
  }
  // The same bytes from a copy of the group at buf + off in LDS (off 4-byte aligned).
  __device__ __forceinline__ static W load_lds(const uint8_t* buf, int off, int g) {
    const uint8_t* p = buf + off + 68 * g;
    W L;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4a4 v = ld16(p + 16 * i);
      L.w[4 * i] = v.x, L.w[4 * i + 1] = v.y, L.w[4 * i + 2] = v.z, L.w[4 * i + 3] = v.w;
    }
    L.w[16] = ld4(p + 64);
    return L;
  }
  // A operands of activation row m, 256-value group b, from the Q8_K activations in global memory.
  __device__ __forceinline__ static F frag_g(const Act& act, int m, int b, int g) {
    F f;
    const int8_t* arow = act.q + (size_t)m * act.k + (size_t)b * QK + 64 * g;
#pragma unroll
    for (int t = 0; t < 4; ++t) f.a[t] = __builtin_bit_cast(i32x4, ld16s(arow + 16 * t));
    return f;
  }
  // block value sum_k d_k * p_k in k order; fold xd * value (mx_dot_q8_0.c:8-18)
  __device__ static float fold(float acc, float xd, float v, float) { return fmaf(xd, v, acc); }
  __device__ static P prep(const W& L, int g) {
    P p;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p.qb[0][i] = __builtin_amdgcn_alignbyte(L.w[i + 1], L.w[i], 2);
      p.qb[1][i] = __builtin_amdgcn_alignbyte(L.w[i + 5], L.w[i + 4], 2);
      p.qb[2][i] = L.w[9 + i];
      p.qb[3][i] = L.w[13 + i];
    }
    // this lane holds the d of blocks 2 g and 2 g + 1; lane n + 16 g2 holds those of 2 g2..
    const int ln = (int)(__lane_id() & 15);
    const uint32_t mine = (L.w[0] & 0xFFFFu) | (L.w[8] & 0xFFFF0000u);
#pragma unroll
    for (int g2 = 0; g2 < 4; ++g2) {
      const uint32_t v = (uint32_t)__shfl((int)mine, ln + 16 * g2, 64);
      p.dk[2 * g2] = half_to_float(v);
      p.dk[2 * g2 + 1] = half_to_float(v >> 16);
    }
    (void)g;
    return p;
  }
  __device__ static F frag(const ActTile& A, int bb, int mt, int ln, int g) {
    F f;
    const int8_t* arow = A.q + (16 * mt + ln) * A.qs + bb * QK + 64 * g;
#pragma unroll
    for (int t = 0; t < 4; ++t) f.a[t] = __builtin_bit_cast(i32x4, *(const u32x4*)(arow + 16 * t));
    return f;
  }
  template <bool kFresh = false, class S>
  __device__ static void value(const P& p, const F& f, int g, S&& sink) {
    float bs[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < 8; ++k) {  // block k = 2 g2 + h: MFMAs t = 2 h, 2 h + 1 of lane group g2
      const int g2 = k >> 1, h = k & 1;
      const bool on = g == g2;
      i32x4 D = {0, 0, 0, 0};
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const int t = 2 * h + tt;
        const i32x4 b = masked_b<kFresh>(p.qb[t], on);
        D = __builtin_amdgcn_mfma_i32_16x16x64_i8(f.a[t], b, D, 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) bs[i] = fmaf(p.dk[k], (float)D[i], bs[i]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) sink(i, bs[i], 0.0f);
  }
  // value() with the eight blocks' MFMA pairs issued before any is scaled; the same fp32 steps
  template <class S>
  __device__ static void value_wide(const P& p, const F& f, int g, S&& sink) {
    i32x4 D[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int g2 = k >> 1, h = k & 1;
      const bool on = g == g2;
      D[k] = i32x4{0, 0, 0, 0};
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
        D[k] = __builtin_amdgcn_mfma_i32_16x16x64_i8(f.a[2 * h + tt], masked_b<false>(p.qb[2 * h + tt], on),
                                                     D[k], 0, 0, 0);
    }
    float bs[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < 8; ++k)
#pragma unroll
      for (int i = 0; i < 4; ++i) bs[i] = fmaf(p.dk[k], (float)D[k][i], bs[i]);
#pragma unroll
    for (int i = 0; i < 4; ++i) sink(i, bs[i], 0.0f);
  }
};

template <int TYPE>
struct TileOf;
template <> struct TileOf<T_Q4_K> { using T = TileQ4; };
template <> struct TileOf<T_Q6_K> { using T = TileQ6; };
template <> struct TileOf<T_Q8_0> { using T = TileQ8; };
}  // namespace mxa
