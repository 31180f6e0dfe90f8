// Matrix-core matmul for M > 4 activation rows (batched decode and prefill), Q4_K / Q6_K / Q8_0.
//
// Tiling. A workgroup of 1, 2 or 4 waves owns 16 consecutive weight rows per wave and 16 * MT
// activation rows (the host picks the wave count that gives the GPU enough workgroups); grid.y walks the activation rows, so a weight block is read once per 16 * MT
// activation rows. The Q8_K activations (always pre-quantized in the workspace here) are staged in
// LDS per chunk of kCB blocks; each wave keeps its rows' blocks of the next chunk in registers
// while it computes the current one.
//
// Operands of v_mfma_i32_16x16x64_i8: A (16 activation rows m x 64 k) from LDS, B (64 k x 16 weight
// rows n) built in registers from the packed bytes. Lane l supplies row (l % 16) and k-group
// g = l / 16 of both; its output holds n = l % 16 and m = 4 g + i (i < 4). The k-group / MFMA t
// assignment of the 256 values of a block differs per type and is chosen so that every lane-group
// slice of an MFMA lies inside one scale sub-block:
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
// (app/native/src/mx_dot_k_ssse3.c:150-154, 200-206; mx_dot_q8_0.c:8-18) and the blocks are folded
// in order 0..nb-1, so the outputs equal the oracle and the decode kernels bit for bit.
#include "mxa_kernels.hpp"

#pragma clang fp contract(off)

namespace mxa {
namespace {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // 16-byte aligned (LDS reads)

constexpr int kCB = 2;                    // blocks per activation chunk
constexpr int kQStride = kCB * QK + 16;   // LDS bytes per activation row (padding: distinct banks)
constexpr int kBStride = kCB * 16 + 8;    // LDS halves per activation row of bsums

__device__ __forceinline__ i32x4 as_i32x4(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  return i32x4{(int)a, (int)b, (int)c, (int)d};
}

// Each byte of u times s (s * byte <= 255, so no carry crosses a byte): v_pk_mul_lo_u16.
__device__ __forceinline__ uint32_t mul_bytes(uint32_t u, uint32_t s) {
  const u16x2 a = __builtin_bit_cast(u16x2, u);
  const u16x2 b = {(uint16_t)s, (uint16_t)s};
  return __builtin_bit_cast(uint32_t, a * b);
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
  template <class S>
  __device__ static void value(const P& p, const F& f, int, S&& sink) {
    i32x4 sum = {0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < 4; ++t) sum = __builtin_amdgcn_mfma_i32_16x16x64_i8(f.a[t], p.bh[t], sum, 0, 0, 0);
    sum = sum * 8;
#pragma unroll
    for (int t = 0; t < 4; ++t) sum = __builtin_amdgcn_mfma_i32_16x16x64_i8(f.a[t], p.bl[t], sum, 0, 0, 0);
    // summ = sum over the 16 bsums of min_{s/2} * bsum: A = bsums (k = 4g..4g+3), B = mins
    const f32x4 summ = __builtin_amdgcn_mfma_f32_16x16x16f16(f.bs, p.bmin, f32x4{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) sink(i, fmaf(p.d, (float)sum[i], -(p.dmin * summ[i])), 0.0f);
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
  template <class S>
  __device__ static void value(const P& p, const F& f, int g, S&& sink) {
    int sumi[4] = {0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int g2 = 0; g2 < 4; ++g2) {
        const bool on = g == g2;  // B restricted to lane group g2: one sub-block's dot
        const i32x4 b = as_i32x4(on ? p.bu[t].x : 0u, on ? p.bu[t].y : 0u, on ? p.bu[t].z : 0u, on ? p.bu[t].w : 0u);
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
  template <class S>
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
        const i32x4 b = as_i32x4(on ? p.qb[t].x : 0u, on ? p.qb[t].y : 0u, on ? p.qb[t].z : 0u, on ? p.qb[t].w : 0u);
        D = __builtin_amdgcn_mfma_i32_16x16x64_i8(f.a[t], b, D, 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) bs[i] = fmaf(p.dk[k], (float)D[i], bs[i]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) sink(i, bs[i], 0.0f);
  }
};

template <int TYPE>
struct TileOf;
template <> struct TileOf<T_Q4_K> { using T = TileQ4; };
template <> struct TileOf<T_Q6_K> { using T = TileQ6; };
template <> struct TileOf<T_Q8_0> { using T = TileQ8; };

// Row-tiled kernel: MT activation tiles x NT weight tiles of 16 rows per wave, 4 waves.
template <int TYPE, int MT, int NT>
__global__ __launch_bounds__(256) void mtile_kernel(const uint8_t* w, long long row_bytes, Act act,
                                                    float* __restrict__ y, long long ldy, int M, int N) {
  using Tile = typename TileOf<TYPE>::T;
  using W = typename Tile::W;
  constexpr int kRows = 16 * MT;
  __shared__ __align__(16) int8_t Aq[kRows * kQStride];
  __shared__ __align__(16) _Float16 Ab[kRows * kBStride];
  __shared__ __align__(16) float Ad[kCB * kRows];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int ln = lane & 15, g = lane >> 4;
  const int n0 = xcd_tile(blockIdx.x, gridDim.x) * 4 * 16 * NT + 16 * NT * wave;
  const int m0 = blockIdx.y * kRows;
  const uint8_t* row[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) row[nt] = w + (size_t)min(n0 + 16 * nt + ln, N - 1) * row_bytes;
  const int nb = act.nb;
  float acc[MT][NT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[mt][nt][i] = 0.0f;

  W cur[NT], nxt[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) cur[nt] = Tile::load(row[nt], 0, g);

  // Activation staging, software-pipelined: chunk c + 1 is loaded into registers while chunk c
  // is computed, and written to LDS between the two barriers. Thread tid owns the same pieces of
  // every chunk (rows >= M repeat row M - 1, blocks >= cn repeat the chunk's last block: those
  // results are never stored).
  constexpr int kQPieces = kRows * kCB * 16;                   // 16-byte pieces of q8
  constexpr int kQPer = (kQPieces + 255) / 256;
  constexpr int kBPieces = kRows * kCB * 2;                    // halves of a block's 16 bsums
  constexpr int kBPer = (kBPieces + 255) / 256;
  constexpr int kDPer = (kRows * kCB + 255) / 256;
  struct Stage {
    u32x4a4 q[kQPer];
    u32x4a4 b[kBPer];
    float d[kDPer];
  };
  auto load_stage = [&](int c0) {
    Stage st;
    const int cn = min(kCB, nb - c0);
#pragma unroll
    for (int j = 0; j < kQPer; ++j) {
      const int p = min(tid + 256 * j, kQPieces - 1);
      const int r = p / (kCB * 16), o = p - r * (kCB * 16), bb = min(o >> 4, cn - 1), pc = o & 15;
      st.q[j] = ld16((const uint8_t*)(act.q + (size_t)min(m0 + r, M - 1) * act.k + (size_t)(c0 + bb) * QK) + 16 * pc);
    }
#pragma unroll
    for (int j = 0; j < kBPer; ++j) {
      const int p = min(tid + 256 * j, kBPieces - 1);
      const int r = p / (kCB * 2), o = p - r * (kCB * 2), bb = min(o >> 1, cn - 1), hf = o & 1;
      st.b[j] = ld16((const uint8_t*)(act.bsums + ((size_t)min(m0 + r, M - 1) * nb + c0 + bb) * 16) + 16 * hf);
    }
#pragma unroll
    for (int j = 0; j < kDPer; ++j) {
      const int p = min(tid + 256 * j, kRows * kCB - 1), bb = p / kRows, r = p - bb * kRows;
      st.d[j] = act.d[(size_t)min(m0 + r, M - 1) * nb + c0 + min(bb, cn - 1)];
    }
    return st;
  };
  auto store_stage = [&](const Stage& st) {
#pragma unroll
    for (int j = 0; j < kQPer; ++j) {
      const int p = tid + 256 * j;
      if (p < kQPieces) {
        const int r = p / (kCB * 16), o = p - r * (kCB * 16);
        *(u32x4a4*)(Aq + r * kQStride + (o >> 4) * QK + 16 * (o & 15)) = st.q[j];
      }
    }
#pragma unroll
    for (int j = 0; j < kBPer; ++j) {
      const int p = tid + 256 * j;
      if (p < kBPieces) {  // bsums as fp16 (exact: |.| <= 2032)
        const int r = p / (kCB * 2), o = p - r * (kCB * 2);
        const uint32_t wv[4] = {st.b[j].x, st.b[j].y, st.b[j].z, st.b[j].w};
        f16x8 hv;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          hv[2 * i] = (_Float16)(float)(int16_t)(wv[i] & 0xFFFFu);
          hv[2 * i + 1] = (_Float16)(float)(int16_t)(wv[i] >> 16);
        }
        *(f16x8*)(Ab + r * kBStride + (o >> 1) * 16 + 8 * (o & 1)) = hv;
      }
    }
#pragma unroll
    for (int j = 0; j < kDPer; ++j) {
      const int p = tid + 256 * j;
      if (p < kRows * kCB) Ad[p] = st.d[j];
    }
  };

  static_assert(4 * 64 == 256, "four waves");
  {
    const Stage st0 = load_stage(0);
    store_stage(st0);
  }
  __syncthreads();
  for (int c0 = 0; c0 < nb; c0 += kCB) {
    const int cn = min(kCB, nb - c0);
    const bool more = c0 + kCB < nb;
    Stage st;
    if (more) st = load_stage(c0 + kCB);
    // the chunk's blocks in order; the next block's weights load meanwhile
    const ActTile A{Aq, Ab, kQStride, kBStride};
#pragma unroll
    for (int i = 0; i < kCB; ++i) {
      if (i < cn) {
        const int b = c0 + i;
        if (b + 1 < nb) {
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) nxt[nt] = Tile::load(row[nt], b + 1, g);
        }
        typename Tile::P pp[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) pp[nt] = Tile::prep(cur[nt], g);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const typename Tile::F f = Tile::frag(A, i, mt, ln, g);
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
            Tile::value(pp[nt], f, g, [&](int e, float v, float dd) {
              acc[mt][nt][e] = Tile::fold(acc[mt][nt][e], Ad[i * kRows + 16 * mt + 4 * g + e], v, dd);
            });
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) cur[nt] = nxt[nt];
      }
    }
    __syncthreads();  // every wave is done with this chunk's LDS
    if (more) {
      store_stage(st);
      __syncthreads();
    }
  }
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int n = n0 + 16 * nt + ln;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = m0 + 16 * mt + 4 * g + i;
        if (m < M && n < N) y[(size_t)m * ldy + n] = acc[mt][nt][i];
      }
  }
}

// Batched decode (M <= 16): 32 weight rows per workgroup and the blocks of each chunk split over
// the 4 waves (wave w takes blocks w and w + 4 of an 8-block chunk, for both 16-row tiles), so that
// N = 4096..14336 still gives the GPU 128..448 workgroups. The block values go through LDS and are
// folded in block order by the thread that owns the output.
constexpr int kDecCh = 8;                     // blocks per chunk
constexpr int kDecQStride = kDecCh * QK + 16;
constexpr int kDecBStride = kDecCh * 16 + 8;

// kDecRT 16-row weight tiles per workgroup: 2, or 1 for Q6_K (its per-lane block bytes need twice
// the registers; one tile keeps two waves per SIMD).
template <int TYPE, int kDecRT>
__global__ __launch_bounds__(256) void mdec_kernel(const uint8_t* w, long long row_bytes, Act act,
                                                   float* __restrict__ y, long long ldy, int M, int N) {
  using Tile = typename TileOf<TYPE>::T;
  using W = typename Tile::W;
  __shared__ __align__(16) int8_t Aq[16 * kDecQStride];
  __shared__ __align__(16) _Float16 Ab[16 * kDecBStride];
  __shared__ float Ad[kDecCh * 16];
  __shared__ float Tp[kDecRT][kDecCh][16][16];  // block values [tile][block][m][n]
  __shared__ float Dp[kDecRT][kDecCh][16];      // the block's weight scale where the fold uses one

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int ln = lane & 15, g = lane >> 4;
  const int n0 = xcd_tile(blockIdx.x, gridDim.x) * 16 * kDecRT;
  const uint8_t* rows[kDecRT];
#pragma unroll
  for (int t = 0; t < kDecRT; ++t) rows[t] = w + (size_t)min(n0 + 16 * t + ln, N - 1) * row_bytes;
  const int nb = act.nb;
  constexpr int kOut = kDecRT * 256 / 256;  // outputs per thread: kDecRT tiles x 16 x 16 / 256
  float acc[kOut];
#pragma unroll
  for (int k = 0; k < kOut; ++k) acc[k] = 0.0f;

  W cur[2][kDecRT], nxt[2][kDecRT];
  {
    const int cn = min(kDecCh, nb);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int t = 0; t < kDecRT; ++t) cur[i][t] = Tile::load(rows[t], min(wave + 4 * i, cn - 1), g);
  }
  for (int c0 = 0; c0 < nb; c0 += kDecCh) {
    const int cn = min(kDecCh, nb - c0);
    // 1. the chunk's activations into LDS (rows >= M repeat row M - 1, blocks >= cn repeat the
    //    chunk's last block: those values are never folded or stored)
    for (int p = tid; p < 16 * kDecCh * 16; p += 256) {
      const int r = p / (kDecCh * 16), o = p - r * (kDecCh * 16), bb = min(o >> 4, cn - 1), pc = o & 15;
      *(u32x4a4*)(Aq + r * kDecQStride + (o >> 4) * QK + 16 * pc) =
          ld16((const uint8_t*)(act.q + (size_t)min(r, M - 1) * act.k + (size_t)(c0 + bb) * QK) + 16 * pc);
    }
    {
      const int r = tid >> 4, o = tid & 15, bb = min(o >> 1, cn - 1), hf = o & 1;
      const u32x4a4 v = ld16((const uint8_t*)(act.bsums + ((size_t)min(r, M - 1) * nb + c0 + bb) * 16) + 16 * hf);
      const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
      f16x8 hv;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        hv[2 * i] = (_Float16)(float)(int16_t)(wv[i] & 0xFFFFu);
        hv[2 * i + 1] = (_Float16)(float)(int16_t)(wv[i] >> 16);
      }
      *(f16x8*)(Ab + r * kDecBStride + (o >> 1) * 16 + 8 * hf) = hv;
    }
    if (tid < kDecCh * 16) {
      const int bb = tid >> 4, r = tid & 15;
      Ad[tid] = act.d[(size_t)min(r, M - 1) * nb + c0 + min(bb, cn - 1)];
    }
    // 2. weights of the next chunk
    const int c1 = c0 + kDecCh;
    if (c1 < nb) {
      const int cn1 = min(kDecCh, nb - c1);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int t = 0; t < kDecRT; ++t) nxt[i][t] = Tile::load(rows[t], c1 + min(wave + 4 * i, cn1 - 1), g);
    }
    __syncthreads();
    // 3. this wave's blocks, both tiles: values into LDS
    const ActTile A{Aq, Ab, kDecQStride, kDecBStride};
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int bb = wave + 4 * i;
      if (bb < cn) {
        const typename Tile::F f = Tile::frag(A, bb, 0, ln, g);
#pragma unroll
        for (int t = 0; t < kDecRT; ++t) {
          const typename Tile::P pp = Tile::prep(cur[i][t], g);
          Tile::value(pp, f, g, [&](int e, float v, float dd) {
            Tp[t][bb][4 * g + e][ln] = v;
            if (g == 0 && e == 0) Dp[t][bb][ln] = dd;
          });
        }
      }
    }
    __syncthreads();
    // 4. fold the chunk's blocks in order: thread -> outputs (tile, m, n)
#pragma unroll
    for (int k = 0; k < kOut; ++k) {
      const int idx = tid + 256 * k, t = idx >> 8, m = (idx >> 4) & 15, n = idx & 15;
      for (int bb = 0; bb < cn; ++bb) acc[k] = Tile::fold(acc[k], Ad[bb * 16 + m], Tp[t][bb][m][n], Dp[t][bb][n]);
    }
    __syncthreads();
    if (c1 < nb) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int t = 0; t < kDecRT; ++t) cur[i][t] = nxt[i][t];
    }
  }
#pragma unroll
  for (int k = 0; k < kOut; ++k) {
    const int idx = tid + 256 * k, t = idx >> 8, m = (idx >> 4) & 15, n = n0 + 16 * t + (idx & 15);
    if (m < M && n < N) y[(size_t)m * ldy + n] = acc[k];
  }
}

template <int TYPE, int MT, int NT>
int launch_mt(const uint8_t* w, long long row_bytes, const Act& act, float* y, long long ldy, int M,
              int N, hipStream_t stream) {
  const int rows = 4 * 16 * NT;
  const dim3 grid((N + rows - 1) / rows, (M + 16 * MT - 1) / (16 * MT));
  hipLaunchKernelGGL((mtile_kernel<TYPE, MT, NT>), grid, dim3(256), 0, stream, w, row_bytes, act, y,
                     ldy, M, N);
  return 0;
}

template <int TYPE>
int launch_mt_type(const uint8_t* w, long long row_bytes, const Act& act, float* y, long long ldy,
                   int M, int N, hipStream_t stream) {
  // M <= 16: the block-split kernel unless the 64-row tiles alone give >= 512 workgroups
  if (M <= 16 && N < 512 * 64) {
    constexpr int RT = TYPE == T_Q6_K ? 1 : 2;
    const int tiles = (N + 16 * RT - 1) / (16 * RT);
    hipLaunchKernelGGL((mdec_kernel<TYPE, RT>), dim3(tiles), dim3(256), 0, stream, w, row_bytes, act, y, ldy, M, N);
    return 0;
  }
  // up to 64 rows: 16-row activation tiles; prefill: 64 activation rows x (Q4_K) 128 weight rows
  // per workgroup; Q6_K / Q8_0 keep 64 weight rows (their B operands need twice the registers)
  if (M <= 64) return launch_mt<TYPE, 1, 1>(w, row_bytes, act, y, ldy, M, N, stream);
  constexpr int NT = 1;
  return launch_mt<TYPE, 4, NT>(w, row_bytes, act, y, ldy, M, N, stream);
}

}  // namespace

bool mtile_supported(int type) { return type == T_Q4_K || type == T_Q6_K || type == T_Q8_0; }

int launch_mtile(int type, const uint8_t* w, long long row_bytes, const Act& act, float* y,
                 long long ldy, int m_rows, int n_rows, hipStream_t stream) {
  if (act.q == nullptr || m_rows < 1) return -1;
  switch (type) {
    case T_Q4_K: return launch_mt_type<T_Q4_K>(w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
    case T_Q6_K: return launch_mt_type<T_Q6_K>(w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
    case T_Q8_0: return launch_mt_type<T_Q8_0>(w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
    default: return -1;
  }
}

}  // namespace mxa
