// Decode GEMV for packed GGUF weights: y[m, n] = sum_k x[m, k] * W[n, k] for a few activation
// rows m (a decode step or a small batch of concurrent replies).
//
// Work split. A workgroup (4 waves) owns 16 consecutive weight rows. In every wave, lane
// (r = lane / 4, j = lane % 4) handles quarter j of row r's blocks; the 4 waves take the blocks of
// the row in turn (block b goes to wave b % 4), so the workgroup streams its rows' bytes with
// 16-byte loads. Each wave issues the loads of its next group of 4 blocks before it computes the
// current group, and the first group's loads go out before anything else, so the weight stream
// starts at the first instruction.
//
// Activations. The workgroup copies the Q8_K activations of a chunk of blocks (int8 values,
// bsums, scales; raw floats for IQ4_XS) into LDS once; every lane then reads them from LDS.
//
// Numerics (the reference C kernel's, app/native/src/mx_gemm.c:241-261): K-quant and Q8_0 rows
// use Q8_K activations and exact integer block dots (v_dot4_i32_i8, then a 4-lane integer
// reduction); IQ4_XS uses the raw float activations. The per-block float results go to LDS and
// one thread per (row, activation row) folds them over the blocks in order 0..nb-1 with the same
// fused multiply-adds as the CPU oracle, so K-quant and Q8_0 outputs equal it bit for bit.
#include <type_traits>

#include "mxa_kernels.hpp"

#pragma clang fp contract(off)

namespace mxa {
namespace {

constexpr int kRows = 16;   // weight rows per workgroup
constexpr int kWaves = 4;   // waves per workgroup
constexpr int kGroup = 4;   // blocks a wave loads ahead of computing them
constexpr int kThreads = 64 * kWaves;

// LDS bytes per (activation row, block) staged for a type, and the chunk of blocks staged per
// pass so the staged activations take at most 16 KB.
template <int TYPE>
struct Stage {
  static constexpr int kBytes = TYPE == T_IQ4_XS ? QK * 4 : QK + 32 + 4;
};
template <int TYPE, int MAXM>
struct Chunk {
  static constexpr int raw = 16384 / (MAXM * Stage<TYPE>::kBytes);
  static constexpr int value = raw < 1 ? 1 : raw;
};

// Activations of one chunk in LDS: row m, block bb (0..kChunk) of the chunk.
struct LdsAct {
  const int8_t* q;       // q[(m * chunk + bb) * 256 + e]
  const int16_t* bsums;  // bsums[(m * chunk + bb) * 16 + s]
  const float* x;        // x[(m * chunk + bb) * 256 + e]  (IQ4_XS)
  int chunk;
};

// 16 bytes at a 2-byte aligned address: one aligned 16-byte load (plus one dword when the
// address is not 4-byte aligned) and v_alignbyte. Reads at most 2 bytes on either side of
// [p, p + 16), which callers keep inside the same packed block or its predecessor.
__device__ __forceinline__ u32x4a4 ld16_a2(const uint8_t* p) {
  const uintptr_t a = (uintptr_t)p;
  const uint8_t* base = (const uint8_t*)(a & ~(uintptr_t)3);
  const uint32_t sh = (uint32_t)(a & 3);
  const u32x4a4 v = ld16_stream(base);
  uint32_t e = 0;
  if (sh != 0) e = ld4(base + 16);
  u32x4a4 r;
  r.x = __builtin_amdgcn_alignbyte(v.y, v.x, sh);
  r.y = __builtin_amdgcn_alignbyte(v.z, v.y, sh);
  r.z = __builtin_amdgcn_alignbyte(v.w, v.z, sh);
  r.w = __builtin_amdgcn_alignbyte(e, v.w, sh);
  return r;
}

// Maximum over each row of 16 lanes: quad butterflies, then the half-row and row mirrors.
__device__ __forceinline__ float row16_max(float v) {
  auto dpp = [](float x, auto ctrl) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x),
                                                                 decltype(ctrl)::value, 0xF, 0xF,
                                                                 false));
  };
  v = fmaxf(v, dpp(v, std::integral_constant<int, 0xB1>{}));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp(v, std::integral_constant<int, 0x4E>{}));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp(v, std::integral_constant<int, 0x141>{}));  // row_half_mirror
  v = fmaxf(v, dpp(v, std::integral_constant<int, 0x140>{}));  // row_mirror
  return v;
}

__device__ __forceinline__ int lo16(uint32_t w) { return (int16_t)(w & 0xFFFFu); }
__device__ __forceinline__ int hi16(uint32_t w) { return (int16_t)(w >> 16); }

template <int TYPE>
struct Ops;

// ---- Q4_K: {f16 d, f16 dmin, u8 scales[12], u8 qs[128]}, 144 bytes -------------------------
// Lane j holds qs[32j, 32j+32): low nibbles are sub-block 2j, high nibbles sub-block 2j+1.
template <>
struct Ops<T_Q4_K> {
  static constexpr int kBytes = 144;
  static constexpr bool kHasD = false;
  struct Lane {
    u32x4a4 hdr, qa, qb;
  };
  __device__ static Lane load(const uint8_t* row, int b, int j) {
    const uint8_t* blk = row + (size_t)b * kBytes;
    Lane L;
    L.hdr = ld16_stream(blk);
    L.qa = ld16_stream(blk + 16 + 32 * j);
    L.qb = ld16_stream(blk + 32 + 32 * j);
    return L;
  }
  // V[m] = d * sumi - dmin * summ (mx_dot_k_ssse3.c:150-154), fused as the oracle does.
  template <int MAXM>
  __device__ static void compute(const Lane& L, const LdsAct& a, int bb, int j, int M, float* V,
                                 float& D) {
    const float d = half_to_float(L.hdr.x), dmin = half_to_float(L.hdr.x >> 16);
    const K4Scales s = k4_scales(L.hdr.y, L.hdr.z, L.hdr.w);
    const int sc0 = (int)k4_pick(s.sc_lo, s.sc_hi, 2 * j);
    const int sc1 = (int)k4_pick(s.sc_lo, s.sc_hi, 2 * j + 1);
    const int mn0 = (int)k4_pick(s.mn_lo, s.mn_hi, 2 * j);
    const int mn1 = (int)k4_pick(s.mn_lo, s.mn_hi, 2 * j + 1);
    const uint32_t q[8] = {L.qa.x, L.qa.y, L.qa.z, L.qa.w, L.qb.x, L.qb.y, L.qb.z, L.qb.w};
#pragma unroll
    for (int m = 0; m < MAXM; ++m) {
      if (m < M) {
        const int blk = m * a.chunk + bb;
        const int8_t* q8 = a.q + blk * QK + 64 * j;
        const i32x4a4 x0 = ld16s(q8), x1 = ld16s(q8 + 16), x2 = ld16s(q8 + 32), x3 = ld16s(q8 + 48);
        const int xl[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        const int xh[8] = {x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
        int sl = 0, sh = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          sl = sdot4(q[i] & 0x0F0F0F0Fu, (uint32_t)xl[i], sl);
          sh = sdot4((q[i] >> 4) & 0x0F0F0F0Fu, (uint32_t)xh[i], sh);
        }
        const u32x2a4 bs = *(const u32x2a4*)(a.bsums + blk * 16 + 4 * j);
        int sumi = sc0 * sl + sc1 * sh;
        int summ = mn0 * (lo16(bs.x) + hi16(bs.x)) + mn1 * (lo16(bs.y) + hi16(bs.y));
        sumi = quad_sum(sumi);
        summ = quad_sum(summ);
        V[m] = fmaf(d, (float)sumi, -(dmin * (float)summ));
      }
    }
    D = 0.0f;
  }
  __device__ static float fold(float acc, float xd, float v, float) { return fmaf(xd, v, acc); }
};

// ---- Q6_K: {u8 ql[128], u8 qh[64], i8 scales[16], f16 d}, 210 bytes ------------------------
// Lane j: half h = j/2, lanes l0..l0+15 (l0 = 16 (j%2)) of the four 32-element groups of that
// half, i.e. elements 128h + 32g + l0 + i with scale index 8h + 2g + j%2.
template <>
struct Ops<T_Q6_K> {
  static constexpr int kBytes = 210;
  static constexpr bool kHasD = true;
  struct Lane {
    u32x4a4 A, B, H, S;
    uint32_t d;
  };
  __device__ static Lane load(const uint8_t* row, int b, int j) {
    const uint8_t* blk = row + (size_t)b * kBytes;
    const int h = j >> 1, l0 = 16 * (j & 1);
    Lane L;
    L.A = ld16_a2(blk + 64 * h + l0);
    L.B = ld16_a2(blk + 64 * h + 32 + l0);
    L.H = ld16_a2(blk + 128 + 32 * h + l0);
    L.S = ld16_a2(blk + 192);
    L.d = *(const uint16_t*)(blk + 208);
    return L;
  }
  // V[m] = sumi = sum_s sc_s * sum((u - 32) * q8)  (mx_dot_k_ssse3.c:196-205)
  template <int MAXM>
  __device__ static void compute(const Lane& L, const LdsAct& a, int bb, int j, int M, float* V,
                                 float& D) {
    const int h = j >> 1, jo = j & 1;
    const uint32_t Sa = h ? L.S.z : L.S.x, Sb = h ? L.S.w : L.S.y;
    int sc[4];
    sc[0] = (int8_t)(uint8_t)(Sa >> (8 * jo));
    sc[1] = (int8_t)(uint8_t)(Sa >> (8 * (jo + 2)));
    sc[2] = (int8_t)(uint8_t)(Sb >> (8 * jo));
    sc[3] = (int8_t)(uint8_t)(Sb >> (8 * (jo + 2)));
    const uint32_t A[4] = {L.A.x, L.A.y, L.A.z, L.A.w};
    const uint32_t B[4] = {L.B.x, L.B.y, L.B.z, L.B.w};
    const uint32_t H[4] = {L.H.x, L.H.y, L.H.z, L.H.w};
    uint32_t U[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      U[0][i] = q6_codes<0>(A[i], H[i]);
      U[1][i] = q6_codes<1>(B[i], H[i]);
      U[2][i] = q6_codes<2>(A[i], H[i]);
      U[3][i] = q6_codes<3>(B[i], H[i]);
    }
#pragma unroll
    for (int m = 0; m < MAXM; ++m) {
      if (m < M) {
        const int blk = m * a.chunk + bb;
        const int8_t* q8 = a.q + blk * QK + 128 * h + 16 * jo;
        const u32x4a4 bw = *(const u32x4a4*)(a.bsums + blk * 16 + 8 * h);
        const uint32_t bwv[4] = {bw.x, bw.y, bw.z, bw.w};
        int sumi = 0;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const i32x4a4 x = ld16s(q8 + 32 * g);
          int s = 0;
          s = sdot4(U[g][0], (uint32_t)x.x, s);
          s = sdot4(U[g][1], (uint32_t)x.y, s);
          s = sdot4(U[g][2], (uint32_t)x.z, s);
          s = sdot4(U[g][3], (uint32_t)x.w, s);
          const int bsg = jo ? hi16(bwv[g]) : lo16(bwv[g]);
          sumi += sc[g] * (s - 32 * bsg);
        }
        V[m] = (float)quad_sum(sumi);
      }
    }
    D = half_to_float(L.d);
  }
  // acc += (y.d * d) * sumi  (mx_dot_k_ssse3.c:206)
  __device__ static float fold(float acc, float xd, float v, float d) {
    return fmaf(xd * d, v, acc);
  }
};

// ---- Q8_0: {f16 d, i8 qs[32]}, 34 bytes, eight per 256 values -------------------------------
// Lane j holds Q8_0 blocks 2j and 2j+1 of the 256-value group: 68 bytes at 68j, dword aligned.
template <>
struct Ops<T_Q8_0> {
  static constexpr int kBytes = 272;  // one 256-value group of eight blocks
  static constexpr bool kHasD = false;
  struct Lane {
    uint32_t w[17];
  };
  __device__ static Lane load(const uint8_t* row, int b, int j) {
    const uint8_t* p = row + (size_t)b * kBytes + 68 * j;
    Lane L;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4a4 v = ld16_stream(p + 16 * i);
      L.w[4 * i] = v.x, L.w[4 * i + 1] = v.y, L.w[4 * i + 2] = v.z, L.w[4 * i + 3] = v.w;
    }
    L.w[16] = ld4(p + 64);
    return L;
  }
  // V[m] = block_sum: sum over k = 0..7 of d_k * sum(qs * q8), in k order (mx_dot_q8_0.c:8-18)
  template <int MAXM>
  __device__ static void compute(const Lane& L, const LdsAct& a, int bb, int j, int M, float* V,
                                 float& D) {
    const float d0 = half_to_float(L.w[0]), d1 = half_to_float(L.w[8] >> 16);
    uint32_t qa[8], qb[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      qa[i] = __builtin_amdgcn_alignbyte(L.w[i + 1], L.w[i], 2);
      qb[i] = L.w[9 + i];
    }
    const float dk[8] = {quad_bcast<0>(d0), quad_bcast<0>(d1), quad_bcast<1>(d0),
                         quad_bcast<1>(d1), quad_bcast<2>(d0), quad_bcast<2>(d1),
                         quad_bcast<3>(d0), quad_bcast<3>(d1)};
#pragma unroll
    for (int m = 0; m < MAXM; ++m) {
      if (m < M) {
        const int8_t* q8 = a.q + (m * a.chunk + bb) * QK + 64 * j;
        const i32x4a4 x0 = ld16s(q8), x1 = ld16s(q8 + 16), x2 = ld16s(q8 + 32), x3 = ld16s(q8 + 48);
        const int xa[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        const int xb[8] = {x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
        int p0 = 0, p1 = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          p0 = sdot4(qa[i], (uint32_t)xa[i], p0);
          p1 = sdot4(qb[i], (uint32_t)xb[i], p1);
        }
        const int pk[8] = {quad_bcast<0>(p0), quad_bcast<0>(p1), quad_bcast<1>(p0),
                           quad_bcast<1>(p1), quad_bcast<2>(p0), quad_bcast<2>(p1),
                           quad_bcast<3>(p0), quad_bcast<3>(p1)};
        float bs = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) bs = fmaf(dk[k], (float)pk[k], bs);
        V[m] = bs;
      }
    }
    D = 0.0f;
  }
  __device__ static float fold(float acc, float xd, float v, float) { return fmaf(xd, v, acc); }
};

// ---- IQ4_XS: {f16 d, u16 scales_h, u8 scales_l[4], u8 qs[128]}, 136 bytes --------------------
// Lane j holds sub-blocks 2j and 2j+1 (qs[32j, 32j+32)); activations are the raw floats.
template <>
struct Ops<T_IQ4_XS> {
  static constexpr int kBytes = 136;
  static constexpr bool kHasD = false;
  struct Lane {
    u32x2a4 hdr;
    u32x4a4 qa, qb;
  };
  __device__ static Lane load(const uint8_t* row, int b, int j) {
    const uint8_t* blk = row + (size_t)b * kBytes;
    Lane L;
    L.hdr = ld8(blk);
    L.qa = ld16_stream(blk + 8 + 32 * j);
    L.qb = ld16_stream(blk + 24 + 32 * j);
    return L;
  }
  // V[m] = sum over the block of x * (dl * grid) as dl * (sum x * grid) per sub-block
  // (mx_dot_f32.c:42-55 up to the order of the float additions).
  template <int MAXM>
  __device__ static void compute(const Lane& L, const LdsAct& a, int bb, int j, int M, float* V,
                                 float& D) {
    const float d = half_to_float(L.hdr.x);
    const uint32_t sh = L.hdr.x >> 16, sl = L.hdr.y;
    const int ls0 = (int)(((sl >> (8 * j)) & 15u) | (((sh >> (4 * j)) & 3u) << 4));
    const int ls1 = (int)(((sl >> (8 * j + 4)) & 15u) | (((sh >> (4 * j + 2)) & 3u) << 4));
    const float dl0 = d * (float)(ls0 - 32), dl1 = d * (float)(ls1 - 32);
    const uint32_t qs[8] = {L.qa.x, L.qa.y, L.qa.z, L.qa.w, L.qb.x, L.qb.y, L.qb.z, L.qb.w};
    uint32_t gl[8], gh[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      gl[i] = iq4_lookup4(qs[i] & 0x0F0F0F0Fu);
      gh[i] = iq4_lookup4((qs[i] >> 4) & 0x0F0F0F0Fu);
    }
#pragma unroll
    for (int m = 0; m < MAXM; ++m) {
      if (m < M) {
        const float* xs = a.x + (m * a.chunk + bb) * QK + 64 * j;
        float p[2] = {0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float4 xl = *(const float4*)(xs + 32 * t + 4 * i);
            const float4 xh = *(const float4*)(xs + 32 * t + 16 + 4 * i);
            const uint32_t g0 = gl[4 * t + i], g1 = gh[4 * t + i];
            p[t] = fmaf(xl.x, sbyte_f<0>(g0), p[t]);
            p[t] = fmaf(xl.y, sbyte_f<1>(g0), p[t]);
            p[t] = fmaf(xl.z, sbyte_f<2>(g0), p[t]);
            p[t] = fmaf(xl.w, sbyte_f<3>(g0), p[t]);
            p[t] = fmaf(xh.x, sbyte_f<0>(g1), p[t]);
            p[t] = fmaf(xh.y, sbyte_f<1>(g1), p[t]);
            p[t] = fmaf(xh.z, sbyte_f<2>(g1), p[t]);
            p[t] = fmaf(xh.w, sbyte_f<3>(g1), p[t]);
          }
        }
        V[m] = quad_sum(fmaf(dl1, p[1], dl0 * p[0]));
      }
    }
    D = 0.0f;
  }
  __device__ static float fold(float acc, float, float v, float) { return acc + v; }
};

// FUSEQ: the workgroup quantizes the float activations to Q8_K itself (16 lanes per 256-value
// block, the arithmetic of quantize_q8k_kernel), instead of reading them from the workspace; for
// M <= 4 this saves a kernel launch per projection.
template <int TYPE, int MAXM, bool PIPE, bool FUSEQ>
__global__ __launch_bounds__(256) void gemv_kernel(const uint8_t* w,
                                                   long long row_bytes, Act act,
                                                   float* __restrict__ y, long long ldy, int M,
                                                   int N) {
  using O = Ops<TYPE>;
  static_assert(!FUSEQ || (TYPE != T_IQ4_XS && MAXM <= 4), "fused quantization: M <= 4");
  constexpr int kChunk = FUSEQ ? 16 / MAXM : Chunk<TYPE, MAXM>::value;
  constexpr bool kFloatAct = TYPE == T_IQ4_XS;
  constexpr int kQBytes = kChunk * (kFloatAct ? QK * 4 : QK);  // staged bytes per row m
  constexpr int kQLoads = (kQBytes + kThreads * 16 - 1) / (kThreads * 16);
  constexpr int kBLoads = kFloatAct ? 0 : (kChunk * 32 + kThreads * 16 - 1) / (kThreads * 16);
  __shared__ __align__(16) int8_t Xq[kFloatAct ? 16 : MAXM * kChunk * QK];
  __shared__ __align__(16) int16_t Xb[kFloatAct ? 8 : MAXM * kChunk * 16];
  __shared__ float Xd[kFloatAct ? 1 : MAXM * kChunk];
  __shared__ __align__(16) float Xf[kFloatAct ? MAXM * kChunk * QK : 4];
  __shared__ float Vs[MAXM][kChunk][kRows];
  __shared__ float Ds[O::kHasD ? kChunk : 1][kRows];

  const int n0 = xcd_tile(blockIdx.x, gridDim.x) * kRows;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int r = lane >> 2, j = lane & 3;
  const int n = min(n0 + r, N - 1);  // rows past N recompute row N-1; never stored
  const uint8_t* row = w + (size_t)n * row_bytes;
  const int nb = act.nb;
  const int fr = tid & (kRows - 1), fm = tid >> 4;
  const LdsAct la{Xq, Xb, Xf, kChunk};
  float acc = 0.0f;

  for (int c0 = 0; c0 < nb; c0 += kChunk) {
    const int cn = min(kChunk, nb - c0);
    // this wave's blocks of the chunk are bb = wave + kWaves * i, i < mine
    const int mine = cn > wave ? (cn - wave + kWaves - 1) / kWaves : 0;
    // Every load below is unconditional, at an address clamped into its buffer (a clamped
    // activation piece is stored twice to the same place; a clamped weight block is loaded and
    // not used), so the compiler issues them back to back without branches.

    // 1. this chunk's activations (all M rows) into registers, before the weight loads, so
    //    that waiting for them (loads retire in order) never waits for HBM.
    const int q_per_m = cn * (kFloatAct ? QK * 4 : QK);
    const uint8_t* q_src = kFloatAct ? (const uint8_t*)(act.x + (size_t)c0 * QK)
                                     : (const uint8_t*)(act.q + (size_t)c0 * QK);
    const size_t q_row = (size_t)act.k * (kFloatAct ? 4 : 1);
    u32x4a4 sq[MAXM][kQLoads];
    u32x4a4 sb[MAXM][kBLoads > 0 ? kBLoads : 1];
    float sd[MAXM];
    // FUSEQ: lanes 16g..16g+15 own row m = g / kChunk, block bb = g % kChunk; lane part p of the
    // group holds elements 16p..16p+15 of that block
    const int fq_g = tid >> 4, fq_p = tid & 15;
    const int fq_m = min(fq_g / kChunk, M - 1), fq_bb = min(fq_g % kChunk, cn - 1);
    float4 fx[FUSEQ ? 4 : 1];
    if constexpr (FUSEQ) {
      const float* src = act.x + (size_t)fq_m * act.k + (size_t)(c0 + fq_bb) * QK + 16 * fq_p;
#pragma unroll
      for (int i = 0; i < 4; ++i) fx[i] = *(const float4*)(src + 4 * i);
    }
#pragma unroll
    for (int m = 0; m < (FUSEQ ? 0 : MAXM); ++m) {
      const int mc = min(m, M - 1);
#pragma unroll
      for (int t = 0; t < kQLoads; ++t)
        sq[m][t] = ld16(q_src + mc * q_row + min(tid * 16 + t * kThreads * 16, q_per_m - 16));
      if constexpr (!kFloatAct) {
#pragma unroll
        for (int t = 0; t < kBLoads; ++t)
          sb[m][t] = ld16((const uint8_t*)act.bsums + ((size_t)mc * nb + c0) * 32 +
                          min(tid * 16 + t * kThreads * 16, cn * 32 - 16));
        sd[m] = act.d[(size_t)mc * nb + c0 + min(tid, cn - 1)];
      }
    }

    // 2. the weight loads of this wave's first group of blocks
    typename O::Lane cur[kGroup];
#pragma unroll
    for (int u = 0; u < kGroup; ++u)
      cur[u] = O::load(row, c0 + min(wave + kWaves * u, cn - 1), j);

    // keep every load above issued before the first wait below (the scheduler would otherwise
    // interleave the LDS stores, and their waits, with the weight loads)
    __builtin_amdgcn_sched_barrier(0);

    // 3. activations into LDS, laid out [m][block of the chunk][...]
    if constexpr (FUSEQ) {
      // Q8_K of this lane's 16 values (app/native/src/mx_common.c:42-69, as quantize_q8k_kernel)
      const float v[16] = {fx[0].x, fx[0].y, fx[0].z, fx[0].w, fx[1].x, fx[1].y, fx[1].z, fx[1].w,
                           fx[2].x, fx[2].y, fx[2].z, fx[2].w, fx[3].x, fx[3].y, fx[3].z, fx[3].w};
      float amax = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[i]));
      amax = row16_max(amax);
      int q[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) q[i] = 0;
      if (amax != 0.0f) {
        const float iscale = 127.0f / amax;
#pragma unroll
        for (int i = 0; i < 16; ++i) q[i] = (int)fminf(fmaxf(rintf(v[i] * iscale), -127.0f), 127.0f);
      }
      int bsum = 0;
      u32x4a4 packed;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        packed[i] = (uint32_t)(q[4 * i] & 0xFF) | ((uint32_t)(q[4 * i + 1] & 0xFF) << 8) |
                    ((uint32_t)(q[4 * i + 2] & 0xFF) << 16) | ((uint32_t)(q[4 * i + 3] & 0xFF) << 24);
        bsum += q[4 * i] + q[4 * i + 1] + q[4 * i + 2] + q[4 * i + 3];
      }
      *(u32x4a4*)(Xq + fq_m * kQBytes + fq_bb * QK + 16 * fq_p) = packed;
      Xb[(fq_m * kChunk + fq_bb) * 16 + fq_p] = (int16_t)bsum;
      if (fq_p == 0) Xd[fq_m * kChunk + fq_bb] = amax / 127.0f;
    }
#pragma unroll
    for (int m = 0; m < (FUSEQ ? 0 : MAXM); ++m) {
      const int mc = min(m, M - 1);
#pragma unroll
      for (int t = 0; t < kQLoads; ++t) {
        const int o = min(tid * 16 + t * kThreads * 16, q_per_m - 16);
        uint8_t* dst = kFloatAct ? (uint8_t*)Xf + mc * kQBytes + o : (uint8_t*)Xq + mc * kQBytes + o;
        *(u32x4a4*)dst = sq[m][t];
      }
      if constexpr (!kFloatAct) {
#pragma unroll
        for (int t = 0; t < kBLoads; ++t)
          *(u32x4a4*)((uint8_t*)Xb + mc * kChunk * 32 +
                      min(tid * 16 + t * kThreads * 16, cn * 32 - 16)) = sb[m][t];
        Xd[mc * kChunk + min(tid, cn - 1)] = sd[m];
      }
    }
    __syncthreads();

    // 4. compute, one group of kGroup blocks at a time; the first group runs on every path (so
    //    its loads stay above the barrier), and with PIPE the next group's weight loads are in
    //    flight while a group is computed
    for (int g = 0;; g += kGroup) {
      typename O::Lane nxt[PIPE ? kGroup : 1];
      if constexpr (PIPE) {
#pragma unroll
        for (int u = 0; u < kGroup; ++u)
          nxt[u] = O::load(row, c0 + min(wave + kWaves * (g + kGroup + u), cn - 1), j);
      }
#pragma unroll
      for (int u = 0; u < kGroup; ++u) {
        // computed on every path (on a clamped, valid block past `mine`) so that the compiler
        // keeps the weight loads where they are issued; only the store is conditional
        const int bb = wave + kWaves * (g + u);
        const int bbc = min(bb, cn - 1);
        float V[MAXM];
        float D;
        O::template compute<MAXM>(cur[u], la, bbc, j, M, V, D);
        if (j == 0 && g + u < mine) {
#pragma unroll
          for (int m = 0; m < MAXM; ++m)
            if (m < M) Vs[m][bb][r] = V[m];
          if (O::kHasD) Ds[O::kHasD ? bb : 0][r] = D;
        }
      }
      if (!PIPE || g + kGroup >= mine) break;  // without PIPE a wave owns one group (launch_m)
      if constexpr (PIPE) {
#pragma unroll
        for (int u = 0; u < kGroup; ++u) cur[u] = nxt[u];
      }
    }
    __syncthreads();
    if (fm < M) {
#pragma unroll 8
      for (int bb = 0; bb < cn; ++bb)
        acc = O::fold(acc, kFloatAct ? 0.0f : Xd[kFloatAct ? 0 : fm * kChunk + bb], Vs[fm][bb][fr],
                      Ds[O::kHasD ? bb : 0][fr]);
    }
    __syncthreads();
  }
  if (fm < M && n0 + fr < N) y[(size_t)fm * ldy + n0 + fr] = acc;
}

template <int TYPE, int MAXM, bool FUSEQ>
void launch_m(const uint8_t* w, long long row_bytes, const Act& act, float* y, long long ldy,
              int M, int N, hipStream_t stream) {
  const int tiles = (N + kRows - 1) / kRows;
  // Without the prefetch buffer a wave must own at most kGroup blocks of every chunk.
  const int chunk = min(act.nb, FUSEQ ? 16 / MAXM : Chunk<TYPE, MAXM>::value);
  if (chunk <= kWaves * kGroup)
    hipLaunchKernelGGL((gemv_kernel<TYPE, MAXM, false, FUSEQ>), dim3(tiles), dim3(kThreads), 0,
                       stream, w, row_bytes, act, y, ldy, M, N);
  else
    hipLaunchKernelGGL((gemv_kernel<TYPE, MAXM, true, FUSEQ>), dim3(tiles), dim3(kThreads), 0,
                       stream, w, row_bytes, act, y, ldy, M, N);
}

template <int TYPE, int MAXM>
void launch_m(const uint8_t* w, long long row_bytes, const Act& act, float* y, long long ldy,
              int M, int N, hipStream_t stream) {
  launch_m<TYPE, MAXM, false>(w, row_bytes, act, y, ldy, M, N, stream);
}

template <int TYPE>
void launch_type(const uint8_t* w, long long row_bytes, const Act& act, float* y, long long ldy,
                 int M, int N, hipStream_t stream) {
  if constexpr (TYPE != T_IQ4_XS) {
    if (act.q == nullptr) {
      // fused quantization (the caller checked M <= 4 and passed the float activations)
      if (M == 1) launch_m<TYPE, 1, true>(w, row_bytes, act, y, ldy, M, N, stream);
      else if (M == 2) launch_m<TYPE, 2, true>(w, row_bytes, act, y, ldy, M, N, stream);
      else launch_m<TYPE, 4, true>(w, row_bytes, act, y, ldy, M, N, stream);
      return;
    }
  }
  for (int m0 = 0; m0 < M; m0 += 16) {
    const int mm = min(16, M - m0);
    Act a = act;
    a.q = act.q ? act.q + (size_t)m0 * act.k : nullptr;
    a.d = act.d ? act.d + (size_t)m0 * act.nb : nullptr;
    a.bsums = act.bsums ? act.bsums + (size_t)m0 * act.nb * 16 : nullptr;
    a.x = act.x ? act.x + (size_t)m0 * act.k : nullptr;
    float* yy = y + (size_t)m0 * ldy;
    if (mm == 1) launch_m<TYPE, 1>(w, row_bytes, a, yy, ldy, mm, N, stream);
    else if (mm == 2) launch_m<TYPE, 2>(w, row_bytes, a, yy, ldy, mm, N, stream);
    else if (mm <= 4) launch_m<TYPE, 4>(w, row_bytes, a, yy, ldy, mm, N, stream);
    else if (mm <= 8) launch_m<TYPE, 8>(w, row_bytes, a, yy, ldy, mm, N, stream);
    else launch_m<TYPE, 16>(w, row_bytes, a, yy, ldy, mm, N, stream);
  }
}

}  // namespace

int launch_gemv(int type, const uint8_t* w, long long row_bytes, const Act& act, float* y,
                long long ldy, int m_rows, int n_rows, hipStream_t stream) {
  switch (type) {
    case T_Q4_K: launch_type<T_Q4_K>(w, row_bytes, act, y, ldy, m_rows, n_rows, stream); return 0;
    case T_Q6_K: launch_type<T_Q6_K>(w, row_bytes, act, y, ldy, m_rows, n_rows, stream); return 0;
    case T_Q8_0: launch_type<T_Q8_0>(w, row_bytes, act, y, ldy, m_rows, n_rows, stream); return 0;
    case T_IQ4_XS:
      launch_type<T_IQ4_XS>(w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
      return 0;
    default: return -1;
  }
}

}  // namespace mxa
