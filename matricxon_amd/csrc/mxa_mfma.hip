// Q4_K matmul on the matrix cores for batched decode (up to 16 activation rows per pass).
//
// Operands. A (16 x 64 int8, rows = activation rows m) is the Q8_K activations, staged in LDS per
// chunk of blocks. B (64 x 16 int8, columns = weight rows n) is built in registers from the
// packed bytes: a Q4_K block's value is (d*sc)*u - dmin*m with u a 4-bit code and sc, m six-bit
// sub-block scale and min, and the integer part sum(sc*u*q8) of the reference's block dot
// (app/native/src/mx_dot_k_ssse3.c:109-157) is computed exactly as
//     8 * sum((sc >> 3) * u * q8) + sum((sc & 7) * u * q8)
// where each plane's bytes (sc >> 3) * u and (sc & 7) * u are at most 7 * 15 = 105 and so fit
// int8: two passes of v_mfma_i32_16x16x64_i8 over the block's 256 values, with a shift in
// between. The min term sum(m * bsums) is one v_mfma_f32_16x16x16_f16 of the 16 bsums (|.| <= 2032)
// against the mins (<= 63), both exact in fp16, with an exact fp32 result (< 2^24).
//
// Each lane of a wave supplies row (lane % 16) and k-group (lane / 16) of both operands; the
// k-group g of a block is qs[32g, 32g+32), i.e. elements 64g..64g+63 (sub-blocks 2g and 2g+1),
// split over the four MFMAs t = 0..3 as elements 64g + 16t + (0..15) for A and B alike, so the
// contraction runs over exactly the block's 256 values whatever order the hardware uses inside a
// k-group. The output lane l holds column n = l % 16, rows m = 4 (l / 16) + i.
//
// Numerics: per (m, n, block) T = fmaf(d, sumi, -(dmin * summ)); the outputs are folded over the
// blocks in order with acc = fmaf(xd, T, acc), the CPU oracle's order, so results are bit-identical
// to it and to the dot4 GEMV.
#include "mxa_kernels.hpp"

#pragma clang fp contract(off)

namespace mxa {
namespace {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));

constexpr int kTiles = 2;                 // 16-row weight tiles per workgroup
constexpr int kCh = 8;                    // blocks per LDS chunk
constexpr int kWaves = 4;
constexpr int kBlocksPerWave = kCh / kWaves;
constexpr int kQStride = kCh * QK + 16;   // LDS bytes per activation row (16 B of padding keeps
                                          // the 16 rows of an A read in distinct banks)
constexpr int kBStride = kCh * 16 + 8;    // LDS halves per activation row of bsums

struct Q4Lane {
  u32x4a4 hdr, qa, qb;
};

__device__ __forceinline__ Q4Lane load_q4(const uint8_t* row, int b, int g) {
  const uint8_t* blk = row + (size_t)b * 144;
  Q4Lane L;
  L.hdr = ld16_stream(blk);
  L.qa = ld16_stream(blk + 16 + 32 * g);
  L.qb = ld16_stream(blk + 32 + 32 * g);
  return L;
}

// Each byte of u times s (s * byte <= 255, so no carry crosses a byte): v_pk_mul_lo_u16.
__device__ __forceinline__ uint32_t mul_bytes(uint32_t u, uint32_t s) {
  const u16x2 a = __builtin_bit_cast(u16x2, u);
  const u16x2 b = {(uint16_t)s, (uint16_t)s};
  return __builtin_bit_cast(uint32_t, a * b);
}

__device__ __forceinline__ i32x4 as_i32x4(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  return i32x4{(int)a, (int)b, (int)c, (int)d};
}

// T values of one (16 weight rows) x (16 activation rows) x (one block) tile.
__device__ __forceinline__ f32x4 q4k_tile(const Q4Lane& L, const int8_t* Aq_row, const _Float16* Ab_row,
                                          int bb, int g) {
  const float d = half_to_float(L.hdr.x), dmin = half_to_float(L.hdr.x >> 16);
  const K4Scales s = k4_scales(L.hdr.y, L.hdr.z, L.hdr.w);
  const uint32_t sc0 = k4_pick(s.sc_lo, s.sc_hi, 2 * g), sc1 = k4_pick(s.sc_lo, s.sc_hi, 2 * g + 1);
  const uint32_t mn0 = k4_pick(s.mn_lo, s.mn_hi, 2 * g), mn1 = k4_pick(s.mn_lo, s.mn_hi, 2 * g + 1);
  const uint32_t sh0 = sc0 >> 3, sl0 = sc0 & 7, sh1 = sc1 >> 3, sl1 = sc1 & 7;
  const uint32_t q[8] = {L.qa.x, L.qa.y, L.qa.z, L.qa.w, L.qb.x, L.qb.y, L.qb.z, L.qb.w};
  uint32_t u[4][4];  // MFMA t: 16 codes as bytes
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    u[0][i] = q[i] & 0x0F0F0F0Fu;
    u[1][i] = q[4 + i] & 0x0F0F0F0Fu;
    u[2][i] = (q[i] >> 4) & 0x0F0F0F0Fu;
    u[3][i] = (q[4 + i] >> 4) & 0x0F0F0F0Fu;
  }
  i32x4 a[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) a[t] = *(const i32x4*)(Aq_row + bb * QK + 64 * g + 16 * t);
  i32x4 acc = {0, 0, 0, 0};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t sh = t < 2 ? sh0 : sh1;
    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(
        a[t], as_i32x4(mul_bytes(u[t][0], sh), mul_bytes(u[t][1], sh), mul_bytes(u[t][2], sh),
                       mul_bytes(u[t][3], sh)),
        acc, 0, 0, 0);
  }
  acc = acc * 8;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t sl = t < 2 ? sl0 : sl1;
    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(
        a[t], as_i32x4(mul_bytes(u[t][0], sl), mul_bytes(u[t][1], sl), mul_bytes(u[t][2], sl),
                       mul_bytes(u[t][3], sl)),
        acc, 0, 0, 0);
  }
  // summ = sum over the 16 bsums of min_{s/2} * bsum: A = bsums (k = 4g..4g+3), B = mins.
  const f16x4 amin = *(const f16x4*)(Ab_row + bb * 16 + 4 * g);
  const _Float16 m0 = (_Float16)(float)mn0, m1 = (_Float16)(float)mn1;
  const f16x4 bmin = {m0, m0, m1, m1};
  const f32x4 summ = __builtin_amdgcn_mfma_f32_16x16x16f16(amin, bmin, f32x4{0, 0, 0, 0}, 0, 0, 0);
  f32x4 T;
#pragma unroll
  for (int i = 0; i < 4; ++i) T[i] = fmaf(d, (float)acc[i], -(dmin * summ[i]));
  return T;
}

__global__ __launch_bounds__(256) void q4k_mfma_decode_kernel(const uint8_t* w, long long row_bytes,
                                                              Act act, float* __restrict__ y,
                                                              long long ldy, int M, int N) {
  __shared__ __align__(16) int8_t Aq[16 * kQStride];
  __shared__ __align__(16) _Float16 Ab[16 * kBStride];
  __shared__ float Ax[kCh][16];
  __shared__ float Tp[kTiles][kCh][16][16];

  const int n0 = xcd_tile(blockIdx.x, gridDim.x) * 16 * kTiles;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int ln = lane & 15, g = lane >> 4;
  const uint8_t* rows[kTiles];
#pragma unroll
  for (int t = 0; t < kTiles; ++t) rows[t] = w + (size_t)min(n0 + 16 * t + ln, N - 1) * row_bytes;
  const int nb = act.nb;
  float acc[2] = {0.0f, 0.0f};

  // weight loads of the first chunk (blocks wave, wave + 4 of the chunk, both tiles)
  Q4Lane cur[kBlocksPerWave][kTiles];
  {
    const int cn = min(kCh, nb);
#pragma unroll
    for (int i = 0; i < kBlocksPerWave; ++i)
#pragma unroll
      for (int t = 0; t < kTiles; ++t)
        cur[i][t] = load_q4(rows[t], min(wave + kWaves * i, cn - 1), g);
  }

  for (int c0 = 0; c0 < nb; c0 += kCh) {
    const int cn = min(kCh, nb - c0);
    // 1. activations of the chunk into registers (clamped addresses: rows >= M repeat row M-1,
    //    blocks >= cn repeat block cn-1; those results are never stored)
    u32x4a4 sq[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int p = tid + 256 * s, r = p >> 7, off = min((p & 127) * 16, cn * QK - 16);
      sq[s] = ld16((const uint8_t*)(act.q + (size_t)min(r, M - 1) * act.k + (size_t)c0 * QK) + off);
    }
    const int br = tid >> 4, bbb = min((tid & 15) >> 1, cn - 1), bhalf = tid & 1;
    const u32x4a4 sbs = ld16((const uint8_t*)(act.bsums + ((size_t)min(br, M - 1) * nb + c0 + bbb) * 16 + 8 * bhalf));
    const int xr = (tid >> 3) & 15, xbb = min(tid & 7, cn - 1);
    const float sxd = act.d[(size_t)min(xr, M - 1) * nb + c0 + xbb];

    // 2. weight loads of the next chunk
    Q4Lane nxt[kBlocksPerWave][kTiles];
    const int c1 = c0 + kCh;
    if (c1 < nb) {
      const int cn1 = min(kCh, nb - c1);
#pragma unroll
      for (int i = 0; i < kBlocksPerWave; ++i)
#pragma unroll
        for (int t = 0; t < kTiles; ++t)
          nxt[i][t] = load_q4(rows[t], c1 + min(wave + kWaves * i, cn1 - 1), g);
    }
    __builtin_amdgcn_sched_barrier(0);

    // 3. into LDS
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int p = tid + 256 * s, r = p >> 7, off = min((p & 127) * 16, cn * QK - 16);
      *(u32x4a4*)(Aq + r * kQStride + off) = sq[s];
    }
    {
      f16x8 h;
      const uint32_t wv[4] = {sbs.x, sbs.y, sbs.z, sbs.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        h[2 * i] = (_Float16)(float)(int16_t)(wv[i] & 0xFFFFu);
        h[2 * i + 1] = (_Float16)(float)(int16_t)(wv[i] >> 16);
      }
      *(f16x8*)(Ab + br * kBStride + bbb * 16 + 8 * bhalf) = h;
    }
    if (tid < 128) Ax[xbb][xr] = sxd;
    __syncthreads();

    // 4. this wave's blocks of the chunk, both tiles
#pragma unroll
    for (int i = 0; i < kBlocksPerWave; ++i) {
      const int bb = wave + kWaves * i;
      const int bbc = min(bb, cn - 1);
#pragma unroll
      for (int t = 0; t < kTiles; ++t) {
        const f32x4 T = q4k_tile(cur[i][t], Aq + ln * kQStride, Ab + ln * kBStride, bbc, g);
        if (bb < cn) {
#pragma unroll
          for (int e = 0; e < 4; ++e) Tp[t][bb][4 * g + e][ln] = T[e];
        }
      }
    }
    __syncthreads();
    // 5. fold the chunk's blocks in order: thread -> outputs (tile, m, n) = idx >> 8, (idx >> 4) & 15, idx & 15
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int idx = tid + 256 * k, t = idx >> 8, m = (idx >> 4) & 15, n = idx & 15;
      for (int bb = 0; bb < cn; ++bb) acc[k] = fmaf(Ax[bb][m], Tp[t][bb][m][n], acc[k]);
    }
    __syncthreads();
    if (c1 < nb) {
#pragma unroll
      for (int i = 0; i < kBlocksPerWave; ++i)
#pragma unroll
        for (int t = 0; t < kTiles; ++t) cur[i][t] = nxt[i][t];
    }
  }
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int idx = tid + 256 * k, t = idx >> 8, m = (idx >> 4) & 15, n = n0 + 16 * t + (idx & 15);
    if (m < M && n < N) y[(size_t)m * ldy + n] = acc[k];
  }
}

}  // namespace

bool mfma_decode_supported(int type, int m_rows) { return type == T_Q4_K && m_rows >= 1 && m_rows <= 16; }

int launch_mfma_decode(int type, const uint8_t* w, long long row_bytes, const Act& act, float* y,
                       long long ldy, int m_rows, int n_rows, hipStream_t stream) {
  if (!mfma_decode_supported(type, m_rows) || act.q == nullptr) return -1;
  const int tiles = (n_rows + 16 * kTiles - 1) / (16 * kTiles);
  hipLaunchKernelGGL(q4k_mfma_decode_kernel, dim3(tiles), dim3(256), 0, stream, w, row_bytes, act,
                     y, ldy, m_rows, n_rows);
  return 0;
}

int launch_matmul(int type, const uint8_t* w, long long row_bytes, const Act& act, float* y,
                  long long ldy, int m_rows, int n_rows, hipStream_t stream) {
  if (m_rows <= kFusedQuantMaxRows)
    return launch_gemv_lpb(type, w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
  if (act.q != nullptr && mtile_supported(type))
    return launch_mtile(type, w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
  if (type == T_IQ4_XS && m_rows >= kIq4MfmaMinRows && act.xsplit != nullptr)
    return launch_iq4_prefill(w, row_bytes, act.x, act.xsplit, y, ldy, m_rows, act.k, n_rows, stream);
  if (type == T_IQ4_XS) {
    // float activations: the decode kernel in passes of kFusedQuantMaxRows rows (the summation
    // order of the decode kernels, so a row's result does not depend on a batch of up to 16)
    for (int m0 = 0; m0 < m_rows; m0 += kFusedQuantMaxRows) {
      Act a = act;
      a.q = nullptr;
      a.x = act.x + (size_t)m0 * act.k;
      const int st = launch_gemv_lpb(type, w, row_bytes, a, y + (size_t)m0 * ldy, ldy,
                                     min(kFusedQuantMaxRows, m_rows - m0), n_rows, stream);
      if (st != 0) return st;
    }
    return 0;
  }
  if (act.q != nullptr && mfma_decode_supported(type, 1)) {
    // passes of up to 16 activation rows on the matrix cores
    for (int m0 = 0; m0 < m_rows; m0 += 16) {
      const int mm = min(16, m_rows - m0);
      Act a = act;
      a.q = act.q + (size_t)m0 * act.k;
      a.d = act.d + (size_t)m0 * act.nb;
      a.bsums = act.bsums + (size_t)m0 * act.nb * 16;
      a.x = act.x ? act.x + (size_t)m0 * act.k : nullptr;
      const int st = launch_mfma_decode(type, w, row_bytes, a, y + (size_t)m0 * ldy, ldy, mm,
                                        n_rows, stream);
      if (st != 0) return st;
    }
    return 0;
  }
  return launch_gemv(type, w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
}

}  // namespace mxa
