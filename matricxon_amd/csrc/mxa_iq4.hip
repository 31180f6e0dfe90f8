// IQ4_XS prefill (M > 16) on the matrix cores.
//
// The reference multiplies fp32 activations by dl * K[q] (app/native/src/mx_dot_f32.c:32-58, K the
// IQ4_NL grid, dl = d * (ls - 32) per 32-value sub-block). Here x is first split into two bf16
// parts, x = hi + lo (hi = x rounded to bf16, lo = the rest rounded to bf16; relative error of the
// pair about 2^-17), written to the workspace by split_bf16_kernel. The grid values are small
// integers, exact in bf16, so v_mfma_f32_16x16x32_bf16 on (hi, K) then (lo, K) gives sum(K * x) of
// one sub-block per MFMA pair: with A = x (16 activation rows x 32 k) and B = K (32 k x 16 weight
// rows), lane l supplies row (l % 16) and k-group g = l / 16, i.e. elements 32 t + 8 g + (0..7) of
// sub-block t. The sub-block scale dl is applied in fp32 after the MFMA. The result meets the
// float tolerance against the reference (rel-L2 <= 1e-4); its summation order differs from the
// decode kernels', which is why batches of up to 16 rows stay on those.
#include "mxa_kernels.hpp"

#pragma clang fp contract(off)

namespace mxa {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // 16-byte aligned

constexpr int kXStride = QK * 2 + 16;      // LDS bytes per activation row (bf16), padded

// bf16 bits of x rounded to nearest even (NaN stays NaN, overflow gives +-Inf).
__device__ __forceinline__ uint32_t bf16_rne(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

__global__ __launch_bounds__(256) void split_bf16_kernel(const float* __restrict__ x,
                                                         uint16_t* __restrict__ hi,
                                                         uint16_t* __restrict__ lo, long long n4) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n4) return;
  const float4 v = ((const float4*)x)[i];
  const float e[4] = {v.x, v.y, v.z, v.w};
  uint32_t h[4], l[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    h[k] = bf16_rne(e[k]);
    const float rest = e[k] - __builtin_bit_cast(float, h[k] << 16);  // exact in fp32
    l[k] = bf16_rne(rest);
  }
  ((uint2*)hi)[i] = uint2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
  ((uint2*)lo)[i] = uint2{l[0] | (l[1] << 16), l[2] | (l[3] << 16)};
}

// Eight bf16 grid values (as four dwords) for the eight 4-bit indices in the low nibbles of the
// bytes of (a, b).
__device__ __forceinline__ u32x4a4 grid_bf16x8(uint32_t a, uint32_t b) {
  const uint32_t ka = iq4_lookup4(a), kb = iq4_lookup4(b);
  uint32_t f[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[i] = __builtin_bit_cast(uint32_t, (float)(int8_t)(uint8_t)(ka >> (8 * i)));
    f[4 + i] = __builtin_bit_cast(uint32_t, (float)(int8_t)(uint8_t)(kb >> (8 * i)));
  }
  // bf16 = the top half of an fp32 holding a small integer (exact); two per dword
  return u32x4a4{__builtin_amdgcn_perm(f[1], f[0], 0x07060302u), __builtin_amdgcn_perm(f[3], f[2], 0x07060302u),
                 __builtin_amdgcn_perm(f[5], f[4], 0x07060302u), __builtin_amdgcn_perm(f[7], f[6], 0x07060302u)};
}

struct IQ4W {
  uint32_t hdr[2];   // d | scales_h, scales_l
  uint32_t qs[16];   // for sub-block t: qs[16 t + 8 (g & 1) ..] as two dwords
};

__device__ __forceinline__ IQ4W load_iq4(const uint8_t* row, int b, int g) {
  const uint8_t* blk = row + (size_t)b * 136;  // 8-byte aligned blocks (4-byte aligned rows)
  IQ4W L;
  const u32x2a4 h = ld8(blk);
  L.hdr[0] = h.x, L.hdr[1] = h.y;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const u32x2a4 v = ld8(blk + 8 + 16 * t + 8 * (g & 1));
    L.qs[2 * t] = v.x, L.qs[2 * t + 1] = v.y;
  }
  return L;
}

// A workgroup takes 16 NT weight rows per wave (8 waves) x 16 MT activation rows. The activations
// of a block (bf16 hi and lo, 2 x 512 B per row) go to one of two LDS buffers: the next block's
// are loaded into registers while the current block is computed and written to the other buffer
// afterwards, so one barrier per block suffices (a buffer is rewritten only after every wave has
// passed the barrier that ends its last use). Per sub-block t the B operand is the grid values of
// elements 32 t + 8 g .. of row n; one MFMA pair (hi, then lo) gives sum(K * x), scaled by dl in
// fp32, sub-blocks and blocks in order. Every wave reads the workgroup's activation tiles from LDS,
// so the NT weight tiles of a wave share each A-operand read (LDS bytes per MFMA / NT).
constexpr int kIq4Waves = 8;

template <int MT, int NT>
__global__ __launch_bounds__(64 * kIq4Waves) void iq4_mtile_kernel(const uint8_t* w, long long row_bytes,
                                                                   const uint16_t* __restrict__ xh,
                                                                   const uint16_t* __restrict__ xl,
                                                                   int K, YOut y,
                                                                   long long ldy, int M, int N) {
  constexpr int kRows = 16 * MT;
  constexpr int kWgRows = 16 * NT * kIq4Waves;
  constexpr int kBuf = 2 * kRows * kXStride;                  // hi rows, then lo rows
  constexpr int kPieces = kRows * 64 / (64 * kIq4Waves);      // 16-byte pieces per thread
  extern __shared__ __align__(16) uint8_t smem[];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int ln = lane & 15, g = lane >> 4;
  const int n0 = xcd_tile(blockIdx.x, gridDim.x) * kWgRows + 16 * NT * wave;
  const int m0 = blockIdx.y * kRows;
  const uint8_t* row[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) row[nt] = w + (size_t)min(n0 + 16 * nt + ln, N - 1) * row_bytes;
  const int nb = K / QK;
  f32x4 acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // thread tid stages pieces p = tid + 512 i: row p / 64, hi (p % 64 < 32) or lo, piece p % 32;
  // rows >= M repeat row M - 1
  u32x4a4 stage[kPieces];
  auto load_x = [&](int b) {
#pragma unroll
    for (int i = 0; i < kPieces; ++i) {
      const int p = tid + 64 * kIq4Waves * i, r = p >> 6, pc = p & 63, part = pc >> 5, q = pc & 31;
      const size_t src = (size_t)min(m0 + r, M - 1) * K + (size_t)b * QK;
      stage[i] = ld16((const uint8_t*)((part ? xl : xh) + src) + 16 * q);
    }
  };
  auto store_x = [&](uint8_t* buf) {
#pragma unroll
    for (int i = 0; i < kPieces; ++i) {
      const int p = tid + 64 * kIq4Waves * i, r = p >> 6, pc = p & 63, part = pc >> 5, q = pc & 31;
      *(u32x4a4*)(buf + part * kRows * kXStride + r * kXStride + 16 * q) = stage[i];
    }
  };
  IQ4W cur[NT], nxt[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) cur[nt] = load_iq4(row[nt], 0, g);
  load_x(0);
  store_x(smem);
  __syncthreads();
  for (int b = 0; b < nb; ++b) {
    if (b + 1 < nb) {
      load_x(b + 1);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) nxt[nt] = load_iq4(row[nt], b + 1, g);
    }
    const uint8_t* Xh = smem + (b & 1) * kBuf;
    const uint8_t* Xl = Xh + kRows * kXStride;
    // sub-block t's scale bits and index words move to the front as t advances (no indexing by
    // t). Two weight tiles unroll the loop by four (fully unrolled they need more than the 256
    // VGPRs of two waves per SIMD; rolled, the moves cost 5% more time), one tile fully, where
    // the moves vanish.
    float dh[NT];
    uint32_t shs[NT], sls[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      dh[nt] = half_to_float(cur[nt].hdr[0]);
      shs[nt] = cur[nt].hdr[0] >> 16, sls[nt] = cur[nt].hdr[1];
    }
#pragma unroll(NT == 1 ? 8 : 4)
    for (int t = 0; t < 8; ++t) {
      float dl[NT];
      bf16x8 bk[NT];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int ls = (int)((sls[nt] & 15u) | ((shs[nt] & 3u) << 4));
        sls[nt] >>= 4, shs[nt] >>= 2;
        dl[nt] = dh[nt] * (float)(ls - 32);
        const uint32_t q0 = cur[nt].qs[0], q1 = cur[nt].qs[1];
#pragma unroll
        for (int j = 0; j < 14; ++j) cur[nt].qs[j] = cur[nt].qs[j + 2];
        const uint32_t i0 = (g >= 2 ? q0 >> 4 : q0) & 0x0F0F0F0Fu, i1 = (g >= 2 ? q1 >> 4 : q1) & 0x0F0F0F0Fu;
        bk[nt] = __builtin_bit_cast(bf16x8, grid_bf16x8(i0, i1));
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int off = (16 * mt + ln) * kXStride + 2 * (32 * t + 8 * g);
        const bf16x8 ah = __builtin_bit_cast(bf16x8, *(const u32x4*)(Xh + off));
        const bf16x8 al = __builtin_bit_cast(bf16x8, *(const u32x4*)(Xl + off));
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          f32x4 D = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bk[nt], f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
          D = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bk[nt], D, 0, 0, 0);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[mt][nt][i] = fmaf(dl[nt], D[i], acc[mt][nt][i]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);  // one sub-block's operands live at a time
    }
    if (b + 1 < nb) {
      store_x(smem + ((b + 1) & 1) * kBuf);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) cur[nt] = nxt[nt];
    }
    __syncthreads();
  }
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int n = n0 + 16 * nt + ln;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = m0 + 16 * mt + 4 * g + i;
        if (m < M && n < N) y.put((size_t)m * ldy + n, acc[mt][nt][i]);
      }
  }
}

}  // namespace

size_t iq4_prefill_workspace(int m_rows, int k) { return (size_t)m_rows * k * 2 * 2; }

int launch_iq4_prefill(const uint8_t* w, long long row_bytes, const float* x, void* workspace,
                       YOut y, long long ldy, int m_rows, int k, int n_rows, hipStream_t stream) {
  uint16_t* hi = (uint16_t*)workspace;
  uint16_t* lo = hi + (size_t)m_rows * k;
  const long long n4 = (long long)m_rows * k / 4;
  hipLaunchKernelGGL(split_bf16_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, stream, x, hi,
                     lo, n4);
  constexpr int MT = 4;
  constexpr int kLds = 2 * 2 * 16 * MT * kXStride;
  const int mblocks = (m_rows + 16 * MT - 1) / (16 * MT);
  auto go = [&](auto kern, int wg_rows) {
    allow_lds((const void*)kern, kLds);
    const dim3 grid((n_rows + wg_rows - 1) / wg_rows, mblocks);
    hipLaunchKernelGGL(kern, grid, dim3(64 * kIq4Waves), kLds, stream, w, row_bytes, hi, lo, k, y,
                       ldy, m_rows, n_rows);
    return 0;
  };
  // two weight tiles per wave where that still gives at least two rounds of workgroups (measured
  // on MI355X per call, the same bits: 4096 x 4096 M = 2048 302 vs 340-347 us, 14336 x 4096
  // M = 2048 947 vs 1105; at M = 512 the halved grid left CUs idle, 153 vs 96 us)
  constexpr int kRows2 = 16 * 2 * kIq4Waves;
  if ((long long)((n_rows + kRows2 - 1) / kRows2) * mblocks >= 2LL * cu_count())
    return go(iq4_mtile_kernel<MT, 2>, kRows2);
  return go(iq4_mtile_kernel<MT, 1>, 16 * kIq4Waves);
}

}  // namespace mxa
