// Decode GEMV, lane-per-block form: y[m, n] = sum_k x[m, k] * W[n, k] for up to 4 activation rows.
//
// Memory. A wave owns R consecutive weight rows (R * nb <= 64 blocks; one row per pass of 64 blocks
// when nb > 64). Those rows are one contiguous byte range, which the wave copies into its own LDS
// region with global_load_lds_dwordx4: every instruction moves 1 KB of consecutive bytes (16 per
// lane), the fully coalesced pattern that keeps HBM streaming. All of a wave's copies are issued
// at its first instruction, before anything waits.
//
// Compute. Lane i of the wave then owns block i of that range (row i / nb, block i % nb) and reads
// it from LDS: no cross-lane reduction, and LDS absorbs the blocks' alignment (Q6_K's 210-byte
// blocks are read as dwords and realigned with v_alignbyte). The workgroup quantizes the float
// activations to Q8_K once into LDS (the arithmetic of quantize_q8k_kernel; IQ4_XS keeps floats).
//
// Numerics (app/native/src/mx_dot_k_ssse3.c:115-154): exact integer block dots, then the per-block float
// value goes to a wave-private LDS buffer and one lane per (row, activation row) folds the blocks
// in order 0..nb-1 with the CPU oracle's fused multiply-adds: results equal it bit for bit (IQ4_XS:
// float activations, within tolerance).
#include "mxa_kernels.hpp"
#include "mxa_lpb.hpp"

#pragma clang fp contract(off)

namespace mxa {
namespace {

// LDS layout of a workgroup (dynamic shared memory):
//   [act]  per activation row m and staged block bb: 256 q8 + kActPad | ... then bsums (32 B each)
//          and scales (4 B each); IQ4_XS: 1024 B of floats + kActPad per block
//   [wave] per wave: the weight bytes region (reg_bytes), then V / D buffers
// One 16-byte piece (four floats, piece pc of 64) of a float activation block staged at `blk`. For
// the fp32-activation types the quad of lanes holding pieces 4j .. 4j + 3 also writes sum j of the
// block's sixteen sums of 16 ((x0 + x1) + (x2 + x3) per lane, then across the quad); every lane
// of that quad must be active.
template <int TYPE>
__device__ __forceinline__ void stage_float_piece(uint8_t* blk, int pc, const uint8_t* src) {
  const u32x4a4 u = ld16(src);
  *(u32x4a4*)(blk + 16 * pc) = u;
  if constexpr (ActTraits<TYPE>::kSums) {
    // the elements are copied to scalars first: this compiler bit-casts an element expression of
    // an ext_vector (u.y) as element 0
    const uint32_t e0 = u[0], e1 = u[1], e2 = u[2], e3 = u[3];
    const float s = quad_sum((__builtin_bit_cast(float, e0) + __builtin_bit_cast(float, e1)) +
                             (__builtin_bit_cast(float, e2) + __builtin_bit_cast(float, e3)));
    if ((pc & 3) == 0) *(float*)(blk + 4 * QK + pc) = s;  // sum pc / 4
  }
}

struct Geometry {
  int rows_per_wave;    // R
  int blocks_per_pass;  // blocks of one row in a pass (nb when R > 1)
  int reg_bytes;        // weight region per wave
  int act_blocks;       // activation blocks staged per pass
};

// The rows of weight tile blockIdx.x (of gridDim.x) against M <= MAXM activation rows.
template <int TYPE, int MAXM, bool FUSEQ>
__device__ __forceinline__ void lpb_rows(const uint8_t* __restrict__ w, long long row_bytes,
                                         const Act& act, YOut y, long long ldy, int M, int N,
                                         const Geometry& geo) {
  using L = Lpb<TYPE>;
  constexpr bool kFloatAct = ActTraits<TYPE>::kFloat;
  constexpr int kActBlk = ActTraits<TYPE>::kBlk;
  extern __shared__ __align__(16) uint8_t smem[];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, nw = blockDim.x >> 6;
  const int R = geo.rows_per_wave, bpp = geo.blocks_per_pass, nb = act.nb;
  const int ab = geo.act_blocks;  // == bpp
  uint8_t* act_q = smem;                                        // [MAXM][ab][kActBlk]
  int16_t* act_bs = (int16_t*)(smem + MAXM * ab * kActBlk);      // [MAXM][ab][16]
  float* act_d = (float*)(act_bs + MAXM * ab * 16);              // [MAXM][ab]
  uint8_t* region = smem + ((MAXM * ab * (kActBlk + 32 + 4) + 15) & ~15);
  const int wave_bytes = geo.reg_bytes + MAXM * 64 * 4 * 2;  // weights, then V and D (64 each)
  uint8_t* wreg = region + wave * wave_bytes;
  float* Vbuf = (float*)(wreg + geo.reg_bytes);                 // [MAXM][64]
  float* Dbuf = Vbuf + MAXM * 64;                                // [64]

  const int tile_rows = R * nw;
  const int n_wave0 = xcd_tile(blockIdx.x, gridDim.x) * tile_rows + wave * R;  // first row of the wave
  const uint8_t* w_end = w + (size_t)N * row_bytes;
  // (row, activation row) pairs f = lane + 64 j (j < MAXM): row f % R, activation row f / R;
  // R * M <= 64 * MAXM. Several passes happen only when R == 1.
  float acc[MAXM];
#pragma unroll
  for (int j = 0; j < MAXM; ++j) acc[j] = 0.0f;

  for (int c0 = 0; c0 < nb; c0 += bpp) {
    const int cb = min(bpp, nb - c0);  // blocks of each row in this pass
    // 1. the wave's bytes: R rows x cb blocks, one contiguous range when cb == nb (else R == 1)
    const int nrows = max(0, min(R, N - n_wave0));
    const uint8_t* src0 = w + (size_t)min(n_wave0, N - 1) * row_bytes + (size_t)c0 * L::kBytes;
    const uintptr_t s_al = (uintptr_t)src0 & ~(uintptr_t)15;
    const int mis = (int)((uintptr_t)src0 - s_al);
    const int span = (cb == nb ? nrows * (int)row_bytes : cb * L::kBytes);
    const int n_ins = (mis + span + 1023) >> 10;
    // copies are whole aligned 16-byte chunks: the first and last may extend past the matrix,
    // but a 16-byte aligned chunk holding one of its bytes never leaves that byte's page
    const uintptr_t last = ((uintptr_t)w_end - 1) & ~(uintptr_t)15;
    for (int t = 0; t < n_ins; ++t) {
      const uintptr_t a = min(s_al + (uintptr_t)(t * 1024 + lane * 16), last);
      __builtin_amdgcn_global_load_lds((const void*)a, (lds_void*)(wreg + t * 1024), 16, 0, 0);
    }

    // 2. activations of the pass into LDS (all M rows), quantized here when FUSEQ
    if constexpr (FUSEQ) {
      // 16 lanes per (m, block); lane part p holds values 16p..16p+15
      for (int g = tid >> 4; g < M * cb; g += blockDim.x >> 4) {
        const int m = g / cb, bb = g - m * cb, p = tid & 15;
        const float* src = act.x + (size_t)m * act.k + (size_t)(c0 + bb) * QK + 16 * p;
        float v[16];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float4 f = *(const float4*)(src + 4 * i);
          v[4 * i] = f.x, v[4 * i + 1] = f.y, v[4 * i + 2] = f.z, v[4 * i + 3] = f.w;
        }
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[i]));
        amax = max16(amax);
        int q[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) q[i] = 0;
        if (amax != 0.0f) {
          const float iscale = 127.0f / amax;
#pragma unroll
          for (int i = 0; i < 16; ++i) q[i] = (int)fminf(fmaxf(rintf(v[i] * iscale), -127.0f), 127.0f);
        }
        u32x4a4 packed;
        int bsum = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          packed[i] = (uint32_t)(q[4 * i] & 0xFF) | ((uint32_t)(q[4 * i + 1] & 0xFF) << 8) |
                      ((uint32_t)(q[4 * i + 2] & 0xFF) << 16) | ((uint32_t)(q[4 * i + 3] & 0xFF) << 24);
          bsum += q[4 * i] + q[4 * i + 1] + q[4 * i + 2] + q[4 * i + 3];
        }
        *(u32x4a4*)(act_q + (m * ab + bb) * kActBlk + 16 * p) = packed;
        act_bs[(m * ab + bb) * 16 + p] = (int16_t)bsum;
        if (p == 0) act_d[m * ab + bb] = amax / 127.0f;
      }
    } else if constexpr (kFloatAct) {
      // 16-byte pieces of float rows; whole waves take part (M * cb * 64 is a multiple of 64)
      for (int i = tid; i < M * cb * 64; i += blockDim.x) {
        const int m = i / (cb * 64), o = i - m * cb * 64, bb = o >> 6, pc = o & 63;
        stage_float_piece<TYPE>(act_q + (m * ab + bb) * kActBlk, pc,
                                (const uint8_t*)(act.x + (size_t)m * act.k + (size_t)(c0 + bb) * QK) + 16 * pc);
      }
    } else {
      for (int i = tid; i < M * cb * 16; i += blockDim.x) {  // 16-byte pieces of q8 rows
        const int m = i / (cb * 16), o = i - m * cb * 16, bb = o >> 4, pc = o & 15;
        *(u32x4a4*)(act_q + (m * ab + bb) * kActBlk + 16 * pc) =
            ld16((const uint8_t*)(act.q + (size_t)m * act.k + (size_t)(c0 + bb) * QK) + 16 * pc);
      }
      for (int i = tid; i < M * cb * 2; i += blockDim.x) {
        const int m = i / (cb * 2), o = i - m * cb * 2, bb = o >> 1, hf = o & 1;
        *(u32x4a4*)(act_bs + (m * ab + bb) * 16 + 8 * hf) =
            ld16((const uint8_t*)(act.bsums + ((size_t)m * nb + c0 + bb) * 16) + 16 * hf);
      }
      for (int i = tid; i < M * cb; i += blockDim.x) {
        const int m = i / cb, bb = i - m * cb;
        act_d[m * ab + bb] = act.d[(size_t)m * nb + c0 + bb];
      }
    }
    // weight bytes landed (global_load_lds completes into LDS before vmcnt drops), activations
    // written: one barrier for the workgroup
    __builtin_amdgcn_s_waitcnt(0x3F70);  // vmcnt(0)
    __syncthreads();

    // 3. lane -> block
    const int fb = min(lane, nrows * cb - 1);
    const int r = fb / cb, b = fb - r * cb;
    if (nrows > 0) {
      const int boff = mis + (cb == nb ? r * (int)row_bytes : 0) + b * L::kBytes;
      ActBlock ablk[MAXM];
#pragma unroll
      for (int m = 0; m < MAXM; ++m) {
        const int mc = min(m, M - 1);
        ablk[m].q = (const int8_t*)(act_q + (mc * ab + b) * kActBlk);
        ablk[m].bsums = act_bs + (mc * ab + b) * 16;
        ablk[m].d = 0.0f;
        ablk[m].x = (const float*)(act_q + (mc * ab + b) * kActBlk);
      }
      float V[MAXM], D;
      L::template compute<MAXM, ActBlock>(wreg, boff, ablk, M, V, D);
      if (lane < nrows * cb) {
#pragma unroll
        for (int m = 0; m < MAXM; ++m)
          if (m < M) Vbuf[m * 64 + lane] = V[m];
        if (L::kHasD) Dbuf[lane] = D;
      }
      __builtin_amdgcn_wave_barrier();
      // 4. fold this pass's blocks of each pair, in order
#pragma unroll
      for (int j = 0; j < MAXM; ++j) {
        const int f = lane + 64 * j, fr = f % R, fm = f / R;
        if (f < R * M && fr < nrows) {
          const int base = fr * cb;
          for (int bb = 0; bb < cb; ++bb) {
            const float xd = kFloatAct ? 0.0f : act_d[fm * ab + bb];
            acc[j] = L::fold(acc[j], xd, Vbuf[fm * 64 + base + bb], L::kHasD ? Dbuf[base + bb] : 0.0f);
          }
        }
      }
    }
    __syncthreads();  // before the next pass overwrites LDS
  }
#pragma unroll
  for (int j = 0; j < MAXM; ++j) {
    const int f = lane + 64 * j, fr = f % R, fm = f / R;
    if (f < R * M && fr < N - n_wave0) y.put((size_t)fm * ldy + n_wave0 + fr, acc[j]);
  }
}

template <int TYPE, int MAXM, bool FUSEQ>
__global__ __launch_bounds__(512) void gemv_lpb_kernel(const uint8_t* __restrict__ w,
                                                       long long row_bytes, Act act,
                                                       YOut y, long long ldy,
                                                       int M, int N, Geometry geo) {
  lpb_rows<TYPE, MAXM, FUSEQ>(w, row_bytes, act, y, ldy, M, N, geo);
}

// Grouped MoE projection on float activations (IQ4_XS experts): expert e = blockIdx.y multiplies
// its rows [offsets[e], offsets[e + 1]) of x by its weight (w + e * expert_stride), writing the same
// rows of y, four rows at a time through the decode body: chunk z of the expert's rows by the
// workgroups of blockIdx.z == z mod gridDim.z, so every row is computed whatever the grid's depth.
// Each row takes the decode kernels' summation order, so it equals that row multiplied alone. The
// offsets come from the device: clamped to [0, total_rows), a bad table gives wrong rows, never an
// access outside x or y.
template <int TYPE>
__global__ __launch_bounds__(512) void moe_lpb_kernel(const uint8_t* __restrict__ w,
                                                      long long row_bytes, long long expert_stride,
                                                      Act act, const int32_t* __restrict__ offsets,
                                                      int total_rows, YOut y, long long ldy, int N,
                                                      Geometry geo) {
  const int e = blockIdx.y;
  const int begin = min(max(offsets[e], 0), total_rows);
  const int end = min(max(offsets[e + 1], begin), total_rows);
  for (int p0 = begin + 4 * (int)blockIdx.z; p0 < end; p0 += 4 * (int)gridDim.z) {
    Act a = act;  // rows p0 .. p0 + 3, uniform over the workgroup
    a.x = act.x + (size_t)p0 * act.k;
    lpb_rows<TYPE, 4, false>(w + (size_t)e * expert_stride, row_bytes, a, y.at((long long)p0 * ldy),
                             ldy, min(4, end - p0), N, geo);
    __syncthreads();  // the next chunk restages the LDS this one read
  }
}

// Rows per wave, blocks per pass and LDS of the lane-per-block kernel for MAXM activation rows;
// false when the workgroup does not fit LDS.
template <int TYPE, int MAXM>
bool lpb_geometry(int nb, Geometry& geo, int& nw, int& lds) {
  using L = Lpb<TYPE>;
  constexpr bool kFloatAct = ActTraits<TYPE>::kFloat;
  constexpr int kActBlk = ActTraits<TYPE>::kBlk;
  // blocks staged per pass: a wave's 64 lanes, and (float activations, 1 KB per block and row)
  // at most ~40 KB of activations
  const int cap = kFloatAct ? max(1, min(kWaveLanes, 40960 / (MAXM * kActBlk))) : kWaveLanes;
  if (nb <= cap) {
    geo.rows_per_wave = kWaveLanes / nb;
    geo.blocks_per_pass = nb;
  } else {
    geo.rows_per_wave = 1;
    geo.blocks_per_pass = cap;
  }
  const int pass_bytes = geo.rows_per_wave * geo.blocks_per_pass * L::kBytes;
  geo.reg_bytes = ((pass_bytes + 15 + 1023) / 1024) * 1024;
  geo.act_blocks = geo.blocks_per_pass;
  const int act_lds = MAXM * geo.act_blocks * (kActBlk + 32 + 4) + 16;
  const int wave_lds = geo.reg_bytes + MAXM * 64 * 4 * 2;
  // two workgroups per CU (<= 80 KB each), at most 8 waves
  nw = max(1, min(8, (80 * 1024 - act_lds) / wave_lds));
  lds = act_lds + nw * wave_lds;
  return lds <= 160 * 1024;
}

template <int TYPE, int MAXM, bool FUSEQ>
int launch_lpb(const uint8_t* w, long long row_bytes, const Act& act, YOut y, long long ldy,
               int M, int N, hipStream_t stream) {
  Geometry geo;
  int nw = 0, lds = 0;
  if (!lpb_geometry<TYPE, MAXM>(act.nb, geo, nw, lds)) return -1;
  const int tile_rows = geo.rows_per_wave * nw;
  const int grid = (N + tile_rows - 1) / tile_rows;
  auto kern = gemv_lpb_kernel<TYPE, MAXM, FUSEQ>;
  if (lds > 64 * 1024) allow_lds((const void*)kern, 160 * 1024);
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * nw), lds, stream, w, row_bytes, act, y, ldy, M, N, geo);
  return 0;
}

// ------------------------------------------------------------------------------------------------
// Pipelined form (blocks per row <= 64): compute overlaps the arrival of the weight bytes.
//
// A workgroup has `act_waves` waves that only stage the activations and `weight_waves` waves
// that only move and multiply weights. vmcnt (a wave's count of outstanding memory operations)
// is per wave, but the vector-memory queue of a CU is shared and drains in order: the activation
// waves issue their loads first and the weight waves start copying only after a barrier, so the
// activations never wait behind weight bytes. A weight wave owns R consecutive rows, i.e. R * nb
// consecutive blocks of one contiguous byte range, and walks them in stages of 64 blocks (one per
// lane) through a ring of P + 1 LDS buffers: it keeps P stages of copies in flight, waits only for
// the copies of the stage it computes next (copies complete in issue order), issues the copies
// of the stage P ahead into the buffer it has just finished with, and computes. Copies are issued
// only as fast as the queue drains, so a wave that tried to issue everything up front would sit
// in the issue queue instead of computing. After its last stage one lane per (row, activation
// row) folds the row's nb block values in order.
//
// LONG: a wave whose range has more blocks than the value ring (kVRing) folds, after each stage,
// every row that stage completed, keeps its outputs in LDS until the end, and may run with a
// single stage buffer (P == 0: the next stage is requested as soon as this one is computed).
// Its LDS then no longer grows with the rows per wave, so 8 weight waves fit where the block
// values of all rows did not (the Q6_K vocabulary head: 3 waves per CU before, each SIMD with a
// single wave issuing ~470 VALU per 64-block stage at a fraction of its rate). The short form
// keeps its own instantiation: folding inside its loop measured slower (10.3 vs 9.1 us).

// Block values of a LONG weight wave wait in a ring of this many slots per activation row until
// their row is complete (a row has at most 64 blocks, so 64 + nb - 1 slots are enough).
constexpr int kVRing = 128;
// LDS of a weight wave beside its stage buffers: its block values and D (all of them, or the ring
// and the folded outputs of its R rows when LONG); a multiple of 16 so that every wave's buffers
// stay 16-byte aligned.
template <int MAXM>
__host__ __device__ constexpr int wave_value_bytes(bool long_form, int R, int nb) {
  return long_form ? (kVRing * 4 * (MAXM + 1) + R * MAXM * 4 + 15) & ~15 : R * nb * 4 * (MAXM + 1);
}

struct PipeGeo {
  int rows_per_wave;  // R
  int weight_waves;
  int act_waves;
  int ahead;          // P: stages of copies in flight while a stage is computed
  int buf_kb;         // KB of one stage buffer (the most copies a stage needs)
};

// Stage 64 s .. 64 s + 63 of a range of nblk blocks that starts `mis` bytes past a 16-byte
// boundary needs this many 1 KB copies (64 blocks are a multiple of 16 bytes for every type, so
// every stage starts `mis` bytes past a boundary too).
template <int KB>
__device__ __forceinline__ int stage_copies(int s, int nblk, int mis) {
  const int nbk = min(64, nblk - 64 * s);
  return (mis + nbk * KB + 1023) >> 10;
}

// The activation waves: M rows x nb blocks into LDS (quantized to Q8_K when FUSEQ; copied from
// the workspace, or as floats for IQ4_XS). Executes the workgroup's first barrier once its first
// loads are issued, and the second when everything is in LDS.
template <int TYPE, bool FUSEQ>
__device__ __forceinline__ void stage_activations(const Act& act, int M, int aw, int na, int lane,
                                                  uint8_t* act_q, int16_t* act_bs, float* act_d) {
  constexpr bool kFloatAct = ActTraits<TYPE>::kFloat;
  constexpr int kActBlk = ActTraits<TYPE>::kBlk;
  const int nb = act.nb, total = M * nb;
  if constexpr (FUSEQ) {
    // 16 lanes per (m, block): lane part p holds values 16p..16p+15; kBatch groups per lane are
    // loaded before any is quantized
    constexpr int kBatch = 4;
    const int per = 4 * na, p = lane & 15;
    float4 v[kBatch][4];
    auto load = [&](int g0) {
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int g = min(g0 + i * per, total - 1);
        const int m = g / nb, b = g - m * nb;
        const float* src = act.x + (size_t)m * act.k + (size_t)b * QK + 16 * p;
#pragma unroll
        for (int q = 0; q < 4; ++q) v[i][q] = *(const float4*)(src + 4 * q);
      }
    };
    int gw = 4 * aw;  // the wave's first group (its lanes 16r.. take group gw + r); gw < total
    int g0 = gw + (lane >> 4);
    load(g0);
    __builtin_amdgcn_s_barrier();  // first barrier: these loads are queued ahead of any copy
    for (;;) {
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int g = g0 + i * per;
        if (g < total) {  // uniform over the 16 lanes of the group
          const int m = g / nb, b = g - m * nb;
          const float x[16] = {v[i][0].x, v[i][0].y, v[i][0].z, v[i][0].w, v[i][1].x, v[i][1].y,
                               v[i][1].z, v[i][1].w, v[i][2].x, v[i][2].y, v[i][2].z, v[i][2].w,
                               v[i][3].x, v[i][3].y, v[i][3].z, v[i][3].w};
          float amax = 0.0f;
#pragma unroll
          for (int e = 0; e < 16; ++e) amax = fmaxf(amax, fabsf(x[e]));
          amax = max16(amax);
          int q[16];
#pragma unroll
          for (int e = 0; e < 16; ++e) q[e] = 0;
          if (amax != 0.0f) {
            const float iscale = 127.0f / amax;
#pragma unroll
            for (int e = 0; e < 16; ++e) q[e] = (int)fminf(fmaxf(rintf(x[e] * iscale), -127.0f), 127.0f);
          }
          u32x4a4 packed;
          int bsum = 0;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            packed[e] = (uint32_t)(q[4 * e] & 0xFF) | ((uint32_t)(q[4 * e + 1] & 0xFF) << 8) |
                        ((uint32_t)(q[4 * e + 2] & 0xFF) << 16) | ((uint32_t)(q[4 * e + 3] & 0xFF) << 24);
            bsum += q[4 * e] + q[4 * e + 1] + q[4 * e + 2] + q[4 * e + 3];
          }
          *(u32x4a4*)(act_q + (m * nb + b) * kActBlk + 16 * p) = packed;
          act_bs[(m * nb + b) * 16 + p] = (int16_t)bsum;
          if (p == 0) act_d[m * nb + b] = amax / 127.0f;
        }
      }
      gw += per * kBatch;
      g0 += per * kBatch;
      if (gw >= total) break;  // wave-uniform
      load(g0);
    }
  } else {
    __builtin_amdgcn_s_barrier();  // first barrier
    if constexpr (kFloatAct) {
      // 16-byte pieces of float rows; whole waves take part
      for (int i = aw * 64 + lane; i < total * 64; i += na * 64) {
        const int g = i >> 6, pc = i & 63, m = g / nb, b = g - m * nb;
        stage_float_piece<TYPE>(act_q + g * kActBlk, pc,
                                (const uint8_t*)(act.x + (size_t)m * act.k + (size_t)b * QK) + 16 * pc);
      }
    } else {
      for (int i = aw * 64 + lane; i < total * 16; i += na * 64) {  // 16-byte pieces of q8 rows
        const int g = i >> 4, pc = i & 15, m = g / nb, b = g - m * nb;
        *(u32x4a4*)(act_q + g * kActBlk + 16 * pc) =
            ld16((const uint8_t*)(act.q + (size_t)m * act.k + (size_t)b * QK) + 16 * pc);
      }
      for (int i = aw * 64 + lane; i < total * 2; i += na * 64)  // (m, b) bsums are contiguous
        *(u32x4a4*)(act_bs + 8 * i) = ld16((const uint8_t*)(act.bsums + 8 * (size_t)i));
      for (int i = aw * 64 + lane; i < total; i += na * 64) act_d[i] = act.d[i];
    }
  }
  // Nothing of this wave stays outstanding (the compiler may merge the barrier below with the
  // weight waves' one, and its wait bookkeeping would carry these loads over to them).
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();  // second barrier: the activations are in LDS
}

// ACTREG (one activation row, 64 % nb == 0): lane l's block of the row is l % nb in every stage,
// so the lane keeps that block's Q8_K values in registers instead of reading LDS per stage.
// One workgroup's share of a pipelined decode: rows of workgroup tile `tile` (R rows per weight
// wave) of one packed weight.
template <int TYPE, int MAXM, bool FUSEQ, bool ACTREG, bool LONG = false>
__device__ __forceinline__ void pipe_rows(uint8_t* smem, const uint8_t* w, long long row_bytes,
                                          const Act& act, YOut y, long long ldy,
                                          int M, int N, const PipeGeo& geo, int tile) {
  static_assert(!ACTREG || (MAXM == 1 && (TYPE == T_Q4_K || TYPE == T_Q8_0)),
                "register activations: one Q8_K row, types whose compute leaves room for them");
  using L = Lpb<TYPE>;
  constexpr bool kFloatAct = ActTraits<TYPE>::kFloat;
  constexpr int kActBlk = ActTraits<TYPE>::kBlk;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar control flow
  const int nb = act.nb, na = geo.act_waves, total = M * nb;
  uint8_t* act_q = smem;                                    // [M * nb][kActBlk]
  int16_t* act_bs = (int16_t*)(smem + total * kActBlk);     // [M * nb][16]
  float* act_d = (float*)(act_bs + total * 16);             // [M * nb]
  uint8_t* region = smem + ((total * (kActBlk + 32 + 4) + 15) & ~15);

  if (wave < na) {  // activation wave
    stage_activations<TYPE, FUSEQ>(act, M, wave, na, lane, act_q, act_bs, act_d);
    return;
  }

  const int R = geo.rows_per_wave, P = geo.ahead, ww = wave - na;
  // block values: all R * nb of them, or (LONG) block j at ring slot j % kVRing
  const int vslots = LONG ? kVRing : R * nb;
  const int buf_bytes = geo.buf_kb * 1024;
  const int nbuf = max(1, min(P + 1, (R * nb + 63) >> 6));  // P >= the stage count: no reuse
  const int wave_bytes = nbuf * buf_bytes + wave_value_bytes<MAXM>(LONG, R, nb);
  uint8_t* wreg = region + ww * wave_bytes;
  float* Vbuf = (float*)(wreg + nbuf * buf_bytes);  // [MAXM][vslots]
  float* Dbuf = Vbuf + MAXM * vslots;                   // [vslots]
  float* Ybuf = Dbuf + vslots;                          // LONG: [MAXM][R] folded outputs

  const int n0 = (tile * geo.weight_waves + ww) * R;
  const int nrows = max(0, min(R, N - n0));
  const int nblk = nrows * nb, stages = (nblk + 63) >> 6;
  const uint8_t* src0 = w + (size_t)min(n0, N - 1) * row_bytes;
  const uintptr_t s_al = (uintptr_t)src0 & ~(uintptr_t)15;
  const int mis = (int)((uintptr_t)src0 - s_al);
  // whole aligned 16-byte chunks: the first and last may extend past the matrix, but a 16-byte
  // aligned chunk holding one of its bytes never leaves that byte's page
  const uintptr_t last = ((uintptr_t)(w + (size_t)N * row_bytes) - 1) & ~(uintptr_t)15;
  const uint32_t lds_w = lds_addr(wreg);
  auto issue = [&](int s) {
    const uintptr_t g = s_al + (uintptr_t)s * 64 * L::kBytes + (uintptr_t)lane * 16;
    const uint32_t dst = lds_w + (uint32_t)((s % nbuf) * buf_bytes);
    const int n = stage_copies<L::kBytes>(s, nblk, mis);
    if (s + 1 < stages) {  // the bytes of a later stage follow: no copy passes the matrix end
      for (int t = 0; t < n; ++t) copy16_to_lds_nt((const void*)(g + (uintptr_t)t * 1024), dst + t * 1024);
    } else {
      for (int t = 0; t < n; ++t) copy16_to_lds_nt((const void*)min(g + (uintptr_t)t * 1024, last), dst + t * 1024);
    }
  };

  __builtin_amdgcn_s_barrier();  // first barrier: the activation loads are queued
  for (int s = 0; s < min(max(P, 1), stages); ++s) issue(s);
  __builtin_amdgcn_s_barrier();  // second barrier: the activations are in LDS
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");

  // lane l computes block 64 s + l of the range: block b = (64 s + l) mod nb of its row, kept
  // incrementally (stage s + 1 adds 64 mod nb); lanes past the range end redo its last block
  const int step = 64 % nb;
  int b = lane % nb;
  const int lane_off = mis + (int)__umul24(lane, L::kBytes);
  ActRegs areg;
  if constexpr (ACTREG) {
#pragma unroll
    for (int i = 0; i < 16; ++i) areg.q[i] = *(const i32x4a4*)(act_q + b * kActBlk + 16 * i);
    areg.bs[0] = *(const u32x4a4*)(act_bs + 16 * b);
    areg.bs[1] = *(const u32x4a4*)(act_bs + 16 * b + 8);
  }
  // LONG fold: rows folded .. upto - 1, whose blocks are all computed; pair f -> activation row
  // f / cnt, row folded + f % cnt; blocks in order; outputs to Ybuf (a store here would count on
  // vmcnt and hold up the next stage's wait)
  int folded = 0;
  auto fold_rows = [&](int upto) {
    const int cnt = upto - folded;
    for (int f = lane; f < cnt * M; f += 64) {
      const int fm = f / cnt, fr = folded + (f - fm * cnt);
      const float* v = Vbuf + fm * kVRing;
      const float* xd = act_d + fm * nb;
      const int base = fr * nb;  // the row's first block in the range
      float acc = 0.0f;
      int bb = 0;
      for (; bb + 16 <= nb; bb += 16) {
        float vv[16], xx[16], ww[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int slot = (base + bb + i) & (kVRing - 1);
          vv[i] = v[slot];
          xx[i] = kFloatAct ? 0.0f : xd[bb + i];
          ww[i] = L::kHasD ? Dbuf[slot] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) acc = L::fold(acc, xx[i], vv[i], ww[i]);
      }
      for (; bb < nb; ++bb) {
        const int slot = (base + bb) & (kVRing - 1);
        acc = L::fold(acc, kFloatAct ? 0.0f : xd[bb], v[slot], L::kHasD ? Dbuf[slot] : 0.0f);
      }
      Ybuf[fm * R + fr] = acc;
    }
    folded = upto;
  };
  for (int s = 0; s < stages; ++s) {
    // copies issued after stage s: stages s + 1 .. min(s + P - 1, stages - 1)
    int after = 0;
    for (int k = s + 1; k <= min(s + P - 1, stages - 1); ++k) after += stage_copies<L::kBytes>(k, nblk, mis);
    wait_vmcnt(after);
    if (P > 0 && s + P < stages) issue(s + P);
    int jl = lane, boff = lane_off, bb = b;
    if (64 * s + 64 > nblk) {  // partial last stage
      jl = min(lane, nblk - 1 - 64 * s);
      boff = mis + (int)__umul24(jl, L::kBytes);
      bb = (64 * s + jl) % nb;
    }
    const int aoff = (int)__umul24(bb, kActBlk);
    ActBlock ablk[MAXM];
#pragma unroll
    for (int m = 0; m < MAXM; ++m) {
      const int row = min(m, M - 1) * nb;
      ablk[m].q = (const int8_t*)(act_q + row * kActBlk + aoff);
      ablk[m].bsums = act_bs + row * 16 + bb * 16;
      ablk[m].d = 0.0f;
      ablk[m].x = (const float*)(act_q + row * kActBlk + aoff);
    }
    float V[MAXM], D;
    if constexpr (ACTREG)  // lanes past the range end compute with their own block: never stored
      L::template compute<1, ActRegs>(wreg + (s % nbuf) * buf_bytes, boff, &areg, 1, V, D);
    else
      L::template compute<MAXM, ActBlock>(wreg + (s % nbuf) * buf_bytes, boff, ablk, M, V, D);
    b += step;
    b = b >= nb ? b - nb : b;
    if constexpr (LONG) {
      // one buffer: its bytes have all been read (the compute used them), so the next stage can
      // be requested into it before this stage's rows are folded
      if (P == 0 && s + 1 < stages) issue(s + 1);
    }
    const int j = LONG ? (64 * s + jl) & (kVRing - 1) : 64 * s + jl;
    if (jl == lane) {
#pragma unroll
      for (int m = 0; m < MAXM; ++m)
        if (m < M) Vbuf[m * vslots + j] = V[m];
      if (L::kHasD) Dbuf[j] = D;
    }
    if constexpr (LONG) {
      // rows complete after this stage are folded now, while the next stage is in flight: a row
      // still open spans at most nb - 1 earlier slots, and the next stage writes 64 later ones
      __builtin_amdgcn_wave_barrier();
      fold_rows(min(64 * (s + 1), nblk) / nb);
    }
  }
  __builtin_amdgcn_wave_barrier();
  if constexpr (LONG) {
    for (int f = lane; f < nrows * M; f += 64) {  // consecutive lanes, consecutive rows
      const int fm = f / nrows, fr = f - fm * nrows;
      y.put((size_t)fm * ldy + n0 + fr, Ybuf[fm * R + fr]);
    }
    return;
  }
  // fold: pair f -> row f % nrows, activation row f / nrows; blocks in order
  for (int f = lane; f < nrows * M; f += 64) {
    const int fm = f / nrows, fr = f - fm * nrows;
    const float* v = Vbuf + fm * vslots + fr * nb;
    const float* dd = Dbuf + fr * nb;
    const float* xd = act_d + fm * nb;
    float acc = 0.0f;
    int bb = 0;
    // 16 blocks' operands are read from LDS before they are folded: the chain of dependent
    // fmas then waits for one LDS round trip, not one per block
    for (; bb + 16 <= nb; bb += 16) {
      float vv[16], xx[16], ww[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        vv[i] = v[bb + i];
        xx[i] = kFloatAct ? 0.0f : xd[bb + i];
        ww[i] = L::kHasD ? dd[bb + i] : 0.0f;
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) acc = L::fold(acc, xx[i], vv[i], ww[i]);
    }
    for (; bb < nb; ++bb)
      acc = L::fold(acc, kFloatAct ? 0.0f : xd[bb], v[bb], L::kHasD ? dd[bb] : 0.0f);
    y.put((size_t)fm * ldy + n0 + fr, acc);
  }
}

// The launch geometry packed into two dwords: with the pointers and sizes in front, every argument
// the first memory requests need is among the 14 dwords that arrive preloaded in SGPRs, so no
// wave starts with a scalar load of a kernel argument (or of the launch's own gridDim).
struct PipePack {
  uint32_t a;  // rows_per_wave | weight_waves << 12 | act_waves << 16 | ahead << 20 | buf_kb << 24
  uint32_t b;  // nb | grid << 8
};
inline bool pipe_pack(const PipeGeo& g, int nb, int grid, PipePack& p) {
  if (g.rows_per_wave > 0xFFF || g.weight_waves > 0xF || g.act_waves > 0xF || g.ahead > 0xF ||
      g.buf_kb > 0xFF || nb > 0xFF || grid > 0xFFFFFF)
    return false;
  p.a = (uint32_t)g.rows_per_wave | (uint32_t)g.weight_waves << 12 | (uint32_t)g.act_waves << 16 |
        (uint32_t)g.ahead << 20 | (uint32_t)g.buf_kb << 24;
  p.b = (uint32_t)nb | (uint32_t)grid << 8;
  return true;
}

template <int TYPE, int MAXM, bool FUSEQ, bool ACTREG, bool LONG>
__global__ __launch_bounds__(768) void gemv_pipe_kernel(const uint8_t* w, const float* x,
                                                         YOut y, int row_bytes,
                                                         int N, int M, int ldy, uint32_t pack_a,
                                                         uint32_t pack_b, const int8_t* q,
                                                         const float* d, const int16_t* bsums) {
  extern __shared__ __align__(16) uint8_t smem[];
  PipeGeo geo;
  geo.rows_per_wave = pack_a & 0xFFF;
  geo.weight_waves = (pack_a >> 12) & 0xF;
  geo.act_waves = (pack_a >> 16) & 0xF;
  geo.ahead = (pack_a >> 20) & 0xF;
  geo.buf_kb = pack_a >> 24;
  const int nb = pack_b & 0xFF, grid = pack_b >> 8;
  Act act;
  act.q = q, act.d = d, act.bsums = bsums, act.x = x;
  act.k = nb * QK, act.nb = nb, act.xsplit = nullptr, act.xbf16 = 0;
  pipe_rows<TYPE, MAXM, FUSEQ, ACTREG, LONG>(smem, w, row_bytes, act, y, ldy, M, N, geo,
                                             xcd_tile(blockIdx.x, grid));
}

// Several packed weights that share the activations (e.g. q, k and v) in one launch: workgroups
// wg0 .. of segment s take its rows, R_s rows per weight wave; outputs go to columns of y.
constexpr int kMaxSegs = 4;
struct PipeSeg {
  const uint8_t* w;
  long long row_bytes;
  YOut y;  // the segment's first output column
  int n, type, wg0, rows_per_wave;
};
struct PipeSegs {
  PipeSeg s[kMaxSegs];
  int count;
};

template <int MAXM, bool FUSEQ, bool ACTREG>
__global__ __launch_bounds__(768) void gemv_pipe_multi_kernel(PipeSegs segs, Act act, long long ldy,
                                                               int M, PipeGeo geo) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int wg = blockIdx.x;
  int i = 0;
  while (i + 1 < segs.count && wg >= segs.s[i + 1].wg0) ++i;
  const PipeSeg sg = segs.s[i];
  PipeGeo g = geo;
  g.rows_per_wave = sg.rows_per_wave;
  switch (sg.type) {
    case T_Q4_K:
      pipe_rows<T_Q4_K, MAXM, FUSEQ, ACTREG>(smem, sg.w, sg.row_bytes, act, sg.y, ldy, M, sg.n, g, wg - sg.wg0);
      break;
    case T_Q8_0:
      pipe_rows<T_Q8_0, MAXM, FUSEQ, ACTREG>(smem, sg.w, sg.row_bytes, act, sg.y, ldy, M, sg.n, g, wg - sg.wg0);
      break;
    default:
      pipe_rows<T_Q6_K, MAXM, FUSEQ, false>(smem, sg.w, sg.row_bytes, act, sg.y, ldy, M, sg.n, g, wg - sg.wg0);
      break;
  }
}

// Returns -1 when the shape does not suit the pipelined form (the caller uses gemv_lpb_kernel).
template <int TYPE, int MAXM, bool FUSEQ>
int launch_pipe(const uint8_t* w, long long row_bytes, const Act& act, YOut y, long long ldy,
                int M, int N, hipStream_t stream) {
  using L = Lpb<TYPE>;
  constexpr int kActBlk = ActTraits<TYPE>::kBlk;
  constexpr int kLdsMax = 160 * 1024;
  const int nb = act.nb;
  if (nb > kWaveLanes) return -1;
  // copies of a full stage: with 16-byte aligned rows every range starts on a copy boundary,
  // else up to 15 bytes past one
  const int mis_max = (((uintptr_t)w & 15) == 0 && row_bytes % 16 == 0) ? 0 : 15;
  const int kBufKb = (mis_max + 64 * L::kBytes + 1023) / 1024;
  const int total = M * nb;
  const int act_lds = total * (kActBlk + 32 + 4) + 16;
  if (act_lds > 80 * 1024) return -1;  // the rest of LDS must still hold 2+ waves' buffers
  const int na = min(4, (total + 15) / 16);
  const int ncu = cu_count();
  PipeGeo geo;
  geo.act_waves = na;
  geo.buf_kb = kBufKb;
  auto wave_bytes = [&](int P, int R, bool long_form) {
    return max(1, min(P + 1, (R * nb + 63) / 64)) * kBufKb * 1024 +
           wave_value_bytes<MAXM>(long_form, R, nb);
  };
  // First choice: one workgroup per CU whose waves stream all their rows (every row requested in
  // one round). When the rows' block values do not fit beside the buffers: two workgroups per CU
  // of about 8 stages per wave, so that one fills its pipeline while the other drains. One stage
  // in flight per wave and as many waves as fit (up to 8, two per SIMD) measured fastest on
  // MI355X: more copies in flight only lengthen the queue at HBM.
  int P = 0, nw = 0, R = 0;
  bool ok = false, persistent = false, long_form = false;
  for (int mode = 0; mode < 4 && !ok; ++mode) {
    persistent = mode < 2;
    P = mode % 2 == 0 ? 1 : 2;
    const int budget = (persistent ? kLdsMax : kLdsMax / 2) - act_lds;
    for (nw = 8; nw >= 2 && !ok; --nw) {  // nw + na <= 12 waves: the kernel's launch bound
      R = persistent ? (int)((N + (long long)ncu * nw - 1) / ((long long)ncu * nw)) : max(1, 512 / nb);
      ok = nw * wave_bytes(P, R, false) <= budget;
      if (ok) break;
    }
  }
  // Fewer than 8 persistent weight waves: the LONG form with one stage buffer per wave fits 8
  // (two per SIMD) when each wave's range outgrows the value ring.
  if (ok && persistent && nw < 8) {
    const int R8 = (int)((N + (long long)ncu * 8 - 1) / ((long long)ncu * 8));
    if (R8 * nb > kVRing && 8 * wave_bytes(0, R8, true) <= kLdsMax - act_lds) {
      P = 0;
      nw = 8;
      R = R8;
      long_form = true;
    }
  }
  if (!ok || kBufKb * P > kMaxCopies) return -1;
  geo.ahead = P;
  geo.weight_waves = nw;
  geo.rows_per_wave = R;
  const int lds = act_lds + nw * wave_bytes(P, R, long_form);
  if (lds > kLdsMax) return -1;
  const int grid = (int)((N + (long long)nw * R - 1) / ((long long)nw * R));
  constexpr bool kRegOk = MAXM == 1 && (TYPE == T_Q4_K || TYPE == T_Q8_0);
  const bool actreg = kRegOk && 64 % nb == 0;
  auto kern = long_form ? gemv_pipe_kernel<TYPE, MAXM, FUSEQ, false, true>
              : actreg  ? gemv_pipe_kernel<TYPE, MAXM, FUSEQ, kRegOk, false>
                        : gemv_pipe_kernel<TYPE, MAXM, FUSEQ, false, false>;
  allow_lds((const void*)kern, kLdsMax);
  PipePack pk;
  if (!pipe_pack(geo, nb, grid, pk) || ldy > 0x7FFFFFFF || row_bytes > 0x7FFFFFFF) return -1;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * (nw + na)), lds, stream, w, act.x, y,
                     (int)row_bytes, N, M, (int)ldy, pk.a, pk.b, act.q, act.d, act.bsums);
  return 0;
}

template <int TYPE>
constexpr int kStageKb = (15 + 64 * Lpb<TYPE>::kBytes + 1023) / 1024;  // copies of a full stage

// One launch over several weights of the K-quant / Q8_0 types that share the activations. Each
// weight gets workgroups in proportion to its bytes (at least one) and its own rows per wave; the
// stage buffers are sized for the largest block type. -1 when the shapes do not fit.
template <int MAXM, bool FUSEQ>
int launch_pipe_multi(const DecodeSeg* seg, int count, const Act& act, long long ldy, int M,
                      hipStream_t stream) {
  constexpr int kLdsMax = 160 * 1024;
  constexpr int kActBlk = QK + kActPad;
  const int nb = act.nb;
  if (count < 1 || count > kMaxSegs || nb > kWaveLanes) return -1;
  int buf_kb = 0;
  double total = 0.0;
  for (int i = 0; i < count; ++i) {
    const int t = seg[i].type;
    if (t != T_Q4_K && t != T_Q6_K && t != T_Q8_0) return -1;
    buf_kb = max(buf_kb, t == T_Q4_K ? kStageKb<T_Q4_K> : t == T_Q6_K ? kStageKb<T_Q6_K> : kStageKb<T_Q8_0>);
    total += (double)seg[i].n * (double)seg[i].row_bytes;
  }
  const int act_lds = M * nb * (kActBlk + 32 + 4) + 16;
  if (act_lds > 80 * 1024) return -1;
  const int na = min(4, (M * nb + 15) / 16);
  const int ncu = cu_count();
  PipeGeo geo;
  geo.act_waves = na;
  geo.buf_kb = buf_kb;
  PipeSegs segs;
  segs.count = count;
  int lds = 0, grid = 0;
  bool ok = false;
  for (int P = 1; P <= 2 && !ok; ++P) {
    for (int nw = 8; nw >= 2 && !ok; --nw) {
      int wg0 = 0, wave_max = 0;
      for (int i = 0; i < count; ++i) {
        const int share = max(1, (int)((double)ncu * seg[i].n * seg[i].row_bytes / total + 0.5));
        const int R = (seg[i].n + share * nw - 1) / (share * nw);
        const int wgs = (seg[i].n + nw * R - 1) / (nw * R);
        segs.s[i] = PipeSeg{seg[i].w, seg[i].row_bytes, seg[i].y, seg[i].n, seg[i].type, wg0, R};
        wg0 += wgs;
        const int nbuf = min(P + 1, (R * nb + 63) / 64);
        wave_max = max(wave_max, nbuf * buf_kb * 1024 + R * nb * 4 * (MAXM + 1));
      }
      if (act_lds + nw * wave_max <= kLdsMax && buf_kb * P <= kMaxCopies) {
        ok = true;
        geo.ahead = P;
        geo.weight_waves = nw;
        geo.rows_per_wave = 0;  // per segment
        lds = act_lds + nw * wave_max;
        grid = wg0;
      }
    }
  }
  if (!ok) return -1;
  const bool actreg = MAXM == 1 && 64 % nb == 0;
  auto kern = actreg ? gemv_pipe_multi_kernel<MAXM, FUSEQ, MAXM == 1> : gemv_pipe_multi_kernel<MAXM, FUSEQ, false>;
  allow_lds((const void*)gemv_pipe_multi_kernel<MAXM, FUSEQ, MAXM == 1>, kLdsMax);
  allow_lds((const void*)gemv_pipe_multi_kernel<MAXM, FUSEQ, false>, kLdsMax);
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * (geo.weight_waves + na)), lds, stream, segs, act,
                     ldy, M, geo);
  return 0;
}

template <int TYPE, int MAXM, bool FUSEQ>
int launch_decode(const uint8_t* w, long long row_bytes, const Act& act, YOut y, long long ldy,
                  int M, int N, hipStream_t stream) {
  if (launch_pipe<TYPE, MAXM, FUSEQ>(w, row_bytes, act, y, ldy, M, N, stream) == 0) return 0;
  return launch_lpb<TYPE, MAXM, FUSEQ>(w, row_bytes, act, y, ldy, M, N, stream);
}

template <int TYPE>
int launch_lpb_type(const uint8_t* w, long long row_bytes, const Act& act, YOut y, long long ldy,
                    int M, int N, hipStream_t stream) {
  constexpr bool kQ8K = !ActTraits<TYPE>::kFloat;
  const bool fuse = kQ8K && act.q == nullptr;
  if (M == 1) return fuse ? launch_decode<TYPE, 1, kQ8K>(w, row_bytes, act, y, ldy, M, N, stream)
                          : launch_decode<TYPE, 1, false>(w, row_bytes, act, y, ldy, M, N, stream);
  if (M == 2) return fuse ? launch_decode<TYPE, 2, kQ8K>(w, row_bytes, act, y, ldy, M, N, stream)
                          : launch_decode<TYPE, 2, false>(w, row_bytes, act, y, ldy, M, N, stream);
  return fuse ? launch_decode<TYPE, 4, kQ8K>(w, row_bytes, act, y, ldy, M, N, stream)
              : launch_decode<TYPE, 4, false>(w, row_bytes, act, y, ldy, M, N, stream);
}

}  // namespace

int launch_decode_multi(const DecodeSeg* seg, int count, const Act& act, long long ldy,
                        int m_rows, hipStream_t stream) {
  if (m_rows < 1 || m_rows > kFusedQuantMaxRows) return -1;
  const bool fuse = act.q == nullptr;
  if (m_rows == 1 && launch_gemv_wave_multi(seg, count, act, stream) == 0) return 0;
  if (fuse && act.xbf16) return -1;  // only the floor-shaped kernel reads bfloat16 x
  if (m_rows == 1) return fuse ? launch_pipe_multi<1, true>(seg, count, act, ldy, m_rows, stream)
                               : launch_pipe_multi<1, false>(seg, count, act, ldy, m_rows, stream);
  if (m_rows == 2) return fuse ? launch_pipe_multi<2, true>(seg, count, act, ldy, m_rows, stream)
                               : launch_pipe_multi<2, false>(seg, count, act, ldy, m_rows, stream);
  return fuse ? launch_pipe_multi<4, true>(seg, count, act, ldy, m_rows, stream)
              : launch_pipe_multi<4, false>(seg, count, act, ldy, m_rows, stream);
}

int launch_gemv_lpb(int type, const uint8_t* w, long long row_bytes, const Act& act, YOut y,
                    long long ldy, int m_rows, int n_rows, hipStream_t stream) {
  if (m_rows < 1 || m_rows > 4) return -1;
  if (m_rows == 1) {
    // one activation row: the floor-shaped kernel wherever it applies (measured faster at every
    // size on MI355X: Q4_K 4096 x 4096 3.8 vs 5.3 us, 14336 x 4096 7.4 vs 8.6 us), else the
    // workgroup-resident kernel for weights up to 12 MB
    if (launch_gemv_wave(type, w, row_bytes, act, y, n_rows, stream) == 0) return 0;
    if (act.q == nullptr && act.xbf16) return -1;  // only the floor-shaped kernel reads bf16 x
    if (launch_gemv_res(type, w, row_bytes, act, y, n_rows, stream) == 0) return 0;
  }
  if (m_rows >= 2 && launch_gemv_wave_m(type, w, row_bytes, act, y, ldy, m_rows, n_rows, stream) == 0)
    return 0;
  if (act.q == nullptr && act.xbf16) return -1;
  switch (type) {
    case T_Q4_K: return launch_lpb_type<T_Q4_K>(w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
    case T_Q6_K: return launch_lpb_type<T_Q6_K>(w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
    case T_Q8_0: return launch_lpb_type<T_Q8_0>(w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
    case T_IQ4_XS: return launch_lpb_type<T_IQ4_XS>(w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
    default: return -1;
  }
}

int launch_moe_lpb(int type, const uint8_t* w, long long row_bytes, long long expert_stride,
                   int n_experts, const Act& act, const int32_t* offsets, int total_rows,
                   int max_rows, YOut y, long long ldy, int n_rows, hipStream_t stream) {
  if (type != T_IQ4_XS || act.x == nullptr || act.xbf16 || ((uintptr_t)act.x & 15) != 0 ||
      n_experts < 1 || n_experts > 65535 || max_rows < 1 || n_rows < 1 || total_rows < 1)
    return -1;
  Geometry geo;
  int nw = 0, lds = 0;
  if (!lpb_geometry<T_IQ4_XS, 4>(act.nb, geo, nw, lds)) return -1;
  const int chunks = min((max_rows + 3) / 4, 65535);
  const int tile_rows = geo.rows_per_wave * nw;
  const dim3 grid((n_rows + tile_rows - 1) / tile_rows, n_experts, chunks);
  auto kern = moe_lpb_kernel<T_IQ4_XS>;
  if (lds > 64 * 1024) allow_lds((const void*)kern, 160 * 1024);
  hipLaunchKernelGGL(kern, grid, dim3(64 * nw), lds, stream, w, row_bytes, expert_stride, act,
                     offsets, total_rows, y, ldy, n_rows, geo);
  return 0;
}

int launch_gemv_f32(int type, const uint8_t* w, long long row_bytes, const float* x, int k,
                    YOut y, long long ldy, int m_rows, int n_rows, hipStream_t stream) {
  if (m_rows < 1 || m_rows > 4) return -1;
  Act act;
  act.q = nullptr, act.d = nullptr, act.bsums = nullptr, act.x = x;
  act.k = k, act.nb = k / QK, act.xsplit = nullptr, act.xbf16 = 0;
  // the floor-shaped kernel where it applies (the same bits as the pipelined kernel; measured on
  // MI355X, one row: Q4_K 14336 x 4096 11.3 vs 17.2 us, 4096 x 4096 5.7 vs 11.1, Q8_0 4096 x 4096
  // 7.0 vs 11.9, Q6_K 4096 x 14336 18.7 vs 27.7, the 128256 x 4096 head 83 vs 94; four rows Q4_K
  // 14336 x 4096 31.2 vs 50.3)
  if (type != T_IQ4_XS &&
      launch_gemv_wave_f32(type, w, row_bytes, act, y, ldy, m_rows, n_rows, stream) == 0)
    return 0;
  switch (type) {
    case T_Q4_K: return launch_lpb_type<T_Q4_K_F>(w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
    case T_Q6_K: return launch_lpb_type<T_Q6_K_F>(w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
    case T_Q8_0: return launch_lpb_type<T_Q8_0_F>(w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
    case T_IQ4_XS:
      // IQ4_XS always multiplies float activations: the kernels mxa_gemm uses for it (the same
      // summation order in every kernel, so the same bits)
      if (launch_gemv_wave_m(type, w, row_bytes, act, y, ldy, m_rows, n_rows, stream) == 0 ||
          (m_rows == 1 && launch_gemv_res(type, w, row_bytes, act, y, n_rows, stream) == 0))
        return 0;
      return launch_lpb_type<T_IQ4_XS>(w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
    default: return -1;
  }
}

}  // namespace mxa
