// Matrix-core matmul for M > 4 activation rows (batched decode and prefill), Q4_K / Q6_K / Q8_0.
//
// Tiling. A workgroup of WAVES waves owns 16 * NT consecutive weight rows per wave and 16 * MT
// activation rows; grid.y walks the activation rows, so a weight block is read once per 16 * MT
// activation rows and an activation chunk once per 16 * NT * WAVES weight rows. The Q8_K
// activations (always pre-quantized in the workspace here) are staged in LDS per chunk of kCB
// blocks, in two buffers: the next chunk is loaded into registers while the current one is
// computed and written to the other buffer afterwards, so one barrier per chunk suffices (a
// buffer is rewritten only after every wave has passed the barrier that ends its last use). Each
// wave loads its rows' block two ahead while it computes the current one.
//
// Operands: the tile builders of mxa_tiles.hpp, with A (16 activation rows x 64 k) read from LDS.
// The blocks are folded in order 0..nb-1, so the outputs equal the oracle and the decode kernels
// bit for bit.
#include "mxa_kernels.hpp"
#include "mxa_tiles.hpp"

#pragma clang fp contract(off)

namespace mxa {
namespace {

constexpr int kCB = 2;                    // blocks per activation chunk
constexpr int kQStride = kCB * QK + 16;   // LDS bytes per activation row (padding: distinct banks)
constexpr int kBStride = kCB * 16 + 8;    // LDS halves per activation row of bsums


// LDS bytes of one activation chunk buffer for 16 * MT rows: q8 | bsums (fp16) | d.
template <int MT>
constexpr int kMtBuf = ((16 * MT * kQStride + 16 * MT * kBStride * 2 + kCB * 16 * MT * 4) + 15) / 16 * 16;

// Row-tiled body: MT activation tiles x NT weight tiles of 16 rows per wave, WAVES waves;
// workgroup wg of n_wg along N, activation tile group mg (rows 16 MT mg ..) of M rows.
template <int TYPE, int MT, int NT, int WAVES>
__device__ __forceinline__ void mtile_rows(const uint8_t* w, long long row_bytes, const Act& act,
                                           YOut y, long long ldy, int M, int N, int wg, int n_wg,
                                           int mg) {
  using Tile = typename TileOf<TYPE>::T;
  using W = typename Tile::W;
  constexpr int kRows = 16 * MT;
  constexpr int kThreads = 64 * WAVES;
  extern __shared__ __align__(16) uint8_t smem[];  // two chunk buffers of kMtBuf<MT> bytes
  auto aq = [&](int buf) { return (int8_t*)(smem + buf * kMtBuf<MT>); };
  auto ab = [&](int buf) { return (_Float16*)(smem + buf * kMtBuf<MT> + kRows * kQStride); };
  auto ad = [&](int buf) { return (float*)(smem + buf * kMtBuf<MT> + kRows * kQStride + kRows * kBStride * 2); };

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int ln = lane & 15, g = lane >> 4;
  const int n0 = xcd_tile(wg, n_wg) * WAVES * 16 * NT + 16 * NT * wave;
  const int m0 = mg * kRows;
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

  // weight blocks two ahead of the one computed (one ahead measured 4-6% slower: a block's
  // compute does not cover the load latency; three ahead no faster)
  W cur[NT], nxt[NT], nx2[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    cur[nt] = Tile::load(row[nt], 0, g);
    nxt[nt] = Tile::load(row[nt], min(1, nb - 1), g);
  }

  // Activation staging, software-pipelined: chunk c + 1 is loaded into registers while chunk c
  // is computed, and written to LDS between the two barriers. Thread tid owns the same pieces of
  // every chunk (rows >= M repeat row M - 1, blocks >= cn repeat the chunk's last block: those
  // results are never stored).
  constexpr int kQPieces = kRows * kCB * 16;                   // 16-byte pieces of q8
  constexpr int kQPer = (kQPieces + kThreads - 1) / kThreads;
  constexpr int kBPieces = kRows * kCB * 2;                    // halves of a block's 16 bsums
  constexpr int kBPer = (kBPieces + kThreads - 1) / kThreads;
  constexpr int kDPer = (kRows * kCB + kThreads - 1) / kThreads;
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
      const int p = min(tid + kThreads * j, kQPieces - 1);
      const int r = p / (kCB * 16), o = p - r * (kCB * 16), bb = min(o >> 4, cn - 1), pc = o & 15;
      st.q[j] = ld16((const uint8_t*)(act.q + (size_t)min(m0 + r, M - 1) * act.k + (size_t)(c0 + bb) * QK) + 16 * pc);
    }
#pragma unroll
    for (int j = 0; j < kBPer; ++j) {
      const int p = min(tid + kThreads * j, kBPieces - 1);
      const int r = p / (kCB * 2), o = p - r * (kCB * 2), bb = min(o >> 1, cn - 1), hf = o & 1;
      st.b[j] = ld16((const uint8_t*)(act.bsums + ((size_t)min(m0 + r, M - 1) * nb + c0 + bb) * 16) + 16 * hf);
    }
#pragma unroll
    for (int j = 0; j < kDPer; ++j) {
      const int p = min(tid + kThreads * j, kRows * kCB - 1), bb = p / kRows, r = p - bb * kRows;
      st.d[j] = act.d[(size_t)min(m0 + r, M - 1) * nb + c0 + min(bb, cn - 1)];
    }
    return st;
  };
  auto store_stage = [&](const Stage& st, int buf) {
    int8_t* Aq = aq(buf);
    _Float16* Ab = ab(buf);
    float* Ad = ad(buf);
#pragma unroll
    for (int j = 0; j < kQPer; ++j) {
      const int p = tid + kThreads * j;
      if (p < kQPieces) {
        const int r = p / (kCB * 16), o = p - r * (kCB * 16);
        *(u32x4a4*)(Aq + r * kQStride + (o >> 4) * QK + 16 * (o & 15)) = st.q[j];
      }
    }
#pragma unroll
    for (int j = 0; j < kBPer; ++j) {
      const int p = tid + kThreads * j;
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
      const int p = tid + kThreads * j;
      if (p < kRows * kCB) Ad[p] = st.d[j];
    }
  };

  {
    const Stage st0 = load_stage(0);
    store_stage(st0, 0);
  }
  __syncthreads();
  for (int c0 = 0; c0 < nb; c0 += kCB) {
    const int cn = min(kCB, nb - c0), buf = (c0 / kCB) & 1;
    const bool more = c0 + kCB < nb;
    Stage st;
    if (more) st = load_stage(c0 + kCB);
    // the chunk's blocks in order; the next block's weights load meanwhile
    const ActTile A{aq(buf), ab(buf), kQStride, kBStride};
    const float* Ad = ad(buf);
#pragma unroll
    for (int i = 0; i < kCB; ++i) {
      if (i < cn) {
        const int b = c0 + i;
        if (b + 2 < nb) {
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) nx2[nt] = Tile::load(row[nt], b + 2, g);
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
          // no scheduling barrier between tiles: the compiler overlaps one tile's fold with the
          // next tile's A reads and MFMAs (222 VGPRs at MT = 8, no spills; measured 7% faster at
          // M = 512 and 6% at M = 2048 than one tile at a time)
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          cur[nt] = nxt[nt];
          nxt[nt] = nx2[nt];
        }
      }
    }
    if (more) store_stage(st, buf ^ 1);
    __syncthreads();  // the next chunk is in LDS; every wave is done with this one
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

template <int TYPE, int MT, int NT, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void mtile_kernel(const uint8_t* w, long long row_bytes, Act act,
                                                           YOut y, long long ldy, int M,
                                                           int N) {
  mtile_rows<TYPE, MT, NT, WAVES>(w, row_bytes, act, y, ldy, M, N, blockIdx.x, gridDim.x,
                                  blockIdx.y);
}

// Grouped MoE projection on the row-tiled body: every expert's rows [offsets[e], offsets[e + 1])
// (clamped into [0, total_rows), as moe_dec_kernel below clamps them) are cut into chunks of 16 MT
// rows, and workgroup z of the grid's third dimension takes item z of the list of (expert, chunk)
// pairs, experts in order, so a weight tile is read once per 16 MT rows of its expert instead of
// once per 16. Every wave finds its item from the offset table (lane l counts the chunks of
// experts 4 l .. 4 l + 3, a wave prefix sum locates item z), so the list covers every row whatever
// the routing: an expert that a token names twice has more rows than tokens, and the host sizes
// the grid by n_experts + ceil(total_rows / (16 MT)), which bounds the list's length. A workgroup
// past the list's end exits. n_experts <= 256. (One chunk per workgroup: a loop over chunks made
// the Q6_K body spill.)
template <int TYPE, int MT, int NT, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void moe_mtile_kernel(const uint8_t* w, long long row_bytes,
                                                               long long expert_stride, Act act,
                                                               const int32_t* __restrict__ offsets,
                                                               int n_experts, int total_rows, YOut y,
                                                               long long ldy, int N) {
  int e, p0, M;
  // past the list: uniform over the workgroup, before any barrier
  if (!moe_chunk_item(offsets, n_experts, total_rows, 16 * MT, blockIdx.z, e, p0, M)) return;
  Act a = act;
  a.q = act.q + (size_t)p0 * act.k;
  a.d = act.d + (size_t)p0 * act.nb;
  a.bsums = act.bsums + (size_t)p0 * act.nb * 16;
  mtile_rows<TYPE, MT, NT, WAVES>(w + (size_t)e * expert_stride, row_bytes, a,
                                  y.at((size_t)p0 * ldy), ldy, M, N, blockIdx.x, gridDim.x, 0);
}

// Batched decode (M <= 16): 32 weight rows per workgroup and the blocks of each chunk split over
// the 4 waves (wave w takes blocks w and w + 4 of an 8-block chunk, for both 16-row tiles), so that
// N = 4096..14336 still gives the GPU 128..448 workgroups. The block values go through LDS and are
// folded in block order by the thread that owns the output.
constexpr int kDecCh = 8;                     // blocks per chunk
constexpr int kDecQStride = kDecCh * QK + 16;
constexpr int kDecBStride = kDecCh * 16 + 8;

// kDecRT 16-row weight tiles per group: 2, or 1 for Q6_K (its per-lane block bytes need twice
// the registers; one tile keeps two waves per SIMD). The body of one workgroup: groups
// wg * kGroups .. + kGroups - 1 of n_wg * kGroups (16 kDecRT rows each) against M <= 16
// activation rows. A chunk's activations are staged once for all of the workgroup's groups (at
// 16 activation rows they weigh as much as 32 weight rows of the chunk), and each (chunk, group)
// step loads the next step's weights while it computes.
template <int TYPE, int kDecRT, int kGroups = 1>
__device__ __forceinline__ void mdec_rows(const uint8_t* w, long long row_bytes, const Act& act,
                                          YOut y, long long ldy, int M, int N, int wg,
                                          int n_wg) {
  using Tile = typename TileOf<TYPE>::T;
  using W = typename Tile::W;
  __shared__ __align__(16) int8_t Aq[16 * kDecQStride];
  __shared__ __align__(16) _Float16 Ab[16 * kDecBStride];
  __shared__ float Ad[kDecCh * 16];
  __shared__ float Tp[kDecRT][kDecCh][16][16];  // block values [tile][block][m][n]
  __shared__ float Dp[kDecRT][kDecCh][16];      // the block's weight scale where the fold uses one

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int ln = lane & 15, g = lane >> 4;
  const int n0 = xcd_tile(wg, n_wg) * 16 * kDecRT * kGroups;
  auto row_of = [&](int grp, int t) {
    return w + (size_t)min(n0 + 16 * (kDecRT * grp + t) + ln, N - 1) * row_bytes;
  };
  const int nb = act.nb;
  constexpr int kOut = kDecRT * 256 / 256;  // outputs per thread and group: kDecRT x 16 x 16 / 256
  float acc[kGroups][kOut];
#pragma unroll
  for (int grp = 0; grp < kGroups; ++grp)
#pragma unroll
    for (int k = 0; k < kOut; ++k) acc[grp][k] = 0.0f;

  // this wave's blocks wave and wave + 4 of chunk c0 for group grp (blocks past the chunk repeat
  // its last one: their values are never folded)
  auto load_step = [&](W (&dst)[2][kDecRT], int c0, int grp) {
    const int cn = min(kDecCh, nb - c0);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int t = 0; t < kDecRT; ++t) dst[i][t] = Tile::load(row_of(grp, t), c0 + min(wave + 4 * i, cn - 1), g);
  };
  W cur[2][kDecRT], nxt[2][kDecRT];
  load_step(cur, 0, 0);
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
    const ActTile A{Aq, Ab, kDecQStride, kDecBStride};
#pragma unroll
    for (int grp = 0; grp < kGroups; ++grp) {
      // 2. the next step's weights: the next group of this chunk, or the first of the next chunk
      const bool more = grp + 1 < kGroups || c0 + kDecCh < nb;
      if (more) load_step(nxt, grp + 1 < kGroups ? c0 : c0 + kDecCh, grp + 1 < kGroups ? grp + 1 : 0);
      __syncthreads();  // the chunk is in LDS; the previous step's fold has read Tp
      // 3. this wave's blocks, every tile of the group: values into LDS
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
      // 4. fold the chunk's blocks in order: thread -> outputs (tile, m, n) of the group
#pragma unroll
      for (int k = 0; k < kOut; ++k) {
        const int idx = tid + 256 * k, t = idx >> 8, m = (idx >> 4) & 15, n = idx & 15;
        for (int bb = 0; bb < cn; ++bb)
          acc[grp][k] = Tile::fold(acc[grp][k], Ad[bb * 16 + m], Tp[t][bb][m][n], Dp[t][bb][n]);
      }
      if (more) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int t = 0; t < kDecRT; ++t) cur[i][t] = nxt[i][t];
      }
    }
    __syncthreads();  // every fold has read Ad and Tp before the next chunk is staged
  }
#pragma unroll
  for (int grp = 0; grp < kGroups; ++grp)
#pragma unroll
    for (int k = 0; k < kOut; ++k) {
      const int idx = tid + 256 * k, t = idx >> 8, m = (idx >> 4) & 15;
      const int n = n0 + 16 * (kDecRT * grp + t) + (idx & 15);
      if (m < M && n < N) y.put((size_t)m * ldy + n, acc[grp][k]);
    }
}

template <int TYPE, int kDecRT>
__global__ __launch_bounds__(256) void mdec_kernel(const uint8_t* w, long long row_bytes, Act act,
                                                   YOut y, long long ldy, int M, int N) {
  mdec_rows<TYPE, kDecRT>(w, row_bytes, act, y, ldy, M, N, blockIdx.x, gridDim.x);
}

// Grouped MoE projection: expert e = blockIdx.y multiplies its rows [offsets[e], offsets[e + 1])
// of the Q8_K activations by its packed weight (w + e * expert_stride); the outputs go to the same
// rows of y. The expert's rows are taken 16 at a time, chunk z by the workgroups of blockIdx.z ==
// z mod gridDim.z, so every row is computed whatever the grid's depth (the host sizes it from a
// bound it knows without a sync; an expert with more rows loops). A workgroup whose expert has no
// row in its chunks exits. The offsets come from the device, so they are clamped to
// [0, total_rows): a bad table gives wrong rows, never an access outside the activations or y.
// Two waves per SIMD asked of the compiler: the chunk loop left to itself took Q6_K to 272 VGPRs
// (one workgroup per CU instead of two; the down projection ran 1.5x longer), with the bound it
// fits 206 VGPRs with no scratch (Q8_0 227, Q4_K 202).
template <int TYPE, int kDecRT, int kGroups>
__global__ __launch_bounds__(256, 2) void moe_dec_kernel(const uint8_t* w, long long row_bytes,
                                                      long long expert_stride, Act act,
                                                      const int32_t* __restrict__ offsets,
                                                      int total_rows, YOut y,
                                                      long long ldy, int N) {
  const int e = blockIdx.y;
  const int begin = min(max(offsets[e], 0), total_rows);
  const int end = min(max(offsets[e + 1], begin), total_rows);
  for (int p0 = begin + 16 * (int)blockIdx.z; p0 < end; p0 += 16 * (int)gridDim.z) {
    const int M = min(16, end - p0);  // uniform over the workgroup
    Act a = act;
    a.q = act.q + (size_t)p0 * act.k;
    a.d = act.d + (size_t)p0 * act.nb;
    a.bsums = act.bsums + (size_t)p0 * act.nb * 16;
    mdec_rows<TYPE, kDecRT, kGroups>(w + (size_t)e * expert_stride, row_bytes, a, y.at((size_t)p0 * ldy),
                                     ldy, M, N, blockIdx.x, gridDim.x);
    __syncthreads();  // the next chunk rewrites the LDS tiles this one read
  }
}

template <int TYPE, int MT, int NT, int WAVES>
int launch_mt(const uint8_t* w, long long row_bytes, const Act& act, YOut y, long long ldy, int M,
              int N, hipStream_t stream) {
  constexpr int kLds = 2 * kMtBuf<MT>;
  allow_lds((const void*)mtile_kernel<TYPE, MT, NT, WAVES>, kLds);
  const int rows = WAVES * 16 * NT;
  const dim3 grid((N + rows - 1) / rows, (M + 16 * MT - 1) / (16 * MT));
  hipLaunchKernelGGL((mtile_kernel<TYPE, MT, NT, WAVES>), grid, dim3(64 * WAVES), kLds, stream, w,
                     row_bytes, act, y, ldy, M, N);
  return 0;
}

template <int TYPE>
int launch_mt_type(const uint8_t* w, long long row_bytes, const Act& act, YOut y, long long ldy,
                   int M, int N, hipStream_t stream) {
  // M <= 16: the streaming kernel, else the block-split kernel unless the 64-row tiles alone give
  // >= 512 workgroups
  // M <= 16: the per-wave streaming kernel where its slots fit LDS (measured on MI355X at M = 16,
  // the same bits: Q4_K 4096 x 4096 5.7 vs 7.1 us, 1024 x 4096 5.4 vs 6.3, Q8_0 4096 x 4096 7.1 vs
  // 8.4; Q4_K 14336 x 4096 12.1 vs 12.0-12.3), then the copy-wave kernels
  if (M <= 16 && launch_bwave(TYPE, w, row_bytes, act, y, ldy, M, N, stream) == 0) return 0;
  if (M <= 16 && launch_bflow(TYPE, w, row_bytes, act, y, ldy, M, N, stream) == 0) return 0;
  if (M <= 16 && launch_bres(TYPE, w, row_bytes, act, y, ldy, M, N, stream) == 0) return 0;
  if (M <= 16 && launch_bstream(TYPE, w, row_bytes, act, y, ldy, M, N, stream) == 0) return 0;
  if (M <= 16 && N < 512 * 64) {
    constexpr int RT = TYPE == T_Q6_K ? 1 : 2;
    const int tiles = (N + 16 * RT - 1) / (16 * RT);
    hipLaunchKernelGGL((mdec_kernel<TYPE, RT>), dim3(tiles), dim3(256), 0, stream, w, row_bytes, act, y, ldy, M, N);
    return 0;
  }
  // up to 64 rows: 16-row activation tiles and 64 weight rows per workgroup; prefill: 64
  // activation rows x 128 weight rows (8 waves)
  if (M <= 64) return launch_mt<TYPE, 1, 1, 4>(w, row_bytes, act, y, ldy, M, N, stream);
  constexpr int NT = 1;
  if constexpr (TYPE == T_Q4_K)
    if (M > 256) return launch_mt<TYPE, 8, NT, 8>(w, row_bytes, act, y, ldy, M, N, stream);
  return launch_mt<TYPE, 4, NT, 8>(w, row_bytes, act, y, ldy, M, N, stream);
}

}  // namespace

bool mtile_supported(int type) { return type == T_Q4_K || type == T_Q6_K || type == T_Q8_0; }

int launch_moe_dec(int type, const uint8_t* w, long long row_bytes, long long expert_stride,
                   int n_experts, const Act& act, const int32_t* offsets, int total_rows,
                   int max_rows, YOut y, long long ldy, int n_rows, hipStream_t stream) {
  if (act.q == nullptr || n_experts < 1 || n_experts > 65535 || max_rows < 1 || n_rows < 1 ||
      total_rows < 1)
    return -1;
  const int chunks = (max_rows + 15) / 16;
  if (chunks > 65535) return -1;
  // Past 32 rows per expert (the bound), 64-row chunks through the prefill tile body read each
  // weight tile once per 64 rows instead of once per 16 (measured on MI355X, eager forward at
  // 128 tokens, the same bits: 8 experts top 2, 4096 x 14336, 607 vs 1058 us; 40 experts top 8,
  // 1536 x 512, 99-113 vs 176 us; at 16 tokens both forms tie)
  // Up to 32 rows, expert matrices of 4096 rows and more take 16-row chunks through the same body
  // (64 weight rows per 4-wave workgroup): same box, forward only, 8 experts top 2 (4096 x 14336),
  // 8 / 16 / 24 / 32 tokens 404 / 392 / 406 / 410 vs 443 / 429 / 441 / 445 us on the decode tile;
  // the 40 small experts (512 and 1536 rows) tie or lose, so they keep the decode tile.
  constexpr int kMoeMtileMinRows = 32, kMoeSmallTileMinN = 4096;
  // mt activation tiles and `waves` waves of 16 weight rows per workgroup; the grid's third
  // dimension bounds the (expert, chunk) list whatever the per-expert counts
  auto go_mt = [&](auto k_q4, auto k_q8, auto k_q6, int mt, int waves, int lds) {
    const int rows = 16 * mt, wg_rows = 16 * waves;
    const dim3 grid((n_rows + wg_rows - 1) / wg_rows, 1, n_experts + (total_rows + rows - 1) / rows);
    auto run = [&](auto kern) {
      allow_lds((const void*)kern, lds);
      hipLaunchKernelGGL(kern, grid, dim3(64 * waves), lds, stream, w, row_bytes, expert_stride,
                         act, offsets, n_experts, total_rows, y, ldy, n_rows);
      return 0;
    };
    switch (type) {
      case T_Q4_K: return run(k_q4);
      case T_Q8_0: return run(k_q8);
      case T_Q6_K: return run(k_q6);
      default: return -1;
    }
  };
  // Up to 96 rows per expert, expert matrices of 1024 rows and more take the batched-decode
  // bodies (short and long rows) in 16-row chunks, the CUs shared among the experts that can have
  // rows. Measured on MI355X, eager forward of 64 experts top 8 (2048 x 1024) at 4 / 16 / 32 / 64
  // tokens 100 / 171 / 188 / 204 us against 123 / 170 / 186 / 222 on the decode tile and prefill
  // tile bodies, 16 experts top 4 (3072 x 2048) 104 / 97 / 109 / 166 against 135 / 131 / 140 /
  // 178; 8 experts top 2 (4096 x 14336), the same bits:
  // 16 / 24 / 32 / 48 / 64 / 80 / 96 tokens 304 / 299 / 298 / 538 / 536 / 558 / 545 us against
  // 395 / 415 / 414 / 571 / 596 / 608 / 598 on the prefill tile bodies; at 112 / 128 tokens the
  // decode bodies lose (786 / 794 vs 594 / 607 us: more 16-row chunks per expert), so larger bounds
  // keep the prefill tile body.
  constexpr int kMoeDecodeBodyMaxRows = 96, kMoeDecodeBodyMinN = 1024;
  if (max_rows <= kMoeDecodeBodyMaxRows && n_rows >= kMoeDecodeBodyMinN &&
      launch_moe_bwave(type, w, row_bytes, expert_stride, n_experts, act, offsets, total_rows, y,
                       ldy, n_rows, stream) == 0)
    return 0;
  const bool list_fits = n_experts <= 256 && n_experts + (total_rows + 15) / 16 <= 65535;
  if (list_fits && max_rows > kMoeMtileMinRows)
    return go_mt(moe_mtile_kernel<T_Q4_K, 4, 1, 8>, moe_mtile_kernel<T_Q8_0, 4, 1, 8>,
                 moe_mtile_kernel<T_Q6_K, 4, 1, 8>, 4, 8, 2 * kMtBuf<4>);
  if (list_fits && n_rows >= kMoeSmallTileMinN)
    return go_mt(moe_mtile_kernel<T_Q4_K, 1, 1, 4>, moe_mtile_kernel<T_Q8_0, 1, 1, 4>,
                 moe_mtile_kernel<T_Q6_K, 1, 1, 4>, 1, 4, 2 * kMtBuf<1>);
  // Tile groups per workgroup (each group's chunk of activations staged once for all of them):
  // the most of 4, 2, 1 that still gives two workgroups per CU (Q8_0 at most 2: four spill).
  // Measured on MI355X, eager forward of 8 experts top 2 (4096 x 14336; Q4_K gate / up, Q6_K
  // down), the same bits: 16 tokens 498 vs 523 us, 128 tokens 1146 vs 1364; with four groups
  // forced, 40 small experts at 16 tokens lost (214 vs 204 us) to the smaller grid.
  auto go = [&](auto k1, auto k2, auto k4, int rt, int gmax) {
    const long long want = 2LL * cu_count();
    const int t1 = (n_rows + 16 * rt - 1) / (16 * rt);
    auto grid_of = [&](int gs) { return (long long)((t1 + gs - 1) / gs) * n_experts * chunks; };
    const int gs = gmax >= 4 && grid_of(4) >= want ? 4 : gmax >= 2 && grid_of(2) >= want ? 2 : 1;
    const dim3 grid((t1 + gs - 1) / gs, n_experts, chunks);
    if (gs == 4)
      hipLaunchKernelGGL(k4, grid, dim3(256), 0, stream, w, row_bytes, expert_stride, act, offsets,
                         total_rows, y, ldy, n_rows);
    else if (gs == 2)
      hipLaunchKernelGGL(k2, grid, dim3(256), 0, stream, w, row_bytes, expert_stride, act, offsets,
                         total_rows, y, ldy, n_rows);
    else
      hipLaunchKernelGGL(k1, grid, dim3(256), 0, stream, w, row_bytes, expert_stride, act, offsets,
                         total_rows, y, ldy, n_rows);
    return 0;
  };
  switch (type) {
    case T_Q4_K:
      return go(moe_dec_kernel<T_Q4_K, 2, 1>, moe_dec_kernel<T_Q4_K, 2, 2>,
                moe_dec_kernel<T_Q4_K, 2, 4>, 2, 4);
    case T_Q8_0:  // k4 is never taken (gmax 2): the two-group form stands in
      return go(moe_dec_kernel<T_Q8_0, 2, 1>, moe_dec_kernel<T_Q8_0, 2, 2>,
                moe_dec_kernel<T_Q8_0, 2, 2>, 2, 2);
    case T_Q6_K:
      return go(moe_dec_kernel<T_Q6_K, 1, 1>, moe_dec_kernel<T_Q6_K, 1, 2>,
                moe_dec_kernel<T_Q6_K, 1, 4>, 1, 4);
    default: return -1;
  }
}

int launch_mtile(int type, const uint8_t* w, long long row_bytes, const Act& act, YOut y,
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
