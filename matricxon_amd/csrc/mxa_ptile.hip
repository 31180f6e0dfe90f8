// Prefill (M >= 128 activation rows) on the matrix cores, weights and activations streamed through
// LDS: Q4_K (the other types keep mtile_kernel: their B operands need the registers that more
// activation tiles per wave would take).
//
// Tiles. A tile is 128 weight rows x 64 activation rows; a persistent workgroup per CU takes
// tiles t = slot, slot + grid, ... with the activation tile varying fastest and consecutive slots
// on one XCD, so the workgroups that share a weight tile run at the same time on one L2 and its
// second and later reads hit in cache. Eight compute waves each own 16 of the weight rows and all 64 activation rows (four
// 16-row MFMA tiles), so one B operand build (the VALU-heavy part) feeds 4 x 9 MFMAs.
//
// Stages. A stage is one tile and one 256-value block: the 128 weight rows' block (row pieces at
// an odd LDS chunk stride) and the activations' block, which the quantizer's regrouped layout
// holds as one contiguous range (q rows padded to 272 bytes, bsums as fp16, d). Four copy waves
// move stages into three LDS buffers with global_load_lds_dwordx4 and hand them to the compute
// waves through LDS counters, as in the streaming batched decode: ready[b] counts copy waves whose
// share of the stage in buffer b has landed, done[b] counts compute waves finished with it.
//
// Numerics. Every compute wave folds each (row, activation row) output over the blocks in order
// 0..nb-1 with the oracle's fused steps (app/native/src/mx_gemm.c:241-261): results equal the
// decode kernels and the oracle bit for bit.
#include "mxa_kernels.hpp"
#include "mxa_tiles.hpp"

#pragma clang fp contract(off)

namespace mxa {
namespace {

constexpr int kPtComputeWaves = 8;
constexpr int kPtCopyWaves = 4;
constexpr int kPtRows = 16 * kPtComputeWaves;  // weight rows per tile
constexpr int kPtMTiles = kPrefillRows / 16;    // 16-row activation tiles per compute wave
constexpr int kPtBuf = 3;

template <int TYPE>
constexpr int kPtBlockBytes = TYPE == T_Q4_K ? 144 : TYPE == T_Q6_K ? 210 : 272;

// LDS chunks per weight row piece (one block at any start offset), odd for distinct banks.
__host__ __device__ constexpr int pt_row_chunks(int block_bytes) {
  return ((block_bytes + 15 + 15) / 16) | 1;
}

struct PtGeo {
  int wbytes;     // LDS bytes of a stage's weight part (whole 1 KB copies)
  int buf_bytes;  // wbytes + kPrefillStageBytes rounded up to 1 KB
  int nmt;        // activation tiles
  int tiles;      // weight tiles x activation tiles
};

__device__ __forceinline__ int pt_load(const int* p) {
  return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void pt_add(int* p, int v) {
  __hip_atomic_fetch_add(p, v, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void pt_wait(const int* p, int target) {
  while (pt_load(p) < target) __builtin_amdgcn_s_sleep(1);
}

template <int TYPE>
__global__ __launch_bounds__(768) void ptile_kernel(const uint8_t* w, long long row_bytes, Act act,
                                                    float* __restrict__ y, long long ldy, int M,
                                                    int N, PtGeo geo) {
  using Tile = typename TileOf<TYPE>::T;
  constexpr int TB = kPtBlockBytes<TYPE>;
  constexpr int RS = pt_row_chunks(TB);
  constexpr int kWCopies = kPtRows * RS / 64;                            // exact: RS is per row
  constexpr int kACopies = (kPrefillStageBytes / 16 + 63) / 64;
  extern __shared__ __align__(16) uint8_t smem[];

  const int tid = threadIdx.x, lane = tid & 63, ln = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nb = act.nb;
  const int buf_bytes = geo.buf_bytes, wbytes = geo.wbytes;
  // tiles slot, slot + grid, ..: consecutive slots share an XCD, so the activation tiles of one
  // weight tile run on one XCD and share its L2
  const int slot = xcd_tile((int)blockIdx.x, (int)gridDim.x);
  const int my_tiles = (geo.tiles - slot + (int)gridDim.x - 1) / (int)gridDim.x;
  const int S = my_tiles * nb;
  int* ready = (int*)(smem + kPtBuf * buf_bytes);
  int* done = ready + kPtBuf;
  if (tid < 2 * kPtBuf) ready[tid] = 0;
  __syncthreads();

  auto tile_nt = [&](int s) { return (slot + (s / nb) * (int)gridDim.x) / geo.nmt; };
  auto tile_mt = [&](int s) { return (slot + (s / nb) * (int)gridDim.x) % geo.nmt; };

  if (wave >= kPtComputeWaves) {
    // ------------------------------------------------------------------ copy waves
    const int c = wave - kPtComputeWaves;
    const uint32_t lds0 = lds_addr(smem);
    // copies of a stage this wave issues: weight copies q = c, c + 4, ..; activation copies alike
    const int my_copies = (kWCopies - c + kPtCopyWaves - 1) / kPtCopyWaves +
                          (kACopies - c + kPtCopyWaves - 1) / kPtCopyWaves;
    auto issue = [&](int s) {
      const int b = s % nb, nt = tile_nt(s), mt = tile_mt(s);
      const uint32_t dst = lds0 + (uint32_t)((s % kPtBuf) * buf_bytes);
      // weight rows nt * kPtRows .. (rows past N repeat row N - 1: never stored)
      for (int q = c; q < kWCopies; q += kPtCopyWaves) {
        const int e = 64 * q + lane, j = e / RS, k = e - j * RS;
        const uintptr_t ra = (uintptr_t)(w + (size_t)min(nt * kPtRows + j, N - 1) * row_bytes + (size_t)b * TB);
        const int crow = (int)(((ra & 15) + TB + 15) >> 4);
        if (k < crow) copy16_to_lds((const void*)((ra & ~(uintptr_t)15) + 16 * k), dst + 1024 * q);
      }
      // the activation tile's block: one contiguous range
      const uint8_t* as = act.ablk + ((size_t)mt * nb + b) * kPrefillStageBytes + 16 * lane;
      for (int q = c; q < kACopies; q += kPtCopyWaves) {
        if (64 * q + lane < kPrefillStageBytes / 16)
          copy16_to_lds(as + 1024 * q, dst + (uint32_t)wbytes + 1024 * q);
      }
    };
    auto buffer_free = [&](int s) {
      return s < kPtBuf || pt_load(&done[s % kPtBuf]) >= (s / kPtBuf) * kPtComputeWaves;
    };
    int issued = 0;
    while (issued < min(kPtBuf, S)) issue(issued++);
    for (int sig = 0; sig < S; ++sig) {
      if (issued == sig) {
        pt_wait(&done[sig % kPtBuf], (sig / kPtBuf) * kPtComputeWaves);
        issue(issued++);
      }
      wait_vmcnt(my_copies * (issued - sig - 1));
      if (lane == 0) pt_add(&ready[sig % kPtBuf], 1);
      while (issued < S && buffer_free(issued)) issue(issued++);
    }
    return;
  }

  // -------------------------------------------------------------------- compute waves
  float acc[kPtMTiles][4];
#pragma unroll
  for (int ml = 0; ml < kPtMTiles; ++ml)
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[ml][e] = 0.0f;
  const int jrow = 16 * wave + ln;  // this lane's weight row in the tile
  for (int s = 0; s < S; ++s) {
    const int b = s % nb, nt = tile_nt(s), mt = tile_mt(s), buf = s % kPtBuf;
    pt_wait(&ready[buf], (s / kPtBuf + 1) * kPtCopyWaves);
    const uint8_t* st = smem + buf * buf_bytes;
    const int n = nt * kPtRows + jrow;
    const int roff = jrow * RS * 16 +
                     (int)((uintptr_t)(w + (size_t)min(n, N - 1) * row_bytes + (size_t)b * TB) & 15);
    const typename Tile::P pp = Tile::prep(Tile::load_lds(st, roff, g), g);
    const ActTile A{(const int8_t*)(st + wbytes), (const _Float16*)(st + wbytes + kPrefillRows * kPrefillQStride),
                    kPrefillQStride, 16};
    const float* ad = (const float*)(st + wbytes + kPrefillRows * (kPrefillQStride + 32));
#pragma unroll
    for (int ml = 0; ml < kPtMTiles; ++ml) {
      const typename Tile::F f = Tile::frag(A, 0, ml, ln, g);
      Tile::template value<true>(pp, f, g, [&](int e, float v, float dd) {
        acc[ml][e] = Tile::fold(acc[ml][e], ad[16 * ml + 4 * g + e], v, dd);
      });
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's reads of the buffer are done
    if (lane == 0) pt_add(&done[buf], 1);
    if (b == nb - 1) {  // the tile's outputs
#pragma unroll
      for (int ml = 0; ml < kPtMTiles; ++ml)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int m = mt * kPrefillRows + 16 * ml + 4 * g + e;
          if (m < M && n < N) y[(size_t)m * ldy + n] = acc[ml][e];
          acc[ml][e] = 0.0f;
        }
    }
  }
}

template <int TYPE>
int launch_pt(const uint8_t* w, long long row_bytes, const Act& act, float* y, long long ldy, int M,
              int N, hipStream_t stream) {
  constexpr int kLdsMax = 160 * 1024;
  PtGeo geo;
  geo.wbytes = (kPtRows * pt_row_chunks(kPtBlockBytes<TYPE>) * 16 + 1023) / 1024 * 1024;
  geo.buf_bytes = (geo.wbytes + kPrefillStageBytes + 1023) / 1024 * 1024;
  const int lds = kPtBuf * geo.buf_bytes + 4 * kPtBuf * 4;
  if (lds > kLdsMax) return -1;
  geo.nmt = (M + kPrefillRows - 1) / kPrefillRows;
  const long long tiles = (long long)((N + kPtRows - 1) / kPtRows) * geo.nmt;
  if (tiles > (1 << 30)) return -1;
  geo.tiles = (int)tiles;
  static bool lds_set = false;
  if (!lds_set) {
    (void)hipFuncSetAttribute((const void*)ptile_kernel<TYPE>, hipFuncAttributeMaxDynamicSharedMemorySize,
                              kLdsMax);
    lds_set = true;
  }
  const int grid = min(geo.tiles, cu_count());
  hipLaunchKernelGGL((ptile_kernel<TYPE>), dim3(grid), dim3(64 * (kPtComputeWaves + kPtCopyWaves)), lds,
                     stream, w, row_bytes, act, y, ldy, M, N, geo);
  return 0;
}

}  // namespace

int launch_ptile(int type, const uint8_t* w, long long row_bytes, const Act& act, float* y,
                 long long ldy, int m_rows, int n_rows, hipStream_t stream) {
  if (act.ablk == nullptr || m_rows < kPrefillMinRows || n_rows < 1) return -1;
  switch (type) {
    case T_Q4_K: return launch_pt<T_Q4_K>(w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
    default: return -1;
  }
}

}  // namespace mxa
