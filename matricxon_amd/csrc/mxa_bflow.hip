// Batched decode (up to 16 activation rows, rows of up to 16 blocks) on the matrix cores, with the
// workgroup's whole weight share resident in LDS.
//
// Work split. One workgroup per CU owns R consecutive weight rows (R = ceil(N / CUs)): T =
// ceil(R / 16) tiles of 16 rows, every one of them in LDS at once, so no buffer is ever reused.
// Row j sits in a row slot of rs 16-byte chunks (rs odd, so the 16 rows a B-operand read touches
// fall in different banks); row slots follow each other, so tile t starts at row slot 16 t.
//
// Copy waves. Four waves stream the rows in with global_load_lds_dwordx4, copy q moving LDS
// chunks 64 q .. 64 q + 63 of the row slots (chunk k of slot j is byte 16 k of row j, or for the
// padding chunk the next row's first bytes), copy q by copy wave q mod 4, in order. They do
// nothing else: a CU accepts only about 64 KB of copies in flight and a wave stalls at the
// instruction beyond that, so the stream runs at full rate from the first microsecond whatever
// the compute waves wait for. After a copy has landed (its own vmcnt) a copy wave publishes its
// frontier: every copy below min over copy waves of (k + 4 * landed_k) is in LDS. A lane's source
// address advances by 64 * 4 chunks per copy, a row boundary or two at a time.
//
// Compute waves. They split the blocks of a row: wave w owns blocks w * C .. w * C + C - 1 and
// keeps their Q8_K activations (the MFMA A operands of all 16 activation rows) in registers. For
// each tile, once the frontier has passed the tile's last chunk, a wave builds the B operands of
// its blocks from LDS with the tile builders of mxa_tiles.hpp and writes the block values over
// its own blocks' bytes in the row slots (no other wave reads those bytes, and every copy into
// them has landed), then counts computed[t]. One tile later (and after the last tile) every
// compute wave folds its share of a finished tile: output (weight row, activation row) over
// blocks 0..nb-1 in order with the oracle's fused steps (app/native/src/mx_dot_k_ssse3.c:115-154), so
// the results equal the other decode kernels and the oracle bit for bit.
//
// Every counter only grows and every wait is for a value the other waves always reach; each wait
// also gives up after a bounded number of polls, so no wave can spin forever. A wait that gave up
// turns what its wave writes next (block values or outputs) into NaN, so such a trip cannot pass
// for a result.
#include "mxa_kernels.hpp"
#include "mxa_tiles.hpp"

#pragma clang fp contract(off)

namespace mxa {
namespace {

template <int TYPE>
constexpr int kBfBlockBytes = TYPE == T_Q4_K ? 144 : TYPE == T_Q6_K ? 210 : 272;
constexpr int kBfCopyWaves = 4;
constexpr int kBfMaxTiles = 16;
constexpr int kBfLds = 160 * 1024;
constexpr int kBfSpinLimit = 1 << 22;  // polls before a wait gives up (about 0.1 s)

struct BfGeo {
  int rows_per_wg;  // R
  int rs;           // LDS chunks per row slot (odd)
  int ncw;          // compute waves: ceil(nb / C)
  int ctrl_off;     // LDS offset of the activation scales, then the counters
};

typedef __attribute__((address_space(3))) int lds_int;
typedef int i32x4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i32x4v lds_i32x4;

// LDS counters through LDS-qualified pointers (a volatile access through a generic pointer
// becomes a flat instruction, which counts on vmcnt and would wait for every copy in flight).
__device__ __forceinline__ int bf_load(int* p) { return *(volatile lds_int*)(lds_int*)p; }
__device__ __forceinline__ void bf_store(int* p, int v) { *(volatile lds_int*)(lds_int*)p = v; }
__device__ __forceinline__ void bf_add(int* p, int v) {
  __atomic_fetch_add((lds_int*)p, v, __ATOMIC_RELAXED);
}
// Copies below the smallest of the four copy-wave frontiers (one 16-byte LDS read) have landed.
__device__ __forceinline__ int bf_frontier(int* cnt) {
  const i32x4v f = *(volatile lds_i32x4*)(lds_i32x4*)cnt;
  return min(min(f.x, f.y), min(f.z, f.w));
}

// Copy wave cw of a tile: copies q = cw, cw + 4, ... < nqt (1 KB each) of the tile's 16 row slots;
// chunk e = 64 q + lane is chunk k = e mod rs of row slot j = e / rs, i.e. the 16 bytes at
// j * row_bytes + 16 k from the tile's first row (aligned rows: the weight and the row size are
// multiples of 16; the padding chunk reads the next row's first bytes). The offsets are the same
// in every tile, so a lane computes them once.
constexpr int kBfMaxMine = 18;  // a copy wave's copies per tile (rows of up to 4.5 KB)

struct BfCopies {
  uint32_t off[kBfMaxMine];  // byte offset from the tile's first row
  int row[kBfMaxMine];       // row slot of the lane's chunk (>= 16: past the tile, not copied)
  int mine;
};

__device__ __forceinline__ BfCopies bf_offsets(long long row_bytes, int rs, int nqt, int cw,
                                               int lane) {
  BfCopies c;
  c.mine = (nqt - cw + kBfCopyWaves - 1) / kBfCopyWaves;
#pragma unroll
  for (int i = 0; i < kBfMaxMine; ++i) {
    const int e = 64 * (cw + kBfCopyWaves * i) + lane;
    const int j = e / rs, k = e - j * rs;
    c.off[i] = (uint32_t)(j * (int)row_bytes + 16 * k);
    c.row[i] = j;
  }
  return c;
}

template <int TYPE, int C>
__device__ __forceinline__ void bflow_rows(uint8_t* smem, const uint8_t* w, long long row_bytes,
                                           const Act& act, YOut y, long long ldy,
                                           int M, int N, const BfGeo& geo, int wg) {
  using Tile = typename TileOf<TYPE>::T;
  using F = typename Tile::F;
  constexpr int TB = kBfBlockBytes<TYPE>;
  constexpr int NC = kBfCopyWaves;

  const int tid = threadIdx.x, lane = tid & 63, ln = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ncw = geo.ncw, nb = act.nb, rs = geo.rs;
  const int tb = 16 * rs * 16;  // bytes of a tile's 16 row slots
  const int r0 = wg * geo.rows_per_wg;
  const int rows = max(0, min(geo.rows_per_wg, N - r0));
  const int T = (rows + 15) >> 4;
  float* Ad = (float*)(smem + geo.ctrl_off);  // activation scales [nb][16 m]
  int* cnt = (int*)(Ad + nb * 16);             // [4] tiles landed per copy wave, then computed[T]
  int* computed = cnt + NC;
  if (tid < NC + kBfMaxTiles) bf_store(cnt + tid, 0);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the counters are zero before the barrier
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");

  // row slot j of the workgroup's rows (tile j / 16, slot j % 16); where compute wave wv leaves
  // its block values of row slot j: over its own blocks' bytes (4-byte aligned; C * 17 floats fit
  // in one block of any type)
  auto row_off = [&](int j) { return j * rs * 16; };
  auto val_off = [&](int j, int wv) { return (row_off(j) + wv * C * TB + 3) & ~3; };

  if (wave >= ncw) {
    // ------------------------------------------------------------------ copy waves
    // Tile t's copies land at LDS tb * t + 1024 q. A copy wave keeps two tiles of copies in flight
    // and publishes tile t once its own copies of it have landed; rows past the workgroup's rows
    // are not copied (the lanes that would compute them use the last row, never stored).
    __builtin_amdgcn_s_setprio(3);
    const int cw = wave - ncw;
    const int nqt = (16 * rs + 63) >> 6;
    const BfCopies cp = bf_offsets(row_bytes, rs, nqt, cw, lane);
    const uint8_t* last = w + (size_t)N * row_bytes - 16;
    const uint32_t lds0 = lds_addr(smem);
    auto issue = [&](int t) {
      const uint8_t* base = w + (size_t)(r0 + 16 * t) * row_bytes;
      const int live = rows - 16 * t;  // row slots of the tile that hold a row
      // every row slot holds a row and the padding chunks' next row exists: no clamp, no masks
      const bool whole = live >= 16 && r0 + 16 * t + 17 <= N;
#pragma unroll
      for (int i = 0; i < kBfMaxMine; ++i) {
        if (i < cp.mine) {
          const uint32_t dst = lds0 + (uint32_t)(tb * t + 1024 * (cw + NC * i));
          if (whole) {
            if (cp.row[i] < 16) copy16_to_lds_s_nt(base, cp.off[i], dst);
          } else if (cp.row[i] < min(live, 16)) {
            copy16_to_lds_nt((const void*)min((uintptr_t)(base + cp.off[i]), (uintptr_t)last), dst);
          }
        }
      }
    };
    // copies issued per tile by this wave (a copy with no live lane is not issued)
    auto issued_in = [&](int t) {
      const int live = min(rows - 16 * t, 16);
      int n = 0;
#pragma unroll
      for (int i = 0; i < kBfMaxMine; ++i) n += (i < cp.mine && 64 * (cw + NC * i) < live * rs) ? 1 : 0;
      return n;
    };
    for (int t = 0; t < T; ++t) {
      issue(t);
      if (t >= 1) {  // tile t - 1 has landed once only tile t's copies are outstanding
        wait_vmcnt(issued_in(t));
        bf_store(cnt + cw, t);
      }
    }
    wait_vmcnt(0);
    bf_store(cnt + cw, T);  // also published by a wave with no copies
    // Folds: tile by tile as the compute waves finish them; lane l of copy wave cw takes output
    // o = 64 cw + l = (row slot o / 16, activation row o % 16) over blocks 0..nb-1 in order
    // (mx_dot_k_ssse3.c:115-154), 256 lanes for the 256 outputs of a tile.
    // The folds of all but the last tile overlap the compute waves' work and yield to it; the last
    // one is all that is left, at high priority.
    __builtin_amdgcn_s_setprio(0);
    const int o = 64 * cw + lane, nl = o >> 4, m = o & 15;
    float xd[16];  // the lane's activation scales, the same in every tile (nb <= 16)
    bool xd_loaded = false;
    for (int t = 0; t < T; ++t) {
      int spin = 0;
      while (bf_load(computed + t) < ncw && ++spin < kBfSpinLimit) __builtin_amdgcn_s_sleep(1);
      const bool gave_up = spin >= kBfSpinLimit;
      asm volatile("" ::: "memory");
      if (t == T - 1) __builtin_amdgcn_s_setprio(3);
      if (!xd_loaded) {  // written by the compute waves before they counted tile 0
#pragma unroll
        for (int b = 0; b < 16; ++b) xd[b] = b < nb ? Ad[b * 16 + m] : 0.0f;
        xd_loaded = true;
      }
      const int j = 16 * t + nl;
      if (j < rows && m < M) {
        float vv[16], dd[16];
#pragma unroll
        for (int b = 0; b < 16; ++b) {  // operands read ahead of the dependent chain
          if (b < nb) {
            const int wv = b / C, cc = b - wv * C;
            const float* src = (const float*)(smem + val_off(j, wv));
            vv[b] = src[cc * 16 + m];
            dd[b] = src[C * 16 + cc];
          }
        }
        float acc = 0.0f;
#pragma unroll
        for (int b = 0; b < 16; ++b)
          if (b < nb) acc = Tile::fold(acc, xd[b], vv[b], dd[b]);
        y.put((size_t)m * ldy + r0 + j, gave_up ? __builtin_nanf("") : acc);
      }
    }
    return;
  }

  // ---------------------------------------------------------------------- compute waves
  // A operands of the wave's blocks (activation rows >= M repeat row M - 1: computed, never
  // stored); the activation scales go to LDS for the folds.
  const int am = min(ln, M - 1);
  F f[C];
#pragma unroll
  for (int c = 0; c < C; ++c) f[c] = Tile::frag_g(act, am, min(wave * C + c, nb - 1), g);
  for (int i = tid; i < nb * 16; i += 64 * ncw) Ad[i] = act.d[(size_t)min(i & 15, M - 1) * nb + (i >> 4)];
  __builtin_amdgcn_s_waitcnt(0xC07F);

  for (int t = 0; t < T; ++t) {
    int spin = 0;
    for (; spin < kBfSpinLimit; ++spin) {  // the four copy waves' tiles in one read
      if (bf_frontier(cnt) > t) break;
      __builtin_amdgcn_s_sleep(2);
    }
    const bool gave_up = spin == kBfSpinLimit;
    asm volatile("" ::: "memory");
    const int j = 16 * t + min(ln, rows - 16 * t - 1);  // lanes past the rows compute its last row
    float v[C][4], dv[C];
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int b = wave * C + c;
      if (b < nb) {
        const typename Tile::P pp = Tile::prep(Tile::load_lds(smem, row_off(j) + b * TB, g), g);
        Tile::value(pp, f[c], g, [&](int e, float val, float dd) {
          v[c][e] = val;
          dv[c] = dd;
        });
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's reads of the tile are done
    if (16 * t + ln < rows) {
      float* dst = (float*)(smem + val_off(16 * t + ln, wave));
#pragma unroll
      for (int c = 0; c < C; ++c) {
        if (wave * C + c < nb) {
#pragma unroll
          for (int e = 0; e < 4; ++e) dst[c * 16 + 4 * g + e] = gave_up ? __builtin_nanf("") : v[c][e];
          if (g == 0) dst[C * 16 + c] = gave_up ? __builtin_nanf("") : dv[c];
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // the values are in LDS before they are counted
    if (lane == 0) bf_add(computed + t, 1);
  }
}

// The arguments in the order the waves first need them, the geometry packed into two dwords, so
// that what the first requests need arrives preloaded in SGPRs (structures never do):
// pack_a = rows_per_wg | ncw << 12 | M << 16 | nb << 21, pack_b = rs | ctrl_off << 12.
template <int TYPE, int C>
__global__ __launch_bounds__(1024) void bflow_kernel(const uint8_t* w, uint32_t pack_a,
                                                     uint32_t pack_b, int N, int row_bytes,
                                                     const int8_t* q, const int16_t* bsums,
                                                     const float* d, YOut y,
                                                     int ldy) {
  extern __shared__ __align__(16) uint8_t smem[];
  BfGeo geo;
  geo.rows_per_wg = pack_a & 0xFFF;
  geo.ncw = (pack_a >> 12) & 0xF;
  geo.rs = pack_b & 0xFFF;
  geo.ctrl_off = pack_b >> 12;
  const int M = (pack_a >> 16) & 0x1F, nb = pack_a >> 21;
  Act act;
  act.q = q, act.d = d, act.bsums = bsums, act.x = nullptr;
  act.k = nb * QK, act.nb = nb, act.xsplit = nullptr, act.xbf16 = 0;
  bflow_rows<TYPE, C>(smem, w, row_bytes, act, y, ldy, M, N, geo, blockIdx.x);
}

__host__ constexpr int bf_row_chunks(long long row_bytes) {
  return (int)(((row_bytes + 15) / 16 + 1) | 1);
}

template <int TYPE, int C>
int launch_bf(const uint8_t* w, long long row_bytes, const Act& act, YOut y, long long ldy, int M,
              int N, hipStream_t stream) {
  const int nb = act.nb;
  const int ncu = cu_count();
  const int R = (int)((N + (long long)ncu - 1) / ncu);
  const int T = (R + 15) / 16;
  BfGeo geo;
  geo.rows_per_wg = R;
  geo.rs = bf_row_chunks(row_bytes);
  geo.ncw = (nb + C - 1) / C;
  const int nqt = (16 * geo.rs + 63) / 64;  // copies per tile
  if (T > kBfMaxTiles || geo.ncw + kBfCopyWaves > 16 || (nqt + kBfCopyWaves - 1) / kBfCopyWaves > kBfMaxMine)
    return -1;
  // every row slot of every tile, then the activation scales and the counters
  geo.ctrl_off = T * 16 * geo.rs * 16;
  const int lds = geo.ctrl_off + nb * 16 * 4 + (kBfCopyWaves + kBfMaxTiles) * 4;
  if (lds > kBfLds) return -1;
  if (R > 0xFFF || geo.rs > 0xFFF || geo.ctrl_off > 0xFFFFF || nb > 0x7FF || row_bytes > 0x7FFFFFFF ||
      ldy > 0x7FFFFFFF)
    return -1;
  const uint32_t pack_a = (uint32_t)R | (uint32_t)geo.ncw << 12 | (uint32_t)M << 16 | (uint32_t)nb << 21;
  const uint32_t pack_b = (uint32_t)geo.rs | (uint32_t)geo.ctrl_off << 12;
  allow_lds((const void*)bflow_kernel<TYPE, C>, kBfLds);
  const int grid = (int)((N + (long long)R - 1) / R);
  hipLaunchKernelGGL((bflow_kernel<TYPE, C>), dim3(grid), dim3(64 * (geo.ncw + kBfCopyWaves)), lds,
                     stream, w, pack_a, pack_b, N, (int)row_bytes, act.q, act.bsums, act.d, y, (int)ldy);
  return 0;
}

}  // namespace

int launch_bflow(int type, const uint8_t* w, long long row_bytes, const Act& act, YOut y,
                 long long ldy, int m_rows, int n_rows, hipStream_t stream) {
  if (act.q == nullptr || m_rows < 1 || m_rows > 16 || n_rows < 1 || act.nb > 16) return -1;
  if ((((uintptr_t)w | (uintptr_t)row_bytes) & 15) != 0) return -1;
  switch (type) {
    case T_Q4_K: return launch_bf<T_Q4_K, 2>(w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
    case T_Q6_K: return launch_bf<T_Q6_K, 2>(w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
    case T_Q8_0: return launch_bf<T_Q8_0, 2>(w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
    default: return -1;
  }
}

}  // namespace mxa
