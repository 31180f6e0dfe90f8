// Batched decode (up to 16 activation rows, rows of up to 16 blocks) on the matrix cores, the weight
// rows streamed through LDS tile by tile in order.
//
// Work split. One workgroup per CU owns R consecutive weight rows (R = ceil(N / CUs), at least
// 16): T = ceil(R / 16) tiles of 16 rows, held in P tile slots of LDS (tile t in slot t % P; all
// of them when they fit). The compute waves split the blocks of a row: wave w owns blocks
// w * C .. w * C + C - 1, whose Q8_K activations (the MFMA A operands of all 16 activation rows)
// it loads once into registers. For each tile in order it waits until the tile has landed, builds
// the B operands from LDS with the tile builders of mxa_tiles.hpp and writes the block values over
// the bytes of its own blocks in the slot, which no other wave reads.
//
// Copies. Two groups of four copy waves take alternate tiles and request them in order with
// global_load_lds_dwordx4 (every fourth 1 KB copy of a tile per wave): a group requests its tile
// once the other group has requested the tile before (issued) and the slot's previous tile is
// folded, then waits for it to land (vmcnt) and counts ready[t]. Two tiles are in flight, so the
// tiles land one after another (a deeper burst makes all of them land late) and the compute waves
// start on tile 0 while later tiles still stream. For aligned rows a lane's copy offsets are the
// same in every tile and are computed once, so a copy is one instruction.
//
// Fold. Once every compute wave has counted computed[t], the tile's copy group folds a quarter of
// its outputs per wave: (weight row, activation row) over blocks 0..nb-1 in order with the oracle's
// fused steps (app/native/src/mx_dot_k_ssse3.c:115-154), so the results equal the other decode kernels
// and the oracle bit for bit; then it counts folded[t], which frees the slot. A group folds
// whatever is computed while it waits to request, so neither group waits on the other for long.
// Every counter only grows and every wait is for an earlier event of another wave, so the waits
// always end.
//
// Layout of a slot: 16 row slots of rs 16-byte chunks (rs odd, so the 16 rows a B-operand read
// touches fall in different banks); a row's bytes start at chunk 0 plus the row's address modulo
// 16.
#include "mxa_kernels.hpp"
#include "mxa_tiles.hpp"

#pragma clang fp contract(off)

namespace mxa {
namespace {

template <int TYPE>
constexpr int kBrBlockBytes = TYPE == T_Q4_K ? 144 : TYPE == T_Q6_K ? 210 : 272;
constexpr int kBrCopyWaves = 8;  // two groups of four
constexpr int kBrMaxTiles = 64;  // tiles per workgroup (R <= 1024)
constexpr int kBrMaxMine = 18;   // a copy wave's copies per tile (its only ones in flight)
constexpr int kBrLdsMax = 160 * 1024;
constexpr int kBrCtrlInts = 3 * kBrMaxTiles + 1;  // ready, computed, folded, issued

struct BrGeo {
  int rows_per_wg;  // R
  int rs;           // LDS chunks per row slot
  int tile_bytes;   // 16 row slots
  int copies;       // 1 KB copies per tile (16 * rs chunks)
  int slots;        // P
  int ncw;          // compute waves: ceil(nb / C)
  int ctrl_off;     // LDS offset of the activation scales, then the counters
};

__host__ __device__ constexpr int br_row_chunks(long long row_bytes) {
  return (int)(((row_bytes + 15 + 15) / 16) | 1);
}

__device__ __forceinline__ int br_load(const int* p) {
  return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void br_add(int* p, int v) {
  __hip_atomic_fetch_add(p, v, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
}

template <int TYPE, int C>
__device__ __forceinline__ void bres_rows(uint8_t* smem, const uint8_t* w, long long row_bytes,
                                          const Act& act, YOut y, long long ldy,
                                          int M, int N, const BrGeo& geo, int wg) {
  using Tile = typename TileOf<TYPE>::T;
  using F = typename Tile::F;
  constexpr int TB = kBrBlockBytes<TYPE>;

  const int tid = threadIdx.x, lane = tid & 63, ln = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ncw = geo.ncw, nb = act.nb, rs = geo.rs, tb = geo.tile_bytes, P = geo.slots;
  const int r0 = wg * geo.rows_per_wg;
  const int rows = min(geo.rows_per_wg, N - r0);  // >= 1: the grid is ceil(N / R)
  const int T = (rows + 15) >> 4;
  float* Ad = (float*)(smem + geo.ctrl_off);  // activation scales [nb][16 m]
  int* ready = (int*)(Ad + nb * 16);          // [T]: tile t has landed (4 counts)
  int* computed = ready + kBrMaxTiles;        // [T]: compute waves done with tile t
  int* folded = computed + kBrMaxTiles;       // [T]: tile t folded (4 counts): its slot is free
  int* issued = folded + kBrMaxTiles;         // copy waves done requesting their share of a tile
  for (int i = tid; i < kBrCtrlInts; i += blockDim.x) ready[i] = 0;
  __syncthreads();

  // Row slot j of tile t holds row min(16 t + j, rows - 1) of the workgroup (slots past the end
  // repeat its last row); the row's first byte sits at this LDS offset within the slot.
  auto row_ptr = [&](int t, int j) {
    return w + (size_t)(r0 + min(16 * t + j, rows - 1)) * row_bytes;
  };
  auto row_off = [&](int t, int j) { return j * rs * 16 + (int)((uintptr_t)row_ptr(t, j) & 15); };
  // Where compute wave wv leaves its block values of row slot j: over its own blocks' bytes
  // (4-byte aligned; C * 17 floats fit in one block of any type).
  auto val_off = [&](int t, int j, int wv) { return (row_off(t, j) + wv * C * TB + 3) & ~3; };
  auto slot = [&](int t) { return smem + (t % P) * tb; };

  if (wave >= ncw) {
    // ------------------------------------------------------------------ copy waves
    // Copy q of a tile moves chunks e = 64 q + lane: chunk k of row slot j, e = j rs + k. Copy
    // group grp (waves 4 grp .. 4 grp + 3) takes tiles grp, grp + 2, ...: wave cg of the group
    // issues q = cg, cg + 4, ... (mine copies per tile).
    const int c = wave - ncw, grp = c >> 2, cg = c & 3, nq = geo.copies;
    const int mine = (nq - cg + 3) / 4;
    const uint32_t base = lds_addr(smem);
    // a 16-byte aligned chunk holding a byte of the matrix never leaves that byte's page
    const uintptr_t last = ((uintptr_t)(w + (size_t)N * row_bytes) - 1) & ~(uintptr_t)15;
    // Aligned rows (the usual case): chunk e of a tile is byte j * row_bytes + 16 k from its first
    // row, the same offset in every tile, computed once per lane. Chunks past a row's bytes read
    // the next row's first bytes into the slot's padding, so such a tile needs a row after it.
    const bool aligned = (((uintptr_t)w | (uintptr_t)row_bytes) & 15) == 0;
    uint32_t voff[kBrMaxMine];
    bool lane_last = true;  // the lane's chunk of the wave's last copy lies in the 16 row slots
    {
      // j = e / rs from a float product: e < 2^13 and e + 1/2 is at least 1/(2 rs) from a
      // multiple of rs, far more than the product's rounding error
      const float inv_rs = 1.0f / (float)rs;
#pragma unroll
      for (int i = 0; i < kBrMaxMine; ++i) {
        const int e = 64 * (cg + 4 * i) + lane;
        const int j = (int)(((float)e + 0.5f) * inv_rs), k = e - j * rs;
        voff[i] = (uint32_t)(j * (int)row_bytes + 16 * k);
        if (i == mine - 1) lane_last = j < 16;
      }
    }
    auto issue = [&](int t) {
      const uint32_t dst = base + (uint32_t)((t % P) * tb);
      if (aligned && r0 + 16 * t + 17 <= N) {
        const uint8_t* tbase = w + (size_t)(r0 + 16 * t) * row_bytes;
#pragma unroll
        for (int i = 0; i < kBrMaxMine; ++i) {
          if (i < mine - 1 || (i == mine - 1 && lane_last))
            copy16_to_lds_s(tbase, voff[i], dst + 1024 * (cg + 4 * i));
        }
        return;
      }
      for (int q = cg; q < nq; q += 4) {  // every such copy has live lanes
        const int e = 64 * q + lane, j = e / rs, k = e - j * rs;
        const uintptr_t ra = (uintptr_t)row_ptr(t, min(j, 15));
        const int crow = (int)(((ra & 15) + row_bytes + 15) >> 4);
        if (j < 16 && k < crow) {
          const uintptr_t a = (ra & ~(uintptr_t)15) + 16 * k;
          copy16_to_lds((const void*)(a < last ? a : last), dst + 1024 * q);
        }
      }
    };
    // Folds quarter cg of tile t: output o = 64 cg + lane is (row slot o / 16, activation row
    // o % 16); then counts folded[t].
    const int o = 64 * cg + lane, nl = o >> 4, m = o & 15;
    auto fold = [&](int t) {
      if (16 * t + nl < rows && m < M) {
        const uint8_t* tile = slot(t);
        const int ro = row_off(t, nl);
        float acc = 0.0f;
        int b = 0;
        for (; b + 8 <= nb; b += 8) {  // operands read ahead of the dependent chain
          float xv[8], vv[8], dd[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const int bb = b + i, wv = bb / C, cc = bb - wv * C;
            const float* src = (const float*)(tile + ((ro + wv * C * TB + 3) & ~3));
            xv[i] = Ad[bb * 16 + m];
            vv[i] = src[cc * 16 + m];
            dd[i] = src[C * 16 + cc];
          }
#pragma unroll
          for (int i = 0; i < 8; ++i) acc = Tile::fold(acc, xv[i], vv[i], dd[i]);
        }
        for (; b < nb; ++b) {
          const int wv = b / C, cc = b - wv * C;
          const float* src = (const float*)(tile + ((ro + wv * C * TB + 3) & ~3));
          acc = Tile::fold(acc, Ad[b * 16 + m], src[cc * 16 + m], src[C * 16 + cc]);
        }
        y.put((size_t)m * ldy + r0 + 16 * t + nl, acc);
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the slot reads are done
      if (lane == 0) br_add(&folded[t], 1);
    };
    int nf = grp;  // the group's next tile to fold
    auto fold_ready = [&]() {
      bool any = false;
      while (nf < T && br_load(&computed[nf]) >= ncw) {
        fold(nf);
        nf += 2;
        any = true;
      }
      return any;
    };
    for (int t = grp; t < T; t += 2) {
      // tiles before t requested, and the slot's previous tile folded (by either group)
      while (br_load(issued) < 4 * t || (t >= P && br_load(&folded[t - P]) < 4))
        if (!fold_ready()) __builtin_amdgcn_s_sleep(1);
      issue(t);
      if (lane == 0) br_add(issued, 1);
      wait_vmcnt(0);  // the wave's only copies in flight: its share of tile t
      if (lane == 0) br_add(&ready[t], 1);
      fold_ready();
    }
    while (nf < T) {
      while (br_load(&computed[nf]) < ncw) __builtin_amdgcn_s_sleep(1);
      fold(nf);
      nf += 2;
    }
    return;
  }

  // ---------------------------------------------------------------------- compute waves
  // A operands of the wave's blocks (activation rows >= M repeat row M - 1: computed, never
  // stored); the activation scales go to LDS for the fold (each wave's stores complete before its
  // first count).
  const int am = min(ln, M - 1);
  F f[C];
#pragma unroll
  for (int c = 0; c < C; ++c) f[c] = Tile::frag_g(act, am, min(wave * C + c, nb - 1), g);
  for (int i = tid; i < nb * 16; i += 64 * ncw) Ad[i] = act.d[(size_t)min(i & 15, M - 1) * nb + (i >> 4)];
  for (int t = 0; t < T; ++t) {
    while (br_load(&ready[t]) < 4) __builtin_amdgcn_s_sleep(1);  // a copy group's four waves
    uint8_t* tile = slot(t);
    const int j = min(ln, rows - 16 * t - 1);  // lanes past the tile's rows compute its last row
    const int roff = row_off(t, j);
    float v[C][4], dv[C];
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int b = wave * C + c;
      if (b < nb) {
        const typename Tile::P pp = Tile::prep(Tile::load_lds(tile, roff + b * TB, g), g);
        Tile::value(pp, f[c], g, [&](int e, float val, float dd) {
          v[c][e] = val;
          dv[c] = dd;
        });
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's reads of the tile are done
    float* dst = (float*)(tile + val_off(t, ln, wave));
#pragma unroll
    for (int c = 0; c < C; ++c) {
      if (wave * C + c < nb) {
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[c * 16 + 4 * g + e] = v[c][e];
        if (g == 0) dst[C * 16 + c] = dv[c];
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // the values are in LDS before they are counted
    if (lane == 0) br_add(&computed[t], 1);
  }
}

template <int TYPE, int C>
__global__ __launch_bounds__(1024) void bres_kernel(const uint8_t* w, long long row_bytes, Act act,
                                                    YOut y, long long ldy, int M,
                                                    int N, BrGeo geo) {
  extern __shared__ __align__(16) uint8_t smem[];
  bres_rows<TYPE, C>(smem, w, row_bytes, act, y, ldy, M, N, geo, blockIdx.x);
}

// Several weights sharing the activations in one launch: workgroups wg0 .. of segment s take its
// rows with its own geometry.
constexpr int kBrMaxSegs = 4;
struct BrSeg {
  const uint8_t* w;
  long long row_bytes;
  YOut y;  // the segment's first output column
  int n, type, wg0;
  BrGeo geo;
};
struct BrSegs {
  BrSeg s[kBrMaxSegs];
  int count;
};

template <int C>
__global__ __launch_bounds__(1024) void bres_multi_kernel(BrSegs segs, Act act, long long ldy, int M) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int wg = blockIdx.x;
  int i = 0;
  while (i + 1 < segs.count && wg >= segs.s[i + 1].wg0) ++i;
  const BrSeg& sg = segs.s[i];
  switch (sg.type) {
    case T_Q4_K: bres_rows<T_Q4_K, C>(smem, sg.w, sg.row_bytes, act, sg.y, ldy, M, sg.n, sg.geo, wg - sg.wg0); break;
    case T_Q6_K: bres_rows<T_Q6_K, C>(smem, sg.w, sg.row_bytes, act, sg.y, ldy, M, sg.n, sg.geo, wg - sg.wg0); break;
    default: bres_rows<T_Q8_0, C>(smem, sg.w, sg.row_bytes, act, sg.y, ldy, M, sg.n, sg.geo, wg - sg.wg0); break;
  }
}

// Geometry of one weight (row_bytes, nb blocks per row, R rows per workgroup) in an LDS of
// lds_max bytes; false when it does not fit. *lds: the bytes it uses.
inline bool br_geometry(BrGeo& geo, long long row_bytes, int nb, int C, int R, int lds_max, int* lds) {
  geo.rows_per_wg = R;
  geo.rs = br_row_chunks(row_bytes);
  geo.tile_bytes = 16 * geo.rs * 16;
  geo.copies = (16 * geo.rs + 63) / 64;
  geo.ncw = (nb + C - 1) / C;
  const int T = (R + 15) / 16;
  if (T > kBrMaxTiles || geo.ncw + kBrCopyWaves > 16) return false;
  // a copy wave's share of one tile: its offsets stay in registers
  if ((geo.copies + 3) / 4 > kBrMaxMine) return false;
  const int ctrl = nb * 16 * 4 + kBrCtrlInts * 4;
  geo.slots = min(T, (lds_max - ctrl) / geo.tile_bytes);
  if (geo.slots < min(T, 2)) return false;  // a slot per copy group
  geo.ctrl_off = geo.slots * geo.tile_bytes;
  *lds = geo.ctrl_off + ctrl;
  return true;
}

template <int TYPE, int C>
int launch_br(const uint8_t* w, long long row_bytes, const Act& act, YOut y, long long ldy, int M,
              int N, hipStream_t stream) {
  const int ncu = cu_count();
  const int R = max(16, (int)((N + (long long)ncu - 1) / ncu));
  BrGeo geo;
  int lds = 0;
  if (!br_geometry(geo, row_bytes, act.nb, C, R, kBrLdsMax, &lds)) return -1;
  allow_lds((const void*)bres_kernel<TYPE, C>, kBrLdsMax);
  const int grid = (int)((N + (long long)R - 1) / R);
  hipLaunchKernelGGL((bres_kernel<TYPE, C>), dim3(grid), dim3(64 * (geo.ncw + kBrCopyWaves)), lds,
                     stream, w, row_bytes, act, y, ldy, M, N, geo);
  return 0;
}

template <int TYPE>
int launch_br_type(const uint8_t* w, long long row_bytes, const Act& act, YOut y, long long ldy,
                   int M, int N, hipStream_t stream) {
  if (act.nb <= 8) return launch_br<TYPE, 1>(w, row_bytes, act, y, ldy, M, N, stream);
  return launch_br<TYPE, 2>(w, row_bytes, act, y, ldy, M, N, stream);
}

template <int C>
int launch_br_multi(const DecodeSeg* seg, int count, const Act& act, long long ldy, int M,
                    hipStream_t stream) {
  if (count < 1 || count > kBrMaxSegs) return -1;
  const int ncu = cu_count();
  double total = 0.0;
  for (int i = 0; i < count; ++i) {
    if (seg[i].type != T_Q4_K && seg[i].type != T_Q6_K && seg[i].type != T_Q8_0) return -1;
    total += (double)seg[i].n * (double)seg[i].row_bytes;
  }
  BrSegs segs;
  segs.count = count;
  int wg0 = 0, lds = 0;
  for (int i = 0; i < count; ++i) {  // workgroups in proportion to the bytes of each weight
    const int share = max(1, (int)((double)ncu * seg[i].n * seg[i].row_bytes / total + 0.5));
    const int R = max(16, (seg[i].n + share - 1) / share);
    int l = 0;
    segs.s[i] = BrSeg{seg[i].w, seg[i].row_bytes, seg[i].y, seg[i].n, seg[i].type, wg0, BrGeo{}};
    if (!br_geometry(segs.s[i].geo, seg[i].row_bytes, act.nb, C, R, kBrLdsMax, &l)) return -1;
    lds = max(lds, l);
    wg0 += (seg[i].n + R - 1) / R;
  }
  allow_lds((const void*)bres_multi_kernel<C>, kBrLdsMax);
  const int ncw = (act.nb + C - 1) / C;
  hipLaunchKernelGGL((bres_multi_kernel<C>), dim3(wg0), dim3(64 * (ncw + kBrCopyWaves)), lds, stream,
                     segs, act, ldy, M);
  return 0;
}

}  // namespace

int launch_bres(int type, const uint8_t* w, long long row_bytes, const Act& act, YOut y,
                long long ldy, int m_rows, int n_rows, hipStream_t stream) {
  if (act.q == nullptr || m_rows < 1 || m_rows > 16 || n_rows < 1 || act.nb > 16) return -1;
  switch (type) {
    case T_Q4_K: return launch_br_type<T_Q4_K>(w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
    case T_Q6_K: return launch_br_type<T_Q6_K>(w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
    case T_Q8_0: return launch_br_type<T_Q8_0>(w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
    default: return -1;
  }
}

int launch_bres_multi(const DecodeSeg* seg, int count, const Act& act, long long ldy, int m_rows,
                      hipStream_t stream) {
  if (act.q == nullptr || m_rows < 1 || m_rows > 16 || act.nb > 16) return -1;
  if (act.nb <= 8) return launch_br_multi<1>(seg, count, act, ldy, m_rows, stream);
  return launch_br_multi<2>(seg, count, act, ldy, m_rows, stream);
}

}  // namespace mxa
