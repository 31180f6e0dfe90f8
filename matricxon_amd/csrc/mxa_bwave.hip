// Batched decode (up to 16 activation rows, rows of up to 16 blocks) on the matrix cores, with every
// wave streaming and computing its own units: no copy waves, no wave ever waits for another.
//
// Work split. One workgroup per CU owns R consecutive weight rows (R = ceil(N / CUs)), T =
// ceil(R / 16) tiles of 16 rows. Its waves split the blocks of a row: wave w owns blocks w C ..
// w C + C - 1 of every row and keeps their Q8_K activations (the MFMA A operands of all 16
// activation rows), staged through LDS with whole-row copies, in registers. Its unit of a tile is
// those C blocks of the tile's 16 rows: 16 pieces of C * block bytes, one per row, which the wave
// gathers itself with 1 KB global_load_lds_dwordx4 copies (lane -> one 16-byte chunk of one row's
// piece; a row's piece is one contiguous run of the row) into its own LDS slot for that tile.
//
// Stream. A wave keeps D tiles of its copies in flight: it requests tiles 0 .. D - 1, and tile
// t + D as soon as tile t has landed (its own vmcnt: copies complete in issue order). The CU's
// queue thus holds D tiles of every wave, and a wave starts on a tile the moment its own pieces
// of it have landed, not the whole tile.
//
// Compute. For each tile, the wave builds the B operands of its blocks from its slot with the
// tile builders of mxa_tiles.hpp (the arithmetic of the other batched kernels) and keeps the
// block values. Every output (weight row, activation row) is then folded over blocks 0..nb-1 in
// order with the oracle's fused steps (app/native/src/mx_dot_k_ssse3.c:115-154, 200-206;
// mx_dot_q8_0.c:8-18), so results equal the other decode kernels and the oracle bit for bit.
//
// Two forms. Resident (up to 8 tiles whose slots all fit LDS): nothing is reused, so no wave ever
// waits for another; block values go over the slot's own bytes, and after its last tile every
// wave meets the others at one barrier and the workgroup folds all outputs. No output is stored
// before that barrier: a store counts on the same vmcnt as the copies, and a wave with a store
// pending would wait for later tiles' copies at its next copy wait. (Folding each tile after a
// barrier of its own, its outputs parked in LDS: 12.4 vs 12.1 us at Q4_K 14336 x 4096, M = 16.)
// Ring (more tiles, e.g. a vocabulary head): D + 1 slots per wave cycle, and each tile's values
// go to a two-entry value ring folded after a per-tile barrier (below). Long rows (more than 16
// blocks, `bwlong_kernel`): the unit is a tile x a part of eight blocks with its own staged
// activations, the fold carried across a tile's parts (below).
#include "mxa_kernels.hpp"
#include "mxa_tiles.hpp"

#pragma clang fp contract(off)

namespace mxa {
namespace {

template <int TYPE>
constexpr int kBwBlockBytes = TYPE == T_Q4_K ? 144 : TYPE == T_Q6_K ? 210 : 272;
constexpr int kBwMaxTiles = 8;
constexpr int kBwMaxCopies = 8;  // 1 KB copies of one wave's unit of a tile
constexpr int kBwLds = 160 * 1024;

typedef __attribute__((address_space(3))) int lds_int;
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));

// A wave's activation operands travel through LDS: C blocks of 16 activation rows, each row's 256
// q8 bytes as 16 pieces of 16 bytes (piece p of row r at slot (p + r) mod 16: the 16 rows of one
// MFMA operand read fall in different banks), then (Q4_K, Q6_K) the rows' 32 bytes of bsums. They
// are gathered with 1 KB copies of whole 256-byte row runs (16 cache lines a copy; the MFMA-shaped
// register loads touch 64 lines an instruction and read each line four times) into the wave's
// slots of its last two tiles, requested only later, or into an area of their own.
template <int TYPE>
__host__ __device__ constexpr int a_stage_bytes(int C) {
  return C * 16 * QK + (TYPE != T_Q8_0 ? C * 16 * 32 : 0);
}

// The staging copies of blocks b0 .. b0 + C - 1 (clamped to the row's blocks): copy 4 c + i moves
// rows 4 i .. 4 i + 3 of block c; copy 4 C the bsums of both blocks (lane -> block, row, half).
template <int TYPE, int C>
__device__ __forceinline__ int a_stage(const Act& act, int M, int b0, int lane, uint32_t dst) {
  const int nb = act.nb;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int b = min(b0 + c, nb - 1);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * i + (lane >> 4), s = lane & 15, p = (s - r) & 15;
      const int8_t* src = act.q + (size_t)min(r, M - 1) * act.k + (size_t)b * QK + 16 * p;
      copy16_to_lds(src, dst + (uint32_t)(c * 16 * QK + 1024 * i));
    }
  }
  if constexpr (TYPE == T_Q8_0) {
    return 4 * C;
  } else {
    if (lane < 32 * C) {
      const int c = lane >> 5, r = (lane & 31) >> 1, h = lane & 1;
      const int b = min(b0 + c, nb - 1);
      copy16_to_lds((const uint8_t*)(act.bsums + ((size_t)min(r, M - 1) * nb + b) * 16) + 16 * h,
                    dst + (uint32_t)(C * 16 * QK));
    }
    return 4 * C + 1;
  }
}

// The tile builders of these kernels: Q6_K on the 32-deep MFMA (TileQ6s: half the B masking
// and MFMA cycles of TileQ6, whose 64-deep form the prefill kernels keep), the others as shared.
template <int TYPE>
struct BwTileOf {
  using T = typename TileOf<TYPE>::T;
};
template <>
struct BwTileOf<T_Q6_K> {
  using T = TileQ6s;
};

// The MFMA A operands of block c from the staging area (lane: activation row ln, k-group g).
template <int TYPE>
__device__ __forceinline__ typename BwTileOf<TYPE>::T::F a_read(const uint8_t* ast, int C, int c,
                                                                int ln, int g) {
  typename BwTileOf<TYPE>::T::F f;
  const uint8_t* row = ast + c * 16 * QK + ln * QK;
  if constexpr (TYPE == T_Q6_K) {  // chunk cc: bytes 32 cc + 8 g .. + 7 (piece 2 cc + g / 2)
#pragma unroll
    for (int cc = 0; cc < 8; ++cc) {
      const int p = 2 * cc + (g >> 1);
      const long v = *(const long*)(row + 16 * ((p + ln) & 15) + 8 * (g & 1));
      f.a[0][cc] = (g >> 1) == 0 ? v : 0;  // the copy for sub-block 2 cc (lane groups 0, 1)
      f.a[1][cc] = (g >> 1) == 1 ? v : 0;  // and for sub-block 2 cc + 1 (lane groups 2, 3)
    }
  } else {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int p = 4 * g + t;
      f.a[t] = __builtin_bit_cast(i32x4, *(const u32x4*)(row + 16 * ((p + ln) & 15)));
    }
  }
  if constexpr (TYPE != T_Q8_0) {
    const uint2 v = *(const uint2*)(ast + C * 16 * QK + c * 512 + 32 * ln + 8 * g);
    f.bs = f16x4{(_Float16)(float)(int16_t)(v.x & 0xFFFFu), (_Float16)(float)(int16_t)(v.x >> 16),
                 (_Float16)(float)(int16_t)(v.y & 0xFFFFu), (_Float16)(float)(int16_t)(v.y >> 16)};
  }
  return f;
}

struct BwGeo {
  int R;     // rows per workgroup
  int rs;    // 16-byte chunks per row piece in a slot (odd)
  int D;     // tiles of copies in flight per wave
  int ncw;   // waves: ceil(nb / C)
};

// Values of one tile in the RING form: [block][row][m] floats, then the blocks' d [block][row].
constexpr int kBwValBytes = (16 * 256 + 16 * 16) * 4;

// pack = R | rs << 12 | D << 20 | ncw << 24 | staging in the last two tiles' slots << 29;
// packm = M | nb << 8.
// RING: more tiles than stay resident. A wave keeps S = D + 1 slots and requests tile t + D into
// the slot of tile t - 1, which it has finished reading itself (no other wave reads a slot). The
// block values go to a two-entry value ring, the waves meet at a barrier after every tile and the
// first 256 threads fold that tile's outputs and store them; the barrier of tile t + 1 also keeps
// any wave from writing tile t + 2's values before tile t's fold has read the entry. The operands'
// staging area is the region from the slots of index D through the value ring (first used after
// a barrier that follows every wave's reads of its operands).
// The body of one workgroup: rows wg * R .. of the weight at w (bwave_kernel, and one weight of
// a shared-input group in bwave_multi_kernel).
template <int TYPE, int C, bool RING>
__device__ __forceinline__ void bwave_rows(uint8_t* smem, const uint8_t* __restrict__ w,
                                           uint32_t pack, uint32_t packm, int N, int row_bytes,
                                           const int8_t* q, const int16_t* bsums, const float* d,
                                           YOut y, int ldy, int wg) {
  using Tile = typename BwTileOf<TYPE>::T;
  using F = typename Tile::F;
  constexpr int TB = kBwBlockBytes<TYPE>;

  const int R = pack & 0xFFF, rs = (pack >> 12) & 0xFF, D = (pack >> 20) & 0xF;
  const int ncw = (pack >> 24) & 0x1F;
  const bool stage_in_slots = ((pack >> 29) & 1) != 0;
  const int M = packm & 0x1F, nb = (packm >> 8) & 0xFF;
  Act act;
  act.q = q, act.d = d, act.bsums = bsums, act.x = nullptr;
  act.k = nb * QK, act.nb = nb, act.xsplit = nullptr, act.xbf16 = 0;

  const int tid = threadIdx.x, lane = tid & 63, ln = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r0 = wg * R;
  const int rows = min(R, N - r0);  // >= 1: the grid is ceil(N / R)
  const int T = (rows + 15) >> 4;   // tiles this workgroup computes
  const int TG = (R + 15) >> 4;     // tiles of the layout the host sized (the last workgroup
                                    // may have fewer rows; its slots keep the same places)
  const int slot_bytes = 16 * rs * 16;
  constexpr int kStage = a_stage_bytes<TYPE>(C);
  const int S = D + 1;  // RING: slots per wave
  // resident: tile t of wave wv; RING: slot t mod S of every wave, slot index major
  auto slot = [&](int wv, int t) {
    return RING ? smem + ((t % S) * ncw + wv) * slot_bytes : smem + (wv * TG + t) * slot_bytes;
  };
  uint8_t* vring = smem + S * ncw * slot_bytes;  // RING: two entries of kBwValBytes
  // the wave's staging area: resident, its slots of tiles TG - 2, TG - 1 (the host puts it there
  // only when TG - 2 >= D, so those tiles, if this workgroup has them, are requested after the
  // operands are read) or an area of its own after all slots; RING, from slot index D on
  uint8_t* ast = RING ? smem + D * ncw * slot_bytes + wave * kStage
               : stage_in_slots ? slot(wave, TG - 2) : smem + ncw * TG * slot_bytes + wave * kStage;

  // this wave's blocks, and its piece of a row: chunks [c_lo, c_hi) of the row (16-byte aligned
  // chunks covering bytes b0 TB .. (b0 + cb) TB; rows are 16-byte multiples, so they stay inside)
  const int b0 = wave * C, cb = min(C, nb - b0);
  const int c_lo = (b0 * TB) >> 4, c_hi = ((b0 + cb) * TB + 15) >> 4;
  const int nch = c_hi - c_lo;
  const int skew = b0 * TB - 16 * c_lo;  // byte of block b0 in the row piece
  const int ncp = (16 * rs + 63) >> 6;   // copies per unit

  // 1. the A operands into the staging area, and the activation scales of the lane's fold row
  //    m = lane % 16 into registers (four 16-byte loads, nb % 4 == 0), issued before any weight
  //    copy so that they land first. The scale loads are inline assembly, so the compiler's wait
  //    insertion never waits for them (it would wait for every copy issued after them); no
  //    branch or copy of their registers comes before the wave's own wait. The compiler takes
  //    these registers as written at issue: a spill or reuse of them before the wait would read
  //    or clobber registers the loads still write (a variant that spilled here faulted), so the
  //    build refuses any kernel of this file that uses scratch memory.
  const int am = min(ln, M - 1);
  const int n_stage = a_stage<TYPE, C>(act, M, b0, lane, lds_addr(ast));
  f32x4 xq[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float* p = d + (size_t)am * nb + min(4 * i, nb - 4);
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(xq[i]) : "v"(p) : "memory");
  }
  (void)n_stage;

  // 2. the copies: lane chunk e = 64 i + lane of the unit is chunk e % rs of row e / rs
  uint32_t off[kBwMaxCopies];
  int crow[kBwMaxCopies];
#pragma unroll
  for (int i = 0; i < kBwMaxCopies; ++i) {
    const int e = 64 * i + lane, j = e / rs, c = e - j * rs;
    crow[i] = c < nch ? j : 16;  // 16: not copied (padding chunk or past the unit)
    off[i] = (uint32_t)(j * row_bytes + 16 * (c_lo + c));
  }
  // copies issued for tile t (an instruction none of whose lanes copies is not issued)
  auto issued = [&](int t) {
    const int live = min(16, rows - 16 * t);
    return min(ncp, ((live - 1) * rs + nch + 63) >> 6);
  };
  auto issue = [&](int t) {
    const uint8_t* base = w + (size_t)(r0 + 16 * t) * row_bytes;
    const int live = min(16, rows - 16 * t);
    const uint32_t dst = lds_addr(slot(wave, t));
#pragma unroll
    for (int i = 0; i < kBwMaxCopies; ++i)
      if (i < ncp && crow[i] < live) copy16_to_lds_s_nt(base, off[i], dst + 1024u * (uint32_t)i);
  };

  int in_flight = 0;  // copies issued after the A loads
  for (int t = 0; t < min(D, T); ++t) {
    issue(t);
    in_flight += issued(t);
  }
  wait_vmcnt(min(in_flight, kMaxCopies));  // the A operands and scales have landed
#pragma unroll
  for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(xq[i]));
  float xd[16];
#pragma unroll
  for (int b = 0; b < 16; ++b) xd[b] = xq[b >> 2][b & 3];
  F f[C];
#pragma unroll
  for (int c = 0; c < C; ++c) f[c] = a_read<TYPE>(ast, C, c, ln, g);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the staging area is read before tiles land in it
  // RING: a wave's staging area spans other waves' slots of index D and the value ring, so every
  // wave has read its operands before any wave requests tile D or writes values
  if constexpr (RING) {
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  }

  // RING: the outputs a fold thread computed for the previous tile (two when the workgroup has
  // fewer than 256 threads), stored only after the next tile's wait and request, so that their
  // stores are not pending at that wait (with D = 1 the wait is for every outstanding operation)
  float pend[2] = {0.0f, 0.0f};
  size_t pend_at[2] = {0, 0};
  bool pend_ok[2] = {false, false};
  for (int t = 0; t < T; ++t) {
    // tile t has landed once only the later tiles' copies are outstanding (a store of an earlier
    // fold issued since can only make this wait longer, never shorter: loads complete in order)
    int later = 0;
    for (int u = t + 1; u < min(t + D, T); ++u) later += issued(u);
    wait_vmcnt(later);
    if (t + D < T) issue(t + D);
    if constexpr (RING) {
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        if (pend_ok[k]) y.put(pend_at[k], pend[k]);
        pend_ok[k] = false;
      }
    }
    const int live = min(16, rows - 16 * t);
    uint8_t* sl = slot(wave, t);
    const int jr = min(ln, live - 1);  // lanes past the rows compute the last row, never folded
    float v[C][4], dv[C];
#pragma unroll
    for (int c = 0; c < C; ++c) {
      if (c < cb) {
        const typename Tile::P pp =
            Tile::prep(Tile::load_lds(sl, jr * rs * 16 + skew + c * TB, g), g);
        Tile::value_wide(pp, f[c], g, [&](int e, float val, float dd) {
          v[c][e] = val;
          dv[c] = dd;
        });
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the slot's bytes are read
    if constexpr (RING) {
      // block values into the value ring: [block][row][m], then d [block][row]
      float* vals = (float*)(vring + (t & 1) * kBwValBytes);
#pragma unroll
      for (int c = 0; c < C; ++c) {
        if (c < cb) {
#pragma unroll
          for (int e = 0; e < 4; ++e) vals[((b0 + c) * 16 + ln) * 16 + 4 * g + e] = v[c][e];
          if (g == 0) vals[16 * 256 + (b0 + c) * 16 + ln] = dv[c];
        }
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      // fold tile t: output o = (row j, activation row m = o % 16, the thread's own), by the
      // first 256 threads, or by all of them, two outputs each, in a workgroup of two waves (rows
      // of four blocks). Blocks past nb hold stale values and are never folded.
      const int nf = min(64 * ncw, 256);
      if (tid < nf) {
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const int o = tid + k * nf, j = o >> 4, m = o & 15;
          if (o < 256 && j < live && m < M) {
            float vv[16], dd[16];
#pragma unroll
            for (int b = 0; b < 16; ++b) {  // operands read ahead of the dependent chain
              vv[b] = vals[(b * 16 + j) * 16 + m];
              dd[b] = vals[16 * 256 + b * 16 + j];
            }
            float acc = 0.0f;
            if (nb == 16) {
#pragma unroll
              for (int b = 0; b < 16; ++b) acc = Tile::fold(acc, xd[b], vv[b], dd[b]);
            } else {
#pragma unroll
              for (int b = 0; b < 16; ++b)
                if (b < nb) acc = Tile::fold(acc, xd[b], vv[b], dd[b]);
            }
            pend[k] = acc;
            pend_at[k] = (size_t)m * ldy + r0 + 16 * t + j;
            pend_ok[k] = true;
          }
        }
      }
    } else {
      // block values over the slot: [c][row][m], then (Q6_K) the blocks' d [c][row]
      float* vals = (float*)sl;
#pragma unroll
      for (int c = 0; c < C; ++c) {
        if (c < cb) {
#pragma unroll
          for (int e = 0; e < 4; ++e) vals[(c * 16 + ln) * 16 + 4 * g + e] = v[c][e];
          if (g == 0) vals[C * 256 + c * 16 + ln] = dv[c];
        }
      }
    }
  }
  if constexpr (RING) {
#pragma unroll
    for (int k = 0; k < 2; ++k)
      if (pend_ok[k]) y.put(pend_at[k], pend[k]);
    return;
  }
  // 3. every wave has written its block values of every tile: the workgroup folds all outputs
  //    (tile t, weight row j, activation row m), m the thread's own row (its scales in registers)
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  // The 16 reads of an output are unconditional and their slot offsets scalar (a runtime branch
  // and a vector multiply per read made this loop ~1.3 us of a 12 us kernel); blocks past nb read
  // the last wave's slot and are never folded.
  // A thread folds two outputs (o, o + step) at a time, their chains interleaved, and the chains
  // of full 16-block rows carry no per-block select. Output o is (tile t, weight row j,
  // activation row m = o % 16 = the lane's own row, whose scales xd holds).
  const int wstride = TG * slot_bytes / 4;  // floats between one wave's slots and the next's
  const int nout = T * 256, step = 64 * ncw;
  auto read_vals = [&](int o, float* vv, float* dd) {
    const int t = o >> 8, j = (o >> 4) & 15, m = o & 15;
    const float* tb = (const float*)slot(0, t);
#pragma unroll
    for (int b = 0; b < 16; ++b) {  // operands read ahead of the dependent chain
      const int wv = min(b / C, ncw - 1), cc = b % C;
      const float* src = tb + wv * wstride;
      vv[b] = src[(cc * 16 + j) * 16 + m];
      dd[b] = src[C * 256 + cc * 16 + j];
    }
  };
  auto store = [&](int o, float acc) {
    const int t = o >> 8, j = (o >> 4) & 15, m = o & 15;
    if (o < nout && j < rows - 16 * t && m < M) y.put((size_t)m * ldy + r0 + 16 * t + j, acc);
  };
  for (int o = tid; o < nout; o += 2 * step) {
    const int o2 = o + step;
    float v0[16], d0[16], v1[16], d1[16];
    read_vals(o, v0, d0);
    read_vals(o2 < nout ? o2 : o, v1, d1);  // past the end: o's operands again, never stored
    float a0 = 0.0f, a1 = 0.0f;
    if (nb == 16) {
#pragma unroll
      for (int b = 0; b < 16; ++b) {
        a0 = Tile::fold(a0, xd[b], v0[b], d0[b]);
        a1 = Tile::fold(a1, xd[b], v1[b], d1[b]);
      }
    } else {
#pragma unroll
      for (int b = 0; b < 16; ++b) {
        if (b < nb) {
          a0 = Tile::fold(a0, xd[b], v0[b], d0[b]);
          a1 = Tile::fold(a1, xd[b], v1[b], d1[b]);
        }
      }
    }
    store(o, a0);
    store(o2, a1);
  }
}

template <int TYPE, int C, bool RING>
__global__ __launch_bounds__(C == 1 ? 1024 : 512) void bwave_kernel(const uint8_t* __restrict__ w, uint32_t pack,
                                                        uint32_t packm, int N, int row_bytes,
                                                        const int8_t* q, const int16_t* bsums,
                                                        const float* d, YOut y, int ldy) {
  extern __shared__ __align__(16) uint8_t smem[];
  bwave_rows<TYPE, C, RING>(smem, w, pack, packm, N, row_bytes, q, bsums, d, y, ldy, (int)blockIdx.x);
}

// Shared-input weights (q|k|v): up to four K-quant weights of the same input in one launch, each
// in the resident form with workgroups in proportion to its bytes (its own rows per workgroup,
// slot shape and depth in its pack word); a workgroup runs the body of its weight's type.
constexpr int kBwMaxSegs = 4;
struct BwSeg {
  const uint8_t* w;
  YOut y;  // the weight's first output column (row stride ldy)
  uint32_t pack;
  int n, row_bytes, type, wg0;
};
struct BwSegs {
  BwSeg s[kBwMaxSegs];
  int count;
};

__global__ __launch_bounds__(512) void bwave_multi_kernel(BwSegs segs, uint32_t packm,
                                                          const int8_t* q, const int16_t* bsums,
                                                          const float* d, int ldy) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int wg = blockIdx.x;
  int i = 0;
  while (i + 1 < segs.count && wg >= segs.s[i + 1].wg0) ++i;
  const BwSeg& sg = segs.s[i];
  if (sg.type == T_Q6_K)
    bwave_rows<T_Q6_K, 2, false>(smem, sg.w, sg.pack, packm, sg.n, sg.row_bytes, q, bsums, d, sg.y,
                                 ldy, wg - sg.wg0);
  else
    bwave_rows<T_Q4_K, 2, false>(smem, sg.w, sg.pack, packm, sg.n, sg.row_bytes, q, bsums, d, sg.y,
                                 ldy, wg - sg.wg0);
}

template <int C>
constexpr int ncw_of(int nb) {
  return (nb + C - 1) / C;  // waves per workgroup: C blocks of each row per wave
}

// The resident geometry of R rows per workgroup of nb-block rows: the pack word and its LDS bytes;
// false when the rows need the ring form or do not fit.
template <int TYPE, int C>
bool bw_resident(int nb, int R, int depth, uint32_t* pack, int* lds) {
  constexpr int TB = kBwBlockBytes<TYPE>;
  constexpr int kStage = a_stage_bytes<TYPE>(C);
  const int T = (R + 15) / 16;
  const int ncw = (nb + C - 1) / C;
  int nch = 0;
  for (int wv = 0; wv < ncw; ++wv) {
    const int b0 = wv * C, cb = min(C, nb - b0);
    nch = max(nch, ((b0 + cb) * TB + 15) / 16 - (b0 * TB) / 16);
  }
  const int rs = nch | 1;
  const int ncp = (16 * rs + 63) / 64;
  const int slot_bytes = 16 * rs * 16;
  if (ncp > kBwMaxCopies || ncw > 16 || nb % 4 != 0 || (C * 256 + C * 16) * 4 > slot_bytes ||
      R > 0xFFF || rs > 0xFF || T > kBwMaxTiles)
    return false;
  const int D = max(1, min(depth, min(T, 15)));
  const bool in_slots = T - 2 >= D && 2 * slot_bytes >= kStage;
  const int l = ncw * T * slot_bytes + (in_slots ? 0 : ncw * kStage);
  if (l > kBwLds) return false;
  *pack = (uint32_t)R | (uint32_t)rs << 12 | (uint32_t)D << 20 | (uint32_t)ncw << 24 |
          (uint32_t)in_slots << 29;
  *lds = l;
  return true;
}

// The launch geometry of R rows per workgroup of nb-block rows at `depth` tiles in flight: the
// pack word, the LDS bytes and whether the rows take the ring form; false when they fit neither.
template <int TYPE, int C>
bool bw_plan(int nb, int R, int depth, uint32_t* pack, int* lds, bool* ring) {
  constexpr int TB = kBwBlockBytes<TYPE>;
  constexpr int kStage = a_stage_bytes<TYPE>(C);
  const int T = (R + 15) / 16;
  const int ncw = (nb + C - 1) / C;
  // the widest row piece of any wave, in 16-byte chunks, made odd (bank spread of the 16 rows)
  int nch = 0;
  for (int wv = 0; wv < ncw; ++wv) {
    const int b0 = wv * C, cb = min(C, nb - b0);
    nch = max(nch, ((b0 + cb) * TB + 15) / 16 - (b0 * TB) / 16);
  }
  const int rs = nch | 1;
  const int ncp = (16 * rs + 63) / 64;
  const int slot_bytes = 16 * rs * 16;
  // values [C][16][16] and d [C][16] fit a slot; the scales of a row in four 16-byte loads
  if (R < 1 || ncp > kBwMaxCopies || ncw > 16 || nb % 4 != 0 ||
      (C * 256 + C * 16) * 4 > slot_bytes || R > 0xFFF || rs > 0xFF)
    return false;
  // Resident: every tile's slot stays in LDS, the operands' staging area in the last two tiles'
  // slots when those are requested only after the operands are read (T - 2 >= D), else an area
  // of its own.
  int D = max(1, min(depth, min(T, 15)));
  const bool in_slots = T - 2 >= D && 2 * slot_bytes >= kStage;
  const int lds_res = ncw * T * slot_bytes + (in_slots ? 0 : ncw * kStage);
  *ring = T > kBwMaxTiles || lds_res > kBwLds;
  *lds = lds_res;
  if (*ring) {
    // S = D + 1 slots per wave and the value ring; the staging area from slot index D on
    for (D = min(depth, 15); D >= 1; --D) {
      *lds = (D + 1) * ncw * slot_bytes + 2 * kBwValBytes;
      if (*lds <= kBwLds && ncw * kStage <= ncw * slot_bytes + 2 * kBwValBytes) break;
    }
    if (D < 1) return false;
  }
  *pack = (uint32_t)R | (uint32_t)rs << 12 | (uint32_t)D << 20 | (uint32_t)ncw << 24 |
          (uint32_t)(!*ring && in_slots) << 29;
  return true;
}

template <int TYPE, int C>
int launch_bw(const uint8_t* w, long long row_bytes, const Act& act, YOut y, long long ldy, int M,
              int N, int depth, hipStream_t stream) {
  const int nb = act.nb;
  const int ncu = cu_count();
  const int R = (int)((N + (long long)ncu - 1) / ncu);
  uint32_t pack;
  int lds;
  bool ring;
  if (ldy > 0x7FFFFFFF || row_bytes > 0x7FFFFFFF || !bw_plan<TYPE, C>(nb, R, depth, &pack, &lds, &ring))
    return -1;
  const uint32_t packm = (uint32_t)M | (uint32_t)nb << 8;
  auto kern = ring ? bwave_kernel<TYPE, C, true> : bwave_kernel<TYPE, C, false>;
  allow_lds((const void*)kern, kBwLds);
  const int grid = (int)((N + (long long)R - 1) / R);
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * ncw_of<C>(nb)), lds, stream, w, pack, packm, N,
                     (int)row_bytes, act.q, act.bsums, act.d, y, (int)ldy);
  return 0;
}

// Grouped MoE experts: rows [offsets[e], offsets[e + 1]) of the activations (clamped into
// [0, total_rows)) go through expert e, whose weight starts at w + e * expert_stride. The rows are
// cut into 16-row chunks, and workgroup wg = blockIdx.x % wpe of item blockIdx.x / wpe of the
// (expert, chunk) list runs the batched-decode body on its R rows of that expert's weight for the
// chunk; a workgroup past the list's end exits. (One chunk per workgroup, so an expert that a
// token names twice, with more rows than tokens, is still covered: a loop over chunks spilled.)
template <int TYPE, int C, bool RING>
__global__ __launch_bounds__(C == 1 ? 1024 : 512) void moe_bwave_kernel(
    const uint8_t* __restrict__ w, long long expert_stride, uint32_t pack, int nb, int N,
    int row_bytes, const int8_t* q, const int16_t* bsums, const float* d,
    const int32_t* __restrict__ offsets, int n_experts, int total_rows, YOut y, int ldy, int wpe) {
  extern __shared__ __align__(16) uint8_t smem[];
  int e, p0, m;
  if (!moe_chunk_item(offsets, n_experts, total_rows, 16, (int)blockIdx.x / wpe, e, p0, m)) return;
  bwave_rows<TYPE, C, RING>(smem, w + (size_t)e * expert_stride, pack,
                            (uint32_t)m | (uint32_t)nb << 8, N, row_bytes,
                            q + (size_t)p0 * nb * QK, bsums + (size_t)p0 * nb * 16,
                            d + (size_t)p0 * nb, y.at((long long)p0 * ldy), ldy,
                            (int)blockIdx.x % wpe);
}

template <int TYPE, int C>
int launch_moe_bw(const uint8_t* w, long long row_bytes, long long expert_stride, int n_experts,
                  const Act& act, const int32_t* offsets, int total_rows, YOut y, long long ldy,
                  int N, int depth, hipStream_t stream) {
  const int nb = act.nb;
  // at most min(n_experts, total_rows) experts have rows: their workgroups fill the CUs
  const long long busy = min(n_experts, total_rows);
  const int R = (int)((N * busy + cu_count() - 1) / cu_count());
  uint32_t pack;
  int lds;
  bool ring;
  if (ldy > 0x7FFFFFFF || row_bytes > 0x7FFFFFFF || !bw_plan<TYPE, C>(nb, R, depth, &pack, &lds, &ring))
    return -1;
  // the list has at most n_experts + ceil(total_rows / 16) items (each expert's last chunk may
  // be partial)
  const int wpe = (N + R - 1) / R;
  const long long items = n_experts + (total_rows + 15LL) / 16;
  if (wpe * items > 0x7FFFFFFF) return -1;
  auto kern = ring ? moe_bwave_kernel<TYPE, C, true> : moe_bwave_kernel<TYPE, C, false>;
  allow_lds((const void*)kern, kBwLds);
  hipLaunchKernelGGL(kern, dim3((unsigned)(wpe * items)), dim3(64 * ncw_of<C>(nb)), lds, stream,
                     w, expert_stride, pack, nb, N, (int)row_bytes, act.q, act.bsums, act.d,
                     offsets, n_experts, total_rows, y, (int)ldy, wpe);
  return 0;
}

// Long rows (more than 16 blocks, e.g. the FFN down projection's 56): the rows are cut into parts
// of PB = ncw * C blocks and the stream's unit is (tile t, part p), tile-major. The A operands of
// a part differ from the next part's, and at 16 activation rows a CU's share of them outgrows its
// share of the weight (56 blocks: 229 KB of Q8_K against 188 KB of Q6_K), so every unit stages its
// own: a wave's slot holds the part's A operands (the whole-row-run copies above), the 16 rows'
// activation scales of its blocks (one 16-byte copy per row), and its weight pieces. A wave reads
// its landed unit into registers and only then requests unit u + D into the same slot, so D slots
// per wave keep D units in flight while one is computed. The waves put block values, block d and
// activation
// scales of a unit into a two-entry value ring; after a per-unit barrier the first 256 threads
// fold that unit's blocks into their output's running sum, which carries from part to part of a
// tile (blocks in order), and store it after the tile's last part, so the results equal the
// oracle and the other decode kernels bit for bit. Every part starts on a 16-byte boundary of the
// row (PB * block bytes a multiple of 16), so a wave's per-lane copy offsets serve every unit.
template <int TYPE, int C>
__device__ __forceinline__ void bwlong_rows(uint8_t* smem, const uint8_t* __restrict__ w,
                                            uint32_t pack, uint32_t packm, int N, int row_bytes,
                                            const int8_t* q, const int16_t* bsums, const float* d,
                                            YOut y, int ldy, int wg) {
  using Tile = typename BwTileOf<TYPE>::T;
  using F = typename Tile::F;
  constexpr int TB = kBwBlockBytes<TYPE>;
  constexpr int kStageA = a_stage_bytes<TYPE>(C);
  constexpr int kStage = kStageA + 256;  // then the scales: row r's 16 bytes at 16 r
  constexpr int kNA = 4 * C + (TYPE != T_Q8_0 ? 1 : 0) + 1;  // staging copies of a unit

  const int R = pack & 0xFFF, rs = (pack >> 12) & 0xFF, D = (pack >> 20) & 0xF;
  const int ncw = (pack >> 24) & 0x1F;
  const int M = packm & 0x1F, nb = (packm >> 8) & 0xFF;
  Act act;
  act.q = q, act.d = d, act.bsums = bsums, act.x = nullptr;
  act.k = nb * QK, act.nb = nb, act.xsplit = nullptr, act.xbf16 = 0;

  const int tid = threadIdx.x, lane = tid & 63, ln = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r0 = wg * R;
  const int rows = min(R, N - r0);  // >= 1: the grid is ceil(N / R)
  const int T = (rows + 15) >> 4;
  const int PB = ncw * C, P = (nb + PB - 1) / PB, U = T * P;
  const int slot_bytes = kStage + 16 * rs * 16;
  auto slot = [&](int u) { return smem + ((u % D) * ncw + wave) * slot_bytes; };
  // value ring entry: values [PB][row][m], block d [PB][row], activation scales [PB][m]
  const int val_bytes = PB * (256 + 16 + 16) * 4;
  uint8_t* vring = smem + D * ncw * slot_bytes;

  // this wave's blocks of a part: bw .. bw + C - 1 (relative); its row piece: chunks c_lo0 ..
  const int bw = wave * C;
  const int c_lo0 = (bw * TB) >> 4;
  const int skew = bw * TB - 16 * c_lo0;
  const int ncp = (16 * rs + 63) >> 6;
  auto cb_of = [&](int p) { return min(C, nb - (p * PB + bw)); };  // <= 0: no block in part p
  auto nch_of = [&](int p) {
    const int cb = cb_of(p);
    return cb <= 0 ? 0 : ((bw + cb) * TB + 15) / 16 - c_lo0;
  };

  // the copies: lane chunk e = 64 i + lane of the unit is chunk e % rs of row e / rs
  uint32_t off[kBwMaxCopies];
  int crow[kBwMaxCopies], cch[kBwMaxCopies];
#pragma unroll
  for (int i = 0; i < kBwMaxCopies; ++i) {
    const int e = 64 * i + lane, j = e / rs, c = e - j * rs;
    crow[i] = j;
    cch[i] = c;
    off[i] = (uint32_t)(j * row_bytes + 16 * (c_lo0 + c));
  }
  auto issued = [&](int u) {
    const int t = u / P, p = u - t * P;
    const int live = min(16, rows - 16 * t), nch = nch_of(p);
    return nch == 0 ? 0 : kNA + min(ncp, ((live - 1) * rs + nch + 63) >> 6);
  };
  auto issue = [&](int u) {
    const int t = u / P, p = u - t * P;
    const int nch = nch_of(p);
    if (nch == 0) return;
    const int live = min(16, rows - 16 * t), b0 = p * PB + bw;
    const uint32_t dst = lds_addr(slot(u));
    a_stage<TYPE, C>(act, M, b0, lane, dst);
    if (lane < 16)  // row lane's scales of blocks (b0 & ~3) .. + 3 (nb % 4 == 0: in the row)
      copy16_to_lds(d + (size_t)min(lane, M - 1) * nb + (b0 & ~3), dst + kStageA);
    const uint8_t* base = w + (size_t)(r0 + 16 * t) * row_bytes + (size_t)p * PB * TB;
#pragma unroll
    for (int i = 0; i < kBwMaxCopies; ++i)
      if (i < ncp && crow[i] < live && cch[i] < nch)
        copy16_to_lds_s_nt(base, off[i], dst + kStage + 1024u * (uint32_t)i);
  };

  for (int u = 0; u < min(D, U); ++u) issue(u);

  float acc = 0.0f, pend = 0.0f;
  size_t pend_at = 0;
  bool pend_ok = false;
  for (int u = 0; u < U; ++u) {
    // unit u has landed once only the later units' copies are outstanding
    int later = 0;
    for (int v = u + 1; v < min(u + D, U); ++v) later += issued(v);
    wait_vmcnt(later);
    const int t = u / P, p = u - t * P;
    const int live = min(16, rows - 16 * t), cb = cb_of(p), b0 = p * PB + bw;
    // the unit's operands, scales and weight bytes into registers; then its slot takes unit u + D
    F f[C];
    float xs[C];
    typename Tile::W wl[C];
    if (cb > 0) {
      const uint8_t* sl = slot(u);
      const int jr = min(ln, live - 1);  // lanes past the rows compute the last row, never folded
#pragma unroll
      for (int c = 0; c < C; ++c) {
        if (c < cb) {
          f[c] = a_read<TYPE>(sl, C, c, ln, g);
          xs[c] = *(const float*)(sl + kStageA + 16 * ln + 4 * ((b0 + c) & 3));
          wl[c] = Tile::load_lds(sl + kStage, jr * rs * 16 + skew + c * TB, g);
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the slot is read
    // unit u + D into the slot just read: with one unit in flight the CU's copy queue is empty
    // now, so the request goes ahead of this unit's compute; with more, only after it (the CU
    // takes ~64 KB of copies in flight, and a request made while unit u + 1 is still landing
    // stalls the wave at the copy instruction until that unit drains)
    if (D == 1 && u + 1 < U) issue(u + 1);
    if (pend_ok) y.put(pend_at, pend);  // the previous tile's output, stored after the wait
    pend_ok = false;
    float* vals = (float*)(vring + (u & 1) * val_bytes);
    if (cb > 0) {
#pragma unroll
      for (int c = 0; c < C; ++c) {
        if (c < cb) {
          float v[4], dv = 0.0f;
          const typename Tile::P pp = Tile::prep(wl[c], g);
          Tile::value_wide(pp, f[c], g, [&](int e, float val, float dd) {
            v[e] = val;
            dv = dd;
          });
#pragma unroll
          for (int e = 0; e < 4; ++e) vals[((bw + c) * 16 + ln) * 16 + 4 * g + e] = v[e];
          if (g == 0) {
            vals[PB * 256 + (bw + c) * 16 + ln] = dv;
            vals[PB * 272 + (bw + c) * 16 + ln] = xs[c];  // scale of activation row m = ln
          }
        }
      }
    }
    if (D > 1 && u + D < U) issue(u + D);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): values written
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (tid < 256) {  // fold unit u into output (row j, activation row m = the thread's own)
      const int j = tid >> 4, m = tid & 15;
      const int nbp = min(PB, nb - p * PB);
      if (p == 0) acc = 0.0f;
      float vv[16], dd[16], xd[16];
#pragma unroll
      for (int b = 0; b < 16; ++b) {  // operands read ahead of the dependent chain
        if (b < nbp) {
          vv[b] = vals[(b * 16 + j) * 16 + m];
          dd[b] = vals[PB * 256 + b * 16 + j];
          xd[b] = vals[PB * 272 + b * 16 + m];
        }
      }
#pragma unroll
      for (int b = 0; b < 16; ++b)
        if (b < nbp) acc = Tile::fold(acc, xd[b], vv[b], dd[b]);
      if (p == P - 1 && j < live && m < M) {
        pend = acc;
        pend_at = (size_t)m * ldy + r0 + 16 * t + j;
        pend_ok = true;
      }
    }
  }
  if (pend_ok) y.put(pend_at, pend);
}

template <int TYPE, int C>
__global__ __launch_bounds__(512) void bwlong_kernel(const uint8_t* __restrict__ w, uint32_t pack,
                                                     uint32_t packm, int N, int row_bytes,
                                                     const int8_t* q, const int16_t* bsums,
                                                     const float* d, YOut y, int ldy) {
  extern __shared__ __align__(16) uint8_t smem[];
  bwlong_rows<TYPE, C>(smem, w, pack, packm, N, row_bytes, q, bsums, d, y, ldy, (int)blockIdx.x);
}

// The long-row body for grouped MoE experts, as moe_bwave_kernel runs the short-row one: item
// blockIdx.x / wpe of the (expert, 16-row chunk) list, its rows of workgroup blockIdx.x % wpe.
template <int TYPE, int C>
__global__ __launch_bounds__(512) void moe_bwlong_kernel(
    const uint8_t* __restrict__ w, long long expert_stride, uint32_t pack, int nb, int N,
    int row_bytes, const int8_t* q, const int16_t* bsums, const float* d,
    const int32_t* __restrict__ offsets, int n_experts, int total_rows, YOut y, int ldy, int wpe) {
  extern __shared__ __align__(16) uint8_t smem[];
  int e, p0, m;
  if (!moe_chunk_item(offsets, n_experts, total_rows, 16, (int)blockIdx.x / wpe, e, p0, m)) return;
  bwlong_rows<TYPE, C>(smem, w + (size_t)e * expert_stride, pack, (uint32_t)m | (uint32_t)nb << 8,
                       N, row_bytes, q + (size_t)p0 * nb * QK, bsums + (size_t)p0 * nb * 16,
                       d + (size_t)p0 * nb, y.at((long long)p0 * ldy), ldy, (int)blockIdx.x % wpe);
}

// The long-row geometry of R rows per workgroup, ncw waves of C blocks per part, at `depth`
// units in flight: the pack word and the LDS bytes; false when it does not fit.
template <int TYPE, int C>
bool bwl_plan(int nb, int R, int ncw, int depth, uint32_t* pack, int* lds) {
  constexpr int TB = kBwBlockBytes<TYPE>;
  constexpr int kStage = a_stage_bytes<TYPE>(C) + 256;
  const int PB = ncw * C;
  int nch = 0;  // the widest row piece of a wave within a part, in 16-byte chunks, made odd
  for (int wv = 0; wv < ncw; ++wv) nch = max(nch, ((wv + 1) * C * TB + 15) / 16 - (wv * C * TB) / 16);
  const int rs = nch | 1;
  const int ncp = (16 * rs + 63) / 64;
  const int slot_bytes = kStage + 16 * rs * 16;
  const int val_bytes = PB * (256 + 16 + 16) * 4;
  if (R < 1 || nb <= 16 || nb > 255 || nb % 4 != 0 || (PB * TB) % 16 != 0 || PB > 16 ||
      ncp > kBwMaxCopies || R > 0xFFF || rs > 0xFF)
    return false;
  int D = min(depth, 15);
  for (; D >= 1; --D) {
    *lds = D * ncw * slot_bytes + 2 * val_bytes;
    if (*lds <= kBwLds) break;
  }
  if (D < 1) return false;
  *pack = (uint32_t)R | (uint32_t)rs << 12 | (uint32_t)D << 20 | (uint32_t)ncw << 24;
  return true;
}

template <int TYPE, int C>
int launch_moe_bwl(const uint8_t* w, long long row_bytes, long long expert_stride, int n_experts,
                   const Act& act, const int32_t* offsets, int total_rows, YOut y, long long ldy,
                   int N, int ncw, int depth, hipStream_t stream) {
  const int nb = act.nb;
  // at most min(n_experts, total_rows) experts have rows: their workgroups fill the CUs
  const long long busy = min(n_experts, total_rows);
  const int R = (int)((N * busy + cu_count() - 1) / cu_count());
  uint32_t pack;
  int lds;
  if (ldy > 0x7FFFFFFF || row_bytes > 0x7FFFFFFF || !bwl_plan<TYPE, C>(nb, R, ncw, depth, &pack, &lds))
    return -1;
  const int wpe = (N + R - 1) / R;
  const long long items = n_experts + (total_rows + 15LL) / 16;
  if (wpe * items > 0x7FFFFFFF) return -1;
  auto kern = moe_bwlong_kernel<TYPE, C>;
  allow_lds((const void*)kern, kBwLds);
  hipLaunchKernelGGL(kern, dim3((unsigned)(wpe * items)), dim3(64 * ncw), lds, stream, w,
                     expert_stride, pack, nb, N, (int)row_bytes, act.q, act.bsums, act.d, offsets,
                     n_experts, total_rows, y, (int)ldy, wpe);
  return 0;
}

template <int TYPE, int C>
int launch_bwl(const uint8_t* w, long long row_bytes, const Act& act, YOut y, long long ldy, int M,
               int N, int ncw, int depth, hipStream_t stream) {
  const int nb = act.nb;
  const int ncu = cu_count();
  const int R = (int)((N + (long long)ncu - 1) / ncu);
  uint32_t pack;
  int lds;
  if (ldy > 0x7FFFFFFF || row_bytes > 0x7FFFFFFF || !bwl_plan<TYPE, C>(nb, R, ncw, depth, &pack, &lds))
    return -1;
  const uint32_t packm = (uint32_t)M | (uint32_t)nb << 8;
  auto kern = bwlong_kernel<TYPE, C>;
  allow_lds((const void*)kern, kBwLds);
  const int grid = (int)((N + (long long)R - 1) / R);
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * ncw), lds, stream, w, pack, packm, N,
                     (int)row_bytes, act.q, act.bsums, act.d, y, (int)ldy);
  return 0;
}

}  // namespace

int launch_bwave_multi(const DecodeSeg* seg, int count, const Act& act, long long ldy, int m_rows,
                       hipStream_t stream) {
  if (act.q == nullptr || m_rows < 1 || m_rows > 16 || count < 2 || count > kBwMaxSegs ||
      act.nb > 16 || ldy > 0x7FFFFFFF)
    return -1;
  const int ncu = cu_count();
  double total = 0.0;
  for (int i = 0; i < count; ++i) {
    if ((seg[i].type != T_Q4_K && seg[i].type != T_Q6_K) || seg[i].n < 1 ||
        (((uintptr_t)seg[i].w | (uintptr_t)seg[i].row_bytes) & 15) != 0 || seg[i].row_bytes > 0x7FFFFFFF)
      return -1;
    total += (double)seg[i].n * (double)seg[i].row_bytes;
  }
  BwSegs segs;
  segs.count = count;
  int wg0 = 0, lds = 0;
  constexpr int kDepth = 2;
  // Workgroups in proportion to the bytes of each weight; a weight whose share of tiles does not
  // fit LDS gets fewer tiles per workgroup (Q6_K 1024 x 4096 at 18 rows: two tiles and a separate
  // staging area, 184 KB). A workgroup takes most of a CU's LDS, so the group must fit one round
  // of the CUs: the shares shrink until it does, and a group that cannot (gate|up: seven tiles
  // per CU) is left to the other kernels.
  double budget = ncu;
  for (int attempt = 0; attempt < 6; ++attempt) {
    wg0 = 0, lds = 0;
    for (int i = 0; i < count; ++i) {
      const int share = max(1, (int)(budget * seg[i].n * seg[i].row_bytes / total));
      int R = (seg[i].n + share - 1) / share;
      uint32_t pack = 0;
      int l = 0;
      for (;;) {
        const bool ok = seg[i].type == T_Q6_K ? bw_resident<T_Q6_K, 2>(act.nb, R, kDepth, &pack, &l)
                                              : bw_resident<T_Q4_K, 2>(act.nb, R, kDepth, &pack, &l);
        if (ok) break;
        if (R <= 16) return -1;
        R = 16 * ((R - 1) / 16);
      }
      segs.s[i] = BwSeg{seg[i].w, seg[i].y, pack, seg[i].n, (int)seg[i].row_bytes, seg[i].type, wg0};
      lds = max(lds, l);
      wg0 += (seg[i].n + R - 1) / R;
    }
    if (wg0 <= ncu) break;
    budget *= (double)ncu / wg0;
  }
  if (wg0 > ncu) return -1;
  const uint32_t packm = (uint32_t)m_rows | (uint32_t)act.nb << 8;
  allow_lds((const void*)bwave_multi_kernel, kBwLds);
  const int ncw = (act.nb + 1) / 2;
  hipLaunchKernelGGL(bwave_multi_kernel, dim3(wg0), dim3(64 * ncw), lds, stream, segs, packm, act.q,
                     act.bsums, act.d, (int)ldy);
  return 0;
}

int launch_bwave(int type, const uint8_t* w, long long row_bytes, const Act& act, YOut y,
                 long long ldy, int m_rows, int n_rows, hipStream_t stream) {
  if (act.q == nullptr || m_rows < 1 || m_rows > 16 || n_rows < 1) return -1;
  if ((((uintptr_t)w | (uintptr_t)row_bytes) & 15) != 0) return -1;
  if (act.nb > 16) {
    // long rows: parts of eight blocks, one per wave; one unit in flight (two measured slower,
    // Q6_K 4096 x 14336 M = 16 25.4 vs 23.4 us: each unit's compute, ~1.6-2.4 us per block and
    // wave at two waves per SIMD, is the limit, and the deeper queue stalls its issue)
    constexpr int kLongDepth = 1;
    switch (type) {
      case T_Q4_K: return launch_bwl<T_Q4_K, 1>(w, row_bytes, act, y, ldy, m_rows, n_rows, 8, kLongDepth, stream);
      case T_Q6_K: return launch_bwl<T_Q6_K, 1>(w, row_bytes, act, y, ldy, m_rows, n_rows, 8, kLongDepth, stream);
      case T_Q8_0: return launch_bwl<T_Q8_0, 1>(w, row_bytes, act, y, ldy, m_rows, n_rows, 8, kLongDepth, stream);
      default: return -1;
    }
  }
  // Two tiles of copies in flight (three measured no faster where the slots allow it); two
  // blocks per wave, one for Q8_0 (its 272-byte groups: 16 waves, 7.1 vs 8.4 us at 4096 x 4096,
  // M = 16; Q4_K 4096 x 4096 6.1 vs 5.7 us with one)
  constexpr int kDepth = 2;
  switch (type) {
    case T_Q4_K: return launch_bw<T_Q4_K, 2>(w, row_bytes, act, y, ldy, m_rows, n_rows, kDepth, stream);
    case T_Q6_K: return launch_bw<T_Q6_K, 2>(w, row_bytes, act, y, ldy, m_rows, n_rows, kDepth, stream);
    case T_Q8_0: return launch_bw<T_Q8_0, 1>(w, row_bytes, act, y, ldy, m_rows, n_rows, kDepth, stream);
    default: return -1;
  }
}

int launch_moe_bwave(int type, const uint8_t* w, long long row_bytes, long long expert_stride,
                     int n_experts, const Act& act, const int32_t* offsets, int total_rows,
                     YOut y, long long ldy, int n_rows, hipStream_t stream) {
  if (act.q == nullptr || n_experts < 1 || n_experts > 256 || total_rows < 1 || n_rows < 1)
    return -1;
  if ((((uintptr_t)w | (uintptr_t)row_bytes | (uintptr_t)expert_stride) & 15) != 0) return -1;
  // the parts, depths and blocks per wave of the single-matrix launches above
  if (act.nb > 16) {
    constexpr int kLongDepth = 1;
    switch (type) {
      case T_Q4_K: return launch_moe_bwl<T_Q4_K, 1>(w, row_bytes, expert_stride, n_experts, act, offsets, total_rows, y, ldy, n_rows, 8, kLongDepth, stream);
      case T_Q6_K: return launch_moe_bwl<T_Q6_K, 1>(w, row_bytes, expert_stride, n_experts, act, offsets, total_rows, y, ldy, n_rows, 8, kLongDepth, stream);
      case T_Q8_0: return launch_moe_bwl<T_Q8_0, 1>(w, row_bytes, expert_stride, n_experts, act, offsets, total_rows, y, ldy, n_rows, 8, kLongDepth, stream);
      default: return -1;
    }
  }
  constexpr int kDepth = 2;
  switch (type) {
    case T_Q4_K: return launch_moe_bw<T_Q4_K, 2>(w, row_bytes, expert_stride, n_experts, act, offsets, total_rows, y, ldy, n_rows, kDepth, stream);
    case T_Q6_K: return launch_moe_bw<T_Q6_K, 2>(w, row_bytes, expert_stride, n_experts, act, offsets, total_rows, y, ldy, n_rows, kDepth, stream);
    case T_Q8_0: return launch_moe_bw<T_Q8_0, 1>(w, row_bytes, expert_stride, n_experts, act, offsets, total_rows, y, ldy, n_rows, kDepth, stream);
    default: return -1;
  }
}

}  // namespace mxa
