// Batched decode (up to 16 activation rows) on the matrix cores, weights streamed through LDS.
//
// Work split. One persistent workgroup per CU owns R consecutive weight rows (R = N / CUs, at
// least 16), cut into 16-row tiles (the last may be partial). A stage is a tile's rows over kb
// blocks: whole rows up to 16 blocks, else parts of 8 blocks taken in order (np parts per tile).
// The compute waves split a stage's blocks: wave w owns blocks b0 = w * C .. b0 + C - 1 of the
// part, so the Q8_K activations of those blocks (the MFMA A operands of all 16 activation rows)
// stay in the wave's registers (with several parts, the next part's are loaded meanwhile).
//
// Memory. A stage (one contiguous byte range for whole rows, else 16 row pieces) moves into one of
// nbuf LDS stage buffers with global_load_lds_dwordx4 (1 KB of consecutive bytes per instruction)
// issued by four copy waves, each issuing every fourth copy of every stage, stages in order.
// Issuing a copy stalls while the memory system is saturated, so copying and computing are
// separate waves, and they hand stages over through LDS counters rather than workgroup barriers
// (a barrier would make the compute waves wait for a copy wave stuck behind its issue queue):
//   ready[b]  counts copy waves whose share of the stage in buffer b has landed (vmcnt);
//   done[b]   counts compute waves finished with buffer b (a copy wave reuses it at the next
//             multiple of the compute-wave count);
//   vals[v]   counts compute waves whose block values of a stage are in value buffer v; once it
//             is complete each copy wave folds its quarter of the stage's outputs;
//   folded[v] counts those quarters (a compute wave may overwrite value buffer v once every
//             quarter of the stage that used it last is folded); nfold counts all quarters.
// Copy waves fold whenever they would otherwise wait, so compute waves never wait for one
// another. Every counter only grows and every wait is for an earlier stage, so the waits always
// end. In LDS each row piece starts on a 16-byte chunk boundary and the piece stride is an odd
// number of chunks, so the 16 rows a B-operand read touches fall in different banks. B operands
// are built from the LDS copy with the tile builders of mxa_tiles.hpp (lane = weight row).
//
// Fold. One copy-wave lane per (weight row, activation row) folds the block values in order
// 0..nb-1, part after part, with the oracle's fused steps (app/native/src/mx_dot_k_ssse3.c:115-154), so
// results equal the decode kernels and the oracle bit for bit. Outputs wait in an LDS ring of
// tiles that the compute waves write out, coalesced.
#include "mxa_kernels.hpp"
#include "mxa_tiles.hpp"

#pragma clang fp contract(off)

namespace mxa {
namespace {

template <int TYPE>
constexpr int kBlockBytes = TYPE == T_Q4_K ? 144 : TYPE == T_Q6_K ? 210 : 272;

// LDS chunks (16 bytes) per row piece: enough for the piece at any start offset, rounded up to
// odd.
__host__ __device__ constexpr int row_chunks(long long piece_bytes) {
  return (int)(((piece_bytes + 15 + 15) / 16) | 1);
}

struct BsGeo {
  int rows_per_wg;  // R
  int kb;           // blocks per stage piece (a stage is 16 rows x kb blocks); np = ceil(nb / kb)
  int rs;           // LDS chunks per row piece
  int nbuf;         // stage buffers
  int buf_bytes;    // bytes of one stage buffer (whole 1 KB copies)
  int ntp;          // block-value buffers
  int ncw;          // compute waves (ceil(kb / C)); the kCopyWaves waves after them copy
};

constexpr int kCopyWaves = 4;
constexpr int kFirstStages = 2;  // stages requested before the first one lands (at most nbuf)
constexpr int kOutTiles = 8;     // tiles of outputs staged in LDS before they are written out
constexpr int kMaxBuf = 4;
constexpr int kPartBlocks = 8;   // blocks per stage piece when a row has more than 16
// Copies of one stage a copy wave issues at most: 16 rows of up to 16 blocks, 1 KB each.
template <int TYPE>
constexpr int kStageCopies = (16 * 16 * (16 * kBlockBytes<TYPE> / 16 + 2) + 1023) / 1024;
constexpr int kCtrlInts = 16;  // ready[4] done[4] vals[2] folded[2] nfold

__device__ __forceinline__ int lds_load(const int* p) {
  return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ int lds_add(int* p, int v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// Waits until *p >= target (workgroup-scope acquire: later LDS reads see what the counting waves
// wrote before they counted).
__device__ __forceinline__ void wait_at_least(const int* p, int target) {
  while (lds_load(p) < target) __builtin_amdgcn_s_sleep(1);
}

// Workgroup `wg` of one packed weight: rows wg * R .. of it, in stages s = (tile t, part p) in
// order, t = s / np, p = s % np.
template <int TYPE, int C>
__device__ __forceinline__ void bstream_rows(uint8_t* smem, const uint8_t* w, long long row_bytes,
                                             const Act& act, YOut y, long long ldy,
                                             int M, int N, const BsGeo& geo, int wg) {
  using Tile = typename TileOf<TYPE>::T;
  using F = typename Tile::F;
  constexpr int TB = kBlockBytes<TYPE>;
  constexpr int kLaneCopies = (kStageCopies<TYPE> + kCopyWaves - 1) / kCopyWaves;

  const int tid = threadIdx.x, lane = tid & 63, ln = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ncw = geo.ncw, nct = 64 * ncw;  // compute waves and their threads
  const int nb = act.nb, kb = geo.kb, np = (nb + kb - 1) / kb;
  const int r0 = wg * geo.rows_per_wg;
  const int rows = min(geo.rows_per_wg, N - r0);  // >= 1: the grid is ceil(N / R)
  const int T = (rows + 15) >> 4, S = T * np;
  const int rs = geo.rs, nbuf = geo.nbuf, buf_bytes = geo.buf_bytes, ntp = geo.ntp;

  uint8_t* stage = smem;                                    // [nbuf][buf_bytes]
  float* Tp0 = (float*)(smem + nbuf * buf_bytes);           // [ntp]: block values [kb][16 n][16 m]
  float* Dp0 = Tp0 + ntp * kb * 256;                        // [ntp]: block weight scales [kb][16 n]
  float* Ad = Dp0 + ntp * kb * 16;                          // activation scales [nb][16 m]
  float* Yo = Ad + nb * 16;                                 // outputs [kOutTiles][16 n][16 m]
  int* ctrl = (int*)(Yo + kOutTiles * 256);
  int* ready = ctrl;
  int* done = ctrl + 4;
  int* vals = ctrl + 8;
  int* folded = ctrl + 10;
  int* nfold = ctrl + 12;  // quarter folds of all stages
  if (tid < kCtrlInts) ctrl[tid] = 0;
  __syncthreads();

  auto tile_rows = [&](int t) { return min(16, rows - 16 * t); };
  auto part_blocks = [&](int p) { return min(kb, nb - p * kb); };
  // the stage's first byte: row 16 t, block kb * p
  auto stage_base = [&](int s) {
    return w + (size_t)(r0 + 16 * (s / np)) * row_bytes + (size_t)(s % np) * kb * TB;
  };
  // LDS offset of a row piece's first byte
  auto piece_off = [&](int s, int j) {
    return j * rs * 16 + (int)((uintptr_t)(stage_base(s) + (size_t)j * row_bytes) & 15);
  };

  // Folds outputs [o_lo, o_lo + 64) (o = 16 n + m, one per lane) of stage s into acc once every
  // compute wave's values of the stage are in LDS; the tile's last part writes the staging ring.
  auto fold = [&](int s, int o_lo, float& acc) {
    const int t = s / np, p = s % np, rv = tile_rows(t), sv = s % ntp, nk = part_blocks(p);
    const float* Tp = Tp0 + sv * kb * 256;
    const float* Dp = Dp0 + sv * kb * 16;
    const float* Ap = Ad + p * kb * 16;
    const int o = o_lo + lane, n = o >> 4, m = o & 15;
    if (p == 0) acc = 0.0f;
    if (n < rv && m < M) {
      int bq = 0;
      for (; bq + 8 <= nk; bq += 8) {  // operands read ahead of the dependent chain
        float xv[8], vv[8], dv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          xv[i] = Ap[(bq + i) * 16 + m];
          vv[i] = Tp[(bq + i) * 256 + n * 16 + m];
          dv[i] = Dp[(bq + i) * 16 + n];
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) acc = Tile::fold(acc, xv[i], vv[i], dv[i]);
      }
      for (; bq < nk; ++bq) acc = Tile::fold(acc, Ap[bq * 16 + m], Tp[bq * 256 + n * 16 + m], Dp[bq * 16 + n]);
      if (p == np - 1) Yo[(t % kOutTiles) * 256 + o] = acc;
    }
  };

  if (wave >= ncw) {
    // ------------------------------------------------------------------ copy waves
    // Copy q of a stage moves chunks e = 64 q + lane (chunk k of row piece j); copy wave c issues
    // q = c, c + kCopyWaves, ... of every stage, so the stages are requested in order.
    const int c = wave - ncw;
    // a 16-byte aligned chunk holding a byte of the matrix never leaves that byte's page
    const uintptr_t last = ((uintptr_t)(w + (size_t)N * row_bytes) - 1) & ~(uintptr_t)15;
    const uint32_t stage_lds = lds_addr(stage);
    auto last_chunk = [&](int s) {  // index of the stage's last chunk that holds its bytes
      const int rv = tile_rows(s / np);
      const uintptr_t ra = (uintptr_t)(stage_base(s) + (size_t)(rv - 1) * row_bytes);
      return (rv - 1) * rs + (int)(((ra & 15) + part_blocks(s % np) * TB + 15) >> 4) - 1;
    };
    auto my_copies = [&](int s) {
      const int nq = (last_chunk(s) >> 6) + 1;
      return nq > c ? (nq - c + kCopyWaves - 1) / kCopyWaves : 0;
    };
    // Aligned pieces (16-byte aligned rows and piece offsets, the usual case): chunk e of any
    // stage sits at a fixed offset from the stage's first byte, so the lane's offsets are
    // computed once; kq keeps the chunk's index within its piece.
    const bool aligned = (((uintptr_t)w | (uintptr_t)row_bytes | (uintptr_t)(kb * TB)) & 15) == 0;
    long long off[kLaneCopies];
    int kq[kLaneCopies];
#pragma unroll
    for (int i = 0; i < kLaneCopies; ++i) {
      const int e = 64 * (c + kCopyWaves * i) + lane, j = e / rs;
      kq[i] = e - j * rs;
      off[i] = (long long)j * row_bytes + 16 * kq[i];
    }
    auto issue = [&](int s) {
      const int ll = last_chunk(s);
      const uint8_t* sb = stage_base(s);
      const uint32_t dst = stage_lds + (uint32_t)((s % nbuf) * buf_bytes);
      const int pbytes = part_blocks(s % np) * TB;
      if (aligned) {
        const int pc = pbytes >> 4;  // chunks of a piece
#pragma unroll
        for (int i = 0; i < kLaneCopies; ++i) {
          const int q = c + kCopyWaves * i;
          if (64 * q <= ll) {  // wave-uniform; such a copy always has live lanes
            if (kq[i] < pc && 64 * q + lane <= ll) copy16_to_lds(sb + off[i], dst + 1024 * q);
          }
        }
        return;
      }
      int j = (64 * c + lane) / rs, k = (64 * c + lane) - j * rs;  // of chunk 64 q + lane
      for (int q = c; 64 * q <= ll; q += kCopyWaves) {  // every such copy has live lanes
        const int e = 64 * q + lane;
        const uintptr_t ra = (uintptr_t)(sb + (size_t)j * row_bytes);
        const int crow = (int)(((ra & 15) + pbytes + 15) >> 4);
        if (e <= ll && k < crow) {
          const uintptr_t a = (ra & ~(uintptr_t)15) + 16 * k;
          copy16_to_lds((const void*)(a < last ? a : last), dst + 1024 * q);
        }
        for (k += 64 * kCopyWaves; k >= rs; k -= rs) ++j;
      }
    };
    auto buffer_free = [&](int s) {  // the stage that used s's buffer before is computed
      return s < nbuf || lds_load(&done[s % nbuf]) >= (s / nbuf) * ncw;
    };
    // This wave folds a quarter of every stage (64 outputs, one per lane), stages in order,
    // whenever it would otherwise wait: the compute waves never wait for one another.
    int nf = 0;
    float acc = 0.0f;
    auto vals_complete = [&](int s) { return lds_load(&vals[s % ntp]) >= (s / ntp + 1) * ncw; };
    auto fold_next = [&]() {
      fold(nf, 64 * c, acc);
      __builtin_amdgcn_s_waitcnt(0xC07F);
      if (lane == 0) {
        lds_add(&folded[nf % ntp], 1);
        lds_add(nfold, 1);
      }
      ++nf;
    };
    // Signal stages in order as they land; refill buffers as they free up. Block on a buffer only
    // when no copy is in flight (and fold meanwhile), so a landed stage is never held back behind
    // a full issue queue.
    int issued = 0;
    while (issued < min(min(kFirstStages, nbuf), S)) issue(issued++);
    for (int sig = 0; sig < S; ++sig) {
      if (issued == sig) {
        while (!buffer_free(sig)) {
          if (nf < S && vals_complete(nf)) fold_next();
          else __builtin_amdgcn_s_sleep(1);
        }
        issue(issued++);
      }
      int after = 0;
      for (int k = sig + 1; k < issued; ++k) after += my_copies(k);
      wait_vmcnt(after);
      if (lane == 0) lds_add(&ready[sig % nbuf], 1);
      while (issued < S && buffer_free(issued)) issue(issued++);
      while (nf < S && vals_complete(nf)) fold_next();
    }
    while (nf < S) {
      wait_at_least(&vals[nf % ntp], (nf / ntp + 1) * ncw);
      fold_next();
    }
    return;
  }

  // -------------------------------------------------------------------- compute waves
  // The wave's blocks of a part: b0 .. b0 + C - 1 within it. Their A operands (activation rows
  // >= M repeat row M - 1: computed, never stored) stay in registers; with several parts per
  // row, the next part's operands are loaded while the current stage is computed.
  const int b0 = wave * C;
  const int am = min(ln, M - 1);
  F Fc[C], Fn[C];
  auto load_frags = [&](int p, F* dst) {
#pragma unroll
    for (int c = 0; c < C; ++c) dst[c] = Tile::frag_g(act, am, min(p * kb + b0 + c, nb - 1), g);
  };
  load_frags(0, Fc);
  // (a folder reads every wave's scales: each wave's stores complete before its first count)
  for (int i = tid; i < nb * 16; i += nct) Ad[i] = act.d[(size_t)min(i & 15, M - 1) * nb + (i >> 4)];

  // Outputs of finished tiles go from the staging ring to y, coalesced along n.
  auto flush = [&](int t0, int t1) {  // tiles t0 .. t1 - 1, all folded
    const int n0 = 16 * t0, nr = min(rows, 16 * t1) - n0;
    for (int i = tid; i < nr * M; i += nct) {
      const int m = i / nr, n = n0 + (i - m * nr);
      y.put((size_t)m * ldy + r0 + n, Yo[((n >> 4) % kOutTiles) * 256 + (n & 15) * 16 + m]);
    }
  };

  for (int s = 0; s < S; ++s) {
    const int t = s / np, p = s % np, b = s % nbuf, sv = s % ntp;
    if (np > 1 && s + 1 < S) load_frags((s + 1) % np, Fn);
    if (p == 0 && t >= kOutTiles && t % kOutTiles == 0) {  // the staging ring is full: write it out
      wait_at_least(nfold, t * np * kCopyWaves);
      flush(t - kOutTiles, t);
    }
    wait_at_least(&ready[b], (s / nbuf + 1) * kCopyWaves);  // stage s has landed
    if (s >= ntp) wait_at_least(&folded[sv], (s / ntp) * kCopyWaves);  // value buffer sv is free
    const int j = min(ln, tile_rows(t) - 1);  // rows past the tile's end compute its last row
    const uint8_t* buf = stage + b * buf_bytes;
    const int roff = piece_off(s, j);
    const int nk = part_blocks(p);
    float* Tp = Tp0 + sv * kb * 256;
    float* Dp = Dp0 + sv * kb * 16;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int bl = b0 + c;  // block within the part
      if (bl < nk) {
        const typename Tile::W wv = Tile::load_lds(buf, roff + bl * TB, g);
        const typename Tile::P pp = Tile::prep(wv, g);
        Tile::value(pp, Fc[c], g, [&](int e, float v, float dd) {
          Tp[bl * 256 + ln * 16 + 4 * g + e] = v;
          if (g == 0 && e == 0) Dp[bl * 16 + ln] = dd;
        });
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the stage reads and value writes are done
    if (lane == 0) {
      lds_add(&done[b], 1);
      lds_add(&vals[sv], 1);
    }
    if (np > 1) {
#pragma unroll
      for (int c = 0; c < C; ++c) Fc[c] = Fn[c];
    }
  }
  wait_at_least(nfold, S * kCopyWaves);
  flush(T - 1 - (T - 1) % kOutTiles, T);
}

template <int TYPE, int C>
__global__ __launch_bounds__(768) void bstream_kernel(const uint8_t* w, long long row_bytes, Act act,
                                                      YOut y, long long ldy, int M,
                                                      int N, BsGeo geo) {
  extern __shared__ __align__(16) uint8_t smem[];
  bstream_rows<TYPE, C>(smem, w, row_bytes, act, y, ldy, M, N, geo, blockIdx.x);
}

// Several weights sharing the activations in one launch: workgroups wg0 .. of segment s take its
// rows; each segment has its own rows per workgroup and stage geometry.
constexpr int kMaxSegs = 4;
struct BsSeg {
  const uint8_t* w;
  long long row_bytes;
  YOut y;  // the segment's first output column
  int n, type, wg0, rows_per_wg, rs, buf_bytes;
};
struct BsSegs {
  BsSeg s[kMaxSegs];
  int count;
};

template <int C>
__global__ __launch_bounds__(768) void bstream_multi_kernel(BsSegs segs, Act act, long long ldy, int M,
                                                            BsGeo geo) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int wg = blockIdx.x;
  int i = 0;
  while (i + 1 < segs.count && wg >= segs.s[i + 1].wg0) ++i;
  const BsSeg sg = segs.s[i];
  BsGeo g = geo;
  g.rows_per_wg = sg.rows_per_wg;
  g.rs = sg.rs;
  g.buf_bytes = sg.buf_bytes;
  switch (sg.type) {
    case T_Q4_K: bstream_rows<T_Q4_K, C>(smem, sg.w, sg.row_bytes, act, sg.y, ldy, M, sg.n, g, wg - sg.wg0); break;
    case T_Q6_K: bstream_rows<T_Q6_K, C>(smem, sg.w, sg.row_bytes, act, sg.y, ldy, M, sg.n, g, wg - sg.wg0); break;
    default: bstream_rows<T_Q8_0, C>(smem, sg.w, sg.row_bytes, act, sg.y, ldy, M, sg.n, g, wg - sg.wg0); break;
  }
}

// Stage pieces: whole rows for up to 16 blocks, else kPartBlocks blocks.
inline int stage_blocks(int nb) { return nb <= 16 ? nb : kPartBlocks; }

template <int TYPE>
int stage_buffer_bytes(int kb) {  // bytes of one stage buffer, or -1
  const int bytes = (16 * row_chunks((long long)kb * kBlockBytes<TYPE>) * 16 + 1023) / 1024 * 1024;
  return bytes / 1024 > kStageCopies<TYPE> ? -1 : bytes;
}

// LDS bytes for nbuf stage buffers of buf_bytes and ntp value buffers.
inline int bs_lds_bytes(int nbuf, int buf_bytes, int ntp, int kb, int nb) {
  return nbuf * buf_bytes + ntp * kb * (256 + 16) * 4 + nb * 16 * 4 + kOutTiles * 256 * 4 +
         kCtrlInts * 4;
}

// Picks stage and value buffers for LDS; false when nothing fits.
inline bool bs_buffers(BsGeo& geo, int buf_bytes, int kb, int nb) {
  constexpr int kLdsMax = 160 * 1024;
  const int pref[5][2] = {{4, 2}, {3, 2}, {3, 1}, {2, 2}, {2, 1}};
  for (int i = 0; i < 5; ++i) {
    // a copy wave's outstanding copies (nbuf stages) stay within what vmcnt counts
    if (pref[i][0] * ((buf_bytes / 1024 + kCopyWaves - 1) / kCopyWaves) > kMaxCopies) continue;
    if (bs_lds_bytes(pref[i][0], buf_bytes, pref[i][1], kb, nb) <= kLdsMax) {
      geo.nbuf = pref[i][0];
      geo.ntp = pref[i][1];
      return true;
    }
  }
  return false;
}

template <int TYPE, int C>
int launch_bs(const uint8_t* w, long long row_bytes, const Act& act, YOut y, long long ldy, int M,
              int N, hipStream_t stream) {
  const int nb = act.nb;
  const int ncu = cu_count();
  BsGeo geo;
  geo.kb = stage_blocks(nb);
  geo.ncw = (geo.kb + C - 1) / C;
  if (geo.ncw + kCopyWaves > 12) return -1;
  geo.rows_per_wg = max(16, (int)((N + (long long)ncu - 1) / ncu));
  geo.rs = row_chunks((long long)geo.kb * kBlockBytes<TYPE>);
  geo.buf_bytes = stage_buffer_bytes<TYPE>(geo.kb);
  if (geo.buf_bytes < 0 || !bs_buffers(geo, geo.buf_bytes, geo.kb, nb)) return -1;
  const int lds = bs_lds_bytes(geo.nbuf, geo.buf_bytes, geo.ntp, geo.kb, nb);
  allow_lds((const void*)bstream_kernel<TYPE, C>, 160 * 1024);
  const int grid = (int)((N + (long long)geo.rows_per_wg - 1) / geo.rows_per_wg);
  hipLaunchKernelGGL((bstream_kernel<TYPE, C>), dim3(grid), dim3(64 * (geo.ncw + kCopyWaves)), lds,
                     stream, w, row_bytes, act, y, ldy, M, N, geo);
  return 0;
}

template <int TYPE>
int launch_bs_type(const uint8_t* w, long long row_bytes, const Act& act, YOut y, long long ldy,
                   int M, int N, hipStream_t stream) {
  const int nb = act.nb;
  // one or two blocks per compute wave and stage: at most 8 compute waves
  if (nb <= 8 || nb > 16) return launch_bs<TYPE, 1>(w, row_bytes, act, y, ldy, M, N, stream);
  return launch_bs<TYPE, 2>(w, row_bytes, act, y, ldy, M, N, stream);
}

template <int C>
int launch_bs_multi(const DecodeSeg* seg, int count, const Act& act, long long ldy, int M,
                    hipStream_t stream) {
  const int nb = act.nb;
  const int ncu = cu_count();
  BsGeo geo;
  geo.kb = stage_blocks(nb);
  geo.ncw = (geo.kb + C - 1) / C;
  if (count < 1 || count > kMaxSegs || geo.ncw + kCopyWaves > 12) return -1;
  BsSegs segs;
  segs.count = count;
  int buf_max = 0, bytes[kMaxSegs];
  double total = 0.0;
  for (int i = 0; i < count; ++i) {
    const int t = seg[i].type;
    bytes[i] = t == T_Q4_K ? stage_buffer_bytes<T_Q4_K>(geo.kb)
             : t == T_Q6_K ? stage_buffer_bytes<T_Q6_K>(geo.kb)
             : t == T_Q8_0 ? stage_buffer_bytes<T_Q8_0>(geo.kb) : -1;
    if (bytes[i] < 0) return -1;
    buf_max = max(buf_max, bytes[i]);
    total += (double)seg[i].n * (double)seg[i].row_bytes;
  }
  if (!bs_buffers(geo, buf_max, geo.kb, nb)) return -1;
  int wg0 = 0;
  for (int i = 0; i < count; ++i) {
    const int share = max(1, (int)((double)ncu * seg[i].n * seg[i].row_bytes / total + 0.5));
    const int R = max(16, (seg[i].n + share - 1) / share);
    const int tb = seg[i].type == T_Q4_K ? 144 : seg[i].type == T_Q6_K ? 210 : 272;
    segs.s[i] = BsSeg{seg[i].w, seg[i].row_bytes, seg[i].y, seg[i].n, seg[i].type, wg0, R,
                      row_chunks((long long)geo.kb * tb), bytes[i]};
    wg0 += (seg[i].n + R - 1) / R;
  }
  const int lds = bs_lds_bytes(geo.nbuf, buf_max, geo.ntp, geo.kb, nb);
  allow_lds((const void*)bstream_multi_kernel<C>, 160 * 1024);
  hipLaunchKernelGGL((bstream_multi_kernel<C>), dim3(wg0), dim3(64 * (geo.ncw + kCopyWaves)), lds,
                     stream, segs, act, ldy, M, geo);
  return 0;
}

}  // namespace

int launch_bstream(int type, const uint8_t* w, long long row_bytes, const Act& act, YOut y,
                   long long ldy, int m_rows, int n_rows, hipStream_t stream) {
  if (act.q == nullptr || m_rows < 1 || m_rows > 16 || n_rows < 1) return -1;
  switch (type) {
    case T_Q4_K: return launch_bs_type<T_Q4_K>(w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
    case T_Q6_K: return launch_bs_type<T_Q6_K>(w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
    case T_Q8_0: return launch_bs_type<T_Q8_0>(w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
    default: return -1;
  }
}

int launch_bstream_multi(const DecodeSeg* seg, int count, const Act& act, long long ldy,
                         int m_rows, hipStream_t stream) {
  if (act.q == nullptr || m_rows < 1 || m_rows > 16) return -1;
  if (act.nb <= 8 || act.nb > 16) return launch_bs_multi<1>(seg, count, act, ldy, m_rows, stream);
  return launch_bs_multi<2>(seg, count, act, ldy, m_rows, stream);
}

}  // namespace mxa
