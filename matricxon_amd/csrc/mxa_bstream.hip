// Batched decode (up to 16 activation rows) on the matrix cores, weights streamed through LDS.
//
// Work split. One persistent workgroup per CU owns R consecutive weight rows (R = N / CUs, at
// least 16), cut into 16-row tiles (the last may be partial). Its compute waves split K: wave w
// owns the C consecutive blocks b0 = w * C .. b0 + C - 1 of every row, so the Q8_K activations of
// those blocks (the MFMA A operands of all 16 activation rows) stay in the wave's registers for
// the whole call.
//
// Memory. A stage is one tile: 16 whole rows, one contiguous byte range, moved into one of nbuf
// LDS stage buffers with global_load_lds_dwordx4 (1 KB of consecutive bytes per instruction) by
// four copy waves, each issuing every fourth copy of every tile, tiles in order. Issuing a copy
// stalls while the memory system is saturated, so copying and computing are separate waves, and
// they hand stages over through LDS counters rather than workgroup barriers (a barrier would make
// the compute waves wait for a copy wave stuck behind its own issue queue):
//   ready[b]  counts copy waves whose share of the tile in buffer b has landed (vmcnt);
//   done[b]   counts compute waves finished with buffer b (the copy wave reuses it at the next
//             multiple of the compute-wave count);
//   vals[s]   counts compute waves whose block values of a tile are in value buffer s; once it
//             is complete every compute wave folds its share of the tile's outputs;
//   folded[s] counts those shares (a wave may overwrite value buffer s once every share of the
//             tile that used it last is folded).
// Every counter only grows and every wait is for an earlier tile, so the waits always end. In LDS
// each row starts on a 16-byte chunk boundary and the row stride is an odd number of chunks, so
// the 16 rows a B-operand read touches fall in different banks. B operands are built from the LDS
// copy with the tile builders of mxa_tiles.hpp (lane = weight row).
//
// Fold. One thread per (weight row, activation row) folds its nb block values in order 0..nb-1
// with the oracle's fused steps (app/native/src/mx_gemm.c:241-261), so results equal the decode
// kernels and the oracle bit for bit. Outputs wait in LDS and are written once, coalesced, at the
// end.
#include "mxa_kernels.hpp"
#include "mxa_tiles.hpp"

#pragma clang fp contract(off)

namespace mxa {
namespace {

template <int TYPE>
constexpr int kBlockBytes = TYPE == T_Q4_K ? 144 : TYPE == T_Q6_K ? 210 : 272;

// LDS chunks (16 bytes) per row: enough for the row at any start offset, rounded up to odd.
__host__ __device__ constexpr int row_chunks(long long row_bytes) {
  return (int)(((row_bytes + 15 + 15) / 16) | 1);
}

struct BsGeo {
  int rows_per_wg;  // R
  int rs;           // LDS chunks per row
  int nbuf;         // stage buffers
  int buf_bytes;    // bytes of one stage buffer (whole 1 KB copies)
  int ntp;          // block-value buffers
  int ncw;          // compute waves (ceil(nb / C)); the kCopyWaves waves after them copy
};

constexpr int kCopyWaves = 4;
constexpr int kFirstTiles = 2;  // tiles requested before the first one lands (at most nbuf)
constexpr int kOutTiles = 8;    // tiles of outputs staged in LDS before they are written out
// Copies of one tile a copy wave issues at most: 16 rows of up to nb = 16 blocks, 1 KB each.
template <int TYPE>
constexpr int kTileCopies = (16 * 16 * (16 * kBlockBytes<TYPE> / 16 + 2) + 1023) / 1024;
constexpr int kCtrlInts = 16;  // ready[4] done[4] vals[2] folded[2]

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

// Workgroup `wg` of one packed weight: rows wg * R .. of it.
template <int TYPE, int C>
__device__ __forceinline__ void bstream_rows(uint8_t* smem, const uint8_t* w, long long row_bytes,
                                             const Act& act, float* __restrict__ y, long long ldy,
                                             int M, int N, const BsGeo& geo, int wg) {
  using Tile = typename TileOf<TYPE>::T;
  constexpr int TB = kBlockBytes<TYPE>;
  constexpr int kLaneCopies = (kTileCopies<TYPE> + kCopyWaves - 1) / kCopyWaves;

  const int tid = threadIdx.x, lane = tid & 63, ln = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ncw = geo.ncw, nct = 64 * ncw;  // compute waves and their threads
  const int nb = act.nb;
  const int r0 = wg * geo.rows_per_wg;
  const int rows = min(geo.rows_per_wg, N - r0);  // >= 1: the grid is ceil(N / R)
  const int T = (rows + 15) >> 4;
  const int rs = geo.rs, nbuf = geo.nbuf, buf_bytes = geo.buf_bytes, ntp = geo.ntp;

  uint8_t* stage = smem;                                    // [nbuf][buf_bytes]
  float* Tp0 = (float*)(smem + nbuf * buf_bytes);           // [ntp]: block values [nb][16 n][16 m]
  float* Dp0 = Tp0 + ntp * nb * 256;                        // [ntp]: block weight scales [nb][16 n]
  float* Ad = Dp0 + ntp * nb * 16;                          // activation scales [nb][16 m]
  float* Yo = Ad + nb * 16;                                 // outputs [kOutTiles][16 n][16 m]
  int* ctrl = (int*)(Yo + kOutTiles * 256);
  int* ready = ctrl;
  int* done = ctrl + 4;
  int* vals = ctrl + 8;
  int* folded = ctrl + 10;
  int* nfold = ctrl + 12;  // quarter folds of all tiles
  if (tid < kCtrlInts) ctrl[tid] = 0;
  __syncthreads();

  auto tile_rows = [&](int t) { return min(16, rows - 16 * t); };
  auto tile_base = [&](int t) { return w + (size_t)(r0 + 16 * t) * row_bytes; };

  // Folds outputs [o_lo, o_hi) (o = 16 n + m) of tile t once every compute wave's values of the
  // tile are in LDS, into the output staging.
  auto fold = [&](int t, int o_lo, int o_hi) {
    const int rv = tile_rows(t), sv = t % ntp;
    const float* Tp = Tp0 + sv * nb * 256;
    const float* Dp = Dp0 + sv * nb * 16;
    float* Yt = Yo + (t % kOutTiles) * 256;
    for (int o = o_lo + lane; o < o_hi; o += 64) {
      const int n = o >> 4, m = o & 15;
      if (n < rv && m < M) {
        float acc = 0.0f;
        int bq = 0;
        for (; bq + 8 <= nb; bq += 8) {  // operands read ahead of the dependent chain
          float xv[8], vv[8], dv[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            xv[i] = Ad[(bq + i) * 16 + m];
            vv[i] = Tp[(bq + i) * 256 + n * 16 + m];
            dv[i] = Dp[(bq + i) * 16 + n];
          }
#pragma unroll
          for (int i = 0; i < 8; ++i) acc = Tile::fold(acc, xv[i], vv[i], dv[i]);
        }
        for (; bq < nb; ++bq) acc = Tile::fold(acc, Ad[bq * 16 + m], Tp[bq * 256 + n * 16 + m], Dp[bq * 16 + n]);
        Yt[o] = acc;
      }
    }
  };

  if (wave >= ncw) {
    // ------------------------------------------------------------------ copy waves
    // Copy q of a tile moves chunks e = 64 q + lane (chunk k of tile row j); copy wave c issues
    // q = c, c + kCopyWaves, ... of every tile, so the tiles are requested in order.
    const int c = wave - ncw;
    // a 16-byte aligned chunk holding a byte of the matrix never leaves that byte's page
    const uintptr_t last = ((uintptr_t)(w + (size_t)N * row_bytes) - 1) & ~(uintptr_t)15;
    const uint32_t stage_lds = lds_addr(stage);
    auto last_chunk = [&](int t) {  // index of the tile's last chunk that holds matrix bytes
      const int rv = tile_rows(t);
      const uintptr_t ra = (uintptr_t)(tile_base(t) + (size_t)(rv - 1) * row_bytes);
      return (rv - 1) * rs + (int)(((ra & 15) + row_bytes + 15) >> 4) - 1;
    };
    auto my_copies = [&](int t) {
      const int nq = (last_chunk(t) >> 6) + 1;
      return nq > c ? (nq - c + kCopyWaves - 1) / kCopyWaves : 0;
    };
    // 16-byte aligned rows (the usual case): chunk e of any tile sits at a fixed offset from the
    // tile's first byte, so the lane's offsets for its copies are computed once. -1 marks the LDS
    // padding chunk at the end of a row, which no copy fills.
    const bool rows_aligned = (((uintptr_t)w | (uintptr_t)row_bytes) & 15) == 0;
    const int rc = (int)(row_bytes >> 4);  // chunks of an aligned row
    int off[kLaneCopies];
#pragma unroll
    for (int i = 0; i < kLaneCopies; ++i) {
      const int e = 64 * (c + kCopyWaves * i) + lane, j = e / rs, k = e - j * rs;
      off[i] = k < rc ? 16 * (e - j * (rs - rc)) : -1;
    }
    auto issue = [&](int t) {
      const int ll = last_chunk(t);
      const uint8_t* tb = tile_base(t);
      const uint32_t dst = stage_lds + (uint32_t)((t % nbuf) * buf_bytes);
      if (rows_aligned) {
#pragma unroll
        for (int i = 0; i < kLaneCopies; ++i) {
          const int q = c + kCopyWaves * i;
          if (64 * q <= ll) {  // wave-uniform; such a copy always has live lanes
            if (off[i] >= 0 && 64 * q + lane <= ll) copy16_to_lds(tb + off[i], dst + 1024 * q);
          }
        }
        return;
      }
      int j = (64 * c + lane) / rs, k = (64 * c + lane) - j * rs;  // of chunk 64 q + lane
      for (int q = c; 64 * q <= ll; q += kCopyWaves) {  // every such copy has live lanes
        const int e = 64 * q + lane;
        const uintptr_t ra = (uintptr_t)(tb + (size_t)j * row_bytes);
        const int crow = (int)(((ra & 15) + row_bytes + 15) >> 4);
        if (e <= ll && k < crow) {
          const uintptr_t a = (ra & ~(uintptr_t)15) + 16 * k;
          copy16_to_lds((const void*)(a < last ? a : last), dst + 1024 * q);
        }
        for (k += 64 * kCopyWaves; k >= rs; k -= rs) ++j;
      }
    };
    auto buffer_free = [&](int t) {  // the tile that used t's buffer before is computed
      return t < nbuf || lds_load(&done[t % nbuf]) >= (t / nbuf) * ncw;
    };
    // This wave folds a quarter of every tile (64 outputs, one per lane), tiles in order, whenever
    // it would otherwise wait: the compute waves never wait for one another.
    int nf = 0;
    auto vals_complete = [&](int t) { return lds_load(&vals[t % ntp]) >= (t / ntp + 1) * ncw; };
    auto fold_next = [&]() {
      fold(nf, 64 * c, 64 * c + 64);
      __builtin_amdgcn_s_waitcnt(0xC07F);
      if (lane == 0) {
        lds_add(&folded[nf % ntp], 1);
        lds_add(nfold, 1);
      }
      ++nf;
    };
    auto fold_ready = [&]() {
      while (nf < T && vals_complete(nf)) fold_next();
    };
    // Signal tiles in order as they land; refill buffers as they free up. Block on a buffer only
    // when no copy is in flight (and fold meanwhile), so a landed tile is never held back behind
    // a full issue queue.
    int issued = 0;
    while (issued < min(min(kFirstTiles, nbuf), T)) issue(issued++);
    for (int sig = 0; sig < T; ++sig) {
      if (issued == sig) {
        while (!buffer_free(sig)) {
          if (nf < T && vals_complete(nf)) fold_next();
          else __builtin_amdgcn_s_sleep(1);
        }
        issue(issued++);
      }
      int after = 0;
      for (int k = sig + 1; k < issued; ++k) after += my_copies(k);
      wait_vmcnt(after);
      if (lane == 0) lds_add(&ready[sig % nbuf], 1);
      while (issued < T && buffer_free(issued)) issue(issued++);
      fold_ready();
    }
    while (nf < T) {
      wait_at_least(&vals[nf % ntp], (nf / ntp + 1) * ncw);
      fold_next();
    }
    return;
  }

  // -------------------------------------------------------------------- compute waves
  // The wave's blocks, their A operands (activation rows >= M repeat row M - 1: computed, never
  // stored) and the activation scales.
  const int b0 = wave * C, cw = min(C, nb - b0);  // cw >= 1: the host launches ceil(nb / C) waves
  typename Tile::F F[C];
  const int am = min(ln, M - 1);
#pragma unroll
  for (int c = 0; c < C; ++c) F[c] = Tile::frag_g(act, am, min(b0 + c, nb - 1), g);
  // (a folder reads every wave's scales: each wave's stores complete before its first count)
  for (int i = tid; i < nb * 16; i += nct) Ad[i] = act.d[(size_t)min(i & 15, M - 1) * nb + (i >> 4)];

  // Outputs of finished tiles go from the staging ring to y, coalesced along n.
  auto flush = [&](int t0, int t1) {  // tiles t0 .. t1 - 1, all folded
    const int n0 = 16 * t0, nr = min(rows, 16 * t1) - n0;
    for (int i = tid; i < nr * M; i += nct) {
      const int m = i / nr, n = n0 + (i - m * nr);
      y[(size_t)m * ldy + r0 + n] = Yo[((n >> 4) % kOutTiles) * 256 + (n & 15) * 16 + m];
    }
  };

  for (int t = 0; t < T; ++t) {
    const int b = t % nbuf, sv = t % ntp;
    if (t >= kOutTiles && t % kOutTiles == 0) {  // the staging ring is full: write it out
      wait_at_least(nfold, t * kCopyWaves);
      flush(t - kOutTiles, t);
    }
    wait_at_least(&ready[b], (t / nbuf + 1) * kCopyWaves);  // tile t has landed
    if (t >= ntp) wait_at_least(&folded[sv], (t / ntp) * kCopyWaves);  // value buffer sv is free
    const int rv = tile_rows(t);
    const int j = min(ln, rv - 1);  // rows past the tile's end compute its last row: never stored
    const uint8_t* buf = stage + b * buf_bytes;
    const int roff = j * rs * 16 + (int)((uintptr_t)(tile_base(t) + (size_t)j * row_bytes) & 15);
    float* Tp = Tp0 + sv * nb * 256;
    float* Dp = Dp0 + sv * nb * 16;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      if (c < cw) {
        const int bb = b0 + c;
        const typename Tile::W wv = Tile::load_lds(buf, roff + bb * TB, g);
        const typename Tile::P pp = Tile::prep(wv, g);
        Tile::value(pp, F[c], g, [&](int e, float v, float dd) {
          Tp[bb * 256 + ln * 16 + 4 * g + e] = v;
          if (g == 0 && e == 0) Dp[bb * 16 + ln] = dd;
        });
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the stage reads and value writes are done
    if (lane == 0) {
      lds_add(&done[b], 1);
      lds_add(&vals[sv], 1);
    }
  }
  wait_at_least(nfold, T * kCopyWaves);
  flush(T - 1 - (T - 1) % kOutTiles, T);
}

template <int TYPE, int C>
__global__ __launch_bounds__(768) void bstream_kernel(const uint8_t* w, long long row_bytes, Act act,
                                                      float* __restrict__ y, long long ldy, int M,
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
  float* y;  // the segment's first output column
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

template <int TYPE, int C>
int launch_bs(const uint8_t* w, long long row_bytes, const Act& act, float* y, long long ldy, int M,
              int N, hipStream_t stream) {
  constexpr int kLdsMax = 160 * 1024;
  const int nb = act.nb;
  const int ncu = cu_count();
  BsGeo geo;
  geo.ncw = (nb + C - 1) / C;
  geo.rows_per_wg = max(16, (int)((N + (long long)ncu - 1) / ncu));
  geo.rs = row_chunks(row_bytes);
  geo.buf_bytes = (16 * geo.rs * 16 + 1023) / 1024 * 1024;
  if (geo.buf_bytes / 1024 > kTileCopies<TYPE>) return -1;
  auto lds_bytes = [&](int nbuf, int ntp) {
    return nbuf * geo.buf_bytes + ntp * nb * (256 + 16) * 4 + nb * 16 * 4 + kOutTiles * 256 * 4 +
           kCtrlInts * 4;
  };
  // preference: three stage buffers and two value buffers, then fewer
  geo.nbuf = 0;
  const int pref[4][2] = {{3, 2}, {3, 1}, {2, 2}, {2, 1}};
  for (int i = 0; i < 4 && geo.nbuf == 0; ++i)
    if (lds_bytes(pref[i][0], pref[i][1]) <= kLdsMax) geo.nbuf = pref[i][0], geo.ntp = pref[i][1];
  if (geo.nbuf == 0 || geo.ncw + kCopyWaves > 12) return -1;
  // a copy wave's outstanding copies (nbuf tiles) stay within what vmcnt counts
  if (geo.nbuf * ((geo.buf_bytes / 1024 + kCopyWaves - 1) / kCopyWaves) > kMaxCopies) return -1;
  const int lds = lds_bytes(geo.nbuf, geo.ntp);
  static bool lds_set = false;
  if (!lds_set) {
    (void)hipFuncSetAttribute((const void*)bstream_kernel<TYPE, C>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, kLdsMax);
    lds_set = true;
  }
  const int grid = (int)((N + (long long)geo.rows_per_wg - 1) / geo.rows_per_wg);
  hipLaunchKernelGGL((bstream_kernel<TYPE, C>), dim3(grid), dim3(64 * (geo.ncw + kCopyWaves)), lds,
                     stream, w, row_bytes, act, y, ldy, M, N, geo);
  return 0;
}

template <int TYPE>
int launch_bs_type(const uint8_t* w, long long row_bytes, const Act& act, float* y, long long ldy,
                   int M, int N, hipStream_t stream) {
  const int nb = act.nb;
  if (nb <= 8) return launch_bs<TYPE, 1>(w, row_bytes, act, y, ldy, M, N, stream);
  if (nb <= 16) return launch_bs<TYPE, 2>(w, row_bytes, act, y, ldy, M, N, stream);
  return -1;
}

template <int TYPE>
int stage_bytes_ok(long long row_bytes) {  // bytes of a tile's stage buffer, or -1
  const int bytes = (16 * row_chunks(row_bytes) * 16 + 1023) / 1024 * 1024;
  return bytes / 1024 > kTileCopies<TYPE> ? -1 : bytes;
}

template <int C>
int launch_bs_multi(const DecodeSeg* seg, int count, const Act& act, long long ldy, int M,
                    hipStream_t stream) {
  constexpr int kLdsMax = 160 * 1024;
  const int nb = act.nb;
  const int ncu = cu_count();
  BsGeo geo;
  geo.ncw = (nb + C - 1) / C;
  if (count < 1 || count > kMaxSegs || geo.ncw + kCopyWaves > 12) return -1;
  BsSegs segs;
  segs.count = count;
  int buf_max = 0;
  double total = 0.0;
  for (int i = 0; i < count; ++i) {
    const int t = seg[i].type;
    const int bytes = t == T_Q4_K ? stage_bytes_ok<T_Q4_K>(seg[i].row_bytes)
                    : t == T_Q6_K ? stage_bytes_ok<T_Q6_K>(seg[i].row_bytes)
                    : t == T_Q8_0 ? stage_bytes_ok<T_Q8_0>(seg[i].row_bytes) : -1;
    if (bytes < 0) return -1;
    buf_max = max(buf_max, bytes);
    total += (double)seg[i].n * (double)seg[i].row_bytes;
  }
  auto lds_bytes = [&](int nbuf, int ntp) {
    return nbuf * buf_max + ntp * nb * (256 + 16) * 4 + nb * 16 * 4 + kOutTiles * 256 * 4 +
           kCtrlInts * 4;
  };
  geo.nbuf = 0;
  const int pref[4][2] = {{3, 2}, {3, 1}, {2, 2}, {2, 1}};
  for (int i = 0; i < 4 && geo.nbuf == 0; ++i)
    if (lds_bytes(pref[i][0], pref[i][1]) <= kLdsMax) geo.nbuf = pref[i][0], geo.ntp = pref[i][1];
  if (geo.nbuf == 0 || geo.nbuf * ((buf_max / 1024 + kCopyWaves - 1) / kCopyWaves) > kMaxCopies) return -1;
  int wg0 = 0;
  for (int i = 0; i < count; ++i) {
    const int share = max(1, (int)((double)ncu * seg[i].n * seg[i].row_bytes / total + 0.5));
    const int R = max(16, (seg[i].n + share - 1) / share);
    const int t = seg[i].type;
    segs.s[i] = BsSeg{seg[i].w, seg[i].row_bytes, seg[i].y, seg[i].n, t, wg0, R,
                      row_chunks(seg[i].row_bytes),
                      t == T_Q4_K ? stage_bytes_ok<T_Q4_K>(seg[i].row_bytes)
                      : t == T_Q6_K ? stage_bytes_ok<T_Q6_K>(seg[i].row_bytes)
                                    : stage_bytes_ok<T_Q8_0>(seg[i].row_bytes)};
    wg0 += (seg[i].n + R - 1) / R;
  }
  const int lds = lds_bytes(geo.nbuf, geo.ntp);
  static bool lds_set = false;
  if (!lds_set) {
    (void)hipFuncSetAttribute((const void*)bstream_multi_kernel<C>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, kLdsMax);
    lds_set = true;
  }
  hipLaunchKernelGGL((bstream_multi_kernel<C>), dim3(wg0), dim3(64 * (geo.ncw + kCopyWaves)), lds,
                     stream, segs, act, ldy, M, geo);
  return 0;
}

}  // namespace

int launch_bstream(int type, const uint8_t* w, long long row_bytes, const Act& act, float* y,
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
  if (act.nb <= 8) return launch_bs_multi<1>(seg, count, act, ldy, m_rows, stream);
  if (act.nb <= 16) return launch_bs_multi<2>(seg, count, act, ldy, m_rows, stream);
  return -1;
}

}  // namespace mxa
