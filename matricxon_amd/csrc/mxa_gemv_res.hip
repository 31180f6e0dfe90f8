// Decode GEMV for one activation row over a workgroup-resident weight share: y[n] = sum_k x[k] *
// W[n, k]. Used for weights up to about 12 MB (the small projections of a decode step); larger
// ones take the pipelined lane-per-block kernel (mxa_gemv_lpb.hip), which measured faster there.
//
// Memory. One workgroup per CU owns RW consecutive weight rows (one contiguous byte range) and
// keeps all of them in LDS: no buffer is ever reused, so no wave waits for another to free one.
// Copy waves stream the range in with global_load_lds_dwordx4 (1 KB per instruction) and do
// nothing else, so the stream never waits for compute; compute waves quantize the activations,
// then take units of 32 groups (256-value super-blocks, or eight Q8_0 blocks) as soon as the
// copies holding them have landed. The hand-over is a frontier per copy wave in LDS.
//
// Compute. In a unit the lane pair 2g, 2g + 1 owns group g and lane c its values 128c..128c+127:
// integer dot products of that half, summed over the pair through DPP (exact), then the group's
// float value, which goes into LDS over the group's own bytes.
//
// Numerics (app/native/src/mx_dot_k_ssse3.c:115-154, mx_dot_k_ssse3.c:109-209, mx_dot_q8_0.c:5-22): the
// per-group float steps are the CPU oracle's, and after its units a wave folds each of its rows
// over the row's groups in order 0..nb-1 (one lane per row), so results equal the oracle bit for
// bit. IQ4_XS keeps float activations and uses the summation order of every other IQ4_XS kernel.
#include "mxa_kernels.hpp"

#pragma clang fp contract(off)

namespace mxa {
namespace {

constexpr int kResMaxWaves = 16;
constexpr long long kResMaxBytes = 12LL << 20;  // weights this kernel takes (see launch_gemv_res)
constexpr int kResLds = 160 * 1024;
constexpr int kResTail = 16;  // LDS bytes after the last region: dword reads of a block's last bytes

// x in LDS, one slot per 256-value group b. The copies land at the start of the slot (the 256
// floats, or for activations that arrive as Q8_K: q8 at +0, 16 bsums at +256, the 16-byte piece
// of the d array holding d[b] at +288). The wave that owns the group then rewrites it, in place,
// as the operands the units read, laid out so that the 16-byte reads of the lanes of consecutive
// groups spread over the 16-byte bank groups instead of all landing on one (a 1 KB slot stride
// alone maps every group to the same banks): Q8_K chunk c (q8 values 64c..64c+63) at
// 64 (b & 1) + 80 c, bsums at 384 + 32 (b & 3), d at 512 + 4 (b & 3); IQ4_XS float chunk c at
// 64 (b & 1) + 272 c.
constexpr int kSlotQ8 = 1024;
constexpr int kSlotF32 = 1152;
constexpr int kRawBs = 256;
constexpr int kRawD = 288;

__device__ __forceinline__ int xq_chunk(int b, int c) { return 64 * (b & 1) + 80 * c; }
__device__ __forceinline__ int xq_bs(int b) { return 384 + 32 * (b & 3); }
__device__ __forceinline__ int xq_d(int b) { return 512 + 4 * (b & 3); }
__device__ __forceinline__ int xf_chunk(int b, int c) { return 64 * (b & 1) + 272 * c; }

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // 16-byte aligned
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));  // 8-byte aligned

__device__ __forceinline__ float lane_read(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

// LDS wait for this wave's own reads and writes, then a workgroup barrier without any wait on
// vmcnt (the weight copies stay in flight across it).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt at their maximum
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
}

// NW dwords of LDS starting at byte `off` of `base` (off 2-byte aligned at worst).
template <int NW>
__device__ __forceinline__ void lds_dwords(const uint8_t* base, int off, uint32_t* w) {
  const uint32_t* p = (const uint32_t*)(base + (off & ~3));
  const uint32_t sh = (uint32_t)(off & 3);
  uint32_t raw[NW + 1];
#pragma unroll
  for (int i = 0; i < NW + 1; ++i) raw[i] = p[i];
#pragma unroll
  for (int i = 0; i < NW; ++i) w[i] = __builtin_amdgcn_alignbyte(raw[i + 1], raw[i], sh);
}

// Q8_K operands of one lane: q8 values 128c..128c+127 of its group (chunks 2c and 2c+1) and its
// eight 16-value bsums 8c..8c+7 (four packed pairs: sub-blocks 4c..4c+3).
struct QOps {
  uint32_t q[32];
  uint32_t bs[4];
};

// The lane's operands of group b from its slot (operand layout).
__device__ __forceinline__ void load_qops(const uint8_t* slot, int b, int c, QOps& o, float& xd) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint8_t* q = slot + xq_chunk(b, 2 * c + h);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4 v = *(const u32x4*)(q + 16 * i);
      o.q[16 * h + 4 * i] = v.x, o.q[16 * h + 4 * i + 1] = v.y;
      o.q[16 * h + 4 * i + 2] = v.z, o.q[16 * h + 4 * i + 3] = v.w;
    }
  }
  const u32x4 bs = *(const u32x4*)(slot + xq_bs(b) + 16 * c);
  o.bs[0] = bs.x, o.bs[1] = bs.y, o.bs[2] = bs.z, o.bs[3] = bs.w;
  xd = *(const float*)(slot + xq_d(b));
}

__device__ __forceinline__ int bs_pair_sum(uint32_t w) {
  return (int)(int16_t)(w & 0xFFFFu) + (int)(int16_t)(w >> 16);
}

// The two lanes of a pair (2g, 2g + 1) through DPP: the sum, and one lane's value for both.
__device__ __forceinline__ int pair_sum(int v) { return v + quad_xor1(v); }
__device__ __forceinline__ float pair_sum(float v) {
  return v + __builtin_bit_cast(float, quad_xor1(__builtin_bit_cast(int, v)));
}
template <int I>
__device__ __forceinline__ float pair_bcast(float v) {
  constexpr int sel = I | (I << 2) | ((2 + I) << 4) | ((2 + I) << 6);
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), sel,
                                                               0xF, 0xF, false));
}

template <int TYPE>
struct Pair;

// Q4_K: lane c holds qs bytes 64c..64c+63, i.e. sub-blocks 4c..4c+3 (chunk 2c + k: sub-block
// 4c + 2k in its low nibbles, 4c + 2k + 1 in its high ones). Group value fmaf(d, sumi, -(dmin *
// summ)); fold fmaf(y.d, value, acc) (mx_dot_k_ssse3.c:150-154).
template <>
struct Pair<T_Q4_K> {
  static constexpr int kBytes = 144;
  static constexpr bool kQ8K = true;
  __device__ static void compute(const uint8_t* blk, int c, const QOps& x, float xd, float& A,
                                 float& B) {
    // 144-byte groups of a 16-byte aligned range: 16-byte reads
    const u32x4 h = *(const u32x4*)blk;
    uint32_t q[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4 v = *(const u32x4*)(blk + 16 + 64 * c + 16 * i);
      q[4 * i] = v.x, q[4 * i + 1] = v.y, q[4 * i + 2] = v.z, q[4 * i + 3] = v.w;
    }
    const K4Scales s = k4_scales(h.y, h.z, h.w);
    const uint32_t sc = c ? s.sc_hi : s.sc_lo, mn = c ? s.mn_hi : s.mn_lo;  // byte k: sub-block 4c + k
    int sumi16 = 0, summ = 0;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      int lo = 0, hs = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t w = q[8 * k + i];
        lo = sdot4(w & 0x0F0F0F0Fu, x.q[16 * k + i], lo);
        // high nibbles as signed bytes 16 h - 128: sum(h * x) = (sum((16 h - 128) x) + 128 X) / 16
        hs = sdot4((w & 0xF0F0F0F0u) ^ 0x80808080u, x.q[16 * k + 8 + i], hs);
      }
      const int sc0 = (int)((sc >> (16 * k)) & 0xFFu), sc1 = (int)((sc >> (16 * k + 8)) & 0xFFu);
      sumi16 += 16 * __mul24(sc0, lo) + __mul24(sc1, hs + 128 * bs_pair_sum(x.bs[2 * k + 1]));
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) summ += __mul24((int)((mn >> (8 * k)) & 0xFFu), bs_pair_sum(x.bs[k]));
    sumi16 = pair_sum(sumi16);
    summ = pair_sum(summ);
    const float d = half_to_float(h.x), dmin = half_to_float(h.x >> 16);
    B = fmaf(d, (float)(sumi16 >> 4), -(dmin * (float)summ));
    A = xd;
  }
};

// Q6_K: lane c holds half c of the block (elements 128c..128c+127): ql bytes 64c..64c+63, qh
// bytes 32c..32c+31, scales 8c..8c+7. sumi = sum_s sc_s * sum((u - 32) * q8); fold
// fmaf(y.d * d, sumi, acc) (mx_dot_k_ssse3.c:167-209).
template <>
struct Pair<T_Q6_K> {
  static constexpr int kBytes = 210;
  static constexpr bool kQ8K = true;
  // the group may start 2 bytes past a dword boundary: read through lds_dwords from the base
  __device__ static void compute(const uint8_t* base, int off, int c, const QOps& x, float xd,
                                 float& A, float& B) {
    uint32_t l[16], qh[8], scw[2], dw[1];
    lds_dwords<16>(base, off + 64 * c, l);
    lds_dwords<8>(base, off + 128 + 32 * c, qh);
    lds_dwords<2>(base, off + 192 + 8 * c, scw);
    lds_dwords<1>(base, off + 208, dw);
    int sumi = 0;
#pragma unroll
    for (int g = 0; g < 4; ++g) {  // elements 128c + 32g .. +31: sub-blocks 8c + 2g + {0, 1}
#pragma unroll
      for (int half16 = 0; half16 < 2; ++half16) {
        int sdot = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int wi = 4 * half16 + i;
          const uint32_t lw = l[(g & 1) * 8 + wi];
          const uint32_t u = g == 0 ? q6_codes<0>(lw, qh[wi]) : g == 1 ? q6_codes<1>(lw, qh[wi])
                           : g == 2 ? q6_codes<2>(lw, qh[wi]) : q6_codes<3>(lw, qh[wi]);
          sdot = sdot4(u, x.q[8 * g + wi], sdot);
        }
        const int sbi = 2 * g + half16;  // scale byte sbi of the lane's eight
        const int sc = (int)(int8_t)(uint8_t)(scw[sbi >> 2] >> (8 * (sbi & 3)));
        const uint32_t bw = x.bs[g];
        const int bs = half16 ? (int)(int16_t)(bw >> 16) : (int)(int16_t)(bw & 0xFFFFu);
        sumi += __mul24(sc, sdot - 32 * bs);
      }
    }
    sumi = pair_sum(sumi);
    B = (float)sumi;
    A = xd * half_to_float(dw[0]);
  }
};

// Q8_0: lane c holds the 34-byte blocks 4c..4c+3 of the group (bytes 136c..136c+135). The group
// value is sum_k d_k * (qs_k . q8) in k order 0..7 (mx_dot_q8_0.c:8-18): the pair's partial dot
// products are exchanged so both lanes run the same chain.
template <>
struct Pair<T_Q8_0> {
  static constexpr int kBytes = 272;
  static constexpr bool kQ8K = true;
  __device__ static void compute(const uint8_t* blk, int c, const QOps& x, float xd, float& A,
                                 float& B) {
    float dk[4], fk[4];
#pragma unroll
    for (int m = 0; m < 2; ++m) {  // block pairs 4c + 2m, 4c + 2m + 1: 68 bytes, 17 words
      uint32_t w[17];
      const uint8_t* p = blk + 136 * c + 68 * m;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const u32x4a4 v = *(const u32x4a4*)(p + 16 * i);
        w[4 * i] = v.x, w[4 * i + 1] = v.y, w[4 * i + 2] = v.z, w[4 * i + 3] = v.w;
      }
      w[16] = *(const uint32_t*)(p + 64);
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        dk[2 * m + e] = e == 0 ? half_to_float(w[0]) : half_to_float(w[8] >> 16);
        int acc = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t qs = e == 0 ? __builtin_amdgcn_alignbyte(w[i + 1], w[i], 2) : w[9 + i];
          acc = sdot4(qs, x.q[8 * (2 * m + e) + i], acc);
        }
        fk[2 * m + e] = (float)acc;
      }
    }
    float bs = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) bs = fmaf(pair_bcast<0>(dk[e]), pair_bcast<0>(fk[e]), bs);
#pragma unroll
    for (int e = 0; e < 4; ++e) bs = fmaf(pair_bcast<1>(dk[e]), pair_bcast<1>(fk[e]), bs);
    B = bs;
    A = xd;
  }
};

// IQ4_XS (float activations): lane c holds sub-blocks 4c..4c+3 (qs bytes 64c..64c+63). Quarter
// value fmaf(dl1, p1, dl0 * p0) with p a sequential fmaf over the sub-block; the block value
// (q0 + q1) + (q2 + q3); rows add the group values in order. The order of every IQ4_XS kernel here.
template <>
struct Pair<T_IQ4_XS> {
  static constexpr int kBytes = 136;
  static constexpr bool kQ8K = false;
  // xq: the lane's 128 floats as two chunks of 64 (x0: values 128c.., x1: 128c + 64..)
  __device__ static void compute(const uint8_t* blk, int c, const float* x0, const float* x1,
                                 float& A, float& B) {
    // 136-byte groups of a 16-byte aligned range are 8-byte aligned: 8-byte reads
    const u32x2 hw = *(const u32x2*)blk;
    const float d = half_to_float(hw.x);
    const uint32_t sh = hw.x >> 16, sl = hw.y;
    uint32_t qw[16];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const u32x2 v = *(const u32x2*)(blk + 8 + 64 * c + 8 * i);
      qw[2 * i] = v.x, qw[2 * i + 1] = v.y;
    }
    float L[2];
#pragma unroll
    for (int jq = 0; jq < 2; ++jq) {  // quarter 2c + jq: sub-blocks 4c + 2jq + {0, 1}
      float p[2], dl[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int tl = 2 * jq + t;  // sub-block 4c + tl of the block
        const int ib = 4 * c + tl;
        const int ls = (int)(((sl >> (4 * ib)) & 15u) | (((sh >> (2 * ib)) & 3u) << 4));
        dl[t] = d * (float)(ls - 32);
        const float* xs = (jq == 0 ? x0 : x1) + 32 * t;  // values 32 ib .. 32 ib + 31
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t w = qw[4 * tl + i];
          const uint32_t gl = iq4_lookup4(w & 0x0F0F0F0Fu), gh = iq4_lookup4((w >> 4) & 0x0F0F0F0Fu);
          const float4 xl = *(const float4*)(xs + 4 * i);
          const float4 xh = *(const float4*)(xs + 16 + 4 * i);
          acc = fmaf(xl.x, sbyte_f<0>(gl), acc);
          acc = fmaf(xl.y, sbyte_f<1>(gl), acc);
          acc = fmaf(xl.z, sbyte_f<2>(gl), acc);
          acc = fmaf(xl.w, sbyte_f<3>(gl), acc);
          acc = fmaf(xh.x, sbyte_f<0>(gh), acc);
          acc = fmaf(xh.y, sbyte_f<1>(gh), acc);
          acc = fmaf(xh.z, sbyte_f<2>(gh), acc);
          acc = fmaf(xh.w, sbyte_f<3>(gh), acc);
        }
        p[t] = acc;
      }
      L[jq] = fmaf(dl[1], p[1], dl[0] * p[0]);
    }
    B = pair_sum(L[0] + L[1]);
    A = 1.0f;  // fmaf(1, v, acc) == acc + v
  }
};

// 8-byte aligned spot inside group j's bytes of the wave's region for its fold operands.
template <int GB>
__device__ __forceinline__ int fold_slot(int j) {
  if constexpr (GB % 8 == 0)
    return j * GB;
  else
    return (j * GB + 7) & ~7;
}

// Row r of the workgroup's rows: its groups' fold operands (left in LDS by the units) folded
// in order 0..nb-1 with the oracle's fused steps (mx_dot_k_ssse3.c:115-154); y points at row 0's output.
template <int GB>
__device__ __forceinline__ void fold_row(const uint8_t* reg, int r, int nb, YOut y) {
  float acc = 0.0f;
  const int j0 = r * nb;
  int bb = 0;
  for (; bb + 8 <= nb; bb += 8) {
    float2 v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = *(const float2*)(reg + fold_slot<GB>(j0 + bb + i));
#pragma unroll
    for (int i = 0; i < 8; ++i) acc = fmaf(v[i].x, v[i].y, acc);
  }
  for (; bb < nb; ++bb) {
    const float2 v = *(const float2*)(reg + fold_slot<GB>(j0 + bb));
    acc = fmaf(v.x, v.y, acc);
  }
  y.put(r, acc);
}

struct ResGeo {
  int rows_per_wg;  // consecutive weight rows of one workgroup
  int copy_waves;   // waves 0 .. copy_waves - 1 stream those rows into LDS
  int slot;         // LDS bytes of an x slot
};

constexpr int kInFlight = 8;  // copies a copy wave keeps outstanding while it publishes progress

constexpr int kCounters = 64;  // LDS bytes of the hand-over counters at the start of LDS
constexpr int kUnit = 32;      // groups per unit: one per lane pair of a wave
// Every wait on a counter gives up after this many polls (about 0.1 s): the published values
// always reach what is waited for, and the limit only guarantees that a wave cannot spin forever
// should that ever not hold. A wave whose wait gave up writes NaN as its groups' fold operands, so
// every output it touched is NaN rather than a plausible wrong value.
constexpr int kSpinLimit = 1 << 22;
constexpr int kXReady = 8;     // counter index: activation groups ready as operands

// Hand-over counters, accessed through LDS-qualified pointers: a volatile access through a generic
// pointer becomes a flat instruction, which counts on vmcnt and makes its wave wait for every copy
// it has in flight.
typedef __attribute__((address_space(3))) int lds_i32;
typedef int i32x4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ int lds_load(int* p) { return *(volatile lds_i32*)(lds_i32*)p; }
__device__ __forceinline__ void lds_store(int* p, int v) { *(volatile lds_i32*)(lds_i32*)p = v; }
// Copies below the smallest of the four copy-wave frontiers (one 16-byte LDS read) have landed.
typedef __attribute__((address_space(3))) i32x4v lds_i32x4;
__device__ __forceinline__ int frontier(int* cnt) {
  const i32x4v f = *(volatile lds_i32x4*)(lds_i32x4*)cnt;
  return min(min(f.x, f.y), min(f.z, f.w));
}
__device__ __forceinline__ void lds_add(int* p, int v) {
  __atomic_fetch_add((lds_i32*)p, v, __ATOMIC_RELAXED);
}

// Copy wave `cw` of nc: copies t = cw, cw + nc, ... < ct of the rows at src (1 KB each, to LDS
// byte address r_lds + 1024 t), K in flight; publishes its frontier cw + nc * landed in cnt[cw].
// Only the range's last copy can reach past the matrix: it alone is clamped per lane.
template <int K>
__device__ __forceinline__ void copy_rows(const uint8_t* src, const uint8_t* last, uint32_t r_lds,
                                          int ct, int nc, int cw, int lane, int* cnt) {
  const uint32_t voff = (uint32_t)lane * 16;
  int n = 0;
  for (int t = cw; t < ct; t += nc) {
    if (t + 1 < ct)
      copy16_to_lds_s(src + t * 1024, voff, r_lds + (uint32_t)(t * 1024));
    else
      copy16_to_lds((const void*)min((uintptr_t)(src + t * 1024 + voff), (uintptr_t)last),
                    r_lds + (uint32_t)(t * 1024));
    if (++n > K) {
      __builtin_amdgcn_s_waitcnt((K & 15) | ((K >> 4) << 14) | 0x0F70);  // vmcnt(K)
      lds_store(cnt + cw, cw + nc * (n - K));
    }
  }
  // the last copies are published one by one as they land, so the final units start in order
  for (int k = min(K, n) - 1; k > 0; --k) {
    wait_vmcnt(k);
    lds_store(cnt + cw, cw + nc * (n - k));
  }
  // always published, also by a wave with no copies: cw + nc * n >= ct
  wait_vmcnt(0);
  lds_store(cnt + cw, cw + nc * n);
}

// Roles. Copy waves move the workgroup's rows (one contiguous, 16-byte aligned byte range) into
// LDS with global_load_lds_dwordx4, 1 KB per instruction, copy t by copy wave t mod NC, in
// order. A CU accepts only about 64 KB of copies in flight and a wave stalls at the instruction
// beyond that, so the copy waves do nothing else: the stream stays saturated from the first
// microsecond whatever the compute waves are waiting for. After a copy has landed (its own
// vmcnt), a copy wave publishes its frontier in LDS: every copy below min over copy waves of
// (k + NC * landed_k) is in LDS. Compute waves first copy and prepare the activations (their
// copies go out before any weight copy), then take units of kUnit groups in turn and start each as
// soon as the frontier passes its last byte. The whole share of the workgroup stays in LDS, so no
// buffer is ever reused and no wave waits for another to free one.
//
// XQ8K: the activations arrive as Q8_K in the workspace (copied); otherwise as floats, quantized
// to Q8_K in the kernel (IQ4_XS keeps them). ACTREG: every unit's groups sit at the same block
// positions of their rows (16 % nb == 0), so a lane loads its Q8_K operands once.
template <int TYPE, bool XQ8K, bool ACTREG>
__global__ __launch_bounds__(1024) void gemv_res_kernel(const uint8_t* __restrict__ w,
                                                          long long row_bytes, Act act,
                                                          YOut y, int N,
                                                          ResGeo geo) {
  using Q = Pair<TYPE>;
  constexpr int GB = Q::kBytes;  // bytes of one 256-value group
  extern __shared__ __align__(16) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int NC = geo.copy_waves, NW = (int)(blockDim.x >> 6) - NC;
  const int nb = act.nb, RW = geo.rows_per_wg, slot = geo.slot;
  int* cnt = (int*)smem;
  uint8_t* xs = smem + kCounters;
  uint8_t* reg = xs + nb * slot;

  const int n0 = xcd_tile(blockIdx.x, gridDim.x) * RW;
  const int nrows = max(0, min(RW, N - n0));
  const uint8_t* src0 = w + (size_t)min(n0, N - 1) * row_bytes;
  const int CT = (nrows * (int)row_bytes + 1023) >> 10;  // the workgroup's copies
  // the last copy may extend past the rows, but not past the matrix's last 16-byte chunk
  const uint8_t* last = w + (size_t)N * row_bytes - 16;
  const int groups = nrows * nb, units = (groups + kUnit - 1) / kUnit;

  // frontiers of absent copy waves (k >= NC) never hold anyone back
  if (threadIdx.x < kCounters / 4)
    lds_store(cnt + threadIdx.x, threadIdx.x < 4 && (int)threadIdx.x >= NC ? 0x7FFFFFFF : 0);
  // 1. compute waves copy the activations; the barrier puts those copies ahead of every weight copy
  if (wave >= NC) {
    const uint32_t xs_lds = lds_addr(xs);
    for (int b = wave - NC; b < nb; b += NW) {
      if constexpr (XQ8K) {
        // lanes 0-15: q8 values; 16-17: the 16 bsums; 18: the 16 bytes of d holding d[b]
        if (lane < 19) {
          const uint8_t* src = lane < 16 ? (const uint8_t*)(act.q + QK * b) + 16 * lane
                             : lane < 18 ? (const uint8_t*)(act.bsums + 16 * b) + 16 * (lane - 16)
                                         : (const uint8_t*)(act.d + 4 * (b >> 2));
          copy16_to_lds(src, xs_lds + (uint32_t)(slot * b));
        }
      } else {
        copy16_to_lds(act.x + QK * b + 4 * lane, xs_lds + (uint32_t)(slot * b));
      }
    }
  }
  lds_barrier();

  if (wave < NC) {
    // 2a. copy wave: priority over the compute waves of its SIMD, so the stream never waits for
    // an instruction slot
    __builtin_amdgcn_s_setprio(3);
    copy_rows<kInFlight>(src0, last, lds_addr(reg), CT, NC, wave, lane, cnt);
  } else {
    // 2b. compute wave: the activation groups it copied become operands (a wave reads its whole
    // slot into registers before it writes any of it)
    const int cw = wave - NC;
    wait_vmcnt(0);
    int done = 0;
    for (int b = cw; b < nb; b += NW, ++done) {
      uint8_t* sl = xs + slot * b;
      if constexpr (!Q::kQ8K) {
        const float4 v = *(const float4*)(sl + 16 * lane);  // values 4 lane .. 4 lane + 3
        __builtin_amdgcn_s_waitcnt(0xC07F);
        *(float4*)(sl + xf_chunk(b, lane >> 4) + 16 * (lane & 15)) = v;
      } else {
        uint32_t qw;
        int bsum;
        float d;
        if constexpr (XQ8K) {
          qw = *(const uint32_t*)(sl + 4 * lane);
          bsum = *(const int16_t*)(sl + kRawBs + 2 * (lane >> 2));
          d = *(const float*)(sl + kRawD + 4 * (b & 3));
        } else {
          // quantize (mx_quantize_row_q8_k, mx_common.c:42-69): lane l holds values 4l..4l+3
          const float4 v = *(const float4*)(sl + 16 * lane);
          float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
          amax = max16(amax);
          amax = fmaxf(fmaxf(lane_read(amax, 0), lane_read(amax, 16)),
                       fmaxf(lane_read(amax, 32), lane_read(amax, 48)));
          int q0 = 0, q1 = 0, q2 = 0, q3 = 0;
          if (amax != 0.0f) {
            const float iscale = 127.0f / amax;
            q0 = (int)fminf(fmaxf(rintf(v.x * iscale), -127.0f), 127.0f);
            q1 = (int)fminf(fmaxf(rintf(v.y * iscale), -127.0f), 127.0f);
            q2 = (int)fminf(fmaxf(rintf(v.z * iscale), -127.0f), 127.0f);
            q3 = (int)fminf(fmaxf(rintf(v.w * iscale), -127.0f), 127.0f);
          }
          bsum = quad_sum(q0 + q1 + q2 + q3);  // lanes 4i..4i+3: values 16i..16i+15
          qw = (uint32_t)(q0 & 0xFF) | ((uint32_t)(q1 & 0xFF) << 8) |
               ((uint32_t)(q2 & 0xFF) << 16) | ((uint32_t)(q3 & 0xFF) << 24);
          d = amax / 127.0f;
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);
        *(uint32_t*)(sl + xq_chunk(b, lane >> 4) + 4 * (lane & 15)) = qw;
        if ((lane & 3) == 0) *(int16_t*)(sl + xq_bs(b) + 2 * (lane >> 2)) = (int16_t)bsum;
        if (lane == 0) *(float*)(sl + xq_d(b)) = d;
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    if (done > 0 && lane == 0) lds_add(cnt + kXReady, done);
    bool gave_up = false;  // some wait of this wave ran out of polls
    {
      int spin = 0;
      while (lds_load(cnt + kXReady) < nb && ++spin < kSpinLimit) __builtin_amdgcn_s_sleep(2);
      gave_up |= spin >= kSpinLimit;
    }
    asm volatile("" ::: "memory");

    // 3. units v = cw, cw + NW, ... of kUnit groups of the workgroup's rows
    const int g = lane >> 1, c = lane & 1;
    QOps xq;
    float xd = 0.0f;
    if constexpr (ACTREG) {
      const int b = g % nb;
      load_qops(xs + slot * b, b, c, xq, xd);
    }
    for (int v = cw; v < units; v += NW) {
      const int gcount = min(kUnit, groups - kUnit * v);
      const int lastc = ((kUnit * v + gcount) * GB - 1) >> 10;  // copy holding the unit's last byte
      int spin = 0;
      for (; spin < kSpinLimit; ++spin) {  // the four frontiers in one LDS read
        const int f = frontier(cnt);
        if (f > lastc) break;
        // a copy lands about every 40 ns per CU: sleep longer when the unit is further away, so
        // that waiting waves take few issue slots from working ones
        if (lastc - f > 8)
          __builtin_amdgcn_s_sleep(8);
        else
          __builtin_amdgcn_s_sleep(1);
      }
      gave_up |= spin == kSpinLimit;
      asm volatile("" ::: "memory");
      const int j = kUnit * v + min(g, gcount - 1);  // lanes past the rows redo their last group
      float A, B;
      if constexpr (Q::kQ8K) {
        if constexpr (!ACTREG) {
          const int b = j % nb;
          load_qops(xs + slot * b, b, c, xq, xd);
        }
        if constexpr (TYPE == T_Q6_K)
          Q::compute(reg, j * GB, c, xq, xd, A, B);
        else
          Q::compute(reg + j * GB, c, xq, xd, A, B);
      } else {
        const int b = j % nb;
        const uint8_t* sl = xs + slot * b;
        Q::compute(reg + j * GB, c, (const float*)(sl + xf_chunk(b, 2 * c)),
                   (const float*)(sl + xf_chunk(b, 2 * c + 1)), A, B);
      }
      // the group's fold operands go over its own bytes, which no lane reads again and no later
      // copy writes (later copies start past the unit's last byte)
      if (gave_up) A = B = __builtin_nanf("");
      if (c == 0 && g < gcount) *(float2*)(reg + fold_slot<GB>(j)) = float2{A, B};
    }
    if constexpr (ACTREG) {
      // units hold whole rows (kUnit % nb == 0): after its last unit the wave folds the rows of
      // all its units, one lane per row (unit cw + NW * (l / per), row l % per of it)
      const int per = kUnit / nb;
      for (int l = lane; l < per * ((units - cw + NW - 1) / NW); l += 64) {
        const int r = (cw + NW * (l / per)) * per + l % per;
        if (r < nrows) fold_row<GB>(reg, r, nb, y.at(n0));
      }
    }
  }
  if constexpr (ACTREG) return;
  lds_barrier();
  // 4. fold: one thread per row takes the row's groups in order 0..nb-1 (mx_dot_k_ssse3.c:115-154)
  for (int r = threadIdx.x; r < nrows; r += blockDim.x) fold_row<GB>(reg, r, nb, y.at(n0));
}

template <int TYPE, bool XQ8K>
int launch_res_t(const uint8_t* w, long long row_bytes, const Act& act, YOut y, int N,
                  hipStream_t stream) {
  using Q = Pair<TYPE>;
  const int nb = act.nb;
  if (nb < 1 || N < 1 || (long long)nb * Q::kBytes != row_bytes) return -1;
  if (((uintptr_t)w & 15) != 0 || row_bytes % 16 != 0) return -1;
  const int slot = Q::kQ8K ? kSlotQ8 : kSlotF32;
  const int fixed = kCounters + nb * slot + kResTail;
  const int ncu = cu_count();
  // rows per workgroup: one workgroup per CU when its rows fit LDS beside the activations
  int RW = (N + ncu - 1) / ncu;
  const int max_rows = (int)((kResLds - fixed) / row_bytes);
  if (max_rows < 1) return -1;
  if (RW > max_rows) RW = max_rows;
  const int region = (int)(((RW * row_bytes + 1023) / 1024) * 1024);
  if (fixed + region > kResLds) {
    RW = (int)(((kResLds - fixed) / 1024) * 1024 / row_bytes);
    if (RW < 1) return -1;
  }
  const int CT = (int)((RW * row_bytes + 1023) / 1024);
  const int units = (RW * nb + kUnit - 1) / kUnit;
  // 4 copy waves with 8 copies in flight each (32 KB per CU) and up to 12 compute waves measured
  // fastest on MI355X; more copies in flight delay the activations and the first units
  const int NC = min(4, CT), NWc = min(kResMaxWaves - NC, min(12, units));
  if ((nb + NWc - 1) / NWc > kMaxCopies) return -1;
  ResGeo geo{RW, NC, slot};
  const int lds = fixed + (int)(((RW * row_bytes + 1023) / 1024) * 1024);
  const int grid = (N + RW - 1) / RW;
  const bool actreg = Q::kQ8K && kUnit % nb == 0;
  auto kern = actreg ? gemv_res_kernel<TYPE, XQ8K, Q::kQ8K> : gemv_res_kernel<TYPE, XQ8K, false>;
  allow_lds((const void*)gemv_res_kernel<TYPE, XQ8K, Q::kQ8K>, kResLds);
  allow_lds((const void*)gemv_res_kernel<TYPE, XQ8K, false>, kResLds);
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * (NC + NWc)), lds, stream, w, row_bytes, act, y, N,
                     geo);
  return 0;
}

}  // namespace

int launch_gemv_res(int type, const uint8_t* w, long long row_bytes, const Act& act, YOut y,
                     int n_rows, hipStream_t stream) {
  // Measured on MI355X against the pipelined lane-per-block kernel: faster for weights up to
  // about 12 MB (Q4_K 4096 x 4096: 5.2 vs 5.7 us; Q6_K 1024 x 4096: 6.3 vs 6.7 us), slower above
  // (Q4_K 14336 x 4096: 10.2 vs 9.7 us; Q6_K 128256 x 4096: 117 vs 108 us).
  if ((long long)n_rows * row_bytes > kResMaxBytes) return -1;
  if (((uintptr_t)act.x & 15) != 0 || (act.q == nullptr && act.xbf16)) return -1;
  const bool q8k = act.q != nullptr;
  switch (type) {
    case T_Q4_K: return q8k ? launch_res_t<T_Q4_K, true>(w, row_bytes, act, y, n_rows, stream)
                            : launch_res_t<T_Q4_K, false>(w, row_bytes, act, y, n_rows, stream);
    case T_Q6_K: return q8k ? launch_res_t<T_Q6_K, true>(w, row_bytes, act, y, n_rows, stream)
                            : launch_res_t<T_Q6_K, false>(w, row_bytes, act, y, n_rows, stream);
    case T_Q8_0: return q8k ? launch_res_t<T_Q8_0, true>(w, row_bytes, act, y, n_rows, stream)
                            : launch_res_t<T_Q8_0, false>(w, row_bytes, act, y, n_rows, stream);
    case T_IQ4_XS: return q8k ? -1 : launch_res_t<T_IQ4_XS, false>(w, row_bytes, act, y, n_rows, stream);
    default: return -1;
  }
}

}  // namespace mxa
