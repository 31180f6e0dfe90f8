// Decode GEMV for one activation row in the shape of the read floor: one workgroup per CU whose
// waves request every byte of their rows at their first instructions, then compute each row set
// as it lands. y[n] = sum_k x[k] * W[n, k] for K-quant / Q8_0 weights with nb = K / 256 in
// {4, 8, 16, 32, 56, 64}, and on float activations (one row): IQ4_XS and the fp32-activation
// forms of the K-quants and Q8_0.
//
// Memory. Wave v of a workgroup owns R = 64 / nb consecutive rows (64 blocks, or one row of 56
// with eight lanes idle; one byte range, 16-byte aligned because row_bytes is) and issues all of
// its range's 1 KB copies
// (global_load_lds_dwordx4, fully coalesced) into its own LDS stage before anything waits. The CU
// takes them in as its memory pipeline drains (it accepts ~64 KB in flight, so half the waves sit
// in their issue loop for microseconds); the whole matrix is in flight from the start and lands
// in the order HBM returns it. A wave waits only for its own copies (vmcnt), never for another
// wave's. With more rows than the CUs' waves hold, a wave takes further row sets, each requested
// once the previous one is computed.
//
// Activations. The first waves (stagers) also bring the activations into LDS with LDS-DMA copies
// issued before their weight copies: fp32 x, which they then quantize to Q8_K (16 lanes per
// 256-value block, the arithmetic of quantize_q8k_kernel), or the caller's Q8_K blocks, gathered
// per lane straight into place. Being copies, not loads, these are waited for with the stager's
// own vmcnt (a compiler-tracked load would make it wait for every weight copy issued after it).
// The stagers publish through an LDS counter, not a barrier, so a wave still issuing copies holds
// up no other. The q8 values sit in LDS as [16-byte piece i][block b]: the 64 lanes of a wave
// reading piece i of blocks lane % nb touch consecutive 16-byte words.
//
// Compute. Lane l computes block l of its wave's range whole (row l / nb, block l % nb), with the
// lane-per-block arithmetic of the pipelined decode kernel (mxa_lpb.hpp), Q4_K and Q8_0 with the
// lane's activation block in registers; one lane per row folds the row's block values in order
// with the CPU oracle's fused steps, so results equal it bit for bit
// (app/native/src/mx_dot_k_ssse3.c:115-209, mx_dot_q8_0.c:5-22). IQ4_XS keeps float
// activations: the stagers copy x as [16-byte piece][block] (consecutive lanes read consecutive
// 16-byte words) and lanes run the IQ4_XS block arithmetic every IQ4_XS kernel here shares, so a
// row's result does not depend on the kernel. nb is a template parameter: as a run-time value it
// costs the compute section ~1.7x the instructions (measured 8.0 vs 7.3 us).
#include "mxa_kernels.hpp"
#include "mxa_lpb.hpp"

#pragma clang fp contract(off)

namespace mxa {
namespace {

constexpr int kWaveMaxWaves = 16;
constexpr long long kWaveIq4MinBytes = 4ll << 20;
constexpr int kWaveLds = 160 * 1024;

template <int TYPE, int NB>
constexpr int wave_stage_bytes() {  // a wave's R = 64 / NB rows of NB blocks, in whole 1 KB copies
  return ((64 / NB) * NB * Lpb<TYPE>::kBytes + 1023) / 1024 * 1024;
}
// LDS of one wave: stage, block values V and (Q6_K) block scales D
// LDS of one wave: stage, block values V (one set per activation row) and (Q6_K) block scales D
template <int TYPE, int NB, int MAXM = 1>
constexpr int wave_region_bytes() {
  return wave_stage_bytes<TYPE, NB>() + 64 * 4 * (MAXM + (Lpb<TYPE>::kHasD ? 1 : 0));
}
// Activation area: per activation row, q8 pieces (nb * 256 bytes), bsums and d each in whole 1 KB
// copy windows (a gathering copy writes 1 KB); then the counter, then (fp32 x) nb KB of staged x
// per row.
__host__ __device__ constexpr int wave_bs_off(int nb) { return nb * QK; }
__host__ __device__ constexpr int wave_d_off(int nb) { return nb * QK + (nb * 32 + 1023) / 1024 * 1024; }
__host__ __device__ constexpr int wave_row_act(int nb) { return wave_d_off(nb) + 1024; }
__host__ __device__ constexpr int wave_flag_off(int nb, int m) { return m * wave_row_act(nb); }
__host__ __device__ constexpr int wave_x_off(int nb, int m) { return wave_flag_off(nb, m) + 16; }
__host__ __device__ constexpr int wave_act_bytes(int nb, bool fuseq, int m = 1) {
  return wave_x_off(nb, m) + (fuseq ? m * nb * 1024 : 0);
}
// Float activations kept as they are (IQ4_XS and the fp32-activation types): per row, fp32 x as
// [16-byte piece][block] (nb KB), then for the fp32-activation types the sixteen sums of 16 of each
// block ([block][16] floats); after the rows, the counter.
__host__ __device__ constexpr int wave_xf_row(int nb, bool sums) { return nb * (sums ? 1088 : 1024); }
__host__ __device__ constexpr int wave_xf_flag_off(int nb, int m, bool sums) { return m * wave_xf_row(nb, sums); }
__host__ __device__ constexpr int wave_xf_act_bytes(int nb, int m, bool sums) {
  return m * wave_xf_row(nb, sums) + 16;
}

// Q8_K activations staged as [piece i][block b][16 bytes]: the accessor of block b.
struct ActPieces {
  const int8_t* q;  // piece 0 of the block
  int stride;       // bytes between pieces (16 nb)
  const int16_t* bsums;
  __device__ i32x4a4 q16(int off) const { return *(const i32x4a4*)(q + (off >> 4) * stride); }
  __device__ u32x4a4 bs8(int h) const { return *(const u32x4a4*)(bsums + 8 * h); }
  __device__ uint32_t bs2(int j) const { return *(const uint32_t*)(bsums + 2 * j); }
  __device__ float4 x4(int) const { return float4{0.0f, 0.0f, 0.0f, 0.0f}; }
};

// fp32 activations staged as [16-byte piece][block]: the accessor of block b (consecutive lanes
// read consecutive 16-byte words).
struct ActXPieces {
  const float* x;     // piece 0 of the block
  int stride;         // floats between pieces (4 nb)
  const float* sums;  // the block's sixteen sums of 16 (fp32-activation types)
  __device__ float4 x4(int off) const { return *(const float4*)(x + (off >> 2) * stride); }
  __device__ float4 s4(int c) const { return *(const float4*)(sums + 4 * c); }  // sums 4c .. 4c + 3
  __device__ float s1(int j) const { return sums[j]; }
};

typedef __attribute__((address_space(3))) int lds_int;

// A wait that gives up after this many polls (the counter always reaches its target: each stager
// counts once after a bounded amount of work); a wave that gives up writes NaN.
constexpr int kWaveSpinLimit = 1 << 22;

// pack: waves | stagers << 8 | (activation rows | bf16 x << 7) << 16 | late row waves << 24: the
// first `waves` waves of the workgroup
// own rows, the first `stagers` also stage the activations (the workgroup has max(waves, stagers)
// waves; one that owns no rows only stages).
// The workgroup's work: workgroup wg of n_wg over the N rows of one weight, for M <= MAXM
// activation rows (y row m at y + m ldy).
template <int TYPE, int NB, bool FUSEQ, bool ACTREG, int MAXM = 1, bool LOOP = false>
__device__ __forceinline__ void wave_rows(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                          YOut y, int N, int row_bytes, int waves,
                                          int nq, int M, int ldy, const int8_t* __restrict__ aq,
                                          const float* __restrict__ ad,
                                          const int16_t* __restrict__ abs_, int wg, int n_wg,
                                          int late = 0, bool xbf16 = false) {
  using L = Lpb<TYPE>;
  static_assert(!ACTREG || MAXM == 1, "activations in registers for one row only");
  // float activations, unquantized (IQ4_XS, the fp32-activation types; these also use sums of 16)
  constexpr bool kXF = ActTraits<TYPE>::kFloat, kSums = ActTraits<TYPE>::kSums;
  constexpr int kXRow = wave_xf_row(NB, kSums);
  static_assert(!kXF || (!FUSEQ && !ACTREG), "float activations are staged, not quantized");
  constexpr int kStage = wave_stage_bytes<TYPE, NB>(), kCopies = kStage / 1024;
  constexpr int R = 64 / NB, kRounds = NB / 4, kRowAct = wave_row_act(NB), K = NB * QK;
  // bytes of a set in its last copy: the lanes past them are masked off, so a set whose bytes
  // end inside a copy (Q6_K 4 x 3360 = 13440: 896 bytes over) does not read the next set's rows,
  // which that set's own copies read again (lane 0 always copies: the instruction count that the
  // waits rely on is unchanged)
  constexpr int kTail = R * NB * Lpb<TYPE>::kBytes - (kCopies - 1) * 1024;
  static_assert(kTail > 0 && kTail <= 1024, "the last copy holds part of the set");
  if constexpr (MAXM == 1) M = 1;  // constant LDS offsets for the one-row kernel
  extern __shared__ __align__(16) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // activation row m: q8 pieces [16][NB][16] at smem + kRowAct m, bsums [NB][16], d [NB]
  const auto act_q = [&](int m) { return smem + kRowAct * m; };
  const auto act_bs = [&](int m) { return (int16_t*)(smem + kRowAct * m + wave_bs_off(NB)); };
  const auto act_d = [&](int m) { return (float*)(smem + kRowAct * m + wave_d_off(NB)); };
  lds_int* flag =
      (lds_int*)(lds_u8*)(smem + (kXF ? wave_xf_flag_off(NB, M, kSums) : wave_flag_off(NB, M)));
  float* xs = (float*)(smem + wave_x_off(NB, M));  // fp32 x: row m at xs + m K
  // late: the last `late` row waves have their regions in the fp32 x staging area, free once the
  // stagers have quantized x, so those waves request their rows only then (more row waves than
  // the LDS holds beside the staging area)
  // the launcher uses them for these alone
  constexpr bool kLate = FUSEQ && !kXF && (NB == 56 || (TYPE == T_Q6_K && MAXM == 4));
  const int late_idx = kLate ? wave - (waves - late) : -1;
  const bool late_wave = late_idx >= 0;
  uint8_t* wreg = late_wave ? (uint8_t*)xs + late_idx * wave_region_bytes<TYPE, NB, MAXM>()
                            : smem + (kXF ? wave_xf_act_bytes(NB, M, kSums) : wave_act_bytes(NB, FUSEQ, M)) +
                                  wave * wave_region_bytes<TYPE, NB, MAXM>();
  float* Vbuf = (float*)(wreg + kStage);  // row m's block values at Vbuf + 64 m
  float* Dbuf = Vbuf + 64 * MAXM;

  if (tid == 0) *flag = 0;
  __syncthreads();  // nothing is outstanding yet: the barrier waits for no memory

  // stager copies, ahead of this wave's weight copies: fp32 x one 1 KB block per copy (rounds of
  // four blocks of one row: wave, wave + nq, ..), or the Q8_K parts gathered into place (copy j
  // by stager j % nq)
  const bool stager = wave < nq;
  constexpr int kQ = NB / 4, kBs = (NB * 2 + 63) / 64, kPer = kQ + kBs + 1;  // gather copies per row
  if (stager) {
    if constexpr (kXF) {
      // float x as [16-byte piece][block]: copy j of row m moves slots s = 64 j + lane (piece
      // s / NB of block s % NB)
      for (int jm = wave; jm < NB * M; jm += nq) {
        const int m = jm / NB, j = jm % NB, sl = 64 * j + lane;
        copy16_to_lds((const void*)(x + (size_t)m * K + (sl % NB) * QK + 4 * (sl / NB)),
                      lds_addr(smem + m * kXRow) + 1024u * (uint32_t)j);
      }
    } else if constexpr (FUSEQ) {
      for (int r = wave; r < kRounds * M; r += nq) {
        const int m = r / kRounds, g0 = 4 * (r % kRounds);
        if (xbf16) {  // bfloat16 x: a 1 KB copy moves two blocks
          const uint16_t* xh = (const uint16_t*)x + (size_t)m * K;
          for (int g = g0; g < g0 + 4; g += 2)
            copy16_to_lds((const void*)(xh + g * QK + 8 * lane),
                          lds_addr((uint16_t*)xs + m * K + g * QK));
        } else {
          for (int g = g0; g < g0 + 4; ++g)
            copy16_to_lds((const void*)(x + (size_t)m * K + g * QK + 4 * lane),
                          lds_addr(xs + m * K + g * QK));
        }
      }
    } else {
      // Copy j of row m: q8 pieces (j < kQ; slot s = 64 j + lane: piece s / NB of block s % NB),
      // bsums (eight per slot), or the scales (four per slot); slots past the last repeat it.
      // Selected without branches: as a three-way branch on j this loop was compiled with the
      // scales' LDS destination left unset (the copy landed on the bsums).
      for (int jm = wave; jm < kPer * M; jm += nq) {
        const int m = jm / kPer, j = jm % kPer;
        const int sq = 64 * min(j, kQ - 1) + lane;
        const int sb = min(64 * max(j - kQ, 0) + lane, 2 * NB - 1);
        const int8_t* const pq = aq + (size_t)m * K + (sq % NB) * QK + 16 * (sq / NB);
        const int16_t* const pb = abs_ + (size_t)m * NB * 16 + 8 * sb;
        const float* const pd = ad + (size_t)m * NB + 4 * min(lane, NB / 4 - 1);
        const void* src = j < kQ ? (const void*)pq : j < kQ + kBs ? (const void*)pb : (const void*)pd;
        const int off = j < kQ ? 1024 * j
                      : j < kQ + kBs ? wave_bs_off(NB) + 1024 * (j - kQ) : wave_d_off(NB);
        copy16_to_lds(src, lds_addr(act_q(m)) + (uint32_t)off);
      }
    }
  }

  // Row set s (rows R s .. R s + R - 1), in rounds of n_wg * waves sets: in the first round the
  // workgroup's waves take sets tile * waves + wave (contiguous per workgroup); in later rounds
  // wave v of every workgroup takes set v * n_wg + tile of the round, so a partial last round
  // spreads over all workgroups rather than filling the first ones. Each set's copies are issued
  // once the previous set is computed. Every copy of a set's range is issued (the last ones may
  // pass it: they read the next set's rows, or stop at the matrix's last 16-byte word, and land
  // in this wave's stage).
  const bool has_rows = wave < waves;
  const int n_sets = (N + R - 1) / R, set_stride = n_wg * waves;
  const int tile = xcd_tile(wg, n_wg);
  int set = tile * waves + wave, round0 = 0;
  const uintptr_t last = ((uintptr_t)(w + (size_t)N * row_bytes) - 1) & ~(uintptr_t)15;
  const uint32_t lds_w = lds_addr(wreg), lane16 = 16u * (uint32_t)lane;
  // Copies clamped to the matrix's last 16-byte word. With the set loop: a wave-uniform base and
  // 32-bit lane offsets (one VGPR for every copy's address, which keeps the loop out of scratch);
  // in one pass, 64-bit lane addresses (measured 0.5-2% faster there).
  const auto issue = [&](int s) {
    const uintptr_t src = (uintptr_t)w + (uintptr_t)min(s * R, N - 1) * (uintptr_t)row_bytes;
    if constexpr (LOOP) {
      const uint64_t span = (uint64_t)(last - src);
      const uint32_t lim = span > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)span;
#pragma unroll
      for (int c = 0; c < kCopies; ++c)
        if (c + 1 < kCopies || kTail == 1024 || lane16 < (uint32_t)kTail)
          copy16_to_lds_s_nt((const void*)src, min(lane16 + (uint32_t)(c * 1024), lim), lds_w + c * 1024);
    } else {
#pragma unroll
      for (int c = 0; c < kCopies; ++c)
        if (c + 1 < kCopies || kTail == 1024 || lane16 < (uint32_t)kTail)
          copy16_to_lds_nt((const void*)min(src + (uintptr_t)c * 1024 + (uintptr_t)lane16, last),
                           lds_w + c * 1024);
    }
  };
  if (has_rows && !late_wave) issue(set);

  if (stager) {
    // the activation copies, issued first, have landed (a late wave has requested no rows yet)
    wait_vmcnt(has_rows && !late_wave ? kCopies : 0);
    if constexpr (FUSEQ) {
      const int p = lane & 15;
      for (int r = wave; r < kRounds * M; r += nq) {
        const int m = r / kRounds, g = 4 * (r % kRounds) + (lane >> 4);
        float v[16];
        if (xbf16) {  // the values widened exactly
          const uint16_t* src = (const uint16_t*)xs + m * K + g * QK + 16 * p;
          const uint4 a = *(const uint4*)src, b = *(const uint4*)(src + 8);
          const uint32_t hv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            v[2 * i] = bf16_to_float(hv[i]);
            v[2 * i + 1] = bf16_to_float(hv[i] >> 16);
          }
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float4 f = *(const float4*)(xs + m * K + g * QK + 16 * p + 4 * q);
            v[4 * q] = f.x, v[4 * q + 1] = f.y, v[4 * q + 2] = f.z, v[4 * q + 3] = f.w;
          }
        }
        // the steps of q8k_part16, piece p of block g going to 16 (p NB + g)
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[i]));
        amax = max16(amax);
        int qv[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) qv[i] = 0;
        if (amax != 0.0f) {
          const float iscale = 127.0f / amax;
#pragma unroll
          for (int i = 0; i < 16; ++i) qv[i] = (int)fminf(fmaxf(rintf(v[i] * iscale), -127.0f), 127.0f);
        }
        uint32_t packed[4];
        int bsum = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          packed[i] = (uint32_t)(qv[4 * i] & 0xFF) | ((uint32_t)(qv[4 * i + 1] & 0xFF) << 8) |
                      ((uint32_t)(qv[4 * i + 2] & 0xFF) << 16) | ((uint32_t)(qv[4 * i + 3] & 0xFF) << 24);
          bsum += qv[4 * i] + qv[4 * i + 1] + qv[4 * i + 2] + qv[4 * i + 3];
        }
        *(uint4*)(act_q(m) + (p * NB + g) * 16) = uint4{packed[0], packed[1], packed[2], packed[3]};
        act_bs(m)[g * 16 + p] = (int16_t)bsum;
        if (p == 0) act_d(m)[g] = amax / 127.0f;
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS writes are done
    }
    if constexpr (kSums) {
      // sum j of block b: the pieces 4j .. 4j + 3 come from every stager's copies, so once all
      // have counted; each piece (x0 + x1) + (x2 + x3), then (p0 + p1) + (p2 + p3), the order of
      // the pipelined kernel's staging
      __builtin_amdgcn_wave_barrier();
      if (lane == 0) __hip_atomic_fetch_add(flag, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
      int sspin = 0;
      while (__hip_atomic_load(flag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < nq &&
             ++sspin < kWaveSpinLimit)
        __builtin_amdgcn_s_sleep(1);
      if (sspin >= kWaveSpinLimit) return;  // the compute waves then give up too (NaN)
      for (int r = wave * 64 + lane; r < M * NB * 16; r += nq * 64) {
        const int m = r / (NB * 16), bb = (r / 16) % NB, j = r % 16;
        const float* xr = (const float*)(smem + m * kXRow);
        float ps[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float4 v = *(const float4*)(xr + 4 * ((4 * j + i) * NB + bb));
          ps[i] = (v.x + v.y) + (v.z + v.w);
        }
        ((float*)(smem + m * kXRow + NB * 1024))[bb * 16 + j] = (ps[0] + ps[1]) + (ps[2] + ps[3]);
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the sums are written
    }
    __builtin_amdgcn_wave_barrier();
    if (lane == 0) __hip_atomic_fetch_add(flag, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
  }

  if (!has_rows) return;
  int spin = 0;
  const int staged = kSums ? 2 * nq : nq;  // the stagers count twice when they also sum
  while (__hip_atomic_load(flag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < staged &&
         ++spin < kWaveSpinLimit)
    __builtin_amdgcn_s_sleep(1);
  const bool gave_up = spin >= kWaveSpinLimit;
  if (late_wave) issue(set);  // the stagers are done with x

  const int b = lane % NB;
  ActPieces ap[MAXM];
  ActXPieces xp[MAXM];
#pragma unroll
  for (int m = 0; m < MAXM; ++m) {
    ap[m].q = (const int8_t*)(act_q(m) + b * 16);
    ap[m].stride = NB * 16;
    ap[m].bsums = act_bs(m) + b * 16;
    xp[m].x = (const float*)(smem + m * kXRow) + 4 * b;
    xp[m].stride = 4 * NB;
    xp[m].sums = (const float*)(smem + m * kXRow + NB * 1024) + 16 * b;
  }
  // fold lanes: lane l folds row l % R of the set against activation row l / R
  const int fr = lane % R, fm = lane / R;
  for (;;) {
    const int n0 = set * R;
    const int nrows = max(0, min(R, N - n0));
    const int jl = min(lane, max(nrows, 1) * NB - 1);  // lanes past the range redo its last block
    // the lane's activation block into registers while the set's copies land (again for every
    // set: held across sets, they crowd the compute into scratch)
    ActRegs areg;
    if constexpr (ACTREG) {
#pragma unroll
      for (int i = 0; i < 16; ++i) areg.q[i] = ap[0].q16(16 * i);
      areg.bs[0] = ap[0].bs8(0);
      areg.bs[1] = ap[0].bs8(1);
    }
    wait_vmcnt(0);
    float V[MAXM], D;
    if constexpr (kXF)
      L::template compute<MAXM, ActXPieces>(wreg, jl * L::kBytes, xp, M, V, D);
    else if constexpr (ACTREG)
      L::template compute<1, ActRegs>(wreg, jl * L::kBytes, &areg, 1, V, D);
    else
      L::template compute<MAXM, ActPieces>(wreg, jl * L::kBytes, ap, M, V, D);
    round0 += set_stride;
    const int next = round0 + wave * n_wg + tile;
#pragma unroll
    for (int m = 0; m < MAXM; ++m)
      if (m < M) Vbuf[64 * m + lane] = V[m];
    if (L::kHasD) Dbuf[lane] = D;
    __builtin_amdgcn_wave_barrier();
    if (fm < M && fr < nrows) {
      // blocks whose operands are read before they are folded (a divisor of NB)
      constexpr int kC = NB < 16 ? NB : NB % 16 == 0 ? 16 : 8;
      static_assert(NB % kC == 0, "fold chunks cover the row exactly");
      const float* xd = act_d(fm);
      float acc = 0.0f;
#pragma unroll
      for (int bb = 0; bb < NB; bb += kC) {
        float vv[kC], xx[kC], dd[kC];
#pragma unroll
        for (int i = 0; i < kC; ++i) {
          vv[i] = Vbuf[64 * fm + fr * NB + bb + i];
          xx[i] = kXF ? 0.0f : xd[bb + i];
          dd[i] = L::kHasD ? Dbuf[fr * NB + bb + i] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < kC; ++i) acc = L::fold(acc, xx[i], vv[i], dd[i]);
      }
      y.put((size_t)fm * ldy + n0 + fr, gave_up ? __builtin_nanf("") : acc);
    }
    if (!LOOP || next >= n_sets) break;
    // the next set into the stage once this one's reads have returned (issued after the fold:
    // issued between compute and fold, its addresses crowd the compute into scratch)
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();  // every lane's fold has read Vbuf before it is rewritten
    issue(next);
    set = next;
  }
}

// LOOP: waves may take more than one row set (a single pass compiles without the set loop)
template <int TYPE, int NB, bool FUSEQ, bool ACTREG, int MAXM, bool LOOP>
__global__ __launch_bounds__(64 * kWaveMaxWaves) void gemv_wave_kernel(
    const uint8_t* __restrict__ w, const float* __restrict__ x, YOut y, int N,
    int row_bytes, uint32_t pack, int ldy, const int8_t* __restrict__ aq,
    const float* __restrict__ ad, const int16_t* __restrict__ abs_) {
  wave_rows<TYPE, NB, FUSEQ, ACTREG, MAXM, LOOP>(w, x, y, N, row_bytes, pack & 0xFF, (pack >> 8) & 0xFF,
                                           (pack >> 16) & 0x7F, ldy, aq, ad, abs_, blockIdx.x,
                                           gridDim.x, (int)(pack >> 24), ((pack >> 23) & 1) != 0);
}

// Several weights that share the activation row (q|k|v, gate|up), one launch: each weight's
// workgroups follow the previous weight's, and a workgroup runs the single-weight form of its
// weight's block type.
constexpr int kWaveMaxSegs = 4;
struct WaveSeg {
  const uint8_t* w;
  YOut y;
  int n, row_bytes, type, wg0, waves, n_wg;
};
struct WaveSegs {
  WaveSeg s[kWaveMaxSegs];
  int count;
  int xbf16;  // x holds bfloat16 values
};

template <int NB, bool FUSEQ, bool LOOP>
__global__ __launch_bounds__(64 * kWaveMaxWaves) void gemv_wave_multi_kernel(
    WaveSegs segs, const float* __restrict__ x, int nq, const int8_t* __restrict__ aq,
    const float* __restrict__ ad, const int16_t* __restrict__ abs_) {
  int si = 0;
#pragma unroll
  for (int i = 1; i < kWaveMaxSegs; ++i)
    if (i < segs.count && (int)blockIdx.x >= segs.s[i].wg0) si = i;
  const WaveSeg& g = segs.s[si];
  const int wg = (int)blockIdx.x - g.wg0;
  if (g.type == T_Q4_K)
    wave_rows<T_Q4_K, NB, FUSEQ, true, 1, LOOP>(g.w, x, g.y, g.n, g.row_bytes, g.waves, nq, 1, 0, aq,
                                                ad, abs_, wg, g.n_wg, 0, segs.xbf16 != 0);
  else if (g.type == T_Q8_0)
    wave_rows<T_Q8_0, NB, FUSEQ, true, 1, LOOP>(g.w, x, g.y, g.n, g.row_bytes, g.waves, nq, 1, 0, aq,
                                                ad, abs_, wg, g.n_wg, 0, segs.xbf16 != 0);
  else
    wave_rows<T_Q6_K, NB, FUSEQ, false, 1, LOOP>(g.w, x, g.y, g.n, g.row_bytes, g.waves, nq, 1, 0,
                                                 aq, ad, abs_, wg, g.n_wg, 0, segs.xbf16 != 0);
}

// One token's routed experts (MoE decode): pair p multiplies expert ids[p] (a device array; an id
// outside [0, n_experts) is clamped, so a bad routing reads a valid expert, never past the
// weights) by activation row p * x_step (0: every pair shares the token's row). G workgroups per
// pair run the single-weight form.
template <int TYPE, int NB, bool FUSEQ, bool ACTREG, bool LOOP>
__global__ __launch_bounds__(64 * kWaveMaxWaves) void gemv_wave_pairs_kernel(
    const uint8_t* __restrict__ w, long long expert_stride, const int32_t* __restrict__ ids,
    int n_experts, const float* __restrict__ x, int x_step, YOut y, int N,
    int row_bytes, uint32_t pack, int G, const int8_t* __restrict__ aq,
    const float* __restrict__ ad, const int16_t* __restrict__ abs_) {
  constexpr int K = NB * QK;
  const int p = (int)blockIdx.x / G, wg = (int)blockIdx.x - p * G;
  const int e = min(max(ids[p], 0), n_experts - 1);
  const size_t r = (size_t)p * x_step;  // the pair's activation row
  const bool xbf16 = FUSEQ && ((pack >> 23) & 1) != 0;  // x holds bfloat16 values
  const float* xr = xbf16 ? (const float*)((const uint16_t*)x + r * K) : x + r * K;
  wave_rows<TYPE, NB, FUSEQ, ACTREG, 1, LOOP>(
      w + (size_t)e * expert_stride, FUSEQ ? xr : x, y.at((size_t)p * N), N, row_bytes,
      pack & 0xFF, (pack >> 8) & 0xFF, 1, 0, FUSEQ ? aq : aq + r * K, FUSEQ ? ad : ad + r * NB,
      FUSEQ ? abs_ : abs_ + r * NB * 16, wg, G, 0, xbf16);
}

template <int TYPE, int NB, bool FUSEQ, int MAXM>
int launch_wave_t(const uint8_t* w, long long row_bytes, const Act& act, YOut y, long long ldy,
                  int M, int N, hipStream_t stream) {
  constexpr bool kXF = ActTraits<TYPE>::kFloat, kSums = ActTraits<TYPE>::kSums;
  // activation registers: not for Q6_K (its compute leaves no room for them) or float x
  constexpr bool kReg = !kXF && TYPE != T_Q6_K && MAXM == 1;
  if (kXF && act.xbf16) return -1;  // float activations are staged as float32 only
  constexpr int R = 64 / NB;
  const int ncu = cu_count();
  const int per_cu = (int)(((long long)N + ncu - 1) / ncu);
  const int act_lds = kXF ? wave_xf_act_bytes(NB, M, kSums) : wave_act_bytes(NB, FUSEQ, M);
  const int region = wave_region_bytes<TYPE, NB, MAXM>();
  const int fit = (kWaveLds - act_lds) / region;
  // with x quantized in the kernel, further row waves in the fp32 x staging area (they request
  // their rows once x is quantized; 4096 x 14336 on MI355X: Q4_K 10.0 -> 8.95 us, Q6_K 14.9 ->
  // 12.9, Q8_0 15.6 -> 13.6, Q6_K 2048 x 14336 10.2 -> 8.7; Q6_K three rows 14336 x 4096 18.5 ->
  // 15.9). Only 56-block rows and Q6_K's three rows gain: on Q4_K two rows 14336 x 4096 went
  // from 8.5 to 10.4 us, elsewhere within 2%.
  const int late_fit =
      FUSEQ && !kXF && (NB == 56 || (TYPE == T_Q6_K && MAXM == 4)) ? (M * NB * 1024) / region : 0;
  const int waves = min(min(kWaveMaxWaves, fit + late_fit), (per_cu + R - 1) / R);
  const int late = max(0, waves - fit);
  // More rows than one round of workgroups holds: one workgroup per CU whose waves take further
  // row sets, each requested once the previous set is computed (measured on MI355X against the
  // pipelined kernel and against rounds of workgroups: Q4_K 28672 x 4096 14.8 vs 17.1 and 15.7
  // us, 128256 x 4096 47.3 vs 52.9 us pipelined; Q6_K 14336 x 4096 10.2 vs 13.7, the 128256 x 4096
  // head 71.5 vs 77.2, 8192 x 16384 27.9 vs 29.4; Q8_0 14336 x 4096 11.3 vs 13.1). 56-block rows
  // (K = 14336) with fp32 x staged in the kernel leave room for few weight waves (56 KB of x) and
  // still measured faster (4096 x 14336: Q4_K 10.0 vs 11.3 us, Q6_K 14.8 vs 15.4, Q8_0 15.6 vs
  // 15.8; Q6_K 6144 x 14336 18.8 vs 22.3); on workspace Q8_K more waves fit (Q4_K 8.9, Q6_K 13.1,
  // Q8_0 13.8 us).
  if (waves < 1 || ldy > 0x7FFFFFFF) return -1;
  constexpr int kSets = 64;  // row sets per wave at most
  const int grid = min((N + waves * R - 1) / (waves * R), ncu);
  if ((long long)waves * R * grid * kSets < N) return -1;
  // stagers: a round of four blocks each, in waves of their own when the workgroup has fewer
  // row waves (quantizing a round is ~140 VALU: four rounds on one wave cost ~1 us at N = 1024)
  const int nq = min(kWaveMaxWaves, M * NB / 4);
  const int nw = max(waves, nq);
  const int lds = act_lds + (waves - late) * region;  // row waves only
  auto kern = (long long)grid * waves * R < N ? gemv_wave_kernel<TYPE, NB, FUSEQ, kReg, MAXM, true>
                                              : gemv_wave_kernel<TYPE, NB, FUSEQ, kReg, MAXM, false>;
  allow_lds((const void*)kern, kWaveLds);
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * nw), lds, stream, w, act.x, y, N, (int)row_bytes,
                     (uint32_t)waves | (uint32_t)nq << 8 |
                         (uint32_t)(M | (FUSEQ && act.xbf16 ? 0x80 : 0)) << 16 | (uint32_t)late << 24,
                     (int)ldy, act.q,
                     act.d, act.bsums);
  return 0;
}

template <int TYPE, int NB, int MAXM>
int launch_wave_m(const uint8_t* w, long long row_bytes, const Act& act, YOut y, long long ldy,
                  int M, int N, hipStream_t stream) {
  if constexpr (ActTraits<TYPE>::kFloat)  // float activations, staged unquantized
    return act.q == nullptr ? launch_wave_t<TYPE, NB, false, MAXM>(w, row_bytes, act, y, ldy, M, N, stream)
                            : -1;
  else
    return act.q == nullptr
               ? launch_wave_t<TYPE, NB, true, MAXM>(w, row_bytes, act, y, ldy, M, N, stream)
               : launch_wave_t<TYPE, NB, false, MAXM>(w, row_bytes, act, y, ldy, M, N, stream);
}

// One activation row: every nb the kernel is built for. Two to four rows: 8-, 16- and 32-block
// rows, measured on MI355X against the pipelined kernel (same bits): two rows Q4_K 4096 x 4096 5.1
// vs 6.5 us, 14336 x 4096 8.5 vs 10.7, 28672 x 4096 13.4 vs 19.3; Q6_K 4096 x 4096 6.5 vs 7.9;
// Q8_0 6.6 vs 7.4. Three rows: Q4_K 4096 x 4096 6.5 vs 7.5, 14336 x 4096 12.0 vs 12.2, 28672 x
// 4096 18.4 vs 21.0; Q6_K 4096 x 4096 8.0 vs 8.9, 14336 x 4096 18.4 vs 19.8; Q8_0 7.9 vs 8.2.
// Four rows for Q4_K (14336 x 4096 13.7 vs 16.2 us; Q8_0 11.5 vs 9.0 and Q6_K 14336 x 4096
// 23.6 vs 22.1 stay pipelined). Float activations (IQ4_XS, the fp32-activation forms), two to
// four rows: Q4_K 14336 x 4096 16.9 / 24.6 / 31.2 vs 26.3 / 35.8 / 50.3 us, Q6_K 14336 x 4096
// 20.4 / 28 / 40 vs 28.7 / 38.8 / 58.9, IQ4_XS 14336 x 4096 22.8 / 27.7 / 37.8 vs 31.9 / 43.3 /
// 50.3; Q8_0 two rows only (4096 x 4096 10.8 vs 13.4; three rows 15.2 vs 14.5).
template <int TYPE, int NB>
int launch_wave_nb(const uint8_t* w, long long row_bytes, const Act& act, YOut y, long long ldy,
                   int M, int N, hipStream_t stream) {
  if (M == 1) return launch_wave_m<TYPE, NB, 1>(w, row_bytes, act, y, ldy, M, N, stream);
  if constexpr (NB == 8 || NB == 16 || NB == 32) {
    if (M == 2) return launch_wave_m<TYPE, NB, 2>(w, row_bytes, act, y, ldy, M, N, stream);
    if (TYPE != T_Q8_0_F && (M == 3 || (M == 4 && (TYPE == T_Q4_K || ActTraits<TYPE>::kFloat))))
      return launch_wave_m<TYPE, NB, 4>(w, row_bytes, act, y, ldy, M, N, stream);
  }
  return -1;
}

template <int TYPE>
int launch_wave_type(const uint8_t* w, long long row_bytes, const Act& act, YOut y,
                     long long ldy, int M, int N, hipStream_t stream) {
  switch (act.nb) {
    case 4: return launch_wave_nb<TYPE, 4>(w, row_bytes, act, y, ldy, M, N, stream);
    case 8: return launch_wave_nb<TYPE, 8>(w, row_bytes, act, y, ldy, M, N, stream);
    case 16: return launch_wave_nb<TYPE, 16>(w, row_bytes, act, y, ldy, M, N, stream);
    case 32: return launch_wave_nb<TYPE, 32>(w, row_bytes, act, y, ldy, M, N, stream);
    case 56: return launch_wave_nb<TYPE, 56>(w, row_bytes, act, y, ldy, M, N, stream);
    case 64: return launch_wave_nb<TYPE, 64>(w, row_bytes, act, y, ldy, M, N, stream);
    default: return -1;
  }
}

template <int NB>
int region_of(int type) {
  return type == T_Q4_K ? wave_region_bytes<T_Q4_K, NB>()
       : type == T_Q8_0 ? wave_region_bytes<T_Q8_0, NB>()
                        : wave_region_bytes<T_Q6_K, NB>();
}

// Each weight gets CUs in proportion to its bytes (at least one), one workgroup each, with as many
// row waves as spread its rows over them; a weight with more rows than one pass of its
// workgroups holds takes further row sets, as in the single-weight form.
template <int NB, bool FUSEQ>
int launch_wave_multi_t(const DecodeSeg* seg, int count, const Act& act, hipStream_t stream) {
  constexpr int R = 64 / NB;
  constexpr int kSets = 64;  // row sets per wave at most
  const int ncu = cu_count();
  const int act_lds = wave_act_bytes(NB, FUSEQ);
  double total = 0.0;
  for (int i = 0; i < count; ++i) total += (double)seg[i].n * (double)seg[i].row_bytes;
  // CU shares: rounded down, at least one, the CUs left over to the largest weights in turn
  int share[kWaveMaxSegs], used = 0;
  for (int i = 0; i < count; ++i) {
    share[i] = max(1, (int)((double)ncu * seg[i].n * seg[i].row_bytes / total));
    used += share[i];
  }
  for (int left = ncu - used; left > 0;) {
    int best = 0;
    for (int i = 1; i < count; ++i)
      if ((double)seg[i].n * seg[i].row_bytes / share[i] >
          (double)seg[best].n * seg[best].row_bytes / share[best])
        best = i;
    ++share[best];
    --left;
  }
  WaveSegs segs{};
  segs.count = count;
  segs.xbf16 = FUSEQ && act.xbf16 ? 1 : 0;
  int grid = 0, nw = min(kWaveMaxWaves, NB / 4), lds = act_lds;
  bool loop = false;
  for (int i = 0; i < count; ++i) {
    const int region = region_of<NB>(seg[i].type);
    const int fit = (kWaveLds - act_lds) / region;
    const int per_wg = (seg[i].n + share[i] - 1) / share[i];
    const int waves = min(min(kWaveMaxWaves, fit), (per_wg + R - 1) / R);
    if (waves < 1) return -1;
    const int wgs = min(share[i], (seg[i].n + waves * R - 1) / (waves * R));
    if ((long long)waves * R * wgs * kSets < seg[i].n) return -1;
    loop = loop || (long long)waves * R * wgs < seg[i].n;
    segs.s[i] = WaveSeg{seg[i].w, seg[i].y, seg[i].n, (int)seg[i].row_bytes, seg[i].type, grid,
                        waves, wgs};
    grid += wgs;
    nw = max(nw, waves);
    lds = max(lds, act_lds + waves * region);
  }
  if (grid > ncu) return -1;
  auto kern = loop ? gemv_wave_multi_kernel<NB, FUSEQ, true> : gemv_wave_multi_kernel<NB, FUSEQ, false>;
  allow_lds((const void*)kern, kWaveLds);
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * nw), lds, stream, segs, act.x,
                     min(kWaveMaxWaves, NB / 4), act.q, act.d, act.bsums);
  return 0;
}

template <int NB>
int launch_wave_multi_nb(const DecodeSeg* seg, int count, const Act& act, hipStream_t stream) {
  return act.q == nullptr ? launch_wave_multi_t<NB, true>(seg, count, act, stream)
                          : launch_wave_multi_t<NB, false>(seg, count, act, stream);
}

// n_pairs experts' weights of one token at once: the pairs share the CUs, G workgroups each.
template <int TYPE, int NB, bool FUSEQ>
int launch_pairs_t(const uint8_t* w, long long row_bytes, long long expert_stride,
                   const int32_t* ids, int n_experts, int n_pairs, int x_step, const Act& act,
                   YOut y, int N, hipStream_t stream) {
  constexpr bool kReg = TYPE != T_Q6_K;
  constexpr int R = 64 / NB;
  if constexpr (NB == 56 && FUSEQ && TYPE != T_Q4_K) return -1;
  const int ncu = cu_count();
  const int act_lds = wave_act_bytes(NB, FUSEQ, 1);
  const int region = wave_region_bytes<TYPE, NB, 1>();
  const int fit = (kWaveLds - act_lds) / region;
  const long long total = (long long)n_pairs * N;
  const int per_cu = (int)((total + ncu - 1) / ncu);
  const int waves = min(min(kWaveMaxWaves, fit), (per_cu + R - 1) / R);
  if (waves < 1) return -1;
  const int G = min((N + waves * R - 1) / (waves * R), max(1, ncu / n_pairs));
  constexpr int kSets = 64;
  if ((long long)waves * R * G * kSets < N || (long long)G * n_pairs > 0x7FFFFFFF) return -1;
  const int nq = min(kWaveMaxWaves, NB / 4);
  const int nw = max(waves, nq);
  const int lds = act_lds + waves * region;
  auto kern = (long long)G * waves * R < N ? gemv_wave_pairs_kernel<TYPE, NB, FUSEQ, kReg, true>
                                          : gemv_wave_pairs_kernel<TYPE, NB, FUSEQ, kReg, false>;
  allow_lds((const void*)kern, kWaveLds);
  hipLaunchKernelGGL(kern, dim3(G * n_pairs), dim3(64 * nw), lds, stream, w, expert_stride, ids,
                     n_experts, act.x, x_step, y, N, (int)row_bytes,
                     (uint32_t)waves | (uint32_t)nq << 8 | 1u << 16 | (FUSEQ && act.xbf16 ? 1u << 23 : 0u),
                     G, act.q, act.d, act.bsums);
  return 0;
}

template <int TYPE, int NB>
int launch_pairs_nb(const uint8_t* w, long long row_bytes, long long expert_stride,
                    const int32_t* ids, int n_experts, int n_pairs, int x_step, const Act& act,
                    YOut y, int N, hipStream_t stream) {
  return act.q == nullptr
             ? launch_pairs_t<TYPE, NB, true>(w, row_bytes, expert_stride, ids, n_experts, n_pairs,
                                              x_step, act, y, N, stream)
             : launch_pairs_t<TYPE, NB, false>(w, row_bytes, expert_stride, ids, n_experts, n_pairs,
                                               x_step, act, y, N, stream);
}

template <int TYPE>
int launch_pairs_type(const uint8_t* w, long long row_bytes, long long expert_stride,
                      const int32_t* ids, int n_experts, int n_pairs, int x_step, const Act& act,
                      YOut y, int N, hipStream_t stream) {
  switch (act.nb) {
#define MXA_PAIRS_NB(nb) \
  case nb: return launch_pairs_nb<TYPE, nb>(w, row_bytes, expert_stride, ids, n_experts, n_pairs, x_step, act, y, N, stream);
    MXA_PAIRS_NB(4)
    MXA_PAIRS_NB(8)
    MXA_PAIRS_NB(16)
    MXA_PAIRS_NB(32)
    MXA_PAIRS_NB(56)
    MXA_PAIRS_NB(64)
#undef MXA_PAIRS_NB
    default: return -1;
  }
}

}  // namespace

int launch_gemv_wave_m(int type, const uint8_t* w, long long row_bytes, const Act& act, YOut y,
                       long long ldy, int m_rows, int n_rows, hipStream_t stream) {
  if (n_rows < 1 || m_rows < 1 || m_rows > 4) return -1;
  if (((uintptr_t)w & 15) != 0 || row_bytes % 16 != 0 || row_bytes > 0x7FFFFFFF) return -1;
  // activations move in 16-byte pieces: fp32 x, or the Q8_K parts (q rows and bsums are 16-byte
  // multiples, d is 256-byte aligned in the workspace layout)
  if (act.q == nullptr ? ((uintptr_t)act.x & 15) != 0
                       : (((uintptr_t)act.q | (uintptr_t)act.bsums | (uintptr_t)act.d) & 15) != 0)
    return -1;
  switch (type) {
    case T_Q4_K: return launch_wave_type<T_Q4_K>(w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
    case T_Q8_0: return launch_wave_type<T_Q8_0>(w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
    case T_Q6_K: return launch_wave_type<T_Q6_K>(w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
    case T_IQ4_XS:
      // float activations; below ~4 MB of weight the resident kernel is faster (one row)
      // (measured on MI355X, the same bits: 14336 x 4096 12.9 vs 17.7 us, 4096 x 14336 15.7 vs
      // 24.5, the 128256 x 4096 head 79.3 vs 92, 4096 x 4096 6.5 vs 7.1; 1024 x 4096 4.9 vs 4.7)
      if ((long long)n_rows * row_bytes < kWaveIq4MinBytes) return -1;
      return launch_wave_type<T_IQ4_XS>(w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
    default: return -1;
  }
}

int launch_gemv_wave_f32(int type, const uint8_t* w, long long row_bytes, const Act& act, YOut y,
                         long long ldy, int m_rows, int n_rows, hipStream_t stream) {
  if (n_rows < 1 || m_rows < 1 || m_rows > 4 || act.q != nullptr || act.xbf16 ||
      ((uintptr_t)act.x & 15) != 0)
    return -1;
  if (((uintptr_t)w & 15) != 0 || row_bytes % 16 != 0 || row_bytes > 0x7FFFFFFF) return -1;
  switch (type) {
    case T_Q4_K: return launch_wave_type<T_Q4_K_F>(w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
    case T_Q6_K: return launch_wave_type<T_Q6_K_F>(w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
    case T_Q8_0: return launch_wave_type<T_Q8_0_F>(w, row_bytes, act, y, ldy, m_rows, n_rows, stream);
    default: return -1;
  }
}

int launch_gemv_wave(int type, const uint8_t* w, long long row_bytes, const Act& act, YOut y,
                     int n_rows, hipStream_t stream) {
  return launch_gemv_wave_m(type, w, row_bytes, act, y, n_rows, 1, n_rows, stream);
}

int launch_gemv_wave_multi(const DecodeSeg* seg, int count, const Act& act, hipStream_t stream) {
  if (count < 1 || count > kWaveMaxSegs) return -1;
  for (int i = 0; i < count; ++i) {
    const int t = seg[i].type;
    if ((t != T_Q4_K && t != T_Q6_K && t != T_Q8_0) || seg[i].n < 1 ||
        ((uintptr_t)seg[i].w & 15) != 0 || seg[i].row_bytes % 16 != 0 ||
        seg[i].row_bytes > 0x7FFFFFFF)
      return -1;
  }
  if (act.q == nullptr ? ((uintptr_t)act.x & 15) != 0
                       : (((uintptr_t)act.q | (uintptr_t)act.bsums | (uintptr_t)act.d) & 15) != 0)
    return -1;
  switch (act.nb) {
    case 4: return launch_wave_multi_nb<4>(seg, count, act, stream);
    case 8: return launch_wave_multi_nb<8>(seg, count, act, stream);
    case 16: return launch_wave_multi_nb<16>(seg, count, act, stream);
    case 32: return launch_wave_multi_nb<32>(seg, count, act, stream);
    default: return -1;
  }
}

int launch_gemv_wave_pairs(int type, const uint8_t* w, long long row_bytes, long long expert_stride,
                           const int32_t* ids, int n_experts, int n_pairs, int x_step,
                           const Act& act, YOut y, int n_rows, hipStream_t stream) {
  if (n_rows < 1 || n_pairs < 1 || n_experts < 1 || ids == nullptr || (x_step != 0 && x_step != 1) ||
      (act.xbf16 && act.q != nullptr))
    return -1;
  if (((uintptr_t)w & 15) != 0 || row_bytes % 16 != 0 || row_bytes > 0x7FFFFFFF ||
      expert_stride % 16 != 0 || expert_stride < (long long)n_rows * row_bytes)
    return -1;
  if (act.q == nullptr ? ((uintptr_t)act.x & 15) != 0
                       : (((uintptr_t)act.q | (uintptr_t)act.bsums | (uintptr_t)act.d) & 15) != 0)
    return -1;
  switch (type) {
    case T_Q4_K: return launch_pairs_type<T_Q4_K>(w, row_bytes, expert_stride, ids, n_experts, n_pairs, x_step, act, y, n_rows, stream);
    case T_Q8_0: return launch_pairs_type<T_Q8_0>(w, row_bytes, expert_stride, ids, n_experts, n_pairs, x_step, act, y, n_rows, stream);
    case T_Q6_K: return launch_pairs_type<T_Q6_K>(w, row_bytes, expert_stride, ids, n_experts, n_pairs, x_step, act, y, n_rows, stream);
    default: return -1;
  }
}

}  // namespace mxa
