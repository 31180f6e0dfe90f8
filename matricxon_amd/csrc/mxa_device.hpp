// Device-side building blocks shared by the kernels: GGUF block field decoding, cross-lane
// reductions inside a quad of lanes, dword-aligned loads, and the activation descriptor.
// Everything here is written for gfx950 (CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mxa {

constexpr int QK = 256;  // elements per super-block (and per Q8_K activation block)

enum GgmlType : int { T_Q8_0 = 8, T_Q4_K = 12, T_Q6_K = 14, T_IQ4_XS = 23 };

// 16 bytes from a 4-byte aligned address: gfx950 global loads only need dword alignment, so
// this is one global_load_dwordx4.
typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef int32_t i32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x2a4 __attribute__((ext_vector_type(2), aligned(4)));

__device__ __forceinline__ u32x4a4 ld16(const uint8_t* p) { return *(const u32x4a4*)p; }
__device__ __forceinline__ i32x4a4 ld16s(const int8_t* p) { return *(const i32x4a4*)p; }
__device__ __forceinline__ u32x2a4 ld8(const uint8_t* p) { return *(const u32x2a4*)p; }
__device__ __forceinline__ uint32_t ld4(const uint8_t* p) { return *(const uint32_t*)p; }

// Non-temporal 16-byte load for weight bytes that are read exactly once per call.
__device__ __forceinline__ u32x4a4 ld16_stream(const uint8_t* p) {
  return __builtin_nontemporal_load((const u32x4a4*)p);
}

// IEEE half (low 16 bits of h) to float. v_cvt_f32_f16 widens exactly; f16 subnormals become
// normal floats (f16/f64 denormals are preserved in the default kernel mode).
__device__ __forceinline__ float half_to_float(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(h & 0xFFFFu));
}

// Quad (4-lane) butterflies through DPP: lane ^ 1 and lane ^ 2.
__device__ __forceinline__ int quad_xor1(int v) {
  return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
}
__device__ __forceinline__ int quad_xor2(int v) {
  return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
}
__device__ __forceinline__ int quad_sum(int v) {
  v += quad_xor1(v);
  return v + quad_xor2(v);
}
__device__ __forceinline__ float quad_sum(float v) {
  v += __builtin_bit_cast(float, quad_xor1(__builtin_bit_cast(int, v)));
  return v + __builtin_bit_cast(float, quad_xor2(__builtin_bit_cast(int, v)));
}
// Maximum over the 16 lanes of a DPP row (lanes 16r..16r+15): quad butterflies, then the
// half-row and row mirrors. fmaxf ignores a NaN operand.
__device__ __forceinline__ float max16(float v) {
#define MXA_DPP_MAX(ctrl) \
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), ctrl, 0xF, 0xF, false)))
  MXA_DPP_MAX(0xB1);
  MXA_DPP_MAX(0x4E);
  MXA_DPP_MAX(0x141);
  MXA_DPP_MAX(0x140);
#undef MXA_DPP_MAX
  return v;
}

// Value of lane (quad base + i) broadcast to the whole quad.
template <int I>
__device__ __forceinline__ int quad_bcast(int v) {
  return __builtin_amdgcn_update_dpp(0, v, I | (I << 2) | (I << 4) | (I << 6), 0xF, 0xF, false);
}
template <int I>
__device__ __forceinline__ float quad_bcast(float v) {
  return __builtin_bit_cast(float, quad_bcast<I>(__builtin_bit_cast(int, v)));
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int acc) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, acc, false);
}

// The 16 six-bit scales and mins of a Q4_K block as bytes of four words (scales 0-3, mins 0-3,
// scales 4-7, mins 4-7) from the three words of its 12-byte field. Pairs 0-3 are the low six
// bits of bytes j / j+4; pairs 4-7 are byte j+8's low / high nibble plus the top two bits of
// byte j / j+4 (app/gguf/dequant/kquants.py:10-23).
struct K4Scales {
  uint32_t sc_lo, mn_lo, sc_hi, mn_hi;
};
__device__ __forceinline__ K4Scales k4_scales(uint32_t w0, uint32_t w1, uint32_t w2) {
  K4Scales s;
  s.sc_lo = w0 & 0x3F3F3F3Fu;
  s.mn_lo = w1 & 0x3F3F3F3Fu;
  s.sc_hi = (w2 & 0x0F0F0F0Fu) | ((w0 >> 2) & 0x30303030u);
  s.mn_hi = ((w2 >> 4) & 0x0F0F0F0Fu) | ((w1 >> 2) & 0x30303030u);
  return s;
}
// Byte k (0..7) of the scale (or min) vector.
__device__ __forceinline__ uint32_t k4_pick(uint32_t lo, uint32_t hi, int k) {
  return ((k < 4 ? lo : hi) >> (8 * (k & 3))) & 0xFFu;
}

// Q6_K: the unsigned 6-bit codes u = q + 32 of four consecutive elements of group g (0..3), as
// bytes, from a dword of ql (low nibbles for g = 0/1, high for g = 2/3) and the matching dword
// of qh (bits 2g..2g+1), per app/gguf/dequant/kquants.py:144-147.
template <int G>
__device__ __forceinline__ uint32_t q6_codes(uint32_t ql, uint32_t qh) {
  const uint32_t nib = (G < 2) ? (ql & 0x0F0F0F0Fu) : ((ql >> 4) & 0x0F0F0F0Fu);
  const uint32_t hb = (G == 0)   ? (qh << 4)
                      : (G == 1) ? (qh << 2)
                      : (G == 2) ? qh
                                 : (qh >> 2);
  return nib | (hb & 0x30303030u);
}

// IQ4_NL grid (app/gguf/dequant/iq_ternary.py:18-21) packed as signed bytes, four per word.
__device__ __forceinline__ uint32_t iq4_grid_word(int w) {
  // -127,-104,-83,-65 | -49,-35,-22,-10 | 1,13,25,38 | 53,69,89,113
  constexpr uint32_t W0 = 0xBFAD9881u, W1 = 0xF6EADDCFu, W2 = 0x26190D01u, W3 = 0x71594535u;
  return w == 0 ? W0 : w == 1 ? W1 : w == 2 ? W2 : W3;
}
// Four grid values (signed bytes) for the four 4-bit indices held in the low nibbles of the
// bytes of `idx` (high nibbles must be zero).
__device__ __forceinline__ uint32_t iq4_lookup4(uint32_t idx) {
  const uint32_t sel = idx & 0x07070707u;
  const uint32_t lo = __builtin_amdgcn_perm(iq4_grid_word(1), iq4_grid_word(0), sel);
  const uint32_t hi = __builtin_amdgcn_perm(iq4_grid_word(3), iq4_grid_word(2), sel);
  // byte mask 0xFF where index bit 3 is set: perm selector 0x0c gives 0x00, 0x0d gives 0xFF.
  const uint32_t msel = ((idx >> 3) & 0x01010101u) | 0x0C0C0C0Cu;
  const uint32_t mask = __builtin_amdgcn_perm(0u, 0u, msel);
  return (hi & mask) | (lo & ~mask);
}

// Signed byte k of w as float.
template <int K>
__device__ __forceinline__ float sbyte_f(uint32_t w) {
  return (float)(int8_t)(uint8_t)(w >> (8 * K));
}

// ------------------------------------------------------------------ bfloat16 activations / outputs
// float -> bfloat16, round to nearest even; a NaN becomes the quiet NaN 0x7FC0 (torch's cast,
// c10::detail::round_to_nearest_even).
__host__ __device__ __forceinline__ uint16_t bf16_rne(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
// bfloat16 (low 16 bits of h) -> float, exact.
__device__ __forceinline__ float bf16_to_float(uint32_t h) {
  return __builtin_bit_cast(float, (h & 0xFFFFu) << 16);
}

// The output rows of a matmul: float32, or bfloat16 (each value rounded as bf16_rne), one
// pointer-sized kernel argument. The element type rides in bit 0 of the address (outputs are at
// least 2-byte aligned); at() keeps it, so offsets count elements of either type.
struct YOut {
  uintptr_t v;
  __host__ __device__ static YOut f32(float* p) { return YOut{(uintptr_t)p}; }
  __host__ __device__ static YOut bf16(void* p) { return YOut{(uintptr_t)p | 1u}; }
  __host__ __device__ bool is_bf16() const { return (v & 1u) != 0; }
  __host__ __device__ YOut at(long long i) const {
    return YOut{v + (uintptr_t)(i * (is_bf16() ? 2 : 4))};
  }
  // Global-memory stores (an address that went through an integer would otherwise become a flat
  // store, which also counts on lgkmcnt: every later LDS wait would then wait for the store).
  __device__ __forceinline__ void put(long long i, float x) const {
    if (v & 1u)
      ((__attribute__((address_space(1))) uint16_t*)(v - 1))[i] = bf16_rne(x);
    else
      ((__attribute__((address_space(1))) float*)v)[i] = x;
  }
};

// Q8_K activations on the device, as produced by the quantize kernel: q (M, K) int8 row-major,
// d (M, nb) float, bsums (M, nb, 16) int16. `x` is the raw float (M, K) input (IQ4_XS reads it).
struct Act {
  const int8_t* q;
  const float* d;
  const int16_t* bsums;
  const float* x;
  int k;
  int nb;
  void* xsplit;  // IQ4_XS prefill: workspace for the bf16 split of x (nullptr when not provided)
  int xbf16;     // x holds bfloat16 values (only the kernels that quantize x themselves take it)
};

// ------------------------------------------------------------------ LDS copies and their waits
// A weight wave streams packed bytes into LDS with global_load_lds_dwordx4 and waits for them
// with its own s_waitcnt: copies complete in issue order, so "the copies of stage s have landed"
// is "at most n copies are outstanding", n being the copies issued after stage s.

typedef __attribute__((address_space(3))) uint8_t lds_u8;

// LDS byte address of a pointer into shared memory.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const lds_u8*)p;
}

// s_waitcnt vmcnt(n) for a wave-uniform n in [0, 63]; lgkmcnt and expcnt are not waited for.
__device__ __forceinline__ void wait_vmcnt(int n) {
#define MXA_VM(k) \
  case k: __builtin_amdgcn_s_waitcnt(((k) & 15) | (((k) >> 4) << 14) | 0x0F70); break;
#define MXA_VM8(k) MXA_VM(k) MXA_VM(k + 1) MXA_VM(k + 2) MXA_VM(k + 3) MXA_VM(k + 4) \
  MXA_VM(k + 5) MXA_VM(k + 6) MXA_VM(k + 7)
  switch (n) {
    MXA_VM8(0) MXA_VM8(8) MXA_VM8(16) MXA_VM8(24) MXA_VM8(32) MXA_VM8(40) MXA_VM8(48) MXA_VM8(56)
    default: __builtin_amdgcn_s_waitcnt(0x0F70); break;
  }
#undef MXA_VM8
#undef MXA_VM
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
}

constexpr int kMaxCopies = 63;  // the largest vmcnt: copies a weight wave may have outstanding

// global_load_lds_dwordx4: 16 bytes per lane from `g` to LDS byte address m0 + 16 * lane. Issued
// as inline assembly so that the compiler's own wait insertion does not see it (it would add
// vmcnt(0) before unrelated instructions); the kernel waits for these copies itself.
__device__ __forceinline__ void copy16_to_lds(const void* g, uint32_t lds_addr) {
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(lds_addr) : "memory");
}
// The same with the non-temporal cache policy: for bytes read exactly once per launch, so that the
// stream does not evict from the caches what the launch reads again (its own code, the
// activations).
__device__ __forceinline__ void copy16_to_lds_nt(const void* g, uint32_t lds_addr) {
  asm volatile("global_load_lds_dwordx4 %0, off nt" ::"v"(g), "{m0}"(lds_addr) : "memory");
}
// The same from a wave-uniform base plus a 32-bit per-lane byte offset (no 64-bit address math).
__device__ __forceinline__ void copy16_to_lds_s(const void* base, uint32_t off, uint32_t lds_addr) {
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "{m0}"(lds_addr) : "memory");
}
__device__ __forceinline__ void copy16_to_lds_s_nt(const void* base, uint32_t off, uint32_t lds_addr) {
  asm volatile("global_load_lds_dwordx4 %0, %1 nt" ::"v"(off), "s"(base), "{m0}"(lds_addr) : "memory");
}

// Grid-order tile index for workgroup `wg` of `n_wg` such that consecutive tiles land on the same
// XCD: workgroups are dealt to the 8 XCDs round-robin, so XCD x gets a contiguous tile range.
__device__ __forceinline__ int xcd_tile(int wg, int n_wg) {
  constexpr int kXcd = 8;
  const int q = n_wg / kXcd, r = n_wg % kXcd;
  const int x = wg % kXcd, k = wg / kXcd;
  return x * q + (x < r ? x : r) + k;
}

// Item `item` of a grouped MoE launch's (expert, chunk) work list: the rows [offsets[e],
// offsets[e + 1]) of expert e (clamped into [0, total_rows)) cut into chunks of `rows`, experts in
// order. One wave-wide prefix sum locates it (lane l counts the chunks of experts 4 l .. 4 l + 3,
// so n_experts <= 256): its expert e, first row p0 and row count m (1 .. rows). False past the
// list's end. Every lane of the wave must call it; the results are uniform over the wave.
__device__ __forceinline__ bool moe_chunk_item(const int32_t* __restrict__ offsets, int n_experts,
                                               int total_rows, int rows, int item, int& e,
                                               int& p0, int& m) {
  const int lane = threadIdx.x & 63;
  auto span = [&](int x, int& b, int& en) {
    b = min(max(offsets[x], 0), total_rows);
    en = min(max(offsets[x + 1], b), total_rows);
  };
  int cnt[4], lane_sum = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int x = 4 * lane + j;
    int c = 0;
    if (x < n_experts) {
      int b, en;
      span(x, b, en);
      c = (en - b + rows - 1) / rows;
    }
    cnt[j] = c;
    lane_sum += c;
  }
  int incl = lane_sum;  // inclusive prefix over the lanes
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int v = __shfl_up(incl, off, 64);
    if (lane >= off) incl += v;
  }
  const bool mine = item >= incl - lane_sum && item < incl;
  const uint64_t owner_mask = __ballot(mine);
  if (owner_mask == 0) return false;
  int e_sel = 0, c_sel = 0;
  if (mine) {
    int r = item - (incl - lane_sum);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (r >= 0 && r < cnt[j]) e_sel = 4 * lane + j, c_sel = r;
      r -= cnt[j];
    }
  }
  const int owner = __builtin_ctzll(owner_mask);
  e = __builtin_amdgcn_readlane(e_sel, owner);
  const int c = __builtin_amdgcn_readlane(c_sel, owner);
  int begin, end;
  span(e, begin, end);
  p0 = begin + rows * c;
  m = min(rows, end - p0);
  return true;
}

}  // namespace mxa
