// device_math.h -- exact-by-construction device numerics for the decode step.
//
// Every function here performs the same sequence of correctly rounded IEEE
// operations as its CPU restatement, so results are bit-identical.  The whole
// library is compiled with -ffp-contract=off; fused multiply-adds are written
// explicitly with __builtin_fmaf.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rstr {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// 2^k for k in [-126, 127], built from the exponent field.
__device__ __forceinline__ float pow2i(int k) { return __int_as_float((k + 127) << 23); }

// exp(x): Cody-Waite reduction by ln2 (hi/lo split), degree-7 Taylor series of
// e^r on |r| <= ln2/2, then scaling by 2^n in two exact steps (so results that
// land in the subnormal range round once).  Own implementation of the textbook
// method; the constants are ln2, log2(e) and 1/k! rounded to float.
__device__ __forceinline__ float dexp(float x) {
  if (x != x) return x;
  if (x > 0x1.62e43p+6f) return __builtin_inff();
  if (x < -0x1.9fe36ap+6f) return 0.0f;
  float n = __builtin_rintf(x * 0x1.715476p+0f);
  float r = __builtin_fmaf(-n, 0x1.62e4p-1f, x);
  r = __builtin_fmaf(-n, 0x1.7f7d1cp-20f, r);
  float p = 0x1.a01a02p-13f;
  p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
  p = __builtin_fmaf(p, r, 0x1.111112p-7f);
  p = __builtin_fmaf(p, r, 0x1.555556p-5f);
  p = __builtin_fmaf(p, r, 0x1.555556p-3f);
  p = __builtin_fmaf(p, r, 0x1.0p-1f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  int ni = (int)n;
  int n1 = ni / 2;
  int n2 = ni - n1;
  return (p * pow2i(n1)) * pow2i(n2);
}

// GELU in its tanh form, tanh(u) = 1 - 2/(e^{2u}+1).
__device__ __forceinline__ float dgelu(float g) {
  float g3 = (g * g) * g;
  float u = 0x1.988454p-1f * (g + 0x1.6e4e26p-5f * g3);
  float e = dexp(u + u);
  float t = 1.0f - 2.0f / (e + 1.0f);
  return (0.5f * g) * (1.0f + t);
}

__device__ __forceinline__ float dsilu(float g) { return g / (1.0f + dexp(-g)); }

// fp32 -> fp16 with round-to-nearest-even (v_cvt_f16_f32 in the default mode).
__device__ __forceinline__ uint16_t f2h_bits(float f) {
  _Float16 h = (_Float16)f;
  return __builtin_bit_cast(uint16_t, h);
}

// Activation block scale: RN(amax/127) rounded up to a 4-bit significand and
// kept in [2^-21, 480], so q*d is an exact fp16 value for every |q| <= 127
// (7 + 4 significant bits, at least 2^-24, at most 60960); 0 for amax 0.  The
// projection folds d into its integer block dot exactly.
__device__ __forceinline__ float act_scale(float amax) {
  if (!(amax > 0.0f)) return 0.0f;
  uint32_t b = __float_as_uint(amax / 127.0f);
  if (b & 0xFFFFFu) b = (b & ~0xFFFFFu) + 0x100000u;
  return fminf(fmaxf(__uint_as_float(b), 0x1p-21f), 480.0f);
}

// ---- counter-based synthetic weights --------------------------------------
#define RSTR_GOLDEN 0x9E3779B97F4A7C15ull
__host__ __device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  uint64_t z = x + RSTR_GOLDEN;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
__host__ __device__ __forceinline__ uint64_t tensor_key(uint64_t seed, int layer, int role) {
  uint64_t tag = ((uint64_t)(uint32_t)(layer + 1) << 16) | (uint64_t)(uint32_t)role;
  return splitmix64(splitmix64(seed) ^ tag);
}
// Irwin-Hall sum of twelve 16-bit uniforms: exact integer sum, exact double
// centring, one double multiply-add, one rounding to float.
__device__ __forceinline__ float synth_normal(uint64_t key, uint64_t index, double mean, double std) {
  uint64_t s = 0;
#pragma unroll
  for (int j = 0; j < 3; j++) {
    uint64_t r = splitmix64(key + (3u * index + (uint64_t)j) * RSTR_GOLDEN);
    s += (r & 0xFFFFu) + ((r >> 16) & 0xFFFFu) + ((r >> 32) & 0xFFFFu) + (r >> 48);
  }
  double v = ((double)s + 6.0) / 65536.0 - 6.0;
  return (float)(mean + std * v);
}

// Loads of data that a step reads exactly once (quantised weights and their
// scales): non-temporal, so their lines are the first to leave L2 and the
// activation tiles that every column tile re-reads stay resident.
template <class T>
__device__ __forceinline__ T ld_stream(const T* p) {
  return __builtin_nontemporal_load(p);
}

// ---- wavefront reductions ----------------------------------------------------
// lane exchange v[lane ^ M]: quad permutes for M < 4 (DPP), the swizzle
// unit inside 32-lane halves for M < 32, bpermute across halves.
template <int M>
__device__ __forceinline__ float xor_lane(float v) {
  if constexpr (M == 1)
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));
  else if constexpr (M == 2)
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true));
  else if constexpr (M < 32)
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x1F | (M << 10)));
  else
    return __shfl_xor(v, M, 64);
}

// v[lane'] where lane' mirrors lane inside its aligned 8-lane group
// (i -> 7 - i): one DPP row_half_mirror.
__device__ __forceinline__ float half_mirror_lane(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, true));
}

// v + v[lane ^ M] and max(v, v[lane ^ M]).  For M = 16 and 32 one gfx950
// lane swap (v_permlane16_swap / v_permlane32_swap, both operands copies of
// v) leaves the pair {v[lo], v[hi]} of lanes lo = min(i, i^M),
// hi = max(i, i^M) in both lanes, without the LDS crossbar; fp add and max
// commute, so every lane gets the bits of v + xor_lane<M>(v).  The swap is
// written in assembly: the compiler folds the builtin with two equal
// operands into an identity (both results v), which drops the exchange.
// Hazard checks do not see inside the statement, so it supplies the two wait
// states a swap needs after a VALU write of its operands (the padding the
// compiler emits before the builtin's swaps).
template <int M>
__device__ __forceinline__ void lane_pair(float v, float& lo, float& hi) {
  float a = v, b = v;
  if constexpr (M == 16)
    asm("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  else
    asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  lo = a;
  hi = b;
}
template <int M>
__device__ __forceinline__ float xor_add(float v) {
  if constexpr (M == 16 || M == 32) {
    float a, b;
    lane_pair<M>(v, a, b);
    return a + b;
  } else {
    return v + xor_lane<M>(v);
  }
}
template <int M>
__device__ __forceinline__ float xor_max(float v) {
  if constexpr (M == 16 || M == 32) {
    float a, b;
    lane_pair<M>(v, a, b);
    return fmaxf(a, b);
  } else {
    return fmaxf(v, xor_lane<M>(v));
  }
}

// xor butterfly: level m combines lanes i and i^m.  Because fp add commutes,
// both lanes hold the same value and the result is the balanced pairwise tree
// over lane order.
__device__ __forceinline__ float wave_tree_sum(float v) {
  v = xor_add<1>(v);
  v = xor_add<2>(v);
  v = xor_add<4>(v);
  v = xor_add<8>(v);
  v = xor_add<16>(v);
  return xor_add<32>(v);
}
__device__ __forceinline__ float wave_max(float v) {
  v = xor_max<1>(v);
  v = xor_max<2>(v);
  v = xor_max<4>(v);
  v = xor_max<8>(v);
  v = xor_max<16>(v);
  return xor_max<32>(v);
}

}  // namespace rstr
