// kaon_device.h -- gfx950 device helpers shared by the optimizer-step kernels.
//
// Every helper reproduces one rounding step of the reference's torch-CPU
// arithmetic (K-Optimizers "kaon" 0.7.4) so the HIP step is bit-exact with the
// CPU restatement under oracle/.  The whole library is compiled with
// -ffp-contract=off: only the explicit __fmaf_rn calls below fuse.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kaon_amd.h"

#define KAON_WG 256          // threads per workgroup of every step kernel (4 wave64)
#define KAON_CHUNK 8         // elements per chunk: one 16-byte bf16 vector

namespace kaon {

// Global-memory view of a generic pointer.  Descriptor pointers are generic
// (they are read from the descriptor table), and accesses through generic
// pointers compile to flat_* instructions, which also count against lgkmcnt
// and so hold up waits on LDS and scalar loads; through this view they are
// global_* instructions.
#define KAON_G __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ KAON_G T* G(T* p) {
  return (KAON_G T*)p;
}
// vector types for 16- and 8-byte accesses through global views
typedef uint32_t ku4 __attribute__((ext_vector_type(4)));
typedef uint32_t ku2 __attribute__((ext_vector_type(2)));
typedef float kf4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------ bf16
__device__ __forceinline__ float bf2f(uint32_t h) { return __uint_as_float(h << 16); }

// fp32 -> bf16 round-to-nearest-even, NaN -> 0x7FC0 (c10::BFloat16 semantics).
__device__ __forceinline__ uint32_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return u >> 16;
}
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }

// ------------------------------------------------------------------ fp16
__device__ __forceinline__ float h2f(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }
// fp32 -> fp16 round-to-nearest-even (v_cvt_f16_f32 in the default rounding
// mode: overflow to inf, fp16 subnormals kept), NaN -> 0x7E00 with the sign
// (c10::Half semantics).
__device__ __forceinline__ uint32_t f2h(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return ((u >> 16) & 0x8000u) | 0x7E00u;
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}
__device__ __forceinline__ float rhf(float f) { return h2f(f2h(f)); }

// torch.lerp on CPU: self + w*(end-self) if |w| < 0.5 else end - (end-self)*(1-w),
// each as one fused multiply-add (ATen/native/Lerp.h:22-35).
__device__ __forceinline__ float klerp(float a, float b, float w) {
  const float d = b - a;
  return fabsf(w) < 0.5f ? __fmaf_rn(w, d, a) : __fmaf_rn(w - 1.0f, d, b);
}
// The same with the branch known at compile time (LO: |w| < 0.5); the caller
// picks LO once per launch from the uniform weight.
template <bool LO>
__device__ __forceinline__ float klerp_b(float a, float b, float w) {
  const float d = b - a;
  return LO ? __fmaf_rn(w, d, a) : __fmaf_rn(w - 1.0f, d, b);
}

// Correctly rounded a / b from a precomputed r = RN64(1/b).  The fp64 product
// has relative error < 2^-52 while an fp32 quotient of two fp32 values is at
// least 2^-49 (relative) away from every fp32 rounding midpoint it is not equal
// to, so rounding the fp64 product to fp32 gives RN32(a/b) for all finite
// inputs (exact quotients included); inf and NaN propagate as in IEEE division.
__device__ __forceinline__ float div_r64(float a, double r) { return (float)((double)a * r); }
__device__ __forceinline__ double rcp64(float b) { return 1.0 / (double)b; }
// A reciprocal for div_r64 without the IEEE division sequence, for finite
// normal b with 2^-126 <= |b| < 2^126: v_rcp_f64 and two Newton steps
// r' = r + r (1 - b r) leave r within a few 2^-53 of 1/b (relative), so the
// product's error stays far inside div_r64's 2^-49 margin and the quotient is
// RN32(a/b) as with RN64(1/b).
__device__ __forceinline__ double rcp64_nr(float b) {
  const double d = (double)b;
  double r = __builtin_amdgcn_rcp(d);
  double e = __builtin_fma(-d, r, 1.0);
  r = __builtin_fma(r, e, r);
  e = __builtin_fma(-d, r, 1.0);
  return __builtin_fma(r, e, r);
}

__device__ __forceinline__ float ksign(float x) { return x > 0.0f ? 1.0f : (x < 0.0f ? -1.0f : 0.0f); }

// An empty asm statement that reads v: the loads producing v complete here.
// Used where a value loaded before a loop or inside a uniform branch would
// otherwise make the compiler wait for every load in flight (prefetches
// included) at the first use after the merge.
__device__ __forceinline__ void settle(uint32_t v) { asm volatile("" : : "v"(v)); }
__device__ __forceinline__ void settle(float v) { asm volatile("" : : "v"(v)); }

// The same pointer, opaque to the optimizer: loads through it are not hoisted
// out of the enclosing loop (used where keeping a loop-invariant load's result
// live across iterations would cost more registers than loading it again).
template <class T>
__device__ __forceinline__ T* opaque(T* p) {
  uint64_t v = (uint64_t)p;
  asm volatile("" : "+s"(v));
  return (T*)v;
}

// ------------------------------------------------------------------ Philox
// Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11), published multipliers and
// Weyl increments.  SR noise: key = (seed lo32, step), counter = (chunk lo,
// chunk hi, tensor id, stream) with chunk = element / 8; the 8 elements of a
// chunk take the 8 16-bit halves of the output, low half first.
// a ^ b ^ c in one v_bitop3_b32 (truth table 0x96)
__device__ __forceinline__ uint32_t xor3(uint32_t a, uint32_t b, uint32_t c) {
  return __builtin_amdgcn_bitop3_b32(a, b, c, 0x96);
}

__device__ __forceinline__ void philox10(uint32_t c[4], uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint64_t p0 = (uint64_t)0xD2511F53u * c[0];
    const uint64_t p1 = (uint64_t)0xCD9E8D57u * c[2];
    const uint32_t n0 = xor3((uint32_t)(p1 >> 32), c[1], k0);
    const uint32_t n2 = xor3((uint32_t)(p0 >> 32), c[3], k1);
    c[1] = (uint32_t)p1;
    c[3] = (uint32_t)p0;
    c[0] = n0;
    c[2] = n2;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
}

// Noise words for the aligned chunk [e0, e0+8) (e0 % 8 == 0).
__device__ __forceinline__ void noise8(uint64_t seed, uint32_t step, uint32_t tid, uint32_t stream,
                                       int64_t e0, const uint16_t* inj, int cnt, uint32_t w[8]) {
  if (inj) {
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = i < cnt ? (uint32_t)G(inj)[e0 + i] : 0u;
    return;
  }
  const uint64_t ch = (uint64_t)e0 >> 3;
  uint32_t c[4] = {(uint32_t)ch, (uint32_t)(ch >> 32), tid, stream};
  philox10(c, (uint32_t)seed, step);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    w[2 * i] = c[i] & 0xFFFFu;
    w[2 * i + 1] = c[i] >> 16;
  }
}

// Noise word of one element (any alignment).
__device__ __forceinline__ uint32_t noise1(uint64_t seed, uint32_t step, uint32_t tid, uint32_t stream,
                                           int64_t e, const uint16_t* inj) {
  if (inj) return G(inj)[e];
  const uint64_t ch = (uint64_t)e >> 3;
  uint32_t c[4] = {(uint32_t)ch, (uint32_t)(ch >> 32), tid, stream};
  philox10(c, (uint32_t)seed, step);
  const int wi = (int)(e & 7);
  return (c[wi >> 1] >> ((wi & 1) * 16)) & 0xFFFFu;
}

// _add_stochastic_bf16_ bit trick: int32 add of the 16-bit noise, clear the
// low half; the cast to bf16 is then exact (NaN -> 0x7FC0).
// The same as a 32-bit word: the bf16 result in the high half, zeros below
// (so the word is also the fp32 value of the rounded bf16).
__device__ __forceinline__ uint32_t sr_word(float x, uint32_t noise) {
  const uint32_t b = (__float_as_uint(x) + noise) & 0xFFFF0000u;
  const float f = __uint_as_float(b);
  return f != f ? 0x7FC00000u : b;
}
__device__ __forceinline__ uint32_t sr_bf16(float x, uint32_t noise) { return sr_word(x, noise) >> 16; }

// Two words' high halves packed low-first into one word (v_perm_b32).
__device__ __forceinline__ uint32_t pack_hi16(uint32_t lo, uint32_t hi) {
  return __builtin_amdgcn_perm(hi, lo, 0x07060302u);
}

// ------------------------------------------------------------------ loads
// Chunk loads into fp32 (8 elements, `cnt` valid; vec = 16-byte vector path).
template <int DT>
__device__ __forceinline__ void ld8(const void* base, int64_t off, int cnt, bool vec, float o[8]) {
  if (DT == KAON_BF16) {
    const KAON_G uint16_t* b = G((const uint16_t*)base + off);
    if (vec) {
      const ku4 v = *(const KAON_G ku4*)b;
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        o[2 * i] = __uint_as_float(w[i] << 16);
        o[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = i < cnt ? bf2f(b[i]) : 0.0f;
    }
  } else if (DT == KAON_F16) {
    const KAON_G uint16_t* b = G((const uint16_t*)base + off);
    if (vec) {
      const ku4 v = *(const KAON_G ku4*)b;
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        o[2 * i] = h2f(w[i] & 0xFFFFu);
        o[2 * i + 1] = h2f(w[i] >> 16);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = i < cnt ? h2f(b[i]) : 0.0f;
    }
  } else {
    const KAON_G float* b = G((const float*)base + off);
    if (vec) {
      const kf4 v0 = *(const KAON_G kf4*)b;
      const kf4 v1 = *(const KAON_G kf4*)(b + 4);
      o[0] = v0.x; o[1] = v0.y; o[2] = v0.z; o[3] = v0.w;
      o[4] = v1.x; o[5] = v1.y; o[6] = v1.z; o[7] = v1.w;
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = i < cnt ? b[i] : 0.0f;
    }
  }
}

// Raw bf16 chunk (bits) load/store.
__device__ __forceinline__ void ld8_bits(const void* base, int64_t off, int cnt, bool vec, uint32_t o[8]) {
  const KAON_G uint16_t* b = G((const uint16_t*)base + off);
  if (vec) {
    const ku4 v = *(const KAON_G ku4*)b;
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = w[i] & 0xFFFFu;
      o[2 * i + 1] = w[i] >> 16;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = i < cnt ? (uint32_t)b[i] : 0u;
  }
}
__device__ __forceinline__ void st8_bits(void* base, int64_t off, int cnt, bool vec, const uint32_t o[8]) {
  KAON_G uint16_t* b = G((uint16_t*)base + off);
  if (vec) {
    ku4 v;
    v.x = (o[0] & 0xFFFFu) | (o[1] << 16);
    v.y = (o[2] & 0xFFFFu) | (o[3] << 16);
    v.z = (o[4] & 0xFFFFu) | (o[5] << 16);
    v.w = (o[6] & 0xFFFFu) | (o[7] << 16);
    *(KAON_G ku4*)b = v;
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (i < cnt) b[i] = (uint16_t)o[i];
  }
}
__device__ __forceinline__ void st8_f32(void* base, int64_t off, int cnt, bool vec, const float o[8]) {
  KAON_G float* b = G((float*)base + off);
  if (vec) {
    *(KAON_G kf4*)b = kf4{o[0], o[1], o[2], o[3]};
    *(KAON_G kf4*)(b + 4) = kf4{o[4], o[5], o[6], o[7]};
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (i < cnt) b[i] = o[i];
  }
}

// ------------------------------------------------------------------ reductions
// Canonical 64-lane sum (the oracle's CSUM): every lane has accumulated, in
// order, the elements of its chunks l, l+64, ...; the lane sums are then
// combined by an xor butterfly with offsets 32, 16, 8, 4, 2, 1: at each step
// every lane adds its partner's value (a + b == b + a bit for bit, so lanes l
// and l^o end each step holding the same value and all lanes end with the
// canonical sum).  The steps run on the VALU: v_permlane32_swap and
// v_permlane16_swap exchange the halves / rows for offsets 32 and 16; a row
// rotation by 8 is the xor-8 partner; a rotation by 4 reads lane (i +- 4) mod
// 16, which after the xor-8 step holds the xor-4 partner's value; quad
// permutes give offsets 2 and 1.  Call with all 64 lanes active.
__device__ __forceinline__ uint32_t dpp_ror8(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x128, 0xF, 0xF, false);
}
__device__ __forceinline__ uint32_t dpp_ror4(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x124, 0xF, 0xF, false);
}
__device__ __forceinline__ uint32_t dpp_xor2(uint32_t x) {  // quad_perm [2,3,0,1]
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x4E, 0xF, 0xF, false);
}
__device__ __forceinline__ uint32_t dpp_xor1(uint32_t x) {  // quad_perm [1,0,3,2]
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0xB1, 0xF, 0xF, false);
}

// Butterfly with a commutative combine: OP(a, partner) at offsets 32..1.
template <typename Op>
__device__ __forceinline__ uint32_t wave_butterfly(uint32_t a, Op op) {
  {
    const auto r = __builtin_amdgcn_permlane32_swap(a, a, false, false);
    a = op(r[0], r[1]);
  }
  {
    const auto r = __builtin_amdgcn_permlane16_swap(a, a, false, false);
    a = op(r[0], r[1]);
  }
  a = op(a, dpp_ror8(a));
  a = op(a, dpp_ror4(a));
  a = op(a, dpp_xor2(a));
  a = op(a, dpp_xor1(a));
  return __builtin_amdgcn_readfirstlane(a);
}

__device__ __forceinline__ float wave_csum(float a) {
  return __uint_as_float(wave_butterfly(__float_as_uint(a), [](uint32_t x, uint32_t y) {
    return __float_as_uint(__uint_as_float(x) + __uint_as_float(y));
  }));
}

__device__ __forceinline__ float wave_max(float a) {
  return __uint_as_float(wave_butterfly(__float_as_uint(a), [](uint32_t x, uint32_t y) {
    return __float_as_uint(fmaxf(__uint_as_float(x), __uint_as_float(y)));
  }));
}

__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t a) {
  return wave_butterfly(a, [](uint32_t x, uint32_t y) { return x + y; });
}

__device__ __forceinline__ float uniform_f(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, x)));
}

// Non-negative float max through its bit pattern (monotone for x >= 0).
__device__ __forceinline__ uint32_t fmax_bits(uint32_t a, float x) {
  const uint32_t b = __float_as_uint(x);
  return b > a ? b : a;
}

// Round two floats to bf16 (RNE) and back with the gfx950 conversion
// instruction.  Matches f2bf() for every non-NaN input (checked exhaustively
// on the device); a NaN stays NaN with an unspecified payload, so use it only
// for values that are never stored.
typedef __bf16 kaon_bf16x2 __attribute__((ext_vector_type(2)));
typedef float kaon_f32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void rbf2(float& a, float& b) {
  kaon_f32x2 v = {a, b};
  const uint32_t w = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, kaon_bf16x2));
  a = __uint_as_float(w << 16);
  b = __uint_as_float(w & 0xFFFF0000u);
}
// The same instruction as a packed pair: f2bf(a) | f2bf(b) << 16 for non-NaN
// inputs.  For intermediates whose NaN payload is never observed.
__device__ __forceinline__ uint32_t f2bf2(float a, float b) {
  kaon_f32x2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, kaon_bf16x2));
}

}  // namespace kaon
