// Shared device helpers for the flashgrpo_amd HIP kernels (gfx950 / CDNA4).
//
// bf16 storage is raw uint16_t; conversions use round-to-nearest-even, the
// rounding torch applies when it casts fp32 to bf16.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "fg_exp2_table.h"

#define FG_DEVICE __device__ __forceinline__

namespace fg {

enum Dtype : int { kF32 = 0, kBF16 = 1 };

// ------------------------------------------------------------------ errors
// Host-side error state (thread-local message, returned by fg_last_error).
void set_error(const std::string& msg);
int fail(const std::string& msg);          // sets the message, returns -1
int check_launch(const char* what);        // hipGetLastError -> code

#define FG_REQUIRE(cond, msg)              \
  do {                                     \
    if (!(cond)) return ::fg::fail(msg);   \
  } while (0)

inline int elem_bytes(int dtype) { return dtype == kBF16 ? 2 : 4; }

// ------------------------------------------------------------------ bf16
FG_DEVICE float bf16_to_f32(uint16_t u) { return __uint_as_float(((uint32_t)u) << 16); }

FG_DEVICE uint16_t f32_to_bf16(float f) {
  uint32_t b = __float_as_uint(f);
  if ((b & 0x7f800000u) == 0x7f800000u && (b & 0x007fffffu)) return (uint16_t)((b >> 16) | 0x40);
  b += 0x7fffu + ((b >> 16) & 1u);
  return (uint16_t)(b >> 16);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two floats to packed bf16 (lo = a, hi = b), round-to-nearest-even: one
// v_cvt_pk_bf16_f32 on gfx950. Equals f32_to_bf16 on finite inputs.
FG_DEVICE uint32_t pack_bf16x2(float a, float b) {
  f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// x rounded to the nearest bf16 (ties to even), as a float: one v_cvt_pk_bf16_f32 and a shift.
FG_DEVICE float round_bf16(float x) { return __uint_as_float(pack_bf16x2(x, 0.0f) << 16); }

// SiLU(x) = x / (1 + e^-x), the quotient taken as x times the hardware reciprocal
// (v_rcp_f32, 1 ulp) instead of the ten-instruction IEEE division: within 2 ulp of the
// correctly rounded value, so a bf16 rounding of it differs only next to a rounding tie.
FG_DEVICE float silu_f32(float x) { return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

template <int DT>
FG_DEVICE float load_elem(const void* p, int64_t i) {
  if constexpr (DT == kBF16)
    return bf16_to_f32(((const uint16_t*)p)[i]);
  else
    return ((const float*)p)[i];
}

template <int DT>
FG_DEVICE void store_elem(void* p, int64_t i, float v) {
  if constexpr (DT == kBF16)
    ((uint16_t*)p)[i] = f32_to_bf16(v);
  else
    ((float*)p)[i] = v;
}

// Load 8 consecutive elements starting at i (i a multiple of 8 and the row
// base 16-byte aligned for bf16 / 32-byte aligned for fp32).
template <int DT>
FG_DEVICE void load8(const void* p, int64_t i, float (&v)[8]) {
  if constexpr (DT == kBF16) {
    uint4 r = *(const uint4*)((const uint16_t*)p + i);
    uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[2 * j] = __uint_as_float(w[j] << 16);
      v[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
    }
  } else {
    float4 a = *(const float4*)((const float*)p + i);
    float4 b = *(const float4*)((const float*)p + i + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
}

template <int DT>
FG_DEVICE void store8(void* p, int64_t i, const float (&v)[8]) {
  if constexpr (DT == kBF16) {
    *(uint4*)((uint16_t*)p + i) = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                                             pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7]));
  } else {
    *(float4*)((float*)p + i) = make_float4(v[0], v[1], v[2], v[3]);
    *(float4*)((float*)p + i + 4) = make_float4(v[4], v[5], v[6], v[7]);
  }
}

// ------------------------------------------------------------------ ordering keys
// Order-preserving uint32 key of a float: -0 maps to +0's key and every NaN to
// the largest key, so (key desc, index asc) is a total order agreeing with <.
FG_DEVICE uint32_t sort_key32(float f) {
  if (f != f) return 0xffffffffu;
  if (f == 0.0f) return 0x80000000u;
  uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// Composite rank key: larger is better; unique per index.
FG_DEVICE uint64_t rank_key(float f, uint32_t idx) {
  return ((uint64_t)sort_key32(f) << 32) | (uint64_t)(0xffffffffu - idx);
}
FG_DEVICE uint32_t rank_key_index(uint64_t k) { return 0xffffffffu - (uint32_t)(k & 0xffffffffu); }
FG_DEVICE float rank_key_value(uint64_t k) {
  uint32_t key = (uint32_t)(k >> 32);
  uint32_t b = (key & 0x80000000u) ? (key & 0x7fffffffu) : ~key;
  return __uint_as_float(b);
}

// ------------------------------------------------------------------ sampling weight
// The integer weight of logit x in a row with maximum m (NaN ignored):
//   a = trunc(min((m - x) * kt, kWeightZmax))   fp32 ops, each rounded; kt = kWeightKt / T
//   q = floor(2^40 * 2^-(a / 2^20))             = 2^40 * exp(-(m - x) / T), 2^20 steps per octave
// evaluated as w = T[r] - (D[r] * f >> 10) for the table entry r = bits 10-19 of a (T[r] =
// round(2^31 * 2^(-r/1024)), D[r] = T[r] - T[r+1]) and the low bits f = bits 0-9, then
// q = (w << 32) >> (23 + (a >> 20)). x = m gives 2^40; -inf, NaN and anything 40 octaves
// below m give 0 (the clamp keeps the shift at most 63). tbl: kExp2Table staged in LDS.
FG_DEVICE uint64_t weight_q40(float m, float x, float kt, const uint64_t* tbl) {
#pragma clang fp contract(off)
  const float z = fminf((m - x) * kt, kWeightZmax);
  const uint32_t a = (uint32_t)z;
  const uint64_t e = tbl[(a >> 10) & 1023u];
  const uint32_t w = (uint32_t)e - (__umul24((uint32_t)(e >> 32), a & 1023u) >> 10);
  return ((uint64_t)w << 32) >> ((a >> 20) + 23u);
}

// kt for temperature T (> 0 divides, otherwise no scaling), correctly rounded.
FG_DEVICE float weight_kt(bool scale, float T) { return scale ? __fdiv_rn(kWeightKt, T) : kWeightKt; }

// Copies kExp2Table into LDS (every thread of the block takes part; a barrier must
// follow before the first weight_q40).
FG_DEVICE void exp2_table_to_lds(uint64_t* dst) {
  for (int i = threadIdx.x; i < 1024; i += blockDim.x) dst[i] = kExp2Table[i];
}

// floor(a * u / 2^32) for a < 2^64, u < 2^32.
FG_DEVICE uint64_t mulhi_u64_u32(uint64_t a, uint32_t u) {
  uint64_t hi = (a >> 32) * (uint64_t)u;
  uint64_t lo = ((a & 0xffffffffull) * (uint64_t)u) >> 32;
  return hi + lo;
}

// ------------------------------------------------------------------ counter noise
// SplitMix64 output finalizer (Steele, Lea, Flood 2014).
FG_DEVICE uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
// u32 noise keyed by (seed, step, sequence id, draw index).
FG_DEVICE uint32_t counter_noise(uint64_t seed, uint64_t step, uint32_t seq, uint32_t draw) {
  uint64_t key = ((step & 0xffffffffull) << 32) | ((uint64_t)(seq & 0xffffffu) << 8) | (draw & 0xffu);
  return (uint32_t)(mix64(mix64(seed + 0x9E3779B97F4A7C15ull) ^ key) >> 32);
}

// ------------------------------------------------------------------ wave reductions
FG_DEVICE float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
FG_DEVICE float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
FG_DEVICE uint64_t shfl_xor_u64(uint64_t v, int o) {
  uint32_t lo = __shfl_xor((unsigned)(v & 0xffffffffu), o, 64);
  uint32_t hi = __shfl_xor((unsigned)(v >> 32), o, 64);
  return ((uint64_t)hi << 32) | lo;
}
FG_DEVICE uint64_t shfl_up_u64(uint64_t v, int o) {
  uint32_t lo = __shfl_up((unsigned)(v & 0xffffffffu), o, 64);
  uint32_t hi = __shfl_up((unsigned)(v >> 32), o, 64);
  return ((uint64_t)hi << 32) | lo;
}
FG_DEVICE uint64_t shfl_u64(uint64_t v, int src) {
  uint32_t lo = __shfl((unsigned)(v & 0xffffffffu), src, 64);
  uint32_t hi = __shfl((unsigned)(v >> 32), src, 64);
  return ((uint64_t)hi << 32) | lo;
}
FG_DEVICE uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += shfl_xor_u64(v, o);
  return v;
}
FG_DEVICE uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    uint64_t w = shfl_xor_u64(v, o);
    v = w > v ? w : v;
  }
  return v;
}
// Inclusive prefix sum across the 64 lanes.
FG_DEVICE uint64_t wave_incl_scan_u64(uint64_t v) {
  int lane = threadIdx.x & 63;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    uint64_t w = shfl_up_u64(v, o);
    if (lane >= o) v += w;
  }
  return v;
}

}  // namespace fg
