// Shared device helpers for the gfx950 fake-quant kernels.
//
// * dtype codes and element load/store with round-to-nearest-even narrowing;
// * OCP E4M3FN encoding computed from the fp32 bits (RNE, saturating to
//   +-448), identical to the CPU oracle's codec;
// * error reporting for the C ABI (thread-local last-error string).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdio>
#include <cstring>

namespace lbfq {

enum DType : int { kF32 = 0, kF16 = 1, kBF16 = 2 };

constexpr float kFp8Max = 448.0f;
// fp32(1e-4): the reference's amax floor (quant_triton.py:10).
constexpr float kAmaxFloor = 1e-4f;

__host__ __device__ inline int dtype_size(int dt) { return dt == kF32 ? 4 : 2; }

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// fp32 -> bf16 with round-to-nearest-even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// fp32 -> fp16 with round-to-nearest-even (the default rounding mode).
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// Load element i of a tensor of dtype dt as fp32 (exact widening).
__device__ __forceinline__ float load_as_f32(const void* p, int64_t i, int dt) {
  if (dt == kBF16) return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
  if (dt == kF16) return f16_bits_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
  return reinterpret_cast<const float*>(p)[i];
}

// Round fp32 to dtype dt (RNE) and return the rounded value as fp32.
__device__ __forceinline__ float round_to_dtype(float v, int dt) {
  if (dt == kBF16) return bf16_bits_to_f32(f32_to_bf16_bits(v));
  if (dt == kF16) return f16_bits_to_f32(f32_to_f16_bits(v));
  return v;
}

// v as a materialised fp32 register value.  Before a narrowing to fp16 the
// compiler otherwise selects fptrunc(a * b) (and a +- b) as a mixed-precision
// FMA with a +0 addend: that rounds the exact result once instead of the
// fp32 result (a double-rounding difference at fp16 ties) and turns a -0
// product into +0.
__device__ __forceinline__ float as_f32(float v) {
  asm volatile("" : "+v"(v));
  return v;
}

__device__ __forceinline__ void store_from_f32(void* p, int64_t i, int dt, float v) {
  if (dt == kBF16) reinterpret_cast<uint16_t*>(p)[i] = f32_to_bf16_bits(v);
  else if (dt == kF16) reinterpret_cast<uint16_t*>(p)[i] = f32_to_f16_bits(v);
  else reinterpret_cast<float*>(p)[i] = v;
}

// OCP E4M3FN encode, round-to-nearest-even on the fp32 bits.  Finite values
// with |x| >= 448 saturate to +-448 (the reference clamps first, or uses a
// satfinite conversion); NaN maps to 0x7F.
__host__ __device__ __forceinline__ uint8_t e4m3_encode(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  uint32_t sign = (u >> 31) << 7;
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return 0x7f;
  if (a >= 0x43e00000u) return static_cast<uint8_t>(sign | 0x7e);
  if (a >= 0x3c800000u) {  // normal: 2^-6 <= |x| < 448
    int e = static_cast<int>(a >> 23) - 127;
    uint32_t mant = a & 0x7fffffu;
    uint32_t q = mant >> 20;
    uint32_t rem = mant & 0xfffffu;
    if (rem > 0x80000u || (rem == 0x80000u && (q & 1u))) ++q;
    if (q == 8u) { q = 0; ++e; }
    return static_cast<uint8_t>(sign | (static_cast<uint32_t>(e + 7) << 3) | q);
  }
  // subnormal: |x| * 2^9 rounded to an integer in [0, 8]
  uint32_t E = a >> 23;
  uint32_t M = E ? ((a & 0x7fffffu) | 0x800000u) : (a & 0x7fffffu);
  uint32_t Eeff = E ? E : 1u;
  uint32_t shift = 141u - Eeff;
  if (shift > 31u) return static_cast<uint8_t>(sign);
  uint32_t q = M >> shift;
  uint32_t dropped = M - (q << shift);
  uint32_t half = 1u << (shift - 1u);
  if (dropped > half || (dropped == half && (q & 1u))) ++q;
  return static_cast<uint8_t>(sign | q);
}

__host__ __device__ __forceinline__ float e4m3_decode(uint8_t c) {
  uint32_t s = c >> 7, e = (c >> 3) & 0xf, m = c & 7;
  float v;
  if (e == 0) v = static_cast<float>(m) * (1.0f / 512.0f);
  else v = (1.0f + static_cast<float>(m) * 0.125f) * ldexpf(1.0f, static_cast<int>(e) - 7);
  return s ? -v : v;
}

// Quantise one value with scale sc exactly as the reference does:
// e4m3(clamp(x / sc, -448, 448)) with an IEEE fp32 division.
__device__ __forceinline__ uint8_t quant_e4m3(float x, float sc) {
  float q = x / sc;
  q = fminf(fmaxf(q, -kFp8Max), kFp8Max);
  return e4m3_encode(q);
}

// x / s for a fixed divisor s > 0 with r = 1/s (correctly rounded, computed
// once): one product and one FMA correction of its residual (Markstein).  The
// result is the correctly rounded quotient -- the reference's IEEE x / s --
// for every quotient of magnitude >= 2^-12; smaller ones encode to E4M3 zero
// either way, whose sign (code 0x80 for a negative quotient) is x's: the
// correction turns a -0 product into +0, so the sign is taken from x.
// (Checked against IEEE division over ~2e10 cases; a reduced sweep is a CPU test.)
__device__ __forceinline__ float div_by(float x, float s, float r) {
  const float q = x * r;
  return __builtin_copysignf(fmaf(fmaf(-q, s, x), r, q), x);
}

// Encode q / sc (|q / sc| <= 448 after the clamp) with the hardware RNE
// converter; its agreement with the reference encoder over every code,
// midpoint, neighbour of a midpoint and the subnormal range is a GPU test.
__device__ __forceinline__ uint32_t cvt4_e4m3(const float q[4]) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], w, true);
  return static_cast<uint32_t>(w);
}

__device__ __forceinline__ float clamp448(float q) { return __builtin_amdgcn_fmed3f(q, -kFp8Max, kFp8Max); }

// ceil(log2(r)) for positive normal fp32 r, exact from the bits.
__device__ __forceinline__ int ceil_log2_exact(float r) {
  uint32_t u = __float_as_uint(r);
  int e = static_cast<int>(u >> 23) - 127;
  return e + ((u & 0x7fffffu) != 0u ? 1 : 0);
}

// ceil(log2(r / 448)) for positive normal fp32 r, with the quotient rounded
// as an IEEE fp32 division would round it, from r's bits: 448 = 1.75 * 2^8,
// so with r = (1 + f) 2^E the quotient lies in (2^(E-9), 2^(E-8)] when
// 1 + f <= 1.75 and in (2^(E-8), 2^(E-7)) otherwise; a quotient within half
// an ulp of a power of two only arises from 1 + f = 1.75 exactly (then it is
// that power) or from the float next to it (then it rounds away from it).
__device__ __forceinline__ int ceil_log2_div448(float r) {
  const uint32_t u = __float_as_uint(r);
  return static_cast<int>(u >> 23) - 127 - 8 + ((u & 0x7fffffu) > 0x600000u ? 1 : 0);
}

// Power-of-two MX scale 2^clamp(ceil(log2(amax/448)), -127, 127) as fp32.
__device__ __forceinline__ float mx_scale_from_amax(float amax) {
  float r = amax / kFp8Max;
  int e = ceil_log2_exact(r);
  e = e < -127 ? -127 : (e > 127 ? 127 : e);
  return ldexpf(1.0f, e);
}

}  // namespace lbfq

// ---- C-ABI error plumbing -------------------------------------------------
extern "C" const char* lbfq_last_error(void);
void lbfq_set_error(const char* fmt, ...);

#define LBFQ_CHECK_ARG(cond, ...)      \
  do {                                 \
    if (!(cond)) {                     \
      lbfq_set_error(__VA_ARGS__);     \
      return -1;                       \
    }                                  \
  } while (0)

#define LBFQ_LAUNCH_CHECK(name)                                                   \
  do {                                                                            \
    hipError_t _e = hipGetLastError();                                            \
    if (_e != hipSuccess) {                                                       \
      lbfq_set_error("%s: launch failed: %s", name, hipGetErrorString(_e));       \
      return -2;                                                                  \
    }                                                                             \
  } while (0)
