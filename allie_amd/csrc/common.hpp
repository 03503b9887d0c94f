// Shared device helpers for the Allie gfx950 kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define ALLIE_DEV __device__ __forceinline__

typedef uint16_t bf16_t;  // storage type: raw bf16 bits
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// fp32 -> bf16, round to nearest even: gfx950's v_cvt_pk_bf16_f32 converts
// two values per instruction (NaN stays NaN).
ALLIE_DEV uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2_t v;
  v[0] = (__bf16)lo;
  v[1] = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, v);
}
ALLIE_DEV uint32_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
ALLIE_DEV float bf2f(uint32_t b) { return __uint_as_float(b << 16); }
ALLIE_DEV float round_bf16(float f) { return (float)(__bf16)f; }
// two values rounded to bf16 and widened back (one conversion instruction)
ALLIE_DEV void round_bf16x2(float& a, float& b) {
  const uint32_t p = pack_bf16x2(a, b);
  a = __uint_as_float(p << 16);
  b = __uint_as_float(p & 0xffff0000u);
}

// Elements OFF .. OFF+7 of x -> hi = bf16(x), lo = bf16(x - hi): hi + lo
// carries ~16 mantissa bits of x (for MFMA operands that need more than
// bf16's 8).
template <int OFF>
ALLIE_DEV void split_bf16x8(const f32x16_t& x, bf16x8_t& hi, bf16x8_t& lo) {
  uint32_t h[4], l[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float x0 = x[OFF + 2 * e], x1 = x[OFF + 2 * e + 1];
    h[e] = pack_bf16x2(x0, x1);
    l[e] = pack_bf16x2(x0 - __uint_as_float(h[e] << 16), x1 - __uint_as_float(h[e] & 0xffff0000u));
  }
  hi = __builtin_bit_cast(bf16x8_t, u32x4_t{h[0], h[1], h[2], h[3]});
  lo = __builtin_bit_cast(bf16x8_t, u32x4_t{l[0], l[1], l[2], l[3]});
}

// OCP fp8 e4m3fn -> fp32 (exact).  bias 7, no infinities, 0x7f/0xff = NaN.
ALLIE_DEV float fp8e4m3_to_f32(uint32_t v) {
  uint32_t s = (v & 0x80u) << 24;
  uint32_t e = (v >> 3) & 0xfu;
  uint32_t m = v & 0x7u;
  if (e == 0) {  // subnormal: m * 2^-9
    float f = (float)m * 0.001953125f;
    return __uint_as_float(__float_as_uint(f) | s);
  }
  if (e == 15 && m == 7) return __uint_as_float(0x7fc00000u | s);
  return __uint_as_float(s | ((e + 120u) << 23) | (m << 20));
}
// fp8 e4m3fn -> bf16 bits (exact: 3 mantissa bits fit in bf16's 7)
ALLIE_DEV uint32_t fp8e4m3_to_bf16(uint32_t v) { return __float_as_uint(fp8e4m3_to_f32(v)) >> 16; }

// x combined with the x of lane l ^ 16 / l ^ 32 through gfx950's
// v_permlane16_swap / v_permlane32_swap (lanes exchanged between 16-lane rows
// / wave halves in registers, no LDS round trip as with a bpermute); both
// lanes of a pair get the same bits (the lower lane's operand first).
ALLIE_DEV float xor16_max(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
ALLIE_DEV float xor16_sum(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
ALLIE_DEV float xor32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
ALLIE_DEV float xor32_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// sum over the wave in registers: DPP within rows of 16 lanes (xor 1, 2,
// then half-row and row mirrors), then across rows by v_permlane16/32_swap;
// no LDS instruction (wave_sum's shuffles are ds_bpermute round trips).  Every
// lane gets the same bits.
template <int CTRL>
ALLIE_DEV float dpp_mov_f(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xf, 0xf, false));
}
ALLIE_DEV float wave_sum_regs(float v) {
  v += dpp_mov_f<0xb1>(v);   // quad_perm [1, 0, 3, 2]
  v += dpp_mov_f<0x4e>(v);   // quad_perm [2, 3, 0, 1]
  v += dpp_mov_f<0x141>(v);  // row_half_mirror: lane i + lane 7 - i of each 8
  v += dpp_mov_f<0x140>(v);  // row_mirror: lane i + lane 15 - i of each 16
  return xor32_sum(xor16_sum(v));
}

ALLIE_DEV float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
ALLIE_DEV float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// tanh from exp: tanh(x) = 1 - 2 / (exp(2x) + 1); saturates cleanly for |x| large.
ALLIE_DEV float tanh_fast(float x) {
  float e = __expf(2.0f * x);
  return 1.0f - 2.0f / (e + 1.0f);
}

// gelu_new for the bf16 epilogues: 0.5 x (1 + tanh(u)) == x * sigmoid(2 u)
// with u = sqrt(2/pi) (x + 0.044715 x^3); hardware exp2 and reciprocal
// (relative error ~1e-7, far below the bf16 rounding of the result).
ALLIE_DEV float gelu_tanh_fast(float x) {
  const float k2 = -2.0f * 0.7978845608028654f * 1.4426950408889634f;  // -2 sqrt(2/pi) log2(e)
  // k2 u = x (k2 + k2 0.044715 x^2)
  const float t = x * fmaf(x * x, k2 * 0.044715f, k2);
  const float e = __builtin_amdgcn_exp2f(t);
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}

// gelu_new (tanh form), evaluated in fp32 with the precise tanh (fp32 path).
ALLIE_DEV float gelu_tanh(float x) {
  const float k0 = 0.7978845608028654f;  // sqrt(2/pi)
  float inner = k0 * (x + 0.044715f * (x * x * x));
  return (0.5f * x) * (1.0f + tanhf(inner));
}
