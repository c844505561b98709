// Internal helpers shared by the HIP sources of the int8 KV path (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#include "../../include/nova_kv.h"

namespace nkv {

// ---------------------------------------------------------------- status / errors

void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);
int check_launch(const char* what);

// ---------------------------------------------------------------- vector types

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t as_u32(half2_t h) { return __builtin_bit_cast(uint32_t, h); }
__device__ __forceinline__ half2_t as_h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }

// v_perm_b32: result byte i = sel byte i in 0..3 -> b.byte[sel], 4..7 -> a.byte[sel-4],
// 0x0c -> 0x00 (checked on gfx950).
__device__ __forceinline__ uint32_t perm(uint32_t a, uint32_t b, uint32_t sel) {
  return __builtin_amdgcn_perm(a, b, sel);
}

// Two uint8 codes (bytes lo/hi of `x` picked by `sel`) -> half2 (1024 + code), exact.
// sel 0x04010400 takes bytes 0,1; 0x04030402 takes bytes 2,3.
constexpr uint32_t kBias1024 = 0x64646464u;
constexpr uint32_t kSelB01 = 0x04010400u;
constexpr uint32_t kSelB23 = 0x04030402u;

__device__ __forceinline__ half2_t codes_to_h2(uint32_t x, uint32_t sel) {
  const half2_t k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
  return as_h2(perm(kBias1024, x, sel)) - k1024;  // exact: integers 0..255
}

// Signed int8 codes (two's-complement bytes) to fp16, exactly: flipping the sign bit gives
// code + 128 in 0..255, converted as above, minus 1152.
__device__ __forceinline__ half2_t scodes_to_h2(uint32_t x, uint32_t sel) {
  const half2_t k1152 = {(_Float16)1152.0f, (_Float16)1152.0f};
  return as_h2(perm(kBias1024, x ^ 0x80808080u, sel)) - k1152;
}

// fp16 <-> fp32 with explicit round-to-nearest-even.
__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }
__device__ __forceinline__ uint16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) return (uint16_t)((u >> 16) | 0x40);  // NaN
  u += 0x7fffu + ((u >> 16) & 1u);  // round to nearest even
  return (uint16_t)(u >> 16);
}

// Cross-lane helpers (wave64).
__device__ __forceinline__ float shfl_xor(float v, int m) { return __shfl_xor(v, m, 64); }
__device__ __forceinline__ float shfl(float v, int src) { return __shfl(v, src, 64); }

// The int8t64 ruler arithmetic shared by every quantizer in this library, written with
// explicit round-to-nearest intrinsics so that no contraction changes a bit:
//   step = max((mx - mn) / 255, 1e-8), code = clamp(rint((x - mn) / step), 0, 255).
__device__ __forceinline__ float ruler_step(float mn, float mx) {
  return fmaxf(__fdiv_rn(__fsub_rn(mx, mn), 255.0f), 1e-8f);
}
__device__ __forceinline__ uint32_t ruler_code(float x, float mn, float step) {
  float r = __builtin_rintf(__fdiv_rn(__fsub_rn(x, mn), step));
  r = fminf(fmaxf(r, 0.0f), 255.0f);
  return (uint32_t)r;
}

// The same code with the quotient taken as (x - mn) * inv, inv = rcp(step) (<= 1 ulp).
// For quotients in [0, 256] that product is within 2^-14 of the exact quotient, and the
// correctly rounded quotient within 2^-16 of it, so both round to the same integer unless
// the product lies within 2^-12 of a half-integer; there the IEEE division decides. The
// result is identical to ruler_code for every input.
__device__ __forceinline__ uint32_t ruler_code_rcp(float x, float mn, float step, float inv) {
  const float d = __fsub_rn(x, mn);
  float q = __fmul_rn(d, inv);
  if (__builtin_fabsf((q - __builtin_floorf(q)) - 0.5f) < 0x1p-12f) q = __fdiv_rn(d, step);
  const float r = fminf(fmaxf(__builtin_rintf(q), 0.0f), 255.0f);
  return (uint32_t)r;
}
__device__ __forceinline__ float ruler_inv(float step) { return __builtin_amdgcn_rcpf(step); }

// The per-token symmetric ("tok") arithmetic: scale = max(absmax / 127, 1e-8) in fp32 (stored
// as fp16), code = clamp(rint(x / scale), -127, 127) with the fp32 scale.
__device__ __forceinline__ float sym_scale(float amax) { return fmaxf(__fdiv_rn(amax, 127.0f), 1e-8f); }
__device__ __forceinline__ uint32_t sym_code(float x, float scale) {
  const float r = fminf(fmaxf(__builtin_rintf(__fdiv_rn(x, scale)), -127.0f), 127.0f);
  return (uint32_t)(int32_t)r & 0xffu;
}

// Max over the 16 lanes of each 16-lane row (DPP only).
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xf, 0xf, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xf, 0xf, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xf, 0xf, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xf, 0xf, false)));
  return v;
}

// One 128-value row quantized by the 16 lanes of a 16-lane row, 8 values per lane: returns
// the lane's 8 packed codes and (in every lane) the fp32 scale.
__device__ __forceinline__ uint2 sym_quant8(const float (&v)[8], float& scale) {
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) amax = fmaxf(amax, __builtin_fabsf(v[j]));
  scale = sym_scale(row16_max(amax));
  uint32_t c[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) c[j] = sym_code(v[j], scale);
  return uint2{c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24), c[4] | (c[5] << 8) | (c[6] << 16) | (c[7] << 24)};
}

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace nkv
