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

// ---- the decode-step projections' arithmetic, shared by the GEMV kernels and the fused
// projection + attention step, so that both compute the same bits

// Wave sum (every lane gets it), in a fixed order.
__device__ __forceinline__ float hsum64(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// acc + the dot product of 8 fp16 weights and 8 fp16 inputs (fp32 accumulation, pairwise).
__device__ __forceinline__ float dot8(uint4 w, uint4 x, float acc) {
  acc = __builtin_amdgcn_fdot2(as_h2(w.x), as_h2(x.x), acc, false);
  acc = __builtin_amdgcn_fdot2(as_h2(w.y), as_h2(x.y), acc, false);
  acc = __builtin_amdgcn_fdot2(as_h2(w.z), as_h2(x.z), acc, false);
  acc = __builtin_amdgcn_fdot2(as_h2(w.w), as_h2(x.w), acc, false);
  return acc;
}

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// A weight load: 16 bytes, nontemporal (weights stream through once per decode step).
__device__ __forceinline__ uint4 ld_weight(const uint16_t* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return uint4{v.x, v.y, v.z, v.w};
}

// The sum of squares of 8 fp16 inputs, added to ss in element order.
__device__ __forceinline__ float sumsq8(uint4 x, float ss) {
  const uint32_t u[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const half2_t h = as_h2(u[e]);
    ss += (float)h.x * (float)h.x;
    ss += (float)h.y * (float)h.y;
  }
  return ss;
}

// 8 inputs normalized as torch's fp16 RMSNorm evaluates them: fp16(fp16(x * r) * gamma).
__device__ __forceinline__ uint4 rms_scale8(uint4 x, uint4 g, float r) {
  uint32_t u[4] = {x.x, x.y, x.z, x.w};
  const uint32_t gu[4] = {g.x, g.y, g.z, g.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const half2_t h = as_h2(u[e]), gg = as_h2(gu[e]);
    half2_t o;
    o.x = (_Float16)((float)(_Float16)((float)h.x * r) * (float)gg.x);
    o.y = (_Float16)((float)(_Float16)((float)h.y * r) * (float)gg.y);
    u[e] = as_u32(o);
  }
  return uint4{u[0], u[1], u[2], u[3]};
}

// One head vector's q/k RMSNorm and rotary embedding in torch's fp16 order, for the lane that
// holds elements l and l + 64 (a, b; the pair rotate_half mixes): the mean of squares over the
// wave, x * cos + rotate_half(x) * sin with cos/sin of f = pos * inv_freq[l] rounded to fp16
// and every product and sum rounded to fp16. Returns the two fp16 results (lo: element l).
__device__ __forceinline__ void qk_norm_rope_lane(float a, float b, float ga, float gb, float eps, float f,
                                                  uint16_t& lo16, uint16_t& hi16) {
  // torch rounds each product to fp16 before the sum: no fusing into an fp16 fma here
#pragma clang fp contract(off)
  const float ss = hsum64(a * a + b * b);
  const float r = rsqrtf(ss * (1.0f / 128.0f) + eps);
  const float na = (float)(_Float16)((float)(_Float16)(a * r) * ga);
  const float nb = (float)(_Float16)((float)(_Float16)(b * r) * gb);
  const float c = (float)(_Float16)cosf(f), s = (float)(_Float16)sinf(f);
  const float lo = (float)(_Float16)(na * c) + (float)(_Float16)(-nb * s);
  const float hi = (float)(_Float16)(nb * c) + (float)(_Float16)(na * s);
  lo16 = f2h(lo);
  hi16 = f2h(hi);
}

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace nkv
