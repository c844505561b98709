// Batch-1 decode projections of the synthetic skeleton around the int8 KV path: RMSNorm
// fused into a GEMV (optionally with the residual add), the SwiGLU MLP's gate/up GEMV fused
// with its activation, and the per-head q/k RMSNorm + rotary embedding.
//
// The GEMVs are HBM-bound: every weight byte is read once, 16 bytes per lane per load (a wave
// load covers 1 KiB of one row), and the dot products accumulate in fp32 (v_dot2_f32_f16).
// The first batch of weight loads is issued before the input is normalized, so the norm's
// reduction and barrier hide under the HBM latency. The normalized input sits in LDS (dynamic,
// sized to the input), shared by the workgroup's rows.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "nkv_common.h"

namespace nkv {

namespace {

constexpr int GV_MAX_IN = 16384;  // input features (the LDS copy takes 2 bytes each)
constexpr int GV_UNROLL = 4;      // 16-byte chunks per lane per row in one load batch

__device__ __forceinline__ float hsum64(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ float dot8(uint4 w, uint4 x, float acc) {
  acc = __builtin_amdgcn_fdot2(as_h2(w.x), as_h2(x.x), acc, false);
  acc = __builtin_amdgcn_fdot2(as_h2(w.y), as_h2(x.y), acc, false);
  acc = __builtin_amdgcn_fdot2(as_h2(w.z), as_h2(x.z), acc, false);
  acc = __builtin_amdgcn_fdot2(as_h2(w.w), as_h2(x.w), acc, false);
  return acc;
}

__device__ __forceinline__ _Float16 as_half(uint16_t b) { return __builtin_bit_cast(_Float16, b); }
__device__ __forceinline__ uint16_t half_bits(_Float16 h) { return __builtin_bit_cast(uint16_t, h); }

// The input into LDS as fp16: x itself, or its RMSNorm in the order torch evaluates
// fp16(fp16(x * rsqrt(mean(x^2) + eps)) * gamma), with the mean in fp32.
template <int W>
__device__ __forceinline__ void load_input(const uint16_t* x, const uint16_t* gamma, float eps, int n, uint16_t* xs) {
  __shared__ float part[W];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float r = 1.0f;
  if (gamma) {
    float ss = 0.0f;
    for (int i = tid; i < n; i += 64 * W) {
      const float v = (float)as_half(x[i]);
      ss += v * v;
    }
    ss = hsum64(ss);
    if (lane == 0) part[wave] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < W; ++w) tot += part[w];
    r = rsqrtf(tot * (1.0f / (float)n) + eps);  // torch: mean = sum * (1/n), then rsqrt
  }
  for (int i = tid; i < n; i += 64 * W) {
    _Float16 v = as_half(x[i]);
    if (gamma) v = (_Float16)((float)(_Float16)((float)v * r) * (float)as_half(gamma[i]));
    xs[i] = half_bits(v);
  }
  __syncthreads();
}

// One load batch: chunks c0 + 64 u (u < GV_UNROLL) of each of the NR rows (row j at rp[j],
// absent when !rv[j]); chunks past the row end read as zero.
template <int NR>
__device__ __forceinline__ void load_batch(const uint16_t* const (&rp)[NR], const bool (&rv)[NR], int c0, int nch,
                                           uint4 (&wv)[NR][GV_UNROLL]) {
#pragma unroll
  for (int j = 0; j < NR; ++j)
#pragma unroll
    for (int u = 0; u < GV_UNROLL; ++u) {
      const int c = c0 + 64 * u;
      wv[j][u] = (rv[j] && c < nch) ? *reinterpret_cast<const uint4*>(rp[j] + 8 * c) : uint4{0, 0, 0, 0};
    }
}

template <int NR>
__device__ __forceinline__ void dot_batch(const uint4 (&wv)[NR][GV_UNROLL], const uint16_t* xs, int c0, int nch,
                                          float (&acc)[NR]) {
#pragma unroll
  for (int u = 0; u < GV_UNROLL; ++u) {
    const int c = c0 + 64 * u;
    if (c < nch) {
      const uint4 xv = *reinterpret_cast<const uint4*>(xs + 8 * c);
#pragma unroll
      for (int j = 0; j < NR; ++j) acc[j] = dot8(wv[j][u], xv, acc[j]);
    }
  }
}

// acc[j] = row j . xn for the NR rows rp[], the input normalized into LDS between the first
// load batch and its products; wave sums land in every lane.
template <int NR, int W>
__device__ __forceinline__ void rows_dot(const uint16_t* const (&rp)[NR], const bool (&rv)[NR], int in,
                                         const uint16_t* x, const uint16_t* gamma, float eps, uint16_t* xs,
                                         float (&acc)[NR]) {
  const int lane = threadIdx.x & 63, nch = in / 8;
  uint4 wv[NR][GV_UNROLL];
  load_batch<NR>(rp, rv, lane, nch, wv);
  load_input<W>(x, gamma, eps, in, xs);
#pragma unroll
  for (int j = 0; j < NR; ++j) acc[j] = 0.0f;
  for (int c0 = lane;;) {
    dot_batch<NR>(wv, xs, c0, nch, acc);
    c0 += 64 * GV_UNROLL;
    if (c0 >= nch) break;
    load_batch<NR>(rp, rv, c0, nch, wv);
  }
#pragma unroll
  for (int j = 0; j < NR; ++j) acc[j] = hsum64(acc[j]);
}

// y = W xn (+ residual) in fp16: wave w of workgroup b takes rows (b W + w) R ... + R - 1.
template <int R, int W>
__global__ __launch_bounds__(64 * W) void gemv_kernel(const uint16_t* x, const uint16_t* gamma, float eps,
                                                      const uint16_t* w, int64_t out, int in,
                                                      const uint16_t* residual, uint16_t* y) {
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t o0 = ((int64_t)blockIdx.x * W + wave) * R;
  const uint16_t* rp[R];
  bool rv[R];
#pragma unroll
  for (int j = 0; j < R; ++j) {
    rv[j] = o0 + j < out;
    rp[j] = w + (rv[j] ? o0 + j : 0) * (int64_t)in;
  }
  float acc[R];
  rows_dot<R, W>(rp, rv, in, x, gamma, eps, xs, acc);
  if (lane == 0) {
#pragma unroll
    for (int j = 0; j < R; ++j) {
      if (!rv[j]) break;
      _Float16 r = (_Float16)acc[j];  // the projection's fp16 result, then the residual add in fp16
      if (residual) r = (_Float16)((float)r + (float)as_half(residual[o0 + j]));
      y[o0 + j] = half_bits(r);
    }
  }
}

// act[j] = fp16(silu(g_j)) * u_j with g = rows [0, inter) and u = rows [inter, 2 inter) of the
// stacked gate/up weight, as torch evaluates F.silu(gate(x)) * up(x) in fp16. Each wave takes
// R gate rows and the R matching up rows.
template <int R, int W>
__global__ __launch_bounds__(64 * W) void swiglu_kernel(const uint16_t* x, const uint16_t* gamma, float eps,
                                                        const uint16_t* wgu, int64_t inter, int in, uint16_t* act) {
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t j0 = ((int64_t)blockIdx.x * W + wave) * R;
  const uint16_t* rp[2 * R];
  bool rv[2 * R];
#pragma unroll
  for (int j = 0; j < R; ++j) {
    rv[j] = rv[R + j] = j0 + j < inter;
    rp[j] = wgu + (rv[j] ? j0 + j : 0) * (int64_t)in;
    rp[R + j] = rp[j] + inter * (int64_t)in;
  }
  float acc[2 * R];
  rows_dot<2 * R, W>(rp, rv, in, x, gamma, eps, xs, acc);
  if (lane == 0) {
#pragma unroll
    for (int j = 0; j < R; ++j) {
      if (!rv[j]) break;
      const float g = (float)(_Float16)acc[j], u = (float)(_Float16)acc[R + j];
      const _Float16 s = (_Float16)(g / (1.0f + expf(-g)));
      act[j0 + j] = half_bits((_Float16)((float)s * u));
    }
  }
}

// In place on one token's stacked projection [hq + 2 hkv][128]: RMSNorm over each of the
// hq + hkv q and k heads (fp32 mean of squares, the q or k gamma), then the rotary embedding
// at position *pos, in torch's order: x * cos + rotate_half(x) * sin with cos/sin of
// (float)pos * inv_freq[i mod 64] rounded to fp16 and every product and sum rounded to fp16.
// One wave per head; lane l holds elements l and l + 64, the pair rotate_half mixes.
__global__ __launch_bounds__(64) void qk_norm_rope_kernel(uint16_t* qkv, int hq, const uint16_t* q_gamma,
                                                          const uint16_t* k_gamma, float eps, const float* inv_freq,
                                                          const int64_t* pos) {
  const int head = blockIdx.x, l = threadIdx.x;
  uint16_t* p = qkv + (int64_t)head * 128;
  const uint16_t* g = head < hq ? q_gamma : k_gamma;
  const float a = (float)as_half(p[l]), b = (float)as_half(p[l + 64]);
  const float ss = hsum64(a * a + b * b);
  const float r = rsqrtf(ss * (1.0f / 128.0f) + eps);
  const float na = (float)(_Float16)((float)(_Float16)(a * r) * (float)as_half(g[l]));
  const float nb = (float)(_Float16)((float)(_Float16)(b * r) * (float)as_half(g[l + 64]));
  const float f = (float)*pos * inv_freq[l];
  const float c = (float)(_Float16)cosf(f), s = (float)(_Float16)sinf(f);
  const float lo = (float)(_Float16)(na * c) + (float)(_Float16)(-nb * s);
  const float hi = (float)(_Float16)(nb * c) + (float)(_Float16)(na * s);
  p[l] = half_bits((_Float16)lo);
  p[l + 64] = half_bits((_Float16)hi);
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check(const char* what, const void* x, const void* w, const void* y, int64_t out, int64_t in) {
  if (!x || !w || !y) return fail(NKV_ERR_INVALID, "%s: null pointer argument", what);
  if (out <= 0 || in <= 0 || in % 8 || in > GV_MAX_IN)
    return fail(NKV_ERR_INVALID, "%s: sizes out=%lld in=%lld (in a positive multiple of 8, at most %d)", what,
                (long long)out, (long long)in, GV_MAX_IN);
  if (!al16(x) || !al16(w)) return fail(NKV_ERR_UNSUPPORTED, "%s: x and W must be 16-byte aligned", what);
  return NKV_OK;
}

template <int R, int W>
void launch_gemv(const uint16_t* x, const uint16_t* gamma, float eps, const uint16_t* w, int64_t out, int in,
                 const uint16_t* residual, uint16_t* y, hipStream_t s) {
  const unsigned blocks = (unsigned)((out + R * W - 1) / (R * W));
  hipLaunchKernelGGL((gemv_kernel<R, W>), dim3(blocks), dim3(64 * W), (size_t)in * 2, s, x, gamma, eps, w, out, in,
                     residual, y);
}

}  // namespace

}  // namespace nkv

using namespace nkv;

extern "C" int nkv_gemv(const uint16_t* x, const uint16_t* gamma, float eps, const uint16_t* w, int64_t out_features,
                        int64_t in_features, const uint16_t* residual, uint16_t* y, void* stream) {
  set_error("");
  if (int rc = check("gemv", x, w, y, out_features, in_features)) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int in = (int)in_features;
  // large outputs (the lm_head): 4 rows per wave; otherwise one row per wave and two waves
  // per workgroup, so that a 2560-row projection is 1280 workgroups, 5 per CU
  if (out_features >= 16384)
    launch_gemv<4, 4>(x, gamma, eps, w, out_features, in, residual, y, s);
  else
    launch_gemv<1, 2>(x, gamma, eps, w, out_features, in, residual, y, s);
  return check_launch("gemv");
}

extern "C" int nkv_swiglu_gemv(const uint16_t* x, const uint16_t* gamma, float eps, const uint16_t* w_gate_up,
                               int64_t intermediate, int64_t in_features, uint16_t* act, void* stream) {
  set_error("");
  if (int rc = check("swiglu_gemv", x, w_gate_up, act, intermediate, in_features)) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  constexpr int R = 1, W = 2;
  const unsigned blocks = (unsigned)((intermediate + R * W - 1) / (R * W));
  hipLaunchKernelGGL((swiglu_kernel<R, W>), dim3(blocks), dim3(64 * W), (size_t)in_features * 2, s, x, gamma, eps,
                     w_gate_up, intermediate, (int)in_features, act);
  return check_launch("swiglu_gemv");
}

extern "C" int nkv_qk_norm_rope(uint16_t* qkv, int64_t hq, int64_t hkv, int64_t head_dim, const uint16_t* q_gamma,
                                const uint16_t* k_gamma, float eps, const float* inv_freq, const int64_t* pos,
                                void* stream) {
  set_error("");
  if (!qkv || !q_gamma || !k_gamma || !inv_freq || !pos) return fail(NKV_ERR_INVALID, "qk_norm_rope: null pointer");
  if (head_dim != 128) return fail(NKV_ERR_UNSUPPORTED, "qk_norm_rope: head_dim %lld (only 128)", (long long)head_dim);
  if (hq <= 0 || hkv <= 0 || hq > 4096 || hkv > 4096)
    return fail(NKV_ERR_INVALID, "qk_norm_rope: heads hq=%lld hkv=%lld", (long long)hq, (long long)hkv);
  hipLaunchKernelGGL(qk_norm_rope_kernel, dim3((unsigned)(hq + hkv)), dim3(64), 0, static_cast<hipStream_t>(stream),
                     qkv, (int)hq, q_gamma, k_gamma, eps, inv_freq, pos);
  return check_launch("qk_norm_rope");
}
