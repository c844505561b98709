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
#include <type_traits>

#include "nkv_common.h"

namespace nkv {

namespace {

constexpr int GV_MAX_IN = 16384;  // input features (the LDS copy takes 2 bytes each)
constexpr int GV_WAVES = 8;       // rows (waves) per workgroup

__device__ __forceinline__ _Float16 as_half(uint16_t b) { return __builtin_bit_cast(_Float16, b); }
__device__ __forceinline__ uint16_t half_bits(_Float16 h) { return __builtin_bit_cast(uint16_t, h); }

// The workgroup's share of the input vector: thread t holds 16-byte chunks t + 64 W k of x (and
// of gamma when NORM), k < XC, so that XC 64 W >= 64 NL >= the input's chunk count.
template <int NL, int W, bool NORM>
struct InputChunks {
  static constexpr int XC = (NL + W - 1) / W;
  uint4 x[XC];
  uint4 g[NORM ? XC : 1];

  __device__ __forceinline__ void issue(const uint16_t* xp, const uint16_t* gp, int nch) {
#pragma unroll
    for (int k = 0; k < XC; ++k) {
      const int c = (int)threadIdx.x + 64 * W * k;
      x[k] = c < nch ? *reinterpret_cast<const uint4*>(xp + 8 * c) : uint4{0, 0, 0, 0};
      if (NORM) g[k] = c < nch ? *reinterpret_cast<const uint4*>(gp + 8 * c) : uint4{0, 0, 0, 0};
    }
  }

  // The input into LDS as fp16: x itself, or its RMSNorm in the order torch evaluates
  // fp16(fp16(x * rsqrt(mean(x^2) + eps)) * gamma), with the mean in fp32.
  __device__ __forceinline__ void stage(float eps, int n, int nch, uint16_t* xs) {
    __shared__ float part[W];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float r = 1.0f;
    if (NORM) {
      float ss = 0.0f;
#pragma unroll
      for (int k = 0; k < XC; ++k) ss = sumsq8(x[k], ss);
      ss = hsum64(ss);
      if (lane == 0) part[wave] = ss;
      __syncthreads();
      float tot = 0.0f;
#pragma unroll
      for (int w = 0; w < W; ++w) tot += part[w];
      r = rsqrtf(tot * (1.0f / (float)n) + eps);  // torch: mean = sum * (1/n), then rsqrt
    }
#pragma unroll
    for (int k = 0; k < XC; ++k) {
      const int c = tid + 64 * W * k;
      if (c < nch) {
        const uint4 v = NORM ? rms_scale8(x[k], g[k], r) : x[k];
        *reinterpret_cast<uint4*>(xs + 8 * c) = v;
      }
    }
    __syncthreads();
  }
};

// acc[j] = row j . xn for the NR rows rp[] (absent when !rv[j]), each row of nch 16-byte
// chunks: lane l holds chunks l + 64 u (u < NL; NL * 64 >= nch), so that a wave load covers
// 1 KiB of a row. The input chunks are loaded first, then every weight load of the wave's
// rows; the input is normalized into LDS while the weights are in flight (the in-order load
// counter lets the input arrive without waiting for the weights), and a wave waits for HBM once.
// Wave sums land in every lane.
template <int NL, int NR, int W, bool NORM>
__device__ __forceinline__ void rows_dot(InputChunks<NL, W, NORM>& ic, const uint16_t* const (&rp)[NR],
                                         const bool (&rv)[NR], int in, float eps, uint16_t* xs, float (&acc)[NR]) {
  const int lane = threadIdx.x & 63, nch = in / 8;
  uint4 wv[NR][NL];
#pragma unroll
  for (int j = 0; j < NR; ++j)
#pragma unroll
    for (int u = 0; u < NL; ++u) {
      const int c = lane + 64 * u;
      wv[j][u] = (rv[j] && c < nch) ? ld_weight(rp[j] + 8 * c) : uint4{0, 0, 0, 0};
    }
  ic.stage(eps, in, nch, xs);
#pragma unroll
  for (int j = 0; j < NR; ++j) acc[j] = 0.0f;
#pragma unroll
  for (int u = 0; u < NL; ++u) {
    const int c = lane + 64 * u;
    if (c < nch) {
      const uint4 xv = *reinterpret_cast<const uint4*>(xs + 8 * c);
#pragma unroll
      for (int j = 0; j < NR; ++j) acc[j] = dot8(wv[j][u], xv, acc[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < NR; ++j) acc[j] = hsum64(acc[j]);
}

// y = W xn (+ residual) in fp16, one row per wave: wave w of workgroup b takes row b W + w.
template <int NL, int W, bool NORM>
__global__ __launch_bounds__(64 * W) void gemv_kernel(const uint16_t* x, const uint16_t* gamma, float eps,
                                                      const uint16_t* w, int64_t out, int in,
                                                      const uint16_t* residual, uint16_t* y) {
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t o = (int64_t)blockIdx.x * W + wave;
  const bool rv[1] = {o < out};
  InputChunks<NL, W, NORM> ic;
  ic.issue(x, gamma, in / 8);
  const uint16_t res = (residual && rv[0]) ? residual[o] : (uint16_t)0;  // before the weights, too
  const uint16_t* const rp[1] = {w + (rv[0] ? o : 0) * (int64_t)in};
  float acc[1];
  rows_dot<NL, 1, W, NORM>(ic, rp, rv, in, eps, xs, acc);
  if (lane == 0 && rv[0]) {
    _Float16 r = (_Float16)acc[0];  // the projection's fp16 result, then the residual add in fp16
    if (residual) r = (_Float16)((float)r + (float)as_half(res));
    y[o] = half_bits(r);
  }
}

// act[j] = fp16(silu(g_j)) * u_j with g = rows [0, inter) and u = rows [inter, 2 inter) of the
// stacked gate/up weight, as torch evaluates F.silu(gate(x)) * up(x) in fp16. Each wave takes
// one gate row and the matching up row.
template <int NL, int W, bool NORM>
__global__ __launch_bounds__(64 * W) void swiglu_kernel(const uint16_t* x, const uint16_t* gamma, float eps,
                                                        const uint16_t* wgu, int64_t inter, int in, uint16_t* act) {
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t j = (int64_t)blockIdx.x * W + wave;
  const bool ok = j < inter;
  const bool rv[2] = {ok, ok};
  InputChunks<NL, W, NORM> ic;
  ic.issue(x, gamma, in / 8);
  const uint16_t* g_row = wgu + (ok ? j : 0) * (int64_t)in;
  const uint16_t* const rp[2] = {g_row, g_row + inter * (int64_t)in};
  float acc[2];
  rows_dot<NL, 2, W, NORM>(ic, rp, rv, in, eps, xs, acc);
  if (lane == 0 && ok) {
    const float g = (float)(_Float16)acc[0], u = (float)(_Float16)acc[1];
    const _Float16 s = (_Float16)(g / (1.0f + expf(-g)));
    act[j] = half_bits((_Float16)((float)s * u));
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
  uint16_t lo, hi;
  qk_norm_rope_lane((float)as_half(p[l]), (float)as_half(p[l + 64]), (float)as_half(g[l]), (float)as_half(g[l + 64]),
                    eps, (float)*pos * inv_freq[l], lo, hi);
  p[l] = lo;
  p[l + 64] = hi;
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Whether the fp16 ranges [a, a + an) and [b, b + bn) share an element.
bool overlap(const void* a, int64_t an, const void* b, int64_t bn) {
  const uintptr_t pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
  return pa < pb + 2 * (uintptr_t)bn && pb < pa + 2 * (uintptr_t)an;
}

// Every workgroup reads all of x while others write their rows of y: y must not overlap x.
int check(const char* what, const void* x, const void* w, const void* y, int64_t out, int64_t in) {
  if (!x || !w || !y) return fail(NKV_ERR_INVALID, "%s: null pointer argument", what);
  if (out <= 0 || out > INT32_MAX || in <= 0 || in % 8 || in > GV_MAX_IN)
    return fail(NKV_ERR_INVALID, "%s: sizes out=%lld in=%lld (out in [1, 2^31), in a positive multiple of 8, at most %d)",
                what, (long long)out, (long long)in, GV_MAX_IN);
  if (!al16(x) || !al16(w)) return fail(NKV_ERR_UNSUPPORTED, "%s: x and W must be 16-byte aligned", what);
  if (overlap(x, in, y, out)) return fail(NKV_ERR_INVALID, "%s: the output overlaps x", what);
  return NKV_OK;
}

template <int N>
using nl_t = std::integral_constant<int, N>;

// Calls f(nl_t<NL>{}) for the smallest supported NL with 64 NL >= nch (16-byte chunks per
// row), so that a lane holds its chunks of a row in NL registers of 16 bytes.
template <class F>
void with_nl(int nch, F&& f) {
  const int nl = (nch + 63) / 64;
  if (nl <= 1) f(nl_t<1>{});
  else if (nl <= 2) f(nl_t<2>{});
  else if (nl <= 3) f(nl_t<3>{});
  else if (nl <= 4) f(nl_t<4>{});
  else if (nl <= 5) f(nl_t<5>{});
  else if (nl <= 6) f(nl_t<6>{});
  else if (nl <= 8) f(nl_t<8>{});
  else if (nl <= 10) f(nl_t<10>{});
  else if (nl <= 12) f(nl_t<12>{});
  else if (nl <= 16) f(nl_t<16>{});
  else if (nl <= 20) f(nl_t<20>{});
  else if (nl <= 24) f(nl_t<24>{});
  else f(nl_t<32>{});  // GV_MAX_IN / 8 / 64 = 32
}

template <int W>
void launch_gemv_w(const uint16_t* x, const uint16_t* gamma, float eps, const uint16_t* w, int64_t out, int in,
                   const uint16_t* residual, uint16_t* y, hipStream_t s) {
  const unsigned blocks = (unsigned)((out + W - 1) / W);
  with_nl(in / 8, [&](auto nl) {
    constexpr int NL = decltype(nl)::value;
    if (gamma)
      hipLaunchKernelGGL((gemv_kernel<NL, W, true>), dim3(blocks), dim3(64 * W), (size_t)in * 2, s, x, gamma, eps, w,
                         out, in, residual, y);
    else
      hipLaunchKernelGGL((gemv_kernel<NL, W, false>), dim3(blocks), dim3(64 * W), (size_t)in * 2, s, x, gamma, eps, w,
                         out, in, residual, y);
  });
}

template <int W>
void launch_swiglu_w(const uint16_t* x, const uint16_t* gamma, float eps, const uint16_t* wgu, int64_t inter, int in,
                     uint16_t* act, hipStream_t s) {
  const unsigned blocks = (unsigned)((inter + W - 1) / W);
  with_nl(in / 8, [&](auto nl) {
    constexpr int NL = decltype(nl)::value;
    if (gamma)
      hipLaunchKernelGGL((swiglu_kernel<NL, W, true>), dim3(blocks), dim3(64 * W), (size_t)in * 2, s, x, gamma, eps,
                         wgu, inter, in, act);
    else
      hipLaunchKernelGGL((swiglu_kernel<NL, W, false>), dim3(blocks), dim3(64 * W), (size_t)in * 2, s, x, gamma, eps,
                         wgu, inter, in, act);
  });
}

// Eight rows (waves) per workgroup, so the input is read and normalized once per eight rows.
// Outputs of 1024 to 2560 rows: ten, one workgroup per CU or fewer (2560 rows: 256 workgroups;
// the down projection 10.23 us against 10.52 us as 640 workgroups of four). Other outputs under
// 4096 rows: four.
void launch_gemv(const uint16_t* x, const uint16_t* gamma, float eps, const uint16_t* w, int64_t out, int in,
                 const uint16_t* residual, uint16_t* y, hipStream_t s) {
  if (out >= 1024 && out <= 2560)
    launch_gemv_w<10>(x, gamma, eps, w, out, in, residual, y, s);
  else if (out < 4096)
    launch_gemv_w<4>(x, gamma, eps, w, out, in, residual, y, s);
  else
    launch_gemv_w<GV_WAVES>(x, gamma, eps, w, out, in, residual, y, s);
}

// (two rows per wave: beyond 16 chunks per lane and row, four waves per workgroup leave each
// wave the registers for both rows' loads)
void launch_swiglu(const uint16_t* x, const uint16_t* gamma, float eps, const uint16_t* wgu, int64_t inter, int in,
                   uint16_t* act, hipStream_t s) {
  if (in / 8 > 16 * 64)
    launch_swiglu_w<4>(x, gamma, eps, wgu, inter, in, act, s);
  else
    launch_swiglu_w<GV_WAVES>(x, gamma, eps, wgu, inter, in, act, s);
}

}  // namespace

}  // namespace nkv

using namespace nkv;

extern "C" int nkv_gemv(const uint16_t* x, const uint16_t* gamma, float eps, const uint16_t* w, int64_t out_features,
                        int64_t in_features, const uint16_t* residual, uint16_t* y, void* stream) {
  set_error("");
  if (int rc = check("gemv", x, w, y, out_features, in_features)) return rc;
  if (gamma && !al16(gamma)) return fail(NKV_ERR_UNSUPPORTED, "gemv: gamma must be 16-byte aligned");
  // row o reads residual[o] and writes y[o] in one wave: y may be the residual, not a shifted view of it
  if (residual && residual != y && overlap(residual, out_features, y, out_features))
    return fail(NKV_ERR_INVALID, "gemv: y must be the residual itself or not overlap it");
  launch_gemv(x, gamma, eps, w, out_features, (int)in_features, residual, y, static_cast<hipStream_t>(stream));
  return check_launch("gemv");
}

extern "C" int nkv_swiglu_gemv(const uint16_t* x, const uint16_t* gamma, float eps, const uint16_t* w_gate_up,
                               int64_t intermediate, int64_t in_features, uint16_t* act, void* stream) {
  set_error("");
  if (int rc = check("swiglu_gemv", x, w_gate_up, act, intermediate, in_features)) return rc;
  if (gamma && !al16(gamma)) return fail(NKV_ERR_UNSUPPORTED, "swiglu_gemv: gamma must be 16-byte aligned");
  launch_swiglu(x, gamma, eps, w_gate_up, intermediate, (int)in_features, act, static_cast<hipStream_t>(stream));
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
