// Asymmetric int8 quantize / dequantize kernels (token axis and channel axis).
//
// Token axis, the format the decode path reads (src/nova/kvquant.py:136-149):
// one wave quantizes one (slab, group of `gs` tokens, 128-channel chunk).
// Lanes 0..15 own 8 consecutive channels each (16-byte loads, one 128-element
// row = 256 contiguous bytes per 16 lanes) and lanes (l >> 4) stride over the
// group's rows, so every load instruction reads four whole rows. Min/max are
// reduced across the four row-lanes with cross-lane shuffles; groups of at most
// 64 tokens stay in registers between the two passes.
#include "nkv_common.h"

#include <mutex>
#include <string>

namespace nkv {

static thread_local std::string g_err;

void set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
}

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(NKV_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return NKV_OK;
}

// ---------------------------------------------------------------- element loads

template <int DT>
struct Elem8;

template <>
struct Elem8<NKV_F16> {
  static __device__ __forceinline__ void load(const void* base, int64_t off, float (&v)[8]) {
    uint4 u = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + off);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = h2f((uint16_t)(w[i] & 0xffffu));
      v[2 * i + 1] = h2f((uint16_t)(w[i] >> 16));
    }
  }
};

template <>
struct Elem8<NKV_BF16> {
  static __device__ __forceinline__ void load(const void* base, int64_t off, float (&v)[8]) {
    uint4 u = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + off);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
};

template <>
struct Elem8<NKV_F32> {
  static __device__ __forceinline__ void load(const void* base, int64_t off, float (&v)[8]) {
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(base) + off);
    float4 a = p[0], b = p[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
};

__device__ __forceinline__ uint2 pack_codes8(const float (&x)[8], const float (&mn)[8],
                                             const float (&st)[8], const float (&inv)[8]) {
  uint32_t c[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) c[i] = ruler_code_rcp(x[i], mn[i], st[i], inv[i]);
  uint2 r;
  r.x = c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24);
  r.y = c[4] | (c[5] << 8) | (c[6] << 16) | (c[7] << 24);
  return r;
}

__device__ __forceinline__ uint4 pack_h8(const float (&v)[8]) {
  uint4 r;
  r.x = (uint32_t)f2h(v[0]) | ((uint32_t)f2h(v[1]) << 16);
  r.y = (uint32_t)f2h(v[2]) | ((uint32_t)f2h(v[3]) << 16);
  r.z = (uint32_t)f2h(v[4]) | ((uint32_t)f2h(v[5]) << 16);
  r.w = (uint32_t)f2h(v[6]) | ((uint32_t)f2h(v[7]) << 16);
  return r;
}

// ---------------------------------------------------------------- token-axis quantize

struct QuantTokArgs {
  const void* x;
  int64_t x_rs;
  int64_t rows, n, dim, gs, ngroups, nchunks;
  uint8_t* codes;
  int64_t c_rs;
  uint16_t* mins;
  uint16_t* steps;
  int64_t s_rs;
  int64_t items;
  // page destination (paged cache): group gi of slab r goes to page table[first_group + gi], KV
  // head r, tensor `which` (0 K, 1 V) of the page layout [K codes 64 x 128 | V codes | kst | kmn |
  // vst | vmn]; groups whose table entry is outside [0, num_pages) are skipped
  uint8_t* pages;
  const int32_t* table;
  int64_t first_group, num_pages;
  int which;
};

constexpr int64_t PAGE_GROUP_BYTES = 2 * 64 * 128 + 4 * 128 * 2;  // 17408

constexpr int kQuantWaves = 4;
constexpr int kCacheRows = 16;  // rows per lane kept in registers (groups of <= 64 tokens)

template <int DT, bool CACHE, bool PAGES = false>
__global__ __launch_bounds__(64 * kQuantWaves) void quant_token_kernel(QuantTokArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * kQuantWaves + (threadIdx.x >> 6);
  if (item >= a.items) return;
  const int64_t chunk = item % a.nchunks;
  const int64_t gi = (item / a.nchunks) % a.ngroups;
  const int64_t r = item / (a.nchunks * a.ngroups);
  const int cl = lane & 15, rl = lane >> 4;
  const int64_t ch = chunk * 128 + cl * 8;
  const bool active = ch < a.dim;
  const int64_t t0 = gi * a.gs;
  const int64_t nr = min(a.gs, a.n - t0);

  float mn[8], mx[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) { mn[j] = __builtin_huge_valf(); mx[j] = -__builtin_huge_valf(); }
  float cache[CACHE ? kCacheRows : 1][8];

  if (active) {
    const int64_t base = r * a.x_rs + ch;
    if (CACHE) {
#pragma unroll
      for (int i = 0; i < kCacheRows; ++i) {
        const int64_t t = rl + 4 * i;
        if (t < nr) {
          Elem8<DT>::load(a.x, base + (t0 + t) * a.dim, cache[i]);
#pragma unroll
          for (int j = 0; j < 8; ++j) { mn[j] = fminf(mn[j], cache[i][j]); mx[j] = fmaxf(mx[j], cache[i][j]); }
        }
      }
    } else {
      for (int64_t t = rl; t < nr; t += 4) {
        float v[8];
        Elem8<DT>::load(a.x, base + (t0 + t) * a.dim, v);
#pragma unroll
        for (int j = 0; j < 8; ++j) { mn[j] = fminf(mn[j], v[j]); mx[j] = fmaxf(mx[j], v[j]); }
      }
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    mn[j] = fminf(mn[j], shfl_xor(mn[j], 16));
    mn[j] = fminf(mn[j], shfl_xor(mn[j], 32));
    mx[j] = fmaxf(mx[j], shfl_xor(mx[j], 16));
    mx[j] = fmaxf(mx[j], shfl_xor(mx[j], 32));
  }
  if (!active) return;
  float st[8], inv[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) { st[j] = ruler_step(mn[j], mx[j]); inv[j] = ruler_inv(st[j]); }
  uint8_t* codes = a.codes;
  uint16_t* mins = a.mins;
  uint16_t* steps = a.steps;
  int64_t so = r * a.s_rs + gi * a.dim + ch;
  int64_t cbase = r * a.c_rs + ch;
  if constexpr (PAGES) {
    // token t of the group is row t of its page's code block; the rulers follow the code blocks
    const int32_t page = a.table[a.first_group + gi];
    if (page < 0 || page >= a.num_pages) return;
    uint8_t* pg = a.pages + ((int64_t)page * a.rows + r) * PAGE_GROUP_BYTES;
    codes = pg + a.which * 64 * 128;
    cbase = ch - t0 * a.dim;  // (t0 + t) * dim below addresses row t
    steps = reinterpret_cast<uint16_t*>(pg + 2 * 64 * 128) + a.which * 2 * 128;
    mins = steps + 128;
    so = ch;
  }
  if (rl == 0) {
    *reinterpret_cast<uint4*>(mins + so) = pack_h8(mn);
    *reinterpret_cast<uint4*>(steps + so) = pack_h8(st);
  }
  if (CACHE) {
#pragma unroll
    for (int i = 0; i < kCacheRows; ++i) {
      const int64_t t = rl + 4 * i;
      if (t < nr) *reinterpret_cast<uint2*>(codes + cbase + (t0 + t) * a.dim) = pack_codes8(cache[i], mn, st, inv);
    }
  } else {
    const int64_t base = r * a.x_rs + ch;
    for (int64_t t = rl; t < nr; t += 4) {
      float v[8];
      Elem8<DT>::load(a.x, base + (t0 + t) * a.dim, v);
      *reinterpret_cast<uint2*>(codes + cbase + (t0 + t) * a.dim) = pack_codes8(v, mn, st, inv);
    }
  }
}

// ---------------------------------------------------------------- channel-axis quantize

struct QuantChanArgs {
  const void* x;
  int64_t x_rs;
  int64_t rows, n, dim, gc, ngc;
  uint8_t* codes;
  int64_t c_rs;
  uint16_t* mins;
  uint16_t* steps;
  int64_t s_rs;
  int64_t items;  // rows * n * ngc
};

template <int DT>
__device__ __forceinline__ float load1(const void* p, int64_t off) {
  if (DT == NKV_F16) return h2f(static_cast<const uint16_t*>(p)[off]);
  if (DT == NKV_BF16) return bf2f(static_cast<const uint16_t*>(p)[off]);
  return static_cast<const float*>(p)[off];
}

template <int DT>
__global__ __launch_bounds__(256) void quant_channel_kernel(QuantChanArgs a) {
  const int64_t item = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= a.items) return;
  const int64_t g = item % a.ngc;
  const int64_t t = (item / a.ngc) % a.n;
  const int64_t r = item / (a.ngc * a.n);
  const int64_t xo = r * a.x_rs + t * a.dim + g * a.gc;
  float mn = __builtin_huge_valf(), mx = -__builtin_huge_valf();
  for (int64_t j = 0; j < a.gc; ++j) {
    float v = load1<DT>(a.x, xo + j);
    mn = fminf(mn, v);
    mx = fmaxf(mx, v);
  }
  const float st = ruler_step(mn, mx);
  const float inv = ruler_inv(st);
  const int64_t co = r * a.c_rs + t * a.dim + g * a.gc;
  for (int64_t j = 0; j < a.gc; ++j) a.codes[co + j] = (uint8_t)ruler_code_rcp(load1<DT>(a.x, xo + j), mn, st, inv);
  const int64_t so = r * a.s_rs + t * a.ngc + g;
  a.mins[so] = f2h(mn);
  a.steps[so] = f2h(st);
}

// ---------------------------------------------------------------- dequantize

struct DequantArgs {
  const uint8_t* codes;
  int64_t c_rs;
  const uint16_t* mins;
  const uint16_t* steps;
  int64_t s_rs;
  int64_t rows, n, dim, group, axis;
  void* out;
  int64_t o_rs;
  int64_t items;  // rows * n * dim / 8
};

template <int OT>
__device__ __forceinline__ void store8(void* out, int64_t off, const float (&v)[8]) {
  if (OT == NKV_F16) {
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(out) + off) = pack_h8(v);
  } else if (OT == NKV_BF16) {
    uint4 r;
    r.x = (uint32_t)f2bf(v[0]) | ((uint32_t)f2bf(v[1]) << 16);
    r.y = (uint32_t)f2bf(v[2]) | ((uint32_t)f2bf(v[3]) << 16);
    r.z = (uint32_t)f2bf(v[4]) | ((uint32_t)f2bf(v[5]) << 16);
    r.w = (uint32_t)f2bf(v[6]) | ((uint32_t)f2bf(v[7]) << 16);
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(out) + off) = r;
  } else {
    float4* p = reinterpret_cast<float4*>(static_cast<float*>(out) + off);
    p[0] = make_float4(v[0], v[1], v[2], v[3]);
    p[1] = make_float4(v[4], v[5], v[6], v[7]);
  }
}

template <int OT>
__global__ __launch_bounds__(256) void dequant_kernel(DequantArgs a) {
  const int64_t item = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= a.items) return;
  const int64_t per_row = a.dim / 8;
  const int64_t c8 = (item % per_row) * 8;
  const int64_t t = (item / per_row) % a.n;
  const int64_t r = item / (per_row * a.n);
  const uint2 cw = *reinterpret_cast<const uint2*>(a.codes + r * a.c_rs + t * a.dim + c8);
  float v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t code = ((j < 4 ? cw.x : cw.y) >> (8 * (j & 3))) & 0xffu;
    int64_t so;
    if (a.axis == NKV_AXIS_TOKEN) {
      so = r * a.s_rs + (t / a.group) * a.dim + c8 + j;
    } else {
      const int64_t ngc = a.dim / a.group;
      so = r * a.s_rs + t * ngc + (c8 + j) / a.group;
    }
    // the product of an 8-bit code and an fp16 step is exact in fp32; one rounding in the add
    v[j] = __fadd_rn(__fmul_rn((float)code, h2f(a.steps[so])), h2f(a.mins[so]));
  }
  store8<OT>(a.out, r * a.o_rs + t * a.dim + c8, v);
}

// ---------------------------------------------------------------- per-token symmetric ("tok")

// One (slab, token) row of 128 values per 16-lane row: lane l & 15 quantizes values
// 8 (l & 15) .. + 7 (16-byte loads, 8-byte code stores); a wave covers 4 tokens, a
// 256-thread workgroup 16. The absmax is reduced with DPP within the 16-lane row.
struct QuantSymArgs {
  const void* x;
  int64_t x_rs;
  int64_t rows, n;
  uint8_t* codes;
  int64_t c_rs;
  uint16_t* scales;
  int64_t s_rs;
  int64_t items;  // rows * n
  // page destination (paged cache): token t of slab r is token first_token + t of a sequence,
  // stored in page table[(first_token + t) / 64], KV head r, row (first_token + t) % 64 of
  // tensor `which` (0 K, 1 V) of the page layout [K codes 64 x 128 | V codes | K scales 64 |
  // V scales 64]; tokens whose table entry is outside [0, num_pages) are skipped
  uint8_t* pages;
  const int32_t* table;
  int64_t first_token, num_pages;
  int which;
};

constexpr int64_t PAGE_TOK_BYTES = 2 * 64 * 128 + 2 * 64 * 2;  // 16640

template <int DT, bool PAGES = false>
__global__ __launch_bounds__(256) void quant_sym_kernel(QuantSymArgs a) {
  const int64_t item = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const bool on = item < a.items;  // whole 16-lane rows agree
  const int c8 = (threadIdx.x & 15) * 8;
  const int64_t r = on ? item / a.n : 0, t = on ? item % a.n : 0;
  float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (on) Elem8<DT>::load(a.x, r * a.x_rs + t * 128 + c8, v);
  float scale;
  const uint2 cw = sym_quant8(v, scale);
  if (!on) return;
  uint8_t* code_row = a.codes + r * a.c_rs + t * 128;
  uint16_t* scale_at = a.scales + r * a.s_rs + t;
  if constexpr (PAGES) {
    const int64_t tok = a.first_token + t;
    const int32_t page = a.table[tok / 64];
    if (page < 0 || page >= a.num_pages) return;
    uint8_t* pg = a.pages + ((int64_t)page * a.rows + r) * PAGE_TOK_BYTES;
    code_row = pg + a.which * 64 * 128 + (tok % 64) * 128;
    scale_at = reinterpret_cast<uint16_t*>(pg + 2 * 64 * 128) + a.which * 64 + tok % 64;
  }
  *reinterpret_cast<uint2*>(code_row + c8) = cw;
  if (c8 == 0) *scale_at = f2h(scale);
}

struct DequantSymArgs {
  const uint8_t* codes;
  int64_t c_rs;
  const uint16_t* scales;
  int64_t s_rs;
  int64_t rows, n;
  void* out;
  int64_t o_rs;
  int64_t items;  // rows * n * 16
};

template <int OT>
__global__ __launch_bounds__(256) void dequant_sym_kernel(DequantSymArgs a) {
  const int64_t item = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= a.items) return;
  const int c8 = (int)(item % 16) * 8;
  const int64_t t = (item / 16) % a.n, r = item / (16 * a.n);
  const uint2 cw = *reinterpret_cast<const uint2*>(a.codes + r * a.c_rs + t * 128 + c8);
  const float sc = h2f(a.scales[r * a.s_rs + t]);
  float v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int code = (int)(int8_t)(((j < 4 ? cw.x : cw.y) >> (8 * (j & 3))) & 0xffu);
    v[j] = __fmul_rn((float)code, sc);  // exact in fp32; rounded once by the store
  }
  store8<OT>(a.out, r * a.o_rs + t * 128 + c8, v);
}

// ---------------------------------------------------------------- copy (traffic calibration)

__global__ __launch_bounds__(256) void copy16_kernel(const uint4* __restrict__ src,
                                                     uint4* __restrict__ dst, int64_t n16) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < n16; i += stride) dst[i] = src[i];
}

// Read-only streaming probe: every lane reads 16-byte words with a grid stride and folds
// them into one XOR checksum per workgroup (written so the loads cannot be elided).
__global__ __launch_bounds__(256) void read_bw_kernel(const uint4* __restrict__ src, int64_t n16,
                                                      uint32_t* __restrict__ sink) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  uint32_t x = 0;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const uint4 a = src[i], b = src[i + stride], c = src[i + 2 * stride], d = src[i + 3 * stride];
    x ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
  }
  for (; i < n16; i += stride) {
    const uint4 a = src[i];
    x ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  for (int m = 32; m >= 1; m >>= 1) x ^= (uint32_t)__shfl_xor((int)x, m, 64);
  __shared__ uint32_t part[4];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = x;
  __syncthreads();
  if (threadIdx.x == 0) sink[blockIdx.x] = part[0] ^ part[1] ^ part[2] ^ part[3];
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace nkv

using namespace nkv;

extern "C" int nkv_abi_version(void) { return NKV_ABI_VERSION; }

extern "C" const char* nkv_last_error(void) { return g_err.c_str(); }

extern "C" int nkv_quantize_int8(const void* x, int x_dtype, int64_t x_row_stride, int64_t rows,
                                 int64_t n, int64_t dim, int64_t group, int axis, uint8_t* codes,
                                 int64_t codes_row_stride, uint16_t* mins, uint16_t* steps,
                                 int64_t scale_row_stride, void* stream) {
  g_err.clear();
  if (x_dtype != NKV_F16 && x_dtype != NKV_BF16 && x_dtype != NKV_F32)
    return fail(NKV_ERR_INVALID, "quantize: unknown dtype %d", x_dtype);
  if (rows < 0 || n < 0 || dim <= 0 || group < 0)
    return fail(NKV_ERR_INVALID, "quantize: bad sizes rows=%lld n=%lld dim=%lld group=%lld",
                (long long)rows, (long long)n, (long long)dim, (long long)group);
  if (rows == 0 || n == 0) return NKV_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (axis == NKV_AXIS_TOKEN) {
    const int64_t gs = group ? group : n;
    if (dim % 8) return fail(NKV_ERR_UNSUPPORTED, "quantize: head_dim %lld is not a multiple of 8", (long long)dim);
    const int esz = x_dtype == NKV_F32 ? 4 : 2;
    if (!aligned16(x) || !aligned16(mins) || !aligned16(steps) || (reinterpret_cast<uintptr_t>(codes) & 7u) ||
        (x_row_stride * esz) % 16 || codes_row_stride % 8 || (scale_row_stride * 2) % 16)
      return fail(NKV_ERR_UNSUPPORTED, "quantize: buffers or row strides are not 16-byte aligned");
    QuantTokArgs a{x, x_row_stride, rows, n, dim, gs, cdiv(n, gs), cdiv(dim, 128), codes,
                   codes_row_stride, mins, steps, scale_row_stride, 0};
    a.items = rows * a.ngroups * a.nchunks;
    const dim3 grid((unsigned)cdiv(a.items, kQuantWaves)), block(64 * kQuantWaves);
    const bool cache = gs <= 4 * kCacheRows;
#define NKV_QT(DT)                                                                        \
  if (cache) hipLaunchKernelGGL((quant_token_kernel<DT, true>), grid, block, 0, s, a);    \
  else hipLaunchKernelGGL((quant_token_kernel<DT, false>), grid, block, 0, s, a);
    if (x_dtype == NKV_F16) { NKV_QT(NKV_F16) }
    else if (x_dtype == NKV_BF16) { NKV_QT(NKV_BF16) }
    else { NKV_QT(NKV_F32) }
#undef NKV_QT
    return check_launch("quantize_int8(token)");
  }
  if (axis == NKV_AXIS_CHANNEL) {
    const int64_t gc = group ? group : dim;
    if (dim % gc) return fail(NKV_ERR_INVALID, "head_dim %lld is not divisible by group_size %lld", (long long)dim, (long long)gc);
    QuantChanArgs a{x, x_row_stride, rows, n, dim, gc, dim / gc, codes, codes_row_stride,
                    mins, steps, scale_row_stride, 0};
    a.items = rows * n * a.ngc;
    const dim3 grid((unsigned)cdiv(a.items, 256)), block(256);
    if (x_dtype == NKV_F16) hipLaunchKernelGGL(quant_channel_kernel<NKV_F16>, grid, block, 0, s, a);
    else if (x_dtype == NKV_BF16) hipLaunchKernelGGL(quant_channel_kernel<NKV_BF16>, grid, block, 0, s, a);
    else hipLaunchKernelGGL(quant_channel_kernel<NKV_F32>, grid, block, 0, s, a);
    return check_launch("quantize_int8(channel)");
  }
  return fail(NKV_ERR_INVALID, "axis must be channel (0) or token (1), got %d", axis);
}

extern "C" int nkv_paged_quantize_t64(const void* x, int x_dtype, int64_t x_head_stride, int64_t hkv, int64_t n,
                                      int which, uint8_t* pages, const int32_t* table_row, int64_t first_group,
                                      int64_t num_pages, void* stream) {
  g_err.clear();
  if (x_dtype != NKV_F16 && x_dtype != NKV_BF16 && x_dtype != NKV_F32)
    return fail(NKV_ERR_INVALID, "paged_quantize: unknown dtype %d", x_dtype);
  if (hkv <= 0 || n < 0 || n % 64 || first_group < 0 || (which != 0 && which != 1) || num_pages <= 0)
    return fail(NKV_ERR_INVALID, "paged_quantize: bad sizes hkv=%lld n=%lld (whole groups of 64) first_group=%lld "
                "which=%d num_pages=%lld", (long long)hkv, (long long)n, (long long)first_group, which,
                (long long)num_pages);
  if (n == 0) return NKV_OK;
  if (!x || !pages || !table_row) return fail(NKV_ERR_INVALID, "paged_quantize: null pointer argument");
  const int esz = x_dtype == NKV_F32 ? 4 : 2;
  if (!aligned16(x) || !aligned16(pages) || (x_head_stride * esz) % 16 || x_head_stride < n * 128)
    return fail(NKV_ERR_UNSUPPORTED, "paged_quantize: x must be 16-byte aligned with a head stride >= n * 128");
  QuantTokArgs a{x, x_head_stride, hkv, n, 128, 64, n / 64, 1, nullptr, 0, nullptr, nullptr, 0, 0,
                 pages, table_row, first_group, num_pages, which};
  a.items = hkv * a.ngroups;
  const dim3 grid((unsigned)cdiv(a.items, kQuantWaves)), block(64 * kQuantWaves);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (x_dtype == NKV_F16) hipLaunchKernelGGL((quant_token_kernel<NKV_F16, true, true>), grid, block, 0, s, a);
  else if (x_dtype == NKV_BF16) hipLaunchKernelGGL((quant_token_kernel<NKV_BF16, true, true>), grid, block, 0, s, a);
  else hipLaunchKernelGGL((quant_token_kernel<NKV_F32, true, true>), grid, block, 0, s, a);
  return check_launch("paged_quantize_t64");
}

extern "C" int nkv_dequantize_int8(const uint8_t* codes, int64_t codes_row_stride,
                                   const uint16_t* mins, const uint16_t* steps,
                                   int64_t scale_row_stride, int64_t rows, int64_t n, int64_t dim,
                                   int64_t group, int axis, void* out, int out_dtype,
                                   int64_t out_row_stride, void* stream) {
  g_err.clear();
  if (out_dtype != NKV_F16 && out_dtype != NKV_BF16 && out_dtype != NKV_F32)
    return fail(NKV_ERR_INVALID, "dequantize: unknown dtype %d", out_dtype);
  if (axis != NKV_AXIS_TOKEN && axis != NKV_AXIS_CHANNEL)
    return fail(NKV_ERR_INVALID, "axis must be channel (0) or token (1), got %d", axis);
  if (rows < 0 || n < 0 || dim <= 0 || group < 0) return fail(NKV_ERR_INVALID, "dequantize: bad sizes");
  if (rows == 0 || n == 0) return NKV_OK;
  if (dim % 8) return fail(NKV_ERR_UNSUPPORTED, "dequantize: head_dim %lld is not a multiple of 8", (long long)dim);
  const int64_t g = group ? group : (axis == NKV_AXIS_TOKEN ? n : dim);
  if (axis == NKV_AXIS_CHANNEL && dim % g) return fail(NKV_ERR_INVALID, "head_dim is not divisible by group_size");
  const int esz = out_dtype == NKV_F32 ? 4 : 2;
  if ((reinterpret_cast<uintptr_t>(codes) & 7u) || codes_row_stride % 8 || !aligned16(out) ||
      (out_row_stride * esz) % 16)
    return fail(NKV_ERR_UNSUPPORTED, "dequantize: buffers or row strides are not aligned");
  DequantArgs a{codes, codes_row_stride, mins, steps, scale_row_stride, rows, n, dim, g, axis,
                out, out_row_stride, rows * n * (dim / 8)};
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)cdiv(a.items, 256)), block(256);
  if (out_dtype == NKV_F16) hipLaunchKernelGGL(dequant_kernel<NKV_F16>, grid, block, 0, s, a);
  else if (out_dtype == NKV_BF16) hipLaunchKernelGGL(dequant_kernel<NKV_BF16>, grid, block, 0, s, a);
  else hipLaunchKernelGGL(dequant_kernel<NKV_F32>, grid, block, 0, s, a);
  return check_launch("dequantize_int8");
}

extern "C" int nkv_quantize_tok(const void* x, int x_dtype, int64_t x_row_stride, int64_t rows, int64_t n,
                                int64_t dim, int8_t* codes, int64_t codes_row_stride, uint16_t* scales,
                                int64_t scale_row_stride, void* stream) {
  g_err.clear();
  if (x_dtype != NKV_F16 && x_dtype != NKV_BF16 && x_dtype != NKV_F32)
    return fail(NKV_ERR_INVALID, "quantize_tok: unknown dtype %d", x_dtype);
  if (rows < 0 || n < 0 || dim <= 0)
    return fail(NKV_ERR_INVALID, "quantize_tok: bad sizes rows=%lld n=%lld dim=%lld", (long long)rows,
                (long long)n, (long long)dim);
  if (dim != 128) return fail(NKV_ERR_UNSUPPORTED, "quantize_tok: head_dim %lld (only 128 is built)", (long long)dim);
  if (rows == 0 || n == 0) return NKV_OK;
  const int esz = x_dtype == NKV_F32 ? 4 : 2;
  if (!x || !codes || !scales || !aligned16(x) || (reinterpret_cast<uintptr_t>(codes) & 7u) ||
      (reinterpret_cast<uintptr_t>(scales) & 1u) || (x_row_stride * esz) % 16 || codes_row_stride % 8)
    return fail(NKV_ERR_UNSUPPORTED, "quantize_tok: buffers or row strides are not aligned");
  QuantSymArgs a{x, x_row_stride, rows, n, reinterpret_cast<uint8_t*>(codes), codes_row_stride, scales,
                 scale_row_stride, rows * n};
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)cdiv(a.items, 16)), block(256);
  if (x_dtype == NKV_F16) hipLaunchKernelGGL(quant_sym_kernel<NKV_F16>, grid, block, 0, s, a);
  else if (x_dtype == NKV_BF16) hipLaunchKernelGGL(quant_sym_kernel<NKV_BF16>, grid, block, 0, s, a);
  else hipLaunchKernelGGL(quant_sym_kernel<NKV_F32>, grid, block, 0, s, a);
  return check_launch("quantize_tok");
}

extern "C" int nkv_paged_quantize_tok(const void* x, int x_dtype, int64_t x_head_stride, int64_t hkv, int64_t n,
                                      int which, uint8_t* pages, const int32_t* table_row, int64_t first_token,
                                      int64_t num_pages, void* stream) {
  g_err.clear();
  if (x_dtype != NKV_F16 && x_dtype != NKV_BF16 && x_dtype != NKV_F32)
    return fail(NKV_ERR_INVALID, "paged_quantize_tok: unknown dtype %d", x_dtype);
  if (hkv <= 0 || n < 0 || first_token < 0 || (which != 0 && which != 1) || num_pages <= 0)
    return fail(NKV_ERR_INVALID, "paged_quantize_tok: bad sizes hkv=%lld n=%lld first_token=%lld which=%d "
                "num_pages=%lld", (long long)hkv, (long long)n, (long long)first_token, which, (long long)num_pages);
  if (n == 0) return NKV_OK;
  if (!x || !pages || !table_row) return fail(NKV_ERR_INVALID, "paged_quantize_tok: null pointer argument");
  const int esz = x_dtype == NKV_F32 ? 4 : 2;
  if (!aligned16(x) || !aligned16(pages) || (x_head_stride * esz) % 16 || x_head_stride < n * 128)
    return fail(NKV_ERR_UNSUPPORTED, "paged_quantize_tok: x must be 16-byte aligned with a head stride >= n * 128");
  QuantSymArgs a{x, x_head_stride, hkv, n, nullptr, 0, nullptr, 0, hkv * n, pages, table_row, first_token,
                 num_pages, which};
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)cdiv(a.items, 16)), block(256);
  if (x_dtype == NKV_F16) hipLaunchKernelGGL((quant_sym_kernel<NKV_F16, true>), grid, block, 0, s, a);
  else if (x_dtype == NKV_BF16) hipLaunchKernelGGL((quant_sym_kernel<NKV_BF16, true>), grid, block, 0, s, a);
  else hipLaunchKernelGGL((quant_sym_kernel<NKV_F32, true>), grid, block, 0, s, a);
  return check_launch("paged_quantize_tok");
}

extern "C" int nkv_dequantize_tok(const int8_t* codes, int64_t codes_row_stride, const uint16_t* scales,
                                  int64_t scale_row_stride, int64_t rows, int64_t n, int64_t dim, void* out,
                                  int out_dtype, int64_t out_row_stride, void* stream) {
  g_err.clear();
  if (out_dtype != NKV_F16 && out_dtype != NKV_BF16 && out_dtype != NKV_F32)
    return fail(NKV_ERR_INVALID, "dequantize_tok: unknown dtype %d", out_dtype);
  if (rows < 0 || n < 0 || dim <= 0) return fail(NKV_ERR_INVALID, "dequantize_tok: bad sizes");
  if (dim != 128) return fail(NKV_ERR_UNSUPPORTED, "dequantize_tok: head_dim %lld (only 128 is built)", (long long)dim);
  if (rows == 0 || n == 0) return NKV_OK;
  const int esz = out_dtype == NKV_F32 ? 4 : 2;
  if (!codes || !scales || !out || (reinterpret_cast<uintptr_t>(codes) & 7u) || codes_row_stride % 8 ||
      !aligned16(out) || (out_row_stride * esz) % 16)
    return fail(NKV_ERR_UNSUPPORTED, "dequantize_tok: buffers or row strides are not aligned");
  DequantSymArgs a{reinterpret_cast<const uint8_t*>(codes), codes_row_stride, scales, scale_row_stride, rows, n,
                   out, out_row_stride, rows * n * 16};
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)cdiv(a.items, 256)), block(256);
  if (out_dtype == NKV_F16) hipLaunchKernelGGL(dequant_sym_kernel<NKV_F16>, grid, block, 0, s, a);
  else if (out_dtype == NKV_BF16) hipLaunchKernelGGL(dequant_sym_kernel<NKV_BF16>, grid, block, 0, s, a);
  else hipLaunchKernelGGL(dequant_sym_kernel<NKV_F32>, grid, block, 0, s, a);
  return check_launch("dequantize_tok");
}

extern "C" int nkv_copy_bytes(const void* src, void* dst, int64_t nbytes, void* stream) {
  g_err.clear();
  if (nbytes < 0 || nbytes % 16 || !aligned16(src) || !aligned16(dst))
    return fail(NKV_ERR_INVALID, "copy: nbytes must be a multiple of 16 and buffers 16-byte aligned");
  if (nbytes == 0) return NKV_OK;
  const int64_t n16 = nbytes / 16;
  const unsigned blocks = (unsigned)std::min<int64_t>(cdiv(n16, 256), 2048);
  hipLaunchKernelGGL(copy16_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint4*>(src), static_cast<uint4*>(dst), n16);
  return check_launch("copy_bytes");
}

extern "C" int nkv_read_bw(const void* src, int64_t nbytes, uint32_t* sink, int64_t blocks, void* stream) {
  g_err.clear();
  if (!src || !sink || nbytes <= 0 || nbytes % 16 || !aligned16(src))
    return fail(NKV_ERR_INVALID, "read_bw: nbytes must be a positive multiple of 16 and src 16-byte aligned");
  if (blocks <= 0 || blocks > (1 << 20)) return fail(NKV_ERR_INVALID, "read_bw: blocks must be in [1, 2^20]");
  hipLaunchKernelGGL(read_bw_kernel, dim3((unsigned)blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint4*>(src), nbytes / 16, sink);
  return check_launch("read_bw");
}
