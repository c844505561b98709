// Split-K int8 decode attention, ring append and the fused decode step (gfx950, wave64).
//
// Work decomposition. One launch covers one layer. Workgroup `bid` serves KV head
// `bid % hkv` (with 8 KV heads every workgroup of a head lands on the same XCD, so
// its partials stay in one L2) and part `bid / hkv`. Parts 0..n_parts-1 split the
// whole 64-token groups of the int8 prefix evenly; part n_parts (when present) is
// the ring worker: it appends the new token and requantizes the ring (fused step),
// then attends over the ring or over the group the ring just completed. Each of
// the 4 waves of a workgroup runs its own online softmax over every 4th group of
// the workgroup's range; the waves merge through LDS, the workgroup writes one
// (m, l, acc) partial, and the last workgroup of the head to finish (an atomic
// counter that it also resets) merges the partials and writes out / lse.
//
// Per 64-token group and wave (D = 128, up to 16 query heads per KV head):
//   S^T[token][head] = K[token][:] . Q[head][:]  — 4 token blocks x 8 k-steps of
//     v_mfma_f32_16x16x16f16; K rows are dequantized in registers with packed
//     fp16 math: fp16(code * step16 + min16) with one rounding (the reference
//     computes the same product exactly in fp32 and rounds the sum to fp16).
//   online softmax in the log2 domain, fp32, over the 16 scores a lane holds.
//   O[head][dim] += P[head][token] . V[token][dim] — P is split into two fp16
//     halves (hi + lo, scaled by 2^15 so small weights keep 22 bits) and V codes
//     are byte-transposed in registers into the MFMA B layout.
// The P operand of the PV product is exactly the S^T output layout, so no data
// moves between the two products.
#include "nkv_common.h"

namespace nkv {

constexpr int D = 128;
constexpr int GT = 64;      // tokens per ruler group == ring slots
constexpr int WAVES = 4;    // waves per workgroup
constexpr int THREADS = 64 * WAVES;
constexpr float P_SCALE = 32768.0f;       // 2^15
constexpr float INV_P_SCALE = 1.0f / 32768.0f;
constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;
constexpr float NEG_INF = -__builtin_huge_valf();

enum TailMode : int { TAIL_NONE = 0, TAIL_MASK = 1, TAIL_SCALARS = 2, TAIL_FUSED = 3 };

struct AttnArgs {
  const uint16_t* q;
  uint8_t* kq;
  uint16_t* kmn;
  uint16_t* kst;
  uint8_t* vq;
  uint16_t* vmn;
  uint16_t* vst;
  uint16_t* tail_k;
  uint16_t* tail_v;
  const uint8_t* tail_mask;  // TAIL_MASK
  const int64_t* used_dev;
  const int64_t* pg_dev;
  const int64_t* written_dev;
  const int64_t* first_dev;
  const int64_t* pos_dev;  // TAIL_FUSED
  int64_t* written_out;
  int64_t* qlen_out;
  int64_t* pg_out;
  const uint16_t* k_new;
  const uint16_t* v_new;
  int64_t kv_hs;
  int64_t used, pg;  // host values when the device pointers are null
  int64_t capacity, ngroups_cap;
  int64_t tail_slots;
  int hq, hkv, gq;
  int n_parts, nslots;
  int tail_mode;
  float sl2;  // softmax scale * log2(e)
  uint16_t* out;
  float* lse;
  float* ws;
  uint32_t* counters;
};

// Online-softmax state of one wave. m, l: head (lane & 15), log2 domain.
// acc[cb][i]: head 4*(lane>>4) + i, dim 8*(lane&15) + cb, scaled by 2^15.
struct WaveState {
  float m, l;
  float4_t acc[8];
};

__device__ __forceinline__ void state_init(WaveState& st) {
  st.m = NEG_INF;
  st.l = 0.0f;
#pragma unroll
  for (int cb = 0; cb < 8; ++cb) st.acc[cb] = float4_t{0.f, 0.f, 0.f, 0.f};
}

__device__ __forceinline__ half2_t bcast_half(uint32_t w, int hi) {
  return as_h2(perm(w, w, hi ? 0x03020302u : 0x01000100u));
}

// Q as the MFMA B operand: lane (c, g) holds head c's dims 16g + 64hh + 4j + [0..3]
// for k-step 4hh + j (zero rows for c >= gq).
__device__ __forceinline__ void load_q(const AttnArgs& a, int h, half4_t (&qb)[8]) {
  const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    uint4 w0 = {0, 0, 0, 0}, w1 = {0, 0, 0, 0};
    if (c < a.gq) {
      const uint16_t* row = a.q + (int64_t)(h * a.gq + c) * D + 16 * g + 64 * hh;
      w0 = *reinterpret_cast<const uint4*>(row);
      w1 = *reinterpret_cast<const uint4*>(row + 8);
    }
    const uint32_t w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const half2_t lo = as_h2(w[2 * j]), hi = as_h2(w[2 * j + 1]);
      qb[4 * hh + j] = half4_t{lo.x, lo.y, hi.x, hi.y};
    }
  }
}

// Online-softmax update with the 16 masked scores s[b][i] (token 16b + 4g + i, head c),
// returns P split into hi/lo fp16 A operands and rescales the accumulator.
__device__ __forceinline__ void softmax_step(WaveState& st, float (&s)[4][4], half4_t (&phi)[4],
                                             half4_t (&plo)[4]) {
  const int lane = threadIdx.x & 63, g = lane >> 4;
  float mloc = NEG_INF;
#pragma unroll
  for (int b = 0; b < 4; ++b)
#pragma unroll
    for (int i = 0; i < 4; ++i) mloc = fmaxf(mloc, s[b][i]);
  mloc = fmaxf(mloc, shfl_xor(mloc, 16));
  mloc = fmaxf(mloc, shfl_xor(mloc, 32));
  const float m_new = fmaxf(st.m, mloc);
  const float m_use = m_new == NEG_INF ? 0.0f : m_new;
  const float alpha = __builtin_amdgcn_exp2f(st.m - m_use);
  float lsum = 0.0f;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[i] = __builtin_amdgcn_exp2f(s[b][i] - m_use);
      lsum += p[i];
    }
    const float q0 = p[0] * P_SCALE, q1 = p[1] * P_SCALE, q2 = p[2] * P_SCALE, q3 = p[3] * P_SCALE;
    const half2_t h01 = __builtin_bit_cast(half2_t, __builtin_amdgcn_cvt_pkrtz(q0, q1));
    const half2_t h23 = __builtin_bit_cast(half2_t, __builtin_amdgcn_cvt_pkrtz(q2, q3));
    const half2_t l01 = __builtin_bit_cast(half2_t, __builtin_amdgcn_cvt_pkrtz(q0 - (float)h01.x, q1 - (float)h01.y));
    const half2_t l23 = __builtin_bit_cast(half2_t, __builtin_amdgcn_cvt_pkrtz(q2 - (float)h23.x, q3 - (float)h23.y));
    phi[b] = half4_t{h01.x, h01.y, h23.x, h23.y};
    plo[b] = half4_t{l01.x, l01.y, l23.x, l23.y};
  }
  lsum += shfl_xor(lsum, 16);
  lsum += shfl_xor(lsum, 32);
  st.l = st.l * alpha + lsum;
  st.m = m_new;
  // accumulator rows belong to head 4g + i; its alpha sits in lane 4g + i
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float ai = shfl(alpha, 4 * g + i);
#pragma unroll
    for (int cb = 0; cb < 8; ++cb) st.acc[cb][i] *= ai;
  }
}

// One 64-token group of the int8 cache: tokens [t0, t0 + 64) of head h, `nvalid` of them
// valid. Rows at or beyond `capacity` are never loaded.
__device__ __forceinline__ void attend_group_int8(const AttnArgs& a, WaveState& st,
                                                  const half4_t (&qb)[8], int h, int64_t grp,
                                                  int nvalid) {
  const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
  const int64_t t0 = grp * GT;
  const int64_t last = a.capacity - 1;
  const uint8_t* kq_h = a.kq + (int64_t)h * a.capacity * D;
  const uint8_t* vq_h = a.vq + (int64_t)h * a.capacity * D;
  const int64_t ro = ((int64_t)h * a.ngroups_cap + grp) * D;

  // ---- loads
  uint4 kc[4][2];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int64_t row = min(t0 + 16 * b + c, last);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
      kc[b][hh] = *reinterpret_cast<const uint4*>(kq_h + row * D + 16 * g + 64 * hh);
  }
  uint2 vc[4][4];
#pragma unroll
  for (int b = 0; b < 4; ++b)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t row = min(t0 + 16 * b + 4 * g + r, last);
      vc[b][r] = *reinterpret_cast<const uint2*>(vq_h + row * D + 8 * c);
    }
  uint32_t ksw[2][8], kmw[2][8];
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const uint4* ps = reinterpret_cast<const uint4*>(a.kst + ro + 16 * g + 64 * hh);
    const uint4* pm = reinterpret_cast<const uint4*>(a.kmn + ro + 16 * g + 64 * hh);
    const uint4 s0 = ps[0], s1 = ps[1], m0 = pm[0], m1 = pm[1];
    ksw[hh][0] = s0.x; ksw[hh][1] = s0.y; ksw[hh][2] = s0.z; ksw[hh][3] = s0.w;
    ksw[hh][4] = s1.x; ksw[hh][5] = s1.y; ksw[hh][6] = s1.z; ksw[hh][7] = s1.w;
    kmw[hh][0] = m0.x; kmw[hh][1] = m0.y; kmw[hh][2] = m0.z; kmw[hh][3] = m0.w;
    kmw[hh][4] = m1.x; kmw[hh][5] = m1.y; kmw[hh][6] = m1.z; kmw[hh][7] = m1.w;
  }
  const uint4 vsu = *reinterpret_cast<const uint4*>(a.vst + ro + 8 * c);
  const uint4 vmu = *reinterpret_cast<const uint4*>(a.vmn + ro + 8 * c);

  // ---- S^T = K Q^T
  float4_t S[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    S[b] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const uint32_t kw[4] = {kc[b][hh].x, kc[b][hh].y, kc[b][hh].z, kc[b][hh].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const half2_t k01 = __builtin_elementwise_fma(codes_to_h2(kw[j], kSelB01),
                                                      as_h2(ksw[hh][2 * j]), as_h2(kmw[hh][2 * j]));
        const half2_t k23 = __builtin_elementwise_fma(codes_to_h2(kw[j], kSelB23),
                                                      as_h2(ksw[hh][2 * j + 1]), as_h2(kmw[hh][2 * j + 1]));
        S[b] = __builtin_amdgcn_mfma_f32_16x16x16f16(half4_t{k01.x, k01.y, k23.x, k23.y},
                                                     qb[4 * hh + j], S[b], 0, 0, 0);
      }
    }
  }
  float s[4][4];
#pragma unroll
  for (int b = 0; b < 4; ++b)
#pragma unroll
    for (int i = 0; i < 4; ++i) s[b][i] = (16 * b + 4 * g + i) < nvalid ? S[b][i] * a.sl2 : NEG_INF;

  half4_t phi[4], plo[4];
  softmax_step(st, s, phi, plo);

  // ---- O += P V. Invalid tokens carry p = 0; their codes are zeroed so that a
  // garbage ruler cannot turn 0 * v into NaN.
  const uint32_t vsw[4] = {vsu.x, vsu.y, vsu.z, vsu.w};
  const uint32_t vmw[4] = {vmu.x, vmu.y, vmu.z, vmu.w};
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool ok = (16 * b + 4 * g + r) < nvalid;
      lo[r] = ok ? vc[b][r].x : 0u;
      hi[r] = ok ? vc[b][r].y : 0u;
    }
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const uint32_t w0 = half ? hi[0] : lo[0], w1 = half ? hi[1] : lo[1];
      const uint32_t w2 = half ? hi[2] : lo[2], w3 = half ? hi[3] : lo[3];
      const uint32_t t01a = perm(w1, w0, 0x05010400u), t01b = perm(w1, w0, 0x07030602u);
      const uint32_t t23a = perm(w3, w2, 0x05010400u), t23b = perm(w3, w2, 0x07030602u);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int cb = 4 * half + k;
        const uint32_t x01 = (k < 2) ? t01a : t01b;
        const uint32_t x23 = (k < 2) ? t23a : t23b;
        const uint32_t sel = (k & 1) ? kSelB23 : kSelB01;
        const half2_t stp = bcast_half(vsw[cb >> 1], cb & 1);
        const half2_t mnp = bcast_half(vmw[cb >> 1], cb & 1);
        const half2_t v01 = __builtin_elementwise_fma(codes_to_h2(x01, sel), stp, mnp);
        const half2_t v23 = __builtin_elementwise_fma(codes_to_h2(x23, sel), stp, mnp);
        const half4_t vb = half4_t{v01.x, v01.y, v23.x, v23.y};
        st.acc[cb] = __builtin_amdgcn_mfma_f32_16x16x16f16(phi[b], vb, st.acc[cb], 0, 0, 0);
        st.acc[cb] = __builtin_amdgcn_mfma_f32_16x16x16f16(plo[b], vb, st.acc[cb], 0, 0, 0);
      }
    }
  }
}

// The fp16 ring (slots [0, tail_slots)) of head h; slot validity from `valid_bits`
// (bit i = slot i takes part).
__device__ __forceinline__ void attend_ring_f16(const AttnArgs& a, WaveState& st,
                                                const half4_t (&qb)[8], int h, uint64_t valid_bits) {
  const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
  const int64_t last = a.tail_slots - 1;
  const uint16_t* k_h = a.tail_k + (int64_t)h * a.tail_slots * D;
  const uint16_t* v_h = a.tail_v + (int64_t)h * a.tail_slots * D;

  float4_t S[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    S[b] = float4_t{0.f, 0.f, 0.f, 0.f};
    const int64_t row = min((int64_t)(16 * b + c), last);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const uint4* p = reinterpret_cast<const uint4*>(k_h + row * D + 16 * g + 64 * hh);
      const uint4 w0 = p[0], w1 = p[1];
      const uint32_t w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const half2_t lo = as_h2(w[2 * j]), hi = as_h2(w[2 * j + 1]);
        S[b] = __builtin_amdgcn_mfma_f32_16x16x16f16(half4_t{lo.x, lo.y, hi.x, hi.y},
                                                     qb[4 * hh + j], S[b], 0, 0, 0);
      }
    }
  }
  float s[4][4];
#pragma unroll
  for (int b = 0; b < 4; ++b)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int slot = 16 * b + 4 * g + i;
      s[b][i] = ((valid_bits >> slot) & 1ull) ? S[b][i] * a.sl2 : NEG_INF;
    }
  half4_t phi[4], plo[4];
  softmax_step(st, s, phi, plo);

#pragma unroll
  for (int b = 0; b < 4; ++b) {
    uint4 vr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int slot = 16 * b + 4 * g + r;
      const int64_t row = min((int64_t)slot, last);
      vr[r] = *reinterpret_cast<const uint4*>(v_h + row * D + 8 * c);
      if (!((valid_bits >> slot) & 1ull)) vr[r] = uint4{0, 0, 0, 0};
    }
#pragma unroll
    for (int cb = 0; cb < 8; ++cb) {
      const uint32_t sel = (cb & 1) ? 0x07060302u : 0x05040100u;
      const int wi = cb >> 1;
      const uint32_t w0 = wi == 0 ? vr[0].x : wi == 1 ? vr[0].y : wi == 2 ? vr[0].z : vr[0].w;
      const uint32_t w1 = wi == 0 ? vr[1].x : wi == 1 ? vr[1].y : wi == 2 ? vr[1].z : vr[1].w;
      const uint32_t w2 = wi == 0 ? vr[2].x : wi == 1 ? vr[2].y : wi == 2 ? vr[2].z : vr[2].w;
      const uint32_t w3 = wi == 0 ? vr[3].x : wi == 1 ? vr[3].y : wi == 2 ? vr[3].z : vr[3].w;
      const half2_t v01 = as_h2(perm(w1, w0, sel)), v23 = as_h2(perm(w3, w2, sel));
      const half4_t vb = half4_t{v01.x, v01.y, v23.x, v23.y};
      st.acc[cb] = __builtin_amdgcn_mfma_f32_16x16x16f16(phi[b], vb, st.acc[cb], 0, 0, 0);
      st.acc[cb] = __builtin_amdgcn_mfma_f32_16x16x16f16(plo[b], vb, st.acc[cb], 0, 0, 0);
    }
  }
}

// Requantize the ring of one tensor (K or V) of head h into ruler group `gcur`, after
// writing the new token into slot `slot`. One wave: lanes (l & 15) own 8 channels,
// lanes (l >> 4) own rows (l >> 4) + 4i. Same arithmetic as the bulk quantizer.
__device__ __forceinline__ void append_ring_tensor(uint16_t* ring_h, const uint16_t* new_h,
                                                   uint8_t* codes_h, uint16_t* mn_g, uint16_t* st_g,
                                                   int slot, int64_t gcur, int64_t capacity) {
  const int lane = threadIdx.x & 63, cl = lane & 15, rl = lane >> 4;
  uint4 rows[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int r = rl + 4 * i;
    if (r == slot) {
      rows[i] = *reinterpret_cast<const uint4*>(new_h + 8 * cl);
      *reinterpret_cast<uint4*>(ring_h + r * D + 8 * cl) = rows[i];
    } else {
      rows[i] = *reinterpret_cast<const uint4*>(ring_h + r * D + 8 * cl);
    }
  }
  float mn[8], mx[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) { mn[j] = __builtin_huge_valf(); mx[j] = -__builtin_huge_valf(); }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t w[4] = {rows[i].x, rows[i].y, rows[i].z, rows[i].w};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float v = h2f((uint16_t)(w[j >> 1] >> (16 * (j & 1))));
      mn[j] = fminf(mn[j], v);
      mx[j] = fmaxf(mx[j], v);
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    mn[j] = fminf(mn[j], shfl_xor(mn[j], 16));
    mn[j] = fminf(mn[j], shfl_xor(mn[j], 32));
    mx[j] = fmaxf(mx[j], shfl_xor(mx[j], 16));
    mx[j] = fmaxf(mx[j], shfl_xor(mx[j], 32));
  }
  float stp[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) stp[j] = ruler_step(mn[j], mx[j]);
  if (rl == 0) {
    uint4 m4, s4;
    m4.x = (uint32_t)f2h(mn[0]) | ((uint32_t)f2h(mn[1]) << 16);
    m4.y = (uint32_t)f2h(mn[2]) | ((uint32_t)f2h(mn[3]) << 16);
    m4.z = (uint32_t)f2h(mn[4]) | ((uint32_t)f2h(mn[5]) << 16);
    m4.w = (uint32_t)f2h(mn[6]) | ((uint32_t)f2h(mn[7]) << 16);
    s4.x = (uint32_t)f2h(stp[0]) | ((uint32_t)f2h(stp[1]) << 16);
    s4.y = (uint32_t)f2h(stp[2]) | ((uint32_t)f2h(stp[3]) << 16);
    s4.z = (uint32_t)f2h(stp[4]) | ((uint32_t)f2h(stp[5]) << 16);
    s4.w = (uint32_t)f2h(stp[6]) | ((uint32_t)f2h(stp[7]) << 16);
    *reinterpret_cast<uint4*>(mn_g + 8 * cl) = m4;
    *reinterpret_cast<uint4*>(st_g + 8 * cl) = s4;
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int r = rl + 4 * i;
    const int64_t t = gcur * GT + r;
    if (t < capacity) {
      const uint32_t w[4] = {rows[i].x, rows[i].y, rows[i].z, rows[i].w};
      uint32_t cc[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) cc[j] = ruler_code(h2f((uint16_t)(w[j >> 1] >> (16 * (j & 1)))), mn[j], stp[j]);
      uint2 o;
      o.x = cc[0] | (cc[1] << 8) | (cc[2] << 16) | (cc[3] << 24);
      o.y = cc[4] | (cc[5] << 8) | (cc[6] << 16) | (cc[7] << 24);
      *reinterpret_cast<uint2*>(codes_h + t * D + 8 * cl) = o;
    }
  }
}

__device__ __forceinline__ void append_head(const AttnArgs& a, int h, int which, int64_t pos) {
  const int slot = (int)(pos % GT);
  const int64_t gcur = pos / GT;
  const int64_t ro = ((int64_t)h * a.ngroups_cap + gcur) * D;
  if (which == 0)
    append_ring_tensor(a.tail_k + (int64_t)h * GT * D, a.k_new + h * a.kv_hs, a.kq + (int64_t)h * a.capacity * D,
                       a.kmn + ro, a.kst + ro, slot, gcur, a.capacity);
  else
    append_ring_tensor(a.tail_v + (int64_t)h * GT * D, a.v_new + h * a.kv_hs, a.vq + (int64_t)h * a.capacity * D,
                       a.vmn + ro, a.vst + ro, slot, gcur, a.capacity);
}

__device__ __forceinline__ void write_scalars(const AttnArgs& a, int64_t pos) {
  const int64_t written = pos + 1;
  const int64_t qlen = written / GT * GT;
  *a.written_out = written;
  *a.qlen_out = qlen;
  *a.pg_out = qlen / GT;
}

// Slot validity of the ring: slot i holds p = u - ((u - i) mod 64), valid iff qlen <= p <= u, p >= first.
__device__ __forceinline__ uint64_t ring_bits(int64_t written, int64_t qlen, int64_t first) {
  const int64_t u = written - 1;
  uint64_t bits = 0;
  for (int i = 0; i < GT; ++i) {
    int64_t d = (u - i) % GT;
    if (d < 0) d += GT;
    const int64_t p = u - d;
    if (p >= qlen && p <= u && p >= first) bits |= 1ull << i;
  }
  return bits;
}

// ---------------------------------------------------------------- the kernel

__global__ __launch_bounds__(THREADS, 2) void attn_decode_kernel(AttnArgs a) {
  extern __shared__ float lds[];
  __shared__ int s_last;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int h = blockIdx.x % a.hkv;
  const int part = blockIdx.x / a.hkv;
  const bool is_tail = part == a.n_parts;

  WaveState st;
  state_init(st);
  half4_t qb[8];
  load_q(a, h, qb);

  // token limit of the int8 prefix and where the ring stands
  int64_t U;
  int64_t pos = 0;
  bool pos_ok = true;
  if (a.tail_mode == TAIL_FUSED) {
    pos = *a.pos_dev;
    pos_ok = pos >= 0 && pos < a.capacity;  // a position outside the cache appends nothing
    U = pos_ok ? pos / GT * GT : 0;         // whole groups before the ring's group
  } else {
    const int64_t used = a.used_dev ? *a.used_dev : a.used;
    const int64_t pgv = a.pg_dev ? *a.pg_dev : a.pg;
    U = min(used, pgv * GT);
  }
  U = max<int64_t>(0, min(U, a.ngroups_cap * GT));

  if (!is_tail) {
    const int64_t W = (U + GT - 1) / GT;
    const int64_t gs = (int64_t)part * W / a.n_parts;
    const int64_t ge = (int64_t)(part + 1) * W / a.n_parts;
    for (int64_t grp = gs + wave; grp < ge; grp += WAVES) {
      const int nvalid = (int)min<int64_t>(GT, U - grp * GT);
      attend_group_int8(a, st, qb, h, grp, nvalid);
    }
  } else {
    if (a.tail_mode == TAIL_FUSED && pos_ok) {
      if (wave < 2) append_head(a, h, wave, pos);
      if (h == 0 && tid == 0) write_scalars(a, pos);
      __threadfence_block();
      __syncthreads();
      if (wave == 0) {
        const int64_t written = pos + 1;
        const int64_t qlen = written / GT * GT;
        if (qlen > U) {
          attend_group_int8(a, st, qb, h, pos / GT, GT);  // the ring just completed its group
        } else {
          const int64_t first = a.first_dev ? *a.first_dev : 0;
          attend_ring_f16(a, st, qb, h, ring_bits(written, qlen, first));
        }
      }
    } else if (a.tail_mode != TAIL_FUSED && wave == 0) {
      uint64_t bits;
      if (a.tail_mode == TAIL_MASK) {
        bits = 0;
        for (int i = 0; i < a.tail_slots; ++i) bits |= (uint64_t)(a.tail_mask[i] != 0) << i;
      } else {
        const int64_t written = *a.written_dev;
        const int64_t first = a.first_dev ? *a.first_dev : 0;
        bits = ring_bits(written, U, first);
      }
      attend_ring_f16(a, st, qb, h, bits);
    }
  }

  // ---- merge the waves through LDS: per wave [m: gq][l: gq][acc: gq * D]
  const int gq = a.gq;
  const int pw = gq * (D + 2);
  float* lw = lds + wave * pw;
  {
    const int c = lane & 15, g = lane >> 4;
    if (g == 0 && c < gq) { lw[c] = st.m; lw[gq + c] = st.l; }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int head = 4 * g + i;
      if (head < gq)
#pragma unroll
        for (int cb = 0; cb < 8; ++cb) lw[2 * gq + head * D + 8 * c + cb] = st.acc[cb][i];
    }
  }
  __syncthreads();
  const int nslots = a.nslots;
  float* part_ws = a.ws + ((int64_t)h * nslots + part) * pw;
  for (int e = tid; e < gq * D; e += THREADS) {
    const int head = e / D;
    float m = NEG_INF;
    for (int w = 0; w < WAVES; ++w) m = fmaxf(m, lds[w * pw + head]);
    const float mu = m == NEG_INF ? 0.0f : m;
    float acc = 0.0f, l = 0.0f;
    for (int w = 0; w < WAVES; ++w) {
      const float wt = __builtin_amdgcn_exp2f(lds[w * pw + head] - mu);
      acc += lds[w * pw + 2 * gq + e] * wt;
      l += lds[w * pw + gq + head] * wt;
    }
    part_ws[2 * gq + e] = acc;
    if ((e % D) == 0) { part_ws[head] = m; part_ws[gq + head] = l; }
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(a.counters + h, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == (uint32_t)(nslots - 1);
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();

  // ---- last workgroup of head h: merge all partials of the head
  float* wts = lds;               // [nslots][gq] weights
  float* mh = lds + nslots * gq;  // [gq] merged max
  const float* head_ws = a.ws + (int64_t)h * nslots * pw;
  if (tid < gq) {
    float m = NEG_INF;
    for (int s = 0; s < nslots; ++s) m = fmaxf(m, __builtin_nontemporal_load(head_ws + (int64_t)s * pw + tid));
    mh[tid] = m;
  }
  __syncthreads();
  for (int e = tid; e < nslots * gq; e += THREADS) {
    const int s = e / gq, head = e % gq;
    const float m = mh[head];
    const float ms = __builtin_nontemporal_load(head_ws + (int64_t)s * pw + head);
    wts[e] = ms == NEG_INF ? 0.0f : __builtin_amdgcn_exp2f(ms - m);
  }
  __syncthreads();
  for (int e = tid; e < gq * D; e += THREADS) {
    const int head = e / D;
    float acc = 0.0f, l = 0.0f;
    for (int s = 0; s < nslots; ++s) {
      const float wt = wts[s * gq + head];
      acc += __builtin_nontemporal_load(head_ws + (int64_t)s * pw + 2 * gq + e) * wt;
      l += __builtin_nontemporal_load(head_ws + (int64_t)s * pw + gq + head) * wt;
    }
    const int qh = h * gq + head;
    a.out[(int64_t)qh * D + (e % D)] = f2h(l > 0.0f ? acc / l * INV_P_SCALE : 0.0f);
    if (a.lse && (e % D) == 0) a.lse[qh] = l > 0.0f ? (mh[head] + __log2f(l)) * LN2 : NEG_INF;
  }
  if (tid == 0) __hip_atomic_store(a.counters + h, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Standalone append (two waves per KV head: K and V).
__global__ __launch_bounds__(128) void append_kernel(AttnArgs a) {
  const int h = blockIdx.x;
  const int64_t pos = *a.pos_dev;
  if (pos < 0 || pos >= a.capacity) return;  // a position outside the cache appends nothing
  append_head(a, h, threadIdx.x >> 6, pos);
  if (h == 0 && threadIdx.x == 0) write_scalars(a, pos);
}

__global__ void ring_mask_kernel(const int64_t* written, const int64_t* qlen, const int64_t* first,
                                 int64_t slots, uint8_t* mask) {
  const int i = threadIdx.x;
  if (i >= slots) return;
  const int64_t u = *written - 1;
  int64_t d = (u - i) % slots;
  if (d < 0) d += slots;
  const int64_t p = u - d;
  mask[i] = (p >= *qlen && p <= u && p >= (first ? *first : 0)) ? 1 : 0;
}

// ---------------------------------------------------------------- host side

static int64_t default_parts(int64_t hkv, int64_t groups) {
  // about 2 workgroups per CU over the 256 CUs of an MI355X, at least 2 groups per part
  const int64_t target_wgs = 512;
  int64_t parts = std::max<int64_t>(1, target_wgs / std::max<int64_t>(1, hkv));
  parts = std::min<int64_t>(parts, std::max<int64_t>(1, groups / 2));
  return parts;
}

static int64_t part_floats(int64_t hq, int64_t hkv) { return (hq / hkv) * (D + 2); }

static size_t lds_bytes(int gq, int nslots) {
  const size_t merge = (size_t)WAVES * gq * (D + 2) * sizeof(float);
  const size_t final_ = ((size_t)nslots * gq + gq) * sizeof(float);
  return std::max(merge, final_);
}

static int check_heads(int64_t hq, int64_t hkv, int64_t head_dim) {
  if (hkv <= 0 || hq <= 0 || hq % hkv) return fail(NKV_ERR_INVALID, "Q heads %lld not divisible by KV heads %lld", (long long)hq, (long long)hkv);
  if (hq / hkv > 16) return fail(NKV_ERR_INVALID, "%lld Q heads per KV head exceeds the padding limit 16", (long long)(hq / hkv));
  if (head_dim != D) return fail(NKV_ERR_UNSUPPORTED, "head_dim %lld: the HIP kernels are built for head_dim 128", (long long)head_dim);
  return NKV_OK;
}

static int launch_attn(AttnArgs& a, int64_t n_parts, int64_t workspace_bytes, hipStream_t s, const char* what) {
  a.n_parts = (int)n_parts;
  a.nslots = (int)(n_parts + (a.tail_mode != TAIL_NONE ? 1 : 0));
  const int64_t need = (int64_t)a.hkv * a.nslots * part_floats(a.hq, a.hkv) * (int64_t)sizeof(float);
  if (workspace_bytes < need) return fail(NKV_ERR_INVALID, "%s: workspace of %lld bytes, need %lld", what, (long long)workspace_bytes, (long long)need);
  const size_t shm = lds_bytes(a.gq, a.nslots);
  if (shm > 64 * 1024) return fail(NKV_ERR_UNSUPPORTED, "%s: n_parts %lld needs too much LDS", what, (long long)n_parts);
  hipLaunchKernelGGL(attn_decode_kernel, dim3((unsigned)(a.hkv * a.nslots)), dim3(THREADS), shm, s, a);
  return check_launch(what);
}

static bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace nkv

using namespace nkv;

extern "C" int64_t nkv_attn_workspace_bytes(int64_t hkv, int64_t hq, int64_t n_parts) {
  if (hkv <= 0 || hq <= 0 || n_parts < 0) return 0;
  return hkv * (n_parts + 1) * part_floats(hq, hkv) * (int64_t)sizeof(float);
}

extern "C" int64_t nkv_attn_default_parts(int64_t hkv, int64_t groups) { return default_parts(hkv, groups); }

extern "C" int nkv_attn_decode_t64(const uint16_t* q, const uint8_t* kq, const uint16_t* kmn,
                                   const uint16_t* kst, const uint8_t* vq, const uint16_t* vmn,
                                   const uint16_t* vst, int64_t hq, int64_t hkv, int64_t head_dim,
                                   int64_t capacity, int64_t used, int64_t prefix_groups,
                                   const int64_t* used_dev, const int64_t* prefix_groups_dev,
                                   const uint16_t* tail_k, const uint16_t* tail_v,
                                   const int64_t* written_dev, const int64_t* first_dev,
                                   uint16_t* out, float* lse_out, void* workspace,
                                   int64_t workspace_bytes, uint32_t* counters, int64_t n_parts,
                                   void* stream) {
  set_error("");
  if (int rc = check_heads(hq, hkv, head_dim)) return rc;
  if (capacity <= 0) return fail(NKV_ERR_INVALID, "capacity must be positive");
  if (!q || !kq || !kmn || !kst || !vq || !vmn || !vst || !out || !workspace || !counters)
    return fail(NKV_ERR_INVALID, "attn_decode: null pointer argument");
  if (!al16(q) || !al16(kq) || !al16(vq) || !al16(kmn) || !al16(kst) || !al16(vmn) || !al16(vst))
    return fail(NKV_ERR_UNSUPPORTED, "attn_decode: buffers must be 16-byte aligned");
  if ((tail_k == nullptr) != (tail_v == nullptr)) return fail(NKV_ERR_INVALID, "tail_k and tail_v go together");
  if (tail_k && !written_dev) return fail(NKV_ERR_INVALID, "the ring needs written_dev");
  if (!used_dev && (used < 0 || used > capacity)) return fail(NKV_ERR_INVALID, "used=%lld outside [0, %lld]", (long long)used, (long long)capacity);
  const int64_t ngroups = cdiv(capacity, GT);
  if ((used_dev == nullptr) != (prefix_groups_dev == nullptr))
    return fail(NKV_ERR_INVALID, "used_dev and prefix_groups_dev go together");
  int64_t pg = prefix_groups;
  if (!prefix_groups_dev) {
    if (pg < 0) pg = cdiv(used, GT);
    if (pg > ngroups) return fail(NKV_ERR_INVALID, "prefix_groups=%lld exceeds the %lld rulers", (long long)pg, (long long)ngroups);
  }
  if (n_parts <= 0) n_parts = default_parts(hkv, used_dev ? ngroups : cdiv(std::min(used, pg * GT), GT));
  AttnArgs a{};
  a.q = q; a.kq = const_cast<uint8_t*>(kq); a.kmn = const_cast<uint16_t*>(kmn); a.kst = const_cast<uint16_t*>(kst);
  a.vq = const_cast<uint8_t*>(vq); a.vmn = const_cast<uint16_t*>(vmn); a.vst = const_cast<uint16_t*>(vst);
  a.tail_k = const_cast<uint16_t*>(tail_k); a.tail_v = const_cast<uint16_t*>(tail_v);
  a.used_dev = used_dev; a.pg_dev = prefix_groups_dev; a.written_dev = written_dev; a.first_dev = first_dev;
  a.used = used; a.pg = pg; a.capacity = capacity; a.ngroups_cap = ngroups; a.tail_slots = GT;
  a.hq = (int)hq; a.hkv = (int)hkv; a.gq = (int)(hq / hkv);
  a.tail_mode = tail_k ? TAIL_SCALARS : TAIL_NONE;
  a.sl2 = LOG2E / sqrtf((float)head_dim);
  a.out = out; a.lse = lse_out; a.ws = static_cast<float*>(workspace); a.counters = counters;
  return launch_attn(a, n_parts, workspace_bytes, static_cast<hipStream_t>(stream), "attn_decode_t64");
}

extern "C" int nkv_append_t64(const uint16_t* k_new, const uint16_t* v_new, int64_t kv_head_stride,
                              uint8_t* kq, uint16_t* kmn, uint16_t* kst, uint8_t* vq, uint16_t* vmn,
                              uint16_t* vst, uint16_t* tail_k, uint16_t* tail_v, const int64_t* pos_dev,
                              int64_t* written_dev, int64_t* qlen_dev, int64_t* pg_dev, int64_t hkv,
                              int64_t head_dim, int64_t capacity, void* stream) {
  set_error("");
  if (head_dim != D) return fail(NKV_ERR_UNSUPPORTED, "head_dim %lld: the HIP kernels are built for head_dim 128", (long long)head_dim);
  if (hkv <= 0 || capacity <= 0) return fail(NKV_ERR_INVALID, "append: bad sizes");
  if (!k_new || !v_new || !kq || !kmn || !kst || !vq || !vmn || !vst || !tail_k || !tail_v || !pos_dev ||
      !written_dev || !qlen_dev || !pg_dev)
    return fail(NKV_ERR_INVALID, "append: null pointer argument");
  if (!al16(k_new) || !al16(v_new) || kv_head_stride % 8 || !al16(tail_k) || !al16(tail_v) || !al16(kq) || !al16(vq))
    return fail(NKV_ERR_UNSUPPORTED, "append: buffers must be 16-byte aligned");
  AttnArgs a{};
  a.k_new = k_new; a.v_new = v_new; a.kv_hs = kv_head_stride;
  a.kq = kq; a.kmn = kmn; a.kst = kst; a.vq = vq; a.vmn = vmn; a.vst = vst;
  a.tail_k = tail_k; a.tail_v = tail_v; a.pos_dev = pos_dev;
  a.written_out = written_dev; a.qlen_out = qlen_dev; a.pg_out = pg_dev;
  a.capacity = capacity; a.ngroups_cap = cdiv(capacity, GT); a.hkv = (int)hkv;
  hipLaunchKernelGGL(append_kernel, dim3((unsigned)hkv), dim3(128), 0, static_cast<hipStream_t>(stream), a);
  return check_launch("append_t64");
}

extern "C" int nkv_decode_step_t64(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                                   int64_t kv_head_stride, uint8_t* kq, uint16_t* kmn, uint16_t* kst,
                                   uint8_t* vq, uint16_t* vmn, uint16_t* vst, uint16_t* tail_k,
                                   uint16_t* tail_v, const int64_t* pos_dev, const int64_t* first_dev,
                                   int64_t* written_dev, int64_t* qlen_dev, int64_t* pg_dev, int64_t hq,
                                   int64_t hkv, int64_t head_dim, int64_t capacity, uint16_t* out,
                                   float* lse_out, void* workspace, int64_t workspace_bytes,
                                   uint32_t* counters, int64_t n_parts, void* stream) {
  set_error("");
  if (int rc = check_heads(hq, hkv, head_dim)) return rc;
  if (capacity <= 0) return fail(NKV_ERR_INVALID, "capacity must be positive");
  if (!q || !k_new || !v_new || !kq || !kmn || !kst || !vq || !vmn || !vst || !tail_k || !tail_v ||
      !pos_dev || !written_dev || !qlen_dev || !pg_dev || !out || !workspace || !counters)
    return fail(NKV_ERR_INVALID, "decode_step: null pointer argument");
  if (!al16(q) || !al16(k_new) || !al16(v_new) || kv_head_stride % 8 || !al16(tail_k) || !al16(tail_v) ||
      !al16(kq) || !al16(vq) || !al16(kmn) || !al16(kst) || !al16(vmn) || !al16(vst))
    return fail(NKV_ERR_UNSUPPORTED, "decode_step: buffers must be 16-byte aligned");
  const int64_t ngroups = cdiv(capacity, GT);
  if (n_parts <= 0) n_parts = default_parts(hkv, ngroups);
  AttnArgs a{};
  a.q = q; a.k_new = k_new; a.v_new = v_new; a.kv_hs = kv_head_stride;
  a.kq = kq; a.kmn = kmn; a.kst = kst; a.vq = vq; a.vmn = vmn; a.vst = vst;
  a.tail_k = tail_k; a.tail_v = tail_v; a.pos_dev = pos_dev; a.first_dev = first_dev;
  a.written_out = written_dev; a.qlen_out = qlen_dev; a.pg_out = pg_dev;
  a.capacity = capacity; a.ngroups_cap = ngroups; a.tail_slots = GT;
  a.hq = (int)hq; a.hkv = (int)hkv; a.gq = (int)(hq / hkv);
  a.tail_mode = TAIL_FUSED;
  a.sl2 = LOG2E / sqrtf((float)head_dim);
  a.out = out; a.lse = lse_out; a.ws = static_cast<float*>(workspace); a.counters = counters;
  return launch_attn(a, n_parts, workspace_bytes, static_cast<hipStream_t>(stream), "decode_step_t64");
}

extern "C" int nkv_tail_attend(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                               const uint8_t* mask, int64_t hq, int64_t hkv, int64_t head_dim,
                               int64_t slots, uint16_t* out, float* lse, void* workspace,
                               int64_t workspace_bytes, uint32_t* counters, void* stream) {
  set_error("");
  if (int rc = check_heads(hq, hkv, head_dim)) return rc;
  if (slots <= 0 || slots > GT) return fail(NKV_ERR_UNSUPPORTED, "tail_attend: %lld slots (1..64 supported)", (long long)slots);
  if (!q || !k || !v || !mask || !out || !workspace || !counters) return fail(NKV_ERR_INVALID, "tail_attend: null pointer argument");
  if (!al16(q) || !al16(k) || !al16(v)) return fail(NKV_ERR_UNSUPPORTED, "tail_attend: buffers must be 16-byte aligned");
  AttnArgs a{};
  a.q = q; a.tail_k = const_cast<uint16_t*>(k); a.tail_v = const_cast<uint16_t*>(v); a.tail_mask = mask;
  a.capacity = 1; a.ngroups_cap = 1; a.tail_slots = slots;
  a.hq = (int)hq; a.hkv = (int)hkv; a.gq = (int)(hq / hkv);
  a.tail_mode = TAIL_MASK;
  a.sl2 = LOG2E / sqrtf((float)head_dim);
  a.out = out; a.lse = lse; a.ws = static_cast<float*>(workspace); a.counters = counters;
  return launch_attn(a, 0, workspace_bytes, static_cast<hipStream_t>(stream), "tail_attend");
}

extern "C" int nkv_ring_mask(const int64_t* written_dev, const int64_t* qlen_dev, const int64_t* first_dev,
                             int64_t slots, uint8_t* mask, void* stream) {
  set_error("");
  if (!written_dev || !qlen_dev || !mask) return fail(NKV_ERR_INVALID, "ring_mask: null pointer argument");
  if (slots <= 0 || slots > 1024) return fail(NKV_ERR_INVALID, "ring_mask: %lld slots", (long long)slots);
  hipLaunchKernelGGL(ring_mask_kernel, dim3(1), dim3((unsigned)slots), 0, static_cast<hipStream_t>(stream),
                     written_dev, qlen_dev, first_dev, slots, mask);
  return check_launch("ring_mask");
}
