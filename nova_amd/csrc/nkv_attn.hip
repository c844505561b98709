// Split-K int8 decode attention, ring append and the fused decode step (gfx950, wave64).
//
// Work decomposition. One layer is two launches on one stream.
//   Prefix kernel: workgroup `bid` serves KV head `bid % hkv` and part `bid / hkv` and
//     streams its share of the whole 64-token groups of the int8 prefix into one
//     partial (m, l, acc per query head). With 8 KV heads, consecutive workgroups land
//     on the 8 XCDs round-robin, so every workgroup of a head runs on one XCD. In the
//     fused step, the new token's append (ring slot, requantization of the ring into
//     the current group: 4 units of 64 channels of K or V per head) runs in parts 0..3
//     ahead of their streams; the prefix never reads the group it writes.
//   Tail kernel: one workgroup per KV head attends over the fp16 ring (or over the group
//     the new token completed) and merges all partials by log-sum-exp into out / lse.
//     The launch boundary orders the partials and the append before it.
//
// Streaming. Each of the 8 waves of a prefix workgroup owns every 8th group of the
// workgroup's range and a private LDS stage. A group is moved HBM -> LDS by 20
// asynchronous `global_load_lds_dwordx4` (K codes 8 x 1 KiB, V codes 8 x 1 KiB, the four
// fp16 rulers 4 x 256 B). Those loads are issued from inline assembly, and the wave waits
// for them with an explicit `s_waitcnt vmcnt(n)`: left to the compiler, a wait for all
// outstanding loads would be placed before every LDS read and serialize the stream.
// Rows are stored with their 16-byte chunks XOR-swizzled by `swz(row)`, which makes
// both LDS read patterns below free of bank conflicts.
//
// Per 64-token group and wave (D = 128, up to 16 query heads per KV head):
//   S^T[token][head] = K[token][:] . Q[head][:] — 4 token blocks x 4 k-steps of
//     v_mfma_f32_16x16x32_f16. K codes are read with ds_read_b128 and dequantized in
//     registers with packed fp16 math: fp16(code * step16 + min16), one rounding.
//   online softmax in the log2 domain, fp32, over the 16 scores a lane holds.
//   O[head][dim] += P[head][token] . V[token][dim] — 2 token blocks of 32 x 8 dim
//     blocks. P is split into two fp16 halves (hi + lo, scaled by 2^15 so that small
//     weights keep 22 bits). ds_read_b64_tr_b8 delivers the V codes already
//     transposed into the MFMA B layout (8 tokens of one dim per lane), so all 8 codes
//     of a lane share one ruler.
// The P operand of the PV product is exactly the S^T output layout of two token
// blocks, so no data moves between the two products.
#include "nkv_common.h"

#include <mutex>
#include <vector>

namespace nkv {

#ifndef NKV_WAVES
#define NKV_WAVES 8
#endif


constexpr int D = 128;
constexpr int GT = 64;              // tokens per ruler group == ring slots
constexpr int WAVES = NKV_WAVES;    // waves per workgroup
constexpr int THREADS = 64 * WAVES;
constexpr int CODE_BYTES = GT * D;                        // one tensor's codes of one group
constexpr int RULER_BYTES = 4 * D * 2;                    // kst, kmn, vst, vmn of one group
constexpr int HALF_CODE = 32 * D;                          // one tensor's codes of a half group
constexpr int HALF_SLOT = 2 * HALF_CODE;                   // K | V codes of a half group
constexpr int WAVE_LDS = 2 * HALF_SLOT + 2 * RULER_BYTES;  // two slots + two ruler sets
constexpr int LDS_BYTES = WAVES * WAVE_LDS;                // 144 KiB
constexpr int DMA_FIRST_HALF = 2 * (HALF_CODE / 1024) + 4; // with the group's rulers
constexpr int DMA_SECOND_HALF = 2 * (HALF_CODE / 1024);
// the per-token symmetric format: a half-group slot holds K and V codes and the 32 K and
// 32 V fp16 scales of its tokens
constexpr int TOK_SCALE_BYTES = 32 * 2;
constexpr int HALF_SLOT_TOK = 2 * HALF_CODE + 2 * TOK_SCALE_BYTES;
constexpr int WAVE_LDS_TOK = 2 * HALF_SLOT_TOK;
constexpr int LDS_BYTES_TOK = WAVES * WAVE_LDS_TOK;        // 130 KiB
constexpr int DMA_HALF_TOK = 2 * (HALF_CODE / 1024) + 2;
constexpr int RING_BYTES = GT * D * 2;                    // one fp16 ring tensor of one head
// paged layout: one page = one 64-token group of one KV head, K codes | V codes | kst | kmn | vst | vmn
constexpr int PAGE_BYTES = 2 * CODE_BYTES + RULER_BYTES;  // 17 KiB, a multiple of 128
constexpr int DMA_FIRST_HALF_PAGED = 2 * (HALF_CODE / 1024) + 1;  // the rulers are one 1 KiB load
// paged per-token symmetric layout: one page = 64 tokens of one KV head, K codes | V codes |
// K scales (64 fp16) | V scales
constexpr int PAGE_TOK_BYTES = 2 * CODE_BYTES + 2 * GT * 2;  // 16640, a multiple of 128
enum Layout : int { CONTIG_T64 = 0, CONTIG_TOK = 1, PAGED_T64 = 2, PAGED_TOK = 3 };
constexpr float P_SCALE_LOG2 = 15.0f;  // the softmax weights carry a factor 2^15
constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;
constexpr float NEG_INF = -__builtin_huge_valf();

static_assert(DMA_FIRST_HALF == 12 && DMA_SECOND_HALF == 8 && DMA_HALF_TOK == 10, "loads per half group");
static_assert(PAGE_BYTES % 128 == 0 && PAGE_TOK_BYTES % 128 == 0, "pages are 128-byte aligned");
static_assert(LDS_BYTES <= 150 * 1024 && LDS_BYTES_TOK <= 150 * 1024, "LDS of one workgroup");

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef int v2i_t __attribute__((vector_size(8)));
typedef __attribute__((address_space(3))) v2i_t lds_v2i_t;

enum TailMode : int { TAIL_NONE = 0, TAIL_MASK = 1, TAIL_SCALARS = 2, TAIL_FUSED = 3 };
// TAIL_FUSED with `tok`: the new token itself is the tail (its codes written by the prefix kernel).

constexpr int FLAG_COPIES = 8;  // copies of the chained step's issue flags (one per polling KV head group)

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
  uint16_t* ksc;  // per-token symmetric format: fp16 scales [hkv, capacity]
  uint16_t* vsc;
  int tok;        // 1: per-token symmetric int8 codes and scales, 0: int8t64
  // paged batch (int8t64): pages [num_pages][hkv][PAGE_BYTES], page table [nseq][table_stride],
  // rings [nseq][hkv][K, V][64][D], pos_dev [nseq]; prefix work unit w serves sequence
  // wg_map[w] >> 16, part wg_map[w] & 0xffff of seq_parts[2b + 1] starting at unit seq_parts[2b]
  uint8_t* pages;
  const int32_t* table;
  int64_t table_stride;
  int64_t num_pages;   // page ids outside [0, num_pages) (e.g. -1, unassigned) are no page
  uint16_t* rings;
  const int32_t* wg_map;
  const int32_t* seq_parts;
  int nseq, total_parts;
  int64_t kv_ss;  // k_new / v_new sequence stride (elements)
  int64_t kv_hs;
  int64_t used, pg;  // host values when the device pointers are null
  int64_t capacity, ngroups_cap;
  int64_t tail_slots;
  int hq, hkv, gq;
  int n_parts;
  int tail_mode;
  float sl2;  // softmax scale * log2(e)
  uint16_t* out;
  float* lse;
  float* ws;
  // fused tail: the last prefix workgroup of each head runs the tail. Its ticket comes from
  // counter i = head (paged: sequence * hkv + head) at tail_ctr_end[-1 - i], the workspace's
  // last bytes; the counters start at zero and every launch leaves them at zero.
  int inline_tail;
  int* tail_ctr_end;
  // the chained step: this layer's output also as tagged words (two fp16 values in the low 32
  // bits, `ftag` in the high 32) for the next layer's inputs that are views of it; null otherwise
  uint64_t* fwd_out;
  uint32_t ftag;
  // the chained step's dependency between layers: 0, a forwarded input waits only for the words
  // it reads (written by its own head's merger); 1, every input of layer l also waits until every
  // head's merger has finished layer l - 1
  int dep_all;
  // the paged int8t64 decode step: the tail of each (sequence, KV head) also appends the new token
  // (its ring slot, and the requantized group of pos in its page), so no append launch precedes it
  int tail_append;
  // the chained step with dep_all: this layer's issue flags, one word per query head, set to the
  // launch's tag (relaxed, agent scope) as soon as that head's output stores are issued; the
  // readers of layer l + 1 wait until all hq carry the tag. Null otherwise.
  uint32_t* issue_flags;
  uint32_t* flags_base;  // layer 0's issue flags; layer l's at flags_base + l FLAG_COPIES hq
  int n_layers;
  // the L2 hand-over: l2_xcc = the device's XCD count n when workgroups b and b + n share an XCD
  // and n divides hkv (the workgroups of a KV head then share one XCD), 0 when off
  int l2_xcc;
  // the fused projection step (attn_prefix_kernel with QKV): the layer's input x [hidden] and its
  // RMSNorm gamma, the stacked projection w_qkv [(hq + 2 hkv) D][hidden], the q/k head-norm
  // gammas [D], the RoPE frequencies [D / 2]; hand: the tagged row words [hkv][QKV_HAND_ROWS],
  // qkv_epoch [hkv]: the tags' source per KV head; qkv_out: the normalized and rotated q / k and
  // v [(hq + 2 hkv) D], or null
  const uint16_t* x;
  const uint16_t* x_gamma;
  const uint16_t* w_qkv;
  const uint16_t* q_gamma;
  const uint16_t* k_gamma;
  const float* inv_freq;
  float eps_x, eps_qk;
  int hidden;
  uint64_t* hand;
  int* qkv_epoch;
  uint16_t* qkv_out;
  // the fused projection step with the output projection: w_o [hidden][hq D] and h1 = x + w_o out
  // [hidden] (the merging workgroups publish out as tagged words through fwd_out, stored at agent
  // scope (fwd_agent) since every workgroup reads every head's words, with issue_flags)
  const uint16_t* w_o;
  uint16_t* h1_out;
  int fwd_agent;
};

// XOR key of the 16-byte chunk positions of LDS row `row` (a token within its group).
// K reads (16 consecutive rows, one chunk) and V transpose reads (rows 4g + {0..3} of
// two 16-row blocks, one chunk) both hit 16 distinct bank positions per 16 lanes.
__device__ __forceinline__ int swz(int row) { return ((row >> 1) & 7) ^ (((row >> 4) & 1) << 2); }

// fp16 ring tensor in LDS: row r (256 B) keeps its 16-byte chunk c at position c ^ (r & 15),
// so the 16 rows a K operand read touches land on 16 distinct banks.
__device__ __forceinline__ int ring_chunk_pos(int row, int chunk) { return chunk ^ (row & 15); }

// Reductions over the 4 lanes {l, l^16, l^32, l^48} with the gfx950 permlane swaps (VALU
// only, no LDS round trip). permlane16_swap(x, x) returns rows (0,0,2,2) and (1,1,3,3) of
// x, permlane32_swap(x, x) its lower and upper halves twice.
__device__ __forceinline__ float max4rows(float v) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float sum4rows(float v) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Online-softmax state of one wave. m, l: head (lane & 15), log2 domain; m is a reference
// maximum (at least every score seen so far, times sl2), the weights are 2^(s sl2 - m + 15).
// acc[cb][i]: head 4*(lane>>4) + i, dim 16*cb + (lane&15), in the same scale.
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

__device__ __forceinline__ float4_t mfma32(half8_t a, half8_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ half8_t as_h8(uint4 w) { return __builtin_bit_cast(half8_t, w); }

// 8 codes (bytes of w0, w1) -> fp16(code * st + mn) per element, rulers per element.
__device__ __forceinline__ half8_t dq8(uint32_t w0, uint32_t w1, uint4 st, uint4 mn) {
  const half2_t a = __builtin_elementwise_fma(codes_to_h2(w0, kSelB01), as_h2(st.x), as_h2(mn.x));
  const half2_t b = __builtin_elementwise_fma(codes_to_h2(w0, kSelB23), as_h2(st.y), as_h2(mn.y));
  const half2_t c = __builtin_elementwise_fma(codes_to_h2(w1, kSelB01), as_h2(st.z), as_h2(mn.z));
  const half2_t d = __builtin_elementwise_fma(codes_to_h2(w1, kSelB23), as_h2(st.w), as_h2(mn.w));
  return half8_t{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
}

// 8 codes sharing one ruler (st, mn given as half2 splats).
__device__ __forceinline__ half8_t dq8_splat(uint32_t w0, uint32_t w1, half2_t st, half2_t mn) {
  const half2_t a = __builtin_elementwise_fma(codes_to_h2(w0, kSelB01), st, mn);
  const half2_t b = __builtin_elementwise_fma(codes_to_h2(w0, kSelB23), st, mn);
  const half2_t c = __builtin_elementwise_fma(codes_to_h2(w1, kSelB01), st, mn);
  const half2_t d = __builtin_elementwise_fma(codes_to_h2(w1, kSelB23), st, mn);
  return half8_t{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
}

// The thread index for code that runs once per layer (the tails, the chained step's merger):
// read through an opaque move, so that values derived from it are recomputed where they are used
// rather than hoisted out of the chained kernel's layer loop and kept live across it (which
// exhausts the register file there).
__device__ __forceinline__ int tail_tid() {
  int t;
  asm volatile("v_mov_b32 %0, %1" : "=v"(t) : "v"((int)__builtin_amdgcn_workitem_id_x()));
  return t;
}

// Q as the B operand of v_mfma_f32_16x16x32_f16: lane (c, g) holds head c's dims
// 16g + 64hh + 8e + [0..7] for k-step 2hh + e (zeros for c >= gq).
__device__ __forceinline__ void load_q(const uint16_t* qh, int gq, half8_t (&qb)[4]) {
  const int lane = tail_tid() & 63, c = lane & 15, g = lane >> 4;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    uint4 w = {0, 0, 0, 0};
    if (c < gq) w = *reinterpret_cast<const uint4*>(qh + c * D + 16 * g + 64 * (k >> 1) + 8 * (k & 1));
    qb[k] = as_h8(w);
  }
  // Make the compiler complete these loads here, before the untracked LDS streams start:
  // a wait it placed later would also wait for every group in flight.
  asm volatile("" ::"v"(qb[0]), "v"(qb[1]), "v"(qb[2]), "v"(qb[3]));
}

// ---------------------------------------------------------------- HBM -> LDS streaming

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const lds_void_t*)p;
}

// A pointer the wave holds in common, moved to scalar registers.
__device__ __forceinline__ const void* uniform_ptr(const void* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<const void*>(((uint64_t)hi << 32) | lo);
}

// One `global_load_lds_dwordx4`: lane L's 16 bytes at sbase + voff land at LDS byte
// address lds + 16 * L (sbase and lds are wave-uniform).
__device__ __forceinline__ void dma16(const void* sbase, uint32_t voff, uint32_t lds) {
  lds = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds) : "memory");
}

// The same, nontemporal: for the decode prefix's codes and rulers, which a step reads once
// (about 3-5% faster than the default policy on the 32k decode step).
__device__ __forceinline__ void dma16_stream(const void* sbase, uint32_t voff, uint32_t lds) {
  lds = __builtin_amdgcn_readfirstlane(lds);
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(voff), "s"(sbase), "s"(lds) : "memory");
}

// Issue the loads of half `hf` (tokens 32 hf .. 32 hf + 31) of group `grp` of head h: 32
// K and 32 V code rows (4 + 4 loads) into the slot at `slot` (K codes, then V codes), and
// with `with_rulers` (by default for hf == 0) the group's rulers (4 loads) into `rs`. Rows are swizzled as in a full
// stage; token rows at or beyond the capacity are never read (the last row is repeated).
// Lane `lane`'s byte offset within a half's rows for load j: row 8 j + lane / 8, its 16-byte
// chunk lane % 8 at the swizzled position (the same for every half, so the compiler keeps the
// four offsets in registers across the streaming loop).
__device__ __forceinline__ uint32_t half_row_off(int lane, int j) {
  const int row = 8 * j + (lane >> 3);
  return (uint32_t)(row * D) + (((lane & 7) ^ swz(row)) << 4);
}

__device__ __forceinline__ void issue_half(const AttnArgs& a, int h, int64_t grp, int hf, uint32_t slot, uint32_t rs,
                                           bool with_rulers) {
  const int lane = threadIdx.x & 63;
  const int64_t t0 = grp * GT + 32 * hf;
  slot = __builtin_amdgcn_readfirstlane(slot);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // earlier reads of this slot are done
  if (t0 + 32 <= a.capacity) {
    // the half's rows from the half's first row on: per-lane offsets that do not change
    const void* kb = uniform_ptr(a.kq + ((int64_t)h * a.capacity + t0) * D);
    const void* vb = uniform_ptr(a.vq + ((int64_t)h * a.capacity + t0) * D);
#pragma unroll
    for (int j = 0; j < 4; ++j) dma16_stream(kb, half_row_off(lane, j), slot + 1024 * j);
#pragma unroll
    for (int j = 0; j < 4; ++j) dma16_stream(vb, half_row_off(lane, j), slot + HALF_CODE + 1024 * j);
  } else {
    // (a half that reaches the capacity: rows clamped to the last one; the opaque lane keeps
    // the compiler from precomputing these offsets for every fixed group and holding them)
    const void* kb = uniform_ptr(a.kq + (int64_t)h * a.capacity * D);
    const void* vb = uniform_ptr(a.vq + (int64_t)h * a.capacity * D);
    const int olane = tail_tid() & 63;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = 8 * j + (olane >> 3);
      const uint32_t off = (uint32_t)(min<int64_t>(t0 + row, a.capacity - 1) * D) + (((olane & 7) ^ swz(row)) << 4);
      dma16_stream(kb, off, slot + 1024 * j);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = 8 * j + (olane >> 3);
      const uint32_t off = (uint32_t)(min<int64_t>(t0 + row, a.capacity - 1) * D) + (((olane & 7) ^ swz(row)) << 4);
      dma16_stream(vb, off, slot + HALF_CODE + 1024 * j);
    }
  }
  if (with_rulers) {
    rs = __builtin_amdgcn_readfirstlane(rs);
    const int64_t ro = ((int64_t)h * a.ngroups_cap + grp) * D;
    const uint32_t roff = (uint32_t)(8 * (lane & 15)) * 2;
    const int which = lane >> 4;
    if (which == 0) dma16_stream(uniform_ptr(a.kst + ro), roff, rs);
    if (which == 1) dma16_stream(uniform_ptr(a.kmn + ro), roff, rs);
    if (which == 2) dma16_stream(uniform_ptr(a.vst + ro), roff, rs);
    if (which == 3) dma16_stream(uniform_ptr(a.vmn + ro), roff, rs);
  }
}
__device__ __forceinline__ void issue_half(const AttnArgs& a, int h, int64_t grp, int hf, uint32_t slot, uint32_t rs) {
  issue_half(a, h, grp, hf, slot, rs, hf == 0);
}

// The code rows of one tensor (K or V) of half `hf` of group `grp` (4 loads into `dst`), and a
// group's rulers (4 loads into `rs`): issue_half in pieces, for the chained step's pipelined
// loop, which reloads a K slot and a V slot at different times.
__device__ __forceinline__ void issue_rows(const uint8_t* codes, const AttnArgs& a, int h, int64_t grp, int hf,
                                           uint32_t dst) {
  const int lane = threadIdx.x & 63;
  const int64_t t0 = grp * GT + 32 * hf;
  dst = __builtin_amdgcn_readfirstlane(dst);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // earlier reads of this slot are done
  if (t0 + 32 <= a.capacity) {
    const void* b = uniform_ptr(codes + ((int64_t)h * a.capacity + t0) * D);
#pragma unroll
    for (int j = 0; j < 4; ++j) dma16_stream(b, half_row_off(lane, j), dst + 1024 * j);
  } else {
    const void* b = uniform_ptr(codes + (int64_t)h * a.capacity * D);
    const int olane = tail_tid() & 63;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = 8 * j + (olane >> 3);
      const uint32_t off = (uint32_t)(min<int64_t>(t0 + row, a.capacity - 1) * D) + (((olane & 7) ^ swz(row)) << 4);
      dma16_stream(b, off, dst + 1024 * j);
    }
  }
}
__device__ __forceinline__ void issue_rulers(const AttnArgs& a, int h, int64_t grp, uint32_t rs) {
  const int lane = threadIdx.x & 63;
  rs = __builtin_amdgcn_readfirstlane(rs);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  const int64_t ro = ((int64_t)h * a.ngroups_cap + grp) * D;
  const uint32_t roff = (uint32_t)(8 * (lane & 15)) * 2;
  const int which = lane >> 4;
  if (which == 0) dma16_stream(uniform_ptr(a.kst + ro), roff, rs);
  if (which == 1) dma16_stream(uniform_ptr(a.kmn + ro), roff, rs);
  if (which == 2) dma16_stream(uniform_ptr(a.vst + ro), roff, rs);
  if (which == 3) dma16_stream(uniform_ptr(a.vmn + ro), roff, rs);
}

// s_waitcnt vmcnt(n) for a wave-uniform n in {0, 4, 8, 12, 16}
__device__ __forceinline__ void vm_wait_n(int n) {
  if (n <= 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  else if (n == 4) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
  else if (n == 8) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  else if (n == 12) asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
}

// The per-token symmetric format's half group: 32 K and 32 V code rows (4 + 4 loads) into
// the slot, then the 32 K and 32 V scales of those tokens (one load each, 4 lanes).
// Token rows stay below the capacity (a multiple of 64 in this format).
__device__ __forceinline__ void issue_half_tok(const AttnArgs& a, int h, int64_t grp, int hf, uint32_t slot) {
  const int lane = threadIdx.x & 63;
  const int64_t t0 = grp * GT + 32 * hf;
  const void* kb = uniform_ptr(a.kq + ((int64_t)h * a.capacity + t0) * D);
  const void* vb = uniform_ptr(a.vq + ((int64_t)h * a.capacity + t0) * D);
  slot = __builtin_amdgcn_readfirstlane(slot);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // earlier reads of this slot are done
#pragma unroll
  for (int j = 0; j < 4; ++j) dma16_stream(kb, half_row_off(lane, j), slot + 1024 * j);
#pragma unroll
  for (int j = 0; j < 4; ++j) dma16_stream(vb, half_row_off(lane, j), slot + HALF_CODE + 1024 * j);
  if (lane < 4) dma16_stream(uniform_ptr(a.ksc + (int64_t)h * a.capacity + t0), 16u * lane, slot + 2 * HALF_CODE);
  if (lane < 4) dma16_stream(uniform_ptr(a.vsc + (int64_t)h * a.capacity + t0), 16u * lane, slot + 2 * HALF_CODE + TOK_SCALE_BYTES);
}

// Page of group `grp` of sequence b, or -1 when the table has no valid page there (an entry
// outside [0, num_pages), such as the -1 of an unassigned or released slot).
__device__ __forceinline__ int64_t page_of(const AttnArgs& a, int b, int64_t grp) {
  if (grp < 0 || grp >= a.table_stride) return -1;
  const int32_t page = a.table[(int64_t)b * a.table_stride + grp];
  return page >= 0 && page < a.num_pages ? page : -1;
}

// The paged layout's half group: the group's page holds K code rows, V code rows and the
// four rulers contiguously; 4 + 4 loads of code rows and, with hf == 0, one 1 KiB load of
// the rulers (kst | kmn | vst | vmn, the order of a ruler set in LDS).
__device__ __forceinline__ void issue_half_paged(const AttnArgs& a, int b, int h, int64_t grp, int hf, uint32_t slot,
                                                 uint32_t rs) {
  const int lane = threadIdx.x & 63;
  // a prefix group's page is valid whenever the current group's is (pages are reserved from
  // group 0 up); should the table say otherwise, page 0 is read rather than memory outside the pool
  const int64_t page = max<int64_t>(page_of(a, b, grp), 0);
  const uint8_t* base = a.pages + (page * a.hkv + h) * PAGE_BYTES;
  const void* pb = uniform_ptr(base);
  slot = __builtin_amdgcn_readfirstlane(slot);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // earlier reads of this slot are done
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = 8 * j + (lane >> 3);
    dma16_stream(pb, (uint32_t)((32 * hf + row) * D + (((lane & 7) ^ swz(row)) << 4)), slot + 1024 * j);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = 8 * j + (lane >> 3);
    dma16_stream(pb, (uint32_t)(CODE_BYTES + (32 * hf + row) * D + (((lane & 7) ^ swz(row)) << 4)), slot + HALF_CODE + 1024 * j);
  }
  if (hf == 0) dma16_stream(pb, (uint32_t)(2 * CODE_BYTES + 16 * lane), __builtin_amdgcn_readfirstlane(rs));
}

// The paged per-token symmetric layout's half group: 4 + 4 loads of code rows from the page,
// then the half's 32 K and 32 V scales (one load each, 4 lanes), into the same slot layout as
// issue_half_tok.
__device__ __forceinline__ void issue_half_paged_tok(const AttnArgs& a, int b, int h, int64_t grp, int hf,
                                                     uint32_t slot) {
  const int lane = threadIdx.x & 63;
  const int64_t page = max<int64_t>(page_of(a, b, grp), 0);  // as in issue_half_paged
  const void* pb = uniform_ptr(a.pages + (page * a.hkv + h) * PAGE_TOK_BYTES);
  slot = __builtin_amdgcn_readfirstlane(slot);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // earlier reads of this slot are done
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = 8 * j + (lane >> 3);
    dma16_stream(pb, (uint32_t)((32 * hf + row) * D + (((lane & 7) ^ swz(row)) << 4)), slot + 1024 * j);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = 8 * j + (lane >> 3);
    dma16_stream(pb, (uint32_t)(CODE_BYTES + (32 * hf + row) * D + (((lane & 7) ^ swz(row)) << 4)), slot + HALF_CODE + 1024 * j);
  }
  if (lane < 4) dma16_stream(pb, (uint32_t)(2 * CODE_BYTES + 64 * hf + 16 * lane), slot + 2 * HALF_CODE);
  if (lane < 4) dma16_stream(pb, (uint32_t)(2 * CODE_BYTES + 2 * GT + 64 * hf + 16 * lane), slot + 2 * HALF_CODE + TOK_SCALE_BYTES);
}

// Half `hf` of group `grp` in the per-token symmetric format, from either layout.
template <bool PAGED>
__device__ __forceinline__ void issue_tok(const AttnArgs& a, int b, int h, int64_t grp, int hf, uint32_t slot) {
  if constexpr (PAGED) issue_half_paged_tok(a, b, h, grp, hf, slot);
  else issue_half_tok(a, h, grp, hf, slot);
}

// Q of KV head h (gq rows of 256 bytes) into LDS at `dst`, by one wave.
__device__ __forceinline__ void issue_q(const uint16_t* qh, int gq, uint32_t dst) {
  const int lane = threadIdx.x & 63;
  const int bytes = gq * D * 2;
  const void* qg = uniform_ptr(qh);
  for (int k = 0; k < bytes; k += 1024)
    if (k + 16 * lane < bytes) dma16(qg, (uint32_t)(k + 16 * lane), dst + k);
}

// The B operand of load_q, from Q rows in LDS.
__device__ __forceinline__ void load_q_lds(const uint16_t* q_lds, int gq, half8_t (&qb)[4]) {
  const int lane = tail_tid() & 63, c = lane & 15, g = lane >> 4;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    uint4 w = {0, 0, 0, 0};
    if (c < gq) w = *reinterpret_cast<const uint4*>(q_lds + c * D + 16 * g + 64 * (k >> 1) + 8 * (k & 1));
    qb[k] = as_h8(w);
  }
}

__device__ __forceinline__ void wait_groups_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// ---------------------------------------------------------------- one group's attention

constexpr float DEC_TAU = 8.0f;  // headroom of the reference maximum (log2 domain)

// Online-softmax update from the raw scores S[b][i] (q.k, token 16b + 4g + i, head c; -inf
// where masked), in the log2 domain: m is a reference maximum, at least every S * sl2 seen,
// and p = 2^(S sl2 - m). P comes out scaled by 2^15 (folded into the exponent) and split into
// hi/lo fp16 A operands of token blocks (0,1) and (2,3); l accumulates the same scaled weights
// (out = acc / l). m moves only when a score passes it, to DEC_TAU above the block's maximum,
// and only then are the accumulators rescaled.
template <int NB>
__device__ __forceinline__ void softmax_step(WaveState& st, float (&s)[2 * NB][4], float sl2, half8_t (&phi)[NB],
                                             half8_t (&plo)[NB], int gq) {
  const int lane = threadIdx.x & 63, g = lane >> 4;
  float mloc = NEG_INF;
#pragma unroll
  for (int b = 0; b < 2 * NB; ++b)
#pragma unroll
    for (int i = 0; i < 4; ++i) mloc = fmaxf(mloc, s[b][i]);
  mloc = max4rows(mloc) * sl2;
  // the reference maximum moves only when a score passes it, and then DEC_TAU above the new
  // maximum: P = 2^(S sl2 - m + 15) <= 2^15 always, and the accumulators are rescaled rarely
  const float m_new = mloc > st.m ? mloc + DEC_TAU : st.m;
  const float m_use = m_new == NEG_INF ? 0.0f : m_new;
  const float alpha = __builtin_amdgcn_exp2f(st.m - m_use);
  const float off = P_SCALE_LOG2 - m_use;
  float lsum = 0.0f;
  _Float16 hi[NB][8], lo[NB][8];
#pragma unroll
  for (int b = 0; b < 2 * NB; ++b) {
    float q[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      q[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[b][i], sl2, off));
      lsum += q[i];
    }
#pragma unroll
    for (int i = 0; i < 4; i += 2) {
      const half2_t h = __builtin_bit_cast(half2_t, __builtin_amdgcn_cvt_pkrtz(q[i], q[i + 1]));
      const half2_t l = __builtin_bit_cast(half2_t, __builtin_amdgcn_cvt_pkrtz(q[i] - (float)h.x, q[i + 1] - (float)h.y));
      hi[b >> 1][4 * (b & 1) + i] = h.x;
      hi[b >> 1][4 * (b & 1) + i + 1] = h.y;
      lo[b >> 1][4 * (b & 1) + i] = l.x;
      lo[b >> 1][4 * (b & 1) + i + 1] = l.y;
    }
  }
#pragma unroll
  for (int B = 0; B < NB; ++B) {
    phi[B] = half8_t{hi[B][0], hi[B][1], hi[B][2], hi[B][3], hi[B][4], hi[B][5], hi[B][6], hi[B][7]};
    plo[B] = half8_t{lo[B][0], lo[B][1], lo[B][2], lo[B][3], lo[B][4], lo[B][5], lo[B][6], lo[B][7]};
  }
  st.l = st.l * alpha + sum4rows(lsum);
  const bool moved = st.m != m_new;
  st.m = m_new;
  // accumulator rows belong to head 4g + i; its alpha sits in lane 4g + i. Nothing to do
  // while no maximum of the wave moved (alpha == 1 in every lane).
  if (__builtin_amdgcn_ballot_w64(moved) == 0) return;
  if (gq <= 4) {
    // rows of g >= 1 are padding heads: one scalar alpha per row
    float ai[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) ai[i] = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(alpha), i));
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int cb = 0; cb < 8; ++cb) st.acc[cb][i] *= ai[i];
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float ai = shfl(alpha, 4 * g + i);
#pragma unroll
      for (int cb = 0; cb < 8; ++cb) st.acc[cb][i] *= ai;
    }
  }
}

// One group's rulers as a lane uses them: V's (splatted) for dim 16 cb + c, read from the
// group's ruler rows in LDS (kst | kmn | vst | vmn, 128 fp16 each) once per group and used by
// both halves; K's step and min for the dims of the lane's K operand chunks are read from `rul`
// by each half, so that they are not live across the softmax and the PV product (keeping them
// for both halves took 32 more VGPRs, and the chained kernel's loop had none to spare).
struct LaneRulers {
  half2_t vsp[8], vmp[8];
  const uint8_t* rul;
};

__device__ __forceinline__ void load_k_rulers(const uint8_t* rul, uint4 (&kst4)[2][2], uint4 (&kmn4)[2][2]) {
  const int g = (threadIdx.x & 63) >> 4;
  const uint16_t* rks = reinterpret_cast<const uint16_t*>(rul);
#pragma unroll
  for (int hh = 0; hh < 2; ++hh)
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      kst4[hh][e] = *reinterpret_cast<const uint4*>(rks + 16 * g + 64 * hh + 8 * e);
      kmn4[hh][e] = *reinterpret_cast<const uint4*>(rks + D + 16 * g + 64 * hh + 8 * e);
    }
}

__device__ __forceinline__ void load_rulers(const uint8_t* rul, LaneRulers& r) {
  const int lane = threadIdx.x & 63, c = lane & 15;
  const uint16_t* rks = reinterpret_cast<const uint16_t*>(rul);
  r.rul = rul;
#pragma unroll
  for (int cb = 0; cb < 8; ++cb) {
    const _Float16 vs = __builtin_bit_cast(_Float16, rks[2 * D + 16 * cb + c]);
    const _Float16 vm = __builtin_bit_cast(_Float16, rks[3 * D + 16 * cb + c]);
    r.vsp[cb] = half2_t{vs, vs};
    r.vmp[cb] = half2_t{vm, vm};
  }
}

// 32 NB tokens of one int8 group resident in LDS: K codes at `kc`, V codes at `vc` (rows of
// 128 bytes, chunks swizzled by swz(row)), the group's rulers in `ru`; `nvalid` of the tokens
// are valid.
template <int NB>
__device__ __forceinline__ void attend_block(const AttnArgs& a, WaveState& st, const half8_t (&qb)[4],
                                             const uint8_t* kc, const uint8_t* vc, const LaneRulers& ru, int nvalid) {
  const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
  uint4 kst4[2][2], kmn4[2][2];
  load_k_rulers(ru.rul, kst4, kmn4);

  // ---- S^T = K Q^T
  float4_t S[2 * NB];
#pragma unroll
  for (int b = 0; b < 2 * NB; ++b) {
    S[b] = float4_t{0.f, 0.f, 0.f, 0.f};
    const int row = 16 * b + c;
    const int key = swz(row);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const uint4 kw = *reinterpret_cast<const uint4*>(kc + row * D + (((g + 4 * hh) ^ key) << 4));
      S[b] = mfma32(dq8(kw.x, kw.y, kst4[hh][0], kmn4[hh][0]), qb[2 * hh], S[b]);
      S[b] = mfma32(dq8(kw.z, kw.w, kst4[hh][1], kmn4[hh][1]), qb[2 * hh + 1], S[b]);
    }
  }
  float s[2 * NB][4];
#pragma unroll
  for (int b = 0; b < 2 * NB; ++b)
#pragma unroll
    for (int i = 0; i < 4; ++i) s[b][i] = S[b][i];
  if (nvalid < 32 * NB) {
#pragma unroll
    for (int b = 0; b < 2 * NB; ++b)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (16 * b + 4 * g + i >= nvalid) s[b][i] = NEG_INF;
  }

  half8_t phi[NB], plo[NB];
  softmax_step<NB>(st, s, a.sl2, phi, plo, a.gq);

  // ---- O += P V. Lane (c, g) of a transpose read supplies row k(g, c >> 1) and half
  // (c & 1) of the 16-dim chunk; it receives dim 16cb + c of the 8 tokens k(g, 0..7),
  // k(g, r) = 16 * (2B + (r >> 2)) + 4g + (r & 3), the token order of P's k-slots. All the
  // half's transpose reads are issued before the first product (one wait for all of them;
  // reading them before the softmax instead measured slower).
  const auto& vsp = ru.vsp;
  const auto& vmp = ru.vmp;
  const int r = c >> 1;
  u32x2 vw[NB][8];
#pragma unroll
  for (int B = 0; B < NB; ++B) {
    const int row = 16 * (2 * B + (r >> 2)) + 4 * g + (r & 3);
#pragma unroll
    for (int cb = 0; cb < 8; ++cb)
      vw[B][cb] = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                      (lds_v2i_t*)(const lds_void_t*)(vc + row * D + 8 * (c & 1) + ((cb ^ swz(row)) << 4))));
  }

#pragma unroll
  for (int B = 0; B < NB; ++B) {
    if (nvalid >= 32 * NB) {
#pragma unroll
      for (int cb = 0; cb < 8; ++cb) {
        const half8_t vb = dq8_splat(vw[B][cb].x, vw[B][cb].y, vsp[cb], vmp[cb]);
        st.acc[cb] = mfma32(phi[B], vb, st.acc[cb]);
        st.acc[cb] = mfma32(plo[B], vb, st.acc[cb]);
      }
    } else {
      // invalid tokens of a partial group get code 0 (finite value, weight 0)
      uint32_t m[2] = {0u, 0u};
#pragma unroll
      for (int rr = 0; rr < 8; ++rr) {
        const int tok = 16 * (2 * B + (rr >> 2)) + 4 * g + (rr & 3);
        if (tok < nvalid) m[rr >> 2] |= 0xffu << (8 * (rr & 3));
      }
      const u32x2 keep = u32x2{m[0], m[1]};
#pragma unroll
      for (int cb = 0; cb < 8; ++cb) {
        const u32x2 vm = vw[B][cb] & keep;
        const half8_t vb = dq8_splat(vm.x, vm.y, vsp[cb], vmp[cb]);
        st.acc[cb] = mfma32(phi[B], vb, st.acc[cb]);
        st.acc[cb] = mfma32(plo[B], vb, st.acc[cb]);
      }
    }
  }
}

// The two halves of attend_block<1> for a full half (32 valid tokens), so that a caller can put
// one half's PV product and the next half's QK product in one basic block, where the compiler
// interleaves them (the chained step's software-pipelined loop).
// S[b][i]: q.k of token 16b + 4g + i and head c (the layout softmax_step takes).
__device__ __forceinline__ void qk_half(const uint8_t* kc, const uint8_t* rul, const half8_t (&qb)[4], float (&s)[2][4]) {
  const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
  uint4 kst4[2][2], kmn4[2][2];
  load_k_rulers(rul, kst4, kmn4);
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    float4_t S = float4_t{0.f, 0.f, 0.f, 0.f};
    const int row = 16 * b + c;
    const int key = swz(row);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const uint4 kw = *reinterpret_cast<const uint4*>(kc + row * D + (((g + 4 * hh) ^ key) << 4));
      S = mfma32(dq8(kw.x, kw.y, kst4[hh][0], kmn4[hh][0]), qb[2 * hh], S);
      S = mfma32(dq8(kw.z, kw.w, kst4[hh][1], kmn4[hh][1]), qb[2 * hh + 1], S);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) s[b][i] = S[i];
  }
}

// O += P V for a full half: V codes at `vc`, the lane's V rulers in `ru` (the product of
// attend_block<1> for nvalid = 32).
__device__ __forceinline__ void pv_half(WaveState& st, const uint8_t* vc, const LaneRulers& ru, const half8_t& phi,
                                        const half8_t& plo) {
  const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
  const int r = c >> 1;
  const int row = 16 * (r >> 2) + 4 * g + (r & 3);
  u32x2 vw[8];
#pragma unroll
  for (int cb = 0; cb < 8; ++cb)
    vw[cb] = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                 (lds_v2i_t*)(const lds_void_t*)(vc + row * D + 8 * (c & 1) + ((cb ^ swz(row)) << 4))));
#pragma unroll
  for (int cb = 0; cb < 8; ++cb) {
    const half8_t vb = dq8_splat(vw[cb].x, vw[cb].y, ru.vsp[cb], ru.vmp[cb]);
    st.acc[cb] = mfma32(phi, vb, st.acc[cb]);
    st.acc[cb] = mfma32(plo, vb, st.acc[cb]);
  }
}

// PV of one full half fused with QK of the next: all LDS reads first, then each of the 8
// V column blocks (dequantize + 2 MFMA) alternates with one of the 8 K operand pieces
// (dequantize + 1 MFMA, the two token blocks' chains alternating), so that the matrix core and
// the VALU each have independent work in flight.
__device__ __forceinline__ void pv_qk_half(WaveState& st, const uint8_t* vc, const LaneRulers& ru, const half8_t& phi,
                                           const half8_t& plo, const uint8_t* kc, const uint8_t* rul,
                                           const half8_t (&qb)[4], float (&s)[2][4]) {
  const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
  const int r = c >> 1;
  const int vrow = 16 * (r >> 2) + 4 * g + (r & 3);
  u32x2 vw[8];
#pragma unroll
  for (int cb = 0; cb < 8; ++cb)
    vw[cb] = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                 (lds_v2i_t*)(const lds_void_t*)(vc + vrow * D + 8 * (c & 1) + ((cb ^ swz(vrow)) << 4))));
  uint4 kst4[2][2], kmn4[2][2];
  load_k_rulers(rul, kst4, kmn4);
  uint4 kw[2][2];
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int row = 16 * b + c;
      kw[b][hh] = *reinterpret_cast<const uint4*>(kc + row * D + (((g + 4 * hh) ^ swz(row)) << 4));
    }
  float4_t S[2] = {float4_t{0.f, 0.f, 0.f, 0.f}, float4_t{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const half8_t vb = dq8_splat(vw[i].x, vw[i].y, ru.vsp[i], ru.vmp[i]);
    st.acc[i] = mfma32(phi, vb, st.acc[i]);
    st.acc[i] = mfma32(plo, vb, st.acc[i]);
    const int b = i & 1, j = i >> 1, hh = j >> 1, e = j & 1;
    const uint32_t w0 = e ? kw[b][hh].z : kw[b][hh].x, w1 = e ? kw[b][hh].w : kw[b][hh].y;
    S[b] = mfma32(dq8(w0, w1, kst4[hh][e], kmn4[hh][e]), qb[2 * hh + e], S[b]);
  }
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int i = 0; i < 4; ++i) s[b][i] = S[b][i];
}

// fp16(code * scale) for 8 signed codes sharing one fp16 scale, and for 8 codes with one
// scale each: the product of an 8-bit integer and an fp16 is exact in fp32, so the packed
// fp16 multiply rounds it once, as fp16(fp32(code) * fp32(scale)) does.
__device__ __forceinline__ half8_t dq8_sym(uint32_t w0, uint32_t w1, half2_t s) {
  const half2_t a = scodes_to_h2(w0, kSelB01) * s;
  const half2_t b = scodes_to_h2(w0, kSelB23) * s;
  const half2_t c = scodes_to_h2(w1, kSelB01) * s;
  const half2_t d = scodes_to_h2(w1, kSelB23) * s;
  return half8_t{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
}
__device__ __forceinline__ half8_t dq8_sym_v(uint32_t w0, uint32_t w1, uint4 s) {
  const half2_t a = scodes_to_h2(w0, kSelB01) * as_h2(s.x);
  const half2_t b = scodes_to_h2(w0, kSelB23) * as_h2(s.y);
  const half2_t c = scodes_to_h2(w1, kSelB01) * as_h2(s.z);
  const half2_t d = scodes_to_h2(w1, kSelB23) * as_h2(s.w);
  return half8_t{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
}

// attend_block for 32 tokens of the per-token symmetric format: codes as in attend_block
// (signed), the tokens' K scales at `ksc` and V scales at `vsc` (32 fp16 each).
__device__ __forceinline__ void attend_block_tok(const AttnArgs& a, WaveState& st, const half8_t (&qb)[4],
                                                 const uint8_t* kc, const uint8_t* vc, const uint16_t* ksc,
                                                 const uint16_t* vsc, int nvalid) {
  const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
  // ---- S^T = K Q^T; lane (c, g) holds token 16b + c, whose scale it splats
  float4_t S[2];
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    S[b] = float4_t{0.f, 0.f, 0.f, 0.f};
    const int row = 16 * b + c;
    const int key = swz(row);
    const _Float16 ks = __builtin_bit_cast(_Float16, ksc[row]);
    const half2_t ks2 = half2_t{ks, ks};
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const uint4 kw = *reinterpret_cast<const uint4*>(kc + row * D + (((g + 4 * hh) ^ key) << 4));
      S[b] = mfma32(dq8_sym(kw.x, kw.y, ks2), qb[2 * hh], S[b]);
      S[b] = mfma32(dq8_sym(kw.z, kw.w, ks2), qb[2 * hh + 1], S[b]);
    }
  }
  float s[2][4];
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int i = 0; i < 4; ++i) s[b][i] = (16 * b + 4 * g + i) < nvalid ? S[b][i] : NEG_INF;
  half8_t phi[1], plo[1];
  softmax_step<1>(st, s, a.sl2, phi, plo, a.gq);

  // ---- O += P V: lane (c, g) receives dim 16cb + c of tokens 4g + {0..3} and 16 + 4g +
  // {0..3}; their 8 scales are the same for every cb. Invalid tokens get code 0 and scale 0.
  const int r = c >> 1;
  const int row = 16 * (r >> 2) + 4 * g + (r & 3);
  const int key = swz(row);
  const uint8_t* rowp = vc + row * D + 8 * (c & 1);
  const uint2 s_lo = *reinterpret_cast<const uint2*>(vsc + 4 * g);
  const uint2 s_hi = *reinterpret_cast<const uint2*>(vsc + 16 + 4 * g);
  uint4 vs = uint4{s_lo.x, s_lo.y, s_hi.x, s_hi.y};
  u32x2 keep = {~0u, ~0u};
  if (nvalid < 32) {
    uint32_t m[2] = {0u, 0u}, hm[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int rr = 0; rr < 8; ++rr) {
      const int tok = 16 * (rr >> 2) + 4 * g + (rr & 3);
      if (tok < nvalid) {
        m[rr >> 2] |= 0xffu << (8 * (rr & 3));
        hm[rr >> 1] |= 0xffffu << (16 * (rr & 1));
      }
    }
    keep = u32x2{m[0], m[1]};
    vs = uint4{vs.x & hm[0], vs.y & hm[1], vs.z & hm[2], vs.w & hm[3]};
  }
  u32x2 vw[8];  // (all eight transpose reads before the first product)
#pragma unroll
  for (int cb = 0; cb < 8; ++cb)
    vw[cb] = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                 (lds_v2i_t*)(const lds_void_t*)(rowp + ((cb ^ key) << 4))));
#pragma unroll
  for (int cb = 0; cb < 8; ++cb) {
    const u32x2 vm = vw[cb] & keep;
    const half8_t vb = dq8_sym_v(vm.x, vm.y, vs);
    st.acc[cb] = mfma32(phi[0], vb, st.acc[cb]);
    st.acc[cb] = mfma32(plo[0], vb, st.acc[cb]);
  }
}


// Online-softmax update with the 4 masked scores s[i] (token 4g + i of a 16-token block,
// head c); returns P as the A operand of v_mfma_f32_16x16x16_f16 (hi/lo halves).
__device__ __forceinline__ void softmax_step4(WaveState& st, const float (&s)[4], float sl2, half4_t& phi,
                                              half4_t& plo, int gq) {
  const int lane = tail_tid() & 63, g = lane >> 4;
  const float mloc = max4rows(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]))) * sl2;
  const float m_new = fmaxf(st.m, mloc);
  const float m_use = m_new == NEG_INF ? 0.0f : m_new;
  const float alpha = __builtin_amdgcn_exp2f(st.m - m_use);
  const float off = P_SCALE_LOG2 - m_use;
  float q[4], lsum = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    q[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[i], sl2, off));
    lsum += q[i];
  }
  const half2_t h01 = __builtin_bit_cast(half2_t, __builtin_amdgcn_cvt_pkrtz(q[0], q[1]));
  const half2_t h23 = __builtin_bit_cast(half2_t, __builtin_amdgcn_cvt_pkrtz(q[2], q[3]));
  const half2_t l01 = __builtin_bit_cast(half2_t, __builtin_amdgcn_cvt_pkrtz(q[0] - (float)h01.x, q[1] - (float)h01.y));
  const half2_t l23 = __builtin_bit_cast(half2_t, __builtin_amdgcn_cvt_pkrtz(q[2] - (float)h23.x, q[3] - (float)h23.y));
  phi = half4_t{h01.x, h01.y, h23.x, h23.y};
  plo = half4_t{l01.x, l01.y, l23.x, l23.y};
  st.l = st.l * alpha + sum4rows(lsum);
  st.m = m_new;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float ai = gq <= 4 ? __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(alpha), i)) : shfl(alpha, 4 * g + i);
#pragma unroll
    for (int cb = 0; cb < 8; ++cb) st.acc[cb][i] *= ai;
  }
}

// Ring tokens 16 * blk .. 16 * blk + 15 of one head, resident in LDS (K at `rk`, V at `rv`,
// layout of ring_chunk_pos), slot validity from `valid_bits`. QK^T on 16x16x32 MFMA with
// the same Q operand as the prefix; PV on 16x16x16 (16 tokens), whose P operand is the
// S^T output layout of the block.
__device__ __forceinline__ void attend_ring16(const AttnArgs& a, WaveState& st, const half8_t (&qb)[4],
                                              const uint8_t* rk, const uint8_t* rv, int blk, uint64_t valid_bits) {
  const int lane = tail_tid() & 63, c = lane & 15, g = lane >> 4;
  float4_t S = {0.f, 0.f, 0.f, 0.f};
  const int row = 16 * blk + c;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int chunk = 2 * g + 8 * (k >> 1) + (k & 1);
    const uint4 kw = *reinterpret_cast<const uint4*>(rk + row * (2 * D) + (ring_chunk_pos(row, chunk) << 4));
    S = mfma32(as_h8(kw), qb[k], S);
  }
  float sc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int slot = 16 * blk + 4 * g + i;
    sc[i] = ((valid_bits >> slot) & 1ull) ? S[i] : NEG_INF;
  }
  half4_t phi, plo;
  softmax_step4(st, sc, a.sl2, phi, plo, a.gq);
  // V as the B operand: lane (c, g) holds tokens 16 blk + 4g + [0..3] of dim 16 cb + c
#pragma unroll
  for (int cb = 0; cb < 8; ++cb) {
    _Float16 v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int slot = 16 * blk + 4 * g + r;
      const int chunk = 2 * cb + (c >> 3);
      const uint16_t bits = *reinterpret_cast<const uint16_t*>(rv + slot * (2 * D) + (ring_chunk_pos(slot, chunk) << 4) + 2 * (c & 7));
      v[r] = ((valid_bits >> slot) & 1ull) ? __builtin_bit_cast(_Float16, bits) : (_Float16)0.0f;
    }
    const half4_t vb = half4_t{v[0], v[1], v[2], v[3]};
    st.acc[cb] = __builtin_amdgcn_mfma_f32_16x16x16f16(phi, vb, st.acc[cb], 0, 0, 0);
    st.acc[cb] = __builtin_amdgcn_mfma_f32_16x16x16f16(plo, vb, st.acc[cb], 0, 0, 0);
  }
}

// ---------------------------------------------------------------- ring append

__device__ __forceinline__ float min4rows(float v) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fminf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fminf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ const uint16_t* ring_of(const AttnArgs& a, int h, int which) {
  return (which == 0 ? a.tail_k : a.tail_v) + (int64_t)h * a.tail_slots * D;
}
// The step's new token of KV head h (of sequence b in a batch: kv_ss is 0 otherwise).
__device__ __forceinline__ const uint16_t* fresh_of(const AttnArgs& a, int b, int h, int which) {
  return (which == 0 ? a.k_new : a.v_new) + (int64_t)b * a.kv_ss + (int64_t)h * a.kv_hs;
}
// Ring slot `slot` of tensor `which` (0 K, 1 V) of KV head h (of sequence b when paged).
template <bool PAGED>
__device__ __forceinline__ uint16_t* ring_row(const AttnArgs& a, int b, int h, int which, int slot) {
  if constexpr (PAGED) return a.rings + ((((int64_t)b * a.hkv + h) * 2 + which) * GT + slot) * D;
  else return const_cast<uint16_t*>(ring_of(a, h, which)) + (int64_t)slot * D;
}
// Where the append of the token at `pos` rules its group (int8t64): tensor `which`'s code rows
// (row stride D) and its step / min rulers (one fp16 per channel), and the rows that exist (a
// contiguous cache ends at its capacity; a page always holds 64). Paged: the group's page of KV
// head h, K codes | V codes | kst | kmn | vst | vmn (the caller has checked that it exists).
struct GroupDst {
  uint8_t* codes;
  uint16_t* st;
  uint16_t* mn;
  int rows;
};
template <bool PAGED>
__device__ __forceinline__ GroupDst group_dst(const AttnArgs& a, int b, int h, int64_t pos, int which, int64_t page = -1);

// The per-token symmetric append of the token at `pos`: waves 0 and 1 of the calling
// workgroup quantize K and V of KV head h (lanes 0..15, 8 values each) and store the codes
// and the fp16 scale at position pos.
// (The fused tail quantizes the new token itself from k_new / v_new, so nothing in the launch
// reads these stores; the prefix reads only the tokens before pos.)
__device__ __forceinline__ void append_tok_rows(const AttnArgs& a, int h, int64_t pos) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (wave > 1 || lane >= 16) return;
  const uint4 w = *reinterpret_cast<const uint4*>(fresh_of(a, 0, h, wave) + 8 * lane);
  const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
  float v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = h2f((uint16_t)(wv[j >> 1] >> (16 * (j & 1))));
  float scale;
  const uint2 cw = sym_quant8(v, scale);
  const int64_t row = (int64_t)h * a.capacity + pos;
  *reinterpret_cast<uint2*>((wave == 0 ? a.kq : a.vq) + row * D + 8 * lane) = cw;
  if (lane == 0) ((wave == 0 ? a.ksc : a.vsc))[row] = f2h(scale);
}

// The same for sequence b of the paged layout: row pos % 64 of the page of pos (a valid page,
// checked by the caller) and its scale.
__device__ __forceinline__ void append_tok_rows_paged(const AttnArgs& a, int b, int h, int64_t pos) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (wave > 1 || lane >= 16) return;
  const uint4 w = *reinterpret_cast<const uint4*>(fresh_of(a, b, h, wave) + 8 * lane);
  const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
  float v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = h2f((uint16_t)(wv[j >> 1] >> (16 * (j & 1))));
  float scale;
  const uint2 cw = sym_quant8(v, scale);
  uint8_t* pg = a.pages + (page_of(a, b, pos / GT) * a.hkv + h) * PAGE_TOK_BYTES;
  const int slot = (int)(pos % GT);
  *reinterpret_cast<uint2*>(pg + wave * CODE_BYTES + slot * D + 8 * lane) = cw;
  if (lane == 0) reinterpret_cast<uint16_t*>(pg + 2 * CODE_BYTES)[wave * GT + slot] = f2h(scale);
}

__device__ __forceinline__ void write_scalars(const AttnArgs& a, int64_t pos) {
  const int64_t written = pos + 1;
  const int64_t qlen = written / GT * GT;
  *a.written_out = written;
  if (a.qlen_out) *a.qlen_out = qlen;
  if (a.pg_out) *a.pg_out = qlen / GT;
}

// Slot validity of the ring: slot i holds p = u - ((u - i) mod 64), valid iff qlen <= p <= u,
// p >= first (u = written - 1). Lane i decides slot i; the wave's ballot is the mask.
__device__ __forceinline__ uint64_t ring_bits(int64_t written, int64_t qlen, int64_t first) {
  const int i = tail_tid() & 63;
  const int64_t u = written - 1;
  const int64_t p = u - ((u - i) & (GT - 1));
  return __builtin_amdgcn_ballot_w64(p >= qlen && p <= u && p >= first);
}

// ---------------------------------------------------------------- append units

// The fused step's append is split into APPEND_UNITS units per KV head (8 channels of K or
// V each), one per prefix workgroup, run ahead of its stream. A unit's source rows (the
// 64 ring rows and the new token, 16 bytes each) come into LDS through one HBM -> LDS load
// of wave 0, issued with the groups.
constexpr int UNIT_CH = 8;
constexpr int APPEND_UNITS = 2 * D / UNIT_CH;
constexpr int UNIT_SRC_BYTES = (GT + 1) * UNIT_CH * 2;

// Where one append unit reads and writes: the ring rows and the new token of one tensor of
// one head, and the current group's code rows and ruler rows of that tensor.
struct UnitIO {
  const uint16_t* ring;   // [64][D] fp16, row stride D
  const uint16_t* fresh;  // [D] fp16
  uint8_t* codes;         // the group's row 0 (row stride D)
  int code_rows;          // rows stored (the cache capacity can end inside the group)
  uint16_t* mn;           // the group's [D] ruler rows
  uint16_t* st;
};

// A unit of the contiguous layout: unit u covers channels 8 (u % 16) .. + 7 of tensor u / 16.
__device__ __forceinline__ UnitIO unit_io(const AttnArgs& a, int h, int unit, int64_t pos) {
  const int which = unit / (D / UNIT_CH);
  const int64_t gcur = pos / GT, ro = ((int64_t)h * a.ngroups_cap + gcur) * D;
  UnitIO io;
  io.ring = ring_of(a, h, which);
  io.fresh = fresh_of(a, 0, h, which);
  io.codes = (which == 0 ? a.kq : a.vq) + ((int64_t)h * a.capacity + gcur * GT) * D;
  io.code_rows = (int)min<int64_t>(GT, a.capacity - gcur * GT);
  io.mn = (which == 0 ? a.kmn : a.vmn) + ro;
  io.st = (which == 0 ? a.kst : a.vst) + ro;
  return io;
}

// A unit of the paged layout: sequence b's ring and page of the current group.
__device__ __forceinline__ UnitIO unit_io_paged(const AttnArgs& a, int b, int h, int unit, int64_t pos) {
  const int which = unit / (D / UNIT_CH);
  const int64_t page = page_of(a, b, pos / GT);  // checked >= 0 by the caller
  uint8_t* base = a.pages + (page * a.hkv + h) * PAGE_BYTES;
  UnitIO io;
  io.ring = a.rings + (((int64_t)b * a.hkv + h) * 2 + which) * GT * D;
  io.fresh = (which == 0 ? a.k_new : a.v_new) + (int64_t)b * a.kv_ss + (int64_t)h * a.kv_hs;
  io.codes = base + which * CODE_BYTES;
  io.code_rows = GT;
  io.st = reinterpret_cast<uint16_t*>(base + 2 * CODE_BYTES) + which * 2 * D;
  io.mn = io.st + D;
  return io;
}

__device__ __forceinline__ void issue_unit_rows(const UnitIO& io, int unit, uint32_t src) {
  const int lane = threadIdx.x & 63, ch0 = unit % (D / UNIT_CH) * UNIT_CH;
  dma16(uniform_ptr(io.ring + ch0), (uint32_t)(lane * D * 2), src);
  if (lane == 0) dma16(uniform_ptr(io.fresh + ch0), 0u, src + GT * UNIT_CH * 2);
}

__device__ __forceinline__ float ror8(float v) {  // lane l <- lane l ^ 8 within each 16-lane row
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xf, 0xf, false));
}

// Requantization of append unit `unit` for the token at `pos`, once its source rows are in
// `src` (LDS, visible to the workgroup): the ring with the new token in slot pos % 64 is
// ruled per channel over all 64 slots into the current group exactly as the bulk quantizer
// rules a group, and the group's codes and rulers and the new ring slot are stored through
// `io`. Thread t takes channel t & 7 of the unit and ring rows (t >> 3) + 8 WAVES i.
// `xch` is 8 x 2 WAVES floats of LDS; one workgroup barrier inside.
__device__ __forceinline__ void append_unit(const UnitIO& io, int unit, int64_t pos, const uint16_t* src, float* xch) {
  constexpr int RPT = GT / (8 * WAVES);  // ring rows per thread
  static_assert(RPT * 8 * WAVES == GT, "8 WAVES must divide the 64 ring rows");
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, r0 = t >> 3, c = t & 7;
  const int ch = unit % (D / UNIT_CH) * UNIT_CH + c;
  const int slot = (int)(pos % GT);
  uint16_t bits[RPT];
  float v[RPT];
  float mn = __builtin_huge_valf(), mx = -__builtin_huge_valf();
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int r = r0 + 8 * WAVES * i;
    bits[i] = src[(r == slot ? GT : r) * UNIT_CH + c];
    v[i] = h2f(bits[i]);
    mn = fminf(mn, v[i]);
    mx = fmaxf(mx, v[i]);
  }
  // extremes over the wave's rows (lane >> 3): lane ^ 8 within each 16-lane row, then across rows
  mn = min4rows(fminf(mn, ror8(mn)));
  mx = max4rows(fmaxf(mx, ror8(mx)));
  if (lane < UNIT_CH) { xch[c * 2 * WAVES + wave] = mn; xch[c * 2 * WAVES + WAVES + wave] = mx; }
  __syncthreads();
  float lo = xch[c * 2 * WAVES], hi = xch[c * 2 * WAVES + WAVES];
#pragma unroll
  for (int w = 1; w < WAVES; ++w) {
    lo = fminf(lo, xch[c * 2 * WAVES + w]);
    hi = fmaxf(hi, xch[c * 2 * WAVES + WAVES + w]);
  }
  const float step = ruler_step(lo, hi), inv = ruler_inv(step);
  if (r0 == 0) {
    // agent-scope stores: the fused tail of this launch may read the group (it completes)
    __hip_atomic_store(io.mn + ch, f2h(lo), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(io.st + ch, f2h(step), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  uint16_t* ring = const_cast<uint16_t*>(io.ring) + ch;
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int r = r0 + 8 * WAVES * i;
    if (r < io.code_rows)
      __hip_atomic_store(io.codes + r * D + ch, (uint8_t)ruler_code_rcp(v[i], lo, step, inv), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    if (r == slot) ring[slot * D] = bits[i];
  }
}

// A wide unit: 64 channels of one tensor of one head, for the standalone paged append
// (few, larger workgroups). Each wave loads 8 of the 64 ring rows (128 bytes of each), wave 0
// also the new token's 128 bytes; thread t takes ring row t >> 3 and channels 8 (t & 7) + [0..7].
constexpr int WIDE_CH = 64;
constexpr int WIDE_UNITS = 2 * D / WIDE_CH;
constexpr int WIDE_SRC_BYTES = (GT + 1) * WIDE_CH * 2;

__device__ __forceinline__ void issue_wide_rows(const UnitIO& io, int ch0, uint32_t src) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row = 8 * wave + (lane >> 3);
  dma16(uniform_ptr(io.ring + ch0), (uint32_t)(row * D * 2 + (lane & 7) * 16), __builtin_amdgcn_readfirstlane(src + 1024 * wave));
  if (wave == 0 && lane < 8)
    dma16(uniform_ptr(io.fresh + ch0), (uint32_t)(lane * 16), __builtin_amdgcn_readfirstlane(src + GT * WIDE_CH * 2));
}

// append_unit for a wide unit (channels ch0 .. ch0 + 63); `xch` 64 x 16 floats and `rul` 64
// float4 of LDS; two workgroup barriers inside.
__device__ __forceinline__ void append_wide(const UnitIO& io, int ch0, int64_t pos, const uint8_t* src, float* xch,
                                            float4* rul) {
  static_assert(THREADS == 8 * GT, "one thread per 8 channels of a ring row");
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, r = t >> 3, c8 = t & 7;
  const int slot = (int)(pos % GT);
  const uint4 w = *reinterpret_cast<const uint4*>(src + (r == slot ? GT : r) * (WIDE_CH * 2) + 16 * c8);
  const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
  float v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    v[j] = h2f((uint16_t)(wv[j >> 1] >> (16 * (j & 1))));
    const float mn = min4rows(fminf(v[j], ror8(v[j])));
    const float mx = max4rows(fmaxf(v[j], ror8(v[j])));
    if (lane < 8) {
      xch[(8 * c8 + j) * 16 + wave] = mn;
      xch[(8 * c8 + j) * 16 + 8 + wave] = mx;
    }
  }
  __syncthreads();
  if (t < WIDE_CH) {
    const float4* x4 = reinterpret_cast<const float4*>(xch + 16 * t);
    const float4 m0 = x4[0], m1 = x4[1], M0 = x4[2], M1 = x4[3];
    const float lo = fminf(fminf(fminf(m0.x, m0.y), fminf(m0.z, m0.w)), fminf(fminf(m1.x, m1.y), fminf(m1.z, m1.w)));
    const float hi = fmaxf(fmaxf(fmaxf(M0.x, M0.y), fmaxf(M0.z, M0.w)), fmaxf(fmaxf(M1.x, M1.y), fmaxf(M1.z, M1.w)));
    const float step = ruler_step(lo, hi);
    rul[t] = float4{lo, step, ruler_inv(step), 0.0f};
    io.mn[ch0 + t] = f2h(lo);
    io.st[ch0 + t] = f2h(step);
  }
  __syncthreads();
  uint32_t cc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float4 rj = rul[8 * c8 + j];
    cc[j] = ruler_code_rcp(v[j], rj.x, rj.y, rj.z);
  }
  if (r < io.code_rows)
    *reinterpret_cast<uint2*>(io.codes + r * D + ch0 + 8 * c8) =
        uint2{cc[0] | (cc[1] << 8) | (cc[2] << 16) | (cc[3] << 24), cc[4] | (cc[5] << 8) | (cc[6] << 16) | (cc[7] << 24)};
  if (r == slot) *reinterpret_cast<uint4*>(const_cast<uint16_t*>(io.ring) + slot * D + ch0 + 8 * c8) = w;
}

// ---------------------------------------------------------------- partials

// Floats of one partial: [acc: gq * D][m: gq][l: gq], rounded up to 4 floats so that every
// partial starts 16-byte aligned. acc is scaled by 2^15, m is in the log2 domain.
__host__ __device__ __forceinline__ int part_stride(int gq) { return gq * D + ((2 * gq + 3) & ~3); }

// Whole-wave reductions on VALU data movement only: DPP within each 16-lane row (lane ^ 1,
// lane ^ 2, then rotations by 4 and 8), then the permlane swaps across rows.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<0xB1>(v));   // quad_perm [1, 0, 3, 2]
  v = fmaxf(v, dpp<0x4E>(v));   // quad_perm [2, 3, 0, 1]
  v = fmaxf(v, dpp<0x124>(v));  // row_ror 4
  v = fmaxf(v, dpp<0x128>(v));  // row_ror 8
  return max4rows(v);
}
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += dpp<0x124>(v);
  v += dpp<0x128>(v);
  return sum4rows(v);
}

// Write one wave's online-softmax state as a partial at `dst` (LDS or memory): lane (c, g)
// holds m, l of head c (replicated over g) and acc of heads 4g + i, dims 16cb + c.
__device__ __forceinline__ void store_wave_partial(const WaveState& st, int gq, float* dst) {
  const int lane = tail_tid() & 63, c = lane & 15, g = lane >> 4;
  if (g == 0 && c < gq) { dst[gq * D + c] = st.m; dst[gq * D + gq + c] = st.l; }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int head = 4 * g + i;
    if (head < gq)
#pragma unroll
      for (int cb = 0; cb < 8; ++cb) dst[head * D + 16 * cb + c] = st.acc[cb][i];
  }
}

// Token limit of the int8 prefix for this launch: whole groups before the ring's group in
// the fused step (from the write position), else min(used, 64 * prefix_groups).
__device__ __forceinline__ int64_t prefix_limit(const AttnArgs& a, int64_t& pos, bool& pos_ok) {
  int64_t U;
  pos = 0;
  pos_ok = true;
  if (a.tail_mode == TAIL_FUSED) {
    pos = *a.pos_dev;
    pos_ok = pos >= 0 && pos < a.capacity;  // a position outside the cache appends nothing
    U = pos_ok ? (a.tok ? pos : pos / GT * GT) : 0;
  } else if (a.tok) {
    U = a.used_dev ? *a.used_dev : a.used;
  } else {
    const int64_t used = a.used_dev ? *a.used_dev : a.used;
    const int64_t pgv = a.pg_dev ? *a.pg_dev : a.pg;
    U = min(used, pgv * GT);
  }
  return max<int64_t>(0, min(U, a.ngroups_cap * GT));
}

// ---------------------------------------------------------------- kernel A: the prefix

// Workgroup (h, part) streams the 64-token groups [gs, ge) of KV head h's int8 prefix and
// writes one partial to ws[h][part]. Plain stores: the tail kernel that reads them runs
// after this launch completes. In the fused step, workgroup part < APPEND_UNITS first runs
// append unit `part` of head h (the prefix never reads the group it writes), and the grid
// has max(n_parts, APPEND_UNITS) parts per head; parts >= n_parts only append.
// ---------------------------------------------------------------- the tail (ring + merge)

constexpr int TB_WAVES = 8;
constexpr int TB_THREADS = 64 * TB_WAVES;
constexpr int RING_PARTS = 4;  // the ring's 64 tokens as 4 partials of 16
constexpr int MERGE_PRE = 32;  // partials per column pair loaded up front
constexpr int WTS = 256;       // weights one merging wave holds: up to 256 prefix partials
static_assert(TB_WAVES == WAVES, "the prefix kernel's last workgroup runs the tail with its own waves");

struct TailSmem {
  uint8_t ring_lds[2 * RING_BYTES];          // K | V values
  float ring_part[RING_PARTS][16 * D + 32];  // the ring's partials
  float wts[TB_WAVES * WTS];                 // prefix merge weights, per merging wave
  float pre_acc[16 * D];                     // prefix: sum_s w_s acc_s per column
  float pre_m[16], pre_l[16];                // per head: m_p, l_p
  float rq_ext[2][2 * D];                    // local requantization: per channel min / max of two half rings
  int lost[TB_WAVES];                        // a merging wave gave up waiting for a partial word
  uint32_t fwd[(16 + 2) * D / 2];            // the chained step: forwarded q, k_new, v_new of the head (fp16 pairs)
  uint8_t xpose[RING_PARTS * GT * 64];       // the chained step's append: each ring wave's 64 x 64 codes
  int ring_staged;                           // ring waves that have staged their slots (the chained step's append)
  int ring_done;                             // ring waves whose partial is in ring_part (TB_DIRECT)
};
constexpr int MERGER_MAX_PARTS = 64;         // prefix parts per head of a fused launch
constexpr int MERGER_MAX_HEADS = 64;         // KV heads of a fused launch: its part-0 workgroups wait for the others
constexpr int MERGER_SPIN_LIMIT = 1 << 22;   // polls (each followed by a short sleep) before giving up
static_assert(sizeof(TailSmem) <= LDS_BYTES && sizeof(TailSmem) <= LDS_BYTES_TOK,
              "the tail's LDS fits in the prefix kernel's stages");

// Loads of data other workgroups of the same launch wrote with agent-scope stores: coherent
// at agent scope (they bypass the XCD-local L2) when `co`, plain loads otherwise.
__device__ __forceinline__ float ld_f(const float* p, bool co) {
  return co ? __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : *p;
}
__device__ __forceinline__ float2 ld_f2(const float* p, bool co) {
  if (!co) return *reinterpret_cast<const float2*>(p);
  return __builtin_bit_cast(float2, __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED,
                                                      __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ uint2 ld_u2(const uint8_t* p, bool co) {
  if (!co) return *reinterpret_cast<const uint2*>(p);
  return __builtin_bit_cast(uint2, __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ uint4 ld_u4(const uint16_t* p, bool co) {
  if (!co) return *reinterpret_cast<const uint4*>(p);
  const uint64_t* q = reinterpret_cast<const uint64_t*>(p);
  const uint64_t x = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint64_t y = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return uint4{(uint32_t)x, (uint32_t)(x >> 32), (uint32_t)y, (uint32_t)(y >> 32)};
}
__device__ __forceinline__ uint16_t ld_u16(const uint16_t* p, bool co) {
  return co ? __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : *p;
}

// ---- published partials. A prefix partial's values are stored as their float bits XOR PUB_KEY,
// with relaxed agent-scope atomic stores, and every tail sets the words it consumed back to zero:
// between launches a workspace's partials are zero, and in a launch a zero word is one not
// written yet. PUB_KEY is a signalling-NaN pattern, and arithmetic never returns a signalling NaN
// (IEEE operations quiet them), so no value encodes to zero. A tail in the same launch as its
// producers polls the words themselves (relaxed agent-scope atomic loads): per-location
// coherence hands it each producer's value once the word is non-zero, without a flag, fence or
// counter (a flag would need release / acquire ordering, i.e. L2 writeback and invalidation).
// ---- XCD-local hand-over. The workgroups of one launch are dealt to the device's n XCDs in
// turn (workgroup b on XCD (b + k) mod n, the start k varying between launches), and every
// workgroup of KV head h has b = h mod hkv, so with n dividing hkv they share one XCD and its L2.
// Words handed between them are then plain stores into that L2, read by agent-scope loads that
// hit the L2's dirty line (0.25 us per hand-over between idle workgroups, against 0.43 us through
// memory). The host turns this on per device (l2_xcc) after a probe has seen the dealing rule
// (nkv_l2_handover). Were a reader on another XCD than its writer, it would not see the word:
// its wait is bounded, gives up, and poisons its outputs with NaN.
__device__ __forceinline__ uint32_t xcc_id() {
  uint32_t v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  return v;
}

__device__ __forceinline__ bool l2_local(const AttnArgs& a) { return a.l2_xcc != 0; }

constexpr uint32_t PUB_KEY = 0x7FBADBADu;
constexpr uint64_t PUB_KEY2 = ((uint64_t)PUB_KEY << 32) | PUB_KEY;

// A word handed to a workgroup on the same XCD (`l2`, l2_local) is a plain store: it stays in the
// XCD's L2, where the reader's agent-scope loads find it (they miss the CU's L1 and hit lines the
// L2 holds dirty); otherwise an agent-scope store, written through to memory.
template <typename T>
__device__ __forceinline__ void hand_st(T* p, T w, bool l2) {
  if (l2) __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
  else __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// 16 zero bytes, handed over like a published word
__device__ __forceinline__ void zero_st16(uint4* p, bool l2) {
  if (l2) {
    *p = uint4{0u, 0u, 0u, 0u};
  } else {
    hand_st(reinterpret_cast<uint64_t*>(p), uint64_t(0), false);
    hand_st(reinterpret_cast<uint64_t*>(p) + 1, uint64_t(0), false);
  }
}
__device__ __forceinline__ void pub_st(float* p, float v, bool l2) {
  hand_st(reinterpret_cast<uint32_t*>(p), __float_as_uint(v) ^ PUB_KEY, l2);
}
__device__ __forceinline__ void pub_st2(float* p, float x, float y, bool l2) {
  hand_st(reinterpret_cast<uint64_t*>(p), (((uint64_t)__float_as_uint(y) << 32) | __float_as_uint(x)) ^ PUB_KEY2, l2);
}
__device__ __forceinline__ uint32_t pub_ld(const float* p) {
  return __hip_atomic_load(reinterpret_cast<const uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t pub_ld2(const float* p) {
  return __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float pub_f(uint32_t w) { return __uint_as_float(w ^ PUB_KEY); }
__device__ __forceinline__ float2 pub_f2(uint64_t w) {
  w ^= PUB_KEY2;
  return float2{__uint_as_float((uint32_t)w), __uint_as_float((uint32_t)(w >> 32))};
}
// Reload a word while it is zero, sleeping between polls; `budget` is the caller's remaining
// polls (a word still zero when it runs out stays zero: the caller reports it).
__device__ __forceinline__ uint32_t pub_repoll(const float* p, uint32_t w, int& budget) {
  while (w == 0 && budget > 0) {
    --budget;
    __builtin_amdgcn_s_sleep(1);
    w = pub_ld(p);
  }
  return w;
}
__device__ __forceinline__ uint64_t pub_repoll2(const float* p, uint64_t w, int& budget) {
  while (w == 0 && budget > 0) {
    --budget;
    __builtin_amdgcn_s_sleep(1);
    w = pub_ld2(p);
  }
  return w;
}

// The ring held in LDS (64 rows of K, then of V; ring_chunk_pos layout) requantized as one
// int8t64 group, exactly as the append rules the group of the token at `pos`: per channel
// min / max over the 64 rows, step = max((max - min) / 255, 1e-8), codes by ruler_code_rcp.
// With STORE the codes (rows below the capacity) and the rulers go to group pos / 64 of head
// h's cache: the append itself, from the ring that holds the new token in its slot. With `deq`
// the LDS values become the ones the prefix kernel would read back, fp16(code * step16 +
// min16) with one rounding (when the token completes its group, the tail attends those).
// Thread t takes channel t & 255 (K, then V) and rows 32 (t >> 8) .. + 31.
template <bool PAGED>
__device__ __forceinline__ GroupDst group_dst(const AttnArgs& a, int b, int h, int64_t pos, int which, int64_t page) {
  const int64_t gcur = pos / GT;
  GroupDst g;
  if constexpr (PAGED) {
    // (page: the group's page when the caller has read it already, else -1)
    uint8_t* base = a.pages + ((page >= 0 ? page : page_of(a, b, gcur)) * a.hkv + h) * PAGE_BYTES;
    uint16_t* rul = reinterpret_cast<uint16_t*>(base + 2 * CODE_BYTES);
    g.codes = base + which * CODE_BYTES;
    g.st = rul + (which ? 2 : 0) * D;
    g.mn = rul + (which ? 3 : 1) * D;
    g.rows = GT;
  } else {
    const int64_t ro = ((int64_t)h * a.ngroups_cap + gcur) * D;
    g.codes = (which ? a.vq : a.kq) + ((int64_t)h * a.capacity + gcur * GT) * D;
    g.st = (which ? a.vst : a.kst) + ro;
    g.mn = (which ? a.vmn : a.kmn) + ro;
    g.rows = (int)min<int64_t>(GT, a.capacity - gcur * GT);
  }
  return g;
}

template <bool STORE, bool PAGED = false>
__device__ __forceinline__ void requant_ring_lds(uint8_t* ring_lds, float (&ext)[2][2 * D], bool deq,
                                                 const AttnArgs* a = nullptr, int h = 0, int64_t pos = 0, int b = 0,
                                                 int64_t page = -1) {
  const int t = tail_tid(), ch = t & (2 * D - 1), half = t >> 8;
  uint8_t* base = ring_lds + (ch >> 7) * RING_BYTES;
  const int c = ch & (D - 1);
  float v[32];
  float mn = __builtin_huge_valf(), mx = -__builtin_huge_valf();
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const int r = 32 * half + i;
    v[i] = h2f(*reinterpret_cast<const uint16_t*>(base + r * (2 * D) + (ring_chunk_pos(r, c >> 3) << 4) + 2 * (c & 7)));
    mn = fminf(mn, v[i]);
    mx = fmaxf(mx, v[i]);
  }
  // the two halves' extremes meet in `ext` (row = half): first the minima, then the maxima
  ext[half][ch] = mn;
  __syncthreads();
  const float lo = fminf(ext[0][ch], ext[1][ch]);
  __syncthreads();
  ext[half][ch] = mx;
  __syncthreads();
  const float hi = fmaxf(ext[0][ch], ext[1][ch]);
  const float step = ruler_step(lo, hi), inv = ruler_inv(step);
  const half2_t st2 = half2_t{(_Float16)step, (_Float16)step};
  const half2_t mn2 = half2_t{(_Float16)lo, (_Float16)lo};
  uint8_t* codes = nullptr;
  int rows = 0;
  if constexpr (STORE) {
    // group pos / 64: code rows at the group's first token, rulers at its ruler row
    const GroupDst g = group_dst<PAGED>(*a, b, h, pos, ch >> 7, page);
    codes = g.codes + c;
    rows = g.rows;
    if (half == 0) {
      g.mn[c] = f2h(lo);
      g.st[c] = f2h(step);
    }
  }
#pragma unroll
  for (int i = 0; i < 32; i += 2) {
    const uint32_t c0 = ruler_code_rcp(v[i], lo, step, inv), c1 = ruler_code_rcp(v[i + 1], lo, step, inv);
    if constexpr (STORE) {
      const int r = 32 * half + i;
      if (r < rows) codes[r * D] = (uint8_t)c0;
      if (r + 1 < rows) codes[(r + 1) * D] = (uint8_t)c1;
    }
    if (!deq) continue;
    const half2_t code = half2_t{(_Float16)(float)c0, (_Float16)(float)c1};
    const half2_t y = __builtin_elementwise_fma(code, st2, mn2);
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int r = 32 * half + i + e;
      *reinterpret_cast<_Float16*>(base + r * (2 * D) + (ring_chunk_pos(r, c >> 3) << 4) + 2 * (c & 7)) = y[e];
    }
  }
}

// The append of the token at `pos` from the ring held in LDS (the 64 slots, the new token in its
// slot; ring_chunk_pos layout) by 256 threads (waves 0..3, or 4..7 with tbase 256): thread t
// (counted from tbase) rules channel t & 127 of K
// (t < 128) or V over the 64 slots, exactly as append_unit rules it, and stores its two ruler
// values; the wave's 64 x 64 codes go through `xpose` (4 KiB of LDS per wave) so that lane r
// stores row r's 64 codes with four 16-byte stores (rows below the capacity). No workgroup
// barrier: the caller's waves 0..3 have all staged the ring before.
template <bool PAGED = false>
__device__ __forceinline__ void append_ring_channels(const AttnArgs& a, int h, int64_t pos, const uint8_t* ring_lds,
                                                     uint8_t* xpose, int b = 0, int64_t page = -1, int tbase = 0) {
  const int t = tail_tid() - tbase, wave = t >> 6, lane = t & 63, which = t >> 7, c = t & (D - 1);
  const uint8_t* base = ring_lds + which * RING_BYTES;
  float v[GT];
  float mn = __builtin_huge_valf(), mx = -__builtin_huge_valf();
#pragma unroll
  for (int r = 0; r < GT; ++r) {
    v[r] = h2f(*reinterpret_cast<const uint16_t*>(base + r * (2 * D) + (ring_chunk_pos(r, c >> 3) << 4) + 2 * (c & 7)));
    mn = fminf(mn, v[r]);
    mx = fmaxf(mx, v[r]);
  }
  const float step = ruler_step(mn, mx), inv = ruler_inv(step);
  const GroupDst g = group_dst<PAGED>(a, b, h, pos, which, page);
  g.mn[c] = f2h(mn);
  g.st[c] = f2h(step);
  // codes: column `lane` of the wave's [64 rows][64 channels] block, then row `lane` of it
  uint8_t* xw = xpose + wave * (GT * 64);
#pragma unroll
  for (int r = 0; r < GT; ++r) xw[r * 64 + lane] = (uint8_t)ruler_code_rcp(v[r], mn, step, inv);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // (one wave: its LDS accesses run in order)
  if (lane < g.rows) {
    uint4* dst = reinterpret_cast<uint4*>(g.codes + (int64_t)lane * D + 64 * (wave & 1));
    const uint4* src = reinterpret_cast<const uint4*>(xw + lane * 64);
#pragma unroll
    for (int k = 0; k < 4; ++k) dst[k] = src[k];
  }
}

// The tail of one decode step for KV head h (of sequence b when paged), by the 8 waves of the
// calling workgroup. The prefix partials merge into (m_p, l_p, acc_p): m_p = max_s m_s,
// w_s = 2^(m_s - m_p), l_p = sum_s w_s l_s, acc_p = sum_s w_s acc_s (waves 4..7, one head
// each, two columns per lane); meanwhile waves 0..3 attend over the ring, one partial of 16
// tokens each; the ring's partials then join by log-sum-exp into out / lse.
//
// The ring: the 64 fp16 slots of earlier launches, with the new token's slot taken from k_new /
// v_new in the fused step (this launch's append writes that slot concurrently). When the new
// token completes its group, the group is read as int8, as the prefix will read it: the ring is
// requantized and dequantized here, bit for bit as the append computes it. In the per-token
// symmetric format the new token alone is the tail, quantized here as the append quantizes it.
// So the tail reads nothing that this launch writes except the partials.
//
// The prefix partials are published words (pub_st). In the fused launch (`run` TAIL_MERGER: the
// head's part-0 workgroup; TAIL_LAST: the last of a paged sequence's workgroups to take its
// ticket) other workgroups may still be writing them: the merging waves load each partial's m
// and l, re-polling the words still zero (sleeping between polls, giving up after
// MERGER_SPIN_LIMIT polls: the output is then NaN), then the column pairs likewise. The merge
// runs in partial order, so the result does not depend on the order of arrival. Every consumed
// word is set back to zero. TAIL_KERNEL (the separate tail kernel) finds every word written.
enum TailRun : int { TAIL_KERNEL = 0, TAIL_LAST = 1, TAIL_MERGER = 2 };

// What a ring wave (wave < RING_PARTS) loads before the tail's LDS work: the K and V rows of
// its 16 ring slots (rows 16 wave + (lane >> 4) + 4 i, 16-byte chunk lane & 15) and, in the wave
// that holds the new token's slot, that token's K and V rows; or, in the per-token symmetric
// format, the new token alone (wave 0: lanes 0..15 K, 16..31 V). The contiguous fused step's
// merger issues these loads as its prefix loop ends, so their latency overlaps its own partial.
struct TailLoads {
  uint4 k[4], v[4], fk, fv, tok;
};

template <bool PAGED>
__device__ __forceinline__ void tail_load_rows(const AttnArgs& a, int h, int b, int64_t pos, bool pos_ok, TailLoads& t,
                                               bool fresh_paged = false) {
  const int wave = tail_tid() >> 6, lane = tail_tid() & 63, cl = lane & 15, rl = lane >> 4;
  const bool fused = PAGED || a.tail_mode == TAIL_FUSED;
  const bool ring = (PAGED || a.tail_mode != TAIL_NONE) && (!fused || pos_ok);
  const bool tok1 = ring && a.tok;
  const uint4 z = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int i = 0; i < 4; ++i) t.k[i] = t.v[i] = z;
  t.fk = t.fv = t.tok = z;
  if (!ring || wave >= RING_PARTS) return;
  if (tok1) {
    if (wave == 0 && lane < 32) t.tok = *reinterpret_cast<const uint4*>(fresh_of(a, b, h, rl) + 8 * cl);
    return;
  }
  const uint16_t* rk = PAGED ? a.rings + (((int64_t)b * a.hkv + h) * 2) * GT * D : ring_of(a, h, 0);
  const uint16_t* rv = PAGED ? rk + GT * D : ring_of(a, h, 1);
  const int slots = PAGED ? GT : (int)a.tail_slots;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t o = (int64_t)min(16 * wave + rl + 4 * i, slots - 1) * D + 8 * cl;
    t.k[i] = *reinterpret_cast<const uint4*>(rk + o);
    t.v[i] = *reinterpret_cast<const uint4*>(rv + o);
  }
  // the new token's slot: from the step's input, not the ring this launch writes
  if ((PAGED ? fresh_paged : a.tail_mode == TAIL_FUSED) && (int)(pos % GT) >> 4 == wave) {
    t.fk = *reinterpret_cast<const uint4*>(fresh_of(a, b, h, 0) + 8 * cl);
    t.fv = *reinterpret_cast<const uint4*>(fresh_of(a, b, h, 1) + 8 * cl);
  }
}

// `flags` (the chained-layer kernel's merger): TB_APPEND, the tail also appends the new token:
// it stores the token into its ring slot (per-token symmetric: the token's codes and scale) and
// rules its group: from the staged ring into the token's channels of group pos / 64
// (append_ring_channels), or, when the token completes the group, by requantizing the whole ring
// from LDS; TB_KEEP_BLOCK, the consumed partial block is left for the caller to zero;
// TB_POISON, the caller's own wait for its inputs gave up: the output is NaN; TB_DIRECT (with
// TB_KEEP_BLOCK, the caller having set sm.ring_done to zero), when every merging wave owns one
// head: each merging wave combines its head with the ring partials and stores the outputs itself
// as soon as its merge is done (no workgroup barrier; a head whose words never arrived is NaN
// alone), and the tail returns without a final barrier; TB_RING_SLOT (paged, with pos_ok): no
// ring attention here: the ring partial that paged_ring_tail publishes in the sequence's ring
// slot takes the ring partials' place in the direct combine (without the direct path it is
// merged as one more prefix partial).
constexpr int TB_APPEND = 1, TB_KEEP_BLOCK = 2, TB_POISON = 4, TB_DIRECT = 8, TB_RING_SLOT = 16;

// The paged workspace: per KV head, per sequence b, its seq_parts[2b + 1] prefix partial slots
// and one more, the ring slot (the paged int8t64 step's ring partial, published by the first of
// the sequence's workgroups to finish its prefix share for the last one): total_parts + nseq
// slots per KV head, so that the ring slot follows the sequence's prefix partials.
__device__ __forceinline__ float* paged_block(const AttnArgs& a, int h, int b) {
  return a.ws + ((int64_t)h * (a.total_parts + a.nseq) + a.seq_parts[2 * b] + b) * part_stride(a.gq);
}
__device__ __forceinline__ float* paged_ring_slot(const AttnArgs& a, int h, int b) {
  return paged_block(a, h, b) + (int64_t)a.seq_parts[2 * b + 1] * part_stride(a.gq);
}

template <bool PAGED>
__device__ __forceinline__ void tail_body(const AttnArgs& a, int h, int b, TailSmem& sm, int run, int64_t pos,
                                          bool pos_ok, int64_t U, const TailLoads* pre = nullptr,
                                          const half8_t (*pre_q)[4] = nullptr, int flags = 0, int64_t page = -1,
                                          int64_t tag_in = -1) {
  const int tid = tail_tid(), wave = tid >> 6, lane = tid & 63;
  // the tag of the tagged output words and flags: the caller's, else a.ftag
  const uint32_t ftag = tag_in >= 0 ? (uint32_t)tag_in : a.ftag;
  const bool poll = run != TAIL_KERNEL;  // partials written in this launch: poll their words
  const int gq = a.gq, pw = part_stride(gq), cols = gq * D;
  const int P0 = PAGED ? min(a.seq_parts[2 * b + 1], WTS) : a.n_parts;  // prefix partials
  const bool fused = PAGED || a.tail_mode == TAIL_FUSED;
  // TB_RING_SLOT: another workgroup attends over the ring and publishes one ring partial in the
  // sequence's ring slot (the slot after its P0 prefix partials: ring_slot needs P0 equal to the
  // sequence's parts, which the caller checks). The direct path merges the prefix partials
  // first and polls the ring slot in its combine, where the ring partials go; otherwise the slot
  // is merged as prefix partial P0.
  const bool ring_slot = PAGED && (flags & TB_RING_SLOT) && pos_ok;
  const bool ring = (PAGED || a.tail_mode != TAIL_NONE) && (!fused || pos_ok) && !(PAGED && (flags & TB_RING_SLOT));
  // while waves 0..3 attend over the ring, the others merge the prefix partials
  const int mbase = ring ? RING_PARTS : 0, nmw = TB_WAVES - mbase;
  const bool direct = (flags & TB_DIRECT) && (flags & TB_KEEP_BLOCK) && P0 + 1 <= 64 && nmw >= gq;
  const bool slot_in_combine = ring_slot && direct;
  const int P = P0 + (ring_slot && !direct ? 1 : 0);
  float* hws = PAGED ? paged_block(a, h, b) : a.ws + (int64_t)h * P0 * pw;
  auto pp = [&](int64_t u) -> float* { return hws + u * pw; };

  // ---- loads: the ring rows (or the new token) and q of the ring waves, the merging waves'
  // partial words
  const bool completes = ring && fused && pos_ok && !a.tok && (pos + 1) % GT == 0;  // the token completes its group
  const bool tok1 = ring && a.tok;  // per-token symmetric fused step: the tail is the new token
  // appends: the chained step's merger, or the paged int8t64 step's tail (TB_APPEND)
  const bool appends = (flags & TB_APPEND) && fused && pos_ok && !(PAGED && a.tok);
  const bool fresh_on = ring && !tok1 && (PAGED ? appends : a.tail_mode == TAIL_FUSED);
  const int fresh_slot = (int)(pos % GT);
  TailLoads tl;
  if (pre) tl = *pre;
  else if (ring) tail_load_rows<PAGED>(a, h, b, pos, pos_ok, tl, PAGED && appends);
  const int64_t first = (!PAGED && ring && a.first_dev) ? *a.first_dev : 0;
  const bool mask_on = ring && a.tail_mode == TAIL_MASK && lane < a.tail_slots && a.tail_mask[lane] != 0;
  half8_t qb[4];
  const int64_t qh0 = (int64_t)b * a.hq + h * gq;  // first query head of this workgroup
  if (ring && wave < RING_PARTS) {
    if (pre_q) {
#pragma unroll
      for (int k = 0; k < 4; ++k) qb[k] = (*pre_q)[k];
    } else {
      load_q(a.q + qh0 * D, gq, qb);
    }
  }
  const int head0 = wave - mbase;
  const bool merging = head0 >= 0 && head0 < gq;
  float mm = NEG_INF, ll = 0.0f;  // merging wave: lane s's m / l of its first head
  uint32_t rm = PUB_KEY, rl = PUB_KEY;  // their published words (beyond P: words of 0.0)
  uint64_t rv[MERGE_PRE];               // and those of its columns 2 lane, 2 lane + 1 of the first MERGE_PRE partials
  int budget = (flags & TB_POISON) ? 0 : MERGER_SPIN_LIMIT;  // (poisoned: the output is NaN anyway)
  if (merging) {
    // (the chained step's merger, appending, loads them first in the poll below: their registers
    // would otherwise stay live across the requantization, which the partials are far from being
    // ready for; the last workgroup's tail finds them all issued)
    const bool pre_ld = !(flags & TB_APPEND) || run == TAIL_LAST;
    if (lane < P) {
      rm = pre_ld ? pub_ld(pp(lane) + gq * D + head0) : 0u;
      rl = pre_ld ? pub_ld(pp(lane) + gq * D + gq + head0) : 0u;
    }
#pragma unroll
    for (int u = 0; u < MERGE_PRE; ++u)
      rv[u] = u < P ? (pre_ld ? pub_ld2(pp(u) + head0 * D + 2 * lane) : 0ull) : PUB_KEY2;
  }

  // ---- each ring wave stages its own 16 slots in LDS (chunk ^ (row & 15) layout), the new token
  // over its slot, and attends over them: no workgroup barrier, except when the token completes
  // its group (the whole ring is then requantized, by every thread, between two barriers)
  uint8_t* ring_k = sm.ring_lds;
  uint8_t* ring_v = sm.ring_lds + RING_BYTES;
  if (ring && wave < RING_PARTS) {
    const int cl = lane & 15, rw = lane >> 4;
    if (tok1) {
      if (wave == 0 && lane < 32) {
        const uint32_t wv[4] = {tl.tok.x, tl.tok.y, tl.tok.z, tl.tok.w};
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = h2f((uint16_t)(wv[j >> 1] >> (16 * (j & 1))));
        float scale;
        const uint2 cw = sym_quant8(v, scale);
        const _Float16 sc = (_Float16)scale;
        *reinterpret_cast<half8_t*>((rw == 0 ? ring_k : ring_v) + (ring_chunk_pos(0, cl) << 4)) =
            dq8_sym(cw.x, cw.y, half2_t{sc, sc});
        if (appends) {
          const int64_t row = (int64_t)h * a.capacity + pos;
          *reinterpret_cast<uint2*>((rw == 0 ? a.kq : a.vq) + row * D + 8 * cl) = cw;
          if (cl == 0) (rw == 0 ? a.ksc : a.vsc)[row] = f2h(scale);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 16 * wave + rw + 4 * i, o = r * (2 * D) + (ring_chunk_pos(r, cl) << 4);
        *reinterpret_cast<uint4*>(ring_k + o) = tl.k[i];
        *reinterpret_cast<uint4*>(ring_v + o) = tl.v[i];
      }
      // (program order: these stores land after the quarter's stores of the same row)
      if (fresh_on && fresh_slot >> 4 == wave && (fresh_slot & 3) == rw) {
        const int o = fresh_slot * (2 * D) + (ring_chunk_pos(fresh_slot, cl) << 4);
        *reinterpret_cast<uint4*>(ring_k + o) = tl.fk;
        *reinterpret_cast<uint4*>(ring_v + o) = tl.fv;
        if (appends) {  // the ring slot of the new token
          *reinterpret_cast<uint4*>(ring_row<PAGED>(a, b, h, 0, fresh_slot) + 8 * cl) = tl.fk;
          *reinterpret_cast<uint4*>(ring_row<PAGED>(a, b, h, 1, fresh_slot) + 8 * cl) = tl.fv;
        }
      }
    }
  }
  // the chained step's append of a token that does not complete its group: the ring waves rule it
  // from the staged ring after their attention, while the merging waves poll (nothing in the launch
  // reads that group); they meet through ring_staged (set to zero by the caller before the tail)
  const bool ring_append = appends && !completes && !tok1;
  if (ring_append && wave < RING_PARTS) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (lane == 0) __hip_atomic_fetch_add(&sm.ring_staged, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  if (appends && completes) {
    __syncthreads();
    requant_ring_lds<true, PAGED>(sm.ring_lds, sm.rq_ext, true, &a, h, pos, b, page);
    __syncthreads();
  } else if (completes) {
    __syncthreads();
    requant_ring_lds<false>(sm.ring_lds, sm.rq_ext, true);
    __syncthreads();
  } else {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's slots are in LDS
  }

  if (wave < mbase) {
    // ---- ring attention: 4 waves x 16 tokens, one partial each
    const int64_t written = fused ? pos + 1 : (a.tail_mode == TAIL_SCALARS ? *a.written_dev : 0);
    uint64_t bits;
    if (completes) bits = ~0ull;
    else if (tok1) bits = wave == 0 ? 1ull : 0ull;
    else if (a.tail_mode == TAIL_MASK) bits = __builtin_amdgcn_ballot_w64(mask_on);
    else bits = ring_bits(written, U, first);
    WaveState st;
    state_init(st);
    attend_ring16(a, st, qb, ring_k, ring_v, wave, bits);
    store_wave_partial(st, gq, sm.ring_part[wave]);
    if (direct) {  // the merging waves read it as soon as every ring wave has counted itself
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (lane == 0) __hip_atomic_fetch_add(&sm.ring_done, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    if (ring_append) {
      while (__hip_atomic_load(&sm.ring_staged, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < RING_PARTS)
        __builtin_amdgcn_s_sleep(1);
      append_ring_channels<PAGED>(a, h, pos, sm.ring_lds, sm.xpose, b, page);
    }
  } else if (merging) {
    // (this code runs once per launch on a cold instruction cache, at ~30 ns per 64-byte line:
    // the common shape, one head per merging wave and P <= 64, takes a short straight path)
    bool lost = false;  // a word never arrived (the wait gave up)
    if (poll) {
      // ---- every word still zero is reloaded together (m, l and the column pairs: the last
      // partial's words then arrive in one round trip), until none is left
      for (;;) {
        bool miss = rm == 0 || rl == 0;
#pragma unroll
        for (int u = 0; u < MERGE_PRE; ++u) miss |= rv[u] == 0;
        if (!__builtin_amdgcn_ballot_w64(miss)) break;
        if (budget <= 0) {
          lost = true;
          break;
        }
        --budget;
        __builtin_amdgcn_s_sleep(1);
        if (rm == 0) rm = pub_ld(pp(lane) + gq * D + head0);
        if (rl == 0) rl = pub_ld(pp(lane) + gq * D + gq + head0);
#pragma unroll
        for (int u = 0; u < MERGE_PRE; ++u)
          if (rv[u] == 0) rv[u] = pub_ld2(pp(u) + head0 * D + 2 * lane);
      }
    }
    if (lane < P) {
      mm = pub_f(rm);
      ll = pub_f(rl);
    }
    const bool one_head = P <= 64 && head0 + nmw >= gq;  // the common shape
    // ---- prefix merge, one head at a time per merging wave (lane s (+ 64 k) = partial s for
    // the weights, two columns per lane for the sum): m_p = max_s m_s, w_s = 2^(m_s - m_p),
    // l_p = sum_s w_s l_s, pre_acc = sum_s w_s acc_s
    float* wb = sm.wts + wave * WTS;
    if (one_head) {
      // one head, one chunk of partials: lane s holds m_s and l_s already
      const float ms = lane < P ? mm : NEG_INF;
      const float m = wave_max(ms);
      const float w = (lane < P && ms != NEG_INF) ? __builtin_amdgcn_exp2f(ms - m) : 0.0f;
      wb[lane] = w;
      const float l = wave_sum(lane < P ? ll * w : 0.0f);
      float2 acc = {0.0f, 0.0f};
#pragma unroll
      for (int u = 0; u < MERGE_PRE; ++u) {
        const float2 vv = pub_f2(rv[u]);
        acc.x += vv.x * wb[u];
        acc.y += vv.y * wb[u];
      }
#pragma unroll 1
      for (int sb = MERGE_PRE; sb < P; sb += 8) {
        uint64_t w8[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
          w8[j] = sb + j < P ? pub_ld2(pp(sb + j) + head0 * D + 2 * lane) : 1;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if (sb + j >= P) break;
          const uint64_t wv = pub_repoll2(pp(sb + j) + head0 * D + 2 * lane, w8[j], budget);
          lost |= wv == 0;
          const float2 vv = pub_f2(wv);
          acc.x += vv.x * wb[sb + j];
          acc.y += vv.y * wb[sb + j];
        }
      }
      if (direct) {
        // ---- combine (the combine below, for this head's column pair 2 lane, 2 lane + 1)
        if (ring)
          while (__hip_atomic_load(&sm.ring_done, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < RING_PARTS)
            __builtin_amdgcn_s_sleep(1);
        const int col = head0 * D + 2 * lane;
        float M = m, mr[RING_PARTS], lr[RING_PARTS];
        float2 ar[RING_PARTS];
#pragma unroll
        for (int r = 0; r < RING_PARTS; ++r) {
          mr[r] = ring ? sm.ring_part[r][gq * D + head0] : NEG_INF;
          lr[r] = ring ? sm.ring_part[r][gq * D + gq + head0] : 0.0f;
          ar[r] = ring ? *reinterpret_cast<const float2*>(sm.ring_part[r] + col) : float2{0.0f, 0.0f};
        }
        if (slot_in_combine) {
          // the ring workgroup's partial, in place of the four ring partials
          const float* rs = pp(P0);
          const uint32_t wm = pub_repoll(rs + gq * D + head0, pub_ld(rs + gq * D + head0), budget);
          const uint32_t wl = pub_repoll(rs + gq * D + gq + head0, pub_ld(rs + gq * D + gq + head0), budget);
          const uint64_t wv = pub_repoll2(rs + col, pub_ld2(rs + col), budget);
          lost |= wm == 0 || wl == 0 || wv == 0;
          mr[0] = pub_f(wm);
          lr[0] = pub_f(wl);
          ar[0] = pub_f2(wv);
        }
#pragma unroll
        for (int r = 0; r < RING_PARTS; ++r) M = fmaxf(M, mr[r]);
        const bool failed = (flags & TB_POISON) != 0 || __builtin_amdgcn_ballot_w64(lost) != 0;
        const float Mu = M == NEG_INF ? 0.0f : M;
        const float alpha = m == NEG_INF ? 0.0f : __builtin_amdgcn_exp2f(m - Mu);
        float ox = alpha * acc.x, oy = alpha * acc.y, lt = alpha * l;
#pragma unroll
        for (int r = 0; r < RING_PARTS; ++r) {
          const float beta = mr[r] == NEG_INF ? 0.0f : __builtin_amdgcn_exp2f(mr[r] - Mu);
          ox += beta * ar[r].x;
          oy += beta * ar[r].y;
          lt += beta * lr[r];
        }
        const int64_t qh = qh0 + head0;
        ox = failed ? __builtin_nanf("") : (lt > 0.0f ? ox / lt : 0.0f);
        oy = failed ? __builtin_nanf("") : (lt > 0.0f ? oy / lt : 0.0f);
        const uint32_t pair = (uint32_t)f2h(ox) | ((uint32_t)f2h(oy) << 16);
        *reinterpret_cast<uint32_t*>(a.out + qh * D + 2 * lane) = pair;
        if (a.fwd_out)
          hand_st(a.fwd_out + qh * D / 2 + lane, ((uint64_t)ftag << 32) | pair, l2_local(a) && !a.fwd_agent);
        if (a.lse && lane == 0)
          a.lse[qh] = failed ? __builtin_nanf("") : (lt > 0.0f ? (M + __log2f(lt) - P_SCALE_LOG2) * LN2 : NEG_INF);
        // this head's outputs are issued: count it for the readers of the next layer (they
        // validate the words themselves, so no ordering is needed)
        if (a.issue_flags && lane == 0) {
#pragma unroll
          for (int c = 0; c < FLAG_COPIES; ++c)
            __hip_atomic_store(a.issue_flags + c * a.hq + qh, ftag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      } else {
        *reinterpret_cast<float2*>(sm.pre_acc + head0 * D + 2 * lane) = acc;
        if (lane == 0) {
          sm.pre_m[head0] = m;
          sm.pre_l[head0] = l;
        }
      }
    } else {
      for (int head = head0; head < gq; head += nmw) {
        const bool own = head == head0;
        float ls[WTS / 64];
        float m = NEG_INF;
#pragma unroll 1
        for (int k = 0; k < WTS / 64; ++k) {
          const int s = 64 * k + lane;
          ls[k] = 0.0f;
          if (s >= P) continue;
          float ms;
          if (own && k == 0) {
            ms = mm;
            ls[k] = ll;
          } else {
            const float* pm = pp(s) + gq * D + head;
            const uint32_t wm = pub_repoll(pm, pub_ld(pm), budget);
            const uint32_t wl = pub_repoll(pm + gq, pub_ld(pm + gq), budget);
            lost |= wm == 0 || wl == 0;
            ms = pub_f(wm);
            ls[k] = pub_f(wl);
          }
          wb[s] = ms;
          m = fmaxf(m, ms);
        }
        m = wave_max(m);
        float l = 0.0f;
#pragma unroll 1
        for (int k = 0; k < WTS / 64; ++k) {
          const int s = 64 * k + lane;
          if (s >= P) continue;
          const float ms = wb[s];
          const float w = ms == NEG_INF ? 0.0f : __builtin_amdgcn_exp2f(ms - m);
          wb[s] = w;
          l += ls[k] * w;
        }
        l = wave_sum(l);
        float2 acc = {0.0f, 0.0f};
        int s0 = 0;
        if (own) {
#pragma unroll
          for (int u = 0; u < MERGE_PRE; ++u) {
            const float w = u < P ? wb[u] : 0.0f;
            const float2 vv = pub_f2(rv[u]);
            acc.x += vv.x * w;
            acc.y += vv.y * w;
          }
          s0 = MERGE_PRE;
        }
#pragma unroll 1
        for (int sb = s0; sb < P; sb += 8) {
          uint64_t w8[8];
#pragma unroll
          for (int j = 0; j < 8; ++j)
            w8[j] = sb + j < P ? pub_ld2(pp(sb + j) + head * D + 2 * lane) : 1;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            if (sb + j >= P) break;
            const uint64_t wv = pub_repoll2(pp(sb + j) + head * D + 2 * lane, w8[j], budget);
            lost |= wv == 0;
            const float2 vv = pub_f2(wv);
            acc.x += vv.x * wb[sb + j];
            acc.y += vv.y * wb[sb + j];
          }
        }
        *reinterpret_cast<float2*>(sm.pre_acc + head * D + 2 * lane) = acc;
        if (lane == 0) {
          sm.pre_m[head] = m;
          sm.pre_l[head] = l;
        }
      }
    }
    if (lane == 0) sm.lost[wave] = __builtin_amdgcn_ballot_w64(lost) != 0;
  }
  if (direct) return;
  __syncthreads();

  // ---- combine: one column per thread. Prefix: acc_p = sum_s w_s acc_s; then with the
  // ring's partials r: M = max(m_p, m_r), alpha = 2^(m_p - M), beta_r = 2^(m_r - M)
  bool failed = (flags & TB_POISON) != 0;
  for (int w = mbase; w < TB_WAVES; ++w) failed |= w - mbase < gq && sm.lost[w] != 0;
  for (int col = tid; col < cols; col += TB_THREADS) {
    const int head = col / D;
    const float accp = sm.pre_acc[col];
    const float mp = sm.pre_m[head];
    float M = mp, mr[RING_PARTS], lr[RING_PARTS], ar[RING_PARTS];
#pragma unroll
    for (int r = 0; r < RING_PARTS; ++r) {
      if (ring) {
        mr[r] = sm.ring_part[r][gq * D + head];
        lr[r] = sm.ring_part[r][gq * D + gq + head];
        ar[r] = sm.ring_part[r][col];
      } else {
        mr[r] = NEG_INF;
        lr[r] = 0.0f;
        ar[r] = 0.0f;
      }
      M = fmaxf(M, mr[r]);
    }
    const float Mu = M == NEG_INF ? 0.0f : M;
    const float alpha = mp == NEG_INF ? 0.0f : __builtin_amdgcn_exp2f(mp - Mu);
    float acc = alpha * accp, l = alpha * sm.pre_l[head];
#pragma unroll
    for (int r = 0; r < RING_PARTS; ++r) {
      const float beta = mr[r] == NEG_INF ? 0.0f : __builtin_amdgcn_exp2f(mr[r] - Mu);
      acc += beta * ar[r];
      l += beta * lr[r];
    }
    const int64_t qh = qh0 + head;
    const int d = col % D;
    // acc and l carry the same 2^15 scale; a merger that gave up writes NaN
    const float o = failed ? __builtin_nanf("") : (l > 0.0f ? acc / l : 0.0f);
    const uint16_t o16 = f2h(o);
    a.out[(int64_t)qh * D + d] = o16;
    if (a.fwd_out) {  // (columns come in pairs of neighbouring lanes: d even in the even lane)
      const uint32_t pair = (uint32_t)__shfl_xor((int)o16, 1, 64);
      if ((d & 1) == 0)
        hand_st(a.fwd_out + ((int64_t)qh * D + d) / 2, ((uint64_t)ftag << 32) | o16 | (pair << 16),
                l2_local(a) && !a.fwd_agent);
    }
    if (a.lse && d == 0) a.lse[qh] = failed ? __builtin_nanf("") : (l > 0.0f ? (M + __log2f(l) - P_SCALE_LOG2) * LN2 : NEG_INF);
  }
  if (a.issue_flags) {  // every column issued: the workgroup's gq heads flagged at once
    __syncthreads();
    if (tid < gq * FLAG_COPIES)
      __hip_atomic_store(a.issue_flags + (tid / gq) * a.hq + qh0 + tid % gq, ftag, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }
  // ---- every word of the head's partials was consumed before the barrier above: the whole
  // block [hws, hws + P pw) goes back to zero (plain 16-byte stores by every thread; pw is a
  // multiple of 4; no one touches these words again in this launch, and the launch boundary
  // orders the stores before the next launch's accesses)
  if (flags & TB_KEEP_BLOCK) return;
  uint4* blk = reinterpret_cast<uint4*>(hws);
  for (int i = tid; i < P * pw / 4; i += TB_THREADS) blk[i] = uint4{0u, 0u, 0u, 0u};
}

// The paged int8t64 step's ring work for (sequence b, KV head h), by the first of the sequence's
// workgroups to finish its prefix share (pos_ok): the ring rows and the new token (`tl`, loaded by
// tail_load_rows as its prefix loop ended; q the loop's operand `qb`) staged in LDS as tail_body
// stages them; then waves 0..3 attend over the ring (4 x 16 tokens) and publish the
// four ring partials merged into one (pub_st) in the ring slot (paged_ring_slot), while waves
// 4..7 append the new token (its ring slot; its group's codes and rulers in the page, from the
// staged ring). A token that completes its group is appended by requantizing the whole ring, by
// every thread before the attention, the ring then attended as int8 as in tail_body. The last of
// the sequence's workgroups merges the ring slot with the prefix partials (TB_RING_SLOT).
__device__ __forceinline__ void paged_ring_tail(const AttnArgs& a, int h, int b, TailSmem& sm, int64_t pos, int64_t U,
                                                const TailLoads& tl, const half8_t (&qb)[4]) {
  const int tid = tail_tid(), wave = tid >> 6, lane = tid & 63;
  const int gq = a.gq;
  const int64_t page = page_of(a, b, pos / GT);  // (the append needs it last)
  const bool completes = (pos + 1) % GT == 0;
  const int fresh_slot = (int)(pos % GT);
  uint8_t* ring_k = sm.ring_lds;
  uint8_t* ring_v = sm.ring_lds + RING_BYTES;
  if (wave < RING_PARTS) {
    const int cl = lane & 15, rw = lane >> 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * wave + rw + 4 * i, o = r * (2 * D) + (ring_chunk_pos(r, cl) << 4);
      *reinterpret_cast<uint4*>(ring_k + o) = tl.k[i];
      *reinterpret_cast<uint4*>(ring_v + o) = tl.v[i];
    }
    // (program order: these stores land after the quarter's stores of the same row)
    if (fresh_slot >> 4 == wave && (fresh_slot & 3) == rw) {
      const int o = fresh_slot * (2 * D) + (ring_chunk_pos(fresh_slot, cl) << 4);
      *reinterpret_cast<uint4*>(ring_k + o) = tl.fk;
      *reinterpret_cast<uint4*>(ring_v + o) = tl.fv;
      *reinterpret_cast<uint4*>(ring_row<true>(a, b, h, 0, fresh_slot) + 8 * cl) = tl.fk;
      *reinterpret_cast<uint4*>(ring_row<true>(a, b, h, 1, fresh_slot) + 8 * cl) = tl.fv;
    }
  }
  __syncthreads();  // the whole ring is in LDS
  if (completes) {
    requant_ring_lds<true, true>(sm.ring_lds, sm.rq_ext, true, &a, h, pos, b, page);
    __syncthreads();
  }
  if (wave >= RING_PARTS) {
    // waves 4..7: the append of a token that does not complete its group (one that does was
    // stored above), beside the ring attention
    if (!completes) append_ring_channels<true>(a, h, pos, sm.ring_lds, sm.xpose, b, page, 64 * RING_PARTS);
    return;
  }
  WaveState st;
  state_init(st);
  attend_ring16(a, st, qb, ring_k, ring_v, wave, completes ? ~0ull : ring_bits(pos + 1, U, 0));
  store_wave_partial(st, gq, sm.ring_part[wave]);
  // the four ring waves meet (sm.ring_done, zero before the tail), not the workgroup
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  if (lane == 0) __hip_atomic_fetch_add(&sm.ring_done, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
  while (__hip_atomic_load(&sm.ring_done, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < RING_PARTS)
    __builtin_amdgcn_s_sleep(1);
  // one partial from the four: m = max_r m_r, w_r = 2^(m_r - m), l = sum_r w_r l_r,
  // acc = sum_r w_r acc_r, two columns a thread of waves 0..3
  float* dst = paged_ring_slot(a, h, b);
  const bool l2 = l2_local(a);
  for (int e = 2 * tid; e < gq * D; e += 2 * 64 * RING_PARTS) {
    const int head = e / D;
    float m = NEG_INF;
#pragma unroll
    for (int r = 0; r < RING_PARTS; ++r) m = fmaxf(m, sm.ring_part[r][gq * D + head]);
    const float mu = m == NEG_INF ? 0.0f : m;
    float x = 0.0f, y = 0.0f, l = 0.0f;
#pragma unroll
    for (int r = 0; r < RING_PARTS; ++r) {
      const float mr = sm.ring_part[r][gq * D + head];
      const float w = mr == NEG_INF ? 0.0f : __builtin_amdgcn_exp2f(mr - mu);
      l += sm.ring_part[r][gq * D + gq + head] * w;
      x += sm.ring_part[r][e] * w;
      y += sm.ring_part[r][e + 1] * w;
    }
    pub_st2(dst + e, x, y, l2);
    if (e % D == 0) {
      pub_st(dst + gq * D + head, m, l2);
      pub_st(dst + gq * D + gq + head, l, l2);
    }
  }
}

// ---------------------------------------------------------------- the fused projection step
//
// nkv_decode_step_qkv_t64 runs a decoder layer's input RMSNorm, its stacked q/k/v projection and
// the q/k head norms with the rotary embedding in the fused decode step's launch, ahead of the
// append, prefix and tail: the first K/V groups stream in while the projection is computed. The
// (gq + 2) D rows of KV head h's block (its gq q heads, its k and v head) are split over the
// head's workgroups; each computes its rows exactly as gemv_kernel does (the same input chunks
// per thread, reduction and summation order, fp16 results), publishes them as tagged words (the
// launch's tag in the high half: qkv_epoch[h] + 1) and reads back the head's vectors. Waves
// QKV_WAVES.. compute nothing: they issue every wave's first group and the append unit's ring
// rows, so that the computing waves' load counters hold no LDS-DMA while they wait for rows.
constexpr uint64_t LAYER_WAIT_TICKS = 20000000ull;  // 0.2 s of the 100 MHz real-time counter per wait
constexpr int QKV_WAVES = 6;                   // waves computing rows
constexpr int QKV_MAX_NL = 6;                  // 16-byte input chunks per lane and row
constexpr int QKV_MAX_HIDDEN = 64 * 8 * QKV_MAX_NL;  // 3072: the input chunks fit one chunk per thread
constexpr int QKV_ROWS = 4;                    // rows of a wave in flight at once
constexpr int QKV_MAX_GQ = 4;                 // q heads per KV head (waves 0..3 fetch them)
constexpr int QKV_HAND_ROWS = (QKV_MAX_GQ + 2) * D;  // tagged row words per KV head

// The append unit's ring rows (the new token comes from the prologue, in LDS).
__device__ __forceinline__ void issue_unit_ring(const UnitIO& io, int unit, uint32_t src) {
  const int lane = threadIdx.x & 63, ch0 = unit % (D / UNIT_CH) * UNIT_CH;
  dma16(uniform_ptr(io.ring + ch0), (uint32_t)(lane * D * 2), src);
}

// The prologue (`issued`: an LDS counter at zero, which each computing wave increments once its
// first rows' weight loads are issued): this workgroup's rows of head h's block, computed and
// published; then the head's
// q vectors (normalized, rotated) into q_lds, k (normalized, rotated) and v into kv_lds [2][D],
// the append unit's 8 channels of the new token into unit_src's last row (`unit` >= 0), and, in
// part 0, k / v into the step's k_new / v_new and every vector into qkv_out. No workgroup barrier:
// each computing wave normalizes its own copy of the input, in the order gemv_kernel does
// (lane l holds input chunks l + 64 u, which gemv_kernel's wave u holds in lane l: the wave sums
// of the squares are its waves' sums, added in the same order). Returns false when a wait for
// rows gave up (its vectors are then NaN).
// (always inlined: called out of line, it takes the kernel's arguments by reference, which then
// live in scratch memory for the whole launch)
__device__ __forceinline__ bool qkv_prologue(const AttnArgs& a, int h, int part, int parts, int64_t pos, uint32_t tag, int unit,
                             uint16_t* q_lds, uint16_t* kv_lds, uint16_t* unit_src, int* issued) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nch = a.hidden / 8, nl = (nch + 63) / 64;
  const int gq = a.gq, nrows = (gq + 2) * D;
  const int rw = (nrows + parts - 1) / parts, r0 = min(part * rw, nrows), r1 = min(r0 + rw, nrows);
  const int rpw = (rw + QKV_WAVES - 1) / QKV_WAVES;
  const bool l2 = l2_local(a);
  uint64_t* hw = a.hand + (int64_t)h * QKV_HAND_ROWS;
  if (wave < QKV_WAVES) {
    const int wr0 = min(r0 + wave * rpw, r1), wr1 = min(wr0 + rpw, r1);
    // head h's row r of the stacked weight: its gq q heads, then its k head, then its v head
    auto row_ptr = [&](int r) -> const uint16_t* {
      const int vec = r / D, d = r % D;
      const int64_t g = vec < gq ? (int64_t)h * gq + vec : (vec == gq ? a.hq + h : a.hq + a.hkv + h);
      return a.w_qkv + (g * D + d) * (int64_t)a.hidden;
    };
    uint4 xn[QKV_MAX_NL], gm[QKV_MAX_NL];
#pragma unroll
    for (int u = 0; u < QKV_MAX_NL; ++u) {
      const int c = lane + 64 * u;
      const bool in = u < nl && c < nch;
      xn[u] = in ? *reinterpret_cast<const uint4*>(a.x + 8 * c) : uint4{0u, 0u, 0u, 0u};
      gm[u] = in ? *reinterpret_cast<const uint4*>(a.x_gamma + 8 * c) : uint4{0u, 0u, 0u, 0u};
    }
    uint4 wv[QKV_ROWS][QKV_MAX_NL];
    auto issue = [&](int rb) {
#pragma unroll
      for (int j = 0; j < QKV_ROWS; ++j)
#pragma unroll
        for (int u = 0; u < QKV_MAX_NL; ++u) {
          const int c = lane + 64 * u;
          wv[j][u] = (u < nl && rb + j < wr1 && c < nch) ? ld_weight(row_ptr(rb + j) + 8 * c) : uint4{0u, 0u, 0u, 0u};
        }
    };
    issue(wr0);  // the first rows' weights fly while the input is normalized
    // (counted once issued: the other waves hold the first groups' loads back until every
    // computing wave's weights are requested, so that HBM serves the rows first)
    if (lane == 0) __hip_atomic_fetch_add(issued, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    float tot = 0.0f;
#pragma unroll
    for (int u = 0; u < QKV_MAX_NL; ++u) tot += hsum64(sumsq8(xn[u], 0.0f));  // (chunks past the input are 0)
    const float r = rsqrtf(tot * (1.0f / (float)a.hidden) + a.eps_x);  // torch: mean = sum * (1/n), then rsqrt
#pragma unroll
    for (int u = 0; u < QKV_MAX_NL; ++u) xn[u] = rms_scale8(xn[u], gm[u], r);
    // the rows: fp32 dot products in gemv_kernel's order, rounded to fp16, published as tagged words
    for (int rb = wr0; rb < wr1; rb += QKV_ROWS) {
      if (rb != wr0) issue(rb);
      float acc[QKV_ROWS];
#pragma unroll
      for (int j = 0; j < QKV_ROWS; ++j) acc[j] = 0.0f;
#pragma unroll
      for (int u = 0; u < QKV_MAX_NL; ++u) {
        if (u < nl && lane + 64 * u < nch) {
#pragma unroll
          for (int j = 0; j < QKV_ROWS; ++j) acc[j] = dot8(wv[j][u], xn[u], acc[j]);
        }
      }
#pragma unroll
      for (int j = 0; j < QKV_ROWS; ++j) {
        const float sum = hsum64(acc[j]);
        if (lane == 0 && rb + j < wr1) hand_st(hw + rb + j, ((uint64_t)tag << 32) | f2h(sum), l2);
      }
    }
  }
  // the head's vectors: wave v < gq takes q head v, wave 4 k, wave 5 v; lane l its elements l and
  // l + 64 (the pair the rotary embedding mixes)
  bool ok = true;
  const int vec = wave < gq ? wave : (wave == 4 ? gq : (wave == 5 ? gq + 1 : -1));
  if (vec >= 0) {
    const uint64_t* src = hw + vec * D;
    uint64_t w0 = 0, w1 = 0;  // (tag 0 is never current)
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    for (;;) {
      if ((uint32_t)(w0 >> 32) != tag) w0 = __hip_atomic_load(src + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if ((uint32_t)(w1 >> 32) != tag) w1 = __hip_atomic_load(src + lane + 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const bool miss = (uint32_t)(w0 >> 32) != tag || (uint32_t)(w1 >> 32) != tag;
      if (!__builtin_amdgcn_ballot_w64(miss)) break;
      if (__builtin_amdgcn_s_memrealtime() - t0 > LAYER_WAIT_TICKS) {
        ok = false;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    uint16_t lo = (uint16_t)w0, hi = (uint16_t)w1;
    if (vec <= gq) {
      const uint16_t* g = vec < gq ? a.q_gamma : a.k_gamma;
      qk_norm_rope_lane(h2f(lo), h2f(hi), h2f(g[lane]), h2f(g[lane + 64]), a.eps_qk, (float)pos * a.inv_freq[lane],
                        lo, hi);
    }
    if (!ok) lo = hi = 0x7E00u;  // NaN
    uint16_t* dst = vec < gq ? q_lds + vec * D : kv_lds + (vec - gq) * D;
    dst[lane] = lo;
    dst[lane + 64] = hi;
    // the append unit's channels of the new token (unit u: channels 8 (u % 16) .. + 7 of k (u < 16) or v)
    const int which = vec - gq, ch0 = unit % (D / UNIT_CH) * UNIT_CH;
    if (which >= 0 && unit >= 0 && unit / (D / UNIT_CH) == which) {
      if (lane - ch0 >= 0 && lane - ch0 < UNIT_CH) unit_src[GT * UNIT_CH + lane - ch0] = lo;
      if (lane + 64 - ch0 >= 0 && lane + 64 - ch0 < UNIT_CH) unit_src[GT * UNIT_CH + lane + 64 - ch0] = hi;
    }
    if (part == 0) {
      if (which >= 0) {  // the step's new token, read by this workgroup's tail
        uint16_t* kv = const_cast<uint16_t*>(which == 0 ? a.k_new : a.v_new) + (int64_t)h * a.kv_hs;
        kv[lane] = lo;
        kv[lane + 64] = hi;
      }
      if (a.qkv_out) {
        const int64_t g = vec < gq ? (int64_t)h * gq + vec : (vec == gq ? a.hq + h : a.hq + a.hkv + h);
        a.qkv_out[g * D + lane] = lo;
        a.qkv_out[g * D + lane + 64] = hi;
      }
    }
  }
  return ok;
}

// ---- the output projection in the attention block's launch (w_o): h1 = x + W_o out, where out
// is every head's attention output of this launch. The mergers (part 0 of each head) finish
// last; the other workgroups, done with their partials, stream W_o meanwhile: reader wave g of the
// R WAVES (R = the workgroups of parts 1..) takes rows g and g + R WAVES. A row is computed as
// nkv_gemv computes it (lane l holds 16-byte chunks l + 64 u, fp32 dot products in chunk order,
// the wave sum in hsum64's order, the fp16 result, then the residual added in fp16), so h1 is
// bit for bit that launch's. out arrives as the mergers' tagged words (agent scope): each wave
// polls the hq issue flags of its copy, then every thread fetches its words (reloading those
// still stale) into LDS. A wait that gives up leaves NaN in the row.
constexpr int OP_NL = 8;  // 16-byte chunks per lane of a W_o row: hq D <= 4096

__device__ __forceinline__ void oproj_rows(const AttnArgs& a, int h, int part, uint32_t tag, uint8_t* lds_raw) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nw = ((int)gridDim.x - a.hkv) * WAVES;
  const int g = ((part - 1) * a.hkv + h) * WAVES + wave;
  const int nch = a.hq * D / 8;
  const int r0 = g, r1 = g + nw;
  const bool v0 = r0 < a.hidden, v1 = r1 < a.hidden;
  // (the barrier waits for the partial's stores: W_o then goes out ~2 us after the partial,
  // when fewer parts still stream; issued before it, the step measured 0.6% slower)
  __syncthreads();  // every wave is past the partial's merge: the stages are free for out
  uint4 w0[OP_NL], w1[OP_NL];
#pragma unroll
  for (int u = 0; u < OP_NL; ++u) {
    const int c = lane + 64 * u;
    w0[u] = v0 && c < nch ? ld_weight(a.w_o + (int64_t)r0 * nch * 8 + 8 * c) : uint4{0, 0, 0, 0};
  }
#pragma unroll
  for (int u = 0; u < OP_NL; ++u) {
    const int c = lane + 64 * u;
    w1[u] = v1 && c < nch ? ld_weight(a.w_o + (int64_t)r1 * nch * 8 + 8 * c) : uint4{0, 0, 0, 0};
  }
  const uint16_t x0 = v0 ? a.x[r0] : (uint16_t)0, x1 = v1 ? a.x[r1] : (uint16_t)0;
  // every head's output issued: the hq flags of copy h mod FLAG_COPIES (hq <= 64, one per lane)
  const uint32_t* flags = a.issue_flags + (h % FLAG_COPIES) * a.hq;
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  bool ok = true;
  uint32_t f = lane < a.hq ? 0u : tag;
  for (;;) {
    if (f != tag) f = __hip_atomic_load(flags + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (!__builtin_amdgcn_ballot_w64(f != tag)) break;
    if (__builtin_amdgcn_s_memrealtime() - t0 > LAYER_WAIT_TICKS) {
      ok = false;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  // the words (hq D / 2 of them): thread t takes t + THREADS j
  uint32_t* o32 = reinterpret_cast<uint32_t*>(lds_raw);
  const int nwords = nch * 4;
  for (int e = tid; e < nwords; e += THREADS) {
    uint64_t w = __hip_atomic_load(a.fwd_out + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    while (ok && (uint32_t)(w >> 32) != tag) {  // (a flag seen before its head's words)
      if (__builtin_amdgcn_s_memrealtime() - t0 > LAYER_WAIT_TICKS) {
        ok = false;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
      w = __hip_atomic_load(a.fwd_out + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    o32[e] = (uint32_t)(w >> 32) == tag ? (uint32_t)w : 0x7E007E00u;
  }
  __syncthreads();
  const uint4* o4 = reinterpret_cast<const uint4*>(lds_raw);
  float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
  for (int u = 0; u < OP_NL; ++u) {
    const int c = lane + 64 * u;
    if (c < nch) {
      const uint4 xv = o4[c];
      acc0 = dot8(w0[u], xv, acc0);
      acc1 = dot8(w1[u], xv, acc1);
    }
  }
  acc0 = hsum64(acc0);
  acc1 = hsum64(acc1);
  if (lane == 0) {  // the projection's fp16 result, then the residual added in fp16
    if (v0)
      a.h1_out[r0] = f2h((float)(_Float16)((float)(_Float16)acc0 + (float)__builtin_bit_cast(_Float16, x0)));
    if (v1)
      a.h1_out[r1] = f2h((float)(_Float16)((float)(_Float16)acc1 + (float)__builtin_bit_cast(_Float16, x1)));
  }
}

template <int LAYOUT, bool QKV = false>
__global__ __launch_bounds__(THREADS, 1) void attn_prefix_kernel(AttnArgs a) {
  constexpr bool TOK = LAYOUT == CONTIG_TOK || LAYOUT == PAGED_TOK;
  constexpr bool PAGED = LAYOUT == PAGED_T64 || LAYOUT == PAGED_TOK;
  __shared__ __attribute__((aligned(16))) uint8_t lds_raw[TOK ? LDS_BYTES_TOK : LDS_BYTES];
  __shared__ __attribute__((aligned(16))) uint16_t unit_src[TOK || PAGED ? 8 : UNIT_SRC_BYTES / 2];
  __shared__ __attribute__((aligned(16))) uint16_t q_lds[16 * D];
  __shared__ __attribute__((aligned(16))) float xch[UNIT_CH * 2 * WAVES];
  __shared__ int ticket;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = blockIdx.x % a.hkv;
  // work unit -> (sequence, part of its prefix, parts of that sequence, partial slot)
  int b = 0, part = blockIdx.x / a.hkv, nparts = a.n_parts;
  const int pslot = part;
  if constexpr (PAGED) {
    const int m = a.wg_map[pslot];
    b = m >> 16;
    part = m & 0xffff;
    nparts = a.seq_parts[2 * b + 1];
  }
  constexpr int wave_lds = TOK ? WAVE_LDS_TOK : WAVE_LDS;
  constexpr int slot_bytes = TOK ? HALF_SLOT_TOK : HALF_SLOT;
  uint8_t* my_stages = lds_raw + wave * wave_lds;
  const uint32_t my_lds = __builtin_amdgcn_readfirstlane(lds_addr(my_stages));
  const uint32_t src_lds = __builtin_amdgcn_readfirstlane(lds_addr(unit_src));

  int64_t pos;
  bool pos_ok;
  int64_t U;
  if constexpr (PAGED) {
    // int8t64: the ring holds the group of pos (appended before this launch); per-token
    // symmetric: the prefix is every token before pos, and this launch appends pos
    pos = a.pos_dev[b];
    pos_ok = pos >= 0 && page_of(a, b, pos / GT) >= 0;  // the current group has a page
    U = pos_ok ? (TOK ? pos : pos / GT * GT) : 0;
  } else {
    U = prefix_limit(a, pos, pos_ok);
  }
  // the fused step's append: int8t64 units in parts < APPEND_UNITS (the grid has at least
  // that many parts), the per-token symmetric token in part 0 (of each sequence when paged;
  // the paged int8t64 step appends in a launch of its own)
  const bool append = (PAGED ? TOK : a.tail_mode == TAIL_FUSED) && pos_ok && (TOK ? part == 0 : part < APPEND_UNITS);
  const bool prefix = part < nparts;

  const int64_t W = (U + GT - 1) / GT;
  const int64_t gs = prefix ? (int64_t)part * W / nparts : 0;
  const int64_t ge = prefix ? (int64_t)(part + 1) * W / nparts : 0;
  // Groups gs + gi, gi < ng: wave w takes gi = w, w + WAVES, ... (a fixed assignment, so a
  // partial's summation order, and the result, are the same on every run). A group's
  // halves (32 tokens) go to slots 0 and 1 (int8t64: its rulers to the wave's ruler set,
  // alternating); the next group's halves are issued as each slot is freed.
  const int ng = (int)(ge - gs);
  const uint32_t rul_lds = my_lds + 2 * HALF_SLOT;
  UnitIO uio{};
  if (!TOK && !PAGED && append) uio = unit_io(a, h, part, pos);
  [[maybe_unused]] uint32_t qkv_tag = 0;
  if constexpr (QKV) {
    // the projection first (q, and the new token's k / v, come from it); the first groups' first
    // halves and the append unit's ring rows are issued by the waves that do not compute, and have
    // landed when the workgroup meets below; each wave issues its second half after that (the
    // workgroup's loads leave in issue order, so a shallower queue lets the q polls through sooner)
    __shared__ __attribute__((aligned(16))) uint16_t kv_lds[2 * D];
    __shared__ int issued;
    if (tid == 0) issued = 0;
    __syncthreads();
    qkv_tag = (uint32_t)__hip_atomic_load(a.qkv_epoch + h, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    if (wave >= QKV_WAVES) {
      // after every computing wave's first weight loads (bounded: 2^16 short sleeps)
      for (int n = 0; n < (1 << 16); ++n) {
        if (__hip_atomic_load(&issued, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= QKV_WAVES) break;
        __builtin_amdgcn_s_sleep(1);
      }
      for (int w = wave - QKV_WAVES; w < WAVES; w += WAVES - QKV_WAVES) {
        if (w >= ng) break;
        const uint32_t wl = __builtin_amdgcn_readfirstlane(lds_addr(lds_raw + w * wave_lds));
        issue_half(a, h, gs + w, 0, wl, wl + 2 * HALF_SLOT);
      }
      if (wave == QKV_WAVES && append) issue_unit_ring(uio, part, src_lds);
    }
    const bool ok = qkv_prologue(a, h, part, (int)(gridDim.x / a.hkv), pos, qkv_tag, append ? part : -1, q_lds,
                                 kv_lds, unit_src, &issued);
    (void)ok;  // (a wait that gave up leaves NaN vectors: the outputs are NaN)
    if (wave >= QKV_WAVES) wait_groups_all();
  } else {
  // Q and the append unit's rows are loaded ahead of the groups, so that waiting for them
  // leaves the groups in flight
  if (wave == 0 && prefix)
    issue_q(a.q + ((int64_t)b * a.hq + h * a.gq) * D, a.gq, __builtin_amdgcn_readfirstlane(lds_addr(q_lds)));
  if (!TOK && wave == 0 && append) issue_unit_rows(uio, part, src_lds);

  if (wave < ng) {
    if constexpr (TOK) {
      issue_tok<PAGED>(a, b, h, gs + wave, 0, my_lds);
      issue_tok<PAGED>(a, b, h, gs + wave, 1, my_lds + HALF_SLOT_TOK);
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * DMA_HALF_TOK) : "memory");
    } else if constexpr (PAGED) {
      issue_half_paged(a, b, h, gs + wave, 0, my_lds, rul_lds);
      issue_half_paged(a, b, h, gs + wave, 1, my_lds + HALF_SLOT, rul_lds);
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(DMA_FIRST_HALF_PAGED + DMA_SECOND_HALF) : "memory");
    } else {
      issue_half(a, h, gs + wave, 0, my_lds, rul_lds);
      issue_half(a, h, gs + wave, 1, my_lds + HALF_SLOT, rul_lds);
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(DMA_FIRST_HALF + DMA_SECOND_HALF) : "memory");
    }
  } else {
    wait_groups_all();
  }
  }  // QKV
  __syncthreads();
  if constexpr (QKV) {
    if (wave < ng) issue_half(a, h, gs + wave, 1, my_lds + HALF_SLOT, rul_lds);
  }

  if (append) {
    if constexpr (PAGED) append_tok_rows_paged(a, b, h, pos);
    else if constexpr (TOK) append_tok_rows(a, h, pos);
    else append_unit(uio, part, pos, unit_src, xch);
    if (!PAGED && blockIdx.x == 0 && tid == 0) write_scalars(a, pos);
  }

  half8_t qb[4];  // (kept for the merger's tail: the ring attention uses the same operand)
  TailLoads tl;
  const bool merger = !PAGED && a.inline_tail && part == 0;  // the contiguous fused step's merging workgroup
  if (prefix) {
    WaveState st;
    state_init(st);
    load_q_lds(q_lds, a.gq, qb);

    int gi = wave;
    for (int rs = 0; gi < ng; rs ^= 1) {
      const int64_t grp = gs + gi;
      const uint8_t* rul = my_stages + 2 * HALF_SLOT + rs * RULER_BYTES;
      const uint8_t* slot1 = my_stages + slot_bytes;
      LaneRulers ru;
      // first half (slot 0); the second half, issued after it, may stay in flight
      if constexpr (TOK) {
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(DMA_HALF_TOK) : "memory");
        attend_block_tok(a, st, qb, my_stages, my_stages + HALF_CODE,
                         reinterpret_cast<const uint16_t*>(my_stages + 2 * HALF_CODE),
                         reinterpret_cast<const uint16_t*>(my_stages + 2 * HALF_CODE + TOK_SCALE_BYTES),
                         (int)min<int64_t>(32, U - grp * GT));
      } else {
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(DMA_SECOND_HALF) : "memory");
        load_rulers(rul, ru);  // the group's rulers, for both halves
        attend_block<1>(a, st, qb, my_stages, my_stages + HALF_CODE, ru, (int)min<int64_t>(32, U - grp * GT));
      }
      const int nx = gi + WAVES;
      // second half (slot 1)
      const int nv2 = (int)min<int64_t>(32, U - grp * GT - 32);
      if constexpr (TOK) {
        if (nx < ng) issue_tok<PAGED>(a, b, h, gs + nx, 0, my_lds);
        if (nx < ng) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(DMA_HALF_TOK) : "memory");
        else wait_groups_all();
        if (nv2 > 0)
          attend_block_tok(a, st, qb, slot1, slot1 + HALF_CODE, reinterpret_cast<const uint16_t*>(slot1 + 2 * HALF_CODE),
                           reinterpret_cast<const uint16_t*>(slot1 + 2 * HALF_CODE + TOK_SCALE_BYTES), nv2);
        if (nx < ng) issue_tok<PAGED>(a, b, h, gs + nx, 1, my_lds + HALF_SLOT_TOK);
      } else if constexpr (PAGED) {
        if (nx < ng) issue_half_paged(a, b, h, gs + nx, 0, my_lds, rul_lds + (rs ^ 1) * RULER_BYTES);
        if (nx < ng) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(DMA_FIRST_HALF_PAGED) : "memory");
        else wait_groups_all();
        if (nv2 > 0) attend_block<1>(a, st, qb, slot1, slot1 + HALF_CODE, ru, nv2);
        if (nx < ng) issue_half_paged(a, b, h, gs + nx, 1, my_lds + HALF_SLOT, 0u);
      } else {
        if (nx < ng) issue_half(a, h, gs + nx, 0, my_lds, rul_lds + (rs ^ 1) * RULER_BYTES);
        if (nx < ng) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(DMA_FIRST_HALF) : "memory");
        else wait_groups_all();
        if (nv2 > 0) attend_block<1>(a, st, qb, slot1, slot1 + HALF_CODE, ru, nv2);
        if (nx < ng) issue_half(a, h, gs + nx, 1, my_lds + HALF_SLOT, 0u);
      }
      gi = nx;
    }

    // the merger's ring rows, loaded while the partial below is merged and published
    if (merger) tail_load_rows<false>(a, h, b, pos, pos_ok, tl);
    // the paged int8t64 step with its ring work split off: every workgroup of the (sequence, KV
    // head) loads the ring rows and the new token here, for the case that its ticket makes it the
    // ring workgroup (paged_ring_tail)
    if constexpr (PAGED && !TOK) {
      if (a.tail_append && pos_ok && nparts > 1 && nparts < WTS) tail_load_rows<true>(a, h, b, pos, pos_ok, tl, true);
    }
    // ---- merge the waves through LDS and publish the partial word by word (pub_st): each wave
    // puts its partial into its own stage (free once its own loop has ended), then each thread
    // merges two columns, computing its head's wave weights 2^(m_w - m) itself (one barrier)
    const int gq = a.gq, pw = part_stride(gq);
    store_wave_partial(st, gq, reinterpret_cast<float*>(my_stages));
    __syncthreads();
    // (paged: unit pslot is part `part` of sequence b, whose units begin at seq_parts[2b] = pslot - part,
    // so its slot is that of paged_block without reading seq_parts)
    float* dst = a.ws + ((int64_t)h * (PAGED ? a.total_parts + a.nseq : a.n_parts) + pslot + (PAGED ? b : 0)) * pw;
    auto wpart = [&](int w) { return reinterpret_cast<const float*>(lds_raw + w * wave_lds); };
    // (a paged sequence's partials beyond the WTS its tail merges are not published)
    const bool publish = !PAGED || part < WTS;
    const bool l2 = l2_local(a);
    for (int e = 2 * tid; e < gq * D && publish; e += 2 * THREADS) {
      const int head = e / D;
      float pm = NEG_INF;
#pragma unroll
      for (int w = 0; w < WAVES; ++w) pm = fmaxf(pm, wpart(w)[gq * D + head]);
      const float mu = pm == NEG_INF ? 0.0f : pm;
      float cw[WAVES], pl = 0.0f;
#pragma unroll
      for (int w = 0; w < WAVES; ++w) {
        cw[w] = __builtin_amdgcn_exp2f(wpart(w)[gq * D + head] - mu);
        pl += wpart(w)[gq * D + gq + head] * cw[w];
      }
      float x = 0.0f, y = 0.0f;
#pragma unroll
      for (int w = 0; w < WAVES; ++w) {
        x += wpart(w)[e] * cw[w];
        y += wpart(w)[e + 1] * cw[w];
      }
      pub_st2(dst + e, x, y, l2);
      if (e % D == 0) {
        pub_st(dst + gq * D + head, pm, l2);
        pub_st(dst + gq * D + gq + head, pl, l2);
      }
    }
  }  // prefix

  if constexpr (QKV) {
    if (a.w_o && part >= 1) {  // the output projection's rows, while the mergers finish
      oproj_rows(a, h, part, qkv_tag, lds_raw);
      return;
    }
  }

  // ---- fused tail. The contiguous layouts: part 0 of each head merges, polling the other
  // partials' words (the other workgroups never wait, and the hkv merging workgroups leave the
  // rest of the device to them, so every partial arrives). Paged: each workgroup takes a ticket on
  // its (sequence, head) counter once its partial is issued; the last one merges (every other
  // partial is then issued: it polls for the words still in flight) and sets the counter back to
  // zero (every other increment precedes its own in the counter's modification order).
  // (pos, pos_ok, U as the prologue read them: the tail needs no second round trip for them)
  if (!a.inline_tail) return;
  if constexpr (!PAGED) {
    if (!merger) return;
  }
  __syncthreads();  // the stages and the merge's LDS are dead: the tail reuses them
  TailSmem& sm = *reinterpret_cast<TailSmem*>(lds_raw);
  if constexpr (PAGED) {
    const int last = nparts - 1;
    int* ctr = a.tail_ctr_end - 1 - (b * a.hkv + h);
    if (tid == 0) {
      const int t = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (t == last) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      ticket = t;
      sm.ring_staged = 0;
      sm.ring_done = 0;
    }
    __syncthreads();
    // int8t64 with its append and more than one workgroup for (b, h): the first to take a ticket
    // attends over the ring, publishes the ring partial and appends the new token while the others
    // stream; the last merges the prefix partials with that ring partial. Otherwise the last does
    // all of the tail.
    const bool split = !TOK && a.tail_append && pos_ok && nparts > 1 && nparts < WTS;
    if (split && ticket == 0) {
      paged_ring_tail(a, h, b, sm, pos, U, tl, qb);
    } else if (ticket == last) {
      // direct: each merging wave combines its head as soon as the ring partials are in; the ring
      // waves (if any) append the new token after their partial, not before the combine
      const int tb = split ? TB_RING_SLOT : (!TOK && a.tail_append ? TB_APPEND : 0);
      tail_body<true>(a, h, b, sm, TAIL_LAST, pos, pos_ok, U, nullptr, nullptr, tb | TB_DIRECT | TB_KEEP_BLOCK);
      // every word of the sequence's partials (the first min(parts, WTS)) and of its ring slot was
      // consumed: back to zero
      __syncthreads();
      const int P = min(nparts, WTS) + (split ? 1 : 0), pw = part_stride(a.gq);
      uint4* blk = reinterpret_cast<uint4*>(paged_block(a, h, b));
      for (int i = tid; i < P * pw / 4; i += THREADS) blk[i] = uint4{0u, 0u, 0u, 0u};
    }
  } else {
    tail_body<false>(a, h, b, sm, TAIL_MERGER, pos, pos_ok, U, &tl, &qb, 0, -1, QKV ? (int64_t)qkv_tag : -1);
    // every workgroup of head h has read its rows (before publishing the partials just merged):
    // the next launch's tag
    if constexpr (QKV) {
      if (tid == 0) __hip_atomic_store(a.qkv_epoch + h, (int)qkv_tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ---------------------------------------------------------------- kernel C: chained layers
//
// One decode step of n_layers layers in one launch (nkv_decode_layers_t64 / _tok). Layer l is
// the fused step of its own cache (append, split-K prefix, ring, merge), and its inputs (q,
// k_new, v_new) may be outputs of layer l - 1: a model's layers chained through their outputs.
//
// Grid: hkv x (P + 1) workgroups of 8 waves, all resident at once (one per CU; the host checks
// the occupancy before launching). Workgroup (h, 0) is head h's merger: per layer it appends
// the new token (the ring, staged in LDS for the ring attention, requantized into the current
// group), attends over the ring, merges the P prefix partials of its head, writes out / lse and
// counts itself on the layer's completion counter. Workgroup (h, p + 1) streams part p of
// head h's int8 prefix into one published partial, as the prefix kernel does.
//
// Ordering. A merger adds to its layer's counter with an agent-scope release after every wave's
// out / lse stores have completed and the workgroup has met at a barrier, and it also stores the
// output as tagged words. Layer l's inputs are read in one of two ways:
//  - forwarded: q is the whole of layer l - 1's output, and (for a merger) head h's k_new / v_new
//    rows lie in the rows head h's merger wrote. The reader reloads the tagged words it needs
//    until they carry this launch's tag (per-location coherence, no fence). Without dep_all
//    nothing else is waited for: each head's layers then chain on their own. With dep_all, lanes
//    0 .. hq - 1 also poll layer l - 1's issue flags in the same rounds until every query head's
//    output is issued.
//  - otherwise one lane waits for layer l - 1's counter to reach hkv (relaxed agent-scope polls,
//    then an agent-scope acquire fence) and the inputs are plain loads.
// The host refuses inputs that these waits do not order (nkv_decode_layers_t64). The prefix
// partials use the published-word protocol of the fused tail (per-location coherence, no flag);
// each layer has its own partial block. Head h's merger sets its layer-(l + 1) block back to
// zero before its layer-l output, which no part of head h can publish layer l + 1 without;
// layer 0's slots are set back to zero by their writers at the end of the launch. The partials
// and the forwarded outputs are handed between workgroups of one KV head, which share an XCD:
// with the XCD-local hand-over (l2_xcc) they stay in its L2.
//
// Overlap. Nothing in a layer's prefix depends on an earlier layer (the append writes only the
// current group, which the prefix does not read), so as soon as a streaming workgroup has
// published its layer-l partial, its waves issue their first group of layer l + 1 into their
// LDS stages, and HBM keeps streaming while the mergers finish layer l. Wave 7 loads q after the
// wait.
//
// Termination. Every wait gives up after a bounded number of polls; a streaming workgroup that
// gave up publishes an l of NaN, so the merged output is NaN, and sets the error word. At the
// end every workgroup takes an exit ticket (acquire-release); the last one sets the layer
// counters and the ticket back to zero, so every launch starts and ends with them at zero.
constexpr int IN_WAVE = WAVES - 1;                 // a streaming workgroup's input wave

// The sync words of a chained launch at the workspace's end (tail_ctr_end): done[l] at
// end[-1 - l], the exit ticket at end[-1 - n_layers], the error word at end[-2 - n_layers], the
// launch counter (the forwarding tags) at end[-3 - n_layers].
__device__ __forceinline__ int* layer_done(const AttnArgs& a, int l) { return a.tail_ctr_end - 1 - l; }
// issued[l] (dep_all) below them: at end[-4 - n_layers - l]
// issue flags of layer l (dep_all): hq words after the tagged outputs of every layer
// (every flag is stored in FLAG_COPIES copies, [layer][copy][hq], and KV head h's readers poll copy
// h mod FLAG_COPIES: each 128-byte line of flags is polled by one head's workgroups, not by all)
__device__ __forceinline__ uint32_t* layer_flags(const AttnArgs& a, int l) {
  return a.flags_base + (int64_t)l * FLAG_COPIES * a.hq;
}

// Layer l's arguments: the cache and step pointers of its table entry (nkv_layer_t64, or
// nkv_layer_tok for the per-token symmetric format), and its own partial block.
template <bool TOK>
__device__ __forceinline__ AttnArgs layer_args(const AttnArgs& a, const void* layers, int l, uint32_t ftag) {
  AttnArgs la = a;
  la.ftag = ftag;
  // the table through the constant address space: scalar loads (the host wrote it before the
  // launch), which do not queue behind the workgroup's vector loads and DMA
  if constexpr (TOK) {
    const __attribute__((address_space(4))) nkv_layer_tok& e =
        ((const __attribute__((address_space(4))) nkv_layer_tok*)(uintptr_t)layers)[l];
    la.q = e.q;
    la.k_new = e.k_new;
    la.v_new = e.v_new;
    la.kq = reinterpret_cast<uint8_t*>(e.kq);
    la.vq = reinterpret_cast<uint8_t*>(e.vq);
    la.ksc = e.ksc;
    la.vsc = e.vsc;
    la.out = e.out;
    la.lse = e.lse;
  } else {
    const __attribute__((address_space(4))) nkv_layer_t64& e =
        ((const __attribute__((address_space(4))) nkv_layer_t64*)(uintptr_t)layers)[l];
    la.q = e.q;
    la.k_new = e.k_new;
    la.v_new = e.v_new;
    la.kq = e.kq;
    la.kmn = e.kmn;
    la.kst = e.kst;
    la.vq = e.vq;
    la.vmn = e.vmn;
    la.vst = e.vst;
    la.tail_k = e.tail_k;
    la.tail_v = e.tail_v;
    la.out = e.out;
    la.lse = e.lse;
  }
  la.ws = a.ws + (int64_t)l * a.hkv * a.n_parts * part_stride(a.gq);
  la.fwd_out = a.fwd_out + (int64_t)l * a.hq * D / 2;  // (read by layer l + 1 only)
  la.issue_flags = a.dep_all ? layer_flags(a, l) : nullptr;
  return la;
}

// The previous layer's output pointer (the chained step's forwarding source).
template <bool TOK>
__device__ __forceinline__ const uint16_t* layer_out(const void* layers, int l) {
  if constexpr (TOK) return static_cast<const nkv_layer_tok*>(layers)[l].out;
  else return static_cast<const nkv_layer_t64*>(layers)[l].out;
}

// Whether [p, p + n) (fp16 elements) lies inside [base, base + len).
__device__ __forceinline__ bool within(const uint16_t* p, int64_t n, const uint16_t* base, int64_t len) {
  return p >= base && p + n <= base + len;
}

// Forwarded inputs: layer l's q, and the merger's k_new / v_new rows of head h, when they are views
// of layer l - 1's output, are read from that output's tagged words (AttnArgs::fwd_out of layer
// l - 1): lane i takes words i + 64 j, reloading those whose tag is not yet `tag` (relaxed
// agent-scope loads: per-location coherence hands over each word once written, no counter or
// fence), and stores their fp16 pairs to LDS at `dst` (q rows, then k_new, then v_new).
// With `flags` (the all-head dependency: the layer's issue flags, nflags <= 64 of them), lane i
// also polls flag i in the same rounds until it carries the tag: the wait ends when every word
// and every flag does, with no extra round trip. The flags only order (the words validate
// themselves), so their polls are relaxed and no fence follows.
// gq <= FWD_MAX_GQ. false when the wait gave up (after LAYER_WAIT_TICKS, or at once with `lost`).
constexpr int FWD_MAX_GQ = 4;
__device__ __forceinline__ bool fwd_fetch(const uint64_t* q, const uint64_t* k, const uint64_t* v, int gq,
                                          uint32_t tag, uint32_t* dst, bool lost, const uint32_t* flags = nullptr,
                                          int nflags = 0) {
  const int lane = tail_tid() & 63;
  uint64_t w[FWD_MAX_GQ + 2];
#pragma unroll
  for (int j = 0; j < FWD_MAX_GQ + 2; ++j) w[j] = 0;  // (tag 0 is never current)
  const bool kv = k != nullptr;
  bool ok = !lost;
  uint32_t fl = flags != nullptr && lane < nflags ? 0u : tag;  // (lanes beyond nflags poll nothing)
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  while (ok) {
#pragma unroll
    for (int j = 0; j < FWD_MAX_GQ; ++j)
      if (j < gq && (uint32_t)(w[j] >> 32) != tag) w[j] = __hip_atomic_load(q + lane + 64 * j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (kv && (uint32_t)(w[FWD_MAX_GQ] >> 32) != tag)
      w[FWD_MAX_GQ] = __hip_atomic_load(k + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (kv && (uint32_t)(w[FWD_MAX_GQ + 1] >> 32) != tag)
      w[FWD_MAX_GQ + 1] = __hip_atomic_load(v + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (fl != tag) fl = __hip_atomic_load(flags + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    bool miss = fl != tag;
#pragma unroll
    for (int j = 0; j < FWD_MAX_GQ; ++j) miss |= j < gq && (uint32_t)(w[j] >> 32) != tag;
    miss |= kv && ((uint32_t)(w[FWD_MAX_GQ] >> 32) != tag || (uint32_t)(w[FWD_MAX_GQ + 1] >> 32) != tag);
    if (!__builtin_amdgcn_ballot_w64(miss)) break;
    if (__builtin_amdgcn_s_memrealtime() - t0 > LAYER_WAIT_TICKS) ok = false;
    __builtin_amdgcn_s_sleep(1);
  }
#pragma unroll
  for (int j = 0; j < FWD_MAX_GQ; ++j)
    if (j < gq) dst[lane + 64 * j] = (uint32_t)w[j];
  if (kv) {
    dst[gq * 64 + lane] = (uint32_t)w[FWD_MAX_GQ];
    dst[gq * 64 + 64 + lane] = (uint32_t)w[FWD_MAX_GQ + 1];
  }
  return ok;
}

// Wait (lane 0 of the calling wave) until layer l's counter reaches `target`, then an
// agent-scope acquire fence by the whole wave; false when the wait gave up (after
// LAYER_WAIT_TICKS, or at once when an earlier wait of the workgroup gave up: `lost`).
__device__ __forceinline__ bool wait_layer(const AttnArgs& a, int l, int target, bool lost) {
  bool ok = !lost;
  if ((tail_tid() & 63) == 0 && ok) {
    const int* ctr = layer_done(a, l);
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    while (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
      if (__builtin_amdgcn_s_memrealtime() - t0 > LAYER_WAIT_TICKS) {
        ok = false;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  return __builtin_amdgcn_readfirstlane(ok ? 1 : 0) != 0;
}

// One layer of head h's merger (workgroup (h, 0) of the chained kernel): wait for layer l - 1,
// append + ring + merge of layer l into out / lse, count itself on layer l's counter. Returns
// whether its wait gave up. It first sets head h's partial block of layer l + 1 back to zero
// (it was consumed in the previous launch): no part of head h publishes into it before this
// merger's layer-l output, which follows these stores' completion. With the XCD-local hand-over
// the block's lines are then dirty in the L2 when the merger polls them, so every poll is an L2
// hit. Layer 0's block is set back to zero by its writers at the end of the launch.
template <bool TOK>
__device__ __forceinline__ bool merger_layer(const AttnArgs& args, const void* layers, int l, int h, uint8_t* lds_raw,
                                          int64_t pos, bool pos_ok, int64_t U, bool lost) {
  __shared__ int lost_sh;
  const int tid = tail_tid(), wave = tid >> 6;
  AttnArgs la = args;
  const int gq = la.gq;
  TailSmem& sm = *reinterpret_cast<TailSmem*>(lds_raw);
  // q the whole of layer l - 1's output, and head h's k_new and v_new rows inside the rows this
  // merger wrote there (head h's q heads): forwarded from the tagged words, with no counter wait
  // unless every head is waited for (dep_all). Rows written by another head's merger are read
  // after layer l - 1's counter (that head's chain may run ahead or behind this one).
  bool fwd = false;
  const uint16_t* prev = nullptr;
  if (l > 0 && gq <= FWD_MAX_GQ) {
    prev = layer_out<TOK>(layers, l - 1);
    const uint16_t* mine = prev + (int64_t)h * gq * D;
    fwd = la.q == prev && within(la.k_new + (int64_t)h * la.kv_hs, D, mine, (int64_t)gq * D) &&
          within(la.v_new + (int64_t)h * la.kv_hs, D, mine, (int64_t)gq * D);
  }
  if (tid == 0) {
    sm.ring_staged = 0;
    sm.ring_done = 0;
  }
  if (l + 1 < la.n_layers) {
    const int P = la.n_parts, pw = part_stride(gq);
    uint4* nb = reinterpret_cast<uint4*>(la.ws + ((int64_t)la.hkv * P + (int64_t)h * P) * pw);
    const bool l2 = l2_local(la);
    for (int i = tid; i < P * pw / 4; i += THREADS) zero_st16(nb + i, l2);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // (before the barrier below)
  }
  if (wave == IN_WAVE) {
    bool ok = true;
    if (fwd) {
      const uint64_t* src = la.fwd_out - (int64_t)la.hq * D / 2;  // layer l - 1's tagged words
      ok = fwd_fetch(src + (int64_t)h * gq * D / 2, src + ((la.k_new - prev) + (int64_t)h * la.kv_hs) / 2,
                     src + ((la.v_new - prev) + (int64_t)h * la.kv_hs) / 2, gq, la.ftag, sm.fwd, lost,
                     la.dep_all ? layer_flags(la, l - 1) + (h % FLAG_COPIES) * la.hq : nullptr, la.hq);
    } else if (l > 0) {
      ok = wait_layer(la, l - 1, la.hkv, lost);
    }
    if (tid == IN_WAVE * 64) lost_sh = ok ? 0 : 1;
  }
  __syncthreads();
  const bool gave_up = lost_sh != 0;
  if (l == 0 && blockIdx.x == 0 && tid == 0 && pos_ok) write_scalars(la, pos);
  half8_t qb[4];
  if (fwd) {  // the tail reads them from LDS
    const uint16_t* f = reinterpret_cast<const uint16_t*>(sm.fwd);
    load_q_lds(f, gq, qb);
    la.k_new = f + gq * D;
    la.v_new = f + gq * D + D;
    la.kv_hs = 0;
  }
  tail_body<false>(la, h, 0, sm, TAIL_MERGER, pos, pos_ok, U, nullptr, fwd ? &qb : nullptr,
                   TB_APPEND | TB_KEEP_BLOCK | TB_DIRECT | (lost || gave_up ? TB_POISON : 0));
  // every wave's stores (out, lse, the ring slot) complete before the workgroup meets; then one
  // release at agent scope publishes them all with the count
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) __hip_atomic_fetch_add(layer_done(la, l), 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
  return gave_up;
}

template <int LAYOUT>
__global__ __launch_bounds__(THREADS, 1) void attn_layers_kernel(AttnArgs a, const void* layers, int n_layers) {
  static_assert(LAYOUT == CONTIG_T64 || LAYOUT == CONTIG_TOK, "contiguous caches");
  constexpr bool TOK = LAYOUT == CONTIG_TOK;
  __shared__ __attribute__((aligned(16))) uint8_t lds_raw[TOK ? LDS_BYTES_TOK : LDS_BYTES];
  __shared__ __attribute__((aligned(16))) uint16_t q_lds[16 * D];
  __shared__ int lost_sh;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = blockIdx.x % a.hkv, role = blockIdx.x / a.hkv;
  const int P = a.n_parts, gq = a.gq, pw = part_stride(gq);
  int64_t pos;
  bool pos_ok;
  const int64_t U = prefix_limit(a, pos, pos_ok);
  const int64_t W = (U + GT - 1) / GT;
  const bool merger = role == 0;
  const int part = role - 1;
  const int64_t gs = merger ? 0 : (int64_t)part * W / P;
  const int64_t ge = merger ? 0 : (int64_t)(part + 1) * W / P;
  const int ng = (int)(ge - gs);
  constexpr int wave_lds = TOK ? WAVE_LDS_TOK : WAVE_LDS;
  constexpr int slot_bytes = TOK ? HALF_SLOT_TOK : HALF_SLOT;
  uint8_t* my_stages = lds_raw + wave * wave_lds;
  const uint32_t my_lds = __builtin_amdgcn_readfirstlane(lds_addr(my_stages));
  const uint32_t rul_lds = my_lds + 2 * HALF_SLOT;
  bool lost = false;  // a counter wait of this workgroup gave up
  // this launch's forwarding tag: the launch counter (advanced at the exit) + 1; tag 0, that of
  // a zero-filled workspace, is never current
  int* const epoch = a.tail_ctr_end - 3 - n_layers;
  const uint32_t ftag = (uint32_t)__hip_atomic_load(epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;

  // the wave's first group (both halves; int8t64: its rulers into ruler set 0)
  // The part's groups: the first `whole` go whole to the waves, strided (wave w takes w, w + 8,
  // ..); when at most 4 groups are left over a multiple of 8, their halves go one per wave to
  // waves 0 .. extra - 1 (no wave then takes more than one half beyond the others), else they go
  // whole as well. An extra half brings its group's rulers.
  const int rest = ng % WAVES;
  const int whole = 2 * rest <= WAVES ? ng - rest : ng, extra = 2 * (ng - whole);
  const bool has_x = wave < extra;
  const int64_t xg = gs + whole + (wave >> 1);
  const int xh = wave & 1;
  // the half of the extra group, with the rulers, into slot 0 and ruler set `set`
  auto issue_extra = [&](const AttnArgs& la, int set) {
    if constexpr (TOK) issue_tok<false>(la, 0, h, xg, xh, my_lds);
    else issue_half(la, h, xg, xh, my_lds, rul_lds + set * RULER_BYTES, true);
  };
  // the wave's first item: its first whole group (both halves), or its extra half
  auto issue_first = [&](const AttnArgs& la) {
    if (wave < whole) {
      if constexpr (TOK) {
        issue_tok<false>(la, 0, h, gs + wave, 0, my_lds);
        issue_tok<false>(la, 0, h, gs + wave, 1, my_lds + HALF_SLOT_TOK);
      } else {
        issue_half(la, h, gs + wave, 0, my_lds, rul_lds);
        issue_half(la, h, gs + wave, 1, my_lds + HALF_SLOT, rul_lds);
      }
    } else if (has_x) {
      issue_extra(la, 0);
    }
  };
  if (merger) {
    for (int l = 0; l < n_layers; ++l) lost |= merger_layer<TOK>(layer_args<TOK>(a, layers, l, ftag), layers, l, h, lds_raw, pos, pos_ok, U, lost);
    // one layer: its consumed partial block back to zero (with more, layer 0's slots are zeroed by
    // their writers, below, and every later block by this merger in the next launch)
    if (n_layers == 1) {
      uint4* blk = reinterpret_cast<uint4*>(a.ws + (int64_t)h * P * pw);
      for (int i = tid; i < P * pw / 4; i += THREADS) blk[i] = uint4{0u, 0u, 0u, 0u};
    }
  } else {
  if (wave != IN_WAVE) issue_first(layer_args<TOK>(a, layers, 0, ftag));
  for (int l = 0; l < n_layers; ++l) {
    const AttnArgs la = layer_args<TOK>(a, layers, l, ftag);

    // ---- streaming part: q of layer l once layer l - 1 is complete (layer 0: the input wave's
    // first group goes behind q; later layers: it was prefetched with the others' and has long
    // landed when the counter wait ends, so waiting for q waits for nothing else)
    if (wave == IN_WAVE) {
      bool ok = true;
      if (l > 0 && gq <= FWD_MAX_GQ && la.q == layer_out<TOK>(layers, l - 1)) {
        // q is layer l - 1's output: its tagged words (head h's rows, written by head h's merger),
        // and with dep_all layer l - 1's counter as well
        ok = fwd_fetch(la.fwd_out - (int64_t)la.hq * D / 2 + (int64_t)h * gq * D / 2, nullptr, nullptr, gq, la.ftag,
                       reinterpret_cast<uint32_t*>(q_lds), lost,
                       a.dep_all ? layer_flags(a, l - 1) + (h % FLAG_COPIES) * a.hq : nullptr, a.hq);
      } else {
        ok = l == 0 || wait_layer(a, l - 1, a.hkv, lost);
        issue_q(la.q + (int64_t)h * gq * D, gq, __builtin_amdgcn_readfirstlane(lds_addr(q_lds)));
        wait_groups_all();
      }
      if (tid == IN_WAVE * 64) lost_sh = ok ? 0 : 1;
      if (l == 0) issue_first(la);
    }
    __syncthreads();
    lost |= lost_sh != 0;
    WaveState st;
    state_init(st);
    half8_t qb[4];
    load_q_lds(q_lds, gq, qb);
    if constexpr (TOK) {
      int rs = 0;  // ruler set of the group in the slots
      for (int gi = wave; gi < whole; gi += WAVES, rs ^= 1) {
        const int64_t grp = gs + gi;
        const uint8_t* slot1 = my_stages + slot_bytes;
        const bool nx_whole = gi + WAVES < whole, nx_extra = !nx_whole && has_x;
        const int nv1 = (int)min<int64_t>(32, U - grp * GT), nv2 = (int)min<int64_t>(32, U - grp * GT - 32);
        // first half (slot 0; the second half may still be in flight), then the next item's first
        // loads into slot 0 (the next group's half 0 and rulers, or the extra half and its rulers)
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(DMA_HALF_TOK) : "memory");
        attend_block_tok(la, st, qb, my_stages, my_stages + HALF_CODE,
                         reinterpret_cast<const uint16_t*>(my_stages + 2 * HALF_CODE),
                         reinterpret_cast<const uint16_t*>(my_stages + 2 * HALF_CODE + TOK_SCALE_BYTES), nv1);
        if (nx_whole) issue_tok<false>(la, 0, h, grp + WAVES, 0, my_lds);
        else if (nx_extra) issue_extra(la, rs ^ 1);
        if (nx_whole || nx_extra) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(DMA_HALF_TOK) : "memory");
        else wait_groups_all();
        if (nv2 > 0)
          attend_block_tok(la, st, qb, slot1, slot1 + HALF_CODE, reinterpret_cast<const uint16_t*>(slot1 + 2 * HALF_CODE),
                           reinterpret_cast<const uint16_t*>(slot1 + 2 * HALF_CODE + TOK_SCALE_BYTES), nv2);
        if (nx_whole) issue_tok<false>(la, 0, h, grp + WAVES, 1, my_lds + HALF_SLOT_TOK);
      }
      if (has_x) {
        // the extra half, in slot 0 with its rulers in set rs (issued by the last whole group, or
        // by issue_first when the wave has none)
        const int nvx = (int)max<int64_t>(0, min<int64_t>(32, U - xg * GT - 32 * xh));
        wait_groups_all();
        if (nvx > 0) {
          attend_block_tok(la, st, qb, my_stages, my_stages + HALF_CODE,
                           reinterpret_cast<const uint16_t*>(my_stages + 2 * HALF_CODE),
                           reinterpret_cast<const uint16_t*>(my_stages + 2 * HALF_CODE + TOK_SCALE_BYTES), nvx);
        }
      }
    } else {
      // ---- int8t64 (here every half is full: U is a multiple of 64), software-pipelined over
      // the wave's halves k = 0 .. nh - 1 (its whole groups' halves, then its extra half). Half
      // k has its K codes in K slot k % 2, its V codes in V slot k % 2 and its group's rulers in
      // set (item of k) % 2. Region k holds PV(k) and QK(k + 1) in one basic block, which the
      // compiler interleaves; after it V slot k % 2 takes V(k + 2) and K slot (k + 1) % 2 takes
      // K(k + 3) (with its group's rulers when it starts an item), both read two regions later.
      const int nwh = wave < whole ? 2 * ((whole - 1 - wave) / WAVES + 1) : 0;
      const int nh = nwh + (has_x ? 1 : 0);
      auto hgrp = [&](int k) { return k < nwh ? gs + wave + (int64_t)WAVES * (k >> 1) : xg; };
      auto hhf = [&](int k) { return k < nwh ? (k & 1) : xh; };
      auto hset = [&](int k) { return (k < nwh ? (k >> 1) : (nwh >> 1)) & 1; };
      auto hstart = [&](int k) { return k >= nwh || (k & 1) == 0; };
      auto kslot = [&](int k) { return my_stages + (k & 1) * HALF_SLOT; };
      auto rset = [&](int k) { return my_stages + 2 * HALF_SLOT + hset(k) * RULER_BYTES; };
      // the loads issued (counted for the waits: 0, 4 or 8, and 0 or 4)
      auto issue_k = [&](int k) -> int {
        if (k >= nh) return 0;
        issue_rows(la.kq, la, h, hgrp(k), hhf(k), my_lds + (k & 1) * HALF_SLOT);
        if (!hstart(k)) return 4;
        issue_rulers(la, h, hgrp(k), rul_lds + hset(k) * RULER_BYTES);
        return 8;
      };
      auto issue_v = [&](int k) -> int {
        if (k >= nh) return 0;
        issue_rows(la.vq, la, h, hgrp(k), hhf(k), my_lds + (k & 1) * HALF_SLOT + HALF_CODE);
        return 4;
      };
      if (nh > 0) {
        // the prefetched first item (K0 V0 R0, then K1 V1 when it has two halves): QK(0) needs
        // K0 and R0
        vm_wait_n(nh >= 2 && !hstart(1) ? DMA_SECOND_HALF : 0);
        float s[2][4];
        half8_t phi[1], plo[1];
        qk_half(kslot(0), rset(0), qb, s);
        int pend = issue_k(2);
        softmax_step<1>(st, s, la.sl2, phi, plo, gq);
        LaneRulers ru;
        for (int k = 0; k + 1 < nh; ++k) {
          vm_wait_n(pend);  // V(k), K(k + 1) and its rulers have landed
          if (hstart(k)) load_rulers(rset(k), ru);
          pv_qk_half(st, kslot(k) + HALF_CODE, ru, phi[0], plo[0], kslot(k + 1), rset(k + 1), qb, s);
          pend = issue_v(k + 2);
          pend += issue_k(k + 3);
          softmax_step<1>(st, s, la.sl2, phi, plo, gq);
        }
        vm_wait_n(pend);
        if (hstart(nh - 1)) load_rulers(rset(nh - 1), ru);
        pv_half(st, kslot(nh - 1) + HALF_CODE, ru, phi[0], plo[0]);
      }
    }

    // ---- merge the waves through LDS and publish the partial word by word: each wave puts its
    // partial into its own stage (free once its own loop has ended), then each thread merges two
    // columns, computing its head's wave weights 2^(m_w - m) itself (one barrier on the way)
    const int ptid = tail_tid();  // (per layer: nothing derived from it stays live across the loop)
    store_wave_partial(st, gq, reinterpret_cast<float*>(my_stages));
    __syncthreads();
    {
      float* dst = la.ws + ((int64_t)h * P + part) * pw;
      auto wpart = [&](int w) { return reinterpret_cast<const float*>(lds_raw + w * wave_lds); };
      const bool l2 = l2_local(la);
      for (int e = 2 * ptid; e < gq * D; e += 2 * THREADS) {
        const int head = e / D;
        float pm = NEG_INF;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) pm = fmaxf(pm, wpart(w)[gq * D + head]);
        const float mu = pm == NEG_INF ? 0.0f : pm;
        float cw[WAVES], pl = 0.0f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
          cw[w] = __builtin_amdgcn_exp2f(wpart(w)[gq * D + head] - mu);
          pl += wpart(w)[gq * D + gq + head] * cw[w];
        }
        float x = 0.0f, y = 0.0f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
          x += wpart(w)[e] * cw[w];
          y += wpart(w)[e + 1] * cw[w];
        }
        pub_st2(dst + e, x, y, l2);
        if (e % D == 0) {
          pub_st(dst + gq * D + head, pm, l2);
          pub_st(dst + gq * D + gq + head, lost ? __builtin_nanf("") : pl, l2);  // a lost wait poisons the merge
        }
      }
    }
    // ---- the stages are free: the next layer's first groups stream while this layer merges
    __syncthreads();
    if (l + 1 < n_layers) issue_first(layer_args<TOK>(a, layers, l + 1, ftag));
  }
  // head h's merger has consumed this part's partial of layer 0: this workgroup read layer
  // n_layers - 1's q after that merger finished layer n_layers - 2 >= 0 (from its tagged words,
  // or after the counter that it joins only once it has merged). That slot back to zero, polled
  // first by the next launch (the later layers' blocks are zeroed by the merger before use)
  if (n_layers > 1) {
    uint4* slot = reinterpret_cast<uint4*>(a.ws + ((int64_t)h * P + part) * pw);
    for (int i = tid; i < pw / 4; i += THREADS) slot[i] = uint4{0u, 0u, 0u, 0u};
  }
  }

  // ---- exit ticket: the last workgroup sets the counters back to zero
  __syncthreads();
  if (tid == 0) {
    int* exit_ctr = a.tail_ctr_end - 1 - n_layers;
    if (lost) __hip_atomic_store(exit_ctr - 1, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int t = __hip_atomic_fetch_add(exit_ctr, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (t == (int)gridDim.x - 1) {
      for (int l = 0; l < n_layers; ++l) __hip_atomic_store(layer_done(a, l), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(exit_ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(epoch, (int)ftag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ---------------------------------------------------------------- read-ceiling probe
//
// The streaming of the decode kernels without their math: `gridDim.x` workgroups of 8 waves, one
// per CU (128 KiB of LDS each). The buffer is read in chunks of 8 KiB (8 nontemporal LDS-DMA loads
// of 16 bytes per lane, as the prefix kernel issues them); chunk c goes to wave c mod (8 x blocks),
// which keeps two chunks in flight in two 8 KiB LDS slots and folds one dword per lane of each
// landed chunk into an XOR checksum (so every load is consumed). The achievable HBM read rate of
// the decode path's load pattern, measured in the same process as the path itself.
constexpr int RB_CHUNK = 8192;
__global__ __launch_bounds__(THREADS, 1) void read_lds_kernel(const uint8_t* src, int64_t nchunks, uint32_t* sink) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[WAVES * 2 * RB_CHUNK];
  __shared__ uint32_t part[WAVES];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int64_t nw = (int64_t)gridDim.x * WAVES;
  const uint32_t base = __builtin_amdgcn_readfirstlane(lds_addr(lds + wave * 2 * RB_CHUNK));
  auto issue = [&](int64_t ch, int slot) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the slot's last read is done
    const void* sb = uniform_ptr(src + ch * RB_CHUNK);
#pragma unroll
    for (int j = 0; j < RB_CHUNK / 1024; ++j) dma16_stream(sb, (uint32_t)(1024 * j + 16 * lane), base + slot * RB_CHUNK + 1024 * j);
  };
  int64_t c = (int64_t)blockIdx.x * WAVES + wave;
  if (c < nchunks) issue(c, 0);
  if (c + nw < nchunks) issue(c + nw, 1);
  uint32_t x = 0;
  for (int slot = 0; c < nchunks; c += nw, slot ^= 1) {
    if (c + nw < nchunks) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    x ^= *reinterpret_cast<const uint32_t*>(lds + (wave * 2 + slot) * RB_CHUNK + 16 * lane);
    if (c + 2 * nw < nchunks) issue(c + 2 * nw, slot);
  }
  for (int m = 32; m >= 1; m >>= 1) x ^= (uint32_t)__shfl_xor((int)x, m, 64);
  if (lane == 0) part[wave] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t y = 0;
    for (int w = 0; w < WAVES; ++w) y ^= part[w];
    sink[blockIdx.x] = y;
  }
}

// ---------------------------------------------------------------- kernel B: ring + merge

// One workgroup per KV head (per sequence and KV head when paged), after the prefix kernel.
template <bool PAGED>
__global__ __launch_bounds__(TB_THREADS, 1) void attn_tail_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) TailSmem sm;
  const int h = PAGED ? blockIdx.x % a.hkv : blockIdx.x;
  const int b = PAGED ? blockIdx.x / a.hkv : 0;
  int64_t pos;
  bool pos_ok;
  int64_t U;
  if constexpr (PAGED) {
    pos = a.pos_dev[b];
    pos_ok = pos >= 0 && page_of(a, b, pos / GT) >= 0;  // the current group has a page
    U = pos_ok ? pos / GT * GT : 0;
  } else {
    U = prefix_limit(a, pos, pos_ok);
  }
  tail_body<PAGED>(a, h, b, sm, TAIL_KERNEL, pos, pos_ok, U);
}

// Standalone append: one workgroup per append unit (APPEND_UNITS per KV head).
__global__ __launch_bounds__(THREADS) void append_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t unit_src[UNIT_SRC_BYTES / 2];
  __shared__ __attribute__((aligned(16))) float xch[UNIT_CH * 2 * WAVES];
  const int h = blockIdx.x / APPEND_UNITS, unit = blockIdx.x % APPEND_UNITS;
  const int64_t pos = *a.pos_dev;
  if (pos < 0 || pos >= a.capacity) return;  // a position outside the cache appends nothing
  const UnitIO io = unit_io(a, h, unit, pos);
  if (threadIdx.x < 64) issue_unit_rows(io, unit, __builtin_amdgcn_readfirstlane(lds_addr(unit_src)));
  wait_groups_all();
  __syncthreads();
  append_unit(io, unit, pos, unit_src, xch);
  if (blockIdx.x == 0 && threadIdx.x == 0) write_scalars(a, pos);
}

// Paged batch append: one workgroup per (sequence, KV head, wide unit of 64 channels).
__global__ __launch_bounds__(THREADS) void append_paged_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t src[WIDE_SRC_BYTES];
  __shared__ __attribute__((aligned(16))) float xch[WIDE_CH * 16];
  __shared__ float4 rul[WIDE_CH];
  const int w = blockIdx.x % WIDE_UNITS, h = (blockIdx.x / WIDE_UNITS) % a.hkv;
  const int b = blockIdx.x / (WIDE_UNITS * a.hkv);
  const int64_t pos = a.pos_dev[b];
  if (pos < 0 || page_of(a, b, pos / GT) < 0) return;  // a position without a page appends nothing
  const int which = w / (D / WIDE_CH), ch0 = (w % (D / WIDE_CH)) * WIDE_CH;
  const UnitIO io = unit_io_paged(a, b, h, which * (D / UNIT_CH), pos);
  issue_wide_rows(io, ch0, lds_addr(src));
  wait_groups_all();
  __syncthreads();
  append_wide(io, ch0, pos, src, xch, rul);
}

// Standalone per-token symmetric append: one workgroup of 2 waves (K, V) per KV head.
__global__ __launch_bounds__(128) void append_tok_kernel(AttnArgs a) {
  const int64_t pos = *a.pos_dev;
  if (pos < 0 || pos >= a.capacity) return;  // a position outside the cache appends nothing
  append_tok_rows(a, blockIdx.x, pos);
  if (blockIdx.x == 0 && threadIdx.x == 0) write_scalars(a, pos);
}

// Zeroes `n` ints (n a multiple of 4, p 16-byte aligned) with vector stores.
__global__ __launch_bounds__(256) void clear_ints_kernel(int* p, int n) {
  for (int i = 4 * (blockIdx.x * 256 + threadIdx.x); i < n; i += 4 * 256 * gridDim.x)
    *reinterpret_cast<int4*>(p + i) = int4{0, 0, 0, 0};
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

// ---------------------------------------------------------------- chunked prefill (MFMA)
//
// Causal attention of a chunk of M query tokens over the int8t64 cache [0, U) (U a multiple
// of 64) and over Mk >= M fp16 K/V tokens that follow it: query token i sits at fp16 index
// qoff + i (qoff = Mk - M) and attends fp16 tokens j <= qoff + i. With qoff = 0 the fp16
// tokens are the chunk's own; with qoff > 0 they are an fp16 history plus the chunk (the
// staged prefill, whose history is not quantized yet). Query rows of KV head
// h: row r = (token r / gq, q head h gq + r % gq), M gq rows per head. Workgroup (h, tile,
// split) takes rows 256 tile .. + 255 (8 waves x 2 MFMA row blocks of 16) and the split's
// share of the 64-token groups: cache groups [split G / S, (split + 1) G / S) and chunk
// groups j = split (mod S) up to its last query token. Per group, the 8 waves dequantize
// the int8 codes once into fp16 LDS tiles (K row-major, V transposed, both padded against
// bank conflicts), then every wave runs QK^T and PV on v_mfma_f32_16x16x32_f16 for its 32
// rows. The cache groups take one workgroup barrier each: the tiles are double-buffered and
// the next group is dequantized beside the current group's last product. P is a single fp16
// operand (scaled by 2^15), as a fused fp16 attention kernel computes it. Each workgroup
// writes one partial per row; a combine kernel merges the splits.
constexpr int PF_WAVES = 8;
constexpr int PF_THREADS = 64 * PF_WAVES;
constexpr int PF_RB = 2;                             // MFMA row blocks per wave
constexpr int PF_WG_PER_CU = 1;                      // workgroups resident per CU (~206 VGPRs per lane)
constexpr int PF_ROWS = PF_WAVES * PF_RB * 16;       // 256 query rows per workgroup
constexpr int PF_KROW = D + 8;                       // fp16 K tile row stride (halves)
constexpr int PF_VROW = GT + 16;                     // fp16 V^T tile row stride (halves, 16-byte rows)
constexpr float PF_TAU = 8.0f;                       // lazy softmax rescaling threshold (log2)
constexpr int PF_PART = D + 4;                       // floats per row partial: acc[128], m, l, pad
#ifndef PF_SCHED
#define PF_SCHED 1
#endif
#ifndef PF_SCHED_V
#define PF_SCHED_V 3  // VALU instructions scheduled after each interleaved MFMA
#endif
// instruction classes of __builtin_amdgcn_sched_group_barrier
constexpr int PF_SG_VALU = 0x2, PF_SG_MFMA = 0x8, PF_SG_DSR = 0x100;

// token slot of the V^T tile: P's k-slot order (slot 8g + r of a 32-token block <-> token
// 16 (r >> 2) + 4g + (r & 3))
__device__ __forceinline__ int pf_vslot(int t) {
  const int u = t & 31;
  return (t & 32) + 8 * ((u >> 2) & 3) + 4 * (u >> 4) + (u & 3);
}

struct PrefillArgs {
  const uint16_t* q;   // [hq][M][D]
  const uint16_t* kc;  // fp16 K: head h's token j at kc + h * kc_hs + j * D, j < Mk
  const uint16_t* vc;  // fp16 V, the same layout
  const uint8_t* kq;
  const uint16_t* kmn;
  const uint16_t* kst;
  const uint8_t* vq;
  const uint16_t* vmn;
  const uint16_t* vst;
  int64_t capacity, ngroups_cap, U;
  int M, hq, hkv, gq, splits, tiles;
  int Mk, qoff;    // fp16 tokens, and the fp16 index of query token 0
  int64_t kc_hs;   // head stride of kc / vc (elements)
  float sl2;
  float* ws;       // [splits][hkv * M * gq][PF_PART]
  uint16_t* out;   // [hq][M][D]
};

// Online softmax of one 16-row block over 64 tokens, from the raw scores S[b][i] (token
// 16b + 4g + i, row c; -inf where masked): m is a reference maximum in the log2 domain, within
// PF_TAU below the row's maximum of S * sl2, and P comes out as exp2(S sl2 - m + 15 - PF_TAU)
// <= 2^15 in two fp16 A operands (tokens of blocks 0,1 and 2,3). The row sums of P are taken on
// the matrix core by the caller (P times a ones operand, in the accumulator layout), which leaves
// the VALU the maximum, the exponentials and the conversions; the caller rescales the
// accumulators and those sums by alpha, only when m moves.
__device__ __forceinline__ void pf_softmax(WaveState& st, const float (&S)[4][4], float sl2, half8_t (&ph)[2],
                                           float& alpha_out, bool& moved_out) {
  float smax = NEG_INF;
#pragma unroll
  for (int b = 0; b < 4; ++b)
#pragma unroll
    for (int i = 0; i < 4; ++i) smax = fmaxf(smax, S[b][i]);
  smax = max4rows(smax);
  const float m_cand = fmaxf(st.m, smax * sl2);
  const float m_new = m_cand > st.m + PF_TAU ? m_cand : st.m;
  const float m_use = m_new == NEG_INF ? 0.0f : m_new;
  const float alpha = __builtin_amdgcn_exp2f(st.m - m_use);
  const float off = 15.0f - PF_TAU - m_use;
  _Float16 p16[2][8];
#pragma unroll
  for (int b = 0; b < 4; ++b)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      p16[b >> 1][4 * (b & 1) + i] = (_Float16)__builtin_amdgcn_exp2f(__builtin_fmaf(S[b][i], sl2, off));
#pragma unroll
  for (int B = 0; B < 2; ++B)
    ph[B] = half8_t{p16[B][0], p16[B][1], p16[B][2], p16[B][3], p16[B][4], p16[B][5], p16[B][6], p16[B][7]};
  moved_out = st.m != m_new;
  alpha_out = alpha;
  st.m = m_new;
}

__global__ __launch_bounds__(PF_THREADS, PF_WG_PER_CU) void prefill_chunk_kernel(PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t stage[2][2 * CODE_BYTES + RULER_BYTES];
  __shared__ __attribute__((aligned(16))) uint16_t ktile_buf[2][GT * PF_KROW];
  __shared__ __attribute__((aligned(16))) uint16_t vtile_buf[2][D * PF_VROW];
  const int tid = threadIdx.x, lane = tid & 63, c = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = blockIdx.x % a.hkv, tile = (blockIdx.x / a.hkv) % a.tiles, split = blockIdx.x / (a.hkv * a.tiles);
  const int rows_h = a.M * a.gq;
  const int row0 = tile * PF_ROWS + wave * PF_RB * 16;  // first row of this wave

  // ---- Q operands (B of S^T = K Q^T): lane (c, g) holds row 16 rb + c, dims of k-step k
  half8_t qb[PF_RB][4];
#pragma unroll
  for (int rb = 0; rb < PF_RB; ++rb) {
    const int r = row0 + 16 * rb + c;
    const bool ok = r < rows_h;
    const int tk = ok ? r / a.gq : 0, hd = h * a.gq + (ok ? r % a.gq : 0);
    const uint16_t* qr = a.q + ((int64_t)hd * a.M + tk) * D;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint4 w = {0, 0, 0, 0};
      if (ok) w = *reinterpret_cast<const uint4*>(qr + 16 * g + 64 * (k >> 1) + 8 * (k & 1));
      qb[rb][k] = as_h8(w);
    }
  }
  asm volatile("" ::"v"(qb[0][0]), "v"(qb[0][1]), "v"(qb[0][2]), "v"(qb[0][3]), "v"(qb[PF_RB - 1][0]),
               "v"(qb[PF_RB - 1][1]), "v"(qb[PF_RB - 1][2]), "v"(qb[PF_RB - 1][3]));
  WaveState st[PF_RB];
  float4_t lsum[PF_RB];  // rows 4g + i of each row block: the sums of P, on the matrix core
#pragma unroll
  for (int rb = 0; rb < PF_RB; ++rb) {
    state_init(st[rb]);
    lsum[rb] = float4_t{0.f, 0.f, 0.f, 0.f};
  }
  const _Float16 one = (_Float16)1.0f;
  const half8_t ones = half8_t{one, one, one, one, one, one, one, one};

  const int64_t G = a.U / GT;
  const int64_t cs = (int64_t)split * G / a.splits, ce = (int64_t)(split + 1) * G / a.splits;
  const int last_tok = min(rows_h - 1, (tile + 1) * PF_ROWS - 1) / a.gq;  // last query token of the tile
  const int nchunk = min((a.Mk + GT - 1) / GT, (last_tok + a.qoff) / GT + 1);

  // cache group loads: wave w issues K and V code rows 8w .. 8w + 7 and half w & 1 of ruler
  // w >> 1 (kst, kmn, vst, vmn)
  auto issue = [&](int64_t grp, int sb) {
    const uint32_t base = __builtin_amdgcn_readfirstlane(lds_addr(stage[sb]));
    const void* kb = uniform_ptr(a.kq + ((int64_t)h * a.capacity + grp * GT) * D);
    const void* vb = uniform_ptr(a.vq + ((int64_t)h * a.capacity + grp * GT) * D);
    const int row = 8 * wave + (lane >> 3);
    const uint32_t off = (uint32_t)(row * D + (((lane & 7) ^ swz(row)) << 4));
    dma16(kb, off, base + 1024 * wave);
    dma16(vb, off, base + CODE_BYTES + 1024 * wave);
    const int64_t ro = ((int64_t)h * a.ngroups_cap + grp) * D + 64 * (wave & 1);
    const int rw = wave >> 1;
    const uint16_t* rsrc = rw == 0 ? a.kst : rw == 1 ? a.kmn : rw == 2 ? a.vst : a.vmn;
    if (lane < 8) dma16(uniform_ptr(rsrc + ro), (uint32_t)(16 * lane), base + 2 * CODE_BYTES + 256 * rw + 128 * (wave & 1));
  };
  constexpr int DMA_PF = 3;  // loads per wave and group

  // ---- MFMA phase over the tiles in LDS; `mask_base` >= 0: chunk tokens from that index (causal)
  auto attend_tiles = [&](int mask_base, int tb, auto&& tail_work) {
    const uint16_t* ktile = ktile_buf[tb];
    const uint16_t* vtile = vtile_buf[tb];
    float4_t S[PF_RB][4];
#pragma unroll
    for (int rb = 0; rb < PF_RB; ++rb)
#pragma unroll
      for (int b = 0; b < 4; ++b) S[rb][b] = float4_t{0.f, 0.f, 0.f, 0.f};
    half8_t ph[PF_RB][2];
    float alpha[PF_RB];
    bool moved[PF_RB];
    // the K and V operands of the group, each read from LDS once for both row blocks
    half8_t kop[4][4], vop[2][8];
    auto load_k = [&]() {
#pragma unroll
      for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int k = 0; k < 4; ++k)
          kop[b][k] = *reinterpret_cast<const half8_t*>(ktile + (16 * b + c) * PF_KROW + 16 * g + 64 * (k >> 1) + 8 * (k & 1));
    };
    auto load_v = [&]() {
#pragma unroll
      for (int B = 0; B < 2; ++B)
#pragma unroll
        for (int cb = 0; cb < 8; ++cb)
          vop[B][cb] = *reinterpret_cast<const half8_t*>(vtile + (16 * cb + c) * PF_VROW + 32 * B + 8 * g);
    };
    auto qk = [&](int rb) {
#pragma unroll
      for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int k = 0; k < 4; ++k) S[rb][b] = mfma32(kop[b][k], qb[rb][k], S[rb][b]);
    };
    auto softmax = [&](int rb) {
      float sc[4][4];
      const int tq = (row0 + 16 * rb + c) / a.gq;  // query token of row c (score column)
#pragma unroll
      for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int kt = mask_base + 16 * b + 4 * g + i;
          sc[b][i] = (mask_base < 0 || kt <= tq + a.qoff) ? S[rb][b][i] : NEG_INF;
        }
      // rows of the S^T layout are q rows c; the causal test above needs the row of column
      // c, which is lane-independent of g: scores of lane (c, g) all belong to row c
      pf_softmax(st[rb], sc, a.sl2, ph[rb], alpha[rb], moved[rb]);
#if PF_SCHED
      // P is computed here, beside the other row block's products, not sunk past the rescale
      asm volatile("" : "+v"(ph[rb][0]), "+v"(ph[rb][1]));
#endif
    };
    auto pv = [&](int rb) {
#pragma unroll
      for (int B = 0; B < 2; ++B)
#pragma unroll
        for (int cb = 0; cb < 8; ++cb) st[rb].acc[cb] = mfma32(ph[rb][B], vop[B][cb], st[rb].acc[cb]);
#pragma unroll
      for (int B = 0; B < 2; ++B) lsum[rb] = mfma32(ph[rb][B], ones, lsum[rb]);
    };
    // the accumulator rescale with the row sums (rare: only when a row's reference maximum moved)
    auto rescale = [&](int rb) {
      if (__builtin_amdgcn_ballot_w64(moved[rb]) == 0) return;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float ai = shfl(alpha[rb], 4 * g + i);
#pragma unroll
        for (int cb = 0; cb < 8; ++cb) st[rb].acc[cb][i] *= ai;
        lsum[rb][i] *= ai;
      }
    };
    // QK(1) beside softmax(0), PV(0) beside softmax(1): the matrix core and the VALU each have
    // the other row block's work (the rescales, rare, between)
    static_assert(PF_RB == 2, "two row blocks per wave");
    load_k();
    qk(0);
#if PF_SCHED
    // a wave issues in order: without an explicit interleave the compiler emits QK(1) as one run
    // of MFMAs and softmax(0) as one run of VALU instructions, and the matrix core idles through
    // the softmax. QK(0) (with the K operand reads) first, then QK(1) one MFMA at a time between
    // softmax(0)'s instructions
    __builtin_amdgcn_sched_barrier(0);
#endif
    qk(1);
    softmax(0);
#if PF_SCHED
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      __builtin_amdgcn_sched_group_barrier(PF_SG_MFMA, 1, 0);
      __builtin_amdgcn_sched_group_barrier(PF_SG_VALU, PF_SCHED_V, 0);
    }
#endif
    rescale(0);
    load_v();
    pv(0);
    softmax(1);
#if PF_SCHED
    // PV(0) between softmax(1)'s instructions, after the V operand reads
    __builtin_amdgcn_sched_group_barrier(PF_SG_DSR, 16, 1);
#pragma unroll
    for (int i = 0; i < 18; ++i) {
      __builtin_amdgcn_sched_group_barrier(PF_SG_MFMA, 1, 1);
      __builtin_amdgcn_sched_group_barrier(PF_SG_VALU, PF_SCHED_V, 1);
    }
#endif
    rescale(1);
    // PV(1) and the caller's work (the next group's dequantization) in one basic block: the
    // compiler interleaves the two by itself
    tail_work();
    pv(1);
  };

  // ---- cache groups: two LDS stages of int8 codes and two fp16 tile buffers. Group t's codes
  // are dequantized into tile buffer t & 1 during group t - 1's last product (PV of the second
  // row block), so a group takes one workgroup barrier: after it, tile buffer t & 1 is complete,
  // the codes of group t + 1 have landed, and every wave is done with tile buffer (t + 1) & 1 and
  // with the stage of group t
  auto dequant = [&](const uint8_t* sg, uint16_t* ktile, uint16_t* vtile) {
    const uint16_t* rks = reinterpret_cast<const uint16_t*>(sg + 2 * CODE_BYTES);
    // K: thread t dequantizes row t >> 3, dims 16 (t & 7) .. + 15
    const int row = tid >> 3, key = swz(row);
    {
      const int ch = tid & 7;  // 16-dim chunk
      const uint4 kw = *reinterpret_cast<const uint4*>(sg + row * D + ((ch ^ key) << 4));
      const uint4 s0 = *reinterpret_cast<const uint4*>(rks + 16 * ch), s1 = *reinterpret_cast<const uint4*>(rks + 16 * ch + 8);
      const uint4 m0 = *reinterpret_cast<const uint4*>(rks + D + 16 * ch), m1 = *reinterpret_cast<const uint4*>(rks + D + 16 * ch + 8);
      *reinterpret_cast<half8_t*>(ktile + row * PF_KROW + 16 * ch) = dq8(kw.x, kw.y, s0, m0);
      *reinterpret_cast<half8_t*>(ktile + row * PF_KROW + 16 * ch + 8) = dq8(kw.z, kw.w, s1, m1);
    }
    // V: transposed reads; wave w covers dim block w of both 32-token blocks
    const int r = c >> 1;
#pragma unroll
    for (int B = 0; B < 2; ++B)
      {
        const int cb = wave;
        const int vrow = 16 * (2 * B + (r >> 2)) + 4 * g + (r & 3);
        const u32x2 vw = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr8_b64_v2i32(
            (lds_v2i_t*)(const lds_void_t*)(sg + CODE_BYTES + vrow * D + 8 * (c & 1) + ((cb ^ swz(vrow)) << 4))));
        const _Float16 vs = __builtin_bit_cast(_Float16, rks[2 * D + 16 * cb + c]);
        const _Float16 vm = __builtin_bit_cast(_Float16, rks[3 * D + 16 * cb + c]);
        *reinterpret_cast<half8_t*>(vtile + (16 * cb + c) * PF_VROW + 32 * B + 8 * g) =
            dq8_splat(vw.x, vw.y, half2_t{vs, vs}, half2_t{vm, vm});
      }
  };
  if (cs < ce) {
    issue(cs, 0);
    if (cs + 1 < ce) {
      issue(cs + 1, 1);
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(DMA_PF) : "memory");
    } else {
      wait_groups_all();
    }
    __syncthreads();  // stage 0 is complete
    dequant(stage[0], ktile_buf[0], vtile_buf[0]);
  }
  for (int64_t grp = cs; grp < ce; ++grp) {
    const int tb = (int)((grp - cs) & 1);  // tile buffer and stage of group grp
    wait_groups_all();                     // the codes of group grp + 1 (the only loads in flight)
    __syncthreads();
    if (grp + 2 < ce) issue(grp + 2, tb);  // into the stage of group grp, dequantized before the barrier
    // (after the last group the dequantization reads a stale stage into a tile buffer nothing
    // reads again: unconditional, so that it stays in one basic block with the product)
    attend_tiles(-1, tb, [&]() { dequant(stage[tb ^ 1], ktile_buf[tb ^ 1], vtile_buf[tb ^ 1]); });
  }

  // ---- fp16 groups (causal): j = split, split + S, ...
  for (int j = split; j < nchunk; j += a.splits) {
    __syncthreads();  // every wave is done with the tiles
    {
      uint16_t* ktile = ktile_buf[0];
      uint16_t* vtile = vtile_buf[0];
      const int row = tid >> 3, cp = tid & 7, t = GT * j + row;
      const bool ok = t < a.Mk;
      const uint16_t* kr = a.kc + (int64_t)h * a.kc_hs + (int64_t)(ok ? t : 0) * D + 16 * cp;
      const uint16_t* vr = a.vc + (int64_t)h * a.kc_hs + (int64_t)(ok ? t : 0) * D + 16 * cp;
      const int vs = pf_vslot(row);
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const uint4 kw = ok ? *reinterpret_cast<const uint4*>(kr + 8 * e) : uint4{0, 0, 0, 0};
        const uint4 vw = ok ? *reinterpret_cast<const uint4*>(vr + 8 * e) : uint4{0, 0, 0, 0};
        *reinterpret_cast<uint4*>(ktile + row * PF_KROW + 16 * cp + 8 * e) = kw;
        const uint32_t wv[4] = {vw.x, vw.y, vw.z, vw.w};
#pragma unroll
        for (int q2 = 0; q2 < 8; ++q2)
          vtile[(16 * cp + 8 * e + q2) * PF_VROW + vs] = (uint16_t)(wv[q2 >> 1] >> (16 * (q2 & 1)));
      }
    }
    __syncthreads();
    attend_tiles(GT * j, 0, []() {});
  }

  // ---- one partial per row: acc[128] and l (both x 2^15), m (log2 domain)
  const int64_t total_rows = (int64_t)a.hkv * rows_h;
#pragma unroll
  for (int rb = 0; rb < PF_RB; ++rb) {
    const int rbase = row0 + 16 * rb;
    float* dst = a.ws + ((int64_t)split * total_rows + (int64_t)h * rows_h) * PF_PART;
    if (g == 0 && rbase + c < rows_h) dst[(int64_t)(rbase + c) * PF_PART + D] = st[rb].m;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (c == 0 && rbase + 4 * g + i < rows_h) dst[(int64_t)(rbase + 4 * g + i) * PF_PART + D + 1] = lsum[rb][i];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = rbase + 4 * g + i;
      if (r < rows_h)
#pragma unroll
        for (int cb = 0; cb < 8; ++cb) dst[(int64_t)r * PF_PART + 16 * cb + c] = st[rb].acc[cb][i];
    }
  }
}

// Merge of the splits' partials: one thread per (row, 4 dims).
__global__ __launch_bounds__(256) void prefill_combine_kernel(PrefillArgs a) {
  const int rows_h = a.M * a.gq;
  const int64_t total_rows = (int64_t)a.hkv * rows_h;
  const int64_t item = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (item >= total_rows * (D / 4)) return;
  const int64_t row = item / (D / 4);
  const int d4 = (int)(item % (D / 4)) * 4;
  float m = NEG_INF;
  for (int s = 0; s < a.splits; ++s) m = fmaxf(m, a.ws[((int64_t)s * total_rows + row) * PF_PART + D]);
  const float mu = m == NEG_INF ? 0.0f : m;
  float4 acc = {0.f, 0.f, 0.f, 0.f};
  float l = 0.0f;
  for (int s = 0; s < a.splits; ++s) {
    const float* p = a.ws + ((int64_t)s * total_rows + row) * PF_PART;
    const float ms = p[D];
    const float w = ms == NEG_INF ? 0.0f : __builtin_amdgcn_exp2f(ms - mu);
    const float4 v = *reinterpret_cast<const float4*>(p + d4);
    acc.x += v.x * w; acc.y += v.y * w; acc.z += v.z * w; acc.w += v.w * w;
    l += p[D + 1] * w;
  }
  const int h = (int)(row / rows_h), r = (int)(row % rows_h);
  const int tk = r / a.gq, hd = h * a.gq + r % a.gq;
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;  // acc and l carry the same 2^15 scale
  uint16_t* o = a.out + ((int64_t)hd * a.M + tk) * D + d4;
  *reinterpret_cast<uint2*>(o) = uint2{(uint32_t)f2h(acc.x * inv) | ((uint32_t)f2h(acc.y * inv) << 16),
                                       (uint32_t)f2h(acc.z * inv) | ((uint32_t)f2h(acc.w * inv) << 16)};
}

// ---------------------------------------------------------------- host side

// ---- the XCD-local hand-over per device: the XCD count when on, 0 (off) until nkv_l2_handover
// has probed the device
constexpr int L2_DEVICES = 64;
constexpr int XCD_PROBE_WGS = 4096;
static std::mutex g_l2_mu;
static int g_l2_xcc[L2_DEVICES];
static __device__ uint32_t g_xcd_probe[XCD_PROBE_WGS];

__global__ __launch_bounds__(64) void xcd_probe_kernel(uint32_t* out) {
  if (threadIdx.x == 0) out[blockIdx.x] = xcc_id();
}

// Core clock probe: workgroup b (one wave) runs `iters` rounds of two dependent FMAs and records
// its XCD and how far the core clock counter (s_memtime) and the 100 MHz real-time counter
// (s_memrealtime) advanced meanwhile: out[3 b .. 3 b + 2]. The FMAs' result is kept by a
// comparison that never holds, so the loop stays.
__global__ __launch_bounds__(64) void clock_probe_kernel(uint64_t* out, int iters) {
  const uint64_t t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  float x = threadIdx.x * 1e-3f, y = 1.0001f;
  for (int i = 0; i < iters; ++i) {
    x = __builtin_fmaf(x, y, 1e-7f);
    y = __builtin_fmaf(y, 0.99999f, 1e-6f);
  }
  const uint64_t t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  if (threadIdx.x == 0) {
    out[3 * blockIdx.x] = xcc_id();
    out[3 * blockIdx.x + 1] = t1 - t0 + (x == -1.0f ? (uint64_t)y : 0);
    out[3 * blockIdx.x + 2] = r1 - r0;
  }
}

extern "C" int nkv_clock_probe(uint64_t* out, int64_t blocks, int64_t iters, void* stream) {
  set_error("");
  if (!out || blocks <= 0 || blocks > 1024 || iters <= 0 || iters > (1 << 24))
    return fail(NKV_ERR_INVALID, "clock_probe: out required, 1 <= blocks <= 1024, 1 <= iters <= 2^24");
  hipLaunchKernelGGL(clock_probe_kernel, dim3((unsigned)blocks), dim3(64), 0, static_cast<hipStream_t>(stream), out,
                     (int)iters);
  return check_launch("clock_probe");
}

// The launch's hand-over fields: on when the current device was probed and its XCD count divides
// hkv (so that workgroups b = h mod hkv of KV head h share XCD b mod n).
static void l2_args(AttnArgs& a) {
  a.l2_xcc = 0;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= L2_DEVICES) return;
  std::lock_guard<std::mutex> lock(g_l2_mu);
  const int n = g_l2_xcc[dev];
  if (n > 0 && a.hkv % n == 0) a.l2_xcc = n;
}

// Prefix work units per KV head: at least 8 groups (one per wave) per workgroup, and at
// most one workgroup per CU (256 CUs).
static int64_t default_parts(int64_t hkv, int64_t groups) {
  const int64_t max_parts = std::max<int64_t>(1, 256 / std::max<int64_t>(1, hkv));
  return std::min<int64_t>(max_parts, std::max<int64_t>(1, cdiv(groups, 8)));
}

static int64_t part_floats(int64_t hq, int64_t hkv) { return part_stride((int)(hq / hkv)); }
// Bytes of the fused tail's publication area: `n` ints (per head a counter and a flag per
// partial; paged, a counter per sequence and head), rounded up to 256 bytes.
static int64_t ctr_bytes(int64_t n) { return (n * (int64_t)sizeof(int) + 255) / 256 * 256; }
static int64_t sync_bytes(int64_t hkv, int64_t n_parts) { return ctr_bytes(hkv * (1 + std::max<int64_t>(1, n_parts))); }

static int check_heads(int64_t hq, int64_t hkv, int64_t head_dim) {
  if (hkv <= 0 || hq <= 0 || hq % hkv) return fail(NKV_ERR_INVALID, "Q heads %lld not divisible by KV heads %lld", (long long)hq, (long long)hkv);
  if (hq / hkv > 16) return fail(NKV_ERR_INVALID, "%lld Q heads per KV head exceeds the padding limit 16", (long long)(hq / hkv));
  if (head_dim != D) return fail(NKV_ERR_UNSUPPORTED, "head_dim %lld: the HIP kernels are built for head_dim 128", (long long)head_dim);
  return NKV_OK;
}

// Kernel A over n_parts prefix parts (none when n_parts == 0), then kernel B.
constexpr int LAUNCH_PREFIX = 1, LAUNCH_TAIL = 2;

// `fusable`: the workspace is one the caller keeps zero-filled for these entry points (the
// decode-step family), so both launches may become one with the last-workgroup tail.
static int launch_attn(AttnArgs& a, int64_t n_parts, int64_t workspace_bytes, hipStream_t s, const char* what,
                       int launches = LAUNCH_PREFIX | LAUNCH_TAIL, bool fusable = false) {
  if (n_parts < 0) return fail(NKV_ERR_INVALID, "%s: n_parts %lld is negative", what, (long long)n_parts);
  a.n_parts = (int)n_parts;
  // both launches in one call: the prefix kernel's part-0 workgroup of each head runs the tail
  // (at most MERGER_MAX_PARTS parts and MERGER_MAX_HEADS heads; beyond, the two launches)
  const bool fuse = fusable && n_parts > 0 && n_parts <= MERGER_MAX_PARTS && a.hkv <= MERGER_MAX_HEADS &&
                    launches == (LAUNCH_PREFIX | LAUNCH_TAIL);
  const int64_t part_bytes = (int64_t)a.hkv * std::max<int64_t>(1, n_parts) * part_floats(a.hq, a.hkv) * (int64_t)sizeof(float);
  const int64_t need = part_bytes + (fuse ? sync_bytes(a.hkv, n_parts) : 0);
  if (n_parts > 0 && workspace_bytes < need)
    return fail(NKV_ERR_INVALID, "%s: workspace of %lld bytes, need %lld", what, (long long)workspace_bytes, (long long)need);
  if (n_parts > 256) return fail(NKV_ERR_UNSUPPORTED, "%s: n_parts %lld exceeds the 256 partials the merge holds", what, (long long)n_parts);
  if (a.capacity > (int64_t(1) << 24))  // code row offsets of one head stay 32-bit
    return fail(NKV_ERR_UNSUPPORTED, "%s: capacity %lld exceeds 16M tokens", what, (long long)a.capacity);
  a.inline_tail = fuse ? 1 : 0;
  a.tail_ctr_end = reinterpret_cast<int*>(reinterpret_cast<char*>(a.ws) + (workspace_bytes & ~int64_t(3)));
  l2_args(a);
  if (n_parts > 0 && (launches & LAUNCH_PREFIX)) {
    const int64_t parts = a.tail_mode == TAIL_FUSED && !a.tok ? std::max<int64_t>(n_parts, APPEND_UNITS) : n_parts;
    if (a.tok) hipLaunchKernelGGL(attn_prefix_kernel<CONTIG_TOK>, dim3((unsigned)(a.hkv * parts)), dim3(THREADS), 0, s, a);
    else hipLaunchKernelGGL(attn_prefix_kernel<CONTIG_T64>, dim3((unsigned)(a.hkv * parts)), dim3(THREADS), 0, s, a);
    if (int rc = check_launch(what)) return rc;
  }
  if (!(launches & LAUNCH_TAIL) || fuse) return NKV_OK;
  hipLaunchKernelGGL(attn_tail_kernel<false>, dim3((unsigned)a.hkv), dim3(TB_THREADS), 0, s, a);
  return check_launch(what);
}

static bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Whether the byte ranges [a, a + an) and [b, b + bn) share a byte.
static bool overlaps(const void* a, int64_t an, const void* b, int64_t bn) {
  const uintptr_t pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
  return pa < pb + (uintptr_t)bn && pb < pa + (uintptr_t)an;
}

// The fused projection step's workspace: the decode step's partials (n_parts per KV head), the
// tagged row words [hkv][QKV_HAND_ROWS], the tags' epochs [hkv] (256-byte padded), the new token's
// k / v [hkv][2][D] fp16, the output's tagged words [hq D / 2] and issue flags [FLAG_COPIES][hq]
// (with w_o), and the step's counters at the end.
static int64_t up256(int64_t n) { return (n + 255) / 256 * 256; }
static int64_t qkv_part_bytes(int64_t hkv, int64_t hq, int64_t n_parts) {
  return up256(hkv * std::max<int64_t>(1, n_parts) * part_floats(hq, hkv) * (int64_t)sizeof(float));
}
static int64_t qkv_workspace_bytes(int64_t hkv, int64_t hq, int64_t n_parts) {
  return qkv_part_bytes(hkv, hq, n_parts) + hkv * QKV_HAND_ROWS * 8 + up256(hkv * 4) + up256(hkv * 2 * D * 2) +
         up256(hq * D / 2 * 8) + up256(FLAG_COPIES * hq * 4) + sync_bytes(hkv, n_parts);
}

// Workgroups of the fused projection step resident at once on the current device (every
// workgroup of a KV head waits for rows the others compute, so the grid must fit at once).
static std::mutex g_qkv_mu;
static int g_qkv_resident[L2_DEVICES];
static int qkv_resident(int* out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= L2_DEVICES)
    return fail(NKV_ERR_HIP, "decode_step_qkv_t64: no usable current device (%d)", dev);
  std::lock_guard<std::mutex> lock(g_qkv_mu);
  int& r = g_qkv_resident[dev];
  if (!r) {
    int cus = 0, per_cu = 0;
    hipError_t e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e == hipSuccess)
      e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, attn_prefix_kernel<CONTIG_T64, true>, THREADS, 0);
    if (e != hipSuccess) return fail(NKV_ERR_HIP, "decode_step_qkv_t64: occupancy query: %s", hipGetErrorString(e));
    r = cus * per_cu;
  }
  *out = r;
  return NKV_OK;
}

}  // namespace nkv

using namespace nkv;

extern "C" int64_t nkv_attn_workspace_bytes(int64_t hkv, int64_t hq, int64_t n_parts) {
  if (hkv <= 0 || hq <= 0 || n_parts < 0 || hq % hkv) return 0;
  return hkv * std::max<int64_t>(1, n_parts) * part_floats(hq, hkv) * (int64_t)sizeof(float) + sync_bytes(hkv, n_parts);
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
                                   int64_t workspace_bytes, int64_t n_parts, void* stream) {
  set_error("");
  if (int rc = check_heads(hq, hkv, head_dim)) return rc;
  if (capacity <= 0) return fail(NKV_ERR_INVALID, "capacity must be positive");
  if (!q || !kq || !kmn || !kst || !vq || !vmn || !vst || !out || !workspace)
    return fail(NKV_ERR_INVALID, "attn_decode: null pointer argument");
  if (!al16(q) || !al16(kq) || !al16(vq) || !al16(kmn) || !al16(kst) || !al16(vmn) || !al16(vst) || !al16(workspace))
    return fail(NKV_ERR_UNSUPPORTED, "attn_decode: buffers must be 16-byte aligned");
  if ((tail_k == nullptr) != (tail_v == nullptr)) return fail(NKV_ERR_INVALID, "tail_k and tail_v go together");
  if (tail_k && !written_dev) return fail(NKV_ERR_INVALID, "the ring needs written_dev");
  if (tail_k && (!al16(tail_k) || !al16(tail_v))) return fail(NKV_ERR_UNSUPPORTED, "attn_decode: the ring must be 16-byte aligned");
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
  a.out = out; a.lse = lse_out; a.ws = static_cast<float*>(workspace);
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
  if (!al16(k_new) || !al16(v_new) || kv_head_stride % 8 || !al16(tail_k) || !al16(tail_v) || !al16(kq) || !al16(vq) ||
      !al16(kmn) || !al16(kst) || !al16(vmn) || !al16(vst))
    return fail(NKV_ERR_UNSUPPORTED, "append: buffers must be 16-byte aligned");
  AttnArgs a{};
  a.k_new = k_new; a.v_new = v_new; a.kv_hs = kv_head_stride;
  a.kq = kq; a.kmn = kmn; a.kst = kst; a.vq = vq; a.vmn = vmn; a.vst = vst;
  a.tail_k = tail_k; a.tail_v = tail_v; a.pos_dev = pos_dev;
  a.written_out = written_dev; a.qlen_out = qlen_dev; a.pg_out = pg_dev;
  a.capacity = capacity; a.ngroups_cap = cdiv(capacity, GT); a.hkv = (int)hkv; a.tail_slots = GT;
  hipLaunchKernelGGL(append_kernel, dim3((unsigned)(hkv * APPEND_UNITS)), dim3(THREADS), 0, static_cast<hipStream_t>(stream), a);
  return check_launch("append_t64");
}

static int decode_step(const char* what, int launches, const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                                   int64_t kv_head_stride, uint8_t* kq, uint16_t* kmn, uint16_t* kst,
                                   uint8_t* vq, uint16_t* vmn, uint16_t* vst, uint16_t* tail_k,
                                   uint16_t* tail_v, const int64_t* pos_dev, const int64_t* first_dev,
                                   int64_t* written_dev, int64_t* qlen_dev, int64_t* pg_dev, int64_t hq,
                                   int64_t hkv, int64_t head_dim, int64_t capacity, uint16_t* out,
                                   float* lse_out, void* workspace, int64_t workspace_bytes,
                                   int64_t n_parts, void* stream) {
  set_error("");
  if (int rc = check_heads(hq, hkv, head_dim)) return rc;
  if (capacity <= 0) return fail(NKV_ERR_INVALID, "capacity must be positive");
  if (!q || !k_new || !v_new || !kq || !kmn || !kst || !vq || !vmn || !vst || !tail_k || !tail_v ||
      !pos_dev || !written_dev || !qlen_dev || !pg_dev || !out || !workspace)
    return fail(NKV_ERR_INVALID, "%s: null pointer argument", what);
  if (!al16(q) || !al16(k_new) || !al16(v_new) || kv_head_stride % 8 || !al16(tail_k) || !al16(tail_v) ||
      !al16(kq) || !al16(vq) || !al16(kmn) || !al16(kst) || !al16(vmn) || !al16(vst) || !al16(workspace))
    return fail(NKV_ERR_UNSUPPORTED, "%s: buffers must be 16-byte aligned", what);
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
  a.out = out; a.lse = lse_out; a.ws = static_cast<float*>(workspace);
  return launch_attn(a, n_parts, workspace_bytes, static_cast<hipStream_t>(stream), what, launches, true);
}

extern "C" int nkv_decode_step_t64(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                                   int64_t kv_head_stride, uint8_t* kq, uint16_t* kmn, uint16_t* kst,
                                   uint8_t* vq, uint16_t* vmn, uint16_t* vst, uint16_t* tail_k,
                                   uint16_t* tail_v, const int64_t* pos_dev, const int64_t* first_dev,
                                   int64_t* written_dev, int64_t* qlen_dev, int64_t* pg_dev, int64_t hq,
                                   int64_t hkv, int64_t head_dim, int64_t capacity, uint16_t* out,
                                   float* lse_out, void* workspace, int64_t workspace_bytes,
                                   int64_t n_parts, void* stream) {
  return decode_step("decode_step_t64", LAUNCH_PREFIX | LAUNCH_TAIL, q, k_new, v_new, kv_head_stride, kq, kmn, kst, vq, vmn, vst, tail_k, tail_v, pos_dev, first_dev,
                     written_dev, qlen_dev, pg_dev, hq, hkv, head_dim, capacity, out, lse_out, workspace,
                     workspace_bytes, n_parts, stream);
}

extern "C" int nkv_decode_step_partials_t64(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                                   int64_t kv_head_stride, uint8_t* kq, uint16_t* kmn, uint16_t* kst,
                                   uint8_t* vq, uint16_t* vmn, uint16_t* vst, uint16_t* tail_k,
                                   uint16_t* tail_v, const int64_t* pos_dev, const int64_t* first_dev,
                                   int64_t* written_dev, int64_t* qlen_dev, int64_t* pg_dev, int64_t hq,
                                   int64_t hkv, int64_t head_dim, int64_t capacity, uint16_t* out,
                                   float* lse_out, void* workspace, int64_t workspace_bytes,
                                   int64_t n_parts, void* stream) {
  return decode_step("decode_step_partials_t64", LAUNCH_PREFIX, q, k_new, v_new, kv_head_stride, kq, kmn, kst, vq, vmn, vst, tail_k, tail_v, pos_dev, first_dev,
                     written_dev, qlen_dev, pg_dev, hq, hkv, head_dim, capacity, out, lse_out, workspace,
                     workspace_bytes, n_parts, stream);
}

extern "C" int nkv_decode_step_combine_t64(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                                   int64_t kv_head_stride, uint8_t* kq, uint16_t* kmn, uint16_t* kst,
                                   uint8_t* vq, uint16_t* vmn, uint16_t* vst, uint16_t* tail_k,
                                   uint16_t* tail_v, const int64_t* pos_dev, const int64_t* first_dev,
                                   int64_t* written_dev, int64_t* qlen_dev, int64_t* pg_dev, int64_t hq,
                                   int64_t hkv, int64_t head_dim, int64_t capacity, uint16_t* out,
                                   float* lse_out, void* workspace, int64_t workspace_bytes,
                                   int64_t n_parts, void* stream) {
  return decode_step("decode_step_combine_t64", LAUNCH_TAIL, q, k_new, v_new, kv_head_stride, kq, kmn, kst, vq, vmn, vst, tail_k, tail_v, pos_dev, first_dev,
                     written_dev, qlen_dev, pg_dev, hq, hkv, head_dim, capacity, out, lse_out, workspace,
                     workspace_bytes, n_parts, stream);
}

// ---- the decode step on a library-held scratch array (no allocation anywhere)
//
// Layout: [partials: NKV_STATIC_PART_BYTES | publication area: NKV_STATIC_SYNC_BYTES]. The
// step writes partials upward from the start and keeps its counters and flags downward from
// the end, so any mix of configurations within the limits keeps the two regions apart, and
// the publication area, cleared once, stays cleared (each call leaves its counters at zero).
constexpr int64_t STATIC_BYTES = int64_t(NKV_STATIC_PART_BYTES) + NKV_STATIC_SYNC_BYTES;
static_assert(NKV_STATIC_PART_BYTES % 256 == 0 && NKV_STATIC_SYNC_BYTES % 256 == 0, "256-byte regions");

static __device__ __align__(256) unsigned char scratch[STATIC_BYTES];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[MAX_DEVICES];  // device address of `scratch` per device, set once

// Device address of the current device's `scratch`. The first call on a device looks it up
// (the host-side name is not a device address) and clears the publication area with a kernel
// on `s`, ordered before the caller's launches on that stream.
int static_scratch(hipStream_t s, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES)
    return fail(NKV_ERR_HIP, "decode_step_static_t64: no usable current device (%d)", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(NKV_ERR_HIP, "decode_step_static_t64: hipGetSymbolAddress: %s", hipGetErrorString(e));
    const int n = (int)(STATIC_BYTES / (int64_t)sizeof(int));
    hipLaunchKernelGGL(clear_ints_kernel, dim3((unsigned)cdiv(n, 4 * 256)), dim3(256), 0, s, static_cast<int*>(p), n);
    if (int rc = check_launch("decode_step_static_t64: clear")) return rc;
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return NKV_OK;
}
}  // namespace

extern "C" int nkv_decode_step_static_t64(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                                          int64_t kv_head_stride, uint8_t* kq, uint16_t* kmn, uint16_t* kst,
                                          uint8_t* vq, uint16_t* vmn, uint16_t* vst, uint16_t* tail_k,
                                          uint16_t* tail_v, const int64_t* pos_dev, const int64_t* first_dev,
                                          int64_t* written_dev, int64_t* qlen_dev, int64_t* pg_dev, int64_t hq,
                                          int64_t hkv, int64_t head_dim, int64_t capacity, uint16_t* out,
                                          float* lse_out, int64_t n_parts, void* stream) {
  const char* what = "decode_step_static_t64";
  set_error("");
  if (int rc = check_heads(hq, hkv, head_dim)) return rc;
  if (capacity <= 0) return fail(NKV_ERR_INVALID, "capacity must be positive");
  if (n_parts < 0) return fail(NKV_ERR_INVALID, "%s: n_parts %lld is negative", what, (long long)n_parts);
  if (n_parts == 0) n_parts = default_parts(hkv, cdiv(capacity, GT));
  const int64_t part_bytes = hkv * n_parts * part_floats(hq, hkv) * (int64_t)sizeof(float);
  const int64_t sync = sync_bytes(hkv, n_parts);
  if (part_bytes > NKV_STATIC_PART_BYTES || sync > NKV_STATIC_SYNC_BYTES)
    return fail(NKV_ERR_UNSUPPORTED,
                "%s: %lld partial bytes and %lld publication bytes exceed the static scratch (%d and %d bytes)",
                what, (long long)part_bytes, (long long)sync, NKV_STATIC_PART_BYTES, NKV_STATIC_SYNC_BYTES);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  void* ws = nullptr;
  if (int rc = static_scratch(s, &ws)) return rc;
  return decode_step(what, LAUNCH_PREFIX | LAUNCH_TAIL, q, k_new, v_new, kv_head_stride, kq, kmn, kst, vq, vmn, vst,
                     tail_k, tail_v, pos_dev, first_dev, written_dev, qlen_dev, pg_dev, hq, hkv, head_dim, capacity,
                     out, lse_out, ws, STATIC_BYTES, n_parts, stream);
}

extern "C" int nkv_l2_handover(int enable, int64_t* xcds, void* stream) {
  if (xcds) *xcds = 0;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= L2_DEVICES)
    return fail(NKV_ERR_HIP, "l2_handover: no usable current device (%d)", dev);
  int on = 0;
  if (enable) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess) n = 0;
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(g_xcd_probe));
    if (e != hipSuccess || !p) return fail(NKV_ERR_HIP, "l2_handover: hipGetSymbolAddress: %s", hipGetErrorString(e));
    hipStream_t s = static_cast<hipStream_t>(stream);
    std::vector<uint32_t> got(XCD_PROBE_WGS);
    hipLaunchKernelGGL(xcd_probe_kernel, dim3(XCD_PROBE_WGS), dim3(64), 0, s, static_cast<uint32_t*>(p));
    if (int rc = check_launch("l2_handover: probe")) return rc;
    e = hipMemcpyAsync(got.data(), p, sizeof(uint32_t) * XCD_PROBE_WGS, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return fail(NKV_ERR_HIP, "l2_handover: probe readback: %s", hipGetErrorString(e));
    // on only for 1..8 XCDs (a power of two) dealt in turn: workgroup b on the XCD of workgroup
    // b mod n, the first n on n distinct XCDs
    bool ok = n >= 1 && n <= 8 && (n & (n - 1)) == 0;
    for (int b = 0; ok && b < XCD_PROBE_WGS; ++b) ok = got[b] == got[b % n];
    for (int i = 0; ok && i < n; ++i)
      for (int j = 0; j < i; ++j) ok = ok && got[i] != got[j];
    if (ok) on = n;
  }
  {
    std::lock_guard<std::mutex> lock(g_l2_mu);
    g_l2_xcc[dev] = on;
  }
  if (xcds) *xcds = on;
  return NKV_OK;
}

extern "C" int64_t nkv_decode_step_qkv_workspace_bytes(int64_t hkv, int64_t hq, int64_t capacity, int64_t n_parts) {
  if (hkv <= 0 || hq <= 0 || capacity <= 0) return 0;
  if (n_parts <= 0) n_parts = default_parts(hkv, cdiv(capacity, GT));
  return qkv_workspace_bytes(hkv, hq, n_parts);
}

extern "C" int nkv_decode_step_qkv_t64(const uint16_t* x, const uint16_t* x_gamma, float x_eps, const uint16_t* w_qkv,
                                       int64_t hidden, const uint16_t* q_gamma, const uint16_t* k_gamma, float qk_eps,
                                       const float* inv_freq, uint16_t* qkv_out, uint8_t* kq, uint16_t* kmn,
                                       uint16_t* kst, uint8_t* vq, uint16_t* vmn, uint16_t* vst, uint16_t* tail_k,
                                       uint16_t* tail_v, const int64_t* pos_dev, const int64_t* first_dev,
                                       int64_t* written_dev, int64_t* qlen_dev, int64_t* pg_dev, int64_t hq,
                                       int64_t hkv, int64_t head_dim, int64_t capacity, uint16_t* out, float* lse_out,
                                       const uint16_t* w_o, uint16_t* h1_out, void* workspace, int64_t workspace_bytes,
                                       int64_t n_parts, void* stream) {
  const char* what = "decode_step_qkv_t64";
  set_error("");
  if (int rc = check_heads(hq, hkv, head_dim)) return rc;
  if (hq / hkv > QKV_MAX_GQ)
    return fail(NKV_ERR_UNSUPPORTED, "%s: %lld q heads per KV head (at most %d)", what, (long long)(hq / hkv), QKV_MAX_GQ);
  if (capacity <= 0) return fail(NKV_ERR_INVALID, "%s: capacity must be positive", what);
  if (hidden <= 0 || hidden % 8 || hidden > QKV_MAX_HIDDEN)
    return fail(NKV_ERR_UNSUPPORTED, "%s: hidden size %lld (a positive multiple of 8, at most %d)", what,
                (long long)hidden, QKV_MAX_HIDDEN);
  if (!x || !x_gamma || !w_qkv || !q_gamma || !k_gamma || !inv_freq || !kq || !kmn || !kst || !vq || !vmn || !vst ||
      !tail_k || !tail_v || !pos_dev || !written_dev || !qlen_dev || !pg_dev || !out || !workspace)
    return fail(NKV_ERR_INVALID, "%s: null pointer argument", what);
  if (!al16(x) || !al16(x_gamma) || !al16(w_qkv) || !al16(tail_k) || !al16(tail_v) || !al16(kq) || !al16(vq) ||
      !al16(kmn) || !al16(kst) || !al16(vmn) || !al16(vst) || !al16(workspace))
    return fail(NKV_ERR_UNSUPPORTED, "%s: buffers must be 16-byte aligned", what);
  if (capacity > (int64_t(1) << 24)) return fail(NKV_ERR_UNSUPPORTED, "%s: capacity %lld exceeds 16M tokens", what, (long long)capacity);
  const int64_t ngroups = cdiv(capacity, GT);
  if (n_parts <= 0) n_parts = default_parts(hkv, ngroups);
  if (n_parts > MERGER_MAX_PARTS || hkv > MERGER_MAX_HEADS)
    return fail(NKV_ERR_UNSUPPORTED, "%s: %lld parts per KV head, %lld KV heads (at most %d and %d)", what,
                (long long)n_parts, (long long)hkv, MERGER_MAX_PARTS, MERGER_MAX_HEADS);
  const int64_t parts = std::max<int64_t>(n_parts, APPEND_UNITS), grid = hkv * parts;
  int resident = 0;
  if (int rc = qkv_resident(&resident)) return rc;
  if (grid > resident)
    return fail(NKV_ERR_UNSUPPORTED, "%s: %lld workgroups exceed the %d this device holds at once (the workgroups of a "
                "KV head wait for each other's rows)", what, (long long)grid, resident);
  const int64_t need = qkv_workspace_bytes(hkv, hq, n_parts);
  if (workspace_bytes < need)
    return fail(NKV_ERR_INVALID, "%s: workspace of %lld bytes, need %lld", what, (long long)workspace_bytes, (long long)need);
  if (w_o) {
    const int64_t readers = grid - hkv;
    if (!h1_out) return fail(NKV_ERR_INVALID, "%s: w_o without h1_out", what);
    if (!al16(w_o)) return fail(NKV_ERR_UNSUPPORTED, "%s: w_o must be 16-byte aligned", what);
    if (hq * D > OP_NL * 64 * 8 || hq > 64)
      return fail(NKV_ERR_UNSUPPORTED, "%s: the output projection takes at most %d query heads", what, OP_NL * 64 * 8 / D);
    if (hidden > 2 * readers * WAVES)
      return fail(NKV_ERR_UNSUPPORTED, "%s: hidden size %lld exceeds two rows per reader wave (%lld)", what,
                  (long long)hidden, (long long)(2 * readers * WAVES));
    // h1 is written after every workgroup has read x: it may be x itself, or apart from it and from out
    if (h1_out != x && overlaps(h1_out, hidden * 2, x, hidden * 2))
      return fail(NKV_ERR_INVALID, "%s: h1_out must be x itself or not overlap it", what);
    if (overlaps(h1_out, hidden * 2, out, hq * D * 2)) return fail(NKV_ERR_INVALID, "%s: h1_out overlaps out", what);
  }
  char* ws = static_cast<char*>(workspace);
  uint64_t* hand = reinterpret_cast<uint64_t*>(ws + qkv_part_bytes(hkv, hq, n_parts));
  int* epoch = reinterpret_cast<int*>(hand + hkv * QKV_HAND_ROWS);
  uint16_t* kvbuf = reinterpret_cast<uint16_t*>(reinterpret_cast<char*>(epoch) + up256(hkv * 4));
  uint64_t* owords = reinterpret_cast<uint64_t*>(reinterpret_cast<char*>(kvbuf) + up256(hkv * 2 * D * 2));
  uint32_t* oflags = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(owords) + up256(hq * D / 2 * 8));
  AttnArgs a{};
  a.k_new = kvbuf; a.v_new = kvbuf + D; a.kv_hs = 2 * D;
  a.kq = kq; a.kmn = kmn; a.kst = kst; a.vq = vq; a.vmn = vmn; a.vst = vst;
  a.tail_k = tail_k; a.tail_v = tail_v; a.pos_dev = pos_dev; a.first_dev = first_dev;
  a.written_out = written_dev; a.qlen_out = qlen_dev; a.pg_out = pg_dev;
  a.capacity = capacity; a.ngroups_cap = ngroups; a.tail_slots = GT;
  a.hq = (int)hq; a.hkv = (int)hkv; a.gq = (int)(hq / hkv);
  a.tail_mode = TAIL_FUSED;
  a.sl2 = LOG2E / sqrtf((float)head_dim);
  a.out = out; a.lse = lse_out; a.ws = static_cast<float*>(workspace);
  a.n_parts = (int)n_parts;
  a.inline_tail = 1;
  a.tail_ctr_end = reinterpret_cast<int*>(ws + (workspace_bytes & ~int64_t(3)));
  a.x = x; a.x_gamma = x_gamma; a.w_qkv = w_qkv; a.q_gamma = q_gamma; a.k_gamma = k_gamma; a.inv_freq = inv_freq;
  a.eps_x = x_eps; a.eps_qk = qk_eps; a.hidden = (int)hidden;
  a.hand = hand; a.qkv_epoch = epoch; a.qkv_out = qkv_out;
  if (w_o) {
    a.w_o = w_o; a.h1_out = h1_out; a.fwd_out = owords; a.issue_flags = oflags; a.fwd_agent = 1;
  }
  l2_args(a);
  hipLaunchKernelGGL((attn_prefix_kernel<CONTIG_T64, true>), dim3((unsigned)grid), dim3(THREADS), 0,
                     static_cast<hipStream_t>(stream), a);
  return check_launch(what);
}

extern "C" int nkv_tail_attend(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                               const uint8_t* mask, int64_t hq, int64_t hkv, int64_t head_dim,
                               int64_t slots, uint16_t* out, float* lse, void* stream) {
  set_error("");
  if (int rc = check_heads(hq, hkv, head_dim)) return rc;
  if (slots <= 0 || slots > GT) return fail(NKV_ERR_UNSUPPORTED, "tail_attend: %lld slots (1..64 supported)", (long long)slots);
  if (!q || !k || !v || !mask || !out || !lse) return fail(NKV_ERR_INVALID, "tail_attend: null pointer argument");
  if (!al16(q) || !al16(k) || !al16(v)) return fail(NKV_ERR_UNSUPPORTED, "tail_attend: buffers must be 16-byte aligned");
  AttnArgs a{};
  a.q = q; a.tail_k = const_cast<uint16_t*>(k); a.tail_v = const_cast<uint16_t*>(v); a.tail_mask = mask;
  a.capacity = 1; a.ngroups_cap = 1; a.tail_slots = slots;
  a.hq = (int)hq; a.hkv = (int)hkv; a.gq = (int)(hq / hkv);
  a.tail_mode = TAIL_MASK;
  a.sl2 = LOG2E / sqrtf((float)head_dim);
  a.out = out; a.lse = lse;
  return launch_attn(a, 0, 0, static_cast<hipStream_t>(stream), "tail_attend");
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

// ---------------------------------------------------------------- per-token symmetric format

static int check_tok_cache(const char* what, int64_t capacity, const void* kq, const void* ksc, const void* vq,
                           const void* vsc) {
  if (capacity <= 0 || capacity % GT) return fail(NKV_ERR_INVALID, "%s: capacity %lld must be a positive multiple of 64", what, (long long)capacity);
  if (!kq || !ksc || !vq || !vsc) return fail(NKV_ERR_INVALID, "%s: null pointer argument", what);
  if (!al16(kq) || !al16(vq) || !al16(ksc) || !al16(vsc)) return fail(NKV_ERR_UNSUPPORTED, "%s: buffers must be 16-byte aligned", what);
  return NKV_OK;
}

extern "C" int nkv_attn_decode_tok(const uint16_t* q, const int8_t* kq, const uint16_t* ksc, const int8_t* vq,
                                   const uint16_t* vsc, int64_t hq, int64_t hkv, int64_t head_dim, int64_t capacity,
                                   int64_t used, const int64_t* used_dev, uint16_t* out, float* lse_out,
                                   void* workspace, int64_t workspace_bytes, int64_t n_parts, void* stream) {
  set_error("");
  if (int rc = check_heads(hq, hkv, head_dim)) return rc;
  if (int rc = check_tok_cache("attn_decode_tok", capacity, kq, ksc, vq, vsc)) return rc;
  if (!q || !out || !workspace) return fail(NKV_ERR_INVALID, "attn_decode_tok: null pointer argument");
  if (!al16(q) || !al16(workspace)) return fail(NKV_ERR_UNSUPPORTED, "attn_decode_tok: buffers must be 16-byte aligned");
  if (!used_dev && (used < 0 || used > capacity)) return fail(NKV_ERR_INVALID, "used=%lld outside [0, %lld]", (long long)used, (long long)capacity);
  const int64_t ngroups = capacity / GT;
  if (n_parts <= 0) n_parts = default_parts(hkv, used_dev ? ngroups : cdiv(used, GT));
  AttnArgs a{};
  a.q = q; a.kq = reinterpret_cast<uint8_t*>(const_cast<int8_t*>(kq)); a.vq = reinterpret_cast<uint8_t*>(const_cast<int8_t*>(vq));
  a.ksc = const_cast<uint16_t*>(ksc); a.vsc = const_cast<uint16_t*>(vsc); a.tok = 1;
  a.used_dev = used_dev; a.used = used; a.capacity = capacity; a.ngroups_cap = ngroups;
  a.hq = (int)hq; a.hkv = (int)hkv; a.gq = (int)(hq / hkv);
  a.tail_mode = TAIL_NONE;
  a.sl2 = LOG2E / sqrtf((float)head_dim);
  a.out = out; a.lse = lse_out; a.ws = static_cast<float*>(workspace);
  return launch_attn(a, n_parts, workspace_bytes, static_cast<hipStream_t>(stream), "attn_decode_tok");
}

extern "C" int nkv_append_tok(const uint16_t* k_new, const uint16_t* v_new, int64_t kv_head_stride, int8_t* kq,
                              uint16_t* ksc, int8_t* vq, uint16_t* vsc, const int64_t* pos_dev, int64_t* written_dev,
                              int64_t hkv, int64_t head_dim, int64_t capacity, void* stream) {
  set_error("");
  if (head_dim != D) return fail(NKV_ERR_UNSUPPORTED, "head_dim %lld: the HIP kernels are built for head_dim 128", (long long)head_dim);
  if (hkv <= 0) return fail(NKV_ERR_INVALID, "append_tok: bad sizes");
  if (int rc = check_tok_cache("append_tok", capacity, kq, ksc, vq, vsc)) return rc;
  if (!k_new || !v_new || !pos_dev || !written_dev) return fail(NKV_ERR_INVALID, "append_tok: null pointer argument");
  if (!al16(k_new) || !al16(v_new) || kv_head_stride % 8) return fail(NKV_ERR_UNSUPPORTED, "append_tok: buffers must be 16-byte aligned");
  AttnArgs a{};
  a.k_new = k_new; a.v_new = v_new; a.kv_hs = kv_head_stride;
  a.kq = reinterpret_cast<uint8_t*>(kq); a.vq = reinterpret_cast<uint8_t*>(vq); a.ksc = ksc; a.vsc = vsc; a.tok = 1;
  a.pos_dev = pos_dev; a.written_out = written_dev; a.capacity = capacity; a.hkv = (int)hkv;
  hipLaunchKernelGGL(append_tok_kernel, dim3((unsigned)hkv), dim3(128), 0, static_cast<hipStream_t>(stream), a);
  return check_launch("append_tok");
}

static int decode_step_tok(const char* what, int launches, const uint16_t* q, const uint16_t* k_new,
                           const uint16_t* v_new, int64_t kv_head_stride, int8_t* kq, uint16_t* ksc, int8_t* vq,
                           uint16_t* vsc, const int64_t* pos_dev, int64_t* written_dev, int64_t hq, int64_t hkv,
                           int64_t head_dim, int64_t capacity, uint16_t* out, float* lse_out, void* workspace,
                           int64_t workspace_bytes, int64_t n_parts, void* stream) {
  set_error("");
  if (int rc = check_heads(hq, hkv, head_dim)) return rc;
  if (int rc = check_tok_cache("decode_step_tok", capacity, kq, ksc, vq, vsc)) return rc;
  if (!q || !k_new || !v_new || !pos_dev || !written_dev || !out || !workspace)
    return fail(NKV_ERR_INVALID, "decode_step_tok: null pointer argument");
  if (!al16(q) || !al16(k_new) || !al16(v_new) || kv_head_stride % 8 || !al16(workspace))
    return fail(NKV_ERR_UNSUPPORTED, "decode_step_tok: buffers must be 16-byte aligned");
  const int64_t ngroups = capacity / GT;
  if (n_parts <= 0) n_parts = default_parts(hkv, ngroups);
  AttnArgs a{};
  a.q = q; a.k_new = k_new; a.v_new = v_new; a.kv_hs = kv_head_stride;
  a.kq = reinterpret_cast<uint8_t*>(kq); a.vq = reinterpret_cast<uint8_t*>(vq); a.ksc = ksc; a.vsc = vsc; a.tok = 1;
  a.pos_dev = pos_dev; a.written_out = written_dev;
  a.capacity = capacity; a.ngroups_cap = ngroups; a.tail_slots = GT;
  a.hq = (int)hq; a.hkv = (int)hkv; a.gq = (int)(hq / hkv);
  a.tail_mode = TAIL_FUSED;
  a.sl2 = LOG2E / sqrtf((float)head_dim);
  a.out = out; a.lse = lse_out; a.ws = static_cast<float*>(workspace);
  return launch_attn(a, n_parts, workspace_bytes, static_cast<hipStream_t>(stream), what, launches, true);
}

#define NKV_STEP_TOK_PARAMS                                                                                      \
  const uint16_t *q, const uint16_t *k_new, const uint16_t *v_new, int64_t kv_head_stride, int8_t *kq,          \
      uint16_t *ksc, int8_t *vq, uint16_t *vsc, const int64_t *pos_dev, int64_t *written_dev, int64_t hq,        \
      int64_t hkv, int64_t head_dim, int64_t capacity, uint16_t *out, float *lse_out, void *workspace,          \
      int64_t workspace_bytes, int64_t n_parts, void *stream
#define NKV_STEP_TOK_ARGS                                                                                        \
  q, k_new, v_new, kv_head_stride, kq, ksc, vq, vsc, pos_dev, written_dev, hq, hkv, head_dim, capacity, out,   \
      lse_out, workspace, workspace_bytes, n_parts, stream

extern "C" int nkv_decode_step_tok(NKV_STEP_TOK_PARAMS) {
  return decode_step_tok("decode_step_tok", LAUNCH_PREFIX | LAUNCH_TAIL, NKV_STEP_TOK_ARGS);
}
extern "C" int nkv_decode_step_partials_tok(NKV_STEP_TOK_PARAMS) {
  return decode_step_tok("decode_step_partials_tok", LAUNCH_PREFIX, NKV_STEP_TOK_ARGS);
}
extern "C" int nkv_decode_step_combine_tok(NKV_STEP_TOK_PARAMS) {
  return decode_step_tok("decode_step_combine_tok", LAUNCH_TAIL, NKV_STEP_TOK_ARGS);
}

// ---------------------------------------------------------------- paged batch (int8t64)

extern "C" int64_t nkv_paged_workspace_bytes(int64_t hkv, int64_t hq, int64_t total_parts) {
  if (hkv <= 0 || hq <= 0 || total_parts <= 0 || hq % hkv) return 0;
  // per KV head total_parts prefix partial slots and a ring slot per sequence (nseq <= total_parts)
  return 2 * hkv * total_parts * part_floats(hq, hkv) * (int64_t)sizeof(float) + ctr_bytes(hkv * total_parts);
}

// (`rings` is NULL for the per-token symmetric format, which keeps none)
static int paged_args(const char* what, AttnArgs& a, const uint8_t* pages, const int32_t* page_table,
                      int64_t table_stride, int64_t num_pages, const uint16_t* rings, const int64_t* pos_dev,
                      int64_t nseq, int64_t hkv, int64_t head_dim, bool tok = false) {
  if (head_dim != D) return fail(NKV_ERR_UNSUPPORTED, "head_dim %lld: the HIP kernels are built for head_dim 128", (long long)head_dim);
  if (num_pages <= 0 || num_pages > (int64_t(1) << 31))
    return fail(NKV_ERR_INVALID, "%s: num_pages %lld", what, (long long)num_pages);
  if (nseq <= 0 || nseq > 32767 || hkv <= 0 || table_stride <= 0)
    return fail(NKV_ERR_INVALID, "%s: bad sizes nseq=%lld hkv=%lld table_stride=%lld", what, (long long)nseq,
                (long long)hkv, (long long)table_stride);
  if (!pages || !page_table || (!tok && !rings) || !pos_dev) return fail(NKV_ERR_INVALID, "%s: null pointer argument", what);
  if (!al16(pages) || (!tok && !al16(rings))) return fail(NKV_ERR_UNSUPPORTED, "%s: buffers must be 16-byte aligned", what);
  a.pages = const_cast<uint8_t*>(pages);
  a.table = page_table;
  a.table_stride = table_stride;
  a.num_pages = num_pages;
  a.rings = const_cast<uint16_t*>(rings);
  a.pos_dev = pos_dev;
  a.nseq = (int)nseq;
  a.hkv = (int)hkv;
  a.tail_mode = TAIL_FUSED;
  a.tail_slots = GT;
  a.tok = tok ? 1 : 0;
  return NKV_OK;
}

extern "C" int nkv_paged_append_t64(const uint16_t* k_new, const uint16_t* v_new, int64_t kv_seq_stride,
                                    int64_t kv_head_stride, uint8_t* pages, const int32_t* page_table,
                                    int64_t table_stride, int64_t num_pages, uint16_t* rings, const int64_t* pos_dev,
                                    int64_t nseq, int64_t hkv, int64_t head_dim, void* stream) {
  set_error("");
  AttnArgs a{};
  if (int rc = paged_args("paged_append_t64", a, pages, page_table, table_stride, num_pages, rings, pos_dev, nseq, hkv,
                          head_dim))
    return rc;
  if (!k_new || !v_new) return fail(NKV_ERR_INVALID, "paged_append_t64: null pointer argument");
  if (!al16(k_new) || !al16(v_new) || kv_head_stride % 8 || kv_seq_stride % 8)
    return fail(NKV_ERR_UNSUPPORTED, "paged_append_t64: k_new / v_new must be 16-byte aligned");
  a.k_new = k_new; a.v_new = v_new; a.kv_hs = kv_head_stride; a.kv_ss = kv_seq_stride;
  hipLaunchKernelGGL(append_paged_kernel, dim3((unsigned)(nseq * hkv * WIDE_UNITS)), dim3(THREADS), 0,
                     static_cast<hipStream_t>(stream), a);
  return check_launch("paged_append_t64");
}

// The paged prefix launch with its fused tails. int8t64 (`tok` false): the step's token is
// already in its sequence's ring (nkv_paged_append_t64 ran before), k_new / v_new are unused.
// Per-token symmetric (`tok`): the launch appends k_new / v_new itself and attends them as the tail.
static int paged_attn(const char* what, const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                      int64_t kv_seq_stride, int64_t kv_head_stride, const uint8_t* pages, const int32_t* page_table,
                      int64_t table_stride, int64_t num_pages, const uint16_t* rings, const int64_t* pos_dev,
                      int64_t nseq, int64_t hq,
                      int64_t hkv, int64_t head_dim, const int32_t* wg_map, const int32_t* seq_parts,
                      int64_t total_parts, uint16_t* out, float* lse_out, void* workspace, int64_t workspace_bytes,
                      void* stream, bool tok = false, bool append = false) {
  set_error("");
  if (int rc = check_heads(hq, hkv, head_dim)) return rc;
  AttnArgs a{};
  if (int rc = paged_args(what, a, pages, page_table, table_stride, num_pages, rings, pos_dev, nseq, hkv, head_dim, tok))
    return rc;
  if (tok || append) {
    if (!k_new || !v_new) return fail(NKV_ERR_INVALID, "%s: null pointer argument", what);
    if (!al16(k_new) || !al16(v_new) || kv_head_stride % 8 || kv_seq_stride % 8)
      return fail(NKV_ERR_UNSUPPORTED, "%s: k_new / v_new must be 16-byte aligned", what);
    a.k_new = k_new; a.v_new = v_new; a.kv_hs = kv_head_stride; a.kv_ss = kv_seq_stride;
  }
  if (!q || !wg_map || !seq_parts || !out || !workspace) return fail(NKV_ERR_INVALID, "%s: null pointer argument", what);
  if (!al16(q) || !al16(workspace)) return fail(NKV_ERR_UNSUPPORTED, "%s: buffers must be 16-byte aligned", what);
  if (total_parts < nseq || total_parts > 65535)
    return fail(NKV_ERR_INVALID, "%s: total_parts %lld outside [nseq, 65535]", what, (long long)total_parts);
  const int64_t need = nkv_paged_workspace_bytes(hkv, hq, total_parts);
  if (workspace_bytes < need)
    return fail(NKV_ERR_INVALID, "%s: workspace of %lld bytes, need %lld", what, (long long)workspace_bytes, (long long)need);
  a.q = q; a.hq = (int)hq; a.gq = (int)(hq / hkv);
  a.wg_map = wg_map; a.seq_parts = seq_parts; a.total_parts = (int)total_parts;
  a.sl2 = LOG2E / sqrtf((float)head_dim);
  a.out = out; a.lse = lse_out; a.ws = static_cast<float*>(workspace);
  // one launch: the last prefix workgroup of each (sequence, KV head) runs its tail
  a.inline_tail = 1;
  a.tail_append = append ? 1 : 0;
  a.tail_ctr_end = reinterpret_cast<int*>(static_cast<char*>(workspace) + (workspace_bytes & ~int64_t(3)));
  l2_args(a);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (tok) hipLaunchKernelGGL(attn_prefix_kernel<PAGED_TOK>, dim3((unsigned)(hkv * total_parts)), dim3(THREADS), 0, s, a);
  else hipLaunchKernelGGL(attn_prefix_kernel<PAGED_T64>, dim3((unsigned)(hkv * total_parts)), dim3(THREADS), 0, s, a);
  return check_launch(what);
}

extern "C" int nkv_paged_attn_decode_t64(const uint16_t* q, const uint8_t* pages, const int32_t* page_table,
                                         int64_t table_stride, int64_t num_pages, const uint16_t* rings,
                                         const int64_t* pos_dev, int64_t nseq, int64_t hq, int64_t hkv,
                                         int64_t head_dim, const int32_t* wg_map, const int32_t* seq_parts,
                                         int64_t total_parts, uint16_t* out, float* lse_out, void* workspace,
                                         int64_t workspace_bytes, void* stream) {
  return paged_attn("paged_attn_decode_t64", q, nullptr, nullptr, 0, 0, pages, page_table, table_stride, num_pages,
                    rings, pos_dev, nseq, hq, hkv, head_dim, wg_map, seq_parts, total_parts, out, lse_out, workspace,
                    workspace_bytes, stream);
}

extern "C" int nkv_paged_decode_step_t64(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                                         int64_t kv_seq_stride, int64_t kv_head_stride, uint8_t* pages,
                                         const int32_t* page_table, int64_t table_stride, int64_t num_pages,
                                         uint16_t* rings, const int64_t* pos_dev, int64_t nseq, int64_t hq,
                                         int64_t hkv, int64_t head_dim, const int32_t* wg_map,
                                         const int32_t* seq_parts, int64_t total_parts, uint16_t* out, float* lse_out,
                                         void* workspace, int64_t workspace_bytes, void* stream) {
  // one launch: the tail of each (sequence, KV head) appends the new token from k_new / v_new
  // (nothing else in the launch reads the ring slot or the group it writes)
  return paged_attn("paged_decode_step_t64", q, k_new, v_new, kv_seq_stride, kv_head_stride, pages, page_table,
                    table_stride, num_pages, rings, pos_dev, nseq, hq, hkv, head_dim, wg_map, seq_parts, total_parts,
                    out, lse_out, workspace, workspace_bytes, stream, false, true);
}

extern "C" int nkv_paged_decode_step_tok(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                                         int64_t kv_seq_stride, int64_t kv_head_stride, uint8_t* pages,
                                         const int32_t* page_table, int64_t table_stride, int64_t num_pages,
                                         const int64_t* pos_dev, int64_t nseq, int64_t hq, int64_t hkv,
                                         int64_t head_dim, const int32_t* wg_map, const int32_t* seq_parts,
                                         int64_t total_parts, uint16_t* out, float* lse_out, void* workspace,
                                         int64_t workspace_bytes, void* stream) {
  return paged_attn("paged_decode_step_tok", q, k_new, v_new, kv_seq_stride, kv_head_stride, pages, page_table,
                    table_stride, num_pages, nullptr, pos_dev, nseq, hq, hkv, head_dim, wg_map, seq_parts, total_parts,
                    out, lse_out, workspace, workspace_bytes, stream, true);
}

// ---------------------------------------------------------------- chunked prefill

// Splits of the cache's groups: enough workgroups for every resident slot (256 CUs x
// PF_WG_PER_CU), at least one group per split.
extern "C" int64_t nkv_prefill_default_splits(int64_t hkv, int64_t hq, int64_t m, int64_t used) {
  if (hkv <= 0 || hq <= 0 || m <= 0 || used < 0 || hq % hkv) return 0;
  const int64_t tiles = cdiv(m * (hq / hkv), PF_ROWS);
  return std::max<int64_t>(1, std::min<int64_t>(cdiv(256 * PF_WG_PER_CU, hkv * tiles), std::max<int64_t>(1, used / GT)));
}

extern "C" int64_t nkv_prefill_workspace_bytes(int64_t hkv, int64_t hq, int64_t m, int64_t splits) {
  if (hkv <= 0 || hq <= 0 || m <= 0 || splits <= 0 || hq % hkv) return 0;
  return splits * hq * m * PF_PART * (int64_t)sizeof(float);
}

static int prefill_attn(const char* what, const uint16_t* q, int64_t m, const uint16_t* k16, const uint16_t* v16,
                        int64_t m_kv, int64_t kv_head_stride, const uint8_t* kq, const uint16_t* kmn,
                        const uint16_t* kst, const uint8_t* vq, const uint16_t* vmn, const uint16_t* vst,
                        int64_t capacity, int64_t used, int64_t hq, int64_t hkv, int64_t head_dim, uint16_t* out,
                        void* workspace, int64_t workspace_bytes, int64_t splits, void* stream) {
  set_error("");
  if (int rc = check_heads(hq, hkv, head_dim)) return rc;
  if (m <= 0 || m > (1 << 20)) return fail(NKV_ERR_INVALID, "%s: query length %lld", what, (long long)m);
  if (m_kv < m || m_kv > (1 << 24))
    return fail(NKV_ERR_INVALID, "%s: %lld fp16 tokens for %lld queries", what, (long long)m_kv, (long long)m);
  if (kv_head_stride < m_kv * D || kv_head_stride % 8)
    return fail(NKV_ERR_INVALID, "%s: fp16 K/V head stride %lld (need >= %lld, a multiple of 8)", what,
                (long long)kv_head_stride, (long long)(m_kv * D));
  if (used < 0 || used % GT || used > capacity)
    return fail(NKV_ERR_INVALID, "%s: used=%lld must be a multiple of 64 within the capacity %lld", what,
                (long long)used, (long long)capacity);
  if (!q || !k16 || !v16 || !out || !workspace || (used > 0 && (!kq || !kmn || !kst || !vq || !vmn || !vst)))
    return fail(NKV_ERR_INVALID, "%s: null pointer argument", what);
  if (!al16(q) || !al16(k16) || !al16(v16) || !al16(out) || !al16(workspace) ||
      (used > 0 && (!al16(kq) || !al16(vq) || !al16(kmn) || !al16(kst) || !al16(vmn) || !al16(vst))))
    return fail(NKV_ERR_UNSUPPORTED, "%s: buffers must be 16-byte aligned", what);
  const int64_t gq = hq / hkv, rows_h = m * gq, tiles = cdiv(rows_h, PF_ROWS);
  if (splits <= 0) splits = nkv_prefill_default_splits(hkv, hq, m, used);
  if (workspace_bytes < nkv_prefill_workspace_bytes(hkv, hq, m, splits))
    return fail(NKV_ERR_INVALID, "%s: workspace of %lld bytes, need %lld", what, (long long)workspace_bytes,
                (long long)nkv_prefill_workspace_bytes(hkv, hq, m, splits));
  PrefillArgs a{};
  a.q = q; a.kc = k16; a.vc = v16;
  a.kq = kq; a.kmn = kmn; a.kst = kst; a.vq = vq; a.vmn = vmn; a.vst = vst;
  a.capacity = capacity; a.ngroups_cap = cdiv(capacity, GT); a.U = used;
  a.M = (int)m; a.hq = (int)hq; a.hkv = (int)hkv; a.gq = (int)gq; a.splits = (int)splits; a.tiles = (int)tiles;
  a.Mk = (int)m_kv; a.qoff = (int)(m_kv - m); a.kc_hs = kv_head_stride;
  a.sl2 = LOG2E / sqrtf((float)head_dim);
  a.ws = static_cast<float*>(workspace); a.out = out;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(prefill_chunk_kernel, dim3((unsigned)(hkv * tiles * splits)), dim3(PF_THREADS), 0, s, a);
  if (int rc = check_launch(what)) return rc;
  const int64_t items = hq * m * (D / 4);
  hipLaunchKernelGGL(prefill_combine_kernel, dim3((unsigned)cdiv(items, 256)), dim3(256), 0, s, a);
  return check_launch(what);
}

extern "C" int nkv_prefill_attn_t64(const uint16_t* q, const uint16_t* k_chunk, const uint16_t* v_chunk, int64_t m,
                                    const uint8_t* kq, const uint16_t* kmn, const uint16_t* kst, const uint8_t* vq,
                                    const uint16_t* vmn, const uint16_t* vst, int64_t capacity, int64_t used,
                                    int64_t hq, int64_t hkv, int64_t head_dim, uint16_t* out, void* workspace,
                                    int64_t workspace_bytes, int64_t splits, void* stream) {
  return prefill_attn("prefill_attn_t64", q, m, k_chunk, v_chunk, m, m * D, kq, kmn, kst, vq, vmn, vst, capacity,
                      used, hq, hkv, head_dim, out, workspace, workspace_bytes, splits, stream);
}

extern "C" int nkv_prefill_attn_hist_t64(const uint16_t* q, int64_t m, const uint16_t* k16, const uint16_t* v16,
                                         int64_t m_kv, int64_t kv_head_stride, const uint8_t* kq, const uint16_t* kmn,
                                         const uint16_t* kst, const uint8_t* vq, const uint16_t* vmn,
                                         const uint16_t* vst, int64_t capacity, int64_t used, int64_t hq, int64_t hkv,
                                         int64_t head_dim, uint16_t* out, void* workspace, int64_t workspace_bytes,
                                         int64_t splits, void* stream) {
  return prefill_attn("prefill_attn_hist_t64", q, m, k16, v16, m_kv, kv_head_stride, kq, kmn, kst, vq, vmn, vst,
                      capacity, used, hq, hkv, head_dim, out, workspace, workspace_bytes, splits, stream);
}

// ---- the chained decode step: every layer of one token in one launch (kernel C)

namespace {
std::mutex g_layers_mu;
int g_layers_resident[MAX_DEVICES][2];  // workgroups of attn_layers_kernel resident at once (0: not known yet)

// Workgroups of the chained kernel (int8t64 or per-token symmetric) that the current device
// holds at once: CUs x workgroups per CU from the occupancy query.
int layers_resident(bool tok, int* out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES)
    return fail(NKV_ERR_HIP, "decode_layers: no usable current device (%d)", dev);
  std::lock_guard<std::mutex> lock(g_layers_mu);
  int& r = g_layers_resident[dev][tok ? 1 : 0];
  if (!r) {
    int cus = 0, per_cu = 0;
    hipError_t e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e == hipSuccess)
      e = tok ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, attn_layers_kernel<CONTIG_TOK>, THREADS, 0)
              : hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, attn_layers_kernel<CONTIG_T64>, THREADS, 0);
    if (e != hipSuccess) return fail(NKV_ERR_HIP, "decode_layers: occupancy query: %s", hipGetErrorString(e));
    r = cus * per_cu;
  }
  *out = r;
  return NKV_OK;
}

// n_layers counters, the exit ticket, the error word, the launch counter
// n_layers counters, the exit ticket, the error word, the launch counter
int64_t layers_sync_bytes(int64_t n_layers) { return ctr_bytes(n_layers + 3); }
// each layer's output as tagged words (forwarded to the next layer's inputs)
// (and, after them, each layer's issue flags: one word per query head)
int64_t layers_fwd_bytes(int64_t hq, int64_t n_layers) {
  return n_layers * hq * D / 2 * (int64_t)sizeof(uint64_t) + n_layers * FLAG_COPIES * hq * (int64_t)sizeof(uint32_t);
}

// Streaming parts per KV head: one workgroup per 8 groups at most, and hkv (parts + 1) workgroups
// resident at once.
int64_t layers_parts(int64_t hkv, int64_t groups, int resident) {
  const int64_t fit = resident / std::max<int64_t>(1, hkv) - 1;
  return std::min<int64_t>(std::min<int64_t>(fit, WTS), std::max<int64_t>(1, cdiv(groups, 8)));
}

bool al8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }

// Whether the chained launch's waits order every read of its inputs (the layer table in host
// memory). Head h of layer l reads q rows h gq .. h gq + gq - 1 and the k_new / v_new rows at
// h kv_head_stride. A row that lies in layer j's output must lie within the rows of one head w
// (the rows w's merger writes), and then:
//  - w == h: head h's own chain orders it (layer j before layer l, or layer l's reads before its
//    merge, or the reads of layer l before layer j > l is merged);
//  - j < l: read after layer l - 1's all-head counter (such a row is never forwarded);
//  - j == l: refused, head w writes the row while head h may still have to read it;
//  - j > l: ordered only when every layer waits for every head (dep_all: head w starts layer j
//    after every head has finished layer j - 1 >= l); refused otherwise.
template <class E>
int check_chain_inputs(const E* t, int64_t n_layers, int64_t hq, int64_t hkv, int64_t kv_hs, bool dep_all,
                       const char* what) {
  const int64_t gq = hq / hkv, n = hq * D;
  for (int64_t l = 0; l < n_layers; ++l) {
    for (int64_t h = 0; h < hkv; ++h) {
      for (int64_t r = 0; r < gq + 2; ++r) {
        const char* nm = r < gq ? "q" : r == gq ? "k_new" : "v_new";
        const uint16_t* p = r < gq ? t[l].q + (h * gq + r) * D : (r == gq ? t[l].k_new : t[l].v_new) + h * kv_hs;
        const uintptr_t a0 = reinterpret_cast<uintptr_t>(p), a1 = a0 + 2 * D;
        for (int64_t j = 0; j < n_layers; ++j) {
          const uintptr_t o0 = reinterpret_cast<uintptr_t>(t[j].out), o1 = o0 + 2 * n;
          if (a1 <= o0 || a0 >= o1) continue;
          const int64_t w0 = a0 >= o0 ? (int64_t)(a0 - o0) / (2 * gq * D) : -1;
          const int64_t w1 = a1 <= o1 ? (int64_t)(a1 - 1 - o0) / (2 * gq * D) : -1;
          if (w0 < 0 || w1 != w0)
            return fail(NKV_ERR_INVALID, "%s: layer %lld head %lld: a %s row straddles the rows of layer %lld's output "
                        "that different heads write", what, (long long)l, (long long)h, nm, (long long)j);
          if (w0 == h || j < l) continue;
          if (j == l)
            return fail(NKV_ERR_INVALID, "%s: layer %lld head %lld reads its %s row from the same layer's output of "
                        "KV head %lld, which may already be overwritten", what, (long long)l, (long long)h, nm,
                        (long long)w0);
          if (!dep_all)
            return fail(NKV_ERR_INVALID, "%s: layer %lld head %lld reads its %s row from layer %lld's output of KV "
                        "head %lld, which that head's chain may overwrite first; only the all-head dependency "
                        "orders this", what, (long long)l, (long long)h, nm, (long long)j, (long long)w0);
        }
      }
    }
  }
  return NKV_OK;
}

// Launch of attn_layers_kernel: the checks common to both formats, the grid, the launch.
int launch_layers(AttnArgs& a, bool tok, const void* layers_dev, int64_t n_layers, int64_t n_parts,
                  int64_t workspace_bytes, hipStream_t s, const char* what) {
  if (n_layers <= 0 || n_layers > (1 << 20)) return fail(NKV_ERR_INVALID, "%s: n_layers %lld outside [1, 2^20]", what, (long long)n_layers);
  if (!layers_dev || !al8(layers_dev)) return fail(NKV_ERR_INVALID, "%s: the layer table must be a non-null, 8-byte aligned device array", what);
  if (a.capacity > (int64_t(1) << 24)) return fail(NKV_ERR_UNSUPPORTED, "%s: capacity %lld exceeds 16M tokens", what, (long long)a.capacity);
  int resident = 0;
  if (int rc = layers_resident(tok, &resident)) return rc;
  if (n_parts <= 0) n_parts = layers_parts(a.hkv, a.ngroups_cap, resident);
  if (n_parts < 1 || n_parts > WTS)
    return fail(NKV_ERR_UNSUPPORTED, "%s: %lld streaming parts per KV head (1..%d)", what, (long long)n_parts, WTS);
  const int64_t grid = (int64_t)a.hkv * (n_parts + 1);
  if (grid > resident)
    return fail(NKV_ERR_UNSUPPORTED,
                "%s: %lld workgroups (%d KV heads x (%lld parts + 1)) exceed the %d this device holds at once",
                what, (long long)grid, a.hkv, (long long)n_parts, resident);
  const int64_t part_bytes = n_layers * a.hkv * n_parts * part_floats(a.hq, a.hkv) * (int64_t)sizeof(float);
  const int64_t need = part_bytes + layers_fwd_bytes(a.hq, n_layers) + layers_sync_bytes(n_layers);
  if (!a.ws || !al16(a.ws)) return fail(NKV_ERR_INVALID, "%s: the workspace must be a non-null, 16-byte aligned buffer", what);
  if (workspace_bytes < need)
    return fail(NKV_ERR_INVALID, "%s: workspace of %lld bytes, need %lld", what, (long long)workspace_bytes, (long long)need);
  if (a.dep_all && a.hq > 64) return fail(NKV_ERR_UNSUPPORTED, "%s: the all-head dependency polls at most 64 query heads' flags", what);
  a.n_parts = (int)n_parts;
  a.n_layers = (int)n_layers;
  a.tail_ctr_end = reinterpret_cast<int*>(reinterpret_cast<char*>(a.ws) + (workspace_bytes & ~int64_t(3)));
  a.fwd_out = reinterpret_cast<uint64_t*>(reinterpret_cast<char*>(a.ws) + part_bytes);
  a.flags_base = reinterpret_cast<uint32_t*>(a.fwd_out + n_layers * a.hq * D / 2);
  l2_args(a);
  if (tok) hipLaunchKernelGGL(attn_layers_kernel<CONTIG_TOK>, dim3((unsigned)grid), dim3(THREADS), 0, s, a, layers_dev, (int)n_layers);
  else hipLaunchKernelGGL(attn_layers_kernel<CONTIG_T64>, dim3((unsigned)grid), dim3(THREADS), 0, s, a, layers_dev, (int)n_layers);
  return check_launch(what);
}
}  // namespace

extern "C" int64_t nkv_layers_workspace_bytes(int64_t hkv, int64_t hq, int64_t n_parts, int64_t n_layers) {
  if (hkv <= 0 || hq <= 0 || hq % hkv || n_parts <= 0 || n_layers <= 0) return 0;
  return n_layers * hkv * n_parts * part_floats(hq, hkv) * (int64_t)sizeof(float) + layers_fwd_bytes(hq, n_layers) +
         layers_sync_bytes(n_layers);
}

extern "C" int64_t nkv_layers_default_parts(int64_t hkv, int64_t capacity, int tok) {
  set_error("");
  int resident = 0;
  if (hkv <= 0 || capacity <= 0 || layers_resident(tok != 0, &resident) != NKV_OK) return 0;
  const int64_t parts = layers_parts(hkv, cdiv(capacity, GT), resident);
  return parts >= 1 && hkv * (parts + 1) <= resident ? parts : 0;
}

// The input rules alone (host only; the chained launches run them too when given layers_host).
template <class E>
int chain_check(const char* what, const E* layers_host, int64_t n_layers, int64_t kv_head_stride, int64_t hq,
                int64_t hkv, int dep) {
  set_error("");
  if (int rc = check_heads(hq, hkv, D)) return rc;
  if (!layers_host) return fail(NKV_ERR_INVALID, "%s: null layer table", what);
  if (n_layers <= 0 || n_layers > (1 << 20)) return fail(NKV_ERR_INVALID, "%s: n_layers %lld outside [1, 2^20]", what, (long long)n_layers);
  if (dep != NKV_DEP_HEAD && dep != NKV_DEP_ALL) return fail(NKV_ERR_INVALID, "%s: dep %d is not NKV_DEP_HEAD or NKV_DEP_ALL", what, dep);
  return check_chain_inputs(layers_host, n_layers, hq, hkv, kv_head_stride, dep == NKV_DEP_ALL, what);
}

extern "C" int nkv_decode_layers_check_t64(const nkv_layer_t64* layers_host, int64_t n_layers, int64_t kv_head_stride,
                                           int64_t hq, int64_t hkv, int dep) {
  return chain_check("decode_layers_check_t64", layers_host, n_layers, kv_head_stride, hq, hkv, dep);
}

extern "C" int nkv_decode_layers_check_tok(const nkv_layer_tok* layers_host, int64_t n_layers, int64_t kv_head_stride,
                                           int64_t hq, int64_t hkv, int dep) {
  return chain_check("decode_layers_check_tok", layers_host, n_layers, kv_head_stride, hq, hkv, dep);
}

extern "C" int nkv_decode_layers_t64(const nkv_layer_t64* layers_dev, const nkv_layer_t64* layers_host,
                                     int64_t n_layers, int64_t kv_head_stride, const int64_t* pos_dev,
                                     const int64_t* first_dev, int64_t* written_dev, int64_t* qlen_dev,
                                     int64_t* pg_dev, int64_t hq, int64_t hkv, int64_t head_dim, int64_t capacity,
                                     void* workspace, int64_t workspace_bytes, int64_t n_parts, int dep,
                                     void* stream) {
  const char* what = "decode_layers_t64";
  set_error("");
  if (int rc = check_heads(hq, hkv, head_dim)) return rc;
  if (capacity <= 0) return fail(NKV_ERR_INVALID, "capacity must be positive");
  if (!pos_dev || !written_dev || !qlen_dev || !pg_dev) return fail(NKV_ERR_INVALID, "%s: null scalar pointer", what);
  if (kv_head_stride % 8) return fail(NKV_ERR_UNSUPPORTED, "%s: kv_head_stride must keep 16-byte alignment", what);
  for (int64_t l = 0; layers_host && l < n_layers; ++l) {
    const nkv_layer_t64& e = layers_host[l];
    const void* p[] = {e.q, e.k_new, e.v_new, e.kq, e.kmn, e.kst, e.vq, e.vmn, e.vst, e.tail_k, e.tail_v, e.out};
    for (const void* x : p)
      if (!x || !al16(x)) return fail(NKV_ERR_INVALID, "%s: layer %lld: null or unaligned pointer", what, (long long)l);
    if (e.lse && (reinterpret_cast<uintptr_t>(e.lse) & 3u)) return fail(NKV_ERR_INVALID, "%s: layer %lld: unaligned lse", what, (long long)l);
  }
  if (dep != NKV_DEP_HEAD && dep != NKV_DEP_ALL) return fail(NKV_ERR_INVALID, "%s: dep %d is not NKV_DEP_HEAD or NKV_DEP_ALL", what, dep);
  if (layers_host && n_layers > 0 && n_layers <= (1 << 20))
    if (int rc = check_chain_inputs(layers_host, n_layers, hq, hkv, kv_head_stride, dep == NKV_DEP_ALL, what)) return rc;
  AttnArgs a{};
  a.kv_hs = kv_head_stride;
  a.dep_all = dep == NKV_DEP_ALL;
  a.pos_dev = pos_dev; a.first_dev = first_dev;
  a.written_out = written_dev; a.qlen_out = qlen_dev; a.pg_out = pg_dev;
  a.capacity = capacity; a.ngroups_cap = cdiv(capacity, GT); a.tail_slots = GT;
  a.hq = (int)hq; a.hkv = (int)hkv; a.gq = (int)(hq / hkv);
  a.tail_mode = TAIL_FUSED;
  a.inline_tail = 1;
  a.sl2 = LOG2E / sqrtf((float)head_dim);
  a.ws = static_cast<float*>(workspace);
  return launch_layers(a, false, layers_dev, n_layers, n_parts, workspace_bytes, static_cast<hipStream_t>(stream), what);
}

extern "C" int nkv_decode_layers_tok(const nkv_layer_tok* layers_dev, const nkv_layer_tok* layers_host,
                                     int64_t n_layers, int64_t kv_head_stride, const int64_t* pos_dev,
                                     int64_t* written_dev, int64_t hq, int64_t hkv, int64_t head_dim,
                                     int64_t capacity, void* workspace, int64_t workspace_bytes, int64_t n_parts,
                                     int dep, void* stream) {
  const char* what = "decode_layers_tok";
  set_error("");
  if (int rc = check_heads(hq, hkv, head_dim)) return rc;
  if (capacity <= 0 || capacity % GT) return fail(NKV_ERR_INVALID, "%s: capacity %lld must be a positive multiple of 64", what, (long long)capacity);
  if (!pos_dev || !written_dev) return fail(NKV_ERR_INVALID, "%s: null scalar pointer", what);
  if (kv_head_stride % 8) return fail(NKV_ERR_UNSUPPORTED, "%s: kv_head_stride must keep 16-byte alignment", what);
  for (int64_t l = 0; layers_host && l < n_layers; ++l) {
    const nkv_layer_tok& e = layers_host[l];
    const void* p[] = {e.q, e.k_new, e.v_new, e.kq, e.ksc, e.vq, e.vsc, e.out};
    for (const void* x : p)
      if (!x || !al16(x)) return fail(NKV_ERR_INVALID, "%s: layer %lld: null or unaligned pointer", what, (long long)l);
    if (e.lse && (reinterpret_cast<uintptr_t>(e.lse) & 3u)) return fail(NKV_ERR_INVALID, "%s: layer %lld: unaligned lse", what, (long long)l);
  }
  if (dep != NKV_DEP_HEAD && dep != NKV_DEP_ALL) return fail(NKV_ERR_INVALID, "%s: dep %d is not NKV_DEP_HEAD or NKV_DEP_ALL", what, dep);
  if (layers_host && n_layers > 0 && n_layers <= (1 << 20))
    if (int rc = check_chain_inputs(layers_host, n_layers, hq, hkv, kv_head_stride, dep == NKV_DEP_ALL, what)) return rc;
  AttnArgs a{};
  a.kv_hs = kv_head_stride;
  a.dep_all = dep == NKV_DEP_ALL;
  a.tok = 1;
  a.pos_dev = pos_dev; a.written_out = written_dev;
  a.capacity = capacity; a.ngroups_cap = capacity / GT; a.tail_slots = GT;
  a.hq = (int)hq; a.hkv = (int)hkv; a.gq = (int)(hq / hkv);
  a.tail_mode = TAIL_FUSED;
  a.inline_tail = 1;
  a.sl2 = LOG2E / sqrtf((float)head_dim);
  a.ws = static_cast<float*>(workspace);
  return launch_layers(a, true, layers_dev, n_layers, n_parts, workspace_bytes, static_cast<hipStream_t>(stream), what);
}

extern "C" int nkv_read_bw_lds(const void* src, int64_t nbytes, uint32_t* sink, int64_t blocks, void* stream) {
  set_error("");
  if (!src || !al16(src) || nbytes <= 0 || nbytes % RB_CHUNK)
    return fail(NKV_ERR_INVALID, "read_bw_lds: nbytes must be a positive multiple of %d and src 16-byte aligned", RB_CHUNK);
  if (!sink || blocks <= 0 || blocks > (1 << 20)) return fail(NKV_ERR_INVALID, "read_bw_lds: blocks must be in [1, 2^20] with a sink");
  hipLaunchKernelGGL(read_lds_kernel, dim3((unsigned)blocks), dim3(THREADS), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint8_t*>(src), nbytes / RB_CHUNK, sink);
  return check_launch("read_bw_lds");
}
