/*
 * nova_kv.h — C ABI of the MI355X (gfx950) int8 KV-cache decode path.
 *
 * Every entry point takes raw device pointers, element counts/strides and a
 * hipStream_t passed as `void*` (the caller's current stream; pass the stream
 * that torch is capturing on to record the launch into a hipGraph). Nothing
 * here allocates device memory, synchronizes the device or reads device memory
 * on the host, so every call is safe inside stream capture (except the two
 * nkv_l2_handover calls, which are made once, outside capture). Scratch memory
 * (`workspace`) is owned by the caller, except for nkv_decode_step_static_t64, whose
 * scratch is a fixed array the library holds on each GPU.
 *
 * Return value: NKV_OK, or a NKV_ERR_* code; `nkv_last_error()` then returns
 * a message for the calling thread. Launches are asynchronous: a fault inside
 * a kernel surfaces at the next synchronizing HIP call, as for any HIP kernel.
 *
 * Tensor layouts follow the reference (batch 1): codes `[H_kv, L, D]` uint8,
 * rulers `[H_kv, ceil(L/64), D]` fp16, ring `[H_kv, 64, D]` fp16, device
 * scalars are single int64 values. fp16 buffers are typed `uint16_t`.
 *
 * Each declaration names the reference interface it replaces (file:line of
 * captain-wangrun-cn/Nova).
 */
#ifndef NOVA_KV_H
#define NOVA_KV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NKV_ABI_VERSION 11

#define NKV_OK 0
#define NKV_ERR_INVALID 1     /* argument outside what the reference accepts */
#define NKV_ERR_UNSUPPORTED 2 /* accepted by the reference, not built for this GPU path */
#define NKV_ERR_HIP 3         /* HIP launch/runtime error */

#define NKV_F16 0
#define NKV_BF16 1
#define NKV_F32 2

#define NKV_AXIS_CHANNEL 0
#define NKV_AXIS_TOKEN 1

/* ABI version of the loaded library (NKV_ABI_VERSION at build time). */
int nkv_abi_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char* nkv_last_error(void);

/*
 * Asymmetric int8 quantization, one (min, step) ruler per group.
 * Replaces `kvquant.quantize_int8(x, group_size, axis)` (src/nova/kvquant.py:118-149).
 *
 * x: `rows` slabs of `[n, dim]` (dim contiguous, token stride = dim), slab
 * stride `x_row_stride` elements; dtype NKV_F16 / NKV_BF16 / NKV_F32.
 * axis NKV_AXIS_TOKEN: groups of `group` tokens per channel (0 = all n),
 *   rulers `[rows, ceil(n/group), dim]`, the last group ruled by its real
 *   tokens (the reference's replicate pad, kvquant.py:138-143).
 * axis NKV_AXIS_CHANNEL: groups of `group` channels per token (0 = all dim),
 *   rulers `[rows, n, dim/group]`.
 * codes: uint8 slabs of `[n, dim]`, slab stride `codes_row_stride`.
 * mins/steps: fp16 slabs, slab stride `scale_row_stride`.
 * step = max((max-min)/255, 1e-8) in fp32, code = clamp(rint((x-min)/step), 0, 255),
 * min/step stored as fp16 (round to nearest even) — bit-exact with the reference.
 */
int nkv_quantize_int8(const void* x, int x_dtype, int64_t x_row_stride, int64_t rows, int64_t n,
                      int64_t dim, int64_t group, int axis, uint8_t* codes,
                      int64_t codes_row_stride, uint16_t* mins, uint16_t* steps,
                      int64_t scale_row_stride, void* stream);

/*
 * Inverse of nkv_quantize_int8: out = round(fp32(code)*fp32(step) + fp32(min)) in
 * `out_dtype` (NKV_F16 / NKV_BF16 / NKV_F32).
 * Replaces `kvquant.dequantize_int8` (src/nova/kvquant.py:152-176).
 * Same slab/stride conventions as nkv_quantize_int8; `out` slab stride is
 * `out_row_stride` elements.
 */
int nkv_dequantize_int8(const uint8_t* codes, int64_t codes_row_stride, const uint16_t* mins,
                        const uint16_t* steps, int64_t scale_row_stride, int64_t rows, int64_t n,
                        int64_t dim, int64_t group, int axis, void* out, int out_dtype,
                        int64_t out_row_stride, void* stream);

/*
 * Split-K int8 decode attention for one layer, `int8t64` cache, head_dim 128.
 * Replaces `kvattn.int8_attn_decode` (src/nova/kvattn.py:281-427), i.e. the
 * Triton `_int8_attn_partial_kernel` + `_int8_attn_combine_kernel`
 * (kvattn.py:110-253), and — when `tail_k` is given — `tail_attend` plus the
 * log-sum-exp merge of `KVInt8Cache.attend` (kvattn.py:447-482, 835-862).
 * Two launches on `stream`: the prefix kernel (hkv * n_parts workgroups, one
 * partial each into `workspace`), then the tail kernel (hkv workgroups: ring,
 * merge, out / lse).
 *
 * q [hq, 128] fp16 (RoPE applied); hq % hkv == 0, hq/hkv <= 16.
 * Prefix: tokens [0, used) of the int8 cache, limited to `prefix_groups`
 *   whole rulers; the values come from `used_dev` / `prefix_groups_dev`
 *   (device int64) when non-NULL, else from `used` / `prefix_groups`.
 * Tail (optional, tail_k != NULL): the 64-slot fp16 ring; slot i holds
 *   position p = u - ((u - i) mod 64), u = *written_dev - 1, and takes part iff
 *   used <= p <= u and p >= *first_dev.
 * out [hq, 128] fp16 = softmax(q k^T / sqrt(128)) v over prefix U tail.
 * lse_out [hq] fp32 (may be NULL) = log-sum-exp of the scaled scores; an empty
 *   key set gives out 0 and lse -inf (kvattn.py:244-253).
 * workspace: >= nkv_attn_workspace_bytes(hkv, hq, n_parts) bytes of device memory,
 *   16-byte aligned (any contents).
 * n_parts: prefix work units per KV head (fixed for a captured graph); 0 picks one
 *   from `capacity` (or from `used` when no device scalar is given).
 * Calls that overlap on one GPU must not share `workspace`.
 */
int nkv_attn_decode_t64(const uint16_t* q, const uint8_t* kq, const uint16_t* kmn,
                        const uint16_t* kst, const uint8_t* vq, const uint16_t* vmn,
                        const uint16_t* vst, int64_t hq, int64_t hkv, int64_t head_dim,
                        int64_t capacity, int64_t used, int64_t prefix_groups,
                        const int64_t* used_dev, const int64_t* prefix_groups_dev,
                        const uint16_t* tail_k, const uint16_t* tail_v,
                        const int64_t* written_dev, const int64_t* first_dev, uint16_t* out,
                        float* lse_out, void* workspace, int64_t workspace_bytes,
                        int64_t n_parts, void* stream);

/* Bytes of `workspace` that nkv_attn_decode_t64 / nkv_decode_step_t64 need. */
int64_t nkv_attn_workspace_bytes(int64_t hkv, int64_t hq, int64_t n_parts);

/* The n_parts value that `n_parts = 0` resolves to for `groups` rulers per head. */
int64_t nkv_attn_default_parts(int64_t hkv, int64_t groups);

/*
 * Streaming append of one decode token into the int8 cache of one layer.
 * Replaces `KVInt8Cache.update` on the decode path with `_quantize_ring` and
 * `_sync_scalars` (src/nova/kvattn.py:668-743, 699-710): writes k/v into ring
 * slot pos%64, requantizes all 64 ring slots (in slot order) into ruler group
 * pos//64, and sets written = pos+1, qlen = 64*floor(written/64), pg = qlen/64.
 * k_new/v_new: [hkv, 128] fp16 with head stride `kv_head_stride` elements.
 */
int nkv_append_t64(const uint16_t* k_new, const uint16_t* v_new, int64_t kv_head_stride,
                   uint8_t* kq, uint16_t* kmn, uint16_t* kst, uint8_t* vq, uint16_t* vmn,
                   uint16_t* vst, uint16_t* tail_k, uint16_t* tail_v, const int64_t* pos_dev,
                   int64_t* written_dev, int64_t* qlen_dev, int64_t* pg_dev, int64_t hkv,
                   int64_t head_dim, int64_t capacity, void* stream);

/*
 * One decode step of one layer: nkv_append_t64 followed by nkv_attn_decode_t64
 * over the int8 prefix and the ring, with the same cache state and scalars as the
 * two-call sequence and the same output up to float summation order. One launch: the
 * prefix kernel also performs the append (the prefix never reads the group it writes),
 * and the last of each head's workgroups to finish runs the tail (ring attention and the
 * combine; the new token's ring slot is read from k_new / v_new). Its ticket comes from
 * a completion counter per head kept in the last bytes of `workspace`: the workspace must
 * be zero-filled before its first use and serve only the decode-step entry points of one
 * configuration; every call leaves the counters at zero. Replaces the `KVInt8Cache.update` +
 * `KVInt8Cache.attend` pair that `LeanAttention.forward` issues per layer
 * (src/nova/layers.py:132-136).
 */
int nkv_decode_step_t64(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                        int64_t kv_head_stride, uint8_t* kq, uint16_t* kmn, uint16_t* kst,
                        uint8_t* vq, uint16_t* vmn, uint16_t* vst, uint16_t* tail_k,
                        uint16_t* tail_v, const int64_t* pos_dev, const int64_t* first_dev,
                        int64_t* written_dev, int64_t* qlen_dev, int64_t* pg_dev, int64_t hq,
                        int64_t hkv, int64_t head_dim, int64_t capacity, uint16_t* out,
                        float* lse_out, void* workspace, int64_t workspace_bytes,
                        int64_t n_parts, void* stream);

/*
 * nkv_decode_step_t64 as two launches in two calls, with the same arguments:
 * _partials (the prefix kernel: the append and one partial per workgroup into
 * `workspace`; `out` / `lse_out` are not written) followed by _combine (the tail kernel:
 * ring attention and the log-sum-exp combine into out / lse) on one stream equals one
 * nkv_decode_step_t64 call. They replace the reference's split of the decode attention
 * into `_int8_attn_partial_kernel` and `_int8_attn_combine_kernel`
 * (src/nova/kvattn.py:110-253), and let a caller time or schedule the two separately.
 * Between the two calls, `workspace` and the cache must not be touched.
 */
int nkv_decode_step_partials_t64(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                                 int64_t kv_head_stride, uint8_t* kq, uint16_t* kmn, uint16_t* kst,
                                 uint8_t* vq, uint16_t* vmn, uint16_t* vst, uint16_t* tail_k,
                                 uint16_t* tail_v, const int64_t* pos_dev, const int64_t* first_dev,
                                 int64_t* written_dev, int64_t* qlen_dev, int64_t* pg_dev, int64_t hq,
                                 int64_t hkv, int64_t head_dim, int64_t capacity, uint16_t* out,
                                 float* lse_out, void* workspace, int64_t workspace_bytes,
                                 int64_t n_parts, void* stream);
int nkv_decode_step_combine_t64(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                                int64_t kv_head_stride, uint8_t* kq, uint16_t* kmn, uint16_t* kst,
                                uint8_t* vq, uint16_t* vmn, uint16_t* vst, uint16_t* tail_k,
                                uint16_t* tail_v, const int64_t* pos_dev, const int64_t* first_dev,
                                int64_t* written_dev, int64_t* qlen_dev, int64_t* pg_dev, int64_t hq,
                                int64_t hkv, int64_t head_dim, int64_t capacity, uint16_t* out,
                                float* lse_out, void* workspace, int64_t workspace_bytes,
                                int64_t n_parts, void* stream);

/*
 * A decoder layer's attention block for one decode token in one launch: the input RMSNorm and
 * the stacked q/k/v projection, the per-head q and k RMSNorm and the rotary embedding at
 * *pos_dev, then nkv_decode_step_t64's append and attention of the token. Replaces the
 * `q_proj` / `k_proj` / `v_proj`, `q_norm` / `k_norm`, `apply_rotary_pos_emb` and
 * `update` + `attend` sequence of `LeanAttention.forward` (src/nova/layers.py:99-137) for one
 * token, with the input norm of `LeanDecoderLayer` (src/nova/layers.py:177-218).
 *
 * x [hidden] fp16 (the residual stream), x_gamma [hidden] (its RMSNorm weight, x_eps),
 * w_qkv [(hq + 2 hkv) * 128][hidden] fp16 (q heads, then k heads, then v heads); hidden a
 * multiple of 8, at most 3072. q_gamma / k_gamma [128] fp16 (the head norms, qk_eps),
 * inv_freq [64] fp32 (the RoPE frequencies). qkv_out, when not NULL, receives the normalized
 * and rotated q and k and the v rows [(hq + 2 hkv) * 128] fp16. The cache, scalar, output and
 * n_parts arguments are nkv_decode_step_t64's; hq / hkv <= 4.
 * The results are those of nkv_gemv(x, x_gamma, x_eps, w_qkv) + nkv_qk_norm_rope +
 * nkv_decode_step_t64, bit for bit. While the first K/V groups stream in, the workgroups of
 * each KV head compute that head's (hq / hkv + 2) * 128 rows between them and hand them over
 * (tagged words, through the XCD's L2 when the hand-over is on, nkv_l2_handover), so every
 * workgroup of a KV head waits for the others: the grid (hkv * max(n_parts, 32) workgroups)
 * must fit the device at once, or the call returns NKV_ERR_UNSUPPORTED.
 * With w_o (not NULL) the launch also runs the block's output projection and residual add
 * (`o_proj` and the residual of LeanDecoderLayer, src/nova/layers.py:137,207):
 * h1_out[hidden] = x + w_o out, w_o [hidden][hq * 128] fp16, bit for bit what
 * nkv_gemv(out, NULL, 0, w_o, hidden, hq * 128, x, h1) computes after the step; hq <= 32,
 * hidden at most two rows per wave of the workgroups beyond the first of each KV head
 * (2 * 8 * (grid - hkv)). The merging workgroups publish out as tagged words; the others,
 * done with their part of the cache, stream w_o meanwhile and wait for them. h1_out may be x
 * itself (the residual stream updated in place) but must not overlap out. NULL w_o: no
 * projection, h1_out unused.
 * workspace: nkv_decode_step_qkv_workspace_bytes(hkv, hq, capacity, n_parts) bytes,
 * zero-filled before its first use; it may also serve nkv_decode_step_t64 with the same
 * n_parts (the same partials and counters, which both leave at zero; the row words and
 * their tags lie beyond the partials). A wait for rows is bounded (0.2 s): the outputs are
 * then NaN.
 */
int64_t nkv_decode_step_qkv_workspace_bytes(int64_t hkv, int64_t hq, int64_t capacity, int64_t n_parts);
int nkv_decode_step_qkv_t64(const uint16_t* x, const uint16_t* x_gamma, float x_eps, const uint16_t* w_qkv,
                            int64_t hidden, const uint16_t* q_gamma, const uint16_t* k_gamma, float qk_eps,
                            const float* inv_freq, uint16_t* qkv_out, uint8_t* kq, uint16_t* kmn,
                            uint16_t* kst, uint8_t* vq, uint16_t* vmn, uint16_t* vst, uint16_t* tail_k,
                            uint16_t* tail_v, const int64_t* pos_dev, const int64_t* first_dev,
                            int64_t* written_dev, int64_t* qlen_dev, int64_t* pg_dev, int64_t hq,
                            int64_t hkv, int64_t head_dim, int64_t capacity, uint16_t* out, float* lse_out,
                            const uint16_t* w_o, uint16_t* h1_out, void* workspace, int64_t workspace_bytes,
                            int64_t n_parts, void* stream);

/* Limits of nkv_decode_step_static_t64's scratch: partial results, and the publication
 * area (completion counters and flags). */
#define NKV_STATIC_PART_BYTES (4 << 20)
#define NKV_STATIC_SYNC_BYTES 16384

/*
 * nkv_decode_step_t64 without a workspace argument. It has no counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under hipGraph
 * capture that may not call hipMalloc, tight serving loops, harnesses that forbid
 * allocation). Same arguments, kernels, cache state and output, bit for bit, as
 * nkv_decode_step_t64 with the same n_parts; neither the caller nor the call allocates.
 * The partials and the counters live in a scratch array of NKV_STATIC_PART_BYTES +
 * NKV_STATIC_SYNC_BYTES bytes that the library holds on every GPU it runs on until the
 * process ends. Its address is looked up on the first call on a device (the current
 * device), which also clears the publication area with a kernel on `stream`; every
 * call leaves it cleared. When that first call happens under hipGraph capture, the clear
 * kernel is recorded into the graph as well; replaying it is harmless (the area is
 * already clear whenever no call is in flight), but a caller that captures may prefer to
 * make one eager call first.
 * A call needs hkv * n_parts * 4 * (gq * 128 + ((2 * gq + 3) & ~3)) partial bytes
 * (gq = hq / hkv) <= NKV_STATIC_PART_BYTES and 4 * hkv * (1 + n_parts) publication bytes
 * <= NKV_STATIC_SYNC_BYTES; larger calls return NKV_ERR_UNSUPPORTED.
 * All calls on one GPU share its array: calls that overlap on one GPU (other streams,
 * other threads) race and give wrong results. Calls in order on one stream do not.
 */
int nkv_decode_step_static_t64(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                               int64_t kv_head_stride, uint8_t* kq, uint16_t* kmn, uint16_t* kst,
                               uint8_t* vq, uint16_t* vmn, uint16_t* vst, uint16_t* tail_k,
                               uint16_t* tail_v, const int64_t* pos_dev, const int64_t* first_dev,
                               int64_t* written_dev, int64_t* qlen_dev, int64_t* pg_dev, int64_t hq,
                               int64_t hkv, int64_t head_dim, int64_t capacity, uint16_t* out,
                               float* lse_out, int64_t n_parts, void* stream);

/*
 * fp16 ring attention with a boolean slot mask and its log-sum-exp.
 * Replaces `kvattn.tail_attend(q, k, v, tail_mask)` (src/nova/kvattn.py:447-482).
 * q [hq, 128]; k/v [hkv, slots, 128] fp16 (slots <= 64); mask [slots] uint8 (0/1);
 * out [hq, 128] fp16; lse [hq] fp32. An all-false mask gives out 0, lse -inf.
 */
int nkv_tail_attend(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                    const uint8_t* mask, int64_t hq, int64_t hkv, int64_t head_dim,
                    int64_t slots, uint16_t* out, float* lse, void* stream);

/*
 * Ring validity mask from the device scalars.
 * Replaces `KVInt8Cache.ring_mask` (src/nova/kvattn.py:819-833).
 * mask[i] = (qlen <= p <= u) && (p >= first), p = u - ((u - i) mod slots),
 * u = *written_dev - 1; mask is uint8 [slots].
 */
int nkv_ring_mask(const int64_t* written_dev, const int64_t* qlen_dev, const int64_t* first_dev,
                  int64_t slots, uint8_t* mask, void* stream);

/*
 * ---- Per-token symmetric int8 format ("tok") ----
 * An extension with no counterpart in the reference's storage formats: one symmetric
 * absmax scale per (token, KV head) row of 128, the layout the decode-path specification
 * asks for (int8 codes [H_kv, L, 128], fp16 scales [H_kv, L]). Rounding follows the
 * conventions of kvquant.quantize_int8 (src/nova/kvquant.py:136-149): fp32 arithmetic,
 * round half to even, a 1e-8 floor on the fp32 scale, the scale stored as fp16 and the
 * codes computed with the fp32 scale:
 *   scale = max(max|x| / 127, 1e-8), code = clamp(rint(x / scale), -127, 127),
 *   dequantized value = fp16(code * scale16).
 * A cache in this format keeps every token as int8 (no fp16 ring); its capacity is a
 * multiple of 64.
 */

/* Quantize `rows` slabs of `[n, 128]` (token stride 128, slab stride x_row_stride
 * elements; NKV_F16 / NKV_BF16 / NKV_F32) into codes (slab stride codes_row_stride) and
 * scales (slab stride scale_row_stride). One wave reduces the absmax of 4 rows. */
int nkv_quantize_tok(const void* x, int x_dtype, int64_t x_row_stride, int64_t rows, int64_t n,
                     int64_t dim, int8_t* codes, int64_t codes_row_stride, uint16_t* scales,
                     int64_t scale_row_stride, void* stream);

/* Inverse: out = fp16/bf16/fp32 of code * scale16 (exact in fp32, rounded once). */
int nkv_dequantize_tok(const int8_t* codes, int64_t codes_row_stride, const uint16_t* scales,
                       int64_t scale_row_stride, int64_t rows, int64_t n, int64_t dim, void* out,
                       int out_dtype, int64_t out_row_stride, void* stream);

/* Split-K decode attention over tokens [0, used) of a tok cache (`used` from used_dev
 * when non-NULL). Same launches, q / out / lse / workspace / n_parts contract as
 * nkv_attn_decode_t64 (the counterpart of src/nova/kvattn.py:281-427 for this format). */
int nkv_attn_decode_tok(const uint16_t* q, const int8_t* kq, const uint16_t* ksc, const int8_t* vq,
                        const uint16_t* vsc, int64_t hq, int64_t hkv, int64_t head_dim,
                        int64_t capacity, int64_t used, const int64_t* used_dev, uint16_t* out,
                        float* lse_out, void* workspace, int64_t workspace_bytes, int64_t n_parts,
                        void* stream);

/* Append of one decode token: quantizes k_new / v_new ([hkv, 128], head stride
 * kv_head_stride) into position *pos_dev and sets *written_dev = pos + 1. */
int nkv_append_tok(const uint16_t* k_new, const uint16_t* v_new, int64_t kv_head_stride, int8_t* kq,
                   uint16_t* ksc, int8_t* vq, uint16_t* vsc, const int64_t* pos_dev,
                   int64_t* written_dev, int64_t hkv, int64_t head_dim, int64_t capacity,
                   void* stream);

/* One decode step: nkv_append_tok then attention over [0, pos]. One launch: the prefix
 * kernel over [0, pos) (which also performs the append); the last of each head's
 * workgroups runs the tail (the new token and the combine). */
int nkv_decode_step_tok(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                        int64_t kv_head_stride, int8_t* kq, uint16_t* ksc, int8_t* vq, uint16_t* vsc,
                        const int64_t* pos_dev, int64_t* written_dev, int64_t hq, int64_t hkv,
                        int64_t head_dim, int64_t capacity, uint16_t* out, float* lse_out,
                        void* workspace, int64_t workspace_bytes, int64_t n_parts, void* stream);

/* nkv_decode_step_tok as two launches in two calls with the same arguments, as
 * nkv_decode_step_partials_t64 / _combine_t64 are for the int8t64 step. */
int nkv_decode_step_partials_tok(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                                 int64_t kv_head_stride, int8_t* kq, uint16_t* ksc, int8_t* vq,
                                 uint16_t* vsc, const int64_t* pos_dev, int64_t* written_dev, int64_t hq,
                                 int64_t hkv, int64_t head_dim, int64_t capacity, uint16_t* out,
                                 float* lse_out, void* workspace, int64_t workspace_bytes,
                                 int64_t n_parts, void* stream);
int nkv_decode_step_combine_tok(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                                int64_t kv_head_stride, int8_t* kq, uint16_t* ksc, int8_t* vq,
                                uint16_t* vsc, const int64_t* pos_dev, int64_t* written_dev, int64_t hq,
                                int64_t hkv, int64_t head_dim, int64_t capacity, uint16_t* out,
                                float* lse_out, void* workspace, int64_t workspace_bytes,
                                int64_t n_parts, void* stream);

/*
 * ---- Chained decode step: every layer of one token in one launch ----
 * The decode step of a stack of layers whose inputs may be outputs of an earlier layer (q,
 * k_new, v_new of layer l read from what layer l - 1 wrote, as a model's layers are chained).
 * Layer l computes exactly nkv_decode_step_t64 (nkv_decode_step_tok) on its own cache: the same
 * cache state and scalars bit for bit, the same output up to float summation order. Replaces
 * the per-layer `KVInt8Cache.update` + `KVInt8Cache.attend` pairs that the graph-decode loop
 * issues once per layer (src/nova/decode.py:301-320 running src/nova/layers.py:132-136 for every
 * layer), for stacks whose inter-layer work is itself in the chain (here: outputs consumed
 * directly as the next layer's inputs).
 *
 * One launch of hkv * (n_parts + 1) workgroups that must all be resident at once; the call
 * checks that against the device's occupancy and returns NKV_ERR_UNSUPPORTED when they are
 * not. Per KV head, n_parts workgroups stream the int8 prefix and one merges (append, ring,
 * combine). Layer l + 1's codes, which do not depend on layer l, stream in while layer l is
 * merged.
 *
 * When the inputs of layer l are read (`dep`):
 *  - Forwarded inputs. When q of layer l is the whole output of layer l - 1, head h's q rows
 *    are read from a tagged copy of that output, each word as soon as head h's merger has
 *    written it (no counter, no fence); the same for head h's k_new / v_new rows when they lie
 *    in the rows of that output that head h's merger writes (its q heads h gq .. h gq + gq - 1).
 *    With NKV_DEP_HEAD nothing else is waited for: each KV head's layers then chain on their
 *    own, and head h may start layer l before another head has finished layer l - 1. With
 *    NKV_DEP_ALL every input of layer l is read only after every query head's output of layer
 *    l - 1 has been issued: each merging wave sets its head's issue flag of the layer to the
 *    launch's tag right after its output stores, and the reader polls all hq (<= 64) flags in the
 *    same rounds as its words. That is the dependency of a model, where every q head of layer l
 *    depends on every head of layer l - 1.
 *  - Every other input of layer l is read after layer l - 1's completion counter has reached
 *    hkv (an agent-scope release by each merger, acquire by the reader), in either mode.
 *  Inputs these waits do not order are refused (NKV_ERR_INVALID) when layers_host is given:
 *  a row that lies in layer j's output must lie within one head w's rows there; with w != h it
 *  must not be layer l's own output (j == l), and j > l (a value of the previous step that head
 *  w overwrites in this launch) needs NKV_DEP_ALL. With layers_host NULL the caller guarantees
 *  this.
 *
 * layers_dev: device array of n_layers entries, read by the kernel (it must stay unchanged
 * while launches that use it are pending); layers_host: the same entries in host memory,
 * checked here (every pointer non-null and 16-byte aligned, lse may be NULL; the input rules
 * above), or NULL to skip the check. Every layer shares the device scalars (pos_dev, first_dev:
 * the step's position; written/qlen/pg written once), capacity, head counts and kv_head_stride.
 *
 * workspace: nkv_layers_workspace_bytes(hkv, hq, n_parts, n_layers) bytes, zero-filled before
 * its first use and then dedicated to calls with this (hkv, hq, n_parts, n_layers): a call
 * leaves layer 0's partial block and the layer counters at zero, but the later layers' partial
 * blocks (each set back to zero by its head's merger before the layer is published), the tagged
 * copies of the outputs, the issue flags and the launch counter (the tags' source) keep their
 * values, so the buffer must be zero-filled again before it serves another configuration or
 * another entry point.
 * n_parts <= 0 takes nkv_layers_default_parts.
 *
 * Failure mode. The waits assume every workgroup of the grid runs at once. The occupancy check
 * sees the device, not what else runs on it: when another kernel or process holds CUs, some
 * workgroups start late, a wait may give up (after 0.2 s each), the affected outputs become NaN
 * and the int at byte offset (workspace_bytes & ~3) - 4 * (n_layers + 2) is set to 1; it stays
 * set. A caller polls that error word (ChainedStep.check() does) outside its timed or captured
 * loop; a launch never hangs.
 */
#define NKV_DEP_HEAD 0
#define NKV_DEP_ALL 1

typedef struct nkv_layer_t64 {
  const uint16_t* q;      /* [hq, 128] fp16 */
  const uint16_t* k_new;  /* [hkv, 128] fp16, head stride kv_head_stride */
  const uint16_t* v_new;
  uint8_t* kq;            /* the layer's cache, as nkv_decode_step_t64 takes it */
  uint16_t* kmn;
  uint16_t* kst;
  uint8_t* vq;
  uint16_t* vmn;
  uint16_t* vst;
  uint16_t* tail_k;
  uint16_t* tail_v;
  uint16_t* out;          /* [hq, 128] fp16 */
  float* lse;             /* [hq] fp32, or NULL */
} nkv_layer_t64;

typedef struct nkv_layer_tok {
  const uint16_t* q;
  const uint16_t* k_new;
  const uint16_t* v_new;
  int8_t* kq;             /* the layer's cache, as nkv_decode_step_tok takes it */
  uint16_t* ksc;
  int8_t* vq;
  uint16_t* vsc;
  uint16_t* out;
  float* lse;
} nkv_layer_tok;

int64_t nkv_layers_workspace_bytes(int64_t hkv, int64_t hq, int64_t n_parts, int64_t n_layers);

/* Streaming parts per KV head for a cache of `capacity` tokens on the current device
 * (tok != 0: the per-token symmetric kernel); 0 when the device cannot hold the grid. */
int64_t nkv_layers_default_parts(int64_t hkv, int64_t capacity, int tok);

int nkv_decode_layers_t64(const nkv_layer_t64* layers_dev, const nkv_layer_t64* layers_host,
                          int64_t n_layers, int64_t kv_head_stride, const int64_t* pos_dev,
                          const int64_t* first_dev, int64_t* written_dev, int64_t* qlen_dev,
                          int64_t* pg_dev, int64_t hq, int64_t hkv, int64_t head_dim, int64_t capacity,
                          void* workspace, int64_t workspace_bytes, int64_t n_parts, int dep, void* stream);

int nkv_decode_layers_tok(const nkv_layer_tok* layers_dev, const nkv_layer_tok* layers_host,
                          int64_t n_layers, int64_t kv_head_stride, const int64_t* pos_dev,
                          int64_t* written_dev, int64_t hq, int64_t hkv, int64_t head_dim,
                          int64_t capacity, void* workspace, int64_t workspace_bytes, int64_t n_parts,
                          int dep, void* stream);

/* The input rules of nkv_decode_layers_t64 / _tok (above: which rows of earlier outputs a layer
 * may read under `dep`) checked on a host table alone, without a GPU: NKV_OK, or NKV_ERR_INVALID
 * with nkv_last_error() naming the first row refused. Only the pointer values are used. The
 * launches run the same check when given layers_host. */
int nkv_decode_layers_check_t64(const nkv_layer_t64* layers_host, int64_t n_layers, int64_t kv_head_stride,
                                int64_t hq, int64_t hkv, int dep);
int nkv_decode_layers_check_tok(const nkv_layer_tok* layers_host, int64_t n_layers, int64_t kv_head_stride,
                                int64_t hq, int64_t hkv, int dep);

/*
 * ---- Paged batch of ragged sequences (int8t64) ----
 * No counterpart in the reference, which decodes one sequence and pads lengths to
 * power-of-two buckets with an additive -inf mask (src/nova/decode.py:39-48, 200-205);
 * here each sequence is attended over exactly its own tokens, which equals that masked
 * computation without reading the padding. The per-sequence arithmetic is the int8t64
 * step's (nkv_decode_step_t64).
 * pages: uint8 [num_pages][hkv][17408], one page = one 64-token group of one KV head:
 *   K codes [64][128], V codes [64][128], then fp16 kst[128], kmn[128], vst[128], vmn[128].
 * page_table: int32 [nseq][table_stride], group g of sequence b lives in page
 *   page_table[b * table_stride + g] (the same ids in every layer's pool); an entry outside
 *   [0, num_pages), such as -1 for an unassigned slot, is no page: a sequence whose current group
 *   (pos / 64) has no page neither appends nor attends (its output is 0, its lse -inf), and a
 *   prefix group without a page reads page 0 rather than memory outside the pool.
 * rings: fp16 [nseq][hkv][2][64][128] (K then V; slot = position mod 64).
 * pos_dev: int64 [nseq], the position each sequence appends at this step.
 * k_new / v_new: [nseq][hkv][128] fp16 with strides kv_seq_stride / kv_head_stride.
 * Prefix work unit w (w < total_parts) serves sequence wg_map[w] >> 16, part
 * wg_map[w] & 0xffff of its seq_parts[2b + 1] parts; seq_parts[2b] is its first unit (a
 * sequence's units are consecutive, w = seq_parts[2b] + part). A sequence has at most 256 parts
 * (the tail's merge holds 256 partials; it ignores partials beyond them).
 * q / out: [nseq][hq][128] fp16; lse_out [nseq][hq] fp32 (may be NULL).
 * The workspace holds per KV head one partial slot per unit and one per sequence (the int8t64
 * step's ring partial, after the sequence's prefix partials), then the completion counters;
 * its size is bounded with nseq <= total_parts.
 */
int64_t nkv_paged_workspace_bytes(int64_t hkv, int64_t hq, int64_t total_parts);

/* Whole groups of one sequence's prompt quantized straight into its pages (the int8t64
 * arithmetic of nkv_quantize_int8, bit for bit): x [hkv][n][128] (head stride x_head_stride
 * elements, NKV_F16 / NKV_BF16 / NKV_F32), n a multiple of 64; tokens 64 g .. 64 g + 63 of x form
 * the sequence's group first_group + g, stored as tensor `which` (0 K, 1 V) of KV head h in page
 * table_row[first_group + g] (codes and that tensor's two rulers). Groups whose entry is outside
 * [0, num_pages) are skipped. Replaces the bulk quantize of KVInt8Cache.finish_prefill
 * (src/nova/kvattn.py:745-783) for a paged cache; the reference has no paged layout. */
int nkv_paged_quantize_t64(const void* x, int x_dtype, int64_t x_head_stride, int64_t hkv, int64_t n, int which,
                           uint8_t* pages, const int32_t* table_row, int64_t first_group, int64_t num_pages,
                           void* stream);

/* Append of one token per sequence: ring slot pos % 64, requantization of the ring into
 * the sequence's page of group pos / 64 (which must be assigned). */
int nkv_paged_append_t64(const uint16_t* k_new, const uint16_t* v_new, int64_t kv_seq_stride,
                         int64_t kv_head_stride, uint8_t* pages, const int32_t* page_table,
                         int64_t table_stride, int64_t num_pages, uint16_t* rings, const int64_t* pos_dev,
                         int64_t nseq, int64_t hkv, int64_t head_dim, void* stream);

/* Decode attention of every sequence over its whole groups before pos and its ring
 * (tokens up to and including pos). One launch of the prefix kernel (total_parts * hkv
 * workgroups); the last workgroup of each (sequence, KV head) runs its tail. workspace:
 * zero-filled before its first use, >= nkv_paged_workspace_bytes bytes, its last bytes
 * hold the completion counters (left at zero by every call). */
int nkv_paged_attn_decode_t64(const uint16_t* q, const uint8_t* pages, const int32_t* page_table,
                              int64_t table_stride, int64_t num_pages, const uint16_t* rings,
                              const int64_t* pos_dev, int64_t nseq, int64_t hq, int64_t hkv, int64_t head_dim,
                              const int32_t* wg_map, const int32_t* seq_parts, int64_t total_parts,
                              uint16_t* out, float* lse_out, void* workspace, int64_t workspace_bytes,
                              void* stream);

/* What nkv_paged_append_t64 then nkv_paged_attn_decode_t64 compute in one launch (cache state
 * bit for bit; outputs up to float summation order): the new token comes from k_new / v_new.
 * With more than one workgroup for a (sequence, KV head), the first to finish its prefix share
 * stages the ring with the new token, attends over it, publishes the ring partial and, beside
 * that, stores the token in its ring slot and requantizes the group of pos into its page; the
 * last merges the prefix partials with the ring partial. With one workgroup it does all of it.
 * Nothing else in the launch reads that slot or that page. */
int nkv_paged_decode_step_t64(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                              int64_t kv_seq_stride, int64_t kv_head_stride, uint8_t* pages,
                              const int32_t* page_table, int64_t table_stride, int64_t num_pages,
                              uint16_t* rings, const int64_t* pos_dev, int64_t nseq, int64_t hq, int64_t hkv,
                              int64_t head_dim, const int32_t* wg_map, const int32_t* seq_parts,
                              int64_t total_parts, uint16_t* out, float* lse_out, void* workspace,
                              int64_t workspace_bytes, void* stream);

/*
 * ---- Paged batch in the per-token symmetric format ----
 * Per-token, per-KV-head symmetric int8 codes with one fp16 scale per token and KV head (the
 * arithmetic of nkv_quantize_tok) in a paged, 128-byte-aligned layout. It replaces the
 * contiguous [B, H_kv, max_len, D] storage of KVInt8Cache (src/nova/kvattn.py:589-601) for a
 * batch of sequences; the reference has no paged layout and no per-token format.
 * pages: uint8 [num_pages][hkv][NKV_PAGE_TOK_BYTES], one page = 64 tokens of one KV head:
 *   K codes int8 [64][128], V codes int8 [64][128], then fp16 K scales [64], V scales [64].
 *   Token p of a sequence is row p % 64 of its page page_table[b * table_stride + p / 64].
 * page_table, pos_dev, k_new / v_new, wg_map / seq_parts, q / out / lse_out, workspace: as for
 *   the int8t64 paged batch above. There are no rings.
 */
#define NKV_PAGE_T64_BYTES 17408
#define NKV_PAGE_TOK_BYTES 16640

/* Tokens first_token .. first_token + n - 1 of one sequence quantized straight into its pages
 * (nkv_quantize_tok's arithmetic, bit for bit): x [hkv][n][128] (head stride x_head_stride
 * elements, NKV_F16 / NKV_BF16 / NKV_F32); token first_token + t goes to row (first_token + t)
 * % 64 of tensor `which` (0 K, 1 V) of KV head h in page table_row[(first_token + t) / 64],
 * its scale beside. Tokens whose entry is outside [0, num_pages) are skipped. Replaces the
 * prefill store of KVInt8Cache.update (src/nova/kvattn.py:668-698) for this layout. */
int nkv_paged_quantize_tok(const void* x, int x_dtype, int64_t x_head_stride, int64_t hkv, int64_t n, int which,
                           uint8_t* pages, const int32_t* table_row, int64_t first_token, int64_t num_pages,
                           void* stream);

/* One decode step of every sequence in one launch: the token at pos_dev[b] is quantized into
 * its page (by the first prefix workgroup of each sequence and KV head), and each sequence
 * attends over its tokens [0, pos_b] (the prefix [0, pos_b) from the pages, the new token
 * quantized and dequantized in the tail exactly as stored). A sequence whose page of pos_b is
 * missing neither appends nor attends (output 0, lse -inf). */
int nkv_paged_decode_step_tok(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                              int64_t kv_seq_stride, int64_t kv_head_stride, uint8_t* pages,
                              const int32_t* page_table, int64_t table_stride, int64_t num_pages,
                              const int64_t* pos_dev, int64_t nseq, int64_t hq, int64_t hkv, int64_t head_dim,
                              const int32_t* wg_map, const int32_t* seq_parts, int64_t total_parts,
                              uint16_t* out, float* lse_out, void* workspace, int64_t workspace_bytes,
                              void* stream);

/*
 * ---- Chunked prefill attention over the int8t64 cache (MFMA) ----
 * Replaces the fp16 staging + causal SDPA of KVInt8Cache.attend_prefill
 * (src/nova/kvattn.py:791-815) for a cache whose first `used` tokens (a multiple of 64) are
 * int8t64: a chunk of m query tokens at positions used .. used + m - 1 attends causally to
 * the dequantized cache [0, used) and to its own fp16 K/V.
 * q [hq][m][128], k_chunk / v_chunk [hkv][m][128], out [hq][m][128], fp16.
 * Two launches: the chunk kernel (hkv * ceil(m * hq / hkv / rows) * splits workgroups on
 * v_mfma_f32_16x16x32_f16, one partial per query row and split into `workspace`) and a
 * combine kernel. splits <= 0 picks one.
 */
int64_t nkv_prefill_workspace_bytes(int64_t hkv, int64_t hq, int64_t m, int64_t splits);
/* The splits value `splits <= 0` resolves to (enough workgroups to fill the GPU). */
int64_t nkv_prefill_default_splits(int64_t hkv, int64_t hq, int64_t m, int64_t used);
int nkv_prefill_attn_t64(const uint16_t* q, const uint16_t* k_chunk, const uint16_t* v_chunk, int64_t m,
                         const uint8_t* kq, const uint16_t* kmn, const uint16_t* kst, const uint8_t* vq,
                         const uint16_t* vmn, const uint16_t* vst, int64_t capacity, int64_t used,
                         int64_t hq, int64_t hkv, int64_t head_dim, uint16_t* out, void* workspace,
                         int64_t workspace_bytes, int64_t splits, void* stream);

/*
 * The same attention with an fp16 history before the chunk: replaces the staged branch of
 * KVInt8Cache.attend_prefill (src/nova/kvattn.py:791-815), where the prompt's earlier chunks
 * are still fp16 in the staging area. k16 / v16 hold m_kv >= m fp16 tokens per KV head (head
 * h's token j at k16 + h * kv_head_stride + j * 128); query token i (i < m) attends the int8
 * tokens [0, used) and the fp16 tokens j <= (m_kv - m) + i. With m_kv == m and
 * kv_head_stride == m * 128 this is nkv_prefill_attn_t64.
 */
int nkv_prefill_attn_hist_t64(const uint16_t* q, int64_t m, const uint16_t* k16, const uint16_t* v16,
                              int64_t m_kv, int64_t kv_head_stride, const uint8_t* kq, const uint16_t* kmn,
                              const uint16_t* kst, const uint8_t* vq, const uint16_t* vmn, const uint16_t* vst,
                              int64_t capacity, int64_t used, int64_t hq, int64_t hkv, int64_t head_dim,
                              uint16_t* out, void* workspace, int64_t workspace_bytes, int64_t splits,
                              void* stream);

/*
 * Plain device copy (16-byte vector loads and stores). Used to calibrate the
 * HBM traffic counters (FETCH_SIZE / WRITE_SIZE) against a known byte count;
 * no counterpart in the reference. nbytes must be a multiple of 16.
 */
int nkv_copy_bytes(const void* src, void* dst, int64_t nbytes, void* stream);

/*
 * Read-bandwidth probe: `blocks` workgroups of 256 lanes read `nbytes` from `src` with
 * 16-byte loads and write one XOR checksum per workgroup to sink[blocks]. Times the
 * HBM read ceiling a single launch of a given size reaches, the counterpart of the
 * reference's read-and-reduce ceiling bench (src/diagnostics/bench_int8_unpack.py:58-102).
 * nbytes must be a multiple of 16.
 */
int nkv_read_bw(const void* src, int64_t nbytes, uint32_t* sink, int64_t blocks, void* stream);

/*
 * Core clock probe: `blocks` workgroups of one wave each run `iters` rounds of two dependent
 * FMAs; workgroup b writes out[3b] = its XCD, out[3b+1] = the core clock counter's advance
 * (s_memtime) and out[3b+2] = the 100 MHz real-time counter's advance (s_memrealtime), so
 * that 100 * out[3b+1] / out[3b+2] is its XCD's core clock in MHz while it ran. Launched right
 * after a timed run, it reads the clock that run left (the clocks move over milliseconds).
 * out holds 3 * blocks words; 1 <= blocks <= 1024, 1 <= iters <= 2^24. No counterpart in the
 * reference (measurement only).
 */
int nkv_clock_probe(uint64_t* out, int64_t blocks, int64_t iters, void* stream);

/*
 * The same ceiling for the decode kernels' own load pattern: `blocks` workgroups of 8 waves
 * (one per CU) read `src` in 8 KiB chunks with nontemporal LDS-DMA loads (global_load_lds,
 * 16 bytes per lane), two chunks in flight per wave, as the prefix and chained kernels stream
 * their codes; one XOR checksum per workgroup to sink[blocks]. nbytes must be a multiple of 8192.
 * Counterpart of the reference's read + unpack ceiling (src/diagnostics/bench_int8_unpack.py:58-102).
 */
int nkv_read_bw_lds(const void* src, int64_t nbytes, uint32_t* sink, int64_t blocks, void* stream);

/*
 * XCD-local hand-over (no counterpart in the reference: a placement property of this GPU).
 * The split-K launches hand each workgroup's partial (and, in the chained step, each layer's
 * forwarded output) to a workgroup of the same KV head. The device deals the workgroups of a
 * launch to its n XCDs (each with its own L2) in turn: workgroup b runs on XCD (b + k) mod n,
 * the start k varying between launches (graph replays rotate it). The workgroups of KV head h
 * are b = h mod hkv, so when n divides hkv they share one XCD: the words are then stored into
 * that L2 (plain stores) instead of being written through to memory, and the reader's
 * agent-scope loads find them there (0.25 us per hand-over between idle workgroups against
 * 0.43 us; the 36-layer chained step at 32k runs ~10% faster). Writes that other XCDs read
 * (issue flags, counters) stay agent-scope.
 *
 * nkv_l2_handover(1, ..) probes the current device (a launch of 4096 workgroups that record
 * their XCD, read back synchronously: call it outside stream capture) and turns the hand-over
 * on for that device when workgroup b ran on the XCD of workgroup b mod n for every b, the
 * first n on distinct XCDs, with n = the device's XCD count, a power of two <= 8; *xcds = n,
 * or 0 when it stays off. nkv_l2_handover(0, ..) turns it off (every hand-over through memory).
 * A device that was never probed hands over through memory. Were the dealing rule broken in a
 * later launch, a reader would not see a writer's L2: its bounded wait gives up and its outputs
 * are NaN (the chained step also sets its error word), and the workspace is then to be
 * zero-filled again before reuse.
 */
int nkv_l2_handover(int enable, int64_t* xcds, void* stream);

/* ---------------------------------------------------------------- decode-step projections
 *
 * Batch-1 fp16 kernels of the synthetic decoder that drives the int8 KV path end to end.
 * They replace torch ops of the decoder layer (RMSNorm + nn.Linear in src/nova/norm.py:35-41
 * and src/nova/layers.py:99-162,165-195), not a kernel of the reference; they exist so that a
 * captured decode step is a few launches per layer. All vectors are contiguous fp16; weights
 * are row-major [out][in]; x, gamma and W 16-byte aligned; in_features a multiple of 8, at most 16384.
 */

/*
 * y[o] = fp16(sum_i W[o][i] * xn[i]) (+ residual[o], added in fp16), xn = x when gamma is
 * NULL, else RMSNorm(x) = fp16(fp16(x * rsqrt(mean(x^2) + eps)) * gamma) with an fp32 mean.
 * Dot products accumulate in fp32. `residual` may be NULL; y may be residual itself but must not
 * overlap x or a shifted view of residual (NKV_ERR_INVALID).
 */
int nkv_gemv(const uint16_t* x, const uint16_t* gamma, float eps, const uint16_t* w, int64_t out_features,
             int64_t in_features, const uint16_t* residual, uint16_t* y, void* stream);

/*
 * The SwiGLU MLP's first half: act[j] = fp16(silu(g_j)) * u_j, g = W[0:inter] xn and
 * u = W[inter:2 inter] xn (each rounded to fp16), W the stacked [gate; up] weight of
 * [2 * intermediate][in_features], xn as in nkv_gemv (LeanMLP, src/nova/layers.py:173-174).
 * act must not overlap x (NKV_ERR_INVALID).
 */
int nkv_swiglu_gemv(const uint16_t* x, const uint16_t* gamma, float eps, const uint16_t* w_gate_up,
                    int64_t intermediate, int64_t in_features, uint16_t* act, void* stream);

/*
 * In place on one token's stacked projection qkv [hq + 2 hkv][128] (q heads, k heads, v heads):
 * per-head RMSNorm of the q and k heads (q_gamma / k_gamma, fp32 mean of squares), then the
 * rotary embedding at position *pos (device int64): x * cos + rotate_half(x) * sin with
 * cos/sin = fp16(cos/sin((float)pos * inv_freq[i mod 64])), fp32 inv_freq[64]. v is untouched.
 */
int nkv_qk_norm_rope(uint16_t* qkv, int64_t hq, int64_t hkv, int64_t head_dim, const uint16_t* q_gamma,
                     const uint16_t* k_gamma, float eps, const float* inv_freq, const int64_t* pos, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NOVA_KV_H */
