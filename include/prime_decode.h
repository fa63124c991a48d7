/* C ABI of the MI355X (gfx950) SmolLM2 decode megakernel library `libprime_decode.so`.
 *
 * Every entry point takes plain device pointers and sizes; no torch types cross this boundary.
 * Launches are asynchronous on `stream` (a hipStream_t, or NULL for the null stream); the return
 * value is 0 or a status code (see prime_decode_status_string / decode360_status_string).
 *
 * Reference interfaces each entry replaces (paths under Mantissagithub/prime-kernels):
 *   decode360, decode360_workspace_bytes, decode360_debug_bytes, decode360_status_string
 *       prime_kernels/decode_megakernel_360m/csrc/block360_kernel.inc:849-938
 *   mk_decode, mk_workspace_bytes, mk_status_string, mk_query
 *       prime_kernels/decode_megakernel/csrc/megakernel.cu:833-927
 *   block360_decode, block360_workspace_bytes, block360_debug_bytes, block360_status_string
 *       research/smollm2_360m_block/block360_kernel.inc:398-479
 * pk_decode / pk_workspace_bytes / pk_query are this library's superset of both (model choice,
 * layer count, LM head with greedy ids and optional logits); they have no single counterpart.
 */
#ifndef PRIME_DECODE_H
#define PRIME_DECODE_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes (block360.cu:42-51 keeps the same numbers). */
#define PK_OK 0
#define PK_ERR_BATCH 9101        /* batch outside the supported range */
#define PK_ERR_MAX_SEQ 9102      /* max_seq_len / seq_lens outside the supported range */
#define PK_ERR_NULL 9103         /* a required pointer is NULL */
#define PK_ERR_COOP 9104         /* cooperative launch unsupported */
#define PK_ERR_RESIDENCY 9105    /* workgroups cannot all be resident (LDS / CU count) */
#define PK_ERR_ARCH 9106         /* device is not gfx950 */
#define PK_ERR_ALIGN 9107        /* KV offsets/strides not multiples of 8 elements, or pointers not 16-B aligned */
#define PK_ERR_SCRATCH 9108      /* workspace or debug buffer too small */
#define PK_ERR_BLOCK 9109        /* block_size != 16, bt_stride too small, or bad layer index */
#define PK_ERR_MODEL 9110        /* unknown model id or layer count */
#define PK_ERR_DEBUG 9111        /* per-stage debug capture requested for a model/format without it */
#define PK_ERR_CAPTURE 9112      /* the first use of a device (its state's allocation) happened under stream capture */
#define PK_ERR_ABORTED 9113      /* a previous step on this device gave up a bounded wait; its outputs were poisoned */
#define PK_ERR_STATE 9114        /* the library's per-device state could not be allocated */
#define PK_ERR_NOALLOC 9115      /* pk_decode_noalloc: batch, weights or context beyond what its fixed array holds */

/* Options for pk_set_option. */
#define PK_OPT_COOPERATIVE 1     /* 1: launch with hipLaunchCooperativeKernel (default 0, or PK_LAUNCH=cooperative) */
#define PK_OPT_SPLIT_ROLE 2      /* 0: batch-1 steps stay on the general kernel (default 1, or PK_SPLIT_ROLE=0) */
#define PK_OPT_L2_RECORDS 3      /* 0: batch-1 attention records stay in uncached memory even when a KV head's
                                    chunks share an XCD (the path a placement mismatch takes; default 1) */
#define PK_OPT_SKEW 4            /* != 0: arrival-skew test, the seed of pseudo-random delays every workgroup
                                    takes before publishing exchange data (results must not change; default 0) */
#define PK_OPT_SPLIT_WIDE 5      /* 0: batch-1 contexts beyond the narrow split-role limit go to the general
                                    kernel instead of the wide split-role layout (default 1, or PK_SPLIT_WIDE=0) */

/* Models. */
#define PK_MODEL_SMOLLM2_360M 360
#define PK_MODEL_SMOLLM2_135M 135

/* Bytes of the `scratch` argument the decode entry points require (present and at least this large).
 * The scratch carries nothing between calls, as in the reference, where it is plain torch memory
 * (decode_megakernel_360m/__init__.py:40-48): every word the kernels exchange lives in state the
 * library allocates per device (uncached device memory for the exchange words, ordinary device memory
 * for records that stay in one XCD's L2, a pinned host status word pair) on pk_init or the first
 * decode call on the device, and keeps until the process ends.  As with the reference's per-device
 * scratch, steps on one device must not run concurrently from two streams. */
size_t pk_workspace_bytes(int model);

/* Allocate and zero the current device's state now, outside any stream capture (a first use under
 * capture returns PK_ERR_CAPTURE), and clear pk_decode_noalloc's array on the device.  Returns 0 or a
 * status code.  No reference counterpart. */
int pk_init(void);

/* Library options (PK_OPT_*).  Returns the previous value, or -1 for an unknown option.  No reference
 * counterpart. */
int pk_set_option(int option, int value);

/* Diagnostics (no reference counterpart).  pk_state_read synchronises `stream` and copies n header
 * words of the current device's state (0 step epoch, 1 epoch of the last step that gave up a bounded
 * wait, 2 its wait site).  pk_state_status reads the pending failure report {epoch, wait site}
 * without clearing it; the next decode call on the device returns PK_ERR_ABORTED and clears it. */
int pk_state_read(void* stream, size_t word, unsigned* out, int n);
int pk_state_status(void* stream, unsigned* out);
/* pk_state_status that also clears the report, so the next decode call does not report that step
 * again (no reference counterpart). */
int pk_state_take(void* stream, unsigned* out);
/* Test hooks (synchronous; no reference counterpart): set the step epoch of the current device's
 * state, or mark the next step as failed so that each of its bounded waits gives up at once. */
int pk_test_set_epoch(void* stream, unsigned epoch);
int pk_test_abort_next(void* stream);
/* Test hook (synchronous; no reference counterpart): the next pk_decode_noalloc step on the current
 * device gives up each of its bounded waits at once (the device's array must have been used). */
int pk_test_abort_next_noalloc(void* stream);
/* Test hook (synchronous; no reference counterpart): the exchange-unit integrity check.  Workgroups
 * publish 16-byte units {3 payload words, tag} with the decode kernels' stores, the payload a function
 * of (tag, unit), and read every unit back with the kernels' polling loads, comparing the payload of
 * each unit they accept.  mode 0: all 256 workgroups, uncached memory (pk_decode's cross-XCD units);
 * 1: ordinary memory (pk_decode_noalloc's array); 2: the 32 workgroups of one XCD, plain stores
 * (attention records through the XCD's L2).  slot: 16 (four units per 64-byte line, from different
 * workgroups) or 64 (one per line).  out[4] = {torn units, polls given up, units checked, mask of
 * the XCC ids the participating workgroups ran on}. */
int pk_test_exchange_units(int mode, int rounds, int slot, unsigned* out);

/* One greedy decode step for B = 1..16 sequences (vLLM FLASH_ATTN metadata, paged KV
 * [blocks, KVH, 16, 128]; contexts may differ per sequence).  B = 1 (bf16 or MXFP8 weights) runs the
 * split-role kernel: its narrow layout for contexts up to PK_NOALLOC_MAX_SEQ_360M / _135M tokens (for
 * 135M builds with 4 and 6 attention chunks per KV head up to 1025 and 1537 tokens, the 10-chunk
 * build above), its wide layout (attention over KVH XCDs) up to PK_SR_WIDE_MAX_SEQ, the general GEMV
 * kernel beyond
 * (PK_OPT_SPLIT_ROLE / PK_OPT_SPLIT_WIDE switch the split-role layouts off).  B = 2 without
 * layer_outputs runs as two batch-1 steps, one per sequence (faster than one batched step of two);
 * B >= 2 otherwise runs the batched kernel, whose projections and LM head are
 * MFMA tiles over all B tokens, so the weights are read once per step for the whole batch.  The
 * reference caps SmolLM2-360M at B <= 2 (decode_megakernel_360m/__init__.py:46).
 *   layers: device table [n_layers][6] of pointers (norm1, qkv, o, norm2, gate_up, down), bf16.
 *   kv: device table [n_layers] of cache base pointers; K at k_off, V at v_off (elements).
 *   out_hidden [B, H] bf16 receives the final-normed hidden state.
 *   out_ids [B] int64 and/or out_logits [B, 49152] bf16 request the tied LM head (NULL: skipped).
 *   layer_outputs [n_layers, B, H] bf16 is optional. */
int pk_decode(void* stream, int model, int B, int n_layers, const void* input_ids, int ids_i64,
              const void* embed, const void* final_norm, const void* positions, const void* seq_lens,
              const void* block_table, int bt_stride, const void* slot_mapping, const void* layers,
              void* const* kv, long long k_off, long long v_off, long long block_stride,
              long long token_stride, long long head_stride, int block_size, const void* cos_sin,
              int cs_fp32, void* out_hidden, void* layer_outputs, void* out_ids, void* out_logits,
              void* scratch, size_t scratch_bytes, int max_seq_len);

/* pk_decode_noalloc's failure report, read from its fixed array on the current device (synchronises
 * `stream`; allocates nothing): out[0] the epoch of the last step that gave up a bounded wait (0: none
 * since the array was cleared or the report last cleared), out[1] its wait site, out[2] the epoch of
 * the last step.  clear != 0 resets the report.  No reference counterpart. */
int pk_noalloc_status(void* stream, int clear, unsigned* out);

/* Limits of pk_decode_noalloc: its fixed per-device array, and the largest max_seq_len per model. */
#define PK_NOALLOC_SCRATCH_BYTES 8388608
#define PK_NOALLOC_MAX_SEQ_360M 1537
#define PK_NOALLOC_MAX_SEQ_135M 2561
/* Longest context (tokens attended) of the split-role kernel's wide layout, both models. */
#define PK_SR_WIDE_MAX_SEQ 9729

/* pk_decode that allocates nothing, for callers that cannot allocate device memory: code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc.  It has no counterpart in
 * the reference.  Arguments are pk_decode's without `scratch`/`scratch_bytes`.  Every word its
 * kernel exchanges lives in one array of PK_NOALLOC_SCRATCH_BYTES per device that is compiled into
 * the library (a device global each GPU holds until the process ends); it calls no hipMalloc,
 * hipFree or other allocating routine.  It runs the split-role batch-1 kernel only: B must be 1,
 * the weights bf16, and max_seq_len (the block table's capacity) at most PK_NOALLOC_MAX_SEQ_360M or
 * PK_NOALLOC_MAX_SEQ_135M; anything else returns PK_ERR_NOALLOC and launches nothing.  The first call
 * on a device clears the array with a fill kernel on `stream` (pk_init also clears it; when the first
 * call is captured, every replay of the graph clears it).  All calls on one device share the array
 * and each leaves its contents for the next: calls that overlap on one device (from two streams, or
 * beside another decode step) race.  A step that gives up a bounded wait poisons its outputs (token
 * ids -1, NaN hidden state and logits) and leaves its epoch and wait site in the array's header, which
 * pk_noalloc_status reads; pk_state_status does not see it. */
int pk_decode_noalloc(void* stream, int model, int B, int n_layers, const void* input_ids, int ids_i64,
                      const void* embed, const void* final_norm, const void* positions, const void* seq_lens,
                      const void* block_table, int bt_stride, const void* slot_mapping, const void* layers,
                      void* const* kv, long long k_off, long long v_off, long long block_stride,
                      long long token_stride, long long head_stride, int block_size, const void* cos_sin,
                      int cs_fp32, void* out_hidden, void* layer_outputs, void* out_ids, void* out_logits,
                      int max_seq_len);

/* pk_decode with per-stage debug capture (SmolLM2-360M bf16, B <= 2) and, for 360M, an optional
 * lossless gate/up table (prime_lossless.h; NULL: dense).  `debug` (16-byte aligned, at least
 * decode360_debug_bytes() bytes, NULL: no capture) receives the reference's layout
 * (block360_kernel.inc:1-20): for every layer the bf16 rows [2][N] of norm1, qkv, attn, o, h1,
 * norm2, gate, up, silu, act, down, out (row b = sequence b); for layer `debug_layer_index`
 * (-1: none) also the rotated queries [2][960], bf16(q.k), the scaled scores and the probabilities
 * [2][15][8192] (positions from 8192 on are not recorded) and the P.V output [2][960].  Other
 * models or MXFP8 weights return PK_ERR_DEBUG when `debug` is set. */
int pk_decode_debug(void* stream, int model, int B, int n_layers, const void* input_ids, int ids_i64,
                    const void* embed, const void* final_norm, const void* positions, const void* seq_lens,
                    const void* block_table, int bt_stride, const void* slot_mapping, const void* layers,
                    void* const* kv, long long k_off, long long v_off, long long block_stride,
                    long long token_stride, long long head_stride, int block_size, const void* cos_sin,
                    int cs_fp32, void* out_hidden, void* layer_outputs, void* out_ids, void* out_logits,
                    void* scratch, size_t scratch_bytes, int max_seq_len, const void* encoded_gu_table,
                    void* debug, size_t debug_bytes, int debug_layer_index);

/* pk_decode with MXFP8 projection weights (SmolLM2-360M only): `layers` is a device table
 * [n_layers][10] of (norm1, qkv, qkv_scales, o, o_scales, norm2, gate_up, gate_up_scales, down,
 * down_scales): e4m3 bytes [rows, cols] and e8m0 scale codes [rows, pk_mxfp8_scale_stride(cols)],
 * one per 32 consecutive weights of a row, each row padded with zeros to a multiple of 16 bytes.
 * Norms, embedding and the tied LM head stay bf16.  B must be 1 (PK_ERR_BATCH otherwise).
 * No reference counterpart: BASELINE config 5. */
int pk_decode_mxfp8(void* stream, int model, int B, int n_layers, const void* input_ids, int ids_i64,
                    const void* embed, const void* final_norm, const void* positions, const void* seq_lens,
                    const void* block_table, int bt_stride, const void* slot_mapping, const void* layers,
                    void* const* kv, long long k_off, long long v_off, long long block_stride,
                    long long token_stride, long long head_stride, int block_size, const void* cos_sin,
                    int cs_fp32, void* out_hidden, void* layer_outputs, void* out_ids, void* out_logits,
                    void* scratch, size_t scratch_bytes, int max_seq_len);

/* Bytes per row of the MXFP8 scale array for rows of `cols` weights (cols/32 rounded up to 16). */
size_t pk_mxfp8_scale_stride(int cols);

/* Quantise a bf16 matrix [rows, cols] (cols a multiple of 32) to MXFP8 on the device, asynchronously
 * on `stream`: per 32 weights of a row, scale code s = e8m0(amax / 448) rounded toward +inf
 * (saturating), weights e4m3(bf16(x * 2^(127-s))) rounded to nearest even, saturating at +-448 --
 * the rule prime_kernels/rmsnorm/test.cu:126-144 applies.  q [rows, cols], scales
 * [rows, pk_mxfp8_scale_stride(cols)]; all pointers 16-byte aligned. */
int pk_quantize_mxfp8(void* stream, const void* src, void* q, void* scales, int rows, int cols);

/* Device properties relevant to the launch (current device). Returns a status. */
int pk_query(int* cu_count, int* coop, int* max_lds_per_block, int* is_gfx950, size_t* lds_bytes);

/* Diagnostics: record per-phase wall-clock timestamps (100 MHz) of subsequent launches into
 * `buf` ([256][n_layers*40 + 4] uint64, device memory); NULL disables. No reference counterpart. */
void pk_set_trace(void* buf);

/* Human-readable status (static storage). */
const char* prime_decode_status_string(int status);

/* ---- reference-compatible entry points -------------------------------------------------- */

/* SmolLM2-360M, 32 layers, hidden state out (block360_kernel.inc:852-862, same argument list).
 * `debug` (optional, B <= 2) receives the per-stage capture described at pk_decode_debug;
 * `debug_layer_index` must be -1..31. */
int decode360(void* stream, int B, const void* input_ids, const void* embed, const void* final_norm,
              const void* positions, const void* seq_lens, const void* block_table, int bt_stride,
              const void* slot_mapping, const void* layers, void* const* kv, long long k_off,
              long long v_off, long long block_stride, long long token_stride, long long head_stride,
              int block_size, const void* cos_sin, int cs_fp32, void* out_hidden, void* layer_outputs,
              void* scratch, size_t scratch_bytes, void* debug, size_t debug_bytes, int max_seq_len,
              int debug_layer_index);
size_t decode360_workspace_bytes(void);   /* block360_kernel.inc:849 */
size_t decode360_debug_bytes(void);       /* block360_kernel.inc:850 */
const char* decode360_status_string(int status);  /* block360_kernel.inc:925-938 */

/* Research single-block ABI (research/smollm2_360m_block/block360_kernel.inc:399-470, same argument
 * list): one SmolLM2-360M decoder block, hidden states [B, 960] in (B = 1, 2), the block output
 * [B, 960] out (no final norm), `layer` a device table of the 6 layer pointers, `kv` that layer's
 * paged cache.  `debug` (optional, block360_debug_bytes()) receives the block's stage layout
 * (block360_kernel.inc:1-8): norm1, qkv, attn, h1, norm2, act, out, each [4][N] (row b = sequence
 * b).  The scratch (block360_workspace_bytes()) follows pk_workspace_bytes' rules. */
int block360_decode(void* stream, int B, const void* hidden, const void* positions, const void* seq_lens,
                    const void* block_table, int bt_stride, const void* slot_mapping, const void* layer, void* kv,
                    long long k_off, long long v_off, long long block_stride, long long token_stride,
                    long long head_stride, int block_size, const void* cos_sin, int cs_fp32, void* out_hidden,
                    void* scratch, size_t scratch_bytes, void* debug, size_t debug_bytes, int max_seq_len);
size_t block360_workspace_bytes(void);        /* block360_kernel.inc:398 */
size_t block360_debug_bytes(void);            /* block360_kernel.inc:399 */
const char* block360_status_string(int status);

/* SmolLM2-135M, 30 layers (megakernel.cu:844-851, same argument list). */
int mk_decode(void* stream, int B, const void* input_ids, int ids_i64, const void* positions,
              const void* seq_lens, const void* block_table, int bt_stride, const void* slot_mapping,
              const void* layers, const void* embed, const void* final_norm, void* const* kv_layers,
              long long k_off, long long v_off, long long block_stride, long long token_stride,
              long long head_stride, int block_size, const void* cos_sin, int cs_fp32,
              void* out_hidden, void* scratch, size_t scratch_bytes, int max_seq_len);
size_t mk_workspace_bytes(int B, int max_seq_len);  /* megakernel.cu:838-842 */
const char* mk_status_string(int status);            /* megakernel.cu:914-927 */

#ifdef __cplusplus
}
#endif

#endif /* PRIME_DECODE_H */
