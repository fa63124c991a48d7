/* C ABI of the lossless bf16 gate/up codec and the decode step that streams its encoding
 * (part of `libprime_decode.so`; see prime_decode.h for the decode ABI conventions).
 *
 * Reference interfaces each entry replaces (paths under Mantissagithub/prime-kernels):
 *   EncodedGULayer                     prime_kernels/lossless_bf16/csrc/encoded_gu.h:6-13
 *   lossless_scan_workspace_bytes      prime_kernels/lossless_bf16/csrc/lossless_bf16.cu:107-112
 *   lossless_encode_layer              prime_kernels/lossless_bf16/csrc/lossless_bf16.cu:114-144
 *   lossless_decode_layer              prime_kernels/lossless_bf16/csrc/lossless_bf16.cu:146-154
 *   lossless_write_descriptor          prime_kernels/lossless_bf16/csrc/lossless_bf16.cu:156-168
 *   decode360_lossless                 prime_kernels/decode_megakernel_360m_lossless/csrc/
 *                                      block360_kernel.inc:639-649
 * pk_decode_lossless is this library's superset (pk_decode's LM head and layer count) and has no
 * single counterpart.
 *
 * Format (one [5120, 960] bf16 gate_up matrix per layer, chunks of 8 consecutive weights of a
 * row, 120 per row, numbered row-major):
 *   plane      uint8  [5120, 960]   sign bit and 7 mantissa bits of every weight
 *   headers    uint32 [5120, 120]   min exponent << 24 | eight 3-bit exponent deltas, or
 *                                   0xFF << 24 | ordinal for an escaped chunk (exponent spread
 *                                   above 7, or every exponent 255)
 *   raw        uint16 [capacity*8]  the 8 original words of escaped chunk `ordinal`
 *   row_offsets uint32 [5121]       escaped chunks before each row
 *   enabled    uint32               1 when every escape fit in `raw`; 0 sends the decode step to
 *                                   the dense matrix for that layer
 */
#ifndef PRIME_LOSSLESS_H
#define PRIME_LOSSLESS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

struct EncodedGULayer {
  const uint8_t* plane;
  const uint32_t* headers;
  const uint16_t* raw;
  const uint32_t* row_offsets;
  const uint32_t* enabled;
};

/* Bytes of the `scan_workspace` lossless_encode_layer needs (per-row escape counts). */
size_t lossless_scan_workspace_bytes(void);

/* Encode one bf16 [5120, 960] matrix asynchronously on `stream` (a hipStream_t).  flags [614400]
 * receives 1 for escaped chunks, prefix [614400] the inclusive count of escaped chunks up to each
 * chunk (prefix[614399] is the total), row_offsets [5121] as above.  Escapes with ordinal >=
 * `capacity` are not stored and set *enabled = 0.  All pointers device memory, 16-byte aligned. */
int lossless_encode_layer(const void* input, void* plane, void* headers, void* raw, void* row_offsets,
                          void* flags, void* prefix, void* scan_workspace, size_t scan_workspace_bytes,
                          void* enabled, uint32_t capacity, void* stream);

/* Decode one encoded matrix back to bf16 [5120, 960] (bit-exact).  Only for a matrix whose enabled
 * flag is 1: a disabled one has escape ordinals past its table. */
int lossless_decode_layer(const void* plane, const void* headers, const void* raw, void* output, void* stream);

/* Write entry `index` of a device table of EncodedGULayer (stream-ordered). */
int lossless_write_descriptor(void* table, int index, const void* plane, const void* headers, const void* raw,
                              const void* row_offsets, const void* enabled, void* stream);

/* decode360 with the gate/up weights of every enabled layer read from `encoded_gu_table` (a device
 * table [32] of EncodedGULayer; NULL: all dense).  Bit-identical to decode360 on the dense weights.
 * Batches of 2 or more read the dense matrices. */
int decode360_lossless(void* stream, int B, const void* input_ids, const void* embed, const void* final_norm,
                       const void* positions, const void* seq_lens, const void* block_table, int bt_stride,
                       const void* slot_mapping, const void* layers, void* const* kv, long long k_off,
                       long long v_off, long long block_stride, long long token_stride, long long head_stride,
                       int block_size, const void* cos_sin, int cs_fp32, void* out_hidden, void* layer_outputs,
                       void* scratch, size_t scratch_bytes, void* debug, size_t debug_bytes, int max_seq_len,
                       int debug_layer_index, const void* encoded_gu_table);

/* pk_decode (prime_decode.h) for SmolLM2-360M with the encoded gate/up table. */
int pk_decode_lossless(void* stream, int model, int B, int n_layers, const void* input_ids, int ids_i64,
                       const void* embed, const void* final_norm, const void* positions, const void* seq_lens,
                       const void* block_table, int bt_stride, const void* slot_mapping, const void* layers,
                       void* const* kv, long long k_off, long long v_off, long long block_stride,
                       long long token_stride, long long head_stride, int block_size, const void* cos_sin,
                       int cs_fp32, void* out_hidden, void* layer_outputs, void* out_ids, void* out_logits,
                       void* scratch, size_t scratch_bytes, int max_seq_len, const void* encoded_gu_table);

#ifdef __cplusplus
}
#endif

#endif /* PRIME_LOSSLESS_H */
