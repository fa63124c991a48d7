// Device-side definitions shared by the decode kernels (decode_megakernel.hip: the general
// batch-1 and batched kernels; decode_sr.hip: the split-role batch-1 kernel): model geometry,
// launch constants, the kernel parameter block, bf16 / cross-lane / memory-scope helpers, LDS-DMA,
// diagnostic timestamps and bounded waits.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "../../include/prime_decode.h"
#include "../../include/prime_lossless.h"

namespace pk {

// Diagnostic timestamp buffer for the next launches (pk_set_trace); one definition for the library.
inline unsigned long long* g_trace = nullptr;

template <int H_, int NH_, int KVH_, int I_, int L_>
struct Geom {
  static constexpr int H = H_, NH = NH_, KVH = KVH_, D = 64, I = I_, L = L_, V = 49152;
  static constexpr int QKV = (NH + 2 * KVH) * D;
  static constexpr int GQA = NH / KVH;
  static constexpr int WF = 0;  // projection weights: 0 bf16, 1 MXFP8 (e4m3 + e8m0 scale per 32)
  static_assert(GQA == 3, "SmolLM2 uses 3 query heads per KV head");
};
using G360 = Geom<960, 15, 5, 2560, 32>;   // decode_megakernel_360m/__init__.py:27-35
using G135 = Geom<576, 9, 3, 1536, 30>;    // decode_megakernel/__init__.py:37-43
// SmolLM2-360M with MXFP8 projection weights (embedding / LM head and norms stay bf16).
struct G360Q : G360 {
  static constexpr int WF = 1;
};

// E8M0 scale code -> fp32 2^(s-127) (code 0 is the fp32 denormal 2^-127; 255 is NaN).
__device__ __forceinline__ float e8m0_f32(uint32_t s) {
  return __uint_as_float(s == 0 ? 0x00400000u : s == 255 ? 0x7fc00000u : s << 23);
}

// MXFP8 scales are stored one byte per 32 weights, each row padded to a multiple of 16 bytes so
// that every row segment a workgroup streams starts and ends on a 16-byte boundary.
__host__ __device__ constexpr int scale_stride(int K) { return ((K / 32 + 15) / 16) * 16; }

constexpr int NWG = 256;                 // persistent workgroups (one per CU)
#ifndef PK_PRODUCER_WAVES
#define PK_PRODUCER_WAVES 4
#endif
#ifndef PK_DMA_DEPTH
#define PK_DMA_DEPTH 4                   // general batch-1 kernel (MXFP8 ctx 8192: 4 / 3 / 8 = 1,279 / 1,278 / 1,275 tok/s)
#endif
#ifndef PK_POLL_SLEEP
#define PK_POLL_SLEEP 0                  // s_sleep units (64 clocks) between polls (0: -0.2% at batch 1, -0.9% at 16, against 1)
#endif
constexpr int NPW = PK_PRODUCER_WAVES;   // producer waves per workgroup (LDS-DMA issue is per-wave bound)
constexpr int NCW = 4;                   // consumer waves per workgroup
constexpr int NCT = 64 * NCW;            // consumer threads
constexpr int WG_THREADS = 64 * (NPW + NCW);
constexpr uint32_t RING = 128u * 1024u;  // LDS ring bytes (power of two)
constexpr uint32_t PKT = 1024;           // one LDS-DMA instruction: 64 lanes x 16 B
constexpr int DEPTH = PK_DMA_DEPTH;      // packets in flight per producer wave (batch 1)
// The batched kernel: a producer wave marks a packet as landed only once DEPTH_B - 1 newer ones
// are issued (or its queue drains), so a deep queue hides the end of each K or V segment from the
// consumers until the next segment has streamed; at config 4 depth 32 / 16 / 8 / 4 / 3 / 2 gave
// 7,695 / 7,709 / 7,892 / 8,362 / 8,409 / 8,401 tok/s.
#ifndef PK_B_DOWN_SPLIT
#define PK_B_DOWN_SPLIT 1                // batched down: two workgroups per row group, half the sequences each
#endif
#ifndef PK_DMA_DEPTH_B
#define PK_DMA_DEPTH_B 3
#endif
constexpr int DEPTH_B = PK_DMA_DEPTH_B;
constexpr int TC_MAX = 288;              // max cached tokens per attention chunk (72 KB of K/V)
// Batch-1 chunking of a KV head's cached tokens: chunks of up to TC_LONG tokens, but at least
// C_SHORT chunks of at least TC_SHORT tokens while the context allows (measured at 360M batch 1:
// more chunks shorten each chunk's work, and the exchanges between a head's chunks, through its
// XCD's L2, cost little more with every chunk as long as the leader polls all partial records
// in one batch)
constexpr int TC_LONG = 128;
constexpr int TC_SHORT = 64;
constexpr int C_SHORT = 16;
constexpr int LM_ROWS = 16;              // LM-head rows per ring segment (batched kernel: one MFMA tile)
constexpr int LM_ROWS_G = 24;            // LM-head rows per ring segment (general batch-1 kernel), 6 per wave
constexpr int MAX_B = 16;                // exchange-buffer slots per layer
constexpr int REC_WORDS = 3 * 64;        // attention partial: 3 heads x sum(p.v)[64], 64-bit words
constexpr int STAT_WORDS = 6;            // chunk softmax statistics: 3 heads x (max, sum), 64-bit words
constexpr uint32_t SPIN_LIMIT = 1u << 22;
constexpr int kMaxSeq = 12288;          // tokens per sequence (block_table capacity)

// Workspace header words.  The abort word holds the epoch of the step that gave up a bounded wait
// (0: none), so a later step, with a later epoch, is not affected by it.
constexpr int HDR_EPOCH = 0;
constexpr int HDR_ABORT = 1;
constexpr int HDR_ABORT_WHERE = 2;
constexpr size_t HDR_WORDS = 64;
// The scratch the decode entry points require (present and at least this large; unused).
constexpr size_t SCRATCH_BYTES = 256;

struct LayerW {
  const void* norm1;        // [H] bf16
  const void* qkv;          // [(NH+2KVH)*D, H]: q rows, then k rows, then v rows (bf16 or e4m3)
  const void* o;            // [H, H]
  const void* norm2;        // [H] bf16
  const void* gate_up;      // [2I, H]: gate rows, then up rows
  const void* down;         // [H, I]
  const uint8_t* qkv_s;     // MXFP8 only: e8m0 scales [rows, scale_stride(K)] of the matrix above
  const uint8_t* o_s;
  const uint8_t* gate_up_s;
  const uint8_t* down_s;
};

struct Params {
  const void* const* layers;   // [L][6] bf16 (norm1, qkv, o, norm2, gate_up, down) or [L][10] MXFP8
                               // (norm1, qkv, qkv_s, o, o_s, norm2, gate_up, gate_up_s, down, down_s)
  const uint16_t* embed;       // [V, H]
  const uint16_t* final_norm;  // [H]
  const void* input_ids;       // [B] int32 or int64 (ids_i64)
  void* const* kv;             // [L] paged caches
  const int64_t* positions;    // [B]
  const int32_t* seq_lens;     // [B] tokens attended, including the new one
  const int32_t* block_table;  // [B, bt_stride]
  const int64_t* slot_mapping; // [B]
  const void* cos_sin;         // [max_pos, D]: cos [0, D/2), sin [D/2, D)
  uint16_t* out_hidden;        // [B, H] final-normed hidden
  uint16_t* layer_outputs;     // optional [L, B, H]
  uint16_t* out_logits;        // optional [B, V]
  int64_t* out_ids;            // optional [B] greedy ids
  uint32_t* ws;                // workspace (header + exchange buffers), zero-initialised once
  long long k_off, v_off, block_stride, token_stride, head_stride;  // elements
  int bt_stride;
  int cs_fp32;
  int B;
  int n_layers;
  int lm_head;                 // 1: run the LM head + argmax
  int max_seq;                 // block_table capacity in tokens (seq_lens are clamped to it)
  int ids_i64;
  unsigned long long* trace;   // optional per-phase timestamps (diagnostics)
  uint32_t trace_lds;          // LDS byte offset of the launch's timestamp buffer (when tracing)
  uint32_t* xws;               // optional: batch-1 attention records in ordinary device memory
  const EncodedGULayer* encoded_gu;  // optional [L] lossless gate/up encodings (batch-1 bf16 kernel)
  uint16_t* debug;             // optional per-stage capture (Dbg layout), batch <= 2
  int debug_layer;             // layer whose attention internals are captured (-1: none)
  const uint16_t* input_hidden;  // optional [B, H]: layer 0's input instead of the embedding rows
  uint32_t* host_status;       // host-visible [2]: epoch and wait site of the last step that gave up a wait
  int h_dim;                   // hidden size of the model (for the poisoned hidden state)
  int l2_records;              // 0: batch-1 attention records stay in the uncached workspace
  uint32_t skew;               // != 0: seed of the arrival-skew test's delays before each publish
  int sr_max_s;                // > 0: split-role kernels were launched for this step and do contexts up
                               // to sr_max_s tokens (the general batch-1 kernel then leaves them)
  int sr_min_s;                // a split-role kernel does contexts in (sr_min_s, sr_max_s] (its launch's
                               // copy of the parameters; the narrow layout takes the short ones)
};

// Split-role batch-1 kernel (decode_sr.hip): launch, the sizes of its workspace regions (bytes), and
// the longest context it takes (tokens attended, new one included; 0: not available for the model).
// `wide`: 0 the narrow layout, 1 the wide one, 2 and 3 the narrow layout with fewer attention chunks
// for the shorter contexts (135M: 4 chunks up to 1,025 tokens, 6 up to 1,537).
__attribute__((visibility("hidden"))) int sr_launch(int model, int wf, int wide, const Params& p, uint32_t* region,
                                                 uint32_t* local, hipStream_t stream, int cooperative);
// region: the largest over every compiled layout (all != 0) or over the narrow bf16 ones
// (pk_decode_noalloc); local: the group-A records of the narrow (wide == 0) or the wide layouts.
__attribute__((visibility("hidden"))) size_t sr_region_bytes(int all);
__attribute__((visibility("hidden"))) size_t sr_local_bytes(int wide);
__attribute__((visibility("hidden"))) int sr_max_seq(int model, int wide);

// ------------------------------------------------------------------------------------------------
// Scalar and cross-lane helpers
// ------------------------------------------------------------------------------------------------

__device__ __forceinline__ float bf2f(uint32_t b) { return __uint_as_float(b << 16); }
__device__ __forceinline__ float bf_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf_hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
// fp32 -> bf16, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
__device__ __forceinline__ float rnd(float f) { return float((__bf16)f); }
// Two fp32 -> packed bf16 pair {lo = a, hi = b}, one instruction.
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  const bf16x2 v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}
// Operand and accumulator types of v_mfma_f32_16x16x32_bf16.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// acc + a.lo*b.lo + a.hi*b.hi over packed bf16 pairs (v_dot2_f32_bf16).
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), acc, false);
}

// DPP move: lanes whose source is outside the row, or that the row/bank masks disable, get `old`.
template <int CTRL, int RM = 0xf, int BM = 0xf>
__device__ __forceinline__ float dpp(float old, float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old),
                                                               __builtin_bit_cast(int, v), CTRL, RM, BM, false));
}
__device__ __forceinline__ float lane63(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
// Wave64 sum / max through DPP row shifts and row broadcasts; the result is uniform.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<0x111>(0.f, v);            // row_shr:1
  v += dpp<0x112>(0.f, v);            // row_shr:2
  v += dpp<0x114, 0xf, 0xe>(0.f, v);  // row_shr:4, banks 1-3
  v += dpp<0x118, 0xf, 0xc>(0.f, v);  // row_shr:8, banks 2-3
  v += dpp<0x142, 0xa>(0.f, v);       // row_bcast:15 into rows 1, 3
  v += dpp<0x143, 0xc>(0.f, v);       // row_bcast:31 into rows 2, 3
  return lane63(v);
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<0x111>(v, v));
  v = fmaxf(v, dpp<0x112>(v, v));
  v = fmaxf(v, dpp<0x114, 0xf, 0xe>(v, v));
  v = fmaxf(v, dpp<0x118, 0xf, 0xc>(v, v));
  v = fmaxf(v, dpp<0x142, 0xa>(v, v));
  v = fmaxf(v, dpp<0x143, 0xc>(v, v));
  return lane63(v);
}
// Lane swaps of gfx950: swap32 exchanges lanes 32-63 of `a` with lanes 0-31 of `b`; swap16 exchanges
// the odd 16-lane rows of `a` with the even rows of `b` (v_permlane32_swap_b32 / v_permlane16_swap_b32).
__device__ __forceinline__ void swap32(float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
                                                  false, false);
  // through plain integers: __builtin_bit_cast of r[1] itself reads element 0 with this compiler
  const uint32_t r0 = r[0], r1 = r[1];
  a = __uint_as_float(r0);
  b = __uint_as_float(r1);
}
__device__ __forceinline__ void swap16(float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
                                                  false, false);
  // through plain integers: __builtin_bit_cast of r[1] itself reads element 0 with this compiler
  const uint32_t r0 = r[0], r1 = r[1];
  a = __uint_as_float(r0);
  b = __uint_as_float(r1);
}
// Totals of N per-lane values over the wave (N <= 8), returned uniform, in about 2.5 N + 8 VALU
// instructions: a transposed butterfly.  The cross-half swap leaves value 2i's partial sums in lanes
// 0-31 and value 2i+1's in lanes 32-63 of one register; the cross-row swap then leaves one value per
// 16-lane row (rows 0-3 holding values 4j, 4j+2, 4j+1, 4j+3); four full-row DPP steps finish each row.
template <bool MAX>
__device__ __forceinline__ float comb(float a, float b) { return MAX ? fmaxf(a, b) : a + b; }
template <int N, bool MAX = false>
__device__ __forceinline__ void wave_rows(float (&v)[N]) {
  static_assert(N >= 1 && N <= 8, "up to 8 values");
  constexpr int P = (N + 1) / 2, Q = (P + 1) / 2;
  float a[P], b[Q];
#pragma unroll
  for (int i = 0; i < P; ++i) {
    float x = v[2 * i], y = 2 * i + 1 < N ? v[2 * i + 1] : v[2 * i];
    swap32(x, y);
    a[i] = comb<MAX>(x, y);
  }
#pragma unroll
  for (int j = 0; j < Q; ++j) {
    float x = a[2 * j], y = 2 * j + 1 < P ? a[2 * j + 1] : a[2 * j];
    swap16(x, y);
    b[j] = comb<MAX>(x, y);
  }
#pragma unroll
  for (int j = 0; j < Q; ++j) b[j] = comb<MAX>(b[j], dpp<0x128>(0.f, b[j]));  // row_ror:8
#pragma unroll
  for (int j = 0; j < Q; ++j) b[j] = comb<MAX>(b[j], dpp<0x124>(0.f, b[j]));  // row_ror:4
#pragma unroll
  for (int j = 0; j < Q; ++j) b[j] = comb<MAX>(b[j], dpp<0x4e>(0.f, b[j]));   // quad_perm [2,3,0,1]
#pragma unroll
  for (int j = 0; j < Q; ++j) b[j] = comb<MAX>(b[j], dpp<0xb1>(0.f, b[j]));   // quad_perm [1,0,3,2]
  auto lane_of = [](float f, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, f), l));
  };
#pragma unroll
  for (int j = 0; j < Q; ++j) {
    v[4 * j] = lane_of(b[j], 0);
    if (4 * j + 1 < N) v[4 * j + 1] = lane_of(b[j], 32);
    if (4 * j + 2 < N) v[4 * j + 2] = lane_of(b[j], 16);
    if (4 * j + 3 < N) v[4 * j + 3] = lane_of(b[j], 48);
  }
}

// Total (sum, or max for MAX) of a value over the four 16-lane rows of a wave, for each of the 16
// columns; every lane gets its column's total (one cross-half and one cross-row swap).
template <bool MAX>
__device__ __forceinline__ float column_total(float v) {
  float a = v, b = v;
  swap32(a, b);
  v = comb<MAX>(a, b);
  a = v;
  b = v;
  swap16(a, b);
  return comb<MAX>(a, b);
}

// DPP row shifts by 3i lanes (i < 5, a compile-time constant after unrolling): row_shr moves lane
// c - 3i to lane c, row_shl lane c + 3i to lane c, within each 16-lane row (lanes with no source get
// -inf for the max variant, 0 otherwise).
template <bool NEG_INF>
__device__ __forceinline__ float dpp_shr3(int i, float v) {
  const float o = NEG_INF ? -INFINITY : 0.f;
  switch (i) {
    case 1: return dpp<0x113>(o, v);
    case 2: return dpp<0x116>(o, v);
    case 3: return dpp<0x119>(o, v);
    case 4: return dpp<0x11c>(o, v);
    default: return v;
  }
}
__device__ __forceinline__ uint32_t dpp_shl3u(int i, uint32_t v) {
  const float f = __uint_as_float(v);
  switch (i) {
    case 1: return __float_as_uint(dpp<0x103>(0.f, f));
    case 2: return __float_as_uint(dpp<0x106>(0.f, f));
    case 3: return __float_as_uint(dpp<0x109>(0.f, f));
    case 4: return __float_as_uint(dpp<0x10c>(0.f, f));
    default: return v;
  }
}
// Per-head totals (sum, or max for MAX) of the compacted layout: lane c of each row holds a value of
// head c % 3 (c < 15; lane 15 must hold the identity).  Lanes c, c-3, c-6, c-9, c-12 are combined
// within the row (lanes 12-14 then hold the row's totals of heads 0-2), the four rows are combined,
// and the three totals come back wave-uniform.
template <bool MAX>
__device__ __forceinline__ void head_totals(float v, float (&out)[3]) {
  v = comb<MAX>(v, dpp_shr3<MAX>(1, v));
  v = comb<MAX>(v, dpp_shr3<MAX>(2, v));
  v = comb<MAX>(v, dpp_shr3<MAX>(4, v));
  v = column_total<MAX>(v);
#pragma unroll
  for (int h = 0; h < 3; ++h)
    out[h] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 12 + h));
}

// wave_max / wave_sum of N values at once: the same steps per value, the N chains interleaved so
// that each DPP step's wait states are filled by the other chains instead of s_nop.
template <int N>
__device__ __forceinline__ void wave_max_n(float (&v)[N]) {
#pragma unroll
  for (int k = 0; k < N; ++k) v[k] = fmaxf(v[k], dpp<0x111>(v[k], v[k]));
#pragma unroll
  for (int k = 0; k < N; ++k) v[k] = fmaxf(v[k], dpp<0x112>(v[k], v[k]));
#pragma unroll
  for (int k = 0; k < N; ++k) v[k] = fmaxf(v[k], dpp<0x114, 0xf, 0xe>(v[k], v[k]));
#pragma unroll
  for (int k = 0; k < N; ++k) v[k] = fmaxf(v[k], dpp<0x118, 0xf, 0xc>(v[k], v[k]));
#pragma unroll
  for (int k = 0; k < N; ++k) v[k] = fmaxf(v[k], dpp<0x142, 0xa>(v[k], v[k]));
#pragma unroll
  for (int k = 0; k < N; ++k) v[k] = fmaxf(v[k], dpp<0x143, 0xc>(v[k], v[k]));
#pragma unroll
  for (int k = 0; k < N; ++k) v[k] = lane63(v[k]);
}
template <int N>
__device__ __forceinline__ void wave_sum_n(float (&v)[N]) {
#pragma unroll
  for (int k = 0; k < N; ++k) v[k] += dpp<0x111>(0.f, v[k]);
#pragma unroll
  for (int k = 0; k < N; ++k) v[k] += dpp<0x112>(0.f, v[k]);
#pragma unroll
  for (int k = 0; k < N; ++k) v[k] += dpp<0x114, 0xf, 0xe>(0.f, v[k]);
#pragma unroll
  for (int k = 0; k < N; ++k) v[k] += dpp<0x118, 0xf, 0xc>(0.f, v[k]);
#pragma unroll
  for (int k = 0; k < N; ++k) v[k] += dpp<0x142, 0xa>(0.f, v[k]);
#pragma unroll
  for (int k = 0; k < N; ++k) v[k] += dpp<0x143, 0xc>(0.f, v[k]);
#pragma unroll
  for (int k = 0; k < N; ++k) v[k] = lane63(v[k]);
}
// Sum over each aligned group of 8 lanes; every lane of the group gets the group sum.
__device__ __forceinline__ float group8_sum(float v) {
  v += dpp<0xb1>(0.f, v);                  // quad_perm [1,0,3,2]
  v += dpp<0x4e>(0.f, v);                  // quad_perm [2,3,0,1]
  float t = dpp<0x104, 0xf, 0x5>(0.f, v);  // row_shl:4 into banks 0, 2
  t = dpp<0x114, 0xf, 0xa>(t, v);          // row_shr:4 into banks 1, 3
  return v + t;
}

// Device-scope (coherent across XCDs) accesses for exchange words.
__device__ __forceinline__ uint32_t ld_dev(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_dev64(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev64(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Plain 64-bit store (no cache-policy bits): through the write-through L1 into the XCD's L2, where
// device-scope loads from the same XCD see it.
__device__ __forceinline__ void st_l2(uint64_t* p, uint64_t v) {
  typedef __attribute__((address_space(1))) uint64_t g_u64;
  *(g_u64*)(p) = v;
}
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
// Stores into caller memory through a pointer read from LDS (the KV cache base): without the
// explicit global address space the compiler emits a flat store, which also counts on the LDS
// counter, so the wave's next wait for an LDS read would also wait for this store's completion.
typedef __attribute__((address_space(1))) u32x4 g_u32x4;
typedef __attribute__((address_space(1))) uint16_t g_u16;
__device__ __forceinline__ void st_global16(uint16_t* dst, uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  const u32x4 v = {a, b, c, d};
  *(g_u32x4*)(dst) = v;
}
__device__ __forceinline__ void st_global2(uint16_t* dst, uint16_t v) { *(g_u16*)(dst) = v; }
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff, 0x00020000);
}
// 16-byte device-scope load (sc1); each 32-bit word is read atomically.
__device__ __forceinline__ u32x4 ld_dev128(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, int(byte_off), 0, 16);
}

// LDS words shared between the waves of one workgroup.
__device__ __forceinline__ uint32_t ld_lds(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void st_lds(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// One LDS-DMA packet: lane i copies 16 bytes from `g` to LDS byte address m0 + 16*i.  Written as
// inline asm so the compiler does not force vmcnt(0) before the producer's LDS counter writes;
// the producer waits on vmcnt itself.
__device__ __forceinline__ void dma16(const void* g, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds_addr), "v"(g)
               : "memory", "m0");
}
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xc07f); }

// Diagnostic timestamps: TR_EVENTS per layer per workgroup, plus TR_TAIL at the end.  During the
// launch they are kept in LDS, past the kernel's own shared memory, as the low 32 bits of the
// 100 MHz clock, and written out as full 64-bit values when the workgroup ends: a global store
// per event would add its acknowledgement to the next wait on the wave's memory counter, and so
// stretch the phases being timed.
constexpr int TR_EVENTS = 40;
constexpr int TR_TAIL = 4;
constexpr int TR_LAYERS = 32;
constexpr uint32_t TRACE_LDS_BYTES = uint32_t(TR_LAYERS * TR_EVENTS + TR_TAIL) * 4u;
__device__ __forceinline__ uint32_t* trace_lds(const Params& p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_raw[];
  return reinterpret_cast<uint32_t*>(smem_raw + p.trace_lds);
}
__device__ __forceinline__ void trace_at(const Params& p, int layer, int ev, int n_layers) {
  if (p.trace) trace_lds(p)[layer * TR_EVENTS + ev] = uint32_t(wall_clock64());
}
__device__ __forceinline__ void trace_tail(const Params& p, int k) {
  if (p.trace) trace_lds(p)[p.n_layers * TR_EVENTS + k] = uint32_t(wall_clock64());
}
// Before the workgroup's first barrier: clear the buffer (0 = event not reached).
__device__ __forceinline__ void trace_begin(const Params& p) {
  if (p.trace)
    for (int i = threadIdx.x; i < p.n_layers * TR_EVENTS + TR_TAIL; i += blockDim.x) trace_lds(p)[i] = 0u;
}
// After the workgroup's last barrier: full timestamps, each the latest clock value with its low bits
// (the launch is far shorter than the 43 s the low 32 bits cover).
__device__ __forceinline__ void trace_end(const Params& p) {
  if (!p.trace) return;
  const uint64_t now = wall_clock64();
  const int n = p.n_layers * TR_EVENTS + TR_TAIL;
  const uint32_t* t = trace_lds(p);
  unsigned long long* out = p.trace + size_t(blockIdx.x) * size_t(n);
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const uint32_t lo = t[i];
    out[i] = lo ? now - uint64_t(uint32_t(uint32_t(now) - lo)) : 0ull;
  }
}

// ------------------------------------------------------------------------------------------------
// Bounded waits.  Every spin gives up after SPIN_LIMIT polls, or as soon as it sees that another
// wait of the same step gave up (the abort word holds that step's epoch), so a logic error or a
// workgroup that never arrives ends the launch instead of hanging the GPU.  The step's outputs
// are then poisoned by workgroup 0 (NaN hidden state and logits, ids -1) and the next call on the
// same workspace reports the failure.
// ------------------------------------------------------------------------------------------------

__device__ __forceinline__ void raise_abort(uint32_t* ws, uint32_t epoch, int where) {
  st_dev(ws + HDR_ABORT_WHERE, uint32_t(where));
  st_dev(ws + HDR_ABORT, epoch);
}
__device__ __forceinline__ bool aborted(const uint32_t* ws, uint32_t epoch) { return ld_dev(ws + HDR_ABORT) == epoch; }

struct Spin {
  uint32_t n = 0;
  uint32_t* ws;
  uint32_t epoch;
  int where;
  __device__ __forceinline__ Spin(uint32_t* ws_, uint32_t ep, int w) : ws(ws_), epoch(ep), where(w) {}
  // Returns false when the wait must be abandoned.
  __device__ __forceinline__ bool again() {
    ++n;
    if ((n & 127u) == 0) {
      if (aborted(ws, epoch)) return false;
      if (n >= SPIN_LIMIT) {
        raise_abort(ws, epoch, where);
        return false;
      }
    }
    __builtin_amdgcn_s_sleep(PK_POLL_SLEEP);
    return true;
  }
};

// Arrival-skew test (Params::skew != 0): before publishing exchange data, a workgroup sleeps a
// pseudo-random 0..23 x 512 cycles drawn from (seed, workgroup, layer, site), so values arrive in
// orders the hardware rarely produces on its own.  Results must not change.  Uniform per wave.
__device__ __forceinline__ void skew_delay(uint32_t seed, int wg, int l, int site) {
  if (seed == 0u) return;
  uint32_t h = seed * 0x9e3779b1u ^ uint32_t(wg) * 0x85ebca77u ^ uint32_t(l * 64 + site) * 0xc2b2ae3du;
  h ^= h >> 15;
  h *= 0x2c1b3c6du;
  h ^= h >> 12;
  for (uint32_t k = h % 24u; k > 0u; --k) __builtin_amdgcn_s_sleep(8);
}

// A layer's lossless gate/up encoding as this workgroup streams it (on = 0: dense gate/up): the
// plane / header / escape arrays, and for gate (0) and up (1) the first escape ordinal of the
// workgroup's rows and their number of escapes.
struct GUE {
  const uint8_t* plane;
  const uint32_t* hdr;
  const uint16_t* raw;
  uint32_t on;
  uint32_t first[2];
  uint32_t cnt[2];
};

// The 8 bf16 words (4 packed pairs) of a lossless chunk: plane bytes p (sign | mantissa) and the
// header's base exponent and 3-bit deltas give word_i = (p_i & 0x80) << 8 | (base + d_i) << 7 |
// (p_i & 0x7f) (prime_kernels/lossless_bf16/csrc/lossless_bf16.cu:94-101).  Per pair of words,
// in one register: v_perm copies plane bytes 2j, 2j+1 into both bytes of the low / high half, so
// one mask keeps each sign at bit 15 / 31 and each mantissa at bits 0-6 / 16-22; the pair's 6 delta
// bits d times 0x100080 is d << 7 | d << 20, whose bits 7-9 and 23-25 are the two deltas in
// exponent position; the base exponent is added to both halves at once.  No field overflows into
// the next: every exponent of a plain chunk is at most 254 + 7 < 256.
__device__ __forceinline__ uint4 lossless_chunk(uint2 p, uint32_t h) {
  const uint32_t base7 = (h >> 24) * 0x00800080u;
  uint32_t out[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t t = __builtin_amdgcn_perm(0u, j < 2 ? p.x : p.y, (j & 1) ? 0x03030202u : 0x01010000u);
    const uint32_t d = __builtin_amdgcn_ubfe(h, 6 * j, 6);
    const uint32_t e7 = (__umul24(d, 0x100080u) & 0x03800380u) + base7;
    out[j] = (t & 0x807F807Fu) | e7;
  }
  return make_uint4(out[0], out[1], out[2], out[3]);
}

// Index field values of a workgroup's end record: one of its waits gave up / no LM head.
constexpr uint32_t LM_DEAD = 0xffffu, LM_NONE = 0xfffeu;
constexpr int G_HMAX = 960;

// Workgroup 0, when a step gave up a wait: the abort word (if no wait raised it), the host-visible
// report {epoch, wait site}, and sequence b's hidden state set to NaN.  Called by every consumer
// thread `ct` of workgroup 0.  The callers then also set every logits row of the step to NaN; a
// workgroup still in its last phases when workgroup 0 gave up waiting for it can store its own rows
// after that, so only the token ids (-1) and the hidden state are guaranteed to be poisoned.
__device__ __forceinline__ void step_failed(const Params& p, uint32_t epoch, int ct, int b) {
  if (ct == 0) {
    if (ld_dev(p.ws + HDR_ABORT) != epoch) raise_abort(p.ws, epoch, 25);
    if (p.host_status) {
      __hip_atomic_store(p.host_status + 1, ld_dev(p.ws + HDR_ABORT_WHERE), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      __hip_atomic_store(p.host_status, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
  }
  for (int i = ct; i < G_HMAX; i += 256) if (i < p.h_dim) p.out_hidden[size_t(b) * p.h_dim + i] = 0x7fc0;
}

// Step epoch: read from the workspace header at the start of the launch; workgroup 0 stores it
// back once every workgroup has reported its end.  Epoch 0 is skipped (a zeroed workspace).
__device__ __forceinline__ uint32_t step_epoch(const uint32_t* ws) {
  const uint32_t e = ld_dev(ws + HDR_EPOCH) + 1u;
  return e == 0u ? 1u : e;
}

// Balanced split of n items over `parts`: part i gets [split_lo(n, parts, i), split_lo(n, parts, i + 1)).
__host__ __device__ constexpr int split_lo(int n, int parts, int i) { return int((long long)n * i / parts); }
// The qkv vector in slot order.  Its q and k parts are laid out by RoPE pair: slots 2p and 2p + 1
// hold dims d and d + 32 (d = p % 32) of head p / 32 (the q heads, then the k heads), so that the
// workgroup producing a unit of slots holds both halves of its pairs and applies RoPE itself;
// the v part is in row order.  qkv_row(s) is the projection row of slot s.
template <class G>
__device__ __forceinline__ int qkv_row(int s) {
  constexpr int ROPE = (G::NH + G::KVH) * 64;
  if (s >= ROPE) return s;
  const int pr = s >> 1;
  return (pr >> 5) * 64 + (pr & 31) + 32 * (s & 1);
}

// Bytes of a ring segment rounded up to whole LDS-DMA packets.
__host__ __device__ constexpr uint32_t pad_pkt(uint32_t b) { return (b + PKT - 1) & ~(PKT - 1); }

// ------------------------------------------------------------------------------------------------
// GEMV operands
// ------------------------------------------------------------------------------------------------

// A lane owns the 16-byte weight chunks j = lane + 64*c of every row; a chunk holds EPC weights
// (8 bf16, or 16 e4m3 values), i.e. EPC/8 blocks of 8 activations.
template <int K, int EPC = 8>
struct Chunks {
  static constexpr int CH = K / EPC;
  static constexpr int CPL = (CH + 63) / 64;
  static constexpr int SUB = EPC / 8;
};
// A lane's activation (or norm-weight) operand for K-long rows of chunk size EPC: 8 values per uint4.
template <int K, int EPC = 8>
using XChunks = uint4[Chunks<K, EPC>::CPL][EPC / 8];

// Activation chunks of a lane from LDS as packed bf16 pairs: plain (the values are bf16 already),
// or RMS-normalised with LlamaRMSNorm rounding y = bf16(w * bf16(x * rs)) (modeling_llama.py:62-67).
template <int K, int EPC, bool NORM>
__device__ __forceinline__ void load_x(XChunks<K, EPC>& x, const float* xs,
                                       const XChunks<K, EPC>& nw, float rs, int lane) {
#pragma unroll
  for (int c = 0; c < Chunks<K, EPC>::CPL; ++c) {
    const int ch = lane + 64 * c;
#pragma unroll
    for (int i = 0; i < EPC / 8; ++i) {
      if (ch < Chunks<K, EPC>::CH) {
        const float* src = xs + ch * EPC + 8 * i;
        const float4 a = *reinterpret_cast<const float4*>(src);
        const float4 b = *reinterpret_cast<const float4*>(src + 4);
        const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        uint32_t o[4];
        if (NORM) {
          const uint32_t u[4] = {nw[c][i].x, nw[c][i].y, nw[c][i].z, nw[c][i].w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t t = pack2(v[2 * e] * rs, v[2 * e + 1] * rs);
            o[e] = pack2(bf_lo(u[e]) * bf_lo(t), bf_hi(u[e]) * bf_hi(t));
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = pack2(v[2 * e], v[2 * e + 1]);
        }
        x[c][i] = make_uint4(o[0], o[1], o[2], o[3]);
      } else {
        x[c][i] = make_uint4(0, 0, 0, 0);
      }
    }
  }
}

__device__ __forceinline__ float rms_scale(float sumsq, int n) {
  const float mean = sumsq / float(n);
  return 1.0f / sqrtf(mean + 1e-5f);
}

}  // namespace pk
