// SmolLM2 single-token decode step as one persistent HIP kernel per step for gfx950 (MI355X): the
// general batch-1 kernel (decode_kernel) and the batched kernel (decode_kernel_b); the split-role
// batch-1 kernel is in decode_sr.hip.  The launch is an ordinary hipLaunchKernel of one workgroup
// per CU, which relies on all 256 workgroups being resident at once (true on an otherwise idle
// device: a workgroup waiting for one that is not resident gives up after its bounded wait and the
// step comes back poisoned and reported); PK_LAUNCH=cooperative or pk_set_option(PK_OPT_COOPERATIVE)
// launches with hipLaunchCooperativeKernel instead, which guarantees co-residency for 18 us more per
// step (measured at batch 1, context 1024; the same bits either way).
//
// One workgroup per CU (256), 8 wave64s each:
//   waves 0..3  producers: stream this workgroup's share of every weight matrix (and its KV-cache
//               chunk) from HBM into a 128 KB LDS ring (64 KB in the batched kernel) with LDS-DMA
//               loads (global_load_lds_dwordx4), DEPTH (batched: DEPTH_B) 1 KB packets in flight
//               per wave, running ahead of the dependency chain because weights and cached K/V do
//               not depend on activations.
//   waves 4..7  consumers: pull their rows from the ring into VGPRs, wait for the phase input,
//               compute, publish the phase output.
//
// Phases per layer (the reference's eight grid barriers per layer, block360_kernel.inc:96-803,
// become data-flow edges):
//   P1 RMSNorm(x) + QKV GEMV             -> qkv (pre-RoPE, bf16)
//   P2 RoPE + GQA attention over KV chunks: chunk softmax statistics are exchanged so every
//      probability is rounded with the global max and sum, as HF does; chunk leaders add the
//      fp32 partial sums of p.v                  -> attn (bf16)
//   P3 O GEMV + residual                  -> h1
//   P4 RMSNorm(h1) + gate/up GEMV + SwiGLU -> act
//   P5 down GEMV + residual               -> x (layer output)
//   then final RMSNorm + tied LM head GEMV with per-workgroup argmax, and a 256-way argmax.
//
// Inter-workgroup exchange: no counters, no fences.  In the general kernel every exchanged value
// is written as a 64-bit word {bf16 or fp32 value, tag32} with device-scope relaxed atomic stores,
// into a buffer owned by one (layer, phase, sequence).  Readers poll those words with device-scope
// (sc1) loads until every tag equals this step's epoch, so the data arrives with the "ready"
// signal in one round trip.  The batched kernel instead writes each phase output as a plain
// [B][K] bf16 array with sc1 2-byte stores, then each workgroup raises one tagged flag per
// (phase, layer) after its stores have completed; readers poll the flags, then copy the array.
// The epoch is a device counter bumped by workgroup 0 at the end of every step.
#include <hip/hip_runtime.h>

#include <mutex>
#include <vector>

#include <cstddef>
#include <cstdint>


#include "pk_common.h"

namespace pk {


// ------------------------------------------------------------------------------------------------
// Geometry and launch constants
// ------------------------------------------------------------------------------------------------

// Per-stage debug capture, the reference's layout (block360_kernel.inc:1-20), bf16 elements:
// per layer [norm1, qkv, attn, o, h1, norm2, gate, up, silu, act, down, out], each [2][N] (rows for
// sequences 0 and 1); then, for layer `debug_layer` only, the rotated queries [2][H], bf16(q.k)
// [2][NH][8192], the scaled scores and the probabilities (same shape) and the P.V output [2][H].
// Positions from 8192 on are not recorded.
template <class G>
struct Dbg {
  static constexpr size_t MB = 2, SEQ = 8192;
  static constexpr size_t NORM1 = 0, QKV = NORM1 + MB * G::H, ATTN = QKV + MB * G::QKV, O = ATTN + MB * G::H,
                          H1 = O + MB * G::H, NORM2 = H1 + MB * G::H, GATE = NORM2 + MB * G::H,
                          UP = GATE + MB * G::I, SILU = UP + MB * G::I, ACT = SILU + MB * G::I,
                          DOWN = ACT + MB * G::I, OUT = DOWN + MB * G::H, LAYER = OUT + MB * G::H;
  static constexpr size_t STAGES = size_t(G::L) * LAYER, AQ = STAGES, AQK = AQ + MB * G::H,
                          ASC = AQK + MB * G::NH * SEQ, APR = ASC + MB * G::NH * SEQ, APV = APR + MB * G::NH * SEQ,
                          TOTAL = APV + MB * G::H;
  __device__ static size_t head_pos(int b, int head, int pos) { return (size_t(b) * G::NH + head) * SEQ + pos; }
};


// Exchange-buffer layout (32-bit words).  The per-layer vectors (qkv, attn, h1, act, x) of tagged
// bf16 words are stored line-interleaved: 64-byte line k of vector (kind, layer, b) is line slot
// (b * XLINES + k) * XSLOTS + layer * NKIND + kind, so the consecutive lines of one vector are
// XSLOTS * 64 bytes apart (10 KB for 32 layers) and spread over the HBM channels instead of
// concentrating every reader's polls on the one or two channels a contiguous vector would hit.
// The batch-1 kernel writes each exchange word to XREP copies, in the sequence slots 0..XREP-1 of
// the vector (unused at batch 1), and workgroup i polls copy i mod XREP: every 64-byte line is then
// polled by NWG / XREP workgroups instead of all of them.  A line polled by every workgroup queues
// NWG requests at its memory channel each polling round, which made one round of uncached loads
// take ~0.75 us inside the step.  Measured at 360M batch 1: 4 copies slightly ahead of 8, 16
// behind (the extra stores cost more than the shorter queues save).
enum XKind { X_QKV, X_ATTN, X_H1, X_ACT, X_X, NKIND };
constexpr int XREP = 4;
static_assert(XREP <= MAX_B && NWG % XREP == 0, "copies live in the sequence slots");
template <class G>
struct WS {
  static constexpr int XSLOTS = G::L * NKIND;
  static constexpr int XMAX = G::QKV > G::I ? (G::QKV > G::H ? G::QKV : G::H) : (G::I > G::H ? G::I : G::H);
  static constexpr int XLINES = XMAX / 8;  // 64-byte lines of 8 words {bf16 value, tag32}
  static_assert(G::QKV % 8 == 0 && G::H % 8 == 0 && G::I % 8 == 0 && (G::H + G::KVH * 64) % 8 == 0,
                "vector segments start on 64-byte lines");
  static constexpr size_t X0 = HDR_WORDS;
  static constexpr size_t XWORDS = size_t(MAX_B) * XLINES * XSLOTS * 16;
  static constexpr size_t REC0 = X0 + XWORDS;
  static constexpr size_t REC_LAYER = size_t(NWG) * REC_WORDS * 2;
  static constexpr size_t STAT0 = REC0 + REC_LAYER * G::L;
  static constexpr size_t STAT_LAYER = size_t(NWG) * STAT_WORDS * 2;
  static constexpr size_t LM0 = STAT0 + STAT_LAYER * G::L;
  // per-workgroup {XCC id, tag32} words: where the batch-1 attention workgroups really run
  static constexpr size_t XCC0 = LM0 + size_t(MAX_B) * NWG * 2;
  static constexpr size_t TOTAL = XCC0 + size_t(NWG) * 2;
  __device__ static size_t xcc(int wg) { return XCC0 + size_t(wg) * 2; }
  // 32-bit word offset of the 64-bit word {bf16 value, tag32} of element i of vector (kind, layer l, sequence b)
  __device__ static size_t xw(int kind, int l, int b, int i) {
    return X0 + (((size_t(b) * XLINES + size_t(i >> 3)) * XSLOTS + size_t(l) * NKIND + kind) * 8 + size_t(i & 7)) * 2;
  }
  __device__ static size_t rec(int l, int item) { return REC0 + l * REC_LAYER + size_t(item) * REC_WORDS * 2; }
  // The batch-1 attention records (partials and statistics, REC0 .. LM0) can live in a separate
  // buffer of XREC_WORDS words at the same relative offsets.
  static constexpr size_t XREC_WORDS = LM0 - REC0;
  __device__ static size_t stat(int l, size_t item) { return STAT0 + l * STAT_LAYER + item * STAT_WORDS * 2; }
  __device__ static size_t lm(int b, int wg) { return LM0 + (size_t(b) * NWG + wg) * 2; }
};

// ------------------------------------------------------------------------------------------------
// Per-workgroup plan: which rows / chunk this workgroup owns.  Computed identically by all waves.
// ------------------------------------------------------------------------------------------------


template <class G>
struct Plan {
  int wg;
  int q0, q1;   // QKV rows
  int o0, o1;   // O rows (only workgroups without an attention chunk, when those are at least half)
  int a0, a1;   // act indices (gate rows a0..a1-1, up rows I+a0..)
  int d0, d1;   // down rows
  int v0, v1;   // LM-head rows
  int n_lm;     // LM segments
  // attention (batch 1)
  int att;      // 1: this workgroup owns an attention chunk
  int natt;     // workgroups with a chunk (which ones: `att`, never an index range)
  int g, c, C, t0, t1;   // kv head, chunk, chunks, cached token range [t0, t1)
  int S, pos;   // tokens attended (incl. new) and the new token's position
  long long slot;  // KV slot of the new token (slot_mapping[0]; < 0: no append)
  int leader;   // owns the new token, merges the chunk partials and appends K/V
  int xcd;      // chunk c of KV head g on workgroup g + 8c: a head's chunks share one XCD and
                // exchange their records through its L2 (p.xws, ordinary memory)

  __device__ __forceinline__ void init(const Params& p, int wg_) {
    wg = wg_;
    S = min(max(p.seq_lens[0], 1), p.max_seq);
    pos = int(max(p.positions[0], (int64_t)0));
    slot = p.slot_mapping[0];
    const int old = S - 1;
    int C0 = old <= 0 ? 1 : max((old + TC_LONG - 1) / TC_LONG, min((old + TC_SHORT - 1) / TC_SHORT, C_SHORT));
    C0 = min(C0, NWG / G::KVH);
    // at most NCT - 192 chunks: a chunk's merge slice (192 / C values, rounded up) times C records
    // is then at most NCT (one read per consumer thread); 12288 / 64 tokens fit a chunk
    static_assert(kMaxSeq / (NCT - REC_WORDS) <= TC_MAX, "the chunk cap leaves chunks of at most TC_MAX");
    C0 = min(C0, NCT - REC_WORDS);
    // no more chunks than one XCD holds (NWG / 8, the same-XCD records below) while chunks of at
    // most TC_MAX tokens allow it: at 8192 cached tokens 32 chunks of 256-288 instead of 47 of 176
    C0 = min(C0, max(NWG / 8, (old + TC_MAX - 1) / TC_MAX));
    const int tc = old <= 0 ? 16 : ((old + C0 - 1) / C0 + 15) / 16 * 16;
    C = old <= 0 ? 1 : (old + tc - 1) / tc;
    natt = G::KVH * C;
    // Workgroups are dispatched to the 8 XCDs round-robin (workgroup i on XCC (i + s) mod 8, where
    // the start s carries over from earlier dispatches), so with chunk c of head g on workgroup
    // g + 8c every chunk of a head shares an XCD and its L2.  Each attention workgroup checks this
    // at run time (its hardware XCC id against those of the head's other chunks, before the first
    // record) and keeps the records in the uncached workspace when it does not hold.
    xcd = p.xws != nullptr && C <= NWG / 8 && G::KVH <= 8;
    att = xcd ? ((wg % 8) < G::KVH && (wg / 8) < C) : wg < natt;
    int below = 0;  // attention workgroups with a lower index
    if (xcd) {
      for (int r = 0; r < G::KVH; ++r) below += r < wg ? min(C, (wg - r + 7) / 8) : 0;
    } else {
      below = min(wg, natt);
    }
    g = c = t0 = t1 = leader = 0;
    if (att) {
      g = xcd ? wg % 8 : wg / C;
      c = xcd ? wg / 8 : wg % C;
      t0 = min(c * tc, old);
      t1 = min((c + 1) * tc, old);
      leader = c == C - 1;
    }
    // QKV and O rows go to the workgroups without an attention chunk when those are at least
    // half: attention workgroups also stream their KV chunk, and their P2 precedes P3.
    if (natt <= NWG / 2) {
      const int nw = NWG - natt, i = wg - below;
      q0 = att ? 0 : split_lo(G::QKV, nw, i);
      q1 = att ? 0 : split_lo(G::QKV, nw, i + 1);
      o0 = att ? 0 : split_lo(G::H, nw, i);
      o1 = att ? 0 : split_lo(G::H, nw, i + 1);
    } else {
      q0 = split_lo(G::QKV, NWG, wg); q1 = split_lo(G::QKV, NWG, wg + 1);
      o0 = split_lo(G::H, NWG, wg); o1 = split_lo(G::H, NWG, wg + 1);
    }
    a0 = split_lo(G::I, NWG, wg);   a1 = split_lo(G::I, NWG, wg + 1);
    d0 = split_lo(G::H, NWG, wg);   d1 = split_lo(G::H, NWG, wg + 1);
    if (p.lm_head) {
      v0 = split_lo(G::V, NWG, wg); v1 = split_lo(G::V, NWG, wg + 1);
    } else {
      v0 = v1 = 0;
    }
    n_lm = (v1 - v0 + LM_ROWS_G - 1) / LM_ROWS_G;
  }
};

// Most rows any wave computes per phase (balanced split, then round-robin over the NCW waves).
template <class G>
struct Rows {
  static constexpr int per_wave(int rows_per_wg) { return (rows_per_wg + NCW - 1) / NCW; }
  static constexpr int QKV = per_wave((G::QKV + NWG / 2 - 1) / (NWG / 2));
  static constexpr int O = per_wave((G::H + NWG / 2 - 1) / (NWG / 2));
  static constexpr int ACT = per_wave((G::I + NWG - 1) / NWG);
  static constexpr int DOWN = per_wave((G::H + NWG - 1) / NWG);
  static constexpr int LM = LM_ROWS_G / NCW;
};

// Segments a workgroup streams, in stream order.  Per layer: norm1 weights, QKV rows, the
// rotary cos/sin row (attention workgroups), the KV chunk, O rows, norm2 weights, gate rows,
// up rows, down rows; after the last layer: the final-norm weights and the LM-head segments.
// Small vectors go through the ring too, so no consumer ever waits on a global load for them.
enum SegKind {
  S_NORM1, S_QKV, S_QKV_S, S_CS, S_KV, S_O, S_O_S, S_NORM2, S_GATE, S_GATE_S, S_GATE_H, S_GATE_R, S_UP, S_UP_S,
  S_UP_H, S_UP_R, S_DOWN, S_DOWN_S, SEGS_PER_LAYER
};
constexpr int S_FNORM = 100, S_LM = 101;

// Lossless gate/up (e != nullptr with e->on, bf16 weights only): S_GATE / S_UP carry the plane rows
// (1 byte per weight), S_*_H the header rows (4 bytes per 8 weights), S_*_R the escaped chunks of the
// workgroup's rows (16 bytes each); dense layers have empty S_*_H / S_*_R segments.
template <class G>
__device__ __forceinline__ uint32_t seg_bytes(const Plan<G>& P, int kind, int lm_index, int cs_fp32,
                                              const GUE* e = nullptr) {
  constexpr uint32_t WB = G::WF ? 1u : 2u;  // bytes per projection weight
  const bool enc = G::WF == 0 && e != nullptr && e->on != 0u;
  switch (kind) {
    case S_NORM1: return P.q1 > P.q0 ? G::H * 2 : 0u;
    case S_NORM2:
    case S_FNORM: return G::H * 2;
    case S_QKV: return uint32_t(P.q1 - P.q0) * G::H * WB;
    case S_QKV_S: return G::WF ? uint32_t(P.q1 - P.q0) * scale_stride(G::H) : 0u;
    case S_CS: return P.att ? (cs_fp32 ? 256u : 128u) : 0u;
    case S_KV: return P.att ? uint32_t(P.t1 - P.t0) * 256u : 0u;
    case S_O: return uint32_t(P.o1 - P.o0) * G::H * WB;
    case S_O_S: return G::WF ? uint32_t(P.o1 - P.o0) * scale_stride(G::H) : 0u;
    case S_GATE:
    case S_UP: return uint32_t(P.a1 - P.a0) * G::H * (enc ? 1u : WB);
    case S_GATE_S:
    case S_UP_S: return G::WF ? uint32_t(P.a1 - P.a0) * scale_stride(G::H) : 0u;
    case S_GATE_H:
    case S_UP_H: return enc ? uint32_t(P.a1 - P.a0) * (G::H / 8) * 4u : 0u;
    case S_GATE_R: return enc ? e->cnt[0] * 16u : 0u;
    case S_UP_R: return enc ? e->cnt[1] * 16u : 0u;
    case S_DOWN: return uint32_t(P.d1 - P.d0) * G::I * WB;
    case S_DOWN_S: return G::WF ? uint32_t(P.d1 - P.d0) * scale_stride(G::I) : 0u;
    default: {
      const int r0 = P.v0 + lm_index * LM_ROWS_G;
      const int r1 = min(r0 + LM_ROWS_G, P.v1);
      return uint32_t(r1 - r0) * G::H * 2;
    }
  }
}


// Ring byte offset (within a KV segment) of 16-byte piece `part` of K (v=0) or V (v=1) of token j.
__device__ __forceinline__ uint32_t kv_slot(int j, int v, int part) {
  return uint32_t(j) * 256u + uint32_t(v) * 128u + uint32_t((part + j) & 7) * 16u;
}

// ------------------------------------------------------------------------------------------------
// Shared memory layout
// ------------------------------------------------------------------------------------------------

template <class G>
struct Smem {
  static constexpr int XS = G::I > G::H ? G::I : G::H;
  // Attention inputs and scores share storage with the phase-input vector: attention starts after
  // a consumer barrier that follows the last xs read of P1, and every xs write after attention
  // follows the attention barrier, after which only wml/wo (separate) are read.
  struct Attn {
    float qkvw[NCW][5 * 64];     // per-wave attention inputs (3 q heads, k_new, v_new; pre-RoPE)
    float sc[3][TC_MAX + 4];     // per-head scores
    uint16_t pb[3][TC_MAX + 4];  // per-head probabilities (bf16), pairs read as 32-bit words
  };
  uint8_t ring[RING];
  union {
    float xs[XS];                // current phase input (bf16 values as fp32)
    Attn at;
  };
  float xkeep[G::H];             // layer input x (residual for O)
  float h1keep[G::H];            // h1 (residual for down)
  float red[NCW];
  float wml[NCW][2][3];          // per-wave softmax max / sum per head
  float wo[NCW][3][64];          // per-wave P.V partial per head
  float mg[NCT];                 // attention merge: the head's chunk records of this chunk's slice
  LayerW lw[G::L];               // layer pointer table (read by the producers from LDS)
  const void* kvp[G::L];         // per-layer KV cache base
  GUE gue[G::L];                 // per-layer lossless gate/up streams of this workgroup
  int32_t blk[TC_MAX / 16 + 2];
  float lm_val[NCW];
  int32_t lm_idx[NCW];
  alignas(16) uint32_t front[NPW];  // per producer wave: stream bytes below which its packets landed
  uint32_t consumed[NCW];
  uint32_t cbar;
};

// ------------------------------------------------------------------------------------------------
// Producer wave
// ------------------------------------------------------------------------------------------------

// NPW producer waves share the stream: global packet n (1 KB of the stream, ring slot n mod
// RING/PKT) is issued by wave n % NPW.  Each wave keeps at most DEPTH of its packets in flight and
// publishes front[w] = start of its oldest packet that may still be in flight; consumers take the
// minimum over the waves.  Nothing here waits on a compiler-visible vector-memory load: the
// pointer tables and block ids come from LDS, so the only vmcnt waits are the explicit ones.
template <class G>
__device__ __forceinline__ void producer(const Params& p, const Plan<G>& P, Smem<G>& sm, uint32_t epoch) {
  const int pw = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const uint32_t ring_base = uint32_t(reinterpret_cast<uintptr_t>(sm.ring));
  // Block ids of this workgroup's attention chunk (the same for every layer).
  if (pw == 0 && P.att) {
    const int nb = (P.t1 > P.t0) ? ((P.t1 - 1) / 16 - P.t0 / 16 + 1) : 0;
    for (int i = lane; i < nb; i += 64) sm.blk[i] = p.block_table[P.t0 / 16 + i];
  }
  wait_vmcnt<0>();
  __builtin_amdgcn_s_barrier();  // consumers may read blk[] after this

  uint32_t n = 0;  // global packet index at the start of the current segment
  uint32_t room = RING;  // ring bytes the consumers have released, plus the ring size
  Spin spin(p.ws, epoch, 1);
  bool dead = false;
  auto cmin = [&]() -> uint32_t {
    uint32_t c = ld_lds(&sm.consumed[0]);
#pragma unroll
    for (int w = 1; w < NCW; ++w) c = min(c, ld_lds(&sm.consumed[w]));
    return c;
  };
  auto publish = [&](uint32_t first_pending_packet) {
    if (lane == 0) st_lds(&sm.front[pw], first_pending_packet * PKT);
  };
  auto issue_segment = [&](int kind, int layer, int lm_index) {
    const GUE* ge = kind >= S_GATE && kind <= S_UP_R ? &sm.gue[layer] : nullptr;
    const uint32_t bytes = seg_bytes(P, kind, lm_index, p.cs_fp32, ge);
    const uint32_t npk = pad_pkt(bytes) / PKT;
    if (npk == 0) return;
    const uint8_t* base = nullptr;
    const uint8_t* cache = nullptr;
    if (kind == S_KV) {
      cache = reinterpret_cast<const uint8_t*>(sm.kvp[layer]);
    } else if (kind == S_FNORM) {
      base = reinterpret_cast<const uint8_t*>(p.final_norm);
    } else if (kind == S_LM) {
      base = reinterpret_cast<const uint8_t*>(p.embed) + size_t(P.v0 + lm_index * LM_ROWS_G) * G::H * 2;
    } else if (kind == S_CS) {
      base = reinterpret_cast<const uint8_t*>(p.cos_sin) + size_t(P.pos) * 64 * (p.cs_fp32 ? 4 : 2);
    } else {
      const LayerW& Lw = sm.lw[layer];
      constexpr size_t WB = G::WF ? 1 : 2;
      constexpr size_t SH = scale_stride(G::H), SI = scale_stride(G::I);
      auto u8 = [](const void* q) { return reinterpret_cast<const uint8_t*>(q); };
      switch (kind) {
        case S_NORM1: base = u8(Lw.norm1); break;
        case S_QKV: base = u8(Lw.qkv) + size_t(P.q0) * G::H * WB; break;
        case S_QKV_S: base = Lw.qkv_s + size_t(P.q0) * SH; break;
        case S_O: base = u8(Lw.o) + size_t(P.o0) * G::H * WB; break;
        case S_O_S: base = Lw.o_s + size_t(P.o0) * SH; break;
        case S_NORM2: base = u8(Lw.norm2); break;
        case S_GATE:
          base = ge->on ? ge->plane + size_t(P.a0) * G::H : u8(Lw.gate_up) + size_t(P.a0) * G::H * WB;
          break;
        case S_GATE_S: base = Lw.gate_up_s + size_t(P.a0) * SH; break;
        case S_GATE_H: base = u8(ge->hdr + size_t(P.a0) * (G::H / 8)); break;
        case S_GATE_R: base = u8(ge->raw + size_t(ge->first[0]) * 8); break;
        case S_UP:
          base = ge->on ? ge->plane + size_t(G::I + P.a0) * G::H
                        : u8(Lw.gate_up) + size_t(G::I + P.a0) * G::H * WB;
          break;
        case S_UP_S: base = Lw.gate_up_s + size_t(G::I + P.a0) * SH; break;
        case S_UP_H: base = u8(ge->hdr + size_t(G::I + P.a0) * (G::H / 8)); break;
        case S_UP_R: base = u8(ge->raw + size_t(ge->first[1]) * 8); break;
        case S_DOWN: base = u8(Lw.down) + size_t(P.d0) * G::I * WB; break;
        default: base = Lw.down_s + size_t(P.d0) * SI; break;
      }
    }
    for (uint32_t i = (uint32_t(pw) + NPW - n % NPW) % NPW; i < npk && !dead; i += NPW) {
      const uint32_t gn = n + i;
      // `room`: the end of the free ring as last read; the consumers' counters only grow, so they are
      // read again only when a packet would pass it
      if ((gn + 1) * PKT > room && (gn + 1) * PKT > (room = cmin() + RING)) {
        wait_vmcnt<0>();
        publish(gn);
        while ((gn + 1) * PKT > (room = cmin() + RING))
          if (!spin.again()) { dead = true; break; }
        if (dead) break;
      }
      const uint32_t off = i * PKT + uint32_t(lane) * 16u;
      const uint8_t* src;
      if (kind == S_KV) {
        // 4 tokens per packet, 256 B each: 8 K slots then 8 V slots of 16 B.  Slot s of chunk
        // token j holds piece (s - j) mod 8, so 8 consecutive tokens read with one piece index hit
        // 8 different LDS banks (kv_slot).
        const int jt = int(i) * 4 + (lane >> 4);
        const int t = P.t0 + jt;
        const int piece = (lane >> 3) & 1;
        const int part = ((lane & 7) - jt) & 7;
        const int blk = off < bytes ? sm.blk[t / 16 - P.t0 / 16] : 0;
        const long long e = (long long)blk * p.block_stride + (long long)(t & 15) * p.token_stride +
                            (long long)P.g * p.head_stride + (piece ? p.v_off : p.k_off) + part * 8;
        src = cache + e * 2;
      } else {
        src = base + off;
      }
      if (off < bytes) dma16(src, __builtin_amdgcn_readfirstlane(ring_base + ((gn * PKT) & (RING - 1))));
      wait_vmcnt<DEPTH>();
      // of this wave's packets gn, gn-NPW, ..., the last DEPTH may still be in flight
      if (gn >= uint32_t(DEPTH - 1) * NPW) publish(gn - uint32_t(DEPTH - 1) * NPW);
    }
    n += npk;
  };
  for (int l = 0; l < p.n_layers && !dead; ++l)
    for (int kind = 0; kind < SEGS_PER_LAYER && !dead; ++kind) issue_segment(kind, l, 0);
  if (!dead) issue_segment(S_FNORM, 0, 0);
  for (int j = 0; j < P.n_lm && !dead; ++j) issue_segment(S_LM, 0, j);
  wait_vmcnt<0>();
  publish(dead ? 0x3fffffu : n);
}

// ------------------------------------------------------------------------------------------------
// Consumer waves
// ------------------------------------------------------------------------------------------------

template <class G, class SM = Smem<G>, class PL = Plan<G>>
struct Consumer {
  static constexpr uint32_t RB = sizeof(SM::ring);  // ring bytes (a power of two)
  const Params& p;
  const PL& P;
  SM& sm;
  int cw, lane, ct;          // consumer wave, lane, consumer thread id
  uint32_t pos = 0;          // stream cursor (mirrors the producer)
  uint32_t bar_gen = 0;
  uint32_t tag32;
  bool dead = false;
  int xr;                    // the copy of the batch-1 exchange vectors this workgroup polls
  bool l2rec = false;        // the head's chunks share this XCC: records go through its L2

  __device__ __forceinline__ Consumer(const Params& p_, const PL& P_, SM& sm_, uint32_t ep)
      : p(p_), P(P_), sm(sm_) {
    xr = P.wg % XREP;
    cw = (threadIdx.x >> 6) - NPW;
    lane = threadIdx.x & 63;
    ct = cw * 64 + lane;
    tag32 = ep;
  }

  // Makes the lane ids opaque at a phase boundary, so per-lane addresses are recomputed inside the
  // layer loop instead of being hoisted out of it and kept live in registers.
  __device__ __forceinline__ void refresh() { asm volatile("" : "+v"(lane), "+v"(ct)); }

  // Batch-1 exchange word: element i of vector (kind, layer l), written to every copy.
  __device__ __forceinline__ void st_x(int kind, int l, int i, uint64_t v) const {
    skew_delay(p.skew, P.wg, l, kind);
#pragma unroll
    for (int r = 0; r < XREP; ++r) st_dev64(reinterpret_cast<uint64_t*>(p.ws + WS<G>::xw(kind, l, r, i)), v);
  }

  // Claims the next segment of the stream; returns its start position.
  __device__ __forceinline__ uint32_t next_seg(uint32_t bytes) {
    const uint32_t s = pos;
    pos += pad_pkt(bytes);
    return s;
  }
  // Lowest stream position landed in the ring over the producer waves, in one 16-byte LDS read.
  // The producers publish a position after their DMA into LDS completed, so every ring byte below
  // a value read here is in place; the last value is kept in `seen` (positions only grow) and a
  // wait for bytes below it needs no LDS read at all.
  static_assert(NPW == 4, "one 16-byte read of the producer positions");
  uint32_t seen = 0;
  __device__ __forceinline__ uint32_t filled() const {
    typedef __attribute__((address_space(3))) const volatile u32x4 lds_u32x4;
    const u32x4 f = *(lds_u32x4*)(sm.front);
    return min(min(f.x, f.y), min(f.z, f.w));
  }
  __device__ __forceinline__ void wait_filled(uint32_t end) {
    if (dead || end <= seen) return;
    Spin spin(p.ws, tag32, 2);
    while ((seen = filled()) < end)
      if (!spin.again()) { dead = true; return; }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);  // the ring reads that follow stay after the wait
  }
  __device__ __forceinline__ void release(uint32_t end) {
    wait_lgkm0();  // ring reads of this wave have returned
    if (lane == 0) st_lds(&sm.consumed[cw], end);
  }
  // Barrier over the NCW consumer waves (LDS counter; the producer never joins).
  __device__ __forceinline__ void cbar() {
    bar_gen += NCW;
    if (lane == 0) __hip_atomic_fetch_add(&sm.cbar, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    Spin spin(p.ws, tag32, 3);
    while (ld_lds(&sm.cbar) < bar_gen)
      if (!spin.again()) { dead = true; break; }
  }
  __device__ __forceinline__ uint4 ring16(uint32_t at) const {
    return *reinterpret_cast<const uint4*>(sm.ring + (at & (RB - 1)));
  }
  __device__ __forceinline__ uint32_t ring4(uint32_t at) const {
    return *reinterpret_cast<const uint32_t*>(sm.ring + (at & (RB - 1)));
  }
  __device__ __forceinline__ uint2 ring8(uint32_t at) const {
    return *reinterpret_cast<const uint2*>(sm.ring + (at & (RB - 1)));
  }
  // an exchange word {bf16 value, tag32}; a 16-byte load holds two of them
  __device__ __forceinline__ uint64_t w64(float v) const { return (uint64_t(tag32) << 32) | f2bf(v); }
  __device__ __forceinline__ bool ok2(u32x4 v) const { return v.y == tag32 && v.w == tag32; }

  // Poll `n` (even) tagged exchange words, two per 16-byte load, split over all consumer threads;
  // writes the values (fp32) to dst[] (and keep[] when given).  Every load of a thread is in flight
  // at once; only pairs whose tags are stale are polled again.  Returns this wave's sum of squares.
  template <int MAXG>
  __device__ __forceinline__ float poll_split(int kind, int l, int b, int n, float* dst, float* keep) {
    const __amdgpu_buffer_rsrc_t r = rsrc(p.ws);
    auto at = [&](int i) { return uint32_t(WS<G>::xw(kind, l, b, i)) * 4u; };
    u32x4 v[MAXG];
    uint32_t pend = 0;
#pragma unroll
    for (int g = 0; g < MAXG; ++g) {
      const int i = (ct + g * NCT) * 2;
      if (i < n) { v[g] = ld_dev128(r, at(i)); pend |= 1u << g; }
    }
    float ss = 0.f;
    Spin spin(p.ws, tag32, 4);
    while (true) {
#pragma unroll
      for (int g = 0; g < MAXG; ++g) {
        if ((pend >> g) & 1u) {
          if (ok2(v[g])) {
            const int i = (ct + g * NCT) * 2;
            const float f0 = bf_lo(v[g].x), f1 = bf_lo(v[g].z);
            *reinterpret_cast<float2*>(dst + i) = make_float2(f0, f1);
            if (keep) *reinterpret_cast<float2*>(keep + i) = make_float2(f0, f1);
            ss += f0 * f0 + f1 * f1;
            pend &= ~(1u << g);
          }
        }
      }
      if (!pend) break;
      if (dead || !spin.again()) { dead = true; break; }
#pragma unroll
      for (int g = 0; g < MAXG; ++g)
        if ((pend >> g) & 1u) v[g] = ld_dev128(r, at((ct + g * NCT) * 2));
    }
    return wave_sum(ss);
  }

  // Poll three element ranges [e0, e0+n0), [e1, e1+n1), [e2, e2+n2) of the qkv vector of layer l
  // (each an even number of elements starting on an even element, total <= 512) with this wave
  // alone (no barrier); values -> dst[0 .. n0 + n1 + n2).  All loads of a lane are in flight at once.
  __device__ __forceinline__ void poll_wave3(int l, int b, int e0, int n0, int e1, int n1, int e2, int n2,
                                             float* dst) {
    const __amdgpu_buffer_rsrc_t r = rsrc(p.ws);
    auto load = [&](int i) -> u32x4 {
      const int e = i < n0 ? e0 + i : (i < n0 + n1 ? e1 + i - n0 : e2 + i - n0 - n1);
      return ld_dev128(r, uint32_t(WS<G>::xw(X_QKV, l, b, e)) * 4u);
    };
    const int n = n0 + n1 + n2;
    constexpr int NL = 4;  // 16-byte loads per lane: 2 values each
    u32x4 v[NL];
    uint32_t pend = 0;
#pragma unroll
    for (int k = 0; k < NL; ++k) {
      const int i = (lane + 64 * k) * 2;
      if (i < n) { v[k] = load(i); pend |= 1u << k; }
    }
    Spin spin(p.ws, tag32, 7);
    while (true) {
#pragma unroll
      for (int k = 0; k < NL; ++k)
        if (((pend >> k) & 1u) && ok2(v[k])) {
          *reinterpret_cast<float2*>(dst + (lane + 64 * k) * 2) = make_float2(bf_lo(v[k].x), bf_lo(v[k].z));
          pend &= ~(1u << k);
        }
      if (!pend) break;
      if (dead || !spin.again()) { dead = true; break; }
#pragma unroll
      for (int k = 0; k < NL; ++k)
        if ((pend >> k) & 1u) v[k] = load((lane + 64 * k) * 2);
    }
  }

  // Sum of the per-wave values in red[] after a barrier (fixed order: deterministic).
  __device__ __forceinline__ float block_total(float wave_value) {
    if (lane == 0) sm.red[cw] = wave_value;
    cbar();
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < NCW; ++w) t += sm.red[w];
    return t;
  }
};

// Norm weights of a lane's chunks (8-element blocks), from the ring segment that carries them.
template <class G, int K, int EPC>
__device__ __forceinline__ void load_normw(const Consumer<G>& C, XChunks<K, EPC>& nw,
                                           uint32_t seg) {
#pragma unroll
  for (int c = 0; c < Chunks<K, EPC>::CPL; ++c) {
    const int ch = C.lane + 64 * c;
#pragma unroll
    for (int i = 0; i < EPC / 8; ++i)
      nw[c][i] = ch < Chunks<K, EPC>::CH ? C.ring16(seg + uint32_t(ch * EPC + 8 * i) * 2u) : make_uint4(0, 0, 0, 0);
  }
}

// out[r] = row (cw + NCW*r) of a ring segment . x, reading the weights straight from LDS.  The
// reads are unconditional (ring addresses wrap, so rows past `nrows` read stale ring bytes whose
// results are never stored), so all of a wave's LDS reads issue back to back before one wait; the
// chunks past the row end (K/8 not a multiple of 64) are zeroed, since their lanes join the sum.
template <class G, int K, int MAXR>
__device__ __forceinline__ void dots_ring(const Consumer<G>& C, uint32_t seg, int nrows,
                                          const XChunks<K, 8>& x, float (&out)[MAXR]) {
  (void)nrows;
  constexpr int CPL = Chunks<K>::CPL, CH = Chunks<K>::CH;
  uint4 w[MAXR][CPL];
#pragma unroll
  for (int r = 0; r < MAXR; ++r) {
    const uint32_t row = uint32_t(C.cw + NCW * r);
#pragma unroll
    for (int c = 0; c < CPL; ++c)
      w[r][c] = C.ring16(seg + row * uint32_t(K * 2) + uint32_t(C.lane + 64 * c) * 16u);
  }
  if (CH % 64 != 0) {
    const bool tail_ok = C.lane + 64 * (CPL - 1) < CH;
#pragma unroll
    for (int r = 0; r < MAXR; ++r)
      if (!tail_ok) w[r][CPL - 1] = make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int r = 0; r < MAXR; ++r) {
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      acc = dot2(w[r][c].x, x[c][0].x, acc);
      acc = dot2(w[r][c].y, x[c][0].y, acc);
      acc = dot2(w[r][c].z, x[c][0].z, acc);
      acc = dot2(w[r][c].w, x[c][0].w, acc);
    }
    out[r] = acc;
  }
#pragma unroll
  for (int r = 0; r < MAXR; ++r) out[r] = wave_sum(out[r]);
}

// MXFP8 rows: out[r] = row (cw + NCW*r) . x with the row's e4m3 weights (K bytes in segment
// `segq`) scaled by its e8m0 codes (scale_stride(K) bytes per row in segment `segs`).  Each 16-byte
// chunk (16 weights, one scale block of 32 covers two chunks) becomes 8 bf16 pairs with
// v_cvt_scalef32_pk_bf16_fp8 -- exactly bf16(e4m3 * 2^(s-127)), the dequantised weight -- and
// meets the activations in v_dot2_f32_bf16, so the sums equal the bf16 path's on the
// dequantised matrix.  Rows past `nrows` read stale ring bytes and are never stored.
template <class G, int K, int MAXR>
__device__ __forceinline__ void dots_ring_q(const Consumer<G>& C, uint32_t segq, uint32_t segs,
                                            const XChunks<K, 16>& x, float (&out)[MAXR]) {
  constexpr int CPL = Chunks<K, 16>::CPL, CH = Chunks<K, 16>::CH;
  constexpr uint32_t SK = scale_stride(K);
  uint4 w[MAXR][CPL];
  uint32_t sc[MAXR][CPL];
#pragma unroll
  for (int r = 0; r < MAXR; ++r) {
    const uint32_t row = uint32_t(C.cw + NCW * r);
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const uint32_t ch = uint32_t(C.lane + 64 * c);
      w[r][c] = C.ring16(segq + row * uint32_t(K) + ch * 16u);
      sc[r][c] = C.sm.ring[(segs + row * SK + (ch >> 1)) & (C.RB - 1)];
    }
  }
  if (CH % 64 != 0) {
    const bool tail_ok = C.lane + 64 * (CPL - 1) < CH;
#pragma unroll
    for (int r = 0; r < MAXR; ++r)
      if (!tail_ok) { w[r][CPL - 1] = make_uint4(0, 0, 0, 0); sc[r][CPL - 1] = 127u; }
  }
#pragma unroll
  for (int r = 0; r < MAXR; ++r) {
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const float f = e8m0_f32(sc[r][c]);
      const uint32_t q[4] = {w[r][c].x, w[r][c].y, w[r][c].z, w[r][c].w};
      const uint32_t a[8] = {x[c][0].x, x[c][0].y, x[c][0].z, x[c][0].w, x[c][1].x, x[c][1].y, x[c][1].z, x[c][1].w};
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const bf16x2 lo = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(int(q[d]), f, false);
        const bf16x2 hi = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(int(q[d]), f, true);
        acc = dot2(__builtin_bit_cast(uint32_t, lo), a[2 * d], acc);
        acc = dot2(__builtin_bit_cast(uint32_t, hi), a[2 * d + 1], acc);
      }
    }
    out[r] = acc;
  }
#pragma unroll
  for (int r = 0; r < MAXR; ++r) out[r] = wave_sum(out[r]);
}

// The lossless-encoded gate and up rows of P4 as the 16-byte chunks dots_ring would read from a
// dense segment (bit-identical words): for matrix m, plane rows (K bytes each) in `segp[m]`, header
// rows (K/8 words) in `segh[m]`, the escaped chunks of the workgroup's rows (ordinals first[m],
// first[m]+1, ...) in `segr[m]`.  All plane and header reads of both matrices issue back to back,
// then all escape reads (branch-free: a plain chunk reads escape 0 and discards it), so the phase
// pays two LDS round trips rather than one per chunk.
template <class G, int K, int MAXR, int NM = 2>
__device__ __forceinline__ void decode_lossless2(const Consumer<G>& C, const uint32_t (&segp)[NM],
                                                 const uint32_t (&segh)[NM], const uint32_t (&segr)[NM],
                                                 const uint32_t (&first)[NM],
                                                 uint4 (&w)[NM][MAXR][Chunks<K>::CPL]) {
  constexpr int CPL = Chunks<K>::CPL, CH = Chunks<K>::CH;
  uint2 pl[NM][MAXR][CPL];
  uint32_t hd[NM][MAXR][CPL];
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int r = 0; r < MAXR; ++r) {
      const uint32_t row = uint32_t(C.cw + NCW * r);
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const uint32_t ch = uint32_t(C.lane + 64 * c);
        hd[m][r][c] = C.ring4(segh[m] + (row * uint32_t(CH) + ch) * 4u);
        pl[m][r][c] = C.ring8(segp[m] + row * uint32_t(K) + ch * 8u);
      }
    }
  // Every chunk is rebuilt (an escaped chunk's result is discarded) and the results are made opaque
  // before the escapes are merged: otherwise the compiler turns the merge into a branch per chunk
  // around the rebuild, with an LDS wait and the plane read inside it, serialising the chunks.
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int r = 0; r < MAXR; ++r)
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        w[m][r][c] = lossless_chunk(pl[m][r][c], hd[m][r][c]);
        asm volatile("" : "+v"(w[m][r][c].x), "+v"(w[m][r][c].y), "+v"(w[m][r][c].z), "+v"(w[m][r][c].w));
      }
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int r = 0; r < MAXR; ++r)
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const uint32_t h = hd[m][r][c];
        const bool esc = (h >> 24) == 255u;
        const uint4 e = C.ring16(segr[m] + (esc ? (h & 0xFFFFFFu) - first[m] : 0u) * 16u);
        w[m][r][c].x = esc ? e.x : w[m][r][c].x;
        w[m][r][c].y = esc ? e.y : w[m][r][c].y;
        w[m][r][c].z = esc ? e.z : w[m][r][c].z;
        w[m][r][c].w = esc ? e.w : w[m][r][c].w;
      }
  if (CH % 64 != 0 && C.lane + 64 * (CPL - 1) >= CH)
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int r = 0; r < MAXR; ++r) w[m][r][CPL - 1] = make_uint4(0, 0, 0, 0);
}

// out[r] = w[r] . x for weight chunks already in registers (dots_ring's accumulation order).
template <int K, int MAXR>
__device__ __forceinline__ void dots_regs(const uint4 (&w)[MAXR][Chunks<K>::CPL], const XChunks<K, 8>& x,
                                          float (&out)[MAXR]) {
#pragma unroll
  for (int r = 0; r < MAXR; ++r) {
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < Chunks<K>::CPL; ++c) {
      acc = dot2(w[r][c].x, x[c][0].x, acc);
      acc = dot2(w[r][c].y, x[c][0].y, acc);
      acc = dot2(w[r][c].z, x[c][0].z, acc);
      acc = dot2(w[r][c].w, x[c][0].w, acc);
    }
    out[r] = wave_sum(acc);
  }
}

// Projection rows of a phase in the workgroup's weight format.
template <class G, int K, int MAXR>
__device__ __forceinline__ void gemv(const Consumer<G>& C, uint32_t segw, uint32_t segs, int nrows,
                                     const XChunks<K, G::WF ? 16 : 8>& x,
                                     float (&out)[MAXR]) {
  if constexpr (G::WF) dots_ring_q<G, K, MAXR>(C, segw, segs, x, out);
  else dots_ring<G, K, MAXR>(C, segw, nrows, x, out);
}

// Lane r (r < MAXR) gets out[r] (wave-uniform values), for one store instruction per wave.  The
// lane id is made opaque at every step: a plain select chain on it is recognised as an indexed
// read of the array, which the compiler then places in scratch memory (a global-memory round
// trip on the critical path).
template <int MAXR>
__device__ __forceinline__ float pick(const float (&out)[MAXR], int lane) {
  float v = out[0];
#pragma unroll
  for (int r = 1; r < MAXR; ++r) {
    int lr = lane;
    asm volatile("" : "+v"(lr));
    v = lr == r ? out[r] : v;
  }
  return v;
}


// ------------------------------------------------------------------------------------------------
// P2: attention for one chunk (batch 1).  The chunk's tokens (cached ones, plus the new one for the
// leader) are split over the 4 consumer waves in even-aligned ranges; each wave handles all 3 query
// heads of KV head g for its tokens: RoPE on the queries (and the new key), scores with bf16 dot2,
// the chunk's softmax max and sum of exp, exchanged between the C chunks of KV head g, so each
// probability is bf16(exp(s - M) / L) with the max M and sum L over all tokens, exactly the values
// HF rounds to bf16 before P.V (softmax in fp32, then .to(bf16): modeling_llama.py:207-208).  Then
// P.V with bf16 dot2; one barrier adds the waves' fp32 partials; wave h < 3 owns head 3g+h: it
// writes the chunk's partial record (non-leader), or adds all chunks of KV head g in chunk order
// and rounds once (leader).  The leader's wave 3 appends the new K/V (block360_kernel.inc:124-135).
// ------------------------------------------------------------------------------------------------

template <class G, bool DBG>
__device__ __forceinline__ void attention(Consumer<G>& C, int l, uint32_t segc, uint32_t seg) {
  const Params& p = C.p;
  const Plan<G>& P = C.P;
  Smem<G>& sm = C.sm;
  using W = WS<G>;
  const int b = 0, g = P.g, lane = C.lane, w = C.cw;
  const int T_old = P.t1 - P.t0;
  const int T = T_old + (P.leader ? 1 : 0);
  // this wave's tokens [j0, j1): even-aligned split; the new token (index T_old) is the last one
  auto edge = [&](int k) { return k >= NCW ? T : ((T * k) / NCW) & ~1; };
  const int j0 = edge(w), j1 = edge(w + 1);
  const bool has_new = P.leader && j1 == T && T > j0;
  if (P.q1 > P.q0) C.cbar();  // P1 of this workgroup read xs, which shares storage with sm.at
  float* in = sm.at.qkvw[w];

  const int part = lane & 7, grp = lane >> 3;
  // queries of the 3 heads -> in[0, 192).  The wave with the new token (the leader's last wave,
  // edge(3) < T) also needs the new key and value -> in[192, 320): it issues their loads after q
  // has arrived and looks at them only after the scores of its cached tokens, so the load's round
  // trip (most of a microsecond inside the step) overlaps that work; words not yet current then
  // are polled again.
  C.poll_wave3(l, C.xr, g * 192, 192, 0, 0, 0, 0, in);
  // the new key (lanes 0-15) and value (lanes 16-31) words: loaded now, checked after the scores
  const __amdgpu_buffer_rsrc_t rkv = rsrc(p.ws);
  auto kv_at = [&](int i) {
    return uint32_t(W::xw(X_QKV, l, C.xr, i < 64 ? G::H + g * 64 + i : G::H + G::KVH * 64 + g * 64 + i - 64)) * 4u;
  };
  u32x4 kvw = {0u, 0u, 0u, 0u};
  if (has_new) kvw = ld_dev128(rkv, kv_at(lane * 2));
  C.wait_filled(C.pos);  // cos/sin row and KV chunk are in the ring
  // cos/sin of dims 8*part .. 8*part+7 (mod 32): contiguous in the table row of this position
  auto load_cs = [&](float (&cs8)[8], float (&sn8)[8]) {
    const uint32_t f0 = uint32_t(part & 3) * 8u;
    if (p.cs_fp32) {
      const uint4 c0 = C.ring16(segc + f0 * 4u), c1 = C.ring16(segc + f0 * 4u + 16u);
      const uint4 s0 = C.ring16(segc + 128u + f0 * 4u), s1 = C.ring16(segc + 128u + f0 * 4u + 16u);
      const uint32_t cu[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
      const uint32_t su[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) { cs8[e] = __uint_as_float(cu[e]); sn8[e] = __uint_as_float(su[e]); }
    } else {
      const uint4 c = C.ring16(segc + f0 * 2u), sn = C.ring16(segc + 64u + f0 * 2u);
      const uint32_t cu[4] = {c.x, c.y, c.z, c.w}, su[4] = {sn.x, sn.y, sn.z, sn.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        cs8[2 * e] = bf_lo(cu[e]); cs8[2 * e + 1] = bf_hi(cu[e]);
        sn8[2 * e] = bf_lo(su[e]); sn8[2 * e + 1] = bf_hi(su[e]);
      }
    }
  };
  // RoPE with HF rounding, bf16(bf16(x*cos) + bf16(rotate_half(x)*sin)) (modeling_llama.py:138-160):
  // this lane's dims 8*part..+7 of a head and their rotation partners 8*(part^4)..+7, as float4s;
  // rotate_half negates the partner for the first half (dims < 32).
  const float sgn = part < 4 ? -1.f : 1.f;
  auto rope8 = [&](const float* head, const float (&cs8)[8], const float (&sn8)[8], uint32_t (&out)[4]) {
    const float4 a0 = *reinterpret_cast<const float4*>(head + part * 8);
    const float4 a1 = *reinterpret_cast<const float4*>(head + part * 8 + 4);
    const float4 b0 = *reinterpret_cast<const float4*>(head + (part ^ 4) * 8);
    const float4 b1 = *reinterpret_cast<const float4*>(head + (part ^ 4) * 8 + 4);
    const float x[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    const float y[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
    float r[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = rnd(rnd(x[e] * cs8[e]) + rnd((sgn * y[e]) * sn8[e]));
#pragma unroll
    for (int e = 0; e < 4; ++e) out[e] = pack2(r[2 * e], r[2 * e + 1]);
  };
  wait_lgkm0();
  if (w == 0 && lane == 0) trace_at(p, l, 3, p.n_layers);
  // rotated queries (and, further down, the rotated new key), packed bf16 pairs
  uint32_t q[3][4], kn[4] = {0u, 0u, 0u, 0u};
  {
    float cs8[8], sn8[8];
    load_cs(cs8, sn8);
#pragma unroll
    for (int h = 0; h < 3; ++h) rope8(in + h * 64, cs8, sn8, q[h]);
  }
  // debug capture of layer debug_layer: rotated queries (chunk 0 of each KV head, lanes 0-7)
  const bool dbg_attn = DBG && p.debug != nullptr && l == p.debug_layer;
  if (dbg_attn && P.c == 0 && w == 0 && grp == 0)
#pragma unroll
    for (int h = 0; h < 3; ++h)
      *reinterpret_cast<uint4*>(p.debug + Dbg<G>::AQ + (g * 3 + h) * 64 + part * 8) =
          make_uint4(q[h][0], q[h][1], q[h][2], q[h][3]);
  if (w == 0 && lane == 0) trace_at(p, l, 16, p.n_layers);
  // the new token's score: 8 lanes per token (8 dims each); s = bf16(q.k) * 1/8 (exact scale)
  auto score = [&](int j, const uint4& k, bool keep) {
    float s3[3];
#pragma unroll
    for (int h = 0; h < 3; ++h) {
      float a = dot2(q[h][0], k.x, 0.f);
      a = dot2(q[h][1], k.y, a);
      a = dot2(q[h][2], k.z, a);
      a = dot2(q[h][3], k.w, a);
      s3[h] = group8_sum(a);
    }
    if (part == 0 && keep)
#pragma unroll
      for (int h = 0; h < 3; ++h) {
        sm.at.sc[h][j] = rnd(s3[h]) * 0.125f;
        if (dbg_attn && P.t0 + j < int(Dbg<G>::SEQ)) {
          p.debug[Dbg<G>::AQK + Dbg<G>::head_pos(b, g * 3 + h, P.t0 + j)] = uint16_t(f2bf(s3[h]));
          p.debug[Dbg<G>::ASC + Dbg<G>::head_pos(b, g * 3 + h, P.t0 + j)] = uint16_t(f2bf(rnd(s3[h]) * 0.125f));
        }
      }
  };
  const int jc = min(j1, T_old);  // this wave's cached tokens end here
  // The cached tokens' scores on the matrix cores, 16-token tiles from j0: D[token][head] =
  // K[token][:] . q[head][:] (v_mfma_f32_16x16x32_bf16, two k-steps over the 64 dims).  Lane l
  // supplies row l%16 of A (token tile*16 + l%16, pieces l/16 and l/16 + 4 of its K) and column l%16
  // of B (q of head l%16 < 3, zero columns past it), and receives the scores of head l%16 for tokens
  // tile*16 + 4(l/16) .. +3.  The rotated q pieces go through LDS, over the pre-RoPE q every lane of
  // this wave has read.
  {
    constexpr int MTG = ((TC_MAX + 1 + NCW - 1) / NCW + 2 + 15) / 16;  // tiles of a wave's tokens
    static_assert(MTG <= 5, "a wave's cached tokens fit 5 tiles");
    const int hq = lane & 15, pq = lane >> 4;
    uint4* qr = reinterpret_cast<uint4*>(in);  // [3 heads][8 pieces]
    if (grp == 0)
#pragma unroll
      for (int h = 0; h < 3; ++h) qr[h * 8 + part] = make_uint4(q[h][0], q[h][1], q[h][2], q[h][3]);
    const int ntl = jc > j0 ? (jc - j0 + 15) >> 4 : 0;
    uint4 ka[MTG][2];
#pragma unroll
    for (int i = 0; i < MTG; ++i) {
      ka[i][0] = ka[i][1] = make_uint4(0u, 0u, 0u, 0u);
      if (i < ntl) {
        const int tok = j0 + 16 * i + hq;  // past jc: other ring bytes, whose scores are not kept
        ka[i][0] = C.ring16(seg + kv_slot(tok, 0, pq));
        ka[i][1] = C.ring16(seg + kv_slot(tok, 0, pq + 4));
      }
    }
    uint4 b0 = make_uint4(0u, 0u, 0u, 0u), b1 = make_uint4(0u, 0u, 0u, 0u);
    if (hq < 3) {
      b0 = qr[hq * 8 + pq];
      b1 = qr[hq * 8 + pq + 4];
    }
    const bf16x8 bq0 = __builtin_bit_cast(bf16x8, b0), bq1 = __builtin_bit_cast(bf16x8, b1);
#pragma unroll
    for (int i = 0; i < MTG; ++i) {
      if (i >= ntl) continue;
      floatx4 acc = {0.f, 0.f, 0.f, 0.f};
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ka[i][0]), bq0, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ka[i][1]), bq1, acc, 0, 0, 0);
      if (hq < 3)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int j = j0 + 16 * i + 4 * pq + jj;
          if (j < jc) {
            sm.at.sc[hq][j] = rnd(acc[jj]) * 0.125f;
            if (dbg_attn && P.t0 + j < int(Dbg<G>::SEQ)) {
              p.debug[Dbg<G>::AQK + Dbg<G>::head_pos(b, g * 3 + hq, P.t0 + j)] = uint16_t(f2bf(acc[jj]));
              p.debug[Dbg<G>::ASC + Dbg<G>::head_pos(b, g * 3 + hq, P.t0 + j)] =
                  uint16_t(f2bf(rnd(acc[jj]) * 0.125f));
            }
          }
        }
    }
  }
  if (has_new) {
    // the new key and value, RoPE on the key, and its score (every 8-lane group computes it; the
    // first group keeps it)
    {
      Spin spin(p.ws, C.tag32, 7);
      while (!C.ok2(kvw)) {
        if (C.dead || !spin.again()) { C.dead = true; break; }
        kvw = ld_dev128(rkv, kv_at(lane * 2));
      }
      *reinterpret_cast<float2*>(in + 192 + lane * 2) = make_float2(bf_lo(kvw.x), bf_lo(kvw.z));
    }
    // the cos/sin row is read again (still in the ring): held in registers across the scores it
    // would take 16 of them where the kernel has none to spare
    asm volatile("" ::: "memory");
    float cs8[8], sn8[8];
    load_cs(cs8, sn8);
    rope8(in + 192, cs8, sn8, kn);
    score(T_old, make_uint4(kn[0], kn[1], kn[2], kn[3]), grp == 0);
  }
  wait_lgkm0();
  if (w == 0 && lane == 0) trace_at(p, l, 17, p.n_layers);
  // chunk softmax statistics per head: max and sum of exp over this wave's tokens, then over the
  // chunk (all waves), then over all chunks of KV head g (one exchange of 3 x (max, sum) records).
  // The exponentials here and in the probabilities use the hardware exp2 (__expf): within a few
  // fp32 ulp of expf, far below the bf16 rounding of p.
  // A wave holds at most 128 tokens (chunks are at most TC_MAX + 1), so 2 scores per lane and head.
  static_assert(TC_MAX + 1 - ((3 * (TC_MAX + 1) / NCW) & ~1) <= 128 && (TC_MAX + 1) / NCW + 2 <= 128,
                "per-wave token ranges fit two per lane");
  float sv[3][2];
#pragma unroll
  for (int h = 0; h < 3; ++h)
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int j = j0 + lane + 64 * i;
      sv[h][i] = j < j1 ? sm.at.sc[h][j] : -INFINITY;
    }
  {
    float m3[3], l3[3];
#pragma unroll
    for (int h = 0; h < 3; ++h) m3[h] = fmaxf(sv[h][0], sv[h][1]);
    wave_max_n<3>(m3);
#pragma unroll
    for (int h = 0; h < 3; ++h) {
      l3[h] = 0.f;
#pragma unroll
      for (int i = 0; i < 2; ++i) l3[h] += sv[h][i] == -INFINITY ? 0.f : __expf(sv[h][i] - m3[h]);
    }
    wave_sum_n<3>(l3);
    if (lane == 0)
#pragma unroll
      for (int h = 0; h < 3; ++h) { sm.wml[w][0][h] = m3[h]; sm.wml[w][1][h] = l3[h]; }
  }
  C.cbar();
  // lane 4h + v holds wave v's (max, sum) of head h; max and rescaled sum over each quad of lanes
  float mq = -INFINITY, lq = 0.f;
  if (lane < 4 * 3) {
    mq = sm.wml[lane & 3][0][lane >> 2];
    lq = sm.wml[lane & 3][1][lane >> 2];
  }
  float mx = fmaxf(mq, dpp<0xb1>(mq, mq));  // quad_perm [1,0,3,2]
  mx = fmaxf(mx, dpp<0x4e>(mx, mx));         // quad_perm [2,3,0,1]
  float ex = mq == -INFINITY ? 0.f : lq * __expf(mq - mx);
  ex += dpp<0xb1>(0.f, ex);
  ex += dpp<0x4e>(0.f, ex);
  float Mh[3], Lh[3];
#pragma unroll
  for (int h = 0; h < 3; ++h) {
    Mh[h] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mx), 4 * h));
    Lh[h] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ex), 4 * h));
  }
  const uint64_t tg = uint64_t(C.tag32) << 32;
  if (P.C > 1) {
    if (l == 0 && P.xcd) {
      // do the head's chunks (workgroups g + 8c) really share this XCC?  Every chunk reads the same
      // C ids, so writers and readers of the records agree on where they are.
      const uint32_t mine = __builtin_amdgcn_s_getreg((15 << 11) | (0 << 6) | 20) & 15u;
      uint32_t differ = 0;
      for (int c = lane; c < P.C; c += 64) {
        const uint64_t* src = reinterpret_cast<const uint64_t*>(p.ws + W::xcc(g + 8 * c));
        Spin spin(p.ws, C.tag32, 13);
        uint64_t v = ld_dev64(src);
        while (uint32_t(v >> 32) != C.tag32) {
          if (C.dead || !spin.again()) { C.dead = true; break; }
          v = ld_dev64(src);
        }
        differ |= (uint32_t(v) & 15u) != mine ? 1u : 0u;
      }
      C.l2rec = p.l2_records && __builtin_amdgcn_ballot_w64(differ != 0u) == 0ull;
    }
    // same-XCD records: plain stores reach the shared L2, the (sc1) polls read it there
    const bool l2 = P.xcd && C.l2rec;
    uint64_t* stat_base = reinterpret_cast<uint64_t*>(l2 ? p.xws + (W::stat(l, size_t(g) * P.C) - W::REC0)
                                                         : p.ws + W::stat(l, size_t(g) * P.C));
    skew_delay(p.skew, P.wg, l, 11);
    if (w == 0 && lane < 6) {
      const int h = lane >> 1;
      const float v = (lane & 1) ? (h == 0 ? Lh[0] : h == 1 ? Lh[1] : Lh[2]) : (h == 0 ? Mh[0] : h == 1 ? Mh[1] : Mh[2]);
      if (l2) st_l2(stat_base + size_t(P.c) * STAT_WORDS + lane, tg | __float_as_uint(v));
      else st_dev64(stat_base + size_t(P.c) * STAT_WORDS + lane, tg | __float_as_uint(v));
    }
    // lane k polls chunk k (and k + 64): 3 x 16 bytes = (m, l) of the 3 heads
    const __amdgpu_buffer_rsrc_t r = rsrc(stat_base);
    u32x4 s[2][3];
    uint32_t pend = 0;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int k = lane + 64 * i;
      if (k < P.C) {
#pragma unroll
        for (int h = 0; h < 3; ++h) s[i][h] = ld_dev128(r, uint32_t(k * STAT_WORDS + 2 * h) * 8u);
        pend |= 1u << i;
      }
    }
    auto fresh = [&](const u32x4& v) { return v.y == C.tag32 && v.w == C.tag32; };
    Spin spin(p.ws, C.tag32, 6);
    while (true) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
        if (((pend >> i) & 1u) && fresh(s[i][0]) && fresh(s[i][1]) && fresh(s[i][2])) pend &= ~(1u << i);
      if (!pend) break;
      if (C.dead || !spin.again()) { C.dead = true; break; }
#pragma unroll
      for (int i = 0; i < 2; ++i)
        if ((pend >> i) & 1u)
#pragma unroll
          for (int h = 0; h < 3; ++h) s[i][h] = ld_dev128(r, uint32_t((lane + 64 * i) * STAT_WORDS + 2 * h) * 8u);
    }
#pragma unroll
    for (int h = 0; h < 3; ++h) {
      Mh[h] = -INFINITY;
#pragma unroll
      for (int i = 0; i < 2; ++i)
        if (lane + 64 * i < P.C) Mh[h] = fmaxf(Mh[h], __uint_as_float(s[i][h].x));
    }
    wave_max_n<3>(Mh);
#pragma unroll
    for (int h = 0; h < 3; ++h) {
      Lh[h] = 0.f;
#pragma unroll
      for (int i = 0; i < 2; ++i)
        if (lane + 64 * i < P.C) Lh[h] += __uint_as_float(s[i][h].z) * __expf(__uint_as_float(s[i][h].x) - Mh[h]);
    }
    wave_sum_n<3>(Lh);
  }
  if (w == 0 && lane == 0) trace_at(p, l, 18, p.n_layers);
  // probabilities with the softmax's global max and sum, rounded to bf16 before P.V as HF does
  // (softmax in fp32, then .to(bf16): modeling_llama.py:207-208)
#pragma unroll
  for (int h = 0; h < 3; ++h) {
    const float inv = 1.0f / Lh[h];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int j = j0 + lane + 64 * i;
      if (j < j1) {
        sm.at.pb[h][j] = uint16_t(f2bf(__expf(sv[h][i] - Mh[h]) * inv));
        if (dbg_attn && P.t0 + j < int(Dbg<G>::SEQ))
          p.debug[Dbg<G>::APR + Dbg<G>::head_pos(b, g * 3 + h, P.t0 + j)] = sm.at.pb[h][j];
      }
    }
  }
  wait_lgkm0();
  // P.V: lane = (quarter qv, d4) owns dims 4 d4 .. 4 d4 + 3 (8 bytes of a token's V); token pairs
  // go round-robin to the four 16-lane quarters, whose sums are added at the end
  const int qv = lane >> 4, d4 = lane & 15;
  const int jo1 = min(j1, T_old);
  const int npairs = jo1 > j0 ? (jo1 - j0) / 2 : 0;
  const uint32_t voff = uint32_t(d4 & 1) * 8u;
  float acc[3][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll 4
  for (int k = qv; k < npairs; k += 4) {
    const int j = j0 + 2 * k;
    const uint2 va = C.ring8(seg + kv_slot(j, 1, d4 >> 1) + voff);
    const uint2 vb = C.ring8(seg + kv_slot(j + 1, 1, d4 >> 1) + voff);
    // {v_j[d], v_j+1[d]} for the lane's four dims d
    const uint32_t v0 = __builtin_amdgcn_perm(vb.x, va.x, 0x05040100u), v1 = __builtin_amdgcn_perm(vb.x, va.x, 0x07060302u);
    const uint32_t v2 = __builtin_amdgcn_perm(vb.y, va.y, 0x05040100u), v3 = __builtin_amdgcn_perm(vb.y, va.y, 0x07060302u);
#pragma unroll
    for (int h = 0; h < 3; ++h) {
      const uint32_t pp = *reinterpret_cast<const uint32_t*>(&sm.at.pb[h][j]);
      acc[h][0] = dot2(pp, v0, acc[h][0]);
      acc[h][1] = dot2(pp, v1, acc[h][1]);
      acc[h][2] = dot2(pp, v2, acc[h][2]);
      acc[h][3] = dot2(pp, v3, acc[h][3]);
    }
  }
  if (qv == 0) {
    if (jo1 > j0 && ((jo1 - j0) & 1)) {  // odd cached token at the end of the range
      const int j = jo1 - 1;
      const uint2 v = C.ring8(seg + kv_slot(j, 1, d4 >> 1) + voff);
      const float vf[4] = {bf_lo(v.x), bf_hi(v.x), bf_lo(v.y), bf_hi(v.y)};
#pragma unroll
      for (int h = 0; h < 3; ++h) {
        const float pj = bf2f(sm.at.pb[h][j]);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[h][i] = fmaf(pj, vf[i], acc[h][i]);
      }
    }
    if (has_new) {
#pragma unroll
      for (int h = 0; h < 3; ++h) {
        const float pj = bf2f(sm.at.pb[h][T_old]);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[h][i] = fmaf(pj, in[256 + 4 * d4 + i], acc[h][i]);
      }
    }
  }
#pragma unroll
  for (int h = 0; h < 3; ++h)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[h][i] = column_total<false>(acc[h][i]);
  C.release(C.pos);  // this wave no longer reads the K/V chunk
  if (has_new && P.slot >= 0 && grp < 2) {
    // KV append at slot_mapping[b] (block360_kernel.inc:124-135; slot < 0 skips): lanes 0-7 store
    // the rotated new K, lanes 8-15 the new V, 8 dims (16 bytes) per lane.  Issued after the
    // scores and P.V: a later wait on this wave's memory counter would otherwise hold those
    // phases until the stores are acknowledged.
    uint16_t* cache = reinterpret_cast<uint16_t*>(const_cast<void*>(sm.kvp[l]));
    const long long e = (P.slot / 16) * p.block_stride + (P.slot % 16) * p.token_stride +
                        (long long)g * p.head_stride + (grp ? p.v_off : p.k_off) + part * 8;
    uint32_t val[4];
    if (grp == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) val[i] = kn[i];
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) val[i] = pack2(in[256 + part * 8 + 2 * i], in[256 + part * 8 + 2 * i + 1]);
    }
    uint16_t* dst = cache + e;
    if ((reinterpret_cast<uintptr_t>(dst) & 15u) == 0) {
      st_global16(dst, val[0], val[1], val[2], val[3]);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        st_global2(dst + 2 * i, uint16_t(val[i] & 0xffffu));
        st_global2(dst + 2 * i + 1, uint16_t(val[i] >> 16));
      }
    }
  }
  if (lane < 16)
#pragma unroll
    for (int h = 0; h < 3; ++h)
#pragma unroll
      for (int i = 0; i < 4; ++i) sm.wo[w][h][4 * d4 + i] = acc[h][i];
  C.cbar();
  if (w == 0 && lane == 0) trace_at(p, l, 19, p.n_layers);
  const bool l2 = P.xcd && C.l2rec;
  uint64_t* rec_base = reinterpret_cast<uint64_t*>(l2 ? p.xws + (W::rec(l, 0) - W::REC0) : p.ws + W::rec(l, 0));
  // every chunk (the leader too) publishes its partial sum of p.v, fp32, wave w < 3 head 3g + w
  // (the 4 waves' parts added in fixed wave order)
  if (w < 3) {
    float O = 0.f;
#pragma unroll
    for (int v = 0; v < NCW; ++v) O += sm.wo[v][w][lane];
    if (w == 0 && lane == 0) trace_at(p, l, 4, p.n_layers);
    skew_delay(p.skew, P.wg, l, 12);
    uint64_t* dst = rec_base + size_t(g * P.C + P.c) * REC_WORDS + w * 64 + lane;
    if (l2) st_l2(dst, tg | __float_as_uint(O));
    else st_dev64(dst, tg | __float_as_uint(O));
  }
  // The head's 192 attention values are summed by its C chunks: chunk c adds the slice
  // [192 c / C, 192 (c + 1) / C) over all C records, in chunk order, and rounds once (HF's
  // bf16(p.v) of the whole head).  Read i (i < slice x C <= 192 + C <= NCT: C is capped at
  // NCT - 192) is record i % C of value lo + i / C, one per consumer thread, all in flight
  // together; one thread per value then adds its C records from LDS.
  const int lo = (REC_WORDS * P.c) / P.C, nval = (REC_WORDS * (P.c + 1)) / P.C - lo;
  const int t = C.ct;
  for (int i = t; i < nval * P.C; i += NCT) {
    const int vi = i / P.C, k = i - vi * P.C;
    const uint64_t* src = rec_base + size_t(g * P.C + k) * REC_WORDS + lo + vi;
    uint64_t v = ld_dev64(src);
    Spin spin(p.ws, C.tag32, 5);
    while (uint32_t(v >> 32) != C.tag32) {
      if (C.dead || !spin.again()) { C.dead = true; break; }
      v = ld_dev64(src);
    }
    sm.mg[i] = __uint_as_float(uint32_t(v));
  }
  C.cbar();
  if (w == 0 && lane == 0) trace_at(p, l, 20, p.n_layers);
  if (t < nval) {
    float O = 0.f;
    for (int k = 0; k < P.C; ++k) O += sm.mg[t * P.C + k];
    const int e = g * REC_WORDS + lo + t;  // head 3g + (lo + t) / 64, dim (lo + t) % 64
    C.st_x(X_ATTN, l, e, C.w64(O));
    if (DBG && p.debug) {
      const uint16_t ob = uint16_t(f2bf(O));
      p.debug[size_t(l) * Dbg<G>::LAYER + Dbg<G>::ATTN + e] = ob;
      if (l == p.debug_layer) p.debug[Dbg<G>::APV + e] = ob;
    }
  }
  if (w == 0 && lane == 0) trace_at(p, l, 5, p.n_layers);
}

// ------------------------------------------------------------------------------------------------
// Consumer main loop
// ------------------------------------------------------------------------------------------------

template <class G, bool DBG>
__device__ __forceinline__ void consumer(const Params& p, const Plan<G>& P, Smem<G>& sm, uint32_t epoch) {
  Consumer<G> C(p, P, sm, epoch);
  __builtin_amdgcn_s_barrier();  // pairs with the producer's barrier (blk[] ready)
  using W = WS<G>;
  using R = Rows<G>;
  constexpr int GH = (G::H + NCT * 2 - 1) / (NCT * 2);   // poll loads per thread, H words
  constexpr int GI = (G::I + NCT * 2 - 1) / (NCT * 2);   // ... I words
  constexpr int EW = G::WF ? 16 : 8;                      // activations per 16-byte weight chunk
  const int b = 0;
  auto tr = [&](int l, int ev) { if (C.ct == 0) trace_at(p, l, ev, p.n_layers); };
  // debug capture: this layer's stage rows (sequence 0), and a normalised vector from wave 0
  auto dl = [&](int l) { return p.debug + size_t(l) * Dbg<G>::LAYER; };
  auto dbg_vec = [&](uint16_t* dst, const XChunks<G::H, 8>& v) {
#pragma unroll
    for (int cc = 0; cc < Chunks<G::H>::CPL; ++cc) {
      const int ch = C.lane + 64 * cc;
      if (ch < Chunks<G::H>::CH) *reinterpret_cast<uint4*>(dst + ch * 8) = v[cc][0];
    }
  };
  if (C.ct == 0) trace_tail(p, 0);
  if (P.att && P.xcd && P.C > 1 && C.ct == 0)  // where this chunk runs (HW_REG_XCC_ID)
    st_dev64(reinterpret_cast<uint64_t*>(p.ws + W::xcc(P.wg)),
             (uint64_t(C.tag32) << 32) | (__builtin_amdgcn_s_getreg((15 << 11) | (0 << 6) | 20) & 15u));

  for (int l = 0; l < p.n_layers; ++l) {
    // ---------------- P1: RMSNorm(x) + QKV ----------------
    C.refresh();
    if (P.q1 > P.q0) {
      const uint32_t segn = C.next_seg(seg_bytes(P, S_NORM1, 0, p.cs_fp32));
      const uint32_t seg = C.next_seg(seg_bytes(P, S_QKV, 0, p.cs_fp32));
      const uint32_t segs = C.next_seg(seg_bytes(P, S_QKV_S, 0, p.cs_fp32));
      C.wait_filled(C.pos);
      tr(l, 0);
      XChunks<G::H, EW> nw;
      load_normw<G, G::H, EW>(C, nw, segn);
      float ss;
      if (l == 0) {
        long long id = p.ids_i64 ? reinterpret_cast<const int64_t*>(p.input_ids)[b]
                                 : reinterpret_cast<const int32_t*>(p.input_ids)[b];
        id = min(max(id, 0LL), (long long)G::V - 1);  // an out-of-range id must not read past the table
        const uint16_t* e = p.input_hidden ? p.input_hidden + size_t(b) * G::H : p.embed + size_t(id) * G::H;
        float s = 0.f;
        for (int i = C.ct; i < G::H; i += NCT) {
          const float v = bf2f(e[i]);
          sm.xs[i] = v;
          sm.xkeep[i] = v;
          s += v * v;
        }
        ss = wave_sum(s);
      } else {
        ss = C.template poll_split<GH>(X_X, l - 1, C.xr, G::H, sm.xs, sm.xkeep);
      }
      const float rs = rms_scale(C.block_total(ss), G::H);
      tr(l, 1);
      XChunks<G::H, EW> x;
      load_x<G::H, EW, true>(x, sm.xs, nw, rs, C.lane);
      if constexpr (EW == 8)
        if (DBG && p.debug && P.q0 == 0 && C.cw == 0) dbg_vec(dl(l) + Dbg<G>::NORM1, x);
      tr(l, 21);
      float out[R::QKV];
      gemv<G, G::H, R::QKV>(C, seg, segs, P.q1 - P.q0, x, out);
      C.release(C.pos);
      tr(l, 22);
      const int row = C.cw + NCW * C.lane;
      if (C.lane < R::QKV && row < P.q1 - P.q0) {
        C.st_x(X_QKV, l, P.q0 + row, C.w64(pick(out, C.lane)));
        if (DBG && p.debug) dl(l)[Dbg<G>::QKV + P.q0 + row] = uint16_t(f2bf(pick(out, C.lane)));
      }
      tr(l, 2);
    }
    // ---------------- P2: attention ----------------
    C.refresh();
    {
      const uint32_t segc = C.next_seg(seg_bytes(P, S_CS, 0, p.cs_fp32));
      const uint32_t seg = C.next_seg(seg_bytes(P, S_KV, 0, p.cs_fp32));
      if (P.att) attention<G, DBG>(C, l, segc, seg);
    }
    // ---------------- P3: O + residual ----------------
    C.refresh();
    {
      const uint32_t seg = C.next_seg(seg_bytes(P, S_O, 0, p.cs_fp32));
      const uint32_t segs = C.next_seg(seg_bytes(P, S_O_S, 0, p.cs_fp32));
      const int nrows = P.o1 - P.o0;
      if (nrows > 0) {
        C.wait_filled(C.pos);
        tr(l, 6);
        C.template poll_split<GH>(X_ATTN, l, C.xr, G::H, sm.xs, nullptr);
        C.cbar();
        tr(l, 7);
        XChunks<G::H, EW> x;
        const XChunks<G::H, EW> none = {};
        load_x<G::H, EW, false>(x, sm.xs, none, 1.f, C.lane);
        float out[R::O];
        gemv<G, G::H, R::O>(C, seg, segs, nrows, x, out);
        C.release(C.pos);
        const int row = C.cw + NCW * C.lane;
        if (C.lane < R::O && row < nrows) {
          const int r = P.o0 + row;
          const float o = rnd(pick(out, C.lane));
          C.st_x(X_H1, l, r, C.w64(sm.xkeep[r] + o));
          if (DBG && p.debug) {
            dl(l)[Dbg<G>::O + r] = uint16_t(f2bf(o));
            dl(l)[Dbg<G>::H1 + r] = uint16_t(f2bf(sm.xkeep[r] + o));
          }
        }
        tr(l, 8);
      } else {
        C.release(C.pos);
      }
    }
    // ---------------- P4: RMSNorm(h1) + gate/up + SwiGLU ----------------
    C.refresh();
    {
      const GUE& ge = sm.gue[l];
      const uint32_t segn = C.next_seg(seg_bytes(P, S_NORM2, 0, p.cs_fp32));
      const uint32_t segg = C.next_seg(seg_bytes(P, S_GATE, 0, p.cs_fp32, &ge));
      const uint32_t segg_s = C.next_seg(seg_bytes(P, S_GATE_S, 0, p.cs_fp32, &ge));
      const uint32_t segg_h = C.next_seg(seg_bytes(P, S_GATE_H, 0, p.cs_fp32, &ge));
      const uint32_t segg_r = C.next_seg(seg_bytes(P, S_GATE_R, 0, p.cs_fp32, &ge));
      const uint32_t segu = C.next_seg(seg_bytes(P, S_UP, 0, p.cs_fp32, &ge));
      const uint32_t segu_s = C.next_seg(seg_bytes(P, S_UP_S, 0, p.cs_fp32, &ge));
      const uint32_t segu_h = C.next_seg(seg_bytes(P, S_UP_H, 0, p.cs_fp32, &ge));
      const uint32_t segu_r = C.next_seg(seg_bytes(P, S_UP_R, 0, p.cs_fp32, &ge));
      const int na = P.a1 - P.a0;
      C.wait_filled(C.pos);
      XChunks<G::H, EW> nw;
      load_normw<G, G::H, EW>(C, nw, segn);
      // lossless layer: the gate chunks are rebuilt while the h1 exchange is in flight (the up
      // chunks after it: both sets live across the poll would exceed the register budget)
      uint4 wg[1][R::ACT][Chunks<G::H>::CPL];
      if constexpr (G::WF == 0) {
        if (ge.on) {
          const uint32_t sp[1] = {segg}, sh[1] = {segg_h}, sr[1] = {segg_r}, fo[1] = {ge.first[0]};
          decode_lossless2<G, G::H, R::ACT, 1>(C, sp, sh, sr, fo, wg);
        }
      }
      tr(l, 9);
      const float ss = C.template poll_split<GH>(X_H1, l, C.xr, G::H, sm.xs, sm.h1keep);
      const float rs = rms_scale(C.block_total(ss), G::H);
      tr(l, 10);
      XChunks<G::H, EW> x;
      load_x<G::H, EW, true>(x, sm.xs, nw, rs, C.lane);
      if constexpr (EW == 8)
        if (DBG && p.debug && P.a0 == 0 && C.cw == 0) dbg_vec(dl(l) + Dbg<G>::NORM2, x);
      float og[R::ACT], ou[R::ACT];
      bool done = false;
      if constexpr (G::WF == 0) {
        if (ge.on) {
          const uint32_t sp[1] = {segu}, sh[1] = {segu_h}, sr[1] = {segu_r}, fo[1] = {ge.first[1]};
          uint4 wu[1][R::ACT][Chunks<G::H>::CPL];
          decode_lossless2<G, G::H, R::ACT, 1>(C, sp, sh, sr, fo, wu);
          dots_regs<G::H, R::ACT>(wg[0], x, og);
          dots_regs<G::H, R::ACT>(wu[0], x, ou);
          done = true;
        }
      } else {
        (void)segg_h; (void)segg_r; (void)segu_h; (void)segu_r;
      }
      if (!done) {
        gemv<G, G::H, R::ACT>(C, segg, segg_s, na, x, og);
        gemv<G, G::H, R::ACT>(C, segu, segu_s, na, x, ou);
      }
      C.release(C.pos);
      const int row = C.cw + NCW * C.lane;
      if (C.lane < R::ACT && row < na) {
        const float gv = rnd(pick(og, C.lane)), uv = rnd(pick(ou, C.lane));
        const float silu = rnd(gv / (1.0f + expf(-gv)));
        C.st_x(X_ACT, l, P.a0 + row, C.w64(silu * uv));
        if (DBG && p.debug) {
          const int r = P.a0 + row;
          dl(l)[Dbg<G>::GATE + r] = uint16_t(f2bf(gv));
          dl(l)[Dbg<G>::UP + r] = uint16_t(f2bf(uv));
          dl(l)[Dbg<G>::SILU + r] = uint16_t(f2bf(silu));
          dl(l)[Dbg<G>::ACT + r] = uint16_t(f2bf(silu * uv));
        }
      }
      tr(l, 11);
    }
    // ---------------- P5: down + residual ----------------
    C.refresh();
    {
      const uint32_t seg = C.next_seg(seg_bytes(P, S_DOWN, 0, p.cs_fp32));
      const uint32_t segs = C.next_seg(seg_bytes(P, S_DOWN_S, 0, p.cs_fp32));
      const int nrows = P.d1 - P.d0;
      C.wait_filled(C.pos);
      tr(l, 12);
      C.template poll_split<GI>(X_ACT, l, C.xr, G::I, sm.xs, nullptr);
      C.cbar();
      tr(l, 13);
      XChunks<G::I, EW> x;
      const XChunks<G::I, EW> none = {};
      load_x<G::I, EW, false>(x, sm.xs, none, 1.f, C.lane);
      float out[R::DOWN];
      gemv<G, G::I, R::DOWN>(C, seg, segs, nrows, x, out);
      C.release(C.pos);
      const int row = C.cw + NCW * C.lane;
      if (C.lane < R::DOWN && row < nrows) {
        const int r = P.d0 + row;
        const float y = rnd(sm.h1keep[r] + rnd(pick(out, C.lane)));
        C.st_x(X_X, l, r, C.w64(y));
        if (DBG && p.debug) {
          dl(l)[Dbg<G>::DOWN + r] = uint16_t(f2bf(rnd(pick(out, C.lane))));
          dl(l)[Dbg<G>::OUT + r] = uint16_t(f2bf(y));
        }
        if (p.layer_outputs) p.layer_outputs[(size_t(l) * p.B + b) * G::H + r] = uint16_t(f2bf(y));
      }
      tr(l, 14);
    }
  }
  // ---------------- final RMSNorm + LM head + argmax ----------------
  const uint32_t segf = C.next_seg(seg_bytes(P, S_FNORM, 0, p.cs_fp32));
  C.wait_filled(C.pos);
  XChunks<G::H> nw;  // the final norm and the tied LM head stay bf16
  load_normw<G, G::H, 8>(C, nw, segf);
  C.release(C.pos);
  const float ss = C.template poll_split<GH>(X_X, p.n_layers - 1, C.xr, G::H, sm.xs, nullptr);
  const float rs = rms_scale(C.block_total(ss), G::H);
  XChunks<G::H> x;
  load_x<G::H, 8, true>(x, sm.xs, nw, rs, C.lane);
  if (P.wg == 0) {
    // final-normed hidden state (the reference's out_hidden, block360_kernel.inc:810-815)
#pragma unroll
    for (int c = 0; c < Chunks<G::H>::CPL; ++c) {
      const int ch = C.lane + 64 * c;
      if (C.cw == 0 && ch < Chunks<G::H>::CH)
        *reinterpret_cast<uint4*>(p.out_hidden + size_t(b) * G::H + ch * 8) = x[c][0];
    }
  }
  float best = -INFINITY;
  int best_i = 0x7fffffff;
  for (int j = 0; j < P.n_lm; ++j) {  // no segments without the LM head
    const uint32_t seg = C.next_seg(seg_bytes(P, S_LM, j, p.cs_fp32));
    const int r0 = P.v0 + j * LM_ROWS_G;
    const int nrows = min(LM_ROWS_G, P.v1 - r0);
    C.wait_filled(C.pos);
    float out[R::LM];
    dots_ring<G, G::H, R::LM>(C, seg, nrows, x, out);
    C.release(C.pos);
#pragma unroll
    for (int r = 0; r < R::LM; ++r) {
      const int row = C.cw + NCW * r;
      if (row < nrows) {
        const float v = rnd(out[r]);
        const int idx = r0 + row;
        if (v > best || (v == best && idx < best_i)) { best = v; best_i = idx; }
      }
    }
    if (p.out_logits) {
      const int row = C.cw + NCW * C.lane;
      if (C.lane < R::LM && row < nrows)
        p.out_logits[size_t(b) * G::V + r0 + row] = uint16_t(f2bf(pick(out, C.lane)));
    }
  }
  if (C.lane == 0) { sm.lm_val[C.cw] = best; sm.lm_idx[C.cw] = best_i; }
  C.cbar();
  if (C.ct == 0) trace_tail(p, 1);
  // every workgroup's end record {bf16 best value, 16-bit index, tag32}: index LM_DEAD when one of
  // its waits gave up, LM_NONE without an LM head; workgroup 0 gathers them all
  if (C.ct == 0) {
    float bv = sm.lm_val[0];
    int bi = sm.lm_idx[0];
    for (int w = 1; w < NCW; ++w)
      if (sm.lm_val[w] > bv || (sm.lm_val[w] == bv && sm.lm_idx[w] < bi)) { bv = sm.lm_val[w]; bi = sm.lm_idx[w]; }
    const uint32_t idx = C.dead ? LM_DEAD : p.lm_head ? uint32_t(bi) & 0xffffu : LM_NONE;
    const uint64_t rec = (uint64_t(C.tag32) << 32) | (uint64_t(idx) << 16) | f2bf(bv);
    skew_delay(p.skew, P.wg, p.n_layers, 13);
    st_dev64(reinterpret_cast<uint64_t*>(p.ws + W::lm(b, P.wg)), rec);
  }
  if (P.wg != 0) {
    if (p.out_logits && (C.dead || aborted(p.ws, C.tag32)))  // this workgroup's logits rows are not valid
      for (int i = P.v0 + C.ct; i < P.v1; i += NCT) p.out_logits[size_t(b) * G::V + i] = 0x7fc0;
    return;
  }
  // workgroup 0: argmax over the NWG candidates (first index on ties, as torch.argmax)
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  uint32_t bad = 0;
  for (int q = C.ct; q < NWG; q += NCT) {
    const uint64_t* src = reinterpret_cast<const uint64_t*>(p.ws + W::lm(b, q));
    Spin spin(p.ws, C.tag32, 6);
    uint64_t r = ld_dev64(src);
    while (uint32_t(r >> 32) != C.tag32) {
      if (!spin.again()) { bad = 1; break; }
      r = ld_dev64(src);
    }
    const float v = bf2f(uint32_t(r) & 0xffffu);
    const int i = int((uint32_t(r) >> 16) & 0xffffu);
    bad |= (i == int(LM_DEAD)) ? 1u : 0u;
    if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
  }
  const bool any_bad = __builtin_amdgcn_ballot_w64(bad != 0u) != 0ull;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
  }
  if (C.lane == 0) { sm.lm_val[C.cw] = bv; sm.lm_idx[C.cw] = bi; sm.red[C.cw] = any_bad ? 1.f : 0.f; }
  C.cbar();
  bool fail = C.dead || aborted(p.ws, C.tag32);
  for (int w = 0; w < NCW; ++w) fail = fail || sm.red[w] != 0.f;
  if (C.ct == 0) {
    bv = sm.lm_val[0];
    bi = sm.lm_idx[0];
    for (int w = 1; w < NCW; ++w)
      if (sm.lm_val[w] > bv || (sm.lm_val[w] == bv && sm.lm_idx[w] < bi)) { bv = sm.lm_val[w]; bi = sm.lm_idx[w]; }
    if (p.out_ids) p.out_ids[b] = fail ? -1 : bi;
  }
  if (fail) {
    step_failed(p, C.tag32, C.ct, b);
    if (p.out_logits)  // every logits row of the sequence (best effort: see step_failed)
      for (int i = C.ct; i < G::V; i += NCT) p.out_logits[size_t(b) * G::V + i] = 0x7fc0;
  }
}

// ------------------------------------------------------------------------------------------------
// Kernel
// ------------------------------------------------------------------------------------------------

template <class G, bool DBG = false>
__global__ void __launch_bounds__(WG_THREADS, 1) decode_kernel(Params p) {
  // the split-role kernel, launched before this one, did the step when the context is within its limit
  if (p.sr_max_s > 0 && min(max(p.seq_lens[0], 1), p.max_seq) <= p.sr_max_s) return;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_raw[];
  Smem<G>& sm = *reinterpret_cast<Smem<G>*>(smem_raw);
  if (threadIdx.x == 0) {
    for (int w = 0; w < NPW; ++w) sm.front[w] = 0;
    for (int w = 0; w < NCW; ++w) sm.consumed[w] = 0;
    sm.cbar = 0;
  }
  // pointer tables into LDS, so the producers never wait on a vector-memory load of their own
  for (int i = threadIdx.x; i < p.n_layers; i += WG_THREADS) {
    LayerW w{};
    if (G::WF) {
      const void* const* t = p.layers + size_t(i) * 10;
      w.norm1 = t[0]; w.qkv = t[1]; w.qkv_s = static_cast<const uint8_t*>(t[2]);
      w.o = t[3]; w.o_s = static_cast<const uint8_t*>(t[4]); w.norm2 = t[5];
      w.gate_up = t[6]; w.gate_up_s = static_cast<const uint8_t*>(t[7]);
      w.down = t[8]; w.down_s = static_cast<const uint8_t*>(t[9]);
    } else {
      const void* const* t = p.layers + size_t(i) * 6;
      w.norm1 = t[0]; w.qkv = t[1]; w.o = t[2]; w.norm2 = t[3]; w.gate_up = t[4]; w.down = t[5];
    }
    sm.lw[i] = w;
    sm.kvp[i] = p.kv[i];
    // lossless gate/up: this workgroup's row range of each matrix and its escapes
    GUE e{};
    if (G::WF == 0 && p.encoded_gu != nullptr) {
      const EncodedGULayer d = p.encoded_gu[i];
      if (*d.enabled != 0u) {
        const int a0 = split_lo(G::I, NWG, blockIdx.x), a1 = split_lo(G::I, NWG, blockIdx.x + 1);
        e.plane = d.plane;
        e.hdr = d.headers;
        e.raw = d.raw;
        e.on = 1u;
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          e.first[m] = d.row_offsets[m * G::I + a0];
          e.cnt[m] = d.row_offsets[m * G::I + a1] - e.first[m];
        }
      }
    }
    sm.gue[i] = e;
  }
  trace_begin(p);
  __syncthreads();
  Plan<G> P;
  P.init(p, blockIdx.x);
  const uint32_t epoch = step_epoch(p.ws);
  if (threadIdx.x < 64 * NPW) {
    producer<G>(p, P, sm, epoch);
  } else {
    // the consumer waves are the step's critical path: their instructions win the SIMD's issue
    // over the producer waves' DMA issue and ring polling when both are ready (+4.4% at config 5)
    __builtin_amdgcn_s_setprio(1);
    consumer<G, DBG>(p, P, sm, epoch);
  }
  __syncthreads();
  if (blockIdx.x == 0 && threadIdx.x == 0) st_dev(p.ws + HDR_EPOCH, epoch);
  trace_end(p);
}

// ================================================================================================
// Batched decode: 2..16 sequences per launch, ragged contexts.  The same persistent
// producer/consumer structure as the batch-1 kernel, with three differences:
//  * projections are [rows x 16 tokens] products on the matrix cores (v_mfma_f32_16x16x32_bf16:
//    weight rows from the LDS ring as A, the staged bf16 activations [token][k] as B), the K range
//    split over the four consumer waves and the partial tiles summed in LDS in a fixed order;
//  * the large activation exchanges (x, attn, h1, act: B x K values) are plain bf16 arrays: each
//    workgroup stores its rows, waits for the stores to complete and then sets its flag; readers
//    poll the 256 flags and pull the [B][K] block into LDS with LDS-DMA (half the bytes of tagged
//    words, and no per-word polling); q/k/v stay tagged words as in the batch-1 kernel;
//  * attention is split into (sequence, KV head, chunk) items, several per workgroup, processed
//    in three passes so that no workgroup waits on another while holding work others need:
//    A) scores of every item (K streamed through the ring) and the chunk softmax statistics;
//    B) the global statistics of each (sequence, KV head), probabilities rounded as HF does,
//       P.V (V streamed), partial sums published; C) leaders add their chunks' partials.
// ================================================================================================
constexpr int BMAX = 16;                  // sequences per launch (the MFMA N dimension)
constexpr uint32_t RING_B = 64u * 1024u;  // ring bytes (the staged activations take the rest of LDS)
constexpr int TCB = 256;                  // max cached tokens per attention item
#ifndef PK_TC_CAP
#define PK_TC_CAP TCB                     // preferred largest chunk (sequences past 64 * cap use more)
#endif
constexpr int IPW = 16;                   // max attention items per workgroup
constexpr int MAX_ITEMS = NWG * IPW;


// Batched workspace regions, after the batch-1 layout (so one workspace serves both kernels).
template <class G>
struct WSB {
  static constexpr int XMAX = WS<G>::XMAX;
  static constexpr size_t REC0 = WS<G>::TOTAL;                       // P.V partials, 3 x 64 tagged fp32
  static constexpr size_t STAT0 = REC0 + size_t(MAX_ITEMS) * REC_WORDS * 2;
  static constexpr size_t FLAG0 = STAT0 + size_t(MAX_ITEMS) * STAT_WORDS * 2;
  // FREP copies of each (kind, layer) flag row; workgroup i polls copy i mod FREP (a row that
  // every workgroup polls queues NWG requests per line and polling round)
  static constexpr int FREP = 8;
  static constexpr size_t DATA0 = FLAG0 + size_t(NKIND) * G::L * FREP * NWG;  // 64-byte aligned below
  static constexpr size_t DATA_WORDS = size_t(BMAX) * XMAX / 2;        // one [B][K] bf16 array
  static constexpr size_t TOTAL = DATA0 + size_t(NKIND) * G::L * DATA_WORDS;
  static_assert(DATA0 % 16 == 0 && DATA_WORDS % 256 == 0, "bf16 arrays start on 64-byte lines");
  __device__ static size_t rec(int item) { return REC0 + size_t(item) * REC_WORDS * 2; }
  __device__ static size_t stat(int item) { return STAT0 + size_t(item) * STAT_WORDS * 2; }
  __device__ static size_t flag(int kind, int l, int wg, int r) {
    return FLAG0 + ((size_t(kind) * G::L + l) * FREP + r) * NWG + wg;
  }
  __device__ static size_t data(int kind, int l) { return DATA0 + (size_t(kind) * G::L + l) * DATA_WORDS; }
};

// An attention item: sequence b, KV head g, chunk c of C (the last one is the leader, which also owns
// the new token), index of chunk 0 of (b, g) among all items, cached tokens [t0, t1).
struct ItemB {
  int b, g, c, C, base, t0, t1, pad;
};

template <class G>
struct SmemB {
  static constexpr int XS = G::I > G::H ? G::I : G::H;
  struct Attn {
    float qb[IPW][5 * 64];            // per item: 3 q heads, then (leader items) the new k and v
    uint16_t qr[IPW][4][64];          // per item: the roped q heads and (leaders) new k, bf16
    uint16_t sc[IPW][3][TCB + 4];     // bf16 scores of every item of this workgroup (rows 8-byte aligned)
    uint16_t pb[3][TCB + 4];          // bf16 probabilities (each wave its own token range)
    float own[IPW][3 * 64];           // leader items: this chunk's partial sums of p.v
    float wml[IPW][NCW][2][3];        // per item and wave: softmax max / sum per head
    float cst[IPW][2][3];             // chunk softmax max / sum per item and head
    float gml[IPW][2][3];             // global (all chunks) max / sum per item and head
    float wo[2][NCW][3][64];          // per-wave P.V partials, double-buffered over items
  };
  uint8_t ring[RING_B];
  union {
    uint16_t xs[BMAX * XS];           // staged activations, [token][K] bf16
    Attn at;
  };
  float tile[NCW][256];               // per-wave MFMA partial tiles
  float xk[BMAX][8];                  // residual x of this workgroup's O rows
  float hk[BMAX][8];                  // residual h1 of this workgroup's down rows
  float rsb[BMAX];                    // per-sequence RMS scale
  float red[NCW];
  LayerW lw[G::L];
  const void* kvp[G::L];
  int32_t blk[IPW][TCB / 16 + 2];     // block ids of each item's chunk
  ItemB it[IPW];                      // this workgroup's attention items
  int32_t sS[BMAX], sPos[BMAX], sId[BMAX];
  long long sSlot[BMAX];
  float lm_val[NCW][BMAX];
  int32_t lm_idx[NCW][BMAX];
  alignas(16) uint32_t front[NPW];
  alignas(16) uint32_t consumed[NCW];
  uint32_t cbar;
};
// Attention items at the largest batch and context: each (sequence, KV head) has at most
// ceil((kMaxSeq - 1) / TCB) chunks, and every workgroup holds at most IPW items.
static_assert((G360::KVH > G135::KVH ? G360::KVH : G135::KVH) * BMAX * ((kMaxSeq - 1 + TCB - 1) / TCB) <= MAX_ITEMS,
              "item arrays hold every chunk");
static_assert((kMaxSeq - 1 + TCB - 1) / TCB <= 64, "a (sequence, head) never has more than 64 chunks");

template <class G>
struct PlanB {
  int wg, B;
  int q0, q1, o0, o1, a0, a1, d0, d1, v0, v1, n_lm;
  int db0, db1;  // sequences of this workgroup's down rows
  int tc;      // cached tokens per attention chunk
  int nitems;  // attention items over all workgroups
  int ni;      // items of this workgroup: wg, wg + NWG, ...

  __device__ __forceinline__ int chunks(int S) const {
    const int old = max(S, 1) - 1;
    return old == 0 ? 1 : (old + tc - 1) / tc;
  }
  __device__ __forceinline__ void init(const Params& p, const int32_t* sS, int wg_) {
    wg = wg_;
    B = p.B;
    // QKV slots (qkv_row order) in whole RoPE pairs: the QKV phase applies RoPE to its own rows
    q0 = 2 * split_lo(G::QKV / 2, NWG, wg); q1 = 2 * split_lo(G::QKV / 2, NWG, wg + 1);
    o0 = split_lo(G::H, NWG, wg);   o1 = split_lo(G::H, NWG, wg + 1);
    a0 = split_lo(G::I, NWG, wg);   a1 = split_lo(G::I, NWG, wg + 1);
#if PK_B_DOWN_SPLIT
    // down: 128 row groups, each shared by workgroups wg and wg ^ 8 (one XCD, so the second read of
    // the rows hits its L2), one taking the first half of the sequences and the other the rest, so
    // that each stages half the act array
    {
      const int grp = (wg >> 4) * 8 + (wg & 7), half = (wg >> 3) & 1;
      d0 = split_lo(G::H, NWG / 2, grp); d1 = split_lo(G::H, NWG / 2, grp + 1);
      db0 = half ? (B + 1) / 2 : 0;      db1 = half ? B : (B + 1) / 2;
    }
#else
    d0 = split_lo(G::H, NWG, wg);   d1 = split_lo(G::H, NWG, wg + 1);
    db0 = 0; db1 = B;
#endif
    if (p.lm_head) { v0 = split_lo(G::V, NWG, wg); v1 = split_lo(G::V, NWG, wg + 1); }
    else { v0 = v1 = 0; }
    n_lm = (v1 - v0 + LM_ROWS - 1) / LM_ROWS;
    // chunks of about two items per workgroup, 64..TCB tokens, a multiple of 16, and long enough that
    // no (sequence, head) has more than 64 chunks (one wave lane per chunk gathers their statistics)
    long long tot = 0;
    int most = 0;
    for (int b = 0; b < B; ++b) {
      tot += max(sS[b], 1) - 1;
      most = max(most, max(sS[b], 1) - 1);
    }
    int t = int((tot * G::KVH + 2LL * NWG - 1) / (2LL * NWG));
    t = min(max(t, 64), PK_TC_CAP);
    t = max(t, (most + 63) / 64);
    tc = min((t + 15) / 16 * 16, TCB);
    nitems = 0;
    for (int b = 0; b < B; ++b) nitems += G::KVH * chunks(sS[b]);
    ni = nitems > wg ? (nitems - wg + NWG - 1) / NWG : 0;
  }
  // chunks of exactly tc cached tokens of a sequence (its last chunk may be shorter, or hold no cached
  // token when S = 1)
  __device__ __forceinline__ int full(int S) const { return (max(S, 1) - 1) / tc; }
  // Item `it` of the assignment order (workgroup wg takes items wg, wg + NWG, ...): every full chunk,
  // in (sequence, KV head, chunk) order, then every short last chunk, so that the workgroups holding
  // one item more than the rest hold a short one.  Returns sequence b, KV head g, chunk c of C, the
  // (sequence, head, chunk) index `base` of chunk 0 of (b, g) (base + c keys the chunk's records),
  // and the cached tokens [t0, t1).
  __device__ __forceinline__ void item(const int32_t* sS, int it, int& b, int& g, int& c, int& C, int& base,
                                       int& t0, int& t1) const {
    int nfull = 0;
    for (int s = 0; s < B; ++s) nfull += G::KVH * full(sS[s]);
    int acc = 0, first = 0;  // items of the part passed, (sequence, head, chunk) index of sequence b
    if (it < nfull) {
      for (b = 0; b < B - 1; ++b) {
        const int n = G::KVH * full(sS[b]);
        if (it < acc + n) break;
        acc += n;
        first += G::KVH * chunks(sS[b]);
      }
      const int nf = max(full(sS[b]), 1);
      g = (it - acc) / nf;
      c = (it - acc) - g * nf;
    } else {
      const int r = it - nfull;
      for (b = 0; b < B - 1; ++b) {
        const int n = G::KVH * (chunks(sS[b]) - full(sS[b]));
        if (r < acc + n) break;
        acc += n;
        first += G::KVH * chunks(sS[b]);
      }
      g = r - acc;
      c = full(sS[b]);
    }
    C = chunks(sS[b]);
    base = first + g * C;
    const int old = max(sS[b], 1) - 1;
    t0 = min(c * tc, old);
    t1 = min((c + 1) * tc, old);
  }
};

// K (v = 0) or V (v = 1) slot of 16-byte piece `part` of chunk token j in an item's segment
// (128 bytes per token; piece (s - j) mod 8 in slot s, so 8 consecutive tokens hit 8 banks).
__device__ __forceinline__ uint32_t kvb_slot(int j, int part) {
  return uint32_t(j) * 128u + uint32_t((part + j) & 7) * 16u;
}

// ------------------------------------------------------------------------------------------------
// Batched producer: per layer norm1, QKV rows, the B rotary rows, the K of every item, the V of
// every item, O rows, norm2, gate rows, up rows, down rows; then the final norm and LM-head rows.
// ------------------------------------------------------------------------------------------------
enum SegB { B_NORM1, B_QKV, B_K, B_V, B_O, B_NORM2, B_GATE, B_UP, B_DOWN, B_FNORM, B_LM };

template <class G>
__device__ __forceinline__ uint32_t segb_bytes(const PlanB<G>& P, const ItemB* it, int kind, int idx, int cs_fp32) {
  switch (kind) {
    case B_NORM1: case B_NORM2: case B_FNORM: return G::H * 2;
    case B_QKV: return uint32_t(P.q1 - P.q0) * G::H * 2;
    case B_K: case B_V: return uint32_t(it[idx].t1 - it[idx].t0) * 128u;
    case B_O: return uint32_t(P.o1 - P.o0) * G::H * 2;
    case B_GATE: case B_UP: return uint32_t(P.a1 - P.a0) * G::H * 2;
    case B_DOWN: return uint32_t(P.d1 - P.d0) * G::I * 2;
    default: {
      const int r0 = P.v0 + idx * LM_ROWS;
      return uint32_t(min(r0 + LM_ROWS, P.v1) - r0) * G::H * 2;
    }
  }
}

template <class G>
__device__ __forceinline__ void producer_b(const Params& p, const PlanB<G>& P, SmemB<G>& sm, uint32_t epoch) {
  const int pw = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const uint32_t ring_base = uint32_t(reinterpret_cast<uintptr_t>(sm.ring));
  if (pw == 0) {  // the item table and every item's block ids (the same for every layer)
    for (int k = 0; k < P.ni; ++k) {
      ItemB e;
      P.item(sm.sS, P.wg + k * NWG, e.b, e.g, e.c, e.C, e.base, e.t0, e.t1);
      e.pad = 0;
      if (lane == 0) sm.it[k] = e;
      const int nb = e.t1 > e.t0 ? (e.t1 - 1) / 16 - e.t0 / 16 + 1 : 0;
      for (int i = lane; i < nb; i += 64) sm.blk[k][i] = p.block_table[size_t(e.b) * p.bt_stride + e.t0 / 16 + i];
    }
  }
  wait_vmcnt<0>();
  __builtin_amdgcn_s_barrier();
  uint32_t n = 0;
  Spin spin(p.ws, epoch, 1);
  bool dead = false;
  // Lowest stream position released by every consumer wave, in one 16-byte LDS read.  A stale value
  // is a lower bound (each wave's position only grows), so the last one read is kept in `avail`
  // and read again only when the next packet would pass it: the issue loop does no LDS round trip
  // per packet.  The DMA that reuses released bytes is issued after the read returns, and the
  // consumers' release stores follow their reads of those bytes.
  static_assert(NCW == 4, "one 16-byte read of the consumer positions");
  auto cmin = [&]() -> uint32_t {
    typedef __attribute__((address_space(3))) const volatile u32x4 lds_u32x4;
    const u32x4 c = *(lds_u32x4*)(sm.consumed);
    return min(min(c.x, c.y), min(c.z, c.w));
  };
  uint32_t avail = 0;  // last cmin() + ring bytes: packets ending at or below it may be issued
  auto publish = [&](uint32_t first_pending_packet) {
    if (lane == 0) st_lds(&sm.front[pw], first_pending_packet * PKT);
  };
  auto issue_segment = [&](int kind, int layer, int idx) {
    const uint32_t bytes = segb_bytes(P, sm.it, kind, idx, p.cs_fp32);
    const uint32_t npk = pad_pkt(bytes) / PKT;
    if (npk == 0) return;
    const uint8_t* base = nullptr;
    int ib = 0, ig = 0, it0 = 0;
    const uint8_t* cache = nullptr;
    const LayerW& Lw = sm.lw[layer];
    auto u8 = [](const void* q) { return reinterpret_cast<const uint8_t*>(q); };
    int blkv = 0;  // K/V segments: lane i holds the block id of the item's i-th 16-token block
    switch (kind) {
      case B_NORM1: base = u8(Lw.norm1); break;
      case B_QKV: base = u8(Lw.qkv); break;
      case B_K: case B_V:
        ib = sm.it[idx].b;
        ig = sm.it[idx].g;
        it0 = sm.it[idx].t0;
        cache = u8(sm.kvp[layer]);
        blkv = lane < TCB / 16 + 2 ? sm.blk[idx][lane] : 0;
        break;
      case B_O: base = u8(Lw.o) + size_t(P.o0) * G::H * 2; break;
      case B_NORM2: base = u8(Lw.norm2); break;
      case B_GATE: base = u8(Lw.gate_up) + size_t(P.a0) * G::H * 2; break;
      case B_UP: base = u8(Lw.gate_up) + size_t(G::I + P.a0) * G::H * 2; break;
      case B_DOWN: base = u8(Lw.down) + size_t(P.d0) * G::I * 2; break;
      case B_FNORM: base = u8(p.final_norm); break;
      case B_LM: base = u8(p.embed) + size_t(P.v0 + idx * LM_ROWS) * G::H * 2; break;
      default: break;
    }
    for (uint32_t i = (uint32_t(pw) + NPW - n % NPW) % NPW; i < npk && !dead; i += NPW) {
      const uint32_t gn = n + i;
      if ((gn + 1) * PKT > avail && (gn + 1) * PKT > (avail = cmin() + RING_B)) {
        wait_vmcnt<0>();
        publish(gn);
        while ((gn + 1) * PKT > (avail = cmin() + RING_B))
          if (!spin.again()) { dead = true; break; }
        if (dead) break;
      }
      const uint32_t off = i * PKT + uint32_t(lane) * 16u;
      const uint8_t* src = nullptr;
      if (off < bytes) {
        if (kind == B_K || kind == B_V) {
          // 8 tokens per packet, all in one 16-token block (items start on a block boundary), so
          // the block id is the same for every lane: read it from the register, no LDS wait
          const int jt = int(off >> 7);
          const int part = int(((off >> 4) - uint32_t(jt)) & 7u);
          const int t = it0 + jt;
          const int blk = __builtin_amdgcn_readlane(blkv, int(i >> 1));
          const long long e = (long long)blk * p.block_stride + (long long)(t & 15) * p.token_stride +
                              (long long)ig * p.head_stride + (kind == B_V ? p.v_off : p.k_off) + part * 8;
          src = cache + e * 2;
        } else if (kind == B_QKV) {
          // the workgroup's slots in order, slot s being projection row qkv_row(s)
          const uint32_t r = off / uint32_t(G::H * 2);
          src = base + size_t(qkv_row<G>(P.q0 + int(r))) * G::H * 2 + (off - r * uint32_t(G::H * 2));
        } else {
          src = base + off;
        }
        dma16(src, __builtin_amdgcn_readfirstlane(ring_base + ((gn * PKT) & (RING_B - 1))));
      }
      wait_vmcnt<DEPTH_B>();
      if (gn >= uint32_t(DEPTH_B - 1) * NPW) publish(gn - uint32_t(DEPTH_B - 1) * NPW);
    }
    n += npk;
  };
  for (int l = 0; l < p.n_layers && !dead; ++l) {
    issue_segment(B_NORM1, l, 0);
    issue_segment(B_QKV, l, 0);
    for (int k = 0; k < P.ni && !dead; ++k) issue_segment(B_K, l, k);
    for (int k = 0; k < P.ni && !dead; ++k) issue_segment(B_V, l, k);
    issue_segment(B_O, l, 0);
    issue_segment(B_NORM2, l, 0);
    issue_segment(B_GATE, l, 0);
    issue_segment(B_UP, l, 0);
    issue_segment(B_DOWN, l, 0);
  }
  if (!dead) issue_segment(B_FNORM, 0, 0);
  for (int j = 0; j < P.n_lm && !dead; ++j) issue_segment(B_LM, 0, j);
  wait_vmcnt<0>();
  publish(dead ? 0x3fffffu : n);
}

// ------------------------------------------------------------------------------------------------
// Batched consumer helpers
// ------------------------------------------------------------------------------------------------
template <class G>
using ConsumerB = Consumer<G, SmemB<G>, PlanB<G>>;

// One 16-byte LDS-DMA piece per lane of a coherent (sc1) global read: lane i copies g to m0 + 16 i.
__device__ __forceinline__ void dma16_sc1(const void* g, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off sc1" ::"s"(lds_addr), "v"(g) : "memory", "m0");
}

// Publish this workgroup's part of exchange (kind, l): every wave's stores have completed, then
// one flag word carries the step's tag.
template <class G>
__device__ __forceinline__ void publish_flag(ConsumerB<G>& C, int kind, int l) {
  wait_vmcnt<0>();
  C.cbar();
  skew_delay(C.p.skew, C.P.wg, l, kind);
  if (C.ct < WSB<G>::FREP) st_dev(C.p.ws + WSB<G>::flag(kind, l, C.P.wg, C.ct), C.tag32);
}

// Wait until all workgroups have published (kind, l), then copy the [B][K] bf16 array into xs.
template <class G>
__device__ __forceinline__ void stage_flagged(ConsumerB<G>& C, int kind, int l, int K, int b0 = 0, int b1 = -1) {
  const uint32_t* flags = C.p.ws + WSB<G>::flag(kind, l, 0, C.P.wg % WSB<G>::FREP);
  {
    Spin spin(C.p.ws, C.tag32, 8);
    for (int w = C.ct; w < NWG; w += NCT)
      while (ld_dev(flags + w) != C.tag32)
        if (C.dead || !spin.again()) { C.dead = true; break; }
  }
  C.cbar();
  // rows [b0, b1) of the array (all by default), to the same rows of xs
  if (b1 < 0) b1 = C.P.B;
  const uint8_t* src = reinterpret_cast<const uint8_t*>(C.p.ws + WSB<G>::data(kind, l)) + size_t(b0) * K * 2;
  const uint32_t bytes = uint32_t(b1 - b0) * uint32_t(K) * 2u;
  const uint32_t lds = uint32_t(reinterpret_cast<uintptr_t>(C.sm.xs + size_t(b0) * K));
  for (uint32_t pk = uint32_t(C.cw); pk * PKT < bytes; pk += NCW) {
    const uint32_t off = pk * PKT + uint32_t(C.lane) * 16u;
    if (off < bytes) dma16_sc1(src + off, __builtin_amdgcn_readfirstlane(lds + pk * PKT));
  }
  wait_vmcnt<0>();
  C.cbar();
}

// Store one bf16 of exchange array (kind, l) at [b][i] (coherent store; completes before the flag).
template <class G>
__device__ __forceinline__ void put_bf16(const ConsumerB<G>& C, int kind, int l, int K, int b, int i, float v) {
  const __amdgpu_buffer_rsrc_t r = rsrc(C.p.ws + WSB<G>::data(kind, l));
  __builtin_amdgcn_raw_buffer_store_b16(uint16_t(f2bf(v)), r, (b * K + i) * 2, 0, 16);
}
// A lane's (up to) four consecutive rows i .. i + n - 1 of sequence b in exchange array (kind, l):
// an aligned pair in one 4-byte store, a lone value in a 2-byte one (the exchange's stores, and
// the write requests they cost, halved: config 4 +2.1%; four values in one 8-byte store where
// aligned measured -1% against pairs).
template <class G>
__device__ __forceinline__ void put_rows4(const ConsumerB<G>& C, int kind, int l, int K, int b, int i, int n,
                                          const float (&v)[4]) {
  const __amdgpu_buffer_rsrc_t r = rsrc(C.p.ws + WSB<G>::data(kind, l));
  int j = 0;
  if (n > 0 && (i & 1)) {
    __builtin_amdgcn_raw_buffer_store_b16(uint16_t(f2bf(v[0])), r, (b * K + i) * 2, 0, 16);
    j = 1;
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int jj = j + 2 * k;
    if (jj + 1 < 4 && jj + 1 < n)
      __builtin_amdgcn_raw_buffer_store_b32(pack2(v[jj], v[jj + 1]), r, (b * K + i + jj) * 2, 0, 16);
    else if (jj < 4 && jj < n)
      __builtin_amdgcn_raw_buffer_store_b16(uint16_t(f2bf(v[jj])), r, (b * K + i + jj) * 2, 0, 16);
  }
}

// Per-sequence RMS scale of the staged rows, then the rows normalised in place with
// LlamaRMSNorm rounding y = bf16(w * bf16(x * rs)) (modeling_llama.py:62-67); w from a ring segment.
// Wave w sums the squares of sequences w, w + 4, ... (lane l: 8-value chunks l and l + 64); the
// normalisation then runs over 8-value chunks of all rows, 16-byte LDS reads and writes.
template <class G>
__device__ __forceinline__ void norm_scales(ConsumerB<G>& C) {
  SmemB<G>& sm = C.sm;
  constexpr int CH = G::H / 8;
  constexpr int SPW = (BMAX + NCW - 1) / NCW;  // sequences per wave
  static_assert(CH <= 128, "two 8-value chunks per lane cover a row");
  {
    // the wave's sequences together: every load first, then the sums and their reductions, then
    // lane i forms the scale of the wave's i-th sequence (one divide / square root chain per wave)
    uint4 v[SPW][2];
#pragma unroll
    for (int i = 0; i < SPW; ++i) {
      const int b = C.cw + NCW * i;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int c = C.lane + 64 * h;
        v[i][h] = b < C.P.B && c < CH ? *reinterpret_cast<const uint4*>(sm.xs + b * G::H + c * 8)
                                      : make_uint4(0u, 0u, 0u, 0u);
      }
    }
    float s[SPW];
#pragma unroll
    for (int i = 0; i < SPW; ++i) {
      s[i] = 0.f;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t u[4] = {v[i][h].x, v[i][h].y, v[i][h].z, v[i][h].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float lo = bf_lo(u[e]), hi = bf_hi(u[e]);
          s[i] += lo * lo + hi * hi;
        }
      }
    }
    wave_sum_n<SPW>(s);
    float mine = s[0];
#pragma unroll
    for (int i = 1; i < SPW; ++i) mine = C.lane == i ? s[i] : mine;
    const int b = C.cw + NCW * C.lane;
    if (C.lane < SPW && b < C.P.B) sm.rsb[b] = rms_scale(mine, G::H);
  }
  C.cbar();
}

// 8 staged bf16 values of one row normalised: bf16(w * bf16(x * rs)) per value.
__device__ __forceinline__ uint4 norm8(uint4 x, uint4 w, float rs) {
  const uint32_t xv[4] = {x.x, x.y, x.z, x.w}, wu[4] = {w.x, w.y, w.z, w.w};
  uint32_t o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t t = pack2(bf_lo(xv[e]) * rs, bf_hi(xv[e]) * rs);
    o[e] = pack2(bf_lo(wu[e]) * bf_lo(t), bf_hi(wu[e]) * bf_hi(t));
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// The scales, then the staged rows normalised in place (the final norm, whose rows are an output,
// and the debug build, which captures them; the layers' norms are applied as the projections load
// their operands).
template <class G>
__device__ __forceinline__ void norm_staged(ConsumerB<G>& C, uint32_t segw) {
  SmemB<G>& sm = C.sm;
  constexpr int CH = G::H / 8;
  norm_scales<G>(C);
  // 8-value chunks of all rows, four per thread in flight: loads first, then the stores
  constexpr int U = 4;
  for (int i0 = C.ct; i0 < C.P.B * CH; i0 += U * NCT) {
    uint4 v[U], wv[U];
    float rs[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = min(i0 + u * NCT, C.P.B * CH - 1);
      const int b = i / CH, c = i - b * CH;
      v[u] = *reinterpret_cast<const uint4*>(sm.xs + b * G::H + c * 8);
      wv[u] = C.ring16(segw + uint32_t(c) * 16u);
      rs[u] = sm.rsb[b];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = i0 + u * NCT;
      if (i >= C.P.B * CH) continue;
      const int b = i / CH, c = i - b * CH;
      *reinterpret_cast<uint4*>(sm.xs + b * G::H + c * 8) = norm8(v[u], wv[u], rs[u]);
    }
  }
  C.cbar();
}

// This wave's share of D[row][token] = sum_k W[row][k] * X[token][k] for rows 0..15 of ring segment
// `seg` (K bf16 per row; rows past the segment read stale ring bytes and are discarded) and the
// 16 staged token rows.  Lane l holds D[4*(l/16) + j][l % 16] (v_mfma_f32_16x16x32_bf16 layout).
// With NORM the staged rows are RMS-normalised as they load (norm8 with the scales sm.rsb and the
// weights of ring segment segw), which is what norm_staged would have stored.
template <class G, int K, bool NORM = false>
__device__ __forceinline__ floatx4 mfma_part(const ConsumerB<G>& C, uint32_t seg, int w, int nw, uint32_t segw = 0) {
  constexpr int KS = K / 32;
  const int s0 = KS * w / nw, s1 = KS * (w + 1) / nw;
  const int row = C.lane & 15, kq = (C.lane >> 4) * 8;
  static_assert(!NORM || BMAX == 16, "one token per MFMA column");
  const float rs = NORM ? C.sm.rsb[row] : 0.f;
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
  for (int s = s0; s < s1; ++s) {
    const int k = s * 32 + kq;
    const uint4 a = C.ring16(seg + uint32_t(row * K + k) * 2u);
    uint4 x = *reinterpret_cast<const uint4*>(C.sm.xs + row * K + k);
    if constexpr (NORM) x = norm8(x, C.ring16(segw + uint32_t(k) * 2u), rs);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, x), acc,
                                                 0, 0, 0);
  }
  return acc;
}

// Two tiles (gate and up rows of P4), each over the full K by two waves: waves 0-1 the first,
// waves 2-3 the second; the pair sums are valid in wave 0.
template <class G, int K, bool NORM = false>
__device__ __forceinline__ void mfma_tile_pair(ConsumerB<G>& C, uint32_t seg0, uint32_t seg1, float (*tile)[256],
                                               floatx4& t0, floatx4& t1, uint32_t segw = 0) {
  const floatx4 part = mfma_part<G, K, NORM>(C, C.cw < 2 ? seg0 : seg1, C.cw & 1, 2, segw);
#pragma unroll
  for (int j = 0; j < 4; ++j) tile[C.cw][C.lane * 4 + j] = part[j];
  C.cbar();
  if (C.cw == 0)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      t0[j] = tile[0][C.lane * 4 + j] + tile[1][C.lane * 4 + j];
      t1[j] = tile[2][C.lane * 4 + j] + tile[3][C.lane * 4 + j];
    }
}

// Full tile, K split over the four waves; the partials are summed in wave order (deterministic)
// and the result is valid in wave 0.
template <class G, int K, bool NORM = false>
__device__ __forceinline__ floatx4 mfma_tile(ConsumerB<G>& C, uint32_t seg, float (*tile)[256], uint32_t segw = 0) {
  const floatx4 part = mfma_part<G, K, NORM>(C, seg, C.cw, NCW, segw);
#pragma unroll
  for (int j = 0; j < 4; ++j) tile[C.cw][C.lane * 4 + j] = part[j];
  C.cbar();
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
  if (C.cw == 0)
#pragma unroll
    for (int v = 0; v < NCW; ++v)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] += tile[v][C.lane * 4 + j];
  return acc;
}

// ------------------------------------------------------------------------------------------------
// Batched attention over this workgroup's items (sequence, KV head, chunk of cached tokens):
//   Q  one block-wide poll brings every item's 3 query heads (and, for leader items, the new
//      token's k and v) into LDS;
//   A  per item: RoPE, the KV append (leader), bf16 scores of the chunk's tokens and the per-wave
//      softmax statistics -- no barrier between items (every item has its own buffers); then one
//      barrier and each wave merges the statistics of a quarter of the items and publishes the
//      chunk (max, sum) records;
//   G  one poll of every item's chunk records gives the global max and sum of its (sequence, head);
//   B  per item: p = bf16(exp(s - M) / L) with the global statistics (HF's rounding), P.V over the
//      chunk, the four waves' partials summed in wave order after one barrier; non-leader chunks
//      publish their partial, leaders keep theirs;
//   C  leaders add the other chunks' partials in chunk order and write attn.
// Records and statistics are reused by every layer, so their tags carry the layer as well.
// ------------------------------------------------------------------------------------------------
template <class G, bool DBG>
__device__ __forceinline__ void attention_b(ConsumerB<G>& C, int l) {
  const Params& p = C.p;
  const PlanB<G>& P = C.P;
  SmemB<G>& sm = C.sm;
  const int lane = C.lane, w = C.cw;
  const uint32_t tagb = (C.tag32 << 5) | uint32_t(l);
  const uint64_t tg = uint64_t(tagb) << 32;
  auto tri = [&](int ev) { if (C.ct == 0) trace_at(p, l, ev, p.n_layers); };
  const bool dbg_attn = DBG && p.debug != nullptr && l == p.debug_layer;  // attention internals of this layer
  auto trk = [&](int k, int ev) { if (C.ct == 0 && k < 4) trace_at(p, l, ev, p.n_layers); };
  C.cbar();  // P1's reads of xs (which shares storage with sm.at) are done
  // ---- Q: every item's q (and new k / v) from the exchange words, one poll for all ----
  {
    constexpr int GPI = 5 * 64 / 2;                      // 16-byte loads (2 words) per item
    constexpr int MAXG = (IPW * GPI + NCT - 1) / NCT;
    const __amdgpu_buffer_rsrc_t r = rsrc(p.ws);
    auto word = [&](int gidx) -> int {                   // exchange word of group gidx, -1: none
      const int k = gidx / GPI, e = (gidx - k * GPI) * 2;
      const ItemB& it = sm.it[k];
      if (e < 192) return int(WS<G>::xw(X_QKV, l, it.b, it.g * 192 + e));
      if (it.c != it.C - 1) return -1;                   // only the leader needs the new token
      if (e < 256) return int(WS<G>::xw(X_QKV, l, it.b, G::H + it.g * 64 + (e - 192)));
      return int(WS<G>::xw(X_QKV, l, it.b, G::H + G::KVH * 64 + it.g * 64 + (e - 256)));
    };
    u32x4 v[MAXG];
    int wd[MAXG];
    uint32_t pend = 0;
#pragma unroll
    for (int gi = 0; gi < MAXG; ++gi) {
      const int gidx = C.ct + gi * NCT;
      wd[gi] = gidx < P.ni * GPI ? word(gidx) : -1;
      if (wd[gi] >= 0) {
        v[gi] = ld_dev128(r, uint32_t(wd[gi]) * 4u);
        pend |= 1u << gi;
      }
    }
    Spin spin(p.ws, C.tag32, 12);
    while (true) {
#pragma unroll
      for (int gi = 0; gi < MAXG; ++gi)
        if (((pend >> gi) & 1u) && C.ok2(v[gi])) {
          const int gidx = C.ct + gi * NCT, k = gidx / GPI, e = (gidx - k * GPI) * 2;
          // q heads and the new k (roped by their producers) as bf16 into qr, the new v into qb
          if (e < 256)
            *reinterpret_cast<uint32_t*>(&sm.at.qr[k][e >> 6][e & 63]) = (v[gi].x & 0xffffu) | (v[gi].z << 16);
          else
            *reinterpret_cast<float2*>(&sm.at.qb[k][e]) = make_float2(bf_lo(v[gi].x), bf_lo(v[gi].z));
          pend &= ~(1u << gi);
        }
      if (!pend) break;
      if (C.dead || !spin.again()) { C.dead = true; break; }
#pragma unroll
      for (int gi = 0; gi < MAXG; ++gi)
        if ((pend >> gi) & 1u) v[gi] = ld_dev128(r, uint32_t(wd[gi]) * 4u);
    }
  }
  C.cbar();  // every item's q (and new k, v) in LDS for all waves
  tri(4);
  // ---- A: scores and per-wave statistics of every item ----
  // Scores on the matrix cores: D[token][head] = K[token][:] . q[head][:] as 16-token tiles,
  // v_mfma_f32_16x16x32_bf16 over the 64 dimensions in two k-steps.  Lane l supplies row l%16 of A
  // (token tile*16 + l%16, 8 dimensions of piece 4s + l/16 from the ring) and column l%16 of B (the
  // roped q of head l%16 < 3, the same piece; zero for the padding heads) and receives
  // D[4(l/16) + j][l%16], i.e. head l%16's scores of tokens 4(l/16) + j.  Each wave covers whole
  // 16-token tiles; the rounding is bf16(q.k) * 1/8 as before.
  const int hq = lane & 15, pq = lane >> 4;   // MFMA column (head) and piece of this lane
  for (int k = 0; k < P.ni; ++k) {
    const ItemB it = sm.it[k];
    const int b = it.b, g = it.g;
    const bool leader = it.c == it.C - 1;
    const int T_old = it.t1 - it.t0, T = T_old + (leader ? 1 : 0);
    auto edge = [&](int q) { return q >= NCW ? T : ((T * q) / NCW) & ~15; };
    const int j0 = edge(w), j1 = edge(w + 1);
    const bool has_new = leader && j1 == T && T > j0;
    const uint32_t segk = C.next_seg(uint32_t(T_old) * 128u);
    const float* in = sm.at.qb[k];
    trk(k, 18 + 3 * k);
    C.wait_filled(C.pos);
    trk(k, 19 + 3 * k);
    // the roped pieces pq (dims 8pq .. 8pq+7) and pq + 4 (dims 32 + 8pq ..) of a head, bf16
    auto rope_pair = [&](int hv, uint32_t (&lo)[4], uint32_t (&hi)[4]) {
      const uint4 a = *reinterpret_cast<const uint4*>(&sm.at.qr[k][hv][pq * 8]);
      const uint4 c = *reinterpret_cast<const uint4*>(&sm.at.qr[k][hv][32 + pq * 8]);
      lo[0] = a.x; lo[1] = a.y; lo[2] = a.z; lo[3] = a.w;
      hi[0] = c.x; hi[1] = c.y; hi[2] = c.z; hi[3] = c.w;
    };
    uint32_t qlo[4] = {0u, 0u, 0u, 0u}, qhi[4] = {0u, 0u, 0u, 0u};
    if (hq < 3) rope_pair(hq, qlo, qhi);
    if (dbg_attn && it.c == 0 && w == 0 && hq < 3) {
      uint16_t* dq = p.debug + Dbg<G>::AQ + size_t(b) * G::H + (g * 3 + hq) * 64 + pq * 8;
      *reinterpret_cast<uint4*>(dq) = make_uint4(qlo[0], qlo[1], qlo[2], qlo[3]);
      *reinterpret_cast<uint4*>(dq + 32) = make_uint4(qhi[0], qhi[1], qhi[2], qhi[3]);
    }
    uint32_t klo[4] = {0u, 0u, 0u, 0u}, khi[4] = {0u, 0u, 0u, 0u};
    if (has_new) rope_pair(3, klo, khi);
    if (k == 0) trk(0, 38);  // diagnostics: item 0 roped
    if (has_new && sm.sSlot[b] >= 0 && hq < 2) {  // KV append (block360_kernel.inc:124-135)
      // lane 16q (k) / 16q + 1 (v) writes pieces q and q + 4 of the new token
      const long long slot = sm.sSlot[b];
      uint16_t* cache = reinterpret_cast<uint16_t*>(const_cast<void*>(sm.kvp[l]));
      const long long e = (slot / 16) * p.block_stride + (slot % 16) * p.token_stride +
                          (long long)g * p.head_stride + (hq ? p.v_off : p.k_off);
#pragma unroll
      for (int hv = 0; hv < 2; ++hv) {
        const int piece = pq + 4 * hv;
        uint32_t val[4];
        if (hq == 0) {
#pragma unroll
          for (int i = 0; i < 4; ++i) val[i] = hv ? khi[i] : klo[i];
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) val[i] = pack2(in[256 + piece * 8 + 2 * i], in[256 + piece * 8 + 2 * i + 1]);
        }
        uint16_t* dst = cache + e + piece * 8;
        if ((reinterpret_cast<uintptr_t>(dst) & 15u) == 0) {
          st_global16(dst, val[0], val[1], val[2], val[3]);
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            st_global2(dst + 2 * i, uint16_t(val[i] & 0xffffu));
            st_global2(dst + 2 * i + 1, uint16_t(val[i] >> 16));
          }
        }
      }
    }
    const bf16x8 bq0 = __builtin_bit_cast(bf16x8, make_uint4(qlo[0], qlo[1], qlo[2], qlo[3]));
    const bf16x8 bq1 = __builtin_bit_cast(bf16x8, make_uint4(qhi[0], qhi[1], qhi[2], qhi[3]));
    const int ntiles = (j1 - j0 + 15) / 16;
    static_assert((TCB + 1 + NCW - 1) / NCW + 15 <= 5 * 16, "a wave's tokens of an item fit 5 tiles");
    // per tile: K rows from the ring (or k_new), two MFMAs, the scores bf16(q.k) / 8 (HF) stored
    // for pass B and kept in registers (sv, -inf past the wave's tokens) for the statistics
    // every tile's K rows are read before the first MFMA, so the LDS reads overlap
    uint4 ka[5][2];
#pragma unroll
    for (int ti = 0; ti < 5; ++ti) {
      ka[ti][0] = ka[ti][1] = make_uint4(0u, 0u, 0u, 0u);
      if (ti >= ntiles) continue;
      const int tok = j0 + ti * 16 + hq;       // A row of this lane
      if (tok < T_old) {
        ka[ti][0] = C.ring16(segk + kvb_slot(tok, pq));
        ka[ti][1] = C.ring16(segk + kvb_slot(tok, pq + 4));
      } else if (tok == T_old && leader) {
        ka[ti][0] = make_uint4(klo[0], klo[1], klo[2], klo[3]);
        ka[ti][1] = make_uint4(khi[0], khi[1], khi[2], khi[3]);
      }
    }
    // every K row this wave uses is in registers: the segment goes back to the producers before
    // the MFMAs, so the next item's K streams meanwhile
    wait_lgkm0();
    C.release(C.pos);
    float sv[5][4];
#pragma unroll
    for (int ti = 0; ti < 5; ++ti) {
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) sv[ti][jj] = -INFINITY;
      if (ti >= ntiles) continue;
      floatx4 acc = {0.f, 0.f, 0.f, 0.f};
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ka[ti][0]), bq0, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ka[ti][1]), bq1, acc, 0, 0, 0);
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int t = j0 + ti * 16 + 4 * pq + jj;
        sv[ti][jj] = t < j1 ? rnd(acc[jj]) * 0.125f : -INFINITY;
        const int pos = it.t0 + t;
        if (dbg_attn && hq < 3 && t < j1 && pos < int(Dbg<G>::SEQ)) {
          p.debug[Dbg<G>::AQK + Dbg<G>::head_pos(b, g * 3 + hq, pos)] = uint16_t(f2bf(acc[jj]));
          p.debug[Dbg<G>::ASC + Dbg<G>::head_pos(b, g * 3 + hq, pos)] = uint16_t(f2bf(sv[ti][jj]));
        }
      }
    }
    // the scores of a lane's four consecutive tokens as one 8-byte store per tile, after the MFMAs.
    // Every wave's range but the last ends on a 16-token boundary, so only the last wave's final
    // group can pass its end T, writing -inf into slots T .. T + 2 of the row's padding (T <= TCB + 1).
    if (hq < 3)
#pragma unroll
      for (int ti = 0; ti < 5; ++ti) {
        const int t = j0 + ti * 16 + 4 * pq;
        if (ti < ntiles && t < j1)
          *reinterpret_cast<uint2*>(&sm.at.sc[k][hq][t]) =
              make_uint2(pack2(sv[ti][0], sv[ti][1]), pack2(sv[ti][2], sv[ti][3]));
      }
    wait_lgkm0();
    if (k == 0) trk(0, 39);  // diagnostics: item 0's score tiles stored
    // per-wave (max, sum) of each head: tile ti's head columns 0-2 move to lanes 3ti .. 3ti+2 of
    // each 16-lane row (DPP row_shr:3ti), so lane c holds head c % 3's scores of tile c / 3
    {
      const int ct = hq / 3, ch = hq - 3 * ct;
      float ev[4];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        float v = sv[0][jj];
#pragma unroll
        for (int i = 1; i < 5; ++i) {
          const float t = dpp_shr3<true>(i, sv[i][jj]);
          v = ct == i ? t : v;
        }
        ev[jj] = ct < 5 ? v : -INFINITY;
      }
      float mw[3], lw[3];
      head_totals<true>(fmaxf(fmaxf(ev[0], ev[1]), fmaxf(ev[2], ev[3])), mw);
      const float m = ch == 0 ? mw[0] : ch == 1 ? mw[1] : mw[2];
      float ls = 0.f;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) ls += ev[jj] == -INFINITY ? 0.f : __expf(ev[jj] - m);
      head_totals<false>(ls, lw);
      if (lane == 0)
#pragma unroll
        for (int h = 0; h < 3; ++h) { sm.at.wml[k][w][0][h] = mw[h]; sm.at.wml[k][w][1][h] = lw[h]; }
    }
    trk(k, 20 + 3 * k);
  }
  C.cbar();
  tri(5);
  // ---- chunk statistics: wave w merges items w, w + 4, ... (lanes 0-11: wave lane&3, head lane>>2) ----
  for (int k = w; k < P.ni; k += NCW) {
    const ItemB it = sm.it[k];
    float mq = -INFINITY, lq = 0.f;
    if (lane < 12) { mq = sm.at.wml[k][lane & 3][0][lane >> 2]; lq = sm.at.wml[k][lane & 3][1][lane >> 2]; }
    float mx = fmaxf(mq, dpp<0xb1>(mq, mq));
    mx = fmaxf(mx, dpp<0x4e>(mx, mx));
    float ex = mq == -INFINITY ? 0.f : lq * __expf(mq - mx);
    ex += dpp<0xb1>(0.f, ex);
    ex += dpp<0x4e>(0.f, ex);
    if (lane < 12 && (lane & 3) == 0) { sm.at.cst[k][0][lane >> 2] = mx; sm.at.cst[k][1][lane >> 2] = ex; }
    skew_delay(p.skew, P.wg, l, 14);
    if (it.C > 1 && lane < 12 && (lane & 3) == 0) {
      uint64_t* st = reinterpret_cast<uint64_t*>(p.ws + WSB<G>::stat(it.base + it.c));
      st_dev64(st + 2 * (lane >> 2), tg | __float_as_uint(mx));
      st_dev64(st + 2 * (lane >> 2) + 1, tg | __float_as_uint(ex));
    }
  }
  C.cbar();
  // ---- G: global statistics of every item (wave w: items w, w + 4, ...; lane kc reads chunk kc) ----
  {
    constexpr int MAXI = (IPW + NCW - 1) / NCW;
    u32x4 v[MAXI][3];
    uint32_t pend = 0;
#pragma unroll
    for (int i = 0; i < MAXI; ++i) {
      const int k = w + NCW * i;
      if (k < P.ni && sm.it[k].C > 1 && lane < sm.it[k].C) {
        const __amdgpu_buffer_rsrc_t r = rsrc(p.ws + WSB<G>::stat(sm.it[k].base));
#pragma unroll
        for (int h = 0; h < 3; ++h) v[i][h] = ld_dev128(r, uint32_t(lane * STAT_WORDS + 2 * h) * 8u);
        pend |= 1u << i;
      }
    }
    auto ok = [&](const u32x4 (&x)[3]) {
      return x[0].y == tagb && x[0].w == tagb && x[1].y == tagb && x[1].w == tagb && x[2].y == tagb &&
             x[2].w == tagb;
    };
    Spin spin(p.ws, C.tag32, 9);
    while (true) {
#pragma unroll
      for (int i = 0; i < MAXI; ++i)
        if (((pend >> i) & 1u) && ok(v[i])) pend &= ~(1u << i);
      if (!pend) break;
      if (C.dead || !spin.again()) { C.dead = true; break; }
#pragma unroll
      for (int i = 0; i < MAXI; ++i)
        if ((pend >> i) & 1u) {
          const __amdgpu_buffer_rsrc_t r = rsrc(p.ws + WSB<G>::stat(sm.it[w + NCW * i].base));
#pragma unroll
          for (int h = 0; h < 3; ++h) v[i][h] = ld_dev128(r, uint32_t(lane * STAT_WORDS + 2 * h) * 8u);
        }
    }
#pragma unroll
    for (int i = 0; i < MAXI; ++i) {
      const int k = w + NCW * i;
      if (k >= P.ni) continue;
      const int Cc = sm.it[k].C;
      if (Cc == 1) {
        if (lane < 6) sm.at.gml[k][lane / 3][lane % 3] = sm.at.cst[k][lane / 3][lane % 3];
        continue;
      }
#pragma unroll
      for (int h = 0; h < 3; ++h) {
        const bool mine = lane < Cc;
        const float mk = mine ? __uint_as_float(v[i][h].x) : -INFINITY;
        const float lk = mine ? __uint_as_float(v[i][h].z) : 0.f;
        const float m = wave_max(mk);
        const float ls = wave_sum(mk == -INFINITY ? 0.f : lk * __expf(mk - m));
        if (lane == 0) { sm.at.gml[k][0][h] = m; sm.at.gml[k][1][h] = ls; }
      }
    }
  }
  C.cbar();
  tri(6);
  // ---- B: probabilities and P.V of every item (the softmax exponentials, here and in the
  // statistics above, on the hardware exp2, __expf: within a few fp32 ulp of expf, far below the
  // bf16 rounding of p) ----
  // P.V: lane = (quarter qv, d4) owns dims 4 d4 .. 4 d4 + 3 (8 bytes of a token's V); token pairs
  // go round-robin to the four 16-lane quarters, whose sums are added at the end
  const int qv = lane >> 4, d4 = lane & 15;
  const uint32_t voff = uint32_t(d4 & 1) * 8u;
  for (int k = 0; k < P.ni; ++k) {
    const ItemB it = sm.it[k];
    const bool leader = it.c == it.C - 1;
    const int T_old = it.t1 - it.t0, T = T_old + (leader ? 1 : 0);
    auto edge = [&](int q) { return q >= NCW ? T : ((T * q) / NCW) & ~15; };
    const int j0 = edge(w), j1 = edge(w + 1);
    const bool has_new = leader && j1 == T && T > j0;
    const uint32_t segv = C.next_seg(uint32_t(T_old) * 128u);
    const float* in = sm.at.qb[k];
    {
      // the three heads' statistics and scores are read before any probability is stored
      float M[3], inv[3];
#pragma unroll
      for (int h = 0; h < 3; ++h) {
        M[h] = sm.at.gml[k][0][h];
        inv[h] = 1.0f / sm.at.gml[k][1][h];
      }
      for (int j = j0 + lane; j < j1; j += 64) {
        float s[3];
#pragma unroll
        for (int h = 0; h < 3; ++h) s[h] = bf2f(sm.at.sc[k][h][j]);
#pragma unroll
        for (int h = 0; h < 3; ++h) {
          const uint16_t pv = uint16_t(f2bf(__expf(s[h] - M[h]) * inv[h]));
          sm.at.pb[h][j] = pv;
          if (dbg_attn && it.t0 + j < int(Dbg<G>::SEQ))
            p.debug[Dbg<G>::APR + Dbg<G>::head_pos(it.b, it.g * 3 + h, it.t0 + j)] = pv;
        }
      }
    }
    wait_lgkm0();
    trk(k, 30 + 2 * k);
    C.wait_filled(C.pos);  // this item's V
    const int jo1 = min(j1, T_old);
    const int npairs = jo1 > j0 ? (jo1 - j0) / 2 : 0;
    float acc[3][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll 4
    for (int kp = qv; kp < npairs; kp += 4) {
      const int j = j0 + 2 * kp;
      const uint2 va = C.ring8(segv + kvb_slot(j, d4 >> 1) + voff);
      const uint2 vb = C.ring8(segv + kvb_slot(j + 1, d4 >> 1) + voff);
      // {v_j[d], v_j+1[d]} for the lane's four dims d
      const uint32_t v0 = __builtin_amdgcn_perm(vb.x, va.x, 0x05040100u), v1 = __builtin_amdgcn_perm(vb.x, va.x, 0x07060302u);
      const uint32_t v2 = __builtin_amdgcn_perm(vb.y, va.y, 0x05040100u), v3 = __builtin_amdgcn_perm(vb.y, va.y, 0x07060302u);
#pragma unroll
      for (int h = 0; h < 3; ++h) {
        const uint32_t pp = *reinterpret_cast<const uint32_t*>(&sm.at.pb[h][j]);
        acc[h][0] = dot2(pp, v0, acc[h][0]);
        acc[h][1] = dot2(pp, v1, acc[h][1]);
        acc[h][2] = dot2(pp, v2, acc[h][2]);
        acc[h][3] = dot2(pp, v3, acc[h][3]);
      }
    }
    if (qv == 0) {
      if (jo1 > j0 && ((jo1 - j0) & 1)) {
        const int j = jo1 - 1;
        const uint2 v = C.ring8(segv + kvb_slot(j, d4 >> 1) + voff);
        const float vf[4] = {bf_lo(v.x), bf_hi(v.x), bf_lo(v.y), bf_hi(v.y)};
#pragma unroll
        for (int h = 0; h < 3; ++h) {
          const float pj = bf2f(sm.at.pb[h][j]);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[h][i] = fmaf(pj, vf[i], acc[h][i]);
        }
      }
      if (has_new) {
#pragma unroll
        for (int h = 0; h < 3; ++h) {
          const float pj = bf2f(sm.at.pb[h][T_old]);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[h][i] = fmaf(pj, in[256 + 4 * d4 + i], acc[h][i]);
        }
      }
    }
    C.release(C.pos);  // this item's V is no longer read
#pragma unroll
    for (int h = 0; h < 3; ++h)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[h][i] = column_total<false>(acc[h][i]);
    float (*wo)[3][64] = sm.at.wo[k & 1];
    if (lane < 16)
#pragma unroll
      for (int h = 0; h < 3; ++h)
#pragma unroll
        for (int i = 0; i < 4; ++i) wo[w][h][4 * d4 + i] = acc[h][i];
    // one barrier per item: wo[k & 1] is next written by item k + 2, after the barrier of item k + 1,
    // and pb is only read by the wave that wrote it, before this barrier
    C.cbar();
    if (w < 3) {
      float O = 0.f;
#pragma unroll
      for (int v = 0; v < NCW; ++v) O += wo[v][w][lane];
      skew_delay(p.skew, P.wg, l, 15);
      if (leader) sm.at.own[k][w * 64 + lane] = O;
      else st_dev64(reinterpret_cast<uint64_t*>(p.ws + WSB<G>::rec(it.base + it.c)) + w * 64 + lane, tg | __float_as_uint(O));
    }
    trk(k, 31 + 2 * k);
  }
  tri(7);
  // ---- C: leaders add their chunks' partials (chunk order) and publish attn ----
  for (int k = 0; k < P.ni; ++k) {
    const ItemB it = sm.it[k];
    if (it.c != it.C - 1 || w >= 3) continue;
    const int Cc = it.C, base = it.base;
    float O = 0.f;
    constexpr int MB = 8;
    for (int c0 = 0; c0 < Cc - 1; c0 += MB) {
      const int nc = min(MB, Cc - 1 - c0);
      uint64_t ro[MB];
      uint32_t pend = 0;
#pragma unroll
      for (int kk = 0; kk < MB; ++kk)
        if (kk < nc) {
          ro[kk] = ld_dev64(reinterpret_cast<const uint64_t*>(p.ws + WSB<G>::rec(base + c0 + kk)) + w * 64 + lane);
          pend |= 1u << kk;
        }
      Spin spin(p.ws, C.tag32, 10);
      while (true) {
#pragma unroll
        for (int kk = 0; kk < MB; ++kk)
          if (((pend >> kk) & 1u) && uint32_t(ro[kk] >> 32) == tagb) pend &= ~(1u << kk);
        if (!pend) break;
        if (C.dead || !spin.again()) { C.dead = true; break; }
#pragma unroll
        for (int kk = 0; kk < MB; ++kk)
          if ((pend >> kk) & 1u)
            ro[kk] = ld_dev64(reinterpret_cast<const uint64_t*>(p.ws + WSB<G>::rec(base + c0 + kk)) + w * 64 + lane);
      }
#pragma unroll
      for (int kk = 0; kk < MB; ++kk)
        if (kk < nc) O += __uint_as_float(uint32_t(ro[kk]));
    }
    O += sm.at.own[k][w * 64 + lane];
    {  // lane pairs: the even lane stores both values in one 4-byte store
      const float On = dpp<0xb1>(0.f, O);  // quad_perm [1,0,3,2]: the pair's other lane
      if ((lane & 1) == 0) {
        const __amdgpu_buffer_rsrc_t r = rsrc(p.ws + WSB<G>::data(X_ATTN, l));
        __builtin_amdgcn_raw_buffer_store_b32(pack2(O, On), r, (it.b * G::H + (it.g * 3 + w) * 64 + lane) * 2, 0, 16);
      }
    }
    if (DBG && p.debug) {
      const size_t e = size_t(it.b) * G::H + (it.g * 3 + w) * 64 + lane;
      p.debug[size_t(l) * Dbg<G>::LAYER + Dbg<G>::ATTN + e] = uint16_t(f2bf(O));
      if (dbg_attn) p.debug[Dbg<G>::APV + e] = uint16_t(f2bf(O));
    }
  }
  publish_flag<G>(C, X_ATTN, l);
}

// ------------------------------------------------------------------------------------------------
// Batched consumer
// ------------------------------------------------------------------------------------------------
template <class G, bool DBG>
__device__ __forceinline__ void consumer_b(const Params& p, const PlanB<G>& P, SmemB<G>& sm, uint32_t epoch) {
  ConsumerB<G> C(p, P, sm, epoch);
  __builtin_amdgcn_s_barrier();  // pairs with the producer's barrier (blk[] ready)
  using W = WS<G>;
  const int B = P.B;
  const int nq = P.q1 - P.q0, no = P.o1 - P.o0, na = P.a1 - P.a0, nd = P.d1 - P.d0;
  const int orow = 4 * (C.lane >> 4), tok = C.lane & 15;  // this lane's MFMA output rows / token
  // debug capture (batch <= 2): stage rows of layer l; workgroup 0 copies the normalised vectors
  auto dl = [&](int l) { return p.debug + size_t(l) * Dbg<G>::LAYER; };
  auto dbg_xs = [&](uint16_t* dst) {
    if (P.wg == 0)
      for (int i = C.ct; i < B * G::H; i += NCT) dst[i] = sm.xs[i];
  };
  // Diagnostic timestamps (events per layer: 0 P1 start, 1 staged, 2 weights in, 3 QKV stored,
  // 4 attention start, 5-7 passes A-C done, 8 attn published, 9-11 P3, 12-14 P4, 15-17 P5).
  auto tr = [&](int l, int ev) { if (C.ct == 0) trace_at(p, l, ev, p.n_layers); };
  if (C.ct == 0) trace_tail(p, 0);
  // cos and sin of sequence tok's position for the two RoPE pairs of this lane's QKV slots (the same
  // in every layer; wave 0 applies them)
  float rope_c[2] = {1.f, 1.f}, rope_s[2] = {0.f, 0.f};
  if (C.cw == 0 && tok < B)
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int sl = P.q0 + orow + 2 * k;
      if (sl < (G::NH + G::KVH) * 64) {
        const size_t at = size_t(sm.sPos[tok]) * 64 + ((sl >> 1) & 31);
        rope_c[k] = p.cs_fp32 ? reinterpret_cast<const float*>(p.cos_sin)[at]
                              : bf2f(reinterpret_cast<const uint16_t*>(p.cos_sin)[at]);
        rope_s[k] = p.cs_fp32 ? reinterpret_cast<const float*>(p.cos_sin)[at + 32]
                              : bf2f(reinterpret_cast<const uint16_t*>(p.cos_sin)[at + 32]);
      }
    }
  for (int l = 0; l < p.n_layers; ++l) {
    // ---------------- P1: RMSNorm(x) + QKV ----------------
    C.refresh();
    tr(l, 0);
    {
      const uint32_t segn = C.next_seg(G::H * 2);
      const uint32_t segq = C.next_seg(uint32_t(nq) * G::H * 2);
      if (l == 0) {
        for (int i = C.ct; i < B * (G::H / 8); i += NCT) {
          const int b = i / (G::H / 8), c8 = i - b * (G::H / 8);
          *reinterpret_cast<uint4*>(sm.xs + b * G::H + c8 * 8) =
              *reinterpret_cast<const uint4*>((p.input_hidden ? p.input_hidden + size_t(b) * G::H
                                                              : p.embed + size_t(sm.sId[b]) * G::H) + c8 * 8);
        }
        C.cbar();
      } else {
        stage_flagged<G>(C, X_X, l - 1, G::H);
      }
      tr(l, 1);
      for (int i = C.ct; i < B * no; i += NCT) {
        const int b = i / no, r = i - b * no;
        sm.xk[b][r] = bf2f(sm.xs[b * G::H + P.o0 + r]);
      }
      C.wait_filled(C.pos);
      tr(l, 2);
      floatx4 acc;
      if constexpr (DBG) {
        norm_staged<G>(C, segn);
        if (p.debug) dbg_xs(dl(l) + Dbg<G>::NORM1);
        acc = mfma_tile<G, G::H>(C, segq, sm.tile);
      } else {
        norm_scales<G>(C);
        acc = mfma_tile<G, G::H, true>(C, segq, sm.tile, segn);
      }
      C.release(C.pos);
      skew_delay(p.skew, P.wg, l, 16);
      if (C.cw == 0 && tok < B) {
        // q = bf16(W x); slot pairs (orow, orow + 1), (orow + 2, orow + 3) of the q and k parts get
        // HF's RoPE, bf16(bf16(x cos) + bf16(rotate_half(x) sin)) (modeling_llama.py:138-160)
        float o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = rnd(acc[j]);
#pragma unroll
        for (int j = 0; j < 4; j += 2)
          if (P.q0 + orow + j < (G::NH + G::KVH) * 64) {
            const float x0 = o[j], x1 = o[j + 1], cs = rope_c[j / 2], sn = rope_s[j / 2];
            o[j] = rnd(rnd(x0 * cs) + rnd((-x1) * sn));
            o[j + 1] = rnd(rnd(x1 * cs) + rnd(x0 * sn));
          }
        // slots j and j + 2 are projection rows r and r + 1 (within a head or in the v part): their
        // two words {value, tag} in one 16-byte store when r is even
        const __amdgpu_buffer_rsrc_t rq = rsrc(p.ws);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int s0 = P.q0 + orow + (P.q0 + orow >= (G::NH + G::KVH) * 64 ? 2 * j : j);
          const int s1 = s0 + (P.q0 + orow >= (G::NH + G::KVH) * 64 ? 1 : 2);
          const int j0 = s0 - P.q0 - orow, j1 = s1 - P.q0 - orow;
          const bool ok0 = orow + j0 < nq, ok1 = orow + j1 < nq;
          if (!ok0) continue;
          const int r0 = qkv_row<G>(s0), r1 = qkv_row<G>(s1);
          if (ok1 && r1 == r0 + 1 && (r0 & 1) == 0) {
            const u32x4 v = {f2bf(o[j0]), C.tag32, f2bf(o[j1]), C.tag32};
            __builtin_amdgcn_raw_buffer_store_b128(v, rq, int(W::xw(X_QKV, l, tok, r0) * 4u), 0, 16);
          } else {
            st_dev64(reinterpret_cast<uint64_t*>(p.ws + W::xw(X_QKV, l, tok, r0)), C.w64(o[j0]));
            if (ok1) st_dev64(reinterpret_cast<uint64_t*>(p.ws + W::xw(X_QKV, l, tok, r1)), C.w64(o[j1]));
          }
        }
        if (DBG && p.debug)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (orow + j < nq)
              dl(l)[Dbg<G>::QKV + size_t(tok) * G::QKV + qkv_row<G>(P.q0 + orow + j)] = uint16_t(f2bf(acc[j]));
      }
      tr(l, 3);
    }
    // ---------------- P2: attention ----------------
    C.refresh();
    {
      attention_b<G, DBG>(C, l);
      tr(l, 8);
    }
    // ---------------- P3: O + residual ----------------
    C.refresh();
    {
      const uint32_t sego = C.next_seg(uint32_t(no) * G::H * 2);
      stage_flagged<G>(C, X_ATTN, l, G::H);
      tr(l, 9);
      C.wait_filled(C.pos);
      tr(l, 10);
      const floatx4 acc = mfma_tile<G, G::H>(C, sego, sm.tile);
      C.release(C.pos);
      if (C.cw == 0 && tok < B) {
        float hv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          hv[j] = orow + j < no ? sm.xk[tok][orow + j] + rnd(acc[j]) : 0.f;
          if (DBG && p.debug && orow + j < no) {
            const size_t e = size_t(tok) * G::H + P.o0 + orow + j;
            dl(l)[Dbg<G>::O + e] = uint16_t(f2bf(acc[j]));
            dl(l)[Dbg<G>::H1 + e] = uint16_t(f2bf(hv[j]));
          }
        }
        put_rows4<G>(C, X_H1, l, G::H, tok, P.o0 + orow, no - orow, hv);
      }
      publish_flag<G>(C, X_H1, l);
      tr(l, 11);
    }
    // ---------------- P4: RMSNorm(h1) + gate/up + SwiGLU ----------------
    C.refresh();
    {
      const uint32_t segn = C.next_seg(G::H * 2);
      const uint32_t segg = C.next_seg(uint32_t(na) * G::H * 2);
      const uint32_t segu = C.next_seg(uint32_t(na) * G::H * 2);
      stage_flagged<G>(C, X_H1, l, G::H);
      tr(l, 12);
      for (int i = C.ct; i < B * nd; i += NCT) {
        const int b = i / nd, r = i - b * nd;
        sm.hk[b][r] = bf2f(sm.xs[b * G::H + P.d0 + r]);
      }
      C.wait_filled(C.pos);
      tr(l, 13);
      floatx4 gt = {0.f, 0.f, 0.f, 0.f}, up = {0.f, 0.f, 0.f, 0.f};
      if constexpr (DBG) {
        norm_staged<G>(C, segn);
        if (p.debug) dbg_xs(dl(l) + Dbg<G>::NORM2);
        mfma_tile_pair<G, G::H>(C, segg, segu, sm.tile, gt, up);
      } else {
        norm_scales<G>(C);
        mfma_tile_pair<G, G::H, true>(C, segg, segu, sm.tile, gt, up, segn);
      }
      C.release(C.pos);
      if (C.cw == 0 && tok < B) {
        float av[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float gv = rnd(gt[j]), uv = rnd(up[j]);
          const float silu = rnd(gv / (1.0f + expf(-gv)));
          av[j] = silu * uv;
          if (DBG && p.debug && orow + j < na) {
            const size_t e = size_t(tok) * G::I + P.a0 + orow + j;
            dl(l)[Dbg<G>::GATE + e] = uint16_t(f2bf(gv));
            dl(l)[Dbg<G>::UP + e] = uint16_t(f2bf(uv));
            dl(l)[Dbg<G>::SILU + e] = uint16_t(f2bf(silu));
            dl(l)[Dbg<G>::ACT + e] = uint16_t(f2bf(silu * uv));
          }
        }
        put_rows4<G>(C, X_ACT, l, G::I, tok, P.a0 + orow, na - orow, av);
      }
      publish_flag<G>(C, X_ACT, l);
      tr(l, 14);
    }
    // ---------------- P5: down + residual ----------------
    C.refresh();
    {
      const uint32_t segd = C.next_seg(uint32_t(nd) * G::I * 2);
      stage_flagged<G>(C, X_ACT, l, G::I, P.db0, P.db1);
      tr(l, 15);
      C.wait_filled(C.pos);
      tr(l, 16);
      const floatx4 acc = mfma_tile<G, G::I>(C, segd, sm.tile);
      C.release(C.pos);
      if (C.cw == 0 && tok >= P.db0 && tok < P.db1) {
        float yv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float y = orow + j < nd ? rnd(sm.hk[tok][orow + j] + rnd(acc[j])) : 0.f;
          yv[j] = y;
          if (orow + j < nd) {
            if (DBG && p.debug) {
              const size_t e = size_t(tok) * G::H + P.d0 + orow + j;
              dl(l)[Dbg<G>::DOWN + e] = uint16_t(f2bf(acc[j]));
              dl(l)[Dbg<G>::OUT + e] = uint16_t(f2bf(y));
            }
            if (p.layer_outputs) p.layer_outputs[(size_t(l) * B + tok) * G::H + P.d0 + orow + j] = uint16_t(f2bf(y));
          }
        }
        put_rows4<G>(C, X_X, l, G::H, tok, P.d0 + orow, nd - orow, yv);
      }
      publish_flag<G>(C, X_X, l);
      tr(l, 17);
    }
  }
  // ---------------- final RMSNorm + LM head + argmax ----------------
  const uint32_t segf = C.next_seg(G::H * 2);
  stage_flagged<G>(C, X_X, p.n_layers - 1, G::H);
  C.wait_filled(C.pos);
  norm_staged<G>(C, segf);
  C.release(C.pos);
  if (P.wg == 0)
    for (int i = C.ct; i < B * G::H; i += NCT) p.out_hidden[i] = sm.xs[i];
  // LM segment j (16 rows, one MFMA tile over the full K) is computed by wave j % NCW (none
  // without the LM head)
  float best = -INFINITY;
  int bidx = 0x7fffffff;
  for (int j = 0; j < P.n_lm; ++j) {
    const int r0 = P.v0 + j * LM_ROWS;
    const int nrows = min(LM_ROWS, P.v1 - r0);
    const uint32_t seg = C.next_seg(uint32_t(nrows) * G::H * 2);
    if (j % NCW != C.cw) {  // another wave's segment: this wave will not read it
      C.release(C.pos);
      continue;
    }
    C.wait_filled(C.pos);
    const floatx4 acc = mfma_part<G, G::H>(C, seg, 0, 1);
    C.release(C.pos);
    if (tok < B)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
        if (orow + jj < nrows) {
          const float v = rnd(acc[jj]);
          const int idx = r0 + orow + jj;
          if (v > best || (v == best && idx < bidx)) { best = v; bidx = idx; }
          if (p.out_logits) p.out_logits[size_t(tok) * G::V + idx] = uint16_t(f2bf(acc[jj]));
        }
  }
  C.release(C.pos);
#pragma unroll
  for (int o = 16; o <= 32; o <<= 1) {  // lanes l, l+16, l+32, l+48 hold the same token
    const float ov = __shfl_xor(best, o);
    const int oi = __shfl_xor(bidx, o);
    if (ov > best || (ov == best && oi < bidx)) { best = ov; bidx = oi; }
  }
  if (C.lane < BMAX) { sm.lm_val[C.cw][C.lane] = best; sm.lm_idx[C.cw][C.lane] = bidx; }
  C.cbar();
  if (C.ct == 0) trace_tail(p, 1);
  if (C.ct < B) {
    float bv = sm.lm_val[0][C.ct];
    int bi = sm.lm_idx[0][C.ct];
    for (int v = 1; v < NCW; ++v)
      if (sm.lm_val[v][C.ct] > bv || (sm.lm_val[v][C.ct] == bv && sm.lm_idx[v][C.ct] < bi)) {
        bv = sm.lm_val[v][C.ct];
        bi = sm.lm_idx[v][C.ct];
      }
    const uint32_t idx = C.dead ? LM_DEAD : p.lm_head ? uint32_t(bi) & 0xffffu : LM_NONE;
    const uint64_t rec = (uint64_t(C.tag32) << 32) | (uint64_t(idx) << 16) | f2bf(bv);
    skew_delay(p.skew, P.wg, p.n_layers, 13);
    st_dev64(reinterpret_cast<uint64_t*>(p.ws + W::lm(C.ct, P.wg)), rec);
  }
  if (P.wg != 0) {
    if (p.out_logits && (C.dead || aborted(p.ws, C.tag32)))  // this workgroup's logits rows are not valid
      for (int b = 0; b < B; ++b)
        for (int i = P.v0 + C.ct; i < P.v1; i += NCT) p.out_logits[size_t(b) * G::V + i] = 0x7fc0;
    return;
  }
  C.cbar();  // lm_val is reused below
  uint32_t bad = 0;
  // workgroup 0: per sequence, argmax over the NWG candidates (first index on ties, as torch.argmax)
  for (int b = 0; b < B; ++b) {
    const uint64_t* src = reinterpret_cast<const uint64_t*>(p.ws + W::lm(b, C.ct));
    Spin spin(p.ws, C.tag32, 11);
    uint64_t r = ld_dev64(src);
    while (uint32_t(r >> 32) != C.tag32) {
      if (!spin.again()) { bad = 1; break; }
      r = ld_dev64(src);
    }
    float bv = bf2f(uint32_t(r) & 0xffffu);
    int bi = int((uint32_t(r) >> 16) & 0xffffu);
    bad |= (bi == int(LM_DEAD)) ? 1u : 0u;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o);
      const int oi = __shfl_xor(bi, o);
      if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
    }
    if (C.lane == 0) { sm.lm_val[C.cw][b] = bv; sm.lm_idx[C.cw][b] = bi; }
  }
  const bool any_bad = __builtin_amdgcn_ballot_w64(bad != 0u) != 0ull;
  if (C.lane == 0) sm.red[C.cw] = any_bad ? 1.f : 0.f;
  C.cbar();
  bool fail = C.dead || aborted(p.ws, C.tag32);
  for (int w = 0; w < NCW; ++w) fail = fail || sm.red[w] != 0.f;
  if (C.ct < B) {
    float bv = sm.lm_val[0][C.ct];
    int bi = sm.lm_idx[0][C.ct];
    for (int v = 1; v < NCW; ++v)
      if (sm.lm_val[v][C.ct] > bv || (sm.lm_val[v][C.ct] == bv && sm.lm_idx[v][C.ct] < bi)) {
        bv = sm.lm_val[v][C.ct];
        bi = sm.lm_idx[v][C.ct];
      }
    if (p.out_ids) p.out_ids[C.ct] = fail ? -1 : bi;
  }
  if (fail)
    for (int b = 0; b < B; ++b) {
      step_failed(p, C.tag32, C.ct, b);
      if (p.out_logits)  // every logits row of the sequence (best effort: see step_failed)
        for (int i = C.ct; i < G::V; i += NCT) p.out_logits[size_t(b) * G::V + i] = 0x7fc0;
    }
}

template <class G, bool DBG = false>
__global__ void __launch_bounds__(WG_THREADS, 1) decode_kernel_b(Params p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_raw[];
  SmemB<G>& sm = *reinterpret_cast<SmemB<G>*>(smem_raw);
  if (threadIdx.x == 0) {
    for (int w = 0; w < NPW; ++w) sm.front[w] = 0;
    for (int w = 0; w < NCW; ++w) sm.consumed[w] = 0;
    sm.cbar = 0;
  }
  for (int i = threadIdx.x; i < p.n_layers; i += WG_THREADS) {
    const void* const* t = p.layers + size_t(i) * 6;
    LayerW w{};
    w.norm1 = t[0]; w.qkv = t[1]; w.o = t[2]; w.norm2 = t[3]; w.gate_up = t[4]; w.down = t[5];
    sm.lw[i] = w;
    sm.kvp[i] = p.kv[i];
  }
  if (threadIdx.x < p.B) {
    const int t = threadIdx.x;
    sm.sS[t] = min(max(p.seq_lens[t], 1), p.max_seq);
    sm.sPos[t] = int(max(p.positions[t], (int64_t)0));
    sm.sSlot[t] = p.slot_mapping[t];
    const long long id = p.ids_i64 ? reinterpret_cast<const int64_t*>(p.input_ids)[t]
                                   : reinterpret_cast<const int32_t*>(p.input_ids)[t];
    sm.sId[t] = int(min(max(id, 0LL), (long long)G::V - 1));
  }
  trace_begin(p);
  __syncthreads();
  PlanB<G> P;
  P.init(p, sm.sS, blockIdx.x);
  const uint32_t epoch = step_epoch(p.ws);
  if (threadIdx.x < 64 * NPW) {
    producer_b<G>(p, P, sm, epoch);
  } else {
    // the consumer waves are the step's critical path: their instructions win the SIMD's issue
    // over the producer waves' DMA issue and ring polling when both are ready (+4.7% at config 4)
    __builtin_amdgcn_s_setprio(1);
    consumer_b<G, DBG>(p, P, sm, epoch);
  }
  __syncthreads();
  if (blockIdx.x == 0 && threadIdx.x == 0) st_dev(p.ws + HDR_EPOCH, epoch);
  trace_end(p);
}

template <class G>
constexpr size_t lds_bytes() { return sizeof(Smem<G>); }
constexpr size_t trace_offset(size_t lds) { return (lds + 15) & ~size_t(15); }
template <class G>
constexpr size_t lds_bytes_b() { return sizeof(SmemB<G>); }
static_assert(sizeof(SmemB<G360>) <= 160 * 1024, "LDS budget of one gfx950 workgroup");
static_assert(sizeof(SmemB<G135>) <= 160 * 1024, "LDS budget of one gfx950 workgroup");
static_assert(sizeof(Smem<G360>) <= 160 * 1024, "LDS budget of one gfx950 workgroup");
static_assert(sizeof(Smem<G135>) <= 160 * 1024, "LDS budget of one gfx950 workgroup");
static_assert(sizeof(Smem<G360Q>) <= 160 * 1024, "LDS budget of one gfx950 workgroup");
static_assert(trace_offset(sizeof(SmemB<G360>)) + TRACE_LDS_BYTES <= 160 * 1024 &&
                  trace_offset(sizeof(SmemB<G135>)) + TRACE_LDS_BYTES <= 160 * 1024 &&
                  trace_offset(sizeof(Smem<G360>)) + TRACE_LDS_BYTES <= 160 * 1024 &&
                  trace_offset(sizeof(Smem<G135>)) + TRACE_LDS_BYTES <= 160 * 1024 &&
                  trace_offset(sizeof(Smem<G360Q>)) + TRACE_LDS_BYTES <= 160 * 1024,
              "room for the diagnostic timestamp buffer");

// ------------------------------------------------------------------------------------------------
// MXFP8 quantisation of bf16 weights: per 32 consecutive elements of a row, scale code
// s = e8m0(amax / 448) rounded toward +inf (saturating at 254), then each element becomes
// e4m3(bf16(x * 2^(127-s))) with round-to-nearest-even and saturation to +-448
// (the OCP MX rule as prime_kernels/rmsnorm/test.cu:126-144 applies it).  One thread per block.
// ------------------------------------------------------------------------------------------------
__device__ __forceinline__ uint32_t e8m0_ceil(float f) {
  if (f != f) return 255u;
  const uint32_t u = __float_as_uint(f);
  const uint32_t e = (u >> 23) & 255u, m = u & 0x7fffffu;
  if (e == 255u) return 254u;
  if (e == 0u) return m > 0x400000u ? 1u : 0u;  // zero and values up to 2^-127 -> 2^-127
  const uint32_t c = e + (m ? 1u : 0u);
  return c > 254u ? 254u : c;
}

__device__ __forceinline__ uint32_t e4m3_sat(float v) {  // v holds a bf16 value
  const uint32_t sgn = (__float_as_uint(v) >> 31) << 7;
  if (v != v) return sgn | 0x7fu;
  const float a = fabsf(v);
  if (a >= 448.f) return sgn | 0x7eu;
  if (a < 0.015625f) return sgn | uint32_t(__builtin_rintf(a * 512.f));  // subnormal steps of 2^-9
  int e = int((__float_as_uint(a) >> 23) & 255u) - 127;
  const float mant = a * __uint_as_float(uint32_t(127 - e) << 23);  // in [1, 2), exact
  uint32_t m = uint32_t(__builtin_rintf((mant - 1.f) * 8.f));
  if (m == 8u) { m = 0u; ++e; }
  return sgn | (uint32_t(e + 7) << 3) | m;
}

__global__ void __launch_bounds__(256) quantize_mxfp8(const uint16_t* src, uint8_t* q, uint8_t* sc, int rows,
                                                      int cols, int sk) {
  const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
  if (t >= (long long)rows * sk) return;
  const int row = int(t / sk), blk = int(t % sk);
  uint8_t* srow = sc + size_t(row) * sk;
  if (blk >= cols / 32) {  // row padding of the scale array
    srow[blk] = 0;
    return;
  }
  const uint16_t* x = src + size_t(row) * cols + size_t(blk) * 32;
  float amax = 0.f;
  for (int k = 0; k < 32; ++k) amax = fmaxf(amax, fabsf(bf2f(x[k])));
  const uint32_t code = e8m0_ceil(amax * (1.f / 448.f));
  const float inv = __uint_as_float(code >= 254u ? 0x00400000u : (254u - code) << 23);  // 2^(127-s)
  uint32_t packed[8];
  for (int k = 0; k < 32; k += 4) {
    uint32_t w = 0;
    for (int i = 0; i < 4; ++i) w |= e4m3_sat(rnd(bf2f(x[k + i]) * inv)) << (8 * i);
    packed[k / 4] = w;
  }
  uint4* qo = reinterpret_cast<uint4*>(q + size_t(row) * cols + size_t(blk) * 32);
  qo[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
  qo[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
  srow[blk] = uint8_t(code);
}

struct DeviceInfo {
  int ok = 0, status = 0, cus = 0, coop = 0, max_lds = 0, gfx950 = 0;
};

static DeviceInfo query_device() {
  DeviceInfo d;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) { d.status = e; return d; }
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, dev);
  if (e != hipSuccess) { d.status = e; return d; }
  d.cus = prop.multiProcessorCount;
  d.gfx950 = __builtin_strncmp(prop.gcnArchName, "gfx950", 6) == 0;
  e = hipDeviceGetAttribute(&d.coop, hipDeviceAttributeCooperativeLaunch, dev);
  if (e != hipSuccess) { d.status = e; return d; }
  e = hipDeviceGetAttribute(&d.max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
  if (e != hipSuccess) { d.status = e; return d; }
  d.ok = 1;
  return d;
}

// Per-device launch state: properties are queried and the LDS attribute set once per device.
template <class G>
struct LaunchCache {
  static constexpr int MAX_DEV = 64;
  int ready[MAX_DEV] = {};
  int status[MAX_DEV] = {};
};

// Library options (pk_set_option), initialised from the environment: PK_LAUNCH=cooperative makes
// every decode launch cooperative (hipLaunchCooperativeKernel, 18 us more per step than an ordinary
// launch of the same grid at batch 1, context 1024; the grid is one workgroup per CU either way, and
// the results are the same bits), PK_SPLIT_ROLE=0 keeps batch-1 steps on the general kernel,
// PK_SPLIT_WIDE=0 sends contexts beyond the narrow split-role limit to the general kernel.
struct Options {
  int cooperative = -1;
  int split_role = -1;
  int split_wide = -1;
  int l2_records = 1;
  uint32_t skew = 0;
};
static Options g_opt;
static int opt_cooperative() {
  if (g_opt.cooperative < 0) {
    const char* e = getenv("PK_LAUNCH");
    g_opt.cooperative = (e && __builtin_strcmp(e, "cooperative") == 0) ? 1 : 0;
  }
  return g_opt.cooperative;
}
static int opt_split_role() {
  if (g_opt.split_role < 0) {
    const char* e = getenv("PK_SPLIT_ROLE");
    g_opt.split_role = (e && e[0] == '0') ? 0 : 1;
  }
  return g_opt.split_role;
}
static int opt_split_wide() {
  if (g_opt.split_wide < 0) {
    const char* e = getenv("PK_SPLIT_WIDE");
    g_opt.split_wide = (e && e[0] == '0') ? 0 : 1;
  }
  return g_opt.split_wide;
}

// ------------------------------------------------------------------------------------------------
// Library-owned exchange state.  Every exchange word carries the step epoch, so the memory the
// kernels exchange through must hold nothing the library did not write.  The library allocates it
// per device on first use (pk_init, or the first decode call) -- uncached device memory for the
// exchange words (header: epoch, abort word, wait site), ordinary device memory for the batch-1
// records that stay in one XCD's L2, and a pinned host word pair the kernels set when a step gave up
// a bounded wait -- zeroes it once and keeps it until the process ends (uncached memory that a kernel
// has read is never returned to the allocator).  A caller's scratch buffer (the reference ABI's
// `scratch`) is checked for presence and size only and carries nothing between calls.  As with the
// reference's per-device scratch, steps on one device must not run concurrently from two streams.
// ------------------------------------------------------------------------------------------------
struct DevState {
  int dev;
  uint32_t* ws;     // uncached: general layout, then the split-role region
  uint32_t* rec;    // ordinary: general batch-1 records, then the split-role group-A records
  uint32_t* host;   // pinned host memory: [0] epoch of the last step that gave up a wait, [1] its wait site
  uint32_t* host_dev;
};
constexpr int MAX_STATES = 64;
static std::mutex g_state_mu;
static DevState g_states[MAX_STATES];
static int g_nstates = 0;

static constexpr size_t round_up(size_t n, size_t a) { return (n + a - 1) / a * a; }
static constexpr size_t ws_general_bytes() {
  return round_up((WSB<G360>::TOTAL > WSB<G135>::TOTAL ? WSB<G360>::TOTAL : WSB<G135>::TOTAL) * 4, 4096);
}
static constexpr size_t rec_general_bytes() {
  return round_up((WS<G360>::XREC_WORDS > WS<G135>::XREC_WORDS ? WS<G360>::XREC_WORDS : WS<G135>::XREC_WORDS) * 4, 4096);
}
static size_t ws_bytes() { return ws_general_bytes() + round_up(sr_region_bytes(1), 4096); }
// the split-role group-A records: the narrow layout's, then the wide layout's (separate lines, so
// that no XCD's L2 holds a line another layout writes from another XCD)
static size_t rec_wide_off() { return rec_general_bytes() + round_up(sr_local_bytes(0), 4096); }
static size_t rec_bytes() { return rec_wide_off() + round_up(sr_local_bytes(1), 4096); }

__global__ void __launch_bounds__(256) zero_fill(uint4* p, size_t n) {
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

static int get_state(const void* stream, DevState** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lk(g_state_mu);
  for (int i = 0; i < g_nstates; ++i)
    if (g_states[i].dev == dev) {
      *out = &g_states[i];
      return PK_OK;
    }
  if (g_nstates == MAX_STATES) return PK_ERR_STATE;
  // the allocation and zero fill cannot be captured: a first use under capture is refused
  if (stream) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(reinterpret_cast<hipStream_t>(const_cast<void*>(stream)), &cs);
    if (e != hipSuccess) return e;
    if (cs != hipStreamCaptureStatusNone) return PK_ERR_CAPTURE;
  }
  DevState st{};
  st.dev = dev;
  if (hipExtMallocWithFlags(reinterpret_cast<void**>(&st.ws), ws_bytes(), hipDeviceMallocUncached) != hipSuccess)
    return PK_ERR_STATE;
  if (hipMalloc(reinterpret_cast<void**>(&st.rec), rec_bytes()) != hipSuccess) return PK_ERR_STATE;
  if (hipHostMalloc(reinterpret_cast<void**>(&st.host), 64, hipHostMallocMapped) != hipSuccess) return PK_ERR_STATE;
  if (hipHostGetDevicePointer(reinterpret_cast<void**>(&st.host_dev), st.host, 0) != hipSuccess) return PK_ERR_STATE;
  for (int i = 0; i < 16; ++i) st.host[i] = 0u;
  hipLaunchKernelGGL(zero_fill, dim3(2048), dim3(256), 0, nullptr, reinterpret_cast<uint4*>(st.ws), ws_bytes() / 16);
  hipLaunchKernelGGL(zero_fill, dim3(2048), dim3(256), 0, nullptr, reinterpret_cast<uint4*>(st.rec), rec_bytes() / 16);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  if ((e = hipDeviceSynchronize()) != hipSuccess) return e;
  g_states[g_nstates] = st;
  *out = &g_states[g_nstates++];
  return PK_OK;
}

// A step on this state gave up a bounded wait since the last call: report it once.
static int take_abort(DevState* st) {
  const uint32_t ep = __atomic_load_n(&st->host[0], __ATOMIC_ACQUIRE);
  if (ep == 0u) return PK_OK;
  __atomic_store_n(&st->host[0], 0u, __ATOMIC_RELEASE);
  return PK_ERR_ABORTED;
}

// ------------------------------------------------------------------------------------------------
// State of pk_decode_noalloc: one fixed array per device, compiled into the library, holding the
// split-role kernel's header words, exchange region and group-A records.  In host code `scratch`
// only names the variable for the runtime: its device address, which differs per device, comes
// from hipGetSymbolAddress once per device (with that device current) and only that address is
// used.  Nothing here allocates.
// ------------------------------------------------------------------------------------------------
namespace noalloc {
constexpr size_t HDR_BYTES = 4096;  // header words: step epoch, abort word, wait site
static __device__ __align__(256) uint8_t scratch[PK_NOALLOC_SCRATCH_BYTES];
struct Dev {
  uint8_t* ptr;  // device address of this device's `scratch`
  int cleared;   // a fill outside any capture has been issued
};
static std::mutex mu;
static Dev devs[MAX_STATES];  // by device ordinal
static size_t region_off() { return HDR_BYTES; }
static size_t local_off() { return HDR_BYTES + round_up(sr_region_bytes(0), 4096); }
static size_t used_bytes() { return local_off() + round_up(sr_local_bytes(0), 4096); }

// The current device's array, cleared before its first use by a fill on `stream` (under capture
// the fill is recorded, so every replay of the graph clears the array before its own step).  With
// `sync`, the fill is waited for.  Called with `mu` held.
static int base_locked(hipStream_t stream, bool sync, uint8_t** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= MAX_STATES) return PK_ERR_STATE;
  Dev& d = devs[dev];
  if (!d.ptr) {
    void* q = nullptr;
    if ((e = hipGetSymbolAddress(&q, HIP_SYMBOL(scratch))) != hipSuccess) return e;
    if (!q || used_bytes() > PK_NOALLOC_SCRATCH_BYTES) return PK_ERR_STATE;
    d.ptr = static_cast<uint8_t*>(q);
  }
  if (!d.cleared) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if ((e = hipStreamIsCapturing(stream, &cs)) != hipSuccess) return e;
    hipLaunchKernelGGL(zero_fill, dim3(1024), dim3(256), 0, stream, reinterpret_cast<uint4*>(d.ptr),
                       used_bytes() / 16);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if (cs == hipStreamCaptureStatusNone) {
      if (sync && (e = hipStreamSynchronize(stream)) != hipSuccess) return e;
      d.cleared = 1;
    }
  }
  *out = d.ptr;
  return PK_OK;
}
static int base(hipStream_t stream, bool sync, uint8_t** out) {
  std::lock_guard<std::mutex> lk(mu);
  return base_locked(stream, sync, out);
}
}  // namespace noalloc

template <class G, bool BATCHED, bool DBG = false>
static int launch(const Params& p, hipStream_t stream) {
  static LaunchCache<G> cache;
  const void* fn;
  size_t lds;
  if constexpr (BATCHED) {
    fn = reinterpret_cast<const void*>(decode_kernel_b<G, DBG>);
    lds = lds_bytes_b<G>();
  } else {
    fn = reinterpret_cast<const void*>(decode_kernel<G, DBG>);
    lds = lds_bytes<G>();
  }
  const size_t lds_traced = trace_offset(lds) + TRACE_LDS_BYTES;  // with the timestamp buffer
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= LaunchCache<G>::MAX_DEV) return PK_ERR_RESIDENCY;
  if (!cache.ready[dev]) {
    const DeviceInfo d = query_device();
    int st = 0;
    if (!d.ok) st = d.status;
    else if (!d.gfx950) st = PK_ERR_ARCH;
    else if (!d.coop) st = PK_ERR_COOP;
    else if (d.cus < NWG || size_t(d.max_lds) < lds_traced) st = PK_ERR_RESIDENCY;
    else {
      e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, int(lds_traced));
      if (e != hipSuccess) st = e;
    }
    cache.status[dev] = st;
    cache.ready[dev] = 1;
  }
  if (cache.status[dev]) return cache.status[dev];
  Params q = p;
  if (BATCHED) q.xws = nullptr;
  if (q.trace) {
    if (q.n_layers > TR_LAYERS) return PK_ERR_MODEL;
    q.trace_lds = uint32_t(trace_offset(lds));
    lds = lds_traced;
  }
  void* args[] = {&q};
  if (opt_cooperative()) e = hipLaunchCooperativeKernel(fn, dim3(NWG), dim3(WG_THREADS), args, lds, stream);
  else e = hipLaunchKernel(fn, dim3(NWG), dim3(WG_THREADS), args, lds, stream);
  if (e != hipSuccess) return e;
  return hipGetLastError();
}

template <class G>
static int decode_impl(void* stream, int B, int n_layers, const void* input_ids, int ids_i64,
                       const void* embed, const void* final_norm, const void* positions,
                       const void* seq_lens, const void* block_table, int bt_stride,
                       const void* slot_mapping, const void* layers, void* const* kv, long long k_off,
                       long long v_off, long long block_stride, long long token_stride,
                       long long head_stride, int block_size, const void* cos_sin, int cs_fp32,
                       void* out_hidden, void* layer_outputs, void* out_ids, void* out_logits,
                       void* scratch, size_t scratch_bytes, int max_seq_len, const void* encoded_gu = nullptr,
                       void* debug = nullptr, size_t debug_bytes = 0, int debug_layer = -1,
                       const void* input_hidden = nullptr, bool noalloc = false) {
  if (B < 1 || B > (G::WF ? 1 : BMAX)) return PK_ERR_BATCH;  // MXFP8 weights: batch 1 only
  if (debug_layer < -1 || debug_layer >= G::L) return PK_ERR_BLOCK;
  if (debug) {  // per-stage capture: the reference's SmolLM2-360M bf16 layout, at most 2 sequences
    if (G::WF || G::H != 960 || G::L != 32) return PK_ERR_DEBUG;
    if (B > int(Dbg<G>::MB)) return PK_ERR_BATCH;
    if (debug_bytes < Dbg<G>::TOTAL * 2) return PK_ERR_SCRATCH;
    if (reinterpret_cast<uintptr_t>(debug) & 15u) return PK_ERR_ALIGN;
  }
  // the lossless gate/up codec has the 360M gate_up shape [5120, 960]
  if (encoded_gu && (G::WF || G::H != 960 || G::I != 2560)) return PK_ERR_MODEL;
  if (n_layers < 1 || n_layers > G::L) return PK_ERR_MODEL;
  if (max_seq_len < 1 || max_seq_len > kMaxSeq) return PK_ERR_MAX_SEQ;
  if (!input_ids || !embed || !final_norm || !positions || !seq_lens || !block_table ||
      !slot_mapping || !layers || !kv || !cos_sin || !out_hidden || (!scratch && !noalloc))
    return PK_ERR_NULL;
  if (!noalloc && scratch_bytes < SCRATCH_BYTES) return PK_ERR_SCRATCH;
  if (block_size != 16 || bt_stride < 1 || (long long)bt_stride * block_size < max_seq_len) return PK_ERR_BLOCK;
  if (k_off % 8 || v_off % 8 || block_stride % 8 || token_stride % 8 || head_stride % 8 || k_off < 0 ||
      v_off < 0 || block_stride < 0 || token_stride < 0 || head_stride < 0)
    return PK_ERR_ALIGN;
  auto mis = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) != 0; };
  if (mis(embed) || mis(final_norm) || mis(layers) || mis(kv) || mis(out_hidden) || mis(scratch) ||
      (encoded_gu && mis(encoded_gu)) || (input_hidden && mis(input_hidden)) ||
      (layer_outputs && mis(layer_outputs)) || (out_logits && mis(out_logits)))
    return PK_ERR_ALIGN;
  Params p{};
  p.layers = reinterpret_cast<const void* const*>(layers);
  p.embed = reinterpret_cast<const uint16_t*>(embed);
  p.final_norm = reinterpret_cast<const uint16_t*>(final_norm);
  p.input_ids = input_ids;
  p.ids_i64 = ids_i64 ? 1 : 0;
  p.kv = kv;
  p.positions = reinterpret_cast<const int64_t*>(positions);
  p.seq_lens = reinterpret_cast<const int32_t*>(seq_lens);
  p.block_table = reinterpret_cast<const int32_t*>(block_table);
  p.bt_stride = bt_stride;
  p.slot_mapping = reinterpret_cast<const int64_t*>(slot_mapping);
  p.cos_sin = cos_sin;
  p.cs_fp32 = cs_fp32 ? 1 : 0;
  p.out_hidden = reinterpret_cast<uint16_t*>(out_hidden);
  p.h_dim = G::H;
  p.l2_records = g_opt.l2_records;
  p.skew = g_opt.skew;
  p.layer_outputs = reinterpret_cast<uint16_t*>(layer_outputs);
  p.out_logits = reinterpret_cast<uint16_t*>(out_logits);
  p.out_ids = reinterpret_cast<int64_t*>(out_ids);
  p.ws = reinterpret_cast<uint32_t*>(scratch);
  p.k_off = k_off;
  p.v_off = v_off;
  p.block_stride = block_stride;
  p.token_stride = token_stride;
  p.head_stride = head_stride;
  p.B = B;
  p.n_layers = n_layers;
  p.lm_head = (out_ids || out_logits) ? 1 : 0;
  p.max_seq = max_seq_len;
  p.trace = g_trace;
  p.encoded_gu = reinterpret_cast<const EncodedGULayer*>(encoded_gu);  // read by the batch-1 kernel
  p.debug = reinterpret_cast<uint16_t*>(debug);
  p.debug_layer = debug_layer;
  p.input_hidden = reinterpret_cast<const uint16_t*>(input_hidden);
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (noalloc) {  // the split-role kernel on the fixed array; no library state is touched
    if constexpr (G::WF == 0) {
      const int model = G::H == 960 ? PK_MODEL_SMOLLM2_360M : PK_MODEL_SMOLLM2_135M;
      const int lim = sr_max_seq(model, 0);
      if (B != 1 || debug || encoded_gu || input_hidden || max_seq_len > lim) return PK_ERR_NOALLOC;
      uint8_t* base = nullptr;
      const int rc = noalloc::base(s, false, &base);
      if (rc != PK_OK) return rc;
      p.ws = reinterpret_cast<uint32_t*>(base);
      p.xws = nullptr;
      p.host_status = nullptr;
      p.sr_max_s = lim;
      p.sr_min_s = 0;
      return sr_launch(model, 0, 0, p, reinterpret_cast<uint32_t*>(base + noalloc::region_off()),
                       reinterpret_cast<uint32_t*>(base + noalloc::local_off()), s, opt_cooperative());
    } else {
      return PK_ERR_NOALLOC;
    }
  }
  DevState* state = nullptr;
  const int st = get_state(stream, &state);
  if (st != PK_OK) return st;
  const int ab = take_abort(state);
  if (ab != PK_OK) return ab;
  p.ws = state->ws;
  p.xws = state->rec;
  p.host_status = state->host_dev;
  if constexpr (G::WF == 0 && G::H == 960 && G::L == 32) {  // kernels with the capture compiled in
    if (debug) return B > 1 ? launch<G, true, true>(p, s) : launch<G, false, true>(p, s);
  }
  // Batch 1: the split-role kernel's narrow layout takes contexts up to its limit, the wide layout
  // the next range, the general kernel the rest.  Each kernel that can get a context is launched;
  // each reads the context length on the device and exactly one does the step, so the host never has
  // to read it (no synchronisation, and the launches can be captured in a graph).
  auto batch1 = [&](Params p) -> int {
  if (opt_split_role() && !input_hidden) {
    const int model = G::H == 960 ? PK_MODEL_SMOLLM2_360M : PK_MODEL_SMOLLM2_135M;
    uint32_t* region = reinterpret_cast<uint32_t*>(reinterpret_cast<uint8_t*>(state->ws) + ws_general_bytes());
    uint8_t* rec = reinterpret_cast<uint8_t*>(state->rec);
    const int narrow = sr_max_seq(model, 0);
    int e = PK_OK;
    p.sr_min_s = 0;
    if (G::WF == 0) {
      // narrow builds with fewer attention chunks for the shorter contexts, where the model has them
      for (int build = 2; build <= 3; ++build) {
        const int lim = sr_max_seq(model, build);
        if (lim <= p.sr_min_s) continue;
        p.sr_max_s = lim;
        e = sr_launch(model, 0, build, p, region, reinterpret_cast<uint32_t*>(rec + rec_general_bytes()), s,
                      opt_cooperative());
        if (e != PK_OK) return e;
        if (max_seq_len <= lim) return PK_OK;  // no context can reach another kernel
        p.sr_min_s = lim;
      }
    }
    p.sr_max_s = narrow;
    e = sr_launch(model, G::WF, 0, p, region, reinterpret_cast<uint32_t*>(rec + rec_general_bytes()), s,
                  opt_cooperative());
    if (e != PK_OK) return e;
    if (max_seq_len <= p.sr_max_s) return PK_OK;  // no context can reach another kernel
    if (opt_split_wide()) {
      p.sr_min_s = narrow;
      p.sr_max_s = sr_max_seq(model, 1);
      e = sr_launch(model, G::WF, 1, p, region, reinterpret_cast<uint32_t*>(rec + rec_wide_off()), s, opt_cooperative());
      if (e != PK_OK) return e;
      if (max_seq_len <= p.sr_max_s) return PK_OK;
    }
  }
  return launch<G, false>(p, s);
  };
  if constexpr (G::WF == 0)
    if (B > 1) {
      if (B == 2 && opt_split_role() && !input_hidden && !layer_outputs) {
        // two sequences: each as a batch-1 step of its own, on the split-role kernel.  Two such steps
        // take less time than one batched step of two (360M, contexts drawn from 128..4096: 1.03
        // against 1.42 ms); from three sequences on, the batched kernel, which reads the weights
        // once for all of them, is faster (1.39 ms at three)
        for (int b = 0; b < 2; ++b) {
          Params q = p;
          q.B = 1;
          q.input_ids = static_cast<const uint8_t*>(input_ids) + b * (ids_i64 ? 8 : 4);
          q.positions = p.positions + b;
          q.seq_lens = p.seq_lens + b;
          q.block_table = p.block_table + size_t(b) * size_t(bt_stride);
          q.slot_mapping = p.slot_mapping + b;
          q.out_hidden = p.out_hidden + size_t(b) * G::H;
          q.out_ids = p.out_ids ? p.out_ids + b : nullptr;
          q.out_logits = p.out_logits ? p.out_logits + size_t(b) * G::V : nullptr;
          const int e = batch1(q);
          if (e != PK_OK) return e;
        }
        return PK_OK;
      }
      return launch<G, true>(p, s);
    }
  return batch1(p);
}

}  // namespace pk

// ------------------------------------------------------------------------------------------------
// C ABI
// ------------------------------------------------------------------------------------------------

// Diagnostics: per-phase wall-clock timestamps for the next launches (NULL disables).
// Layout: [256 workgroups][n_layers * 40 + 4] uint64.
extern "C" void pk_set_trace(void* buf) { pk::g_trace = reinterpret_cast<unsigned long long*>(buf); }

// Allocate and zero the current device's state now (outside any stream capture); later calls on
// the device use it.  Returns 0 or a status code.
extern "C" int pk_init(void) {
  pk::DevState* st = nullptr;
  const int rc = pk::get_state(nullptr, &st);
  if (rc != PK_OK) return rc;
  uint8_t* base = nullptr;
  return pk::noalloc::base(nullptr, true, &base);
}

// Options (initially from PK_LAUNCH / PK_SPLIT_ROLE): PK_OPT_COOPERATIVE 1 launches the decode
// kernels with hipLaunchCooperativeKernel, PK_OPT_SPLIT_ROLE 0 keeps batch-1 steps on the general
// kernel.  Returns the previous value, or -1 for an unknown option.
extern "C" int pk_set_option(int option, int value) {
  if (option == PK_OPT_COOPERATIVE) {
    const int old = pk::opt_cooperative();
    pk::g_opt.cooperative = value ? 1 : 0;
    return old;
  }
  if (option == PK_OPT_SPLIT_ROLE) {
    const int old = pk::opt_split_role();
    pk::g_opt.split_role = value ? 1 : 0;
    return old;
  }
  if (option == PK_OPT_L2_RECORDS) {
    const int old = pk::g_opt.l2_records;
    pk::g_opt.l2_records = value ? 1 : 0;
    return old;
  }
  if (option == PK_OPT_SPLIT_WIDE) {
    const int old = pk::opt_split_wide();
    pk::g_opt.split_wide = value ? 1 : 0;
    return old;
  }
  if (option == PK_OPT_SKEW) {
    const int old = int(pk::g_opt.skew);
    pk::g_opt.skew = uint32_t(value);
    return old;
  }
  return -1;
}

// Synchronous copy (after synchronising `stream`) of n header words of the current device's state
// (0 epoch, 1 the epoch of the last step that gave up a wait, 2 its wait site).
extern "C" int pk_state_read(void* stream, size_t word, unsigned* out, int n) {
  pk::DevState* st = nullptr;
  const int rc = pk::get_state(stream, &st);
  if (rc != PK_OK) return rc;
  if (n < 0 || word + size_t(n) > 64) return PK_ERR_BLOCK;
  hipError_t e = hipStreamSynchronize(reinterpret_cast<hipStream_t>(stream));
  if (e != hipSuccess) return e;
  return hipMemcpy(out, st->ws + word, size_t(n) * 4, hipMemcpyDeviceToHost);
}

// The pending failure report of the current device without clearing it: out[0] the epoch of the
// last step that gave up a wait (0: none since the last report), out[1] its wait site.
extern "C" int pk_state_status(void* stream, unsigned* out) {
  pk::DevState* st = nullptr;
  const int rc = pk::get_state(stream, &st);
  if (rc != PK_OK) return rc;
  out[0] = __atomic_load_n(&st->host[0], __ATOMIC_ACQUIRE);
  out[1] = __atomic_load_n(&st->host[1], __ATOMIC_ACQUIRE);
  return PK_OK;
}

// The pending failure report of the current device, cleared: the next decode call then does not
// report that step again.  out[0] the epoch (0: none), out[1] the wait site.
extern "C" int pk_state_take(void* stream, unsigned* out) {
  pk::DevState* st = nullptr;
  const int rc = pk::get_state(stream, &st);
  if (rc != PK_OK) return rc;
  out[1] = __atomic_load_n(&st->host[1], __ATOMIC_ACQUIRE);
  out[0] = __atomic_exchange_n(&st->host[0], 0u, __ATOMIC_ACQ_REL);
  return PK_OK;
}

// Test hooks (synchronous).  pk_test_set_epoch sets the step epoch of the current device's state
// (for tests that cross the 32-bit wrap); pk_test_abort_next marks the next step as already failed,
// so every bounded wait of that step gives up at its first check and the kernels end normally
// with poisoned outputs.
extern "C" int pk_test_set_epoch(void* stream, unsigned epoch) {
  pk::DevState* st = nullptr;
  const int rc = pk::get_state(stream, &st);
  if (rc != PK_OK) return rc;
  hipError_t e = hipStreamSynchronize(reinterpret_cast<hipStream_t>(stream));
  if (e != hipSuccess) return e;
  return hipMemcpy(st->ws + pk::HDR_EPOCH, &epoch, 4, hipMemcpyHostToDevice);
}
// pk_decode_noalloc's failure report, read from the header of the current device's fixed array
// (synchronises `stream`): out[0] the epoch of the last step that gave up a bounded wait (0: none
// since the array was cleared or the report last cleared), out[1] its wait site, out[2] the epoch
// of the last step.  With `clear`, the report is reset to none.  Allocates nothing.
extern "C" int pk_noalloc_status(void* stream, int clear, unsigned* out) {
  if (!out) return PK_ERR_NULL;
  out[0] = out[1] = out[2] = 0u;
  uint8_t* base = nullptr;
  {
    std::lock_guard<std::mutex> lk(pk::noalloc::mu);
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= pk::MAX_STATES) return PK_ERR_STATE;
    base = pk::noalloc::devs[dev].ptr;
  }
  if (!base) return PK_OK;  // never used on this device: no step, no failure
  hipError_t e = hipStreamSynchronize(reinterpret_cast<hipStream_t>(stream));
  if (e != hipSuccess) return e;
  uint32_t h[3] = {0u, 0u, 0u};
  if ((e = hipMemcpy(h, base, sizeof(h), hipMemcpyDeviceToHost)) != hipSuccess) return e;
  out[0] = h[pk::HDR_ABORT];
  out[1] = out[0] ? h[pk::HDR_ABORT_WHERE] : 0u;
  out[2] = h[pk::HDR_EPOCH];
  if (clear && out[0]) {
    const uint32_t z = 0u;
    if ((e = hipMemcpy(base + pk::HDR_ABORT * 4, &z, 4, hipMemcpyHostToDevice)) != hipSuccess) return e;
  }
  return PK_OK;
}

// Test hook (synchronous): the next pk_decode_noalloc step on the current device gives up each of its
// bounded waits at once (the array must have been used).
extern "C" int pk_test_abort_next_noalloc(void* stream) {
  uint8_t* base = nullptr;
  {
    std::lock_guard<std::mutex> lk(pk::noalloc::mu);
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= pk::MAX_STATES) return PK_ERR_STATE;
    base = pk::noalloc::devs[dev].ptr;
  }
  if (!base) return PK_ERR_STATE;
  hipError_t e = hipStreamSynchronize(reinterpret_cast<hipStream_t>(stream));
  if (e != hipSuccess) return e;
  uint32_t ep = 0;
  if ((e = hipMemcpy(&ep, base + pk::HDR_EPOCH * 4, 4, hipMemcpyDeviceToHost)) != hipSuccess) return e;
  ep = ep + 1u == 0u ? 1u : ep + 1u;
  return hipMemcpy(base + pk::HDR_ABORT * 4, &ep, 4, hipMemcpyHostToDevice);
}

extern "C" int pk_test_abort_next(void* stream) {
  pk::DevState* st = nullptr;
  const int rc = pk::get_state(stream, &st);
  if (rc != PK_OK) return rc;
  hipError_t e = hipStreamSynchronize(reinterpret_cast<hipStream_t>(stream));
  if (e != hipSuccess) return e;
  unsigned ep = 0;
  if ((e = hipMemcpy(&ep, st->ws + pk::HDR_EPOCH, 4, hipMemcpyDeviceToHost)) != hipSuccess) return e;
  ep = ep + 1u == 0u ? 1u : ep + 1u;
  return hipMemcpy(st->ws + pk::HDR_ABORT, &ep, 4, hipMemcpyHostToDevice);
}

// The scratch the decode entry points require.  It carries nothing between calls (all exchange
// state is the library's own), so only its presence and this size are checked.
extern "C" size_t pk_workspace_bytes(int model) {
  if (model == PK_MODEL_SMOLLM2_360M || model == PK_MODEL_SMOLLM2_135M) return pk::SCRATCH_BYTES;
  return 0;
}

extern "C" int pk_decode(void* stream, int model, int B, int n_layers, const void* input_ids, int ids_i64,
                         const void* embed, const void* final_norm, const void* positions,
                         const void* seq_lens, const void* block_table, int bt_stride,
                         const void* slot_mapping, const void* layers, void* const* kv, long long k_off,
                         long long v_off, long long block_stride, long long token_stride,
                         long long head_stride, int block_size, const void* cos_sin, int cs_fp32,
                         void* out_hidden, void* layer_outputs, void* out_ids, void* out_logits,
                         void* scratch, size_t scratch_bytes, int max_seq_len) {
  if (model == PK_MODEL_SMOLLM2_360M)
    return pk::decode_impl<pk::G360>(stream, B, n_layers, input_ids, ids_i64, embed, final_norm, positions,
                                     seq_lens, block_table, bt_stride, slot_mapping, layers, kv, k_off, v_off,
                                     block_stride, token_stride, head_stride, block_size, cos_sin, cs_fp32,
                                     out_hidden, layer_outputs, out_ids, out_logits, scratch, scratch_bytes,
                                     max_seq_len);
  if (model == PK_MODEL_SMOLLM2_135M)
    return pk::decode_impl<pk::G135>(stream, B, n_layers, input_ids, ids_i64, embed, final_norm, positions,
                                     seq_lens, block_table, bt_stride, slot_mapping, layers, kv, k_off, v_off,
                                     block_stride, token_stride, head_stride, block_size, cos_sin, cs_fp32,
                                     out_hidden, layer_outputs, out_ids, out_logits, scratch, scratch_bytes,
                                     max_seq_len);
  return PK_ERR_MODEL;
}

extern "C" int pk_decode_noalloc(void* stream, int model, int B, int n_layers, const void* input_ids, int ids_i64,
                                 const void* embed, const void* final_norm, const void* positions,
                                 const void* seq_lens, const void* block_table, int bt_stride,
                                 const void* slot_mapping, const void* layers, void* const* kv, long long k_off,
                                 long long v_off, long long block_stride, long long token_stride,
                                 long long head_stride, int block_size, const void* cos_sin, int cs_fp32,
                                 void* out_hidden, void* layer_outputs, void* out_ids, void* out_logits,
                                 int max_seq_len) {
  if (model == PK_MODEL_SMOLLM2_360M)
    return pk::decode_impl<pk::G360>(stream, B, n_layers, input_ids, ids_i64, embed, final_norm, positions,
                                     seq_lens, block_table, bt_stride, slot_mapping, layers, kv, k_off, v_off,
                                     block_stride, token_stride, head_stride, block_size, cos_sin, cs_fp32,
                                     out_hidden, layer_outputs, out_ids, out_logits, nullptr, 0, max_seq_len,
                                     nullptr, nullptr, 0, -1, nullptr, true);
  if (model == PK_MODEL_SMOLLM2_135M)
    return pk::decode_impl<pk::G135>(stream, B, n_layers, input_ids, ids_i64, embed, final_norm, positions,
                                     seq_lens, block_table, bt_stride, slot_mapping, layers, kv, k_off, v_off,
                                     block_stride, token_stride, head_stride, block_size, cos_sin, cs_fp32,
                                     out_hidden, layer_outputs, out_ids, out_logits, nullptr, 0, max_seq_len,
                                     nullptr, nullptr, 0, -1, nullptr, true);
  return PK_ERR_MODEL;
}

extern "C" int pk_decode_lossless(void* stream, int model, int B, int n_layers, const void* input_ids,
                                  int ids_i64, const void* embed, const void* final_norm, const void* positions,
                                  const void* seq_lens, const void* block_table, int bt_stride,
                                  const void* slot_mapping, const void* layers, void* const* kv, long long k_off,
                                  long long v_off, long long block_stride, long long token_stride,
                                  long long head_stride, int block_size, const void* cos_sin, int cs_fp32,
                                  void* out_hidden, void* layer_outputs, void* out_ids, void* out_logits,
                                  void* scratch, size_t scratch_bytes, int max_seq_len, const void* encoded_gu_table) {
  if (model != PK_MODEL_SMOLLM2_360M) return PK_ERR_MODEL;
  return pk::decode_impl<pk::G360>(stream, B, n_layers, input_ids, ids_i64, embed, final_norm, positions, seq_lens,
                                   block_table, bt_stride, slot_mapping, layers, kv, k_off, v_off, block_stride,
                                   token_stride, head_stride, block_size, cos_sin, cs_fp32, out_hidden, layer_outputs,
                                   out_ids, out_logits, scratch, scratch_bytes, max_seq_len, encoded_gu_table);
}

extern "C" int pk_decode_debug(void* stream, int model, int B, int n_layers, const void* input_ids, int ids_i64,
                               const void* embed, const void* final_norm, const void* positions,
                               const void* seq_lens, const void* block_table, int bt_stride,
                               const void* slot_mapping, const void* layers, void* const* kv, long long k_off,
                               long long v_off, long long block_stride, long long token_stride,
                               long long head_stride, int block_size, const void* cos_sin, int cs_fp32,
                               void* out_hidden, void* layer_outputs, void* out_ids, void* out_logits,
                               void* scratch, size_t scratch_bytes, int max_seq_len, const void* encoded_gu_table,
                               void* debug, size_t debug_bytes, int debug_layer_index) {
  if (model == PK_MODEL_SMOLLM2_360M)
    return pk::decode_impl<pk::G360>(stream, B, n_layers, input_ids, ids_i64, embed, final_norm, positions,
                                     seq_lens, block_table, bt_stride, slot_mapping, layers, kv, k_off, v_off,
                                     block_stride, token_stride, head_stride, block_size, cos_sin, cs_fp32,
                                     out_hidden, layer_outputs, out_ids, out_logits, scratch, scratch_bytes,
                                     max_seq_len, encoded_gu_table, debug, debug_bytes, debug_layer_index);
  if (model == PK_MODEL_SMOLLM2_135M)
    return pk::decode_impl<pk::G135>(stream, B, n_layers, input_ids, ids_i64, embed, final_norm, positions,
                                     seq_lens, block_table, bt_stride, slot_mapping, layers, kv, k_off, v_off,
                                     block_stride, token_stride, head_stride, block_size, cos_sin, cs_fp32,
                                     out_hidden, layer_outputs, out_ids, out_logits, scratch, scratch_bytes,
                                     max_seq_len, encoded_gu_table, debug, debug_bytes, debug_layer_index);
  return PK_ERR_MODEL;
}

extern "C" int pk_decode_mxfp8(void* stream, int model, int B, int n_layers, const void* input_ids, int ids_i64,
                               const void* embed, const void* final_norm, const void* positions,
                               const void* seq_lens, const void* block_table, int bt_stride,
                               const void* slot_mapping, const void* layers, void* const* kv, long long k_off,
                               long long v_off, long long block_stride, long long token_stride,
                               long long head_stride, int block_size, const void* cos_sin, int cs_fp32,
                               void* out_hidden, void* layer_outputs, void* out_ids, void* out_logits,
                               void* scratch, size_t scratch_bytes, int max_seq_len) {
  if (model != PK_MODEL_SMOLLM2_360M) return PK_ERR_MODEL;
  return pk::decode_impl<pk::G360Q>(stream, B, n_layers, input_ids, ids_i64, embed, final_norm, positions,
                                    seq_lens, block_table, bt_stride, slot_mapping, layers, kv, k_off, v_off,
                                    block_stride, token_stride, head_stride, block_size, cos_sin, cs_fp32,
                                    out_hidden, layer_outputs, out_ids, out_logits, scratch, scratch_bytes,
                                    max_seq_len);
}

extern "C" size_t pk_mxfp8_scale_stride(int cols) { return cols > 0 ? size_t(pk::scale_stride(cols)) : 0; }

extern "C" int pk_quantize_mxfp8(void* stream, const void* src, void* q, void* scales, int rows, int cols) {
  if (!src || !q || !scales) return PK_ERR_NULL;
  if (rows < 1 || cols < 32 || cols % 32) return PK_ERR_BLOCK;
  if ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(scales)) & 15u)
    return PK_ERR_ALIGN;
  const int sk = pk::scale_stride(cols);
  const long long n = (long long)rows * sk;
  hipLaunchKernelGGL(pk::quantize_mxfp8, dim3(unsigned((n + 255) / 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), reinterpret_cast<const uint16_t*>(src),
                     reinterpret_cast<uint8_t*>(q), reinterpret_cast<uint8_t*>(scales), rows, cols, sk);
  return hipGetLastError();
}

extern "C" int pk_query(int* cu_count, int* coop, int* max_lds_per_block, int* is_gfx950, size_t* lds_bytes) {
  const pk::DeviceInfo d = pk::query_device();
  if (!d.ok) return d.status;
  if (cu_count) *cu_count = d.cus;
  if (coop) *coop = d.coop;
  if (max_lds_per_block) *max_lds_per_block = d.max_lds;
  if (is_gfx950) *is_gfx950 = d.gfx950;
  if (lds_bytes) *lds_bytes = pk::lds_bytes<pk::G360>();
  return 0;
}

extern "C" const char* prime_decode_status_string(int status) {
  switch (status) {
    case PK_OK: return "ok";
    case PK_ERR_BATCH: return "batch_out_of_range";
    case PK_ERR_MAX_SEQ: return "max_seq_len_out_of_range";
    case PK_ERR_NULL: return "null_device_pointer";
    case PK_ERR_COOP: return "cooperative_launch_unsupported";
    case PK_ERR_RESIDENCY: return "shared_memory_or_residency_limit";
    case PK_ERR_ARCH: return "kernel_requires_gfx950";
    case PK_ERR_ALIGN: return "kv_offsets_or_pointers_not_16_byte_aligned";
    case PK_ERR_SCRATCH: return "scratch_or_debug_buffer_too_small";
    case PK_ERR_BLOCK: return "block_size_or_stride_invalid";
    case PK_ERR_MODEL: return "unknown_model_or_layer_count";
    case PK_ERR_DEBUG: return "debug_capture_unavailable";
    case PK_ERR_CAPTURE: return "first_use_of_the_device_under_stream_capture";
    case PK_ERR_ABORTED: return "a_previous_step_on_this_device_gave_up_a_bounded_wait";
    case PK_ERR_STATE: return "library_state_allocation_failed";
    case PK_ERR_NOALLOC: return "no_alloc_entry_point_takes_batch_1_bf16_weights_and_max_seq_len_up_to_its_limit";
    default: return hipGetErrorString(static_cast<hipError_t>(status));
  }
}

extern "C" size_t decode360_workspace_bytes(void) { return pk_workspace_bytes(PK_MODEL_SMOLLM2_360M); }
extern "C" size_t decode360_debug_bytes(void) { return pk::Dbg<pk::G360>::TOTAL * sizeof(uint16_t); }
extern "C" const char* decode360_status_string(int status) { return prime_decode_status_string(status); }

extern "C" int decode360(void* stream, int B, const void* input_ids, const void* embed, const void* final_norm,
                         const void* positions, const void* seq_lens, const void* block_table, int bt_stride,
                         const void* slot_mapping, const void* layers, void* const* kv, long long k_off,
                         long long v_off, long long block_stride, long long token_stride, long long head_stride,
                         int block_size, const void* cos_sin, int cs_fp32, void* out_hidden, void* layer_outputs,
                         void* scratch, size_t scratch_bytes, void* debug, size_t debug_bytes, int max_seq_len,
                         int debug_layer_index) {
  if (debug_layer_index < -1 || debug_layer_index >= pk::G360::L) return PK_ERR_BLOCK;
  return pk_decode_debug(stream, PK_MODEL_SMOLLM2_360M, B, pk::G360::L, input_ids, 0, embed, final_norm, positions,
                         seq_lens, block_table, bt_stride, slot_mapping, layers, kv, k_off, v_off, block_stride,
                         token_stride, head_stride, block_size, cos_sin, cs_fp32, out_hidden, layer_outputs, nullptr,
                         nullptr, scratch, scratch_bytes, max_seq_len, nullptr, debug, debug_bytes,
                         debug_layer_index);
}

extern "C" int decode360_lossless(void* stream, int B, const void* input_ids, const void* embed,
                                  const void* final_norm, const void* positions, const void* seq_lens,
                                  const void* block_table, int bt_stride, const void* slot_mapping, const void* layers,
                                  void* const* kv, long long k_off, long long v_off, long long block_stride,
                                  long long token_stride, long long head_stride, int block_size, const void* cos_sin,
                                  int cs_fp32, void* out_hidden, void* layer_outputs, void* scratch,
                                  size_t scratch_bytes, void* debug, size_t debug_bytes, int max_seq_len,
                                  int debug_layer_index, const void* encoded_gu_table) {
  if (debug_layer_index < -1 || debug_layer_index >= pk::G360::L) return PK_ERR_BLOCK;
  return pk_decode_debug(stream, PK_MODEL_SMOLLM2_360M, B, pk::G360::L, input_ids, 0, embed, final_norm, positions,
                         seq_lens, block_table, bt_stride, slot_mapping, layers, kv, k_off, v_off, block_stride,
                         token_stride, head_stride, block_size, cos_sin, cs_fp32, out_hidden, layer_outputs, nullptr,
                         nullptr, scratch, scratch_bytes, max_seq_len, encoded_gu_table, debug, debug_bytes,
                         debug_layer_index);
}

// ---- research single-block ABI (research/smollm2_360m_block/block360_kernel.inc:399-470) ----
// One SmolLM2-360M decoder block from hidden states [B, H] to the block output [B, H] (B = 1, 2):
// the decode kernels with the block's input in place of the embedding rows and the layer output
// taken from their layer_outputs.  The scratch holds, after the decode workspace, the one-entry
// cache table, a discarded final-normed hidden state and a capture area in the decode360 layout,
// which a small kernel repacks into the block's own stage layout (block360_kernel.inc:1-8:
// norm1, qkv, attn, h1, norm2, act, out, rows of 4 sequences).
namespace pk {
constexpr size_t BLK_MAXB = 4;
constexpr size_t BLK_NORM1 = 0, BLK_QKV = BLK_NORM1 + BLK_MAXB * 960, BLK_ATTN = BLK_QKV + BLK_MAXB * 1600,
                 BLK_H1 = BLK_ATTN + BLK_MAXB * 960, BLK_NORM2 = BLK_H1 + BLK_MAXB * 960,
                 BLK_ACT = BLK_NORM2 + BLK_MAXB * 960, BLK_OUT = BLK_ACT + BLK_MAXB * 2560,
                 BLK_DEBUG = BLK_OUT + BLK_MAXB * 960;
constexpr size_t BLK_WS = (SCRATCH_BYTES + 255) / 256 * 256;              // the decode entry's scratch
constexpr size_t BLK_KVT = BLK_WS;                                      // cache table (one pointer)
constexpr size_t BLK_HID = BLK_KVT + 256;                               // discarded final hidden [2][960]
constexpr size_t BLK_CAP = BLK_HID + 4096;                              // capture area (Dbg layout)
constexpr size_t BLK_TOTAL = BLK_CAP + (Dbg<G360>::TOTAL * 2 + 255) / 256 * 256;

__global__ void blk_table(void** slot, void* kv) {
  if (threadIdx.x == 0) *slot = kv;
}
__global__ void __launch_bounds__(256) blk_repack(const uint16_t* cap, uint16_t* dbg, int B) {
  using D = Dbg<G360>;
  const size_t src[7] = {D::NORM1, D::QKV, D::ATTN, D::H1, D::NORM2, D::ACT, D::OUT};
  const size_t dst[7] = {BLK_NORM1, BLK_QKV, BLK_ATTN, BLK_H1, BLK_NORM2, BLK_ACT, BLK_OUT};
  const int n[7] = {960, 1600, 960, 960, 960, 2560, 960};
  for (int st = 0; st < 7; ++st)
    for (int i = blockIdx.x * 256 + threadIdx.x; i < B * n[st]; i += gridDim.x * 256) {
      const int b = i / n[st], e = i - b * n[st];
      dbg[dst[st] + size_t(b) * n[st] + e] = cap[src[st] + size_t(b) * n[st] + e];
    }
}
}  // namespace pk

extern "C" size_t block360_workspace_bytes(void) { return pk::BLK_TOTAL; }
extern "C" size_t block360_debug_bytes(void) { return pk::BLK_DEBUG * sizeof(uint16_t); }
extern "C" const char* block360_status_string(int status) { return prime_decode_status_string(status); }

extern "C" int block360_decode(void* stream, int B, const void* hidden, const void* positions, const void* seq_lens,
                               const void* block_table, int bt_stride, const void* slot_mapping, const void* layer,
                               void* kv, long long k_off, long long v_off, long long block_stride,
                               long long token_stride, long long head_stride, int block_size, const void* cos_sin,
                               int cs_fp32, void* out_hidden, void* scratch, size_t scratch_bytes, void* debug,
                               size_t debug_bytes, int max_seq_len) {
  if (B < 1 || B > 2) return PK_ERR_BATCH;
  if (max_seq_len < 1 || max_seq_len > pk::kMaxSeq) return PK_ERR_MAX_SEQ;
  if (!hidden || !positions || !seq_lens || !block_table || !slot_mapping || !layer || !kv || !cos_sin ||
      !out_hidden || !scratch)
    return PK_ERR_NULL;
  if (scratch_bytes < pk::BLK_TOTAL || (debug && debug_bytes < block360_debug_bytes())) return PK_ERR_SCRATCH;
  auto mis = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) != 0; };
  if (mis(hidden) || mis(layer) || mis(kv) || mis(out_hidden) || mis(scratch) || (debug && mis(debug)))
    return PK_ERR_ALIGN;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  uint8_t* ws = static_cast<uint8_t*>(scratch);
  void** kvt = reinterpret_cast<void**>(ws + pk::BLK_KVT);
  pk::blk_table<<<1, 64, 0, s>>>(kvt, kv);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  // The block has no final norm: the decode kernel's final-normed output goes to a discarded area
  // (its norm weights: any readable [960] bf16 array, here the input itself).
  int st = pk::decode_impl<pk::G360>(stream, B, 1, hidden, 0, hidden, hidden, positions, seq_lens, block_table,
                                      bt_stride, slot_mapping, layer, kvt, k_off, v_off, block_stride, token_stride,
                                      head_stride, block_size, cos_sin, cs_fp32, ws + pk::BLK_HID, out_hidden,
                                      nullptr, nullptr, ws, pk::BLK_WS, max_seq_len, nullptr,
                                      debug ? ws + pk::BLK_CAP : nullptr, debug ? pk::Dbg<pk::G360>::TOTAL * 2 : 0,
                                      debug ? 0 : -1, hidden);
  if (st != PK_OK || !debug) return st;
  pk::blk_repack<<<32, 256, 0, s>>>(reinterpret_cast<const uint16_t*>(ws + pk::BLK_CAP),
                                    static_cast<uint16_t*>(debug), B);
  return hipGetLastError();
}

extern "C" size_t mk_workspace_bytes(int B, int max_seq_len) {
  (void)B;
  (void)max_seq_len;
  return pk_workspace_bytes(PK_MODEL_SMOLLM2_135M);
}
extern "C" const char* mk_status_string(int status) { return prime_decode_status_string(status); }

extern "C" int mk_decode(void* stream, int B, const void* input_ids, int ids_i64, const void* positions,
                         const void* seq_lens, const void* block_table, int bt_stride, const void* slot_mapping,
                         const void* layers, const void* embed, const void* final_norm, void* const* kv_layers,
                         long long k_off, long long v_off, long long block_stride, long long token_stride,
                         long long head_stride, int block_size, const void* cos_sin, int cs_fp32,
                         void* out_hidden, void* scratch, size_t scratch_bytes, int max_seq_len) {
  return pk_decode(stream, PK_MODEL_SMOLLM2_135M, B, pk::G135::L, input_ids, ids_i64, embed, final_norm,
                   positions, seq_lens, block_table, bt_stride, slot_mapping, layers, kv_layers, k_off, v_off,
                   block_stride, token_stride, head_stride, block_size, cos_sin, cs_fp32, out_hidden, nullptr,
                   nullptr, nullptr, scratch, scratch_bytes, max_seq_len);
}
