// SmolLM2 batch-1 decode step, split-role persistent kernel for gfx950 (MI355X).
//
// The 256 workgroups (one per CU, dispatched to the 8 XCDs round-robin) take one of two roles:
//   group A, the workgroups on the first AX XCDs (wg % 8 < AX): attention over the KV cache (C
//           chunks per KV head), the sum of the chunk partials and the O projection + residual -> h1;
//   group F, the others: RMSNorm + gate/up + SwiGLU, down + residual -> x, RMSNorm + the QKV
//           projection.
// Two layouts of group A are compiled:
//   narrow (AX = 1): the 32 workgroups of XCD 0, C = 32 / KVH chunks per KV head of at most 256
//           cached tokens; the O workgroups read the chunks' partial sums from XCD 0's L2;
//   wide (AX = KVH): KV head g on XCD g, 32 chunks per head of at most 304 cached tokens, for long
//           contexts; chunk c of a head adds slice c of the head's partials over the 32 chunks and
//           publishes that slice of the attention vector to every XCD.
// Per layer the data cross XCDs four times (h1 A->F, act F->F, x F->F, q/k/v F->A), five in the
// wide layout (also the attention vector); the exchanges among one KV head's chunks (softmax
// statistics, P.V partials) stay inside its XCD and go through its L2.  The two groups alternate:
// while one works, the other streams its next layer's weights (or KV chunk) into its LDS ring, so
// no workgroup has DMA in flight when it polls for data (an exchange poll issued behind outstanding
// DMA on the same CU waits for that DMA; measured, a hop costs 0.3-1.2 us more with the CU's own
// DMA in flight).
//
// Exchange format: 16-byte units {three 32-bit payload words, 32-bit step tag}, written with one
// 16-byte store and read with one 16-byte load (a payload of 6 bf16 or 3 fp32).  A reader polls a
// unit until its tag equals the step epoch and then uses the payload read by that same load: the
// scheme relies on a 16-byte store being seen whole by a 16-byte load (never the new tag with an
// old payload), which the GPU test test_gpu_safety.py::test_exchange_units_are_never_torn checks.
// Cross-XCD units live in uncached device memory (device-scope stores and loads) for pk_decode; for
// pk_decode_noalloc they live in an ordinary (cached) device array, where the device-scope (sc1)
// stores and loads alone keep them coherent across XCDs.  Group A's records live in ordinary device
// memory written with plain stores into the XCD's L2 and read with device-scope loads.  At the start
// of a launch the group-A workgroups check that the ones exchanging records really share one XCC
// (hardware register XCC_ID); if not, the records go through the uncached workspace instead.
//
// Projection weights are bf16 or MXFP8 (G::WF): e4m3 rows plus one e8m0 scale per 32 weights,
// dequantised to bf16(e4m3 * 2^(s-127)) as they are loaded into registers, so every dot product
// runs the bf16 path's v_dot2_f32_bf16 sequence on the dequantised matrix.
//
// Rounding points are those of HF eager Llama (modeling_llama.py), as in the general kernel:
// RMSNorm bf16(w * bf16(x * rsqrt(mean(x^2) + eps))), every projection bf16(W.x) with fp32
// accumulation, RoPE bf16(bf16(x cos) +- bf16(rot(x) sin)), scores bf16(q.k) / 8, softmax in fp32
// with p rounded to bf16 using the global max and sum of the head, bf16(sum p.v), residuals
// bf16(x + bf16(o)), silu bf16(g / (1 + exp(-g))), act bf16(silu * u).
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <type_traits>

#include "pk_common.h"

namespace pk {
namespace sr {

constexpr int VPU = 6;                   // bf16 values per 16-byte unit
#ifndef PK_SR_REP
#define PK_SR_REP 1
#endif
#ifndef PK_SR_UPL_360
#define PK_SR_UPL_360 2
#endif
#ifndef PK_SR_UPL_135
#define PK_SR_UPL_135 1
#endif
constexpr int REP = PK_SR_REP;           // copies of each cross-XCD unit
#ifndef PK_SR_DEPTH
#define PK_SR_DEPTH 4
#endif
// DMA packets in flight per producer wave (narrow layout; depth 2 / 3 / 4 / 6 / 8 / 12: config 3
// 2,081 / 2,112 / 2,116 / 2,114 / 2,108 / 2,108 tok/s, config 2 2,447 / 2,450 / 2,450 / 2,441 /
// 2,399 / 2,398)
constexpr int DEPTH_SR = PK_SR_DEPTH;
#ifndef PK_SR_DEPTH_W
#define PK_SR_DEPTH_W 4   // wide layout (config 5: 2 / 3 / 4 / 6 / 8 / 16 = 1,691 / 1,698 / 1,701 / 1,663 / 1,642 / 1,584 tok/s)
#endif
#ifndef PK_SR_STATS_CHUNK_W
#define PK_SR_STATS_CHUNK_W 1
#endif
#ifndef PK_SR_PRIO_W
#define PK_SR_PRIO_W 1    // wide layout: consumer waves at issue priority 1 (0: -7% at config 5)
#endif


// 16-token tiles of a chunk per consumer wave (attention): at most MT
constexpr int MT = 5;

// The kernel's geometry: the model's (G0, with its weight format G0::WF), group A's XCD count, and
// the attention chunks per KV head (0: as many as group A's workgroups allow).
template <class G0, int AX_, int CX_ = 0>
struct SrG : G0 {
  static constexpr int AX = AX_;
  static constexpr int CX = CX_;
};

template <class G>
struct SG {
  static constexpr int AX = G::AX;                      // XCDs of group A
  static constexpr bool WIDE = AX > 1;
  static constexpr int AG = 32 * AX;                    // group A workgroups
  static constexpr int FG = NWG - AG;                   // group F workgroups
  static constexpr int TCS = WIDE ? 304 : 256;          // max cached tokens per attention chunk
  static constexpr int HU = (G::H + VPU - 1) / VPU;     // units of an H-vector
  static constexpr int IU = (G::I + VPU - 1) / VPU;     // units of the act vector
  static constexpr int QU = (G::QKV + VPU - 1) / VPU;   // units of the qkv vector
  static constexpr int C = G::CX ? G::CX : AG / G::KVH;  // attention chunks per KV head
  static constexpr int NATT = C * G::KVH;
  static constexpr int PU = 22;                         // narrow: units of one head's 64 fp32 partial sums
  static constexpr int PUC = WIDE ? 64 : 3 * PU;        // partial-sum units per chunk record
  static constexpr int OU = (HU + AG - 1) / AG;         // most O units per group-A workgroup
  // gate/up + SwiGLU: on group F in the narrow layout; on every workgroup in the wide one (group A,
  // idle between its O projection and the next layer's q, takes its share after the O rows)
  static constexpr bool GU_ALL = WIDE;
  static constexpr int GUW = GU_ALL ? NWG : FG;         // workgroups sharing the act units
  static constexpr int NAU = (IU + GUW - 1) / GUW;      // most act units per workgroup
  static constexpr int NXU = (HU + FG - 1) / FG;        // most x (down) units per group-F workgroup
  static constexpr int NQU = (QU + FG - 1) / FG;        // most qkv units per group-F workgroup
  static constexpr int NIT = (2 * NAU + NCW - 1) / NCW; // gate/up 6-row items per wave (one)
  static constexpr int NPART = 2 * NAU > NCW * NXU ? 2 * NAU : NCW * NXU;  // rows of SmemSR::part
  // O rows loaded before the attention partials are polled (10 chunk records per thread leave no
  // room for them in the narrow SmolLM2-135M build without spills)
  static constexpr bool O_EARLY = WIDE || C <= 6;
  static constexpr uint32_t WB = G::WF ? 1u : 2u;       // bytes per projection weight
  static constexpr int DEPTH = WIDE ? PK_SR_DEPTH_W : DEPTH_SR;  // DMA packets in flight per producer wave
  static constexpr int PRIO = WIDE ? PK_SR_PRIO_W : 1;           // consumer waves' issue priority
  // LM-head rows per ring segment (narrow 32, 8 per consumer wave: config 3 +0.2%, config 2 +0.45%
  // against 24; wide 24: 32 gave -0.3% at config 5, -0.8% at 4096 tokens; 16: -1.5%)
  static constexpr int LMR = WIDE ? 24 : 32;
  // softmax statistics: each wave publishes its own (narrow), or each chunk combines its waves first
  // and publishes once (wide: 32 chunks x 4 waves would be 256 units for every wave to poll)
  static constexpr bool STATS_CHUNK = WIDE && PK_SR_STATS_CHUNK_W;
  __device__ static bool in_a(int wg) { return (wg & 7) < AX; }
  static_assert(G::GQA == 3 && (3 * 64) % VPU == 0 && G::H % VPU == 0, "head groups are whole units");
  static_assert(!WIDE || AX == G::KVH, "the wide layout puts one KV head on each of its XCDs");
  static_assert(C >= 1 && C <= 32 && (!WIDE || C == 32), "chunks per KV head");
  static_assert(TCS + 1 <= MT * 16 * NCW, "a chunk's tiles (and the new token) fit MT tiles per wave");
  static_assert(NQU <= NCW, "the QKV phase gives each wave at most one unit");
  static_assert(NXU <= 2 && NIT == 1, "down units and gate/up items per workgroup");
  static_assert(OU * VPU <= 8 * NCW, "the O rows fit 8 per wave");
};

// Workspace (uncached, 32-bit words), placed after the general kernels' layout (base word SR0) so
// that no word is ever read in a format it was not written in; the header (epoch, abort) is shared.
enum SKind { K_H1, K_ACT, K_X, K_XQ, K_ATT, NK };
template <class G>
struct SWS {
  using S = SG<G>;
  // cross-XCD units per 64-byte line (fewer: fewer polls per line).  360M, 2 against 1: config 3
  // +0.8%, config 5 +1.0%, 4096 tokens +3.0%; 135M, 2 against 1: config 2 -1.5%
  static constexpr int UPL = G::H == 960 ? PK_SR_UPL_360 : PK_SR_UPL_135;
  static constexpr int LINES = (S::IU + UPL - 1) / UPL;
  static constexpr int NKL = S::WIDE ? NK : K_ATT;            // vector kinds of the layout (narrow: no K_ATT)
  static constexpr int SLOTS = (G::L + 1) * NKL;
  static constexpr size_t XCC_TAB = 0;                        // the group-A XCC ids, one unit per rank
  static constexpr size_t X0 = XCC_TAB + size_t(S::AG) * 16;  // cross-XCD vectors (bytes from the region base)
  static constexpr size_t XBYTES = size_t(REP) * LINES * SLOTS * 64;
  static constexpr size_t LMR = X0 + XBYTES;                  // per-workgroup end records: NWG units
  static constexpr size_t LOC = LMR + size_t(NWG) * 16;      // group-A records when they cannot stay in L2
  // group-A records per layer, in units: statistics (2 per wave of a chunk), partials (PUC per chunk:
  // narrow, 3 heads x PU units; wide, the chunk's 192 values in order, 3 per unit)
  static constexpr size_t STAT_U = 0, PART_U = size_t(S::AG) * NCW * 2;
  static constexpr size_t LOC_LAYER = (PART_U + size_t(S::AG) * S::PUC) * 16;
  static constexpr size_t LOC_BYTES = LOC_LAYER * G::L;
  static constexpr size_t BYTES = LOC + LOC_BYTES;
  // unit u of vector (kind, layer l, copy r): UPL units per line; consecutive lines of a vector are
  // SLOTS lines apart, so one vector's lines spread over the memory channels
  __device__ static uint32_t xoff(int kind, int l, int r, int u) {
    return uint32_t(X0 + ((size_t(r) * LINES + size_t(u / UPL)) * SLOTS + size_t(l) * NKL + kind) * 64 +
                    size_t(u % UPL) * 16);
  }
  __device__ static uint32_t loc(int l, size_t unit) { return uint32_t(size_t(l) * LOC_LAYER + unit * 16); }
};

typedef __attribute__((address_space(1))) u32x4 g_u32x4_t;

template <int AUX>
__device__ __forceinline__ void st_unit(__amdgpu_buffer_rsrc_t r, uint32_t off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, int(off), 0, AUX);
}
__device__ __forceinline__ u32x4 ld_unit(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, int(off), 0, 16);  // device scope (sc1)
}

// LlamaRMSNorm's scale rsqrt(mean(x^2) + eps) with the hardware reciprocal square root (HF on the GPU
// uses an approximate rsqrt too) and the mean as sum * (1/n); within an ulp of the exact scale.
template <int N>
__device__ __forceinline__ float rms_rsq(float sumsq) {
  return rsqrtf(sumsq * (1.0f / float(N)) + 1e-5f);
}

// ------------------------------------------------------------------------------------------------
// Per-workgroup plan
// ------------------------------------------------------------------------------------------------

template <class G>
struct PlanSR {
  using GG = SG<G>;
  int wg, a, rank;
  // group F: act units [au0, au1), x units [xu0, xu1), qkv units [qu0, qu1) and their row ranges
  int au0, au1, xu0, xu1, qu0, qu1;
  int a0, a1, d0, d1, q0, q1;
  // group A: attention chunk (KV head g, chunk c of C), cached tokens [t0, t1); O units [ou0, ou1)
  int att, g, c, leader, t0, t1, S, pos;
  long long slot;
  int ou0, ou1, o0, o1;
  // LM head rows [v0, v1) in n_lm segments
  int v0, v1, n_lm;

  __device__ __forceinline__ void init(const Params& p, int wg_) {
    constexpr int AX = GG::AX;
    wg = wg_;
    a = GG::in_a(wg);
    // group A: rank c KVH + g is chunk c of KV head g (wide: head g on XCD g, chunk c = wg / 8)
    rank = a ? (wg >> 3) * AX + (wg & 7) : (wg >> 3) * (8 - AX) + (wg & 7) - AX;
    au0 = au1 = xu0 = xu1 = qu0 = qu1 = a0 = a1 = d0 = d1 = q0 = q1 = 0;
    att = g = c = leader = t0 = t1 = ou0 = ou1 = o0 = o1 = 0;
    S = min(max(p.seq_lens[0], 1), p.max_seq);
    pos = int(max(p.positions[0], (int64_t)0));
    slot = p.slot_mapping[0];
    if (a) {
      att = rank < GG::NATT;
      g = rank % G::KVH;
      c = rank / G::KVH;
      leader = att && c == GG::C - 1;
      const int old = S - 1;
      const int tc = old <= 0 ? 16 : ((old + GG::C - 1) / GG::C + 15) / 16 * 16;
      t0 = att ? min(c * tc, old) : 0;
      t1 = att ? min((c + 1) * tc, old) : 0;
      ou0 = split_lo(GG::HU, GG::AG, rank);
      ou1 = split_lo(GG::HU, GG::AG, rank + 1);
      o0 = ou0 * VPU;
      o1 = min(ou1 * VPU, G::H);
    } else {
      au0 = split_lo(GG::IU, GG::FG, rank); au1 = split_lo(GG::IU, GG::FG, rank + 1);
      xu0 = split_lo(GG::HU, GG::FG, rank); xu1 = split_lo(GG::HU, GG::FG, rank + 1);
      qu0 = split_lo(GG::QU, GG::FG, rank); qu1 = split_lo(GG::QU, GG::FG, rank + 1);
      d0 = xu0 * VPU; d1 = min(xu1 * VPU, G::H);
      q0 = qu0 * VPU; q1 = min(qu1 * VPU, G::QKV);
    }
    if (GG::GU_ALL) {
      au0 = split_lo(GG::IU, NWG, wg);
      au1 = split_lo(GG::IU, NWG, wg + 1);
    }
    a0 = au0 * VPU;
    a1 = min(au1 * VPU, G::I);
    if (p.lm_head) {
      v0 = split_lo(G::V, NWG, wg);
      v1 = split_lo(G::V, NWG, wg + 1);
    } else {
      v0 = v1 = 0;
    }
    n_lm = (v1 - v0 + GG::LMR - 1) / GG::LMR;
  }
};

// Segments in stream order.  Group F, bracket k (0 <= k <= L): the MLP of layer k-1 (norm2, gate
// rows, up rows, down rows; k >= 1) then norm1 and the QKV rows of layer k (k < L); bracket L ends
// with the final-norm weights and the LM-head segments (in the wide layout F's gate and up rows are
// its share of the act units only).  Group A, bracket k < L: the KV chunk and the O rows of layer k,
// in the wide layout then its gate/up share of layer k (norm2, gate rows, up rows); bracket L: the
// final-norm weights and the LM-head segments.
// MXFP8 weights: every weight segment (gate, up, down, QKV, O) is followed by its scale rows (the _S
// segments, scale_stride(K) bytes per row; empty for bf16 weights).
enum SRSeg { R_NORM2, R_GATE, R_GATE_S, R_GATE_H, R_GATE_R, R_UP, R_UP_S, R_UP_H, R_UP_R, R_DOWN, R_DOWN_S,
             R_NORM1, R_QKV, R_QKV_S, R_KV, R_O, R_O_S, R_FNORM, R_LM };

template <class G>
__device__ __forceinline__ uint32_t sr_bytes(const PlanSR<G>& P, int kind, int lm_index, const GUE* e = nullptr) {
  const bool enc = e != nullptr && e->on != 0u;  // this layer's gate/up through the lossless codec
  constexpr uint32_t WB = SG<G>::WB;
  constexpr uint32_t SH = G::WF ? uint32_t(scale_stride(G::H)) : 0u, SI = G::WF ? uint32_t(scale_stride(G::I)) : 0u;
  switch (kind) {
    case R_NORM2:
    case R_NORM1:
    case R_FNORM: return G::H * 2;
    case R_GATE_S:
    case R_UP_S: return uint32_t(P.a1 - P.a0) * SH;
    case R_DOWN_S: return uint32_t(P.d1 - P.d0) * SI;
    case R_QKV_S: return uint32_t(P.q1 - P.q0) * SH;
    case R_O_S: return uint32_t(P.o1 - P.o0) * SH;
    case R_GATE:
    case R_UP: return uint32_t(P.a1 - P.a0) * G::H * (enc ? 1u : WB);  // plane rows: 1 byte per weight
    case R_GATE_H:
    case R_UP_H: return enc ? uint32_t(P.a1 - P.a0) * (G::H / 8) * 4u : 0u;  // one header per 8 weights
    case R_GATE_R: return enc ? e->cnt[0] * 16u : 0u;                      // the rows' escaped chunks
    case R_UP_R: return enc ? e->cnt[1] * 16u : 0u;
    case R_DOWN: return uint32_t(P.d1 - P.d0) * G::I * WB;
    case R_QKV: return uint32_t(P.q1 - P.q0) * G::H * WB;
    case R_KV: return uint32_t(P.t1 - P.t0) * 256u;
    case R_O: return uint32_t(P.o1 - P.o0) * G::H * WB;
    default: {
      const int r0 = P.v0 + lm_index * SG<G>::LMR;
      return uint32_t(min(SG<G>::LMR, P.v1 - r0)) * G::H * 2;
    }
  }
}

// ------------------------------------------------------------------------------------------------
// Shared memory
// ------------------------------------------------------------------------------------------------

template <class G>
struct SmemSR {
  static constexpr int XS = G::I > G::H ? G::I : G::H;
  struct Attn {
    float qkvw[NCW][5 * 64];     // per-wave attention inputs (3 q heads, k_new, v_new; pre-RoPE)
  };
  uint8_t ring[RING];
  union {
    float xs[XS];                // the phase input vector (bf16 values as fp32)
    Attn at;
  };
  float keep[G::H];              // F: h1 (residual of down); A: x (residual of O, its own rows)
  float wo[NCW][3][64];          // per-wave P.V partials
  float wml[NCW][2][3];          // per-wave softmax max / sum per head (chunk-combined statistics)
  float red[NCW];
  LayerW lw[G::L];
  GUE gue[G::L];                 // group F: each layer's lossless gate/up stream of this workgroup
  const void* kvp[G::L];
  int32_t blk[SG<G>::TCS / 16 + 2];
  float lm_val[NCW];
  int32_t lm_idx[NCW];
  alignas(16) uint32_t front[NPW];
  alignas(16) uint32_t zero16[4];  // a 16-byte zero line: what lanes past the end of a row read
  float part[SG<G>::NPART][8];     // per-wave (per-item) partial results combined across the waves
  uint32_t consumed[NCW];
  uint32_t cbar;
  uint32_t go;                   // brackets the consumers have finished
  uint32_t loc_l2;               // group A: 1 when its records go through the XCD's L2
};

// ------------------------------------------------------------------------------------------------
// Producer waves: bracket k is issued once the consumers have finished bracket k-1, so the DMA of a
// bracket runs while this workgroup waits for the other group, never during its own exchanges.
// ------------------------------------------------------------------------------------------------

template <class G>
__device__ __forceinline__ void producer_sr(const Params& p, const PlanSR<G>& P, SmemSR<G>& sm, uint32_t epoch) {
  const int pw = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const uint32_t ring_base = uint32_t(reinterpret_cast<uintptr_t>(sm.ring));
  uint32_t n = 0;  // global packet index at the start of the current segment
  uint32_t room = RING;  // ring bytes the consumers have released, plus the ring size
  Spin spin(p.ws, epoch, 21);
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
  auto issue = [&](int kind, int layer, int lm_index) {
    const GUE* ge = kind >= R_GATE && kind <= R_UP_R ? &sm.gue[layer] : nullptr;
    const uint32_t bytes = sr_bytes(P, kind, lm_index, ge);
    const uint32_t npk = pad_pkt(bytes) / PKT;
    if (npk == 0 || dead) return;
    const uint8_t* base = nullptr;
    const uint8_t* cache = nullptr;
    auto u8 = [](const void* q) { return reinterpret_cast<const uint8_t*>(q); };
    const LayerW& Lw = sm.lw[layer];
    constexpr size_t WB = SG<G>::WB;
    constexpr size_t SH = scale_stride(G::H), SI = scale_stride(G::I);
    switch (kind) {
      case R_NORM2: base = u8(Lw.norm2); break;
      case R_GATE: base = ge->on ? ge->plane + size_t(P.a0) * G::H : u8(Lw.gate_up) + size_t(P.a0) * G::H * WB; break;
      case R_GATE_S: base = Lw.gate_up_s + size_t(P.a0) * SH; break;
      case R_GATE_H: base = u8(ge->hdr + size_t(P.a0) * (G::H / 8)); break;
      case R_GATE_R: base = u8(ge->raw + size_t(ge->first[0]) * 8); break;
      case R_UP:
        base = ge->on ? ge->plane + size_t(G::I + P.a0) * G::H : u8(Lw.gate_up) + size_t(G::I + P.a0) * G::H * WB;
        break;
      case R_UP_S: base = Lw.gate_up_s + size_t(G::I + P.a0) * SH; break;
      case R_UP_H: base = u8(ge->hdr + size_t(G::I + P.a0) * (G::H / 8)); break;
      case R_UP_R: base = u8(ge->raw + size_t(ge->first[1]) * 8); break;
      case R_DOWN: base = u8(Lw.down) + size_t(P.d0) * G::I * WB; break;
      case R_DOWN_S: base = Lw.down_s + size_t(P.d0) * SI; break;
      case R_NORM1: base = u8(Lw.norm1); break;
      case R_QKV:
      case R_QKV_S: break;  // rows gathered in slot order below
      case R_KV: cache = u8(sm.kvp[layer]); break;
      case R_O: base = u8(Lw.o) + size_t(P.o0) * G::H * WB; break;
      case R_O_S: base = Lw.o_s + size_t(P.o0) * SH; break;
      case R_FNORM: base = u8(p.final_norm); break;
      default: base = u8(p.embed) + size_t(P.v0 + lm_index * SG<G>::LMR) * G::H * 2; break;
    }
    for (uint32_t i = (uint32_t(pw) + NPW - n % NPW) % NPW; i < npk && !dead; i += NPW) {
      const uint32_t gn = n + i;
      // ring space: `room` is the end of the free ring as last read; the consumers' counters are read
      // again only when a packet would pass it
      if ((gn + 1) * PKT > room) {
        room = cmin() + RING;
        if ((gn + 1) * PKT > room) {
          wait_vmcnt<0>();
          publish(gn);
          while ((gn + 1) * PKT > (room = cmin() + RING))
            if (!spin.again()) { dead = true; break; }
          if (dead) break;
        }
      }
      const uint32_t off = i * PKT + uint32_t(lane) * 16u;
      const uint8_t* src;
      if (kind == R_KV) {
        // 4 tokens per packet, 256 B each: 8 K slots then 8 V slots of 16 B, slot s of token j
        // holding piece (s - j) mod 8 so that 8 consecutive tokens spread over 8 LDS banks
        const int jt = int(i) * 4 + (lane >> 4);
        const int t = P.t0 + jt;
        const int piece = (lane >> 3) & 1;
        const int part = ((lane & 7) - jt) & 7;
        const int blk = off < bytes ? sm.blk[t / 16 - P.t0 / 16] : 0;
        const long long e = (long long)blk * p.block_stride + (long long)(t & 15) * p.token_stride +
                            (long long)P.g * p.head_stride + (piece ? p.v_off : p.k_off) + part * 8;
        src = cache + e * 2;
      } else if (kind == R_QKV || kind == R_QKV_S) {
        // rows in slot order (qkv_row): byte `off` of the segment is in row q0 + off / (row bytes)
        const uint32_t rb = kind == R_QKV ? uint32_t(G::H * WB) : uint32_t(SH);
        const uint32_t ri = off / rb, cb = off - ri * rb;
        src = (kind == R_QKV ? u8(Lw.qkv) : Lw.qkv_s) + size_t(qkv_row<G>(P.q0 + int(ri))) * rb + cb;
      } else {
        src = base + off;
      }
      if (off < bytes) dma16(src, __builtin_amdgcn_readfirstlane(ring_base + ((gn * PKT) & (RING - 1))));
      wait_vmcnt<SG<G>::DEPTH>();
      if (gn >= uint32_t(SG<G>::DEPTH - 1) * NPW) publish(gn - uint32_t(SG<G>::DEPTH - 1) * NPW);
    }
    n += npk;
  };
  auto wait_go = [&](uint32_t k) {
    wait_vmcnt<0>();
    publish(n);
    while (!dead && ld_lds(&sm.go) < k) {
      if (!spin.again()) dead = true;
      __builtin_amdgcn_s_sleep(2);
    }
  };
  const int L = p.n_layers;
  for (int k = 0; k <= L && !dead; ++k) {
    if (k > 0) wait_go(uint32_t(k));
    if (P.a) {
      if (k < L) {
        issue(R_KV, k, 0);
        issue(R_O, k, 0);
        issue(R_O_S, k, 0);
        if (SG<G>::GU_ALL) {  // its gate/up share of the layer, needed after the O rows
          issue(R_NORM2, k, 0);
          issue(R_GATE, k, 0);
          issue(R_GATE_S, k, 0);
          issue(R_GATE_H, k, 0);
          issue(R_GATE_R, k, 0);
          issue(R_UP, k, 0);
          issue(R_UP_S, k, 0);
          issue(R_UP_H, k, 0);
          issue(R_UP_R, k, 0);
        }
      } else {
        issue(R_FNORM, 0, 0);
      }
    } else {
      if (k > 0) {
        issue(R_NORM2, k - 1, 0);
        issue(R_GATE, k - 1, 0);
        issue(R_GATE_S, k - 1, 0);
        issue(R_GATE_H, k - 1, 0);
        issue(R_GATE_R, k - 1, 0);
        issue(R_UP, k - 1, 0);
        issue(R_UP_S, k - 1, 0);
        issue(R_UP_H, k - 1, 0);
        issue(R_UP_R, k - 1, 0);
        issue(R_DOWN, k - 1, 0);
        issue(R_DOWN_S, k - 1, 0);
      }
      if (k < L) {
        issue(R_NORM1, k, 0);
        issue(R_QKV, k, 0);
        issue(R_QKV_S, k, 0);
      } else {
        issue(R_FNORM, 0, 0);
      }
    }
  }
  // LM head: every segment right after the last bracket, each as ring space frees (not waiting for
  // the consumers' final poll of x: +0.2% at config 3, +0.6% at config 5)
  for (int j = 0; j < P.n_lm && !dead; ++j) issue(R_LM, 0, j);
  wait_vmcnt<0>();
  publish(dead ? 0x3fffffu : n);
}

// ------------------------------------------------------------------------------------------------
// Consumer waves
// ------------------------------------------------------------------------------------------------

template <class G>
struct CSR {
  static constexpr uint32_t RB = RING;
  using W = SWS<G>;
  const Params& p;
  const PlanSR<G>& P;
  SmemSR<G>& sm;
  int cw, lane, ct;
  uint32_t pos = 0, bar_gen = 0, seen = 0, tag;
  bool dead = false;
  uint32_t* region;             // the split-role region of the uncached workspace
  __amdgpu_buffer_rsrc_t rx;    // ... as a buffer resource
  __amdgpu_buffer_rsrc_t rl;    // group-A records (the XCD's L2, or the region's fallback area)
  int xr;                       // the copy of the cross-XCD vectors this workgroup polls
  uint32_t pos_kv_end = 0;      // group A: stream position after this layer's KV chunk

  __device__ __forceinline__ CSR(const Params& p_, const PlanSR<G>& P_, SmemSR<G>& sm_, uint32_t ep,
                                 uint32_t* region_)
      : p(p_), P(P_), sm(sm_), tag(ep), region(region_) {
    cw = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6) - NPW);  // wave-uniform, in an SGPR
    lane = threadIdx.x & 63;
    ct = cw * 64 + lane;
    rx = rsrc(region_);
    rl = rx;
    xr = (P.wg >> 3) % REP;
  }
  // lane, thread and wave indices made opaque once per bracket, so that nothing derived from them is
  // hoisted out of the layer loop (and spilled there)
  __device__ __forceinline__ void refresh() { asm volatile("" : "+v"(lane), "+v"(ct), "+s"(cw)); }
  __device__ __forceinline__ uint32_t next_seg(uint32_t bytes) {
    const uint32_t s = pos;
    pos += pad_pkt(bytes);
    return s;
  }
  __device__ __forceinline__ uint32_t filled() const {
    typedef __attribute__((address_space(3))) const volatile u32x4 lds_u32x4;
    const u32x4 f = *(lds_u32x4*)(sm.front);
    return min(min(f.x, f.y), min(f.z, f.w));
  }
  __device__ __forceinline__ void wait_filled(uint32_t end) {
    if (dead || end <= seen) return;
    Spin spin(p.ws, tag, 22);
    while ((seen = filled()) < end)
      if (!spin.again()) { dead = true; return; }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
  }
  __device__ __forceinline__ void release(uint32_t end) {
    wait_lgkm0();
    if (lane == 0) st_lds(&sm.consumed[cw], end);
  }
  __device__ __forceinline__ void cbar() {
    bar_gen += NCW;
    if (lane == 0) __hip_atomic_fetch_add(&sm.cbar, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    Spin spin(p.ws, tag, 23);
    while (ld_lds(&sm.cbar) < bar_gen)
      if (!spin.again()) { dead = true; break; }
  }
  __device__ __forceinline__ float block_total(float wave_value) {
    if (lane == 0) sm.red[cw] = wave_value;
    cbar();
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < NCW; ++w) t += sm.red[w];
    return t;
  }
  __device__ __forceinline__ uint4 ring16(uint32_t at) const {
    return *reinterpret_cast<const uint4*>(sm.ring + (at & (RB - 1)));
  }
  __device__ __forceinline__ uint2 ring8(uint32_t at) const {
    return *reinterpret_cast<const uint2*>(sm.ring + (at & (RB - 1)));
  }
  __device__ __forceinline__ uint32_t ring4(uint32_t at) const {
    return *reinterpret_cast<const uint32_t*>(sm.ring + (at & (RB - 1)));
  }
  // ring16(at), or the zero line when !ok (one select on the address, no branch)
  __device__ __forceinline__ uint4 ring16z(uint32_t at, bool ok) const {
    const uint4* q = ok ? reinterpret_cast<const uint4*>(sm.ring + (at & (RB - 1)))
                        : reinterpret_cast<const uint4*>(sm.zero16);
    return *q;
  }
  // the consumers have finished bracket k: the producers may stream the next one
  __device__ __forceinline__ void bracket_done(uint32_t k) {
    if (ct == 0) st_lds(&sm.go, k);
  }
  __device__ __forceinline__ u32x4 unit6(const float (&v)[VPU]) const {
    return u32x4{pack2(v[0], v[1]), pack2(v[2], v[3]), pack2(v[4], v[5]), tag};
  }
  // one unit of cross-XCD vector (kind, l), to every copy
  __device__ __forceinline__ void put_x(int kind, int l, int u, u32x4 v) const {
    skew_delay(p.skew, P.wg, l, kind);
#pragma unroll
    for (int r = 0; r < REP; ++r) st_unit<16>(rx, W::xoff(kind, l, r, u), v);
  }
  // one unit of the group-A records (layer l, unit index)
  __device__ __forceinline__ void put_loc(int l, size_t unit, u32x4 v) const {
    skew_delay(p.skew, P.wg, l, 8);
    if (sm.loc_l2) st_unit<0>(rl, W::loc(l, unit), v);
    else st_unit<16>(rl, W::loc(l, unit), v);
  }

  // Poll n units, unit i at byte offset off(i) of resource r, spread over `nthr` threads starting
  // at thread `tid` (at most MAXU per thread); use(i, unit) for each once its tag is current, or
  // use(i, unit, k) with the thread's slot k (i = tid + k nthr) when `use` takes three arguments.
  template <int MAXU, class OFF, class USE>
  __device__ __forceinline__ void poll(__amdgpu_buffer_rsrc_t r, int n, int tid, int nthr, OFF off, USE use, int site) {
    u32x4 v[MAXU];
    uint32_t pend = 0;
#pragma unroll
    for (int k = 0; k < MAXU; ++k) {
      const int i = tid + k * nthr;
      if (i < n) { v[k] = ld_unit(r, off(i)); pend |= 1u << k; }
    }
    Spin spin(p.ws, tag, site);
    while (true) {
#pragma unroll
      for (int k = 0; k < MAXU; ++k)
        if (((pend >> k) & 1u) && v[k].w == tag) {
          if constexpr (std::is_invocable_v<USE, int, const u32x4&, int>) use(tid + k * nthr, v[k], k);
          else use(tid + k * nthr, v[k]);
          pend &= ~(1u << k);
        }
      if (!pend) break;
      if (dead || !spin.again()) { dead = true; break; }
#pragma unroll
      for (int k = 0; k < MAXU; ++k)
        if ((pend >> k) & 1u) v[k] = ld_unit(r, off(tid + k * nthr));
    }
  }
  // Poll all units of cross-XCD vector (kind, l) with n values into xs[] (and keep[] when given),
  // split over the consumer threads; returns this wave's sum of squares of the values.
  template <int MAXU>
  __device__ __forceinline__ float poll_vec(int kind, int l, int n, float* dst, float* keep, int site) {
    const int nu = (n + VPU - 1) / VPU;
    float ss = 0.f;
    poll<MAXU>(rx, nu, ct, NCT, [&](int u) { return W::xoff(kind, l, xr, u); },
               [&](int u, const u32x4& v) {
                 const float f[VPU] = {bf_lo(v.x), bf_hi(v.x), bf_lo(v.y), bf_hi(v.y), bf_lo(v.z), bf_hi(v.z)};
#pragma unroll
                 for (int e = 0; e < VPU; ++e) {
                   const int i = u * VPU + e;
                   if (i < n) {
                     dst[i] = f[e];
                     if (keep) keep[i] = f[e];
                     ss += f[e] * f[e];
                   }
                 }
               },
               site);
    return wave_sum(ss);
  }
};

// Rows r0 .. r0 + N - 1 of a ring segment of K-long bf16 rows, dotted with a lane's activation
// chunks (chunk lane + 64 c of each row); the N sums are returned wave-uniform.  Lanes past a row's
// last chunk read the zero line (their activation chunk is zero too, but ring bytes past a row may
// hold anything).  Rows past the segment read other ring bytes, whose sums the caller discards.
template <int K, int N, class CT>
__device__ __forceinline__ void ring_rows(const CT& C, uint32_t seg, int r0, uint4 (&w)[N][Chunks<K>::CPL]) {
  constexpr int CPL = Chunks<K>::CPL, CH = Chunks<K>::CH;
  const bool tail_ok = CH % 64 == 0 || C.lane + 64 * (CPL - 1) < CH;
#pragma unroll
  for (int r = 0; r < N; ++r)
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const uint32_t at = seg + uint32_t(r0 + r) * uint32_t(K * 2) + uint32_t(C.lane + 64 * c) * 16u;
      w[r][c] = c == CPL - 1 ? C.ring16z(at, tail_ok) : C.ring16(at);
    }
}

// 8 e4m3 weights with their e8m0 scale code as the bf16 words of the dense path: bf16(e4m3 *
// 2^(s-127)) per weight (v_cvt_scalef32_pk_bf16_fp8, two weights per conversion).
__device__ __forceinline__ uint4 deq8(uint2 q, uint32_t s) {
  const float f = e8m0_f32(s);
  return make_uint4(__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(int(q.x), f, false)),
                    __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(int(q.x), f, true)),
                    __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(int(q.y), f, false)),
                    __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(int(q.y), f, true)));
}

// ring_rows for the model's weight format: MXFP8 rows (K e4m3 bytes per row in `seg`, scale_stride(K)
// scale bytes per row in `segs`) become the bf16 words ring_rows would return for the dequantised
// matrix; lanes past a row's last chunk get zeros (weights 0 with scale 2^0).
template <class G, int K, int N, class CT>
__device__ __forceinline__ void wrows(const CT& C, uint32_t seg, uint32_t segs, int r0, uint4 (&w)[N][Chunks<K>::CPL]) {
  if constexpr (G::WF == 0) {
    ring_rows<K, N>(C, seg, r0, w);
  } else {
    constexpr int CPL = Chunks<K>::CPL, CH = Chunks<K>::CH;
    constexpr uint32_t SK = scale_stride(K);
    const bool tail_ok = CH % 64 == 0 || C.lane + 64 * (CPL - 1) < CH;
    uint2 q[N][CPL];
    uint32_t sc[N][CPL];
#pragma unroll
    for (int r = 0; r < N; ++r)
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const uint32_t row = uint32_t(r0 + r), ch = uint32_t(C.lane + 64 * c);
        const bool ok = c < CPL - 1 || tail_ok;
        q[r][c] = ok ? C.ring8(seg + row * uint32_t(K) + ch * 8u) : make_uint2(0u, 0u);
        sc[r][c] = ok ? uint32_t(C.sm.ring[(segs + row * SK + (ch >> 2)) & (RING - 1)]) : 127u;
      }
#pragma unroll
    for (int r = 0; r < N; ++r)
#pragma unroll
      for (int c = 0; c < CPL; ++c) w[r][c] = deq8(q[r][c], sc[r][c]);
  }
}

// The same chunks rebuilt from a lossless segment set: plane rows (K bytes each) at segp, header rows
// (K/8 words) at segh, the escaped chunks of the segment's rows (ordinals first, first + 1, ...) at
// segr.  Every chunk is rebuilt (an escaped one's result is then replaced by its raw chunk), so the
// words are the dense ones bit for bit; lanes past a row's last chunk get zeros, as from the zero line.
template <int K, int N, class CT>
__device__ __forceinline__ void lossless_rows(const CT& C, uint32_t segp, uint32_t segh, uint32_t segr, uint32_t first,
                                              int r0, uint4 (&w)[N][Chunks<K>::CPL]) {
  constexpr int CPL = Chunks<K>::CPL, CH = Chunks<K>::CH;
  const bool tail_ok = CH % 64 == 0 || C.lane + 64 * (CPL - 1) < CH;
  uint2 pl[N][CPL];
  uint32_t hd[N][CPL];
#pragma unroll
  for (int r = 0; r < N; ++r)
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const uint32_t row = uint32_t(r0 + r), ch = uint32_t(C.lane + 64 * c);
      hd[r][c] = C.ring4(segh + (row * uint32_t(CH) + ch) * 4u);
      pl[r][c] = C.ring8(segp + row * uint32_t(K) + ch * 8u);
    }
#pragma unroll
  for (int r = 0; r < N; ++r)
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      w[r][c] = lossless_chunk(pl[r][c], hd[r][c]);
      asm volatile("" : "+v"(w[r][c].x), "+v"(w[r][c].y), "+v"(w[r][c].z), "+v"(w[r][c].w));
    }
#pragma unroll
  for (int r = 0; r < N; ++r)
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const uint32_t h = hd[r][c];
      const bool esc = (h >> 24) == 255u;
      const uint4 e = C.ring16(segr + (esc ? (h & 0xFFFFFFu) - first : 0u) * 16u);
      const bool ok = c < CPL - 1 || tail_ok;
      w[r][c].x = !ok ? 0u : esc ? e.x : w[r][c].x;
      w[r][c].y = !ok ? 0u : esc ? e.y : w[r][c].y;
      w[r][c].z = !ok ? 0u : esc ? e.z : w[r][c].z;
      w[r][c].w = !ok ? 0u : esc ? e.w : w[r][c].w;
    }
}

// out[r] = w[r] . x over a lane's chunks, totals over the wave, returned wave-uniform.
template <int K, int N>
__device__ __forceinline__ void dots_w(const uint4 (&w)[N][Chunks<K>::CPL], const XChunks<K, 8>& x, float (&out)[N]) {
  constexpr int CPL = Chunks<K>::CPL;
#pragma unroll
  for (int r = 0; r < N; ++r) {
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
  wave_rows<N>(out);
}

template <int K, int N, class CT>
__device__ __forceinline__ void dots_n(const CT& C, uint32_t seg, int r0, const XChunks<K, 8>& x, float (&out)[N]) {
  uint4 w[N][Chunks<K>::CPL];
  ring_rows<K, N>(C, seg, r0, w);
  dots_w<K, N>(w, x, out);
}

// Partial dots over one wave's quarter of K (chunks [w CH/4, (w+1) CH/4) of each row, chunk
// w CH/4 + lane + 64 c for this lane; `x` holds the lane's activation chunks of that quarter).
template <int K>
struct Quarter {
  static constexpr int CH = K / 8, CHW = CH / NCW, CPL = (CHW + 63) / 64;
  static_assert(CH % NCW == 0, "K splits evenly over the waves");
};
template <int K, int N, class CT>
__device__ __forceinline__ void quarter_rows(const CT& C, uint32_t seg, int r0, uint4 (&w)[N][Quarter<K>::CPL]) {
  using Q = Quarter<K>;
  const bool tail_ok = Q::CHW % 64 == 0 || C.lane + 64 * (Q::CPL - 1) < Q::CHW;
#pragma unroll
  for (int r = 0; r < N; ++r)
#pragma unroll
    for (int c = 0; c < Q::CPL; ++c) {
      const uint32_t at = seg + uint32_t(r0 + r) * uint32_t(K * 2) + uint32_t(C.cw * Q::CHW + C.lane + 64 * c) * 16u;
      w[r][c] = c == Q::CPL - 1 ? C.ring16z(at, tail_ok) : C.ring16(at);
    }
}
// quarter_rows for the model's weight format (MXFP8 as in wrows).
template <class G, int K, int N, class CT>
__device__ __forceinline__ void wquarter(const CT& C, uint32_t seg, uint32_t segs, int r0, uint4 (&w)[N][Quarter<K>::CPL]) {
  using Q = Quarter<K>;
  if constexpr (G::WF == 0) {
    quarter_rows<K, N>(C, seg, r0, w);
  } else {
    constexpr uint32_t SK = scale_stride(K);
    const bool tail_ok = Q::CHW % 64 == 0 || C.lane + 64 * (Q::CPL - 1) < Q::CHW;
    uint2 q[N][Q::CPL];
    uint32_t sc[N][Q::CPL];
#pragma unroll
    for (int r = 0; r < N; ++r)
#pragma unroll
      for (int c = 0; c < Q::CPL; ++c) {
        const uint32_t row = uint32_t(r0 + r), ch = uint32_t(C.cw * Q::CHW + C.lane + 64 * c);
        const bool ok = c < Q::CPL - 1 || tail_ok;
        q[r][c] = ok ? C.ring8(seg + row * uint32_t(K) + ch * 8u) : make_uint2(0u, 0u);
        sc[r][c] = ok ? uint32_t(C.sm.ring[(segs + row * SK + (ch >> 2)) & (RING - 1)]) : 127u;
      }
#pragma unroll
    for (int r = 0; r < N; ++r)
#pragma unroll
      for (int c = 0; c < Q::CPL; ++c) w[r][c] = deq8(q[r][c], sc[r][c]);
  }
}
template <int K, int N>
__device__ __forceinline__ void dots_quarter_w(const uint4 (&w)[N][Quarter<K>::CPL], const uint4 (&x)[Quarter<K>::CPL],
                                               float (&out)[N]) {
  using Q = Quarter<K>;
#pragma unroll
  for (int r = 0; r < N; ++r) {
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < Q::CPL; ++c) {
      acc = dot2(w[r][c].x, x[c].x, acc);
      acc = dot2(w[r][c].y, x[c].y, acc);
      acc = dot2(w[r][c].z, x[c].z, acc);
      acc = dot2(w[r][c].w, x[c].w, acc);
    }
    out[r] = acc;
  }
  wave_rows<N>(out);
}

// Norm weights of a lane's chunks from the ring segment that carries them.
template <int K, class CT>
__device__ __forceinline__ void normw(const CT& C, XChunks<K, 8>& nw, uint32_t seg) {
#pragma unroll
  for (int c = 0; c < Chunks<K>::CPL; ++c) {
    const int ch = C.lane + 64 * c;
    nw[c][0] = ch < Chunks<K>::CH ? C.ring16(seg + uint32_t(ch * 16)) : make_uint4(0, 0, 0, 0);
  }
}

// ------------------------------------------------------------------------------------------------
// Group A: attention for one chunk (KV head g, chunk c), then the merge, O and h1
// ------------------------------------------------------------------------------------------------

// 16-token tiles of a chunk, tile t to wave t % NCW: at most MT per wave
struct ChunkRegs {
  uint32_t va[MT][4][2];    // V of the wave's tiles: A operands of the P.V tiles (bf16 pairs)
};
// Waves that take the chunk's 16-token tiles (tile t to wave t % NW, its (t / NW)-th): all NCW,
// except in the leader chunk when the first NCW - 1 can hold every tile; its last wave then has
// only the new token, whose k and v come from other producers than q and tend to arrive later.
template <class G>
__device__ __forceinline__ int tile_waves(const PlanSR<G>& P, int NT) {
  return P.leader && NT <= (NCW - 1) * MT ? NCW - 1 : NCW;
}

// The wave's V from the ring into registers, long before q arrives (the chunk was streamed in during
// the previous layer; V needs one 2-byte read per element, K is loaded with 16-byte reads just
// before q).  P.V uses v_mfma_f32_16x16x16_bf16 with V as the A operand, once per 16 dims: lane l
// supplies V[tile*16 + 4(l/16) + e][16 mf + l%16], e < 4.  Cached tokens only (the new token is
// handled apart): later elements are zero.  Reads past the chunk stay inside the ring.
template <class G>
__device__ __forceinline__ void chunk_load(CSR<G>& C, uint32_t seg, ChunkRegs& R) {
  const PlanSR<G>& P = C.P;
  SmemSR<G>& sm = C.sm;
  const int w = C.cw, lane = C.lane;
  const int T_old = P.t1 - P.t0;
  const int NT = (T_old + 15) >> 4;
  const int NW = tile_waves<G>(P, NT);
  const int nt = w < NW && NT > w ? (NT - w + NW - 1) / NW : 0;
  const int hq = lane & 15, pq = lane >> 4;
  // V element (mf, e) of this lane sits at byte tile*4096 + vo[mf][e] of the segment: token
  // 4 pq + e of the tile, piece (dim / 8 + token) % 8 of the token's V half, dim 16 mf + hq
  uint32_t vo[4][4];
#pragma unroll
  for (int mf = 0; mf < 4; ++mf)
#pragma unroll
    for (int e = 0; e < 4; ++e)
      vo[mf][e] = uint32_t(4 * pq + e) * 256u + 128u + uint32_t((2 * mf + (hq >> 3) + 4 * pq + e) & 7) * 16u +
                  uint32_t(hq & 7) * 2u;
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    if (i >= nt) {  // defined all the same: registers left undefined stay live across the layer loop
#pragma unroll
      for (int mf = 0; mf < 4; ++mf) R.va[i][mf][0] = R.va[i][mf][1] = 0u;
      continue;
    }
    const int tile = w + NW * i;
    const uint32_t base = seg + uint32_t(tile) * 4096u;
    uint32_t h[4][4];
#pragma unroll
    for (int mf = 0; mf < 4; ++mf)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        h[mf][e] = *reinterpret_cast<const uint16_t*>(sm.ring + ((base + vo[mf][e]) & (RING - 1)));
#pragma unroll
    for (int mf = 0; mf < 4; ++mf) {
      const int j = tile * 16 + 4 * pq;
      const uint32_t v0 = j < T_old ? h[mf][0] : 0u, v1 = j + 1 < T_old ? h[mf][1] : 0u;
      const uint32_t v2 = j + 2 < T_old ? h[mf][2] : 0u, v3 = j + 3 < T_old ? h[mf][3] : 0u;
      R.va[i][mf][0] = v0 | (v1 << 16);
      R.va[i][mf][1] = v2 | (v3 << 16);
    }
  }
}

template <class G>
__device__ __forceinline__ void attention_sr(CSR<G>& C, int l, uint32_t seg, ChunkRegs& R) {
  using S = SG<G>;
  using W = SWS<G>;
  const Params& p = C.p;
  const PlanSR<G>& P = C.P;
  SmemSR<G>& sm = C.sm;
  const int g = P.g, lane = C.lane, w = C.cw;
  const int T_old = P.t1 - P.t0;
  // 16-token tiles of the chunk's cached tokens, tile t to wave t % NW (tile_waves); the new token
  // (the leader's) is taken apart by the last wave, which has the fewest tiles or none
  const int NT = (T_old + 15) >> 4;
  const int NW = tile_waves<G>(P, NT);
  const int nt = w < NW && NT > w ? (NT - w + NW - 1) / NW : 0;
  const bool has_new = P.leader && w == NCW - 1;
  const int hq = lane & 15, pq = lane >> 4;
  float* in = sm.at.qkvw[w];
  uint32_t (&va)[MT][4][2] = R.va;
  // K of the wave's tiles, the A operands of the score tiles (v_mfma_f32_16x16x32_bf16): lane l
  // supplies row l%16 (token tile*16 + l%16), dims 8(l/16) .. +7 and 32 + 8(l/16) .. +7
  uint4 ka[MT][2];
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    ka[i][0] = ka[i][1] = make_uint4(0u, 0u, 0u, 0u);
    if (i >= nt) continue;
    const int tok = (w + NW * i) * 16 + hq;
    const uint32_t row = seg + uint32_t(tok) * 256u;
    ka[i][0] = C.ring16(row + uint32_t((pq + tok) & 7) * 16u);
    ka[i][1] = C.ring16(row + uint32_t((pq + 4 + tok) & 7) * 16u);
  }
  // q of the 3 heads of KV head g (units 32g .. 32g + 31), and for the wave with the new token the
  // units holding its k and v rows
  {
    const int kb = G::H + 64 * g, vb = G::H + G::KVH * 64 + 64 * g;
    const int ku0 = kb / VPU, kn = (kb + 63) / VPU - ku0 + 1;
    const int vu0 = vb / VPU, vn = (vb + 63) / VPU - vu0 + 1;
    const int nq = 32, nu = has_new ? nq + kn + vn : nq;
    C.template poll<1>(C.rx, nu, lane, 64,
                       [&](int i) {
                         const int u = i < nq ? 32 * g + i : (i < nq + kn ? ku0 + i - nq : vu0 + i - nq - kn);
                         return W::xoff(K_XQ, l, C.xr, u);
                       },
                       [&](int i, const u32x4& v) {
                         const float f[VPU] = {bf_lo(v.x), bf_hi(v.x), bf_lo(v.y), bf_hi(v.y), bf_lo(v.z), bf_hi(v.z)};
                         // q and k slots come in RoPE-pair order (qkv_row): local slot r of a
                         // head is dim r / 2 + 32 (r % 2); v slots are in row order
                         if (i < nq) {
#pragma unroll
                           for (int e = 0; e < VPU; ++e) {
                             const int ls = i * VPU + e;
                             in[(ls & ~63) + ((ls & 63) >> 1) + 32 * (ls & 1)] = f[e];
                           }
                         } else {
                           const int kv = i < nq + kn ? 0 : 1;
                           const int u = kv ? vu0 + i - nq - kn : ku0 + i - nq;
                           const int base = kv ? vb : kb;
#pragma unroll
                           for (int e = 0; e < VPU; ++e) {
                             const int row = u * VPU + e - base;
                             const int dim = kv ? row : (row >> 1) + 32 * (row & 1);
                             if (row >= 0 && row < 64) in[192 + 64 * kv + dim] = f[e];
                           }
                         }
                       },
                       30);
  }
  if (w == 0 && lane == 0) trace_at(p, l, 34, p.n_layers);
  if (has_new && lane == 0) trace_at(p, l, 38, p.n_layers);
  wait_lgkm0();
  if (w == 0 && lane == 0) trace_at(p, l, 3, p.n_layers);
  if (has_new && lane == 0) trace_at(p, l, 4, p.n_layers);
  // q of head hq < 3 and the new token's k (both roped by their producers) as bf16 pieces pq (dims
  // 8pq .. 8pq+7) and pq + 4 (dims 32 + 8pq ..), the operands below
  auto pieces = [&](const float* head, uint32_t (&lo)[4], uint32_t (&hi)[4]) {
    const float4 a0 = *reinterpret_cast<const float4*>(head + pq * 8);
    const float4 a1 = *reinterpret_cast<const float4*>(head + pq * 8 + 4);
    const float4 b0 = *reinterpret_cast<const float4*>(head + 32 + pq * 8);
    const float4 b1 = *reinterpret_cast<const float4*>(head + 32 + pq * 8 + 4);
    lo[0] = pack2(a0.x, a0.y); lo[1] = pack2(a0.z, a0.w); lo[2] = pack2(a1.x, a1.y); lo[3] = pack2(a1.z, a1.w);
    hi[0] = pack2(b0.x, b0.y); hi[1] = pack2(b0.z, b0.w); hi[2] = pack2(b1.x, b1.y); hi[3] = pack2(b1.z, b1.w);
  };
  uint32_t qlo[4] = {0u, 0u, 0u, 0u}, qhi[4] = {0u, 0u, 0u, 0u};
  if (hq < 3) pieces(in + hq * 64, qlo, qhi);
  uint32_t klo[4] = {0u, 0u, 0u, 0u}, khi[4] = {0u, 0u, 0u, 0u};
  // the new token's scores q_h . k_new: lane (h, pq) dots pieces pq and pq + 4, the four rows add up
  float s_new[3] = {-INFINITY, -INFINITY, -INFINITY};
  if (has_new) {
    pieces(in + 192, klo, khi);
    float d = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      d = dot2(qlo[i], klo[i], d);
      d = dot2(qhi[i], khi[i], d);
    }
    d = column_total<false>(d);
#pragma unroll
    for (int h = 0; h < 3; ++h)
      s_new[h] = rnd(__builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, d), h))) * 0.125f;
  }
  if (w == 0 && lane == 0) trace_at(p, l, 35, p.n_layers);
  if (has_new && lane == 0) trace_at(p, l, 5, p.n_layers);
  // Scores on the matrix cores, D[token][head] = K[token][:] . q[head][:] per tile (two k-steps over
  // the 64 dims); lane l supplies column l%16 of B (q of head l%16 < 3, zero padding columns) and
  // receives D[4(l/16) + jj][l%16], the score of head l%16 for token tile*16 + 4(l/16) + jj.  Rows
  // of tokens past the chunk hold other ring bytes' products and are masked below.
  floatx4 sacc[MT];
  {
    const bf16x8 bq0 = __builtin_bit_cast(bf16x8, make_uint4(qlo[0], qlo[1], qlo[2], qlo[3]));
    const bf16x8 bq1 = __builtin_bit_cast(bf16x8, make_uint4(qhi[0], qhi[1], qhi[2], qhi[3]));
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      floatx4 acc = {0.f, 0.f, 0.f, 0.f};
      if (i < nt) {
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ka[i][0]), bq0, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ka[i][1]), bq1, acc, 0, 0, 0);
      }
      sacc[i] = acc;
    }
  }
  if (w == 0 && lane == 0) trace_at(p, l, 36, p.n_layers);
  if (has_new && lane == 0) trace_at(p, l, 9, p.n_layers);
  // The softmax exponentials inside attention use the hardware exp2 (__expf): within a few fp32 ulp
  // of expf, far below the bf16 rounding of p.
  // The wave's softmax statistics.  Only columns 0-2 of a score tile hold heads, so tile i's columns
  // move to lanes 3i .. 3i+2 of each 16-lane row (DPP row_shr:3i): lane c of a row then holds the
  // scores of head c % 3 in tile c / 3 (c < 3 MT), four tokens, and the exps below run on 4 values
  // per lane instead of 4 MT.  Scores bf16(q.k) / 8 as HF; ev keeps exp(s - m_wave).  Once the
  // head's global max M and sum L are known the probabilities are bf16(ev * exp(m_wave - M) / L),
  // HF's bf16(exp(s - M) / L) up to fp32 rounding.
  static_assert(3 * MT <= 16, "three columns per tile fit a 16-lane row");
  const int ct = hq / 3, ch = hq - 3 * ct;
  float ev[4] = {0.f, 0.f, 0.f, 0.f}, m = -INFINITY;
  float mw[3], lw[3], ev_new[3];
  if (nt > 0) {
    {
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        float v = sacc[0][jj];
#pragma unroll
        for (int i = 1; i < MT; ++i) {
          const float t = dpp_shr3<true>(i, sacc[i][jj]);
          v = ct == i ? t : v;
        }
        const int t = (w + NW * ct) * 16 + 4 * pq + jj;
        const bool ok = ct < nt && t < T_old;
        ev[jj] = ok ? rnd(v) * 0.125f : -INFINITY;
      }
    }
    m = fmaxf(fmaxf(ev[0], ev[1]), fmaxf(ev[2], ev[3]));
    head_totals<true>(m, mw);
#pragma unroll
    for (int h = 0; h < 3; ++h) mw[h] = fmaxf(mw[h], s_new[h]);
    m = ch == 0 ? mw[0] : ch == 1 ? mw[1] : mw[2];
    float lsum = 0.f;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      ev[jj] = ev[jj] == -INFINITY ? 0.f : __expf(ev[jj] - m);
      lsum += ev[jj];
    }
    head_totals<false>(lsum, lw);
#pragma unroll
    for (int h = 0; h < 3; ++h) {
      ev_new[h] = s_new[h] == -INFINITY ? 0.f : __expf(s_new[h] - mw[h]);
      lw[h] += ev_new[h];
    }
  } else {
    // no cached tile (the leader's new-token wave when the other waves hold every tile): the new
    // token's scores alone, max s_new and sum exp(0) = 1, the values the general path gives
#pragma unroll
    for (int h = 0; h < 3; ++h) {
      mw[h] = s_new[h];
      ev_new[h] = s_new[h] == -INFINITY ? 0.f : 1.f;
      lw[h] = ev_new[h];
    }
    m = ch == 0 ? mw[0] : ch == 1 ? mw[1] : mw[2];
  }
  if (w == 0 && lane == 0) trace_at(p, l, 37, p.n_layers);
  if (has_new && lane == 0) trace_at(p, l, 39, p.n_layers);
  float Mh[3], Lh[3];
  if constexpr (S::STATS_CHUNK) {
    // the chunk's waves combined first, m_c = max_v m_v and l_c = (e_0 + e_1) + (e_2 + e_3) with
    // e_v = l_v exp(m_v - m_c) (lanes 4h + v), then one record per chunk: chunk c' of head g
    // (group-A rank g + KVH c') has {max x3, tag}, {sum x3, tag} at units 2 rank + {0, 1}
    if (lane == 0)
#pragma unroll
      for (int h = 0; h < 3; ++h) {
        sm.wml[w][0][h] = mw[h];
        sm.wml[w][1][h] = lw[h];
      }
    C.cbar();
    float mq = -INFINITY, lq = 0.f;
    if (lane < 4 * 3) {
      mq = sm.wml[lane & 3][0][lane >> 2];
      lq = sm.wml[lane & 3][1][lane >> 2];
    }
    float mx = fmaxf(mq, dpp<0xb1>(mq, mq));
    mx = fmaxf(mx, dpp<0x4e>(mx, mx));
    float ex = mq == -INFINITY ? 0.f : lq * __expf(mq - mx);
    ex += dpp<0xb1>(0.f, ex);
    ex += dpp<0x4e>(0.f, ex);
    if (w == 0) {
      float v[3];
#pragma unroll
      for (int h = 0; h < 3; ++h) {
        const float mc = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mx), 4 * h));
        const float lc = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ex), 4 * h));
        v[h] = lane ? lc : mc;
      }
      if (lane < 2)
        C.put_loc(l, W::STAT_U + size_t(P.rank) * 2 + lane,
                  u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), C.tag});
    }
    if (w == 0 && lane == 0) trace_at(p, l, 17, p.n_layers);
    // lane 2c polls the maxima of chunk c, lane 2c + 1 its sums; a_c = l_c exp(m_c - M) in lane 2c + 1;
    // per row k (chunks 8k .. 8k + 7) T_k = ((a7 + a6) + (a5 + a4)) + ((a3 + a2) + (a1 + a0)), L =
    // (T_3 + T_2) + (T_1 + T_0): the association of the per-wave merge, so the same bits
    static_assert(2 * S::C == 64, "one statistics unit per lane, four rows of eight chunks");
    float st[3] = {(lane & 1) ? 0.f : -INFINITY, (lane & 1) ? 0.f : -INFINITY, (lane & 1) ? 0.f : -INFINITY};
    C.template poll<1>(C.rl, 2 * S::C, lane, 64,
                       [&](int i) { return W::loc(l, W::STAT_U + size_t(g + G::KVH * (i >> 1)) * 2 + (i & 1)); },
                       [&](int, const u32x4& v) {
                         st[0] = __uint_as_float(v.x);
                         st[1] = __uint_as_float(v.y);
                         st[2] = __uint_as_float(v.z);
                       },
                       31);
    float m[3], M[3];
#pragma unroll
    for (int h = 0; h < 3; ++h) {
      const float mo = dpp<0xb1>(0.f, st[h]);
      m[h] = (lane & 1) ? mo : st[h];
      M[h] = m[h];
    }
    wave_max_n<3>(M);
#pragma unroll
    for (int h = 0; h < 3; ++h) {
      float a = ((lane & 1) && m[h] != -INFINITY) ? st[h] * __expf(m[h] - M[h]) : 0.f;
      a += dpp<0x4e>(0.f, a);  // quad_perm [2,3,0,1]: lane 4q + 3 = a_{2q+1} + a_{2q}
      a += dpp<0x114>(0.f, a); // row_shr:4: lane 8p + 7 = (a_{4p+3} + a_{4p+2}) + (a_{4p+1} + a_{4p})
      a += dpp<0x118>(0.f, a); // row_shr:8: lane 16k + 15 = T_k
      a += dpp<0x142, 0xa>(0.f, a);  // row_bcast:15 into rows 1, 3: lane 31 = T_1 + T_0, lane 63 = T_3 + T_2
      a += dpp<0x143, 0xc>(0.f, a);  // row_bcast:31 into rows 2, 3: lane 63 = (T_3 + T_2) + (T_1 + T_0)
      Mh[h] = M[h];
      Lh[h] = lane63(a);
    }
  } else {
  // exchange (max, sum) with every wave of the head's chunks, each wave publishing its own without
  // waiting for the other waves of its chunk: wave v of chunk c' (group-A rank g + KVH c') has the
  // record {max x3, tag}, {sum x3, tag} at units (rank NCW + v) 2 + {0, 1}
  if (lane < 2)
    C.put_loc(l, W::STAT_U + (size_t(P.rank) * NCW + w) * 2 + lane,
              lane ? u32x4{__float_as_uint(lw[0]), __float_as_uint(lw[1]), __float_as_uint(lw[2]), C.tag}
                   : u32x4{__float_as_uint(mw[0]), __float_as_uint(mw[1]), __float_as_uint(mw[2]), C.tag});
  if (w == 0 && lane == 0) trace_at(p, l, 17, p.n_layers);
  {
    // unit i = 2k + s (k = NCW c' + v) is polled by lane i % 64: an even lane the maxima of one
    // (chunk, wave), the odd lane next to it the sums of the same one
    constexpr int NU = 2 * NCW * S::C, MU = (NU + 63) / 64;
    static_assert(MU <= 4, "four statistics units per lane at most");
    float st[MU][3];
#pragma unroll
    for (int k = 0; k < MU; ++k)
#pragma unroll
      for (int h = 0; h < 3; ++h) st[k][h] = (lane & 1) ? 0.f : -INFINITY;
    C.template poll<MU>(C.rl, NU, lane, 64,
                        [&](int i) {
                          const int pr = i >> 1, c = pr / NCW, v = pr - c * NCW;
                          return W::loc(l, W::STAT_U + (size_t(g + G::KVH * c) * NCW + v) * 2 + (i & 1));
                        },
                        [&](int, const u32x4& v, int k) {
                          st[k][0] = __uint_as_float(v.x);
                          st[k][1] = __uint_as_float(v.y);
                          st[k][2] = __uint_as_float(v.z);
                        },
                        31);
    // Merge with the association of a two-level merge (the waves of each chunk, then the chunks), so
    // the sums round as they did when each chunk combined its waves before the exchange, all in DPP
    // moves.  Lanes 8j .. 8j + 7 of slot k hold the four waves of chunk c = 8k + j (an even lane the
    // maxima, the odd one the sums); chunk c: m_c = max_v m_cv, l_c = (e_c0 + e_c1) + (e_c2 + e_c3)
    // with e_cv = l_cv exp(m_cv - m_c), in lane 8j + 1; then a_c = l_c exp(m_c - M) and per slot
    // T_k = ((a7 + a6) + (a5 + a4)) + ((a3 + a2) + (a1 + a0)) over its eight chunks, L the T_k added
    // pairwise.  With up to 8 chunks this is the sum a 64-lane scan gives with a_c in lane 2c + 1, and
    // up to 16 chunks the same with the chunks past 8 added last.
    float mc[MU][3], lc[MU][3], M[3] = {-INFINITY, -INFINITY, -INFINITY};
#pragma unroll
    for (int k = 0; k < MU; ++k)
#pragma unroll
      for (int h = 0; h < 3; ++h) {
        const float mo = dpp<0xb1>(0.f, st[k][h]);                 // quad_perm [1,0,3,2]: the pair's other lane
        const float m = (lane & 1) ? mo : st[k][h];
        float x = fmaxf(m, dpp<0x4e>(m, m));                      // quad_perm [2,3,0,1]: waves v, v ^ 1
        x = fmaxf(x, dpp<0x141>(x, x));                            // row_half_mirror: the other quad
        mc[k][h] = x;
        M[h] = fmaxf(M[h], x);
        float e = ((lane & 1) && lane + 64 * k < NU && m != -INFINITY) ? st[k][h] * __expf(m - x) : 0.f;
        e += dpp<0x4e>(0.f, e);                                    // odd lanes: e_c0 + e_c1, e_c2 + e_c3
        e += dpp<0xb1>(0.f, e);                                    // ... copied into the even lanes
        e += dpp<0x141>(0.f, e);                                   // lane 8j + 1: (e_c0 + e_c1) + (e_c2 + e_c3)
        lc[k][h] = e;
      }
    wave_max_n<3>(M);
    float T[MU][3];
#pragma unroll
    for (int k = 0; k < MU; ++k)
#pragma unroll
      for (int h = 0; h < 3; ++h) {
        float a = ((lane & 7) == 1 && mc[k][h] != -INFINITY) ? lc[k][h] * __expf(mc[k][h] - M[h]) : 0.f;
        a += dpp<0x118>(0.f, a);                                   // row_shr:8: lane 16r + 9 = a_{2r+1} + a_{2r}
        a = dpp<0x116>(0.f, a);                                    // row_shr:6: ... into lane 16r + 15
        a += dpp<0x142, 0xa>(0.f, a);                              // row_bcast:15 into rows 1, 3
        a += dpp<0x143, 0xc>(0.f, a);                              // row_bcast:31 into rows 2, 3
        T[k][h] = lane63(a);
      }
    float sum[3];
#pragma unroll
    for (int h = 0; h < 3; ++h) {
      if constexpr (MU == 1) sum[h] = T[0][h];
      else if constexpr (MU == 2) sum[h] = T[1][h] + T[0][h];
      else if constexpr (MU == 3) sum[h] = T[2][h] + (T[1][h] + T[0][h]);
      else sum[h] = (T[3][h] + T[2][h]) + (T[1][h] + T[0][h]);
    }
#pragma unroll
    for (int h = 0; h < 3; ++h) { Mh[h] = M[h]; Lh[h] = sum[h]; }
  }
  }
  if (w == 0 && lane == 0) trace_at(p, l, 18, p.n_layers);
  // P.V on the matrix cores with the probabilities rounded to bf16 as HF does.  The scores'
  // accumulator layout is the B layout of v_mfma_f32_16x16x16_bf16 (lane l: head l%16, tokens
  // tile*16 + 4(l/16) + e), so tile i's B operand is the compacted probabilities moved back from
  // lanes 3i .. 3i+2 (DPP row_shl:3i); columns 3-15 of B and D are unused.  D[4(l/16) + j][l%16]
  // accumulates dim 16 mf + 4(l/16) + j of head l%16 over the wave's tiles.
  typedef short bf16x4_t __attribute__((ext_vector_type(4)));
  floatx4 oacc[4];
#pragma unroll
  for (int mf = 0; mf < 4; ++mf) oacc[mf] = floatx4{0.f, 0.f, 0.f, 0.f};
  {
    const float Mq = ch == 0 ? Mh[0] : ch == 1 ? Mh[1] : Mh[2];
    const float Lq = ch == 0 ? Lh[0] : ch == 1 ? Lh[1] : Lh[2];
    const float scale = m != -INFINITY ? __expf(m - Mq) * (1.0f / Lq) : 0.f;
    const uint32_t p01 = pack2(ev[0] * scale, ev[1] * scale), p23 = pack2(ev[2] * scale, ev[3] * scale);
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      if (i >= nt) continue;
      const uint2 pb = make_uint2(dpp_shl3u(i, p01), dpp_shl3u(i, p23));
#pragma unroll
      for (int mf = 0; mf < 4; ++mf)
        oacc[mf] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
            __builtin_bit_cast(bf16x4_t, make_uint2(va[i][mf][0], va[i][mf][1])), __builtin_bit_cast(bf16x4_t, pb),
            oacc[mf], 0, 0, 0);
    }
    if (has_new && hq < 3) {
      // the new token: p = bf16(exp(s_new - m_wave) exp(m_wave - M) / L) of head hq times its v
      const float mh = hq == 0 ? mw[0] : hq == 1 ? mw[1] : mw[2];
      const float en = hq == 0 ? ev_new[0] : hq == 1 ? ev_new[1] : ev_new[2];
      const float Mn = hq == 0 ? Mh[0] : hq == 1 ? Mh[1] : Mh[2];
      const float Ln = hq == 0 ? Lh[0] : hq == 1 ? Lh[1] : Lh[2];
      const float pn = rnd(en * (__expf(mh - Mn) * (1.0f / Ln)));
#pragma unroll
      for (int mf = 0; mf < 4; ++mf) {
        const float4 v = *reinterpret_cast<const float4*>(in + 256 + 16 * mf + 4 * pq);
        oacc[mf][0] = fmaf(pn, v.x, oacc[mf][0]);
        oacc[mf][1] = fmaf(pn, v.y, oacc[mf][1]);
        oacc[mf][2] = fmaf(pn, v.z, oacc[mf][2]);
        oacc[mf][3] = fmaf(pn, v.w, oacc[mf][3]);
      }
    }
  }
  C.release(C.pos_kv_end);
  // KV append at slot_mapping[0] (block360_kernel.inc:124-135; slot < 0 skips): lane 16 q (k) and
  // lane 16 q + 1 (v) store pieces q and q + 4 of the new token, 16 bytes each.  The wide layout
  // stores here, the narrow one after the barrier below (the same code), since the barrier waits
  // for the stores to complete: the narrow layout's last wave publishes no partials and its
  // workgroups wait for the other chunks next, while the wide layout's next barrier gates its own
  // slice of them.
  if (S::WIDE && has_new && P.slot >= 0 && hq < 2) {
    uint16_t* cache = reinterpret_cast<uint16_t*>(const_cast<void*>(sm.kvp[l]));
    const long long e = (P.slot / 16) * p.block_stride + (P.slot % 16) * p.token_stride +
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
  if (hq < 3)
#pragma unroll
    for (int mf = 0; mf < 4; ++mf)
      *reinterpret_cast<float4*>(&sm.wo[w][hq][16 * mf + 4 * pq]) = make_float4(oacc[mf][0], oacc[mf][1], oacc[mf][2], oacc[mf][3]);
  C.cbar();
  if (w == 0 && lane == 0) trace_at(p, l, 19, p.n_layers);
  if (!S::WIDE && has_new && P.slot >= 0 && hq < 2) {
    uint16_t* cache = reinterpret_cast<uint16_t*>(const_cast<void*>(sm.kvp[l]));
    const long long e = (P.slot / 16) * p.block_stride + (P.slot % 16) * p.token_stride +
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
  if constexpr (S::WIDE) {
    // the chunk's 192 partial sums (3 heads x 64 dims, each added over the waves in wave order, fp32),
    // lane t of wave 0 publishing unit t = values 3t .. 3t + 2
    if (w == 0) {
      float f[3];
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        const int v = 3 * lane + k, h = v >> 6, d = v & 63;
        f[k] = ((sm.wo[0][h][d] + sm.wo[1][h][d]) + sm.wo[2][h][d]) + sm.wo[3][h][d];
      }
      C.put_loc(l, W::PART_U + size_t(P.rank) * S::PUC + lane,
                u32x4{__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]), C.tag});
    }
    if (w == 0 && lane == 0) trace_at(p, l, 20, p.n_layers);
    return;
  }
  // wave h < 3: head 3g + h.  The chunk's partial sum of p.v in fixed wave order, fp32.
  float O = 0.f;
  if (w < 3) {
#pragma unroll
    for (int v = 0; v < NCW; ++v) O += sm.wo[v][w][lane];
  }
  if (w < 3) {
    // PU units of 3 floats per head; lane 3u writes unit u (floats 3u .. 3u+2).  The workgroups doing
    // the O projection add the chunks' partials of each head in chunk order.
    const float f1 = __shfl_down(O, 1), f2 = __shfl_down(O, 2);
    if (lane % 3 == 0)
      C.put_loc(l, W::PART_U + size_t(P.rank) * S::PUC + size_t(w) * S::PU + lane / 3,
                u32x4{__float_as_uint(O), __float_as_uint(lane + 1 < 64 ? f1 : 0.f),
                      __float_as_uint(lane + 2 < 64 ? f2 : 0.f), C.tag});
  }
  if (w == 0 && lane == 0) trace_at(p, l, 20, p.n_layers);
}

// The attention vector of layer l into xs: per head unit (three dims of one head) the partial sums
// of the head's C chunks, added in chunk order in fp32 and rounded to bf16 once (HF's bf16(p.v)).
// Thread t takes head units t, t + NCT, ...; each is polled in all C chunk records.
template <class G>
__device__ __forceinline__ void attention_vector(CSR<G>& C, int l) {
  using S = SG<G>;
  using W = SWS<G>;
  constexpr int NHU = G::NH * S::PU;                 // head units of the attention vector
  constexpr int R = (NHU + NCT - 1) / NCT;
  static_assert(R * S::C <= 24, "partials polled per thread");
  static_assert(R <= 2, "two head units per thread at most");
  // chunk c of head h = 3g + w is group-A rank g + KVH c: its records are KVH * 3 * PU units apart,
  // and head unit hu = h PU + u of chunk 0 is record PART_U + (3 g + w) PU + u = PART_U + hu
  constexpr uint32_t CSTRIDE = uint32_t(G::KVH) * 3u * uint32_t(S::PU) * 16u;
  const int hu0 = C.ct, hu1 = C.ct + NCT;
  const uint32_t b0 = W::loc(l, W::PART_U + size_t(hu0 < NHU ? hu0 : 0));
  const uint32_t b1 = W::loc(l, W::PART_U + size_t(hu1 < NHU ? hu1 : 0));
  u32x4 v0[S::C], v1[S::C];
  // every load issued at once; then each head unit's set is polled to completion and summed
#pragma unroll
  for (int c = 0; c < S::C; ++c) v0[c] = ld_unit(C.rl, b0 + uint32_t(c) * CSTRIDE);
  if (R > 1 && hu1 < NHU)
#pragma unroll
    for (int c = 0; c < S::C; ++c) v1[c] = ld_unit(C.rl, b1 + uint32_t(c) * CSTRIDE);
  auto settle = [&](u32x4 (&v)[S::C], uint32_t b, int hu) {
    if (hu >= NHU) return;
    Spin spin(C.p.ws, C.tag, 36);
    while (true) {
      uint32_t pend = 0;
#pragma unroll
      for (int c = 0; c < S::C; ++c) pend |= v[c].w != C.tag ? 1u << c : 0u;
      if (!pend) break;
      if (C.dead || !spin.again()) { C.dead = true; break; }
#pragma unroll
      for (int c = 0; c < S::C; ++c)
        if ((pend >> c) & 1u) v[c] = ld_unit(C.rl, b + uint32_t(c) * CSTRIDE);
    }
    float t0 = 0.f, t1 = 0.f, t2 = 0.f;
#pragma unroll
    for (int c = 0; c < S::C; ++c) {
      t0 += __uint_as_float(v[c].x);
      t1 += __uint_as_float(v[c].y);
      t2 += __uint_as_float(v[c].z);
    }
    const int h = hu / S::PU, d = 3 * (hu - h * S::PU);
    float* dst = C.sm.xs + h * 64 + d;
    dst[0] = rnd(t0);
    if (d + 1 < 64) dst[1] = rnd(t1);
    if (d + 2 < 64) dst[2] = rnd(t2);
  };
  settle(v0, b0, hu0);
  if (R > 1) settle(v1, b1, hu1);
}

// Wide layout: slice c of KV head g's attention values (values 6c .. 6c + 5 of its 3 heads x 64
// dims): the 32 chunks' partial sums added in chunk order in fp32 and rounded to bf16 once (HF's
// bf16(p.v)), published as unit 32 g + c of the cross-XCD attention vector.  Wave 0: lane i polls
// unit 2c + (i & 1) of chunk i >> 1's record, the sums run over LDS.
template <class G>
__device__ __forceinline__ void attention_slice(CSR<G>& C, int l) {
  using S = SG<G>;
  using W = SWS<G>;
  static_assert(S::WIDE && 2 * S::C <= 64 && S::C * 6 <= NCW * 3 * 64, "one poll per lane; the slices fit sm.wo");
  const PlanSR<G>& P = C.P;
  if (C.cw != 0) return;
  const int lane = C.lane;
  float* flat = &C.sm.wo[0][0][0];  // [chunk][6]
  C.template poll<1>(C.rl, 2 * S::C, lane, 64,
                     [&](int i) {
                       return W::loc(l, W::PART_U + size_t(P.g + G::KVH * (i >> 1)) * S::PUC + size_t(2 * P.c + (i & 1)));
                     },
                     [&](int i, const u32x4& v) {
                       float* d = flat + (i >> 1) * 6 + (i & 1) * 3;
                       d[0] = __uint_as_float(v.x);
                       d[1] = __uint_as_float(v.y);
                       d[2] = __uint_as_float(v.z);
                     },
                     37);
  wait_lgkm0();
  __builtin_amdgcn_wave_barrier();
  float t = 0.f;
  if (lane < VPU)
#pragma unroll 8
    for (int j = 0; j < S::C; ++j) t += flat[j * 6 + lane];
  const float b = rnd(t);
  float a[VPU];
#pragma unroll
  for (int k = 0; k < VPU; ++k) a[k] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, b), k));
  if (lane == 0) C.put_x(K_ATT, l, S::C * P.g + P.c, C.unit6(a));
}

// ------------------------------------------------------------------------------------------------
// The LM head (both groups): final RMSNorm of x_L, this workgroup's rows of the tied embedding,
// its greedy candidate; then the end record every workgroup writes, gathered by workgroup 0
// ------------------------------------------------------------------------------------------------

template <class G>
__device__ __forceinline__ void lm_head_sr(CSR<G>& C) {
  using S = SG<G>;
  using W = SWS<G>;
  const Params& p = C.p;
  const PlanSR<G>& P = C.P;
  SmemSR<G>& sm = C.sm;
  const int L = p.n_layers;
  const uint32_t segf = C.next_seg(sr_bytes(P, R_FNORM, 0));
  C.wait_filled(C.pos);
  XChunks<G::H, 8> nw;
  normw<G::H>(C, nw, segf);
  C.release(C.pos);
  C.refresh();
  const float ss = C.template poll_vec<1>(K_X, L, G::H, sm.xs, nullptr, 33);
  const float rs = rms_rsq<G::H>(C.block_total(ss));
  C.bracket_done(uint32_t(L + 1));
  XChunks<G::H, 8> x;
  load_x<G::H, 8, true>(x, sm.xs, nw, rs, C.lane);
  if (P.wg == 0 && C.cw == 0) {
#pragma unroll
    for (int c = 0; c < Chunks<G::H>::CPL; ++c) {
      const int ch = C.lane + 64 * c;
      if (ch < Chunks<G::H>::CH) *reinterpret_cast<uint4*>(p.out_hidden + ch * 8) = x[c][0];
    }
  }
  float best = -INFINITY;
  int best_i = 0x7fffffff;
  for (int j = 0; j < P.n_lm; ++j) {
    const uint32_t seg = C.next_seg(sr_bytes(P, R_LM, j));
    const int r0 = P.v0 + j * S::LMR;
    const int nrows = min(S::LMR, P.v1 - r0);
    C.wait_filled(C.pos);
    constexpr int RW = S::LMR / NCW;  // rows cw RW .. cw RW + RW - 1 of the segment
    float out[RW];
    dots_n<G::H, RW>(C, seg, C.cw * RW, x, out);
    C.release(C.pos);
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const int row = C.cw * RW + r;
      if (row < nrows) {
        const float v = rnd(out[r]);
        const int idx = r0 + row;
        if (v > best || (v == best && idx < best_i)) { best = v; best_i = idx; }
        if (p.out_logits && C.lane == 0) p.out_logits[r0 + row] = uint16_t(f2bf(out[r]));
      }
    }
  }
  if (C.lane == 0) { sm.lm_val[C.cw] = best; sm.lm_idx[C.cw] = best_i; }
  C.cbar();
  if (C.ct == 0) trace_tail(p, 1);
  if (p.out_logits && (C.dead || aborted(p.ws, C.tag)))
    for (int i = P.v0 + C.ct; i < P.v1; i += NCT) p.out_logits[i] = 0x7fc0;
  // the end record of this workgroup: {best value, its index, dead flag, tag}
  if (C.ct == 0) {
    float bv = sm.lm_val[0];
    int bi = sm.lm_idx[0];
    for (int w = 1; w < NCW; ++w)
      if (sm.lm_val[w] > bv || (sm.lm_val[w] == bv && sm.lm_idx[w] < bi)) { bv = sm.lm_val[w]; bi = sm.lm_idx[w]; }
    skew_delay(p.skew, P.wg, p.n_layers, 9);
    st_unit<16>(C.rx, uint32_t(W::LMR + size_t(P.wg) * 16), u32x4{__float_as_uint(bv), uint32_t(bi), C.dead ? 1u : 0u, C.tag});
  }
  (void)S::HU;
}

// ------------------------------------------------------------------------------------------------
// Consumer main loops
// ------------------------------------------------------------------------------------------------

// Wide layout: group A's share of RMSNorm(h1) + gate/up + SwiGLU of layer l, after its O rows (the
// phase group F runs, without keeping h1 for the down residual): one 6-row gate or up item per wave,
// its weights in registers before h1 arrives, act units published.
template <class G>
__device__ __forceinline__ void gate_up_a(CSR<G>& C, int l) {
  static_assert(SG<G>::GU_ALL && SG<G>::NIT == 1, "one gate/up item per wave");
  const Params& p = C.p;
  const PlanSR<G>& P = C.P;
  SmemSR<G>& sm = C.sm;
  auto tr = [&](int ev) { if (C.ct == 0) trace_at(p, l, ev, p.n_layers); };
  C.refresh();
  const GUE& ge = sm.gue[l];
  const uint32_t segn = C.next_seg(sr_bytes(P, R_NORM2, 0));
  const uint32_t segg = C.next_seg(sr_bytes(P, R_GATE, 0, &ge));
  const uint32_t segg_s = C.next_seg(sr_bytes(P, R_GATE_S, 0));
  const uint32_t segg_h = C.next_seg(sr_bytes(P, R_GATE_H, 0, &ge));
  const uint32_t segg_r = C.next_seg(sr_bytes(P, R_GATE_R, 0, &ge));
  const uint32_t segu = C.next_seg(sr_bytes(P, R_UP, 0, &ge));
  const uint32_t segu_s = C.next_seg(sr_bytes(P, R_UP_S, 0));
  const uint32_t segu_h = C.next_seg(sr_bytes(P, R_UP_H, 0, &ge));
  const uint32_t segu_r = C.next_seg(sr_bytes(P, R_UP_R, 0, &ge));
  C.wait_filled(C.pos);
  XChunks<G::H, 8> nw;
  normw<G::H>(C, nw, segn);
  const int nunits = P.au1 - P.au0;
  const bool item = C.cw < 2 * nunits;
  uint4 w[VPU][Chunks<G::H>::CPL];
  if (item) {
    const int j = C.cw % nunits, m = C.cw < nunits ? 0 : 1;
    if (ge.on)
      lossless_rows<G::H, VPU>(C, m ? segu : segg, m ? segu_h : segg_h, m ? segu_r : segg_r, ge.first[m], j * VPU, w);
    else
      wrows<G, G::H, VPU>(C, m ? segu : segg, m ? segu_s : segg_s, j * VPU, w);
  }
  tr(9);
  const float ss = C.template poll_vec<1>(K_H1, l, G::H, sm.xs, nullptr, 43);
  const float rs = rms_rsq<G::H>(C.block_total(ss));
  tr(10);
  {
    XChunks<G::H, 8> x;
    load_x<G::H, 8, true>(x, sm.xs, nw, rs, C.lane);
    if (item) {
      float o[VPU];
      dots_w<G::H, VPU>(w, x, o);
      if (C.lane == 0)
#pragma unroll
        for (int e = 0; e < VPU; ++e) sm.part[C.cw][e] = o[e];
    }
    C.cbar();
    if (C.cw < nunits) {
      const int e = min(C.lane, VPU - 1);
      const float gv = rnd(sm.part[C.cw][e]), uv = rnd(sm.part[nunits + C.cw][e]);
      const float act = rnd(gv / (1.0f + expf(-gv))) * uv;
      float a[VPU];
#pragma unroll
      for (int k = 0; k < VPU; ++k)
        a[k] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, act), k));
      if (C.lane == 0) C.put_x(K_ACT, l, P.au0 + C.cw, C.unit6(a));
    }
  }
  C.release(C.pos);
  tr(11);
}

template <class G>
__device__ __forceinline__ void consumer_f(CSR<G>& C) {
  using S = SG<G>;
  using W = SWS<G>;
  const Params& p = C.p;
  const PlanSR<G>& P = C.P;
  SmemSR<G>& sm = C.sm;
  const int L = p.n_layers;
  auto tr = [&](int l, int ev) { if (C.ct == 0) trace_at(p, l, ev, p.n_layers); };
  // cos and sin (fp32 values) of this position for the three RoPE pairs of the wave's qkv unit,
  // which is the same in every layer
  float rc[VPU / 2], rsn[VPU / 2];
  {
    const int s0 = (P.qu0 + C.cw) * VPU;
#pragma unroll
    for (int k = 0; k < VPU / 2; ++k) {
      const int d = ((s0 + 2 * k) >> 1) & 31;
      const size_t at = size_t(P.pos) * 64;
      rc[k] = p.cs_fp32 ? reinterpret_cast<const float*>(p.cos_sin)[at + d]
                        : bf2f(reinterpret_cast<const uint16_t*>(p.cos_sin)[at + d]);
      rsn[k] = p.cs_fp32 ? reinterpret_cast<const float*>(p.cos_sin)[at + 32 + d]
                         : bf2f(reinterpret_cast<const uint16_t*>(p.cos_sin)[at + 32 + d]);
    }
  }
  for (int k = 0; k <= L; ++k) {
    if (k > 0) {
      const int l = k - 1;
      // ---- RMSNorm(h1) + gate/up + SwiGLU of layer l ----
      C.refresh();
      const GUE& ge = sm.gue[l];
      const uint32_t segn = C.next_seg(sr_bytes(P, R_NORM2, 0));
      const uint32_t segg = C.next_seg(sr_bytes(P, R_GATE, 0, &ge));
      const uint32_t segg_s = C.next_seg(sr_bytes(P, R_GATE_S, 0));
      const uint32_t segg_h = C.next_seg(sr_bytes(P, R_GATE_H, 0, &ge));
      const uint32_t segg_r = C.next_seg(sr_bytes(P, R_GATE_R, 0, &ge));
      const uint32_t segu = C.next_seg(sr_bytes(P, R_UP, 0, &ge));
      const uint32_t segu_s = C.next_seg(sr_bytes(P, R_UP_S, 0));
      const uint32_t segu_h = C.next_seg(sr_bytes(P, R_UP_H, 0, &ge));
      const uint32_t segu_r = C.next_seg(sr_bytes(P, R_UP_R, 0, &ge));
      C.wait_filled(C.pos);
      XChunks<G::H, 8> nw;
      normw<G::H>(C, nw, segn);
      // items: the gate rows of units 0 .. n-1, then the up rows of the same units, 6 rows each, item
      // w on wave w; its weights go from the ring into registers before h1 arrives.
      const int nunits = P.au1 - P.au0;
      const bool item = C.cw < 2 * nunits;
      uint4 w[VPU][Chunks<G::H>::CPL];
      if (item) {
        const int j = C.cw % nunits, m = C.cw < nunits ? 0 : 1;
        if (ge.on)  // the dense words rebuilt from the lossless stream (bit-identical)
          lossless_rows<G::H, VPU>(C, m ? segu : segg, m ? segu_h : segg_h, m ? segu_r : segg_r, ge.first[m],
                                   j * VPU, w);
        else
          wrows<G, G::H, VPU>(C, m ? segu : segg, m ? segu_s : segg_s, j * VPU, w);
      }
      tr(l, 9);
      const float ss = C.template poll_vec<1>(K_H1, l, G::H, sm.xs, sm.keep, 40);
      const float rs = rms_rsq<G::H>(C.block_total(ss));
      tr(l, 10);
      {
        XChunks<G::H, 8> x;
        load_x<G::H, 8, true>(x, sm.xs, nw, rs, C.lane);
        tr(l, 21);
        if (item) {
          float o[VPU];
          dots_w<G::H, VPU>(w, x, o);
          if (C.lane == 0)
#pragma unroll
            for (int e = 0; e < VPU; ++e) sm.part[C.cw][e] = o[e];
        }
        tr(l, 22);
        C.cbar();
        tr(l, 23);
        // unit j (wave j): lane e < 6 forms value e, silu(bf16(gate)) * bf16(up); lane 0 stores it
        if (C.cw < nunits) {
          const int j = C.cw;
          const int e = min(C.lane, VPU - 1);
          const float gv = rnd(sm.part[j][e]), uv = rnd(sm.part[nunits + j][e]);
          const float act = rnd(gv / (1.0f + expf(-gv))) * uv;
          float a[VPU];
#pragma unroll
          for (int k = 0; k < VPU; ++k)
            a[k] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, act), k));
          if (C.lane == 0) C.put_x(K_ACT, l, P.au0 + j, C.unit6(a));
        }
        tr(l, 24);
      }
      C.release(C.pos);
      tr(l, 11);
      // ---- down + residual of layer l -> x_{l+1} ----
      C.refresh();
      const uint32_t segd = C.next_seg(sr_bytes(P, R_DOWN, 0));
      const uint32_t segd_s = C.next_seg(sr_bytes(P, R_DOWN_S, 0));
      C.wait_filled(C.pos);
      if constexpr (S::NXU == 1) {
        const bool has_down = P.xu1 > P.xu0;  // workgroups without down rows do not need act
        // each wave: its quarter of K for the unit's 6 rows, weights into registers before act arrives;
        // the quarters are added in wave order
        using Q = Quarter<G::I>;
        uint4 wd[VPU][Q::CPL];
        if (has_down) wquarter<G, G::I, VPU>(C, segd, segd_s, 0, wd);
        if (has_down) C.template poll_vec<2>(K_ACT, l, G::I, sm.xs, nullptr, 41);
        C.cbar();
        tr(l, 13);
        if (has_down) {
          uint4 xq[Q::CPL];
#pragma unroll
          for (int c = 0; c < Q::CPL; ++c) {
            const int cq = C.lane + 64 * c;
            const float* src = sm.xs + (C.cw * Q::CHW + min(cq, Q::CHW - 1)) * 8;
            const float4 a = *reinterpret_cast<const float4*>(src);
            const float4 b = *reinterpret_cast<const float4*>(src + 4);
            const bool ok = cq < Q::CHW;
            xq[c] = make_uint4(ok ? pack2(a.x, a.y) : 0u, ok ? pack2(a.z, a.w) : 0u, ok ? pack2(b.x, b.y) : 0u,
                               ok ? pack2(b.z, b.w) : 0u);
          }
          tr(l, 28);
          float od[VPU];
          dots_quarter_w<G::I, VPU>(wd, xq, od);
          if (C.lane == 0)
#pragma unroll
            for (int e = 0; e < VPU; ++e) sm.part[C.cw][e] = od[e];
          C.cbar();
          tr(l, 29);
          if (C.cw == 0) {
            float y[VPU];
#pragma unroll
            for (int e = 0; e < VPU; ++e) {
              const float d = ((sm.part[0][e] + sm.part[1][e]) + sm.part[2][e]) + sm.part[3][e];
              const int r = min(P.d0 + e, G::H - 1);
              y[e] = rnd(sm.keep[r] + rnd(d));
            }
            if (C.lane == 0) C.put_x(K_X, l + 1, P.xu0, C.unit6(y));
            if (p.layer_outputs && C.lane < VPU && P.d0 + C.lane < G::H) {
              float yl = y[0];
#pragma unroll
              for (int e = 1; e < VPU; ++e) yl = C.lane == e ? y[e] : yl;
              p.layer_outputs[size_t(l) * G::H + P.d0 + C.lane] = uint16_t(f2bf(yl));
            }
          }
        }
      } else {
        const int nx = P.xu1 - P.xu0;  // workgroups without down rows do not need act
        // each wave: its quarter of K for every unit's 6 rows, the weights in registers before act
        // arrives; the quarters are added in wave order
        using Q = Quarter<G::I>;
        uint4 wd[S::NXU][VPU][Q::CPL];
#pragma unroll
        for (int u = 0; u < S::NXU; ++u)
          if (u < nx) wquarter<G, G::I, VPU>(C, segd, segd_s, u * VPU, wd[u]);
        if (nx > 0) C.template poll_vec<2>(K_ACT, l, G::I, sm.xs, nullptr, 41);
        C.cbar();
        tr(l, 13);
        if (nx > 0) {
          uint4 xq[Q::CPL];
#pragma unroll
          for (int c = 0; c < Q::CPL; ++c) {
            const int cq = C.lane + 64 * c;
            const float* src = sm.xs + (C.cw * Q::CHW + min(cq, Q::CHW - 1)) * 8;
            const float4 a = *reinterpret_cast<const float4*>(src);
            const float4 b = *reinterpret_cast<const float4*>(src + 4);
            const bool ok = cq < Q::CHW;
            xq[c] = make_uint4(ok ? pack2(a.x, a.y) : 0u, ok ? pack2(a.z, a.w) : 0u, ok ? pack2(b.x, b.y) : 0u,
                               ok ? pack2(b.z, b.w) : 0u);
          }
          tr(l, 28);
#pragma unroll
          for (int u = 0; u < S::NXU; ++u) {
            if (u >= nx) break;
            float od[VPU];
            dots_quarter_w<G::I, VPU>(wd[u], xq, od);
            if (C.lane == 0)
#pragma unroll
              for (int e = 0; e < VPU; ++e) sm.part[u * NCW + C.cw][e] = od[e];
          }
          C.cbar();
          tr(l, 29);
          if (C.cw < nx) {
            const int u = C.cw;
            float y[VPU];
#pragma unroll
            for (int e = 0; e < VPU; ++e) {
              const float* q = &sm.part[u * NCW][e];
              const float d = ((q[0] + q[8]) + q[16]) + q[24];  // the four waves' quarters, in wave order
              const int r = min(P.d0 + u * VPU + e, G::H - 1);
              y[e] = rnd(sm.keep[r] + rnd(d));
            }
            if (C.lane == 0) C.put_x(K_X, l + 1, P.xu0 + u, C.unit6(y));
            const int r0 = P.d0 + u * VPU;
            if (p.layer_outputs && C.lane < VPU && r0 + C.lane < G::H) {
              float yl = y[0];
#pragma unroll
              for (int e = 1; e < VPU; ++e) yl = C.lane == e ? y[e] : yl;
              p.layer_outputs[size_t(l) * G::H + r0 + C.lane] = uint16_t(f2bf(yl));
            }
          }
        }
      }
      C.release(C.pos);
      tr(l, 14);
    }
    if (k == L) break;
    // ---- RMSNorm(x) + QKV of layer k ----
    const int l = k;
    C.refresh();
    const uint32_t segn = C.next_seg(sr_bytes(P, R_NORM1, 0));
    const uint32_t segq = C.next_seg(sr_bytes(P, R_QKV, 0));
    const uint32_t segq_s = C.next_seg(sr_bytes(P, R_QKV_S, 0));
    C.wait_filled(C.pos);
    XChunks<G::H, 8> nw;
    normw<G::H>(C, nw, segn);
    // the weights of the wave's unit (a workgroup has at most NCW units), before x arrives
    const int nq = P.qu1 - P.qu0;
    uint4 wq[VPU][Chunks<G::H>::CPL];
    if (C.cw < nq) wrows<G, G::H, VPU>(C, segq, segq_s, C.cw * VPU, wq);
    tr(l, 0);
    float ss;
    if (l == 0) {
      long long id = p.ids_i64 ? reinterpret_cast<const int64_t*>(p.input_ids)[0]
                               : reinterpret_cast<const int32_t*>(p.input_ids)[0];
      id = min(max(id, 0LL), (long long)G::V - 1);
      const uint16_t* e = p.embed + size_t(id) * G::H;
      float s = 0.f;
      for (int i = C.ct; i < G::H; i += NCT) {
        const float v = bf2f(e[i]);
        sm.xs[i] = v;
        s += v * v;
      }
      ss = wave_sum(s);
    } else {
      ss = C.template poll_vec<1>(K_X, l, G::H, sm.xs, nullptr, 42);
    }
    const float rs = rms_rsq<G::H>(C.block_total(ss));
    tr(l, 1);
    {
      XChunks<G::H, 8> x;
      load_x<G::H, 8, true>(x, sm.xs, nw, rs, C.lane);
      tr(l, 25);
      if (C.cw < nq) {
        float o[VPU];
        dots_w<G::H, VPU>(wq, x, o);
        tr(l, 26);
        // q = bf16(W x); the pairs of the q and k slots get HF's RoPE,
        // bf16(bf16(x cos) + bf16(rotate_half(x) sin)), here
        const int s0 = (P.qu0 + C.cw) * VPU;
#pragma unroll
        for (int e = 0; e < VPU; e += 2) {
          const float x0 = rnd(o[e]), x1 = rnd(o[e + 1]);
          o[e] = x0;
          o[e + 1] = x1;
          if (s0 + e < (G::NH + G::KVH) * 64) {
            const float cs = rc[e / 2], sn = rsn[e / 2];
            o[e] = rnd(rnd(x0 * cs) + rnd((-x1) * sn));
            o[e + 1] = rnd(rnd(x1 * cs) + rnd(x0 * sn));
          }
        }
        if (C.lane == 0) C.put_x(K_XQ, l, P.qu0 + C.cw, C.unit6(o));
        tr(l, 27);
      }
    }
    C.release(C.pos);
    tr(l, 2);
    C.bracket_done(uint32_t(k + 1));
  }
  lm_head_sr<G>(C);
  (void)S::HU;
  (void)sizeof(W);
}

template <class G>
__device__ __forceinline__ void consumer_a(CSR<G>& C) {
  using S = SG<G>;
  using W = SWS<G>;
  const Params& p = C.p;
  const PlanSR<G>& P = C.P;
  SmemSR<G>& sm = C.sm;
  const int L = p.n_layers;
  auto tr = [&](int l, int ev) { if (C.ct == 0) trace_at(p, l, ev, p.n_layers); };
  // layer 0's input rows (the residual of this workgroup's O rows)
  {
    long long id = p.ids_i64 ? reinterpret_cast<const int64_t*>(p.input_ids)[0]
                             : reinterpret_cast<const int32_t*>(p.input_ids)[0];
    id = min(max(id, 0LL), (long long)G::V - 1);
    for (int r = P.o0 + C.ct; r < P.o1; r += NCT) sm.keep[r] = bf2f(p.embed[size_t(id) * G::H + r]);
  }
  // are the group-A workgroups that exchange records on one XCC (narrow: all of them, since the O
  // workgroups read every chunk's partials; wide: the 32 chunks of each KV head)?  Each publishes its
  // XCC_ID and reads those of its peers.
  {
    const uint32_t xcc = __builtin_amdgcn_s_getreg((15 << 11) | (0 << 6) | 20) & 15u;
    if (C.ct == 0) st_unit<16>(C.rx, uint32_t(W::XCC_TAB + size_t(P.rank) * 16), u32x4{xcc, 0u, 0u, C.tag});
    uint32_t mismatch = 0;
    constexpr int NP = S::WIDE ? S::C : S::AG;
    static_assert(NP <= 64, "one peer per lane");
    C.template poll<1>(C.rx, NP, C.lane, 64,
                       [&](int i) { return uint32_t(W::XCC_TAB + size_t(S::WIDE ? P.g + G::KVH * i : i) * 16); },
                       [&](int, const u32x4& v) { mismatch |= v.x != xcc ? 1u : 0u; }, 34);
    mismatch = __builtin_amdgcn_ballot_w64(mismatch != 0u) != 0ull ? 1u : 0u;
    if (C.ct == 0) sm.loc_l2 = (mismatch == 0u && p.xws != nullptr && p.l2_records) ? 1u : 0u;
    C.cbar();
    C.rl = sm.loc_l2 ? rsrc(p.xws) : rsrc(reinterpret_cast<uint8_t*>(C.region) + W::LOC);
  }
  for (int l = 0; l < L; ++l) {
    C.refresh();
    const uint32_t segkv = C.next_seg(sr_bytes(P, R_KV, 0));
    C.pos_kv_end = C.pos;
    const uint32_t sego = C.next_seg(sr_bytes(P, R_O, 0));
    const uint32_t sego_s = C.next_seg(sr_bytes(P, R_O_S, 0));
    ChunkRegs R;
    tr(l, 0);
    if (P.att) {
      // the KV chunk only: the O rows (needed after the attention) may still be streaming, as they
      // are in the first layer, whose chunk streams into an empty ring at the start of the launch
      // (tile reads past the chunk's last token read other ring bytes, which the masks discard)
      C.wait_filled(C.pos_kv_end);
      tr(l, 21);
      chunk_load<G>(C, segkv, R);
      tr(l, 22);
    }
    // x_l rows of this workgroup's O rows (the residual): layer 0 read the embedding above
    if (l > 0) {
      const int nu = P.ou1 - P.ou0;
      C.template poll<1>(C.rx, nu, C.ct, NCT, [&](int i) { return W::xoff(K_X, l, C.xr, P.ou0 + i); },
                         [&](int i, const u32x4& v) {
                           const float f[VPU] = {bf_lo(v.x), bf_hi(v.x), bf_lo(v.y), bf_hi(v.y), bf_lo(v.z), bf_hi(v.z)};
#pragma unroll
                           for (int e = 0; e < VPU; ++e) {
                             const int r = (P.ou0 + i) * VPU + e;
                             if (r < G::H) sm.keep[r] = f[e];
                           }
                         },
                         35);
    }
    tr(l, 6);
    if (P.att) attention_sr<G>(C, l, segkv, R);
    else C.release(C.pos_kv_end);
    // every group-A workgroup: the merged attention vector, then its O rows + residual -> h1
    C.cbar();  // the attention scratch shares storage with xs
    C.wait_filled(C.pos);
    // the workgroup's O rows, RW consecutive rows per wave, into registers: while the partials
    // arrive where the register budget allows it (SmolLM2-360M), else after them
    constexpr int RW = (S::OU * VPU + NCW - 1) / NCW;
    static_assert(RW <= 8, "sm.part holds 8 values per wave");
    uint4 wo[RW][Chunks<G::H>::CPL];
    if (S::O_EARLY) wrows<G, G::H, RW>(C, sego, sego_s, C.cw * RW, wo);
    C.refresh();  // the record loads below may not move up into the attention code
    if constexpr (S::WIDE) {
      // this chunk's slice of the attention vector, then the whole vector from every XCD
      tr(l, 16);
      attention_slice<G>(C, l);
      tr(l, 12);
      C.template poll_vec<1>(K_ATT, l, G::H, sm.xs, nullptr, 38);
      tr(l, 15);
    } else {
      attention_vector<G>(C, l);
    }
    if (!S::O_EARLY) wrows<G, G::H, RW>(C, sego, sego_s, C.cw * RW, wo);
    tr(l, 30);
    C.cbar();
    tr(l, 7);
    {
      XChunks<G::H, 8> x;
      const XChunks<G::H, 8> none = {};
      load_x<G::H, 8, false>(x, sm.xs, none, 1.f, C.lane);
      tr(l, 31);
      // the O rows' dots; then wave 0: h1 = bf16(x + bf16(o)) per row and one unit per lane
      float o[RW];
      dots_w<G::H, RW>(wo, x, o);
      if (C.lane == 0)
#pragma unroll
        for (int r = 0; r < RW; ++r) sm.part[C.cw][r] = o[r];
      tr(l, 32);
      C.cbar();  // also: every wave has read xs
      const int nrows = P.o1 - P.o0;
      if (C.cw == 0 && nrows > 0) {
        const int r = min(C.lane, nrows - 1);
        const float h = rnd(sm.keep[P.o0 + r] + rnd(sm.part[r / RW][r % RW]));
        if (C.lane < nrows) sm.xs[C.lane] = h;
        wait_lgkm0();
        if (C.lane < P.ou1 - P.ou0) {
          float v[VPU];
#pragma unroll
          for (int e = 0; e < VPU; ++e) v[e] = sm.xs[C.lane * VPU + e];
          C.put_x(K_H1, l, P.ou0 + C.lane, C.unit6(v));
        }
      }
      tr(l, 33);
    }
    C.release(C.pos);
    tr(l, 8);
    // the producers may stream the next bracket (wide: while this layer's gate/up share, streamed
    // with this bracket, is computed)
    C.bracket_done(uint32_t(l + 1));
    if constexpr (S::GU_ALL) gate_up_a<G>(C, l);
  }
  lm_head_sr<G>(C);
}


// Workgroup 0: every workgroup's end record; the step's greedy id, or, when any workgroup gave up a
// wait, poisoned outputs (ids -1, NaN hidden state) and the host-visible status.  Then the epoch.
template <class G>
__device__ __forceinline__ void final_gather(CSR<G>& C) {
  using W = SWS<G>;
  const Params& p = C.p;
  SmemSR<G>& sm = C.sm;
  const uint32_t epoch = C.tag;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  uint32_t bad = 0;
  static_assert(NWG == NCT, "one end record per consumer thread");
  {
    Spin spin(p.ws, epoch, 24);
    const uint32_t off = uint32_t(W::LMR + size_t(C.ct) * 16);
    u32x4 v = ld_unit(C.rx, off);
    while (v.w != epoch) {
      if (!spin.again()) { bad = 1; break; }
      v = ld_unit(C.rx, off);
    }
    if (!bad) {
      bv = __uint_as_float(v.x);
      bi = int(v.y);
      bad = v.z;
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
  }
  const bool any_bad = __builtin_amdgcn_ballot_w64(bad != 0u) != 0ull;
  C.cbar();  // the LM phase's reads of lm_val / lm_idx / red are over
  if (C.lane == 0) { sm.lm_val[C.cw] = bv; sm.lm_idx[C.cw] = bi; sm.red[C.cw] = any_bad ? 1.f : 0.f; }
  C.cbar();
  bool fail = C.dead || aborted(p.ws, epoch);
  for (int w = 0; w < NCW; ++w) fail = fail || sm.red[w] != 0.f;
  if (fail) {
    if (C.ct == 0 && !aborted(p.ws, epoch)) raise_abort(p.ws, epoch, 25);
    for (int i = C.ct; i < G::H; i += NCT) p.out_hidden[i] = 0x7fc0;
    if (p.out_logits)  // every logits row (best effort: a straggler may still store its own rows)
      for (int i = C.ct; i < G::V; i += NCT) p.out_logits[i] = 0x7fc0;
  }
  if (C.ct == 0) {
    bv = sm.lm_val[0];
    bi = sm.lm_idx[0];
    for (int w = 1; w < NCW; ++w)
      if (sm.lm_val[w] > bv || (sm.lm_val[w] == bv && sm.lm_idx[w] < bi)) { bv = sm.lm_val[w]; bi = sm.lm_idx[w]; }
    if (p.out_ids) p.out_ids[0] = fail ? -1 : bi;
    if (fail && p.host_status) {
      __hip_atomic_store(p.host_status + 1, ld_dev(p.ws + HDR_ABORT_WHERE), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      __hip_atomic_store(p.host_status, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    st_dev(p.ws + HDR_EPOCH, epoch);
  }
}

// ------------------------------------------------------------------------------------------------
// Kernel
// ------------------------------------------------------------------------------------------------

template <class G>
__global__ void __launch_bounds__(WG_THREADS, 1) decode_sr(Params p, uint32_t* region) {
  // each launched kernel takes its own range of contexts (narrow, wide, then the general kernel
  // beyond; all are launched and exactly one does the step)
  {
    const int S = min(max(p.seq_lens[0], 1), p.max_seq);
    if (S <= p.sr_min_s || S > p.sr_max_s) return;
  }
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_raw[];
  SmemSR<G>& sm = *reinterpret_cast<SmemSR<G>*>(smem_raw);
  if (threadIdx.x == 0) {
    for (int w = 0; w < NPW; ++w) sm.front[w] = 0;
    for (int w = 0; w < NCW; ++w) sm.consumed[w] = 0;
    for (int i = 0; i < 4; ++i) sm.zero16[i] = 0u;
    sm.cbar = 0;
    sm.go = 0;
    sm.loc_l2 = 0;
  }
  PlanSR<G> P;
  P.init(p, blockIdx.x);
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
    // lossless gate/up (SmolLM2-360M): this workgroup's act rows [a0, a1) of each matrix and their escapes
    GUE e{};
    if (G::WF == 0 && p.encoded_gu != nullptr && (!P.a || SG<G>::GU_ALL) && P.a1 > P.a0) {
      const EncodedGULayer d = p.encoded_gu[i];
      if (*d.enabled != 0u) {
        e.plane = d.plane;
        e.hdr = d.headers;
        e.raw = d.raw;
        e.on = 1u;
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          e.first[m] = d.row_offsets[m * G::I + P.a0];
          e.cnt[m] = d.row_offsets[m * G::I + P.a1] - e.first[m];
        }
      }
    }
    sm.gue[i] = e;
  }
  if (P.att) {
    const int nb = (P.t1 > P.t0) ? ((P.t1 - 1) / 16 - P.t0 / 16 + 1) : 0;
    for (int i = threadIdx.x; i < nb; i += WG_THREADS) sm.blk[i] = p.block_table[P.t0 / 16 + i];
  }
  trace_begin(p);
  __syncthreads();
  const uint32_t epoch = step_epoch(p.ws);
  if (threadIdx.x < 64 * NPW) {
    producer_sr<G>(p, P, sm, epoch);
  } else {
    // the consumer waves are the step's critical path: their instructions win the SIMD's issue
    // over the producer waves' DMA issue and ring polling when both are ready (+3.4% at ctx 1024)
    if constexpr (SG<G>::PRIO == 1) __builtin_amdgcn_s_setprio(1);
    CSR<G> C(p, P, sm, epoch, region);
    if (P.a) consumer_a<G>(C);
    else consumer_f<G>(C);
    if (blockIdx.x == 0) final_gather<G>(C);
  }
  __syncthreads();
  trace_end(p);
}

// ------------------------------------------------------------------------------------------------
// Exchange-unit integrity check (test hook).  `rounds` rounds; in round r each participating
// workgroup stores `upw` units (one per lane of its first wave) with tag = base + r and three payload
// words derived from (tag, unit), exactly as the decode kernels publish (one 16-byte store with the
// given cache bits), into a region of its own for the round; then every participant polls all units
// of the round with the decode kernels' 16-byte device-scope loads and compares the payload of every
// unit it accepts (tag current) with the expected words.  out[0] counts mismatches (a torn unit:
// current tag, stale or mixed payload), out[1] polls given up, out[2] units checked, out[3] is the
// mask of XCC ids the participants ran on.  Every wait is bounded; a mismatch is counted, never
// waited on.
// ------------------------------------------------------------------------------------------------

__device__ __forceinline__ uint32_t unit_word(uint32_t tag, uint32_t unit, uint32_t k) {
  uint32_t h = tag * 0x9e3779b1u ^ (unit + 1u) * 0x85ebca77u ^ (k + 1u) * 0xc2b2ae3du;
  h ^= h >> 15;
  h *= 0x2c1b3c6du;
  h ^= h >> 12;
  return h;
}

template <int AUX_ST>
__global__ void __launch_bounds__(NCT, 1) unit_check(uint8_t* buf, uint32_t buf_bytes, uint32_t base, int rounds,
                                                     int upw, int slot, int one_xcd, uint32_t* out) {
  const int wg = blockIdx.x, t = threadIdx.x;
  if (one_xcd && (wg & 7) != 0) return;
  const int np = one_xcd ? NWG / 8 : NWG;                // participating workgroups
  const int rank = one_xcd ? wg >> 3 : wg;
  const int nu = np * upw;                               // units per round
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(buf, (short)0, int(buf_bytes), 0x00020000);
  uint32_t bad = 0, gave_up = 0, checked = 0;
  for (int k = 0; k < rounds; ++k) {
    const uint32_t tag = base + uint32_t(k);
    const uint32_t round_off = uint32_t(k) * uint32_t(nu) * uint32_t(slot);
    if (t < upw) {
      const uint32_t u = uint32_t(rank * upw + t);
      st_unit<AUX_ST>(r, round_off + u * uint32_t(slot),
                      u32x4{unit_word(tag, u, 0), unit_word(tag, u, 1), unit_word(tag, u, 2), tag});
    }
    for (int u = t; u < nu; u += NCT) {
      const uint32_t off = round_off + uint32_t(u) * uint32_t(slot);
      u32x4 v = ld_unit(r, off);
      uint32_t n = 0;
      while (v.w != tag && ++n < (1u << 20)) {
        asm volatile("" ::: "memory");  // the load is issued again on every pass (not hoisted)
        v = ld_unit(r, off);
      }
      if (v.w != tag) { ++gave_up; continue; }
      ++checked;
      bad += (v.x != unit_word(tag, u, 0) || v.y != unit_word(tag, u, 1) || v.z != unit_word(tag, u, 2)) ? 1u : 0u;
    }
  }
  if (bad) atomicAdd(out + 0, bad);
  if (gave_up) atomicAdd(out + 1, gave_up);
  atomicAdd(out + 2, checked);
  if (t == 0) atomicOr(out + 3, 1u << (__builtin_amdgcn_s_getreg((15 << 11) | (0 << 6) | 20) & 15u));  // XCC_ID
}

}  // namespace sr
}  // namespace pk

// ------------------------------------------------------------------------------------------------
// Host side
// ------------------------------------------------------------------------------------------------

// Test hook: the exchange-unit integrity check on the current device (synchronous).  mode 0: 256
// workgroups, uncached memory, device-scope stores and loads (pk_decode's cross-XCD units); mode 1:
// the same in ordinary device memory (pk_decode_noalloc's array); mode 2: the 32 workgroups of one
// XCD under round-robin dispatch, ordinary memory, plain stores and device-scope loads (group A's
// records through the XCD's L2).  `slot` is the bytes between units (16: four units, stored by
// different workgroups, share each 64-byte line; 64: one unit per line as the decode kernels place
// them).  out receives {mismatches, polls given up, units checked, mask of the XCC ids the
// participating workgroups ran on}.  The buffers are allocated on the
// first call on a device and kept until the process ends.  No reference counterpart.
extern "C" int pk_test_exchange_units(int mode, int rounds, int slot, unsigned* out) {
  using namespace pk;
  static uint8_t* ubuf[64] = {};
  static uint8_t* cbuf[64] = {};
  static uint32_t* cnt[64] = {};
  static uint32_t next_base[64] = {};
  constexpr int UPW = 4;                      // units per workgroup and round
  constexpr size_t BYTES = size_t(64) << 20;
  if (mode < 0 || mode > 2 || (slot != 16 && slot != 64) || rounds < 1 ||
      size_t(rounds) * NWG * UPW * size_t(slot) > BYTES || out == nullptr)
    return PK_ERR_BLOCK;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= 64) return PK_ERR_RESIDENCY;
  if (!ubuf[dev]) {
    if ((e = hipExtMallocWithFlags(reinterpret_cast<void**>(&ubuf[dev]), BYTES, hipDeviceMallocUncached)) != hipSuccess) return e;
    if ((e = hipMalloc(reinterpret_cast<void**>(&cbuf[dev]), BYTES)) != hipSuccess) return e;
    if ((e = hipMalloc(reinterpret_cast<void**>(&cnt[dev]), 16)) != hipSuccess) return e;
    if ((e = hipMemset(ubuf[dev], 0, BYTES)) != hipSuccess) return e;
    if ((e = hipMemset(cbuf[dev], 0, BYTES)) != hipSuccess) return e;
    next_base[dev] = 1u;
  }
  if ((e = hipMemset(cnt[dev], 0, 16)) != hipSuccess) return e;  // 4 counters
  const uint32_t base = next_base[dev];
  next_base[dev] += uint32_t(rounds);
  uint8_t* buf = mode == 0 ? ubuf[dev] : cbuf[dev];
  const uint32_t bytes = uint32_t(BYTES);
  int one_xcd = mode == 2 ? 1 : 0;
  void* args[] = {&buf, const_cast<uint32_t*>(&bytes), const_cast<uint32_t*>(&base), &rounds,
                  const_cast<int*>(&UPW), &slot, &one_xcd, &cnt[dev]};
  const void* fn = mode == 2 ? reinterpret_cast<const void*>(sr::unit_check<0>)
                             : reinterpret_cast<const void*>(sr::unit_check<16>);
  // one workgroup per CU: the LDS this launch asks for keeps a second one off every CU
  if ((e = hipLaunchKernel(fn, dim3(NWG), dim3(NCT), args, 96 * 1024, nullptr)) != hipSuccess) return e;
  if ((e = hipDeviceSynchronize()) != hipSuccess) return e;
  uint32_t h[4] = {0, 0, 0, 0};
  if ((e = hipMemcpy(h, cnt[dev], 16, hipMemcpyDeviceToHost)) != hipSuccess) return e;
  for (int i = 0; i < 4; ++i) out[i] = h[i];
  return PK_OK;
}

namespace pk {
namespace sr {

// The compiled kernels: narrow and wide layouts of SmolLM2-360M (bf16 and MXFP8 weights) and of
// SmolLM2-135M.
using N360 = SrG<G360, 1>;
using N135 = SrG<G135, 1>;
using N360Q = SrG<G360Q, 1>;
using W360 = SrG<G360, G360::KVH>;
using W135 = SrG<G135, G135::KVH>;
using W360Q = SrG<G360Q, G360Q::KVH>;
// SmolLM2-135M's shorter contexts: 4 chunks per KV head (12 attending workgroups, the other 20 of
// group A only project O) up to 1,025 tokens, 6 up to 1,537, instead of 10: fewer records in both
// attention exchanges and the O rows preloaded (config 2: 2,455 -> 2,624 tok/s; 1,200 tokens:
// 2,438 -> 2,577; 3 or 6 chunks at config 2: -1.7%, -1.1%); the 10-chunk build takes the contexts
// above 1,537
using N135S = SrG<G135, 1, 4>;
using N135M = SrG<G135, 1, 6>;

// Longest context (tokens attended, the new one included) the kernel takes: C chunks of at most TCS
// cached tokens per KV head, and a chunk's K/V plus the workgroup's O rows within the LDS ring.
template <class G>
constexpr int max_seq() {
  using S = SG<G>;
  constexpr uint32_t o_bytes = pad_pkt(uint32_t(S::OU) * VPU * G::H * S::WB) +
                               (G::WF ? pad_pkt(uint32_t(S::OU) * VPU * uint32_t(scale_stride(G::H))) : 0u);
  constexpr int tc_ring = int((RING - o_bytes - 2 * PKT) / 256u) / 16 * 16;
  constexpr int tc = tc_ring < S::TCS ? tc_ring : S::TCS;
  return S::C * tc + 1;
}
static_assert(max_seq<N360>() >= 1281 && max_seq<N135>() >= 769, "the narrow layout covers configs 2 and 3");
static_assert(max_seq<W360Q>() >= 8192 + 288 && max_seq<W360>() == max_seq<W360Q>() && max_seq<W135>() >= max_seq<W360>(),
              "the wide layout covers config 5 (context 8192, then the benchmark's steps)");
static_assert(max_seq<N360Q>() == max_seq<N360>(), "one narrow limit per model");
static_assert(max_seq<N135S>() >= 769 && max_seq<N135S>() < max_seq<N135M>() && max_seq<N135M>() < max_seq<N135>(),
              "the 4-chunk 135M build covers config 2; each shorter build ends below the next");
static_assert(max_seq<N360>() == PK_NOALLOC_MAX_SEQ_360M && max_seq<N135>() == PK_NOALLOC_MAX_SEQ_135M,
              "the context limits pk_decode_noalloc documents");
constexpr size_t pages(size_t n) { return (n + 4095) / 4096 * 4096; }
static_assert(4096 + pages(SWS<N360>::BYTES) + pages(SWS<N360>::LOC_BYTES) <= PK_NOALLOC_SCRATCH_BYTES &&
                  4096 + pages(SWS<N135>::BYTES) + pages(SWS<N135>::LOC_BYTES) <= PK_NOALLOC_SCRATCH_BYTES,
              "header, region and group-A records fit pk_decode_noalloc's array");

template <class G>
constexpr size_t lds_bytes() { return sizeof(SmemSR<G>); }
template <class G>
constexpr bool lds_fits() { return (sizeof(SmemSR<G>) + 15) / 16 * 16 + TRACE_LDS_BYTES <= 160 * 1024; }
static_assert(lds_fits<N360>() && lds_fits<N135>() && lds_fits<N360Q>() && lds_fits<W360>() && lds_fits<W135>() &&
                  lds_fits<W360Q>() && lds_fits<N135S>() && lds_fits<N135M>(),
              "LDS budget of one gfx950 workgroup, with the diagnostic timestamps");

template <class G>
static int launch(const Params& p, uint32_t* region, uint32_t* local, hipStream_t stream, int cooperative) {
  static int ready[64] = {};
  static int status[64] = {};
  const void* fn = reinterpret_cast<const void*>(decode_sr<G>);
  size_t lds = lds_bytes<G>();
  const size_t trace_off = (lds + 15) / 16 * 16;
  const size_t lds_traced = trace_off + TRACE_LDS_BYTES;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= 64) return PK_ERR_RESIDENCY;
  if (!ready[dev]) {
    hipDeviceProp_t prop;
    int st = 0, max_lds = 0;
    if ((e = hipGetDeviceProperties(&prop, dev)) != hipSuccess) st = e;
    else if ((e = hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev)) != hipSuccess) st = e;
    else if (__builtin_strncmp(prop.gcnArchName, "gfx950", 6) != 0) st = PK_ERR_ARCH;
    else if (prop.multiProcessorCount < NWG || size_t(max_lds) < lds_traced) st = PK_ERR_RESIDENCY;
    else if ((e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, int(lds_traced))) != hipSuccess) st = e;
    status[dev] = st;
    ready[dev] = 1;
  }
  if (status[dev]) return status[dev];
  Params q = p;
  q.xws = local;
  if (q.trace) {
    if (q.n_layers > TR_LAYERS) return PK_ERR_MODEL;
    q.trace_lds = uint32_t(trace_off);
    lds = lds_traced;
  }
  void* args[] = {&q, &region};
  if (cooperative) e = hipLaunchCooperativeKernel(fn, dim3(NWG), dim3(WG_THREADS), args, lds, stream);
  else e = hipLaunchKernel(fn, dim3(NWG), dim3(WG_THREADS), args, lds, stream);
  if (e != hipSuccess) return e;
  return hipGetLastError();
}

}  // namespace sr

int sr_launch(int model, int wf, int wide, const Params& p, uint32_t* region, uint32_t* local, hipStream_t stream,
              int cooperative) {
  if (wide >= 2) {  // the narrow layout with fewer chunks, for the shorter contexts (135M only)
    if (model == PK_MODEL_SMOLLM2_135M && !wf && wide == 2) return sr::launch<sr::N135S>(p, region, local, stream, cooperative);
    if (model == PK_MODEL_SMOLLM2_135M && !wf && wide == 3) return sr::launch<sr::N135M>(p, region, local, stream, cooperative);
    return PK_ERR_MODEL;
  }
  if (model == PK_MODEL_SMOLLM2_360M && wf)
    return wide ? sr::launch<sr::W360Q>(p, region, local, stream, cooperative)
                : sr::launch<sr::N360Q>(p, region, local, stream, cooperative);
  if (model == PK_MODEL_SMOLLM2_360M)
    return wide ? sr::launch<sr::W360>(p, region, local, stream, cooperative)
                : sr::launch<sr::N360>(p, region, local, stream, cooperative);
  if (model == PK_MODEL_SMOLLM2_135M && !wf)
    return wide ? sr::launch<sr::W135>(p, region, local, stream, cooperative)
                : sr::launch<sr::N135>(p, region, local, stream, cooperative);
  return PK_ERR_MODEL;
}
template <class A, class B>
static constexpr size_t zmax(A a, B b) { return size_t(a) > size_t(b) ? size_t(a) : size_t(b); }
size_t sr_region_bytes(int all) {
  using namespace sr;
  const size_t narrow = zmax(SWS<N360>::BYTES, SWS<N135>::BYTES);
  return all ? zmax(zmax(zmax(zmax(narrow, SWS<N360Q>::BYTES), SWS<N135S>::BYTES), SWS<N135M>::BYTES),
                   zmax(zmax(SWS<W360>::BYTES, SWS<W135>::BYTES), SWS<W360Q>::BYTES))
             : narrow;
}
size_t sr_local_bytes(int wide) {
  using namespace sr;
  return wide ? zmax(zmax(SWS<W360>::LOC_BYTES, SWS<W135>::LOC_BYTES), SWS<W360Q>::LOC_BYTES)
              : zmax(zmax(zmax(SWS<N360>::LOC_BYTES, SWS<N135>::LOC_BYTES), SWS<N360Q>::LOC_BYTES),
                     zmax(SWS<N135S>::LOC_BYTES, SWS<N135M>::LOC_BYTES));
}
int sr_max_seq(int model, int wide) {
  using namespace sr;
  if (model == PK_MODEL_SMOLLM2_360M) return wide >= 2 ? 0 : wide ? max_seq<W360>() : max_seq<N360>();
  if (model == PK_MODEL_SMOLLM2_135M)
    return wide == 3 ? max_seq<N135M>() : wide == 2 ? max_seq<N135S>() : wide ? max_seq<W135>() : max_seq<N135>();
  return 0;
}

}  // namespace pk
