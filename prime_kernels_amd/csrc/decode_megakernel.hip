// SmolLM2 single-token decode step as one persistent cooperative HIP kernel for gfx950 (MI355X).
//
// One workgroup per CU (256), 5 wave64s each:
//   wave 0      producer: streams this workgroup's share of every weight matrix (and its KV-cache
//               chunk) from HBM into a 128 KB LDS ring with LDS-DMA loads
//               (global_load_lds_dwordx4), up to DEPTH 1 KB packets in flight, running ahead of
//               the dependency chain because weights and cached K/V do not depend on activations.
//   waves 1..4  consumers: pull their rows from the ring into VGPRs, wait for the phase input,
//               compute, publish the phase output.
//
// Phases per layer (the reference's eight grid barriers per layer, block360_kernel.inc:96-803,
// become data-flow edges):
//   P1 RMSNorm(x) + QKV GEMV             -> qkv (pre-RoPE, bf16)
//   P2 RoPE + GQA attention partials over a KV chunk; chunk leaders merge (log-sum-exp)
//                                         -> attn (bf16)
//   P3 O GEMV + residual                  -> h1
//   P4 RMSNorm(h1) + gate/up GEMV + SwiGLU -> act
//   P5 down GEMV + residual               -> x (layer output)
//   then final RMSNorm + tied LM head GEMV with per-workgroup argmax, and a 256-way argmax.
//
// Inter-workgroup exchange: no counters, no fences.  Every exchanged value is written as a
// 32-bit word {tag16, bf16} (or a 64-bit word {tag32, fp32}) with device-scope relaxed atomic
// stores, into a buffer owned by one (layer, phase, sequence).  Readers poll those words with
// device-scope (sc1) loads until every tag equals this step's epoch, so the data arrives with
// the "ready" signal in one round trip.  The epoch is a device counter bumped by workgroup 0 at
// the end of every step.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "../../include/prime_decode.h"

namespace pk {

static unsigned long long* g_trace = nullptr;

// ------------------------------------------------------------------------------------------------
// Geometry and launch constants
// ------------------------------------------------------------------------------------------------

template <int H_, int NH_, int KVH_, int I_, int L_>
struct Geom {
  static constexpr int H = H_, NH = NH_, KVH = KVH_, D = 64, I = I_, L = L_, V = 49152;
  static constexpr int QKV = (NH + 2 * KVH) * D;
  static constexpr int GQA = NH / KVH;
  static_assert(GQA == 3, "SmolLM2 uses 3 query heads per KV head");
};
using G360 = Geom<960, 15, 5, 2560, 32>;   // decode_megakernel_360m/__init__.py:27-35
using G135 = Geom<576, 9, 3, 1536, 30>;    // decode_megakernel/__init__.py:37-43

constexpr int NWG = 256;                 // persistent workgroups (one per CU)
constexpr int NCW = 4;                   // consumer waves per workgroup
constexpr int NCT = 64 * NCW;            // consumer threads
constexpr int WG_THREADS = 64 * (1 + NCW);
constexpr uint32_t RING = 128u * 1024u;  // LDS ring bytes (power of two)
constexpr uint32_t PKT = 1024;           // one LDS-DMA instruction: 64 lanes x 16 B
constexpr int DEPTH = 48;                // packets in flight per workgroup
constexpr int TC_MAX = 256;              // max cached tokens per attention chunk (64 KB of K/V)
constexpr int TC_TARGET = 128;           // preferred tokens per chunk
constexpr int LM_ROWS = 16;              // LM-head rows per ring segment
constexpr int MAX_B = 16;                // exchange-buffer slots per layer
constexpr int REC_WORDS = 3 * 66;        // attention partial: 3 heads x (m, l, o[64]), 64-bit words
constexpr uint32_t SPIN_LIMIT = 1u << 22;
constexpr int kMaxSeq = 12288;          // tokens per sequence (block_table capacity)

// Workspace header words.
constexpr int HDR_EPOCH = 0;
constexpr int HDR_ABORT = 1;
constexpr int HDR_ABORT_WHERE = 2;
constexpr size_t HDR_WORDS = 64;

struct LayerW {
  const uint16_t* norm1;    // [H]
  const uint16_t* qkv;      // [(NH+2KVH)*D, H]: q rows, then k rows, then v rows
  const uint16_t* o;        // [H, H]
  const uint16_t* norm2;    // [H]
  const uint16_t* gate_up;  // [2I, H]: gate rows, then up rows
  const uint16_t* down;     // [H, I]
};

struct Params {
  const LayerW* layers;
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
  int ids_i64;
  unsigned long long* trace;   // optional per-phase timestamps (diagnostics)
};

// Exchange-buffer layout (32-bit words).
template <class G>
struct WS {
  static constexpr size_t PER_B = size_t(G::QKV) + 3 * G::H + G::I;  // qkv, attn, h1, act, x
  static constexpr size_t LAYER = PER_B * MAX_B;
  static constexpr size_t REC0 = HDR_WORDS + LAYER * G::L;
  static constexpr size_t REC_LAYER = size_t(NWG) * REC_WORDS * 2;
  static constexpr size_t LM0 = REC0 + REC_LAYER * G::L;
  static constexpr size_t TOTAL = LM0 + size_t(MAX_B) * NWG * 2;
  __device__ static size_t qkv(int l, int b) { return HDR_WORDS + l * LAYER + b * PER_B; }
  __device__ static size_t attn(int l, int b) { return qkv(l, b) + G::QKV; }
  __device__ static size_t h1(int l, int b) { return attn(l, b) + G::H; }
  __device__ static size_t act(int l, int b) { return h1(l, b) + G::H; }
  __device__ static size_t x(int l, int b) { return act(l, b) + G::I; }
  __device__ static size_t rec(int l, int item) { return REC0 + l * REC_LAYER + size_t(item) * REC_WORDS * 2; }
  __device__ static size_t lm(int b, int wg) { return LM0 + (size_t(b) * NWG + wg) * 2; }
};

// ------------------------------------------------------------------------------------------------
// Scalar helpers
// ------------------------------------------------------------------------------------------------

__device__ __forceinline__ float bf2f(uint32_t b) { return __uint_as_float(b << 16); }

// fp32 -> bf16 bits, round to nearest even (NaN stays NaN).
__device__ __forceinline__ uint32_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
__device__ __forceinline__ float rnd(float f) { return bf2f(f2bf(f)); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
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

// Diagnostic timestamps: TR_EVENTS per layer per workgroup, plus TR_TAIL at the end.
constexpr int TR_EVENTS = 16;
constexpr int TR_TAIL = 4;
__device__ __forceinline__ void trace_at(const Params& p, int layer, int ev, int n_layers) {
  if (p.trace)
    p.trace[size_t(blockIdx.x) * (size_t(n_layers) * TR_EVENTS + TR_TAIL) + size_t(layer) * TR_EVENTS + ev] =
        wall_clock64();
}

// ------------------------------------------------------------------------------------------------
// Per-workgroup plan: which rows / chunk this workgroup owns.  Computed identically by all waves.
// ------------------------------------------------------------------------------------------------

__device__ __forceinline__ int split_lo(int n, int parts, int i) { return int((long long)n * i / parts); }

template <class G>
struct Plan {
  int wg;
  int q0, q1;   // QKV rows
  int o0, o1;   // O rows
  int a0, a1;   // act indices (gate rows a0..a1-1, up rows I+a0..)
  int d0, d1;   // down rows
  int v0, v1;   // LM-head rows
  int n_lm;     // LM segments
  // attention (batch 1)
  int att;      // 1: this workgroup owns an attention chunk
  int g, c, C, t0, t1;   // kv head, chunk, chunks, cached token range [t0, t1)
  int S, pos;   // tokens attended (incl. new) and the new token's position
  int leader;   // owns the new token, merges the chunk partials and appends K/V

  __device__ void init(const Params& p, int wg_) {
    wg = wg_;
    q0 = split_lo(G::QKV, NWG, wg); q1 = split_lo(G::QKV, NWG, wg + 1);
    o0 = split_lo(G::H, NWG, wg);   o1 = split_lo(G::H, NWG, wg + 1);
    a0 = split_lo(G::I, NWG, wg);   a1 = split_lo(G::I, NWG, wg + 1);
    d0 = split_lo(G::H, NWG, wg);   d1 = split_lo(G::H, NWG, wg + 1);
    if (p.lm_head) {
      v0 = split_lo(G::V, NWG, wg); v1 = split_lo(G::V, NWG, wg + 1);
    } else {
      v0 = v1 = 0;
    }
    n_lm = (v1 - v0 + LM_ROWS - 1) / LM_ROWS;
    S = max(p.seq_lens[0], 1);
    pos = int(max(p.positions[0], (int64_t)0));
    const int old = S - 1;
    int C0 = old <= 0 ? 1 : (old + TC_TARGET - 1) / TC_TARGET;
    const int cmax = NWG / G::KVH;
    C0 = min(C0, cmax);
    int tc = old <= 0 ? 16 : ((old + C0 - 1) / C0 + 15) / 16 * 16;
    C = old <= 0 ? 1 : (old + tc - 1) / tc;
    const int items = G::KVH * C;
    att = wg < items;
    g = c = t0 = t1 = leader = 0;
    if (att) {
      g = wg / C;
      c = wg % C;
      t0 = min(c * tc, old);
      t1 = min((c + 1) * tc, old);
      leader = c == C - 1;
    }
  }
};

// Byte sizes of the segments a workgroup streams, in stream order.
// Per layer: 0 QKV rows, 1 KV chunk, 2 O rows, 3 gate rows, 4 up rows, 5 down rows;
// then n_lm LM-head segments.
constexpr int SEGS_PER_LAYER = 6;

template <class G>
__device__ __forceinline__ uint32_t seg_bytes(const Plan<G>& P, int kind, int lm_index) {
  switch (kind) {
    case 0: return uint32_t(P.q1 - P.q0) * G::H * 2;
    case 1: return P.att ? uint32_t(P.t1 - P.t0) * 256u : 0u;
    case 2: return uint32_t(P.o1 - P.o0) * G::H * 2;
    case 3:
    case 4: return uint32_t(P.a1 - P.a0) * G::H * 2;
    case 5: return uint32_t(P.d1 - P.d0) * G::I * 2;
    default: {
      const int r0 = P.v0 + lm_index * LM_ROWS;
      const int r1 = min(r0 + LM_ROWS, P.v1);
      return uint32_t(r1 - r0) * G::H * 2;
    }
  }
}

__device__ __forceinline__ uint32_t pad_pkt(uint32_t b) { return (b + PKT - 1) & ~(PKT - 1); }

// ------------------------------------------------------------------------------------------------
// Shared memory layout
// ------------------------------------------------------------------------------------------------

template <class G>
struct Smem {
  static constexpr int XS = G::I > G::H ? G::I : G::H;
  uint8_t ring[RING];
  float xs[XS];              // current phase input (bf16 values as fp32)
  float xkeep[G::H];         // layer input x (residual for O)
  float h1keep[G::H];        // h1 (residual for down)
  float red[64];
  float qrot[3 * 64];
  float knew[64];
  float vnew[64];
  float sc[3 * (TC_MAX + 1)];
  float opart[NCW * 3 * 64];
  float ml[8];
  int32_t blk[TC_MAX / 16 + 2];
  float lm_val[NCW];
  int32_t lm_idx[NCW];
  uint32_t filled;
  uint32_t consumed[NCW];
  uint32_t cbar;
};

// ------------------------------------------------------------------------------------------------
// Spin helper with a bound and a global abort word, so a logic error cannot hang the GPU.
// ------------------------------------------------------------------------------------------------

struct Spin {
  uint32_t n = 0;
  uint32_t* abort_word;
  int where;
  __device__ Spin(uint32_t* ws, int w) : abort_word(ws + HDR_ABORT), where(w) {}
  // Returns false when the wait must be abandoned.
  __device__ __forceinline__ bool again() {
    ++n;
    if ((n & 127u) == 0) {
      if (ld_dev(abort_word)) return false;
      if (n >= SPIN_LIMIT) {
        st_dev(abort_word, 1u);
        st_dev(abort_word + 1, uint32_t(where));
        return false;
      }
    }
    __builtin_amdgcn_s_sleep(1);
    return true;
  }
};

// ------------------------------------------------------------------------------------------------
// Producer wave
// ------------------------------------------------------------------------------------------------

template <class G>
__device__ void producer(const Params& p, const Plan<G>& P, Smem<G>& sm) {
  const int lane = threadIdx.x & 63;
  const uint32_t ring_base = uint32_t(reinterpret_cast<uintptr_t>(sm.ring));
  // Block ids of this workgroup's attention chunk (same for every layer).
  if (P.att) {
    const int nb = (P.t1 > P.t0) ? ((P.t1 - 1) / 16 - P.t0 / 16 + 1) : 0;
    for (int i = lane; i < nb; i += 64) sm.blk[i] = p.block_table[P.t0 / 16 + i];
  }
  wait_vmcnt<0>();
  __builtin_amdgcn_s_barrier();  // consumers may read blk[] after this

  uint32_t pos = 0;
  Spin spin(p.ws, 1);
  bool dead = false;
  auto ring_space = [&]() -> bool {
    uint32_t cmin = ld_lds(&sm.consumed[0]);
#pragma unroll
    for (int w = 1; w < NCW; ++w) cmin = min(cmin, ld_lds(&sm.consumed[w]));
    return pos + PKT <= cmin + RING;
  };
  auto issue_segment = [&](int kind, int layer, int lm_index) {
    const uint32_t bytes = seg_bytes(P, kind, lm_index);
    const uint32_t npk = pad_pkt(bytes) / PKT;
    const uint8_t* base = nullptr;
    if (kind != 1) {
      const LayerW* Lw = p.layers + layer;
      switch (kind) {
        case 0: base = reinterpret_cast<const uint8_t*>(Lw->qkv) + size_t(P.q0) * G::H * 2; break;
        case 2: base = reinterpret_cast<const uint8_t*>(Lw->o) + size_t(P.o0) * G::H * 2; break;
        case 3: base = reinterpret_cast<const uint8_t*>(Lw->gate_up) + size_t(P.a0) * G::H * 2; break;
        case 4: base = reinterpret_cast<const uint8_t*>(Lw->gate_up) + size_t(G::I + P.a0) * G::H * 2; break;
        case 5: base = reinterpret_cast<const uint8_t*>(Lw->down) + size_t(P.d0) * G::I * 2; break;
        default: base = reinterpret_cast<const uint8_t*>(p.embed) + size_t(P.v0 + lm_index * LM_ROWS) * G::H * 2; break;
      }
    }
    const uint8_t* cache = kind == 1 ? reinterpret_cast<const uint8_t*>(p.kv[layer]) : nullptr;
    for (uint32_t k = 0; k < npk; ++k) {
      while (!ring_space()) {
        wait_vmcnt<0>();
        st_lds(&sm.filled, pos);
        if (!spin.again()) { dead = true; return; }
      }
      const uint32_t off = k * PKT + uint32_t(lane) * 16u;
      const uint8_t* src;
      if (kind == 1) {
        // 4 tokens per packet; per token 8 lanes of K (128 B) then 8 lanes of V.
        const int t = P.t0 + int(k) * 4 + (lane >> 4);
        const int piece = (lane >> 3) & 1;
        const int part = lane & 7;
        const int blk = sm.blk[t / 16 - P.t0 / 16];
        const long long e = (long long)blk * p.block_stride + (long long)(t & 15) * p.token_stride +
                            (long long)P.g * p.head_stride + (piece ? p.v_off : p.k_off) + part * 8;
        src = cache + e * 2;
      } else {
        src = base + off;
      }
      if (off < bytes) dma16(src, __builtin_amdgcn_readfirstlane(ring_base + (pos & (RING - 1))));
      pos += PKT;
      wait_vmcnt<DEPTH>();
      if (pos >= uint32_t(DEPTH) * PKT) st_lds(&sm.filled, pos - uint32_t(DEPTH) * PKT);
    }
  };
  for (int l = 0; l < p.n_layers && !dead; ++l) {
    for (int kind = 0; kind < SEGS_PER_LAYER && !dead; ++kind) issue_segment(kind, l, 0);
    if (lane == 0) trace_at(p, l, 15, p.n_layers);
  }
  for (int j = 0; j < P.n_lm && !dead; ++j) issue_segment(6, 0, j);
  wait_vmcnt<0>();
  st_lds(&sm.filled, pos);
}

// ------------------------------------------------------------------------------------------------
// Consumer waves
// ------------------------------------------------------------------------------------------------

template <class G>
struct Consumer {
  const Params& p;
  const Plan<G>& P;
  Smem<G>& sm;
  int cw, lane, ct;          // consumer wave, lane, consumer thread id
  uint32_t pos = 0;          // stream cursor (mirrors the producer)
  uint32_t bar_gen = 0;
  uint32_t epoch, tag16, tag32;
  bool dead = false;

  __device__ Consumer(const Params& p_, const Plan<G>& P_, Smem<G>& sm_, uint32_t ep)
      : p(p_), P(P_), sm(sm_) {
    cw = (threadIdx.x >> 6) - 1;
    lane = threadIdx.x & 63;
    ct = cw * 64 + lane;
    epoch = ep;
    tag32 = ep;
    tag16 = ((ep - 1u) % 65535u) + 1u;
  }

  // Claims the next segment of the stream; returns its start position.
  __device__ uint32_t next_seg(uint32_t bytes) {
    const uint32_t s = pos;
    pos += pad_pkt(bytes);
    return s;
  }
  __device__ void wait_filled(uint32_t end) {
    if (dead) return;
    Spin spin(p.ws, 2);
    while (ld_lds(&sm.filled) < end)
      if (!spin.again()) { dead = true; return; }
  }
  __device__ void release(uint32_t end) {
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): ring reads of this wave have returned
    if (lane == 0) st_lds(&sm.consumed[cw], end);
  }
  // Barrier over the NCW consumer waves.
  __device__ void cbar() {
    bar_gen += NCW;
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if (lane == 0) __hip_atomic_fetch_add(&sm.cbar, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    Spin spin(p.ws, 3);
    while (ld_lds(&sm.cbar) < bar_gen)
      if (!spin.again()) { dead = true; break; }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  }

  __device__ __forceinline__ uint4 ring16(uint32_t at) const {
    return *reinterpret_cast<const uint4*>(sm.ring + (at & (RING - 1)));
  }

  // Poll `n` tagged bf16 words at ws+off into sm.xs (as fp32); every consumer thread takes
  // 4-word groups.  Returns the wave-partial sum of squares (for RMSNorm) in every lane.
  __device__ void poll_vec(size_t off, int n, float* dst) {
    const uint32_t* src = p.ws + off;
    __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)src, (short)0, 0x7fffffff, 0x00020000);
    for (int i = ct * 4; i < n; i += NCT * 4) {
      Spin spin(p.ws, 4);
      while (true) {
        const uint32_t rem = uint32_t(n - i);
        uint32_t w0, w1, w2, w3;
        if (rem >= 4) {
          typedef uint32_t u4 __attribute__((ext_vector_type(4)));
          u4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, i * 4, 0, 16);
          w0 = v.x; w1 = v.y; w2 = v.z; w3 = v.w;
        } else {
          w0 = ld_dev(src + i);
          w1 = rem > 1 ? ld_dev(src + i + 1) : (tag16 << 16);
          w2 = rem > 2 ? ld_dev(src + i + 2) : (tag16 << 16);
          w3 = tag16 << 16;
        }
        if ((w0 >> 16) == tag16 && (w1 >> 16) == tag16 && (w2 >> 16) == tag16 && (w3 >> 16) == tag16) {
          dst[i] = bf2f(w0 & 0xffffu);
          if (rem > 1) dst[i + 1] = bf2f(w1 & 0xffffu);
          if (rem > 2) dst[i + 2] = bf2f(w2 & 0xffffu);
          if (rem > 3) dst[i + 3] = bf2f(w3 & 0xffffu);
          break;
        }
        if (dead || !spin.again()) { dead = true; break; }
      }
    }
  }

  // Sum of squares of dst[0..n) (fixed order), broadcast to all consumer lanes.  Ends with cbar.
  __device__ float sumsq(const float* v, int n) {
    float s = 0.f;
    for (int i = ct; i < n; i += NCT) s += v[i] * v[i];
    s = wave_sum(s);
    if (lane == 0) sm.red[cw] = s;
    cbar();
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < NCW; ++w) t += sm.red[w];
    return t;
  }

  __device__ __forceinline__ void put16(size_t off, float v) {
    st_dev(p.ws + off, (tag16 << 16) | f2bf(v));
  }
};

// x values (fp32) for the 16-byte chunks a lane owns: chunk j = lane + 64*c.
template <int K>
struct XRegs {
  static constexpr int CH = K / 8;
  static constexpr int CPL = (CH + 63) / 64;
  float v[CPL][8];
};

// Dot products of `nr` rows (held as 16-byte chunks per lane) with x; returns the wave-reduced
// sums in lane-independent registers.
template <int K, int MAXR>
__device__ __forceinline__ void dots(const uint4 (&w)[MAXR][XRegs<K>::CPL], const XRegs<K>& x, int nr,
                                     int lane, float (&out)[MAXR]) {
  constexpr int CPL = XRegs<K>::CPL;
  constexpr int CH = XRegs<K>::CH;
#pragma unroll
  for (int r = 0; r < MAXR; ++r) {
    float acc = 0.f;
    if (r < nr) {
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        if (lane + 64 * c < CH) {
          const uint32_t u[4] = {w[r][c].x, w[r][c].y, w[r][c].z, w[r][c].w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            acc = fmaf(bf2f(u[e] & 0xffffu), x.v[c][2 * e], acc);
            acc = fmaf(__uint_as_float(u[e] & 0xffff0000u), x.v[c][2 * e + 1], acc);
          }
        }
      }
    }
    out[r] = acc;
  }
#pragma unroll
  for (int r = 0; r < MAXR; ++r) out[r] = wave_sum(out[r]);
}

// Loads rows [first + cw + NCW*i] of a segment (row length K elements) into registers.
template <class G, int K, int MAXR>
__device__ __forceinline__ int pull(Consumer<G>& C, uint32_t seg_start, int nrows,
                                    uint4 (&w)[MAXR][XRegs<K>::CPL], int (&rows)[MAXR]) {
  constexpr int CPL = XRegs<K>::CPL;
  constexpr int CH = XRegs<K>::CH;
  int nr = 0;
#pragma unroll
  for (int r = 0; r < MAXR; ++r) {
    const int row = C.cw + NCW * r;
    rows[r] = row;
    if (row < nrows) {
      nr = r + 1;
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const int ch = C.lane + 64 * c;
        if (ch < CH) w[r][c] = C.ring16(seg_start + uint32_t(row) * K * 2 + uint32_t(ch) * 16);
      }
    }
  }
  return nr;
}

// Normalised x registers: xr = bf16(w * bf16(x * rs)) per element (LlamaRMSNorm rounding).
template <int K>
__device__ __forceinline__ void load_x(XRegs<K>& xr, const float* xs, int lane) {
  constexpr int CH = XRegs<K>::CH;
#pragma unroll
  for (int c = 0; c < XRegs<K>::CPL; ++c) {
    const int ch = lane + 64 * c;
#pragma unroll
    for (int e = 0; e < 8; ++e) xr.v[c][e] = ch < CH ? xs[ch * 8 + e] : 0.f;
  }
}
template <int K>
__device__ __forceinline__ void load_x_norm(XRegs<K>& xr, const float* xs, const uint16_t* w, float rs, int lane) {
  constexpr int CH = XRegs<K>::CH;
#pragma unroll
  for (int c = 0; c < XRegs<K>::CPL; ++c) {
    const int ch = lane + 64 * c;
    if (ch < CH) {
      const uint4 wv = *reinterpret_cast<const uint4*>(w + ch * 8);
      const uint32_t u[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xr.v[c][2 * e] = rnd(bf2f(u[e] & 0xffffu) * rnd(xs[ch * 8 + 2 * e] * rs));
        xr.v[c][2 * e + 1] = rnd(__uint_as_float(u[e] & 0xffff0000u) * rnd(xs[ch * 8 + 2 * e + 1] * rs));
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) xr.v[c][e] = 0.f;
    }
  }
}

__device__ __forceinline__ float rms_scale(float sumsq, int n) {
  const float mean = sumsq / float(n);
  return 1.0f / sqrtf(mean + 1e-5f);
}

// ---- phase bodies ------------------------------------------------------------------------------

// Rows per wave for each GEMV phase (ceil over the balanced split, then over NCW waves).
template <class G>
struct Rows {
  static constexpr int QKV = ((G::QKV + NWG - 1) / NWG + NCW - 1) / NCW;
  static constexpr int O = ((G::H + NWG - 1) / NWG + NCW - 1) / NCW;
  static constexpr int ACT = ((G::I + NWG - 1) / NWG + NCW - 1) / NCW;
  static constexpr int DOWN = ((G::H + NWG - 1) / NWG + NCW - 1) / NCW;
};

// P2 for one attention chunk (batch 1): RoPE on q (and the new k), scores over the ring-resident
// cached K plus the new token, fp32 softmax partial (m, l, o), then either a partial record
// (non-leader) or the log-sum-exp merge of all chunks of this KV head (leader), which also
// appends the new K/V to the paged cache (block360_kernel.inc:124-135).
template <class G>
__device__ void attention(Consumer<G>& C, int l, uint32_t seg) {
  const Params& p = C.p;
  const Plan<G>& P = C.P;
  Smem<G>& sm = C.sm;
  using W = WS<G>;
  const int b = 0, g = P.g, lane = C.lane;
  const int T_old = P.t1 - P.t0;
  const int T = T_old + (P.leader ? 1 : 0);
  constexpr int SCS = TC_MAX + 1;

  C.wait_filled(C.pos);
  C.poll_vec(W::qkv(l, b) + size_t(g) * 192, 192, sm.xs);
  if (P.leader) {
    C.poll_vec(W::qkv(l, b) + G::H + size_t(g) * 64, 64, sm.xs + 192);
    C.poll_vec(W::qkv(l, b) + G::H + G::KVH * 64 + size_t(g) * 64, 64, sm.xs + 256);
  }
  C.cbar();
  if (C.ct == 0) trace_at(p, l, 3, p.n_layers);
  // RoPE, HF rounding: bf16(bf16(x*cos) + bf16(rotate_half(x)*sin)) (modeling_llama.py:138-160)
  const int nrot = P.leader ? 256 : 192;
  for (int i = C.ct; i < nrot; i += NCT) {
    const int d = i & 63, base = i - d, f = d & 31;
    float c, s;
    if (p.cs_fp32) {
      const float* row = reinterpret_cast<const float*>(p.cos_sin) + size_t(P.pos) * 64;
      c = row[f];
      s = row[32 + f];
    } else {
      const uint16_t* row = reinterpret_cast<const uint16_t*>(p.cos_sin) + size_t(P.pos) * 64;
      c = bf2f(row[f]);
      s = bf2f(row[32 + f]);
    }
    const float x = sm.xs[i];
    const float rot = d < 32 ? -sm.xs[base + d + 32] : sm.xs[base + d - 32];
    const float r = rnd(rnd(x * c) + rnd(rot * s));
    if (i < 192) sm.qrot[i] = r;
    else sm.knew[d] = r;
  }
  if (P.leader)
    for (int i = C.ct; i < 64; i += NCT) sm.vnew[i] = sm.xs[256 + i];
  C.cbar();

  // scores: 8 lanes per token (8 dims each), 32 tokens per pass over the 4 consumer waves
  const int grp = C.cw * 8 + (lane >> 3);
  const int part = lane & 7;
  float q[3][8];
#pragma unroll
  for (int h = 0; h < 3; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) q[h][e] = sm.qrot[h * 64 + part * 8 + e];
  for (int j0 = 0; j0 < T; j0 += 32) {
    const int j = j0 + grp;
    float k8[8];
    if (j < T_old) {
      const uint4 kv = C.ring16(seg + uint32_t(j) * 256u + uint32_t(part) * 16u);
      const uint32_t u[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) { k8[2 * e] = bf2f(u[e] & 0xffffu); k8[2 * e + 1] = __uint_as_float(u[e] & 0xffff0000u); }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) k8[e] = j < T ? sm.knew[part * 8 + e] : 0.f;
    }
    float dd[3];
#pragma unroll
    for (int h = 0; h < 3; ++h) {
      float a = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) a = fmaf(q[h][e], k8[e], a);
      a += __shfl_xor(a, 1);
      a += __shfl_xor(a, 2);
      a += __shfl_xor(a, 4);
      dd[h] = a;
    }
    if (part == 0 && j < T)
#pragma unroll
      for (int h = 0; h < 3; ++h) sm.sc[h * SCS + j] = rnd(dd[h]) * 0.125f;
  }
  C.cbar();
  // per-head max and exp-sum (wave h handles head h)
  if (C.cw < 3) {
    const int h = C.cw;
    float m = -INFINITY;
    for (int j = lane; j < T; j += 64) m = fmaxf(m, sm.sc[h * SCS + j]);
    m = wave_max(m);
    float s = 0.f;
    for (int j = lane; j < T; j += 64) {
      const float e = expf(sm.sc[h * SCS + j] - m);
      sm.sc[h * SCS + j] = e;
      s += e;
    }
    s = wave_sum(s);
    if (lane == 0) { sm.ml[h] = m; sm.ml[4 + h] = s; }
  }
  C.cbar();
  // PV: acc[h][e] over this lane group's tokens
  float acc[3][8];
#pragma unroll
  for (int h = 0; h < 3; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;
  for (int j = grp; j < T; j += 32) {
    float v8[8];
    if (j < T_old) {
      const uint4 vv = C.ring16(seg + uint32_t(j) * 256u + 128u + uint32_t(part) * 16u);
      const uint32_t u[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) { v8[2 * e] = bf2f(u[e] & 0xffffu); v8[2 * e + 1] = __uint_as_float(u[e] & 0xffff0000u); }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v8[e] = sm.vnew[part * 8 + e];
    }
#pragma unroll
    for (int h = 0; h < 3; ++h) {
      const float pj = sm.sc[h * SCS + j];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[h][e] = fmaf(pj, v8[e], acc[h][e]);
    }
  }
#pragma unroll
  for (int h = 0; h < 3; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float a = acc[h][e];
      a += __shfl_xor(a, 8);
      a += __shfl_xor(a, 16);
      a += __shfl_xor(a, 32);
      acc[h][e] = a;
    }
  if (lane < 8)
#pragma unroll
    for (int h = 0; h < 3; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) sm.opart[(C.cw * 3 + h) * 64 + lane * 8 + e] = acc[h][e];
  C.cbar();
  if (C.ct == 0) trace_at(p, l, 4, p.n_layers);
  C.release(C.pos);  // K/V chunk no longer needed
  const int t = C.ct;
  float o_own = 0.f;
  if (t < 192) {
    const int h = t >> 6, d = t & 63;
#pragma unroll
    for (int w = 0; w < NCW; ++w) o_own += sm.opart[(w * 3 + h) * 64 + d];
  }
  uint64_t* rec_base = reinterpret_cast<uint64_t*>(p.ws + W::rec(l, 0));
  if (!P.leader) {
    uint64_t* rec = rec_base + size_t(P.wg) * REC_WORDS;
    const uint64_t tg = uint64_t(C.tag32) << 32;
    if (t < 192) {
      const int h = t >> 6, d = t & 63;
      st_dev64(rec + h * 66 + 2 + d, tg | __float_as_uint(o_own));
    } else if (t < 198) {
      const int h = (t - 192) >> 1, k = (t - 192) & 1;
      st_dev64(rec + h * 66 + k, tg | __float_as_uint(sm.ml[k * 4 + h]));
    }
    return;
  }
  // leader: online log-sum-exp merge in chunk order 0..C-1 (this chunk is C-1)
  if (t < 192) {
    const int h = t >> 6, d = t & 63;
    float M = -INFINITY, Ls = 0.f, O = 0.f;
    for (int c = 0; c < P.C; ++c) {
      float mc, lc, oc;
      if (c == P.C - 1) {
        mc = sm.ml[h];
        lc = sm.ml[4 + h];
        oc = o_own;
      } else {
        const uint64_t* rec = rec_base + size_t(g * P.C + c) * REC_WORDS + h * 66;
        uint64_t w0, w1, w2;
        Spin spin(p.ws, 5);
        while (true) {
          w0 = ld_dev64(rec);
          w1 = ld_dev64(rec + 1);
          w2 = ld_dev64(rec + 2 + d);
          if (uint32_t(w0 >> 32) == C.tag32 && uint32_t(w1 >> 32) == C.tag32 && uint32_t(w2 >> 32) == C.tag32) break;
          if (C.dead || !spin.again()) { C.dead = true; break; }
        }
        mc = __uint_as_float(uint32_t(w0));
        lc = __uint_as_float(uint32_t(w1));
        oc = __uint_as_float(uint32_t(w2));
      }
      const float Mn = fmaxf(M, mc);
      const float a = M == -INFINITY ? 0.f : expf(M - Mn);
      const float bsc = mc == -INFINITY ? 0.f : expf(mc - Mn);
      Ls = Ls * a + lc * bsc;
      O = O * a + oc * bsc;
      M = Mn;
    }
    C.put16(W::attn(l, b) + size_t(g * 3 + h) * 64 + d, O / Ls);
    if (t == 0) trace_at(p, l, 5, p.n_layers);
  }
  // append the new token's K (rotated) and V at slot_mapping[b]; slot < 0 skips
  const long long slot = p.slot_mapping[b];
  if (slot >= 0 && t < 128) {
    uint16_t* cache = reinterpret_cast<uint16_t*>(p.kv[l]);
    const long long blk = slot / 16, off = slot % 16;
    const long long e = blk * p.block_stride + off * p.token_stride + (long long)g * p.head_stride +
                        (t < 64 ? p.k_off : p.v_off) + (t & 63);
    cache[e] = uint16_t(f2bf(t < 64 ? sm.knew[t] : sm.vnew[t - 64]));
  }
}

template <class G>
__device__ void consumer(const Params& p, const Plan<G>& P, Smem<G>& sm, uint32_t epoch) {
  Consumer<G> C(p, P, sm, epoch);
  __builtin_amdgcn_s_barrier();  // pairs with the producer's barrier (blk[] ready)
  using W = WS<G>;
  const int lane = C.lane;
  const int b = 0;
  auto tr = [&](int l, int ev) { if (C.ct == 0) trace_at(p, l, ev, p.n_layers); };
  if (C.ct == 0 && p.trace)
    p.trace[size_t(blockIdx.x) * (size_t(p.n_layers) * TR_EVENTS + TR_TAIL) + size_t(p.n_layers) * TR_EVENTS] = wall_clock64();

  for (int l = 0; l < p.n_layers; ++l) {
    const LayerW Lw = p.layers[l];
    // ---------------- P1: RMSNorm(x) + QKV ----------------
    {
      const uint32_t seg = C.next_seg(seg_bytes(P, 0, 0));
      const int nrows = P.q1 - P.q0;
      C.wait_filled(seg + pad_pkt(seg_bytes(P, 0, 0)));
      tr(l, 0);
      uint4 w[Rows<G>::QKV][XRegs<G::H>::CPL];
      int rows[Rows<G>::QKV];
      const int nr = pull<G, G::H, Rows<G>::QKV>(C, seg, nrows, w, rows);
      C.release(C.pos);
      if (l == 0) {
        const long long id = p.ids_i64 ? reinterpret_cast<const int64_t*>(p.input_ids)[b]
                                       : reinterpret_cast<const int32_t*>(p.input_ids)[b];
        const uint16_t* e = p.embed + size_t(id) * G::H;
        for (int i = C.ct; i < G::H; i += NCT) sm.xs[i] = bf2f(e[i]);
      } else {
        C.poll_vec(W::x(l - 1, b), G::H, sm.xs);
      }
      C.cbar();
      tr(l, 1);
      for (int i = C.ct; i < G::H; i += NCT) sm.xkeep[i] = sm.xs[i];
      const float rs = rms_scale(C.sumsq(sm.xs, G::H), G::H);
      XRegs<G::H> xr;
      load_x_norm<G::H>(xr, sm.xs, Lw.norm1, rs, lane);
      float out[Rows<G>::QKV];
      dots<G::H, Rows<G>::QKV>(w, xr, nr, lane, out);
      if (lane == 0)
        for (int r = 0; r < nr; ++r) C.put16(W::qkv(l, b) + P.q0 + rows[r], rnd(out[r]));
      tr(l, 2);
    }
    // ---------------- P2: attention ----------------
    {
      const uint32_t seg = C.next_seg(seg_bytes(P, 1, 0));
      if (P.att) attention(C, l, seg);
    }
    // ---------------- P3: O + residual ----------------
    {
      const uint32_t seg = C.next_seg(seg_bytes(P, 2, 0));
      const int nrows = P.o1 - P.o0;
      C.wait_filled(C.pos);
      uint4 w[Rows<G>::O][XRegs<G::H>::CPL];
      int rows[Rows<G>::O];
      const int nr = pull<G, G::H, Rows<G>::O>(C, seg, nrows, w, rows);
      C.release(C.pos);
      tr(l, 6);
      C.poll_vec(W::attn(l, b), G::H, sm.xs);
      C.cbar();
      tr(l, 7);
      XRegs<G::H> xr;
      load_x<G::H>(xr, sm.xs, lane);
      float out[Rows<G>::O];
      dots<G::H, Rows<G>::O>(w, xr, nr, lane, out);
      if (lane == 0)
        for (int r = 0; r < nr; ++r) {
          const int row = P.o0 + rows[r];
          C.put16(W::h1(l, b) + row, sm.xkeep[row] + rnd(out[r]));
        }
      tr(l, 8);
    }
    // ---------------- P4: RMSNorm(h1) + gate/up + SwiGLU ----------------
    {
      const uint32_t segg = C.next_seg(seg_bytes(P, 3, 0));
      const uint32_t segu = C.next_seg(seg_bytes(P, 4, 0));
      const int na = P.a1 - P.a0;
      C.wait_filled(C.pos);
      uint4 wg[Rows<G>::ACT][XRegs<G::H>::CPL];
      uint4 wu[Rows<G>::ACT][XRegs<G::H>::CPL];
      int rows[Rows<G>::ACT];
      const int nr = pull<G, G::H, Rows<G>::ACT>(C, segg, na, wg, rows);
      pull<G, G::H, Rows<G>::ACT>(C, segu, na, wu, rows);
      C.release(C.pos);
      tr(l, 9);
      C.poll_vec(W::h1(l, b), G::H, sm.xs);
      C.cbar();
      tr(l, 10);
      for (int i = C.ct; i < G::H; i += NCT) sm.h1keep[i] = sm.xs[i];
      const float rs = rms_scale(C.sumsq(sm.xs, G::H), G::H);
      XRegs<G::H> xr;
      load_x_norm<G::H>(xr, sm.xs, Lw.norm2, rs, lane);
      float og[Rows<G>::ACT], ou[Rows<G>::ACT];
      dots<G::H, Rows<G>::ACT>(wg, xr, nr, lane, og);
      dots<G::H, Rows<G>::ACT>(wu, xr, nr, lane, ou);
      if (lane == 0)
        for (int r = 0; r < nr; ++r) {
          const float gv = rnd(og[r]), uv = rnd(ou[r]);
          const float silu = rnd(gv / (1.0f + expf(-gv)));
          C.put16(W::act(l, b) + P.a0 + rows[r], silu * uv);
        }
      tr(l, 11);
    }
    // ---------------- P5: down + residual ----------------
    {
      const uint32_t seg = C.next_seg(seg_bytes(P, 5, 0));
      const int nrows = P.d1 - P.d0;
      C.wait_filled(C.pos);
      uint4 w[Rows<G>::DOWN][XRegs<G::I>::CPL];
      int rows[Rows<G>::DOWN];
      const int nr = pull<G, G::I, Rows<G>::DOWN>(C, seg, nrows, w, rows);
      C.release(C.pos);
      tr(l, 12);
      C.poll_vec(W::act(l, b), G::I, sm.xs);
      C.cbar();
      tr(l, 13);
      XRegs<G::I> xr;
      load_x<G::I>(xr, sm.xs, lane);
      float out[Rows<G>::DOWN];
      dots<G::I, Rows<G>::DOWN>(w, xr, nr, lane, out);
      if (lane == 0)
        for (int r = 0; r < nr; ++r) {
          const int row = P.d0 + rows[r];
          const float y = rnd(sm.h1keep[row] + rnd(out[r]));
          C.put16(W::x(l, b) + row, y);
          if (p.layer_outputs) p.layer_outputs[(size_t(l) * p.B + b) * G::H + row] = uint16_t(f2bf(y));
        }
      tr(l, 14);
    }
  }
  // ---------------- final RMSNorm + LM head + argmax ----------------
  C.poll_vec(W::x(p.n_layers - 1, b), G::H, sm.xs);
  C.cbar();
  const float rs = rms_scale(C.sumsq(sm.xs, G::H), G::H);
  XRegs<G::H> xr;
  load_x_norm<G::H>(xr, sm.xs, p.final_norm, rs, lane);
  if (P.wg == 0) {
    // final-normed hidden state (the reference's out_hidden, block360_kernel.inc:810-815)
    for (int i = C.ct; i < G::H; i += NCT)
      p.out_hidden[size_t(b) * G::H + i] =
          uint16_t(f2bf(rnd(bf2f(p.final_norm[i]) * rnd(sm.xs[i] * rs))));
  }
  if (!p.lm_head) return;
  float best = -INFINITY;
  int best_i = 0x7fffffff;
  for (int j = 0; j < P.n_lm; ++j) {
    const uint32_t seg = C.next_seg(seg_bytes(P, 6, j));
    const int r0 = P.v0 + j * LM_ROWS;
    const int nrows = min(LM_ROWS, P.v1 - r0);
    C.wait_filled(C.pos);
    constexpr int MR = LM_ROWS / NCW;
    uint4 w[MR][XRegs<G::H>::CPL];
    int rows[MR];
    const int nr = pull<G, G::H, MR>(C, seg, nrows, w, rows);
    C.release(C.pos);
    float out[MR];
    dots<G::H, MR>(w, xr, nr, lane, out);
    for (int r = 0; r < nr; ++r) {
      const float v = rnd(out[r]);
      const int idx = r0 + rows[r];
      if (lane == 0 && p.out_logits) p.out_logits[size_t(b) * G::V + idx] = uint16_t(f2bf(v));
      if (v > best || (v == best && idx < best_i)) { best = v; best_i = idx; }
    }
  }
  if (lane == 0) { sm.lm_val[C.cw] = best; sm.lm_idx[C.cw] = best_i; }
  C.cbar();
  if (C.ct == 0 && p.trace)
    p.trace[size_t(blockIdx.x) * (size_t(p.n_layers) * TR_EVENTS + TR_TAIL) + size_t(p.n_layers) * TR_EVENTS + 1] = wall_clock64();
  if (C.ct == 0) {
    float bv = sm.lm_val[0];
    int bi = sm.lm_idx[0];
    for (int w = 1; w < NCW; ++w)
      if (sm.lm_val[w] > bv || (sm.lm_val[w] == bv && sm.lm_idx[w] < bi)) { bv = sm.lm_val[w]; bi = sm.lm_idx[w]; }
    const uint64_t rec = (uint64_t(C.tag32) << 32) | (uint64_t(uint32_t(bi) & 0xffffu) << 16) | f2bf(bv);
    st_dev64(reinterpret_cast<uint64_t*>(p.ws + W::lm(b, P.wg)), rec);
  }
  if (P.wg != 0) return;
  // workgroup 0: argmax over the NWG candidates (first index on ties, as torch.argmax)
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int q = C.ct; q < NWG; q += NCT) {
    const uint64_t* src = reinterpret_cast<const uint64_t*>(p.ws + W::lm(b, q));
    Spin spin(p.ws, 6);
    uint64_t r;
    while (true) {
      r = ld_dev64(src);
      if (uint32_t(r >> 32) == C.tag32) break;
      if (C.dead || !spin.again()) { C.dead = true; break; }
    }
    const float v = bf2f(uint32_t(r) & 0xffffu);
    const int i = int((uint32_t(r) >> 16) & 0xffffu);
    if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
  }
  if (lane == 0) { sm.lm_val[C.cw] = bv; sm.lm_idx[C.cw] = bi; }
  C.cbar();
  if (C.ct == 0) {
    bv = sm.lm_val[0];
    bi = sm.lm_idx[0];
    for (int w = 1; w < NCW; ++w)
      if (sm.lm_val[w] > bv || (sm.lm_val[w] == bv && sm.lm_idx[w] < bi)) { bv = sm.lm_val[w]; bi = sm.lm_idx[w]; }
    if (p.out_ids) p.out_ids[b] = bi;
  }
}

// ------------------------------------------------------------------------------------------------
// Kernel
// ------------------------------------------------------------------------------------------------

template <class G>
__global__ void __launch_bounds__(WG_THREADS, 1) decode_kernel(Params p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_raw[];
  Smem<G>& sm = *reinterpret_cast<Smem<G>*>(smem_raw);
  if (threadIdx.x == 0) {
    sm.filled = 0;
    for (int w = 0; w < NCW; ++w) sm.consumed[w] = 0;
    sm.cbar = 0;
  }
  __syncthreads();
  Plan<G> P;
  P.init(p, blockIdx.x);
  uint32_t epoch = ld_dev(p.ws + HDR_EPOCH) + 1u;
  if (epoch == 0) epoch = 1;
  if (threadIdx.x < 64) producer<G>(p, P, sm);
  else consumer<G>(p, P, sm, epoch);
  __syncthreads();
  if (blockIdx.x == 0 && threadIdx.x == 0) st_dev(p.ws + HDR_EPOCH, epoch);
}

template <class G>
constexpr size_t lds_bytes() { return sizeof(Smem<G>); }

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

template <class G>
static int launch(const Params& p, hipStream_t stream) {
  const DeviceInfo d = query_device();
  if (!d.ok) return d.status;
  if (!d.gfx950) return PK_ERR_ARCH;
  if (!d.coop) return PK_ERR_COOP;
  if (d.cus < NWG || size_t(d.max_lds) < lds_bytes<G>()) return PK_ERR_RESIDENCY;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(decode_kernel<G>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, int(lds_bytes<G>()));
  if (e != hipSuccess) return e;
  Params q = p;
  void* args[] = {&q};
  e = hipLaunchCooperativeKernel(reinterpret_cast<const void*>(decode_kernel<G>), dim3(NWG),
                                 dim3(WG_THREADS), args, lds_bytes<G>(), stream);
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
                       void* scratch, size_t scratch_bytes, int max_seq_len) {
  if (B != 1) return PK_ERR_BATCH;
  if (n_layers < 1 || n_layers > G::L) return PK_ERR_MODEL;
  if (max_seq_len < 1 || max_seq_len > kMaxSeq) return PK_ERR_MAX_SEQ;
  if (!input_ids || !embed || !final_norm || !positions || !seq_lens || !block_table ||
      !slot_mapping || !layers || !kv || !cos_sin || !out_hidden || !scratch)
    return PK_ERR_NULL;
  if (scratch_bytes < WS<G>::TOTAL * 4) return PK_ERR_SCRATCH;
  if (block_size != 16 || bt_stride < 1 || (long long)bt_stride * block_size < max_seq_len) return PK_ERR_BLOCK;
  if (k_off % 8 || v_off % 8 || block_stride % 8 || token_stride % 8 || head_stride % 8 || k_off < 0 ||
      v_off < 0 || block_stride < 0 || token_stride < 0 || head_stride < 0)
    return PK_ERR_ALIGN;
  auto mis = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) != 0; };
  if (mis(embed) || mis(final_norm) || mis(layers) || mis(kv) || mis(out_hidden) || mis(scratch) ||
      (layer_outputs && mis(layer_outputs)) || (out_logits && mis(out_logits)))
    return PK_ERR_ALIGN;
  Params p{};
  p.layers = reinterpret_cast<const LayerW*>(layers);
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
  p.trace = g_trace;
  return launch<G>(p, reinterpret_cast<hipStream_t>(stream));
}

}  // namespace pk

// ------------------------------------------------------------------------------------------------
// C ABI
// ------------------------------------------------------------------------------------------------

// Diagnostics: per-phase wall-clock timestamps for the next launches (NULL disables).
// Layout: [256 workgroups][n_layers * 16 + 4] uint64.
extern "C" void pk_set_trace(void* buf) { pk::g_trace = reinterpret_cast<unsigned long long*>(buf); }

extern "C" size_t pk_workspace_bytes(int model) {
  if (model == PK_MODEL_SMOLLM2_360M) return pk::WS<pk::G360>::TOTAL * 4;
  if (model == PK_MODEL_SMOLLM2_135M) return pk::WS<pk::G135>::TOTAL * 4;
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
    default: return hipGetErrorString(static_cast<hipError_t>(status));
  }
}

extern "C" size_t decode360_workspace_bytes(void) { return pk_workspace_bytes(PK_MODEL_SMOLLM2_360M); }
extern "C" size_t decode360_debug_bytes(void) { return 0; }
extern "C" const char* decode360_status_string(int status) { return prime_decode_status_string(status); }

extern "C" int decode360(void* stream, int B, const void* input_ids, const void* embed, const void* final_norm,
                         const void* positions, const void* seq_lens, const void* block_table, int bt_stride,
                         const void* slot_mapping, const void* layers, void* const* kv, long long k_off,
                         long long v_off, long long block_stride, long long token_stride, long long head_stride,
                         int block_size, const void* cos_sin, int cs_fp32, void* out_hidden, void* layer_outputs,
                         void* scratch, size_t scratch_bytes, void* debug, size_t debug_bytes, int max_seq_len,
                         int debug_layer_index) {
  (void)debug_bytes;
  if (debug_layer_index < -1 || debug_layer_index >= pk::G360::L) return PK_ERR_BLOCK;
  if (debug) return PK_ERR_DEBUG;
  return pk_decode(stream, PK_MODEL_SMOLLM2_360M, B, pk::G360::L, input_ids, 0, embed, final_norm, positions,
                   seq_lens, block_table, bt_stride, slot_mapping, layers, kv, k_off, v_off, block_stride,
                   token_stride, head_stride, block_size, cos_sin, cs_fp32, out_hidden, layer_outputs, nullptr,
                   nullptr, scratch, scratch_bytes, max_seq_len);
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
