// Lossless bf16 gate/up codec for gfx950: encode, decode and descriptor entry points of
// include/prime_lossless.h.  The format and its rules follow
// prime_kernels/lossless_bf16/csrc/lossless_bf16.cu:16-103 (see the header for the layout).
//
// Encoding is three launches on the caller's stream:
//   1. rows   one wave per row: 120 chunks over the 64 lanes (chunks l and l + 64), the plane
//             bytes, the header of every plain chunk, the escape flags, and the row's escape
//             count (ballots);
//   2. scan   one workgroup: exclusive scan of the 5,120 row counts -> row_offsets, and the
//             enabled flag (total <= capacity);
//   3. place  one wave per row again: each escaped chunk's ordinal is its row offset plus the
//             escapes before it in the row (a masked popcount of the ballots), which goes into its
//             header; its 8 words go to raw when the ordinal fits; prefix gets every chunk's
//             inclusive count.
// Only row counts cross workgroups, so no device-wide scan library is needed.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/prime_lossless.h"

namespace {

constexpr int kRows = 5120;
constexpr int kCols = 960;
constexpr int kChunk = 8;
constexpr int kChunksPerRow = kCols / kChunk;  // 120
constexpr int kChunks = kRows * kChunksPerRow;
constexpr int kWavesPerBlock = 4;
static_assert(kChunksPerRow <= 128, "two chunks per lane cover a row");

__device__ __forceinline__ uint64_t lanes_below(int lane) { return (uint64_t(1) << lane) - 1u; }

// Plane bytes and header of one chunk (8 words as a uint4 of packed pairs).
__device__ __forceinline__ bool encode_chunk(uint4 v, uint2& plane, uint32_t& header) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  uint32_t e[8], pb[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t lo = w[i] & 0xFFFFu, hi = w[i] >> 16;
    e[2 * i] = (lo >> 7) & 255u;
    e[2 * i + 1] = (hi >> 7) & 255u;
    pb[2 * i] = ((lo >> 8) & 0x80u) | (lo & 0x7Fu);
    pb[2 * i + 1] = ((hi >> 8) & 0x80u) | (hi & 0x7Fu);
  }
  uint32_t emin = e[0], emax = e[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) {
    emin = min(emin, e[i]);
    emax = max(emax, e[i]);
  }
  const bool escape = emin == 255u || emax - emin > 7u;
  uint32_t packed = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) packed |= (escape ? 0u : e[i] - emin) << (3 * i);
  plane.x = pb[0] | (pb[1] << 8) | (pb[2] << 16) | (pb[3] << 24);
  plane.y = pb[4] | (pb[5] << 8) | (pb[6] << 16) | (pb[7] << 24);
  header = escape ? 0xFF000000u : ((emin << 24) | packed);
  return escape;
}

__global__ void __launch_bounds__(64 * kWavesPerBlock) lz_rows(const uint4* input, uint2* plane, uint32_t* headers,
                                                               uint32_t* flags, uint32_t* row_counts) {
  const int row = blockIdx.x * kWavesPerBlock + int(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= kRows) return;
  bool esc[2] = {false, false};
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int c = lane + 64 * h;
    if (c < kChunksPerRow) {
      const size_t chunk = size_t(row) * kChunksPerRow + c;
      uint2 pl;
      uint32_t hd;
      esc[h] = encode_chunk(input[chunk], pl, hd);
      plane[chunk] = pl;
      headers[chunk] = hd;
      flags[chunk] = esc[h] ? 1u : 0u;
    }
  }
  const uint64_t b0 = __ballot(esc[0]), b1 = __ballot(esc[1]);
  if (lane == 0) row_counts[row] = uint32_t(__popcll(b0) + __popcll(b1));
}

// Exclusive scan of the row counts in one workgroup of 1024 threads (5 rows per thread).
__global__ void __launch_bounds__(1024) lz_scan(const uint32_t* row_counts, uint32_t* row_offsets,
                                                uint32_t* enabled, uint32_t capacity) {
  constexpr int kPer = (kRows + 1023) / 1024;
  __shared__ uint32_t wave_tot[16];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  uint32_t v[kPer], s = 0;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int r = t * kPer + i;
    v[i] = r < kRows ? row_counts[r] : 0u;
    s += v[i];
  }
  // inclusive scan of s over the wave
  uint32_t inc = s;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t u = __shfl_up(inc, o);
    if (lane >= o) inc += u;
  }
  if (lane == 63) wave_tot[wave] = inc;
  __syncthreads();
  uint32_t before = 0;
  for (int w = 0; w < wave; ++w) before += wave_tot[w];
  uint32_t run = before + inc - s;  // exclusive start of this thread's rows
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int r = t * kPer + i;
    if (r < kRows) row_offsets[r] = run;
    run += v[i];
  }
  if (t == 1023) {
    row_offsets[kRows] = run;
    *enabled = run <= capacity ? 1u : 0u;
  }
}

__global__ void __launch_bounds__(64 * kWavesPerBlock) lz_place(const uint4* input, const uint32_t* flags,
                                                                const uint32_t* row_offsets, uint32_t* headers,
                                                                uint32_t* prefix, uint4* raw, uint32_t capacity) {
  const int row = blockIdx.x * kWavesPerBlock + int(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= kRows) return;
  bool esc[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int c = lane + 64 * h;
    esc[h] = c < kChunksPerRow && flags[size_t(row) * kChunksPerRow + c] != 0u;
  }
  const uint64_t b0 = __ballot(esc[0]), b1 = __ballot(esc[1]);
  const uint32_t base = row_offsets[row];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int c = lane + 64 * h;
    if (c >= kChunksPerRow) continue;
    const size_t chunk = size_t(row) * kChunksPerRow + c;
    const uint32_t before = h == 0 ? uint32_t(__popcll(b0 & lanes_below(lane)))
                                   : uint32_t(__popcll(b0) + __popcll(b1 & lanes_below(lane)));
    prefix[chunk] = base + before + (esc[h] ? 1u : 0u);
    if (esc[h]) {
      const uint32_t ordinal = base + before;
      headers[chunk] = 0xFF000000u | ordinal;
      if (ordinal < capacity) raw[ordinal] = input[chunk];
    }
  }
}

// The 8 words of a chunk from its plane bytes and header (escape: its raw words).
__device__ __forceinline__ uint4 decode_chunk(uint2 p, uint32_t h, const uint4* raw) {
  if ((h >> 24) == 255u) return raw[h & 0xFFFFFFu];
  const uint32_t base2 = (h >> 24) * 0x10001u;
  uint32_t out[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t src = j < 2 ? p.x : p.y;
    // bytes 2(j&1) and 2(j&1)+1 of src into bits 0-7 and 16-23
    const uint32_t t = __builtin_amdgcn_perm(0u, src, (j & 1) ? 0x0c030c02u : 0x0c010c00u);
    const uint32_t d = (h >> (6 * j)) & 63u;
    const uint32_t ex = base2 + (d & 7u) + ((d >> 3) << 16);
    out[j] = ((t & 0x00800080u) << 8) | (t & 0x007F007Fu) | (ex << 7);
  }
  return make_uint4(out[0], out[1], out[2], out[3]);
}

__global__ void __launch_bounds__(256) lz_decode(const uint2* plane, const uint32_t* headers, const uint4* raw,
                                                 uint4* output) {
  const int chunk = blockIdx.x * 256 + threadIdx.x;
  if (chunk >= kChunks) return;
  output[chunk] = decode_chunk(plane[chunk], headers[chunk], raw);
}

__global__ void lz_descriptor(EncodedGULayer* table, int index, EncodedGULayer entry) {
  if (threadIdx.x == 0) table[index] = entry;
}

bool misaligned(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) != 0; }

}  // namespace

extern "C" size_t lossless_scan_workspace_bytes(void) { return size_t(kRows) * sizeof(uint32_t); }

extern "C" int lossless_encode_layer(const void* input, void* plane, void* headers, void* raw, void* row_offsets,
                                     void* flags, void* prefix, void* scan_workspace, size_t scan_workspace_bytes,
                                     void* enabled, uint32_t capacity, void* stream) {
  if (!input || !plane || !headers || !row_offsets || !flags || !prefix || !scan_workspace || !enabled ||
      (capacity > 0 && !raw))
    return 9103;  // PK_ERR_NULL
  if (scan_workspace_bytes < lossless_scan_workspace_bytes()) return 9108;  // PK_ERR_SCRATCH
  if (misaligned(input) || misaligned(plane) || misaligned(headers) || (raw && misaligned(raw)))
    return 9107;  // PK_ERR_ALIGN
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int blocks = kRows / kWavesPerBlock;
  auto* counts = static_cast<uint32_t*>(scan_workspace);
  lz_rows<<<blocks, 64 * kWavesPerBlock, 0, s>>>(static_cast<const uint4*>(input), static_cast<uint2*>(plane),
                                                 static_cast<uint32_t*>(headers), static_cast<uint32_t*>(flags),
                                                 counts);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  lz_scan<<<1, 1024, 0, s>>>(counts, static_cast<uint32_t*>(row_offsets), static_cast<uint32_t*>(enabled), capacity);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  lz_place<<<blocks, 64 * kWavesPerBlock, 0, s>>>(static_cast<const uint4*>(input),
                                                  static_cast<const uint32_t*>(flags),
                                                  static_cast<const uint32_t*>(row_offsets),
                                                  static_cast<uint32_t*>(headers), static_cast<uint32_t*>(prefix),
                                                  static_cast<uint4*>(raw), capacity);
  return hipGetLastError();
}

extern "C" int lossless_decode_layer(const void* plane, const void* headers, const void* raw, void* output,
                                     void* stream) {
  if (!plane || !headers || !raw || !output) return 9103;
  if (misaligned(plane) || misaligned(headers) || misaligned(raw) || misaligned(output)) return 9107;
  lz_decode<<<(kChunks + 255) / 256, 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      static_cast<const uint2*>(plane), static_cast<const uint32_t*>(headers), static_cast<const uint4*>(raw),
      static_cast<uint4*>(output));
  return hipGetLastError();
}

extern "C" int lossless_write_descriptor(void* table, int index, const void* plane, const void* headers,
                                         const void* raw, const void* row_offsets, const void* enabled,
                                         void* stream) {
  if (!table || index < 0) return 9103;
  const EncodedGULayer entry{static_cast<const uint8_t*>(plane), static_cast<const uint32_t*>(headers),
                             static_cast<const uint16_t*>(raw), static_cast<const uint32_t*>(row_offsets),
                             static_cast<const uint32_t*>(enabled)};
  lz_descriptor<<<1, 64, 0, reinterpret_cast<hipStream_t>(stream)>>>(static_cast<EncodedGULayer*>(table), index,
                                                                      entry);
  return hipGetLastError();
}
