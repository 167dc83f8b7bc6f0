// Token permute / unpermute by expert for gfx950.
//
// Row map (reference: make_row_id_map, L/triton_permute.py:283-393).  The
// destination of (token t, expert e) is row(e, t) = off_e + rank(e, t): the
// permuted buffer is expert-major and token-ascending.  For E <= 24 two
// launches (count, then rowmap_scan_emit_kernel, which derives each tile's
// offsets from the counts itself); else three:
//   count : one workgroup per 256-token tile; each wave ballots the 0/1 mask
//           of every expert and the per-tile counts go to a [B, E, tiles]
//           table (expert-major, so the global order is a linear scan);
//   scan  : one workgroup per batch does the exclusive prefix over that table
//           (it also yields group_sizes);
//   emit  : re-ballots the tile's mask, ranks each routed token inside its
//           wave with popcount, and writes the packed per-token entry in the
//           reference format (rows and experts in descending order, n_routed
//           last, the reference's stale values in columns [n, E)).
// No atomics are used, so the result is deterministic by construction.
// Short batches of a contiguous bool mask (T <= 4096, E <= 64: one apply's
// routing) take one launch instead (rowmap_fused_kernel): each workgroup
// counts the whole batch with 16-byte loads, then emits its own tile.
//
// Payload kernels move rows in 16-byte vectors: permute reads a token's row
// once and writes it to each of the token's slots; unpermute gathers the slots
// and reduces in fp32 registers.  The forward pair spreads (token, chunk)
// pairs over all lanes; the backward and k/v/lr kernels give one 64-lane wave
// to one token.
#include "common.h"

namespace uttt {
namespace {

constexpr int kTile = 256;         // tokens per row-map workgroup
constexpr int kMaxExperts = 128;   // row-map LDS tables are sized for this
constexpr int kTokPerBlock = 4;    // payload kernels: 4 waves = 4 tokens

template <int MB>
__device__ __forceinline__ bool mask_bit(const void* map, int64_t idx) {
  if constexpr (MB == 1) return reinterpret_cast<const uint8_t*>(map)[idx] != 0;
  return reinterpret_cast<const int32_t*>(map)[idx] != 0;
}

// Selection bits of one token (bit e of word e / 32).  `base` must address a
// real token (callers clamp the token index; `valid` masks the result), and
// experts past E re-read expert E-1: every load is then unconditional, so all
// loads of a 32-expert group are in flight before the first is used and a
// tile pays one memory latency per group.  (Loads under a per-lane condition
// would each be followed by a wait before the merge of the two paths.)
// NMAX: a compile-time bound on E (only that many loads are issued).
template <int MB, int NMAX = kMaxExperts>
__device__ __forceinline__ void load_mask_bits(const void* map, int64_t base, int64_t s_e, int E,
                                               bool valid, uint32_t bits[kMaxExperts / 32]) {
#pragma unroll
  for (int g = 0; g < kMaxExperts / 32; ++g) {
    bits[g] = 0u;
    if (32 * g < NMAX && 32 * g < E) {  // wave-uniform
      bool bv[32];
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        const int e = min(32 * g + i, E - 1);
        bv[i] = 32 * g + i < NMAX && mask_bit<MB>(map, base + (int64_t)e * s_e);
      }
#pragma unroll
      for (int i = 0; i < 32; ++i)
        bits[g] |= (uint32_t)(valid && 32 * g + i < E && bv[i]) << i;
    }
  }
}

__device__ __forceinline__ bool bit_of(const uint32_t bits[kMaxExperts / 32], int e) {
  const uint32_t w = e < 32 ? bits[0] : e < 64 ? bits[1] : e < 96 ? bits[2] : bits[3];
  return (w >> (e & 31)) & 1u;
}

// ------------------------------------------------------------ row map ------
// Per-wave expert counts of a tile (one ballot per expert), and the ballots
// themselves when `wmask` is given.  Lane i of pass h keeps the ballot of
// expert 64 h + i (a select, no branch per expert; the unrolled experts of a
// 32-bit word are independent, so their compares overlap), and the wave
// stores 64 experts at once.  NMAX < kMaxExperts: a compile-time bound on E;
// the ballots of all NMAX experts are taken (those past E are empty), which
// leaves no branch in the loop.
template <int NMAX = kMaxExperts>
__device__ __forceinline__ void wave_counts(const uint32_t bits[kMaxExperts / 32], int E,
                                            int (*wcnt)[kMaxExperts],
                                            uint64_t (*wmask)[kMaxExperts] = nullptr) {
  const int w = threadIdx.x / kWave, lane = lane_id();
#pragma unroll
  for (int h = 0; h < kMaxExperts / 64; ++h) {
    if (64 * h >= NMAX || 64 * h >= E) break;  // wave-uniform
    uint64_t mine = 0;
#pragma unroll
    for (int g2 = 0; g2 < 2; ++g2) {
      const int g = 2 * h + g2;
      const int ng = min(32, E - 32 * g);
      const uint32_t word = bits[g];
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        if (32 * g + i < NMAX && (NMAX < kMaxExperts || i < ng)) {
          const uint64_t bal = __ballot((word >> i) & 1u);
          mine = lane == 32 * g2 + i ? bal : mine;
        }
      }
    }
    const int e = 64 * h + lane;
    if (e < E) {
      wcnt[w][e] = __popcll(mine);
      if (wmask != nullptr) wmask[w][e] = mine;
    }
  }
}

// Experts per tile row of the tile-major count table: E rounded up to a power
// of two, at least 4 (so kTile % Ep == 0); the padding counts zero.
__host__ __device__ __forceinline__ int padded_experts(int E) {
  int p = 4;
  while (p < E) p <<= 1;
  return p;
}

// EP > 0: the count table is tile-major, [B, tiles, EP] with EP =
// padded_experts(E) (read by rowmap_scan_emit_kernel<MB, EP>), else
// expert-major, [B, E, tiles] (rowmap_scan_kernel).
template <int MB, int EP = 0>
__global__ __launch_bounds__(kTile) void rowmap_count_kernel(
    const void* map, int64_t s_b, int64_t s_e, int64_t s_t, int T, int E, int ntiles,
    int32_t* counts) {
  constexpr bool TM = EP > 0;
  constexpr int NMAX = TM ? EP : kMaxExperts;
  __shared__ int wcnt[kTile / kWave][kMaxExperts];
  const int tile = blockIdx.x, b = blockIdx.y;
  const int t = tile * kTile + threadIdx.x;
  const int64_t base = (int64_t)b * s_b + (int64_t)min(t, T - 1) * s_t;
  uint32_t bits[kMaxExperts / 32];
  load_mask_bits<MB, NMAX>(map, base, s_e, E, t < T, bits);
  wave_counts<NMAX>(bits, E, wcnt);
  __syncthreads();
  const int Ep = TM ? EP : E;
  for (int e = threadIdx.x; e < Ep; e += kTile) {
    int c = 0;
    if (e < E) {
#pragma unroll
      for (int i = 0; i < kTile / kWave; ++i) c += wcnt[i][e];
    }
    counts[TM ? ((int64_t)b * ntiles + tile) * Ep + e : ((int64_t)b * E + e) * ntiles + tile] = c;
  }
}

// Exclusive scan of counts[b] (E * ntiles entries, expert-major) in place.
constexpr int kScanThreads = 1024;
constexpr int kScanPer = 4;

__global__ __launch_bounds__(kScanThreads) void rowmap_scan_kernel(int32_t* counts, int E,
                                                                   int ntiles,
                                                                   int32_t* group_sizes) {
  __shared__ int wave_tot[kScanThreads / kWave];
  __shared__ int expert_start[kMaxExperts + 1];
  __shared__ int carry_s;
  const int b = blockIdx.x;
  const int n = E * ntiles;
  int32_t* c = counts + (int64_t)b * n;
  const int tid = threadIdx.x, w = tid / kWave, lane = lane_id();
  if (tid == 0) carry_s = 0;
  __syncthreads();
  for (int base = 0; base < n; base += kScanThreads * kScanPer) {
    int v[kScanPer];
    int sum = 0;
#pragma unroll
    for (int i = 0; i < kScanPer; ++i) {
      int idx = base + tid * kScanPer + i;
      v[i] = idx < n ? c[idx] : 0;
      sum += v[i];
    }
    // inclusive scan of per-thread sums across the wave
    int incl = sum;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      int o = __shfl_up(incl, d, kWave);
      if (lane >= d) incl += o;
    }
    if (lane == kWave - 1) wave_tot[w] = incl;
    __syncthreads();
    int wave_off = 0;
    for (int i = 0; i < w; ++i) wave_off += wave_tot[i];
    int block_tot = 0;
    for (int i = 0; i < kScanThreads / kWave; ++i) block_tot += wave_tot[i];
    int run = carry_s + wave_off + incl - sum;  // exclusive prefix of this thread
#pragma unroll
    for (int i = 0; i < kScanPer; ++i) {
      int idx = base + tid * kScanPer + i;
      if (idx < n) {
        c[idx] = run;
        if (idx % ntiles == 0) expert_start[idx / ntiles] = run;
      }
      run += v[i];
    }
    __syncthreads();
    if (tid == 0) carry_s += block_tot;
    __syncthreads();
  }
  if (tid == 0) expert_start[E] = carry_s;
  __syncthreads();
  if (group_sizes != nullptr) {
    for (int e = tid; e < E; e += kScanThreads)
      group_sizes[(int64_t)b * E + e] = expert_start[e + 1] - expert_start[e];
  }
}

// STAGE: the tile's packed entries (kTile x (2E+1) int32, contiguous in the
// output) are assembled in LDS and written out with consecutive lanes on
// consecutive words; without it each lane stores its own entry directly,
// which strides the lanes 4 * (2E+1) bytes apart.
constexpr int kStageMaxW = 57;  // STAGE: kTile * (2E+1) * 4 bytes plus the 6.5 KiB of tables <= 64 KiB

// Packed entries of one 256-token tile, given its tokens' selection bits, the
// per-wave counts (wcnt) and selection ballots (wmask) of the tile and each
// expert's first row for the tile (toff): rows and experts in descending
// order, n_routed last, the reference's stale values in columns [n, E) (the
// row where routed, else -1), zeros in [E + n, 2E).  Each lane walks only its
// own experts, so the cost per token is its n_routed, not E.  STAGE assembles
// the tile in LDS (`stage`, kTile * (2E+1) words) and writes it with
// consecutive lanes on consecutive words; without it each lane stores its own
// entry, which strides the lanes 4 * (2E+1) bytes apart.  WOFF: toff holds
// each wave's first row per expert ([kTile / kWave][kMaxExperts], flattened:
// the tile's offset plus the earlier waves' counts) instead of the tile's.
// src (batch b's [rows] array, or null): the inverse map, src[row] = token.
template <bool STAGE, bool COPY_OUT = STAGE, bool WOFF = false>
__device__ __forceinline__ void emit_tile(const uint32_t bits[kMaxExperts / 32], int T, int E,
                                          int tile, int b, const int (*wcnt)[kMaxExperts],
                                          const uint64_t (*wmask)[kMaxExperts], const int* toff,
                                          int32_t* stage, int32_t* row_id_map,
                                          int32_t* src = nullptr) {
  const int t = tile * kTile + threadIdx.x;
  const int w = threadIdx.x / kWave;
  const int n = __popc(bits[0]) + __popc(bits[1]) + __popc(bits[2]) + __popc(bits[3]);
  const int W = 2 * E + 1;
  int32_t* row = STAGE ? stage + threadIdx.x * W : row_id_map + ((int64_t)b * T + t) * W;
  if (t < T) {
    for (int c = n; c < E; ++c) row[c] = -1;  // stale columns; routed ones are set below
    for (int c = E + n; c < 2 * E; ++c) row[c] = 0;
    row[2 * E] = n;
    const uint64_t below = (1ull << lane_id()) - 1ull;
    int j = 0;
#pragma unroll
    for (int g = kMaxExperts / 32 - 1; g >= 0; --g) {
      uint32_t m = bits[g];
      while (m != 0u) {  // this token's experts, highest first
        const int hb = 31 - __clz(m);
        m &= ~(1u << hb);
        const int e = 32 * g + hb;
        int r;
        if constexpr (WOFF) {
          r = toff[w * kMaxExperts + e] + __popcll(wmask[w][e] & below);
        } else {
          r = toff[e] + __popcll(wmask[w][e] & below);
          for (int i = 0; i < w; ++i) r += wcnt[i][e];
        }
        row[j] = r;
        row[E + j] = e;
        ++j;
        if (e >= n) row[e] = r;
        if (src != nullptr) src[r] = t;
      }
    }
  }
  if constexpr (STAGE && COPY_OUT) {
    __syncthreads();
    const int nt = min(kTile, T - tile * kTile);
    int32_t* g = row_id_map + ((int64_t)b * T + (int64_t)tile * kTile) * W;
    for (int i = threadIdx.x; i < nt * W; i += kTile) g[i] = stage[i];
  }
}

template <int MB, bool STAGE>
__global__ __launch_bounds__(kTile) void rowmap_emit_kernel(
    const void* map, int64_t s_b, int64_t s_e, int64_t s_t, int T, int E, int ntiles,
    const int32_t* offsets, int32_t* row_id_map) {
  extern __shared__ int32_t stage[];
  __shared__ int wcnt[kTile / kWave][kMaxExperts];
  __shared__ uint64_t wmask[kTile / kWave][kMaxExperts];
  __shared__ int toff[kMaxExperts];
  const int tile = blockIdx.x, b = blockIdx.y;
  const int t = tile * kTile + threadIdx.x;
  const int64_t base = (int64_t)b * s_b + (int64_t)min(t, T - 1) * s_t;
  uint32_t bits[kMaxExperts / 32];
  load_mask_bits<MB>(map, base, s_e, E, t < T, bits);
  wave_counts(bits, E, wcnt, wmask);
  for (int e = threadIdx.x; e < E; e += kTile)
    toff[e] = offsets[((int64_t)b * E + e) * ntiles + tile];
  __syncthreads();
  emit_tile<STAGE>(bits, T, E, tile, b, wcnt, wmask, toff, stage, row_id_map);
}

// Scan and emit in one launch (after rowmap_count_kernel<MB, EP>: two
// launches for the row map), for E <= kScanEmitMaxE.  Every workgroup derives
// its own tile's offsets from the count table ([tiles, EP] ints of the batch,
// 16 KiB at T = 65536, E = 16).  EP is a power of two dividing kTile, so in a
// chunk of kTile tiles lane l reads the EP words q * kTile + l, all of expert
// l % EP, and sums them (and those of the tiles before this one) in
// registers; lane shuffles and a per-wave table reduce the sums per expert,
// and wave 0 scans the totals over the experts and leaves each wave's first
// row per expert for the emit.  The loads of the first chunk are issued
// together with the tile's mask loads (one memory latency).  Redundant over
// the workgroups, but it replaces the one-workgroup scan launch and the
// workspace round trip of the offsets.  E <= 24: the staged emit's
// kTile * (2E + 1) words plus the static tables stay within 64 KiB.
constexpr int kScanEmitMaxE = 24;

// One chunk of a batch's tile-major count table from word w0 on, consecutive
// lanes on consecutive words (cv[q] = word w0 + q * kTile + lane, q < EP);
// addresses are clamped into the table, so the loads are unconditional and
// all in flight before the first is used.
template <int EP>
__device__ __forceinline__ void load_count_chunk(const int32_t* cb, int w0, int nwords,
                                                 int cv[EP]) {
#pragma unroll
  for (int q = 0; q < EP; ++q) cv[q] = cb[min(w0 + q * kTile + (int)threadIdx.x, nwords - 1)];
}

// VEC (T % 4 == 0, 16-byte aligned row_id_map): the staged tile goes out in
// 16-byte stores (a tile's nt * (2E + 1) words are then a multiple of 4 and
// start 16-byte aligned).
template <int MB, int EP, bool VEC>
__global__ __launch_bounds__(kTile) void rowmap_scan_emit_kernel(
    const void* map, int64_t s_b, int64_t s_e, int64_t s_t, int T, int E, int ntiles,
    const int32_t* counts, int32_t* group_sizes, int32_t* row_id_map) {
  extern __shared__ int32_t stage[];  // kTile * (2E + 1) words
  __shared__ int wcnt[kTile / kWave][kMaxExperts];
  __shared__ uint64_t wmask[kTile / kWave][kMaxExperts];
  __shared__ int woff[kTile / kWave][kMaxExperts];
  __shared__ int red[2][kTile / kWave][EP];
  const int tile = blockIdx.x, b = blockIdx.y;
  const int t = tile * kTile + threadIdx.x;
  const int w = threadIdx.x / kWave, lane = lane_id();
  const int64_t base = (int64_t)b * s_b + (int64_t)min(t, T - 1) * s_t;
  const int32_t* cb = counts + (int64_t)b * ntiles * EP;
  const int nwords = ntiles * EP;
  int cv[EP];
  load_count_chunk<EP>(cb, 0, nwords, cv);
  uint32_t bits[kMaxExperts / 32];
  load_mask_bits<MB, EP>(map, base, s_e, E, t < T, bits);
  // word q of this lane: expert lane % EP of tile i0 + q * (kTile / EP) + jl
  constexpr int tpq = kTile / EP;
  const int jl = threadIdx.x / EP;
  int tot = 0, bef = 0;
  for (int i0 = 0; i0 < ntiles; i0 += kTile) {
    if (i0 > 0) load_count_chunk<EP>(cb, i0 * EP, nwords, cv);
#pragma unroll
    for (int q = 0; q < EP; ++q) {
      const int j = i0 + q * tpq + jl;
      const int c = j < ntiles ? cv[q] : 0;
      tot += c;
      bef += j < tile ? c : 0;
    }
  }
#pragma unroll
  for (int d = EP; d < kWave; d <<= 1) {  // lanes of one expert: equal lane % EP
    tot += __shfl_xor(tot, d, kWave);
    bef += __shfl_xor(bef, d, kWave);
  }
  if (lane < EP) {
    red[0][w][lane] = tot;
    red[1][w][lane] = bef;
  }
  wave_counts<EP>(bits, E, wcnt, wmask);
  __syncthreads();
  if (threadIdx.x < kWave) {  // wave 0: lane e holds expert e (padding experts count 0)
    const int e = threadIdx.x;
    int te = 0, be = 0;
    if (e < EP) {
#pragma unroll
      for (int i = 0; i < kTile / kWave; ++i) {
        te += red[0][i][e];
        be += red[1][i][e];
      }
    }
    int incl = te;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const int o = __shfl_up(incl, d, kWave);
      if (e >= d) incl += o;
    }
    if (e < E) {
      int r = incl - te + be;
#pragma unroll
      for (int i = 0; i < kTile / kWave; ++i) {
        woff[i][e] = r;
        r += wcnt[i][e];
      }
      if (group_sizes != nullptr && tile == 0) group_sizes[(int64_t)b * E + e] = te;
    }
  }
  __syncthreads();
  if constexpr (!VEC) {
    emit_tile<true, true, true>(bits, T, E, tile, b, wcnt, wmask, &woff[0][0], stage, row_id_map);
  } else {
    emit_tile<true, false, true>(bits, T, E, tile, b, wcnt, wmask, &woff[0][0], stage, nullptr);
    __syncthreads();
    const int nt = min(kTile, T - tile * kTile);
    const int nw4 = nt * (2 * E + 1) / 4;
    uint4* g = reinterpret_cast<uint4*>(row_id_map + ((int64_t)b * T + (int64_t)tile * kTile) *
                                                         (2 * E + 1));
    const uint4* sv = reinterpret_cast<const uint4*>(stage);
    for (int i = threadIdx.x; i < nw4; i += kTile) g[i] = sv[i];
  }
}

// One-launch row map for short batches of a contiguous bool mask (s_t = 1,
// T % 16 == 0, 16-byte aligned rows): T <= kFusedMaxTiles * kTile tokens and
// E <= kFusedMaxE.  Every workgroup counts the whole batch itself -- the mask
// is E * T bytes (64 KiB at T = 2048, E = 32) -- each (expert, 256-token tile)
// count by the 16 lanes of one DPP row with one 16-byte load each (summed by
// DPP adds), 16 pairs per round and 16 rounds of loads in flight together,
// so the count costs one memory latency per 256 pairs and a wave's loads
// cover 1 KiB of one expert's row; then it
// takes its tile's offsets from those counts and emits the tile staged in
// LDS, written out in 16-byte vectors.
// This replaces the count / scan / emit launches (and their workspace round
// trip) where the three launches' fixed costs dominate.
constexpr int kFusedMaxTiles = 16;
constexpr int kFusedMaxE = 64;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int d = kWave / 2; d > 0; d >>= 1) v += __shfl_xor(v, d, kWave);
  return v;
}

// Sum over each aligned group of 16 lanes (one DPP row), the total in every
// lane: four DPP adds (swap neighbours, swap pairs, mirror the 8-lane halves,
// mirror the row), no LDS round trip as a shuffle takes.
template <int CTRL>
__device__ __forceinline__ int dpp_i32(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}
__device__ __forceinline__ int row_sum16(int v) {
  v += dpp_i32<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v += dpp_i32<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v += dpp_i32<0x141>(v);  // row_half_mirror
  v += dpp_i32<0x140>(v);  // row_mirror
  return v;
}

__device__ __forceinline__ int nonzero_bytes(uint32_t w) {
  w |= w >> 4;
  w |= w >> 2;
  w |= w >> 1;
  return __popc(w & 0x01010101u);
}

// EB: a compile-time bound on E (16, 32 or 64): the mask loads and the
// ballots of the tile run over EB experts with no per-expert branch.
// part_bal (the router's per-block balance partials [B, nblk_r, E]) given,
// one more workgroup per batch (blockIdx.x == ntiles) sums them into bal_sum
// [B, E], beside the tiles: expert e by wave e % 4, lane l adding blocks l
// and l + 64, then a fixed-order wave sum.
template <int EB>
__global__ __launch_bounds__(kTile) void rowmap_fused_kernel(const uint8_t* __restrict__ map,
                                                             int64_t s_b, int64_t s_e, int T,
                                                             int E, int ntiles,
                                                             int32_t* group_sizes,
                                                             int32_t* row_id_map,
                                                             const float* __restrict__ part_bal,
                                                             int nblk_r, float* bal_sum,
                                                             int32_t* src_rows, int64_t src_sb) {
  __shared__ __attribute__((aligned(16))) int32_t stage[kTile * (2 * kFusedMaxE + 1)];
  __shared__ int cnt[kFusedMaxE][kFusedMaxTiles];
  __shared__ int wcnt[kTile / kWave][kMaxExperts];
  __shared__ uint64_t wmask[kTile / kWave][kMaxExperts];
  __shared__ int toff[kMaxExperts];
  const int tile = blockIdx.x, b = blockIdx.y;
  if (tile == ntiles) {  // the balance-sum workgroup (part_bal given)
    const int w = threadIdx.x / kWave, lane = lane_id();
    const float* pb = part_bal + (int64_t)b * nblk_r * E;
    constexpr int kPer = EB / (kTile / kWave);  // experts per wave
    float v[kPer][2];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {  // every load first, from clamped addresses
      const int e = min(w + (kTile / kWave) * u, E - 1);
#pragma unroll
      for (int h = 0; h < 2; ++h)
        v[u][h] = pb[(int64_t)min(lane + kWave * h, nblk_r - 1) * E + e];
    }
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int e = w + (kTile / kWave) * u;
      float x = lane < nblk_r ? v[u][0] : 0.0f;
      x += lane + kWave < nblk_r ? v[u][1] : 0.0f;
      x = wave_sum(x);
      if (lane == 0 && e < E) bal_sum[(int64_t)b * E + e] = x;
    }
    return;
  }
  const int t = tile * kTile + threadIdx.x;
  const uint8_t* mb = map + (int64_t)b * s_b;
  // this tile's bits first: their loads overlap the whole-batch count
  uint32_t bits[kMaxExperts / 32];
  load_mask_bits<1, EB>(mb, min(t, T - 1), s_e, E, t < T, bits);
  // whole-batch counts: pair q = (expert, tile) is read by a group of 16
  // lanes, one 16-token vector each (a wave reads 4 consecutive pairs: 1 KiB
  // of one expert's row), and summed across the group with shuffles; the
  // loads of kRounds rounds of 16 pairs go out together, from clamped
  // (always valid) addresses
  constexpr int kVecPerTile = kTile / 16;
  constexpr int kRounds = 16;
  const int nvec = T / 16, npairs = E * ntiles;
  const int grp = threadIdx.x / kVecPerTile, gl = threadIdx.x % kVecPerTile;
  // q / ntiles as a float product: exact here (q < 2^10, ntiles <= 16: the
  // product stays within 1e-4 of e + (i + 0.5) / ntiles)
  const float inv_nt = 1.0f / (float)ntiles;
  for (int q0 = 0; q0 < npairs; q0 += kRounds * (kTile / kVecPerTile)) {
    uint4 v[kRounds];
    int qe[kRounds], qi[kRounds];
#pragma unroll
    for (int r = 0; r < kRounds; ++r) {
      const int q = min(q0 + r * (kTile / kVecPerTile) + grp, npairs - 1);
      qe[r] = (int)(((float)q + 0.5f) * inv_nt);
      qi[r] = q - qe[r] * ntiles;
      v[r] = reinterpret_cast<const uint4*>(mb + (int64_t)qe[r] * s_e)[min(
          qi[r] * kVecPerTile + gl, nvec - 1)];
    }
#pragma unroll
    for (int r = 0; r < kRounds; ++r) {
      const int q = q0 + r * (kTile / kVecPerTile) + grp;
      const int e = qe[r], i = qi[r];
      const bool live = q < npairs && i * kVecPerTile + gl < nvec;
      int c = live ? nonzero_bytes(v[r].x) + nonzero_bytes(v[r].y) + nonzero_bytes(v[r].z) +
                         nonzero_bytes(v[r].w)
                   : 0;
      static_assert(kVecPerTile == 16, "one DPP row per pair");
      c = row_sum16(c);
      if (gl == 0 && q < npairs) cnt[e][i] = c;
    }
  }
  wave_counts<EB>(bits, E, wcnt, wmask);
  __syncthreads();
  // offsets of this tile: exclusive scan over experts of the totals (wave 0,
  // E <= 64 = one lane per expert) plus the expert's count in earlier tiles
  if (threadIdx.x < kWave) {
    const int e = threadIdx.x;
    int total = 0, before = 0;
    if (e < E) {
#pragma unroll
      for (int i = 0; i < kFusedMaxTiles; ++i) {  // all reads in flight together
        const int c = i < ntiles ? cnt[e][i] : 0;
        total += c;
        before += i < tile ? c : 0;
      }
    }
    int incl = total;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const int o = __shfl_up(incl, d, kWave);
      if (e >= d) incl += o;
    }
    if (e < E) {
      toff[e] = incl - total + before;
      if (group_sizes != nullptr && tile == 0) group_sizes[(int64_t)b * E + e] = total;
    }
  }
  __syncthreads();
  emit_tile<true, false>(bits, T, E, tile, b, wcnt, wmask, toff, stage, nullptr,
                         src_rows != nullptr ? src_rows + b * src_sb : nullptr);
  __syncthreads();
  // the tile's entries are nt * (2E+1) words, a multiple of 4 (nt % 16 == 0),
  // and start 16-byte aligned (T % 16 == 0, aligned output)
  const int nt = min(kTile, T - tile * kTile);
  const int nw4 = nt * (2 * E + 1) / 4;
  uint4* g = reinterpret_cast<uint4*>(row_id_map + ((int64_t)b * T + (int64_t)tile * kTile) *
                                                       (2 * E + 1));
  const uint4* sv = reinterpret_cast<const uint4*>(stage);
  for (int i = threadIdx.x; i < nw4; i += kTile) g[i] = sv[i];
}

// ---------------------------------------------------------- vector copy ----
template <int VB>
struct Vec;
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
template <>
struct Vec<16> { using T = u32x4_t; };
template <>
struct Vec<8> { using T = u32x2_t; };
template <>
struct Vec<4> { using T = uint32_t; };
template <>
struct Vec<2> { using T = uint16_t; };

// Largest of 16/8/4/2 dividing the row size and the base addresses.
inline int pick_vec_bytes(int64_t row_bytes, std::initializer_list<const void*> ptrs) {
  for (int vb : {16, 8, 4, 2}) {
    bool ok = (row_bytes % vb) == 0;
    for (const void* p : ptrs) ok = ok && ((reinterpret_cast<uintptr_t>(p) % vb) == 0);
    if (ok) return vb;
  }
  return 1;
}

__device__ __forceinline__ int64_t tok_index(int b, int t, int T) { return (int64_t)b * T + t; }

// ------------------------------------------------- chunked payload kernels --
// The hot permute / unpermute kernels spread the flat (token, chunk) space of
// the payload over all lanes: thread i handles the 16-byte chunks
// base + u * 256 (u < CU) of the flattened B*T x CH grid, so every lane moves
// full vectors whatever the row length.  A thread issues all its independent
// loads first -- the payload chunk and the row-map entries of slots 0 and 1,
// then the probs, then (unpermute) the gathered rows -- so the dependent chain
// row map -> probs -> payload costs one memory latency per level rather than
// one per slot.  Slots past the first two (top-k > 2) take a plain loop.  The
// row-map entries of a token are re-read by its CH chunk threads and hit in
// cache.  Payload rows are read once and outputs written once, so both move
// with non-temporal loads and stores (measured: permute 55.4 -> 54.2 us,
// unpermute 58.0 -> 53.7 us at the configs[2] shape).
constexpr int kCT = 256;     // threads per workgroup
constexpr int kCU = 2;       // chunks per thread
constexpr bool kNT = true;   // non-temporal payload stores

template <bool NT, class V>
__device__ __forceinline__ void store_vec(V* p, const V& v) {
  if constexpr (NT) {
    __builtin_nontemporal_store(v, p);
  } else {
    *p = v;
  }
}

// Row-map entries of slots 0 and 1.  Columns [n, E) of the expert half hold
// 0 and, for E == 1, column E + 1 is the count: the expert index of a slot
// that is not routed is forced to 0 so that it addresses a valid probs entry.
// The raw words are loaded first and decoded after every chunk's loads are
// issued: a decode next to its load would wait for it there.
struct Slots2 {
  int n, r0, r1, e0, e1;
};
struct SlotsRaw {
  int4 w;  // {row 0, row 1, expert 0, n}
  int e1;  // expert of slot 1
};
__device__ __forceinline__ SlotsRaw load_slots_raw(const int32_t* __restrict__ rm, int E) {
  SlotsRaw r;
  r.w = make_int4(rm[0], rm[1], rm[E], rm[2 * E]);
  r.e1 = rm[E + 1];
  return r;
}
__device__ __forceinline__ Slots2 decode_slots(const SlotsRaw& r) {
  Slots2 s;
  s.r0 = r.w.x;
  s.r1 = r.w.y;
  s.n = r.w.w;
  s.e0 = s.n < 1 ? 0 : r.w.z;
  s.e1 = s.n < 2 ? 0 : r.e1;
  return s;
}

// The gates of slots 0 and 1 (1 without probs), loaded unconditionally: a
// missing probs tensor reads word 0 of the row map and the value is replaced,
// so no load sits under a branch (the compiler waits for a load under a branch
// where the paths join, and with it for every access in flight).
template <int CU>
__device__ __forceinline__ void gate_pair(const float* __restrict__ probs,
                                          const int32_t* __restrict__ rmap, int64_t p_sb,
                                          int64_t p_se, int64_t p_st, int T, const uint32_t (&bt)[CU],
                                          const Slots2 (&s)[CU], float (&p0)[CU], float (&p1)[CU]) {
  const bool has = probs != nullptr;
  const float* pbase = has ? probs : reinterpret_cast<const float*>(rmap);
  const int64_t sb = has ? p_sb : 0, se = has ? p_se : 0, stt = has ? p_st : 0;
#pragma unroll
  for (int u = 0; u < CU; ++u) {
    const int b = (int)(bt[u] / (uint32_t)T), t = (int)(bt[u] - (uint32_t)b * T);
    const float* pb = pbase + b * sb + (int64_t)t * stt;
    const float a0 = pb[(int64_t)s[u].e0 * se];
    const float a1 = pb[(int64_t)s[u].e1 * se];
    p0[u] = has ? a0 : 1.0f;
    p1[u] = has ? a1 : 1.0f;
  }
}

template <int VB, int CU, bool NT>
__global__ __launch_bounds__(kCT) void permute_chunk_kernel(
    const uint8_t* __restrict__ inp, int64_t row_bytes, int CH, int BT, int T,
    const int32_t* __restrict__ rmap, int E, const float* __restrict__ probs, int64_t p_sb,
    int64_t p_se, int64_t p_st, uint8_t* __restrict__ out, int num_out,
    float* __restrict__ pprobs) {
  using V = typename Vec<VB>::T;
  const uint32_t total = (uint32_t)BT * (uint32_t)CH;
  const uint32_t base = blockIdx.x * (kCT * CU) + threadIdx.x;
  V v[CU];
  SlotsRaw raw[CU];
  Slots2 s[CU];
  uint32_t bt[CU], c[CU];
#pragma unroll
  for (int u = 0; u < CU; ++u) {
    const uint32_t idx = base + u * kCT;
    const uint32_t q = idx < total ? idx : total - 1;  // dead lanes re-read the last chunk
    bt[u] = q / (uint32_t)CH;
    c[u] = q - bt[u] * (uint32_t)CH;
    raw[u] = load_slots_raw(rmap + (int64_t)bt[u] * (2 * E + 1), E);
    v[u] = __builtin_nontemporal_load(
        reinterpret_cast<const V*>(inp + (int64_t)bt[u] * row_bytes + (int64_t)c[u] * VB));
  }
  // every chunk's first-level loads issue before any of their values is used
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int u = 0; u < CU; ++u) s[u] = decode_slots(raw[u]);
  float p0[CU], p1[CU];
  gate_pair<CU>(probs, rmap, p_sb, p_se, p_st, T, bt, s, p0, p1);
  // The rows of slots 0 and 1, taken in straight-line code once every load is
  // in flight: the empty asm defines them here, so neither they nor their
  // loads can sink into the per-lane store branches below (a load sunk there
  // would issue only after the previous chunk's stores).
  const bool has = probs != nullptr;
  V o0[CU], o1[CU];
#pragma unroll
  for (int u = 0; u < CU; ++u) {
    o0[u] = has && p0[u] == 0.0f ? V{} : v[u];
    o1[u] = has && p1[u] == 0.0f ? V{} : v[u];
    asm volatile("" : "+v"(o0[u]), "+v"(o1[u]));
  }
#pragma unroll
  for (int u = 0; u < CU; ++u) {
    if (base + u * kCT >= total) continue;
    const int b = (int)(bt[u] / (uint32_t)T), t = (int)(bt[u] - (uint32_t)b * T);
    uint8_t* dst_b = out + (int64_t)b * num_out * row_bytes + (int64_t)c[u] * VB;
    auto put = [&](int row, float pr, const V& o) __attribute__((always_inline)) {
      if (row < 0 || row >= num_out) return;
      if (has && c[u] == 0) pprobs[(int64_t)b * num_out + row] = pr;
      store_vec<NT>(reinterpret_cast<V*>(dst_b + (int64_t)row * row_bytes), o);
    };
    const int n = s[u].n;
    if (n > 0) put(s[u].r0, p0[u], o0[u]);
    if (n > 1) put(s[u].r1, p1[u], o1[u]);
    const int32_t* rm = rmap + (int64_t)bt[u] * (2 * E + 1);
    for (int j = 2; j < n; ++j) {
      const float pr =
          has ? probs[b * p_sb + (int64_t)rm[E + j] * p_se + (int64_t)t * p_st] : 1.0f;
      put(rm[j], pr, has && pr == 0.0f ? V{} : v[u]);
    }
  }
}

// out[t] = cast(sum_j fp32(y[row_j]) * p_j) in slot order (fma, one rounding
// per slot); without probs the plain sum in slot order.
template <class TT, int VE, int CU, bool NT>
__global__ __launch_bounds__(kCT) void unpermute_chunk_kernel(
    const typename TT::S* __restrict__ inp, int H, int CH, int BT, int T, int num_out,
    const int32_t* __restrict__ rmap, int E, const float* __restrict__ probs, int64_t p_sb,
    int64_t p_se, int64_t p_st, typename TT::S* __restrict__ out) {
  using S = typename TT::S;
  using VO = typename Vec<(int)sizeof(S) * VE>::T;
  const uint32_t total = (uint32_t)BT * (uint32_t)CH;
  const uint32_t base = blockIdx.x * (kCT * CU) + threadIdx.x;
  SlotsRaw raw[CU];
  Slots2 s[CU];
  uint32_t bt[CU], c[CU];
#pragma unroll
  for (int u = 0; u < CU; ++u) {
    const uint32_t idx = base + u * kCT;
    const uint32_t q = idx < total ? idx : total - 1;
    bt[u] = q / (uint32_t)CH;
    c[u] = q - bt[u] * (uint32_t)CH;
    raw[u] = load_slots_raw(rmap + (int64_t)bt[u] * (2 * E + 1), E);
  }
  // every chunk's slot loads issue before any is used
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int u = 0; u < CU; ++u) s[u] = decode_slots(raw[u]);
  float p0[CU], p1[CU];
  VO x0[CU], x1[CU];
  bool ok0[CU], ok1[CU];
  gate_pair<CU>(probs, rmap, p_sb, p_se, p_st, T, bt, s, p0, p1);
#pragma unroll
  for (int u = 0; u < CU; ++u) {
    const int b = (int)(bt[u] / (uint32_t)T);
    const S* src_b = inp + (int64_t)b * num_out * H + (int64_t)c[u] * VE;
    ok0[u] = s[u].n > 0 && s[u].r0 >= 0 && s[u].r0 < num_out;
    ok1[u] = s[u].n > 1 && s[u].r1 >= 0 && s[u].r1 < num_out;
    // both gathers from valid rows (row 0 for an empty slot; num_out >= 1 is
    // checked on the host) and unconditional, so they are in flight together
    x0[u] = __builtin_nontemporal_load(
        reinterpret_cast<const VO*>(src_b + (int64_t)(ok0[u] ? s[u].r0 : 0) * H));
    x1[u] = __builtin_nontemporal_load(
        reinterpret_cast<const VO*>(src_b + (int64_t)(ok1[u] ? s[u].r1 : 0) * H));
  }
#pragma unroll
  for (int u = 0; u < CU; ++u) {
    if (base + u * kCT >= total) continue;
    float acc[VE];
#pragma unroll
    for (int i = 0; i < VE; ++i) acc[i] = 0.0f;
    auto add = [&](const VO& raw, float pr) __attribute__((always_inline)) {
      S e[VE];
      __builtin_memcpy(e, &raw, sizeof(e));
      if (probs != nullptr) {
#pragma unroll
        for (int i = 0; i < VE; ++i) acc[i] = __builtin_fmaf(TT::load(e[i]), pr, acc[i]);
      } else {
#pragma unroll
        for (int i = 0; i < VE; ++i) acc[i] += TT::load(e[i]);
      }
    };
    if (ok0[u]) add(x0[u], p0[u]);
    if (ok1[u]) add(x1[u], p1[u]);
    const int n = s[u].n;
    if (n > 2) {
      const int b = (int)(bt[u] / (uint32_t)T), t = (int)(bt[u] - (uint32_t)b * T);
      const int32_t* rm = rmap + (int64_t)bt[u] * (2 * E + 1);
      const S* src_b = inp + (int64_t)b * num_out * H + (int64_t)c[u] * VE;
      for (int j = 2; j < n; ++j) {
        const int row = rm[j];
        if (row < 0 || row >= num_out) continue;
        const float pr =
            probs != nullptr ? probs[b * p_sb + (int64_t)rm[E + j] * p_se + (int64_t)t * p_st]
                             : 1.0f;
        add(*reinterpret_cast<const VO*>(src_b + (int64_t)row * H), pr);
      }
    }
    S o[VE];
#pragma unroll
    for (int i = 0; i < VE; ++i) o[i] = TT::store(acc[i]);
    VO ov;
    __builtin_memcpy(&ov, o, sizeof(ov));
    store_vec<NT>(reinterpret_cast<VO*>(out + (int64_t)bt[u] * H + (int64_t)c[u] * VE), ov);
  }
}

// --------------------------------------------------------------- permute ---
template <int VB>
__global__ __launch_bounds__(kTokPerBlock* kWave) void permute_fwd_kernel(
    const uint8_t* __restrict__ inp, int64_t row_bytes, int T, const int32_t* __restrict__ rmap,
    int E, const float* __restrict__ probs, int64_t p_sb, int64_t p_se, int64_t p_st,
    uint8_t* __restrict__ out, int num_out, float* __restrict__ pprobs) {
  using V = typename Vec<VB>::T;
  const int t = blockIdx.x * kTokPerBlock + threadIdx.x / kWave;
  const int b = blockIdx.y;
  if (t >= T) return;
  const int lane = lane_id();
  const int32_t* rm = rmap + tok_index(b, t, T) * (2 * E + 1);
  const int n = rm[2 * E];
  if (probs != nullptr && lane < n && lane < kWave) {
    for (int j = lane; j < n; j += kWave) {
      const int row = rm[j];
      const int e = rm[E + j];
      if (row >= 0 && row < num_out)
        pprobs[(int64_t)b * num_out + row] = probs[b * p_sb + e * p_se + t * p_st];
    }
  }
  const uint8_t* src = inp + tok_index(b, t, T) * row_bytes;
  uint8_t* dst_b = out + (int64_t)b * num_out * row_bytes;
  for (int64_t off = (int64_t)lane * VB; off < row_bytes; off += (int64_t)kWave * VB) {
    const V v = *reinterpret_cast<const V*>(src + off);
    for (int j = 0; j < n; ++j) {
      const int row = rm[j];
      if (row < 0 || row >= num_out) continue;
      V o = v;
      if (probs != nullptr) {
        const int e = rm[E + j];
        if (probs[b * p_sb + e * p_se + t * p_st] == 0.0f) o = V{};
      }
      *reinterpret_cast<V*>(dst_b + (int64_t)row * row_bytes + off) = o;
    }
  }
}

// grad_inp[t] = sum_j grad_out[row_j], fp32 in slot order.
template <class TT, int VE>
__global__ __launch_bounds__(kTokPerBlock* kWave) void permute_bwd_kernel(
    const typename TT::S* __restrict__ gout, int H, int T, const int32_t* __restrict__ rmap,
    int E, int num_out, const float* __restrict__ gpp, typename TT::S* __restrict__ ginp,
    float* __restrict__ gprobs) {
  using S = typename TT::S;
  const int t = blockIdx.x * kTokPerBlock + threadIdx.x / kWave;
  const int b = blockIdx.y;
  if (t >= T) return;
  const int lane = lane_id();
  const int32_t* rm = rmap + tok_index(b, t, T) * (2 * E + 1);
  const int n = rm[2 * E];
  for (int h0 = lane * VE; h0 < H; h0 += kWave * VE) {
    float acc[VE];
#pragma unroll
    for (int i = 0; i < VE; ++i) acc[i] = 0.0f;
    for (int j = 0; j < n; ++j) {
      const int row = rm[j];
      if (row < 0 || row >= num_out) continue;
      const S* src = gout + ((int64_t)b * num_out + row) * H + h0;
#pragma unroll
      for (int i = 0; i < VE; ++i) acc[i] += TT::load(src[i]);
    }
    S* dst = ginp + tok_index(b, t, T) * H + h0;
#pragma unroll
    for (int i = 0; i < VE; ++i) dst[i] = TT::store(acc[i]);
  }
  if (gprobs != nullptr) {
    for (int e = lane; e < E; e += kWave) {
      float val = 0.0f;
      for (int j = 0; j < n; ++j) {
        const int row = rm[j];
        if (rm[E + j] == e && row >= 0 && row < num_out) val = gpp[(int64_t)b * num_out + row];
      }
      gprobs[((int64_t)b * E + e) * T + t] = val;
    }
  }
}

// ------------------------------------------------------------- unpermute ---

template <class TT, int VE>
__global__ __launch_bounds__(kTokPerBlock* kWave) void unpermute_bwd_kernel(
    const typename TT::S* __restrict__ gout, const typename TT::S* __restrict__ fwd_inp, int H,
    int T, const int32_t* __restrict__ rmap, int E, int num_out, const float* __restrict__ probs,
    int64_t p_sb, int64_t p_se, int64_t p_st, typename TT::S* __restrict__ ginp,
    float* __restrict__ gprobs, int64_t g_sb, int64_t g_se, int64_t g_st) {
  using S = typename TT::S;
  const int t = blockIdx.x * kTokPerBlock + threadIdx.x / kWave;
  const int b = blockIdx.y;
  if (t >= T) return;
  const int lane = lane_id();
  const int32_t* rm = rmap + tok_index(b, t, T) * (2 * E + 1);
  const int n = rm[2 * E];
  // experts that are not routed get a zero gradient
  for (int e = lane; e < E; e += kWave) {
    bool routed = false;
    for (int j = 0; j < n; ++j) routed = routed || (rm[E + j] == e);
    if (!routed) gprobs[b * g_sb + (int64_t)e * g_se + (int64_t)t * g_st] = 0.0f;
  }
  const S* g = gout + tok_index(b, t, T) * H;
  for (int j = 0; j < n; ++j) {
    const int row = rm[j];
    const int e = rm[E + j];
    if (row < 0 || row >= num_out) continue;
    const float p = probs[b * p_sb + (int64_t)e * p_se + (int64_t)t * p_st];
    const S* y = fwd_inp + ((int64_t)b * num_out + row) * H;
    S* gi = ginp + ((int64_t)b * num_out + row) * H;
    float dot = 0.0f;
    for (int h0 = lane * VE; h0 < H; h0 += kWave * VE) {
#pragma unroll
      for (int i = 0; i < VE; ++i) {
        const float gv = TT::load(g[h0 + i]);
        gi[h0 + i] = TT::store(gv * p);
        dot = __builtin_fmaf(TT::load(y[h0 + i]), gv, dot);
      }
    }
    dot = wave_sum(dot);
    if (lane == 0) gprobs[b * g_sb + (int64_t)e * g_se + (int64_t)t * g_st] = dot;
  }
}

// ------------------------------------------------------ permute k, v, lr ---
template <class KT, class VT, int VE>
__global__ __launch_bounds__(kTokPerBlock* kWave) void permute_kv_fwd_kernel(
    const typename KT::S* __restrict__ k, const typename VT::S* __restrict__ v,
    const uint8_t* __restrict__ lr0, const uint8_t* __restrict__ lr1,
    const uint8_t* __restrict__ lr2, int lr_bytes, int H, int T,
    const int32_t* __restrict__ rmap, int E, const float* __restrict__ probs, int64_t p_sb,
    int64_t p_se, int64_t p_st, typename KT::S* __restrict__ k_out,
    typename KT::S* __restrict__ v_out, uint8_t* __restrict__ lr0_out,
    uint8_t* __restrict__ lr1_out, uint8_t* __restrict__ lr2_out, int num_out) {
  using SK = typename KT::S;
  using SV = typename VT::S;
  const int t = blockIdx.x * kTokPerBlock + threadIdx.x / kWave;
  const int b = blockIdx.y;
  if (t >= T) return;
  const int lane = lane_id();
  const int32_t* rm = rmap + tok_index(b, t, T) * (2 * E + 1);
  const int n = rm[2 * E];
  // per-token learning rates: plain copies, one lane per slot
  for (int j = lane; j < n; j += kWave) {
    const int row = rm[j];
    if (row < 0 || row >= num_out) continue;
    const int64_t src = tok_index(b, t, T) * lr_bytes;
    const int64_t dst = ((int64_t)b * num_out + row) * lr_bytes;
    if (lr_bytes == 4) {
      *reinterpret_cast<uint32_t*>(lr0_out + dst) = *reinterpret_cast<const uint32_t*>(lr0 + src);
      *reinterpret_cast<uint32_t*>(lr1_out + dst) = *reinterpret_cast<const uint32_t*>(lr1 + src);
      *reinterpret_cast<uint32_t*>(lr2_out + dst) = *reinterpret_cast<const uint32_t*>(lr2 + src);
    } else {
      *reinterpret_cast<uint16_t*>(lr0_out + dst) = *reinterpret_cast<const uint16_t*>(lr0 + src);
      *reinterpret_cast<uint16_t*>(lr1_out + dst) = *reinterpret_cast<const uint16_t*>(lr1 + src);
      *reinterpret_cast<uint16_t*>(lr2_out + dst) = *reinterpret_cast<const uint16_t*>(lr2 + src);
    }
  }
  const SK* ks = k + tok_index(b, t, T) * H;
  const SV* vs = v + tok_index(b, t, T) * H;
  for (int h0 = lane * VE; h0 < H; h0 += kWave * VE) {
    SK kx[VE];
    float vx[VE];
#pragma unroll
    for (int i = 0; i < VE; ++i) {
      kx[i] = ks[h0 + i];
      vx[i] = VT::load(vs[h0 + i]);
    }
    for (int j = 0; j < n; ++j) {
      const int row = rm[j];
      if (row < 0 || row >= num_out) continue;
      const float p = probs[b * p_sb + (int64_t)rm[E + j] * p_se + (int64_t)t * p_st];
      SK* kd = k_out + ((int64_t)b * num_out + row) * H + h0;
      SK* vd = v_out + ((int64_t)b * num_out + row) * H + h0;
#pragma unroll
      for (int i = 0; i < VE; ++i) {
        kd[i] = kx[i];
        vd[i] = KT::store(vx[i] * p);
      }
    }
  }
}

template <class KT, class VT, class LT, int VE>
__global__ __launch_bounds__(kTokPerBlock* kWave) void permute_kv_bwd_kernel(
    const typename KT::S* __restrict__ gk, const typename KT::S* __restrict__ gv,
    const typename LT::S* __restrict__ glr0, const typename LT::S* __restrict__ glr1,
    const typename LT::S* __restrict__ glr2, const typename VT::S* __restrict__ v,
    const float* __restrict__ probs, int64_t p_sb, int64_t p_se, int64_t p_st, int H, int T,
    const int32_t* __restrict__ rmap, int E, int num_out, typename KT::S* __restrict__ grad_k,
    typename VT::S* __restrict__ grad_v, typename LT::S* __restrict__ grad_lr0,
    typename LT::S* __restrict__ grad_lr1, typename LT::S* __restrict__ grad_lr2,
    float* __restrict__ grad_probs) {
  using SK = typename KT::S;
  using SV = typename VT::S;
  const int t = blockIdx.x * kTokPerBlock + threadIdx.x / kWave;
  const int b = blockIdx.y;
  if (t >= T) return;
  const int lane = lane_id();
  const int32_t* rm = rmap + tok_index(b, t, T) * (2 * E + 1);
  const int n = rm[2 * E];
  if (lane == 0) {
    float a0 = 0.f, a1 = 0.f, a2 = 0.f;
    for (int j = 0; j < n; ++j) {
      const int row = rm[j];
      if (row < 0 || row >= num_out) continue;
      const int64_t r = (int64_t)b * num_out + row;
      a0 += LT::load(glr0[r]);
      a1 += LT::load(glr1[r]);
      a2 += LT::load(glr2[r]);
    }
    grad_lr0[tok_index(b, t, T)] = LT::store(a0);
    grad_lr1[tok_index(b, t, T)] = LT::store(a1);
    grad_lr2[tok_index(b, t, T)] = LT::store(a2);
  }
  for (int e = lane; e < E; e += kWave) {
    bool routed = false;
    for (int j = 0; j < n; ++j) routed = routed || (rm[E + j] == e);
    if (!routed) grad_probs[((int64_t)b * E + e) * T + t] = 0.0f;
  }
  // fp32 partial dot products for the prob gradient, one per slot (n <= E)
  const SV* vs = v + tok_index(b, t, T) * H;
  for (int j = 0; j < n; ++j) {
    const int row = rm[j];
    if (row < 0 || row >= num_out) continue;
    const float p = probs[b * p_sb + (int64_t)rm[E + j] * p_se + (int64_t)t * p_st];
    const SK* gvr = gv + ((int64_t)b * num_out + row) * H;
    float dot = 0.0f;
    if (p != 0.0f) {
      for (int h0 = lane * VE; h0 < H; h0 += kWave * VE) {
#pragma unroll
        for (int i = 0; i < VE; ++i) dot = __builtin_fmaf(KT::load(gvr[h0 + i]), VT::load(vs[h0 + i]), dot);
      }
    }
    dot = wave_sum(dot);
    if (lane == 0) grad_probs[((int64_t)b * E + rm[E + j]) * T + t] = dot;
  }
  for (int h0 = lane * VE; h0 < H; h0 += kWave * VE) {
    float ak[VE], av[VE];
#pragma unroll
    for (int i = 0; i < VE; ++i) ak[i] = av[i] = 0.0f;
    for (int j = 0; j < n; ++j) {
      const int row = rm[j];
      if (row < 0 || row >= num_out) continue;
      const float p = probs[b * p_sb + (int64_t)rm[E + j] * p_se + (int64_t)t * p_st];
      const int64_t r = ((int64_t)b * num_out + row) * H + h0;
#pragma unroll
      for (int i = 0; i < VE; ++i) {
        ak[i] += KT::load(gk[r + i]);
        av[i] = __builtin_fmaf(KT::load(gv[r + i]), p, av[i]);
      }
    }
#pragma unroll
    for (int i = 0; i < VE; ++i) {
      grad_k[tok_index(b, t, T) * H + h0 + i] = KT::store(ak[i]);
      grad_v[tok_index(b, t, T) * H + h0 + i] = VT::store(av[i]);
    }
  }
}

inline dim3 tok_grid(int T, int B) { return dim3((T + kTokPerBlock - 1) / kTokPerBlock, B); }
inline dim3 tok_block() { return dim3(kTokPerBlock * kWave); }

// Elements per lane chunk: 16 bytes when the row and the pointers allow it.
template <class TT>
int pick_ve(int H, std::initializer_list<const void*> ptrs) {
  const int eb = sizeof(typename TT::S);
  const int vb = pick_vec_bytes((int64_t)H * eb, ptrs);
  const int ve = vb / eb;
  return ve >= 8 ? 8 : ve >= 4 ? 4 : ve >= 2 ? 2 : 1;
}

#define UTTT_VE_SWITCH(ve, ...)          \
  switch (ve) {                          \
    case 8: { constexpr int VE = 8; __VA_ARGS__; } break; \
    case 4: { constexpr int VE = 4; __VA_ARGS__; } break; \
    case 2: { constexpr int VE = 2; __VA_ARGS__; } break; \
    default: { constexpr int VE = 1; __VA_ARGS__; } break; \
  }

#define UTTT_DTYPE_SWITCH(dt, TT, ...)                             \
  switch (dt) {                                                    \
    case UTTT_F32: { using TT = F32T; __VA_ARGS__; } break;         \
    case UTTT_BF16: { using TT = BF16T; __VA_ARGS__; } break;       \
    case UTTT_F16: { using TT = F16T; __VA_ARGS__; } break;         \
    default: set_error("unsupported dtype code %d", (int)dt); return UTTT_ERR_ARG; \
  }

}  // namespace

bool rowmap_fused_fits(int T, int E) {
  const int ntiles = (T + kTile - 1) / kTile;
  return T >= 1 && T % 16 == 0 && ntiles <= kFusedMaxTiles && E >= 1 && E <= kFusedMaxE;
}

bool launch_rowmap_fused(const uint8_t* mask, int64_t s_b, int64_t s_e, int B, int T, int E,
                         int32_t* group_sizes, int32_t* row_id_map, const float* part_bal,
                         int nblk_r, float* bal_sum, hipStream_t st, int32_t* src_rows,
                         int64_t src_sb) {
  const int ntiles = (T + kTile - 1) / kTile;
  const bool aligned = ((reinterpret_cast<uintptr_t>(mask) |
                         reinterpret_cast<uintptr_t>(row_id_map)) & 15u) == 0;
  if (B < 1 || T < 1 || T % 16 != 0 || s_e % 16 != 0 || s_b % 16 != 0 || !aligned ||
      ntiles > kFusedMaxTiles || E < 1 || E > kFusedMaxE ||
      (part_bal != nullptr && (nblk_r < 1 || nblk_r > 2 * kWave)))
    return false;
  const dim3 grid(ntiles + (part_bal != nullptr ? 1 : 0), B);
  if (E <= 16)
    hipLaunchKernelGGL(rowmap_fused_kernel<16>, grid, dim3(kTile), 0, st, mask, s_b, s_e, T, E,
                       ntiles, group_sizes, row_id_map, part_bal, nblk_r, bal_sum, src_rows, src_sb);
  else if (E <= 32)
    hipLaunchKernelGGL(rowmap_fused_kernel<32>, grid, dim3(kTile), 0, st, mask, s_b, s_e, T, E,
                       ntiles, group_sizes, row_id_map, part_bal, nblk_r, bal_sum, src_rows, src_sb);
  else
    hipLaunchKernelGGL(rowmap_fused_kernel<kFusedMaxE>, grid, dim3(kTile), 0, st, mask, s_b, s_e,
                       T, E, ntiles, group_sizes, row_id_map, part_bal, nblk_r, bal_sum, src_rows,
                       src_sb);
  return true;
}

}  // namespace uttt

using namespace uttt;

extern "C" size_t uttt_row_id_map_workspace_bytes(int B, int T, int E) {
  if (B <= 0 || T <= 0 || E <= 0) return 0;
  const int ntiles = (T + kTile - 1) / kTile;
  const int per_tile = E <= kScanEmitMaxE ? padded_experts(E) : E;  // count-table row
  return (size_t)B * per_tile * ntiles * sizeof(int32_t);
}

extern "C" int uttt_make_row_id_map(const void* routing_map, int mask_bytes, int64_t s_b,
                                    int64_t s_e, int64_t s_t, int B, int T, int E,
                                    int32_t* row_id_map, int32_t* group_sizes, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  UTTT_REQUIRE(B >= 0 && T >= 0 && E >= 1, "make_row_id_map: bad sizes B=%d T=%d E=%d", B, T, E);
  UTTT_REQUIRE(E <= kMaxExperts, "make_row_id_map: E=%d exceeds %d", E, kMaxExperts);
  UTTT_REQUIRE(mask_bytes == 1 || mask_bytes == 4, "make_row_id_map: mask element size %d", mask_bytes);
  if (B == 0) return UTTT_OK;
  const size_t need = uttt_row_id_map_workspace_bytes(B, T > 0 ? T : 1, E);
  UTTT_REQUIRE(workspace != nullptr && workspace_bytes >= need,
               "make_row_id_map: workspace %zu < %zu bytes", workspace_bytes, need);
  UTTT_REQUIRE(row_id_map != nullptr, "make_row_id_map: null row_id_map");
  hipStream_t st = as_stream(stream);
  if (T == 0) {
    if (group_sizes != nullptr) {
      return zero_fill_async(group_sizes, sizeof(int32_t) * B * E, st, "make_row_id_map");
    }
    return UTTT_OK;
  }
  UTTT_REQUIRE(routing_map != nullptr, "make_row_id_map: null routing_map");
  const int ntiles = (T + kTile - 1) / kTile;
  const bool vec_ok = ((reinterpret_cast<uintptr_t>(routing_map) |
                        reinterpret_cast<uintptr_t>(row_id_map)) & 15u) == 0;
  if (mask_bytes == 1 && s_t == 1 && T % 16 == 0 && s_e % 16 == 0 && s_b % 16 == 0 && vec_ok &&
      ntiles <= kFusedMaxTiles && E <= kFusedMaxE) {
    launch_rowmap_fused(static_cast<const uint8_t*>(routing_map), s_b, s_e, B, T, E,
                        group_sizes, row_id_map, nullptr, 0, nullptr, st);
    return check_launch("make_row_id_map");
  }
  int32_t* counts = reinterpret_cast<int32_t*>(workspace);
  auto launch = [&](auto mb) {
    constexpr int MB = decltype(mb)::value;
    if (E <= kScanEmitMaxE) {  // count, then scan + emit (two launches)
      const bool vec = T % 4 == 0 && (reinterpret_cast<uintptr_t>(row_id_map) & 15u) == 0;
      const size_t lds = sizeof(int32_t) * kTile * (2 * E + 1);
      auto two = [&](auto ep) {
        constexpr int EP = decltype(ep)::value;
        hipLaunchKernelGGL((rowmap_count_kernel<MB, EP>), dim3(ntiles, B), dim3(kTile), 0, st,
                           routing_map, s_b, s_e, s_t, T, E, ntiles, counts);
        if (vec)
          hipLaunchKernelGGL((rowmap_scan_emit_kernel<MB, EP, true>), dim3(ntiles, B),
                             dim3(kTile), lds, st, routing_map, s_b, s_e, s_t, T, E, ntiles,
                             counts, group_sizes, row_id_map);
        else
          hipLaunchKernelGGL((rowmap_scan_emit_kernel<MB, EP, false>), dim3(ntiles, B),
                             dim3(kTile), lds, st, routing_map, s_b, s_e, s_t, T, E, ntiles,
                             counts, group_sizes, row_id_map);
      };
      switch (padded_experts(E)) {
        case 4: two(std::integral_constant<int, 4>{}); break;
        case 8: two(std::integral_constant<int, 8>{}); break;
        case 16: two(std::integral_constant<int, 16>{}); break;
        default: two(std::integral_constant<int, 32>{}); break;
      }
      return;
    }
    hipLaunchKernelGGL(rowmap_count_kernel<MB>, dim3(ntiles, B), dim3(kTile), 0, st, routing_map,
                       s_b, s_e, s_t, T, E, ntiles, counts);
    hipLaunchKernelGGL(rowmap_scan_kernel, dim3(B), dim3(kScanThreads), 0, st, counts, E, ntiles,
                       group_sizes);
    if (2 * E + 1 <= kStageMaxW) {
      hipLaunchKernelGGL((rowmap_emit_kernel<MB, true>), dim3(ntiles, B), dim3(kTile),
                         sizeof(int32_t) * kTile * (2 * E + 1), st, routing_map, s_b, s_e, s_t, T,
                         E, ntiles, counts, row_id_map);
    } else {
      hipLaunchKernelGGL((rowmap_emit_kernel<MB, false>), dim3(ntiles, B), dim3(kTile), 0, st,
                         routing_map, s_b, s_e, s_t, T, E, ntiles, counts, row_id_map);
    }
  };
  if (mask_bytes == 1) {
    launch(std::integral_constant<int, 1>{});
  } else {
    launch(std::integral_constant<int, 4>{});
  }
  return check_launch("make_row_id_map");
}

extern "C" int uttt_permute_fwd(const void* inp, int dtype, int B, int T, int H,
                                const int32_t* row_id_map, int E, const float* probs, int64_t p_sb,
                                int64_t p_se, int64_t p_st, void* out, int num_out,
                                float* permuted_probs, void* stream) {
  const int eb = dtype_bytes(dtype);
  UTTT_REQUIRE(eb > 0, "permute_fwd: unsupported dtype %d", dtype);
  UTTT_REQUIRE(B >= 0 && T >= 0 && H >= 0 && E >= 1 && num_out >= 0, "permute_fwd: bad sizes");
  UTTT_REQUIRE(probs == nullptr || permuted_probs != nullptr || num_out == 0,
               "permute_fwd: probs given without permuted_probs");
  if (B == 0 || T == 0 || H == 0) {
    if (probs != nullptr && B > 0 && T > 0 && H == 0) {
      // rows are empty but the permuted probs still have to be produced
    } else {
      return UTTT_OK;
    }
  }
  const int64_t row_bytes = (int64_t)H * eb;
  const int vb = pick_vec_bytes(row_bytes > 0 ? row_bytes : 16, {inp, out});
  hipStream_t st = as_stream(stream);
#define UTTT_LAUNCH_PERM(VBv)                                                                   \
  do {                                                                                          \
    if (row_bytes > 0) {                                                                        \
      const int CH = (int)(row_bytes / VBv);                                                    \
      const int64_t chunks = (int64_t)B * T * CH;                                               \
      UTTT_REQUIRE(chunks < (1ll << 31), "permute_fwd: payload too large (%lld chunks)",        \
                   (long long)chunks);                                                          \
      const unsigned grid = (unsigned)((chunks + kCT * kCU - 1) / (kCT * kCU));                 \
      hipLaunchKernelGGL((permute_chunk_kernel<VBv, kCU, kNT>), dim3(grid), dim3(kCT), 0, st,   \
                         reinterpret_cast<const uint8_t*>(inp), row_bytes, CH, B * T, T,        \
                         row_id_map, E, probs, p_sb, p_se, p_st,                                \
                         reinterpret_cast<uint8_t*>(out), num_out, permuted_probs);             \
    } else {                                                                                    \
      hipLaunchKernelGGL(permute_fwd_kernel<VBv>, tok_grid(T, B), tok_block(), 0, st,           \
                         reinterpret_cast<const uint8_t*>(inp), row_bytes, T, row_id_map, E,    \
                         probs, p_sb, p_se, p_st, reinterpret_cast<uint8_t*>(out), num_out,     \
                         permuted_probs);                                                       \
    }                                                                                           \
  } while (0)
  switch (vb) {
    case 16: UTTT_LAUNCH_PERM(16); break;
    case 8: UTTT_LAUNCH_PERM(8); break;
    case 4: UTTT_LAUNCH_PERM(4); break;
    default: UTTT_LAUNCH_PERM(2); break;
  }
#undef UTTT_LAUNCH_PERM
  return check_launch("permute_fwd");
}

extern "C" int uttt_permute_bwd(const void* grad_out, int dtype, int B, int T, int H,
                                const int32_t* row_id_map, int E, int num_out,
                                const float* grad_permuted_probs, void* grad_inp,
                                float* grad_probs, void* stream) {
  UTTT_REQUIRE(B >= 0 && T >= 0 && H >= 0 && E >= 1, "permute_bwd: bad sizes");
  UTTT_REQUIRE((grad_permuted_probs == nullptr) == (grad_probs == nullptr),
               "permute_bwd: grad_permuted_probs and grad_probs go together");
  if (B == 0 || T == 0) return UTTT_OK;
  hipStream_t st = as_stream(stream);
  UTTT_DTYPE_SWITCH(dtype, TT, {
    using S = typename TT::S;
    const int ve = pick_ve<TT>(H, {grad_out, grad_inp});
    UTTT_VE_SWITCH(ve, hipLaunchKernelGGL((permute_bwd_kernel<TT, VE>), tok_grid(T, B), tok_block(),
                                          0, st, reinterpret_cast<const S*>(grad_out), H, T,
                                          row_id_map, E, num_out, grad_permuted_probs,
                                          reinterpret_cast<S*>(grad_inp), grad_probs));
  });
  return check_launch("permute_bwd");
}

extern "C" int uttt_unpermute_fwd(const void* inp, int dtype, int B, int num_out, int H,
                                  const int32_t* row_id_map, int T, int E, const float* probs,
                                  int64_t p_sb, int64_t p_se, int64_t p_st, void* out,
                                  void* stream) {
  UTTT_REQUIRE(B >= 0 && T >= 0 && H >= 0 && E >= 1 && num_out >= 0, "unpermute_fwd: bad sizes");
  if (B == 0 || T == 0 || H == 0) return UTTT_OK;
  hipStream_t st = as_stream(stream);
  if (num_out == 0) {  // no slot holds a row: every output row is the empty sum
    const int eb = dtype_bytes(dtype);
    UTTT_REQUIRE(eb > 0, "unpermute_fwd: unsupported dtype %d", dtype);
    return zero_fill_async(out, (size_t)B * T * H * eb, st, "unpermute_fwd");
  }
  UTTT_DTYPE_SWITCH(dtype, TT, {
    using S = typename TT::S;
    const int ve = pick_ve<TT>(H, {inp, out});
    const int CH = H / ve;
    const int64_t chunks = (int64_t)B * T * CH;
    UTTT_REQUIRE(chunks < (1ll << 31), "unpermute_fwd: payload too large (%lld chunks)",
                 (long long)chunks);
    const unsigned grid = (unsigned)((chunks + kCT * kCU - 1) / (kCT * kCU));
    // pick_ve never yields a chunk above 16 bytes; those instantiations are skipped
    UTTT_VE_SWITCH(ve, if constexpr (sizeof(S) * VE <= 16) {
      hipLaunchKernelGGL((unpermute_chunk_kernel<TT, VE, kCU, kNT>), dim3(grid), dim3(kCT), 0, st,
                         reinterpret_cast<const S*>(inp), H, CH, B * T, T, num_out, row_id_map, E,
                         probs, p_sb, p_se, p_st, reinterpret_cast<S*>(out));
    });
  });
  return check_launch("unpermute_fwd");
}

extern "C" int uttt_unpermute_bwd(const void* grad_out, const void* fwd_inp, int dtype, int B,
                                  int T, int H, const int32_t* row_id_map, int E, int num_out,
                                  const float* probs, int64_t p_sb, int64_t p_se, int64_t p_st,
                                  void* grad_inp, float* grad_probs, int64_t gp_sb, int64_t gp_se,
                                  int64_t gp_st, void* stream) {
  UTTT_REQUIRE(B >= 0 && T >= 0 && H >= 0 && E >= 1, "unpermute_bwd: bad sizes");
  UTTT_REQUIRE(probs != nullptr && grad_probs != nullptr, "unpermute_bwd: probs are required");
  if (B == 0 || T == 0) return UTTT_OK;
  hipStream_t st = as_stream(stream);
  UTTT_DTYPE_SWITCH(dtype, TT, {
    using S = typename TT::S;
    const int ve = pick_ve<TT>(H, {grad_out, fwd_inp, grad_inp});
    UTTT_VE_SWITCH(ve, hipLaunchKernelGGL((unpermute_bwd_kernel<TT, VE>), tok_grid(T, B),
                                          tok_block(), 0, st,
                                          reinterpret_cast<const S*>(grad_out),
                                          reinterpret_cast<const S*>(fwd_inp), H, T, row_id_map,
                                          E, num_out, probs, p_sb, p_se, p_st,
                                          reinterpret_cast<S*>(grad_inp), grad_probs, gp_sb,
                                          gp_se, gp_st));
  });
  return check_launch("unpermute_bwd");
}

namespace {
template <class KT, class VT>
int launch_permute_kv_fwd(const void* k, const void* v, const void* lr0, const void* lr1,
                          const void* lr2, int lr_bytes, int B, int T, int H,
                          const int32_t* row_id_map, int E, const float* probs, int64_t p_sb,
                          int64_t p_se, int64_t p_st, void* k_out, void* v_out, void* lr0_out,
                          void* lr1_out, void* lr2_out, int num_out, hipStream_t st) {
  const int vek = pick_ve<KT>(H, {k, k_out, v_out});
  const int vev = pick_ve<VT>(H, {v});
  const int ve = vek < vev ? vek : vev;
  UTTT_VE_SWITCH(
      ve, hipLaunchKernelGGL((permute_kv_fwd_kernel<KT, VT, VE>), tok_grid(T, B), tok_block(), 0,
                             st, reinterpret_cast<const typename KT::S*>(k),
                             reinterpret_cast<const typename VT::S*>(v),
                             reinterpret_cast<const uint8_t*>(lr0),
                             reinterpret_cast<const uint8_t*>(lr1),
                             reinterpret_cast<const uint8_t*>(lr2), lr_bytes, H, T, row_id_map, E,
                             probs, p_sb, p_se, p_st, reinterpret_cast<typename KT::S*>(k_out),
                             reinterpret_cast<typename KT::S*>(v_out),
                             reinterpret_cast<uint8_t*>(lr0_out),
                             reinterpret_cast<uint8_t*>(lr1_out),
                             reinterpret_cast<uint8_t*>(lr2_out), num_out));
  return check_launch("permute_kv_lrs_fwd");
}

template <class KT, class VT, class LT>
int launch_permute_kv_bwd(const void* gk, const void* gv, const void* glr0, const void* glr1,
                          const void* glr2, const void* v, const float* probs, int64_t p_sb,
                          int64_t p_se, int64_t p_st, int B, int T, int H,
                          const int32_t* row_id_map, int E, int num_out, void* grad_k,
                          void* grad_v, void* grad_lr0, void* grad_lr1, void* grad_lr2,
                          float* grad_probs, hipStream_t st) {
  const int vek = pick_ve<KT>(H, {gk, gv, grad_k});
  const int vev = pick_ve<VT>(H, {v, grad_v});
  const int ve = vek < vev ? vek : vev;
  using SL = typename LT::S;
  UTTT_VE_SWITCH(
      ve, hipLaunchKernelGGL((permute_kv_bwd_kernel<KT, VT, LT, VE>), tok_grid(T, B), tok_block(),
                             0, st, reinterpret_cast<const typename KT::S*>(gk),
                             reinterpret_cast<const typename KT::S*>(gv),
                             reinterpret_cast<const SL*>(glr0), reinterpret_cast<const SL*>(glr1),
                             reinterpret_cast<const SL*>(glr2),
                             reinterpret_cast<const typename VT::S*>(v), probs, p_sb, p_se, p_st,
                             H, T, row_id_map, E, num_out,
                             reinterpret_cast<typename KT::S*>(grad_k),
                             reinterpret_cast<typename VT::S*>(grad_v),
                             reinterpret_cast<SL*>(grad_lr0), reinterpret_cast<SL*>(grad_lr1),
                             reinterpret_cast<SL*>(grad_lr2), grad_probs));
  return check_launch("permute_kv_lrs_bwd");
}
}  // namespace

extern "C" int uttt_permute_kv_lrs_fwd(const void* k, int k_dtype, const void* v, int v_dtype,
                                       const void* lr0, const void* lr1, const void* lr2,
                                       int lr_bytes, int B, int T, int H,
                                       const int32_t* row_id_map, int E, const float* probs,
                                       int64_t p_sb, int64_t p_se, int64_t p_st, void* k_out,
                                       void* v_out, void* lr0_out, void* lr1_out, void* lr2_out,
                                       int num_out, void* stream) {
  UTTT_REQUIRE(B >= 0 && T >= 0 && H >= 0 && E >= 1 && num_out >= 0,
               "permute_kv_lrs_fwd: bad sizes");
  UTTT_REQUIRE(lr_bytes == 2 || lr_bytes == 4, "permute_kv_lrs_fwd: lr element size %d", lr_bytes);
  UTTT_REQUIRE(probs != nullptr, "permute_kv_lrs_fwd: probs are required");
  if (B == 0 || T == 0) return UTTT_OK;
  hipStream_t st = as_stream(stream);
  UTTT_DTYPE_SWITCH(k_dtype, KT, {
    UTTT_DTYPE_SWITCH(v_dtype, VT, {
      return launch_permute_kv_fwd<KT, VT>(k, v, lr0, lr1, lr2, lr_bytes, B, T, H, row_id_map, E,
                                           probs, p_sb, p_se, p_st, k_out, v_out, lr0_out,
                                           lr1_out, lr2_out, num_out, st);
    });
  });
  return UTTT_OK;
}

extern "C" int uttt_permute_kv_lrs_bwd(const void* gk, const void* gv, int k_dtype,
                                       const void* glr0, const void* glr1, const void* glr2,
                                       int glr_dtype, const void* v, int v_dtype,
                                       const float* probs, int64_t p_sb, int64_t p_se,
                                       int64_t p_st, int B, int T, int H,
                                       const int32_t* row_id_map, int E, int num_out,
                                       void* grad_k, void* grad_v, void* grad_lr0,
                                       void* grad_lr1, void* grad_lr2, float* grad_probs,
                                       void* stream) {
  UTTT_REQUIRE(B >= 0 && T >= 0 && H >= 0 && E >= 1 && num_out >= 0,
               "permute_kv_lrs_bwd: bad sizes");
  UTTT_REQUIRE(probs != nullptr && grad_probs != nullptr, "permute_kv_lrs_bwd: probs required");
  if (B == 0 || T == 0) return UTTT_OK;
  hipStream_t st = as_stream(stream);
  UTTT_DTYPE_SWITCH(k_dtype, KT, {
    UTTT_DTYPE_SWITCH(v_dtype, VT, {
      UTTT_DTYPE_SWITCH(glr_dtype, LT, {
        return launch_permute_kv_bwd<KT, VT, LT>(gk, gv, glr0, glr1, glr2, v, probs, p_sb, p_se,
                                                 p_st, B, T, H, row_id_map, E, num_out, grad_k,
                                                 grad_v, grad_lr0, grad_lr1, grad_lr2, grad_probs,
                                                 st);
      });
    });
  });
  return UTTT_OK;
}
