// MFMA building blocks for the grouped fast-weight GEMMs on gfx950.
//
// Tiling: a workgroup of 256 threads = 4 waves in a 2x2 grid computes a
// BM x BN output tile; each wave owns a (BM/2) x (BN/2) sub-tile made of
// 32x32 blocks, each accumulated by v_mfma_f32_32x32x16_bf16 (fp32
// accumulate, K = 16 per instruction).  The K loop advances BK = 32 per
// stage through two LDS buffers: the global loads of stage s+1 are issued
// into registers before the MFMAs of stage s and written to the other LDS
// buffer after them, so one barrier per stage suffices.
//
// Operand tiles live in LDS as [rows][BK + kPad] bf16 (rows = M for A, N for
// B; K contiguous) so that every MFMA fragment is one 16-byte LDS read.
// Global operands come in two storage orders:
//   KMajor : element (r, k) at base + r*ld + k  (K contiguous).  Rows may
//            start anywhere; k offsets are multiples of 8 (16-byte loads).
//   RMajor : element (r, k) at base + k*ld + r  (rows contiguous).  k may
//            start anywhere (token offsets); r offsets are multiples of 8.
//            The tile is transposed on its way into LDS: a thread loads KG
//            consecutive k-rows of 8 r-values and writes, for each r, its
//            KG k-values as one LDS word.
// Out-of-range rows / k are read as zero, so partial tiles need no special
// casing in the MFMA loop.
#pragma once

#include "common.h"

namespace uttt {
namespace gemm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kBK = 32;
constexpr int kPad = 8;               // bf16 elements of row padding in LDS
constexpr int kLdsRow = kBK + kPad;   // LDS row pitch in elements (80 bytes)

enum Major { KMajor = 0, RMajor = 1 };

// A global operand: base pointer of the current group, leading dimension in
// elements, and the valid extents (rows beyond r_end / k beyond k_end read 0).
struct Operand {
  const uint16_t* base;
  int64_t ld;
  int r_end;   // valid rows are [0, r_end) relative to the tile origin's frame
  int k_end;   // valid k are [0, k_end)
};

// Per-thread staging registers for one ROWS x kBK tile.
template <int ROWS, int MAJOR>
struct TileRegs {
  static constexpr int kVecs = ROWS * kBK / 8;            // 16-byte vectors per tile
  static constexpr int kPerThread = kVecs / kThreads;     // vectors per thread
  static_assert(kVecs % kThreads == 0, "tile must split evenly over 256 threads");
  uint4 v[kPerThread];

  // Load rows [r0, r0+ROWS) x k [k0, k0+kBK) of `op` into registers.
  __device__ __forceinline__ void load(const Operand& op, int r0, int k0) {
    const int tid = threadIdx.x;
    if constexpr (MAJOR == KMajor) {
      // vector i of the tile: row = i / (kBK/8), k-chunk = i % (kBK/8)
#pragma unroll
      for (int j = 0; j < kPerThread; ++j) {
        const int i = tid + j * kThreads;
        const int r = r0 + i / (kBK / 8);
        const int k = k0 + (i % (kBK / 8)) * 8;
        if (r < op.r_end && k < op.k_end)
          v[j] = *reinterpret_cast<const uint4*>(op.base + (int64_t)r * op.ld + k);
        else
          v[j] = uint4{0u, 0u, 0u, 0u};
      }
    } else {
      // thread owns a KG x 8 block: k-rows [kq*KG, +KG), r-chunk rc
      constexpr int KG = kPerThread;
      constexpr int RC = ROWS / 8;   // r-chunks per tile
      const int rc = tid % RC;
      const int kq = tid / RC;       // < kBK / KG
      const int r = r0 + rc * 8;
#pragma unroll
      for (int j = 0; j < KG; ++j) {
        const int k = k0 + kq * KG + j;
        if (r < op.r_end && k < op.k_end)
          v[j] = *reinterpret_cast<const uint4*>(op.base + (int64_t)k * op.ld + r);
        else
          v[j] = uint4{0u, 0u, 0u, 0u};
      }
    }
  }

  // Write the staged vectors into an LDS tile [ROWS][kLdsRow].
  __device__ __forceinline__ void store(uint16_t* lds) const {
    const int tid = threadIdx.x;
    if constexpr (MAJOR == KMajor) {
#pragma unroll
      for (int j = 0; j < kPerThread; ++j) {
        const int i = tid + j * kThreads;
        const int r = i / (kBK / 8);
        const int k = (i % (kBK / 8)) * 8;
        *reinterpret_cast<uint4*>(lds + r * kLdsRow + k) = v[j];
      }
    } else {
      constexpr int KG = kPerThread;
      constexpr int RC = ROWS / 8;
      const int rc = tid % RC;
      const int kq = tid / RC;
      const uint16_t* e = reinterpret_cast<const uint16_t*>(v);  // e[j*8 + c] = (k=j, r=c)
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        uint16_t* dst = lds + (rc * 8 + c) * kLdsRow + kq * KG;
        if constexpr (KG == 4) {
          uint2 w;
          w.x = (uint32_t)e[0 * 8 + c] | ((uint32_t)e[1 * 8 + c] << 16);
          w.y = (uint32_t)e[2 * 8 + c] | ((uint32_t)e[3 * 8 + c] << 16);
          *reinterpret_cast<uint2*>(dst) = w;
        } else if constexpr (KG == 2) {
          *reinterpret_cast<uint32_t*>(dst) = (uint32_t)e[c] | ((uint32_t)e[8 + c] << 16);
        } else {
          dst[0] = e[c];
        }
      }
    }
  }
};

// One wave's MFMA work on one LDS stage: ACC(mb, nb) += A(mb) * B(nb) over
// kBK, for MB x NB blocks of 32x32.  `a_lds` / `b_lds` point at the wave's
// first row inside the LDS tiles.
template <int MB, int NB>
__device__ __forceinline__ void mma_stage(f32x16 (&acc)[MB][NB], const uint16_t* a_lds,
                                          const uint16_t* b_lds) {
  const int lane = threadIdx.x & 63;
  const int row = lane & 31;
  const int kh = (lane >> 5) * 8;
#pragma unroll
  for (int ks = 0; ks < kBK; ks += 16) {
    bf16x8 a[MB], b[NB];
#pragma unroll
    for (int i = 0; i < MB; ++i)
      a[i] = *reinterpret_cast<const bf16x8*>(a_lds + (i * 32 + row) * kLdsRow + ks + kh);
#pragma unroll
    for (int j = 0; j < NB; ++j)
      b[j] = *reinterpret_cast<const bf16x8*>(b_lds + (j * 32 + row) * kLdsRow + ks + kh);
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int j = 0; j < NB; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
  }
}

template <int MB, int NB>
__device__ __forceinline__ void zero_acc(f32x16 (&acc)[MB][NB]) {
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
}

// Position of accumulator element v of this lane inside its 32x32 block:
// row (M) = 8*(v/4) + 4*(lane/32) + v%4, column (N) = lane%32.
__device__ __forceinline__ int acc_row(int v) {
  return 8 * (v >> 2) + 4 * ((threadIdx.x & 63) >> 5) + (v & 3);
}
__device__ __forceinline__ int acc_col() { return threadIdx.x & 31; }

// ------------------------------------------------------------ scheduling ----
// Token-grouped problems (N = routed tokens): the tokens of expert e in batch
// b occupy [off(b,e), off(b,e)+g(b,e)) of that batch.  The grid covers an
// upper bound of ceil(N/BN) + E n-tiles per batch; each workgroup finds its
// (expert, n-tile) from a scan of group_sizes[b] held in LDS, and leaves if
// its tile index is past the batch's real tile count.
struct TokenTile {
  int e;       // expert, or -1 when the workgroup has no tile
  int start;   // first token of the expert's segment
  int size;    // segment length
  int n0;      // first token of this tile, relative to the segment
};

template <int BN>
__device__ TokenTile find_token_tile(const int32_t* __restrict__ gs_b, int E, int N, int tile,
                                     int* s_scratch /* >= 4 ints */) {
  // Lanes of wave 0 walk the experts 64 at a time with a running prefix of
  // token counts and tile counts.  Segments are clamped to [0, N), so a
  // group_sizes row that over-counts (the reference does not check
  // sum == N) can never move a tile outside the token buffer.
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    int tok_base = 0, tile_base = 0;
    int found_e = -1, found_start = 0, found_size = 0, found_n0 = 0;
    for (int e0 = 0; e0 < E; e0 += 64) {
      const int e = e0 + lane;
      const int graw = e < E ? gs_b[e] : 0;
      const int g = graw > 0 ? graw : 0;
      int tok_incl = g;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const int a = __shfl_up(tok_incl, d, 64);
        if (lane >= d) tok_incl += a;
      }
      const int start = tok_base + tok_incl - g;
      const int avail = start < N ? N - start : 0;
      const int gc = g < avail ? g : avail;            // clamped segment size
      const int nt = (gc + BN - 1) / BN;
      int tile_incl = nt;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const int b = __shfl_up(tile_incl, d, 64);
        if (lane >= d) tile_incl += b;
      }
      const int tile_excl = tile_base + tile_incl - nt;
      const bool hit = e < E && tile >= tile_excl && tile < tile_excl + nt;
      const uint64_t bal = __ballot(hit);
      if (bal != 0ull) {
        const int src = __ffsll((unsigned long long)bal) - 1;
        found_e = e0 + src;
        found_start = __shfl(start, src, 64);
        found_size = __shfl(gc, src, 64);
        found_n0 = (tile - __shfl(tile_excl, src, 64)) * BN;
        break;
      }
      tok_base += __shfl(tok_incl, 63, 64);
      tile_base += __shfl(tile_incl, 63, 64);
    }
    if (lane == 0) {
      s_scratch[0] = found_e;
      s_scratch[1] = found_start;
      s_scratch[2] = found_size;
      s_scratch[3] = found_n0;
    }
  }
  __syncthreads();
  TokenTile t{s_scratch[0], s_scratch[1], s_scratch[2], s_scratch[3]};
  return t;
}

// Segment [start, start+size) of expert e in batch b (weight-gradient
// problems, where the tokens are the reduction dimension), clamped to [0, N).
__device__ __forceinline__ void expert_segment(const int32_t* __restrict__ gs_b, int e, int N,
                                               int* start, int* size) {
  int s = 0;
  for (int i = 0; i < e; ++i) s += gs_b[i] > 0 ? gs_b[i] : 0;
  int g = gs_b[e] > 0 ? gs_b[e] : 0;
  if (s > N) s = N;
  if (g > N - s) g = N - s;
  *start = s;
  *size = g;
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + __expf(-x)); }

}  // namespace gemm
}  // namespace uttt
