// Asynchronous MFMA GEMM pipeline for gfx950 (the core of every grouped
// fast-weight GEMM).
//
// Workgroup: 256 threads = 4 waves in a 2x2 grid.  A workgroup multiplies two
// 128-row A tiles (A0, A1) by one 128-row B tile per K step of kBK = 64 into
// two fp32 accumulators (acc0 = A0 B^T, acc1 = A1 B^T); each wave owns a 64x64
// quadrant of both, as 2x2 blocks of v_mfma_f32_32x32x16_bf16.
//
// Global -> LDS: global_load_lds_dwordx4 (16 bytes per lane straight into LDS,
// no register staging) into a ring of three stages, so the loads of step k+2
// are in flight while step k is multiplied; the only waits are explicit
// s_waitcnt vmcnt counts and one s_barrier per step.  Each stage lives in its
// own __shared__ array so the compiler can tell the in-flight LDS writes from
// the LDS reads of the current stage.
//
// LDS tile layouts (16-byte chunks, XOR-swizzled against bank conflicts):
//   KMajor tile (operand stored [rows][K], K contiguous): 128 rows x 8 chunks;
//     chunk c of row r sits at slot r*8 + (c ^ (r & 7)).  Fragments are one
//     ds_read_b128 (8 consecutive k of one row).
//   RMajor tile (operand stored [K][rows], rows contiguous): 64 k-rows x 16
//     chunks; chunk c of k-row k sits at slot k*16 + (c ^ swz(k)).  Fragments
//     are two ds_read_b64_tr_b16: within a group of 16 lanes, source lane
//     s = 4j + q reads k-row j, rows 4q..4q+3, and the hardware hands lane i
//     the column i of that 4x16 block, i.e. 4 consecutive k of row i.
// Lanes whose chunk lies outside the operand read a 16-byte zero block, so
// partial tiles need no special casing in the MFMA loop.
#pragma once

#include "common.h"

namespace uttt {
namespace pipe {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kBK = 64;
constexpr int kTileRows = 128;
constexpr int kTileBytes = kTileRows * kBK * 2;                  // 16 KiB
constexpr int kStageBytes = 3 * kTileBytes;                      // A0 | A1 | B
constexpr int kLoadsPerTile = kTileBytes / 16 / kThreads;        // 4 per thread
constexpr int kLoadsPerStage = 3 * kLoadsPerTile;                // 12 per wave

enum Major { KMajor = 0, RMajor = 1 };

// 16 zero bytes (zero-initialised device memory, never written): the source
// of every masked-off lane of a tile load.
__device__ __attribute__((aligned(16))) uint4 g_zero16;

#define UTTT_LDS(p) ((__attribute__((address_space(3))) void*)(p))

// s_waitcnt vmcnt(N) leaving the export and LDS counters alone (gfx9
// encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

__device__ __forceinline__ void block_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// A global operand of one group: element (r, k) is at
//   KMajor: base[r * ld + k]      RMajor: base[k * ld + r]
// rows [0, r_end) and k [0, k_end) are valid; the rest reads as zero.
struct Operand {
  const uint16_t* base;
  int64_t ld;
  int r_end;
  int k_end;
};

__device__ __forceinline__ int rswz(int k) { return ((k & 7) << 1) & 15; }

// Issue this wave's share (kLoadsPerTile instructions) of the loads of the
// 128-row x kBK tile at (r0, k0) of `op` into the LDS tile at `dst`.
template <int MAJOR>
__device__ __forceinline__ void load_tile(const Operand& op, int r0, int k0, uint8_t* dst) {
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
#pragma unroll
  for (int t = 0; t < kLoadsPerTile; ++t) {
    const int base = (t * 4 + w) * 64;  // first slot of this instruction
    const int s = base + lane;
    const void* src = &g_zero16;
    if constexpr (MAJOR == KMajor) {
      const int r = s >> 3;
      const int c = (s & 7) ^ (r & 7);
      const int gr = r0 + r, gk = k0 + c * 8;
      if (gr < op.r_end && gk < op.k_end) src = op.base + (int64_t)gr * op.ld + gk;
    } else {
      const int k = s >> 4;
      const int c = (s & 15) ^ rswz(k);
      const int gk = k0 + k, gr = r0 + c * 8;
      if (gk < op.k_end && gr < op.r_end) src = op.base + (int64_t)gk * op.ld + gr;
    }
    __builtin_amdgcn_global_load_lds(src, UTTT_LDS(dst + base * 16), 16, 0, 0);
  }
}

// MFMA operand fragment of rows [rb, rb+32), k-substep ks (16 k) of an LDS tile.
template <int MAJOR>
__device__ __forceinline__ bf16x8 frag(const uint8_t* tile, int rb, int ks) {
  const int lane = threadIdx.x & 63;
  if constexpr (MAJOR == KMajor) {
    const int r = rb + (lane & 31);
    const int c = 2 * ks + (lane >> 5);
    return *reinterpret_cast<const bf16x8*>(tile + (r * 8 + (c ^ (r & 7))) * 16);
  } else {
    const int g = lane >> 4, s = lane & 15;
    const int j = s >> 2, q = s & 3;
    const int r = rb + 16 * (g & 1) + 4 * q;
    const int c = r >> 3;
    const int kb = 16 * ks + 8 * (g >> 1) + j;
    const int k0 = kb, k1 = kb + 4;
    const uint8_t* p0 = tile + (k0 * 16 + (c ^ rswz(k0))) * 16 + 8 * (q & 1);
    const uint8_t* p1 = tile + (k1 * 16 + (c ^ rswz(k1))) * 16 + 8 * (q & 1);
    const i16x4 x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) i16x4*)(p0));
    const i16x4 x1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) i16x4*)(p1));
    const i16x8 x = __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(bf16x8, x);
  }
}

// acc_a[i][j] += A_a(wave rows i) * B(wave cols j) over one stage, a = 0, 1.
template <int AMAJ, int BMAJ>
__device__ __forceinline__ void mma_stage(f32x16 (&acc0)[2][2], f32x16 (&acc1)[2][2],
                                          const uint8_t* st, int wm, int wn, bool two) {
  const uint8_t* a0 = st;
  const uint8_t* a1 = st + kTileBytes;
  const uint8_t* b = st + 2 * kTileBytes;
#pragma unroll
  for (int ks = 0; ks < kBK / 16; ++ks) {
    bf16x8 fb[2], fa[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) fb[j] = frag<BMAJ>(b, wn * 64 + j * 32, ks);
#pragma unroll
    for (int i = 0; i < 2; ++i) fa[i] = frag<AMAJ>(a0, wm * 64 + i * 32, ks);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        acc0[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc0[i][j], 0, 0, 0);
    if (two) {
#pragma unroll
      for (int i = 0; i < 2; ++i) fa[i] = frag<AMAJ>(a1, wm * 64 + i * 32, ks);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc1[i][j] =
              __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc1[i][j], 0, 0, 0);
    }
  }
}

// Three-stage ring: load(step, stage) issues kLoadsPerStage loads per wave;
// mma(stage) consumes one.  Step kt waits for its own loads while step kt+1's
// may still be in flight, then issues step kt+2 into the stage step kt-1 used.
template <class LoadFn, class MmaFn>
__device__ __forceinline__ void run_pipeline(int nk, LoadFn&& load, MmaFn&& mma, uint8_t* s0,
                                             uint8_t* s1, uint8_t* s2) {
  if (nk > 0) load(0, s0);
  if (nk > 1) load(1, s1);
  auto step = [&](int kt, uint8_t* cur, uint8_t* nxt) {
    if (kt + 1 < nk)
      wait_vmcnt<kLoadsPerStage>();
    else
      wait_vmcnt<0>();
    block_barrier();
    if (kt + 2 < nk) load(kt + 2, nxt);
    mma(cur);
  };
  for (int kt = 0; kt < nk; kt += 3) {
    step(kt, s0, s2);
    if (kt + 1 < nk) step(kt + 1, s1, s0);
    if (kt + 2 < nk) step(kt + 2, s2, s1);
  }
}

template <int N>
__device__ __forceinline__ void zero(f32x16 (&acc)[N][N]) {
#pragma unroll
  for (int i = 0; i < N; ++i)
#pragma unroll
    for (int j = 0; j < N; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
}

// Row (M) of accumulator element v of this lane inside its 32x32 block is
// 8*(v/4) + 4*(lane/32) + v%4; its column (N) is lane%32.
__device__ __forceinline__ int acc_row(int v) {
  return 8 * (v >> 2) + 4 * ((threadIdx.x & 63) >> 5) + (v & 3);
}
__device__ __forceinline__ int acc_col() { return threadIdx.x & 31; }

}  // namespace pipe
}  // namespace uttt

namespace uttt {
namespace pipe {

// ------------------------------------------------------------ scheduling ----
// Token-grouped problems (N = routed tokens): the tokens of expert e in batch
// b occupy [off(b,e), off(b,e)+g(b,e)) of that batch.  The grid covers an
// upper bound of ceil(N/BN) + E n-tiles per batch; each workgroup finds its
// (expert, n-tile) with a wave-level scan of group_sizes[b] and leaves if its
// tile index is past the batch's real tile count.  Segments are clamped to
// [0, N), so a group_sizes row that over-counts (the reference does not check
// sum == N) can never move a tile outside the token buffer.
struct TokenTile {
  int e;       // expert, or -1 when the workgroup has no tile
  int start;   // first token of the expert's segment
  int size;    // segment length
  int n0;      // first token of this tile, relative to the segment
};

template <int BN>
__device__ TokenTile find_token_tile(const int32_t* __restrict__ gs_b, int E, int N, int tile,
                                     int* s_scratch /* >= 4 ints */) {
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
      const int gc = g < avail ? g : avail;
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
  return TokenTile{s_scratch[0], s_scratch[1], s_scratch[2], s_scratch[3]};
}

// Segment [start, start+size) of expert e in batch b, clamped to [0, N).
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
__device__ __forceinline__ float bf16r(float x) { return bf16_to_f32(f32_to_bf16(x)); }

// Four consecutive-row results (rows m..m+3 of token column n) as one store
// into a token-major [.., N, ld] buffer (m a multiple of 4).
__device__ __forceinline__ void store4(uint16_t* out, int64_t ld, int64_t n, int m, float a,
                                       float b, float c, float d) {
  uint2 w;
  w.x = (uint32_t)f32_to_bf16(a) | ((uint32_t)f32_to_bf16(b) << 16);
  w.y = (uint32_t)f32_to_bf16(c) | ((uint32_t)f32_to_bf16(d) << 16);
  *reinterpret_cast<uint2*>(out + n * ld + m) = w;
}
__device__ __forceinline__ void store4(float* out, int64_t ld, int64_t n, int m, float a, float b,
                                       float c, float d) {
  *reinterpret_cast<float4*>(out + n * ld + m) = make_float4(a, b, c, d);
}
__device__ __forceinline__ void load4(const uint16_t* in, int64_t ld, int64_t n, int m,
                                      float* v) {
  const uint2 w = *reinterpret_cast<const uint2*>(in + n * ld + m);
  v[0] = bf16_to_f32((uint16_t)(w.x & 0xffffu));
  v[1] = bf16_to_f32((uint16_t)(w.x >> 16));
  v[2] = bf16_to_f32((uint16_t)(w.y & 0xffffu));
  v[3] = bf16_to_f32((uint16_t)(w.y >> 16));
}
__device__ __forceinline__ void load4(const float* in, int64_t ld, int64_t n, int m, float* v) {
  const float4 f = *reinterpret_cast<const float4*>(in + n * ld + m);
  v[0] = f.x;
  v[1] = f.y;
  v[2] = f.z;
  v[3] = f.w;
}

}  // namespace pipe
}  // namespace uttt
