// uTTT-Dense UPDATE stage 1 for small heads, fused: per head and token
//   Y0 = W0 k, Y2 = W2 k, DH = W1^T v            (fp32, K = D)
//   DY0 = sigmoid(Y0) Y2 DH (1 + Y0 (1 - sigmoid(Y0))) lr0
//   DY2 = silu(Y0) DH lr2,   Hid = silu(Y0) Y2 lr1   (stored bf16)
// Reference: compute_update, uttt_dense/modeling_recurrent_lact.py:409-432
// (gate_before_act, hidden_before_mul, dhidden, silu_backprop; the lr factors
// of dw0 / dw1 / dw2 at :425-432 are applied here to the token-side operands'
// partners, DY0 / Hid / DY2, so the weight gradients that follow are plain
// products DY^T k and v^T Hid).  The values and rounding points are those of
// the grouped stage 1 (a DH product to fp32, then the SwiGLU-derivative
// epilogue on fp32 Y0 / Y2 / DH).
//
// One workgroup = 128 tokens of one head, 32 per token group; a wave keeps
// its group's k^T and v^T fragments in registers for the whole kernel and
// walks 32-unit hidden blocks: Y0, Y2 and DH of a block land in the same
// accumulator layout (lane = token, 16 hidden units per lane), so the
// epilogue is lane-local and DH never leaves the registers.  The weights come
// from a fragment-ordered copy (uttt_dense_pack_update_weights) in which the
// A-operand rows of every block are permuted so that each lane's 16
// accumulator rows are 16 consecutive hidden units: every output row segment
// is two 16-byte stores.  For D <= 192 (dense_update_s1_staged_kernel) two
// waves share a token group and split the blocks, the weight fragments pass
// through LDS once per workgroup; for larger heads (dense_update_s1_kernel)
// 4 waves each walk every block, loading the fragments into registers.
#include <stdint.h>

#include "common.h"

namespace uttt {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kUpdWaves = 4;
constexpr int kUpdTok = 32 * kUpdWaves;  // tokens per workgroup


inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

__device__ __forceinline__ bf16x8_t ld16(const uint16_t* p) {
  return *reinterpret_cast<const bf16x8_t*>(p);
}

// Logistic sigmoid with the hardware exp and reciprocal (the grouped stage
// 1's formula).
__device__ __forceinline__ float sigm(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __expf(-x));
}

// Hidden offset (within a 32-unit block) of A-operand row slot rho of
// v_mfma_f32_32x32x16: accumulator element j of lane half g is row
// 8 (j / 4) + 4 g + j % 4, so this makes it hidden unit 16 g + j.
__host__ __device__ constexpr int upd_row_hidden(int rho) {
  return 16 * ((rho >> 2) & 1) + 4 * (rho >> 3) + (rho & 3);
}

// Fragment-ordered copy for the update, per head three parts of I*D bf16,
// each [I/32 blocks][D/16 k steps][64 lanes][8]; lane (r, g) of block blk,
// step s holds, with h = 32 blk + upd_row_hidden(r):
//   part 0: W0[h][16 s + 8 g .. + 8]      part 1: W2[h][16 s + 8 g .. + 8]
//   part 2: W1[16 s + 8 g + j][h], j = 0 .. 7  (a column of W1: W1^T row h)
__global__ __launch_bounds__(256) void dense_pack_update_kernel(
    const uint16_t* __restrict__ w02, const uint16_t* __restrict__ w1, int D, int I,
    uint16_t* __restrict__ packed) {
  const int bh = blockIdx.y;
  const int per_mat = I * D / 8;  // 16-byte chunks per part (<= 16384)
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= 3 * per_mat) return;
  const int KS = D / 16;
  const int m = c / per_mat;
  const int q = (c - m * per_mat) >> 6;  // blk * KS + s
  const int blk = q / KS, s = q - blk * KS;
  const int lane = c & 63, r = lane & 31, g = lane >> 5;
  const int h = 32 * blk + upd_row_hidden(r);
  uint4 v;
  if (m < 2) {
    v = *reinterpret_cast<const uint4*>(w02 + (int64_t)bh * 2 * I * D + (m * I + h) * D + 16 * s +
                                        8 * g);
  } else {
    const uint16_t* col = w1 + (int64_t)bh * D * I + (16 * s + 8 * g) * I + h;
    uint16_t e[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) e[j] = col[j * I];
    v = make_uint4(e[0] | (uint32_t)e[1] << 16, e[2] | (uint32_t)e[3] << 16,
                   e[4] | (uint32_t)e[5] << 16, e[6] | (uint32_t)e[7] << 16);
  }
  *reinterpret_cast<uint4*>(packed + (int64_t)bh * 3 * I * D + 8 * (int64_t)c) = v;
}

__device__ __forceinline__ void store16(uint16_t* p, const float* f) {
  uint4 v;
  v.x = pack_bf16x2(f[0], f[1]);
  v.y = pack_bf16x2(f[2], f[3]);
  v.z = pack_bf16x2(f[4], f[5]);
  v.w = pack_bf16x2(f[6], f[7]);
  *reinterpret_cast<uint4*>(p) = v;
}

// The layers' own inputs (LAYERED): token t of head bh = bb * H + hh is row
// bb * l + t % l of layer t / l, at column hh * D of that layer's [b, l, H*D]
// k and v; its lr is entry j of the layer's [b, l, 3] lr (lr_per_head: entry
// 3 hh + j of [b, l, 3H]), fp32 or bf16 (LR), no lr at all when lr.p[0] is
// null.  The gathered-head layout ([BH, N, D] k, v and fp32 lr [BH, N])
// holds the same values, so both give the same bits.
struct S1Layers {
  LayerPtrs k, v, lr;
  int l, H, lr_per_head;
};

// The inputs of one lane's token t of head bh: its k^T and v^T fragments
// (k = 16 s + 8 g .. + 8), its three lr values (1 without lr) and its row of
// the head's outputs.  t past N is clamped to N - 1 (every address valid).
template <int D, class LR, bool LAYERED>
struct S1Token {
  bf16x8_t kf[D / 16], vf[D / 16];
  float l0 = 1.0f, l1 = 1.0f, l2 = 1.0f;
  int64_t row;
  bool valid;

  __device__ __forceinline__ void load(const uint16_t* kh, const uint16_t* vh, const float* lr0,
                                       const float* lr1, const float* lr2, const S1Layers& ly,
                                       int N, int bh, int t, int g) {
    constexpr int KS = D / 16;
    valid = t < N;
    const int tc = min(t, N - 1);
    row = (int64_t)bh * N + tc;
    if constexpr (LAYERED) {
      // a wave's 32 tokens lie in one layer (l is a multiple of 32)
      const int li = __builtin_amdgcn_readfirstlane(tc / ly.l);
      const int bb = bh / ly.H, hh = bh - bb * ly.H;
      const int64_t tr = (int64_t)bb * ly.l + (tc - li * ly.l);  // row of the layer's tensors
      const uint16_t* kp = static_cast<const uint16_t*>(ly.k.p[li]) + (tr * ly.H + hh) * D;
      const uint16_t* vp = static_cast<const uint16_t*>(ly.v.p[li]) + (tr * ly.H + hh) * D;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        kf[s] = ld16(kp + 16 * s + 8 * g);
        vf[s] = ld16(vp + 16 * s + 8 * g);
      }
      using S = typename LR::S;
      const bool has = ly.lr.p[0] != nullptr;
      // a missing lr reads the first k element (a valid address) and is ignored
      const S* lp = has ? static_cast<const S*>(ly.lr.p[li]) +
                              tr * (ly.lr_per_head ? 3 * ly.H : 3) + (ly.lr_per_head ? 3 * hh : 0)
                        : reinterpret_cast<const S*>(kp);
      const S a = lp[0], b = lp[has ? 1 : 0], c = lp[has ? 2 : 0];
      if (has) {
        l0 = LR::load(a);
        l1 = LR::load(b);
        l2 = LR::load(c);
      }
    } else {
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        kf[s] = ld16(kh + row * D + 16 * s + 8 * g);
        vf[s] = ld16(vh + row * D + 16 * s + 8 * g);
      }
      // a missing lr reads the first k element (a valid address) and is ignored
      const float* fb = reinterpret_cast<const float*>(kh);
      const float l0r = *(lr0 ? lr0 + row : fb), l1r = *(lr1 ? lr1 + row : fb),
                  l2r = *(lr2 ? lr2 + row : fb);
      l0 = lr0 ? l0r : 1.0f;
      l1 = lr1 ? l1r : 1.0f;
      l2 = lr2 ? l2r : 1.0f;
    }
  }

  // The SwiGLU-derivative epilogue of hidden block blk from its accumulators
  // (lane = token, 16 consecutive hidden units per lane) and its six 16-byte
  // stores (valid tokens only).
  __device__ __forceinline__ void epilogue(const f32x16_t& y0, const f32x16_t& y2,
                                           const f32x16_t& dh, uint16_t* dyr, uint16_t* hr, int I,
                                           int blk) const {
    float d0[16], d2[16], hh[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const float sg = sigm(y0[u]);
      const float sw = sg * y0[u];
      d0[u] = sg * y2[u] * dh[u] * (1.0f + y0[u] * (1.0f - sg)) * l0;
      d2[u] = sw * dh[u] * l2;
      hh[u] = sw * y2[u] * l1;
    }
    if (valid) {
      uint16_t* o = dyr + 32 * blk;
      store16(o, d0);
      store16(o + 8, d0 + 8);
      store16(o + I, d2);
      store16(o + I + 8, d2 + 8);
      store16(hr + 32 * blk, hh);
      store16(hr + 32 * blk + 8, hh + 8);
    }
  }
};

// Four waves, one per 32 tokens, each walking all hidden blocks with its
// weight fragments loaded from the packed copy into registers per block
// (larger heads, and grids too small to fill the chip).  PIPE (D <= 192):
// two register sets, block b + 1's loads in flight while block b is
// multiplied and its epilogue runs (the last prefetch re-reads the last
// block: unconditional loads keep the wait counts exact).
template <int D, bool PIPE, class LR, bool LAYERED>
__global__ __launch_bounds__(kUpdWaves * 64) void dense_update_s1_kernel(
    const uint16_t* __restrict__ kh, const uint16_t* __restrict__ vh,
    const float* __restrict__ lr0, const float* __restrict__ lr1, const float* __restrict__ lr2,
    S1Layers ly, int N, int I, const uint16_t* __restrict__ packed, uint16_t* __restrict__ dy,
    uint16_t* __restrict__ hid) {
  constexpr int KS = D / 16;
  const int bh = blockIdx.y;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r = lane & 31, g = lane >> 5;
  S1Token<D, LR, LAYERED> tk;
  tk.load(kh, vh, lr0, lr1, lr2, ly, N, bh, blockIdx.x * kUpdTok + 32 * w + r, g);
  const uint16_t* ph = packed + (int64_t)bh * 3 * I * D + lane * 8;
  const int64_t part = (int64_t)I * D;
  uint16_t* dyr = dy + tk.row * 2 * I + 16 * g;
  uint16_t* hr = hid + tk.row * I + 16 * g;
  const int nblk = I / 32;

  auto load_blk = [&](bf16x8_t (&a0)[KS], bf16x8_t (&a2)[KS], bf16x8_t (&a1)[KS], int blk)
      __attribute__((always_inline)) {
    const uint16_t* p0 = ph + (int64_t)blk * KS * 64 * 8;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      a0[s] = ld16(p0 + s * 64 * 8);
      a2[s] = ld16(p0 + part + s * 64 * 8);
      a1[s] = ld16(p0 + 2 * part + s * 64 * 8);
    }
  };
  auto compute_blk = [&](const bf16x8_t (&a0)[KS], const bf16x8_t (&a2)[KS],
                         const bf16x8_t (&a1)[KS], int blk) __attribute__((always_inline)) {
    f32x16_t y0, y2, dh;
#pragma unroll
    for (int v = 0; v < 16; ++v) y0[v] = y2[v] = dh[v] = 0.0f;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      y0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0[s], tk.kf[s], y0, 0, 0, 0);
      y2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a2[s], tk.kf[s], y2, 0, 0, 0);
      dh = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1[s], tk.vf[s], dh, 0, 0, 0);
    }
    tk.epilogue(y0, y2, dh, dyr, hr, I, blk);
  };

  if constexpr (PIPE) {
    bf16x8_t A0[KS], A2[KS], A1[KS], B0[KS], B2[KS], B1[KS];
    load_blk(A0, A2, A1, 0);
    for (int blk = 0; blk < nblk; blk += 2) {
      load_blk(B0, B2, B1, min(blk + 1, nblk - 1));
      compute_blk(A0, A2, A1, blk);
      if (blk + 1 >= nblk) break;
      load_blk(A0, A2, A1, min(blk + 2, nblk - 1));
      compute_blk(B0, B2, B1, blk + 1);
    }
  } else {
    for (int blk = 0; blk < nblk; ++blk) {
      bf16x8_t a0[KS], a2[KS], a1[KS];
      load_blk(a0, a2, a1, blk);
      __builtin_amdgcn_sched_barrier(0);
      compute_blk(a0, a2, a1, blk);
    }
  }
}

// D <= 192: 8 waves, two per group of 32 tokens.  Waves w and w + 4 hold the
// same tokens' k / v fragments and take the even / odd hidden block of each
// pair of blocks, so the two waves of a SIMD share its matrix core and vector
// ALU (one's epilogue can run beside the other's products).  A pair's weight
// fragments -- six per k step, each 1 KiB of the packed copy -- go straight
// from global memory into LDS once per workgroup (global_load_lds, one
// fragment per wave instruction; each wave read all of them from the vector
// cache in the four-wave kernel), double-buffered: per pair, the next pair's
// loads issue first, then this block's products read the current buffer.
// The fragment reads are inline asm, which the compiler's wait-count pass
// does not model, so it does not hold them behind the loads into the other
// buffer (it cannot tell the two apart); every wait on them is explicit.
// After the products one wait covers the next pair's loads (older memory
// operations: the previous block's stores), then the epilogue stores, then
// an LDS-only barrier.
constexpr int kStgWaves = 8;
// grids of at least this many workgroups take the staged kernel
// (uttt_debug_set_s1_staged moves it)
int g_s1_staged_min_grid = 256;

typedef int s1_i32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ s1_i32x4 s1_ds_read(uint32_t addr) {
  s1_i32x4 v;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr) : "memory");
  return v;
}
// s_waitcnt lgkmcnt(N), tied to the fragment registers, so that no MFMA
// reading them moves above it
template <int N>
__device__ __forceinline__ void s1_lgkm_wait(s1_i32x4& a, s1_i32x4& b, s1_i32x4& c) {
  asm volatile("s_waitcnt lgkmcnt(%3)" : "+v"(a), "+v"(b), "+v"(c) : "i"(N) : "memory");
}
__device__ __forceinline__ void s1_lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <int D, class LR, bool LAYERED>
__global__ __launch_bounds__(kStgWaves * 64) void dense_update_s1_staged_kernel(
    const uint16_t* __restrict__ kh, const uint16_t* __restrict__ vh,
    const float* __restrict__ lr0, const float* __restrict__ lr1, const float* __restrict__ lr2,
    S1Layers ly, int N, int I, const uint16_t* __restrict__ packed, uint16_t* __restrict__ dy,
    uint16_t* __restrict__ hid) {
  constexpr int KS = D / 16;
  constexpr int kBlkChunks = 3 * KS * 64;    // 16-byte chunks of one block's three parts
  constexpr int kPairChunks = 2 * kBlkChunks;
  constexpr int kFrags = 6 * KS;             // 1 KiB fragments of a pair
  constexpr int kFragsPerWave = (kFrags + kStgWaves - 1) / kStgWaves;
  // two arrays, so that the compiler sees a stage's reads apart from the loads
  // into the other
  __shared__ __attribute__((aligned(16))) uint4 st0[kPairChunks];
  __shared__ __attribute__((aligned(16))) uint4 st1[kPairChunks];
  const int bh = blockIdx.y;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int half = w >> 2, tw = w & 3;  // block parity, token group
  const int r = lane & 31, g = lane >> 5;
  S1Token<D, LR, LAYERED> tk;
  tk.load(kh, vh, lr0, lr1, lr2, ly, N, bh, blockIdx.x * kUpdTok + 32 * tw + r, g);
  const uint16_t* ph = packed + (int64_t)bh * 3 * I * D;
  const int64_t part = (int64_t)I * D;
  uint16_t* dyr = dy + tk.row * 2 * I + 16 * g;
  uint16_t* hr = hid + tk.row * I + 16 * g;
  const int nblk = I / 32, npair = (nblk + 1) / 2;

  // pair p's fragment f (block 2 p + f / (3 KS) clamped to the last block,
  // part, k step) straight into the LDS stage at f KiB
  auto issue = [&](uint4 (&dst)[kPairChunks], int p) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kFragsPerWave; ++i) {
      const int f = w + kStgWaves * i;  // wave-uniform
      if (kFrags % kStgWaves == 0 || f < kFrags) {
        const int slot = f / (3 * KS), rem = f - slot * (3 * KS);
        const int pt = rem / KS, s = rem - pt * KS;
        const int blk = min(2 * p + slot, nblk - 1);
        const uint16_t* src = ph + pt * part + ((int64_t)blk * KS + s) * 64 * 8 + lane * 8;
        __builtin_amdgcn_global_load_lds(
            src, (__attribute__((address_space(3))) void*)(&dst[f * 64]), 16, 0, 0);
      }
    }
  };
  auto step = [&](const uint4 (&cur)[kPairChunks], uint4 (&nxt)[kPairChunks], int p)
      __attribute__((always_inline)) {
    const int blk = 2 * p + half;
    if (p + 1 < npair) issue(nxt, p + 1);
    const bool mine = blk < nblk;  // wave-uniform
    f32x16_t y0, y2, dh;
#pragma unroll
    for (int v = 0; v < 16; ++v) y0[v] = y2[v] = dh[v] = 0.0f;
    if (mine) {
      // fragment (part, k step s) of this wave's block at base + 1 KiB
      // (part KS + s); step s + 1's three reads issue before step s's MFMAs
      const uint32_t base = (uint32_t)(uintptr_t)(
          (const __attribute__((address_space(3))) uint4*)(&cur[half * kBlkChunks + lane]));
      s1_i32x4 f0 = s1_ds_read(base), f2 = s1_ds_read(base + (KS << 10)),
               f1 = s1_ds_read(base + (2 * KS << 10));
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        s1_i32x4 n0, n2, n1;
        if (s + 1 < KS) {
          n0 = s1_ds_read(base + ((s + 1) << 10));
          n2 = s1_ds_read(base + ((KS + s + 1) << 10));
          n1 = s1_ds_read(base + ((2 * KS + s + 1) << 10));
          s1_lgkm_wait<3>(f0, f2, f1);
        } else {
          s1_lgkm_wait<0>(f0, f2, f1);
        }
        y0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, f0), tk.kf[s],
                                                     y0, 0, 0, 0);
        y2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, f2), tk.kf[s],
                                                     y2, 0, 0, 0);
        dh = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, f1), tk.vf[s],
                                                     dh, 0, 0, 0);
        if (s + 1 < KS) {
          f0 = n0;
          f2 = n2;
          f1 = n1;
        }
      }
    }
    // the next pair's loads have landed before this block's stores issue
    // (tied to the accumulators, so it stays after this block's MFMAs)
    asm volatile("s_waitcnt vmcnt(0)" : "+v"(y0), "+v"(y2), "+v"(dh) :: "memory");
    if (mine) tk.epilogue(y0, y2, dh, dyr, hr, I, blk);
    s1_lds_barrier();  // every wave's loads into nxt are in, every read of cur done
  };

  issue(st0, 0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  s1_lds_barrier();
  for (int p = 0; p < npair; p += 2) {
    step(st0, st1, p);
    if (p + 1 >= npair) break;
    step(st1, st0, p + 1);
  }
}

template <int D, class LR = F32T, bool LAYERED = false>
void launch_update_s1(int BH, int N, int I, hipStream_t st, const uint16_t* k, const uint16_t* v,
                      const float* a, const float* b, const float* c, const uint16_t* p,
                      uint16_t* o, uint16_t* h, const S1Layers& ly = S1Layers{}) {
  const dim3 grid((unsigned)((N + kUpdTok - 1) / kUpdTok), (unsigned)BH);
  // the staged kernel where the grid fills the chip (configs[1]'s write:
  // 768 workgroups, 100 -> 89 us); on small grids (configs[0]: 16) its
  // per-pair load wait and barrier cost more than the shared loads save
  // (50.5 -> 56.7 us), and the four-wave kernel with register prefetch runs
  if constexpr (D <= 192) {
    if ((int64_t)grid.x * grid.y >= g_s1_staged_min_grid) {
      hipLaunchKernelGGL((dense_update_s1_staged_kernel<D, LR, LAYERED>), grid,
                         dim3(kStgWaves * 64), 0, st, k, v, a, b, c, ly, N, I, p, o, h);
      return;
    }
  }
  hipLaunchKernelGGL((dense_update_s1_kernel<D, (D <= 192), LR, LAYERED>), grid,
                     dim3(kUpdWaves * 64), 0, st, k, v, a, b, c, ly, N, I, p, o, h);
}

}  // namespace
}  // namespace uttt

using namespace uttt;

extern "C" int uttt_debug_set_s1_staged(int mode) {
  UTTT_REQUIRE(mode >= 0 && mode <= 2, "debug_set_s1_staged: mode=%d (0, 1 or 2)", mode);
  const int prev = g_s1_staged_min_grid == 256 ? 0 : g_s1_staged_min_grid == 0 ? 1 : 2;
  g_s1_staged_min_grid = mode == 0 ? 256 : mode == 1 ? 0 : 0x7fffffff;
  return prev;
}

extern "C" int uttt_dense_update_supported(int D, int I) {
  return (D == 64 || D == 96 || D == 128 || D == 192 || D == 256) && I >= 32 && I <= 512 &&
         I % 32 == 0;
}

extern "C" int uttt_dense_pack_update_weights(const void* w0_w2, const void* w1, int BH, int D,
                                              int I, void* packed, void* stream) {
  UTTT_REQUIRE(BH >= 0, "dense_pack_update_weights: bad sizes");
  UTTT_REQUIRE(uttt_dense_update_supported(D, I),
               "dense_pack_update_weights: D=%d must be 64, 96, 128, 192 or 256 and I=%d a "
               "multiple of 32 in [32, 512]", D, I);
  if (BH == 0) return UTTT_OK;
  UTTT_REQUIRE(BH <= 65535, "dense_pack_update_weights: BH=%d exceeds 65535", BH);
  UTTT_REQUIRE(w0_w2 && w1 && packed, "dense_pack_update_weights: null pointer");
  UTTT_REQUIRE(aligned16(w0_w2) && aligned16(packed),
               "dense_pack_update_weights: w0_w2 and packed must be 16-byte aligned");
  const int nch = 3 * I * D / 8;
  hipLaunchKernelGGL(dense_pack_update_kernel, dim3((unsigned)((nch + 255) / 256), (unsigned)BH),
                     dim3(256), 0, as_stream(stream), static_cast<const uint16_t*>(w0_w2),
                     static_cast<const uint16_t*>(w1), D, I, static_cast<uint16_t*>(packed));
  return check_launch("dense_pack_update_weights");
}

extern "C" int uttt_dense_update_stage1(const void* kh, const void* vh, const void* lr0,
                                        const void* lr1, const void* lr2, int BH, int N, int D,
                                        int I, const void* packed, void* dy, void* hid,
                                        void* stream) {
  UTTT_REQUIRE(BH >= 0 && N >= 0, "dense_update_stage1: bad sizes");
  UTTT_REQUIRE(uttt_dense_update_supported(D, I),
               "dense_update_stage1: D=%d must be 64, 96, 128, 192 or 256 and I=%d a multiple "
               "of 32 in [32, 512]", D, I);
  if (BH == 0 || N == 0) return UTTT_OK;
  UTTT_REQUIRE(BH <= 65535, "dense_update_stage1: BH=%d exceeds 65535", BH);
  UTTT_REQUIRE(kh && vh && packed && dy && hid, "dense_update_stage1: null pointer");
  UTTT_REQUIRE(aligned16(kh) && aligned16(vh) && aligned16(packed) && aligned16(dy) &&
                   aligned16(hid),
               "dense_update_stage1: k, v, packed, dy and hid must be 16-byte aligned");
  UTTT_REQUIRE((lr0 == nullptr) == (lr1 == nullptr) && (lr0 == nullptr) == (lr2 == nullptr),
               "dense_update_stage1: give all three lr or none");
  hipStream_t st = as_stream(stream);
  const auto* k = static_cast<const uint16_t*>(kh);
  const auto* v = static_cast<const uint16_t*>(vh);
  const auto* a = static_cast<const float*>(lr0);
  const auto* b = static_cast<const float*>(lr1);
  const auto* c = static_cast<const float*>(lr2);
  const auto* p = static_cast<const uint16_t*>(packed);
  auto* o = static_cast<uint16_t*>(dy);
  auto* h = static_cast<uint16_t*>(hid);
  switch (D) {
    case 64: launch_update_s1<64>(BH, N, I, st, k, v, a, b, c, p, o, h); break;
    case 96: launch_update_s1<96>(BH, N, I, st, k, v, a, b, c, p, o, h); break;
    case 128: launch_update_s1<128>(BH, N, I, st, k, v, a, b, c, p, o, h); break;
    case 192: launch_update_s1<192>(BH, N, I, st, k, v, a, b, c, p, o, h); break;
    default: launch_update_s1<256>(BH, N, I, st, k, v, a, b, c, p, o, h); break;
  }
  return check_launch("dense_update_stage1");
}

extern "C" int uttt_dense_update_stage1_layers(const void* const* k_layers,
                                               const void* const* v_layers,
                                               const void* const* lr_layers, int lr_dtype,
                                               int lr_per_head, int L, int b, int l, int H, int D,
                                               int I, const void* packed, void* dy, void* hid,
                                               void* stream) {
  UTTT_REQUIRE(L >= 0 && L <= kMaxLayers && b >= 0 && l >= 0 && H >= 1,
               "dense_update_stage1_layers: bad sizes (L=%d must be at most %d)", L, kMaxLayers);
  UTTT_REQUIRE(uttt_dense_update_supported(D, I),
               "dense_update_stage1_layers: D=%d must be 64, 96, 128, 192 or 256 and I=%d a "
               "multiple of 32 in [32, 512]", D, I);
  if (L == 0 || b == 0 || l == 0) return UTTT_OK;
  UTTT_REQUIRE(l % 32 == 0, "dense_update_stage1_layers: l=%d must be a multiple of 32", l);
  const int BH = b * H;
  const int64_t N = (int64_t)L * l;
  UTTT_REQUIRE(BH <= 65535 && N < ((int64_t)1 << 31) && (int64_t)b * l * H * D < ((int64_t)1 << 40),
               "dense_update_stage1_layers: sizes too large");
  UTTT_REQUIRE(k_layers && v_layers && packed && dy && hid,
               "dense_update_stage1_layers: null pointer");
  UTTT_REQUIRE(aligned16(packed) && aligned16(dy) && aligned16(hid),
               "dense_update_stage1_layers: packed, dy and hid must be 16-byte aligned");
  S1Layers ly{};
  ly.l = l;
  ly.H = H;
  ly.lr_per_head = lr_per_head ? 1 : 0;
  for (int i = 0; i < L; ++i) {
    UTTT_REQUIRE(k_layers[i] && v_layers[i] && aligned16(k_layers[i]) && aligned16(v_layers[i]),
                 "dense_update_stage1_layers: layer %d's k and v must be 16-byte aligned", i);
    ly.k.p[i] = k_layers[i];
    ly.v.p[i] = v_layers[i];
    ly.lr.p[i] = lr_layers ? lr_layers[i] : nullptr;
    UTTT_REQUIRE(lr_layers == nullptr || lr_layers[i] != nullptr,
                 "dense_update_stage1_layers: null lr of layer %d", i);
  }
  hipStream_t st = as_stream(stream);
  const auto* p = static_cast<const uint16_t*>(packed);
  auto* o = static_cast<uint16_t*>(dy);
  auto* h = static_cast<uint16_t*>(hid);
  const int n = (int)N;
  UTTT_DTYPE_SWITCH_LR(lr_dtype, LR, {
    switch (D) {
      case 64: launch_update_s1<64, LR, true>(BH, n, I, st, nullptr, nullptr, nullptr, nullptr, nullptr, p, o, h, ly); break;
      case 96: launch_update_s1<96, LR, true>(BH, n, I, st, nullptr, nullptr, nullptr, nullptr, nullptr, p, o, h, ly); break;
      case 128: launch_update_s1<128, LR, true>(BH, n, I, st, nullptr, nullptr, nullptr, nullptr, nullptr, p, o, h, ly); break;
      case 192: launch_update_s1<192, LR, true>(BH, n, I, st, nullptr, nullptr, nullptr, nullptr, nullptr, p, o, h, ly); break;
      default: launch_update_s1<256, LR, true>(BH, n, I, st, nullptr, nullptr, nullptr, nullptr, nullptr, p, o, h, ly); break;
    }
  });
  return check_launch("dense_update_stage1_layers");
}
