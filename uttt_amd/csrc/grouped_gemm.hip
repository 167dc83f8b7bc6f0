// Grouped SwiGLU fast-weight GEMMs for gfx950 (bf16 MFMA, fp32 accumulate).
//
// Notation per group (batch b, expert e): the expert's routed tokens are the
// contiguous segment seg(b,e) of the permuted token axis (lengths from
// group_sizes[b, e], in expert order); w0 = W0_W2[b,e,:I], w2 = W0_W2[b,e,I:],
// w1 = W1[b,e] ([D, I]).
//
//   gate_up   (APPLY, first half)   H[n, i]  = silu(w0 x_n)_i * (w2 x_n)_i
//   gemm_nt   (APPLY, down proj)    Y[n, m]  = sum_k W[m, k] X[n, k]
//   update_s1 (UPDATE, stage 1)     Y0 = w0 k_n, Y2 = w2 k_n, DH = w1^T v_n ->
//       DY0 = lr0 sig(Y0) Y2 DH (1 + Y0 (1 - sig(Y0))), DY2 = lr2 silu(Y0) DH,
//       Hid = lr1 silu(Y0) Y2
//   wgrad     (UPDATE, stage 2)     dW[m, c] = sum_{n in seg} A[n, m] B[n, c]
//
// Intermediates (H, DY0_DY2, Hid) are written token-major ([B, N, rows]) on
// the fused path so that every operand is read with 16-byte vectors: the
// tokens of a segment start anywhere, and only the token index may be
// unaligned.  The kernel-level compat entry points can also write the
// reference's [B, rows, N] layout.
#include "gemm_core.h"

namespace uttt {
namespace {

using namespace gemm;

__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

// ------------------------------------------------------------ store helpers
// Four consecutive-row results (rows m..m+3 of column n) as one 8-byte store
// into a token-major [.., N, ld] buffer (m is a multiple of 4).
__device__ __forceinline__ void store4_tok(uint16_t* out, int64_t ld, int n, int m,
                                           float a, float b, float c, float d) {
  uint2 w;
  w.x = (uint32_t)f32_to_bf16(a) | ((uint32_t)f32_to_bf16(b) << 16);
  w.y = (uint32_t)f32_to_bf16(c) | ((uint32_t)f32_to_bf16(d) << 16);
  *reinterpret_cast<uint2*>(out + (int64_t)n * ld + m) = w;
}

// ======================================================= APPLY: gate / up ==
// Grid: x = m_tiles * n_tiles_ub * B (m fastest).  LDS: two stages of
// [w0 tile | w2 tile | x tile].
template <int BM, int BN>
__global__ __launch_bounds__(kThreads) void gate_up_kernel(
    const uint16_t* __restrict__ w02, const uint16_t* __restrict__ x,
    const int32_t* __restrict__ gs, uint16_t* __restrict__ hid, int E, int I, int D, int N,
    int m_tiles, int n_tiles_ub, int token_major) {
  constexpr int MB = BM / 64, NB = BN / 64;
  constexpr int kStage = (2 * BM + BN) * kLdsRow;
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * kStage];
  __shared__ int scratch[4];

  const int bid = blockIdx.x;
  const int mt = bid % m_tiles;
  const int nt = (bid / m_tiles) % n_tiles_ub;
  const int b = bid / (m_tiles * n_tiles_ub);
  const TokenTile tt = find_token_tile<BN>(gs + (int64_t)b * E, E, N, nt, scratch);
  if (tt.e < 0) return;
  const int m0 = mt * BM;

  const uint16_t* wbase = w02 + ((int64_t)b * E + tt.e) * 2 * I * D;
  const Operand A0{wbase, D, I, D};
  const Operand A1{wbase + (int64_t)I * D, D, I, D};
  const Operand B0{x + ((int64_t)b * N + tt.start) * D, D, tt.size, D};

  TileRegs<BM, KMajor> ra0, ra1;
  TileRegs<BN, KMajor> rb0;
  f32x16 acc0[MB][NB], acc2[MB][NB];
  zero_acc(acc0);
  zero_acc(acc2);

  ra0.load(A0, m0, 0);
  ra1.load(A1, m0, 0);
  rb0.load(B0, tt.n0, 0);
  ra0.store(lds);
  ra1.store(lds + BM * kLdsRow);
  rb0.store(lds + 2 * BM * kLdsRow);
  __syncthreads();

  const int w = wave_id();
  const int wa = (w >> 1) * (BM / 2) * kLdsRow;
  const int wb = (w & 1) * (BN / 2) * kLdsRow;
  int cur = 0;
  for (int k0 = 0; k0 < D; k0 += kBK) {
    const bool next = k0 + kBK < D;
    if (next) {
      ra0.load(A0, m0, k0 + kBK);
      ra1.load(A1, m0, k0 + kBK);
      rb0.load(B0, tt.n0, k0 + kBK);
    }
    const uint16_t* st = lds + cur * kStage;
    mma_stage<MB, NB>(acc0, st + wa, st + 2 * BM * kLdsRow + wb);
    mma_stage<MB, NB>(acc2, st + BM * kLdsRow + wa, st + 2 * BM * kLdsRow + wb);
    if (next) {
      uint16_t* nx = lds + (cur ^ 1) * kStage;
      ra0.store(nx);
      ra1.store(nx + BM * kLdsRow);
      rb0.store(nx + 2 * BM * kLdsRow);
    }
    __syncthreads();
    cur ^= 1;
  }

  // epilogue: h = y2 * y0 * sigmoid(y0), bf16
  uint16_t* hb = hid + (int64_t)b * N * I;
  const int mw = m0 + (w >> 1) * (BM / 2);
  const int nw = tt.n0 + (w & 1) * (BN / 2);
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int n = nw + j * 32 + acc_col();
      if (n >= tt.size) continue;
      const int tok = tt.start + n;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = mw + i * 32 + acc_row(q * 4);
        if (m >= I) continue;
        float h[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float y0 = acc0[i][j][q * 4 + r];
          const float y2 = acc2[i][j][q * 4 + r];
          h[r] = y2 * (y0 * sigmoidf_(y0));
        }
        if (token_major) {
          store4_tok(hb, I, tok, m, h[0], h[1], h[2], h[3]);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) hb[(int64_t)(m + r) * N + tok] = f32_to_bf16(h[r]);
        }
      }
    }
}

// ============================================= APPLY: down projection / NT ==
// Y[b, tok, m] = sum_p sum_k W_p[b, e, m, k] X_p[b, tok, k] for tok in
// seg(b, e), over NPAIR operand pairs accumulated into one result (NPAIR = 1:
// the down projection; NPAIR = 2: the UPDATE backward's grad_K / grad_V).
// AMAJOR = KMajor: W stored [M, K]; RMajor: W stored [K, M] (the product with
// W^T, e.g. grad_X = W0_W2^T DY).
struct NtPair {
  const uint16_t* w;
  const uint16_t* x;
};

template <int BM, int BN, int AMAJOR, int NPAIR>
__global__ __launch_bounds__(kThreads) void gemm_nt_kernel(
    NtPair p0, NtPair p1, const int32_t* __restrict__ gs, uint16_t* __restrict__ y, int E, int M,
    int K, int N, int m_tiles, int n_tiles_ub) {
  constexpr int MB = BM / 64, NB = BN / 64;
  constexpr int kPair = (BM + BN) * kLdsRow;
  constexpr int kStage = NPAIR * kPair;
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * kStage];
  __shared__ int scratch[4];

  const int bid = blockIdx.x;
  const int mt = bid % m_tiles;
  const int nt = (bid / m_tiles) % n_tiles_ub;
  const int b = bid / (m_tiles * n_tiles_ub);
  const TokenTile tt = find_token_tile<BN>(gs + (int64_t)b * E, E, N, nt, scratch);
  if (tt.e < 0) return;
  const int m0 = mt * BM;

  const int64_t woff = ((int64_t)b * E + tt.e) * M * K;
  const int64_t xoff = ((int64_t)b * N + tt.start) * K;
  const int64_t lda = AMAJOR == KMajor ? K : M;
  Operand A[NPAIR], Bo[NPAIR];
  A[0] = Operand{p0.w + woff, lda, M, K};
  Bo[0] = Operand{p0.x + xoff, K, tt.size, K};
  if constexpr (NPAIR > 1) {
    A[1] = Operand{p1.w + woff, lda, M, K};
    Bo[1] = Operand{p1.x + xoff, K, tt.size, K};
  }
  TileRegs<BM, AMAJOR> ra[NPAIR];
  TileRegs<BN, KMajor> rb[NPAIR];
  f32x16 acc[MB][NB];
  zero_acc(acc);

#pragma unroll
  for (int q = 0; q < NPAIR; ++q) {
    ra[q].load(A[q], m0, 0);
    rb[q].load(Bo[q], tt.n0, 0);
    ra[q].store(lds + q * kPair);
    rb[q].store(lds + q * kPair + BM * kLdsRow);
  }
  __syncthreads();

  const int w = wave_id();
  const int wa = (w >> 1) * (BM / 2) * kLdsRow;
  const int wb = (w & 1) * (BN / 2) * kLdsRow;
  int cur = 0;
  for (int k0 = 0; k0 < K; k0 += kBK) {
    const bool next = k0 + kBK < K;
    if (next) {
#pragma unroll
      for (int q = 0; q < NPAIR; ++q) {
        ra[q].load(A[q], m0, k0 + kBK);
        rb[q].load(Bo[q], tt.n0, k0 + kBK);
      }
    }
    const uint16_t* st = lds + cur * kStage;
#pragma unroll
    for (int q = 0; q < NPAIR; ++q)
      mma_stage<MB, NB>(acc, st + q * kPair + wa, st + q * kPair + BM * kLdsRow + wb);
    if (next) {
      uint16_t* nx = lds + (cur ^ 1) * kStage;
#pragma unroll
      for (int q = 0; q < NPAIR; ++q) {
        ra[q].store(nx + q * kPair);
        rb[q].store(nx + q * kPair + BM * kLdsRow);
      }
    }
    __syncthreads();
    cur ^= 1;
  }

  uint16_t* yb = y + (int64_t)b * N * M;
  const int mw = m0 + (w >> 1) * (BM / 2);
  const int nw = tt.n0 + (w & 1) * (BN / 2);
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int n = nw + j * 32 + acc_col();
      if (n >= tt.size) continue;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = mw + i * 32 + acc_row(q * 4);
        if (m >= M) continue;
        store4_tok(yb, M, tt.start + n, m, acc[i][j][q * 4 + 0], acc[i][j][q * 4 + 1],
                   acc[i][j][q * 4 + 2], acc[i][j][q * 4 + 3]);
      }
    }
}

// ================================================== UPDATE stage 1 =========
// Three accumulators: Y0 = w0 K^T, Y2 = w2 K^T (sharing the K tile) and
// DH = w1^T V^T (w1 read transposed from [D, I]).  LR is the storage type of
// the per-token learning rates (widened to fp32).
template <int BM, int BN, class LR>
__global__ __launch_bounds__(kThreads) void update_s1_kernel(
    const uint16_t* __restrict__ w02, const uint16_t* __restrict__ w1,
    const uint16_t* __restrict__ kk, const uint16_t* __restrict__ vv,
    const typename LR::S* __restrict__ lr0, const typename LR::S* __restrict__ lr1,
    const typename LR::S* __restrict__ lr2, const int32_t* __restrict__ gs,
    uint16_t* __restrict__ dy, uint16_t* __restrict__ hid, int E, int I, int D, int N,
    int m_tiles, int n_tiles_ub, int token_major) {
  constexpr int MB = BM / 64, NB = BN / 64;
  constexpr int kStage = (3 * BM + 2 * BN) * kLdsRow;
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * kStage];
  __shared__ int scratch[4];

  const int bid = blockIdx.x;
  const int mt = bid % m_tiles;
  const int nt = (bid / m_tiles) % n_tiles_ub;
  const int b = bid / (m_tiles * n_tiles_ub);
  const TokenTile tt = find_token_tile<BN>(gs + (int64_t)b * E, E, N, nt, scratch);
  if (tt.e < 0) return;
  const int m0 = mt * BM;

  const uint16_t* wbase = w02 + ((int64_t)b * E + tt.e) * 2 * I * D;
  const Operand A0{wbase, D, I, D};
  const Operand A1{wbase + (int64_t)I * D, D, I, D};
  const Operand A2{w1 + ((int64_t)b * E + tt.e) * D * I, I, I, D};  // (r=i, k=d) at d*I + i
  const Operand B0{kk + ((int64_t)b * N + tt.start) * D, D, tt.size, D};
  const Operand B1{vv + ((int64_t)b * N + tt.start) * D, D, tt.size, D};

  TileRegs<BM, KMajor> ra0, ra1;
  TileRegs<BM, RMajor> ra2;
  TileRegs<BN, KMajor> rb0, rb1;
  f32x16 ay0[MB][NB], ay2[MB][NB], adh[MB][NB];
  zero_acc(ay0);
  zero_acc(ay2);
  zero_acc(adh);

  constexpr int oA1 = BM * kLdsRow, oA2 = 2 * BM * kLdsRow;
  constexpr int oB0 = 3 * BM * kLdsRow, oB1 = 3 * BM * kLdsRow + BN * kLdsRow;
  ra0.load(A0, m0, 0);
  ra1.load(A1, m0, 0);
  ra2.load(A2, m0, 0);
  rb0.load(B0, tt.n0, 0);
  rb1.load(B1, tt.n0, 0);
  ra0.store(lds);
  ra1.store(lds + oA1);
  ra2.store(lds + oA2);
  rb0.store(lds + oB0);
  rb1.store(lds + oB1);
  __syncthreads();

  const int w = wave_id();
  const int wa = (w >> 1) * (BM / 2) * kLdsRow;
  const int wb = (w & 1) * (BN / 2) * kLdsRow;
  int cur = 0;
  for (int k0 = 0; k0 < D; k0 += kBK) {
    const bool next = k0 + kBK < D;
    if (next) {
      ra0.load(A0, m0, k0 + kBK);
      ra1.load(A1, m0, k0 + kBK);
      ra2.load(A2, m0, k0 + kBK);
      rb0.load(B0, tt.n0, k0 + kBK);
      rb1.load(B1, tt.n0, k0 + kBK);
    }
    const uint16_t* st = lds + cur * kStage;
    mma_stage<MB, NB>(ay0, st + wa, st + oB0 + wb);
    mma_stage<MB, NB>(ay2, st + oA1 + wa, st + oB0 + wb);
    mma_stage<MB, NB>(adh, st + oA2 + wa, st + oB1 + wb);
    if (next) {
      uint16_t* nx = lds + (cur ^ 1) * kStage;
      ra0.store(nx);
      ra1.store(nx + oA1);
      ra2.store(nx + oA2);
      rb0.store(nx + oB0);
      rb1.store(nx + oB1);
    }
    __syncthreads();
    cur ^= 1;
  }

  const int I2 = 2 * I;
  uint16_t* dyb = dy + (int64_t)b * N * I2;
  uint16_t* hb = hid + (int64_t)b * N * I;
  const int mw = m0 + (w >> 1) * (BM / 2);
  const int nw = tt.n0 + (w & 1) * (BN / 2);
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const int n = nw + j * 32 + acc_col();
    if (n >= tt.size) continue;
    const int tok = tt.start + n;
    const int64_t li = (int64_t)b * N + tok;
    const float l0 = lr0 ? LR::load(lr0[li]) : 1.0f;
    const float l1 = lr1 ? LR::load(lr1[li]) : 1.0f;
    const float l2 = lr2 ? LR::load(lr2[li]) : 1.0f;
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = mw + i * 32 + acc_row(q * 4);
        if (m >= I) continue;
        float d0[4], d2[4], hh[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float y0 = ay0[i][j][q * 4 + r];
          const float y2 = ay2[i][j][q * 4 + r];
          const float dh = adh[i][j][q * 4 + r];
          const float sg = sigmoidf_(y0);
          const float sw = sg * y0;
          d0[r] = sg * y2 * dh * (1.0f + y0 * (1.0f - sg)) * l0;
          d2[r] = sw * dh * l2;
          hh[r] = sw * y2 * l1;
        }
        if (token_major) {
          store4_tok(dyb, I2, tok, m, d0[0], d0[1], d0[2], d0[3]);
          store4_tok(dyb, I2, tok, I + m, d2[0], d2[1], d2[2], d2[3]);
          store4_tok(hb, I, tok, m, hh[0], hh[1], hh[2], hh[3]);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            dyb[(int64_t)(m + r) * N + tok] = f32_to_bf16(d0[r]);
            dyb[(int64_t)(I + m + r) * N + tok] = f32_to_bf16(d2[r]);
            hb[(int64_t)(m + r) * N + tok] = f32_to_bf16(hh[r]);
          }
        }
      }
  }
}

// ================================================== weight gradients =======
// Weight-gradient products with the routed tokens as the reduction axis:
//   out[b, e, m, c] = sum_{n in seg(b,e)} A[b, n, m] * Bop[b, n, c]
// with A [B, N, R] and Bop [B, N, C] token-major (rows contiguous).  Up to two
// such tasks share one launch (the UPDATE's dW0_W2 and dW1); `transposed`
// stores out as [C, R] instead of [R, C].  An empty segment writes zeros.
struct WgradTask {
  const uint16_t* a;
  const uint16_t* b;
  uint16_t* out;
  int R, C;
  int transposed;
  int m_tiles, c_tiles;
};

template <int BM, int BN>
__global__ __launch_bounds__(kThreads) void wgrad_kernel(WgradTask t0, WgradTask t1,
                                                         const int32_t* __restrict__ gs, int E,
                                                         int N) {
  constexpr int MB = BM / 64, NB = BN / 64;
  constexpr int kStage = (BM + BN) * kLdsRow;
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * kStage];

  const int n0_tiles = t0.m_tiles * t0.c_tiles;
  const int tiles_per_group = n0_tiles + t1.m_tiles * t1.c_tiles;
  const int bid = blockIdx.x;
  const int t = bid % tiles_per_group;
  const int be = bid / tiles_per_group;
  const int b = be / E, e = be % E;
  const WgradTask& tk = t < n0_tiles ? t0 : t1;
  const int tl = t < n0_tiles ? t : t - n0_tiles;
  const int m0 = (tl / tk.c_tiles) * BM, c0 = (tl % tk.c_tiles) * BN;
  const int R = tk.R, C = tk.C;

  int start, size;
  expert_segment(gs + (int64_t)b * E, e, N, &start, &size);
  const Operand A0{tk.a + ((int64_t)b * N + start) * R, R, R, size};
  const Operand B0{tk.b + ((int64_t)b * N + start) * C, C, C, size};

  TileRegs<BM, RMajor> ra0;
  TileRegs<BN, RMajor> rb0;
  f32x16 acc[MB][NB];
  zero_acc(acc);

  ra0.load(A0, m0, 0);
  rb0.load(B0, c0, 0);
  ra0.store(lds);
  rb0.store(lds + BM * kLdsRow);
  __syncthreads();

  const int w = wave_id();
  const int wa = (w >> 1) * (BM / 2) * kLdsRow;
  const int wb = (w & 1) * (BN / 2) * kLdsRow;
  int cur = 0;
  for (int k0 = 0; k0 < size; k0 += kBK) {
    const bool next = k0 + kBK < size;
    if (next) {
      ra0.load(A0, m0, k0 + kBK);
      rb0.load(B0, c0, k0 + kBK);
    }
    const uint16_t* st = lds + cur * kStage;
    mma_stage<MB, NB>(acc, st + wa, st + BM * kLdsRow + wb);
    if (next) {
      uint16_t* nx = lds + (cur ^ 1) * kStage;
      ra0.store(nx);
      rb0.store(nx + BM * kLdsRow);
    }
    __syncthreads();
    cur ^= 1;
  }

  const int mw = m0 + (w >> 1) * (BM / 2);
  const int cw = c0 + (w & 1) * (BN / 2);
  uint16_t* ob = tk.out + ((int64_t)b * E + e) * R * C;
  if (!tk.transposed) {  // [R, C]
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const int c = cw + j * 32 + acc_col();
        if (c >= C) continue;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int m = mw + i * 32 + acc_row(v);
          if (m < R) ob[(int64_t)m * C + c] = f32_to_bf16(acc[i][j][v]);
        }
      }
  } else {  // [C, R]: four consecutive m of one c are one 8-byte store
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const int c = cw + j * 32 + acc_col();
        if (c >= C) continue;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int m = mw + i * 32 + acc_row(q * 4);
          if (m >= R) continue;
          store4_tok(ob, R, c, m, acc[i][j][q * 4 + 0], acc[i][j][q * 4 + 1],
                     acc[i][j][q * 4 + 2], acc[i][j][q * 4 + 3]);
        }
      }
  }
}

// ============================================ UPDATE backward, stage 1 ======
// Backward of the UPDATE op given the upstream gradients GW0_W2 = dL/dDW0_W2
// and GW1 = dL/dDW1.  Six accumulators per tile:
//   Y0, Y2 = w0 k, w2 k;  GY0, GY2 = gw0 k, gw2 k;  DH = w1^T v;  GDH = gw1^T v
// each rounded to bf16 (the reference stores them bf16 between its four-GEMM
// kernel and its pointwise pass), then the second-order SwiGLU pointwise pass
// in fp32 in the epilogue.  Writes token-major bf16 dx0_x2 / grad_x0_x2
// ([N, 2I]), grad_dh / hidden_lr1 ([N, I]) and, per m-tile, fp32 partial
// sums over the tile's hidden rows of the three learning-rate gradients
// (lr_part[3][m_tiles][B][N]).
__device__ __forceinline__ float bf16r(float x) { return bf16_to_f32(f32_to_bf16(x)); }

template <int BM, int BN, class LR>
__global__ __launch_bounds__(kThreads) void update_bwd_s1_kernel(
    const uint16_t* __restrict__ w02, const uint16_t* __restrict__ w1,
    const uint16_t* __restrict__ gw02, const uint16_t* __restrict__ gw1,
    const uint16_t* __restrict__ kk, const uint16_t* __restrict__ vv,
    const typename LR::S* __restrict__ lr0, const typename LR::S* __restrict__ lr1,
    const typename LR::S* __restrict__ lr2, const int32_t* __restrict__ gs,
    uint16_t* __restrict__ dx02, uint16_t* __restrict__ gx02, uint16_t* __restrict__ gdh,
    uint16_t* __restrict__ hlr, float* __restrict__ lr_part, int B, int E, int I, int D, int N,
    int m_tiles, int n_tiles_ub) {
  constexpr int MB = BM / 64, NB = BN / 64;
  static_assert(NB == 1, "one 32-column block per wave");
  constexpr int kA = BM * kLdsRow, kB = BN * kLdsRow;
  constexpr int kStage = 6 * kA + 2 * kB;
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * kStage];
  __shared__ int scratch[4];
  __shared__ float red[3][2][BN];  // lr partials of the two row-halves of the tile

  const int bid = blockIdx.x;
  const int mt = bid % m_tiles;
  const int nt = (bid / m_tiles) % n_tiles_ub;
  const int b = bid / (m_tiles * n_tiles_ub);
  const TokenTile tt = find_token_tile<BN>(gs + (int64_t)b * E, E, N, nt, scratch);
  if (tt.e < 0) return;
  const int m0 = mt * BM;

  const int64_t we = ((int64_t)b * E + tt.e) * 2 * I * D;
  const int64_t w1e = ((int64_t)b * E + tt.e) * D * I;
  Operand A[6] = {
      Operand{w02 + we, D, I, D},
      Operand{w02 + we + (int64_t)I * D, D, I, D},
      Operand{gw02 + we, D, I, D},
      Operand{gw02 + we + (int64_t)I * D, D, I, D},
      Operand{w1 + w1e, I, I, D},    // w1^T: (r=i, k=d) at d*I + i
      Operand{gw1 + w1e, I, I, D},
  };
  const Operand B0{kk + ((int64_t)b * N + tt.start) * D, D, tt.size, D};
  const Operand B1{vv + ((int64_t)b * N + tt.start) * D, D, tt.size, D};

  TileRegs<BM, KMajor> ra[4];
  TileRegs<BM, RMajor> rt[2];
  TileRegs<BN, KMajor> rb0, rb1;
  f32x16 acc[6][MB][NB];
#pragma unroll
  for (int q = 0; q < 6; ++q) zero_acc(acc[q]);

  auto load = [&](int k0) {
#pragma unroll
    for (int q = 0; q < 4; ++q) ra[q].load(A[q], m0, k0);
    rt[0].load(A[4], m0, k0);
    rt[1].load(A[5], m0, k0);
    rb0.load(B0, tt.n0, k0);
    rb1.load(B1, tt.n0, k0);
  };
  auto store = [&](uint16_t* st) {
#pragma unroll
    for (int q = 0; q < 4; ++q) ra[q].store(st + q * kA);
    rt[0].store(st + 4 * kA);
    rt[1].store(st + 5 * kA);
    rb0.store(st + 6 * kA);
    rb1.store(st + 6 * kA + kB);
  };
  load(0);
  store(lds);
  __syncthreads();

  const int w = wave_id();
  const int wa = (w >> 1) * (BM / 2) * kLdsRow;
  const int wb = (w & 1) * (BN / 2) * kLdsRow;
  int cur = 0;
  for (int k0 = 0; k0 < D; k0 += kBK) {
    const bool next = k0 + kBK < D;
    if (next) load(k0 + kBK);
    const uint16_t* st = lds + cur * kStage;
#pragma unroll
    for (int q = 0; q < 4; ++q) mma_stage<MB, NB>(acc[q], st + q * kA + wa, st + 6 * kA + wb);
    mma_stage<MB, NB>(acc[4], st + 4 * kA + wa, st + 6 * kA + kB + wb);
    mma_stage<MB, NB>(acc[5], st + 5 * kA + wa, st + 6 * kA + kB + wb);
    if (next) store(lds + (cur ^ 1) * kStage);
    __syncthreads();
    cur ^= 1;
  }

  const int I2 = 2 * I;
  const int mw = m0 + (w >> 1) * (BM / 2);
  const int ncol = (w & 1) * (BN / 2) + acc_col();   // column inside the tile
  const int n = tt.n0 + ncol;
  const bool nvalid = n < tt.size;
  const int tok = tt.start + n;
  float L0 = 0.f, L1 = 0.f, L2 = 0.f;
  if (nvalid) {
    const int64_t li = (int64_t)b * N + tok;
    L0 = LR::load(lr0[li]);
    L1 = LR::load(lr1[li]);
    L2 = LR::load(lr2[li]);
  }
  float s0 = 0.f, s1 = 0.f, s2 = 0.f;
  uint16_t* dxb = dx02 + (int64_t)b * N * I2;
  uint16_t* gxb = gx02 + (int64_t)b * N * I2;
  uint16_t* ghb = gdh + (int64_t)b * N * I;
  uint16_t* hlb = hlr + (int64_t)b * N * I;
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int m = mw + i * 32 + acc_row(q * 4);
      if (!nvalid || m >= I) continue;
      float o_gdh[4], o_gx0[4], o_gx2[4], o_dx0[4], o_dx2[4], o_hl[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int v = q * 4 + r;
        const float x0 = bf16r(acc[0][i][0][v]);
        const float x2 = bf16r(acc[1][i][0][v]);
        const float gd0 = bf16r(acc[2][i][0][v]);
        const float gd2 = bf16r(acc[3][i][0][v]);
        const float dh = bf16r(acc[4][i][0][v]);
        const float gd = bf16r(acc[5][i][0][v]);
        const float sg = sigmoidf_(x0);
        const float silu = sg * x0;
        const float mul = sg * (1.0f + x0 * (1.0f - sg));   // silu'(x0)
        const float ds = sg * (1.0f - sg);                   // sigmoid'(x0)
        o_gdh[r] = gd0 * L0 * x2 * mul + gd2 * L2 * silu;
        o_gx2[r] = gd0 * L0 * dh * mul + gd * L1 * silu;
        const float gsig = gd0 * L0 * dh * x2 * (1.0f + x0 - 2.0f * sg * x0);
        o_gx0[r] = (gd2 * L2 * dh + gd * L1 * x2) * mul + gd0 * L0 * dh * x2 * ds + gsig * ds;
        s0 += gd0 * dh * x2 * mul;
        s1 += gd * x2 * silu;
        s2 += gd2 * dh * silu;
        o_dx0[r] = dh * x2 * mul * L0;
        o_dx2[r] = silu * dh * L2;
        o_hl[r] = L1 * x2 * silu;
      }
      store4_tok(ghb, I, tok, m, o_gdh[0], o_gdh[1], o_gdh[2], o_gdh[3]);
      store4_tok(gxb, I2, tok, m, o_gx0[0], o_gx0[1], o_gx0[2], o_gx0[3]);
      store4_tok(gxb, I2, tok, I + m, o_gx2[0], o_gx2[1], o_gx2[2], o_gx2[3]);
      store4_tok(dxb, I2, tok, m, o_dx0[0], o_dx0[1], o_dx0[2], o_dx0[3]);
      store4_tok(dxb, I2, tok, I + m, o_dx2[0], o_dx2[1], o_dx2[2], o_dx2[3]);
      store4_tok(hlb, I, tok, m, o_hl[0], o_hl[1], o_hl[2], o_hl[3]);
    }
  // lanes l and l^32 hold the same column (other rows): fold them, then the
  // two waves of a column half meet in LDS
  s0 += __shfl_xor(s0, 32, 64);
  s1 += __shfl_xor(s1, 32, 64);
  s2 += __shfl_xor(s2, 32, 64);
  if ((threadIdx.x & 63) < 32) {
    red[0][w >> 1][ncol] = s0;
    red[1][w >> 1][ncol] = s1;
    red[2][w >> 1][ncol] = s2;
  }
  __syncthreads();
  if (threadIdx.x < BN) {
    const int c = threadIdx.x;
    const int nn = tt.n0 + c;
    if (nn < tt.size) {
      const int64_t o = ((int64_t)mt * B + b) * N + tt.start + nn;
      const int64_t plane = (int64_t)m_tiles * B * N;
      lr_part[o] = red[0][0][c] + red[0][1][c];
      lr_part[plane + o] = red[1][0][c] + red[1][1][c];
      lr_part[2 * plane + o] = red[2][0][c] + red[2][1][c];
    }
  }
}

// grad_lr_j[b, tok] = sum over m-tiles of lr_part[j][mt][b][tok] (fixed
// order); tokens past the batch's routed total get 0.
template <class LR>
__global__ __launch_bounds__(256) void lr_grad_reduce_kernel(const float* __restrict__ lr_part,
                                                             const int32_t* __restrict__ gs,
                                                             int B, int E, int N, int m_tiles,
                                                             typename LR::S* __restrict__ g0,
                                                             typename LR::S* __restrict__ g1,
                                                             typename LR::S* __restrict__ g2) {
  const int b = blockIdx.y;
  const int tok = blockIdx.x * 256 + threadIdx.x;
  if (tok >= N) return;
  int total = 0;
  for (int e = 0; e < E; ++e) {
    const int g = gs[(int64_t)b * E + e];
    total += g > 0 ? g : 0;
  }
  const int64_t plane = (int64_t)m_tiles * B * N;
  float a0 = 0.f, a1 = 0.f, a2 = 0.f;
  if (tok < total) {
    for (int mt = 0; mt < m_tiles; ++mt) {
      const int64_t o = ((int64_t)mt * B + b) * N + tok;
      a0 += lr_part[o];
      a1 += lr_part[plane + o];
      a2 += lr_part[2 * plane + o];
    }
  }
  const int64_t li = (int64_t)b * N + tok;
  g0[li] = LR::store(a0);
  g1[li] = LR::store(a1);
  g2[li] = LR::store(a2);
}

// =============================================================== transpose ==
// out[b, c, r] = in[b, r, c] for 2-byte elements, via a 64x64 LDS tile.
__global__ __launch_bounds__(256) void transpose16_kernel(const uint16_t* __restrict__ in,
                                                          uint16_t* __restrict__ out, int R,
                                                          int C, int r_tiles, int c_tiles) {
  __shared__ uint16_t tile[64][66];
  const int bid = blockIdx.x;
  const int ct = bid % c_tiles;
  const int rt = (bid / c_tiles) % r_tiles;
  const int b = bid / (c_tiles * r_tiles);
  const uint16_t* ib = in + (int64_t)b * R * C;
  uint16_t* ob = out + (int64_t)b * R * C;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int yy = ty; yy < 64; yy += 4) {
    const int r = rt * 64 + yy, c = ct * 64 + tx;
    if (r < R && c < C) tile[yy][tx] = ib[(int64_t)r * C + c];
  }
  __syncthreads();
  for (int yy = ty; yy < 64; yy += 4) {
    const int c = ct * 64 + yy, r = rt * 64 + tx;
    if (r < R && c < C) ob[(int64_t)c * R + r] = tile[tx][yy];
  }
}

// ------------------------------------------------------------- host side ----
constexpr int kApplyBM = 128, kApplyBN = 128;
constexpr int kS1BM = 128, kS1BN = 64;
constexpr int kWgBM = 128, kWgBN = 128;

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_grid(int64_t blocks, const char* what) {
  if (blocks > 0x7fffffffLL) {
    set_error("%s: problem too large for one launch (%lld workgroups)", what, (long long)blocks);
    return UTTT_ERR_UNSUPPORTED;
  }
  return UTTT_OK;
}

}  // namespace
}  // namespace uttt

using namespace uttt;

extern "C" int uttt_grouped_gate_up(const void* w0_w2, const void* x, const int32_t* group_sizes,
                                    int B, int E, int I, int D, int N, void* hidden,
                                    int token_major, void* stream) {
  UTTT_REQUIRE(B >= 0 && E >= 1 && I >= 0 && D >= 0 && N >= 0, "grouped_gate_up: bad sizes");
  UTTT_REQUIRE(I % 8 == 0 && D % 8 == 0, "grouped_gate_up: I=%d and D=%d must be multiples of 8", I, D);
  if (B == 0 || N == 0 || I == 0) return UTTT_OK;
  UTTT_REQUIRE(w0_w2 && x && group_sizes && hidden, "grouped_gate_up: null pointer");
  UTTT_REQUIRE(aligned16(w0_w2) && aligned16(x) && aligned16(hidden),
               "grouped_gate_up: tensors must be 16-byte aligned");
  const int m_tiles = (I + kApplyBM - 1) / kApplyBM;
  const int n_ub = (N + kApplyBN - 1) / kApplyBN + E;
  const int64_t blocks = (int64_t)m_tiles * n_ub * B;
  if (int rc = check_grid(blocks, "grouped_gate_up")) return rc;
  hipLaunchKernelGGL((gate_up_kernel<kApplyBM, kApplyBN>), dim3((unsigned)blocks), dim3(kThreads),
                     0, as_stream(stream), static_cast<const uint16_t*>(w0_w2),
                     static_cast<const uint16_t*>(x), group_sizes, static_cast<uint16_t*>(hidden),
                     E, I, D, N, m_tiles, n_ub, token_major);
  return check_launch("grouped_gate_up");
}

extern "C" int uttt_grouped_gemm_nt(const void* w, const void* x, const int32_t* group_sizes,
                                    int B, int E, int M, int K, int N, void* y, void* stream) {
  UTTT_REQUIRE(B >= 0 && E >= 1 && M >= 0 && K >= 0 && N >= 0, "grouped_gemm_nt: bad sizes");
  UTTT_REQUIRE(M % 8 == 0 && K % 8 == 0, "grouped_gemm_nt: M=%d and K=%d must be multiples of 8", M, K);
  if (B == 0 || N == 0 || M == 0) return UTTT_OK;
  UTTT_REQUIRE(w && x && group_sizes && y, "grouped_gemm_nt: null pointer");
  UTTT_REQUIRE(aligned16(w) && aligned16(x) && aligned16(y),
               "grouped_gemm_nt: tensors must be 16-byte aligned");
  const int m_tiles = (M + kApplyBM - 1) / kApplyBM;
  const int n_ub = (N + kApplyBN - 1) / kApplyBN + E;
  const int64_t blocks = (int64_t)m_tiles * n_ub * B;
  if (int rc = check_grid(blocks, "grouped_gemm_nt")) return rc;
  const NtPair p{static_cast<const uint16_t*>(w), static_cast<const uint16_t*>(x)};
  hipLaunchKernelGGL((gemm_nt_kernel<kApplyBM, kApplyBN, KMajor, 1>), dim3((unsigned)blocks),
                     dim3(kThreads), 0, as_stream(stream), p, p, group_sizes,
                     static_cast<uint16_t*>(y), E, M, K, N, m_tiles, n_ub);
  return check_launch("grouped_gemm_nt");
}

extern "C" int uttt_grouped_gemm_tn(const void* w, const void* x, const int32_t* group_sizes,
                                    int B, int E, int M, int K, int N, void* y, void* stream) {
  UTTT_REQUIRE(B >= 0 && E >= 1 && M >= 0 && K >= 0 && N >= 0, "grouped_gemm_tn: bad sizes");
  UTTT_REQUIRE(M % 8 == 0 && K % 8 == 0, "grouped_gemm_tn: M=%d and K=%d must be multiples of 8", M, K);
  if (B == 0 || N == 0 || M == 0) return UTTT_OK;
  UTTT_REQUIRE(w && x && group_sizes && y, "grouped_gemm_tn: null pointer");
  UTTT_REQUIRE(aligned16(w) && aligned16(x) && aligned16(y),
               "grouped_gemm_tn: tensors must be 16-byte aligned");
  const int m_tiles = (M + kApplyBM - 1) / kApplyBM;
  const int n_ub = (N + kApplyBN - 1) / kApplyBN + E;
  const int64_t blocks = (int64_t)m_tiles * n_ub * B;
  if (int rc = check_grid(blocks, "grouped_gemm_tn")) return rc;
  const NtPair p{static_cast<const uint16_t*>(w), static_cast<const uint16_t*>(x)};
  hipLaunchKernelGGL((gemm_nt_kernel<kApplyBM, kApplyBN, RMajor, 1>), dim3((unsigned)blocks),
                     dim3(kThreads), 0, as_stream(stream), p, p, group_sizes,
                     static_cast<uint16_t*>(y), E, M, K, N, m_tiles, n_ub);
  return check_launch("grouped_gemm_tn");
}

extern "C" int uttt_grouped_update_stage1(const void* w0_w2, const void* w1, const void* k,
                                          const void* v, const void* lr0, const void* lr1,
                                          const void* lr2, int lr_dtype,
                                          const int32_t* group_sizes, int B, int E, int I, int D,
                                          int N, void* dy0_dy2, void* hidden, int token_major,
                                          void* stream) {
  UTTT_REQUIRE(B >= 0 && E >= 1 && I >= 0 && D >= 0 && N >= 0, "grouped_update_stage1: bad sizes");
  UTTT_REQUIRE(I % 8 == 0 && D % 8 == 0,
               "grouped_update_stage1: I=%d and D=%d must be multiples of 8", I, D);
  if (B == 0 || N == 0 || I == 0) return UTTT_OK;
  UTTT_REQUIRE(w0_w2 && w1 && k && v && group_sizes && dy0_dy2 && hidden,
               "grouped_update_stage1: null pointer");
  UTTT_REQUIRE((lr0 == nullptr) == (lr1 == nullptr) && (lr1 == nullptr) == (lr2 == nullptr),
               "grouped_update_stage1: pass all three lr vectors or none");
  UTTT_REQUIRE(aligned16(w0_w2) && aligned16(w1) && aligned16(k) && aligned16(v) &&
                   aligned16(dy0_dy2) && aligned16(hidden),
               "grouped_update_stage1: tensors must be 16-byte aligned");
  const int m_tiles = (I + kS1BM - 1) / kS1BM;
  const int n_ub = (N + kS1BN - 1) / kS1BN + E;
  const int64_t blocks = (int64_t)m_tiles * n_ub * B;
  if (int rc = check_grid(blocks, "grouped_update_stage1")) return rc;
  hipStream_t st = as_stream(stream);
  UTTT_DTYPE_SWITCH_LR(lr_dtype, LR, {
    hipLaunchKernelGGL((update_s1_kernel<kS1BM, kS1BN, LR>), dim3((unsigned)blocks), dim3(kThreads),
                       0, st, static_cast<const uint16_t*>(w0_w2), static_cast<const uint16_t*>(w1),
                       static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v),
                       static_cast<const typename LR::S*>(lr0),
                       static_cast<const typename LR::S*>(lr1),
                       static_cast<const typename LR::S*>(lr2), group_sizes,
                       static_cast<uint16_t*>(dy0_dy2), static_cast<uint16_t*>(hidden), E, I, D, N,
                       m_tiles, n_ub, token_major);
  });
  return check_launch("grouped_update_stage1");
}

namespace uttt {
namespace {
WgradTask make_task(const void* a, const void* b, void* out, int R, int C, int transposed) {
  WgradTask t;
  t.a = static_cast<const uint16_t*>(a);
  t.b = static_cast<const uint16_t*>(b);
  t.out = static_cast<uint16_t*>(out);
  t.R = R;
  t.C = C;
  t.transposed = transposed;
  t.m_tiles = (R + kWgBM - 1) / kWgBM;
  t.c_tiles = (C + kWgBN - 1) / kWgBN;
  return t;
}

int launch_wgrad(const WgradTask& t0, const WgradTask& t1, const int32_t* gs, int B, int E, int N,
                 hipStream_t st, const char* what) {
  const int64_t per_group = (int64_t)t0.m_tiles * t0.c_tiles + (int64_t)t1.m_tiles * t1.c_tiles;
  const int64_t blocks = per_group * E * B;
  if (blocks == 0) return UTTT_OK;
  if (int rc = check_grid(blocks, what)) return rc;
  hipLaunchKernelGGL((wgrad_kernel<kWgBM, kWgBN>), dim3((unsigned)blocks), dim3(kThreads), 0, st,
                     t0, t1, gs, E, N);
  return check_launch(what);
}
}  // namespace
}  // namespace uttt

extern "C" int uttt_grouped_wgrad_pair(const void* dy0_dy2_tok, const void* k,
                                       const void* hidden_tok, const void* v,
                                       const int32_t* group_sizes, int B, int E, int I, int D,
                                       int N, void* dw0_w2, void* dw1, void* stream) {
  UTTT_REQUIRE(B >= 0 && E >= 1 && I >= 0 && D >= 0 && N >= 0, "grouped_wgrad_pair: bad sizes");
  UTTT_REQUIRE(I % 8 == 0 && D % 8 == 0,
               "grouped_wgrad_pair: I=%d and D=%d must be multiples of 8", I, D);
  if (B == 0 || I == 0 || D == 0) return UTTT_OK;
  UTTT_REQUIRE(dy0_dy2_tok && k && hidden_tok && v && group_sizes && dw0_w2 && dw1,
               "grouped_wgrad_pair: null pointer");
  UTTT_REQUIRE(aligned16(dy0_dy2_tok) && aligned16(k) && aligned16(hidden_tok) && aligned16(v) &&
                   aligned16(dw0_w2) && aligned16(dw1),
               "grouped_wgrad_pair: tensors must be 16-byte aligned");
  const WgradTask t0 = make_task(dy0_dy2_tok, k, dw0_w2, 2 * I, D, 0);
  const WgradTask t1 = make_task(hidden_tok, v, dw1, I, D, 1);
  return launch_wgrad(t0, t1, group_sizes, B, E, N, as_stream(stream), "grouped_wgrad_pair");
}

extern "C" int uttt_grouped_wgrad(const void* a_tok, const void* b_tok,
                                  const int32_t* group_sizes, int B, int E, int R, int C, int N,
                                  void* out, int transposed, void* stream) {
  UTTT_REQUIRE(B >= 0 && E >= 1 && R >= 0 && C >= 0 && N >= 0, "grouped_wgrad: bad sizes");
  UTTT_REQUIRE(R % 8 == 0 && C % 8 == 0, "grouped_wgrad: R=%d and C=%d must be multiples of 8",
               R, C);
  if (B == 0 || R == 0 || C == 0) return UTTT_OK;
  UTTT_REQUIRE(a_tok && b_tok && group_sizes && out, "grouped_wgrad: null pointer");
  UTTT_REQUIRE(aligned16(a_tok) && aligned16(b_tok) && aligned16(out),
               "grouped_wgrad: tensors must be 16-byte aligned");
  const WgradTask t0 = make_task(a_tok, b_tok, out, R, C, transposed);
  WgradTask t1 = t0;
  t1.m_tiles = 0;
  t1.c_tiles = 0;
  return launch_wgrad(t0, t1, group_sizes, B, E, N, as_stream(stream), "grouped_wgrad");
}

extern "C" int uttt_transpose_2byte(const void* in, int B, int R, int C, void* out, void* stream) {
  UTTT_REQUIRE(B >= 0 && R >= 0 && C >= 0, "transpose_2byte: bad sizes");
  if (B == 0 || R == 0 || C == 0) return UTTT_OK;
  UTTT_REQUIRE(in && out, "transpose_2byte: null pointer");
  const int rt = (R + 63) / 64, ct = (C + 63) / 64;
  const int64_t blocks = (int64_t)rt * ct * B;
  if (int rc = check_grid(blocks, "transpose_2byte")) return rc;
  hipLaunchKernelGGL(transpose16_kernel, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                     static_cast<const uint16_t*>(in), static_cast<uint16_t*>(out), R, C, rt, ct);
  return check_launch("transpose_2byte");
}

namespace uttt {
namespace {
constexpr int kUbBM = 128, kUbBN = 64;

struct UpdateBwdWs {
  size_t dx, gx, gdh, hlr, part, total;
};
UpdateBwdWs update_bwd_ws(int B, int I, int N) {
  auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
  const int m_tiles = (I + kUbBM - 1) / kUbBM;
  UpdateBwdWs w;
  w.dx = 0;
  w.gx = w.dx + up((size_t)B * N * 2 * I * 2);
  w.gdh = w.gx + up((size_t)B * N * 2 * I * 2);
  w.hlr = w.gdh + up((size_t)B * N * I * 2);
  w.part = w.hlr + up((size_t)B * N * I * 2);
  w.total = w.part + up((size_t)3 * m_tiles * B * N * 4);
  return w;
}
}  // namespace
}  // namespace uttt

extern "C" size_t uttt_update_bwd_workspace_bytes(int B, int I, int N) {
  if (B <= 0 || I <= 0 || N <= 0) return 0;
  return update_bwd_ws(B, I, N).total;
}

extern "C" int uttt_grouped_update_bwd(
    const void* w0_w2, const void* w1, const void* k, const void* v, const void* lr0,
    const void* lr1, const void* lr2, int lr_dtype, const int32_t* group_sizes,
    const void* grad_dw0_w2, const void* grad_dw1, int B, int E, int I, int D, int N,
    void* grad_w0_w2, void* grad_w1, void* grad_k, void* grad_v, void* grad_lr0, void* grad_lr1,
    void* grad_lr2, void* workspace, size_t workspace_bytes, void* stream) {
  UTTT_REQUIRE(B >= 0 && E >= 1 && I >= 0 && D >= 0 && N >= 0, "grouped_update_bwd: bad sizes");
  UTTT_REQUIRE(I % 8 == 0 && D % 8 == 0,
               "grouped_update_bwd: I=%d and D=%d must be multiples of 8", I, D);
  if (B == 0 || N == 0 || I == 0 || D == 0) return UTTT_OK;
  UTTT_REQUIRE(w0_w2 && w1 && k && v && lr0 && lr1 && lr2 && group_sizes && grad_dw0_w2 &&
                   grad_dw1 && grad_w0_w2 && grad_w1 && grad_k && grad_v && grad_lr0 &&
                   grad_lr1 && grad_lr2 && workspace,
               "grouped_update_bwd: null pointer");
  UTTT_REQUIRE(aligned16(w0_w2) && aligned16(w1) && aligned16(k) && aligned16(v) &&
                   aligned16(grad_dw0_w2) && aligned16(grad_dw1) && aligned16(grad_w0_w2) &&
                   aligned16(grad_w1) && aligned16(grad_k) && aligned16(grad_v) &&
                   aligned16(workspace),
               "grouped_update_bwd: tensors must be 16-byte aligned");
  const UpdateBwdWs ws = update_bwd_ws(B, I, N);
  UTTT_REQUIRE(workspace_bytes >= ws.total, "grouped_update_bwd: workspace %zu < %zu bytes",
               workspace_bytes, ws.total);
  uint8_t* wsb = static_cast<uint8_t*>(workspace);
  uint16_t* dx = reinterpret_cast<uint16_t*>(wsb + ws.dx);
  uint16_t* gx = reinterpret_cast<uint16_t*>(wsb + ws.gx);
  uint16_t* gdh = reinterpret_cast<uint16_t*>(wsb + ws.gdh);
  uint16_t* hlr = reinterpret_cast<uint16_t*>(wsb + ws.hlr);
  float* part = reinterpret_cast<float*>(wsb + ws.part);
  hipStream_t st = as_stream(stream);
  const auto* W02 = static_cast<const uint16_t*>(w0_w2);
  const auto* W1 = static_cast<const uint16_t*>(w1);
  const auto* GW02 = static_cast<const uint16_t*>(grad_dw0_w2);
  const auto* GW1 = static_cast<const uint16_t*>(grad_dw1);

  // 1. six GEMMs + second-order pointwise pass
  const int m_tiles = (I + kUbBM - 1) / kUbBM;
  const int n_ub = (N + kUbBN - 1) / kUbBN + E;
  const int64_t blocks = (int64_t)m_tiles * n_ub * B;
  if (int rc = check_grid(blocks, "grouped_update_bwd")) return rc;
  UTTT_DTYPE_SWITCH_LR(lr_dtype, LR, {
    using S = typename LR::S;
    hipLaunchKernelGGL((update_bwd_s1_kernel<kUbBM, kUbBN, LR>), dim3((unsigned)blocks),
                       dim3(kThreads), 0, st, W02, W1, GW02, GW1,
                       static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v),
                       static_cast<const S*>(lr0), static_cast<const S*>(lr1),
                       static_cast<const S*>(lr2), group_sizes, dx, gx, gdh, hlr, part, B, E, I,
                       D, N, m_tiles, n_ub);
    if (int rc = check_launch("grouped_update_bwd(stage 1)")) return rc;
    // 2. learning-rate gradients
    hipLaunchKernelGGL((lr_grad_reduce_kernel<LR>), dim3((N + 255) / 256, B), dim3(256), 0, st,
                       part, group_sizes, B, E, N, m_tiles, static_cast<S*>(grad_lr0),
                       static_cast<S*>(grad_lr1), static_cast<S*>(grad_lr2));
    if (int rc = check_launch("grouped_update_bwd(lr grads)")) return rc;
  });
  // 3. grad_K = GW0_W2^T dx0_x2 + W0_W2^T grad_x0_x2;  grad_V = W1 grad_dh + GW1 hidden_lr1
  {
    const int mt2 = (D + kApplyBM - 1) / kApplyBM;
    const int nub2 = (N + kApplyBN - 1) / kApplyBN + E;
    const int64_t blocks2 = (int64_t)mt2 * nub2 * B;
    if (int rc = check_grid(blocks2, "grouped_update_bwd")) return rc;
    hipLaunchKernelGGL((gemm_nt_kernel<kApplyBM, kApplyBN, RMajor, 2>), dim3((unsigned)blocks2),
                       dim3(kThreads), 0, st, NtPair{GW02, dx}, NtPair{W02, gx}, group_sizes,
                       static_cast<uint16_t*>(grad_k), E, D, 2 * I, N, mt2, nub2);
    if (int rc = check_launch("grouped_update_bwd(grad_K)")) return rc;
    hipLaunchKernelGGL((gemm_nt_kernel<kApplyBM, kApplyBN, KMajor, 2>), dim3((unsigned)blocks2),
                       dim3(kThreads), 0, st, NtPair{W1, gdh}, NtPair{GW1, hlr}, group_sizes,
                       static_cast<uint16_t*>(grad_v), E, D, I, N, mt2, nub2);
    if (int rc = check_launch("grouped_update_bwd(grad_V)")) return rc;
  }
  // 4. weight gradients of the weights
  const WgradTask t0 = make_task(gx, k, grad_w0_w2, 2 * I, D, 0);
  const WgradTask t1 = make_task(gdh, v, grad_w1, I, D, 1);
  return launch_wgrad(t0, t1, group_sizes, B, E, N, st, "grouped_update_bwd(weights)");
}
