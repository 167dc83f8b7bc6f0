// Grouped SwiGLU fast-weight GEMMs for gfx950 (bf16 MFMA, fp32 accumulate),
// all on the asynchronous pipeline of gemm_pipe.h.
//
// Notation per group (batch b, expert e): the expert's routed tokens are the
// contiguous segment seg(b,e) of the permuted token axis (lengths from
// group_sizes[b, e], in expert order); w0 = W0_W2[b,e,:I], w2 = W0_W2[b,e,I:],
// w1 = W1[b,e] ([D, I]).
//
// Two kernel families:
//   tn_kernel  token-grouped products Y[n, m] = sum_k A[m, k] X[n, k] for the
//              tokens n of each expert: two 128-row A tiles against one
//              256-token tile, with a problem-specific epilogue (SwiGLU for the
//              APPLY, the lr-scaled SwiGLU' for the UPDATE, the second-order
//              SwiGLU pass for the UPDATE backward, or a plain store).  An
//              optional second operand pair is chained along K (grad_K =
//              GW0_W2^T dx + W0_W2^T gx in one accumulator).
//   wg_kernel  weight gradients out[x, y] = sum_{n in seg} P[n, y] Q[n, x] with
//              the tokens as the reduction axis (both operands token-major,
//              read through the LDS transposing loads).
// Intermediates are token-major ([B, N, rows]); the kernel-level compat entry
// points can also write the reference's [B, rows, N] layout.
#include <algorithm>
#include <type_traits>

#include "gemm_pipe.h"

namespace uttt {
namespace {

using namespace pipe;

// ====================================================== token-grouped GEMM ==
struct TnArgs {
  const uint16_t* a[2][2];  // [pair][tile] A matrix (batch 0, expert 0)
  const uint16_t* x[2];     // [pair] token-major B (batch 0)
  int K[2];                 // [pair] reduction length (K[1] = 0: one product)
  int64_t lda;              // A leading dimension (K for KMajor, rows for RMajor)
  int64_t a_group;          // elements per (b, e) group of A
  int row_off[2];           // [tile] first A row of the tile = m0 + row_off
  int row_end[2];           // [tile] valid A rows are < row_end
  int m_step, m_tiles, n_tiles_ub;
  int gm, gn, n_super_m;    // XCD super-tiles: gm m-tiles x gn n-tiles (see tn_kernel);
                            // gm = 0: plain order (m-tile fastest)
  int B, E, N;
  int two;                  // tile 1 multiplied
  int sym;                  // symmetric output (one square group per batch, m_step equal to
                            // the token tile): only tiles on or below the diagonal are computed
  const int32_t* gs;
};

// Loop over this wave's accumulator quads: f(t, r, n, v[4]) with tile t, tile
// row r (rows r..r+3 hold v[0..3]) and tile token column n.  Indices are
// compile-time (static_for) so the accumulators stay in registers.
template <int NA, class F>
__device__ __forceinline__ void for_quads(const f32x16 (&acc0)[NA][kNB],
                                          const f32x16 (&acc1)[NA][kNB], int wm, int wn, bool two,
                                          F&& f) {
  static_for<2 * NA * kNB * 4>([&](auto idx) __attribute__((always_inline)) {
    constexpr int t = idx / (NA * kNB * 4);
    constexpr int i = (idx / (kNB * 4)) % NA;
    constexpr int j = (idx / 4) % kNB;
    constexpr int q = idx % 4;
    if (t == 1 && !two) return;
    const f32x16& a = t == 0 ? acc0[i][j] : acc1[i][j];
    const float v[4] = {a[q * 4], a[q * 4 + 1], a[q * 4 + 2], a[q * 4 + 3]};
    f(t, wm * 32 * NA + i * 32 + acc_row(q * 4), wn * 128 + j * 32 + acc_col(), v);
  });
}

// Paired quads of the two accumulators (same rows of A0 and A1): f(r, n, a[4], b[4]).
template <int NA, class F>
__device__ __forceinline__ void for_pairs(const f32x16 (&acc0)[NA][kNB],
                                          const f32x16 (&acc1)[NA][kNB], int wm, int wn, F&& f) {
  static_for<NA * kNB * 4>([&](auto idx) __attribute__((always_inline)) {
    constexpr int i = idx / (kNB * 4);
    constexpr int j = (idx / 4) % kNB;
    constexpr int q = idx % 4;
    const float a[4] = {acc0[i][j][q * 4], acc0[i][j][q * 4 + 1], acc0[i][j][q * 4 + 2],
                        acc0[i][j][q * 4 + 3]};
    const float b[4] = {acc1[i][j][q * 4], acc1[i][j][q * 4 + 1], acc1[i][j][q * 4 + 2],
                        acc1[i][j][q * 4 + 3]};
    f(wm * 32 * NA + i * 32 + acc_row(q * 4), wn * 128 + j * 32 + acc_col(), a, b);
  });
}

struct TileCtx {
  int b, m0, wm, wn, mt;
  TokenTile tt;
  float* lds0;  // two stage buffers (32 KiB each), free once the K loop is done
  float* lds1;
};

// ------------------------------------------------ coalesced epilogue frame --
// The accumulators hold, per lane, 4 consecutive rows of one token: written
// straight to a token-major tensor every wave instruction touches 32 tokens.
// The heavy epilogues instead go through LDS, one 64-token quarter of the
// tile at a time: the two waves owning the quarter write acc0 / acc1 as
// fp32 [token][128 rows] (16-byte chunks XOR-swizzled by token, conflict-free),
// then thread t takes token (t / 16) and rows 8 (t % 16) .. +7, so 16 lanes
// cover 128 contiguous rows of one token: 16-byte global loads and stores.
template <int Q, int NA>
__device__ __forceinline__ void stage_quarter(const f32x16 (&acc0)[NA][kNB],
                                              const f32x16 (&acc1)[NA][kNB], const TileCtx& c) {
  if (c.wn != Q / 2) return;
  static_for<NA * 2 * 4>([&](auto idx) __attribute__((always_inline)) {
    constexpr int i = idx / 8;
    constexpr int jl = (idx / 4) % 2;
    constexpr int q = idx % 4;
    constexpr int jj = 2 * (Q % 2) + jl;
    const int n = jl * 32 + acc_col();
    const int r = c.wm * 32 * NA + i * 32 + acc_row(q * 4);
    const int off = n * 128 + (((r >> 2) ^ (n & 31)) << 2);
    *reinterpret_cast<float4*>(c.lds0 + off) =
        make_float4(acc0[i][jj][q * 4], acc0[i][jj][q * 4 + 1], acc0[i][jj][q * 4 + 2],
                    acc0[i][jj][q * 4 + 3]);
    *reinterpret_cast<float4*>(c.lds1 + off) =
        make_float4(acc1[i][jj][q * 4], acc1[i][jj][q * 4 + 1], acc1[i][jj][q * 4 + 2],
                    acc1[i][jj][q * 4 + 3]);
  });
}

// Rows 8g .. 8g+7 of staged token n.
__device__ __forceinline__ void staged8(const float* reg, int n, int g, float (&v)[8]) {
  const float4 a = *reinterpret_cast<const float4*>(reg + n * 128 + (((2 * g) ^ (n & 31)) << 2));
  const float4 b =
      *reinterpret_cast<const float4*>(reg + n * 128 + (((2 * g + 1) ^ (n & 31)) << 2));
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// Sum over each aligned group of 16 lanes, the total in every lane: four
// DPP adds (swap neighbours, swap pairs, mirror the 8-lane halves, mirror
// the 16-lane row), no LDS round trip.  Every lane adds the same operands in
// a commutated order, so all 16 hold the same bits.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float sum16(float v) {
  v += dpp_f32<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v += dpp_f32<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v += dpp_f32<0x141>(v);  // row_half_mirror
  v += dpp_f32<0x140>(v);  // row_mirror
  return v;
}

__device__ __forceinline__ void unpack8(const uint4& u, float (&v)[8]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    v[2 * k] = bf16_to_f32((uint16_t)(w[k] & 0xffffu));
    v[2 * k + 1] = bf16_to_f32((uint16_t)(w[k] >> 16));
  }
}
__device__ __forceinline__ void load8(const uint16_t* p, float (&v)[8]) {
  unpack8(*reinterpret_cast<const uint4*>(p), v);
}
__device__ __forceinline__ void load8(const float* p, float (&v)[8]) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}
__device__ __forceinline__ void store8(uint16_t* p, const float (&v)[8]) {
  uint4 u;
  u.x = pack_bf16x2(v[0], v[1]);
  u.y = pack_bf16x2(v[2], v[3]);
  u.z = pack_bf16x2(v[4], v[5]);
  u.w = pack_bf16x2(v[6], v[7]);
  *reinterpret_cast<uint4*>(p) = u;
}
// The same store with a non-temporal hint, for outputs read back only much
// later (the saved tensors of the UPDATE's backward).
typedef unsigned int nt_store_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void store8_nt(uint16_t* p, const float (&v)[8]) {
  const nt_store_u32x4 u = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                            pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7])};
  __builtin_nontemporal_store(u, reinterpret_cast<nt_store_u32x4*>(p));
}
__device__ __forceinline__ void store8(float* p, const float (&v)[8]) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  *reinterpret_cast<float4*>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
}

// Runs body(n, g) for the 64 x 16 (token, row-group) items of every quarter
// of the tile, n = token index inside the tile (0..255), g = row group.
// The barriers order only the LDS staging buffer (s_waitcnt lgkmcnt(0) +
// s_barrier): a __syncthreads() would also wait for every global store of the
// quarter to complete (its workgroup-scope fence), four store drains per tile
// with the matrix core idle.
template <int NA, class Body>
__device__ __forceinline__ void staged_epilogue(const f32x16 (&acc0)[NA][kNB],
                                                const f32x16 (&acc1)[NA][kNB], const TileCtx& c,
                                                Body&& body) {
  block_barrier();  // every wave is done reading the stage buffers
  static_for<4>([&](auto QQ) __attribute__((always_inline)) {
    constexpr int Q = QQ;
    stage_quarter<Q>(acc0, acc1, c);
    block_barrier();
#pragma unroll
    for (int k = 0; k < kItemsOf<NA>; ++k) {
      const int it = threadIdx.x + kThreadsOf<NA> * k;
      body(it >> 4, Q * 64 + (it >> 4), it & 15);
    }
    block_barrier();
  });
}

// The staged epilogue in two phases per quarter: fetch(n, g) for the thread's
// four items first -- its global loads from clamped (always valid) addresses,
// straight-line code issued before the quarter is staged, so all of them are
// in flight together and overlap the staging -- then use(nl, n, g, raw) on
// each.  (Loads inside a per-item `if (valid)` would each be waited for
// before the next item's loads issue.)
template <int NA, class FetchFn, class UseFn>
__device__ __forceinline__ void staged_epilogue_prefetch(const f32x16 (&acc0)[NA][kNB],
                                                         const f32x16 (&acc1)[NA][kNB],
                                                         const TileCtx& c, FetchFn&& fetch,
                                                         UseFn&& use) {
  block_barrier();  // every wave is done reading the stage buffers
  static_for<4>([&](auto QQ) __attribute__((always_inline)) {
    constexpr int Q = QQ;
    decltype(fetch(0, 0)) raw[kItemsOf<NA>];
#pragma unroll
    for (int k = 0; k < kItemsOf<NA>; ++k) {
      const int it = threadIdx.x + kThreadsOf<NA> * k;
      raw[k] = fetch(Q * 64 + (it >> 4), it & 15);
    }
    stage_quarter<Q>(acc0, acc1, c);
    block_barrier();
#pragma unroll
    for (int k = 0; k < kItemsOf<NA>; ++k) {
      const int it = threadIdx.x + kThreadsOf<NA> * k;
      use(it >> 4, Q * 64 + (it >> 4), it & 15, raw[k]);
    }
    block_barrier();
  });
}

// The staged epilogue with each quarter's inputs fetched one quarter ahead:
// fetch(n, g) of quarter Q + 1 is issued before quarter Q's stores.  The
// vector memory counter counts loads and stores together, in issue order, so a
// load issued after a quarter's stores is only known to have landed once
// those stores have completed (written back past L2): fetched after them, a
// quarter's inputs waited for the previous quarter's stores at every quarter.
// Ahead of them, the wait at quarter Q + 1 covers only the stores of quarter
// Q - 1, which had a whole quarter to drain.  start() runs after quarter 0's
// fetch and before quarter 0 is staged (LDS writes of per-tile values).
template <int NA, class FetchFn, class UseFn, class StartFn>
__device__ __forceinline__ void staged_epilogue_ahead(const f32x16 (&acc0)[NA][kNB],
                                                      const f32x16 (&acc1)[NA][kNB],
                                                      const TileCtx& c, FetchFn&& fetch,
                                                      UseFn&& use, StartFn&& start) {
  using Raw = decltype(fetch(0, 0));
  Raw raw[2][kItemsOf<NA>];
  auto fetch_q = [&](auto qq, Raw (&dst)[kItemsOf<NA>]) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < kItemsOf<NA>; ++k) {
      const int it = threadIdx.x + kThreadsOf<NA> * k;
      dst[k] = fetch(decltype(qq)::value * 64 + (it >> 4), it & 15);
    }
  };
  block_barrier();  // every wave is done reading the stage buffers
  fetch_q(std::integral_constant<int, 0>{}, raw[0]);
  start();
  static_for<4>([&](auto QQ) __attribute__((always_inline)) {
    constexpr int Q = QQ;
    if constexpr (Q < 3) fetch_q(std::integral_constant<int, Q + 1>{}, raw[(Q + 1) & 1]);
    stage_quarter<Q>(acc0, acc1, c);
    block_barrier();
#pragma unroll
    for (int k = 0; k < kItemsOf<NA>; ++k) {
      const int it = threadIdx.x + kThreadsOf<NA> * k;
      use(it >> 4, Q * 64 + (it >> 4), it & 15, raw[Q & 1][k]);
    }
    block_barrier();
  });
}

// The tile's per-token lr values (three [B, N] arrays) as fp32 in LDS, past
// the staged quarter in lds0 (64 tokens x 128 rows of fp32): thread t loads
// the values of tile token t % 256 (clamped to the segment, so every address
// is valid; a null array reads as 1) before the epilogue's first barrier and
// writes them from start(); use() reads them with token_lr.  One set of loads
// per tile instead of three per item and quarter.
constexpr int kLrLds = 64 * 128;  // float offset in lds0
template <class LR>
struct TokenLrs {
  using S = typename LR::S;
  S v[3];
  __device__ __forceinline__ void load(const TileCtx& c, int N, const S* l0, const S* l1,
                                       const S* l2, const S* fallback) {
    const int n = threadIdx.x & (kBRows - 1);
    const int64_t li = (int64_t)c.b * N + c.tt.start + min(c.tt.n0 + n, c.tt.size - 1);
    v[0] = *(l0 ? l0 + li : fallback);
    v[1] = *(l1 ? l1 + li : fallback);
    v[2] = *(l2 ? l2 + li : fallback);
  }
  __device__ __forceinline__ void write(const TileCtx& c, bool h0, bool h1, bool h2) const {
    float* d = c.lds0 + kLrLds;
    const int n = threadIdx.x & (kBRows - 1);  // threads past 256 write the same values again
    d[n] = h0 ? LR::load(v[0]) : 1.0f;
    d[kBRows + n] = h1 ? LR::load(v[1]) : 1.0f;
    d[2 * kBRows + n] = h2 ? LR::load(v[2]) : 1.0f;
  }
};
__device__ __forceinline__ float token_lr(const TileCtx& c, int j, int n) {
  return c.lds0[kLrLds + j * kBRows + n];
}

// --- epilogue: plain store of both tiles into a token-major [B, N, ld] buffer
// Every epilogue states kStaleColumnsUnused: true only when it reads, stores
// or reduces nothing of the token columns at or past its segment's end.  The
// MFMA-skipping (SKIP) variant leaves stale LDS data in those columns'
// products, so only such epilogues may take it.
template <class OutT>
struct EpiStoreArgs {
  OutT* out;
  int64_t ld;
  int col_off[2];  // tile t, row r -> column m0 + col_off[t] + r
  int col_end[2];  // stored while that column < col_end[t]
  int N;
};

// STAGED (the launcher's choice when the output is 16-byte aligned; ld and
// the column offsets are multiples of 8): through the LDS frame, so every
// store instruction writes 4 tokens x 256 contiguous bytes (bf16) instead of
// 32 tokens x 16 bytes; otherwise straight from the accumulators.
template <class OutT, bool STAGED = false>
struct EpiStore {
  static constexpr bool kStaleColumnsUnused = true;  // per-column stores, masked by segment
  using Args = EpiStoreArgs<OutT>;
  template <int NA>
  __device__ __forceinline__ static void apply(const Args& ea, const f32x16 (&acc0)[NA][kNB],
                                               const f32x16 (&acc1)[NA][kNB], const TileCtx& c,
                                               bool two) {
    OutT* ob = ea.out + (int64_t)c.b * ea.N * ea.ld;
    if constexpr (STAGED) {
      staged_epilogue(acc0, acc1, c, [&](int nl, int n, int g) __attribute__((always_inline)) {
        if (c.tt.n0 + n >= c.tt.size) return;
        OutT* row = ob + (int64_t)(c.tt.start + c.tt.n0 + n) * ea.ld;
        static_for<2>([&](auto T) __attribute__((always_inline)) {
          constexpr int t = T;
          if (t == 1 && !two) return;
          const int col = c.m0 + ea.col_off[t] + 8 * g;
          if (col >= ea.col_end[t]) return;  // col_end is a multiple of 8
          float v[8];
          staged8(t == 0 ? c.lds0 : c.lds1, nl, g, v);
          store8(row + col, v);
        });
      });
    } else {
      for_quads(acc0, acc1, c.wm, c.wn, two, [&](int t, int r, int n, const float* v) __attribute__((always_inline)) {
        const int col = c.m0 + ea.col_off[t] + r;
        if (c.tt.n0 + n < c.tt.size && col < ea.col_end[t])
          store4(ob, ea.ld, c.tt.start + c.tt.n0 + n, col, v[0], v[1], v[2], v[3]);
      });
    }
  }
};

// --- epilogue: o = bf16(bf16(alpha * in) + bf16(beta * bf16(acc))) (no `in`:
// o = bf16(beta * bf16(acc))), stored to `out`, and bf16(gamma * o) to `out2`
// when given; all token-major [B, N, ld] at the product's position.  The
// Newton-Schulz steps with the bf16 rounding after every operation that the
// reference's bf16 tensor arithmetic has: A = X X^T (with c A as out2),
// B = b A + (c A) A, X' = a X + B X.
// Through the LDS frame (16-byte accesses along the token rows; the arrays
// are 16-byte aligned workspace with ld a multiple of 8).
// SYM: the product is symmetric and only tiles on or below the diagonal run
// (TnArgs::sym); a tile strictly below the diagonal also stores its
// transpose, every thread 8 consecutive tokens of one output row (`in` is
// symmetric too, so the transposed element is read from the transposed
// position).
struct EpiLinCombArgs {
  uint16_t* out;
  uint16_t* out2;
  const uint16_t* in;
  int64_t ld;
  int col_end;
  int N;
  float alpha, beta, gamma;
};

// 8 consecutive elements at offset `at` of every array; xin = in[at .. at + 7]
// as loaded (ignored without `in`).
__device__ __forceinline__ void lincomb8(const EpiLinCombArgs& ea, const float (&v)[8],
                                         const uint4& xin, int64_t at) {
  float x[8], o[8];
  unpack8(xin, x);
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const float p = bf16r(ea.beta * bf16r(v[u]));
    o[u] = ea.in != nullptr ? bf16r(bf16r(ea.alpha * x[u]) + p) : p;
  }
  store8(ea.out + at, o);
  if (ea.out2 != nullptr) {
#pragma unroll
    for (int u = 0; u < 8; ++u) o[u] *= ea.gamma;
    store8(ea.out2 + at, o);
  }
}

template <bool SYM = false>
struct EpiLinComb {
  static constexpr bool kStaleColumnsUnused = true;
  using Args = EpiLinCombArgs;
  template <int NA>
  __device__ __forceinline__ static void apply(const Args& ea, const f32x16 (&acc0)[NA][kNB],
                                               const f32x16 (&acc1)[NA][kNB], const TileCtx& c,
                                               bool two) {
    const int64_t bo = (int64_t)c.b * ea.N * ea.ld;
    (void)two;  // past col_end when tile 1 is not multiplied
    // `in` is read from valid addresses whether or not it is given (out's,
    // ignored then), all of a quarter's loads before any is used: a load
    // under a branch, or one used at once, waits for every store in flight
    const uint16_t* src = ea.in != nullptr ? ea.in : ea.out;
    const bool mirror = SYM && c.m0 < c.tt.n0;  // uniform: a tile strictly below the diagonal
    block_barrier();                             // every wave is done reading the stage buffers
    static_for<4>([&](auto QQ) __attribute__((always_inline)) {
      constexpr int Q = QQ;
      // the tile itself: token nl of the quarter, rows 8 g .. 8 g + 7 of each part
      uint4 xt[kItemsOf<NA>][2];
#pragma unroll
      for (int k = 0; k < kItemsOf<NA>; ++k) {
        const int it = threadIdx.x + kThreadsOf<NA> * k;
        const int nl = it >> 4, g = it & 15;
        const bool tok_ok = c.tt.n0 + Q * 64 + nl < c.tt.size;
        const int64_t tok = c.tt.start + c.tt.n0 + Q * 64 + nl;
#pragma unroll
        for (int part = 0; part < 2; ++part) {
          const int col = c.m0 + part * kTileRows + 8 * g;
          const int64_t at = tok_ok && col < ea.col_end ? bo + tok * ea.ld + col : bo;
          xt[k][part] = *reinterpret_cast<const uint4*>(src + at);
        }
      }
      // its transpose: row `col` of the output, 8 consecutive tokens
      uint4 xm[2 * kItemsOf<NA>];
      if (mirror) {
#pragma unroll
        for (int k = 0; k < 2 * kItemsOf<NA>; ++k) {
          const int it = threadIdx.x + kThreadsOf<NA> * k;
          const int r = it & 127, part = (it >> 7) & 1, g8 = it >> 8;
          const int nq = Q * 64 + 8 * g8;
          const int col = c.m0 + part * kTileRows + r;
          const bool ok = c.tt.n0 + nq < c.tt.size && col < ea.col_end;  // multiples of 8
          const int64_t at = ok ? bo + (int64_t)col * ea.ld + c.tt.start + c.tt.n0 + nq : bo;
          xm[k] = *reinterpret_cast<const uint4*>(src + at);
        }
      }
      stage_quarter<Q>(acc0, acc1, c);
      block_barrier();
#pragma unroll
      for (int k = 0; k < kItemsOf<NA>; ++k) {
        const int it = threadIdx.x + kThreadsOf<NA> * k;
        const int nl = it >> 4, g = it & 15;
        if (c.tt.n0 + Q * 64 + nl >= c.tt.size) continue;
        const int64_t tok = c.tt.start + c.tt.n0 + Q * 64 + nl;
#pragma unroll
        for (int part = 0; part < 2; ++part) {
          const int col = c.m0 + part * kTileRows + 8 * g;
          if (col >= ea.col_end) continue;  // col_end is a multiple of 8
          float v[8];
          staged8(part == 0 ? c.lds0 : c.lds1, nl, g, v);
          lincomb8(ea, v, xt[k][part], bo + tok * ea.ld + col);
        }
      }
      if (mirror) {
#pragma unroll
        for (int k = 0; k < 2 * kItemsOf<NA>; ++k) {
          const int it = threadIdx.x + kThreadsOf<NA> * k;
          const int r = it & 127, part = (it >> 7) & 1, g8 = it >> 8;
          const int nq = Q * 64 + 8 * g8;
          const int col = c.m0 + part * kTileRows + r;
          if (c.tt.n0 + nq >= c.tt.size || col >= ea.col_end) continue;
          const float* lds = part == 0 ? c.lds0 : c.lds1;
          float v[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const int nl = 8 * g8 + u;
            v[u] = lds[nl * 128 + (((r >> 2) ^ (nl & 31)) << 2) + (r & 3)];
          }
          lincomb8(ea, v, xm[k], bo + (int64_t)col * ea.ld + c.tt.start + c.tt.n0 + nq);
        }
      }
      block_barrier();
    });
  }
};

// --- epilogue: APPLY gate/up, h = y2 * silu(y0) (acc0 = w0 rows, acc1 = w2 rows)
struct EpiSwiGLU {
  static constexpr bool kStaleColumnsUnused = true;  // per-column stores, masked by segment
  struct Args {
    uint16_t* out;
    int I, N, token_major;
  };
  template <int NA>
  __device__ __forceinline__ static void apply(const Args& ea, const f32x16 (&acc0)[NA][kNB],
                                               const f32x16 (&acc1)[NA][kNB], const TileCtx& c,
                                               bool) {
    uint16_t* hb = ea.out + (int64_t)c.b * ea.N * ea.I;
    for_pairs(acc0, acc1, c.wm, c.wn, [&](int r, int n, const float* y0, const float* y2) __attribute__((always_inline)) {
      const int m = c.m0 + r;
      if (c.tt.n0 + n >= c.tt.size || m >= ea.I) return;
      const int tok = c.tt.start + c.tt.n0 + n;
      float h[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) h[u] = y2[u] * (y0[u] * sigmoidf_(y0[u]));
      if (ea.token_major) {
        store4(hb, ea.I, tok, m, h[0], h[1], h[2], h[3]);
      } else {
#pragma unroll
        for (int u = 0; u < 4; ++u) hb[(int64_t)(m + u) * ea.N + tok] = f32_to_bf16(h[u]);
      }
    });
  }
};

// --- epilogue: UPDATE stage 1 (acc0 = Y0, acc1 = Y2; DH fp32 from the pre-pass)
//   DY0 = lr0 sig(Y0) Y2 DH (1 + Y0 (1 - sig(Y0))), DY2 = lr2 silu(Y0) DH,
//   Hid = lr1 silu(Y0) Y2; lr = 1 when the lr pointers are null.
template <class LR>
struct EpiS1 {
  static constexpr bool kStaleColumnsUnused = false;  // not audited for the SKIP variant
  struct Args {
    const float* dh;  // [B, N, I]
    const typename LR::S *lr0, *lr1, *lr2;
    uint16_t* dy;     // [B, N, 2I] or [B, 2I, N]
    uint16_t* hid;    // [B, N, I] or [B, I, N]
    uint16_t* y_save;   // optional [B, N, 2I]: bf16(Y0 | Y2) for the backward
    uint16_t* dh_save;  // optional [B, N, I]: bf16(DH)
    int I, N, token_major;
  };
  template <int NA>
  __device__ __forceinline__ static void apply(const Args& ea, const f32x16 (&acc0)[NA][kNB],
                                               const f32x16 (&acc1)[NA][kNB], const TileCtx& c,
                                               bool) {
    const int I = ea.I, I2 = 2 * I;
    const float* dhb = ea.dh + (int64_t)c.b * ea.N * I;
    uint16_t* dyb = ea.dy + (int64_t)c.b * ea.N * I2;
    uint16_t* hb = ea.hid + (int64_t)c.b * ea.N * I;
    using S = typename LR::S;
    struct Raw {
      float4 dh0, dh1;
    };
    auto fetch = [&](int n, int g) __attribute__((always_inline)) {
      const int m = c.m0 + 8 * g;
      const int tok = c.tt.start + min(c.tt.n0 + n, c.tt.size - 1);  // clamped: always valid
      const float* p = dhb + (int64_t)tok * I + (m < I ? m : 0);
      Raw r;
      r.dh0 = *reinterpret_cast<const float4*>(p);
      r.dh1 = *reinterpret_cast<const float4*>(p + 4);
      return r;
    };
    // a missing lr reads the first element of dh (every load from a valid
    // address: a load under a branch is followed by a wait on every access in
    // flight) and is stored as 1
    TokenLrs<LR> lrs;
    lrs.load(c, ea.N, ea.lr0, ea.lr1, ea.lr2, reinterpret_cast<const S*>(ea.dh));
    auto start = [&]() __attribute__((always_inline)) {
      lrs.write(c, ea.lr0 != nullptr, ea.lr1 != nullptr, ea.lr2 != nullptr);
    };
    staged_epilogue_ahead(acc0, acc1, c, fetch, [&](int nl, int n, int g, const Raw& rw) __attribute__((always_inline)) {
      const int m = c.m0 + 8 * g;
      if (c.tt.n0 + n >= c.tt.size || m >= I) return;
      const int tok = c.tt.start + c.tt.n0 + n;
      const float l0 = token_lr(c, 0, n);
      const float l1 = token_lr(c, 1, n);
      const float l2 = token_lr(c, 2, n);
      float y0[8], y2[8], d0[8], d2[8], hh[8];
      float dh[8] = {rw.dh0.x, rw.dh0.y, rw.dh0.z, rw.dh0.w,
                     rw.dh1.x, rw.dh1.y, rw.dh1.z, rw.dh1.w};
      staged8(c.lds0, nl, g, y0);
      staged8(c.lds1, nl, g, y2);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float sg = sigmoidf_(y0[u]);
        const float sw = sg * y0[u];
        d0[u] = sg * y2[u] * dh[u] * (1.0f + y0[u] * (1.0f - sg)) * l0;
        d2[u] = sw * dh[u] * l2;
        hh[u] = sw * y2[u] * l1;
      }
      if (ea.y_save != nullptr) {  // the values the backward would recompute, rounded as it does
        store8_nt(ea.y_save + (int64_t)c.b * ea.N * I2 + (int64_t)tok * I2 + m, y0);
        store8_nt(ea.y_save + (int64_t)c.b * ea.N * I2 + (int64_t)tok * I2 + I + m, y2);
        store8_nt(ea.dh_save + (int64_t)c.b * ea.N * I + (int64_t)tok * I + m, dh);
      }
      if (ea.token_major) {
        store8(dyb + (int64_t)tok * I2 + m, d0);
        store8(dyb + (int64_t)tok * I2 + I + m, d2);
        store8(hb + (int64_t)tok * I + m, hh);
      } else {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          dyb[(int64_t)(m + u) * ea.N + tok] = f32_to_bf16(d0[u]);
          dyb[(int64_t)(I + m + u) * ea.N + tok] = f32_to_bf16(d2[u]);
          hb[(int64_t)(m + u) * ea.N + tok] = f32_to_bf16(hh[u]);
        }
      }
    }, start);
  }
};

// --- epilogue: UPDATE backward, second-order SwiGLU pass (acc0 = Y0, acc1 = Y2)
// inputs stored bf16 by the pre-passes, as the reference stores the outputs of
// its four-GEMM kernel: GY = [GW0 k | GW2 k] and DHG = [w1^T v | gw1^T v],
// both [B, N, 2I]; Y0 / Y2 are rounded to bf16 here for the same reason.
// Outputs (bf16, token-major): grad_dh [N, I], grad_x0_x2 [N, 2I],
// dx0_x2 [N, 2I], hidden_lr1 [N, I]; fp32 lr-gradient partial sums over this
// tile's 128 hidden rows, lr_part[j][mt][b][tok].
template <class LR>
struct EpiBwd {
  static constexpr bool kStaleColumnsUnused = false;  // reduces over tile rows per token
  struct Args {
    const uint16_t* gy;
    const uint16_t* dhg;
    const typename LR::S *lr0, *lr1, *lr2;
    uint16_t *gdh, *gx, *dx, *hlr;
    float* lr_part;
    int I, N, B, m_tiles;
  };
  template <int NA>
  __device__ __forceinline__ static void apply(const Args& ea, const f32x16 (&acc0)[NA][kNB],
                                               const f32x16 (&acc1)[NA][kNB], const TileCtx& c,
                                               bool) {
    const int I = ea.I, I2 = 2 * I;
    const int64_t bo2 = (int64_t)c.b * ea.N * I2, bo1 = (int64_t)c.b * ea.N * I;
    const int64_t plane = (int64_t)ea.m_tiles * ea.B * ea.N;
    using S = typename LR::S;
    struct Raw {
      uint4 gd0, gd2, dh, gd;
      S l0, l1, l2;
    };
    auto fetch = [&](int n, int g) __attribute__((always_inline)) {
      const int m = c.m0 + 8 * g;
      const int tok = c.tt.start + min(c.tt.n0 + n, c.tt.size - 1);  // clamped: always valid
      const int mc = m < I ? m : 0;
      const int64_t li = (int64_t)c.b * ea.N + tok;
      const int64_t r2 = bo2 + (int64_t)tok * I2;
      Raw r;
      r.gd0 = *reinterpret_cast<const uint4*>(ea.gy + r2 + mc);
      r.gd2 = *reinterpret_cast<const uint4*>(ea.gy + r2 + I + mc);
      r.dh = *reinterpret_cast<const uint4*>(ea.dhg + r2 + mc);
      r.gd = *reinterpret_cast<const uint4*>(ea.dhg + r2 + I + mc);
      r.l0 = ea.lr0[li];
      r.l1 = ea.lr1[li];
      r.l2 = ea.lr2[li];
      return r;
    };
    staged_epilogue_prefetch(acc0, acc1, c, fetch, [&](int nl, int n, int g, const Raw& rw) __attribute__((always_inline)) {
      const int m = c.m0 + 8 * g;
      const bool ok = c.tt.n0 + n < c.tt.size && m < I;
      const int tok = c.tt.start + c.tt.n0 + n;
      float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f;
      if (ok) {
        const float L0 = LR::load(rw.l0);
        const float L1 = LR::load(rw.l1);
        const float L2 = LR::load(rw.l2);
        float x0[8], x2[8], gd0[8], gd2[8], dh[8], gd[8];
        staged8(c.lds0, nl, g, x0);
        staged8(c.lds1, nl, g, x2);
        const int64_t r2 = bo2 + (int64_t)tok * I2, r1 = bo1 + (int64_t)tok * I;
        unpack8(rw.gd0, gd0);
        unpack8(rw.gd2, gd2);
        unpack8(rw.dh, dh);
        unpack8(rw.gd, gd);
        float o_gdh[8], o_gx0[8], o_gx2[8], o_dx0[8], o_dx2[8], o_hl[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const float y0 = bf16r(x0[u]);
          const float y2 = bf16r(x2[u]);
          const float sg = sigmoidf_(y0);
          const float silu = sg * y0;
          const float mul = sg * (1.0f + y0 * (1.0f - sg));  // silu'(y0)
          const float ds = sg * (1.0f - sg);                  // sigmoid'(y0)
          o_gdh[u] = gd0[u] * L0 * y2 * mul + gd2[u] * L2 * silu;
          o_gx2[u] = gd0[u] * L0 * dh[u] * mul + gd[u] * L1 * silu;
          const float gsig = gd0[u] * L0 * dh[u] * y2 * (1.0f + y0 - 2.0f * sg * y0);
          o_gx0[u] = (gd2[u] * L2 * dh[u] + gd[u] * L1 * y2) * mul +
                     gd0[u] * L0 * dh[u] * y2 * ds + gsig * ds;
          s0 += gd0[u] * dh[u] * y2 * mul;
          s1 += gd[u] * y2 * silu;
          s2 += gd2[u] * dh[u] * silu;
          o_dx0[u] = dh[u] * y2 * mul * L0;
          o_dx2[u] = silu * dh[u] * L2;
          o_hl[u] = L1 * y2 * silu;
        }
        store8(ea.gdh + r1 + m, o_gdh);
        store8(ea.gx + r2 + m, o_gx0);
        store8(ea.gx + r2 + I + m, o_gx2);
        store8(ea.dx + r2 + m, o_dx0);
        store8(ea.dx + r2 + I + m, o_dx2);
        store8(ea.hlr + r1 + m, o_hl);
      }
      // the 16 lanes of one token hold its 128 rows: sum them for this tile's
      // lr-gradient partial
      s0 = sum16(s0);
      s1 = sum16(s1);
      s2 = sum16(s2);
      if (g == 0 && c.tt.n0 + n < c.tt.size) {
        const int64_t o = ((int64_t)c.mt * ea.B + c.b) * ea.N + tok;
        ea.lr_part[o] = s0;
        ea.lr_part[plane + o] = s1;
        ea.lr_part[2 * plane + o] = s2;
      }
    });
  }
};

// --- epilogue: UPDATE backward from the forward's saved values (acc0 = GY0 =
// gw0 k, acc1 = GY2 = gw2 k): the second-order pass of EpiBwd with Y0 | Y2 and
// DH read from the forward's bf16 saves (the values the reference's backward
// recomputes and stores bf16) and GD = gw1^T v from its own launch (bf16), so
// Y0, Y2 and DH are not recomputed and GY is used from the registers, rounded
// to bf16 where the reference stores it.  Outputs as EpiBwd.
template <class LR>
struct EpiBwdSaved {
  static constexpr bool kStaleColumnsUnused = false;  // reduces over tile rows per token
  struct Args {
    const uint16_t* y_saved;   // [B, N, 2I]
    const uint16_t* dh_saved;  // [B, N, I]
    const uint16_t* gd;        // [B, N, I]
    const typename LR::S *lr0, *lr1, *lr2;
    uint16_t *gdh, *gx, *dx, *hlr;
    float* lr_part;
    int I, N, B, m_tiles;
  };
  template <int NA>
  __device__ __forceinline__ static void apply(const Args& ea, const f32x16 (&acc0)[NA][kNB],
                                               const f32x16 (&acc1)[NA][kNB], const TileCtx& c,
                                               bool) {
    const int I = ea.I, I2 = 2 * I;
    const int64_t bo2 = (int64_t)c.b * ea.N * I2, bo1 = (int64_t)c.b * ea.N * I;
    const int64_t plane = (int64_t)ea.m_tiles * ea.B * ea.N;
    using S = typename LR::S;
    struct Raw {
      uint4 y0, y2, dh, gd;
    };
    auto fetch = [&](int n, int g) __attribute__((always_inline)) {
      const int m = c.m0 + 8 * g;
      const int tok = c.tt.start + min(c.tt.n0 + n, c.tt.size - 1);  // clamped: always valid
      const int mc = m < I ? m : 0;
      const int64_t r2 = bo2 + (int64_t)tok * I2, r1 = bo1 + (int64_t)tok * I;
      Raw r;
      r.y0 = *reinterpret_cast<const uint4*>(ea.y_saved + r2 + mc);
      r.y2 = *reinterpret_cast<const uint4*>(ea.y_saved + r2 + I + mc);
      r.dh = *reinterpret_cast<const uint4*>(ea.dh_saved + r1 + mc);
      r.gd = *reinterpret_cast<const uint4*>(ea.gd + r1 + mc);
      return r;
    };
    TokenLrs<LR> lrs;
    lrs.load(c, ea.N, ea.lr0, ea.lr1, ea.lr2, ea.lr0);
    auto start = [&]() __attribute__((always_inline)) { lrs.write(c, true, true, true); };
    auto use = [&](int nl, int n, int g, const Raw& rw) __attribute__((always_inline)) {
      const int m = c.m0 + 8 * g;
      const bool ok = c.tt.n0 + n < c.tt.size && m < I;
      const int tok = c.tt.start + c.tt.n0 + n;
      float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f;
      if (ok) {
        const float L0 = token_lr(c, 0, n);
        const float L1 = token_lr(c, 1, n);
        const float L2 = token_lr(c, 2, n);
        float gy0[8], gy2[8], y0v[8], y2v[8], dh[8], gd[8];
        staged8(c.lds0, nl, g, gy0);
        staged8(c.lds1, nl, g, gy2);
        unpack8(rw.y0, y0v);
        unpack8(rw.y2, y2v);
        unpack8(rw.dh, dh);
        unpack8(rw.gd, gd);
        const int64_t r2 = bo2 + (int64_t)tok * I2, r1 = bo1 + (int64_t)tok * I;
        float o_gdh[8], o_gx0[8], o_gx2[8], o_dx0[8], o_dx2[8], o_hl[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const float y0 = y0v[u], y2 = y2v[u];
          const float gd0 = bf16r(gy0[u]), gd2 = bf16r(gy2[u]);
          const float sg = sigmoidf_(y0);
          const float silu = sg * y0;
          const float mul = sg * (1.0f + y0 * (1.0f - sg));  // silu'(y0)
          const float ds = sg * (1.0f - sg);                  // sigmoid'(y0)
          o_gdh[u] = gd0 * L0 * y2 * mul + gd2 * L2 * silu;
          o_gx2[u] = gd0 * L0 * dh[u] * mul + gd[u] * L1 * silu;
          const float gsig = gd0 * L0 * dh[u] * y2 * (1.0f + y0 - 2.0f * sg * y0);
          o_gx0[u] = (gd2 * L2 * dh[u] + gd[u] * L1 * y2) * mul + gd0 * L0 * dh[u] * y2 * ds +
                     gsig * ds;
          s0 += gd0 * dh[u] * y2 * mul;
          s1 += gd[u] * y2 * silu;
          s2 += gd2 * dh[u] * silu;
          o_dx0[u] = dh[u] * y2 * mul * L0;
          o_dx2[u] = silu * dh[u] * L2;
          o_hl[u] = L1 * y2 * silu;
        }
        store8(ea.gdh + r1 + m, o_gdh);
        store8(ea.gx + r2 + m, o_gx0);
        store8(ea.gx + r2 + I + m, o_gx2);
        store8(ea.dx + r2 + m, o_dx0);
        store8(ea.dx + r2 + I + m, o_dx2);
        store8(ea.hlr + r1 + m, o_hl);
      }
      s0 = sum16(s0);
      s1 = sum16(s1);
      s2 = sum16(s2);
      if (g == 0 && c.tt.n0 + n < c.tt.size) {
        const int64_t o = ((int64_t)c.mt * ea.B + c.b) * ea.N + tok;
        ea.lr_part[o] = s0;
        ea.lr_part[plane + o] = s1;
        ea.lr_part[2 * plane + o] = s2;
      }
    };
    // Four waves fetch one quarter ahead (two quarters of inputs in
    // registers); eight waves have half the registers per thread and fetch
    // each quarter just before staging it (one quarter in registers: the
    // double buffer spills there).
    if constexpr (NA == 2) {
      staged_epilogue_ahead(acc0, acc1, c, fetch, use, start);
    } else {
      block_barrier();  // every wave is done reading the stage buffers
      start();
      staged_epilogue_prefetch(acc0, acc1, c, fetch, use);
    }
  }
};

template <int AMAJ, class Epi, bool SKIP, int NA>
__global__ __launch_bounds__(kThreadsOf<NA>) void tn_kernel(TnArgs a, typename Epi::Args ea) {
  __shared__ __attribute__((aligned(16))) uint8_t st0[kStageBytes];
  __shared__ __attribute__((aligned(16))) uint8_t st1[kStageBytes];

  // Tile order: workgroup i runs on XCD i % kXcds, each XCD with its own L2.
  // The (m-tile, n-tile) plane (n-tiles of all batches in a row) is cut into
  // gm x gn super-tiles and each XCD takes whole ones, so the ~32 workgroups
  // an XCD runs at once share gm A slices and gn B slices per K step in its
  // L2 instead of fetching the B tile once per XCD.
  // Small grids (a few rounds of workgroups) keep the plain order, which
  // spreads the work evenly over the XCDs.
  const int bid = blockIdx.x;
  int mt, ntg;
  if (a.gm > 0) {
    const int xcd = bid % kXcds, loc = bid / kXcds;
    const int per = a.gm * a.gn;
    const int sup = (loc / per) * kXcds + xcd;
    const int p = loc % per;
    mt = (sup % a.n_super_m) * a.gm + p % a.gm;
    ntg = (sup / a.n_super_m) * a.gn + p / a.gm;
  } else {
    mt = bid % a.m_tiles;
    ntg = bid / a.m_tiles;
  }
  if (mt >= a.m_tiles || ntg >= a.B * a.n_tiles_ub) return;  // padding of the super-tile grid
  const int b = ntg / a.n_tiles_ub, nt = ntg % a.n_tiles_ub;
  const TokenTile tt = find_token_tile<kBRows>(a.gs + (int64_t)b * a.E, a.E, a.N, nt);
  if (tt.e < 0 || (a.sym && mt * a.m_step > tt.n0)) return;
  const int m0 = mt * a.m_step;

  const int64_t ag = ((int64_t)b * a.E + tt.e) * a.a_group;
  const Operand A00{a.a[0][0] + ag, a.lda, a.row_end[0], a.K[0]};
  const Operand A01{a.a[0][1] + ag, a.lda, a.row_end[1], a.K[0]};
  const Operand A10{a.a[1][0] + ag, a.lda, a.row_end[0], a.K[1]};
  const Operand A11{a.a[1][1] + ag, a.lda, a.row_end[1], a.K[1]};
  const Operand X0{a.x[0] + ((int64_t)b * a.N + tt.start) * a.K[0], a.K[0], tt.size, a.K[0]};
  const Operand X1{a.x[1] + ((int64_t)b * a.N + tt.start) * a.K[1], a.K[1], tt.size, a.K[1]};
  const int nk0 = (a.K[0] + kBK - 1) / kBK;
  const int nk1 = (a.K[1] + kBK - 1) / kBK;
  const int r0 = m0 + a.row_off[0], r1 = m0 + a.row_off[1];
  const bool two = a.two != 0;

  f32x16 acc0[NA][kNB], acc1[NA][kNB];
  zero(acc0);
  zero(acc1);
  TileLoader<AMAJ, kWavesOf<NA>> la0, la1;
  TileLoader<KMajor, kWavesOf<NA>> lx0, lx1;
  la0.init(A00, r0);
  la1.init(A01, r1);
  lx0.init(X0, tt.n0);
  lx1.init(X0, tt.n0 + kTileRows);
  Rsrc rs[4];
  auto prep = [&](int kt) __attribute__((always_inline)) {
    if (nk1 > 0 && kt == nk0) {  // switch to the second operand pair (chained K)
      la0.init(A10, r0);
      la1.init(A11, r1);
      lx0.init(X1, tt.n0);
      lx1.init(X1, tt.n0 + kTileRows);
    }
    const int lstep = nk1 > 0 && kt >= nk0 ? kt - nk0 : kt;
    rs[0] = la0.rsrc(lstep);
    rs[1] = la1.rsrc(lstep);
    rs[2] = lx0.rsrc(lstep);
    rs[3] = lx1.rsrc(lstep);
  };
  auto issue = [&](auto p, uint8_t* st) __attribute__((always_inline)) {
    constexpr int tile = decltype(p)::value / kLoadsPerTileOf<NA>;
    constexpr int t = decltype(p)::value % kLoadsPerTileOf<NA>;
    if constexpr (tile == 0) la0.issue(rs[0], t, st);
    else if constexpr (tile == 1) la1.issue(rs[1], t, st + kTileBytes);
    else if constexpr (tile == 2 && SKIP) lx0.issue_rows(rs[2], t, st + 2 * kTileBytes);
    else if constexpr (tile == 2) lx0.issue(rs[2], t, st + 2 * kTileBytes);
    else if constexpr (SKIP) lx1.issue_rows(rs[3], t, st + 3 * kTileBytes);
    else lx1.issue(rs[3], t, st + 3 * kTileBytes);
  };
  const int w = threadIdx.x >> 6;
  const int wm = w >> 1, wn = w & 1;
  (void)two;
  uint8_t* const ring[kStages] = {st0, st1};
  // SKIP: a wave whose first 32-token column block holds every token of its
  // half of the tile skips the MFMAs of its other three blocks (small
  // experts' tiles under skewed routing); loads, reads and barriers are the
  // same.  Without SKIP the branch is gone at compile time.
  const int vt = tt.size - tt.n0 - wn * (kBRows / 2);
  const bool full = !SKIP || __builtin_amdgcn_readfirstlane(vt > 32 ? 1 : 0) != 0;
  (void)vt;
  auto read = [&](const uint8_t* st, auto ks, HalfFrags<NA>& f, auto only)
                  __attribute__((always_inline)) {
    read_half<AMAJ, KMajor, decltype(ks)::value, kNB, decltype(only)::value, NA>(f, st, wm, wn);
  };
  run_pipeline<half_lds_ops<AMAJ, KMajor, kNB, NA>(), SKIP>(nk0 + nk1, full, prep, issue, read,
                                                             acc0, acc1, ring);
  const TokenTile tte{tt.e, after_loop(tt.start), after_loop(tt.size), after_loop(tt.n0)};
  const TileCtx c{after_loop(b), after_loop(m0), after_loop(wm), after_loop(wn), mt, tte,
                  reinterpret_cast<float*>(st0), reinterpret_cast<float*>(st1)};
  Epi::apply(ea, acc0, acc1, c, two);
}

// ==================================================== APPLY: skinny tiles ==
// The per-layer APPLY routes a few thousand rows over the experts, most of
// them few rows each under a skewed router, so its products stream every
// expert's weights once per token tile with little arithmetic per byte: they
// are bound by the bytes each CU keeps in flight.  tn_kernel keeps one 64 KiB
// stage in flight, half of it the token tile that is mostly clamped
// duplicates here.  This variant pairs the 256-row weight tile (A0 | A1 as in
// tn_kernel; A0 alone when !TWO) with 128-token tiles in a three-stage ring of
// 48 KiB stages, so two stages (96 KiB) are in flight while one is
// multiplied.  Wave w owns rows [32 w, 32 w + 32) of A0 and A1 and all four
// 32-column token blocks; the blocks past the segment end are not multiplied
// (JN blocks, the same for every wave).  Token rows past the segment are
// clamped copies of its last row (TileLoader), so no stale LDS data reaches
// any product.  The accumulation runs in the same k order with the same MFMA
// as tn_kernel, so both give identical results.
// Tile order: XCD x runs tiles [x * per_xcd, (x + 1) * per_xcd) of the
// (batch, m-tile, token tile) upper-bound order, token tile fastest: the
// token tiles of one expert and m-tile run together on one XCD and share the
// weight slice through its L2.  The down projection of one batch (em) instead
// cuts the real (token tile, m-tile) pairs into 8 equal XCD ranges in
// expert-major order (see apply_kernel).
constexpr int kApTok = 128;
constexpr int kApStageBytes = 3 * kTileBytes;  // A0 | A1 | X: 48 KiB, three of them

struct ApArgs {
  const uint16_t* a;  // weights of (b, e) at a + (b * E + e) * a_group, K-major rows
  const uint16_t* x;  // tokens [B, N, K]
  int64_t lda, a_group;
  int K;
  int row_off1;       // A1 row of tile row r: m0 + row_off1 + r
  int row_end0, row_end1;
  int m_step, m_tiles, n_tiles_ub;
  int64_t tiles, per_xcd;
  int B, E, N;
  int em;             // one batch: expert-major order over the real pairs (else upper-bound order)
  const int32_t* gs;
  // gathered token rows (src non-null): routed row p of batch b is row
  // src[b * src_sb + p] of x [B, T, K] instead of row p of a permuted copy
  const int32_t* src;
  int64_t src_sb;
  int T;
};

// Per-wave accumulators: acc[t][j] = rows [32 w, 32 w + 32) of tile t x token block j.
struct ApCtx {
  int b, m0, w;
  TokenTile tt;
  float* lds;  // the stage ring (144 KiB), free once the K loop is done
};

// The down projection's epilogue stages the tile through LDS: wave w writes its fp32
// values of rows 32 w .. 32 w + 31 (4 consecutive rows of one token per lane
// and MFMA quad) as [token][128 rows] (16-byte chunks XOR-swizzled by token,
// as stage_quarter), then thread t stores rows 8 (t % 16) .. +7 of token
// t / 16 (+ 16 per round): 16 lanes write 256 contiguous bytes of one token
// row instead of every store instruction touching 32 tokens.
__device__ __forceinline__ void ap_stage_quad(float* part, int n, int r, const float (&v)[4]) {
  *reinterpret_cast<float4*>(part + n * 128 + (((r >> 2) ^ (n & 31)) << 2)) =
      make_float4(v[0], v[1], v[2], v[3]);
}

// APPLY gate/up: h = y2 * silu(y0), token-major [B, N, I] (EpiSwiGLU's formula)
struct ApSwiGLU {
  struct Args {
    uint16_t* out;
    int I, N;
  };
  template <bool TWO>
  __device__ __forceinline__ static void apply(const Args& ea, const f32x16 (&acc)[2][4],
                                               const ApCtx& c) {
    static_assert(TWO, "gate/up pairs the w0 and w2 tiles");
    // straight from the accumulators: staging through LDS measured 1% slower
    // here (190.3 -> 192.1 us at the 760M chunk), unlike the down projection
    uint16_t* hb = ea.out + (int64_t)c.b * ea.N * ea.I;
    static_for<16>([&](auto idx) __attribute__((always_inline)) {
      constexpr int j = idx / 4, q = idx % 4;
      const int n = j * 32 + acc_col();
      const int m = c.m0 + c.w * 32 + acc_row(q * 4);
      if (c.tt.n0 + n >= c.tt.size || m >= ea.I) return;
      float h[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float y0 = acc[0][j][q * 4 + u], y2 = acc[1][j][q * 4 + u];
        h[u] = y2 * (y0 * sigmoidf_(y0));
      }
      store4(hb, ea.I, c.tt.start + c.tt.n0 + n, m, h[0], h[1], h[2], h[3]);
    });
  }
};

// Plain bf16 store of the tiles (both when TWO), token-major [B, N, ld]:
// tile t row r is column m0 + t * 128 + r, stored while below col_end.
struct ApStore {
  struct Args {
    uint16_t* out;
    int64_t ld;
    int col_end, N;
  };
  template <bool TWO>
  __device__ __forceinline__ static void apply(const Args& ea, const f32x16 (&acc)[2][4],
                                               const ApCtx& c) {
    uint16_t* ob = ea.out + (int64_t)c.b * ea.N * ea.ld;
    block_barrier();  // every wave is done reading the ring
    static_for<(TWO ? 2 : 1) * 16>([&](auto idx) __attribute__((always_inline)) {
      constexpr int t = idx / 16, j = (idx / 4) % 4, q = idx % 4;
      const float v[4] = {acc[t][j][q * 4], acc[t][j][q * 4 + 1], acc[t][j][q * 4 + 2],
                          acc[t][j][q * 4 + 3]};
      ap_stage_quad(c.lds + t * 128 * 128, j * 32 + acc_col(), c.w * 32 + acc_row(q * 4), v);
    });
    block_barrier();
#pragma unroll 1
    for (int k = 0; k < 8; ++k) {
      const int it = threadIdx.x + kThreads * k;
      const int n = it >> 4, g = it & 15;
      if (c.tt.n0 + n >= c.tt.size) continue;
      uint16_t* row = ob + (int64_t)(c.tt.start + c.tt.n0 + n) * ea.ld;
#pragma unroll
      for (int t = 0; t < (TWO ? 2 : 1); ++t) {
        const int col = c.m0 + t * kTileRows + 8 * g;
        if (col >= ea.col_end) continue;  // col_end is a multiple of 8
        float v[8];
        staged8(c.lds + t * 128 * 128, n, g, v);
        store8(row + col, v);
      }
    }
  }
};

struct ApFrags {
  bf16x8 a[2], b[4];
};

// s_waitcnt lgkmcnt(N) that redefines the fragment registers (no MFMA that
// reads them can move above it).
template <int N>
__device__ __forceinline__ void ap_lgkm_wait(ApFrags& f) {
  i32x4 r[6] = {__builtin_bit_cast(i32x4, f.a[0]), __builtin_bit_cast(i32x4, f.a[1]),
                __builtin_bit_cast(i32x4, f.b[0]), __builtin_bit_cast(i32x4, f.b[1]),
                __builtin_bit_cast(i32x4, f.b[2]), __builtin_bit_cast(i32x4, f.b[3])};
  asm volatile("s_waitcnt lgkmcnt(%6)"
               : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]), "+v"(r[4]), "+v"(r[5])
               : "i"(N)
               : "memory");
  f.a[0] = __builtin_bit_cast(bf16x8, r[0]);
  f.a[1] = __builtin_bit_cast(bf16x8, r[1]);
  f.b[0] = __builtin_bit_cast(bf16x8, r[2]);
  f.b[1] = __builtin_bit_cast(bf16x8, r[3]);
  f.b[2] = __builtin_bit_cast(bf16x8, r[4]);
  f.b[3] = __builtin_bit_cast(bf16x8, r[5]);
}

// Fragment reads of k-substep KS of the stage at LDS byte address s: A rows
// of this wave (A1 when TWO) and the JN token blocks.  LDS ops: TWO + 1 + JN.
template <bool TWO, int JN, int KS>
__device__ __forceinline__ void ap_read(ApFrags& f, uint32_t s, uint32_t a_lane) {
  constexpr int kRow = kChunks * 16;
  const uint32_t l = s + kmaj_lane<KS>();
  f.a[0] = ds_b128_asm<0>(l + a_lane);
  if constexpr (TWO) f.a[1] = ds_b128_asm<kTileBytes>(l + a_lane);
  static_for<JN>([&](auto J) __attribute__((always_inline)) {
    f.b[J] = ds_b128_asm<2 * kTileBytes + decltype(J)::value * 32 * kRow>(l);
  });
}

template <bool TWO, int JN>
__device__ __forceinline__ void ap_mma(f32x16 (&acc)[2][4], const ApFrags& f) {
  static_for<JN>([&](auto J) __attribute__((always_inline)) {
    constexpr int j = J;
    acc[0][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[0], f.b[j], acc[0][j], 0, 0, 0);
    if constexpr (TWO)
      acc[1][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[1], f.b[j], acc[1][j], 0, 0, 0);
  });
}

// The K loop.  Step k: wait for stage k's loads (stage k+1's may stay in
// flight), barrier
// (stage k visible to every wave; every wave done reading the buffer of stage
// k-1), issue stage k+2 into that buffer, then the four k-substeps of stage k
// with the fragments of substep s+1 read while substep s multiplies.
template <bool TWO, int JN>
__device__ __forceinline__ void ap_loop(TileLoader<KMajor>& la0, TileLoader<KMajor>& la1,
                                        TileLoader<KMajor>& lx, int nk, uint8_t* ring,
                                        f32x16 (&acc)[2][4]) {
  // load T of a wave covers token rows 32 T .. 32 T + 31 of the tile (8 per
  // wave), so only the JN blocks that are multiplied are loaded; the LDS rows
  // of the others keep stale data that no fragment read touches
  constexpr int kLPS = (TWO ? 2 : 1) * kLoadsPerTile + JN;
  constexpr int kOps = (TWO ? 2 : 1) + JN;
  auto issue_stage = [&](int k, uint8_t* st) __attribute__((always_inline)) {
    const Rsrc r0 = la0.rsrc(k);
    const Rsrc r1 = TWO ? la1.rsrc(k) : r0;
    const Rsrc rx = lx.rsrc(k);
    static_for<kLoadsPerTile>([&](auto T) __attribute__((always_inline)) {
      la0.issue(r0, T, st);
      if constexpr (TWO) la1.issue(r1, T, st + kTileBytes);
      if constexpr (decltype(T)::value < JN) lx.issue(rx, T, st + 2 * kTileBytes);
    });
  };
  const uint32_t a_lane = (uint32_t)(wave_id() * 32 * kChunks * 16);
  uint8_t* p0 = ring;
  uint8_t* p1 = ring + kApStageBytes;
  uint8_t* p2 = ring + 2 * kApStageBytes;
  issue_stage(0, p0);
  if (nk > 1) issue_stage(1, p1);
  ApFrags f[2];
  for (int k = 0; k < nk; ++k) {
    if (k + 1 < nk)
      wait_vmcnt<kLPS>();
    else
      wait_vmcnt<0>();
    block_barrier();
    __builtin_amdgcn_sched_barrier(0);
    if (k + 2 < nk) issue_stage(k + 2, p2);
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t s = lds_addr(p0);
    ap_read<TWO, JN, 0>(f[0], s, a_lane);
    static_for<kSubsteps>([&](auto KS) __attribute__((always_inline)) {
      constexpr int ks = KS;
      if constexpr (ks + 1 < kSubsteps) {
        ap_read<TWO, JN, ks + 1>(f[(ks + 1) & 1], s, a_lane);
        ap_lgkm_wait<kOps>(f[ks & 1]);
      } else {
        ap_lgkm_wait<0>(f[ks & 1]);
      }
      ap_mma<TWO, JN>(acc, f[ks & 1]);
      __builtin_amdgcn_sched_barrier(0);
    });
    uint8_t* t = p0;
    p0 = p1;
    p1 = p2;
    p2 = t;
  }
}

template <class Epi, bool TWO>
__global__ __launch_bounds__(kThreads) void apply_kernel(ApArgs a, typename Epi::Args ea) {
  __shared__ __attribute__((aligned(16))) uint8_t ring[3 * kApStageBytes];
  const int bid = blockIdx.x;
  int mt, b;
  TokenTile tt;
  if (a.em) {
    // One batch: the real pair count R * m_tiles is known on the device, so
    // the pairs are cut into 8 equal XCD ranges in expert-major order (token
    // tile fastest inside an expert): an XCD streams each of its experts'
    // weight slices once and reuses it from L2 for that expert's token tiles,
    // and reads a small expert's tokens once for all its m-tiles.  Workgroups
    // past their XCD's range leave at once.
    tt = find_pair_em_xcd<kApTok>(a.gs, a.E, a.N, a.m_tiles, bid, &mt);
    b = 0;
  } else {
    const int64_t t = (int64_t)(bid % kXcds) * a.per_xcd + bid / kXcds;
    if (t >= a.tiles) return;
    const int nt = (int)(t % a.n_tiles_ub);
    const int64_t rest = t / a.n_tiles_ub;
    mt = (int)(rest % a.m_tiles);
    b = (int)(rest / a.m_tiles);
    tt = find_token_tile<kApTok>(a.gs + (int64_t)b * a.E, a.E, a.N, nt);
  }
  if (tt.e < 0) return;
  const int m0 = mt * a.m_step;
  const int64_t ag = ((int64_t)b * a.E + tt.e) * a.a_group;
  const Operand A0{a.a + ag, a.lda, a.row_end0, a.K};
  const Operand A1{a.a + ag, a.lda, a.row_end1, a.K};
  const Operand X{a.x + ((int64_t)b * a.N + tt.start) * a.K, a.K, tt.size, a.K};
  TileLoader<KMajor> la0, la1, lx;
  la0.init(A0, m0);
  la1.init(A1, m0 + a.row_off1);
  if (a.src != nullptr)
    lx.init_gather(a.x + (int64_t)b * a.T * a.K, a.K, a.K,
                   a.src + b * a.src_sb + tt.start + tt.n0, tt.size - tt.n0, a.T);
  else
    lx.init(X, tt.n0);
  const int nk = (a.K + kBK - 1) / kBK;
  f32x16 acc[2][4];
  zero(acc);
  const int valid = tt.size - tt.n0;  // >= 1
  const int jn = valid >= 3 * 32 + 1 ? 4 : (valid + 31) / 32;
  if (jn == 4) ap_loop<TWO, 4>(la0, la1, lx, nk, ring, acc);
  else if (jn == 3) ap_loop<TWO, 3>(la0, la1, lx, nk, ring, acc);
  else if (jn == 2) ap_loop<TWO, 2>(la0, la1, lx, nk, ring, acc);
  else ap_loop<TWO, 1>(la0, la1, lx, nk, ring, acc);
  const TokenTile tte{tt.e, after_loop(tt.start), after_loop(tt.size), after_loop(tt.n0)};
  const ApCtx c{after_loop(b), after_loop(m0), after_loop((int)(threadIdx.x >> 6)), tte,
                 reinterpret_cast<float*>(ring)};
  Epi::template apply<TWO>(ea, acc, c);
}

// ======================================================= weight gradients ==
// out[b, e, x, y] = sum_{n in seg(b,e)} P[b, n, y] Q[b, n, x]; P [B, N, Y] and
// Q [B, N, X] token-major.  A tile = 2 x 128 rows of y, B tile = 256 rows of
// x, so every lane holds four consecutive y of one x: 8-byte stores along the
// contiguous y axis.  Up to two tasks share a launch.
//
// Split K: when the launch has too few output tiles to fill the chip (one
// expert with small weights, the dense case), each tile's token segment is cut
// into `splits` runs of whole K steps; workgroup (tile, s) writes its fp32
// partial product to part[s][b, e] and wg_reduce_kernel sums the partials in
// split order into the bf16 output (deterministic).
struct WgTask {
  const uint16_t* p;
  const uint16_t* q;
  uint16_t* out;
  float* part;  // [splits][B*E][X][Y] fp32 when splits > 1
  int X, Y;
  int y_tiles, x_tiles;
};

// The uTTT-Dense aggregate write's token operands straight from every
// layer's own tensors (LAYERED): one expert per batch (head) bh = bb * H + hh
// with all N = L * l tokens, split K once per layer (run = l, a multiple of
// kBK), and run li reads task 0's P (k) and task 1's Q (v) as layer li's
// [b, l, H*D] rows bb * l .. + l at column hh * D (row stride H * D).
struct WgLayers {
  LayerPtrs k, v;
  int l, H, D;
};

// SPLIT: fp32 partials (the two epilogues in one kernel do not fit the
// register file: each alone does)
template <bool SPLIT, int NA, bool LAYERED = false>
__global__ __launch_bounds__(kThreadsOf<NA>) void wg_kernel(WgTask t0, WgTask t1,
                                                      const int32_t* __restrict__ gs, int E,
                                                      int N, int BE, int splits,
                                                      WgLayers ly) {
  __shared__ __attribute__((aligned(16))) uint8_t st0[kStageBytes];
  __shared__ __attribute__((aligned(16))) uint8_t st1[kStageBytes];

  const int n0_tiles = t0.y_tiles * t0.x_tiles;
  const int per_group = n0_tiles + t1.y_tiles * t1.x_tiles;
  const int bid = blockIdx.x;
  const int t = bid % per_group;  // tiles of one (split, b, e) are neighbours: shared rows in L2
  const int be = (bid / per_group) % BE;
  const int split = bid / per_group / BE;
  const int b = be / E, e = be % E;
  const bool first = t < n0_tiles;
  const WgTask& tk = first ? t0 : t1;
  const int tl = first ? t : t - n0_tiles;
  const int y0 = (tl / tk.x_tiles) * 2 * kTileRows;
  const int x0 = (tl % tk.x_tiles) * kBRows;
  const int X = tk.X, Y = tk.Y;

  int start, size;
  if constexpr (LAYERED) {
    start = 0;  // the head's whole token axis (group sizes are not read)
    size = N;
  } else {
    expert_segment(gs + (int64_t)b * E, e, N, &start, &size);
  }
  // this split's run of the segment: whole K steps, the last run may be short or empty
  const int run = ((size + kBK - 1) / kBK + splits - 1) / splits * kBK;
  const int lo = min(size, split * run);
  size = min(size - lo, run);
  start += lo;
  Operand P{tk.p + ((int64_t)b * N + start) * Y, Y, Y, size};
  Operand Q{tk.q + ((int64_t)b * N + start) * X, X, X, size};
  if constexpr (LAYERED) {
    // run == l: this split is layer `split`, its first token row bb * l
    const int bb = b / ly.H, hh = b - bb * ly.H;
    const int64_t off = (int64_t)bb * ly.l * ly.H * ly.D + (int64_t)hh * ly.D;
    const int64_t ld = (int64_t)ly.H * ly.D;
    if (first)
      P = Operand{static_cast<const uint16_t*>(ly.k.p[split]) + off, ld, Y, size};
    else
      Q = Operand{static_cast<const uint16_t*>(ly.v.p[split]) + off, ld, X, size};
  }

  f32x16 acc0[NA][kNB], acc1[NA][kNB];
  zero(acc0);
  zero(acc1);
  TileLoader<RMajor, kWavesOf<NA>> lp0, lp1, lq0, lq1;
  lp0.init(P, y0);
  lp1.init(P, y0 + kTileRows);
  lq0.init(Q, x0);
  lq1.init(Q, x0 + kTileRows);
  Rsrc rs[4];
  auto prep = [&](int kt) __attribute__((always_inline)) {
    rs[0] = lp0.rsrc(kt);
    rs[1] = lp1.rsrc(kt);
    rs[2] = lq0.rsrc(kt);
    rs[3] = lq1.rsrc(kt);
  };
  auto issue = [&](auto p, uint8_t* st) __attribute__((always_inline)) {
    constexpr int tile = decltype(p)::value / kLoadsPerTileOf<NA>;
    constexpr int t = decltype(p)::value % kLoadsPerTileOf<NA>;
    if constexpr (tile == 0) lp0.issue(rs[0], t, st);
    else if constexpr (tile == 1) lp1.issue(rs[1], t, st + kTileBytes);
    else if constexpr (tile == 2) lq0.issue(rs[2], t, st + 2 * kTileBytes);
    else lq1.issue(rs[3], t, st + 3 * kTileBytes);
  };
  const int w = threadIdx.x >> 6;
  const int wm = w >> 1, wn = w & 1;
  auto read = [&](const uint8_t* st, auto ks, HalfFrags<NA>& f, auto only)
                  __attribute__((always_inline)) {
    read_half<RMajor, RMajor, decltype(ks)::value, kNB, decltype(only)::value, NA>(f, st, wm, wn);
  };
  uint8_t* const ring[kStages] = {st0, st1};
  run_pipeline<half_lds_ops<RMajor, RMajor, kNB, NA>(), false>((size + kBK - 1) / kBK, true, prep,
                                                               issue, read, acc0, acc1, ring);

  // the epilogue re-derives its indices from an opaque copy of the block id,
  // so none of them is held across the K loop
  const int bid2 = __builtin_amdgcn_readfirstlane(after_loop(bid));
  const int t2 = bid2 % per_group;
  const int be2 = (bid2 / per_group) % BE;
  const bool first2 = t2 < n0_tiles;
  const WgTask& tk2 = first2 ? t0 : t1;
  const int tl2 = first2 ? t2 : t2 - n0_tiles;
  const int ye = (tl2 / tk2.x_tiles) * 2 * kTileRows, xe = (tl2 % tk2.x_tiles) * kBRows;
  const int X2 = tk2.X, Y2 = tk2.Y;
  if constexpr (!SPLIT) {
    // through the LDS frame (16-byte stores, 256 contiguous bytes per x row);
    // the launcher passes 16-byte-aligned outputs only (Y is a multiple of 8)
    uint16_t* ob = tk2.out + (int64_t)be2 * X2 * Y2;
    const TileCtx c{0, 0, after_loop(wm), after_loop(wn), 0, TokenTile{0, 0, 0, 0},
                    reinterpret_cast<float*>(st0), reinterpret_cast<float*>(st1)};
    staged_epilogue(acc0, acc1, c, [&](int nl, int n, int g) __attribute__((always_inline)) {
      const int x = xe + n;
      if (x >= X2) return;
      uint16_t* row = ob + (int64_t)x * Y2;
      static_for<2>([&](auto T) __attribute__((always_inline)) {
        const int y = ye + decltype(T)::value * kTileRows + 8 * g;
        if (y >= Y2) return;
        float v[8];
        staged8(decltype(T)::value == 0 ? c.lds0 : c.lds1, nl, g, v);
        store8(row + y, v);
      });
    });
  } else {
    float* pb = tk2.part + ((int64_t)(bid2 / per_group / BE) * BE + be2) * X2 * Y2;
    for_quads(acc0, acc1, after_loop(wm), after_loop(wn), true, [&](int tt, int r, int n, const float* v) __attribute__((always_inline)) {
      const int y = ye + tt * kTileRows + r;
      const int x = xe + n;
      if (y < Y2 && x < X2) store4(pb, Y2, x, y, v[0], v[1], v[2], v[3]);
    });
  }
}

typedef float nt_f32x4 __attribute__((ext_vector_type(4)));

// out = bf16(sum_s part[s]) over both tasks' n0 and n1 elements (multiples of
// 8), the splits added in order 0, 1, ...; partials are read once (non-temporal).
__global__ __launch_bounds__(256) void wg_reduce_kernel(WgTask t0, WgTask t1, int64_t n0,
                                                        int64_t n1, int splits) {
  const int64_t g0 = n0 / 8, total = g0 + n1 / 8;
  for (int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x; g < total;
       g += (int64_t)gridDim.x * 256) {
    const bool first = g < g0;
    const float* part = first ? t0.part : t1.part;
    uint16_t* out = first ? t0.out : t1.out;
    const int64_t n = first ? n0 : n1;
    const int64_t i = (first ? g : g - g0) * 8;
    nt_f32x4 a = {0.f, 0.f, 0.f, 0.f}, c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
    for (int s = 0; s < splits; ++s) {
      const nt_f32x4* src = reinterpret_cast<const nt_f32x4*>(part + s * n + i);
      a += __builtin_nontemporal_load(src);
      c += __builtin_nontemporal_load(src + 1);
    }
    uint4 w;
    w.x = pack_bf16x2(a.x, a.y);
    w.y = pack_bf16x2(a.z, a.w);
    w.z = pack_bf16x2(c.x, c.y);
    w.w = pack_bf16x2(c.z, c.w);
    *reinterpret_cast<uint4*>(out + i) = w;
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

// ============================================ Newton-Schulz orthogonalisation ==
// Per matrix G [R, C] (BE of them): X = bf16(G) as [m, n] = [min, max] (G
// transposed when R > C), X /= bf16(bf16(||X||_F) + 1e-7), five steps of
// A = X X^T, B = b A + (c A) A, X = a X + B X, then bf16(X * scale) back in
// G's orientation.  Reference: zeropower_via_newtonschulz5,
// uttt_llm/flame/custom_models/uttt_moe/ttt_operation.py:19-46.
constexpr int kNsParts = 64;   // partial sums of squares per matrix

// part[be, p] = sum of bf16(g)^2 over the p-th of kNsParts equal slices of matrix be.
template <class TT>
__global__ __launch_bounds__(256) void ns_sumsq_kernel(const typename TT::S* __restrict__ g,
                                                       int64_t elems, float* __restrict__ part) {
  __shared__ float red[256];
  const int be = blockIdx.y, p = blockIdx.x;
  const int64_t per = (elems + kNsParts - 1) / kNsParts;
  const int64_t lo = p * per, hi = lo + per < elems ? lo + per : elems;
  const typename TT::S* gb = g + (int64_t)be * elems;
  float acc = 0.0f;
  for (int64_t i = lo + threadIdx.x; i < hi; i += 256) {
    const float x = bf16r(TT::load(gb[i]));
    acc = __builtin_fmaf(x, x, acc);
  }
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) part[(int64_t)be * kNsParts + p] = red[0];
}

// denom[be] = bf16(bf16(sqrt(sum of parts)) + 1e-7) (fixed order); gs[be] = m.
__global__ __launch_bounds__(256) void ns_norm_kernel(const float* __restrict__ part, int BE,
                                                      int m, float* __restrict__ denom,
                                                      int32_t* __restrict__ gs) {
  const int be = blockIdx.x * 256 + threadIdx.x;
  if (be >= BE) return;
  float s = 0.0f;
  for (int p = 0; p < kNsParts; ++p) s += part[(int64_t)be * kNsParts + p];
  denom[be] = bf16r(bf16r(sqrtf(s)) + 1e-7f);
  gs[be] = m;
}

// dst [BE, Rd, Cd] from src [BE, Rs, Cs] through 64x64 LDS tiles; TRANS: dst = src^T.
//   PREP:  dst = bf16(bf16(src) / denom[be])
//   FINAL: dst = bf16(src * scale)
template <class TS, bool TRANS, bool PREP>
__global__ __launch_bounds__(256) void ns_tile_kernel(const typename TS::S* __restrict__ src,
                                                      int Rs, int Cs, const float* __restrict__ denom,
                                                      float scale, uint16_t* __restrict__ dst,
                                                      int rt, int ct) {
  __shared__ float tile[64][65];
  const int bid = blockIdx.x;
  const int tc = bid % ct, tr = (bid / ct) % rt, be = bid / (ct * rt);
  const int Rd = TRANS ? Cs : Rs, Cd = TRANS ? Rs : Cs;
  const typename TS::S* sb = src + (int64_t)be * Rs * Cs;
  uint16_t* db = dst + (int64_t)be * Rd * Cd;
  const float mul = PREP ? 0.0f : scale;
  const float dv = PREP ? denom[be] : 1.0f;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  // source tile rows/cols: the dst tile (tr, tc) maps to src tile (tc, tr) when transposing
  const int sr0 = (TRANS ? tc : tr) * 64, sc0 = (TRANS ? tr : tc) * 64;
  for (int yy = ty; yy < 64; yy += 4) {
    const int r = sr0 + yy, cc = sc0 + tx;
    float v = 0.0f;
    if (r < Rs && cc < Cs) {
      const float x = TS::load(sb[(int64_t)r * Cs + cc]);
      v = PREP ? bf16r(bf16r(x) / dv) : bf16r(x * mul);
    }
    tile[yy][tx] = v;
  }
  __syncthreads();
  for (int yy = ty; yy < 64; yy += 4) {
    const int r = tr * 64 + yy, cc = tc * 64 + tx;
    if (r < Rd && cc < Cd) db[(int64_t)r * Cd + cc] = f32_to_bf16(TRANS ? tile[tx][yy] : tile[yy][tx]);
  }
}

// ------------------------------------------------------------- host side ----
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_grid(int64_t blocks, const char* what) {
  if (blocks > 0x7fffffffLL) {
    set_error("%s: problem too large for one launch (%lld workgroups)", what, (long long)blocks);
    return UTTT_ERR_UNSUPPORTED;
  }
  return UTTT_OK;
}



// TnArgs of one token-grouped product family.
TnArgs tn_args(const void* a0, const void* a1, const void* x, int K, int64_t lda, int64_t a_group,
               int off0, int off1, int end0, int end1, int m_step, int M_rows, int B, int E,
               int N, const int32_t* gs) {
  TnArgs t{};
  t.a[0][0] = static_cast<const uint16_t*>(a0);
  t.a[0][1] = static_cast<const uint16_t*>(a1);
  t.a[1][0] = t.a[0][0];
  t.a[1][1] = t.a[0][1];
  t.x[0] = static_cast<const uint16_t*>(x);
  t.x[1] = t.x[0];
  t.K[0] = K;
  t.K[1] = 0;
  t.lda = lda;
  t.a_group = a_group;
  t.row_off[0] = off0;
  t.row_off[1] = off1;
  t.row_end[0] = end0;
  t.row_end[1] = end1;
  t.m_step = m_step;
  t.m_tiles = (M_rows + m_step - 1) / m_step;
  t.n_tiles_ub = (N + kBRows - 1) / kBRows + E;
  t.E = E;
  t.N = N;
  t.two = 1;
  t.sym = 0;
  t.gs = gs;
  (void)B;
  return t;
}

// Grids from this many tiles up (8 rounds of one workgroup per CU) take the
// XCD super-tile order.  A process-wide value so that tests can send small
// grids down the same path (uttt_debug_set_supertile_min_tiles).
constexpr int64_t kXcdMapMinTiles = 8 * 256;
int64_t g_xcd_map_min_tiles = kXcdMapMinTiles;

// Super-tile shape for m_tiles m-tiles: gm x gn with gm * gn <= 32 (one
// workgroup per CU of an XCD), minimising the slices fetched per tile,
// (gm + gn) / (gm gn), times the m padding.
void super_tile(int m_tiles, int* gm, int* gn) {
  double best = 1e30;
  for (int m = 1; m <= 8 && m <= m_tiles; ++m) {
    const int n = 32 / m;
    const double pad = (double)((m_tiles + m - 1) / m * m) / m_tiles;
    const double score = (double)(m + n) / (m * n) * pad;
    if (score < best - 1e-9) {
      best = score;
      *gm = m;
      *gn = n;
    }
  }
}

// Epilogues whose launches take the MFMA-skipping variant when tokens per
// expert are few (the per-layer APPLY): K-major gate/up and bf16 products.
// The variant leaves stale LDS contents (possibly NaN / Inf from an earlier
// kernel) in the products of token columns past the segment, so an epilogue
// may join only if it never touches those columns (kStaleColumnsUnused).
template <int AMAJ, class Epi>
constexpr bool kSkippable =
    AMAJ == KMajor && (std::is_same_v<Epi, EpiSwiGLU> || std::is_same_v<Epi, EpiStore<uint16_t>> ||
                       std::is_same_v<Epi, EpiStore<uint16_t, true>>);
static_assert(kSkippable<KMajor, EpiSwiGLU> <= EpiSwiGLU::kStaleColumnsUnused &&
                  kSkippable<KMajor, EpiStore<uint16_t>> <= EpiStore<uint16_t>::kStaleColumnsUnused &&
                  kSkippable<KMajor, EpiStore<uint16_t, true>> <=
                      EpiStore<uint16_t, true>::kStaleColumnsUnused &&
                  !kSkippable<KMajor, EpiS1<BF16T>> && !kSkippable<KMajor, EpiBwd<BF16T>> &&
                  !kSkippable<KMajor, EpiBwdSaved<BF16T>>,
              "the SKIP variant needs an epilogue that ignores stale token columns");

// Wave layout of the token-grouped and weight-gradient products (NA of
// gemm_pipe.h): 2 = four waves, one per SIMD; 1 = eight waves, two per SIMD.
// kDefaultNA is the layout each family launches with;
// uttt_debug_set_gemm_layout forces one process-wide (tests run both).
// Measured at the 760M batched-update shapes (interleaved runs, per launch):
// the staged bf16 stores (GD and grad_K, row-major A: 2279 -> 2185-2207 us;
// grad_V: 1720 / 1722 us) and the saved-tensor backward epilogue (bf16 lr:
// 2845-2849 against 2719-2735 us, its inputs fetched per quarter) take eight
// waves; the weight gradients (2393-2408 against 2440-2448 us) and the rest
// (stage 1 2358 / 2346-2351, DH 1057-1060 / 1054-1068) keep four.
template <class Epi>
constexpr int kDefaultNA = 2;
template <>
constexpr int kDefaultNA<EpiStore<uint16_t, true>> = 1;
template <>
constexpr int kDefaultNA<EpiBwdSaved<BF16T>> = 1;
constexpr int kDefaultWgNA = 2;
// Epilogues with an eight-wave kernel (every one here; a family without one
// would set this false and launch four waves under a forced layout too).
template <class Epi>
constexpr bool kHasNA1 = true;
int g_gemm_na = 0;  // 0: each family's default
int g_ns_path = 0;  // uttt_newton_schulz5: 0 by the sizes, 1 always the multi-launch path
int pick_na(int def) { return g_gemm_na != 0 ? g_gemm_na : def; }

template <int AMAJ, class Epi, bool SKIP, int NA>
void launch_tn_kernel(int64_t blocks, const TnArgs& t, const typename Epi::Args& ea,
                      hipStream_t st) {
  hipLaunchKernelGGL((tn_kernel<AMAJ, Epi, SKIP, NA>), dim3((unsigned)blocks),
                     dim3(kThreadsOf<NA>), 0, st, t, ea);
}

template <int AMAJ, class Epi, bool SKIP>
void launch_tn_layout(int64_t blocks, const TnArgs& t, const typename Epi::Args& ea,
                      hipStream_t st) {
  if constexpr (kHasNA1<Epi>) {
    if (pick_na(kDefaultNA<Epi>) == 1) {
      launch_tn_kernel<AMAJ, Epi, SKIP, 1>(blocks, t, ea, st);
      return;
    }
  }
  launch_tn_kernel<AMAJ, Epi, SKIP, 2>(blocks, t, ea, st);
}

template <int AMAJ, class Epi>
int launch_tn(TnArgs t, const typename Epi::Args& ea, int B, hipStream_t st,
              const char* what) {
  const int64_t tiles = (int64_t)t.m_tiles * t.n_tiles_ub * B;
  if (tiles == 0) return UTTT_OK;
  // the tile loads keep 32-bit lane offsets below 2^31 (bit 31 marks the K
  // tail): 128 rows of at most 2^23 elements
  UTTT_REQUIRE(t.lda < (1 << 23) && t.K[0] < (1 << 23) && t.K[1] < (1 << 23),
               "%s: operand rows of 2^23 or more elements are not supported", what);
  t.B = B;
  int64_t blocks = tiles;
  if (tiles >= g_xcd_map_min_tiles) {
    super_tile(t.m_tiles, &t.gm, &t.gn);
    t.n_super_m = (t.m_tiles + t.gm - 1) / t.gm;
    const int64_t n_super_n = ((int64_t)B * t.n_tiles_ub + t.gn - 1) / t.gn;
    const int64_t supers = (t.n_super_m * n_super_n + kXcds - 1) / kXcds * kXcds;
    blocks = supers * t.gm * t.gn;
  } else {
    t.gm = t.gn = 0;
    t.n_super_m = 1;
  }
  if (int rc = check_grid(blocks, what)) return rc;
  // fewer than 256 tokens per expert on average: many tiles at segment ends
  if constexpr (kSkippable<AMAJ, Epi>) {
    static_assert(Epi::kStaleColumnsUnused, "SKIP variant with an epilogue that reads stale columns");
    if ((int64_t)t.N < (int64_t)kBRows * t.E) {
      launch_tn_layout<AMAJ, Epi, true>(blocks, t, ea, st);
      return check_launch(what);
    }
  }
  launch_tn_layout<AMAJ, Epi, false>(blocks, t, ea, st);
  return check_launch(what);
}

// APPLY path: 0 = tn_kernel, 1 = apply_kernel, -1 = by the sizes.  Both give
// identical results; a process-wide value so that tests can run either path
// (uttt_debug_set_apply_path).
int g_apply_path = -1;
bool g_apply_down_two = false;  // down products on 256-row tiles (default 128: twice the tiles)
constexpr int kCUs = 256;       // MI355X compute units

// Gate/up (256-row weight tiles either way): the skinny 128-token tiles when
// the experts average at most 256 routed rows (configs[3]: 129 -> 100 us per
// apply with the down projection below; configs[4] gate/up 188 -> 184 us).
bool use_apply_kernel(int64_t N, int E) {
  return g_apply_path == 1 || g_apply_path == 2 ||
         (g_apply_path < 0 && N <= (int64_t)kBRows * E);
}

// The down projection (and every uttt_grouped_gemm_nt): the skinny tiles
// (128 weight rows x 128 tokens) when the general 256x256 tiles would not
// fill the chip once even at their upper-bound count, else the general tiles.
// configs[3] (3 x 32 tiles of 256): 38.9 -> 21.5 us; configs[4] (6 x 48):
// the general tiles, 101 us against 110 us on the skinny ones.
bool use_apply_kernel_nt(int64_t N, int E, int B, int M) {
  if (g_apply_path >= 0) return g_apply_path > 0;
  if (N > (int64_t)kBRows * E) return false;
  const int64_t tn_tiles =
      (int64_t)B * ((M + kBRows - 1) / kBRows) * ((N + kBRows - 1) / kBRows + E);
  return tn_tiles < kCUs;
}

template <class Epi, bool TWO>
int launch_apply(ApArgs a, int M_rows, const typename Epi::Args& ea, hipStream_t st,
                 const char* what) {
  a.m_tiles = (M_rows + a.m_step - 1) / a.m_step;
  a.n_tiles_ub = (a.N + kApTok - 1) / kApTok + a.E;
  a.tiles = (int64_t)a.B * a.m_tiles * a.n_tiles_ub;
  if (a.tiles == 0) return UTTT_OK;
  UTTT_REQUIRE(a.lda < (1 << 23) && a.K < (1 << 23),
               "%s: operand rows of 2^23 or more elements are not supported", what);
  // the expert-major order measured 5% faster for the down projection and 4%
  // slower for gate/up (whose 256-row weight tiles are read by more m-tiles)
  a.em = a.B == 1 && std::is_same_v<Epi, ApStore>;
  a.per_xcd = (a.tiles + kXcds - 1) / kXcds;
  const int64_t blocks = a.per_xcd * kXcds;
  if (int rc = check_grid(blocks, what)) return rc;
  hipLaunchKernelGGL((apply_kernel<Epi, TWO>), dim3((unsigned)blocks), dim3(kThreads), 0, st, a,
                     ea);
  return check_launch(what);
}

// The weight-streaming APPLY products on apply_kernel: w [B, E, M, K] K-major,
// x [B, N, K]; A1 rows at row_off1 (TWO).
ApArgs apply_args(const void* w, const void* x, int K, int64_t a_group, int row_off1, int end0,
                  int end1, int m_step, int B, int E, int N, const int32_t* gs) {
  ApArgs a{};
  a.a = static_cast<const uint16_t*>(w);
  a.x = static_cast<const uint16_t*>(x);
  a.lda = K;
  a.a_group = a_group;
  a.K = K;
  a.row_off1 = row_off1;
  a.row_end0 = end0;
  a.row_end1 = end1;
  a.m_step = m_step;
  a.B = B;
  a.E = E;
  a.N = N;
  a.gs = gs;
  return a;
}

// Wide single product: y[b, n, m] = sum_k A(m, k) x[b, n, k] with M rows in
// m-tiles of 256 (tile 1 = rows +128).  Optional second pair chained on K.
template <int AMAJ, class OutT>
int launch_wide(const void* a, const void* x, int K, const void* a_2, const void* x_2, int K_2,
                int M, int64_t lda, int64_t a_group, OutT* y, int B, int E, int N,
                const int32_t* gs, hipStream_t st, const char* what) {
  TnArgs t = tn_args(a, a, x, K, lda, a_group, 0, kTileRows, M, M, 2 * kTileRows, M, B, E, N, gs);
  if (K_2 > 0) {
    t.a[1][0] = t.a[1][1] = static_cast<const uint16_t*>(a_2);
    t.x[1] = static_cast<const uint16_t*>(x_2);
    t.K[1] = K_2;
  }
  const EpiStoreArgs<OutT> ea{y, M, {0, kTileRows}, {M, M}, N};
  if (aligned16(y)) return launch_tn<AMAJ, EpiStore<OutT, true>>(t, ea, B, st, what);
  return launch_tn<AMAJ, EpiStore<OutT>>(t, ea, B, st, what);
}

// y[b, n, m] = bf16(bf16(alpha in) + bf16(beta bf16(sum_k A(m, k) x[b, n, k]))) (and
// y2 = bf16(gamma y) when y2), E = 1 group of N rows per batch, M rows in m-tiles of 256.
template <int AMAJ>
int launch_lincomb(const void* a, const void* x, int K, int M, int64_t lda, int64_t a_group,
                   const uint16_t* in, float alpha, float beta, uint16_t* y, uint16_t* y2,
                   float gamma, int B, int N, const int32_t* gs, hipStream_t st,
                   const char* what, bool sym = false) {
  TnArgs t = tn_args(a, a, x, K, lda, a_group, 0, kTileRows, M, M, 2 * kTileRows, M, B, 1, N, gs);
  t.sym = sym ? 1 : 0;
  const EpiLinCombArgs ea{y, y2, in, M, M, N, alpha, beta, gamma};
  if (sym) return launch_tn<AMAJ, EpiLinComb<true>>(t, ea, B, st, what);
  return launch_tn<AMAJ, EpiLinComb<>>(t, ea, B, st, what);
}

WgTask wg_task(const void* p, const void* q, void* out, int X, int Y) {
  WgTask t;
  t.p = static_cast<const uint16_t*>(p);
  t.q = static_cast<const uint16_t*>(q);
  t.out = static_cast<uint16_t*>(out);
  t.part = nullptr;
  t.X = X;
  t.Y = Y;
  t.y_tiles = (Y + 2 * kTileRows - 1) / (2 * kTileRows);
  t.x_tiles = (X + kBRows - 1) / kBRows;
  return t;
}

// Split K is used when the tiles fill under half of the chip's 256 CUs (one
// 128 KiB-LDS workgroup per CU): as many splits as fit one pass over the CUs,
// each at least kMinSplitSteps K steps of the mean segment N / E, at most
// kMaxSplits.  A pure function of the sizes, so the workspace query and the
// launch agree.
constexpr int kMinSplitSteps = 8;
constexpr int kMaxSplits = 32;

int wg_splits(const WgTask& t0, const WgTask& t1, int B, int E, int N) {
  const int64_t per = (int64_t)t0.y_tiles * t0.x_tiles + (int64_t)t1.y_tiles * t1.x_tiles;
  const int64_t blocks = per * E * B;
  if (blocks == 0 || 2 * blocks > kCUs) return 1;
  const int64_t mean_steps = ((int64_t)N / E + kBK - 1) / kBK;
  const int64_t s = std::min<int64_t>({kCUs / blocks, mean_steps / kMinSplitSteps, kMaxSplits});
  return (int)std::max<int64_t>(1, s);
}

// fp32 partials of both tasks, the second at a 256-byte boundary
size_t wg_part_bytes(const WgTask& t0, const WgTask& t1, int B, int E, int splits,
                     size_t* off1) {
  const size_t be = (size_t)B * E;
  *off1 = ((size_t)splits * be * t0.X * t0.Y * sizeof(float) + 255) & ~(size_t)255;
  return splits > 1 ? *off1 + (size_t)splits * be * t1.X * t1.Y * sizeof(float) : 0;
}

// splits = 1: one pass, bf16 stores, no workspace
int launch_wg(WgTask t0, WgTask t1, const int32_t* gs, int B, int E, int N, int splits,
              void* workspace, size_t workspace_bytes, hipStream_t st, const char* what,
              const WgLayers* ly = nullptr) {
  const int64_t per = (int64_t)t0.y_tiles * t0.x_tiles + (int64_t)t1.y_tiles * t1.x_tiles;
  const int64_t blocks = per * E * B * splits;
  if (blocks == 0) return UTTT_OK;
  if (int rc = check_grid(blocks, what)) return rc;
  UTTT_REQUIRE(t0.X < (1 << 23) && t0.Y < (1 << 23) && t1.X < (1 << 23) && t1.Y < (1 << 23),
               "%s: operand rows of 2^23 or more elements are not supported", what);
  if (splits > 1) {
    size_t off1;
    const size_t need = wg_part_bytes(t0, t1, B, E, splits, &off1);
    UTTT_REQUIRE(workspace && workspace_bytes >= need && aligned16(workspace),
                 "%s: workspace of %zu bytes needed (got %zu)", what, need, workspace_bytes);
    t0.part = static_cast<float*>(workspace);
    t1.part = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + off1);
  }
  // the plain epilogue stores 16 bytes at a time
  UTTT_REQUIRE(splits > 1 || (aligned16(t0.out) && (t1.y_tiles * t1.x_tiles == 0 || aligned16(t1.out))),
               "%s: outputs must be 16-byte aligned", what);
  const bool eight = pick_na(kDefaultWgNA) == 1;
  if (ly != nullptr) {  // the layered operands (four waves)
    if (splits == 1)
      hipLaunchKernelGGL((wg_kernel<false, 2, true>), dim3((unsigned)blocks),
                         dim3(kThreadsOf<2>), 0, st, t0, t1, gs, E, N, B * E, 1, *ly);
    else
      hipLaunchKernelGGL((wg_kernel<true, 2, true>), dim3((unsigned)blocks), dim3(kThreadsOf<2>),
                         0, st, t0, t1, gs, E, N, B * E, splits, *ly);
  } else if (splits == 1 && eight)
    hipLaunchKernelGGL((wg_kernel<false, 1>), dim3((unsigned)blocks), dim3(kThreadsOf<1>), 0, st,
                       t0, t1, gs, E, N, B * E, 1, WgLayers{});
  else if (splits == 1)
    hipLaunchKernelGGL((wg_kernel<false, 2>), dim3((unsigned)blocks), dim3(kThreadsOf<2>), 0, st,
                       t0, t1, gs, E, N, B * E, 1, WgLayers{});
  else if (eight)
    hipLaunchKernelGGL((wg_kernel<true, 1>), dim3((unsigned)blocks), dim3(kThreadsOf<1>), 0, st,
                       t0, t1, gs, E, N, B * E, splits, WgLayers{});
  else
    hipLaunchKernelGGL((wg_kernel<true, 2>), dim3((unsigned)blocks), dim3(kThreadsOf<2>), 0, st,
                       t0, t1, gs, E, N, B * E, splits, WgLayers{});
  if (int rc = check_launch(what)) return rc;
  if (splits == 1) return UTTT_OK;
  const int64_t n0 = (int64_t)B * E * t0.X * t0.Y, n1 = (int64_t)B * E * t1.X * t1.Y;
  const int64_t groups = (n0 + n1) / 8;
  const unsigned rblocks = (unsigned)std::min<int64_t>((groups + 255) / 256, 4096);
  hipLaunchKernelGGL(wg_reduce_kernel, dim3(rblocks), dim3(256), 0, st, t0, t1, n0, n1, splits);
  return check_launch(what);
}

size_t up256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace
}  // namespace uttt

using namespace uttt;

// ================================================================ C ABI ====
extern "C" int uttt_grouped_gate_up(const void* w0_w2, const void* x, const int32_t* group_sizes,
                                    int B, int E, int I, int D, int N, void* hidden,
                                    int token_major, void* stream) {
  UTTT_REQUIRE(B >= 0 && E >= 1 && I >= 0 && D >= 0 && N >= 0, "grouped_gate_up: bad sizes");
  UTTT_REQUIRE(I % 8 == 0 && D % 8 == 0, "grouped_gate_up: I=%d and D=%d must be multiples of 8", I, D);
  if (B == 0 || N == 0 || I == 0) return UTTT_OK;
  UTTT_REQUIRE(w0_w2 && x && group_sizes && hidden, "grouped_gate_up: null pointer");
  UTTT_REQUIRE(aligned16(w0_w2) && aligned16(x) && aligned16(hidden),
               "grouped_gate_up: tensors must be 16-byte aligned");
  if (token_major && use_apply_kernel(N, E)) {
    const ApArgs a = apply_args(w0_w2, x, D, (int64_t)2 * I * D, I, I, 2 * I, kTileRows, B, E, N,
                                group_sizes);
    const ApSwiGLU::Args ea{static_cast<uint16_t*>(hidden), I, N};
    return launch_apply<ApSwiGLU, true>(a, I, ea, as_stream(stream), "grouped_gate_up");
  }
  const TnArgs t = tn_args(w0_w2, w0_w2, x, D, D, (int64_t)2 * I * D, 0, I, I, 2 * I, kTileRows,
                           I, B, E, N, group_sizes);
  const EpiSwiGLU::Args ea{static_cast<uint16_t*>(hidden), I, N, token_major};
  return launch_tn<KMajor, EpiSwiGLU>(t, ea, B, as_stream(stream), "grouped_gate_up");
}

extern "C" int uttt_grouped_gate_up_gathers(long long N, int E) {
  return use_apply_kernel(N, E) ? 1 : 0;
}

extern "C" int uttt_grouped_gate_up_gather(const void* w0_w2, const void* x, int T,
                                           const int32_t* src_rows, long long src_sb,
                                           const int32_t* group_sizes, int B, int E, int I, int D,
                                           int N, void* hidden, void* stream) {
  UTTT_REQUIRE(B >= 0 && E >= 1 && I >= 0 && D >= 0 && N >= 0 && T >= 0 && src_sb >= N,
               "grouped_gate_up_gather: bad sizes");
  UTTT_REQUIRE(I % 8 == 0 && D % 8 == 0,
               "grouped_gate_up_gather: I=%d and D=%d must be multiples of 8", I, D);
  if (B == 0 || N == 0 || I == 0) return UTTT_OK;
  UTTT_REQUIRE(use_apply_kernel(N, E),
               "grouped_gate_up_gather: N=%d routed rows over E=%d experts take the general "
               "tiles, which read a permuted copy (uttt_grouped_gate_up)", N, E);
  // the gathered rows' 32-bit lane offsets: every row of x starts below 2^30 elements
  UTTT_REQUIRE(T >= 1 && (int64_t)T * D < ((int64_t)1 << 30),
               "grouped_gate_up_gather: T=%d rows of D=%d elements exceed 2^30", T, D);
  UTTT_REQUIRE(w0_w2 && x && src_rows && group_sizes && hidden,
               "grouped_gate_up_gather: null pointer");
  UTTT_REQUIRE(aligned16(w0_w2) && aligned16(x) && aligned16(hidden),
               "grouped_gate_up_gather: tensors must be 16-byte aligned");
  ApArgs a = apply_args(w0_w2, x, D, (int64_t)2 * I * D, I, I, 2 * I, kTileRows, B, E, N,
                        group_sizes);
  a.src = src_rows;
  a.src_sb = src_sb;
  a.T = T;
  const ApSwiGLU::Args ea{static_cast<uint16_t*>(hidden), I, N};
  return launch_apply<ApSwiGLU, true>(a, I, ea, as_stream(stream), "grouped_gate_up_gather");
}

extern "C" int uttt_grouped_gemm_nt(const void* w, const void* x, const int32_t* group_sizes,
                                    int B, int E, int M, int K, int N, void* y, void* stream) {
  UTTT_REQUIRE(B >= 0 && E >= 1 && M >= 0 && K >= 0 && N >= 0, "grouped_gemm_nt: bad sizes");
  UTTT_REQUIRE(M % 8 == 0 && K % 8 == 0, "grouped_gemm_nt: M=%d and K=%d must be multiples of 8", M, K);
  if (B == 0 || N == 0 || M == 0) return UTTT_OK;
  UTTT_REQUIRE(w && x && group_sizes && y, "grouped_gemm_nt: null pointer");
  UTTT_REQUIRE(aligned16(w) && aligned16(x) && aligned16(y),
               "grouped_gemm_nt: tensors must be 16-byte aligned");
  if (use_apply_kernel_nt(N, E, B, M)) {
    const ApStore::Args ea{static_cast<uint16_t*>(y), M, M, N};
    if (g_apply_down_two) {
      const ApArgs a = apply_args(w, x, K, (int64_t)M * K, kTileRows, M, M, 2 * kTileRows, B, E, N,
                                  group_sizes);
      return launch_apply<ApStore, true>(a, M, ea, as_stream(stream), "grouped_gemm_nt");
    }
    const ApArgs a = apply_args(w, x, K, (int64_t)M * K, kTileRows, M, M, kTileRows, B, E, N,
                                group_sizes);
    return launch_apply<ApStore, false>(a, M, ea, as_stream(stream), "grouped_gemm_nt");
  }
  return launch_wide<KMajor>(w, x, K, nullptr, nullptr, 0, M, K, (int64_t)M * K,
                             static_cast<uint16_t*>(y), B, E, N, group_sizes, as_stream(stream),
                             "grouped_gemm_nt");
}

extern "C" int uttt_grouped_gemm_tn(const void* w, const void* x, const int32_t* group_sizes,
                                    int B, int E, int M, int K, int N, void* y, void* stream) {
  UTTT_REQUIRE(B >= 0 && E >= 1 && M >= 0 && K >= 0 && N >= 0, "grouped_gemm_tn: bad sizes");
  UTTT_REQUIRE(M % 8 == 0 && K % 8 == 0, "grouped_gemm_tn: M=%d and K=%d must be multiples of 8", M, K);
  if (B == 0 || N == 0 || M == 0) return UTTT_OK;
  UTTT_REQUIRE(w && x && group_sizes && y, "grouped_gemm_tn: null pointer");
  UTTT_REQUIRE(aligned16(w) && aligned16(x) && aligned16(y),
               "grouped_gemm_tn: tensors must be 16-byte aligned");
  return launch_wide<RMajor>(w, x, K, nullptr, nullptr, 0, M, M, (int64_t)M * K,
                             static_cast<uint16_t*>(y), B, E, N, group_sizes, as_stream(stream),
                             "grouped_gemm_tn");
}

extern "C" int uttt_grouped_gemm_nt2(const void* wa, const void* xa, const void* wb,
                                     const void* xb, const int32_t* group_sizes, int B, int E,
                                     int M, int K, int N, void* y, void* stream) {
  UTTT_REQUIRE(B >= 0 && E >= 1 && M >= 0 && K >= 0 && N >= 0, "grouped_gemm_nt2: bad sizes");
  UTTT_REQUIRE(M % 8 == 0 && K % 8 == 0, "grouped_gemm_nt2: M=%d and K=%d must be multiples of 8", M, K);
  if (B == 0 || N == 0 || M == 0) return UTTT_OK;
  UTTT_REQUIRE(wa && xa && wb && xb && group_sizes && y, "grouped_gemm_nt2: null pointer");
  UTTT_REQUIRE(aligned16(wa) && aligned16(xa) && aligned16(wb) && aligned16(xb) && aligned16(y),
               "grouped_gemm_nt2: tensors must be 16-byte aligned");
  return launch_wide<KMajor>(wa, xa, K, wb, xb, K, M, K, (int64_t)M * K,
                             static_cast<uint16_t*>(y), B, E, N, group_sizes, as_stream(stream),
                             "grouped_gemm_nt2");
}

extern "C" int uttt_grouped_gemm_tn2(const void* wa, const void* xa, const void* wb,
                                     const void* xb, const int32_t* group_sizes, int B, int E,
                                     int M, int K, int N, void* y, void* stream) {
  UTTT_REQUIRE(B >= 0 && E >= 1 && M >= 0 && K >= 0 && N >= 0, "grouped_gemm_tn2: bad sizes");
  UTTT_REQUIRE(M % 8 == 0 && K % 8 == 0, "grouped_gemm_tn2: M=%d and K=%d must be multiples of 8", M, K);
  if (B == 0 || N == 0 || M == 0) return UTTT_OK;
  UTTT_REQUIRE(wa && xa && wb && xb && group_sizes && y, "grouped_gemm_tn2: null pointer");
  UTTT_REQUIRE(aligned16(wa) && aligned16(xa) && aligned16(wb) && aligned16(xb) && aligned16(y),
               "grouped_gemm_tn2: tensors must be 16-byte aligned");
  return launch_wide<RMajor>(wa, xa, K, wb, xb, K, M, M, (int64_t)M * K,
                             static_cast<uint16_t*>(y), B, E, N, group_sizes, as_stream(stream),
                             "grouped_gemm_tn2");
}

extern "C" int uttt_debug_set_apply_path(int path) {
  const int prev = g_apply_path;
  g_apply_path = path < 0 ? -1 : path > 0 ? 1 : 0;
  g_apply_down_two = path == 2;
  return prev;
}

extern "C" int uttt_debug_set_ns_path(int path) {
  UTTT_REQUIRE(path == 0 || path == 1, "debug_set_ns_path: path=%d (0 or 1)", path);
  const int prev = g_ns_path;
  g_ns_path = path;
  return prev;
}

extern "C" int uttt_debug_set_gemm_layout(int na) {
  UTTT_REQUIRE(na == 0 || na == 1 || na == 2, "debug_set_gemm_layout: na=%d (0, 1 or 2)", na);
  const int prev = g_gemm_na;
  g_gemm_na = na;
  return prev;
}

extern "C" long long uttt_debug_set_supertile_min_tiles(long long min_tiles) {
  const long long prev = (long long)g_xcd_map_min_tiles;
  g_xcd_map_min_tiles = min_tiles < 0 ? kXcdMapMinTiles : (int64_t)min_tiles;
  return prev;
}

extern "C" size_t uttt_update_stage1_workspace_bytes(int B, int I, int N) {
  if (B <= 0 || I <= 0 || N <= 0) return 0;
  return up256((size_t)B * N * I * sizeof(float));
}

extern "C" int uttt_grouped_update_stage1(const void* w0_w2, const void* w1, const void* k,
                                          const void* v, const void* lr0, const void* lr1,
                                          const void* lr2, int lr_dtype,
                                          const int32_t* group_sizes, int B, int E, int I, int D,
                                          int N, void* dy0_dy2, void* hidden, int token_major,
                                          void* y0_y2_save, void* dh_save, void* workspace,
                                          size_t workspace_bytes, void* stream) {
  UTTT_REQUIRE(B >= 0 && E >= 1 && I >= 0 && D >= 0 && N >= 0, "grouped_update_stage1: bad sizes");
  UTTT_REQUIRE(I % 8 == 0 && D % 8 == 0,
               "grouped_update_stage1: I=%d and D=%d must be multiples of 8", I, D);
  if (B == 0 || N == 0 || I == 0) return UTTT_OK;
  UTTT_REQUIRE(w0_w2 && w1 && k && v && group_sizes && dy0_dy2 && hidden && workspace,
               "grouped_update_stage1: null pointer");
  UTTT_REQUIRE((lr0 == nullptr) == (lr1 == nullptr) && (lr1 == nullptr) == (lr2 == nullptr),
               "grouped_update_stage1: pass all three lr vectors or none");
  UTTT_REQUIRE((y0_y2_save == nullptr) == (dh_save == nullptr),
               "grouped_update_stage1: pass both saved tensors or none");
  UTTT_REQUIRE(aligned16(w0_w2) && aligned16(w1) && aligned16(k) && aligned16(v) &&
                   aligned16(dy0_dy2) && aligned16(hidden) && aligned16(workspace) &&
                   (y0_y2_save == nullptr || (aligned16(y0_y2_save) && aligned16(dh_save))),
               "grouped_update_stage1: tensors must be 16-byte aligned");
  const size_t need = uttt_update_stage1_workspace_bytes(B, I, N);
  UTTT_REQUIRE(workspace_bytes >= need, "grouped_update_stage1: workspace %zu < %zu bytes",
               workspace_bytes, need);
  hipStream_t st = as_stream(stream);
  float* dh = static_cast<float*>(workspace);
  // DH = w1^T v (fp32, token-major [N, I]): the reference keeps DH in fp32
  if (int rc = launch_wide<RMajor>(w1, v, D, nullptr, nullptr, 0, I, I, (int64_t)D * I, dh, B, E,
                                   N, group_sizes, st, "grouped_update_stage1(DH)"))
    return rc;
  const TnArgs t = tn_args(w0_w2, w0_w2, k, D, D, (int64_t)2 * I * D, 0, I, I, 2 * I, kTileRows,
                           I, B, E, N, group_sizes);
  UTTT_DTYPE_SWITCH_LR(lr_dtype, LR, {
    using S = typename LR::S;
    const typename EpiS1<LR>::Args ea{dh,
                                      static_cast<const S*>(lr0),
                                      static_cast<const S*>(lr1),
                                      static_cast<const S*>(lr2),
                                      static_cast<uint16_t*>(dy0_dy2),
                                      static_cast<uint16_t*>(hidden),
                                      static_cast<uint16_t*>(y0_y2_save),
                                      static_cast<uint16_t*>(dh_save),
                                      I,
                                      N,
                                      token_major};
    return launch_tn<KMajor, EpiS1<LR>>(t, ea, B, st, "grouped_update_stage1");
  });
  return UTTT_OK;
}

extern "C" size_t uttt_grouped_wgrad_pair_workspace_bytes(int B, int E, int I, int D, int N) {
  if (B <= 0 || E <= 0 || I <= 0 || D <= 0 || N <= 0) return 0;
  const WgTask t0 = wg_task(nullptr, nullptr, nullptr, 2 * I, D);
  const WgTask t1 = wg_task(nullptr, nullptr, nullptr, D, I);
  size_t off1;
  return wg_part_bytes(t0, t1, B, E, wg_splits(t0, t1, B, E, N), &off1);
}

extern "C" int uttt_grouped_wgrad_pair(const void* dy0_dy2_tok, const void* k,
                                       const void* hidden_tok, const void* v,
                                       const int32_t* group_sizes, int B, int E, int I, int D,
                                       int N, void* dw0_w2, void* dw1, void* workspace,
                                       size_t workspace_bytes, void* stream) {
  UTTT_REQUIRE(B >= 0 && E >= 1 && I >= 0 && D >= 0 && N >= 0, "grouped_wgrad_pair: bad sizes");
  UTTT_REQUIRE(I % 8 == 0 && D % 8 == 0,
               "grouped_wgrad_pair: I=%d and D=%d must be multiples of 8", I, D);
  if (B == 0 || I == 0 || D == 0) return UTTT_OK;
  UTTT_REQUIRE(dy0_dy2_tok && k && hidden_tok && v && group_sizes && dw0_w2 && dw1,
               "grouped_wgrad_pair: null pointer");
  UTTT_REQUIRE(aligned16(dy0_dy2_tok) && aligned16(k) && aligned16(hidden_tok) && aligned16(v) &&
                   aligned16(dw0_w2) && aligned16(dw1),
               "grouped_wgrad_pair: tensors must be 16-byte aligned");
  // dW0_W2 [2I][D] = DY^T K;  dW1 [D][I] = V^T Hid
  const WgTask t0 = wg_task(k, dy0_dy2_tok, dw0_w2, 2 * I, D);
  const WgTask t1 = wg_task(hidden_tok, v, dw1, D, I);
  return launch_wg(t0, t1, group_sizes, B, E, N, wg_splits(t0, t1, B, E, N), workspace,
                   workspace_bytes, as_stream(stream), "grouped_wgrad_pair");
}

extern "C" size_t uttt_dense_wgrad_pair_layers_workspace_bytes(int L, int b, int H, int I,
                                                              int D) {
  if (L <= 1 || b <= 0 || H <= 0 || I <= 0 || D <= 0) return 0;
  const WgTask t0 = wg_task(nullptr, nullptr, nullptr, 2 * I, D);
  const WgTask t1 = wg_task(nullptr, nullptr, nullptr, D, I);
  size_t off1;
  return wg_part_bytes(t0, t1, b * H, 1, L, &off1);
}

extern "C" int uttt_dense_wgrad_pair_layers(const void* dy0_dy2_tok, const void* const* k_layers,
                                            const void* hidden_tok, const void* const* v_layers,
                                            int L, int b, int l, int H, int I, int D,
                                            void* dw0_w2, void* dw1, void* workspace,
                                            size_t workspace_bytes, void* stream) {
  UTTT_REQUIRE(L >= 0 && L <= kMaxLayers && b >= 0 && l >= 0 && H >= 1 && I >= 0 && D >= 0,
               "dense_wgrad_pair_layers: bad sizes (L=%d must be at most %d)", L, kMaxLayers);
  UTTT_REQUIRE(I % 8 == 0 && D % 8 == 0,
               "dense_wgrad_pair_layers: I=%d and D=%d must be multiples of 8", I, D);
  if (L == 0 || b == 0 || l == 0 || I == 0 || D == 0) return UTTT_OK;
  UTTT_REQUIRE(l % kBK == 0, "dense_wgrad_pair_layers: l=%d must be a multiple of %d", l, kBK);
  const int64_t N = (int64_t)L * l;
  UTTT_REQUIRE(N < ((int64_t)1 << 30) && (int64_t)H * D < (1 << 23),
               "dense_wgrad_pair_layers: sizes too large");
  UTTT_REQUIRE(dy0_dy2_tok && k_layers && hidden_tok && v_layers && dw0_w2 && dw1,
               "dense_wgrad_pair_layers: null pointer");
  UTTT_REQUIRE(aligned16(dy0_dy2_tok) && aligned16(hidden_tok) && aligned16(dw0_w2) &&
                   aligned16(dw1),
               "dense_wgrad_pair_layers: tensors must be 16-byte aligned");
  WgLayers ly{};
  ly.l = l;
  ly.H = H;
  ly.D = D;
  for (int i = 0; i < L; ++i) {
    UTTT_REQUIRE(k_layers[i] && v_layers[i] && aligned16(k_layers[i]) && aligned16(v_layers[i]),
                 "dense_wgrad_pair_layers: layer %d's k and v must be 16-byte aligned", i);
    ly.k.p[i] = k_layers[i];
    ly.v.p[i] = v_layers[i];
  }
  // dW0_W2 [2I][D] = DY^T K;  dW1 [D][I] = V^T Hid; one K run per layer
  const WgTask t0 = wg_task(nullptr, dy0_dy2_tok, dw0_w2, 2 * I, D);
  const WgTask t1 = wg_task(hidden_tok, nullptr, dw1, D, I);
  return launch_wg(t0, t1, nullptr, b * H, 1, (int)N, L, workspace, workspace_bytes,
                   as_stream(stream), "dense_wgrad_pair_layers", &ly);
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
  // [R][C] = A^T B: x = R (Q = A), y = C (P = B);  [C][R]: x = C (Q = B), y = R (P = A)
  const WgTask t0 = transposed ? wg_task(a_tok, b_tok, out, C, R) : wg_task(b_tok, a_tok, out, R, C);
  WgTask t1 = t0;
  t1.y_tiles = 0;
  t1.x_tiles = 0;
  return launch_wg(t0, t1, group_sizes, B, E, N, 1, nullptr, 0, as_stream(stream), "grouped_wgrad");
}

namespace uttt {
namespace {
struct UpdateBwdWs {
  size_t dhg, gy, dx, gx, gdh, hlr, part, total;
};
UpdateBwdWs update_bwd_ws(int B, int I, int N) {
  const size_t t2 = up256((size_t)B * N * 2 * I * 2), t1 = up256((size_t)B * N * I * 2);
  const int m_tiles = (I + kTileRows - 1) / kTileRows;
  UpdateBwdWs w;
  w.dhg = 0;
  w.gy = w.dhg + t2;
  w.dx = w.gy + t2;
  w.gx = w.dx + t2;
  w.gdh = w.gx + t2;
  w.hlr = w.gdh + t1;
  w.part = w.hlr + t1;
  w.total = w.part + up256((size_t)3 * m_tiles * B * N * 4);
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
    const void* grad_dw0_w2, const void* grad_dw1, const void* y0_y2_saved,
    const void* dh_saved, int B, int E, int I, int D, int N,
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
                   aligned16(workspace) &&
                   (y0_y2_saved == nullptr || (aligned16(y0_y2_saved) && aligned16(dh_saved))),
               "grouped_update_bwd: tensors must be 16-byte aligned");
  UTTT_REQUIRE((y0_y2_saved == nullptr) == (dh_saved == nullptr),
               "grouped_update_bwd: pass both saved tensors or none");
  const UpdateBwdWs ws = update_bwd_ws(B, I, N);
  UTTT_REQUIRE(workspace_bytes >= ws.total, "grouped_update_bwd: workspace %zu < %zu bytes",
               workspace_bytes, ws.total);
  uint8_t* wsb = static_cast<uint8_t*>(workspace);
  uint16_t* dhg = reinterpret_cast<uint16_t*>(wsb + ws.dhg);
  uint16_t* gy = reinterpret_cast<uint16_t*>(wsb + ws.gy);
  uint16_t* dx = reinterpret_cast<uint16_t*>(wsb + ws.dx);
  uint16_t* gx = reinterpret_cast<uint16_t*>(wsb + ws.gx);
  uint16_t* gdh = reinterpret_cast<uint16_t*>(wsb + ws.gdh);
  uint16_t* hlr = reinterpret_cast<uint16_t*>(wsb + ws.hlr);
  float* part = reinterpret_cast<float*>(wsb + ws.part);
  hipStream_t st = as_stream(stream);
  const int64_t g02 = (int64_t)2 * I * D, g1 = (int64_t)D * I;
  const int m_tiles = (I + kTileRows - 1) / kTileRows;

  if (y0_y2_saved != nullptr) {
    // from the forward's saved bf16 Y0 | Y2 and DH: GD = gw1^T v (bf16 [N, I]),
    // then GY0 | GY2 = gw0_w2 k with the second-order pass on the registers
    uint16_t* gd = dhg;
    if (int rc = launch_wide<RMajor>(grad_dw1, v, D, nullptr, nullptr, 0, I, I, g1, gd, B, E, N,
                                     group_sizes, st, "grouped_update_bwd(GD)"))
      return rc;
    const TnArgs t = tn_args(grad_dw0_w2, grad_dw0_w2, k, D, D, g02, 0, I, I, 2 * I, kTileRows, I,
                             B, E, N, group_sizes);
    UTTT_DTYPE_SWITCH_LR(lr_dtype, LR, {
      using S = typename LR::S;
      const typename EpiBwdSaved<LR>::Args ea{static_cast<const uint16_t*>(y0_y2_saved),
                                              static_cast<const uint16_t*>(dh_saved),
                                              gd,
                                              static_cast<const S*>(lr0),
                                              static_cast<const S*>(lr1),
                                              static_cast<const S*>(lr2),
                                              gdh,
                                              gx,
                                              dx,
                                              hlr,
                                              part,
                                              I,
                                              N,
                                              B,
                                              m_tiles};
      if (int rc = launch_tn<KMajor, EpiBwdSaved<LR>>(t, ea, B, st, "grouped_update_bwd(GY)"))
        return rc;
      hipLaunchKernelGGL((lr_grad_reduce_kernel<LR>), dim3((N + 255) / 256, B), dim3(256), 0, st,
                         part, group_sizes, B, E, N, m_tiles, static_cast<S*>(grad_lr0),
                         static_cast<S*>(grad_lr1), static_cast<S*>(grad_lr2));
      if (int rc = check_launch("grouped_update_bwd(lr grads)")) return rc;
    });
  } else {
  // 1. DHG = [w1^T v | gw1^T v]  (bf16 [N, 2I])
  {
    const TnArgs t = tn_args(w1, grad_dw1, v, D, I, g1, 0, 0, I, I, kTileRows, I, B, E, N,
                             group_sizes);
    const EpiStoreArgs<uint16_t> ea{dhg, 2 * I, {0, I}, {I, 2 * I}, N};
    if (int rc = aligned16(dhg)
                     ? launch_tn<RMajor, EpiStore<uint16_t, true>>(t, ea, B, st,
                                                                   "grouped_update_bwd(DH)")
                     : launch_tn<RMajor, EpiStore<uint16_t>>(t, ea, B, st, "grouped_update_bwd(DH)"))
      return rc;
  }
  // 2. GY = [gw0 k | gw2 k]  (bf16 [N, 2I])
  {
    const TnArgs t = tn_args(grad_dw0_w2, grad_dw0_w2, k, D, D, g02, 0, I, I, 2 * I, kTileRows, I,
                             B, E, N, group_sizes);
    const EpiStoreArgs<uint16_t> ea{gy, 2 * I, {0, I}, {I, 2 * I}, N};
    if (int rc = aligned16(gy)
                     ? launch_tn<KMajor, EpiStore<uint16_t, true>>(t, ea, B, st,
                                                                   "grouped_update_bwd(GY)")
                     : launch_tn<KMajor, EpiStore<uint16_t>>(t, ea, B, st, "grouped_update_bwd(GY)"))
      return rc;
  }
  // 3. Y0, Y2 = w0 k, w2 k with the second-order pointwise pass; 4. lr grads
  {
    const TnArgs t = tn_args(w0_w2, w0_w2, k, D, D, g02, 0, I, I, 2 * I, kTileRows, I, B, E, N,
                             group_sizes);
    UTTT_DTYPE_SWITCH_LR(lr_dtype, LR, {
      using S = typename LR::S;
      const typename EpiBwd<LR>::Args ea{gy,
                                         dhg,
                                         static_cast<const S*>(lr0),
                                         static_cast<const S*>(lr1),
                                         static_cast<const S*>(lr2),
                                         gdh,
                                         gx,
                                         dx,
                                         hlr,
                                         part,
                                         I,
                                         N,
                                         B,
                                         m_tiles};
      if (int rc = launch_tn<KMajor, EpiBwd<LR>>(t, ea, B, st, "grouped_update_bwd(pointwise)"))
        return rc;
      hipLaunchKernelGGL((lr_grad_reduce_kernel<LR>), dim3((N + 255) / 256, B), dim3(256), 0, st,
                         part, group_sizes, B, E, N, m_tiles, static_cast<S*>(grad_lr0),
                         static_cast<S*>(grad_lr1), static_cast<S*>(grad_lr2));
      if (int rc = check_launch("grouped_update_bwd(lr grads)")) return rc;
    });
  }
  }
  // 5. grad_K = GW0_W2^T dx0_x2 + W0_W2^T grad_x0_x2 (K = 2I, chained)
  if (int rc = launch_wide<RMajor>(grad_dw0_w2, dx, 2 * I, w0_w2, gx, 2 * I, D, D, g02,
                                   static_cast<uint16_t*>(grad_k), B, E, N, group_sizes, st,
                                   "grouped_update_bwd(grad_K)"))
    return rc;
  // 6. grad_V = W1 grad_dh + GW1 hidden_lr1 (K = I, chained)
  if (int rc = launch_wide<KMajor>(w1, gdh, I, grad_dw1, hlr, I, D, I, g1,
                                   static_cast<uint16_t*>(grad_v), B, E, N, group_sizes, st,
                                   "grouped_update_bwd(grad_V)"))
    return rc;
  // 7. grad_W0_W2 [2I][D] = grad_x0_x2^T K;  grad_W1 [D][I] = V^T grad_dh
  const WgTask t0 = wg_task(k, gx, grad_w0_w2, 2 * I, D);
  const WgTask t1 = wg_task(gdh, v, grad_w1, D, I);
  return launch_wg(t0, t1, group_sizes, B, E, N, 1, nullptr, 0, st, "grouped_update_bwd(weights)");
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

// ============================================================ Newton-Schulz ==
namespace {
struct NsWs {
  size_t gs, denom, part, x0, x1, a, ac, bm, total;
};
NsWs ns_ws(int BE, int m, int n) {
  NsWs w{};
  size_t o = 0;
  w.gs = o;
  o += up256((size_t)BE * 4);
  w.denom = o;
  o += up256((size_t)BE * 4);
  w.part = o;
  o += up256((size_t)BE * kNsParts * 4);
  w.x0 = o;
  o += up256((size_t)BE * m * n * 2);
  w.x1 = o;
  o += up256((size_t)BE * m * n * 2);
  w.a = o;
  o += up256((size_t)BE * m * m * 2);
  w.ac = o;
  o += up256((size_t)BE * m * m * 2);
  w.bm = o;
  o += up256((size_t)BE * m * m * 2);
  w.total = o;
  return w;
}
}  // namespace

extern "C" size_t uttt_newton_schulz5_workspace_bytes(int BE, int rows, int cols) {
  if (BE <= 0 || rows <= 0 || cols <= 0) return 0;
  const int m = rows < cols ? rows : cols, n = rows < cols ? cols : rows;
  return ns_ws(BE, m, n).total;
}

extern "C" int uttt_newton_schulz5(const void* g, int g_dtype, int BE, int rows, int cols,
                                   float out_scale, void* out, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  UTTT_REQUIRE(BE >= 0 && rows >= 0 && cols >= 0, "newton_schulz5: bad sizes");
  if (BE == 0 || rows == 0 || cols == 0) return UTTT_OK;
  UTTT_REQUIRE(rows % 8 == 0 && cols % 8 == 0,
               "newton_schulz5: rows=%d and cols=%d must be multiples of 8", rows, cols);
  UTTT_REQUIRE(g && out && workspace, "newton_schulz5: null pointer");
  UTTT_REQUIRE(aligned16(out) && aligned16(workspace), "newton_schulz5: tensors must be 16-byte aligned");
  UTTT_REQUIRE(g_dtype == UTTT_F32 || g_dtype == UTTT_BF16,
               "newton_schulz5: the update must be fp32 or bf16 (code %d)", g_dtype);
  const bool trans = rows > cols;
  const int m = trans ? cols : rows, n = trans ? rows : cols;
  const NsWs w = ns_ws(BE, m, n);
  UTTT_REQUIRE(workspace_bytes >= w.total, "newton_schulz5: workspace %zu < %zu bytes",
               workspace_bytes, w.total);
  hipStream_t st = as_stream(stream);
  if (g_ns_path == 0 && aligned16(g) && ns_small_fits(rows, cols))
    return launch_ns_small(g, g_dtype, BE, rows, cols, out_scale, static_cast<uint16_t*>(out),
                           st);
  uint8_t* wb = static_cast<uint8_t*>(workspace);
  int32_t* gs = reinterpret_cast<int32_t*>(wb + w.gs);
  float* denom = reinterpret_cast<float*>(wb + w.denom);
  float* part = reinterpret_cast<float*>(wb + w.part);
  uint16_t* X = reinterpret_cast<uint16_t*>(wb + w.x0);
  uint16_t* Xn = reinterpret_cast<uint16_t*>(wb + w.x1);
  uint16_t* A = reinterpret_cast<uint16_t*>(wb + w.a);
  uint16_t* Ac = reinterpret_cast<uint16_t*>(wb + w.ac);
  uint16_t* Bm = reinterpret_cast<uint16_t*>(wb + w.bm);
  const int64_t elems = (int64_t)m * n;
  // 1. norm
  UTTT_DTYPE_SWITCH_LR(g_dtype, TT, {
    hipLaunchKernelGGL((ns_sumsq_kernel<TT>), dim3(kNsParts, BE), dim3(256), 0, st,
                       static_cast<const typename TT::S*>(g), elems, part);
  });
  if (int rc = check_launch("newton_schulz5(norm)")) return rc;
  hipLaunchKernelGGL(ns_norm_kernel, dim3((BE + 255) / 256), dim3(256), 0, st, part, BE, m, denom, gs);
  if (int rc = check_launch("newton_schulz5(norm)")) return rc;
  // 2. X = bf16(bf16(G') / denom), G' = G^T when rows > cols
  {
    const int rt = (m + 63) / 64, ct = (n + 63) / 64;
    const int64_t blocks = (int64_t)rt * ct * BE;
    if (int rc = check_grid(blocks, "newton_schulz5(prep)")) return rc;
    UTTT_DTYPE_SWITCH_LR(g_dtype, TT, {
      using S = typename TT::S;
      if (trans)
        hipLaunchKernelGGL((ns_tile_kernel<TT, true, true>), dim3((unsigned)blocks), dim3(256), 0,
                           st, static_cast<const S*>(g), rows, cols, denom, 1.0f, X, rt, ct);
      else
        hipLaunchKernelGGL((ns_tile_kernel<TT, false, true>), dim3((unsigned)blocks), dim3(256),
                           0, st, static_cast<const S*>(g), rows, cols, denom, 1.0f, X, rt, ct);
    });
    if (int rc = check_launch("newton_schulz5(prep)")) return rc;
  }
  // 3. five steps (the reference's coefficient table)
  static const float kCoef[5][3] = {{4.0848f, -6.8946f, 2.9270f},
                                    {3.9505f, -6.3029f, 2.6377f},
                                    {3.7418f, -5.5913f, 2.3037f},
                                    {2.8769f, -3.1427f, 1.2046f},
                                    {2.8366f, -3.0525f, 1.2012f}};
  for (int it = 0; it < 5; ++it) {
    const float ca = kCoef[it][0], cb = kCoef[it][1], cc = kCoef[it][2];
    // A = X X^T and Ac = c A  ([m, m]: x = X as m rows of K = n, A operand = X).
    // A is symmetric bit for bit (element (i, j) and (j, i) take the same
    // products in the same k order): only the 256-tiles on or below the
    // diagonal are multiplied and those below it also store their transposes
    // (EpiLinComb), which takes 15 of the 36 tiles of a 1536-wide matrix off
    // the matrix cores
    if (int rc = launch_lincomb<KMajor>(X, X, n, m, n, elems, nullptr, 0.0f, 1.0f, A, Ac, cc, BE, m,
                                        gs, st, "newton_schulz5(X X^T)", true))
      return rc;
    // B = b A + (c A) A  (x = Ac, A operand = A: A is symmetric, so row j of A
    // is column j).  The full product: (c A) A is symmetric in exact
    // arithmetic only, since element (i, j) sums bf16(c A[i, k]) A[k, j] and
    // element (j, i) sums A[i, k] bf16(c A[k, j]), so mirroring one triangle
    // would round half of B differently from the reference's product
    if (int rc = launch_lincomb<KMajor>(A, Ac, m, m, m, (int64_t)m * m, A, cb, 1.0f, Bm, nullptr,
                                        0.0f, BE, m, gs, st, "newton_schulz5(B)", false))
      return rc;
    // X' = a X + B X  ([m, n]: x = B, A operand = X read row-major: A(j, k) = X[k, j])
    if (int rc = launch_lincomb<RMajor>(X, Bm, m, n, n, elems, X, ca, 1.0f, Xn, nullptr, 0.0f, BE,
                                        m, gs, st, "newton_schulz5(B X)"))
      return rc;
    uint16_t* tmp = X;
    X = Xn;
    Xn = tmp;
  }
  // 4. out = bf16(X * scale) in G's orientation
  {
    const int Rd = rows, Cd = cols;
    const int rt = (Rd + 63) / 64, ct = (Cd + 63) / 64;
    const int64_t blocks = (int64_t)rt * ct * BE;
    if (int rc = check_grid(blocks, "newton_schulz5(out)")) return rc;
    if (trans)
      hipLaunchKernelGGL((ns_tile_kernel<BF16T, true, false>), dim3((unsigned)blocks), dim3(256), 0,
                         st, X, m, n, nullptr, out_scale, static_cast<uint16_t*>(out), rt, ct);
    else
      hipLaunchKernelGGL((ns_tile_kernel<BF16T, false, false>), dim3((unsigned)blocks), dim3(256),
                         0, st, X, m, n, nullptr, out_scale, static_cast<uint16_t*>(out), rt, ct);
    if (int rc = check_launch("newton_schulz5(out)")) return rc;
  }
  return UTTT_OK;
}
