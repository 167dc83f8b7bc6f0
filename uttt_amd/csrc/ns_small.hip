// Newton-Schulz orthogonalisation of small matrices in one launch.
// Reference: zeropower_via_newtonschulz5,
// uttt_llm/flame/custom_models/uttt_moe/ttt_operation.py:19-46, as applied to
// the d x d slices of the uTTT-Dense write (uttt_dense/modeling_recurrent_lact.py:1192-1209).
//
// uttt_newton_schulz5 runs a matrix through 20 launches (norm, prep, five
// steps of three GEMMs, output).  A d x d slice (d = 96 or 192) gives each of
// those GEMMs one 256 x 256 tile, so the call costs 20 launch latencies for a
// few microseconds of matrix-core work per matrix.  Here one workgroup of 4
// waves (one per SIMD, so the accumulators can take the second register
// file) takes one matrix through the whole computation with X [m, n] and the
// m x m products in LDS (bf16, rows padded by 8 elements):
//   1. the matrix is loaded once and kept as bf16(G) in LDS; its squared
//      Frobenius norm is summed exactly as the multi-launch path sums it (64
//      contiguous parts, each by 256 threads with strided fused multiply-adds
//      and the same halving tree, then the parts in order), so the
//      denominator bf16(bf16(sqrt(s)) + 1e-7) is the same value;
//   2. X = bf16(bf16(G') / denom), G' = G^T when G has more rows than columns;
//   3. five steps of A = X X^T, B = b A + (c A) A, X = a X + B X, with the
//      multi-launch path's rounding points: A = bf16(acc), c A rounded to bf16
//      as it is read, B = bf16(bf16(b A) + bf16(acc)), X = bf16(bf16(a X) +
//      bf16(acc));
//   4. out = bf16(X * scale) in G's orientation.
// Every product element is one chain of v_mfma_f32_32x32x16_bf16 over K in
// increasing 16-wide steps, with the row operand in the source-A slot and the
// token operand in source B, as the grouped GEMM kernels compute it; so the
// result is the multi-launch path's bit for bit (a test compares the two).
// A product's output goes to LDS only after every wave has finished reading
// the buffer it overwrites (the values wait in registers across a barrier).
#include "common.h"

namespace uttt {
namespace {

typedef __bf16 nsb_bf16x8 __attribute__((ext_vector_type(8)));
typedef float nsb_f32x16 __attribute__((ext_vector_type(16)));

constexpr int kNsbWaves = 4;
constexpr int kNsbThreads = 64 * kNsbWaves;
constexpr int kNsbPad = 8;             // bf16 elements past the end of every LDS row
constexpr int kNsbBuf = 192 * (192 + kNsbPad);  // elements of one LDS buffer (76800 bytes)
constexpr int kNsbParts = 64;          // the norm's partial sums (as the multi-launch path)
constexpr int kNsbPartThreads = 256;   // threads per partial sum (as the multi-launch path)

__device__ __forceinline__ float nsb_round(float x) { return bf16_to_f32(f32_to_bf16(x)); }

// The reference's coefficient table, step `it` (a selection on the step
// index rather than a private array, which a runtime index would place in
// scratch memory).
__device__ __forceinline__ void nsb_coef(int it, float& a, float& b, float& c) {
  a = it == 0 ? 4.0848f : it == 1 ? 3.9505f : it == 2 ? 3.7418f : it == 3 ? 2.8769f : 2.8366f;
  b = it == 0 ? -6.8946f : it == 1 ? -6.3029f : it == 2 ? -5.5913f : it == 3 ? -3.1427f : -3.0525f;
  c = it == 0 ? 2.9270f : it == 1 ? 2.6377f : it == 2 ? 2.3037f : it == 3 ? 1.2046f : 1.2012f;
}

__device__ __forceinline__ nsb_bf16x8 nsb_row8(const uint16_t* p) {
  return *reinterpret_cast<const nsb_bf16x8*>(p);
}

// The blocks of one product that this wave owns: the product has RB row
// blocks and TB token blocks of 32; wave w = (w & 1, w >> 1) of the 2 x 2 wave
// grid owns row blocks r0 .. r0 + hr - 1 and token blocks t0 .. t0 + ht - 1
// (hr = ceil(RB / 2), ht = ceil(TB / 2), each at most kNsbHalf), those below
// RB and TB.
constexpr int kNsbHalf = 3;
struct NsbOwn {
  int r0, t0, hr, ht, RB, TB;
  __device__ __forceinline__ NsbOwn(int rb, int tb) : RB(rb), TB(tb) {
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    hr = (rb + 1) >> 1;
    ht = (tb + 1) >> 1;
    r0 = (w & 1) * hr;
    t0 = (w >> 1) * ht;
  }
  __device__ __forceinline__ bool row(int i) const { return i < hr && r0 + i < RB; }
  __device__ __forceinline__ bool tok(int j) const { return j < ht && t0 + j < TB; }
};

// acc[i][j] = sum over k < K of A(row, k) * B(token, k) for the wave's row
// block r0 + i and token block t0 + j, one MFMA chain per block over K in
// 16-wide steps.  Per step the wave reads its row fragments fa(row0, k0) and
// token fragments fb(token0, k0) once (8 consecutive k of the lane's row:
// k0 + 8 (lane / 32) ..), the next step's reads issued before this step's
// MFMAs; xb(fragment) is applied to a token fragment where it is used.  The
// loop has no branch: a block index past the product's edge reads the last
// block instead, and its result is never stored (a branch per block kept the
// compiler copying every accumulator out of the MFMA registers at each step).
template <class FA, class FB, class XB>
__device__ __forceinline__ void nsb_product(nsb_f32x16 (&acc)[kNsbHalf][kNsbHalf], const NsbOwn& o,
                                            int K, FA&& fa, FB&& fb, XB&& xb) {
  int ra[kNsbHalf], tb[kNsbHalf];
#pragma unroll
  for (int i = 0; i < kNsbHalf; ++i) {
    ra[i] = 32 * min(o.r0 + i, o.RB - 1);
    tb[i] = 32 * min(o.t0 + i, o.TB - 1);
  }
#pragma unroll
  for (int i = 0; i < kNsbHalf; ++i)
#pragma unroll
    for (int j = 0; j < kNsbHalf; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
  nsb_bf16x8 a[kNsbHalf], b[kNsbHalf];
#pragma unroll
  for (int i = 0; i < kNsbHalf; ++i) a[i] = fa(ra[i], 0);
#pragma unroll
  for (int j = 0; j < kNsbHalf; ++j) b[j] = fb(tb[j], 0);
  for (int k0 = 0; k0 < K; k0 += 16) {
    const int kn = min(k0 + 16, K - 16);  // the last step re-reads itself
    nsb_bf16x8 an[kNsbHalf], bn[kNsbHalf];
#pragma unroll
    for (int i = 0; i < kNsbHalf; ++i) an[i] = fa(ra[i], kn);
#pragma unroll
    for (int j = 0; j < kNsbHalf; ++j) bn[j] = fb(tb[j], kn);
#pragma unroll
    for (int j = 0; j < kNsbHalf; ++j) {
      const nsb_bf16x8 bj = xb(b[j]);
#pragma unroll
      for (int i = 0; i < kNsbHalf; ++i)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], bj, acc[i][j], 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < kNsbHalf; ++i) {
      a[i] = an[i];
      b[i] = bn[i];
    }
  }
}

// Element v of a lane's accumulator: row 8 (v / 4) + 4 (lane / 32) + v % 4 of
// the block, token lane % 32.
__device__ __forceinline__ int nsb_acc_row(int v) {
  return 8 * (v >> 2) + 4 * ((threadIdx.x & 63) >> 5) + (v & 3);
}

template <class TT>
__global__ __launch_bounds__(kNsbThreads) void ns_small_kernel(const typename TT::S* __restrict__ g,
                                                               int rows, int cols, float scale,
                                                               uint16_t* __restrict__ out) {
  using S = typename TT::S;
  __shared__ __attribute__((aligned(16))) uint16_t xs[kNsbBuf];
  __shared__ __attribute__((aligned(16))) uint16_t as[kNsbBuf];
  __shared__ float denom_s;
  const int tid = threadIdx.x, lane = tid & 63;
  const bool trans = rows > cols;
  const int m = trans ? cols : rows, n = trans ? rows : cols;
  const int ldx = n + kNsbPad, lda = m + kNsbPad;
  const int elems = rows * cols;
  const S* gb = g + (int64_t)blockIdx.x * elems;

  // 1. bf16(G) into `as` in G's own layout, 16-byte loads all in flight per batch
  {
    constexpr int kPer = 16 / (int)sizeof(S);  // elements per load
    const int nchunk = elems / kPer;
    for (int c0 = 0; c0 < nchunk; c0 += 4 * kNsbThreads) {
      uint4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int c = min(c0 + u * kNsbThreads + tid, nchunk - 1);
        v[u] = reinterpret_cast<const uint4*>(gb)[c];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int c = c0 + u * kNsbThreads + tid;
        if (c >= nchunk) continue;
        if constexpr (sizeof(S) == 4) {
          const float f[4] = {__uint_as_float(v[u].x), __uint_as_float(v[u].y),
                              __uint_as_float(v[u].z), __uint_as_float(v[u].w)};
          uint2 o;
          o.x = pack_bf16x2(f[0], f[1]);
          o.y = pack_bf16x2(f[2], f[3]);
          *reinterpret_cast<uint2*>(as + 4 * c) = o;
        } else {
          *reinterpret_cast<uint4*>(as + 8 * c) = v[u];
        }
      }
    }
  }
  __syncthreads();
  // the norm: part p of 64 covers elements [p per, (p + 1) per), thread t of
  // 256 adds elements t, t + 256, ... of it (at most 3: per <= 576); the 64
  // partial sums of a thread stay in registers, the halving tree's two
  // cross-wave levels go through LDS and its levels 32 .. 1 are shuffles in
  // wave 0 (lane t adds lane t + w, the same pairs as the tree in LDS)
  {
    static_assert(kNsbThreads == kNsbPartThreads, "one thread per partial-sum thread");
    const int per = (elems + kNsbParts - 1) / kNsbParts;
    float part[kNsbParts];
#pragma unroll
    for (int p = 0; p < kNsbParts; ++p) {
      const int lo = p * per, hi = min(lo + per, elems);
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        const int i = lo + tid + kNsbPartThreads * j;
        const float x = bf16_to_f32(as[min(i, elems - 1)]);
        acc = i < hi ? __builtin_fmaf(x, x, acc) : acc;
      }
      part[p] = acc;
    }
    float* red = reinterpret_cast<float*>(xs);  // [64][128]
    if (tid >= 128) {
#pragma unroll
      for (int p = 0; p < kNsbParts; ++p) red[p * 128 + tid - 128] = part[p];
    }
    __syncthreads();
    if (tid < 128) {
#pragma unroll
      for (int p = 0; p < kNsbParts; ++p) part[p] += red[p * 128 + tid];
    }
    __syncthreads();
    if (tid >= 64 && tid < 128) {
#pragma unroll
      for (int p = 0; p < kNsbParts; ++p) red[p * 64 + tid - 64] = part[p];
    }
    __syncthreads();
    if (tid < 64) {  // wave 0
#pragma unroll
      for (int p = 0; p < kNsbParts; ++p) {
        float v = part[p] + red[p * 64 + tid];
#pragma unroll
        for (int w = 32; w >= 1; w >>= 1) v += __shfl_down(v, w, 64);
        part[p] = v;
      }
      if (tid == 0) {
        float s = 0.0f;
#pragma unroll
        for (int p = 0; p < kNsbParts; ++p) s += part[p];
        denom_s = nsb_round(nsb_round(sqrtf(s)) + 1e-7f);
      }
    }
    __syncthreads();
  }
  // 2. X = bf16(bf16(G') / denom) into xs ([m][ldx]), 8 columns per item
  {
    const float dv = denom_s;
    const int n8 = n / 8;
    for (int e = tid; e < m * n8; e += kNsbThreads) {
      const int r = e / n8, c = 8 * (e - r * n8);
      float x[8];
      if (trans) {
#pragma unroll
        for (int u = 0; u < 8; ++u) x[u] = bf16_to_f32(as[(c + u) * cols + r]);
      } else {
        const uint4 v = *reinterpret_cast<const uint4*>(as + r * cols + c);
        const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          x[2 * u] = bf16_to_f32((uint16_t)(wv[u] & 0xffff));
          x[2 * u + 1] = bf16_to_f32((uint16_t)(wv[u] >> 16));
        }
      }
      uint4 o;
      o.x = pack_bf16x2(nsb_round(x[0] / dv), nsb_round(x[1] / dv));
      o.y = pack_bf16x2(nsb_round(x[2] / dv), nsb_round(x[3] / dv));
      o.z = pack_bf16x2(nsb_round(x[4] / dv), nsb_round(x[5] / dv));
      o.w = pack_bf16x2(nsb_round(x[6] / dv), nsb_round(x[7] / dv));
      *reinterpret_cast<uint4*>(xs + r * ldx + c) = o;
    }
  }
  __syncthreads();

  // 3. five steps
  const int mb = m / 32, nbk = n / 32;
  const int kl = 8 * (lane >> 5), rl = lane & 31;
  const NsbOwn own_mm(mb, mb), own_x(nbk, mb);
  nsb_f32x16 acc[kNsbHalf][kNsbHalf];
  uint32_t keep[kNsbHalf][kNsbHalf][8];  // a product's bf16 results held across the barrier
  // acc element 4 v4 + u of block (i, j): row 32 (r0 + i) + nsb_acc_row(4 v4) + u,
  // token 32 (t0 + j) + lane % 32
  auto unpack4 = [](uint2 p, float (&f)[4]) __attribute__((always_inline)) {
    f[0] = bf16_to_f32((uint16_t)(p.x & 0xffff));
    f[1] = bf16_to_f32((uint16_t)(p.x >> 16));
    f[2] = bf16_to_f32((uint16_t)(p.y & 0xffff));
    f[3] = bf16_to_f32((uint16_t)(p.y >> 16));
  };
  for (int it = 0; it < 5; ++it) {
    float ca, cb, cc;
    nsb_coef(it, ca, cb, cc);
    // A[t][r] = bf16(sum_k X[r][k] X[t][k])  (K = n); nothing reads `as`
    // during this product, so it is written directly
    auto xrow = [&](int r0, int k0) __attribute__((always_inline)) {
      return nsb_row8(xs + (r0 + rl) * ldx + k0 + kl);
    };
    auto same = [](nsb_bf16x8 f) __attribute__((always_inline)) { return f; };
    nsb_product(acc, own_mm, n, xrow, xrow, same);
#pragma unroll
    for (int i = 0; i < kNsbHalf; ++i)
#pragma unroll
      for (int j = 0; j < kNsbHalf; ++j) {
        if (!own_mm.row(i) || !own_mm.tok(j)) continue;
        const int r0 = 32 * (own_mm.r0 + i), t = 32 * (own_mm.t0 + j) + rl;
#pragma unroll
        for (int v4 = 0; v4 < 4; ++v4) {
          uint2 o;
          o.x = pack_bf16x2(acc[i][j][4 * v4], acc[i][j][4 * v4 + 1]);
          o.y = pack_bf16x2(acc[i][j][4 * v4 + 2], acc[i][j][4 * v4 + 3]);
          *reinterpret_cast<uint2*>(as + t * lda + r0 + nsb_acc_row(4 * v4)) = o;
        }
      }
    __syncthreads();
    // B[t][r] = bf16(bf16(b A[t][r]) + bf16(sum_k A[r][k] bf16(c A[t][k])))  (K = m)
    auto arow = [&](int r0, int k0) __attribute__((always_inline)) {
      return nsb_row8(as + (r0 + rl) * lda + k0 + kl);
    };
    auto times_c = [&](nsb_bf16x8 a) __attribute__((always_inline)) {
      nsb_bf16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = static_cast<__bf16>(cc * static_cast<float>(a[e]));
      return o;
    };
    nsb_product(acc, own_mm, m, arow, arow, times_c);
#pragma unroll
    for (int i = 0; i < kNsbHalf; ++i)
#pragma unroll
      for (int j = 0; j < kNsbHalf; ++j) {
        if (!own_mm.row(i) || !own_mm.tok(j)) continue;
        const int r0 = 32 * (own_mm.r0 + i), t = 32 * (own_mm.t0 + j) + rl;
#pragma unroll
        for (int v4 = 0; v4 < 4; ++v4) {
          float a4[4], o[4];
          unpack4(*reinterpret_cast<const uint2*>(as + t * lda + r0 + nsb_acc_row(4 * v4)), a4);
#pragma unroll
          for (int u = 0; u < 4; ++u)
            o[u] = nsb_round(nsb_round(cb * a4[u]) + nsb_round(acc[i][j][4 * v4 + u]));
          keep[i][j][2 * v4] = pack_bf16x2(o[0], o[1]);
          keep[i][j][2 * v4 + 1] = pack_bf16x2(o[2], o[3]);
        }
      }
    __syncthreads();  // every wave is done reading A
#pragma unroll
    for (int i = 0; i < kNsbHalf; ++i)
#pragma unroll
      for (int j = 0; j < kNsbHalf; ++j) {
        if (!own_mm.row(i) || !own_mm.tok(j)) continue;
        const int r0 = 32 * (own_mm.r0 + i), t = 32 * (own_mm.t0 + j) + rl;
#pragma unroll
        for (int v4 = 0; v4 < 4; ++v4)
          *reinterpret_cast<uint2*>(as + t * lda + r0 + nsb_acc_row(4 * v4)) =
              make_uint2(keep[i][j][2 * v4], keep[i][j][2 * v4 + 1]);
      }
    __syncthreads();
    // X'[t][j] = bf16(bf16(a X[t][j]) + bf16(sum_k X[k][j] B[t][k]))  (K = m).
    // The row operand is a column of X, read with two transposing LDS reads:
    // in each group of 16 lanes, lane 4 kk + q reads 4 columns (4 q .. +3 of
    // the group's 16) of k-row kk of a 4-row block, and lane i receives
    // column i of that block, i.e. 4 consecutive k of its own column; the
    // second read takes the next 4 k-rows.
    const int grp = lane >> 4, gs = lane & 15;
    const int tr_k = 8 * (grp >> 1) + (gs >> 2), tr_j = 16 * (grp & 1) + 4 * (gs & 3);
    auto xcol = [&](int j0, int k0) __attribute__((always_inline)) {
      typedef short nsb_i16x4 __attribute__((ext_vector_type(4)));
      typedef __attribute__((address_space(3))) nsb_i16x4 lds_i16x4;
      const uint16_t* p = xs + (k0 + tr_k) * ldx + j0 + tr_j;
      const nsb_i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
      const nsb_i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p + 4 * ldx));
      return __builtin_bit_cast(nsb_bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    };
    auto brow = [&](int t0, int k0) __attribute__((always_inline)) {
      return nsb_row8(as + (t0 + rl) * lda + k0 + kl);
    };
    nsb_product(acc, own_x, m, xcol, brow, same);
#pragma unroll
    for (int i = 0; i < kNsbHalf; ++i)
#pragma unroll
      for (int j = 0; j < kNsbHalf; ++j) {
        if (!own_x.row(i) || !own_x.tok(j)) continue;
        const int j0 = 32 * (own_x.r0 + i), t = 32 * (own_x.t0 + j) + rl;
#pragma unroll
        for (int v4 = 0; v4 < 4; ++v4) {
          float x4[4], o[4];
          unpack4(*reinterpret_cast<const uint2*>(xs + t * ldx + j0 + nsb_acc_row(4 * v4)), x4);
#pragma unroll
          for (int u = 0; u < 4; ++u)
            o[u] = nsb_round(nsb_round(ca * x4[u]) + nsb_round(acc[i][j][4 * v4 + u]));
          keep[i][j][2 * v4] = pack_bf16x2(o[0], o[1]);
          keep[i][j][2 * v4 + 1] = pack_bf16x2(o[2], o[3]);
        }
      }
    __syncthreads();  // every wave is done reading X
#pragma unroll
    for (int i = 0; i < kNsbHalf; ++i)
#pragma unroll
      for (int j = 0; j < kNsbHalf; ++j) {
        if (!own_x.row(i) || !own_x.tok(j)) continue;
        const int j0 = 32 * (own_x.r0 + i), t = 32 * (own_x.t0 + j) + rl;
#pragma unroll
        for (int v4 = 0; v4 < 4; ++v4)
          *reinterpret_cast<uint2*>(xs + t * ldx + j0 + nsb_acc_row(4 * v4)) =
              make_uint2(keep[i][j][2 * v4], keep[i][j][2 * v4 + 1]);
      }
    __syncthreads();
  }

  // 4. out = bf16(X * scale) in G's orientation, 8 output columns per item
  uint16_t* ob = out + (int64_t)blockIdx.x * elems;
  for (int i = tid; i < elems / 8; i += kNsbThreads) {
    const int r = (8 * i) / cols, c = 8 * i - r * cols;
    uint16_t x[8];
    if (trans) {
#pragma unroll
      for (int u = 0; u < 8; ++u) x[u] = xs[(c + u) * ldx + r];
    } else {
      const uint4 q = *reinterpret_cast<const uint4*>(xs + r * ldx + c);
      const uint32_t wq[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        x[2 * u] = (uint16_t)(wq[u] & 0xffff);
        x[2 * u + 1] = (uint16_t)(wq[u] >> 16);
      }
    }
    // (one rounding: packing rounds x * scale to bf16 as the multi-launch
    // path's bf16(bf16(x * scale)) does)
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = bf16_to_f32(x[u]) * scale;
    uint4 o;
    o.x = pack_bf16x2(v[0], v[1]);
    o.y = pack_bf16x2(v[2], v[3]);
    o.z = pack_bf16x2(v[4], v[5]);
    o.w = pack_bf16x2(v[6], v[7]);
    *reinterpret_cast<uint4*>(ob + 8 * i) = o;
  }
}

}  // namespace

// Whether a [rows, cols] matrix takes the one-launch path: both sides
// multiples of 32 and at most 192 (every product then has at most 6 x 6
// blocks: 3 x 3 per wave, and X and the m x m products fit one LDS buffer
// each).
bool ns_small_fits(int rows, int cols) {
  const int m = rows < cols ? rows : cols, n = rows < cols ? cols : rows;
  return m >= 32 && m % 32 == 0 && n % 32 == 0 && n <= 64 * kNsbHalf &&
         (int64_t)m * (n + kNsbPad) <= kNsbBuf;
}

int launch_ns_small(const void* g, int g_dtype, int BE, int rows, int cols, float scale,
                    uint16_t* out, hipStream_t st) {
  if (g_dtype == UTTT_F32)
    hipLaunchKernelGGL((ns_small_kernel<F32T>), dim3((unsigned)BE), dim3(kNsbThreads), 0, st,
                       static_cast<const float*>(g), rows, cols, scale, out);
  else
    hipLaunchKernelGGL((ns_small_kernel<BF16T>), dim3((unsigned)BE), dim3(kNsbThreads), 0, st,
                       static_cast<const uint16_t*>(g), rows, cols, scale, out);
  return check_launch("newton_schulz5(one launch)");
}

}  // namespace uttt
