// uTTT-Dense read for small heads, fused: out = W1 (silu(W0 x) * (W2 x)) per
// head, reading x and writing out in the model's [b, l, H*D] layout.
// Reference: _apply_fast_weights, uttt_dense/modeling_recurrent_lact.py:241-261
// (the rearrange of x at :251, the three bmm at :256-260, the output
// rearrange at :261).
//
// One workgroup = 4 waves = 32 tokens of one head.  The hidden units are cut
// into 32-wide blocks, block j owned by wave j % 4.  For each of its blocks a
// wave
//   1. computes Y0 = W0[blk] x^T and Y2 = W2[blk] x^T (32 hidden x 32 tokens,
//      K = D) on v_mfma_f32_32x32x16_bf16, x^T fragments held in registers
//      for the whole kernel;
//   2. forms h = bf16(Y2 * silu(Y0)) in the accumulator layout (lane = token,
//      16 hidden units per lane);
//   3. feeds h straight back as the B operand of out^T += W1[:, blk] h^T: the
//      accumulator's hidden units are a permutation of the MFMA's k slots, and
//      the W1 fragments are loaded in that same permutation (two 8-byte
//      loads), so h never leaves the registers.
// The four waves' fp32 partials of out^T meet in LDS and are summed in wave
// order; the bf16 result is stored as 16-byte runs of each token's head
// columns.  Rounding points as the grouped path's: fp32 Y0/Y2, bf16 h, fp32
// accumulation of the down product, one bf16 rounding of out.
//
// The weights ((2I + I) x D bf16 per head) are read by every token tile of the
// head from L2; x and out cross HBM once.
#include <stdint.h>

#include "common.h"

namespace uttt {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kReadTok = 32;  // tokens per workgroup
constexpr int kReadWaves = 4;

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

__device__ __forceinline__ bf16x8_t ld16(const uint16_t* p) {
  return *reinterpret_cast<const bf16x8_t*>(p);
}
__device__ __forceinline__ bf16x4_t ld8(const uint16_t* p) {
  return *reinterpret_cast<const bf16x4_t*>(p);
}
__device__ __forceinline__ float silu_mul(float y0, float y2) {
  return y2 * (y0 * __builtin_amdgcn_rcpf(1.0f + __expf(-y0)));
}

// Fragment-ordered copy of one head's weights (uttt_dense_pack_weights), the
// same bytes as W0_W2 [2I, D] and W1 [D, I] regrouped so that each of the
// read's fragment loads is 64 lanes x 16 consecutive bytes (8 cache lines)
// instead of 16 bytes from each of 32 weight rows:
//   W0 / W2 part m (0 / 1): [I/32 blocks][D/16 k steps][64 lanes][8], lane
//     (r, g) holding row 32 blk + r, columns 16 s + 8 g .. + 8 of W_m;
//   W1 part: [I/32 blocks][2 halves q][D/32 column blocks db][64 lanes][8],
//     lane (r, g) holding W1[32 db + r][32 blk + 16 q + 4 g .. + 4] then
//     W1[32 db + r][32 blk + 16 q + 8 + 4 g .. + 4].
__host__ __device__ constexpr int64_t packed_head_elems(int D, int I) { return (int64_t)3 * I * D; }

__global__ __launch_bounds__(256) void dense_pack_kernel(const uint16_t* __restrict__ w02,
                                                         const uint16_t* __restrict__ w1, int D,
                                                         int I, uint16_t* __restrict__ packed) {
  // 32-bit index math: a head holds at most 3 * 512 * 256 / 8 = 49152 chunks
  const int bh = blockIdx.y;
  const int nch = 3 * I * D / 8;  // 16-byte chunks per head
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= nch) return;
  const int KS = D / 16, DB = D / 32;
  const int per_mat = I * D / 8;
  const int lane = c & 63, r = lane & 31, g = lane >> 5;
  uint4 v;
  if (c < 2 * per_mat) {
    const int m = c >= per_mat;
    const int q = (c - m * per_mat) >> 6;  // blk * KS + s
    const int blk = q / KS, s = q - blk * KS;
    const uint16_t* src = w02 + (int64_t)bh * 2 * I * D + (m * I + blk * 32 + r) * D + 16 * s +
                          8 * g;
    v = *reinterpret_cast<const uint4*>(src);
  } else {
    const int q = (c - 2 * per_mat) >> 6;  // (blk * 2 + half) * DB + db
    const int qd = q / DB, db = q - qd * DB, half = qd & 1, blk = qd >> 1;
    const uint16_t* row =
        w1 + (int64_t)bh * D * I + (db * 32 + r) * I + blk * 32 + 16 * half + 4 * g;
    const uint2 lo = *reinterpret_cast<const uint2*>(row);
    const uint2 hi = *reinterpret_cast<const uint2*>(row + 8);
    v = make_uint4(lo.x, lo.y, hi.x, hi.y);
  }
  *reinterpret_cast<uint4*>(packed + (int64_t)bh * packed_head_elems(D, I) + 8 * c) = v;
}

// PACKED: the weights come from the fragment-ordered copy (w02 = the packed
// copy, w1 unused).
template <int D, int UB, bool PACKED>
__global__ __launch_bounds__(kReadWaves * 64) void dense_read_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w02,
    const uint16_t* __restrict__ w1, int l, int H, int I, uint16_t* __restrict__ out) {
  constexpr int KS = D / 16;  // k steps of the up products
  constexpr int DB = D / 32;  // 32-row blocks of out^T
  constexpr int LD = D + 4;   // LDS row stride (floats), padded
  __shared__ __attribute__((aligned(16))) float part[kReadWaves][kReadTok * LD];

  const int bh = blockIdx.y;  // b * H + head
  const int bb = bh / H, hh = bh % H;
  const int t0 = blockIdx.x * kReadTok;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r = lane & 31, g = lane >> 5;

  // x^T fragments: token t0 + r (clamped), k = 16 s + 8 g .. + 8
  const int tok = min(t0 + r, l - 1);
  const uint16_t* xr = x + (((int64_t)bb * l + tok) * H + hh) * D + 8 * g;
  bf16x8_t xf[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) xf[s] = ld16(xr + 16 * s);

  f32x16_t acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[db][v] = 0.0f;

  const uint16_t* w0h = w02 + (int64_t)bh * 2 * I * D;
  const uint16_t* w1h = w1 + (int64_t)bh * D * I;
  const int nblk = I / 32;
#pragma unroll
  for (int u = 0; u < UB; ++u) {
    const int blk = w + kReadWaves * u;
    if (blk >= nblk) break;  // wave-uniform
    // every weight fragment of the block is requested before the first
    // product: the L2 latency is paid once per block, not once per k step
    bf16x8_t a0f[KS], a2f[KS];
    bf16x8_t w1f[2][DB];
    if constexpr (PACKED) {
      const uint16_t* ph = w02 + (int64_t)bh * packed_head_elems(D, I);
      const uint16_t* p0 = ph + ((int64_t)blk * KS * 64 + lane) * 8;
      const uint16_t* p2 = p0 + (int64_t)I * D;
      const uint16_t* p1 = ph + 2 * (int64_t)I * D + ((int64_t)blk * 2 * DB * 64 + lane) * 8;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        a0f[s] = ld16(p0 + s * 64 * 8);
        a2f[s] = ld16(p2 + s * 64 * 8);
      }
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int db = 0; db < DB; ++db) w1f[q][db] = ld16(p1 + (q * DB + db) * 64 * 8);
    } else {
      const uint16_t* a0 = w0h + (int64_t)(blk * 32 + r) * D + 8 * g;
      const uint16_t* a2 = a0 + (int64_t)I * D;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        a0f[s] = ld16(a0 + 16 * s);
        a2f[s] = ld16(a2 + 16 * s);
      }
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const uint16_t* b1 = w1h + (int64_t)(db * 32 + r) * I + blk * 32 + 16 * q + 4 * g;
          w1f[q][db] = __builtin_shufflevector(ld8(b1), ld8(b1 + 8), 0, 1, 2, 3, 4, 5, 6, 7);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // 1. Y0, Y2 for hidden units blk*32 .. +32 (A = weight rows, B = x^T)
    f32x16_t y0, y2;
#pragma unroll
    for (int v = 0; v < 16; ++v) y0[v] = y2[v] = 0.0f;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      y0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0f[s], xf[s], y0, 0, 0, 0);
      y2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a2f[s], xf[s], y2, 0, 0, 0);
    }
    // 2. h: element v of this lane is hidden unit 8 (v / 4) + 4 g + v % 4 of
    //    the block, token t0 + r
    bf16x8_t hq[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      uint4 p;
      p.x = pack_bf16x2(silu_mul(y0[8 * q], y2[8 * q]), silu_mul(y0[8 * q + 1], y2[8 * q + 1]));
      p.y = pack_bf16x2(silu_mul(y0[8 * q + 2], y2[8 * q + 2]), silu_mul(y0[8 * q + 3], y2[8 * q + 3]));
      p.z = pack_bf16x2(silu_mul(y0[8 * q + 4], y2[8 * q + 4]), silu_mul(y0[8 * q + 5], y2[8 * q + 5]));
      p.w = pack_bf16x2(silu_mul(y0[8 * q + 6], y2[8 * q + 6]), silu_mul(y0[8 * q + 7], y2[8 * q + 7]));
      hq[q] = __builtin_bit_cast(bf16x8_t, p);
    }
    // 3. out^T[dcol, token] += sum_j W1[dcol, j] h[j, token]; k step q takes
    //    h elements 8q .. 8q+7, i.e. hidden units 16q + 4g + 0..3 and
    //    16q + 8 + 4g + 0..3, and the W1 fragment holds the same units
#pragma unroll
    for (int q = 0; q < 2; ++q) {
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w1f[q][db], hq[q], acc[db], 0, 0, 0);
      }
    }
  }

  // partials: lane (token r) holds out^T rows db*32 + 8 (v/4) + 4 g + v%4
  float* pw = part[w] + r * LD;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int v4 = 0; v4 < 4; ++v4)
      *reinterpret_cast<float4*>(pw + db * 32 + 8 * v4 + 4 * g) =
          make_float4(acc[db][4 * v4], acc[db][4 * v4 + 1], acc[db][4 * v4 + 2],
                      acc[db][4 * v4 + 3]);
  __syncthreads();

  // sum in wave order, 8 columns per item, 16-byte stores
  constexpr int CPT = D / 8;  // 8-column chunks per token
  for (int i = threadIdx.x; i < kReadTok * CPT; i += kReadWaves * 64) {
    const int t = i / CPT, c = (i % CPT) * 8;
    if (t0 + t >= l) continue;
    float4 lo = *reinterpret_cast<const float4*>(&part[0][t * LD + c]);
    float4 hi = *reinterpret_cast<const float4*>(&part[0][t * LD + c + 4]);
#pragma unroll
    for (int ww = 1; ww < kReadWaves; ++ww) {
      const float4 a = *reinterpret_cast<const float4*>(&part[ww][t * LD + c]);
      const float4 b = *reinterpret_cast<const float4*>(&part[ww][t * LD + c + 4]);
      lo.x += a.x; lo.y += a.y; lo.z += a.z; lo.w += a.w;
      hi.x += b.x; hi.y += b.y; hi.z += b.z; hi.w += b.w;
    }
    uint4 o;
    o.x = pack_bf16x2(lo.x, lo.y);
    o.y = pack_bf16x2(lo.z, lo.w);
    o.z = pack_bf16x2(hi.x, hi.y);
    o.w = pack_bf16x2(hi.z, hi.w);
    *reinterpret_cast<uint4*>(out + (((int64_t)bb * l + t0 + t) * H + hh) * D + c) = o;
  }
}

template <int D, bool PACKED>
int launch_dense_read(int ub, dim3 grid, hipStream_t st, const uint16_t* x, const uint16_t* w02,
                      const uint16_t* w1, int l, int H, int I, uint16_t* out) {
  const dim3 block(kReadWaves * 64);
  switch (ub) {
    case 1: hipLaunchKernelGGL((dense_read_kernel<D, 1, PACKED>), grid, block, 0, st, x, w02, w1, l, H, I, out); break;
    case 2: hipLaunchKernelGGL((dense_read_kernel<D, 2, PACKED>), grid, block, 0, st, x, w02, w1, l, H, I, out); break;
    case 3: hipLaunchKernelGGL((dense_read_kernel<D, 3, PACKED>), grid, block, 0, st, x, w02, w1, l, H, I, out); break;
    default: hipLaunchKernelGGL((dense_read_kernel<D, 4, PACKED>), grid, block, 0, st, x, w02, w1, l, H, I, out); break;
  }
  return check_launch("dense_read");
}

template <bool PACKED>
int dense_read_dispatch(int D, int ub, dim3 grid, hipStream_t st, const uint16_t* x,
                        const uint16_t* w02, const uint16_t* w1, int l, int H, int I,
                        uint16_t* out) {
  switch (D) {
    case 64: return launch_dense_read<64, PACKED>(ub, grid, st, x, w02, w1, l, H, I, out);
    case 96: return launch_dense_read<96, PACKED>(ub, grid, st, x, w02, w1, l, H, I, out);
    case 128: return launch_dense_read<128, PACKED>(ub, grid, st, x, w02, w1, l, H, I, out);
    case 192: return launch_dense_read<192, PACKED>(ub, grid, st, x, w02, w1, l, H, I, out);
    default: return launch_dense_read<256, PACKED>(ub, grid, st, x, w02, w1, l, H, I, out);
  }
}

}  // namespace
}  // namespace uttt

using namespace uttt;

extern "C" int uttt_dense_read_supported(int D, int I) {
  return (D == 64 || D == 96 || D == 128 || D == 192 || D == 256) && I >= 32 && I % 32 == 0 &&
         I <= 512;
}

extern "C" int uttt_dense_read(const void* x, int b, int l, int H, int D, const void* w0_w2,
                               const void* w1, int I, void* out, void* stream) {
  UTTT_REQUIRE(b >= 0 && l >= 0 && H >= 1, "dense_read: bad sizes");
  UTTT_REQUIRE(uttt_dense_read_supported(D, I),
               "dense_read: D=%d must be 64, 96, 128, 192 or 256 and I=%d a multiple of 32 "
               "in [32, 512]", D, I);
  if (b == 0 || l == 0) return UTTT_OK;
  UTTT_REQUIRE((int64_t)b * H <= 65535, "dense_read: b*H=%lld exceeds 65535", (long long)b * H);
  UTTT_REQUIRE(x && w0_w2 && w1 && out, "dense_read: null pointer");
  UTTT_REQUIRE(aligned16(x) && aligned16(w0_w2) && aligned16(w1) && aligned16(out),
               "dense_read: tensors must be 16-byte aligned");
  const int ub = (I / 32 + kReadWaves - 1) / kReadWaves;
  const dim3 grid((unsigned)((l + kReadTok - 1) / kReadTok), (unsigned)(b * H));
  hipStream_t st = as_stream(stream);
  return dense_read_dispatch<false>(D, ub, grid, st, static_cast<const uint16_t*>(x),
                                    static_cast<const uint16_t*>(w0_w2),
                                    static_cast<const uint16_t*>(w1), l, H, I,
                                    static_cast<uint16_t*>(out));
}

extern "C" int uttt_dense_pack_weights(const void* w0_w2, const void* w1, int BH, int D, int I,
                                       void* packed, void* stream) {
  UTTT_REQUIRE(BH >= 0, "dense_pack_weights: bad sizes");
  UTTT_REQUIRE(uttt_dense_read_supported(D, I),
               "dense_pack_weights: D=%d must be 64, 96, 128, 192 or 256 and I=%d a multiple of "
               "32 in [32, 512]", D, I);
  if (BH == 0) return UTTT_OK;
  UTTT_REQUIRE(BH <= 65535, "dense_pack_weights: BH=%d exceeds 65535", BH);
  UTTT_REQUIRE(w0_w2 && w1 && packed, "dense_pack_weights: null pointer");
  UTTT_REQUIRE(aligned16(w0_w2) && aligned16(w1) && aligned16(packed),
               "dense_pack_weights: tensors must be 16-byte aligned");
  const int64_t nch = (int64_t)3 * I * D / 8;
  const dim3 grid((unsigned)((nch + 255) / 256), (unsigned)BH);
  hipLaunchKernelGGL(dense_pack_kernel, grid, dim3(256), 0, as_stream(stream),
                     static_cast<const uint16_t*>(w0_w2), static_cast<const uint16_t*>(w1), D, I,
                     static_cast<uint16_t*>(packed));
  return check_launch("dense_pack_weights");
}

extern "C" int uttt_dense_read_packed(const void* x, int b, int l, int H, int D,
                                      const void* packed, int I, void* out, void* stream) {
  UTTT_REQUIRE(b >= 0 && l >= 0 && H >= 1, "dense_read_packed: bad sizes");
  UTTT_REQUIRE(uttt_dense_read_supported(D, I),
               "dense_read_packed: D=%d must be 64, 96, 128, 192 or 256 and I=%d a multiple of "
               "32 in [32, 512]", D, I);
  if (b == 0 || l == 0) return UTTT_OK;
  UTTT_REQUIRE((int64_t)b * H <= 65535, "dense_read_packed: b*H=%lld exceeds 65535",
               (long long)b * H);
  UTTT_REQUIRE(x && packed && out, "dense_read_packed: null pointer");
  UTTT_REQUIRE(aligned16(x) && aligned16(packed) && aligned16(out),
               "dense_read_packed: tensors must be 16-byte aligned");
  const int ub = (I / 32 + kReadWaves - 1) / kReadWaves;
  const dim3 grid((unsigned)((l + kReadTok - 1) / kReadTok), (unsigned)(b * H));
  return dense_read_dispatch<true>(D, ub, grid, as_stream(stream),
                                   static_cast<const uint16_t*>(x),
                                   static_cast<const uint16_t*>(packed), nullptr, l, H, I,
                                   static_cast<uint16_t*>(out));
}
