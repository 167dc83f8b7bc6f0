// Row-wise preprocessing of the fast-weight update inputs for gfx950: the
// optional silu of k and v and the l2 norm x / (|x| + 1e-5) over each row
// (a head of k, or v's whole feature vector).  Reference:
//   l2_norm              uttt_llm/flame/custom_models/uttt_moe/ref_base.py:182-186
//   _preprocess_update_inputs (qkv_silu, v_norm, qk_norm with the "l2" norms)
//                        uttt_llm/flame/custom_models/uttt_moe/modeling_recurrent_lact.py:641-648
//
// Rounding points are those of the reference's tensor arithmetic in the
// storage dtype: silu rounds to the dtype; the norm is an fp32 sum of squares
// rounded to the dtype, the eps is added in the dtype, and the quotient is
// rounded to the dtype (fp32 rows: every step in fp32).
//
// One wave per row, 8 elements (one 16-byte bf16 vector or two fp32 ones)
// per lane step; the row stays in registers between the sum and the divide,
// so the row is read once and written once.
#include "common.h"

namespace uttt {
namespace {

constexpr int kMaxChunksPerLane = 8;  // rows of up to 64 * 8 * 8 = 4096 elements

template <class TT>
__device__ __forceinline__ void load8(const typename TT::S* p, float (&v)[8]) {
  if constexpr (sizeof(typename TT::S) == 2) {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[2 * k] = TT::load((uint16_t)(w[k] & 0xffffu));
      v[2 * k + 1] = TT::load((uint16_t)(w[k] >> 16));
    }
  } else {
    const float4 a = *reinterpret_cast<const float4*>(p);
    const float4 b = *reinterpret_cast<const float4*>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
}

template <class TT>
__device__ __forceinline__ void store8(typename TT::S* p, const float (&v)[8]) {
  if constexpr (sizeof(typename TT::S) == 2) {
    uint4 u;
    u.x = (uint32_t)TT::store(v[0]) | ((uint32_t)TT::store(v[1]) << 16);
    u.y = (uint32_t)TT::store(v[2]) | ((uint32_t)TT::store(v[3]) << 16);
    u.z = (uint32_t)TT::store(v[4]) | ((uint32_t)TT::store(v[5]) << 16);
    u.w = (uint32_t)TT::store(v[6]) | ((uint32_t)TT::store(v[7]) << 16);
    *reinterpret_cast<uint4*>(p) = u;
  } else {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4*>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
  }
}

// the storage dtype's rounding of an fp32 value
template <class TT>
__device__ __forceinline__ float rnd(float x) {
  return TT::load(TT::store(x));
}

template <class TT>
__global__ __launch_bounds__(256) void rows_silu_l2_kernel(const typename TT::S* __restrict__ in,
                                                           int64_t rows, int D, int64_t ld_in,
                                                           int silu, int l2,
                                                           typename TT::S* __restrict__ out,
                                                           int64_t ld_out) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const int chunks = D / 8;
  const typename TT::S* src = in + row * ld_in;
  typename TT::S* dst = out + row * ld_out;
  float v[kMaxChunksPerLane][8];
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < kMaxChunksPerLane; ++c) {
    const int ch = lane + 64 * c;
    // clamped (always valid) address, every load issued before any use
    load8<TT>(src + 8 * (ch < chunks ? ch : chunks - 1), v[c]);
  }
#pragma unroll
  for (int c = 0; c < kMaxChunksPerLane; ++c) {
    const bool ok = lane + 64 * c < chunks;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      float x = v[c][u];
      if (silu) x = rnd<TT>(x / (1.0f + __expf(-x)));
      v[c][u] = x;
      if (ok) ss = __builtin_fmaf(x, x, ss);
    }
  }
  float scale_den = 1.0f;
  if (l2) {
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) ss += __shfl_xor(ss, d, 64);
    const float nrm = rnd<TT>(sqrtf(ss));
    scale_den = rnd<TT>(nrm + 1e-5f);
  }
#pragma unroll
  for (int c = 0; c < kMaxChunksPerLane; ++c) {
    const int ch = lane + 64 * c;
    if (ch >= chunks) continue;
    float o[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) o[u] = l2 ? v[c][u] / scale_den : v[c][u];
    store8<TT>(dst + 8 * ch, o);
  }
}

}  // namespace
}  // namespace uttt

using namespace uttt;

extern "C" int uttt_rows_silu_l2norm(const void* in, int dtype, int64_t rows, int D,
                                     int64_t ld_in, int silu, int l2, void* out, int64_t ld_out,
                                     void* stream) {
  UTTT_REQUIRE(rows >= 0 && D >= 0, "rows_silu_l2norm: bad sizes rows=%lld D=%d",
               (long long)rows, D);
  if (rows == 0 || D == 0) return UTTT_OK;
  UTTT_REQUIRE(in && out, "rows_silu_l2norm: null pointer");
  UTTT_REQUIRE(D % 8 == 0 && ld_in % 8 == 0 && ld_out % 8 == 0 && ld_in >= D && ld_out >= D,
               "rows_silu_l2norm: D=%d and the row strides must be multiples of 8 (D <= strides)",
               D);
  UTTT_REQUIRE(D <= 64 * 8 * kMaxChunksPerLane, "rows_silu_l2norm: D=%d exceeds %d", D,
               64 * 8 * kMaxChunksPerLane);
  UTTT_REQUIRE(((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) & 15u) == 0,
               "rows_silu_l2norm: tensors must be 16-byte aligned");
  UTTT_REQUIRE(dtype == UTTT_BF16 || dtype == UTTT_F32 || dtype == UTTT_F16,
               "rows_silu_l2norm: dtype code %d", dtype);
  const int64_t blocks = (rows + 3) / 4;
  UTTT_REQUIRE(blocks <= 0x7fffffffLL, "rows_silu_l2norm: too many rows");
  hipStream_t st = as_stream(stream);
  UTTT_DTYPE_SWITCH_LR(dtype, TT, {
    using S = typename TT::S;
    hipLaunchKernelGGL(rows_silu_l2_kernel<TT>, dim3((unsigned)blocks), dim3(256), 0, st,
                       static_cast<const S*>(in), rows, D, ld_in, silu, l2, static_cast<S*>(out),
                       ld_out);
  });
  return check_launch("rows_silu_l2norm");
}
