// Row-wise preprocessing of the fast-weight inputs for gfx950, forward and
// backward: optional silu, then an optional parameter-free norm over each row
// (l2: x / (|x| + 1e-5); rms: x * rsqrt(mean(x^2) + 1e-5)), then an optional
// rotary embedding over blocks of rope_dim features (first half / second
// half pairs, positions from the row's token index plus an offset).
// Reference:
//   _preprocess_update_inputs  uttt_llm/flame/custom_models/uttt_moe/modeling_recurrent_lact.py:630-657
//   q path of the MoE read      ibid. :588-601
//   l2_norm, rms_norm           uttt_llm/flame/custom_models/uttt_moe/ref_base.py:181-195
//   the fast-weight rotary      ref_base.py:342-355 (RotaryEmbedding of rotary.py, bf16 cos / sin
//                               tables of rotary.py:394-433, non-interleaved kernel rotary.py:83-104)
//
// Rounding points are the reference's: F.silu rounds to the storage dtype;
// l2_norm / rms_norm are torch.compile'd, so the norm and the denominator stay
// in fp32 and only the normalised value is rounded to the storage dtype; the
// rotary input is cast to the tables' dtype (bf16), rotated in fp32 with the
// bf16 table values and stored in bf16.  The backward rounds where the
// reference's autograd does: the rotary backward (the conjugate rotation)
// stores bf16, the compiled norm's backward and the silu backward store the
// input dtype.
//
// One wave per row, 8 elements (one 16-byte bf16 vector or two fp32 ones)
// per lane step; the row stays in registers between the reductions and the
// element pass, so the row is read once and written once.  A rotary pair
// (j, j + R) of a block sits R / 8 lanes apart in the same lane step (blocks
// of 2R elements tile the 512 elements of a step when 2R divides 512), so the
// partner values come from one lane exchange.
#include <type_traits>

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

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int d = 32; d > 0; d >>= 1) v += __shfl_xor(v, d, 64);
  return v;
}

enum Norm { kNone = 0, kL2 = 1, kRms = 2 };

// Geometry shared by the forward and backward kernels.
struct Rows {
  int64_t rows;
  int D;               // row length (a norm row: a head of q / k, or all of v)
  int64_t ld_in, ld_out;
  int silu, norm;
  // rotary (rope_half = 0: none); table row = token % seq_len + pos_offset
  const uint16_t* cos;  // [table_rows, rope_half] bf16
  const uint16_t* sin;
  int rope_half, rows_per_token, seq_len, pos_offset;
};

// The rotary step of one lane step's chunk (8 elements of a row at element
// offset e0 of the token): x -> the rotated values, with `conj` the conjugate
// (the backward).  Every lane of the wave calls it (the exchange is a
// shuffle); lanes past the row end carry values that are never stored.
__device__ __forceinline__ void rope8(float (&x)[8], const Rows& a, int64_t row, int e0,
                                      bool conj) {
  const int R = a.rope_half;
  const int tok_pos = (int)((row / a.rows_per_token) % a.seq_len) + a.pos_offset;
  const int j0 = e0 % (2 * R);
  const bool first = j0 < R;
  const int jj = first ? j0 : j0 - R;
  const uint4 cu = *reinterpret_cast<const uint4*>(a.cos + (int64_t)tok_pos * R + jj);
  const uint4 su = *reinterpret_cast<const uint4*>(a.sin + (int64_t)tok_pos * R + jj);
  const uint32_t cw[4] = {cu.x, cu.y, cu.z, cu.w}, sw[4] = {su.x, su.y, su.z, su.w};
  const int dl = R / 8;  // partner lane distance
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const float c = bf16_to_f32((uint16_t)(u & 1 ? cw[u / 2] >> 16 : cw[u / 2] & 0xffffu));
    float s = bf16_to_f32((uint16_t)(u & 1 ? sw[u / 2] >> 16 : sw[u / 2] & 0xffffu));
    if (conj) s = -s;
    const float p = __shfl_xor(x[u], dl, 64);
    // first half: x0 cos - x1 sin; second half: x0 sin + x1 cos (x0 = partner)
    x[u] = first ? x[u] * c - p * s : p * s + x[u] * c;
  }
}

template <class TI, bool ROPE>
__global__ __launch_bounds__(256) void rows_prep_kernel(const typename TI::S* __restrict__ in,
                                                        Rows a,
                                                        typename std::conditional<ROPE, BF16T, TI>::type::S* __restrict__ out) {
  using TO = typename std::conditional<ROPE, BF16T, TI>::type;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;  // wave-uniform
  const int lane = threadIdx.x & 63;
  const int chunks = a.D / 8;
  const typename TI::S* src = in + row * a.ld_in;
  typename TO::S* dst = out + row * a.ld_out;
  float v[kMaxChunksPerLane][8];
#pragma unroll
  for (int c = 0; c < kMaxChunksPerLane; ++c) {
    const int ch = lane + 64 * c;
    // clamped (always valid) address, every load issued before any use
    load8<TI>(src + 8 * (ch < chunks ? ch : chunks - 1), v[c]);
  }
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < kMaxChunksPerLane; ++c) {
    const bool ok = lane + 64 * c < chunks;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      float x = v[c][u];
      if (a.silu) x = rnd<TI>(x / (1.0f + __expf(-x)));
      v[c][u] = x;
      if (ok) ss = __builtin_fmaf(x, x, ss);
    }
  }
  float den = 1.0f, scale = 1.0f;
  if (a.norm == kL2) {
    den = sqrtf(wave_sum(ss)) + 1e-5f;
  } else if (a.norm == kRms) {
    scale = __builtin_amdgcn_rsqf(wave_sum(ss) / (float)a.D + 1e-5f);
  }
  const int e_row = ROPE ? (int)(row % a.rows_per_token) * a.D : 0;
#pragma unroll
  for (int c = 0; c < kMaxChunksPerLane; ++c) {
    if (64 * c >= chunks) break;  // wave-uniform
    const int ch = lane + 64 * c;
    float o[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      float y = v[c][u];
      if (a.norm == kL2) y = y / den;
      else if (a.norm == kRms) y = y * scale;
      o[u] = rnd<TI>(y);  // the norm's output, in the input dtype
    }
    if constexpr (ROPE) {
#pragma unroll
      for (int u = 0; u < 8; ++u) o[u] = rnd<BF16T>(o[u]);  // cast to the tables' dtype
      rope8(o, a, row, e_row + 8 * (ch < chunks ? ch : chunks - 1), false);
    }
    if (ch < chunks) store8<TO>(dst + 8 * ch, o);
  }
}

// grad_in of the row preprocessing given grad_out (the output's dtype):
// conjugate rotation (bf16), the norm's backward on the recomputed silu
// output (fp32, rounded to the input dtype), the silu backward (rounded to
// the input dtype).
template <class TI, bool ROPE>
__global__ __launch_bounds__(256) void rows_prep_bwd_kernel(
    const typename TI::S* __restrict__ in, Rows a,
    const typename std::conditional<ROPE, BF16T, TI>::type::S* __restrict__ gout,
    typename TI::S* __restrict__ gin) {
  using TO = typename std::conditional<ROPE, BF16T, TI>::type;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;  // wave-uniform
  const int lane = threadIdx.x & 63;
  const int chunks = a.D / 8;
  const typename TI::S* src = in + row * a.ld_in;
  const typename TO::S* gsrc = gout + row * a.ld_out;
  typename TI::S* dst = gin + row * a.ld_in;
  float x[kMaxChunksPerLane][8], g[kMaxChunksPerLane][8];
#pragma unroll
  for (int c = 0; c < kMaxChunksPerLane; ++c) {
    const int ch = lane + 64 * c;
    const int cc = ch < chunks ? ch : chunks - 1;
    load8<TI>(src + 8 * cc, x[c]);
    load8<TO>(gsrc + 8 * cc, g[c]);
  }
  const int e_row = ROPE ? (int)(row % a.rows_per_token) * a.D : 0;
  float ss = 0.0f, dot = 0.0f;
#pragma unroll
  for (int c = 0; c < kMaxChunksPerLane; ++c) {
    const int ch = lane + 64 * c;
    const bool ok = ch < chunks;
    if constexpr (ROPE) {
      if (64 * c < chunks) {  // wave-uniform
        rope8(g[c], a, row, e_row + 8 * (ok ? ch : chunks - 1), true);
#pragma unroll
        for (int u = 0; u < 8; ++u) g[c][u] = rnd<TI>(rnd<BF16T>(g[c][u]));
      }
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float s = a.silu ? rnd<TI>(x[c][u] / (1.0f + __expf(-x[c][u]))) : x[c][u];
      if (ok) {
        ss = __builtin_fmaf(s, s, ss);
        dot = __builtin_fmaf(s, g[c][u], dot);
      }
    }
  }
  float den = 1.0f, coef = 0.0f, scale = 1.0f;
  if (a.norm == kL2) {
    const float n = sqrtf(wave_sum(ss));
    dot = wave_sum(dot);
    den = n + 1e-5f;
    coef = n > 0.0f ? dot / (n * den * den) : 0.0f;
  } else if (a.norm == kRms) {
    scale = __builtin_amdgcn_rsqf(wave_sum(ss) / (float)a.D + 1e-5f);
    dot = wave_sum(dot);
    coef = dot * scale * scale * scale / (float)a.D;
  }
#pragma unroll
  for (int c = 0; c < kMaxChunksPerLane; ++c) {
    const int ch = lane + 64 * c;
    if (ch >= chunks) continue;
    float o[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float xv = x[c][u];
      const float sg = 1.0f / (1.0f + __expf(-xv));
      const float s = a.silu ? rnd<TI>(xv * sg) : xv;
      float gs = g[c][u];
      if (a.norm == kL2) gs = rnd<TI>(gs / den - s * coef);
      else if (a.norm == kRms) gs = rnd<TI>(scale * gs - s * coef);
      o[u] = a.silu ? gs * (sg * (1.0f + xv * (1.0f - sg))) : gs;
    }
    store8<TI>(dst + 8 * ch, o);
  }
}

int check_rows(const Rows& a, const void* in, const void* out, int dtype, const char* what) {
  UTTT_REQUIRE(a.rows >= 0 && a.D >= 0, "%s: bad sizes rows=%lld D=%d", what, (long long)a.rows,
               a.D);
  UTTT_REQUIRE(in && out, "%s: null pointer", what);
  UTTT_REQUIRE(a.D % 8 == 0 && a.ld_in % 8 == 0 && a.ld_out % 8 == 0 && a.ld_in >= a.D &&
                   a.ld_out >= a.D,
               "%s: D=%d and the row strides must be multiples of 8 (D <= strides)", what, a.D);
  UTTT_REQUIRE(a.D <= 64 * 8 * kMaxChunksPerLane, "%s: D=%d exceeds %d", what, a.D,
               64 * 8 * kMaxChunksPerLane);
  UTTT_REQUIRE(((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) & 15u) == 0,
               "%s: tensors must be 16-byte aligned", what);
  UTTT_REQUIRE(dtype == UTTT_BF16 || dtype == UTTT_F32 || dtype == UTTT_F16, "%s: dtype code %d",
               what, dtype);
  UTTT_REQUIRE(a.silu == 0 || a.silu == 1, "%s: silu must be 0 or 1", what);
  UTTT_REQUIRE(a.norm == kNone || a.norm == kL2 || a.norm == kRms,
               "%s: norm must be 0 (none), 1 (l2) or 2 (rms)", what);
  UTTT_REQUIRE((a.rows + 3) / 4 <= 0x7fffffffLL, "%s: too many rows", what);
  if (a.rope_half > 0) {
    const int R = a.rope_half;
    UTTT_REQUIRE(R == 8 || R == 16 || R == 32 || R == 64 || R == 128,
                 "%s: rope_dim=%d must be 16, 32, 64, 128 or 256", what, 2 * R);
    UTTT_REQUIRE(a.D % (2 * R) == 0, "%s: rows of D=%d must hold whole rotary blocks of %d", what,
                 a.D, 2 * R);
    UTTT_REQUIRE(a.cos && a.sin && ((reinterpret_cast<uintptr_t>(a.cos) |
                                     reinterpret_cast<uintptr_t>(a.sin)) & 15u) == 0,
                 "%s: rotary tables must be 16-byte aligned", what);
    UTTT_REQUIRE(a.rows_per_token >= 1 && a.seq_len >= 1 && a.pos_offset >= 0,
                 "%s: rows_per_token=%d, seq_len=%d, pos_offset=%d", what, a.rows_per_token,
                 a.seq_len, a.pos_offset);
    UTTT_REQUIRE(a.rows % ((int64_t)a.rows_per_token * a.seq_len) == 0,
                 "%s: %lld rows are not whole sequences of %d tokens x %d rows", what,
                 (long long)a.rows, a.seq_len, a.rows_per_token);
  }
  return UTTT_OK;
}

Rows make_rows(int64_t rows, int D, int64_t ld_in, int64_t ld_out, int silu, int norm,
               const void* cos, const void* sin, int rope_dim, int rows_per_token, int seq_len,
               int pos_offset) {
  Rows a;
  a.rows = rows;
  a.D = D;
  a.ld_in = ld_in;
  a.ld_out = ld_out;
  a.silu = silu;
  a.norm = norm;
  a.cos = static_cast<const uint16_t*>(cos);
  a.sin = static_cast<const uint16_t*>(sin);
  a.rope_half = rope_dim > 0 ? rope_dim / 2 : 0;
  a.rows_per_token = rows_per_token;
  a.seq_len = seq_len;
  a.pos_offset = pos_offset;
  return a;
}

}  // namespace
}  // namespace uttt

using namespace uttt;

extern "C" int uttt_rows_preprocess(const void* in, int dtype, int64_t rows, int D, int64_t ld_in,
                                    int silu, int norm, const void* rope_cos,
                                    const void* rope_sin, int rope_dim, int rows_per_token,
                                    int seq_len, int pos_offset, int table_rows, void* out,
                                    int64_t ld_out, void* stream) {
  const Rows a = make_rows(rows, D, ld_in, ld_out, silu, norm, rope_cos, rope_sin, rope_dim,
                           rows_per_token, seq_len, pos_offset);
  if (rows == 0 || D == 0) return UTTT_OK;
  if (int rc = check_rows(a, in, out, dtype, "rows_preprocess")) return rc;
  UTTT_REQUIRE(rope_dim == 0 || pos_offset + seq_len <= table_rows,
               "rows_preprocess: positions up to %d past the rotary table's %d rows",
               pos_offset + seq_len, table_rows);
  const unsigned blocks = (unsigned)((rows + 3) / 4);
  hipStream_t st = as_stream(stream);
  UTTT_DTYPE_SWITCH_LR(dtype, TT, {
    using S = typename TT::S;
    if (rope_dim > 0)
      hipLaunchKernelGGL((rows_prep_kernel<TT, true>), dim3(blocks), dim3(256), 0, st,
                         static_cast<const S*>(in), a, static_cast<uint16_t*>(out));
    else
      hipLaunchKernelGGL((rows_prep_kernel<TT, false>), dim3(blocks), dim3(256), 0, st,
                         static_cast<const S*>(in), a, static_cast<S*>(out));
  });
  return check_launch("rows_preprocess");
}

extern "C" int uttt_rows_preprocess_bwd(const void* in, int dtype, const void* grad_out,
                                        int64_t rows, int D, int64_t ld_in, int64_t ld_out,
                                        int silu, int norm, const void* rope_cos,
                                        const void* rope_sin, int rope_dim, int rows_per_token,
                                        int seq_len, int pos_offset, int table_rows,
                                        void* grad_in, void* stream) {
  const Rows a = make_rows(rows, D, ld_in, ld_out, silu, norm, rope_cos, rope_sin, rope_dim,
                           rows_per_token, seq_len, pos_offset);
  if (rows == 0 || D == 0) return UTTT_OK;
  if (int rc = check_rows(a, in, grad_in, dtype, "rows_preprocess_bwd")) return rc;
  UTTT_REQUIRE(grad_out && (reinterpret_cast<uintptr_t>(grad_out) & 15u) == 0,
               "rows_preprocess_bwd: grad_out must be a 16-byte aligned tensor");
  UTTT_REQUIRE(rope_dim == 0 || pos_offset + seq_len <= table_rows,
               "rows_preprocess_bwd: positions up to %d past the rotary table's %d rows",
               pos_offset + seq_len, table_rows);
  const unsigned blocks = (unsigned)((rows + 3) / 4);
  hipStream_t st = as_stream(stream);
  UTTT_DTYPE_SWITCH_LR(dtype, TT, {
    using S = typename TT::S;
    if (rope_dim > 0)
      hipLaunchKernelGGL((rows_prep_bwd_kernel<TT, true>), dim3(blocks), dim3(256), 0, st,
                         static_cast<const S*>(in), a, static_cast<const uint16_t*>(grad_out),
                         static_cast<S*>(grad_in));
    else
      hipLaunchKernelGGL((rows_prep_bwd_kernel<TT, false>), dim3(blocks), dim3(256), 0, st,
                         static_cast<const S*>(in), a, static_cast<const S*>(grad_out),
                         static_cast<S*>(grad_in));
  });
  return check_launch("rows_preprocess_bwd");
}
