// Fast-weight WRITE step for gfx950: optional momentum, the step
// U = W + s * G, and the norm-preserving projection P = U / (|U| + 1e-5) * nu
// of every row segment, with nu the segment's norm before the step.
//
// reference: _apply_moe_update_dense,
//   uttt_llm/flame/custom_models/uttt_moe/modeling_recurrent_lact.py:754-825
//   (segment = whole row of the fp32 master, nu from the master, the master
//   takes P), and _apply_shared_update,
//   uttt_llm/flame/custom_models/uttt_dense/modeling_recurrent_lact.py:1109-1240
//   (segment = d-wide piece of a row, nu from the bf16 fast weight, the master
//   keeps U unless master renorm is on).
//
// One 64-lane wave owns one segment of S elements; lane l holds the 16-byte
// chunks l, l + 64, ... of it in registers, so each tensor is read once and
// written once (HBM-bound: 4 + |G| + 4 + 2 bytes per element, plus 8 with
// momentum and 2 when nu comes from the fast weight).  The arithmetic keeps
// the reference's operation order in fp32: G + M * m, W + G * s as a separate
// multiply and add, U / (|U| + eps) * nu as divide then multiply.
#include "common.h"

namespace uttt {
namespace {

constexpr int kWS = 256;  // 4 waves = 4 segments per workgroup

struct alignas(8) Half4 {
  uint16_t h[4];
};

// Every tensor of the write is read once and written once, so all of them
// move with non-temporal loads and stores (measured at C4: the pool write
// 1.26 -> 0.96 ms).
typedef float nt_f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int nt_u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float4 nt_load4(const float* p) {
  const nt_f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const nt_f32x4*>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void nt_store4(float* p, const float4& v) {
  const nt_f32x4 w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, reinterpret_cast<nt_f32x4*>(p));
}
__device__ __forceinline__ Half4 nt_load_h4(const uint16_t* p) {
  const nt_u32x2 raw = __builtin_nontemporal_load(reinterpret_cast<const nt_u32x2*>(p));
  Half4 v;
  __builtin_memcpy(&v, &raw, sizeof(v));
  return v;
}
__device__ __forceinline__ void nt_store_h4(uint16_t* p, const Half4& v) {
  nt_u32x2 raw;
  __builtin_memcpy(&raw, &v, sizeof(raw));
  __builtin_nontemporal_store(raw, reinterpret_cast<nt_u32x2*>(p));
}

template <class GT>
__device__ __forceinline__ float4 load_grad4(const typename GT::S* p) {
  if constexpr (sizeof(typename GT::S) == 4) {
    return nt_load4(reinterpret_cast<const float*>(p));
  } else {
    const Half4 v = nt_load_h4(reinterpret_cast<const uint16_t*>(p));
    return make_float4(GT::load(v.h[0]), GT::load(v.h[1]), GT::load(v.h[2]), GT::load(v.h[3]));
  }
}

__device__ __forceinline__ float sumsq4(float4 v) {
  float s = v.x * v.x;
  s = __builtin_fmaf(v.y, v.y, s);
  s = __builtin_fmaf(v.z, v.z, s);
  return __builtin_fmaf(v.w, v.w, s);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int d = kWave / 2; d > 0; d >>= 1) v += __shfl_xor(v, d, kWave);
  return v;
}

// master / master_out and mom_in / mom_out may alias (in-place write): every
// element is read into registers before the same lane overwrites it.
template <class GT, int NV, bool MOM, bool FASTNORM>
__global__ __launch_bounds__(kWS) void write_step_kernel(
    const float* master, const uint16_t* __restrict__ fast_in,
    const typename GT::S* __restrict__ grad, const float* mom_in, const float* __restrict__ m_coeff,
    float lr_scale, int64_t nseg, int64_t seg_per_batch, int S, int renorm_master,
    float* master_out, uint16_t* __restrict__ fast_out, float* mom_out) {
#pragma clang fp contract(off)
  const int64_t seg = (int64_t)blockIdx.x * (kWS / kWave) + threadIdx.x / kWave;
  if (seg >= nseg) return;  // whole wave leaves together
  const int lane = lane_id();
  const int64_t base = seg * S;
  const float mc = MOM ? m_coeff[seg / seg_per_batch] : 0.0f;
  float4 u[NV];
  float ss_old = 0.0f, ss_new = 0.0f;
  // Every load is unconditional (a lane past the row end re-reads the row's
  // first vector and zeroes it), so all NV vectors of a lane are in flight
  // together; loads under the per-lane `e < S` would each be waited for
  // before the next iteration's loads issue.
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int e = 4 * (lane + kWave * i);
    const bool ok = e < S;
    const int ec = ok ? e : 0;
    const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const float4 wl = nt_load4(master + base + ec);
    const float4 gl = load_grad4<GT>(grad + base + ec);
    const float4 w = ok ? wl : z;
    float4 g = ok ? gl : z;
    if constexpr (FASTNORM) {
      const Half4 f = nt_load_h4(fast_in + base + ec);
      const float4 fv = make_float4(bf16_to_f32(f.h[0]), bf16_to_f32(f.h[1]),
                                    bf16_to_f32(f.h[2]), bf16_to_f32(f.h[3]));
      ss_old += sumsq4(ok ? fv : z);
    } else {
      ss_old += sumsq4(w);
    }
    if constexpr (MOM) {
      const float4 ml = nt_load4(mom_in + base + ec);
      const float4 m = ok ? ml : z;
      g.x = g.x + m.x * mc;
      g.y = g.y + m.y * mc;
      g.z = g.z + m.z * mc;
      g.w = g.w + m.w * mc;
      if (ok) nt_store4(mom_out + base + e, g);
    }
    u[i].x = w.x + g.x * lr_scale;
    u[i].y = w.y + g.y * lr_scale;
    u[i].z = w.z + g.z * lr_scale;
    u[i].w = w.w + g.w * lr_scale;
    ss_new += sumsq4(u[i]);
  }
  const float nu = sqrtf(wave_sum(ss_old));
  const float den = sqrtf(wave_sum(ss_new)) + 1e-5f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int e = 4 * (lane + kWave * i);
    if (e < S) {
      float4 p;
      p.x = u[i].x / den * nu;
      p.y = u[i].y / den * nu;
      p.z = u[i].z / den * nu;
      p.w = u[i].w / den * nu;
      nt_store4(master_out + base + e, renorm_master ? p : u[i]);
      Half4 f;
      f.h[0] = f32_to_bf16(p.x);
      f.h[1] = f32_to_bf16(p.y);
      f.h[2] = f32_to_bf16(p.z);
      f.h[3] = f32_to_bf16(p.w);
      nt_store_h4(fast_out + base + e, f);
    }
  }
}

// Unit-row write: U = master + grad (one fp32 add), master_out = U and
// fast_out = bf16(U / max(|U|, 1e-5)), the clamped divide of F.normalize.
// Rows are addressed by group, row r of group g at g * group_stride + r * C
// (per tensor), so the w0 and w2 halves of a packed [B, E, 2I, D] tensor are
// read and written in place as B*E groups of I rows.  One wave per row, as in
// write_step_kernel; master_out may alias master (same strides).
template <class GT, int NV>
__global__ __launch_bounds__(kWS) void write_unit_rows_kernel(
    const float* master, int64_t master_gs, const typename GT::S* __restrict__ grad,
    int64_t grad_gs, int64_t nrows, int R, int C, float* master_out, int64_t master_out_gs,
    uint16_t* __restrict__ fast_out, int64_t fast_gs) {
#pragma clang fp contract(off)
  const int64_t row = (int64_t)blockIdx.x * (kWS / kWave) + threadIdx.x / kWave;
  if (row >= nrows) return;  // whole wave leaves together
  const int lane = lane_id();
  const int64_t g = row / R, r = row - g * R;
  const float* w_row = master + g * master_gs + r * C;
  const typename GT::S* g_row = grad + g * grad_gs + r * C;
  float4 u[NV];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int e = 4 * (lane + kWave * i);
    const bool ok = e < C;
    const int ec = ok ? e : 0;
    const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const float4 wl = nt_load4(w_row + ec);
    const float4 gl = load_grad4<GT>(g_row + ec);
    const float4 w = ok ? wl : z;
    const float4 gv = ok ? gl : z;
    u[i] = make_float4(w.x + gv.x, w.y + gv.y, w.z + gv.z, w.w + gv.w);
    ss += sumsq4(u[i]);
  }
  const float nrm = sqrtf(wave_sum(ss));
  const float den = nrm < 1e-5f ? 1e-5f : nrm;  // clamp_min: a NaN norm stays NaN
  float* mo_row = master_out + g * master_out_gs + r * C;
  uint16_t* f_row = fast_out + g * fast_gs + r * C;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int e = 4 * (lane + kWave * i);
    if (e < C) {
      nt_store4(mo_row + e, u[i]);
      Half4 f;
      f.h[0] = f32_to_bf16(u[i].x / den);
      f.h[1] = f32_to_bf16(u[i].y / den);
      f.h[2] = f32_to_bf16(u[i].z / den);
      f.h[3] = f32_to_bf16(u[i].w / den);
      nt_store_h4(f_row + e, f);
    }
  }
}

// Prenorm write of the single-layer LaCT (prenorm_block_causal_lact_swiglu,
// uttt_nvs/models/kernels/ttt_operation.py:217-367): U = main + grad (one fp32
// add: the step carries its learning rates), main_out = U and
// fast_out = bf16(U / (|U| + 1e-5) * nu) with nu = norms[row], the row norm
// captured once at the start of the sequence (ttt_operation.py:258-260), so
// every chunk's weights are projected back onto the same norms
// (ttt_operation.py:351-353).  One wave per row, as write_step_kernel; main_out
// may alias main.
template <class GT, int NV>
__global__ __launch_bounds__(kWS) void write_prenorm_kernel(
    const float* main_w, const typename GT::S* __restrict__ grad,
    const float* __restrict__ norms, int64_t nrows, int C, float* main_out,
    uint16_t* __restrict__ fast_out) {
#pragma clang fp contract(off)
  const int64_t row = (int64_t)blockIdx.x * (kWS / kWave) + threadIdx.x / kWave;
  if (row >= nrows) return;  // whole wave leaves together
  const int lane = lane_id();
  const int64_t base = row * C;
  const float nu = norms[row];
  float4 u[NV];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int e = 4 * (lane + kWave * i);
    const bool ok = e < C;
    const int ec = ok ? e : 0;
    const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const float4 wl = nt_load4(main_w + base + ec);
    const float4 gl = load_grad4<GT>(grad + base + ec);
    const float4 w = ok ? wl : z;
    const float4 g = ok ? gl : z;
    u[i] = make_float4(w.x + g.x, w.y + g.y, w.z + g.z, w.w + g.w);
    ss += sumsq4(u[i]);
  }
  const float den = sqrtf(wave_sum(ss)) + 1e-5f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int e = 4 * (lane + kWave * i);
    if (e < C) {
      nt_store4(main_out + base + e, u[i]);
      Half4 f;
      f.h[0] = f32_to_bf16(u[i].x / den * nu);
      f.h[1] = f32_to_bf16(u[i].y / den * nu);
      f.h[2] = f32_to_bf16(u[i].z / den * nu);
      f.h[3] = f32_to_bf16(u[i].w / den * nu);
      nt_store_h4(fast_out + base + e, f);
    }
  }
}

// norms[row] = |row| in fp32 (the sequence-start norms of the prenorm write).
template <class TT, int NV>
__global__ __launch_bounds__(kWS) void row_norms_kernel(const typename TT::S* __restrict__ w,
                                                        int64_t nrows, int C,
                                                        float* __restrict__ norms) {
  const int64_t row = (int64_t)blockIdx.x * (kWS / kWave) + threadIdx.x / kWave;
  if (row >= nrows) return;
  const int lane = lane_id();
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int e = 4 * (lane + kWave * i);
    const bool ok = e < C;
    const float4 v = load_grad4<TT>(w + row * C + (ok ? e : 0));
    ss += ok ? sumsq4(v) : 0.0f;
  }
  ss = wave_sum(ss);
  if (lane == 0) norms[row] = sqrtf(ss);
}

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// out = raw + m_coeff[b] * mom (fp32, the product rounded before the sum as the
// reference's separate tensor ops do): the momentum step on its own, for the
// Muon write, where the orthogonalisation sits between it and the write.
template <class TT>
__global__ __launch_bounds__(256) void momentum_add_kernel(const typename TT::S* __restrict__ raw,
                                                           const float* __restrict__ mom,
                                                           const float* __restrict__ m_coeff,
                                                           int64_t per_batch, int64_t total,
                                                           float* __restrict__ out) {
#pragma clang fp contract(off)
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const float c = m_coeff[i / per_batch];
  const float p = __builtin_nontemporal_load(mom + i) * c;
  __builtin_nontemporal_store(TT::load(__builtin_nontemporal_load(raw + i)) + p, out + i);
}

}  // namespace
}  // namespace uttt

using namespace uttt;

extern "C" int uttt_write_step(const float* master, const void* fast_in, const void* grad,
                               int grad_dtype, const float* mom_in, const float* m_coeff,
                               float lr_scale, int B, int64_t rows_per_batch, int C, int seg,
                               int norm_from_fast, int renorm_master, float* master_out,
                               void* fast_out, float* mom_out, void* stream) {
  UTTT_REQUIRE(B >= 0 && rows_per_batch >= 0 && C >= 0, "write_step: bad sizes");
  UTTT_REQUIRE(seg > 0 && seg % 4 == 0 && seg <= 4096 && C % seg == 0,
               "write_step: segment %d must be a multiple of 4, at most 4096, and divide C=%d",
               seg, C);
  UTTT_REQUIRE(grad_dtype == UTTT_F32 || grad_dtype == UTTT_BF16 || grad_dtype == UTTT_F16,
               "write_step: unsupported grad dtype %d", grad_dtype);
  UTTT_REQUIRE((mom_in == nullptr) == (mom_out == nullptr) &&
                   (mom_in == nullptr || m_coeff != nullptr),
               "write_step: momentum needs mom_in, mom_out and m_coeff together");
  UTTT_REQUIRE(!norm_from_fast || fast_in != nullptr, "write_step: norm_from_fast needs fast_in");
  const int64_t nseg = (int64_t)B * rows_per_batch * (C / seg);
  if (nseg == 0) return UTTT_OK;
  UTTT_REQUIRE(master && grad && master_out && fast_out, "write_step: null tensor");
  UTTT_REQUIRE(aligned(master, 16) && aligned(master_out, 16) && aligned(mom_in, 16) &&
                   aligned(mom_out, 16) && aligned(fast_out, 8) && aligned(fast_in, 8) &&
                   aligned(grad, dtype_bytes(grad_dtype) * 4),
               "write_step: tensors must be 16-byte (fp32) / 8-byte (bf16) aligned");
  const int64_t seg_per_batch = rows_per_batch * (C / seg);
  // the launch needs grid * 256 < 2^32 threads
  UTTT_REQUIRE(nseg < (1ll << 26), "write_step: %lld segments exceed one launch", (long long)nseg);
  const unsigned grid = (unsigned)((nseg + kWS / kWave - 1) / (kWS / kWave));
  hipStream_t st = as_stream(stream);
  const int nv = (seg + 4 * kWave - 1) / (4 * kWave);
  const int nvp = nv <= 1 ? 1 : nv <= 2 ? 2 : nv <= 4 ? 4 : nv <= 8 ? 8 : nv <= 12 ? 12 : 16;
  const bool mom = mom_in != nullptr;
  const auto* fin = reinterpret_cast<const uint16_t*>(fast_in);
  auto* fout = reinterpret_cast<uint16_t*>(fast_out);
#define UTTT_WS_LAUNCH(NV, MOM, FN)                                                              \
  hipLaunchKernelGGL((write_step_kernel<TT, NV, MOM, FN>), dim3(grid), dim3(kWS), 0, st, master, \
                     fin, reinterpret_cast<const typename TT::S*>(grad), mom_in, m_coeff,        \
                     lr_scale, nseg, seg_per_batch, seg, renorm_master, master_out, fout, mom_out)
#define UTTT_WS_FLAGS(NV)                                     \
  do {                                                        \
    if (mom) {                                                \
      if (norm_from_fast) UTTT_WS_LAUNCH(NV, true, true);     \
      else UTTT_WS_LAUNCH(NV, true, false);                   \
    } else {                                                  \
      if (norm_from_fast) UTTT_WS_LAUNCH(NV, false, true);    \
      else UTTT_WS_LAUNCH(NV, false, false);                  \
    }                                                         \
  } while (0)
  UTTT_DTYPE_SWITCH_LR(grad_dtype, TT, {
    switch (nvp) {
      case 1: UTTT_WS_FLAGS(1); break;
      case 2: UTTT_WS_FLAGS(2); break;
      case 4: UTTT_WS_FLAGS(4); break;
      case 8: UTTT_WS_FLAGS(8); break;
      case 12: UTTT_WS_FLAGS(12); break;
      default: UTTT_WS_FLAGS(16); break;
    }
  });
#undef UTTT_WS_FLAGS
#undef UTTT_WS_LAUNCH
  return check_launch("write_step");
}

extern "C" int uttt_momentum_add(const void* raw, int raw_dtype, const float* mom,
                                 const float* m_coeff, int B, int64_t per_batch, float* out,
                                 void* stream) {
  UTTT_REQUIRE(B >= 0 && per_batch >= 0, "momentum_add: bad sizes");
  const int64_t total = (int64_t)B * per_batch;
  if (total == 0) return UTTT_OK;
  UTTT_REQUIRE(raw && mom && m_coeff && out, "momentum_add: null pointer");
  UTTT_REQUIRE(raw_dtype == UTTT_F32 || raw_dtype == UTTT_BF16,
               "momentum_add: the update must be fp32 or bf16 (code %d)", raw_dtype);
  const int64_t blocks = (total + 255) / 256;
  UTTT_REQUIRE(blocks <= 0x7fffffffLL, "momentum_add: too many elements for one launch");
  hipStream_t st = as_stream(stream);
  UTTT_DTYPE_SWITCH_LR(raw_dtype, TT, {
    hipLaunchKernelGGL((momentum_add_kernel<TT>), dim3((unsigned)blocks), dim3(256), 0, st,
                       static_cast<const typename TT::S*>(raw), mom, m_coeff, per_batch, total,
                       out);
  });
  return check_launch("momentum_add");
}

extern "C" int uttt_write_unit_rows(const float* master, int64_t master_gs, const void* grad,
                                    int grad_dtype, int64_t grad_gs, int64_t groups, int R, int C,
                                    float* master_out, int64_t master_out_gs, void* fast_out,
                                    int64_t fast_gs, void* stream) {
  UTTT_REQUIRE(groups >= 0 && R >= 0 && C >= 0, "write_unit_rows: bad sizes");
  UTTT_REQUIRE(C % 4 == 0 && C <= 4096,
               "write_unit_rows: rows of %d elements (must be a multiple of 4, at most 4096)", C);
  UTTT_REQUIRE(grad_dtype == UTTT_F32 || grad_dtype == UTTT_BF16 || grad_dtype == UTTT_F16,
               "write_unit_rows: unsupported grad dtype %d", grad_dtype);
  const int64_t nrows = groups * R;
  if (nrows == 0 || C == 0) return UTTT_OK;
  UTTT_REQUIRE(master && grad && master_out && fast_out, "write_unit_rows: null tensor");
  const int64_t rc = (int64_t)R * C;
  UTTT_REQUIRE(master_gs >= rc && grad_gs >= rc && master_out_gs >= rc && fast_gs >= rc &&
                   master_gs % 4 == 0 && grad_gs % 4 == 0 && master_out_gs % 4 == 0 &&
                   fast_gs % 4 == 0,
               "write_unit_rows: group strides must hold R*C elements and be multiples of 4");
  UTTT_REQUIRE(aligned(master, 16) && aligned(master_out, 16) && aligned(fast_out, 8) &&
                   aligned(grad, dtype_bytes(grad_dtype) * 4),
               "write_unit_rows: tensors must be 16-byte (fp32) / 8-byte (bf16) aligned");
  UTTT_REQUIRE(nrows < (1ll << 26), "write_unit_rows: %lld rows exceed one launch",
               (long long)nrows);
  const unsigned grid = (unsigned)((nrows + kWS / kWave - 1) / (kWS / kWave));
  hipStream_t st = as_stream(stream);
  const int nv = (C + 4 * kWave - 1) / (4 * kWave);
  const int nvp = nv <= 1 ? 1 : nv <= 2 ? 2 : nv <= 4 ? 4 : nv <= 8 ? 8 : nv <= 12 ? 12 : 16;
  auto* fout = reinterpret_cast<uint16_t*>(fast_out);
#define UTTT_WU_LAUNCH(NV)                                                                       \
  hipLaunchKernelGGL((write_unit_rows_kernel<TT, NV>), dim3(grid), dim3(kWS), 0, st, master,     \
                     master_gs, reinterpret_cast<const typename TT::S*>(grad), grad_gs, nrows, R, \
                     C, master_out, master_out_gs, fout, fast_gs)
  UTTT_DTYPE_SWITCH_LR(grad_dtype, TT, {
    switch (nvp) {
      case 1: UTTT_WU_LAUNCH(1); break;
      case 2: UTTT_WU_LAUNCH(2); break;
      case 4: UTTT_WU_LAUNCH(4); break;
      case 8: UTTT_WU_LAUNCH(8); break;
      case 12: UTTT_WU_LAUNCH(12); break;
      default: UTTT_WU_LAUNCH(16); break;
    }
  });
#undef UTTT_WU_LAUNCH
  return check_launch("write_unit_rows");
}

// NV = vectors of 4 per lane: C <= 256 * NV
#define UTTT_NV_SWITCH(C, NV, ...)                                   \
  if ((C) <= 256) { constexpr int NV = 1; __VA_ARGS__; }             \
  else if ((C) <= 1024) { constexpr int NV = 4; __VA_ARGS__; }       \
  else if ((C) <= 2048) { constexpr int NV = 8; __VA_ARGS__; }       \
  else { constexpr int NV = 16; __VA_ARGS__; }

extern "C" int uttt_row_norms(const void* w, int dtype, int64_t rows, int C, float* norms,
                              void* stream) {
  UTTT_REQUIRE(rows >= 0 && C >= 0, "row_norms: bad sizes");
  if (rows == 0) return UTTT_OK;
  UTTT_REQUIRE(w && norms, "row_norms: null pointer");
  UTTT_REQUIRE(C % 4 == 0 && C > 0 && C <= 4096,
               "row_norms: rows of %d elements (a multiple of 4, at most 4096)", C);
  UTTT_REQUIRE(aligned(w, 16), "row_norms: w must be 16-byte aligned");
  UTTT_REQUIRE(dtype == UTTT_F32 || dtype == UTTT_BF16 || dtype == UTTT_F16,
               "row_norms: unsupported dtype %d", dtype);
  const int64_t blocks = (rows + kWS / kWave - 1) / (kWS / kWave);
  UTTT_REQUIRE(blocks <= 0x7fffffffLL, "row_norms: too many rows");
  hipStream_t st = as_stream(stream);
  UTTT_DTYPE_SWITCH_LR(dtype, TT, {
    UTTT_NV_SWITCH(C, NV, {
      hipLaunchKernelGGL((row_norms_kernel<TT, NV>), dim3((unsigned)blocks), dim3(kWS), 0, st,
                         static_cast<const typename TT::S*>(w), rows, C, norms);
    });
  });
  return check_launch("row_norms");
}

extern "C" int uttt_write_prenorm(const float* main_w, const void* grad, int grad_dtype,
                                  const float* norms, int64_t rows, int C, float* main_out,
                                  void* fast_out, void* stream) {
  UTTT_REQUIRE(rows >= 0 && C >= 0, "write_prenorm: bad sizes");
  if (rows == 0) return UTTT_OK;
  UTTT_REQUIRE(main_w && grad && norms && main_out && fast_out, "write_prenorm: null pointer");
  UTTT_REQUIRE(C % 4 == 0 && C > 0 && C <= 4096,
               "write_prenorm: rows of %d elements (a multiple of 4, at most 4096)", C);
  UTTT_REQUIRE(aligned(main_w, 16) && aligned(grad, 8) && aligned(main_out, 16) &&
                   aligned(fast_out, 8),
               "write_prenorm: misaligned tensor");
  UTTT_REQUIRE(grad_dtype == UTTT_F32 || grad_dtype == UTTT_BF16 || grad_dtype == UTTT_F16,
               "write_prenorm: unsupported grad dtype %d", grad_dtype);
  const int64_t blocks = (rows + kWS / kWave - 1) / (kWS / kWave);
  UTTT_REQUIRE(blocks <= 0x7fffffffLL, "write_prenorm: too many rows");
  hipStream_t st = as_stream(stream);
  UTTT_DTYPE_SWITCH_LR(grad_dtype, GT, {
    UTTT_NV_SWITCH(C, NV, {
      hipLaunchKernelGGL((write_prenorm_kernel<GT, NV>), dim3((unsigned)blocks), dim3(kWS), 0, st,
                         main_w, static_cast<const typename GT::S*>(grad), norms, rows, C,
                         main_out, static_cast<uint16_t*>(fast_out));
    });
  });
  return check_launch("write_prenorm");
}
