// Second-order SwiGLU pointwise pass of the UPDATE backward, as a standalone
// HBM-bound kernel for the kernel-level compat function.
//
// reference: triton_swiglu_bwd_bwd_fused_cat_inp_out /
//   ref_pytorch_swiglu_bwd_bwd_fused_cat_inp_out,
//   uttt_llm/flame/custom_models/uttt_moe/lact_moe_triton/triton_pointwise_kernels.py:240-436
//
// For the first-order map of the UPDATE (per element, s = sigmoid(x0),
// silu = x0 s, m = s (1 + x0 (1 - s))):
//   dx0 = lr0 dh x2 m,  dx2 = lr2 dh silu,  hidden_lr1 = lr1 x2 silu,
// this pass returns those three values and the vector-Jacobian product with
// the cotangents (grad_dx0, grad_dx2, grad_hidden_lr1): grad_dh, grad_x0,
// grad_x2 per element and grad_lr0/1/2 summed over the feature rows.  All
// arithmetic is fp32; element outputs are rounded once to the activations'
// dtype, the lr gradients to the lrs' dtype.
//
// Layout [B, rows, L] with L (tokens) contiguous.  Thread = one token column;
// a workgroup covers 256 columns x 64 rows, so the lr sums are formed as
// per-chunk partials and reduced in chunk order by a second launch
// (deterministic, no atomics).  The fused UPDATE backward does not use this
// pass: there the same math runs in the GEMM epilogue.
#include "common.h"

namespace uttt {
namespace {

constexpr int kPwThreads = 256;
constexpr int kPwRows = 64;

template <class XT, class LT>
__global__ __launch_bounds__(kPwThreads) void swiglu_bwd_bwd_kernel(
    const typename XT::S* __restrict__ dh, const typename XT::S* __restrict__ x0x2,
    const typename LT::S* __restrict__ lr0, const typename LT::S* __restrict__ lr1,
    const typename LT::S* __restrict__ lr2, const typename XT::S* __restrict__ gdx,
    const typename XT::S* __restrict__ ghl, int B, int D, int L, int nchunk,
    typename XT::S* __restrict__ g_dh, typename XT::S* __restrict__ g_x, float* __restrict__ part,
    typename XT::S* __restrict__ dx, typename XT::S* __restrict__ hl) {
  const int l = blockIdx.x * kPwThreads + threadIdx.x;
  const int chunk = blockIdx.y, b = blockIdx.z;
  if (l >= L) return;
  const float l0 = LT::load(lr0[(int64_t)b * L + l]);
  const float l1 = LT::load(lr1[(int64_t)b * L + l]);
  const float l2 = LT::load(lr2[(int64_t)b * L + l]);
  const int d0 = chunk * kPwRows, d1 = min(D, d0 + kPwRows);
  const int64_t base1 = (int64_t)b * D * L + l;        // [B, D, L] tensors
  const int64_t base2 = (int64_t)b * 2 * D * L + l;    // [B, 2D, L] tensors
  float p0 = 0.0f, p1 = 0.0f, p2 = 0.0f;
  for (int d = d0; d < d1; ++d) {
    const int64_t i1 = base1 + (int64_t)d * L;
    const int64_t i0 = base2 + (int64_t)d * L, i2 = base2 + (int64_t)(d + D) * L;
    const float h = XT::load(dh[i1]);
    const float x0 = XT::load(x0x2[i0]), x2 = XT::load(x0x2[i2]);
    const float g0 = XT::load(gdx[i0]), g2 = XT::load(gdx[i2]);
    const float gh = XT::load(ghl[i1]);
    const float s = 1.0f / (1.0f + __expf(-x0));
    const float silu = x0 * s;
    const float m = s * (1.0f + x0 * (1.0f - s));
    const float ds = s * (1.0f - s);
    const float a0 = g0 * l0, a2 = g2 * l2, a1 = gh * l1;
    g_dh[i1] = XT::store(a0 * x2 * m + a2 * silu);
    g_x[i2] = XT::store(a0 * h * m + a1 * silu);
    // d m / d x0 = s (1 - s) (2 + x0 (1 - 2 s))
    g_x[i0] = XT::store((a2 * h + a1 * x2) * m + a0 * h * x2 * ds * (2.0f + x0 * (1.0f - 2.0f * s)));
    p0 += g0 * h * x2 * m;
    p1 += gh * x2 * silu;
    p2 += g2 * h * silu;
    dx[i0] = XT::store(h * x2 * m * l0);
    dx[i2] = XT::store(silu * h * l2);
    hl[i1] = XT::store(l1 * x2 * silu);
  }
  const int64_t pb = ((int64_t)b * nchunk + chunk) * L + l;
  const int64_t pj = (int64_t)B * nchunk * L;
  part[pb] = p0;
  part[pb + pj] = p1;
  part[pb + 2 * pj] = p2;
}

template <class LT>
__global__ __launch_bounds__(kPwThreads) void swiglu_lr_reduce_kernel(
    const float* __restrict__ part, int B, int L, int nchunk, typename LT::S* __restrict__ o0,
    typename LT::S* __restrict__ o1, typename LT::S* __restrict__ o2) {
  const int l = blockIdx.x * kPwThreads + threadIdx.x;
  const int b = blockIdx.y;
  if (l >= L) return;
  const int64_t pj = (int64_t)B * nchunk * L;
  typename LT::S* outs[3] = {o0, o1, o2};
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    float acc = 0.0f;
    for (int c = 0; c < nchunk; ++c) acc += part[j * pj + ((int64_t)b * nchunk + c) * L + l];
    outs[j][(int64_t)b * L + l] = LT::store(acc);
  }
}

inline int pw_chunks(int D) { return (D + kPwRows - 1) / kPwRows; }

}  // namespace
}  // namespace uttt

using namespace uttt;

extern "C" size_t uttt_swiglu_bwd_bwd_workspace_bytes(int B, int D, int L) {
  if (B <= 0 || D <= 0 || L <= 0) return 0;
  return sizeof(float) * 3 * (size_t)B * pw_chunks(D) * L;
}

extern "C" int uttt_swiglu_bwd_bwd(const void* dh, const void* x0_x2, int x_dtype, const void* lr0,
                                   const void* lr1, const void* lr2, int lr_dtype,
                                   const void* grad_dx0_dx2, const void* grad_hidden_lr1, int B,
                                   int D, int L, void* grad_dh, void* grad_x0_x2, void* grad_lr0,
                                   void* grad_lr1, void* grad_lr2, void* dx0_x2, void* hidden_lr1,
                                   void* workspace, size_t workspace_bytes, void* stream) {
  UTTT_REQUIRE(B >= 0 && D >= 0 && L >= 0, "swiglu_bwd_bwd: bad sizes");
  if (B == 0 || L == 0) return UTTT_OK;
  UTTT_REQUIRE(D > 0, "swiglu_bwd_bwd: D must be positive");
  UTTT_REQUIRE(B <= 65535, "swiglu_bwd_bwd: B=%d exceeds one launch", B);
  const size_t need = uttt_swiglu_bwd_bwd_workspace_bytes(B, D, L);
  UTTT_REQUIRE(workspace != nullptr && workspace_bytes >= need,
               "swiglu_bwd_bwd: workspace %zu < %zu bytes", workspace_bytes, need);
  UTTT_REQUIRE(dh && x0_x2 && lr0 && lr1 && lr2 && grad_dx0_dx2 && grad_hidden_lr1 && grad_dh &&
                   grad_x0_x2 && grad_lr0 && grad_lr1 && grad_lr2 && dx0_x2 && hidden_lr1,
               "swiglu_bwd_bwd: null pointer");
  const int nchunk = pw_chunks(D);
  hipStream_t st = as_stream(stream);
  const dim3 grid((L + kPwThreads - 1) / kPwThreads, nchunk, B);
  float* part = static_cast<float*>(workspace);
  UTTT_DTYPE_SWITCH_LR(x_dtype, XT, {
    using S = typename XT::S;
    UTTT_DTYPE_SWITCH_LR(lr_dtype, LT, {
      using R = typename LT::S;
      hipLaunchKernelGGL((swiglu_bwd_bwd_kernel<XT, LT>), grid, dim3(kPwThreads), 0, st,
                         static_cast<const S*>(dh), static_cast<const S*>(x0_x2),
                         static_cast<const R*>(lr0), static_cast<const R*>(lr1),
                         static_cast<const R*>(lr2), static_cast<const S*>(grad_dx0_dx2),
                         static_cast<const S*>(grad_hidden_lr1), B, D, L, nchunk,
                         static_cast<S*>(grad_dh), static_cast<S*>(grad_x0_x2), part,
                         static_cast<S*>(dx0_x2), static_cast<S*>(hidden_lr1));
      hipLaunchKernelGGL((swiglu_lr_reduce_kernel<LT>), dim3((L + kPwThreads - 1) / kPwThreads, B),
                         dim3(kPwThreads), 0, st, part, B, L, nchunk, static_cast<R*>(grad_lr0),
                         static_cast<R*>(grad_lr1), static_cast<R*>(grad_lr2));
    });
  });
  return check_launch("swiglu_bwd_bwd");
}
