// MoE router for gfx950: selection scores, balance probabilities, top-k mask,
// combine weights, group sizes and the load-balancing loss.
//
// reference: create_router_mask_sizes_probs,
//   uttt_llm/flame/custom_models/uttt_moe/moe_routing.py:7-75, and the logits
//   of FastWeightMLPSubNN._route_tokens,
//   uttt_llm/flame/custom_models/uttt_moe/modeling_recurrent_lact.py:147-169
//   (logits = R x^T in fp32).
//
// Per token t of batch b, over the E experts (all fp32):
//   softmax      : sel = l;                      bal = softmax(sel)
//   norm_softmax : z = l / max(|l|, eps);        sel = z * scale; bal = softmax(sel)
//   norm_relu    : sel = relu(z) * scale;  S = sum sel;
//                  bal = S > 0 ? sel / max(S, 1e-9) : 1 / E
//   mask = top-k of (sel + bias) (equal scores: the lower expert index first)
//   combine = bal * alpha                                   (selected_prob)
//           | bal * mask / max(sum bal * mask, 1e-9) * alpha (topk_renorm)
//   group_sizes[b, e] = sum_t mask;  lb_loss = E * sum_e mean_bt(bal) * freq_e,
//   freq_e = mean_b(group_sizes) / sum_e mean_b(group_sizes).
//
// Kernels:
//   router_select_kernel : one thread per token, logits given ([B,E,T] strided);
//   router_fused_kernel  : 32 tokens per workgroup, logits = R x^T accumulated
//                          in fp32 from LDS tiles of x and R (D in steps of
//                          64), then the same per-token selection;
//   router_finalize_kernel: one workgroup sums the per-block expert partials
//                          in block order (deterministic: no atomics) into
//                          group_sizes and lb_loss.
#include "common.h"

namespace uttt {
namespace {

constexpr int kRT = 256;       // threads per workgroup
constexpr int kFTok = 32;      // fused kernel: tokens per workgroup
constexpr int kFD = 64;        // fused kernel: D step
constexpr int kMaxE = 128;

struct SelectArgs {
  const float* bias;
  int64_t bias_sb;
  int B, E, T, topk, router_type, combine_mode;
  float alpha, scale, norm_eps;
  uint8_t* mask;      // [B, E, T]
  float* combine;     // [B, E, T]
  float* balance;     // [B, E, T]
  float* part_bal;    // [B, nblk, E]
  int32_t* part_cnt;  // [B, nblk, E]
  int nblk;
};

__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
  for (int d = kWave / 2; d > 0; d >>= 1) v += __shfl_xor(v, d, kWave);
  return v;
}
__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int d = kWave / 2; d > 0; d >>= 1) v += __shfl_xor(v, d, kWave);
  return v;
}

template <int EB>
using MaskBits = uint32_t[(EB + 31) / 32];

template <int EB>
__device__ __forceinline__ bool bit(const MaskBits<EB>& m, int e) {
  return (m[e >> 5] >> (e & 31)) & 1u;
}

// Selection for one token whose E logits are in v[] (overwritten with the
// routing scores); `live` false for padding lanes past T (they write nothing
// and leave zero balance and an empty mask for the block partials).
template <int EB>
__device__ __forceinline__ void select_token(float (&v)[EB], const SelectArgs& a, int b, int t,
                                             bool live, float (&bal)[EB], MaskBits<EB>& m) {
  const int E = a.E;
  if (a.router_type != 0) {   // v <- selection scores
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < EB; ++e)
      if (e < E) ss += v[e] * v[e];
    const float n = fmaxf(sqrtf(ss), a.norm_eps);
#pragma unroll
    for (int e = 0; e < EB; ++e) {
      const float z = v[e] / n;
      v[e] = (a.router_type == 1 ? z : fmaxf(z, 0.0f)) * a.scale;
    }
  }
  if (a.router_type == 2) {
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < EB; ++e)
      if (e < E) s += v[e];
    const float den = fmaxf(s, 1e-9f);
#pragma unroll
    for (int e = 0; e < EB; ++e) bal[e] = s > 0.0f ? v[e] / den : 1.0f / (float)E;
  } else {
    float mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < EB; ++e)
      if (e < E) mx = fmaxf(mx, v[e]);
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < EB; ++e) {
      bal[e] = e < E ? expf(v[e] - mx) : 0.0f;
      s += bal[e];
    }
#pragma unroll
    for (int e = 0; e < EB; ++e) bal[e] = bal[e] / s;
  }
  // v <- routing scores (selection scores + bias); top-k as k arg-max passes,
  // the lower expert index winning ties
  const float* bias = a.bias != nullptr ? a.bias + (int64_t)b * a.bias_sb : nullptr;
#pragma unroll
  for (int e = 0; e < EB; ++e) v[e] = e < E ? (bias != nullptr ? v[e] + bias[e] : v[e]) : -INFINITY;
#pragma unroll
  for (int w = 0; w < (EB + 31) / 32; ++w) m[w] = 0u;
  for (int j = 0; j < a.topk; ++j) {
    float best = 0.0f;
    int bi = -1;
#pragma unroll
    for (int e = 0; e < EB; ++e) {
      const bool cand = e < E && !bit<EB>(m, e) && (bi < 0 || v[e] > best);
      best = cand ? v[e] : best;
      bi = cand ? e : bi;
    }
#pragma unroll
    for (int w = 0; w < (EB + 31) / 32; ++w)
      if ((bi >> 5) == w) m[w] |= 1u << (bi & 31);
  }
  float rsum = 0.0f;
  if (a.combine_mode == 1) {
#pragma unroll
    for (int e = 0; e < EB; ++e)
      if (bit<EB>(m, e)) rsum += bal[e];
  }
  const float rden = fmaxf(rsum, 1e-9f);
  if (live) {
    const int64_t base = (int64_t)b * E * a.T + t;
#pragma unroll
    for (int e = 0; e < EB; ++e) {
      if (e >= E) break;
      const int64_t i = base + (int64_t)e * a.T;
      const bool on = bit<EB>(m, e);
      a.mask[i] = on ? 1 : 0;
      a.balance[i] = bal[e];
      const float c = a.combine_mode == 1 ? (on ? bal[e] : 0.0f) / rden : bal[e];
      a.combine[i] = c * a.alpha;
    }
  } else {
#pragma unroll
    for (int e = 0; e < EB; ++e) bal[e] = 0.0f;
#pragma unroll
    for (int w = 0; w < (EB + 31) / 32; ++w) m[w] = 0u;
  }
}

// Per-expert sums over the tokens of the first `nwaves` waves into
// part[b][blk][e] (wave sums in LDS, then added in wave order).
template <int EB>
__device__ __forceinline__ void block_partials(const float (&bal)[EB], const MaskBits<EB>& m,
                                               const SelectArgs& a, int b, int blk, int nwaves,
                                               float* s_bal, int* s_cnt) {
  const int w = threadIdx.x / kWave, lane = lane_id();
  if (w < nwaves) {
#pragma unroll
    for (int e = 0; e < EB; ++e) {
      if (e >= a.E) break;
      const float sb = wave_sum_f(bal[e]);
      const int sc = wave_sum_i(bit<EB>(m, e) ? 1 : 0);
      if (lane == 0) {
        s_bal[w * kMaxE + e] = sb;
        s_cnt[w * kMaxE + e] = sc;
      }
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < a.E; e += kRT) {
    float sb = 0.0f;
    int sc = 0;
    for (int i = 0; i < nwaves; ++i) {
      sb += s_bal[i * kMaxE + e];
      sc += s_cnt[i * kMaxE + e];
    }
    const int64_t o = ((int64_t)b * a.nblk + blk) * a.E + e;
    a.part_bal[o] = sb;
    a.part_cnt[o] = sc;
  }
}

template <int EB>
__global__ __launch_bounds__(kRT) void router_select_kernel(const float* __restrict__ logits,
                                                            int64_t l_sb, int64_t l_se,
                                                            int64_t l_st, SelectArgs a) {
  __shared__ float s_bal[(kRT / kWave) * kMaxE];
  __shared__ int s_cnt[(kRT / kWave) * kMaxE];
  const int blk = blockIdx.x, b = blockIdx.y;
  const int t = blk * kRT + threadIdx.x;
  const bool live = t < a.T;
  const int tt = live ? t : a.T - 1;
  float l[EB];
#pragma unroll
  for (int e = 0; e < EB; ++e)
    l[e] = e < a.E ? logits[(int64_t)b * l_sb + (int64_t)e * l_se + (int64_t)tt * l_st] : 0.0f;
  float bal[EB];
  MaskBits<EB> m;
  select_token<EB>(l, a, b, t, live, bal, m);
  block_partials<EB>(bal, m, a, b, blk, kRT / kWave, s_bal, s_cnt);
}

template <class XT, int EB>
__global__ __launch_bounds__(kRT) void router_fused_kernel(
    const typename XT::S* __restrict__ x, const float* __restrict__ rw, int64_t w_sb, int D,
    float* __restrict__ logits_out, SelectArgs a) {
  using S = typename XT::S;
  constexpr int kGroups = kRT / kFTok;          // 8 expert groups
  constexpr int kPer = (EB + kGroups - 1) / kGroups;
  __shared__ float xs[kFTok][kFD + 1];
  __shared__ float ws[EB][kFD + 1];
  __shared__ float lg[kFTok][EB + 1];
  __shared__ float s_bal[(kRT / kWave) * kMaxE];
  __shared__ int s_cnt[(kRT / kWave) * kMaxE];
  const int blk = blockIdx.x, b = blockIdx.y;
  const int t0 = blk * kFTok;
  const int tok = threadIdx.x % kFTok, grp = threadIdx.x / kFTok;
  const int E = a.E;
  const float* R = rw + (int64_t)b * w_sb;
  float acc[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j) acc[j] = 0.0f;
  for (int d0 = 0; d0 < D; d0 += kFD) {
    // stage x[t0 .. t0+32)[d0 .. d0+64) and R[0 .. E)[d0 .. d0+64) as fp32
    for (int i = threadIdx.x; i < kFTok * kFD; i += kRT) {
      const int r = i / kFD, c = i % kFD;
      const int t = t0 + r, d = d0 + c;
      xs[r][c] = (t < a.T && d < D) ? XT::load(x[((int64_t)b * a.T + t) * D + d]) : 0.0f;
    }
    for (int i = threadIdx.x; i < EB * kFD; i += kRT) {
      const int r = i / kFD, c = i % kFD;
      const int d = d0 + c;
      ws[r][c] = (r < E && d < D) ? R[(int64_t)r * D + d] : 0.0f;
    }
    __syncthreads();
#pragma unroll 4
    for (int c = 0; c < kFD; ++c) {
      const float xv = xs[tok][c];
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int e = grp + kGroups * j;
        if (e < EB) acc[j] = __builtin_fmaf(ws[e][c], xv, acc[j]);
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int e = grp + kGroups * j;
    if (e < EB) lg[tok][e] = acc[j];
  }
  __syncthreads();
  if (logits_out != nullptr) {
    for (int i = threadIdx.x; i < E * kFTok; i += kRT) {
      const int e = i / kFTok, r = i % kFTok;
      if (t0 + r < a.T) logits_out[((int64_t)b * E + e) * a.T + t0 + r] = lg[r][e];
    }
  }
  float bal[EB];
  MaskBits<EB> m;
  if (threadIdx.x < kWave) {   // wave 0 selects; lanes >= kFTok are padding
    const int t = t0 + threadIdx.x;
    const bool live = threadIdx.x < kFTok && t < a.T;
    float l[EB];
#pragma unroll
    for (int e = 0; e < EB; ++e) l[e] = (threadIdx.x < kFTok && e < E) ? lg[threadIdx.x][e] : 0.0f;
    select_token<EB>(l, a, b, t, live, bal, m);
  }
  block_partials<EB>(bal, m, a, b, blk, 1, s_bal, s_cnt);
}

// One workgroup: group_sizes[b][e] and balance sums over the blocks, then
// lb_loss = E * sum_e (sum_b bal_sum[b][e] / (B T)) * freq_e.
__global__ __launch_bounds__(kRT) void router_finalize_kernel(const float* __restrict__ part_bal,
                                                              const int32_t* __restrict__ part_cnt,
                                                              int B, int E, int T, int nblk,
                                                              int32_t* __restrict__ group_sizes,
                                                              float* __restrict__ lb_loss) {
  __shared__ float pm[kMaxE];
  __shared__ float gm[kMaxE];
  for (int e = threadIdx.x; e < E; e += kRT) {
    float sb = 0.0f, sg = 0.0f;
    for (int b = 0; b < B; ++b) {
      float bb = 0.0f;
      int cc = 0;
      for (int k = 0; k < nblk; ++k) {
        const int64_t o = ((int64_t)b * nblk + k) * E + e;
        bb += part_bal[o];
        cc += part_cnt[o];
      }
      if (group_sizes != nullptr) group_sizes[(int64_t)b * E + e] = cc;
      sb += bb;
      sg += (float)cc;
    }
    pm[e] = sb / ((float)B * (float)T);
    gm[e] = sg / (float)B;
  }
  __syncthreads();
  if (threadIdx.x == 0 && lb_loss != nullptr) {
    float tot = 0.0f;
    for (int e = 0; e < E; ++e) tot += gm[e];
    float lb = 0.0f;
    for (int e = 0; e < E; ++e) lb += pm[e] * (gm[e] / tot);
    *lb_loss = lb * (float)E;
  }
}

inline int e_bucket(int E) { return E <= 8 ? 8 : E <= 16 ? 16 : E <= 32 ? 32 : E <= 64 ? 64 : 128; }

#define UTTT_EB_SWITCH(E, ...)                                     \
  switch (e_bucket(E)) {                                           \
    case 8: { constexpr int EB = 8; __VA_ARGS__; } break;          \
    case 16: { constexpr int EB = 16; __VA_ARGS__; } break;        \
    case 32: { constexpr int EB = 32; __VA_ARGS__; } break;        \
    case 64: { constexpr int EB = 64; __VA_ARGS__; } break;        \
    default: { constexpr int EB = 128; __VA_ARGS__; } break;       \
  }

int check_select_args(int B, int E, int T, int topk, int router_type, int combine_mode,
                      const char* what) {
  UTTT_REQUIRE(B >= 0 && T >= 0 && E >= 1 && E <= kMaxE, "%s: E=%d must be in [1, %d]", what, E,
               kMaxE);
  UTTT_REQUIRE(topk >= 1 && topk <= E, "%s: topk=%d must be in [1, E=%d]", what, topk, E);
  UTTT_REQUIRE(router_type >= 0 && router_type <= 2,
               "%s: router_type %d (0 softmax, 1 norm_softmax, 2 norm_relu)", what, router_type);
  UTTT_REQUIRE(combine_mode == 0 || combine_mode == 1,
               "%s: combine_mode %d (0 selected_prob, 1 topk_renorm)", what, combine_mode);
  UTTT_REQUIRE((int64_t)B * E <= 65535 * 64, "%s: B*E too large", what);
  return UTTT_OK;
}

size_t ws_bytes(int B, int T, int E) {
  const int64_t nblk = (T + kFTok - 1) / kFTok;   // the finer of the two tilings
  return (size_t)(2 * sizeof(float) * B * nblk * E);
}

}  // namespace
}  // namespace uttt

using namespace uttt;

extern "C" size_t uttt_router_workspace_bytes(int B, int T, int E) {
  if (B <= 0 || T <= 0 || E <= 0) return 0;
  return ws_bytes(B, T, E);
}

static int finish_router(float* part_bal, int32_t* part_cnt, int B, int E, int T, int nblk,
                         int32_t* group_sizes, float* lb_loss, hipStream_t st, const char* what) {
  if (int rc = check_launch(what)) return rc;
  hipLaunchKernelGGL(router_finalize_kernel, dim3(1), dim3(kRT), 0, st, part_bal, part_cnt, B, E,
                     T, nblk, group_sizes, lb_loss);
  return check_launch(what);
}

extern "C" int uttt_router_select(const float* logits, int64_t l_sb, int64_t l_se, int64_t l_st,
                                  const float* bias, int64_t bias_sb, int B, int E, int T,
                                  int topk, int router_type, int combine_mode, float alpha,
                                  float router_scale, float norm_eps, void* mask,
                                  int32_t* group_sizes, float* combine, float* balance,
                                  float* lb_loss, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  if (int rc = check_select_args(B, E, T, topk, router_type, combine_mode, "router_select"))
    return rc;
  if (B == 0 || T == 0) return UTTT_OK;
  UTTT_REQUIRE(logits && mask && combine && balance, "router_select: null pointer");
  UTTT_REQUIRE(workspace != nullptr && workspace_bytes >= ws_bytes(B, T, E),
               "router_select: workspace %zu < %zu bytes", workspace_bytes, ws_bytes(B, T, E));
  const int nblk = (T + kRT - 1) / kRT;
  SelectArgs a{bias, bias_sb, B, E, T, topk, router_type, combine_mode, alpha,
               router_scale > 0.0f ? router_scale : sqrtf((float)E), norm_eps,
               static_cast<uint8_t*>(mask), combine, balance,
               static_cast<float*>(workspace),
               reinterpret_cast<int32_t*>(static_cast<float*>(workspace) + (int64_t)B * nblk * E),
               nblk};
  hipStream_t st = as_stream(stream);
  UTTT_EB_SWITCH(E, hipLaunchKernelGGL((router_select_kernel<EB>), dim3(nblk, B), dim3(kRT), 0,
                                       st, logits, l_sb, l_se, l_st, a));
  return finish_router(a.part_bal, a.part_cnt, B, E, T, nblk, group_sizes, lb_loss, st,
                       "router_select");
}

extern "C" int uttt_route_tokens(const void* x, int x_dtype, const float* router_w, int64_t w_sb,
                                 int B, int T, int D, int E, const float* bias, int64_t bias_sb,
                                 int topk, int router_type, int combine_mode, float alpha,
                                 float router_scale, float norm_eps, float* logits_out,
                                 void* mask, int32_t* group_sizes, float* combine,
                                 float* balance, float* lb_loss, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  if (int rc = check_select_args(B, E, T, topk, router_type, combine_mode, "route_tokens"))
    return rc;
  UTTT_REQUIRE(D >= 1, "route_tokens: D=%d", D);
  if (B == 0 || T == 0) return UTTT_OK;
  UTTT_REQUIRE(x && router_w && mask && combine && balance, "route_tokens: null pointer");
  UTTT_REQUIRE(workspace != nullptr && workspace_bytes >= ws_bytes(B, T, E),
               "route_tokens: workspace %zu < %zu bytes", workspace_bytes, ws_bytes(B, T, E));
  const int nblk = (T + kFTok - 1) / kFTok;
  SelectArgs a{bias, bias_sb, B, E, T, topk, router_type, combine_mode, alpha,
               router_scale > 0.0f ? router_scale : sqrtf((float)E), norm_eps,
               static_cast<uint8_t*>(mask), combine, balance,
               static_cast<float*>(workspace),
               reinterpret_cast<int32_t*>(static_cast<float*>(workspace) + (int64_t)B * nblk * E),
               nblk};
  hipStream_t st = as_stream(stream);
  UTTT_DTYPE_SWITCH_LR(x_dtype, XT, {
    using S = typename XT::S;
    UTTT_EB_SWITCH(E, hipLaunchKernelGGL((router_fused_kernel<XT, EB>), dim3(nblk, B), dim3(kRT),
                                         0, st, static_cast<const S*>(x), router_w, w_sb, D,
                                         logits_out, a));
  });
  return finish_router(a.part_bal, a.part_cnt, B, E, T, nblk, group_sizes, lb_loss, st,
                       "route_tokens");
}
