// Loss-free load balancing of the MoE router: the per-expert selection bias
// that the router adds to its scores before top-k, moved one fixed step
// toward the experts that received fewer rows than the mean.
//
// reference: uttt_llm/flame/custom_models/uttt_moe/modeling_recurrent_lact.py
//   _loss_free_counts_for_scope :1646-1654, _store_loss_free_counts :1695-1712
//   (the counts), _maybe_update_loss_free_bias :1662-1693 (the step).
//
// Both kernels are tiny ([L, E] floats) and run as one workgroup, so every
// reduction has one fixed order and the result does not depend on the launch.
// Counts are sums of integer row counts held in fp32 (exact below 2^24).
// Means follow torch's GPU mean: the fp32 sum times the fp32 reciprocal 1/E.
#include "common.h"

namespace uttt {
namespace {

constexpr int kLF = 256;

// Sum of v over the workgroup, in a fixed tree order; every thread gets it.
__device__ float block_sum(float v, float* red) {
  const int t = threadIdx.x;
  red[t] = v;
  __syncthreads();
#pragma unroll
  for (int s = kLF / 2; s > 0; s >>= 1) {
    if (t < s) red[t] = red[t] + red[t + s];
    __syncthreads();
  }
  const float r = red[0];
  __syncthreads();
  return r;
}

// pending[l, e] += sum_b apply[l, b, e] + sum_b update[l, b, e]   (layer scope)
// pending[e]    += sum_l (sum_b apply[l, b, e] + sum_b update[l, b, e])  (pool)
// steps += 1.  The sums run in the reference's order: over b for each
// tensor, the two added, then over l.
__global__ __launch_bounds__(kLF) void store_counts_kernel(const float* __restrict__ apply_f,
                                                           const float* __restrict__ update_f,
                                                           int L, int B, int E, int pool,
                                                           float* pending, long long* steps) {
#pragma clang fp contract(off)
  const int n_out = pool ? E : L * E;
  for (int o = threadIdx.x; o < n_out; o += kLF) {
    const int l0 = pool ? 0 : o / E, l1 = pool ? L : l0 + 1, e = o % E;
    float acc = 0.0f;
    for (int l = l0; l < l1; ++l) {
      float a = 0.0f, u = 0.0f;
      for (int b = 0; b < B; ++b) {
        a = a + apply_f[((int64_t)l * B + b) * E + e];
        u = u + update_f[((int64_t)l * B + b) * E + e];
      }
      acc = l == l0 ? a + u : acc + (a + u);
    }
    pending[o] = pending[o] + acc;
  }
  if (threadIdx.x == 0) steps[0] = steps[0] + 1;
}

// mode 1 (warm-up): counts = 0.  mode 2 (step), for each of `rows` rows of E:
//   bias += rate * sign(mean(counts) - counts);  bias -= mean(bias);
//   clamp to [-bias_max, bias_max] when bias_max >= 0;  counts = 0;
// and num_updates += 1.  Nothing happens when the counts sum to <= 0.
__global__ __launch_bounds__(kLF) void bias_step_kernel(float* bias, float* counts, int rows,
                                                        int E, int mode, float rate, float bias_max,
                                                        long long* num_updates) {
#pragma clang fp contract(off)
  __shared__ float red[kLF];
  const int n = rows * E;
  float part = 0.0f;
  for (int i = threadIdx.x; i < n; i += kLF) part = part + counts[i];
  if (!(block_sum(part, red) > 0.0f)) return;  // uniform: every thread sees the same sum
  if (mode == 2) {
    const float inv_e = 1.0f / (float)E;
    for (int r = 0; r < rows; ++r) {
      float* br = bias + (int64_t)r * E;
      const float* cr = counts + (int64_t)r * E;
      float cs = 0.0f;
      for (int e = threadIdx.x; e < E; e += kLF) cs = cs + cr[e];
      const float target = block_sum(cs, red) * inv_e;
      float bs = 0.0f;
      for (int e = threadIdx.x; e < E; e += kLF) {
        const float d = target - cr[e];
        const float sg = d > 0.0f ? 1.0f : d < 0.0f ? -1.0f : 0.0f;
        const float nb = br[e] + rate * sg;
        br[e] = nb;  // each thread re-reads only its own elements below
        bs = bs + nb;
      }
      const float mean = block_sum(bs, red) * inv_e;
      for (int e = threadIdx.x; e < E; e += kLF) {
        float nb = br[e] - mean;
        if (bias_max >= 0.0f) nb = fminf(fmaxf(nb, -bias_max), bias_max);
        br[e] = nb;
      }
    }
  }
  __syncthreads();  // every count read above happens before any is cleared
  for (int i = threadIdx.x; i < n; i += kLF) counts[i] = 0.0f;
  if (mode == 2 && threadIdx.x == 0) num_updates[0] = num_updates[0] + 1;
}

}  // namespace
}  // namespace uttt

using namespace uttt;

extern "C" int uttt_loss_free_store_counts(const float* apply_freqs, const float* update_freqs,
                                           int L, int B, int E, int pool, float* pending_counts,
                                           long long* steps, void* stream) {
  UTTT_REQUIRE(L >= 0 && B >= 0 && E >= 0, "loss_free_store_counts: bad sizes");
  UTTT_REQUIRE(steps != nullptr, "loss_free_store_counts: null step counter");
  const int64_t n_out = pool ? (int64_t)E : (int64_t)L * E;
  UTTT_REQUIRE(n_out <= (1 << 24), "loss_free_store_counts: %lld counts exceed one workgroup's loop",
               (long long)n_out);
  UTTT_REQUIRE(n_out == 0 || pending_counts != nullptr, "loss_free_store_counts: null counts");
  UTTT_REQUIRE((int64_t)L * B * E == 0 || (apply_freqs && update_freqs),
               "loss_free_store_counts: null frequencies");
  hipLaunchKernelGGL(store_counts_kernel, dim3(1), dim3(kLF), 0, as_stream(stream), apply_freqs,
                     update_freqs, L, B, E, pool, pending_counts, steps);
  return check_launch("loss_free_store_counts");
}

extern "C" int uttt_loss_free_bias_step(float* bias, float* counts, int rows, int E, int mode,
                                        float rate, float bias_max, long long* num_updates,
                                        void* stream) {
  UTTT_REQUIRE(rows >= 0 && E >= 0, "loss_free_bias_step: bad sizes");
  UTTT_REQUIRE(mode == 1 || mode == 2, "loss_free_bias_step: mode must be 1 (clear) or 2 (step)");
  UTTT_REQUIRE((int64_t)rows * E <= (1 << 24), "loss_free_bias_step: too many counts");
  if ((int64_t)rows * E == 0) return UTTT_OK;
  UTTT_REQUIRE(bias && counts && num_updates, "loss_free_bias_step: null pointer");
  hipLaunchKernelGGL(bias_step_kernel, dim3(1), dim3(kLF), 0, as_stream(stream), bias, counts, rows,
                     E, mode, rate, bias_max, num_updates);
  return check_launch("loss_free_bias_step");
}
