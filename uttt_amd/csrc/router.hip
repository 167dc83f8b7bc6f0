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
//   router_mfma_kernel   : logits = R x^T for 32 tokens x all experts per
//                          workgroup (fp32 matrix cores, the waves splitting
//                          D; for batches of at most 8 tokens the vector ALU,
//                          with no padded rows), then the selection of those
//                          tokens with 32 lanes per token;
//   router_reduce_kernel : one workgroup per (batch, expert) adds the select
//                          blocks' partial counts and balance sums with a
//                          fixed tree (deterministic: no atomics); skipped
//                          when a batch is one block, whose sums are final;
//   router_lb_kernel     : lb_loss from those sums.
#include <type_traits>

#include "common.h"

namespace uttt {
namespace {

constexpr int kRT = 256;       // threads per workgroup
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
  // with one block per batch the block's sums are final and go here directly
  int32_t* group_sizes;  // [B, E] or null
  float* bal_sum;        // [B, E]
  int32_t* cnt_sum;      // [B, E]
};

// Where block blk of batch b leaves its per-expert sums for expert e.
__device__ __forceinline__ void put_partial(const SelectArgs& a, int b, int blk, int e, float s,
                                            int c) {
  if (a.nblk == 1) {
    const int64_t o = (int64_t)b * a.E + e;
    a.bal_sum[o] = s;
    a.cnt_sum[o] = c;
    if (a.group_sizes != nullptr) a.group_sizes[o] = c;
  } else {
    const int64_t o = ((int64_t)b * a.nblk + blk) * a.E + e;
    a.part_bal[o] = s;
    a.part_cnt[o] = c;
  }
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

// Per-expert sums over the block's NTOK tokens into part[b][blk][e]: the
// token holders write their rows (balance, mask bit) to LDS, then thread e
// adds the column in token order (deterministic).  `row` is this thread's
// token row, or -1 for threads that hold none.
template <int EB, int NTOK>
__device__ __forceinline__ void block_partials(const float (&bal)[EB], const MaskBits<EB>& m,
                                               int row, const SelectArgs& a, int b, int blk,
                                               float (*sb)[EB + 1], uint8_t (*sc)[EB + 1]) {
  if (row >= 0) {
#pragma unroll
    for (int e = 0; e < EB; ++e) {
      sb[row][e] = bal[e];
      sc[row][e] = bit<EB>(m, e) ? 1 : 0;
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < a.E; e += blockDim.x) {
    float s = 0.0f;
    int c = 0;
    for (int i = 0; i < NTOK; ++i) {
      s += sb[i][e];
      c += sc[i][e];
    }
    put_partial(a, b, blk, e, s, c);
  }
}

// Selection over given logits (logits[b*l_sb + e*l_se + t*l_st]), one thread
// per token, sel_tpb(EB) tokens per block (the LDS transpose of the partial
// sums stays at 33 KB).
constexpr int sel_tpb(int EB) { return EB <= 32 ? 256 : EB <= 64 ? 128 : 64; }

template <int EB>
__global__ __launch_bounds__(sel_tpb(EB)) void router_select_kernel(const float* __restrict__ logits,
                                                                    int64_t l_sb, int64_t l_se,
                                                                    int64_t l_st, SelectArgs a) {
  constexpr int TPB = sel_tpb(EB);
  __shared__ float sb[TPB][EB + 1];
  __shared__ uint8_t sc[TPB][EB + 1];
  const int blk = blockIdx.x, b = blockIdx.y;
  const int t = blk * TPB + threadIdx.x;
  const bool live = t < a.T;
  const float* p = logits + (int64_t)b * l_sb + (int64_t)(live ? t : a.T - 1) * l_st;
  float l[EB];
#pragma unroll
  for (int e = 0; e < EB; ++e) l[e] = e < a.E ? p[(int64_t)e * l_se] : 0.0f;
  float bal[EB];
  MaskBits<EB> m;
  select_token<EB>(l, a, b, t, live, bal, m);
  block_partials<EB, TPB>(bal, m, threadIdx.x, a, b, blk, sb, sc);
}

typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

// 8 consecutive features of one row as fp32 (zero past D or for a dead row).
template <class XT, bool VEC>
__device__ __forceinline__ void load8(const typename XT::S* p, int d, int D, bool ok,
                                     float (&o)[8]) {
  if constexpr (VEC) {  // D % 8 == 0 and 16-byte aligned rows
    // unconditional load (a lane that is off reads its row's first 8
    // features and zeroes them), so the loads of consecutive calls stay in
    // flight together; a load under a per-lane condition would be waited
    // for where the two paths merge
    const bool in = ok && d + 8 <= D;
    const typename XT::S* q = p + (in ? d : 0);
    float v[8];
    if constexpr (sizeof(typename XT::S) == 4) {
      const float4 u = *reinterpret_cast<const float4*>(q);
      const float4 w = *reinterpret_cast<const float4*>(q + 4);
      v[0] = u.x; v[1] = u.y; v[2] = u.z; v[3] = u.w;
      v[4] = w.x; v[5] = w.y; v[6] = w.z; v[7] = w.w;
    } else {
      const uint4 u = *reinterpret_cast<const uint4*>(q);
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[2 * i] = XT::load(static_cast<typename XT::S>(w[i] & 0xffffu));
        v[2 * i + 1] = XT::load(static_cast<typename XT::S>(w[i] >> 16));
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = in ? v[i] : 0.0f;
    return;
  }
  if (ok && d + 8 <= D && ((reinterpret_cast<uintptr_t>(p + d) & (sizeof(typename XT::S) * 8 - 1)) == 0)) {
    if constexpr (sizeof(typename XT::S) == 4) {
      const float4 u = *reinterpret_cast<const float4*>(p + d);
      const float4 v = *reinterpret_cast<const float4*>(p + d + 4);
      o[0] = u.x; o[1] = u.y; o[2] = u.z; o[3] = u.w;
      o[4] = v.x; o[5] = v.y; o[6] = v.z; o[7] = v.w;
    } else {
      const uint4 u = *reinterpret_cast<const uint4*>(p + d);
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        o[2 * i] = XT::load(static_cast<typename XT::S>(w[i] & 0xffffu));
        o[2 * i + 1] = XT::load(static_cast<typename XT::S>(w[i] >> 16));
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = (ok && d + i < D) ? XT::load(p[d + i]) : 0.0f;
  }
}

// The bytes of 8 consecutive features (16 B for 2-byte types, 32 B for fp32)
// as loaded, converted only where they are used: a load ring of these keeps
// its loads in flight (converting right after the load, as load8 does, waits
// for each load in turn).  Rows of whole 16-byte vectors only (D % 8 == 0,
// aligned); a lane that is off reads its row's first 8 features and `in`
// zeroes them at the conversion.
template <class XT>
struct Raw8 {
  static constexpr int kV = sizeof(typename XT::S) / 2;
  uint4 u[kV];
  bool in;
};

template <class XT>
__device__ __forceinline__ void load_raw8(const typename XT::S* p, int d, int D, bool ok,
                                          Raw8<XT>& r) {
  r.in = ok && d + 8 <= D;
  const uint4* q = reinterpret_cast<const uint4*>(p + (r.in ? d : 0));
#pragma unroll
  for (int i = 0; i < Raw8<XT>::kV; ++i) r.u[i] = q[i];
}

template <class XT>
__device__ __forceinline__ void cvt8(const Raw8<XT>& r, float (&o)[8]) {
  float v[8];
  if constexpr (sizeof(typename XT::S) == 4) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      v[4 * i] = __uint_as_float(r.u[i].x);
      v[4 * i + 1] = __uint_as_float(r.u[i].y);
      v[4 * i + 2] = __uint_as_float(r.u[i].z);
      v[4 * i + 3] = __uint_as_float(r.u[i].w);
    }
  } else {
    const uint32_t w[4] = {r.u[0].x, r.u[0].y, r.u[0].z, r.u[0].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = XT::load(static_cast<typename XT::S>(w[i] & 0xffffu));
      v[2 * i + 1] = XT::load(static_cast<typename XT::S>(w[i] >> 16));
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = r.in ? v[i] : 0.0f;
}

// Reductions over the 32 lanes of a half-wave (fixed xor butterflies).
__device__ __forceinline__ float half_sum(float v) {
#pragma unroll
  for (int o = 16; o >= 1; o >>= 1) v += __shfl_xor(v, o, 32);
  return v;
}
__device__ __forceinline__ float half_max(float v) {
#pragma unroll
  for (int o = 16; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 32));
  return v;
}
// The larger score, equal scores resolved to the lower expert index.
__device__ __forceinline__ void half_argmax(float& v, int& i) {
#pragma unroll
  for (int o = 16; o >= 1; o >>= 1) {
    const float ov = __shfl_xor(v, o, 32);
    const int oi = __shfl_xor(i, o, 32);
    if (ov > v || (ov == v && oi < i)) {
      v = ov;
      i = oi;
    }
  }
}

// The selection of select_token for one token on the 32 lanes of a half-wave:
// lane j holds experts j, j + 32, ... (lg[q] = logit of expert j + 32q).
// Same scores, balance, top-k (k arg-max passes, equal scores to the lower
// expert index) and combine weights; the sums over experts are butterflies.
// Writes the token's mask / balance / combine entries when live, and its row
// of the block partials (zeros when not live).
// bias_v[q]: the routing bias of expert j + 32 q (0 without a bias), loaded
// by the caller ahead of time.
template <int NET>
__device__ __forceinline__ void select_lanes(const float (&lg)[NET], const float (&bias_v)[NET],
                                             const SelectArgs& a, int b, int t, bool live, int j,
                                             float* sb_row, uint8_t* sc_row) {
  const int E = a.E;
  float v[NET];
  bool ok[NET];
#pragma unroll
  for (int q = 0; q < NET; ++q) {
    ok[q] = j + 32 * q < E;
    v[q] = ok[q] ? lg[q] : 0.0f;
  }
  if (a.router_type != 0) {   // v <- selection scores
    float ss = 0.0f;
#pragma unroll
    for (int q = 0; q < NET; ++q) ss += v[q] * v[q];
    const float n = fmaxf(sqrtf(half_sum(ss)), a.norm_eps);
#pragma unroll
    for (int q = 0; q < NET; ++q) {
      const float z = v[q] / n;
      v[q] = ok[q] ? (a.router_type == 1 ? z : fmaxf(z, 0.0f)) * a.scale : 0.0f;
    }
  }
  float bal[NET];
  if (a.router_type == 2) {
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < NET; ++q) s += v[q];
    s = half_sum(s);
    const float den = fmaxf(s, 1e-9f);
#pragma unroll
    for (int q = 0; q < NET; ++q) bal[q] = ok[q] ? (s > 0.0f ? v[q] / den : 1.0f / (float)E) : 0.0f;
  } else {
    float mx = -INFINITY;
#pragma unroll
    for (int q = 0; q < NET; ++q)
      if (ok[q]) mx = fmaxf(mx, v[q]);
    mx = half_max(mx);
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < NET; ++q) {
      bal[q] = ok[q] ? expf(v[q] - mx) : 0.0f;
      s += bal[q];
    }
    s = half_sum(s);
#pragma unroll
    for (int q = 0; q < NET; ++q) bal[q] = bal[q] / s;
  }
  float r[NET];
  bool sel[NET];
#pragma unroll
  for (int q = 0; q < NET; ++q) {
    r[q] = ok[q] ? (a.bias != nullptr ? v[q] + bias_v[q] : v[q]) : -INFINITY;
    sel[q] = false;
  }
  for (int k = 0; k < a.topk; ++k) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;   // no candidate
#pragma unroll
    for (int q = 0; q < NET; ++q) {
      const bool cand = ok[q] && !sel[q] && (bi == 0x7fffffff || r[q] > bv);
      bv = cand ? r[q] : bv;
      bi = cand ? j + 32 * q : bi;
    }
    half_argmax(bv, bi);
#pragma unroll
    for (int q = 0; q < NET; ++q) sel[q] = sel[q] || (j + 32 * q == bi);
  }
  float rsum = 0.0f;
  if (a.combine_mode == 1) {
#pragma unroll
    for (int q = 0; q < NET; ++q) rsum += sel[q] ? bal[q] : 0.0f;
    rsum = half_sum(rsum);
  }
  const float rden = fmaxf(rsum, 1e-9f);
  const int64_t base = (int64_t)b * E * a.T + t;
#pragma unroll
  for (int q = 0; q < NET; ++q) {
    if (!ok[q]) continue;
    const int e = j + 32 * q;
    if (live) {
      const int64_t i = base + (int64_t)e * a.T;
      a.mask[i] = sel[q] ? 1 : 0;
      a.balance[i] = bal[q];
      const float c = a.combine_mode == 1 ? (sel[q] ? bal[q] : 0.0f) / rden : bal[q];
      a.combine[i] = c * a.alpha;
    }
    sb_row[e] = live ? bal[q] : 0.0f;
    sc_row[e] = (live && sel[q]) ? 1 : 0;
  }
}

// Fused router for a block of 32 tokens x NET*32 experts: logits, then the
// selection of those tokens in the same workgroup.
//
// Logits, full blocks (SMALL = false): on the fp32 matrix cores
// (v_mfma_f32_32x32x2_f32: exact fp32 products, fp32 accumulation).  Wave w
// of NW covers the feature range [w*D/NW, (w+1)*D/NW) in chunks of 16: lane
// (r = lane % 32, h = lane / 32) feeds token t0 + r and expert 32*j + r with
// features d0 + 8h + s for s < 8, one MFMA per s (the k index of the MFMA is
// h, so each chunk's 16 features enter exactly once).  Accumulator element v
// of lane l is (token 8*(v/4) + 4*(l/32) + v%4, expert l%32).  The NW partial
// sums are added in wave order in LDS.
// Logits, batches of at most kSmallT tokens (SMALL, NET <= 2, NW = 8): on the
// vector ALU, so no MFMA work is spent on padding rows; thread i takes expert
// i / TPE and the 8-feature chunks i % TPE + TPE*m, and the TPE partial dot
// products of an expert are summed with a butterfly.
// Selection: 32 lanes per token (select_lanes), NW*2 tokens at a time.
// VEC: rows of whole 16-byte vectors (D % 8 == 0, aligned x and weights).
constexpr int kSmallT = 8;
template <class XT, int NET, int NW, bool SMALL, bool VEC>
__global__ __launch_bounds__(NW * kWave) void router_mfma_kernel(
    const typename XT::S* __restrict__ x, const float* __restrict__ rw, int64_t w_sb, int D,
    float* __restrict__ logits_out, SelectArgs a) {
  constexpr int EB = NET * 32;
  constexpr int NTH = NW * kWave;
  __shared__ float red[SMALL ? 1 : NW][NET][32][33];
  __shared__ float sb[32][EB + 1];
  __shared__ uint8_t sc[32][EB + 1];
  const int blk = blockIdx.x, b = blockIdx.y;
  const int t0 = blk * 32;
  const int w = threadIdx.x / kWave, lane = lane_id();
  const int E = a.E, T = a.T;
  const float* R = rw + (int64_t)b * w_sb;
  // the routing bias of this lane's experts for the selection, loaded now
  // (unconditionally, from a valid address without a bias) so that its
  // latency hides under the logits
  float bias_v[NET];
  {
    const int jl = threadIdx.x % 32;
    const float* bp = a.bias != nullptr ? a.bias + (int64_t)b * a.bias_sb : R;
#pragma unroll
    for (int q = 0; q < NET; ++q) {
      const int e = jl + 32 * q;
      const float v = bp[e < E ? e : 0];
      bias_v[q] = a.bias != nullptr && e < E ? v : 0.0f;
    }
  }
  if constexpr (SMALL) {
    static_assert(NTH % EB == 0, "threads must split evenly over the experts");
    constexpr int TPE = NTH / EB;
    const int e = threadIdx.x / TPE, sl = threadIdx.x % TPE;
    const int nt = min(T - t0, kSmallT);
    const int nch = (D + 7) / 8;
    float acc[kSmallT];
#pragma unroll
    for (int t = 0; t < kSmallT; ++t) acc[t] = 0.0f;
    const float* Re = R + (int64_t)(e < E ? e : 0) * D;
    // the batch's nt live tokens as a compile-time count (uniform per block):
    // every load unconditional, all of a chunk's in flight together (a load
    // under a per-token branch would be waited for before the next issues)
    auto logits = [&](auto NTC) __attribute__((always_inline)) {
      constexpr int NT = decltype(NTC)::value;
      if constexpr (NT <= 2) {
#pragma unroll 2
        for (int c = sl; c < nch; c += TPE) {
          float wv[8], xv[NT][8];
          load8<F32T, VEC>(Re, c * 8, D, e < E, wv);
#pragma unroll
          for (int t = 0; t < NT; ++t)
            load8<XT, VEC>(x + ((int64_t)b * T + t0 + t) * D, c * 8, D, true, xv[t]);
#pragma unroll
          for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[t] = fmaf(xv[t][i], wv[i], acc[t]);
        }
      } else {
        // three or more tokens: the loads of U chunks all issue before their
        // FMAs (one L2 round trip per group; per routing call at D = 1536,
        // E = 32: 8 tokens 21.9 -> 17.0 us, 4 tokens 15.9 -> 15.7 us; one or
        // two tokens keep the loop above, which the grouping made 5% slower).
        // The FMAs keep the chunk order and chunks past the row add nothing,
        // so the sums are the same bits.
        constexpr int U = NT <= 4 ? 3 : 2;
        for (int c0 = sl; c0 < nch; c0 += U * TPE) {
          float wv[U][8], xv[U][NT][8];
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const int c = c0 + u * TPE;
            load8<F32T, VEC>(Re, c * 8, D, e < E && c < nch, wv[u]);
#pragma unroll
            for (int t = 0; t < NT; ++t)
              load8<XT, VEC>(x + ((int64_t)b * T + t0 + t) * D, c * 8, D, c < nch, xv[u][t]);
          }
#pragma unroll
          for (int u = 0; u < U; ++u) {
            if (c0 + u * TPE < nch) {
#pragma unroll
              for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[t] = fmaf(xv[u][t][i], wv[u][i], acc[t]);
            }
          }
        }
      }
    };
    static_assert(kSmallT == 8, "one case per token count");
    switch (nt) {
      case 1: logits(std::integral_constant<int, 1>{}); break;
      case 2: logits(std::integral_constant<int, 2>{}); break;
      case 3: logits(std::integral_constant<int, 3>{}); break;
      case 4: logits(std::integral_constant<int, 4>{}); break;
      case 5: logits(std::integral_constant<int, 5>{}); break;
      case 6: logits(std::integral_constant<int, 6>{}); break;
      case 7: logits(std::integral_constant<int, 7>{}); break;
      default: logits(std::integral_constant<int, 8>{}); break;
    }
#pragma unroll
    for (int t = 0; t < kSmallT; ++t) {
#pragma unroll
      for (int o = TPE / 2; o >= 1; o >>= 1) acc[t] += __shfl_xor(acc[t], o, TPE);
    }
    for (int t = 0; t < 32; ++t)
      if (sl == 0 && e < EB) red[0][e / 32][t][e % 32] = t < kSmallT ? acc[t < kSmallT ? t : 0] : 0.0f;
    __syncthreads();
  } else {
    const int r = lane % 32, h = lane / 32;
    const bool tv = t0 + r < T;
    const typename XT::S* xrow = x + ((int64_t)b * T + (tv ? t0 + r : 0)) * D;
    const int nch = (D + 15) / 16;
    const int per = (nch + NW - 1) / NW;
    const int c_lo = w * per, c_hi = min(nch, c_lo + per);
    f32x16_t acc[NET];
#pragma unroll
    for (int j = 0; j < NET; ++j) acc[j] = f32x16_t{};
    // one chunk's MFMAs: 16 features (8 per lane half) of the token and NET
    // expert blocks
    auto mma = [&](const float (&xo)[8], const float (&wo)[NET][8]) __attribute__((always_inline)) {
      if constexpr (std::is_same_v<XT, BF16T>) {
        // bf16 x: each fp32 weight is split exactly into three bf16 parts
        // (hi + mid + lo = w for normal w: 3 x 8 mantissa bits), so the
        // products x*hi, x*mid, x*lo are exact and the fp32 accumulation
        // gives fp32 logits on the bf16 matrix cores (one 32x32x16 MFMA
        // per part covers the lane pair's 16 features; the f32 path needs 8
        // 32x32x2 MFMAs of twice the cycles)
        bf16x8_t xb;
#pragma unroll
        for (int i = 0; i < 8; ++i) xb[i] = static_cast<__bf16>(xo[i]);  // exact
#pragma unroll
        for (int j = 0; j < NET; ++j) {
          bf16x8_t hi, mid, lo;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float w = wo[j][i];
            hi[i] = static_cast<__bf16>(w);
            const float r1 = w - static_cast<float>(hi[i]);
            mid[i] = static_cast<__bf16>(r1);
            lo[i] = static_cast<__bf16>(r1 - static_cast<float>(mid[i]));
          }
          acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xb, hi, acc[j], 0, 0, 0);
          acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xb, mid, acc[j], 0, 0, 0);
          acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xb, lo, acc[j], 0, 0, 0);
        }
      } else {
#pragma unroll
        for (int j = 0; j < NET; ++j)
#pragma unroll
          for (int s8 = 0; s8 < 8; ++s8)
            acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(xo[s8], wo[j][s8], acc[j], 0, 0, 0);
      }
    };
    // a ring of DEPTH chunks in flight: each chunk's slot is refilled with the
    // chunk DEPTH ahead right after its MFMAs issue; slots past the range
    // hold zeros, whose MFMAs add nothing
    if constexpr (VEC) {
      // (a deeper ring, or refills pinned in place by scheduling barriers,
      // measured slower: each load instruction touches 32 rows, and more of
      // them in flight evict the L1 lines the next chunks reuse)
      constexpr int DEPTH = NET <= 2 ? 4 : 2;
      // the ring holds the loaded bytes; each slot is converted when used
      auto fetch = [&](int c, Raw8<XT>& xo, Raw8<F32T> (&wo)[NET]) __attribute__((always_inline)) {
        const int d = c * 16 + 8 * h;
        const bool in = c < c_hi;
        load_raw8<XT>(xrow, d, D, tv && in, xo);
#pragma unroll
        for (int j = 0; j < NET; ++j) {
          const int e = 32 * j + r;
          load_raw8<F32T>(R + (int64_t)(e < E ? e : 0) * D, d, D, in && e < E, wo[j]);
        }
      };
      Raw8<XT> xr[DEPTH];
      Raw8<F32T> wr[DEPTH][NET];
#pragma unroll
      for (int q = 0; q < DEPTH; ++q) fetch(c_lo + q, xr[q], wr[q]);
      for (int c = c_lo; c < c_hi; c += DEPTH) {
#pragma unroll
        for (int q = 0; q < DEPTH; ++q) {
          float xo[8], wo[NET][8];
          cvt8<XT>(xr[q], xo);
#pragma unroll
          for (int j = 0; j < NET; ++j) cvt8<F32T>(wr[q][j], wo[j]);
          mma(xo, wo);
          fetch(c + q + DEPTH, xr[q], wr[q]);
        }
      }
    } else {
      constexpr int DEPTH = NET <= 2 ? 4 : 2;
      auto fetch = [&](int c, float (&xo)[8], float (&wo)[NET][8]) __attribute__((always_inline)) {
        const int d = c * 16 + 8 * h;
        const bool in = c < c_hi;
        load8<XT, false>(xrow, d, D, tv && in, xo);
#pragma unroll
        for (int j = 0; j < NET; ++j) {
          const int e = 32 * j + r;
          load8<F32T, false>(R + (int64_t)(e < E ? e : 0) * D, d, D, in && e < E, wo[j]);
        }
      };
      float xr[DEPTH][8], wr[DEPTH][NET][8];
#pragma unroll
      for (int q = 0; q < DEPTH; ++q) fetch(c_lo + q, xr[q], wr[q]);
      for (int c = c_lo; c < c_hi; c += DEPTH) {
#pragma unroll
        for (int q = 0; q < DEPTH; ++q) {
          mma(xr[q], wr[q]);
          fetch(c + q + DEPTH, xr[q], wr[q]);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < NET; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) red[w][j][8 * (v / 4) + 4 * h + v % 4][r] = acc[j][v];
    __syncthreads();
    for (int i = threadIdx.x; i < NET * 32 * 32; i += NTH) {
      const int j = i / 1024, tok = (i / 32) % 32, e = i % 32;
      float v = red[0][j][tok][e];
#pragma unroll
      for (int q = 1; q < NW; ++q) v += red[q][j][tok][e];
      red[0][j][tok][e] = v;
    }
    __syncthreads();
  }
  if (logits_out != nullptr) {
    for (int i = threadIdx.x; i < E * 32; i += NTH) {
      const int e = i / 32, tok = i % 32;
      if (t0 + tok < T) logits_out[((int64_t)b * E + e) * T + t0 + tok] = red[0][e / 32][tok][e % 32];
    }
  }
  // selection: half-wave g of the block's 2*NW takes the live tokens g,
  // g + 2*NW, ... (the block sums below read only live rows)
  const int g = threadIdx.x / 32, jl = threadIdx.x % 32;
  const int ntok = min(32, T - t0);
  for (int tok = g; tok < ntok; tok += 2 * NW) {
    float lg[NET];
#pragma unroll
    for (int q = 0; q < NET; ++q) lg[q] = red[0][q][tok][jl];
    select_lanes<NET>(lg, bias_v, a, b, t0 + tok, true, jl, sb[tok], sc[tok]);
  }
  // only sb / sc are read across threads below: an LDS barrier, which does
  // not wait for the selection's global stores as __syncthreads() would
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  for (int e = threadIdx.x; e < E; e += NTH) {
    // all 32 rows read first (one LDS latency), then added in token order
    float sv[32];
    int cv[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      sv[i] = sb[i][e];
      cv[i] = sc[i][e];
    }
    float s = 0.0f;
    int c = 0;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      s += i < ntok ? sv[i] : 0.0f;
      c += i < ntok ? cv[i] : 0;
    }
    put_partial(a, b, blk, e, s, c);
  }
}

// group_sizes[b][e] and the balance sum of (b, e) over the select blocks:
// one workgroup per (b, e); thread i adds blocks i, i + 256, ... in order, then
// a fixed tree over the 256 thread sums (deterministic).
__global__ __launch_bounds__(kRT) void router_reduce_kernel(const float* __restrict__ part_bal,
                                                            const int32_t* __restrict__ part_cnt,
                                                            int E, int nblk,
                                                            int32_t* __restrict__ group_sizes,
                                                            float* __restrict__ bal_sum,
                                                            int32_t* __restrict__ cnt_sum) {
  __shared__ float sb[kRT];
  __shared__ int sc[kRT];
  const int be = blockIdx.x, b = be / E, e = be % E;
  float fb = 0.0f;
  int ic = 0;
  for (int k = threadIdx.x; k < nblk; k += kRT) {
    const int64_t o = ((int64_t)b * nblk + k) * E + e;
    fb += part_bal[o];
    ic += part_cnt[o];
  }
  sb[threadIdx.x] = fb;
  sc[threadIdx.x] = ic;
  __syncthreads();
  for (int w = kRT / 2; w > 0; w >>= 1) {
    if (threadIdx.x < w) {
      sb[threadIdx.x] += sb[threadIdx.x + w];
      sc[threadIdx.x] += sc[threadIdx.x + w];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    if (group_sizes != nullptr) group_sizes[be] = sc[0];
    bal_sum[be] = sb[0];
    cnt_sum[be] = sc[0];
  }
}

// lb_loss = E * sum_e (sum_b bal_sum[b][e] / (B T)) * freq_e,
// freq_e = mean_b(count) / sum_e mean_b(count).  One workgroup.
__global__ __launch_bounds__(kRT) void router_lb_kernel(const float* __restrict__ bal_sum,
                                                        const int32_t* __restrict__ cnt_sum,
                                                        int B, int E, int T,
                                                        float* __restrict__ lb_loss) {
  __shared__ float pm[kMaxE];
  __shared__ float gm[kMaxE];
  for (int e = threadIdx.x; e < E; e += kRT) {
    float s = 0.0f, g = 0.0f;
    for (int b = 0; b < B; ++b) {
      s += bal_sum[(int64_t)b * E + e];
      g += (float)cnt_sum[(int64_t)b * E + e];
    }
    pm[e] = s / ((float)B * (float)T);
    gm[e] = g / (float)B;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
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
  UTTT_REQUIRE(B <= 65535 && (int64_t)B * E <= 0x7fffffff, "%s: B=%d too large", what, B);
  return UTTT_OK;
}

// Workspace layout: [part_bal: B*nblk*E fp32][part_cnt: B*nblk*E int32]
// [bal_sum: B*E fp32][cnt_sum: B*E int32]; nblk = ceil(T / tokens per block).
struct Ws {
  float* part_bal;
  int32_t* part_cnt;
  float* bal_sum;
  int32_t* cnt_sum;
  int nblk;
  size_t bytes;
};
Ws ws_layout(void* base, int B, int T, int E, int blk_tokens) {
  const int nblk = (T + blk_tokens - 1) / blk_tokens;
  auto up = [](size_t v) { return (v + 255) & ~(size_t)255; };
  char* p = static_cast<char*>(base);
  Ws w{};
  size_t off = 0;
  w.part_bal = reinterpret_cast<float*>(p + off);
  off += up(sizeof(float) * (size_t)B * nblk * E);
  w.part_cnt = reinterpret_cast<int32_t*>(p + off);
  off += up(sizeof(int32_t) * (size_t)B * nblk * E);
  w.bal_sum = reinterpret_cast<float*>(p + off);
  off += up(sizeof(float) * (size_t)B * E);
  w.cnt_sum = reinterpret_cast<int32_t*>(p + off);
  off += up(sizeof(int32_t) * (size_t)B * E);
  w.nblk = nblk;
  w.bytes = off;
  return w;
}

SelectArgs make_args(const Ws& w, const float* bias, int64_t bias_sb, int B, int E, int T,
                     int topk, int router_type, int combine_mode, float alpha, float router_scale,
                     float norm_eps, void* mask, float* combine, float* balance,
                     int32_t* group_sizes) {
  return SelectArgs{bias, bias_sb, B, E, T, topk, router_type, combine_mode, alpha,
                    router_scale > 0.0f ? router_scale : sqrtf((float)E), norm_eps,
                    static_cast<uint8_t*>(mask), combine, balance, w.part_bal, w.part_cnt,
                    w.nblk, group_sizes, w.bal_sum, w.cnt_sum};
}

// group sizes, balance sums and lb_loss from the block partials
int finish(const Ws& w, int B, int E, int T, int32_t* group_sizes, float* lb_loss, hipStream_t st,
           const char* what) {
  if (w.nblk > 1)   // one block per batch: the select kernel wrote the sums
    hipLaunchKernelGGL(router_reduce_kernel, dim3(B * E), dim3(kRT), 0, st, w.part_bal,
                       w.part_cnt, E, w.nblk, group_sizes, w.bal_sum, w.cnt_sum);
  if (lb_loss != nullptr)
    hipLaunchKernelGGL(router_lb_kernel, dim3(1), dim3(kRT), 0, st, w.bal_sum, w.cnt_sum, B, E, T,
                       lb_loss);
  return check_launch(what);
}

// The fused logits + selection launch of route_tokens (nblk blocks of 32
// tokens per batch).
int launch_route_kernel(const void* x, int x_dtype, const float* router_w, int64_t w_sb, int B,
                        int T, int D, int E, int nblk, const SelectArgs& a, float* logits_out,
                        hipStream_t st) {
  const int net = (E + 31) / 32;
#define UTTT_ROUTE_LAUNCH(NET, NW, SMALL)                                                       \
  if (vec)                                                                                      \
    hipLaunchKernelGGL((router_mfma_kernel<XT, NET, NW, SMALL, true>), dim3(nblk, B),          \
                       dim3(NW * kWave), 0, st, static_cast<const S*>(x), router_w, w_sb, D,     \
                       logits_out, a);                                                          \
  else                                                                                          \
    hipLaunchKernelGGL((router_mfma_kernel<XT, NET, NW, SMALL, false>), dim3(nblk, B),         \
                       dim3(NW * kWave), 0, st, static_cast<const S*>(x), router_w, w_sb, D,     \
                       logits_out, a)
  // a few tokens per batch (generation): vector-ALU logits, no padded MFMA rows
  const bool small = T <= kSmallT;
  // rows of whole 16-byte vectors: every feature load is one unconditional vector load
  const bool vec = D % 8 == 0 && w_sb % 4 == 0 &&
                   ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(router_w)) & 15u) == 0;
  UTTT_DTYPE_SWITCH_LR(x_dtype, XT, {
    using S = typename XT::S;
    switch (net) {
      case 1:
        if (small) UTTT_ROUTE_LAUNCH(1, 8, true);
        else UTTT_ROUTE_LAUNCH(1, 8, false);
        break;
      case 2:
        if (small) UTTT_ROUTE_LAUNCH(2, 8, true);
        else UTTT_ROUTE_LAUNCH(2, 8, false);
        break;
      case 3: UTTT_ROUTE_LAUNCH(3, 4, false); break;
      default: UTTT_ROUTE_LAUNCH(4, 4, false); break;
    }
  });
#undef UTTT_ROUTE_LAUNCH
  return check_launch("route_tokens");
}

}  // namespace
}  // namespace uttt

using namespace uttt;

extern "C" size_t uttt_router_workspace_bytes(int B, int T, int E, int D) {
  if (B <= 0 || T <= 0 || E <= 0) return 0;
  return ws_layout(nullptr, B, T, E, D > 0 ? 32 : sel_tpb(e_bucket(E))).bytes;
}

extern "C" int uttt_router_select(const float* logits, int64_t l_sb, int64_t l_se, int64_t l_st,
                                  const float* bias, int64_t bias_sb, int B, int E, int T,
                                  int topk, int router_type, int combine_mode, float alpha,
                                  float router_scale, float norm_eps, void* mask,
                                  int32_t* group_sizes, float* combine, float* balance,
                                  float* lb_loss, float* balance_sum, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  if (int rc = check_select_args(B, E, T, topk, router_type, combine_mode, "router_select"))
    return rc;
  if (B == 0 || T == 0) return UTTT_OK;
  UTTT_REQUIRE(logits && mask && combine && balance, "router_select: null pointer");
  Ws w = ws_layout(workspace, B, T, E, sel_tpb(e_bucket(E)));
  UTTT_REQUIRE(workspace != nullptr && workspace_bytes >= w.bytes,
               "router_select: workspace %zu < %zu bytes", workspace_bytes, w.bytes);
  if (balance_sum != nullptr) w.bal_sum = balance_sum;
  const SelectArgs a = make_args(w, bias, bias_sb, B, E, T, topk, router_type, combine_mode,
                                 alpha, router_scale, norm_eps, mask, combine, balance,
                                 group_sizes);
  hipStream_t st = as_stream(stream);
  UTTT_EB_SWITCH(E, hipLaunchKernelGGL((router_select_kernel<EB>), dim3(w.nblk, B),
                                       dim3(sel_tpb(EB)), 0, st, logits, l_sb, l_se, l_st, a));
  if (int rc = check_launch("router_select")) return rc;
  return finish(w, B, E, T, group_sizes, lb_loss, st, "router_select");
}

extern "C" int uttt_route_tokens(const void* x, int x_dtype, const float* router_w, int64_t w_sb,
                                 int B, int T, int D, int E, const float* bias, int64_t bias_sb,
                                 int topk, int router_type, int combine_mode, float alpha,
                                 float router_scale, float norm_eps, float* logits_out,
                                 void* mask, int32_t* group_sizes, float* combine,
                                 float* balance, float* lb_loss, float* balance_sum,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = check_select_args(B, E, T, topk, router_type, combine_mode, "route_tokens"))
    return rc;
  UTTT_REQUIRE(D >= 1, "route_tokens: D=%d", D);
  if (B == 0 || T == 0) return UTTT_OK;
  UTTT_REQUIRE(x && router_w && mask && combine && balance, "route_tokens: null pointer");
  Ws w = ws_layout(workspace, B, T, E, 32);
  UTTT_REQUIRE(workspace != nullptr && workspace_bytes >= w.bytes,
               "route_tokens: workspace %zu < %zu bytes", workspace_bytes, w.bytes);
  if (balance_sum != nullptr) w.bal_sum = balance_sum;
  const SelectArgs a = make_args(w, bias, bias_sb, B, E, T, topk, router_type, combine_mode,
                                 alpha, router_scale, norm_eps, mask, combine, balance,
                                 group_sizes);
  hipStream_t st = as_stream(stream);
  if (int rc = launch_route_kernel(x, x_dtype, router_w, w_sb, B, T, D, E, w.nblk, a, logits_out,
                                   st))
    return rc;
  return finish(w, B, E, T, group_sizes, lb_loss, st, "route_tokens");
}

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

extern "C" size_t uttt_route_tokens_map_workspace_bytes(int B, int T, int E, int D) {
  if (B <= 0 || T <= 0 || E <= 0) return 0;
  return align256(uttt_router_workspace_bytes(B, T, E, D)) +
         uttt_row_id_map_workspace_bytes(B, T, E);
}

extern "C" int uttt_route_tokens_map_src_rows(int T, int E) {
  return rowmap_fused_fits(T, E) ? 1 : 0;
}

extern "C" int uttt_route_tokens_map(const void* x, int x_dtype, const float* router_w,
                                     int64_t w_sb, int B, int T, int D, int E, const float* bias,
                                     int64_t bias_sb, int topk, int router_type, int combine_mode,
                                     float alpha, float router_scale, float norm_eps, void* mask,
                                     int32_t* group_sizes, float* combine, float* balance,
                                     float* balance_sum, int32_t* row_id_map,
                                     int32_t* src_rows, void* workspace, size_t workspace_bytes,
                                     void* stream) {
  if (int rc = check_select_args(B, E, T, topk, router_type, combine_mode, "route_tokens_map"))
    return rc;
  UTTT_REQUIRE(src_rows == nullptr || rowmap_fused_fits(T, E),
               "route_tokens_map: the inverse map (src_rows) needs T %% 16 == 0, T <= 4096 and "
               "E <= 64 (T=%d, E=%d)", T, E);
  UTTT_REQUIRE(D >= 1, "route_tokens_map: D=%d", D);
  if (B == 0 || T == 0) return UTTT_OK;
  UTTT_REQUIRE(x && router_w && mask && combine && balance && group_sizes && balance_sum &&
                   row_id_map,
               "route_tokens_map: null pointer");
  Ws w = ws_layout(workspace, B, T, E, 32);
  const size_t rm_off = align256(w.bytes);
  const size_t need = rm_off + uttt_row_id_map_workspace_bytes(B, T, E);
  UTTT_REQUIRE(workspace != nullptr && workspace_bytes >= need,
               "route_tokens_map: workspace %zu < %zu bytes", workspace_bytes, need);
  w.bal_sum = balance_sum;
  const SelectArgs a = make_args(w, bias, bias_sb, B, E, T, topk, router_type, combine_mode,
                                 alpha, router_scale, norm_eps, mask, combine, balance,
                                 group_sizes);
  hipStream_t st = as_stream(stream);
  if (int rc = launch_route_kernel(x, x_dtype, router_w, w_sb, B, T, D, E, w.nblk, a, nullptr,
                                   st))
    return rc;
  // the one-launch row map also adds the selection blocks' balance partials
  // (group sizes are its own counts), so no reduce launch runs
  const uint8_t* m8 = static_cast<const uint8_t*>(mask);
  const int64_t s_b = (int64_t)E * T, s_e = T;
  if (launch_rowmap_fused(m8, s_b, s_e, B, T, E, group_sizes, row_id_map,
                          w.nblk > 1 ? w.part_bal : nullptr, w.nblk, balance_sum, st, src_rows,
                          (int64_t)T * topk))
    return check_launch("route_tokens_map");
  UTTT_REQUIRE(src_rows == nullptr,
               "route_tokens_map: the inverse map (src_rows) needs 16-byte aligned mask and "
               "row map");
  if (int rc = finish(w, B, E, T, group_sizes, nullptr, st, "route_tokens_map")) return rc;
  return uttt_make_row_id_map(mask, 1, s_b, s_e, 1, B, T, E, row_id_map, nullptr,
                              static_cast<uint8_t*>(workspace) + rm_off, workspace_bytes - rm_off,
                              stream);
}

