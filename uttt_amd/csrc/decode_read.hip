// Routed SwiGLU fast-weight read for a few tokens per sequence (generation):
// the uTTT-MoE apply of uttt_llm/flame/custom_models/uttt_moe/
// modeling_recurrent_lact.py:296-349 (route -> permute -> grouped SwiGLU
// apply -> gate-weighted unpermute) for T <= 64 tokens per batch, without the
// row map, the permuted copy or the unpermute pass.
//
// At decode every selected expert sees one or a few rows, so the work is two
// grouped GEMVs bound by reading the selected experts' weights from HBM:
//   kernel 1 (gate/up): per active (b, e) and row i of w0 / w2, the dot
//     products with the expert's tokens; hidden = bf16(y2 * (y0 * sigmoid(y0)))
//     into a [B, E, T, I] workspace (bf16, as the reference stores it between
//     its two GEMMs, L/lact_swiglu_ffn.py:37-61);
//   kernel 2 (down + combine): per row d of w1, for the batch's active experts
//     in descending expert order (the unpermute's slot order, rows sorted
//     descending, L/triton_permute.py:331-374), y = bf16(w1[d,:] . hidden)
//     (the grouped down GEMM's bf16 store) and out[t, d] = bf16(sum fma(y, p))
//     accumulated in fp32 (the unpermute, L/triton_permute.py:765-850).
// The active experts and their tokens come straight from the router's mask by
// wave ballots (E <= 64, T <= 64).  Each wave streams whole 16-byte chunks of
// its weight rows with every load of a row issued before the first FMA;
// reductions are fixed butterflies, so results are deterministic.
#include <mutex>

#include "common.h"

namespace uttt {
namespace {

constexpr int kDecThreads = 256;          // 4 waves
constexpr int kDecWaves = kDecThreads / kWave;
constexpr int kMaxTok = 4;                // tokens per register group (T > 1)
constexpr int kMaxChunks = 8;             // 16-byte chunks per lane: rows up to 4096
constexpr int kDecTargetBlocks = 1024;    // kernel 1 grid: about 4 workgroups per CU

template <int MB>
__device__ __forceinline__ bool mask_at(const void* m, int64_t off) {
  if constexpr (MB == 1) return reinterpret_cast<const uint8_t*>(m)[off] != 0;
  else return reinterpret_cast<const int32_t*>(m)[off] != 0;
}

// Bit e set iff expert e has at least one selected token in batch b.
template <int MB>
__device__ __forceinline__ uint64_t active_experts(const void* mask, int64_t s_b, int64_t s_e,
                                                   int64_t s_t, int b, int T, int E) {
  const int e = lane_id();
  bool any = false;
  if (e < E) {
    const int64_t base = (int64_t)b * s_b + (int64_t)e * s_e;
#pragma unroll 8
    for (int t = 0; t < T; ++t) any |= mask_at<MB>(mask, base + (int64_t)t * s_t);
  }
  return __ballot(any);
}

// Bit t set iff token t of batch b selected expert e.
template <int MB>
__device__ __forceinline__ uint64_t expert_tokens(const void* mask, int64_t s_b, int64_t s_e,
                                                  int64_t s_t, int b, int e, int T) {
  const int t = lane_id();
  const bool sel = t < T && mask_at<MB>(mask, (int64_t)b * s_b + (int64_t)e * s_e + (int64_t)t * s_t);
  return __ballot(sel);
}

// Index of the n-th set bit of m (n < popcount(m)).
__device__ __forceinline__ int nth_bit(uint64_t m, int n) {
  for (int i = 0; i < n; ++i) m &= m - 1;
  return __ffsll((unsigned long long)m) - 1;
}

// Bits lo .. hi-1 (0 <= lo < hi <= 64).
__device__ __forceinline__ uint64_t bit_range(int lo, int hi) {
  const uint64_t below_hi = hi >= 64 ? ~0ull : (1ull << hi) - 1ull;
  return below_hi & ~((1ull << lo) - 1ull);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ __forceinline__ float dot8(const uint4& w, const uint4& x, float acc) {
  const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
  const uint32_t xv[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    acc = fmaf(__uint_as_float(wv[q] << 16), __uint_as_float(xv[q] << 16), acc);
    acc = fmaf(__uint_as_float(wv[q] & 0xffff0000u), __uint_as_float(xv[q] & 0xffff0000u), acc);
  }
  return acc;
}

__device__ __forceinline__ float sigmoid_(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __expf(-x));
}

// Kernel 1.  grid (G, S, B): slot s of batch b takes the active experts s,
// s + S, s + 2S, ... (any number of them); wave w of workgroup g owns the row
// pairs i0 = (g * 4 + w) * RP + n * stride, stride = G * 4 * RP, with RP = 2
// row pairs per step for rows of up to 1536 elements and 1 beyond.
// Per token group the x chunks are loaded once; the row loop keeps two
// register sets of weights, loading the next row pairs while the current ones
// are reduced, so a wave streams without draining between rows.
template <int CPL>
constexpr int rows_k1() { return CPL <= 3 ? 2 : 1; }

// p[ch] where `ok`, else zeros; the load itself is unconditional (a lane
// that is off reads p[0], which every caller keeps valid), so a wave's loads
// of a step are all in flight before the first is used -- a load under a
// per-lane condition is waited for where the two paths merge.
__device__ __forceinline__ uint4 load_or_zero(const uint4* p, int ch, bool ok) {
  const uint4 v = p[ok ? ch : 0];
  return ok ? v : make_uint4(0, 0, 0, 0);
}

template <int MB, int CPL, int MT>
__global__ __launch_bounds__(kDecThreads) void decode_gate_up_kernel(
    const uint16_t* __restrict__ x, int T, int D, const uint16_t* __restrict__ w02,
    int E, int I, const void* __restrict__ mask, int64_t s_b, int64_t s_e, int64_t s_t,
    uint16_t* __restrict__ hid) {
  constexpr int RP = rows_k1<CPL>();
  const int b = blockIdx.z;
  const int wave = threadIdx.x / kWave;
  const int lane = lane_id();
  const int first = (blockIdx.x * kDecWaves + wave) * RP;
  const int stride = gridDim.x * kDecWaves * RP;
  if (first >= I) return;
  const int nch = D / 8;
  const uint64_t act = active_experts<MB>(mask, s_b, s_e, s_t, b, T, E);
  const int nact = __popcll(act);
  for (int slot = blockIdx.y; slot < nact; slot += gridDim.y) {
    const int e = nth_bit(act, slot);
    const uint64_t tm = expert_tokens<MB>(mask, s_b, s_e, s_t, b, e, T);
    const uint16_t* wb = w02 + ((int64_t)b * E + e) * (int64_t)(2 * I) * D;
    auto load = [&](int i0, uint4 (&w0)[RP][CPL], uint4 (&w2)[RP][CPL])
        __attribute__((always_inline)) {
#pragma unroll
      for (int r = 0; r < RP; ++r) {
        const int i = min(i0 + r, I - 1);
        const uint4* p0 = reinterpret_cast<const uint4*>(wb + (int64_t)i * D);
        const uint4* p2 = reinterpret_cast<const uint4*>(wb + (int64_t)(I + i) * D);
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
          const int ch = lane + c * kWave;
          w0[r][c] = load_or_zero(p0, ch, ch < nch);
          w2[r][c] = load_or_zero(p2, ch, ch < nch);
        }
      }
    };
    uint64_t rest = tm;
    while (rest) {                              // token groups of MT
      int tok[MT];
      int nt = 0;
#pragma unroll
      for (int j = 0; j < MT; ++j) {
        tok[j] = rest ? __ffsll((unsigned long long)rest) - 1 : -1;
        if (rest) { rest &= rest - 1; ++nt; }
      }
      uint4 xv[MT][CPL];
#pragma unroll
      for (int j = 0; j < MT; ++j) {
        const uint4* px = reinterpret_cast<const uint4*>(x + ((int64_t)b * T + max(tok[j], 0)) * D);
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
          const int ch = lane + c * kWave;
          xv[j][c] = load_or_zero(px, ch, j < nt && ch < nch);
        }
      }
      auto compute = [&](int i0, const uint4 (&w0)[RP][CPL],
                         const uint4 (&w2)[RP][CPL]) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < MT; ++j) {
          if (j >= nt) break;
          uint16_t* hrow = hid + (((int64_t)b * E + e) * T + tok[j]) * I;
#pragma unroll
          for (int r = 0; r < RP; ++r) {
            float a0 = 0.0f, a2 = 0.0f;
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
              a0 = dot8(w0[r][c], xv[j][c], a0);
              a2 = dot8(w2[r][c], xv[j][c], a2);
            }
            const float y0 = wave_sum(a0);
            const float y2 = wave_sum(a2);
            if (lane == 0 && i0 + r < I) hrow[i0 + r] = f32_to_bf16(y2 * (y0 * sigmoid_(y0)));
          }
        }
      };
      uint4 wa0[RP][CPL], wa2[RP][CPL], wb0[RP][CPL], wb2[RP][CPL];
      int i0 = first;
      load(i0, wa0, wa2);
      while (true) {                            // two row steps per turn: A then B
        const int i1 = i0 + stride;
        if (i1 < I) load(i1, wb0, wb2);
        compute(i0, wa0, wa2);
        if (i1 >= I) break;
        const int i2 = i1 + stride;
        if (i2 < I) load(i2, wa0, wa2);
        compute(i1, wb0, wb2);
        if (i2 >= I) break;
        i0 = i2;
      }
    }
  }
}

// One row d of w1 for every token of batch b: the active experts act in
// descending order (two at a time, both rows' loads in flight before their
// token sets are read), y = bf16(w1[d,:] . hidden), out = bf16(sum fma(y, p)).
template <int MB, int CPL, int MT>
__device__ __forceinline__ void down_row(
    const uint16_t* __restrict__ hid, int T, int D, const uint16_t* __restrict__ w1, int E,
    int I, const void* __restrict__ mask, int64_t s_b, int64_t s_e, int64_t s_t,
    const float* __restrict__ probs, int64_t p_sb, int64_t p_se, int64_t p_st,
    uint16_t* __restrict__ out, int b, int d, uint64_t act) {
  const int lane = lane_id();
  const int nch = I / 8;
  for (int g0 = 0; g0 < T; g0 += MT) {         // token groups of MT
    const uint64_t gmask = bit_range(g0, min(T, g0 + MT));
    float acc[MT];
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[j] = 0.0f;
    uint64_t rest = act;
    while (rest) {
      int ex[2];
      ex[0] = 63 - __clzll((long long)rest);
      rest &= ~(1ull << ex[0]);
      ex[1] = rest ? 63 - __clzll((long long)rest) : -1;
      if (ex[1] >= 0) rest &= ~(1ull << ex[1]);
      uint4 w[2][CPL];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int e = ex[q] >= 0 ? ex[q] : ex[0];
        const uint4* pw = reinterpret_cast<const uint4*>(
            w1 + (((int64_t)b * E + e) * D + d) * (int64_t)I);
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
          const int ch = lane + c * kWave;
          w[q][c] = load_or_zero(pw, ch, ch < nch && ex[q] >= 0);
        }
      }
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        if (ex[q] < 0) break;
        const int e = ex[q];
        const uint64_t tm = expert_tokens<MB>(mask, s_b, s_e, s_t, b, e, T) & gmask;
#pragma unroll
        for (int j = 0; j < MT; ++j) {
          const int t = g0 + j;
          if (t >= T || !((tm >> t) & 1ull)) continue;
          const uint4* ph = reinterpret_cast<const uint4*>(hid + (((int64_t)b * E + e) * T + t) * I);
          float a = 0.0f;
#pragma unroll
          for (int c = 0; c < CPL; ++c) {
            const int ch = lane + c * kWave;
            a = dot8(w[q][c], load_or_zero(ph, ch, ch < nch), a);  // w is 0 past nch
          }
          const float y = bf16_to_f32(f32_to_bf16(wave_sum(a)));
          const float p = probs[(int64_t)b * p_sb + (int64_t)e * p_se + (int64_t)t * p_st];
          acc[j] = fmaf(y, p, acc[j]);
        }
      }
    }
    if (lane == 0) {
#pragma unroll
      for (int j = 0; j < MT; ++j) {
        const int t = g0 + j;
        if (t < T) out[((int64_t)b * T + t) * D + d] = f32_to_bf16(acc[j]);
      }
    }
  }
}

// Kernel 2.  grid (ceil(D / kDecWaves), B): one row d of w1 per wave.
template <int MB, int CPL, int MT>
__global__ __launch_bounds__(kDecThreads) void decode_down_kernel(
    const uint16_t* __restrict__ hid, int T, int D, const uint16_t* __restrict__ w1, int E,
    int I, const void* __restrict__ mask, int64_t s_b, int64_t s_e, int64_t s_t,
    const float* __restrict__ probs, int64_t p_sb, int64_t p_se, int64_t p_st,
    uint16_t* __restrict__ out) {
  const int b = blockIdx.y;
  const int d = blockIdx.x * kDecWaves + threadIdx.x / kWave;
  if (d >= D) return;
  const uint64_t act = active_experts<MB>(mask, s_b, s_e, s_t, b, T, E);
  down_row<MB, CPL, MT>(hid, T, D, w1, E, I, mask, s_b, s_e, s_t, probs, p_sb, p_se, p_st, out,
                        b, d, act);
}

// Kernel 2 for one token per batch with at most two selected experts (the
// top-2 decode step).  grid (G, B): wave w of workgroup g owns the rows
// d = g * 4 + w + n * stride, stride = G * 4.  The two experts, their gates
// and hidden vectors are read once per wave; the rows of w1 then stream
// through two register sets (the next row's loads issue before the current
// row's reductions).  A batch whose token selected more than two experts
// takes the general per-row path.
template <int MB, int CPL>
__global__ __launch_bounds__(kDecThreads) void decode_down_t1_kernel(
    const uint16_t* __restrict__ hid, int D, const uint16_t* __restrict__ w1, int E, int I,
    const void* __restrict__ mask, int64_t s_b, int64_t s_e, int64_t s_t,
    const float* __restrict__ probs, int64_t p_sb, int64_t p_se, int64_t p_st,
    uint16_t* __restrict__ out) {
  const int b = blockIdx.y;
  const int wave = threadIdx.x / kWave;
  const int lane = lane_id();
  const int first = blockIdx.x * kDecWaves + wave;
  const int stride = gridDim.x * kDecWaves;
  if (first >= D) return;
  const int nch = I / 8;
  uint64_t act = active_experts<MB>(mask, s_b, s_e, s_t, b, 1, E);
  if (__popcll(act) > 2) {
    for (int d = first; d < D; d += stride)
      down_row<MB, CPL, 1>(hid, 1, D, w1, E, I, mask, s_b, s_e, s_t, probs, p_sb, p_se, p_st,
                           out, b, d, act);
    return;
  }
  int ex[2];
  float p[2];
  uint4 h[2][CPL];
#pragma unroll
  for (int q = 0; q < 2; ++q) {               // descending expert order
    ex[q] = act ? 63 - __clzll((long long)act) : -1;
    if (act) act &= ~(1ull << ex[q]);
    const int e = max(ex[q], 0);
    p[q] = ex[q] >= 0 ? probs[(int64_t)b * p_sb + (int64_t)e * p_se] : 0.0f;
    const uint4* ph = reinterpret_cast<const uint4*>(hid + ((int64_t)b * E + e) * I);
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int ch = lane + c * kWave;
      h[q][c] = load_or_zero(ph, ch, ex[q] >= 0 && ch < nch);
    }
  }
  auto load = [&](int d, uint4 (&w)[2][CPL]) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint4* pw = reinterpret_cast<const uint4*>(
          w1 + (((int64_t)b * E + max(ex[q], 0)) * D + d) * (int64_t)I);
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        const int ch = lane + c * kWave;
        w[q][c] = load_or_zero(pw, ch, ex[q] >= 0 && ch < nch);
      }
    }
  };
  auto compute = [&](int d, const uint4 (&w)[2][CPL]) __attribute__((always_inline)) {
    float acc = 0.0f;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      if (ex[q] < 0) break;
      float a = 0.0f;
#pragma unroll
      for (int c = 0; c < CPL; ++c) a = dot8(w[q][c], h[q][c], a);
      acc = fmaf(bf16_to_f32(f32_to_bf16(wave_sum(a))), p[q], acc);
    }
    if (lane == 0) out[(int64_t)b * D + d] = f32_to_bf16(acc);
  };
  uint4 wa[2][CPL], wb[2][CPL];
  int d = first;
  load(d, wa);
  while (true) {                                // two rows per turn: A then B
    const int d1 = d + stride;
    if (d1 < D) load(d1, wb);
    compute(d, wa);
    if (d1 >= D) break;
    const int d2 = d1 + stride;
    if (d2 < D) load(d2, wa);
    compute(d1, wb);
    if (d2 >= D) break;
    d = d2;
  }
}

template <int MB>
int launch_decode(const uint16_t* x, int B, int T, int D, const uint16_t* w02, const uint16_t* w1,
                  int E, int I, const void* mask, int64_t s_b, int64_t s_e, int64_t s_t,
                  const float* probs, int64_t p_sb, int64_t p_se, int64_t p_st, int S,
                  uint16_t* out, uint16_t* hid, hipStream_t st) {
  const int cpl_d = (D / 8 + kWave - 1) / kWave;
  const int cpl_i = (I / 8 + kWave - 1) / kWave;
  const dim3 g2((D + kDecWaves - 1) / kDecWaves, B);
  // kernel 1: enough workgroups to cover the chip about four times over, each
  // wave streaming several row pairs; one token per batch (the decode step)
  // keeps a single accumulator set
  auto k1 = [&](auto c) {
    constexpr int C = decltype(c)::value;
    constexpr int RP = rows_k1<C>();
    const int g_max = (I + kDecWaves * RP - 1) / (kDecWaves * RP);
    const dim3 g1(max(1, min(g_max, (kDecTargetBlocks + S * B - 1) / (S * B))), S, B);
    constexpr int MT = C <= 4 ? kMaxTok : 2;   // longer rows: fewer x registers
    if (T == 1)
      hipLaunchKernelGGL((decode_gate_up_kernel<MB, C, 1>), g1, dim3(kDecThreads), 0, st, x, T,
                         D, w02, E, I, mask, s_b, s_e, s_t, hid);
    else
      hipLaunchKernelGGL((decode_gate_up_kernel<MB, C, MT>), g1, dim3(kDecThreads), 0, st, x, T,
                         D, w02, E, I, mask, s_b, s_e, s_t, hid);
  };
  auto k2 = [&](auto c) {
    constexpr int C = decltype(c)::value;
    if (T == 1) {
      const dim3 g(max(1, min((int)g2.x, (kDecTargetBlocks + B - 1) / B)), B);
      hipLaunchKernelGGL((decode_down_t1_kernel<MB, C>), g, dim3(kDecThreads), 0, st, hid, D,
                         w1, E, I, mask, s_b, s_e, s_t, probs, p_sb, p_se, p_st, out);
    } else {
      hipLaunchKernelGGL((decode_down_kernel<MB, C, kMaxTok>), g2, dim3(kDecThreads), 0, st, hid,
                         T, D, w1, E, I, mask, s_b, s_e, s_t, probs, p_sb, p_se, p_st, out);
    }
  };
  auto by_cpl = [&](int c, auto&& fn) {
    switch (c) {
      case 1: fn(std::integral_constant<int, 1>{}); break;
      case 2: fn(std::integral_constant<int, 2>{}); break;
      case 3: fn(std::integral_constant<int, 3>{}); break;
      case 4: fn(std::integral_constant<int, 4>{}); break;
      case 5: fn(std::integral_constant<int, 5>{}); break;
      case 6: fn(std::integral_constant<int, 6>{}); break;
      default: fn(std::integral_constant<int, kMaxChunks>{}); break;
    }
  };
  by_cpl(cpl_d, k1);
  if (int rc = check_launch("moe_decode_read: gate/up")) return rc;
  by_cpl(cpl_i, k2);
  return check_launch("moe_decode_read: down");
}

}  // namespace
}  // namespace uttt

using namespace uttt;

extern "C" size_t uttt_moe_decode_read_workspace_bytes(int B, int T, int E, int I) {
  if (B <= 0 || T <= 0 || E <= 0 || I <= 0) return 0;
  return (size_t)B * E * T * I * sizeof(uint16_t);
}

namespace {

// The read after argument checks, with the hidden buffer `hid` of at least
// uttt_moe_decode_read_workspace_bytes(B, T, E, I) bytes.
int decode_read_checked(const void* x, int B, int T, int D, const void* w0_w2, const void* w1,
                        int E, int I, const void* expert_mask, int mask_bytes, int64_t m_sb,
                        int64_t m_se, int64_t m_st, const float* probs, int64_t p_sb,
                        int64_t p_se, int64_t p_st, int topk, void* out, void* hid,
                        hipStream_t st) {
  const int S = min(E, topk * T);
  auto* xs = reinterpret_cast<const uint16_t*>(x);
  auto* w02 = reinterpret_cast<const uint16_t*>(w0_w2);
  auto* w1s = reinterpret_cast<const uint16_t*>(w1);
  auto* o = reinterpret_cast<uint16_t*>(out);
  auto* h = reinterpret_cast<uint16_t*>(hid);
  if (mask_bytes == 1)
    return launch_decode<1>(xs, B, T, D, w02, w1s, E, I, expert_mask, m_sb, m_se, m_st, probs,
                            p_sb, p_se, p_st, S, o, h, st);
  return launch_decode<4>(xs, B, T, D, w02, w1s, E, I, expert_mask, m_sb, m_se, m_st, probs, p_sb,
                          p_se, p_st, S, o, h, st);
}

// Shape and pointer checks shared by both entry points; sets *done when
// there is nothing to launch beyond what it did (an empty problem, or the
// zero output of I = 0).
int decode_read_args(const void* x, int B, int T, int D, const void* w0_w2, const void* w1,
                     int E, int I, const void* expert_mask, int mask_bytes, const float* probs,
                     int topk, void* out, hipStream_t st, const char* what, bool* done) {
  *done = true;
  UTTT_REQUIRE(B >= 0 && T >= 0 && D >= 0 && I >= 0 && E >= 1,
               "%s: bad sizes B=%d T=%d D=%d I=%d E=%d", what, B, T, D, I, E);
  UTTT_REQUIRE(E <= 64, "%s: E=%d exceeds 64", what, E);
  UTTT_REQUIRE(T <= 64, "%s: T=%d tokens per batch exceed 64 (use the grouped apply)", what, T);
  UTTT_REQUIRE(D % 8 == 0 && I % 8 == 0, "%s: D=%d and I=%d must be multiples of 8", what, D, I);
  UTTT_REQUIRE(D <= 8 * kWave * kMaxChunks && I <= 8 * kWave * kMaxChunks,
               "%s: D=%d and I=%d must be at most %d", what, D, I, 8 * kWave * kMaxChunks);
  UTTT_REQUIRE(mask_bytes == 1 || mask_bytes == 4, "%s: mask element size %d", what, mask_bytes);
  UTTT_REQUIRE(topk >= 1, "%s: topk=%d", what, topk);
  if (B == 0 || T == 0 || D == 0) return UTTT_OK;
  UTTT_REQUIRE(x && w0_w2 && w1 && expert_mask && probs && out, "%s: null pointer", what);
  if (I == 0) return zero_fill_async(out, sizeof(uint16_t) * (size_t)B * T * D, st, what);
  *done = false;
  return UTTT_OK;
}

}  // namespace

extern "C" int uttt_moe_decode_read(const void* x, int B, int T, int D, const void* w0_w2,
                                    const void* w1, int E, int I, const void* expert_mask,
                                    int mask_bytes, int64_t m_sb, int64_t m_se, int64_t m_st,
                                    const float* probs, int64_t p_sb, int64_t p_se, int64_t p_st,
                                    int topk, void* out, void* workspace, size_t workspace_bytes,
                                    void* stream) {
  hipStream_t st = as_stream(stream);
  bool done = false;
  if (int rc = decode_read_args(x, B, T, D, w0_w2, w1, E, I, expert_mask, mask_bytes, probs,
                                topk, out, st, "moe_decode_read", &done))
    return rc;
  if (done) return UTTT_OK;
  const size_t need = uttt_moe_decode_read_workspace_bytes(B, T, E, I);
  UTTT_REQUIRE(workspace != nullptr && workspace_bytes >= need,
               "moe_decode_read: workspace %zu < %zu bytes", workspace_bytes, need);
  return decode_read_checked(x, B, T, D, w0_w2, w1, E, I, expert_mask, mask_bytes, m_sb, m_se,
                             m_st, probs, p_sb, p_se, p_st, topk, out, workspace, st);
}

// ------------------------------------------------- no-allocation variant ----
// The same read with its hidden buffer in a file-scope device array instead
// of a caller workspace, for callers that cannot allocate (code under HIP
// graph capture, serving loops).  Each GPU the library runs on holds its own
// copy of the array until the process ends.  The kernels address it through
// the pointer hipGetSymbolAddress returns for the current device, taken once
// per device on the first call there (the array's name is a host-side
// stand-in, not a device address).  Calls that overlap on one GPU (other
// streams, other threads) share the array and race; calls in stream order do
// not.  The second kernel reads only hidden entries the first kernel wrote in
// the same call, so the array needs no clearing between calls.
constexpr size_t kNoAllocScratchBytes = (size_t)8 << 20;   // 8 MiB per GPU
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device (looked up once per device).
int scratch_on_current_device(void** ptr, const char* what) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("%s: no usable current device (%d)", what, dev);
    return UTTT_ERR_HIP;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || p == nullptr) {
      set_error("%s: hipGetSymbolAddress of the scratch array failed on device %d: %s", what,
                dev, hipGetErrorString(err));
      return UTTT_ERR_HIP;
    }
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return UTTT_OK;
}
}  // namespace

extern "C" int uttt_moe_decode_read_noalloc(const void* x, int B, int T, int D,
                                            const void* w0_w2, const void* w1, int E, int I,
                                            const void* expert_mask, int mask_bytes,
                                            int64_t m_sb, int64_t m_se, int64_t m_st,
                                            const float* probs, int64_t p_sb, int64_t p_se,
                                            int64_t p_st, int topk, void* out, void* stream) {
  const char* what = "moe_decode_read_noalloc";
  hipStream_t st = as_stream(stream);
  bool done = false;
  if (int rc = decode_read_args(x, B, T, D, w0_w2, w1, E, I, expert_mask, mask_bytes, probs,
                                topk, out, st, what, &done))
    return rc;
  if (done) return UTTT_OK;
  const size_t need = uttt_moe_decode_read_workspace_bytes(B, T, E, I);
  UTTT_REQUIRE(need <= kNoAllocScratchBytes,
               "%s: B*E*T*I*2 = %zu bytes of hidden state exceed the %zu-byte scratch array "
               "(use uttt_moe_decode_read with a workspace)",
               what, need, kNoAllocScratchBytes);
  int dev_st = -1, dev_cur = -1;
  if (st != nullptr && hipStreamGetDevice(st, &dev_st) == hipSuccess &&
      hipGetDevice(&dev_cur) == hipSuccess)
    UTTT_REQUIRE(dev_st == dev_cur, "%s: the stream belongs to device %d, the current device is %d",
                 what, dev_st, dev_cur);
  void* hid = nullptr;
  if (int rc = scratch_on_current_device(&hid, what)) return rc;
  return decode_read_checked(x, B, T, D, w0_w2, w1, E, I, expert_mask, mask_bytes, m_sb, m_se,
                             m_st, probs, p_sb, p_se, p_st, topk, out, hid, st);
}
