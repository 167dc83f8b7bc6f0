// uTTT-Dense head layout: the per-head split of activations that the dense
// fast-weight read and write run on, as single HBM-bound launches.
//
//   gather_heads_kernel   for L layers at once (the aggregate write batches
//                         every layer's tokens per head):
//                           kh[bb*H + hh, li*l + t, :] = k_li[bb, t, hh*d : hh*d + d]
//                           (vh likewise from v_li), and
//                           lr_j[bb*H + hh, li*l + t] = lr_li[bb, t, j]       (shared lr)
//                                                     = lr_li[bb, t, 3*hh + j] (per head)
//                         as fp32.  Reference: the rearranges 'b l (h d) ->
//                         (b h) l d' of k and v and 'b l h -> (b h) l 1' of the
//                         lr columns in compute_update,
//                         uttt_dense/modeling_recurrent_lact.py:370-398, and of
//                         the read input at :251; the per-layer concatenation
//                         replaces the layer loop of _aggregate_memory_update
//                         (:1302-1386).
//   scatter_heads_kernel  the inverse for one tensor: out[bb, t, hh*d + c] =
//                         y[bb*H + hh, t, c] ('(b h) l hd -> b l (h hd)', :261).
//
// Both move 16-byte chunks (d a multiple of 8): a source row [H*d] of one
// token is read contiguously; each head's d-element run lands contiguously.
// Sources are read once (non-temporal loads); destinations are stored
// normally, since the grouped kernels read them next.
#include <stdint.h>

#include <algorithm>

#include "common.h"

namespace uttt {
namespace {

constexpr int kHeadThreads = 256;

typedef uint32_t nt_u32x4 __attribute__((ext_vector_type(4)));

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

__device__ __forceinline__ void copy16(const void* src, void* dst) {
  const nt_u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const nt_u32x4*>(src));
  *reinterpret_cast<nt_u32x4*>(dst) = v;
}

// blockIdx.y = layer (uniform, so the pointer comes from the kernel arguments
// with a scalar load)
template <class LR>
__global__ __launch_bounds__(kHeadThreads) void gather_heads_kernel(
    LayerPtrs ks, LayerPtrs vs, LayerPtrs lrs, int lr_per_head, int L, int b, int l, int H,
    int d, uint16_t* __restrict__ kh, uint16_t* __restrict__ vh, float* __restrict__ lr0,
    float* __restrict__ lr1, float* __restrict__ lr2) {
  const int li = blockIdx.y;
  const uint16_t* k = static_cast<const uint16_t*>(ks.p[li]);
  const uint16_t* v = static_cast<const uint16_t*>(vs.p[li]);
  const int cpr = H * d / 8;  // 16-byte chunks per token row
  const int chunks = b * l * cpr;  // below 2^31 (checked on the host)
  const int64_t rows_out = (int64_t)L * l;  // tokens per head after the concatenation
  const int stride = gridDim.x * kHeadThreads;
  for (int g = blockIdx.x * kHeadThreads + threadIdx.x; g < chunks; g += stride) {
    const int c = g % cpr;
    const int bt = g / cpr;  // bb * l + t
    const int t = bt % l, bb = bt / l;
    const int hh = c * 8 / d, o = c * 8 - hh * d;
    const int64_t dst = (((int64_t)bb * H + hh) * rows_out + (int64_t)li * l + t) * d + o;
    copy16(k + (int64_t)g * 8, kh + dst);
    if (v) copy16(v + (int64_t)g * 8, vh + dst);
  }
  if (!lr0) return;
  using S = typename LR::S;
  const S* lr = static_cast<const S*>(lrs.p[li]);
  const int items = b * l * H;
  for (int g = blockIdx.x * kHeadThreads + threadIdx.x; g < items; g += stride) {
    const int hh = g % H;
    const int bt = g / H;
    const int t = bt % l, bb = bt / l;
    const S* src = lr + (int64_t)bt * (lr_per_head ? 3 * H : 3) + (lr_per_head ? 3 * hh : 0);
    const int64_t dst = ((int64_t)bb * H + hh) * rows_out + (int64_t)li * l + t;
    lr0[dst] = LR::load(src[0]);
    lr1[dst] = LR::load(src[1]);
    lr2[dst] = LR::load(src[2]);
  }
}

__global__ __launch_bounds__(kHeadThreads) void scatter_heads_kernel(const uint16_t* __restrict__ y,
                                                                    int b, int l, int H, int d,
                                                                    uint16_t* __restrict__ out) {
  const int cpr = H * d / 8;
  const int chunks = b * l * cpr;
  const int stride = gridDim.x * kHeadThreads;
  for (int g = blockIdx.x * kHeadThreads + threadIdx.x; g < chunks; g += stride) {
    const int c = g % cpr;
    const int bt = g / cpr;
    const int t = bt % l, bb = bt / l;
    const int hh = c * 8 / d, o = c * 8 - hh * d;
    copy16(y + (((int64_t)bb * H + hh) * l + t) * d + o, out + (int64_t)g * 8);
  }
}

unsigned grid_for(int64_t work) {
  // one chunk per thread (every load in flight at once) up to 2^16
  // workgroups per layer, then grid-stride
  const int64_t blocks = (work + kHeadThreads - 1) / kHeadThreads;
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>(blocks, 65536));
}

}  // namespace
}  // namespace uttt

using namespace uttt;

extern "C" int uttt_dense_gather_heads(const void* const* k_layers, const void* const* v_layers,
                                       const void* const* lr_layers, int lr_dtype,
                                       int lr_per_head, int L, int b, int l, int H, int d,
                                       void* kh, void* vh, float* lr0, float* lr1, float* lr2,
                                       void* stream) {
  UTTT_REQUIRE(L >= 0 && L <= kMaxLayers && b >= 0 && l >= 0 && H >= 1 && d >= 0,
               "dense_gather_heads: bad sizes (L=%d must be at most %d)", L, kMaxLayers);
  UTTT_REQUIRE(d % 8 == 0, "dense_gather_heads: d=%d must be a multiple of 8", d);
  if (L == 0 || b == 0 || l == 0 || d == 0) return UTTT_OK;
  UTTT_REQUIRE((int64_t)b * l * H * d / 8 + (1 << 21) < INT32_MAX,
               "dense_gather_heads: b*l*H*d too large for one layer");
  UTTT_REQUIRE(k_layers && kh, "dense_gather_heads: null pointer");
  UTTT_REQUIRE((v_layers != nullptr) == (vh != nullptr), "dense_gather_heads: v and vh go together");
  const bool with_lr = lr_layers != nullptr;
  UTTT_REQUIRE(!with_lr || (lr0 && lr1 && lr2), "dense_gather_heads: lr outputs missing");
  UTTT_REQUIRE(aligned16(kh) && (!vh || aligned16(vh)), "dense_gather_heads: outputs must be 16-byte aligned");
  LayerPtrs ks{}, vs{}, lrs{};
  for (int i = 0; i < L; ++i) {
    ks.p[i] = k_layers[i];
    UTTT_REQUIRE(ks.p[i] && aligned16(ks.p[i]), "dense_gather_heads: k of layer %d null or unaligned", i);
    if (v_layers) {
      vs.p[i] = v_layers[i];
      UTTT_REQUIRE(vs.p[i] && aligned16(vs.p[i]), "dense_gather_heads: v of layer %d null or unaligned", i);
    }
    if (with_lr) {
      lrs.p[i] = lr_layers[i];
      UTTT_REQUIRE(lrs.p[i], "dense_gather_heads: lr of layer %d null", i);
    }
  }
  const dim3 grid(grid_for((int64_t)b * l * H * d / 8), (unsigned)L);
  hipStream_t st = as_stream(stream);
  UTTT_DTYPE_SWITCH_LR(with_lr ? lr_dtype : (int)UTTT_F32, LR, {
    hipLaunchKernelGGL((gather_heads_kernel<LR>), grid, dim3(kHeadThreads), 0, st, ks, vs, lrs,
                       lr_per_head, L, b, l, H, d, static_cast<uint16_t*>(kh),
                       static_cast<uint16_t*>(vh), with_lr ? lr0 : nullptr, lr1, lr2);
  });
  return check_launch("dense_gather_heads");
}

extern "C" int uttt_dense_scatter_heads(const void* y, int b, int l, int H, int d, void* out,
                                        void* stream) {
  UTTT_REQUIRE(b >= 0 && l >= 0 && H >= 1 && d >= 0, "dense_scatter_heads: bad sizes");
  UTTT_REQUIRE(d % 8 == 0, "dense_scatter_heads: d=%d must be a multiple of 8", d);
  if (b == 0 || l == 0 || d == 0) return UTTT_OK;
  UTTT_REQUIRE((int64_t)b * l * H * d / 8 + (1 << 21) < INT32_MAX,
               "dense_scatter_heads: b*l*H*d too large");
  UTTT_REQUIRE(y && out && aligned16(y) && aligned16(out),
               "dense_scatter_heads: null or unaligned pointer");
  hipLaunchKernelGGL(scatter_heads_kernel, dim3(grid_for((int64_t)b * l * H * d / 8)),
                     dim3(kHeadThreads), 0, as_stream(stream), static_cast<const uint16_t*>(y), b,
                     l, H, d, static_cast<uint16_t*>(out));
  return check_launch("dense_scatter_heads");
}
