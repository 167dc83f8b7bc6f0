// Shared helpers for the gfx950 kernels of libuttt_hip.so: status handling,
// dtype conversion (round-to-nearest-even bf16, as torch and Triton use) and
// small wave-level primitives for 64-lane CDNA wavefronts.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <initializer_list>

#include "../../include/uttt_hip.h"

namespace uttt {

// ---------------------------------------------------------------- status ----
void set_error(const char* fmt, ...);
int check_launch(const char* what);
// Zero `bytes` bytes at p on stream st with a fill kernel (graph-capture safe).
int zero_fill_async(void* p, size_t bytes, hipStream_t st, const char* what);

// The one-launch row map (permute.hip) of a contiguous bool mask [B, E, T]
// (element strides s_b, s_e, 1), which also sums a router's per-block balance
// partials part_bal [B, nblk_r, E] into bal_sum [B, E] when part_bal is given.
// src_rows (optional, [B] rows of src_sb entries): the inverse map, src_rows
// [b, row] = the token routed to that row.  Returns false, launching nothing,
// when the shape does not fit it (rowmap_fused_fits: T % 16, T <= 4096,
// E <= 64; and 16-byte aligned mask rows and row map).
bool rowmap_fused_fits(int T, int E);
bool launch_rowmap_fused(const uint8_t* mask, int64_t s_b, int64_t s_e, int B, int T, int E,
                         int32_t* group_sizes, int32_t* row_id_map, const float* part_bal,
                         int nblk_r, float* bal_sum, hipStream_t st, int32_t* src_rows = nullptr,
                         int64_t src_sb = 0);

// Newton-Schulz of BE small matrices [rows, cols] in one launch (one
// workgroup per matrix, the whole computation in LDS; ns_small.hip), for the
// shapes ns_small_fits accepts; g fp32 or bf16 (g_dtype), 16-byte aligned.
bool ns_small_fits(int rows, int cols);
int launch_ns_small(const void* g, int g_dtype, int BE, int rows, int cols, float scale,
                    uint16_t* out, hipStream_t st);

// Per-layer base pointers passed by value as a kernel argument (the
// aggregate uTTT-Dense write reads every layer's own k, v, lr tensors).
constexpr int kMaxLayers = 64;
struct LayerPtrs {
  const void* p[kMaxLayers];
};

#define UTTT_REQUIRE(cond, ...)          \
  do {                                   \
    if (!(cond)) {                       \
      ::uttt::set_error(__VA_ARGS__);    \
      return UTTT_ERR_ARG;               \
    }                                    \
  } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline int dtype_bytes(int dt) {
  switch (dt) {
    case UTTT_F32: return 4;
    case UTTT_BF16: return 2;
    case UTTT_F16: return 2;
    default: return 0;
  }
}

// ------------------------------------------------------------ conversion ----
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// fp32 -> bf16 with the gfx950 hardware conversion (v_cvt_pk_bf16_f32: round
// to nearest even, NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
// Two values as one packed word (a in the low half): one conversion instruction.
typedef __bf16 uttt_bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  const uttt_bf16x2_t v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}
// fp32 -> fp16 with the hardware conversion (round to nearest even).
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// Element traits: storage type and conversions for the three payload dtypes.
struct F32T {
  using S = float;
  static constexpr int code = UTTT_F32;
  __device__ __forceinline__ static float load(S v) { return v; }
  __device__ __forceinline__ static S store(float f) { return f; }
};
struct BF16T {
  using S = uint16_t;
  static constexpr int code = UTTT_BF16;
  __device__ __forceinline__ static float load(S v) { return bf16_to_f32(v); }
  __device__ __forceinline__ static S store(float f) { return f32_to_bf16(f); }
};
struct F16T {
  using S = uint16_t;
  static constexpr int code = UTTT_F16;
  __device__ __forceinline__ static float load(S v) { return f16_to_f32(v); }
  __device__ __forceinline__ static S store(float f) { return f32_to_f16(f); }
};

// Dispatch on a float dtype code: binds TT to the element traits.
#define UTTT_DTYPE_SWITCH_LR(dt, TT, ...)                                           \
  switch (dt) {                                                                     \
    case UTTT_F32: { using TT = ::uttt::F32T; __VA_ARGS__; } break;                 \
    case UTTT_BF16: { using TT = ::uttt::BF16T; __VA_ARGS__; } break;               \
    case UTTT_F16: { using TT = ::uttt::F16T; __VA_ARGS__; } break;                 \
    default: ::uttt::set_error("unsupported dtype code %d", (int)(dt)); return UTTT_ERR_ARG; \
  }

// ------------------------------------------------------------------ wave ----
constexpr int kWave = 64;

__device__ __forceinline__ int lane_id() { return __lane_id(); }

// Number of set bits of `mask` strictly below this lane.
__device__ __forceinline__ int lanes_below(uint64_t mask) {
  return __popcll(mask & ((1ull << lane_id()) - 1ull));
}

}  // namespace uttt
