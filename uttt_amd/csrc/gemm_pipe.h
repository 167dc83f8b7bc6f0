// Asynchronous MFMA GEMM pipeline for gfx950 (the core of every grouped
// fast-weight GEMM).
//
// Workgroup: 256 threads = 4 waves in a 2x2 grid.  Per K step of kBK = 32 a
// workgroup multiplies two 128-row A tiles (A0, A1) by a 256-row B tile (two
// 128-row halves B0, B1) into two fp32 accumulators acc0 = A0 B^T and
// acc1 = A1 B^T (each 128 x 256).  Wave (wm, wn) owns rows [64 wm, 64 wm + 64)
// of both accumulators and columns [128 wn, 128 wn + 128): 2 x 4 blocks of
// 32x32 per accumulator, each fed by v_mfma_f32_32x32x16_bf16 (fp32
// accumulate), i.e. 16 MFMAs per 8 fragment reads.
//
// Global -> LDS: global_load_lds_dwordx4 (16 bytes per lane straight into LDS,
// no register staging) into a ring of five 32 KiB stages (all 160 KiB of LDS),
// so the loads of steps k+1..k+4 are in flight while step k is multiplied; the only waits are
// explicit s_waitcnt vmcnt counts and one s_barrier per step.  Each stage lives
// in its own __shared__ array so the compiler can tell the in-flight LDS
// writes from the LDS reads of the current stage.
//
// LDS tile layouts (16-byte chunks, XOR-swizzled against bank conflicts):
//   KMajor tile (operand stored [rows][K], K contiguous): 128 rows x 4 chunks;
//     chunk c of row r sits at slot r*4 + (c ^ kswz(r)).  Fragments are one
//     ds_read_b128 (8 consecutive k of one row).
//   RMajor tile (operand stored [K][rows], rows contiguous): 32 k-rows x 16
//     chunks; chunk c of k-row k sits at slot k*16 + (c ^ rswz(k)).  Fragments
//     are two ds_read_b64_tr_b16: within a group of 16 lanes, source lane
//     s = 4j + q reads k-row j, rows 4q..4q+3, and the hardware hands lane i
//     the column i of that 4x16 block, i.e. 4 consecutive k of row i.
// Lanes whose chunk lies outside the operand read a 16-byte zero block, so
// partial tiles need no special casing in the MFMA loop.
#pragma once

#include <utility>

#include "common.h"

namespace uttt {
namespace pipe {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kBK = 32;
constexpr int kTileRows = 128;                                   // rows per LDS tile
constexpr int kBRows = 2 * kTileRows;                            // B rows per workgroup
constexpr int kTileBytes = kTileRows * kBK * 2;                  // 8 KiB
constexpr int kStageBytes = 4 * kTileBytes;                      // A0 | A1 | B0 | B1
constexpr int kStages = 5;                                       // LDS ring: 160 KiB
constexpr int kLoadsPerTile = kTileBytes / 16 / kThreads;        // 2 per thread
constexpr int kLoadsPerStage = 4 * kLoadsPerTile;                // 8 per wave
constexpr int kNB = 4;                                           // 32-col blocks per wave
constexpr int kXcds = 8;                                         // MI355X: 8 XCDs, 32 CUs each

enum Major { KMajor = 0, RMajor = 1 };

// 16 zero bytes (zero-initialised device memory, never written): the source
// of every masked-off lane of a tile load.
__device__ __attribute__((aligned(16))) uint4 g_zero16;

#define UTTT_LDS(p) ((__attribute__((address_space(3))) void*)(p))

// Wave index inside the workgroup as a wave-uniform (scalar) value.
__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}

// A pointer that is the same for every lane, marked wave-uniform so that it
// stays in scalar registers (and addresses built from it use the scalar-base
// form of the global loads).
template <class T>
__device__ __forceinline__ T* uniform_ptr(T* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<T*>(((uint64_t)hi << 32) | lo);
}

// s_waitcnt vmcnt(N) leaving the export and LDS counters alone (gfx9
// encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

__device__ __forceinline__ void block_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// A global operand of one group: element (r, k) is at
//   KMajor: base[r * ld + k]      RMajor: base[k * ld + r]
// rows [0, r_end) and k [0, k_end) are valid; the rest reads as zero.
struct Operand {
  const uint16_t* base;
  int64_t ld;
  int r_end;
  int k_end;
};

// Swizzles.  A 16-lane group of ds_read_b128 reads 16 consecutive rows of one
// logical chunk; rows are 64 bytes, so row r sits in quarter (r & 3) of a
// 256-byte bank line and the 4 rows sharing a quarter must use 4 different
// chunk slots: slot = c ^ ((r >> 2) & 3).  A 32-lane half of
// ds_read_b64_tr_b16 reads 4 k-rows x 4 chunks (a 64-byte aligned block) of
// 256-byte rows; XOR with 4 * (k & 3) sends the 4 k-rows to 4 different
// 64-byte blocks of the bank line.
__device__ __forceinline__ int kswz(int r) { return (r >> 2) & 3; }
__device__ __forceinline__ int rswz(int k) { return (k & 3) << 2; }

// Loads of one 128-row x kBK tile of an operand for a whole K loop.  The
// tile origin and its per-step advance are wave-uniform (scalar registers);
// each lane keeps only the 32-bit byte offsets of its kLoadsPerTile chunks, so
// a load is one global_load_lds_dwordx4 with a scalar base and a vector
// offset, and a whole step costs a few scalar instructions.  Rows past the
// operand's end are clamped onto its last valid row (their products land in
// output rows or token columns that are never stored); only the K tail (the
// last step when k_end is not a multiple of kBK) reads zeros for k >= k_end,
// through the masked form.  Steps past the last re-read the last step into a
// stage that is never multiplied.
template <int MAJOR>
struct TileLoader {
  const uint8_t* base;    // wave-uniform: byte address of the tile origin at step 0
  int64_t kstep;          // bytes advanced per K step
  int last;               // last step holding data
  int k_end;
  uint32_t off[kLoadsPerTile];

  __device__ __forceinline__ void init(const Operand& op, int r0) {
    const int lane = threadIdx.x & 63;
    const int w = wave_id();
    k_end = op.k_end;
    last = (op.k_end + kBK - 1) / kBK - 1;
    int nrows = op.r_end - r0;
    const uint16_t* org;
    if (nrows > 0) {
      org = MAJOR == KMajor ? op.base + (int64_t)r0 * op.ld : op.base + r0;
    } else {  // no valid row: read the operand's first rows instead
      org = op.base;
      nrows = MAJOR == KMajor ? 1 : 8;
    }
    base = uniform_ptr(reinterpret_cast<const uint8_t*>(org));
    kstep = MAJOR == KMajor ? (int64_t)kBK * 2 : (int64_t)kBK * op.ld * 2;
#pragma unroll
    for (int t = 0; t < kLoadsPerTile; ++t) {
      const int s = (t * 4 + w) * 64 + lane;
      if constexpr (MAJOR == KMajor) {
        const int r = s >> 2;
        const int c = (s & 3) ^ kswz(r);
        const int rr = r < nrows ? r : nrows - 1;
        off[t] = (uint32_t)(rr * (int)op.ld + c * 8) * 2u;
      } else {
        const int k = s >> 4;
        const int c = (s & 15) ^ rswz(k);
        const int cmax = (nrows >> 3) - 1;
        const int cc = c < cmax ? c : cmax;
        off[t] = (uint32_t)(k * (int)op.ld + cc * 8) * 2u;
      }
    }
  }

  __device__ __forceinline__ int clamp_step(int step) const { return step < last ? step : last; }
  // Wave-uniform address of step `step`'s tile origin.
  __device__ __forceinline__ const uint8_t* step_base(int step) const {
    return uniform_ptr(base + (int64_t)clamp_step(step) * kstep);
  }
  // Whether the loads of `step` need the masked (K tail) form.
  __device__ __forceinline__ bool tail(int step) const {
    return clamp_step(step) == last && (k_end % kBK) != 0;
  }

  // Issue load t of this wave's share of the step at `sb` into LDS tile `dst`.
  template <bool MASKED>
  __device__ __forceinline__ void issue(const uint8_t* sb, int step, int t, uint8_t* dst) const {
    uint8_t* d = dst + (t * 4 + wave_id()) * 64 * 16;
    if constexpr (!MASKED) {
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(sb + off[t]), UTTT_LDS(d), 16,
                                       0, 0);
    } else {
      const int lane = threadIdx.x & 63;
      const int s = (t * 4 + wave_id()) * 64 + lane;
      int kk;
      if constexpr (MAJOR == KMajor) {
        const int r = s >> 2;
        kk = ((s & 3) ^ kswz(r)) * 8;
      } else {
        kk = s >> 4;
      }
      const bool ok = clamp_step(step) * kBK + kk < k_end;
      const uintptr_t src =
          ok ? reinterpret_cast<uintptr_t>(sb + off[t]) : reinterpret_cast<uintptr_t>(&g_zero16);
      __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(src), UTTT_LDS(d), 16, 0, 0);
    }
  }
};

typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

// LDS byte address of a __shared__ pointer.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)((const __attribute__((address_space(3))) void*)p);
}

// The two LDS fragment reads as inline asm.  The compiler's wait-count pass
// does not model these, so it can neither stall them behind in-flight LDS-DMA
// loads nor insert the lgkmcnt wait their consumers need: run_pipeline<kAsm>
// places every wait itself.  "memory" keeps them in program order with the
// loads and barriers.
__device__ __forceinline__ i16x4 ds_tr16_asm(const void* p) {
  i32x2 v;
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(v) : "v"(lds_addr(p)) : "memory");
  return __builtin_bit_cast(i16x4, v);
}
__device__ __forceinline__ bf16x8 ds_b128_asm(const void* p) {
  i32x4 v;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(lds_addr(p)) : "memory");
  return __builtin_bit_cast(bf16x8, v);
}

// MFMA operand fragment of rows [rb, rb+32), k-substep ks (16 k) of an LDS tile.
template <int MAJOR, bool ASM = false>
__device__ __forceinline__ bf16x8 frag(const uint8_t* tile, int rb, int ks) {
  const int lane = threadIdx.x & 63;
  if constexpr (MAJOR == KMajor) {
    const int r = rb + (lane & 31);
    const int c = 2 * ks + (lane >> 5);
    const uint8_t* p = tile + (r * 4 + (c ^ kswz(r))) * 16;
    if constexpr (ASM) return ds_b128_asm(p);
    return *reinterpret_cast<const bf16x8*>(p);
  } else {
    const int g = lane >> 4, s = lane & 15;
    const int j = s >> 2, q = s & 3;
    const int r = rb + 16 * (g & 1) + 4 * q;
    const int c = r >> 3;
    const int kb = 16 * ks + 8 * (g >> 1) + j;
    const int k0 = kb, k1 = kb + 4;
    const uint8_t* p0 = tile + (k0 * 16 + (c ^ rswz(k0))) * 16 + 8 * (q & 1);
    const uint8_t* p1 = tile + (k1 * 16 + (c ^ rswz(k1))) * 16 + 8 * (q & 1);
    i16x4 x0, x1;
    if constexpr (ASM) {
      x0 = ds_tr16_asm(p0);
      x1 = ds_tr16_asm(p1);
    } else {
      x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)(p0));
      x1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)(p1));
    }
    const i16x8 x = __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(bf16x8, x);
  }
}

// Fragments of one k-substep (16 k) of a stage: this wave's 4 column blocks of
// B and its 2 row blocks of A0 / A1.
struct HalfFrags {
  bf16x8 b[kNB], a0[2], a1[2];
};

template <int AMAJ, int BMAJ, bool ASM = false>
__device__ __forceinline__ void read_half(HalfFrags& f, const uint8_t* st, int ks, int wm,
                                          int wn) {
  const uint8_t* a0 = st;
  const uint8_t* a1 = st + kTileBytes;
  const uint8_t* b = st + (2 + wn) * kTileBytes;  // this wave's B half
#pragma unroll
  for (int j = 0; j < kNB; ++j) f.b[j] = frag<BMAJ, ASM>(b, j * 32, ks);
#pragma unroll
  for (int i = 0; i < 2; ++i) f.a0[i] = frag<AMAJ, ASM>(a0, wm * 64 + i * 32, ks);
#pragma unroll
  for (int i = 0; i < 2; ++i) f.a1[i] = frag<AMAJ, ASM>(a1, wm * 64 + i * 32, ks);
}

// LDS instructions of one read_half: a KMajor fragment is one ds_read_b128,
// an RMajor one two ds_read_b64_tr_b16.
template <int AMAJ, int BMAJ>
constexpr int half_lds_ops() {
  return kNB * (BMAJ == KMajor ? 1 : 2) + 4 * (AMAJ == KMajor ? 1 : 2);
}

// s_waitcnt on the LDS counter that the compiler must treat as redefining the
// fragment registers, so no MFMA reading them can move above it.
template <int N>
__device__ __forceinline__ void lgkm_wait_tied(HalfFrags& f) {
  i32x4 r[8] = {__builtin_bit_cast(i32x4, f.b[0]),  __builtin_bit_cast(i32x4, f.b[1]),
                __builtin_bit_cast(i32x4, f.b[2]),  __builtin_bit_cast(i32x4, f.b[3]),
                __builtin_bit_cast(i32x4, f.a0[0]), __builtin_bit_cast(i32x4, f.a0[1]),
                __builtin_bit_cast(i32x4, f.a1[0]), __builtin_bit_cast(i32x4, f.a1[1])};
  asm volatile("s_waitcnt lgkmcnt(%8)"
               : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]), "+v"(r[4]), "+v"(r[5]),
                 "+v"(r[6]), "+v"(r[7])
               : "i"(N)
               : "memory");
  f.b[0] = __builtin_bit_cast(bf16x8, r[0]);
  f.b[1] = __builtin_bit_cast(bf16x8, r[1]);
  f.b[2] = __builtin_bit_cast(bf16x8, r[2]);
  f.b[3] = __builtin_bit_cast(bf16x8, r[3]);
  f.a0[0] = __builtin_bit_cast(bf16x8, r[4]);
  f.a0[1] = __builtin_bit_cast(bf16x8, r[5]);
  f.a1[0] = __builtin_bit_cast(bf16x8, r[6]);
  f.a1[1] = __builtin_bit_cast(bf16x8, r[7]);
}

// f(std::integral_constant<int, i>) for i = 0 .. N-1 with compile-time i, so
// that accumulator indices stay constants whatever the unroller decides (a
// runtime index would move the accumulator arrays to scratch memory).
template <class F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
  (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// acc_a[i][j] += A_a(wave rows i) * B(wave cols j) over one k-substep, a = 0, 1.
__device__ __forceinline__ void mma_half(f32x16 (&acc0)[2][kNB], f32x16 (&acc1)[2][kNB],
                                         const HalfFrags& f) {
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < kNB; ++j)
      acc0[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a0[i], f.b[j], acc0[i][j], 0, 0, 0);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < kNB; ++j)
      acc1[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a1[i], f.b[j], acc1[i][j], 0, 0, 0);
}

// The same 16 MFMAs with between(p) (p = 0 .. 7, a compile-time constant)
// issued after MFMAs 2p and 2p+1, each in its own scheduling region: the wave
// issues the work of `between` while the matrix core is busy.
template <class Between>
__device__ __forceinline__ void mma_half(f32x16 (&acc0)[2][kNB], f32x16 (&acc1)[2][kNB],
                                         const HalfFrags& f, Between&& between) {
  static_for<16>([&](auto I) __attribute__((always_inline)) {
    constexpr int a = decltype(I)::value / 8;
    constexpr int i = (decltype(I)::value / 4) % 2;
    constexpr int j = decltype(I)::value % 4;
    if constexpr (a == 0)
      acc0[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a0[i], f.b[j], acc0[i][j], 0, 0, 0);
    else
      acc1[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a1[i], f.b[j], acc1[i][j], 0, 0, 0);
    if constexpr (decltype(I)::value % 2 == 1) {
      __builtin_amdgcn_sched_barrier(0);
      between(std::integral_constant<int, decltype(I)::value / 2>{});
      __builtin_amdgcn_sched_barrier(0);
    }
  });
}

// The K loop: a ring of kStages LDS stages; the loads of step kt+kStages are
// issued during step kt, so kStages-1 steps are in flight while one is
// multiplied (four stages, 128 KiB, cover the L2-miss latency seen under
// load; three did not).
//   prep(kt)                 readies the loads of step kt (operand switch,
//                            per-step scalar bases) and returns whether they
//                            need the masked (K tail) form
//   issue(p, masked, stage)  issues load p (0 .. kLoadsPerStage-1, a constant)
//                            of the prepared step into `stage`
//   read(stage, ks, frags)   the fragment reads of k-substep ks, inline asm,
//                            NLDS LDS instructions
// Step kt (stage cur, next stage nxt):
//   read (kt, 1) -> f1;  prep(kt + kStages);  wait for f0;  MFMAs of f0
//   wait for this wave's loads of stage kt+1 and for f1, barrier (stage kt+1
//   has landed for every wave, and every wave is done reading stage kt)
//   read (kt+1, 0) -> f0;  MFMAs of f1 with the loads of step kt+kStages
//   into stage cur interleaved between them
// so with one wave per SIMD the matrix core is fed while the next fragments
// and the next stage arrive.  The fragment reads are inline asm because the
// compiler's wait-count pass cannot tell them from the in-flight LDS-DMA
// writes and would drain every load (vmcnt(0)) or every read (lgkmcnt(0))
// in front of them; every wait here is explicit.  Before the MFMAs of f0 the
// NLDS reads of f1 are the only younger LDS operations, so lgkmcnt(min(NLDS,
// 15)) leaves f0 complete (any other LGKM operation only makes it stricter).
template <int NLDS, class PrepFn, class IssueFn, class ReadFn>
__device__ __forceinline__ void run_pipeline(int nk, PrepFn&& prep, IssueFn&& issue, ReadFn&& read,
                                             f32x16 (&acc0)[2][kNB], f32x16 (&acc1)[2][kNB],
                                             uint8_t* const (&ring)[kStages]) {
  if (nk <= 0) return;
  constexpr int kW = NLDS < 15 ? NLDS : 15;
  HalfFrags f0, f1;
  auto load_all = [&](int kt, uint8_t* st) __attribute__((always_inline)) {
    if (prep(kt))
      static_for<kLoadsPerStage>([&](auto p) __attribute__((always_inline)) {
        issue(p, std::true_type{}, st);
      });
    else
      static_for<kLoadsPerStage>([&](auto p) __attribute__((always_inline)) {
        issue(p, std::false_type{}, st);
      });
  };
  static_for<kStages>([&](auto i) __attribute__((always_inline)) { load_all(i, ring[i]); });
  wait_vmcnt<(kStages - 1) * kLoadsPerStage>();
  block_barrier();
  read(ring[0], 0, f0);
  auto step = [&](int kt, uint8_t* cur, const uint8_t* nxt) __attribute__((always_inline)) {
    read(cur, 1, f1);
    const bool masked = prep(kt + kStages);
    lgkm_wait_tied<kW>(f0);
    mma_half(acc0, acc1, f0);
    __builtin_amdgcn_sched_barrier(0);
    wait_vmcnt<(kStages - 2) * kLoadsPerStage>();
    lgkm_wait_tied<0>(f1);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    read(nxt, 0, f0);
    // the rare K-tail step issues its masked loads up front; otherwise the
    // loads ride between the MFMAs (branches hold loads only, so the
    // accumulators never meet at a join)
    if (masked)
      static_for<kLoadsPerStage>([&](auto p) __attribute__((always_inline)) {
        issue(p, std::true_type{}, cur);
      });
    __builtin_amdgcn_sched_barrier(0);
    mma_half(acc0, acc1, f1, [&](auto p) __attribute__((always_inline)) {
      if (!masked) issue(p, std::false_type{}, cur);
    });
    __builtin_amdgcn_sched_barrier(0);
  };
  int kt = 0;
  for (; kt + kStages <= nk; kt += kStages)
    static_for<kStages>([&](auto i) __attribute__((always_inline)) {
      step(kt + i, ring[i], ring[(i + 1) % kStages]);
    });
  static_for<kStages - 1>([&](auto i) __attribute__((always_inline)) {
    if (kt + i < nk) step(kt + i, ring[i], ring[(i + 1) % kStages]);
  });
  lgkm_wait_tied<0>(f0);  // the reads of the stage past the end
  wait_vmcnt<0>();        // and the loads issued past the end
}

template <int M, int N>
__device__ __forceinline__ void zero(f32x16 (&acc)[M][N]) {
#pragma unroll
  for (int i = 0; i < M; ++i)
#pragma unroll
    for (int j = 0; j < N; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
}

// Row (M) of accumulator element v of this lane inside its 32x32 block is
// 8*(v/4) + 4*(lane/32) + v%4; its column (N) is lane%32.
__device__ __forceinline__ int acc_row(int v) {
  return 8 * (v >> 2) + 4 * ((threadIdx.x & 63) >> 5) + (v & 3);
}
__device__ __forceinline__ int acc_col() { return threadIdx.x & 31; }

// ------------------------------------------------------------ scheduling ----
// Token-grouped problems (N = routed tokens): the tokens of expert e in batch
// b occupy [off(b,e), off(b,e)+g(b,e)) of that batch.  The grid covers an
// upper bound of ceil(N/BN) + E n-tiles per batch; each workgroup finds its
// (expert, n-tile) with a wave-level scan of group_sizes[b] and leaves if its
// tile index is past the batch's real tile count.  Segments are clamped to
// [0, N), so a group_sizes row that over-counts (the reference does not check
// sum == N) can never move a tile outside the token buffer.
struct TokenTile {
  int e;       // expert, or -1 when the workgroup has no tile
  int start;   // first token of the expert's segment
  int size;    // segment length
  int n0;      // first token of this tile, relative to the segment
};

template <int BN>
__device__ TokenTile find_token_tile(const int32_t* __restrict__ gs_b, int E, int N, int tile,
                                     int* s_scratch /* >= 4 ints */) {
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    int tok_base = 0, tile_base = 0;
    int found_e = -1, found_start = 0, found_size = 0, found_n0 = 0;
    for (int e0 = 0; e0 < E; e0 += 64) {
      const int e = e0 + lane;
      const int graw = e < E ? gs_b[e] : 0;
      const int g = graw > 0 ? graw : 0;
      int tok_incl = g;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const int a = __shfl_up(tok_incl, d, 64);
        if (lane >= d) tok_incl += a;
      }
      const int start = tok_base + tok_incl - g;
      const int avail = start < N ? N - start : 0;
      const int gc = g < avail ? g : avail;
      const int nt = (gc + BN - 1) / BN;
      int tile_incl = nt;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const int b = __shfl_up(tile_incl, d, 64);
        if (lane >= d) tile_incl += b;
      }
      const int tile_excl = tile_base + tile_incl - nt;
      const bool hit = e < E && tile >= tile_excl && tile < tile_excl + nt;
      const uint64_t bal = __ballot(hit);
      if (bal != 0ull) {
        const int src = __ffsll((unsigned long long)bal) - 1;
        found_e = e0 + src;
        found_start = __shfl(start, src, 64);
        found_size = __shfl(gc, src, 64);
        found_n0 = (tile - __shfl(tile_excl, src, 64)) * BN;
        break;
      }
      tok_base += __shfl(tok_incl, 63, 64);
      tile_base += __shfl(tile_incl, 63, 64);
    }
    if (lane == 0) {
      s_scratch[0] = found_e;
      s_scratch[1] = found_start;
      s_scratch[2] = found_size;
      s_scratch[3] = found_n0;
    }
  }
  __syncthreads();
  // wave-uniform: the tile origins built from these live in scalar registers
  return TokenTile{__builtin_amdgcn_readfirstlane(s_scratch[0]),
                   __builtin_amdgcn_readfirstlane(s_scratch[1]),
                   __builtin_amdgcn_readfirstlane(s_scratch[2]),
                   __builtin_amdgcn_readfirstlane(s_scratch[3])};
}

// Segment [start, start+size) of expert e in batch b, clamped to [0, N).
__device__ __forceinline__ void expert_segment(const int32_t* __restrict__ gs_b, int e, int N,
                                               int* start, int* size) {
  int s = 0;
  for (int i = 0; i < e; ++i) s += gs_b[i] > 0 ? gs_b[i] : 0;
  int g = gs_b[e] > 0 ? gs_b[e] : 0;
  if (s > N) s = N;
  if (g > N - s) g = N - s;
  *start = s;
  *size = g;
}

// Logistic sigmoid with the hardware exp and reciprocal (about 1 ulp of fp32
// each, far below the bf16 resolution of every output built from it).
__device__ __forceinline__ float sigmoidf_(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __expf(-x));
}
__device__ __forceinline__ float bf16r(float x) { return bf16_to_f32(f32_to_bf16(x)); }

// Four consecutive-row results (rows m..m+3 of token column n) as one store
// into a token-major [.., N, ld] buffer (m a multiple of 4).
__device__ __forceinline__ void store4(uint16_t* out, int64_t ld, int64_t n, int m, float a,
                                       float b, float c, float d) {
  uint2 w;
  w.x = pack_bf16x2(a, b);
  w.y = pack_bf16x2(c, d);
  *reinterpret_cast<uint2*>(out + n * ld + m) = w;
}
__device__ __forceinline__ void store4(float* out, int64_t ld, int64_t n, int m, float a, float b,
                                       float c, float d) {
  *reinterpret_cast<float4*>(out + n * ld + m) = make_float4(a, b, c, d);
}
__device__ __forceinline__ void load4(const uint16_t* in, int64_t ld, int64_t n, int m,
                                      float* v) {
  const uint2 w = *reinterpret_cast<const uint2*>(in + n * ld + m);
  v[0] = bf16_to_f32((uint16_t)(w.x & 0xffffu));
  v[1] = bf16_to_f32((uint16_t)(w.x >> 16));
  v[2] = bf16_to_f32((uint16_t)(w.y & 0xffffu));
  v[3] = bf16_to_f32((uint16_t)(w.y >> 16));
}
__device__ __forceinline__ void load4(const float* in, int64_t ld, int64_t n, int m, float* v) {
  const float4 f = *reinterpret_cast<const float4*>(in + n * ld + m);
  v[0] = f.x;
  v[1] = f.y;
  v[2] = f.z;
  v[3] = f.w;
}

}  // namespace pipe
}  // namespace uttt
