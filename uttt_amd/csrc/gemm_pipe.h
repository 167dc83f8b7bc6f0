// Asynchronous MFMA GEMM pipeline for gfx950 (the core of every grouped
// fast-weight GEMM).
//
// Per K step of kBK = 64 a workgroup multiplies two 128-row A tiles (A0, A1)
// by a 256-row B tile (two 128-row halves B0, B1) into two fp32 accumulators
// acc0 = A0 B^T and acc1 = A1 B^T (each 128 x 256), with
// v_mfma_f32_32x32x16_bf16 (fp32 accumulate) on 32x32 blocks.  Two wave
// layouts, NA = the 32-row blocks of each A tile that one wave owns:
//   NA = 2: 256 threads = 4 waves (one per SIMD) in a 2x2 grid; wave
//     (wm, wn) owns rows [64 wm, 64 wm + 64) of both accumulators and columns
//     [128 wn, 128 wn + 128): 2 x 4 blocks per accumulator, 256 fp32
//     accumulators per lane; per k-substep 16 MFMAs per 8 fragment reads.
//   NA = 1: 512 threads = 8 waves (two per SIMD) in a 4x2 grid; wave (wm, wn)
//     owns rows [32 wm, 32 wm + 32) and the same 128 columns: 1 x 4 blocks
//     per accumulator, 128 accumulators per lane; per k-substep 8 MFMAs per
//     6 fragment reads.  A SIMD holds two waves, so one wave's MFMAs run
//     while the other waits on its reads, loads or barrier.
//
// Global -> LDS: buffer_load_dwordx4 ... lds (16 bytes per lane straight into
// LDS, no register staging) into two 64 KiB stages (kBK = 64), the loads of stage
// k+1 in flight while stage k is multiplied; the only waits are
// explicit s_waitcnt vmcnt counts and one s_barrier per step.  Each stage lives
// in its own __shared__ array so the compiler can tell the in-flight LDS
// writes from the LDS reads of the current stage.
//
// LDS tile layouts (16-byte chunks, XOR-swizzled against bank conflicts):
//   KMajor tile (operand stored [rows][K], K contiguous): 128 rows x 8 chunks;
//     chunk c of row r sits at slot r*8 + (c ^ kswz(r)).  Fragments are one
//     ds_read_b128 (8 consecutive k of one row).
//   RMajor tile (operand stored [K][rows], rows contiguous): 64 k-rows x 16
//     chunks; chunk c of k-row k sits at slot k*16 + (c ^ rswz(k)).  Fragments
//     are two ds_read_b64_tr_b16: within a group of 16 lanes, source lane
//     s = 4j + q reads k-row j, rows 4q..4q+3, and the hardware hands lane i
//     the column i of that 4x16 block, i.e. 4 consecutive k of row i.
// Lanes whose chunk lies at or past the operand's K end load zeros (the
// buffer descriptor's record bound), so partial tiles need no special casing
// in the MFMA loop.
#pragma once

#include <utility>

#include "common.h"

namespace uttt {
namespace pipe {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;                                    // NA = 2 layout (and APPLY)
constexpr int kBK = 64;
constexpr int kTileRows = 128;                                   // rows per LDS tile
constexpr int kBRows = 2 * kTileRows;                            // B rows per workgroup
constexpr int kTileBytes = kTileRows * kBK * 2;                  // 16 KiB
constexpr int kStageBytes = 4 * kTileBytes;                      // A0 | A1 | B0 | B1
constexpr int kStages = 2;                                       // LDS ring: 128 KiB
constexpr int kChunks = kBK / 8;                                 // 16-byte chunks per KMajor row
constexpr int kSubsteps = kBK / 16;                              // MFMA k-substeps per stage
constexpr int kLoadsPerTile = kTileBytes / 16 / kThreads;        // 4 per thread
constexpr int kLoadsPerStage = 4 * kLoadsPerTile;                // 16 per wave
constexpr int kNB = 4;                                           // 32-col blocks per wave
constexpr int kXcds = 8;                                         // MI355X: 8 XCDs, 32 CUs each

// Wave layout NA (see above): waves, threads, and LDS-DMA loads per thread
// per tile and per stage.
template <int NA> constexpr int kWavesOf = 8 / NA;
template <int NA> constexpr int kThreadsOf = 64 * kWavesOf<NA>;
template <int NA> constexpr int kLoadsPerTileOf = kTileBytes / 16 / kThreadsOf<NA>;
template <int NA> constexpr int kLoadsPerStageOf = 4 * kLoadsPerTileOf<NA>;
// Staged-epilogue items (token, 8-row group) per thread per 64-token quarter.
template <int NA> constexpr int kItemsOf = 64 * 16 / kThreadsOf<NA>;

enum Major { KMajor = 0, RMajor = 1 };

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
// logical chunk; KMajor rows are 128 bytes (one cache line of the operand), so
// row r sits in half (r & 1) of a 256-byte bank line and the 8 rows sharing a
// half must use 8 different chunk slots: slot = c ^ ((r >> 1) & 7).  A 32-lane
// half of ds_read_b64_tr_b16 reads 4 k-rows x 4 chunks (a 64-byte aligned
// block) of 256-byte rows; XOR with 4 * (k & 3) sends the 4 k-rows to 4
// different 64-byte blocks of the bank line.
__device__ __forceinline__ int kswz(int r) { return (r >> 1) & 7; }
__device__ __forceinline__ int rswz(int k) { return (k & 3) << 2; }

// Loads of one 128-row x kBK tile of an operand for a whole K loop, as
// buffer-form LDS-DMA (buffer_load_dwordx4 ... lds: 16 bytes per lane from a
// scalar descriptor plus the lane's 32-bit offset, straight into LDS at
// M0 + 16 * lane).  The tile origin and its per-step advance are wave-uniform;
// each lane keeps only the byte offsets of its kLoadsPerTile chunks, so a load
// costs a few scalar instructions and no vector ones.  Rows past the
// operand's end are clamped onto its last valid row (their products land in
// output rows or token columns that are never stored).  Every k >= k_end reads
// as zero through the descriptor's record bound (out-of-range lanes of a
// buffer load return zeros and touch no memory), so every step issues the
// same loads:
//   - each step past the last (the K loop runs whole ring iterations and
//     issues ahead of the end): no records at all;
//   - the K tail of an RMajor operand (k-rows contiguous): the bound ends at
//     the first k-row past k_end;
//   - the K tail of a KMajor operand (k contiguous inside a row): the lanes
//     whose chunk lies at or past k_end get bit 31 set in their offset and
//     the bound is 2^31 (offsets of valid chunks stay below it: rows of at
//     most 2^23 elements).
// Word 3 of a raw buffer descriptor on gfx9 (32-bit data format, no swizzle).
constexpr int kBufferWord3 = 0x00020000;
typedef __amdgpu_buffer_rsrc_t Rsrc;

// NW: the workgroup's waves (each lane of each wave loads kLPT chunks of a tile).
template <int MAJOR, int NW = 4>
struct TileLoader {
  static constexpr int kLPT = kTileBytes / 16 / (64 * NW);
  static_assert(kLPT >= 1 && kLPT <= kLoadsPerTile, "4 or 8 waves");
  const uint8_t* base;    // wave-uniform: byte address of the tile origin at step 0
  int64_t kstep;          // bytes advanced per K step
  int last;               // last step holding data
  int k_end;
  int nvalid;             // valid rows from the tile origin (KMajor: rows of 8 per load)
  int ld2;                // RMajor: bytes per k-row of the operand
  int col2;               // RMajor: byte offset of the tile origin inside its k-row
  // kLPT entries used; the array has a fixed bound (a bound that depends on
  // NW made hipcc's host pass reject later uses of the loader's functions)
  uint32_t off[kLoadsPerTile];
  int wofs;               // wave-uniform: this wave's LDS byte offset inside a tile

  __device__ __forceinline__ void init(const Operand& op, int r0) {
    const int lane = threadIdx.x & 63;
    const int w = wave_id();
    k_end = op.k_end;
    last = (op.k_end + kBK - 1) / kBK - 1;
    int nrows = op.r_end - r0;
    nvalid = nrows > 0 ? nrows : 0;
    // kept in a scalar register for the whole loop (opaque, so not re-derived
    // from the thread id before every load)
    wofs = w * 64 * 16;
    asm volatile("" : "+s"(wofs));
    ld2 = (int)op.ld * 2;
    const uint16_t* org;
    if (nrows > 0) {
      org = MAJOR == KMajor ? op.base + (int64_t)r0 * op.ld : op.base + r0;
      col2 = r0 * 2;
    } else {  // no valid row: read the operand's first rows instead
      org = op.base;
      nrows = MAJOR == KMajor ? 1 : 8;
      col2 = 0;
    }
    base = uniform_ptr(reinterpret_cast<const uint8_t*>(org));
    kstep = MAJOR == KMajor ? (int64_t)kBK * 2 : (int64_t)kBK * op.ld * 2;
#pragma unroll
    for (int t = 0; t < kLPT; ++t) {
      const int s = (t * NW + w) * 64 + lane;
      if constexpr (MAJOR == KMajor) {
        const int r = s / kChunks;
        const int c = (s % kChunks) ^ kswz(r);
        const int rr = r < nrows ? r : nrows - 1;
        off[t] = (uint32_t)(rr * (int)op.ld + c * 8) * 2u;
      } else {
        const int k = s >> 4;
        const int c = (s & 15) ^ rswz(k);
        const int cmax = (nrows >> 3) - 1;
        const int cc = c < cmax ? c : cmax;
        off[t] = (uint32_t)(k * (int)op.ld + cc * 8) * 2u;
      }
      asm volatile("" : "+v"(off[t]));
    }
  }

  // KMajor rows gathered through a row index: tile row r is row idx[r] of the
  // operand at `org` (rows of ld elements, k < k_end valid), for r < nrows
  // (nrows >= 1); later rows repeat row idx[nrows - 1], as init clamps them.
  // An index outside [0, rows_total) reads row rows_total - 1 (never out of
  // bounds).  Offsets stay 32-bit: rows_total rows of ld elements are below
  // 2^30 elements.
  __device__ __forceinline__ void init_gather(const uint16_t* org, int64_t ld, int k_end_,
                                              const int32_t* __restrict__ idx, int nrows,
                                              int rows_total) {
    static_assert(MAJOR == KMajor, "gathered rows are KMajor token rows");
    const int lane = threadIdx.x & 63;
    const int w = wave_id();
    k_end = k_end_;
    last = (k_end + kBK - 1) / kBK - 1;
    nvalid = nrows;
    wofs = w * 64 * 16;
    asm volatile("" : "+s"(wofs));
    ld2 = (int)ld * 2;
    col2 = 0;
    base = uniform_ptr(reinterpret_cast<const uint8_t*>(org));
    kstep = (int64_t)kBK * 2;
#pragma unroll
    for (int t = 0; t < kLPT; ++t) {
      const int s = (t * NW + w) * 64 + lane;
      const int r = s / kChunks;
      const int c = (s % kChunks) ^ kswz(r);
      const uint32_t ix = (uint32_t)idx[r < nrows ? r : nrows - 1];
      const int row = ix < (uint32_t)rows_total ? (int)ix : rows_total - 1;
      off[t] = (uint32_t)(row * (int)ld + c * 8) * 2u;
      asm volatile("" : "+v"(off[t]));
    }
  }

  __device__ __forceinline__ int clamp_step(int step) const { return step < last ? step : last; }

  // The descriptor of step `step` (call once per step, in step order: the
  // KMajor K tail marks its out-of-range lanes for the steps after it too,
  // which have no records anyway).
  __device__ __forceinline__ Rsrc rsrc(int step) {
    const uint8_t* sb = uniform_ptr(base + (int64_t)clamp_step(step) * kstep);
    uint32_t recs = 0xFFFFFFFFu;
    if (step > last) {
      recs = 0;
    } else if (step == last && (k_end % kBK) != 0) {
      if constexpr (MAJOR == RMajor) {
        recs = (uint32_t)((k_end - step * kBK) * ld2 - col2);
      } else {
        recs = 0x80000000u;
        const int lane = threadIdx.x & 63, w = wofs >> 10, kt = k_end % kBK;
#pragma unroll
        for (int t = 0; t < kLPT; ++t) {
          const int sl = (t * NW + w) * 64 + lane;
          const int r = sl / kChunks;
          const int c = (sl % kChunks) ^ kswz(r);
          if (c * 8 >= kt) off[t] |= 0x80000000u;
        }
      }
    }
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(sb), (short)0, (int)recs,
                                             kBufferWord3);
  }

  // Issue load t of this wave's share of a step (descriptor rs) into LDS tile
  // `dst`.  issue_rows (KMajor token tiles of the APPLY products): a load whose
  // 8 rows all lie past the valid rows is not issued; its LDS slots keep stale
  // values, which only reach the products of token columns that are never
  // stored.  Fewer loads per stage than kLoadsPerStage: the pipeline then
  // waits on vmcnt(0) wherever it would count loads.
  __device__ __forceinline__ void issue(const Rsrc& rs, int t, uint8_t* dst) const {
    uint8_t* d = dst + t * NW * 64 * 16 + wofs;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, UTTT_LDS(d), 16, off[t], 0, 0, 0);
  }
  __device__ __forceinline__ void issue_rows(const Rsrc& rs, int t, uint8_t* dst) const {
    static_assert(MAJOR == KMajor, "row skipping is for KMajor token tiles");
    if (t * NW * (64 / kChunks) + (wofs >> 7) >= nvalid) return;  // wave-uniform
    issue(rs, t, dst);
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
template <int OFF>
__device__ __forceinline__ i16x4 ds_tr16_asm(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset field");
  i32x2 v;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF) : "memory");
  return __builtin_bit_cast(i16x4, v);
}
template <int OFF>
__device__ __forceinline__ bf16x8 ds_b128_asm(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset field");
  i32x4 v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF) : "memory");
  return __builtin_bit_cast(bf16x8, v);
}

// Fragment addressing.  An MFMA operand fragment covers 32 rows (rb a
// multiple of 32) and one k-substep KS (16 k) of an LDS tile.
//   KMajor: lane l reads row rb + l%32, chunk 2 KS + l/32; the XOR key
//     kswz(row) = kswz(l%32) does not depend on rb, so the fragments of all
//     row blocks share one lane offset and differ by rb * 128 bytes (an
//     immediate offset of the read).
//   RMajor: the lane's two reads sit at k-rows k0 and k0 + 4 of the substep;
//     rswz(k0) does not depend on KS, so substep KS adds KS * 16 k-rows
//     (4096 bytes) and the second read 1024 bytes, both immediates.
// So a substep's reads need one address register per tile (KMajor) or per
// row block (RMajor) and everything else is an immediate offset.
template <int KS>
__device__ __forceinline__ uint32_t kmaj_lane() {
  const int lane = threadIdx.x & 63;
  const int r = lane & 31;
  const int c = 2 * KS + (lane >> 5);
  return (uint32_t)((r * kChunks + (c ^ kswz(r))) * 16);
}
__device__ __forceinline__ uint32_t rmaj_lane(int rb) {
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, s = lane & 15;
  const int j = s >> 2, q = s & 3;
  const int r = rb + 16 * (g & 1) + 4 * q;
  const int c = r >> 3;
  const int k0 = 8 * (g >> 1) + j;
  return (uint32_t)((k0 * 16 + (c ^ rswz(k0))) * 16 + 8 * (q & 1));
}
template <int MAJOR, int KS, int OFF>
__device__ __forceinline__ bf16x8 frag_at(uint32_t base) {
  if constexpr (MAJOR == KMajor) {
    return ds_b128_asm<OFF>(base);
  } else {
    const i16x4 x0 = ds_tr16_asm<OFF + KS * 4096>(base);
    const i16x4 x1 = ds_tr16_asm<OFF + KS * 4096 + 1024>(base);
    const i16x8 x = __builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(bf16x8, x);
  }
}

// Fragments of one k-substep (16 k) of a stage: this wave's 4 column blocks of
// B and its NA row blocks of A0 / A1.
template <int NA>
struct HalfFrags {
  bf16x8 b[kNB], a0[NA], a1[NA];
};

// ONLY >= 0: fragment ONLY alone (0 .. NB-1: B blocks, then a0[0], a1[0], a0[1], a1[1]
// for NA = 2, a0[0], a1[0] for NA = 1).
template <int AMAJ, int BMAJ, int KS, int NB = kNB, int ONLY = -1, int NA = 2>
__device__ __forceinline__ void read_half(HalfFrags<NA>& f, const uint8_t* st, int wm, int wn) {
  constexpr int kRow = kChunks * 16;  // bytes per KMajor tile row
  const uint32_t s = lds_addr(st);
  const uint32_t sb = s + (2 + wn) * kTileBytes;  // this wave's B half
  if constexpr (BMAJ == KMajor) {
    const uint32_t b = sb + kmaj_lane<KS>();
    static_for<NB>([&](auto J) __attribute__((always_inline)) {
      if constexpr (ONLY < 0 || ONLY == decltype(J)::value)
        f.b[J] = frag_at<KMajor, KS, decltype(J)::value * 32 * kRow>(b);
    });
  } else {
    static_for<NB>([&](auto J) __attribute__((always_inline)) {
      if constexpr (ONLY < 0 || ONLY == decltype(J)::value)
        f.b[J] = frag_at<RMajor, KS, 0>(sb + rmaj_lane(decltype(J)::value * 32));
    });
  }
  if constexpr (AMAJ == KMajor) {
    const uint32_t a = s + wm * 32 * NA * kRow + kmaj_lane<KS>();
    static_for<NA>([&](auto I) __attribute__((always_inline)) {
      constexpr int i = decltype(I)::value;
      if constexpr (ONLY < 0 || ONLY == NB + 2 * i)
        f.a0[I] = frag_at<KMajor, KS, i * 32 * kRow>(a);
      if constexpr (ONLY < 0 || ONLY == NB + 2 * i + 1)
        f.a1[I] = frag_at<KMajor, KS, kTileBytes + i * 32 * kRow>(a);
    });
  } else {
    static_for<NA>([&](auto I) __attribute__((always_inline)) {
      constexpr int i = decltype(I)::value;
      if constexpr (ONLY < 0 || ONLY == NB + 2 * i || ONLY == NB + 2 * i + 1) {
        const uint32_t a = s + rmaj_lane(wm * 32 * NA + i * 32);
        if constexpr (ONLY < 0 || ONLY == NB + 2 * i) f.a0[I] = frag_at<RMajor, KS, 0>(a);
        if constexpr (ONLY < 0 || ONLY == NB + 2 * i + 1)
          f.a1[I] = frag_at<RMajor, KS, kTileBytes>(a);
      }
    });
  }
}

// LDS instructions of one read_half: a KMajor fragment is one ds_read_b128,
// an RMajor one two ds_read_b64_tr_b16.
template <int AMAJ, int BMAJ, int NB = kNB, int NA = 2>
constexpr int half_lds_ops() {
  return NB * (BMAJ == KMajor ? 1 : 2) + 2 * NA * (AMAJ == KMajor ? 1 : 2);
}

// s_waitcnt on the LDS counter that the compiler must treat as redefining the
// fragment registers, so no MFMA reading them can move above it.
template <int N>
__device__ __forceinline__ void lgkm_wait_tied(HalfFrags<2>& f) {
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
template <int N>
__device__ __forceinline__ void lgkm_wait_tied(HalfFrags<1>& f) {
  i32x4 r[6] = {__builtin_bit_cast(i32x4, f.b[0]),  __builtin_bit_cast(i32x4, f.b[1]),
                __builtin_bit_cast(i32x4, f.b[2]),  __builtin_bit_cast(i32x4, f.b[3]),
                __builtin_bit_cast(i32x4, f.a0[0]), __builtin_bit_cast(i32x4, f.a1[0])};
  asm volatile("s_waitcnt lgkmcnt(%6)"
               : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]), "+v"(r[4]), "+v"(r[5])
               : "i"(N)
               : "memory");
  f.b[0] = __builtin_bit_cast(bf16x8, r[0]);
  f.b[1] = __builtin_bit_cast(bf16x8, r[1]);
  f.b[2] = __builtin_bit_cast(bf16x8, r[2]);
  f.b[3] = __builtin_bit_cast(bf16x8, r[3]);
  f.a0[0] = __builtin_bit_cast(bf16x8, r[4]);
  f.a1[0] = __builtin_bit_cast(bf16x8, r[5]);
}

// MFMAs per k-substep and wave: both accumulators x NA row blocks x kNB
// column blocks.
template <int NA> constexpr int kMmaOf = 2 * NA * kNB;

// acc_a[i][j] += A_a(wave rows i) * B(wave cols j) over one k-substep, a = 0, 1.
// MFMA q of a substep: the 2 NA of column block 0 first, then the others,
// which a wave whose block 0 already covers every token of its columns skips
// (`full` false: small experts' tiles under skewed routing).  The fragment
// reads are the same either way, so every wait count holds on both paths.
// (Without skipping, the order is accumulator-major: consecutive MFMAs share
// their A fragment.)
template <int Q, bool SKIP, int NA>
__device__ __forceinline__ void mma_q(f32x16 (&acc0)[NA][kNB], f32x16 (&acc1)[NA][kNB],
                                      const HalfFrags<NA>& f) {
  constexpr int j = SKIP ? Q / (2 * NA) : Q % kNB;
  constexpr int a = SKIP ? (Q % (2 * NA)) / NA : Q / (kNB * NA);
  constexpr int i = SKIP ? Q % NA : (Q / kNB) % NA;
  if constexpr (a == 0)
    acc0[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a0[i], f.b[j], acc0[i][j], 0, 0, 0);
  else
    acc1[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a1[i], f.b[j], acc1[i][j], 0, 0, 0);
}

template <bool SKIP, int NA>
__device__ __forceinline__ void mma_half(f32x16 (&acc0)[NA][kNB], f32x16 (&acc1)[NA][kNB],
                                         const HalfFrags<NA>& f, bool full) {
  static_for<2 * NA>([&](auto Q) __attribute__((always_inline)) { mma_q<Q, SKIP>(acc0, acc1, f); });
  if (!SKIP || full)
    static_for<kMmaOf<NA> - 2 * NA>([&](auto Q) __attribute__((always_inline)) {
      mma_q<2 * NA + decltype(Q)::value, SKIP>(acc0, acc1, f);
    });
}

// The same MFMAs with between(q) (a compile-time constant, 0 .. kMmaOf - 1)
// issued after MFMA q, each in its own scheduling region: the wave issues the
// work of `between` while the matrix core is busy; without the skipped MFMAs,
// their slots' work is issued back to back.
template <bool SKIP, int NA, class Between>
__device__ __forceinline__ void mma_half(f32x16 (&acc0)[NA][kNB], f32x16 (&acc1)[NA][kNB],
                                         const HalfFrags<NA>& f, bool full, Between&& between) {
  constexpr int kFirst = 2 * NA;
  static_for<kFirst>([&](auto Q) __attribute__((always_inline)) {
    mma_q<Q, SKIP>(acc0, acc1, f);
    __builtin_amdgcn_sched_barrier(0);
    between(Q);
    __builtin_amdgcn_sched_barrier(0);
  });
  if (!SKIP || full) {
    static_for<kMmaOf<NA> - kFirst>([&](auto Q) __attribute__((always_inline)) {
      constexpr int q = kFirst + decltype(Q)::value;
      mma_q<q, SKIP>(acc0, acc1, f);
      __builtin_amdgcn_sched_barrier(0);
      between(std::integral_constant<int, q>{});
      __builtin_amdgcn_sched_barrier(0);
    });
  } else {
    static_for<kMmaOf<NA> - kFirst>([&](auto Q) __attribute__((always_inline)) {
      between(std::integral_constant<int, kFirst + decltype(Q)::value>{});
    });
  }
  __builtin_amdgcn_sched_barrier(0);
}

// The K loop: two LDS stages of kBK = 64 (KMajor operand rows are then whole
// 128-byte cache lines: an LDS-DMA instruction touches 8 lines instead of 16,
// which doubles what a CU's L1 can stream from L2).
//   prep(kt)                 readies the loads of stage kt (operand switch,
//                            per-stage descriptors)
//   issue(p, stage)          issues load p (0 .. kLoadsPerStageOf<NA>-1, a
//                            constant) of the prepared stage into `stage`
//   read(stage, ks, frags, only)  the fragment reads of k-substep ks (a
//                            constant), inline asm: fragment `only` (B blocks
//                            0-3, then A0/A1 of row block 0, then of row
//                            block 1 for NA = 2) or, for only = -1, all of them
// Stage kt (buffer cur, next buffer nxt), fragments double-buffered in f[2]:
//   substeps j < kSubsteps-1: wait for f[j&1]; its kMmaOf MFMAs, with the
//     reads of (kt, j+1) -> f[(j+1)&1] one fragment after each of the first
//     MFMAs, and the loads of stage kt+1 that the previous stage left over
//     (below); prep(kt+2) after substep kSubsteps-2
//   last substep: wait for this wave's loads of stage kt+1 and for the last
//     fragments, barrier (stage kt+1 has landed for every wave, and every wave
//     is done reading stage kt), then the MFMAs of the last substep with the
//     reads of (kt+1, 0) -> f[0] and the first loads of stage kt+2 into cur
//     between them.
// With one wave per SIMD (NA = 2) the matrix core only stays busy if the wave
// issues its next MFMA as soon as the previous one leaves the pipe (32 clocks
// for 32x32x16), so everything else rides between MFMAs in small pieces:
// measured with clock stamps around each phase, the 16 loads of a stage issued
// back to back cost ~1000 clocks of idle matrix core per stage, and 8 to 16
// reads issued as a block plus the wait for the first of them ~100 clocks per
// substep.  Hence one fragment read after each of the first MFMAs, loads of 3
// scalar instructions each (buffer descriptor and M0 prepared per stage, no
// branch), and the loads of one stage spread over the last substep of stage kt
// and the first substep of stage kt+1 (kLdSplit); those issued in stage kt+1
// still have its last substeps to land.  NA = 1 keeps the same schedule with
// half the MFMAs, reads and loads per wave, two waves per SIMD.
// The fragment reads are inline asm because the compiler's wait-count pass
// cannot tell them from the in-flight LDS-DMA writes and would drain every
// load (vmcnt(0)) or every read (lgkmcnt(0)) in front of them; every wait
// here is explicit.  At the start of a substep the only LDS reads in flight
// are those of its own fragments, so lgkmcnt(0) costs nothing there.
#ifndef UTTT_LD_SPLIT
#define UTTT_LD_SPLIT 8, 8, 0, 0
#endif
// Loads of a stage (in sixteenths) issued in: the last substep of the stage
// before, then substeps 0, 1, 2 of the stage before the one they fill.
constexpr int kLdSplit[4] = {UTTT_LD_SPLIT};
static_assert(kLdSplit[0] + kLdSplit[1] + kLdSplit[2] + kLdSplit[3] == 16,
              "every load of a stage has a slot");

// The load (0 .. kLoadsPerStageOf<NA>-1) issued after MFMA q of phase ph (0 =
// last substep, 1..3 = substeps 0..2 of the next stage), or -1: phase ph's n
// loads sit after MFMAs 0, M/n, 2*M/n, ... of the M = kMmaOf<NA> of a substep.
template <int PH, int Q, int NA>
constexpr int load_slot() {
  constexpr int per = kLoadsPerStageOf<NA>;
  int lo = 0;
  for (int i = 0; i < PH; ++i) lo += kLdSplit[i] * per / 16;
  const int n = kLdSplit[PH] * per / 16;
  if (n == 0) return -1;
  for (int i = 0; i < n; ++i)
    if (i * kMmaOf<NA> / n == Q) return lo + i;
  return -1;
}

template <int NLDS, bool SKIP, int NA, class PrepFn, class IssueFn, class ReadFn>
__device__ __forceinline__ void run_pipeline(int nk, bool full, PrepFn&& prep, IssueFn&& issue,
                                             ReadFn&& read,
                                             f32x16 (&acc0)[NA][kNB], f32x16 (&acc1)[NA][kNB],
                                             uint8_t* const (&ring)[kStages]) {
  if (nk <= 0) return;
  constexpr int kFrags = kNB + 2 * NA;  // fragment reads of a substep (one per MFMA slot)
  constexpr int kPerStage = kLoadsPerStageOf<NA>;
  static_assert(kSubsteps % 2 == 0 && kSubsteps == 4, "fragment double buffer parity");
  static_assert(NLDS <= 2 * kMmaOf<NA>, "two LDS reads per MFMA slot at most");
  static_assert(kFrags <= kMmaOf<NA>, "one fragment per MFMA slot");
  static_assert(kLdSplit[0] * kPerStage % 16 == 0 && kLdSplit[1] * kPerStage % 16 == 0 &&
                    kLdSplit[2] * kPerStage % 16 == 0 && kLdSplit[3] * kPerStage % 16 == 0,
                "the load split must divide the stage's loads");
  using All = std::integral_constant<int, -1>;
  HalfFrags<NA> f[2];
  static_for<kStages>([&](auto i) __attribute__((always_inline)) {
    prep(decltype(i)::value);
    static_for<kPerStage>([&](auto p) __attribute__((always_inline)) {
      issue(p, ring[decltype(i)::value]);
    });
  });
  // stage 0 landed: counted while stage 1 issued its kPerStage DMAs
  if (SKIP)  // the token tiles may issue fewer loads per stage
    wait_vmcnt<0>();
  else
    wait_vmcnt<(kStages - 1) * kPerStage>();
  block_barrier();
  read(ring[0], std::integral_constant<int, 0>{}, f[0], All{});
  // stage 1 was loaded whole before the loop: stage 0 has no leftover loads
  bool leftovers = false;
  auto step = [&](int kt, uint8_t* cur, uint8_t* nxt) __attribute__((always_inline)) {
    static_for<kSubsteps - 1>([&](auto J) __attribute__((always_inline)) {
      constexpr int j = J;
      lgkm_wait_tied<0>(f[j & 1]);
      mma_half<SKIP>(acc0, acc1, f[j & 1], full, [&](auto q) __attribute__((always_inline)) {
        constexpr int Q = decltype(q)::value;
        if constexpr (Q < kFrags)
          read(cur, std::integral_constant<int, j + 1>{}, f[(j + 1) & 1],
               std::integral_constant<int, Q>{});
        constexpr int p = load_slot<j + 1, Q, NA>();
        if constexpr (p >= 0)
          if (leftovers) issue(std::integral_constant<int, p>{}, nxt);
      });
      if constexpr (j == kSubsteps - 2) prep(kt + kStages);
      __builtin_amdgcn_sched_barrier(0);
    });
    constexpr int jl = kSubsteps - 1;
    wait_vmcnt<(kStages - 2) * kPerStage>();
    lgkm_wait_tied<0>(f[jl & 1]);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_sched_barrier(0);
    mma_half<SKIP>(acc0, acc1, f[jl & 1], full, [&](auto q) __attribute__((always_inline)) {
      if constexpr (decltype(q)::value < kFrags)
        read(nxt, std::integral_constant<int, 0>{}, f[(jl + 1) & 1],
             std::integral_constant<int, decltype(q)::value>{});
      constexpr int p = load_slot<0, decltype(q)::value, NA>();
      if constexpr (p >= 0) issue(std::integral_constant<int, p>{}, cur);
    });
    leftovers = true;
    __builtin_amdgcn_sched_barrier(0);
  };
  // whole ring iterations only (one copy of the step code: a separate tail
  // would keep its own addressing live across the loop); steps past nk
  // multiply the zeros their loads wrote (no records)
  for (int kt = 0; kt < nk; kt += kStages)
    static_for<kStages>([&](auto i) __attribute__((always_inline)) {
      step(kt + i, ring[i], ring[(i + 1) % kStages]);
    });
  lgkm_wait_tied<0>(f[0]);  // the reads of the stage past the end
  wait_vmcnt<0>();        // and the loads issued past the end
}

// Opaque copies of the values an epilogue addresses with, taken after the K
// loop: nothing computed from them can be hoisted above the loop, where it
// would stay live across it (the loop needs every register: with the fragment
// reads in asm, a spill of a fragment register between its read and its wait
// would save the value from before the read).
__device__ __forceinline__ int after_loop(int v) {
  asm volatile("" : "+v"(v));
  return v;
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

// Wave-wide sums with DPP adds (no LDS round trip): the inclusive prefix
// sum over the 64 lanes (row shifts by 1, 2, 4, 8 inside each 16-lane row,
// then row 15 and lane 31 broadcast into the later rows), and a lane's value
// read by every lane.  Lanes outside a shift's row take the added 0.
template <int CTRL, int ROWS>
__device__ __forceinline__ int dpp_add_src(int x) {
  return __builtin_amdgcn_update_dpp(0, x, CTRL, ROWS, 0xf, false);
}
__device__ __forceinline__ int wave_incl_scan(int x) {
  x += dpp_add_src<0x111, 0xf>(x);  // row_shr:1
  x += dpp_add_src<0x112, 0xf>(x);  // row_shr:2
  x += dpp_add_src<0x114, 0xf>(x);  // row_shr:4
  x += dpp_add_src<0x118, 0xf>(x);  // row_shr:8
  x += dpp_add_src<0x142, 0xa>(x);  // row_bcast:15 into rows 1 and 3
  x += dpp_add_src<0x143, 0xc>(x);  // row_bcast:31 into rows 2 and 3
  return x;
}
__device__ __forceinline__ int lane_value(int x, int lane) {
  return __builtin_amdgcn_readlane(x, lane);
}

// The token tile of one workgroup.  Every wave scans group_sizes itself (the
// same result in each: no LDS broadcast and no barrier before the first
// loads).
template <int BN>
__device__ TokenTile find_token_tile(const int32_t* __restrict__ gs_b, int E, int N, int tile) {
  const int lane = threadIdx.x & 63;
  int tok_base = 0, tile_base = 0;
  for (int e0 = 0; e0 < E; e0 += 64) {
    const int e = e0 + lane;
    const int graw = e < E ? gs_b[e] : 0;
    const int g = graw > 0 ? graw : 0;
    const int tok_incl = wave_incl_scan(g);
    const int start = min(tok_base + tok_incl - g, N);
    const int gc = min(g, N - start);
    const int nt = (gc + BN - 1) / BN;
    const int tile_incl = wave_incl_scan(nt);
    const int tile_excl = tile_base + tile_incl - nt;
    const bool hit = e < E && tile >= tile_excl && tile < tile_excl + nt;
    const uint64_t bal = __ballot(hit);
    if (bal != 0ull) {
      const int src = __ffsll((unsigned long long)bal) - 1;
      return TokenTile{__builtin_amdgcn_readfirstlane(e0 + src), lane_value(start, src),
                       lane_value(gc, src), (tile - lane_value(tile_excl, src)) * BN};
    }
    tok_base += lane_value(tok_incl, 63);
    tile_base += lane_value(tile_incl, 63);
  }
  return TokenTile{-1, 0, 0, 0};
}

// The expert-major pair of workgroup `bid` when the real pairs (token tiles x
// M m-tiles, the tiles counted with find_token_tile's clamping of segments to
// [0, N)) are cut into kXcds equal ranges, workgroup bid taking the
// (bid / kXcds)-th pair of range bid % kXcds: every wave counts the token
// tiles and finds the pair in registers (no LDS, no barrier); e = -1 for a
// workgroup past its range.
template <int BN>
__device__ TokenTile find_pair_em_xcd(const int32_t* __restrict__ gs_b, int E, int N, int M,
                                      int bid, int* mt) {
  const int lane = threadIdx.x & 63;
  // pass 1: total token tiles R
  int tok_base = 0, R = 0;
  for (int e0 = 0; e0 < E; e0 += 64) {
    const int e = e0 + lane;
    const int graw = e < E ? gs_b[e] : 0;
    const int g = graw > 0 ? graw : 0;
    const int tok_incl = wave_incl_scan(g);
    const int start = min(tok_base + tok_incl - g, N);
    const int gc = min(g, N - start);
    R += lane_value(wave_incl_scan((gc + BN - 1) / BN), 63);
    tok_base += lane_value(tok_incl, 63);
  }
  const int64_t total = (int64_t)R * M;
  const int64_t per = (total + kXcds - 1) / kXcds;
  const int64_t loc = bid / kXcds;
  const int64_t t = (int64_t)(bid % kXcds) * per + loc;
  *mt = 0;
  if (loc >= per || t >= total) return TokenTile{-1, 0, 0, 0};
  // pass 2: the expert whose pairs hold t (group_sizes are in L1 now); the
  // pair counts fit in 32 bits (tiles of a batch times the m-tiles)
  tok_base = 0;
  int pair_base = 0;
  const int ti = (int)t;
  for (int e0 = 0; e0 < E; e0 += 64) {
    const int e = e0 + lane;
    const int graw = e < E ? gs_b[e] : 0;
    const int gg = graw > 0 ? graw : 0;
    const int tok_incl = wave_incl_scan(gg);
    const int start = min(tok_base + tok_incl - gg, N);
    const int gc = min(gg, N - start);
    const int nt = (gc + BN - 1) / BN;
    const int pairs_incl = wave_incl_scan(nt * M);
    const int pairs_excl = pair_base + pairs_incl - nt * M;
    const bool hit = e < E && nt > 0 && ti >= pairs_excl && ti < pairs_excl + nt * M;
    const uint64_t bal = __ballot(hit);
    if (bal != 0ull) {
      const int src = __ffsll((unsigned long long)bal) - 1;
      const int ntb = lane_value(nt, src);
      const int local = ti - lane_value(pairs_excl, src);
      *mt = local / ntb;
      return TokenTile{__builtin_amdgcn_readfirstlane(e0 + src), lane_value(start, src),
                       lane_value(gc, src), (local % ntb) * BN};
    }
    tok_base += lane_value(tok_incl, 63);
    pair_base += lane_value(pairs_incl, 63);
  }
  return TokenTile{-1, 0, 0, 0};
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
