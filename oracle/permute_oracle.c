/*
 * permute_oracle.c - CPU restatement of uTTT's token permute path, used ONLY
 * as the checker of the HIP kernels (tests, smoke check, bench CPU baseline).
 * It is not part of the product and is never linked into libuttt_hip.so.
 *
 * Each function restates the reference algorithm step by step (not the HIP
 * design): the three passes of make_row_id_map with a 512-token block
 * cumsum, a workspace prefix and a per-token descending sort, then the
 * per-token loops of the permute / unpermute kernels.
 *
 * Reference: uttt_llm/flame/custom_models/uttt_moe/lact_moe_triton/
 *            triton_permute.py (cited as P:line below).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define OR_F32 0
#define OR_BF16 1
#define OR_F16 2

static float bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* round to nearest even, as torch's .to(bfloat16) and Triton's cast */
static uint16_t f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static float load_el(const void* p, int64_t i, int dtype) {
  if (dtype == OR_F32) return ((const float*)p)[i];
  return bf16_to_f32(((const uint16_t*)p)[i]);
}

static void store_el(void* p, int64_t i, int dtype, float v) {
  if (dtype == OR_F32)
    ((float*)p)[i] = v;
  else
    ((uint16_t*)p)[i] = f32_to_bf16(v);
}

/* make_row_id_map (P:283-393).  mask: int32 0/1, contiguous [B, E, T].
 * out: [B, T, 2E+1], zero-filled first like routing_map.new_zeros (P:314). */
void oracle_make_row_id_map(const int32_t* mask, int B, int T, int E, int32_t* out) {
  const int BLK = 512; /* P:317 */
  const int nblk = (T + BLK - 1) / BLK;
  const int W = 2 * E + 1;
  int32_t* ws = (int32_t*)malloc(sizeof(int32_t) * (size_t)E * nblk + 1);
  memset(out, 0, sizeof(int32_t) * (size_t)B * T * W);
  for (int b = 0; b < B; ++b) {
    const int32_t* m = mask + (int64_t)b * E * T;
    int32_t* o = out + (int64_t)b * T * W;
    /* pass 1 (P:100-160): block-local inclusive cumsum times the mask into
     * column e; the block's count goes to the workspace */
    for (int e = 0; e < E; ++e) {
      for (int blk = 0; blk < nblk; ++blk) {
        int run = 0;
        for (int t = blk * BLK; t < T && t < (blk + 1) * BLK; ++t) {
          int v = m[(int64_t)e * T + t];
          run += v;
          o[(int64_t)t * W + e] = run * v;
        }
        ws[e * nblk + blk] = run;
      }
    }
    /* pass 2 (P:163-228): add every workspace entry before (e, blk) in
     * expert-major order; zero entries become -1 */
    for (int e = 0; e < E; ++e) {
      for (int blk = 0; blk < nblk; ++blk) {
        int before = 0;
        for (int i = 0; i < e * nblk + blk; ++i) before += ws[i];
        for (int t = blk * BLK; t < T && t < (blk + 1) * BLK; ++t) {
          int v = o[(int64_t)t * W + e];
          o[(int64_t)t * W + e] = (v == 0) ? -1 : v + before - 1;
        }
      }
    }
    /* pass 3 (P:231-280): per token, sort its E entries descending together
     * with their column indices; store only the first n_routed of each */
    int32_t vals[256], idx[256];
    for (int t = 0; t < T; ++t) {
      int32_t* r = o + (int64_t)t * W;
      int n = 0;
      for (int e = 0; e < E; ++e) {
        vals[e] = r[e];
        idx[e] = e;
        if (r[e] != -1) ++n;
      }
      for (int i = 1; i < E; ++i) { /* insertion sort, descending */
        int32_t v = vals[i], x = idx[i];
        int j = i - 1;
        while (j >= 0 && vals[j] < v) {
          vals[j + 1] = vals[j];
          idx[j + 1] = idx[j];
          --j;
        }
        vals[j + 1] = v;
        idx[j + 1] = x;
      }
      for (int i = 0; i < n; ++i) {
        r[i] = vals[i];
        r[E + i] = idx[i];
      }
      r[2 * E] = n;
    }
  }
  free(ws);
}

/* _permute_kernel (P:396-473): out[row_j] = inp[t], or zeros when
 * probs[e_j, t] == 0; permuted_probs[row_j] = probs[e_j, t].
 * probs: contiguous [B, E, T] fp32 or NULL. */
void oracle_permute(const void* inp, int elem_bytes, int B, int T, int H, const int32_t* rmap,
                    int E, const float* probs, void* out, int num_out, float* pprobs) {
  const int W = 2 * E + 1;
  const int64_t rb = (int64_t)H * elem_bytes;
  for (int b = 0; b < B; ++b)
    for (int t = 0; t < T; ++t) {
      const int32_t* r = rmap + ((int64_t)b * T + t) * W;
      const char* src = (const char*)inp + ((int64_t)b * T + t) * rb;
      for (int j = 0; j < r[2 * E]; ++j) {
        int row = r[j], e = r[E + j];
        char* dst = (char*)out + ((int64_t)b * num_out + row) * rb;
        if (probs) {
          float p = probs[((int64_t)b * E + e) * T + t];
          pprobs[(int64_t)b * num_out + row] = p;
          if (p == 0.0f) {
            memset(dst, 0, (size_t)rb);
            continue;
          }
        }
        memcpy(dst, src, (size_t)rb);
      }
    }
}

/* _unpermute_kernel (P:765-850): out[t] = cast(acc), acc (fp32) starting at
 * 0 and updated in slot order by acc = fma(y[row_j], p_j, acc) -- the
 * multiply-then-accumulate of P:842-845 as Triton fuses it by default -- or
 * acc += y[row_j] without probs. */
void oracle_unpermute(const void* inp, int dtype, int B, int num_out, int H, const int32_t* rmap,
                      int T, int E, const float* probs, void* out) {
  const int W = 2 * E + 1;
  float* acc = (float*)malloc(sizeof(float) * (size_t)(H > 0 ? H : 1));
  for (int b = 0; b < B; ++b)
    for (int t = 0; t < T; ++t) {
      const int32_t* r = rmap + ((int64_t)b * T + t) * W;
      for (int h = 0; h < H; ++h) acc[h] = 0.0f;
      for (int j = 0; j < r[2 * E]; ++j) {
        int64_t src = ((int64_t)b * num_out + r[j]) * H;
        if (probs) {
          float p = probs[((int64_t)b * E + r[E + j]) * T + t];
          for (int h = 0; h < H; ++h) acc[h] = fmaf(load_el(inp, src + h, dtype), p, acc[h]);
        } else {
          for (int h = 0; h < H; ++h) acc[h] += load_el(inp, src + h, dtype);
        }
      }
      for (int h = 0; h < H; ++h) store_el(out, ((int64_t)b * T + t) * H + h, dtype, acc[h]);
    }
  free(acc);
}

/* _permute_kv_with_lrs_kernel (P:1333-1493): k copied to each slot, v scaled
 * by p in fp32 and rounded once to k's dtype (P:1479-1480), lrs copied. */
void oracle_permute_kv_lrs(const void* k, int k_dtype, const void* v, int v_dtype,
                           const void* lr0, const void* lr1, const void* lr2, int lr_bytes, int B,
                           int T, int H, const int32_t* rmap, int E, const float* probs,
                           void* k_out, void* v_out, void* lr0_out, void* lr1_out, void* lr2_out,
                           int num_out) {
  const int W = 2 * E + 1;
  const int kb = k_dtype == OR_F32 ? 4 : 2;
  for (int b = 0; b < B; ++b)
    for (int t = 0; t < T; ++t) {
      const int32_t* r = rmap + ((int64_t)b * T + t) * W;
      const int64_t tok = (int64_t)b * T + t;
      for (int j = 0; j < r[2 * E]; ++j) {
        const int64_t row = (int64_t)b * num_out + r[j];
        const float p = probs[((int64_t)b * E + r[E + j]) * T + t];
        memcpy((char*)k_out + row * H * kb, (const char*)k + tok * H * kb, (size_t)H * kb);
        for (int h = 0; h < H; ++h)
          store_el(v_out, row * H + h, k_dtype, load_el(v, tok * H + h, v_dtype) * p);
        memcpy((char*)lr0_out + row * lr_bytes, (const char*)lr0 + tok * lr_bytes, lr_bytes);
        memcpy((char*)lr1_out + row * lr_bytes, (const char*)lr1 + tok * lr_bytes, lr_bytes);
        memcpy((char*)lr2_out + row * lr_bytes, (const char*)lr2 + tok * lr_bytes, lr_bytes);
      }
    }
}
