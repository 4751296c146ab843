/*
 * pa_oracle.c -- CPU restatement of vllm-lite's paged-attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the HIP kernels are
 * compared against and the "restated ref-CPU" baseline that bench.py times.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it.  Nothing in the product library links or calls it.
 *
 * The reference is Rust + candle 0.11.0 and cannot be built here (no cargo,
 * candle not vendored), so its algorithm is restated in plain C.  Every
 * function cites the reference file:line it follows (paths relative to the
 * vllm-lite repository root).
 *
 * Layouts (all row-major, all contiguous):
 *   cache  [num_blocks, H, 16, D]   crates/model/src/paged_tensor/tensor_store/mod.rs:62
 *   token  [H, D]                   one token's K or V (write_kv's [1, H, D])
 *   q      [T, Hq, D]  (token-major, the layout the GPU entry points take)
 *
 * dtype codes: 0 = f32, 1 = bf16 (raw uint16 bit patterns).  Copies are
 * bit-exact for both; arithmetic widens bf16 to f32 first (the oracle
 * consumes the bf16-rounded values the GPU sees).
 *
 * Pinning status of each function (what checks it besides itself):
 *   oracle_write_kv / oracle_read_kv / oracle_write_kv_batch /
 *   oracle_write_prefill_kv / oracle_slot_mapping / oracle_reshape_and_cache
 *       -> the reference's known-answer tests restated as golden fixtures
 *          (the JSON fixtures under tests/golden) and closed-form index checks.
 *   oracle_expand_kv        -> util/tests.rs:296-313 golden vector.
 *   oracle_attention*       -> util/tests.rs:394-458 fixture vs an
 *          independent numpy float64 softmax, single-key (out = V) and
 *          uniform-key (out = mean V) closed forms, chunk invariance.
 *   oracle_block_hash       -> hand-computed values for short inputs and
 *          the saturating float->u64 cast cases.
 *   oracle_quant_write_kv / oracle_quant_read_kv -> closed-form int8 grid
 *          checks (scale = max|x| / 127, values on the integer grid).
 *   oracle_rope_inv_freq / oracle_rope -> closed forms (identity at
 *          position 0, cos/sin at position 1, rotation direction, per-type
 *          frequency tables).
 *   oracle_argmax_logits    -> the reference's sampling.rs:468-490 known
 *          answers (first of equal maxima, negatives, empty, one element)
 *          and numpy's argmax on NaN-free rows.
 *   oracle_fp8_encode / oracle_fp8_decode -> the reference's own test values,
 *          torch's independent float8_e4m3fn conversions wherever that
 *          format and the reference's coincide, exhaustive round trips and a
 *          brute-force nearest-value search.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define PA_BLOCK 16 /* crates/traits/src/types.rs:13 BLOCK_SIZE */

enum { ORC_OK = 0, ORC_ERR_ARG = -1, ORC_ERR_BOUNDS = -2 };

static inline float bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline uint16_t f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40); /* quiet NaN */
  u += 0x7fffu + ((u >> 16) & 1u); /* round to nearest even */
  return (uint16_t)(u >> 16);
}

static inline size_t esize(int dtype) { return dtype == 1 ? 2 : 4; }

static inline float load_el(const void* p, size_t i, int dtype) {
  return dtype == 1 ? bf16_to_f32(((const uint16_t*)p)[i]) : ((const float*)p)[i];
}

static inline void store_el(void* p, size_t i, float x, int dtype) {
  if (dtype == 1)
    ((uint16_t*)p)[i] = f32_to_bf16(x);
  else
    ((float*)p)[i] = x;
}

uint16_t oracle_f32_to_bf16(float f) { return f32_to_bf16(f); }
float oracle_bf16_to_f32(uint16_t h) { return bf16_to_f32(h); }

/* ------------------------------------------------------------------------ */
/* KV store                                                                 */
/* ------------------------------------------------------------------------ */

/* PagedKvCache::write_kv, non-quantised branch.
 * crates/model/src/paged_tensor/tensor_store/buffer.rs:103-267.
 * Bounds checks follow :126-137 (block_id < num_blocks, token_offset < 16);
 * the per-head copy into [h][token_offset][:] follows :201-207.
 * k/v: [H, D] (the [1, H, D] tensor without its unit axis). */
int oracle_write_kv(void* k_cache, void* v_cache, int num_blocks, int H, int D,
                    int64_t block_id, int64_t token_offset, const void* k, const void* v,
                    int dtype) {
  if (block_id < 0 || block_id >= num_blocks) return ORC_ERR_BOUNDS;
  if (token_offset < 0 || token_offset >= PA_BLOCK) return ORC_ERR_BOUNDS;
  size_t es = esize(dtype);
  for (int h = 0; h < H; ++h) {
    size_t dst = (((size_t)block_id * H + h) * PA_BLOCK + (size_t)token_offset) * D;
    memcpy((char*)k_cache + dst * es, (const char*)k + (size_t)h * D * es, D * es);
    memcpy((char*)v_cache + dst * es, (const char*)v + (size_t)h * D * es, D * es);
  }
  return ORC_OK;
}

/* PagedKvCache::write_kv_batch.
 * crates/model/src/paged_tensor/tensor_store/buffer.rs:27-95.
 * Capacity check :69-75 ((num_blocks - block_id) * 16 >= offset + T), then a
 * walk that advances to block_id + 1 when the offset wraps (:77-92), i.e. the
 * run assumes physically consecutive blocks.  k/v: [T, H, D]. */
int oracle_write_kv_batch(void* k_cache, void* v_cache, int num_blocks, int H, int D,
                          int64_t block_id, int64_t token_offset, const void* k, const void* v,
                          int T, int dtype) {
  if (block_id < 0 || block_id >= num_blocks || token_offset < 0) return ORC_ERR_BOUNDS;
  int64_t cap = ((int64_t)num_blocks - block_id) * PA_BLOCK;
  if (token_offset + T > cap) return ORC_ERR_BOUNDS;
  size_t es = esize(dtype);
  int64_t blk = block_id, off = token_offset;
  for (int t = 0; t < T; ++t) {
    int rc = oracle_write_kv(k_cache, v_cache, num_blocks, H, D, blk, off,
                             (const char*)k + (size_t)t * H * D * es,
                             (const char*)v + (size_t)t * H * D * es, dtype);
    if (rc) return rc;
    if (++off >= PA_BLOCK) {
      ++blk;
      off = 0;
    }
  }
  return ORC_OK;
}

/* PagedKvCache::read_kv, non-quantised branch.
 * crates/model/src/paged_tensor/tensor_store/buffer.rs:273-339.
 * Walk block_ids in order; block b covers tokens [16b, 16b+16); stop at
 * seq_len (headroom blocks ignored, :302-304); result [seq_len, H, D]
 * (cat along tokens then transpose, :335-336).  Returns the number of tokens
 * produced (0 for an empty table or seq_len 0, :279-284), or a negative code
 * if a block id is out of range (candle's narrow would fail there). */
int oracle_read_kv(const void* k_cache, const void* v_cache, int num_blocks, int H, int D,
                   const int64_t* block_ids, int n_ids, int seq_len, void* out_k, void* out_v,
                   int dtype) {
  if (n_ids <= 0 || seq_len <= 0) return 0;
  size_t es = esize(dtype);
  int produced = 0;
  for (int b = 0; b < n_ids; ++b) {
    int start = b * PA_BLOCK;
    if (start >= seq_len) break;
    int end = start + PA_BLOCK < seq_len ? start + PA_BLOCK : seq_len;
    int64_t blk = block_ids[b];
    if (blk < 0 || blk >= num_blocks) return ORC_ERR_BOUNDS;
    for (int t = start; t < end; ++t)
      for (int h = 0; h < H; ++h) {
        size_t src = (((size_t)blk * H + h) * PA_BLOCK + (size_t)(t - start)) * D;
        size_t dst = ((size_t)t * H + h) * D;
        memcpy((char*)out_k + dst * es, (const char*)k_cache + src * es, D * es);
        memcpy((char*)out_v + dst * es, (const char*)v_cache + src * es, D * es);
      }
    produced = end;
  }
  return produced;
}

/* Slot mapping used by write_prefill_kv and read_decode_kv.
 * crates/model/src/components/attention/paged_gqa.rs:39-52 and :86-97:
 *   global_pos = positions[t] (or t when positions is short, :40)
 *   block_id   = block_ids[global_pos / 16], falling back to block 0 when the
 *                table is too short (:51, :97)
 *   offset     = global_pos % 16
 * Flat slot = block_id * 16 + offset.  n_pos < 0 means "no positions given". */
void oracle_slot_mapping(const int64_t* block_ids, int n_ids, const int64_t* positions,
                         int n_pos, int T, int64_t* slots_out) {
  for (int t = 0; t < T; ++t) {
    int64_t pos = (positions && t < n_pos) ? positions[t] : t;
    int64_t bi = pos / PA_BLOCK;
    int64_t blk = (bi >= 0 && bi < n_ids) ? block_ids[bi] : 0;
    slots_out[t] = blk * PA_BLOCK + pos % PA_BLOCK;
  }
}

/* write_prefill_kv: per-token write_kv at the mapped slot.
 * crates/model/src/components/attention/paged_gqa.rs:29-63.
 * k/v here are token-major [T, H, D] (the reference's [1, H, T, D] transposed;
 * the per-token slice it writes is the same [H, D]). */
int oracle_write_prefill_kv(void* k_cache, void* v_cache, int num_blocks, int H, int D,
                            const int64_t* block_ids, int n_ids, const int64_t* positions,
                            int n_pos, int T, const void* k, const void* v, int dtype) {
  size_t es = esize(dtype);
  for (int t = 0; t < T; ++t) {
    int64_t pos = (positions && t < n_pos) ? positions[t] : t;
    int64_t bi = pos / PA_BLOCK;
    int64_t blk = (bi >= 0 && bi < n_ids) ? block_ids[bi] : 0;
    int64_t slot = blk * PA_BLOCK + pos % PA_BLOCK;
    int rc = oracle_write_kv(k_cache, v_cache, num_blocks, H, D, slot / PA_BLOCK,
                             slot % PA_BLOCK, (const char*)k + (size_t)t * H * D * es,
                             (const char*)v + (size_t)t * H * D * es, dtype);
    if (rc) return rc;
  }
  return ORC_OK;
}

/* Explicit-slot scatter (the batched form the GPU entry point takes).
 * Semantics = write_kv at (slot / 16, slot % 16) for every token whose slot
 * is >= 0 and < num_blocks * 16; other tokens are skipped.  k/v [T, H, D]. */
int oracle_reshape_and_cache(const void* k, const void* v, void* k_cache, void* v_cache,
                             const int64_t* slots, int T, int H, int D, int num_blocks,
                             int dtype) {
  size_t es = esize(dtype);
  int skipped = 0;
  for (int t = 0; t < T; ++t) {
    int64_t s = slots[t];
    if (s < 0 || s >= (int64_t)num_blocks * PA_BLOCK) {
      ++skipped;
      continue;
    }
    oracle_write_kv(k_cache, v_cache, num_blocks, H, D, s / PA_BLOCK, s % PA_BLOCK,
                    (const char*)k + (size_t)t * H * D * es,
                    (const char*)v + (size_t)t * H * D * es, dtype);
  }
  return skipped;
}

/* expand_kv: blocked GQA replication, query head h reads kv head h / g.
 * crates/model/src/components/attention/util.rs:55-87 (repeat factor
 * div_ceil(Hq, Hkv), then narrow to Hq).  in [S, Hkv, D] -> out [S, Hq, D]. */
void oracle_expand_kv(const float* in, int S, int Hkv, int Hq, int D, float* out) {
  int rep = (Hq + Hkv - 1) / Hkv;
  for (int s = 0; s < S; ++s)
    for (int h = 0; h < Hq; ++h)
      memcpy(out + ((size_t)s * Hq + h) * D, in + ((size_t)s * Hkv + h / rep) * D,
             (size_t)D * sizeof(float));
}

/* Block content hash. crates/model/src/paged_tensor/tensor_store/layout.rs:51-58:
 *   fold(0, |acc, x| acc * 31 + (|x| * 1000.0) as u64)   (wrapping u64)
 * The f32 multiply happens in f32; Rust's `as u64` saturates (NaN -> 0,
 * negatives -> 0, >= 2^64 -> u64::MAX). */
uint64_t oracle_block_hash(const float* data, int64_t n) {
  uint64_t acc = 0;
  for (int64_t i = 0; i < n; ++i) {
    float y = fabsf(data[i]) * 1000.0f;
    uint64_t x;
    if (isnan(y) || y <= 0.0f)
      x = 0;
    else if (y >= 18446744073709551616.0f)
      x = UINT64_MAX;
    else
      x = (uint64_t)y;
    acc = acc * 31u + x;
  }
  return acc;
}

/* Greedy sampling. crates/traits/src/sampling.rs:439-453:
 *   enumerate().fold((0, -inf), |(bi, bv), (i, v)| if v > bv {(i, v)} else {(bi, bv)})
 * i.e. the first strict maximum; NaN never compares greater; an empty row or
 * one with nothing above -inf keeps index 0. */
int64_t oracle_argmax_logits(const float* x, int64_t n) {
  int64_t bi = 0;
  float bv = -INFINITY;
  for (int64_t i = 0; i < n; ++i)
    if (x[i] > bv) {
      bi = i;
      bv = x[i];
    }
  return bi;
}

/* ------------------------------------------------------------------------ */
/* Attention                                                                */
/* ------------------------------------------------------------------------ */

/* One query head against dense K/V rows: the reference's
 *   qk = q · kᵀ ; qk += mask ; qk *= scale ; p = softmax(qk) ; out = p · v
 * crates/model/src/components/attention/paged_gqa.rs:149-164 (mask then
 * scale) and util.rs:160-171 / :213-226 (same order).  Keys j > last_visible
 * carry the -inf mask (util.rs:119-139, j <= past + i).  f32 accumulation in
 * index order.  kvs: pointer to row 0 of K (stride k_stride floats between
 * token rows), likewise V.  scores: scratch of n_keys floats. */
static void attend_row_f32(const float* q, const float* k, const float* v, size_t kv_stride,
                           int n_keys, int last_visible, int D, float scale, float* scores,
                           float* out) {
  float mx = -INFINITY;
  for (int j = 0; j < n_keys; ++j) {
    float s;
    if (j <= last_visible) {
      s = 0.f;
      const float* kr = k + (size_t)j * kv_stride;
      for (int d = 0; d < D; ++d) s += q[d] * kr[d];
      s *= scale;
    } else {
      s = -INFINITY;
    }
    scores[j] = s;
    if (s > mx) mx = s;
  }
  float sum = 0.f;
  for (int j = 0; j < n_keys; ++j) {
    float e = (scores[j] == -INFINITY) ? 0.f : expf(scores[j] - mx);
    scores[j] = e;
    sum += e;
  }
  for (int d = 0; d < D; ++d) out[d] = 0.f;
  for (int j = 0; j < n_keys; ++j) {
    float p = scores[j] / sum;
    const float* vr = v + (size_t)j * kv_stride;
    for (int d = 0; d < D; ++d) out[d] += p * vr[d];
  }
}

/* Same in float64 ("truth" mode for tolerance studies). */
static void attend_row_f64(const double* q, const float* k, const float* v, size_t kv_stride,
                           int n_keys, int last_visible, int D, double scale, double* scores,
                           double* out) {
  double mx = -INFINITY;
  for (int j = 0; j < n_keys; ++j) {
    double s;
    if (j <= last_visible) {
      s = 0.0;
      const float* kr = k + (size_t)j * kv_stride;
      for (int d = 0; d < D; ++d) s += q[d] * (double)kr[d];
      s *= scale;
    } else {
      s = -INFINITY;
    }
    scores[j] = s;
    if (s > mx) mx = s;
  }
  double sum = 0.0;
  for (int j = 0; j < n_keys; ++j) {
    double e = (scores[j] == -INFINITY) ? 0.0 : exp(scores[j] - mx);
    scores[j] = e;
    sum += e;
  }
  for (int d = 0; d < D; ++d) out[d] = 0.0;
  for (int j = 0; j < n_keys; ++j) {
    double p = scores[j] / sum;
    const float* vr = v + (size_t)j * kv_stride;
    for (int d = 0; d < D; ++d) out[d] += p * (double)vr[d];
  }
}

/* Dense GQA attention with the chunked-prefill mask.
 * compute_gqa_attention + prefill_continue_causal_mask:
 * crates/model/src/components/attention/paged_gqa.rs:135-164.
 *   q [Tq, Hq, D], k/v [Tk, Hkv, D] with Tk = past + Tq.  Query row i sees
 *   keys j <= past + i.  Query head h reads kv head h / (Hq / Hkv), the
 *   blocked grouping of expand_kv (util.rs:55-87).
 * past = 0, Tk = Tq is the fresh-prefill square mask (util.rs:97-107) and
 * Tq = 1, past = Tk - 1 is decode (paged_attention with a 1x1 mask).
 * f64 = 1 runs the float64 truth mode.  out [Tq, Hq, D] f32. */
int oracle_attention(const float* q, const float* k, const float* v, int Tq, int Tk, int past,
                     int Hq, int Hkv, int D, float scale, int f64, float* out) {
  if (Hq % Hkv != 0 || Tk < past + Tq) return ORC_ERR_ARG;
  int g = Hq / Hkv;
  float* sc = (float*)malloc(sizeof(double) * (Tk > 0 ? Tk : 1));
  double* qd = (double*)malloc(sizeof(double) * D);
  double* od = (double*)malloc(sizeof(double) * D);
  for (int i = 0; i < Tq; ++i)
    for (int h = 0; h < Hq; ++h) {
      const float* qr = q + ((size_t)i * Hq + h) * D;
      const float* kr = k + (size_t)(h / g) * D;
      const float* vr = v + (size_t)(h / g) * D;
      float* o = out + ((size_t)i * Hq + h) * D;
      if (f64) {
        for (int d = 0; d < D; ++d) qd[d] = qr[d];
        attend_row_f64(qd, kr, vr, (size_t)Hkv * D, Tk, past + i, D, (double)scale,
                       (double*)sc, od);
        for (int d = 0; d < D; ++d) o[d] = (float)od[d];
      } else {
        attend_row_f32(qr, kr, vr, (size_t)Hkv * D, Tk, past + i, D, scale, sc, o);
      }
    }
  free(sc);
  free(qd);
  free(od);
  return ORC_OK;
}

/* The reference's per-sequence paged path, batched over sequences:
 *   read_kv (gather the sequence's blocks into dense [L, H, D]),
 *   expand_kv (materialise Hq heads), then dense attention with the mask.
 * Decode:  crates/model/src/components/attention/rope_gqa.rs:385-429 ->
 *          paged_gqa.rs:71-112 (read + append; the new token is already in
 *          the cache here, written by the scatter) -> util.rs:150-176.
 * Prefill: rope_gqa.rs:315-372 (read past, write new, rectangular mask).
 * The cache here holds Hkv heads; the expansion to Hq is materialised like
 * the reference's expand_kv so the CPU baseline does the same work.
 *
 * q [sum_i Tq_i, Hq, D] (dtype), caches [NB, Hkv, 16, D] (dtype),
 * block_tables [B, max_blocks] int32, q_start [B+1] (cumulative query
 * rows), past [B] (tokens before this step's queries), out like q (dtype).
 * A sequence attends to keys 0 .. past + Tq - 1.  n_threads > 0 sets the
 * OpenMP team (OpenMP over (sequence, query head)). */
int oracle_paged_attention(const void* q, const void* k_cache, const void* v_cache,
                           const int32_t* block_tables, int max_blocks, const int32_t* q_start,
                           const int32_t* past, int B, int Hq, int Hkv, int D, int num_blocks,
                           float scale, int dtype, int f64, int n_threads, void* out) {
  if (Hq % Hkv != 0) return ORC_ERR_ARG;
  int g = Hq / Hkv;
  for (int b = 0; b < B; ++b) {
    int L = past[b] + (q_start[b + 1] - q_start[b]);
    if ((L + PA_BLOCK - 1) / PA_BLOCK > max_blocks) return ORC_ERR_BOUNDS;
    for (int i = 0; i < (L + PA_BLOCK - 1) / PA_BLOCK; ++i)
      if (block_tables[(size_t)b * max_blocks + i] < 0 ||
          block_tables[(size_t)b * max_blocks + i] >= num_blocks)
        return ORC_ERR_BOUNDS;
  }
#ifdef _OPENMP
  if (n_threads > 0) omp_set_num_threads(n_threads);
#else
  (void)n_threads;
#endif
  int rc_all = ORC_OK;
  for (int b = 0; b < B; ++b) {
    int Tq = q_start[b + 1] - q_start[b];
    int L = past[b] + Tq;
    if (Tq <= 0) continue;
    /* read_kv gather into dense f32 [L, Hkv, D] then expand to [L, Hq, D]. */
    float* kd = (float*)malloc(sizeof(float) * (size_t)L * Hkv * D + 4);
    float* vd = (float*)malloc(sizeof(float) * (size_t)L * Hkv * D + 4);
    float* ke = (float*)malloc(sizeof(float) * (size_t)L * Hq * D + 4);
    float* ve = (float*)malloc(sizeof(float) * (size_t)L * Hq * D + 4);
#pragma omp parallel for schedule(static)
    for (int t = 0; t < L; ++t) {
      int64_t blk = block_tables[(size_t)b * max_blocks + t / PA_BLOCK];
      for (int h = 0; h < Hkv; ++h) {
        size_t src = (((size_t)blk * Hkv + h) * PA_BLOCK + (size_t)(t % PA_BLOCK)) * D;
        size_t dst = ((size_t)t * Hkv + h) * D;
        for (int d = 0; d < D; ++d) {
          kd[dst + d] = load_el(k_cache, src + d, dtype);
          vd[dst + d] = load_el(v_cache, src + d, dtype);
        }
      }
    }
    oracle_expand_kv(kd, L, Hkv, Hq, D, ke);
    oracle_expand_kv(vd, L, Hkv, Hq, D, ve);
#pragma omp parallel
    {
      float* sc = (float*)malloc(sizeof(double) * (size_t)L + 8);
      float* qr = (float*)malloc(sizeof(float) * D);
      float* o = (float*)malloc(sizeof(float) * D);
      double* qd = (double*)malloc(sizeof(double) * D);
      double* od = (double*)malloc(sizeof(double) * D);
#pragma omp for schedule(dynamic) collapse(2)
      for (int i = 0; i < Tq; ++i)
        for (int h = 0; h < Hq; ++h) {
          size_t row = ((size_t)(q_start[b] + i) * Hq + h) * D;
          for (int d = 0; d < D; ++d) qr[d] = load_el(q, row + d, dtype);
          if (f64) {
            for (int d = 0; d < D; ++d) qd[d] = qr[d];
            attend_row_f64(qd, ke + (size_t)h * D, ve + (size_t)h * D, (size_t)Hq * D, L,
                           past[b] + i, D, (double)scale, (double*)sc, od);
            for (int d = 0; d < D; ++d) o[d] = (float)od[d];
          } else {
            attend_row_f32(qr, ke + (size_t)h * D, ve + (size_t)h * D, (size_t)Hq * D, L,
                           past[b] + i, D, scale, sc, o);
          }
          for (int d = 0; d < D; ++d) store_el(out, row + d, o[d], dtype);
        }
      free(sc);
      free(qr);
      free(o);
      free(qd);
      free(od);
    }
    (void)g;
    free(kd);
    free(vd);
    free(ke);
    free(ve);
  }
  return rc_all;
}

/* ------------------------------------------------------------------------ */
/* int8-in-f32 block quantisation (PagedKvCache with quantized = true)       */
/* ------------------------------------------------------------------------ */

/* write_kv, quantised branch. buffer.rs:184-231: dequantise the whole block
 * with its stored scale, overwrite one token slot, then requantise the K and
 * V blocks together with scale = max(max|K|, max|V|) / 127 (1.0 for an
 * all-zero block) and values round(x / scale) (round half away from zero,
 * Rust f32::round).  scales [num_blocks] holds the per-block scale
 * (mod.rs:69 initialises it to 1.0). */
int oracle_quant_write_kv(float* k_cache, float* v_cache, float* scales, int num_blocks, int H,
                          int D, int64_t block_id, int64_t token_offset, const float* k,
                          const float* v) {
  if (block_id < 0 || block_id >= num_blocks) return ORC_ERR_BOUNDS;
  if (token_offset < 0 || token_offset >= PA_BLOCK) return ORC_ERR_BOUNDS;
  size_t n = (size_t)H * PA_BLOCK * D;
  float* kb = k_cache + (size_t)block_id * n;
  float* vb = v_cache + (size_t)block_id * n;
  float s_old = scales[block_id];
  for (size_t i = 0; i < n; ++i) {
    kb[i] *= s_old;
    vb[i] *= s_old;
  }
  for (int h = 0; h < H; ++h) {
    memcpy(kb + ((size_t)h * PA_BLOCK + token_offset) * D, k + (size_t)h * D, D * sizeof(float));
    memcpy(vb + ((size_t)h * PA_BLOCK + token_offset) * D, v + (size_t)h * D, D * sizeof(float));
  }
  float km = 0.f, vm = 0.f;
  for (size_t i = 0; i < n; ++i) {
    km = fmaxf(km, fabsf(kb[i]));
    vm = fmaxf(vm, fabsf(vb[i]));
  }
  float mx = fmaxf(km, vm);
  float scale = mx > 0.f ? mx / 127.0f : 1.0f;
  for (size_t i = 0; i < n; ++i) {
    kb[i] = roundf(kb[i] / scale);
    vb[i] = roundf(vb[i] / scale);
  }
  scales[block_id] = scale;
  return ORC_OK;
}

/* read_kv, quantised branch (buffer.rs:320-331): each block goes through
 * candle's affine(scale, 0.0), i.e. x * scale + 0.0 in f32 (so a stored -0
 * reads back as +0).  Same walk as oracle_read_kv, f32 only. */
int oracle_quant_read_kv(const float* k_cache, const float* v_cache, const float* scales,
                         int num_blocks, int H, int D, const int64_t* block_ids, int n_ids,
                         int seq_len, float* out_k, float* out_v) {
  int n = oracle_read_kv(k_cache, v_cache, num_blocks, H, D, block_ids, n_ids, seq_len, out_k,
                         out_v, 0);
  if (n <= 0) return n;
  for (int t = 0; t < n; ++t) {
    float s = scales[block_ids[t / PA_BLOCK]];
    for (size_t i = 0; i < (size_t)H * D; ++i) {
      out_k[(size_t)t * H * D + i] = out_k[(size_t)t * H * D + i] * s + 0.0f;
      out_v[(size_t)t * H * D + i] = out_v[(size_t)t * H * D + i] * s + 0.0f;
    }
  }
  return n;
}

/* ------------------------------------------------------------------------ */
/* Rotary position embedding                                               */
/* ------------------------------------------------------------------------ */

/* Inverse-frequency table of RoPE, crates/model/src/components/positional/
 * rope.rs:335-505: default theta^(-2i/d) (:498-505); linear divides by the
 * factor (:347-357); YaRN uses theta * factor^(d/(d-2)) (:367-392); dynamic
 * NTK recomputes the factor from the current length (:405-443, scale =
 * factor * cur/orig - (factor - 1) with one rounding); Su divides by
 * short/long per-dim factors on either side of the wavelength boundary
 * (:445-488).  Factors within f32 epsilon of 1 keep the default table.
 * rope_type: 0 default, 1 linear, 2 yarn, 3 dynamic, 4 su. */
void oracle_rope_inv_freq(int head_dim, float theta, int rope_type, float factor, int orig_max,
                          int cur_seq_len, const float* short_factor, const float* long_factor,
                          float* out) {
  int half = head_dim / 2;
  float th = theta;
  int near_one = fabsf(factor - 1.0f) < 1.1920929e-07f;
  if (rope_type == 2 && !near_one) {
    float d = (float)head_dim;
    th = theta * powf(factor, d / (d - 2.0f));
  } else if (rope_type == 3 && orig_max > 0 && cur_seq_len > orig_max && !near_one) {
    float scale = fmaf(factor, (float)cur_seq_len / (float)orig_max, -(factor - 1.0f));
    float d = (float)head_dim;
    th = theta * powf(scale, d / (d - 2.0f));
  }
  for (int i = 0; i < half; ++i) out[i] = powf(th, -2.0f * (float)i / (float)head_dim);
  if (rope_type == 1 && !near_one)
    for (int i = 0; i < half; ++i) out[i] = out[i] / factor;
  if (rope_type == 4 && orig_max > 0) {
    int boundary = half;
    for (int i = 0; i < half; ++i)
      if (2.0f * 3.14159265358979323846f / out[i] > (float)orig_max) {
        boundary = i;
        break;
      }
    for (int i = 0; i < half; ++i) {
      const float* f = i < boundary ? short_factor : long_factor;
      out[i] = out[i] / (f ? f[i] : 1.0f);
    }
  }
}

/* Rotate-half RoPE on x [T, H, D] (dtype), in place, token t at position
 * positions[t].  crates/model/src/components/positional/rope.rs:507-568:
 * angle = pos * inv_freq[i] (f32), x1' = x1 cos - x2 sin,
 * x2' = x2 cos + x1 sin on the halves x1 = x[:D/2], x2 = x[D/2:]. */
void oracle_rope(void* x, int T, int H, int D, const int64_t* positions, const float* inv_freq,
                 int dtype) {
  int half = D / 2;
  for (int t = 0; t < T; ++t)
    for (int h = 0; h < H; ++h) {
      size_t base = ((size_t)t * H + h) * D;
      for (int i = 0; i < half; ++i) {
        float angle = (float)positions[t] * inv_freq[i];
        float c = cosf(angle), s = sinf(angle);
        float x1 = load_el(x, base + i, dtype), x2 = load_el(x, base + half + i, dtype);
        store_el(x, base + i, x1 * c - x2 * s, dtype);
        store_el(x, base + half + i, x2 * c + x1 * s, dtype);
      }
    }
}

/* ---------------------------------------------------------------------- */
/* FP8 E4M3 KV codec, the reference's convention                           */
/* ---------------------------------------------------------------------- */

/* crates/model/src/components/kv_cache_fp8.rs:143-186
 * (Fp8Quantizer::float32_to_fp8_e4m3): sign bit 7, 4-bit exponent with
 * bias 7, 3-bit mantissa; normals only.  NaN -> 0x80, +-inf -> 0x7C / 0xFC;
 * |v| < 2^-6 (biased exponent <= 0 before rounding) -> +0; biased exponent
 * > 14 (before or after rounding) saturates to 0x7B / 0xFB; the [1, 2)
 * significand is rounded to 3 fraction bits half-up (fma(f, 8, 0.5)
 * truncated), a carry to 2.0 bumping the exponent. */
uint8_t oracle_fp8_encode(float v) {
  if (isnan(v)) return 0x80;
  if (isinf(v)) return v > 0 ? 0x7C : 0xFC;
  const uint8_t sign = signbit(v) ? 1 : 0;
  const float a = fabsf(v);
  if (a == 0.0f) return 0;
  int e2;
  const float half = frexpf(a, &e2); /* a = half * 2^e2, half in [0.5, 1) */
  const float f = half * 2.0f;       /* [1, 2) */
  int be = (e2 - 1) + 7;
  if (be <= 0) return 0;
  const uint8_t sat = sign ? 0xFB : 0x7B;
  if (be > 14) return sat;
  const unsigned im = (unsigned)fmaf(f, 8.0f, 0.5f); /* 8 .. 16 */
  unsigned frac;
  if (im >= 16) {
    be += 1;
    frac = 0;
  } else {
    frac = im - 8;
  }
  if (be > 14) return sat;
  return (uint8_t)((sign << 7) | ((unsigned)be << 3) | frac);
}

/* crates/model/src/components/kv_cache_fp8.rs:188-212
 * (fp8_e4m3_to_float16), as the f32 value of that f16: 0x80 -> NaN,
 * 0x7C / 0xFC -> +-inf, exponent and mantissa 0 -> +-0, otherwise
 * (-1)^s * 2^(e - 7) * (1 + m / 8) for every exponent field 0 .. 15. */
float oracle_fp8_decode(uint8_t b) {
  if (b == 0x80) return NAN;
  if (b == 0x7C) return INFINITY;
  if (b == 0xFC) return -INFINITY;
  const int sign = b >> 7, e = (b >> 3) & 15, m = b & 7;
  if (e == 0 && m == 0) return sign ? -0.0f : 0.0f;
  const float v = ldexpf(1.0f + (float)m / 8.0f, e - 7);
  return sign ? -v : v;
}

void oracle_fp8_encode_n(const float* x, uint8_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_fp8_encode(x[i]);
}

void oracle_fp8_decode_n(const uint8_t* x, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_fp8_decode(x[i]);
}
