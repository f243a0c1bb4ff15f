/*
 * CPU oracle for kvserve's attention hot path. TEST INFRASTRUCTURE ONLY: it is the checker
 * of tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, never a product path.
 *
 * Plain fp64 brute force, written from the closed form of the reference's semantics:
 *   paged attention  src/kvserve/attention.py:47-82 (TorchAttention.forward: causal mask
 *                    offset by the cached context, GQA head h -> kv head h / G) and
 *                    src/kvserve/kernels/paged_attention.py:50-115 (l == 0 -> divide by 1,
 *                    rows past q_len write nothing);
 *   reshape_and_cache src/kvserve/attention.py:39-45 (write_kv);
 *   slot formula     src/kvserve/kv_cache.py:155-169 (slot, slots).
 *
 * KVO_MUT_* flags plant one plausible mistake each; the tests show that every pinning check
 * (known answers, invariances, cross-checks) rejects at least the mutants it targets.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define KVO_MUT_GQA_MODULO 1   /* kv head = h % Hkv instead of h / G */
#define KVO_MUT_CAUSAL_OFF 2   /* query i sees keys 0 .. ctx + i - 1 (drops its own key) */
#define KVO_MUT_NO_SCALE 4     /* forgets the softmax scale */
#define KVO_MUT_PAGE_INDEX 8   /* page of key j taken as table[j % W] instead of table[j / BS] */
#define KVO_MUT_CTX_ZERO 16    /* causal offset ignores the cached context (ctx = 0) */
#define KVO_MUT_NO_MAXSHIFT 32 /* softmax without the max shift: same value until exp overflows */

/*
 * q [T, H, D], k_cache / v_cache [num_blocks, BS, Hkv, D], out [T, H, D], all contiguous fp64.
 * block_tables [B, W] int64; seq_lens [B]; query_start_loc [B + 1].
 * Returns 0, or -1 if a visible key's block id is outside [0, num_blocks) or the metadata
 * is inconsistent (the reference would index out of bounds).
 */
int kvo_paged_attention(const double* q, int64_t T, int32_t H, int32_t D, const double* k_cache,
                        const double* v_cache, int64_t num_blocks, int32_t BS, int32_t Hkv,
                        const int64_t* block_tables, int32_t W, const int64_t* seq_lens,
                        const int64_t* query_start_loc, int32_t B, double scale, int32_t flags, double* out) {
  if (H <= 0 || Hkv <= 0 || H % Hkv != 0 || D <= 0 || BS <= 0 || W <= 0) return -1;
  const int32_t G = H / Hkv;
  const double sc = (flags & KVO_MUT_NO_SCALE) ? 1.0 : scale;
  double* w = NULL;
  int64_t w_cap = 0;
  for (int32_t s = 0; s < B; ++s) {
    const int64_t q0 = query_start_loc[s], q1 = query_start_loc[s + 1];
    if (q0 < 0 || q1 < q0 || q1 > T) { free(w); return -1; }
    const int64_t q_len = q1 - q0;
    const int64_t ctx = (flags & KVO_MUT_CTX_ZERO) ? 0 : seq_lens[s] - q_len;
    for (int64_t i = 0; i < q_len; ++i) {
      int64_t n_keys = ctx + i + 1;  /* keys 0 .. ctx + i */
      if (flags & KVO_MUT_CAUSAL_OFF) n_keys -= 1;
      if (n_keys > seq_lens[s]) n_keys = seq_lens[s];
      if (n_keys < 0) n_keys = 0;
      if (n_keys > (int64_t)W * BS) { free(w); return -1; }
      if (n_keys > w_cap) {
        free(w);
        w_cap = n_keys;
        w = (double*)malloc(sizeof(double) * (size_t)(w_cap > 0 ? w_cap : 1));
      }
      for (int32_t h = 0; h < H; ++h) {
        const int32_t kvh = (flags & KVO_MUT_GQA_MODULO) ? h % Hkv : h / G;
        const double* qr = q + ((q0 + i) * H + h) * D;
        double* o = out + ((q0 + i) * H + h) * D;
        double mx = -INFINITY;
        for (int64_t j = 0; j < n_keys; ++j) {
          const int64_t page = (flags & KVO_MUT_PAGE_INDEX) ? j % W : j / BS;
          const int64_t blk = block_tables[(int64_t)s * W + page];
          if (blk < 0 || blk >= num_blocks) { free(w); return -1; }
          const double* kr = k_cache + ((blk * BS + j % BS) * Hkv + kvh) * D;
          double dot = 0.0;
          for (int32_t d = 0; d < D; ++d) dot += qr[d] * kr[d];
          w[j] = sc * dot;
          if (w[j] > mx) mx = w[j];
        }
        const double shift = (flags & KVO_MUT_NO_MAXSHIFT) ? 0.0 : mx;
        double sum = 0.0;
        for (int64_t j = 0; j < n_keys; ++j) {
          w[j] = exp(w[j] - shift);
          sum += w[j];
        }
        for (int32_t d = 0; d < D; ++d) o[d] = 0.0;
        for (int64_t j = 0; j < n_keys; ++j) {
          const int64_t page = (flags & KVO_MUT_PAGE_INDEX) ? j % W : j / BS;
          const int64_t blk = block_tables[(int64_t)s * W + page];
          const double* vr = v_cache + ((blk * BS + j % BS) * Hkv + kvh) * D;
          for (int32_t d = 0; d < D; ++d) o[d] += w[j] * vr[d];
        }
        const double inv = sum == 0.0 ? 1.0 : 1.0 / sum; /* empty row -> zeros */
        for (int32_t d = 0; d < D; ++d) o[d] *= inv;
      }
    }
  }
  free(w);
  return 0;
}

/*
 * write_kv: row t of k / v ([T, Hkv, D], elem_bytes per element, contiguous) is copied to
 * slot slots[t] of the contiguous caches [num_blocks, BS, Hkv, D]. Tokens are applied in
 * order, so the last of duplicate slots wins. Slots outside the pool are skipped.
 */
void kvo_reshape_and_cache(const void* k, const void* v, int64_t T, int32_t Hkv, int32_t D, int32_t elem_bytes,
                           const int64_t* slots, void* k_cache, void* v_cache, int64_t num_blocks, int32_t BS) {
  const size_t row = (size_t)Hkv * D * elem_bytes;
  for (int64_t t = 0; t < T; ++t) {
    const int64_t s = slots[t];
    if (s < 0 || s >= num_blocks * BS) continue;
    memcpy((char*)k_cache + (size_t)s * row, (const char*)k + (size_t)t * row, row);
    memcpy((char*)v_cache + (size_t)s * row, (const char*)v + (size_t)t * row, row);
  }
}

/* Slots of positions [start, start + n) of one sequence, one run per block
 * (src/kvserve/kv_cache.py:159-169). Returns the count written (n). */
int64_t kvo_slots(const int64_t* table, int32_t bs, int64_t start, int64_t n, int64_t* out) {
  int64_t pos = start, end = start + n, k = 0;
  while (pos < end) {
    const int64_t page = pos / bs;
    int64_t block_end = (page + 1) * bs;
    if (block_end > end) block_end = end;
    const int64_t base = table[page] * bs - page * bs;
    for (int64_t x = pos; x < block_end; ++x) out[k++] = base + x;
    pos = block_end;
  }
  return k;
}
