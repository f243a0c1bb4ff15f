/*
 * kvhip.h - C ABI of the MI355X (gfx950) paged-attention backend for kvserve.
 *
 * Plain C: pointers, sizes and int64 strides only; no torch or HIP types cross this
 * boundary (a stream is passed as the opaque hipStream_t handle, typed void*).
 * Every entry point is reentrant, allocates no device memory, never synchronises the
 * stream and never throws: failures come back as a status code.
 *
 * Status codes: 0 = OK, < 0 = invalid argument (see KVH_E_*), > 0 = hipError_t of a
 * failed launch. kvh_strerror() turns either kind into text.
 *
 * Element types (KVH_DTYPE_*) select the storage type of q, k, v, the caches and out.
 * bf16/fp16 use the MFMA kernels (fp32 accumulation); fp32 uses exact fp32 FMA.
 *
 * Tensor conventions (all strides in ELEMENTS, last dim contiguous):
 *   q, out             [num_tokens, num_heads, head_dim]   flat token batch
 *   k, v (new tokens)  [num_tokens, num_kv_heads, head_dim]
 *   k_cache, v_cache   [num_blocks, block_size, num_kv_heads, head_dim]
 *                      cache_strides = {block, slot, head}
 *   block_tables       int64 [num_seqs, row_stride], first max_blocks_per_seq used
 *   seq_lens           int64 [num_seqs]  context length INCLUDING this step's tokens
 *   query_start_loc    int64 [num_seqs + 1] prefix sums of per-sequence query lengths
 *   slot_mapping       int64 [num_tokens] flat slot = block * block_size + offset
 */
#ifndef KVHIP_H
#define KVHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KVH_ABI_VERSION 1

#if defined(__GNUC__)
#define KVH_API __attribute__((visibility("default")))
#else
#define KVH_API
#endif

enum kvh_dtype {
  KVH_DTYPE_F32 = 0,
  KVH_DTYPE_F16 = 1,
  KVH_DTYPE_BF16 = 2,
};

enum kvh_status {
  KVH_OK = 0,
  KVH_E_NULL = -1,        /* a required pointer is NULL */
  KVH_E_SHAPE = -2,       /* a size (or an FP8 scale) is out of range or inconsistent */
  KVH_E_DTYPE = -3,       /* unknown dtype */
  KVH_E_ALIGN = -4,       /* pointer/stride not aligned for the vector kernels */
  KVH_E_UNSUPPORTED = -5, /* valid, but not a head_dim/block_size/GQA combination built here */
  KVH_E_WORKSPACE = -6,   /* workspace missing or smaller than kvh_paged_attention_workspace_size() */
  KVH_E_SCRATCH = -7,     /* kvh_paged_attention_static: the launch needs more than KVH_STATIC_SCRATCH_BYTES */
};

/* ABI version this library was built with (KVH_ABI_VERSION). */
KVH_API int kvh_abi_version(void);

/* Static text for a status code (negative: argument errors, positive: hipError_t). */
KVH_API const char* kvh_strerror(int status);

/*
 * reshape_and_cache: scatter this step's K/V rows into the paged pool.
 *   k_cache[slot / block_size, slot % block_size, h, :] = k[t, h, :]   (same for v)
 * with slot = slot_mapping[t]. k and v may have any token/head stride (v is usually a
 * strided view of the fused QKV output). Duplicate slots are allowed (CUDA-graph padding
 * rows all write the scratch slot); which duplicate wins is unspecified, as with the
 * reference. Slots outside [0, num_blocks * block_size) are skipped.
 *
 * Replaces TorchAttention.write_kv, src/kvserve/attention.py:39-45 (two index_put_ scatters).
 */
KVH_API int kvh_reshape_and_cache(const void* k, int64_t k_tok_stride, int64_t k_head_stride,
                          const void* v, int64_t v_tok_stride, int64_t v_head_stride,
                          void* k_cache, const int64_t k_cache_strides[3],
                          void* v_cache, const int64_t v_cache_strides[3],
                          const int64_t* slot_mapping, int64_t num_tokens, int64_t num_blocks,
                          int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                          int32_t dtype, void* stream);

/*
 * FP8 KV cache. k_cache / v_cache hold OCP FP8 E4M3 bytes (PyTorch's float8_e4m3fn: bias 7,
 * no infinities, 0x7f / 0xff NaN, largest finite 448), same shape and strides (in elements =
 * bytes) as a 16-bit cache, with one positive scale per tensor: a value x is stored as
 *   e4m3(clamp(x / scale, -448, 448))      round to nearest even; NaN stays NaN
 * which is PyTorch's (x.float() / scale).clamp(-448, 448).to(torch.float8_e4m3fn) bit for bit,
 * and read back as e4m3 * scale. The reference has no FP8 cache (a roadmap item,
 * README.md:431); this format halves the bytes decode attention streams.
 *
 * reshape_and_cache_fp8: kvh_reshape_and_cache into an E4M3 cache; dtype is that of k and v
 * (fp32, fp16 or bf16). head_dim % 8 == 0; k, v 16-byte aligned with strides multiples of 16
 * bytes; caches 8-byte aligned with strides multiples of 8.
 */
KVH_API int kvh_reshape_and_cache_fp8(const void* k, int64_t k_tok_stride, int64_t k_head_stride,
                              const void* v, int64_t v_tok_stride, int64_t v_head_stride,
                              void* k_cache, const int64_t k_cache_strides[3],
                              void* v_cache, const int64_t v_cache_strides[3],
                              const int64_t* slot_mapping, int64_t num_tokens, int64_t num_blocks,
                              int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                              int32_t dtype, float k_scale, float v_scale, void* stream);

/*
 * rope_and_cache: the step before attention in one pass. From this step's fused QKV
 * projection qkv [num_tokens, (num_heads + 2 num_kv_heads) head_dim] (token stride
 * qkv_tok_stride; query heads first, then key heads, then value heads) it computes, for
 * token t at position p = positions[t] (clamped to the tables),
 *   x' = x * cos[p] + rotate_half(x) * sin[p],  rotate_half(x) = (-x[D/2:], x[:D/2])
 * for every query and key head, writes the rotated queries to q_out [num_tokens, num_heads,
 * head_dim] and scatters the rotated keys and the unrotated values into the paged pool at
 * slot_mapping[t] like kvh_reshape_and_cache (slots outside the pool are skipped).
 * cos_table / sin_table: fp32 [max_positions, head_dim] (both halves of a row present).
 * For 16-bit storage the table values are rounded to the storage type and each product and
 * the sum are rounded to it, which reproduces PyTorch's separate bf16 / fp16 operations
 * bit for bit. head_dim must be a multiple of 16 (8 for fp32); pointers 16-byte aligned and
 * strides multiples of 16 bytes.
 *
 * Replaces the split + RoPE of Attention.project (src/kvserve/model.py:84-94, :55-70) and
 * TorchAttention.write_kv (src/kvserve/attention.py:39-45): one kernel instead of about a
 * dozen elementwise kernels and two index_put_ scatters per layer.
 */
KVH_API int kvh_rope_and_cache(const void* qkv, int64_t qkv_tok_stride, const int64_t* positions,
                       const float* cos_table, const float* sin_table, int64_t max_positions,
                       void* q_out, int64_t q_tok_stride, int64_t q_head_stride,
                       void* k_cache, const int64_t k_cache_strides[3],
                       void* v_cache, const int64_t v_cache_strides[3],
                       const int64_t* slot_mapping, int64_t num_tokens, int64_t num_blocks,
                       int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                       int32_t dtype, void* stream);

/* rope_and_cache into E4M3 caches (see reshape_and_cache_fp8): the rotated keys, rounded to
 * the storage type exactly as above, and the values are stored with k_scale / v_scale. */
KVH_API int kvh_rope_and_cache_fp8(const void* qkv, int64_t qkv_tok_stride, const int64_t* positions,
                           const float* cos_table, const float* sin_table, int64_t max_positions,
                           void* q_out, int64_t q_tok_stride, int64_t q_head_stride,
                           void* k_cache, const int64_t k_cache_strides[3],
                           void* v_cache, const int64_t v_cache_strides[3],
                           const int64_t* slot_mapping, int64_t num_tokens, int64_t num_blocks,
                           int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                           int32_t dtype, float k_scale, float v_scale, void* stream);

/*
 * prepare_metadata: one step's attention metadata, built on the device from block tables that
 * stay resident in HBM. table_pool int64 [pool_rows, pool_row_stride] holds one row per live
 * sequence (its block table, first pool_width entries usable) and persists across calls; the
 * caller sends only what changed. packed is DEVICE memory (one upload per step), int32:
 *   [num_seqs][4]     row, start (first position computed this step), q_len, n_blocks
 *   [num_updates][3]  row, column, block id: set table_pool[row][column] = block id first
 *                     (at most one update per entry per call)
 *   [num_tokens]      input token ids, present only when input_ids != NULL
 * For sequence b (in order; query_start_loc[b] = sum of the earlier q_len) and its token i,
 * position p = start + i:
 *   slot_mapping[t] = table_pool[row][p / block_size] * block_size + p % block_size  (-1 when
 *                     p / block_size >= n_blocks), positions[t] = p, input_ids[t] = token id,
 *   seq_lens[b] = start + q_len, query_lens[b] = q_len,
 *   block_tables[b][c] = table_pool[row][c] for c < n_blocks, bt_pad for n_blocks <= c < bt_width.
 * num_pad_seqs rows follow, each one token: slot pad_slot, position 0, token 0, seq_len 1,
 * q_len 1, a block-table row of bt_pad. Output arrays hold num_tokens + num_pad_seqs tokens and
 * num_seqs + num_pad_seqs rows (+1 for query_start_loc); positions, input_ids and query_lens may
 * be NULL; bt_width = 0 leaves block_tables untouched. Updates outside the pool are skipped.
 *
 * Replaces build_metadata (src/kvserve/model_runner.py:165-197, the Triton layout: tables
 * 0-padded, bt_pad = 0) with the slot formula of KVCacheManager.slots (kv_cache.py:155-169),
 * and the static-buffer refresh of DecodeGraphRunner.run (src/kvserve/cuda_graph.py:111-134:
 * scratch padding, bt_pad = scratch block, only the first bt_width columns written).
 */
KVH_API int kvh_prepare_metadata(const int32_t* packed, int32_t num_seqs, int32_t num_pad_seqs, int32_t num_updates,
                         int64_t num_tokens, int64_t* table_pool, int32_t pool_rows, int64_t pool_row_stride,
                         int32_t pool_width, int64_t* block_tables, int64_t bt_row_stride, int32_t bt_width,
                         int64_t bt_pad, int64_t* slot_mapping, int64_t* positions, int64_t* input_ids,
                         int64_t* seq_lens, int64_t* query_lens, int64_t* query_start_loc, int64_t pad_slot,
                         int32_t block_size, void* stream);

/*
 * Bytes of device workspace kvh_paged_attention needs for this launch shape. Depends only
 * on static quantities (shapes, the block-table width and max_query_len), so a CUDA/HIP
 * graph can allocate it once at capture. May return 0.
 */
KVH_API size_t kvh_paged_attention_workspace_size(int64_t num_tokens, int32_t num_seqs, int32_t num_heads,
                                          int32_t num_kv_heads, int32_t head_dim,
                                          int32_t max_blocks_per_seq, int32_t block_size,
                                          int32_t max_query_len, int32_t dtype);

/*
 * Paged attention over a flat batch that mixes decode tokens and prefill chunks.
 * For query token i of sequence s (absolute position ctx + i, ctx = seq_len - q_len) and
 * head h (kv head h / (num_heads / num_kv_heads)):
 *   out[t, h] = softmax_j(scale * q[t, h] . K[j]) V[j],  j = 0 .. ctx + i   (causal)
 * with K/V read at cache[block_tables[s, j / block_size], j % block_size, h_kv].
 * A row with no visible key writes zeros.
 *
 * max_query_len must bound every sequence's query length (host int, as in the reference);
 * max_blocks_per_seq is the block-table width W (static under graph capture). Only the
 * first ceil(seq_len / block_size) table entries of a row are read; ids outside
 * [0, num_blocks) are treated as empty pages. The call does not depend on max_seq_len.
 *
 * Shared prefixes: for a decode-only batch (max_query_len * G <= 16) with
 * max_blocks_per_seq * block_size > 8192, a small kernel first finds on the device the
 * longest run of table columns that every decode sequence with >= 256 context tokens shares
 * with the first one (prefix caching hands them the same physical blocks); those keys are
 * then read once per group of 16 / (max_query_len * G) sequences instead of once per
 * sequence. The result is the same attention; the workspace size covers it.
 *
 * Replaces paged_attention(), src/kvserve/kernels/paged_attention.py:118-157, as called by
 * TritonAttention.forward, src/kvserve/attention.py:88-102.
 */
KVH_API int kvh_paged_attention(const void* q, int64_t q_tok_stride, int64_t q_head_stride,
                        const void* k_cache, const int64_t k_cache_strides[3],
                        const void* v_cache, const int64_t v_cache_strides[3],
                        int64_t num_blocks,
                        void* out, int64_t o_tok_stride, int64_t o_head_stride,
                        const int64_t* block_tables, int64_t bt_row_stride, int32_t max_blocks_per_seq,
                        const int64_t* seq_lens, const int64_t* query_start_loc,
                        int64_t num_tokens, int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads,
                        int32_t head_dim, int32_t block_size, int32_t max_query_len, float scale,
                        int32_t dtype, void* workspace, size_t workspace_bytes, void* stream);

/*
 * kvh_paged_attention_static: kvh_paged_attention without a workspace argument and without
 * any allocation. No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops and harnesses that forbid
 * hipMalloc); the caller passes only inputs and outputs. The split-K workspace is a static
 * device array of this library, KVH_STATIC_SCRATCH_BYTES (256 MiB) per device, held by every
 * device the library runs on until the process ends. Launches whose workspace
 * (kvh_paged_attention_workspace_size) exceeds it return KVH_E_SCRATCH before any GPU work.
 * At 8 kv heads x 128 (bf16) that admits decode batches of up to ~7k sequences, 5-token
 * verify of up to ~1.4k sequences and mixed prefill + decode steps with up to ~1.4k
 * sequences (the 2048-token step of 4 prefills and 512 decodes needs 205 MB).
 * Results are those of kvh_paged_attention on the same inputs, bit for bit.
 * All calls on one device share its array and nothing in it needs clearing between calls;
 * calls that overlap in time on one device (several host threads, or streams that do not
 * serialise) race on it. The stream must belong to the current device.
 */
#define KVH_STATIC_SCRATCH_BYTES (256u << 20)
KVH_API int kvh_paged_attention_static(const void* q, int64_t q_tok_stride, int64_t q_head_stride,
                               const void* k_cache, const int64_t k_cache_strides[3],
                               const void* v_cache, const int64_t v_cache_strides[3],
                               int64_t num_blocks,
                               void* out, int64_t o_tok_stride, int64_t o_head_stride,
                               const int64_t* block_tables, int64_t bt_row_stride, int32_t max_blocks_per_seq,
                               const int64_t* seq_lens, const int64_t* query_start_loc,
                               int64_t num_tokens, int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads,
                               int32_t head_dim, int32_t block_size, int32_t max_query_len, float scale,
                               int32_t dtype, void* stream);

/*
 * kvh_paged_attention over E4M3 caches (see reshape_and_cache_fp8): keys and values are
 * e4m3 * k_scale and e4m3 * v_scale. q and out are fp16 or bf16 (dtype); the E4M3 values
 * convert exactly to dtype for the MFMA contractions, k_scale joins the softmax scale and
 * v_scale the output normalisation, P is rounded to dtype before P.V as in the 16-bit path.
 * Cache strides must be multiples of 16 bytes; workspace as kvh_paged_attention_workspace_size
 * for the same shape and dtype.
 */
KVH_API int kvh_paged_attention_fp8(const void* q, int64_t q_tok_stride, int64_t q_head_stride,
                            const void* k_cache, const int64_t k_cache_strides[3],
                            const void* v_cache, const int64_t v_cache_strides[3],
                            int64_t num_blocks,
                            void* out, int64_t o_tok_stride, int64_t o_head_stride,
                            const int64_t* block_tables, int64_t bt_row_stride, int32_t max_blocks_per_seq,
                            const int64_t* seq_lens, const int64_t* query_start_loc,
                            int64_t num_tokens, int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads,
                            int32_t head_dim, int32_t block_size, int32_t max_query_len, float scale,
                            float k_scale, float v_scale, int32_t dtype,
                            void* workspace, size_t workspace_bytes, void* stream);

/*
 * Engine-harness kernels (no counterpart in the attention path; they serve the Llama layer
 * around it, src/kvserve/model.py:22-32 and its MLP), fp16 / bf16 rows with 16-byte aligned
 * pointers and strides that are multiples of 8 elements:
 *
 * add_rmsnorm: x' = x + delta rounded to dtype (written to x_out), then
 *   h_out = weight * (x' * rsqrt(mean(x'^2) + eps)).to(dtype), the statistics in fp32; with
 *   delta == NULL it is the plain RMSNorm of x (x_out unused). One pass instead of an add and
 *   seven PyTorch kernels. hidden % 8 == 0.
 */
KVH_API int kvh_add_rmsnorm(const void* x, int64_t x_tok_stride, const void* delta, int64_t delta_tok_stride,
                            const void* weight, void* x_out, int64_t x_out_tok_stride,
                            void* h_out, int64_t h_tok_stride, int64_t num_tokens, int32_t hidden, float eps,
                            int32_t dtype, void* stream);

/* silu_mul: out[t] = silu(gate_up[t, :I]).to(dtype) * gate_up[t, I:2I] (the fused gate/up
 * projection's halves), I = intermediate, I % 8 == 0, num_tokens <= 65535. */
KVH_API int kvh_silu_mul(const void* gate_up, int64_t gate_up_tok_stride, void* out, int64_t out_tok_stride,
                         int64_t num_tokens, int32_t intermediate, int32_t dtype, void* stream);

/* gemv: y[i][j] = sum_k x[i][k] * weight[j][k] (nn.Linear, weight [n, k] row-major) for
 * m <= 8 rows, fp32 accumulation, rounded to dtype; k % 8 == 0. Streams the weight once. */
KVH_API int kvh_gemv(const void* x, int64_t x_row_stride, const void* weight, int64_t w_row_stride,
                     void* y, int64_t y_row_stride, int32_t m, int32_t n, int32_t k, int32_t dtype, void* stream);

/* gemv_silu_mul: the fused gate_up projection followed by silu_mul (model.py MLP,
 * act(gate) * up of the chunked gate_up output), for m <= 4 rows: with g[i][j], u[i][j] the
 * projections on weight rows j and inter + j (w_gate_up is [2 * inter, k] row-major), each
 * rounded to dtype, y[i][j] = (silu(g).to(dtype) * u).to(dtype) -- the bits of kvh_gemv then
 * kvh_silu_mul. k % 8 == 0. */
/* gemv_rope_and_cache: the QKV projection of m <= 64 decode rows followed by
 * kvh_rope_and_cache (kv_fp8 = 0) or kvh_rope_and_cache_fp8 (kv_fp8 != 0) in one launch:
 * qkv = x @ w_qkv^T (w_qkv [(num_heads + 2 num_kv_heads) head_dim, k] row-major, fp32 sums
 * rounded to dtype, as kvh_gemv), then the rotated queries to q_out and the rotated keys and
 * the values to the caches at slot_mapping (slots outside the pool skipped), with the same bits
 * as the two calls in sequence. Replaces the QKV projection and Attention.project + write_kv of
 * a decode step (src/kvserve/model.py:84-94, src/kvserve/attention.py:39-45) at batch sizes
 * where the projection streams its weight; k % 8 == 0, head_dim even (m > 4: the MFMA form,
 * k % 1024 == 0 and head_dim % 16 == 0). */
KVH_API int kvh_gemv_rope_and_cache(const void* x, int64_t x_row_stride, const void* w_qkv, int64_t w_row_stride,
                                    int32_t m, int32_t k, const int64_t* positions, const float* cos_table,
                                    const float* sin_table, int64_t max_positions, void* q_out,
                                    int64_t q_tok_stride, int64_t q_head_stride, void* k_cache,
                                    const int64_t k_cache_strides[3], void* v_cache,
                                    const int64_t v_cache_strides[3], const int64_t* slot_mapping,
                                    int64_t num_blocks, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                    int32_t block_size, int32_t dtype, int32_t kv_fp8, float k_scale,
                                    float v_scale, void* stream);

/* gemm_skinny: y = x @ weight^T (nn.Linear, weight [n, k] row-major) for m <= 64 rows on the
 * MFMA units, fp32 accumulation (8 k-slices summed in order), rounded to dtype; n % 16 == 0,
 * k % 1024 == 0. For the decode-sized batches between kvh_gemv's 4 rows and a full GEMM. */
KVH_API int kvh_gemm_skinny(const void* x, int64_t x_row_stride, const void* weight, int64_t w_row_stride,
                            void* y, int64_t y_row_stride, int32_t m, int32_t n, int32_t k, int32_t dtype,
                            void* stream);

/* gemm_skinny_silu_mul: kvh_gemm_skinny of the fused gate_up projection (w_gate_up [2 inter, k])
 * followed by kvh_silu_mul in one launch, with the same bits; m <= 64, inter % 8 == 0,
 * k % 1024 == 0. */
KVH_API int kvh_gemm_skinny_silu_mul(const void* x, int64_t x_row_stride, const void* w_gate_up,
                                     int64_t w_row_stride, void* y, int64_t y_row_stride, int32_t m, int32_t inter,
                                     int32_t k, int32_t dtype, void* stream);

KVH_API int kvh_gemv_silu_mul(const void* x, int64_t x_row_stride, const void* w_gate_up, int64_t w_row_stride,
                              void* y, int64_t y_row_stride, int32_t m, int32_t inter, int32_t k, int32_t dtype,
                              void* stream);

/*
 * Launch-timing hook for benchmarks (no counterpart in the reference). When armed with an
 * array of n <= 8 hipEvent_t handles (created by the caller with timing enabled), the NEXT
 * kvh_paged_attention call on this host thread records events[0] on its stream before its
 * first kernel and events[k] right after its k-th kernel (k = 1 .. n-1), then disarms
 * itself. The call still launches all of its work. Pass events = NULL to disarm.
 */
KVH_API int kvh_profile_arm(void* const* events, int32_t num_events);

/* Kernels launched by the last kvh_paged_attention call on this thread, in launch order:
 * writes up to cap kernel-kind codes (KVH_KERNEL_*) and returns how many there were. */
enum kvh_kernel_kind {
  KVH_KERNEL_DECODE = 1,   /* stream-K decode-class work (q_len small) */
  KVH_KERNEL_PREFILL = 2,  /* stream-K prefill-class tiles (q_len large) */
  KVH_KERNEL_REDUCE = 3,   /* log-sum-exp merge of split decode segments and prefill tiles */
  KVH_KERNEL_F32 = 4,      /* exact fp32 path */
  KVH_KERNEL_SHARE = 5,    /* shared-prefix plan of the cascade decode (long tables, decode-only batches) */
  KVH_KERNEL_VALU16 = 6,   /* 16-bit shapes the MFMA kernels do not tile (vector-ALU kernel) */
};
KVH_API int kvh_last_launch_kernels(int32_t* kinds, int32_t cap);

/*
 * Measurement probes for benchmarks (no counterpart in the reference): the attainable rate of
 * the resources the attention kernels are bound by, with the access width they use.
 *   KVH_PROBE_STREAM_READ: reads `bytes` of src (16-byte loads, 8 in flight per thread, each
 *     workgroup a contiguous 1 / blocks of the buffer), writes one uint32 per thread of
 *     `blocks` x 256 to dst (an XOR of its reads).
 *   KVH_PROBE_COPY: copies `bytes` of src to dst (same loads and ranges, 16-byte stores).
 *   KVH_PROBE_MFMA: each wave of `blocks` x 4 runs 4 independent chains of `iters`
 *     v_mfma_f32_16x16x32_bf16 (16384 FLOP each); writes one float per thread to dst.
 *   KVH_PROBE_COISSUE: `blocks` workgroups of 512 threads (one per CU): on each SIMD one wave
 *     runs `iters` steps of 4 MFMA chains and a second wave `bytes` steps of a softmax's vector
 *     work (16 FMA + 16 exp2 + 8 bf16 packs + 8 dot2); either count may be 0 (those waves idle);
 *     writes one float per thread to dst.
 *   KVH_PROBE_INTERLEAVE: each wave of `blocks` x 4 runs `iters` steps of 8 MFMA chains, every
 *     MFMA followed by `bytes` (0-4) independent FMAs of the same wave; one float per thread.
 *   KVH_PROBE_STREAM_READ_NT: KVH_PROBE_STREAM_READ with non-temporal loads (the decode
 *     kernels' K/V loads).
 *   KVH_PROBE_PAGE_GATHER: reads the `bytes` / 4096 pages of 4 KB of src, a power-of-two count,
 *     in a scattered order (page (j * 0x9E3779B1) mod count at walk position j), each wave of
 *     `blocks` x 4 its own run of positions with 4 pages in flight, non-temporal loads (the
 *     decode kernels' access pattern); dst as for KVH_PROBE_STREAM_READ.
 * src and dst 16-byte aligned, bytes a positive multiple of 16 (stream / copy; of 4096 with a
 * power-of-two quotient for the page gather), blocks in [1, 65535], iters > 0 (mfma,
 * interleave). Launches on `stream` and returns at once.
 */
enum kvh_probe_kind {
  KVH_PROBE_STREAM_READ = 0,
  KVH_PROBE_COPY = 1,
  KVH_PROBE_MFMA = 2,
  KVH_PROBE_COISSUE = 3,
  KVH_PROBE_INTERLEAVE = 4,
  KVH_PROBE_STREAM_READ_NT = 5,
  KVH_PROBE_PAGE_GATHER = 6,
};
KVH_API int kvh_probe(int32_t kind, const void* src, void* dst, int64_t bytes, int32_t blocks, int32_t iters,
                      void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KVHIP_H */
