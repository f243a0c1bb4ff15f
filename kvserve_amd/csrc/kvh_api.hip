// C ABI of libkvhip: argument validation, the static launch plan and dispatch.
// Host code only; kernels live in paged_attention*.hip and reshape_and_cache.hip.
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <mutex>

#include "kvhip.h"  // include/ is on the include path
#include "kvh_device.h"
#include "kvh_internal.h"

namespace kvh {

namespace {

constexpr size_t kAlign = 256;
size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int elem_bytes(int dtype) { return dtype == KVH_DTYPE_F32 ? 4 : 2; }

// Launch-timing state of this host thread (see kvh_profile_arm).
struct ProfileState {
  void* events[8] = {nullptr};
  int32_t num_events = 0;
  int32_t last_kinds[8] = {0};
  int32_t last_count = 0;
};
thread_local ProfileState g_prof;

}  // namespace

void LaunchLog::after_launch(int kind, hipStream_t s) {
  if (launched < 8) kinds[launched] = kind;
  ++launched;
  if (events && launched < num_events && events[launched]) (void)hipEventRecord((hipEvent_t)events[launched], s);
}

Plan make_plan(int64_t T, int32_t B, int32_t H, int32_t Hkv, int32_t D, int32_t W, int32_t BS, int32_t max_q,
               int32_t dtype) {
  Plan pl{};
  pl.G = H / Hkv;
  if (max_q < 1) max_q = 1;
  const int G = pl.G;
  if ((int64_t)max_q * G <= 64) {
    // decode / speculative-verify batch: every sequence takes the stream-K decode kernel
    pl.QS = max_q;
    pl.launch_prefill = false;
  } else {
    // mixed batch: single-tile rows stream-K, everything longer on the prefill kernel
    pl.QS = G >= 16 ? 1 : 16 / G;
    pl.launch_prefill = true;
  }
  pl.NT = (pl.QS * G + 15) / 16;
  pl.RS = pl.QS * G;
  pl.HGW = Hkv % 8 == 0 ? 8 : (Hkv % 4 == 0 ? 4 : (Hkv % 2 == 0 ? 2 : 1));
  pl.slots = (int64_t)B * Hkv / pl.HGW + kMaxDecodeWaves / pl.HGW;
  pl.short_decode = !pl.launch_prefill && pl.NT == 1 && (int64_t)W * BS <= kShortTokens;
  if (dtype == KVH_DTYPE_F32 || !mfma_shape(D, BS, G) || pl.short_decode) {
    pl.ws_acc_bytes = pl.ws_ml_bytes = pl.ws_job_bytes = pl.ws_pacc_bytes = pl.ws_pml_bytes = pl.ws_plan_bytes =
        pl.ws_bytes = 0;
  } else {
    const size_t rows = (size_t)pl.slots * pl.HGW * pl.RS;
    pl.ws_acc_bytes = align_up(rows * D * sizeof(float));
    pl.ws_ml_bytes = align_up(rows * 2 * sizeof(float));
    const size_t jobs = kMaxDecodeWaves + (pl.launch_prefill ? kMaxPrefillUnits : 0);
    pl.ws_job_bytes = align_up(jobs * kJobInts * sizeof(int32_t));
    const size_t prows = pl.launch_prefill ? (size_t)2 * kMaxPrefillUnits * kPrefillRows : 0;
    pl.ws_pacc_bytes = align_up(prows * D * sizeof(float));
    pl.ws_pml_bytes = align_up(prows * 2 * sizeof(float));
    // plan: header, sequence list, flat starts, unit starts
    pl.ws_plan_bytes = pl.launch_prefill ? align_up(4 * sizeof(int64_t)) + align_up((size_t)B * sizeof(int32_t)) +
                                               align_up(((size_t)B + 1) * sizeof(int64_t)) +
                                               align_up((size_t)kMaxPrefillUnits * kPreRec * sizeof(int32_t))
                                         : 0;
    // cascade over a shared prefix: share header, decode list, prefix partials, merge jobs
    pl.cascade = !pl.launch_prefill && pl.NT == 1 && B >= 2 && (int64_t)W * BS > kCascadeMinTokens;
    // A prefix group stacks the query rows of SG = XR / RS members into NX 16-row tiles
    // (XR = 16 NX rows). When the batch holds more than one tile's worth: over 16-bit caches
    // four tiles (64 rows), so up to 64 / RS members read the shared K/V once; over E4M3
    // caches two (32 rows), the most that keeps the kernel at two waves per SIMD, which its
    // conversions need (cascade_tiles). The partials are sized for every choice.
    pl.NX = pl.cascade && (int64_t)B * pl.RS > 16 ? 4 : 1;
    const int64_t nhg = Hkv / pl.HGW;
    auto prefix_rows = [&](int nx) {
      const int xr = 16 * nx, sg = cascade_group(pl.RS, nx);
      return (((int64_t)B + sg - 1) / sg * nhg + kMaxCascadeWaves / pl.HGW) * pl.HGW * xr;
    };
    pl.xrows = pl.cascade ? std::max({prefix_rows(cascade_tiles(pl.NX, false)), prefix_rows(cascade_tiles(pl.NX, true)),
                                      prefix_rows(1)})
                          : 0;
    pl.ws_x_bytes = pl.cascade ? align_up(kShareHdr * sizeof(int64_t)) + align_up((size_t)B * sizeof(int32_t)) +
                                     align_up((size_t)pl.xrows * D * sizeof(float)) +
                                     align_up((size_t)pl.xrows * 2 * sizeof(float)) +
                                     align_up((size_t)B * nhg * kJobInts * sizeof(int32_t))
                               : 0;
    pl.ws_bytes = pl.ws_acc_bytes + pl.ws_ml_bytes + pl.ws_job_bytes + pl.ws_pacc_bytes + pl.ws_pml_bytes +
                  pl.ws_plan_bytes + pl.ws_x_bytes;
  }
  (void)T;
  return pl;
}

}  // namespace kvh

using namespace kvh;

extern "C" {

int kvh_abi_version(void) { return KVH_ABI_VERSION; }

const char* kvh_strerror(int status) {
  switch (status) {
    case KVH_OK: return "ok";
    case KVH_E_NULL: return "kvhip: a required pointer is NULL";
    case KVH_E_SHAPE: return "kvhip: size out of range or inconsistent";
    case KVH_E_DTYPE: return "kvhip: unknown dtype";
    case KVH_E_ALIGN: return "kvhip: pointer or stride not aligned (16-byte rows required)";
    case KVH_E_UNSUPPORTED: return "kvhip: unsupported head_dim / block_size / GQA combination";
    case KVH_E_WORKSPACE: return "kvhip: workspace missing or too small";
    case KVH_E_SCRATCH:
      return "kvhip: launch needs more workspace than the library's static scratch holds "
             "(KVH_STATIC_SCRATCH_BYTES); use kvh_paged_attention with a workspace";
    default: break;
  }
  if (status > 0) return hipGetErrorString((hipError_t)status);
  return "kvhip: unknown status";
}

int kvh_reshape_and_cache(const void* k, int64_t k_tok_stride, int64_t k_head_stride, const void* v,
                          int64_t v_tok_stride, int64_t v_head_stride, void* k_cache,
                          const int64_t k_cache_strides[3], void* v_cache, const int64_t v_cache_strides[3],
                          const int64_t* slot_mapping, int64_t num_tokens, int64_t num_blocks, int32_t num_kv_heads,
                          int32_t head_dim, int32_t block_size, int32_t dtype, void* stream) {
  if (dtype < KVH_DTYPE_F32 || dtype > KVH_DTYPE_BF16) return KVH_E_DTYPE;
  if (num_tokens < 0 || num_blocks < 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0)
    return KVH_E_SHAPE;
  const int eb = elem_bytes(dtype);
  // a token's K and V rows are indexed with 32-bit integers (element copies at worst)
  if (num_tokens > 0x7fffffffLL || (int64_t)num_kv_heads * head_dim * eb > (1 << 26)) return KVH_E_SHAPE;
  if (num_tokens == 0) return KVH_OK;
  if (!k || !v || !k_cache || !v_cache || !k_cache_strides || !v_cache_strides || !slot_mapping) return KVH_E_NULL;
  const int64_t strides[] = {k_tok_stride, k_head_stride, v_tok_stride, v_head_stride,
                             k_cache_strides[0], k_cache_strides[1], k_cache_strides[2],
                             v_cache_strides[0], v_cache_strides[1], v_cache_strides[2]};
  const int vec_elems = 16 / eb;
  bool vec16 = (head_dim * eb) % 16 == 0 && aligned16(k) && aligned16(v) && aligned16(k_cache) && aligned16(v_cache);
  for (int64_t s : strides) {
    if (s < 0) return KVH_E_SHAPE;
    vec16 = vec16 && s % vec_elems == 0;
  }
  const uintptr_t emask = (uintptr_t)eb - 1;
  if (((uintptr_t)k | (uintptr_t)v | (uintptr_t)k_cache | (uintptr_t)v_cache) & emask) return KVH_E_ALIGN;
  return launch_reshape_and_cache(k, k_tok_stride, k_head_stride, v, v_tok_stride, v_head_stride, k_cache,
                                  k_cache_strides, v_cache, v_cache_strides, slot_mapping, num_tokens, num_blocks,
                                  num_kv_heads, head_dim, block_size, eb, vec16, (hipStream_t)stream);
}

int kvh_reshape_and_cache_fp8(const void* k, int64_t k_tok_stride, int64_t k_head_stride, const void* v,
                              int64_t v_tok_stride, int64_t v_head_stride, void* k_cache,
                              const int64_t k_cache_strides[3], void* v_cache, const int64_t v_cache_strides[3],
                              const int64_t* slot_mapping, int64_t num_tokens, int64_t num_blocks,
                              int32_t num_kv_heads, int32_t head_dim, int32_t block_size, int32_t dtype,
                              float k_scale, float v_scale, void* stream) {
  if (dtype < KVH_DTYPE_F32 || dtype > KVH_DTYPE_BF16) return KVH_E_DTYPE;
  if (num_tokens < 0 || num_blocks < 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0)
    return KVH_E_SHAPE;
  if (!(k_scale > 0.f && k_scale < INFINITY && v_scale > 0.f && v_scale < INFINITY)) return KVH_E_SHAPE;
  if (num_tokens > 0x7fffffffLL || (int64_t)num_kv_heads * head_dim > (1 << 26)) return KVH_E_SHAPE;
  if (head_dim % 8 != 0) return KVH_E_UNSUPPORTED;
  if (num_tokens == 0) return KVH_OK;
  if (!k || !v || !k_cache || !v_cache || !k_cache_strides || !v_cache_strides || !slot_mapping) return KVH_E_NULL;
  const int vec = 16 / elem_bytes(dtype);  // source elements per 16 bytes
  const int64_t src[] = {k_tok_stride, k_head_stride, v_tok_stride, v_head_stride};
  const int64_t dst[] = {k_cache_strides[0], k_cache_strides[1], k_cache_strides[2],
                         v_cache_strides[0], v_cache_strides[1], v_cache_strides[2]};
  for (int64_t st : src) {
    if (st < 0) return KVH_E_SHAPE;
    if (st % vec) return KVH_E_ALIGN;
  }
  for (int64_t st : dst) {
    if (st < 0) return KVH_E_SHAPE;
    if (st % 8) return KVH_E_ALIGN;  // 8-byte stores of E4M3 bytes
  }
  if (!aligned16(k) || !aligned16(v) || ((uintptr_t)k_cache & 7u) || ((uintptr_t)v_cache & 7u)) return KVH_E_ALIGN;
  return launch_reshape_and_cache_fp8(k, k_tok_stride, k_head_stride, v, v_tok_stride, v_head_stride, k_cache,
                                      k_cache_strides, v_cache, v_cache_strides, slot_mapping, num_tokens, num_blocks,
                                      num_kv_heads, head_dim, block_size, dtype, k_scale, v_scale,
                                      (hipStream_t)stream);
}

}  // extern "C"

static int rope_and_cache_impl(const void* qkv, int64_t qkv_tok_stride, const int64_t* positions,
                               const float* cos_table, const float* sin_table, int64_t max_positions, void* q_out,
                               int64_t q_tok_stride, int64_t q_head_stride, void* k_cache,
                               const int64_t k_cache_strides[3], void* v_cache, const int64_t v_cache_strides[3],
                               const int64_t* slot_mapping, int64_t num_tokens, int64_t num_blocks, int32_t num_heads,
                               int32_t num_kv_heads, int32_t head_dim, int32_t block_size, int32_t dtype, bool kv8,
                               float k_scale, float v_scale, void* stream) {
  if (kv8 && !(k_scale > 0.f && k_scale < INFINITY && v_scale > 0.f && v_scale < INFINITY)) return KVH_E_SHAPE;
  if (dtype < KVH_DTYPE_F32 || dtype > KVH_DTYPE_BF16) return KVH_E_DTYPE;
  if (num_tokens < 0 || num_blocks < 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 ||
      max_positions <= 0)
    return KVH_E_SHAPE;
  if (num_tokens > 0x7fffffffLL || num_heads > 65535 || num_kv_heads > 65535) return KVH_E_SHAPE;
  if (num_tokens == 0) return KVH_OK;
  if (!qkv || !positions || !cos_table || !sin_table || !q_out || !k_cache || !v_cache || !k_cache_strides ||
      !v_cache_strides || !slot_mapping)
    return KVH_E_NULL;
  const int vec = 16 / elem_bytes(dtype);  // elements per 16-byte vector (E4M3 cache: vec bytes)
  if (head_dim % (2 * vec) != 0 || head_dim > 1024) return KVH_E_UNSUPPORTED;
  const int64_t strides[] = {qkv_tok_stride, q_tok_stride, q_head_stride, k_cache_strides[0], k_cache_strides[1],
                             k_cache_strides[2], v_cache_strides[0], v_cache_strides[1], v_cache_strides[2]};
  for (int64_t st : strides) {
    if (st < 0) return KVH_E_SHAPE;
    if (st % vec) return KVH_E_ALIGN;
  }
  if (qkv_tok_stride < (int64_t)(num_heads + 2 * num_kv_heads) * head_dim) return KVH_E_SHAPE;
  const bool caches_ok = kv8 ? !(((uintptr_t)k_cache | (uintptr_t)v_cache) & (uintptr_t)(vec - 1))
                             : aligned16(k_cache) && aligned16(v_cache);
  if (!aligned16(qkv) || !aligned16(q_out) || !caches_ok) return KVH_E_ALIGN;
  return launch_rope_and_cache(qkv, qkv_tok_stride, positions, cos_table, sin_table, max_positions, q_out,
                               q_tok_stride, q_head_stride, k_cache, k_cache_strides, v_cache, v_cache_strides,
                               slot_mapping, num_tokens, num_blocks, num_heads, num_kv_heads, head_dim, block_size,
                               dtype, kv8, k_scale, v_scale, (hipStream_t)stream);
}

extern "C" {

int kvh_rope_and_cache(const void* qkv, int64_t qkv_tok_stride, const int64_t* positions, const float* cos_table,
                       const float* sin_table, int64_t max_positions, void* q_out, int64_t q_tok_stride,
                       int64_t q_head_stride, void* k_cache, const int64_t k_cache_strides[3], void* v_cache,
                       const int64_t v_cache_strides[3], const int64_t* slot_mapping, int64_t num_tokens,
                       int64_t num_blocks, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                       int32_t block_size, int32_t dtype, void* stream) {
  return rope_and_cache_impl(qkv, qkv_tok_stride, positions, cos_table, sin_table, max_positions, q_out,
                             q_tok_stride, q_head_stride, k_cache, k_cache_strides, v_cache, v_cache_strides,
                             slot_mapping, num_tokens, num_blocks, num_heads, num_kv_heads, head_dim, block_size,
                             dtype, false, 1.f, 1.f, stream);
}

int kvh_rope_and_cache_fp8(const void* qkv, int64_t qkv_tok_stride, const int64_t* positions,
                           const float* cos_table, const float* sin_table, int64_t max_positions, void* q_out,
                           int64_t q_tok_stride, int64_t q_head_stride, void* k_cache,
                           const int64_t k_cache_strides[3], void* v_cache, const int64_t v_cache_strides[3],
                           const int64_t* slot_mapping, int64_t num_tokens, int64_t num_blocks, int32_t num_heads,
                           int32_t num_kv_heads, int32_t head_dim, int32_t block_size, int32_t dtype, float k_scale,
                           float v_scale, void* stream) {
  return rope_and_cache_impl(qkv, qkv_tok_stride, positions, cos_table, sin_table, max_positions, q_out,
                             q_tok_stride, q_head_stride, k_cache, k_cache_strides, v_cache, v_cache_strides,
                             slot_mapping, num_tokens, num_blocks, num_heads, num_kv_heads, head_dim, block_size,
                             dtype, true, k_scale, v_scale, stream);
}

int kvh_prepare_metadata(const int32_t* packed, int32_t num_seqs, int32_t num_pad_seqs, int32_t num_updates,
                         int64_t num_tokens, int64_t* table_pool, int32_t pool_rows, int64_t pool_row_stride,
                         int32_t pool_width, int64_t* block_tables, int64_t bt_row_stride, int32_t bt_width,
                         int64_t bt_pad, int64_t* slot_mapping, int64_t* positions, int64_t* input_ids,
                         int64_t* seq_lens, int64_t* query_lens, int64_t* query_start_loc, int64_t pad_slot,
                         int32_t block_size, void* stream) {
  if (num_seqs < 0 || num_pad_seqs < 0 || num_updates < 0 || num_tokens < 0 || pool_rows <= 0 || pool_width <= 0 ||
      pool_row_stride < pool_width || bt_width < 0 || block_size <= 0)
    return KVH_E_SHAPE;
  if (num_seqs + (int64_t)num_pad_seqs < 1 || num_seqs + (int64_t)num_pad_seqs > (1 << 24) ||
      num_tokens > 0x7fffffffLL || num_tokens + num_pad_seqs > 0x7fffffffLL)
    return KVH_E_SHAPE;
  if (bt_width > 0 && (!block_tables || bt_row_stride < bt_width)) return block_tables ? KVH_E_SHAPE : KVH_E_NULL;
  if (!table_pool || !slot_mapping || !seq_lens || !query_start_loc) return KVH_E_NULL;
  if (!packed && (num_seqs > 0 || num_updates > 0 || (input_ids && num_tokens > 0))) return KVH_E_NULL;
  const uintptr_t a8 = (uintptr_t)table_pool | (uintptr_t)block_tables | (uintptr_t)slot_mapping |
                       (uintptr_t)positions | (uintptr_t)input_ids | (uintptr_t)seq_lens | (uintptr_t)query_lens |
                       (uintptr_t)query_start_loc;
  if ((a8 & 7u) || ((uintptr_t)packed & 3u)) return KVH_E_ALIGN;
  MetaParams m{};
  m.seqs = packed;
  m.tokens = input_ids ? packed + 4 * (int64_t)num_seqs + 3 * (int64_t)num_updates : nullptr;
  m.pool = table_pool;
  m.pool_rows = pool_rows;
  m.pool_width = pool_width;
  m.pool_rs = pool_row_stride;
  m.bt = bt_width > 0 ? block_tables : nullptr;
  m.bt_rs = bt_row_stride;
  m.bt_width = bt_width;
  m.bt_pad = bt_pad;
  m.slots = slot_mapping;
  m.positions = positions;
  m.input_ids = input_ids;
  m.seq_lens = seq_lens;
  m.query_lens = query_lens;
  m.qsl = query_start_loc;
  m.pad_slot = pad_slot;
  m.T = num_tokens;
  m.B = num_seqs;
  m.P = num_pad_seqs;
  m.BS = block_size;
  return launch_prepare_metadata(m, packed ? packed + 4 * (int64_t)num_seqs : nullptr, num_updates,
                                 (hipStream_t)stream);
}

static int check_attention_shape(int64_t num_tokens, int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads,
                                 int32_t head_dim, int32_t max_blocks_per_seq, int32_t block_size, int32_t dtype) {
  if (dtype < KVH_DTYPE_F32 || dtype > KVH_DTYPE_BF16) return KVH_E_DTYPE;
  if (num_tokens < 0 || num_seqs < 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 ||
      block_size <= 0 || max_blocks_per_seq <= 0)
    return KVH_E_SHAPE;
  if (num_heads % num_kv_heads != 0) return KVH_E_SHAPE;
  if (num_seqs > 65535 || num_heads > 65535 || num_tokens > 0x7fffffffLL) return KVH_E_UNSUPPORTED;
  // query rows (token, head of a group) are indexed with 32-bit integers
  if (num_tokens * (num_heads / num_kv_heads) > 0x7fffffffLL) return KVH_E_UNSUPPORTED;
  if ((int64_t)max_blocks_per_seq * block_size >= 0x7fffffffLL) return KVH_E_UNSUPPORTED;
  // rows of whole 16-byte vectors, at most 256 elements (the vector-ALU kernel's query row)
  if (head_dim % (dtype == KVH_DTYPE_F32 ? 4 : 8) != 0 || head_dim > 256) return KVH_E_UNSUPPORTED;
  return KVH_OK;
}

size_t kvh_paged_attention_workspace_size(int64_t num_tokens, int32_t num_seqs, int32_t num_heads,
                                          int32_t num_kv_heads, int32_t head_dim, int32_t max_blocks_per_seq,
                                          int32_t block_size, int32_t max_query_len, int32_t dtype) {
  if (check_attention_shape(num_tokens, num_seqs, num_heads, num_kv_heads, head_dim, max_blocks_per_seq, block_size,
                            dtype) != KVH_OK)
    return 0;
  return make_plan(num_tokens, num_seqs, num_heads, num_kv_heads, head_dim, max_blocks_per_seq, block_size,
                   max_query_len, dtype)
      .ws_bytes;
}

}  // extern "C"

// kvh_paged_attention and kvh_paged_attention_fp8 (kv8: E4M3 caches with scales k_scale, v_scale).
static int paged_attention_impl(const void* q, int64_t q_tok_stride, int64_t q_head_stride, const void* k_cache,
                                const int64_t k_cache_strides[3], const void* v_cache,
                                const int64_t v_cache_strides[3], int64_t num_blocks, void* out, int64_t o_tok_stride,
                                int64_t o_head_stride, const int64_t* block_tables, int64_t bt_row_stride,
                                int32_t max_blocks_per_seq, const int64_t* seq_lens, const int64_t* query_start_loc,
                                int64_t num_tokens, int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads,
                                int32_t head_dim, int32_t block_size, int32_t max_query_len, float scale,
                                int32_t dtype, bool kv8, float k_scale, float v_scale, void* workspace,
                                size_t workspace_bytes, void* stream) {
  // the timing hook covers exactly one call, whatever its outcome
  LaunchLog log;
  void* armed[8];
  const int32_t n_armed = g_prof.num_events;
  memcpy(armed, g_prof.events, sizeof(armed));
  g_prof.num_events = 0;
  g_prof.last_count = 0;

  int st = check_attention_shape(num_tokens, num_seqs, num_heads, num_kv_heads, head_dim, max_blocks_per_seq,
                                 block_size, dtype);
  if (st != KVH_OK) return st;
  if (num_tokens == 0 || num_seqs == 0) return KVH_OK;
  if (!q || !k_cache || !v_cache || !k_cache_strides || !v_cache_strides || !out || !block_tables || !seq_lens ||
      !query_start_loc)
    return KVH_E_NULL;
  // num_blocks >= 1: the kernels read block 0 in place of an absent tile (and mask it out)
  if (num_blocks < 1 || bt_row_stride < max_blocks_per_seq) return KVH_E_SHAPE;
  if (kv8) {
    // E4M3 caches feed the 16-bit MFMA path only
    if (dtype == KVH_DTYPE_F32 || !mfma_shape(head_dim, block_size, num_heads / num_kv_heads))
      return KVH_E_UNSUPPORTED;
    if (!(k_scale > 0.f && k_scale < INFINITY && v_scale > 0.f && v_scale < INFINITY)) return KVH_E_SHAPE;
  }
  const int64_t strides[] = {q_tok_stride, q_head_stride, o_tok_stride, o_head_stride,
                             k_cache_strides[0], k_cache_strides[1], k_cache_strides[2],
                             v_cache_strides[0], v_cache_strides[1], v_cache_strides[2]};
  const int vec_elems = dtype == KVH_DTYPE_F32 ? 4 : 8;
  for (int i = 0; i < 10; ++i) {
    if (strides[i] < 0) return KVH_E_SHAPE;
    // E4M3 cache rows are read 16 bytes at a time: 16 one-byte elements
    if (strides[i] % (kv8 && i >= 4 ? 16 : vec_elems)) return KVH_E_ALIGN;
  }
  if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(out)) return KVH_E_ALIGN;

  const Plan plan = make_plan(num_tokens, num_seqs, num_heads, num_kv_heads, head_dim, max_blocks_per_seq, block_size,
                              max_query_len, dtype);
  if (plan.ws_bytes > 0 && (!workspace || workspace_bytes < plan.ws_bytes || !aligned16(workspace)))
    return KVH_E_WORKSPACE;

  PAParams p{};
  p.q = q;
  p.q_ts = q_tok_stride;
  p.q_hs = q_head_stride;
  p.kc = k_cache;
  p.k_sb = k_cache_strides[0];
  p.k_ss = k_cache_strides[1];
  p.k_sh = k_cache_strides[2];
  p.vc = v_cache;
  p.v_sb = v_cache_strides[0];
  p.v_ss = v_cache_strides[1];
  p.v_sh = v_cache_strides[2];
  p.num_blocks = num_blocks;
  p.out = out;
  p.o_ts = o_tok_stride;
  p.o_hs = o_head_stride;
  p.bt = block_tables;
  p.bt_rs = bt_row_stride;
  p.seq_lens = seq_lens;
  p.qsl = query_start_loc;
  p.T = num_tokens;
  p.W = max_blocks_per_seq;
  p.B = num_seqs;
  p.H = num_heads;
  p.Hkv = num_kv_heads;
  p.G = plan.G;
  p.BS = block_size;
  p.scale = scale;
  p.qk_scale = scale * kLog2e * (kv8 ? k_scale : 1.f);
  p.v_scale = kv8 ? v_scale : 1.f;
  p.QS = plan.QS;
  p.RS = plan.RS;
  p.HGW = plan.HGW;
  p.NU = 0;   // set by the decode launcher from the device's occupancy
  p.NUP = 0;  // set by the prefill launcher likewise
  p.CASC = 0;  // set by the launcher when the plan has the cascade path
  {
    const int nx = cascade_tiles(plan.NX, kv8);  // cascade prefix group: 16-row tiles (see make_plan)
    p.XR = 16 * nx;
    p.SG = cascade_group(plan.RS, nx);
  }
  p.PR = kPrefillRows;  // the prefill launcher sets its own tile rows
  if (plan.ws_bytes) {
    char* w = (char*)workspace;
    p.ws_acc = (float*)w;
    w += plan.ws_acc_bytes;
    p.ws_ml = (float*)w;
    w += plan.ws_ml_bytes;
    p.ws_job = (int32_t*)w;
    w += plan.ws_job_bytes;
    p.ws_pacc = plan.ws_pacc_bytes ? (float*)w : nullptr;
    w += plan.ws_pacc_bytes;
    p.ws_pml = plan.ws_pml_bytes ? (float*)w : nullptr;
    w += plan.ws_pml_bytes;
    if (plan.ws_plan_bytes) {
      p.ws_plan_hdr = (int64_t*)w;
      w += align_up(4 * sizeof(int64_t));
      p.ws_pre_list = (int32_t*)w;
      w += align_up((size_t)num_seqs * sizeof(int32_t));
      p.ws_pre_beg = (int64_t*)w;
      w += align_up(((size_t)num_seqs + 1) * sizeof(int64_t));
      p.ws_pre_unit = (int32_t*)w;
      w += align_up((size_t)kMaxPrefillUnits * kPreRec * sizeof(int32_t));
    }
    if (plan.ws_x_bytes) {
      const size_t rows = (size_t)plan.xrows;
      p.ws_share = (int64_t*)w;
      w += align_up(kShareHdr * sizeof(int64_t));
      p.ws_dec_list = (int32_t*)w;
      w += align_up((size_t)num_seqs * sizeof(int32_t));
      p.ws_xacc = (float*)w;
      w += align_up(rows * head_dim * sizeof(float));
      p.ws_xml = (float*)w;
      w += align_up(rows * 2 * sizeof(float));
      p.ws_xjob = (int32_t*)w;
    }
  }

  hipStream_t s = (hipStream_t)stream;
  if (n_armed > 0) {
    log.events = armed;
    log.num_events = n_armed;
    if (armed[0]) (void)hipEventRecord((hipEvent_t)armed[0], s);
  }
  if (dtype == KVH_DTYPE_F32 || !mfma_shape(head_dim, block_size, plan.G))
    st = launch_paged_attention_valu(p, head_dim, dtype, max_query_len < 1 ? 1 : max_query_len, s, log);
  else
    st = launch_paged_attention_mfma(p, plan, head_dim, dtype, kv8, max_query_len < 1 ? 1 : max_query_len, s, log);
  g_prof.last_count = log.launched;
  for (int i = 0; i < 8; ++i) g_prof.last_kinds[i] = log.kinds[i];
  return st;
}

// ---------------------------------------------------------------------------------------
// Static scratch for kvh_paged_attention_static: the split-K workspace as a device array of
// this library, so a caller that cannot allocate (HIP graph capture, serving loops that
// forbid hipMalloc) passes only inputs and outputs. Each device holds its own copy for the
// life of the process. In host code `g_static_scratch` is only the host-side handle of the
// array: its device address comes from hipGetSymbolAddress, once per device, with that
// device current, and only that address is ever handed to kernels.
static __device__ __align__(256) unsigned char g_static_scratch[KVH_STATIC_SCRATCH_BYTES];

namespace {
constexpr int kMaxScratchDevices = 64;
std::atomic<void*> g_scratch_addr[kMaxScratchDevices];
std::mutex g_scratch_mu;

// Device address of the current device's scratch (resolved on its first use there).
int static_scratch_address(void** addr) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxScratchDevices) return KVH_E_UNSUPPORTED;
  void* a = g_scratch_addr[dev].load(std::memory_order_acquire);
  if (!a) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    a = g_scratch_addr[dev].load(std::memory_order_relaxed);
    if (!a) {
      e = hipGetSymbolAddress(&a, HIP_SYMBOL(g_static_scratch));
      if (e != hipSuccess) return (int)e;
      if (!a) return (int)hipErrorInvalidSymbol;
      g_scratch_addr[dev].store(a, std::memory_order_release);
    }
  }
  *addr = a;
  return KVH_OK;
}
}  // namespace

extern "C" {

int kvh_paged_attention_static(const void* q, int64_t q_tok_stride, int64_t q_head_stride, const void* k_cache,
                               const int64_t k_cache_strides[3], const void* v_cache,
                               const int64_t v_cache_strides[3], int64_t num_blocks, void* out,
                               int64_t o_tok_stride, int64_t o_head_stride, const int64_t* block_tables,
                               int64_t bt_row_stride, int32_t max_blocks_per_seq, const int64_t* seq_lens,
                               const int64_t* query_start_loc, int64_t num_tokens, int32_t num_seqs,
                               int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                               int32_t max_query_len, float scale, int32_t dtype, void* stream) {
  int st = check_attention_shape(num_tokens, num_seqs, num_heads, num_kv_heads, head_dim, max_blocks_per_seq,
                                 block_size, dtype);
  if (st != KVH_OK) return st;
  if (num_tokens == 0 || num_seqs == 0) return KVH_OK;
  const size_t need = make_plan(num_tokens, num_seqs, num_heads, num_kv_heads, head_dim, max_blocks_per_seq,
                                block_size, max_query_len, dtype)
                          .ws_bytes;
  if (need > (size_t)KVH_STATIC_SCRATCH_BYTES) return KVH_E_SCRATCH;
  void* ws = nullptr;
  if (need > 0 && (st = static_scratch_address(&ws)) != KVH_OK) return st;
  return paged_attention_impl(q, q_tok_stride, q_head_stride, k_cache, k_cache_strides, v_cache, v_cache_strides,
                              num_blocks, out, o_tok_stride, o_head_stride, block_tables, bt_row_stride,
                              max_blocks_per_seq, seq_lens, query_start_loc, num_tokens, num_seqs, num_heads,
                              num_kv_heads, head_dim, block_size, max_query_len, scale, dtype, false, 1.f, 1.f, ws,
                              need > 0 ? (size_t)KVH_STATIC_SCRATCH_BYTES : 0, stream);
}

int kvh_paged_attention(const void* q, int64_t q_tok_stride, int64_t q_head_stride, const void* k_cache,
                        const int64_t k_cache_strides[3], const void* v_cache, const int64_t v_cache_strides[3],
                        int64_t num_blocks, void* out, int64_t o_tok_stride, int64_t o_head_stride,
                        const int64_t* block_tables, int64_t bt_row_stride, int32_t max_blocks_per_seq,
                        const int64_t* seq_lens, const int64_t* query_start_loc, int64_t num_tokens, int32_t num_seqs,
                        int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                        int32_t max_query_len, float scale, int32_t dtype, void* workspace, size_t workspace_bytes,
                        void* stream) {
  return paged_attention_impl(q, q_tok_stride, q_head_stride, k_cache, k_cache_strides, v_cache, v_cache_strides,
                              num_blocks, out, o_tok_stride, o_head_stride, block_tables, bt_row_stride,
                              max_blocks_per_seq, seq_lens, query_start_loc, num_tokens, num_seqs, num_heads,
                              num_kv_heads, head_dim, block_size, max_query_len, scale, dtype, false, 1.f, 1.f,
                              workspace, workspace_bytes, stream);
}

int kvh_paged_attention_fp8(const void* q, int64_t q_tok_stride, int64_t q_head_stride, const void* k_cache,
                            const int64_t k_cache_strides[3], const void* v_cache, const int64_t v_cache_strides[3],
                            int64_t num_blocks, void* out, int64_t o_tok_stride, int64_t o_head_stride,
                            const int64_t* block_tables, int64_t bt_row_stride, int32_t max_blocks_per_seq,
                            const int64_t* seq_lens, const int64_t* query_start_loc, int64_t num_tokens,
                            int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                            int32_t block_size, int32_t max_query_len, float scale, float k_scale, float v_scale,
                            int32_t dtype, void* workspace, size_t workspace_bytes, void* stream) {
  return paged_attention_impl(q, q_tok_stride, q_head_stride, k_cache, k_cache_strides, v_cache, v_cache_strides,
                              num_blocks, out, o_tok_stride, o_head_stride, block_tables, bt_row_stride,
                              max_blocks_per_seq, seq_lens, query_start_loc, num_tokens, num_seqs, num_heads,
                              num_kv_heads, head_dim, block_size, max_query_len, scale, dtype, true, k_scale, v_scale,
                              workspace, workspace_bytes, stream);
}

static bool a16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int kvh_add_rmsnorm(const void* x, int64_t x_tok_stride, const void* delta, int64_t delta_tok_stride,
                    const void* weight, void* x_out, int64_t x_out_tok_stride, void* h_out, int64_t h_tok_stride,
                    int64_t num_tokens, int32_t hidden, float eps, int32_t dtype, void* stream) {
  if (dtype != KVH_DTYPE_F16 && dtype != KVH_DTYPE_BF16) return KVH_E_DTYPE;
  if (num_tokens < 0 || num_tokens > 0x7fffffffLL || hidden <= 0 || !(eps >= 0.f)) return KVH_E_SHAPE;
  if (hidden % 8 != 0) return KVH_E_UNSUPPORTED;
  if (num_tokens == 0) return KVH_OK;
  if (!x || !weight || !h_out || (delta && !x_out)) return KVH_E_NULL;
  const int64_t st[] = {x_tok_stride, h_tok_stride, delta_tok_stride, x_out_tok_stride};
  for (int i = 0; i < (delta ? 4 : 2); ++i) {  // without delta, x_out and its stride are unused
    if (st[i] < hidden) return KVH_E_SHAPE;
    if (st[i] % 8) return KVH_E_ALIGN;
  }
  if (!a16(x) || !a16(weight) || !a16(h_out) || (delta && (!a16(delta) || !a16(x_out)))) return KVH_E_ALIGN;
  return launch_add_rmsnorm(x, x_tok_stride, delta, delta_tok_stride, weight, x_out, x_out_tok_stride, h_out,
                            h_tok_stride, num_tokens, hidden, eps, dtype, (hipStream_t)stream);
}

int kvh_silu_mul(const void* gate_up, int64_t gate_up_tok_stride, void* out, int64_t out_tok_stride,
                 int64_t num_tokens, int32_t intermediate, int32_t dtype, void* stream) {
  if (dtype != KVH_DTYPE_F16 && dtype != KVH_DTYPE_BF16) return KVH_E_DTYPE;
  if (num_tokens < 0 || num_tokens > 65535 || intermediate <= 0) return KVH_E_SHAPE;
  if (intermediate % 8 != 0) return KVH_E_UNSUPPORTED;
  if (num_tokens == 0) return KVH_OK;
  if (!gate_up || !out) return KVH_E_NULL;
  if (gate_up_tok_stride < 2 * (int64_t)intermediate || out_tok_stride < intermediate) return KVH_E_SHAPE;
  if (gate_up_tok_stride % 8 || out_tok_stride % 8 || !a16(gate_up) || !a16(out)) return KVH_E_ALIGN;
  return launch_silu_mul(gate_up, gate_up_tok_stride, out, out_tok_stride, num_tokens, intermediate, dtype,
                         (hipStream_t)stream);
}

int kvh_gemv(const void* x, int64_t x_row_stride, const void* weight, int64_t w_row_stride, void* y,
             int64_t y_row_stride, int32_t m, int32_t n, int32_t k, int32_t dtype, void* stream) {
  if (dtype != KVH_DTYPE_F16 && dtype != KVH_DTYPE_BF16) return KVH_E_DTYPE;
  if (m < 0 || n < 0 || k <= 0) return KVH_E_SHAPE;
  if (m > 8 || k % 8 != 0) return KVH_E_UNSUPPORTED;
  if (m == 0 || n == 0) return KVH_OK;
  if (!x || !weight || !y) return KVH_E_NULL;
  if (x_row_stride < k || w_row_stride < k || y_row_stride < n) return KVH_E_SHAPE;
  if (x_row_stride % 8 || w_row_stride % 8 || !a16(x) || !a16(weight) || ((uintptr_t)y & 1u)) return KVH_E_ALIGN;
  return launch_gemv(x, x_row_stride, weight, w_row_stride, y, y_row_stride, m, n, k, dtype, (hipStream_t)stream);
}

int kvh_gemv_silu_mul(const void* x, int64_t x_row_stride, const void* w_gate_up, int64_t w_row_stride, void* y,
                      int64_t y_row_stride, int32_t m, int32_t inter, int32_t k, int32_t dtype, void* stream) {
  if (dtype != KVH_DTYPE_F16 && dtype != KVH_DTYPE_BF16) return KVH_E_DTYPE;
  if (m < 0 || inter < 0 || k <= 0) return KVH_E_SHAPE;
  if (m > 4 || k % 8 != 0) return KVH_E_UNSUPPORTED;
  if (m == 0 || inter == 0) return KVH_OK;
  if (!x || !w_gate_up || !y) return KVH_E_NULL;
  if (x_row_stride < k || w_row_stride < k || y_row_stride < inter) return KVH_E_SHAPE;
  if (x_row_stride % 8 || w_row_stride % 8 || !a16(x) || !a16(w_gate_up) || ((uintptr_t)y & 1u)) return KVH_E_ALIGN;
  return launch_gemv_silu_mul(x, x_row_stride, w_gate_up, w_row_stride, y, y_row_stride, m, inter, k, dtype,
                              (hipStream_t)stream);
}

int kvh_gemv_rope_and_cache(const void* x, int64_t x_row_stride, const void* w_qkv, int64_t w_row_stride,
                            int32_t m, int32_t k, const int64_t* positions, const float* cos_table,
                            const float* sin_table, int64_t max_positions, void* q_out, int64_t q_tok_stride,
                            int64_t q_head_stride, void* k_cache, const int64_t k_cache_strides[3], void* v_cache,
                            const int64_t v_cache_strides[3], const int64_t* slot_mapping, int64_t num_blocks,
                            int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                            int32_t dtype, int32_t kv_fp8, float k_scale, float v_scale, void* stream) {
  if (dtype != KVH_DTYPE_F16 && dtype != KVH_DTYPE_BF16) return KVH_E_DTYPE;
  if (kv_fp8 && !(k_scale > 0.f && k_scale < INFINITY && v_scale > 0.f && v_scale < INFINITY)) return KVH_E_SHAPE;
  if (m < 0 || k <= 0 || num_blocks < 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 ||
      block_size <= 0 || max_positions <= 0)
    return KVH_E_SHAPE;
  if (m > 64 || k % 8 != 0 || head_dim % 2 != 0 || head_dim > 1024 || num_heads > 65535 || num_kv_heads > 65535)
    return KVH_E_UNSUPPORTED;
  if (m > 4 && (k % 1024 != 0 || head_dim % 16 != 0)) return KVH_E_UNSUPPORTED;  // the skinny form
  if (m == 0) return KVH_OK;
  if (!x || !w_qkv || !positions || !cos_table || !sin_table || !q_out || !k_cache || !v_cache || !k_cache_strides ||
      !v_cache_strides || !slot_mapping)
    return KVH_E_NULL;
  const int64_t strides[] = {q_tok_stride, q_head_stride, k_cache_strides[0], k_cache_strides[1],
                             k_cache_strides[2], v_cache_strides[0], v_cache_strides[1], v_cache_strides[2]};
  for (int64_t st : strides)
    if (st < 0) return KVH_E_SHAPE;
  if (x_row_stride < k || w_row_stride < k) return KVH_E_SHAPE;
  if (x_row_stride % 8 || w_row_stride % 8 || !a16(x) || !a16(w_qkv) || ((uintptr_t)q_out & 1u)) return KVH_E_ALIGN;
  if (!kv_fp8 && (((uintptr_t)k_cache | (uintptr_t)v_cache) & 1u)) return KVH_E_ALIGN;
  return launch_gemv_rope_and_cache(x, x_row_stride, w_qkv, w_row_stride, m, k, positions, cos_table, sin_table,
                                    max_positions, q_out, q_tok_stride, q_head_stride, k_cache, k_cache_strides,
                                    v_cache, v_cache_strides, slot_mapping, num_blocks, num_heads, num_kv_heads,
                                    head_dim, block_size, dtype, kv_fp8 != 0, k_scale, v_scale, (hipStream_t)stream);
}

int kvh_gemm_skinny(const void* x, int64_t x_row_stride, const void* weight, int64_t w_row_stride, void* y,
                    int64_t y_row_stride, int32_t m, int32_t n, int32_t k, int32_t dtype, void* stream) {
  if (dtype != KVH_DTYPE_F16 && dtype != KVH_DTYPE_BF16) return KVH_E_DTYPE;
  if (m < 0 || n < 0 || k <= 0) return KVH_E_SHAPE;
  if (m > 64 || n % 16 != 0 || k % 1024 != 0) return KVH_E_UNSUPPORTED;
  if (m == 0 || n == 0) return KVH_OK;
  if (!x || !weight || !y) return KVH_E_NULL;
  if (x_row_stride < k || w_row_stride < k || y_row_stride < n) return KVH_E_SHAPE;
  if (x_row_stride % 8 || w_row_stride % 8 || !a16(x) || !a16(weight) || ((uintptr_t)y & 1u)) return KVH_E_ALIGN;
  return launch_gemm_skinny(x, x_row_stride, weight, w_row_stride, y, y_row_stride, m, n, k, false, dtype,
                            (hipStream_t)stream);
}

int kvh_gemm_skinny_silu_mul(const void* x, int64_t x_row_stride, const void* w_gate_up, int64_t w_row_stride,
                             void* y, int64_t y_row_stride, int32_t m, int32_t inter, int32_t k, int32_t dtype,
                             void* stream) {
  if (dtype != KVH_DTYPE_F16 && dtype != KVH_DTYPE_BF16) return KVH_E_DTYPE;
  if (m < 0 || inter < 0 || k <= 0) return KVH_E_SHAPE;
  if (m > 64 || inter % 8 != 0 || k % 1024 != 0) return KVH_E_UNSUPPORTED;
  if (m == 0 || inter == 0) return KVH_OK;
  if (!x || !w_gate_up || !y) return KVH_E_NULL;
  if (x_row_stride < k || w_row_stride < k || y_row_stride < inter) return KVH_E_SHAPE;
  if (x_row_stride % 8 || w_row_stride % 8 || !a16(x) || !a16(w_gate_up) || ((uintptr_t)y & 1u)) return KVH_E_ALIGN;
  return launch_gemm_skinny(x, x_row_stride, w_gate_up, w_row_stride, y, y_row_stride, m, inter, k, true, dtype,
                            (hipStream_t)stream);
}

int kvh_profile_arm(void* const* events, int32_t num_events) {
  if (!events || num_events <= 0) {
    g_prof.num_events = 0;
    return KVH_OK;
  }
  if (num_events > 8) num_events = 8;
  for (int i = 0; i < num_events; ++i) g_prof.events[i] = events[i];
  g_prof.num_events = num_events;
  return KVH_OK;
}

int kvh_probe(int32_t kind, const void* src, void* dst, int64_t bytes, int32_t blocks, int32_t iters,
              void* stream) {
  if (kind < KVH_PROBE_STREAM_READ || kind > KVH_PROBE_PAGE_GATHER) return KVH_E_SHAPE;
  if (blocks < 1 || blocks > 65535) return KVH_E_SHAPE;
  const bool compute = kind >= KVH_PROBE_MFMA && kind <= KVH_PROBE_INTERLEAVE;
  if (!dst || (!compute && !src)) return KVH_E_NULL;
  if ((kind == KVH_PROBE_MFMA || kind == KVH_PROBE_INTERLEAVE) && iters <= 0) return KVH_E_SHAPE;
  if (kind == KVH_PROBE_INTERLEAVE && (bytes < 0 || bytes > 4)) return KVH_E_SHAPE;
  if (kind == KVH_PROBE_COISSUE && (iters < 0 || bytes < 0 || bytes > 0x7fffffff || (iters == 0 && bytes == 0)))
    return KVH_E_SHAPE;
  if (!compute && (bytes <= 0 || bytes % 16 != 0)) return KVH_E_SHAPE;
  if (kind == KVH_PROBE_PAGE_GATHER && (bytes % 4096 != 0 || ((bytes / 4096) & (bytes / 4096 - 1)) != 0))
    return KVH_E_SHAPE;  // a power-of-two count of 4 KB pages
  if (!aligned16(dst) || (!compute && !aligned16(src))) return KVH_E_ALIGN;
  return launch_probe(kind, src, dst, bytes, blocks, iters, (hipStream_t)stream);
}

int kvh_last_launch_kernels(int32_t* kinds, int32_t cap) {
  const int n = g_prof.last_count;
  for (int i = 0; i < n && i < cap && i < 8; ++i) kinds[i] = g_prof.last_kinds[i];
  return n;
}

}  // extern "C"
