// Host/device shared launch structures of libkvhip (not part of the public C ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace kvh {

// Upper bound on the waves one decode launch uses (256 CUs x 8 waves per SIMD x 4 SIMDs
// would be 8192); the workspace is sized for it, so its size never depends on the device.
constexpr int32_t kMaxDecodeWaves = 8192;
// Workgroup slots of the prefill workspace: 256 CUs x 3 tiles of kPrefillRows rows; a launch
// of PR-row tiles takes at most kMaxPrefillUnits x kPrefillRows / PR units (512 at PR = 192).
constexpr int32_t kMaxPrefillUnits = 768;
// Query rows ((token, head) pairs of one kv head) of one prefill workgroup's tile; the
// prefill workspace holds 2 slots x kMaxPrefillUnits x kPrefillRows partial rows, and a
// launch's units x 2 x its tile rows (PAParams::PR) stay within that.
constexpr int32_t kPrefillRows = 128;
// Cascade decode over a shared prefix: planned when a decode-only batch has at most 16 query
// rows per sequence (one 16-row tile) and block tables longer than kCascadeMinTokens; used
// when the cascade members (decode-class sequences with at least kCascadeMinChunks chunks of
// context) share at least kCascadeMinChunks chunks of table prefix.
constexpr int32_t kCascadeMinTokens = 8192;
// Cascade launches use at most kMaxCascadeWaves waves (a 256-CU device holds 2048 waves of
// the single-tile decode kernel and 1024 of the 64-row-group one): the prefix partials, up
// to 64 rows per (slot, head), are sized for that many units, not for kMaxDecodeWaves.
constexpr int32_t kMaxCascadeWaves = 2048;
// Short decode: a decode-only batch of single-tile rows whose block tables hold at most
// kShortTokens keys takes one workgroup per (sequence, kv head); its 4 waves split the chunks
// and combine their partials in LDS, so nothing goes through the workspace and no merge
// launch follows.
constexpr int32_t kShortTokens = 1024;
constexpr int32_t kCascadeMinChunks = 8;
constexpr int32_t kShareHdr = 8;  // int64: shared tokens, prefix groups, row of the shared table, sequences
// Merge job record: int32 fields, one record per work unit (decode units first).
constexpr int32_t kJobInts = 16;
// Prefill plan record: int32 fields, one 64-byte record per prefill workgroup: [0] its unit u
// (-1: idle), [1] list index, [2] kv head, [3] tile, [4] offset within the tile, [5] sequence,
// [6] query length, [7] kv length, and int64 pairs: [8..9] first query token, [10..11]
// context length, [12..13] and [14..15] the flat range [x0, x1) of the unit.
constexpr int32_t kPreRec = 16;
constexpr int32_t kMaxJobs = kMaxDecodeWaves + kMaxPrefillUnits;

// Everything a paged-attention kernel reads, by value in the kernel argument segment.
// Strides are in elements; cache strides are {block, slot, head}.
struct PAParams {
  const void* q;
  int64_t q_ts, q_hs;
  const void* kc;
  int64_t k_sb, k_ss, k_sh;
  const void* vc;
  int64_t v_sb, v_ss, v_sh;
  int64_t num_blocks;
  void* out;
  int64_t o_ts, o_hs;
  const int64_t* bt;
  int64_t bt_rs;
  const int64_t* seq_lens;
  const int64_t* qsl;
  int64_t T;
  int32_t W, B, H, Hkv, G, BS;
  float scale;     // softmax scale as given
  float qk_scale;  // scale * log2(e) (* the K scale of an E4M3 cache): scores in the exp2 domain
  int32_t QS;      // sequences with 0 < q_len <= QS are decode class (stream-K kernel)
  int32_t RS;      // query rows of a decode-class sequence at most: QS * G
  int32_t HGW;     // kv heads (waves) per work unit of the decode kernel: 8, 4, 2 or 1
  int32_t NU;      // work units the decode launch provides (waves / HGW)
  int32_t NUP;     // work units (workgroups) of the prefill launch (16-bit cache), else 0
  int32_t PLAN;    // 1: workgroup 0 of the decode launch writes the prefill plan
  int32_t CASC;    // 1: the share kernel ran before the decode launch (cascade over a shared prefix)
  int32_t SG;      // cascade: decode-class sequences per prefix group (XR / RS)
  int32_t XR;      // cascade: query rows per prefix group tile (16 NX: 16, 32 or 64)
  int32_t R1;      // decode: units whose workgroups all sit in the first dispatch round (one per CU)
  int32_t PR;      // query rows ((token, head) pairs of one kv head) per prefill tile
  float v_scale;   // factor of every output row: the V scale of an E4M3 cache, else 1
  float* ws_acc;   // [slots, HGW, RS, D] unnormalised partial outputs of split decode segments
  float* ws_ml;    // [slots, HGW, RS, 2] running max (exp2 domain) and sum of each partial
  float* ws_pacc;  // [2 NUP, PR, D] partial outputs of split prefill tiles (capacity: kPrefillRows)
  float* ws_pml;   // [2 NUP, PR, 2]
  int32_t* ws_job; // [kMaxJobs, kJobInts] merge jobs, rewritten by every unit on every call
  // prefill plan, written by the decode launch's workgroup 0 before any prefill unit starts:
  int64_t* ws_plan_hdr;  // [4]: flat size C, active units NUa, prefill sequences n_pre
  int32_t* ws_pre_list;  // [B] the prefill-class sequences in order
  int64_t* ws_pre_beg;   // [B + 1] flat start of each (ws_pre_beg[n_pre] = C)
  int32_t* ws_pre_unit;  // [kMaxPrefillUnits, kPreRec] one record per prefill workgroup
  // cascade, written by pa_share_kernel before the decode launch:
  int64_t* ws_share;     // [kShareHdr]: shared prefix tokens (multiple of 32, 0: none), groups, r0, sequences
  int32_t* ws_dec_list;  // [B] decode-class sequences in order
  float* ws_xacc;        // [xslots, HGW, XR, D] partials of the prefix segments
  float* ws_xml;         // [xslots, HGW, XR, 2]
  int32_t* ws_xjob;      // [B * Hkv / HGW, kJobInts] merge jobs per (sequence, head group)
};

// Launch plan: a pure function of static shapes (graph-capture safe).
struct Plan {
  int32_t G, QS, NT, RS;    // GQA group, decode-class q_len cap, 16-row tiles, rows per sequence
  int32_t HGW;              // kv heads per decode work unit
  bool launch_prefill;      // max_query_len > QS
  bool cascade;             // the share kernel runs and the decode kernel may take the cascade path
  bool short_decode;        // one workgroup per (sequence, kv head), no workspace, no merge
  int32_t NX;               // cascade: 16-row tiles of a prefix group over 16-bit caches (1 or 4)
  int64_t xrows;            // cascade: prefix partial rows (slots x HGW x tile rows)
  int64_t slots;            // partial slots: B * Hkv / HGW + kMaxDecodeWaves / HGW
  size_t ws_acc_bytes, ws_ml_bytes, ws_job_bytes, ws_pacc_bytes, ws_pml_bytes, ws_plan_bytes, ws_x_bytes, ws_bytes;
};

// Cascade: decode-class sequences per prefix group of nx 16-row tiles, RS rows each.
inline int32_t cascade_group(int32_t RS, int32_t nx) { return RS >= 16 * nx ? 1 : 16 * nx / RS; }
// 16-row tiles of a cascade prefix group: the plan's NX (4 or 1) over 16-bit caches, at most 2
// over E4M3 caches.
inline int32_t cascade_tiles(int32_t NX, bool kv8) { return kv8 && NX > 2 ? 2 : NX; }

Plan make_plan(int64_t T, int32_t B, int32_t H, int32_t Hkv, int32_t D, int32_t W, int32_t BS, int32_t max_q,
               int32_t dtype);

// Kernel launchers (return hipError_t as int). `kinds` collects launched kernel kinds.
struct LaunchLog {
  void* const* events = nullptr;
  int32_t num_events = 0;
  int32_t launched = 0;
  int32_t kinds[8] = {0};
  void after_launch(int kind, hipStream_t s);
};

int launch_paged_attention_mfma(PAParams& p, const Plan& plan, int32_t D, int32_t dtype, bool kv8, int32_t max_q,
                                hipStream_t s, LaunchLog& log);
// Whether a 16-bit launch takes the MFMA kernels: head sizes 64 and 128, pages a whole number
// of 16-token tiles, GQA groups of at most 64 rows per token (four 16-row tiles). Every other
// 16-bit shape, and fp32, takes the vector-ALU kernel (no workspace).
inline bool mfma_shape(int32_t D, int32_t BS, int32_t G) {
  return (D == 64 || D == 128) && BS % 16 == 0 && G <= 64;
}
int launch_paged_attention_valu(const PAParams& p, int32_t D, int32_t dtype, int32_t max_q, hipStream_t s,
                                LaunchLog& log);
int launch_reshape_and_cache(const void* k, int64_t k_ts, int64_t k_hs, const void* v, int64_t v_ts,
                             int64_t v_hs, void* kc, const int64_t* kcs, void* vc, const int64_t* vcs,
                             const int64_t* slots, int64_t T, int64_t num_blocks, int32_t Hkv, int32_t D,
                             int32_t BS, int32_t elem_bytes, bool vec16, hipStream_t s);

// Metadata expansion (kvh_prepare_metadata): pointers into the packed upload and the outputs.
struct MetaParams {
  const int32_t* seqs;    // [B][4] row, start, q_len, n_blocks
  const int32_t* tokens;  // [T] input ids, or null
  int64_t* pool;          // [pool_rows, pool_rs] resident block tables
  int32_t pool_rows, pool_width;
  int64_t pool_rs;
  int64_t* bt;  // [B + P, bt_rs] batch block tables (first bt_width columns written), or null
  int64_t bt_rs;
  int32_t bt_width;
  int64_t bt_pad;
  int64_t* slots;      // [T + P]
  int64_t* positions;  // [T + P] or null
  int64_t* input_ids;  // [T + P] or null
  int64_t* seq_lens;   // [B + P]
  int64_t* query_lens; // [B + P] or null
  int64_t* qsl;        // [B + P + 1]
  int64_t pad_slot;
  int64_t T;  // real tokens
  int32_t B, P, BS;
};

int launch_prepare_metadata(const MetaParams& m, const int32_t* updates, int32_t num_updates, hipStream_t s);

// Measurement probes (probes.hip): 0 stream read, 1 copy, 2 MFMA rate.
int launch_probe(int kind, const void* src, void* dst, int64_t bytes, int32_t blocks, int32_t iters, hipStream_t s);

// Engine-harness kernels (engine_ops.hip).
int launch_add_rmsnorm(const void* x, int64_t x_ts, const void* d, int64_t d_ts, const void* w, void* xo,
                       int64_t xo_ts, void* h, int64_t h_ts, int64_t T, int32_t hd, float eps, int32_t dtype,
                       hipStream_t s);
int launch_silu_mul(const void* gu, int64_t gu_ts, void* out, int64_t o_ts, int64_t T, int32_t inter, int32_t dtype,
                    hipStream_t s);
int launch_gemv(const void* x, int64_t x_rs, const void* w, int64_t w_rs, void* y, int64_t y_rs, int32_t m, int32_t n,
                int32_t k, int32_t dtype, hipStream_t s);
int launch_gemm_skinny(const void* x, int64_t x_rs, const void* w, int64_t w_rs, void* y, int64_t y_rs, int32_t m,
                       int32_t n, int32_t k, bool glu, int32_t dtype, hipStream_t s);
int launch_gemv_silu_mul(const void* x, int64_t x_rs, const void* w, int64_t w_rs, void* y, int64_t y_rs, int32_t m,
                         int32_t inter, int32_t k, int32_t dtype, hipStream_t s);

int launch_rope_and_cache(const void* qkv, int64_t qkv_ts, const int64_t* positions, const float* cos_t,
                          const float* sin_t, int64_t max_pos, void* q_out, int64_t q_ts, int64_t q_hs, void* kc,
                          const int64_t* kcs, void* vc, const int64_t* vcs, const int64_t* slots, int64_t T,
                          int64_t num_blocks, int32_t H, int32_t Hkv, int32_t D, int32_t BS, int32_t dtype,
                          bool kv8, float k_scale, float v_scale, hipStream_t s);
int launch_gemv_rope_and_cache(const void* x, int64_t x_rs, const void* w, int64_t w_rs, int32_t m, int32_t k,
                               const int64_t* positions, const float* cos_t, const float* sin_t, int64_t max_pos,
                               void* q_out, int64_t q_ts, int64_t q_hs, void* kc, const int64_t* kcs, void* vc,
                               const int64_t* vcs, const int64_t* slots, int64_t num_blocks, int32_t H, int32_t Hkv,
                               int32_t D, int32_t BS, int32_t dtype, bool kv8, float k_scale, float v_scale,
                               hipStream_t s);
int launch_reshape_and_cache_fp8(const void* k, int64_t k_ts, int64_t k_hs, const void* v, int64_t v_ts,
                                 int64_t v_hs, void* kc, const int64_t* kcs, void* vc, const int64_t* vcs,
                                 const int64_t* slots, int64_t T, int64_t num_blocks, int32_t Hkv, int32_t D,
                                 int32_t BS, int32_t dtype, float k_scale, float v_scale, hipStream_t s);

}  // namespace kvh
