// Paged attention for gfx950 (CDNA4): bf16/fp16 storage, fp32 accumulation on MFMA.
//
// Semantics follow the reference kernel (src/kvserve/kernels/paged_attention.py:24-115):
// query i of a sequence sits at absolute position ctx + i (ctx = seq_len - q_len) and sees
// keys 0 .. ctx + i; head h reads kv head h / G; scores are scaled by scale * log2(e) and
// exponentiated with exp2; a row whose running max is still -inf uses 0 as its shift
// (the reference's m_safe, :100-105); the output is acc / (l == 0 ? 1 : l) (:113);
// P is rounded to the storage type before the P.V contraction (:106-110).
//
// Work decomposition (MI355X-first, not the reference's (seq, kv_head, q_tile) grid):
//  * One wave owns all query rows of a (sequence, kv_head) GQA group that it works on:
//    row r -> (query token r / G, head kv_head * G + r % G), in tiles of 16 rows.
//  * A wave walks the KV context in 32-token chunks (two 16-token MFMA tiles) and computes
//    S^T = K Q^T, so the accumulator layout of S^T (lane holds column = query row, four
//    consecutive keys) is already the B-operand layout of O^T = V^T P^T. Softmax state
//    (max m, sum l) therefore lives in the same lanes as the output column it scales:
//    no cross-lane traffic between the two contractions except one row-max per chunk.
//  * The block ids a wave needs are fetched 64 pages at a time with one vector load (lane
//    l holds page page0 + l) and read per page with readlane, so no global load sits on
//    the K/V address path. K of the next chunk is issued as soon as the scores are done
//    and V of the next chunk as soon as P.V is done: loads overlap compute without a
//    second register buffer.
//  * Decode class (q_len <= QS): stream-K. The launch takes a fixed share of the waves the GPU
//    holds resident (all of them resident at once, never more than the static shape can
//    give work); the decode work of all sequences is one flat space of 32-token chunks
//    that is cut into equal contiguous ranges, one per work unit of up to 8 waves (adjacent
//    kv heads of the same rows: a token's 8 heads are one contiguous 2 KB row at D = 128).
//    Each wave pays one start-up; a sequence split between units leaves partials that the
//    merge kernel combines with a log-sum-exp. The split is computed on the device from
//    seq_lens (no host sync).
//  * Prefill class (q_len > QS): stream-K as well, over (sequence, kv head, 128-row tile,
//    chunk); a workgroup of 4 waves shares each K/V chunk through an LDS ring filled by
//    direct global->LDS loads, each wave computing 32 query rows.
// Grids depend only on static shapes and the device's occupancy, never on per-step
// lengths, so every launch is HIP-graph capturable.
#include <type_traits>

#include "kvh_device.h"
#include "kvh_internal.h"

namespace kvh {

constexpr int kChunk = 32;  // tokens per wave iteration
constexpr int kWavesPerWG = 4;
// 16-row tiles per prefill wave: 3 over 16-bit caches (48 rows, 238 VGPRs at D = 128, 2 workgroups per
// CU), 2 over E4M3 caches (whose conversion registers leave no room for a third)
template <bool KV8>
constexpr int prefill_nt() {
  return KV8 ? 2 : 3;
}

// ---------------------------------------------------------------------------------------
// Block ids of 64 consecutive pages, one per lane; -1 marks a page that must not be read
// (past the sequence, or an id outside the pool).
struct PageWindow {
  int ids;
  int page0;
};

__device__ __forceinline__ void load_window(PageWindow& pw, const PAParams& p, const int64_t* btrow, int page0,
                                            int page_end) {
  const int lane = threadIdx.x & 63;
  const int pg = page0 + lane;
  int id = -1;
  if (pg < page_end) {
    const int64_t b = btrow[pg];
    if (b >= 0 && b < p.num_blocks) id = (int)b;
  }
  pw.ids = id;
  pw.page0 = page0;
}

// Block id of `page` (wave-uniform), refreshing the window when the page leaves it. A
// refresh keeps kWindowHistory pages below `page` so pages a few chunks behind (still being
// computed while later chunks are loaded) stay readable with peek_block.
constexpr int kWindowHistory = 8;

__device__ __forceinline__ int page_block(PageWindow& pw, const PAParams& p, const int64_t* btrow, int page,
                                          int page_end) {
  if (page >= page_end) return -1;
  if (page - pw.page0 >= 64 || page < pw.page0)
    load_window(pw, p, btrow, page >= kWindowHistory ? page - kWindowHistory : 0, page_end);
  return __builtin_amdgcn_readlane(pw.ids, page - pw.page0);
}

// Block id of `page` if the window holds it, else -1 (no refresh, no memory access).
__device__ __forceinline__ int peek_block(const PageWindow& pw, int page) {
  const int rel = page - pw.page0;
  return (rel >= 0 && rel < 64) ? __builtin_amdgcn_readlane(pw.ids, rel) : -1;
}

// Per-lane registers of one 32-token chunk of one kv head.
template <int D>
struct KRegs {
  u32x4 k[2][D / 32];  // tile t, 8-element vector c: token 16t + n, d = 32c + 8j ..
                       // (one load instruction per c reads 64 contiguous bytes of each row)
};
template <int D>
struct VRegs {
  static constexpr int VW = D / 16;  // V elements per lane per token: d = VW n .. VW n + VW - 1
  uint32_t v[8][VW / 2];             // token t8 = 4 tile + e  <->  chunk token 16 tile + 4j + e
};

// The same chunk from an E4M3 cache (KV8), as loaded; converted to 16-bit MFMA operands at
// use. K: 16 bytes per lane per pair of operands: lane (j, n) holds token 16t + n, bytes
// d = 64c + 16j .. +15, and operand 2c + h takes d = 64c + 16j + 8h .. +7 (the query operand
// uses the same k-slot order). V: lane (j, m) holds d = VW m .. VW m + VW - 1 of 8 tokens.
template <int D>
struct KRegs8 {
  u32x4 k[2][D / 64];
};
template <int D>
struct VRegs8 {
  static constexpr int VW = D / 16;
  uint32_t v[8][VW / 4];  // token t8 as in VRegs, 4 E4M3 values per dword
};

// Uniform description of a chunk: first token and the block of each 16-token tile.
struct ChunkRef {
  int tok0;
  int blk[2];  // -1: tile absent
};

__device__ __forceinline__ ChunkRef chunk_ref(PageWindow& pw, const PAParams& p, const int64_t* btrow, int tok0,
                                              int tok_hi, int page_end) {
  ChunkRef c;
  c.tok0 = tok0;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int tt = tok0 + 16 * t;
    c.blk[t] = tt < tok_hi ? page_block(pw, p, btrow, tt / p.BS, page_end) : -1;
  }
  return c;
}

// Lane byte offsets inside a (block, kv head) page, fixed for the whole kernel.
struct LaneOffsets {
  uint32_t k;  // (n * k_ss + 8 j) * 2
  uint32_t v;  // (4j * v_ss + VW n) * 2
};

template <int D, bool KV8 = false>
__device__ __forceinline__ LaneOffsets lane_offsets(const PAParams& p) {
  const int lane = threadIdx.x & 63;
  const int j = lane >> 4, n = lane & 15;
  LaneOffsets o;
  if (KV8) {  // one byte per element
    o.k = (uint32_t)(n * (uint32_t)p.k_ss + 16 * j);
    o.v = (uint32_t)(4 * j * (uint32_t)p.v_ss + (D / 16) * n);
  } else {
    o.k = (uint32_t)(n * (uint32_t)p.k_ss + 8 * j) * 2u;
    o.v = (uint32_t)(4 * j * (uint32_t)p.v_ss + (D / 16) * n) * 2u;
  }
  return o;
}

// K/V of the decode kernels are read once per launch: non-temporal loads (NTL; the `nt` cache
// policy), which the caches do not keep. Against ordinary loads, HBM-cold: C2 decode
// 222.7 -> 200.0 us, C5 88.5 -> 80.4 us, C3's decode part 782 -> 722 us, C2 over E4M3
// 128.7 -> 122.8 us. The short decode kernel keeps ordinary loads: on C1's 5 MB batch the
// non-temporal ones took 11.9 us against 10.8.
template <class T, bool NTL>
__device__ __forceinline__ T stream_load(const void* p) {
  if constexpr (NTL)
    return __builtin_nontemporal_load((const T*)p);
  else
    return *(const T*)p;
}

// Loads are unconditional so the chunk loop stays straight-line (no waits merged at
// branch joins): an absent tile (blk < 0) reads block 0, which the API guarantees exists,
// and is masked out of the scores and zeroed out of V like any invalid key.
template <int D, bool NTL>
__device__ __forceinline__ void load_k(KRegs<D>& r, const PAParams& p, const ChunkRef& c, int kvh, uint32_t k_lane) {
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int64_t blk = c.blk[t] >= 0 ? c.blk[t] : 0;
    const int slot0 = (c.tok0 + 16 * t) % p.BS;
    const char* page = (const char*)p.kc + (blk * p.k_sb + (int64_t)kvh * p.k_sh + (int64_t)slot0 * p.k_ss) * 2;
#pragma unroll
    for (int cc = 0; cc < D / 32; ++cc) r.k[t][cc] = stream_load<u32x4, NTL>(page + k_lane + 64 * cc);
  }
}

template <int D, bool NTL>
__device__ __forceinline__ void load_v(VRegs<D>& r, const PAParams& p, const ChunkRef& c, int kvh, uint32_t v_lane) {
  constexpr int VD = D / 32;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int64_t blk = c.blk[t] >= 0 ? c.blk[t] : 0;
    const int slot0 = (c.tok0 + 16 * t) % p.BS;
    const char* page = (const char*)p.vc + (blk * p.v_sb + (int64_t)kvh * p.v_sh + (int64_t)slot0 * p.v_ss) * 2;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const char* src = page + (int64_t)e * p.v_ss * 2 + v_lane;
      if constexpr (VD == 4) {
        const u32x4 x = stream_load<u32x4, NTL>(src);
        r.v[4 * t + e][0] = x[0];
        r.v[4 * t + e][1] = x[1];
        r.v[4 * t + e][2] = x[2];
        r.v[4 * t + e][3] = x[3];
      } else {
        const u32x2 x = stream_load<u32x2, NTL>(src);
        r.v[4 * t + e][0] = x[0];
        r.v[4 * t + e][1] = x[1];
      }
    }
  }
}

template <int D, bool NTL>
__device__ __forceinline__ void load_k(KRegs8<D>& r, const PAParams& p, const ChunkRef& c, int kvh, uint32_t k_lane) {
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int64_t blk = c.blk[t] >= 0 ? c.blk[t] : 0;
    const int slot0 = (c.tok0 + 16 * t) % p.BS;
    const char* page = (const char*)p.kc + blk * p.k_sb + (int64_t)kvh * p.k_sh + (int64_t)slot0 * p.k_ss;
#pragma unroll
    for (int cc = 0; cc < D / 64; ++cc) r.k[t][cc] = stream_load<u32x4, NTL>(page + k_lane + 64 * cc);
  }
}

template <int D, bool NTL>
__device__ __forceinline__ void load_v(VRegs8<D>& r, const PAParams& p, const ChunkRef& c, int kvh, uint32_t v_lane) {
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int64_t blk = c.blk[t] >= 0 ? c.blk[t] : 0;
    const int slot0 = (c.tok0 + 16 * t) % p.BS;
    const char* page = (const char*)p.vc + blk * p.v_sb + (int64_t)kvh * p.v_sh + (int64_t)slot0 * p.v_ss;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const char* src = page + (int64_t)e * p.v_ss + v_lane;
      if constexpr (D == 128) {
        const u32x2 x = stream_load<u32x2, NTL>(src);
        r.v[4 * t + e][0] = x[0];
        r.v[4 * t + e][1] = x[1];
      } else {
        r.v[4 * t + e][0] = stream_load<uint32_t, NTL>(src);
      }
    }
  }
}

// K operand cc of tile `tile` of an E4M3 chunk, converted (exactly) to E's type.
template <class E, int D>
__device__ __forceinline__ u32x4 k_operand(const KRegs8<D>& r, int tile, int cc) {
  const u32x4 w = r.k[tile][cc >> 1];
  const uint32_t a = w[2 * (cc & 1)], b = w[2 * (cc & 1) + 1];
  return u32x4{E::template from_fp8x2<false>(a), E::template from_fp8x2<true>(a), E::template from_fp8x2<false>(b),
               E::template from_fp8x2<true>(b)};
}

// Online-softmax state of one wave over NT tiles of 16 query rows.
template <int D, int NT>
struct WaveState {
  u32x4 q[NT][D / 32];    // B operand of S^T = K Q^T
  f32x4 acc[NT][D / 16];  // O^T accumulators: column = row, rows 4j+e <-> d = VW*(4j+e) + i
  float m[NT], l[NT];     // m: running max (exp2 domain, -inf when empty); l: lane-partial sum
  int limit[NT];          // keys visible to this lane's row (0 for padding rows)
  float thr[NT], nsh[NT]; // prefill only: raw-score bound that moves m, and -m (0 while m = -inf)
};

// Q rows of tile t: global row r = row0 + 16t + n, valid when r < R.
template <int D, int NT, bool KV8 = false>
__device__ __forceinline__ void load_q(WaveState<D, NT>& s, const PAParams& p, int64_t q_start, int R, int row0,
                                       int kvh, int64_t ctx, int64_t kv_total) {
  const int lane = threadIdx.x & 63;
  const int j = lane >> 4, n = lane & 15;
  const uint16_t* q = (const uint16_t*)p.q;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int r = row0 + 16 * t + n;
    s.m[t] = -INFINITY;
    s.l[t] = 0.f;
    s.thr[t] = -INFINITY;
    s.nsh[t] = 0.f;
#pragma unroll
    for (int i = 0; i < D / 16; ++i) s.acc[t][i] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (r < R) {
      const int qi = r / p.G, g = r % p.G;
      const uint16_t* qp = q + (q_start + qi) * p.q_ts + (int64_t)(kvh * p.G + g) * p.q_hs;
#pragma unroll
      for (int c = 0; c < D / 32; ++c) {
        // operand c holds d = 32c + 8j .. +7, or with an E4M3 cache 64(c / 2) + 16j + 8(c % 2) .. +7
        const int d0 = KV8 ? 64 * (c >> 1) + 16 * j + 8 * (c & 1) : 32 * c + 8 * j;
        s.q[t][c] = *(const u32x4*)(qp + d0);
      }
      s.limit[t] = (int)clamp64(ctx + qi + 1, 0, kv_total);
    } else {
#pragma unroll
      for (int c = 0; c < D / 32; ++c) s.q[t][c] = u32x4{0, 0, 0, 0};
      s.limit[t] = 0;
    }
  }
}

// Scores of one chunk and the online-softmax update; returns the P^T B operands.
// MASKED = false only when every token of the chunk is visible to every valid row.
// LAZY: skip the accumulator rescale when no row max moved (a uniform branch; exact, and a
// win for decode where the max settles early); otherwise the body is straight-line so the
// row tiles' dependency chains interleave.
template <class E, int D, int NT, bool MASKED, bool LAZY = true, class KR>
__device__ __forceinline__ void chunk_scores(WaveState<D, NT>& s, const KR& kr, const PAParams& p,
                                             const ChunkRef& c, u32x4 pt[NT]) {
  const int j = (threadIdx.x & 63) >> 4;
  f32x4 st[NT][2];
  if constexpr (std::is_same_v<KR, KRegs<D>>) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int tile = 0; tile < 2; ++tile) {
        f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int cc = 0; cc < D / 32; ++cc) a = E::mfma(kr.k[tile][cc], s.q[t][cc], a);
        st[t][tile] = a;
      }
  } else {  // E4M3: convert each tile's operands once for all row tiles
#pragma unroll
    for (int tile = 0; tile < 2; ++tile) {
      u32x4 k[D / 32];
#pragma unroll
      for (int cc = 0; cc < D / 32; ++cc) k[cc] = k_operand<E, D>(kr, tile, cc);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int cc = 0; cc < D / 32; ++cc) a = E::mfma(k[cc], s.q[t][cc], a);
        st[t][tile] = a;
      }
    }
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    float mx = -INFINITY;
#pragma unroll
    for (int tile = 0; tile < 2; ++tile) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float x = st[t][tile][e] * p.qk_scale;
        if (MASKED) {
          const int tok = c.tok0 + 16 * tile + 4 * j + e;
          if (!(c.blk[tile] >= 0 && tok < s.limit[t])) x = -INFINITY;
        }
        st[t][tile][e] = x;
        mx = fmaxf(mx, x);
      }
    }
    mx = max_over_groups(mx);
    const float m_old = s.m[t];
    const float m_new = fmaxf(m_old, mx);
    const float m_safe = m_new == -INFINITY ? 0.f : m_new;
    if (!LAZY || __builtin_amdgcn_ballot_w64(m_new > m_old)) {
      const float alpha = fast_exp2(m_old - m_safe);
      s.l[t] *= alpha;
#pragma unroll
      for (int i = 0; i < D / 16; ++i) s.acc[t][i] *= alpha;
    }
    s.m[t] = m_new;
    float pv[8], psum = 0.f;
#pragma unroll
    for (int tile = 0; tile < 2; ++tile)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x = fast_exp2(st[t][tile][e] - m_safe);
        pv[4 * tile + e] = x;
        psum += x;
      }
    s.l[t] += psum;
#pragma unroll
    for (int w = 0; w < 4; ++w) pt[t][w] = E::pack2(pv[2 * w], pv[2 * w + 1]);
  }
}

// Prefill variant of chunk_scores, built for VALU economy (prefill is MFMA/VALU bound):
//  * the max is taken over raw scores and the scale c = |scale| log2(e) > 0 is folded into
//    the exp2 argument (one FMA per score); a sign flip of Q makes c > 0 exact;
//  * the running shift m only moves when some row's max exceeds it by more than
//    kRescaleSlack (exp2 domain), so P <= 2^kRescaleSlack and the accumulators are
//    rescaled rarely (a uniform branch). Numerator and denominator share the shift, so the
//    result is the softmax whatever shift is used;
//  * MASKED = false for chunks whose keys every valid row of the wave sees.
constexpr float kRescaleSlack = 8.f;

template <class E, int D, int NT>
__device__ __forceinline__ void pf_scores(const WaveState<D, NT>& s, const KRegs<D>& kr, f32x4 st[NT][2]) {
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int tile = 0; tile < 2; ++tile) {
      f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int cc = 0; cc < D / 32; ++cc) a = E::mfma(kr.k[tile][cc], s.q[t][cc], a);
      st[t][tile] = a;
    }
}

// Causal / absent-page mask of one chunk's scores (-inf where the key is not visible).
template <int NT>
__device__ __forceinline__ void pf_mask(f32x4 st[NT][2], const int limit[NT], const ChunkRef& ch) {
  const int j = (threadIdx.x & 63) >> 4;
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int tile = 0; tile < 2; ++tile) {
      // keys tok < lim are kept: the row's causal limit, or none for an absent page
      const int lim = ch.blk[tile] >= 0 ? limit[t] - (ch.tok0 + 16 * tile + 4 * j) : INT32_MIN;
#pragma unroll
      for (int e = 0; e < 4; ++e) st[t][tile][e] = e < lim ? st[t][tile][e] : -INFINITY;
    }
}

// Per-lane maxima of one chunk's (masked) raw scores: the lane's 8 keys of each of its rows.
// The cross-lane reduction is left to the rare branch that moves a row's shift: a row's
// maximum passes its threshold exactly when one of its four lanes' maxima does.
template <int NT>
__device__ __forceinline__ void pf_lanemax(const f32x4 st[NT][2], float mx[NT]) {
#pragma unroll
  for (int t = 0; t < NT; ++t)
    mx[t] = fmaxf(fmaxf(fmaxf(st[t][0][0], st[t][0][1]), fmaxf(st[t][0][2], st[t][0][3])),
                  fmaxf(fmaxf(st[t][1][0], st[t][1][1]), fmaxf(st[t][1][2], st[t][1][3])));
}

// Online-softmax update from (masked) raw scores and per-lane maxima; c > 0 so a -inf
// score gives P = 0. The row test is one compare against thr = (m + kRescaleSlack) / c,
// kept with nsh = -m and only recomputed when a row's shift moves (a uniform branch, where
// the lane maxima are reduced over the row's four lanes). The row sums are taken from the
// packed (rounded) P with v_dot2 against ones: the same P values the P.V contraction uses.
template <class E, int D, int NT>
__device__ __forceinline__ void pf_softmax(WaveState<D, NT>& s, const f32x4 st[NT][2], const float mxs[NT], float c,
                                           u32x4 pt[NT]) {
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    if (__builtin_amdgcn_ballot_w64(mxs[t] > s.thr[t])) {
      const float mrow = max_over_groups(mxs[t]);
      const float m_new = fmaxf(s.m[t], mrow * c);  // -inf stays -inf (c > 0)
      // the ballot is wave-wide: a row with no visible key so far keeps m = -inf
      const bool empty = m_new == -INFINITY;
      const float alpha = empty ? 1.f : fast_exp2(s.m[t] - m_new);
      s.l[t] *= alpha;
#pragma unroll
      for (int i = 0; i < D / 16; ++i) s.acc[t][i] *= alpha;
      s.m[t] = m_new;
      s.thr[t] = empty ? -INFINITY : (m_new + kRescaleSlack) / c;
      s.nsh[t] = empty ? 0.f : -m_new;
    }
    float pv[8];
#pragma unroll
    for (int tile = 0; tile < 2; ++tile)
#pragma unroll
      for (int e = 0; e < 4; ++e) pv[4 * tile + e] = fast_exp2(__builtin_fmaf(st[t][tile][e], c, s.nsh[t]));
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      pt[t][w] = E::pack2(pv[2 * w], pv[2 * w + 1]);
      s.l[t] = E::dot2_ones(pt[t][w], s.l[t]);
    }
  }
}

// O^T += V^T P^T for one chunk. In the masked case, slots at or past seq_len may hold any
// bits (stale or never written cache slots): P is 0 there but 0 * NaN is NaN, so V is
// zeroed like the reference's masked loads (other=0.0).
template <class E, int D, int NT, bool MASKED>
__device__ __forceinline__ void chunk_pv(WaveState<D, NT>& s, VRegs<D>& vr, const ChunkRef& c, int data_end,
                                         const u32x4 pt[NT]) {
  constexpr int VW = D / 16;
  const int j = (threadIdx.x & 63) >> 4;
  if (MASKED) {
#pragma unroll
    for (int t8 = 0; t8 < 8; ++t8) {
      const int tok = c.tok0 + 16 * (t8 >> 2) + 4 * j + (t8 & 3);
      const bool keep = c.blk[t8 >> 2] >= 0 && tok < data_end;
#pragma unroll
      for (int x = 0; x < VW / 2; ++x) vr.v[t8][x] = keep ? vr.v[t8][x] : 0u;  // select, no branch
    }
  }
  // V^T A operand i: element 4*tile + e of lane (j, m) = V[token 16*tile + 4j + e][VW*m + i]
#pragma unroll
  for (int i = 0; i < VW; ++i) {
    u32x4 va;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t a = vr.v[2 * w][i >> 1], b = vr.v[2 * w + 1][i >> 1];
      va[w] = (i & 1) ? pick_halves<1>(a, b) : pick_halves<0>(a, b);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) s.acc[t][i] = E::mfma(va, pt[t], s.acc[t][i]);
  }
}

// O^T += V^T P^T from an E4M3 V chunk. The A operand of output column group i wants, in dword
// w, element i of tokens t8 = 2w and 2w + 1; one byte permute gathers that pair for two
// neighbouring i (bytes b0, b1 of the dwords), and the two halves of the result convert to
// the two operands' dwords. Masked tokens are zeroed in the raw bytes (E4M3 0x00 is +0).
template <class E, int D, int NT, bool MASKED>
__device__ __forceinline__ void chunk_pv(WaveState<D, NT>& s, VRegs8<D>& vr, const ChunkRef& c, int data_end,
                                         const u32x4 pt[NT]) {
  constexpr int VW = D / 16;
  const int j = (threadIdx.x & 63) >> 4;
  if (MASKED) {
#pragma unroll
    for (int t8 = 0; t8 < 8; ++t8) {
      const int tok = c.tok0 + 16 * (t8 >> 2) + 4 * j + (t8 & 3);
      const bool keep = c.blk[t8 >> 2] >= 0 && tok < data_end;
#pragma unroll
      for (int x = 0; x < VW / 4; ++x) vr.v[t8][x] = keep ? vr.v[t8][x] : 0u;
    }
  }
#pragma unroll
  for (int x = 0; x < VW / 4; ++x)
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
      // bytes 2hb and 2hb + 1 of dword x: elements i0 = 4x + 2hb and i0 + 1
      const uint32_t sel = hb ? 0x07030602u : 0x05010400u;
      u32x4 va0, va1;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t pr = __builtin_amdgcn_perm(vr.v[2 * w + 1][x], vr.v[2 * w][x], sel);
        va0[w] = E::template from_fp8x2<false>(pr);
        va1[w] = E::template from_fp8x2<true>(pr);
      }
      const int i0 = 4 * x + 2 * hb;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        s.acc[t][i0] = E::mfma(va0, pt[t], s.acc[t][i0]);
        s.acc[t][i0 + 1] = E::mfma(va1, pt[t], s.acc[t][i0 + 1]);
      }
    }
}

// Chunk loop of one wave over tokens tok_begin, tok_begin + stride, ... < tok_hi.
// The body is straight-line (masks always applied, loads unconditional) and the loads are
// pinned in the order K(c+1), V(c+1) with scheduling barriers, so each s_waitcnt waits for
// exactly the operand it guards while the other half of the next chunk stays in flight.
template <class E, int D, int NT, bool KV8 = false, bool NTL = true>
__device__ __forceinline__ void run_chunks(WaveState<D, NT>& s, const PAParams& p, const int64_t* btrow, int kvh,
                                           int tok_begin, int stride, int tok_hi, int data_end) {
  if (tok_begin >= tok_hi) return;
  const int page_end = (tok_hi + p.BS - 1) / p.BS;
  const LaneOffsets lo = lane_offsets<D, KV8>(p);
  PageWindow pw;
  load_window(pw, p, btrow, tok_begin / p.BS, page_end);
  ChunkRef c = chunk_ref(pw, p, btrow, tok_begin, tok_hi, page_end);
  std::conditional_t<KV8, KRegs8<D>, KRegs<D>> kr;
  std::conditional_t<KV8, VRegs8<D>, VRegs<D>> vr;
  load_k<D, NTL>(kr, p, c, kvh, lo.k);
  __builtin_amdgcn_sched_barrier(0);
  load_v<D, NTL>(vr, p, c, kvh, lo.v);
  __builtin_amdgcn_sched_barrier(0);
  // Every iteration has a next chunk, so its loads are unconditional; the last chunk is
  // peeled off below the loop.
  while (c.tok0 + stride < tok_hi) {
    const ChunkRef cn = chunk_ref(pw, p, btrow, c.tok0 + stride, tok_hi, page_end);
    u32x4 pt[NT];
    chunk_scores<E, D, NT, true>(s, kr, p, c, pt);
    __builtin_amdgcn_sched_barrier(0);
    load_k<D, NTL>(kr, p, cn, kvh, lo.k);
    __builtin_amdgcn_sched_barrier(0);
    chunk_pv<E, D, NT, true>(s, vr, c, data_end, pt);
    __builtin_amdgcn_sched_barrier(0);
    load_v<D, NTL>(vr, p, cn, kvh, lo.v);
    __builtin_amdgcn_sched_barrier(0);
    c = cn;
  }
  u32x4 pt[NT];
  chunk_scores<E, D, NT, true>(s, kr, p, c, pt);
  chunk_pv<E, D, NT, true>(s, vr, c, data_end, pt);
}

template <class E, int VW>
__device__ __forceinline__ void store_row_vec(uint16_t* dst, const float* o, float inv) {
  if constexpr (VW == 8) {
    u32x4 x;
#pragma unroll
    for (int w = 0; w < 4; ++w) x[w] = E::pack2(o[2 * w] * inv, o[2 * w + 1] * inv);
    *(u32x4*)dst = x;
  } else {
    u32x2 x;
#pragma unroll
    for (int w = 0; w < 2; ++w) x[w] = E::pack2(o[2 * w] * inv, o[2 * w + 1] * inv);
    *(u32x2*)dst = x;
  }
}

struct SeqView {
  int64_t qs;    // first flat token of the sequence
  int q_len;
  int64_t ctx;   // seq_len - q_len (cached tokens before this step)
  int kv_total;  // keys present: seq_len clamped to the block-table capacity
};

// From the raw metadata of a sequence: query_start_loc[s], query_start_loc[s + 1], seq_lens[s].
__device__ __forceinline__ SeqView seq_view_from(const PAParams& p, int64_t qs_raw, int64_t qe_raw, int64_t sl) {
  SeqView v;
  v.qs = clamp64(qs_raw, 0, p.T);
  const int64_t qe = clamp64(qe_raw, v.qs, p.T);
  v.q_len = (int)(qe - v.qs);
  v.ctx = sl - v.q_len;
  v.kv_total = (int)clamp64(sl, 0, (int64_t)p.W * p.BS);
  return v;
}

__device__ __forceinline__ SeqView seq_view(const PAParams& p, int seq) {
  return seq_view_from(p, p.qsl[seq], p.qsl[seq + 1], p.seq_lens[seq]);
}

// seq_view for a wave-uniform sequence index, with wave-uniform (scalar) results.
__device__ __forceinline__ SeqView seq_view_uniform(const PAParams& p, int seq) {
  SeqView v = seq_view(p, seq);
  v.qs = uni64(v.qs);
  v.q_len = uni(v.q_len);
  v.ctx = uni64(v.ctx);
  v.kv_total = uni(v.kv_total);
  return v;
}

// Float offset of float4 c4 of row r in a head's group of `cap` partial rows (one split
// piece's fp32 accumulators, written by write_rows, read by the merge) in the tile-block
// layout (multi-tile rows over E4M3 caches: write_rows<..., BLK> and merge_job<..., BLK>). The
// rows are kept in 16-row tiles in the order the accumulator lanes hold them: lane (j, n) of
// a tile holds row n, d = VW (4j + e) + i, i.e. float4 c4 = VW j + k with k = e VW / 4 + i / 4,
// and that float4 lies at (k * 4 + j) * m + n of the tile's m-row block (m = min(16, cap -
// 16 t)). Each store instruction of a wave (one k) then writes 64 m contiguous bytes; with rows
// laid out whole it writes 16 bytes to each of 4 lines of every row. HBM-cold, three runs
// each: C5 over E4M3 (two row tiles) decode 58.9 -> 51.3 us, merge 11.1 -> 12.1; single-tile
// rows over E4M3 (C2, C4) gained 0.3-0.6 us in the decode kernel and lost 0.6-1.3 us in the
// merge, and over 16-bit caches the decode kernels gained at most 0.8 us and the merges lost
// up to 1.0, so those keep whole rows.
template <int D>
__device__ __forceinline__ int part_ofs(int r, int c4, int cap) {
  constexpr int VW = D / 16;
  const int t = r >> 4, n = r & 15, m = min(16, cap - 16 * t);
  return 16 * t * D + (((c4 % VW) * 4 + c4 / VW) * m + n) * 4;
}

// Writes one wave's result for its 16-row tiles: the normalised output row, or (partial)
// the unnormalised acc (BLK: laid out by part_ofs in the head's cap-row group starting at ws
// row row_base; else whole rows at ws row row_base + r), running max m and sum l of a piece of
// a split segment (at ws row row_base + r). Lane (j, n) holds row row0 + 16t + n,
// d = VW (4j + e) + i.
template <class E, int D, int NT, bool BLK = false>
__device__ __forceinline__ void write_rows(const WaveState<D, NT>& s, const PAParams& p, const SeqView& sv, int R,
                                           int row0, int kvh, bool partial, float* ws_acc, float* ws_ml,
                                           int64_t row_base, int cap) {
  constexpr int VW = D / 16;
  const int lane = threadIdx.x & 63;
  const int j = lane >> 4, n = lane & 15;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const float L = sum_over_groups(s.l[t]);
    const int r = row0 + 16 * t + n;
    if (r >= R) continue;
    if (!partial) {
      const int qi = r / p.G, g = r % p.G;
      const float inv = p.v_scale / (L == 0.f ? 1.f : L);
      uint16_t* base = (uint16_t*)p.out + (sv.qs + qi) * p.o_ts + (int64_t)(kvh * p.G + g) * p.o_hs;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float o[VW];
#pragma unroll
        for (int i = 0; i < VW; ++i) o[i] = s.acc[t][i][e];
        store_row_vec<E, VW>(base + VW * (4 * j + e), o, inv);
      }
    } else {
      const int64_t idx = row_base + r;
      if constexpr (BLK) {
        // part_ofs with the tile t and its row count m uniform: float4 k of this lane at
        // lp + k 16 m floats (row0 = 0 in every partial write)
        const int m = min(16, cap - 16 * t);
        float* lp = ws_acc + (row_base + 16 * t) * D + (j * m + n) * 4;
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int i = 0; i < VW; i += 4)
            *(f32x4*)(lp + (e * (VW / 4) + i / 4) * 16 * m) =
                f32x4{s.acc[t][i][e], s.acc[t][i + 1][e], s.acc[t][i + 2][e], s.acc[t][i + 3][e]};
      } else {
        float* dst = ws_acc + idx * D;
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int i = 0; i < VW; i += 4)
            *(f32x4*)(dst + VW * (4 * j + e) + i) =
                f32x4{s.acc[t][i][e], s.acc[t][i + 1][e], s.acc[t][i + 2][e], s.acc[t][i + 3][e]};
      }
      if (j == 0) {
        ws_ml[idx * 2] = s.m[t];
        ws_ml[idx * 2 + 1] = L;
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// Merge jobs. A split segment is merged by one workgroup of pa_merge_kernel, described by
// the unit that computed its first piece: kind, number of pieces, slots of the pieces
// (piece i lives in slot0 for i = 0, else in slotb + stride * i), and where its rows go.
constexpr int32_t kJobNone = 0, kJobDecode = 1, kJobPrefill = 2;

__device__ __forceinline__ void write_job(int32_t* job, int kind, int pieces, int64_t slot0, int64_t slotb,
                                          int stride, int64_t qs, int R, int rbase, int kvh0) {
  job[1] = pieces;
  job[2] = (int32_t)slot0;
  job[3] = (int32_t)slotb;
  job[4] = stride;
  job[5] = (int32_t)qs;  // flat token index: < 2^31 (validated)
  job[6] = R;
  job[7] = rbase;
  job[8] = kvh0;
  job[0] = kind;
}

// ---------------------------------------------------------------------------------------
// Decode-class work as one flat chunk space (stream-K). A segment is (sequence, head
// group of HGW kv heads), ordered sequence-major; a decode-class sequence (0 < q_len <= QS)
// contributes c_s = max(1, ceil(kv_total / 32)) chunks to each of its NHG = Hkv / HGW
// segments, any other sequence none. C = NHG * sum_s c_s. Work unit u of NU' takes the
// chunks [u C / NU', (u + 1) C / NU'), NU' = min(NU, ceil(C / kMinUnitChunks)); the HGW
// waves of a unit take the HGW heads of each segment, so they stream adjacent slices of the
// same cache rows. A segment split between units leaves one partial per unit in slot
// (segment index + unit); the unit holding a split segment's first piece records a merge job.
constexpr int kMinUnitChunks = 2;

// A cascade member: a decode-class sequence with at least kCascadeMinChunks chunks of context
// (so padding rows and short sequences never limit the shared length).
__device__ __forceinline__ bool cascade_member(const PAParams& p, const SeqView& v) {
  return v.q_len > 0 && v.q_len <= p.QS && clamp64(v.ctx, 0, v.kv_total) >= kCascadeMinChunks * kChunk;
}

// skip: keys [0, skip) of every cascade member are computed by the prefix segments
// (skip <= its context then), so its own segments cover [skip, kv_total).
__device__ __forceinline__ int seq_chunks(const PAParams& p, const SeqView& v, int skip) {
  if (v.q_len == 0 || v.q_len > p.QS) return 0;
  const int sk = skip > 0 && cascade_member(p, v) ? skip : 0;
  return max(1, (v.kv_total - sk + kChunk - 1) / kChunk);
}

// 64 sequences of the chunk prefix sum; lane l describes sequence blk0 + l.
struct SeqWindow {
  int blk0;   // first sequence of the window
  int base;   // chunks (per segment) of all sequences before blk0
  int c;      // this lane's sequence
  int excl;   // sequences blk0 .. blk0 + l - 1
  int total;  // the whole window
  int nbase;  // cascade members before blk0
  int nexcl;  // cascade members blk0 .. blk0 + l - 1
  int ntotal; // cascade members of the whole window
  int mem;    // this lane's sequence is a cascade member
  int qs, ql, ctx, kvt;  // this lane's SeqView (ctx clamped to [-q_len, kv_total])
};

__device__ __forceinline__ void scan_window(SeqWindow& sw, const PAParams& p, int blk0, int base, int nbase,
                                            int skip) {
  const int lane = threadIdx.x & 63;
  const int s = blk0 + lane;
  int c = 0, mem = 0, qs = 0, ql = 0, cx = 0, kt = 0;
  if (s < p.B) {
    const SeqView v = seq_view(p, s);
    c = seq_chunks(p, v, skip);
    mem = cascade_member(p, v) ? 1 : 0;
    // 32-bit copies for the segment walk: qs <= T < 2^31 and kv_total < 2^31 (checked on the
    // host); ctx is only read as clamp(ctx + qi + 1, 0, kv_total) for 0 <= qi < q_len and as
    // clamp(ctx, 0, kv_total), which clamping it to [-q_len, kv_total] leaves unchanged
    qs = (int)v.qs;
    ql = v.q_len;
    kt = v.kv_total;
    cx = (int)clamp64(v.ctx, -(int64_t)v.q_len, v.kv_total);
  }
  int incl = c, ninc = mem;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o), z = __shfl_up(ninc, o);
    if (lane >= o) {
      incl += y;
      ninc += z;
    }
  }
  sw.blk0 = blk0;
  sw.base = base;
  sw.c = c;
  sw.excl = incl - c;
  sw.total = __builtin_amdgcn_readlane(incl, 63);  // uniform (a shuffle result would not be)
  sw.nbase = nbase;
  sw.nexcl = ninc - mem;
  sw.ntotal = __builtin_amdgcn_readlane(ninc, 63);
  sw.mem = mem;
  sw.qs = qs;
  sw.ql = ql;
  sw.ctx = cx;
  sw.kvt = kt;
}

__device__ __forceinline__ int64_t active_units(int64_t C, int NU) {
  const int64_t want = (C + kMinUnitChunks - 1) / kMinUnitChunks;
  return want < 1 ? 1 : (want < NU ? want : NU);
}

// Stream-K split of the decode kernel's flat positions [0, C) over NUa units by cost, and by
// unit capacity: the first P positions (cascade prefix segments) cost wp each, the others wr;
// the first R1 units (those dispatched in the first round, one workgroup per CU) take K1 parts
// of the total cost each, the later ones K2. With cum(u) the parts of units before u and
// Q = cum(NUa), unit u takes the positions whose cost start cost(x) lies in
// [T cum(u) / Q, T cum(u + 1) / Q), T = cost(C); wp = wr = K1 = K2 = 1 is the plain split
// [u C / NUa, (u + 1) C / NUa).
struct CostSplit {
  int64_t P, C, NUa, wp, wr, T, R1, K1, K2, Q;
  __device__ CostSplit(int64_t P_, int64_t C_, int64_t NUa_, int64_t wp_, int64_t wr_, int64_t R1_, int64_t K1_,
                       int64_t K2_)
      : P(P_), C(C_), NUa(NUa_), wp(wp_), wr(wr_), T(wp_ * P_ + wr_ * (C_ - P_)), R1(R1_ < NUa_ ? R1_ : NUa_),
        K1(K1_), K2(K2_), Q(K1 * R1 + K2 * (NUa - R1)) {}
  __device__ int64_t cost(int64_t x) const { return x < P ? wp * x : wp * P + wr * (x - P); }
  // the first position whose cost start is >= c
  __device__ int64_t first(int64_t c) const { return c <= wp * P ? (c + wp - 1) / wp : P + (c - wp * P + wr - 1) / wr; }
  __device__ int64_t cum(int64_t u) const { return u <= R1 ? K1 * u : K1 * R1 + K2 * (u - R1); }
  __device__ int64_t begin(int64_t u) const { return first(T * cum(u) / Q); }
  // the last unit u with cum(u) <= m
  __device__ int64_t unit_at(int64_t m) const { return m < K1 * R1 ? m / K1 : R1 + (m - K1 * R1) / K2; }
  // the unit that takes position x: the last u with T cum(u) / Q <= cost(x)
  __device__ int64_t unit_of(int64_t x) const { return unit_at(((cost(x) + 1) * Q - 1) / T); }
};
// Cost of a 64-row prefix position against any other position, in eighths: the 4x MFMA and
// softmax work per chunk of the prefix tiles makes their units finish last under an even split
// (HBM-cold C4: units of prefix positions ended at 151-162 us, the others at 141-145 us).
// Measured on C4's decode kernel, HBM-cold: weights 8 (even) 178.7 us, 9 170.6, 10 159.4,
// 11 154.4, 12 155.5, 13 156.1, 14 156.4, 16 158.5.
// The 32-row groups over E4M3 caches keep the even split (C4 over E4M3, HBM-cold: weights 7
// 92.7 us, 8 91.3, 9 92.3, 10 93.4, 12 96.0).
constexpr int64_t kPrefix64Cost = 11, kChunkCost = 8;
// Shares of a first- and a second-round unit when a launch over E4M3 caches holds two
// workgroups per CU: the first-dispatched workgroup of a CU ran ahead of the second (C2 over
// E4M3, per-wave timeline: mean ends 82.5 and 101.3 us). HBM-cold, decode kernel, shares 1/1 ->
// 4/3: C4 over E4M3 102.9 -> 98.6 us, C3's decode part 404 -> 401 us, C2 118 -> 117 us (9/7,
// 3/2 and 5/3 no better). The 16-bit kernels at D = 64, also two per CU, ran the reference's
// grid 2-7% slower with 4/3 and keep equal shares.
constexpr int64_t kRound1Share = 4, kRound2Share = 3;

constexpr int kPlanThreads = 256;    // the decode kernel's workgroup
constexpr int kPlanLdsSeqs = 1024;  // flat starts kept in LDS for the unit search (else global)
__device__ void plan_prefill(const PAParams& p);

// ---------------------------------------------------------------------------------------
// Cascade decode over a shared prefix (prefix caching hands several sequences the same
// physical blocks at the start of their tables). pa_share_kernel (one workgroup, before the
// decode launch) lists the cascade members (decode-class sequences with kCascadeMinChunks
// chunks of context or more) and finds the longest common table prefix: the first S blocks
// of every member's table equal those of the first one (valid ids), and all their query rows
// see those keys (S BS <= every member's context). The shared length L = min(S BS, smallest
// member context) rounded down to 32-token chunks (0 when below kCascadeMinChunks chunks or
// fewer than 2 members). The decode kernel then computes keys [0, L) once per group of SG
// members (their query rows stacked into one tile of XR = 16 or 64 rows, so the shared K/V
// are read members / SG times instead of once per member) and each member's own keys [L, kv_total)
// as usual; other sequences take their whole range as usual. The merge kernel combines the
// partials of every (sequence, head group) from one record each.
__device__ __forceinline__ int block_min(int v, int* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  int r = red[0];
#pragma unroll
  for (int i = 1; i < kPlanThreads / 64; ++i) r = min(r, red[i]);
  return r;
}

constexpr int kShareLdsList = 1024;  // members whose ids stay in LDS for the column compare
constexpr int kShareCols = 4;        // columns per thread and pass
constexpr int kShareRows = 16;       // member rows loaded together

__global__ __launch_bounds__(kPlanThreads) void pa_share_kernel(PAParams p) {
  __shared__ int s_wsum[kPlanThreads / 64];
  __shared__ int red[kPlanThreads / 64];
  __shared__ int s_list[kShareLdsList];
  const int tid = threadIdx.x;
  const int per = (p.B + kPlanThreads - 1) / kPlanThreads;
  const int s0 = min(tid * per, p.B), s1 = min(s0 + per, p.B);
  int cnt = 0, minctx = 0x7fffffff;
  for (int sq = s0; sq < s1; ++sq) {
    const SeqView v = seq_view(p, sq);
    if (cascade_member(p, v)) {
      ++cnt;
      minctx = min(minctx, (int)clamp64(v.ctx, 0, v.kv_total));
    }
  }
  // exclusive scan of the counts: within the wave by shuffles, then over the 4 wave sums
  const int lane = tid & 63, wv = tid >> 6;
  int incl = cnt;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o);
    if (lane >= o) incl += y;
  }
  if (lane == 63) s_wsum[wv] = incl;
  __syncthreads();
  int nd = 0, k = incl - cnt;
#pragma unroll
  for (int w = 0; w < kPlanThreads / 64; ++w) {
    const int ws = s_wsum[w];
    nd += ws;
    if (w < wv) k += ws;
  }
  for (int sq = s0; sq < s1; ++sq) {
    if (cascade_member(p, seq_view(p, sq))) {
      p.ws_dec_list[k] = sq;
      if (k < kShareLdsList) s_list[k] = sq;
      ++k;
    }
  }
  minctx = block_min(minctx, red);  // its barriers make the list visible to the workgroup
  int shared_tok = 0, r0 = 0;
  if (nd >= 2 && minctx >= kCascadeMinChunks * kChunk) {
    r0 = s_list[0];
    const int64_t* t0 = p.bt + (int64_t)r0 * p.bt_rs;
    const int jmax = min((minctx + p.BS - 1) / p.BS, p.W);
    int first_bad = jmax;
    // columns j0 + 256 c + tid (c < kShareCols) per pass; every load of a pass is independent,
    // kShareRows members x kShareCols columns in flight per thread
    for (int j0 = 0; j0 < jmax; j0 += kPlanThreads * kShareCols) {
      bool ok[kShareCols];
      int64_t ref[kShareCols];
#pragma unroll
      for (int c = 0; c < kShareCols; ++c) ok[c] = true;
      for (int m = 1; m < nd; m += kShareRows) {
        // the reference entries and kShareRows members' entries of this pass in one round of loads
        int64_t row[kShareRows];
#pragma unroll
        for (int u = 0; u < kShareRows; ++u) {
          const int mm = m + u;
          const int sq = mm >= nd ? r0 : (mm < kShareLdsList ? s_list[mm] : p.ws_dec_list[mm]);
          row[u] = (int64_t)sq * p.bt_rs;
        }
        int64_t v[kShareCols][kShareRows];
#pragma unroll
        for (int c = 0; c < kShareCols; ++c) {
          const int j = j0 + kPlanThreads * c + tid;
          ref[c] = j < jmax ? t0[j] : 0;
#pragma unroll
          for (int u = 0; u < kShareRows; ++u) v[c][u] = j < jmax ? p.bt[row[u] + j] : 0;
        }
#pragma unroll
        for (int c = 0; c < kShareCols; ++c)
#pragma unroll
          for (int u = 0; u < kShareRows; ++u) ok[c] = ok[c] && v[c][u] == ref[c];
      }
#pragma unroll
      for (int c = 0; c < kShareCols; ++c) {
        const int j = j0 + kPlanThreads * c + tid;
        ok[c] = j >= jmax || (ok[c] && ref[c] >= 0 && ref[c] < p.num_blocks);
      }
      int bad = jmax;
#pragma unroll
      for (int c = kShareCols - 1; c >= 0; --c)
        if (!ok[c]) bad = j0 + kPlanThreads * c + tid;
      first_bad = block_min(bad, red);
      if (first_bad < jmax) break;  // workgroup-uniform
    }
    shared_tok = (int)min((int64_t)first_bad * p.BS, (int64_t)minctx) / kChunk * kChunk;
    if (shared_tok < kCascadeMinChunks * kChunk) shared_tok = 0;
  }
  if (tid == 0) {
    p.ws_share[0] = shared_tok;
    p.ws_share[1] = (nd + p.SG - 1) / p.SG;
    p.ws_share[2] = r0;
    p.ws_share[3] = nd;
  }
}

// Q rows of a prefix group (NX 16-row tiles, XR = 16 NX rows): row r = 16 t + n is member
// r / RS of group grp (its decode-list index grp SG + r / RS), row r % RS of that sequence;
// every valid row sees all L shared keys. Same k-slot order as load_q.
template <int D, int NX, bool KV8>
__device__ __forceinline__ void load_q_group(WaveState<D, NX>& s, const PAParams& p, int grp, int nd, int L,
                                             int kvh) {
  const int lane = threadIdx.x & 63;
  const int j = lane >> 4, n = lane & 15;
#pragma unroll
  for (int t = 0; t < NX; ++t) {
    s.m[t] = -INFINITY;
    s.l[t] = 0.f;
    s.thr[t] = -INFINITY;
    s.nsh[t] = 0.f;
#pragma unroll
    for (int i = 0; i < D / 16; ++i) s.acc[t][i] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int r = 16 * t + n;
    const int mem = r / p.RS, rr = r % p.RS;
    const int idx = grp * p.SG + mem;
    bool valid = mem < p.SG && idx < nd;
    const int seq = valid ? p.ws_dec_list[idx] : 0;
    const SeqView sv = seq_view(p, seq);
    const int qi = rr / p.G, g = rr % p.G;
    valid = valid && qi < sv.q_len;
    if (valid) {
      const uint16_t* qp = (const uint16_t*)p.q + (sv.qs + qi) * p.q_ts + (int64_t)(kvh * p.G + g) * p.q_hs;
#pragma unroll
      for (int c = 0; c < D / 32; ++c) {
        const int d0 = KV8 ? 64 * (c >> 1) + 16 * j + 8 * (c & 1) : 32 * c + 8 * j;
        s.q[t][c] = *(const u32x4*)(qp + d0);
      }
      s.limit[t] = L;
    } else {
#pragma unroll
      for (int c = 0; c < D / 32; ++c) s.q[t][c] = u32x4{0, 0, 0, 0};
      s.limit[t] = 0;
    }
  }
}

__device__ __forceinline__ void write_job_x(int32_t* job, int pieces, int64_t slot0, int64_t qs, int R, int kvh0,
                                            int xpieces, int64_t xslot0, int xrow) {
  job[1] = pieces;
  job[2] = (int32_t)slot0;
  job[3] = (int32_t)slot0;
  job[4] = 1;
  job[5] = (int32_t)qs;
  job[6] = R;
  job[7] = 0;
  job[8] = kvh0;
  job[9] = xpieces;
  job[10] = (int32_t)xslot0;
  job[11] = xrow;
  job[0] = kJobDecode;
}

// Decode class: grid (NU * HGW / 4) workgroups of 4 waves; wave w of workgroup b is head
// w % HGW of unit (4 b + w) / HGW. In mixed batches (PLAN) workgroup 0 computes the prefill
// plan instead and the units start at workgroup 1. KV8: the cache is E4M3. NX: 16-row tiles
// of a cascade prefix group (XR = 16 NX rows; 1 outside the cascade).
template <class E, int D, int NT, bool KV8, int NX>
__global__ __launch_bounds__(256) void pa_decode_kernel(PAParams p) {
  if (p.PLAN && blockIdx.x == 0) {
    plan_prefill(p);
    return;
  }
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int gw = (blockIdx.x - (p.PLAN ? 1 : 0)) * kWavesPerWG + wave;
  const int unit = gw / p.HGW;
  // With two workgroups per CU, the second-round units (unit >= R1, each sharing its CUs with
  // a first-round unit) take the two head halves the other way round, so every CU reads both
  // halves of the token rows: a workgroup reading the first half of E4M3 rows (1 KB, heads 0-3)
  // ran ~11% slower than one reading the second, whichever XCD it sat on and with the data's
  // heads rotated, and a CU holding two of them set the launch. HBM-cold, decode kernel: C2
  // over E4M3 122.1 -> 118.3 us, C4 105.4 -> 102.5, C3's decode part 417 -> 405; the
  // reference's D = 64 grid 3-4% faster at its large points; one workgroup per CU unchanged.
  const int hw = (gw % p.HGW) ^ (p.HGW == 8 && p.R1 < p.NU && unit >= p.R1 ? 4 : 0);
  const int NHG = p.Hkv / p.HGW;

  // This unit's merge job: none unless it owns a split segment (below). Written on every
  // call, so the merge kernel never sees a stale record.
  int32_t* job = p.ws_job + (int64_t)unit * kJobInts;
  const bool job_writer = hw == 0 && lane == 0 && unit < p.NU;
  if (job_writer) job[0] = kJobNone;

  // Cascade: keys [0, L) of every decode-class sequence come from the prefix segments, which
  // take the first P = groups * NHG * L / 32 positions of the flat space.
  int L = 0, ngrp = 0, r0 = 0, nd = 0;
  if constexpr (NT == 1) {
    if (p.CASC) {
      L = (int)uni64(p.ws_share[0]);
      ngrp = (int)uni64(p.ws_share[1]);
      r0 = (int)uni64(p.ws_share[2]);
      nd = (int)uni64(p.ws_share[3]);
    }
  }
  const int Lc = L / kChunk;
  const int64_t P = L > 0 ? (int64_t)ngrp * NHG * Lc : 0;

  // Chunks per segment over all sequences (every wave computes the sum itself).
  int Cs = 0, Ns = 0;
  for (int blk0 = 0; blk0 < p.B; blk0 += 64) {
    SeqWindow sw;
    scan_window(sw, p, blk0, Cs, Ns, L);
    Cs += sw.total;
    Ns += sw.ntotal;
  }
  const int64_t C = P + (int64_t)Cs * NHG;
  const int64_t NUa = active_units(C, p.NU);
  if (unit >= NUa) return;
  const bool weighted = NX == 4 && P > 0;
  const bool rounds = KV8 && p.R1 < NUa;  // E4M3, two workgroups per CU: second-round shares
  const CostSplit split(P, C, NUa, weighted ? kPrefix64Cost : 1, weighted ? kChunkCost : 1, p.R1,
                        rounds ? kRound1Share : 1, rounds ? kRound2Share : 1);
  const int64_t a = split.begin(unit), b = split.begin(unit + 1);
  if (a >= b) return;

  int64_t pos = a;
  if constexpr (NT == 1) {
    // prefix segments (g, hg): the XR-row tiles of group g against keys [0, L) of head group
    // hg, read through the first sequence's table (the shared blocks); always partial
    while (pos < b && pos < P) {
      const int64_t pseg = pos / Lc;
      const int grp = (int)(pseg / NHG), hg = (int)(pseg % NHG);
      const int64_t seg_beg = pseg * Lc, seg_end = seg_beg + Lc;
      const int64_t y = b < seg_end ? b : seg_end;
      const int kvh = hg * p.HGW + hw;
      WaveState<D, NX> st;
      load_q_group<D, NX, KV8>(st, p, grp, nd, L, kvh);
      const int64_t* btrow = p.bt + (int64_t)r0 * p.bt_rs;
      // 16- and 32-row groups each read the shared keys: ordinary loads, so the other groups'
      // reads hit the Infinity Cache (non-temporal ones ran C4 over E4M3 103 -> 108 us with
      // 16-row groups)
      run_chunks<E, D, NX, KV8, (NX > 2)>(st, p, btrow, kvh, (int)(pos - seg_beg) * kChunk, kChunk,
                                          (int)(y - seg_beg) * kChunk, L);
      SeqView none{};
      write_rows<E, D, NX>(st, p, none, 16 * NX, 0, kvh, true, p.ws_xacc, p.ws_xml,
                           ((pseg + unit) * p.HGW + hw) * (16 * NX), 16 * NX);
      pos = y;
    }
  }

  // walk the segments overlapping [a, b) (positions past the prefix region)
  SeqWindow sw;
  scan_window(sw, p, 0, 0, 0, L);
  while (pos < b) {
    while (P + (int64_t)(sw.base + sw.total) * NHG <= pos)
      scan_window(sw, p, sw.blk0 + 64, sw.base + sw.total, sw.nbase + sw.ntotal, L);
    const int64_t start = P + (int64_t)(sw.base + sw.excl) * NHG;  // first chunk of this lane's sequence
    const uint64_t hit = __builtin_amdgcn_ballot_w64(sw.c > 0 && start <= pos && pos < start + (int64_t)sw.c * NHG);
    if (hit == 0) break;  // cannot happen for consistent metadata; never index lane 64
    const int l = __builtin_ctzll(hit);
    const int seq = sw.blk0 + l;
    const int c = __builtin_amdgcn_readlane(sw.c, l);
    const int64_t seq_start = P + (int64_t)(sw.base + __builtin_amdgcn_readlane(sw.excl, l)) * NHG;
    const int hg = (int)((pos - seq_start) / c);
    const int64_t seg_beg = seq_start + (int64_t)hg * c, seg_end = seg_beg + c;
    const int64_t y = b < seg_end ? b : seg_end;
    const int kvh = hg * p.HGW + hw;

    // the sequence's view from the window's lane l (no second, dependent read of the
    // metadata before the query and page-table loads: C2 200.1 -> 198.9 us HBM-cold, C2 over
    // E4M3 117.0 -> 115.9)
    SeqView sv;
    sv.qs = __builtin_amdgcn_readlane(sw.qs, l);
    sv.q_len = __builtin_amdgcn_readlane(sw.ql, l);
    sv.ctx = __builtin_amdgcn_readlane(sw.ctx, l);
    sv.kv_total = __builtin_amdgcn_readlane(sw.kvt, l);
    const int R = sv.q_len * p.G;
    const bool member = L > 0 && __builtin_amdgcn_readlane(sw.mem, l);
    const int skip = member ? L : 0;
    const int tok_lo = skip + (int)(pos - seg_beg) * kChunk;
    const int tok_hi = min(skip + (int)(y - seg_beg) * kChunk, sv.kv_total);
    WaveState<D, NT> st;
    load_q<D, NT, KV8>(st, p, sv.qs, R, 0, kvh, sv.ctx, sv.kv_total);
    const int64_t* btrow = p.bt + (int64_t)seq * p.bt_rs;
    run_chunks<E, D, NT, KV8>(st, p, btrow, kvh, tok_lo, kChunk, tok_hi, sv.kv_total);
    const bool whole = pos == seg_beg && y == seg_end && !member;
    const int64_t slot = (int64_t)seq * NHG + hg + unit;
    write_rows<E, D, NT, (KV8 && NT > 1)>(st, p, sv, R, 0, kvh, !whole, p.ws_acc, p.ws_ml, (slot * p.HGW + hw) * p.RS,
                                         p.RS);
    if (L > 0) {
      if (hw == 0 && lane == 0 && pos == seg_beg) {
        // one record per (seq, hg), written on every call: none for a whole segment; else the
        // segment's own pieces in slot + i (units unit .. u1) and, for a member, the prefix
        // segment (grp, hg)'s in pseg + uf + i (units uf .. ul), rows xrow .. of its tiles
        int32_t* xj = p.ws_xjob + ((int64_t)seq * NHG + hg) * kJobInts;
        const int64_t u1 = split.unit_of(seg_end - 1);
        if (whole) {
          xj[0] = kJobNone;
        } else if (member) {
          const int idx = sw.nbase + __builtin_amdgcn_readlane(sw.nexcl, l);
          const int grp = idx / p.SG, mem = idx % p.SG;
          const int64_t pseg = (int64_t)grp * NHG + hg;
          const int64_t x0 = pseg * Lc, x1 = x0 + Lc - 1;
          const int64_t uf = split.unit_of(x0), ul = split.unit_of(x1);
          write_job_x(xj, (int)(u1 - unit + 1), slot, sv.qs, R, hg * p.HGW, (int)(ul - uf + 1), pseg + uf,
                      mem * p.RS);
        } else {
          write_job_x(xj, (int)(u1 - unit + 1), slot, sv.qs, R, hg * p.HGW, 0, 0, 0);
        }
      }
    } else if (job_writer && pos == seg_beg && y < seg_end) {
      // the segment starts here and continues in units unit + 1 .. u1: piece i is in slot + i
      const int64_t u1 = split.unit_of(seg_end - 1);
      write_job(job, kJobDecode, (int)(u1 - unit + 1), slot, slot, 1, sv.qs, R, 0, hg * p.HGW);
    }
    pos = y;
  }
}

// Short decode (plan.short_decode: a decode-only batch of single-tile rows over block tables
// of at most kShortTokens keys): workgroup (kvh, seq) owns that sequence's rows of kv head kvh.
// Its 4 waves take chunks w, w + 4, w + 8, ... of the keys, then waves 1-3 hand their online-
// softmax state to wave 0 through LDS. The accumulator layout is the same in every wave, so
// the combination is per lane: M = max_w m_w, acc = sum_w 2^(m_w - M) acc_w, and likewise the
// lane-partial sums; wave 0 then writes the normalised rows. Nothing goes through the
// workspace and no merge launch follows: a batch this small is bound by latency, and the
// merge launch was a third of it.
template <class E, int D, bool KV8>
__global__ __launch_bounds__(256) void pa_decode_short_kernel(PAParams p) {
  constexpr int NI = D / 16;
  __shared__ f32x4 x_acc[kWavesPerWG - 1][NI][64];
  __shared__ float x_ml[kWavesPerWG - 1][2][64];
  const int kvh = blockIdx.x, seq = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const SeqView sv = seq_view_uniform(p, seq);
  if (sv.q_len == 0 || sv.q_len > p.QS) return;  // uniform over the workgroup
  const int R = sv.q_len * p.G;
  WaveState<D, 1> st;
  load_q<D, 1, KV8>(st, p, sv.qs, R, 0, kvh, sv.ctx, sv.kv_total);
  const int64_t* btrow = p.bt + (int64_t)seq * p.bt_rs;
  run_chunks<E, D, 1, KV8, false>(st, p, btrow, kvh, w * kChunk, kWavesPerWG * kChunk, sv.kv_total, sv.kv_total);
  if (w > 0) {
#pragma unroll
    for (int i = 0; i < NI; ++i) x_acc[w - 1][i][lane] = st.acc[0][i];
    x_ml[w - 1][0][lane] = st.m[0];
    x_ml[w - 1][1][lane] = st.l[0];
  }
  __syncthreads();
  if (w != 0) return;
  float mw[kWavesPerWG - 1];
  float M = st.m[0];
#pragma unroll
  for (int k = 0; k < kWavesPerWG - 1; ++k) {
    mw[k] = x_ml[k][0][lane];
    M = fmaxf(M, mw[k]);
  }
  const float ms = M == -INFINITY ? 0.f : M;  // no key seen by any wave: every weight is 0
  const float a0 = fast_exp2(st.m[0] - ms);
  st.l[0] *= a0;
#pragma unroll
  for (int i = 0; i < NI; ++i) st.acc[0][i] *= a0;
#pragma unroll
  for (int k = 0; k < kWavesPerWG - 1; ++k) {
    const float ak = fast_exp2(mw[k] - ms);
    st.l[0] += ak * x_ml[k][1][lane];
#pragma unroll
    for (int i = 0; i < NI; ++i) st.acc[0][i] += ak * x_acc[k][i][lane];
  }
  st.m[0] = M;
  write_rows<E, D, 1>(st, p, sv, R, 0, kvh, false, nullptr, nullptr, 0, 16);
}

// Log-sum-exp merge of split segments. A job covers `rows` partial rows per piece (HGW
// heads x RS rows for decode, PAParams::PR rows of one head for prefill); row x of piece i
// sits at (slot(i) * rows + x) in the partial arrays (whole rows; decode pieces of multi-tile
// rows over E4M3 caches in the tile-block layout of part_ofs). Each workgroup merges
// MR = F 1024 / D rows of one job: workgroups 0 .. NU * CD - 1 take decode unit b / CD, rows
// MR (b % CD) ..; the next NUP * (PR / MR) take prefill record b' / (PR / MR), rows
// MR (b' % (PR / MR)) ... Every thread owns F float4 of the MR rows and merges them online
// over the pieces, kMergeBatch / F pieces per round of loads. Rows are normalised at the store.
constexpr int kMergeBatch = 16;
// rows per merge workgroup with F float4 of one row per thread: F 1024 / D (decode-only
// batches F = 1: 8 rows at D = 128; mixed batches F = 4: 32 rows)
template <int D, int F = 1>
constexpr int merge_rows() {
  return F * 256 * 4 / D;
}

// F = 1 in decode-only batches; in mixed batches F = 4, since there a head's RS = 16 / G row
// slots mostly hold a single query's G rows and the workgroups past them return at once, and
// a prefill tile's rows merge from 2-3 pieces each, so a thread keeps more loads in flight
// with more float4 (C3, HBM-cold, three runs each: merge 24.7 -> 23.0 us against F = 2)
template <int D, bool MIXED>
constexpr int merge_rows_decode() {
  return MIXED ? merge_rows<D, 4>() : merge_rows<D, 1>();
}

// One workgroup's share of a merge job: rows MR = F * 1024 / D of it (chunk), F float4 of
// one row per thread.
// BLK: the decode pieces are in the tile-block layout (multi-tile rows over E4M3 caches, never
// with a cascade prefix).
template <class E, int D, int F, bool BLK>
__device__ __forceinline__ void merge_job(const PAParams& p, const int32_t* job, int chunk, bool casc) {
  constexpr int Q4 = D / 4;  // float4 per row
  constexpr int kMergeRows = merge_rows<D, F>();
  const int kind = job[0];
  if (kind == kJobNone) return;
  const bool dec = kind == kJobDecode;
  const int rows = dec ? p.HGW * p.RS : p.PR;
  const int pieces = job[1];
  const int64_t slot0 = job[2], slotb = job[3];
  const int stride = job[4];
  const int64_t qs = job[5];
  const int R = job[6], rbase = job[7], kvh0 = job[8];
  const int rph = dec ? p.RS : p.PR;  // rows per head
  // only the rows that reach the output: rv = min(rph, R - rbase) of each head's rph; the
  // workgroup's 16 are valid rows x0 .. x0 + 15, valid row v being piece row (v / rv) rph + v % rv
  const int rv = min(rph, R - rbase);
  const int x0 = chunk * kMergeRows;
  if (rv <= 0 || x0 >= (rows / rph) * rv) return;
  const int nr = min(kMergeRows, (rows / rph) * rv - x0);
  auto prow = [&](int v) { return (v / rv) * rph + v % rv; };
  const float* acc = dec ? p.ws_acc : p.ws_pacc;
  const float* ml = dec ? p.ws_ml : p.ws_pml;
  // Two piece sets: 0 = the job's own partials, row x of piece i at base(0, i) + x; 1 (cascade)
  // = the prefix segment's, row x (head x / RS, row x % RS) at row xrow + x % RS of that head's
  // XR-row tile, base(1, i) = (xslot0 + i) HGW XR.
  const int xpieces = casc ? job[9] : 0;
  const int64_t xslot0 = casc ? job[10] : 0;
  const int xrow = casc ? job[11] : 0;
  auto roff = [&](int set, int x) -> int64_t { return set == 0 ? x : (x / rph) * p.XR + xrow + x % rph; };
  auto base = [&](int set, int i) -> int64_t {
    return set == 0 ? (i == 0 ? slot0 : slotb + (int64_t)stride * i) * rows : (xslot0 + i) * p.HGW * p.XR;
  };
  const int nsets = xpieces > 0 ? 2 : 1;
  const int t = threadIdx.x;
  const int nq = nr * Q4;
  int qc[F];
#pragma unroll
  for (int f = 0; f < F; ++f) qc[f] = min(t + 256 * f, nq - 1);  // clamped: loads stay in the rows
  // item q -> (row of the workgroup's nr, float4 column): rows fastest for decode pieces in
  // the tile-block layout, which holds a column's tile rows in consecutive float4s (so
  // consecutive threads read consecutive float4s); columns fastest for whole rows
  auto qrow = [&](int q) {
    if constexpr (BLK) return dec ? q % nr : q / Q4;
    return q / Q4;
  };
  auto qcol = [&](int q) {
    if constexpr (BLK) return dec ? q / nr : q % Q4;
    return q % Q4;
  };

  // Online merge: kMergeBatch pieces at a time, every load of a batch (the m/l pair of each
  // float4's row and the float4) issued before any is used; the running max M moves per batch.
  f32x4 o[F];
  float M[F], Ls[F];
#pragma unroll
  for (int f = 0; f < F; ++f) {
    o[f] = f32x4{0.f, 0.f, 0.f, 0.f};
    M[f] = -INFINITY;
    Ls[f] = 0.f;
  }
  for (int set = 0; set < nsets; ++set) {
    const int n = set ? xpieces : pieces;
    const float* ap = set ? p.ws_xacc : acc;
    const float* mp = set ? p.ws_xml : ml;
    int64_t rr[F];  // this thread's rows relative to the piece base
    int64_t ro[F];  // and its float4's float offset from the piece base
#pragma unroll
    for (int f = 0; f < F; ++f) {
      rr[f] = roff(set, prow(x0 + qrow(qc[f])));
      const int c4 = qcol(qc[f]);
      ro[f] = rr[f] * D + 4 * c4;
      if constexpr (BLK) {
        if (dec) {  // decode pieces: per-head groups of cap rows
          const int cap = set ? p.XR : p.RS;
          const int rh = (int)(rr[f] % cap);
          ro[f] = (rr[f] - rh) * D + part_ofs<D>(rh, c4, cap);
        }
      }
    }
    auto batch = [&](int i0, auto kb) {
      constexpr int KB = decltype(kb)::value;
      float2 mv[KB][F];
      f32x4 av[KB][F];
#pragma unroll
      for (int k = 0; k < KB; ++k) {
        const int64_t bk = base(set, min(i0 + k, n - 1));
#pragma unroll
        for (int f = 0; f < F; ++f) {
          mv[k][f] = *(const float2*)(mp + (bk + rr[f]) * 2);
          if constexpr (BLK)
            av[k][f] = *(const f32x4*)(ap + bk * D + ro[f]);
          else
            av[k][f] = *(const f32x4*)(ap + (bk + rr[f]) * D + 4 * (qc[f] % Q4));
        }
      }
#pragma unroll
      for (int f = 0; f < F; ++f) {
        float mb = M[f];
#pragma unroll
        for (int k = 0; k < KB; ++k) mb = i0 + k < n ? fmaxf(mb, mv[k][f].x) : mb;
        const float ms = mb == -INFINITY ? 0.f : mb;  // all -inf so far: every weight is 0
        const float alpha = fast_exp2(M[f] - ms);
        o[f] *= alpha;
        Ls[f] *= alpha;
#pragma unroll
        for (int k = 0; k < KB; ++k) {
          const float w = i0 + k < n ? fast_exp2(mv[k][f].x - ms) : 0.f;
          Ls[f] += w * mv[k][f].y;
          o[f] += w * av[k][f];
        }
        M[f] = mb;
      }
    };
    // batches of kMergeBatch / F pieces (16 float4 loads in flight per thread), the rest as
    // 8 + 4 + 2 + 1: no load is issued for a missing piece
    constexpr int KB = kMergeBatch / F;
    int i0 = 0;
    for (; n - i0 >= KB; i0 += KB) batch(i0, std::integral_constant<int, KB>{});
    if (KB > 8 && n - i0 >= 8) {
      batch(i0, std::integral_constant<int, 8>{});
      i0 += 8;
    }
    if (n - i0 >= 4) {
      batch(i0, std::integral_constant<int, 4>{});
      i0 += 4;
    }
    if (n - i0 >= 2) {
      batch(i0, std::integral_constant<int, 2>{});
      i0 += 2;
    }
    if (n - i0 >= 1) batch(i0, std::integral_constant<int, 1>{});
  }
#pragma unroll
  for (int f = 0; f < F; ++f) {
    const int q = t + 256 * f;
    if (q >= nq) continue;
    const int xr = qrow(q), col = 4 * qcol(q);
    const int x = prow(x0 + xr);
    const int hw = x / rph, r = rbase + x % rph;
    const float inv = p.v_scale / (Ls[f] == 0.f ? 1.f : Ls[f]);
    uint16_t* dst = (uint16_t*)p.out + (qs + r / p.G) * p.o_ts + (int64_t)((kvh0 + hw) * p.G + r % p.G) * p.o_hs + col;
    *(u32x2*)dst = u32x2{E::pack2(o[f][0] * inv, o[f][1] * inv), E::pack2(o[f][2] * inv, o[f][3] * inv)};
  }
}

// MIXED: the batch has prefill-class sequences (prefill records after the decode units);
// decode and prefill jobs then both take 2 float4 per thread (16 rows at D = 128).
template <class E, int D, bool MIXED, bool BLK>
__global__ __launch_bounds__(256) void pa_merge_kernel(PAParams p) {
  constexpr int F = MIXED ? 4 : 1;
  constexpr int MR = merge_rows<D, F>();
  static_assert(!MIXED || ((kWavesPerWG * 16 * prefill_nt<false>()) % MR == 0 &&
                           (kWavesPerWG * 16 * prefill_nt<true>()) % MR == 0),
                "a prefill tile's rows split into whole merge chunks");
  const int CD = (p.HGW * p.RS + MR - 1) / MR;
  const int b = blockIdx.x;
  const int32_t* job;
  int chunk;
  bool casc = false;
  if (p.CASC && p.ws_share[0] > 0) {
    // cascade: one record per (sequence, head group), written for decode-class sequences
    const int NHG = p.Hkv / p.HGW;
    if (b >= p.B * NHG * CD) return;
    const int seg = b / CD;
    const SeqView v = seq_view(p, seg / NHG);
    if (v.q_len == 0 || v.q_len > p.QS) return;
    job = p.ws_xjob + (int64_t)seg * kJobInts;
    chunk = b % CD;
    casc = true;
  } else if (b < p.NU * CD) {
    job = p.ws_job + (int64_t)(b / CD) * kJobInts;
    chunk = b % CD;
  } else {
    if constexpr (!MIXED) return;
    const int bp = b - p.NU * CD;
    if (bp >= p.NUP * (p.PR / MR)) return;
    job = p.ws_job + ((int64_t)kMaxDecodeWaves + bp / (p.PR / MR)) * kJobInts;
    chunk = bp % (p.PR / MR);
  }
  merge_job<E, D, F, BLK>(p, job, chunk, casc);
}

// ---------------------------------------------------------------------------------------
// Prefill class (q_len > QS): a workgroup of 4 waves computes 64 NT query rows of one
// (sequence, kv head) (PAParams::PR: 192 over 16-bit caches, 128 over E4M3 caches), wave w
// holding rows 16 NT w .. 16 NT (w + 1) - 1 of the tile.
//
// The 4 waves share every 32-key K/V chunk through a 3-stage LDS ring filled by direct
// global->LDS loads (no VGPR staging): chunk c + 2 is in flight while chunk c is computed.
// K rows are stored in groups of kRowsPerLoad (one wave-wide load each): row r of a group
// holds, in 16-byte slot s, the row's global slot s ^ r, and each group after the first
// starts kKPad bytes further on, so the K-operand reads (one slot of 16 consecutive rows)
// hit 16 distinct bank groups while the swizzle of a load does not depend on which group it
// fills: a wave's loads share one lane offset and differ by a uniform step. Waves wait with
// s_waitcnt on their own loads, then a bare s_barrier makes all four waves' loads of the
// chunk visible.
template <int D>
struct PrefillLds {
  static_assert(D == 64 || D == 128, "prefill head sizes");
  static constexpr int kRowBytes = D * 2;                // one token row of one kv head
  static constexpr int kSlots = kRowBytes / 16;          // 16-byte slots per row
  static constexpr int kRowsPerLoad = 1024 / kRowBytes;  // rows one wave-wide load fills
  static constexpr int kTileBytes = kChunk * kRowBytes;  // K (or V) of one chunk
  static constexpr int kLoadsPerTile = kTileBytes / 1024;
  static constexpr int kLoadsPerWave = 2 * kLoadsPerTile / kWavesPerWG;  // K and V, split over 4 waves
  // D = 64: 8-row groups already cover the 8 slots; D = 128: 4-row groups, each shifted by
  // 4 slots from the previous (group g of a 16-row half spans bank groups 4 g + (0..3)).
  static constexpr int kKPad = kRowsPerLoad < kSlots ? 16 * kRowsPerLoad : 0;
  static constexpr int kKLoadBytes = 1024 + kKPad;          // one K row group
  static constexpr int kKHalfBytes = 16 / kRowsPerLoad * kKLoadBytes;  // 16 K rows
  static constexpr int kKBytes = kLoadsPerTile * kKLoadBytes;  // K of one chunk (V follows)
  static constexpr int kStages = 3;
  static constexpr int kStageBytes = kKBytes + kTileBytes;
};

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// One wave's share of the direct global->LDS loads of a chunk: kLoadsPerWave loads of
// kRowsPerLoad rows each, all of K or all of V and all in the same 16-token half, so one
// uniform base address per wave and chunk. Load k reads lane offset loff from the base plus
// k ustep bytes (SGPR base + VGPR offset form, one offset register for all loads) into the
// stage at dst + k lstride.
template <int D>
struct PfLoads {
  using L = PrefillLds<D>;
  static_assert(L::kLoadsPerWave * L::kRowsPerLoad == 16, "a wave's loads cover one 16-token half");
  static_assert(L::kLoadsPerTile % L::kLoadsPerWave == 0, "a wave's loads are all K or all V");
  const char* cache;  // kc or vc, at this kv head
  int64_t sb2, ss2;   // block and slot strides of that cache in bytes
  int h;              // the half (0: tokens 0-15 of the chunk, 1: 16-31)
  int dst;            // LDS byte offset of the first load within a stage
  int lstride;        // LDS bytes from one load to the next
  uint32_t ustep;     // global bytes from one load to the next (wave-uniform)
  uint32_t loff;      // the lane's global byte offset in the first load
};

// EB: bytes per cache element (2; 1 for an E4M3 cache, whose granules are the same 8
// elements in 8 bytes, converted on their way to the 16-bit stage).
template <int D, int EB = 2>
__device__ __forceinline__ void pf_loads_init(PfLoads<D>& pl, const PAParams& p, int w, int kvh) {
  using L = PrefillLds<D>;
  const int lane = threadIdx.x & 63;
  const int row_in = lane / L::kSlots, slot = lane % L::kSlots;
  const int g0 = w * L::kLoadsPerWave;
  const bool v = g0 / L::kLoadsPerTile != 0;
  const int i0 = g0 % L::kLoadsPerTile;
  pl.sb2 = EB * (v ? p.v_sb : p.k_sb);
  pl.ss2 = EB * (v ? p.v_ss : p.k_ss);
  pl.cache = (const char*)(v ? p.vc : p.kc) + (int64_t)kvh * (v ? p.v_sh : p.k_sh) * EB;
  pl.h = i0 * L::kRowsPerLoad / 16;
  if (!v) {
    // load k fills row group i0 + k: rows (i0 + k) R + row_in of the chunk, token
    // (k R + row_in) of half h's page (R = kRowsPerLoad, k R + row_in < 16), slot s ^ row_in
    pl.dst = i0 * L::kKLoadBytes;
    pl.lstride = L::kKLoadBytes;
    pl.ustep = (uint32_t)(L::kRowsPerLoad * pl.ss2);
    pl.loff = (uint32_t)(row_in * pl.ss2) + 8u * EB * (uint32_t)(slot ^ row_in);
  } else {
    // V stage layout: blocks b = h (D/16) + i of 512 bytes, block b holding d = 16i .. 16i+15
    // of the 16 tokens of half h, token-major (32 bytes per token). 16-byte granule P of the
    // stage is token (P % 32) / 2 of the half, global 16-byte chunk 2 (b % (D/16)) + P % 2.
    // Load k is granules P = 64 (i0 + k) + lane: the same token, chunk 4 k further on
    // (b % (D/16) = 2 k + lane / 32, since i0 is 0 or half the loads of a tile).
    pl.h = 2 * i0 / (D / 16);
    const int b = (64 * i0 + lane) / 32, tok = (lane % 32) / 2, chunk = 2 * (b % (D / 16)) + lane % 2;
    pl.dst = L::kKBytes + i0 * 1024;
    pl.lstride = 1024;
    pl.ustep = 32u * EB;
    pl.loff = (uint32_t)(tok * pl.ss2) + 8u * EB * (uint32_t)chunk;
  }
}

// Page descriptors of 64 consecutive chunks (c0 .. c0 + 63 of the tile's key space), one
// chunk per lane, refreshed every 64 chunks: no address arithmetic per chunk. Lane l holds
// the byte offset (within this wave's cache, at its kv head) of its half of chunk c0 + l;
// ok0 / ok1 have bit l set when half 0 / half 1 of that chunk is a page of the pool inside
// the tile's key range (a missing half is read from block 0 and masked).
struct PfWindow {
  uint32_t off_lo, off_hi;  // VGPRs
  uint64_t ok0, ok1;        // SGPRs
  int c0;
  int first_bad;            // first chunk >= c0 with a missing half (c0 + 64 when none)
};

__device__ __forceinline__ void pf_window(PfWindow& win, const PAParams& p, const int64_t* btrow, int c0, int c_end,
                                          int page_end, int hmine, int64_t sb2, int64_t ss2) {
  const int lane = threadIdx.x & 63;
  const int c = c0 + lane;
  const int r = p.BS / 16;  // 16-token halves per page (BS % 16 == 0)
  int id[2];
  bool ok[2], in[2];
  int off[2];
  int64_t raw[2];
  // both loads are issued before either is used (one memory round trip). Every lane loads
  // (column 0 when its page is outside the range: W >= 1), so the load is no divergent
  // branch whose join could hold a spill store ahead of the exec restore.
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int hh = 2 * c + h;
    const int pg = hh / r;
    off[h] = (hh - pg * r) * 16;
    in[h] = c < c_end && pg < page_end;
    raw[h] = btrow[in[h] ? pg : 0];
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int64_t b = in[h] ? raw[h] : -1;
    ok[h] = b >= 0 && b < p.num_blocks;
    id[h] = ok[h] ? (int)b : 0;
  }
  win.ok0 = __builtin_amdgcn_ballot_w64(ok[0]);
  win.ok1 = __builtin_amdgcn_ballot_w64(ok[1]);
  const uint64_t bad = ~(win.ok0 & win.ok1);
  win.first_bad = c0 + (bad ? (int)__builtin_ctzll(bad) : 64);
  const int idm = hmine ? id[1] : id[0];
  const int offm = hmine ? off[1] : off[0];
  const uint64_t o = (uint64_t)(uint32_t)idm * (uint64_t)sb2 + (uint64_t)(uint32_t)offm * (uint64_t)ss2;
  win.off_lo = (uint32_t)o;
  win.off_hi = (uint32_t)(o >> 32);
  win.c0 = c0;
}

// DMA of chunk ci (which the window holds) into the stage at LDS byte offset `stage`. The
// chunk's base address and the lanes' offsets pass through empty asm statements so that
// instruction selection (per basic block) sees sgpr64 + zext(vgpr32) and picks the
// SGPR-base + 32-bit VGPR-offset form; otherwise the hoisted 64-bit offsets cost two VGPRs
// and an add per load.
template <int D>
__device__ __forceinline__ void pf_issue(char* lds, int stage, const PfLoads<D>& pl, const PfWindow& win, int ci) {
  using L = PrefillLds<D>;
  const int rel = ci - win.c0;
  const uint64_t o = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(win.off_hi, rel) << 32) |
                     (uint32_t)__builtin_amdgcn_readlane(win.off_lo, rel);
  uint32_t off = pl.loff;
  asm volatile("" : "+v"(off));  // a 32-bit offset in this block: the loads' VGPR operand
#pragma unroll
  for (int k = 0; k < L::kLoadsPerWave; ++k) {
    uint64_t base = (uint64_t)(uintptr_t)pl.cache + o + (uint64_t)k * pl.ustep;
    asm volatile("" : "+s"(base));
    __builtin_amdgcn_global_load_lds((const void*)((const char*)(uintptr_t)base + off),
                                     (lds_ptr_t)(lds + stage + pl.dst + k * pl.lstride), 16, 0, 0);
  }
}

// Lane byte addresses of the K-operand reads (slot cc of rows n and 16 + n; the XOR swizzle
// of a row only depends on row % 16, so both 16-row tiles share them).
template <int D>
__device__ __forceinline__ void pf_k_lanes(uint32_t ka[D / 32], const char* lds) {
  using L = PrefillLds<D>;
  const int lane = threadIdx.x & 63;
  const int j = lane >> 4, n = lane & 15;
#pragma unroll
  for (int cc = 0; cc < D / 32; ++cc)
    ka[cc] = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)lds +
             n / L::kRowsPerLoad * L::kKLoadBytes + n % L::kRowsPerLoad * L::kRowBytes +
             16 * ((4 * cc + j) ^ (n % L::kRowsPerLoad));
}

// S^T of one chunk from the K stage, one 16-key tile at a time (16 registers of K operands
// live instead of 32).
template <class E, int D, int NT>
__device__ __forceinline__ void pf_scores_lds(const WaveState<D, NT>& s, const uint32_t ka[D / 32], int stage,
                                              f32x4 st[NT][2]) {
  using L = PrefillLds<D>;
  typedef const __attribute__((address_space(3))) u32x4* lds_u32x4_ptr;
#pragma unroll
  for (int tile = 0; tile < 2; ++tile) {
    u32x4 k[D / 32];
#pragma unroll
    for (int cc = 0; cc < D / 32; ++cc)
      k[cc] = *(lds_u32x4_ptr)(uintptr_t)(ka[cc] + (uint32_t)(stage + tile * L::kKHalfBytes));
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int cc = 0; cc < D / 32; ++cc) a = E::mfma(k[cc], s.q[t][cc], a);
      st[t][tile] = a;
    }
  }
}

// O^T += V^T P^T from the V stage with gfx950 transpose reads. ds_read_b64_tr_b16 hands lane
// 4q + r of each 16-lane group element r of the 8 bytes read by lanes 4k + q (k = 0..3). With
// lane l reading block b at byte 8 l, group j (lanes 16j ..) reads tokens 4j .. 4j + 3 of the
// half, and lane (j, n) receives V[token 4j + k][16i + n] for k = 0..3: the A-operand slots of
// output tile i in the same token order as P^T (tokens 4j + e of half 0, then of half 1).
// The accumulator row 4j + e of tile i is then d = 16i + 4j + e. MASKED zeroes the V of
// tokens that are absent or at/after data_end (other=0.0 in the reference's masked loads).
//
// The reads are inline asm on purpose. The compiler cannot tell a transpose read of this
// stage from the LDS DMA still filling the next stages, so for the builtin it inserts
// s_waitcnt vmcnt(0) first, which drains every K/V load in flight and exposes the full
// memory latency once per chunk. The kernel orders DMA and reads itself (s_waitcnt vmcnt on
// its own loads + s_barrier), so the reads are issued as asm and waited for with
// lgkmcnt(n) counting only the transpose reads issued after the awaited pair: LDS results
// return in order, so that wait is exact even when other LDS or scalar loads are in flight.
template <int N>
struct StaticFor {
  template <class F>
  static __device__ __forceinline__ void run(F&& f) {
    StaticFor<N - 1>::run(f);
    f(std::integral_constant<int, N - 1>{});
  }
};
template <>
struct StaticFor<0> {
  template <class F>
  static __device__ __forceinline__ void run(F&&) {}
};

template <int D>
struct VTr {
  u32x2 lo[D / 16], hi[D / 16];  // tokens 0-15 / 16-31 of the chunk for output tile i
};

template <int OFF>
__device__ __forceinline__ void ds_read_tr16_b64(u32x2& dst, uint32_t lds_addr) {
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(dst) : "v"(lds_addr), "i"(OFF));
}

// Pair i (tile i's two transpose reads) for i in [I0, I1), from the V tile at byte offset
// VOFF (a compile-time constant, folded into the instructions' offset field) from `base`.
template <int D, int VOFF, int I0, int I1>
__device__ __forceinline__ void pf_v_issue(VTr<D>& v, uint32_t base) {
  StaticFor<I1 - I0>::run([&](auto I) {
    constexpr int i = I0 + decltype(I)::value;
    ds_read_tr16_b64<VOFF + 512 * i>(v.lo[i], base);
    ds_read_tr16_b64<VOFF + 512 * (D / 16 + i)>(v.hi[i], base);
  });
}

__device__ __forceinline__ uint32_t lds_lane_addr(const char* tile, int bytes_per_lane) {
  const int lane = threadIdx.x & 63;
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)tile + (uint32_t)(bytes_per_lane * lane);
}

template <int N>
__device__ __forceinline__ void lgkm_wait_tied(u32x2& a, u32x2& b) {
  // s_waitcnt lgkmcnt(N); the operands tie the awaited registers to the wait so no use of
  // them is scheduled above it
  asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(a), "+v"(b) : "i"(N));
}

// Pairs 0 and 1 were issued by the caller (kVLead pairs ahead); pair i + kVLead is issued
// right after tile i's MFMAs, so at the wait for pair i exactly the kVLead - 1 later pairs
// may still be in flight.
constexpr int kVLead = 2;

template <class E, int D, int NT, bool MASKED, int VOFF>
__device__ __forceinline__ void pf_pv(WaveState<D, NT>& s, VTr<D>& v, uint32_t vbase, const ChunkRef& c,
                                      int data_end, const u32x4 pt[NT]) {
  constexpr int NI = D / 16;
  const int lane = threadIdx.x & 63;
  const int j = lane >> 4;
  uint32_t keep[4] = {~0u, ~0u, ~0u, ~0u};  // dword w: tokens of slots 2w, 2w + 1
  if (MASKED) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int h = w >> 1;
      const int tok = c.tok0 + 16 * h + 4 * j + 2 * (w & 1);
      const bool ok = c.blk[h] >= 0;
      keep[w] = (ok && tok < data_end ? 0x0000ffffu : 0u) | (ok && tok + 1 < data_end ? 0xffff0000u : 0u);
    }
  }
  StaticFor<NI>::run([&](auto I) {
    constexpr int i = decltype(I)::value;
    constexpr int later = (i + kVLead <= NI ? kVLead - 1 : NI - 1 - i);  // pairs issued after pair i
    lgkm_wait_tied<2 * later>(v.lo[i], v.hi[i]);
    u32x4 va = {v.lo[i][0], v.lo[i][1], v.hi[i][0], v.hi[i][1]};
    if (MASKED) {
#pragma unroll
      for (int w = 0; w < 4; ++w) va[w] &= keep[w];
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) s.acc[t][i] = E::mfma(va, pt[t], s.acc[t][i]);
    if constexpr (i + kVLead < NI) pf_v_issue<D, VOFF, i + kVLead, i + kVLead + 1>(v, vbase);
  });
}

// Prefill output / partial rows from the pf_pv accumulator layout (d = 16i + 4j + e).
template <class E, int D, int NT>
__device__ __forceinline__ void pf_write_rows(const WaveState<D, NT>& s, const PAParams& p, const SeqView& sv,
                                              int R, int row0, int kvh, bool partial, int64_t row_base) {
  const int lane = threadIdx.x & 63;
  const int j = lane >> 4, n = lane & 15;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const float L = sum_over_groups(s.l[t]);
    const int r = row0 + 16 * t + n;
    if (r >= R) continue;
    if (!partial) {
      const int qi = r / p.G, g = r % p.G;
      const float inv = p.v_scale / (L == 0.f ? 1.f : L);
      uint16_t* base = (uint16_t*)p.out + (sv.qs + qi) * p.o_ts + (int64_t)(kvh * p.G + g) * p.o_hs + 4 * j;
#pragma unroll
      for (int i = 0; i < D / 16; ++i)
        *(u32x2*)(base + 16 * i) = u32x2{E::pack2(s.acc[t][i][0] * inv, s.acc[t][i][1] * inv),
                                         E::pack2(s.acc[t][i][2] * inv, s.acc[t][i][3] * inv)};
    } else {
      const int64_t idx = row_base + r;
      float* dst = p.ws_pacc + idx * D + 4 * j;
#pragma unroll
      for (int i = 0; i < D / 16; ++i) *(f32x4*)(dst + 16 * i) = s.acc[t][i];
      if (j == 0) {
        p.ws_pml[idx * 2] = s.m[t];
        p.ws_pml[idx * 2 + 1] = L;
      }
    }
  }
}

template <int N>
__device__ __forceinline__ void wait_vm() {
  // s_waitcnt vmcnt(N), expcnt/lgkmcnt left free (gfx9 encoding)
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Wave priority from the unit's remaining share of its work (`total` positions, `rest` of
// them after this tile, n - i chunks of the tile left at chunk i): the arbiter favours older
// waves, so workgroups that started together on a CU drift apart and the last one runs its
// tail alone; raising the priority of the workgroups that are behind keeps them together.
// The level min(3, kPrioSteps left / (total + 1)), left = rest + n - i, falls over the last
// 3 / kPrioSteps of the unit's work (eighths: the workgroups on a CU stay closer at the end
// than with quarters, C3 2% faster; sixteenths gain nothing more). It only falls as i grows,
// so it is set at a tile's first chunk and again at the chunks where it drops: lvl(i) >= k
// exactly for i <= rest + n - ceil(k (total + 1) / kPrioSteps). (A host test evaluates both
// expressions from this source against the per-chunk formula.)
constexpr int kPrioSteps = 8;
struct PfPriority {
  int next_drop;  // first chunk whose level is below the current one
  __device__ __forceinline__ void set(int i, int n, int rest, int total) {
    const int lvl = min(3, (kPrioSteps * (rest + n - i)) / (total + 1));
    if (lvl >= 2)
      lvl == 3 ? __builtin_amdgcn_s_setprio(3) : __builtin_amdgcn_s_setprio(2);
    else
      lvl == 1 ? __builtin_amdgcn_s_setprio(1) : __builtin_amdgcn_s_setprio(0);
    next_drop = lvl > 0 ? rest + n - (lvl * (total + 1) + kPrioSteps - 1) / kPrioSteps + 1 : INT32_MAX;
  }
};

// The query tile as the score MFMAs take it, and the exp2 argument's factor c > 0: the
// argument is fma(score, c, -m) in fp32 (the scale is never rounded into a 16-bit Q, whose
// rounding would move large scores by up to 2^-9 of their size); for a negative scale
// S c = (-Q) K^T |c| (a sign flip of Q is exact), for a zero scale every score is
// 0 = (0 Q) K^T 1.
template <class E, int D, int NT>
__device__ __forceinline__ float pf_q_ready(WaveState<D, NT>& s, const PAParams& p) {
  float c = fabsf(p.qk_scale);
  if (p.qk_scale < 0.f) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int cc = 0; cc < D / 32; ++cc) s.q[t][cc] ^= 0x80008000u;
  } else if (p.qk_scale == 0.f) {
    c = 1.f;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int cc = 0; cc < D / 32; ++cc) s.q[t][cc] = u32x4{0u, 0u, 0u, 0u};
  }
  return c;
}

// One workgroup's pass over chunks [c_lo, c_hi) of tile t of (seq, kvh): the whole tile
// (written out) or a piece of it (partial in slot `slot` of the prefill partial arrays).
//
// Per chunk a wave waits for its own loads of the chunk, meets the other three at a bare
// s_barrier (the chunk is complete in LDS and the stage of chunk i - 1 is free), refills that
// stage with chunk i + 2 and computes chunk i. Three loops keep every accumulator in place
// (no merge at a branch join): chunks every valid row of the wave sees whole (unmasked, the
// ring stage of each step known at compile time, so every LDS address is an immediate
// offset), the chunks on the causal diagonal or with a missing page (masked), then the
// chunks past the wave's rows (loads and barriers only).
template <class E, int D>
__device__ __forceinline__ void prefill_tile(char* lds, const PAParams& p, const SeqView& sv, int R, int seq,
                                             int kvh, int t, int c_lo, int c_hi, int w, bool partial,
                                             int64_t slot, int rest, int total) {
  constexpr int NT = prefill_nt<false>();
  constexpr int PRW = kWavesPerWG * 16 * NT;  // rows of a tile
  using L = PrefillLds<D>;
  c_lo = uni(c_lo);
  c_hi = uni(c_hi);
  const int wg_row0 = t * PRW;
  const int wg_last = min(wg_row0 + PRW - 1, R - 1);
  const int kv_lim = (int)clamp64(sv.ctx + wg_last / p.G + 1, 0, sv.kv_total);
  const int row0 = wg_row0 + w * 16 * NT;
  const int my_last = min(row0 + 16 * NT - 1, R - 1);
  const int my_lim = row0 < R ? (int)clamp64(sv.ctx + my_last / p.G + 1, 0, sv.kv_total) : 0;

  // keys below every valid row's causal limit (that of the wave's first row)
  const int lim_all = row0 < R ? (int)clamp64(sv.ctx + row0 / p.G + 1, 0, sv.kv_total) : 0;

  // the page window first: the first chunks' loads wait for it, the query tile is not
  // needed before they are in flight
  const int64_t* btrow = p.bt + (int64_t)seq * p.bt_rs;
  const int page_end = (kv_lim + p.BS - 1) / p.BS;
  PfLoads<D> pl;
  pf_loads_init<D>(pl, p, w, kvh);
  PfWindow win;
  pf_window(win, p, btrow, c_lo, c_hi, page_end, pl.h, pl.sb2, pl.ss2);
  WaveState<D, NT> s;
  load_q<D, NT>(s, p, sv.qs, R, row0, kvh, sv.ctx, sv.kv_total);
  uint32_t ka[D / 32];
  pf_k_lanes<D>(ka, lds);
  const uint32_t vbase = lds_lane_addr(lds, 8);

  // every wave has finished reading the ring (previous tile) before it is refilled
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  const int n = c_hi - c_lo;
  // this wave's rows see chunks c_lo .. c_lo + n_my - 1 only; it keeps taking part in the
  // loads and barriers of the rest
  const int n_my = max(0, min(n, (my_lim + kChunk - 1) / kChunk - c_lo));
  int n_int = max(0, min(n_my, min(lim_all / kChunk, win.first_bad) - c_lo));
  pf_issue<D>(lds, 0, pl, win, c_lo);
  if (n > 1) pf_issue<D>(lds, L::kStageBytes, pl, win, c_lo + 1);
  // Q and the page window were loaded together, Q is transformed while the first chunks load
  const float c = pf_q_ready<E, D, NT>(s, p);

  PfPriority prio;
  prio.set(0, n, rest, total);
  // step i: wait for chunk i, then refill the stage chunk i - 1 used (`next`) with chunk i + 2
  auto sync = [&](int i, int next) {
    if (i >= prio.next_drop) prio.set(i, n, rest, total);
    const int ci2 = c_lo + i + 2;
    if (i + 2 < n && ci2 - win.c0 >= 64) {  // the window moves on (every 62 chunks)
      pf_window(win, p, btrow, c_lo + i, c_hi, page_end, pl.h, pl.sb2, pl.ss2);
      // the unmasked run reaches as far as the new window allows (the old window's end
      // capped it; a missing page before this point has already ended the run)
      n_int = max(0, min(n_my, min(lim_all / kChunk, win.first_bad) - c_lo));
    }
    __builtin_amdgcn_sched_barrier(0);
    if (i + 1 < n)
      wait_vm<L::kLoadsPerWave>();  // chunk i + 1 may stay in flight
    else
      wait_vm<0>();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    if (i + 2 < n) pf_issue<D>(lds, next, pl, win, ci2);
    __builtin_amdgcn_sched_barrier(0);
  };
  // chunk i from the stage at byte offset SOFF + stage (SOFF a compile-time constant)
  auto compute = [&](int i, int stage, auto soff, auto masked) {
    constexpr int SOFF = decltype(soff)::value;
    constexpr bool MASKED = decltype(masked)::value;
    f32x4 sc[NT][2];
    pf_scores_lds<E, D, NT>(s, ka, SOFF + stage, sc);
    ChunkRef cr;
    cr.tok0 = (c_lo + i) * kChunk;
    cr.blk[0] = cr.blk[1] = 0;
    if (MASKED) {
      const int rel = c_lo + i - win.c0;
      cr.blk[0] = (win.ok0 >> rel) & 1 ? 0 : -1;
      cr.blk[1] = (win.ok1 >> rel) & 1 ? 0 : -1;
      pf_mask<NT>(sc, s.limit, cr);
    }
    float mx[NT];
    pf_lanemax<NT>(sc, mx);
    // the V transpose reads go out once the scores are in (every QK MFMA has completed, so
    // the reads may reuse the K registers); their latency hides under the exponentials
    __builtin_amdgcn_sched_barrier(0);
    VTr<D> vt;
    const uint32_t vb = vbase + (uint32_t)stage;
    pf_v_issue<D, SOFF + L::kKBytes, 0, kVLead>(vt, vb);
    __builtin_amdgcn_sched_barrier(0);
    u32x4 pt[NT];
    pf_softmax<E, D, NT>(s, sc, mx, c, pt);
    pf_pv<E, D, NT, MASKED, SOFF + L::kKBytes>(s, vt, vb, cr, sv.kv_total, pt);
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, L::kStageBytes>;
  using S2 = std::integral_constant<int, 2 * L::kStageBytes>;
  int i = 0;
  while (i < n_int) {  // unmasked, unrolled by the ring's 3 stages
    sync(i, 2 * L::kStageBytes);
    compute(i, 0, S0{}, std::false_type{});
    if (++i >= n_int) break;
    sync(i, 0);
    compute(i, 0, S1{}, std::false_type{});
    if (++i >= n_int) break;
    sync(i, L::kStageBytes);
    compute(i, 0, S2{}, std::false_type{});
    ++i;
  }
  int stg = i % 3;
  for (; i < n_my; ++i) {  // masked
    const int next = stg == 0 ? 2 : stg - 1;
    sync(i, next * L::kStageBytes);
    compute(i, stg * L::kStageBytes, S0{}, std::true_type{});
    stg = stg == 2 ? 0 : stg + 1;
  }
  for (; i < n; ++i) {  // past this wave's rows: loads and barriers only
    const int next = stg == 0 ? 2 : stg - 1;
    sync(i, next * L::kStageBytes);
    stg = stg == 2 ? 0 : stg + 1;
  }
  pf_write_rows<E, D, NT>(s, p, sv, R, row0, kvh, partial, slot * PRW - wg_row0);
}

// prefill_tile over an E4M3 cache. Direct global->LDS loads cannot convert, so each lane
// loads, as E4M3, the 8-element granules the DMA would have moved (half the bytes, the
// same offsets halved), converts them exactly to E's 16-bit type and writes them to the LDS
// positions the DMA would have filled: the stage layout, the operand reads and the compute
// are those of prefill_tile. Two register sets keep the loads two chunks ahead; chunk i is
// converted and written right before the barrier that publishes it, so two LDS stages
// suffice (stage i % 2 was last read by chunk i - 2, before the previous barrier).
template <class E, int D>
__device__ __forceinline__ void prefill_tile_kv8(char* lds, const PAParams& p, const SeqView& sv, int R, int seq,
                                                 int kvh, int t, int c_lo, int c_hi, int w, bool partial,
                                                 int64_t slot, int rest, int total) {
  constexpr int NT = prefill_nt<true>();
  constexpr int PRW = kWavesPerWG * 16 * NT;  // rows of a tile
  using L = PrefillLds<D>;
  constexpr int KLW = L::kLoadsPerWave;
  typedef __attribute__((address_space(3))) u32x4* lds_u32x4_ptr;
  c_lo = uni(c_lo);
  c_hi = uni(c_hi);
  const int lane = threadIdx.x & 63;
  const int wg_row0 = t * PRW;
  const int wg_last = min(wg_row0 + PRW - 1, R - 1);
  const int kv_lim = (int)clamp64(sv.ctx + wg_last / p.G + 1, 0, sv.kv_total);
  const int row0 = wg_row0 + w * 16 * NT;
  const int my_last = min(row0 + 16 * NT - 1, R - 1);
  const int my_lim = row0 < R ? (int)clamp64(sv.ctx + my_last / p.G + 1, 0, sv.kv_total) : 0;
  const int lim_all = row0 < R ? (int)clamp64(sv.ctx + row0 / p.G + 1, 0, sv.kv_total) : 0;

  // the page window first: the first chunks' loads wait for it, the query tile is not
  // needed before they are in flight
  const int64_t* btrow = p.bt + (int64_t)seq * p.bt_rs;
  const int page_end = (kv_lim + p.BS - 1) / p.BS;
  PfLoads<D> pl;
  pf_loads_init<D, 1>(pl, p, w, kvh);
  PfWindow win;
  pf_window(win, p, btrow, c_lo, c_hi, page_end, pl.h, pl.sb2, pl.ss2);
  WaveState<D, NT> s;
  load_q<D, NT>(s, p, sv.qs, R, row0, kvh, sv.ctx, sv.kv_total);
  uint32_t ka[D / 32];
  pf_k_lanes<D>(ka, lds);
  const uint32_t vbase = lds_lane_addr(lds, 8);

  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();  // every wave has finished reading the stages (previous tile)
  __builtin_amdgcn_sched_barrier(0);
  const int n = c_hi - c_lo;
  const int n_my = max(0, min(n, (my_lim + kChunk - 1) / kChunk - c_lo));
  int n_int = max(0, min(n_my, min(lim_all / kChunk, win.first_bad) - c_lo));

  u32x2 raw[2][KLW];
  auto issue = [&](u32x2 (&r)[KLW], int ci) {
    const int rel = ci - win.c0;
    const uint64_t o = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(win.off_hi, rel) << 32) |
                       (uint32_t)__builtin_amdgcn_readlane(win.off_lo, rel);
    uint32_t off = pl.loff;
    asm volatile("" : "+v"(off));
#pragma unroll
    for (int k = 0; k < KLW; ++k) {
      uint64_t base = (uint64_t)(uintptr_t)pl.cache + o + (uint64_t)k * pl.ustep;
      asm volatile("" : "+s"(base));
      r[k] = *(const u32x2*)((const char*)(uintptr_t)base + off);
    }
  };
  issue(raw[0], c_lo);
  if (n > 1) issue(raw[1], c_lo + 1);
  const float c = pf_q_ready<E, D, NT>(s, p);

  PfPriority prio;  // wave priority as in prefill_tile
  prio.set(0, n, rest, total);
  // step i: wait for chunk i's bytes, convert them into stage i % 2, publish, load chunk i + 2
  auto sync = [&](int i, auto set) {
    constexpr int S = decltype(set)::value;
    if (i >= prio.next_drop) prio.set(i, n, rest, total);
    const int ci2 = c_lo + i + 2;
    if (i + 2 < n && ci2 - win.c0 >= 64) {
      pf_window(win, p, btrow, c_lo + i, c_hi, page_end, pl.h, pl.sb2, pl.ss2);
      // the unmasked run reaches as far as the new window allows (the old window's end
      // capped it; a missing page before this point has already ended the run)
      n_int = max(0, min(n_my, min(lim_all / kChunk, win.first_bad) - c_lo));
    }
    __builtin_amdgcn_sched_barrier(0);
    if (i + 1 < n)
      wait_vm<KLW>();  // chunk i + 1 may stay in flight
    else
      wait_vm<0>();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < KLW; ++k) {
      const u32x2 r = raw[S][k];
      const u32x4 o = {E::template from_fp8x2<false>(r[0]), E::template from_fp8x2<true>(r[0]),
                       E::template from_fp8x2<false>(r[1]), E::template from_fp8x2<true>(r[1])};
      *(lds_u32x4_ptr)(uintptr_t)((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)lds +
                                  (uint32_t)(S * L::kStageBytes + pl.dst + k * pl.lstride + 16 * lane)) = o;
    }
    __syncthreads();  // the stage's writes are complete and visible; nothing else in flight
    __builtin_amdgcn_sched_barrier(0);
    if (i + 2 < n) issue(raw[S], ci2);
    __builtin_amdgcn_sched_barrier(0);
  };
  // chunk i from the stage at byte offset SOFF + stage (one masked instance with a runtime
  // stage: two static ones in the masked loop double the live ranges and spill)
  auto compute = [&](int i, int stage, auto soff, auto masked) {
    constexpr int SOFF = decltype(soff)::value;
    constexpr bool MASKED = decltype(masked)::value;
    f32x4 sc[NT][2];
    pf_scores_lds<E, D, NT>(s, ka, SOFF + stage, sc);
    ChunkRef cr;
    cr.tok0 = (c_lo + i) * kChunk;
    cr.blk[0] = cr.blk[1] = 0;
    if (MASKED) {
      const int rel = c_lo + i - win.c0;
      cr.blk[0] = (win.ok0 >> rel) & 1 ? 0 : -1;
      cr.blk[1] = (win.ok1 >> rel) & 1 ? 0 : -1;
      pf_mask<NT>(sc, s.limit, cr);
    }
    float mx[NT];
    pf_lanemax<NT>(sc, mx);
    __builtin_amdgcn_sched_barrier(0);
    VTr<D> vt;
    const uint32_t vb = vbase + (uint32_t)stage;
    pf_v_issue<D, SOFF + L::kKBytes, 0, kVLead>(vt, vb);
    __builtin_amdgcn_sched_barrier(0);
    u32x4 pt[NT];
    pf_softmax<E, D, NT>(s, sc, mx, c, pt);
    pf_pv<E, D, NT, MASKED, SOFF + L::kKBytes>(s, vt, vb, cr, sv.kv_total, pt);
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, L::kStageBytes>;
  int i = 0;
  while (i < n_int) {  // unmasked, unrolled by the two stages
    sync(i, I0{});
    compute(i, 0, S0{}, std::false_type{});
    if (++i >= n_int) break;
    sync(i, I1{});
    compute(i, 0, S1{}, std::false_type{});
    ++i;
  }
  for (; i < n; ++i) {  // masked, then past this wave's rows (loads, conversions, barriers)
    if (i & 1)
      sync(i, I1{});
    else
      sync(i, I0{});
    if (i < n_my) compute(i, (i & 1) * L::kStageBytes, S0{}, std::true_type{});
  }
  pf_write_rows<E, D, NT>(s, p, sv, R, row0, kvh, partial, slot * PRW - wg_row0);
}

// Chunks of tile t (rows 128 t .. of R): those its last row can see, at least one so that
// every tile is visited and written.
__device__ __forceinline__ int pre_tile_chunks(const PAParams& p, const SeqView& sv, int R, int t) {
  const int last = min(p.PR * t + p.PR - 1, R - 1);
  const int lim = (int)clamp64(sv.ctx + last / p.G + 1, 0, sv.kv_total);
  return max(1, (lim + kChunk - 1) / kChunk);
}

// Fixed cost of a tile (Q load, pipeline fill, output write) in chunk steps: each tile
// occupies kTileCost + chunks positions of the flat space, the first kTileCost virtual.
constexpr int kTileCost = 4;

// Flat positions of all tiles of one kv head of a prefill-class sequence; 0 for others.
__device__ __forceinline__ int64_t pre_seq_chunks(const PAParams& p, const SeqView& sv) {
  if (sv.q_len <= p.QS) return 0;
  const int R = sv.q_len * p.G;
  const int tiles = (R + p.PR - 1) / p.PR;
  int64_t n = 0;
  for (int t = 0; t < tiles; ++t) n += kTileCost + pre_tile_chunks(p, sv, R, t);
  return n;
}

// Prefill plan, computed by workgroup 0 of the decode launch in mixed batches (so it runs
// under the decode work instead of ahead of it): the list of prefill-class sequences, the
// flat start of each (prefix sums of Hkv x pre_seq_chunks) and, for each prefill workgroup,
// a record of where its unit starts (below). Every prefill workgroup then starts from one
// scalar load of its record instead of scanning the batch or chasing the unit -> sequence
// -> lengths chain through memory.
__device__ void plan_prefill(const PAParams& p) {
  __shared__ int64_t s_pos[kPlanThreads];
  __shared__ int32_t s_cnt[kPlanThreads];
  __shared__ int64_t s_beg[kPlanLdsSeqs + 1];
  const int tid = threadIdx.x;
  const int per = (p.B + kPlanThreads - 1) / kPlanThreads;
  const int s0 = min(tid * per, p.B), s1 = min(s0 + per, p.B);
  int64_t pos = 0;
  int cnt = 0;
  for (int sq = s0; sq < s1; ++sq) {
    const int64_t c = (int64_t)p.Hkv * pre_seq_chunks(p, seq_view(p, sq));
    pos += c;
    cnt += c > 0;
  }
  s_pos[tid] = pos;
  s_cnt[tid] = cnt;
  __syncthreads();
  for (int o = 1; o < kPlanThreads; o <<= 1) {  // inclusive scan over the threads' ranges
    const int64_t a = tid >= o ? s_pos[tid - o] : 0;
    const int b = tid >= o ? s_cnt[tid - o] : 0;
    __syncthreads();
    s_pos[tid] += a;
    s_cnt[tid] += b;
    __syncthreads();
  }
  const int64_t C = s_pos[kPlanThreads - 1];
  const int n_pre = s_cnt[kPlanThreads - 1];
  int64_t beg = s_pos[tid] - pos;
  int k = s_cnt[tid] - cnt;
  for (int sq = s0; sq < s1; ++sq) {
    const int64_t c = (int64_t)p.Hkv * pre_seq_chunks(p, seq_view(p, sq));
    if (c > 0) {
      p.ws_pre_list[k] = sq;
      p.ws_pre_beg[k] = beg;
      if (k < kPlanLdsSeqs) s_beg[k] = beg;
      beg += c;
      ++k;
    }
  }
  const int NUa = C > 0 ? (int)active_units(C, p.NUP) : 0;
  if (tid == 0) {
    p.ws_plan_hdr[0] = C;
    p.ws_plan_hdr[1] = NUa;
    p.ws_plan_hdr[2] = n_pre;
    p.ws_pre_beg[n_pre] = C;
    if (n_pre <= kPlanLdsSeqs) s_beg[n_pre] = C;
  }
  __syncthreads();  // the list and starts are visible to the whole workgroup
  const int64_t* beg_tab = n_pre <= kPlanLdsSeqs ? s_beg : p.ws_pre_beg;
  const int q8 = NUa / 8, r8 = NUa % 8;
  for (int b = tid; b < p.NUP; b += kPlanThreads) {
    // workgroup b's unit, as prefill_units deals them: XCD by XCD (b % 8), then b / 8
    const int xcd = b % 8, jj = b / 8;
    int32_t* d = p.ws_pre_unit + (int64_t)b * kPreRec;
    if (NUa == 0 || jj >= q8 + (xcd < r8 ? 1 : 0)) {
      d[0] = -1;  // idle, rewritten on every call
      continue;
    }
    const int u = xcd * q8 + min(xcd, r8) + jj;
    const int64_t x0 = u * C / NUa;
    int lo = 0, hi = n_pre - 1;  // last sequence starting at or before x0
    while (lo < hi) {
      const int mid = (lo + hi + 1) / 2;
      if (beg_tab[mid] <= x0)
        lo = mid;
      else
        hi = mid - 1;
    }
    const int seq = p.ws_pre_list[lo];
    const SeqView sv = seq_view(p, seq);
    const int R = sv.q_len * p.G;
    const int64_t per_kvh = (beg_tab[lo + 1] - beg_tab[lo]) / p.Hkv;
    const int64_t off = x0 - beg_tab[lo];
    const int kvh = (int)(off / per_kvh);
    int64_t rem = off % per_kvh;
    int t = 0;
    for (int n_t = pre_tile_chunks(p, sv, R, 0); rem >= kTileCost + n_t; n_t = pre_tile_chunks(p, sv, R, t)) {
      rem -= kTileCost + n_t;
      ++t;
    }
    const int64_t x1 = (u + 1) * C / NUa;
    d[1] = lo;
    d[2] = kvh;
    d[3] = t;
    d[4] = (int)rem;  // < kTileCost + chunks of one tile
    d[5] = seq;
    d[6] = sv.q_len;
    d[7] = sv.kv_total;
    *(int64_t*)(d + 8) = sv.qs;
    *(int64_t*)(d + 10) = sv.ctx;
    *(int64_t*)(d + 12) = x0;
    *(int64_t*)(d + 14) = x1;
    d[0] = u;
  }
}

// Stream-K over the prefill-class work: a flat space of (sequence, kv head, tile, chunk),
// sequence-major, in which tile t of (seq, kvh) occupies kTileCost + pre_tile_chunks
// positions (its fixed cost counted like chunk steps). The launch has one workgroup per
// resident slot (NUP, a multiple of 8); NUa = min(NUP, ceil(C / kMinUnitChunks)) of them are
// work units, unit u taking positions [u C / NUa, (u + 1) C / NUa), so every unit gets the
// same amount of work whatever the mix of prompt lengths. A tile split between units leaves
// partials: unit u keeps the piece of its first non-empty tile in slot 2u and of its last in
// slot 2u + 1 (tiles in between are whole and written out), and the unit holding a split
// tile's first piece records its merge job (in the record of its workgroup). Workgroups are
// dealt to the 8 XCDs round-robin, so the units are numbered XCD by XCD: the units of one
// XCD are contiguous in the flat space and read the same sequence's K/V through that
// XCD's L2.
// The units' walk over the flat space (shared by both prefill kernels): `tile(sv, R, seq,
// kvh, t, c_lo, c_hi, partial, slot, rest, total)` computes chunks [c_lo, c_hi) of tile t.
template <class TileFn>
__device__ __forceinline__ void prefill_units(const PAParams& p, TileFn&& tile) {
  // this workgroup's record (one 64-byte load) and the plan header, issued together and
  // ahead of any store
  static_assert(kPreRec == 16, "one i32x16 per record");
  const i32x16 rec = *(const i32x16*)(p.ws_pre_unit + (int64_t)blockIdx.x * kPreRec);
  const int64_t hdr_c = p.ws_plan_hdr[0], hdr_nua = p.ws_plan_hdr[1], hdr_npre = p.ws_plan_hdr[2];
  int32_t* job = p.ws_job + (int64_t)(kMaxDecodeWaves + blockIdx.x) * kJobInts;
  if (threadIdx.x == 0) job[0] = kJobNone;
  const int u = uni(rec[0]);
  if (u < 0) return;  // idle workgroup (workgroup-uniform)
  const int64_t C = uni64(hdr_c);
  const int NUa = (int)uni64(hdr_nua);
  const int n_pre = (int)uni64(hdr_npre);
  const auto pair = [&](int i) { return (int64_t)(((uint64_t)(uint32_t)rec[i + 1] << 32) | (uint32_t)rec[i]); };
  int k = uni(rec[1]);
  int kvh = uni(rec[2]);
  int t = uni(rec[3]);
  int64_t rem = uni(rec[4]);
  int seq = uni(rec[5]);
  SeqView sv;
  sv.q_len = uni(rec[6]);
  sv.kv_total = uni(rec[7]);
  sv.qs = uni64(pair(8));
  sv.ctx = uni64(pair(10));
  int64_t x = uni64(pair(12));
  const int64_t x1 = uni64(pair(14));
  const int total = (int)(x1 - x);  // positions of this unit: < 2^31 (C / NUa + 1)
  int R = sv.q_len * p.G;
  int tiles = (R + p.PR - 1) / p.PR;
  int n_t = pre_tile_chunks(p, sv, R, t);
  // a: this unit's first position within the tile. Positions a .. b - 1 of a tile are its
  // chunks max(0, a - kTileCost) .. max(0, b - kTileCost) - 1, the same map at both ends
  // of every unit, so the pieces partition the chunks; a range inside the virtual prefix is
  // empty and skipped.
  int64_t a = rem;
  bool first = true;
  for (;;) {
    const int64_t tw = kTileCost + n_t;
    const int64_t b = min(tw, a + (x1 - x));
    const int c_lo = (int)max((int64_t)0, a - kTileCost), c_hi = (int)max((int64_t)0, b - kTileCost);
    if (c_hi > c_lo) {
      const bool whole = c_lo == 0 && c_hi == n_t;
      const int64_t slot = 2 * (int64_t)u + (first ? 0 : 1);
      const int rest = (int)(x1 - (x + (b - a)));
      tile(sv, R, seq, kvh, t, c_lo, c_hi, !whole, slot, rest, total);
      if (threadIdx.x == 0 && c_lo == 0 && c_hi < n_t) {
        // the tile continues in units u + 1 .. u1, each holding it as its first piece
        const int64_t x_last = x + (tw - a) - 1;
        const int64_t u1 = ((x_last + 1) * NUa - 1) / C;
        write_job(job, kJobPrefill, (int)(u1 - u + 1), slot, 2 * (int64_t)u, 2, sv.qs, R, t * p.PR, kvh);
      }
      first = false;
    }
    x += b - a;
    if (x >= x1) break;
    a = 0;
    if (++t == tiles) {
      t = 0;
      if (++kvh == p.Hkv) {
        kvh = 0;
        if (++k >= n_pre) return;  // cannot happen: the flat space ends with the last sequence
        seq = uni(p.ws_pre_list[k]);
        sv = seq_view_uniform(p, seq);
        R = sv.q_len * p.G;
        tiles = (R + p.PR - 1) / p.PR;
      }
    }
    n_t = pre_tile_chunks(p, sv, R, t);
  }
}

// 4-wave workgroups of 64 NT rows (PAParams::PR), 2 per CU.
template <class E, int D, bool KV8>
__global__ __launch_bounds__(256, 2) void pa_prefill_kernel(PAParams p) {
  using L = PrefillLds<D>;
  __shared__ __attribute__((aligned(1024))) char lds[(KV8 ? 2 : L::kStages) * L::kStageBytes];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  prefill_units(p, [&](const SeqView& sv, int R, int seq, int kvh, int t, int c_lo, int c_hi, bool partial,
                       int64_t slot, int rest, int total) {
    if constexpr (KV8)
      prefill_tile_kv8<E, D>(lds, p, sv, R, seq, kvh, t, c_lo, c_hi, w, partial, slot, rest, total);
    else
      prefill_tile<E, D>(lds, p, sv, R, seq, kvh, t, c_lo, c_hi, w, partial, slot, rest, total);
  });
}

// ---------------------------------------------------------------------------------------
// Workgroups of `kernel` (block_threads each) the current device holds at once, CUs x per
// CU, cached per device and kernel; per_cu_out, if given, receives the per-CU count (waves
// per SIMD for 4-wave workgroups).
static int resident_blocks(const void* kernel, int block_threads = 256, int* per_cu_out = nullptr) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    if (per_cu_out) *per_cu_out = 1;
    return 256;
  }
  struct Entry {
    int dev;
    const void* kernel;
    int blocks, per_cu;
  };
  static thread_local Entry cache[16];
  static thread_local int cache_n = 0;
  for (int i = 0; i < cache_n; ++i)
    if (cache[i].dev == dev && cache[i].kernel == kernel) {
      if (per_cu_out) *per_cu_out = cache[i].per_cu;
      return cache[i].blocks;
    }
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block_threads, 0) != hipSuccess || per_cu <= 0)
    per_cu = 1;
  const int blocks = cus * per_cu;
  if (cache_n < 16) cache[cache_n++] = Entry{dev, kernel, blocks, per_cu};
  if (per_cu_out) *per_cu_out = per_cu;
  return blocks;
}

template <class E, int D, int NT, bool KV8, int NX = 1>
static int launch_decode_nt(PAParams& p, hipStream_t s) {
  const void* k = (const void*)&pa_decode_kernel<E, D, NT, KV8, NX>;
  const int plan_wgs = p.PLAN ? 1 : 0;  // workgroup 0 plans the prefill launch
  int per_cu = 1;
  const int resident = resident_blocks(k, 256, &per_cu);
  int waves = (resident - plan_wgs) * kWavesPerWG;
  if (waves > kMaxDecodeWaves) waves = kMaxDecodeWaves;
  int64_t units = waves / p.HGW;
  // 16-bit caches: half the resident waves. Each split segment leaves one fp32 partial per
  // unit (RS x D per wave), written here and read back by the merge; with half the units the
  // pieces are twice as long and the partial traffic halves, while the waves left (one per
  // SIMD of the two the D = 128 kernels fit, two of four at D = 64) still keep HBM busy
  // (measured HBM-cold, C2 5.46 -> 5.62 TB/s, C5 3.88 -> 4.20 TB/s; a quarter of the waves
  // loses 10-20%). E4M3 caches convert every element before the MFMA and keep
  // two thirds (2 of the 3 waves per SIMD the kernel fits): with three, the last-dispatched
  // workgroups of each CU finish up to 50% later than the first (HBM-cold C2 2%, C4 4% slower
  // than with two), while half the waves is 5% slower. An E4M3 kernel that fits two waves per
  // SIMD (the two-tile verify rows, the 32-row cascade tiles) keeps both: C5 over E4M3 decode
  // 64.8 -> 58.1 us HBM-cold against two thirds of them. A kernel that fits one wave per SIMD
  // (the 64-row cascade tiles, 48 or 64 verify rows) keeps them all: halving would idle half
  // the CUs.
  if (per_cu >= 2) {
    if (!KV8)
      units /= 2;
    else if (per_cu >= 3)
      units = units * 2 / 3;
  }
  if (p.CASC && units > kMaxCascadeWaves / p.HGW) units = kMaxCascadeWaves / p.HGW;  // prefix partial slots
  // No launch takes more units than its static shape can give work (kMinUnitChunks chunks of
  // at most W BS keys per segment): a small batch dispatches a grid of its own size, and the
  // merge launch scans that many job records, not one per wave the device could hold.
  const int64_t seg_chunks = ((int64_t)p.W * p.BS + kChunk - 1) / kChunk;
  const int64_t max_chunks = (int64_t)(p.Hkv / p.HGW) * p.B * (seg_chunks > 1 ? seg_chunks : 1);
  const int64_t cap = (max_chunks + kMinUnitChunks - 1) / kMinUnitChunks;
  if (units > cap) units = cap;
  if (units < 1) units = 1;
  p.NU = (int32_t)units;
  const int wgs = (p.NU * p.HGW + kWavesPerWG - 1) / kWavesPerWG;
  // units whose last workgroup is dispatched before every CU holds one (unit u's waves are
  // u HGW .. (u + 1) HGW - 1, behind the planning workgroup)
  const int cus = per_cu > 0 ? resident / per_cu : resident;
  const int64_t r1 = (int64_t)kWavesPerWG * (cus - plan_wgs) / p.HGW;
  p.R1 = (int32_t)(wgs + plan_wgs > cus ? (r1 < 0 ? 0 : (r1 < units ? r1 : units)) : units);
  hipLaunchKernelGGL((pa_decode_kernel<E, D, NT, KV8, NX>), dim3(wgs + plan_wgs), dim3(256), 0, s, p);
  return (int)hipGetLastError();
}

template <class E, int D, bool KV8>
static int launch_mfma_typed(PAParams& p, const Plan& plan, int32_t max_q, hipStream_t s, LaunchLog& log) {
  int err = 0;
  if (plan.short_decode) {
    hipLaunchKernelGGL((pa_decode_short_kernel<E, D, KV8>), dim3(p.Hkv, p.B), dim3(256), 0, s, p);
    if ((err = (int)hipGetLastError())) return err;
    log.after_launch(1, s);
    return 0;
  }
  p.PLAN = plan.launch_prefill ? 1 : 0;
  p.CASC = plan.cascade ? 1 : 0;
  if (plan.cascade) {
    hipLaunchKernelGGL(pa_share_kernel, dim3(1), dim3(kPlanThreads), 0, s, p);
    if ((err = (int)hipGetLastError())) return err;
    log.after_launch(5, s);
  }
  if (plan.launch_prefill) {
    // the unit count is fixed before the decode launch: both kernels write merge jobs. Units x
    // 2 partial slots x tile rows stay within the workspace's kMaxPrefillUnits x 2 x kPrefillRows.
    p.PR = kWavesPerWG * 16 * prefill_nt<KV8>();
    int units = resident_blocks((const void*)&pa_prefill_kernel<E, D, KV8>);
    const int cap = kMaxPrefillUnits * kPrefillRows / p.PR;
    if (units > cap) units = cap;
    p.NUP = units / 8 * 8;
    if (p.NUP < 8) p.NUP = 8;
  }
  switch (plan.NT) {
    case 1:
      if constexpr (!KV8) {
        if (plan.cascade && p.XR == 64) {  // 64-row prefix groups (16-bit caches)
          err = launch_decode_nt<E, D, 1, KV8, 4>(p, s);
          break;
        }
      } else {
        if (plan.cascade && p.XR == 32) {  // 32-row prefix groups (E4M3 caches)
          err = launch_decode_nt<E, D, 1, KV8, 2>(p, s);
          break;
        }
      }
      err = launch_decode_nt<E, D, 1, KV8>(p, s);
      break;
    case 2: err = launch_decode_nt<E, D, 2, KV8>(p, s); break;
    case 3: err = launch_decode_nt<E, D, 3, KV8>(p, s); break;
    case 4: err = launch_decode_nt<E, D, 4, KV8>(p, s); break;
    default: return (int)hipErrorInvalidValue;
  }
  if (err) return err;
  log.after_launch(1, s);
  if (plan.launch_prefill) {
    hipLaunchKernelGGL((pa_prefill_kernel<E, D, KV8>), dim3(p.NUP), dim3(256), 0, s, p);
    if ((err = (int)hipGetLastError())) return err;
    log.after_launch(2, s);
  }
  const int mr = plan.launch_prefill ? merge_rows_decode<D, true>() : merge_rows_decode<D, false>();
  const int cd = (p.HGW * p.RS + mr - 1) / mr;
  const int nseg = plan.cascade ? p.B * (p.Hkv / p.HGW) : 0;  // cascade records
  const dim3 mg((p.NU > nseg ? p.NU : nseg) * cd + p.NUP * (p.PR / merge_rows<D, 4>()));
  // the partials' layout: tile blocks where the decode kernel wrote them so (write_rows<...,
  // KV8 && NT > 1>: multi-tile rows over E4M3 caches), whole rows otherwise
  if (plan.launch_prefill)
    hipLaunchKernelGGL((pa_merge_kernel<E, D, true, false>), mg, dim3(256), 0, s, p);
  else if (KV8 && plan.NT > 1)
    hipLaunchKernelGGL((pa_merge_kernel<E, D, false, true>), mg, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((pa_merge_kernel<E, D, false, false>), mg, dim3(256), 0, s, p);
  if ((err = (int)hipGetLastError())) return err;
  log.after_launch(3, s);
  return 0;
}

template <bool KV8>
static int launch_mfma_kv(PAParams& p, const Plan& plan, int32_t D, int32_t dtype, int32_t max_q, hipStream_t s,
                          LaunchLog& log) {
  const bool bf = dtype == 2;
  if (D == 128)
    return bf ? launch_mfma_typed<BF16, 128, KV8>(p, plan, max_q, s, log)
              : launch_mfma_typed<F16, 128, KV8>(p, plan, max_q, s, log);
  if (D == 64)
    return bf ? launch_mfma_typed<BF16, 64, KV8>(p, plan, max_q, s, log)
              : launch_mfma_typed<F16, 64, KV8>(p, plan, max_q, s, log);
  return (int)hipErrorInvalidValue;
}

int launch_paged_attention_mfma(PAParams& p, const Plan& plan, int32_t D, int32_t dtype, bool kv8, int32_t max_q,
                                hipStream_t s, LaunchLog& log) {
  return kv8 ? launch_mfma_kv<true>(p, plan, D, dtype, max_q, s, log)
             : launch_mfma_kv<false>(p, plan, D, dtype, max_q, s, log);
}

}  // namespace kvh
