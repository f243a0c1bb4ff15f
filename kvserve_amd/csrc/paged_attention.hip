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
//  * Decode class (q_len <= QS): a workgroup of 4 waves owns one split-K partition of
//    PS tokens; waves take interleaved chunks, merge in LDS, and either write the final
//    row (single-partition sequences) or an unnormalised partial that the reduce kernel
//    merges with a log-sum-exp (multi-partition sequences).
//  * Prefill class (q_len > QS): a workgroup of 4 waves owns 4 x 32 query rows; each
//    wave streams every key its rows can see (causal limit of its last row).
// Grids depend only on static shapes (block-table width, max_query_len), never on
// per-step lengths, so every launch is HIP-graph capturable.
#include "kvh_device.h"
#include "kvh_internal.h"

namespace kvh {

constexpr int kChunk = 32;   // tokens per wave iteration
constexpr int kWavesPerWG = 4;
constexpr int kPrefillNQT = 2;  // 16-row tiles per prefill wave

#ifndef KVH_DECODE_PIPE
#define KVH_DECODE_PIPE false
#endif
#ifndef KVH_PREFILL_PIPE
#define KVH_PREFILL_PIPE false
#endif

// ---------------------------------------------------------------------------------------
// Per-lane registers of one 32-token chunk of one kv head.
template <int D>
struct KVChunk {
  static constexpr int KC = D / 32;  // 8-element K vectors per 16-token tile per lane
  static constexpr int VW = D / 16;  // V elements per lane per token (d = VW*n .. VW*n+VW-1)
  static constexpr int VD = VW / 2;  // ... as dwords
  u32x4 k[2][KC];
  uint32_t v[8][VD];  // token t8 = 4*tile + e  <->  chunk token 16*tile + 4j + e
};

template <int D>
__device__ __forceinline__ void load_chunk(KVChunk<D>& c, const PAParams& p, const int64_t* btrow,
                                           int kvh, int tok0, int tok_end, bool tile_ok[2]) {
  const int lane = threadIdx.x & 63;
  const int j = lane >> 4, n = lane & 15;
  const uint16_t* kc = (const uint16_t*)p.kc;
  const uint16_t* vc = (const uint16_t*)p.vc;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int tt = tok0 + 16 * t;  // first token of the tile (wave-uniform)
    bool ok = tt < tok_end;
    int64_t blk = 0;
    if (ok) {
      blk = btrow[tt / p.BS];
      ok = blk >= 0 && blk < p.num_blocks;
    }
    tile_ok[t] = ok;
    if (ok) {
      const int slot0 = tt % p.BS;
      const uint16_t* kp = kc + blk * p.k_sb + (int64_t)(slot0 + n) * p.k_ss + kvh * p.k_sh + (D / 4) * j;
#pragma unroll
      for (int cc = 0; cc < KVChunk<D>::KC; ++cc) c.k[t][cc] = *(const u32x4*)(kp + 8 * cc);
      const uint16_t* vp = vc + blk * p.v_sb + (int64_t)(slot0 + 4 * j) * p.v_ss + kvh * p.v_sh + KVChunk<D>::VW * n;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if constexpr (KVChunk<D>::VD == 4) {
          u32x4 x = *(const u32x4*)(vp + e * p.v_ss);
          c.v[4 * t + e][0] = x[0]; c.v[4 * t + e][1] = x[1]; c.v[4 * t + e][2] = x[2]; c.v[4 * t + e][3] = x[3];
        } else {
          u32x2 x = *(const u32x2*)(vp + e * p.v_ss);
          c.v[4 * t + e][0] = x[0]; c.v[4 * t + e][1] = x[1];
        }
      }
    } else {
#pragma unroll
      for (int cc = 0; cc < KVChunk<D>::KC; ++cc) c.k[t][cc] = u32x4{0, 0, 0, 0};
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int x = 0; x < KVChunk<D>::VD; ++x) c.v[4 * t + e][x] = 0;
    }
  }
}

// Online-softmax state of one wave over NT tiles of 16 query rows.
template <int D, int NT>
struct WaveState {
  u32x4 q[NT][D / 32];     // B operand of S^T = K Q^T
  f32x4 acc[NT][D / 16];   // O^T accumulators: column = row, rows 4j+e <-> d = VW*(4j+e) + i
  float m[NT], l[NT];      // m: running max (exp2 domain, -inf when empty); l: lane-partial sum
  int limit[NT];           // keys visible to this lane's row (0 for padding rows)
};

// Q rows of tile t: global row r = row0 + 16t + n, valid when r < R.
template <int D, int NT>
__device__ __forceinline__ void load_q(WaveState<D, NT>& s, const PAParams& p, int64_t q_start, int R,
                                       int row0, int kvh, int64_t ctx, int64_t kv_total) {
  const int lane = threadIdx.x & 63;
  const int j = lane >> 4, n = lane & 15;
  const uint16_t* q = (const uint16_t*)p.q;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int r = row0 + 16 * t + n;
    s.m[t] = -INFINITY;
    s.l[t] = 0.f;
#pragma unroll
    for (int i = 0; i < D / 16; ++i) s.acc[t][i] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (r < R) {
      const int qi = r / p.G, g = r % p.G;
      const uint16_t* qp = q + (q_start + qi) * p.q_ts + (int64_t)(kvh * p.G + g) * p.q_hs + (D / 4) * j;
#pragma unroll
      for (int c = 0; c < D / 32; ++c) s.q[t][c] = *(const u32x4*)(qp + 8 * c);
      s.limit[t] = (int)clamp64(ctx + qi + 1, 0, kv_total);
    } else {
#pragma unroll
      for (int c = 0; c < D / 32; ++c) s.q[t][c] = u32x4{0, 0, 0, 0};
      s.limit[t] = 0;
    }
  }
}

// One 32-token chunk: S^T, mask, online softmax, O^T += V^T P^T.
// MASKED = false is only used when every token of the chunk is visible to every valid row.
template <class E, int D, int NT, bool MASKED>
__device__ __forceinline__ void compute_chunk(WaveState<D, NT>& s, KVChunk<D>& c, const PAParams& p,
                                              int tok0, int data_end, const bool tile_ok[2]) {
  const int lane = threadIdx.x & 63;
  const int j = lane >> 4;
  constexpr int VW = KVChunk<D>::VW;

  // Slots at or past seq_len may hold any bits (stale or never written cache slots);
  // P is 0 there but 0 * NaN is NaN, so V is zeroed like the reference's masked loads
  // (other=0.0). Tokens below seq_len are this step's or cached K/V: finite.
  if (MASKED) {
#pragma unroll
    for (int t8 = 0; t8 < 8; ++t8) {
      const int tok = tok0 + 16 * (t8 >> 2) + 4 * j + (t8 & 3);
      if (!(tile_ok[t8 >> 2] && tok < data_end))
#pragma unroll
        for (int x = 0; x < KVChunk<D>::VD; ++x) c.v[t8][x] = 0;
    }
  }

  // Scores and softmax for every row tile first (K dies here), then the P.V MFMAs with
  // each V^T operand built right before use so only one is live at a time.
  u32x4 pt[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    f32x4 st[2];
#pragma unroll
    for (int tile = 0; tile < 2; ++tile) {
      f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int cc = 0; cc < D / 32; ++cc) a = E::mfma(c.k[tile][cc], s.q[t][cc], a);
      st[tile] = a;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int tile = 0; tile < 2; ++tile) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float x = st[tile][e] * p.qk_scale;
        if (MASKED) {
          const int tok = tok0 + 16 * tile + 4 * j + e;
          if (!(tile_ok[tile] && tok < s.limit[t])) x = -INFINITY;
        }
        st[tile][e] = x;
        mx = fmaxf(mx, x);
      }
    }
    mx = max_over_groups(mx);
    const float m_new = fmaxf(s.m[t], mx);
    const float m_safe = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = fast_exp2(s.m[t] - m_safe);
    s.m[t] = m_new;
    float pv[8], psum = 0.f;
#pragma unroll
    for (int tile = 0; tile < 2; ++tile)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x = fast_exp2(st[tile][e] - m_safe);
        pv[4 * tile + e] = x;
        psum += x;
      }
    s.l[t] = s.l[t] * alpha + psum;
#pragma unroll
    for (int w = 0; w < 4; ++w) pt[t][w] = E::pack2(pv[2 * w], pv[2 * w + 1]);
#pragma unroll
    for (int i = 0; i < VW; ++i) s.acc[t][i] *= alpha;
  }

  // V^T A operand i: element 4*tile + e of lane (j, m) = V[token 16*tile + 4j + e][VW*m + i]
#pragma unroll
  for (int i = 0; i < VW; ++i) {
    u32x4 va;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t a = c.v[2 * w][i >> 1], b = c.v[2 * w + 1][i >> 1];
      va[w] = (i & 1) ? pick_halves<1>(a, b) : pick_halves<0>(a, b);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) s.acc[t][i] = E::mfma(va, pt[t], s.acc[t][i]);
  }
}


// ---------------------------------------------------------------------------------------
// Chunk loop of one wave over tokens tok_begin, tok_begin + stride, ... < tok_hi.
// PIPE: keep the next chunk's loads in flight while the current one is computed (two
// register buffers, unrolled so no buffer is ever copied: a copy would wait on its loads);
// otherwise one buffer and latency is hidden by the other waves on the SIMD.
template <class E, int D, int NT, bool PIPE>
__device__ __forceinline__ void run_chunks(WaveState<D, NT>& s, const PAParams& p, const int64_t* btrow, int kvh,
                                           int tok_begin, int stride, int tok_hi, int vis_all, int data_end) {
  int tok0 = tok_begin;
  if (tok0 >= tok_hi) return;
  if constexpr (!PIPE) {
    for (; tok0 < tok_hi; tok0 += stride) {
      KVChunk<D> ca;
      bool oka[2];
      load_chunk<D>(ca, p, btrow, kvh, tok0, tok_hi, oka);
      if (tok0 + kChunk <= vis_all && oka[0] && oka[1])
        compute_chunk<E, D, NT, false>(s, ca, p, tok0, data_end, oka);
      else
        compute_chunk<E, D, NT, true>(s, ca, p, tok0, data_end, oka);
    }
  } else {
    KVChunk<D> ca, cb;
    bool oka[2], okb[2];
    load_chunk<D>(ca, p, btrow, kvh, tok0, tok_hi, oka);
    while (true) {
      int nxt = tok0 + stride;
      if (nxt < tok_hi) load_chunk<D>(cb, p, btrow, kvh, nxt, tok_hi, okb);
      if (tok0 + kChunk <= vis_all && oka[0] && oka[1])
        compute_chunk<E, D, NT, false>(s, ca, p, tok0, data_end, oka);
      else
        compute_chunk<E, D, NT, true>(s, ca, p, tok0, data_end, oka);
      tok0 = nxt;
      if (tok0 >= tok_hi) break;
      nxt = tok0 + stride;
      if (nxt < tok_hi) load_chunk<D>(ca, p, btrow, kvh, nxt, tok_hi, oka);
      if (tok0 + kChunk <= vis_all && okb[0] && okb[1])
        compute_chunk<E, D, NT, false>(s, cb, p, tok0, data_end, okb);
      else
        compute_chunk<E, D, NT, true>(s, cb, p, tok0, data_end, okb);
      tok0 = nxt;
      if (tok0 >= tok_hi) break;
    }
  }
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
  int64_t qs;      // first flat token of the sequence
  int q_len;
  int64_t ctx;     // seq_len - q_len (cached tokens before this step)
  int kv_total;    // keys present: seq_len clamped to the block-table capacity
};

__device__ __forceinline__ SeqView seq_view(const PAParams& p, int seq) {
  SeqView v;
  v.qs = clamp64(p.qsl[seq], 0, p.T);
  const int64_t qe = clamp64(p.qsl[seq + 1], v.qs, p.T);
  v.q_len = (int)(qe - v.qs);
  const int64_t sl = p.seq_lens[seq];
  v.ctx = sl - v.q_len;
  v.kv_total = (int)clamp64(sl, 0, (int64_t)p.W * p.BS);
  return v;
}

// ---------------------------------------------------------------------------------------
// Decode class: grid (P, Hkv, B), 4 waves per workgroup = one split-K partition.
template <class E, int D, int NT>
__global__ __launch_bounds__(256) void pa_decode_kernel(PAParams p) {
  constexpr int VW = D / 16;
  const int part = blockIdx.x, kvh = blockIdx.y, seq = blockIdx.z;
  const int lane = threadIdx.x & 63;
  const int j = lane >> 4, n = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  const SeqView sv = seq_view(p, seq);
  if (sv.q_len == 0 || sv.q_len > p.QS) return;
  const int n_parts = max(1, (sv.kv_total + p.PS - 1) / p.PS);
  if (part >= n_parts) return;
  const int tok_lo = part * p.PS;
  const int tok_hi = min(tok_lo + p.PS, sv.kv_total);
  const int R = sv.q_len * p.G;
  const int vis_all = (int)clamp64(sv.ctx + 1, 0, sv.kv_total);

  WaveState<D, NT> s;
  load_q<D, NT>(s, p, sv.qs, R, 0, kvh, sv.ctx, sv.kv_total);
  const int64_t* btrow = p.bt + (int64_t)seq * p.bt_rs;
  run_chunks<E, D, NT, KVH_DECODE_PIPE>(s, p, btrow, kvh, tok_lo + kChunk * w, kChunk * kWavesPerWG, tok_hi, vis_all,
                       sv.kv_total);

  // Merge the four waves' states through LDS, one 16-row tile at a time.
  __shared__ float s_m[kWavesPerWG][16], s_l[kWavesPerWG][16];
  __shared__ __attribute__((aligned(16))) float s_acc[kWavesPerWG][16][D + 4];
  const int row = threadIdx.x >> 4, seg = threadIdx.x & 15;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const float lt = sum_over_groups(s.l[t]);
    if (t > 0) __syncthreads();
    if (j == 0) {
      s_m[w][n] = s.m[t];
      s_l[w][n] = lt;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int i = 0; i < VW; ++i) s_acc[w][n][VW * (4 * j + e) + i] = s.acc[t][i][e];
    __syncthreads();
    const int r = 16 * t + row;
    if (r < R) {
      float mw[kWavesPerWG], M = -INFINITY;
#pragma unroll
      for (int x = 0; x < kWavesPerWG; ++x) {
        mw[x] = s_m[x][row];
        M = fmaxf(M, mw[x]);
      }
      const float msafe = M == -INFINITY ? 0.f : M;
      float L = 0.f, f[kWavesPerWG];
#pragma unroll
      for (int x = 0; x < kWavesPerWG; ++x) {
        f[x] = fast_exp2(mw[x] - msafe);
        L += f[x] * s_l[x][row];
      }
      float o[VW];
#pragma unroll
      for (int i = 0; i < VW; ++i) {
        float a = 0.f;
#pragma unroll
        for (int x = 0; x < kWavesPerWG; ++x) a += f[x] * s_acc[x][row][VW * seg + i];
        o[i] = a;
      }
      const int qi = r / p.G, g = r % p.G;
      const int64_t tok = sv.qs + qi;
      const int head = kvh * p.G + g;
      if (n_parts == 1) {
        const float inv = 1.f / (L == 0.f ? 1.f : L);
        uint16_t* dst = (uint16_t*)p.out + tok * p.o_ts + (int64_t)head * p.o_hs + VW * seg;
        store_row_vec<E, VW>(dst, o, inv);
      } else {
        const int64_t idx = (tok * p.H + head) * p.P + part;
        float* dst = p.ws_acc + idx * D + VW * seg;
#pragma unroll
        for (int i = 0; i < VW; i += 4) *(f32x4*)(dst + i) = f32x4{o[i], o[i + 1], o[i + 2], o[i + 3]};
        if (seg == 0) {
          p.ws_ml[idx * 2] = M;
          p.ws_ml[idx * 2 + 1] = L;
        }
      }
    }
  }
}

// Log-sum-exp merge of the partitions of multi-partition decode-class sequences.
// Grid (Hkv, B); each thread owns 4 consecutive output elements of one row.
template <class E, int D>
__global__ __launch_bounds__(256) void pa_reduce_kernel(PAParams p) {
  constexpr int TPR = D / 4;
  constexpr int RPP = 256 / TPR;
  const int kvh = blockIdx.x, seq = blockIdx.y;
  const SeqView sv = seq_view(p, seq);
  if (sv.q_len == 0 || sv.q_len > p.QS) return;
  const int n_parts = max(1, (sv.kv_total + p.PS - 1) / p.PS);
  if (n_parts == 1) return;
  const int R = sv.q_len * p.G;
  const int sub = threadIdx.x / TPR, seg = threadIdx.x % TPR;
  for (int r = sub; r < R; r += RPP) {
    const int qi = r / p.G, g = r % p.G;
    const int64_t tok = sv.qs + qi;
    const int head = kvh * p.G + g;
    const int64_t base = (tok * p.H + head) * p.P;
    float M = -INFINITY;
    for (int x = 0; x < n_parts; ++x) M = fmaxf(M, p.ws_ml[(base + x) * 2]);
    const float msafe = M == -INFINITY ? 0.f : M;
    float L = 0.f;
    f32x4 o = {0.f, 0.f, 0.f, 0.f};
    for (int x = 0; x < n_parts; ++x) {
      const float f = fast_exp2(p.ws_ml[(base + x) * 2] - msafe);
      L += f * p.ws_ml[(base + x) * 2 + 1];
      o += f * *(const f32x4*)(p.ws_acc + (base + x) * D + 4 * seg);
    }
    const float inv = 1.f / (L == 0.f ? 1.f : L);
    uint16_t* dst = (uint16_t*)p.out + tok * p.o_ts + (int64_t)head * p.o_hs + 4 * seg;
    u32x2 v;
    v[0] = E::pack2(o[0] * inv, o[1] * inv);
    v[1] = E::pack2(o[2] * inv, o[3] * inv);
    *(u32x2*)dst = v;
  }
}

// ---------------------------------------------------------------------------------------
// Prefill class: grid (ceil(max_q * G / 128), Hkv, B); wave w owns rows
// (blockIdx.x * 4 + w) * 32 .. + 31 of its sequence's R = q_len * G rows.
template <class E, int D>
__global__ __launch_bounds__(256) void pa_prefill_kernel(PAParams p) {
  constexpr int NT = kPrefillNQT;
  constexpr int VW = D / 16;
  const int kvh = blockIdx.y, seq = blockIdx.z;
  const int lane = threadIdx.x & 63;
  const int j = lane >> 4, n = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  const SeqView sv = seq_view(p, seq);
  if (sv.q_len <= p.QS) return;
  const int R = sv.q_len * p.G;
  const int row0 = (blockIdx.x * kWavesPerWG + w) * (16 * NT);
  if (row0 >= R) return;
  const int last_row = min(row0 + 16 * NT - 1, R - 1);
  const int kv_lim = (int)clamp64(sv.ctx + last_row / p.G + 1, 0, sv.kv_total);
  const int vis_all = (int)clamp64(sv.ctx + row0 / p.G + 1, 0, sv.kv_total);

  WaveState<D, NT> s;
  load_q<D, NT>(s, p, sv.qs, R, row0, kvh, sv.ctx, sv.kv_total);
  const int64_t* btrow = p.bt + (int64_t)seq * p.bt_rs;
  run_chunks<E, D, NT, KVH_PREFILL_PIPE>(s, p, btrow, kvh, 0, kChunk, kv_lim, vis_all, sv.kv_total);

#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const float L = sum_over_groups(s.l[t]);
    const int r = row0 + 16 * t + n;
    if (r < R) {
      const float inv = 1.f / (L == 0.f ? 1.f : L);
      const int qi = r / p.G, g = r % p.G;
      uint16_t* base = (uint16_t*)p.out + (sv.qs + qi) * p.o_ts + (int64_t)(kvh * p.G + g) * p.o_hs;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float o[VW];
#pragma unroll
        for (int i = 0; i < VW; ++i) o[i] = s.acc[t][i][e];
        store_row_vec<E, VW>(base + VW * (4 * j + e), o, inv);
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
template <class E, int D, int NT>
static int launch_decode_nt(const PAParams& p, const Plan& plan, hipStream_t s) {
  dim3 grid(plan.P, p.Hkv, p.B);
  hipLaunchKernelGGL((pa_decode_kernel<E, D, NT>), grid, dim3(256), 0, s, p);
  return (int)hipGetLastError();
}

template <class E, int D>
static int launch_mfma_typed(const PAParams& p, const Plan& plan, hipStream_t s, LaunchLog& log) {
  int err = 0;
  switch (plan.NT) {
    case 1: err = launch_decode_nt<E, D, 1>(p, plan, s); break;
    case 2: err = launch_decode_nt<E, D, 2>(p, plan, s); break;
    case 3: err = launch_decode_nt<E, D, 3>(p, plan, s); break;
    case 4: err = launch_decode_nt<E, D, 4>(p, plan, s); break;
    default: return (int)hipErrorInvalidValue;
  }
  if (err) return err;
  log.after_launch(1, s);
  if (plan.launch_prefill) {
    dim3 grid(plan.pre_tiles, p.Hkv, p.B);
    hipLaunchKernelGGL((pa_prefill_kernel<E, D>), grid, dim3(256), 0, s, p);
    if ((err = (int)hipGetLastError())) return err;
    log.after_launch(2, s);
  }
  if (plan.P > 1) {
    dim3 grid(p.Hkv, p.B);
    hipLaunchKernelGGL((pa_reduce_kernel<E, D>), grid, dim3(256), 0, s, p);
    if ((err = (int)hipGetLastError())) return err;
    log.after_launch(3, s);
  }
  return 0;
}

int launch_paged_attention_mfma(const PAParams& p, const Plan& plan, int32_t D, int32_t dtype, hipStream_t s,
                                LaunchLog& log) {
  const bool bf = dtype == 2;
  if (D == 128) return bf ? launch_mfma_typed<BF16, 128>(p, plan, s, log) : launch_mfma_typed<F16, 128>(p, plan, s, log);
  if (D == 64) return bf ? launch_mfma_typed<BF16, 64>(p, plan, s, log) : launch_mfma_typed<F16, 64>(p, plan, s, log);
  return (int)hipErrorInvalidValue;
}

}  // namespace kvh
