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
//  * Decode class (q_len <= QS): stream-K. The launch keeps exactly as many waves as the GPU
//    holds resident; the decode work of all sequences is one flat space of 32-token chunks
//    that is cut into equal contiguous ranges, one per work unit of up to 4 waves (adjacent
//    kv heads of the same rows). No wave idles in a tail and each pays one start-up; a
//    sequence split between units leaves partials that the reduce kernel merges with a
//    log-sum-exp. The split is computed on the device from seq_lens (no host sync).
//  * Prefill class (q_len > QS): a workgroup of 4 waves owns 4 x 32 query rows; each
//    wave streams every key its rows can see (causal limit of its last row).
// Grids depend only on static shapes (block-table width, max_query_len), never on
// per-step lengths, so every launch is HIP-graph capturable.
#include "kvh_device.h"
#include "kvh_internal.h"

namespace kvh {

constexpr int kChunk = 32;  // tokens per wave iteration
constexpr int kWavesPerWG = 4;
constexpr int kPrefillNQT = 2;  // 16-row tiles per prefill wave

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

// Block id of `page` (wave-uniform), refreshing the window when the page leaves it.
__device__ __forceinline__ int page_block(PageWindow& pw, const PAParams& p, const int64_t* btrow, int page,
                                          int page_end) {
  if (page >= page_end) return -1;
  if (page - pw.page0 >= 64 || page < pw.page0) load_window(pw, p, btrow, page, page_end);
  return __builtin_amdgcn_readlane(pw.ids, page - pw.page0);
}

// Per-lane registers of one 32-token chunk of one kv head.
template <int D>
struct KRegs {
  u32x4 k[2][D / 32];  // tile t, 8-element vector c: token 16t + n, d = (D/4) j + 8c ..
};
template <int D>
struct VRegs {
  static constexpr int VW = D / 16;  // V elements per lane per token: d = VW n .. VW n + VW - 1
  uint32_t v[8][VW / 2];             // token t8 = 4 tile + e  <->  chunk token 16 tile + 4j + e
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
  uint32_t k;  // (n * k_ss + (D/4) j) * 2
  uint32_t v;  // (4j * v_ss + VW n) * 2
};

template <int D>
__device__ __forceinline__ LaneOffsets lane_offsets(const PAParams& p) {
  const int lane = threadIdx.x & 63;
  const int j = lane >> 4, n = lane & 15;
  LaneOffsets o;
  o.k = (uint32_t)(n * (uint32_t)p.k_ss + (D / 4) * j) * 2u;
  o.v = (uint32_t)(4 * j * (uint32_t)p.v_ss + (D / 16) * n) * 2u;
  return o;
}

// Loads are unconditional so the chunk loop stays straight-line (no waits merged at
// branch joins): an absent tile (blk < 0) reads block 0, which the API guarantees exists,
// and is masked out of the scores and zeroed out of V like any invalid key.
template <int D>
__device__ __forceinline__ void load_k(KRegs<D>& r, const PAParams& p, const ChunkRef& c, int kvh, uint32_t k_lane) {
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int64_t blk = c.blk[t] >= 0 ? c.blk[t] : 0;
    const int slot0 = (c.tok0 + 16 * t) % p.BS;
    const char* page = (const char*)p.kc + (blk * p.k_sb + (int64_t)kvh * p.k_sh + (int64_t)slot0 * p.k_ss) * 2;
#pragma unroll
    for (int cc = 0; cc < D / 32; ++cc) r.k[t][cc] = *(const u32x4*)(page + k_lane + 16 * cc);
  }
}

template <int D>
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
        const u32x4 x = *(const u32x4*)src;
        r.v[4 * t + e][0] = x[0];
        r.v[4 * t + e][1] = x[1];
        r.v[4 * t + e][2] = x[2];
        r.v[4 * t + e][3] = x[3];
      } else {
        const u32x2 x = *(const u32x2*)src;
        r.v[4 * t + e][0] = x[0];
        r.v[4 * t + e][1] = x[1];
      }
    }
  }
}

// Online-softmax state of one wave over NT tiles of 16 query rows.
template <int D, int NT>
struct WaveState {
  u32x4 q[NT][D / 32];    // B operand of S^T = K Q^T
  f32x4 acc[NT][D / 16];  // O^T accumulators: column = row, rows 4j+e <-> d = VW*(4j+e) + i
  float m[NT], l[NT];     // m: running max (exp2 domain, -inf when empty); l: lane-partial sum
  int limit[NT];          // keys visible to this lane's row (0 for padding rows)
};

// Q rows of tile t: global row r = row0 + 16t + n, valid when r < R.
template <int D, int NT>
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

// Scores of one chunk and the online-softmax update; returns the P^T B operands.
// MASKED = false only when every token of the chunk is visible to every valid row.
template <class E, int D, int NT, bool MASKED>
__device__ __forceinline__ void chunk_scores(WaveState<D, NT>& s, const KRegs<D>& kr, const PAParams& p,
                                             const ChunkRef& c, u32x4 pt[NT]) {
  const int j = (threadIdx.x & 63) >> 4;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    f32x4 st[2];
#pragma unroll
    for (int tile = 0; tile < 2; ++tile) {
      f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int cc = 0; cc < D / 32; ++cc) a = E::mfma(kr.k[tile][cc], s.q[t][cc], a);
      st[tile] = a;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int tile = 0; tile < 2; ++tile) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float x = st[tile][e] * p.qk_scale;
        if (MASKED) {
          const int tok = c.tok0 + 16 * tile + 4 * j + e;
          if (!(c.blk[tile] >= 0 && tok < s.limit[t])) x = -INFINITY;
        }
        st[tile][e] = x;
        mx = fmaxf(mx, x);
      }
    }
    mx = max_over_groups(mx);
    const float m_old = s.m[t];
    const float m_new = fmaxf(m_old, mx);
    const float m_safe = m_new == -INFINITY ? 0.f : m_new;
    // Rescale only when some row's max moved: alpha is exactly 1 otherwise.
    if (__builtin_amdgcn_ballot_w64(m_new > m_old)) {
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
        const float x = fast_exp2(st[tile][e] - m_safe);
        pv[4 * tile + e] = x;
        psum += x;
      }
    s.l[t] += psum;
#pragma unroll
    for (int w = 0; w < 4; ++w) pt[t][w] = E::pack2(pv[2 * w], pv[2 * w + 1]);
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

// Chunk loop of one wave over tokens tok_begin, tok_begin + stride, ... < tok_hi.
// The body is straight-line (masks always applied, loads unconditional) and the loads are
// pinned in the order K(c+1), V(c+1) with scheduling barriers, so each s_waitcnt waits for
// exactly the operand it guards while the other half of the next chunk stays in flight.
template <class E, int D, int NT>
__device__ __forceinline__ void run_chunks(WaveState<D, NT>& s, const PAParams& p, const int64_t* btrow, int kvh,
                                           int tok_begin, int stride, int tok_hi, int data_end) {
  if (tok_begin >= tok_hi) return;
  const int page_end = (tok_hi + p.BS - 1) / p.BS;
  const LaneOffsets lo = lane_offsets<D>(p);
  PageWindow pw;
  load_window(pw, p, btrow, tok_begin / p.BS, page_end);
  ChunkRef c = chunk_ref(pw, p, btrow, tok_begin, tok_hi, page_end);
  KRegs<D> kr;
  VRegs<D> vr;
  load_k<D>(kr, p, c, kvh, lo.k);
  __builtin_amdgcn_sched_barrier(0);
  load_v<D>(vr, p, c, kvh, lo.v);
  __builtin_amdgcn_sched_barrier(0);
  // Every iteration has a next chunk, so its loads are unconditional; the last chunk is
  // peeled off below the loop.
  while (c.tok0 + stride < tok_hi) {
    const ChunkRef cn = chunk_ref(pw, p, btrow, c.tok0 + stride, tok_hi, page_end);
    u32x4 pt[NT];
    chunk_scores<E, D, NT, true>(s, kr, p, c, pt);
    __builtin_amdgcn_sched_barrier(0);
    load_k<D>(kr, p, cn, kvh, lo.k);
    __builtin_amdgcn_sched_barrier(0);
    chunk_pv<E, D, NT, true>(s, vr, c, data_end, pt);
    __builtin_amdgcn_sched_barrier(0);
    load_v<D>(vr, p, cn, kvh, lo.v);
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

// Writes one wave's result for its 16-row tiles: the normalised output row, or (partial)
// the unnormalised acc, running max m and sum l of a piece of a split segment, at
// ws row index row_base + r. Lane (j, n) holds row row0 + 16t + n, d = VW (4j + e) + i.
template <class E, int D, int NT>
__device__ __forceinline__ void write_rows(const WaveState<D, NT>& s, const PAParams& p, const SeqView& sv, int R,
                                           int row0, int kvh, bool partial, int64_t row_base) {
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
      const float inv = 1.f / (L == 0.f ? 1.f : L);
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
      float* dst = p.ws_acc + idx * D;
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int i = 0; i < VW; i += 4)
          *(f32x4*)(dst + VW * (4 * j + e) + i) =
              f32x4{s.acc[t][i][e], s.acc[t][i + 1][e], s.acc[t][i + 2][e], s.acc[t][i + 3][e]};
      if (j == 0) {
        p.ws_ml[idx * 2] = s.m[t];
        p.ws_ml[idx * 2 + 1] = L;
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// Decode-class work as one flat chunk space (stream-K). A segment is (sequence, head
// group of HGW kv heads), ordered sequence-major; a decode-class sequence (0 < q_len <= QS)
// contributes c_s = max(1, ceil(kv_total / 32)) chunks to each of its NHG = Hkv / HGW
// segments, any other sequence none. C = NHG * sum_s c_s. Work unit u of NU' takes the
// chunks [u C / NU', (u + 1) C / NU'), NU' = min(NU, ceil(C / kMinUnitChunks)); the HGW
// waves of a unit take the HGW heads of each segment, so they stream adjacent slices of the
// same cache rows. A segment split between units leaves one partial per unit in slot
// (segment index + unit), which pa_reduce_kernel merges.
constexpr int kMinUnitChunks = 4;

__device__ __forceinline__ int seq_chunks(const PAParams& p, int s) {
  const SeqView v = seq_view(p, s);
  if (v.q_len == 0 || v.q_len > p.QS) return 0;
  return max(1, (v.kv_total + kChunk - 1) / kChunk);
}

// 64 sequences of the chunk prefix sum; lane l describes sequence blk0 + l.
struct SeqWindow {
  int blk0;   // first sequence of the window
  int base;   // chunks (per segment) of all sequences before blk0
  int c;      // this lane's sequence
  int excl;   // sequences blk0 .. blk0 + l - 1
  int total;  // the whole window
};

__device__ __forceinline__ void scan_window(SeqWindow& sw, const PAParams& p, int blk0, int base) {
  const int lane = threadIdx.x & 63;
  const int s = blk0 + lane;
  const int c = s < p.B ? seq_chunks(p, s) : 0;
  int incl = c;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o);
    if (lane >= o) incl += y;
  }
  sw.blk0 = blk0;
  sw.base = base;
  sw.c = c;
  sw.excl = incl - c;
  sw.total = __builtin_amdgcn_readlane(incl, 63);  // uniform (a shuffle result would not be)
}

__device__ __forceinline__ int64_t active_units(int64_t C, int NU) {
  const int64_t want = (C + kMinUnitChunks - 1) / kMinUnitChunks;
  return want < 1 ? 1 : (want < NU ? want : NU);
}

// Decode class: grid (NU * HGW / 4) workgroups of 4 waves; wave w of workgroup b is head
// w % HGW of unit (4 b + w) / HGW.
template <class E, int D, int NT>
__global__ __launch_bounds__(256) void pa_decode_kernel(PAParams p) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int gw = blockIdx.x * kWavesPerWG + wave;
  const int unit = gw / p.HGW, hw = gw % p.HGW;
  const int NHG = p.Hkv / p.HGW;

  // Prefix sums of chunks per segment over all sequences (every wave computes them; the
  // first wave also publishes them for the reduce kernel).
  int Cs = 0;
  for (int blk0 = 0; blk0 < p.B; blk0 += 64) {
    SeqWindow sw;
    scan_window(sw, p, blk0, Cs);
    if (gw == 0 && blk0 + lane < p.B) p.ws_cum[blk0 + lane] = Cs + sw.excl;
    Cs += sw.total;
  }
  if (gw == 0 && lane == 0) p.ws_cum[p.B] = Cs;
  const int64_t C = (int64_t)Cs * NHG;
  const int64_t NUa = active_units(C, p.NU);
  if (unit >= NUa) return;
  const int64_t a = unit * C / NUa, b = (unit + 1) * C / NUa;
  if (a >= b) return;

  // walk the segments overlapping [a, b)
  SeqWindow sw;
  scan_window(sw, p, 0, 0);
  int64_t pos = a;
  while (pos < b) {
    while ((int64_t)(sw.base + sw.total) * NHG <= pos) scan_window(sw, p, sw.blk0 + 64, sw.base + sw.total);
    const int64_t start = (int64_t)(sw.base + sw.excl) * NHG;  // first chunk of this lane's sequence
    const uint64_t hit = __builtin_amdgcn_ballot_w64(sw.c > 0 && start <= pos && pos < start + (int64_t)sw.c * NHG);
    if (hit == 0) break;  // cannot happen for consistent metadata; never index lane 64
    const int l = __builtin_ctzll(hit);
    const int seq = sw.blk0 + l;
    const int c = __builtin_amdgcn_readlane(sw.c, l);
    const int64_t seq_start = (int64_t)(sw.base + __builtin_amdgcn_readlane(sw.excl, l)) * NHG;
    const int hg = (int)((pos - seq_start) / c);
    const int64_t seg_beg = seq_start + (int64_t)hg * c, seg_end = seg_beg + c;
    const int64_t y = b < seg_end ? b : seg_end;
    const int kvh = hg * p.HGW + hw;

    const SeqView sv = seq_view(p, seq);
    const int R = sv.q_len * p.G;
    const int tok_lo = (int)(pos - seg_beg) * kChunk;
    const int tok_hi = min((int)(y - seg_beg) * kChunk, sv.kv_total);
    WaveState<D, NT> st;
    load_q<D, NT>(st, p, sv.qs, R, 0, kvh, sv.ctx, sv.kv_total);
    const int64_t* btrow = p.bt + (int64_t)seq * p.bt_rs;
    run_chunks<E, D, NT>(st, p, btrow, kvh, tok_lo, kChunk, tok_hi, sv.kv_total);
    const bool whole = pos == seg_beg && y == seg_end;
    const int64_t slot = (int64_t)seq * NHG + hg + unit;
    write_rows<E, D, NT>(st, p, sv, R, 0, kvh, !whole, (slot * p.HGW + hw) * p.RS);
    pos = y;
  }
}

// Log-sum-exp merge of the pieces of split decode segments. Grid (RS, Hkv, B): one wave per
// query row; lane owns D / 64 consecutive elements. Units u0 .. u1 hold the pieces of the
// row's segment [seg_beg, seg_end); a segment held by one unit was written out directly.
template <class E, int D>
__global__ __launch_bounds__(64) void pa_reduce_kernel(PAParams p) {
  constexpr int PL = D / 64;  // elements per lane
  const int r = blockIdx.x, kvh = blockIdx.y, seq = blockIdx.z;
  const int lane = threadIdx.x;
  const SeqView sv = seq_view(p, seq);
  if (sv.q_len == 0 || sv.q_len > p.QS) return;
  if (r >= sv.q_len * p.G) return;
  const int NHG = p.Hkv / p.HGW;
  const int hg = kvh / p.HGW, hw = kvh % p.HGW;
  const int c = max(1, (sv.kv_total + kChunk - 1) / kChunk);
  const int64_t C = (int64_t)p.ws_cum[p.B] * NHG;
  const int64_t NUa = active_units(C, p.NU);
  const int64_t seg_beg = (int64_t)p.ws_cum[seq] * NHG + (int64_t)hg * c, seg_end = seg_beg + c;
  const int64_t u0 = ((seg_beg + 1) * NUa - 1) / C, u1 = (seg_end * NUa - 1) / C;
  if (u0 == u1) return;
  const int64_t seg = (int64_t)seq * NHG + hg;
  auto row = [&](int64_t u) { return ((seg + u) * p.HGW + hw) * p.RS + r; };
  float M = -INFINITY;
  for (int64_t u = u0; u <= u1; ++u) M = fmaxf(M, p.ws_ml[row(u) * 2]);
  const float msafe = M == -INFINITY ? 0.f : M;
  float L = 0.f;
  float o[PL];
#pragma unroll
  for (int i = 0; i < PL; ++i) o[i] = 0.f;
#pragma unroll 4
  for (int64_t u = u0; u <= u1; ++u) {
    const int64_t idx = row(u);
    const float f = fast_exp2(p.ws_ml[idx * 2] - msafe);
    L += f * p.ws_ml[idx * 2 + 1];
    const float* acc = p.ws_acc + idx * D + PL * lane;
    if constexpr (PL == 2) {
      const float2 x = *(const float2*)acc;
      o[0] += f * x.x;
      o[1] += f * x.y;
    } else {
      o[0] += f * acc[0];
    }
  }
  const float inv = 1.f / (L == 0.f ? 1.f : L);
  const int qi = r / p.G, g = r % p.G;
  uint16_t* dst = (uint16_t*)p.out + (sv.qs + qi) * p.o_ts + (int64_t)(kvh * p.G + g) * p.o_hs + PL * lane;
  if constexpr (PL == 2) {
    *(uint32_t*)dst = E::pack2(o[0] * inv, o[1] * inv);
  } else {
    *dst = (uint16_t)(E::pack2(o[0] * inv, 0.f) & 0xffffu);
  }
}

// ---------------------------------------------------------------------------------------
// Prefill class: grid (ceil(max_q * G / 128), Hkv, B); wave w owns rows
// (blockIdx.x * 4 + w) * 32 .. + 31 of its sequence's R = q_len * G rows.
template <class E, int D>
__global__ __launch_bounds__(256) void pa_prefill_kernel(PAParams p) {
  constexpr int NT = kPrefillNQT;
  const int kvh = blockIdx.y, seq = blockIdx.z;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  const SeqView sv = seq_view(p, seq);
  if (sv.q_len <= p.QS) return;
  const int R = sv.q_len * p.G;
  const int row0 = (blockIdx.x * kWavesPerWG + w) * (16 * NT);
  if (row0 >= R) return;
  const int last_row = min(row0 + 16 * NT - 1, R - 1);
  const int kv_lim = (int)clamp64(sv.ctx + last_row / p.G + 1, 0, sv.kv_total);

  WaveState<D, NT> s;
  load_q<D, NT>(s, p, sv.qs, R, row0, kvh, sv.ctx, sv.kv_total);
  const int64_t* btrow = p.bt + (int64_t)seq * p.bt_rs;
  run_chunks<E, D, NT>(s, p, btrow, kvh, 0, kChunk, kv_lim, sv.kv_total);
  write_rows<E, D, NT>(s, p, sv, R, row0, kvh, false, 0);
}

// ---------------------------------------------------------------------------------------
// Waves one decode launch can keep resident on the current device, from the occupancy of
// the instantiation actually launched (cached per device and kernel).
static int resident_waves(const void* kernel) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256 * kWavesPerWG;
  static thread_local int cache_dev = -1;
  static thread_local const void* cache_kernel = nullptr;
  static thread_local int cache_waves = 0;
  if (dev == cache_dev && kernel == cache_kernel) return cache_waves;
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, 256, 0) != hipSuccess || per_cu <= 0) per_cu = 1;
  int waves = cus * per_cu * kWavesPerWG;
  if (waves > kMaxDecodeWaves) waves = kMaxDecodeWaves;
  cache_dev = dev;
  cache_kernel = kernel;
  cache_waves = waves;
  return waves;
}

template <class E, int D, int NT>
static int launch_decode_nt(PAParams& p, hipStream_t s) {
  const void* k = (const void*)&pa_decode_kernel<E, D, NT>;
  const int waves = resident_waves(k);
  p.NU = waves / p.HGW;
  const int wgs = (p.NU * p.HGW + kWavesPerWG - 1) / kWavesPerWG;
  hipLaunchKernelGGL((pa_decode_kernel<E, D, NT>), dim3(wgs), dim3(256), 0, s, p);
  return (int)hipGetLastError();
}

template <class E, int D>
static int launch_mfma_typed(PAParams& p, const Plan& plan, hipStream_t s, LaunchLog& log) {
  int err = 0;
  switch (plan.NT) {
    case 1: err = launch_decode_nt<E, D, 1>(p, s); break;
    case 2: err = launch_decode_nt<E, D, 2>(p, s); break;
    case 3: err = launch_decode_nt<E, D, 3>(p, s); break;
    case 4: err = launch_decode_nt<E, D, 4>(p, s); break;
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
  dim3 grid(plan.RS, p.Hkv, p.B);
  hipLaunchKernelGGL((pa_reduce_kernel<E, D>), grid, dim3(64), 0, s, p);
  if ((err = (int)hipGetLastError())) return err;
  log.after_launch(3, s);
  return 0;
}

int launch_paged_attention_mfma(PAParams& p, const Plan& plan, int32_t D, int32_t dtype, hipStream_t s,
                                LaunchLog& log) {
  const bool bf = dtype == 2;
  if (D == 128)
    return bf ? launch_mfma_typed<BF16, 128>(p, plan, s, log) : launch_mfma_typed<F16, 128>(p, plan, s, log);
  if (D == 64) return bf ? launch_mfma_typed<BF16, 64>(p, plan, s, log) : launch_mfma_typed<F16, 64>(p, plan, s, log);
  return (int)hipErrorInvalidValue;
}

}  // namespace kvh
