// rope_and_cache: the step before paged attention in one pass. From the fused QKV
// projection of this step's tokens it writes the rotated queries for attention and
// scatters the rotated keys and the values into the paged pool.
//
// Semantics (bit for bit) of the reference's Attention.project + write_kv,
// src/kvserve/model.py:84-94 and src/kvserve/attention.py:39-45:
//   q, k, v = qkv.split([H D, Hkv D, Hkv D]) viewed as heads of D
//   cos = cos_table[positions].to(dtype); sin likewise                  (model.py:63-64)
//   q' = q * cos + rotate_half(q) * sin; k' likewise, rotate_half(x) = cat(-x2, x1)
//   k_cache.view(-1, Hkv, D)[slots] = k'; v_cache.view(-1, Hkv, D)[slots] = v
// Each of the three elementwise steps rounds to the storage type, as PyTorch's separate
// kernels do: bf16 through fp32 (products of two bf16 values are exact in fp32, the sum is
// rounded to fp32 then to bf16), fp16 rounded once from the exact result. fp32 storage
// rounds nothing extra.
//
// One workgroup per token: its items are (head, 8 (4 for fp32) consecutive d of the first
// half) pairs for the query and key heads, with the matching elements of the second half,
// then 16-byte vectors of the value rows. Positions outside the tables are clamped; slots
// outside the pool skip the cache writes (as reshape_and_cache does).
#include <type_traits>

#include "kvh_device.h"
#include "kvh_internal.h"

namespace kvh {

template <int DT>  // KVH_DTYPE_*: 0 fp32, 1 fp16, 2 bf16
struct RopeElem {
  static constexpr int kBytes = DT == 0 ? 4 : 2;
  static constexpr int kVec = 16 / kBytes;  // elements per 16-byte vector
  static __device__ __forceinline__ float rnd(float x) {
    if constexpr (DT == 2) return (float)(__bf16)x;
    else if constexpr (DT == 1) return (float)(_Float16)x;
    else return x;
  }
  // a * b and a + b of two storage-type values, rounded once to the storage type: fp16 in
  // native half arithmetic (one rounding of the exact result, as PyTorch's half kernels
  // give), bf16 through fp32 (PyTorch's float opmath: the fp32 result rounded to bf16).
  static __device__ __forceinline__ float mul(float a, float b) {
    if constexpr (DT == 1) return (float)((_Float16)a * (_Float16)b);
    else return rnd(a * b);
  }
  static __device__ __forceinline__ float add(float a, float b) {
    if constexpr (DT == 1) return (float)((_Float16)a + (_Float16)b);
    else return rnd(a + b);
  }
  static __device__ __forceinline__ void load(const uint8_t* p, float (&x)[kVec]) {
    const u32x4 w = *(const u32x4*)p;
    if constexpr (DT == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = __uint_as_float(w[i]);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint16_t h = (uint16_t)(w[i / 2] >> (16 * (i & 1)));
        x[i] = DT == 2 ? BF16::to_f32(h) : F16::to_f32(h);
      }
    }
  }
  static __device__ __forceinline__ void store(uint8_t* p, const float (&x)[kVec]) {
    u32x4 w;
    if constexpr (DT == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = __float_as_uint(x[i]);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = DT == 2 ? BF16::pack2(x[2 * i], x[2 * i + 1]) : F16::pack2(x[2 * i], x[2 * i + 1]);
    }
    *(u32x4*)p = w;
  }
};

// V values (8, or 4 for fp32) prepared for E4M3 and stored as V bytes.
template <int V>
__device__ __forceinline__ void store_fp8(uint8_t* dst, const float (&x)[V], float scale) {
  float y[V];
#pragma unroll
  for (int i = 0; i < V; ++i) y[i] = fp8_prep(x[i], scale);
  if constexpr (V == 8)
    *(u32x2*)dst = u32x2{fp8_pack4(y[0], y[1], y[2], y[3]), fp8_pack4(y[4], y[5], y[6], y[7])};
  else
    *(uint32_t*)dst = fp8_pack4(y[0], y[1], y[2], y[3]);
}

// KV8: the cache is E4M3 (kvh_rope_and_cache_fp8): the rotated keys, rounded to the storage
// type as above, and the values are then stored as e4m3(clamp(x / scale, -448, 448)).
template <int DT, bool KV8>
__global__ __launch_bounds__(256) void rope_and_cache_kernel(
    const uint8_t* qkv, int64_t qkv_ts, const int64_t* positions, const float* cos_t, const float* sin_t,
    int64_t max_pos, uint8_t* q_out, int64_t q_ts, int64_t q_hs, uint8_t* kc, int64_t k_sb, int64_t k_ss,
    int64_t k_sh, uint8_t* vc, int64_t v_sb, int64_t v_ss, int64_t v_sh, const int64_t* slots, int64_t num_slots,
    int H, int Hkv, int D, int BS, float k_scale, float v_scale) {
  using R = RopeElem<DT>;
  constexpr int V = R::kVec;
  constexpr int EB = R::kBytes;
  constexpr int CB = KV8 ? 1 : EB;  // bytes per cache element
  const int64_t t = blockIdx.x;
  const int half = D / 2;
  const int pv = half / V;  // vectors per half row
  const int n_rot = (H + Hkv) * pv;
  const int n_v = Hkv * (D / V);
  const int64_t pos = clamp64(positions[t], 0, max_pos - 1);
  const float* cr = cos_t + pos * D;
  const float* sr = sin_t + pos * D;
  const int64_t slot = slots[t];
  const bool in_pool = slot >= 0 && slot < num_slots;
  const int64_t blk = in_pool ? slot / BS : 0, off = in_pool ? slot % BS : 0;
  const uint8_t* row = qkv + t * qkv_ts * EB;
  for (int it = threadIdx.x; it < n_rot + n_v; it += 256) {
    if (it < n_rot) {
      const int h = it / pv;  // 0 .. H - 1 query heads, then H .. H + Hkv - 1 key heads
      const int d = (it % pv) * V;
      const uint8_t* src = row + ((int64_t)h * D + d) * EB;
      float lo[V], hi[V], o_lo[V], o_hi[V];
      R::load(src, lo);
      R::load(src + half * EB, hi);
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const float c_lo = R::rnd(cr[d + j]), c_hi = R::rnd(cr[d + half + j]);
        const float s_lo = R::rnd(sr[d + j]), s_hi = R::rnd(sr[d + half + j]);
        o_lo[j] = R::add(R::mul(lo[j], c_lo), R::mul(-hi[j], s_lo));
        o_hi[j] = R::add(R::mul(hi[j], c_hi), R::mul(lo[j], s_hi));
      }
      if (h < H) {
        uint8_t* dst = q_out + (t * q_ts + (int64_t)h * q_hs + d) * EB;
        R::store(dst, o_lo);
        R::store(dst + half * EB, o_hi);
      } else {
        if (!in_pool) continue;
        uint8_t* dst = kc + (blk * k_sb + off * k_ss + (int64_t)(h - H) * k_sh + d) * CB;
        if constexpr (KV8) {
          store_fp8<V>(dst, o_lo, k_scale);
          store_fp8<V>(dst + half, o_hi, k_scale);
        } else {
          R::store(dst, o_lo);
          R::store(dst + half * EB, o_hi);
        }
      }
    } else {
      if (!in_pool) continue;
      const int r = it - n_rot;
      const int h = r / (D / V), d = (r % (D / V)) * V;
      const uint8_t* src = row + ((int64_t)(H + Hkv + h) * D + d) * EB;
      uint8_t* dst = vc + (blk * v_sb + off * v_ss + (int64_t)h * v_sh + d) * CB;
      if constexpr (KV8) {
        float x[V];
        R::load(src, x);
        store_fp8<V>(dst, x, v_scale);
      } else {
        *(u32x4*)dst = *(const u32x4*)src;
      }
    }
  }
}

int launch_rope_and_cache(const void* qkv, int64_t qkv_ts, const int64_t* positions, const float* cos_t,
                          const float* sin_t, int64_t max_pos, void* q_out, int64_t q_ts, int64_t q_hs, void* kc,
                          const int64_t* kcs, void* vc, const int64_t* vcs, const int64_t* slots, int64_t T,
                          int64_t num_blocks, int32_t H, int32_t Hkv, int32_t D, int32_t BS, int32_t dtype,
                          bool kv8, float k_scale, float v_scale, hipStream_t s) {
  if (T == 0) return 0;
  const int64_t num_slots = num_blocks * BS;
#define KVH_LAUNCH_ROPE(DT, KV8)                                                                                  \
  hipLaunchKernelGGL((rope_and_cache_kernel<DT, KV8>), dim3((unsigned)T), dim3(256), 0, s, (const uint8_t*)qkv,  \
                     qkv_ts, positions, cos_t, sin_t, max_pos, (uint8_t*)q_out, q_ts, q_hs, (uint8_t*)kc, kcs[0],  \
                     kcs[1], kcs[2], (uint8_t*)vc, vcs[0], vcs[1], vcs[2], slots, num_slots, H, Hkv, D, BS,        \
                     k_scale, v_scale)
  if (dtype == 2) {
    if (kv8) KVH_LAUNCH_ROPE(2, true); else KVH_LAUNCH_ROPE(2, false);
  } else if (dtype == 1) {
    if (kv8) KVH_LAUNCH_ROPE(1, true); else KVH_LAUNCH_ROPE(1, false);
  } else {
    if (kv8) KVH_LAUNCH_ROPE(0, true); else KVH_LAUNCH_ROPE(0, false);
  }
#undef KVH_LAUNCH_ROPE
  return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------------------
// gemv_rope_and_cache: the QKV projection of m <= 4 decode rows (y = x W^T, W [(H + 2 Hkv) D,
// k]) with rope_and_cache as its epilogue, in one launch. Wave w owns the pair of weight rows
// (h D + d, h D + d + D / 2) of head h = w / (D / 2), d = w % (D / 2): the two elements
// RoPE mixes. Each row's sum is taken exactly as gemv_kernel takes it (lane l walks
// k = 8 l + 1024 i (+ 512), 8 explicit FMAs per vector, the rest in 512-steps, then a
// butterfly), rounded to the storage type, and then goes through rope_and_cache_kernel's
// arithmetic: the result has the bits of kvh_gemv followed by kvh_rope_and_cache(_fp8).
struct GemvRopeArgs {
  const uint16_t* x;
  int64_t x_rs;
  const uint16_t* w;
  int64_t w_rs;
  int k;
  const int64_t* positions;
  const float* cos_t;
  const float* sin_t;
  int64_t max_pos;
  uint8_t* q_out;
  int64_t q_ts, q_hs;
  uint8_t* kc;
  int64_t k_sb, k_ss, k_sh;
  uint8_t* vc;
  int64_t v_sb, v_ss, v_sh;
  const int64_t* slots;
  int64_t num_slots;
  int H, Hkv, D, BS;
  float k_scale, v_scale;
};

template <int DT, bool KV8>
__device__ __forceinline__ void store_one(uint8_t* dst, float x, float scale) {
  if constexpr (KV8) {
    *dst = (uint8_t)(fp8_pack4(fp8_prep(x, scale), 0.f, 0.f, 0.f) & 0xffu);
  } else {
    const uint32_t b = DT == 2 ? BF16::pack2(x, 0.f) : F16::pack2(x, 0.f);
    *(uint16_t*)dst = (uint16_t)(b & 0xffffu);
  }
}

// rope_and_cache of one pair (d, d + D / 2) of head h for token row `row`, from the two fp32
// projection sums
template <int DT, bool KV8>
__device__ __forceinline__ void rope_pair_out(const GemvRopeArgs& a, int row, int h, int d, float s_lo, float s_hi) {
  using R = RopeElem<DT>;
  constexpr int CB = KV8 ? 1 : 2;  // bytes per cache element
  const int half = a.D / 2;
  const float lo = R::rnd(s_lo), hi = R::rnd(s_hi);  // the projection's output
  const int64_t slot = a.slots[row];
  const bool in_pool = slot >= 0 && slot < a.num_slots;
  const int64_t blk = in_pool ? slot / a.BS : 0, off = in_pool ? slot % a.BS : 0;
  if (h < a.H + a.Hkv) {
    const int64_t pos = clamp64(a.positions[row], 0, a.max_pos - 1);
    const float* cr = a.cos_t + pos * a.D;
    const float* sr = a.sin_t + pos * a.D;
    const float c_lo = R::rnd(cr[d]), c_hi = R::rnd(cr[d + half]);
    const float s_lo2 = R::rnd(sr[d]), s_hi2 = R::rnd(sr[d + half]);
    const float o_lo = R::add(R::mul(lo, c_lo), R::mul(-hi, s_lo2));
    const float o_hi = R::add(R::mul(hi, c_hi), R::mul(lo, s_hi2));
    if (h < a.H) {
      uint8_t* dst = a.q_out + (row * a.q_ts + (int64_t)h * a.q_hs + d) * 2;
      store_one<DT, false>(dst, o_lo, 1.f);
      store_one<DT, false>(dst + half * 2, o_hi, 1.f);
    } else if (in_pool) {
      uint8_t* dst = a.kc + (blk * a.k_sb + off * a.k_ss + (int64_t)(h - a.H) * a.k_sh + d) * CB;
      store_one<DT, KV8>(dst, o_lo, a.k_scale);
      store_one<DT, KV8>(dst + half * CB, o_hi, a.k_scale);
    }
  } else if (in_pool) {
    uint8_t* dst = a.vc + (blk * a.v_sb + off * a.v_ss + (int64_t)(h - a.H - a.Hkv) * a.v_sh + d) * CB;
    store_one<DT, KV8>(dst, lo, a.v_scale);
    store_one<DT, KV8>(dst + half * CB, hi, a.v_scale);
  }
}

template <int DT, int M, bool KV8>
__global__ __launch_bounds__(256) void gemv_rope_cache_kernel(GemvRopeArgs a) {
  using E = std::conditional_t<DT == 2, BF16, F16>;
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int half = a.D / 2;
  const int nh = a.H + 2 * a.Hkv;
  if (wave >= nh * half) return;
  const int h = wave / half, d = wave % half;
  const uint16_t* wr[2] = {a.w + ((int64_t)h * a.D + d) * a.w_rs, a.w + ((int64_t)h * a.D + d + half) * a.w_rs};
  float acc[M][2];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m][0] = acc[m][1] = 0.f;
  auto fma8 = [&](const u32x4& xv, const u32x4& wv, float& c) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint16_t xb = (uint16_t)(xv[i / 2] >> (16 * (i & 1))), wb = (uint16_t)(wv[i / 2] >> (16 * (i & 1)));
      c = __builtin_fmaf(E::to_f32(xb), E::to_f32(wb), c);
    }
  };
  const int k = a.k, kfull = k / 1024 * 1024;
  for (int k0 = 8 * lane; k0 < kfull; k0 += 1024) {
    u32x4 wv[2][2], xv[2][M];
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
#pragma unroll
      for (int r = 0; r < 2; ++r) wv[s2][r] = *(const u32x4*)(wr[r] + k0 + 512 * s2);
#pragma unroll
      for (int m = 0; m < M; ++m) xv[s2][m] = *(const u32x4*)(a.x + m * a.x_rs + k0 + 512 * s2);
    }
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < 2; ++r) fma8(xv[s2][m], wv[s2][r], acc[m][r]);
  }
  for (int k0 = kfull + 8 * lane; k0 < k; k0 += 512) {
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const u32x4 xv = *(const u32x4*)(a.x + m * a.x_rs + k0);
#pragma unroll
      for (int r = 0; r < 2; ++r) fma8(xv, *(const u32x4*)(wr[r] + k0), acc[m][r]);
    }
  }
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      float v = acc[m][r];
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
      acc[m][r] = v;
    }
  if (lane != 0) return;
#pragma unroll
  for (int m = 0; m < M; ++m) rope_pair_out<DT, KV8>(a, m, h, d, acc[m][0], acc[m][1]);
}

// The same for 5 .. 64 rows on the MFMA units, laid out as the skinny GEMM (engine_ops.hip):
// a workgroup of 8 waves (k-slices) owns 8 pairs (one 16-row A tile: rows h D + d0 + i for
// i < 8, h D + d0 + D / 2 + i - 8 for i >= 8) and MT = ceil(m / 16) B tiles of x; the eight
// partial tiles meet in LDS, are summed in wave order and go through rope_pair_out.
template <int DT, int MT, bool KV8>
__global__ __launch_bounds__(512) void skinny_rope_cache_kernel(GemvRopeArgs a, int m) {
  using E = std::conditional_t<DT == 2, BF16, F16>;
  __shared__ f32x4 red[8][MT][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int i = lane & 15, jg = lane >> 4;
  const int half = a.D / 2;
  const int p0 = blockIdx.x * 8;  // first pair
  const int h = p0 / half, d0 = p0 % half;
  const int64_t wrow = (int64_t)h * a.D + d0 + (i < 8 ? i : half + i - 8);
  const int slice = a.k / 8;
  const int k_lo = wave * slice;
  const uint16_t* wr = a.w + wrow * a.w_rs + k_lo + 8 * jg;
  const uint16_t* xr[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) xr[t] = a.x + (int64_t)min(16 * t + i, m - 1) * a.x_rs + k_lo + 8 * jg;
  f32x4 acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int kk = 0; kk < slice; kk += 128) {
    u32x4 av[4], bv[4][MT];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      av[u] = *(const u32x4*)(wr + kk + 32 * u);
#pragma unroll
      for (int t = 0; t < MT; ++t) bv[u][t] = *(const u32x4*)(xr[t] + kk + 32 * u);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int t = 0; t < MT; ++t) acc[t] = E::mfma(av[u], bv[u][t], acc[t]);
  }
#pragma unroll
  for (int t = 0; t < MT; ++t) red[wave][t][lane] = acc[t];
  __syncthreads();
  for (int q = threadIdx.x; q < MT * 128; q += 512) {
    const int t = q >> 7, mr = (q >> 3) & 15, c = q & 7;
    const int row = 16 * t + mr;
    if (row >= m) continue;
    const int ll = 16 * (c >> 2) + mr, lh = 16 * (2 + (c >> 2)) + mr, r = c & 3;
    float s_lo = 0.f, s_hi = 0.f;
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      s_lo += red[v][t][ll][r];
      s_hi += red[v][t][lh][r];
    }
    rope_pair_out<DT, KV8>(a, row, h, d0 + c, s_lo, s_hi);
  }
}

template <int DT, bool KV8>
static int launch_gemv_rope_dt(const GemvRopeArgs& a, int m, hipStream_t s) {
  const int waves = (a.H + 2 * a.Hkv) * (a.D / 2);
  if (m > 4) {  // the skinny form: one workgroup per 8 pairs
    const dim3 g2((unsigned)(waves / 8)), b2(512);
    switch ((m + 15) / 16) {
      case 1: hipLaunchKernelGGL((skinny_rope_cache_kernel<DT, 1, KV8>), g2, b2, 0, s, a, m); break;
      case 2: hipLaunchKernelGGL((skinny_rope_cache_kernel<DT, 2, KV8>), g2, b2, 0, s, a, m); break;
      case 3: hipLaunchKernelGGL((skinny_rope_cache_kernel<DT, 3, KV8>), g2, b2, 0, s, a, m); break;
      default: hipLaunchKernelGGL((skinny_rope_cache_kernel<DT, 4, KV8>), g2, b2, 0, s, a, m); break;
    }
    return (int)hipGetLastError();
  }
  const dim3 grid((waves + 3) / 4);
  switch (m) {
    case 1: hipLaunchKernelGGL((gemv_rope_cache_kernel<DT, 1, KV8>), grid, dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL((gemv_rope_cache_kernel<DT, 2, KV8>), grid, dim3(256), 0, s, a); break;
    case 3: hipLaunchKernelGGL((gemv_rope_cache_kernel<DT, 3, KV8>), grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL((gemv_rope_cache_kernel<DT, 4, KV8>), grid, dim3(256), 0, s, a); break;
  }
  return (int)hipGetLastError();
}

int launch_gemv_rope_and_cache(const void* x, int64_t x_rs, const void* w, int64_t w_rs, int32_t m, int32_t k,
                               const int64_t* positions, const float* cos_t, const float* sin_t, int64_t max_pos,
                               void* q_out, int64_t q_ts, int64_t q_hs, void* kc, const int64_t* kcs, void* vc,
                               const int64_t* vcs, const int64_t* slots, int64_t num_blocks, int32_t H, int32_t Hkv,
                               int32_t D, int32_t BS, int32_t dtype, bool kv8, float k_scale, float v_scale,
                               hipStream_t s) {
  GemvRopeArgs a{};
  a.x = (const uint16_t*)x, a.x_rs = x_rs, a.w = (const uint16_t*)w, a.w_rs = w_rs, a.k = k;
  a.positions = positions, a.cos_t = cos_t, a.sin_t = sin_t, a.max_pos = max_pos;
  a.q_out = (uint8_t*)q_out, a.q_ts = q_ts, a.q_hs = q_hs;
  a.kc = (uint8_t*)kc, a.k_sb = kcs[0], a.k_ss = kcs[1], a.k_sh = kcs[2];
  a.vc = (uint8_t*)vc, a.v_sb = vcs[0], a.v_ss = vcs[1], a.v_sh = vcs[2];
  a.slots = slots, a.num_slots = num_blocks * BS;
  a.H = H, a.Hkv = Hkv, a.D = D, a.BS = BS, a.k_scale = k_scale, a.v_scale = v_scale;
  if (dtype == 2) return kv8 ? launch_gemv_rope_dt<2, true>(a, m, s) : launch_gemv_rope_dt<2, false>(a, m, s);
  return kv8 ? launch_gemv_rope_dt<1, true>(a, m, s) : launch_gemv_rope_dt<1, false>(a, m, s);
}

}  // namespace kvh
