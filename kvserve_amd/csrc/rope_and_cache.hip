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

}  // namespace kvh
