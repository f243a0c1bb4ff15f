// Paged attention on the vector ALUs: the exact-fp32 path (the reference's IEEE mode,
// src/kvserve/kernels/paged_attention.py:92-95, :106-109, used by its fp32 engine identity
// tests) and the 16-bit path for the shapes the MFMA kernels do not tile: head sizes other than
// 64 and 128 (the reference pads any head size to a power of two and masks it, :64-67, :154),
// pages of fewer than 16 tokens or not a multiple of 16, GQA groups above 64. Correctness path,
// not a bandwidth path: plain fp32 FMA, any head_dim <= 256 whose rows are whole 16-byte
// vectors, any block size.
//
// Grid (B, H, ceil(max_q / kRowsPerWG)); one wave per workgroup walks the query tokens
// q0, q0 + 1, ... of its (sequence, head) one at a time. For each 64-key tile, lane k scores
// key k (full dot product over d, fp32), the wave does an online-softmax update in the exp2
// domain, then every lane accumulates its own d columns over the tile's keys. With 16-bit
// storage P is rounded to the storage type before the P.V sum, the row sum keeps the unrounded
// P and the output is rounded once, as the reference kernel does (:106-115).
#include "kvh_device.h"
#include "kvh_internal.h"

namespace kvh {

constexpr int kRowsPerWG = 8;

// Element access of the three storage types: 16 bytes hold V elements.
struct F32 {
  static constexpr int V = 4;
  static __device__ __forceinline__ float load(const void* p, int64_t i) { return ((const float*)p)[i]; }
  static __device__ __forceinline__ float round(float x) { return x; }
  static __device__ __forceinline__ void store(void* p, int64_t i, float x) { ((float*)p)[i] = x; }
  static __device__ __forceinline__ float elem(const u32x4& w, int e) { return __uint_as_float(w[e]); }
};

template <class E>
struct Half16 {
  static constexpr int V = 8;
  static __device__ __forceinline__ float load(const void* p, int64_t i) { return E::to_f32(((const uint16_t*)p)[i]); }
  static __device__ __forceinline__ float round(float x) { return E::to_f32((uint16_t)(E::pack2(x, 0.f) & 0xffffu)); }
  static __device__ __forceinline__ void store(void* p, int64_t i, float x) {
    ((uint16_t*)p)[i] = (uint16_t)(E::pack2(x, 0.f) & 0xffffu);
  }
  static __device__ __forceinline__ float elem(const u32x4& w, int e) {
    const uint32_t d = w[e >> 1];
    return E::to_f32((uint16_t)((e & 1) ? d >> 16 : d & 0xffffu));
  }
};

template <class S, int DPL>  // d columns per lane: d = lane + 64 * x, x < DPL
__global__ __launch_bounds__(64) void pa_valu_kernel(PAParams p, int D) {
  const int seq = blockIdx.x, head = blockIdx.y;
  const int lane = threadIdx.x;
  const int kvh = head / p.G;
  const int64_t qs = clamp64(p.qsl[seq], 0, p.T);
  const int64_t qe = clamp64(p.qsl[seq + 1], qs, p.T);
  const int q_len = (int)(qe - qs);
  const int64_t sl = p.seq_lens[seq];
  const int64_t ctx = sl - q_len;
  const int kv_total = (int)clamp64(sl, 0, (int64_t)p.W * p.BS);
  const int64_t* btrow = p.bt + (int64_t)seq * p.bt_rs;
  __shared__ float s_q[256];

  const int qi_end = min(q_len, (int)(blockIdx.z + 1) * kRowsPerWG);
  for (int qi = blockIdx.z * kRowsPerWG; qi < qi_end; ++qi) {
    const int64_t tok = qs + qi;
    const int64_t qrow = tok * p.q_ts + (int64_t)head * p.q_hs;
    __syncthreads();
    for (int d = lane; d < D; d += 64) s_q[d] = S::load(p.q, qrow + d);
    __syncthreads();
    const int limit = (int)clamp64(ctx + qi + 1, 0, kv_total);
    float m = -INFINITY, l = 0.f;
    float acc[DPL];
#pragma unroll
    for (int x = 0; x < DPL; ++x) acc[x] = 0.f;

    for (int k0 = 0; k0 < limit; k0 += 64) {
      const int key = k0 + lane;
      float s = -INFINITY;
      int64_t vbase = -1;
      if (key < limit) {
        const int64_t blk = btrow[key / p.BS];
        if (blk >= 0 && blk < p.num_blocks) {
          const int64_t slot = key % p.BS;
          vbase = blk * p.v_sb + slot * p.v_ss + (int64_t)kvh * p.v_sh;
          const int64_t kbase = blk * p.k_sb + slot * p.k_ss + (int64_t)kvh * p.k_sh;
          const u32x4* kp = (const u32x4*)((const char*)p.kc + kbase * (int64_t)(16 / S::V));
          float dot = 0.f;
          for (int d = 0; d < D; d += S::V) {
            const u32x4 w = kp[d / S::V];
#pragma unroll
            for (int e = 0; e < S::V; ++e) dot = __builtin_fmaf(s_q[d + e], S::elem(w, e), dot);
          }
          s = dot * p.qk_scale;
        }
      }
      float mx = s;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
      const float m_new = fmaxf(m, mx);
      const float m_safe = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = exp2f(m - m_safe);
      const float pk = exp2f(s - m_safe);
      float ps = pk;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) ps += __shfl_xor(ps, o);
      l = l * alpha + ps;
      m = m_new;
      const float pr = S::round(pk);  // the P that multiplies V
#pragma unroll
      for (int x = 0; x < DPL; ++x) acc[x] *= alpha;
      const int nk = min(64, limit - k0);
      for (int kk = 0; kk < nk; ++kk) {
        const float pw = __shfl(pr, kk);
        const int64_t vb = __shfl(vbase, kk);
        if (vb < 0) continue;  // empty page: weight is 0 and there is nothing to read
#pragma unroll
        for (int x = 0; x < DPL; ++x) {
          const int d = lane + 64 * x;
          if (d < D) acc[x] = __builtin_fmaf(pw, S::load(p.vc, vb + d), acc[x]);
        }
      }
    }
    const float inv = p.v_scale / (l == 0.f ? 1.f : l);
    const int64_t orow = tok * p.o_ts + (int64_t)head * p.o_hs;
#pragma unroll
    for (int x = 0; x < DPL; ++x) {
      const int d = lane + 64 * x;
      if (d < D) S::store(p.out, orow + d, acc[x] * inv);
    }
  }
}

template <class S>
static int launch_valu(const PAParams& p, int32_t D, int32_t max_q, hipStream_t s) {
  dim3 grid(p.B, p.H, (max_q + kRowsPerWG - 1) / kRowsPerWG);
  if (D <= 64)
    hipLaunchKernelGGL((pa_valu_kernel<S, 1>), grid, dim3(64), 0, s, p, D);
  else if (D <= 128)
    hipLaunchKernelGGL((pa_valu_kernel<S, 2>), grid, dim3(64), 0, s, p, D);
  else
    hipLaunchKernelGGL((pa_valu_kernel<S, 4>), grid, dim3(64), 0, s, p, D);
  return (int)hipGetLastError();
}

int launch_paged_attention_valu(const PAParams& p, int32_t D, int32_t dtype, int32_t max_q, hipStream_t s,
                                LaunchLog& log) {
  int err;
  if (dtype == 0)
    err = launch_valu<F32>(p, D, max_q, s);
  else if (dtype == 1)
    err = launch_valu<Half16<kvh::F16>>(p, D, max_q, s);
  else
    err = launch_valu<Half16<BF16>>(p, D, max_q, s);
  if (!err) log.after_launch(dtype == 0 ? 4 : 6, s);
  return err;
}

}  // namespace kvh
